"""Device memory helpers of the C ABI (ttl_memcpy_d2d, ttl_fill_bytes, ttl_stream_read) on the GPU."""
import numpy as np
import pytest

import ttlab_amd

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("nbytes,src_off,dst_off", [(1 << 20, 0, 0), (4096 + 16, 16, 32), (1000, 3, 0), (17, 0, 5)])
def test_device_copy_is_exact(nbytes, src_off, dst_off):
    dev = ttlab_amd.Device(0)
    data = np.random.default_rng(nbytes).integers(0, 256, nbytes + 64, dtype=np.uint8)
    src = dev.upload(data)
    dst = dev.alloc(nbytes + 64)
    dev.fill(dst, 0xAB)
    dev.copy(dst.offset(dst_off), src.offset(src_off), nbytes)
    got = dst.download(np.uint8)
    expect = np.full(nbytes + 64, 0xAB, np.uint8)
    expect[dst_off:dst_off + nbytes] = data[src_off:src_off + nbytes]
    assert np.array_equal(got, expect)
    dev.close()


@pytest.mark.parametrize("words", [1024, 1500, 4096])
def test_stream_read_reads_every_load(words):
    # thread 0 of block 1 reads words 1024, 1280, 1536, 1792; their XOR is the sink
    # constant only when all four loads arrive, and no other thread's XOR is
    dev = ttlab_amd.Device(0)
    data = np.zeros((max(words, 2048), 4), np.uint32)
    data[1024, 0], data[1280, 1], data[1536, 2], data[1792, 3] = 0x9e000000, 0x00370000, 0x00007900, 0x000000b9
    src = dev.upload(data)
    sink = dev.upload(np.zeros(64, np.uint32))
    ttlab_amd._check(dev.lib.ttl_stream_read(dev.ctx, src.ptr, words * 16, sink.ptr), "ttl_stream_read")
    dev.sync()
    expect = 0x9e3779b9 if words >= 2048 else 0
    assert int(sink.download(np.uint32)[0]) == expect
    with pytest.raises(ttlab_amd.TtlError, match="multiple of 16"):
        ttlab_amd._check(dev.lib.ttl_stream_read(dev.ctx, src.ptr, 24, sink.ptr), "ttl_stream_read")
    src.free()
    sink.free()
    dev.close()
