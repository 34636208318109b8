"""Device memory helpers of the C ABI (ttl_memcpy_d2d, ttl_fill_bytes) on the GPU."""
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
