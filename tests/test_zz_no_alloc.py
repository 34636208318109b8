"""ttl_attention_decode_noalloc (the attention entry point that allocates nothing: its
partials live in a static device array) against ttl_attention_decode with a caller
workspace, through the C ABI: bit-identical outputs on consecutive calls, the second
with a smaller capacity and position, both layer parities; the oracle's
attention_from_cache (model.cpp:255-290) within relative L2 1e-5; and the capacity
limit of the static array reported as an error."""
import numpy as np
import pytest

import oracle_lib as O
import ttlab_amd

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    d = ttlab_amd.Device(0)
    yield d
    d.close()


def run_both(dev, layer_index, position, capacity, seed):
    q = O.synth_normal(seed, 1, 4096, sigma=2.0)
    k = O.synth_normal(seed, 2, capacity * 512, sigma=2.0)
    v = O.synth_normal(seed, 3, capacity * 512)
    sinks = O.synth_normal(seed, 4, 64, sigma=2.0)
    bufs = [dev.upload(a) for a in (q, k, v, sinks, np.array([position], np.int32))]
    qb, kb, vb, sb, pb = bufs
    ws = dev.alloc(dev.lib.ttl_attention_workspace_bytes(capacity))
    out_ws, out_na = dev.alloc(4096 * 4), dev.alloc(4096 * 4)
    dev.attention_decode(qb, kb, vb, sb, pb, capacity, layer_index, ws, out_ws)
    dev.attention_decode_noalloc(qb, kb, vb, sb, pb, capacity, layer_index, out_na)
    a, b = out_ws.download(np.float32), out_na.download(np.float32)
    ref = np.empty(4096, np.float32)
    O.lib.orc_attention(q, k, v, sinks, layer_index, position, ref, np.empty(position + 1, np.float32))
    for buf in bufs + [ws, out_ws, out_na]:
        buf.free()
    return a, b, ref


@pytest.mark.parametrize("layer_index", [1, 0])
def test_noalloc_attention_matches_workspace_entry_point(dev, layer_index):
    # two calls in a row on the shared static array, the second smaller
    for position, capacity, seed in ((4095, 4104, 91), (700, 1088, 92)):
        a, b, ref = run_both(dev, layer_index, position, capacity, seed)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), (layer_index, position)
        assert O.rel_l2(b, ref) <= 1e-5


def test_noalloc_attention_rejects_capacity_beyond_static_partials(dev):
    buf = dev.alloc(4096 * 4)
    pos = dev.upload(np.array([0], np.int32))
    with pytest.raises(ttlab_amd.TtlError, match="capacity must be 1..16384"):
        dev.attention_decode_noalloc(buf, buf, buf, buf, pos, 16385, 1, buf)
    buf.free()
    pos.free()
