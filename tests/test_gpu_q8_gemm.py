"""GPU parity of the batched Q8_0 matmul (ttl_matmul_q8_0, MFMA) against the oracle's
matmul_add_q8_0 (tensor.cpp:529-566) and against an f64 product of the dequantized
weights.  Tolerance: relative L2 <= 1e-5 per token (the MFMA sums the same exact
products in f32 in another order)."""
import numpy as np
import pytest

import oracle_lib as O

pytestmark = pytest.mark.gpu
TOL = 1e-5


@pytest.fixture(scope="module")
def dev():
    import ttlab_amd
    d = ttlab_amd.Device(0)
    yield d
    d.close()


def q8_dense(blocks, rows, cols):
    b = blocks.reshape(rows, cols // 32, 34)
    d = b[:, :, :2].copy().view(np.uint16)[..., 0].view(np.float16).astype(np.float64)
    return (b[:, :, 2:].view(np.int8).astype(np.float64) * d[:, :, None]).reshape(rows, cols)


def oracle_matmul(blocks, bias, rows, cols, x, tokens):
    out = np.empty(tokens * rows, np.float32)
    ws, tr = np.empty(tokens, np.float32), np.empty(tokens * cols, np.float32)
    O.lib.orc_matmul_add_q8_0(blocks, bias, rows, cols, np.ascontiguousarray(x, np.float32).ravel(), tokens, out, ws,
                              tr)
    return out.reshape(tokens, rows)


@pytest.mark.parametrize("cols", [2880, 4096])
@pytest.mark.parametrize("tokens", [1, 5, 64, 70, 200])
def test_q8_matmul_matches_oracle(dev, cols, tokens):
    rows = 176  # 11 row tiles: the last workgroup's waves are partly idle
    blocks = O.synth_q8_0(21, cols + tokens, rows * cols // 32)
    x = O.synth_normal(22, cols + tokens, tokens * cols, sigma=1.5).reshape(tokens, cols)
    bias = O.synth_normal(23, cols, rows, sigma=0.1)
    t = dev.q8_upload(blocks, rows, cols)
    xb, bb, ob = dev.upload(x), dev.upload(bias), dev.alloc(tokens * rows * 4)
    dev.matmul_q8_0(t, bb, xb, tokens, None, ob)
    got = ob.download(np.float32).reshape(tokens, rows)
    ref = oracle_matmul(blocks, bias, rows, cols, x, tokens)
    for p in range(tokens):
        assert O.rel_l2(got[p], ref[p]) <= TOL, p
    exact = x.astype(np.float64) @ q8_dense(blocks, rows, cols).T + bias
    assert O.rel_l2(got, exact) < 1e-6
    for b in (xb, bb, ob):
        b.free()
    t.free()


def test_q8_matmul_residual_and_no_bias(dev):
    rows, cols, tokens = 96, 4096, 33
    blocks = O.synth_q8_0(24, 1, rows * cols // 32)
    x = O.synth_normal(25, 1, tokens * cols).reshape(tokens, cols)
    resid = O.synth_normal(26, 1, tokens * rows, sigma=3.0).reshape(tokens, rows)
    t = dev.q8_upload(blocks, rows, cols)
    xb, rb, ob = dev.upload(x), dev.upload(resid), dev.alloc(tokens * rows * 4)
    dev.matmul_q8_0(t, None, xb, tokens, rb, ob)
    ref = oracle_matmul(blocks, np.zeros(rows, np.float32), rows, cols, x, tokens)
    got = ob.download(np.float32).reshape(tokens, rows)
    for p in range(tokens):
        assert O.rel_l2(got[p], resid[p] + ref[p]) <= TOL, p
    for b in (xb, rb, ob):
        b.free()
    t.free()


def test_q8_matmul_rejects_small_workspace(dev):
    import ctypes as C
    import ttlab_amd
    rows, cols, tokens = 16, 2880, 65
    t = dev.q8_upload(O.synth_q8_0(27, 1, rows * cols // 32), rows, cols)
    xb, ob = dev.alloc(tokens * cols * 4), dev.alloc(tokens * rows * 4)
    need = dev.lib.ttl_matmul_q8_0_workspace_bytes(tokens, cols)
    assert need == 2 * dev.lib.ttl_matmul_q8_0_workspace_bytes(64, cols)
    ws = dev.alloc(need // 2)
    with pytest.raises(ttlab_amd.TtlError, match="workspace"):
        ttlab_amd._check(dev.lib.ttl_matmul_q8_0(dev.ctx, t.handle, None, xb.ptr, tokens, None, ob.ptr, ws.ptr,
                                                 ws.nbytes), "ttl_matmul_q8_0")
    for b in (xb, ob, ws):
        b.free()
    t.free()
