"""GPU parity of the batched Q8_0 matmul (ttl_matmul_q8_0, MFMA) against the oracle's
matmul_add_q8_0 (tensor.cpp:529-566) and against an f64 product of the dequantized
weights.  Tolerance: relative L2 <= 1e-5 per token (the MFMA sums products of the
exact weights and the activations held to 2^-22 of themselves, in f32 in another
order)."""
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


def magnitude_rows(seed, tokens, cols):
    """Token rows for the per-token shift of the f16 planes: scaled by 2^-100 .. 2^100, a row
    whose values span 2^-40 .. 2^40, one large value among values 2^-60 of it, a zero row,
    rows holding +inf, -inf or a NaN, and one value of 1e30 among values near 1."""
    rs = np.random.RandomState(seed)
    x = rs.standard_normal((tokens, cols)).astype(np.float32)
    scale = [2.0 ** -100, 2.0 ** 100, 2.0 ** -30, 2.0 ** 30, 1.0, 1.0, 1.0, 1.0, 1.0, 1.0, 1.0, 2.0 ** -7]
    x *= np.array(scale[:tokens], np.float32)[:, None]
    x[4] *= np.exp2(rs.randint(-40, 41, cols)).astype(np.float32)
    x[5] *= np.float32(2.0 ** -60)
    x[5, 5] = 1.0
    x[6] = 0.0
    x[7, 17] = np.inf
    x[8, 2000] = np.nan
    x[9, 100] = -np.inf
    x[10, 3] = np.float32(1.0e30)
    return x


def assert_matches_with_nonfinite(got, ref, tokens):
    for p in range(tokens):
        bad = ~np.isfinite(ref[p])
        if not bad.any():
            assert O.rel_l2(got[p], ref[p]) <= TOL, p
            continue
        assert np.array_equal(np.isnan(got[p]), np.isnan(ref[p])), p
        inf = np.isinf(ref[p])
        assert np.array_equal(got[p][inf], ref[p][inf]), p
        ok = np.isfinite(ref[p])
        if ok.any():
            assert O.rel_l2(got[p][ok], ref[p][ok]) <= TOL, p


@pytest.mark.parametrize("cols", [2880, 4096])
def test_q8_matmul_token_magnitudes_and_nonfinite(dev, cols):
    """Each token is scaled by its own power of two before its two f16 planes, and its sums
    are scaled back before the bias: tokens of very different magnitudes, a zero token and
    tokens holding infinities or a NaN against the oracle (finite results within 1e-5 per
    token; NaN and infinite outputs where the oracle's are, with its signs)."""
    rows, tokens = 48, 12
    blocks = O.synth_q8_0(31, cols, rows * cols // 32)
    x = magnitude_rows(32 + cols, tokens, cols)
    bias = O.synth_normal(33, cols, rows, sigma=0.1)
    t = dev.q8_upload(blocks, rows, cols)
    xb, bb, ob = dev.upload(x), dev.upload(bias), dev.alloc(tokens * rows * 4)
    try:
        dev.matmul_q8_0(t, bb, xb, tokens, None, ob)
        got = ob.download(np.float32).reshape(tokens, rows)
        with np.errstate(all="ignore"):
            ref = oracle_matmul(blocks, bias, rows, cols, x, tokens)
        assert np.all(np.isfinite(ref[[0, 1, 2, 3, 4, 5, 6, 11]]))
        assert not np.all(np.isfinite(ref[[7, 8, 9]]))
        assert_matches_with_nonfinite(got, ref, tokens)
        assert np.array_equal(got[6], bias)  # a zero token: the bias alone
    finally:
        for b in (xb, bb, ob):
            b.free()
        t.free()


def expected_shifts(x):
    """The f16-plane shift of each row: 15 - e for its largest finite magnitude m = f 2^e,
    f in [0.5, 1); 0 for a row with no nonzero finite value."""
    a = np.where(np.isfinite(x), np.abs(x), 0.0).max(axis=1)
    return np.where(a > 0, 15 - np.frexp(a)[1], 0).astype(np.int32)


def test_q8_matmul_shifted_matches_unshifted(dev):
    """ttl_rms_norm_rows_shifts writes the rows of ttl_rms_norm_rows, bit for bit, and
    each row's f16-plane shift; ttl_matmul_q8_0_shifted on those shifts gives the bits of
    ttl_matmul_q8_0, which computes them itself."""
    rows, cols, tokens = 64, 2880, 70
    raw = O.synth_normal(61, 0, tokens * cols, sigma=3.0).reshape(tokens, cols)
    raw[9] = 0.0
    norm_w = O.synth_normal(61, 1, cols, sigma=1.0)
    norm_w[:100] *= np.float32(2.0 ** 12)  # some rows' largest value from these columns
    blocks = O.synth_q8_0(62, cols, rows * cols // 32)
    bias = O.synth_normal(63, cols, rows, sigma=0.1)
    t = dev.q8_upload(blocks, rows, cols)
    rb, nb, bb = dev.upload(raw), dev.upload(norm_w), dev.upload(bias)
    xa, xs, sh = dev.alloc(tokens * cols * 4), dev.alloc(tokens * cols * 4), dev.alloc(tokens * 4)
    oa, os_ = dev.alloc(tokens * rows * 4), dev.alloc(tokens * rows * 4)
    try:
        dev.rms_norm_rows(rb, tokens, nb, 1e-5, xa)
        dev.rms_norm_rows(rb, tokens, nb, 1e-5, xs, shifts=sh)
        x = xa.download(np.float32).reshape(tokens, cols)
        assert np.array_equal(x.view(np.uint32), xs.download(np.float32).reshape(tokens, cols).view(np.uint32))
        shifts = sh.download(np.int32)
        assert np.array_equal(shifts, expected_shifts(x))
        assert shifts[9] == 0 and len(set(shifts.tolist())) > 1
        dev.matmul_q8_0(t, bb, xa, tokens, None, oa)
        dev.matmul_q8_0(t, bb, xa, tokens, None, os_, shifts=sh)
        a, b = oa.download(np.float32), os_.download(np.float32)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
        ref = oracle_matmul(blocks, bias, rows, cols, x, tokens)
        for p in range(tokens):
            assert O.rel_l2(b.reshape(tokens, rows)[p], ref[p]) <= TOL, p
    finally:
        for buf in (rb, nb, bb, xa, xs, sh, oa, os_):
            buf.free()
        t.free()


def test_q8_matmul_shifted_rejects_null_shifts(dev):
    import ttlab_amd
    rows, cols, tokens = 16, 2880, 3
    t = dev.q8_upload(O.synth_q8_0(64, 1, rows * cols // 32), rows, cols)
    xb, ob = dev.alloc(tokens * cols * 4), dev.alloc(tokens * rows * 4)
    ws = dev.alloc(dev.lib.ttl_matmul_q8_0_workspace_bytes(tokens, cols))
    try:
        with pytest.raises(ttlab_amd.TtlError, match="null shifts"):
            ttlab_amd._check(dev.lib.ttl_matmul_q8_0_shifted(dev.ctx, t.handle, None, xb.ptr, None, tokens, None,
                                                             ob.ptr, ws.ptr, ws.nbytes), "ttl_matmul_q8_0_shifted")
    finally:
        for b in (xb, ob, ws):
            b.free()
        t.free()
