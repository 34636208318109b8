"""Pins the oracle's compute functions (oracle/ttlab_oracle.c a3-a13).

Known answers are the reference's own (tenstorrent/tt-lab tests/host_dispatch.cpp:92-127,
src/tests.cpp:194-234).  Beyond those: brute force in float64 (numpy), exact
cross-body relations of the reference's two multiversioned bodies, and
hand-derived answers for the selection sort's tie and NaN rules (model.cpp:296-309).
"""
import ctypes as C

import numpy as np
import pytest

import oracle_lib as O

lib = O.lib
N = 2880
BODIES = [O.BODY_DEFAULT, O.BODY_V4, O.BODY_V4_SIMD]

E2M1 = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0])


def decode_f64(blocks, rows, cols):
    """Independent float64 decode: E2M1 magnitude, sign bit 3, times 2^(e-127)."""
    b = blocks.reshape(rows, cols // 32, 17)
    scale = np.ldexp(1.0, b[:, :, 0].astype(np.int64) - 127)
    qs = b[:, :, 1:]
    lo, hi = qs & 15, qs >> 4

    def val(c):
        v = E2M1[c & 7]
        return np.where(c & 8, -v, v)
    w = np.concatenate([val(lo), val(hi)], axis=2) * scale[:, :, None]
    return w.reshape(rows, cols)


def mxfp4_kat_matrix():
    expert_bytes = N * (N // 32) * 17
    data = np.zeros(2 * expert_bytes, np.uint8)
    blocks = data[expert_bytes:].reshape(-1, 17)
    blocks[:, 0] = 127
    blocks[:, 1:] = 0x21
    return data


@pytest.mark.parametrize("body", BODIES)
def test_mxfp4_matvec_reference_kat(body):
    # tests/host_dispatch.cpp:92-107: expert 1, scale 127, bytes 0x21, x = 0.5, bias 0.25 -> 1080.25
    data = mxfp4_kat_matrix()
    bias = np.full(2 * N, 0.25, np.float32)
    x = np.full(N, 0.5, np.float32)
    y = O.mxfp4_matvec(data, bias, N, N, x, expert=1, body=body)
    assert np.all(y == np.float32(1080.25))


@pytest.mark.parametrize("body", BODIES)
@pytest.mark.parametrize("count", [3, 16, 17])
def test_mxfp4_selected_matmul_reference_kat(body, count):
    # tests/host_dispatch.cpp:108-126: tokens[s] = count - s, input (s+1)/2,
    # result 1080 (s+1) + 0.25, token 0's row untouched (-1)
    data = mxfp4_kat_matrix()
    bias = np.full(2 * N, 0.25, np.float32)
    tokens = np.array([count - s for s in range(count)], np.uintp)
    transposed = np.empty(N * count, np.float32)
    for s in range(count):
        transposed[s::count] = (s + 1) * 0.5
    workspace = np.empty(4 * count + 8, np.float32)
    out = np.full((count + 1) * N, -1.0, np.float32)
    lib.orc_matmul_add_mxfp4_selected_transposed(data, bias, N, N, transposed, tokens, count, out, workspace, 1,
                                                 body)
    out = out.reshape(count + 1, N)
    assert np.all(out[0] == -1.0)
    for s in range(count):
        assert np.all(out[count - s] == np.float32(1080.0 * (s + 1) + 0.25))


def test_f32_matvec_and_rmsnorm_kats():
    # src/tests.cpp:194-212
    w = np.array([1, 2, 3, 4], np.float32)
    bias = np.array([10, 20], np.float32)
    x = np.array([5, 6], np.float32)
    y = np.empty(2, np.float32)
    lib.orc_matvec_add_f32(w, bias, 2, 2, x, y)
    assert y[0] == 27 and y[1] == 59
    out = np.empty(2, np.float32)
    lib.orc_rms_norm(np.array([3, 4], np.float32), np.array([2, 3], np.float32), 2, 0.0, out)
    scale = 1.0 / np.sqrt(12.5)
    assert abs(out[0] - 6 * scale) <= 1e-6 and abs(out[1] - 12 * scale) <= 1e-6


def test_f32_router_sums_are_sequential_from_the_bias():
    """matvec_add_f32 and matmul_add_f32 (tensor.cpp:186-200, 497-527): per (row, token)
    the sum starts at the bias and adds the rounded f32 products one column after the
    other -- numpy's float32 cumulative sum of [bias, w0 x0, w1 x1, ...] bit for bit."""
    rng = np.random.default_rng(31)
    rows, cols, tokens = 5, 2880, 3
    w = rng.standard_normal((rows, cols)).astype(np.float32)
    bias = rng.standard_normal(rows).astype(np.float32)
    x = rng.standard_normal((tokens, cols)).astype(np.float32)
    expect = np.empty((tokens, rows), np.float32)
    for t in range(tokens):
        for r in range(rows):
            terms = np.concatenate([bias[r:r + 1], (w[r] * x[t]).astype(np.float32)])
            expect[t, r] = np.cumsum(terms, dtype=np.float32)[-1]
    out = np.empty(tokens * rows, np.float32)
    ws, tr = np.empty(tokens, np.float32), np.empty(tokens * cols, np.float32)
    lib.orc_matmul_add_f32(np.ascontiguousarray(w.ravel()), bias, rows, cols, np.ascontiguousarray(x.ravel()), tokens,
                           out, ws, tr)
    assert np.array_equal(out.reshape(tokens, rows).view(np.uint32), expect.view(np.uint32))
    for t in range(tokens):
        y = np.empty(rows, np.float32)
        lib.orc_matvec_add_f32(np.ascontiguousarray(w.ravel()), bias, rows, cols, np.ascontiguousarray(x[t]), y)
        assert np.array_equal(y.view(np.uint32), expect[t].view(np.uint32))
    # a pairwise or fused sum would differ somewhere: the order is what is pinned
    assert not np.array_equal(expect, (x @ w.T + bias).astype(np.float32))


def test_q8_0_matvec_kats():
    # src/tests.cpp:214-234
    data = np.zeros(68, np.uint8)
    data[0:2] = [0x00, 0x3C]
    data[34:36] = [0x00, 0x3C]
    data[2:34] = 1
    data[36:68] = 0xFF
    x = np.ones(32, np.float32)
    y = np.empty(2, np.float32)
    lib.orc_matvec_q8_0(data, 2, 32, x, y)
    assert y[0] == 32 and y[1] == -32
    lib.orc_matvec_add_q8_0(data, np.array([10, 20], np.float32), 2, 32, x, y)
    assert y[0] == 42 and y[1] == -12


def test_mxfp4_matvec_brute_force_all_bodies():
    rows, cols = 256, N
    w = O.synth_mxfp4(11, 0, rows * cols // 32)
    x = O.synth_normal(12, 0, cols)
    bias = O.synth_normal(13, 0, rows, sigma=0.1)
    exact = decode_f64(w, rows, cols) @ x.astype(np.float64) + bias
    outs = [O.mxfp4_matvec(w, bias, rows, cols, x, body=b) for b in BODIES]
    for y in outs:
        assert O.rel_l2(y, exact) < 1e-6
    # v4 restated lane by lane and v4 with AVX-512 intrinsics are the same arithmetic
    if O.has_avx512():
        assert np.array_equal(outs[1].view(np.uint32), outs[2].view(np.uint32))
    # the default and v4 bodies round differently (fused vs unfused), as in the reference
    assert not np.array_equal(outs[0], outs[1])


def test_mxfp4_matvec_default_is_sequential_unfused():
    """Single-row check: the default body equals a float32 sequential unfused loop over
    (block, i, low, high) with weights decoded independently."""
    cols = 96
    w = O.synth_mxfp4(21, 0, cols // 32)
    x = O.synth_normal(22, 0, cols)
    dense = decode_f64(w, 1, cols)[0].astype(np.float32)
    acc = np.float32(0.125)
    for b in range(cols // 32):
        for i in range(16):
            acc = np.float32(acc + np.float32(dense[32 * b + i] * x[32 * b + i]))
            acc = np.float32(acc + np.float32(dense[32 * b + 16 + i] * x[32 * b + 16 + i]))
    y = O.mxfp4_matvec(w, np.array([0.125] * 4, np.float32), 1, cols, x, body=O.BODY_DEFAULT)
    assert y[0] == acc


def test_selected_matmul_matches_matvec_default_and_brute_force():
    rows, cols, count = 64, 320, 7
    w = O.synth_mxfp4(31, 0, 2 * rows * cols // 32)
    bias = O.synth_normal(32, 0, 2 * rows, sigma=0.1)
    x = O.synth_normal(33, 0, 10 * cols).reshape(10, cols)
    tokens = np.array([9, 2, 5, 0, 7, 3, 1], np.uintp)
    tr = np.empty(cols * count, np.float32)
    lib.orc_transpose_selected(cols, np.ascontiguousarray(x), tokens, count, tr)
    for body in BODIES:
        out = np.full(10 * rows, np.nan, np.float32)
        ws = np.empty(4 * count, np.float32)
        lib.orc_matmul_add_mxfp4_selected_transposed(w, bias, rows, cols, tr, tokens, count, out, ws, 1, body)
        out = out.reshape(10, rows)
        dense = decode_f64(w[rows * cols // 32 * 17:], rows, cols)
        for t in tokens:
            exact = dense @ x[t].astype(np.float64) + bias[rows:]
            assert O.rel_l2(out[t], exact) < 1e-6
            if body == O.BODY_DEFAULT:
                # the default matmul walks the same order as the default matvec
                mv = O.mxfp4_matvec(w, bias, rows, cols, x[t], expert=1, body=O.BODY_DEFAULT)
                assert np.array_equal(out[t], mv)
        untouched = [t for t in range(10) if t not in tokens]
        assert np.all(np.isnan(out[untouched]))


def test_router_topk_distinct_values_against_sort():
    rng = np.random.default_rng(3)
    for _ in range(200):
        logits = rng.standard_normal(32).astype(np.float32)
        idx, w = O.router_topk(logits)
        assert list(idx) == list(np.argsort(-logits.astype(np.float64), kind="stable")[:4])
        top = logits[idx].astype(np.float64)
        soft = np.exp(top - top.max())
        soft /= soft.sum()
        assert np.allclose(w, soft, rtol=1e-6, atol=0)


def test_router_topk_tie_and_nan_rules_hand_derived():
    def run(values, k):
        logits = np.full(32, -100.0, np.float32)
        logits[:len(values)] = values
        return list(O.router_topk(logits, k)[0])
    # all equal: nothing is strictly greater, positions are taken in order
    assert list(O.router_topk(np.zeros(32, np.float32))[0]) == [0, 1, 2, 3]
    # [5, 5, 9]: step 0 swaps 9 into position 0 and expert 0 into position 2, so the
    # tie between experts 0 and 1 resolves to expert 1 first (not the lower index)
    assert run([5, 5, 9], 3) == [2, 1, 0]
    # a NaN at the current position is never displaced ('x > NaN' is false)
    assert run([np.nan, 3, 2, 1], 2) == [0, 1]
    assert run([1, np.nan, 3, 2], 2) == [2, 1]
    # a NaN elsewhere is never selected ahead of numbers
    assert run([1, 2, np.nan, 3], 2) == [3, 1]


def test_swiglu_against_float64_and_special_values():
    rng = np.random.default_rng(4)
    g = (rng.standard_normal(4096) * 6).astype(np.float32)
    u = (rng.standard_normal(4096) * 6).astype(np.float32)
    h = np.empty_like(g)
    lib.orc_swiglu(g, u, g.size, h)
    x = np.minimum(g.astype(np.float64), 7.0)
    y = np.clip(u.astype(np.float64), -7.0, 7.0)
    c = float(np.float32(-1.702))
    ref = x / (1.0 + np.exp(c * x)) * (y + 1.0)
    # exp amplifies the rounding of its float32 argument c*x by |c*x|
    tol = 4e-7 * (4.0 + np.abs(c * x))
    assert np.all(np.abs(h - ref) <= tol * np.abs(ref) + 1e-37)
    special_g = np.array([100.0, np.nan, -200.0, 0.0], np.float32)
    special_u = np.array([100.0, 1.0, 1.0, -100.0], np.float32)
    h = np.empty(4, np.float32)
    lib.orc_swiglu(special_g, special_u, 4, h)
    assert h[0] == np.float32(np.float32(7.0 / (1.0 + np.exp(np.float32(-1.702 * 7.0)))) * 8.0) or \
        abs(h[0] - 7.0 / (1.0 + np.exp(-1.702 * 7.0)) * 8.0) < 1e-5
    assert np.isnan(h[1])  # NaN gate propagates through std::min
    assert h[2] == 0.0     # exp overflow -> x / inf -> -0
    assert h[3] == 0.0     # x = 0


def test_rms_norm_against_float64():
    x = O.synth_normal(41, 0, N, sigma=3.0)
    w = O.synth_normal(42, 0, N, mean=1.0, sigma=0.1)
    out = np.empty(N, np.float32)
    lib.orc_rms_norm(x, w, N, 1e-5, out)
    xd = x.astype(np.float64)
    ref = xd / np.sqrt(np.mean(xd * xd) + 1e-5) * w
    assert O.rel_l2(out, ref) < 1e-6


def test_q8_0_matvec_and_matmul_against_float64():
    rows, cols = 128, N
    q = O.synth_q8_0(51, 0, rows * cols // 32)
    x = O.synth_normal(52, 0, 3 * cols).reshape(3, cols)
    bias = O.synth_normal(53, 0, rows, sigma=0.1)
    blocks = q.reshape(rows, cols // 32, 34)
    d = blocks[:, :, :2].copy().view(np.uint16)[..., 0].view(np.float16).astype(np.float64)
    qs = blocks[:, :, 2:].view(np.int8).astype(np.float64)
    dense = (qs * d[:, :, None]).reshape(rows, cols)
    y = np.empty(rows, np.float32)
    lib.orc_matvec_add_q8_0(q, bias, rows, cols, x[0], y)
    assert O.rel_l2(y, dense @ x[0] + bias) < 1e-6
    out = np.empty(3 * rows, np.float32)
    ws = np.empty(3, np.float32)
    tr = np.empty(3 * cols, np.float32)
    lib.orc_matmul_add_q8_0(q, bias, rows, cols, np.ascontiguousarray(x), 3, out, ws, tr)
    assert O.rel_l2(out.reshape(3, rows), (dense @ x.T.astype(np.float64)).T + bias) < 1e-6
    emb = np.empty(cols, np.float32)
    lib.orc_load_token_embedding_q8_0(q, cols, 5, emb)
    assert np.array_equal(emb, dense[5].astype(np.float32))


def test_bf16_matvec_against_float64():
    rows, cols = 64, 512
    w = O.synth_bf16(61, 0, rows * cols)
    x = O.synth_normal(62, 0, cols)
    y = np.empty(rows, np.float32)
    lib.orc_matvec_bf16(w, rows, cols, x, y)
    dense = (w.astype(np.uint32) << 16).view(np.float32).reshape(rows, cols).astype(np.float64)
    assert O.rel_l2(y, dense @ x) < 1e-6


def test_greedy_first_max_and_nan():
    assert lib.orc_greedy(np.array([1, 3, 3, 2], np.float32), 4) == 1
    assert lib.orc_greedy(np.array([np.nan, 3, 9], np.float32), 3) == 0
    assert lib.orc_greedy(np.array([1, np.nan, 9, 9], np.float32), 4) == 2
    assert lib.orc_greedy(np.array([-0.0, 0.0], np.float32), 2) == 0


def test_rope_frequencies_against_float64():
    f = np.empty(32, np.float32)
    lib.orc_rope_frequencies(f)
    base, head = 150000.0, 64.0
    corr = head * np.log(4096 / (32 * 2 * np.pi)) / (2 * np.log(base))
    corr_slow = head * np.log(4096 / (1 * 2 * np.pi)) / (2 * np.log(base))
    low, high = max(0.0, np.floor(corr)), min(63.0, np.ceil(corr_slow))
    pair = np.arange(32)
    theta = base ** (-(2.0 * pair) / head)
    ramp = 1 - np.clip((pair - low) / max(0.001, high - low), 0, 1)
    ref = theta / 32 * (1 - ramp) + theta * ramp
    assert np.allclose(f, ref, rtol=1e-5)
    # the extremes are pure extrapolation (pair 0) and pure interpolation (last pair)
    assert abs(f[0] - 1.0) < 1e-6
    assert abs(f[31] / (theta[31] / 32) - 1) < 1e-5


def test_apply_rope_rotation_property():
    f = np.empty(32, np.float32)
    lib.orc_rope_frequencies(f)
    v = O.synth_normal(71, 0, 8 * 64)
    r = v.copy()
    lib.orc_apply_rope(r, 8, 1234, f)
    mag = 1 + 0.1 * np.log(32.0)
    v2 = v.reshape(8, 2, 32).astype(np.float64)
    r2 = r.reshape(8, 2, 32).astype(np.float64)
    # each (d, d+32) pair is rotated by 1234*f[d] and scaled by 1 + 0.1 ln 32
    ang = 1234.0 * f.astype(np.float64)
    ref0 = (v2[:, 0] * np.cos(ang) - v2[:, 1] * np.sin(ang)) * mag
    ref1 = (v2[:, 0] * np.sin(ang) + v2[:, 1] * np.cos(ang)) * mag
    assert O.rel_l2(r2[:, 0], ref0) < 1e-5 and O.rel_l2(r2[:, 1], ref1) < 1e-5


@pytest.mark.parametrize("layer_index,position", [(0, 5), (1, 5), (0, 300), (1, 300)])
def test_attention_against_float64(layer_index, position):
    T = position + 1
    q = O.synth_normal(81, 0, 64 * 64)
    k = O.synth_normal(82, 0, T * 512)
    v = O.synth_normal(83, 0, T * 512)
    sinks = O.synth_normal(84, 0, 64)
    out = np.empty(64 * 64, np.float32)
    scores = np.empty(T, np.float32)
    lib.orc_attention(q, k, v, sinks, layer_index, position, out, scores)
    first = position + 1 - 128 if (layer_index % 2 == 0 and position + 1 > 128) else 0
    K = k.reshape(T, 8, 64)[first:].astype(np.float64)
    V = v.reshape(T, 8, 64)[first:].astype(np.float64)
    Q = q.reshape(64, 64).astype(np.float64)
    ref = np.empty((64, 64))
    for h in range(64):
        s = K[:, h // 8] @ Q[h] / 8.0
        m = max(s.max(), sinks[h])
        e = np.exp(s - m)
        ref[h] = (e / (e.sum() + np.exp(sinks[h] - m))) @ V[:, h // 8]
    assert O.rel_l2(out, ref.ravel()) < 1e-5


# ---- a9 prefill: GptOssModel::moe_batch's experts (model.cpp:378-460) ----------------

def _small_moe(hidden=64, experts=6, used=2, seed=51):
    """A gpt-oss-shaped MoE layer at a small width, host arrays kept alive on the struct."""
    keep = {}
    keep["router_w"] = O.synth_normal(seed, 1, experts * hidden, sigma=0.1)
    keep["router_b"] = O.synth_normal(seed, 2, experts, sigma=0.1)
    for i, name in enumerate(("gate", "up", "down")):
        keep[name] = O.synth_mxfp4(seed, 10 + i, experts * hidden * hidden // 32)
        keep[name + "_b"] = O.synth_normal(seed, 20 + i, experts * hidden, sigma=0.5)
    s = O.MoeLayer()
    s.hidden, s.expert_hidden, s.experts, s.used = hidden, hidden, experts, used
    s.router_weight, s.router_bias = keep["router_w"].ctypes.data, keep["router_b"].ctypes.data
    s.gate_weight, s.gate_bias = keep["gate"].ctypes.data, keep["gate_b"].ctypes.data
    s.up_weight, s.up_bias = keep["up"].ctypes.data, keep["up_b"].ctypes.data
    s.down_weight, s.down_bias = keep["down"].ctypes.data, keep["down_b"].ctypes.data
    s._keep = keep
    return s


def _routing(count, experts, used, seed):
    rng = np.random.RandomState(seed)
    idx = np.stack([rng.choice(experts, used, replace=False) for _ in range(count)]).astype(np.int64)
    logits = rng.randn(count, used)
    w = np.exp(logits - logits.max(1, keepdims=True))
    return idx, (w / w.sum(1, keepdims=True)).astype(np.float32)


def _moe_batch_experts(s, x, idx, w, body=O.BODY_V4):
    count = x.shape[0]
    out = np.empty(count * s.hidden, np.float32)
    lib.orc_moe_batch_experts(C.byref(s), np.ascontiguousarray(x, np.float32).ravel(), count,
                              np.ascontiguousarray(idx, np.int64).ravel(), np.ascontiguousarray(w, np.float32).ravel(),
                              out, body)
    return out.reshape(count, s.hidden)


def _brute_force_moe(s, x, idx, w):
    H = s.hidden
    k = s._keep
    dense = {n: decode_f64(k[n], s.experts * H, H).reshape(s.experts, H, H) for n in ("gate", "up", "down")}
    bias = {n: k[n + "_b"].astype(np.float64).reshape(s.experts, H) for n in ("gate", "up", "down")}
    out = np.zeros((x.shape[0], H))
    for p in range(x.shape[0]):
        for r in range(idx.shape[1]):
            e = idx[p, r]
            g = dense["gate"][e] @ x[p] + bias["gate"][e]
            u = dense["up"][e] @ x[p] + bias["up"][e]
            xg = np.minimum(g, 7.0)
            h = xg / (1.0 + np.exp(-1.702 * xg)) * (np.clip(u, -7.0, 7.0) + 1.0)
            out[p] += w[p, r] * (dense["down"][e] @ h + bias["down"][e])
    return out



@pytest.mark.parametrize("count", [3, 40])  # 40 tokens: buckets above 4 take the selected matmul
def test_moe_batch_experts_brute_force(count):
    s = _small_moe()
    x = O.synth_normal(52, 0, count * s.hidden).reshape(count, s.hidden)
    idx, w = _routing(count, s.experts, s.used, 53)
    got = _moe_batch_experts(s, x, idx, w)
    exact = _brute_force_moe(s, x.astype(np.float64), idx, w.astype(np.float64))
    assert O.rel_l2(got, exact) < 1e-5
    for p in range(count):
        assert O.rel_l2(got[p], exact[p]) < 1e-5


def test_moe_batch_experts_combines_in_expert_order():
    # model.cpp:450-459 adds each token's expert outputs in ascending expert index, so
    # permuting a token's ranks (with their weights) leaves the result bit-identical,
    # and permuting the tokens permutes the rows bit for bit (every per-(row, token)
    # sum is independent of the other tokens).
    s = _small_moe()
    count = 40
    x = O.synth_normal(54, 0, count * s.hidden).reshape(count, s.hidden)
    idx, w = _routing(count, s.experts, s.used, 55)
    base = _moe_batch_experts(s, x, idx, w)
    flip = idx[:, ::-1].copy(), w[:, ::-1].copy()
    assert np.array_equal(base.view(np.uint32), _moe_batch_experts(s, x, *flip).view(np.uint32))
    perm = np.random.RandomState(56).permutation(count)
    shuffled = _moe_batch_experts(s, x[perm], idx[perm], w[perm])
    assert np.array_equal(base[perm].view(np.uint32), shuffled.view(np.uint32))


def test_moe_batch_routes_then_runs_experts():
    # orc_moe_batch = F32 router matmul + per-token top-k, then orc_moe_batch_experts
    s = _small_moe()
    count = 12
    x = O.synth_normal(57, 0, count * s.hidden).reshape(count, s.hidden)
    out = np.empty(count * s.hidden, np.float32)
    lib.orc_moe_batch(C.byref(s), np.ascontiguousarray(x).ravel(), count, out, O.BODY_V4)
    k = s._keep
    idx = np.empty((count, s.used), np.int64)
    w = np.empty((count, s.used), np.float32)
    for p in range(count):
        logits = np.empty(s.experts, np.float32)
        lib.orc_matvec_add_f32(k["router_w"], k["router_b"], s.experts, s.hidden, np.ascontiguousarray(x[p]), logits)
        idx[p], w[p] = O.router_topk(logits, s.used)
    assert np.array_equal(out.reshape(count, s.hidden), _moe_batch_experts(s, x, idx, w))


@pytest.mark.parametrize("layer_index", [0, 1])
def test_layer_prefill_matches_token_by_token_and_chunks(layer_index):
    """orc_layer_prefill (model.cpp:484-553, batched matmuls and moe_batch) against
    orc_layer_forward per token (model.cpp:571-595, matvecs and moe): the same
    arithmetic summed in other orders, so rel L2 <= 1e-5 per token unless the routing
    is a near-tie.  A prefill split into chunks (positions 0..2, then 3..5) writes the
    same keys and values bit for bit (the Q8_0 matmul sums each token on its own); its
    outputs agree to tolerance only, since moe_batch sends an expert with at most 4
    tokens through the matvec and others through the selected matmul
    (model.cpp:404,435), which round differently."""
    from model_fixtures import HostModelLayer
    host = HostModelLayer(0x77000031, layer_index, 8)
    s = host.struct()
    count, KW, N = 6, 512, 2880
    freqs = np.empty(32, np.float32)
    lib.orc_rope_frequencies(freqs)
    x = O.synth_normal(0x78000031, layer_index, count * N, sigma=1.0)
    kc, vc = np.zeros(count * KW, np.float32), np.zeros(count * KW, np.float32)
    out = np.empty(count * N, np.float32)
    lib.orc_layer_prefill(C.byref(s), layer_index, 0, count, x, freqs, kc, vc, O.BODY_V4, out, None)
    kc2, vc2 = np.zeros(count * KW, np.float32), np.zeros(count * KW, np.float32)
    out2 = np.empty(count * N, np.float32)
    lib.orc_layer_prefill(C.byref(s), layer_index, 0, 3, x[:3 * N], freqs, kc2, vc2, O.BODY_V4, out2[:3 * N], None)
    lib.orc_layer_prefill(C.byref(s), layer_index, 3, 3, x[3 * N:], freqs, kc2, vc2, O.BODY_V4, out2[3 * N:], None)
    assert np.array_equal(kc.view(np.uint32), kc2.view(np.uint32))
    assert np.array_equal(vc.view(np.uint32), vc2.view(np.uint32))
    for p in range(count):
        assert O.rel_l2(out2[p * N:(p + 1) * N], out[p * N:(p + 1) * N]) <= 1e-5, p
    kc3, vc3 = np.zeros(count * KW, np.float32), np.zeros(count * KW, np.float32)
    for p in range(count):
        ref = np.empty(N, np.float32)
        router = np.empty(8, np.float32)
        idx, w = np.empty(4, np.int64), np.empty(4, np.float32)
        q, att, res = np.empty(4096, np.float32), np.empty(4096, np.float32), np.empty(N, np.float32)
        lib.orc_layer_forward(C.byref(s), layer_index, p, np.ascontiguousarray(x[p * N:(p + 1) * N]), freqs, kc3,
                              vc3, O.BODY_V4, ref, q, att, res, router, idx, w)
        assert O.rel_l2(kc[p * KW:(p + 1) * KW], kc3[p * KW:(p + 1) * KW]) <= 1e-5
        top = np.sort(router.astype(np.float64))[::-1]
        if np.any(np.abs(np.diff(top[:5])) < 1e-4):
            continue
        assert O.rel_l2(out[p * N:(p + 1) * N], ref) <= 1e-5, p


def test_mxfp4_overflow_band_is_order_dependent():
    """With E8M0 240..250 and x ~ N(0, 1), partial sums cross 2^128 in some rows, and
    whether a row ends finite, infinite or NaN depends on the summation order: the
    reference's own two bodies (default: one weight at a time; AVX-512: x scaled per
    block, 16 lanes, tree reduction) disagree on many rows.  So no implementation that
    sums in another order can match "the reference" there row by row; the GPU tests
    compare bodies and GPU only where every result overflows (E8M0 >= 250) or none does."""
    blocks = O.synth_mxfp4(0x77000000, 0, N * 90, 240, 250)
    x = O.synth_normal(0x78000000, 0, N)
    zero = np.zeros(N, np.float32)
    d = O.mxfp4_matvec(blocks, zero, N, N, x, expert=0, body=O.BODY_DEFAULT)
    v = O.mxfp4_matvec(blocks, zero, N, N, x, expert=0, body=O.BODY_V4)
    kinds = lambda a: np.where(np.isnan(a), 0, np.where(np.isinf(a), 1, 2))
    assert np.count_nonzero(kinds(d) != kinds(v)) > N // 10
    assert np.isfinite(d).any() and np.isinf(d).any()
