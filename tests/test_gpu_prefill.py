"""GPU parity of the batched prefill path (MFMA) against the oracle.

ttl_matmul_mxfp4_selected vs orc_matmul_add_mxfp4_selected_transposed
(tensor.cpp:306-495) and ttl_moe_prefill_experts vs orc_moe_batch_experts
(model.cpp:378-460), and ttl_moe_prefill (router + experts, model.cpp:340-461)
vs orc_moe_batch.  Exact: the reference's selected-matmul known answer
(tests/host_dispatch.cpp:108-126) and the rows it must leave untouched.
Tolerance: relative L2 <= 1e-5 per token and overall (the MFMA sums exact
products in f32 in another order than the reference).  At the full config-2
shape: the oracle on a sample of tokens (a token's result depends on no other
token), and bitwise invariance under token and rank permutations.
"""
import ctypes as C

import numpy as np
import pytest

import oracle_lib as O
import ttlab_amd
from moe_fixtures import N, DeviceLayer, HostLayer

pytestmark = pytest.mark.gpu
TOL = 1e-5


@pytest.fixture(scope="module")
def dev():
    d = ttlab_amd.Device(0)
    yield d
    d.close()


balanced_routing = ttlab_amd.balanced_routing


def kat_matrix():
    expert_bytes = N * 90 * 17
    data = np.zeros(2 * expert_bytes, np.uint8)
    blocks = data[expert_bytes:].reshape(-1, 17)
    blocks[:, 0] = 127
    blocks[:, 1:] = 0x21
    return data


@pytest.mark.parametrize("count", [3, 16, 17, 64, 65])
def test_selected_matmul_reference_kat(dev, count):
    # tests/host_dispatch.cpp:108-126: expert 1, scale 127, bytes 0x21, bias 0.25,
    # tokens[s] = count - s with input (s+1)/2 -> 1080 (s+1) + 0.25; token 0 untouched
    w = dev.mxfp4_upload(kat_matrix(), N, N, 2)
    bias = dev.upload(np.full(2 * N, 0.25, np.float32))
    x = np.zeros((count + 1, N), np.float32)
    tokens = np.array([count - s for s in range(count)], np.int32)
    for s in range(count):
        x[count - s] = (s + 1) * 0.5
    xb, tb = dev.upload(x), dev.upload(tokens)
    out = dev.upload(np.full((count + 1) * N, -1.0, np.float32))
    dev.matmul_mxfp4_selected(w, bias, xb, N, count + 1, tb, count, out, 1)
    got = out.download(np.float32).reshape(count + 1, N)
    assert np.all(got[0] == -1.0)
    for s in range(count):
        assert np.all(got[count - s] == np.float32(1080.0 * (s + 1) + 0.25)), s
    for b in (bias, xb, tb, out):
        b.free()
    w.free()


@pytest.mark.parametrize("count", [1, 5, 64, 70])
def test_selected_matmul_matches_oracle(dev, count):
    rows_x = 80
    blocks = O.synth_mxfp4(0x77000002, 7, 2 * N * 90)
    bias = O.synth_normal(0x77000002, 8, 2 * N, sigma=0.5)
    x = O.synth_normal(0x78000002, 9, rows_x * N).reshape(rows_x, N)
    tokens = np.random.RandomState(count).permutation(rows_x)[:count].astype(np.int32)
    w = dev.mxfp4_upload(blocks, N, N, 2)
    bb, xb, tb = dev.upload(bias), dev.upload(x), dev.upload(tokens)
    out = dev.upload(np.full(rows_x * N, np.nan, np.float32))
    dev.matmul_mxfp4_selected(w, bb, xb, N, rows_x, tb, count, out, 1)
    got = out.download(np.float32).reshape(rows_x, N)
    tr = np.empty(N * count, np.float32)
    O.lib.orc_transpose_selected(N, np.ascontiguousarray(x).ravel(), tokens.astype(np.uintp), count, tr)
    ref = np.full(rows_x * N, np.nan, np.float32)
    ws = np.empty(5 * count, np.float32)
    O.lib.orc_matmul_add_mxfp4_selected_transposed(blocks, bias, N, N, tr, tokens.astype(np.uintp), count, ref, ws,
                                                   1, O.BODY_V4)
    ref = ref.reshape(rows_x, N)
    for t in tokens:
        err = O.rel_l2(got[t], ref[t])
        assert err <= TOL, (t, err)
    untouched = np.setdiff1d(np.arange(rows_x), tokens)
    assert np.all(np.isnan(got[untouched]))
    for b in (bb, xb, tb, out):
        b.free()
    w.free()


def run_prefill(dev, layer, x, idx, w, dtype):
    count, used = idx.shape
    if dtype == ttlab_amd.TTL_DTYPE_BF16:
        bits = (np.ascontiguousarray(x, np.float32).view(np.uint32) >> 16).astype(np.uint16)
        xb = dev.upload(bits)
    else:
        xb = dev.upload(np.ascontiguousarray(x, np.float32))
    ib, wb = dev.upload(idx.astype(np.int32)), dev.upload(w.astype(np.float32))
    out = dev.alloc(count * N * 4)
    ws = dev.alloc(dev.moe_prefill_workspace_bytes(count, layer.desc.experts, used, dtype))
    dev.moe_prefill_experts(layer.desc, xb, dtype, count, ib, wb, out, ws)
    got = out.download(np.float32).reshape(count, N)
    for b in (xb, ib, wb, out, ws):
        b.free()
    return got


def oracle_prefill(host, x, idx, w):
    count = x.shape[0]
    s = host.oracle_struct()
    out = np.empty(count * N, np.float32)
    O.lib.orc_moe_batch_experts(s, np.ascontiguousarray(x, np.float32).ravel(), count,
                                np.ascontiguousarray(idx, np.int64).ravel(), np.ascontiguousarray(w, np.float32).ravel(),
                                out, O.BODY_V4)
    return out.reshape(count, N)


@pytest.fixture(scope="module")
def layer8(dev):
    host = HostLayer(8, 4, biases=True, seed=0x77000012)
    device = DeviceLayer(dev, host)
    yield host, device
    device.free()


@pytest.mark.parametrize("dtype", [ttlab_amd.TTL_DTYPE_BF16, ttlab_amd.TTL_DTYPE_F32])
def test_moe_prefill_experts_matches_oracle(dev, layer8, dtype):
    host, device = layer8
    count = 32
    if dtype == ttlab_amd.TTL_DTYPE_BF16:
        x = O.synth_normal_bf16(0x78000002, 1, count * N, 1.0).reshape(count, N)
    else:
        x = O.synth_normal(0x78000002, 2, count * N).reshape(count, N)
    idx, w = balanced_routing(count, 8, 4, 3)
    got = run_prefill(dev, device, x, idx, w, dtype)
    ref = oracle_prefill(host, x, idx, w)
    assert O.rel_l2(got, ref) <= TOL
    for p in range(count):
        assert O.rel_l2(got[p], ref[p]) <= TOL, p


def test_moe_prefill_intermediates_exact_path(dev, layer8):
    """The exact path's stages read back per pair (ttl_moe_prefill_intermediates):
    the SwiGLU hidden against orc_swiglu of the oracle's gate and up, the down row
    against the oracle's matvec on the device's own hidden (model.cpp:407-447), both
    within 1e-5; a pair with an invalid expert index reads NaN."""
    host, device = layer8
    count, used = 40, 4
    idx, w = balanced_routing(count, 8, used, 21)
    idx[5, 2] = 8  # out of range
    x = O.synth_normal(0x78000131, 0, count * N).reshape(count, N)
    xb, ib, wb = dev.upload(x), dev.upload(idx), dev.upload(w)
    dtype = ttlab_amd.TTL_DTYPE_F32
    ws = dev.alloc(dev.moe_prefill_workspace_bytes(count, 8, used, dtype))
    out, hid, dwn = dev.alloc(count * N * 4), dev.alloc(count * used * N * 4), dev.alloc(count * used * N * 4)
    try:
        dev.moe_prefill_experts(device.desc, xb, dtype, count, ib, wb, out, ws)
        dev.moe_prefill_intermediates(device.desc, dtype, count, ws, hid, dwn)
        hidden = hid.download(np.float32).reshape(count, used, N)
        down = dwn.download(np.float32).reshape(count, used, N)
        assert np.all(np.isnan(hidden[5, 2])) and np.all(np.isnan(down[5, 2]))
        for p, r in ((0, 0), (3, 1), (17, 3), (39, 2), (5, 1)):
            e = int(idx[p, r])
            gate = O.mxfp4_matvec(host.gate, host.gate_b, N, N, x[p], expert=e, body=O.BODY_DEFAULT)
            up = O.mxfp4_matvec(host.up, host.up_b, N, N, x[p], expert=e, body=O.BODY_DEFAULT)
            h = np.empty(N, np.float32)
            O.lib.orc_swiglu(gate, up, N, h)
            assert O.rel_l2(hidden[p, r], h) <= TOL, (p, r)
            d = O.mxfp4_matvec(host.down, host.down_b, N, N, hidden[p, r], expert=e, body=O.BODY_DEFAULT)
            assert O.rel_l2(down[p, r], d) <= TOL, (p, r)
    finally:
        for b in (xb, ib, wb, ws, out, hid, dwn):
            b.free()


@pytest.mark.parametrize("scales,f16", [({}, (True, True, True)),
                                        ({"down": (110, 125)}, (True, True, False)),
                                        ({"down": (126, 145)}, (True, True, False)),
                                        ({"gate": (110, 125)}, (False, True, True)),
                                        ({"up": (126, 145)}, (True, False, True))])
def test_moe_prefill_decode_paths(dev, scales, f16):
    """The unscaled path's operands: with every gate and up scale in E8M0 114..140, f32
    tokens are two f16 planes of x 2^k (k per token) against f16 weights, else three bf16
    planes; with every down scale in that range the hidden is two f16 planes of h x 2^8,
    else three bf16 planes (ttl_mxfp4_f16_exact says which).  All against the oracle within
    1e-5 per token, for f32 and bf16 tokens; the hidden the down GEMM reads
    (ttl_moe_prefill_intermediates) against orc_swiglu of the oracle's gate and up, and the
    down rows against the oracle's matvec on that hidden, within 1e-5."""
    host = HostLayer(8, 4, biases=True, seed=0x77000140, scales=scales)
    device = DeviceLayer(dev, host)
    count, used = 24, 4
    try:
        assert (device.gate.f16_exact, device.up.f16_exact, device.down.f16_exact) == f16
        idx, w = balanced_routing(count, 8, used, 31)
        for dtype in (ttlab_amd.TTL_DTYPE_F32, ttlab_amd.TTL_DTYPE_BF16):
            if dtype == ttlab_amd.TTL_DTYPE_BF16:
                x = O.synth_normal_bf16(0x78000140, 1, count * N, 1.0).reshape(count, N)
            else:
                x = O.synth_normal(0x78000140, 2, count * N).reshape(count, N)
            got = run_prefill(dev, device, x, idx, w, dtype)
            ref = oracle_prefill(host, x, idx, w)
            for p in range(count):
                assert O.rel_l2(got[p], ref[p]) <= TOL, (dtype, p)
        dtype = ttlab_amd.TTL_DTYPE_F32
        x = O.synth_normal(0x78000140, 3, count * N).reshape(count, N)
        xb, ib, wb = dev.upload(x), dev.upload(idx), dev.upload(w)
        ws = dev.alloc(dev.moe_prefill_workspace_bytes(count, 8, used, dtype))
        out, hid, dwn = dev.alloc(count * N * 4), dev.alloc(count * used * N * 4), dev.alloc(count * used * N * 4)
        try:
            dev.moe_prefill_experts(device.desc, xb, dtype, count, ib, wb, out, ws)
            dev.moe_prefill_intermediates(device.desc, dtype, count, ws, hid, dwn)
            hidden = hid.download(np.float32).reshape(count, used, N)
            down = dwn.download(np.float32).reshape(count, used, N)
            for p, r in ((0, 0), (9, 3), (23, 1)):
                e = int(idx[p, r])
                gate = O.mxfp4_matvec(host.gate, host.gate_b, N, N, x[p], expert=e, body=O.BODY_DEFAULT)
                up = O.mxfp4_matvec(host.up, host.up_b, N, N, x[p], expert=e, body=O.BODY_DEFAULT)
                h = np.empty(N, np.float32)
                O.lib.orc_swiglu(gate, up, N, h)
                assert O.rel_l2(hidden[p, r], h) <= TOL, (p, r)
                d = O.mxfp4_matvec(host.down, host.down_b, N, N, hidden[p, r], expert=e, body=O.BODY_DEFAULT)
                assert O.rel_l2(down[p, r], d) <= TOL, (p, r)
        finally:
            for b in (xb, ib, wb, ws, out, hid, dwn):
                b.free()
    finally:
        device.free()


def test_moe_prefill_f32_token_magnitudes(dev, layer8):
    """f32 tokens as two f16 planes, each token scaled by its own power of two: tokens
    scaled by 2^-100 .. 2^100, one whose values span 2^-40 .. 2^40, a zero token and tokens
    holding infinities or a NaN, against the oracle: finite tokens within 1e-5, the others
    NaN and infinite where the oracle's are."""
    host, device = layer8
    assert device.gate.f16_exact and device.up.f16_exact
    count, used = 12, 4
    rs = np.random.RandomState(0x78000150)
    x = rs.standard_normal((count, N)).astype(np.float32)
    x *= np.array([2.0 ** -100, 2.0 ** 100, 2.0 ** -30, 2.0 ** 30] + [1.0] * 8, np.float32)[:, None]
    x[4] *= np.exp2(rs.randint(-40, 41, N)).astype(np.float32)
    x[5] = 0.0
    x[6, 17] = np.inf
    x[7, 2000] = np.nan
    x[8, 100] = -np.inf
    x[9] *= np.float32(2.0 ** -60)
    x[9, 5] = 1.0
    idx, w = balanced_routing(count, 8, used, 41)
    got = run_prefill(dev, device, x, idx, w, ttlab_amd.TTL_DTYPE_F32)
    with np.errstate(all="ignore"):
        ref = oracle_prefill(host, x, idx, w)
    for p in range(count):
        if np.all(np.isfinite(ref[p])):
            assert O.rel_l2(got[p], ref[p]) <= TOL, p
        else:
            assert np.array_equal(np.isnan(got[p]), np.isnan(ref[p])), p
            inf = np.isinf(ref[p])
            assert np.array_equal(got[p][inf], ref[p][inf]), p
    assert not np.all(np.isfinite(ref[[6, 7, 8]]))


def test_moe_prefill_uneven_buckets_and_invalid_index(dev, layer8):
    # experts with 0, 1, 2 and 70 (two tiles) tokens; one pair with an index out of range
    host, device = layer8
    count = 72
    x = O.synth_normal(0x78000002, 4, count * N).reshape(count, N)
    rng = np.random.RandomState(5)
    idx = np.zeros((count, 4), np.int32)
    for p in range(count):
        idx[p] = [7, 3, 6, 5] if p % 36 == 0 else ([7, 3, 2, 5] if p == 1 else [7, 3, 4, 5])
    idx[:, :] = idx[:, rng.permutation(4)]
    w = rng.rand(count, 4).astype(np.float32)
    bad = idx.copy()
    bad[10, 2] = 8
    got = run_prefill(dev, device, x, bad, w, ttlab_amd.TTL_DTYPE_F32)
    assert np.all(np.isnan(got[10]))
    keep = np.setdiff1d(np.arange(count), [10])
    ref = oracle_prefill(host, x[keep], idx[keep], w[keep])
    for j, p in enumerate(keep):
        assert O.rel_l2(got[p], ref[j]) <= TOL, p
    one = run_prefill(dev, device, x[:1], idx[:1], w[:1], ttlab_amd.TTL_DTYPE_F32)
    assert O.rel_l2(one[0], oracle_prefill(host, x[:1], idx[:1], w[:1])[0]) <= TOL


def test_moe_prefill_config2_shape(dev):
    # benchmark config 2: 512 bf16 tokens, 32 experts, top-4 balanced (64 tokens each)
    count = 512
    idx, w = balanced_routing(count, 32, 4, 11)
    sample = np.random.RandomState(12).choice(count, 6, replace=False)
    # host matrices only for the sampled tokens' experts (the device generates all 32)
    host = HostLayer(32, 4, biases=False, seed=0x77000102, fill_experts=idx[sample].ravel())
    device = DeviceLayer(dev, host)
    try:
        x = O.synth_normal_bf16(0x78000102, 0, count * N, 1.0).reshape(count, N)
        got = run_prefill(dev, device, x, idx, w, ttlab_amd.TTL_DTYPE_BF16)
        assert np.all(np.isfinite(got))
        # the oracle on a sample of tokens: each token's result depends on no other token
        ref = oracle_prefill(host, x[sample], idx[sample], w[sample])
        for j, p in enumerate(sample):
            assert O.rel_l2(got[p], ref[j]) <= TOL, p
        # token order and rank order change the buckets, not any per-token sum
        perm = np.random.RandomState(13).permutation(count)
        shuffled = run_prefill(dev, device, x[perm], idx[perm], w[perm], ttlab_amd.TTL_DTYPE_BF16)
        assert np.array_equal(shuffled.view(np.uint32), got[perm].view(np.uint32))
        flipped = run_prefill(dev, device, x, idx[:, ::-1].copy(), w[:, ::-1].copy(), ttlab_amd.TTL_DTYPE_BF16)
        assert np.array_equal(flipped.view(np.uint32), got.view(np.uint32))
    finally:
        device.free()


def test_prefill_rejects_small_workspace(dev, layer8):
    host, device = layer8
    count = 8
    x = dev.alloc(count * N * 4)
    idx, w = balanced_routing(count, 8, 4, 3)
    ib, wb = dev.upload(idx), dev.upload(w)
    out = dev.alloc(count * N * 4)
    need = dev.moe_prefill_workspace_bytes(count, 8, 4, ttlab_amd.TTL_DTYPE_F32)
    assert need > dev.moe_prefill_workspace_bytes(count, 8, 4, ttlab_amd.TTL_DTYPE_BF16)
    small = dev.alloc(dev.moe_prefill_workspace_bytes(count, 8, 4, ttlab_amd.TTL_DTYPE_BF16))
    with pytest.raises(ttlab_amd.TtlError, match="workspace"):
        dev.moe_prefill_experts(device.desc, x, ttlab_amd.TTL_DTYPE_F32, count, ib, wb, out, small)
    for b in (x, ib, wb, out, small):
        b.free()


def run_moe_prefill(dev, layer, x):
    count = x.shape[0]
    used = layer.desc.used
    xb = dev.upload(np.ascontiguousarray(x, np.float32))
    out = dev.alloc(count * N * 4)
    ib, wb = dev.alloc(count * used * 4), dev.alloc(count * used * 4)
    dev.moe_prefill(layer.desc, xb, count, out, ib, wb)
    got = (out.download(np.float32).reshape(count, N), ib.download(np.int32).reshape(count, used),
           wb.download(np.float32).reshape(count, used))
    for b in (xb, out, ib, wb):
        b.free()
    return got


def oracle_routing(host, x):
    """The router of orc_moe_batch: batched F32 matmul (tensor.cpp:497-527), then top-4
    and softmax per token (model.cpp:296-321)."""
    count, E = x.shape[0], host.experts
    logits = np.empty(count * E, np.float32)
    ws, tr = np.empty(count * 5, np.float32), np.empty(count * N, np.float32)
    O.lib.orc_matmul_add_f32(host.router_w, host.router_b, E, N, np.ascontiguousarray(x, np.float32).ravel(), count,
                             logits, ws, tr)
    idx, w = np.empty((count, 4), np.int64), np.empty((count, 4), np.float32)
    for p in range(count):
        O.lib.orc_router_topk(logits[p * E:(p + 1) * E], E, 4, idx[p], w[p])
    return logits.reshape(count, E), idx, w


def test_moe_prefill_router_and_experts_match_oracle(dev, layer8):
    # GptOssModel::moe_batch (model.cpp:340-461): router + top-4 + softmax per token, then experts
    host, device = layer8
    count = 40
    x = O.synth_normal(0x78000002, 6, count * N).reshape(count, N)
    got, idx, w = run_moe_prefill(dev, device, x)
    logits, ref_idx, ref_w = oracle_routing(host, x)
    ref = np.empty(count * N, np.float32)
    O.lib.orc_moe_batch(host.oracle_struct(), x.ravel(), count, ref, O.BODY_V4)
    ref = ref.reshape(count, N)
    # the batch router forms the reference's own f32 sums: the same indices for every token
    assert np.array_equal(idx, ref_idx)
    assert np.allclose(w, ref_w, rtol=1e-5, atol=1e-7)
    for p in range(count):
        assert O.rel_l2(got[p], ref[p]) <= TOL, p
    # the routing it chose, given back to the experts entry point, gives the same bits
    again = run_prefill(dev, device, x, idx, w, ttlab_amd.TTL_DTYPE_F32)
    assert np.array_equal(again.view(np.uint32), got.view(np.uint32))


def test_moe_prefill_fused_matches_unfused(dev, layer8):
    """ttl_moe_prefill_fused, as the layer loop calls it: the normalized rows with the
    f16-plane shifts ttl_rms_norm_rows_shifts wrote for them, and the residual add in the
    combine, gives the bits of ttl_moe_prefill followed by the f32 add residual + moe."""
    host, device = layer8
    count, used = 40, 4
    raw = O.synth_normal(0x78000160, 0, count * N, sigma=3.0).reshape(count, N)
    raw[9] = 0.0
    norm_w = O.synth_normal(0x78000160, 1, N, sigma=1.0)
    resid = O.synth_normal(0x78000160, 2, count * N).reshape(count, N)
    rb, nb, resb = dev.upload(raw), dev.upload(norm_w), dev.upload(resid)
    xb, sh = dev.alloc(count * N * 4), dev.alloc(count * 4)
    oa, ob = dev.alloc(count * N * 4), dev.alloc(count * N * 4)
    ia, wa, ib2, wb2 = (dev.alloc(count * used * 4) for _ in range(4))
    try:
        dev.rms_norm_rows(rb, count, nb, 1e-5, xb, shifts=sh)
        dev.moe_prefill(device.desc, xb, count, oa, ia, wa)
        dev.moe_prefill(device.desc, xb, count, ob, ib2, wb2, shifts=sh, residual=resb)
        moe = oa.download(np.float32).reshape(count, N)
        fused = ob.download(np.float32).reshape(count, N)
        assert np.array_equal(ia.download(np.int32), ib2.download(np.int32))
        assert np.array_equal((resid + moe).view(np.uint32), fused.view(np.uint32))
    finally:
        for b in (rb, nb, resb, xb, sh, oa, ob, ia, wa, ib2, wb2):
            b.free()


def test_moe_prefill_fused_rejects_misaligned_residual(dev, layer8):
    host, device = layer8
    count = 4
    xb, out = dev.alloc(count * N * 4), dev.alloc(count * N * 4)
    resid = dev.alloc(count * N * 4 + 16)
    ws = dev.alloc(dev.lib.ttl_moe_prefill_batch_workspace_bytes(count, 8, 4))
    try:
        with pytest.raises(ttlab_amd.TtlError, match="16-byte aligned"):
            ttlab_amd._check(dev.lib.ttl_moe_prefill_fused(dev.ctx, C.byref(device.desc), xb.ptr, None,
                                                           C.c_void_p(resid.ptr + 4), count, out.ptr, None, None,
                                                           ws.ptr, ws.nbytes), "ttl_moe_prefill_fused")
    finally:
        for b in (xb, out, resid, ws):
            b.free()


def test_moe_prefill_config2_router(dev):
    # 32 experts, 256 f32 tokens: the oracle on a sample of tokens, routing for all
    count = 256
    x = O.synth_normal(0x78000103, 0, count * N).reshape(count, N)
    sample = np.random.RandomState(14).choice(count, 5, replace=False)
    router_only = HostLayer(32, 4, biases=True, seed=0x77000103, fill_experts=[])
    logits, ref_idx, ref_w = oracle_routing(router_only, x)
    host = HostLayer(32, 4, biases=True, seed=0x77000103, fill_experts=ref_idx[sample].ravel())
    device = DeviceLayer(dev, host)
    try:
        got, idx, w = run_moe_prefill(dev, device, x)
        assert np.all(np.isfinite(got))
        assert np.array_equal(idx, ref_idx)
        assert np.allclose(w, ref_w, rtol=1e-5, atol=1e-7)
        for p in sample:
            ref = np.empty(N, np.float32)
            O.lib.orc_moe_batch(host.oracle_struct(), np.ascontiguousarray(x[p]), 1, ref, O.BODY_V4)
            assert O.rel_l2(got[p], ref) <= TOL, p
    finally:
        device.free()


@pytest.mark.parametrize("experts,count", [(32, 1), (32, 129), (128, 70), (192, 3)])
def test_moe_prefill_router_batch_shapes(dev, experts, count):
    """The batch router against the oracle's batched f32 matmul and top-4: one token, a
    partial last group of 64 tokens, gpt-oss-120b's 128 experts and the 192-expert
    maximum (expert groups of four, the last one partial for none of these).  Indices
    exact for every token, weights to f32 rounding."""
    host = HostLayer(experts, 4, biases=True, seed=0x77000140 + experts, fill_experts=[])
    x = O.synth_normal(0x78000140, experts, count * N).reshape(count, N)
    device = DeviceLayer(dev, host)
    try:
        _, idx, w = run_moe_prefill(dev, device, x)
        _, ref_idx, ref_w = oracle_routing(host, x)
        assert np.array_equal(idx, ref_idx)
        assert np.allclose(w, ref_w, rtol=1e-5, atol=1e-7)
    finally:
        device.free()


def test_moe_prefill_router_exact_path_in_a_batch(dev):
    """Router rows 3, 5 and 9 are identical and lead, so every token's logits tie exactly
    and the reference's selection sort settles the order (first position wins, after its
    swaps); two tokens have no tie at the top.  Indices equal the oracle's for every
    token, weights to f32 rounding."""
    count = 40
    host = HostLayer(32, 4, biases=False, seed=0x7700000C, fill_experts=[])  # no bias: the rows tie
    x0 = O.synth_normal(0x78000005, 0, N)
    x = (x0[None, :] + np.float32(0.25) * O.synth_normal(0x78000005, 1, count * N).reshape(count, N))
    x = x.astype(np.float32)
    w = host.router_w.reshape(32, N).copy()
    lead = np.sign(x0).astype(np.float32) * np.float32(0.05)
    for r in (3, 5, 9):
        w[r] = lead
    for p in (7, 21):  # these tokens' inputs flip the lead rows' sign: no tie at the top
        x[p] = -x[p]
    host.router_w = np.ascontiguousarray(w.ravel())
    device = DeviceLayer(dev, host)
    try:
        _, idx, wts = run_moe_prefill(dev, device, x)
        logits, ref_idx, ref_w = oracle_routing(host, x)
        for p in range(count):
            assert list(idx[p]) == list(ref_idx[p]), (p, idx[p], ref_idx[p])
            if p not in (7, 21):
                assert list(idx[p][:3]) == [3, 5, 9], p
        assert np.allclose(wts, ref_w, rtol=1e-5, atol=1e-7)
    finally:
        device.free()


def test_moe_prefill_zero_tokens_and_input_norm(dev, layer8):
    host, device = layer8
    out, xb = dev.alloc(256), dev.alloc(256)
    ws = dev.alloc(dev.lib.ttl_moe_prefill_batch_workspace_bytes(0, 8, 4))
    assert dev.lib.ttl_moe_prefill(dev.ctx, C.byref(device.desc), xb.ptr, 0, out.ptr, None, None, ws.ptr,
                                   ws.nbytes) == 0
    desc = ttlab_amd.MoeLayerDesc.from_buffer_copy(device.desc)
    desc.input_norm = xb.ptr
    with pytest.raises(ttlab_amd.TtlError, match="input_norm"):
        dev.moe_prefill(desc, xb, 1, out)
    for b in (out, ws, xb):
        b.free()
