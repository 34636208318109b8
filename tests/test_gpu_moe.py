"""GPU parity of the MoE decode path (router + top-k + SwiGLU + combine) against the oracle.

Bit-exact: top-k expert indices (fast certified path and exact path), router logits
on the exact path.  Tolerance: relative L2 <= 1e-5 for the layer output.
"""
import numpy as np
import pytest

import oracle_lib as O
import ttlab_amd
from moe_fixtures import N, X_SEED, DeviceLayer, HostLayer

pytestmark = pytest.mark.gpu
TOL = 1e-5


@pytest.fixture(scope="module")
def dev():
    d = ttlab_amd.Device(0)
    yield d
    d.close()


@pytest.fixture(scope="module")
def layer32(dev):
    host = HostLayer(32, 4, biases=False)
    device = DeviceLayer(dev, host)
    yield host, device
    device.free()


def oracle_router(w, b, x, k):
    logits = np.empty(b.size, np.float32)
    O.lib.orc_matvec_add_f32(w, b, b.size, N, np.ascontiguousarray(x, np.float32), logits)
    idx, wts = O.router_topk(logits, k)
    return logits, idx, wts


def run_router(dev, wbuf, bbuf, experts, x, k, force_exact=False):
    xb = dev.upload(x)
    lb, ib, wb = dev.alloc(experts * 4), dev.alloc(k * 4), dev.alloc(k * 4)
    dev.router_topk(wbuf, bbuf, experts, xb, k, lb, ib, wb, force_exact)
    out = lb.download(np.float32), ib.download(np.int32), wb.download(np.float32)
    for b in (xb, lb, ib, wb):
        b.free()
    return out


# 7, 32, 128, 192: the exact path's workgroup tiles hold 2, 8 and 12 float4 pieces per
# thread (at most 32, 128 and 192 rows)
@pytest.mark.parametrize("experts", [7, 32, 128, 192])
def test_router_fast_and_exact_paths_match_reference(dev, experts):
    w = O.synth_normal_bf16(0x77000009, 20, experts * N, 0.02)
    b = O.synth_normal(0x77000009, 21, experts, sigma=0.05)
    wb, bb = dev.upload(w), dev.upload(b)
    before = dev.router_exact_count()
    certified = 0
    for token in range(24):
        x = O.synth_normal(X_SEED, 100 + token, N)
        ref_logits, ref_idx, ref_w = oracle_router(w, b, x, 4)
        logits, idx, wts = run_router(dev, wb, bb, experts, x, 4)
        assert list(idx) == list(ref_idx), (token, idx, ref_idx)
        assert np.allclose(wts, ref_w, rtol=1e-5, atol=0)
        assert O.rel_l2(logits, ref_logits) < 1e-5
        # the exact path reproduces the reference's sequential f32 sums bit for bit
        logits_x, idx_x, wts_x = run_router(dev, wb, bb, experts, x, 4, force_exact=True)
        assert np.array_equal(logits_x.view(np.uint32), ref_logits.view(np.uint32))
        assert list(idx_x) == list(ref_idx)
        assert np.allclose(wts_x, ref_w, rtol=5e-7, atol=0)
    exact_calls = dev.router_exact_count() - before
    certified = 48 - exact_calls
    print(f"experts {experts}: {exact_calls - 24} of 24 unforced calls needed the exact path")
    assert exact_calls >= 24
    assert certified >= 12  # random logits are rarely within the rounding bound
    wb.free()
    bb.free()


def test_router_exact_ties_follow_reference_selection_sort(dev):
    """Rows 3, 5 and 9 are identical and lead the ranking, so their logits tie exactly.
    The fast path cannot separate them and the kernel falls back to the reference's
    selection sort, whose swaps order the tie as the reference does."""
    experts = 32
    w = O.synth_normal_bf16(0x7700000A, 20, experts * N, 0.02).reshape(experts, N)
    x = O.synth_normal(X_SEED, 7, N)
    lead = np.sign(x).astype(np.float32) * np.float32(0.05)
    for r in (3, 5, 9):
        w[r] = lead
    w = np.ascontiguousarray(w.ravel())
    b = np.zeros(experts, np.float32)
    b[0] = np.float32(0.0)
    wb, bb = dev.upload(w), dev.upload(b)
    before = dev.router_exact_count()
    ref_logits, ref_idx, ref_w = oracle_router(w, b, x, 4)
    assert ref_logits[3] == ref_logits[5] == ref_logits[9]
    logits, idx, wts = run_router(dev, wb, bb, experts, x, 4)
    assert dev.router_exact_count() == before + 1
    assert list(idx) == list(ref_idx)
    assert list(idx[:3]) == [3, 5, 9]
    assert np.array_equal(logits.view(np.uint32), ref_logits.view(np.uint32))
    wb.free()
    bb.free()


def test_moe_decode_exact_routing_inside_gateup(dev):
    """The MoE decode selects its experts inside the gate/up kernel.  With router rows
    3, 5 and 9 identical their logits tie exactly, so no workgroup can certify the
    ranking: every one recomputes the logits in the reference's order and replays its
    selection sort.  The routing must be the reference's and the layer match the oracle."""
    x = O.synth_normal(X_SEED, 7, N)
    lead = np.sign(x).astype(np.float32) * np.float32(0.05)
    router_only = HostLayer(32, 4, biases=False, seed=0x7700000B, fill_experts=[])
    w = router_only.router_w.reshape(32, N).copy()
    for r in (3, 5, 9):
        w[r] = lead
    w = np.ascontiguousarray(w.ravel())
    logits = np.empty(32, np.float32)
    O.lib.orc_matvec_add_f32(w, router_only.router_b, 32, N, x, logits)
    ref_idx, ref_w = O.router_topk(logits, 4)
    assert logits[3] == logits[5] == logits[9] and list(ref_idx[:3]) == [3, 5, 9]
    host = HostLayer(32, 4, biases=False, seed=0x7700000B, fill_experts=ref_idx)
    host.router_w = w
    device = DeviceLayer(dev, host)
    xb, out = dev.upload(x), dev.alloc(N * 4)
    ib, wb = dev.alloc(16), dev.alloc(16)
    before = dev.router_exact_count()
    dev.moe_decode(device.desc, xb, out, ib, wb)
    assert dev.router_exact_count() == before + 1
    assert list(ib.download(np.int32)) == list(ref_idx)
    assert np.allclose(wb.download(np.float32), ref_w, rtol=5e-7, atol=0)
    ref, _, _, _ = host.oracle_moe(x, O.BODY_V4)
    assert O.rel_l2(out.download(np.float32), ref) <= TOL
    for b in (xb, out, ib, wb):
        b.free()
    device.free()


@pytest.mark.parametrize("experts,used", [(7, 4), (64, 16), (128, 4), (192, 8)])
def test_moe_decode_routing_inside_gateup_at_other_widths(dev, experts, used):
    """The gate/up kernel ranks the router rows in one wave, lane l holding experts l,
    l+64 and l+128: one, two and three candidates per lane, and up to 16 ranks.  The
    selected experts and weights must be the reference's."""
    host = HostLayer(experts, used, biases=True, fill_experts=[])
    device = DeviceLayer(dev, host)
    out, ib, wb = dev.alloc(N * 4), dev.alloc(used * 4), dev.alloc(used * 4)
    before = dev.router_exact_count()
    for token in range(4):
        x = O.synth_normal(X_SEED, 100 + token, N)
        xb = dev.upload(x)
        dev.moe_decode(device.desc, xb, out, ib, wb)
        _, ref_idx, ref_w = oracle_router(host.router_w, host.router_b, x, used)
        print(f"experts {experts} used {used} token {token}: {list(ref_idx)}", flush=True)
        assert list(ib.download(np.int32)) == list(ref_idx)
        assert np.allclose(wb.download(np.float32), ref_w, rtol=1e-5, atol=0)
        xb.free()
    # the certified ranking (not the exact fallback) decided most tokens
    assert dev.router_exact_count() - before < 4
    for b in (out, ib, wb):
        b.free()
    device.free()


@pytest.mark.parametrize("body", [O.BODY_V4, O.BODY_DEFAULT])
def test_moe_layer_config1_matches_oracle(dev, layer32, body):
    host, device = layer32
    out = dev.alloc(N * 4)
    ib, wb = dev.alloc(16), dev.alloc(16)
    for token in range(4):
        x = O.synth_normal(X_SEED, token, N)
        xb = dev.upload(x)
        dev.moe_decode(device.desc, xb, out, ib, wb)
        got = out.download(np.float32)
        ref, _, ref_idx, ref_w = host.oracle_moe(x, body)
        assert list(ib.download(np.int32)) == list(ref_idx)
        assert np.allclose(wb.download(np.float32), ref_w, rtol=1e-5, atol=0)
        err = O.rel_l2(got, ref)
        print(f"token {token} body {body}: experts {list(ref_idx)} rel_l2 {err:.3e}")
        assert err <= TOL
        xb.free()
    for b in (out, ib, wb):
        b.free()


def test_moe_layer_with_biases_matches_oracle(dev):
    host = HostLayer(32, 4, biases=True, seed=0x77000002)
    device = DeviceLayer(dev, host)
    out = dev.alloc(N * 4)
    for token in range(3):
        x = O.synth_normal(X_SEED, 50 + token, N)
        xb = dev.upload(x)
        dev.moe_decode(device.desc, xb, out)
        ref, _, _, _ = host.oracle_moe(x, O.BODY_V4)
        assert O.rel_l2(out.download(np.float32), ref) <= TOL
        xb.free()
    out.free()
    device.free()


def test_moe_rejects_mismatched_layers(dev, layer32):
    host, device = layer32
    bad = type(device.desc).from_buffer_copy(device.desc)
    bad.experts = 16
    xb, out = dev.upload(np.zeros(N, np.float32)), dev.alloc(N * 4)
    with pytest.raises(ttlab_amd.TtlError, match="must hold 16 experts"):
        dev.moe_decode(bad, xb, out)
    xb.free()
    out.free()


def test_graph_replays_match_eager_bitwise(dev, layer32):
    """A captured MoE layer replays identically, with eager work between replays."""
    host, device = layer32
    x = dev.upload(O.synth_normal(X_SEED, 77, N))
    eager_out, graph_out = dev.alloc(N * 4), dev.alloc(N * 4)
    ib, wb = dev.alloc(16), dev.alloc(16)
    dev.moe_decode(device.desc, x, eager_out, ib, wb)
    expected = eager_out.download(np.float32)
    graph = dev.capture(lambda: dev.moe_decode(device.desc, x, graph_out, ib, wb))
    for replay in range(4):
        dev.fill(graph_out, 0xFF)
        graph.launch()
        got = graph_out.download(np.float32)
        assert np.array_equal(got.view(np.uint32), expected.view(np.uint32)), replay
        # eager work between replays reuses the same workspace
        other = dev.upload(O.synth_normal(X_SEED, 900 + replay, N))
        dev.moe_decode(device.desc, other, eager_out)
        dev.sync()
        other.free()
    graph.free()
    for b in (x, eager_out, graph_out, ib, wb):
        b.free()


@pytest.mark.parametrize("used", [4, 2])
def test_down_combine_adds_residual_in_reference_order(dev, used):
    """ttl_moe_down_combine (the fused kernel for 4 experts, down + combine otherwise)
    against its parts: the down outputs equal ttl_moe_down's bitwise, and
    out = residual + (0 + w_0 d_0 + w_1 d_1 + ...) evaluated in f32 in that order
    (model.cpp:323-337, 592-594) is bitwise what the kernel writes."""
    host = HostLayer(32, used, biases=True, seed=0x77000003)
    device = DeviceLayer(dev, host)
    x = O.synth_normal(X_SEED, 300 + used, N)
    residual = O.synth_normal(X_SEED, 400 + used, N, sigma=4.0)
    xb, rb = dev.upload(x), dev.upload(residual)
    ib, wb = dev.alloc(4 * used), dev.alloc(4 * used)
    hidden = dev.alloc(used * N * 4)
    ref_down, got_down, out = dev.alloc(used * N * 4), dev.alloc(used * N * 4), dev.alloc(N * 4)
    dev.moe_decode(device.desc, xb, out, ib, wb)             # routing of x
    dev.moe_gateup_swiglu(device.desc, xb, ib, hidden)
    dev.moe_down(device.desc, hidden, ib, ref_down)
    dev.moe_down_combine(device.desc, hidden, ib, wb, rb, out, got_down)
    d = got_down.download(np.float32).reshape(used, N)
    assert np.array_equal(d.view(np.uint32), ref_down.download(np.float32).reshape(used, N).view(np.uint32))
    w = wb.download(np.float32)
    m = np.zeros(N, np.float32)
    for r in range(used):
        m = (m + (w[r] * d[r]).astype(np.float32)).astype(np.float32)
    expect = (residual + m).astype(np.float32)
    assert np.array_equal(out.download(np.float32).view(np.uint32), expect.view(np.uint32))
    # without a residual the output is the MoE layer itself, against the oracle
    dev.moe_down_combine(device.desc, hidden, ib, wb, None, out)
    ref, _, ref_idx, _ = host.oracle_moe(x, O.BODY_V4)
    assert list(ib.download(np.int32)) == list(ref_idx)
    assert O.rel_l2(out.download(np.float32), ref) <= TOL
    for b in (xb, rb, ib, wb, hidden, ref_down, got_down, out):
        b.free()
    device.free()


@pytest.mark.parametrize("experts,norm", [(32, True), (32, False), (128, True)])
def test_gateup_and_down_in_one_launch(dev, experts, norm):
    """ttl_moe_route_gateup_down, the decode step's MoE: gate/up (the ranking at its head)
    and the four experts' down rows in one launch, the down workgroups waiting inside it
    for their expert's hidden.  Against the two-launch form (ttl_moe_route_gateup, then
    ttl_moe_down): the routing and the hidden bit for bit, the down rows to f32 rounding
    (the same products summed in another order); the down rows against the oracle's
    matvec on that hidden within 1e-5 (model.cpp:326-333).  Five tokens back to back
    (the in-launch counts reset between launches), with and without the layer's input
    norm (the step's form: the router rows leave the normalized input for gate/up); no
    wait may end at its bound."""
    host = HostLayer(experts, 4, biases=True, seed=0x77000910 + experts, fill_experts=[])
    device = DeviceLayer(dev, host)
    nb = None
    if norm:
        nb = dev.upload(O.synth_normal(0x77000911, 0, N, sigma=0.05, mean=1.0))
        device.desc.input_norm = nb.ptr
        device.desc.input_norm_epsilon = 1e-5
    assert dev.moe_gateup_down_fused(device.desc), "the grid should be resident at once on gfx950"
    before = dev.handoff_give_ups()
    bufs = [dev.alloc(4 * N * 4) for _ in range(4)] + [dev.alloc(16) for _ in range(4)]
    hid_a, down_a, hid_b, down_b, ia, wa, ib, wb = bufs
    checked = set()
    for token in range(5):
        x = O.synth_normal(X_SEED, 900 + token, N)
        xb = dev.upload(x)
        dev.moe_route_gateup(device.desc, xb, hid_a, ia, wa)
        dev.moe_down(device.desc, hid_a, ia, down_a)
        dev.moe_route_gateup_down(device.desc, xb, hid_b, ib, wb, down_b)
        idx = ia.download(np.int32)
        assert np.array_equal(ib.download(np.int32), idx)
        assert np.array_equal(wb.download(np.uint32), wa.download(np.uint32))
        h_a, h_b = hid_a.download(np.float32), hid_b.download(np.float32)
        assert np.array_equal(h_b.view(np.uint32), h_a.view(np.uint32))
        d_a = down_a.download(np.float32).reshape(4, N)
        d_b = down_b.download(np.float32).reshape(4, N)
        for r in range(4):
            assert O.rel_l2(d_b[r], d_a[r]) <= 1e-6, (token, r)
            e = int(idx[r])
            if e not in checked:  # the host matrices of an expert are generated once
                checked.add(e)
                host_down = O.synth_mxfp4(host.seed, 3000 + e, N * 90)
                ref = O.mxfp4_matvec(host_down, host.down_b[e * N:(e + 1) * N], N, N, h_a.reshape(4, N)[r],
                                     body=O.BODY_DEFAULT)
                assert O.rel_l2(d_b[r], ref) <= TOL, (token, r, e)
        xb.free()
    assert dev.handoff_give_ups() == before
    for b in bufs:
        b.free()
    if nb:
        nb.free()
    device.free()


def test_gateup_swiglu_nonfinite_gates_follow_reference(dev):
    """The clamped SwiGLU's non-finite cases (model.cpp:328-332): std::min(gate, 7) and
    std::clamp(up, -7, 7) return a NaN argument as it is, so a NaN gate or up gives a NaN
    hidden value; a gate of -inf gives -inf / (1 + exp(inf)) = NaN; a gate of +inf or of
    1e30 clamps to 7 and an up of +-inf to +-7, finite.  Forced through the biases of the
    routed experts' rows.  The hidden of ttl_moe_gateup_swiglu against the oracle's gate and
    up matvecs and orc_swiglu: NaN exactly where the oracle has NaN, the finite entries
    within 1e-5; the layer output through down is NaN wherever the oracle's is."""
    host = HostLayer(32, 4, biases=True, seed=0x77000004)
    x = O.synth_normal(X_SEED, 500, N)
    _, _, idx, w = host.oracle_moe(x, O.BODY_V4)  # the routing does not read the gate/up biases
    cases = [("gate", 5, np.nan), ("gate", 6, np.inf), ("gate", 7, -np.inf), ("gate", 8, 1e30),
             ("up", 9, np.nan), ("up", 10, np.inf), ("up", 11, -np.inf), ("up", 12, -1e30)]
    for slot, e in enumerate(idx):
        for kind, row, value in cases:
            bias = host.gate_b if kind == "gate" else host.up_b
            bias[int(e) * N + row + 16 * slot] = value  # other rows in each slot
    device = DeviceLayer(dev, host)
    xb = dev.upload(x)
    ib = dev.upload(np.asarray(idx, np.int32))
    hidden = dev.alloc(4 * N * 4)
    dev.moe_gateup_swiglu(device.desc, xb, ib, hidden)
    got = hidden.download(np.float32).reshape(4, N)
    for slot, e in enumerate(idx):
        gate = O.mxfp4_matvec(host.gate, host.gate_b, N, N, x, int(e), O.BODY_V4)
        up = O.mxfp4_matvec(host.up, host.up_b, N, N, x, int(e), O.BODY_V4)
        ref = np.empty(N, np.float32)
        O.lib.orc_swiglu(gate, up, N, ref)
        nan = np.isnan(ref)
        for kind, row, value in cases:
            r = row + 16 * slot
            expect_nan = (kind == "gate" and (np.isnan(value) or value == -np.inf)) or (kind == "up" and np.isnan(value))
            assert bool(nan[r]) == expect_nan, (slot, kind, row, value)
        assert np.array_equal(np.isnan(got[slot]), nan), slot
        assert np.all(np.isfinite(got[slot][~nan]))
        assert O.rel_l2(got[slot][~nan], ref[~nan]) <= TOL, slot
    # through down and the combine: every output is NaN, as in the oracle
    out = dev.alloc(N * 4)
    dev.moe_decode(device.desc, xb, out)
    ref_out, _, _, _ = host.oracle_moe(x, O.BODY_V4)
    assert np.array_equal(np.isnan(out.download(np.float32)), np.isnan(ref_out))
    for b in (xb, ib, hidden, out):
        b.free()
    device.free()
