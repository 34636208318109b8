"""Pins the oracle's compositions -- orc_moe (model.cpp:292-338), orc_layer_forward
(model.cpp:571-595) and orc_layer_prefill (model.cpp:484-553) -- against the float64
brute force of tests/brute_force.py, which is written from the reference's definitions
and shares no code with the oracle.  Every output the oracle exposes is compared:
query after RoPE, the cache entries, attention, the residual, router logits, the
routing (exactly), the softmax weights and the layer output (relative L2 <= 1e-5).

The checks must catch wiring mistakes, not only rounding: the last tests feed the
oracle a layer with its two norm weights swapped, and run it with the wrong window
(the other layer parity), and show the brute-force comparison rejects both.
"""
import ctypes as C

import numpy as np
import pytest

import brute_force as B
import oracle_lib as O
from model_fixtures import HostModelLayer

lib = O.lib
N, KV, TOL = 2880, 512, 1e-5
SEED = 0x77000041
FREQS = np.empty(32, np.float32)
lib.orc_rope_frequencies(FREQS)

_layers = {}


def layer(experts=8):
    """One layer's host tensors and their float64 decode, shared by the tests (the layer
    index, which picks the attention window, is a separate argument of the oracle);
    above 32 experts the expert matrices are generated as the brute force reads them."""
    if experts not in _layers:
        host = HostModelLayer(SEED, 0, experts, lazy=experts > 32)
        _layers[experts] = (host, B.DenseLayer(host))
    return _layers[experts]


def caches(position, seed):
    """f32 caches holding synthetic keys and values at positions 0 .. position-1."""
    kc = np.zeros((position + 8) * KV, np.float32)
    vc = np.zeros((position + 8) * KV, np.float32)
    kc[:position * KV] = O.synth_normal(seed, 1, position * KV, sigma=1.5)
    vc[:position * KV] = O.synth_normal(seed, 2, position * KV)
    return kc, vc


def oracle_forward(host, layer_index, position, x, kc, vc, body=O.BODY_V4, struct=None):
    s = struct if struct is not None else host.struct()
    out = {k: np.empty(n, np.float32) for k, n in (("x_out", N), ("query", 4096), ("attended", 4096),
                                                    ("residual", N), ("router", host.experts))}
    idx, w = np.empty(4, np.int64), np.empty(4, np.float32)
    lib.orc_layer_forward(C.byref(s), layer_index, position, np.ascontiguousarray(x, np.float32), FREQS, kc, vc,
                          body, out["x_out"], out["query"], out["attended"], out["residual"], out["router"], idx, w)
    out["indices"], out["weights"] = idx, w
    return out


def compare_layer(got, ref, what=""):
    errs = {}
    for key in ("query", "attended", "residual", "router", "x_out"):
        if key in got and key in ref:
            errs[key] = O.rel_l2(got[key], ref[key])
    assert list(got["indices"]) == list(ref["indices"]), (what, got["indices"], ref["indices"])
    errs["weights"] = O.rel_l2(got["weights"], ref["weights"])
    return errs


def brute_caches(kc, vc, rows):
    return (kc.astype(np.float64).reshape(-1, KV)[:rows].copy(), vc.astype(np.float64).reshape(-1, KV)[:rows].copy())


# ---- orc_moe: one decode token at the full width ---------------------------------------

@pytest.mark.parametrize("body", [O.BODY_DEFAULT, O.BODY_V4])
@pytest.mark.parametrize("experts", [32, 128])
def test_moe_decode_against_float64(body, experts):
    host, dense = layer(experts)
    x = B.rms_norm(O.synth_normal(SEED, 90, N, sigma=3.0), host.post_norm).astype(np.float32)
    ref, router, idx, w = B.moe(dense, x)  # generates the routed experts of a lazy layer
    s = host.struct()
    out = np.empty(N, np.float32)
    got_router, got_idx, got_w = np.empty(experts, np.float32), np.empty(4, np.int64), np.empty(4, np.float32)
    lib.orc_moe(C.byref(s.moe), x, out, body, got_router.ctypes.data, got_idx.ctypes.data, got_w.ctypes.data)
    assert list(got_idx) == list(idx)
    assert O.rel_l2(got_router, router) <= TOL
    assert O.rel_l2(got_w, w) <= TOL
    err = O.rel_l2(out, ref)
    print(f"orc_moe {experts} experts body {body}: rel_l2 {err:.2e}")
    assert err <= TOL


def test_moe_decode_combines_in_rank_order():
    """orc_moe's output is bit for bit the reference's loop over the ranks (model.cpp:323-337):
    out = 0, then out += w_r * down_r for r = 0..3 in f32 without fusion, from the pinned
    parts (router matvec and selection, MXFP4 matvecs, SwiGLU).  Summed in expert order
    instead, some element differs -- the order is observable and fixed."""
    host, _ = layer(32)
    x = B.rms_norm(O.synth_normal(SEED, 91, N, sigma=3.0), host.post_norm).astype(np.float32)
    s = host.struct()
    out = np.empty(N, np.float32)
    lib.orc_moe(C.byref(s.moe), x, out, O.BODY_V4, None, None, None)
    logits = np.empty(32, np.float32)
    lib.orc_matvec_add_f32(host.router, host.router_b, 32, N, x, logits)
    idx, w = O.router_topk(logits, 4)
    downs = []
    for e in idx:
        g = O.mxfp4_matvec(host.gate, host.gate_b, N, N, x, expert=int(e), body=O.BODY_V4)
        u = O.mxfp4_matvec(host.up, host.up_b, N, N, x, expert=int(e), body=O.BODY_V4)
        h = np.empty(N, np.float32)
        lib.orc_swiglu(g, u, N, h)
        downs.append(O.mxfp4_matvec(host.down, host.down_b, N, N, h, expert=int(e), body=O.BODY_V4))
    acc = np.zeros(N, np.float32)
    for r in range(4):
        acc = (acc + np.float32(w[r]) * downs[r]).astype(np.float32)
    assert np.array_equal(acc.view(np.uint32), out.view(np.uint32))
    other = np.zeros(N, np.float32)
    for r in np.argsort(idx):
        other = (other + np.float32(w[r]) * downs[r]).astype(np.float32)
    assert not np.array_equal(other.view(np.uint32), out.view(np.uint32))


# ---- orc_layer_forward ---------------------------------------------------------------

@pytest.mark.parametrize("layer_index,position", [(0, 0), (1, 5), (2, 200), (3, 200)])
def test_layer_forward_against_float64(layer_index, position):
    host, dense = layer()
    kc, vc = caches(position, 0x100 + position)
    x = O.synth_normal(SEED, 100 + layer_index, N, sigma=4.0)
    kb, vb = brute_caches(kc, vc, position + 1)
    ref = B.layer_forward(dense, layer_index, position, x, kb, vb, FREQS)
    got = oracle_forward(host, layer_index, position, x, kc, vc)
    errs = compare_layer(got, ref, (layer_index, position))
    errs["key"] = O.rel_l2(kc[position * KV:(position + 1) * KV], ref["key"])
    errs["value"] = O.rel_l2(vc[position * KV:(position + 1) * KV], ref["value"])
    print(f"orc_layer_forward layer {layer_index} position {position}: "
          + ", ".join(f"{k} {v:.1e}" for k, v in errs.items()))
    for k, v in errs.items():
        assert v <= TOL, (k, v)


# ---- orc_layer_prefill ------------------------------------------------------------------

@pytest.mark.parametrize("layer_index,first,count", [(0, 0, 5), (1, 0, 5), (2, 140, 6), (3, 140, 6)])
def test_layer_prefill_against_float64(layer_index, first, count):
    host, dense = layer()
    kc, vc = caches(first, 0x200 + first)
    x = O.synth_normal(SEED, 200 + layer_index, count * N, sigma=4.0)
    kb, vb = brute_caches(kc, vc, first + count)
    refs = B.layer_prefill(dense, layer_index, first, x.reshape(count, N), kb, vb, FREQS)
    out = np.empty(count * N, np.float32)
    res = np.empty(count * N, np.float32)
    lib.orc_layer_prefill(C.byref(host.struct()), layer_index, first, count, x, FREQS, kc, vc, O.BODY_V4, out,
                          res.ctypes.data)
    worst = 0.0
    for t in range(count):
        p = first + t
        for got, ref in ((out[t * N:(t + 1) * N], refs[t]["x_out"]), (res[t * N:(t + 1) * N], refs[t]["residual"]),
                         (kc[p * KV:(p + 1) * KV], kb[p]), (vc[p * KV:(p + 1) * KV], vb[p])):
            err = O.rel_l2(got, ref)
            worst = max(worst, err)
            assert err <= TOL, (layer_index, t, err)
    print(f"orc_layer_prefill layer {layer_index} positions {first}..{first + count - 1}: worst rel_l2 {worst:.1e}")


# ---- the comparison rejects wiring mistakes (planted in the oracle's inputs) -------------

def test_brute_force_rejects_swapped_norms_and_wrong_window():
    layer_index, position = 2, 200
    host, dense = layer()
    kc, vc = caches(position, 0x300)
    x = O.synth_normal(SEED, 300, N, sigma=4.0)
    kb, vb = brute_caches(kc, vc, position + 1)
    ref = B.layer_forward(dense, layer_index, position, x, kb, vb, FREQS)

    swapped = host.struct()
    swapped.attention_norm, swapped.post_attention_norm = swapped.post_attention_norm, swapped.attention_norm
    got = oracle_forward(host, layer_index, position, x, kc.copy(), vc.copy(), struct=swapped)
    assert O.rel_l2(got["query"], ref["query"]) > 100 * TOL
    assert O.rel_l2(got["x_out"], ref["x_out"]) > 100 * TOL

    # the other parity attends over all 201 positions instead of the last 128
    got = oracle_forward(host, layer_index + 1, position, x, kc.copy(), vc.copy())
    assert O.rel_l2(got["query"], ref["query"]) <= TOL  # same projections ...
    assert O.rel_l2(got["attended"], ref["attended"]) > 100 * TOL  # ... different window
