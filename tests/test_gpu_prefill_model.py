"""The model's layer-major prefill (GptOssModel::prefill, model.cpp:463-555) on the
GPU against the oracle's (orc_layer_prefill), layer by layer.

Teacher forcing: each GPU layer's input sequence (ttlm_prefill_state) and the
positions before it go through the oracle's prefill layer; the keys and values the
GPU stored and the next layer's inputs must agree to relative L2 <= 1e-5 per token,
unless the oracle's own router logits for that token are near-tied (then the routing
may differ and the layer output with it).  Then the last token's logits.  A prompt
longer than one pass runs in passes; the second pass is checked the same way, reading
the positions of the first from the GPU's caches.
"""
import ctypes as C

import numpy as np
import pytest

import oracle_lib as O
import ttlab_amd
from model_fixtures import HostModel, N

pytestmark = pytest.mark.gpu
TOL = 1e-5
KW = 512
SEED, LAYERS, EXPERTS, VOCAB = 0x77000041, 2, 32, 4096


def router_near_tie(layer, residual, k=4, eps=1e-4):
    normed = np.empty(N, np.float32)
    O.lib.orc_rms_norm(np.ascontiguousarray(residual, np.float32), layer.post_norm, N, 1e-5, normed)
    logits = np.empty(layer.experts, np.float32)
    O.lib.orc_matvec_add_f32(layer.router, layer.router_b, layer.experts, N, normed, logits)
    s = np.sort(logits.astype(np.float64))[::-1]
    return bool(np.any(np.abs(np.diff(s[:k + 1])) < eps))


def check_pass(gpu, host, first, count, capacity):
    """Teacher-forced oracle prefill of positions first .. first+count-1 per layer."""
    checked = 0
    for l in range(LAYERS):
        layer = host.layers[l]
        x_in = gpu.prefill_state(l, count)
        keys, values = gpu.kv_cache(l, first + count)
        kc, vc = np.zeros(capacity * KW, np.float32), np.zeros(capacity * KW, np.float32)
        kc[:first * KW], vc[:first * KW] = keys[:first * KW], values[:first * KW]
        out, res = np.empty(count * N, np.float32), np.empty(count * N, np.float32)
        s = layer.struct()
        O.lib.orc_layer_prefill(C.byref(s), l, first, count, np.ascontiguousarray(x_in.ravel()), host.freqs, kc, vc,
                                O.BODY_V4, out, res.ctypes.data)
        for p in range(count):
            a, b = (first + p) * KW, (first + p + 1) * KW
            assert O.rel_l2(keys[a:b], kc[a:b]) <= TOL, (l, p)
            assert O.rel_l2(values[a:b], vc[a:b]) <= TOL, (l, p)
        nxt = gpu.prefill_state(l + 1, count)
        for p in range(count):
            err = O.rel_l2(nxt[p], out[p * N:(p + 1) * N])
            if err > TOL:
                assert router_near_tie(layer, res[p * N:(p + 1) * N]), (l, p, err)
                continue
            checked += 1
    return checked


@pytest.fixture(scope="module")
def host():
    return HostModel(SEED, LAYERS, EXPERTS, VOCAB)


def test_prefill_matches_oracle_layer_by_layer(host):
    capacity, count = 64, 24
    gpu = ttlab_amd.Model(LAYERS, EXPERTS, VOCAB, capacity, SEED)
    try:
        tokens = [int(t) for t in np.random.default_rng(41).integers(0, VOCAB, count)]
        logits = gpu.prefill(tokens)
        x0 = gpu.prefill_state(0, count)
        for p, tok in enumerate(tokens):
            assert np.array_equal(x0[p].view(np.uint32), host.embedding(tok).view(np.uint32)), p
        checked = check_pass(gpu, host, 0, count, capacity)
        assert checked >= LAYERS * count - 4
        ref = host.logits(gpu.prefill_state(LAYERS, count)[count - 1])
        assert O.rel_l2(logits, ref) <= TOL
        # decoding continues from the prefilled caches
        nxt = gpu.forward(int(O.lib.orc_greedy(logits, VOCAB)), count)
        assert np.all(np.isfinite(nxt))
    finally:
        gpu.close()


@pytest.mark.parametrize("count", [1, 17])
def test_prefill_short_prompts(host, count):
    """One token (every GEMM tile narrow, one attention block) and 17 (a second attention
    block of one token), teacher-forced against the oracle's prefill layers."""
    capacity = 32
    gpu = ttlab_amd.Model(LAYERS, EXPERTS, VOCAB, capacity, SEED)
    try:
        tokens = [int(t) for t in np.random.default_rng(43 + count).integers(0, VOCAB, count)]
        logits = gpu.prefill(tokens)
        checked = check_pass(gpu, host, 0, count, capacity)
        assert checked >= LAYERS * count - 1
        ref = host.logits(gpu.prefill_state(LAYERS, count)[count - 1])
        assert O.rel_l2(logits, ref) <= TOL
    finally:
        gpu.close()


def test_prefill_in_two_passes(host):
    capacity, count = 600, 530
    gpu = ttlab_amd.Model(LAYERS, EXPERTS, VOCAB, capacity, SEED)
    try:
        batch = gpu.prefill_batch
        assert batch == 512 and count > batch
        tokens = [int(t) for t in np.random.default_rng(42).integers(0, VOCAB, count)]
        logits = gpu.prefill(tokens)
        first = batch
        checked = check_pass(gpu, host, first, count - first, capacity)
        assert checked >= LAYERS * (count - first) - 4
        ref = host.logits(gpu.prefill_state(LAYERS, count - first)[count - first - 1])
        assert O.rel_l2(logits, ref) <= TOL
    finally:
        gpu.close()


def test_prefill_errors_match_reference():
    gpu = ttlab_amd.Model(1, EXPERTS, VOCAB, 16, SEED)
    try:
        with pytest.raises(ttlab_amd.TtlError, match="prefill needs at least one token"):
            gpu.prefill([])
        with pytest.raises(ttlab_amd.TtlError, match="prefill exceeds startup batch capacity"):
            gpu.prefill([1] * 17)
        with pytest.raises(ttlab_amd.TtlError, match="input token is out of range"):
            gpu.prefill([1, VOCAB])
    finally:
        gpu.close()
