"""The C++ decode model (ttlab::HipGptOssModel) against the oracle, layer by layer.

Teacher forcing: at checked positions each GPU layer's own input and KV cache are
fed to the oracle's layer (orc_layer_forward, model.cpp:571-595) and the outputs
compared (relative L2 <= 1e-5): residual after attention, the new cache entries,
the routing (exact unless the oracle's own logits are near-tied) and the layer
output (the next layer's input).  Then logits against the oracle's unembedding
of the GPU's final state, and greedy tokens of a free-running decode.
"""
import numpy as np
import pytest

import oracle_lib as O
import ttlab_amd
from model_fixtures import HostModel, N

pytestmark = pytest.mark.gpu
TOL = 1e-5
SEED, LAYERS, EXPERTS, VOCAB, CAPACITY = 0x77000003, 2, 32, 4096, 160


# 32 experts: the 20b shape (benchmark config 3); 128: the 120b routing width (config 4),
# whose host copy generates only the experts the oracle routes to.
@pytest.fixture(scope="module", params=[EXPERTS, 128], ids=["20b", "120b"])
def models(request):
    experts = request.param
    gpu = ttlab_amd.Model(LAYERS, experts, VOCAB, CAPACITY, SEED)
    host = HostModel(SEED, LAYERS, experts, VOCAB, lazy=experts > 32)
    yield gpu, host
    gpu.close()


def near_tie(router, k=4, eps=1e-4):
    s = np.sort(router.astype(np.float64))[::-1]
    return np.any(np.abs(np.diff(s[:k + 1])) < eps)


def check_layers(gpu, host, position):
    worst = 0.0
    for l in range(LAYERS):
        x_in, residual, idx, w = gpu.layer_state(l)
        keys, values = gpu.kv_cache(l, position + 1)
        kc = np.zeros(CAPACITY * 512, np.float32)
        vc = np.zeros(CAPACITY * 512, np.float32)
        kc[:position * 512] = keys[:position * 512]
        vc[:position * 512] = values[:position * 512]
        ref = host.layer_forward(l, position, x_in, kc, vc)
        worst = max(worst, O.rel_l2(residual, ref["residual"]))
        assert O.rel_l2(residual, ref["residual"]) <= TOL, (l, position)
        assert O.rel_l2(keys[position * 512:], kc[position * 512:(position + 1) * 512]) <= TOL
        assert O.rel_l2(values[position * 512:], vc[position * 512:(position + 1) * 512]) <= TOL
        if list(idx) != list(ref["indices"]):
            assert near_tie(ref["router"]), (l, position, idx, ref["indices"])
            continue  # a flipped near-tie changes the layer output; nothing more to compare
        assert np.allclose(w, ref["weights"], rtol=1e-5, atol=1e-7)
        nxt = gpu.layer_state(l + 1)[0] if l + 1 < LAYERS else gpu.final_state()
        err = O.rel_l2(nxt, ref["x_out"])
        worst = max(worst, err)
        assert err <= TOL, (l, position, err)
    return worst


def test_teacher_forced_layers_and_logits(models):
    gpu, host = models
    tokens = [int(t) for t in np.random.default_rng(5).integers(0, VOCAB, 140)]
    checks = {0, 1, 9, 129, 139}
    for p, tok in enumerate(tokens):
        logits = gpu.forward(tok, p)
        if p in checks:
            x_in0 = gpu.layer_state(0)[0]
            assert np.array_equal(x_in0.view(np.uint32), host.embedding(tok).view(np.uint32))
            worst = check_layers(gpu, host, p)
            ref = host.logits(gpu.final_state())
            err = O.rel_l2(logits, ref)
            print(f"position {p}: worst layer rel_l2 {worst:.2e}, logits rel_l2 {err:.2e}")
            assert err <= TOL
            top = np.sort(ref.astype(np.float64))[-2:]
            if top[1] - top[0] > 1e-4 * abs(top[1]):
                assert gpu.lib and int(np.argmax(logits)) == int(np.argmax(ref))


def test_generate_matches_forward_and_greedy(models):
    gpu, _ = models
    start = 3
    first = gpu.forward(start, 0)
    expected = [int(O.lib.orc_greedy(first, VOCAB))]
    for p in range(1, 6):
        logits = gpu.forward(expected[-1], p)
        expected.append(int(O.lib.orc_greedy(logits, VOCAB)))
    got = gpu.generate(start, 0, 6)
    assert list(got) == expected


def test_free_running_decode_matches_oracle(models):
    """Greedy decode from token 11 for 4 steps, GPU vs oracle (oracle runs its own layers
    and caches); tokens agree unless a step's top-2 logits are near-tied."""
    gpu, host = models
    tok = 11
    kcs = [np.zeros(CAPACITY * 512, np.float32) for _ in range(LAYERS)]
    vcs = [np.zeros(CAPACITY * 512, np.float32) for _ in range(LAYERS)]
    gpu_tokens = gpu.generate(tok, 0, 4)
    for p in range(4):
        x = host.embedding(tok)
        for l in range(LAYERS):
            x = host.layer_forward(l, p, x, kcs[l], vcs[l])["x_out"]
        logits = host.logits(x)
        ref_tok = int(O.lib.orc_greedy(logits, VOCAB))
        top = np.sort(logits.astype(np.float64))[-2:]
        if top[1] - top[0] <= 1e-4 * abs(top[1]):
            break
        assert int(gpu_tokens[p]) == ref_tok, (p, gpu_tokens, ref_tok)
        tok = ref_tok


def test_model_rejects_out_of_range_inputs(models):
    gpu, _ = models
    with pytest.raises(ttlab_amd.TtlError, match="out of range"):
        gpu.forward(VOCAB, 0)
    with pytest.raises(ttlab_amd.TtlError, match="capacity"):
        gpu.forward(1, CAPACITY)


def test_timers_leave_decode_state_intact(models):
    """The bench's kernel timer replays expert launches on scratch memory only: the
    last step's layer state is unchanged, and decode timing reports a positive time."""
    gpu, _ = models
    gpu.forward(5, 0)
    before = [gpu.layer_state(l) for l in range(LAYERS)]
    us = gpu.time_expert_kernel(5)
    assert 0.0 < us < 1e5
    keys, values = gpu.kv_cache(0, 2)
    for kind in ttlab_amd.Model.KERNELS:
        us, launches = gpu.time_kernel(kind, 0, 3)
        expected = {"attention_window": (LAYERS + 1) // 2, "attention_full": LAYERS // 2, "logits": 1}
        assert launches == expected.get(kind, LAYERS), kind
        assert 0.0 < us < 1e5, kind
    k2, v2 = gpu.kv_cache(0, 2)
    assert np.array_equal(keys, k2) and np.array_equal(values, v2)
    after = [gpu.layer_state(l) for l in range(LAYERS)]
    for b, a in zip(before, after):
        for u, v in zip(b, a):
            assert np.array_equal(u, v)
    ms = gpu.time_decode(5, 1, 1, 3)
    assert 0.0 < ms < 1e4


def test_eager_launches_match_graph_replay(models):
    """Kernels launched one by one give bitwise the same tokens and state as the step graph."""
    gpu, _ = models
    graph_tokens = gpu.generate(7, 0, 5)
    graph_state = [gpu.layer_state(l) for l in range(LAYERS)] + [gpu.final_state()]
    gpu.set_graph_replay(False)
    try:
        eager_tokens = gpu.generate(7, 0, 5)
        eager_state = [gpu.layer_state(l) for l in range(LAYERS)] + [gpu.final_state()]
        us = gpu.time_expert_kernel(3)
    finally:
        gpu.set_graph_replay(True)
    assert list(eager_tokens) == list(graph_tokens)
    for g, e in zip(graph_state, eager_state):
        for u, v in zip(g if isinstance(g, tuple) else (g,), e if isinstance(e, tuple) else (e,)):
            assert np.array_equal(u, v)
    assert us > 0.0


def test_synthetic_kv_fill_then_decode(models):
    """ttlm_fill_kv_synthetic writes the generator's N(0, 1) values (per layer, keys on
    stream 2l, values on 2l + 1) into positions [0, n) of every cache; a decode step at
    position n then matches the oracle over that context, layer by layer.  (Last in the
    module: it overwrites the caches the other tests built.)"""
    gpu, host = models
    position, seed = 40, 0x78000300
    gpu.fill_kv_synthetic(position, seed)
    for l in (0, LAYERS - 1):
        keys, values = gpu.kv_cache(l, position)
        assert np.array_equal(keys, O.synth_normal(seed, 2 * l, position * 512))
        assert np.array_equal(values, O.synth_normal(seed, 2 * l + 1, position * 512))
    gpu.forward(5, position)
    check_layers(gpu, host, position)
