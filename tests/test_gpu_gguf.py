"""A gpt-oss model loaded from a GGUF file (ttlm_create_from_gguf) against the oracle.

The file (tests/gguf_writer.py) holds generated weights in the GGUF formats the
reference reads (Q8_0 attention and token embedding, F32 norms/biases/router,
MXFP4 experts, Q8_0 output.weight, model.cpp:141-169); the oracle runs the same
bytes.  Teacher forcing as in test_gpu_model.py: at checked positions every GPU
layer's input and KV cache go through orc_layer_forward (model.cpp:571-595) and
the outputs must agree to relative L2 <= 1e-5 (routing exactly, unless the
oracle's own logits are near-tied); then logits through the Q8_0 unembedding
(model.cpp:596-599) and greedy tokens.
"""
import ctypes as C
import os

import numpy as np
import pytest

import oracle_lib as O
import ttlab_amd
from gguf_writer import GGML_Q8_0, gpt_oss_metadata, gpt_oss_tensors, write_gguf

pytestmark = pytest.mark.gpu
TOL = 1e-5
N, QW, KW = 2880, 4096, 512
LAYERS, EXPERTS, VOCAB, CAPACITY, SEED = 2, 8, 1024, 160, 0x77000005


def generated(name, nbytes):
    """Deterministic weights per tensor name, in each tensor's GGUF format."""
    stream = sum(ord(c) * (i + 1) for i, c in enumerate(name)) % 100003
    if name.endswith("_exps.weight"):
        return O.synth_mxfp4(SEED, stream, nbytes // 17)
    if name.endswith((".weight",)) and ("attn_q" in name or "attn_k" in name or "attn_v" in name or
                                        "attn_output" in name or name in ("token_embd.weight", "output.weight")):
        return O.synth_q8_0(SEED, stream, nbytes // 34)
    n = nbytes // 4
    if "norm" in name:
        return O.synth_normal(SEED, stream, n, sigma=0.05, mean=1.0)
    if "ffn_gate_inp.weight" in name:
        return O.synth_normal_bf16(SEED, stream, n, 0.02)
    if "sinks" in name:
        return O.synth_normal(SEED, stream, n, sigma=1.0)
    return O.synth_normal(SEED, stream, n, sigma=0.05)


class GgufHost:
    """The oracle's view of the same file's weights."""

    def __init__(self, tensors):
        self.t = {name: data for name, _, _, data in tensors}
        self.freqs = np.empty(32, np.float32)
        O.lib.orc_rope_frequencies(self.freqs)

    def layer_struct(self, l):
        t, p = self.t, f"blk.{l}."
        s = O.OrcLayer()
        s.attention_norm = t[p + "attn_norm.weight"].ctypes.data
        s.post_attention_norm = t[p + "post_attention_norm.weight"].ctypes.data
        s.query_weight, s.query_bias = t[p + "attn_q.weight"].ctypes.data, t[p + "attn_q.bias"].ctypes.data
        s.key_weight, s.key_bias = t[p + "attn_k.weight"].ctypes.data, t[p + "attn_k.bias"].ctypes.data
        s.value_weight, s.value_bias = t[p + "attn_v.weight"].ctypes.data, t[p + "attn_v.bias"].ctypes.data
        s.output_weight = t[p + "attn_output.weight"].ctypes.data
        s.output_bias = t[p + "attn_output.bias"].ctypes.data
        s.sinks = t[p + "attn_sinks.weight"].ctypes.data
        m = s.moe
        m.hidden, m.expert_hidden, m.experts, m.used = N, N, EXPERTS, 4
        m.router_weight, m.router_bias = t[p + "ffn_gate_inp.weight"].ctypes.data, t[p + "ffn_gate_inp.bias"].ctypes.data
        for k in ("gate", "up", "down"):
            setattr(m, f"{k}_weight", t[p + f"ffn_{k}_exps.weight"].ctypes.data)
            setattr(m, f"{k}_bias", t[p + f"ffn_{k}_exps.bias"].ctypes.data)
        return s

    def embedding(self, token):
        out = np.empty(N, np.float32)
        O.lib.orc_load_token_embedding_q8_0(self.t["token_embd.weight"], N, token, out)
        return out

    def layer_forward(self, l, position, x_in, kc, vc):
        outs = {k: np.empty(n, np.float32) for k, n in (("x_out", N), ("query", QW), ("attended", QW),
                                                         ("residual", N), ("router", EXPERTS), ("weights", 4))}
        outs["indices"] = np.empty(4, np.int64)
        s = self.layer_struct(l)
        O.lib.orc_layer_forward(C.byref(s), l, position, np.ascontiguousarray(x_in, np.float32), self.freqs, kc, vc,
                                O.BODY_V4, outs["x_out"], outs["query"], outs["attended"], outs["residual"],
                                outs["router"], outs["indices"], outs["weights"])
        return outs

    def logits(self, x_final):
        normed = np.empty(N, np.float32)
        O.lib.orc_rms_norm(np.ascontiguousarray(x_final, np.float32), self.t["output_norm.weight"], N, 1e-5, normed)
        out = np.empty(VOCAB, np.float32)
        O.lib.orc_matvec_q8_0(self.t["output.weight"], VOCAB, N, normed, out)
        return out


@pytest.fixture(scope="module")
def loaded(tmp_path_factory):
    tensors = gpt_oss_tensors(LAYERS, EXPERTS, VOCAB, generated, GGML_Q8_0)
    path = os.path.join(tmp_path_factory.mktemp("gguf"), "gpt-oss-small.gguf")
    write_gguf(path, gpt_oss_metadata(LAYERS, EXPERTS), tensors)
    gpu = ttlab_amd.Model.from_gguf(path, CAPACITY, strict=False)
    yield gpu, GgufHost(tensors), path
    gpu.close()


def near_tie(router, k=4, eps=1e-4):
    s = np.sort(router.astype(np.float64))[::-1]
    return np.any(np.abs(np.diff(s[:k + 1])) < eps)


def test_gguf_model_layers_and_logits_match_oracle(loaded):
    gpu, host, _ = loaded
    tokens = [int(t) for t in np.random.default_rng(7).integers(0, VOCAB, 131)]
    checks = {0, 1, 5, 130}
    for p, tok in enumerate(tokens):
        logits = gpu.forward(tok, p)
        if p not in checks:
            continue
        assert np.array_equal(gpu.layer_state(0)[0].view(np.uint32), host.embedding(tok).view(np.uint32))
        worst = 0.0
        for l in range(LAYERS):
            x_in, residual, idx, w = gpu.layer_state(l)
            keys, values = gpu.kv_cache(l, p + 1)
            kc = np.zeros(CAPACITY * KW, np.float32)
            vc = np.zeros(CAPACITY * KW, np.float32)
            kc[:p * KW], vc[:p * KW] = keys[:p * KW], values[:p * KW]
            ref = host.layer_forward(l, p, x_in, kc, vc)
            assert O.rel_l2(residual, ref["residual"]) <= TOL, (l, p)
            assert O.rel_l2(keys[p * KW:], kc[p * KW:(p + 1) * KW]) <= TOL
            assert O.rel_l2(values[p * KW:], vc[p * KW:(p + 1) * KW]) <= TOL
            if list(idx) != list(ref["indices"]):
                assert near_tie(ref["router"]), (l, p, idx, ref["indices"])
                break
            assert np.allclose(w, ref["weights"], rtol=1e-5, atol=1e-7)
            nxt = gpu.layer_state(l + 1)[0] if l + 1 < LAYERS else gpu.final_state()
            err = O.rel_l2(nxt, ref["x_out"])
            worst = max(worst, err)
            assert err <= TOL, (l, p, err)
        ref_logits = host.logits(gpu.final_state())
        err = O.rel_l2(logits, ref_logits)
        print(f"position {p}: worst layer rel_l2 {worst:.2e}, Q8_0 logits rel_l2 {err:.2e}")
        assert err <= TOL
        top = np.sort(ref_logits.astype(np.float64))[-2:]
        if top[1] - top[0] > 1e-4 * abs(top[1]):
            assert int(np.argmax(logits)) == int(O.lib.orc_greedy(ref_logits, VOCAB))


def test_gguf_model_generates_greedily(loaded):
    gpu, _, _ = loaded
    first = gpu.forward(9, 0)
    expected = [int(O.lib.orc_greedy(first, VOCAB))]
    for p in range(1, 5):
        expected.append(int(O.lib.orc_greedy(gpu.forward(expected[-1], p), VOCAB)))
    assert list(gpu.generate(9, 0, 5)) == expected


def test_strict_load_refuses_the_small_model(loaded):
    _, _, path = loaded
    with pytest.raises(ttlab_amd.TtlError, match="only gpt-oss-20b and gpt-oss-120b are supported"):
        ttlab_amd.Model.from_gguf(path, CAPACITY, strict=True)


def test_gguf_model_prefill_matches_oracle(loaded):
    """Layer-major prefill (model.cpp:463-555) of the file's model: each layer's input
    rows through the oracle's prefill layer, then the Q8_0 logits of the last token."""
    gpu, host, _ = loaded
    count = 21
    tokens = [int(t) for t in np.random.default_rng(17).integers(0, VOCAB, count)]
    logits = gpu.prefill(tokens)
    x0 = gpu.prefill_state(0, count)
    for p, tok in enumerate(tokens):
        assert np.array_equal(x0[p].view(np.uint32), host.embedding(tok).view(np.uint32)), p
    skipped = 0
    for l in range(LAYERS):
        x_in = gpu.prefill_state(l, count)
        keys, values = gpu.kv_cache(l, count)
        kc, vc = np.zeros(CAPACITY * KW, np.float32), np.zeros(CAPACITY * KW, np.float32)
        out, res = np.empty(count * N, np.float32), np.empty(count * N, np.float32)
        s = host.layer_struct(l)
        O.lib.orc_layer_prefill(C.byref(s), l, 0, count, np.ascontiguousarray(x_in.ravel()), host.freqs, kc, vc,
                                O.BODY_V4, out, res.ctypes.data)
        assert O.rel_l2(keys, kc[:count * KW]) <= TOL
        assert O.rel_l2(values, vc[:count * KW]) <= TOL
        nxt = gpu.prefill_state(l + 1, count)
        for p in range(count):
            err = O.rel_l2(nxt[p], out[p * N:(p + 1) * N])
            if err > TOL:
                # only a token whose routing the oracle's own router logits leave near-tied
                normed = np.empty(N, np.float32)
                O.lib.orc_rms_norm(res[p * N:(p + 1) * N], host.t[f"blk.{l}.post_attention_norm.weight"], N, 1e-5,
                                   normed)
                router = np.empty(EXPERTS, np.float32)
                O.lib.orc_matvec_add_f32(host.t[f"blk.{l}.ffn_gate_inp.weight"], host.t[f"blk.{l}.ffn_gate_inp.bias"],
                                         EXPERTS, N, normed, router)
                assert near_tie(router), (l, p, err)
                skipped += 1
    assert skipped <= 2
    ref = host.logits(gpu.prefill_state(LAYERS, count)[count - 1])
    err = O.rel_l2(logits, ref)
    print(f"GGUF prefill of {count} tokens: Q8_0 logits rel_l2 {err:.2e}")
    assert err <= TOL


def test_edge_scales_make_prefill_run_as_decode_steps(tmp_path):
    """A file whose expert weights hold a block with E8M0 scale 0 (or 255) loads, decodes
    every scale exactly through the matvec kernels, and prefills as decode steps: the
    batched MFMA kernels refuse such tensors.  The prompt's logits equal, bit for bit,
    those of GptOssModel::forward run position by position."""
    def with_edge(name, nbytes):
        data = generated(name, nbytes)
        if name == "blk.1.ffn_up_exps.weight":
            data = data.copy()
            data[17 * 12345] = 0  # one block's E8M0 byte
        return data

    tensors = gpt_oss_tensors(LAYERS, EXPERTS, VOCAB, with_edge, GGML_Q8_0)
    path = os.path.join(tmp_path, "gpt-oss-edge.gguf")
    write_gguf(path, gpt_oss_metadata(LAYERS, EXPERTS), tensors)
    gpu = ttlab_amd.Model.from_gguf(path, CAPACITY, strict=False)
    try:
        tokens = [int(t) for t in np.random.default_rng(23).integers(0, VOCAB, 6)]
        logits = gpu.prefill(tokens)
        with pytest.raises(ttlab_amd.TtlError, match="decode steps"):
            gpu.prefill_state(0, len(tokens))
        for p, tok in enumerate(tokens):
            last = gpu.forward(tok, p)
        assert np.array_equal(logits.view(np.uint32), last.view(np.uint32))
    finally:
        gpu.close()
