"""Oracle-side copy of the synthetic gpt-oss model that ttlab::HipGptOssModel generates
on the device (same generator streams, see tt-lab_amd/host/gpt_oss_hip.hpp)."""
import ctypes as C

import numpy as np

import oracle_lib as O

N = 2880
QW, KW = 4096, 512

ATTN_NORM, POST_NORM, QUERY, KEY, VALUE, QKV_BIAS, ATTN_OUT, ATTN_OUT_BIAS, SINKS = 1, 2, 3, 4, 5, 6, 7, 8, 9
ROUTER, ROUTER_BIAS, GATE, UP, DOWN, GATE_BIAS, UP_BIAS, DOWN_BIAS = 10, 11, 12, 13, 14, 15, 16, 17
EMBEDDING, OUTPUT_NORM, UNEMBEDDING = 1, 2, 3


def stream(layer, kind):
    return (layer + 1) * 100000 + kind * 1000


class HostModelLayer:
    """One layer's tensors.  lazy=True leaves the expert matrices zero until
    ensure_experts() generates the ones an oracle run reads (120b-shaped layers hold
    128 experts x 3 x 4.4 MB)."""

    def __init__(self, seed, l, experts, lazy=False):
        n = lambda kind, count, sigma, mean=0.0: O.synth_normal(seed, stream(l, kind), count, sigma=sigma, mean=mean)
        self.attn_norm = n(ATTN_NORM, N, 0.05, 1.0)
        self.post_norm = n(POST_NORM, N, 0.05, 1.0)
        self.q = O.synth_q8_0(seed, stream(l, QUERY), QW * 90)
        self.k = O.synth_q8_0(seed, stream(l, KEY), KW * 90)
        self.v = O.synth_q8_0(seed, stream(l, VALUE), KW * 90)
        qkv_b = n(QKV_BIAS, QW + 2 * KW, 0.05)
        self.q_b, self.k_b, self.v_b = qkv_b[:QW].copy(), qkv_b[QW:QW + KW].copy(), qkv_b[QW + KW:].copy()
        self.o = O.synth_q8_0(seed, stream(l, ATTN_OUT), N * 128)
        self.o_b = n(ATTN_OUT_BIAS, N, 0.05)
        self.sinks = n(SINKS, 64, 1.0)
        self.router = O.synth_normal_bf16(seed, stream(l, ROUTER), experts * N, 0.02)
        self.router_b = n(ROUTER_BIAS, experts, 0.02)
        self.seed, self.l = seed, l
        per = N * 90 * 17
        self.gate, self.up, self.down = (np.zeros(experts * per, np.uint8) for _ in range(3))
        self.filled = set()
        self.ensure_experts(range(experts) if not lazy else [])
        self.gate_b = n(GATE_BIAS, experts * N, 0.05)
        self.up_b = n(UP_BIAS, experts * N, 0.05)
        self.down_b = n(DOWN_BIAS, experts * N, 0.05)
        self.experts = experts

    def ensure_experts(self, ids):
        per = N * 90 * 17
        for e in sorted(set(int(i) for i in ids) - self.filled):
            for arr, kind in ((self.gate, GATE), (self.up, UP), (self.down, DOWN)):
                arr[e * per:(e + 1) * per] = O.synth_mxfp4(self.seed, stream(self.l, kind) + e, N * 90)
            self.filled.add(e)

    def struct(self):
        s = O.OrcLayer()
        s.attention_norm = self.attn_norm.ctypes.data
        s.post_attention_norm = self.post_norm.ctypes.data
        s.query_weight, s.query_bias = self.q.ctypes.data, self.q_b.ctypes.data
        s.key_weight, s.key_bias = self.k.ctypes.data, self.k_b.ctypes.data
        s.value_weight, s.value_bias = self.v.ctypes.data, self.v_b.ctypes.data
        s.output_weight, s.output_bias = self.o.ctypes.data, self.o_b.ctypes.data
        s.sinks = self.sinks.ctypes.data
        m = s.moe
        m.hidden, m.expert_hidden, m.experts, m.used = N, N, self.experts, 4
        m.router_weight, m.router_bias = self.router.ctypes.data, self.router_b.ctypes.data
        m.gate_weight, m.gate_bias = self.gate.ctypes.data, self.gate_b.ctypes.data
        m.up_weight, m.up_bias = self.up.ctypes.data, self.up_b.ctypes.data
        m.down_weight, m.down_bias = self.down.ctypes.data, self.down_b.ctypes.data
        self._keep = s
        return s


class _LazyLayers:
    """Layer l of the host copy is generated the first time it is indexed, so a full
    24- or 36-layer model costs only the layers a test reads."""

    def __init__(self, seed, count, experts, lazy):
        self.seed, self.count, self.experts, self.lazy = seed, count, experts, lazy
        self.built = {}

    def __len__(self):
        return self.count

    def __getitem__(self, l):
        if not 0 <= l < self.count:
            raise IndexError(l)
        if l not in self.built:
            self.built[l] = HostModelLayer(self.seed, l, self.experts, self.lazy)
        return self.built[l]


class HostModel:
    def __init__(self, seed, layers, experts, vocab, lazy=False):
        self.seed, self.vocab = seed, vocab
        self.layers = _LazyLayers(seed, layers, experts, lazy)
        self.output_norm = O.synth_normal(seed, stream(-1, OUTPUT_NORM), N, sigma=0.05, mean=1.0)
        self._unembedding = None
        self.freqs = np.empty(32, np.float32)
        O.lib.orc_rope_frequencies(self.freqs)

    @property
    def unembedding(self):
        """bf16 [vocab][2880], generated on first use (1.16 GB at the full vocabulary)."""
        if self._unembedding is None:
            self._unembedding = O.synth_bf16(self.seed, stream(-1, UNEMBEDDING), self.vocab * N)
        return self._unembedding

    def embedding(self, token):
        row = O.synth_q8_0(self.seed, stream(-1, EMBEDDING), 90, block_offset=token * 90)
        out = np.empty(N, np.float32)
        O.lib.orc_load_token_embedding_q8_0(row, N, 0, out)
        return out

    def layer_forward(self, l, position, x_in, key_cache, value_cache, body=O.BODY_V4):
        """orc_layer_forward; caches are f32 [capacity*512] arrays updated in place."""
        x_out = np.empty(N, np.float32)
        q = np.empty(QW, np.float32)
        att = np.empty(QW, np.float32)
        res = np.empty(N, np.float32)
        router = np.empty(self.layers[l].experts, np.float32)
        idx = np.empty(4, np.int64)
        w = np.empty(4, np.float32)
        layer = self.layers[l]
        kc0, vc0 = key_cache.copy(), value_cache.copy()
        while True:
            s = layer.struct()
            O.lib.orc_layer_forward(C.byref(s), l, position, np.ascontiguousarray(x_in, np.float32), self.freqs,
                                    key_cache, value_cache, body, x_out, q, att, res, router, idx, w)
            if set(int(i) for i in idx) <= layer.filled:
                break
            # a lazy layer had not generated the experts this token routes to: fill, rerun
            layer.ensure_experts(idx)
            key_cache[:], value_cache[:] = kc0, vc0
        return {"x_out": x_out, "query": q, "attended": att, "residual": res, "router": router, "indices": idx,
                "weights": w}

    def logits(self, x_final):
        normed = np.empty(N, np.float32)
        O.lib.orc_rms_norm(np.ascontiguousarray(x_final, np.float32), self.output_norm, N, 1e-5, normed)
        out = np.empty(self.vocab, np.float32)
        O.lib.orc_matvec_bf16(self.unembedding, self.vocab, N, normed, out)
        return out
