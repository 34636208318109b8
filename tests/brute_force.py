"""Float64 brute force of the gpt-oss decoder layer, written from the reference's
definitions (tenstorrent/tt-lab src/model.cpp, src/tensor.cpp) without the oracle's
code: numpy decodes the formats, sums in float64 and evaluates the transcendental
functions in float64.  Test infrastructure: it checks the oracle, which checks the GPU.

Where the reference fixes a rounding as part of the definition, the brute force keeps
it: RoPE's angle is the float32 product float(position) * frequency (model.cpp:237),
so the frequency table (float32, checked against its closed form by
test_oracle_compute.test_rope_frequencies_against_float64) is an input here.
"""
import numpy as np

N = 2880
HEAD, Q_HEADS, KV_HEADS, WINDOW = 64, 64, 8, 128
E2M1 = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0])


def mxfp4_dense(blocks, rows, cols):
    """GGUF MXFP4 rows as float64: E2M1 magnitude (code & 7), sign bit 3, times
    2^(e-127); byte 1+i's low nibble is element i and its high nibble element i+16
    (tensor.cpp:34-44, 283-296)."""
    b = np.asarray(blocks).reshape(rows, cols // 32, 17)
    scale = np.ldexp(1.0, b[:, :, 0].astype(np.int64) - 127)
    qs = b[:, :, 1:]
    lo, hi = qs & 15, qs >> 4

    def val(c):
        v = E2M1[c & 7]
        return np.where(c & 8, -v, v)
    w = np.concatenate([val(lo), val(hi)], axis=2) * scale[:, :, None]
    return w.reshape(rows, cols)


def q8_dense(blocks, rows, cols):
    """GGUF Q8_0 rows as float64: per 32 values an IEEE half scale, then 32 int8."""
    b = np.asarray(blocks).reshape(rows, cols // 32, 34)
    d = b[:, :, :2].copy().view(np.uint16)[..., 0].view(np.float16).astype(np.float64)
    return (b[:, :, 2:].view(np.int8).astype(np.float64) * d[:, :, None]).reshape(rows, cols)


def rms_norm(x, w, eps=1e-5):
    x = np.asarray(x, np.float64)
    return x / np.sqrt(np.mean(x * x) + eps) * np.asarray(w, np.float64)


def rope(vec, heads, position, freqs32):
    """model.cpp:230-245: pairs (d, d + 32) of each head rotated by theta = the float32
    product float(position) * frequency, scaled by 1 + 0.1 ln 32 (rope_scale 1/32)."""
    theta = (np.float32(position) * np.asarray(freqs32, np.float32)).astype(np.float64)
    mag = 1.0 + 0.1 * np.log(32.0)
    c, s = np.cos(theta) * mag, np.sin(theta) * mag
    v = np.asarray(vec, np.float64).reshape(heads, HEAD)
    x, y = v[:, :HEAD // 2], v[:, HEAD // 2:]
    return np.concatenate([x * c - y * s, x * s + y * c], axis=1).ravel()


def attention(q, kc, vc, sinks, layer_index, position):
    """model.cpp:255-290: even layers see the last 128 positions, odd layers all; the
    sink takes part in the max and the denominator only."""
    first = position + 1 - WINDOW if (layer_index % 2 == 0 and position + 1 > WINDOW) else 0
    K = np.asarray(kc, np.float64).reshape(-1, KV_HEADS, HEAD)[first:position + 1]
    V = np.asarray(vc, np.float64).reshape(-1, KV_HEADS, HEAD)[first:position + 1]
    Q = np.asarray(q, np.float64).reshape(Q_HEADS, HEAD)
    out = np.empty((Q_HEADS, HEAD))
    for h in range(Q_HEADS):
        kv = h // (Q_HEADS // KV_HEADS)
        s = K[:, kv] @ Q[h] / 8.0
        m = max(s.max(), float(sinks[h]))
        e = np.exp(s - m)
        out[h] = (e / (e.sum() + np.exp(float(sinks[h]) - m))) @ V[:, kv]
    return out.ravel()


class DenseLayer:
    """One layer's weights decoded to float64 (expert matrices on first use)."""

    def __init__(self, host_layer):
        L = host_layer
        self.src = L
        self.attn_norm, self.post_norm = L.attn_norm, L.post_norm
        self.q, self.k, self.v = (q8_dense(L.q, 4096, N), q8_dense(L.k, 512, N), q8_dense(L.v, 512, N))
        self.q_b, self.k_b, self.v_b = (a.astype(np.float64) for a in (L.q_b, L.k_b, L.v_b))
        self.o, self.o_b = q8_dense(L.o, N, 4096), L.o_b.astype(np.float64)
        self.sinks = L.sinks.astype(np.float64)
        self.experts = L.experts
        self.router = L.router.astype(np.float64).reshape(L.experts, N)
        self.router_b = L.router_b.astype(np.float64)
        self.biases = {n: b.astype(np.float64).reshape(L.experts, N)
                       for n, b in (("gate", L.gate_b), ("up", L.up_b), ("down", L.down_b))}
        self._experts = {}

    def expert(self, name, e):
        key = (name, int(e))
        if key not in self._experts:
            self.src.ensure_experts([e])
            per = N * 90 * 17
            raw = getattr(self.src, name)[int(e) * per:(int(e) + 1) * per]
            self._experts[key] = mxfp4_dense(raw, N, N)
        return self._experts[key]


def moe(layer, x, used=4):
    """GptOssModel::moe (model.cpp:292-338) in float64: router logits, the `used`
    largest (earliest index first among equals), softmax over them, and per expert the
    clamped SwiGLU (alpha 1.702, limit 7) between gate/up and down."""
    x = np.asarray(x, np.float64)
    router = layer.router @ x + layer.router_b
    order = sorted(range(layer.experts), key=lambda j: (-router[j], j))[:used]
    sel = router[order]
    w = np.exp(sel - sel.max())
    w /= w.sum()
    out = np.zeros(N)
    for r, e in enumerate(order):
        g = layer.expert("gate", e) @ x + layer.biases["gate"][e]
        u = layer.expert("up", e) @ x + layer.biases["up"][e]
        xg = np.minimum(g, 7.0)
        h = xg / (1.0 + np.exp(-1.702 * xg)) * (np.clip(u, -7.0, 7.0) + 1.0)
        out += w[r] * (layer.expert("down", e) @ h + layer.biases["down"][e])
    return out, router, np.array(order), w


def qkv(layer, x, position, freqs32):
    n1 = rms_norm(x, layer.attn_norm)
    q = rope(layer.q @ n1 + layer.q_b, Q_HEADS, position, freqs32)
    k = rope(layer.k @ n1 + layer.k_b, KV_HEADS, position, freqs32)
    v = layer.v @ n1 + layer.v_b
    return q, k, v


def after_attention(layer, x, attended):
    """Output projection, residual, post-attention norm, MoE, second residual
    (model.cpp:584-595)."""
    residual = np.asarray(x, np.float64) + layer.o @ attended + layer.o_b
    out, router, idx, w = moe(layer, rms_norm(residual, layer.post_norm))
    return {"x_out": residual + out, "residual": residual, "attended": attended, "router": router, "indices": idx,
            "weights": w}


def layer_forward(layer, layer_index, position, x, key_cache, value_cache, freqs32):
    """GptOssModel::forward's layer body (model.cpp:571-595) at `position`.  The caches
    (float64 [>= position + 1][512]) receive the step's key and value."""
    q, k, v = qkv(layer, x, position, freqs32)
    key_cache[position], value_cache[position] = k, v
    att = attention(q, key_cache, value_cache, layer.sinks, layer_index, position)
    res = after_attention(layer, x, att)
    res.update(query=q, key=k, value=v)
    return res


def layer_prefill(layer, layer_index, first, xs, key_cache, value_cache, freqs32):
    """GptOssModel::prefill's layer body (model.cpp:484-553) for the tokens xs at
    positions first, first + 1, ...: every token's key and value are stored before any
    token attends."""
    qs = []
    for t, x in enumerate(xs):
        q, k, v = qkv(layer, x, first + t, freqs32)
        key_cache[first + t], value_cache[first + t] = k, v
        qs.append(q)
    return [after_attention(layer, x, attention(q, key_cache, value_cache, layer.sinks, layer_index, first + t))
            for t, (x, q) in enumerate(zip(xs, qs))]


def mxfp8_exponents(x):
    """The E8M0 exponent X of each 32-element block of x (the rule of
    include/ttlab_hip.h, TTL_DTYPE_F32_AS_MXFP8): the smallest X with
    max|x| / 2^X <= 448, but at least -127 (0 for a zero block; -127 whenever the
    maximum is at most 448 x 2^-127, f32 subnormals included).  Returns int64 X and
    bool finite per block (a block with a non-finite value has no exponent)."""
    b = np.asarray(x, np.float32).reshape(-1, 32).astype(np.float64)
    with np.errstate(invalid="ignore"):
        m = np.abs(b).max(axis=1)
    finite = np.isfinite(b).all(axis=1)
    mant, e = np.frexp(np.where(finite, m, 1.0))  # m = mant 2^e, mant in [0.5, 1)
    X = np.where(mant > 0.875, e - 8, e - 9)      # significand 2 mant > 1.75 -> one more
    X = np.maximum(X, -127)                       # E8M0 byte 0 (below it X wraps)
    X = np.where(finite & (m > 0), X, 0)
    return X.astype(np.int64), finite


def e4m3_round(v):
    """float64 v (|v| below 464) to the nearest OCP E4M3 value, ties to even:
    3 fraction bits, subnormals in steps of 2^-9."""
    a = np.abs(v)
    _, ae = np.frexp(np.maximum(a, 2.0 ** -6))
    step = np.ldexp(1.0, ae - 1 - 3)
    return np.sign(v) * np.round(a / step) * step  # numpy rounds half to even


def mxfp8_dequantize(x, exponents=None):
    """The MXFP8 values of x's 32-element blocks (mxfp8_exponents), widened back to
    float32: elements OCP E4M3 of x / 2^X rounded to nearest even; a block with a
    non-finite value becomes NaN.  exponents (int per block) replaces the rule's X."""
    b = np.asarray(x, np.float32).reshape(-1, 32).astype(np.float64)
    X, finite = mxfp8_exponents(x)
    if exponents is not None:
        X = np.asarray(exponents, np.int64).reshape(-1)
    v = np.ldexp(np.where(finite[:, None], b, 0.0), -X[:, None])
    out = np.ldexp(e4m3_round(v), X[:, None])
    out[~finite] = np.nan
    return out.astype(np.float32).reshape(np.shape(x))
