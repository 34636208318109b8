"""Writes GGUF version-3 files (test infrastructure).

The layout the reference's reader expects (gguf.cpp:145-239): "GGUF", version 3,
tensor and key counts, key/values, tensor descriptors (name, rank, GGML-order
shape, type, offset into the data section), then the data section at the header
end rounded up to the alignment, each tensor at an aligned offset.
"""
import struct

import numpy as np

U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
GGML_F32, GGML_Q8_0, GGML_BF16, GGML_MXFP4 = 0, 8, 30, 39
_SCALAR = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<B", U64: "<Q",
           I64: "<q", F64: "<d"}


def _string(s):
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _value(kind, value):
    if kind == STRING:
        return _string(value)
    if kind == ARRAY:
        element, items = value
        out = struct.pack("<IQ", element, len(items))
        if element == STRING:
            return out + b"".join(_string(i) for i in items)
        return out + b"".join(struct.pack(_SCALAR[element], i) for i in items)
    return struct.pack(_SCALAR[kind], value)


def write_gguf(path, metadata, tensors, alignment=32, version=3, magic=0x46554747):
    """metadata: [(key, kind, value)]; tensors: [(name, shape (GGML order), type, bytes)]."""
    header = struct.pack("<IIQQ", magic, version, len(tensors), len(metadata))
    kv = b"".join(_string(k) + struct.pack("<I", kind) + _value(kind, v) for k, kind, v in metadata)
    infos, offsets, offset = [], [], 0
    for name, shape, ggml_type, data in tensors:
        offsets.append(offset)
        infos.append(_string(name) + struct.pack("<I", len(shape)) + b"".join(struct.pack("<Q", d) for d in shape) +
                     struct.pack("<IQ", ggml_type, offset))
        nbytes = data.nbytes if isinstance(data, np.ndarray) else len(data)
        offset = (offset + nbytes + alignment - 1) // alignment * alignment
    head = header + kv + b"".join(infos)
    with open(path, "wb") as f:
        f.write(head)
        f.write(b"\0" * ((-len(head)) % alignment))
        for _, _, _, data in tensors:
            raw = data.tobytes() if isinstance(data, np.ndarray) else bytes(data)
            f.write(raw)
            f.write(b"\0" * ((-len(raw)) % alignment))


def gpt_oss_metadata(layers, experts, overrides=None, drop=()):
    """The keys GptOssModel's constructor reads (model.cpp:68-97), with its values."""
    md = [
        ("general.architecture", STRING, "gpt-oss"),
        ("gpt-oss.block_count", U32, layers),
        ("gpt-oss.context_length", U32, 131072),
        ("gpt-oss.embedding_length", U32, 2880),
        ("gpt-oss.feed_forward_length", U32, 2880),
        ("gpt-oss.attention.head_count", U32, 64),
        ("gpt-oss.attention.head_count_kv", U32, 8),
        ("gpt-oss.attention.key_length", U32, 64),
        ("gpt-oss.attention.value_length", U32, 64),
        ("gpt-oss.expert_used_count", U32, 4),
        ("gpt-oss.expert_feed_forward_length", U32, 2880),
        ("gpt-oss.attention.sliding_window", U32, 128),
        ("gpt-oss.attention.layer_norm_rms_epsilon", F32, 1e-5),
        ("gpt-oss.rope.freq_base", F32, 150000.0),
        ("gpt-oss.rope.scaling.factor", F32, 32.0),
        ("gpt-oss.rope.scaling.original_context_length", U32, 4096),
        ("gpt-oss.rope.scaling.yarn_beta_fast", F32, 32.0),
        ("gpt-oss.rope.scaling.yarn_beta_slow", F32, 1.0),
        ("gpt-oss.expert_count", U32, experts),
        ("tokenizer.ggml.tokens", ARRAY, (STRING, ["<a>", "<b>"])),
    ]
    overrides = overrides or {}
    out = []
    for key, kind, value in md:
        if key in drop:
            continue
        if key in overrides:
            kind, value = overrides[key]
        out.append((key, kind, value))
    return out


def gpt_oss_tensors(layers, experts, vocab, data, output_type=GGML_Q8_0):
    """Tensor list for a gpt-oss model; data(name, nbytes) returns the bytes of each
    (so tests can fill them with generated weights or zeros)."""
    H, Q, KV = 2880, 4096, 512
    q8 = lambda cols, rows: rows * (cols // 32) * 34
    mx = lambda cols, rows, e: e * rows * (cols // 32) * 17
    t = []

    def add(name, shape, ggml_type, nbytes):
        t.append((name, shape, ggml_type, data(name, nbytes)))

    add("token_embd.weight", [H, vocab], GGML_Q8_0, q8(H, vocab))
    add("output_norm.weight", [H], GGML_F32, 4 * H)
    add("output.weight", [H, vocab], output_type, q8(H, vocab) if output_type == GGML_Q8_0 else 2 * H * vocab)
    for l in range(layers):
        p = f"blk.{l}."
        add(p + "attn_norm.weight", [H], GGML_F32, 4 * H)
        add(p + "post_attention_norm.weight", [H], GGML_F32, 4 * H)
        add(p + "attn_q.weight", [H, Q], GGML_Q8_0, q8(H, Q))
        add(p + "attn_q.bias", [Q], GGML_F32, 4 * Q)
        add(p + "attn_k.weight", [H, KV], GGML_Q8_0, q8(H, KV))
        add(p + "attn_k.bias", [KV], GGML_F32, 4 * KV)
        add(p + "attn_v.weight", [H, KV], GGML_Q8_0, q8(H, KV))
        add(p + "attn_v.bias", [KV], GGML_F32, 4 * KV)
        add(p + "attn_output.weight", [Q, H], GGML_Q8_0, q8(Q, H))
        add(p + "attn_output.bias", [H], GGML_F32, 4 * H)
        add(p + "attn_sinks.weight", [64], GGML_F32, 4 * 64)
        add(p + "ffn_gate_inp.weight", [H, experts], GGML_F32, 4 * H * experts)
        add(p + "ffn_gate_inp.bias", [experts], GGML_F32, 4 * experts)
        for kind in ("gate", "up", "down"):
            add(p + f"ffn_{kind}_exps.weight", [H, H, experts], GGML_MXFP4, mx(H, H, experts))
            add(p + f"ffn_{kind}_exps.bias", [H, experts], GGML_F32, 4 * H * experts)
    return t
