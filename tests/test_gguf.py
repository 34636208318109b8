"""The GGUF reader and the reference's model checks (no device needed).

Files come from tests/gguf_writer.py; ttlm_gguf_inspect runs the reader
(gguf.cpp:145-239's format rules) and GptOssModel's constructor checks
(model.cpp:64-228) and must give the reference's error messages.
"""
import os

import numpy as np
import pytest

import ttlab_amd
from gguf_writer import (GGML_BF16, GGML_F32, GGML_Q8_0, STRING, U32, gpt_oss_metadata, gpt_oss_tensors,
                         write_gguf)

LAYERS, EXPERTS, VOCAB = 1, 4, 32


def zeros(name, nbytes):
    return np.zeros(nbytes, np.uint8)


def model_file(tmp_path, name="m.gguf", layers=LAYERS, experts=EXPERTS, vocab=VOCAB, overrides=None, drop=(),
               output_type=GGML_Q8_0, edit=None, **kw):
    tensors = gpt_oss_tensors(layers, experts, vocab, zeros, output_type)
    if edit:
        tensors = edit(tensors)
    path = os.path.join(tmp_path, name)
    write_gguf(path, gpt_oss_metadata(layers, experts, overrides, drop), tensors, **kw)
    return path


def inspect_error(path, strict=False):
    with pytest.raises(ttlab_amd.TtlError) as e:
        ttlab_amd.gguf_inspect(path, strict)
    return str(e.value)


def test_small_model_file_is_read(tmp_path):
    info = ttlab_amd.gguf_inspect(model_file(tmp_path), strict=False)
    assert info == {"layers": LAYERS, "experts": EXPERTS, "vocab": VOCAB, "output_type": 8,
                    "tensors": 3 + 19 * LAYERS}
    bf = ttlab_amd.gguf_inspect(model_file(tmp_path, "b.gguf", output_type=GGML_BF16), strict=False)
    assert bf["output_type"] == 30


def test_alignment_key(tmp_path):
    # gguf.cpp:218-225: tensor data starts at the header end rounded up to general.alignment
    md = gpt_oss_metadata(LAYERS, EXPERTS) + [("general.alignment", U32, 64)]
    p = os.path.join(tmp_path, "a64.gguf")
    write_gguf(p, md, gpt_oss_tensors(LAYERS, EXPERTS, VOCAB, zeros), alignment=64)
    assert ttlab_amd.gguf_inspect(p, False)["layers"] == LAYERS
    bad = os.path.join(tmp_path, "a48.gguf")
    write_gguf(bad, gpt_oss_metadata(LAYERS, EXPERTS) + [("general.alignment", U32, 48)],
               gpt_oss_tensors(LAYERS, EXPERTS, VOCAB, zeros), alignment=16)
    assert inspect_error(bad).endswith("invalid GGUF alignment")
    wrong = os.path.join(tmp_path, "astr.gguf")
    write_gguf(wrong, gpt_oss_metadata(LAYERS, EXPERTS) + [("general.alignment", STRING, "32")],
               gpt_oss_tensors(LAYERS, EXPERTS, VOCAB, zeros))
    assert inspect_error(wrong).endswith("general.alignment is not uint32")


def test_strict_mode_is_the_references_limits(tmp_path):
    # model.cpp:72-74: only 24 or 36 blocks
    assert inspect_error(model_file(tmp_path), strict=True) == \
        "ttlm_gguf_inspect failed: only gpt-oss-20b and gpt-oss-120b are supported"


def test_reference_error_messages(tmp_path):
    cases = [
        (dict(overrides={"general.architecture": (STRING, "llama")}), "model architecture is not gpt-oss"),
        (dict(overrides={"gpt-oss.attention.sliding_window": (U32, 64)}),
         "unsupported gpt-oss.attention.sliding_window"),
        (dict(overrides={"gpt-oss.rope.freq_base": (U32, 10000)}), "unsupported gpt-oss.rope.freq_base"),
        (dict(drop=("gpt-oss.expert_count",)), "missing GGUF key: gpt-oss.expert_count"),
        (dict(overrides={"gpt-oss.block_count": (STRING, "24")}), "GGUF key is not an integer: gpt-oss.block_count"),
        (dict(overrides={"gpt-oss.expert_count": (U32, 2)}), "unsupported expert count"),
    ]
    for i, (kw, message) in enumerate(cases):
        assert inspect_error(model_file(tmp_path, f"c{i}.gguf", **kw)).endswith(message), (kw, message)


def test_tensor_checks(tmp_path):
    def drop(name):
        return lambda ts: [t for t in ts if t[0] != name]

    def retype(name, ggml_type):
        return lambda ts: [(n, s, ggml_type if n == name else ty, d) for n, s, ty, d in ts]

    def reshape(name, shape):
        return lambda ts: [(n, shape if n == name else s, ty, d) for n, s, ty, d in ts]

    cases = [
        (drop("blk.0.attn_k.bias"), "missing tensor blk.0.attn_k.bias"),
        (retype("blk.0.attn_norm.weight", GGML_Q8_0), "wrong type for tensor blk.0.attn_norm.weight"),
        (reshape("blk.0.attn_sinks.weight", [64, 1]), "wrong rank for tensor blk.0.attn_sinks.weight"),
        (reshape("blk.0.ffn_gate_inp.bias", [EXPERTS + 1]), "wrong shape for tensor blk.0.ffn_gate_inp.bias"),
    ]
    for i, (edit, message) in enumerate(cases):
        assert inspect_error(model_file(tmp_path, f"t{i}.gguf", edit=edit)).endswith(message), message


def test_file_format_errors(tmp_path):
    good = model_file(tmp_path)
    raw = open(good, "rb").read()
    bad_magic = os.path.join(tmp_path, "magic.gguf")
    open(bad_magic, "wb").write(b"GGUX" + raw[4:])
    assert inspect_error(bad_magic).endswith("not a GGUF file")
    v2 = os.path.join(tmp_path, "v2.gguf")
    open(v2, "wb").write(raw[:4] + (2).to_bytes(4, "little") + raw[8:])
    assert inspect_error(v2).endswith("unsupported GGUF version 2")
    short = os.path.join(tmp_path, "short.gguf")
    open(short, "wb").write(raw[:len(raw) - 4096])
    assert inspect_error(short).endswith("tensor extends past end of GGUF file")
    header = os.path.join(tmp_path, "header.gguf")
    open(header, "wb").write(raw[:100])
    assert inspect_error(header).endswith("truncated GGUF file")
    dup = os.path.join(tmp_path, "dup.gguf")
    md = gpt_oss_metadata(LAYERS, EXPERTS)
    write_gguf(dup, md + [md[1]], gpt_oss_tensors(LAYERS, EXPERTS, VOCAB, zeros))
    assert inspect_error(dup).endswith("duplicate GGUF key: gpt-oss.block_count")
    missing = os.path.join(tmp_path, "nope.gguf")
    assert "cannot open" in inspect_error(missing)
    f32_row = os.path.join(tmp_path, "f32.gguf")
    write_gguf(f32_row, md, [("x", [33], 8, np.zeros(64, np.uint8))])
    assert inspect_error(f32_row).endswith("Q8_0 row is not a multiple of 32")
    assert GGML_F32 == 0
