"""The C++ facades from a compiled caller (tests/cpp/facade_check.cpp, built by the
Makefile as tt-lab_amd/build/facade_check), on a GGUF file written here.

- HipGptOssModel driven as main.cpp:373-411 drives GptOssModel: the generated tokens
  and last logits equal bit for bit those of the same model through the C ABI
  (ttlm_*, which test_gpu_gguf.py checks against the oracle), and the reference's
  error messages come back as std::runtime_error (model.cpp:463-472, 557-566,
  gguf.cpp:150-153).
- ttlab_run (host/ttlab_run.cpp), the reference CLI's `run` loop on token ids: the same
  tokens, and the generation ends at tokenizer.ggml.eos_token_id (main.cpp:373-411).
- HipTensorBackend, the tensor.h functions: the embedding row and the F32 router
  matvec (the exact path) equal the oracle's bit for bit; rms_norm, the Q8_0 and
  MXFP4 matvecs and the selected-token matmul agree with it to relative L2 <= 1e-5;
  rows the selection does not name stay untouched.  After the first file is closed,
  the same MXFP4 call on a second file of the same shapes uses the second file's
  weights.
Every facade call in the caller goes through types shaped like the reference's
GgufTensor and GgufFile (gguf.h:38-72), and the model is built with the reference's
constructor arguments (model.h:19-20).
"""
import os
import subprocess

import numpy as np
import pytest

import oracle_lib as O
import ttlab_amd
from gguf_writer import GGML_Q8_0, U32, gpt_oss_metadata, gpt_oss_tensors, write_gguf
from test_gpu_gguf import EXPERTS, LAYERS, VOCAB, generated

pytestmark = pytest.mark.gpu
TOL = 1e-5
N = 2880
BINARY = os.path.join(os.path.dirname(ttlab_amd.LIB_PATH), "facade_check")
CLI = os.path.join(os.path.dirname(ttlab_amd.LIB_PATH), "ttlab_run")
PROMPT = [17, 300, 5, 941, 2, 77, 512]
LIMIT = 5


@pytest.fixture(scope="module")
def run(tmp_path_factory):
    if not os.path.exists(BINARY):
        raise RuntimeError(f"{BINARY} is missing: run __graft_entry__.build() (make -C tt-lab_amd)")
    tensors = gpt_oss_tensors(LAYERS, EXPERTS, VOCAB, generated, GGML_Q8_0)
    tmp = tmp_path_factory.mktemp("facade")
    path = os.path.join(tmp, "gpt-oss-small.gguf")
    # an end-of-sequence id no argmax can produce (the run loop requires the key, as
    # main.cpp does), so the command line generates to its limit
    write_gguf(path, gpt_oss_metadata(LAYERS, EXPERTS) + [("tokenizer.ggml.eos_token_id", U32, VOCAB)], tensors)
    # a second file of the same shapes with other weights
    def moved(name, nbytes):
        data = generated(name, nbytes)
        # the expert blocks one block further on: valid MXFP4, other weights per row
        return np.roll(data.reshape(-1, 17), 1, axis=0).ravel() if name.endswith("_exps.weight") else data

    other = gpt_oss_tensors(LAYERS, EXPERTS, VOCAB, moved, GGML_Q8_0)
    second = os.path.join(tmp, "gpt-oss-small-second.gguf")
    write_gguf(second, gpt_oss_metadata(LAYERS, EXPERTS) + [("tokenizer.ggml.eos_token_id", U32, VOCAB)], other)
    print(f"running {BINARY} on {path} (then {second})", flush=True)
    done = subprocess.run([BINARY, "--second", second, path, str(tmp), str(LIMIT)] + [str(t) for t in PROMPT],
                          capture_output=True, text=True, timeout=300)
    print(done.stdout, done.stderr)
    assert done.returncode == 0, done.stderr
    t = {name: data for name, _, _, data in tensors}
    t.update({"second/" + name: data for name, _, _, data in other})
    return str(tmp), path, t


def floats(tmp, name):
    return np.fromfile(os.path.join(tmp, name), np.float32)


def test_model_loop_matches_the_c_abi_path(run):
    tmp, path, _ = run
    tokens = [int(v) for v in open(os.path.join(tmp, "tokens.txt")).read().split()]
    model = ttlab_amd.Model.from_gguf(path, len(PROMPT) + LIMIT, strict=False)
    try:
        logits = model.prefill(PROMPT)
        expected = []
        for i in range(LIMIT):
            expected.append(int(O.lib.orc_greedy(logits, VOCAB)))
            if i + 1 < LIMIT:
                logits = model.forward(expected[-1], len(PROMPT) + i)
    finally:
        model.close()
    assert tokens == expected
    assert np.array_equal(floats(tmp, "logits.f32").view(np.uint32), logits.view(np.uint32))


def test_reference_error_messages(run):
    tmp, _, _ = run
    lines = open(os.path.join(tmp, "errors.txt")).read().splitlines()
    assert lines[0] == "input token is out of range"
    assert lines[1] == "position exceeds startup token capacity"
    assert lines[2] == "prefill exceeds startup batch capacity"
    assert lines[3] == "prefill needs at least one token"
    assert lines[4] == f"cannot open {tmp}/no-such-model.gguf: No such file or directory"
    assert lines[5] == "tensor dumps are not supported by the gfx950 backend"
    assert lines[6] == "batch capacity exceeds token capacity"  # model.cpp:105-107


def test_tensor_functions_against_oracle(run):
    tmp, _, t = run
    x = np.empty(N, np.float32)
    O.lib.orc_load_token_embedding_q8_0(t["token_embd.weight"], N, PROMPT[0], x)
    assert np.array_equal(floats(tmp, "embedding.f32").view(np.uint32), x.view(np.uint32))

    normed = np.empty(N, np.float32)
    O.lib.orc_rms_norm(x, t["blk.0.attn_norm.weight"], N, 1e-5, normed)
    got_norm = floats(tmp, "norm.f32")
    assert O.rel_l2(got_norm, normed) <= TOL
    # the device's later outputs are checked on the vector the device produced
    normed = got_norm

    q = np.empty(4096, np.float32)
    O.lib.orc_matvec_add_q8_0(t["blk.0.attn_q.weight"], t["blk.0.attn_q.bias"], 4096, N, normed, q)
    assert O.rel_l2(floats(tmp, "q8.f32"), q) <= TOL

    router = np.empty(EXPERTS, np.float32)
    O.lib.orc_matvec_add_f32(t["blk.0.ffn_gate_inp.weight"], t["blk.0.ffn_gate_inp.bias"], EXPERTS, N, normed,
                             router)
    assert np.array_equal(floats(tmp, "router.f32").view(np.uint32), router.view(np.uint32))

    expert = EXPERTS - 1
    gate = np.empty(N, np.float32)
    O.lib.orc_matvec_add_mxfp4(t["blk.0.ffn_gate_exps.weight"], t["blk.0.ffn_gate_exps.bias"], N, N, normed, gate,
                               expert, O.BODY_DEFAULT)
    assert O.rel_l2(floats(tmp, "mxfp4.f32"), gate) <= TOL
    # the second file's gate, on the same input, after the first file was closed
    O.lib.orc_matvec_add_mxfp4(t["second/blk.0.ffn_gate_exps.weight"], t["second/blk.0.ffn_gate_exps.bias"], N, N,
                               normed, gate, expert, O.BODY_DEFAULT)
    assert O.rel_l2(floats(tmp, "mxfp4_second.f32"), gate) <= TOL


def test_selected_matmul_against_oracle(run):
    tmp, _, t = run
    inputs = floats(tmp, "selected_inputs.f32")
    sel = np.array([5, 1, 3], np.uintp)
    transposed = np.empty(3 * N, np.float32)
    O.lib.orc_transpose_selected(N, inputs, sel, 3, transposed)
    ref = np.full(6 * N, np.nan, np.float32)
    ws = np.empty(4 * 3 + 8, np.float32)
    O.lib.orc_matmul_add_mxfp4_selected_transposed(t["blk.0.ffn_gate_exps.weight"], t["blk.0.ffn_gate_exps.bias"], N,
                                                   N, transposed, sel, 3, ref, ws, EXPERTS - 1, O.BODY_DEFAULT)
    got = floats(tmp, "selected.f32").reshape(6, N)
    ref = ref.reshape(6, N)
    for s in (5, 1, 3):
        assert O.rel_l2(got[s], ref[s]) <= TOL, s
    for s in (0, 2, 4):
        assert np.isnan(got[s]).all(), s


def generate_cli(path, limit):
    done = subprocess.run([CLI, "run", "-m", path, "--loose", "-t", ",".join(str(t) for t in PROMPT), "-n",
                           str(limit)], capture_output=True, text=True, timeout=300)
    print(done.stdout, done.stderr)
    assert done.returncode == 0, done.stderr
    return [int(v) for v in done.stdout.split()], done.stderr


def test_command_line_generates_the_c_abi_tokens(run):
    tmp, path, _ = run
    tokens = [int(v) for v in open(os.path.join(tmp, "tokens.txt")).read().split()]
    out, err = generate_cli(path, LIMIT)
    assert out == tokens
    assert f"prefill: {len(PROMPT)} tokens" in err and f"generated: {LIMIT} tokens" in err
    assert f"decode: {LIMIT - 1} evals" in err


def test_command_line_stops_at_end_of_sequence(run):
    tmp, _, _ = run
    tokens = [int(v) for v in open(os.path.join(tmp, "tokens.txt")).read().split()]
    eos = tokens[2]
    path = os.path.join(tmp, "gpt-oss-small-eos.gguf")
    write_gguf(path, gpt_oss_metadata(LAYERS, EXPERTS) + [("tokenizer.ggml.eos_token_id", U32, eos)],
               gpt_oss_tensors(LAYERS, EXPERTS, VOCAB, generated, GGML_Q8_0))
    out, err = generate_cli(path, LIMIT)
    assert out == tokens[:tokens.index(eos)]
    # main.cpp counts the forward that produced the end-of-sequence id
    assert f"generated: {len(out)} tokens" in err and f"decode: {len(out)} evals" in err


def test_command_line_text_prompt(run):
    """`ttlab_run run -p <text>` (main.cpp:291-411): the prompt in the Harmony template,
    encoded by ttlab::Tokenizer (its ids the tokenizer oracle's), generates what the same
    ids given with -t generate, and prints the formatted prompt followed by each
    generated token's bytes (decode_to, special tokens rendered)."""
    import sys
    sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "oracle"))
    import tokenizer_oracle as T
    from gguf_writer import ARRAY, I32, STRING
    from test_tokenizer import CORPUS, SPECIALS, byte_chars, train_merges

    tmp, _, _ = run
    alpha = byte_chars()
    merges = train_merges(CORPUS, 300)
    tokens, seen = list(alpha), set(alpha)
    for a, b in merges:
        if a + b not in seen and len(tokens) < VOCAB - len(SPECIALS):
            seen.add(a + b)
            tokens.append(a + b)
    k = 0
    while len(tokens) < VOCAB - len(SPECIALS):  # filler ordinary tokens, two byte characters each
        t = alpha[(k // 256) % 256] + alpha[k % 256]  # every pair in turn
        k += 1
        if t not in seen:
            seen.add(t)
            tokens.append(t)
    types = [1] * len(tokens) + [3] * len(SPECIALS)
    tokens += SPECIALS
    merge_text = [f"{a} {b}" for a, b in merges]
    md = gpt_oss_metadata(LAYERS, EXPERTS, overrides={"tokenizer.ggml.tokens": (ARRAY, (STRING, tokens))})
    md += [("tokenizer.ggml.model", STRING, "gpt2"), ("tokenizer.ggml.pre", STRING, "gpt-4o"),
           ("tokenizer.ggml.token_type", ARRAY, (I32, types)), ("tokenizer.ggml.merges", ARRAY, (STRING, merge_text)),
           ("tokenizer.ggml.eos_token_id", U32, VOCAB)]
    path = os.path.join(tmp, "gpt-oss-small-text.gguf")
    write_gguf(path, md, gpt_oss_tensors(LAYERS, EXPERTS, VOCAB, generated, GGML_Q8_0))
    oracle = T.Tokenizer(tokens, types, merge_text)
    user = "Hello world, what's 2+2?"
    formatted = T.harmony_prompt(user.encode())
    ids = oracle.encode(formatted)
    by_ids = subprocess.run([CLI, "run", "-m", path, "--loose", "-t", ",".join(str(t) for t in ids), "-n",
                             str(LIMIT)], capture_output=True, timeout=300)
    assert by_ids.returncode == 0, by_ids.stderr
    out_ids = [int(v) for v in by_ids.stdout.split()]
    assert len(out_ids) == LIMIT
    by_text = subprocess.run([CLI, "run", "-m", path, "--loose", "-p", user, "-n", str(LIMIT)], capture_output=True,
                             timeout=300)
    print(by_text.stdout, by_text.stderr.decode())
    assert by_text.returncode == 0, by_text.stderr
    assert by_text.stdout == formatted + b"".join(oracle.decode(t) for t in out_ids) + b"\n"
    assert f"prefill: {len(ids)} tokens".encode() in by_text.stderr
