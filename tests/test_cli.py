"""The generation command line (tt-lab_amd/build/ttlab_run, host/ttlab_run.cpp) without a
device: its argument handling and exit codes (main.cpp:112-260: usage errors exit 2,
model errors print "error: <message>" and exit 1) and `inspect`, which applies the
model checks (model.cpp:64-228) to a file.  Generation is checked on the GPU
(test_gpu_cpp_facade.py)."""
import os
import subprocess

import pytest

import ttlab_amd
from test_gguf import EXPERTS, LAYERS, VOCAB, model_file

CLI = os.path.join(os.path.dirname(ttlab_amd.LIB_PATH), "ttlab_run")


def cli(*args):
    if not os.path.exists(CLI):
        raise RuntimeError(f"{CLI} is missing: run __graft_entry__.build() (make -C tt-lab_amd)")
    return subprocess.run([CLI, *args], capture_output=True, text=True, timeout=120)


def test_usage_errors_exit_2():
    assert cli().returncode == 2
    assert cli("generate").returncode == 2
    assert cli("run", "-t", "1,2").returncode == 2          # no model
    assert cli("run", "-m", "x.gguf").returncode == 2       # no prompt
    bad = cli("run", "-m", "x.gguf", "-t", "1,,2")
    assert bad.returncode == 2 and "invalid token list: 1,,2" in bad.stderr
    assert cli("run", "-m", "x.gguf", "-t", "-3").returncode == 2
    assert cli("run", "-m", "x.gguf", "-t", "1", "-n", "many").returncode == 2
    assert cli("inspect", "-m", "x.gguf", "-t", "1").returncode == 2
    assert cli("--help").returncode == 0


def test_model_errors_exit_1(tmp_path):
    missing = cli("run", "-m", str(tmp_path / "none.gguf"), "-t", "1", "-n", "1")
    assert missing.returncode == 1
    assert missing.stderr.strip() == f"error: cannot open {tmp_path}/none.gguf: No such file or directory"
    small = model_file(tmp_path)
    strict = cli("inspect", "-m", small)
    assert strict.returncode == 1
    assert strict.stderr.strip() == "error: only gpt-oss-20b and gpt-oss-120b are supported"


def test_inspect_prints_the_shape(tmp_path):
    done = cli("inspect", "-m", model_file(tmp_path), "--loose")
    assert done.returncode == 0, done.stderr
    assert done.stdout.strip() == f"gpt-oss model: {LAYERS} layers, {EXPERTS} experts, vocabulary {VOCAB}, " \
                                  "output.weight type 8"


def test_run_requires_the_end_of_sequence_id(tmp_path):
    """main.cpp:379 reads tokenizer.ggml.eos_token_id with GgufFile::integer, which
    throws for a missing key; the run loop does the same before it opens a device."""
    done = cli("run", "-m", model_file(tmp_path), "--loose", "-t", "1,2", "-n", "2")
    assert done.returncode == 1
    assert done.stderr.strip() == "error: missing GGUF key: tokenizer.ggml.eos_token_id"


def test_tokenize_prints_the_ids_of_the_text(tmp_path):
    """`ttlab_run tokenize -m <file> -p <text>`: the reference's print_tokens format
    (main.cpp:99-108, 286-289), the ids of ttlab::Tokenizer without the chat template,
    equal to the tokenizer oracle's; usage errors as the reference's."""
    import sys
    sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "oracle"))
    import tokenizer_oracle as T
    from test_tokenizer import CORPUS, train_merges, write_tokenizer

    path = str(tmp_path / "tok.gguf")
    lists = write_tokenizer(path, train_merges(CORPUS, 300))
    text = "Hello world, I'm here.<|end|> 12345"
    done = cli("tokenize", "-m", path, "-p", text)
    assert done.returncode == 0, done.stderr
    ids = T.Tokenizer(*lists).encode(text.encode())
    assert done.stdout == f"prompt: {text}\ntokens ({len(ids)}): [{', '.join(str(i) for i in ids)}]\n"
    assert cli("tokenize", "-m", path).returncode == 2                       # no text
    assert cli("tokenize", "-m", path, "-p", "x", "-n", "3").returncode == 2  # -n is for run
    assert cli("inspect", "-m", path, "-p", "x").returncode == 2
    assert cli("run", "-m", path, "-p", "x", "-t", "1").returncode == 2
    bad = cli("tokenize", "-m", str(tmp_path / "none.gguf"), "-p", "x")
    assert bad.returncode == 1 and bad.stderr.startswith("error: cannot open")
