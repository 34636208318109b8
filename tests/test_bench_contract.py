"""The bench's command-line contract and the profile summaries it cites (CPU only)."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode != 0
    assert "one GPU" in r.stderr


def test_bench_lists_every_workload():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--help"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 0
    for workload in ("decode", "matvec", "moe", "prefill", "model-prefill"):
        assert workload in r.stdout


def test_profile_summaries_state_their_commands():
    d = os.path.join(ROOT, "profiles")
    names = sorted(n for n in os.listdir(d) if n.endswith(".txt"))
    assert names
    for n in names:
        text = open(os.path.join(d, n)).read()
        assert "rocprofv3" in text and "Command" in text, n
        assert len(text) < 20000, n  # summaries, not raw traces
