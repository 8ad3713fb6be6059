"""The bench's command-line contract, checked without a GPU: it measures one
GPU only and refuses more, and it offers every measured workload."""

import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def _run(*args):
    return subprocess.run([sys.executable, str(ROOT / "bench.py"), *args], cwd=ROOT, capture_output=True, text=True,
                          timeout=120)


def test_more_than_one_gpu_is_refused():
    r = _run("--gpus", "2")
    assert r.returncode != 0
    assert "one GPU" in (r.stdout + r.stderr)


def test_workloads_and_options_are_listed():
    r = _run("--help")
    assert r.returncode == 0
    for name in ("qwen3-4b", "qwen3-4b-var", "qwen2.5-0.5b", "qwen2.5-7b-groups", "deepseek-v3-mla",
                 "qwen3-4b-prefill", "sampler", "sampler-default", "--kv-dtype"):
        assert name in r.stdout, name
