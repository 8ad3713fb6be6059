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


def test_kv_dtype_is_refused_where_no_kv_cache_takes_it():
    for name in ("deepseek-v3-mla", "sampler", "sampler-default"):
        r = _run("--workload", name, "--kv-dtype", "fp8_e4m3")
        assert r.returncode != 0 and "does not apply" in r.stderr, name


def test_cpu_baseline_reports_a_median_with_the_cpu_model():
    """The CPU leg alone (no GPU): median of >= 5 timed reps, model and cores stated."""
    sys.path.insert(0, str(ROOT))
    import argparse

    import bench

    args = argparse.Namespace(context=64, batch=64, cpu_seconds=0.2)
    rec = bench.cpu_baseline(args, 32, 8, 128, 16, 128 ** -0.5, 1_000_000)
    assert rec["kind"] == "port" and rec["reps"] >= 5 and rec["cores"] >= 1 and rec["value"] > 0
    assert rec["cpu_model"] and "median" in rec["sample"]
