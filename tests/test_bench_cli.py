"""bench.py on the CPU: the script compiles, refuses more than one GPU with a
JSON error line, and its time-floored warm-up runs at least the requested
steps (no GPU is touched on these paths)."""

from __future__ import annotations

import json
import os
import py_compile
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BENCH = os.path.join(ROOT, "bench.py")


def test_bench_compiles(tmp_path):
    py_compile.compile(BENCH, cfile=str(tmp_path / "bench.pyc"), doraise=True)


@pytest.mark.parametrize("argv,env", [(["--gpus", "2"], {}), ([], {"WORLD_SIZE": "2"})])
def test_more_than_one_gpu_is_refused(argv, env):
    res = subprocess.run([sys.executable, BENCH, *argv], cwd=ROOT, env={**os.environ, **env},
                         capture_output=True, text=True, timeout=120)
    assert res.returncode == 2
    line = json.loads(res.stdout.strip().splitlines()[-1])
    assert "one GPU" in line["error"]


def test_warm_up_runs_at_least_the_requested_steps(monkeypatch):
    sys.path.insert(0, ROOT)
    try:
        import bench
    finally:
        sys.path.remove(ROOT)
    import torch

    monkeypatch.setattr(torch.cuda, "synchronize", lambda *a, **k: None)
    monkeypatch.setattr(bench, "WARMUP_SECONDS", 0.0)
    seen = []
    assert bench.warm_up(seen.append, 5) == 5
    assert seen == [0, 1, 2, 3, 4]
    monkeypatch.setattr(bench, "WARMUP_SECONDS", 0.05)
    seen.clear()
    n = bench.warm_up(seen.append, 1)
    assert n == len(seen) >= 1 and seen == list(range(n))
