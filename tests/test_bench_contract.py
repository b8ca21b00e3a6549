"""bench.py's host-side contract, on the CPU: more than one GPU is refused with
a message, and the algorithmic bytes per active element are the ones the
metric is defined on (Adam 28, AdamW + amsgrad 36, SGD with momentum 20 minus
the skipped buffer read on a replica's first step, Adagrad 20; frozen rows move
nothing)."""

from __future__ import annotations

import subprocess
import sys
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))

import bench  # noqa: E402


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode != 0
    assert "single GPU" in (r.stdout + r.stderr)


@pytest.mark.parametrize("cfg,per_elem", [(1, 28), (2, 36), (3, 20), (4, 20), (5, 28)])
def test_algorithmic_bytes(cfg, per_elem):
    assert bench.bytes_per_elem(cfg) == per_elem
    op, args, kw, nbytes = bench.make_config(cfg, device="cpu", N=4)
    p, mask = args[0], args[-1]
    assert p.shape == (4, bench.padded_width(bench.CONFIGS[cfg]["layout"]))
    active = int(mask.sum())
    T = p.shape[1]
    want = active * T * per_elem
    if cfg == 3:
        steps = args[3]
        want -= int((mask & (steps == 0)).sum()) * T * 4
    assert nbytes == want
    assert op == bench.CONFIGS[cfg]["op"]
    assert all(t.device == torch.device("cpu") for t in args if isinstance(t, torch.Tensor))
