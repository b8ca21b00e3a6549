"""bench.py's host-side contract, on the CPU: more than one GPU is refused with
a message, and the algorithmic bytes per active element are the ones the
metric is defined on (Adam 28, AdamW + amsgrad 36, SGD with momentum 20,
Adagrad 20; frozen rows move nothing). Config 3's first call alone skips the
momentum-buffer read of its first-step replicas; every timed step is past it."""

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
    assert nbytes == active * T * per_elem
    assert op == bench.CONFIGS[cfg]["op"]
    assert all(t.device == torch.device("cpu") for t in args if isinstance(t, torch.Tensor))


def test_config3_first_call_bytes():
    """The first call's bytes drop by 4 B per element of every active replica
    on its first step (steps 0, bumped to 1); the draw has such replicas."""
    op, args, kw, nbytes = bench.make_config(3, device="cpu")
    mask, steps, T = args[-1], args[3], args[0].shape[1]
    first = int((mask & (steps == 0)).sum())
    assert first > 0
    assert bench.first_step_bytes(3, device="cpu") == nbytes - first * T * 4
    assert bench.first_step_bytes(1, device="cpu") is None


def test_fit_fixed_and_rate_recovers_a_line():
    xs = [1e8, 3e8, 7e8, 1.5e9]
    us = [4.0 + x / 6.5e6 for x in xs]  # 4 us fixed, 6.5 TB/s (6.5e6 bytes per us)
    fit = bench.fit_fixed_and_rate(xs, us)
    assert fit["t0_us"] == pytest.approx(4.0, abs=0.01)
    assert fit["rate_GBs"] == pytest.approx(6500.0, rel=1e-4)
    assert fit["max_residual_us"] == pytest.approx(0.0, abs=0.01)
