"""The product's CPU dispatch key against the reference's CPU kernels.

Every record of tests/golden/cpu_ref.json -- written by the reference's own CPU
operators compiled from /root/reference -- is replayed through
``torch.ops.torchstrap.*_step_`` on CPU tensors, contiguous and strided; the
outputs must match the recorded digests bit for bit.
"""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest
import torch

import cases as C
import churten_amd.kernels  # noqa: F401
from helpers import mismatch
from make_cpu_golden import run_ref

GOLDEN = Path(__file__).resolve().parent / "golden" / "cpu_ref.json"
RECORDS = json.loads(GOLDEN.read_text())["records"]


@pytest.mark.parametrize("rec", RECORDS,
                         ids=lambda r: C.case_id(r["case"]) + ("-strided" if r["strided"] else ""))
def test_cpu_key_bit_exact_to_reference_cpu_kernel(rec):
    out = run_ref(rec["case"], strided=rec["strided"])
    for name, want in rec["digest"].items():
        if C.digest(out[name]) != want:
            detail = ""
            if "values" in rec:
                ref = np.array(rec["values"][name], dtype=np.float32).reshape(out[name].shape)
                detail = mismatch(out[name], ref)
            pytest.fail(f"{name} differs from the reference CPU kernel {detail}")


def test_cpu_key_is_registered_and_gpu_key_is_separate():
    for op in ("adam_step_", "sgd_step_", "adagrad_step_"):
        name = f"torchstrap::{op}"
        assert torch._C._dispatch_has_kernel_for_dispatch_key(name, "CPU")
        assert torch._C._dispatch_has_kernel_for_dispatch_key(name, "CUDA")


DTYPE_RECORDS = json.loads((GOLDEN.parent / "cpu_ref_dtypes.json").read_text())["records"]


@pytest.mark.parametrize(
    "rec", DTYPE_RECORDS,
    ids=lambda r: r["dtype"] + "-" + C.case_id(r["case"]) + ("-strided" if r["strided"] else ""))
def test_cpu_key_other_dtypes_bit_exact_to_reference_cpu_kernel(rec):
    """float64 (the reference's vector body when contiguous, its scalar loop when
    strided), float16 and bfloat16 (its float-accumulating scalar loop): every
    output, steps included, equals the reference CPU build's bit for bit."""
    dt = {"float64": torch.float64, "float16": torch.float16,
          "bfloat16": torch.bfloat16}[rec["dtype"]]
    out = run_ref(rec["case"], strided=rec["strided"], dtype=dt)
    bad = [k for k, want in rec["digest"].items() if C.digest_bytes(out[k]) != want]
    assert not bad, f"{bad} differ from the reference CPU kernel in {rec['dtype']}"


def test_dtype_records_cover_the_matrix():
    """The dtype fixtures hold every optimizer's flag matrix, the frozen row,
    a momentum-0 replica inside a buffered SGD call, and both layouts."""
    seen = {(r["dtype"], r["case"]["op"], r["strided"]) for r in DTYPE_RECORDS}
    assert len(seen) == 3 * 3 * 2
    sgd = [r["case"] for r in DTYPE_RECORDS if r["case"]["op"] == "sgd"]
    assert any(c["momentum"] == "mixed" and c["nesterov"] and c["dampening"] == 0.1
               for c in sgd)
    assert {c["T"] for c in (r["case"] for r in DTYPE_RECORDS)} >= {45, 1000, 16397}
    assert all(r["case"]["mask"] == "one_frozen" for r in DTYPE_RECORDS)


@pytest.mark.parametrize("dtype", [torch.float64, torch.float16, torch.bfloat16])
def test_cpu_other_dtypes_close_to_fp32(dtype):
    R, T = 3, 37
    g = torch.Generator().manual_seed(0)
    base = [torch.randn(R, T, generator=g) for _ in range(5)]
    tol = {torch.float64: 1e-6, torch.float16: 2e-3, torch.bfloat16: 2e-2}[dtype]
    outs = []
    for dt in (torch.float32, dtype):
        p, gr, m, v, mx = (t.to(dt).clone() for t in base)
        m, v, mx = m.abs(), v.abs(), mx.abs()
        steps = torch.zeros(R, dtype=dt)
        full = lambda x: torch.full((R,), x, dtype=dt)  # noqa: E731
        torch.ops.torchstrap.adam_step_(p, gr, m, v, mx, steps, full(0.125), full(0.875),
                                        full(0.9921875), full(2.0**-14), full(2.0**-6),
                                        torch.ones(R, dtype=torch.bool), amsgrad=True,
                                        maximize=False, decoupled_weight_decay=True)
        outs.append([t.float() for t in (p, m, v, mx)])
    for a, b in zip(*outs):
        torch.testing.assert_close(b, a, atol=tol, rtol=tol)


def test_cpu_errors():
    R, T = 2, 4
    z = torch.zeros(R, T)
    v = torch.zeros(R)
    m = torch.ones(R, dtype=torch.bool)
    with pytest.raises(RuntimeError, match="2-D"):
        torch.ops.torchstrap.adam_step_(z[0], z[0], z[0], z[0], None, v, v, v, v, v, v, m,
                                        amsgrad=False, maximize=False, decoupled_weight_decay=True)
    with pytest.raises(RuntimeError, match="amsgrad=True requires max_exp_avg_sqs"):
        torch.ops.torchstrap.adam_step_(z, z, z, z, None, v, v, v, v, v, v, m,
                                        amsgrad=True, maximize=False, decoupled_weight_decay=True)
    with pytest.raises(RuntimeError, match="nesterov=True requires momentum_buffers"):
        torch.ops.torchstrap.sgd_step_(z, z, None, v, v, v, v, v, m, nesterov=True,
                                       maximize=False)
    with pytest.raises(RuntimeError, match="R = 2"):
        torch.ops.torchstrap.adagrad_step_(z, z, z, v, torch.zeros(3), v, v, v, m,
                                           maximize=False)
