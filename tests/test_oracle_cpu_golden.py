"""The oracle's CPU formulation against the reference's own CPU kernels.

tests/golden/cpu_ref.json holds SHA-256 digests of what the reference's CPU
operators (src/torchstrap/kernels/csrc/cpu/*.cpp, compiled from the reference
sources by oracle/Makefile) wrote for every case of tests/golden/cases.py,
contiguous (AVX2 body + row tail) and strided (scalar path). The C oracle must
reproduce every one bit for bit; for the T=45 cases the golden file also holds
the values, so a failure shows where the bits part.
"""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest

import cases as C
from helpers import mismatch
from oracle import oracle as O

GOLDEN = Path(__file__).resolve().parent / "golden" / "cpu_ref.json"
RECORDS = json.loads(GOLDEN.read_text())["records"]


def _id(rec):
    return C.case_id(rec["case"]) + ("-strided" if rec["strided"] else "")


def test_golden_file_covers_every_case():
    ops = {r["case"]["op"] for r in RECORDS}
    assert ops == {"adam", "sgd", "adagrad"}
    assert any(r["strided"] for r in RECORDS) and any(not r["strided"] for r in RECORDS)
    assert len(RECORDS) >= len(C.all_cases())


@pytest.mark.parametrize("rec", RECORDS, ids=_id)
def test_cpu_oracle_bit_exact_to_reference(rec):
    c = rec["case"]
    out = C.run_oracle(c, O.CPU, unit_stride=not rec["strided"])
    for name, want in rec["digest"].items():
        got = C.digest(out[name])
        if got != want:
            detail = ""
            if "values" in rec:
                ref = np.array(rec["values"][name], dtype=np.float32).reshape(out[name].shape)
                detail = mismatch(out[name], ref)
            pytest.fail(f"{name}: oracle differs from the reference CPU kernel {detail}")
