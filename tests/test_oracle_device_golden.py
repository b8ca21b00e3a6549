"""The oracle's device formulation against torch's ROCm fused kernels.

tests/golden/device_ref.json holds, per case and per replica row, SHA-256
digests of what torch's own fused kernels (the device math the reference's GPU
kernels call verbatim) computed on an MI355X, one row per call
(tests/golden/make_device_golden.py). The C oracle's DEVICE formulation, run on
the CPU, must reproduce every recorded row bit for bit; this is what lets the
oracle check the HIP kernels bit-exactly.
"""

from __future__ import annotations

import json
from pathlib import Path

import pytest

import cases as C
from oracle import oracle as O

GOLDEN = Path(__file__).resolve().parent / "golden" / "device_ref.json"
if not GOLDEN.exists():
    pytest.skip("device_ref.json not generated yet", allow_module_level=True)
META = json.loads(GOLDEN.read_text())
RECORDS = META["records"]


def test_golden_was_made_on_mi355x():
    assert META["arch"].startswith("gfx950"), META["arch"]
    assert {r["case"]["op"] for r in RECORDS} == {"adam", "sgd", "adagrad"}
    assert sum(len(r["rows"]) for r in RECORDS) > 2 * len(RECORDS)


@pytest.mark.parametrize("rec", RECORDS, ids=lambda r: C.case_id(r["case"]))
def test_device_oracle_bit_exact_to_rocm_torch(rec):
    c = rec["case"]
    out = C.run_oracle(c, O.DEVICE)
    for r, digests in rec["rows"].items():
        r = int(r)
        for name, want in digests.items():
            row = out[name][r : r + 1] if name == "steps" else out[name][r]
            assert C.digest(row) == want, f"row {r} {name} differs from torch's ROCm kernel"
