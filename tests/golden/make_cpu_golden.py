"""Writes tests/golden/cpu_ref.json: outputs of the reference's own CPU kernels.

The reference's CPU operators (src/torchstrap/kernels/csrc/stubs.cpp and
cpu/{adam,sgd,adagrad}.cpp) are compiled from /root/reference by
``make -C oracle ref`` into oracle/_ref/torchstrap_ref_C.so; this script loads
that library in a process of its own (it registers the same ``torchstrap``
namespace as the product, so the two never share a process), runs every case
of tests/golden/cases.py through ``torch.ops.torchstrap.*_step_`` on CPU
tensors -- contiguous (vector body + row tail) and, for a subset, as a strided
(R, T) view (scalar path) -- and records a SHA-256 digest of every output.
tests/golden/cpu_ref_dtypes.json holds the same kind of records for float64,
float16 and bfloat16 buffers (``dtype_records``).

    python tests/golden/make_cpu_golden.py [--out tests/golden/cpu_ref.json]
                                           [--dtypes-out tests/golden/cpu_ref_dtypes.json]
"""

from __future__ import annotations

import argparse
import json
import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(Path(__file__).resolve().parent))

import cases as C  # noqa: E402

REF_LIB = ROOT / "oracle" / "_ref" / "torchstrap_ref_C.so"


DTYPES = {"float64": torch.float64, "float16": torch.float16, "bfloat16": torch.bfloat16}


def as_layout(a: np.ndarray, strided: bool, dtype=torch.float32) -> torch.Tensor:
    t = torch.from_numpy(a.copy()).to(dtype)
    if not strided:
        return t
    R, T = a.shape
    backing = torch.empty(T, R, dtype=dtype).t()
    backing.copy_(t)
    return backing


def run_ref(c, strided=False, dtype=None):
    """Runs a case through ``torch.ops.torchstrap`` on CPU tensors. Without
    ``dtype`` everything is float32 and the outputs come back as numpy arrays;
    with it, the float32 inputs are rounded to ``dtype`` (params, state,
    gradients, steps and the (R,) hyperparameters alike) and the outputs come
    back as contiguous tensors of that dtype."""
    dt = torch.float32 if dtype is None else dtype
    x = C.make_inputs(c)
    names = C.state_names(c, x)
    st = {k: as_layout(x[k], strided, dt) for k in names}
    vec = {k: torch.from_numpy(x[k].copy()).to(dt) for k in x
           if k not in names and k not in ("grads", "mask") and x[k] is not None}
    vec["mask"] = torch.from_numpy(x["mask"].copy())
    steps = vec.pop("steps")
    ops = torch.ops.torchstrap
    for g in x["grads"]:
        gt = as_layout(g, strided, dt)
        if c["op"] == "adam":
            ops.adam_step_(st["p"], gt, st["m"], st["v"], st.get("mx"), steps, vec["lr"],
                           vec["beta1"], vec["beta2"], vec["eps"], vec["wd"], vec["mask"],
                           c["amsgrad"], c["maximize"], c["decoupled"])
        elif c["op"] == "sgd":
            ops.sgd_step_(st["p"], gt, st.get("mb"), steps, vec["lr"], vec["momentum"],
                          vec["dampening"], vec["wd"], vec["mask"], c["nesterov"],
                          c["maximize"])
        else:
            ops.adagrad_step_(st["p"], gt, st["s"], steps, vec["lr"], vec["lr_decay"],
                              vec["wd"], vec["eps"], vec["mask"], c["maximize"])
    out = {k: st[k].contiguous() for k in names}
    out["steps"] = steps
    if dtype is None:
        out = {k: v.numpy() for k, v in out.items()}
    return out


def dtype_records():
    """Every case of ``cases.dtype_cases()`` in float64, float16 and bfloat16,
    contiguous and strided: the reference's float64 rows take its vector body
    (contiguous) or its scalar loop (strided); its 16-bit rows always take the
    scalar loop, accumulating in float (cpu/adam.cpp:262-268)."""
    records = []
    for name, dt in DTYPES.items():
        for c in C.dtype_cases():
            for strided in (False, True):
                out = run_ref(c, strided, dt)
                records.append({"case": c, "dtype": name, "strided": strided,
                                "digest": {k: C.digest_bytes(v) for k, v in out.items()}})
    return records


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--out", default=str(Path(__file__).resolve().parent / "cpu_ref.json"))
    ap.add_argument("--dtypes-out",
                    default=str(Path(__file__).resolve().parent / "cpu_ref_dtypes.json"))
    args = ap.parse_args()
    if not REF_LIB.exists():
        sys.exit(f"{REF_LIB} is missing: run `make -C oracle ref` first")
    torch.ops.load_library(str(REF_LIB))
    producer = ("reference CPU kernels (src/torchstrap/kernels/csrc/cpu/*.cpp) "
                "built by oracle/Makefile `ref` (-O2 -fno-math-errno -mavx2 -mfma "
                "-mf16c -DCPU_CAPABILITY_AVX2)")
    drec = dtype_records()
    Path(args.dtypes_out).write_text(json.dumps(
        {"producer": producer, "torch": torch.__version__, "records": drec}, indent=0))
    print(f"wrote {len(drec)} records to {args.dtypes_out}")
    records = []
    for c in C.all_cases():
        # a third of the cases also strided, chosen by seed so that adding
        # cases leaves the choice for the others unchanged
        for strided in ((False, True) if c["seed"] % 3 == 0 else (False,)):
            out = run_ref(c, strided)
            rec = {"case": c, "strided": strided,
                   "digest": {k: C.digest(v) for k, v in out.items()}}
            if c["T"] == 45 and not strided:
                rec["values"] = {k: v.ravel().tolist() for k, v in out.items()}
            records.append(rec)
    meta = {"producer": producer, "torch": torch.__version__, "records": records}
    Path(args.out).write_text(json.dumps(meta, indent=0))
    print(f"wrote {len(records)} records to {args.out}")


if __name__ == "__main__":
    main()
