"""Writes device_ref.json: what torch's own ROCm fused kernels compute on the GPU.

The reference's GPU kernels call ATen's device optimizer math verbatim
(src/torchstrap/kernels/csrc/cuda/adam.cu:146-157, cuda/adagrad.cu:141-148)
or transcribe it (cuda/sgd.cu:90-132), one replica row at a time. This script
runs every case of tests/golden/cases.py through exactly that math --
``torch._fused_adam_`` / ``_fused_adamw_`` / ``_fused_sgd_`` /
``_fused_adagrad_`` on the GPU, one replica row per call, with each row's
float32 hyperparameters, the step counter bumped before the call, and
``is_first_step`` derived per row from it -- and records a SHA-256 digest of
every output row. Rows the ATen call cannot express (a momentum-0 replica
inside a call that carries momentum buffers) are not recorded. Frozen rows are
recorded as their inputs.

Run on an MI355X:  python tests/golden/make_device_golden.py --out <path>/device_ref.json
(then copy the file to tests/golden/).
"""

from __future__ import annotations

import argparse
import json
import sys
from pathlib import Path

import numpy as np
import torch

sys.path.insert(0, str(Path(__file__).resolve().parent))

import cases as C  # noqa: E402


def run_rows(c, dev):
    x = C.make_inputs(c)
    names = C.state_names(c, x)
    R = c["R"]
    rows = {}
    for r in range(R):
        st = {k: torch.from_numpy(x[k][r].copy()).to(dev) for k in names}
        step = torch.tensor(float(x["steps"][r]), device=dev)
        expressible = True
        active = bool(x["mask"][r])
        for g_all in x["grads"]:
            if not active:
                break
            g = torch.from_numpy(g_all[r].copy()).to(dev)
            step += 1
            if c["op"] == "adam":
                fused = torch._fused_adamw_ if c["decoupled"] else torch._fused_adam_
                fused([st["p"]], [g], [st["m"]], [st["v"]],
                      [st["mx"]] if c["amsgrad"] else [], [step],
                      lr=float(x["lr"][r]), beta1=float(x["beta1"][r]),
                      beta2=float(x["beta2"][r]), weight_decay=float(x["wd"][r]),
                      eps=float(x["eps"][r]), amsgrad=c["amsgrad"],
                      maximize=c["maximize"], grad_scale=None, found_inf=None)
            elif c["op"] == "sgd":
                mom = float(x["momentum"][r])
                has_buf = "mb" in st
                if has_buf and mom == 0.0:
                    expressible = False
                    break
                torch._fused_sgd_([st["p"]], [g], [st["mb"]] if has_buf else [],
                                  weight_decay=float(x["wd"][r]), momentum=mom,
                                  lr=float(x["lr"][r]),
                                  dampening=float(x["dampening"][r]),
                                  nesterov=c["nesterov"], maximize=c["maximize"],
                                  is_first_step=bool(step.item() == 1.0),
                                  grad_scale=None, found_inf=None)
            else:
                torch._fused_adagrad_([st["p"]], [g], [st["s"]], [step],
                                      lr=float(x["lr"][r]),
                                      lr_decay=float(x["lr_decay"][r]),
                                      weight_decay=float(x["wd"][r]),
                                      eps=float(x["eps"][r]), maximize=c["maximize"],
                                      grad_scale=None, found_inf=None)
        if not expressible:
            continue
        torch.cuda.synchronize()
        out = {k: st[k].cpu().numpy() for k in names}
        out["steps"] = np.array([step.item()], dtype=np.float32)
        rows[r] = {k: C.digest(v) for k, v in out.items()}
    return rows


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--out", default="device_ref.json")
    args = ap.parse_args()
    dev = torch.device("cuda")
    records = []
    for c in C.all_cases():
        records.append({"case": c, "rows": {str(r): d for r, d in run_rows(c, dev).items()}})
    meta = {
        "producer": "torch ROCm fused optimizer kernels, one replica row per call",
        "torch": torch.__version__,
        "hip": torch.version.hip,
        "device": torch.cuda.get_device_name(0),
        "arch": torch.cuda.get_device_properties(0).gcnArchName,
        "records": records,
    }
    Path(args.out).parent.mkdir(parents=True, exist_ok=True)
    Path(args.out).write_text(json.dumps(meta, indent=0))
    print(f"wrote {len(records)} records to {args.out}", flush=True)


if __name__ == "__main__":
    main()
