"""The oracle's CPU formulation against torch's own CPU fused optimizers.

The reference's CPU kernels are written to be bit-identical to torch's CPU
``_fused_adam_`` / ``_fused_adamw_`` / ``_fused_sgd_`` / ``_fused_adagrad_``
at the reference build's vector width (AVX2; test/optimizer/
test_aten_fused_parity.py, *_sgd_*, *_adagrad_*). This pins the oracle's CPU
form a second way, independent of the compiled reference: each replica row of
every case, stepped by the oracle, equals torch's fused kernel on that row
under ``ATEN_CPU_CAPABILITY=avx2`` (set in a child process, before torch
loads), with float32-rounded hyperparameters as the reference's test does.
(SGD rows with momentum 0 inside a call that has buffers are skipped: ATen's
fused SGD takes no buffers when momentum is 0.)
"""

from __future__ import annotations

import json
import os
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]

CHILD = r"""
import json, sys
import numpy as np
import torch
sys.path[:0] = [sys.argv[1], sys.argv[1] + "/tests/golden"]
import cases as C
from oracle import oracle as O

assert torch.backends.cpu.get_cpu_capability() == "AVX2", torch.backends.cpu.get_cpu_capability()
out = {}
for c in C.all_cases():
    if c["T"] not in (45, 64, 1000) or c["nsteps"] < 1:
        continue
    x = C.make_inputs(c)
    R = c["R"]
    want = C.run_oracle(c, O.CPU)
    bad = 0
    compared = 0
    for r in range(R):
        if not x["mask"][r]:
            continue
        t = lambda k: torch.from_numpy(x[k][r].copy())
        step = torch.tensor(float(x["steps"][r]))
        if c["op"] == "adam":
            p, m, v = t("p"), t("m"), t("v")
            mx = [t("mx")] if c["amsgrad"] else []
            fn = torch._fused_adamw_ if c["decoupled"] else torch._fused_adam_
            for g in x["grads"]:
                step += 1
                fn([p], [torch.from_numpy(g[r].copy())], [m], [v], mx, [step],
                   lr=float(x["lr"][r]), beta1=float(x["beta1"][r]), beta2=float(x["beta2"][r]),
                   weight_decay=float(x["wd"][r]), eps=float(x["eps"][r]),
                   amsgrad=c["amsgrad"], maximize=c["maximize"], grad_scale=None, found_inf=None)
            got = {"p": p, "m": m, "v": v}
            if c["amsgrad"]:
                got["mx"] = mx[0]
        elif c["op"] == "sgd":
            if x["mb"] is not None and x["momentum"][r] == 0.0:
                continue  # momentum 0 with a buffer: ATen has no such call
            p = t("p")
            mb = [t("mb")] if x["mb"] is not None else []
            first = float(x["steps"][r]) == 0.0
            for i, g in enumerate(x["grads"]):
                torch._fused_sgd_([p], [torch.from_numpy(g[r].copy())], mb,
                                  weight_decay=float(x["wd"][r]),
                                  momentum=float(x["momentum"][r]), lr=float(x["lr"][r]),
                                  dampening=float(x["dampening"][r]), nesterov=c["nesterov"],
                                  maximize=c["maximize"], is_first_step=first and i == 0,
                                  grad_scale=None, found_inf=None)
            got = {"p": p}
            if mb:
                got["mb"] = mb[0]
        else:
            p, s = t("p"), t("s")
            for g in x["grads"]:
                step += 1
                torch._fused_adagrad_([p], [torch.from_numpy(g[r].copy())], [s], [step],
                                      lr=float(x["lr"][r]), lr_decay=float(x["lr_decay"][r]),
                                      weight_decay=float(x["wd"][r]), eps=float(x["eps"][r]),
                                      maximize=c["maximize"], grad_scale=None, found_inf=None)
            got = {"p": p, "s": s}
        for k, tt in got.items():
            bad += int((tt.numpy().view(np.uint32) != want[k][r].view(np.uint32)).sum())
            compared += tt.numel()
    out[C.case_id(c)] = [bad, compared]
print(json.dumps(out))
"""


@pytest.fixture(scope="module")
def mismatches():
    env = dict(os.environ, ATEN_CPU_CAPABILITY="avx2", HIP_VISIBLE_DEVICES="",
               CUDA_VISIBLE_DEVICES="", OMP_NUM_THREADS="1")
    proc = subprocess.run([sys.executable, "-c", CHILD, str(ROOT)], capture_output=True,
                          text=True, env=env, timeout=900)
    assert proc.returncode == 0, proc.stderr[-3000:]
    return json.loads(proc.stdout.strip().splitlines()[-1])


@pytest.mark.parametrize("op", ["adam", "sgd", "adagrad"])
def test_oracle_cpu_form_equals_torch_cpu_fused_avx2(mismatches, op):
    cases = {k: v for k, v in mismatches.items() if k.startswith(op + "-")}
    assert cases and sum(n for _, n in cases.values()) > 10_000, f"too few {op} elements"
    bad = {k: b for k, (b, _) in cases.items() if b}
    assert not bad, f"{len(bad)}/{len(cases)} {op} cases differ: {dict(list(bad.items())[:5])}"
