"""Benchmark: fused batched optimizer step on one MI355X.

Workload (the north-star configuration): Adam fp32,
N = 128 replicas x T = 25,171,968 params (12 transformer-block tensors per
replica), per-replica lr log-uniform in [1e-5, 1e-3], step uniform in
[1, 10000], active mask Bernoulli(0.9), grads ~ N(0, 1e-3), synthetic seeded
tensors resident in HBM before timing starts. One "step" is one
``torch.ops.torchstrap.adam_step_`` call over the whole (N, T) state.

Printed (one JSON line): value = effective HBM GB/s of the whole step (active
rows x T x 28 B / step time), plus the kernel's roofline (algorithmic bytes of
one update launch / its average duration, measured with HIP events on the
launch stream), the reference CPU kernel timed on this host, the N-instance
torch.optim Python-loop baseline on the same GPU, and the training step's
gradient hand-off (per-parameter scatter then update, vs the fused segmented update).
Configs 1-4 add `mall_residency` (each launch warm vs after a MALL-evicting
read); `--size-sweep N1,N2,...` fits a fixed cost and a streaming rate over
replica counts, and `--geometry ROWS` times config 2's update with ragged and
256-byte rows, with and without frozen replicas.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config 5]
"""

from __future__ import annotations

import argparse
import json
import math
import os
import subprocess
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
HBM_PEAK_GBS = 8000.0  # MI355X HBM3E
FP64_PEAK_TFLOPS = 78.6  # MI355X FP64 vector

# Per-replica tensor layouts of BASELINE.json's configs.
MLP_LAYOUT = [(512, 256), (512,), (256, 512), (256,), (10, 256), (10,)]
CNN_LAYOUT = [(32, 3, 3, 3), (32,), (64, 32, 3, 3), (64,), (128, 4096), (128,),
              (10, 128), (10,)]
BLOCK_LAYOUT = [(4096, 1024)] * 4 + [(1024, 4096)] * 2 + [(1024,)] * 6


def padded_width(layout) -> int:
    raw = sum(math.prod(s) for s in layout)
    return raw + (-raw % 4)


CONFIGS = {
    1: dict(op="adam", N=8, layout=MLP_LAYOUT, amsgrad=False, decoupled=False),
    2: dict(op="adam", N=100, layout=MLP_LAYOUT, amsgrad=True, decoupled=True),
    3: dict(op="sgd", N=32, layout=CNN_LAYOUT),
    4: dict(op="adagrad", N=64, layout=CNN_LAYOUT),
    5: dict(op="adam", N=128, layout=BLOCK_LAYOUT, amsgrad=False, decoupled=False),
}


def bytes_per_elem(cfg: int) -> int:
    c = CONFIGS[cfg]
    if c["op"] == "adam":
        return 36 if c["amsgrad"] else 28
    return 20


def make_config(cfg: int, device="cuda", seed=None, N=None):
    """Synthetic state of one BASELINE.json config, as the op's arguments.

    Returns (op_name, args tuple, kwargs dict, algorithmic bytes of one step).
    """
    import torch

    c = CONFIGS[cfg]
    N = N or c["N"]
    T = padded_width(c["layout"])
    raw = sum(math.prod(s) for s in c["layout"])
    dev = torch.device(device)
    g = torch.Generator(device=dev).manual_seed(1000 + cfg if seed is None else seed)
    f = dict(device=dev, dtype=torch.float32)

    def normal(std, *shape):
        return torch.randn(*shape, generator=g, **f).mul_(std)

    def pad0(t):  # the layout's pad lanes are zero
        if T > raw:
            t[:, raw:] = 0
        return t

    def uniform(lo, hi, n):
        return torch.rand(n, generator=g, **f) * (hi - lo) + lo

    if cfg == 1:
        p, gr = pad0(normal(0.02, N, T)), pad0(normal(1e-2, N, T))
        m, v = torch.zeros(N, T, **f), torch.zeros(N, T, **f)
        steps = torch.full((N,), 1.0, **f)
        mask = torch.ones(N, dtype=torch.bool, device=dev)
        hyp = [torch.full((N,), x, **f) for x in (1e-3, 0.9, 0.999, 1e-8, 0.0)]
        args = (p, gr, m, v, None, steps, *hyp, mask)
        kw = dict(amsgrad=False, maximize=False, decoupled_weight_decay=False)
    elif cfg == 2:
        p, gr = pad0(normal(0.02, N, T)), pad0(normal(1e-2, N, T))
        m = pad0(normal(1e-3, N, T))
        v = pad0(normal(1e-4, N, T).abs_())
        mx = v.clone()
        steps = torch.randint(1, 1001, (N,), generator=g, device=dev).float()
        lr = torch.pow(10.0, uniform(-4, -2, N))
        mask = torch.rand(N, generator=g, device=dev) < 0.75
        hyp = [lr] + [torch.full((N,), x, **f) for x in (0.9, 0.999, 1e-8, 1e-2)]
        args = (p, gr, m, v, mx, steps, *hyp, mask)
        kw = dict(amsgrad=True, maximize=False, decoupled_weight_decay=True)
    elif cfg == 3:
        p, gr = pad0(normal(0.02, N, T)), pad0(normal(1e-2, N, T))
        mb = pad0(normal(1e-2, N, T))
        choices = torch.tensor([0.0, 0.5, 0.9, 0.99], **f)
        mom = choices[torch.randint(0, 4, (N,), generator=g, device=dev)]
        first = torch.rand(N, generator=g, device=dev) < 0.5
        steps = torch.where(first, torch.zeros(N, **f),
                            torch.randint(1, 100, (N,), generator=g, device=dev).float())
        mask = torch.rand(N, generator=g, device=dev) < 0.8
        args = (p, gr, mb, steps, torch.full((N,), 1e-2, **f), mom,
                torch.full((N,), 0.1, **f), torch.zeros(N, **f), mask)
        kw = dict(nesterov=True, maximize=False)
    elif cfg == 4:
        p, gr = pad0(normal(0.02, N, T)), pad0(normal(1e-2, N, T))
        s = normal(1e-3, N, T).abs_().add_(0.1)
        steps = torch.randint(1, 501, (N,), generator=g, device=dev).float()
        mask = torch.ones(N, dtype=torch.bool, device=dev)
        hyp = [torch.full((N,), x, **f) for x in (1e-2, 1e-4, 1e-4, 1e-10)]
        args = (p, gr, s, steps, *hyp, mask)
        kw = dict(maximize=False)
    else:
        p, gr = normal(0.02, N, T), normal(1e-3, N, T)
        m, v = torch.zeros(N, T, **f), torch.zeros(N, T, **f)
        steps = torch.randint(1, 10001, (N,), generator=g, device=dev).float()
        lr = torch.pow(10.0, uniform(-5, -3, N))
        mask = torch.rand(N, generator=g, device=dev) < 0.9
        hyp = [lr] + [torch.full((N,), x, **f) for x in (0.9, 0.999, 1e-8, 0.0)]
        args = (p, gr, m, v, None, steps, *hyp, mask)
        kw = dict(amsgrad=False, maximize=False, decoupled_weight_decay=False)
    active = int(mask.sum().item())
    # Config 3: a replica's first step does not read its momentum buffer, but
    # only the first call has first-step replicas (steps 0, bumped to 1);
    # every later call, the timed ones included, reads every active buffer,
    # so the bytes of a step are the steady state's (first_step_bytes below).
    nbytes = active * T * bytes_per_elem(cfg)
    return c["op"], args, kw, nbytes


def first_step_bytes(cfg: int, device="cuda") -> int | None:
    """Config 3's first call: the steady-state bytes minus the momentum
    buffers its first-step replicas do not read (4 B per element). The same
    seeded draw as the timed state (the device's generator)."""
    if cfg != 3:
        return None
    op_name, args, kw, nbytes = make_config(cfg, device=device)
    mask, steps = args[-1], args[3]
    return nbytes - int((mask & (steps == 0)).sum().item()) * args[0].shape[1] * 4


# ---------------------------------------------------------------------------
# CPU baseline: the reference's CPU kernel (oracle/_ref), in a child process
# ---------------------------------------------------------------------------
CPU_SAMPLE_N = 8
CPU_SHARE = 16


def cpu_worker(cfg: int, steps: int, seconds: float = 10.0) -> None:
    """Child process: time the reference CPU kernel on N = CPU_SAMPLE_N replicas,
    at least `steps` steps and at least `seconds` of CPU work. Waits for a line
    on stdin first (end of input: exit without work), so the parent can start it
    before touching the GPU and let it run after the GPU measurements."""
    if not sys.stdin.readline():
        return
    import torch

    # The GPU box gives one GPU's job a share of 16 host CPUs (its thread and
    # job-size limits are set to 16), whatever the machine has; the baseline
    # uses that whole share, or the affinity set if smaller.
    threads = min(CPU_SHARE, len(os.sched_getaffinity(0)))
    torch.set_num_threads(threads)
    ref = ROOT / "oracle" / "_ref" / "torchstrap_ref_C.so"
    kind = "reference"
    if ref.exists():
        torch.ops.load_library(str(ref))
        op_name, args, kw, nbytes = make_config(cfg, device="cpu", N=CPU_SAMPLE_N)
        fn = getattr(torch.ops.torchstrap, f"{op_name}_step_")
        run = lambda: fn(*args, **kw)  # noqa: E731
    else:  # the C restatement (single-threaded port)
        sys.path.insert(0, str(ROOT))
        from oracle import oracle as O
        kind, threads = "port", 1
        op_name, args, kw, nbytes = make_config(cfg, device="cpu", N=CPU_SAMPLE_N)
        a = [t.numpy() if t is not None else None for t in args]
        step_fn = getattr(O, f"{op_name}_step")
        run = lambda: step_fn(O.CPU, *a, **kw)  # noqa: E731
    run()  # warm
    t0 = time.perf_counter()
    done = 0
    while done < steps or time.perf_counter() - t0 < seconds:
        run()
        done += 1
    steps = done
    dt = (time.perf_counter() - t0) / steps
    print(json.dumps({"value": round(nbytes / dt / 1e9, 3), "unit": "GB/s",
                      "cores": threads, "kind": kind, "us_per_step": round(dt * 1e6, 1),
                      "host": cpu_info(threads),
                      "sample": f"config {cfg} at N={CPU_SAMPLE_N} of {CONFIGS[cfg]['N']} "
                                f"replicas (same T, same per-replica hyperparameters), "
                                f"{steps} steps after 1 warm-up, effective bytes "
                                f"{bytes_per_elem(cfg)} B x active elements"}))


def cpu_baseline_start(cfg: int, steps: int, seconds: float):
    """Starts the CPU-baseline child before this process touches the GPU; it
    idles until cpu_baseline_finish, so no CPU sample runs just before the GPU
    timings. (On one box, three processes that ran the 10 s sample first timed
    the GPU at frac 0.71 against 0.77 for three without it; on another box four
    such pairs showed no difference.)"""
    cmd = [sys.executable, str(Path(__file__).resolve()), "--cpu-worker",
           "--config", str(cfg), "--steps", str(steps), "--cpu-seconds", str(seconds)]
    env = dict(os.environ, HIP_VISIBLE_DEVICES="", CUDA_VISIBLE_DEVICES="")
    return subprocess.Popen(cmd, stdin=subprocess.PIPE, stdout=subprocess.PIPE,
                            stderr=subprocess.PIPE, text=True, env=env)


def cpu_baseline_finish(proc):
    """Lets the child run its timing now and returns its result."""
    try:
        out, err = proc.communicate("go\n", timeout=600)
    except subprocess.TimeoutExpired:
        proc.kill()
        proc.communicate()
        return None
    line = [ln for ln in out.splitlines() if ln.startswith("{")]
    if proc.returncode != 0 or not line:
        sys.stderr.write(err[-2000:])
        return None
    return json.loads(line[-1])


# ---------------------------------------------------------------------------
# GPU measurements
# ---------------------------------------------------------------------------
def abi_update_call(op_name, args, kw, extra_flags: int = 0, dtype_code: int = 0,
                    workspace: bool = True):
    """A no-argument function that enqueues one update through the C ABI on
    torch's current stream, without the step bump, and returns its status.
    Adam and Adagrad go through the workspace entry points, as the operator
    does (their preparation launch then precedes the update); workspace=False
    calls the entry points without one."""
    import ctypes

    import torch

    lib = ctypes.CDLL(str(ROOT / "churten_amd" / "lib" / "libchurten_optim.so"))
    ws = torch.empty(16 * args[0].shape[0], dtype=torch.uint8, device=args[0].device)
    ws_args = (ctypes.c_void_p(ws.data_ptr()), ctypes.c_size_t(ws.numel()))

    class RtBuf(ctypes.Structure):
        _fields_ = [("data", ctypes.c_void_p), ("stride_r", ctypes.c_int64),
                    ("stride_t", ctypes.c_int64)]

    def buf(t):
        return RtBuf(t.data_ptr(), t.stride(0), t.stride(1)) if t is not None else RtBuf(0, 0, 1)

    stream = torch.cuda.current_stream()
    vp = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    p, gr = args[0], args[1]
    R, T = p.shape
    if op_name == "adam":
        bufs = (RtBuf * 5)(*[buf(t) for t in args[:5]])
        flags = ((1 if kw["amsgrad"] else 0) | (2 if kw["decoupled_weight_decay"] else 0)
                 | extra_flags)
        head = (bufs, dtype_code, vp(args[5]), *[vp(t) for t in args[6:11]], vp(args[11]),
                ctypes.c_int64(R), ctypes.c_int64(T), ctypes.c_uint32(flags), ctypes.c_void_p(0))
        if workspace:
            call = lambda: lib.ts_adam_step_ws(  # noqa: E731
                *head, *ws_args, ctypes.c_void_p(stream.cuda_stream))
        else:
            call = lambda: lib.ts_adam_step(*head, ctypes.c_void_p(stream.cuda_stream))  # noqa: E731
    elif op_name == "sgd":
        bufs = (RtBuf * 3)(*[buf(t) for t in args[:3]])
        flags = (8 if kw["nesterov"] else 0) | extra_flags
        call = lambda: lib.ts_sgd_step(  # noqa: E731
            bufs, dtype_code, vp(args[3]), *[vp(t) for t in args[4:8]], vp(args[8]),
            ctypes.c_int64(R), ctypes.c_int64(T), ctypes.c_uint32(flags),
            ctypes.c_void_p(0), ctypes.c_void_p(stream.cuda_stream))
    elif op_name == "adagrad":
        bufs = (RtBuf * 3)(*[buf(t) for t in args[:3]])
        head = (bufs, dtype_code, vp(args[3]), *[vp(t) for t in args[4:8]], vp(args[8]),
                ctypes.c_int64(R), ctypes.c_int64(T), ctypes.c_uint32(extra_flags),
                ctypes.c_void_p(0))
        if workspace:
            call = lambda: lib.ts_adagrad_step_ws(  # noqa: E731
                *head, *ws_args, ctypes.c_void_p(stream.cuda_stream))
        else:
            call = lambda: lib.ts_adagrad_step(*head, ctypes.c_void_p(stream.cuda_stream))  # noqa: E731
    else:
        raise ValueError(op_name)
    def run():
        return call()

    run.keep_alive = (ws, bufs)  # the workspace and the operand table outlive the call
    return run


def kernel_only_timing(op_name, args, kw, launches: int, extra_flags: int = 0,
                       dtype_code: int = 0, workspace: bool = True) -> float:
    """Average duration (ms) of the update: `abi_update_call` bracketed by HIP
    events on the launch stream. With a workspace the preparation launch (the
    per-replica constants, one tiny kernel) is inside the bracket, a few
    microseconds against the update's milliseconds at config 5."""
    import torch

    call = abi_update_call(op_name, args, kw, extra_flags, dtype_code, workspace)
    stream = torch.cuda.current_stream()
    for _ in range(3):
        assert call() == 0
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(launches):
        call()
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / launches


EVICT_BYTES = 1 << 30


def mall_residency_timing(op_name, args, kw, nbytes: int, launches: int):
    """Where an update's operands are served from when its launches run back
    to back: each launch (preparation + update, through the C ABI) timed
    alone between two HIP events, once with the previous launch right before
    it (operands warm in the 256 MB MALL if they fit) and once with a 1 GiB
    read of another buffer between launches, outside the timed interval,
    which evicts them to HBM. Medians over the launches. rocprofv3's
    FETCH_SIZE counts the bytes that leave the L2 whichever of the two serves
    them, so this timing is what tells them apart."""
    import torch

    call = abi_update_call(op_name, args, kw)
    stream = torch.cuda.current_stream()
    evict = torch.ones(EVICT_BYTES // 4, device=args[0].device)
    sink = torch.empty((), device=args[0].device)
    for _ in range(3):
        assert call() == 0
    out = {}
    for mode in ("warm", "evicted"):
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
              for _ in range(launches)]
        for e0, e1 in ev:
            if mode == "evicted":
                torch.amax(evict, dim=0, out=sink)
            else:
                call()  # the previous launch on the same operands
            e0.record(stream)
            call()
            e1.record(stream)
        torch.cuda.synchronize()
        us = sorted(e0.elapsed_time(e1) * 1e3 for e0, e1 in ev)[launches // 2]
        out[f"{mode}_us"] = round(us, 2)
        out[f"{mode}_GBs"] = round(nbytes / (us * 1e-6) / 1e9, 1)
    del evict
    torch.cuda.empty_cache()
    out["evicted_over_warm"] = round(out["evicted_us"] / out["warm_us"], 3)
    out["operand_bytes"] = int(sum(t.numel() * t.element_size() for t in args
                                   if t is not None and t.dim() == 2))
    return out


def geometry_timing(rows: int, launches: int, rounds: int = 3):
    """Config 2's update (AdamW with amsgrad, its hyperparameter draws) at
    `rows` replicas in four geometries, interleaved over `rounds` rounds in
    one process: config 2's T (265,484: rows end off a 256-byte boundary)
    and a T of 265,472 (rows of 4148 x 256 bytes), each with config 2's
    Bernoulli(0.75) mask and with every replica active. GB/s of the active
    rows' algorithmic bytes (36 B per element), best and mean."""
    import torch

    t_cfg = padded_width(CONFIGS[2]["layout"])
    t_aligned = t_cfg - t_cfg % 64
    out = {}
    cases = {}
    for name, T in (("ragged", t_cfg), ("aligned", t_aligned)):
        g = torch.Generator(device="cuda").manual_seed(77)
        f = dict(device="cuda", dtype=torch.float32)
        p = torch.randn(rows, T, generator=g, **f).mul_(0.02)
        gr = torch.randn(rows, T, generator=g, **f).mul_(1e-2)
        m = torch.randn(rows, T, generator=g, **f).mul_(1e-3)
        v = torch.randn(rows, T, generator=g, **f).mul_(1e-4).abs_()
        mx = v.clone()
        steps = torch.randint(1, 1001, (rows,), generator=g, device="cuda").float()
        lr = torch.pow(10.0, torch.rand(rows, generator=g, **f) * 2 - 4)
        hyp = [lr] + [torch.full((rows,), x, **f) for x in (0.9, 0.999, 1e-8, 1e-2)]
        drawn = torch.rand(rows, generator=g, device="cuda") < 0.75
        kw = dict(amsgrad=True, maximize=False, decoupled_weight_decay=True)
        for mname, mask in (("mask_0.75", drawn), ("all_active", torch.ones_like(drawn))):
            args = (p, gr, m, v, mx, steps, *hyp, mask)
            nb = int(mask.sum().item()) * T * 36
            cases[f"{name}_T{T}_{mname}"] = (abi_update_call("adam", args, kw), nb, args)
    res = {k: [] for k in cases}
    stream = torch.cuda.current_stream()
    for rnd in range(rounds):
        for k in (list(cases) if rnd % 2 == 0 else list(cases)[::-1]):
            call, nb, _ = cases[k]
            for _ in range(3):
                assert call() == 0
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            for _ in range(launches):
                call()
            e1.record(stream)
            torch.cuda.synchronize()
            res[k].append(nb / (e0.elapsed_time(e1) / launches * 1e-3) / 1e9)
    for k, rates in res.items():
        out[k] = {"active": int(cases[k][2][-1].sum().item()), "best_GBs": round(max(rates), 1),
                  "mean_GBs": round(sum(rates) / len(rates), 1)}
    del cases
    torch.cuda.empty_cache()
    return out


def size_sweep_timing(cfg: int, ns, launches: int):
    """The config's update on the first n rows of one allocation of max(ns)
    rows (same buffers, same per-replica hyperparameters and mask, so only
    the size changes), kernel-only time per launch, and per launch-size class
    (operands up to 256 MB: small, up to 1 GiB: mid, above: large; each class
    has its own launch shape) a least-squares fit t = t0 + bytes / rate: t0 is
    what a launch costs beyond streaming its bytes (the preparation launch,
    the grid's ramp-up, the drain of its last workgroups), `rate` the
    streaming rate of that shape."""
    import torch

    op_name, full, kw, _ = make_config(cfg, N=max(ns))
    T = full[0].shape[1]
    n_rt = sum(t is not None and t.dim() == 2 for t in full)
    pts = []
    for n in sorted(ns):
        args = tuple(t[:n] if t is not None else None for t in full)
        mask = args[-1]
        active = int(mask.sum().item())
        nbytes = active * T * bytes_per_elem(cfg)
        ms = kernel_only_timing(op_name, args, kw, launches)
        opb = n * T * 4 * n_rt
        pts.append({"N": n, "active": active, "bytes": nbytes, "operand_bytes": opb,
                    "class": "small" if opb <= 256 << 20 else "mid" if opb <= 1 << 30 else "large",
                    "kernel_avg_us": round(ms * 1e3, 2),
                    "GBs": round(nbytes / (ms * 1e-3) / 1e9, 1)})
    del full, args
    torch.cuda.empty_cache()
    fits = {}
    for cls in ("small", "mid", "large"):
        sel = [p for p in pts if p["class"] == cls]
        if len(sel) >= 3:
            fits[cls] = fit_fixed_and_rate([p["bytes"] for p in sel],
                                           [p["kernel_avg_us"] for p in sel])
    return {"points": pts, "fits": fits}


def fit_fixed_and_rate(nbytes, us):
    """Least-squares t = t0 + bytes / rate over (bytes, microseconds) points:
    t0 in microseconds, rate in GB/s, and the largest residual."""
    n = len(nbytes)
    mx, my = sum(nbytes) / n, sum(us) / n
    slope = (sum((x - mx) * (y - my) for x, y in zip(nbytes, us))
             / sum((x - mx) ** 2 for x in nbytes))  # us per byte
    t0 = my - slope * mx
    return {"t0_us": round(t0, 2), "rate_GBs": round(1e-3 / slope, 1),
            "max_residual_us": round(max(abs(y - t0 - slope * x) for x, y in zip(nbytes, us)), 2)}


def loop_baseline(cfg: int, steps: int, fused: bool, hyper):
    """N independent torch.optim optimizers stepped in a Python loop on the
    same GPU (the reference's 'vanilla' baselines: bench_inplace_adam.py:66-96,
    bench_sgd.py:83-102, bench_adagrad.py:96-115), like for like with the
    fused step: the config's optimizer and flags, each replica with its own
    hyperparameters (`hyper`: the op's (N,) vectors on the host), and only the
    active replicas stepped (the fused op skips frozen ones). Returns ms per
    step of the whole loop."""
    import torch

    c = CONFIGS[cfg]
    dev = torch.device("cuda")
    g = torch.Generator(device=dev).manual_seed(7)
    mask = hyper["mask"]
    active = [r for r in range(len(mask)) if bool(mask[r])]
    opts, params = [], []
    for r in active:
        ps = [torch.randn(*s, device=dev, generator=g).mul_(0.02).requires_grad_()
              for s in c["layout"]]
        for t in ps:
            t.grad = torch.randn(t.shape, device=dev, generator=g).mul_(1e-3)
        params.append(ps)
        h = {k: float(v[r]) for k, v in hyper.items() if k != "mask"}
        impl = dict(fused=True) if fused else dict(foreach=True)
        if c["op"] == "adam":
            cls = torch.optim.AdamW if c["decoupled"] else torch.optim.Adam
            opts.append(cls(ps, lr=h["lr"], betas=(h["beta1"], h["beta2"]), eps=h["eps"],
                            weight_decay=h["weight_decay"], amsgrad=c["amsgrad"], **impl))
        elif c["op"] == "sgd":
            # torch.optim.SGD rejects nesterov with dampening != 0: nesterov
            # replicas run with dampening 0, momentum-0 replicas as plain SGD
            nest = h["momentum"] > 0
            opts.append(torch.optim.SGD(ps, lr=h["lr"], momentum=h["momentum"],
                                        dampening=0.0 if nest else h["dampening"],
                                        nesterov=nest, weight_decay=h["weight_decay"],
                                        **impl))
        else:
            opts.append(torch.optim.Adagrad(ps, lr=h["lr"], lr_decay=h["lr_decay"],
                                            weight_decay=h["weight_decay"], eps=h["eps"],
                                            initial_accumulator_value=0.1, **impl))
    for o in opts:
        o.step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        for o in opts:
            o.step()
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / steps
    del opts, params
    torch.cuda.empty_cache()
    return dt * 1e3


HYPER_NAMES = {"adam": ("lr", "beta1", "beta2", "eps", "weight_decay"),
               "sgd": ("lr", "momentum", "dampening", "weight_decay"),
               "adagrad": ("lr", "lr_decay", "weight_decay", "eps")}


def host_hypers(op_name, args):
    """The op's (N,) hyperparameter vectors and mask, on the host."""
    first = 6 if op_name == "adam" else 4
    names = HYPER_NAMES[op_name]
    out = {k: args[first + i].cpu() for i, k in enumerate(names)}
    out["mask"] = args[first + len(names)].cpu()
    return out


def cpu_info(threads: int):
    """The host the CPU baseline ran on: logical CPUs, the affinity set,
    physical cores, the vector ISA torch detects and the one the timed kernel
    is built for."""
    import torch

    phys, model, flags = set(), "", set()
    try:
        cur = {}
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            k, _, v = line.partition(":")
            k, v = k.strip(), v.strip()
            if k == "physical id":
                cur["p"] = v
            elif k == "core id":
                cur["c"] = v
            elif k == "model name" and not model:
                model = v
            elif k == "flags" and not flags:
                flags = set(v.split())
            elif not line.strip() and cur:
                phys.add((cur.get("p"), cur.get("c")))
                cur = {}
        if cur:
            phys.add((cur.get("p"), cur.get("c")))
    except OSError:
        pass
    isa = [f for f in ("avx2", "fma", "f16c", "avx512f", "avx512_bf16", "amx_tile") if f in flags]
    return {"os_cpu_count": os.cpu_count(), "affinity": len(os.sched_getaffinity(0)),
            "physical_cores": len(phys) or None, "threads": threads, "model": model,
            "isa_flags": isa, "torch_cpu_capability": torch.backends.cpu.get_cpu_capability(),
            "kernel_isa": "AVX2/FMA/F16C (the reference's setup.py:49-60 flags)"}


def grad_scatter_timing(cfg: int, steps: int):
    """The training step's gradient hand-off, timed three ways on the same
    state: the reference pattern (one copy per parameter tensor into the
    consolidated gradient buffer, grad_transform.py:29, then the update), the
    fused segmented update that also fills the buffer, and the fused update
    alone. Per-parameter gradients are (N, *shape) tensors, as vmap returns."""
    import torch

    c = CONFIGS[cfg]
    op_name, args, kw, _ = make_config(cfg)
    if op_name != "adam":
        return None
    p, G = args[0], args[1]
    N = p.shape[0]
    g = torch.Generator(device="cuda").manual_seed(11)
    grads, cols, col = [], [], 0
    for s in c["layout"]:
        grads.append(torch.randn(N, *s, device="cuda", generator=g).mul_(1e-3))
        cols.append(col)
        col += math.prod(s)
    views = [G[:, o:o + math.prod(s)].view(N, *s) for o, s in zip(cols, c["layout"])]
    rest = args[2:]
    seg = torch.ops.churten.adam_step_segments_
    upd = torch.ops.torchstrap.adam_step_

    def reference():
        for v, t in zip(views, grads):
            v.copy_(t)
        upd(p, G, *rest, **kw)

    variants = {
        "scatter_then_update_ms": reference,
        "fused_keep_grads_ms": lambda: seg(p, grads, cols, G, *rest, **kw),
        "fused_ms": lambda: seg(p, grads, cols, None, *rest, **kw),
    }
    stream = torch.cuda.current_stream()
    out = {}
    for name, fn in variants.items():
        fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(steps):
            fn()
        e1.record(stream)
        torch.cuda.synchronize()
        out[name] = round(e0.elapsed_time(e1) / steps, 4)
    del args, grads, views, rest, p, G
    torch.cuda.empty_cache()
    out["speedup_keep_grads"] = round(out["scatter_then_update_ms"] / out["fused_keep_grads_ms"], 3)
    out["speedup"] = round(out["scatter_then_update_ms"] / out["fused_ms"], 3)
    return out


TS_STATE_BF16 = 0x20
TS_ADAGRAD_F32 = 0x40


def bf16_state_timing(cfg: int, launches: int):
    """The same update with the optimizer state (moments / buffers / sums) in
    bfloat16 next to float32 params: kernel-only time and effective GB/s over
    the bytes it moves (params and grads 4 B, each state buffer 2 B). Not run
    for config 3, whose first-step replicas skip the buffer read."""
    import torch

    op_name, args, kw, _ = make_config(cfg)
    args = list(args)
    state_idx = {"adam": [2, 3, 4], "sgd": [2], "adagrad": [2]}[op_name]
    for i in state_idx:
        if args[i] is not None:
            args[i] = args[i].to(torch.bfloat16)
    mask = args[-1]
    n_state = sum(args[i] is not None for i in state_idx)
    per_elem = 4 + 4 + 2 * n_state + 4 + 2 * n_state  # read p, g, state; write p, state
    active = int(mask.sum().item())
    T = args[0].shape[1]
    nbytes = active * T * per_elem
    ms = kernel_only_timing(op_name, tuple(args), kw, launches, extra_flags=TS_STATE_BF16)
    del args
    torch.cuda.empty_cache()
    return {"kernel_avg_ms": round(ms, 4), "bytes_per_elem": per_elem,
            "achieved_GBs": round(nbytes / (ms * 1e-3) / 1e9, 1),
            "frac": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "step_equivalent_GBs": round(active * T * bytes_per_elem(cfg) / (ms * 1e-3) / 1e9, 1)}


def bf16_state_shared_timing(adam_args, launches: int, ceiling: bool = True):
    """`bf16_state_timing` for config 5 on the float32 update's own buffers:
    params and grads as they are, the bfloat16 moments (the float32 moments
    narrowed) in the first half of the float32 moments' storage
    (`half_view`). The same pages as the float32 update, so the comparison
    with it is not one between two placements of the buffers in HBM.
    Overwrites the moments."""
    import torch

    p, gr, m, v = adam_args[:4]
    mask = adam_args[11]
    T = p.shape[1]
    narrowed = (m.to(torch.bfloat16), v.to(torch.bfloat16))
    mb, vb = half_view(m, torch.bfloat16), half_view(v, torch.bfloat16)
    mb.copy_(narrowed[0])
    vb.copy_(narrowed[1])
    del narrowed
    args = (p, gr, mb, vb, *adam_args[4:])
    ms = kernel_only_timing("adam", args, {"amsgrad": False, "maximize": False,
                                           "decoupled_weight_decay": False},
                            launches, extra_flags=TS_STATE_BF16)
    per_elem = 20
    nbytes = int(mask.sum().item()) * T * per_elem
    gbs = nbytes / (ms * 1e-3) / 1e9
    out = {"kernel_avg_ms": round(ms, 4), "bytes_per_elem": per_elem,
           "achieved_GBs": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4),
           "step_equivalent_GBs": round(int(mask.sum().item()) * T * bytes_per_elem(5)
                                        / (ms * 1e-3) / 1e9, 1),
           "storage": "first half of the float32 moments' buffers"}
    if ceiling:
        # the same reads and writes without the arithmetic (cb_traffic mode 3),
        # on the same views; c = 0 leaves every value as it is
        shapes = [(1, 0), (1, 10), (1, 12), (1, 14), (1, 16), (2, 0), (2, 8), (2, 10), (2, 12),
                  (2, 14)]
        best, shape, rates = best_traffic(3, (p, gr, mb, vb), mask, 0.0, shapes, per_elem,
                                          launches)
        out["traffic_ceiling"] = {"GBs": best, "shape": shape,
                                  "update_shape_GBs": rates[(1, 16)],
                                  "update_of_ceiling": round(gbs / best, 4)}
    torch.cuda.empty_cache()
    return out


def other_ops_timing(adam_args, launches: int):
    """SGD with momentum and Adagrad on the config-5 buffers (kernel-only time,
    20 B per active element each): the Adam state's moments serve as the
    momentum buffer and as Adagrad's sums. HBM-bound, unlike configs 3 and 4."""
    import torch

    p, gr, m, v = adam_args[:4]
    steps, lr, mask = adam_args[5], adam_args[6], adam_args[11]
    N, T = p.shape
    nbytes = int(mask.sum().item()) * T * 20
    full = lambda x: torch.full((N,), x, dtype=p.dtype, device=p.device)  # noqa: E731
    out = {}
    for name, op, args, kw, kernel in (
            ("sgd", "sgd", (p, gr, m, steps, lr, full(0.9), full(0.0), full(0.0), mask),
             dict(nesterov=False), "stream_kernel<SgdPolicy<float, true, false>>"),
            ("adagrad", "adagrad", (p, gr, v, steps, lr, full(1e-4), full(0.0), full(1e-10), mask),
             {}, "stream_kernel<AdagradPolicy<float>>")):
        ms = kernel_only_timing(op, args, kw, launches)
        gbs = nbytes / (ms * 1e-3) / 1e9
        out[name] = {"kernel": kernel, "kernel_avg_ms": round(ms, 4), "bytes_per_elem": 20,
                     "achieved_GBs": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4)}
    return out


def lds_for_residency(n: int, lds_per_cu: int = 160 * 1024) -> int:
    """Dynamic LDS that fits only n workgroups per CU (the streaming driver's
    residency cap)."""
    x = (lds_per_cu // n) // 256 * 256
    while lds_per_cu // x > n:
        x += 256
    return x


def traffic_rate(mode, bufs, mask, c, packs, cap, per_elem, launches) -> float:
    """GB/s of one cb_traffic pattern (churten_amd/lib/libchurten_bench.so)
    over the active rows of `bufs` (p, g, m, v), `packs` per thread under a
    residency cap of `cap` one-wave workgroups per CU (0: none), timed over
    `launches` back-to-back launches between two HIP events."""
    import ctypes

    import torch

    lib = ctypes.CDLL(str(ROOT / "churten_amd" / "lib" / "libchurten_bench.so"))
    p = bufs[0]
    R, T = p.shape
    active = int(mask.sum().item())
    stream = torch.cuda.current_stream()
    sink = torch.zeros(1, device=p.device)
    vp = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    lds = lds_for_residency(cap) if cap else 0
    call = lambda: lib.cb_traffic(  # noqa: E731
        ctypes.c_int(mode), *[vp(t) for t in bufs], vp(mask), ctypes.c_int64(R),
        ctypes.c_int64(T), ctypes.c_float(c), ctypes.c_uint32(lds), ctypes.c_int(packs),
        vp(sink), ctypes.c_void_p(stream.cuda_stream))
    for _ in range(3):
        assert call() == 0
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(launches):
        call()
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / launches
    return round(active * T * per_elem / (ms * 1e-3) / 1e9, 1)


def best_traffic(mode, bufs, mask, c, shapes, per_elem, launches):
    """The best `traffic_rate` over (packs, cap) shapes: (GB/s, its shape, all rates)."""
    rates = {(k, cap): traffic_rate(mode, bufs, mask, c, k, cap, per_elem, launches)
             for k, cap in shapes}
    (k, cap), r = max(rates.items(), key=lambda kv: kv[1])
    return r, f"{k} pack{'s' if k > 1 else ''}, " + (f"cap {cap}" if cap else "uncapped"), rates


def ceiling_timing(adam_args, launches: int):
    """The Adam step's traffic without its arithmetic on the same config-5
    buffers (churten_amd/lib/libchurten_bench.so), each kind at the best of a
    few launch shapes (one-wave workgroups, 1 or 2 packs per thread, residency
    caps): 4 reads + 3 writes, also at the update kernel's own shape (1 pack,
    12 per CU); the 4 reads alone; the 3 writes alone. `mix_bound` is the rate
    a 16 B read + 12 B write element reaches if reads and writes each ran at
    their own best rate, one after the other. Runs last: the write-only passes
    overwrite the buffers."""
    import torch

    p, gr, m, v = adam_args[:4]
    mask = adam_args[11]
    assert all(t.is_contiguous() and t.shape == p.shape and t.dtype == torch.float32
               for t in (p, gr, m, v))

    def best(mode, c, shapes, per_elem):
        return best_traffic(mode, (p, gr, m, v), mask, c, shapes, per_elem, launches)

    mix, mix_shape, mix_rates = best(
        0, 0.0, [(1, 4), (1, 6), (1, 8), (1, 10), (1, 12), (1, 14), (2, 3), (2, 4), (2, 10)], 28)
    reads, read_shape, _ = best(1, -3.0e38, [(1, 0), (1, 6), (1, 10), (2, 0), (2, 14)], 16)
    writes, write_shape, _ = best(
        2, 0.0, [(1, 4), (1, 6), (1, 8), (1, 10), (1, 12), (2, 4), (2, 8)], 12)
    out = {"mix_4r3w_GBs": mix, "mix_4r3w_shape": mix_shape,
           "mix_4r3w_update_shape_GBs": mix_rates[(1, 12)],
           "read_4_GBs": reads, "read_4_shape": read_shape,
           "write_3_GBs": writes, "write_3_shape": write_shape}
    out["mix_bound_GBs"] = round(28 / (16 / reads + 12 / writes), 1)
    return out


def half_view(t32, dtype):
    """The first half of a contiguous float32 (N, T) buffer's bytes as an
    (N, T) tensor of a 2-byte type: the same physical pages as the start of
    the float32 buffer."""
    return t32.view(-1).view(dtype)[: t32.numel()].view(t32.shape)


def low_precision_timing(adam_args, launches: int):
    """Adam with float16 and with bfloat16 parameters (state in the parameter
    dtype, as torch keeps it) at the config-5 shape and mask: kernel-only time
    and effective GB/s of 14 B per active element. The 16-bit buffers occupy
    the first half of the float32 update's own buffers (`half_view`), so the
    comparison with the float32 update is not one between two placements of
    the buffers in HBM (which alone moves the same kernel by up to +-6%):
    params and grads are the float32 values narrowed, the moments start at
    zero. For float16 eps is 1e-4 (the config's 1e-8 is 0 in half precision,
    which turns lanes with a zero exp_avg_sq into NaN). Overwrites the float32
    buffers."""
    import torch

    p, gr, m, v = adam_args[:4]
    vecs = adam_args[5:11]
    mask = adam_args[11]
    T = p.shape[1]
    nb = int(mask.sum().item()) * T * 14
    dts = (("f16", torch.float16, 2), ("bf16", torch.bfloat16, 3))
    narrowed = {name: (p.to(dt), gr.to(dt)) for name, dt, _ in dts}  # before any overwrite
    out = {}
    for name, dt, code in dts:
        views = [half_view(t, dt) for t in (p, gr, m, v)]
        views[0].copy_(narrowed[name][0])
        views[1].copy_(narrowed[name][1])
        views[2].zero_()
        views[3].zero_()
        hyp = [t.to(dt) for t in vecs]
        if dt == torch.float16:
            hyp[4].fill_(1e-4)  # eps
        args = (*views, None, *hyp, mask)
        ms = kernel_only_timing("adam", args, {"amsgrad": False, "maximize": False,
                                               "decoupled_weight_decay": False},
                                launches, dtype_code=code)
        gbs = nb / (ms * 1e-3) / 1e9
        out[name] = {"kernel_avg_ms": round(ms, 4), "bytes_per_elem": 14,
                     "achieved_GBs": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4),
                     "eps": float(hyp[4][0])}
    del narrowed
    torch.cuda.empty_cache()
    return out


def replica_minor_timing(cfg: int, launches: int):
    """The same update with every (R, T) operand stored replica-minor (a (T, R)
    buffer seen as (R, T): what vmap over a non-leading dimension hands over),
    which the column driver serves: kernel-only time and effective GB/s."""
    import torch

    op_name, args, kw, nbytes = make_config(cfg)
    args = list(args)
    for i in range(len(args)):
        t = args[i]
        if t is not None and t.dim() == 2:
            back = torch.empty(t.shape[1], t.shape[0], dtype=t.dtype, device=t.device)
            back.copy_(t.t())
            args[i] = back.t()
            del t
    ms = kernel_only_timing(op_name, tuple(args), kw, launches)
    del args
    torch.cuda.empty_cache()
    return {"kernel": "column_kernel", "kernel_avg_ms": round(ms, 4),
            "achieved_GBs": round(nbytes / (ms * 1e-3) / 1e9, 1),
            "frac": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}


SNAPSHOT_N = 32


def snapshot_timing(cfg: int):
    """The checkpoint device-to-host path on the config's optimizer state
    (params, grads and the optimizer's (N, T) buffers, as one State) at
    N = SNAPSHOT_N replicas: the initial full copy into the pinned mirror, then
    ``Snapshot.update`` of the active replicas' rows, then the same rows the
    reference's way (device gather, pinned staging, host scatter into a
    pageable mirror)."""
    import torch

    from churten_amd.optimizer import Adam  # noqa: F401  (registers the ops)
    from churten_amd.snapshot import Snapshot
    from churten_amd.state import State

    op_name, args, kw, _ = make_config(cfg, N=SNAPSHOT_N)
    if op_name != "adam":
        return None
    p, g, m, v, mx, steps, lr, b1, b2, eps, wd, mask = args
    N, T = p.shape
    state = State(params=p, buffers=torch.empty(N, 0, device=p.device),
                  param_meta=[("w", torch.Size((N, T)), 0, T)], buffer_meta=[],
                  active_mask=mask, grads=g)
    state.optimizer_state.update(exp_avgs=m, exp_avg_sqs=v, state_steps=steps, lr=lr,
                                 beta1=b1, beta2=b2, eps=eps, weight_decay=wd)
    rt_bytes = 4 * N * T * 4
    t0 = time.perf_counter()
    snap = Snapshot(state)
    t_init = time.perf_counter() - t0
    active = int(mask.sum().item())
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    snap.update(state)
    t_upd = time.perf_counter() - t0
    moved = 4 * active * T * 4
    # the reference's route for the same rows, on the (N, T) leaves
    leaves = [p, g, m, v]
    mirrors = [snap.tensors[k].clone() for k in ("params", "grads")] + [
        snap.tensors["optimizer_state.exp_avgs"].clone(),
        snap.tensors["optimizer_state.exp_avg_sqs"].clone()]  # pageable
    staging = [torch.empty_like(x, pin_memory=True) for x in mirrors]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    idx_cpu = mask.cpu().nonzero().flatten()
    idx = idx_cpu.to(p.device)
    for leaf, stg, mir in zip(leaves, staging, mirrors):
        k = idx.numel()
        stg[:k].copy_(leaf.index_select(0, idx), non_blocking=True)
        torch.cuda.current_stream().synchronize()
        mir[idx_cpu] = stg[:k]
    t_ref = time.perf_counter() - t0
    same = all(torch.equal(mir[idx_cpu], snap.tensors[n][idx_cpu]) for mir, n in zip(
        mirrors, ("params", "grads", "optimizer_state.exp_avgs", "optimizer_state.exp_avg_sqs")))
    del snap, mirrors, staging, state, args, leaves
    torch.cuda.empty_cache()
    return {"sample": f"config {cfg} at N={N}", "state_bytes": rt_bytes,
            "initial_copy_s": round(t_init, 3),
            "initial_GBs": round(rt_bytes / t_init / 1e9, 1),
            "update_bytes": moved, "update_s": round(t_upd, 3),
            "update_GBs": round(moved / t_upd / 1e9, 1),
            "reference_route_s": round(t_ref, 3),
            "reference_route_GBs": round(moved / t_ref / 1e9, 1),
            "mirrors_identical": bool(same)}


def graph_replay_timing(cfg: int, replays: int):
    """One operator call captured in a HIP graph and replayed: the per-step
    time once the host-side launch work is gone (what a captured training step
    sees). Returns microseconds per replay."""
    import torch

    op_name, args, kw, _ = make_config(cfg)
    fn = getattr(torch.ops.torchstrap, f"{op_name}_step_")
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn(*args, **kw)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        fn(*args, **kw)
    graph.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record()
    for _ in range(replays):
        graph.replay()
    e1.record()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) / replays * 1e6
    us = e0.elapsed_time(e1) / replays * 1e3
    del graph, args
    torch.cuda.empty_cache()
    return {"us_per_step": round(us, 2), "wall_us_per_step": round(wall, 2)}


def read_traffic(kernel: str):
    """HBM bytes per launch from the committed rocprofv3 --pmc summary, if any."""
    f = ROOT / "profiles" / f"{kernel}_traffic.json"
    if f.exists():
        try:
            return json.loads(f.read_text()).get("bytes_per_launch")
        except (ValueError, OSError):
            return None
    return None


def calibrate_copy(nbytes: int = 1 << 30, reps: int = 3) -> None:
    """A plain device copy of known size: the per-dispatch FETCH_SIZE and
    WRITE_SIZE it produces under rocprofv3 give the counters' scale."""
    import torch

    src = torch.ones(nbytes // 4, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"calibration": "copy", "bytes_read": nbytes, "bytes_written": nbytes,
                      "dispatches": reps}))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", type=int, default=5, choices=sorted(CONFIGS))
    ap.add_argument("--cpu-steps", type=int, default=5,
                    help="CPU baseline: at least this many steps ...")
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="... and at least this many seconds of CPU work")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-loop-baseline", action="store_true")
    ap.add_argument("--snapshot", action="store_true",
                    help="also time the checkpoint device-to-host path (allocates the "
                         "state's size twice in pinned host memory)")
    ap.add_argument("--no-bf16-state", action="store_true",
                    help="skip the bfloat16-optimizer-state timing")
    ap.add_argument("--no-ceiling", action="store_true",
                    help="skip the traffic-only ceiling passes on the config-5 buffers")
    ap.add_argument("--no-other-ops", action="store_true",
                    help="skip SGD and Adagrad on the config-5 buffers")
    ap.add_argument("--no-low-precision", action="store_true",
                    help="skip Adam with float16 / bfloat16 parameters at the config-5 shape")
    ap.add_argument("--no-replica-minor", action="store_true",
                    help="skip the replica-minor (column driver) timing")
    ap.add_argument("--no-grad-scatter", action="store_true",
                    help="skip the scatter-then-update vs fused segmented timing")
    ap.add_argument("--no-mall", action="store_true",
                    help="skip the warm-vs-evicted MALL timing (configs 1-4)")
    ap.add_argument("--size-sweep", default="",
                    help="comma-separated replica counts: time the config's update at each "
                         "and fit a fixed cost plus a streaming rate (e.g. 50,100,150,200 "
                         "for config 2)")
    ap.add_argument("--geometry", type=int, default=0, metavar="ROWS",
                    help="time config 2's update at ROWS replicas with ragged and 256-byte "
                         "rows, with its mask and all replicas active (e.g. 800)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="run only a plain 1 GiB device copy (reads and writes 2^30 B "
                         "each), to scale rocprofv3 FETCH_SIZE / WRITE_SIZE counters")
    ap.add_argument("--cpu-worker", action="store_true", help=argparse.SUPPRESS)
    args = ap.parse_args()

    if args.cpu_worker:
        cpu_worker(args.config, args.steps, args.cpu_seconds)
        return
    if args.calibrate_copy:
        calibrate_copy()
        return
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one MI355X: the optimizer step is per-replica "
              "independent and this build runs on a single GPU; use --gpus 1.",
              file=sys.stderr)
        sys.exit(2)

    # The CPU-baseline child starts before this process touches the GPU and
    # runs its timing after the GPU measurements.
    cpu_proc = (None if args.no_cpu_baseline
                else cpu_baseline_start(args.config, args.cpu_steps, args.cpu_seconds))

    import torch

    sys.path.insert(0, str(ROOT))
    import churten_amd.kernels  # noqa: F401  (fails loudly if the HIP build is missing)

    op_name, op_args, kw, nbytes = make_config(args.config)
    fn = getattr(torch.ops.torchstrap, f"{op_name}_step_")
    for _ in range(args.warmup):
        fn(*op_args, **kw)
    torch.cuda.synchronize()

    # K steps bracketed by two events on the launch stream (nothing else is
    # enqueued between the steps, as in a training loop).
    stream = torch.cuda.current_stream()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record(stream)
    for _ in range(args.steps):
        fn(*op_args, **kw)
    end.record(stream)
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / args.steps
    step_ms = start.elapsed_time(end) / args.steps
    # Then K more steps with an event between consecutive steps, for the
    # per-step median (recording an event per step costs host time, which
    # shows on microsecond steps, so it stays out of the timed K).
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps + 1)]
    ev[0].record(stream)
    for i in range(args.steps):
        fn(*op_args, **kw)
        ev[i + 1].record(stream)
    torch.cuda.synchronize()
    per_step = sorted(ev[i].elapsed_time(ev[i + 1]) for i in range(args.steps))
    median_ms = per_step[len(per_step) // 2]

    kern_ms = kernel_only_timing(op_name, op_args, kw, max(10, args.steps))
    mall = (mall_residency_timing(op_name, op_args, kw, nbytes, max(10, args.steps))
            if args.config != 5 and not args.no_mall else None)
    # the same update through the entry points without a workspace (every
    # workgroup derives its replica's constants): what the workspace buys
    nows_ms = (kernel_only_timing(op_name, op_args, kw, max(10, args.steps), workspace=False)
               if op_name in ("adam", "adagrad") else None)
    other_ops = (other_ops_timing(op_args, max(10, args.steps // 2))
                 if args.config == 5 and not args.no_other_ops else None)
    # 16-bit variants on the same buffers (they overwrite them), then the
    # traffic ceiling, which overwrites them too
    bf16 = None
    low_prec = None
    if args.config == 5:
        if not args.no_bf16_state:
            bf16 = bf16_state_shared_timing(op_args, max(10, args.steps // 2),
                                            ceiling=not args.no_ceiling)
        if not args.no_low_precision:
            low_prec = low_precision_timing(op_args, max(10, args.steps // 2))
    ceiling = (ceiling_timing(op_args, max(10, args.steps // 2))
               if args.config == 5 and not args.no_ceiling else None)
    if ceiling is not None:
        kern_gbs = nbytes / (kern_ms * 1e-3) / 1e9
        ceiling["update_kernel_of_mix"] = round(kern_gbs / ceiling["mix_4r3w_GBs"], 4)
        ceiling["update_kernel_of_mix_bound"] = round(kern_gbs / ceiling["mix_bound_GBs"], 4)
    achieved = nbytes / (kern_ms * 1e-3) / 1e9
    fp64_roofline = None
    adagrad_f32 = None
    if op_name == "adagrad":
        # second bound: the fp64 update, ~6 FP64 FLOPs per active element (fma = 2, incl. one
        # divide), against the MI355X's 78.6 TFLOP/s FP64 vector peak
        flops = 6 * (nbytes // bytes_per_elem(args.config))
        fp64_roofline = {"bound": "fp64", "achieved": round(flops / (kern_ms * 1e-3) / 1e12, 3),
                         "peak": FP64_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(flops / (kern_ms * 1e-3) / 1e12 / FP64_PEAK_TFLOPS, 4)}
    if op_name == "adagrad":  # the float32 variant on the same state
        f32_ms = kernel_only_timing(op_name, op_args, kw, max(10, args.steps),
                                    extra_flags=TS_ADAGRAD_F32)
        adagrad_f32 = {"kernel_avg_ms": round(f32_ms, 4),
                       "GBs": round(nbytes / (f32_ms * 1e-3) / 1e9, 1)}
    policy = {"adam": "AdamPolicy<float, %s, %s, float>" % (
                  str(kw.get("decoupled_weight_decay")).lower(), str(kw.get("amsgrad")).lower()),
              "sgd": "SgdPolicy<float, %s, %s, float>" % (
                  "true" if op_args[2] is not None else "false", str(kw.get("nesterov")).lower()),
              "adagrad": "AdagradPolicy<float, float>"}[op_name]
    # the instantiation the operator launches: ANY = false (State's layout), PRE (per-replica
    # constants from the workspace: Adam and Adagrad), SMALL (operands that fit the 256 MB MALL)
    n_rt = sum(t is not None and t.dim() == 2 for t in op_args)
    small = op_args[0].numel() * 4 * n_rt <= 256 << 20
    kernel = "stream_kernel<%s, false, %s, %s>" % (policy, str(op_name != "sgd").lower(),
                                                  str(small).lower())
    profile_key = f"{op_name}_stream_kernel_cfg{args.config}"
    hypers = host_hypers(op_name, op_args)
    del op_args
    torch.cuda.empty_cache()

    snapshot = snapshot_timing(args.config) if args.snapshot else None
    graphed = graph_replay_timing(args.config, args.steps) if args.config != 5 else None

    if not args.no_bf16_state and args.config not in (3, 5):
        bf16 = bf16_state_timing(args.config, max(10, args.steps // 2))

    minor = None if args.no_replica_minor else replica_minor_timing(args.config,
                                                                    max(10, args.steps // 2))

    sweep = None
    if args.size_sweep:
        sweep = size_sweep_timing(args.config, [int(x) for x in args.size_sweep.split(",")],
                                  max(10, args.steps))

    geometry = geometry_timing(args.geometry, max(10, args.steps // 5)) if args.geometry else None

    scatter = None
    if not args.no_grad_scatter and op_name == "adam":
        scatter = grad_scatter_timing(args.config, max(5, args.steps // 2))

    loop = {}
    if not args.no_loop_baseline:
        if op_name != "adagrad":  # torch.optim.Adagrad(fused=True) rejects GPU tensors
            loop["fused_ms"] = round(loop_baseline(args.config, 3, True, hypers), 3)
        loop["foreach_ms"] = round(loop_baseline(args.config, 3, False, hypers), 3)

    cpu = None if cpu_proc is None else cpu_baseline_finish(cpu_proc)

    value = nbytes / (step_ms * 1e-3) / 1e9
    c = CONFIGS[args.config]
    out = {
        "metric": "Adam step us + effective HBM GB/s (% of peak) at NxT; speedup vs Python loop",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_ms, 4),
        "us_per_step": round(step_ms * 1e3, 1),
        "median_us_per_step": round(median_ms * 1e3, 1),
        "wall_ms_per_step": round(wall_ms, 4),
        "pct_of_hbm_peak": round(100 * value / HBM_PEAK_GBS, 1),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded torch generators, resident in HBM)",
        "config": {"workload": f"BASELINE.json configs[{args.config - 1}]: {c['op']} fp32, "
                               f"N={c['N']} x T={padded_width(c['layout'])}",
                   "N": c["N"], "T": padded_width(c["layout"]),
                   "active_bytes_per_step": nbytes, "bytes_per_elem": bytes_per_elem(args.config),
                   "first_call_bytes": first_step_bytes(args.config),
                   "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "kernel": kernel, "achieved": round(achieved, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "kernel_avg_ms": round(kern_ms, 4),
                     "traffic": read_traffic(profile_key),
                     "without_workspace": (None if nows_ms is None else {
                         "kernel_avg_ms": round(nows_ms, 4),
                         "achieved": round(nbytes / (nows_ms * 1e-3) / 1e9, 1),
                         "frac": round(nbytes / (nows_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)})},
        "cpu_baseline": cpu,
        "python_loop_baseline": loop or None,
        "grad_scatter_step": scatter,
        "bf16_state": bf16,
        "replica_minor": minor,
        "low_precision_params": low_prec,
        "other_ops_cfg5_shape": other_ops,
        "traffic_ceiling": ceiling,
        "adagrad_f32": adagrad_f32,
        "fp64_roofline": fp64_roofline,
        "snapshot": snapshot,
        "graph_replay": graphed,
        "mall_residency": mall,
        "size_sweep": sweep,
        "geometry": geometry,
        "speedup_vs_python_loop": ({k: round(v / step_ms, 2) for k, v in loop.items()}
                                   if loop else None),
        "python_loop_note": ("torch.optim per replica, own hyperparameters, active replicas "
                             "only" + ("; nesterov replicas with dampening 0 (torch.optim.SGD "
                                       "rejects nesterov with dampening)"
                                       if op_name == "sgd" else "")) if loop else None,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
