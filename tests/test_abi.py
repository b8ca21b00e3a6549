"""The drop-in boundary, checked without a GPU.

* The C ABI library loads and exports every entry point include/churten_optim.h
  declares; argument validation returns hipErrorInvalidValue before any device
  call.
* The operator library registers the three ``torchstrap`` schemas with the
  reference's exact text (src/torchstrap/kernels/csrc/stubs.cpp:25-72), the
  fake kernels and the vmap rules (checked on meta tensors).
* The product never reaches the test oracle.
"""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest
import torch
from torch.func import vmap

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "churten_optim.h"
LIB = ROOT / "churten_amd" / "lib" / "libchurten_optim.so"

REFERENCE_SCHEMAS = {
    "adam_step_": "torchstrap::adam_step_(Tensor(a!) params, Tensor grads, Tensor(b!) exp_avgs, "
                  "Tensor(c!) exp_avg_sqs, Tensor(d!)? max_exp_avg_sqs, Tensor(e!) state_steps, "
                  "Tensor lr, Tensor beta1, Tensor beta2, Tensor eps, Tensor weight_decay, "
                  "Tensor active_mask, bool amsgrad, bool maximize, "
                  "bool decoupled_weight_decay) -> Tensor",
    "sgd_step_": "torchstrap::sgd_step_(Tensor(a!) params, Tensor grads, Tensor(b!)? "
                 "momentum_buffers, Tensor(c!) state_steps, Tensor lr, Tensor momentum, "
                 "Tensor dampening, Tensor weight_decay, Tensor active_mask, bool nesterov, "
                 "bool maximize) -> Tensor",
    "adagrad_step_": "torchstrap::adagrad_step_(Tensor(a!) params, Tensor grads, Tensor(b!) "
                     "state_sums, Tensor(c!) state_steps, Tensor lr, Tensor lr_decay, "
                     "Tensor weight_decay, Tensor eps, Tensor active_mask, "
                     "bool maximize) -> Tensor",
}


def declared_symbols():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:int|size_t)\s+(ts_\w+)\s*\(", text, flags=re.M)))


def test_header_declares_the_entry_points():
    assert declared_symbols() == sorted(
        ["ts_adagrad_step", "ts_adam_step", "ts_bump_steps", "ts_sgd_step", "ts_version",
         "ts_adam_step_segments", "ts_sgd_step_segments", "ts_adagrad_step_segments",
         "ts_scatter_segments", "ts_copy_rows", "ts_workspace_bytes", "ts_adam_step_ws",
         "ts_adagrad_step_ws", "ts_adam_step_segments_ws", "ts_adagrad_step_segments_ws",
         "ts_adam_step_noalloc"])


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(str(LIB))
    for name in declared_symbols():
        assert hasattr(lib, name), name
    assert lib.ts_version() == 200


def test_invalid_arguments_rejected_before_any_launch():
    lib = ctypes.CDLL(str(LIB))
    null = ctypes.c_void_p(0)
    i64 = ctypes.c_int64
    # no operand table
    assert lib.ts_adam_step(null, 0, null, null, null, null, null, null, null, i64(1),
                            i64(4), ctypes.c_uint32(0), null, null) == 1
    assert lib.ts_sgd_step(null, 0, null, null, null, null, null, null, i64(1), i64(4),
                           ctypes.c_uint32(0), null, null) == 1
    assert lib.ts_adagrad_step(null, 0, null, null, null, null, null, null, i64(1), i64(4),
                               ctypes.c_uint32(0), null, null) == 1
    # unknown dtype, negative R
    assert lib.ts_bump_steps(7, null, null, i64(0), null, null) == 1
    assert lib.ts_bump_steps(0, null, null, i64(-1), null, null) == 1


def test_workspace_size_and_bad_workspaces_rejected_before_any_launch():
    """A workspace holds two doubles per replica; a missing, short or
    misaligned one is an invalid argument before anything is enqueued (the
    fake device pointers would fault otherwise)."""
    lib = ctypes.CDLL(str(LIB))
    lib.ts_workspace_bytes.restype = ctypes.c_size_t
    assert lib.ts_workspace_bytes(ctypes.c_int64(0)) == 0
    assert lib.ts_workspace_bytes(ctypes.c_int64(-3)) == 0
    assert lib.ts_workspace_bytes(ctypes.c_int64(5)) == 80
    assert lib.ts_workspace_bytes(ctypes.c_int64(65535)) == 65535 * 16
    fake = ctypes.c_void_p(0x10000)
    bufs = (RTBuf * 5)(*[RTBuf(0x10000 * (i + 1), 16, 1) for i in range(5)])
    seg = (Segment * 1)(Segment(0x90000, 16, 0, 16))
    R, T = ctypes.c_int64(4), ctypes.c_int64(16)
    flags = ctypes.c_uint32(0x10)
    sz = ctypes.c_size_t
    for ws, nbytes in ((None, 64), (0x80000, 63), (0x80004, 64)):
        ws = ctypes.c_void_p(ws)
        assert lib.ts_adam_step_ws(bufs, 0, fake, fake, fake, fake, fake, fake, fake, R, T,
                                   flags, None, ws, sz(nbytes), None) == 1
        assert lib.ts_adagrad_step_ws(bufs, 0, fake, fake, fake, fake, fake, fake, R, T,
                                      flags, None, ws, sz(nbytes), None) == 1
        assert lib.ts_adam_step_segments_ws(bufs, seg, 1, 0, fake, fake, fake, fake, fake,
                                            fake, fake, R, T, flags, None, ws, sz(nbytes),
                                            None) == 1
        assert lib.ts_adagrad_step_segments_ws(bufs, seg, 1, 0, fake, fake, fake, fake, fake,
                                               fake, R, T, flags, None, ws, sz(nbytes),
                                               None) == 1
    # the allocation-free form holds at most 65536 replicas' constants
    assert lib.ts_adam_step_noalloc(bufs, 0, fake, fake, fake, fake, fake, fake, fake,
                                    ctypes.c_int64(65537), T, flags, None, None) == 1


def test_grids_past_the_dispatch_limit_rejected_before_any_launch():
    """A launch counts its work-items in 32 bits, and HIP refuses a larger one.
    A call whose update grid would pass 2^32 - 1 work-items is an invalid
    argument before anything is enqueued (otherwise its preparation launch
    would bump the steps and the update would not run). 16 rows of 2^32
    float32 elements: 2^28 one-wavefront streaming tiles of 256 elements."""
    lib = ctypes.CDLL(str(LIB))
    R, T = 16, 2**32
    fake = ctypes.c_void_p(0x10000)
    bufs = (RTBuf * 5)(*[RTBuf(0x10000 * (i + 1), T, 1) for i in range(5)])
    ws = ctypes.c_void_p(0x80000)
    flags = ctypes.c_uint32(0x10)
    i64, sz = ctypes.c_int64, ctypes.c_size_t
    assert lib.ts_adam_step(bufs, 0, fake, fake, fake, fake, fake, fake, fake, i64(R), i64(T),
                            flags, None, None) == 1
    assert lib.ts_adam_step_ws(bufs, 0, fake, fake, fake, fake, fake, fake, fake, i64(R),
                               i64(T), flags, None, ws, sz(16 * R), None) == 1
    assert lib.ts_adagrad_step_ws(bufs, 0, fake, fake, fake, fake, fake, fake, i64(R), i64(T),
                                  flags, None, ws, sz(16 * R), None) == 1
    assert lib.ts_sgd_step(bufs, 0, fake, fake, fake, fake, fake, fake, i64(R), i64(T), flags,
                           None, None) == 1
    seg = (Segment * 1)(Segment(0x90000, T, 0, T))
    assert lib.ts_adam_step_segments(bufs, seg, 1, 0, fake, fake, fake, fake, fake, fake, fake,
                                     i64(R), i64(T), flags, None, None) == 1
    assert lib.ts_scatter_segments(seg, 1, 0, fake, i64(T), i64(T), i64(R), None) == 1


class Segment(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("stride_r", ctypes.c_int64),
                ("col", ctypes.c_int64), ("numel", ctypes.c_int64)]


class RTBuf(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("stride_r", ctypes.c_int64),
                ("stride_t", ctypes.c_int64)]


@pytest.mark.parametrize("segs", [
    [(0x1000, 16, 8, 8), (0x2000, 16, 0, 12)],   # out of order / overlapping
    [(0x1000, 16, 0, 8), (0x2000, 16, 6, 4)],    # overlapping
    [(0x1000, 16, 12, 8)],                       # past the last column
    [(0x1000, 16, -4, 4)],                       # negative column
    [(0, 16, 0, 4)],                             # no data for a non-empty segment
])
def test_bad_segment_tables_rejected_before_any_launch(segs):
    """Every check runs before the first enqueue: with the (fake, never
    dereferenced) device pointers below, a call that got as far as a launch
    would fault or fail differently; these return hipErrorInvalidValue."""
    lib = ctypes.CDLL(str(LIB))
    fake = ctypes.c_void_p(0x10000)
    bufs = (RTBuf * 5)(*[RTBuf(0x10000 * (i + 1), 16, 1) for i in range(5)])
    table = (Segment * len(segs))(*[Segment(*s) for s in segs])
    R, T = ctypes.c_int64(2), ctypes.c_int64(16)
    flags = ctypes.c_uint32(0x10)
    assert lib.ts_adam_step_segments(bufs, table, len(segs), 0, fake, fake, fake, fake, fake,
                                     fake, fake, R, T, flags, None, None) == 1
    assert lib.ts_sgd_step_segments(bufs, table, len(segs), 0, fake, fake, fake, fake, fake,
                                    fake, R, T, flags, None, None) == 1
    assert lib.ts_adagrad_step_segments(bufs, table, len(segs), 0, fake, fake, fake, fake,
                                        fake, fake, R, T, flags, None, None) == 1
    assert lib.ts_scatter_segments(table, len(segs), 0, fake, ctypes.c_int64(16), T, R,
                                   None) == 1


def test_bf16_state_flag_needs_float32_params():
    lib = ctypes.CDLL(str(LIB))
    fake = ctypes.c_void_p(0x10000)
    bufs = (RTBuf * 5)(*[RTBuf(0x10000 * (i + 1), 16, 1) for i in range(5)])
    R, T = ctypes.c_int64(2), ctypes.c_int64(16)
    for dtype in (1, 2, 3):  # float64, float16, bfloat16 params
        assert lib.ts_adam_step(bufs, dtype, fake, fake, fake, fake, fake, fake, fake, R, T,
                                ctypes.c_uint32(0x20 | 0x10), None, None) == 1
        assert lib.ts_adagrad_step(bufs, dtype, fake, fake, fake, fake, fake, fake, R, T,
                                   ctypes.c_uint32(0x20), None, None) == 1


def test_segmented_calls_reject_a_missing_table_and_nesterov_without_buffer():
    lib = ctypes.CDLL(str(LIB))
    fake = ctypes.c_void_p(0x10000)
    bufs = (RTBuf * 5)(*[RTBuf(0x10000 * (i + 1), 16, 1) for i in range(5)])
    R, T = ctypes.c_int64(2), ctypes.c_int64(16)
    assert lib.ts_adam_step_segments(bufs, None, 3, 0, fake, fake, fake, fake, fake, fake,
                                     fake, R, T, ctypes.c_uint32(0), None, None) == 1
    bufs[2] = RTBuf(0, 0, 1)
    assert lib.ts_sgd_step_segments(bufs, None, 0, 0, fake, fake, fake, fake, fake, fake, R,
                                    T, ctypes.c_uint32(0x8), None, None) == 1


def test_schemas_match_the_reference_text():
    import churten_amd.kernels  # noqa: F401

    for name, want in REFERENCE_SCHEMAS.items():
        got = str(getattr(torch.ops.torchstrap, name).default._schema)
        assert got == want, name


def _meta_adam(R=3, T=8):
    f = dict(device="meta")
    return ([torch.empty(R, T, **f) for _ in range(4)] + [None, torch.empty(R, **f)]
            + [torch.empty(R, **f) for _ in range(5)] + [torch.empty(R, dtype=torch.bool, **f)])


def test_fake_kernels_on_meta_tensors():
    import churten_amd.kernels as K

    out = K.adam_step_(*_meta_adam(), amsgrad=False, maximize=False,
                       decoupled_weight_decay=True)
    assert out.shape == () and out.device.type == "meta" and out.dtype == torch.float32
    m = lambda *s: torch.empty(*s, device="meta")  # noqa: E731
    mask = torch.empty(3, dtype=torch.bool, device="meta")
    out = K.sgd_step_(m(3, 8), m(3, 8), None, m(3), m(3), m(3), m(3), m(3), mask,
                      nesterov=False, maximize=False)
    assert out.shape == ()
    out = K.adagrad_step_(m(3, 8), m(3, 8), m(3, 8), m(3), m(3), m(3), m(3), m(3), mask,
                          maximize=False)
    assert out.shape == ()


def test_vmap_rule_squeezes_replica_dim_on_meta():
    import churten_amd.kernels as K

    B, T = 4, 10
    args = _meta_adam(B, T)
    args[4] = torch.empty(B, T, device="meta")

    def one(p, g, m, v, mx, s, lr, b1, b2, eps, wd, mask):
        return K.adam_step_(p.unsqueeze(0), g.unsqueeze(0), m.unsqueeze(0), v.unsqueeze(0),
                            mx.unsqueeze(0), s.view(1), lr.view(1), b1.view(1), b2.view(1),
                            eps.view(1), wd.view(1), mask.view(1), amsgrad=True,
                            maximize=False, decoupled_weight_decay=True)

    out = vmap(one)(*args)
    # the rule returns one unbatched scalar, which vmap broadcasts over B
    assert out.shape == (B,)


def test_consolidated_helpers():
    from churten_amd.kernels._consolidated import hyp, hyp_mask, lead_squeeze

    t = torch.zeros(5, 3, 1, 7)  # batch dim at 2
    out = lead_squeeze(torch.zeros(7, 1, 5), 2)
    assert out.shape == (5, 7, 1)
    out = lead_squeeze(t.movedim(2, 0), 0)
    assert out.shape == (1, 5, 3, 7)
    assert lead_squeeze(torch.zeros(4, 1, 9), 0).shape == (4, 9)
    assert lead_squeeze(torch.zeros(9, 4), 1).shape == (4, 9)
    assert not lead_squeeze(torch.zeros(9, 4), 1).is_contiguous()
    assert hyp(torch.tensor(2.0), None, 3).tolist() == [2.0, 2.0, 2.0]
    assert hyp(torch.tensor([1.0, 2.0]), None, 2).tolist() == [1.0, 2.0]
    assert hyp_mask(torch.tensor([1.0, 0.0]), 0, 2).dtype == torch.bool
    assert lead_squeeze(t, None) is t


def test_only_cpu_and_gpu_keys_are_served():
    """CPU tensors go to the CPU kernels, GPU tensors to the HIP kernels; any
    other device raises from the dispatcher -- there is no catch-all kernel."""
    import churten_amd.kernels  # noqa: F401

    for name in ["torchstrap::adam_step_", "torchstrap::sgd_step_", "torchstrap::adagrad_step_",
                 "churten::scatter_grads_", "churten::adam_step_segments_",
                 "churten::sgd_step_segments_", "churten::adagrad_step_segments_"]:
        assert torch._C._dispatch_has_kernel_for_dispatch_key(name, "CPU")
        assert torch._C._dispatch_has_kernel_for_dispatch_key(name, "CUDA")
        assert not torch._C._dispatch_has_kernel_for_dispatch_key(name, "CompositeImplicitAutograd")
        assert not torch._C._dispatch_has_kernel_for_dispatch_key(name, "CompositeExplicitAutograd")


def test_product_never_imports_the_oracle():
    for f in (ROOT / "churten_amd").rglob("*"):
        if f.suffix in (".py", ".cpp", ".hip", ".h"):
            text = f.read_text()
            assert "import oracle" not in text and "from oracle" not in text, f
            assert "liboracle" not in text and "optim_oracle" not in text, f


@pytest.mark.parametrize("device", ["cpu", pytest.param("cuda", marks=pytest.mark.gpu)])
def test_ops_trace_under_torch_compile(device):
    """The fake kernels and alias annotations let a step containing the ops be
    captured whole (fullgraph) and functionalized; results equal eager."""
    import churten_amd.kernels as K

    R, T = 3, 20
    g0 = torch.Generator().manual_seed(0)
    mk = lambda: torch.randn(R, T, generator=g0).to(device)  # noqa: E731
    h = [torch.full((R,), x, device=device) for x in (1e-2, 0.9, 0.999, 1e-8, 1e-2)]
    mask = torch.tensor([True, False, True], device=device)

    def step(p, g, m, v, st, b, s):
        K.adam_step_(p, g * 2.0, m, v, None, st, *h, mask, amsgrad=False, maximize=False,
                     decoupled_weight_decay=True)
        K.sgd_step_(b, g, None, st.clone(), h[0], h[4], h[4], h[4], mask, nesterov=False,
                    maximize=False)
        K.adagrad_step_(s, g, s.abs().clone(), st.clone(), h[0], h[4], h[4], h[3], mask,
                        maximize=True)
        return p.sum() + b.sum() + s.sum()

    eager = [mk(), mk(), mk(), mk().abs(), torch.zeros(R, device=device), mk(), mk()]
    comp = [t.clone() for t in eager]
    compiled = torch.compile(step, fullgraph=True, backend="aot_eager")
    g = eager[1]
    for _ in range(2):
        a = step(*eager[:1], g, *eager[2:])
        b = compiled(*comp[:1], g, *comp[2:])
        assert torch.equal(a, b)
    for x, y in zip(eager, comp):
        assert torch.equal(x, y)


def test_build_compiles_every_library_source_and_reports_a_failed_job():
    """build() compiles each translation unit of the library as its own job
    (they run concurrently) and links them once all have finished; a job that
    fails raises from the pool instead of being lost in a worker thread."""
    from churten_amd import _build

    csrc = Path(_build.CSRC)
    assert {p.name for p in csrc.glob("abi_*.hip")} <= set(_build.LIB_SOURCES)
    assert {"optim_kernels.hip", "rows.hip"} <= set(_build.LIB_SOURCES)
    objs, jobs = _build._library_objects(verbose=False)
    assert len(objs) == len(jobs) == len(_build.LIB_SOURCES)
    ran = []

    def ok():
        ran.append(1)

    def fail():
        raise RuntimeError("build step failed (1): hipcc")

    with pytest.raises(RuntimeError, match="build step failed"):
        _build._parallel([ok, fail, ok])
    assert len(ran) == 2
