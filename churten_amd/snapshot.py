"""Ensemble snapshots and checkpoints: the device-to-host path.

Restates the reference's ``Snapshot`` and ``Checkpoint``
(src/torchstrap/callbacks/training.py:16-224) for this build's ``State``:

* ``Snapshot(state)`` keeps a host mirror of every ``(N, ...)`` leaf of the
  state (params, buffers, grads, the optimizer's tensors, ``active_mask``);
  ``update(state, extra_mask)`` copies the rows of the replicas that are active
  (and selected) into it, ``restore_to_live(state, mask)`` copies mirror rows
  back into the live state in place, ``to_file`` / ``from_file`` write and
  lazily read it on disk;
* ``Checkpoint(...)(state, score)`` keeps per-replica best scores and
  snapshots the improved replicas, writing the checkpoint when any improved;
  ``load_best(state)`` restores every row from the file.

The transfer is this build's own: the mirror is pinned host memory, and each
leaf's selected rows move by DMA directly between the live buffer and the
mirror, one copy per run of consecutive rows (``ts_copy_rows`` in
``include/churten_optim.h``), then one stream synchronisation. The reference
gathers the rows on the device, copies them into a second, full-size pinned
staging state and scatters them on the host. The mask comes to the host first,
so an epoch in which no replica improved moves nothing else.

On-disk format (this build's; tensordict's memmap layout is not available
here): a directory holding ``meta.json`` -- format name and version, the batch
size, the offset tables, the optimizer's non-tensor flags, and for every leaf
its file, dtype and shape -- and one raw little-endian file per leaf.
``from_file`` maps those files copy-on-write, so nothing is read before it is
used and nothing is written back.
"""

from __future__ import annotations

import ctypes
import json
import shutil
from contextlib import suppress
from pathlib import Path
from typing import Any, Callable

import numpy as np
import torch

from churten_amd.state import State

__all__ = ["Snapshot", "Checkpoint", "FORMAT", "FORMAT_VERSION"]

FORMAT = "churten-snapshot"
FORMAT_VERSION = 1

_TO_HOST, _TO_DEVICE = 0, 1
_lib = None


def _native():
    global _lib
    if _lib is None:
        path = Path(__file__).resolve().parent / "lib" / "libchurten_optim.so"
        if not path.exists():
            raise ImportError(f"{path} is not built; run `python -m churten_amd._build`")
        lib = ctypes.CDLL(str(path))
        v, i64 = ctypes.c_void_p, ctypes.c_int64
        lib.ts_copy_rows.argtypes = [v, i64, v, i64, i64, v, i64, ctypes.c_int, v]
        lib.ts_copy_rows.restype = ctypes.c_int
        _lib = lib
    return _lib


def _rows_contiguous(t: torch.Tensor) -> bool:
    """Each dim-0 slice is one contiguous block."""
    return t.dim() >= 1 and t[0:1].is_contiguous()


def _copy_rows(dst: torch.Tensor, src: torch.Tensor, rows: np.ndarray | None,
               direction: int) -> None:
    """Rows ``rows`` (host bool array, None = all) of ``src`` into ``dst``, by
    DMA on the current stream (one GPU side, one pinned host side)."""
    R = src.shape[0] if src.dim() else 1
    es = src.element_size()
    row_bytes = (src.numel() // R if R else 0) * es
    mask = None
    if rows is not None:
        mask = np.ascontiguousarray(rows, dtype=np.uint8)
    gpu = src if direction == _TO_HOST else dst
    stream = torch.cuda.current_stream(gpu.device).cuda_stream
    rc = _native().ts_copy_rows(
        dst.data_ptr(), dst.stride(0) * es if dst.dim() else es,
        src.data_ptr(), src.stride(0) * es if src.dim() else es, row_bytes,
        None if mask is None else mask.ctypes.data, R, direction, stream)
    if rc != 0:
        raise RuntimeError(f"ts_copy_rows failed with HIP error {rc}")


def _leaves(state: State) -> dict[str, torch.Tensor]:
    out = {"params": state.params, "buffers": state.buffers, "grads": state.grads,
           "active_mask": state.active_mask}
    for k, v in state.optimizer_state.items():
        if isinstance(v, torch.Tensor):
            out["optimizer_state." + k] = v
    return out


def _optim_meta(state: State) -> dict[str, Any]:
    return {k: v for k, v in state.optimizer_state.items() if not isinstance(v, torch.Tensor)}


class Snapshot:
    """Host mirror of the whole ensemble state, updated and restored by rows."""

    def __init__(self, state: State):
        self.param_meta = [list(m) for m in state.param_meta]
        self.buffer_meta = [list(m) for m in state.buffer_meta]
        self.param_buffer_dtype = state.param_buffer_dtype
        self.optimizer_meta = _optim_meta(state)
        self.batch_size = int(state.params.shape[0])
        pin = state.params.is_cuda
        self._mirror: dict[str, torch.Tensor] = {}
        with torch.no_grad():
            for name, t in _leaves(state).items():
                m = torch.empty(t.shape, dtype=t.dtype, pin_memory=pin)
                self._mirror[name] = m
                self._transfer(m, t, None, _TO_HOST)
            if pin:
                torch.cuda.current_stream(state.params.device).synchronize()

    # -- transfers ---------------------------------------------------------
    @staticmethod
    def _transfer(dst: torch.Tensor, src: torch.Tensor, rows: np.ndarray | None,
                  direction: int) -> None:
        gpu = src if direction == _TO_HOST else dst
        if (gpu.is_cuda and _rows_contiguous(dst) and _rows_contiguous(src)
                and dst.dtype == src.dtype and dst.shape == src.shape):
            _copy_rows(dst, src, rows, direction)
            return
        if rows is None:
            dst.copy_(src)
            return
        idx = torch.from_numpy(np.flatnonzero(rows))
        dst.index_copy_(0, idx.to(dst.device), src.index_select(0, idx.to(src.device)).to(dst.device))

    @property
    def tensors(self) -> dict[str, torch.Tensor]:
        """The mirror's leaves by name (read-only use)."""
        return dict(self._mirror)

    def to_state(self, device=None) -> State:
        """A new ``State`` holding copies of the mirror (on ``device``, default
        CPU), e.g. to resume from a checkpoint in a fresh process."""
        dev = torch.device(device or "cpu")
        t = {k: v.to(dev, copy=True) for k, v in self._mirror.items()}
        state = State(params=t["params"], buffers=t["buffers"],
                      param_meta=[tuple(m) for m in self.param_meta],
                      buffer_meta=[tuple(m) for m in self.buffer_meta],
                      param_buffer_dtype=self.param_buffer_dtype,
                      active_mask=t["active_mask"], grads=t["grads"])
        for k, v in t.items():
            if k.startswith("optimizer_state."):
                state.optimizer_state[k.removeprefix("optimizer_state.")] = v
        state.optimizer_state.update(self.optimizer_meta)
        return state

    @torch.no_grad()
    def update(self, state: State, extra_mask: torch.Tensor | None = None) -> bool:
        """Copy the active (and ``extra_mask``-selected) replicas' rows of every
        leaf into the mirror. Returns whether any row was copied; when none was,
        only the (N,) mask crossed to the host."""
        mask = state.active_mask
        if extra_mask is not None:
            mask = mask & extra_mask.to(mask.device)
        rows = mask.to("cpu").numpy().astype(bool)
        if not rows.any():
            return False
        for name, t in _leaves(state).items():
            self._transfer(self._mirror[name], t, rows, _TO_HOST)
        if state.params.is_cuda:
            torch.cuda.current_stream(state.params.device).synchronize()
        return True

    @torch.no_grad()
    def restore_to_live(self, state: State, mask: torch.Tensor | None = None) -> None:
        """Write mirror rows back into the live state in place (not gated by
        ``active_mask``: the rows that most need restoring are frozen ones).
        ``mask=None`` restores every row."""
        rows = None
        if mask is not None:
            rows = torch.as_tensor(mask, dtype=torch.bool).reshape(-1).to("cpu").numpy()
            if not rows.any():
                return
        for name, t in _leaves(state).items():
            self._transfer(t, self._mirror[name], rows, _TO_DEVICE)
        if state.params.is_cuda:
            torch.cuda.current_stream(state.params.device).synchronize()

    # -- files -------------------------------------------------------------
    def to_file(self, root_dir_path, file_name: str | None = None) -> Path:
        target = Path(root_dir_path) / (file_name or "state_dict")
        if target.is_dir():
            shutil.rmtree(target)
        elif target.exists():
            target.unlink()
        target.mkdir(parents=True)
        leaves = {}
        for i, (name, t) in enumerate(self._mirror.items()):
            fname = f"{i:03d}.bin"
            with open(target / fname, "wb") as f:
                f.write(memoryview(t.contiguous().reshape(-1).view(torch.uint8).numpy()))
            leaves[name] = {"file": fname, "dtype": str(t.dtype).removeprefix("torch."),
                            "shape": list(t.shape)}
        meta = {"format": FORMAT, "version": FORMAT_VERSION, "batch_size": self.batch_size,
                "param_meta": [[n, list(s), o, k] for n, s, o, k in self.param_meta],
                "buffer_meta": [[n, list(s), o, k] for n, s, o, k in self.buffer_meta],
                "param_buffer_dtype": str(self.param_buffer_dtype).removeprefix("torch."),
                "optimizer_meta": self.optimizer_meta, "leaves": leaves}
        (target / "meta.json").write_text(json.dumps(meta, indent=1))
        return target

    @classmethod
    def from_file(cls, root_dir_path, file_name: str | None = None) -> "Snapshot":
        target = Path(root_dir_path) / (file_name or "state_dict")
        meta = json.loads((target / "meta.json").read_text())
        if meta.get("format") != FORMAT or meta.get("version") != FORMAT_VERSION:
            raise ValueError(f"{target} is not a {FORMAT} v{FORMAT_VERSION} directory")
        inst = cls.__new__(cls)
        inst.param_meta = [[n, torch.Size(s), o, k] for n, s, o, k in meta["param_meta"]]
        inst.buffer_meta = [[n, torch.Size(s), o, k] for n, s, o, k in meta["buffer_meta"]]
        inst.param_buffer_dtype = getattr(torch, meta["param_buffer_dtype"])
        inst.optimizer_meta = meta["optimizer_meta"]
        inst.batch_size = meta["batch_size"]
        inst._mirror = {}
        for name, leaf in meta["leaves"].items():
            dtype = getattr(torch, leaf["dtype"])
            nbytes = int(np.prod(leaf["shape"], dtype=np.int64)) * dtype.itemsize
            if nbytes == 0:
                inst._mirror[name] = torch.empty(leaf["shape"], dtype=dtype)
                continue
            raw = np.memmap(target / leaf["file"], dtype=np.uint8, mode="c", shape=(nbytes,))
            inst._mirror[name] = torch.from_numpy(raw).view(dtype).reshape(leaf["shape"])
        return inst


class Checkpoint:
    """Save the ensemble's best-so-far replica rows when a per-replica score
    improves. ``ckpt(state, score)`` returns the ``(N,)`` improved mask."""

    def __init__(self, lower_is_better: bool = True, root_dir="checkpoint",
                 f_state: str = "state_dict", f_history: str = "history.json",
                 fn_prefix: str = "", sink: Callable = print, verbose: bool = True):
        self.lower_is_better = lower_is_better
        self.root_dir = Path(root_dir)
        self.f_state = f_state
        self.f_history = f_history
        self.fn_prefix = fn_prefix
        self.sink = sink
        self.verbose = verbose
        self._snapshot: Snapshot | None = None
        self._best: torch.Tensor | None = None

    @torch.no_grad()
    def __call__(self, state: State, score, history=None) -> torch.Tensor:
        score_cpu = torch.as_tensor(score).detach().to("cpu").reshape(-1).float()
        if self._best is None:
            fill = float("inf") if self.lower_is_better else float("-inf")
            self._best = torch.full_like(score_cpu, fill)
        improved = (score_cpu.lt(self._best) if self.lower_is_better
                    else score_cpu.gt(self._best))
        self._best = torch.where(improved, score_cpu, self._best)
        if self._snapshot is None:
            self._snapshot = Snapshot(state)
        if self._snapshot.update(state, improved.to(state.params.device)):
            self.root_dir.mkdir(parents=True, exist_ok=True)
            self._snapshot.to_file(self.root_dir, self.fn_prefix + self.f_state)
            if history is not None:
                history.to_file(self.root_dir / (self.fn_prefix + self.f_history))
            self._sink(f"Checkpoint saved ({int(improved.sum())} replica(s) improved).")
        return improved

    @torch.no_grad()
    def load_best(self, state: State, history=None) -> None:
        """Restore every row of the saved checkpoint into the live state, and
        the saved history into ``history`` when one is given (an object with
        the reference History's ``from_file`` / ``clear`` / ``update``). A
        checkpoint or history that was never written is not an error: nothing
        is restored (training.py:203-214)."""
        with suppress(FileNotFoundError):
            snap = Snapshot.from_file(self.root_dir, self.fn_prefix + self.f_state)
            snap.restore_to_live(state)
            self._sink("Loaded best checkpoint.")
        if history is not None:
            with suppress(FileNotFoundError):
                loaded = type(history).from_file(self.root_dir / (self.fn_prefix + self.f_history))
                history.clear()
                history.update(loaded)

    def _sink(self, text: str) -> None:
        # a custom sink always receives the message; print only when verbose
        if self.sink is not print or self.verbose:
            self.sink(text)
