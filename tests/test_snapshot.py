"""Snapshot / Checkpoint: the device-to-host path of the ensemble state.

Mirrors the reference's callback tests for these classes
(src/torchstrap/callbacks/training.py:16-224 semantics): the mirror starts as a
copy of every leaf, ``update`` copies only active-and-selected rows, restore is
in place and not gated by ``active_mask``, ``Checkpoint`` keeps per-replica best
scores and writes only when a replica improved, and the files read back
identically. The GPU cases also cover the row-transfer entry point directly
(contiguous and pitched rows, both directions).
"""

from __future__ import annotations

import ctypes
import json
from copy import deepcopy
from pathlib import Path

import numpy as np
import pytest
import torch
from torch.nn import Linear, ReLU, Sequential

from churten_amd.optimizer import Adam
from churten_amd.snapshot import Checkpoint, Snapshot
from churten_amd.state import State

DEVICES = ["cpu", pytest.param("cuda", marks=pytest.mark.gpu)]
LIB = Path(__file__).resolve().parents[1] / "churten_amd" / "lib" / "libchurten_optim.so"


def trained_state(device, n=4, steps=2, state_dtype=None):
    torch.manual_seed(0)
    net = Sequential(Linear(5, 9), ReLU(), Linear(9, 2)).to(device)
    state = State.from_models([deepcopy(net) for _ in range(n)])
    Adam.init(state, lr=torch.linspace(1e-3, 1e-2, n), amsgrad=True, state_dtype=state_dtype)
    g = torch.Generator().manual_seed(1)
    for _ in range(steps):
        grads = {k: torch.randn(*s, generator=g).to(device) for k, s, _, _ in state.param_meta}
        Adam.apply_gradient(state, grads)
    return state


def leaves(state):
    out = {"params": state.params, "grads": state.grads, "active_mask": state.active_mask}
    out.update({k: v for k, v in state.optimizer_state.items() if isinstance(v, torch.Tensor)})
    return out


def mirror_leaf(snap, name):
    t = snap.tensors
    return t[name] if name in t else t["optimizer_state." + name]


@pytest.mark.parametrize("device", DEVICES)
@pytest.mark.parametrize("state_dtype", [None, torch.bfloat16])
def test_mirror_starts_as_a_copy_and_updates_selected_rows(device, state_dtype):
    state = trained_state(device, state_dtype=state_dtype)
    snap = Snapshot(state)
    before = {k: v.cpu().clone() for k, v in leaves(state).items()}
    for k, v in before.items():
        assert torch.equal(mirror_leaf(snap, k), v), k
    if device == "cuda":
        assert snap.tensors["params"].is_pinned()
    # train more; freeze replica 3; select replicas 0 and 3 -> only 0 is copied
    state.active_mask[3] = False
    g = torch.Generator().manual_seed(2)
    grads = {k: torch.randn(*s, generator=g).to(device) for k, s, _, _ in state.param_meta}
    Adam.apply_gradient(state, grads)
    state.params[3] += 1.0  # a frozen replica changed by the user: still not copied
    sel = torch.tensor([True, False, False, True], device=device)
    assert snap.update(state, sel)
    now = {k: v.cpu() for k, v in leaves(state).items()}
    for k in now:
        m = mirror_leaf(snap, k)
        assert torch.equal(m[0], now[k][0]), k
        for r in (1, 2, 3):
            assert torch.equal(m[r], before[k][r]), (k, r)
    assert not snap.update(state, torch.zeros(4, dtype=torch.bool, device=device))


@pytest.mark.parametrize("device", DEVICES)
def test_restore_is_in_place_and_ignores_the_active_mask(device):
    state = trained_state(device)
    snap = Snapshot(state)
    saved = {k: v.cpu().clone() for k, v in leaves(state).items()}
    views = state.params_dict
    state.active_mask[1] = False
    for t in (state.params, state.optimizer_state["exp_avgs"], state.optimizer_state["lr"]):
        t.add_(3.0)
    params_ptr = state.params.data_ptr()
    snap.restore_to_live(state, torch.tensor([False, True, False, False]))
    assert state.params.data_ptr() == params_ptr
    assert torch.equal(state.params[1].cpu(), saved["params"][1])
    assert torch.equal(state.optimizer_state["lr"][1].cpu(), saved["lr"][1])
    assert torch.equal(state.params[0].cpu(), saved["params"][0] + 3.0)
    assert state.active_mask.tolist() == [True, True, True, True]  # restored too
    snap.restore_to_live(state)
    for k, v in leaves(state).items():
        assert torch.equal(v.cpu(), saved[k]), k
    assert torch.equal(views["0.weight"], state.params_dict["0.weight"])


@pytest.mark.parametrize("device", DEVICES)
def test_files_round_trip_lazily(device, tmp_path):
    state = trained_state(device, state_dtype=torch.bfloat16)
    snap = Snapshot(state)
    target = snap.to_file(tmp_path, "ckpt")
    assert (target / "meta.json").exists()
    back = Snapshot.from_file(tmp_path, "ckpt")
    for k, v in snap.tensors.items():
        w = back.tensors[k]
        assert w.dtype == v.dtype and torch.equal(w, v), k
    assert back.optimizer_meta == snap.optimizer_meta and back.batch_size == 4
    # copy-on-write: changing the loaded mirror never touches the file
    back.tensors["params"].fill_(0.0)
    again = Snapshot.from_file(tmp_path, "ckpt")
    assert torch.equal(again.tensors["params"], snap.tensors["params"])
    # a resumed state trains on like the original
    resumed = again.to_state(device)
    assert resumed.optimizer_state["amsgrad"] is True
    for k, v in leaves(state).items():
        assert torch.equal(leaves(resumed)[k], v), k


@pytest.mark.parametrize("device", DEVICES)
def test_checkpoint_keeps_per_replica_best(device, tmp_path):
    state = trained_state(device)
    msgs = []
    ckpt = Checkpoint(root_dir=tmp_path, sink=msgs.append)
    assert ckpt(state, torch.tensor([1.0, 2.0, 3.0, 4.0])).tolist() == [True] * 4
    first = state.params.cpu().clone()
    state.params.add_(1.0)
    improved = ckpt(state, torch.tensor([0.5, 2.5, 3.0, 1.0]))
    assert improved.tolist() == [True, False, False, True]
    assert msgs[-1] == "Checkpoint saved (2 replica(s) improved)."
    n_msgs = len(msgs)
    assert not ckpt(state, torch.tensor([9.0, 9.0, 9.0, 9.0])).any()
    assert len(msgs) == n_msgs  # nothing improved: nothing written
    state.params.add_(5.0)
    ckpt.load_best(state)
    want = first.clone()
    want[[0, 3]] += 1.0
    assert torch.equal(state.params.cpu(), want)


class _History(dict):
    """A stand-in with the reference History's file interface (history.py)."""

    def to_file(self, path):
        Path(path).write_text(json.dumps(self))

    @classmethod
    def from_file(cls, path):
        return cls(json.loads(Path(path).read_text()))


@pytest.mark.parametrize("device", DEVICES)
def test_load_best_without_checkpoint_restores_nothing(device, tmp_path):
    """As training.py:203-214: a checkpoint (or history) that was never
    written is not an error; the live state and the history stay as they are."""
    state = trained_state(device)
    before = state.params.clone()
    msgs = []
    ckpt = Checkpoint(root_dir=tmp_path / "never_written", sink=msgs.append)
    hist = _History(loss=[1.0])
    ckpt.load_best(state)
    ckpt.load_best(state, hist)
    assert torch.equal(state.params, before) and hist == {"loss": [1.0]} and msgs == []


@pytest.mark.parametrize("device", DEVICES)
def test_load_best_restores_the_saved_history(device, tmp_path):
    state = trained_state(device)
    msgs = []
    ckpt = Checkpoint(root_dir=tmp_path, sink=msgs.append)
    ckpt(state, torch.tensor([1.0, 2.0, 3.0, 4.0]), history=_History(loss=[0.5, 0.25]))
    live = _History(loss=[9.0], extra=[1])
    ckpt.load_best(state, live)
    assert live == {"loss": [0.5, 0.25]}
    assert msgs[-1] == "Loaded best checkpoint."


@pytest.mark.gpu
@pytest.mark.parametrize("pad", [0, 3])
def test_copy_rows_entry_point(pad):
    """Contiguous (pad=0) and pitched rows, device -> pinned host -> device."""
    lib = ctypes.CDLL(str(LIB))
    v, i64 = ctypes.c_void_p, ctypes.c_int64
    lib.ts_copy_rows.argtypes = [v, i64, v, i64, i64, v, i64, ctypes.c_int, v]
    R, T = 7, 1001
    src = torch.randn(R, T + pad, device="cuda")[:, :T]
    host = torch.full((R, T + pad), -1.0, pin_memory=True)[:, :T]
    rows = np.array([1, 1, 0, 1, 0, 0, 1], dtype=np.uint8)
    stream = torch.cuda.current_stream().cuda_stream
    assert lib.ts_copy_rows(host.data_ptr(), (T + pad) * 4, src.data_ptr(), (T + pad) * 4,
                            T * 4, rows.ctypes.data, R, 0, stream) == 0
    torch.cuda.synchronize()
    sel = torch.from_numpy(rows.astype(bool))
    assert torch.equal(host[sel], src.cpu()[sel])
    assert (host[~sel] == -1.0).all()
    dst = torch.zeros(R, T + pad, device="cuda")[:, :T]
    assert lib.ts_copy_rows(dst.data_ptr(), (T + pad) * 4, host.data_ptr(), (T + pad) * 4,
                            T * 4, None, R, 1, stream) == 0
    torch.cuda.synchronize()
    assert torch.equal(dst.cpu(), host)


def test_copy_rows_rejects_bad_arguments():
    lib = ctypes.CDLL(str(LIB))
    v, i64 = ctypes.c_void_p, ctypes.c_int64
    lib.ts_copy_rows.argtypes = [v, i64, v, i64, i64, v, i64, ctypes.c_int, v]
    fake = 0x10000
    assert lib.ts_copy_rows(fake, 16, fake, 16, 16, None, 4, 7, None) == 1      # direction
    assert lib.ts_copy_rows(fake, 8, fake, 16, 16, None, 4, 0, None) == 1       # stride < row
    assert lib.ts_copy_rows(None, 16, fake, 16, 16, None, 4, 0, None) == 1      # null dst
    assert lib.ts_copy_rows(None, 16, None, 16, 16, None, 0, 0, None) == 0      # nothing to do
