"""The ``torchstrap`` fused optimizer operators on the MI355X.

Importing this package loads ``churten_amd/kernels/_C.so``, which defines
``torch.ops.torchstrap.adam_step_``, ``sgd_step_`` and ``adagrad_step_`` with
the reference's schemas (src/torchstrap/kernels/csrc/stubs.cpp:25-72) and
implements the GPU dispatch key with hand-written gfx950 HIP kernels (plus the
``torch.ops.churten`` scatter-fused forms, see ``segments``), then adds
the Python ``register_fake`` / ``register_vmap`` rules
(src/torchstrap/kernels/{adam,sgd,adagrad}.py). A device without a registered
kernel raises ``NotImplementedError`` from the dispatcher; a missing build
raises ``ImportError`` here -- there is no fallback implementation.
"""

from __future__ import annotations

import importlib
from pathlib import Path

_HERE = Path(__file__).resolve().parent


def _load_native():
    if not (_HERE / "_C.so").exists():
        raise ImportError(
            "churten_amd.kernels._C is not built; run `python -m churten_amd._build` "
            "(or __graft_entry__.build()) first"
        )
    return importlib.import_module("churten_amd.kernels._C")


_C = _load_native()

from churten_amd.kernels.adam import adam_step_  # noqa: E402
from churten_amd.kernels.sgd import sgd_step_  # noqa: E402
from churten_amd.kernels.adagrad import adagrad_step_, adagrad_step_f32_  # noqa: E402
from churten_amd.kernels.segments import (  # noqa: E402
    adagrad_step_segments_,
    adam_step_segments_,
    scatter_grads_,
    sgd_step_segments_,
)

__all__ = ("adam_step_", "sgd_step_", "adagrad_step_", "adagrad_step_f32_", "scatter_grads_",
           "adam_step_segments_", "sgd_step_segments_", "adagrad_step_segments_")
