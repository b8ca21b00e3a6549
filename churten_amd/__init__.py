"""churten_amd -- MI355X-native fused batched optimizer step.

A from-scratch gfx950 implementation of the ``torchstrap`` ensemble
optimizer's hot path: one operator call updates every parameter of every
replica of an N-replica ensemble held in consolidated ``(N, T)`` buffers.

* ``churten_amd.kernels`` -- the ``torch.ops.torchstrap.*_step_`` operators
  (native library + fake/vmap rules).
"""

__version__ = "0.1.0"
