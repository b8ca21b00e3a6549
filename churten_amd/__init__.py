"""churten_amd -- MI355X-native fused batched optimizer step.

A from-scratch gfx950 implementation of the ``torchstrap`` ensemble
optimizer's hot path: one operator call updates every parameter of every
replica of an N-replica ensemble held in consolidated ``(N, T)`` buffers.

* ``churten_amd.kernels`` -- the ``torch.ops.torchstrap.*_step_`` operators
  (native library + fake/vmap rules), and this build's ``torch.ops.churten``
  additions: the gradient scatter fused into the update, the float32 Adagrad.
* ``churten_amd.state`` -- ``State``, the consolidated ``(N, T)`` layout.
* ``churten_amd.optimizer`` -- ``Adam``, ``SGD``, ``Adagrad`` over a ``State``.
* ``churten_amd.snapshot`` -- ``Snapshot`` / ``Checkpoint``, the
  device-to-host path.
"""

__version__ = "0.4.0"
