"""MI355X-native (gfx950) Lizard attention hot path.

``lizard_reproduction_amd.kernels`` is the drop-in for the reference's
``kernels`` package: ``gla`` (chunked gated linear attention) and ``swa``
(sliding-window softmax with sink logits), forward and backward in bf16, on
hand-written HIP kernels behind the C ABI of ``_lib/liblizard_hip.so``.
"""
from . import kernels
from .kernels import gla, swa

__all__ = ["kernels", "gla", "swa"]
