"""Parameter-holding primitives with the reference's names, shapes and init.

``LayerNorm``, ``LinearNoBias`` and ``af3_linear_init_`` follow
``src/deepfold3/model/primitives.py:47-155`` so state dicts are interchangeable.
In this package they hold parameters; the math runs inside the fused HIP
kernels that read them (``kernels.py``). ``LayerNorm.forward`` runs the HIP
LayerNorm kernel.
"""

from __future__ import annotations

import math

import torch
import torch.nn as nn

TRUNCATED_NORMAL_STDDEV_FACTOR = 0.87962566103423978


def af3_linear_init_(weight: torch.Tensor, initializer: str = "linear") -> None:
    """AF3 variance-scaled truncated normal (``primitives.py:47-61``), truncated at +-2 absolute as there."""
    if initializer == "zeros":
        nn.init.zeros_(weight)
        return
    fan_in = weight.shape[1] if weight.dim() >= 2 else weight.shape[0]
    scale = 1.0 / fan_in
    if initializer == "relu":
        scale *= 2.0
    stddev = math.sqrt(scale) / TRUNCATED_NORMAL_STDDEV_FACTOR
    nn.init.trunc_normal_(weight, mean=0.0, std=stddev, a=-2.0, b=2.0)


class LinearNoBias(nn.Linear):
    """``nn.Linear`` without bias and with AF3 init (``primitives.py:64-76``)."""

    def __init__(self, in_features: int, out_features: int, initializer: str = "linear"):
        super().__init__(in_features, out_features, bias=False)
        af3_linear_init_(self.weight, initializer)


class LayerNorm(nn.LayerNorm):
    """LayerNorm with fp32 statistics, output in the input dtype (``primitives.py:90-155``)."""

    def __init__(self, normalized_shape: int, *, eps: float = 1e-5, elementwise_affine: bool = True, bias: bool = True):
        super().__init__(normalized_shape, eps=eps, elementwise_affine=elementwise_affine, bias=bias)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        from .kernels import layer_norm

        return layer_norm(x, self.weight, self.bias, self.eps)
