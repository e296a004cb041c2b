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


class WeightCache:
    """Prepared (cast / packed) weight operands, rebuilt when a parameter changes.

    One entry per (operand dtype, caller tag); the tag is a folded residual scale, so a
    module called both unscaled (its own ``forward``) and scaled (inside its block) keeps
    both. An entry is valid while every parameter's storage pointer and in-place version
    counter are unchanged, so an optimizer step or ``load_state_dict`` invalidates it.
    """

    _MAX_ENTRIES = 4

    def __init__(self):
        self._entries: dict = {}

    def get(self, params: list[torch.Tensor | None], dtype: torch.dtype, build, tag=None):
        slot = (dtype, tag)
        key = tuple(None if p is None else (p.data_ptr(), p._version) for p in params)
        hit = self._entries.get(slot)
        if hit is not None and hit[0] == key:
            return hit[1]
        if slot not in self._entries and len(self._entries) >= self._MAX_ENTRIES:
            self._entries.clear()
        val = build()
        self._entries[slot] = (key, val)
        return val


def f32(t: torch.Tensor) -> torch.Tensor:
    """A detached contiguous fp32 copy (LayerNorm affine and bias operands)."""
    return t.detach().to(torch.float32).contiguous()


class LayerNorm(nn.LayerNorm):
    """LayerNorm with fp32 statistics, output in the input dtype (``primitives.py:90-155``)."""

    def __init__(self, normalized_shape: int, *, eps: float = 1e-5, elementwise_affine: bool = True, bias: bool = True):
        super().__init__(normalized_shape, eps=eps, elementwise_affine=elementwise_affine, bias=bias)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        from .kernels import layer_norm

        return layer_norm(x, self.weight, self.bias, self.eps)


class TransitionBlock(nn.Module):
    """SwiGLU transition ``y = (silu(a) * b) W2^T`` with ``[a | b] = LN(x) W1^T`` (``primitives.py:193-251``).

    Same parameters and state-dict keys as the reference (``norm.*``, ``linear1.weight``
    ``[2 n C, C]``, ``linear2.weight`` ``[C, n C]``; ``fused_transition.py:63-65``). C=128 with
    factor 4 runs the fused pair-transition kernel (hidden activations stay on chip); any
    other shape runs LayerNorm + two MFMA row GEMMs.
    """

    def __init__(
        self,
        channels: int,
        num_intermediate_factor: int = 4,
        optim=None,
        linear_out_init_gain: float | None = None,
    ):
        super().__init__()
        from .config import require_hip

        require_hip("TransitionBlock", optim)
        c, n = channels, num_intermediate_factor
        self.c, self.n = c, n
        self.norm = LayerNorm(c)
        # Default init as the reference's (primitives.py:219-238): linear1 ("linear_gate",
        # feeding SwiGLU) with the AF3 "relu" scaling, linear2 zero, or, with
        # linear_out_init_gain, a row-orthogonal linear2 scaled by that gain.
        self.linear1 = LinearNoBias(c, 2 * n * c, initializer="relu")
        self.linear2 = LinearNoBias(n * c, c, initializer="zeros")
        if linear_out_init_gain is not None:
            nn.init.orthogonal_(self.linear2.weight, gain=float(linear_out_init_gain))
        self._cache = WeightCache()
        # Residual scale of this branch inside its block (s_ros times the transition's residual
        # gain), folded into linear2 by ``branch`` and ``forward_residual_``.
        self.branch_scale = 1.0

    @property
    def fused_pair(self) -> bool:
        return self.c == 128 and self.n == 4

    def operands(self, cdt: torch.dtype, scale: float = 1.0) -> dict:
        from .kernels import cast_weight, scaled_weight

        params = [self.norm.weight, self.norm.bias, self.linear1.weight, self.linear2.weight]

        def build():
            return dict(
                w1=cast_weight(self.linear1.weight, cdt),
                w2=scaled_weight(self.linear2.weight, scale, cdt),
                lnw=f32(self.norm.weight), lnb=f32(self.norm.bias),
            )  # fmt: skip

        return self._cache.get(params, cdt, build, tag=float(scale))

    def run(self, x: torch.Tensor, out=None, accumulate: bool = False, s2p=None, scale: float = 1.0):
        """The kernels: ``scale * transition(x)``, into ``out`` (added to it with ``accumulate``)."""
        from . import kernel_census
        from .kernels import gemm_dtype_for, pair_transition_forward, transition_forward

        cdt = gemm_dtype_for(x)
        op = self.operands(cdt, scale)
        if self.fused_pair:
            kernel_census.record("TransitionBlock", "hip_pair_transition")
            return pair_transition_forward(
                x, op["lnw"], op["lnb"], self.norm.eps, op["w1"], op["w2"], out=out, accumulate=accumulate, s2p=s2p
            )
        if self.c == 256 and self.n == 4 and x.dtype == torch.bfloat16 and cdt == torch.bfloat16 and s2p is None:
            # the fused 256-channel kernel (hidden activations kept on chip)
            kernel_census.record("TransitionBlock", "hip_pair_transition")
            return pair_transition_forward(
                x, op["lnw"], op["lnb"], self.norm.eps, op["w1"], op["w2"], out=out, accumulate=accumulate
            )
        if s2p is not None:
            raise ValueError("the single_to_pair epilogue is fused only into the C=128 pair transition")
        kernel_census.record("TransitionBlock", "hip_transition")
        return transition_forward(x, op["lnw"], op["lnb"], self.norm.eps, op["w1"], op["w2"], out, accumulate), None

    def _forward_grad(self, x: torch.Tensor, scale: float) -> torch.Tensor:
        """Training path, the reference's fused transition's structure (``fused_transition.py:34-83``:
        LN + linear1, SwiGLU, linear2): the HIP LayerNorm and SwiGLU with their backward, the
        two linears as library GEMMs in autograd (``token_linear``: split-K weight gradients
        over a pair's tokens), ``scale`` on linear2."""
        from .kernels import SwiGLUFunction, layer_norm_for_gemm, token_linear

        xn = layer_norm_for_gemm(x, self.norm.weight, self.norm.bias, self.norm.eps)
        w2 = self.linear2.weight if scale == 1.0 else self.linear2.weight * scale
        return token_linear(SwiGLUFunction.apply(token_linear(xn, self.linear1.weight)), w2)

    def _update(self, x: torch.Tensor, scale: float) -> torch.Tensor:
        if torch.is_grad_enabled():
            from . import kernel_census

            kernel_census.record("TransitionBlock", "hip_transition_grad")
            return self._forward_grad(x, scale)
        return self.run(x, scale=scale)[0]

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        """``transition(x)`` (not added to x); under grad the differentiable path."""
        return self._update(x, 1.0)

    def branch(self, x: torch.Tensor) -> torch.Tensor:
        """``branch_scale * transition(x)``, the update a block adds (out of place)."""
        return self._update(x, self.branch_scale)

    def forward_residual_(self, x: torch.Tensor, s2p=None):
        """``x += branch_scale * transition(x)`` in place; returns ``(x, pair_logits or None)``."""
        return self.run(x, out=x, accumulate=True, s2p=s2p, scale=self.branch_scale)


def make_transition_block(
    channels: int, num_intermediate_factor: int = 4, config=None, linear_out_init_gain: float | None = None
):
    """Reference factory (``optim.py:50-105``): one implementation here, the HIP one."""
    return TransitionBlock(channels, num_intermediate_factor, optim=config, linear_out_init_gain=linear_out_init_gain)
