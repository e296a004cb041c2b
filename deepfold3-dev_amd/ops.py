"""Triangle multiplicative update modules on the HIP kernels.

``TriangleMulOutgoing`` / ``TriangleMulIncoming`` keep the reference's
parameters, state-dict keys and ``forward(z, mask)`` signature
(``src/deepfold3/model/ops.py:179-231``, ``:645-680``); the forward is the
three-launch HIP triangle multiply (K1 project, K2 per-channel MFMA GEMM, K3
output), see ``csrc/trimul.hip``; under grad, ``FusedTriMulFunction`` with the VJP
kernels of ``csrc/trimul_bwd.hip``. Multi-head routed (MHR) variants are not built
and refuse at construction.
"""

from __future__ import annotations

import torch
import torch.nn as nn

from . import kernel_census
from .config import OptimConfig, require_hip
from .inference_guard import NotActive, inference_only
from .kernels import (
    FusedTriMulFunction,
    cast_weight,
    gemm_dtype_for,
    layer_norm_for_gemm,
    pack_trimul_weights,
    scaled_weight,
    trimul_forward,
)
from .primitives import LayerNorm, LinearNoBias, WeightCache


class _TriangleMulBase(nn.Module):
    _outgoing: bool

    def __init__(
        self,
        c_z: int,
        optim: OptimConfig | None = None,
        num_heads: int = 0,
        head_norm: str = "channel",
        router: bool = False,
        router_kind: str = "softmax",
    ):
        super().__init__()
        site = "TriangleMul"
        if num_heads or head_norm != "channel" or router:
            raise NotActive(site, "multi-head routed triangle multiplication is not built")
        require_hip(site, optim)
        self.norm_left = LayerNorm(c_z)
        self.proj = LinearNoBias(c_z, c_z * 2)
        self.gate = LinearNoBias(c_z, c_z * 2, initializer="zeros")
        self.norm_center = LayerNorm(c_z)
        self.out_proj = LinearNoBias(c_z, c_z, initializer="zeros")
        self.out_gate = LinearNoBias(c_z, c_z, initializer="zeros")
        even, odd = torch.arange(0, 2 * c_z, 2), torch.arange(1, 2 * c_z, 2)
        # Interleaved a/b (ops.py:449-450) -> block order; incoming swaps a and b so the
        # contraction stays P Q^T on transposed planes (ops.py:285-288).
        self._block_order = torch.cat((even, odd)) if self._outgoing else torch.cat((odd, even))
        self._cache = WeightCache()
        # Residual scale of this branch (the block's ``s_ros``), folded into out_proj.
        self.branch_scale = 1.0

    def _operands(self, cdt: torch.dtype, scale: float = 1.0):
        params = [
            self.norm_left.weight, self.norm_left.bias, self.proj.weight, self.gate.weight,
            self.norm_center.weight, self.norm_center.bias, self.out_proj.weight, self.out_gate.weight,
        ]  # fmt: skip

        def build():
            order = self._block_order.to(self.proj.weight.device)
            f32 = lambda t: t.detach().to(torch.float32).contiguous()  # noqa: E731
            return dict(
                packed=pack_trimul_weights(self.proj.weight[order], self.gate.weight[order], cdt),
                w_out=scaled_weight(self.out_proj.weight, scale, cdt),
                w_out_gate=cast_weight(self.out_gate.weight, cdt),
                lniw=f32(self.norm_left.weight), lnib=f32(self.norm_left.bias),
                lnow=f32(self.norm_center.weight), lnob=f32(self.norm_center.bias),
            )  # fmt: skip

        return self._cache.get(params, cdt, build, tag=float(scale))

    def _run(self, z: torch.Tensor, mask: torch.Tensor, out: torch.Tensor | None, accumulate: bool,
             scale: float = 1.0) -> torch.Tensor:  # fmt: skip
        kernel_census.record("TriangleMul", "hip_trimul")
        op = self._operands(gemm_dtype_for(z), scale)
        return trimul_forward(
            z, mask, op["lniw"], op["lnib"], self.norm_left.eps, op["packed"], op["lnow"], op["lnob"],
            self.norm_center.eps, op["w_out"], op["w_out_gate"], self._outgoing, out=out, accumulate=accumulate,
        )  # fmt: skip

    def _forward_grad(self, z: torch.Tensor, mask: torch.Tensor, scale: float) -> torch.Tensor:
        """Training path (``ops.py:375-388``): ``norm_left`` (the HIP LayerNorm and its backward),
        then the HIP ``FusedTriMulFunction`` with its VJP kernels; ``scale`` on out_proj."""
        nl = self.norm_left
        x = layer_norm_for_gemm(z, nl.weight, nl.bias, nl.eps)
        order = self._block_order.to(z.device)
        w_out = self.out_proj.weight if scale == 1.0 else self.out_proj.weight * scale
        return FusedTriMulFunction.apply(
            x.contiguous(), mask, self.gate.weight[order], self.proj.weight[order], self.norm_center.weight,
            self.norm_center.bias, w_out, self.out_gate.weight, self.norm_center.eps, self._outgoing,
        )  # fmt: skip

    def _update(self, z: torch.Tensor, mask: torch.Tensor, scale: float) -> torch.Tensor:
        has_batch = z.dim() == 4
        if not has_batch:
            z, mask = z.unsqueeze(0), mask.unsqueeze(0)
        if torch.is_grad_enabled():
            out = self._forward_grad(z, mask, scale)
        else:
            out = self._run(z, mask, None, False, scale)
        return out if has_batch else out.squeeze(0)

    def forward(self, z: torch.Tensor, mask: torch.Tensor) -> torch.Tensor:
        """The update for z [B?, N, N, C] and mask [B?, N, N] (not added to z). Under grad it
        runs the differentiable path (``FusedTriMulFunction``), else the inference kernels."""
        return self._update(z, mask, 1.0)

    def branch(self, z: torch.Tensor, mask: torch.Tensor) -> torch.Tensor:
        """``branch_scale * forward(z, mask)``: the update as its block adds it (out of place)."""
        return self._update(z, mask, self.branch_scale)

    @inference_only("TriangleMul")
    def forward_residual_(self, z: torch.Tensor, mask: torch.Tensor) -> torch.Tensor:
        """``z += branch_scale * update`` in place (fused into K3); z must be contiguous [B, N, N, C]."""
        if not z.is_contiguous():
            raise NotActive("TriangleMul", "in-place residual needs a contiguous z")
        return self._run(z, mask, z, True, self.branch_scale)


class TriangleMulOutgoing(_TriangleMulBase):
    """Triangle multiplication, outgoing: ``X_ij = sum_k a_ik b_jk`` (``ops.py:665-671``)."""

    _outgoing = True


class TriangleMulIncoming(_TriangleMulBase):
    """Triangle multiplication, incoming: ``X_ij = sum_k a_kj b_ki`` (``ops.py:674-680``)."""

    _outgoing = False


class OuterProductMean(nn.Module):
    """MSA -> pair update of the Evoformer block (``ops.py:683-785``): ``a, b`` = two
    projections of LN(msa) times the mask, the outer product ``a[s,i] (x) b[s,j]`` summed over
    the sequences, contracted with ``out_w`` [CH, CH, c_z] plus ``out_b``, divided by
    ``1e-3 +`` the number of sequences holding both residues. Same parameter names as the
    reference (``norm``, ``proj_a``, ``proj_b``, ``out_w``, ``out_b``)."""

    def __init__(self, c_msa: int, c_z: int, c_hidden: int = 32, optim: OptimConfig | None = None):
        super().__init__()
        require_hip("OuterProductMean", optim)
        self.norm = LayerNorm(c_msa)
        self.proj_a = LinearNoBias(c_msa, c_hidden)
        self.proj_b = LinearNoBias(c_msa, c_hidden)
        self.out_w = nn.Parameter(torch.zeros(c_hidden, c_hidden, c_z))  # AF3 final init (zeros)
        self.out_b = nn.Parameter(torch.zeros(c_z))
        self._cache = WeightCache()
        # Residual scale of this branch inside its block (the block's s_ros), folded into out_w
        # and out_b by ``forward_residual_``; ``forward`` is unscaled.
        self.branch_scale = 1.0

    def _operands(self, cdt: torch.dtype, scale: float = 1.0) -> dict:
        from .kernels import cast_weight

        params = [self.norm.weight, self.norm.bias, self.proj_a.weight, self.proj_b.weight, self.out_w, self.out_b]

        def build():
            ch, _, cz = self.out_w.shape
            w_out = self.out_w.detach().to(torch.float32).permute(2, 0, 1).reshape(cz, ch * ch) * scale
            return dict(
                w_ab=cast_weight(torch.cat([self.proj_a.weight, self.proj_b.weight]).detach(), cdt),
                w_out=cast_weight(w_out.contiguous(), cdt),
                b_out=(self.out_b.detach().to(torch.float32) * scale).contiguous(),
                lnw=self.norm.weight.detach().to(torch.float32).contiguous(),
                lnb=self.norm.bias.detach().to(torch.float32).contiguous(),
            )

        return self._cache.get(params, cdt, build, tag=float(scale))

    def _run(self, msa, mask, out, accumulate, scale: float = 1.0):
        from .kernels import outer_product_mean_forward

        kernel_census.record("OuterProductMean", "hip_outer_product_mean")
        op = self._operands(gemm_dtype_for(msa), scale)
        return outer_product_mean_forward(
            msa, mask, op["lnw"], op["lnb"], self.norm.eps, op["w_ab"], op["w_out"], op["b_out"], out=out,
            accumulate=accumulate,
        )  # fmt: skip

    @inference_only("OuterProductMean")
    def forward(self, msa: torch.Tensor, mask: torch.Tensor) -> torch.Tensor:
        """msa [B?, S, N, c_msa], mask [B?, S, N] -> [B?, N, N, c_z] (not added to the pair)."""
        has_batch = msa.dim() == 4
        if not has_batch:
            msa, mask = msa.unsqueeze(0), mask.unsqueeze(0)
        out = self._run(msa, mask, None, False, 1.0)
        return out if has_batch else out.squeeze(0)

    @inference_only("OuterProductMean")
    def forward_residual_(self, pair: torch.Tensor, msa: torch.Tensor, mask: torch.Tensor) -> torch.Tensor:
        """``pair += branch_scale * update`` in place; pair contiguous [B, N, N, c_z] in msa's dtype."""
        if not pair.is_contiguous():
            raise NotActive("OuterProductMean", "in-place residual needs a contiguous pair")
        return self._run(msa, mask, pair, True, self.branch_scale)
