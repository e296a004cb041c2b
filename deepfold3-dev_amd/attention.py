"""Triangle attention and single attention with pair bias on the HIP kernels.

``GridSelfAttention`` (row: ``transpose=False``, starting node; column:
``transpose=True``, ending node) and ``SingleAttention`` keep the reference's
parameters, state-dict keys and ``forward`` signatures
(``src/deepfold3/model/attention.py:56-104``, ``:344-452``). The forward is the
three-launch HIP triangle attention (``csrc/attention.hip``: LN + fused q/k/v/g/pair-bias
projection, flash attention with an online softmax, gated output projection) and the
single-track kernels (``csrc/single.hip``).
"""

from __future__ import annotations

import math

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import kernel_census
from .config import OptimConfig, require_hip
from .inference_guard import NotActive, inference_only
from .kernels import (
    cast_weight,
    gemm_dtype_for,
    grid_attention_forward,
    pack_grid_attn_weights,
    scaled_weight,
    single_attention_forward,
)
from .primitives import LayerNorm, LinearNoBias, WeightCache, f32


class GridSelfAttention(nn.Module):
    """Gated self-attention along rows (starting node) or columns (ending node) of z."""

    def __init__(self, c: int, num_heads: int = 4, transpose: bool = False, optim: OptimConfig | None = None):
        super().__init__()
        assert c % num_heads == 0
        require_hip("GridSelfAttention", optim)
        self.num_heads = num_heads
        self.head_dim = max(c // num_heads, 16)  # attention.py:67
        self.transpose = transpose
        self.scale = self.head_dim**-0.5
        self.norm = LayerNorm(c)
        self.pair_bias = LinearNoBias(c, num_heads)
        self.to_q = LinearNoBias(c, num_heads * self.head_dim)
        self.to_k = LinearNoBias(c, num_heads * self.head_dim)
        self.to_v = LinearNoBias(c, num_heads * self.head_dim)
        self.to_g = LinearNoBias(c, num_heads * self.head_dim, initializer="zeros")
        self.out_proj = LinearNoBias(num_heads * self.head_dim, c, initializer="zeros")
        self._cache = WeightCache()
        # Residual scale of this branch inside its block (the block's ``s_ros``), folded into
        # out_proj by ``branch`` and ``forward_residual_``; ``forward`` is unscaled.
        self.branch_scale = 1.0

    def _operands(self, cdt: torch.dtype, scale: float = 1.0) -> dict:
        params = [
            self.norm.weight, self.norm.bias, self.pair_bias.weight, self.to_q.weight, self.to_k.weight,
            self.to_v.weight, self.to_g.weight, self.out_proj.weight,
        ]  # fmt: skip

        def build():
            return dict(
                w5=pack_grid_attn_weights(
                    self.to_q.weight, self.to_k.weight, self.to_v.weight, self.to_g.weight, self.pair_bias.weight, cdt
                ),
                w_out=scaled_weight(self.out_proj.weight, scale, cdt),
                lnw=f32(self.norm.weight), lnb=f32(self.norm.bias),
            )  # fmt: skip

        return self._cache.get(params, cdt, build, tag=float(scale))

    def _run(self, z, mask, out, accumulate, scale: float = 1.0):
        kernel_census.record("GridSelfAttention.attention", "hip_tri_attn_col" if self.transpose else "hip_tri_attn_row")
        op = self._operands(gemm_dtype_for(z), scale)
        return grid_attention_forward(
            z, mask, op["lnw"], op["lnb"], self.norm.eps, op["w5"], op["w_out"], self.transpose,
            num_heads=self.num_heads, out=out, accumulate=accumulate,
        )  # fmt: skip

    def _forward_grad(self, z: torch.Tensor, mask: torch.Tensor, scale: float) -> torch.Tensor:
        """Training path, as the reference's fused-attention branch (``attention.py:211-257``):
        LayerNorm, pair bias and q/k/v/g projections in autograd, the HIP flash attention with
        its backward (the kernel's masked-row rule), gate and output projection in autograd.
        With 4 heads the attention (``fused._GridAttnCore``) reads the token-major projection
        and writes O and the gradients in that order through strides; other head counts go
        through the kernel-layout ``fused._EvoformerAttention``. Head dimension 32; ``scale`` on
        out_proj."""
        from .fused import _EvoformerAttention, _GridAttnCore

        B, N, _, C = z.shape
        H, D = self.num_heads, self.head_dim
        if D != 32:
            raise NotActive("GridSelfAttention", f"head dim {D}: the differentiable attention is built for 32")
        from .kernels import layer_norm_for_gemm, token_linear

        zn = layer_norm_for_gemm(z, self.norm.weight, self.norm.bias, self.norm.eps)
        pb = token_linear(zn, self.pair_bias.weight).permute(0, 3, 1, 2)  # [B, H, N, N], un-transposed z
        pb = pb.to(torch.float32, memory_format=torch.contiguous_format)
        line_mask = mask.transpose(1, 2) if self.transpose else mask  # [B, lines, keys]
        res_mask = torch.where(line_mask > 0.5, 0.0, -1e9).contiguous()
        w_out = self.out_proj.weight if scale == 1.0 else self.out_proj.weight * scale
        g = torch.sigmoid(token_linear(zn, self.to_g.weight))
        if H == 4:
            # q, k, v in one product over the un-transposed tokens; the attention reads them and
            # writes O (and, backward, the gradients) in that token order through strides
            w_qkv = torch.cat([self.to_q.weight, self.to_k.weight, self.to_v.weight])
            qkv = token_linear(zn, w_qkv).view(B, N, N, 3, H, D)
            o = _GridAttnCore.apply(qkv, res_mask, pb, self.transpose)
            return token_linear(o.view(B, N, N, H * D) * g, w_out)
        # other head counts: the kernel-layout op with its head groups
        w_qkv = torch.cat([self.to_q.weight, self.to_k.weight, self.to_v.weight])
        y = token_linear(zn, w_qkv).view(B, N, N, 3, H, D).unbind(3)  # backward: one stack
        frame = (0, 2, 3, 1, 4) if self.transpose else (0, 1, 3, 2, 4)  # [B, line, H, key, D]
        qkv = [t.permute(*frame).contiguous() for t in y]
        o = _EvoformerAttention.apply(*qkv, res_mask.view(B, N, 1, 1, N), pb.unsqueeze(1), True)
        back = (0, 3, 1, 2, 4) if self.transpose else (0, 1, 3, 2, 4)  # to [B, N, N, H, D]
        o = o.permute(*back).reshape(B, N, N, H * D)
        return token_linear(o * g, w_out)

    def _update(self, z: torch.Tensor, mask: torch.Tensor, scale: float) -> torch.Tensor:
        has_batch = z.dim() == 4
        if not has_batch:
            z, mask = z.unsqueeze(0), mask.unsqueeze(0)
        if torch.is_grad_enabled():
            kernel_census.record("GridSelfAttention.attention", "hip_evo_attn_grad")
            out = self._forward_grad(z, mask, scale)
        else:
            out = self._run(z, mask, None, False, scale)
        return out if has_batch else out.squeeze(0)

    def forward(self, z: torch.Tensor, mask: torch.Tensor) -> torch.Tensor:
        """The update for z [B?, N, N, C], mask [B?, N, N] (not added to z). Under grad it
        runs the differentiable path, else the fused inference kernels."""
        return self._update(z, mask, 1.0)

    def branch(self, z: torch.Tensor, mask: torch.Tensor) -> torch.Tensor:
        """``branch_scale * forward(z, mask)``: the update as its block adds it (out of place)."""
        return self._update(z, mask, self.branch_scale)

    @inference_only("GridSelfAttention")
    def forward_residual_(self, z: torch.Tensor, mask: torch.Tensor) -> torch.Tensor:
        """``z += branch_scale * update`` in place (fused into the output projection)."""
        if not z.is_contiguous():
            raise NotActive("GridSelfAttention", "in-place residual needs a contiguous z")
        return self._run(z, mask, z, True, self.branch_scale)


class MSAAttention(nn.Module):
    """MSA row update of the Evoformer block, AF3's pair-weighted averaging
    (``attention.py:272-341``): weights ``softmax_k(LN(pair) W_h + 1e9 (colmask_k - 1))``
    shared by every MSA row (colmask: any sequence holds residue k), values ``to_v(LN(msa))``,
    gate ``sigmoid(to_g(LN(msa)))``, then ``out_proj``. Same parameter names as the reference."""

    def __init__(self, c_msa: int, c_pair: int, num_heads: int = 8, optim: OptimConfig | None = None):
        super().__init__()
        require_hip("MSAAttention", optim)
        assert c_msa % num_heads == 0
        if num_heads > 16:
            raise NotActive("MSAAttention", f"num_heads={num_heads}: at most 16 heads are built")
        self.num_heads = num_heads
        self.head_dim = c_msa // num_heads
        self.norm = LayerNorm(c_msa)
        self.pair_norm = LayerNorm(c_pair)
        self.pair_logits = LinearNoBias(c_pair, num_heads)
        self.to_v = LinearNoBias(c_msa, num_heads * self.head_dim)
        self.to_g = LinearNoBias(c_msa, num_heads * self.head_dim, initializer="zeros")
        self.out_proj = LinearNoBias(num_heads * self.head_dim, c_msa, initializer="zeros")
        self._cache = WeightCache()
        # Residual scale of this branch inside its block (the block's s_ros), folded into
        # out_proj by ``branch`` and ``forward_residual_``; ``forward`` is unscaled.
        self.branch_scale = 1.0

    def _operands(self, cdt: torch.dtype, scale: float = 1.0) -> dict:
        params = [
            self.norm.weight, self.norm.bias, self.pair_norm.weight, self.pair_norm.bias, self.pair_logits.weight,
            self.to_v.weight, self.to_g.weight, self.out_proj.weight,
        ]  # fmt: skip

        def build():
            w_lg = self.pair_logits.weight.detach()
            pad = torch.zeros(16 - w_lg.shape[0], w_lg.shape[1], dtype=w_lg.dtype, device=w_lg.device)
            return dict(
                w_lg=cast_weight(torch.cat([w_lg, pad]), cdt),
                w_vg=cast_weight(torch.cat([self.to_v.weight, self.to_g.weight]).detach(), cdt),
                w_out=scaled_weight(self.out_proj.weight, scale, cdt),
                lnw=f32(self.norm.weight), lnb=f32(self.norm.bias),
                plnw=f32(self.pair_norm.weight), plnb=f32(self.pair_norm.bias),
            )  # fmt: skip

        return self._cache.get(params, cdt, build, tag=float(scale))

    def _run(self, msa, mask, pair, out, accumulate, scale: float = 1.0):
        from .kernels import msa_pair_avg_forward

        kernel_census.record("MSAAttention", "hip_msa_pair_avg")
        op = self._operands(gemm_dtype_for(msa), scale)
        return msa_pair_avg_forward(
            msa, mask, pair, op["lnw"], op["lnb"], self.norm.eps, op["plnw"], op["plnb"], self.pair_norm.eps,
            op["w_lg"], op["w_vg"], op["w_out"], self.num_heads, out=out, accumulate=accumulate,
        )  # fmt: skip

    @inference_only("MSAAttention")
    def forward(self, msa: torch.Tensor, mask: torch.Tensor, pair: torch.Tensor) -> torch.Tensor:
        """msa [B?, S, N, c_msa], mask [B?, S, N], pair [B?, N, N, c_pair] -> the msa update."""
        return self._update(msa, mask, pair, 1.0)

    @inference_only("MSAAttention")
    def branch(self, msa: torch.Tensor, mask: torch.Tensor, pair: torch.Tensor) -> torch.Tensor:
        """``branch_scale * forward(msa, mask, pair)``: the update as its block adds it."""
        return self._update(msa, mask, pair, self.branch_scale)

    def _update(self, msa, mask, pair, scale):
        has_batch = msa.dim() == 4
        if not has_batch:
            msa, mask, pair = msa.unsqueeze(0), mask.unsqueeze(0), pair.unsqueeze(0)
        out = self._run(msa, mask, pair, None, False, scale)
        return out if has_batch else out.squeeze(0)

    @inference_only("MSAAttention")
    def forward_residual_(self, msa: torch.Tensor, mask: torch.Tensor, pair: torch.Tensor) -> torch.Tensor:
        """``msa += branch_scale * update`` in place; msa contiguous [B, S, N, c_msa]."""
        if not msa.is_contiguous():
            raise NotActive("MSAAttention", "in-place residual needs a contiguous msa")
        return self._run(msa, mask, pair, msa, True, self.branch_scale)


class SingleAttention(nn.Module):
    """Self-attention on the single track with pair-logit bias (``attention.py:344-452``)."""

    def __init__(
        self,
        c: int,
        num_heads: int = 16,
        key_dim: int = 384,
        value_dim: int = 384,
        optim: OptimConfig | None = None,
        pair_bias_gate: bool = False,
        pair_bias_gate_init_tau: float = 0.25,
    ):
        super().__init__()
        require_hip("SingleAttention", optim)
        if key_dim != value_dim or key_dim != c or key_dim // num_heads != 24:
            raise NotActive("SingleAttention", "built for key_dim = value_dim = c with head dim 24")
        self.num_heads = num_heads
        self.key_dim_per_head = key_dim // num_heads
        self.val_dim_per_head = value_dim // num_heads
        self.scale = self.key_dim_per_head**-0.5
        self.norm = LayerNorm(c)
        # Per-head pair-bias gate (attention.py:392-398): tau_h = exp(a_h) scales head h's pair
        # logits, a_h starting at log(tau_0).
        if pair_bias_gate:
            if not pair_bias_gate_init_tau > 0.0:
                raise ValueError(f"pair_bias_gate_init_tau={pair_bias_gate_init_tau}: tau_0 must be positive")
            self.pair_bias_gate_a = nn.Parameter(torch.full((num_heads,), math.log(float(pair_bias_gate_init_tau))))
        else:
            self.register_parameter("pair_bias_gate_a", None)
        self.to_q = nn.Linear(c, key_dim)
        from .primitives import af3_linear_init_

        af3_linear_init_(self.to_q.weight, "linear")
        nn.init.zeros_(self.to_q.bias)
        self.to_k = LinearNoBias(c, key_dim)
        self.to_v = LinearNoBias(c, value_dim)
        self.to_g = LinearNoBias(c, value_dim, initializer="zeros")
        self.out_proj = LinearNoBias(value_dim, c, initializer="zeros")
        self._cache = WeightCache()
        # Residual scale of this branch inside its block (the block's ``s_ros``), folded into
        # out_proj by ``branch`` and ``forward_residual_``; ``forward`` is unscaled.
        self.branch_scale = 1.0

    def _operands(self, cdt: torch.dtype, scale: float = 1.0) -> dict:
        params = [
            self.norm.weight, self.norm.bias, self.to_q.weight, self.to_q.bias, self.to_k.weight, self.to_v.weight,
            self.to_g.weight, self.out_proj.weight,
        ]  # fmt: skip

        def build():
            w = torch.cat([self.to_q.weight, self.to_k.weight, self.to_v.weight, self.to_g.weight]).detach()
            return dict(
                wqkvg=cast_weight(w, cdt), w_out=scaled_weight(self.out_proj.weight, scale, cdt),
                qb=f32(self.to_q.bias), lnw=f32(self.norm.weight), lnb=f32(self.norm.bias),
            )  # fmt: skip

        return self._cache.get(params, cdt, build, tag=float(scale))

    def _run(self, x, mask, pair_logits, out, accumulate, scale: float = 1.0):
        kernel_census.record("SingleAttention", "hip_single_attn")
        op = self._operands(gemm_dtype_for(x), scale)
        return single_attention_forward(
            x, mask, pair_logits, op["lnw"], op["lnb"], self.norm.eps, op["wqkvg"], op["qb"], op["w_out"],
            self.num_heads, out=out, accumulate=accumulate,
        )  # fmt: skip

    def _forward_grad(self, x: torch.Tensor, mask: torch.Tensor, pair_logits: torch.Tensor, scale: float) -> torch.Tensor:
        """Training path: LayerNorm (HIP, with its backward), the q/k/v/g projections and the output
        projection in autograd, and the attention core on the HIP flash attention with its
        backward (``fused._EvoformerAttention``; one line per batch item, the heads' key and value
        dimensions zero-padded to 32 and q scaled so that the kernel's 32^-1/2 gives d^-1/2,
        ``attention.py:415-433``), under the eager masked-row rule in both passes, as the stock
        softmax: a batch item whose keys are all masked attends uniformly."""
        from .fused import _EvoformerAttention
        from .kernels import LayerNormFunction

        B, N, _ = x.shape
        H, Dk, Dv = self.num_heads, self.key_dim_per_head, self.val_dim_per_head
        if Dk > 32 or Dv > 32:
            raise NotActive("SingleAttention", f"head dims {Dk}/{Dv}: the differentiable attention takes up to 32")
        xn = LayerNormFunction.apply(x, self.norm.weight, self.norm.bias, self.norm.eps)
        q = F.linear(xn, self.to_q.weight, self.to_q.bias) * (Dk**-0.5 * 32**0.5)

        def heads(t: torch.Tensor, d: int) -> torch.Tensor:  # [B, N, H d] -> [B, 1, H, N, 32]
            t = t.reshape(B, N, H, d).transpose(1, 2)
            if d < 32:
                t = F.pad(t, (0, 32 - d))
            return t.unsqueeze(1).contiguous()

        Q, K, V = heads(q, Dk), heads(F.linear(xn, self.to_k.weight), Dk), heads(F.linear(xn, self.to_v.weight), Dv)
        res_mask = (1e9 * (mask.float() - 1.0)).view(B, 1, 1, 1, N)
        # the stock path's rule for a batch item whose keys are all masked: uniform weights
        o = _EvoformerAttention.apply(Q, K, V, res_mask, pair_logits.float().unsqueeze(1), True, "eager")
        o = o[:, 0, :, :, :Dv].transpose(1, 2).reshape(B, N, H * Dv)
        g = torch.sigmoid(F.linear(xn, self.to_g.weight))
        w_out = self.out_proj.weight if scale == 1.0 else self.out_proj.weight * scale
        return F.linear(o * g, w_out)

    def _gated(self, pair_logits: torch.Tensor) -> torch.Tensor:
        """Head h's pair logits times tau_h = exp(a_h) in their dtype (``attention.py:422-424``);
        differentiable in a under grad. Without the gate, the logits themselves."""
        if self.pair_bias_gate_a is None:
            return pair_logits
        H = self.num_heads
        tau = torch.exp(self.pair_bias_gate_a).to(pair_logits.dtype)
        return pair_logits * tau.view(*([1] * (pair_logits.dim() - 3)), H, 1, 1)

    def _update(self, x, mask, pair_logits, scale: float) -> torch.Tensor:
        pair_logits = self._gated(pair_logits)
        has_batch = x.dim() == 3
        if not has_batch:
            x, mask, pair_logits = x.unsqueeze(0), mask.unsqueeze(0), pair_logits.unsqueeze(0)
        if torch.is_grad_enabled():
            kernel_census.record("SingleAttention", "hip_evo_attn_grad")
            out = self._forward_grad(x, mask, pair_logits, scale)
        else:
            out = self._run(x, mask, pair_logits, None, False, scale)
        return out if has_batch else out.squeeze(0)

    def forward(self, x: torch.Tensor, mask: torch.Tensor, pair_logits: torch.Tensor) -> torch.Tensor:
        """x [B?, N, c], mask [B?, N], pair_logits [B?, H, N, N] -> update [B?, N, c]. Under grad
        the differentiable path."""
        return self._update(x, mask, pair_logits, 1.0)

    def branch(self, x: torch.Tensor, mask: torch.Tensor, pair_logits: torch.Tensor) -> torch.Tensor:
        """``branch_scale * forward(x, mask, pair_logits)``: the update as its block adds it."""
        return self._update(x, mask, pair_logits, self.branch_scale)

    @inference_only("SingleAttention")
    def forward_residual_(self, x: torch.Tensor, mask: torch.Tensor, pair_logits: torch.Tensor) -> torch.Tensor:
        """``x += branch_scale * update`` in place."""
        if not x.is_contiguous():
            raise NotActive("SingleAttention", "in-place residual needs a contiguous x")
        return self._run(x, mask, self._gated(pair_logits), x, True, self.branch_scale)
