"""Triangle multiplicative update modules on the HIP kernels.

``TriangleMulOutgoing`` / ``TriangleMulIncoming`` keep the reference's
parameters, state-dict keys and ``forward(z, mask)`` signature
(``src/deepfold3/model/ops.py:179-231``, ``:645-680``); the forward is the
three-launch HIP triangle multiply (K1 project, K2 per-channel MFMA GEMM, K3
output), see ``csrc/trimul.hip``; under grad, ``FusedTriMulFunction`` with the VJP
kernels of ``csrc/trimul_bwd.hip``. The multi-head routed (MHR) variants
(``num_heads`` > 0 with a per-head norm and / or the router, ``ops.py:179-345``) run the
same launches with the head mix of ``csrc/mhr.h`` in K3 and in the output VJP.
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
    MHR_HEAD_NORMS,
    MHR_ROUTER_KINDS,
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
        # MHR arguments and their errors as the reference's (ops.py:227-255)
        if head_norm not in MHR_HEAD_NORMS:
            raise ValueError(f"head_norm must be channel|head_rms|head_ln|post_channel, got {head_norm!r}")
        if head_norm == "post_channel" and not router:
            raise ValueError("head_norm='post_channel' is meaningless without router=True")
        if router_kind not in MHR_ROUTER_KINDS:
            raise ValueError(f"router_kind must be softmax|sigmoid, got {router_kind!r}")
        if head_norm != "channel" or router:
            if num_heads <= 0:
                raise ValueError("num_heads > 0 is required for per-head norm or routing")
            if c_z % num_heads:
                raise ValueError(f"c_z={c_z} must be divisible by num_heads={num_heads}")
        require_hip(site, optim)
        self.norm_left = LayerNorm(c_z)
        self.proj = LinearNoBias(c_z, c_z * 2)
        self.gate = LinearNoBias(c_z, c_z * 2, initializer="zeros")
        # head_rms is RMSNorm proper: norm_center keeps its gain and has no shift (ops.py:219-224)
        self.norm_center = LayerNorm(c_z, bias=head_norm != "head_rms")
        self.out_proj = LinearNoBias(c_z, c_z, initializer="zeros")
        self.out_gate = LinearNoBias(c_z, c_z, initializer="zeros")
        self.num_heads = int(num_heads)
        self.head_dim = c_z // num_heads if num_heads else 0
        self.head_norm = head_norm
        self.use_router = bool(router)
        self.router_kind = router_kind
        self.is_mhr = head_norm != "channel" or self.use_router
        # zero-initialised router: g = 1, the module starts as the plain triangle multiply
        self.router = LinearNoBias(c_z, num_heads, initializer="zeros") if self.use_router else None
        self._router_stats: dict[str, float] | None = None
        self.router_stats_enabled = False
        even, odd = torch.arange(0, 2 * c_z, 2), torch.arange(1, 2 * c_z, 2)
        # Interleaved a/b (ops.py:449-450) -> block order; incoming swaps a and b so the
        # contraction stays P Q^T on transposed planes (ops.py:285-288).
        self._block_order = torch.cat((even, odd)) if self._outgoing else torch.cat((odd, even))
        self._cache = WeightCache()
        # Residual scale of this branch (the block's ``s_ros``), folded into out_proj.
        self.branch_scale = 1.0

    def _mix_codes(self) -> tuple[int, int, int] | None:
        """(num_heads, head_norm, router_kind) as the C-ABI's codes for an MHR module, else None."""
        if not self.is_mhr:
            return None
        return self.num_heads, MHR_HEAD_NORMS[self.head_norm], MHR_ROUTER_KINDS[self.router_kind]

    def _operands(self, cdt: torch.dtype, scale: float = 1.0):
        params = [
            self.norm_left.weight, self.norm_left.bias, self.proj.weight, self.gate.weight,
            self.norm_center.weight, self.norm_center.bias, self.out_proj.weight, self.out_gate.weight,
            None if self.router is None else self.router.weight,
        ]  # fmt: skip

        def build():
            order = self._block_order.to(self.proj.weight.device)
            f32 = lambda t: None if t is None else t.detach().to(torch.float32).contiguous()  # noqa: E731
            return dict(
                packed=pack_trimul_weights(self.proj.weight[order], self.gate.weight[order], cdt),
                w_out=scaled_weight(self.out_proj.weight, scale, cdt),
                w_out_gate=cast_weight(self.out_gate.weight, cdt),
                lniw=f32(self.norm_left.weight), lnib=f32(self.norm_left.bias),
                lnow=f32(self.norm_center.weight), lnob=f32(self.norm_center.bias),
                w_router=None if self.router is None else f32(self.router.weight),
            )  # fmt: skip

        return self._cache.get(params, cdt, build, tag=float(scale))

    def _run(self, z: torch.Tensor, mask: torch.Tensor, out: torch.Tensor | None, accumulate: bool,
             scale: float = 1.0) -> torch.Tensor:  # fmt: skip
        kernel_census.record("TriangleMul", "hip_trimul_mhr" if self.is_mhr else "hip_trimul")
        op = self._operands(gemm_dtype_for(z), scale)
        codes = self._mix_codes()
        mix = None if codes is None else (codes[0], codes[1], op["w_router"], codes[2])
        if self.router_stats_enabled and self.use_router:
            self._record_router_stats(self._router_gates(z))
        return trimul_forward(
            z, mask, op["lniw"], op["lnib"], self.norm_left.eps, op["packed"], op["lnow"], op["lnob"],
            self.norm_center.eps, op["w_out"], op["w_out_gate"], self._outgoing, out=out, accumulate=accumulate,
            mix=mix,
        )  # fmt: skip

    def _forward_grad(self, z: torch.Tensor, mask: torch.Tensor, scale: float) -> torch.Tensor:
        """Training path (``ops.py:375-388``): ``norm_left`` (the HIP LayerNorm and its backward),
        then the HIP ``FusedTriMulFunction`` with its VJP kernels (and the MHR mix); ``scale`` on
        out_proj."""
        nl = self.norm_left
        x = layer_norm_for_gemm(z, nl.weight, nl.bias, nl.eps)
        order = self._block_order.to(z.device)
        w_out = self.out_proj.weight if scale == 1.0 else self.out_proj.weight * scale
        if self.router_stats_enabled and self.use_router:
            self._record_router_stats(self._router_gates(z))
        return FusedTriMulFunction.apply(
            x.contiguous(), mask, self.gate.weight[order], self.proj.weight[order], self.norm_center.weight,
            self.norm_center.bias, w_out, self.out_gate.weight, self.norm_center.eps, self._outgoing,
            None if self.router is None else self.router.weight, self._mix_codes(),
        )  # fmt: skip

    # ---- router read-out (ops.py:548-640): detached statistics of the gates, off by default

    @torch.no_grad()
    def _router_gates(self, z: torch.Tensor) -> torch.Tensor:
        """The router's gates g [.., H] (fp32) for z, as the K3 kernel forms them."""
        nl = self.norm_left
        x = layer_norm_for_gemm(z, nl.weight, nl.bias, nl.eps)
        r = F.linear(x.float(), self.router.weight.float())
        h = self.num_heads
        return float(h) * torch.softmax(r, dim=-1) if self.router_kind == "softmax" else 2.0 * torch.sigmoid(r)

    @torch.no_grad()
    def _record_router_stats(self, g: torch.Tensor) -> None:
        """Accumulate the window's entropy, marginal entropy, g's rms / across-pair std / mean and
        head occupancy (shares p = g / sum_h g), as ``_record_router_stats`` (``ops.py:548-620``)."""
        g = g.reshape(-1, self.num_heads)
        p = g / g.sum(-1, keepdim=True).clamp_min(1e-9)
        ent = -(p * (p + 1e-9).log()).sum(-1).mean() / math.log(self.num_heads)
        share = p.mean(0)
        marg = -(share * (share + 1e-9).log()).sum() / math.log(self.num_heads)
        acc = self._router_stats
        if acc is None:
            keys = ("entropy", "marginal_entropy", "g_rms", "g_std", "g_mean", "occupancy_max", "occupancy_min", "n")
            acc = self._router_stats = dict.fromkeys(keys, 0.0)
        acc["entropy"] += float(ent)
        acc["marginal_entropy"] += float(marg)
        acc["g_rms"] += float(g.pow(2).mean(-1).sqrt().mean())
        acc["g_std"] += float(g.std(0).mean())
        acc["g_mean"] += float(g.mean())
        acc["occupancy_max"] += float(share.max())
        acc["occupancy_min"] += float(share.min())
        acc["n"] += 1.0

    def _flush_router_stats(self, reset: bool = True) -> dict[str, float] | None:
        """Window means of the accumulated read-out, or None if nothing ran (``ops.py:622-632``)."""
        acc = self._router_stats
        if acc is None or acc["n"] == 0:
            return None
        n = acc["n"]
        out = {k: v / n for k, v in acc.items() if k != "n"}
        if reset:
            self._router_stats = None
        return out

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
