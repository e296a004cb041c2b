"""PairFormer block and trunk on the HIP kernels.

``PairFormerBlock`` keeps the reference's constructor arguments, submodule names
(so state dicts load unchanged) and ``forward(pair, single, pair_mask, seq_mask)``
signature (``src/deepfold3/model/evoformer.py:178-355``). The branch scaler is the identity;
``residual_out_scale`` and the transitions' residual gains are folded into each branch's
output projection. In eval mode dropout-add is a plain add (``triton/dropout_add.py:236-237``),
so every residual add is fused into the epilogue of the kernel that produces the branch; in
training mode the four dropped pair branches (triangle multiplications and attention) add
through the HIP shared-mask dropout-add (``csrc/dropout.hip``), with grad or without.
``single_to_pair`` is fused into the pair transition's epilogue (it normalises the updated
pair rows).

``PairFormerStack`` is the trunk loop (``evoformer.py:593-601``): it copies the inputs
once and then updates them in place, block after block.
"""

from __future__ import annotations

from functools import partial

import torch
import torch.nn as nn
from torch.utils.checkpoint import checkpoint as _torch_checkpoint

from . import kernel_census
from .attention import GridSelfAttention, SingleAttention
from .config import OptimConfig, require_hip
from .inference_guard import NotActive, inference_only
from .kernels import (
    DropoutAddFunction,
    dropout_add,
    gemm_dtype_for,
    next_dropout_seed,
    rms_residual_add,
    single_to_pair,
)
from .ops import TriangleMulIncoming, TriangleMulOutgoing
from .primitives import LayerNorm, LinearNoBias, WeightCache, f32, make_transition_block

# Per-block activation checkpointing as the reference's trunk loop (``evoformer.py:58``).
_checkpoint = partial(_torch_checkpoint, use_reentrant=False, determinism_check="none")


def _dropout_residual_(module, pair: torch.Tensor, mask: torch.Tensor, p: float, rowwise: bool) -> None:
    """``pair += dropout(module.branch(pair, mask))`` in place: the eval-mode fused residual
    epilogue when ``p == 0``, else the branch out of place and the HIP shared-mask dropout-add
    (``dropout_add.py:221-265``) writing back into ``pair``."""
    if p > 0.0:
        dropout_add(pair, module.branch(pair, mask), p, rowwise, next_dropout_seed(), out=pair)
    else:
        module.forward_residual_(pair, mask)


class PairFormerBlock(nn.Module):
    """One PairFormer layer (AF3 ``PairFormerIteration``), with the single track unless
    ``use_single_track=False`` and with triangle attention unless ``use_triangle_attention=False``
    (the reference's deletable branches, ``evoformer.py:226-236``, ``:302-321``, ``:353``)."""

    def __init__(
        self,
        c_pair: int,
        c_single: int,
        num_pair_heads: int = 4,
        num_single_heads: int = 16,
        single_key_dim: int = 384,
        single_value_dim: int = 384,
        pair_dropout: float = 0.25,
        optim: OptimConfig | None = None,
        residual_out_scale: float = 1.0,
        pair_bias_gate: bool = False,
        pair_bias_gate_init_tau: float = 0.25,
        single_transition_linear_out_init_gain: float | None = None,
        single_transition_residual_gain: float | None = None,
        pair_transition_residual_gain: float | None = None,
        branch_scaler: str = "identity",
        use_triangle_attention: bool = True,
        use_single_track: bool = True,
        trimul_kwargs: dict | None = None,
    ):
        super().__init__()
        require_hip("PairFormerBlock", optim)
        if branch_scaler not in ("identity", "rmsnorm"):
            raise NotActive("PairFormerBlock", f"branch_scaler={branch_scaler!r}: identity and rmsnorm are built")
        if branch_scaler != "identity" and (
            single_transition_residual_gain is not None or pair_transition_residual_gain is not None
        ):
            # config.py:252-269: unit-RMS branches make branch-specific gains a rescaled block gamma
            raise ValueError(f"branch_scaler={branch_scaler!r} takes no per-transition residual gains")
        tk = trimul_kwargs or {}
        self.tri_mul_out = TriangleMulOutgoing(c_pair, optim=optim, **tk)
        self.tri_mul_in = TriangleMulIncoming(c_pair, optim=optim, **tk)
        self.use_triangle_attention = bool(use_triangle_attention)
        if self.use_triangle_attention:
            self.pair_attn_row = GridSelfAttention(c_pair, num_heads=num_pair_heads, transpose=False, optim=optim)
            self.pair_attn_col = GridSelfAttention(c_pair, num_heads=num_pair_heads, transpose=True, optim=optim)
        self.pair_transition = make_transition_block(c_pair, config=optim)
        # The single track reads the pair representation through the pair logits and never
        # writes back, so deleting it leaves the pair update unchanged.
        self.use_single_track = bool(use_single_track)
        if self.use_single_track:
            self.single_to_pair_norm = LayerNorm(c_pair)
            self.single_to_pair = LinearNoBias(c_pair, num_single_heads)
            self.single_attn = SingleAttention(
                c_single, num_heads=num_single_heads, key_dim=single_key_dim, value_dim=single_value_dim,
                optim=optim, pair_bias_gate=pair_bias_gate, pair_bias_gate_init_tau=pair_bias_gate_init_tau,
            )  # fmt: skip
            self.single_transition = make_transition_block(
                c_single, config=optim, linear_out_init_gain=single_transition_linear_out_init_gain
            )
        # Residual scales (evoformer.py:207-217, applied at :282-353): every branch's output
        # is multiplied by s_ros, the two transitions' also by their residual gain (None = 1).
        # Each branch ends in a bias-free output projection, so inside the block the scale is
        # folded into that weight (each branch module's ``branch`` / ``forward_residual_``);
        # the modules' own ``forward`` stays unscaled, as in the reference.
        self.residual_out_scale = float(residual_out_scale)
        self.single_transition_residual_gain = (
            1.0 if single_transition_residual_gain is None else float(single_transition_residual_gain)
        )
        self.pair_transition_residual_gain = (
            1.0 if pair_transition_residual_gain is None else float(pair_transition_residual_gain)
        )
        # Branch scaler (evoformer.py:289-335, branch_scaler.py): "rmsnorm" makes each branch's
        # output unit-RMS per token before s_ros multiplies it, so the scale cannot be folded
        # into the output projections there; the branches return unscaled updates and
        # ``_rms_add`` applies normalisation, scale and residual add in one pass.
        self.branch_scaler_kind = str(branch_scaler)
        self._rms = self.branch_scaler_kind == "rmsnorm"
        s_ros = 1.0 if self._rms else self.residual_out_scale
        for m in self._pair_branches() + ([self.single_attn] if self.use_single_track else []):
            m.branch_scale = s_ros
        self.pair_transition.branch_scale = s_ros * self.pair_transition_residual_gain
        if self.use_single_track:
            self.single_transition.branch_scale = s_ros * self.single_transition_residual_gain
        self.pair_dropout = pair_dropout
        self._s2p_cache = WeightCache()

    def _pair_branches(self) -> list:
        """The pair branches that take dropout, in block order."""
        mods = [self.tri_mul_out, self.tri_mul_in]
        if self.use_triangle_attention:
            mods += [self.pair_attn_row, self.pair_attn_col]
        return mods

    def _dropout_sites(self) -> list:
        """(module, rowwise) of every dropout-add, in the reference's order (``evoformer.py:289-310``)."""
        sites = [(self.tri_mul_out, True), (self.tri_mul_in, True)]
        if self.use_triangle_attention:
            sites += [(self.pair_attn_row, True), (self.pair_attn_col, False)]
        return sites

    def dropout_p(self) -> float:
        """The pair dropout rate in effect: ``pair_dropout`` in training mode, else 0."""
        return float(self.pair_dropout) if self.training else 0.0

    def _rms_add_(self, res: torch.Tensor, upd: torch.Tensor) -> torch.Tensor:
        """``res += s_ros * rms_normalize(upd)`` in place (the "rmsnorm" branch scaler)."""
        return rms_residual_add(res, upd, self.residual_out_scale, out=res)

    def _pair_site_(self, m, pair: torch.Tensor, mask: torch.Tensor, p: float, rowwise: bool) -> None:
        """One dropped pair branch in place: the fused residual epilogue (identity scaler, eval),
        or the branch out of place through the scaler and the shared-mask dropout-add."""
        if not self._rms:
            _dropout_residual_(m, pair, mask, p, rowwise)
        elif p > 0.0:
            b = rms_residual_add(None, m.branch(pair, mask), self.residual_out_scale)
            dropout_add(pair, b, p, rowwise, next_dropout_seed(), out=pair)
        else:
            self._rms_add_(pair, m.branch(pair, mask))

    def _s2p_operands(self, cdt: torch.dtype):
        from .kernels import cast_weight

        params = [self.single_to_pair_norm.weight, self.single_to_pair_norm.bias, self.single_to_pair.weight]

        def build():
            return (
                f32(self.single_to_pair_norm.weight), f32(self.single_to_pair_norm.bias), self.single_to_pair_norm.eps,
                cast_weight(self.single_to_pair.weight, cdt),
            )  # fmt: skip

        return self._s2p_cache.get(params, cdt, build)

    @inference_only("PairFormerBlock")
    def forward_(
        self, pair: torch.Tensor, single: torch.Tensor, pair_mask: torch.Tensor, seq_mask: torch.Tensor
    ) -> tuple[torch.Tensor, torch.Tensor]:
        """In-place block update of contiguous ``pair`` [B, N, N, C] and ``single`` [B, N, Cs]
        (training mode: the shared-mask dropout on the four dropped pair branches)."""
        kernel_census.record("PairFormerBlock", "hip_block_train" if self.dropout_p() > 0 else "hip_block")
        pair_logits = self.pair_forward_(pair, pair_mask)
        if self.use_single_track:
            self.single_forward_(single, seq_mask, pair_logits)
        return pair, single

    def pair_forward_(self, pair: torch.Tensor, pair_mask: torch.Tensor) -> torch.Tensor | None:
        """The pair half of the block, in place; returns the single track's pair logits (None
        without the single track).

        The pair update reads only the pair representation (``evoformer.py:289-321``), so it
        does not depend on the single half of the block. In training mode the four dropped
        branches run out of place and their shared-mask dropout-add writes into ``pair``; the
        masks' seeds are drawn in branch order (``kernels.next_dropout_seed``)."""
        p = self.dropout_p()
        for m, rowwise in self._dropout_sites():
            self._pair_site_(m, pair, pair_mask, p, rowwise)
        if self._rms:
            self._rms_add_(pair, self.pair_transition.branch(pair))
            return self.pair_logits(pair) if self.use_single_track else None
        if not self.use_single_track:
            self.pair_transition.forward_residual_(pair)
            return None
        if self.pair_transition.fused_pair:
            s2p = self._s2p_operands(gemm_dtype_for(pair))
            _, pair_logits = self.pair_transition.forward_residual_(pair, s2p=s2p)
            return pair_logits
        # other channel counts: the generic transition, then single_to_pair on its own
        self.pair_transition.forward_residual_(pair)
        return self.pair_logits(pair)

    def single_forward_(self, single: torch.Tensor, seq_mask: torch.Tensor, pair_logits: torch.Tensor) -> torch.Tensor:
        """The single half of the block, in place (``evoformer.py:322-353``)."""
        if self._rms:
            self._rms_add_(single, self.single_attn.branch(single, seq_mask, pair_logits))
            self._rms_add_(single, self.single_transition.branch(single))
            return single
        self.single_attn.forward_residual_(single, seq_mask, pair_logits)
        self.single_transition.forward_residual_(single)
        return single

    def forward_grad(
        self, pair: torch.Tensor, single: torch.Tensor, pair_mask: torch.Tensor, seq_mask: torch.Tensor
    ) -> tuple[torch.Tensor, torch.Tensor]:
        """The block out of place and differentiable (``evoformer.py:270-355``): each branch's
        training path (triangle multiplications and attention, transitions and single attention
        on the HIP kernels with their backward), every residual scale folded into its branch's
        output projection, the residual adds in autograd; in training mode the four dropped pair
        branches add through the HIP shared-mask dropout-add (``DropoutAddFunction``; seeds drawn
        in branch order, so ``torch.utils.checkpoint``'s recompute regenerates the same masks)."""
        from .kernels import layer_norm_for_gemm, token_linear

        kernel_census.record("PairFormerBlock", "hip_block_grad")
        p_drop = self.dropout_p()
        if self._rms:
            # unit-RMS rows (F.rms_norm, eps 1e-6 as primitives.py:79-87) times s_ros, in autograd
            s_ros = self.residual_out_scale

            def sc(u: torch.Tensor) -> torch.Tensor:
                return s_ros * torch.nn.functional.rms_norm(u, (u.shape[-1],), eps=1e-6)
        else:

            def sc(u: torch.Tensor) -> torch.Tensor:
                return u

        p = pair
        for m, rowwise in self._dropout_sites():
            upd = sc(m.branch(p, pair_mask))
            p = DropoutAddFunction.apply(p, upd, p_drop, rowwise, next_dropout_seed()) if p_drop > 0 else p + upd
        p = p + sc(self.pair_transition.branch(p))
        if not self.use_single_track:
            return p, single
        n = self.single_to_pair_norm
        logits = token_linear(layer_norm_for_gemm(p, n.weight, n.bias, n.eps), self.single_to_pair.weight)
        s = single + sc(self.single_attn.branch(single, seq_mask, logits.movedim(-1, -3)))
        s = s + sc(self.single_transition.branch(s))
        return p, s

    def forward(
        self, pair: torch.Tensor, single: torch.Tensor, pair_mask: torch.Tensor, seq_mask: torch.Tensor
    ) -> tuple[torch.Tensor, torch.Tensor]:
        """Reference signature (``evoformer.py:270-355``): returns new ``(pair, single)``; under
        grad the differentiable path (``forward_grad``), else the in-place kernels on copies."""
        has_batch = pair.dim() == 4
        if not has_batch:
            pair, single = pair.unsqueeze(0), single.unsqueeze(0)
            pair_mask, seq_mask = pair_mask.unsqueeze(0), seq_mask.unsqueeze(0)
        if torch.is_grad_enabled():
            p, s = self.forward_grad(pair, single, pair_mask.to(torch.float32), seq_mask)
        else:
            p, s = self.forward_(pair.contiguous().clone(), single.contiguous().clone(), pair_mask, seq_mask)
        return (p, s) if has_batch else (p.squeeze(0), s.squeeze(0))

    def pair_logits(self, pair: torch.Tensor) -> torch.Tensor:
        """``single_to_pair(single_to_pair_norm(pair)).movedim(-1, -3)`` via the standalone kernel."""
        lw, lb, eps, w = self._s2p_operands(gemm_dtype_for(pair))
        return single_to_pair(pair, lw, lb, eps, w)


class PairFormerStack(nn.Module):
    """The trunk loop over ``num_blocks`` PairFormer blocks (``evoformer.py:593-601``).

    ``layer_attr`` names the ModuleList in the state dict (``blocks`` here; the confidence
    head's stack uses the reference's ``layers``). ``layer_kwargs(i)``, when given, returns
    the constructor arguments that differ per layer (the reference's per-layer residual
    scales, ``evoformer.py:459-489``); they override ``block_kwargs``. With
    ``optim.use_gradient_checkpointing`` each block runs under ``torch.utils.checkpoint``
    (non-reentrant) when autograd is recording, as at ``evoformer.py:58``, ``:593-596``."""

    def __init__(self, num_blocks: int, c_pair: int = 128, c_single: int = 384, optim: OptimConfig | None = None,
                 layer_attr: str = "blocks", layer_kwargs=None, **block_kwargs):  # fmt: skip
        super().__init__()
        self._layer_attr = layer_attr
        self.use_gradient_checkpointing = bool(optim is not None and optim.use_gradient_checkpointing)

        def block(i: int) -> PairFormerBlock:
            kw = dict(block_kwargs)
            if layer_kwargs is not None:
                kw.update(layer_kwargs(i))
            return PairFormerBlock(c_pair, c_single, optim=optim, **kw)

        setattr(self, layer_attr, nn.ModuleList([block(i) for i in range(num_blocks)]))

    @property
    def blocks(self) -> nn.ModuleList:
        return self._modules[self._layer_attr]

    def forward(
        self, pair: torch.Tensor, single: torch.Tensor, pair_mask: torch.Tensor, seq_mask: torch.Tensor
    ) -> tuple[torch.Tensor, torch.Tensor]:
        """Same result as applying the blocks in order. On the GPU the single half of block i
        runs on a second stream, beside the pair half of block i + 1: the pair update never
        reads the single representation, and the single half of block i needs only block i's
        pair logits (an event orders it after them) and block i - 1's single half (same
        stream). The streams join before returning. Under grad the blocks' differentiable
        path runs in order on one stream, each block checkpointed when the optim config asks."""
        if torch.is_grad_enabled():
            pair_mask = pair_mask.to(torch.float32)
            for blk in self.blocks:
                if self.use_gradient_checkpointing:
                    pair, single = _checkpoint(blk.forward_grad, pair, single, pair_mask, seq_mask)
                else:
                    pair, single = blk.forward_grad(pair, single, pair_mask, seq_mask)
            return pair, single
        pair = pair.contiguous().clone()
        single = single.contiguous().clone()
        # One fp32 mask object for every block: the attention kernels' outer-product check
        # of the mask is cached per tensor object, so the trunk checks it once.
        pair_mask = pair_mask.to(torch.float32).contiguous()
        if not pair.is_cuda or len(self.blocks) == 0:
            for blk in self.blocks:
                blk.forward_(pair, single, pair_mask, seq_mask)
            return pair, single
        main = torch.cuda.current_stream(pair.device)
        side = self._side_stream(pair.device)
        side.wait_stream(main)  # single, masks and the clones above
        for blk in self.blocks:
            kernel_census.record("PairFormerBlock", "hip_block_train" if blk.dropout_p() > 0 else "hip_block")
            pair_logits = blk.pair_forward_(pair, pair_mask)
            if not blk.use_single_track:
                continue
            done = torch.cuda.Event()
            done.record(main)
            side.wait_event(done)
            with torch.cuda.stream(side):
                pair_logits.record_stream(side)  # freed on main, still read on side
                blk.single_forward_(single, seq_mask, pair_logits)
        main.wait_stream(side)
        return pair, single

    def _side_stream(self, device) -> torch.cuda.Stream:
        streams = self.__dict__.setdefault("_side_streams", {})
        key = torch.device(device).index
        if key not in streams:
            streams[key] = torch.cuda.Stream(device=device)  # default priority
        return streams[key]


class ConfidencePairFormer(PairFormerStack):
    """The PairFormer layers of the confidence head (``confidence.py:88-117``, run in order
    at ``:304-308``): ``num_layer`` blocks of the trunk's shape (``ConfidenceConfig``,
    ``config.py:578-589``: 4 layers, c_pair 128, c_single 384, 4 pair and 16 single heads),
    state-dict keys ``layers.{i}.*`` as in the reference's ``ConfidenceHead``. The feature
    embedding before the layers and the logit heads after them are outside the hot path."""

    def __init__(self, num_layer: int = 4, c_pair: int = 128, c_single: int = 384, num_pair_heads: int = 4,
                 num_single_heads: int = 16, optim: OptimConfig | None = None, **block_kwargs):  # fmt: skip
        super().__init__(
            num_layer, c_pair, c_single, optim=optim, layer_attr="layers", num_pair_heads=num_pair_heads,
            num_single_heads=num_single_heads, single_key_dim=c_single, single_value_dim=c_single, **block_kwargs,
        )  # fmt: skip


class TemplatePairFormerBlock(nn.Module):
    """Pair-only PairFormer block of the template embedding (``template_embedding.py:180-241``):
    triangle multiplications, row and column attention, and a transition with a smaller
    intermediate factor; same submodule names and ``forward(pair, pair_mask)``.

    Built for num_channels in 64 (the reference's template stack, ``TemplatePairFormerConfig``,
    ``config.py:636-650``: 4 heads of 16), 128 and 256; the triangle attention runs the
    generic-channel path for anything but 128 channels in 4 heads."""

    def __init__(self, num_channels: int, num_heads: int = 4, num_intermediate_factor: int = 2,
                 pair_dropout: float = 0.25, optim: OptimConfig | None = None, residual_out_scale: float = 1.0):  # fmt: skip
        super().__init__()
        require_hip("TemplatePairFormerBlock", optim)
        from .kernels import TRIMUL_CHANNELS

        head_dim = max(num_channels // num_heads, 16)
        if num_channels not in TRIMUL_CHANNELS or num_channels % num_heads or head_dim > 32 or num_heads > 16:
            raise NotActive(
                "TemplatePairFormerBlock",
                f"num_channels={num_channels}, num_heads={num_heads}: built for {TRIMUL_CHANNELS} channels in at "
                "most 16 heads of dimension max(C/H, 16) <= 32",
            )  # fmt: skip
        self.tri_mul_out = TriangleMulOutgoing(num_channels, optim=optim)
        self.tri_mul_in = TriangleMulIncoming(num_channels, optim=optim)
        self.pair_attn_row = GridSelfAttention(num_channels, num_heads=num_heads, transpose=False, optim=optim)
        self.pair_attn_col = GridSelfAttention(num_channels, num_heads=num_heads, transpose=True, optim=optim)
        self.pair_transition = make_transition_block(num_channels, num_intermediate_factor, config=optim)
        self.num_intermediate_factor = num_intermediate_factor
        self.pair_dropout = pair_dropout
        # Every branch is output-scaled by residual_out_scale (template_embedding.py:233-240),
        # folded into each branch's output projection.
        self.residual_out_scale = float(residual_out_scale)
        for m in (self.tri_mul_out, self.tri_mul_in, self.pair_attn_row, self.pair_attn_col, self.pair_transition):
            m.branch_scale = self.residual_out_scale

    def forward_(self, pair: torch.Tensor, pair_mask: torch.Tensor) -> torch.Tensor:
        """In place: ``pair`` [B, N, N, C] contiguous (``template_embedding.py:230-240``); in
        training mode the shared-mask dropout-add on the four dropped branches."""
        p = float(self.pair_dropout) if self.training else 0.0
        kernel_census.record("TemplatePairFormerBlock", "hip_block_train" if p > 0 else "hip_block")
        _dropout_residual_(self.tri_mul_out, pair, pair_mask, p, True)
        _dropout_residual_(self.tri_mul_in, pair, pair_mask, p, True)
        _dropout_residual_(self.pair_attn_row, pair, pair_mask, p, True)
        _dropout_residual_(self.pair_attn_col, pair, pair_mask, p, False)
        self.pair_transition.forward_residual_(pair)
        return pair

    @inference_only("TemplatePairFormerBlock")
    def forward(self, pair: torch.Tensor, pair_mask: torch.Tensor) -> torch.Tensor:
        """Reference signature: ``pair`` [B?, N, N, C], ``pair_mask`` [B?, N, N] -> new pair."""
        has_batch = pair.dim() == 4
        if not has_batch:
            pair, pair_mask = pair.unsqueeze(0), pair_mask.unsqueeze(0)
        out = self.forward_(pair.contiguous().clone(), pair_mask)
        return out if has_batch else out.squeeze(0)


class TrunkRecycler(nn.Module):
    """The recycling embeddings around the trunk (``evoformer.py:400-412``; applied at
    ``:520-526`` and ``:558-561``): ``pair = pair_init + prev_embedding(LN(prev_pair))`` and,
    with the single track, ``single = single_init + prev_single_embedding(LN(prev_single))``.
    Submodule names as in the reference's ``Evoformer`` (``prev_embedding_layer_norm``,
    ``prev_embedding``, ``prev_single_embedding_layer_norm``, ``prev_single_embedding``), so
    the ``evoformer.prev_*`` keys of a checkpoint load unchanged. Both projections start at
    zero (AF3 final init)."""

    def __init__(self, c_pair: int = 128, c_single: int = 384, use_single_track: bool = True,
                 optim: OptimConfig | None = None):  # fmt: skip
        super().__init__()
        require_hip("TrunkRecycler", optim)
        self.prev_embedding_layer_norm = LayerNorm(c_pair)
        self.prev_embedding = LinearNoBias(c_pair, c_pair, initializer="zeros")
        self.use_single_track = bool(use_single_track)
        if self.use_single_track:
            self.prev_single_embedding_layer_norm = LayerNorm(c_single)
            self.prev_single_embedding = LinearNoBias(c_single, c_single, initializer="zeros")
        self._cache = WeightCache()

    def _operands(self, cdt: torch.dtype) -> dict:
        from .kernels import cast_weight

        mods = [(self.prev_embedding_layer_norm, self.prev_embedding)]
        if self.use_single_track:
            mods.append((self.prev_single_embedding_layer_norm, self.prev_single_embedding))
        params = [p for ln, lin in mods for p in (ln.weight, ln.bias, lin.weight)]

        def build():
            return [(f32(ln.weight), f32(ln.bias), ln.eps, cast_weight(lin.weight, cdt)) for ln, lin in mods]

        return self._cache.get(params, cdt, build)

    @inference_only("TrunkRecycler")
    def forward_(
        self, pair: torch.Tensor, single: torch.Tensor, prev_pair: torch.Tensor, prev_single: torch.Tensor
    ) -> tuple[torch.Tensor, torch.Tensor]:
        """In place: ``pair += prev_embedding(LN(prev_pair))`` (and the single track)."""
        from .kernels import recycle_embed_

        kernel_census.record("TrunkRecycler", "hip_recycle_embed")
        ops = self._operands(gemm_dtype_for(pair))
        recycle_embed_(pair, prev_pair, *ops[0])
        if self.use_single_track:
            recycle_embed_(single, prev_single, *ops[1])
        return pair, single

    @inference_only("TrunkRecycler")
    def forward(
        self, pair_init: torch.Tensor, single_init: torch.Tensor, prev_pair: torch.Tensor, prev_single: torch.Tensor
    ) -> tuple[torch.Tensor, torch.Tensor]:
        """New ``(pair, single)``: the initial embeddings plus the recycling embeddings."""
        return self.forward_(
            pair_init.contiguous().clone(), single_init.contiguous().clone(), prev_pair, prev_single
        )


def run_recycles(
    recycler: TrunkRecycler,
    trunk: PairFormerStack,
    pair_init: torch.Tensor,
    single_init: torch.Tensor,
    pair_mask: torch.Tensor,
    seq_mask: torch.Tensor,
    num_recycles: int,
    between=None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """The recycle loop around the trunk (``model.py:385-470``), inference form.

    The previous outputs start at zero (``model.py:311-319``). Each of the
    ``num_recycles + 1`` passes adds the recycling embeddings of the previous pass's outputs
    to the initial embeddings, runs ``between(pair, single)`` -- the stages the reference
    runs between the recycling embedding and the trunk (template embedding, MSA stack;
    outside this build, skipped when None) -- and the trunk; its outputs feed the next pass
    (``model.py:468-470``). Returns the last pass's ``(pair, single)``.
    """
    if num_recycles < 0:
        raise ValueError(f"num_recycles={num_recycles} must be >= 0")
    prev_pair = torch.zeros_like(pair_init)
    prev_single = torch.zeros_like(single_init)
    pair = single = None
    for _ in range(num_recycles + 1):
        pair, single = recycler(pair_init, single_init, prev_pair, prev_single)
        if between is not None:
            pair, single = between(pair, single)
        pair, single = trunk(pair, single, pair_mask, seq_mask)
        prev_pair, prev_single = pair, single
    return pair, single


class EvoformerBlock(nn.Module):
    """One block of the Evoformer MSA stack (``evoformer.py:100-175``): ``pair +=
    OuterProductMean(msa)``, ``msa += MSAAttention(msa, pair)`` (pair-weighted averaging),
    ``msa += msa_transition(msa)``, then the pair half of the PairFormer block (triangle
    multiplications, row and column attention, pair transition). Every branch is
    output-scaled by ``residual_out_scale`` (folded into its output projection). Same
    constructor arguments, submodule names and ``forward(msa, pair, msa_mask, pair_mask)``."""

    def __init__(
        self,
        c_msa: int,
        c_pair: int,
        num_msa_heads: int = 8,
        num_pair_heads: int = 4,
        outer_product_hidden: int = 32,
        msa_dropout: float = 0.15,
        pair_dropout: float = 0.25,
        optim: OptimConfig | None = None,
        residual_out_scale: float = 1.0,
        use_triangle_attention: bool = True,
        trimul_kwargs: dict | None = None,
    ):
        super().__init__()
        from .attention import MSAAttention
        from .ops import OuterProductMean

        require_hip("EvoformerBlock", optim)
        tk = trimul_kwargs or {}
        self.row_attn = MSAAttention(c_msa, c_pair, num_heads=num_msa_heads, optim=optim)
        self.outer_product = OuterProductMean(c_msa, c_pair, c_hidden=outer_product_hidden, optim=optim)
        self.tri_mul_out = TriangleMulOutgoing(c_pair, optim=optim, **tk)
        self.tri_mul_in = TriangleMulIncoming(c_pair, optim=optim, **tk)
        self.use_triangle_attention = bool(use_triangle_attention)
        if self.use_triangle_attention:
            self.pair_attn_row = GridSelfAttention(c_pair, num_heads=num_pair_heads, transpose=False, optim=optim)
            self.pair_attn_col = GridSelfAttention(c_pair, num_heads=num_pair_heads, transpose=True, optim=optim)
        self.pair_transition = make_transition_block(c_pair, config=optim)
        self.msa_transition = make_transition_block(c_msa, config=optim)
        self.msa_dropout = msa_dropout
        self.pair_dropout = pair_dropout
        self.residual_out_scale = float(residual_out_scale)
        mods = [self.row_attn, self.outer_product, self.tri_mul_out, self.tri_mul_in, self.pair_transition,
                self.msa_transition]  # fmt: skip
        if self.use_triangle_attention:
            mods += [self.pair_attn_row, self.pair_attn_col]
        for m in mods:
            m.branch_scale = self.residual_out_scale

    @inference_only("EvoformerBlock")
    def forward_(
        self, msa: torch.Tensor, pair: torch.Tensor, msa_mask: torch.Tensor, pair_mask: torch.Tensor
    ) -> tuple[torch.Tensor, torch.Tensor]:
        """In place on contiguous ``msa`` [B, S, N, c_msa] and ``pair`` [B, N, N, c_pair]; in
        training mode the MSA update of ``row_attn`` takes the row-shared ``msa_dropout`` and the
        pair branches the shared-mask ``pair_dropout`` (``evoformer.py:162-174``; seeds drawn in
        that order)."""
        train = self.training
        p_msa = float(self.msa_dropout) if train else 0.0
        p_pair = float(self.pair_dropout) if train else 0.0
        kernel_census.record("EvoformerBlock", "hip_block_train" if max(p_msa, p_pair) > 0 else "hip_block")
        self.outer_product.forward_residual_(pair, msa, msa_mask)
        if p_msa > 0.0:
            upd = self.row_attn.branch(msa, msa_mask, pair)
            dropout_add(msa, upd, p_msa, True, next_dropout_seed(), out=msa)
        else:
            self.row_attn.forward_residual_(msa, msa_mask, pair)
        self.msa_transition.forward_residual_(msa)
        _dropout_residual_(self.tri_mul_out, pair, pair_mask, p_pair, True)
        _dropout_residual_(self.tri_mul_in, pair, pair_mask, p_pair, True)
        if self.use_triangle_attention:
            _dropout_residual_(self.pair_attn_row, pair, pair_mask, p_pair, True)
            _dropout_residual_(self.pair_attn_col, pair, pair_mask, p_pair, False)
        self.pair_transition.forward_residual_(pair)
        return msa, pair

    @inference_only("EvoformerBlock")
    def forward(
        self, msa: torch.Tensor, pair: torch.Tensor, msa_mask: torch.Tensor, pair_mask: torch.Tensor
    ) -> tuple[torch.Tensor, torch.Tensor]:
        """Reference signature: msa [B?, S, N, c_msa], pair [B?, N, N, c_pair] -> new (msa, pair)."""
        has_batch = msa.dim() == 4
        if not has_batch:
            msa, pair = msa.unsqueeze(0), pair.unsqueeze(0)
            msa_mask, pair_mask = msa_mask.unsqueeze(0), pair_mask.unsqueeze(0)
        m, p = self.forward_(msa.contiguous().clone(), pair.contiguous().clone(), msa_mask, pair_mask)
        return (m, p) if has_batch else (m.squeeze(0), p.squeeze(0))


class EvoformerStack(nn.Module):
    """The MSA stack (``evoformer.py:433-455``, run at ``:575-580``): ``num_layer``
    EvoformerBlocks under the reference's ``msa_stack.{i}`` keys; ``layer_kwargs(i)`` gives
    per-layer constructor arguments (residual scales)."""

    def __init__(self, num_layer: int, c_msa: int = 64, c_pair: int = 128, optim: OptimConfig | None = None,
                 layer_kwargs=None, **block_kwargs):  # fmt: skip
        super().__init__()

        def block(i: int) -> EvoformerBlock:
            kw = dict(block_kwargs)
            if layer_kwargs is not None:
                kw.update(layer_kwargs(i))
            return EvoformerBlock(c_msa, c_pair, optim=optim, **kw)

        self.msa_stack = nn.ModuleList([block(i) for i in range(num_layer)])

    @inference_only("EvoformerStack")
    def forward(
        self, msa: torch.Tensor, pair: torch.Tensor, msa_mask: torch.Tensor, pair_mask: torch.Tensor
    ) -> tuple[torch.Tensor, torch.Tensor]:
        """msa [B, S, N, c_msa], pair [B, N, N, c_pair] -> new (msa, pair) after every block."""
        msa, pair = msa.contiguous().clone(), pair.contiguous().clone()
        pair_mask = pair_mask.to(torch.float32).contiguous()
        for blk in self.msa_stack:
            blk.forward_(msa, pair, msa_mask, pair_mask)
        return msa, pair
