"""PairFormer block and trunk on the HIP kernels.

``PairFormerBlock`` keeps the reference's constructor arguments, submodule names
(so state dicts load unchanged) and ``forward(pair, single, pair_mask, seq_mask)``
signature (``src/deepfold3/model/evoformer.py:178-355``). Eval-mode semantics: the
branch scaler is the identity, ``residual_out_scale`` is 1 and dropout-add is a plain
add (``triton/dropout_add.py:236-237``), so every residual add is fused into the
epilogue of the kernel that produces the branch. ``single_to_pair`` is fused into the
pair transition's epilogue (it normalises the updated pair rows).

``PairFormerStack`` is the trunk loop (``evoformer.py:593-601``): it copies the inputs
once and then updates them in place, block after block.
"""

from __future__ import annotations

import torch
import torch.nn as nn

from . import kernel_census
from .attention import GridSelfAttention, SingleAttention
from .config import OptimConfig, require_hip
from .inference_guard import NotActive, inference_only
from .kernels import gemm_dtype_for, single_to_pair
from .ops import TriangleMulIncoming, TriangleMulOutgoing
from .primitives import LayerNorm, LinearNoBias, WeightCache, f32, make_transition_block


class PairFormerBlock(nn.Module):
    """One PairFormer layer with the single track (AF3 ``PairFormerIteration``)."""

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
        gains = (single_transition_residual_gain, pair_transition_residual_gain)
        if residual_out_scale != 1.0 or any(g not in (None, 1.0) for g in gains) or branch_scaler != "identity":
            raise NotActive("PairFormerBlock", "only unit residual scales and the identity branch scaler are built")
        if not use_triangle_attention or not use_single_track:
            raise NotActive("PairFormerBlock", "the triangle-attention and single-track branches are always built")
        tk = trimul_kwargs or {}
        self.tri_mul_out = TriangleMulOutgoing(c_pair, optim=optim, **tk)
        self.tri_mul_in = TriangleMulIncoming(c_pair, optim=optim, **tk)
        self.use_triangle_attention = True
        self.pair_attn_row = GridSelfAttention(c_pair, num_heads=num_pair_heads, transpose=False, optim=optim)
        self.pair_attn_col = GridSelfAttention(c_pair, num_heads=num_pair_heads, transpose=True, optim=optim)
        self.pair_transition = make_transition_block(c_pair, config=optim)
        self.use_single_track = True
        self.single_to_pair_norm = LayerNorm(c_pair)
        self.single_to_pair = LinearNoBias(c_pair, num_single_heads)
        self.single_attn = SingleAttention(
            c_single, num_heads=num_single_heads, key_dim=single_key_dim, value_dim=single_value_dim, optim=optim,
            pair_bias_gate=pair_bias_gate, pair_bias_gate_init_tau=pair_bias_gate_init_tau,
        )  # fmt: skip
        self.single_transition = make_transition_block(
            c_single, config=optim, linear_out_init_gain=single_transition_linear_out_init_gain
        )
        self.residual_out_scale = 1.0
        self.pair_dropout = pair_dropout
        self._s2p_cache = WeightCache()

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
        """In-place block update of contiguous ``pair`` [B, N, N, C] and ``single`` [B, N, Cs]."""
        if self.training:
            raise NotActive("PairFormerBlock", "training-mode dropout is not built (eval only)")
        kernel_census.record("PairFormerBlock", "hip_block")
        pair_logits = self.pair_forward_(pair, pair_mask)
        self.single_forward_(single, seq_mask, pair_logits)
        return pair, single

    def pair_forward_(self, pair: torch.Tensor, pair_mask: torch.Tensor) -> torch.Tensor:
        """The pair half of the block, in place; returns the single track's pair logits.

        The pair update reads only the pair representation (``evoformer.py:289-321``), so it
        does not depend on the single half of the block.
        """
        self.tri_mul_out.forward_residual_(pair, pair_mask)
        self.tri_mul_in.forward_residual_(pair, pair_mask)
        self.pair_attn_row.forward_residual_(pair, pair_mask)
        self.pair_attn_col.forward_residual_(pair, pair_mask)
        s2p = self._s2p_operands(gemm_dtype_for(pair))
        _, pair_logits = self.pair_transition.forward_residual_(pair, s2p=s2p)
        return pair_logits

    def single_forward_(self, single: torch.Tensor, seq_mask: torch.Tensor, pair_logits: torch.Tensor) -> torch.Tensor:
        """The single half of the block, in place (``evoformer.py:322-353``)."""
        self.single_attn.forward_residual_(single, seq_mask, pair_logits)
        self.single_transition.forward_residual_(single)
        return single

    @inference_only("PairFormerBlock")
    def forward(
        self, pair: torch.Tensor, single: torch.Tensor, pair_mask: torch.Tensor, seq_mask: torch.Tensor
    ) -> tuple[torch.Tensor, torch.Tensor]:
        """Reference signature (``evoformer.py:270-355``): returns new ``(pair, single)``."""
        has_batch = pair.dim() == 4
        if not has_batch:
            pair, single = pair.unsqueeze(0), single.unsqueeze(0)
            pair_mask, seq_mask = pair_mask.unsqueeze(0), seq_mask.unsqueeze(0)
        p, s = self.forward_(pair.contiguous().clone(), single.contiguous().clone(), pair_mask, seq_mask)
        return (p, s) if has_batch else (p.squeeze(0), s.squeeze(0))

    def pair_logits(self, pair: torch.Tensor) -> torch.Tensor:
        """``single_to_pair(single_to_pair_norm(pair)).movedim(-1, -3)`` via the standalone kernel."""
        lw, lb, eps, w = self._s2p_operands(gemm_dtype_for(pair))
        return single_to_pair(pair, lw, lb, eps, w)


class PairFormerStack(nn.Module):
    """The trunk loop over ``num_blocks`` PairFormer blocks (``evoformer.py:593-601``).

    ``layer_attr`` names the ModuleList in the state dict (``blocks`` here; the confidence
    head's stack uses the reference's ``layers``)."""

    def __init__(self, num_blocks: int, c_pair: int = 128, c_single: int = 384, optim: OptimConfig | None = None,
                 layer_attr: str = "blocks", **block_kwargs):  # fmt: skip
        super().__init__()
        self._layer_attr = layer_attr
        setattr(
            self, layer_attr,
            nn.ModuleList([PairFormerBlock(c_pair, c_single, optim=optim, **block_kwargs) for _ in range(num_blocks)]),
        )  # fmt: skip

    @property
    def blocks(self) -> nn.ModuleList:
        return self._modules[self._layer_attr]

    @inference_only("PairFormerStack")
    def forward(
        self, pair: torch.Tensor, single: torch.Tensor, pair_mask: torch.Tensor, seq_mask: torch.Tensor
    ) -> tuple[torch.Tensor, torch.Tensor]:
        """Same result as applying the blocks in order. On the GPU the single half of block i
        runs on a second stream, beside the pair half of block i + 1: the pair update never
        reads the single representation, and the single half of block i needs only block i's
        pair logits (an event orders it after them) and block i - 1's single half (same
        stream). The streams join before returning."""
        pair = pair.contiguous().clone()
        single = single.contiguous().clone()
        if not pair.is_cuda or len(self.blocks) == 0:
            for blk in self.blocks:
                blk.forward_(pair, single, pair_mask, seq_mask)
            return pair, single
        main = torch.cuda.current_stream(pair.device)
        side = self._side_stream(pair.device)
        side.wait_stream(main)  # single, masks and the clones above
        for blk in self.blocks:
            kernel_census.record("PairFormerBlock", "hip_block")
            pair_logits = blk.pair_forward_(pair, pair_mask)
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

    Built for num_channels = 128 (every pair kernel here is); the reference's template
    stack runs at 64 channels (``TemplatePairFormerConfig``, ``config.py:636-650``), which
    refuses by name at construction."""

    def __init__(self, num_channels: int, num_heads: int = 4, num_intermediate_factor: int = 2,
                 pair_dropout: float = 0.25, optim: OptimConfig | None = None, residual_out_scale: float = 1.0):  # fmt: skip
        super().__init__()
        require_hip("TemplatePairFormerBlock", optim)
        if num_channels != 128 or num_heads != 4:
            raise NotActive(
                "TemplatePairFormerBlock",
                f"num_channels={num_channels}, num_heads={num_heads}: the pair kernels are built for 128 channels "
                "and 4 heads of 32",
            )  # fmt: skip
        if residual_out_scale != 1.0:
            raise NotActive("TemplatePairFormerBlock", "only a unit residual scale is built")
        self.tri_mul_out = TriangleMulOutgoing(num_channels, optim=optim)
        self.tri_mul_in = TriangleMulIncoming(num_channels, optim=optim)
        self.pair_attn_row = GridSelfAttention(num_channels, num_heads=num_heads, transpose=False, optim=optim)
        self.pair_attn_col = GridSelfAttention(num_channels, num_heads=num_heads, transpose=True, optim=optim)
        self.pair_transition = make_transition_block(num_channels, num_intermediate_factor, config=optim)
        self.num_intermediate_factor = num_intermediate_factor
        self.pair_dropout = pair_dropout
        self.residual_out_scale = 1.0

    def forward_(self, pair: torch.Tensor, pair_mask: torch.Tensor) -> torch.Tensor:
        """In place: ``pair`` [B, N, N, C] contiguous (``template_embedding.py:230-240``, eval)."""
        if self.training and self.pair_dropout > 0.0:
            raise NotActive("TemplatePairFormerBlock", "training-mode dropout is not built (eval only)")
        kernel_census.record("TemplatePairFormerBlock", "hip_block")
        self.tri_mul_out.forward_residual_(pair, pair_mask)
        self.tri_mul_in.forward_residual_(pair, pair_mask)
        self.pair_attn_row.forward_residual_(pair, pair_mask)
        self.pair_attn_col.forward_residual_(pair, pair_mask)
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
