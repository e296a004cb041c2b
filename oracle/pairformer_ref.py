"""CPU/GPU eager oracle for the DeepFold3 PairFormer block. TEST INFRASTRUCTURE ONLY.

A functional PyTorch restatement of the reference's stock path
(``OptimConfig.none()``, eval mode) that takes the block's state dict. Only
``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg use
it, and only as the checker or as a timed baseline; the product path never calls
it.

Each function follows the reference file:line it cites, keeping its op order
and rounding points: LayerNorm upcasts to fp32 and casts back to the input dtype,
the a/b split of the triangle projection is interleaved (``0::2``/``1::2``), the
attention masks are additive ``1e9 * (mask - 1)``, softmax runs on
``logits.float()`` and casts back, GridSelfAttention post-scales ``QK^T`` and
SingleAttention pre-scales ``q``.

Pinning (what checks this restatement, beyond retyping it):
  * ``tests/golden/*.npz``: fp32 outputs of the reference modules themselves,
    imported on CPU by ``tests/golden/make_golden.py`` (block, every branch,
    masked and unmasked).
  * brute-force loops at tiny N for the triangle contraction, the per-row
    attention and the column-attention transpose semantics
    (``tests/test_oracle.py``).
  * invariants: batch consistency, row-chunked == whole, fully masked rows
    give the mean of V.
  * residual scales: a scale s on every branch equals the unscaled block with each
    branch's bias-free output projection multiplied by s (every branch is linear in
    it); a zero transition gain equals a zeroed ``linear2``; s = 0 returns the inputs.
  * recycling embedding: zero previous outputs give ``init + b W^T`` (LN of a zero row
    is its bias b); LayerNorm's invariance to per-row shifts; linearity in W.
  * outer product mean and MSA pair-weighted averaging: explicit loops at tiny sizes; the
    Evoformer block: its pair half equals the template block's on the OPM-updated pair.
  * kernel-level attention and its backward: a per-row loop for the forward; the centred
    backward equals autograd of the forward in fp64 and finite differences
    (``torch.autograd.gradcheck``); the centring constant sums to the uncentred D.
  * the triangle multiply after its input LayerNorm (``tri_mul_core``): composing it with
    the LayerNorm and the block-order weights gives ``tri_mul`` (pinned by the golden
    vectors); its gradient by finite differences.
  * multi-head routed triangle multiplication (``mhr_head_mix``): a zero router with
    "channel" is exactly the plain ``tri_mul``; head_rms / head_ln give every head unit RMS /
    zero mean before the affine (closed forms, against a per-head loop); the softmax gates
    sum to H, the sigmoid gates equal 2 sigmoid(r); post_channel with uniform gates equals
    channel; a one-hot-scaled head equals scaling out_proj's column block (the gate is a
    per-head factor before out_proj); scaling one head's contraction leaves head_rms /
    head_ln unchanged.
"""

from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

__all__ = [
    "layer_norm",
    "tri_mul",
    "mhr_head_mix",
    "grid_attention",
    "transition",
    "single_to_pair",
    "single_attention",
    "pairformer_block",
    "template_pairformer_block",
    "pairformer_trunk",
    "recycle_embed",
    "recycled_trunk",
    "outer_product_mean",
    "msa_attention",
    "evoformer_block",
    "evo_attention",
    "evo_attention_backward",
    "tri_mul_core",
    "philox4x32_10",
    "dropout_mask",
    "shared_dropout_mask",
    "dropout_add",
]


def layer_norm(x: torch.Tensor, w: torch.Tensor, b: torch.Tensor, eps: float = 1e-5) -> torch.Tensor:
    """fp32 LayerNorm over the last dim, cast back to x's dtype (``primitives.py:90-115``)."""
    return F.layer_norm(x.float(), (x.shape[-1],), w.float(), b.float(), eps).to(x.dtype)


def _sub(p: dict[str, torch.Tensor], prefix: str) -> dict[str, torch.Tensor]:
    return {k[len(prefix) :]: v for k, v in p.items() if k.startswith(prefix)}


def _triangle_matmul(a: torch.Tensor, b: torch.Tensor, outgoing: bool) -> torch.Tensor:
    """``bikc,bjkc->bijc`` (outgoing) or ``bkjc,bkic->bijc`` (incoming), ``ops.py:58-98``."""
    # Both operands are made contiguous before the batched product (same values; a
    # transposed-view right operand of a bf16 batched matmul is avoided on ROCm).
    if outgoing:
        return torch.matmul(a.permute(0, 3, 1, 2).contiguous(), b.permute(0, 3, 2, 1).contiguous()).permute(0, 2, 3, 1)
    return torch.matmul(a.permute(0, 3, 2, 1).contiguous(), b.permute(0, 3, 1, 2).contiguous()).permute(0, 3, 2, 1)


def tri_mul(
    z: torch.Tensor,
    mask: torch.Tensor,
    p: dict[str, torch.Tensor],
    outgoing: bool,
    num_heads: int = 0,
    head_norm: str = "channel",
    router: bool = False,
    router_kind: str = "softmax",
) -> torch.Tensor:
    """Stock ``_TriangleMulBase._compute`` (``ops.py:412-473``), plain heads (AF3) by default,
    or multi-head routed (``num_heads`` > 0 with a per-head norm and / or the router,
    ``ops.py:179-345``, ``:476-545``).

    Args:
        z: [B, N, N, C]; mask: [B, N, N]; p: keys ``norm_left.*``, ``proj.weight``,
        ``gate.weight``, ``norm_center.weight`` (and ``.bias`` except for ``head_rms``),
        ``out_proj.weight``, ``out_gate.weight``, ``router.weight`` [H, C] with the router.
    Returns:
        The update [B, N, N, C] (not added to z).
    """
    z0 = layer_norm(z, p["norm_left.weight"], p["norm_left.bias"])
    proj = F.linear(z0, p["proj.weight"])
    gate = torch.sigmoid(F.linear(z0, p["gate.weight"]))
    out_gate = torch.sigmoid(F.linear(z0, p["out_gate.weight"]))
    router_logits = F.linear(z0, p["router.weight"]) if router else None
    del z0
    proj = proj * gate
    a = proj[..., 0::2]
    b = proj[..., 1::2]
    m = mask.unsqueeze(-1)
    a = (a * m).contiguous()
    b = (b * m).contiguous()
    act = _triangle_matmul(a, b, outgoing)
    del a, b
    if head_norm != "channel" or router:
        act = mhr_head_mix(act, router_logits, p, num_heads, head_norm, router_kind)
    else:
        act = layer_norm(act, p["norm_center.weight"], p["norm_center.bias"])
    act = F.linear(act, p["out_proj.weight"])
    return act * out_gate


def mhr_head_mix(
    act: torch.Tensor, router_logits: torch.Tensor | None, p: dict[str, torch.Tensor], h: int, head_norm: str,
    router_kind: str, eps: float = 1e-5,
) -> torch.Tensor:
    """``_TriangleMulBase._mhr_head_mix`` (``ops.py:476-545``): the contraction [.., C] as H heads
    of d = C / H; "channel" LayerNorms all C, "head_rms" / "head_ln" normalise each head (fp32,
    rounded to act's dtype before the affine of ``norm_center`` viewed [H, d]); the router's
    gates g = H softmax_h(R) or 2 sigmoid(R) (fp32, cast to the heads' dtype) scale each head;
    "post_channel" gates first and LayerNorms all C after."""
    d = act.shape[-1] // h
    w = p["norm_center.weight"]
    bias = p.get("norm_center.bias")

    def gates() -> torch.Tensor:
        r = router_logits.float()
        return float(h) * torch.softmax(r, dim=-1) if router_kind == "softmax" else 2.0 * torch.sigmoid(r)

    if head_norm == "post_channel":
        t = act.unflatten(-1, (h, d))
        if router_logits is not None:
            t = t * gates().to(t.dtype).unsqueeze(-1)
        return layer_norm(t.flatten(-2), w, bias, eps)
    if head_norm == "channel":
        t = layer_norm(act, w, bias, eps).unflatten(-1, (h, d))
    else:
        t32 = act.unflatten(-1, (h, d)).float()
        if head_norm == "head_rms":
            t = (t32 * torch.rsqrt(t32.pow(2).mean(-1, keepdim=True) + eps)).to(act.dtype) * w.view(h, d)
        else:  # head_ln
            mu = t32.mean(-1, keepdim=True)
            t32 = (t32 - mu) * torch.rsqrt(t32.var(-1, keepdim=True, unbiased=False) + eps)
            t = t32.to(act.dtype) * w.view(h, d) + bias.view(h, d)
    if router_logits is not None:
        t = t * gates().to(t.dtype).unsqueeze(-1)
    return t.flatten(-2)


def _grid_attention_rows(
    z_flat: torch.Tensor,
    pb: torch.Tensor,
    mask: torch.Tensor,
    p: dict[str, torch.Tensor],
    B: int,
    N_rows: int,
    N_cols: int,
    H: int,
    D: int,
) -> torch.Tensor:
    """``GridSelfAttention._compute_baseline`` (``attention.py:143-165``)."""
    scale = D**-0.5
    q = F.linear(z_flat, p["to_q.weight"]).view(B * N_rows, N_cols, H, D).permute(0, 2, 1, 3)
    k = F.linear(z_flat, p["to_k.weight"]).view(B * N_rows, N_cols, H, D).permute(0, 2, 1, 3)
    v = F.linear(z_flat, p["to_v.weight"]).view(B * N_rows, N_cols, H, D).permute(0, 2, 1, 3).contiguous()
    logits = torch.matmul(q, k.transpose(-2, -1).contiguous()) * scale
    logits = logits.view(B, N_rows, H, N_cols, N_cols)
    logits = logits + pb.unsqueeze(1)
    logits = logits.reshape(B * N_rows, H, N_cols, N_cols)
    mask_flat = mask.reshape(B * N_rows, N_cols)
    logits = logits + 1e9 * (mask_flat.float() - 1.0).view(B * N_rows, 1, 1, N_cols)
    w = F.softmax(logits.float(), dim=-1).to(z_flat.dtype)
    del logits
    out = torch.matmul(w, v)
    out = out.permute(0, 2, 1, 3).reshape(B * N_rows, N_cols, H * D)
    g = torch.sigmoid(F.linear(z_flat, p["to_g.weight"]))
    return F.linear(out * g, p["out_proj.weight"])


def grid_attention(
    z: torch.Tensor,
    mask: torch.Tensor,
    p: dict[str, torch.Tensor],
    transpose: bool,
    num_heads: int | None = None,
    row_chunk: int = 0,
    lines: torch.Tensor | None = None,
) -> torch.Tensor:
    """Stock ``GridSelfAttention.forward`` (``attention.py:167-269``, no fused kernels).

    The pair bias comes from the un-transposed LN(z) (``attention.py:204-209``);
    column mode transposes LN(z) and the mask, attends, and transposes back.
    ``row_chunk`` evaluates that many rows at a time (rows are independent,
    so it is exact) to bound the fp32 logits. ``lines`` (indices into the
    attended axis: rows of z, or columns when ``transpose``) evaluates only
    those lines and returns ``[B, len(lines), N, C]`` in the attention frame.
    The head count defaults to the rows of the pair-bias weight (one per head).
    """
    B, N, _, C = z.shape
    H = num_heads if num_heads is not None else p["pair_bias.weight"].shape[0]  # one bias row per head
    D = max(C // H, 16)
    zn = layer_norm(z, p["norm.weight"], p["norm.bias"])
    pb = F.linear(zn, p["pair_bias.weight"]).permute(0, 3, 1, 2)  # [B, H, N, N]
    if transpose:
        zn = zn.permute(0, 2, 1, 3)
        mask = mask.permute(0, 2, 1)
    if lines is not None:
        zn = zn[:, lines]
        mask = mask[:, lines]
    N_rows, N_cols = zn.shape[1], zn.shape[2]
    chunk = row_chunk if row_chunk > 0 else N_rows
    outs = []
    for r0 in range(0, N_rows, chunk):
        r1 = min(N_rows, r0 + chunk)
        rows = zn[:, r0:r1].reshape(B * (r1 - r0), N_cols, C)
        o = _grid_attention_rows(rows, pb, mask[:, r0:r1], p, B, r1 - r0, N_cols, H, D)
        outs.append(o.view(B, r1 - r0, N_cols, -1))
    out = torch.cat(outs, dim=1) if len(outs) > 1 else outs[0]
    if transpose and lines is None:
        out = out.permute(0, 2, 1, 3)
    return out


def transition(x: torch.Tensor, p: dict[str, torch.Tensor]) -> torch.Tensor:
    """``TransitionBlock.forward`` (``primitives.py:193-251``): SwiGLU on contiguous halves."""
    h = layer_norm(x, p["norm.weight"], p["norm.bias"])
    h = F.linear(h, p["linear1.weight"])
    a, b = h.chunk(2, dim=-1)
    return F.linear(F.silu(a) * b, p["linear2.weight"])


def single_to_pair(z: torch.Tensor, p: dict[str, torch.Tensor]) -> torch.Tensor:
    """``single_to_pair(single_to_pair_norm(z)).movedim(-1, -3)`` (``evoformer.py:322-328``)."""
    zn = layer_norm(z, p["single_to_pair_norm.weight"], p["single_to_pair_norm.bias"])
    return F.linear(zn, p["single_to_pair.weight"]).movedim(-1, -3)


def single_attention(
    s: torch.Tensor, seq_mask: torch.Tensor, pair_logits: torch.Tensor, p: dict[str, torch.Tensor], num_heads: int = 16
) -> torch.Tensor:
    """``SingleAttention.forward`` (``attention.py:415-452``). With ``pair_bias_gate_a`` in ``p``
    (the per-head pair-bias gate, ``attention.py:392-398``) the pair logits of head h are
    multiplied by tau_h = exp(a_h), cast to their dtype, before they join q k^T
    (``attention.py:422-424``)."""
    B, N, C = s.shape
    H = num_heads
    Dk = p["to_q.weight"].shape[0] // H
    Dv = p["to_v.weight"].shape[0] // H
    xn = layer_norm(s, p["norm.weight"], p["norm.bias"])
    q = F.linear(xn, p["to_q.weight"], p["to_q.bias"]).view(B, N, H, Dk).permute(0, 2, 1, 3)
    k = F.linear(xn, p["to_k.weight"]).view(B, N, H, Dk).permute(0, 2, 1, 3)
    v = F.linear(xn, p["to_v.weight"]).view(B, N, H, Dv).permute(0, 2, 1, 3).contiguous()
    logits = torch.matmul(q * Dk**-0.5, k.transpose(-2, -1).contiguous())
    if "pair_bias_gate_a" in p:
        pair_logits = pair_logits * torch.exp(p["pair_bias_gate_a"]).to(pair_logits.dtype).view(1, H, 1, 1)
    logits = logits + pair_logits
    logits = logits + (1e9 * (seq_mask.float() - 1.0)).view(B, 1, 1, N)
    w = F.softmax(logits.float(), dim=-1).to(xn.dtype)
    out = torch.matmul(w, v).permute(0, 2, 1, 3).reshape(B, N, H * Dv)
    g = torch.sigmoid(F.linear(xn, p["to_g.weight"]))
    return F.linear(out * g, p["out_proj.weight"])


def rms_normalize(x: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """Non-learnable RMSNorm over the last axis (``primitives.py:79-87``): ``x / sqrt(mean x^2 +
    eps)``, the reference's ``F.rms_norm`` with no weight."""
    return F.rms_norm(x, (x.shape[-1],), eps=eps)


def _scaled(x: torch.Tensor, s: float) -> torch.Tensor:
    """``s * x``; a unit scale returns ``x`` itself (the same values, one pass fewer)."""
    return x if s == 1.0 else s * x


def pairformer_block(
    pair: torch.Tensor,
    single: torch.Tensor,
    pair_mask: torch.Tensor,
    seq_mask: torch.Tensor,
    p: dict[str, torch.Tensor],
    row_chunk: int = 0,
    branches: dict[str, torch.Tensor] | None = None,
    scales: dict | None = None,
    use_triangle_attention: bool = True,
    use_single_track: bool = True,
    dropout: dict[str, torch.Tensor] | None = None,
    branch_scaler: str = "identity",
    trimul_kwargs: dict | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """``PairFormerBlock.forward`` (``evoformer.py:270-355``).

    ``trimul_kwargs`` (num_heads, head_norm, router, router_kind) go to both triangle
    multiplies (``evoformer.py:85-92``, the MHR variants of ``tri_mul``).

    ``branch_scaler`` "identity" (AF3) or "rmsnorm" (each branch output made unit-RMS per
    token before its scale, ``branch_scaler.py:38-50``). Eval dropout-add is a plain add (``dropout_add.py:236-237``);
    ``dropout`` (training mode) maps the four dropped sites ``tri_mul_out``, ``tri_mul_in``,
    ``pair_attn_row`` (row-shared masks) and ``pair_attn_col`` (column-shared) to their masks
    (see ``dropout_add``), applied as at ``evoformer.py:289-310``; the transitions and the single
    track take no dropout. ``use_triangle_attention=False`` deletes the two attention branches
    (``:302-310``), ``use_single_track=False`` the single update (``:321-353``; single is returned
    unchanged). ``scales`` may hold ``residual_out_scale`` (s_ros, every branch) and
    ``pair_transition_residual_gain`` / ``single_transition_residual_gain`` (None = 1, the
    transitions' extra factor), applied to each branch output as at ``evoformer.py:282-353``.
    If ``branches`` is a dict, each unscaled branch output is stored in it under the
    reference submodule name.
    """
    sc = scales or {}
    s_ros = float(sc.get("residual_out_scale", 1.0))
    g_pf = sc.get("pair_transition_residual_gain")
    g_sf = sc.get("single_transition_residual_gain")
    s_pf = s_ros * (1.0 if g_pf is None else float(g_pf))
    s_sf = s_ros * (1.0 if g_sf is None else float(g_sf))
    drop = dropout or {}
    if branch_scaler not in ("identity", "rmsnorm"):
        raise ValueError(f"branch_scaler {branch_scaler!r}")
    # The branch scaler before each branch's scale (evoformer.py:289-335): identity, or the
    # non-learnable unit-RMS rows of branch_scaler.py:38-50 (primitives.py:79-87, eps 1e-6).
    sc_fn = (lambda x: x) if branch_scaler == "identity" else rms_normalize

    def add(res: torch.Tensor, upd: torch.Tensor, site: str) -> torch.Tensor:
        return dropout_add(res, upd, drop[site]) if site in drop else res + upd

    out: dict[str, torch.Tensor] = {}
    tk = trimul_kwargs or {}
    out["tri_mul_out"] = tri_mul(pair, pair_mask, _sub(p, "tri_mul_out."), outgoing=True, **tk)
    pair = add(pair, _scaled(sc_fn(out["tri_mul_out"]), s_ros), "tri_mul_out")
    out["tri_mul_in"] = tri_mul(pair, pair_mask, _sub(p, "tri_mul_in."), outgoing=False, **tk)
    pair = add(pair, _scaled(sc_fn(out["tri_mul_in"]), s_ros), "tri_mul_in")
    if use_triangle_attention:
        row = grid_attention(pair, pair_mask, _sub(p, "pair_attn_row."), transpose=False, row_chunk=row_chunk)
        pair = add(pair, _scaled(sc_fn(row), s_ros), "pair_attn_row")
        col = grid_attention(pair, pair_mask, _sub(p, "pair_attn_col."), transpose=True, row_chunk=row_chunk)
        pair = add(pair, _scaled(sc_fn(col), s_ros), "pair_attn_col")
        out.update(pair_attn_row=row, pair_attn_col=col)
    out["pair_transition"] = transition(pair, _sub(p, "pair_transition."))
    pair = pair + _scaled(sc_fn(out["pair_transition"]), s_pf)
    if use_single_track:
        out["pair_logits"] = single_to_pair(pair, p)
        out["single_attn"] = single_attention(single, seq_mask, out["pair_logits"], _sub(p, "single_attn."))
        single = single + _scaled(sc_fn(out["single_attn"]), s_ros)
        out["single_transition"] = transition(single, _sub(p, "single_transition."))
        single = single + _scaled(sc_fn(out["single_transition"]), s_sf)
    if branches is not None:
        branches.update(out)
    return pair, single


def template_pairformer_block(
    pair: torch.Tensor,
    pair_mask: torch.Tensor,
    p: dict[str, torch.Tensor],
    row_chunk: int = 0,
    residual_out_scale: float = 1.0,
    dropout: dict[str, torch.Tensor] | None = None,
) -> torch.Tensor:
    """``TemplatePairFormerBlock.forward`` (``template_embedding.py:220-240``):
    the five pair branches of the PairFormer block in the same order, the transition with
    its own intermediate factor (read from the weights), every branch output-scaled by
    ``residual_out_scale``; ``dropout`` as in ``pairformer_block`` (eval when None)."""
    s = float(residual_out_scale)
    drop = dropout or {}

    def add(res: torch.Tensor, upd: torch.Tensor, site: str) -> torch.Tensor:
        return dropout_add(res, upd, drop[site]) if site in drop else res + upd

    pair = add(pair, _scaled(tri_mul(pair, pair_mask, _sub(p, "tri_mul_out."), outgoing=True), s), "tri_mul_out")
    pair = add(pair, _scaled(tri_mul(pair, pair_mask, _sub(p, "tri_mul_in."), outgoing=False), s), "tri_mul_in")
    row = grid_attention(pair, pair_mask, _sub(p, "pair_attn_row."), transpose=False, row_chunk=row_chunk)
    pair = add(pair, _scaled(row, s), "pair_attn_row")
    col = grid_attention(pair, pair_mask, _sub(p, "pair_attn_col."), transpose=True, row_chunk=row_chunk)
    pair = add(pair, _scaled(col, s), "pair_attn_col")
    return pair + _scaled(transition(pair, _sub(p, "pair_transition.")), s)


def pairformer_trunk(
    pair: torch.Tensor,
    single: torch.Tensor,
    pair_mask: torch.Tensor,
    seq_mask: torch.Tensor,
    blocks: list[dict[str, torch.Tensor]],
    row_chunk: int = 0,
    scales: list[dict] | None = None,
    dropout: list[dict] | None = None,
    **block_flags,
) -> tuple[torch.Tensor, torch.Tensor]:
    """The trunk loop (``evoformer.py:593-601``) without checkpointing or meters;
    ``scales[i]`` are block i's residual scales and ``dropout[i]`` its masks (see
    ``pairformer_block``, which also takes ``block_flags``)."""
    for i, p in enumerate(blocks):
        sc = None if scales is None else scales[i]
        dr = None if dropout is None else dropout[i]
        pair, single = pairformer_block(
            pair, single, pair_mask, seq_mask, p, row_chunk=row_chunk, scales=sc, dropout=dr, **block_flags
        )
    return pair, single


def recycle_embed(
    pair_init: torch.Tensor,
    single_init: torch.Tensor,
    prev_pair: torch.Tensor,
    prev_single: torch.Tensor,
    p: dict[str, torch.Tensor],
) -> tuple[torch.Tensor, torch.Tensor]:
    """The recycling embeddings (``evoformer.py:520-526`` and ``:558-561``):
    ``pair_init + LinearNoBias(LN(prev_pair))`` with keys ``prev_embedding_layer_norm.*`` /
    ``prev_embedding.weight``; the single track likewise with ``prev_single_embedding*``
    when those keys are present (``use_single_track``)."""
    pair = pair_init + F.linear(
        layer_norm(prev_pair, p["prev_embedding_layer_norm.weight"], p["prev_embedding_layer_norm.bias"]),
        p["prev_embedding.weight"],
    )
    single = single_init
    if "prev_single_embedding.weight" in p:
        single = single_init + F.linear(
            layer_norm(
                prev_single, p["prev_single_embedding_layer_norm.weight"], p["prev_single_embedding_layer_norm.bias"]
            ),
            p["prev_single_embedding.weight"],
        )
    return pair, single


def recycled_trunk(
    pair_init: torch.Tensor,
    single_init: torch.Tensor,
    pair_mask: torch.Tensor,
    seq_mask: torch.Tensor,
    recycle_p: dict[str, torch.Tensor],
    blocks: list[dict[str, torch.Tensor]],
    num_recycles: int,
    scales: list[dict] | None = None,
    row_chunk: int = 0,
) -> tuple[torch.Tensor, torch.Tensor]:
    """The recycle loop around the trunk (``model.py:385-470``) with the stages between the
    recycling embedding and the trunk left out: previous outputs start at zero
    (``model.py:315-319``) and feed the next pass (``:468-470``)."""
    prev_pair, prev_single = torch.zeros_like(pair_init), torch.zeros_like(single_init)
    pair = single = None
    for _ in range(num_recycles + 1):
        pair, single = recycle_embed(pair_init, single_init, prev_pair, prev_single, recycle_p)
        pair, single = pairformer_trunk(pair, single, pair_mask, seq_mask, blocks, row_chunk=row_chunk, scales=scales)
        prev_pair, prev_single = pair, single
    return pair, single


def outer_product_mean(msa: torch.Tensor, mask: torch.Tensor, p: dict[str, torch.Tensor]) -> torch.Tensor:
    """``OuterProductMean.forward`` (``ops.py:683-785``): a, b = proj(LN(msa)) * mask,
    ``ab[i,j,e,f] = sum_s a[s,i,e] b[s,j,f]``, ``act = ab . out_w + out_b``, divided by
    ``1e-3 + sum_s m[s,i] m[s,j]``. msa [B, S, N, c_msa], mask [B, S, N] -> [B, N, N, c_z]."""
    m = mask.unsqueeze(-1)
    x = layer_norm(msa, p["norm.weight"], p["norm.bias"])
    a = F.linear(x, p["proj_a.weight"]) * m
    b = F.linear(x, p["proj_b.weight"]) * m
    ab = torch.einsum("bsie,bsjf->bijef", a, b)
    act = torch.einsum("bijef,efc->bijc", ab, p["out_w"]) + p["out_b"]
    mf = mask.float()
    norm = torch.einsum("bsi,bsj->bij", mf, mf)
    return act / (1e-3 + norm.unsqueeze(-1))


def msa_attention(
    msa: torch.Tensor, mask: torch.Tensor, pair: torch.Tensor, p: dict[str, torch.Tensor], num_heads: int = 8
) -> torch.Tensor:
    """``MSAAttention`` (``attention.py:272-341``): pair-weighted averaging. The weights
    ``softmax_k(LN(pair) W_h + 1e9 (colmask_k - 1))`` (colmask = max over sequences of the
    mask, softmax in fp32, cast to msa's dtype) are shared by every MSA row; each row averages
    its values ``to_v(LN(msa))`` with them, gated by ``sigmoid(to_g(LN(msa)))``, then out_proj.
    msa [B, S, N, c_msa], mask [B, S, N], pair [B, N, N, c_pair] -> [B, S, N, c_msa]."""
    B, S, N, C = msa.shape
    H = num_heads
    D = C // H
    logits = F.linear(layer_norm(pair, p["pair_norm.weight"], p["pair_norm.bias"]), p["pair_logits.weight"])
    logits = logits.permute(0, 3, 1, 2)  # [B, H, q, k]
    col_mask, _ = mask.max(dim=-2)
    logits = logits + 1e9 * (col_mask.float() - 1.0).view(B, 1, 1, N)
    w = F.softmax(logits.float(), dim=-1)
    x = layer_norm(msa, p["norm.weight"], p["norm.bias"])
    w = w.to(x.dtype)
    v = F.linear(x, p["to_v.weight"]).view(B, S, N, H, D)
    v_avg = torch.einsum("bhqk,bskhc->bsqhc", w, v).reshape(B, S, N, H * D)
    g = torch.sigmoid(F.linear(x, p["to_g.weight"]))
    return F.linear(v_avg * g, p["out_proj.weight"])


def evoformer_block(
    msa: torch.Tensor,
    pair: torch.Tensor,
    msa_mask: torch.Tensor,
    pair_mask: torch.Tensor,
    p: dict[str, torch.Tensor],
    num_msa_heads: int = 8,
    residual_out_scale: float = 1.0,
    row_chunk: int = 0,
    use_triangle_attention: bool = True,
    dropout: dict[str, torch.Tensor] | None = None,
    trimul_kwargs: dict | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """``EvoformerBlock.forward`` (``evoformer.py:148-175``): pair += OPM(msa),
    msa += MSAAttention(msa, pair), msa += msa_transition(msa), then the pair half of the
    PairFormer block (trimul out, in, attention rows, columns unless
    ``use_triangle_attention=False``, pair transition); every branch output-scaled by
    ``residual_out_scale``. ``dropout`` (training) maps ``row_attn`` (msa, row-shared) and the
    four pair sites of ``pairformer_block`` to their masks; None is eval."""
    s = float(residual_out_scale)
    drop = dropout or {}

    def add(res: torch.Tensor, upd: torch.Tensor, site: str) -> torch.Tensor:
        return dropout_add(res, upd, drop[site]) if site in drop else res + upd

    pair = pair + _scaled(outer_product_mean(msa, msa_mask, _sub(p, "outer_product.")), s)
    msa = add(msa, _scaled(msa_attention(msa, msa_mask, pair, _sub(p, "row_attn."), num_msa_heads), s), "row_attn")
    msa = msa + _scaled(transition(msa, _sub(p, "msa_transition.")), s)
    tk = trimul_kwargs or {}
    pair = add(pair, _scaled(tri_mul(pair, pair_mask, _sub(p, "tri_mul_out."), outgoing=True, **tk), s), "tri_mul_out")
    pair = add(pair, _scaled(tri_mul(pair, pair_mask, _sub(p, "tri_mul_in."), outgoing=False, **tk), s), "tri_mul_in")
    if use_triangle_attention:
        row = grid_attention(pair, pair_mask, _sub(p, "pair_attn_row."), transpose=False, row_chunk=row_chunk)
        pair = add(pair, _scaled(row, s), "pair_attn_row")
        col = grid_attention(pair, pair_mask, _sub(p, "pair_attn_col."), transpose=True, row_chunk=row_chunk)
        pair = add(pair, _scaled(col, s), "pair_attn_col")
    pair = pair + _scaled(transition(pair, _sub(p, "pair_transition.")), s)
    return msa, pair


def evo_attention(
    Q: torch.Tensor,
    K: torch.Tensor,
    V: torch.Tensor,
    res_mask: torch.Tensor,
    pair_bias: torch.Tensor,
    zero_rows: bool = True,
) -> torch.Tensor:
    """The fused attention op in its kernel layout (``_attn_fwd``, ``triton/evo_attention.py:34-135``,
    ``:179-333``): Q, K, V [B,S,H,N,D], res_mask [B,S,1,1,N] additive, pair_bias [B,1,H,N,N];
    softmax(Q K^T D^-1/2 + pair_bias + res_mask) V, softmax over keys. A query row whose
    logits all sit below -1e8 outputs 0 (``zero_rows``, the kernel's rule, ``:307-318``) or
    the mean of V (the stock fp32 path, whose -1e9 logits round to one value)."""
    D = Q.shape[-1]
    logits = torch.matmul(Q, K.transpose(-1, -2).contiguous()) * D**-0.5 + pair_bias + res_mask
    dead = logits.amax(dim=-1, keepdim=True) < -1e8
    out = torch.matmul(torch.softmax(logits, dim=-1), V)
    fill = torch.zeros_like(out) if zero_rows else V.mean(dim=-2, keepdim=True).expand_as(out)
    return torch.where(dead, fill, out)


def evo_attention_backward(
    Q: torch.Tensor, K: torch.Tensor, V: torch.Tensor, res_mask: torch.Tensor, pair_bias: torch.Tensor,
    dO: torch.Tensor,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """Gradients of ``evo_attention(zero_rows=True)`` in the centred form of the reference's
    backward (``_attn_bwd_d`` / ``_dq`` / ``_dk_dv`` / ``_db``, ``triton/evo_attention.py:335-1195``;
    ``docs/optimizations.md:417-483``): per row, imax = first argmax of the logits,
    u_j = dP_j - dP_imax (0 at imax), C = sum_j P_j u_j, dS = P (u - C). Returns dQ, dK, dV
    [B,S,H,N,D] and d_pair_bias [B,1,H,N,N] (dS summed over S)."""
    D = Q.shape[-1]
    scale = D**-0.5
    t = torch.matmul(Q, K.transpose(-1, -2).contiguous()) * scale + pair_bias + res_mask
    dead = t.amax(dim=-1, keepdim=True) < -1e8
    P = torch.where(dead, torch.zeros_like(t), torch.softmax(t, dim=-1))
    dP = torch.matmul(dO, V.transpose(-1, -2).contiguous())
    imax = t.argmax(dim=-1, keepdim=True)
    u = dP - dP.gather(-1, imax)
    u = u.scatter(-1, imax, torch.zeros_like(imax, dtype=u.dtype))
    C = (P * u).sum(dim=-1, keepdim=True)
    dS = P * (u - C)
    dQ = torch.matmul(dS, K) * scale
    dK = torch.matmul(dS.transpose(-1, -2).contiguous(), Q) * scale
    dV = torch.matmul(P.transpose(-1, -2).contiguous(), dO)
    return dQ, dK, dV, dS.sum(dim=1, keepdim=True)


def tri_mul_core(
    x: torch.Tensor,
    mask: torch.Tensor,
    w_gate: torch.Tensor,
    w_proj: torch.Tensor,
    ln_out_w: torch.Tensor,
    ln_out_b: torch.Tensor,
    w_out: torch.Tensor,
    w_out_gate: torch.Tensor,
    eps: float,
    outgoing: bool,
    w_router: torch.Tensor | None = None,
    num_heads: int = 0,
    head_norm: str = "channel",
    router_kind: str = "softmax",
) -> torch.Tensor:
    """``FusedTriMulFunction.forward`` (``triton/fused_trimul.py:285-296``, kernels ``:64-151``,
    ``:264-281``): x = norm_left(z) given; ``w_gate``, ``w_proj`` [2C, C] in block order
    (rows [a; b]); a | b = sigmoid(x Wg^T) (x Wp^T) mask; X_ij = sum_k a_ik b_jk (outgoing) or
    sum_k a_ki b_kj (incoming); out = sigmoid(x Wog^T) (LN(X) Wo^T). Differentiable. With
    ``num_heads`` and a per-head norm or ``w_router`` [H, C], LN(X) is the MHR head mix
    (``mhr_head_mix``) with router logits x Wr^T (``ops.py:412-473``)."""
    C = x.shape[-1]
    ab = torch.sigmoid(F.linear(x, w_gate)) * F.linear(x, w_proj) * mask.unsqueeze(-1)
    a, b = ab[..., :C], ab[..., C:]
    if outgoing:
        X = torch.einsum("bikc,bjkc->bijc", a, b)
    else:
        X = torch.einsum("bkic,bkjc->bijc", a, b)
    if head_norm != "channel" or w_router is not None:
        affine = {"norm_center.weight": ln_out_w}
        if ln_out_b is not None:
            affine["norm_center.bias"] = ln_out_b
        r = None if w_router is None else F.linear(x, w_router)
        xln = mhr_head_mix(X, r, affine, num_heads, head_norm, router_kind, eps)
    else:
        xln = F.layer_norm(X, (C,), ln_out_w, ln_out_b, eps)
    return torch.sigmoid(F.linear(x, w_out_gate)) * F.linear(xln, w_out)


# ---------------------------------------------------------------- training-mode dropout
# Philox4x32 constants (Salmon, Moraes, Dror, Shaw, "Parallel random numbers: as easy as
# 1, 2, 3", SC 2011): round multipliers and Weyl key increments.
_PHILOX_M = (0xD2511F53, 0xCD9E8D57)
_PHILOX_W = (0x9E3779B9, 0xBB67AE85)


def philox4x32_10(counter: np.ndarray, key: tuple[int, int]) -> np.ndarray:
    """Philox4x32 with 10 rounds on ``counter`` [n, 4] uint32 words under ``key`` (two uint32
    words); returns [n, 4] uint32. Each round: (hi0, lo0) = M0 * c0, (hi1, lo1) = M1 * c2
    (64-bit products), c = (hi1 ^ c1 ^ k0, lo1, hi0 ^ c3 ^ k1, lo0); the key gains
    (W0, W1) after every round. Pinned by the published known-answer vectors."""
    c = [counter[:, i].astype(np.uint64) for i in range(4)]
    k0, k1 = np.uint64(key[0] & 0xFFFFFFFF), np.uint64(key[1] & 0xFFFFFFFF)
    m0, m1 = np.uint64(_PHILOX_M[0]), np.uint64(_PHILOX_M[1])
    lo32 = np.uint64(0xFFFFFFFF)
    for _ in range(10):
        p0, p1 = m0 * c[0], m1 * c[2]  # < 2^64: no overflow
        hi0, lo0 = p0 >> np.uint64(32), p0 & lo32
        hi1, lo1 = p1 >> np.uint64(32), p1 & lo32
        c = [hi1 ^ c[1] ^ k0, lo1, hi0 ^ c[3] ^ k1, lo0]
        k0 = (k0 + np.uint64(_PHILOX_W[0])) & lo32
        k1 = (k1 + np.uint64(_PHILOX_W[1])) & lo32
    return np.stack(c, axis=1).astype(np.uint32)


def dropout_mask(n: int, p: float, seed: int) -> torch.Tensor:
    """The n mask entries of a seed (fp32, 0 or 1/(1-p)): entry i keeps when
    u_i = (word i % 4 of Philox4x32-10(counter = i // 4 as a 64-bit word in the first two
    lanes, key = seed) >> 8) * 2^-24 is >= p, the keep rule of ``dropout_add.py:91-94``."""
    q = np.arange((n + 3) // 4, dtype=np.uint64)
    ctr = np.zeros((q.size, 4), dtype=np.uint32)
    ctr[:, 0] = (q & np.uint64(0xFFFFFFFF)).astype(np.uint32)
    ctr[:, 1] = (q >> np.uint64(32)).astype(np.uint32)
    words = philox4x32_10(ctr, (seed & 0xFFFFFFFF, (seed >> 32) & 0xFFFFFFFF)).reshape(-1)[:n]
    u = (words >> np.uint32(8)).astype(np.float32) * np.float32(2.0**-24)
    p32 = np.float32(p)
    scale = np.float32(1.0) / (np.float32(1.0) - p32)
    return torch.from_numpy(np.where(u >= p32, scale, np.float32(0.0)).astype(np.float32))


def shared_dropout_mask(shape: tuple[int, ...], rowwise: bool, p: float, seed: int) -> torch.Tensor:
    """The broadcastable mask of a [B, R, Cc, D] activation: [B, 1, Cc, D] shared along R
    (``dropout_add_rowwise``, share dim -3) or [B, R, 1, D] shared along Cc (columnwise, share
    dim -2), entries in the index order of ``dropout_add.py:81-88``."""
    B, R, Cc, D = shape
    mshape = (B, 1, Cc, D) if rowwise else (B, R, 1, D)
    n = B * (Cc if rowwise else R) * D
    return dropout_mask(n, p, seed).view(mshape)


def dropout_add(residual: torch.Tensor, x: torch.Tensor, mask: torch.Tensor) -> torch.Tensor:
    """Training-mode dropout-add with a given shared mask (``dropout_add.py:57-99``, the fused
    kernel): ``residual + x * mask`` in fp32, rounded once to the residual's dtype."""
    return (residual.float() + x.float() * mask.float()).to(residual.dtype)
