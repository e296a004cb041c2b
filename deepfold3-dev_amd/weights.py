"""Deterministic synthetic weights and inputs for the PairFormer hot path.

State-dict keys and shapes follow the reference ``PairFormerBlock``
(``src/deepfold3/model/evoformer.py:187-268``; keys listed in
``ops.py:219-231``, ``attention.py:71-78``, ``attention.py:382-408``,
``primitives.py:219-227``, ``evoformer.py:237-238``), so a state dict made here
loads into the reference module with ``load_state_dict(strict=True)``.

Weight recipe ("LeCun truncated normal"): every Linear weight, including the
ones the reference zero-initialises (gate, out_proj, out_gate, to_g, linear2),
is drawn from N(0, 1/fan_in) truncated at +-2 sigma. The reference's own
``af3_linear_init_`` (``primitives.py:47-61``) truncates at +-2 *absolute* and
divides the std by 0.8796; this generator does not follow it on purpose: the
reference init zeroes the output projections, which would make every parity
comparison vacuous.

LayerNorm weight is 1 and bias 0 and ``single_attn.to_q.bias`` is 0 unless
``perturb_affine`` is set, in which case they become 1 + 0.1 n, 0.1 n and 0.1 n
(n ~ N(0, 1)), so that a swapped or dropped affine term changes the output.

RNG stream: one CPU ``torch.Generator`` seeded with ``seed``; entries are drawn
in the order of :func:`block_param_spec`, one tensor at a time.
"""

from __future__ import annotations

import hashlib
import math

import torch

C_PAIR = 128
C_SINGLE = 384
NUM_PAIR_HEADS = 4
NUM_SINGLE_HEADS = 16
TRANSITION_FACTOR = 4


def block_param_spec(
    c_pair: int = C_PAIR,
    c_single: int = C_SINGLE,
    num_pair_heads: int = NUM_PAIR_HEADS,
    num_single_heads: int = NUM_SINGLE_HEADS,
    single_key_dim: int = C_SINGLE,
    single_value_dim: int = C_SINGLE,
    factor: int = TRANSITION_FACTOR,
    use_triangle_attention: bool = True,
    use_single_track: bool = True,
    pair_bias_gate: bool = False,
    trimul_num_heads: int = 0,
    trimul_head_norm: str = "channel",
    trimul_router: bool = False,
) -> list[tuple[str, tuple[int, ...], str]]:
    """Ordered ``(key, shape, kind)`` for one PairFormerBlock; kind is ln_w, ln_b, linear, bias
    or log_tau (the single attention's per-head pair-bias gate, ``attention.py:392-398``,
    initialised to log 0.25). A block without triangle attention has no ``pair_attn_*`` keys,
    one without the single track no ``single_*`` keys (``evoformer.py:226-249``). The MHR
    triangle multiply (``ops.py:219-255``) adds ``router.weight`` [H, C] with the router (drawn
    as a linear here, so routing is not uniform) and has no ``norm_center.bias`` for head_rms."""
    c, cs = c_pair, c_single
    spec: list[tuple[str, tuple[int, ...], str]] = []
    for p in ("tri_mul_out.", "tri_mul_in."):
        spec += [
            (p + "norm_left.weight", (c,), "ln_w"),
            (p + "norm_left.bias", (c,), "ln_b"),
            (p + "proj.weight", (2 * c, c), "linear"),
            (p + "gate.weight", (2 * c, c), "linear"),
            (p + "norm_center.weight", (c,), "ln_w"),
            *([(p + "norm_center.bias", (c,), "ln_b")] if trimul_head_norm != "head_rms" else []),
            (p + "out_proj.weight", (c, c), "linear"),
            (p + "out_gate.weight", (c, c), "linear"),
            *([(p + "router.weight", (trimul_num_heads, c), "linear")] if trimul_router else []),
        ]
    hd = max(c // num_pair_heads, 16)  # attention.py:67
    for p in ("pair_attn_row.", "pair_attn_col."):
        spec += [
            (p + "norm.weight", (c,), "ln_w"),
            (p + "norm.bias", (c,), "ln_b"),
            (p + "pair_bias.weight", (num_pair_heads, c), "linear"),
            (p + "to_q.weight", (num_pair_heads * hd, c), "linear"),
            (p + "to_k.weight", (num_pair_heads * hd, c), "linear"),
            (p + "to_v.weight", (num_pair_heads * hd, c), "linear"),
            (p + "to_g.weight", (num_pair_heads * hd, c), "linear"),
            (p + "out_proj.weight", (c, num_pair_heads * hd), "linear"),
        ]
    spec += [
        ("pair_transition.norm.weight", (c,), "ln_w"),
        ("pair_transition.norm.bias", (c,), "ln_b"),
        ("pair_transition.linear1.weight", (2 * factor * c, c), "linear"),
        ("pair_transition.linear2.weight", (c, factor * c), "linear"),
        ("single_to_pair_norm.weight", (c,), "ln_w"),
        ("single_to_pair_norm.bias", (c,), "ln_b"),
        ("single_to_pair.weight", (num_single_heads, c), "linear"),
        ("single_attn.norm.weight", (cs,), "ln_w"),
        ("single_attn.norm.bias", (cs,), "ln_b"),
        ("single_attn.to_q.weight", (single_key_dim, cs), "linear"),
        ("single_attn.to_q.bias", (single_key_dim,), "bias"),
        ("single_attn.to_k.weight", (single_key_dim, cs), "linear"),
        ("single_attn.to_v.weight", (single_value_dim, cs), "linear"),
        ("single_attn.to_g.weight", (single_value_dim, cs), "linear"),
        ("single_attn.out_proj.weight", (cs, single_value_dim), "linear"),
        *([("single_attn.pair_bias_gate_a", (num_single_heads,), "log_tau")] if pair_bias_gate else []),
        ("single_transition.norm.weight", (cs,), "ln_w"),
        ("single_transition.norm.bias", (cs,), "ln_b"),
        ("single_transition.linear1.weight", (2 * factor * cs, cs), "linear"),
        ("single_transition.linear2.weight", (cs, factor * cs), "linear"),
    ]
    if not use_triangle_attention:
        spec = [e for e in spec if not e[0].startswith("pair_attn_")]
    if not use_single_track:
        spec = [e for e in spec if not e[0].startswith("single_")]
    return spec


def lecun_trunc_normal_(t: torch.Tensor, gen: torch.Generator) -> torch.Tensor:
    """N(0, 1/fan_in) truncated at +-2 sigma, fan_in = t.shape[1]."""
    std = 1.0 / math.sqrt(t.shape[1])
    return torch.nn.init.trunc_normal_(t, 0.0, std, -2.0 * std, 2.0 * std, generator=gen)


def make_block_weights(seed: int, perturb_affine: bool = False, **spec_kwargs) -> dict[str, torch.Tensor]:
    """fp32 CPU state dict for one PairFormerBlock, drawn from ``seed``."""
    gen = torch.Generator().manual_seed(int(seed))
    out: dict[str, torch.Tensor] = {}
    for key, shape, kind in block_param_spec(**spec_kwargs):
        t = torch.empty(shape, dtype=torch.float32)
        if kind == "linear":
            lecun_trunc_normal_(t, gen)
        elif kind == "ln_w":
            t.fill_(1.0)
            if perturb_affine:
                t.add_(0.1 * torch.randn(shape, generator=gen))
        elif kind == "log_tau":
            t.fill_(math.log(0.25))
            if perturb_affine:
                t.add_(0.5 * torch.randn(shape, generator=gen))
        else:  # ln_b, bias
            t.zero_()
            if perturb_affine:
                t.add_(0.1 * torch.randn(shape, generator=gen))
        out[key] = t
    return out


def make_trunk_weights(seed: int, num_blocks: int, perturb_affine: bool = False,
                       **spec_kwargs) -> list[dict[str, torch.Tensor]]:  # fmt: skip
    """Per-block state dicts; block ``b`` is drawn from ``seed * 1000 + b``."""
    return [make_block_weights(seed * 1000 + b, perturb_affine, **spec_kwargs) for b in range(num_blocks)]


def evoformer_block_param_spec(
    c_msa: int = 64, c_pair: int = C_PAIR, num_msa_heads: int = 8, num_pair_heads: int = NUM_PAIR_HEADS,
    outer_product_hidden: int = 32, use_triangle_attention: bool = True,
) -> list[tuple[str, tuple[int, ...], str]]:
    """Ordered ``(key, shape, kind)`` for one EvoformerBlock (``evoformer.py:100-146``):
    the MSA parts, then the pair half of the PairFormer block (same keys; no ``pair_attn_*``
    without triangle attention)."""
    cm, cz, ch = c_msa, c_pair, outer_product_hidden
    spec: list[tuple[str, tuple[int, ...], str]] = [
        ("row_attn.norm.weight", (cm,), "ln_w"),
        ("row_attn.norm.bias", (cm,), "ln_b"),
        ("row_attn.pair_norm.weight", (cz,), "ln_w"),
        ("row_attn.pair_norm.bias", (cz,), "ln_b"),
        ("row_attn.pair_logits.weight", (num_msa_heads, cz), "linear"),
        ("row_attn.to_v.weight", (cm, cm), "linear"),
        ("row_attn.to_g.weight", (cm, cm), "linear"),
        ("row_attn.out_proj.weight", (cm, cm), "linear"),
        ("outer_product.norm.weight", (cm,), "ln_w"),
        ("outer_product.norm.bias", (cm,), "ln_b"),
        ("outer_product.proj_a.weight", (ch, cm), "linear"),
        ("outer_product.proj_b.weight", (ch, cm), "linear"),
        ("outer_product.out_w", (ch, ch, cz), "linear3"),
        ("outer_product.out_b", (cz,), "bias"),
    ]
    pair_keys = ("tri_mul_out.", "tri_mul_in.", "pair_attn_row.", "pair_attn_col.", "pair_transition.")
    spec += [
        e
        for e in block_param_spec(c_pair=cz, num_pair_heads=num_pair_heads, use_triangle_attention=use_triangle_attention)
        if e[0].startswith(pair_keys)
    ]
    spec += [
        ("msa_transition.norm.weight", (cm,), "ln_w"),
        ("msa_transition.norm.bias", (cm,), "ln_b"),
        ("msa_transition.linear1.weight", (2 * TRANSITION_FACTOR * cm, cm), "linear"),
        ("msa_transition.linear2.weight", (cm, TRANSITION_FACTOR * cm), "linear"),
    ]
    return spec


def make_evoformer_block_weights(seed: int, perturb_affine: bool = False, **spec_kwargs) -> dict[str, torch.Tensor]:
    """fp32 CPU state dict for one EvoformerBlock from ``seed``: LeCun truncated normal on every
    weight (``out_w`` [CH, CH, c_z] with fan-in CH^2), LayerNorm 1 / 0 and ``out_b`` 0 unless
    ``perturb_affine``."""
    gen = torch.Generator().manual_seed(int(seed))
    out: dict[str, torch.Tensor] = {}
    for key, shape, kind in evoformer_block_param_spec(**spec_kwargs):
        t = torch.empty(shape, dtype=torch.float32)
        if kind == "linear":
            lecun_trunc_normal_(t, gen)
        elif kind == "linear3":
            std = 1.0 / math.sqrt(shape[0] * shape[1])
            torch.nn.init.trunc_normal_(t, 0.0, std, -2.0 * std, 2.0 * std, generator=gen)
        elif kind == "ln_w":
            t.fill_(1.0)
            if perturb_affine:
                t.add_(0.1 * torch.randn(shape, generator=gen))
        else:
            t.zero_()
            if perturb_affine:
                t.add_(0.1 * torch.randn(shape, generator=gen))
        out[key] = t
    return out


def state_dict_sha256(sd: dict[str, torch.Tensor]) -> str:
    """sha256 over keys (sorted) and the little-endian fp32 bytes of each tensor."""
    h = hashlib.sha256()
    for k in sorted(sd):
        h.update(k.encode())
        h.update(sd[k].detach().to(torch.float32).contiguous().numpy().tobytes())
    return h.hexdigest()


def make_inputs(
    n: int,
    seed: int,
    batch: int = 1,
    c_pair: int = C_PAIR,
    c_single: int = C_SINGLE,
    pad_last: int = 0,
    pad_random: int = 0,
) -> dict[str, torch.Tensor]:
    """z ~ N(0,1) [B,N,N,Cz], s ~ N(0,1) [B,N,Cs] (drawn in that order), and the masks.

    ``seq_mask`` zeroes the last ``pad_last`` tokens and ``pad_random`` tokens
    picked from a permutation drawn after ``s``; ``pair_mask = seq (x) seq``,
    as the reference featurizer builds it (``data/feature/featurizer.py:520``).
    """
    gen = torch.Generator().manual_seed(int(seed))
    z = torch.randn(batch, n, n, c_pair, generator=gen)
    s = torch.randn(batch, n, c_single, generator=gen)
    seq = torch.ones(batch, n)
    if pad_last:
        seq[:, n - pad_last :] = 0.0
    if pad_random:
        for b in range(batch):
            idx = torch.randperm(n, generator=gen)[:pad_random]
            seq[b, idx] = 0.0
    pair = seq[:, :, None] * seq[:, None, :]
    return {"pair": z, "single": s, "pair_mask": pair, "seq_mask": seq}


# BASELINE.json configs (inputs only; config 3 and 5 are op-level).
CONFIGS = {
    1: dict(n=64, seed=0),
    2: dict(n=384, seed=1, pad_last=32),
    3: dict(n=1024, seed=2),
    4: dict(n=768, seed=3, pad_random=38),
    5: dict(n=2048, seed=4),
}
