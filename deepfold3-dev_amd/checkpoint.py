"""Reference checkpoints (``.safetensors``) into the HIP stacks.

The reference's inference entry reads the architecture from the ``model_cfg_json`` entry of
the safetensors metadata (``config.py:1895-1958``; read header-only at
``scripts/inference.py:488-500``; a file without it falls back to the config defaults) and
the weights by state-dict key. This module does the same for the parts built here:

- the trunk, ``evoformer.trunk_pairformer.{i}.*``, each block constructed as the
  reference's ``Evoformer`` constructs it from ``PairFormerConfig`` (``evoformer.py:459-489``,
  per-layer residual scales included);
- its recycling embeddings, ``evoformer.prev_*`` (``evoformer.py:400-412``);
- the confidence head's PairFormer layers, ``confidence_head.layers.{i}.*``, constructed
  from ``ConfidenceConfig`` (``confidence.py:88-117``);
- the MSA stack, ``evoformer.msa_stack.{i}.*``, constructed from ``EvoformerConfig``
  (``evoformer.py:433-455``).

Tensors are read one key at a time through safetensors' ``safe_open`` (nothing in the file
is executed, and only the keys under the requested prefix are read). A configuration this
build cannot serve (pair channels other than 64, 128 or 256, pair heads wider than 32)
refuses by name when the stack is constructed or first run; the off-by-default variants (MHR
triangle multiplication, the pair-bias gate, the RMSNorm branch scaler) are built. Stacks without triangle attention or without the single track (the
reference's current ``configs/stage0.yaml`` shape) are built without those branches. Loading
is strict within the prefix: a missing or unexpected key raises.
"""

from __future__ import annotations

import json
import math
import os

import torch

from .config import OptimConfig
from .evoformer import ConfidencePairFormer, EvoformerStack, PairFormerStack, TrunkRecycler

MODEL_CFG_KEY = "model_cfg_json"  # config.py:1898
TRUNK_PREFIX = "evoformer.trunk_pairformer."
RECYCLE_PREFIX = "evoformer."
CONFIDENCE_PREFIX = "confidence_head.layers."
MSA_STACK_PREFIX = "evoformer."

# PairFormerConfig defaults (config.py:122-269), the fields that shape a block.
PAIRFORMER_DEFAULTS: dict = {
    "num_layer": 48,
    "pair_channel": 128,
    "seq_channel": 384,
    "pair_attention": {"num_head": 4},
    "single_attention_num_head": 16,
    "single_key_dim": 384,
    "single_value_dim": 384,
    "pair_dropout": 0.25,
    "residual_output_scaling": False,
    "uniform_residual_scale": False,
    "pair_bias_gate": False,
    "pair_bias_gate_init_tau": 0.25,
    "single_transition_linear_out_init_gain": None,
    "single_transition_residual_gain": None,
    "single_transition_residual_per_layer_extra": False,
    "pair_transition_residual_gain": None,
    "pair_transition_residual_per_layer_extra": False,
    "branch_scaler": "identity",
    "use_triangle_attention": True,
    "trimul_num_heads": 0,
    "trimul_head_norm": "channel",
    "trimul_router": False,
    "trimul_router_kind": "softmax",
    "use_single_track": True,
}

# ConfidenceConfig defaults (config.py:578-615), the fields its PairFormer layers read.
CONFIDENCE_DEFAULTS: dict = {
    "num_layer": 4,
    "pair_channel": 128,
    "seq_channel": 384,
    "pair_attention_num_head": 4,
    "single_attention_num_head": 16,
    "residual_output_scaling": False,
    "uniform_residual_scale": False,
    "pair_bias_gate": False,
    "pair_bias_gate_init_tau": 0.25,
    "single_transition_linear_out_init_gain": None,
    "single_transition_residual_gain": None,
    "single_transition_residual_per_layer_extra": False,
    "pair_transition_residual_gain": None,
    "pair_transition_residual_per_layer_extra": False,
    "branch_scaler": "identity",
}


# EvoformerConfig defaults (config.py:71-121), the fields that shape an MSA-stack block.
EVOFORMER_DEFAULTS: dict = {
    "num_layer": 4,
    "msa_channel": 64,
    "pair_channel": 128,
    "msa_attention": {"num_head": 8},
    "outer_product_num_channel": 32,
    "pair_attention": {"num_head": 4},
    "msa_dropout": 0.15,
    "pair_dropout": 0.25,
    "residual_output_scaling": False,
    "uniform_residual_scale": False,
    "use_triangle_attention": True,
    "trimul_num_heads": 0,
    "trimul_head_norm": "channel",
    "trimul_router": False,
    "trimul_router_kind": "softmax",
}


def read_model_cfg(path: str | os.PathLike) -> dict | None:
    """The checkpoint's embedded ``ModelConfig`` as a plain dict, or None when the
    metadata has no ``model_cfg_json`` entry (``config.py:1914-1933``)."""
    from safetensors import safe_open

    with safe_open(str(path), framework="pt") as f:
        meta = f.metadata()
    if not meta or MODEL_CFG_KEY not in meta:
        return None
    cfg = json.loads(meta[MODEL_CFG_KEY])
    if not isinstance(cfg, dict):
        raise ValueError(f"{path}: {MODEL_CFG_KEY} does not hold a JSON object")
    return cfg


def _section(model_cfg: dict | None, name: str, defaults: dict) -> dict:
    """``defaults`` overridden by the known fields of ``model_cfg[name]`` (unknown fields are
    dropped, as the reference's loader drops them: ``config.py:1940-1956``)."""
    out = json.loads(json.dumps(defaults))
    given = (model_cfg or {}).get(name) or {}
    for k, v in given.items():
        if k not in out:
            continue
        if isinstance(out[k], dict) and isinstance(v, dict):
            out[k].update({kk: vv for kk, vv in v.items() if kk in out[k]})
        else:
            out[k] = v
    return out


def block_residual_scale(layer_idx: int, num_layer: int, per_layer: bool, uniform: bool) -> float:
    """Residual output scale of layer ``layer_idx`` (``primitives.py:20-44``): 1/sqrt(i+1)
    per layer, 1/sqrt(L) uniform, 1 otherwise; both set is an error."""
    if per_layer and uniform:
        raise ValueError("a stack takes either per-layer (residual_output_scaling) or uniform "
                         "(uniform_residual_scale) residual scales, not both")  # fmt: skip
    if per_layer:
        return 1.0 / math.sqrt(float(layer_idx + 1))
    if uniform:
        return 1.0 / math.sqrt(float(num_layer))
    return 1.0


def branch_residual_gain(layer_idx: int, base_gain: float | None, per_layer_extra: bool) -> float | None:
    """A transition's extra residual gain at layer ``layer_idx`` (``evoformer.py:66-82``):
    ``base · (1/sqrt(i+1) if per_layer_extra)``, None (= 1) when neither knob is set."""
    if base_gain is None and not per_layer_extra:
        return None
    g = 1.0 if base_gain is None else float(base_gain)
    if per_layer_extra:
        g /= math.sqrt(float(layer_idx + 1))
    return g


def _layer_scales(cfg: dict, i: int) -> dict:
    return dict(
        residual_out_scale=block_residual_scale(
            i, cfg["num_layer"], cfg["residual_output_scaling"], cfg["uniform_residual_scale"]
        ),
        single_transition_residual_gain=branch_residual_gain(
            i, cfg["single_transition_residual_gain"], cfg["single_transition_residual_per_layer_extra"]
        ),
        pair_transition_residual_gain=branch_residual_gain(
            i, cfg["pair_transition_residual_gain"], cfg["pair_transition_residual_per_layer_extra"]
        ),
    )


def trunk_config(model_cfg: dict | None) -> dict:
    """The trunk's ``PairFormerConfig`` fields (defaults where the checkpoint is silent)."""
    return _section(model_cfg, "pairformer", PAIRFORMER_DEFAULTS)


def confidence_config(model_cfg: dict | None) -> dict:
    """The confidence head's ``ConfidenceConfig`` fields used by its PairFormer layers."""
    return _section(model_cfg, "confidence", CONFIDENCE_DEFAULTS)


def evoformer_config(model_cfg: dict | None) -> dict:
    """The MSA stack's ``EvoformerConfig`` fields."""
    return _section(model_cfg, "evoformer", EVOFORMER_DEFAULTS)


def msa_block_kwargs(ec: dict, layer_idx: int) -> dict:
    """``EvoformerBlock`` arguments of MSA-stack layer ``layer_idx`` (``evoformer.py:433-455``)."""
    return dict(
        num_msa_heads=ec["msa_attention"]["num_head"],
        num_pair_heads=ec["pair_attention"]["num_head"],
        outer_product_hidden=ec["outer_product_num_channel"],
        msa_dropout=ec["msa_dropout"],
        pair_dropout=ec["pair_dropout"],
        residual_out_scale=block_residual_scale(
            layer_idx, ec["num_layer"], ec["residual_output_scaling"], ec["uniform_residual_scale"]
        ),
        use_triangle_attention=ec["use_triangle_attention"],
        trimul_kwargs=dict(
            num_heads=ec["trimul_num_heads"], head_norm=ec["trimul_head_norm"], router=ec["trimul_router"],
            router_kind=ec["trimul_router_kind"],
        ),  # fmt: skip
    )


def trunk_block_kwargs(pf: dict, layer_idx: int) -> dict:
    """``PairFormerBlock`` arguments of trunk layer ``layer_idx`` (``evoformer.py:459-489``)."""
    kw = dict(
        num_pair_heads=pf["pair_attention"]["num_head"],
        num_single_heads=pf["single_attention_num_head"],
        single_key_dim=pf["single_key_dim"],
        single_value_dim=pf["single_value_dim"],
        pair_dropout=pf["pair_dropout"],
        pair_bias_gate=pf["pair_bias_gate"],
        pair_bias_gate_init_tau=pf["pair_bias_gate_init_tau"],
        single_transition_linear_out_init_gain=pf["single_transition_linear_out_init_gain"],
        branch_scaler=pf["branch_scaler"],
        use_triangle_attention=pf["use_triangle_attention"],
        use_single_track=pf["use_single_track"],
        trimul_kwargs=dict(
            num_heads=pf["trimul_num_heads"], head_norm=pf["trimul_head_norm"], router=pf["trimul_router"],
            router_kind=pf["trimul_router_kind"],
        ),  # fmt: skip
    )
    kw.update(_layer_scales(pf, layer_idx))
    return kw


def confidence_block_kwargs(cc: dict, layer_idx: int) -> dict:
    """``PairFormerBlock`` arguments of confidence layer ``layer_idx`` (``confidence.py:88-117``)."""
    kw = dict(
        num_pair_heads=cc["pair_attention_num_head"],
        num_single_heads=cc["single_attention_num_head"],
        single_key_dim=cc["seq_channel"],
        single_value_dim=cc["seq_channel"],
        pair_bias_gate=cc["pair_bias_gate"],
        pair_bias_gate_init_tau=cc["pair_bias_gate_init_tau"],
        single_transition_linear_out_init_gain=cc["single_transition_linear_out_init_gain"],
        branch_scaler=cc["branch_scaler"],
    )
    kw.update(_layer_scales(cc, layer_idx))
    return kw


def build_trunk(model_cfg: dict | None, optim: OptimConfig | None = None) -> PairFormerStack:
    """An (untrained) trunk shaped by the checkpoint's ``pairformer`` section."""
    pf = trunk_config(model_cfg)
    return PairFormerStack(
        pf["num_layer"], pf["pair_channel"], pf["seq_channel"], optim=optim,
        layer_kwargs=lambda i: trunk_block_kwargs(pf, i),
    )  # fmt: skip


def build_recycler(model_cfg: dict | None, optim: OptimConfig | None = None) -> TrunkRecycler:
    pf = trunk_config(model_cfg)
    return TrunkRecycler(pf["pair_channel"], pf["seq_channel"], use_single_track=pf["use_single_track"], optim=optim)


def build_confidence_pairformer(model_cfg: dict | None, optim: OptimConfig | None = None) -> ConfidencePairFormer:
    cc = confidence_config(model_cfg)
    return ConfidencePairFormer(
        cc["num_layer"], cc["pair_channel"], cc["seq_channel"], num_pair_heads=cc["pair_attention_num_head"],
        num_single_heads=cc["single_attention_num_head"], optim=optim,
        layer_kwargs=lambda i: confidence_block_kwargs(cc, i),
    )  # fmt: skip


def build_msa_stack(model_cfg: dict | None, optim: OptimConfig | None = None) -> EvoformerStack:
    ec = evoformer_config(model_cfg)
    return EvoformerStack(
        ec["num_layer"], ec["msa_channel"], ec["pair_channel"], optim=optim,
        layer_kwargs=lambda i: msa_block_kwargs(ec, i),
    )  # fmt: skip


def load_prefixed(module: torch.nn.Module, path: str | os.PathLike, prefix: str, scope: str = "") -> None:
    """Load the tensors stored under ``prefix`` into ``module`` (module keys are the stored
    keys without ``prefix``), strictly: every module key must be present and no other stored
    key may start with ``prefix + scope``."""
    from safetensors import safe_open

    want = module.state_dict()
    found: dict[str, torch.Tensor] = {}
    with safe_open(str(path), framework="pt") as f:
        keys = [k for k in f.keys() if k.startswith(prefix + scope)]
        unexpected = sorted(k[len(prefix) :] for k in keys if k[len(prefix) :] not in want)
        missing = sorted(k for k in want if prefix + k not in keys)
        if missing or unexpected:
            raise KeyError(
                f"{path}: state under {prefix!r} does not match {type(module).__name__}: "
                f"missing {missing[:8]}{'...' if len(missing) > 8 else ''}, "
                f"unexpected {unexpected[:8]}{'...' if len(unexpected) > 8 else ''}"
            )
        for k in want:
            found[k] = f.get_tensor(prefix + k)
    module.load_state_dict(found, strict=True)


def _finish(module: torch.nn.Module, device, dtype) -> torch.nn.Module:
    module.eval()
    if device is not None:
        module.to(device)
    if dtype is not None:
        module.to(dtype)
    return module


def load_trunk(
    path: str | os.PathLike, device=None, dtype: torch.dtype | None = None, optim: OptimConfig | None = None
) -> tuple[PairFormerStack, dict | None]:
    """The trunk of a reference checkpoint; returns ``(stack, embedded model config or None)``.

    ``dtype`` casts the parameters (bf16 for the reference's benchmark regime; None keeps
    the stored dtype, the inference regime's fp32 parameters under bf16 autocast)."""
    cfg = read_model_cfg(path)
    stack = build_trunk(cfg, optim)
    load_prefixed(stack.blocks, path, TRUNK_PREFIX)
    return _finish(stack, device, dtype), cfg


def load_recycler(
    path: str | os.PathLike, device=None, dtype: torch.dtype | None = None, optim: OptimConfig | None = None
) -> TrunkRecycler:
    """The trunk's recycling embeddings (``evoformer.prev_*``) of a reference checkpoint."""
    cfg = read_model_cfg(path)
    rec = build_recycler(cfg, optim)
    load_prefixed(rec, path, RECYCLE_PREFIX, scope="prev_")
    return _finish(rec, device, dtype)


def load_confidence_pairformer(
    path: str | os.PathLike, device=None, dtype: torch.dtype | None = None, optim: OptimConfig | None = None
) -> ConfidencePairFormer:
    """The confidence head's PairFormer layers (``confidence_head.layers.*``)."""
    cfg = read_model_cfg(path)
    stack = build_confidence_pairformer(cfg, optim)
    load_prefixed(stack.layers, path, CONFIDENCE_PREFIX)
    return _finish(stack, device, dtype)


def load_msa_stack(
    path: str | os.PathLike, device=None, dtype: torch.dtype | None = None, optim: OptimConfig | None = None
) -> EvoformerStack:
    """The MSA stack (``evoformer.msa_stack.*``) of a reference checkpoint."""
    cfg = read_model_cfg(path)
    stack = build_msa_stack(cfg, optim)
    load_prefixed(stack, path, MSA_STACK_PREFIX, scope="msa_stack.")
    return _finish(stack, device, dtype)
