"""CPU: reference-format checkpoints (safetensors with the embedded ModelConfig JSON).

The file is written here in the reference's layout: the trunk under
``evoformer.trunk_pairformer.{i}.``, the recycling embeddings under ``evoformer.prev_*``, the
confidence head's layers under ``confidence_head.layers.{i}.``, next to keys of parts this
build does not have, and ``model_cfg_json`` in the metadata (``config.py:1895-1958``). The
tests check the architecture mapping against the reference's closed forms
(``primitives.py:20-44``, ``evoformer.py:66-82``), that every tensor lands where its key
says, strictness, and refusal by name of what is not built. The forward passes of loaded
stacks are compared with the oracle in ``tests/test_checkpoint_gpu.py``.
"""

from __future__ import annotations

import json
import math

import pytest
import torch

from tests._helpers import mod

W = mod("weights")
ck = mod("checkpoint")
guard = mod("inference_guard")


def _recycle(seed: int) -> dict:
    g = torch.Generator().manual_seed(seed)
    return {
        "prev_embedding_layer_norm.weight": 1.0 + 0.2 * torch.randn(128, generator=g),
        "prev_embedding_layer_norm.bias": 0.3 * torch.randn(128, generator=g),
        "prev_embedding.weight": torch.randn(128, 128, generator=g) / 128**0.5,
        "prev_single_embedding_layer_norm.weight": 1.0 + 0.2 * torch.randn(384, generator=g),
        "prev_single_embedding_layer_norm.bias": 0.3 * torch.randn(384, generator=g),
        "prev_single_embedding.weight": torch.randn(384, 384, generator=g) / 384**0.5,
    }


def write_checkpoint(path, model_cfg: dict | None, trunk_layers: int = 2, conf_layers: int = 2, seed: int = 40,
                     msa_layers: int = 0):  # fmt: skip
    """A reference-layout checkpoint; returns the tensors written, by key. With ``msa_layers``
    0 the MSA stack is a stray key the other loaders must leave alone."""
    from safetensors.torch import save_file

    sd = {}
    for i, blk in enumerate(W.make_trunk_weights(seed, trunk_layers, perturb_affine=True)):
        sd.update({f"evoformer.trunk_pairformer.{i}.{k}": v for k, v in blk.items()})
    sd.update({f"evoformer.{k}": v for k, v in _recycle(seed + 1).items()})
    for i, blk in enumerate(W.make_trunk_weights(seed + 2, conf_layers, perturb_affine=True)):
        sd.update({f"confidence_head.layers.{i}.{k}": v for k, v in blk.items()})
    # parts outside the hot path, which the loaders must leave alone
    sd["evoformer.position_activations.weight"] = torch.randn(128, 139)
    if msa_layers:
        for i in range(msa_layers):
            blk = W.make_evoformer_block_weights(seed + 3 + i, perturb_affine=True)
            sd.update({f"evoformer.msa_stack.{i}.{k}": v for k, v in blk.items()})
    else:
        sd["evoformer.msa_stack.0.msa_transition.linear1.weight"] = torch.randn(512, 64)
    sd["confidence_head.pae_logits.weight"] = torch.randn(64, 128)
    sd["diffusion.conditioning.weight"] = torch.randn(8, 8)
    sd = {k: v.contiguous() for k, v in sd.items()}
    meta = None if model_cfg is None else {ck.MODEL_CFG_KEY: json.dumps(model_cfg)}
    save_file(sd, str(path), metadata=meta)
    return sd


CFG = {
    "pairformer": {
        "num_layer": 2,
        "pair_channel": 128,
        "pair_attention": {"num_head": 4, "a_future_field": 3},
        "residual_output_scaling": True,
        "pair_transition_residual_gain": 0.5,
        "single_transition_residual_per_layer_extra": True,
        "a_field_from_a_later_revision": "ignored",
    },
    "confidence": {"num_layer": 2, "uniform_residual_scale": True},
    "evoformer": {"num_layer": 2, "residual_output_scaling": True, "msa_attention": {"num_head": 8}},
    "optim": {"use_fused_triangle_mul": True},
}


def test_residual_scale_rules_match_reference_closed_forms():
    for i in range(5):
        assert ck.block_residual_scale(i, 48, True, False) == pytest.approx(1 / math.sqrt(i + 1), abs=0)
        assert ck.block_residual_scale(i, 48, False, True) == pytest.approx(1 / math.sqrt(48), abs=0)
        assert ck.block_residual_scale(i, 48, False, False) == 1.0
        assert ck.branch_residual_gain(i, None, False) is None
        assert ck.branch_residual_gain(i, 0.25, False) == 0.25
        assert ck.branch_residual_gain(i, None, True) == pytest.approx(1 / math.sqrt(i + 1))
        assert ck.branch_residual_gain(i, 0.25, True) == pytest.approx(0.25 / math.sqrt(i + 1))
    with pytest.raises(ValueError, match="not both"):
        ck.block_residual_scale(0, 4, True, True)


def test_config_sections_defaults_and_unknown_fields():
    pf = ck.trunk_config(CFG)
    assert pf["num_layer"] == 2 and pf["residual_output_scaling"] is True
    assert pf["pair_attention"] == {"num_head": 4}
    assert "a_field_from_a_later_revision" not in pf
    assert pf["seq_channel"] == 384 and pf["use_single_track"] is True  # defaults where silent
    assert ck.trunk_config(None) == ck.PAIRFORMER_DEFAULTS
    assert ck.confidence_config(CFG)["uniform_residual_scale"] is True
    assert ck.confidence_config(None)["num_layer"] == 4


def test_trunk_block_kwargs_per_layer():
    pf = ck.trunk_config(CFG)
    for i in range(2):
        kw = ck.trunk_block_kwargs(pf, i)
        assert kw["residual_out_scale"] == pytest.approx(1 / math.sqrt(i + 1))
        assert kw["pair_transition_residual_gain"] == 0.5
        assert kw["single_transition_residual_gain"] == pytest.approx(1 / math.sqrt(i + 1))
        assert kw["trimul_kwargs"]["num_heads"] == 0 and kw["num_pair_heads"] == 4


def test_read_model_cfg(tmp_path):
    write_checkpoint(tmp_path / "a.safetensors", CFG)
    assert ck.read_model_cfg(tmp_path / "a.safetensors") == CFG
    write_checkpoint(tmp_path / "b.safetensors", None)
    assert ck.read_model_cfg(tmp_path / "b.safetensors") is None


def test_load_trunk_recycler_and_confidence(tmp_path):
    path = tmp_path / "ckpt.safetensors"
    sd = write_checkpoint(path, CFG)
    stack, cfg = ck.load_trunk(path)
    assert cfg == CFG and len(stack.blocks) == 2
    for i, blk in enumerate(stack.blocks):
        for k, v in blk.state_dict().items():
            assert torch.equal(v, sd[f"evoformer.trunk_pairformer.{i}.{k}"]), (i, k)
        s = 1 / math.sqrt(i + 1)
        assert blk.residual_out_scale == pytest.approx(s)
        assert blk.tri_mul_in.branch_scale == pytest.approx(s)
        assert blk.pair_attn_col.branch_scale == pytest.approx(s)
        assert blk.pair_transition.branch_scale == pytest.approx(0.5 * s)
        assert blk.single_transition.branch_scale == pytest.approx(s * s)
        assert not blk.training
    rec = ck.load_recycler(path)
    for k, v in rec.state_dict().items():
        assert torch.equal(v, sd["evoformer." + k]), k
    conf = ck.load_confidence_pairformer(path)
    assert len(conf.layers) == 2
    for i, blk in enumerate(conf.layers):
        assert blk.residual_out_scale == pytest.approx(1 / math.sqrt(2))
        for k, v in blk.state_dict().items():
            assert torch.equal(v, sd[f"confidence_head.layers.{i}.{k}"]), (i, k)
    st2, _ = ck.load_trunk(path, dtype=torch.bfloat16)
    assert all(p.dtype == torch.bfloat16 for p in st2.parameters())


def test_loading_is_strict(tmp_path):
    from safetensors.torch import save_file

    path = tmp_path / "c.safetensors"
    sd = write_checkpoint(path, CFG)
    missing = {k: v for k, v in sd.items() if k != "evoformer.trunk_pairformer.1.pair_attn_row.to_q.weight"}
    save_file(missing, str(tmp_path / "missing.safetensors"), metadata={ck.MODEL_CFG_KEY: json.dumps(CFG)})
    with pytest.raises(KeyError, match="1.pair_attn_row.to_q.weight"):
        ck.load_trunk(tmp_path / "missing.safetensors")
    extra = dict(sd, **{"evoformer.trunk_pairformer.2.tri_mul_out.proj.weight": torch.zeros(256, 128)})
    save_file(extra, str(tmp_path / "extra.safetensors"), metadata={ck.MODEL_CFG_KEY: json.dumps(CFG)})
    with pytest.raises(KeyError, match="2.tri_mul_out.proj.weight"):
        ck.load_trunk(tmp_path / "extra.safetensors")
    extra_prev = dict(sd, **{"evoformer.prev_pos_embedding.weight": torch.zeros(4, 4)})
    save_file(extra_prev, str(tmp_path / "prev.safetensors"))
    with pytest.raises(KeyError, match="prev_pos_embedding"):
        ck.load_recycler(tmp_path / "prev.safetensors")


def test_mhr_trimul_builds_with_the_reference_keys():
    """MHR triangle multiplication (config.py:104-119, ops.py:179-260): the reference's r17
    arm (8 heads, head_ln, softmax router) adds ``router.weight`` [8, C] (zeros) to each
    triangle multiply; head_rms drops ``norm_center.bias``; bad combinations are refused with
    the reference's messages."""
    trunk = ck.build_trunk({"pairformer": {"num_layer": 1, "pair_channel": 256, "pair_attention": {"num_head": 8},
                                           "trimul_num_heads": 8, "trimul_head_norm": "head_ln",
                                           "trimul_router": True}})  # fmt: skip
    sd = trunk.state_dict()
    for site in ("tri_mul_out", "tri_mul_in"):
        r = sd[f"blocks.0.{site}.router.weight"]
        assert r.shape == (8, 256) and not r.any()
        assert f"blocks.0.{site}.norm_center.bias" in sd
        assert trunk.blocks[0].tri_mul_out.is_mhr
    rms = ck.build_trunk({"pairformer": {"num_layer": 1, "trimul_num_heads": 4, "trimul_head_norm": "head_rms"}})
    keys = set(rms.state_dict())
    assert "blocks.0.tri_mul_in.norm_center.bias" not in keys and "blocks.0.tri_mul_in.router.weight" not in keys
    with pytest.raises(ValueError, match="divisible"):
        ck.build_trunk({"pairformer": {"num_layer": 1, "trimul_num_heads": 7, "trimul_head_norm": "head_rms"}})
    with pytest.raises(ValueError, match="num_heads > 0"):
        ck.build_trunk({"pairformer": {"num_layer": 1, "trimul_router": True}})
    with pytest.raises(ValueError, match="meaningless without router"):
        ck.build_trunk({"pairformer": {"num_layer": 1, "trimul_num_heads": 4, "trimul_head_norm": "post_channel"}})
    with pytest.raises(ValueError, match="head_norm"):
        ck.build_trunk({"pairformer": {"num_layer": 1, "trimul_num_heads": 4, "trimul_head_norm": "groupnorm"}})


def test_rmsnorm_branch_scaler_builds_and_refuses_transition_gains():
    """branch_scaler="rmsnorm" builds (config.py:185); with a transition residual gain set it is
    refused as the reference's PairFormerConfig.__post_init__ refuses it (config.py:252-269)."""
    trunk = ck.build_trunk({"pairformer": {"num_layer": 1, "branch_scaler": "rmsnorm"}})
    assert trunk.blocks[0].branch_scaler_kind == "rmsnorm"
    with pytest.raises(ValueError, match="residual gains"):
        ck.build_trunk({"pairformer": {"num_layer": 1, "branch_scaler": "rmsnorm", "pair_transition_residual_gain": 0.5}})


def test_pair_bias_gate_builds_with_its_key_and_init():
    """pair_bias_gate (attention.py:392-398): a [16] parameter single_attn.pair_bias_gate_a per
    block, initialised to log(pair_bias_gate_init_tau); a non-positive tau_0 is refused."""
    trunk = ck.build_trunk({"pairformer": {"num_layer": 2, "pair_bias_gate": True, "pair_bias_gate_init_tau": 0.5}})
    keys = [k for k in trunk.state_dict() if k.endswith("pair_bias_gate_a")]
    assert keys == ["blocks.0.single_attn.pair_bias_gate_a", "blocks.1.single_attn.pair_bias_gate_a"]
    a = trunk.state_dict()[keys[0]]
    assert a.shape == (16,) and torch.allclose(a, torch.full((16,), math.log(0.5)))
    with pytest.raises(ValueError, match="tau_0 must be positive"):
        ck.build_trunk({"pairformer": {"num_layer": 1, "pair_bias_gate": True, "pair_bias_gate_init_tau": 0.0}})


# The reference's current stage-0 model shape (configs/stage0.yaml:50-75): 256 pair channels in 8
# heads, no triangle attention in the trunk or the MSA stack, no single track in the trunk.
STAGE0 = {
    "evoformer": {"num_layer": 2, "msa_channel": 128, "pair_channel": 256, "pair_attention": {"num_head": 8},
                  "msa_attention": {"num_head": 16}, "use_triangle_attention": False, "trimul_num_heads": 0},
    "pairformer": {"num_layer": 2, "pair_channel": 256, "pair_attention": {"num_head": 8},
                   "use_triangle_attention": False, "trimul_num_heads": 0, "use_single_track": False},
    "confidence": {"num_layer": 1, "pair_channel": 256, "pair_attention_num_head": 8},
}  # fmt: skip


def write_stage0_checkpoint(path, seed: int = 60) -> dict:
    """A reference-layout checkpoint of the STAGE0 shape (trunk, recycler without the single
    embedding, MSA stack); returns the tensors by key."""
    from safetensors.torch import save_file

    sd = {}
    for i, blk in enumerate(W.make_trunk_weights(seed, 2, perturb_affine=True, c_pair=256, num_pair_heads=8,
                                                 use_triangle_attention=False, use_single_track=False)):  # fmt: skip
        sd.update({f"evoformer.trunk_pairformer.{i}.{k}": v for k, v in blk.items()})
    g = torch.Generator().manual_seed(seed + 1)
    sd["evoformer.prev_embedding_layer_norm.weight"] = 1.0 + 0.2 * torch.randn(256, generator=g)
    sd["evoformer.prev_embedding_layer_norm.bias"] = 0.3 * torch.randn(256, generator=g)
    sd["evoformer.prev_embedding.weight"] = torch.randn(256, 256, generator=g) / 16.0
    for i in range(2):
        blk = W.make_evoformer_block_weights(seed + 2 + i, perturb_affine=True, c_msa=128, c_pair=256,
                                             num_msa_heads=16, num_pair_heads=8, use_triangle_attention=False)  # fmt: skip
        sd.update({f"evoformer.msa_stack.{i}.{k}": v for k, v in blk.items()})
    sd = {k: v.contiguous() for k, v in sd.items()}
    save_file(sd, str(path), metadata={ck.MODEL_CFG_KEY: json.dumps(STAGE0)})
    return sd


def test_stage0_shape_builds_without_deleted_branches_and_loads(tmp_path):
    """Blocks of a config without triangle attention and without the single track have
    exactly the reference's keys for that shape (no ``pair_attn_*``, no ``single_*``) and load
    strictly; the recycler has no single embedding."""
    path = tmp_path / "stage0.safetensors"
    sd = write_stage0_checkpoint(path)
    trunk, cfg = ck.load_trunk(path)
    assert cfg == STAGE0 and len(trunk.blocks) == 2
    for i, blk in enumerate(trunk.blocks):
        assert not blk.use_triangle_attention and not blk.use_single_track
        keys = set(blk.state_dict())
        assert not any(k.startswith(("pair_attn_", "single_")) for k in keys)
        assert keys == {k[len(f"evoformer.trunk_pairformer.{i}."):] for k in sd if k.startswith(f"evoformer.trunk_pairformer.{i}.")}
    rec = ck.load_recycler(path)
    assert not rec.use_single_track and rec.prev_embedding.weight.shape == (256, 256)
    msa = ck.load_msa_stack(path)
    for blk in msa.msa_stack:
        assert not blk.use_triangle_attention
        assert not any(k.startswith("pair_attn_") for k in blk.state_dict())


def test_msa_block_kwargs_per_layer():
    ec = ck.evoformer_config(CFG)
    assert ec["num_layer"] == 2 and ec["msa_channel"] == 64 and ec["outer_product_num_channel"] == 32
    for i in range(2):
        kw = ck.msa_block_kwargs(ec, i)
        assert kw["residual_out_scale"] == pytest.approx(1 / math.sqrt(i + 1))
        assert kw["num_msa_heads"] == 8 and kw["num_pair_heads"] == 4 and kw["outer_product_hidden"] == 32
    assert ck.evoformer_config(None)["num_layer"] == 4
    assert ck.msa_block_kwargs(ck.evoformer_config(None), 3)["residual_out_scale"] == 1.0


def test_load_msa_stack(tmp_path):
    path = tmp_path / "m.safetensors"
    sd = write_checkpoint(path, CFG, msa_layers=2)
    stack = ck.load_msa_stack(path)
    assert len(stack.msa_stack) == 2
    for i, blk in enumerate(stack.msa_stack):
        s = 1 / math.sqrt(i + 1)
        assert blk.row_attn.branch_scale == pytest.approx(s)
        assert blk.outer_product.branch_scale == pytest.approx(s)
        assert blk.msa_transition.branch_scale == pytest.approx(s)
        assert blk.tri_mul_out.branch_scale == pytest.approx(s)
        for k, v in blk.state_dict().items():
            assert torch.equal(v, sd[f"evoformer.msa_stack.{i}.{k}"]), (i, k)
    # the trunk and the recycler load beside it
    ck.load_trunk(path)
    ck.load_recycler(path)
    stray = tmp_path / "stray.safetensors"
    write_checkpoint(stray, CFG)  # one stray MSA-stack key only
    with pytest.raises(KeyError, match="msa_stack"):
        ck.load_msa_stack(stray)
