"""GPU: stacks loaded from a reference-layout checkpoint, the recycling embedding and the
recycle loop, against the oracle.

- The trunk of a checkpoint whose config sets per-layer residual output scaling, a pair
  transition residual gain and a per-layer single transition gain (``evoformer.py:459-489``
  construction; scales applied at ``:282-353``), fp32 and bf16.
- The confidence head's layers with the uniform residual scale (``confidence.py:88-117``).
- The recycling embeddings (``evoformer.py:520-526``, ``:558-561``) and the recycle loop
  around the trunk (``model.py:385-470``, stages between the embedding and the trunk left
  out on both sides).
- The template block with a residual scale (``template_embedding.py:220-240``).
- The MSA stack with per-layer residual output scaling (``evoformer.py:433-455``), against the
  oracle's Evoformer blocks in order.

fp32 at relL2 <= 1e-5 and max-abs <= 1e-5 max|ref|; bf16 by the reference's rule
relL2(HIP - fp32) <= 2 relL2(eager bf16 - fp32) (tests/triton/test_fused_trimul.py:66-83).
"""

from __future__ import annotations

import pytest
import torch

from oracle import pairformer_ref as R
from tests._helpers import assert_bf16_rule, assert_fp32_close, mod, sub, to
from tests.test_checkpoint import CFG, write_checkpoint

pytestmark = pytest.mark.gpu
W = mod("weights")
ck = mod("checkpoint")
evoformer = mod("evoformer")
BF = torch.bfloat16
SCALE_KEYS = ("residual_out_scale", "pair_transition_residual_gain", "single_transition_residual_gain")


@pytest.fixture(autouse=True)
def _highest():
    torch.set_float32_matmul_precision("highest")


def _trunk_ref(sd: dict, layers: int, prefix: str, cfg_fn, kw_fn):
    blocks = [sub(sd, f"{prefix}{i}.") for i in range(layers)]
    scales = [{k: kw_fn(cfg_fn(CFG), i)[k] for k in SCALE_KEYS} for i in range(layers)]
    return blocks, scales


def test_checkpoint_trunk_fp32(dev, tmp_path):
    path = tmp_path / "t.safetensors"
    sd = write_checkpoint(path, CFG)
    stack, _ = ck.load_trunk(path, device=dev)
    blocks, scales = _trunk_ref(sd, 2, ck.TRUNK_PREFIX, ck.trunk_config, ck.trunk_block_kwargs)
    assert scales[1]["residual_out_scale"] != 1.0 and scales[0]["pair_transition_residual_gain"] == 0.5
    x = W.make_inputs(40, seed=11, pad_last=3)
    print("[checkpoint trunk fp32] N=40", flush=True)
    with torch.no_grad():
        p, s = stack(x["pair"].to(dev), x["single"].to(dev), x["pair_mask"].to(dev), x["seq_mask"].to(dev))
        rp, rs = R.pairformer_trunk(x["pair"], x["single"], x["pair_mask"], x["seq_mask"], blocks, scales=scales)
        up, _ = R.pairformer_trunk(x["pair"], x["single"], x["pair_mask"], x["seq_mask"], blocks)
    assert_fp32_close(p.cpu(), rp, what="checkpoint trunk pair")
    assert_fp32_close(s.cpu(), rs, what="checkpoint trunk single")
    assert (p.cpu() - up).norm() / up.norm() > 1e-3  # the scales act


def test_checkpoint_trunk_bf16_rule(dev, tmp_path):
    path = tmp_path / "t.safetensors"
    sd = write_checkpoint(path, CFG, seed=50)
    stack, _ = ck.load_trunk(path, device=dev, dtype=BF)
    blocks, scales = _trunk_ref(sd, 2, ck.TRUNK_PREFIX, ck.trunk_config, ck.trunk_block_kwargs)
    x = {k: v.to(dev) for k, v in W.make_inputs(96, seed=12, pad_random=6).items()}
    pm, sm = x["pair_mask"], x["seq_mask"]
    print("[checkpoint trunk bf16] N=96", flush=True)
    with torch.no_grad():
        p, s = stack(x["pair"].to(BF), x["single"].to(BF), pm, sm)
        with torch.autocast("cuda", dtype=BF):
            ep, es = R.pairformer_trunk(x["pair"].to(BF), x["single"].to(BF), pm, sm,
                                        [to(b, dev, BF) for b in blocks], scales=scales)  # fmt: skip
        rp, rs = R.pairformer_trunk(x["pair"].to(BF).float(), x["single"].to(BF).float(), pm, sm,
                                    [to(b, dev) for b in blocks], scales=scales)  # fmt: skip
    print("[checkpoint trunk bf16]", assert_bf16_rule(p.cpu(), ep.cpu(), rp.cpu(), "pair"),
          assert_bf16_rule(s.cpu(), es.cpu(), rs.cpu(), "single"), flush=True)  # fmt: skip


def test_checkpoint_confidence_fp32(dev, tmp_path):
    path = tmp_path / "c.safetensors"
    sd = write_checkpoint(path, CFG, seed=60)
    conf = ck.load_confidence_pairformer(path, device=dev)
    blocks, scales = _trunk_ref(sd, 2, ck.CONFIDENCE_PREFIX, ck.confidence_config, ck.confidence_block_kwargs)
    assert scales[0]["residual_out_scale"] == pytest.approx(2**-0.5)
    x = W.make_inputs(33, seed=13, pad_last=2)
    print("[checkpoint confidence fp32] N=33", flush=True)
    with torch.no_grad():
        p, s = conf(x["pair"].to(dev), x["single"].to(dev), x["pair_mask"].to(dev), x["seq_mask"].to(dev))
        rp, rs = R.pairformer_trunk(x["pair"], x["single"], x["pair_mask"], x["seq_mask"], blocks, scales=scales)
    assert_fp32_close(p.cpu(), rp, what="confidence pair")
    assert_fp32_close(s.cpu(), rs, what="confidence single")


def _recycle_inputs(n: int, seed: int):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(1, n, n, 128, generator=g), torch.randn(1, n, 384, generator=g),
            torch.randn(1, n, n, 128, generator=g), torch.randn(1, n, 384, generator=g)]  # fmt: skip


@pytest.mark.parametrize("n", [17, 64])
def test_recycle_embed_fp32(dev, tmp_path, n):
    path = tmp_path / "r.safetensors"
    sd = write_checkpoint(path, CFG, seed=70)
    rec = ck.load_recycler(path, device=dev)
    rp = sub(sd, "evoformer.")
    zp, zs, pp, ps = _recycle_inputs(n, n)
    print(f"[recycle embed fp32] N={n}", flush=True)
    with torch.no_grad():
        p, s = rec(zp.to(dev), zs.to(dev), pp.to(dev), ps.to(dev))
        wp, ws = R.recycle_embed(zp, zs, pp, ps, rp)
    assert_fp32_close(p.cpu(), wp, what="recycled pair")
    assert_fp32_close(s.cpu(), ws, what="recycled single")


def test_recycle_embed_bf16_rule(dev, tmp_path):
    path = tmp_path / "r.safetensors"
    sd = write_checkpoint(path, CFG, seed=71)
    rec = ck.load_recycler(path, device=dev, dtype=BF)
    rp = sub(sd, "evoformer.")
    xs = [t.to(dev).to(BF) for t in _recycle_inputs(96, 5)]
    print("[recycle embed bf16] N=96", flush=True)
    with torch.no_grad():
        p, s = rec(*xs)
        with torch.autocast("cuda", dtype=BF):
            ep, es = R.recycle_embed(*xs, to(rp, dev, BF))
        wp, ws = R.recycle_embed(*[t.float() for t in xs], to(rp, dev))
    print("[recycle embed bf16]", assert_bf16_rule(p.cpu(), ep.cpu(), wp.cpu(), "pair"),
          assert_bf16_rule(s.cpu(), es.cpu(), ws.cpu(), "single"), flush=True)  # fmt: skip


def test_run_recycles_fp32(dev, tmp_path):
    path = tmp_path / "l.safetensors"
    sd = write_checkpoint(path, CFG, seed=80)
    stack, _ = ck.load_trunk(path, device=dev)
    rec = ck.load_recycler(path, device=dev)
    blocks, scales = _trunk_ref(sd, 2, ck.TRUNK_PREFIX, ck.trunk_config, ck.trunk_block_kwargs)
    x = W.make_inputs(24, seed=14, pad_last=2)
    print("[recycle loop fp32] N=24, 2 recycles", flush=True)
    with torch.no_grad():
        p, s = evoformer.run_recycles(rec, stack, x["pair"].to(dev), x["single"].to(dev), x["pair_mask"].to(dev),
                                      x["seq_mask"].to(dev), num_recycles=2)  # fmt: skip
        rp, rs = R.recycled_trunk(x["pair"], x["single"], x["pair_mask"], x["seq_mask"], sub(sd, "evoformer."),
                                  blocks, num_recycles=2, scales=scales)  # fmt: skip
    assert_fp32_close(p.cpu(), rp, what="recycled trunk pair")
    assert_fp32_close(s.cpu(), rs, what="recycled trunk single")


def test_template_block_residual_scale_fp32(dev):
    sd = W.make_block_weights(91, perturb_affine=True, factor=2)
    p = {k: v for k, v in sd.items() if k.startswith(("tri_mul_", "pair_attn_", "pair_transition."))}
    m = evoformer.TemplatePairFormerBlock(128, residual_out_scale=0.5).eval()
    m.load_state_dict(p)
    m = m.to(dev)
    x = W.make_inputs(30, seed=15, pad_last=2)
    print("[template block scaled fp32] N=30", flush=True)
    with torch.no_grad():
        got = m(x["pair"].to(dev), x["pair_mask"].to(dev))
        ref = R.template_pairformer_block(x["pair"], x["pair_mask"], p, residual_out_scale=0.5)
    assert_fp32_close(got.cpu(), ref, what="template block s=0.5")


def test_checkpoint_msa_stack_fp32(dev, tmp_path):
    path = tmp_path / "m.safetensors"
    sd = write_checkpoint(path, CFG, seed=90, msa_layers=2)
    stack = ck.load_msa_stack(path, device=dev)
    ec = ck.evoformer_config(CFG)
    g = torch.Generator().manual_seed(16)
    S, N = 9, 27
    msa = torch.randn(1, S, N, 64, generator=g)
    pair = torch.randn(1, N, N, 128, generator=g)
    mask = (torch.rand(1, S, N, generator=g) > 0.15).float()
    mask[:, :, N - 2 :] = 0.0
    seq = (mask.max(dim=1).values > 0).float()
    pm = seq[:, :, None] * seq[:, None, :]
    print(f"[checkpoint MSA stack fp32] S={S} N={N}", flush=True)
    with torch.no_grad():
        m, p = stack(msa.to(dev), pair.to(dev), mask.to(dev), pm.to(dev))
        rm, rp = msa, pair
        for i in range(2):
            s = ck.msa_block_kwargs(ec, i)["residual_out_scale"]
            rm, rp = R.evoformer_block(rm, rp, mask, pm, sub(sd, f"evoformer.msa_stack.{i}."), residual_out_scale=s)
    assert_fp32_close(m.cpu(), rm, what="checkpoint MSA stack msa")
    assert_fp32_close(p.cpu(), rp, what="checkpoint MSA stack pair")
