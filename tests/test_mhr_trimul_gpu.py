"""GPU: multi-head routed (MHR) triangle multiplication (``ops.py:179-345``, head mix
``:476-545``) on the HIP kernels against the oracle (``R.tri_mul`` / ``R.tri_mul_core`` with
the mix, pinned in test_mhr_oracle.py).

- Inference (``pf_trimul_mhr_fwd``, the mix in K3): fp32 relL2 <= 1e-5 and max-abs <= 1e-5
  max|ref| for every head_norm with and without the router, both router kinds, both
  directions, C = 64 (8 heads of 8), 128 (4 heads of 32) and 256 (8 heads of 32), ragged N
  with padded pairs; bf16: the reference's rule relL2(HIP - fp32) <= 2 relL2(eager bf16 -
  fp32) for the reference's r17 arm (C = 256, 8 heads, head_ln, softmax router) at N = 200
  and 500 (generic and persistent contractions).
- The in-place residual (``forward_residual_``) and a batch of two.
- Training (``FusedTriMulFunction`` with the mix; ``pf_trimul_mhr_train_fwd``,
  ``pf_trimul_mhr_output_vjp``): the update and every gradient (x, both projections,
  norm_center's affine, out_proj, out_gate, the router) against ``R.tri_mul_core``
  differentiated in fp64, fp32 regime, at relL2 <= 1e-5.
- The module under grad in the reference's training regime (fp32 z under bf16 autocast)
  against the fp32 stock path on the CPU: every gradient within 3x the error of the stock
  path under CPU bf16 autocast (+1e-3), as the plain module's test.
- The router read-out of an inert (zero) router: entropy 1, occupancy 1/H, g_mean 1.
"""

from __future__ import annotations

import pytest
import torch

from oracle import pairformer_ref as R
from tests._helpers import assert_bf16_rule, assert_fp32_close, mod, rel_l2, sub, to

pytestmark = pytest.mark.gpu
W = mod("weights")
ops = mod("ops")
kernels = mod("kernels")
BF = torch.bfloat16

MODES = [
    ("channel", True, "softmax"),
    ("head_rms", False, "softmax"),
    ("head_rms", True, "softmax"),
    ("head_ln", True, "softmax"),
    ("head_ln", True, "sigmoid"),
    ("post_channel", True, "softmax"),
    ("post_channel", True, "sigmoid"),
]
MODE_IDS = [f"{h}-{'r' + k[:3] if r else 'norouter'}" for h, r, k in MODES]
HEADS = {64: 8, 128: 4, 256: 8}


@pytest.fixture(autouse=True)
def _highest():
    torch.set_float32_matmul_precision("highest")


def _params(C, outgoing, head_norm, router, seed):
    H = HEADS[C]
    sd = W.make_block_weights(seed, perturb_affine=True, c_pair=C, trimul_num_heads=H, trimul_head_norm=head_norm,
                              trimul_router=router)  # fmt: skip
    return sub(sd, "tri_mul_out." if outgoing else "tri_mul_in.")


def _module(C, outgoing, head_norm, router, kind, p, dev, dtype=torch.float32):
    cls = ops.TriangleMulOutgoing if outgoing else ops.TriangleMulIncoming
    m = cls(C, num_heads=HEADS[C], head_norm=head_norm, router=router, router_kind=kind)
    m.load_state_dict(p)
    return m.to(dev).to(dtype)


def _kw(C, head_norm, router, kind):
    return dict(num_heads=HEADS[C], head_norm=head_norm, router=router, router_kind=kind)


@pytest.mark.parametrize("outgoing", [True, False], ids=["out", "in"])
@pytest.mark.parametrize("C,n,pad", [(64, 24, 3), (128, 70, 5), (256, 33, 2)])
@pytest.mark.parametrize("head_norm,router,kind", MODES, ids=MODE_IDS)
def test_mhr_fp32_matches_oracle(dev, outgoing, C, n, pad, head_norm, router, kind):
    print(f"[mhr fp32] C={C} N={n} {head_norm} router={router} {kind} outgoing={outgoing}", flush=True)
    p = _params(C, outgoing, head_norm, router, seed=C + n)
    inp = W.make_inputs(n, seed=n, pad_last=pad, c_pair=C)
    m = _module(C, outgoing, head_norm, router, kind, p, dev)
    with torch.no_grad():
        got = m(inp["pair"].to(dev), inp["pair_mask"].to(dev))
    ref = R.tri_mul(inp["pair"], inp["pair_mask"], p, outgoing, **_kw(C, head_norm, router, kind))
    assert ref.abs().max() > 1e-3
    assert_fp32_close(got.cpu(), ref, what=f"mhr fp32 {head_norm} C={C}")


@pytest.mark.parametrize("outgoing", [True, False], ids=["out", "in"])
@pytest.mark.parametrize("n", [200, 500])
def test_mhr_bf16_tolerance_rule_r17(dev, outgoing, n):
    print(f"[mhr bf16] N={n} outgoing={outgoing}", flush=True)
    C, kw = 256, _kw(256, "head_ln", True, "softmax")
    p = _params(C, outgoing, "head_ln", True, seed=7)
    inp = W.make_inputs(n, seed=5, pad_random=6, c_pair=C)
    m = _module(C, outgoing, "head_ln", True, "softmax", p, dev, BF)
    zb = inp["pair"].to(dev, BF)
    mb = inp["pair_mask"].to(dev, BF)
    with torch.no_grad():
        got = m(zb, mb)
        eager = R.tri_mul(zb, mb, to(p, dev, BF), outgoing, **kw)
    ref = R.tri_mul(zb.float().cpu(), inp["pair_mask"], p, outgoing, **kw)
    assert got.dtype == BF
    print("  ", assert_bf16_rule(got.cpu(), eager.cpu(), ref, "mhr bf16"), flush=True)


def test_mhr_fused_residual_and_batch(dev):
    C, n = 128, 40
    p = _params(C, True, "head_rms", True, seed=9)
    m = _module(C, True, "head_rms", True, "sigmoid", p, dev)
    g = torch.Generator().manual_seed(3)
    z = torch.randn(2, n, n, C, generator=g)
    mask = (torch.rand(2, n, n, generator=g) > 0.1).float()
    ref = R.tri_mul(z, mask, p, True, **_kw(C, "head_rms", True, "sigmoid"))
    with torch.no_grad():
        zd = z.to(dev)
        upd = m(zd, mask.to(dev))
        acc = zd.clone()
        m.forward_residual_(acc, mask.to(dev))
    assert_fp32_close(upd.cpu(), ref, what="mhr batch")
    assert_fp32_close(acc.cpu(), z + ref, what="mhr residual")


NAMES = ("x", "w_gate", "w_proj", "ln_out_w", "ln_out_b", "w_out", "w_out_gate", "w_router")


@pytest.mark.parametrize("outgoing", [True, False], ids=["out", "in"])
@pytest.mark.parametrize("C,N", [(64, 30), (128, 37), (256, 21)])
@pytest.mark.parametrize("head_norm,router,kind", MODES, ids=MODE_IDS)
def test_mhr_function_fp32_gradients(dev, outgoing, C, N, head_norm, router, kind):
    print(f"[mhr vjp fp32] C={C} N={N} {head_norm} router={router} {kind} outgoing={outgoing}", flush=True)
    H = HEADS[C]
    g = torch.Generator().manual_seed(C + N)
    r = lambda *s: torch.randn(*s, generator=g)  # noqa: E731
    x = r(2, N, N, C)
    mask = (torch.rand(2, N, N, generator=g) > 0.15).float()
    mask[:, N - 2 :, :] = 0.0
    ws = [r(2 * C, C) / C**0.5, r(2 * C, C) / C**0.5, 1 + 0.1 * r(C), 0.1 * r(C), r(C, C) / C**0.5, r(C, C) / C**0.5,
          r(H, C) / C**0.5]  # fmt: skip
    if head_norm == "head_rms":
        ws[3] = None
    if not router:
        ws[6] = None
    cot = r(2, N, N, C)
    mix = (H, kernels.MHR_HEAD_NORMS[head_norm], kernels.MHR_ROUTER_KINDS[kind])
    leaves = [None if t is None else t.to(dev).requires_grad_(True) for t in [x] + ws]
    live = [t for t in leaves if t is not None]
    out = kernels.FusedTriMulFunction.apply(leaves[0], mask.to(dev), *leaves[1:7], 1e-5, outgoing, leaves[7], mix)
    got = torch.autograd.grad(out, live, grad_outputs=cot.to(dev))
    ref_leaves = [None if t is None else t.double().requires_grad_(True) for t in [x] + ws]
    ref = R.tri_mul_core(ref_leaves[0], mask.double(), *ref_leaves[1:7], 1e-5, outgoing, ref_leaves[7], H, head_norm,
                         kind)  # fmt: skip
    want = torch.autograd.grad(ref, [t for t in ref_leaves if t is not None], grad_outputs=cot.double())
    assert_fp32_close(out.detach().cpu(), ref.detach().float(), what="mhr update")
    names = [nm for nm, t in zip(NAMES, leaves) if t is not None]
    for a, b, nm in zip(got, want, names):
        assert a.shape == b.shape, nm
        assert_fp32_close(a.cpu(), b.float(), what=f"mhr d{nm} {head_norm} C={C}")


@pytest.mark.parametrize("C,head_norm", [(256, "head_rms"), (256, "head_ln"), (128, "post_channel")])
def test_mhr_32_heads_forward_and_gradients(dev, C, head_norm):
    """The kernels' 32-head instantiations (more than 16 heads hold the larger LDS arrays), at
    8 and 4 channels per head. (At C = 64, 32 heads have two channels each, where a per-head
    norm's pullback amplifies fp32 rounding by the rstd of two near-equal values beyond the
    1e-5 bar against fp64.)"""
    print(f"[mhr 32 heads] C={C} {head_norm}", flush=True)
    H, N, kind = 32, 26, "softmax" if C != 128 else "sigmoid"
    g = torch.Generator().manual_seed(C + 5)
    r = lambda *s: torch.randn(*s, generator=g)  # noqa: E731
    x = r(1, N, N, C)
    mask = (torch.rand(1, N, N, generator=g) > 0.15).float()
    ws = [r(2 * C, C) / C**0.5, r(2 * C, C) / C**0.5, 1 + 0.1 * r(C), 0.1 * r(C), r(C, C) / C**0.5, r(C, C) / C**0.5,
          r(H, C) / C**0.5]  # fmt: skip
    if head_norm == "head_rms":
        ws[3] = None
    cot = r(1, N, N, C)
    mix = (H, kernels.MHR_HEAD_NORMS[head_norm], kernels.MHR_ROUTER_KINDS[kind])
    leaves = [None if t is None else t.to(dev).requires_grad_(True) for t in [x] + ws]
    out = kernels.FusedTriMulFunction.apply(leaves[0], mask.to(dev), *leaves[1:7], 1e-5, True, leaves[7], mix)
    got = torch.autograd.grad(out, [t for t in leaves if t is not None], grad_outputs=cot.to(dev))
    ref_leaves = [None if t is None else t.double().requires_grad_(True) for t in [x] + ws]
    ref = R.tri_mul_core(ref_leaves[0], mask.double(), *ref_leaves[1:7], 1e-5, True, ref_leaves[7], H, head_norm, kind)
    want = torch.autograd.grad(ref, [t for t in ref_leaves if t is not None], grad_outputs=cot.double())
    assert_fp32_close(out.detach().cpu(), ref.detach().float(), what="mhr32 update")
    names = [nm for nm, t in zip(NAMES, leaves) if t is not None]
    for a, b, nm in zip(got, want, names):
        assert_fp32_close(a.cpu(), b.float(), what=f"mhr32 d{nm}")
    # the inference kernels with the same weights (block order rows [a; b] = interleaved a, b)
    m = ops.TriangleMulOutgoing(C, num_heads=H, head_norm=head_norm, router=True, router_kind=kind)
    even, odd = torch.arange(0, 2 * C, 2), torch.arange(1, 2 * C, 2)
    inv = torch.empty(2 * C, dtype=torch.long)
    inv[torch.cat((even, odd))] = torch.arange(2 * C)
    with torch.no_grad():
        m.norm_left.weight.fill_(1.0)
        m.norm_left.bias.zero_()
        m.gate.weight.copy_(ws[0][inv])
        m.proj.weight.copy_(ws[1][inv])
        m.norm_center.weight.copy_(ws[2])
        if ws[3] is not None:
            m.norm_center.bias.copy_(ws[3])
        m.out_proj.weight.copy_(ws[4])
        m.out_gate.weight.copy_(ws[5])
        m.router.weight.copy_(ws[6])
    m = m.to(dev)
    z = x * 3.0 + 0.5  # norm_left (gain 1, shift 0) of z is x up to the LayerNorm of x's rows
    with torch.no_grad():
        inf = m(z.to(dev), mask.to(dev))
    zl = torch.nn.functional.layer_norm(z.double(), (C,), eps=1e-5)
    ref_inf = R.tri_mul_core(zl, mask.double(), *[None if t is None else t.double() for t in ws[:6]], 1e-5, True,
                             ws[6].double(), H, head_norm, kind)  # fmt: skip
    assert_fp32_close(inf.cpu(), ref_inf.float(), what="mhr32 inference")


def _oracle_grads(p, z, mask, weight, outgoing, autocast, kw):
    leaves = {k: v.clone().requires_grad_(True) for k, v in p.items()}
    zz = z.clone().requires_grad_(True)
    with torch.autocast("cpu", dtype=BF, enabled=autocast):
        out = R.tri_mul(zz, mask, leaves, outgoing, **kw)
    (out.float() * weight).sum().backward()
    return {"z": zz.grad.float(), **{k: t.grad.float() for k, t in leaves.items()}}


@pytest.mark.parametrize("outgoing", [True, False], ids=["out", "in"])
def test_mhr_module_backward_matches_stock_bf16(dev, outgoing):
    """The r17 arm (C = 256, 8 heads, head_ln, softmax router) under bf16 autocast, N = 133."""
    print(f"[mhr module bwd bf16] outgoing={outgoing}", flush=True)
    C, kw = 256, _kw(256, "head_ln", True, "softmax")
    p = _params(C, outgoing, "head_ln", True, seed=17)
    g = torch.Generator().manual_seed(1)
    z = torch.randn(1, 133, 133, C, generator=g)
    mask = (torch.rand(1, 133, 133, generator=g) > 0.1).float()
    weight = torch.randn(z.shape, generator=g)
    ref32 = _oracle_grads(p, z, mask, weight, outgoing, False, kw)
    ref16 = _oracle_grads(p, z, mask, weight, outgoing, True, kw)
    m = _module(C, outgoing, "head_ln", True, "softmax", p, dev)
    x = z.to(dev).requires_grad_(True)
    with torch.autocast("cuda", dtype=BF):
        out = m(x, mask.to(dev))
    (out.float() * weight.to(dev)).sum().backward()
    got = {"z": x.grad.float().cpu(), **{k: t.grad.float().cpu() for k, t in m.named_parameters()}}
    assert set(got) == set(ref32)
    for k, ref in ref32.items():
        e_hip, e_stock = rel_l2(got[k], ref), rel_l2(ref16[k], ref)
        print(f"  {k}: hip {e_hip:.2e} stock-bf16 {e_stock:.2e}", flush=True)
        assert e_hip < 3 * e_stock + 1e-3, k


def test_mhr_inert_router_stats(dev):
    C = 64
    m = ops.TriangleMulOutgoing(C, num_heads=8, head_norm="head_rms", router=True).to(dev)
    m.router_stats_enabled = True
    g = torch.Generator().manual_seed(4)
    z = torch.randn(1, 12, 12, C, generator=g).to(dev)
    mask = torch.ones(1, 12, 12, device=dev)
    with torch.no_grad():
        m(z, mask)
        m(z, mask)
    stats = m._flush_router_stats()
    assert stats["entropy"] == pytest.approx(1.0, abs=1e-4)
    assert stats["occupancy_max"] == pytest.approx(1.0 / 8, abs=1e-4)
    assert stats["g_mean"] == pytest.approx(1.0, abs=1e-5)
    assert m._flush_router_stats() is None


def test_r17_block_fp32_eval_and_grad(dev):
    """The reference's r17 trunk block (configs/df3-stage0-r17.yaml:56-59: 256 pair channels,
    no triangle attention, 8 trimul heads, head_ln, softmax router) against the oracle's block,
    in eval and under grad (the training kernels), N = 36 with padding; z's gradient too."""
    evoformer = mod("evoformer")
    tk = dict(num_heads=8, head_norm="head_ln", router=True)
    sd = W.make_block_weights(70, perturb_affine=True, c_pair=256, num_pair_heads=8, use_triangle_attention=False,
                              trimul_num_heads=8, trimul_head_norm="head_ln", trimul_router=True)  # fmt: skip
    blk = evoformer.PairFormerBlock(256, 384, num_pair_heads=8, use_triangle_attention=False, trimul_kwargs=tk)
    blk.load_state_dict(sd)
    blk = blk.to(dev).eval()
    inp = W.make_inputs(36, seed=71, pad_last=3, c_pair=256)
    args = [inp[k] for k in ("pair", "single", "pair_mask", "seq_mask")]
    rp, rs = R.pairformer_block(*args, sd, use_triangle_attention=False, trimul_kwargs=tk)
    print("[r17 block fp32 eval]", flush=True)
    with torch.no_grad():
        p, s = blk(*[a.to(dev) for a in args])
    assert_fp32_close(p.cpu(), rp, what="r17 pair")
    assert_fp32_close(s.cpu(), rs, what="r17 single")
    print("[r17 block fp32 grad]", flush=True)
    z = args[0].clone().requires_grad_(True)
    rp, rs = R.pairformer_block(z, *args[1:], sd, use_triangle_attention=False, trimul_kwargs=tk)
    g = torch.Generator().manual_seed(72)
    wp = torch.randn(rp.shape, generator=g)
    (rp * wp).sum().backward()
    zd = args[0].to(dev).requires_grad_(True)
    p, s = blk(zd, *[a.to(dev) for a in args[1:]])
    assert_fp32_close(p.detach().cpu(), rp.detach(), what="r17 pair (grad path)")
    (p * wp.to(dev)).sum().backward()
    assert_fp32_close(zd.grad.cpu(), z.grad, what="r17 dz")
