"""GPU: the backward of the fused attention op (``_EvoformerAttention``, evo_attention.py:1295-1472).

- Against the oracle's centred backward in fp64 (itself pinned to autograd and finite
  differences in test_oracle.py): fp32 at relL2 <= 1e-5 and max-abs <= 1e-5 max|ref| for dQ,
  dK, dV and d_pair_bias, with ragged N, random key masks, a fully masked line (zero
  gradients) and head counts 2, 4 and 8.
- The reference's own backward gate (tests/triton/test_evo_attn_robustness.py:340-389):
  shapes (1,1,128,4,32) and (1,2,384,8,32), seeds 0/42/99, fp32 and bf16, per-element
  tolerance atol_frac * max|ref| + rtol |ref| with at most 0.1 % of elements outside, the
  reference's (atol_frac, rtol) policy, here against fp64.
- Softmax collapse (tests/triton/test_evo_attn_softmax_collapse.py): winner-take-all pair
  bias at margin ~14.5; dQ within 0.1 of the true peak and d_pair_bias rows summing to
  <= 0.05 of their peak.
- The module-layout wrapper, bitwise-reproducible gradients, and the stock masked-row rule
  under grad (``masked_rows="eager"``) against autograd of the stock formula, a fully masked
  line included.
- The strided entry points (GridSelfAttention's training path on its token-major
  projection, rows and columns) against the dense ones on the same values: O, dQ, dK, dV
  and d_pair_bias bit for bit; with the forward's saved row LSE (single dQ pass) against
  the two-pass backward, flat and peaked softmax.
"""

from __future__ import annotations

import math

import pytest
import torch

from oracle import pairformer_ref as R
from tests._helpers import assert_fp32_close, mod

pytestmark = pytest.mark.gpu
fused = mod("fused")
NotActive = mod("inference_guard").NotActive
BF = torch.bfloat16


def _inputs(B, S, H, N, dtype, seed, mask_frac=0.85, dead_line=True, sigma=1.0, layout="kernel"):
    g = torch.Generator().manual_seed(seed)
    D = 32
    qs = sigma / math.sqrt(D)
    Q, K = (torch.randn(B, S, H, N, D, generator=g) * qs for _ in range(2))
    V = torch.randn(B, S, H, N, D, generator=g) * sigma
    pb = torch.randn(B, 1, H, N, N, generator=g)
    keep = torch.rand(B, S, 1, 1, N, generator=g) < mask_frac
    keep[..., 0] = True
    if dead_line and S > 1:
        keep[:, 1] = False
    rm = torch.where(keep, 0.0, -1e9)
    dO = torch.randn(B, S, H, N, D, generator=g) * 0.1
    Q, K, V, dO = (t.to(dtype) for t in (Q, K, V, dO))
    return Q, K, V, rm, pb, dO


def _hip_grads(Q, K, V, rm, pb, dO, dev):
    leaves = [t.to(dev).requires_grad_(True) for t in (Q, K, V, pb)]
    out = fused._EvoformerAttention.apply(leaves[0], leaves[1], leaves[2], rm.to(dev), leaves[3], True)
    grads = torch.autograd.grad(out, leaves, grad_outputs=dO.to(dev))
    return [g.float().cpu() for g in grads], out.detach()


def _oracle_grads(Q, K, V, rm, pb, dO):
    return R.evo_attention_backward(*(t.double() for t in (Q, K, V, rm, pb, dO)))


@pytest.mark.parametrize("B,S,H,N", [(2, 3, 4, 50), (1, 2, 8, 128), (1, 3, 2, 70), (1, 2, 4, 200)])
def test_attn_backward_fp32(dev, B, S, H, N):
    print(f"[attn bwd fp32] B={B} S={S} H={H} N={N}", flush=True)
    Q, K, V, rm, pb, dO = _inputs(B, S, H, N, torch.float32, seed=N + H)
    got, out = _hip_grads(Q, K, V, rm, pb, dO, dev)
    want = _oracle_grads(Q, K, V, rm, pb, dO)
    for a, b, name in zip(got, want, ("dQ", "dK", "dV", "d_pair_bias")):
        assert a.shape == b.shape, name
        assert_fp32_close(a, b.float(), what=f"{name} N={N} H={H}")
    # the fully masked line: output and every gradient are 0
    assert torch.count_nonzero(out[:, 1]) == 0
    for a in got[:3]:
        assert torch.count_nonzero(a[:, 1]) == 0


def _metrics(kernel, ref, atol_frac, rtol):
    kf, rf = kernel.double(), ref.double()
    tol = atol_frac * rf.abs().max() + rtol * rf.abs()
    return float(((kf - rf).abs() > tol).double().mean()), bool(torch.isfinite(kf).all())


# (atol_frac, rtol) of the reference's BWD_QKV_POLICY / BWD_BIAS_POLICY (fp32 entries are its TF32 ones)
POLICY = {torch.float32: ((5e-3, 1e-2), (5e-3, 1e-2)), BF: ((5e-3, 5e-2), (5e-3, 2e-2))}


@pytest.mark.parametrize("B,S,N,H", [(1, 1, 128, 4), (1, 2, 384, 8)])
@pytest.mark.parametrize("seed", [0, 42, 99])
@pytest.mark.parametrize("dtype", [torch.float32, BF], ids=["fp32", "bf16"])
def test_attn_backward_reference_gate(dev, dtype, seed, B, S, N, H):
    print(f"[attn bwd gate] {dtype} seed={seed} S={S} N={N} H={H}", flush=True)
    Q, K, V, rm, pb, dO = _inputs(B, S, H, N, dtype, seed, mask_frac=1.0, dead_line=False)
    got, _ = _hip_grads(Q, K, V, rm, pb, dO, dev)
    want = _oracle_grads(Q, K, V, rm, pb, dO)
    qkv, bias = POLICY[dtype]
    for a, b, name in zip(got, want, ("dQ", "dK", "dV", "d_pair_bias")):
        frac, finite = _metrics(a, b, *(bias if name == "d_pair_bias" else qkv))
        assert finite and frac <= 1e-3, f"{name}: fail_frac {frac:.3e}"


def _wta(spike: float, dtype=BF, seed=42):
    """Winner-take-all: +spike on one pair-bias column per head (B1 S2 N256 H8 D32)."""
    B, S, N, H, D = 1, 2, 256, 8, 32
    g = torch.Generator().manual_seed(seed)
    qs = D**-0.5
    Q, K = (torch.randn(B, S, H, N, D, generator=g) * qs for _ in range(2))
    V = torch.randn(B, S, H, N, D, generator=g)
    pb = torch.randn(B, 1, H, N, N, generator=g) * 0.1
    for h in range(H):
        pb[:, :, h, :, (h * 37) % N] += spike
    dO = torch.randn(B, S, H, N, D, generator=g) * 0.1
    rm = torch.zeros(B, S, 1, 1, N)
    Q, K, V, dO = (t.to(dtype) for t in (Q, K, V, dO))
    return Q, K, V, rm, pb, dO


def test_attn_backward_softmax_collapse(dev):
    Q, K, V, rm, pb, dO = _wta(20.0)
    t = torch.matmul(Q.double(), K.double().transpose(-1, -2)) * 32**-0.5 + pb.double()
    imax = t.argmax(-1, keepdim=True)
    margin = (t.gather(-1, imax) - torch.logsumexp(t.scatter(-1, imax, -torch.inf), -1, keepdim=True)).mean()
    assert 13.0 < float(margin) < 16.6
    print(f"[attn bwd collapse] margin {float(margin):.2f}", flush=True)
    got, _ = _hip_grads(Q, K, V, rm, pb, dO, dev)
    want = _oracle_grads(Q, K, V, rm, pb, dO)
    peak = want[0].abs().max()
    assert 3e-8 < float(peak) < 1e-6  # the true dQ is small but not noise
    err = (got[0].double() - want[0]).abs().max()
    assert err <= 0.1 * peak, f"dQ error {float(err):.3e} vs true peak {float(peak):.3e}"
    db = got[3]
    assert want[3].sum(-1).abs().max() <= 1e-6 * want[3].abs().max()
    assert db.sum(-1).abs().max() <= 0.05 * db.abs().max(), "d_pair_bias rows no longer sum to zero"


def test_attn_backward_wrapper_and_determinism(dev):
    B, S, N, H = 1, 4, 96, 4
    Q, K, V, rm, pb, dO = _inputs(B, S, H, N, BF, seed=5, dead_line=False)
    # module layout: q, k, v [B*S, N, H, D], pair_bias [B, H, N, N], mask [B*S, N] (1 keep)
    mask = (rm.view(B * S, N) > -1).float().to(dev)
    q, k, v = (t.transpose(-2, -3).reshape(B * S, N, H, 32).to(dev).requires_grad_(True) for t in (Q, K, V))
    p = pb.view(B, H, N, N).to(dev).requires_grad_(True)
    o = fused.fused_evo_attention(q, k, v, p, mask)
    do = dO.transpose(-2, -3).reshape(B * S, N, H, 32).to(dev)
    g1 = torch.autograd.grad(o, [q, k, v, p], grad_outputs=do)
    got, _ = _hip_grads(Q, K, V, rm, pb, dO, dev)
    assert torch.equal(g1[0].float().cpu().view(B, S, N, H, 32).transpose(-2, -3), got[0])
    assert torch.equal(g1[3].float().cpu(), got[3].view(B, H, N, N))
    again, _ = _hip_grads(Q, K, V, rm, pb, dO, dev)
    for a, b in zip(got, again):
        assert torch.equal(a, b)


def _stock_grads(Q, K, V, rm, pb, dO):
    """Autograd of the stock eager path (``attention.py:151-160``): fp64 products, the softmax on
    the logits cast to fp32 (``softmax(logits.float())``), where a fully masked line's -1e9-shifted
    logits round to one value and its weights are uniform."""
    leaves = [t.double().clone().requires_grad_(True) for t in (Q, K, V, pb)]
    q, k, v, b = leaves
    logits = torch.matmul(q, k.transpose(-1, -2)) * 32**-0.5 + b + rm.double()
    out = torch.matmul(torch.softmax(logits.float(), dim=-1).double(), v)
    return [g.float() for g in torch.autograd.grad(out, leaves, grad_outputs=dO.double())], out.float()


@pytest.mark.parametrize("B,S,H,N", [(1, 3, 4, 50), (2, 2, 4, 128)])
def test_attn_backward_eager_rule(dev, B, S, H, N):
    """``masked_rows="eager"`` under grad: the forward and every gradient follow the stock path,
    a fully masked line included (uniform weights; nonzero gradients there), fp32 at 1e-5."""
    print(f"[attn bwd eager rule] B={B} S={S} H={H} N={N}", flush=True)
    Q, K, V, rm, pb, dO = _inputs(B, S, H, N, torch.float32, seed=N + 3)
    assert bool((rm[:, 1] < 0).all())  # line 1 is fully masked
    leaves = [t.to(dev).requires_grad_(True) for t in (Q, K, V, pb)]
    out = fused._EvoformerAttention.apply(leaves[0], leaves[1], leaves[2], rm.to(dev), leaves[3], True, "eager")
    got = [g.float().cpu() for g in torch.autograd.grad(out, leaves, grad_outputs=dO.to(dev))]
    want, ref_out = _stock_grads(Q, K, V, rm, pb, dO)
    assert_fp32_close(out.detach().cpu(), ref_out, what="O")
    for name, a, b in zip(("dQ", "dK", "dV", "d_pair_bias"), got, want):
        assert_fp32_close(a, b, what=name)
    assert float(got[0][:, 1].abs().max()) > 0 and float(got[2][:, 1].abs().max()) > 0
    # the reference kernel's rule zeroes that line's gradients instead
    zero, _ = _hip_grads(Q, K, V, rm, pb, dO, dev)
    assert float(zero[0][:, 1].abs().max()) == 0.0 and float(zero[2][:, 1].abs().max()) == 0.0


def _grid_module(transpose, c=128, heads=4, seed=7):
    W = mod("weights")
    attention = mod("attention")
    prefix = "pair_attn_col." if transpose else "pair_attn_row."
    p = {k[len(prefix):]: v for k, v in W.make_block_weights(seed, perturb_affine=True, c_pair=c,
                                                            num_pair_heads=heads).items() if k.startswith(prefix)}  # fmt: skip
    m = attention.GridSelfAttention(c, heads, transpose=transpose)
    m.load_state_dict(p)
    return m, p


def _grid_oracle_grads(p, z, mask, weight, transpose, autocast, dtype=torch.float32):
    leaves = {k: v.to(dtype).clone().requires_grad_(True) for k, v in p.items()}
    zz = z.to(dtype).clone().requires_grad_(True)
    with torch.autocast("cpu", dtype=BF, enabled=autocast):
        out = R.grid_attention(zz, mask.to(dtype), leaves, transpose)
    (out.to(dtype) * weight.to(dtype)).sum().backward()
    return {"z": zz.grad.float(), **{k: t.grad.float() for k, t in leaves.items()}}


def _pair_mask(B, N, seed):
    g = torch.Generator().manual_seed(seed)
    m = (torch.rand(B, N, N, generator=g) > 0.1).float()
    m[:, :, 0] = 1.0  # no fully masked line (the training kernel's rule and the stock rule differ there)
    m[:, 0, :] = 1.0
    return m


@pytest.mark.parametrize("transpose", [False, True], ids=["rows", "cols"])
def test_grid_attention_module_backward_fp32(dev, transpose):
    """GridSelfAttention under grad (attention.py:211-257 with the fused op) against the stock
    module differentiated in fp64: every gradient at 1e-5."""
    m, p = _grid_module(transpose)
    N = 45
    g = torch.Generator().manual_seed(8)
    z = torch.randn(1, N, N, 128, generator=g)
    mask = _pair_mask(1, N, 9)
    weight = torch.randn(z.shape, generator=g)
    want = _grid_oracle_grads(p, z, mask, weight, transpose, False, torch.float64)
    m = m.to(dev)
    x = z.to(dev).requires_grad_(True)
    out = m(x, mask.to(dev))
    (out * weight.to(dev)).sum().backward()
    got = {"z": x.grad.cpu(), **{k: t.grad.cpu() for k, t in m.named_parameters()}}
    for k, ref in want.items():
        assert_fp32_close(got[k], ref, what=f"grid attention d{k}")


@pytest.mark.parametrize("transpose", [False, True], ids=["rows", "cols"])
def test_grid_attention_module_backward_bf16(dev, transpose):
    """Under bf16 autocast (the reference's training regime): each gradient within 3x the
    stock path's bf16 error (+1e-3), as tests/triton/test_fused_trimul.py:87-106 gates the
    fused trimul; stock references on the CPU."""
    m, p = _grid_module(transpose, seed=10)
    B, N = 1, 96
    g = torch.Generator().manual_seed(11)
    z = torch.randn(B, N, N, 128, generator=g)
    mask = _pair_mask(B, N, 12)
    weight = torch.randn(z.shape, generator=g)
    ref32 = _grid_oracle_grads(p, z, mask, weight, transpose, False)
    ref16 = _grid_oracle_grads(p, z, mask, weight, transpose, True)
    m = m.to(dev)
    x = z.to(dev).requires_grad_(True)
    with torch.autocast("cuda", dtype=BF):
        out = m(x, mask.to(dev))
    (out.float() * weight.to(dev)).sum().backward()
    got = {"z": x.grad.float().cpu(), **{k: t.grad.float().cpu() for k, t in m.named_parameters()}}
    from tests._helpers import rel_l2

    for k, ref in ref32.items():
        e_hip, e_stock = rel_l2(got[k], ref), rel_l2(ref16[k], ref)
        print(f"  {k}: hip {e_hip:.2e} stock-bf16 {e_stock:.2e}", flush=True)
        assert e_hip < 3 * e_stock + 1e-3, k


def _strided_case(dev, transpose, dtype, bias_sigma):
    B, N, H, D = 2, 45, 4, 32
    g = torch.Generator().manual_seed(17 + int(transpose))
    qkv = (torch.randn(B, N, N, 3, H, D, generator=g) * 0.4).to(dev, dtype)
    keep = torch.rand(B, N, N, generator=g) < 0.85
    keep[:, :, 0] = True
    keep[:, 5] = False  # a fully masked line
    rm = torch.where(keep, 0.0, -1e9).to(dev)  # [B, lines, keys]
    pb = (torch.randn(B, H, N, N, generator=g) * bias_sigma).to(dev)
    dO = torch.randn(B, N, N, H, D, generator=g).to(dev, dtype)
    return qkv, rm, pb, dO


def _run_strided(qkv, rm, pb, dO, transpose, use_lse):
    x = qkv.clone().requires_grad_(True)
    p = pb.clone().requires_grad_(True)
    saved = fused._GridAttnCore.use_lse
    fused._GridAttnCore.use_lse = use_lse
    try:
        o = fused._GridAttnCore.apply(x, rm, p, transpose)
        o.backward(dO)
    finally:
        fused._GridAttnCore.use_lse = saved
    return o, x.grad, p.grad


def _run_dense(qkv, rm, pb, dO, transpose):
    frame = (0, 2, 3, 1, 4) if transpose else (0, 1, 3, 2, 4)  # [B, line, H, key, D]
    back = (0, 3, 1, 2, 4) if transpose else (0, 1, 3, 2, 4)
    x = qkv.clone().requires_grad_(True)
    p = pb.clone().requires_grad_(True)
    q, k, v = (x[:, :, :, i].permute(*frame).contiguous() for i in range(3))
    o = fused._EvoAttnFunction.apply(q, k, v, rm, p).permute(*back)
    o.backward(dO)
    return o, x.grad, p.grad


@pytest.mark.parametrize("dtype", [torch.float32, BF], ids=["fp32", "bf16"])
@pytest.mark.parametrize("transpose", [False, True], ids=["rows", "cols"])
def test_strided_attention_equals_dense(dev, transpose, dtype):
    """fused._GridAttnCore (strides, two-pass backward) against _EvoAttnFunction on the
    permuted, contiguous operands: the same packed operands reach the same kernels, so every
    output is equal."""
    qkv, rm, pb, dO = _strided_case(dev, transpose, dtype, 1.0)
    print(f"[strided attention] transpose={transpose} dtype={dtype}", flush=True)
    o1, gx1, gp1 = _run_strided(qkv, rm, pb, dO, transpose, use_lse=False)
    o2, gx2, gp2 = _run_dense(qkv, rm, pb, dO, transpose)
    assert torch.equal(o1, o2)
    assert torch.equal(gx1, gx2)
    assert torch.equal(gp1, gp2)


@pytest.mark.parametrize("bias_sigma", [1.0, 6.0], ids=["flat", "peaked"])
@pytest.mark.parametrize("dtype", [torch.float32, BF], ids=["fp32", "bf16"])
@pytest.mark.parametrize("transpose", [False, True], ids=["rows", "cols"])
def test_strided_attention_saved_lse(dev, transpose, dtype, bias_sigma):
    """The backward on the forward's saved row LSE (one dQ pass, re-centred on the dominant
    key when it is reached) against the two-pass backward: the same O; gradients within
    relL2 1e-5 of the two-pass fp32 ones in fp32, and in bf16 no further from the fp32
    two-pass gradients than the bf16 two-pass ones (x 1.25 + 1e-4). The peaked case (pair
    bias sigma 6) puts most rows' mass on one key, some of them in the second key tile."""
    qkv, rm, pb, dO = _strided_case(dev, transpose, dtype, bias_sigma)
    print(f"[strided attention lse] transpose={transpose} dtype={dtype} sigma={bias_sigma}", flush=True)
    o1, gx1, gp1 = _run_strided(qkv, rm, pb, dO, transpose, use_lse=True)
    o2, gx2, gp2 = _run_strided(qkv, rm, pb, dO, transpose, use_lse=False)
    assert torch.equal(o1, o2)
    assert torch.isfinite(gx1).all() and torch.isfinite(gp1).all()
    from tests._helpers import rel_l2

    if dtype == torch.float32:
        for a, b, what in ((gx1, gx2, "dqkv"), (gp1, gp2, "dpair_bias")):
            e = rel_l2(a.cpu(), b.cpu())
            print(f"  {what}: relL2 {e:.2e}", flush=True)
            assert e <= 1e-5, what
    else:
        _, rx, rp = _run_strided(qkv.float(), rm, pb, dO.float(), transpose, use_lse=False)
        for a, b, r, what in ((gx1, gx2, rx, "dqkv"), (gp1, gp2, rp, "dpair_bias")):
            e1, e2 = rel_l2(a.float().cpu(), r.cpu()), rel_l2(b.float().cpu(), r.cpu())
            print(f"  {what}: lse {e1:.2e} two-pass {e2:.2e}", flush=True)
            assert e1 <= 1.25 * e2 + 1e-4, what
    # the fully masked line has zero gradients either way
    line = (slice(None), slice(None), 5) if transpose else (slice(None), 5)
    assert not gx1[line].any()
