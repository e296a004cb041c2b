"""GPU: the reference's kernel-level operators (triton/ layer) on the HIP library.

Each op is checked against a plain PyTorch fp32 restatement of the same formula (the
reference's own CPU fallbacks, e.g. fused_pair_bias.py:392-397, layernorm_linear.py:578-583),
at 1e-5 relative in fp32 and by the 2x-eager rule in bf16.
"""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from tests._helpers import assert_bf16_rule, assert_fp32_close, mod, rel_l2

pytestmark = pytest.mark.gpu
fused = mod("fused")
NotActive = mod("inference_guard").NotActive


@pytest.fixture(autouse=True)
def _highest():
    torch.set_float32_matmul_precision("highest")


def _evo_ref(Q, K, V, res_mask, pair_bias, zero_rows):
    """fp32/fp64 restatement: Q, K, V [B,S,H,N,D]; res_mask [B,S,1,1,N]; pair_bias [B,1,H,N,N]."""
    D = Q.shape[-1]
    logits = torch.matmul(Q, K.transpose(-1, -2).contiguous()) * D**-0.5 + pair_bias + res_mask
    w = torch.softmax(logits, dim=-1)
    out = torch.matmul(w, V)
    if Q.dtype == torch.float64:
        # A line whose keys are all masked: the reference kernel writes 0; the stock fp32
        # path rounds every logit to the same -1e9 and averages V uniformly. fp64 keeps the
        # logits apart, so both rules are stated here explicitly.
        dead = (res_mask < -1e8).all(dim=-1, keepdim=True)  # [B,S,1,1,1]
        fill = torch.zeros_like(out) if zero_rows else V.mean(dim=-2, keepdim=True).expand_as(out)
        out = torch.where(dead, fill, out)
    return out


def _evo_inputs(B, S, N, dtype, dev, seed=0):
    g = torch.Generator().manual_seed(seed)
    Q, K, V = (torch.randn(B, S, 4, N, 32, generator=g) for _ in range(3))
    pb = torch.randn(B, 1, 4, N, N, generator=g)
    keep = torch.rand(B, S, 1, 1, N, generator=g) > 0.15
    keep[:, 1] = False  # line 1: every key masked
    res_mask = torch.where(keep, 0.0, -1e9)
    return [t.to(dev, dtype) for t in (Q, K, V)] + [res_mask.to(dev), pb.to(dev)]


@pytest.mark.parametrize("zero_rows", [True, False])
@pytest.mark.parametrize("N", [50, 128, 200])
def test_evo_attention_fp32(dev, zero_rows, N):
    print(f"[evo attn fp32 N={N} zero={zero_rows}]", flush=True)
    Q, K, V, rm, pb = _evo_inputs(2, 5, N, torch.float32, dev, seed=N)
    with torch.no_grad():
        got = fused._EvoformerAttention.apply(Q, K, V, rm, pb, True, "zero" if zero_rows else "eager")
    ref = _evo_ref(*(t.double().cpu() for t in (Q, K, V, rm, pb)), zero_rows)
    assert_fp32_close(got.cpu(), ref.float(), what=f"evo attention N={N}")


def test_evo_attention_layouts_and_wrapper(dev):
    """pre_transposed=False takes [B,S,N,H,D]; fused_evo_attention takes the module layout with -inf masks."""
    B, S, N = 1, 6, 40
    Q, K, V, rm, pb = _evo_inputs(B, S, N, torch.float32, dev, seed=3)
    rm[:, 1] = 0.0  # no fully masked line: the wrapper's -inf masks make such a line NaN in the formula
    with torch.no_grad():
        a = fused._EvoformerAttention.apply(Q, K, V, rm, pb, True)
        b = fused._EvoformerAttention.apply(*(t.transpose(-2, -3) for t in (Q, K, V)), rm, pb, False)
        mask = (rm.view(B * S, N) > -1).float()
        q, k, v = (t.transpose(-2, -3).reshape(B * S, N, 4, 32) for t in (Q, K, V))
        c = fused.fused_evo_attention(q, k, v, pb.view(B, 4, N, N), mask)
    assert torch.allclose(b.transpose(-2, -3), a, atol=1e-6)
    assert torch.allclose(c.view(B, S, N, 4, 32).transpose(-2, -3), a, atol=1e-5)


def test_evo_attention_bf16_rule(dev):
    Q, K, V, rm, pb = _evo_inputs(1, 8, 160, torch.bfloat16, dev, seed=9)
    with torch.no_grad():
        got = fused._EvoformerAttention.apply(Q, K, V, rm, pb, True, "eager")
        eager = _evo_ref(Q, K, V, rm.to(torch.bfloat16), pb.to(torch.bfloat16), False)
    ref = _evo_ref(*(t.double().cpu() for t in (Q, K, V, rm, pb)), False).float()
    print("[evo bf16]", assert_bf16_rule(got.cpu(), eager.cpu(), ref, "evo attention bf16"), flush=True)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("with_mask", [False, True])
def test_fused_pair_bias(dev, dtype, with_mask):
    g = torch.Generator().manual_seed(1)
    B, N, C, H = 2, 37, 128, 4
    z = torch.randn(B, N, N, C, generator=g)
    w, b = 1 + 0.1 * torch.randn(C, generator=g), 0.1 * torch.randn(C, generator=g)
    pw = torch.randn(H, C, generator=g) / C**0.5
    mask = (torch.rand(B, N, generator=g) > 0.2).float() if with_mask else None
    op = fused.FusedPairBias(C, H)
    with torch.no_grad():
        got = op(z.to(dev, dtype), w.to(dev), b.to(dev), pw.to(dev), None if mask is None else mask.to(dev))
    ref = F.linear(F.layer_norm(z.double(), (C,), w.double(), b.double()), pw.double()).permute(0, 3, 1, 2)
    if mask is not None:
        ref = ref + (1.0 - mask.double()[:, None, None, :]) * (-1e9)
    assert got.dtype == dtype and got.shape == (B, H, N, N)
    if dtype == torch.float32:
        keep = ref > -1e8
        assert_fp32_close(got.cpu()[keep], ref[keep].float(), what="pair bias")
        assert torch.all(got.cpu()[~keep] < -9e8)
    else:
        ref_in = F.linear(F.layer_norm(z.to(dtype).double(), (C,), w.double(), b.double()), pw.double()).permute(0, 3, 1, 2)
        keep = ref > -1e8
        assert rel_l2(got.float().cpu()[keep], ref_in[keep]) < 1e-2


def test_fused_layernorm_linear_and_swiglu(dev):
    g = torch.Generator().manual_seed(2)
    M, K, N = 300, 384, 1536
    x = torch.randn(M, K, generator=g)
    w, b = 1 + 0.1 * torch.randn(K, generator=g), 0.1 * torch.randn(K, generator=g)
    W = torch.randn(K, N, generator=g) / K**0.5  # the reference passes [K, N]
    bias = torch.randn(N, generator=g)
    op = fused.FusedLayerNormLinear(K, N, has_linear_bias=True)
    with torch.no_grad():
        got = op(x.to(dev), w.to(dev), b.to(dev), W.to(dev), bias.to(dev))
    ref = F.linear(F.layer_norm(x.double(), (K,), w.double(), b.double()), W.double().T, bias.double())
    assert_fp32_close(got.cpu(), ref.float(), what="LayerNorm + Linear")

    h = torch.randn(7, 33, 2 * 512, generator=g).to(dev, torch.bfloat16)
    with torch.no_grad():
        y = fused.FusedSwiGLU()(h)
    a, c = h.float().chunk(2, dim=-1)
    assert torch.allclose(y.float(), (F.silu(a) * c).to(torch.bfloat16).float(), rtol=1e-2, atol=1e-2)


def test_ln_transpose_module_and_dropout_add(dev):
    g = torch.Generator().manual_seed(4)
    x = torch.randn(2, 9, 11, 128, generator=g)
    w, b = 1 + 0.1 * torch.randn(128, generator=g), 0.1 * torch.randn(128, generator=g)
    with torch.no_grad():
        got = fused.FusedLayerNormTranspose(128, True)(x.to(dev), w.to(dev), b.to(dev))
        res, upd = torch.randn(3, 5, 7, 128, generator=g).to(dev), torch.randn(3, 5, 7, 128, generator=g).to(dev)
        added = fused.dropout_add_rowwise(res, upd, 0.25, False)
        added_c = fused.dropout_add_columnwise(res, upd, 0.25, False)
    ref = F.layer_norm(x.double(), (128,), w.double(), b.double()).permute(0, 2, 1, 3)
    assert_fp32_close(got.cpu(), ref.float(), what="LN transpose")
    assert torch.equal(added, res + upd) and torch.equal(added_c, res + upd)
    # training: the HIP shared-mask dropout-add, the mask of the seed drawn after manual_seed
    from oracle import pairformer_ref as R

    kernels = mod("kernels")
    for rowwise, fn in ((True, fused.dropout_add_rowwise), (False, fused.dropout_add_columnwise)):
        torch.manual_seed(11)
        with torch.no_grad():
            got = fn(res, upd, 0.25, True)
        torch.manual_seed(11)
        m = R.shared_dropout_mask(tuple(res.shape), rowwise, 0.25, kernels.next_dropout_seed())
        assert torch.equal(got.cpu(), R.dropout_add(res.cpu(), upd.cpu(), m))


def test_fused_transition_block_keys(dev):
    blk = fused.FusedTransitionBlock(128, 4).to(dev)
    assert set(blk.state_dict()) == {"norm.weight", "norm.bias", "linear1.weight", "linear2.weight"}
    torch.nn.init.normal_(blk.linear2.weight, std=0.05)
    x = torch.randn(2, 10, 10, 128, device=dev)
    with torch.no_grad():
        y = blk(x)
    xn = F.layer_norm(x.double(), (128,), blk.norm.weight.double(), blk.norm.bias.double())
    hh = xn @ blk.linear1.weight.double().T
    a, c = hh.chunk(2, dim=-1)
    assert_fp32_close(y.cpu(), ((F.silu(a) * c) @ blk.linear2.weight.double().T).float().cpu(), what="transition")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("C", [128, 256, 384, 512])
def test_layer_norm_every_width(dev, dtype, C):
    """LayerNorm.forward (primitives.py:90-115) at every built width: fp32 statistics and
    affine, output in the input dtype. fp32 at 1e-5 against fp64; bf16 within one bf16
    rounding of the fp64 result (|err| <= 2^-8 |ref| + 1e-6) with the input taken as given."""
    g = torch.Generator().manual_seed(C)
    M = 1001  # not a multiple of the 64 rows of a block
    x = (3 * torch.randn(M, C, generator=g) + 0.5).to(dtype)
    ln = mod("primitives").LayerNorm(C).to(dev)
    with torch.no_grad():
        ln.weight.copy_(1 + 0.1 * torch.randn(C, generator=g))
        ln.bias.copy_(0.1 * torch.randn(C, generator=g))
        got = ln(x.to(dev))
    ref = F.layer_norm(x.double(), (C,), ln.weight.double().cpu(), ln.bias.double().cpu(), 1e-5)
    assert got.dtype == dtype and got.shape == x.shape
    if dtype == torch.float32:
        assert_fp32_close(got.cpu(), ref.float(), what=f"layer_norm C={C}")
    else:
        err = (got.double().cpu() - ref).abs()
        assert bool((err <= 2.0**-8 * ref.abs() + 1e-6).all()), f"C={C}: max err {err.max().item():.3e}"


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_ln_transpose_ragged(dev, dtype):
    """FusedLayerNormTranspose at B=2, N1=37, N2=70 (rows not a multiple of a block), both dtypes."""
    g = torch.Generator().manual_seed(11)
    x = torch.randn(2, 37, 70, 128, generator=g).to(dtype)
    w, b = 1 + 0.1 * torch.randn(128, generator=g), 0.1 * torch.randn(128, generator=g)
    with torch.no_grad():
        got = fused.FusedLayerNormTranspose(128, True)(x.to(dev), w.to(dev), b.to(dev))
        same = fused.FusedLayerNormTranspose(128, False)(x.to(dev), w.to(dev), b.to(dev))
    ref = F.layer_norm(x.double(), (128,), w.double(), b.double())
    assert got.shape == (2, 70, 37, 128) and same.shape == x.shape
    assert torch.equal(got.cpu(), same.cpu().permute(0, 2, 1, 3))
    if dtype == torch.float32:
        assert_fp32_close(same.cpu(), ref.float(), what="LN transpose")
    else:
        err = (same.double().cpu() - ref).abs()
        assert bool((err <= 2.0**-8 * ref.abs() + 1e-6).all()), f"max err {err.max().item():.3e}"
