"""GPU: the row GEMM over many rows (at least 16384: the LDS-tiled kernel with the store,
residual-add and SwiGLU epilogues) through the entry points that use it.

- FusedLayerNormLinear (pf_layernorm_linear_fwd): LN(x) W, 20000 rows, K=256, N=1040 (a
  ragged last tile of 16 columns) and N=64; with a bias the small-row kernel serves it.
- The generic transition (pf_transition_fwd): LN -> [256 -> 2048] -> SwiGLU -> [1024 -> 256],
  stored and added into an existing output (the SwiGLU tile pairs the two weight halves).
- Grid attention at 256 channels in 8 heads and at 64 in 4 heads with N=130 (16900 pair rows):
  the projection and output GEMMs on the tiled kernel, against the oracle.

fp32 against a float64 torch reference of the same ops at relL2 <= 1e-5 and max-abs <=
1e-5 max|ref| (the grid attention against the oracle, pinned in test_oracle.py); bf16 by the
reference's rule relL2(HIP - fp32) <= 2 relL2(eager bf16 - fp32)
(tests/triton/test_fused_trimul.py:66-83).
"""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from oracle import pairformer_ref as R
from tests._helpers import assert_bf16_rule, assert_fp32_close, mod, sub, to

pytestmark = pytest.mark.gpu
W = mod("weights")
kernels = mod("kernels")
fused = mod("fused")
attention = mod("attention")
BF = torch.bfloat16


@pytest.fixture(autouse=True)
def _highest():
    torch.set_float32_matmul_precision("highest")


def _ln(x, w, b):
    return F.layer_norm(x, (x.shape[-1],), w, b, 1e-5)


@pytest.mark.parametrize("n_out", [1040, 64])
def test_layernorm_linear_many_rows(dev, n_out):
    g = torch.Generator().manual_seed(70 + n_out)
    M, K = 20000, 256
    x = torch.randn(M, K, generator=g)
    lw, lb = 1 + 0.1 * torch.randn(K, generator=g), 0.1 * torch.randn(K, generator=g)
    w = torch.randn(K, n_out, generator=g) / K**0.5
    m = fused.FusedLayerNormLinear(K, n_out)
    print(f"[layernorm_linear many rows] M={M} K={K} N={n_out}", flush=True)
    with torch.no_grad():
        ref = _ln(x.double(), lw.double(), lb.double()) @ w.double()
        got = m(x.to(dev), lw.to(dev), lb.to(dev), w.to(dev))
        assert_fp32_close(got.cpu(), ref, what=f"LN linear fp32 N={n_out}")
        gotb = m(x.to(dev, BF), lw.to(dev), lb.to(dev), w.to(dev, BF))
        eager = _ln(x.to(dev, BF), lw.to(dev, BF), lb.to(dev, BF)) @ w.to(dev, BF)
    assert_bf16_rule(gotb.cpu(), eager.cpu(), ref.float(), f"LN linear bf16 N={n_out}")


def test_layernorm_linear_many_rows_bias(dev):
    g = torch.Generator().manual_seed(73)
    M, K, N = 20000, 256, 96
    x = torch.randn(M, K, generator=g)
    lw, lb = torch.ones(K), torch.zeros(K)
    w = torch.randn(K, N, generator=g) / K**0.5
    bias = torch.randn(N, generator=g)
    m = fused.FusedLayerNormLinear(K, N, has_linear_bias=True)
    print(f"[layernorm_linear many rows, bias] M={M} K={K} N={N}", flush=True)
    with torch.no_grad():
        ref = _ln(x.double(), lw.double(), lb.double()) @ w.double() + bias.double()
        got = m(x.to(dev), lw.to(dev), lb.to(dev), w.to(dev), bias.to(dev))
    assert_fp32_close(got.cpu(), ref, what="LN linear fp32 with bias")


def _transition_ref(x, lw, lb, w1, w2):
    h = _ln(x, lw, lb) @ w1.t()
    f = w2.shape[1]
    return (F.silu(h[:, :f]) * h[:, f:]) @ w2.t()


@pytest.mark.parametrize("accumulate", [False, True], ids=["store", "add"])
def test_transition_many_rows(dev, accumulate):
    g = torch.Generator().manual_seed(80 + int(accumulate))
    M, C, fac = 20000, 256, 4
    x = torch.randn(M, C, generator=g)
    lw, lb = 1 + 0.1 * torch.randn(C, generator=g), 0.1 * torch.randn(C, generator=g)
    w1 = torch.randn(2 * fac * C, C, generator=g) / C**0.5
    w2 = torch.randn(C, fac * C, generator=g) / (fac * C) ** 0.5
    base = torch.randn(M, C, generator=g)
    print(f"[transition many rows] M={M} C={C} accumulate={accumulate}", flush=True)
    with torch.no_grad():
        ref = _transition_ref(x.double(), lw.double(), lb.double(), w1.double(), w2.double())
        if accumulate:
            ref = ref + base.double()
        out = base.to(dev).clone() if accumulate else None
        got = kernels.transition_forward(x.to(dev), lw.to(dev), lb.to(dev), 1e-5, w1.to(dev), w2.to(dev), out=out,
                                         accumulate=accumulate)  # fmt: skip
        assert_fp32_close(got.cpu(), ref, what=f"transition fp32 accumulate={accumulate}")
        outb = base.to(dev, BF).clone() if accumulate else None
        gotb = kernels.transition_forward(x.to(dev, BF), lw.to(dev), lb.to(dev), 1e-5, w1.to(dev, BF), w2.to(dev, BF),
                                          out=outb, accumulate=accumulate)  # fmt: skip
        eager = _transition_ref(x.to(dev, BF), lw.to(dev, BF), lb.to(dev, BF), w1.to(dev, BF), w2.to(dev, BF))
        if accumulate:
            eager = eager + base.to(dev, BF)
    assert_bf16_rule(gotb.cpu(), eager.cpu(), ref.float(), f"transition bf16 accumulate={accumulate}")


def _attn(dev, c, heads, transpose, seed, dtype):
    prefix = "pair_attn_col." if transpose else "pair_attn_row."
    p = sub(W.make_block_weights(seed, perturb_affine=True, c_pair=c, num_pair_heads=heads), prefix)
    m = attention.GridSelfAttention(c, heads, transpose=transpose).eval()
    m.load_state_dict(p)
    return m.to(dev).to(dtype), p


@pytest.mark.parametrize("transpose", [False, True], ids=["rows", "cols"])
@pytest.mark.parametrize("c,heads", [(64, 4), (256, 8)])
def test_grid_attention_many_rows_fp32(dev, c, heads, transpose):
    n = 130
    m, p = _attn(dev, c, heads, transpose, 90, torch.float32)
    x = W.make_inputs(n, seed=9, pad_last=5)
    z = torch.randn(1, n, n, c, generator=torch.Generator().manual_seed(91))
    print(f"[grid attention many rows fp32] C={c} H={heads} N={n} transpose={transpose}", flush=True)
    with torch.no_grad():
        got = m(z.to(dev), x["pair_mask"].to(dev))
        ref = R.grid_attention(z, x["pair_mask"], p, transpose)
    assert_fp32_close(got.cpu(), ref, what=f"grid attention C={c} H={heads} N={n}")


def test_grid_attention_many_rows_bf16_rule(dev):
    n, c, heads = 136, 256, 8
    m, p = _attn(dev, c, heads, False, 92, BF)
    mask = W.make_inputs(n, seed=10, pad_random=7)["pair_mask"].to(dev)
    z = torch.randn(1, n, n, c, generator=torch.Generator().manual_seed(93)).to(dev).to(BF)
    with torch.no_grad():
        got = m(z, mask)
        with torch.autocast("cuda", dtype=BF):
            eager = R.grid_attention(z, mask, to(p, dev, BF), False)
        ref = R.grid_attention(z.float(), mask, to(p, dev), False)
    print("[grid attention many rows bf16] C=256 H=8 N=136",
          assert_bf16_rule(got.cpu(), eager.cpu(), ref.cpu(), "grid attention C=256 N=136"), flush=True)  # fmt: skip
