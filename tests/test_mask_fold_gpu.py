"""GPU: the two mask paths of grid attention.

When the pair mask is the outer product of its binary diagonal (the trunk's
``seq_mask x seq_mask``, ``featurizer.py:520``), every live line masks the same keys, so the
projection kernel folds ``1e9 (m_k - 1)`` into the shared pair bias and the flash kernel
runs without per-line key masks. Masked keys come out at ~ -1.44e9 on both paths (exp2
gives 0), unmasked keys add exactly 0, padding keys are -inf on both: the outputs must be
bit-identical. Any other mask takes the per-line path; the check must tell them apart.
"""

from __future__ import annotations

import pytest
import torch

from tests._helpers import mod

pytestmark = pytest.mark.gpu
W = mod("weights")
kernels = mod("kernels")
attention = mod("attention")
BF = torch.bfloat16


def _seq_outer(n: int, pad: list[int], b: int = 1, dev="cuda") -> torch.Tensor:
    seq = torch.ones(b, n)
    seq[:, pad] = 0.0
    return (seq[:, :, None] * seq[:, None, :]).to(dev)


def test_outer_product_check(dev):
    n = 50
    outer = _seq_outer(n, [3, 17, 49], dev=dev)
    assert kernels.pair_mask_is_outer(outer)
    km = kernels.outer_key_mask(outer)
    assert torch.equal(km, (torch.diagonal(outer, dim1=1, dim2=2) - 1.0) * 1e9)
    assert kernels.pair_mask_is_outer(torch.ones(2, n, n, device=dev))
    g = torch.Generator().manual_seed(0)
    per_line = (torch.rand(1, n, n, generator=g) > 0.1).float().to(dev)
    assert not kernels.pair_mask_is_outer(per_line)
    frac = (0.5 * _seq_outer(n, [], dev=dev)).contiguous()
    assert not kernels.pair_mask_is_outer(frac)
    off = outer.clone()
    off[0, 3, 10] = 1.0  # key 10 unmasked on line 3, whose own diagonal is 0
    assert not kernels.pair_mask_is_outer(off)
    mixed = torch.cat([_seq_outer(n, [5], dev=dev), per_line])
    assert not kernels.pair_mask_is_outer(mixed)
    # cached per object and version: an in-place change is seen
    outer2 = outer.clone()
    assert kernels.pair_mask_is_outer(outer2)
    outer2[0, 0, 3] = 1.0
    assert not kernels.pair_mask_is_outer(outer2)


def _module(dev, dtype, transpose, seed):
    sd = W.make_block_weights(seed)
    prefix = "pair_attn_col." if transpose else "pair_attn_row."
    m = attention.GridSelfAttention(128, 4, transpose=transpose).to(dev)
    m.load_state_dict({k[len(prefix) :]: v for k, v in sd.items() if k.startswith(prefix)})
    return m.to(dtype).eval()


@pytest.mark.parametrize("dtype", [BF, torch.float32], ids=["bf16", "fp32"])
@pytest.mark.parametrize("transpose", [False, True], ids=["rows", "cols"])
@pytest.mark.parametrize("n,pad", [(70, [1, 40, 69]), (100, list(range(90, 100))), (128, [0, 64])])
def test_folded_mask_is_bit_identical(dev, dtype, transpose, n, pad):
    m = _module(dev, dtype, transpose, 5)
    g = torch.Generator().manual_seed(n)
    z = torch.randn(1, n, n, 128, generator=g).to(dev, dtype)
    mask = _seq_outer(n, pad, dev=dev)
    op = m._operands(kernels.gemm_dtype_for(z))
    args = (z, mask, op["lnw"], op["lnb"], m.norm.eps, op["w5"], op["w_out"], transpose)
    print(f"[mask fold] n={n} transpose={transpose} dtype={dtype}", flush=True)
    with torch.no_grad():
        folded = kernels.grid_attention_forward(*args, mask_outer=True)
        general = kernels.grid_attention_forward(*args, mask_outer=False)
        auto = kernels.grid_attention_forward(*args)
    assert torch.isfinite(folded.float()).all()
    assert torch.equal(folded, general)
    assert torch.equal(auto, folded)


def _module256(dev, transpose, seed):
    sd = W.make_block_weights(seed, c_pair=256, num_pair_heads=8)
    prefix = "pair_attn_col." if transpose else "pair_attn_row."
    m = attention.GridSelfAttention(256, 8, transpose=transpose).to(dev)
    m.load_state_dict({k[len(prefix) :]: v for k, v in sd.items() if k.startswith(prefix)})
    return m.to(BF).eval()


@pytest.mark.parametrize("transpose", [False, True], ids=["rows", "cols"])
@pytest.mark.parametrize("n,pad", [(70, [1, 40, 69]), (200, list(range(190, 200)))])
def test_folded_mask_is_bit_identical_c256(dev, transpose, n, pad):
    """The 256-channel, 8-head bf16 path: both four-head groups fold the key mask the same
    way (rows: a pass over the bias; columns: inside the transpose)."""
    m = _module256(dev, transpose, 6)
    g = torch.Generator().manual_seed(n + 1)
    z = torch.randn(1, n, n, 256, generator=g).to(dev, BF)
    mask = _seq_outer(n, pad, dev=dev)
    op = m._operands(kernels.gemm_dtype_for(z))
    args = (z, mask, op["lnw"], op["lnb"], m.norm.eps, op["w5"], op["w_out"], transpose)
    print(f"[mask fold C=256] n={n} transpose={transpose}", flush=True)
    with torch.no_grad():
        folded = kernels.grid_attention_forward(*args, num_heads=8, mask_outer=True)
        general = kernels.grid_attention_forward(*args, num_heads=8, mask_outer=False)
        auto = kernels.grid_attention_forward(*args, num_heads=8)
    assert torch.isfinite(folded.float()).all()
    assert torch.equal(folded, general)
    assert torch.equal(auto, folded)
