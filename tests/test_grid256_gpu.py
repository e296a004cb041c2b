"""GPU: GridSelfAttention at 256 channels in 8 heads of 32 with bf16 GEMMs (reference
``attention.py:143-269`` at the production width of ``configs/stage0.yaml:54-56``).

This regime runs the persistent projection kernel that writes the flash kernel's frame for
both four-head groups (Q, the K / Vt key-block tiles, the pair bias, the line mask) and the
gate rows, then the flash kernel per group, the gate and the output GEMM. Checked against the
fp32 oracle by the bf16 rule (relL2(HIP - fp32) <= 2 relL2(eager bf16 - fp32)), rows and
columns, with one and several 128-token tiles per line, tokens padded past N, batch 2, the
fp32 residual stream under autocast, the in-place residual, and a bias large enough that the
exact flash pass redoes the fast one.
"""

from __future__ import annotations

import pytest
import torch

from oracle import pairformer_ref as R
from tests._helpers import assert_bf16_rule, mod, rel_l2, sub, to

pytestmark = pytest.mark.gpu
W = mod("weights")
attention = mod("attention")
_lib = mod("_lib")

BF = torch.bfloat16
C, H = 256, 8


@pytest.fixture(autouse=True)
def _highest():
    torch.set_float32_matmul_precision("highest")


def _attn(dev, transpose, seed, dtype, bias_scale=1.0):
    prefix = "pair_attn_col." if transpose else "pair_attn_row."
    p = sub(W.make_block_weights(seed, perturb_affine=True, c_pair=C, num_pair_heads=H), prefix)
    p["pair_bias.weight"] = p["pair_bias.weight"] * bias_scale
    m = attention.GridSelfAttention(C, H, transpose=transpose).eval()
    m.load_state_dict(p)
    return m.to(dev).to(dtype), p


def _z(n, seed, batch=1):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(batch, n, n, C, generator=g)


def _mask(n, seed, batch=1, pad=5):
    return torch.cat([W.make_inputs(n, seed=seed + b, pad_random=pad)["pair_mask"] for b in range(batch)], 0)


def _check(m, p, z, mask, transpose, what, autocast=False):
    with torch.no_grad():
        if autocast:
            with torch.autocast("cuda", dtype=BF):
                got = m(z, mask)
        else:
            got = m(z, mask)
        with torch.autocast("cuda", dtype=BF):
            eager = R.grid_attention(z.to(BF), mask, to(p, z.device, BF), transpose)
        ref = R.grid_attention(z.float(), mask, to(p, z.device), transpose)
    assert bool(torch.isfinite(got).all()), what
    print(f"[grid256 {what}]", assert_bf16_rule(got.float().cpu(), eager.float().cpu(), ref.cpu(), what), flush=True)
    return got


@pytest.mark.parametrize("transpose", [False, True], ids=["rows", "cols"])
@pytest.mark.parametrize("n", [80, 200, 256])
def test_grid256_bf16_rule(dev, n, transpose):
    """One tile per line with padding (80 -> 128), two tiles with padding (200 -> 256), two
    full tiles (256)."""
    m, p = _attn(dev, transpose, 60 + n, BF)
    print(f"[grid256] N={n} transpose={transpose}", flush=True)
    _check(m, p, _z(n, n + 1).to(dev, BF), _mask(n, n + 2).to(dev), transpose, f"N={n} transpose={transpose}")


@pytest.mark.parametrize("transpose", [False, True], ids=["rows", "cols"])
def test_grid256_batch2(dev, transpose):
    m, p = _attn(dev, transpose, 71, BF)
    print(f"[grid256] batch 2 N=96 transpose={transpose}", flush=True)
    z = _z(96, 72, batch=2).to(dev, BF)
    got = _check(m, p, z, _mask(96, 73, batch=2).to(dev), transpose, f"batch2 transpose={transpose}")
    # batch items are independent: item 1 alone gives the same result
    with torch.no_grad():
        one = m(z[1:], _mask(96, 73, batch=2)[1:].to(dev))
    assert torch.equal(one, got[1:])


@pytest.mark.parametrize("transpose", [False, True], ids=["rows", "cols"])
def test_grid256_fp32_stream_autocast(dev, transpose):
    """fp32 residual stream, bf16 GEMM operands (the reference's autocast inference)."""
    m, p = _attn(dev, transpose, 74, torch.float32)
    print(f"[grid256] fp32 stream N=130 transpose={transpose}", flush=True)
    _check(m, p, _z(130, 75).to(dev), _mask(130, 76).to(dev), transpose, f"fp32-stream transpose={transpose}",
           autocast=True)  # fmt: skip


@pytest.mark.parametrize("transpose", [False, True], ids=["rows", "cols"])
def test_grid256_residual_in_place(dev, transpose):
    """forward_residual_ adds the update in the output GEMM's epilogue: equal to z + forward(z)
    up to the rounding of the separately stored update."""
    m, _ = _attn(dev, transpose, 77, BF)
    print(f"[grid256] in-place residual transpose={transpose}", flush=True)
    z = _z(100, 78).to(dev, BF)
    mask = _mask(100, 79).to(dev)
    with torch.no_grad():
        upd = m(z, mask)
        got = m.forward_residual_(z.clone(), mask)
    want = z.float() + upd.float()
    err = (got.float() - want).abs().max().item()
    tol = 2.0 ** -7 * want.abs().max().item()
    assert err <= tol, f"in-place residual: max |diff| {err:.3e} > {tol:.3e}"


@pytest.mark.parametrize("transpose", [False, True], ids=["rows", "cols"])
def test_grid256_exact_redo(dev, transpose):
    """A pair-bias projection scaled by 300 (bias ~ +-1e3) overflows the fast pass; the exact
    pass redoes the flagged blocks and the result still meets the bf16 rule. Lines lose their
    first 32 / 64 keys or a middle block, none all of them: a fully masked line takes the
    eager rule's uniform average, which a bias of this size breaks in the fp32 reference
    (-1e9 + bias rounds to multiples of 64)."""
    m, p = _attn(dev, transpose, 80, BF, bias_scale=300.0)
    print(f"[grid256] exact redo transpose={transpose}", flush=True)
    z = _z(100, 81).to(dev, BF)
    mask = W.make_inputs(100, seed=82)["pair_mask"].clone()
    lines = mask.transpose(1, 2) if transpose else mask  # the line is the mask's row (rows) or column
    lines[0, 3, :32] = 0.0
    lines[0, 6, :64] = 0.0
    lines[0, 50, 32:64] = 0.0
    mask = mask.to(dev)
    with torch.no_grad(), _lib.RedoRecorder() as counts:
        got = m(z, mask)
    assert counts and counts[0] > 0, "the exact pass never ran"
    with torch.no_grad():
        with torch.autocast("cuda", dtype=BF):
            eager = R.grid_attention(z, mask, to(p, dev, BF), transpose)
        ref = R.grid_attention(z.float(), mask, to(p, dev), transpose)
    assert bool(torch.isfinite(got).all())
    e_h, e_e = rel_l2(got.float().cpu(), ref.cpu()), rel_l2(eager.float().cpu(), ref.cpu())
    print(f"[grid256 exact redo transpose={transpose}] hip {e_h:.3e} eager {e_e:.3e} redo {counts}", flush=True)
    assert e_h <= 2 * e_e, f"relL2(hip)={e_h:.3e} > 2 x eager {e_e:.3e}"
