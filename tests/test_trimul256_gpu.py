"""GPU: triangle multiplication at 256 channels with bf16 GEMMs and a bf16 stream (reference
``ops.py:412-473``, ``:645-680`` at the production width of ``configs/stage0.yaml:54-56``).

This regime runs the persistent 256-channel kernels: the weight-streaming projection (K1,
128-position tiles) and the weight-stationary output kernel (K3, 64-position tiles, out_proj
and out_gate rows resident in registers) around the contraction. Checked against the fp32
oracle by the bf16 rule (relL2(HIP - fp32) <= 2 relL2(eager bf16 - fp32)) in both
directions, with tiles cut by N (N = 64, 100, 130, 200), batch 2 (items independent, bit for
bit), and the in-place residual (``forward_residual_``) against z + forward(z).
"""

from __future__ import annotations

import pytest
import torch

from oracle import pairformer_ref as R
from tests._helpers import assert_bf16_rule, mod, sub, to

pytestmark = pytest.mark.gpu
W = mod("weights")
ops = mod("ops")

BF = torch.bfloat16
C = 256


@pytest.fixture(autouse=True)
def _highest():
    torch.set_float32_matmul_precision("highest")


def _trimul(dev, outgoing, seed):
    prefix = "tri_mul_out." if outgoing else "tri_mul_in."
    p = sub(W.make_block_weights(seed, perturb_affine=True, c_pair=C), prefix)
    m = (ops.TriangleMulOutgoing if outgoing else ops.TriangleMulIncoming)(C).eval()
    m.load_state_dict(p)
    return m.to(dev).to(BF), p


def _z(n, seed, batch=1):
    return torch.randn(batch, n, n, C, generator=torch.Generator().manual_seed(seed))


def _mask(n, seed, batch=1, pad=6):
    return torch.cat([W.make_inputs(n, seed=seed + b, pad_random=pad)["pair_mask"] for b in range(batch)], 0)


@pytest.mark.parametrize("outgoing", [True, False], ids=["out", "in"])
@pytest.mark.parametrize("n", [64, 100, 130, 200])
def test_trimul256_bf16_rule(dev, n, outgoing):
    m, p = _trimul(dev, outgoing, 90 + n)
    print(f"[trimul256] N={n} outgoing={outgoing}", flush=True)
    z = _z(n, n + 3).to(dev, BF)
    mask = _mask(n, n + 4).to(dev)
    with torch.no_grad():
        got = m(z, mask)
        with torch.autocast("cuda", dtype=BF):
            eager = R.tri_mul(z, mask, to(p, dev, BF), outgoing)
        ref = R.tri_mul(z.float(), mask, to(p, dev), outgoing)
    assert bool(torch.isfinite(got).all())
    print(f"[trimul256 N={n} outgoing={outgoing}]",
          assert_bf16_rule(got.float().cpu(), eager.float().cpu(), ref.cpu(), f"trimul256 N={n}"), flush=True)  # fmt: skip


@pytest.mark.parametrize("outgoing", [True, False], ids=["out", "in"])
def test_trimul256_batch2(dev, outgoing):
    m, p = _trimul(dev, outgoing, 97)
    print(f"[trimul256] batch 2 N=80 outgoing={outgoing}", flush=True)
    z = _z(80, 98, batch=2).to(dev, BF)
    mask = _mask(80, 99, batch=2).to(dev)
    with torch.no_grad():
        got = m(z, mask)
        one = m(z[1:], mask[1:])
        with torch.autocast("cuda", dtype=BF):
            eager = R.tri_mul(z, mask, to(p, dev, BF), outgoing)
        ref = R.tri_mul(z.float(), mask, to(p, dev), outgoing)
    assert torch.equal(one, got[1:]), "batch items must not interact"
    print(f"[trimul256 batch2 outgoing={outgoing}]",
          assert_bf16_rule(got.float().cpu(), eager.float().cpu(), ref.cpu(), "trimul256 batch2"), flush=True)  # fmt: skip


@pytest.mark.parametrize("outgoing", [True, False], ids=["out", "in"])
def test_trimul256_residual_in_place(dev, outgoing):
    """forward_residual_ adds the update inside K3: equal to z + forward(z) up to the
    rounding of the separately stored update."""
    m, _ = _trimul(dev, outgoing, 101)
    print(f"[trimul256] in-place residual outgoing={outgoing}", flush=True)
    z = _z(100, 102).to(dev, BF)
    mask = _mask(100, 103).to(dev)
    with torch.no_grad():
        upd = m(z, mask)
        got = m.forward_residual_(z.clone(), mask)
    want = z.float() + upd.float()
    err = (got.float() - want).abs().max().item()
    tol = 2.0**-7 * want.abs().max().item()
    assert err <= tol, f"in-place residual: max |diff| {err:.3e} > {tol:.3e}"
