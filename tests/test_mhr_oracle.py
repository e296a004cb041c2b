"""CPU: pin the oracle's multi-head routed triangle multiplication (``R.tri_mul`` with
``num_heads``, ``R.mhr_head_mix``; reference ``ops.py:179-345``, ``:476-545``).

Each check ties the restatement to something it does not retype: the plain ``tri_mul``
(itself pinned by the golden vectors), library norms that the per-head modes reduce to
(``F.group_norm`` with H groups is head_ln, ``F.rms_norm`` over d is head_rms,
``F.layer_norm`` over C is channel), scipy's softmax / expit for the gates, and invariances
(a gate constant over positions equals scaling out_proj's column block of its head; a head's
norm ignores that head's scale). A channel-to-head map transposed (c % H instead of c // d),
a gate on the wrong side of the norm or a dropped mean term fails one of them.
"""

from __future__ import annotations

import pytest
import scipy.special
import torch
import torch.nn.functional as F

from oracle import pairformer_ref as R
from tests._helpers import rel_l2

H, C, N = 4, 16, 6
# The oracle computes its norms and gates in fp32 as the reference does (LayerNorm upcasts,
# the head norms and gates take .float()), so fp64 inputs agree to fp32 rounding.
TOL = 1e-6


@pytest.fixture(autouse=True)
def _highest_precision():
    prev = torch.get_float32_matmul_precision()
    torch.set_float32_matmul_precision("highest")
    yield
    torch.set_float32_matmul_precision(prev)


def _params(c=C, h=H, seed=0, router_std=0.7):
    gen = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=gen, dtype=torch.float64) * 0.5  # noqa: E731
    return {
        "norm_left.weight": 1 + 0.1 * r(c), "norm_left.bias": 0.1 * r(c),
        "proj.weight": r(2 * c, c), "gate.weight": r(2 * c, c),
        "norm_center.weight": 1 + 0.2 * r(c), "norm_center.bias": 0.2 * r(c),
        "out_proj.weight": r(c, c), "out_gate.weight": r(c, c),
        "router.weight": router_std * 2 * r(h, c),
    }  # fmt: skip


def _inputs(seed=1, n=N, c=C):
    gen = torch.Generator().manual_seed(seed)
    z = torch.randn(1, n, n, c, generator=gen, dtype=torch.float64)
    mask = (torch.rand(1, n, n, generator=gen) > 0.2).double()
    return z, mask


@pytest.mark.parametrize("outgoing", [True, False])
def test_zero_router_channel_is_the_plain_trimul(outgoing):
    z, mask = _inputs()
    p = _params()
    p["router.weight"] = torch.zeros(H, C, dtype=torch.float64)
    plain = R.tri_mul(z, mask, p, outgoing)
    for kind in ("softmax", "sigmoid"):
        routed = R.tri_mul(z, mask, p, outgoing, num_heads=H, head_norm="channel", router=True, router_kind=kind)
        assert plain.abs().max() > 1e-2
        assert torch.equal(plain, routed), kind


def _act(seed=2, m=7):
    gen = torch.Generator().manual_seed(seed)
    # heads at very different scales, so a per-head norm is visible
    scale = torch.arange(1, H + 1, dtype=torch.float64).repeat_interleave(C // H)
    return torch.randn(m, C, generator=gen, dtype=torch.float64) * scale + 0.3


def test_head_ln_is_group_norm_with_h_groups():
    p = _params()
    act = _act()
    got = R.mhr_head_mix(act, None, p, H, "head_ln", "softmax")
    want = F.group_norm(act, H, p["norm_center.weight"], p["norm_center.bias"], eps=1e-5)
    assert rel_l2(got, want) < TOL


def test_head_rms_is_rms_norm_over_each_head():
    p = _params()
    p.pop("norm_center.bias")
    act = _act()
    got = R.mhr_head_mix(act, None, p, H, "head_rms", "softmax")
    d = C // H
    want = F.rms_norm(act.unflatten(-1, (H, d)), (d,), eps=1e-5).flatten(-2) * p["norm_center.weight"]
    assert rel_l2(got, want) < TOL
    # every head at unit RMS before the gain (up to eps = 1e-5 against mean squares >= 0.09)
    unit = R.mhr_head_mix(act, None, {"norm_center.weight": torch.ones(C, dtype=torch.float64)}, H, "head_rms", "softmax")
    rms = unit.unflatten(-1, (H, d)).pow(2).mean(-1).sqrt()
    assert torch.allclose(rms, torch.ones_like(rms), atol=1e-4)


def test_channel_mode_is_layer_norm_times_gates():
    p = _params()
    act = _act()
    r = torch.randn(act.shape[0], H, dtype=torch.float64, generator=torch.Generator().manual_seed(5))
    ln = F.layer_norm(act, (C,), p["norm_center.weight"], p["norm_center.bias"], eps=1e-5)
    for kind in ("softmax", "sigmoid"):
        got = R.mhr_head_mix(act, r, p, H, "channel", kind)
        if kind == "softmax":
            g = H * torch.from_numpy(scipy.special.softmax(r.numpy(), axis=-1))
        else:
            g = 2 * torch.from_numpy(scipy.special.expit(r.numpy()))
        assert rel_l2(got, ln * g.repeat_interleave(C // H, dim=-1)) < TOL, kind


def test_post_channel_gates_before_the_layer_norm():
    p = _params()
    act = _act()
    r = torch.randn(act.shape[0], H, dtype=torch.float64, generator=torch.Generator().manual_seed(6))
    got = R.mhr_head_mix(act, r, p, H, "post_channel", "sigmoid")
    g = 2 * torch.from_numpy(scipy.special.expit(r.numpy()))
    gated = act * g.repeat_interleave(C // H, dim=-1)
    want = F.layer_norm(gated, (C,), p["norm_center.weight"], p["norm_center.bias"], eps=1e-5)
    assert rel_l2(got, want) < TOL
    # uniform gates: post_channel is the channel LayerNorm (softmax of equal logits is 1)
    flat = R.mhr_head_mix(act, torch.zeros_like(r), p, H, "post_channel", "softmax")
    assert rel_l2(flat, F.layer_norm(act, (C,), p["norm_center.weight"], p["norm_center.bias"], eps=1e-5)) < TOL


@pytest.mark.parametrize("head_norm", ["head_rms", "head_ln"])
def test_a_head_norm_ignores_that_heads_scale(head_norm):
    p = _params()
    if head_norm == "head_rms":
        p.pop("norm_center.bias")
    act = _act()
    scaled = act.clone()
    scaled[:, C // H : 2 * C // H] *= 40.0
    a = R.mhr_head_mix(act, None, p, H, head_norm, "softmax")
    b = R.mhr_head_mix(scaled, None, p, H, head_norm, "softmax")
    assert rel_l2(a, b) < 1e-5  # eps = 1e-5 against the unscaled head's variance (about 4)
    # a channel-wide norm does see it
    pc = _params()
    assert not torch.allclose(R.mhr_head_mix(act, None, pc, H, "channel", "softmax"),
                              R.mhr_head_mix(scaled, None, pc, H, "channel", "softmax"), atol=1e-3)  # fmt: skip


@pytest.mark.parametrize("outgoing", [True, False])
@pytest.mark.parametrize("head_norm", ["channel", "head_ln"])
def test_position_constant_gates_fold_into_out_proj(outgoing, head_norm):
    """With norm_left's gain 1 and router rows alpha_h * ones, r_h = alpha_h * sum(norm_left.bias)
    at every position (a LayerNorm row sums to its bias's sum), so each head's gate is one
    constant g_h: the routed module equals the unrouted one with out_proj's column block of
    head h multiplied by g_h."""
    z, mask = _inputs(seed=3)
    p = _params(seed=4)
    p["norm_left.weight"] = torch.ones(C, dtype=torch.float64)
    alpha = torch.tensor([0.9, -0.4, 0.2, 1.3], dtype=torch.float64)
    p["router.weight"] = alpha[:, None] * torch.ones(H, C, dtype=torch.float64)
    routed = R.tri_mul(z, mask, p, outgoing, num_heads=H, head_norm=head_norm, router=True)
    r = alpha * p["norm_left.bias"].sum()
    g = H * torch.softmax(r, dim=-1)
    q = dict(p)
    q["out_proj.weight"] = p["out_proj.weight"] * g.repeat_interleave(C // H)[None, :]
    unrouted = R.tri_mul(z, mask, q, outgoing, num_heads=H, head_norm=head_norm, router=False)
    if head_norm == "channel":
        unrouted = R.tri_mul(z, mask, q, outgoing)
    assert routed.abs().max() > 1e-2
    assert rel_l2(routed, unrouted) < TOL


def test_router_changes_more_than_an_output_gate_can():
    """A per-(position, head) factor before out_proj is outside what the post-projection
    gate can express: routed / unrouted varies across positions within an output channel."""
    z, mask = _inputs(seed=7)
    p = _params(seed=8, router_std=1.0)
    routed = R.tri_mul(z, mask, p, True, num_heads=H, head_norm="head_ln", router=True)
    q = dict(p)
    q["router.weight"] = torch.zeros(H, C, dtype=torch.float64)
    flat = R.tri_mul(z, mask, q, True, num_heads=H, head_norm="head_ln", router=True)
    ratio = (routed / flat.clamp(min=1e-3)).flatten(0, 2)
    assert ratio.std(0).max() > 1e-2


@pytest.mark.parametrize("outgoing", [True, False], ids=["out", "in"])
@pytest.mark.parametrize("head_norm,router,kind", [("channel", True, "softmax"), ("head_rms", True, "sigmoid"),
                                                   ("head_ln", False, "softmax"), ("post_channel", True, "sigmoid")])
def test_tri_mul_core_mhr_composes_to_tri_mul(outgoing, head_norm, router, kind):
    """The training-path restatement (``tri_mul_core``, x = norm_left(z), block-order rows)
    with the MHR mix equals the module-level ``tri_mul`` with the same mix."""
    z, mask = _inputs(seed=9, n=7)
    p = _params(seed=10)
    if head_norm == "head_rms":
        p.pop("norm_center.bias")
    even, odd = torch.arange(0, 2 * C, 2), torch.arange(1, 2 * C, 2)
    order = torch.cat((even, odd)) if outgoing else torch.cat((odd, even))
    kw = dict(num_heads=H, head_norm=head_norm, router=router, router_kind=kind)
    want = R.tri_mul(z, mask, p, outgoing, **kw)
    xn = F.layer_norm(z, (C,), p["norm_left.weight"], p["norm_left.bias"], 1e-5)
    got = R.tri_mul_core(xn, mask, p["gate.weight"][order], p["proj.weight"][order], p["norm_center.weight"],
                         p.get("norm_center.bias"), p["out_proj.weight"], p["out_gate.weight"], 1e-5, outgoing,
                         p["router.weight"] if router else None, H, head_norm, kind)  # fmt: skip
    assert rel_l2(got, want) < 1e-5  # tri_mul's LayerNorms run in fp32
