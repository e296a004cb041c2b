"""CPU: pin the oracle (oracle/pairformer_ref.py) to the reference and to independent forms.

1. Golden vectors written by tests/golden/make_golden.py from the reference's own
   PairFormerBlock (fp32, CPU): block outputs and every branch, masked.
2. Brute force at tiny N: explicit loops for the triangle contractions, per-row
   softmax attention, and the column-attention transpose semantics.
3. Invariants: batch consistency, row chunking, fully masked rows = mean of V.
"""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import pairformer_ref as R
from tests._helpers import mod, rel_l2, sub

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
W = mod("weights")


@pytest.fixture(autouse=True)
def _highest_precision():
    prev = torch.get_float32_matmul_precision()
    torch.set_float32_matmul_precision("highest")
    yield
    torch.set_float32_matmul_precision(prev)


def test_weight_generator_matches_golden_sha():
    g = np.load(os.path.join(GOLDEN, "block_n24_masked.npz"))
    assert str(g["weights_sha256"]) == W.state_dict_sha256(W.make_block_weights(7, perturb_affine=True))
    g1 = np.load(os.path.join(GOLDEN, "block_n64_cfg1.npz"))
    assert str(g1["weights_sha256"]) == W.state_dict_sha256(W.make_block_weights(0))


def test_input_generator_matches_golden():
    g = np.load(os.path.join(GOLDEN, "block_n24_masked.npz"))
    inp = W.make_inputs(24, seed=10, pad_last=3)
    for k in ("pair", "single", "pair_mask", "seq_mask"):
        assert torch.equal(inp[k], torch.from_numpy(g["in_" + k])), k


def test_block_and_branches_match_reference_golden():
    g = np.load(os.path.join(GOLDEN, "block_n24_masked.npz"))
    sd = W.make_block_weights(7, perturb_affine=True)
    inp = {k: torch.from_numpy(g["in_" + k]) for k in ("pair", "single", "pair_mask", "seq_mask")}
    br = {}
    with torch.no_grad():
        pair, single = R.pairformer_block(inp["pair"], inp["single"], inp["pair_mask"], inp["seq_mask"], sd, branches=br)
    assert rel_l2(pair, torch.from_numpy(g["out_pair"])) < 1e-6
    assert rel_l2(single, torch.from_numpy(g["out_single"])) < 1e-6
    for k in ("tri_mul_out", "tri_mul_in", "pair_attn_row", "pair_attn_col", "pair_transition", "single_attn",
              "single_transition"):  # fmt: skip
        assert rel_l2(br[k], torch.from_numpy(g["branch_" + k])) < 1e-6, k
    s2p = br["pair_logits"].movedim(-3, -1)
    assert rel_l2(s2p, torch.from_numpy(g["branch_single_to_pair"])) < 1e-6


def test_config1_block_matches_reference_summary():
    g = np.load(os.path.join(GOLDEN, "block_n64_cfg1.npz"))
    sd = W.make_block_weights(0)
    inp = W.make_inputs(64, seed=0)
    with torch.no_grad():
        pair, single = R.pairformer_block(inp["pair"], inp["single"], inp["pair_mask"], inp["seq_mask"], sd)
    assert rel_l2(single, torch.from_numpy(g["out_single"])) < 1e-6
    got = pair.reshape(-1)[torch.from_numpy(g["pair_sample_idx"])]
    assert rel_l2(got, torch.from_numpy(g["pair_sample_val"])) < 1e-6
    p64 = pair.double()
    assert abs(p64.sum().item() - float(g["pair_sum"])) <= 1e-6 * abs(float(g["pair_sumsq"])) ** 0.5 * 64
    assert abs((p64 * p64).sum().item() / float(g["pair_sumsq"]) - 1.0) < 1e-6


# ------------------------------------------------------------------ brute force


def _tiny_trimul_params(c=8, seed=0):
    gen = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=gen) * 0.5  # noqa: E731
    return {
        "norm_left.weight": 1 + 0.1 * r(c), "norm_left.bias": 0.1 * r(c),
        "proj.weight": r(2 * c, c), "gate.weight": r(2 * c, c),
        "norm_center.weight": 1 + 0.1 * r(c), "norm_center.bias": 0.1 * r(c),
        "out_proj.weight": r(c, c), "out_gate.weight": r(c, c),
    }  # fmt: skip


@pytest.mark.parametrize("outgoing", [True, False])
def test_trimul_against_explicit_loops(outgoing):
    N, c = 5, 8
    p = _tiny_trimul_params(c)
    gen = torch.Generator().manual_seed(3)
    z = torch.randn(1, N, N, c, generator=gen, dtype=torch.float64)
    mask = (torch.rand(1, N, N, generator=gen) > 0.3).double()
    p64 = {k: v.double() for k, v in p.items()}
    out = R.tri_mul(z, mask, p64, outgoing)
    # independent restatement with explicit index loops
    zl = F.layer_norm(z, (c,), p64["norm_left.weight"], p64["norm_left.bias"])
    pr = zl @ p64["proj.weight"].T
    gt = torch.sigmoid(zl @ p64["gate.weight"].T)
    ab = pr * gt
    a = torch.zeros(N, N, c, dtype=torch.float64)
    b = torch.zeros(N, N, c, dtype=torch.float64)
    for i in range(N):
        for j in range(N):
            for ch in range(c):
                a[i, j, ch] = ab[0, i, j, 2 * ch] * mask[0, i, j]
                b[i, j, ch] = ab[0, i, j, 2 * ch + 1] * mask[0, i, j]
    X = torch.zeros(N, N, c, dtype=torch.float64)
    for i in range(N):
        for j in range(N):
            for k in range(N):
                X[i, j] += a[i, k] * b[j, k] if outgoing else a[k, j] * b[k, i]
    Xn = F.layer_norm(X, (c,), p64["norm_center.weight"], p64["norm_center.bias"])
    ref = (Xn @ p64["out_proj.weight"].T) * torch.sigmoid(zl[0] @ p64["out_gate.weight"].T)
    assert torch.allclose(out[0], ref, rtol=1e-5, atol=1e-6)  # LN runs in fp32 by design


def _tiny_attn_params(c=8, H=2, seed=1):
    gen = torch.Generator().manual_seed(seed)
    D = max(c // H, 16)
    r = lambda *s: torch.randn(*s, generator=gen) * 0.3  # noqa: E731
    return {
        "norm.weight": 1 + 0.1 * r(c), "norm.bias": 0.1 * r(c), "pair_bias.weight": r(H, c),
        "to_q.weight": r(H * D, c), "to_k.weight": r(H * D, c), "to_v.weight": r(H * D, c),
        "to_g.weight": r(H * D, c), "out_proj.weight": r(c, H * D),
    }, H, D  # fmt: skip


@pytest.mark.parametrize("c,heads", [(8, 2), (64, 4)])  # head dim 16: floored (8 / 2), exact (64 / 4)
@pytest.mark.parametrize("transpose", [False, True])
def test_grid_attention_against_loops(transpose, c, heads):
    N = 5
    p, H, D = _tiny_attn_params(c, H=heads)
    p = {k: v.double() for k, v in p.items()}
    gen = torch.Generator().manual_seed(4)
    z = torch.randn(1, N, N, c, generator=gen, dtype=torch.float64)
    mask = torch.ones(1, N, N, dtype=torch.float64)
    mask[0, 1, 3] = 0
    mask[0, 2, :] = 0  # one fully masked row (and column entries)
    # the head count is given, or (64 channels) taken from the pair-bias rows
    out = R.grid_attention(z, mask, p, transpose=transpose, num_heads=H if c == 8 else None)
    zn = F.layer_norm(z[0], (c,), p["norm.weight"], p["norm.bias"])
    pb = torch.einsum("ijc,hc->hij", zn, p["pair_bias.weight"])  # bias from un-transposed LN(z)
    ref = torch.zeros(N, N, c, dtype=torch.float64)
    for line in range(N):
        for qi in range(N):
            # row mode: positions (line, .); column mode: positions (., line)
            qpos = (line, qi) if not transpose else (qi, line)
            o = torch.zeros(H * D, dtype=torch.float64)
            for h in range(H):
                sl = slice(h * D, (h + 1) * D)
                q = zn[qpos] @ p["to_q.weight"][sl].T
                logits = torch.zeros(N, dtype=torch.float64)
                vs = torch.zeros(N, D, dtype=torch.float64)
                for kj in range(N):
                    kpos = (line, kj) if not transpose else (kj, line)
                    k = zn[kpos] @ p["to_k.weight"][sl].T
                    vs[kj] = zn[kpos] @ p["to_v.weight"][sl].T
                    logits[kj] = q @ k * D**-0.5 + pb[h, qi, kj] + 1e9 * (mask[0][kpos] - 1.0)
                # softmax on fp32 logits, as the reference (attention.py:160): this rounding
                # point is what makes a fully masked row uniform
                w = torch.softmax(logits.float(), 0).double()
                o[sl] = w @ vs
            g = torch.sigmoid(zn[qpos] @ p["to_g.weight"].T)
            ref[qpos] = (o * g) @ p["out_proj.weight"].T
    # LN runs in fp32 by design (primitives.py:90-115): fp32 rounding relative to the output scale
    assert (out[0] - ref).abs().max() <= 1e-6 * ref.abs().max()


def test_fully_masked_row_is_mean_of_v():
    """Eager semantics (attention.py:157-160): an all-masked row attends uniformly."""
    N, c = 6, 8
    p, H, D = _tiny_attn_params(c, seed=2)
    z = torch.randn(1, N, N, c, generator=torch.Generator().manual_seed(5))
    mask = torch.ones(1, N, N)
    mask[0, 3, :] = 0
    out = R.grid_attention(z, mask, p, transpose=False, num_heads=H)
    zn = F.layer_norm(z[0], (c,), p["norm.weight"], p["norm.bias"])
    v = zn[3] @ p["to_v.weight"].T  # [N, H*D]
    o = v.mean(0, keepdim=True).expand(N, -1)
    g = torch.sigmoid(zn[3] @ p["to_g.weight"].T)
    ref = (o * g) @ p["out_proj.weight"].T
    assert torch.allclose(out[0, 3], ref, rtol=1e-5, atol=1e-6)


def test_single_attention_against_loops():
    N, c, H = 5, 16, 4
    gen = torch.Generator().manual_seed(6)
    r = lambda *s: torch.randn(*s, generator=gen, dtype=torch.float64) * 0.3  # noqa: E731
    p = {"norm.weight": 1 + r(c), "norm.bias": r(c), "to_q.weight": r(c, c), "to_q.bias": r(c),
         "to_k.weight": r(c, c), "to_v.weight": r(c, c), "to_g.weight": r(c, c), "out_proj.weight": r(c, c)}  # fmt: skip
    s = r(1, N, c)
    seq = torch.tensor([[1.0, 1, 0, 1, 1]], dtype=torch.float64)
    logits_pair = r(1, H, N, N)
    out = R.single_attention(s, seq, logits_pair, p, num_heads=H)
    D = c // H
    xn = F.layer_norm(s[0], (c,), p["norm.weight"], p["norm.bias"])
    ref = torch.zeros(N, c, dtype=torch.float64)
    for i in range(N):
        o = torch.zeros(c, dtype=torch.float64)
        for h in range(H):
            sl = slice(h * D, (h + 1) * D)
            q = (xn[i] @ p["to_q.weight"][sl].T + p["to_q.bias"][sl]) * D**-0.5
            lg = torch.stack([q @ (xn[j] @ p["to_k.weight"][sl].T) + logits_pair[0, h, i, j] + 1e9 * (seq[0, j] - 1)
                              for j in range(N)])  # fmt: skip
            w = torch.softmax(lg, 0)
            o[sl] = sum(w[j] * (xn[j] @ p["to_v.weight"][sl].T) for j in range(N))
        g = torch.sigmoid(xn[i] @ p["to_g.weight"].T)
        ref[i] = (o * g) @ p["out_proj.weight"].T
    assert torch.allclose(out[0], ref, rtol=1e-5, atol=1e-6)  # LN runs in fp32 by design


def test_transition_swiglu_contiguous_halves():
    c = 8
    gen = torch.Generator().manual_seed(7)
    p = {"norm.weight": torch.ones(c), "norm.bias": torch.zeros(c),
         "linear1.weight": torch.randn(8 * c, c, generator=gen), "linear2.weight": torch.randn(c, 4 * c, generator=gen)}  # fmt: skip
    x = torch.randn(3, c, generator=gen, dtype=torch.float64)
    p = {k: v.double() for k, v in p.items()}
    out = R.transition(x, p)
    xn = F.layer_norm(x, (c,))
    h = xn @ p["linear1.weight"].T
    u = torch.stack([torch.stack([h[r, j] / (1 + torch.exp(-h[r, j])) * h[r, 4 * c + j] for j in range(4 * c)])
                     for r in range(3)])  # fmt: skip
    assert torch.allclose(out, u @ p["linear2.weight"].T, rtol=1e-5, atol=1e-6)  # LN runs in fp32 by design


# ------------------------------------------------------------------ invariants


def test_batch_consistency_and_row_chunking():
    sd = W.make_block_weights(3, perturb_affine=True)
    inp = W.make_inputs(12, seed=2, batch=2, pad_random=2)
    with torch.no_grad():
        pb, sb = R.pairformer_block(inp["pair"], inp["single"], inp["pair_mask"], inp["seq_mask"], sd)
        p1, s1 = R.pairformer_block(inp["pair"][1:], inp["single"][1:], inp["pair_mask"][1:], inp["seq_mask"][1:], sd)
        pc, sc = R.pairformer_block(inp["pair"], inp["single"], inp["pair_mask"], inp["seq_mask"], sd, row_chunk=5)
    assert rel_l2(pb[1:], p1) < 1e-6 and rel_l2(sb[1:], s1) < 1e-6
    assert rel_l2(pc, pb) < 1e-6 and rel_l2(sc, sb) < 1e-6


@pytest.mark.parametrize("transpose", [False, True])
def test_grid_attention_line_subset_equals_whole(transpose):
    """The sampled-line evaluation used at N=2048 picks the same lines out of the whole."""
    sd = W.make_block_weights(6, perturb_affine=True)
    p = sub(sd, "pair_attn_col." if transpose else "pair_attn_row.")
    inp = W.make_inputs(20, seed=4, pad_random=3)
    lines = torch.tensor([0, 7, 19])
    with torch.no_grad():
        whole = R.grid_attention(inp["pair"], inp["pair_mask"], p, transpose=transpose)
        part = R.grid_attention(inp["pair"], inp["pair_mask"], p, transpose=transpose, lines=lines)
    picked = whole[:, :, lines] if transpose else whole[:, lines]
    assert rel_l2(part.transpose(1, 2) if transpose else part, picked) < 1e-6


def test_mask_changes_output():
    sd = W.make_block_weights(4)
    a = W.make_inputs(10, seed=1)
    b = W.make_inputs(10, seed=1, pad_last=2)
    with torch.no_grad():
        pa, _ = R.pairformer_block(a["pair"], a["single"], a["pair_mask"], a["seq_mask"], sd)
        pb, _ = R.pairformer_block(b["pair"], b["single"], b["pair_mask"], b["seq_mask"], sd)
    assert rel_l2(pa, pb) > 1e-3


def test_trunk_is_block_composition():
    blocks = W.make_trunk_weights(9, 2)
    inp = W.make_inputs(8, seed=3)
    with torch.no_grad():
        p, s = R.pairformer_trunk(inp["pair"], inp["single"], inp["pair_mask"], inp["seq_mask"], blocks)
        p1, s1 = R.pairformer_block(inp["pair"], inp["single"], inp["pair_mask"], inp["seq_mask"], blocks[0])
        p2, s2 = R.pairformer_block(p1, s1, inp["pair_mask"], inp["seq_mask"], blocks[1])
    assert torch.equal(p, p2) and torch.equal(s, s2)


def test_template_block_is_the_pair_half_of_the_block():
    """TemplatePairFormerBlock (template_embedding.py:220-240) runs the PairFormer block's
    five pair branches in the same order (evoformer.py:298-321): with the same weights its
    output equals the pinned block's pair output; with a factor-2 transition it differs."""
    sd = W.make_block_weights(13, perturb_affine=True)
    inp = W.make_inputs(12, seed=4, pad_last=2)
    pair_keys = ("tri_mul_out.", "tri_mul_in.", "pair_attn_row.", "pair_attn_col.", "pair_transition.")
    sub = {k: v for k, v in sd.items() if k.startswith(pair_keys)}
    with torch.no_grad():
        want, _ = R.pairformer_block(inp["pair"], inp["single"], inp["pair_mask"], inp["seq_mask"], sd)
        got = R.template_pairformer_block(inp["pair"], inp["pair_mask"], sub)
        sd2 = W.make_block_weights(13, perturb_affine=True, factor=2)
        got2 = R.template_pairformer_block(inp["pair"], inp["pair_mask"], {k: sd2[k] for k in sub})
    assert torch.equal(got, want)
    assert sd2["pair_transition.linear1.weight"].shape == (512, 128)
    assert rel_l2(got2, want) > 1e-3


# Every residual branch ends in a bias-free output projection, so each branch output is
# linear in that weight: the block with a residual scale s on a branch equals the unscaled
# block with that projection's weight multiplied by s.
_OUT_PROJ = {
    "tri_mul_out.out_proj.weight": "ros",
    "tri_mul_in.out_proj.weight": "ros",
    "pair_attn_row.out_proj.weight": "ros",
    "pair_attn_col.out_proj.weight": "ros",
    "pair_transition.linear2.weight": "pair",
    "single_attn.out_proj.weight": "ros",
    "single_transition.linear2.weight": "single",
}


def _f64(d: dict) -> dict:
    return {k: (v.double() if v.is_floating_point() else v) for k, v in d.items()}


def test_residual_scales_equal_scaled_output_projections():
    sd = _f64(W.make_block_weights(21, perturb_affine=True))
    x = _f64(W.make_inputs(10, seed=8, pad_last=2))
    sc = dict(residual_out_scale=0.6, pair_transition_residual_gain=0.5, single_transition_residual_gain=1.7)
    factor = {"ros": 0.6, "pair": 0.6 * 0.5, "single": 0.6 * 1.7}
    scaled = {k: (v * factor[_OUT_PROJ[k]] if k in _OUT_PROJ else v) for k, v in sd.items()}
    with torch.no_grad():
        p, s = R.pairformer_block(x["pair"], x["single"], x["pair_mask"], x["seq_mask"], sd, scales=sc)
        p2, s2 = R.pairformer_block(x["pair"], x["single"], x["pair_mask"], x["seq_mask"], scaled)
        p1, s1 = R.pairformer_block(x["pair"], x["single"], x["pair_mask"], x["seq_mask"], sd)
    assert rel_l2(p, p2) < 1e-12 and rel_l2(s, s2) < 1e-12
    assert rel_l2(p, p1) > 1e-3 and rel_l2(s, s1) > 1e-3  # the scales do act


def test_zero_scales():
    """s_ros = 0 leaves both tracks unchanged; a zero transition gain equals a zeroed linear2
    of that transition only."""
    sd = W.make_block_weights(22, perturb_affine=True)
    x = W.make_inputs(9, seed=2, pad_last=1)
    args = (x["pair"], x["single"], x["pair_mask"], x["seq_mask"])
    with torch.no_grad():
        p0, s0 = R.pairformer_block(*args, sd, scales=dict(residual_out_scale=0.0))
        pz, sz = R.pairformer_block(*args, sd, scales=dict(pair_transition_residual_gain=0.0))
        pw, sw = R.pairformer_block(*args, {**sd, "pair_transition.linear2.weight": torch.zeros(128, 512)})
        qz, tz = R.pairformer_block(*args, sd, scales=dict(single_transition_residual_gain=0.0))
        qw, tw = R.pairformer_block(*args, {**sd, "single_transition.linear2.weight": torch.zeros(384, 1536)})
    assert torch.equal(p0, x["pair"]) and torch.equal(s0, x["single"])
    assert torch.equal(pz, pw) and torch.equal(sz, sw)
    assert torch.equal(qz, qw) and torch.equal(tz, tw)


def test_template_residual_scale_equals_scaled_output_projections():
    sd = _f64(W.make_block_weights(23, perturb_affine=True, factor=2))
    p = {k: v for k, v in sd.items() if k.startswith(("tri_mul_", "pair_attn_", "pair_transition."))}
    x = _f64(W.make_inputs(8, seed=4, pad_last=1))
    scaled = {k: (v * 0.3 if k in _OUT_PROJ else v) for k, v in p.items()}
    with torch.no_grad():
        got = R.template_pairformer_block(x["pair"], x["pair_mask"], p, residual_out_scale=0.3)
        want = R.template_pairformer_block(x["pair"], x["pair_mask"], scaled)
    assert rel_l2(got, want) < 1e-12


def _recycle_weights(seed: int, c: int = 128, cs: int = 384, single: bool = True) -> dict:
    g = torch.Generator().manual_seed(seed)
    p = {
        "prev_embedding_layer_norm.weight": 1.0 + 0.2 * torch.randn(c, generator=g),
        "prev_embedding_layer_norm.bias": 0.5 * torch.randn(c, generator=g),
        "prev_embedding.weight": torch.randn(c, c, generator=g) / c**0.5,
    }
    if single:
        p.update({
            "prev_single_embedding_layer_norm.weight": 1.0 + 0.2 * torch.randn(cs, generator=g),
            "prev_single_embedding_layer_norm.bias": 0.5 * torch.randn(cs, generator=g),
            "prev_single_embedding.weight": torch.randn(cs, cs, generator=g) / cs**0.5,
        })  # fmt: skip
    return p


def test_recycle_embed_zero_prev_is_bias_projection():
    """LayerNorm of a zero row is its bias b, so zero previous outputs add b W^T (W not
    symmetric: a transposed operand would fail)."""
    p = _f64(_recycle_weights(3))
    g = torch.Generator().manual_seed(4)
    zp, zs = torch.randn(1, 6, 6, 128, generator=g).double(), torch.randn(1, 6, 384, generator=g).double()
    pair, single = R.recycle_embed(zp, zs, torch.zeros_like(zp), torch.zeros_like(zs), p)
    wp = p["prev_embedding_layer_norm.bias"] @ p["prev_embedding.weight"].T
    ws = p["prev_single_embedding_layer_norm.bias"] @ p["prev_single_embedding.weight"].T
    assert rel_l2(pair, zp + wp) < 1e-13 and rel_l2(single, zs + ws) < 1e-13
    assert rel_l2(pair, zp + p["prev_embedding_layer_norm.bias"] @ p["prev_embedding.weight"]) > 1e-2


def test_recycle_embed_invariants():
    """LayerNorm removes a per-row shift of the previous outputs; the embedding is linear in
    the projection weight; without the single-track keys the single track passes through."""
    p = _f64(_recycle_weights(5))
    g = torch.Generator().manual_seed(6)
    zp, zs = torch.randn(1, 5, 5, 128, generator=g).double(), torch.randn(1, 5, 384, generator=g).double()
    pp, ps = torch.randn(1, 5, 5, 128, generator=g).double(), torch.randn(1, 5, 384, generator=g).double()
    a, b = R.recycle_embed(zp, zs, pp, ps, p)
    a2, b2 = R.recycle_embed(zp, zs, pp + 3.0 * torch.randn(1, 5, 5, 1, generator=g).double(),
                             ps - 2.0 * torch.randn(1, 5, 1, generator=g).double(), p)  # fmt: skip
    # the oracle's LayerNorm computes in fp32 (primitives.py:90-115), so the shift cancels to fp32 precision
    assert rel_l2(a, a2) < 1e-6 and rel_l2(b, b2) < 1e-6
    p2 = dict(p, **{"prev_embedding.weight": 2.0 * p["prev_embedding.weight"]})
    c, _ = R.recycle_embed(zp, zs, pp, ps, p2)
    assert rel_l2(c - zp, 2.0 * (a - zp)) < 1e-13
    pair_only = {k: v for k, v in p.items() if not k.startswith("prev_single")}
    _, same = R.recycle_embed(zp, zs, pp, ps, pair_only)
    assert same is zs


def test_recycled_trunk_is_recycle_then_trunk():
    blocks = W.make_trunk_weights(31, 2)
    rp = _recycle_weights(7)
    x = W.make_inputs(8, seed=5, pad_last=1)
    args = (x["pair_mask"], x["seq_mask"])
    with torch.no_grad():
        got = R.recycled_trunk(x["pair"], x["single"], *args, rp, blocks, num_recycles=1)
        zp, zs = torch.zeros_like(x["pair"]), torch.zeros_like(x["single"])
        p, s = R.pairformer_trunk(*R.recycle_embed(x["pair"], x["single"], zp, zs, rp), *args, blocks)
        p, s = R.pairformer_trunk(*R.recycle_embed(x["pair"], x["single"], p, s, rp), *args, blocks)
    assert torch.equal(got[0], p) and torch.equal(got[1], s)


def _tiny_evo_params(cm=8, cz=6, ch=3, H=2, seed=5):
    gen = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=gen, dtype=torch.float64) * 0.4  # noqa: E731
    return {
        "outer_product.norm.weight": 1 + 0.1 * r(cm), "outer_product.norm.bias": 0.1 * r(cm),
        "outer_product.proj_a.weight": r(ch, cm), "outer_product.proj_b.weight": r(ch, cm),
        "outer_product.out_w": r(ch, ch, cz), "outer_product.out_b": r(cz),
        "row_attn.norm.weight": 1 + 0.1 * r(cm), "row_attn.norm.bias": 0.1 * r(cm),
        "row_attn.pair_norm.weight": 1 + 0.1 * r(cz), "row_attn.pair_norm.bias": 0.1 * r(cz),
        "row_attn.pair_logits.weight": r(H, cz), "row_attn.to_v.weight": r(cm, cm),
        "row_attn.to_g.weight": r(cm, cm), "row_attn.out_proj.weight": r(cm, cm),
    }  # fmt: skip


def test_outer_product_mean_against_loops():
    """ops.py:683-785: mean over the sequences that have both residues, of the outer product
    of the two projections, through out_w, plus out_b."""
    S, N, cm, cz, ch = 4, 5, 8, 6, 3
    p = _sub_keys(_tiny_evo_params(cm, cz, ch), "outer_product.")
    gen = torch.Generator().manual_seed(6)
    msa = torch.randn(1, S, N, cm, generator=gen, dtype=torch.float64)
    mask = (torch.rand(1, S, N, generator=gen) > 0.3).double()
    got = R.outer_product_mean(msa, mask, p)
    x = F.layer_norm(msa[0], (cm,), p["norm.weight"], p["norm.bias"])
    ref = torch.zeros(N, N, cz, dtype=torch.float64)
    for i in range(N):
        for j in range(N):
            acc = torch.zeros(ch, ch, dtype=torch.float64)
            cnt = 0.0
            for s in range(S):
                a = (x[s, i] @ p["proj_a.weight"].T) * mask[0, s, i]
                b = (x[s, j] @ p["proj_b.weight"].T) * mask[0, s, j]
                acc += torch.outer(a, b)
                cnt += float(mask[0, s, i] * mask[0, s, j])
            for c in range(cz):
                ref[i, j, c] = ((acc * p["out_w"][:, :, c]).sum() + p["out_b"][c]) / (1e-3 + cnt)
    assert (got[0] - ref).abs().max() <= 1e-6 * ref.abs().max()


def _sub_keys(p, prefix):
    return {k[len(prefix) :]: v for k, v in p.items() if k.startswith(prefix)}


def test_msa_attention_against_loops():
    """attention.py:272-341: every MSA row averages its values with the same pair-derived
    weights (softmax over keys of LN(pair) W_h, keys masked when no sequence has them)."""
    S, N, cm, cz, H = 3, 5, 8, 6, 2
    D = cm // H
    p = _sub_keys(_tiny_evo_params(cm, cz, 3, H), "row_attn.")
    gen = torch.Generator().manual_seed(7)
    msa = torch.randn(1, S, N, cm, generator=gen, dtype=torch.float64)
    pair = torch.randn(1, N, N, cz, generator=gen, dtype=torch.float64)
    mask = torch.ones(1, S, N, dtype=torch.float64)
    mask[0, :, 2] = 0  # key 2 absent from every sequence: masked
    mask[0, 1, 4] = 0  # key 4 present in some: kept
    got = R.msa_attention(msa, mask, pair, p, H)
    xp = F.layer_norm(pair[0], (cz,), p["pair_norm.weight"], p["pair_norm.bias"])
    xm = F.layer_norm(msa[0], (cm,), p["norm.weight"], p["norm.bias"])
    ref = torch.zeros(S, N, cm, dtype=torch.float64)
    for s in range(S):
        for q in range(N):
            o = torch.zeros(cm, dtype=torch.float64)
            for h in range(H):
                lg = torch.stack([xp[q, k] @ p["pair_logits.weight"][h] + (0.0 if k != 2 else -1e9) for k in range(N)])
                w = torch.softmax(lg.float(), 0).double()
                sl = slice(h * D, (h + 1) * D)
                o[sl] = sum(w[k] * (xm[s, k] @ p["to_v.weight"][sl].T) for k in range(N))
            g = torch.sigmoid(xm[s, q] @ p["to_g.weight"].T)
            ref[s, q] = (o * g) @ p["out_proj.weight"].T
    assert (got[0] - ref).abs().max() <= 1e-6 * ref.abs().max()


def test_evoformer_block_composition():
    """evoformer.py:148-175: the pair output is the template block's pair half (factor-4
    transition) applied to pair + OPM(msa); the MSA output is msa + attention(msa, that pair)
    + transition of the sum; a residual scale s scales every branch."""
    sd = W.make_block_weights(51, perturb_affine=True)
    pair_keys = ("tri_mul_out.", "tri_mul_in.", "pair_attn_row.", "pair_attn_col.", "pair_transition.")
    p = {k: v for k, v in sd.items() if k.startswith(pair_keys)}
    gen = torch.Generator().manual_seed(8)
    cm = 64
    r = lambda *s: torch.randn(*s, generator=gen) * 0.1  # noqa: E731
    p.update({
        "outer_product.norm.weight": 1 + r(cm), "outer_product.norm.bias": r(cm),
        "outer_product.proj_a.weight": r(32, cm), "outer_product.proj_b.weight": r(32, cm),
        "outer_product.out_w": r(32, 32, 128), "outer_product.out_b": r(128),
        "row_attn.norm.weight": 1 + r(cm), "row_attn.norm.bias": r(cm),
        "row_attn.pair_norm.weight": 1 + r(128), "row_attn.pair_norm.bias": r(128),
        "row_attn.pair_logits.weight": r(8, 128), "row_attn.to_v.weight": r(cm, cm),
        "row_attn.to_g.weight": r(cm, cm), "row_attn.out_proj.weight": r(cm, cm),
        "msa_transition.norm.weight": 1 + r(cm), "msa_transition.norm.bias": r(cm),
        "msa_transition.linear1.weight": r(8 * cm, cm), "msa_transition.linear2.weight": r(cm, 4 * cm),
    })  # fmt: skip
    x = W.make_inputs(7, seed=9, pad_last=1)
    msa = torch.randn(1, 3, 7, cm, generator=gen)
    mmask = (torch.rand(1, 3, 7, generator=gen) > 0.2).float()
    with torch.no_grad():
        m1, z1 = R.evoformer_block(msa, x["pair"], mmask, x["pair_mask"], p)
        z0 = x["pair"] + R.outer_product_mean(msa, mmask, _sub_keys(p, "outer_product."))
        zw = R.template_pairformer_block(z0, x["pair_mask"], {k: v for k, v in p.items() if k.startswith(pair_keys)})
        ma = msa + R.msa_attention(msa, mmask, z0, _sub_keys(p, "row_attn."))
        mw = ma + R.transition(ma, _sub_keys(p, "msa_transition."))
        m2, z2 = R.evoformer_block(msa, x["pair"], mmask, x["pair_mask"], p, residual_out_scale=0.0)
    assert torch.equal(z1, zw) and torch.equal(m1, mw)
    assert torch.equal(z2, x["pair"]) and torch.equal(m2, msa)


def _evo_case(B=1, S=3, H=2, N=6, D=4, seed=0, dead_line=True):
    g = torch.Generator().manual_seed(seed)
    Q, K, V = (torch.randn(B, S, H, N, D, generator=g, dtype=torch.float64) for _ in range(3))
    pb = torch.randn(B, 1, H, N, N, generator=g, dtype=torch.float64)
    keep = torch.rand(B, S, 1, 1, N, generator=g) > 0.3
    keep[..., 0] = True
    if dead_line:
        keep[:, -1] = False
    rm = torch.where(keep, 0.0, -1e9).double()
    dO = torch.randn(B, S, H, N, D, generator=g, dtype=torch.float64)
    return Q, K, V, rm, pb, dO


def test_evo_attention_against_loops():
    """evo_attention.py:179-333: per (line, head, query) softmax over keys of
    q.k / sqrt(D) + bias + mask, weights times V; an all-masked line gives 0 (zero rule) or
    the mean of V (stock rule)."""
    import math

    Q, K, V, rm, pb, _ = _evo_case(seed=1)
    B, S, H, N, D = Q.shape
    for zero in (True, False):
        got = R.evo_attention(Q, K, V, rm, pb, zero_rows=zero)
        for s in range(S):
            for h in range(H):
                for i in range(N):
                    logit = [float(Q[0, s, h, i] @ K[0, s, h, j]) / math.sqrt(D) + float(pb[0, 0, h, i, j])
                             + float(rm[0, s, 0, 0, j]) for j in range(N)]  # fmt: skip
                    if max(logit) < -1e8:
                        want = torch.zeros(D, dtype=torch.float64) if zero else V[0, s, h].mean(0)
                    else:
                        m = max(logit)
                        e = [math.exp(x - m) for x in logit]
                        want = sum(e[j] / sum(e) * V[0, s, h, j] for j in range(N))
                    assert torch.allclose(got[0, s, h, i], want, rtol=1e-12, atol=1e-12), (zero, s, h, i)


def test_evo_attention_backward_equals_autograd():
    """The centred backward (evo_attention.py:335-1195) is the gradient of the zero-rule
    forward: equal to autograd in fp64, including the dead line (all zeros)."""
    Q, K, V, rm, pb, dO = _evo_case(B=2, S=3, H=2, N=9, D=4, seed=2)
    leaves = [t.clone().requires_grad_(True) for t in (Q, K, V, pb)]
    out = R.evo_attention(leaves[0], leaves[1], leaves[2], rm, leaves[3], zero_rows=True)
    want = torch.autograd.grad(out, leaves, grad_outputs=dO)
    got = R.evo_attention_backward(Q, K, V, rm, pb, dO)
    for a, b, name in zip(got, want, ("dQ", "dK", "dV", "d_pair_bias")):
        assert a.shape == b.shape, name
        assert torch.allclose(a, b, rtol=1e-10, atol=1e-12), name
    assert torch.count_nonzero(got[0][:, -1]) == 0 and torch.count_nonzero(got[2][:, -1]) == 0


def test_evo_attention_gradcheck():
    """Finite differences pin the forward's gradient (and so the restated backward)."""
    Q, K, V, rm, pb, _ = _evo_case(B=1, S=2, H=1, N=5, D=3, seed=3, dead_line=False)
    leaves = [t.clone().requires_grad_(True) for t in (Q, K, V, pb)]
    assert torch.autograd.gradcheck(lambda q, k, v, b: R.evo_attention(q, k, v, rm, b), leaves, eps=1e-6,
                                    atol=1e-7)  # fmt: skip


def test_evo_attention_centring_identity():
    """C = sum_j P_j (dP_j - dP_imax) equals D - dP_imax with D = rowsum(P dP) = rowsum(dO O):
    the centred and uncentred dS agree where both are exact (fp64, moderate margins)."""
    Q, K, V, rm, pb, dO = _evo_case(B=1, S=2, H=2, N=8, D=4, seed=4, dead_line=False)
    t = torch.matmul(Q, K.transpose(-1, -2)) * 0.5 + pb + rm
    P = torch.softmax(t, dim=-1)
    dP = torch.matmul(dO, V.transpose(-1, -2))
    out = R.evo_attention(Q, K, V, rm, pb)
    Dv = (dO * out).sum(-1, keepdim=True)
    dS_plain = P * (dP - Dv)
    got = R.evo_attention_backward(Q, K, V, rm, pb, dO)
    assert torch.allclose(got[3], dS_plain.sum(1, keepdim=True), rtol=1e-10, atol=1e-13)


def _block_order(C: int, outgoing: bool) -> torch.Tensor:
    even, odd = torch.arange(0, 2 * C, 2), torch.arange(1, 2 * C, 2)
    return torch.cat((even, odd)) if outgoing else torch.cat((odd, even))


@pytest.mark.parametrize("outgoing", [True, False], ids=["out", "in"])
def test_tri_mul_core_composes_to_tri_mul(outgoing):
    """fused_trimul.py:285-296 after ops.py:380-386: norm_left in front and the block-order
    rows (ops.py:285-288) give the stock triangle multiply (pinned by the golden vectors)."""
    prefix = "tri_mul_out." if outgoing else "tri_mul_in."
    p = {k: v.double() for k, v in sub(W.make_block_weights(21, perturb_affine=True), prefix).items()}
    x = W.make_inputs(11, seed=22, pad_last=2)
    z, mask = x["pair"].double(), x["pair_mask"].double()
    want = R.tri_mul(z, mask, p, outgoing)
    order = _block_order(128, outgoing)
    xn = F.layer_norm(z, (128,), p["norm_left.weight"], p["norm_left.bias"], 1e-5)
    got = R.tri_mul_core(xn, mask, p["gate.weight"][order], p["proj.weight"][order], p["norm_center.weight"],
                         p["norm_center.bias"], p["out_proj.weight"], p["out_gate.weight"], 1e-5, outgoing)  # fmt: skip
    # tri_mul's LayerNorms run in fp32 (primitives.py:110-115): agreement to fp32 rounding
    assert (got - want).abs().max() <= 1e-5 * want.abs().max()
    swapped = R.tri_mul_core(xn, mask, p["gate.weight"][order], p["proj.weight"][order], p["norm_center.weight"],
                             p["norm_center.bias"], p["out_proj.weight"], p["out_gate.weight"], 1e-5, not outgoing)
    assert (swapped - want).abs().max() > 1e-2 * want.abs().max()  # the direction matters


@pytest.mark.parametrize("outgoing", [True, False], ids=["out", "in"])
def test_tri_mul_core_gradcheck(outgoing):
    g = torch.Generator().manual_seed(23)
    B, N, C = 1, 4, 4
    r = lambda *s: torch.randn(*s, generator=g, dtype=torch.float64)  # noqa: E731
    mask = (torch.rand(B, N, N, generator=g) > 0.2).double()
    leaves = [r(B, N, N, C), r(2 * C, C), r(2 * C, C), 1 + 0.1 * r(C), 0.1 * r(C), r(C, C), r(C, C)]
    leaves = [t.requires_grad_(True) for t in leaves]

    def f(x, wg, wp, lw, lb, wo, wog):
        return R.tri_mul_core(x, mask, wg, wp, lw, lb, wo, wog, 1e-5, outgoing)

    assert torch.autograd.gradcheck(f, leaves, eps=1e-6, atol=1e-6)


# ---------------------------------------------------------------- training-mode dropout
# Known-answer vectors of Philox4x32-10 published with the Random123 library (kat_vectors:
# counter words, key words, output words).
PHILOX_KAT = [
    ((0, 0, 0, 0), (0, 0), (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
    ((0xFFFFFFFF,) * 4, (0xFFFFFFFF, 0xFFFFFFFF), (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
    (
        (0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344),
        (0xA4093822, 0x299F31D0),
        (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1),
    ),
]


def test_philox_known_answer_vectors():
    for ctr, key, want in PHILOX_KAT:
        got = R.philox4x32_10(np.array([ctr], dtype=np.uint32), key)[0]
        assert tuple(int(x) for x in got) == want


def test_dropout_mask_values_rate_and_index_order():
    """Entries are 0 or 1/(1-p) (fp32), keep with probability 1 - p, and entry i is word i % 4 of
    the Philox call on counter i // 4 (two calls of the generator, by hand)."""
    p, seed = 0.25, (7 << 40) + 12345
    m = R.dropout_mask(200_003, p, seed)
    scale = np.float32(1.0) / (np.float32(1.0) - np.float32(p))
    vals = set(np.unique(m.numpy()).tolist())
    assert vals == {0.0, float(scale)}
    keep = (m > 0).double().mean().item()
    assert abs(keep - 0.75) < 0.005  # 200k Bernoulli(0.75): sd 0.001
    for i in (0, 1, 2, 3, 4, 7, 99_999, 200_002):
        w = R.philox4x32_10(np.array([[i // 4, 0, 0, 0]], dtype=np.uint32), (seed & 0xFFFFFFFF, seed >> 32))[0, i % 4]
        u = np.float32(int(w) >> 8) * np.float32(2.0**-24)
        assert float(m[i]) == (float(scale) if u >= np.float32(p) else 0.0), i
    assert torch.equal(R.dropout_mask(5, 0.0, 3), torch.ones(5))  # p = 0 keeps all at scale 1
    other = R.dropout_mask(1000, p, seed + 1)
    assert not torch.equal(other, m[:1000])  # another seed, another mask


def test_shared_dropout_mask_axes():
    """Row-shared masks are [B, 1, Cc, D] with entry (b, c, d) at b Cc D + c D + d; column-shared
    [B, R, 1, D] with (b, r, d) at b R D + r D + d (dropout_add.py:81-88)."""
    B, Rr, Cc, D = 2, 3, 5, 4
    flat_r = R.dropout_mask(B * Cc * D, 0.5, 9)
    flat_c = R.dropout_mask(B * Rr * D, 0.5, 9)
    mr = R.shared_dropout_mask((B, Rr, Cc, D), True, 0.5, 9)
    mc = R.shared_dropout_mask((B, Rr, Cc, D), False, 0.5, 9)
    assert mr.shape == (B, 1, Cc, D) and mc.shape == (B, Rr, 1, D)
    for b in range(B):
        for c in range(Cc):
            for d in range(D):
                assert mr[b, 0, c, d] == flat_r[b * Cc * D + c * D + d]
        for r in range(Rr):
            for d in range(D):
                assert mc[b, r, 0, d] == flat_c[b * Rr * D + r * D + d]


def test_dropout_add_closed_forms():
    g = torch.Generator().manual_seed(3)
    res, x = torch.randn(2, 4, 5, 8, generator=g), torch.randn(2, 4, 5, 8, generator=g)
    ones = torch.ones(2, 1, 5, 8)
    assert torch.equal(R.dropout_add(res, x, ones), res + x)
    assert torch.equal(R.dropout_add(res, x, torch.zeros(2, 4, 1, 8)), res)
    m = R.shared_dropout_mask((2, 4, 5, 8), True, 0.25, 11)
    out = R.dropout_add(res, x, m)
    kept = (m > 0).expand_as(x)
    assert torch.equal(out[~kept], res[~kept])
    assert torch.allclose(out[kept], (res + x * (4.0 / 3.0))[kept], rtol=0, atol=1e-6)
    # bf16 residual: fp32 arithmetic rounded once
    rb, xb = res.bfloat16(), x.bfloat16()
    assert torch.equal(R.dropout_add(rb, xb, m), (rb.float() + xb.float() * m).bfloat16())


_DROP_SITES = (("tri_mul_out", True), ("tri_mul_in", True), ("pair_attn_row", True), ("pair_attn_col", False))


def test_block_dropout_composition():
    """Unit masks give the eval block; a zero mask at one site equals the block with that
    branch's output projection zeroed (the branch adds nothing there); a mask that drops some
    entries lands between."""
    sd = W.make_block_weights(31, perturb_affine=True)
    x = W.make_inputs(9, seed=5, pad_last=1)
    args = (x["pair"], x["single"], x["pair_mask"], x["seq_mask"])
    shape = tuple(x["pair"].shape)
    unit = {s: torch.ones((1, 1, 9, 128) if rw else (1, 9, 1, 128)) for s, rw in _DROP_SITES}
    with torch.no_grad():
        p0, s0 = R.pairformer_block(*args, sd)
        p1, s1 = R.pairformer_block(*args, sd, dropout=unit)
        assert torch.equal(p0, p1) and torch.equal(s0, s1)
        for site, rw in _DROP_SITES:
            zero = dict(unit, **{site: torch.zeros_like(unit[site])})
            pz, sz = R.pairformer_block(*args, sd, dropout=zero)
            pw, sw = R.pairformer_block(*args, {**sd, f"{site}.out_proj.weight": torch.zeros(128, 128)})
            assert torch.equal(pz, pw) and torch.equal(sz, sw), site
        masks = {s: R.shared_dropout_mask(shape, rw, 0.25, 100 + i) for i, (s, rw) in enumerate(_DROP_SITES)}
        pd, _ = R.pairformer_block(*args, sd, dropout=masks)
    assert rel_l2(pd, p0) > 1e-3


def test_block_without_deleted_branches():
    """use_triangle_attention=False equals the full block with both attention output
    projections zeroed (evoformer.py:302-310); use_single_track=False leaves single unchanged
    and the pair update that of the full block (the single track never writes to pair)."""
    sd = W.make_block_weights(32, perturb_affine=True)
    x = W.make_inputs(10, seed=6, pad_last=2)
    args = (x["pair"], x["single"], x["pair_mask"], x["seq_mask"])
    no_attn = {k: v for k, v in sd.items() if not k.startswith("pair_attn_")}
    zeroed = {**sd, "pair_attn_row.out_proj.weight": torch.zeros(128, 128),
              "pair_attn_col.out_proj.weight": torch.zeros(128, 128)}  # fmt: skip
    no_single = {k: v for k, v in sd.items() if not k.startswith("single_")}
    with torch.no_grad():
        pa, sa = R.pairformer_block(*args, no_attn, use_triangle_attention=False)
        pz, sz = R.pairformer_block(*args, zeroed)
        ps, ss = R.pairformer_block(*args, no_single, use_single_track=False)
        pf, _ = R.pairformer_block(*args, sd)
    assert torch.equal(pa, pz) and torch.equal(sa, sz)
    assert torch.equal(ps, pf) and ss is x["single"]


def test_evoformer_block_without_triangle_attention():
    sd = W.make_evoformer_block_weights(33, perturb_affine=True)
    no_attn = {k: v for k, v in sd.items() if not k.startswith("pair_attn_")}
    zeroed = {**sd, "pair_attn_row.out_proj.weight": torch.zeros(128, 128),
              "pair_attn_col.out_proj.weight": torch.zeros(128, 128)}  # fmt: skip
    x = W.make_inputs(7, seed=7, pad_last=1)
    gen = torch.Generator().manual_seed(2)
    msa = torch.randn(1, 3, 7, 64, generator=gen)
    mmask = (torch.rand(1, 3, 7, generator=gen) > 0.2).float()
    with torch.no_grad():
        m1, z1 = R.evoformer_block(msa, x["pair"], mmask, x["pair_mask"], no_attn, use_triangle_attention=False)
        m2, z2 = R.evoformer_block(msa, x["pair"], mmask, x["pair_mask"], zeroed)
        # MSA dropout: a zero mask on row_attn equals a zeroed row_attn.out_proj
        m3, z3 = R.evoformer_block(msa, x["pair"], mmask, x["pair_mask"], sd, dropout={"row_attn": torch.zeros(1, 1, 7, 64)})
        m4, z4 = R.evoformer_block(msa, x["pair"], mmask, x["pair_mask"], {**sd, "row_attn.out_proj.weight": torch.zeros(64, 64)})
    assert torch.equal(m1, m2) and torch.equal(z1, z2)
    assert torch.equal(m3, m4) and torch.equal(z3, z4)


def test_pair_bias_gate_pins():
    """The per-head pair-bias gate (attention.py:392-398, :422-424): a = 0 (tau = 1) is the
    ungated attention exactly; a gated block equals the ungated block whose single_to_pair
    weight rows are scaled by tau_h (the logits are linear in that weight); a head with a
    large tau lets its pair logits dominate that head's weights."""
    sd = W.make_block_weights(33, perturb_affine=True, pair_bias_gate=True)
    x = W.make_inputs(11, seed=7, pad_last=2)
    args = (x["pair"], x["single"], x["pair_mask"], x["seq_mask"])
    ungated = {k: v for k, v in sd.items() if k != "single_attn.pair_bias_gate_a"}
    tau = torch.exp(sd["single_attn.pair_bias_gate_a"])
    with torch.no_grad():
        p0, s0 = R.pairformer_block(*args, ungated)
        p1, s1 = R.pairformer_block(*args, {**ungated, "single_attn.pair_bias_gate_a": torch.zeros(16)})
        assert torch.equal(p0, p1) and torch.equal(s0, s1)
        pg, sg = R.pairformer_block(*args, sd)
        folded = {**ungated, "single_to_pair.weight": ungated["single_to_pair.weight"] * tau[:, None]}
        pf, sf = R.pairformer_block(*args, folded)
        assert torch.equal(pg, p0)  # the gate touches only the single track
        assert rel_l2(sg, sf) < 1e-6 and rel_l2(sg, s0) > 1e-4


def test_rms_normalize_closed_forms():
    """primitives.py:79-87: unit RMS per row (up to eps = 1e-6), invariant to a positive row
    scale, zero rows stay zero."""
    g = torch.Generator().manual_seed(9)
    x = torch.randn(50, 128, generator=g) * (0.5 + 10 * torch.rand(50, 1, generator=g))
    y = R.rms_normalize(x)
    rms = y.pow(2).mean(-1).sqrt()
    assert (rms - 1).abs().max() < 1e-5
    assert rel_l2(R.rms_normalize(3.5 * x), y) < 1e-6
    assert torch.equal(R.rms_normalize(torch.zeros(2, 128)), torch.zeros(2, 128))


def test_rmsnorm_branch_scaler_block_invariance():
    """With branch_scaler="rmsnorm" every branch enters the residual stream at unit RMS times
    its scale, so multiplying a branch's output projection by a positive constant changes
    nothing up to eps (and changes the identity-scaler block); the residual scale s then sets the
    size of the first increment: RMS(pair1 - pair0) = s per token, up to eps."""
    sd = W.make_block_weights(34, perturb_affine=True)
    x = W.make_inputs(10, seed=8, pad_last=2)
    args = (x["pair"], x["single"], x["pair_mask"], x["seq_mask"])
    scaled = dict(sd)
    for k, c in (("tri_mul_out.out_proj.weight", 3.0), ("pair_attn_col.out_proj.weight", 0.25),
                 ("pair_transition.linear2.weight", 2.0), ("single_attn.out_proj.weight", 5.0),
                 ("single_transition.linear2.weight", 0.5)):  # fmt: skip
        scaled[k] = sd[k] * c
    with torch.no_grad():
        p0, s0 = R.pairformer_block(*args, sd, branch_scaler="rmsnorm")
        p1, s1 = R.pairformer_block(*args, scaled, branch_scaler="rmsnorm")
        q0, _ = R.pairformer_block(*args, sd)
        q1, _ = R.pairformer_block(*args, scaled)
        # eps = 1e-6 against branch rows of mean square down to ~1e-3: invariance to ~1e-4
        assert rel_l2(p1, p0) < 1e-3 and rel_l2(s1, s0) < 1e-3
        assert rel_l2(q1, q0) > 0.1
        # only tri_mul_out active: the increment is s times a unit-RMS row
        only = {k: (torch.zeros_like(v) if k.endswith(("out_proj.weight", "linear2.weight")) and
                    not k.startswith("tri_mul_out.") else v) for k, v in sd.items()}  # fmt: skip
        p2, _ = R.pairformer_block(*args, only, branch_scaler="rmsnorm", scales={"residual_out_scale": 0.3})
    inc = (p2 - x["pair"]).pow(2).mean(-1).sqrt()
    assert (inc - 0.3).abs().max() < 5e-4  # eps = 1e-6 against rows of mean square >= ~1e-3
