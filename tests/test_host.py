"""CPU: host-side logic -- the kernel census, the refusal contract, the out-buffer check,
the default initialisation of the transition block, and the split-K token linear of the
training path."""

from __future__ import annotations

import math

import pytest
import torch

from tests._helpers import mod

census = mod("kernel_census")
guard = mod("inference_guard")
primitives = mod("primitives")
_lib = mod("_lib")
kernels = mod("kernels")


@pytest.fixture(autouse=True)
def _fresh_census():
    census.reset()
    yield
    census.reset()


def test_census_counts_and_snapshot():
    census.record("site", "a")
    census.record("site", "a")
    census.record("site", "b")
    census.record("other", "x")
    assert census.snapshot() == {"other": {"x": 1}, "site": {"a": 2, "b": 1}}
    census.reset_counts()
    assert census.snapshot() == {}


def test_census_shadowed_levers():
    census.requested("site", "fused")
    assert census.shadowed() == []  # the site has not dispatched yet
    census.record("site", "stock")
    assert census.shadowed() == ["site:fused"]
    census.record("site", "fused_rows")  # a variant of the lever counts as the lever
    assert census.shadowed() == []
    census.reset_counts()
    census.record("site", "stock")
    assert census.shadowed() == ["site:fused"]  # requested levers survive reset_counts


def test_census_inactive_and_warn_once():
    assert census.inactive("lever[C=64]", "gated to C=128") == {"lever[C=64]": "gated to C=128"}
    assert census.inactive("lever[C=64]", "other reason") == {"lever[C=64]": "gated to C=128"}
    assert census.inactive() == {"lever[C=64]": "gated to C=128"}
    assert census.warn_once("k") and not census.warn_once("k")
    text = census.format_census()
    assert "gated lever: lever[C=64]" in text


def test_census_counts_are_exact_under_threads():
    import threading

    def work():
        for _ in range(2000):
            census.record("site", "p")

    threads = [threading.Thread(target=work) for _ in range(8)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert census.snapshot() == {"site": {"p": 16000}}


def test_not_active_names_the_lever_and_records_the_refusal():
    with pytest.raises(guard.NotActive) as ei:
        raise guard.NotActive("GridSelfAttention", "C=64")
    assert ei.value.lever == "GridSelfAttention" and ei.value.reason == "C=64"
    assert "GridSelfAttention" in str(ei.value) and "C=64" in str(ei.value)
    assert census.snapshot() == {"GridSelfAttention": {"refused:C=64": 1}}


def test_inference_only_refuses_under_grad():
    calls = []

    @guard.inference_only("k")
    def kernel(x):
        calls.append(x)
        return x

    with pytest.raises(guard.InferenceOnlyKernelError):
        kernel(1)
    assert calls == [] and census.snapshot() == {"k": {"refused:grad_enabled": 1}}
    with torch.no_grad():
        assert kernel(2) == 2
    with torch.inference_mode():
        assert kernel(3) == 3
    assert calls == [2, 3]


def test_out_buffer_check():
    like = torch.empty(2, 3, 4)
    _lib.check_out("op", torch.empty(2, 3, 4), like)
    for bad in (torch.empty(2, 3, 5), torch.empty(2, 3, 4, dtype=torch.bfloat16), torch.empty(4, 3, 2).transpose(0, 2)):
        with pytest.raises(guard.NotActive):
            _lib.check_out("op", bad, like)


def _trunc_std(sigma: float) -> float:
    """Std of N(0, sigma^2) truncated at +-2 absolute (the AF3 init's truncation)."""
    a = 2.0 / sigma
    phi = math.exp(-a * a / 2) / math.sqrt(2 * math.pi)
    z = math.erf(a / math.sqrt(2))
    return sigma * math.sqrt(1 - 2 * a * phi / z)


@pytest.mark.parametrize("c,n", [(128, 4), (384, 4), (64, 2)])
def test_transition_block_default_init_matches_reference(c, n):
    """Reference defaults (primitives.py:219-238): linear1 with the AF3 'relu' scaling
    (std sqrt(2 / c) / 0.8796 before truncation at +-2), linear2 zero."""
    torch.manual_seed(0)
    blk = primitives.TransitionBlock(c, n)
    w1 = blk.linear1.weight
    assert w1.shape == (2 * n * c, c) and blk.linear2.weight.shape == (c, n * c)
    want = _trunc_std(math.sqrt(2.0 / c) / primitives.TRUNCATED_NORMAL_STDDEV_FACTOR)
    assert abs(w1.std().item() / want - 1) < 0.03, (w1.std().item(), want)
    assert w1.abs().max().item() <= 2.0
    assert torch.count_nonzero(blk.linear2.weight) == 0
    assert set(blk.state_dict()) == {"norm.weight", "norm.bias", "linear1.weight", "linear2.weight"}


def test_transition_block_out_gain_is_row_orthogonal():
    """linear_out_init_gain: linear2 = gain x a row-orthonormal matrix (orthogonal_, primitives.py:238)."""
    torch.manual_seed(1)
    gain = 0.01
    blk = primitives.make_transition_block(384, 4, linear_out_init_gain=gain)
    w = blk.linear2.weight.double()
    assert torch.allclose(w @ w.T, gain**2 * torch.eye(384, dtype=torch.float64), atol=1e-9)


def test_template_block_widths():
    """Built at the reference's template width (64 channels in 4 heads of 16,
    config.py:636-650), at 128 and 256; other widths and heads wider than 32 refuse by name."""
    evoformer = mod("evoformer")
    for c in (64, 128):
        assert sorted({k.split(".")[0] for k in evoformer.TemplatePairFormerBlock(c).state_dict()}) == [
            "pair_attn_col", "pair_attn_row", "pair_transition", "tri_mul_in", "tri_mul_out",
        ]  # fmt: skip
    blk = evoformer.TemplatePairFormerBlock(64)
    assert blk.pair_attn_row.head_dim == 16 and blk.pair_transition.linear1.weight.shape == (256, 64)
    for c, h in ((96, 4), (128, 2)):
        with pytest.raises(guard.NotActive) as ei:
            evoformer.TemplatePairFormerBlock(c, num_heads=h)
        assert ei.value.lever == "TemplatePairFormerBlock"


def test_confidence_layers_keys():
    evoformer = mod("evoformer")
    keys = list(evoformer.ConfidencePairFormer().state_dict())
    assert keys[0].startswith("layers.0.") and any(k.startswith("layers.3.") for k in keys)
    assert not any(k.startswith("layers.4.") for k in keys)


@pytest.mark.parametrize("n", [190, 181])  # M = 36100 = 10 chunks of 3610; 32761 + 1 past a threshold
def test_token_linear_gradients_match_linear(n):
    """The split-K weight gradient (chunks of a batched product, rows past the last whole
    chunk in one more product) against autograd's linear, fp64."""
    g = torch.Generator().manual_seed(n)
    x = torch.randn(1, n, n, 24, generator=g, dtype=torch.float64)
    w = torch.randn(40, 24, generator=g, dtype=torch.float64)
    gy = torch.randn(1, n, n, 40, generator=g, dtype=torch.float64)
    old = kernels.SPLIT_K_TOKENS
    kernels.SPLIT_K_TOKENS = 1000
    try:
        x1, w1 = x.clone().requires_grad_(True), w.clone().requires_grad_(True)
        y1 = kernels.token_linear(x1, w1)
        (y1 * gy).sum().backward()
    finally:
        kernels.SPLIT_K_TOKENS = old
    x2, w2 = x.clone().requires_grad_(True), w.clone().requires_grad_(True)
    y2 = torch.nn.functional.linear(x2, w2)
    (y2 * gy).sum().backward()
    assert torch.equal(y1, y2)
    torch.testing.assert_close(x1.grad, x2.grad, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(w1.grad, w2.grad, rtol=1e-10, atol=1e-10)


def test_split_chunk():
    assert kernels._split_chunk(768 * 768) == 4096
    assert kernels._split_chunk(190 * 190) == 3610
    assert kernels._split_chunk(32761) == 4096  # 181^2 = 32761: no divisor in range
