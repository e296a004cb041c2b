"""GPU: the allocation-free single attention (pf_single_attn_fwd_noalloc) through the C ABI.

It runs the same kernels as pf_single_attn_fwd with the library's static scratch array in
place of a caller workspace, so its output must equal pf_single_attn_fwd's bit for bit.
Two calls in a row, the second on a smaller input (and, for the residual mode, into a
pre-filled output), check that the shared scratch carries nothing from one call into
the next. The refusal of sizes past the array's capacity is tested on the CPU
(tests/test_abi.py), since it returns before any device call.
"""

from __future__ import annotations

import pytest
import torch

from tests._helpers import mod, sub

pytestmark = pytest.mark.gpu
_lib = mod("_lib")
attention = mod("attention")
W = mod("weights")


def _case(dev, dtype, B, N, seed):
    g = torch.Generator().manual_seed(seed)
    s = torch.randn(B, N, 384, generator=g).to(dev, dtype)
    seq = (torch.rand(B, N, generator=g) > 0.1).float().to(dev)
    pl = torch.randn(B, 16, N, N, generator=g).to(dev)
    return s, seq, pl


def _args(op, s, seq, pl, out, accumulate, eps):
    B, N, C = s.shape
    code_z, code_c = _lib.dtype_code(s.dtype), _lib.dtype_code(op["wqkvg"].dtype)
    return [
        s.data_ptr(), seq.data_ptr(), pl.data_ptr(), op["lnw"].data_ptr(), op["lnb"].data_ptr(), eps,
        op["wqkvg"].data_ptr(), op["qb"].data_ptr(), op["w_out"].data_ptr(), B, N, C, 16, code_z, code_c,
        out.data_ptr(), int(accumulate),
    ]  # fmt: skip


def _with_workspace(op, s, seq, pl, out, accumulate, eps):
    B, N, C = s.shape
    code_c = _lib.dtype_code(op["wqkvg"].dtype)
    nbytes = _lib.lib().pf_single_attn_workspace_bytes(B, N, C, 16, code_c)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=s.device)
    _lib.call("pf_single_attn_fwd", *_args(op, s, seq, pl, out, accumulate, eps), ws.data_ptr(), nbytes,
              _lib.stream_of(s))  # fmt: skip


def _no_alloc(op, s, seq, pl, out, accumulate, eps):
    _lib.call("pf_single_attn_fwd_noalloc", *_args(op, s, seq, pl, out, accumulate, eps), _lib.stream_of(s))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_no_alloc_single_attention_matches_workspace_entry(dev, dtype):
    sd = W.make_block_weights(41, perturb_affine=True)
    sa = attention.SingleAttention(384).to(dev)
    sa.load_state_dict(sub(sd, "single_attn."))
    op = sa._operands(dtype)
    eps = sa.norm.eps
    # first call: the larger input, plain output; second: smaller, accumulated into a
    # pre-filled output
    for (B, N, accumulate, seed) in ((1, 700, False, 1), (2, 300, True, 2)):
        print(f"[no-alloc single attention {dtype} B={B} N={N} accumulate={accumulate}]", flush=True)
        s, seq, pl = _case(dev, dtype, B, N, seed)
        base = torch.randn(s.shape, generator=torch.Generator().manual_seed(seed + 10)).to(dev, dtype)
        want, got = base.clone(), base.clone()
        _with_workspace(op, s, seq, pl, want, accumulate, eps)
        _no_alloc(op, s, seq, pl, got, accumulate, eps)
        torch.cuda.synchronize()
        assert torch.isfinite(got).all()
        assert torch.equal(got, want), f"B={B} N={N}: max diff {(got.float() - want.float()).abs().max().item():.3e}"
