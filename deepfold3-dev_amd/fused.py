"""The reference's kernel-level operators (``src/deepfold3/model/triton/``) on the HIP library.

Same class and function names, constructor arguments and call signatures as the
reference, so call sites written against its Triton layer run unchanged:

- ``_EvoformerAttention.apply`` / ``fused_evo_attention`` (``evo_attention.py:1198-1510``)
- ``FusedPairBias`` (``fused_pair_bias.py:348-416``)
- ``FusedLayerNormTranspose`` (``layernorm_transpose.py:269-316``)
- ``FusedLayerNormLinear`` (``layernorm_linear.py:537-592``)
- ``FusedSwiGLU`` (``swiglu.py:192-200``)
- ``FusedTransitionBlock`` (``fused_transition.py:34-83``)
- ``dropout_add_rowwise`` / ``dropout_add_columnwise`` (``dropout_add.py:221-265``)

``_EvoformerAttention`` is differentiable (the HIP backward), and so are the others: under
grad the LayerNorm runs ``kernels.LayerNormFunction`` and SwiGLU ``kernels.SwiGLUFunction``
(HIP forward and backward), the small projections autograd's library GEMMs. Anything the
kernels cannot serve raises ``NotActive``. There is no PyTorch fallback for the kernels.
"""

from __future__ import annotations

import ctypes

import torch
import torch.nn as nn

from . import _lib, kernel_census
from .inference_guard import NotActive
from .kernels import (
    DropoutAddFunction,
    LayerNormFunction,
    SwiGLUFunction,
    cast_weight,
    dropout_add,
    gemm_dtype_for,
    layer_norm_for_gemm,
    ln_transpose,
    next_dropout_seed,
    residual_add,
    token_linear,
)
from .primitives import TransitionBlock, f32

__all__ = [
    "_EvoformerAttention",
    "fused_evo_attention",
    "FusedPairBias",
    "FusedLayerNormTranspose",
    "FusedLayerNormLinear",
    "FusedSwiGLU",
    "FusedTransitionBlock",
    "dropout_add_rowwise",
    "dropout_add_columnwise",
]


def _ws(nbytes: int, device) -> torch.Tensor:
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)


def _evo_fwd(Q, K, V, rm, pb, zero_rows: bool) -> torch.Tensor:
    """Forward in the kernel layout: Q, K, V ``[B,S,H,N,D]`` contiguous, rm ``[B,S,N]`` and
    pb ``[B,H,N,N]`` fp32. The flash kernel runs four heads per line; other head counts are
    zero-padded to a multiple of four and regrouped as extra batch items."""
    B, S, H, N, D = Q.shape
    code = _lib.dtype_code(Q.dtype)
    G = -(-H // 4)
    if H != 4:
        pad = 4 * G - H
        if pad:
            Q, K, V = (torch.cat([t, t.new_zeros(B, S, pad, N, D)], 2) for t in (Q, K, V))
            pb = torch.cat([pb, pb.new_zeros(B, pad, N, N)], 1)
        # (with B = 1 the reshape can return a strided view: the kernel needs dense operands)
        Q, K, V = (t.view(B, S, G, 4, N, D).transpose(1, 2).reshape(B * G, S, 4, N, D).contiguous() for t in (Q, K, V))
        rm = rm.repeat_interleave(G, dim=0)
        pb = pb.reshape(B * G, 4, N, N)
    Bk = Q.shape[0]
    ws_bytes = _lib.lib().pf_evo_attn_workspace_bytes(Bk, S, 4, N, D, code)
    if ws_bytes == 0:
        raise NotActive("evo_attention", f"D={D}: built for D=32")
    out = torch.empty(Q.shape, dtype=Q.dtype, device=Q.device)
    ws = _ws(ws_bytes, Q.device)
    _lib.call(
        "pf_evo_attn_fwd", Q.data_ptr(), K.data_ptr(), V.data_ptr(), rm.data_ptr(), pb.data_ptr(), Bk, S, 4, N, D,
        code, int(zero_rows), out.data_ptr(), ws.data_ptr(), ws_bytes, _lib.stream_of(Q),
    )  # fmt: skip
    _lib.note_redo("pf_evo_attn_redo_flags", ws, Bk, S, 4, N, D, code)
    if H != 4:
        out = out.view(B, G, S, 4, N, D).transpose(1, 2).reshape(B, S, 4 * G, N, D)[:, :, :H].contiguous()
    return out


def _evo_bwd(Q, K, V, rm, pb, dO, zero_rows: bool = True):
    """Backward in the kernel layout (``pf_evo_attn_bwd``): returns dQ, dK, dV (Q's dtype) and
    d_pair_bias ``[B,H,N,N]`` fp32. ``zero_rows`` selects the masked-row rule (True: the
    reference kernel's, zero gradients; False: the eager path's uniform softmax)."""
    B, S, H, N, D = Q.shape
    code = _lib.dtype_code(Q.dtype)
    dO = dO.to(Q.dtype).contiguous()
    ws_bytes = _lib.lib().pf_evo_attn_bwd_workspace_bytes(B, S, H, N, D, code)
    if ws_bytes == 0:
        raise NotActive("evo_attention.backward", f"H={H}, D={D}: built for D=32")
    dQ, dK, dV = (torch.empty(Q.shape, dtype=Q.dtype, device=Q.device) for _ in range(3))
    dpb = torch.empty((B, H, N, N), dtype=torch.float32, device=Q.device)
    ws = _ws(ws_bytes, Q.device)
    _lib.call(
        "pf_evo_attn_bwd", Q.data_ptr(), K.data_ptr(), V.data_ptr(), rm.data_ptr(), pb.data_ptr(), dO.data_ptr(),
        B, S, H, N, D, code, float(D) ** -0.5, int(zero_rows), dQ.data_ptr(), dK.data_ptr(), dV.data_ptr(),
        dpb.data_ptr(), ws.data_ptr(), ws_bytes, _lib.stream_of(Q),
    )  # fmt: skip
    return dQ, dK, dV, dpb


class _EvoAttnFunction(torch.autograd.Function):
    """Kernel-layout attention with the HIP backward; the forward saves its inputs only.
    ``apply(Q, K, V, rm, pb, zero_rows)``: both passes follow the same masked-row rule."""

    @staticmethod
    def forward(ctx, Q, K, V, rm, pb, zero_rows=True):
        ctx.save_for_backward(Q, K, V, rm, pb)
        ctx.zero_rows = bool(zero_rows)
        return _evo_fwd(Q, K, V, rm, pb, ctx.zero_rows)

    @staticmethod
    def backward(ctx, dO):
        Q, K, V, rm, pb = ctx.saved_tensors
        kernel_census.record("evo_attention.backward", "hip_evo_attn_bwd")
        dQ, dK, dV, dpb = _evo_bwd(Q, K, V, rm, pb, dO, ctx.zero_rows)
        return dQ, dK, dV, None, dpb, None


def _strides(*st: int) -> tuple:
    """A long[4] of element strides {batch, line, head, key} and the address to pass."""
    arr = (ctypes.c_long * 4)(*st)
    return arr, ctypes.addressof(arr)


class _GridAttnCore(torch.autograd.Function):
    """The flash attention of ``GridSelfAttention``'s training path on the token-major
    projection (``attention.py:211-257``, the fused branch): ``apply(qkv, res_mask,
    pair_bias, transpose)`` with qkv ``[B, N, N, 3, H, D]`` (q | k | v of every pair position
    (i, j)), res_mask ``[B, lines, N]`` additive fp32, pair_bias ``[B, H, N, N]`` fp32; lines are
    the rows i (transpose False) or the columns j (True). Returns O ``[B, N, N, H, D]`` in the
    same token order. The kernels read q, k, v and dO and write O and dq, dk, dv (into the
    gradient of qkv) through strides (``pf_evo_attn_fwd_strided`` / ``pf_evo_attn_bwd_strided``),
    so nothing is permuted or copied around them. The kernel's masked-line rule (a line whose
    keys are all masked outputs 0). H = 4, D = 32.

    With ``use_lse`` (the default) the forward also writes each row's log-sum-exp and the
    backward's dQ kernel takes it in place of its own pass over the keys for the row maximum
    (``pf_evo_attn_bwd_strided``'s ``lse``; the reference saves softmax_lse the same way,
    ``evo_attention.py:1279-1290``)."""

    use_lse = True

    @staticmethod
    def _layout(qkv, transpose):
        B, N1, N2, _, H, D = qkv.shape
        tok = 3 * H * D
        if transpose:  # lines j, keys i
            sx = (N1 * N2 * tok, tok, D, N2 * tok)
            so = (N1 * N2 * H * D, H * D, D, N2 * H * D)
        else:
            sx = (N1 * N2 * tok, N2 * tok, D, tok)
            so = (N1 * N2 * H * D, N2 * H * D, D, H * D)
        S = N2 if transpose else N1
        return B, S, H, N1, D, sx, so

    @staticmethod
    def forward(ctx, qkv, rm, pb, transpose):
        qkv = qkv.contiguous()
        B, S, H, N, D, sx, so = _GridAttnCore._layout(qkv, transpose)
        code = _lib.dtype_code(qkv.dtype)
        ws_bytes = _lib.lib().pf_evo_attn_workspace_bytes(B, S, H, N, D, code)
        if ws_bytes == 0:
            raise NotActive("GridSelfAttention", f"H={H}, D={D}: the strided attention is built for H=4, D=32")
        out = torch.empty(qkv.shape[:3] + (H, D), dtype=qkv.dtype, device=qkv.device)
        # row log-sum-exp (log2 units) for the backward's single dQ pass; rows padded to 128
        use_lse = _GridAttnCore.use_lse
        lse = torch.empty((B, S, H, -(-N // 128) * 128) if use_lse else (0,), dtype=torch.float32, device=qkv.device)
        ws = _ws(ws_bytes, qkv.device)
        es = qkv.element_size()
        base = qkv.data_ptr()
        ax, px = _strides(*sx)
        ao, po = _strides(*so)
        _lib.call(
            "pf_evo_attn_fwd_strided", base, base + H * D * es, base + 2 * H * D * es, px, rm.data_ptr(),
            pb.data_ptr(), B, S, H, N, D, code, 1, out.data_ptr(), po, lse.data_ptr() if use_lse else None,
            ws.data_ptr(), ws_bytes, _lib.stream_of(qkv),
        )  # fmt: skip
        _lib.note_redo("pf_evo_attn_redo_flags", ws, B, S, H, N, D, code)
        ctx.save_for_backward(qkv, rm, pb, lse)
        ctx.transpose = bool(transpose)
        return out

    @staticmethod
    def backward(ctx, dO):
        qkv, rm, pb, lse = ctx.saved_tensors
        B, S, H, N, D, sx, so = _GridAttnCore._layout(qkv, ctx.transpose)
        code = _lib.dtype_code(qkv.dtype)
        dO = dO.to(qkv.dtype).contiguous()
        ws_bytes = _lib.lib().pf_evo_attn_bwd_workspace_bytes(B, S, H, N, D, code)
        dqkv = torch.empty_like(qkv)
        dpb = torch.empty((B, H, N, N), dtype=torch.float32, device=qkv.device)
        ws = _ws(ws_bytes, qkv.device)
        es = qkv.element_size()
        base, gbase = qkv.data_ptr(), dqkv.data_ptr()
        ax, px = _strides(*sx)
        ao, po = _strides(*so)
        kernel_census.record("GridSelfAttention.backward", "hip_evo_attn_bwd_strided")
        _lib.call(
            "pf_evo_attn_bwd_strided", base, base + H * D * es, base + 2 * H * D * es, px, rm.data_ptr(),
            pb.data_ptr(), dO.data_ptr(), po, lse.data_ptr() if lse.numel() else None, B, S, H, N, D, code,
            float(D) ** -0.5, gbase, gbase + H * D * es, gbase + 2 * H * D * es, px, dpb.data_ptr(), ws.data_ptr(),
            ws_bytes, _lib.stream_of(qkv),
        )  # fmt: skip
        return dqkv, None, dpb, None


class _EvoformerAttention:
    """Flash attention with pair bias and per-line key mask (``evo_attention.py:1198-1292``).

    ``apply(Q, K, V, res_mask, pair_bias, pre_transposed=False, masked_rows="zero")``:
    Q, K, V ``[B, N_seq, N_res, H, D]`` (or ``[B, N_seq, H, N_res, D]`` with
    ``pre_transposed=True``), ``res_mask [B, N_seq, 1, 1, N_res]`` additive fp32,
    ``pair_bias [B, 1, H, N_res, N_res]`` fp32. Returns O in the layout of Q.
    ``masked_rows="zero"`` is the reference kernel's rule for a line whose keys are all
    masked (output 0, ``evo_attention.py:307-318``); ``"eager"`` gives the stock path's
    uniform average (``attention.py:157-160``). D = 32, any H.

    Differentiable in Q, K, V and pair_bias (``evo_attention.py:1295-1472``): under grad the
    backward runs ``pf_evo_attn_bwd`` (centred softmax Jacobian, row statistics recomputed,
    nothing saved but the inputs) under the same masked-row rule as the forward: zero
    gradients for a fully masked line (``"zero"``) or the uniform softmax's Jacobian
    (``"eager"``, what autograd of the stock path gives).
    """

    @staticmethod
    def apply(Q, K, V, res_mask, pair_bias, pre_transposed: bool = False, masked_rows: str = "zero"):
        _lib.require_device("evo_attention", Q, K, V, res_mask, pair_bias)
        if masked_rows not in ("zero", "eager"):
            raise ValueError(f"masked_rows must be 'zero' or 'eager', got {masked_rows!r}")
        grad = torch.is_grad_enabled() and any(t.requires_grad for t in (Q, K, V, pair_bias))
        if not pre_transposed:
            Q, K, V = (t.transpose(-2, -3) for t in (Q, K, V))
        Q, K, V = (t.contiguous() for t in (Q, K, V))
        B, S, H, N, D = Q.shape
        if K.shape != Q.shape or V.shape != Q.shape or K.dtype != Q.dtype or V.dtype != Q.dtype:
            raise NotActive("evo_attention", "Q, K, V must share shape and dtype")
        if D != 32:
            raise NotActive("evo_attention", f"D={D}: built for D=32")
        rm = res_mask.detach().to(torch.float32).expand(B, S, 1, 1, N).reshape(B, S, N).contiguous()
        pb = pair_bias.to(torch.float32).expand(B, 1, H, N, N).reshape(B, H, N, N).contiguous()
        if grad:
            kernel_census.record("evo_attention", "hip_evo_attn_grad")
            out = _EvoAttnFunction.apply(Q, K, V, rm, pb, masked_rows == "zero")
        else:
            kernel_census.record("evo_attention", "hip_evo_attn")
            with torch.no_grad():
                out = _evo_fwd(Q, K, V, rm, pb, masked_rows == "zero")
        if not pre_transposed:
            out = out.transpose(-2, -3).contiguous()
        return out


def fused_evo_attention(q, k, v, pair_bias, mask):
    """Reference wrapper (``evo_attention.py:1475-1510``): q, k, v ``[B*N_rows, N_cols, H, D]``,
    pair_bias ``[B or 1, H, N, N]``, mask ``[B*N_rows, N_cols]`` (1 keep, 0 drop)."""
    BN, N_cols, H, D = q.shape
    B = pair_bias.shape[0]
    N_rows = BN // B
    q5, k5, v5 = (t.view(B, N_rows, N_cols, H, D) for t in (q, k, v))
    res_mask = mask.view(B, N_rows, 1, 1, N_cols).float()
    res_mask = torch.where(res_mask > 0.5, 0.0, float("-inf"))
    if pair_bias.dim() == 4:
        pair_bias = pair_bias.unsqueeze(1)
    o5 = _EvoformerAttention.apply(q5, k5, v5, res_mask, pair_bias.float())
    return o5.view(BN, N_cols, H, D)


class FusedPairBias(nn.Module):
    """LN + ``[C -> H]`` projection + permute to ``[B, H, N, N]`` (stateless; ``fused_pair_bias.py:348-416``)."""

    def __init__(self, c: int, num_heads: int, eps: float = 1e-5):
        super().__init__()
        self.c, self.num_heads, self.eps = c, num_heads, eps

    def forward(self, z, ln_weight, ln_bias, proj_weight, mask=None):
        """Under grad: the HIP LayerNorm with its backward and the projection in autograd."""
        _lib.require_device("FusedPairBias", z)
        if torch.is_grad_enabled():
            kernel_census.record("GridSelfAttention.norm", "hip_pair_bias_grad")
            out = token_linear(layer_norm_for_gemm(z, ln_weight, ln_bias, self.eps), proj_weight).permute(0, 3, 1, 2)
            if mask is not None:
                out = out + (1.0 - mask.to(out.dtype))[:, None, None, :] * (-1e9)
            return out
        B, N, _, C = z.shape
        H = proj_weight.shape[0]
        if C != self.c or H > 16:
            raise NotActive("FusedPairBias", f"C={C}, H={H}: built for C=128, H<=16")
        zc = z.contiguous()
        w16 = torch.zeros(16, C, dtype=torch.float32, device=z.device)
        w16[:H] = proj_weight.detach().float()
        m = None if mask is None else mask.to(torch.float32).contiguous()
        out = torch.empty((B, H, N, N), dtype=z.dtype, device=z.device)
        kernel_census.record("GridSelfAttention.norm", "hip_pair_bias")
        _lib.call(
            "pf_pair_bias_fwd", zc.data_ptr(), _lib.dtype_code(z.dtype), f32(ln_weight).data_ptr(),
            f32(ln_bias).data_ptr(), float(self.eps), w16.data_ptr(), H, _lib.ptr(m), out.data_ptr(), B, N, C,
            _lib.stream_of(zc),
        )  # fmt: skip
        return out


class FusedLayerNormTranspose(nn.Module):
    """``LN(x).permute(0, 2, 1, 3)`` for x ``[B, N1, N2, C]`` (stateless; ``layernorm_transpose.py:269-316``)."""

    def __init__(self, c: int, do_transpose: bool = True, eps: float = 1e-5):
        super().__init__()
        self.c, self.do_transpose, self.eps = c, do_transpose, eps

    def forward(self, x, weight, bias):
        """Under grad: the HIP LayerNorm with its backward, then the permute in autograd."""
        if torch.is_grad_enabled():
            kernel_census.record("GridSelfAttention.norm", "hip_ln_transpose_grad")
            y = LayerNormFunction.apply(x, weight, bias, self.eps)
            return y.permute(0, 2, 1, 3) if self.do_transpose else y
        kernel_census.record("GridSelfAttention.norm", "hip_ln_transpose")
        return ln_transpose(x, weight, bias, self.eps, self.do_transpose)


class FusedLayerNormLinear(nn.Module):
    """``LN(X) W + b`` with W passed as ``[K, N]`` (stateless; ``layernorm_linear.py:537-592``)."""

    def __init__(self, in_features: int, out_features: int, has_linear_bias: bool = False):
        super().__init__()
        self.in_features, self.out_features, self.has_linear_bias = in_features, out_features, has_linear_bias
        self._wkey = None
        self._wval = None

    def _w_nk(self, W: torch.Tensor, cdt: torch.dtype) -> torch.Tensor:
        key = (W.data_ptr(), W._version, tuple(W.shape), cdt)
        if key != self._wkey:
            self._wval = cast_weight(W.detach().t().contiguous(), cdt)
            self._wkey = key
        return self._wval

    def forward(self, X, ln_weight, ln_bias, linear_weight, linear_bias=None):
        """Under grad: the HIP LayerNorm with its backward, then ``LN(X) W + b`` in autograd."""
        if linear_bias is not None and not self.has_linear_bias:
            raise ValueError("linear_bias provided but module configured with has_linear_bias=False")
        _lib.require_device("FusedLayerNormLinear", X)
        K, N = self.in_features, self.out_features
        if tuple(linear_weight.shape) != (K, N):
            raise NotActive("FusedLayerNormLinear", f"weight must be [K, N] = [{K}, {N}]")
        if torch.is_grad_enabled():
            kernel_census.record("FusedLayerNormLinear", "hip_layernorm_grad")
            y = token_linear(layer_norm_for_gemm(X, ln_weight, ln_bias, 1e-5), linear_weight.t())
            return y if linear_bias is None else y + linear_bias
        cdt = gemm_dtype_for(X)
        Xc = X.contiguous()
        M = Xc.numel() // K
        out = torch.empty(Xc.shape[:-1] + (N,), dtype=X.dtype, device=X.device)
        code_c = _lib.dtype_code(cdt)
        ws_bytes = _lib.lib().pf_layernorm_linear_workspace_bytes(M, K, code_c)
        ws = _ws(ws_bytes, X.device)
        b = None if linear_bias is None else f32(linear_bias)
        _lib.call(
            "pf_layernorm_linear_fwd", Xc.data_ptr(), _lib.dtype_code(X.dtype), f32(ln_weight).data_ptr(),
            f32(ln_bias).data_ptr(), 1e-5, self._w_nk(linear_weight, cdt).data_ptr(), _lib.ptr(b), M, K, N, code_c,
            out.data_ptr(), ws.data_ptr(), ws_bytes, _lib.stream_of(Xc),
        )  # fmt: skip
        return out


class FusedSwiGLU(nn.Module):
    """``silu(a) * b`` with ``[a, b] = split(x, 2, dim=-1)`` (``swiglu.py:192-200``)."""

    def forward(self, x):
        """Differentiable: the HIP backward under grad."""
        _lib.require_device("FusedSwiGLU", x)
        if torch.is_grad_enabled():
            return SwiGLUFunction.apply(x)
        xc = x.contiguous()
        D = xc.shape[-1] // 2
        y = torch.empty(xc.shape[:-1] + (D,), dtype=x.dtype, device=x.device)
        _lib.call("pf_swiglu_fwd", xc.data_ptr(), _lib.dtype_code(x.dtype), y.data_ptr(), xc.numel() // (2 * D), D,
                  _lib.stream_of(xc))  # fmt: skip
        return y


class FusedTransitionBlock(TransitionBlock):
    """The reference's fused pair transition (``fused_transition.py:34-83``): same keys, HIP kernels."""

    def __init__(self, channels: int, num_intermediate_factor: int = 4, optim=None):
        super().__init__(channels, num_intermediate_factor, optim=optim)
        self.channels = channels


def _dropout_add(residual, x, p_drop: float, training: bool, site: str, rowwise: bool):
    if training and p_drop > 0.0:
        _lib.require_device(site, residual, x)
        seed = next_dropout_seed()
        if torch.is_grad_enabled() and (residual.requires_grad or x.requires_grad):
            kernel_census.record(site, "hip_dropout_add_grad")
            return DropoutAddFunction.apply(residual, x, p_drop, rowwise, seed)
        kernel_census.record(site, "hip_dropout_add")
        return dropout_add(residual, x, p_drop, rowwise, seed)
    if torch.is_grad_enabled() and (residual.requires_grad or x.requires_grad):
        kernel_census.record(site, "add_grad")
        return residual + x  # eval dropout-add under autograd (dropout_add.py:236-237)
    kernel_census.record(site, "hip_add")
    return residual_add(residual, x)


def dropout_add_rowwise(residual, x, p_drop: float, training: bool, use_fused: bool = True):
    """``residual + dropout(x)`` with the mask shared along dim -3 (``dropout_add.py:221-242``):
    eval is ``residual + x``; training runs the HIP shared-mask dropout-add (differentiable
    under grad; the seed comes from ``kernels.next_dropout_seed``). ``use_fused`` is accepted
    for the reference's signature; there is one implementation."""
    return _dropout_add(residual, x, p_drop, training, "dropout_add_rowwise", True)


def dropout_add_columnwise(residual, x, p_drop: float, training: bool, use_fused: bool = True):
    """``residual + dropout(x)`` with the mask shared along dim -2 (``dropout_add.py:245-265``)."""
    return _dropout_add(residual, x, p_drop, training, "dropout_add_columnwise", False)
