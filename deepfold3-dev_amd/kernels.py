"""Functional HIP ops with the reference kernel layer's signatures (``src/deepfold3/model/triton/``).

Each function here is a thin shim over one C-ABI entry point of
``libpairformer_hip.so``: it checks devices and shapes, allocates the output
and the workspace with torch's caching allocator, and launches on torch's
current stream. There is no torch fallback; a call the kernels cannot serve
raises :class:`NotActive`.
"""

from __future__ import annotations

import weakref

import torch

from . import _lib, kernel_census
from .inference_guard import NotActive, inference_only

__all__ = [
    "gemm_dtype_for",
    "cast_weight",
    "layer_norm",
    "ln_transpose",
    "pack_trimul_weights",
    "trimul_forward",
    "fused_trimul",
    "residual_add",
    "next_dropout_seed",
    "dropout_mask",
    "dropout_add",
    "DropoutAddFunction",
    "pack_grid_attn_weights",
    "grid_attention_forward",
    "pair_transition_forward",
    "single_to_pair",
    "transition_forward",
    "single_attention_forward",
]


def gemm_dtype_for(x: torch.Tensor) -> torch.dtype:
    """GEMM operand dtype for activations ``x``.

    bf16 when ``x`` is bf16 or when bf16 autocast is on for its device (the
    reference's inference regime, ``scripts/inference.py:803-806``); fp32
    otherwise (fp32 MFMA, the 1e-5 parity regime).
    """
    if x.dtype == torch.bfloat16:
        return torch.bfloat16
    dev = x.device.type
    if torch.is_autocast_enabled(dev) and torch.get_autocast_dtype(dev) == torch.bfloat16:
        return torch.bfloat16
    return torch.float32


def _f32(t: torch.Tensor) -> torch.Tensor:
    return t.detach().to(torch.float32).contiguous()


def cast_weight(w: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """A contiguous ``dtype`` copy of ``w`` made by the HIP cast kernel."""
    _lib.require_device("cast_weight", w)
    src = w.detach().contiguous()
    out = torch.empty(src.shape, dtype=dtype, device=src.device)
    _lib.call(
        "pf_cast", src.data_ptr(), _lib.dtype_code(src.dtype), out.data_ptr(), _lib.dtype_code(dtype), src.numel(),
        _lib.stream_of(src),
    )  # fmt: skip
    return out


def scaled_weight(w: torch.Tensor, scale: float, dtype: torch.dtype) -> torch.Tensor:
    """``cast_weight(scale * w)``: a residual branch's output projection with the branch's
    residual scale folded in. Every scaled branch ends in this bias-free linear map, so
    ``x + s F(x)`` is ``x + F'(x)`` with ``W_out' = s W_out`` (``evoformer.py:282-321``)."""
    if scale == 1.0:
        return cast_weight(w, dtype)
    return cast_weight(w.detach().to(torch.float32) * float(scale), dtype)


def residual_add(res: torch.Tensor, x: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """``res + x`` in ``res``'s dtype (eval-mode dropout-add, ``triton/dropout_add.py:221-265``)."""
    _lib.require_device("residual_add", res, x)
    if res.shape != x.shape:
        raise NotActive("residual_add", f"shape mismatch {tuple(res.shape)} vs {tuple(x.shape)}")
    res_c, x_c = res.contiguous(), x.contiguous()
    if out is None:
        out = torch.empty_like(res_c)
    else:
        _lib.check_out("residual_add", out, res_c)
    _lib.call(
        "pf_add", res_c.data_ptr(), _lib.dtype_code(res_c.dtype), x_c.data_ptr(), _lib.dtype_code(x_c.dtype),
        out.data_ptr(), res_c.numel(), _lib.stream_of(res_c),
    )  # fmt: skip
    return out


def rms_residual_add(res: torch.Tensor | None, x: torch.Tensor, scale: float, out: torch.Tensor | None = None,
                     eps: float = 1e-6) -> torch.Tensor:
    """``res + scale * x / sqrt(mean x^2 + eps)`` over the last axis (the RMSNorm branch scaler,
    ``branch_scaler.py:38-50``, then the residual add), or the scaled branch alone when ``res``
    is None; ``out`` may be ``res`` (in place). One HIP pass (pf_rms_residual_add)."""
    _lib.require_device("rms_residual_add", x)
    xc = x.contiguous()
    C = xc.shape[-1]
    ref = xc if res is None else res
    if res is not None and (res.shape != xc.shape or not res.is_contiguous()):
        raise NotActive("rms_residual_add", "res must be contiguous and shaped like x")
    if out is None:
        out = torch.empty_like(ref)
    else:
        _lib.check_out("rms_residual_add", out, ref)
    _lib.call(
        "pf_rms_residual_add", _lib.ptr(res), _lib.dtype_code(ref.dtype), xc.data_ptr(), _lib.dtype_code(xc.dtype),
        out.data_ptr(), xc.numel() // C, C, float(scale), float(eps), _lib.stream_of(xc),
    )  # fmt: skip
    return out


def next_dropout_seed() -> int:
    """A 63-bit seed for one dropout-add, drawn from torch's default CPU generator.

    The reference draws each call's seed from a private generator (``dropout_add.py:33-48``).
    Drawing from the default generator instead makes the masks reproducible under
    ``torch.manual_seed`` and under activation checkpointing: ``torch.utils.checkpoint``
    restores the CPU RNG state before it recomputes a block, so the recomputed forward
    regenerates the masks of the original one."""
    return int(torch.randint(0, 2**63 - 1, (1,), dtype=torch.int64).item())


def _dropout_dims(x: torch.Tensor) -> tuple[int, int, int, int]:
    """[..., R, Cc, D] as (B, R, Cc, D) with the leading dims folded into B."""
    if x.dim() < 3:
        raise NotActive("dropout_add", f"needs [..., R, Cc, D], got shape {tuple(x.shape)}")
    *lead, R, Cc, D = x.shape
    B = 1
    for d in lead:
        B *= d
    if D % 4:
        raise NotActive("dropout_add", f"last dim {D} must be a multiple of 4")
    return B, R, Cc, D


def dropout_mask(shape, rowwise: bool, p: float, seed: int, device) -> torch.Tensor:
    """The shared mask a dropout-add of an activation of ``shape`` [..., R, Cc, D] applies,
    broadcastable to it ([..., 1, Cc, D] row-shared or [..., R, 1, D] column-shared), fp32 entries
    0 or 1/(1-p) (``pf_dropout_mask``)."""
    *lead, R, Cc, D = shape
    mshape = (*lead, 1, Cc, D) if rowwise else (*lead, R, 1, D)
    out = torch.empty(mshape, dtype=torch.float32, device=device)
    _lib.require_device("dropout_mask", out)
    _lib.call("pf_dropout_mask", out.data_ptr(), out.numel(), float(p), int(seed), _lib.stream_of(out))
    return out


def dropout_add(res: torch.Tensor, x: torch.Tensor, p: float, rowwise: bool, seed: int,
                out: torch.Tensor | None = None) -> torch.Tensor:  # fmt: skip
    """Training-mode ``res + dropout(x)`` with the mask shared along dim -3 (``rowwise``) or -2
    (``dropout_add.py:57-99``, ``:221-265``), in ``res``'s dtype; ``out`` may be ``res`` (in place).
    Not differentiable: ``DropoutAddFunction`` is the autograd form."""
    _lib.require_device("dropout_add", res, x)
    if res.shape != x.shape:
        raise NotActive("dropout_add", f"shape mismatch {tuple(res.shape)} vs {tuple(x.shape)}")
    B, R, Cc, D = _dropout_dims(x)
    res_c, x_c = res.contiguous(), x.contiguous()
    if out is None:
        out = torch.empty_like(res_c)
    elif out is not res or not res.is_contiguous():
        _lib.check_out("dropout_add", out, res_c)
    _lib.call(
        "pf_dropout_add_fwd", res_c.data_ptr(), _lib.dtype_code(res_c.dtype), x_c.data_ptr(),
        _lib.dtype_code(x_c.dtype), out.data_ptr(), B, R, Cc, D, int(rowwise), float(p), int(seed),
        _lib.stream_of(res_c),
    )  # fmt: skip
    return out


class DropoutAddFunction(torch.autograd.Function):
    """``apply(res, x, p, rowwise, seed)``: differentiable shared-mask dropout-add on the HIP
    kernels (``dropout_add.py:137-201``): the forward ``pf_dropout_add_fwd``, the backward passes
    the cotangent to ``res`` and regenerates the mask from the seed for ``x``
    (``pf_dropout_bwd``); nothing but the seed is saved."""

    @staticmethod
    def forward(ctx, res, x, p, rowwise, seed):
        ctx.meta = (float(p), bool(rowwise), int(seed), x.dtype, res.dtype)
        return dropout_add(res.detach(), x.detach(), p, rowwise, seed)

    @staticmethod
    def backward(ctx, g):
        p, rowwise, seed, x_dtype, res_dtype = ctx.meta
        g = g.contiguous()
        B, R, Cc, D = _dropout_dims(g)
        gx = torch.empty(g.shape, dtype=x_dtype, device=g.device)
        _lib.call(
            "pf_dropout_bwd", g.data_ptr(), _lib.dtype_code(g.dtype), gx.data_ptr(), _lib.dtype_code(x_dtype), B, R,
            Cc, D, int(rowwise), p, seed, _lib.stream_of(g),
        )  # fmt: skip
        gres = g if g.dtype == res_dtype else g.to(res_dtype)
        return gres, gx, None, None, None


def layer_norm(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor, eps: float = 1e-5) -> torch.Tensor:
    """LayerNorm over the last dim with fp32 statistics, in x's dtype (``primitives.py:90-115``)."""
    _lib.require_device("layer_norm", x, weight, bias)
    C = x.shape[-1]
    xc = x.contiguous()
    out = torch.empty_like(xc)
    _lib.call(
        "pf_layernorm_fwd", xc.data_ptr(), _lib.dtype_code(xc.dtype), _f32(weight).data_ptr(), _f32(bias).data_ptr(),
        float(eps), out.data_ptr(), xc.numel() // C, C, _lib.stream_of(xc),
    )  # fmt: skip
    return out


class LayerNormFunction(torch.autograd.Function):
    """Differentiable LayerNorm on the HIP kernels (``primitives.py:90-115`` semantics: fp32
    statistics, output in x's dtype): ``pf_layernorm_fwd`` and ``pf_layernorm_bwd``, the
    affine gradients summed over rows in a fixed order. ``apply(x, weight, bias, eps)``;
    ``apply(x, weight, bias, eps, out_dtype)`` writes the output in ``out_dtype`` instead
    (``pf_layernorm_fwd_mixed``). The backward takes the cotangent in its own dtype
    (``pf_layernorm_bwd_mixed``) and returns dx in x's dtype."""

    @staticmethod
    def forward(ctx, x, weight, bias, eps, *out_dtype):
        xc = x.detach().contiguous()
        odt = out_dtype[0] if out_dtype and out_dtype[0] is not None else xc.dtype
        if odt == xc.dtype:
            out = layer_norm(xc, weight, bias, eps)
        else:
            _lib.require_device("layer_norm", xc, weight, bias)
            C = xc.shape[-1]
            out = torch.empty(xc.shape, dtype=odt, device=xc.device)
            _lib.call(
                "pf_layernorm_fwd_mixed", xc.data_ptr(), _lib.dtype_code(xc.dtype), _f32(weight).data_ptr(),
                _f32(bias).data_ptr(), float(eps), out.data_ptr(), _lib.dtype_code(odt), xc.numel() // C, C,
                _lib.stream_of(xc),
            )  # fmt: skip
        ctx.save_for_backward(xc, weight)
        ctx.eps = float(eps)
        ctx.dtypes = (weight.dtype, bias.dtype)
        ctx.nextra = len(out_dtype)
        return out

    @staticmethod
    def backward(ctx, dy):
        xc, weight = ctx.saved_tensors
        C = xc.shape[-1]
        M = xc.numel() // C
        dyc = dy.contiguous() if dy.dtype in (torch.float32, torch.bfloat16) else dy.to(xc.dtype).contiguous()
        dx = torch.empty_like(xc)
        dw, db = (torch.empty(C, dtype=torch.float32, device=xc.device) for _ in range(2))
        ws_bytes = _lib.lib().pf_layernorm_bwd_workspace_bytes(M, C)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=xc.device)
        kernel_census.record("LayerNorm.backward", "hip_layernorm_bwd")
        _lib.call(
            "pf_layernorm_bwd_mixed", xc.data_ptr(), _lib.dtype_code(xc.dtype), dyc.data_ptr(),
            _lib.dtype_code(dyc.dtype), _f32(weight).data_ptr(), ctx.eps, dx.data_ptr(), dw.data_ptr(), db.data_ptr(),
            M, C, ws.data_ptr(), ws_bytes, _lib.stream_of(xc),
        )  # fmt: skip
        return (dx, dw.to(ctx.dtypes[0]), db.to(ctx.dtypes[1]), None) + (None,) * ctx.nextra


def layer_norm_for_gemm(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor, eps: float) -> torch.Tensor:
    """Differentiable LayerNorm whose output feeds GEMMs. Under bf16 autocast an fp32 x gives
    the bf16 output the next GEMM would cast it to, in the same pass (the reference's
    autocast path: fp32 LayerNorm, then the cast), and the cotangent comes back in bf16."""
    dev = x.device.type
    if x.dtype == torch.float32 and torch.is_autocast_enabled(dev) and torch.get_autocast_dtype(dev) == torch.bfloat16:
        return LayerNormFunction.apply(x, weight, bias, eps, torch.bfloat16)
    return LayerNormFunction.apply(x, weight, bias, eps)


class SwiGLUFunction(torch.autograd.Function):
    """Differentiable ``silu(x[..., :D]) * x[..., D:]`` on the HIP kernels (``pf_swiglu_fwd``,
    ``pf_swiglu_bwd``; the reference's ``FusedSwiGLU``, ``triton/swiglu.py:60-95``, ``:192-200``)."""

    @staticmethod
    def forward(ctx, x):
        _lib.require_device("swiglu", x)
        xc = x.detach().contiguous()
        D = xc.shape[-1] // 2
        y = torch.empty(xc.shape[:-1] + (D,), dtype=xc.dtype, device=xc.device)
        _lib.call("pf_swiglu_fwd", xc.data_ptr(), _lib.dtype_code(xc.dtype), y.data_ptr(), xc.numel() // (2 * D), D,
                  _lib.stream_of(xc))  # fmt: skip
        ctx.save_for_backward(xc)
        return y

    @staticmethod
    def backward(ctx, dy):
        (xc,) = ctx.saved_tensors
        D = xc.shape[-1] // 2
        dyc = dy.to(xc.dtype).contiguous()
        dx = torch.empty_like(xc)
        kernel_census.record("SwiGLU.backward", "hip_swiglu_bwd")
        _lib.call("pf_swiglu_bwd", xc.data_ptr(), dyc.data_ptr(), _lib.dtype_code(xc.dtype), dx.data_ptr(),
                  xc.numel() // (2 * D), D, _lib.stream_of(xc))  # fmt: skip
        return dx


def ln_transpose(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor, eps: float, do_transpose: bool):
    """``LN(x).permute(0, 2, 1, 3)`` for x [B,N1,N2,C] (``triton/layernorm_transpose.py:269-316``)."""
    _lib.require_device("ln_transpose", x)
    if x.dim() != 4:
        raise NotActive("ln_transpose", "input must be [B, N1, N2, C]")
    B, N1, N2, C = x.shape
    xc = x.contiguous()
    out = torch.empty((B, N2, N1, C) if do_transpose else (B, N1, N2, C), dtype=x.dtype, device=x.device)
    _lib.call(
        "pf_ln_transpose_fwd", xc.data_ptr(), _lib.dtype_code(xc.dtype), _f32(weight).data_ptr(),
        _f32(bias).data_ptr(), float(eps), out.data_ptr(), B, N1, N2, C, int(do_transpose), _lib.stream_of(xc),
    )  # fmt: skip
    return out


# ---------------------------------------------------------------- triangle multiplication

# Channel counts of the triangle-multiplication kernels: 128 (trunk, confidence head; fused
# persistent K1/K3 in bf16), 64 (template stack), 256 (the 256-channel trunk).
TRIMUL_CHANNELS = (64, 128, 256)


def pack_trimul_weights(w_proj: torch.Tensor, w_gate: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """Pack block-ordered ``[2C, C]`` projection and gate weights into the ``[4C, C]`` K1 operand."""
    _lib.require_device("pack_trimul_weights", w_proj, w_gate)
    C = w_proj.shape[1]
    if w_proj.shape != (2 * C, C) or w_gate.shape != (2 * C, C):
        raise NotActive("fused_trimul", f"projection weights must be [2C, C], got {tuple(w_proj.shape)}")
    wp, wg = w_proj.detach().contiguous(), w_gate.detach().to(w_proj.dtype).contiguous()
    packed = torch.empty((4 * C, C), dtype=dtype, device=wp.device)
    _lib.call(
        "pf_trimul_pack_weights", wp.data_ptr(), wg.data_ptr(), _lib.dtype_code(wp.dtype), packed.data_ptr(), C,
        _lib.dtype_code(dtype), _lib.stream_of(wp),
    )  # fmt: skip
    return packed


def trimul_forward(
    z: torch.Tensor,
    mask: torch.Tensor,
    ln_in_w: torch.Tensor,
    ln_in_b: torch.Tensor,
    eps_in: float,
    w_packed: torch.Tensor,
    ln_out_w: torch.Tensor,
    ln_out_b: torch.Tensor,
    eps_out: float,
    w_out: torch.Tensor,
    w_out_gate: torch.Tensor,
    outgoing: bool,
    out: torch.Tensor | None = None,
    accumulate: bool = False,
    mix: tuple | None = None,
) -> torch.Tensor:
    """Launch K1, K2, K3 on prepared operands; returns ``out`` (the update, or z + update if accumulating).

    ``mix = (num_heads, head_norm, w_router, router_kind)`` runs the multi-head routed head mix
    in K3 (``pf_trimul_mhr_fwd``): head_norm and router_kind as ``MHR_HEAD_NORMS`` /
    ``MHR_ROUTER_KINDS`` codes, w_router [H, C] fp32 or None; ``ln_out_b`` may then be None
    (head_rms)."""
    _lib.require_device("fused_trimul", z, mask)
    if z.dim() != 4 or z.shape[1] != z.shape[2]:
        raise NotActive("fused_trimul", f"z must be [B, N, N, C], got {tuple(z.shape)}")
    B, N, _, C = z.shape
    if C not in TRIMUL_CHANNELS:
        raise NotActive("fused_trimul", f"C={C}: built for C in {TRIMUL_CHANNELS}")
    cdt = w_packed.dtype
    if z.dtype == torch.bfloat16 and cdt == torch.float32:
        raise NotActive("fused_trimul", "bf16 activations need bf16 GEMM operands")
    zc = z.contiguous()
    m = mask.to(torch.float32).contiguous()
    if m.shape != (B, N, N):
        raise NotActive("fused_trimul", f"mask must be [B, N, N], got {tuple(mask.shape)}")
    if out is None:
        if accumulate:
            raise ValueError("accumulate=True needs an explicit out tensor")
        out = torch.empty_like(zc)
    else:
        _lib.check_out("fused_trimul", out, zc)
    code_c = _lib.dtype_code(cdt)
    ws_bytes = _lib.lib().pf_trimul_workspace_bytes(B, N, C, code_c)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=z.device)
    args = (
        zc.data_ptr(), m.data_ptr(), _f32(ln_in_w).data_ptr(), _f32(ln_in_b).data_ptr(), float(eps_in),
        w_packed.data_ptr(), _f32(ln_out_w).data_ptr(), _lib.ptr(_f32(ln_out_b) if ln_out_b is not None else None),
        float(eps_out), w_out.data_ptr(), w_out_gate.data_ptr(), B, N, C, int(outgoing), _lib.dtype_code(z.dtype),
        code_c, out.data_ptr(), int(accumulate), ws.data_ptr(), ws_bytes,
    )  # fmt: skip
    if mix is None:
        _lib.call("pf_trimul_fwd", *args, _lib.stream_of(zc))
    else:
        heads, head_norm, w_router, router_kind = mix
        wr = _f32(w_router) if w_router is not None else None
        _lib.call("pf_trimul_mhr_fwd", *args, int(heads), int(head_norm), _lib.ptr(wr), int(router_kind),
                  _lib.stream_of(zc))  # fmt: skip
    return out


# MHR codes of the C-ABI (pf_trimul_mhr_*): head_norm and router kind.
MHR_HEAD_NORMS = {"channel": 0, "head_rms": 1, "head_ln": 2, "post_channel": 3}
MHR_ROUTER_KINDS = {"softmax": 0, "sigmoid": 1}


@inference_only("fused_trimul")
def fused_trimul(
    z: torch.Tensor,
    mask: torch.Tensor,
    outgoing: bool,
    norm_in: torch.nn.Module,
    w_gate: torch.Tensor,
    w_proj: torch.Tensor,
    norm_out: torch.nn.Module,
    w_out: torch.Tensor,
    w_out_gate: torch.Tensor,
) -> torch.Tensor:
    """Triangle multiply in three HIP launches; same arguments as the reference's.

    Reference: ``fused_trimul`` (``triton/fused_trimul.py:332-366``). ``w_gate`` and
    ``w_proj`` are ``[2C, C]`` in block order (rows ``[a; b]``, the module's
    ``_block_order``), ``w_out``/``w_out_gate`` are ``[C, C]``. Returns the update in
    z's dtype. GEMM operands are bf16 for bf16 z or under bf16 autocast, else fp32.
    """
    cdt = gemm_dtype_for(z)
    packed = pack_trimul_weights(w_proj, w_gate, cdt)
    return trimul_forward(
        z, mask, norm_in.weight, norm_in.bias, norm_in.eps, packed, norm_out.weight, norm_out.bias, norm_out.eps,
        cast_weight(w_out, cdt), cast_weight(w_out_gate, cdt), outgoing,
    )  # fmt: skip


def _split_chunk(M: int, target: int = 4096) -> int:
    """Token chunk for a split-K weight gradient over M tokens: the divisor of M in
    [target / 2, 2 target] closest to ``target``, else ``target`` (the rows past the last
    whole chunk are then added by one more product)."""
    best = 0
    for d in range(target // 2, 2 * target + 1):
        if M % d == 0 and (best == 0 or abs(d - target) < abs(best - target)):
            best = d
    return best or target


def _weight_grad_tm(gy: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
    """``gy^T x`` (fp32, or fp64 for fp64 operands) for token-major gy [M, Co] and x [M, Ci]
    with M in the hundreds of thousands: the tokens split into chunks of a batched GEMM (one
    [Co, Ci] tile alone leaves the GPU idle; left operand a strided view, right operand
    contiguous), summed over chunks."""
    acc = torch.promote_types(gy.dtype, torch.float32)
    M = gy.shape[0]
    chunk = _split_chunk(M)
    S = M // chunk
    m0 = S * chunk
    g3 = gy[:m0].view(S, chunk, gy.shape[1]).transpose(1, 2)  # [S, Co, chunk]
    out = torch.bmm(g3, x[:m0].view(S, chunk, x.shape[1])).to(acc).sum(0)
    if m0 < M:
        out += (gy[m0:].t() @ x[m0:]).to(acc)
    return out


class _TokenLinear(torch.autograd.Function):
    """``x W^T`` over many tokens; the weight gradient runs split over token chunks."""

    @staticmethod
    def forward(ctx, x, w):
        ctx.save_for_backward(x, w)
        return torch.nn.functional.linear(x, w)

    @staticmethod
    def backward(ctx, gy):
        x, w = ctx.saved_tensors
        gy = gy.to(x.dtype).contiguous()
        gx = gw = None
        if ctx.needs_input_grad[0]:
            gx = gy @ w
        if ctx.needs_input_grad[1]:
            Ci = x.shape[-1]
            gw = _weight_grad_tm(gy.view(-1, gy.shape[-1]), x.view(-1, Ci)).to(w.dtype)
        return gx, gw


# Below this many tokens a linear's weight gradient is one library GEMM.
SPLIT_K_TOKENS = 32768


def token_linear(x: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """``F.linear(x, weight)`` (no bias) for the training path. Over a pair's tokens
    (``B N^2`` of them) the weight gradient is a GEMM with a reduction dimension in the
    hundreds of thousands and an output of a few hundred rows, which a single library call
    runs on a handful of workgroups; here it runs split over token chunks. Under autocast the
    operands are cast as autocast would cast them, so the numerics are the stock linear's."""
    M = x.numel() // x.shape[-1]
    if not torch.is_grad_enabled() or M < SPLIT_K_TOKENS or not (x.requires_grad or weight.requires_grad):
        return torch.nn.functional.linear(x, weight)
    if torch.is_autocast_enabled("cuda"):
        dt = torch.get_autocast_dtype("cuda")
        x, weight = x.to(dt), weight.to(dt)
    with torch.autocast("cuda", enabled=False):
        return _TokenLinear.apply(x.contiguous(), weight)


class FusedTriMulFunction(torch.autograd.Function):
    """Trainable triangle multiply after the input LayerNorm (``FusedTriMulFunction``,
    ``triton/fused_trimul.py:285-330``); same ``apply`` arguments.

    ``apply(x, mask, w_gate, w_proj, ln_out_w, ln_out_b, w_out, w_out_gate, eps, outgoing)``:
    x [B, N, N, C] is ``norm_left(z)`` (its LayerNorm stays in autograd), ``w_gate`` /
    ``w_proj`` [2C, C] in block order (rows [a; b]). The forward runs the generic K1 and K3
    without the input LayerNorm and K2, and keeps the planes and the contraction; the
    backward runs ``pf_trimul_output_vjp``, the contraction's cotangents ``dP = dX Q``,
    ``dQ = dX^T P`` and the weight gradients as library GEMMs, then ``pf_trimul_project_vjp``.
    GEMM operands are bf16 for bf16 x or under bf16 autocast (the reference's regime), fp32
    otherwise. Returns gradients for x, w_gate, w_proj, ln_out_w, ln_out_b, w_out, w_out_gate.

    Two trailing arguments run the multi-head routed variant (``ops.py:476-545``):
    ``w_router`` [H, C] (or None) and ``mix = (num_heads, head_norm, router_kind)`` as
    ``MHR_HEAD_NORMS`` / ``MHR_ROUTER_KINDS`` codes; ``ln_out_b`` may then be None (head_rms).
    The forward and the output VJP run ``pf_trimul_mhr_train_fwd`` / ``pf_trimul_mhr_output_vjp``
    (which also adds the router's share ``d_r Wr`` of x's cotangent, d_r the router logits'
    cotangent); ``pf_trimul_mhr_router_wgrad`` forms Wr's gradient ``d_r^T x``.
    """

    @staticmethod
    def forward(ctx, x, mask, w_gate, w_proj, ln_out_w, ln_out_b, w_out, w_out_gate, eps, outgoing, w_router=None,
                mix=None):  # fmt: skip
        _lib.require_device("FusedTriMulFunction", x, mask)
        if x.dim() != 4 or x.shape[1] != x.shape[2]:
            raise NotActive("FusedTriMulFunction", f"x must be [B, N, N, C], got {tuple(x.shape)}")
        B, N, _, C = x.shape
        if C not in TRIMUL_CHANNELS:
            raise NotActive("FusedTriMulFunction", f"C={C}: built for C in {TRIMUL_CHANNELS}")
        cdt = gemm_dtype_for(x)
        xc = x.detach().contiguous()
        if xc.dtype not in (torch.float32, torch.bfloat16) or (xc.dtype == torch.bfloat16 and cdt == torch.float32):
            raise NotActive("FusedTriMulFunction", f"x dtype {xc.dtype}")
        m = mask.detach().to(torch.float32).contiguous()
        wp, wg = w_proj.detach().contiguous(), w_gate.detach().to(w_proj.dtype).contiguous()
        w4 = torch.empty((4 * C, C), dtype=cdt, device=x.device)
        _lib.call(
            "pf_trimul_train_pack_weights", wp.data_ptr(), wg.data_ptr(), _lib.dtype_code(wp.dtype), w4.data_ptr(), C,
            _lib.dtype_code(cdt), _lib.stream_of(xc),
        )  # fmt: skip
        wo, wog = cast_weight(w_out, cdt), cast_weight(w_out_gate, cdt)
        lnow = _f32(ln_out_w)
        lnob = _f32(ln_out_b) if ln_out_b is not None else None
        wr = _f32(w_router) if w_router is not None else None
        nbytes = _lib.lib().pf_trimul_workspace_bytes(B, N, C, _lib.dtype_code(cdt))
        planes = torch.empty(nbytes, dtype=torch.uint8, device=x.device)
        out = torch.empty_like(xc)
        kernel_census.record("TriangleMul", "hip_trimul_grad")
        args = (
            xc.data_ptr(), m.data_ptr(), w4.data_ptr(), lnow.data_ptr(), _lib.ptr(lnob), float(eps), wo.data_ptr(),
            wog.data_ptr(), B, N, C, int(bool(outgoing)), _lib.dtype_code(xc.dtype), _lib.dtype_code(cdt),
            planes.data_ptr(), nbytes, out.data_ptr(),
        )  # fmt: skip
        if mix is None:
            _lib.call("pf_trimul_train_fwd", *args, _lib.stream_of(xc))
        else:
            _lib.call("pf_trimul_mhr_train_fwd", *args, int(mix[0]), int(mix[1]), _lib.ptr(wr), int(mix[2]),
                      _lib.stream_of(xc))  # fmt: skip
        ctx.save_for_backward(xc, m, planes, w4, wo, wog, lnow, lnob, wr)
        ctx.eps, ctx.outgoing, ctx.cdt, ctx.mix = float(eps), bool(outgoing), cdt, mix
        ctx.dtypes = (
            x.dtype, w_gate.dtype, w_proj.dtype, ln_out_w.dtype, None if ln_out_b is None else ln_out_b.dtype,
            w_out.dtype, w_out_gate.dtype, None if w_router is None else w_router.dtype,
        )  # fmt: skip
        return out

    @staticmethod
    def backward(ctx, g):
        xc, m, planes, w4, wo, wog, lnow, lnob, wr = ctx.saved_tensors
        cdt, mix = ctx.cdt, ctx.mix
        B, N, _, C = xc.shape
        Np = -(-N // 128) * 128
        M = B * N * N
        dev = xc.device
        code_x, code_c = _lib.dtype_code(xc.dtype), _lib.dtype_code(cdt)
        stream = _lib.stream_of(xc)
        g = g.to(xc.dtype).contiguous()
        kernel_census.record("TriangleMul.backward", "hip_trimul_vjp")
        pl = planes.view(cdt).view(3, B * C, Np, Np)
        gp, gg = (torch.empty((M, C), dtype=cdt, device=dev) for _ in range(2))  # token-major
        xln = torch.empty((M, C), dtype=cdt, device=dev)
        dX = torch.empty((B * C, Np, Np), dtype=cdt, device=dev)
        gx = torch.empty((M, C), dtype=torch.float32, device=dev)
        dlnw, dlnb = (torch.empty(C, dtype=torch.float32, device=dev) for _ in range(2))
        ws_bytes = _lib.lib().pf_trimul_output_vjp_workspace_bytes(B, N, C, code_c)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
        wot, wogt = wo.t().contiguous(), wog.t().contiguous()
        args = (
            g.data_ptr(), pl[2].data_ptr(), xc.data_ptr(), lnow.data_ptr(), _lib.ptr(lnob), ctx.eps, wo.data_ptr(),
            wog.data_ptr(), wot.data_ptr(), wogt.data_ptr(), B, N, C, code_x, code_c, gp.data_ptr(), gg.data_ptr(),
            xln.data_ptr(), dX.data_ptr(), gx.data_ptr(), dlnw.data_ptr(), dlnb.data_ptr(), ws.data_ptr(), ws_bytes,
        )  # fmt: skip
        d_router = None
        if mix is None:
            _lib.call("pf_trimul_output_vjp", *args, stream)
        else:
            dr = None if wr is None else torch.empty((M, int(mix[0])), dtype=torch.float32, device=dev)
            _lib.call("pf_trimul_mhr_output_vjp", *args, int(mix[0]), int(mix[1]), _lib.ptr(wr), int(mix[2]),
                      _lib.ptr(dr), stream)  # fmt: skip
            if dr is not None:  # gx holds the router's share already; Wr's gradient dr^T x
                H = int(mix[0])
                d_router = torch.empty((H, C), dtype=torch.float32, device=dev)
                wb = _lib.lib().pf_trimul_mhr_router_wgrad_workspace_bytes(M, C, H)
                wws = torch.empty(wb, dtype=torch.uint8, device=dev)
                _lib.call("pf_trimul_mhr_router_wgrad", dr.data_ptr(), xc.data_ptr(), code_x, M, C, H,
                          d_router.data_ptr(), wws.data_ptr(), wb, stream)  # fmt: skip
        xb = xc.reshape(M, C).to(cdt)
        d_out = _weight_grad_tm(gp, xln)
        d_out_gate = _weight_grad_tm(gg, xb)
        del gp, gg, xln
        # X = P Q^T per channel plane: dP = dX Q = contract(dX, Q^T), dQ = dX^T P =
        # contract(dX^T, P^T), on the forward's contraction kernels.
        G = B * C
        dpl = torch.empty((2, G, Np, Np), dtype=cdt, device=dev)
        tp = torch.empty((G, Np, Np), dtype=cdt, device=dev)
        _lib.call("pf_planes_transpose", pl[1].data_ptr(), tp.data_ptr(), G, Np, code_c, stream)
        _lib.call("pf_planes_contract", dX.data_ptr(), tp.data_ptr(), dpl[0].data_ptr(), G, Np, code_c, stream)
        _lib.call("pf_planes_transpose", pl[0].data_ptr(), tp.data_ptr(), G, Np, code_c, stream)
        dXt = torch.empty_like(dX)
        _lib.call("pf_planes_transpose", dX.data_ptr(), dXt.data_ptr(), G, Np, code_c, stream)
        del dX
        _lib.call("pf_planes_contract", dXt.data_ptr(), tp.data_ptr(), dpl[1].data_ptr(), G, Np, code_c, stream)
        del dXt, tp
        gpg = torch.empty((M, 4 * C), dtype=cdt, device=dev)  # token-major, the kernel's walk order
        xw = None if ctx.outgoing else torch.empty((M, C), dtype=cdt, device=dev)  # x in that order
        dx = torch.empty_like(xc)
        w4t = w4.t().contiguous()
        _lib.call(
            "pf_trimul_project_vjp", dpl.data_ptr(), xc.data_ptr(), m.data_ptr(), w4.data_ptr(), w4t.data_ptr(),
            gx.data_ptr(), B, N, C, int(ctx.outgoing), code_x, code_c, gpg.data_ptr(), _lib.ptr(xw), dx.data_ptr(),
            stream,
        )  # fmt: skip
        del dpl, gx
        cb = 32 if (cdt == torch.bfloat16 and C == 128) else 16  # channel blocks of the packed rows
        dw4 = _weight_grad_tm(gpg, xb if xw is None else xw).view(C // cb, 4, cb, C)  # rows 4 cb j + cb kind + r
        d_proj = torch.cat([dw4[:, 0].reshape(C, C), dw4[:, 2].reshape(C, C)])
        d_gate = torch.cat([dw4[:, 1].reshape(C, C), dw4[:, 3].reshape(C, C)])
        dt = ctx.dtypes
        return (dx.to(dt[0]), None, d_gate.to(dt[1]), d_proj.to(dt[2]), dlnw.to(dt[3]),
                None if dt[4] is None else dlnb.to(dt[4]), d_out.to(dt[5]), d_out_gate.to(dt[6]), None, None,
                None if d_router is None else d_router.to(dt[7]), None)  # fmt: skip


# ---------------------------------------------------------------- triangle attention


def _workspace(nbytes: int, device) -> torch.Tensor:
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)


def pack_grid_attn_weights(to_q, to_k, to_v, to_g, pair_bias, dtype: torch.dtype) -> torch.Tensor:
    """``[4C + 16, C]`` operand: rows to_q | to_k | to_v | to_g | pair_bias (H rows) | zeros."""
    C = to_q.shape[1]
    H = pair_bias.shape[0]
    pad = torch.zeros(16 - H, C, dtype=to_q.dtype, device=to_q.device)
    w = torch.cat([t.detach() for t in (to_q, to_k, to_v, to_g, pair_bias)] + [pad], dim=0)
    return cast_weight(w, dtype)


# Outer-product checks of pair masks: (weak reference to the mask, its in-place version,
# key mask or None) for the last few masks, so a trunk that passes one mask to every block
# checks it (and synchronises its stream) once.
_OUTER_SEEN: list = []


def outer_key_mask(mask: torch.Tensor) -> torch.Tensor | None:
    """For an fp32 contiguous pair mask [B, N, N] that is the outer product of its diagonal
    with values in {0, 1} (the trunk's ``seq_mask x seq_mask``, ``featurizer.py:520``), the
    diagonal's additive key mask ``1e9 (m[k][k] - 1)`` [B, N]; None for any other mask
    (``pf_pair_mask_outer``). Cached per tensor object and version; the first check of a
    mask reads the result back from the device."""
    for ref, ver, km in _OUTER_SEEN:
        if ref() is mask and ver == mask._version:
            return km
    B, N, _ = mask.shape
    flag = torch.empty(1, dtype=torch.int32, device=mask.device)
    km = torch.empty((B, N), dtype=torch.float32, device=mask.device)
    _lib.call("pf_pair_mask_outer", mask.data_ptr(), B, N, flag.data_ptr(), km.data_ptr(), _lib.stream_of(mask))
    km = km if bool(flag.item()) else None
    live = [e for e in _OUTER_SEEN if e[0]() is not None][-7:]
    _OUTER_SEEN[:] = live + [(weakref.ref(mask), mask._version, km)]
    return km


def pair_mask_is_outer(mask: torch.Tensor) -> bool:
    """Whether ``outer_key_mask(mask)`` applies."""
    return outer_key_mask(mask) is not None


def grid_attention_forward(
    z: torch.Tensor,
    mask: torch.Tensor,
    ln_w: torch.Tensor,
    ln_b: torch.Tensor,
    eps: float,
    w_packed: torch.Tensor,
    w_out: torch.Tensor,
    transpose: bool,
    num_heads: int = 4,
    out: torch.Tensor | None = None,
    accumulate: bool = False,
    mask_outer: bool | None = None,
) -> torch.Tensor:
    """GridSelfAttention on prepared operands (``attention.py:167-269``); returns ``out``.

    ``mask_outer`` selects the kernel path for the mask: True when the mask is the outer
    product of its binary diagonal (checked; the key mask then lives in the pair bias),
    False for the per-line key masks, None for the first when it applies
    (``outer_key_mask``). Both give the same result."""
    _lib.require_device("GridSelfAttention", z, mask)
    if z.dim() != 4 or z.shape[1] != z.shape[2]:
        raise NotActive("GridSelfAttention", f"z must be [B, N, N, C], got {tuple(z.shape)}")
    B, N, _, C = z.shape
    fused = C == 128 and num_heads == 4
    code_c = _lib.dtype_code(w_packed.dtype)
    if not fused and _lib.lib().pf_grid_attn_workspace_bytes(1, 1, C, num_heads, code_c) == 0:
        raise NotActive(
            "GridSelfAttention", f"C={C}, heads={num_heads}: built for C=128 with 4 heads, or C a multiple of 32 with "
            "1-16 heads of dimension max(C/H, 16) <= 32",
        )  # fmt: skip
    cdt = w_packed.dtype
    if z.dtype == torch.bfloat16 and cdt == torch.float32:
        raise NotActive("GridSelfAttention", "bf16 activations need bf16 GEMM operands")
    zc = z.contiguous()
    m = mask.to(torch.float32).contiguous()
    if m.shape != (B, N, N):
        raise NotActive("GridSelfAttention", f"mask must be [B, N, N], got {tuple(mask.shape)}")
    if out is None:
        if accumulate:
            raise ValueError("accumulate=True needs an explicit out tensor")
        out = torch.empty_like(zc)
    else:
        _lib.check_out("GridSelfAttention", out, zc)
    # the outer-product path belongs to the fused 128-channel kernels and the 256-channel,
    # 8-head bf16 path
    folds = fused or (C == 256 and num_heads == 8 and cdt == torch.bfloat16)
    km = outer_key_mask(m) if folds and (mask_outer is None or mask_outer) else None
    if mask_outer and km is None:
        raise NotActive("GridSelfAttention", "mask_outer=True needs a mask that is the outer product of its diagonal")
    ws_bytes = _lib.lib().pf_grid_attn_workspace_bytes(B, N, C, num_heads, code_c)
    ws = _workspace(ws_bytes, z.device)
    _lib.call(
        "pf_grid_attn_fwd", zc.data_ptr(), m.data_ptr(), _f32(ln_w).data_ptr(), _f32(ln_b).data_ptr(), float(eps),
        w_packed.data_ptr(), w_out.data_ptr(), B, N, C, num_heads, int(transpose), _lib.dtype_code(z.dtype), code_c,
        out.data_ptr(), int(accumulate), 0 if km is None else km.data_ptr(), ws.data_ptr(), ws_bytes,
        _lib.stream_of(zc),
    )  # fmt: skip
    _lib.note_redo("pf_grid_attn_redo_flags", ws, B, N, C, num_heads, code_c)
    return out


# ---------------------------------------------------------------- transitions


def pair_transition_forward(
    x: torch.Tensor,
    ln_w: torch.Tensor,
    ln_b: torch.Tensor,
    eps: float,
    w1: torch.Tensor,
    w2: torch.Tensor,
    out: torch.Tensor | None = None,
    accumulate: bool = False,
    s2p: tuple | None = None,
) -> tuple[torch.Tensor, torch.Tensor | None]:
    """Fused pair transition (C=128, factor 4; or C=256, factor 4 with bf16 z and GEMM
    operands, without the single_to_pair epilogue); optionally also the single_to_pair logits.

    ``s2p = (ln_w, ln_b, eps, w_s2p)`` computes ``pair_logits [B, 16, N, N]`` (fp32) from the
    updated rows (``evoformer.py:322-328``). Returns ``(out, pair_logits or None)``.
    """
    _lib.require_device("FusedTransitionBlock", x)
    C = x.shape[-1]
    factor = w1.shape[0] // (2 * C)
    xc = x.contiguous()
    if out is None:
        if accumulate:
            raise ValueError("accumulate=True needs an explicit out tensor")
        out = torch.empty_like(xc)
    else:
        _lib.check_out("FusedTransitionBlock", out, xc)
    M = xc.numel() // C
    logits = None
    s2p_args = [None, None, 0.0, None, None, 0]
    if s2p is not None:
        if x.dim() != 4:
            raise NotActive("single_to_pair", "fused single_to_pair needs x as [B, N, N, C]")
        B, N = x.shape[0], x.shape[1]
        logits = torch.empty((B, 16, N, N), dtype=torch.float32, device=x.device)
        sw, sb, seps, ws2p = s2p
        s2p_args = [_f32(sw).data_ptr(), _f32(sb).data_ptr(), float(seps), ws2p.data_ptr(), logits.data_ptr(), N * N]
    _lib.call(
        "pf_pair_transition_fwd", xc.data_ptr(), _f32(ln_w).data_ptr(), _f32(ln_b).data_ptr(), float(eps),
        w1.data_ptr(), w2.data_ptr(), M, C, factor, _lib.dtype_code(x.dtype), _lib.dtype_code(w1.dtype),
        out.data_ptr(), int(accumulate), *s2p_args, _lib.stream_of(xc),
    )  # fmt: skip
    return out, logits


def single_to_pair(z: torch.Tensor, ln_w, ln_b, eps: float, w_s2p: torch.Tensor) -> torch.Tensor:
    """``single_to_pair(single_to_pair_norm(z)).movedim(-1, -3)`` -> [B, H, N, N] fp32."""
    _lib.require_device("single_to_pair", z)
    B, N, _, C = z.shape
    H = w_s2p.shape[0]
    zc = z.contiguous()
    logits = torch.empty((B, H, N, N), dtype=torch.float32, device=z.device)
    _lib.call(
        "pf_single_to_pair_fwd", zc.data_ptr(), _f32(ln_w).data_ptr(), _f32(ln_b).data_ptr(), float(eps),
        w_s2p.data_ptr(), zc.numel() // C, C, H, N * N, _lib.dtype_code(z.dtype), _lib.dtype_code(w_s2p.dtype),
        logits.data_ptr(), _lib.stream_of(zc),
    )  # fmt: skip
    return logits


def transition_forward(
    x: torch.Tensor,
    ln_w: torch.Tensor,
    ln_b: torch.Tensor,
    eps: float,
    w1: torch.Tensor,
    w2: torch.Tensor,
    out: torch.Tensor | None = None,
    accumulate: bool = False,
) -> torch.Tensor:
    """Generic TransitionBlock forward for any C (``primitives.py:193-251``)."""
    _lib.require_device("TransitionBlock", x)
    C = x.shape[-1]
    factor = w1.shape[0] // (2 * C)
    xc = x.contiguous()
    if out is None:
        if accumulate:
            raise ValueError("accumulate=True needs an explicit out tensor")
        out = torch.empty_like(xc)
    else:
        _lib.check_out("TransitionBlock", out, xc)
    M = xc.numel() // C
    code_c = _lib.dtype_code(w1.dtype)
    ws_bytes = _lib.lib().pf_transition_workspace_bytes(M, C, factor, code_c)
    ws = _workspace(ws_bytes, x.device)
    _lib.call(
        "pf_transition_fwd", xc.data_ptr(), _f32(ln_w).data_ptr(), _f32(ln_b).data_ptr(), float(eps), w1.data_ptr(),
        w2.data_ptr(), M, C, factor, _lib.dtype_code(x.dtype), code_c, out.data_ptr(), int(accumulate),
        ws.data_ptr(), ws_bytes, _lib.stream_of(xc),
    )  # fmt: skip
    return out


def recycle_embed_(
    out: torch.Tensor, prev: torch.Tensor, ln_w: torch.Tensor, ln_b: torch.Tensor, eps: float, w: torch.Tensor
) -> torch.Tensor:
    """``out += LN(prev) w^T`` in place (the recycling embedding, ``evoformer.py:520-526``,
    ``:558-561``); ``w`` [C, C] in the GEMM operand dtype."""
    _lib.require_device("recycle_embed", prev, out)
    C = prev.shape[-1]
    _lib.check_out("recycle_embed", out, prev)
    if tuple(w.shape) != (C, C):
        raise NotActive("recycle_embed", f"weight shape {tuple(w.shape)} is not ({C}, {C})")
    prev_c = prev.contiguous()
    M = prev_c.numel() // C
    code_c = _lib.dtype_code(w.dtype)
    ws_bytes = _lib.lib().pf_recycle_embed_workspace_bytes(M, C, code_c)
    ws = _workspace(ws_bytes, prev.device)
    _lib.call(
        "pf_recycle_embed_fwd", prev_c.data_ptr(), _f32(ln_w).data_ptr(), _f32(ln_b).data_ptr(), float(eps),
        w.data_ptr(), M, C, _lib.dtype_code(prev.dtype), code_c, out.data_ptr(), ws.data_ptr(), ws_bytes,
        _lib.stream_of(prev_c),
    )  # fmt: skip
    return out


# ---------------------------------------------------------------- MSA stack


def outer_product_mean_forward(
    msa: torch.Tensor,
    mask: torch.Tensor,
    ln_w: torch.Tensor,
    ln_b: torch.Tensor,
    eps: float,
    w_ab: torch.Tensor,
    w_out: torch.Tensor,
    b_out: torch.Tensor,
    out: torch.Tensor | None = None,
    accumulate: bool = False,
) -> torch.Tensor:
    """OuterProductMean on prepared operands (``ops.py:683-785``): msa [B, S, N, Cm], mask
    [B, S, N]; returns (or adds into ``out``) the [B, N, N, Cz] update."""
    _lib.require_device("OuterProductMean", msa, mask)
    if msa.dim() != 4:
        raise NotActive("OuterProductMean", f"msa must be [B, S, N, C], got {tuple(msa.shape)}")
    B, S, N, Cm = msa.shape
    CH = w_ab.shape[0] // 2
    Cz = w_out.shape[0]
    mc = msa.contiguous()
    m = mask.to(torch.float32).contiguous()
    if m.shape != (B, S, N):
        raise NotActive("OuterProductMean", f"mask must be [B, S, N], got {tuple(mask.shape)}")
    if out is None:
        if accumulate:
            raise ValueError("accumulate=True needs an explicit out tensor")
        out = torch.empty((B, N, N, Cz), dtype=msa.dtype, device=msa.device)
    else:
        _lib.check_out("OuterProductMean", out, mc, shape=(B, N, N, Cz))
    code_c = _lib.dtype_code(w_ab.dtype)
    ws_bytes = _lib.lib().pf_outer_product_mean_workspace_bytes(B, S, N, Cm, CH, Cz, code_c)
    ws = _workspace(ws_bytes, msa.device)
    _lib.call(
        "pf_outer_product_mean_fwd", mc.data_ptr(), m.data_ptr(), _f32(ln_w).data_ptr(), _f32(ln_b).data_ptr(),
        float(eps), w_ab.data_ptr(), w_out.data_ptr(), _f32(b_out).data_ptr(), B, S, N, Cm, CH, Cz,
        _lib.dtype_code(msa.dtype), _lib.dtype_code(out.dtype), code_c, out.data_ptr(), int(accumulate),
        ws.data_ptr(), ws_bytes, _lib.stream_of(mc),
    )  # fmt: skip
    return out


def msa_pair_avg_forward(
    msa: torch.Tensor,
    mask: torch.Tensor,
    pair: torch.Tensor,
    ln_w: torch.Tensor,
    ln_b: torch.Tensor,
    eps: float,
    pair_ln_w: torch.Tensor,
    pair_ln_b: torch.Tensor,
    pair_eps: float,
    w_logits16: torch.Tensor,
    w_vg: torch.Tensor,
    w_out: torch.Tensor,
    num_heads: int,
    out: torch.Tensor | None = None,
    accumulate: bool = False,
) -> torch.Tensor:
    """MSAAttention (pair-weighted averaging, ``attention.py:272-341``) on prepared operands:
    msa [B, S, N, Cm], mask [B, S, N], pair [B, N, N, Cz] (msa's dtype); returns (or adds into
    ``out``) the [B, S, N, Cm] update."""
    _lib.require_device("MSAAttention", msa, mask, pair)
    if msa.dim() != 4 or pair.dim() != 4:
        raise NotActive("MSAAttention", f"msa [B, S, N, C] and pair [B, N, N, C] expected, got {tuple(msa.shape)}")
    B, S, N, Cm = msa.shape
    Cz = pair.shape[-1]
    if pair.shape[:3] != (B, N, N) or pair.dtype != msa.dtype:
        raise NotActive("MSAAttention", f"pair {tuple(pair.shape)} {pair.dtype} does not match msa {tuple(msa.shape)}")
    mc, pc = msa.contiguous(), pair.contiguous()
    m = mask.to(torch.float32).contiguous()
    if out is None:
        if accumulate:
            raise ValueError("accumulate=True needs an explicit out tensor")
        out = torch.empty_like(mc)
    else:
        _lib.check_out("MSAAttention", out, mc)
    code_c = _lib.dtype_code(w_vg.dtype)
    ws_bytes = _lib.lib().pf_msa_pair_avg_workspace_bytes(B, S, N, Cm, Cz, num_heads, code_c)
    ws = _workspace(ws_bytes, msa.device)
    _lib.call(
        "pf_msa_pair_avg_fwd", mc.data_ptr(), m.data_ptr(), pc.data_ptr(), _f32(ln_w).data_ptr(),
        _f32(ln_b).data_ptr(), float(eps), _f32(pair_ln_w).data_ptr(), _f32(pair_ln_b).data_ptr(), float(pair_eps),
        w_logits16.data_ptr(), w_vg.data_ptr(), w_out.data_ptr(), B, S, N, Cm, Cz, num_heads,
        _lib.dtype_code(msa.dtype), code_c, out.data_ptr(), int(accumulate), ws.data_ptr(), ws_bytes,
        _lib.stream_of(mc),
    )  # fmt: skip
    return out


# ---------------------------------------------------------------- single attention


def single_attention_forward(
    s: torch.Tensor,
    seq_mask: torch.Tensor,
    pair_logits: torch.Tensor,
    ln_w: torch.Tensor,
    ln_b: torch.Tensor,
    eps: float,
    w_qkvg: torch.Tensor,
    q_bias: torch.Tensor,
    w_out: torch.Tensor,
    num_heads: int,
    out: torch.Tensor | None = None,
    accumulate: bool = False,
) -> torch.Tensor:
    """SingleAttention forward (``attention.py:415-452``) on prepared operands."""
    _lib.require_device("SingleAttention", s, seq_mask, pair_logits)
    B, N, C = s.shape
    sc = s.contiguous()
    m = seq_mask.to(torch.float32).contiguous()
    pl = pair_logits.to(torch.float32).contiguous()
    if pl.shape != (B, num_heads, N, N):
        raise NotActive("SingleAttention", f"pair_logits must be [B, H, N, N], got {tuple(pl.shape)}")
    if out is None:
        if accumulate:
            raise ValueError("accumulate=True needs an explicit out tensor")
        out = torch.empty_like(sc)
    else:
        _lib.check_out("SingleAttention", out, sc)
    code_c = _lib.dtype_code(w_qkvg.dtype)
    ws_bytes = _lib.lib().pf_single_attn_workspace_bytes(B, N, C, num_heads, code_c)
    ws = _workspace(ws_bytes, s.device)
    _lib.call(
        "pf_single_attn_fwd", sc.data_ptr(), m.data_ptr(), pl.data_ptr(), _f32(ln_w).data_ptr(),
        _f32(ln_b).data_ptr(), float(eps), w_qkvg.data_ptr(), _f32(q_bias).data_ptr(), w_out.data_ptr(), B, N, C,
        num_heads, _lib.dtype_code(s.dtype), code_c, out.data_ptr(), int(accumulate), ws.data_ptr(), ws_bytes,
        _lib.stream_of(sc),
    )  # fmt: skip
    return out
