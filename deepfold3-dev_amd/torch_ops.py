"""The HIP kernels as registered PyTorch operators (namespace ``deepfold3_amd``).

The functional wrappers in ``kernels`` and ``fused`` call the C ABI through ctypes, which
PyTorch's tracers cannot see into. The operators below wrap the same entry points with
``torch.library.custom_op`` and a fake (shape-only) implementation each, so code built on
them can be traced by ``torch.compile`` / ``torch.export`` (the op stays one opaque node that
runs the HIP kernel) and checked under ``FakeTensorMode`` without a GPU. Each operator
allocates fresh outputs (no argument is mutated) and launches on the current stream.

Operators (argument meaning as in the function they wrap):

- ``layer_norm(x, weight, bias, eps)``: ``kernels.layer_norm`` (LayerNorm over the last dim,
  ``primitives.py:90-115`` of the reference).
- ``ln_transpose(x, weight, bias, eps, do_transpose)``: ``kernels.ln_transpose``
  (``triton/layernorm_transpose.py:269-316``).
- ``swiglu(x)``: SwiGLU of ``[..., 2D]`` into ``[..., D]`` (``triton/swiglu.py:192-200``).
- ``trimul(z, mask, ln_in_w, ln_in_b, eps_in, w_packed, ln_out_w, ln_out_b, eps_out, w_out,
  w_out_gate, outgoing)``: ``kernels.trimul_forward`` on K1-packed weights
  (``triton/fused_trimul.py:332-366``).
- ``evo_attention(q, k, v, res_mask, pair_bias, zero_masked_rows)``: the flash kernel in the
  reference kernel's layout, q/k/v ``[B, S, H, N, 32]``, res_mask ``[B, S, N]`` and pair_bias
  ``[B, H, N, N]`` fp32 (``triton/evo_attention.py:1198-1292``); differentiable through
  ``evo_attention_backward`` (the HIP backward, same masked-row rule) registered as its
  autograd formula. Shapes, dtypes and devices are checked before any launch (and shapes and
  dtypes in the fake implementations too): the kernels read these buffers with the sizes q
  implies, so a broadcast mask or a bf16 bias would be read out of bounds.
"""

from __future__ import annotations

import torch

from . import fused, kernels
from .inference_guard import NotActive

NS = "deepfold3_amd"


@torch.library.custom_op(f"{NS}::layer_norm", mutates_args=())
def layer_norm(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor, eps: float) -> torch.Tensor:
    return kernels.layer_norm(x, weight, bias, eps)


@layer_norm.register_fake
def _(x, weight, bias, eps):
    return torch.empty_like(x, memory_format=torch.contiguous_format)


@torch.library.custom_op(f"{NS}::ln_transpose", mutates_args=())
def ln_transpose(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor, eps: float, do_transpose: bool) -> torch.Tensor:
    return kernels.ln_transpose(x, weight, bias, eps, do_transpose)


@ln_transpose.register_fake
def _(x, weight, bias, eps, do_transpose):
    B, N1, N2, C = x.shape
    return x.new_empty((B, N2, N1, C) if do_transpose else (B, N1, N2, C))


@torch.library.custom_op(f"{NS}::swiglu", mutates_args=())
def swiglu(x: torch.Tensor) -> torch.Tensor:
    with torch.no_grad():
        return kernels.SwiGLUFunction.apply(x)


@swiglu.register_fake
def _(x):
    return x.new_empty(x.shape[:-1] + (x.shape[-1] // 2,))


@torch.library.custom_op(f"{NS}::trimul", mutates_args=())
def trimul(
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
) -> torch.Tensor:
    return kernels.trimul_forward(
        z, mask, ln_in_w, ln_in_b, eps_in, w_packed, ln_out_w, ln_out_b, eps_out, w_out, w_out_gate, outgoing
    )


@trimul.register_fake
def _(z, mask, ln_in_w, ln_in_b, eps_in, w_packed, ln_out_w, ln_out_b, eps_out, w_out, w_out_gate, outgoing):
    return torch.empty_like(z, memory_format=torch.contiguous_format)


_ATTN_DTYPES = (torch.float32, torch.bfloat16)


def _check_evo(q, k, v, res_mask, pair_bias, grad_out=None) -> None:
    """Refuse (``NotActive``) operands the kernels would misread, before anything touches a
    device: q, k, v ``[B, S, H, N, 32]`` of one dtype (fp32 or bf16) and shape, res_mask
    ``[B, S, N]`` and pair_bias ``[B, H, N, N]`` fp32 (the kernel layout; the reference's
    ``[B, S, 1, 1, N]`` mask and ``[B, 1, H, N, N]`` bias go through ``fused._EvoformerAttention``),
    grad_out shaped like q."""
    site = "evo_attention"
    if q.dim() != 5:
        raise NotActive(site, f"q must be [B, S, H, N, D], got shape {tuple(q.shape)}")
    B, S, H, N, D = q.shape
    if q.dtype not in _ATTN_DTYPES:
        raise NotActive(site, f"q dtype {q.dtype}: fp32 or bf16 only")
    for name, t in (("k", k), ("v", v)) + ((("grad_out", grad_out),) if grad_out is not None else ()):
        if tuple(t.shape) != tuple(q.shape):
            raise NotActive(site, f"{name} shape {tuple(t.shape)} != q shape {tuple(q.shape)}")
        if name != "grad_out" and t.dtype != q.dtype:
            raise NotActive(site, f"{name} dtype {t.dtype} != q dtype {q.dtype}")
    if D != 32:
        raise NotActive(site, f"D={D}: built for D=32")
    if res_mask.dtype != torch.float32 or tuple(res_mask.shape) != (B, S, N):
        raise NotActive(site, f"res_mask must be fp32 [B, S, N] = {[B, S, N]}, got {res_mask.dtype} "
                        f"{tuple(res_mask.shape)}")  # fmt: skip
    if pair_bias.dtype != torch.float32 or tuple(pair_bias.shape) != (B, H, N, N):
        raise NotActive(site, f"pair_bias must be fp32 [B, H, N, N] = {[B, H, N, N]}, got {pair_bias.dtype} "
                        f"{tuple(pair_bias.shape)}")  # fmt: skip


def _check_evo_device(*ts) -> None:
    from . import _lib

    _lib.require_device("evo_attention", *ts)
    dev = ts[0].device
    if any(t.device != dev for t in ts):
        raise NotActive("evo_attention", "all operands must be on one device")


@torch.library.custom_op(f"{NS}::evo_attention", mutates_args=())
def evo_attention(
    q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, res_mask: torch.Tensor, pair_bias: torch.Tensor,
    zero_masked_rows: bool,
) -> torch.Tensor:  # fmt: skip
    _check_evo(q, k, v, res_mask, pair_bias)
    _check_evo_device(q, k, v, res_mask, pair_bias)
    return fused._evo_fwd(q.contiguous(), k.contiguous(), v.contiguous(), res_mask.contiguous(),
                          pair_bias.contiguous(), zero_masked_rows)  # fmt: skip


@evo_attention.register_fake
def _(q, k, v, res_mask, pair_bias, zero_masked_rows):
    _check_evo(q, k, v, res_mask, pair_bias)
    return torch.empty_like(q, memory_format=torch.contiguous_format)


@torch.library.custom_op(f"{NS}::evo_attention_backward", mutates_args=())
def evo_attention_backward(
    q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, res_mask: torch.Tensor, pair_bias: torch.Tensor,
    grad_out: torch.Tensor, zero_masked_rows: bool,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:  # fmt: skip
    _check_evo(q, k, v, res_mask, pair_bias, grad_out)
    _check_evo_device(q, k, v, res_mask, pair_bias, grad_out)
    return fused._evo_bwd(q.contiguous(), k.contiguous(), v.contiguous(), res_mask.contiguous(),
                          pair_bias.contiguous(), grad_out, zero_masked_rows)  # fmt: skip


@evo_attention_backward.register_fake
def _(q, k, v, res_mask, pair_bias, grad_out, zero_masked_rows):
    _check_evo(q, k, v, res_mask, pair_bias, grad_out)
    like = lambda t: torch.empty_like(t, memory_format=torch.contiguous_format)  # noqa: E731
    B, S, H, N, D = q.shape
    return like(q), like(k), like(v), q.new_empty((B, H, N, N), dtype=torch.float32)


def _evo_setup(ctx, inputs, output):
    q, k, v, res_mask, pair_bias, zero_masked_rows = inputs
    ctx.zero_masked_rows = zero_masked_rows
    ctx.save_for_backward(q, k, v, res_mask, pair_bias)


def _evo_backward(ctx, grad_out):
    q, k, v, res_mask, pair_bias = ctx.saved_tensors
    dq, dk, dv, dpb = evo_attention_backward(q, k, v, res_mask, pair_bias, grad_out, ctx.zero_masked_rows)
    return dq, dk, dv, None, dpb, None


evo_attention.register_autograd(_evo_backward, setup_context=_evo_setup)

__all__ = ["NS", "layer_norm", "ln_transpose", "swiglu", "trimul", "evo_attention", "evo_attention_backward"]
