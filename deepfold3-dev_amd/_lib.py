"""ctypes binding of ``libpairformer_hip.so`` (the C ABI declared in include/pairformer_hip.h).

The library is built in-tree by ``__graft_entry__.build()`` (``make -C
deepfold3-dev_amd/csrc``). There is no fallback: if the library is missing or a
call fails, this raises. Tensors cross the boundary as raw device pointers;
the stream is torch's current HIP stream.
"""

from __future__ import annotations

import ctypes
import os
import re

import torch

from .inference_guard import NotActive

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libpairformer_hip.so")
HEADER_PATH = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "pairformer_hip.h")

PF_F32 = 0
PF_BF16 = 1

_vp, _i, _f, _sz, _l = ctypes.c_void_p, ctypes.c_int, ctypes.c_float, ctypes.c_size_t, ctypes.c_long

# name -> (restype, argtypes); mirrors include/pairformer_hip.h.
SIGNATURES: dict[str, tuple] = {
    "pf_version": (_i, []),
    "pf_last_error": (ctypes.c_char_p, []),
    "pf_last_error_code": (_i, []),
    "pf_kernel_timer_start": (_i, [ctypes.c_char_p]),
    "pf_kernel_timer_read": (_i, [ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_long)]),
    "pf_kernel_timer_stop": (_i, []),
    "pf_cast": (_i, [_vp, _i, _vp, _i, _sz, _vp]),
    "pf_add": (_i, [_vp, _i, _vp, _i, _vp, _sz, _vp]),
    "pf_dropout_mask": (_i, [_vp, _l, _f, ctypes.c_ulonglong, _vp]),
    "pf_dropout_add_fwd": (_i, [_vp, _i, _vp, _i, _vp, _l, _l, _l, _l, _i, _f, ctypes.c_ulonglong, _vp]),
    "pf_dropout_bwd": (_i, [_vp, _i, _vp, _i, _l, _l, _l, _l, _i, _f, ctypes.c_ulonglong, _vp]),
    "pf_layernorm_fwd": (_i, [_vp, _i, _vp, _vp, _f, _vp, ctypes.c_long, _i, _vp]),
    "pf_layernorm_bwd_workspace_bytes": (_sz, [ctypes.c_long, _i]),
    "pf_layernorm_bwd": (_i, [_vp, _vp, _i, _vp, _f, _vp, _vp, _vp, ctypes.c_long, _i, _vp, _sz, _vp]),
    "pf_layernorm_fwd_mixed": (_i, [_vp, _i, _vp, _vp, _f, _vp, _i, ctypes.c_long, _i, _vp]),
    "pf_layernorm_bwd_mixed": (_i, [_vp, _i, _vp, _i, _vp, _f, _vp, _vp, _vp, ctypes.c_long, _i, _vp, _sz, _vp]),
    "pf_ln_transpose_fwd": (_i, [_vp, _i, _vp, _vp, _f, _vp, _i, _i, _i, _i, _i, _vp]),
    "pf_trimul_workspace_bytes": (_sz, [_i, _i, _i, _i]),
    "pf_trimul_pack_weights": (_i, [_vp, _vp, _i, _vp, _i, _i, _vp]),
    "pf_trimul_train_pack_weights": (_i, [_vp, _vp, _i, _vp, _i, _i, _vp]),
    "pf_trimul_train_fwd": (_i, [_vp] * 3 + [_vp, _vp, _f, _vp, _vp] + [_i] * 6 + [_vp, _sz, _vp, _vp]),
    "pf_trimul_output_vjp_workspace_bytes": (_sz, [_i, _i, _i, _i]),
    "pf_trimul_output_vjp": (_i, [_vp] * 5 + [_f] + [_vp] * 4 + [_i] * 5 + [_vp] * 8 + [_sz, _vp]),
    "pf_trimul_project_vjp": (_i, [_vp] * 6 + [_i] * 6 + [_vp] * 4),
    "pf_planes_transpose": (_i, [_vp, _vp, _i, _i, _i, _vp]),
    "pf_planes_contract": (_i, [_vp, _vp, _vp, _i, _i, _i, _vp]),
    "pf_rms_residual_add": (_i, [_vp, _i, _vp, _i, _vp, _l, _i, _f, _f, _vp]),
    "pf_trimul_mhr_fwd": (
        _i,
        [_vp, _vp, _vp, _vp, _f, _vp, _vp, _vp, _f, _vp, _vp] + [_i] * 6 + [_vp, _i, _vp, _sz] + [_i, _i, _vp, _i, _vp],
    ),
    "pf_trimul_mhr_train_fwd": (
        _i, [_vp] * 3 + [_vp, _vp, _f, _vp, _vp] + [_i] * 6 + [_vp, _sz, _vp] + [_i, _i, _vp, _i, _vp],
    ),
    "pf_trimul_mhr_router_wgrad_workspace_bytes": (_sz, [_l, _i, _i]),
    "pf_trimul_mhr_router_wgrad": (_i, [_vp, _vp, _i, _l, _i, _i, _vp, _vp, _sz, _vp]),
    "pf_trimul_mhr_output_vjp": (
        _i, [_vp] * 5 + [_f] + [_vp] * 4 + [_i] * 5 + [_vp] * 8 + [_sz] + [_i, _i, _vp, _i, _vp, _vp],
    ),
    "pf_trimul_fwd": (
        _i,
        [_vp, _vp, _vp, _vp, _f, _vp, _vp, _vp, _f, _vp, _vp, _i, _i, _i, _i, _i, _i, _vp, _i, _vp, _sz, _vp],
    ),
    "pf_grid_attn_workspace_bytes": (_sz, [_i, _i, _i, _i, _i]),
    "pf_grid_attn_fwd": (
        _i,
        [_vp, _vp, _vp, _vp, _f, _vp, _vp, _i, _i, _i, _i, _i, _i, _i, _vp, _i, _vp, _vp, _sz, _vp],
    ),
    "pf_pair_transition_fwd": (
        _i,
        [_vp, _vp, _vp, _f, _vp, _vp, _l, _i, _i, _i, _i, _vp, _i, _vp, _vp, _f, _vp, _vp, _l, _vp],
    ),
    "pf_single_to_pair_fwd": (_i, [_vp, _vp, _vp, _f, _vp, _l, _i, _i, _l, _i, _i, _vp, _vp]),
    "pf_transition_workspace_bytes": (_sz, [_l, _i, _i, _i]),
    "pf_transition_fwd": (
        _i,
        [_vp, _vp, _vp, _f, _vp, _vp, _l, _i, _i, _i, _i, _vp, _i, _vp, _sz, _vp],
    ),
    "pf_recycle_embed_workspace_bytes": (_sz, [_l, _i, _i]),
    "pf_recycle_embed_fwd": (_i, [_vp, _vp, _vp, _f, _vp, _l, _i, _i, _i, _vp, _vp, _sz, _vp]),
    "pf_outer_product_mean_workspace_bytes": (_sz, [_i, _i, _i, _i, _i, _i, _i]),
    "pf_outer_product_mean_fwd": (
        _i,
        [_vp, _vp, _vp, _vp, _f, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _i, _i, _i, _vp, _i, _vp, _sz, _vp],
    ),
    "pf_msa_pair_avg_workspace_bytes": (_sz, [_i, _i, _i, _i, _i, _i, _i]),
    "pf_msa_pair_avg_fwd": (
        _i,
        [_vp, _vp, _vp, _vp, _vp, _f, _vp, _vp, _f, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _i, _i, _vp, _i, _vp, _sz,
         _vp],
    ),  # fmt: skip
    "pf_evo_attn_workspace_bytes": (_sz, [_i, _i, _i, _i, _i, _i]),
    "pf_evo_attn_fwd": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _i, _vp, _vp, _sz, _vp]),
    "pf_evo_attn_bwd_workspace_bytes": (_sz, [_i, _i, _i, _i, _i, _i]),
    "pf_evo_attn_bwd": (_i, [_vp] * 6 + [_i] * 6 + [_f, _i] + [_vp] * 5 + [_sz, _vp]),
    "pf_evo_attn_fwd_strided": (_i, [_vp] * 6 + [_i] * 7 + [_vp] * 4 + [_sz, _vp]),
    "pf_evo_attn_bwd_strided": (_i, [_vp] * 9 + [_i] * 6 + [_f] + [_vp] * 6 + [_sz, _vp]),
    "pf_pair_mask_outer": (_i, [_vp, _i, _i, _vp, _vp, _vp]),
    "pf_grid_attn_redo_flags": (_i, [_i, _i, _i, _i, _i, ctypes.POINTER(_sz), ctypes.POINTER(_sz)]),
    "pf_evo_attn_redo_flags": (_i, [_i, _i, _i, _i, _i, _i, ctypes.POINTER(_sz), ctypes.POINTER(_sz)]),
    "pf_pair_bias_fwd": (_i, [_vp, _i, _vp, _vp, _f, _vp, _i, _vp, _vp, _i, _i, _i, _vp]),
    "pf_layernorm_linear_workspace_bytes": (_sz, [_l, _i, _i]),
    "pf_layernorm_linear_fwd": (_i, [_vp, _i, _vp, _vp, _f, _vp, _vp, _l, _i, _i, _i, _vp, _vp, _sz, _vp]),
    "pf_swiglu_fwd": (_i, [_vp, _i, _vp, _l, _i, _vp]),
    "pf_swiglu_bwd": (_i, [_vp, _vp, _i, _vp, ctypes.c_long, _i, _vp]),
    "pf_single_attn_workspace_bytes": (_sz, [_i, _i, _i, _i, _i]),
    "pf_single_attn_fwd": (
        _i,
        [_vp, _vp, _vp, _vp, _vp, _f, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _vp, _i, _vp, _sz, _vp],
    ),
    "pf_single_attn_fwd_noalloc": (
        _i,
        [_vp, _vp, _vp, _vp, _vp, _f, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _vp, _i, _vp],
    ),
}

# Capacity of the library's static scratch array (PF_NOALLOC_SCRATCH_BYTES in the header).
NOALLOC_SCRATCH_BYTES = 32 << 20

_lib = None


class PFError(RuntimeError):
    """A C-ABI call returned a non-zero status."""

    def __init__(self, fn: str, code: int, msg: str):
        self.fn, self.code = fn, code
        super().__init__(f"{fn} failed with status {code}: {msg}")


def lib() -> ctypes.CDLL:
    """The loaded library; raises NotActive if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise NotActive("pairformer_hip", f"{LIB_PATH} is not built; run __graft_entry__.build()")
        handle = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def header_symbols() -> list[str]:
    """Function names declared in include/pairformer_hip.h."""
    with open(HEADER_PATH) as f:
        text = f.read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(pf_[a-z0-9_]+)\s*\(", text)))


def call(name: str, *args) -> int:
    """Call ``name`` and raise PFError on a non-zero status."""
    fn = getattr(lib(), name)
    status = fn(*args)
    if status != 0:
        msg = lib().pf_last_error()
        raise PFError(name, status, msg.decode() if msg else "")
    return status


def dtype_code(dt: torch.dtype) -> int:
    if dt == torch.float32:
        return PF_F32
    if dt == torch.bfloat16:
        return PF_BF16
    raise NotActive("pairformer_hip", f"dtype {dt} is not supported (fp32 or bf16 only)")


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream_of(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def require_device(name: str, *ts: torch.Tensor) -> None:
    """Refuse (NotActive) unless every tensor is on a HIP device; there is no CPU path."""
    for t in ts:
        if t is None:
            continue
        if not t.is_cuda:
            raise NotActive(name, "tensors must be on a ROCm GPU; this build has no CPU path")


def kernel_timer_start(kernel: str) -> None:
    """Bracket every later launch of ``kernel`` with HIP events on its stream (totals reset)."""
    call("pf_kernel_timer_start", kernel.encode())


def kernel_timer_read() -> tuple[float, int]:
    """(summed duration in ms, launch count) of the timed kernel so far; waits for its events."""
    total, count = ctypes.c_double(0.0), ctypes.c_long(0)
    call("pf_kernel_timer_read", ctypes.byref(total), ctypes.byref(count))
    return total.value, count.value


def kernel_timer_stop() -> None:
    call("pf_kernel_timer_stop")


def check_out(name: str, out: torch.Tensor, like: torch.Tensor, shape=None, dtype=None) -> None:
    """Refuse a caller-supplied ``out`` the kernels would write out of bounds of (or reinterpret)."""
    shape = tuple(like.shape) if shape is None else tuple(shape)
    dtype = like.dtype if dtype is None else dtype
    if not out.is_contiguous() or out.dtype != dtype or tuple(out.shape) != shape or out.device != like.device:
        raise NotActive(
            name, f"out must be a contiguous {dtype} tensor of shape {shape} on {like.device}, "
            f"got {out.dtype} {tuple(out.shape)} on {out.device} (contiguous={out.is_contiguous()})",
        )  # fmt: skip


# Redo bookkeeping of the flash-attention kernel (a test and debugging aid). While a
# RedoRecorder is active, every attention call reads back its redo flags (one int32 per
# wave of the fast pass; nonzero = recomputed by the exact running-maximum softmax) and
# appends the number of flagged waves. Reading them synchronises the stream.
_redo_log: list | None = None


class RedoRecorder:
    """``with RedoRecorder() as counts: ...`` collects one flagged-wave count per attention call."""

    def __enter__(self) -> list:
        global _redo_log
        self._prev = _redo_log
        _redo_log = []
        return _redo_log

    def __exit__(self, *exc) -> None:
        global _redo_log
        _redo_log = self._prev


def note_redo(query: str, workspace: torch.Tensor, *sizes: int) -> None:
    """Append the flagged-wave count of the call that just used ``workspace`` (if recording)."""
    if _redo_log is None:
        return
    off, cnt = ctypes.c_size_t(0), ctypes.c_size_t(0)
    call(query, *sizes, ctypes.byref(off), ctypes.byref(cnt))
    flags = workspace[off.value : off.value + 4 * cnt.value].view(torch.int32)
    _redo_log.append(int((flags != 0).sum().item()))
