"""CPU: the C-ABI library loads and exports every symbol include/pairformer_hip.h declares."""

from __future__ import annotations

import ctypes
import os

import pytest

from tests._helpers import mod

_lib = mod("_lib")


def test_library_is_built():
    assert os.path.exists(_lib.LIB_PATH), "run __graft_entry__.build() first"


def test_every_header_symbol_is_exported_and_bound():
    lib = ctypes.CDLL(_lib.LIB_PATH)
    names = _lib.header_symbols()
    assert len(names) >= 5
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, f"declared but not exported: {missing}"
    unbound = [n for n in names if n not in _lib.SIGNATURES]
    assert not unbound, f"declared but missing from _lib.SIGNATURES: {unbound}"
    extra = [n for n in _lib.SIGNATURES if n not in names]
    assert not extra, f"bound but not declared in the header: {extra}"


def test_version_and_error_reporting_without_gpu():
    lib = _lib.lib()
    assert lib.pf_version() == 2
    # Argument validation runs before any device work, so it is testable on CPU.
    nul = None
    status = lib.pf_trimul_fwd(
        nul, nul, nul, nul, 1e-5, nul, nul, nul, 1e-5, nul, nul, 1, 8, 128, 1, 0, 0, nul, 0, nul, 0, nul
    )
    assert status == 1  # PF_ERR_INVALID_ARG
    assert b"null pointer" in lib.pf_last_error()
    assert lib.pf_last_error_code() == 1


def test_workspace_query():
    lib = _lib.lib()
    assert lib.pf_trimul_workspace_bytes(1, 768, 128, _lib.PF_BF16) == 3 * 128 * 768 * 768 * 2
    assert lib.pf_trimul_workspace_bytes(1, 100, 128, _lib.PF_F32) == 3 * 128 * 128 * 128 * 4


def test_cpu_tensors_are_refused():
    import torch

    k = mod("kernels")
    NotActive = mod("inference_guard").NotActive
    with pytest.raises(NotActive):
        k.layer_norm(torch.randn(4, 128), torch.ones(128), torch.zeros(128))


def test_noalloc_single_attention_refuses_oversize_without_gpu():
    """The allocation-free entry point refuses sizes whose scratch exceeds its static array
    before any device call (dummy non-null pointers; nothing is launched)."""
    lib = _lib.lib()
    C, H = 384, 16
    per_item = lib.pf_single_attn_workspace_bytes(1, 200, C, H, _lib.PF_BF16)
    B = _lib.NOALLOC_SCRATCH_BYTES // per_item + 1
    assert lib.pf_single_attn_workspace_bytes(B, 200, C, H, _lib.PF_BF16) > _lib.NOALLOC_SCRATCH_BYTES
    d = 16  # a non-null address the call must never dereference
    status = lib.pf_single_attn_fwd_noalloc(
        d, d, d, d, d, 1e-5, d, d, d, B, 200, C, H, _lib.PF_BF16, _lib.PF_BF16, d, 0, None
    )
    assert status == 3  # PF_ERR_WORKSPACE
    assert b"static" in lib.pf_last_error()
    with open(_lib.HEADER_PATH) as f:
        assert f"#define PF_NOALLOC_SCRATCH_BYTES (32u << 20)" in f.read()


def test_dropout_entry_points_validate_before_launch():
    """Bad rates, channel counts and null pointers are refused on the host (no GPU here)."""
    lib = _lib.lib()
    d = 256  # a non-null, aligned address the call must never dereference
    assert lib.pf_dropout_add_fwd(d, 0, d, 0, d, 1, 4, 4, 6, 1, 0.25, 1, None) == 2  # D % 4
    assert b"multiple of 4" in lib.pf_last_error()
    assert lib.pf_dropout_add_fwd(d, 0, d, 0, d, 1, 4, 4, 8, 1, 1.0, 1, None) == 1  # p = 1
    assert lib.pf_dropout_bwd(None, 0, d, 0, 1, 4, 4, 8, 0, 0.1, 1, None) == 1  # null
    assert lib.pf_dropout_mask(None, 8, 0.1, 1, None) == 1
    assert lib.pf_dropout_add_fwd(d + 4, 0, d, 0, d, 1, 4, 4, 8, 1, 0.25, 1, None) == 4  # fp32 not 16-aligned
    # nothing to do: status OK without a launch
    assert lib.pf_dropout_add_fwd(d, 1, d, 1, d, 0, 4, 4, 8, 0, 0.25, 1, None) == 0


def test_planes_contract_validates_before_launch():
    """Null, aliased, misaligned and badly sized plane contractions are refused on the host."""
    lib = _lib.lib()
    d = 256
    assert lib.pf_planes_contract(None, d, d + 4096, 2, 128, 1, None) == 1  # null
    assert lib.pf_planes_contract(d, d, d, 2, 128, 1, None) == 1  # X aliases A
    assert lib.pf_planes_contract(d, d + 4096, d + 8192, 2, 96, 1, None) == 1  # Np % 128
    assert b"multiple of 128" in lib.pf_last_error()
    assert lib.pf_planes_contract(d + 2, d + 4096, d + 8192, 2, 128, 1, None) == 4  # misaligned


def test_rms_residual_add_validates_before_launch():
    """Null operands, bad sizes and dtype codes are refused on the host; M = 0 is a no-op."""
    lib = _lib.lib()
    d = 256
    assert lib.pf_rms_residual_add(d, 1, None, 1, d, 4, 128, 1.0, 1e-6, None) == 1
    assert lib.pf_rms_residual_add(d, 1, d, 1, d, 4, 0, 1.0, 1e-6, None) == 1
    assert lib.pf_rms_residual_add(d, 3, d, 1, d, 4, 128, 1.0, 1e-6, None) == 2
    assert lib.pf_rms_residual_add(None, 1, d, 1, d, 0, 128, 1.0, 1e-6, None) == 0


def test_mhr_trimul_validates_before_launch():
    """The multi-head routed entry points refuse bad head counts, modes, router kinds, a
    post_channel mix without its router and a missing norm shift (outside head_rms) on the
    host; head_rms takes a null shift (then the workspace check is what refuses here)."""
    lib = _lib.lib()
    d = 1 << 20

    def fwd(heads, head_norm, wr, kind, lnb=d):
        # z, mask, ln_in w/b, eps, packed, ln_out w/b, eps, w_out, w_out_gate, B, N, C, outgoing,
        # zdtype, cdtype, out, accumulate, workspace, workspace_bytes (too small), MHR args, stream
        return lib.pf_trimul_mhr_fwd(d, d, d, d, 1e-5, d, d, lnb, 1e-5, d, d, 1, 8, 64, 1, 1, 1, d, 0, d, 16, heads,
                                     head_norm, wr, kind, None)  # fmt: skip

    assert fwd(0, 2, None, 0) == 1
    assert fwd(7, 2, None, 0) == 1 and b"dividing C=64" in lib.pf_last_error()
    assert fwd(64, 2, None, 0) == 1  # beyond 32 heads
    assert fwd(8, 4, None, 0) == 1
    assert fwd(8, 2, d, 2) == 1
    assert fwd(8, 3, None, 0) == 1 and b"post_channel needs the router" in lib.pf_last_error()
    assert fwd(8, 2, None, 0, lnb=None) == 1
    assert fwd(8, 1, None, 0, lnb=None) == 3  # head_rms: no shift needed; refused for the workspace
    assert fwd(8, 3, d, 1) == 3
    # the training forward and the output VJP share the checks
    assert lib.pf_trimul_mhr_train_fwd(d, d, d, d, d, 1e-5, d, d, 1, 8, 64, 1, 1, 1, d, 16, d, 8, 3, None, 0,
                                       None) == 1  # fmt: skip
    assert lib.pf_trimul_mhr_output_vjp(d, d, d, d, d, 1e-5, d, d, d, d, 1, 8, 64, 1, 1, d, d, d, d, d, d, d, d, 16,
                                        8, 2, d, 0, None, None) == 1  # router without d_router_logits  # fmt: skip
    assert b"d_router_logits" in lib.pf_last_error()
