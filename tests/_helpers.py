"""Shared test helpers: tolerance rules and parameter slicing."""

from __future__ import annotations

import importlib

import torch

PKG = "deepfold3_dev_amd"


def mod(name: str):
    return importlib.import_module(f"{PKG}.{name}")


def sub(sd: dict, prefix: str) -> dict:
    return {k[len(prefix) :]: v for k, v in sd.items() if k.startswith(prefix)}


def to(d: dict, device, dtype=None) -> dict:
    return {k: (v.to(device=device, dtype=dtype) if dtype is not None else v.to(device)) for k, v in d.items()}


def rel_l2(a: torch.Tensor, b: torch.Tensor) -> float:
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return ((a - b).norm() / b.norm().clamp_min(1e-30)).item()


def max_abs(a: torch.Tensor, b: torch.Tensor) -> float:
    return (a.detach().double().cpu() - b.detach().double().cpu()).abs().max().item()


# fp32 parity bar: relative L2 and max-abs relative to max|ref| (both 1e-5).
FP32_TOL = 1e-5


def assert_fp32_close(got: torch.Tensor, ref: torch.Tensor, tol: float = FP32_TOL, what: str = ""):
    r = rel_l2(got, ref)
    m = max_abs(got, ref) / ref.detach().abs().max().clamp_min(1e-30).item()
    assert r <= tol and m <= tol, f"{what}: relL2={r:.3e} maxabs/max|ref|={m:.3e} (tol {tol:.0e})"


def assert_bf16_rule(got: torch.Tensor, eager_bf16: torch.Tensor, ref32: torch.Tensor, what: str = "", slack=2.0):
    """The reference's bf16 rule (tests/triton/test_fused_trimul.py:66-83):
    relL2(kernel - fp32 ref) <= 2 * relL2(eager bf16 - fp32 ref)."""
    e_k = rel_l2(got.float(), ref32)
    e_s = rel_l2(eager_bf16.float(), ref32)
    assert e_k <= slack * e_s, f"{what}: relL2(hip)={e_k:.3e} > {slack} x relL2(eager bf16)={e_s:.3e}"
    return e_k, e_s
