"""Refusal contract for the forward-only HIP kernels.

Same contract as the reference (``src/deepfold3/model/inference_guard.py:33-75``):
a kernel that cannot serve a call raises :class:`NotActive` naming itself, and a
forward-only kernel reached with grad enabled raises
:class:`InferenceOnlyKernelError`. Both are recorded in the kernel census.
Nothing falls back silently to another path.
"""

from __future__ import annotations

import functools
from collections.abc import Callable
from typing import TypeVar

import torch

from . import kernel_census

__all__ = ["InferenceOnlyKernelError", "NotActive", "inference_only"]

_F = TypeVar("_F", bound=Callable)


class InferenceOnlyKernelError(RuntimeError):
    """A forward-only kernel was reached with grad enabled."""


class NotActive(Exception):
    """A kernel cannot serve this call.

    Attributes:
        lever: Name of the kernel that refused.
        reason: Why it refused.
    """

    def __init__(self, lever: str, reason: str):
        self.lever = lever
        self.reason = reason
        super().__init__(f"NOT ACTIVE: {lever}: {reason}")
        kernel_census.record(lever, f"refused:{reason}")


def inference_only(lever: str) -> Callable[[_F], _F]:
    """Refuse to run a kernel wherever autograd could build a backward through it."""

    def decorate(fn: _F) -> _F:
        @functools.wraps(fn)
        def wrapper(*args, **kwargs):
            if torch.is_grad_enabled():
                kernel_census.record(lever, "refused:grad_enabled")
                raise InferenceOnlyKernelError(
                    f"{lever} is forward-only: call it under torch.no_grad() or torch.inference_mode()."
                )
            return fn(*args, **kwargs)

        return wrapper  # type: ignore[return-value]

    return decorate
