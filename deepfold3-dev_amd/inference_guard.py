"""How the HIP kernels refuse work, with the reference's exception names.

Interface as in the reference (``src/deepfold3/model/inference_guard.py``): a kernel that
cannot serve a call raises ``NotActive(lever, reason)`` (attributes ``lever`` and
``reason``), a forward-only kernel reached while autograd is recording raises
``InferenceOnlyKernelError``, and ``@inference_only(lever)`` puts that check in front of
a kernel's entry point. Every refusal lands in the kernel census under the path
``"refused:<reason>"`` of the refusing lever, so a run's census shows what was turned
away as well as what ran. No refusal falls back to another implementation.
"""

from __future__ import annotations

import functools
from collections.abc import Callable
from typing import TypeVar

import torch

from . import kernel_census

__all__ = ["InferenceOnlyKernelError", "NotActive", "inference_only", "require_no_grad"]

_F = TypeVar("_F", bound=Callable)

# Census path of a refusal made because autograd was recording.
GRAD_REFUSAL = "refused:grad_enabled"


def _log_refusal(lever: str, why: str) -> None:
    kernel_census.record(lever, why if why.startswith("refused:") else f"refused:{why}")


class InferenceOnlyKernelError(RuntimeError):
    """Autograd was recording when a kernel with no backward was called."""


class NotActive(Exception):
    """``lever`` cannot serve this call, for ``reason``; recorded in the census when raised."""

    def __init__(self, lever: str, reason: str):
        super().__init__(f"{lever} is not active for this call ({reason})")
        self.lever, self.reason = lever, reason
        _log_refusal(lever, reason)


def require_no_grad(lever: str) -> None:
    """Raise InferenceOnlyKernelError if autograd is recording.

    The test is on the global grad mode, not on ``requires_grad`` of the inputs:
    parameters always require grad, so inference passes them in too, while with grad
    mode on a kernel outside autograd would silently cut the graph."""
    if not torch.is_grad_enabled():
        return
    _log_refusal(lever, GRAD_REFUSAL)
    raise InferenceOnlyKernelError(
        f"{lever} has no backward pass; run it under torch.no_grad() or torch.inference_mode()"
    )


def inference_only(lever: str) -> Callable[[_F], _F]:
    """Decorator: ``require_no_grad(lever)`` before every call of the wrapped entry point."""

    def bind(fn: _F) -> _F:
        @functools.wraps(fn)
        def guarded(*args, **kwargs):
            require_no_grad(lever)
            return fn(*args, **kwargs)

        return guarded  # type: ignore[return-value]

    return bind
