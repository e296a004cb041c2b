"""CPU: the HIP kernels are registered PyTorch operators with shape-only fake implementations.

``deepfold3_amd::*`` ops (``torch_ops.py``) let tracers (``torch.compile``, ``torch.export``)
treat each HIP launch as one opaque node. Here, without a GPU: every op is registered, and
under ``FakeTensorMode`` each returns the output shapes and dtypes the kernels produce.
"""

from __future__ import annotations

import torch
from torch._subclasses.fake_tensor import FakeTensorMode

from tests._helpers import mod

T = mod("torch_ops")
OPS = ("layer_norm", "ln_transpose", "swiglu", "trimul", "evo_attention", "evo_attention_backward")


def test_ops_registered():
    for name in OPS:
        assert hasattr(getattr(torch.ops, T.NS), name), name


def test_fake_shapes():
    with FakeTensorMode():
        x = torch.empty(2, 5, 7, 128, dtype=torch.bfloat16)
        w, b = torch.empty(128), torch.empty(128)
        assert T.layer_norm(x, w, b, 1e-5).shape == x.shape
        y = T.ln_transpose(x, w, b, 1e-5, True)
        assert y.shape == (2, 7, 5, 128) and y.dtype == torch.bfloat16
        assert T.ln_transpose(x, w, b, 1e-5, False).shape == x.shape
        assert T.swiglu(torch.empty(3, 4, 1024)).shape == (3, 4, 512)
        z = torch.empty(1, 9, 9, 128)
        wp = torch.empty(512, 128)
        wo = torch.empty(128, 128)
        u = T.trimul(z, torch.empty(1, 9, 9), w, b, 1e-5, wp, w, b, 1e-5, wo, wo, True)
        assert u.shape == z.shape and u.dtype == z.dtype
        q = torch.empty(1, 3, 4, 10, 32, dtype=torch.bfloat16)
        rm, pb = torch.empty(1, 3, 10), torch.empty(1, 4, 10, 10)
        o = T.evo_attention(q, q, q, rm, pb, True)
        assert o.shape == q.shape and o.dtype == q.dtype
        dq, dk, dv, dpb = T.evo_attention_backward(q, q, q, rm, pb, o)
        assert dq.shape == q.shape and dpb.shape == (1, 4, 10, 10) and dpb.dtype == torch.float32
