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
        dq, dk, dv, dpb = T.evo_attention_backward(q, q, q, rm, pb, o, True)
        assert dq.shape == q.shape and dpb.shape == (1, 4, 10, 10) and dpb.dtype == torch.float32
        # the real op returns a contiguous tensor; the fake must report the same strides
        xp = torch.empty(2, 7, 5, 128).permute(0, 2, 1, 3)
        assert T.layer_norm(xp, w, b, 1e-5).is_contiguous()


def test_attention_ops_refuse_bad_operands_before_any_device_call():
    """Wrong dtypes or shapes (a bf16 pair bias, the reference's broadcast [B, S, 1, 1, N] mask,
    K/V unlike Q) raise NotActive from the checks themselves: these are CPU tensors, so a device
    call would have refused differently ("no CPU path")."""
    NotActive = mod("inference_guard").NotActive
    q = torch.zeros(1, 3, 4, 10, 32, dtype=torch.bfloat16)
    rm, pb = torch.zeros(1, 3, 10), torch.zeros(1, 4, 10, 10)
    cases = [
        ((q, q, q, rm, pb.bfloat16()), "pair_bias"),
        ((q, q, q, rm.view(1, 3, 1, 1, 10), pb), "res_mask"),
        ((q, q, q, rm, pb.unsqueeze(1)), "pair_bias"),
        ((q, q.float(), q, rm, pb), "dtype"),
        ((q, q[:, :, :, :9], q, rm, pb), "shape"),
        ((q[..., :16], q[..., :16], q[..., :16], rm, pb), "D=16"),
        ((q.to(torch.float16), q.to(torch.float16), q.to(torch.float16), rm, pb), "dtype"),
    ]
    for args, needle in cases:
        for fn in (lambda *a: T.evo_attention(*a, True), lambda *a: T.evo_attention_backward(*a, a[0], True)):
            try:
                fn(*args)
            except NotActive as e:
                assert needle in str(e), (needle, str(e))
                assert "CPU path" not in str(e)
            else:
                raise AssertionError(f"accepted {needle}")
        with FakeTensorMode():  # the fake implementation refuses the same operands at trace time
            fa = [torch.empty(t.shape, dtype=t.dtype) for t in args]
            try:
                T.evo_attention(*fa, True)
            except NotActive:
                pass
            else:
                raise AssertionError(f"fake accepted {needle}")
    # well-formed CPU operands pass the checks and are refused only for the device
    try:
        T.evo_attention(q, q, q, rm, pb, True)
    except NotActive as e:
        assert "CPU path" in str(e)
    else:
        raise AssertionError("CPU operands accepted")
