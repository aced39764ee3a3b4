"""SwiGLU on MI355X: c = silu(a) * b, forward and backward.

Drop-in for ``kernels/swiglu.py`` of the reference (swiglu.py:112-174). The
backward returns fresh da/db tensors; the reference writes them over the saved
a and b (swiglu.py:104-105,141), which clobbers tensors the caller may still
hold. HBM traffic is the same either way.
"""
from __future__ import annotations

import torch

from . import _lib


def swiglu_forward(a, b):
    """Forward (swiglu.py:112-124)."""
    assert a.shape == b.shape, "a and b must have the same shape"
    assert a.dtype == b.dtype, "a and b must have the same dtype"
    _lib.require_device(a, b)
    a, b = a.contiguous(), b.contiguous()
    c = torch.empty_like(b)
    _lib.call("hk_swiglu_fwd", c.data_ptr(), a.data_ptr(), b.data_ptr(), a.numel(), _lib.dtype_code(a),
              _lib.stream_of(a.device))
    return c


def swiglu_backward(a, b, dc):
    """Backward (swiglu.py:127-141): returns (da, db) as new tensors."""
    _lib.require_device(a, b, dc)
    a, b = a.contiguous(), b.contiguous()
    dc = dc.contiguous()
    if dc.dtype != a.dtype:
        dc = dc.to(a.dtype)
    da = torch.empty_like(a)
    db = torch.empty_like(b)
    _lib.call("hk_swiglu_bwd", da.data_ptr(), db.data_ptr(), a.data_ptr(), b.data_ptr(), dc.data_ptr(), a.numel(),
              _lib.dtype_code(a), _lib.stream_of(a.device))
    return da, db


class HildaSwiGLUFunction(torch.autograd.Function):
    """Autograd wrapper (swiglu.py:148-159)."""

    @staticmethod
    def forward(ctx, a, b):
        c = swiglu_forward(a, b)
        ctx.save_for_backward(a, b)
        return c

    @staticmethod
    def backward(ctx, dc):
        a, b = ctx.saved_tensors
        return swiglu_backward(a, b, dc)


def hilda_swiglu(a, b):
    """Functional interface: SwiGLU(a, b) = SiLU(a) * b (swiglu.py:162-164)."""
    return HildaSwiGLUFunction.apply(a, b)


class SwiGLU(torch.nn.Module):
    """Drop-in SwiGLU activation: forward(a, b) -> SiLU(a) * b (swiglu.py:171-174)."""

    def forward(self, a, b):
        return hilda_swiglu(a, b)
