"""GeGLU on MI355X: c = gelu_tanh(a) * b, forward and backward.

Drop-in for ``kernels/geglu.py`` of the reference (geglu.py:131-195), with the
tanh approximation of GELU, 0.5 a (1 + tanh(sqrt(2/pi) (a + 0.044715 a^3)))
(geglu.py:69-70). Like SwiGLU, the backward returns fresh da/db tensors; the
reference writes them over the saved a and b (geglu.py:123-124,159).
"""
from __future__ import annotations

import torch

from . import _lib


def geglu_forward(a, b):
    """Forward (geglu.py:131-143)."""
    assert a.shape == b.shape, "a and b must have the same shape"
    assert a.dtype == b.dtype, "a and b must have the same dtype"
    _lib.require_device(a, b)
    a, b = a.contiguous(), b.contiguous()
    c = torch.empty_like(b)
    _lib.call("hk_geglu_fwd", c.data_ptr(), a.data_ptr(), b.data_ptr(), a.numel(), _lib.dtype_code(a),
              _lib.stream_of(a.device))
    return c


def geglu_backward(a, b, dc):
    """Backward (geglu.py:146-159): returns (da, db) as new tensors."""
    _lib.require_device(a, b, dc)
    a, b = a.contiguous(), b.contiguous()
    dc = dc.contiguous()
    if dc.dtype != a.dtype:
        dc = dc.to(a.dtype)
    da = torch.empty_like(a)
    db = torch.empty_like(b)
    _lib.call("hk_geglu_bwd", da.data_ptr(), db.data_ptr(), a.data_ptr(), b.data_ptr(), dc.data_ptr(), a.numel(),
              _lib.dtype_code(a), _lib.stream_of(a.device))
    return da, db


class HildaGeGLUFunction(torch.autograd.Function):
    """Autograd wrapper (geglu.py:166-177)."""

    @staticmethod
    def forward(ctx, a, b):
        c = geglu_forward(a, b)
        ctx.save_for_backward(a, b)
        return c

    @staticmethod
    def backward(ctx, dc):
        a, b = ctx.saved_tensors
        return geglu_backward(a, b, dc)


def hilda_geglu(a, b):
    """Functional interface: GeGLU(a, b) = GELU(a) * b (geglu.py:180-182)."""
    return HildaGeGLUFunction.apply(a, b)


class GeGLU(torch.nn.Module):
    """Drop-in GeGLU activation: forward(a, b) -> GELU(a) * b (geglu.py:189-192)."""

    def forward(self, a, b):
        return hilda_geglu(a, b)
