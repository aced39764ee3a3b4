"""RMSNorm on MI355X: y = (x * rstd).to(x.dtype) * w with rstd = 1/sqrt(mean(x^2) + eps).

Drop-in for ``kernels/rms_norm.py`` of the reference (rms_norm.py:261-413):
same functional name, autograd Function, module and argument meaning. The
forward saves only the per-row fp32 ``rstd``; the backward recomputes the
normalised row from ``x`` and sums dW through fp32 partial rows, one per
1024-lane block (the reference switches to atomics for few rows,
rms_norm.py:325-326; here ``dw_mode=DW_ATOMIC`` asks for fp64 atomics, which
measured slower at every size).
"""
from __future__ import annotations

import torch

from . import _lib


def _rows_view(t: torch.Tensor, hidden: int) -> torch.Tensor:
    """2-D [rows, hidden] view with unit column stride (copies only if needed)."""
    t2 = t.reshape(-1, hidden)
    if t2.stride(-1) != 1 or (t2.shape[0] > 1 and t2.stride(0) < hidden):
        t2 = t2.contiguous()
    return t2


def rms_norm_forward(X, W, eps=1e-6):
    """Forward (rms_norm.py:261-306). Returns (Y, X_flat, RSTD)."""
    shape = X.shape
    hidden = shape[-1]
    assert W.dim() == 1 and W.shape[0] == hidden, f"Hidden dim mismatch: {hidden} vs {tuple(W.shape)}"
    dev = _lib.require_device(X, W)
    X_flat = _rows_view(X, hidden)
    W = W.contiguous()
    n_rows = X_flat.shape[0]
    Y = torch.empty((n_rows, hidden), dtype=X.dtype, device=dev)
    RSTD = torch.empty(n_rows, dtype=torch.float32, device=dev)
    _lib.call("hk_rms_norm_fwd", Y.data_ptr(), RSTD.data_ptr(), X_flat.data_ptr(), W.data_ptr(),
              n_rows, hidden, X_flat.stride(0) if n_rows > 0 else hidden, hidden,
              _lib.dtype_code(X), _lib.dtype_code(W), float(eps), _lib.stream_of(dev))
    return Y.view(*shape), X_flat, RSTD


def rms_norm_backward(dY, X, W, RSTD, dw_mode=_lib.DW_AUTO):
    """Backward (rms_norm.py:309-359). Returns (dX, dW) with dW in W's dtype."""
    shape = dY.shape
    hidden = shape[-1]
    dev = _lib.require_device(dY, X, W, RSTD)
    dY_flat = _rows_view(dY, hidden)
    if dY_flat.dtype != X.dtype:
        dY_flat = dY_flat.to(X.dtype)
    n_rows = dY_flat.shape[0]
    dX = torch.empty((n_rows, hidden), dtype=X.dtype, device=dev)
    dW = torch.empty(hidden, dtype=W.dtype, device=dev)
    lib = _lib.load()
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    ws_bytes = lib.hk_rms_norm_bwd_workspace_size(n_rows, hidden, _lib.dtype_code(X), _lib.dtype_code(W),
                                                 dw_mode, idx)
    ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=dev)
    ld_x = X.stride(0) if n_rows > 0 else hidden
    ld_dy = dY_flat.stride(0) if n_rows > 0 else hidden
    _lib.call("hk_rms_norm_bwd", dX.data_ptr(), dW.data_ptr(), dY_flat.data_ptr(), X.data_ptr(), W.data_ptr(),
              RSTD.data_ptr(), n_rows, hidden, ld_dy, ld_x, hidden, _lib.dtype_code(X), _lib.dtype_code(W),
              dw_mode, ws.data_ptr(), ws.numel(), _lib.stream_of(dev))
    return dX.view(*shape), dW


class HildaRMSNormFunction(torch.autograd.Function):
    """Autograd wrapper (rms_norm.py:366-386): saves (X_flat, W, RSTD)."""

    @staticmethod
    def forward(ctx, X, W, eps=1e-6):
        Y, X_flat, RSTD = rms_norm_forward(X, W, eps)
        ctx.save_for_backward(X_flat, W, RSTD)
        return Y

    @staticmethod
    def backward(ctx, dY):
        X_flat, W, RSTD = ctx.saved_tensors
        dX, dW = rms_norm_backward(dY, X_flat, W, RSTD)
        return dX, dW, None


def hilda_rms_norm(X, W, eps=1e-6):
    """Functional interface for RMSNorm (rms_norm.py:389-391)."""
    return HildaRMSNormFunction.apply(X, W, eps)


class RMSNorm(torch.nn.Module):
    """RMSNorm module (rms_norm.py:398-413); weight initialised to fp32 ones.

    ``hidden_size`` is accepted as an alias of ``hidden_dim`` because the
    reference README uses that spelling (README:69).
    """

    def __init__(self, hidden_dim=None, eps=1e-6, *, hidden_size=None):
        super().__init__()
        if hidden_dim is None:
            hidden_dim = hidden_size
        if hidden_dim is None:
            raise TypeError("RMSNorm needs hidden_dim")
        self.eps = eps
        self.weight = torch.nn.Parameter(torch.ones(hidden_dim))

    def forward(self, x):
        return hilda_rms_norm(x, self.weight, self.eps)
