"""FusedAddRMSNorm on MI355X: S = X + R (stored), Y = RMSNorm(S) * W.

Drop-in for ``kernels/fused_add_rms_norm.py`` of the reference
(fused_add_rms_norm.py:172-274). One HBM pass reads X and R and writes S and
Y; the backward reads dY (and the optional residual gradient dS) and the saved
S, and returns the same dX tensor as the gradient of both X and R, like
fused_add_rms_norm.py:230-232.
"""
from __future__ import annotations

import torch

from . import _lib


def _flat(t: torch.Tensor, hidden: int) -> torch.Tensor:
    return t.reshape(-1, hidden).contiguous()


def fused_add_rms_norm_forward(X, R, W, eps=1e-6):
    """Forward (fused_add_rms_norm.py:172-188). Returns (Y, S, RSTD)."""
    shape = X.shape
    hidden = shape[-1]
    assert R.shape == X.shape, f"X and R shapes differ: {tuple(X.shape)} vs {tuple(R.shape)}"
    assert W.dim() == 1 and W.shape[0] == hidden, f"Hidden dim mismatch: {hidden} vs {tuple(W.shape)}"
    dev = _lib.require_device(X, R, W)
    X2 = _flat(X, hidden)
    R2 = _flat(R, hidden)
    if R2.dtype != X2.dtype:
        R2 = R2.to(X2.dtype)
    W = W.contiguous()
    n_rows = X2.shape[0]
    Y = torch.empty_like(X2)
    S = torch.empty_like(X2)
    RSTD = torch.empty(n_rows, dtype=torch.float32, device=dev)
    _lib.call("hk_fused_add_rms_norm_fwd", Y.data_ptr(), S.data_ptr(), RSTD.data_ptr(), X2.data_ptr(),
              R2.data_ptr(), W.data_ptr(), n_rows, hidden, hidden, _lib.dtype_code(X2), _lib.dtype_code(W),
              float(eps), _lib.stream_of(dev))
    return Y.view(shape), S.view(shape), RSTD


def fused_add_rms_norm_backward(dY, dS_out, S, W, RSTD, eps=1e-6, dw_mode=_lib.DW_AUTO):
    """Backward (fused_add_rms_norm.py:191-232). Returns (dX, dR, dW); dR is dX."""
    shape = dY.shape
    hidden = shape[-1]
    dev = _lib.require_device(dY, dS_out, S, W, RSTD)
    dY2 = _flat(dY, hidden)
    S2 = _flat(S, hidden)
    if dY2.dtype != S2.dtype:
        dY2 = dY2.to(S2.dtype)
    dS2 = None
    if dS_out is not None:
        dS2 = _flat(dS_out, hidden)
        if dS2.dtype != S2.dtype:
            dS2 = dS2.to(S2.dtype)
    n_rows = dY2.shape[0]
    dX = torch.empty_like(S2)
    dW = torch.empty(hidden, dtype=W.dtype, device=dev)
    lib = _lib.load()
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    ws_bytes = lib.hk_rms_norm_bwd_workspace_size(n_rows, hidden, _lib.dtype_code(S2), _lib.dtype_code(W),
                                                 dw_mode, idx)
    ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=dev)
    _lib.call("hk_fused_add_rms_norm_bwd", dX.data_ptr(), dW.data_ptr(), dY2.data_ptr(), _lib.ptr(dS2),
              S2.data_ptr(), W.data_ptr(), RSTD.data_ptr(), n_rows, hidden, hidden, _lib.dtype_code(S2),
              _lib.dtype_code(W), dw_mode, ws.data_ptr(), ws.numel(), _lib.stream_of(dev))
    dX_out = dX.view(shape)
    return dX_out, dX_out, dW


class HildaFusedAddRMSNormFunction(torch.autograd.Function):
    """Autograd wrapper (fused_add_rms_norm.py:239-251): returns (Y, S)."""

    @staticmethod
    def forward(ctx, X, R, W, eps):
        Y, S, RSTD = fused_add_rms_norm_forward(X, R, W, eps)
        ctx.save_for_backward(S, W, RSTD)
        ctx.eps = eps
        return Y, S

    @staticmethod
    def backward(ctx, dY, dS_out):
        S, W, RSTD = ctx.saved_tensors
        if dY is None:
            dY = torch.zeros_like(S)
        dX, dR, dW = fused_add_rms_norm_backward(dY, dS_out, S, W, RSTD, ctx.eps)
        return dX, dR, dW, None


def hilda_fused_add_rms_norm(X, R, W, eps=1e-6):
    """Functional interface: returns (Y, S) with S = X + R, Y = RMSNorm(S) * W."""
    return HildaFusedAddRMSNormFunction.apply(X, R, W, eps)


class FusedAddRMSNorm(torch.nn.Module):
    """Fused residual add + RMSNorm module (fused_add_rms_norm.py:263-274)."""

    def __init__(self, hidden_dim, eps=1e-6):
        super().__init__()
        self.eps = eps
        self.weight = torch.nn.Parameter(torch.ones(hidden_dim))

    def forward(self, X, R):
        return hilda_fused_add_rms_norm(X, R, self.weight, self.eps)
