"""KL divergence loss on MI355X (y_pred log-probabilities, y_true probabilities or log-probabilities).

Drop-in for ``kernels/kl_div.py`` of the reference (kl_div.py:114-207). The
forward reads each row once and keeps one fp32 sum per row; the reductions
('batchmean' default, 'sum', 'mean', and 'none' = the per-row sums, as in the
reference) finish on the device. The backward is -y_true * scale (or
-exp(y_true) * scale), with the upstream gradient read on the device instead
of the reference's ``float(grad_output)`` (kl_div.py:147-155). For 'none' it
scales each row by its own upstream value; the reference applies 1.0 to every
row (:155), which agrees whenever the upstream gradient is all ones.
"""
from __future__ import annotations

import torch

from . import _lib

_RED = {"none": 0, "mean": 1, "sum": 2, "batchmean": 3}


def _pair(y_pred, y_true):
    assert y_pred.shape == y_true.shape, "y_pred and y_true must have the same shape"
    _lib.require_device(y_pred, y_true)
    if y_pred.dtype != y_true.dtype:  # widen exactly, as the reference reads both in fp32
        y_pred, y_true = y_pred.float(), y_true.float()
    cols = y_pred.shape[-1] if y_pred.dim() > 0 else 1
    return y_pred.contiguous().reshape(-1, cols), y_true.contiguous().reshape(-1, cols)


def kl_div_forward(y_pred, y_true, reduction='batchmean', log_target=False, eps=1e-10):
    """Forward (kl_div.py:114-138)."""
    if reduction not in _RED:
        raise ValueError(f"reduction must be one of {sorted(_RED)}, got {reduction!r}")
    yp, yt = _pair(y_pred, y_true)
    rows, cols = yp.shape
    dev = yp.device
    loss_rows = torch.empty(rows, dtype=torch.float32, device=dev)
    loss = None if reduction == 'none' else torch.empty((), dtype=torch.float32, device=dev)
    _lib.call("hk_kl_div_fwd", _lib.ptr(loss), loss_rows.data_ptr(), yp.data_ptr(), yt.data_ptr(), rows, cols, cols,
              cols, int(bool(log_target)), float(eps), _RED[reduction], _lib.dtype_code(yp), _lib.stream_of(dev))
    return loss_rows if reduction == 'none' else loss


def kl_div_backward(y_true, grad_output, reduction='batchmean', log_target=False):
    """Backward (kl_div.py:141-166): d loss / d y_pred, in y_true's dtype and shape."""
    _lib.require_device(y_true)
    shape = y_true.shape
    yt = y_true.contiguous().reshape(-1, shape[-1] if y_true.dim() > 0 else 1)
    rows, cols = yt.shape
    g = grad_output.detach().to(torch.float32).contiguous()
    per_row = reduction == 'none'
    factor = {"batchmean": 1.0 / max(rows, 1), "mean": 1.0 / max(rows * cols, 1)}.get(reduction, 1.0)
    dy = torch.empty_like(yt)
    _lib.call("hk_kl_div_bwd", dy.data_ptr(), yt.data_ptr(), g.data_ptr(), int(per_row), float(factor), rows, cols,
              cols, cols, int(bool(log_target)), _lib.dtype_code(yt), _lib.stream_of(yt.device))
    return dy.reshape(shape)


class HildaKLDivFunction(torch.autograd.Function):
    """Autograd wrapper (kl_div.py:173-186)."""

    @staticmethod
    def forward(ctx, y_pred, y_true, reduction, log_target, eps):
        loss = kl_div_forward(y_pred, y_true, reduction, log_target, eps)
        ctx.save_for_backward(y_true)
        ctx.reduction = reduction
        ctx.log_target = log_target
        ctx.pred_dtype = y_pred.dtype
        return loss

    @staticmethod
    def backward(ctx, grad_output):
        y_true, = ctx.saved_tensors
        dy = kl_div_backward(y_true, grad_output, ctx.reduction, ctx.log_target)
        return dy.to(ctx.pred_dtype), None, None, None, None


def hilda_kl_div(y_pred, y_true, reduction='batchmean', log_target=False, eps=1e-10):
    """Functional interface: KL(y_true || y_pred), y_pred in log space (kl_div.py:189-191)."""
    return HildaKLDivFunction.apply(y_pred, y_true, reduction, log_target, eps)


class KLDivLoss(torch.nn.Module):
    """Drop-in replacement for torch.nn.KLDivLoss (kl_div.py:198-207)."""

    def __init__(self, reduction='batchmean', log_target=False, eps=1e-10):
        super().__init__()
        self.reduction = reduction
        self.log_target = log_target
        self.eps = eps

    def forward(self, y_pred, y_true):
        return hilda_kl_div(y_pred, y_true, self.reduction, self.log_target, self.eps)
