"""CrossEntropy on MI355X with ignore_index, gradient computed in the forward pass.

Drop-in for ``kernels/cross_entropy.py`` of the reference (cross_entropy.py:196-313).
Training (logits.requires_grad): one kernel reads each non-ignored row once,
writes its loss and its dlogits = (softmax - onehot) * s, s = 1/max(n_valid, 1)
for 'mean'; ignored rows get loss 0 and a zero gradient row. n_valid stays on
the device. The backward returns the saved dlogits, scaled in place by the
upstream gradient on the device: a scalar gradient of exactly 1 (the usual
``loss.backward()``) makes the scale kernel return at once, which replaces the
reference's host-synchronising ``torch.equal`` test (cross_entropy.py:202-203).
Inference: one read per row gives the per-row loss and lse.

``ignore_index == -1`` keeps the reference's meaning "ignore nothing"
(cross_entropy.py:197-198,219-225), and a 'mean' over zero valid rows is 0.
"""
from __future__ import annotations

import torch

from . import _lib


def _check_inputs(logits, targets):
    assert logits.dim() == 2, f"expected (N, V) logits, got {tuple(logits.shape)}"
    assert targets.dim() == 1 and targets.shape[0] == logits.shape[0], \
        f"expected (N,) targets for (N, V) logits, got {tuple(targets.shape)}"
    _lib.require_device(logits, targets)
    logits = logits.contiguous()
    targets = targets.contiguous()
    if targets.dtype != torch.int64:
        targets = targets.to(torch.int64)
    return logits, targets


def _workspace(n_rows, device):
    nbytes = _lib.load().hk_cross_entropy_workspace_size(n_rows)
    return torch.empty(max(int(nbytes), 256), dtype=torch.uint8, device=device)


def cross_entropy_forward(logits, targets, ignore_index=-100, reduction='mean', needs_grad=False):
    """Fused CrossEntropy forward (cross_entropy.py:206-249).

    Returns (loss, aux, n_valid): aux is the precomputed dlogits on the
    training path and the per-row lse on the inference path; n_valid is an
    int32 device scalar.
    """
    if reduction not in _lib.REDUCTION:
        raise ValueError(f"reduction must be 'none', 'mean' or 'sum', got {reduction!r}")
    logits, targets = _check_inputs(logits, targets)
    n_rows, n_cols = logits.shape
    dev = logits.device
    per_token_loss = torch.empty(n_rows, dtype=torch.float32, device=dev)
    loss = None if reduction == 'none' else torch.empty((), dtype=torch.float32, device=dev)
    ws = _workspace(n_rows, dev)
    red = _lib.REDUCTION[reduction]
    if needs_grad:
        dlogits = torch.empty_like(logits)
        _lib.call("hk_cross_entropy_fwd_grad", dlogits.data_ptr(), per_token_loss.data_ptr(), _lib.ptr(loss),
                  logits.data_ptr(), targets.data_ptr(), n_rows, n_cols, n_cols, n_cols, int(ignore_index), red,
                  _lib.dtype_code(logits), ws.data_ptr(), ws.numel(), _lib.stream_of(dev))
        aux = dlogits
    else:
        lse = torch.empty(n_rows, dtype=torch.float32, device=dev)
        _lib.call("hk_cross_entropy_fwd", lse.data_ptr(), per_token_loss.data_ptr(), _lib.ptr(loss),
                  logits.data_ptr(), targets.data_ptr(), n_rows, n_cols, n_cols, int(ignore_index), red,
                  _lib.dtype_code(logits), ws.data_ptr(), ws.numel(), _lib.stream_of(dev))
        aux = lse
    n_valid = ws[:4].view(torch.int32)[0]
    return (per_token_loss if reduction == 'none' else loss), aux, n_valid


def scale_rows_(out, src, dloss, prev=None, skip_if_one=False):
    """out = src * dloss (scalar or one value per row), optionally / prev; on the device."""
    rows, cols = src.shape
    g = dloss.detach().to(torch.float32).contiguous()
    p = prev.detach().to(torch.float32).contiguous() if prev is not None else None
    _lib.call("hk_scale_rows", out.data_ptr(), src.data_ptr(), g.data_ptr(), _lib.ptr(p), int(g.dim() > 0),
              int(skip_if_one), rows, cols, src.stride(0), out.stride(0), _lib.dtype_code(src),
              _lib.stream_of(src.device))
    return out


def cross_entropy_backward(dloss, saved_grad, reduction='mean', prev_dloss=None):
    """Backward (cross_entropy.py:252-264). saved_grad already carries the loss scaling.

    First call (prev_dloss None): scales saved_grad in place by dloss on the
    device and returns it (a unit scalar dloss leaves it untouched, with no
    host synchronisation). A repeated backward (retain_graph) writes a new
    tensor saved_grad * dloss / prev_dloss.
    """
    if prev_dloss is None:
        return scale_rows_(saved_grad, saved_grad, dloss, None, skip_if_one=(reduction != 'none'))
    return scale_rows_(torch.empty_like(saved_grad), saved_grad, dloss, prev_dloss)


class HildaCrossEntropyFunction(torch.autograd.Function):
    """Autograd wrapper (cross_entropy.py:271-290)."""

    @staticmethod
    def forward(ctx, logits, targets, ignore_index, reduction):
        needs_grad = logits.requires_grad
        loss, aux, _ = cross_entropy_forward(logits, targets, ignore_index, reduction, needs_grad=needs_grad)
        ctx.reduction = reduction
        ctx.has_saved_grad = needs_grad
        ctx.applied_dloss = None
        if needs_grad:
            ctx.save_for_backward(aux)
        return loss

    @staticmethod
    def backward(ctx, dloss):
        if not ctx.has_saved_grad:
            return None, None, None, None
        (saved_grad,) = ctx.saved_tensors
        dlogits = cross_entropy_backward(dloss, saved_grad, ctx.reduction, ctx.applied_dloss)
        if ctx.applied_dloss is None:
            ctx.applied_dloss = dloss.detach()
        return dlogits, None, None, None


def hilda_cross_entropy(logits, targets, ignore_index=-100, reduction='mean'):
    """Functional interface for CrossEntropy (cross_entropy.py:293-295)."""
    return HildaCrossEntropyFunction.apply(logits, targets, ignore_index, reduction)


class CrossEntropyLoss(torch.nn.Module):
    """Drop-in for torch.nn.CrossEntropyLoss on (N, V) logits and (N,) targets
    (cross_entropy.py:302-313)."""

    def __init__(self, ignore_index=-100, reduction='mean'):
        super().__init__()
        self.ignore_index = ignore_index
        self.reduction = reduction

    def forward(self, logits, targets):
        return hilda_cross_entropy(logits, targets, self.ignore_index, self.reduction)
