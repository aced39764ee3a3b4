"""Jensen-Shannon divergence JSD(beta) on MI355X, gradient computed in the forward pass.

Drop-in for ``kernels/jsd.py`` of the reference (jsd.py:97-172): X student and
Y teacher log-probabilities [BT, V]; beta = 0 is KL(P||Q), beta = 1 KL(Q||P),
otherwise beta KL(P||M) + (1 - beta) KL(Q||M) with M = beta P + (1 - beta) Q.
One kernel reads each row once and writes its loss and dX, both divided by
the number of rows whose label is not ignore_index (all rows without labels).
That count stays on the device (the reference reads it on the host,
jsd.py:113-117). The backward scales the saved dX in place by the upstream
gradient on the device, and a unit upstream gradient (``loss.backward()``)
leaves it untouched without a pass over memory; the reference always
multiplies (jsd.py:150-152). A repeated backward writes a new tensor.
"""
from __future__ import annotations

import torch

from . import _lib
from .cross_entropy import cross_entropy_backward


def jsd_forward(X, Y, beta=0.5, labels=None, ignore_index=-100):
    """Forward + gradient (jsd.py:97-135). Returns (loss, dX)."""
    assert X.dim() == 2 and X.shape == Y.shape, "X and Y must be (BT, V) and of the same shape"
    _lib.require_device(X, Y)
    if X.dtype != Y.dtype:  # widen exactly; dX keeps X's dtype
        Xc, Yc = X.float().contiguous(), Y.float().contiguous()
    else:
        Xc, Yc = X.contiguous(), Y.contiguous()
    rows, cols = Xc.shape
    dev = Xc.device
    loss_rows = torch.empty(rows, dtype=torch.float32, device=dev)
    loss = torch.empty((), dtype=torch.float32, device=dev)
    dX = torch.empty_like(Xc)
    lab, ws = None, None
    if labels is not None:
        _lib.require_device(labels)
        lab = labels.contiguous().to(torch.int64)
        ws = torch.empty(int(_lib.load().hk_jsd_workspace_size()), dtype=torch.uint8, device=dev)
    _lib.call("hk_jsd_fwd", loss.data_ptr(), loss_rows.data_ptr(), dX.data_ptr(), Xc.data_ptr(), Yc.data_ptr(),
              _lib.ptr(lab), int(ignore_index), float(beta), rows, cols, cols, cols, cols, _lib.dtype_code(Xc),
              _lib.ptr(ws), 0 if ws is None else ws.numel(), _lib.stream_of(dev))
    return loss, dX.to(X.dtype)


class HildaJSDFunction(torch.autograd.Function):
    """Autograd wrapper (jsd.py:142-152)."""

    @staticmethod
    def forward(ctx, X, Y, beta, labels, ignore_index):
        loss, dX = jsd_forward(X, Y, beta, labels, ignore_index)
        ctx.save_for_backward(dX)
        ctx.applied = None
        return loss

    @staticmethod
    def backward(ctx, grad_output):
        dX, = ctx.saved_tensors
        out = cross_entropy_backward(grad_output, dX, 'sum', ctx.applied)
        if ctx.applied is None:
            ctx.applied = grad_output.detach()
        return out, None, None, None, None


def hilda_jsd(X, Y, beta=0.5, labels=None, ignore_index=-100):
    """Functional interface: JSD(beta)(teacher || student) (jsd.py:155-157)."""
    return HildaJSDFunction.apply(X, Y, beta, labels, ignore_index)


class JSDLoss(torch.nn.Module):
    """Jensen-Shannon divergence loss (jsd.py:164-172)."""

    def __init__(self, beta=0.5, ignore_index=-100):
        super().__init__()
        self.beta = beta
        self.ignore_index = ignore_index

    def forward(self, X, Y, labels=None):
        return hilda_jsd(X, Y, self.beta, labels, self.ignore_index)
