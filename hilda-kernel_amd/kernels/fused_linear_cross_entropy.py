"""FusedLinearCrossEntropy (lm_head + CrossEntropy) on MI355X.

Drop-in for ``kernels/fused_linear_cross_entropy.py`` of the reference
(fused_linear_cross_entropy.py:103-241). The logits are produced `chunk` rows
at a time by a bf16/fp16 MFMA GEMM, turned into the cross-entropy gradient in
place, and contracted back into dhidden and dweight by two more MFMA GEMMs;
the full (BT, V) logits never exist. All gradient work happens in the forward
(as in the reference); the backward scales the saved gradients by the upstream
gradient on the device, with no host synchronisation (the reference uses
``torch.equal`` at :197 and ``.item()`` at :121).

Differences from the reference, by design:
  * grad_weight is summed in fp32 and rounded once (the reference
    accumulates in bf16, :118,161);
  * rows whose target is ignore_index are compacted away on the device
    before the GEMMs, so they cost no FLOPs;
  * reduction='none' gets correct gradients: the forward computes only the
    per-row losses and the backward recomputes the chunks with each row's
    gradient scaled by its upstream gradient (the reference scales everything
    by the first element, :90,197-209).
"""
from __future__ import annotations

import torch

from . import _lib
from .cross_entropy import scale_rows_

DEFAULT_CHUNK = 8192


def fused_linear_cross_entropy_forward(hidden_states, weight, targets, ignore_index=-100, reduction='mean',
                                       compute_grad=True, row_scale=None, chunk=DEFAULT_CHUNK):
    """Forward (fused_linear_cross_entropy.py:103-171).

    Returns (loss, grad_input, grad_weight, n_valid): loss is a scalar, or the
    per-row losses for reduction='none'; the gradients are those of the
    reduced loss (times row_scale per row when given), or None.
    """
    if reduction not in _lib.REDUCTION:
        raise ValueError(f"reduction must be 'none', 'mean' or 'sum', got {reduction!r}")
    assert hidden_states.dim() == 2 and weight.dim() == 2 and hidden_states.shape[1] == weight.shape[1], \
        f"expected hidden (BT, H) and weight (V, H); got {tuple(hidden_states.shape)} and {tuple(weight.shape)}"
    assert targets.dim() == 1 and targets.shape[0] == hidden_states.shape[0]
    if hidden_states.dtype != weight.dtype:
        raise TypeError(f"hidden_states ({hidden_states.dtype}) and weight ({weight.dtype}) dtypes differ")
    if hidden_states.dtype not in (torch.bfloat16, torch.float16, torch.float32):
        raise TypeError(f"fused linear cross entropy takes fp32, bf16 or fp16; got {hidden_states.dtype}")
    dev = _lib.require_device(hidden_states, weight, targets, row_scale)
    hidden_states = hidden_states.contiguous()
    weight = weight.contiguous()
    targets = targets.contiguous()
    if targets.dtype != torch.int64:
        targets = targets.to(torch.int64)
    BT, H = hidden_states.shape
    V = weight.shape[0]
    dt = _lib.dtype_code(hidden_states)
    loss_rows = torch.empty(BT, dtype=torch.float32, device=dev)
    loss = None if reduction == 'none' else torch.empty((), dtype=torch.float32, device=dev)
    grad_input = torch.empty_like(hidden_states) if compute_grad else None
    grad_weight = torch.empty_like(weight) if compute_grad else None
    rs = None
    if row_scale is not None:
        rs = row_scale.detach().to(torch.float32).contiguous()
    lib = _lib.load()
    ws_bytes = lib.hk_fused_linear_cross_entropy_workspace_size(BT, H, V, chunk, dt, int(compute_grad))
    ws = torch.empty(max(int(ws_bytes), 256), dtype=torch.uint8, device=dev)
    _lib.call("hk_fused_linear_cross_entropy", _lib.ptr(loss), loss_rows.data_ptr(), _lib.ptr(grad_input),
              _lib.ptr(grad_weight), hidden_states.data_ptr(), weight.data_ptr(), targets.data_ptr(), _lib.ptr(rs),
              BT, H, V, int(ignore_index), _lib.REDUCTION[reduction], dt, int(chunk), ws.data_ptr(), ws.numel(),
              _lib.stream_of(dev))
    n_valid = ws[:4].view(torch.int32)[0]
    return (loss_rows if reduction == 'none' else loss), grad_input, grad_weight, n_valid


class HildaFusedLinearCrossEntropyFunction(torch.autograd.Function):
    """Autograd wrapper (fused_linear_cross_entropy.py:178-210)."""

    @staticmethod
    def forward(ctx, hidden_states, weight, targets, ignore_index, reduction):
        compute_grad = hidden_states.requires_grad or weight.requires_grad
        ctx.compute_grad = compute_grad
        ctx.reduction = reduction
        ctx.ignore_index = ignore_index
        ctx.applied = None
        if reduction == 'none':
            # per-row upstream gradients are only known in backward: recompute there
            loss, _, _, _ = fused_linear_cross_entropy_forward(hidden_states, weight, targets, ignore_index,
                                                               reduction, compute_grad=False)
            if compute_grad:
                ctx.save_for_backward(hidden_states, weight, targets)
            return loss
        loss, grad_input, grad_weight, _ = fused_linear_cross_entropy_forward(
            hidden_states, weight, targets, ignore_index, reduction, compute_grad=compute_grad)
        if compute_grad:
            ctx.save_for_backward(grad_input, grad_weight)
        return loss

    @staticmethod
    def backward(ctx, grad_output):
        if not ctx.compute_grad:
            return None, None, None, None, None
        if ctx.reduction == 'none':
            hidden_states, weight, targets = ctx.saved_tensors
            _, gi, gw, _ = fused_linear_cross_entropy_forward(hidden_states, weight, targets, ctx.ignore_index,
                                                              'sum', compute_grad=True, row_scale=grad_output)
            return gi, gw, None, None, None
        grad_input, grad_weight = ctx.saved_tensors
        gi = grad_input.view(-1, grad_input.shape[-1])
        gw = grad_weight.view(-1, grad_weight.shape[-1])
        if ctx.applied is None:
            # in place on the device; returns at once when grad_output == 1
            scale_rows_(gi, gi, grad_output, None, skip_if_one=True)
            scale_rows_(gw, gw, grad_output, None, skip_if_one=True)
            ctx.applied = grad_output.detach()
            return grad_input, grad_weight, None, None, None
        # repeated backward (retain_graph): new tensors
        out_i = torch.empty_like(grad_input)
        out_w = torch.empty_like(grad_weight)
        scale_rows_(out_i.view_as(gi), gi, grad_output, ctx.applied)
        scale_rows_(out_w.view_as(gw), gw, grad_output, ctx.applied)
        return out_i, out_w, None, None, None


def hilda_fused_linear_cross_entropy(hidden_states, weight, targets, ignore_index=-100, reduction='mean'):
    """Functional interface: fused lm_head + CE loss (fused_linear_cross_entropy.py:213-220)."""
    return HildaFusedLinearCrossEntropyFunction.apply(hidden_states, weight, targets, ignore_index, reduction)


class FusedLinearCrossEntropyLoss(torch.nn.Module):
    """Fused linear projection + cross-entropy loss (fused_linear_cross_entropy.py:227-241)."""

    def __init__(self, ignore_index=-100, reduction='mean'):
        super().__init__()
        self.ignore_index = ignore_index
        self.reduction = reduction

    def forward(self, hidden_states, weight, targets):
        return hilda_fused_linear_cross_entropy(hidden_states, weight, targets, self.ignore_index, self.reduction)
