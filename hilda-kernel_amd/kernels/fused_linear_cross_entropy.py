"""FusedLinearCrossEntropy (lm_head + CrossEntropy) on MI355X.

Drop-in for ``kernels/fused_linear_cross_entropy.py`` of the reference
(fused_linear_cross_entropy.py:103-241). The logits are produced a chunk of
rows at a time by an MFMA GEMM, turned into the cross-entropy gradient in
place, and contracted back into dhidden and dweight by two more MFMA GEMMs;
the full (BT, V) logits never exist. All gradient work happens in the forward
(as in the reference); the backward scales the saved gradients by the upstream
gradient on the device, with no host synchronisation (the reference uses
``torch.equal`` at :197 and ``.item()`` at :121).

Memory. ``workspace_budget`` picks the memory plan. The default (None, read
from $HILDA_FL_WORKSPACE_BUDGET when set) is the reference's own footprint: a
chunk whose logits are about the size of the hidden states (:112-114) and
grad_weight accumulated in place across chunks, as the reference does (:161).
'fastest' (or -1) lifts the limit, so the op runs as fast as its GEMMs allow;
a byte count takes the fastest plan within it.

Differences from the reference, by design:
  * rows whose target is ignore_index are compacted away on the device
    before the GEMMs, so they cost no FLOPs;
  * with room for it (a larger budget), grad_weight is summed in fp32 and
    rounded once instead of accumulated in the weight dtype (:118,161);
  * any H and V (padded inside the workspace);
  * reduction='none' gets correct gradients: the forward computes only the
    per-row losses and the backward recomputes the chunks with each row's
    gradient scaled by its upstream gradient (the reference scales everything
    by the first element, :90,197-209).
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from .cross_entropy import scale_rows_

DEFAULT_CHUNK = 0  # no cap: the workspace budget sets the chunk (at most 8192 rows)


def fused_linear_cross_entropy_forward(hidden_states, weight, targets, ignore_index=-100, reduction='mean',
                                       compute_grad=True, row_scale=None, chunk=DEFAULT_CHUNK,
                                       workspace_budget=None):
    """Forward (fused_linear_cross_entropy.py:103-171).

    Returns (loss, grad_input, grad_weight, n_valid): loss is a scalar, or the
    per-row losses for reduction='none'; the gradients are those of the
    reduced loss (times row_scale per row when given), or None. chunk caps the
    rows per chunk (0: no cap); workspace_budget: see the module docstring.
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
    budget = _lib.fl_budget(workspace_budget)
    ws_bytes = lib.hk_fused_linear_cross_entropy_workspace_size(BT, H, V, int(chunk), budget, dt, int(compute_grad),
                                                                hidden_states.data_ptr(), weight.data_ptr())
    ws = _lib.workspace(ws_bytes, "fused linear cross entropy", dev)
    _lib.call("hk_fused_linear_cross_entropy", _lib.ptr(loss), loss_rows.data_ptr(), _lib.ptr(grad_input),
              _lib.ptr(grad_weight), hidden_states.data_ptr(), weight.data_ptr(), targets.data_ptr(), _lib.ptr(rs),
              BT, H, V, int(ignore_index), _lib.REDUCTION[reduction], dt, int(chunk), budget, ws.data_ptr(),
              ws.numel(), _lib.stream_of(dev))
    # (a copy: a view would keep the whole workspace alive)
    n_valid = ws[:4].view(torch.int32).clone()[0]
    del ws
    return (loss_rows if reduction == 'none' else loss), grad_input, grad_weight, n_valid


class HildaFusedLinearCrossEntropyFunction(torch.autograd.Function):
    """Autograd wrapper (fused_linear_cross_entropy.py:178-210)."""

    @staticmethod
    def forward(ctx, hidden_states, weight, targets, ignore_index, reduction, workspace_budget=None):
        compute_grad = hidden_states.requires_grad or weight.requires_grad
        ctx.compute_grad = compute_grad
        ctx.reduction = reduction
        ctx.ignore_index = ignore_index
        ctx.budget = workspace_budget
        ctx.applied = None
        if reduction == 'none':
            # per-row upstream gradients are only known in backward: recompute there
            loss, _, _, _ = fused_linear_cross_entropy_forward(hidden_states, weight, targets, ignore_index,
                                                               reduction, compute_grad=False,
                                                               workspace_budget=workspace_budget)
            if compute_grad:
                ctx.save_for_backward(hidden_states, weight, targets)
            return loss
        loss, grad_input, grad_weight, _ = fused_linear_cross_entropy_forward(
            hidden_states, weight, targets, ignore_index, reduction, compute_grad=compute_grad,
            workspace_budget=workspace_budget)
        if compute_grad:
            ctx.save_for_backward(grad_input, grad_weight)
        return loss

    @staticmethod
    def backward(ctx, grad_output):
        if not ctx.compute_grad:
            return None, None, None, None, None, None
        if ctx.reduction == 'none':
            hidden_states, weight, targets = ctx.saved_tensors
            _, gi, gw, _ = fused_linear_cross_entropy_forward(hidden_states, weight, targets, ctx.ignore_index,
                                                              'sum', compute_grad=True, row_scale=grad_output,
                                                              workspace_budget=ctx.budget)
            return gi, gw, None, None, None, None
        grad_input, grad_weight = ctx.saved_tensors
        gi = grad_input.view(-1, grad_input.shape[-1])
        gw = grad_weight.view(-1, grad_weight.shape[-1])
        if ctx.applied is None:
            # in place on the device; returns at once when grad_output == 1
            scale_rows_(gi, gi, grad_output, None, skip_if_one=True)
            scale_rows_(gw, gw, grad_output, None, skip_if_one=True)
            ctx.applied = grad_output.detach()
            return grad_input, grad_weight, None, None, None, None
        # repeated backward (retain_graph): new tensors
        out_i = torch.empty_like(grad_input)
        out_w = torch.empty_like(grad_weight)
        scale_rows_(out_i.view_as(gi), gi, grad_output, ctx.applied)
        scale_rows_(out_w.view_as(gw), gw, grad_output, ctx.applied)
        return out_i, out_w, None, None, None, None


def hilda_fused_linear_cross_entropy(hidden_states, weight, targets, ignore_index=-100, reduction='mean',
                                     workspace_budget=None):
    """Functional interface: fused lm_head + CE loss (fused_linear_cross_entropy.py:213-220).
    workspace_budget (not in the reference): see the module docstring."""
    return HildaFusedLinearCrossEntropyFunction.apply(hidden_states, weight, targets, ignore_index, reduction,
                                                      workspace_budget)


def fused_linear_cross_entropy_plan(BT, H, V, dtype=torch.bfloat16, compute_grad=True, chunk=DEFAULT_CHUNK,
                                    workspace_budget=None):
    """The memory plan a call of that shape takes: a dict of rows per chunk, chunks, the dW mode ('deferred',
    'fp32 accumulator' or 'in output'; for the vocabulary-tiled plan 'vocab tiles, ...' with chunk the
    vocabulary columns a tile and chunks the tiles), whether W^T and D^T are materialised, the dX split cap,
    workspace bytes and the cost model's time estimate (ms)."""
    info = (ctypes.c_int64 * 8)()
    _lib.call("hk_fused_linear_cross_entropy_plan", int(BT), int(H), int(V), int(chunk),
              _lib.fl_budget(workspace_budget), _lib._DTYPE_CODE[dtype], int(compute_grad), None, None, info)
    return plan_dict(info)


def plan_dict(info):
    """A plan query's info[8] as the dict fused_linear_cross_entropy_plan returns."""
    modes = {0: "deferred", 1: "fp32 accumulator", 2: "in output", 3: "vocab tiles, dX fp32",
             4: "vocab tiles, dX in output"}
    return dict(chunk=info[0], chunks=info[1], dw=modes[info[2]], w_transposed=bool(info[3]),
                d_transposed=bool(info[4]), dx_splits=info[5], workspace_bytes=info[6], model_ms=info[7] / 1e6)


class FusedLinearCrossEntropyLoss(torch.nn.Module):
    """Fused linear projection + cross-entropy loss (fused_linear_cross_entropy.py:227-241).
    workspace_budget (not in the reference): see the module docstring."""

    def __init__(self, ignore_index=-100, reduction='mean', workspace_budget=None):
        super().__init__()
        self.ignore_index = ignore_index
        self.reduction = reduction
        self.workspace_budget = workspace_budget

    def forward(self, hidden_states, weight, targets):
        return hilda_fused_linear_cross_entropy(hidden_states, weight, targets, self.ignore_index, self.reduction,
                                                self.workspace_budget)
