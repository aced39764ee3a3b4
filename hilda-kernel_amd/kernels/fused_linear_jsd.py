"""FusedLinearJSD (student and teacher lm_heads + JSD) on MI355X.

Drop-in for ``kernels/fused_linear_jsd.py`` of the reference
(fused_linear_jsd.py:114-275). Per chunk of rows, the student and teacher
logits come from bf16/fp16 MFMA GEMMs, one row kernel takes both
temperature log-softmaxes, the JSD(beta) loss and the student dlogits
(written over the student logits), and two more MFMA GEMMs contract the
dlogits into grad_input and grad_weight; the full (BT, V) logits never exist.
All gradient work happens in the forward (as in the reference); the backward
scales the saved gradients by the upstream gradient on the device, and a unit
upstream gradient leaves them untouched (the reference's ``torch.equal`` test
at :228, without the host synchronisation).

Memory follows ``workspace_budget`` as for FusedLinearCrossEntropy. The
default budget is at least what the reference's chunk loop holds at once
(:133-135,159-203: its chunk's logits, their fp32 log-softmax copies, dX and
dlogits, and the [V, H] product dlogits^T X), so with the same outputs the
default peak memory is at most the reference's.

Differences from the reference, by design:
  * the reference keeps fp32 copies of both logits chunks and of dX
    (:163-188); here the row kernel works from the 16-bit logits in
    registers, in fp32 arithmetic;
  * with room for it (a larger budget), grad_weight is summed in fp32 and
    rounded once (the reference accumulates in the weight dtype, :203);
  * any H, Ht and V (padded inside the workspace);
  * rows labelled ignore_index are compacted away on the device before the
    GEMMs, so they cost no FLOPs (the reference computes their logits);
  * the label count stays on the device (the reference reads it, :139);
  * fp32, bf16 and fp16: the contractions run on fp32 or bf16/fp16 MFMA.
"""
from __future__ import annotations

import torch

from . import _lib
from .cross_entropy import scale_rows_
from .fused_linear_cross_entropy import DEFAULT_CHUNK, plan_dict


def fused_linear_jsd_forward(student_input, student_weight, teacher_input, teacher_weight, labels=None, beta=0.5,
                             temperature=1.0, ignore_index=-100, compute_grad=True, chunk=DEFAULT_CHUNK,
                             workspace_budget=None):
    """Forward (fused_linear_jsd.py:114-205). Returns (loss, grad_input, grad_weight)."""
    si, sw, ti, tw = student_input, student_weight, teacher_input, teacher_weight
    assert si.dim() == 2 and sw.dim() == 2 and si.shape[1] == sw.shape[1], \
        f"expected student input (BT, H) and weight (V, H); got {tuple(si.shape)} and {tuple(sw.shape)}"
    assert ti.dim() == 2 and tw.dim() == 2 and ti.shape[1] == tw.shape[1] and ti.shape[0] == si.shape[0] \
        and tw.shape[0] == sw.shape[0], "expected teacher input (BT, Ht) and weight (V, Ht)"
    if si.dtype not in (torch.bfloat16, torch.float16, torch.float32):
        raise TypeError(f"fused linear JSD takes fp32, bf16 or fp16; got {si.dtype}")
    if not (sw.dtype == ti.dtype == tw.dtype == si.dtype):
        raise TypeError("student and teacher inputs and weights must share one dtype")
    dev = _lib.require_device(si, sw, ti, tw, labels)
    si, sw, ti, tw = si.contiguous(), sw.contiguous(), ti.contiguous(), tw.detach().contiguous()
    ti = ti.detach()
    lab = None
    if labels is not None:
        assert labels.dim() == 1 and labels.shape[0] == si.shape[0]
        lab = labels.contiguous().to(torch.int64)
    BT, H = si.shape
    Ht = ti.shape[1]
    V = sw.shape[0]
    dt = _lib.dtype_code(si)
    loss = torch.empty((), dtype=torch.float32, device=dev)
    grad_input = torch.empty_like(si) if compute_grad else None
    grad_weight = torch.empty_like(sw) if compute_grad else None
    budget = _lib.fl_budget(workspace_budget)
    ws_bytes = _lib.load().hk_fused_linear_jsd_workspace_size(BT, H, Ht, V, int(chunk), budget, dt,
                                                              int(compute_grad), int(lab is not None), si.data_ptr(),
                                                              sw.data_ptr(), ti.data_ptr(), tw.data_ptr())
    ws = _lib.workspace(ws_bytes, "fused linear JSD", dev)
    _lib.call("hk_fused_linear_jsd", loss.data_ptr(), _lib.ptr(grad_input), _lib.ptr(grad_weight), si.data_ptr(),
              sw.data_ptr(), ti.data_ptr(), tw.data_ptr(), _lib.ptr(lab), BT, H, Ht, V, int(ignore_index),
              float(beta), float(temperature), dt, int(chunk), budget, ws.data_ptr(), ws.numel(),
              _lib.stream_of(dev))
    return loss, grad_input, grad_weight


def fused_linear_jsd_plan(BT, H, V, dtype=torch.bfloat16, Ht=None, compute_grad=True, with_labels=False,
                          chunk=DEFAULT_CHUNK, workspace_budget=None):
    """The memory plan a call of that shape takes (not in the reference): the dict fused_linear_cross_entropy_plan
    returns. Ht, the teacher's hidden size, defaults to H."""
    import ctypes
    info = (ctypes.c_int64 * 8)()
    _lib.call("hk_fused_linear_jsd_plan", int(BT), int(H), int(H if Ht is None else Ht), int(V), int(chunk),
              _lib.fl_budget(workspace_budget), _lib._DTYPE_CODE[dtype], int(compute_grad), int(with_labels), None,
              None, None, None, info)
    return plan_dict(info)


class HildaFusedLinearJSDFunction(torch.autograd.Function):
    """Autograd wrapper (fused_linear_jsd.py:212-241)."""

    @staticmethod
    def forward(ctx, student_input, student_weight, teacher_input, teacher_weight, labels, beta, temperature,
                ignore_index, workspace_budget=None):
        compute_grad = student_input.requires_grad or student_weight.requires_grad
        loss, gi, gw = fused_linear_jsd_forward(student_input, student_weight, teacher_input, teacher_weight, labels,
                                                beta, temperature, ignore_index, compute_grad=compute_grad,
                                                workspace_budget=workspace_budget)
        ctx.compute_grad = compute_grad
        ctx.applied = None
        if compute_grad:
            ctx.save_for_backward(gi, gw)
        return loss

    @staticmethod
    def backward(ctx, grad_output):
        none6 = (None,) * 7
        if not ctx.compute_grad:
            return (None, None) + none6
        gi, gw = ctx.saved_tensors
        if ctx.applied is None:
            # in place on the device; returns at once when grad_output == 1
            scale_rows_(gi, gi, grad_output, None, skip_if_one=True)
            scale_rows_(gw, gw, grad_output, None, skip_if_one=True)
            ctx.applied = grad_output.detach()
            return (gi, gw) + none6
        out_i = torch.empty_like(gi)
        out_w = torch.empty_like(gw)
        scale_rows_(out_i, gi, grad_output, ctx.applied)
        scale_rows_(out_w, gw, grad_output, ctx.applied)
        return (out_i, out_w) + none6


def hilda_fused_linear_jsd(student_input, student_weight, teacher_input, teacher_weight, labels=None, beta=0.5,
                           temperature=1.0, ignore_index=-100, workspace_budget=None):
    """Functional interface: fused linear + JSD loss (fused_linear_jsd.py:244-254).
    workspace_budget (not in the reference): see the module docstring."""
    return HildaFusedLinearJSDFunction.apply(student_input, student_weight, teacher_input, teacher_weight, labels,
                                             beta, temperature, ignore_index, workspace_budget)


class FusedLinearJSDLoss(torch.nn.Module):
    """Fused linear projection + JSD loss for distillation (fused_linear_jsd.py:261-275).
    workspace_budget (not in the reference): see the module docstring."""

    def __init__(self, beta=0.5, temperature=1.0, ignore_index=-100, workspace_budget=None):
        super().__init__()
        self.beta = beta
        self.temperature = temperature
        self.ignore_index = ignore_index
        self.workspace_budget = workspace_budget

    def forward(self, student_input, student_weight, teacher_input, teacher_weight, labels=None):
        return hilda_fused_linear_jsd(student_input, student_weight, teacher_input, teacher_weight, labels,
                                      self.beta, self.temperature, self.ignore_index, self.workspace_budget)
