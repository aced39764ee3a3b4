"""GRPO loss (PPO-clip + KL) and selective log-softmax on MI355X.

Drop-in for ``kernels/grpo_loss.py`` of the reference (grpo_loss.py:65-397).

The forward reads each unmasked row of the (B, L+1, V) logits once and, when
the logits require grad, writes that row's gradient in the same pass at unit
upstream gradient (the reference re-reads every row in a separate backward
kernel and zeroes the last position in a third pass, grpo_loss.py:300-330).
Masked tokens and position L get zero gradient rows from the same kernel.
The backward scales the saved gradient in place by the upstream gradient on
the device; a unit gradient (``loss.backward()``) costs one tiny launch.

Per-sequence means, kl_mean and clip_ratio follow grpo_loss.py:290-295; the
mask may be bool/uint8/int32/int64/float (non-binary values weight tokens as
the reference's ``mask.float()`` does).
"""
from __future__ import annotations

import torch

from . import _lib
from .cross_entropy import scale_rows_


def _mask_arg(mask):
    if mask is None:
        return None, 0, 0, 0
    try:
        code = _lib.mask_code(mask)
    except TypeError:
        mask = mask.to(torch.float32)
        code = _lib.mask_code(mask)
    return mask, code, mask.stride(0), mask.stride(1)


def _ids_arg(ids):
    if ids.dtype != torch.int64:
        ids = ids.to(torch.int64)
    return ids


def _f32(t):
    if t is None:
        return None
    return t if t.dtype == torch.float32 else t.to(torch.float32)


@torch.no_grad()
def fused_selective_log_softmax(logits, input_ids, temperature=1.0, mask=None):
    """log_softmax(logits[:, :-1] / T) at input_ids[:, -L:] (grpo_loss.py:65-80); 0 where masked."""
    assert logits.is_contiguous()
    B, L_plus_1, N = logits.shape
    L = L_plus_1 - 1
    _lib.require_device(logits, input_ids, mask)
    input_ids = _ids_arg(input_ids[:, -L:] if L > 0 else input_ids[:, :0])
    if mask is not None:
        mask = mask[:, -L:] if L > 0 else mask[:, :0]
    mask, mcode, msb, msl = _mask_arg(mask)
    log_p = torch.empty(B, L, dtype=torch.float32, device=logits.device)
    _lib.call("hk_selective_log_softmax", log_p.data_ptr(), logits.data_ptr(), input_ids.data_ptr(),
              input_ids.stride(0), input_ids.stride(1), _lib.ptr(mask), mcode, msb, msl, B, L, N,
              float(temperature), _lib.dtype_code(logits), _lib.stream_of(logits.device))
    return log_p


def grpo_loss_forward(logits, completion_ids, advantages, old_logp=None, ref_logp=None, completion_mask=None,
                      temperature=1.0, beta=0.0, eps_low=0.2, eps_high=0.2, compute_grad=False):
    """Forward (grpo_loss.py:241-297), with the gradient fused in when compute_grad.

    Returns (loss, kl_mean or None, clip_ratio, lse, dlogits or None).
    """
    assert logits.is_contiguous()
    B, L_plus_1, N = logits.shape
    L = L_plus_1 - 1
    if beta != 0.0 and ref_logp is None:
        raise ValueError("beta != 0 needs ref_logp")
    dev = _lib.require_device(logits, completion_ids, advantages, old_logp, ref_logp, completion_mask)
    ids = _ids_arg(completion_ids)
    adv = _f32(advantages).contiguous()
    old = _f32(old_logp)
    ref = _f32(ref_logp)
    mask, mcode, msb, msl = _mask_arg(completion_mask)
    f32 = dict(dtype=torch.float32, device=dev)
    loss = torch.empty((), **f32)
    kl_mean = torch.empty((), **f32) if beta != 0.0 else None
    clip_ratio = torch.empty((), **f32)
    lse = torch.empty(B, L, **f32)
    loss_rows = torch.empty(B, L, **f32)
    kl_rows = torch.empty(B, L, **f32)
    clip_rows = torch.empty(B, L, **f32)
    dlogits = torch.empty_like(logits) if compute_grad else None
    ws_bytes = _lib.load().hk_grpo_workspace_size(B, L)
    ws = torch.empty(max(int(ws_bytes), 256), dtype=torch.uint8, device=dev)
    _lib.call("hk_grpo_loss_fwd", _lib.ptr(dlogits), loss.data_ptr(), _lib.ptr(kl_mean), clip_ratio.data_ptr(),
              lse.data_ptr(), loss_rows.data_ptr(), kl_rows.data_ptr(), clip_rows.data_ptr(), logits.data_ptr(),
              ids.data_ptr(), ids.stride(0), ids.stride(1), adv.data_ptr(),
              _lib.ptr(old), old.stride(0) if old is not None else 0, old.stride(1) if old is not None else 0,
              _lib.ptr(ref), ref.stride(0) if ref is not None else 0, ref.stride(1) if ref is not None else 0,
              _lib.ptr(mask), mcode, msb, msl, B, L, N, float(temperature), float(beta), float(eps_low),
              float(eps_high), _lib.dtype_code(logits), ws.data_ptr(), ws.numel(), _lib.stream_of(dev))
    return loss, kl_mean, clip_ratio, lse, dlogits


def grpo_loss_backward(grad_output, dlogits, prev_grad=None):
    """Backward: the forward already holds dloss/dlogits at unit upstream gradient
    (grpo_loss.py:300-330 computes the same quantity in a separate pass)."""
    rows = dlogits.view(-1, dlogits.shape[-1])
    if prev_grad is None:
        scale_rows_(rows, rows, grad_output, None, skip_if_one=True)
        return dlogits
    out = torch.empty_like(dlogits)
    scale_rows_(out.view(-1, out.shape[-1]), rows, grad_output, prev_grad)
    return out


class HildaGRPOLossFunction(torch.autograd.Function):
    """Autograd wrapper (grpo_loss.py:337-362): returns (loss, kl_mean, clip_ratio);
    only loss is differentiable."""

    @staticmethod
    def forward(ctx, logits, completion_ids, advantages, old_logp, ref_logp, completion_mask, temperature, beta,
                eps_low, eps_high):
        compute_grad = logits.requires_grad
        loss, kl_mean, clip_ratio, lse, dlogits = grpo_loss_forward(
            logits, completion_ids, advantages, old_logp, ref_logp, completion_mask, temperature, beta, eps_low,
            eps_high, compute_grad=compute_grad)
        ctx.compute_grad = compute_grad
        ctx.applied = None
        if compute_grad:
            ctx.save_for_backward(dlogits)
        if kl_mean is not None:
            ctx.mark_non_differentiable(kl_mean, clip_ratio)
        else:
            ctx.mark_non_differentiable(clip_ratio)
        return loss, kl_mean, clip_ratio

    @staticmethod
    def backward(ctx, grad_loss, grad_kl, grad_clip):
        nones = (None,) * 9
        if not ctx.compute_grad or grad_loss is None:
            return (None,) + nones
        (dlogits,) = ctx.saved_tensors
        out = grpo_loss_backward(grad_loss, dlogits, ctx.applied)
        if ctx.applied is None:
            ctx.applied = grad_loss.detach()
        return (out,) + nones


def hilda_grpo_loss(logits, completion_ids, advantages, old_logp=None, ref_logp=None, completion_mask=None,
                    temperature=1.0, beta=0.0, eps_low=0.2, eps_high=0.2):
    """Functional interface: GRPO loss (grpo_loss.py:365-375)."""
    return HildaGRPOLossFunction.apply(logits, completion_ids, advantages, old_logp, ref_logp, completion_mask,
                                       temperature, beta, eps_low, eps_high)


class GRPOLoss(torch.nn.Module):
    """GRPO loss module (grpo_loss.py:382-397)."""

    def __init__(self, temperature=1.0, beta=0.0, eps_low=0.2, eps_high=0.2):
        super().__init__()
        self.temperature = temperature
        self.beta = beta
        self.eps_low = eps_low
        self.eps_high = eps_high

    def forward(self, logits, completion_ids, advantages, old_logp=None, ref_logp=None, completion_mask=None):
        return hilda_grpo_loss(logits, completion_ids, advantages, old_logp, ref_logp, completion_mask,
                               self.temperature, self.beta, self.eps_low, self.eps_high)
