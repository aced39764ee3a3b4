"""FusedLinear-GRPO (lm_head + GRPO loss) on MI355X.

The reference has no such op: its GRPO loss takes materialised
(B, L+1, V) logits (grpo_loss.py:241-397). This puts that loss behind the
lm_head the way FusedLinearCrossEntropy does (fused_linear_cross_entropy.py:
103-171): the logits are produced `chunk` rows at a time by a bf16/fp16 MFMA
GEMM, turned into the GRPO gradient in place by the same row kernel as
``hilda_grpo_loss``, and contracted back into dhidden and dweight by two more
MFMA GEMMs. At Qwen-size vocabularies (V = 151936) and B*(L+1) = 16K rows the
logits alone would be 5 GB of bf16.

Arguments mirror ``hilda_grpo_loss`` with (hidden, weight) in place of
logits: hidden is (B, L+1, H), the states whose lm_head logits GRPOLoss would
take; weight is the lm_head [V, H]. Returns (loss, kl_mean, clip_ratio); only
loss is differentiable. All gradient work happens in the forward; the
backward scales the saved gradients by the upstream gradient on the device.
Memory follows ``workspace_budget`` as for FusedLinearCrossEntropy; any H and V.
"""
from __future__ import annotations

import torch

from . import _lib
from .cross_entropy import scale_rows_
from .fused_linear_cross_entropy import plan_dict
from .grpo_loss import _f32, _ids_arg, _mask_arg

DEFAULT_CHUNK = 0  # no cap: the workspace budget sets the chunk (at most 8192 rows)


def fused_linear_grpo_forward(hidden, weight, completion_ids, advantages, old_logp=None, ref_logp=None,
                              completion_mask=None, temperature=1.0, beta=0.0, eps_low=0.2, eps_high=0.2,
                              compute_grad=True, chunk=DEFAULT_CHUNK, workspace_budget=None):
    """Returns (loss, kl_mean or None, clip_ratio, grad_hidden or None, grad_weight or None, rows), rows being
    the per-token (lse, loss, kl, clipped) [B, L] fp32 tensors."""
    assert hidden.dim() == 3 and weight.dim() == 2 and hidden.shape[2] == weight.shape[1], \
        f"expected hidden (B, L+1, H) and weight (V, H); got {tuple(hidden.shape)} and {tuple(weight.shape)}"
    if hidden.dtype != weight.dtype:
        raise TypeError(f"hidden ({hidden.dtype}) and weight ({weight.dtype}) dtypes differ")
    if hidden.dtype not in (torch.bfloat16, torch.float16, torch.float32):
        raise TypeError(f"fused linear GRPO takes fp32, bf16 or fp16; got {hidden.dtype}")
    if beta != 0.0 and ref_logp is None:
        raise ValueError("beta != 0 needs ref_logp")
    dev = _lib.require_device(hidden, weight, completion_ids, advantages, old_logp, ref_logp, completion_mask)
    hidden = hidden.contiguous()
    weight = weight.contiguous()
    B, L_plus_1, H = hidden.shape
    L = L_plus_1 - 1
    V = weight.shape[0]
    ids = _ids_arg(completion_ids)
    adv = _f32(advantages).contiguous()
    old = _f32(old_logp)
    ref = _f32(ref_logp)
    mask, mcode, msb, msl = _mask_arg(completion_mask)
    f32 = dict(dtype=torch.float32, device=dev)
    loss = torch.empty((), **f32)
    kl_mean = torch.empty((), **f32) if beta != 0.0 else None
    clip_ratio = torch.empty((), **f32)
    rows = tuple(torch.empty(B, L, **f32) for _ in range(4))
    grad_hidden = torch.empty_like(hidden) if compute_grad else None
    grad_weight = torch.empty_like(weight) if compute_grad else None
    dt = _lib.dtype_code(hidden)
    budget = _lib.fl_budget(workspace_budget)
    ws_bytes = _lib.load().hk_fused_linear_grpo_workspace_size(B, L, H, V, int(chunk), budget, dt, int(compute_grad),
                                                               hidden.data_ptr(), weight.data_ptr())
    ws = _lib.workspace(ws_bytes, "fused linear GRPO", dev)
    _lib.call("hk_fused_linear_grpo", loss.data_ptr(), _lib.ptr(kl_mean), clip_ratio.data_ptr(),
              *(r.data_ptr() for r in rows), _lib.ptr(grad_hidden), _lib.ptr(grad_weight), hidden.data_ptr(),
              weight.data_ptr(), ids.data_ptr(), ids.stride(0), ids.stride(1), adv.data_ptr(),
              _lib.ptr(old), old.stride(0) if old is not None else 0, old.stride(1) if old is not None else 0,
              _lib.ptr(ref), ref.stride(0) if ref is not None else 0, ref.stride(1) if ref is not None else 0,
              _lib.ptr(mask), mcode, msb, msl, B, L, H, V, float(temperature), float(beta), float(eps_low),
              float(eps_high), dt, int(chunk), budget, ws.data_ptr(), ws.numel(), _lib.stream_of(dev))
    return loss, kl_mean, clip_ratio, grad_hidden, grad_weight, rows


def fused_linear_grpo_plan(B, L, H, V, dtype=torch.bfloat16, compute_grad=True, chunk=DEFAULT_CHUNK,
                           workspace_budget=None):
    """The memory plan a call with B sequences of L completion tokens takes: the dict
    fused_linear_cross_entropy_plan returns (rows per chunk counted over the B*(L+1) positions)."""
    import ctypes
    info = (ctypes.c_int64 * 8)()
    _lib.call("hk_fused_linear_grpo_plan", int(B), int(L), int(H), int(V), int(chunk), _lib.fl_budget(workspace_budget),
              _lib._DTYPE_CODE[dtype], int(compute_grad), None, None, info)
    return plan_dict(info)


class HildaFusedLinearGRPOFunction(torch.autograd.Function):
    """Autograd wrapper: returns (loss, kl_mean, clip_ratio); only loss is differentiable."""

    @staticmethod
    def forward(ctx, hidden, weight, completion_ids, advantages, old_logp, ref_logp, completion_mask, temperature,
                beta, eps_low, eps_high, workspace_budget=None):
        compute_grad = hidden.requires_grad or weight.requires_grad
        loss, kl_mean, clip_ratio, gh, gw, _ = fused_linear_grpo_forward(
            hidden, weight, completion_ids, advantages, old_logp, ref_logp, completion_mask, temperature, beta,
            eps_low, eps_high, compute_grad=compute_grad, workspace_budget=workspace_budget)
        ctx.compute_grad = compute_grad
        ctx.applied = None
        if compute_grad:
            ctx.save_for_backward(gh, gw)
        if kl_mean is not None:
            ctx.mark_non_differentiable(kl_mean, clip_ratio)
        else:
            ctx.mark_non_differentiable(clip_ratio)
        return loss, kl_mean, clip_ratio

    @staticmethod
    def backward(ctx, grad_loss, grad_kl, grad_clip):
        nones = (None,) * 10
        if not ctx.compute_grad or grad_loss is None:
            return (None, None) + nones
        gh, gw = ctx.saved_tensors
        rows_h = gh.view(-1, gh.shape[-1])
        if ctx.applied is None:
            # in place on the device; returns at once when grad_loss == 1
            scale_rows_(rows_h, rows_h, grad_loss, None, skip_if_one=True)
            scale_rows_(gw, gw, grad_loss, None, skip_if_one=True)
            ctx.applied = grad_loss.detach()
            return (gh, gw) + nones
        # repeated backward (retain_graph): new tensors
        out_h = torch.empty_like(gh)
        out_w = torch.empty_like(gw)
        scale_rows_(out_h.view_as(rows_h), rows_h, grad_loss, ctx.applied)
        scale_rows_(out_w, gw, grad_loss, ctx.applied)
        return (out_h, out_w) + nones


def hilda_fused_linear_grpo_loss(hidden, weight, completion_ids, advantages, old_logp=None, ref_logp=None,
                                 completion_mask=None, temperature=1.0, beta=0.0, eps_low=0.2, eps_high=0.2,
                                 workspace_budget=None):
    """Functional interface: GRPO loss of the lm_head logits hidden @ weight.T, without materialising them."""
    return HildaFusedLinearGRPOFunction.apply(hidden, weight, completion_ids, advantages, old_logp, ref_logp,
                                              completion_mask, temperature, beta, eps_low, eps_high, workspace_budget)


class FusedLinearGRPOLoss(torch.nn.Module):
    """GRPOLoss (grpo_loss.py:382-397) over hidden states and the lm_head weight."""

    def __init__(self, temperature=1.0, beta=0.0, eps_low=0.2, eps_high=0.2, workspace_budget=None):
        super().__init__()
        self.temperature = temperature
        self.beta = beta
        self.eps_low = eps_low
        self.eps_high = eps_high
        self.workspace_budget = workspace_budget

    def forward(self, hidden, weight, completion_ids, advantages, old_logp=None, ref_logp=None,
                completion_mask=None):
        return hilda_fused_linear_grpo_loss(hidden, weight, completion_ids, advantages, old_logp, ref_logp,
                                            completion_mask, self.temperature, self.beta, self.eps_low,
                                            self.eps_high, self.workspace_budget)
