"""AttnRes (attention residuals over depth) on MI355X.

Drop-in for ``kernels/attn_res.py`` of the reference (attn_res.py:209-346):
blocks [N, B, T, D] (or a list of N [B, T, D]) -> h [B, T, D], with
k_i = RMSNorm(v_i) * w_norm, scores <w_query, k_i>, a softmax over the N
blocks and h = sum_i alpha_i v_i. One HIP kernel per direction; the backward
sums dW_query / dW_norm over tokens from per-block partial rows (fp64 sum)
instead of per-token fp32 atomics (attn_res.py:189-190).
"""
from __future__ import annotations

import torch

from . import _lib


def _stack(blocks):
    return torch.stack(list(blocks)) if isinstance(blocks, (list, tuple)) else blocks


def attn_res_forward(blocks, w_query, w_norm, eps=1e-6):
    """Forward (attn_res.py:209-257). Returns (h, V_3d, alpha, rstd)."""
    V = _stack(blocks)
    dev = _lib.require_device(V, w_query, w_norm)
    N, D = V.shape[0], V.shape[-1]
    if not (w_query.dtype == w_norm.dtype == V.dtype):
        raise TypeError(f"blocks ({V.dtype}), w_query ({w_query.dtype}) and w_norm ({w_norm.dtype}) must share "
                        f"one dtype")
    V3 = V.reshape(N, -1, D).contiguous()
    ntok = V3.shape[1]
    out = torch.empty(ntok, D, device=dev, dtype=V.dtype)
    alpha = torch.empty(N, ntok, device=dev, dtype=torch.float32)
    rstd = torch.empty(N, ntok, device=dev, dtype=torch.float32)
    _lib.call("hk_attn_res_fwd", out.data_ptr(), alpha.data_ptr(), rstd.data_ptr(), V3.data_ptr(),
              w_query.contiguous().data_ptr(), w_norm.contiguous().data_ptr(), N, ntok, D, float(eps),
              _lib.dtype_code(V3), _lib.stream_of(dev))
    return out.view(list(V.shape[1:])), V3, alpha, rstd


def attn_res_backward(dh, V_3d, w_query, w_norm, alpha, rstd, eps=1e-6):
    """Backward (attn_res.py:260-288). Returns (dV [N, B*T, D], dW_query, dW_norm)."""
    dev = _lib.require_device(dh, V_3d)
    N, ntok, D = V_3d.shape
    dh2 = dh.contiguous().reshape(ntok, D)
    if dh2.dtype != V_3d.dtype:
        dh2 = dh2.to(V_3d.dtype)
    dV = torch.empty_like(V_3d)
    dwq = torch.empty(D, device=dev, dtype=w_query.dtype)
    dwn = torch.empty(D, device=dev, dtype=w_norm.dtype)
    ws = torch.empty(max(int(_lib.load().hk_attn_res_bwd_workspace_size(ntok, D)), 16), dtype=torch.uint8,
                     device=dev)
    _lib.call("hk_attn_res_bwd", dV.data_ptr(), dwq.data_ptr(), dwn.data_ptr(), dh2.data_ptr(), V_3d.data_ptr(),
              w_query.contiguous().data_ptr(), w_norm.contiguous().data_ptr(), alpha.data_ptr(), rstd.data_ptr(), N,
              ntok, D, _lib.dtype_code(V_3d), ws.data_ptr(), ws.numel(), _lib.stream_of(dev))
    return dV, dwq, dwn


class HildaAttnResFunction(torch.autograd.Function):
    """Autograd wrapper (attn_res.py:295-312)."""

    @staticmethod
    def forward(ctx, V_stacked, w_query, w_norm, eps):
        ctx.orig_shape = V_stacked.shape
        h, V3, alpha, rstd = attn_res_forward(V_stacked, w_query, w_norm, eps)
        ctx.save_for_backward(V3, w_query, w_norm, alpha, rstd)
        ctx.eps = eps
        return h

    @staticmethod
    def backward(ctx, dh):
        V3, w_query, w_norm, alpha, rstd = ctx.saved_tensors
        dV, dwq, dwn = attn_res_backward(dh, V3, w_query, w_norm, alpha, rstd, ctx.eps)
        return dV.view(ctx.orig_shape), dwq, dwn, None


def hilda_attn_res(blocks, w_query, w_norm, eps=1e-6):
    """Functional interface: blocks [N, B, T, D] or a list of [B, T, D] -> [B, T, D] (attn_res.py:315-327)."""
    return HildaAttnResFunction.apply(_stack(blocks), w_query, w_norm, eps)


class AttnRes(torch.nn.Module):
    """Attention residuals module (attn_res.py:334-346): parameters w_query ~ 0.02 N(0,1), w_norm = 1."""

    def __init__(self, hidden_dim, eps=1e-6):
        super().__init__()
        self.eps = eps
        self.w_query = torch.nn.Parameter(torch.randn(hidden_dim) * 0.02)
        self.w_norm = torch.nn.Parameter(torch.ones(hidden_dim))

    def forward(self, blocks):
        return hilda_attn_res(blocks, self.w_query, self.w_norm, self.eps)
