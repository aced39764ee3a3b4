"""RoPE on MI355X (rotate-half convention), forward and backward.

Drop-in for ``kernels/rope.py`` of the reference (rope.py:90-228). q and k
are (bsz, n_heads, seq_len, head_dim) with any strides in the first three
dims (e.g. the transposed view of [B, T, H, D] storage); outputs keep the
input layout and no copy is made in either direction — the reference's
backward copies non-contiguous grads (rope.py:156-159) and builds a negated
sin table (:164); here the kernel takes the sign as an argument.
"""
from __future__ import annotations

import torch

from . import _lib


def _launch(x_in, x_out, cos, sin, inverse):
    bsz, n_heads, seq_len, hd = x_in.shape
    if x_in.numel() == 0:
        return
    if x_in.stride(-1) != 1:
        x_in = x_in.contiguous()
    assert x_out.stride(-1) == 1
    assert cos.shape == sin.shape and cos.dim() == 3 and cos.shape[-1] == hd // 2, \
        f"cos/sin must be (1 or bsz, seq, head_dim/2); got {tuple(cos.shape)}"
    assert cos.shape[1] >= seq_len, f"cos/sin cover {cos.shape[1]} positions, need {seq_len}"
    assert cos.shape[0] in (1, bsz)
    assert cos.dtype == sin.dtype and cos.stride() == sin.stride()
    _lib.call("hk_rope", x_out.data_ptr(), x_in.data_ptr(), cos.data_ptr(), sin.data_ptr(),
              bsz, n_heads, seq_len, hd,
              x_in.stride(0), x_in.stride(1), x_in.stride(2),
              x_out.stride(0), x_out.stride(1), x_out.stride(2),
              cos.shape[0], cos.stride(0), cos.stride(1),
              _lib.dtype_code(x_in), _lib.dtype_code(cos), int(inverse), _lib.stream_of(x_in.device))


def _launch_qk(q_in, q_out, k_in, k_out, cos, sin, inverse):
    """q and k in one launch when they share batch, positions, head_dim and dtype."""
    bsz, hq, seq_len, hd = q_in.shape
    same = (k_in.shape[0] == bsz and k_in.shape[2] == seq_len and k_in.shape[3] == hd and k_in.dtype == q_in.dtype
            and q_in.stride(-1) == 1 and k_in.stride(-1) == 1)
    if not same or q_in.numel() == 0 or k_in.numel() == 0:
        _launch(q_in, q_out, cos, sin, inverse)
        _launch(k_in, k_out, cos, sin, inverse)
        return
    assert q_out.stride(-1) == 1 and k_out.stride(-1) == 1
    assert cos.shape == sin.shape and cos.dim() == 3 and cos.shape[-1] == hd // 2, \
        f"cos/sin must be (1 or bsz, seq, head_dim/2); got {tuple(cos.shape)}"
    assert cos.shape[1] >= seq_len, f"cos/sin cover {cos.shape[1]} positions, need {seq_len}"
    assert cos.shape[0] in (1, bsz)
    assert cos.dtype == sin.dtype and cos.stride() == sin.stride()
    _lib.call("hk_rope_qk", q_out.data_ptr(), q_in.data_ptr(), hq,
              q_in.stride(0), q_in.stride(1), q_in.stride(2), q_out.stride(0), q_out.stride(1), q_out.stride(2),
              k_out.data_ptr(), k_in.data_ptr(), k_in.shape[1],
              k_in.stride(0), k_in.stride(1), k_in.stride(2), k_out.stride(0), k_out.stride(1), k_out.stride(2),
              cos.data_ptr(), sin.data_ptr(), bsz, seq_len, hd, cos.shape[0], cos.stride(0), cos.stride(1),
              _lib.dtype_code(q_in), _lib.dtype_code(cos), int(inverse), _lib.stream_of(q_in.device))


def _tables(cos, sin):
    if cos.stride(-1) != 1:
        cos = cos.contiguous()
    if sin.stride(-1) != 1 or sin.stride() != cos.stride():
        sin = sin.contiguous()
        cos = cos.contiguous()
    return cos, sin


def rope_forward(q, k, cos, sin):
    """Forward (rope.py:113-136): returns q_out, k_out (new tensors), cos, sin."""
    _lib.require_device(q, k, cos, sin)
    cos, sin = _tables(cos, sin)
    q_out = torch.empty_like(q)
    k_out = torch.empty_like(k)
    _launch_qk(q, q_out, k, k_out, cos, sin, inverse=False)
    return q_out, k_out, cos, sin


def rope_backward(dq, dk, cos, sin):
    """Backward (rope.py:139-172): the transpose rotation, i.e. the forward with -sin."""
    _lib.require_device(dq, dk, cos, sin)
    cos, sin = _tables(cos, sin)
    # empty_like keeps a dense input's layout and is contiguous for broadcast (zero-stride) grads
    dq_out = torch.empty_like(dq)
    dk_out = torch.empty_like(dk)
    _launch_qk(dq, dq_out, dk, dk_out, cos, sin, inverse=True)
    return dq_out, dk_out


class HildaRopeFunction(torch.autograd.Function):
    """Autograd wrapper (rope.py:179-197): q, k = HildaRopeFunction.apply(q, k, cos, sin)."""

    @staticmethod
    def forward(ctx, q, k, cos, sin):
        q_out, k_out, cos, sin = rope_forward(q, k, cos, sin)
        ctx.save_for_backward(cos, sin)
        return q_out, k_out

    @staticmethod
    def backward(ctx, dq, dk):
        cos, sin = ctx.saved_tensors
        dq_out, dk_out = rope_backward(dq, dk, cos, sin)
        return dq_out, dk_out, None, None


def hilda_rope(q, k, cos, sin):
    """Functional interface for RoPE (rope.py:200-202)."""
    return HildaRopeFunction.apply(q, k, cos, sin)


class RotaryEmbedding(torch.nn.Module):
    """cos/sin cache module (rope.py:209-228); buffers inv_freq, cos_cached, sin_cached
    of shape (1, max_position_embeddings, dim // 2)."""

    def __init__(self, dim, max_position_embeddings=2048, base=10000, device=None):
        super().__init__()
        self.dim = dim
        inv_freq = 1.0 / (base ** (torch.arange(0, dim, 2, dtype=torch.float32, device=device) / dim))
        self.register_buffer("inv_freq", inv_freq)
        self._set_cos_sin_cache(max_position_embeddings, device)

    def _set_cos_sin_cache(self, seq_len, device):
        t = torch.arange(seq_len, device=device, dtype=self.inv_freq.dtype)
        freqs = torch.outer(t, self.inv_freq)
        emb = torch.cat((freqs, freqs), dim=-1)
        self.register_buffer("cos_cached", emb.cos()[None, :, : self.dim // 2])
        self.register_buffer("sin_cached", emb.sin()[None, :, : self.dim // 2])

    def forward(self, x, seq_len=None):
        return self.cos_cached[:, :seq_len], self.sin_cached[:, :seq_len]

    def apply_rotary(self, q, k, cos, sin):
        return hilda_rope(q, k, cos, sin)
