"""GPU parity: RoPE and SwiGLU HIP kernels against the CPU oracle.

RoPE follows benchmarks/bench_rope.py's checks (fp32 forward, the all-ones
backward known answer, autograd backward) on contiguous and transposed
layouts, per-batch cos/sin tables and the C2 shapes. SwiGLU follows
benchmarks/bench_swiglu.py's forward/backward checks plus odd sizes (scalar
tail) and the C2 shape.
"""
import pytest
import torch

import oracle
import workloads as configs
from _util import assert_close, rel_fro, tol, gpu

from kernels import hilda_rope, hilda_swiglu, RotaryEmbedding, SwiGLU
from kernels import rope as rp

pytestmark = pytest.mark.gpu


def _rope_oracle(q, k, cos, sin, dq, dk):
    prec = torch.float64 if q.dtype == torch.float32 else torch.float32
    outs, grads = oracle.fwd_bwd(oracle.rope_ref, [q, k, cos, sin], [dq, dk], dtype=prec,
                                 differentiable=[True, True, False, False])
    return outs, grads


def _make_qk(B, T, Hq, Hk, D, dtype, layout, g):
    if layout == "bhtd":
        q = torch.randn(B, Hq, T, D, generator=g).to(dtype)
        k = torch.randn(B, Hk, T, D, generator=g).to(dtype)
    else:  # [B,T,H,D] storage, (B,H,T,D) view
        q = torch.randn(B, T, Hq, D, generator=g).to(dtype).transpose(1, 2)
        k = torch.randn(B, T, Hk, D, generator=g).to(dtype).transpose(1, 2)
    return q, k


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("layout", ["bhtd", "bthd"])
@pytest.mark.parametrize("dims", [(2, 64, 8, 2, 128), (1, 33, 4, 4, 64), (3, 17, 5, 1, 96), (2, 9, 3, 3, 10)])
@pytest.mark.parametrize("cos_batched", [False, True])
def test_rope_fwd_bwd(dtype, layout, dims, cos_batched):
    B, T, Hq, Hk, D = dims
    g = torch.Generator().manual_seed(B * 1000 + T)
    q, k = _make_qk(B, T, Hq, Hk, D, dtype, layout, g)
    if cos_batched:  # random per-batch tables, like benchmarks/bench_rope.py:79-80
        cos = torch.randn(B, T, D // 2, generator=g)
        sin = torch.randn(B, T, D // 2, generator=g)
    else:
        cos, sin = oracle.rope_tables(D, T + 5, 500000.0)
        cos, sin = cos[:, :T], sin[:, :T]
    dq = torch.randn(q.shape, generator=g).to(dtype)
    dk = torch.randn(k.shape, generator=g).to(dtype)
    (q_ref, k_ref), (dq_ref, dk_ref, _, _) = _rope_oracle(q, k, cos, sin, dq, dk)

    dev = gpu()
    qg = q.to(dev).requires_grad_(True)
    kg = k.to(dev).requires_grad_(True)
    qo, ko = hilda_rope(qg, kg, cos.to(dev), sin.to(dev))
    assert qo.stride() == qg.stride() and ko.stride() == kg.stride()
    torch.autograd.backward([qo, ko], [dq.to(dev), dk.to(dev)])
    t = tol(dtype)
    assert_close(qo, q_ref, name="q", **t)
    assert_close(ko, k_ref, name="k", **t)
    assert_close(qg.grad, dq_ref, name="dq", **t)
    assert_close(kg.grad, dk_ref, name="dk", **t)


def test_rope_backward_known_answer():
    """benchmarks/bench_rope.py:133-146: backward of an all-ones grad is [cos+sin, cos-sin]."""
    B, T, Hq, Hk, D = 2, 256, 32, 8, 128
    g = torch.Generator().manual_seed(3)
    cos = torch.randn(1, T, D // 2, generator=g)
    sin = torch.randn(1, T, D // 2, generator=g)
    dev = gpu()
    dq = torch.ones(B, Hq, T, D, device=dev)
    dk = torch.ones(B, Hk, T, D, device=dev)
    dq_out, dk_out = rp.rope_backward(dq, dk, cos.to(dev), sin.to(dev))
    c, s = cos.unsqueeze(1), sin.unsqueeze(1)
    exp = torch.cat([c + s, c - s], dim=-1)
    assert_close(dq_out, exp.expand(B, Hq, T, D), name="dq", rtol=1e-5, atol=1e-5)
    assert_close(dk_out, exp.expand(B, Hk, T, D), name="dk", rtol=1e-5, atol=1e-5)


def test_rope_position_zero_identity_and_broadcast_grad():
    """cos=1, sin=0 at position 0 gives y = x exactly; a zero-stride grad (from sum()) works."""
    rot = RotaryEmbedding(64, max_position_embeddings=32, base=500000).to(gpu())
    cos, sin = rot(None, seq_len=32)
    q = torch.randn(2, 4, 32, 64, device=gpu(), dtype=torch.bfloat16, requires_grad=True)
    k = torch.randn(2, 2, 32, 64, device=gpu(), dtype=torch.bfloat16, requires_grad=True)
    qo, ko = rot.apply_rotary(q, k, cos, sin)
    assert torch.equal(qo[:, :, 0], q[:, :, 0]) and torch.equal(ko[:, :, 0], k[:, :, 0])
    (qo.sum() + ko.sum()).backward()
    cf, sf = oracle.rope_tables(64, 32, 500000.0)
    c, s = cf.unsqueeze(1), sf.unsqueeze(1)
    exp = torch.cat([c + s, c - s], dim=-1)
    assert_close(q.grad, exp.expand(2, 4, 32, 64), name="dq", **tol(torch.bfloat16))
    assert_close(k.grad, exp.expand(2, 2, 32, 64), name="dk", **tol(torch.bfloat16))


def test_rotary_embedding_buffers():
    """Buffers keep the reference names and shapes so state dicts interchange."""
    rot = RotaryEmbedding(128, max_position_embeddings=64, base=500000)
    assert set(dict(rot.named_buffers())) == {"inv_freq", "cos_cached", "sin_cached"}
    assert rot.cos_cached.shape == (1, 64, 64)
    c, s = oracle.rope_tables(128, 64, 500000.0)
    assert torch.allclose(rot.cos_cached, c) and torch.allclose(rot.sin_cached, s)


def test_rope_c2_config():
    """C2 RoPE: q [4,2048,32,128], k [4,2048,8,128] bf16 in [B,T,H,D] storage, theta 500000."""
    c = configs.c2_rope()
    (q_ref, k_ref), (dq_ref, dk_ref, _, _) = _rope_oracle(c["q"], c["k"], c["cos"], c["sin"], c["dq"], c["dk"])
    dev = gpu()
    q = c["q"].to(dev).requires_grad_(True)  # .to() keeps the transposed strides
    k = c["k"].to(dev).requires_grad_(True)
    assert q.stride() == c["q"].stride()
    qo, ko = hilda_rope(q, k, c["cos"].to(dev), c["sin"].to(dev))
    torch.autograd.backward([qo, ko], [c["dq"].to(dev), c["dk"].to(dev)])
    t = tol(torch.bfloat16)
    assert_close(qo, q_ref, name="q", **t)
    assert_close(ko, k_ref, name="k", **t)
    assert_close(q.grad, dq_ref, name="dq", **t)
    assert_close(k.grad, dk_ref, name="dk", **t)


# --------------------------------------------------------------------------
# SwiGLU
# --------------------------------------------------------------------------
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("shape", [(4, 128, 1024), (2, 33, 1001), (3, 14336), (7,)])
def test_swiglu(dtype, shape):
    g = torch.Generator().manual_seed(len(shape) * 100 + shape[-1])
    a = (2 * torch.randn(*shape, generator=g)).to(dtype)
    b = torch.randn(*shape, generator=g).to(dtype)
    dc = torch.randn(*shape, generator=g).to(dtype)
    prec = torch.float64 if dtype == torch.float32 else torch.float32
    (c_ref,), (da_ref, db_ref) = oracle.fwd_bwd(oracle.swiglu_ref, [a, b], [dc], dtype=prec)
    dev = gpu()
    ag = a.to(dev).requires_grad_(True)
    bg = b.to(dev).requires_grad_(True)
    c = SwiGLU()(ag, bg)
    c.backward(dc.to(dev))
    t = tol(dtype)
    assert_close(c, c_ref, name="c", **t)
    assert_close(ag.grad, da_ref, name="da", **t)
    assert_close(bg.grad, db_ref, name="db", **t)
    # the saved inputs are not overwritten by the backward
    assert torch.equal(ag.detach().cpu(), a) and torch.equal(bg.detach().cpu(), b)


def test_swiglu_zero_gate():
    """a = 0: c = 0 and da = 0.5 * dc * b (silu'(0) = 1/2), db = 0."""
    b = torch.randn(64, 256, device=gpu())
    dc = torch.randn(64, 256, device=gpu())
    a = torch.zeros(64, 256, device=gpu(), requires_grad=True)
    bg = b.clone().requires_grad_(True)
    c = hilda_swiglu(a, bg)
    c.backward(dc)
    assert torch.count_nonzero(c).item() == 0
    assert_close(a.grad, 0.5 * dc * b, name="da", rtol=1e-6, atol=1e-6)
    assert torch.count_nonzero(bg.grad).item() == 0


def test_swiglu_c2_config():
    """C2 SwiGLU bf16 gate/up [8192, 14336]."""
    c = configs.c2_swiglu()
    (c_ref,), (da_ref, db_ref) = oracle.fwd_bwd(oracle.swiglu_ref, [c["a"], c["b"]], [c["dc"]])
    dev = gpu()
    a = c["a"].to(dev).requires_grad_(True)
    b = c["b"].to(dev).requires_grad_(True)
    out = hilda_swiglu(a, b)
    out.backward(c["dc"].to(dev))
    t = tol(torch.bfloat16)
    assert_close(out, c_ref, name="c", **t)
    assert_close(a.grad, da_ref, name="da", **t)
    assert_close(b.grad, db_ref, name="db", **t)
    assert rel_fro(a.grad, da_ref) < 1e-2
