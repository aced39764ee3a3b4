"""GPU parity: the GeGLU HIP kernels against the CPU oracle.

Follows benchmarks/bench_geglu.py's forward and backward checks (its shapes
[512, 11008|14336|28672] in fp16/bf16 and [512, 4096|14336] in fp32, lines
50-57 and 80-84) plus odd sizes (scalar tail), the zero gate, both tails of
the activation and the [8192, 14336] bf16 shape of the reference's benchmark
(bench_geglu.py:185-190).
"""
import pytest
import torch

import oracle
from _util import assert_close, rel_fro, tol, gpu

from kernels import hilda_geglu, GeGLU

pytestmark = pytest.mark.gpu


def _check(a, b, dc, dtype, module=False):
    prec = torch.float64 if dtype == torch.float32 else torch.float32
    (c_ref,), (da_ref, db_ref) = oracle.fwd_bwd(oracle.geglu_ref, [a, b], [dc], dtype=prec)
    dev = gpu()
    ag = a.to(dev).requires_grad_(True)
    bg = b.to(dev).requires_grad_(True)
    c = GeGLU()(ag, bg) if module else hilda_geglu(ag, bg)
    c.backward(dc.to(dev))
    t = tol(dtype)
    assert_close(c, c_ref, name="c", **t)
    assert_close(ag.grad, da_ref, name="da", **t)
    assert_close(bg.grad, db_ref, name="db", **t)
    # the saved inputs are not overwritten by the backward
    assert torch.equal(ag.detach().cpu(), a) and torch.equal(bg.detach().cpu(), b)
    return ag.grad, da_ref


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("shape", [(4, 128, 1024), (2, 33, 1001), (3, 14336), (7,)])
def test_geglu(dtype, shape):
    g = torch.Generator().manual_seed(len(shape) * 100 + shape[-1] + 7)
    a = (2 * torch.randn(*shape, generator=g)).to(dtype)
    b = torch.randn(*shape, generator=g).to(dtype)
    dc = torch.randn(*shape, generator=g).to(dtype)
    _check(a, b, dc, dtype, module=True)


@pytest.mark.parametrize("dtype,D", [(torch.float16, 11008), (torch.bfloat16, 14336), (torch.float16, 28672),
                                     (torch.float32, 4096), (torch.float32, 14336)])
def test_geglu_reference_bench_shapes(dtype, D):
    g = torch.Generator().manual_seed(D)
    a = torch.randn(512, D, generator=g).to(dtype)
    b = torch.randn(512, D, generator=g).to(dtype)
    dc = torch.ones(512, D).to(dtype)  # the reference backward check uses out.sum()
    _check(a, b, dc, dtype)


def test_geglu_zero_gate_and_tails():
    """a = 0: c = 0, da = 0.5 dc b (gelu'(0) = 1/2), db = 0; a = +-30: gelu -> a and -> 0."""
    dev = gpu()
    b = torch.randn(64, 256, device=dev)
    dc = torch.randn(64, 256, device=dev)
    a = torch.zeros(64, 256, device=dev, requires_grad=True)
    bg = b.clone().requires_grad_(True)
    c = hilda_geglu(a, bg)
    c.backward(dc)
    assert torch.count_nonzero(c).item() == 0
    assert_close(a.grad, 0.5 * dc * b, name="da", rtol=1e-6, atol=1e-6)
    assert torch.count_nonzero(bg.grad).item() == 0
    big = torch.full((4, 64), 30.0, device=dev)
    big[1::2] = -30.0
    ag = big.clone().requires_grad_(True)
    bg = torch.ones_like(big, requires_grad=True)
    c = hilda_geglu(ag, bg)
    c.backward(torch.ones_like(c))
    assert_close(c, torch.where(big > 0, big, torch.zeros_like(big)), name="tails", rtol=1e-6, atol=1e-6)
    assert_close(ag.grad, (big > 0).float(), name="da tails", rtol=1e-6, atol=1e-6)


def test_geglu_empty():
    a = torch.empty(0, 16, device=gpu(), requires_grad=True)
    b = torch.empty(0, 16, device=gpu(), requires_grad=True)
    c = hilda_geglu(a, b)
    c.sum().backward()
    assert c.shape == (0, 16) and a.grad.shape == (0, 16)


def test_geglu_mistral_shape():
    """bf16 [8192, 14336], the reference benchmark's Mistral-7B row."""
    g = torch.Generator().manual_seed(14336)
    a = torch.randn(8192, 14336, generator=g).to(torch.bfloat16)
    b = torch.randn(8192, 14336, generator=g).to(torch.bfloat16)
    dc = torch.randn(8192, 14336, generator=g).to(torch.bfloat16)
    da, da_ref = _check(a, b, dc, torch.bfloat16)
    assert rel_fro(da, da_ref) < 1e-2
