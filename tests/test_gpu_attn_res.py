"""GPU parity: the AttnRes HIP kernels against the CPU oracle.

Follows benchmarks/bench_attn_res.py's forward and backward checks (its
configs (N, B, T, D) = (4|8, 2, 64, 4096|8192) in fp16/bf16/fp32, lines 72-135,
against pytorch_attn_res with autograd) and adds odd D, every block count
bound (1, 8, 9, 16, 17, 32), a list of blocks as input, w_norm != 1 and the
module's parameters. The shapes reach every kernel form: register-resident
with 256 or 512 lanes per token (full and partial last packs) and streaming.
"""
import pytest
import torch

import oracle
from _util import assert_close, rel_fro, tol, gpu

from kernels import hilda_attn_res, AttnRes

pytestmark = pytest.mark.gpu


def _case(N, B, T, D, dtype, seed, wn_ones=False):
    g = torch.Generator().manual_seed(seed)
    V = torch.randn(N, B, T, D, generator=g).to(dtype)
    wq = (0.02 * torch.randn(D, generator=g)).to(dtype) if not wn_ones else (torch.randn(D, generator=g) / D ** 0.5).to(dtype)
    wn = torch.ones(D).to(dtype) if wn_ones else (1 + 0.1 * torch.randn(D, generator=g)).to(dtype)
    dh = torch.randn(B, T, D, generator=g).to(dtype)
    return V, wq, wn, dh


def _check(V, wq, wn, dh, dtype):
    prec = torch.float64 if dtype == torch.float32 else torch.float32
    # keys rounded to the input dtype as the reference does; the rest in fp32 (fp64 for fp32 inputs)
    (h_ref,), (dv_ref, dq_ref, dn_ref) = oracle.fwd_bwd(
        lambda v, q, n: oracle.attn_res_ref(v, q, n, key_dtype=dtype), [V, wq, wn], [dh], dtype=prec)
    dev = gpu()
    Vg = V.to(dev).requires_grad_(True)
    qg = wq.to(dev).requires_grad_(True)
    ng = wn.to(dev).requires_grad_(True)
    h = hilda_attn_res(Vg, qg, ng)
    h.backward(dh.to(dev))
    t = tol(dtype)
    assert_close(h, h_ref, name="h", **t)
    assert_close(Vg.grad, dv_ref, name="dV", **t)
    # dW sums over every token: compare relative to their size
    assert rel_fro(qg.grad, dq_ref) < (1e-5 if dtype == torch.float32 else 2e-2), "dW_query"
    assert rel_fro(ng.grad, dn_ref) < (1e-5 if dtype == torch.float32 else 2e-2), "dW_norm"


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("N,D", [(1, 256), (4, 4096), (8, 4096), (9, 1000), (17, 520), (32, 2048), (8, 8192),
                                 (16, 4096), (8, 6000), (16, 3000)])
def test_attn_res(dtype, N, D):
    if dtype == torch.float32 and D > 8 * 256 * 4:
        pytest.skip("fp32 rows are limited to 8192 columns")
    V, wq, wn, dh = _case(N, 2, 64, D, dtype, N * 1000 + D)
    _check(V, wq, wn, dh, dtype)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_attn_res_reference_bench_configs(dtype):
    """bench_attn_res.py:100-109: w_query = 0.02 N(0,1), w_norm = 1, upstream h.sum()."""
    g = torch.Generator().manual_seed(7)
    V = torch.randn(4, 2, 64, 4096, generator=g).to(dtype)
    wq = (0.02 * torch.randn(4096, generator=g)).to(dtype)
    wn = torch.ones(4096).to(dtype)
    _check(V, wq, wn, torch.ones(2, 64, 4096).to(dtype), dtype)


def test_attn_res_list_input_and_module():
    dev = gpu()
    torch.manual_seed(3)
    m = AttnRes(512).to(dev)
    blocks = [torch.randn(2, 8, 512, device=dev) for _ in range(5)]
    h = m(blocks)
    ref = oracle.attn_res_ref(torch.stack(blocks).cpu().double(), m.w_query.detach().cpu().double(),
                              m.w_norm.detach().cpu().double())
    assert h.shape == (2, 8, 512)
    assert_close(h, ref, name="h", rtol=1e-5, atol=1e-5)
    h.sum().backward()
    assert m.w_query.grad.shape == (512,) and m.w_norm.grad.shape == (512,)


def test_attn_res_single_block_identity():
    """N = 1: alpha = 1, h = v, dV = dh, dW = 0."""
    dev = gpu()
    V = torch.randn(1, 3, 7, 256, device=dev, requires_grad=True)
    wq = torch.randn(256, device=dev, requires_grad=True)
    wn = torch.ones(256, device=dev, requires_grad=True)
    h = hilda_attn_res(V, wq, wn)
    dh = torch.randn_like(h)
    h.backward(dh)
    assert_close(h, V.detach()[0], name="h", rtol=1e-6, atol=1e-6)
    assert_close(V.grad[0], dh, name="dV", rtol=1e-6, atol=1e-6)
    assert wq.grad.abs().max().item() < 1e-6 and wn.grad.abs().max().item() < 1e-6
