"""GPU parity: RMSNorm and FusedAddRMSNorm HIP kernels against the CPU oracle.

Mirrors the reference's tests/test_rms_norm.py cases (shapes x dtypes,
zeros, non-contiguous input, module, upstream grad) and adds the C1/C2
configurations, odd widths, the atomic-vs-partial dW paths and bit-exact S.
"""
import zlib

import pytest
import torch

import oracle
import workloads as configs
from _util import assert_close, rel_fro, tol, gpu

from kernels import rms_norm as rn
from kernels import fused_add_rms_norm as fa
from kernels import hilda_rms_norm, RMSNorm, hilda_fused_add_rms_norm, FusedAddRMSNorm
from kernels import _lib

pytestmark = pytest.mark.gpu

DTYPES = [torch.float32, torch.float16, torch.bfloat16]


def _oracle_rms(x, w, dy, eps=1e-6):
    outs, grads = oracle.fwd_bwd(lambda a, b: oracle.rms_norm_ref(a, b, eps), [x, w], [dy], dtype=torch.float64)
    return outs[0], grads[0], grads[1]


# Rows over 32768 fp32 / 65536 16-bit columns run on the streaming kernels (the reference has no cap: it sizes its
# block with next_power_of_2(n_cols), rms_norm.py:331): (2, 2, 65536) in fp32, and 73728 (vectorised) and 65545
# (scalar tail) in every dtype
@pytest.mark.parametrize("shape", [(2, 128, 1024), (4, 256, 2048), (2, 512, 4096), (3, 7, 1000), (5, 3, 1001),
                                   (1, 3, 12288), (2, 2, 65536), (3, 73728), (2, 65545)])
# (dtype, w_fp32): the 16-bit inputs also with the module's default fp32 weight; fp32 inputs once
@pytest.mark.parametrize("dtype, w_fp32", [(torch.float32, False)] +
                         [(d, w) for d in (torch.float16, torch.bfloat16) for w in (False, True)])
def test_rms_norm_fwd_bwd(shape, dtype, w_fp32):
    g = torch.Generator().manual_seed(zlib.crc32(repr((shape, dtype, w_fp32)).encode()))
    x = torch.randn(*shape, generator=g).to(dtype)
    w = (1 + 0.1 * torch.randn(shape[-1], generator=g)).to(torch.float32 if w_fp32 else dtype)
    dy = torch.randn(*shape, generator=g).to(dtype)
    y_ref, dx_ref, dw_ref = _oracle_rms(x, w, dy)

    dev = gpu()
    xg = x.to(dev).requires_grad_(True)
    wg = w.to(dev).requires_grad_(True)
    y = hilda_rms_norm(xg, wg)
    y.backward(dy.to(dev))
    t = tol(dtype)
    assert y.dtype == dtype and xg.grad.dtype == dtype and wg.grad.dtype == w.dtype
    assert_close(y, y_ref, name="y", **t)
    assert_close(xg.grad, dx_ref, name="dx", **t)
    assert_close(wg.grad, dw_ref, name="dw", **tol(w.dtype if dtype == torch.float32 else dtype))
    assert rel_fro(xg.grad, dx_ref) < (1e-5 if dtype == torch.float32 else 1e-2)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("rows,H", [(100, 2048), (3000, 2048), (5001, 4096), (777, 8192)])
def test_rms_norm_dw_paths_agree(dtype, rows, H):
    """Atomic and partial dW reductions give the same dW (and the same dX).
    The shapes give several rows a group and a last block with empty groups
    (H = 4096: four groups a 1024-lane block summed in LDS; H = 8192: two)."""
    g = torch.Generator().manual_seed(rows)
    dev = gpu()
    x = torch.randn(rows, H, generator=g).to(dtype).to(dev)
    w = (1 + 0.1 * torch.randn(H, generator=g)).to(dtype).to(dev)
    dy = torch.randn(rows, H, generator=g).to(dtype).to(dev)
    _, xf, rstd = rn.rms_norm_forward(x, w)
    dxa, dwa = rn.rms_norm_backward(dy, xf, w, rstd, dw_mode=_lib.DW_ATOMIC)
    dxp, dwp = rn.rms_norm_backward(dy, xf, w, rstd, dw_mode=_lib.DW_PARTIAL)
    assert torch.equal(dxa, dxp)
    _, _, dw_ref = _oracle_rms(x.cpu(), w.cpu(), dy.cpu())
    t = tol(dtype)
    assert_close(dwa, dw_ref, name="dw atomic", **t)
    assert_close(dwp, dw_ref, name="dw partial", **t)
    assert_close(dwa, dwp, name="atomic vs partial", **t)


def test_rms_norm_zeros():
    """tests/test_rms_norm.py:67-78: zeros in -> zeros out."""
    x = torch.zeros(2, 64, 1024, device=gpu(), dtype=torch.float16)
    w = torch.ones(1024, device=gpu(), dtype=torch.float16)
    y = hilda_rms_norm(x, w)
    assert torch.count_nonzero(y).item() == 0


def test_rms_norm_non_contiguous():
    """tests/test_rms_norm.py:80-95: a transposed input works."""
    g = torch.Generator().manual_seed(7)
    x = torch.randn(4, 256, 2048, generator=g).to(torch.float16).transpose(0, 1)
    w = torch.randn(2048, generator=g).to(torch.float16)
    y = hilda_rms_norm(x.to(gpu()), w.to(gpu()))
    assert_close(y, oracle.rms_norm_ref(x.float(), w.float()), name="y", rtol=1e-2, atol=1e-2)


def test_rms_norm_module():
    """tests/test_rms_norm.py:156-203: module forward/backward, in a Sequential."""
    torch.manual_seed(0)
    m = RMSNorm(2048).to(gpu()).to(torch.float16)
    x = torch.randn(2, 128, 2048, device=gpu(), dtype=torch.float16, requires_grad=True)
    y = m(x)
    assert y.shape == x.shape and y.dtype == torch.float16
    y.sum().backward()
    assert x.grad is not None and m.weight.grad is not None
    seq = torch.nn.Sequential(torch.nn.Linear(1024, 1024), RMSNorm(1024), torch.nn.Linear(1024, 1024))
    seq = seq.to(gpu()).to(torch.float16)
    assert seq(torch.randn(2, 64, 1024, device=gpu(), dtype=torch.float16)).shape == (2, 64, 1024)
    # the README spelling
    assert RMSNorm(hidden_size=64).weight.shape == (64,)


def test_rms_norm_c1_config():
    """C1: fp32 [4096, 4096] at the north-star fp32 tolerance (1e-5)."""
    c = configs.c1_rms_norm()
    y_ref, dx_ref, dw_ref = _oracle_rms(c["x"], c["w"], c["dy"], c["eps"])
    dev = gpu()
    x = c["x"].to(dev).requires_grad_(True)
    w = c["w"].to(dev).requires_grad_(True)
    y = hilda_rms_norm(x, w, c["eps"])
    y.backward(c["dy"].to(dev))
    assert_close(y, y_ref, name="y", rtol=1e-5, atol=1e-5)
    assert_close(x.grad, dx_ref, name="dx", rtol=1e-5, atol=1e-5)
    assert_close(w.grad, dw_ref, name="dw", rtol=1e-5, atol=1e-5)


# --------------------------------------------------------------------------
# FusedAddRMSNorm
# --------------------------------------------------------------------------
def _oracle_fused(x, r, w, dy, ds, eps=1e-6):
    """Oracle in fp64 on the residual S = X + R rounded to the input dtype, as both
    the reference (Triton stores s in the input dtype) and the kernel round it.
    d(X + R)/dX = d(X + R)/dR = 1, so dX = dR = dS."""
    s = x + r
    zero = torch.zeros_like(s)
    outs, grads = oracle.fwd_bwd(lambda a, b, c: oracle.fused_add_rms_norm_ref(a, b, c, eps), [s, zero, w],
                                 [dy, ds] if ds is not None else [dy], dtype=torch.float64)
    return (outs[0], s), (grads[0], grads[0], grads[2])


@pytest.mark.parametrize("shape", [(4, 64, 4096), (2, 33, 5120), (3, 5, 1000), (3, 73728), (2, 65545)])
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("with_ds", [True, False])
def test_fused_add_rms_norm(shape, dtype, with_ds):
    g = torch.Generator().manual_seed(11)
    x = torch.randn(*shape, generator=g).to(dtype)
    r = torch.randn(*shape, generator=g).to(dtype)
    w = (1 + 0.02 * torch.randn(shape[-1], generator=g)).to(dtype)
    dy = torch.randn(*shape, generator=g).to(dtype)
    ds = torch.randn(*shape, generator=g).to(dtype) if with_ds else None
    (y_ref, s_ref), (dx_ref, dr_ref, dw_ref) = _oracle_fused(x, r, w, dy, ds)

    dev = gpu()
    xg = x.to(dev).requires_grad_(True)
    rg = r.to(dev).requires_grad_(True)
    wg = w.to(dev).requires_grad_(True)
    y, s = hilda_fused_add_rms_norm(xg, rg, wg)
    # S is bit-exact: both sides round the same fp32 sum to the input dtype
    assert torch.equal(s.cpu(), x + r)
    if with_ds:
        torch.autograd.backward([y, s], [dy.to(dev), ds.to(dev)])
    else:
        y.backward(dy.to(dev))
    t = tol(dtype)
    assert_close(y, y_ref, name="y", **t)
    assert_close(xg.grad, dx_ref, name="dx", **t)
    assert_close(rg.grad, dr_ref, name="dr", **t)
    assert_close(wg.grad, dw_ref, name="dw", **t)


def test_fused_add_rms_norm_c2_config():
    """C2 FusedAddRMSNorm bf16 [8192, 4096] against the fp32 oracle."""
    c = configs.c2_fused_add_rms_norm()
    (y_ref, s_ref), (dx_ref, dr_ref, dw_ref) = _oracle_fused(c["x"], c["r"], c["w"], c["dy"], c["ds"], c["eps"])
    dev = gpu()
    x = c["x"].to(dev).requires_grad_(True)
    r = c["r"].to(dev).requires_grad_(True)
    w = c["w"].to(dev).requires_grad_(True)
    y, s = hilda_fused_add_rms_norm(x, r, w, c["eps"])
    torch.autograd.backward([y, s], [c["dy"].to(dev), c["ds"].to(dev)])
    assert torch.equal(s.cpu(), c["x"] + c["r"])
    t = tol(torch.bfloat16)
    assert_close(y, y_ref, name="y", **t)
    assert_close(x.grad, dx_ref, name="dx", **t)
    assert_close(w.grad, dw_ref, name="dw", **t)
    assert rel_fro(x.grad, dx_ref) < 1e-2


def test_fused_add_module():
    m = FusedAddRMSNorm(1024).to(gpu())
    x = torch.randn(3, 1024, device=gpu())
    r = torch.randn(3, 1024, device=gpu())
    y, s = m(x, r)
    assert y.shape == x.shape and torch.equal(s, x + r)
