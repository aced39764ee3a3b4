"""GPU parity: KL divergence and JSD HIP kernels against the CPU oracle.

Follows benchmarks/bench_kl_div.py's checks (F.kl_div with 'batchmean' on
log_softmax / softmax inputs, [512, 32000 | 128256], lines 34-80) and
benchmarks/bench_jsd.py's (pytorch_jsd for beta 0, 1/2, 1, lines 47-96), and
adds every reduction, log targets, odd row lengths (scalar tail), 3-D inputs,
labels with ignored rows, all rows ignored and upstream gradients other than 1.
"""
import pytest
import torch

import oracle
from _util import assert_close, tol, gpu

from kernels import hilda_kl_div, hilda_jsd, KLDivLoss, JSDLoss

pytestmark = pytest.mark.gpu


def _lp(shape, dtype, g):
    return torch.log_softmax(torch.randn(*shape, generator=g), -1).to(dtype)


def _prec(dtype):
    return torch.float64 if dtype == torch.float32 else torch.float32


# --------------------------------------------------------------------------
# KL divergence
# --------------------------------------------------------------------------
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("reduction", ["batchmean", "sum", "mean", "none"])
@pytest.mark.parametrize("log_target", [False, True])
@pytest.mark.parametrize("shape", [(64, 1000), (7, 333), (2, 5, 96)])
def test_kl_div(dtype, reduction, log_target, shape):
    g = torch.Generator().manual_seed(shape[-1] + 3 * len(shape))
    yp = _lp(shape, dtype, g)
    lt = _lp(shape, dtype, g)
    yt = lt if log_target else lt.float().exp().to(dtype)
    rows = yp.numel() // shape[-1]
    up = torch.rand(rows, generator=g) + 0.5 if reduction == "none" else torch.tensor(1.7)
    (ref,), (dref, _) = oracle.fwd_bwd(lambda a, b: oracle.kl_div_ref(a, b, reduction, log_target), [yp, yt],
                                       [up], dtype=_prec(dtype), differentiable=[True, False])
    dev = gpu()
    yg = yp.to(dev).requires_grad_(True)
    out = KLDivLoss(reduction, log_target)(yg, yt.to(dev))
    out.backward(up.to(dev))
    t = tol(dtype)
    assert_close(out, ref, name="loss", **t)
    assert_close(yg.grad, dref, name="dy_pred", **t)


@pytest.mark.parametrize("dtype,V", [(torch.float16, 32000), (torch.float16, 128256), (torch.float32, 32000)])
def test_kl_div_reference_bench_shapes(dtype, V):
    g = torch.Generator().manual_seed(V)
    yp = _lp((512, V), dtype, g)
    yt = torch.softmax(torch.randn(512, V, generator=g), -1).to(dtype)
    (ref,), (dref, _) = oracle.fwd_bwd(oracle.kl_div_ref, [yp, yt], None, dtype=_prec(dtype),
                                       differentiable=[True, False])
    dev = gpu()
    yg = yp.to(dev).requires_grad_(True)
    out = hilda_kl_div(yg, yt.to(dev))
    out.backward()
    t = tol(dtype)
    assert_close(out, ref, name="loss", **t)
    assert_close(yg.grad, dref, name="dy_pred", **t)


def test_kl_div_zero_targets_and_identity():
    """t = 0 contributes nothing (t log max(t, eps) = 0); y_pred = log y_true gives 0."""
    dev = gpu()
    yt = torch.zeros(4, 64, device=dev)
    yt[:, 3] = 1.0
    yp = torch.log_softmax(torch.randn(4, 64, device=dev), -1)
    out = hilda_kl_div(yp, yt, reduction="none")
    assert_close(out, -yp[:, 3], name="one-hot rows", rtol=1e-6, atol=1e-6)
    lt = torch.log_softmax(torch.randn(4, 64, device=dev), -1)
    z = hilda_kl_div(lt, lt.exp(), reduction="sum")
    assert abs(float(z)) < 1e-5


# --------------------------------------------------------------------------
# JSD
# --------------------------------------------------------------------------
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("beta", [0.0, 0.5, 1.0, 0.3])
@pytest.mark.parametrize("with_labels", [False, True])
@pytest.mark.parametrize("shape", [(48, 1000), (9, 333)])
def test_jsd(dtype, beta, with_labels, shape):
    g = torch.Generator().manual_seed(shape[1] + int(beta * 10))
    X = _lp(shape, dtype, g)
    Y = _lp(shape, dtype, g)
    labels = None
    if with_labels:
        labels = torch.randint(0, shape[1], (shape[0],), generator=g)
        labels[::3] = -100
    up = torch.tensor(2.5)
    (ref,), (dref, _, _) = oracle.fwd_bwd(lambda x, y, l: oracle.jsd_ref(x, y, beta, l), [X, Y, labels], [up],
                                          dtype=_prec(dtype), differentiable=[True, False, False])
    dev = gpu()
    xg = X.to(dev).requires_grad_(True)
    out = JSDLoss(beta)(xg, Y.to(dev), None if labels is None else labels.to(dev))
    out.backward(up.to(dev))
    t = tol(dtype)
    assert_close(out, ref, name="loss", **t)
    assert_close(xg.grad, dref, name="dX", **t)
    if with_labels:
        assert torch.count_nonzero(xg.grad[labels.to(dev) == -100]).item() == 0


@pytest.mark.parametrize("dtype,V,beta", [(torch.float16, 32000, 0.5), (torch.float16, 128256, 0.5),
                                          (torch.float32, 32000, 0.5), (torch.float16, 32000, 0.0),
                                          (torch.float16, 32000, 1.0)])
def test_jsd_reference_bench_shapes(dtype, V, beta):
    g = torch.Generator().manual_seed(V + int(beta * 4))
    X = _lp((512, V), dtype, g)
    Y = _lp((512, V), dtype, g)
    (ref,), (dref, _) = oracle.fwd_bwd(lambda x, y: oracle.jsd_ref(x, y, beta), [X, Y], None, dtype=_prec(dtype),
                                       differentiable=[True, False])
    dev = gpu()
    xg = X.to(dev).requires_grad_(True)
    out = hilda_jsd(xg, Y.to(dev), beta=beta)
    out.backward()
    t = tol(dtype)
    assert_close(out, ref, name="loss", **t)
    assert_close(xg.grad, dref, name="dX", **t)


def test_jsd_all_ignored_and_repeated_backward():
    dev = gpu()
    X = torch.log_softmax(torch.randn(6, 128, device=dev), -1).requires_grad_(True)
    Y = torch.log_softmax(torch.randn(6, 128, device=dev), -1)
    out = hilda_jsd(X, Y, 0.5, torch.full((6,), -100, device=dev))
    out.backward()
    assert float(out.detach()) == 0.0 and torch.count_nonzero(X.grad).item() == 0
    X.grad = None
    out = hilda_jsd(X, Y, 0.5)
    out.backward(torch.tensor(2.0, device=dev), retain_graph=True)
    g1 = X.grad.clone()
    X.grad = None
    out.backward(torch.tensor(3.0, device=dev))
    assert_close(X.grad, g1 * 1.5, name="second backward", rtol=1e-6, atol=1e-7)
