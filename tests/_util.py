"""Shared helpers for the parity tests."""
from __future__ import annotations

import torch

# north-star tolerances
TOL = {
    torch.float32: dict(rtol=1e-5, atol=1e-5),
    torch.float16: dict(rtol=1.6e-2, atol=1e-2),
    torch.bfloat16: dict(rtol=1.6e-2, atol=1e-2),
}


def tol(dtype):
    return TOL[dtype]


def assert_close(actual, expected, rtol, atol, name=""):
    """torch.testing.assert_close on CPU fp64 copies, with a readable message."""
    a = actual.detach().to("cpu", torch.float64)
    e = expected.detach().to("cpu", torch.float64)
    assert a.shape == e.shape, f"{name}: shape {tuple(a.shape)} != {tuple(e.shape)}"
    torch.testing.assert_close(a, e, rtol=rtol, atol=atol, msg=lambda m: f"{name}: {m}")


def rel_fro(actual, expected) -> float:
    a = actual.detach().to("cpu", torch.float64)
    e = expected.detach().to("cpu", torch.float64)
    den = e.norm().item()
    return (a - e).norm().item() / (den if den > 0 else 1.0)


def gpu():
    return torch.device("cuda", torch.cuda.current_device())
