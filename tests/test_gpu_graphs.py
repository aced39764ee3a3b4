"""GPU: the ops under HIP graph capture.

The library allocates nothing, never synchronises and records no memset, so a
whole fwd+bwd step can be captured once and replayed. Each test captures a
step, replays it three times with unrelated eager work and a synchronisation
between replays, and checks every replay against the eager result of the same
step, bitwise: every float sum in these steps has a fixed order (no atomics).
"""
import pytest
import torch

from _util import gpu

import kernels as K

pytestmark = pytest.mark.gpu


def _graph(fn):
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            fn()
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        outs = fn()
    return g, outs


def _check_replays(fn):
    eager = [t.detach().clone() for t in fn()]
    torch.cuda.synchronize()
    g, outs = _graph(fn)
    for rep in range(3):
        print(f"replay {rep}", flush=True)
        g.replay()
        junk = torch.randn(1 << 20, device=gpu()).mul_(2.0)  # unrelated eager work between replays
        torch.cuda.synchronize()
        for i, (o, e) in enumerate(zip(outs, eager)):
            assert torch.equal(o, e), f"replay {rep}: output {i} differs from eager"
        del junk


def test_graph_layer_ops_step():
    """FusedAddRMSNorm + RoPE + SwiGLU fwd+bwd (the C2 step at small shapes)."""
    dev = gpu()
    g = torch.Generator(device=dev).manual_seed(3)
    bf = torch.bfloat16
    x = torch.randn(512, 1024, generator=g, device=dev).to(bf).requires_grad_(True)
    r = torch.randn(512, 1024, generator=g, device=dev).to(bf).requires_grad_(True)
    w = (1 + 0.02 * torch.randn(1024, generator=g, device=dev)).to(bf).requires_grad_(True)
    dy, ds = torch.randn_like(x), torch.randn_like(x)
    q = torch.randn(2, 256, 8, 128, generator=g, device=dev).to(bf).transpose(1, 2).requires_grad_(True)
    k = torch.randn(2, 256, 2, 128, generator=g, device=dev).to(bf).transpose(1, 2).requires_grad_(True)
    rot = K.RotaryEmbedding(128, 256, base=500000.0).to(dev)
    cos, sin = rot.cos_cached, rot.sin_cached
    dq, dk = torch.randn_like(q), torch.randn_like(k)
    a = torch.randn(512, 2048, generator=g, device=dev).to(bf).requires_grad_(True)
    b = torch.randn(512, 2048, generator=g, device=dev).to(bf).requires_grad_(True)
    dc = torch.randn_like(a)

    def step():
        y, s = K.hilda_fused_add_rms_norm(x, r, w)
        gx, gr, gw = torch.autograd.grad([y, s], [x, r, w], [dy, ds])
        qo, ko = K.hilda_rope(q, k, cos, sin)
        gq, gk = torch.autograd.grad([qo, ko], [q, k], [dq, dk])
        c = K.hilda_swiglu(a, b)
        ga, gb = torch.autograd.grad([c], [a, b], [dc])
        return y, s, gx, gr, gw, qo, ko, gq, gk, c, ga, gb

    _check_replays(step)


def test_graph_losses_step():
    """CrossEntropy with ignored rows, GRPO, and FusedLinearCE over several chunks (compaction included)."""
    dev = gpu()
    g = torch.Generator(device=dev).manual_seed(5)
    bf = torch.bfloat16
    logits = (2 * torch.randn(256, 4096, generator=g, device=dev)).to(bf).requires_grad_(True)
    t = torch.randint(0, 4096, (256,), generator=g, device=dev)
    t[::7] = -100
    gl = (2 * torch.randn(2, 17, 3000, generator=g, device=dev)).to(bf).requires_grad_(True)
    ids = torch.randint(0, 3000, (2, 16), generator=g, device=dev)
    adv = torch.randn(2, generator=g, device=dev)
    mask = torch.ones(2, 16, dtype=torch.int32, device=dev)
    mask[1, 9:] = 0
    h = torch.randn(300, 128, generator=g, device=dev).to(bf).requires_grad_(True)
    wt = (0.05 * torch.randn(1000, 128, generator=g, device=dev)).to(bf).requires_grad_(True)
    th = torch.randint(0, 1000, (300,), generator=g, device=dev)
    th[100:220] = -100
    from kernels import fused_linear_cross_entropy as fl

    def step():
        loss = K.hilda_cross_entropy(logits, t)
        (gce,) = torch.autograd.grad([loss], [logits])
        gloss, _, clip = K.hilda_grpo_loss(gl, ids, adv, completion_mask=mask)
        (ggl,) = torch.autograd.grad([gloss], [gl])
        fl_loss, gh, gw, _ = fl.fused_linear_cross_entropy_forward(h, wt, th, -100, "mean", compute_grad=True,
                                                                   chunk=64)
        return loss, gce, gloss, clip, ggl, fl_loss, gh, gw

    _check_replays(step)


@pytest.mark.parametrize("form", ["defer,wt,dt", "acc,wt,dt", "out,wmn,dmn", "acc,wmn,dt"])
def test_graph_fused_linear_forms(form, monkeypatch):
    """FusedLinearCE's chunked memory forms under capture. Their transposes run on a second stream between
    event fork/joins (W^T beside the first logits GEMM, each chunk's X^T and D^T beside its dX GEMM), which
    the capture must follow; compacted rows, several chunks."""
    monkeypatch.setenv("HILDA_FL_FORM", form)
    dev = gpu()
    g = torch.Generator(device=dev).manual_seed(11)
    bf = torch.bfloat16
    h = torch.randn(520, 192, generator=g, device=dev).to(bf)
    wt = (0.05 * torch.randn(1500, 192, generator=g, device=dev)).to(bf)
    th = torch.randint(0, 1500, (520,), generator=g, device=dev)
    th[130:260] = -100
    from kernels import fused_linear_cross_entropy as fl

    def step():
        loss, gh, gw, _ = fl.fused_linear_cross_entropy_forward(h, wt, th, -100, "mean", compute_grad=True,
                                                                chunk=128, workspace_budget="fastest")
        return loss, gh, gw

    _check_replays(step)
