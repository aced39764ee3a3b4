"""GPU parity: FusedLinearCrossEntropy (bf16/fp16 MFMA GEMMs + CE) vs the CPU oracle.

Follows benchmarks/bench_fused_linear_ce.py (loss, dH, dW against
``hidden @ W.T`` + F.cross_entropy) with the fp64 oracle, adding ignored rows,
multi-chunk runs with ragged chunk sizes (K not a multiple of 8), every
reduction (including 'none', whose backward the reference gets wrong), the
upstream gradient, and the C5 shape: per-row losses and dhidden rows of a row
sample against the oracle, plus size-independent properties (ignored rows of
dhidden exactly zero; the vocabulary sum of dW vanishes because every
gradient row of the logits sums to zero).
"""
import math

import pytest
import torch

import oracle
import workloads
from _util import assert_close, rel_fro, tol, gpu

from kernels import hilda_fused_linear_cross_entropy, FusedLinearCrossEntropyLoss
from kernels import fused_linear_cross_entropy as fl

pytestmark = pytest.mark.gpu


def _case(BT, H, V, dtype, seed, ignore_frac=0.1):
    g = torch.Generator().manual_seed(seed)
    h = torch.randn(BT, H, generator=g).to(dtype)
    w = (0.02 * torch.randn(V, H, generator=g)).to(dtype)
    t = torch.randint(0, V, (BT,), generator=g)
    t[torch.rand(BT, generator=g) < ignore_frac] = -100
    return h, w, t


def _oracle(h, w, t, reduction="mean", grads=None):
    # logits in the compute dtype as the reference's GEMM returns them, CE in fp64
    def f(a, b):
        logits = (a.double() @ b.double().T).to(h.dtype).double()
        return oracle.cross_entropy_ref(logits, t, -100, reduction)
    return oracle.fwd_bwd(f, [h, w], grads, dtype=torch.float64)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("shape,chunk", [((96, 256, 1000), 4096), ((300, 128, 4096), 4096), ((200, 64, 520), 64),
                                         ((513, 256, 2048), 128), ((64, 4096, 32000), 4096)])
@pytest.mark.parametrize("reduction", ["mean", "sum"])
def test_flce(dtype, shape, chunk, reduction):
    BT, H, V = shape
    h, w, t = _case(BT, H, V, dtype, BT + H + V)
    (l_ref,), (dh_ref, dw_ref) = _oracle(h, w, t, reduction)
    dev = gpu()
    hg = h.to(dev).requires_grad_(True)
    wg = w.to(dev).requires_grad_(True)
    if chunk != 4096:
        loss, gi, gw, _ = fl.fused_linear_cross_entropy_forward(hg.detach(), wg.detach(), t.to(dev), -100, reduction,
                                                                compute_grad=True, chunk=chunk)
        hg.grad, wg.grad = gi, gw
    else:
        loss = hilda_fused_linear_cross_entropy(hg, wg, t.to(dev), -100, reduction)
        loss.backward()
    n_valid = int((t != -100).sum())
    s = n_valid if reduction == "mean" else 1
    lt = dict(rtol=1e-5, atol=1e-5) if dtype == torch.float32 else dict(rtol=2e-3, atol=2e-3)
    assert_close(loss, l_ref, name="loss", **lt)
    tt = tol(dtype)
    assert_close(hg.grad, dh_ref, name="dhidden", **tt)
    assert_close(wg.grad, dw_ref, name="dweight", **tt)
    assert_close(hg.grad.float() * s, dh_ref * s, name="dhidden*n_valid", **tt)
    assert_close(wg.grad.float() * s, dw_ref * s, name="dweight*n_valid", **tt)
    assert rel_fro(hg.grad, dh_ref) < 1e-2 and rel_fro(wg.grad, dw_ref) < 1e-2
    assert torch.count_nonzero(hg.grad[(t == -100).to(dev)]).item() == 0


def test_flce_fp32_reference_check():
    """benchmarks/bench_fused_linear_ce.py:45-49,71-90: the reference's fp32 checks at (256, 4096, 32000),
    hidden ~ N(0,1), weight ~ N(0, 0.02), no ignored targets, mean; here against the fp64 oracle at the
    north-star fp32 tolerance (rtol 1e-5, atol 1e-5), the gradients also multiplied back by n_valid."""
    dtype = torch.float32
    h, w, t = _case(256, 4096, 32000, dtype, 4096, ignore_frac=0.0)
    (l_ref,), (dh_ref, dw_ref) = _oracle(h, w, t, "mean")
    dev = gpu()
    hg = h.to(dev).requires_grad_(True)
    wg = w.to(dev).requires_grad_(True)
    loss = hilda_fused_linear_cross_entropy(hg, wg, t.to(dev))
    loss.backward()
    tt = tol(dtype)
    assert_close(loss, l_ref, name="loss", **tt)
    assert_close(hg.grad, dh_ref, name="dhidden", **tt)
    assert_close(wg.grad, dw_ref, name="dweight", **tt)
    assert_close(hg.grad * 256, dh_ref * 256, name="dhidden*n_valid", **tt)
    assert_close(wg.grad * 256, dw_ref * 256, name="dweight*n_valid", **tt)
    assert rel_fro(hg.grad, dh_ref) < 1e-5 and rel_fro(wg.grad, dw_ref) < 1e-5


def test_flce_reduction_none_and_upstream_grad():
    dtype = torch.bfloat16
    h, w, t = _case(130, 128, 3000, dtype, 21)
    dev = gpu()
    up = torch.randn(130)
    (l_ref,), (dh_ref, dw_ref) = _oracle(h, w, t, "none", [up])
    hg = h.to(dev).requires_grad_(True)
    wg = w.to(dev).requires_grad_(True)
    loss = FusedLinearCrossEntropyLoss(reduction="none")(hg, wg, t.to(dev))
    assert loss.shape == (130,)
    loss.backward(up.to(dev))
    assert_close(loss, l_ref, name="loss rows", rtol=2e-3, atol=2e-3)
    assert rel_fro(hg.grad, dh_ref) < 1e-2 and rel_fro(wg.grad, dw_ref) < 1e-2
    # a scalar upstream gradient other than 1
    (l2,), (dh2, dw2) = _oracle(h, w, t, "mean")
    hg2 = h.to(dev).requires_grad_(True)
    wg2 = w.to(dev).requires_grad_(True)
    (2.5 * hilda_fused_linear_cross_entropy(hg2, wg2, t.to(dev))).backward()
    assert rel_fro(hg2.grad, 2.5 * dh2) < 1e-2 and rel_fro(wg2.grad, 2.5 * dw2) < 1e-2


def test_flce_all_ignored_and_no_grad():
    dev = gpu()
    h, w, t = _case(40, 64, 256, torch.bfloat16, 5)
    hg = h.to(dev).requires_grad_(True)
    wg = w.to(dev).requires_grad_(True)
    loss = hilda_fused_linear_cross_entropy(hg, wg, torch.full((40,), -100, device=dev))
    loss.backward()
    assert loss.item() == 0.0
    assert torch.count_nonzero(hg.grad).item() == 0 and torch.count_nonzero(wg.grad).item() == 0
    with torch.no_grad():
        l_ng = hilda_fused_linear_cross_entropy(h.to(dev), w.to(dev), t.to(dev))
    (l_ref,), _ = _oracle(h, w, t)
    assert_close(l_ng, l_ref, name="no-grad loss", rtol=2e-3, atol=2e-3)


def test_flce_c5_config():
    """C5: hidden [16384, 4096], weight [128256, 4096] bf16, 5% ignored, mean; on the GPU."""
    dev = gpu()
    c = workloads.c5_fused_linear_ce(device=dev)
    h, w, t = c["hidden"], c["weight"], c["targets"]
    loss_rows, _, _, _ = fl.fused_linear_cross_entropy_forward(h, w, t, -100, "none", compute_grad=False)
    hg = h.requires_grad_(True)
    wg = w.requires_grad_(True)
    loss = hilda_fused_linear_cross_entropy(hg, wg, t)
    loss.backward()
    valid = t != -100
    n_valid = int(valid.sum())
    assert torch.count_nonzero(hg.grad[~valid]).item() == 0
    # mean of the per-row losses equals the reduced loss
    assert math.isclose(loss.item(), loss_rows.double().sum().item() / n_valid, rel_tol=1e-5)
    # sum over the vocabulary of dW vanishes (each logits-gradient row sums to zero),
    # relative to the column's L1 mass; what remains is bf16 rounding of D and dW
    gw = wg.grad.float()
    ratio = gw.sum(0).abs() / gw.abs().sum(0)
    assert ratio.max().item() < 1e-2
    # a sample of rows against the oracle: per-row loss and dhidden rows
    idx = torch.arange(0, 16384, 257, device=dev)[:64]
    hs, ts = h[idx].detach().cpu(), t[idx].cpu()
    wc = w.detach().cpu()
    logits = (hs.double() @ wc.double().T).to(torch.bfloat16).double().requires_grad_(True)
    per_row = oracle.cross_entropy_ref(logits, ts, -100, "none")
    per_row.sum().backward()
    assert_close(loss_rows[idx], per_row.detach(), name="loss rows", rtol=2e-3, atol=2e-3)
    dh_ref = logits.grad.to(torch.bfloat16).double() @ wc.double()  # d(sum of rows) / dh for the sample
    assert_close(hg.grad[idx].float() * n_valid, dh_ref, name="dhidden rows * n_valid", **tol(torch.bfloat16))
    assert rel_fro(hg.grad[idx].float() * n_valid, dh_ref) < 1e-2
    # <X, dX> = <W, dW>: both equal sum_{r,v} D_rv Z_rv (Z = X W^T, D the logits gradient), so a
    # dropped chunk, a wrong scale or mispaired rows in either GEMM breaks the equality
    ip_x = (h.detach().double() * hg.grad.double()).sum().item()
    ip_w = (w.detach().double() * wg.grad.double()).sum().item()
    assert math.isclose(ip_x, ip_w, rel_tol=1e-2), (ip_x, ip_w)
    # sampled vocabulary rows of dW against the oracle summed over all 16384 rows: each live row's
    # log-sum-exp from CPU fp32 logits (bf16 products summed in fp32, rounded to bf16 as the GEMM
    # returns them), then D[:, v] and dW[v] = D[:, v]^T X in fp64
    hc = h.detach().cpu()
    tc = t.cpu()
    live = (tc != -100).nonzero().squeeze(1)
    wf = wc.float()
    lse = torch.zeros(16384, dtype=torch.float64)
    for i in range(0, live.numel(), 1024):
        rows = live[i:i + 1024]
        z = (hc[rows].float() @ wf.T).to(torch.bfloat16).float()
        lse[rows] = torch.logsumexp(z, dim=1).double()
    del wf
    gen = torch.Generator().manual_seed(55)
    hit = tc[live][torch.randperm(live.numel(), generator=gen)[:16]]
    vs = torch.cat([hit, torch.randint(0, 128256, (16,), generator=gen)]).unique()
    zv = (hc.double() @ wc[vs].double().T).to(torch.bfloat16).double()  # [BT, len(vs)]
    d = torch.exp(zv - lse[:, None]) - (tc[:, None] == vs[None, :]).double()
    d[tc == -100] = 0.0
    dw_ref = d.T @ hc.double()  # sum-reduction gradient rows
    got = wg.grad[vs.to(dev)].float().cpu() * n_valid
    print(f"C5 dW rows {vs.tolist()}", flush=True)
    assert_close(got, dw_ref, name="dW rows * n_valid", **tol(torch.bfloat16))
    assert rel_fro(got, dw_ref) < 1e-2


@pytest.mark.parametrize("BT,H,V,chunk,dead", [
    (600, 64, 520, 64, (100, 400)),    # several chunks wholly ignored; dW through the fp32 accumulator
    (300, 128, 1000, 64, (64, 256)),   # the same with every chunk's D^T kept and one dW GEMM
    (256, 64, 264, 128, (0, 256)),     # nothing live
])
def test_flce_dead_chunks(BT, H, V, chunk, dead):
    """Ignored rows are compacted away before the GEMMs: whole chunks past the live rows, live rows that end
    mid-chunk, and the two dW paths give the oracle's result with exact zeros on ignored rows."""
    dtype = torch.bfloat16
    h, w, t = _case(BT, H, V, dtype, BT + V, ignore_frac=0.1)
    t[dead[0]:dead[1]] = -100
    (l_ref,), (dh_ref, dw_ref) = _oracle(h, w, t, "sum")
    dev = gpu()
    loss, gi, gw, _ = fl.fused_linear_cross_entropy_forward(h.to(dev), w.to(dev), t.to(dev), -100, "sum",
                                                            compute_grad=True, chunk=chunk)
    print(f"dead chunks BT={BT} H={H} V={V} chunk={chunk} dead={dead}", flush=True)
    assert_close(loss, l_ref, name="loss", rtol=2e-3, atol=2e-3)
    tt = tol(dtype)
    assert_close(gi, dh_ref, name="dhidden", **tt)
    assert_close(gw, dw_ref, name="dweight", **tt)
    if dw_ref.abs().sum() > 0:
        assert rel_fro(gi, dh_ref) < 1e-2 and rel_fro(gw, dw_ref) < 1e-2
    else:
        assert torch.count_nonzero(gw).item() == 0
    assert torch.count_nonzero(gi[(t == -100).to(dev)]).item() == 0
    rows, _, _, _ = fl.fused_linear_cross_entropy_forward(h.to(dev), w.to(dev), t.to(dev), -100, "none",
                                                          compute_grad=False, chunk=chunk)
    assert torch.count_nonzero(rows[(t == -100).to(dev)]).item() == 0


def _int_case(BT, H, V, dtype, seed):
    """hidden and weight with entries in {-1, 0, 1}: every logit is an integer below 2^8, exact in the
    GEMM's fp32 sums and in bf16/fp16, so the oracle sees the same logits as the kernels. Logits are
    ~N(0, 9) for H = 192; rows 3 and 40 are peaked (hidden = sign(weight[v]), logit ~128 at v)."""
    g = torch.Generator().manual_seed(seed)
    h = torch.randint(-1, 2, (BT, H), generator=g).float()
    w = torch.randint(-1, 2, (V, H), generator=g).float()
    t = torch.randint(0, V, (BT,), generator=g)
    t[torch.rand(BT, generator=g) < 0.1] = -100
    for r, v in ((3, 11), (40, V - 2)):
        h[r] = torch.where(w[v] == 0, torch.ones_like(w[v]), w[v])
        t[r] = v
    return h.to(dtype), w.to(dtype), t


def _rows_check(name, actual, expected, slack):
    """Every row whose oracle norm exceeds `slack` within 2% relative Frobenius error plus `slack`."""
    a = actual.detach().to("cpu", torch.float64)
    e = expected.detach().to("cpu", torch.float64)
    n = e.norm(dim=1)
    err = (a - e).norm(dim=1)
    sel = n > max(slack, 1e-30)
    assert sel.any()
    bad = int((err[sel] > 2e-2 * n[sel] + slack).sum())
    worst = (err[sel] / n[sel]).max().item()
    assert bad == 0, f"{name}: {bad} of {int(sel.sum())} rows off, worst rel {worst:.3e}, " \
                     f"{int((a.norm(dim=1)[sel] == 0).sum())} zero rows"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("BT,V", [(256, 4096), (256, 32000), (64, 128256)])
def test_flce_wide_logits(dtype, BT, V):
    """Wide and peaked logits through the chunk engine: every dW row (most of them sums of small
    probabilities only) and every dhidden row within 2% of the oracle. The oracle contracts the
    logits gradient rounded to the compute dtype, as the reference does (it stores the gradient
    over its bf16/fp16 chunk logits, fused_linear_cross_entropy.py:76, and contracts that at
    :158,161); for fp16 each row may also be off by one subnormal step (2^-24) per element."""
    H = 192
    h, w, t = _int_case(BT, H, V, dtype, BT + V)
    print(f"wide FLCE BT={BT} V={V} {dtype}", flush=True)
    z = (h.double() @ w.double().T).requires_grad_(True)  # exact integers
    loss_ref = oracle.cross_entropy_ref(z, t, -100, "sum")
    loss_ref.backward()
    d = oracle.exact_target_grad(z.grad, t).to(dtype).double()  # the peaked rows' targets formed exactly
    dh_ref, dw_ref = d @ w.double(), d.T @ h.double()
    dev = gpu()
    loss, gi, gw, _ = fl.fused_linear_cross_entropy_forward(h.to(dev), w.to(dev), t.to(dev), -100, "sum",
                                                            compute_grad=True, chunk=128)
    assert_close(loss, loss_ref, name="loss", rtol=2e-3, atol=2e-3)
    slack = 2.0 ** -24 * math.sqrt(BT * V) if dtype == torch.float16 else 0.0
    _rows_check("dweight", gw, dw_ref, 2.0 ** -24 * math.sqrt(BT * H) if dtype == torch.float16 else 0.0)
    _rows_check("dhidden", gi, dh_ref, slack)
    assert torch.count_nonzero(gi[(t == -100).to(dev)]).item() == 0
