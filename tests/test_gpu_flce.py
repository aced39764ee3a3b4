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


@pytest.mark.parametrize("budget", ["fastest", None])
def test_flce_c5_config(budget):
    """C5: hidden [16384, 4096], weight [128256, 4096] bf16, 5% ignored, mean; on the GPU, in the unlimited
    plan (two 8192-row chunks, one dW GEMM over every row) and the default one (the reference's chunk: 43
    chunks, dW accumulated in bf16 in the output as the reference's addmm does, fused_linear_cross_entropy.py:161)."""
    dev = gpu()
    c = workloads.c5_fused_linear_ce(device=dev)
    h, w, t = c["hidden"], c["weight"], c["targets"]
    print(f"C5 budget={budget}", flush=True)
    loss_rows, _, _, _ = fl.fused_linear_cross_entropy_forward(h, w, t, -100, "none", compute_grad=False,
                                                               workspace_budget=budget)
    hg = h.requires_grad_(True)
    wg = w.requires_grad_(True)
    loss = hilda_fused_linear_cross_entropy(hg, wg, t, workspace_budget=budget)
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
    # dropped chunk or tile, a wrong scale or mispaired rows in either GEMM breaks the equality. (The default
    # plan here is vocabulary tiles: dW written once per tile, dX summed over 28 tiles in bf16 from softmax
    # terms alone, each row's target term added once at the end; summing the target term in with the rest
    # measured 17% low, its later tiles' softmax terms rounding away against it.)
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


# Every memory plan of the chunk engine: the dW form (every chunk's D^T kept and one GEMM after the loop; an fp32
# accumulator; accumulated in the output), W^T or W read MN-contiguous by the dX GEMM, D^T or D read
# MN-contiguous by the dW GEMM (HILDA_FL_FORM forces one; the budget is unlimited).
FORMS = ["defer,wt,dt", "defer,wmn,dt", "acc,wt,dt", "acc,wt,dmn", "acc,wmn,dt", "acc,wmn,dmn",
         "out,wt,dt", "out,wt,dmn", "out,wmn,dt", "out,wmn,dmn"]
DW_NAME = {"defer": "deferred", "acc": "fp32 accumulator", "out": "in output"}


@pytest.mark.parametrize("form", FORMS)
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_flce_plan_forms(form, dtype, monkeypatch):
    """V = 2000 and H = 264 (neither a multiple of 64), five chunks of 128 rows, a wholly ignored chunk and live
    rows ending mid-chunk: each form against the fp64 oracle, exact zeros on ignored rows."""
    BT, H, V = 600, 264, 2000
    h, w, t = _case(BT, H, V, dtype, 7)
    t[200:330] = -100
    monkeypatch.setenv("HILDA_FL_FORM", form)
    dw, wf, df = form.split(",")
    plan = fl.fused_linear_cross_entropy_plan(BT, H, V, dtype, chunk=128, workspace_budget=-1)
    assert (plan["dw"], plan["w_transposed"], plan["d_transposed"]) == (DW_NAME[dw], wf == "wt", df == "dt")
    assert plan["chunks"] == 5
    (l_ref,), (dh_ref, dw_ref) = _oracle(h, w, t, "sum")
    dev = gpu()
    print(f"FLCE form {form} {dtype}", flush=True)
    loss, gi, gw, _ = fl.fused_linear_cross_entropy_forward(h.to(dev), w.to(dev), t.to(dev), -100, "sum",
                                                            compute_grad=True, chunk=128, workspace_budget=-1)
    assert_close(loss, l_ref, name="loss", rtol=2e-3, atol=2e-3)
    tt = tol(dtype)
    assert_close(gi, dh_ref, name="dhidden", **tt)
    assert rel_fro(gi, dh_ref) < 1e-2
    assert torch.count_nonzero(gi[(t == -100).to(dev)]).item() == 0
    if dw != "out":
        # dW summed in fp32 and rounded once
        assert_close(gw, dw_ref, name="dweight", **tt)
        assert rel_fro(gw, dw_ref) < 1e-2
        return
    # dW accumulated in the 16-bit output, chunk by chunk (the reference's addmm into its bf16 grad_weight,
    # fused_linear_cross_entropy.py:161): emulate that in fp64 over the same chunks of live rows (each chunk's
    # partial added to the running 16-bit sum and rounded). The kernel's error against the exact dW is that
    # arithmetic's (its D entries may sit one rounding step from the emulation's, so compare norms): no
    # larger than the emulation's own error plus a margin, and close to the emulation itself.
    emu = _chunked_dw(h, w, t, 128, dtype)
    e_ours, e_emu = rel_fro(gw, dw_ref), rel_fro(emu, dw_ref)
    print(f"in-output dW: rel error {e_ours:.3e}, emulated reference arithmetic {e_emu:.3e}", flush=True)
    assert e_ours <= 1.5 * e_emu + 1e-3
    assert rel_fro(gw, emu) < 1e-2


def _chunked_dw(h, w, t, C, dtype):
    """dW of the sum-reduced CE accumulated chunk by chunk in `dtype` (live rows compacted in order, C a chunk)."""
    live = (t != -100).nonzero().squeeze(1)
    hd, wd = h.double(), w.double()
    z = (hd[live] @ wd.T).to(dtype).double()
    d = torch.softmax(z, -1)
    d[torch.arange(live.numel()), t[live]] -= 1.0
    d = d.to(dtype).double()  # the gradient stored over the 16-bit logits
    acc = None
    for c0 in range(0, live.numel(), C):
        part = d[c0:c0 + C].T @ hd[live[c0:c0 + C]]
        acc = part.to(dtype).double() if acc is None else (acc + part).to(dtype).double()
    return acc


@pytest.mark.parametrize("form", ["defer,wt,dt", "out,wt,dt"])
def test_flce_plan_forms_fp32(form, monkeypatch):
    """fp32 takes the materialised forms only; accumulating dW in the fp32 output is an fp32 sum, so both
    forms meet the fp32 tolerance (rtol/atol 1e-5) against the fp64 oracle."""
    BT, H, V = 300, 136, 1000
    h, w, t = _case(BT, H, V, torch.float32, 8)
    monkeypatch.setenv("HILDA_FL_FORM", form)
    (l_ref,), (dh_ref, dw_ref) = _oracle(h, w, t, "mean")
    dev = gpu()
    loss, gi, gw, _ = fl.fused_linear_cross_entropy_forward(h.to(dev), w.to(dev), t.to(dev), -100, "mean",
                                                            compute_grad=True, chunk=64, workspace_budget=-1)
    n = int((t != -100).sum())
    tt = tol(torch.float32)
    assert_close(loss, l_ref, name="loss", **tt)
    assert_close(gi * n, dh_ref * n, name="dhidden*n", **tt)
    assert_close(gw * n, dw_ref * n, name="dweight*n", **tt)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("BT,H,V", [(64, 256, 32001), (48, 128, 50257), (96, 257, 1003), (40, 1027, 600)])
@pytest.mark.parametrize("budget", [None, -1])
def test_flce_any_shape(dtype, BT, H, V, budget):
    """Vocabulary and hidden sizes that are not multiples of 8 (GPT-2's 50257, 32001) against the oracle, in
    the default (reference-sized) plan and the unlimited one: the chunk buffer's stride is padded, its columns
    past V are -inf logits and zero gradients, an odd H is padded in the gathered rows and a weight copy."""
    h, w, t = _case(BT, H, V, dtype, BT + H + V)
    (l_ref,), (dh_ref, dw_ref) = _oracle(h, w, t, "mean")
    dev = gpu()
    print(f"FLCE any shape BT={BT} H={H} V={V} {dtype} budget={budget}", flush=True)
    hg = h.to(dev).requires_grad_(True)
    wg = w.to(dev).requires_grad_(True)
    loss = hilda_fused_linear_cross_entropy(hg, wg, t.to(dev), workspace_budget=budget)
    loss.backward()
    n = int((t != -100).sum())
    tt = tol(dtype)
    lt = tt if dtype == torch.float32 else dict(rtol=2e-3, atol=2e-3)
    assert_close(loss, l_ref, name="loss", **lt)
    assert_close(hg.grad.float() * n, dh_ref * n, name="dhidden*n", **tt)
    assert_close(wg.grad.float() * n, dw_ref * n, name="dweight*n", **tt)
    if dtype != torch.float32:
        assert rel_fro(hg.grad, dh_ref) < 1e-2 and rel_fro(wg.grad, dw_ref) < 1e-2
    assert torch.count_nonzero(hg.grad[(t == -100).to(dev)]).item() == 0


@pytest.mark.parametrize("budget", [None, -1])
def test_flce_misaligned_inputs(budget):
    """hidden and weight views that start 2 bytes into their storage (not 16-byte aligned): read element by
    element into the gathered rows and a weight copy, with the same results as aligned copies."""
    BT, H, V = 200, 256, 3000
    dtype = torch.bfloat16
    h, w, t = _case(BT, H, V, dtype, 3)
    dev = gpu()
    hs = torch.empty(BT * H + 1, dtype=dtype, device=dev)
    ws = torch.empty(V * H + 1, dtype=dtype, device=dev)
    hv, wv = hs[1:].view(BT, H), ws[1:].view(V, H)
    hv.copy_(h.to(dev))
    wv.copy_(w.to(dev))
    assert hv.data_ptr() % 16 != 0 and wv.data_ptr() % 16 != 0
    la, gia, gwa, _ = fl.fused_linear_cross_entropy_forward(h.to(dev), w.to(dev), t.to(dev), -100, "none",
                                                            compute_grad=True, workspace_budget=budget)
    lm, gim, gwm, _ = fl.fused_linear_cross_entropy_forward(hv, wv, t.to(dev), -100, "none", compute_grad=True,
                                                            workspace_budget=budget)
    assert torch.equal(la, lm) and torch.equal(gia, gim) and torch.equal(gwa, gwm)


def test_flce_default_and_fastest_plans_agree():
    """The default plan (here vocabulary tiles or row chunks with dW in the output) and the unlimited one give
    the same per-row losses to fp32 rounding (the same logits GEMM; the log-sum-exp reduced in another order)
    and gradients equal to bf16 rounding."""
    BT, H, V = 1024, 512, 20000
    h, w, t = _case(BT, H, V, torch.bfloat16, 12)
    dev = gpu()
    fast = fl.fused_linear_cross_entropy_plan(BT, H, V, torch.bfloat16, workspace_budget=-1)
    lean = fl.fused_linear_cross_entropy_plan(BT, H, V, torch.bfloat16)
    assert lean["workspace_bytes"] < fast["workspace_bytes"] and lean["chunks"] > fast["chunks"]
    out = {}
    for name, b in (("lean", None), ("fast", -1)):
        out[name] = fl.fused_linear_cross_entropy_forward(h.to(dev), w.to(dev), t.to(dev), -100, "none",
                                                          compute_grad=True, workspace_budget=b)
    assert_close(out["lean"][0], out["fast"][0], name="loss rows", rtol=1e-6, atol=1e-6)
    assert rel_fro(out["lean"][1], out["fast"][1]) < 1e-2 and rel_fro(out["lean"][2], out["fast"][2]) < 1e-2


def test_flce_peak_memory_below_unfused():
    """Peak memory of fwd+bwd, measured as the reference's benchmark does (bench_fused_linear_ce.py:171-178,
    leaves allocated inside the measured function): the default plan stays at least 47.7% below torch's
    unfused hidden @ W.T + cross_entropy (the low end of the reference's claim, README.md:42)."""
    BT, H, V = 2048, 1024, 50257
    dtype = torch.float16
    dev = gpu()
    t = torch.randint(0, V, (BT,), device=dev)

    def peak(fn):
        fn()
        torch.cuda.synchronize()
        torch.cuda.reset_peak_memory_stats(dev)
        base = torch.cuda.memory_allocated(dev)
        fn()
        torch.cuda.synchronize()
        return torch.cuda.max_memory_allocated(dev) - base

    def run(f):
        def fn():
            h = torch.randn(BT, H, device=dev, dtype=dtype, requires_grad=True)
            w = torch.randn(V, H, device=dev, dtype=dtype, requires_grad=True)
            f(h, w).backward()
        return fn

    unfused = peak(run(lambda h, w: torch.nn.functional.cross_entropy(h @ w.T, t)))
    ours = peak(run(lambda h, w: hilda_fused_linear_cross_entropy(h, w, t)))
    print(f"peak MiB: unfused {unfused / 2**20:.1f}, default plan {ours / 2**20:.1f}", flush=True)
    assert ours <= (1 - 0.477) * unfused


# The vocabulary-tiled plan (the default at tight budgets): pass 1 folds each tile of Vt vocabulary columns into
# every row's log-sum-exp, pass 2 recomputes the tile's logits, writes its dW rows once (fp32 sums over all
# rows) and adds D W_t to dX (fp32 buffer, or the 16-bit output). HILDA_FL_FORM="vtile,<acc|out>,<Vt>" forces it.
@pytest.mark.parametrize("dx", ["acc", "out"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape", [(600, 264, 2000), (96, 257, 1003)])
def test_flce_vocab_tiles(dx, dtype, shape, monkeypatch):
    """Four tiles of 512 columns over V = 2000 (a short last tile), or two over V = 1003 with H = 257 (padded
    rows); ignored rows; the loss rows bitwise equal to the row-chunked plan's (the same logits GEMM and the
    same per-row arithmetic are not guaranteed, so compared at tolerance) and the gradients against the oracle."""
    BT, H, V = shape
    h, w, t = _case(BT, H, V, dtype, 17)
    t[100:180] = -100
    monkeypatch.setenv("HILDA_FL_FORM", f"vtile,{dx},512")
    plan = fl.fused_linear_cross_entropy_plan(BT, H, V, dtype, workspace_budget=-1)
    assert plan["dw"].startswith("vocab tiles") and plan["chunk"] == 512
    (l_ref,), (dh_ref, dw_ref) = _oracle(h, w, t, "mean")
    dev = gpu()
    print(f"FLCE vocab tiles {dx} {dtype} {shape}", flush=True)
    hg = h.to(dev).requires_grad_(True)
    wg = w.to(dev).requires_grad_(True)
    loss = hilda_fused_linear_cross_entropy(hg, wg, t.to(dev), workspace_budget=-1)
    loss.backward()
    n = int((t != -100).sum())
    tt = tol(dtype)
    assert_close(loss, l_ref, name="loss", rtol=2e-3, atol=2e-3)
    # dW: every vocabulary row written once from an fp32 sum over all rows
    assert_close(wg.grad.float() * n, dw_ref * n, name="dweight*n", **tt)
    assert rel_fro(wg.grad, dw_ref) < 1e-2
    assert_close(hg.grad.float() * n, dh_ref * n, name="dhidden*n", **tt)
    assert rel_fro(hg.grad, dh_ref) < 1e-2
    assert torch.count_nonzero(hg.grad[(t == -100).to(dev)]).item() == 0
    # <X, dX> = <W, dW> = sum D Z: the softmax terms summed across the tiles are not lost to a row's target
    ip_x = (h.double() * hg.grad.double().cpu()).sum().item()
    ip_w = (w.double() * wg.grad.double().cpu()).sum().item()
    assert math.isclose(ip_x, ip_w, rel_tol=1e-2), (ip_x, ip_w)
    # reduction 'none' with per-row upstream gradients goes through the same plan
    up = torch.randn(BT)
    (_,), (dh2, dw2) = _oracle(h, w, t, "none", [up])
    hg2 = h.to(dev).requires_grad_(True)
    wg2 = w.to(dev).requires_grad_(True)
    rows = hilda_fused_linear_cross_entropy(hg2, wg2, t.to(dev), reduction="none", workspace_budget=-1)
    rows.backward(up.to(dev))
    assert rel_fro(hg2.grad, dh2) < 2e-2 and rel_fro(wg2.grad, dw2) < 1e-2


@pytest.mark.parametrize("V", [4096, 32000])
def test_flce_vocab_tiles_peaked_rows(V, monkeypatch):
    """Peaked rows (a logit ~128 above the rest, so p_target rounds to 1) through the tiles: 1 - p_target is
    formed from the other columns' mass, tile by tile, so the target's small gradient stays exact; every dW
    and dhidden row within 2% of the oracle."""
    BT, H = 256, 192
    dtype = torch.bfloat16
    h, w, t = _int_case(BT, H, V, dtype, BT + V)
    monkeypatch.setenv("HILDA_FL_FORM", "vtile,acc,1024")
    z = (h.double() @ w.double().T).requires_grad_(True)
    oracle.cross_entropy_ref(z, t, -100, "sum").backward()
    d = oracle.exact_target_grad(z.grad, t).to(dtype).double()
    dh_ref, dw_ref = d @ w.double(), d.T @ h.double()
    dev = gpu()
    loss, gi, gw, _ = fl.fused_linear_cross_entropy_forward(h.to(dev), w.to(dev), t.to(dev), -100, "sum",
                                                            compute_grad=True, workspace_budget=-1)
    _rows_check("dweight", gw, dw_ref, 0.0)
    _rows_check("dhidden", gi, dh_ref, 0.0)


def test_flce_threads_and_streams():
    """Two host threads, each on its own torch stream, run FusedLinearCE at once in the fastest plan (W^T, X^T and
    D^T transposed on the library's side stream, one per host thread, between event fork/joins); every result
    equals the same call made alone on the default stream, bit for bit (the sums run in a fixed order)."""
    import threading
    dev = gpu()
    g = torch.Generator(device=dev).manual_seed(21)
    bf = torch.bfloat16
    cases = []
    for _ in range(2):
        h = torch.randn(640, 256, generator=g, device=dev).to(bf)
        w = (0.05 * torch.randn(3000, 256, generator=g, device=dev)).to(bf)
        t = torch.randint(0, 3000, (640,), generator=g, device=dev)
        t[::5] = -100
        cases.append((h, w, t))

    def run(h, w, t):
        return fl.fused_linear_cross_entropy_forward(h, w, t, -100, "mean", compute_grad=True, chunk=128,
                                                     workspace_budget="fastest")[:3]

    assert fl.fused_linear_cross_entropy_plan(640, 256, 3000, bf, True, 128, "fastest")["w_transposed"]
    ref = [run(*c) for c in cases]
    torch.cuda.synchronize()
    out, errs = [None, None], []

    def worker(i):
        try:
            s = torch.cuda.Stream(device=dev)
            with torch.cuda.stream(s):
                for _ in range(4):
                    out[i] = run(*cases[i])
            s.synchronize()
        except Exception as e:  # surfaced by the assert below
            errs.append(e)

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(2)]
    for th in threads:
        th.start()
    for th in threads:
        th.join()
    assert not errs, errs
    for i in range(2):
        for a, b in zip(out[i], ref[i]):
            assert torch.equal(a, b)
