"""GPU parity: FusedLinearJSD (student/teacher bf16/fp16 MFMA GEMMs + JSD) vs the CPU oracle.

Follows benchmarks/bench_fused_linear_jsd.py (loss and the student gradients
against linear + log_softmax + JSD, lines 30-41 and 42-96) with an fp64
oracle that rounds the logits to the compute dtype as the reference's GEMMs
return them, and adds beta 0 / 1 / general, temperature, labels with ignored
rows, a teacher hidden size different from the student's, multi-chunk runs
(fp32 accumulation of dW) with ragged chunks, the upstream gradient and a
repeated backward.
"""
import pytest
import torch

import oracle
from _util import assert_close, rel_fro, tol, gpu

from kernels import hilda_fused_linear_jsd, FusedLinearJSDLoss
from kernels import fused_linear_jsd as fj

pytestmark = pytest.mark.gpu


def _case(BT, H, Ht, V, dtype, seed, with_labels=True):
    g = torch.Generator().manual_seed(seed)
    si = torch.randn(BT, H, generator=g).to(dtype)
    sw = (torch.randn(V, H, generator=g) / H ** 0.5).to(dtype)
    ti = torch.randn(BT, Ht, generator=g).to(dtype)
    tw = (torch.randn(V, Ht, generator=g) / Ht ** 0.5).to(dtype)
    labels = None
    if with_labels:
        labels = torch.randint(0, V, (BT,), generator=g)
        labels[torch.rand(BT, generator=g) < 0.2] = -100
    return si, sw, ti, tw, labels


def _oracle(si, sw, ti, tw, labels, beta, T, grads=None):
    dt = si.dtype

    def f(a, b):
        ls = (a.double() @ b.double().T).to(dt).double()
        lt = (ti.double() @ tw.double().T).to(dt).double()
        X = torch.log_softmax(ls / T, -1)
        Y = torch.log_softmax(lt / T, -1)
        return oracle.jsd_ref(X, Y, beta, labels)
    return oracle.fwd_bwd(f, [si, sw], grads, dtype=torch.float64)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("beta", [0.0, 0.5, 1.0])
@pytest.mark.parametrize("shape,chunk", [((96, 256, 256, 1000), 8192), ((300, 128, 64, 4096), 8192),
                                         ((200, 64, 96, 520), 64), ((513, 256, 128, 2048), 128)])
def test_fused_linear_jsd(dtype, beta, shape, chunk):
    BT, H, Ht, V = shape
    T = 1.0 if beta != 0.5 else 2.0
    si, sw, ti, tw, labels = _case(BT, H, Ht, V, dtype, BT + H + V + int(beta * 8))
    (l_ref,), (dh_ref, dw_ref) = _oracle(si, sw, ti, tw, labels, beta, T)
    dev = gpu()
    sg = si.to(dev).requires_grad_(True)
    wg = sw.to(dev).requires_grad_(True)
    if chunk != 8192:
        loss, gi, gw = fj.fused_linear_jsd_forward(sg.detach(), wg.detach(), ti.to(dev), tw.to(dev), labels.to(dev),
                                                   beta, T, -100, compute_grad=True, chunk=chunk)
        sg.grad, wg.grad = gi, gw
    else:
        loss = FusedLinearJSDLoss(beta, T)(sg, wg, ti.to(dev), tw.to(dev), labels.to(dev))
        loss.backward()
    n = max(int((labels != -100).sum()), 1)
    lt = dict(rtol=1e-5, atol=1e-5) if dtype == torch.float32 else dict(rtol=2e-3, atol=2e-3)
    assert_close(loss, l_ref, name="loss", **lt)
    tt = tol(dtype)
    assert_close(sg.grad.float() * n, dh_ref * n, name="dinput*n", **tt)
    assert_close(wg.grad.float() * n, dw_ref * n, name="dweight*n", **tt)
    # The gradients come back in the input dtype. At these sizes |dinput| is ~1e-6, deep in fp16's
    # subnormal range, where the rounding alone moves the Frobenius norm by up to 3%: compare with the
    # oracle rounded to that dtype (the reference returns the same dtype, fused_linear_jsd.py:201-203).
    assert rel_fro(sg.grad, dh_ref.to(dtype)) < 1e-2 and rel_fro(wg.grad, dw_ref.to(dtype)) < 1e-2
    assert torch.count_nonzero(sg.grad[(labels == -100).to(dev)]).item() == 0


def test_fused_linear_jsd_no_labels_upstream_and_repeat():
    dtype = torch.bfloat16
    si, sw, ti, tw, _ = _case(130, 128, 128, 3000, dtype, 31, with_labels=False)
    up = torch.tensor(2.5)
    (l_ref,), (dh_ref, dw_ref) = _oracle(si, sw, ti, tw, None, 0.3, 1.0, [up])
    dev = gpu()
    sg = si.to(dev).requires_grad_(True)
    wg = sw.to(dev).requires_grad_(True)
    loss = hilda_fused_linear_jsd(sg, wg, ti.to(dev), tw.to(dev), None, 0.3)
    loss.backward(up.to(dev), retain_graph=True)
    assert_close(loss, l_ref, name="loss", rtol=2e-3, atol=2e-3)
    assert rel_fro(sg.grad, dh_ref.to(dtype)) < 1e-2 and rel_fro(wg.grad, dw_ref.to(dtype)) < 1e-2
    g1i, g1w = sg.grad.clone(), wg.grad.clone()
    sg.grad, wg.grad = None, None
    loss.backward(torch.tensor(5.0, device=dev))
    assert_close(sg.grad.float(), g1i.float() * 2, name="repeat dinput", rtol=1.6e-2, atol=1e-6)
    assert_close(wg.grad.float(), g1w.float() * 2, name="repeat dweight", rtol=1.6e-2, atol=1e-6)


def test_fused_linear_jsd_reference_bench_shape():
    """benchmarks/bench_fused_linear_jsd.py:78-96: (256, 4096, 32000) fp16, beta 1/2."""
    dtype = torch.float16
    si, sw, ti, tw, _ = _case(256, 4096, 4096, 32000, dtype, 77, with_labels=False)
    (l_ref,), (dh_ref, dw_ref) = _oracle(si, sw, ti, tw, None, 0.5, 1.0)
    dev = gpu()
    sg = si.to(dev).requires_grad_(True)
    wg = sw.to(dev).requires_grad_(True)
    loss = hilda_fused_linear_jsd(sg, wg, ti.to(dev), tw.to(dev))
    loss.backward()
    assert_close(loss, l_ref, name="loss", rtol=2e-3, atol=2e-3)
    assert rel_fro(sg.grad, dh_ref.to(dtype)) < 1e-2 and rel_fro(wg.grad, dw_ref.to(dtype)) < 1e-2


def test_fused_linear_jsd_fp32_reference_check():
    """benchmarks/bench_fused_linear_jsd.py:45-66,72-96: the reference's fp32 checks at (256, 4096, 32000),
    every input ~ N(0, 0.02), beta 1/2; against the fp64 oracle at rtol 1e-5, atol 1e-5, the gradients
    also multiplied back by the 1/BT of the mean."""
    dtype = torch.float32
    g = torch.Generator().manual_seed(78)
    si, sw, ti, tw = (0.02 * torch.randn(*sh, generator=g) for sh in ((256, 4096), (32000, 4096), (256, 4096),
                                                                      (32000, 4096)))
    (l_ref,), (dh_ref, dw_ref) = _oracle(si, sw, ti, tw, None, 0.5, 1.0)
    dev = gpu()
    sg = si.to(dev).requires_grad_(True)
    wg = sw.to(dev).requires_grad_(True)
    loss = hilda_fused_linear_jsd(sg, wg, ti.to(dev), tw.to(dev))
    loss.backward()
    tt = tol(dtype)
    assert_close(loss, l_ref, name="loss", **tt)
    # With every input ~ N(0, 0.02) the two distributions are nearly equal and the gradient entries (~1e-9)
    # are differences of close fp32 terms, so atol 1e-5 would pass anything: each element above a floor is
    # compared with no absolute slack against the oracle with the reference kernel's fp32 log-probs
    # (logits rounded to fp32, log-softmax and JSD in fp32, fused_linear_jsd.py:163-188). Its own distance
    # from the fp64 oracle bounds what fp32 cancellation leaves: at most 1.5e-4 relative above a tenth of
    # the largest entry, 1.5e-3 above a hundredth (dW; dX less). The kernel's log-probs round independently
    # of the oracle's, so the bounds below allow about 3x that.
    d32h, d32w = _fp32_logprob_grads(si, sw, ti, tw, 0.5, 1.0)
    for name, got, ref in (("dinput", sg.grad, d32h), ("dweight", wg.grad, d32w)):
        got = got.double().cpu()
        m = ref.abs().max()
        for floor, rtol in ((0.1, 5e-4), (0.01, 5e-3)):
            sel = ref.abs() > floor * m
            rel = (got - ref).abs()[sel] / ref.abs()[sel]
            assert rel.max().item() <= rtol, f"{name}: {rel.max().item():.3e} above {floor} of the largest entry"
    # and the relative Frobenius error against fp64 (fp32 cancellation: 1.7e-5 measured)
    assert rel_fro(sg.grad, dh_ref) < 1e-4 and rel_fro(wg.grad, dw_ref) < 1e-4


def _fp32_logprob_grads(si, sw, ti, tw, beta, T):
    """dinput, dweight (fp64) of JSD with the log-probs formed in fp32 from fp32-rounded logits, as the
    reference's FusedLinearJSD kernel does; the logit gradient then carried through the linear in fp64."""
    zs = (si.double() @ sw.double().T).float().requires_grad_(True)
    zt = (ti.double() @ tw.double().T).float()
    loss = oracle.jsd_ref(torch.log_softmax(zs / T, -1), torch.log_softmax(zt / T, -1), beta, None)
    loss.backward()
    d = zs.grad.double()
    return d @ sw.double(), d.T @ si.double()


def test_fused_linear_jsd_all_ignored_and_types():
    dtype = torch.bfloat16
    si, sw, ti, tw, _ = _case(40, 64, 64, 512, dtype, 5, with_labels=False)
    dev = gpu()
    sg = si.to(dev).requires_grad_(True)
    wg = sw.to(dev).requires_grad_(True)
    loss = hilda_fused_linear_jsd(sg, wg, ti.to(dev), tw.to(dev), torch.full((40,), -100, device=dev))
    loss.backward()
    assert float(loss.detach()) == 0.0
    assert torch.count_nonzero(sg.grad).item() == 0 and torch.count_nonzero(wg.grad).item() == 0
    with pytest.raises(TypeError):
        hilda_fused_linear_jsd(si.double().to(dev), sw.double().to(dev), ti.double().to(dev), tw.double().to(dev))


@pytest.mark.parametrize("labels_kind,BT,chunk", [("dead_block", 600, 64), ("dead_block", 300, 64),
                                                  ("none", 600, 64)])
def test_fused_linear_jsd_compaction_and_chunks(labels_kind, BT, chunk):
    """With labels the ignored rows are compacted away before the GEMMs (here whole chunks of them, on the fp32
    dW accumulator path at BT 600 and the single-dW-GEMM path at BT 300); without labels every row runs in place."""
    H, Ht, V = 64, 96, 520
    dtype = torch.bfloat16
    si, sw, ti, tw, labels = _case(BT, H, Ht, V, dtype, BT + 7, with_labels=labels_kind != "none")
    if labels is not None:
        labels[100:BT - 50] = -100
    (l_ref,), (dh_ref, dw_ref) = _oracle(si, sw, ti, tw, labels, 0.5, 1.0)
    dev = gpu()
    print(f"FLJSD compaction {labels_kind} BT={BT} chunk={chunk}", flush=True)
    loss, gi, gw = fj.fused_linear_jsd_forward(si.to(dev), sw.to(dev), ti.to(dev), tw.to(dev),
                                               None if labels is None else labels.to(dev), 0.5, 1.0, -100,
                                               compute_grad=True, chunk=chunk)
    n = BT if labels is None else max(int((labels != -100).sum()), 1)
    assert_close(loss, l_ref, name="loss", rtol=2e-3, atol=2e-3)
    tt = tol(dtype)
    assert_close(gi.float() * n, dh_ref * n, name="dinput*n", **tt)
    assert_close(gw.float() * n, dw_ref * n, name="dweight*n", **tt)
    assert rel_fro(gi, dh_ref.to(dtype)) < 1e-2 and rel_fro(gw, dw_ref.to(dtype)) < 1e-2
    if labels is not None:
        assert torch.count_nonzero(gi[(labels == -100).to(dev)]).item() == 0


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("labels_on", [True, False])
@pytest.mark.parametrize("budget", [None, -1])
def test_fused_linear_jsd_any_shape(dtype, labels_on, budget):
    """Student H, teacher Ht and V that are not multiples of 8: padded rows, weight copies and a padded chunk
    stride (zeros past V in both logits chunks), in the default and the unlimited plan, against the oracle."""
    BT, H, Ht, V = 96, 257, 131, 1003
    si, sw, ti, tw, labels = _case(BT, H, Ht, V, dtype, 5, with_labels=labels_on)
    (l_ref,), (dh_ref, dw_ref) = _oracle(si, sw, ti, tw, labels, 0.5, 1.0)
    dev = gpu()
    print(f"FLJSD any shape {dtype} labels={labels_on} budget={budget}", flush=True)
    loss, gi, gw = fj.fused_linear_jsd_forward(si.to(dev), sw.to(dev), ti.to(dev), tw.to(dev),
                                               None if labels is None else labels.to(dev), 0.5, 1.0, -100,
                                               compute_grad=True, chunk=32, workspace_budget=budget)
    n = BT if labels is None else max(int((labels != -100).sum()), 1)
    lt = tol(dtype) if dtype == torch.float32 else dict(rtol=2e-3, atol=2e-3)
    assert_close(loss, l_ref, name="loss", **lt)
    tt = tol(dtype)
    assert_close(gi.float() * n, dh_ref * n, name="dinput*n", **tt)
    assert_close(gw.float() * n, dw_ref * n, name="dweight*n", **tt)


@pytest.mark.parametrize("form", ["out,wmn,dmn", "acc,wt,dmn", "defer,wmn,dt"])
def test_fused_linear_jsd_plan_forms(form, monkeypatch):
    BT, H, Ht, V = 300, 128, 64, 2000
    dtype = torch.bfloat16
    si, sw, ti, tw, labels = _case(BT, H, Ht, V, dtype, 6)
    monkeypatch.setenv("HILDA_FL_FORM", form)
    (l_ref,), (dh_ref, dw_ref) = _oracle(si, sw, ti, tw, labels, 0.5, 1.0)
    dev = gpu()
    loss, gi, gw = fj.fused_linear_jsd_forward(si.to(dev), sw.to(dev), ti.to(dev), tw.to(dev), labels.to(dev), 0.5,
                                               1.0, -100, compute_grad=True, chunk=64, workspace_budget=-1)
    n = max(int((labels != -100).sum()), 1)
    assert_close(loss, l_ref, name="loss", rtol=2e-3, atol=2e-3)
    assert rel_fro(gi, dh_ref.to(dtype)) < 1e-2 and rel_fro(gw, dw_ref.to(dtype)) < 1e-2
    assert_close(gw.float() * n, dw_ref * n, name="dweight*n", **tol(dtype))


def _reference_chunk_bytes(N, H, V, es=2):
    """What fused_linear_jsd_forward holds at once in its dW product (fused_linear_jsd.py:133-135,159-203), 16-bit
    inputs: per logit of its chunk the two logits, their fp32 log-softmax copies, the fp32 dX and dlogits and the
    dlogits cast back, 22 bytes; plus the [V, H] product dlogits^T X."""
    inc = -(-V // H)
    per = -(-N // inc)
    cs = min(1 << (per - 1).bit_length(), N)
    return cs * V * 22 + V * H * es


@pytest.mark.parametrize("N,V", [(4096, 32000), (2048, 128256)])
def test_fused_linear_jsd_reference_memory_configs(N, V):
    """benchmarks/bench_fused_linear_jsd.py:163-165,180: the reference's memory configs, fp16, beta 1/2, no
    labels. The default plan's workspace is within what the reference's chunk loop holds at once, and its loss
    and gradients agree with the unlimited plan's; the student gradient of sampled rows matches the fp64 oracle
    (row r's dX depends on row r alone, scaled by 1/N)."""
    H, dtype = 4096, torch.float16
    dev = gpu()
    g = torch.Generator(device=dev).manual_seed(N + V)
    # logits of standard deviation 3: with unit logits the 1/N-scaled dlogits all round to zero in fp16 (in the
    # reference's arithmetic as here), with much larger ones the softmaxes saturate and the gradient vanishes
    si = torch.randn(N, H, generator=g, device=dev).to(dtype)
    sw = (3 * torch.randn(V, H, generator=g, device=dev) / H ** 0.5).to(dtype)
    ti = torch.randn(N, H, generator=g, device=dev).to(dtype)
    tw = (3 * torch.randn(V, H, generator=g, device=dev) / H ** 0.5).to(dtype)
    plan = fj.fused_linear_jsd_plan(N, H, V, dtype)
    assert plan["workspace_bytes"] <= _reference_chunk_bytes(N, H, V)
    out = {}
    for budget in (None, "fastest"):
        loss, gi, gw = fj.fused_linear_jsd_forward(si, sw, ti, tw, None, 0.5, 1.0, -100, compute_grad=True,
                                                   workspace_budget=budget)
        torch.cuda.synchronize()
        out[budget] = (loss.float().item(), gi.float(), gw.float())
    (ld, gid, gwd), (lf, gif, gwf) = out[None], out["fastest"]
    assert abs(ld - lf) <= 1e-5 * abs(lf)
    assert rel_fro(gid, gif) < 2e-3 and rel_fro(gwd, gwf) < 2e-3
    rows = torch.tensor([0, 1, N // 2, N - 1])
    w64, tw64 = sw.cpu().double(), tw.cpu().double()
    # the rows' logits rounded to fp16 as the GEMMs return them, their dlogits from the oracle's JSD by autograd,
    # rounded to fp16 at the op's 1/N scale as the reference rounds them (fused_linear_jsd.py:201), times W
    ls = (si[rows].cpu().double() @ w64.T).to(dtype).double().requires_grad_(True)
    lt = (ti[rows].cpu().double() @ tw64.T).to(dtype).double()
    oracle.jsd_ref(torch.log_softmax(ls, -1), torch.log_softmax(lt, -1), 0.5, None).backward()
    dl = (ls.grad * (len(rows) / N)).to(dtype).double()  # the oracle's mean is over the sampled rows
    assert dl.abs().max() > 0  # the check is not vacuous
    dh = dl @ w64
    got = gid[rows.to(dev)].cpu().double()
    assert got.abs().max() > 0
    # dX at this scale sits in fp16's subnormal range (spacing 2^-24): one rounding of the fp32 sum apart
    assert_close(got, dh, name="dinput rows", rtol=2e-3, atol=2.0 ** -24)
