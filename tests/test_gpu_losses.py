"""GPU parity: CrossEntropy, selective log-softmax and GRPO HIP kernels vs the CPU oracle.

Mirrors benchmarks/bench_cross_entropy.py (loss, dlogits, ignored-row gradient,
tightened to exactly zero) and benchmarks/bench_grpo.py (loss, gradient) and
adds: row-engine variants (register-resident 256/512/1024-lane, streaming,
unvectorised; test_gpu_row_engine.py reaches every form), reductions, ignore_index=-1, all-ignored, upstream grads != 1,
repeated backward, masks of several dtypes, temperature, and the full C3/C4
shapes (row slices against the oracle plus size-independent properties).

Mean-reduced gradients are tiny (|g| <= 1/n_valid), so besides the required
tolerance they are compared after multiplying back by the reduction scale and
by relative Frobenius error.
"""
import math

import pytest
import torch

import oracle
import workloads
from _util import assert_close, rel_fro, tol, gpu

from kernels import hilda_cross_entropy, CrossEntropyLoss, hilda_grpo_loss, GRPOLoss, fused_selective_log_softmax
from kernels import cross_entropy as ce_mod
from kernels import grpo_loss as grpo_mod

pytestmark = pytest.mark.gpu

DTYPES = [torch.float32, torch.bfloat16, torch.float16]


def _ce_case(N, V, dtype, ignore_frac, seed, scale=2.0):
    g = torch.Generator().manual_seed(seed)
    logits = (scale * torch.randn(N, V, generator=g)).to(dtype)
    t = torch.randint(0, V, (N,), generator=g)
    t[torch.rand(N, generator=g) < ignore_frac] = -100
    return logits, t


# V values cover: 256-lane resident (1000, 4096; 32000 in 16-bit), 512-lane resident (32000 fp32),
# 1024-lane resident (128256 in 16-bit), streaming (128256 fp32, 200000), unvectorised (1001)
@pytest.mark.parametrize("V", [1000, 1001, 4096, 32000, 128256, 200000])
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("reduction", ["mean", "sum", "none"])
def test_cross_entropy_train(V, dtype, reduction):
    N = 24 if V >= 100000 else 64
    logits, t = _ce_case(N, V, dtype, 0.2, V + N)
    (l_ref,), (d_ref,) = oracle.fwd_bwd(lambda z: oracle.cross_entropy_ref(z, t, -100, reduction), [logits],
                                        [torch.ones(N)] if reduction == "none" else None, dtype=torch.float64)
    lg = logits.to(gpu()).requires_grad_(True)
    loss = hilda_cross_entropy(lg, t.to(gpu()), -100, reduction)
    (loss.sum() if reduction == "none" else loss).backward()
    t32 = tol(dtype)
    lt = dict(rtol=1e-5, atol=1e-5) if dtype == torch.float32 else dict(rtol=2e-3, atol=2e-3)
    assert_close(loss, l_ref, name="loss", **lt)
    n_valid = int((t != -100).sum())
    s = n_valid if reduction == "mean" else 1
    assert_close(lg.grad, d_ref, name="dlogits", **t32)
    assert_close(lg.grad.float() * s, d_ref * s, name="dlogits*n_valid", **t32)
    # against the oracle rounded to the storage dtype: fp16 stores these tiny
    # gradients as subnormals on both sides, exactly as the reference does
    assert rel_fro(lg.grad, d_ref.to(dtype)) < (1e-5 if dtype == torch.float32 else 1e-2)
    ign = (t == -100).to(gpu())
    assert torch.count_nonzero(lg.grad[ign]).item() == 0, "ignored rows must have exactly zero gradient"


@pytest.mark.parametrize("reduction", ["mean", "sum", "none"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_cross_entropy_inference(reduction, dtype):
    logits, t = _ce_case(48, 32000, dtype, 0.25, 5)
    ref = oracle.cross_entropy_ref(logits.double(), t, -100, reduction)
    out = hilda_cross_entropy(logits.to(gpu()), t.to(gpu()), -100, reduction)
    lt = dict(rtol=1e-5, atol=1e-5) if dtype == torch.float32 else dict(rtol=2e-3, atol=2e-3)
    assert_close(out, ref, name="loss", **lt)


def test_cross_entropy_edge_cases():
    dev = gpu()
    logits, t = _ce_case(16, 5000, torch.float32, 0.0, 7)
    # ignore_index = -1 is "ignore nothing"
    lg = logits.to(dev).requires_grad_(True)
    out = hilda_cross_entropy(lg, t.to(dev), ignore_index=-1)
    out.backward()
    (l_ref,), (d_ref,) = oracle.fwd_bwd(lambda z: oracle.cross_entropy_ref(z, t, -1), [logits], dtype=torch.float64)
    assert_close(out, l_ref, name="loss(-1)", rtol=1e-5, atol=1e-5)
    assert_close(lg.grad, d_ref, name="grad(-1)", rtol=1e-5, atol=1e-5)
    # every row ignored: loss 0 (not NaN) and zero gradient (cross_entropy.py:141,248)
    lg = logits.to(dev).requires_grad_(True)
    out = hilda_cross_entropy(lg, torch.full((16,), -100, device=dev))
    out.backward()
    assert out.item() == 0.0 and torch.count_nonzero(lg.grad).item() == 0
    assert hilda_cross_entropy(logits.to(dev), torch.full((16,), -100, device=dev)).item() == 0.0
    # uniform logits: loss = log V
    u = torch.zeros(8, 5000, device=dev, requires_grad=True)
    assert math.isclose(hilda_cross_entropy(u, torch.arange(8, device=dev)).item(), math.log(5000), rel_tol=1e-6)
    # module, int32 targets
    m = CrossEntropyLoss(ignore_index=-100, reduction="sum")
    assert_close(m(logits.to(dev), t.to(dev).int()), oracle.cross_entropy_ref(logits.double(), t, -100, "sum"),
                 name="module", rtol=1e-5, atol=1e-4)


def test_cross_entropy_upstream_grad_and_retain_graph():
    dev = gpu()
    logits, t = _ce_case(32, 8000, torch.float32, 0.1, 9)
    lg = logits.to(dev).requires_grad_(True)
    loss = hilda_cross_entropy(lg, t.to(dev))
    (3.0 * loss).backward(retain_graph=True)
    (_,), (d_ref,) = oracle.fwd_bwd(lambda z: oracle.cross_entropy_ref(z, t), [logits], dtype=torch.float64)
    assert_close(lg.grad, 3.0 * d_ref, name="3*grad", rtol=1e-5, atol=1e-5)
    g1 = lg.grad.clone()
    lg.grad = None
    (0.5 * loss).backward()  # second backward through the same graph
    assert_close(lg.grad, 0.5 * d_ref, name="0.5*grad", rtol=1e-5, atol=1e-5)
    assert_close(g1, 3.0 * d_ref, name="first grad unchanged", rtol=1e-5, atol=1e-5)
    # reduction='none' with a per-row upstream gradient
    lg2 = logits.to(dev).requires_grad_(True)
    w = torch.randn(32)
    hilda_cross_entropy(lg2, t.to(dev), reduction="none").backward(w.to(dev))
    (_,), (d2,) = oracle.fwd_bwd(lambda z: oracle.cross_entropy_ref(z, t, -100, "none"), [logits], [w],
                                 dtype=torch.float64)
    assert_close(lg2.grad, d2, name="per-row grad", rtol=1e-5, atol=1e-5)


def _strict_tail(actual, expected, dtype, scale, name):
    """Every gradient element the reference keeps (|expected| * scale > 1e-30) within the relative
    tolerance and with no absolute slack, so a flushed or coarsened tail of small probabilities
    fails. fp32: rtol 5e-5, since 2^(x*log2(e) - lse) of logits |x| ~ 60 carries the rounding of
    a ~100-magnitude exponent (a few 1e-6), which the reference's fp32 exp shares. fp16: the
    reference's own output is fp16, so elements below fp16's normal range (6.1e-5) are compared
    with one subnormal step (2^-24) of slack."""
    a = actual.detach().to("cpu", torch.float64) * scale
    e = expected.detach().to("cpu", torch.float64) * scale
    sel = e.abs() > 1e-30
    assert sel.any()
    rtol = {torch.float32: 5e-5, torch.bfloat16: 1.6e-2, torch.float16: 1.6e-2}[dtype]
    if dtype == torch.float16:
        a, e = actual.detach().to("cpu", torch.float64), expected.detach().to("cpu", torch.float64)
        sel = e.abs() > 1e-30 / scale
        err = (a - e).abs()[sel]
        bound = rtol * e.abs()[sel] + 2.0 ** -24
    else:
        err = (a - e).abs()[sel]
        bound = rtol * e.abs()[sel]
    bad = int((err > bound).sum())
    if bad:
        rel = err / e.abs()[sel]
        k = int(rel.argmax())
        where = tuple(int(i) for i in torch.nonzero(sel)[k])
        raise AssertionError(f"{name}: {bad} of {int(sel.sum())} elements off, worst at {where}: "
                             f"{a[sel][k].item():.6e} vs {e[sel][k].item():.6e} (rel {rel[k].item():.3e}); "
                             f"zeros where the oracle is nonzero: {int((a[sel] == 0).sum())}")


def _wide_ce_case(N, V, dtype, seed):
    """Logits ~ N(0, 8) (trained-LM width) with row 1 peaked (one logit 30 above the row's max)."""
    logits, t = _ce_case(N, V, torch.float32, 0.15, seed, scale=8.0)
    logits[1, 777] = logits[1].max() + 30.0
    t[1] = 5
    t[0] = -100
    return logits.to(dtype), t


# V: 256-lane resident (32000), 1024-lane resident (128256, 151936), streaming (200000)
@pytest.mark.parametrize("V", [32000, 128256, 151936, 200000])
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("reduction", ["mean", "sum"])
def test_cross_entropy_wide_logits(V, dtype, reduction):
    """Wide and peaked rows: the gradient's small probabilities (down to 1e-30) match the oracle
    (kernels/cross_entropy.py:159-166 computes exp in fp32 and rounds once to the logits dtype);
    target entries against oracle.exact_target_grad."""
    N = 12
    logits, t = _wide_ce_case(N, V, dtype, V + 3)
    print(f"wide CE V={V} {dtype} {reduction}", flush=True)
    (l_ref,), (d_ref,) = oracle.fwd_bwd(lambda z: oracle.cross_entropy_ref(z, t, -100, reduction), [logits],
                                        dtype=torch.float64)
    d_ref = oracle.exact_target_grad(d_ref, t)
    lg = logits.to(gpu()).requires_grad_(True)
    loss = hilda_cross_entropy(lg, t.to(gpu()), -100, reduction)
    loss.backward()
    lt = dict(rtol=1e-5, atol=1e-5) if dtype == torch.float32 else dict(rtol=2e-3, atol=2e-3)
    assert_close(loss, l_ref, name="loss", **lt)
    n_valid = int((t != -100).sum())
    s = n_valid if reduction == "mean" else 1
    assert_close(lg.grad, d_ref, name="dlogits", **tol(dtype))
    _strict_tail(lg.grad, d_ref, dtype, s, "dlogits tail")
    assert torch.count_nonzero(lg.grad[(t == -100).to(gpu())]).item() == 0


def test_cross_entropy_c3_config():
    """C3: logits [8192, 128256] bf16 ~ N(0,2), 10% ignored, mean; generated on the GPU.

    All rows: ignored rows exactly zero, valid rows' gradients sum to ~0, loss
    against the oracle's chunked fp64 sum. A 256-row slice: per-element
    gradients against the oracle."""
    dev = gpu()
    c = workloads.c3_cross_entropy(device=dev)
    logits, t = c["logits"], c["targets"]
    lg = logits.requires_grad_(True)
    loss = hilda_cross_entropy(lg, t)
    loss.backward()
    grad = lg.grad
    valid = t != -100
    n_valid = int(valid.sum())
    assert torch.count_nonzero(grad[~valid]).item() == 0
    row_sums = grad[valid].float().sum(-1) * n_valid
    assert row_sums.abs().max().item() < 5e-2  # sum_j (p_j - onehot_j) = 0 up to bf16 rounding
    total = 0.0
    for i in range(0, 8192, 1024):
        total += oracle.cross_entropy_ref(logits[i:i + 1024].detach().cpu().double(), t[i:i + 1024].cpu(), -100,
                                          "sum").item()
    assert math.isclose(loss.item(), total / n_valid, rel_tol=2e-5, abs_tol=1e-5)
    sl = slice(1000, 1256)
    ls, ts = logits[sl].detach().cpu(), t[sl].cpu()
    (_,), (d_ref,) = oracle.fwd_bwd(lambda z: oracle.cross_entropy_ref(z, ts, -100, "sum"), [ls],
                                    dtype=torch.float64)
    assert_close(grad[sl].float() * n_valid, d_ref, name="slice grad * n_valid", **tol(torch.bfloat16))
    assert rel_fro(grad[sl].float() * n_valid, d_ref) < 1e-2


def _ce_raw(logits, t, ignore_index, reduction, ws_bytes):
    """hk_cross_entropy_fwd_grad through the C ABI with a workspace of ws_bytes."""
    from kernels import _lib
    n, V = logits.shape
    d = torch.empty_like(logits)
    rows = torch.empty(n, dtype=torch.float32, device=logits.device)
    loss = torch.empty((), dtype=torch.float32, device=logits.device)
    ws = torch.zeros(ws_bytes, dtype=torch.uint8, device=logits.device)
    _lib.call("hk_cross_entropy_fwd_grad", d.data_ptr(), rows.data_ptr(), loss.data_ptr(), logits.data_ptr(),
              t.data_ptr(), n, V, V, V, int(ignore_index), _lib.REDUCTION[reduction], _lib.dtype_code(logits),
              ws.data_ptr(), ws_bytes, _lib.stream_of(logits.device))
    return d, rows, loss, int(ws[:4].view(torch.int32)[0])


# row counts around the grid sizes (256 and 1024 blocks) and a handful of rows
@pytest.mark.parametrize("V,N", [(128256, 300), (128256, 7), (151936, 260), (32000, 1100), (4096, 3000)])
@pytest.mark.parametrize("ignore_index", [-100, -1])
def test_cross_entropy_plan_matches_strided(V, N, ignore_index):
    """With the full workspace the live rows are dealt out by the launch plan;
    with 256 bytes they are strided over the grid. Both must agree bit for bit,
    with ignored rows, targets out of range (NaN rows) and ignore_index -1."""
    from kernels import _lib
    dev = gpu()
    logits, t = _ce_case(N, V, torch.bfloat16, 0.3, V + N)
    t[1::11] = V + 5  # out of range: a NaN row, never live
    t[2::13] = -7
    if ignore_index == -1:
        t[t == -100] = 3
    logits, t = logits.to(dev), t.to(dev)
    full = _lib.load().hk_cross_entropy_workspace_size(N)
    assert full >= 256 + 4 * N
    d1, r1, l1, nv1 = _ce_raw(logits, t, ignore_index, "mean", full)
    d0, r0, l0, nv0 = _ce_raw(logits, t, ignore_index, "mean", 256)
    valid = (t != ignore_index) if ignore_index != -1 else torch.ones_like(t, dtype=torch.bool)
    assert nv1 == nv0 == int(valid.sum())
    assert torch.equal(d1.view(torch.int16), d0.view(torch.int16))
    assert torch.equal(r1.view(torch.int32), r0.view(torch.int32))
    live = valid & (t >= 0) & (t < V)
    assert torch.isnan(d1[valid & ~live].float()).all()
    (_,), (d_ref,) = oracle.fwd_bwd(lambda z: oracle.cross_entropy_ref(z, t[live].cpu(), -100, "sum"),
                                    [logits[live].cpu()], dtype=torch.float64)
    assert_close(d1[live].float() * nv1, d_ref, name="planned dlogits * n_valid", **tol(torch.bfloat16))


# --------------------------------------------------------------------------
# selective log-softmax and GRPO
# --------------------------------------------------------------------------
def _grpo_case(B, L, V, dtype, seed, mask_kind="int32", beta=0.1, with_old=True):
    g = torch.Generator().manual_seed(seed)
    logits = (2 * torch.randn(B, L + 1, V, generator=g)).to(dtype)
    ids = torch.randint(0, V, (B, L), generator=g)
    adv = torch.randn(B, generator=g)
    logp = oracle.selective_log_softmax_ref(logits.float(), ids)
    old = logp + 0.3 * torch.randn(B, L, generator=g) if with_old else None
    ref = logp + 0.3 * torch.randn(B, L, generator=g) if beta != 0 else None
    lens = torch.randint(max(1, L // 3), L + 1, (B,), generator=g)
    m = torch.arange(L)[None, :] < lens[:, None]
    if mask_kind is None:
        mask = None
    elif mask_kind == "float":
        mask = m.float() * (0.5 + torch.rand(B, L, generator=g))
    else:
        mask = m.to({"int32": torch.int32, "bool": torch.bool, "int64": torch.int64}[mask_kind])
    return logits, ids, adv, old, ref, mask


@pytest.mark.parametrize("V", [500, 4096, 32000, 151936])
@pytest.mark.parametrize("dtype", DTYPES)
def test_selective_log_softmax(V, dtype):
    B, L = (2, 6) if V > 100000 else (3, 17)
    logits, ids, *_ , mask = _grpo_case(B, L, V, dtype, V, "int32")
    full_ids = torch.cat([torch.zeros(B, 1, dtype=torch.int64), ids], dim=1)  # (B, L+1): the op takes ids[:, -L:]
    full_mask = torch.cat([torch.ones(B, 1, dtype=torch.int32), mask], dim=1)
    for T in (1.0, 0.7):
        ref = oracle.selective_log_softmax_ref(logits.double(), full_ids, T, full_mask)
        out = fused_selective_log_softmax(logits.to(gpu()), full_ids.to(gpu()), T, full_mask.to(gpu()))
        lt = dict(rtol=1e-5, atol=1e-5) if dtype == torch.float32 else dict(rtol=1e-4, atol=1e-4)
        assert_close(out, ref, name=f"logp T={T}", **lt)
        assert torch.count_nonzero(out.cpu()[mask == 0]).item() == 0


CASES = [
    # B, L, V, mask, beta, with_old, T, eps_lo, eps_hi
    (3, 16, 500, "int32", 0.1, True, 1.0, 0.2, 0.2),
    (2, 9, 4096, "bool", 0.0, True, 1.0, 0.2, 0.28),
    (4, 12, 32000, None, 0.1, False, 1.0, 0.2, 0.2),
    (2, 5, 32000, "float", 0.04, True, 0.7, 0.1, 0.3),
    (2, 4, 151936, "int64", 0.1, True, 1.0, 0.2, 0.2),
    (2, 7, 1001, "int32", 0.1, True, 1.0, 0.2, 0.2),
]


@pytest.mark.parametrize("case", CASES)
@pytest.mark.parametrize("dtype", DTYPES)
def test_grpo_loss(case, dtype):
    B, L, V, mk, beta, with_old, T, el, eh = case
    logits, ids, adv, old, ref, mask = _grpo_case(B, L, V, dtype, B * 100 + L, mk, beta, with_old)
    outs, (d_ref,) = oracle.fwd_bwd(
        lambda z: oracle.grpo_loss_ref(z, ids, adv.double(), None if old is None else old.double(),
                                       None if ref is None else ref.double(), mask, T, beta, el, eh),
        [logits], dtype=torch.float64)
    dev = gpu()
    lg = logits.to(dev).requires_grad_(True)
    loss, kl, clip = hilda_grpo_loss(lg, ids.to(dev), adv.to(dev), None if old is None else old.to(dev),
                                     None if ref is None else ref.to(dev), None if mask is None else mask.to(dev),
                                     T, beta, el, eh)
    loss.backward()
    lt = dict(rtol=1e-5, atol=1e-5) if dtype == torch.float32 else dict(rtol=1.6e-2, atol=1e-2)
    assert_close(loss, outs[0], name="loss", **lt)
    if beta != 0:
        assert_close(kl, outs[1], name="kl_mean", **lt)
    else:
        assert kl is None
    if dtype == torch.float32:
        assert_close(clip, outs[2], name="clip_ratio", rtol=1e-6, atol=1e-6)
    t = tol(dtype)
    scale = B * L  # undo the 1/(len_b * B) reduction scale
    assert_close(lg.grad.float() * scale, d_ref * scale, name="dlogits*B*L", **t)
    assert rel_fro(lg.grad, d_ref.to(dtype)) < (1e-5 if dtype == torch.float32 else 1e-2)
    # masked tokens and the last position get exactly zero gradient
    assert torch.count_nonzero(lg.grad[:, -1]).item() == 0
    if mask is not None:
        assert torch.count_nonzero(lg.grad[:, :-1][mask.to(dev) == 0]).item() == 0


@pytest.mark.parametrize("V", [32000, 151936])
@pytest.mark.parametrize("dtype", DTYPES)
def test_grpo_loss_wide_logits(V, dtype):
    """GRPO's gradient rows on N(0, 8) logits with one peaked position (its id the peak, so
    1 - p_id ~ 1e-13): the small probabilities and the id entries match the oracle with no
    absolute slack (kernels/grpo_loss.py:229-234); the oracle's id entries are formed exactly
    (oracle.exact_target_grad), since fp64 autograd's p_id - 1 loses them."""
    B, L = 2, 6
    g = torch.Generator().manual_seed(V + 17)
    logits = 8 * torch.randn(B, L + 1, V, generator=g)
    logits[0, 2, 99] = logits[0, 2].max() + 30.0
    logits = logits.to(dtype)
    ids = torch.randint(0, V, (B, L), generator=g)
    ids[0, 2] = 99
    adv = torch.randn(B, generator=g)
    logp = oracle.selective_log_softmax_ref(logits.double(), ids)
    old = (logp + 0.05 * torch.randn(B, L, generator=g, dtype=torch.float64)).float()
    ref = (logp + 0.1 * torch.randn(B, L, generator=g, dtype=torch.float64)).float()
    mask = torch.ones(B, L, dtype=torch.int32)
    mask[1, 4:] = 0
    print(f"wide GRPO V={V} {dtype}", flush=True)
    outs, (d_ref,) = oracle.fwd_bwd(
        lambda z: oracle.grpo_loss_ref(z, ids, adv.double(), old.double(), ref.double(), mask, 1.0, 0.1, 0.2, 0.2),
        [logits],
        dtype=torch.float64)
    dev = gpu()
    lg = logits.to(dev).requires_grad_(True)
    loss, _, _ = hilda_grpo_loss(lg, ids.to(dev), adv.to(dev), old.to(dev), ref.to(dev), mask.to(dev), 1.0, 0.1,
                                 0.2, 0.2)
    loss.backward()
    lt = dict(rtol=1e-5, atol=1e-5) if dtype == torch.float32 else dict(rtol=1.6e-2, atol=1e-2)
    assert_close(loss, outs[0], name="loss", **lt)
    d_ref = torch.cat([oracle.exact_target_grad(d_ref[:, :L], ids), d_ref[:, L:]], dim=1)
    _strict_tail(lg.grad, d_ref, dtype, B * L, "dlogits tail")
    assert torch.count_nonzero(lg.grad[:, -1]).item() == 0


def test_grpo_on_policy_closed_form_and_module():
    """old = logp, beta = 0: loss = -mean(A) and dlogits = -A_b/(len_b*B) * (onehot - p)."""
    B, L, V = 3, 10, 2048
    logits, ids, adv, _, _, mask = _grpo_case(B, L, V, torch.float32, 3, "int32", 0.0, False)
    dev = gpu()
    lg = logits.to(dev).requires_grad_(True)
    loss, kl, clip = GRPOLoss()(lg, ids.to(dev), adv.to(dev), completion_mask=mask.to(dev))
    assert math.isclose(loss.item(), -adv.mean().item(), rel_tol=1e-5, abs_tol=1e-6)
    assert kl is None and clip.item() == 0.0
    (2.0 * loss).backward()
    p = torch.softmax(logits[:, :-1].double(), -1)
    onehot = torch.nn.functional.one_hot(ids, V).double()
    lens = mask.sum(-1).double()
    exp = -2.0 * (adv.double() / (lens * B))[:, None, None] * (onehot - p) * mask[..., None]
    assert_close(lg.grad[:, :-1], exp, name="closed form", rtol=1e-5, atol=1e-6)


def test_grpo_no_grad_forward_matches():
    B, L, V = 2, 8, 3000
    logits, ids, adv, old, ref, mask = _grpo_case(B, L, V, torch.bfloat16, 11)
    dev = gpu()
    args = (ids.to(dev), adv.to(dev), old.to(dev), ref.to(dev), mask.to(dev), 1.0, 0.1)
    a = hilda_grpo_loss(logits.to(dev), *args)
    b = hilda_grpo_loss(logits.to(dev).requires_grad_(True), *args)
    for x, y in zip(a, b):
        assert torch.equal(x, y.detach())


def test_grpo_c4_config():
    """C4: logits [16, 1024, 151936] bf16 (L = 1023), beta 0.1, eps 0.2, prefix masks of
    length [256, 1023], generated on the GPU. The loss, kl_mean and clip_ratio are
    checked against the oracle run sequence by sequence in fp64; two sequences'
    gradients element-wise; zero rows everywhere they must be."""
    dev = gpu()
    c = workloads.c4_grpo(lambda lg, ids: fused_selective_log_softmax(lg, torch.cat(
        [torch.zeros_like(ids[:, :1]), ids], 1)), device=dev)
    logits, ids, adv, old, ref, mask = (c[k] for k in ("logits", "completion_ids", "advantages", "old_logp",
                                                       "ref_logp", "completion_mask"))
    B, L = ids.shape
    lg = logits.requires_grad_(True)
    loss, kl, clip = hilda_grpo_loss(lg, ids, adv, old, ref, mask, 1.0, 0.1, 0.2, 0.2)
    loss.backward()
    grad = lg.grad
    assert torch.count_nonzero(grad[:, -1]).item() == 0
    assert torch.count_nonzero(grad[:, :-1][mask == 0]).item() == 0
    per_seq, kl_sum, clip_sum, msum = [], 0.0, 0.0, 0.0
    d_refs = {}
    for b in range(B):
        dt = torch.float64 if b < 2 else torch.float32  # fp64 where gradients are compared
        lb = logits[b:b + 1].detach().cpu().to(dt).requires_grad_(b < 2)
        args = (ids[b:b + 1].cpu(), adv[b:b + 1].cpu().to(dt), old[b:b + 1].cpu().to(dt),
                ref[b:b + 1].cpu().to(dt), mask[b:b + 1].cpu(), 1.0, 0.1, 0.2, 0.2)
        lo, kb, cb = oracle.grpo_loss_ref(lb, *args)
        m = float(mask[b].sum())
        per_seq.append(lo.item())
        kl_sum += kb.item() * m
        clip_sum += cb.item() * m
        msum += m
        if b < 2:
            lo.backward()
            d_refs[b] = lb.grad / B  # the oracle saw batch size 1
    assert math.isclose(loss.item(), sum(per_seq) / B, rel_tol=2e-3, abs_tol=2e-3)
    assert math.isclose(kl.item(), kl_sum / msum, rel_tol=2e-3, abs_tol=2e-3)
    assert abs(clip.item() - clip_sum / msum) < 2e-3
    for b, d in d_refs.items():
        s = B * float(mask[b].sum())
        assert_close(grad[b].float() * s, d[0] * s, name=f"seq {b} grad", **tol(torch.bfloat16))
        assert rel_fro(grad[b], d[0]) < 1e-2


# hk_scale_rows (the backward's upstream-gradient multiply): 16-byte vectors and
# the per-element form, padded row strides, scalar and per-row factors, a
# previous factor with zeros (rows that must come out 0), in place and out of
# place, and a shape that takes several grid-stride passes. Expected: the fp32
# product rounded to the dtype, bitwise.
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("rows,cols,pad_in,pad_out,per_row,with_prev", [
    (37, 1000, 0, 0, False, False),
    (37, 1000, 8, 24, True, True),
    (19, 1001, 3, 0, True, False),
    (5, 7, 0, 5, False, True),
    (4096, 4096, 0, 0, True, True),
])
def test_scale_rows(dtype, rows, cols, pad_in, pad_out, per_row, with_prev):
    dev = gpu()
    g = torch.Generator().manual_seed(rows * 131 + cols)
    src_full = torch.randn(rows, cols + pad_in, generator=g).to(dtype)
    dl = (torch.rand(rows, generator=g) + 0.5) if per_row else torch.tensor(1.75)
    prev = None
    if with_prev:
        prev = (torch.rand(rows, generator=g) + 0.25) if per_row else torch.tensor(0.625)
        if per_row:
            prev[::3] = 0.0
    src = src_full.to(dev)[:, :cols]
    out = torch.full((rows, cols + pad_out), 7.0, dtype=dtype, device=dev)
    ce_mod.scale_rows_(out[:, :cols], src, dl.to(dev), None if prev is None else prev.to(dev))
    f = dl.float().reshape(-1, 1) if per_row else dl.float().reshape(1, 1)
    if prev is not None:
        p = prev.float().reshape(f.shape)
        f = torch.where(p != 0, f / torch.where(p != 0, p, torch.ones_like(p)), torch.zeros_like(p))
    want = (src_full[:, :cols].float() * f).to(dtype)
    got = out.cpu()
    assert torch.equal(got[:, :cols], want)
    assert torch.all(got[:, cols:] == 7.0)  # the padding of the output rows is not written
    # in place with a unit scalar: skipped on the device, data untouched
    same = src.clone()
    ce_mod.scale_rows_(same, same, torch.tensor(1.0, device=dev), None, skip_if_one=True)
    assert torch.equal(same, src)
