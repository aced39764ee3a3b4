"""CPU tier: pin every oracle function against something other than its own formula.

Each check is chosen so that a plausible slip in the oracle (a dropped term,
a sign, a transposed operand, a wrong reduction) fails: library routines
(F.rms_norm, F.cross_entropy, torch.sigmoid), an independent complex-number
form of RoPE, closed forms of special cases, and brute-force Python loops on
tiny inputs. The reference ships no golden vectors for this path; its
known-answer checks (benchmarks/bench_rope.py:133-146,
tests/test_rms_norm.py:67-78, benchmarks/bench_cross_entropy.py:114-120)
are reproduced here.
"""
import math

import pytest
import torch
import torch.nn.functional as F

import oracle
import workloads as configs

torch.set_default_dtype(torch.float32)


def _g(seed):
    return torch.Generator().manual_seed(seed)


# ---------------------------------------------------------------- RMSNorm
def test_rms_norm_matches_library():
    x = torch.randn(6, 37, generator=_g(0), dtype=torch.float64)
    w = torch.randn(37, generator=_g(1), dtype=torch.float64)
    assert torch.allclose(oracle.rms_norm_ref(x, w, 1e-6), F.rms_norm(x, (37,), w, 1e-6), rtol=1e-12, atol=1e-12)
    xf, wf = x.float(), w.float()
    assert torch.allclose(oracle.rms_norm_ref(xf, wf, 1e-6), F.rms_norm(xf, (37,), wf, 1e-6), rtol=1e-6, atol=1e-6)
    xb = x.to(torch.bfloat16)
    assert oracle.rms_norm_ref(xb, wf).dtype == torch.bfloat16


def test_rms_norm_zeros_and_scale_invariance():
    x = torch.zeros(2, 64, 1024, dtype=torch.float16)
    assert oracle.rms_norm_ref(x, torch.ones(1024, dtype=torch.float16)).abs().max() == 0
    y = torch.randn(4, 256, generator=_g(2), dtype=torch.float64)
    w = torch.randn(256, generator=_g(3), dtype=torch.float64)
    a = oracle.rms_norm_ref(y, w, eps=0.0)
    b = oracle.rms_norm_ref(7.5 * y, w, eps=0.0)
    assert torch.allclose(a, b, rtol=1e-12, atol=1e-12)


def test_rms_norm_closed_form_backward_matches_autograd():
    """The kernels' closed-form dx/dw (kernels/rms_norm.py:186-193) equals fp64 autograd."""
    x = torch.randn(5, 48, generator=_g(4), dtype=torch.float64, requires_grad=True)
    w = torch.randn(48, generator=_g(5), dtype=torch.float64, requires_grad=True)
    dy = torch.randn(5, 48, generator=_g(6), dtype=torch.float64)
    oracle.rms_norm_ref(x, w, 1e-6).backward(dy)
    dx, dw = oracle.rms_norm_bwd_closed_form(dy, x.detach(), w.detach(), 1e-6)
    assert torch.allclose(dx, x.grad, rtol=1e-10, atol=1e-12)
    assert torch.allclose(dw, w.grad, rtol=1e-10, atol=1e-12)
    assert torch.autograd.gradcheck(lambda a, b: oracle.rms_norm_ref(a, b, 1e-6), (x, w))


def test_fused_add_rms_norm_ref():
    x = torch.randn(8, 64, generator=_g(7)).to(torch.bfloat16)
    r = torch.randn(8, 64, generator=_g(8)).to(torch.bfloat16)
    w = (1 + 0.02 * torch.randn(64, generator=_g(9))).to(torch.bfloat16)
    y, s = oracle.fused_add_rms_norm_ref(x, r, w)
    # S is the bf16 rounding of the exact fp32 sum
    assert torch.equal(s, (x.float() + r.float()).to(torch.bfloat16))
    normed = F.rms_norm(s.float(), (64,), None, 1e-6).to(torch.bfloat16)
    assert torch.equal(y, normed * w)


# ---------------------------------------------------------------- RoPE
def _rope_complex(x, cos, sin):
    """Independent form: pair (x_i, x_{i+D/2}) as a complex number times e^{i theta}."""
    d = x.shape[-1] // 2
    z = torch.complex(x[..., :d].double(), x[..., d:].double())
    rot = torch.complex(cos.double(), sin.double()).unsqueeze(1)
    out = z * rot
    return torch.cat([out.real, out.imag], dim=-1)


def test_rope_matches_complex_rotation():
    q = torch.randn(2, 3, 16, 32, generator=_g(10), dtype=torch.float64)
    k = torch.randn(2, 1, 16, 32, generator=_g(11), dtype=torch.float64)
    cos, sin = oracle.rope_tables(32, 16, 500000.0, dtype=torch.float64)
    qe, ke = oracle.rope_ref(q, k, cos, sin)
    assert torch.allclose(qe, _rope_complex(q, cos, sin), atol=1e-12)
    assert torch.allclose(ke, _rope_complex(k, cos, sin), atol=1e-12)


def test_rope_tables_and_invariants():
    cos, sin = oracle.rope_tables(128, 2048, 500000.0)
    assert cos.shape == (1, 2048, 64)
    # position 0 is the identity; cos^2 + sin^2 = 1
    assert torch.all(cos[0, 0] == 1) and torch.all(sin[0, 0] == 0)
    assert torch.allclose(cos ** 2 + sin ** 2, torch.ones_like(cos), atol=1e-6)
    # inv_freq = base^(-2i/d): the last pair rotates slowest
    t = 1000
    assert math.isclose(math.atan2(sin[0, t, 1].item(), cos[0, t, 1].item()),
                        math.remainder(t * 500000.0 ** (-2 / 128), 2 * math.pi), abs_tol=1e-4)
    # rotation preserves each pair's norm
    x = torch.randn(1, 2, 2048, 128, generator=_g(12))
    y, _ = oracle.rope_ref(x, x, cos, sin)
    n0 = x[..., :64] ** 2 + x[..., 64:] ** 2
    n1 = y[..., :64] ** 2 + y[..., 64:] ** 2
    assert torch.allclose(n0, n1, rtol=1e-4, atol=1e-4)


def test_rope_backward_known_answer():
    """benchmarks/bench_rope.py:133-146: all-ones grad -> [cos+sin, cos-sin]."""
    g = _g(13)
    cos = torch.randn(1, 8, 16, generator=g, dtype=torch.float64)
    sin = torch.randn(1, 8, 16, generator=g, dtype=torch.float64)
    q = torch.randn(2, 3, 8, 32, generator=g, dtype=torch.float64, requires_grad=True)
    k = torch.randn(2, 1, 8, 32, generator=g, dtype=torch.float64, requires_grad=True)
    qo, ko = oracle.rope_ref(q, k, cos, sin)
    (qo.sum() + ko.sum()).backward()
    exp = torch.cat([cos + sin, cos - sin], dim=-1).unsqueeze(1)
    assert torch.allclose(q.grad, exp.expand_as(q), atol=1e-12)
    assert torch.allclose(k.grad, exp.expand_as(k), atol=1e-12)


# ---------------------------------------------------------------- SwiGLU
def test_swiglu_ref():
    a = torch.randn(5, 33, generator=_g(14), dtype=torch.float64, requires_grad=True)
    b = torch.randn(5, 33, generator=_g(15), dtype=torch.float64, requires_grad=True)
    c = oracle.swiglu_ref(a, b)
    assert torch.allclose(c, a * torch.sigmoid(a) * b, atol=1e-14)
    z = torch.zeros(4, 8, dtype=torch.float64, requires_grad=True)
    bb = torch.randn(4, 8, generator=_g(16), dtype=torch.float64)
    dc = torch.randn(4, 8, generator=_g(17), dtype=torch.float64)
    oracle.swiglu_ref(z, bb).backward(dc)
    assert torch.allclose(z.grad, 0.5 * dc * bb, atol=1e-14)


# ---------------------------------------------------------------- GeGLU
def test_geglu_ref():
    x = torch.linspace(-12, 12, 2001, dtype=torch.float64)
    one = torch.ones_like(x)
    g = oracle.geglu_ref(x, one)
    gm = oracle.geglu_ref(-x, one)
    # tanh is odd: 0.5x(1+t) + 0.5x(1-t) = x, exactly, for any correct tanh form
    assert torch.allclose(g - gm, x, atol=1e-13)
    # the tanh form stays within 1e-3 of the exact GELU x * Phi(x); without the cubic
    # term or with a wrong sqrt(2/pi) factor the gap exceeds 1e-2 near |x| = 2
    exact = x * 0.5 * (1 + torch.erf(x / math.sqrt(2.0)))
    assert (g - exact).abs().max() < 1e-3
    assert torch.allclose(g[x > 8], x[x > 8], atol=1e-12) and g[x < -8].abs().max() < 1e-12
    z = torch.zeros(3, dtype=torch.float64, requires_grad=True)
    bb = torch.tensor([1.0, -2.0, 0.5], dtype=torch.float64)
    c = oracle.geglu_ref(z, bb)
    assert torch.equal(c, torch.zeros_like(c))
    c.backward(torch.ones_like(c))
    assert torch.allclose(z.grad, 0.5 * bb, atol=1e-15)  # gelu'(0) = 1/2
    a = torch.randn(4, 9, generator=_g(40), dtype=torch.float64, requires_grad=True)
    b = torch.randn(4, 9, generator=_g(41), dtype=torch.float64, requires_grad=True)
    assert torch.autograd.gradcheck(oracle.geglu_ref, (a, b))


# ---------------------------------------------------------------- KL divergence / JSD
def _logprobs(shape, seed):
    return torch.log_softmax(torch.randn(*shape, generator=_g(seed), dtype=torch.float64), -1)


@pytest.mark.filterwarnings("ignore:reduction. 'mean' divides")
@pytest.mark.parametrize("log_target", [False, True])
def test_kl_div_ref(log_target):
    yp = _logprobs((6, 40), 50)
    lt = _logprobs((6, 40), 51)
    yt = lt if log_target else lt.exp()
    for red in ("sum", "mean", "batchmean"):
        exp = F.kl_div(yp, yt, reduction=red, log_target=log_target)
        assert torch.allclose(oracle.kl_div_ref(yp, yt, red, log_target), exp, atol=1e-13), red
    per = F.kl_div(yp, yt, reduction="none", log_target=log_target).sum(-1)
    assert torch.allclose(oracle.kl_div_ref(yp, yt, "none", log_target), per, atol=1e-13)
    assert (per >= 0).all()  # Gibbs' inequality
    same = oracle.kl_div_ref(lt, yt, "none", log_target)
    assert same.abs().max() < 1e-13


def _jsd_brute(X, Y, beta, labels, ignore_index):
    tot, n = 0.0, 0
    for r in range(X.shape[0]):
        if labels is not None and int(labels[r]) == ignore_index:
            continue
        n += 1
        for c in range(X.shape[1]):
            q, p = math.exp(float(X[r, c].detach())), math.exp(float(Y[r, c].detach()))
            if beta == 0:  # the reference's end points are the two plain KLs (jsd.py:67-75)
                tot += p * math.log(p / q)
            elif beta == 1:
                tot += q * math.log(q / p)
            else:
                m = beta * p + (1 - beta) * q
                tot += beta * p * math.log(p / m) + (1 - beta) * q * math.log(q / m)
    return tot / max(n, 1)


def test_jsd_ref():
    X = _logprobs((5, 12), 60).requires_grad_(True)
    Y = _logprobs((5, 12), 61)
    # beta = 0: KL(P||Q); beta = 1: KL(Q||P) (the library's kl_div, batchmean)
    assert torch.allclose(oracle.jsd_ref(X, Y, 0.0), F.kl_div(X, Y, reduction="batchmean", log_target=True),
                          atol=1e-13)
    assert torch.allclose(oracle.jsd_ref(X, Y, 1.0), F.kl_div(Y, X, reduction="batchmean", log_target=True),
                          atol=1e-13)
    j = oracle.jsd_ref(X, Y, 0.5)
    assert torch.allclose(j, oracle.jsd_ref(Y, X, 0.5), atol=1e-13)  # symmetric at beta = 1/2
    assert 0 <= float(j.detach()) <= math.log(2)
    assert float(oracle.jsd_ref(X, X, 0.3).detach()) < 1e-13
    labels = torch.tensor([3, -100, 1, -100, 0])
    for beta in (0.0, 0.25, 0.5, 1.0):
        got = float(oracle.jsd_ref(X, Y, beta, labels).detach())
        assert abs(got - _jsd_brute(X, Y, beta, labels, -100)) < 1e-12, beta
    assert float(oracle.jsd_ref(X, Y, 0.5, torch.full((5,), -100)).detach()) == 0.0
    assert torch.autograd.gradcheck(lambda x: oracle.jsd_ref(x, Y, 0.3, labels), (X,))


def test_fused_linear_jsd_ref():
    g = _g(70)
    BT, H, Ht, V, T = 5, 6, 4, 9, 1.7
    si = torch.randn(BT, H, generator=g, dtype=torch.float64, requires_grad=True)
    sw = torch.randn(V, H, generator=g, dtype=torch.float64, requires_grad=True)
    ti = torch.randn(BT, Ht, generator=g, dtype=torch.float64)
    tw = torch.randn(V, Ht, generator=g, dtype=torch.float64)
    labels = torch.tensor([1, -100, 3, 0, -100])

    def logprobs(inp, w):  # explicit dot products and log-sum-exp
        out = torch.empty(inp.shape[0], w.shape[0], dtype=torch.float64)
        for r in range(inp.shape[0]):
            z = [sum(float(inp[r, k]) * float(w[v, k]) for k in range(inp.shape[1])) / T for v in range(w.shape[0])]
            m = max(z)
            lse = m + math.log(sum(math.exp(zz - m) for zz in z))
            for v in range(w.shape[0]):
                out[r, v] = z[v] - lse
        return out

    X, Y = logprobs(si.detach(), sw.detach()), logprobs(ti, tw)
    for beta in (0.0, 0.4, 1.0):
        got = float(oracle.fused_linear_jsd_ref(si, sw, ti, tw, labels, beta, T).detach())
        assert abs(got - _jsd_brute(X, Y, beta, labels, -100)) < 1e-12, beta
    assert torch.autograd.gradcheck(lambda a, b: oracle.fused_linear_jsd_ref(a, b, ti, tw, labels, 0.4, T), (si, sw))


# ---------------------------------------------------------------- AttnRes
def test_attn_res_ref():
    g = _g(80)
    N, T, D, eps = 3, 4, 6, 1e-6
    V = torch.randn(N, T, D, generator=g, dtype=torch.float64, requires_grad=True)
    wq = torch.randn(D, generator=g, dtype=torch.float64, requires_grad=True)
    wn = (1 + 0.1 * torch.randn(D, generator=g, dtype=torch.float64)).requires_grad_(True)
    h = oracle.attn_res_ref(V, wq, wn, eps).detach()
    Vd, wqd, wnd = V.detach(), wq.detach(), wn.detach()
    for t in range(T):  # brute force: RMSNorm keys, dot, softmax over blocks, weighted sum
        sc = []
        for i in range(N):
            v = [float(Vd[i, t, d]) for d in range(D)]
            r = 1.0 / math.sqrt(sum(x * x for x in v) / D + eps)
            sc.append(sum(float(wqd[d]) * v[d] * r * float(wnd[d]) for d in range(D)))
        m = max(sc)
        e = [math.exp(x - m) for x in sc]
        a = [x / sum(e) for x in e]
        for d in range(D):
            assert abs(float(h[t, d]) - sum(a[i] * float(Vd[i, t, d]) for i in range(N))) < 1e-12
    one = V[:1].detach()
    assert torch.allclose(oracle.attn_res_ref(one, wq.detach(), wn.detach()), one[0], atol=1e-15)
    same = V[:1].detach().expand(4, T, D)
    assert torch.allclose(oracle.attn_res_ref(same, wq.detach(), wn.detach()), same[0], atol=1e-14)
    # a query aligned with block 1's normalised key (and large) puts all the weight on it
    k1 = V[1, 0].detach() / V[1, 0].detach().pow(2).mean().sqrt()
    big = oracle.attn_res_ref(V.detach()[:, :1], 1e3 * k1 / wn.detach(), wn.detach())
    assert torch.allclose(big[0], V[1, 0].detach(), atol=1e-9)
    assert torch.autograd.gradcheck(lambda a, b, c: oracle.attn_res_ref(a, b, c, eps), (V, wq, wn))


# ---------------------------------------------------------------- CrossEntropy
def _ce_brute(logits, targets, ignore_index, reduction):
    losses, n_valid = [], 0
    for r in range(logits.shape[0]):
        t = int(targets[r])
        if t == ignore_index:
            losses.append(0.0)
            continue
        n_valid += 1
        row = [float(v) for v in logits[r]]
        m = max(row)
        lse = m + math.log(sum(math.exp(v - m) for v in row))
        losses.append(lse - row[t])
    if reduction == "none":
        return torch.tensor(losses, dtype=torch.float64)
    total = sum(losses)
    return torch.tensor(total / max(n_valid, 1) if reduction == "mean" else total, dtype=torch.float64)


@pytest.mark.parametrize("reduction", ["mean", "sum", "none"])
def test_cross_entropy_ref_brute_force(reduction):
    logits = 3 * torch.randn(9, 13, generator=_g(18), dtype=torch.float64)
    t = torch.randint(0, 13, (9,), generator=_g(19))
    t[[1, 4]] = -100
    got = oracle.cross_entropy_ref(logits, t, -100, reduction)
    assert torch.allclose(got, _ce_brute(logits, t, -100, reduction), atol=1e-12)


def test_cross_entropy_ref_special_cases():
    V = 1000
    u = torch.zeros(4, V, dtype=torch.float64)
    t = torch.tensor([0, 5, 999, 17])
    assert math.isclose(oracle.cross_entropy_ref(u, t).item(), math.log(V), rel_tol=1e-12)
    x = torch.randn(4, V, generator=_g(20), dtype=torch.float64)
    assert math.isclose(oracle.cross_entropy_ref(x + 123.0, t).item(), oracle.cross_entropy_ref(x, t).item(),
                        rel_tol=1e-10)
    # every row ignored: the reference returns 0 (not NaN) under mean
    assert oracle.cross_entropy_ref(x, torch.full((4,), -100)).item() == 0.0
    # ignore_index = -1 is the "ignore nothing" sentinel
    assert torch.allclose(oracle.cross_entropy_ref(x, t, -1), F.cross_entropy(x, t))
    # ignored rows get exactly zero gradient
    xr = x.clone().requires_grad_(True)
    tt = t.clone()
    tt[2] = -100
    oracle.cross_entropy_ref(xr, tt).backward()
    assert torch.count_nonzero(xr.grad[2]) == 0
    # closed-form gradient (softmax - onehot) / n_valid
    p = torch.softmax(x, -1)
    onehot = F.one_hot(tt.clamp(min=0), V).double()
    exp = (p - onehot) / 3
    exp[2] = 0
    assert torch.allclose(xr.grad, exp, atol=1e-14)


def test_exact_target_grad():
    # ordinary rows: the same as fp64 autograd (and ignored rows untouched)
    x = (3 * torch.randn(6, 50, generator=_g(60), dtype=torch.float64)).requires_grad_(True)
    t = torch.randint(0, 50, (6,), generator=_g(61))
    t[2] = -100
    oracle.cross_entropy_ref(x, t, -100, "sum").backward()
    fixed = oracle.exact_target_grad(x.grad, t)
    assert torch.allclose(fixed, x.grad, rtol=1e-12, atol=1e-15)
    assert torch.equal(fixed[2], x.grad[2])
    # a peaked row [0, -a, -b] with target 0: autograd's p_0 - 1 is exactly 0 in fp64,
    # the closed form -(e^-a + e^-b) / (1 + e^-a + e^-b) is not
    a, b = 45.0, 52.0
    z = torch.tensor([[0.0, -a, -b]], dtype=torch.float64, requires_grad=True)
    tz = torch.tensor([0])
    oracle.cross_entropy_ref(z, tz, -100, "sum").backward()
    assert z.grad[0, 0].item() == 0.0
    ea, eb = math.exp(-a), math.exp(-b)
    want = -(ea + eb) / (1.0 + ea + eb)
    got = oracle.exact_target_grad(z.grad, tz)[0, 0].item()
    assert math.isclose(got, want, rel_tol=1e-12)
    # leading batch dimensions (GRPO's (B, L, V)), and a row scale g carried through
    d = torch.tensor([[[0.5 * ea, 0.5 * eb, 0.0]]], dtype=torch.float64)
    assert math.isclose(oracle.exact_target_grad(d, torch.tensor([[2]]))[0, 0, 2].item(), -0.5 * (ea + eb),
                        rel_tol=1e-12)


# ---------------------------------------------------------------- GRPO
def test_selective_log_softmax_brute_force():
    B, L, V = 2, 3, 7
    logits = torch.randn(B, L + 1, V, generator=_g(21), dtype=torch.float64)
    ids = torch.randint(0, V, (B, L + 1), generator=_g(22))
    mask = torch.ones(B, L + 1, dtype=torch.int32)
    mask[1, -1] = 0
    T = 0.7
    got = oracle.selective_log_softmax_ref(logits, ids, temperature=T, mask=mask)
    for b in range(B):
        for l in range(L):
            idx = int(ids[b, 1 + l])
            row = [float(v) / T for v in logits[b, l]]
            m = max(row)
            exp = row[idx] - (m + math.log(sum(math.exp(v - m) for v in row)))
            if l == L - 1 and b == 1:
                exp = 0.0
            assert math.isclose(got[b, l].item(), exp, rel_tol=1e-6, abs_tol=1e-9)


def test_grpo_closed_form_on_policy():
    """old = logp, beta = 0: loss = -mean(A); dlogits = -A_b/(len_b*B) * (onehot - p)."""
    B, L, V = 3, 5, 11
    logits = torch.randn(B, L + 1, V, generator=_g(23), dtype=torch.float64, requires_grad=True)
    ids = torch.randint(0, V, (B, L), generator=_g(24))
    adv = torch.randn(B, generator=_g(25), dtype=torch.float64)
    mask = torch.ones(B, L, dtype=torch.int32)
    mask[0, 3:] = 0
    mask[2, 1:] = 0
    loss, kl, clip = oracle.grpo_loss_ref(logits, ids, adv, completion_mask=mask)
    assert math.isclose(loss.item(), -adv.mean().item(), rel_tol=1e-12, abs_tol=1e-12)
    assert kl is None and clip.item() == 0.0
    loss.backward()
    p = torch.softmax(logits.detach()[:, :-1], -1)
    onehot = F.one_hot(ids, V).double()
    lens = mask.sum(-1).double()
    exp = -(adv / (lens * B))[:, None, None] * (onehot - p) * mask[..., None]
    assert torch.allclose(logits.grad[:, :-1], exp, atol=1e-14)
    assert torch.count_nonzero(logits.grad[:, -1]) == 0


def test_grpo_kl_zero_at_reference_and_brute_force():
    B, L, V = 2, 4, 6
    g = _g(26)
    logits = torch.randn(B, L + 1, V, generator=g, dtype=torch.float64)
    ids = torch.randint(0, V, (B, L), generator=g)
    adv = torch.tensor([0.7, -1.3], dtype=torch.float64)
    logp = oracle.selective_log_softmax_ref(logits, ids).double()
    _, kl0, _ = oracle.grpo_loss_ref(logits, ids, adv, ref_logp=logp, beta=0.1)
    assert abs(kl0.item()) < 1e-14
    old = logp + 0.4 * torch.randn(B, L, generator=g, dtype=torch.float64)
    ref = logp + 0.3 * torch.randn(B, L, generator=g, dtype=torch.float64)
    mask = torch.tensor([[1, 1, 1, 0], [1, 1, 1, 1]], dtype=torch.int32)
    beta, el, eh = 0.1, 0.2, 0.25
    loss, kl, clip = oracle.grpo_loss_ref(logits, ids, adv, old, ref, mask, 1.0, beta, el, eh)
    per_seq, kls, clips, n = [], 0.0, 0, 0
    for b in range(B):
        s, cnt = 0.0, 0
        for l in range(L):
            if not mask[b, l]:
                continue
            lp = float(logp[b, l])
            ratio = math.exp(lp - float(old[b, l]))
            rc = min(max(ratio, 1 - el), 1 + eh)
            a = float(adv[b])
            k = math.exp(float(ref[b, l]) - lp) - (float(ref[b, l]) - lp) - 1
            s += -min(ratio * a, rc * a) + beta * k
            kls += k
            clips += int((ratio < 1 - el and a < 0) or (ratio > 1 + eh and a > 0))
            cnt += 1
            n += 1
        per_seq.append(s / max(cnt, 1))
    assert math.isclose(loss.item(), sum(per_seq) / B, rel_tol=1e-10)
    assert math.isclose(kl.item(), kls / n, rel_tol=1e-10)
    assert math.isclose(clip.item(), clips / n, rel_tol=1e-6)


# ---------------------------------------------------------------- FLCE
def test_linear_ce_brute_force():
    N, H, V = 5, 4, 6
    g = _g(27)
    h = torch.randn(N, H, generator=g, dtype=torch.float64)
    w = torch.randn(V, H, generator=g, dtype=torch.float64)
    t = torch.tensor([1, -100, 5, 0, 3])
    logits = torch.tensor([[sum(float(h[n, c]) * float(w[v, c]) for c in range(H)) for v in range(V)]
                           for n in range(N)], dtype=torch.float64)
    exp = _ce_brute(logits, t, -100, "mean")
    assert torch.allclose(oracle.linear_ce_ref(h, w, t), exp, atol=1e-12)
    assert oracle.linear_ce_ref(h, w, torch.full((N,), -100)).item() == 0.0


def test_fused_linear_grpo_brute_force_and_closed_form():
    B, L, H, V = 2, 3, 4, 7
    g = _g(41)
    h = torch.randn(B, L + 1, H, generator=g, dtype=torch.float64)
    w = torch.randn(V, H, generator=g, dtype=torch.float64)
    ids = torch.randint(0, V, (B, L), generator=g)
    adv = torch.tensor([0.9, -0.6], dtype=torch.float64)
    # logits by explicit dot products, then the (separately pinned) GRPO loss
    logits = torch.tensor([[[sum(float(h[b, t, c]) * float(w[v, c]) for c in range(H)) for v in range(V)]
                            for t in range(L + 1)] for b in range(B)], dtype=torch.float64)
    logp = oracle.selective_log_softmax_ref(logits, ids).double()
    old = logp + 0.3 * torch.randn(B, L, generator=g, dtype=torch.float64)
    ref = logp + 0.2 * torch.randn(B, L, generator=g, dtype=torch.float64)
    mask = torch.tensor([[1, 1, 0], [1, 1, 1]], dtype=torch.int32)
    args = (ids, adv, old, ref, mask, 0.8, 0.1, 0.2, 0.25)
    for x, y in zip(oracle.fused_linear_grpo_ref(h, w, *args), oracle.grpo_loss_ref(logits, *args)):
        assert math.isclose(x.item(), y.item(), rel_tol=1e-12, abs_tol=1e-14)
    # on-policy, beta = 0, temperature T: loss = -mean(A) and
    # dlogits = -A_b/(len_b*B) * (onehot - softmax(logits/T)) / T, carried through the lm_head by loops
    T = 0.8
    hg = h.clone().requires_grad_(True)
    wg = w.clone().requires_grad_(True)
    loss, kl, clip = oracle.fused_linear_grpo_ref(hg, wg, ids, adv, completion_mask=mask, temperature=T)
    assert math.isclose(loss.item(), -adv.mean().item(), rel_tol=1e-12, abs_tol=1e-12)
    loss.backward()
    lens = mask.sum(-1).double()
    dl = torch.zeros(B, L + 1, V, dtype=torch.float64)
    for b in range(B):
        for t in range(L):
            if not mask[b, t]:
                continue
            z = [float(logits[b, t, v]) / T for v in range(V)]
            mx = max(z)
            e = [math.exp(q - mx) for q in z]
            for v in range(V):
                dl[b, t, v] = -float(adv[b]) / (float(lens[b]) * B) * (float(v == int(ids[b, t])) - e[v] / sum(e)) / T
    dh = torch.tensor([[[sum(float(dl[b, t, v]) * float(w[v, c]) for v in range(V)) for c in range(H)]
                        for t in range(L + 1)] for b in range(B)], dtype=torch.float64)
    dw = torch.tensor([[sum(float(dl[b, t, v]) * float(h[b, t, c]) for b in range(B) for t in range(L + 1))
                        for c in range(H)] for v in range(V)], dtype=torch.float64)
    assert torch.allclose(hg.grad, dh, atol=1e-14) and torch.allclose(wg.grad, dw, atol=1e-14)
    assert torch.count_nonzero(hg.grad[:, -1]) == 0 and torch.count_nonzero(hg.grad[0, 2]) == 0


# ---------------------------------------------------------------- generators
def test_config_generators_small():
    c = configs.c3_cross_entropy(rows=4000, vocab=50)
    frac = (c["targets"] == -100).float().mean().item()
    assert 0.07 < frac < 0.13 and c["logits"].dtype == torch.bfloat16
    c4 = configs.c4_grpo(oracle.selective_log_softmax_ref, B=4, T=300, vocab=40)
    lens = c4["completion_mask"].sum(-1)
    assert c4["logits"].shape == (4, 300, 40) and c4["completion_ids"].shape == (4, 299)
    assert torch.all(lens >= 256) and torch.all(lens <= 299)
    c5 = configs.c5_fused_linear_ce(bt=64, hidden=16, vocab=32)
    assert c5["weight"].shape == (32, 16)
    a = configs.c1_rms_norm(rows=4, hidden=8)
    b = configs.c1_rms_norm(rows=4, hidden=8)
    assert torch.equal(a["x"], b["x"]) and torch.equal(a["dy"], b["dy"])
    r = configs.c2_rope(B=1, T=8, Hq=2, Hk=1, D=16)
    assert r["q"].shape == (1, 2, 8, 16) and r["q"].stride() == (256, 16, 32, 1)
