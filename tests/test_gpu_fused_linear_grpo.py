"""GPU parity: FusedLinear-GRPO (lm_head MFMA GEMMs + the GRPO row kernel, chunked) vs the CPU oracle.

The oracle is the reference's GRPO loss (benchmarks/bench_grpo.py:30-57) on the
lm_head logits hidden @ W.T, with the logits rounded to the compute dtype as the
GEMM returns them, in fp64. Cases: several chunks with a ragged last chunk
(chunk rows not a multiple of L+1, so chunks start mid-sequence), every mask
dtype, on/off-policy, beta 0 and > 0, temperature != 1, asymmetric clip, the
upstream gradient, no-grad forward equal to the grad forward, and agreement with
hilda_grpo_loss on materialised logits. Zero rows of dhidden at masked tokens and
at position L are checked exactly.
"""
import math

import pytest
import torch

import oracle
from _util import assert_close, rel_fro, tol, gpu

from kernels import hilda_fused_linear_grpo_loss, FusedLinearGRPOLoss, hilda_grpo_loss
from kernels import fused_linear_grpo as flg

pytestmark = pytest.mark.gpu


def _case(B, L, H, V, dtype, seed, mask_kind="int32", beta=0.1, with_old=True):
    g = torch.Generator().manual_seed(seed)
    h = torch.randn(B, L + 1, H, generator=g).to(dtype)
    w = (0.05 * torch.randn(V, H, generator=g)).to(dtype)
    ids = torch.randint(0, V, (B, L), generator=g)
    adv = torch.randn(B, generator=g)
    logits = (h.double() @ w.double().T).to(dtype).double()
    logp = oracle.selective_log_softmax_ref(logits, ids).float()
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
    return h, w, ids, adv, old, ref, mask


def _oracle(h, w, ids, adv, old, ref, mask, T, beta, el, eh):
    def f(a, b):
        return oracle.fused_linear_grpo_ref(a, b, ids, adv.double(), None if old is None else old.double(),
                                            None if ref is None else ref.double(), mask, T, beta, el, eh,
                                            logits_dtype=h.dtype)
    return oracle.fwd_bwd(f, [h, w], dtype=torch.float64)


def _dev(x):
    return None if x is None else x.to(gpu())


CASES = [
    # B, L, H, V, mask, beta, with_old, T, eps_lo, eps_hi, chunk
    (3, 16, 64, 512, "int32", 0.1, True, 1.0, 0.2, 0.2, 8192),
    (2, 37, 128, 1000, "bool", 0.0, True, 1.0, 0.2, 0.28, 24),
    (4, 12, 256, 4096, None, 0.1, False, 1.0, 0.2, 0.2, 16),
    (2, 21, 64, 2048, "float", 0.04, True, 0.7, 0.1, 0.3, 40),
    (3, 9, 128, 32000, "int64", 0.1, True, 1.0, 0.2, 0.2, 8),
]


@pytest.mark.parametrize("case", CASES)
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_fused_linear_grpo(case, dtype):
    B, L, H, V, mk, beta, with_old, T, el, eh, chunk = case
    h, w, ids, adv, old, ref, mask = _case(B, L, H, V, dtype, B * 100 + L + H, mk, beta, with_old)
    outs, (dh_ref, dw_ref) = _oracle(h, w, ids, adv, old, ref, mask, T, beta, el, eh)
    print(f"case B={B} L={L} H={H} V={V} {dtype} chunk={chunk}", flush=True)
    dev = gpu()
    hg = h.to(dev).requires_grad_(True)
    wg = w.to(dev).requires_grad_(True)
    args = (ids.to(dev), adv.to(dev), _dev(old), _dev(ref), _dev(mask), T, beta, el, eh)
    if chunk != 8192:
        loss, kl, clip, gh, gw, _ = flg.fused_linear_grpo_forward(hg.detach(), wg.detach(), *args, chunk=chunk)
        hg.grad, wg.grad = gh, gw
    else:
        loss, kl, clip = hilda_fused_linear_grpo_loss(hg, wg, *args)
        loss.backward()
    lt = dict(rtol=1e-5, atol=1e-5) if dtype == torch.float32 else dict(rtol=2e-3, atol=2e-3)
    assert_close(loss, outs[0], name="loss", **lt)
    if beta != 0:
        assert_close(kl, outs[1], name="kl_mean", **lt)
    else:
        assert kl is None
    # the 16-bit logits may round differently from the oracle's at a tie: allow one token's clip decision
    mf = mask.float() if mask is not None else torch.ones(B, L)
    assert abs(clip.item() - outs[2].item()) <= mf.max().item() / mf.sum().item() + 1e-6
    t = tol(dtype)
    scale = B * L  # undo the 1/(len_b * B) reduction scale
    assert_close(hg.grad.float() * scale, dh_ref * scale, name="dhidden*B*L", **t)
    assert_close(wg.grad.float() * scale, dw_ref * scale, name="dweight*B*L", **t)
    assert rel_fro(hg.grad, dh_ref) < 1e-2 and rel_fro(wg.grad, dw_ref) < 1e-2
    # masked tokens and the last position get exactly zero dhidden rows
    assert torch.count_nonzero(hg.grad[:, -1]).item() == 0
    if mask is not None:
        assert torch.count_nonzero(hg.grad[:, :-1][mask.to(dev) == 0]).item() == 0


def test_fused_linear_grpo_matches_grpo_on_logits():
    """The per-token rows and reductions equal hilda_grpo_loss on the same 16-bit logits; the gradients equal
    dlogits carried through the lm_head."""
    B, L, H, V = 2, 30, 128, 3000
    dtype = torch.bfloat16
    h, w, ids, adv, old, ref, mask = _case(B, L, H, V, dtype, 77)
    dev = gpu()
    hd, wd = h.to(dev), w.to(dev)
    args = (ids.to(dev), adv.to(dev), old.to(dev), ref.to(dev), mask.to(dev), 1.0, 0.1, 0.2, 0.2)
    loss, kl, clip, gh, gw, rows = flg.fused_linear_grpo_forward(hd, wd, *args, chunk=16)
    # the 16-bit logits from a library GEMM (2-D, contiguous operands), compared with tolerance
    logits = (hd.reshape(-1, H) @ wd.T.contiguous()).reshape(B, L + 1, V).requires_grad_(True)
    l2, k2, c2 = hilda_grpo_loss(logits, *args)
    l2.backward()
    assert_close(loss, l2, name="loss", rtol=2e-3, atol=2e-3)
    assert_close(kl, k2, name="kl", rtol=2e-3, atol=2e-3)
    dl = logits.grad.float()
    assert rel_fro(gh, dl @ wd.float()) < 1e-2
    assert rel_fro(gw, dl.reshape(-1, V).T @ hd.float().reshape(-1, H)) < 1e-2
    lse = torch.logsumexp((h.double() @ w.double().T)[:, :-1], -1)
    live = mask.bool()
    assert_close(rows[0].cpu()[live], lse[live], name="lse rows", rtol=1e-3, atol=1e-2)
    assert torch.count_nonzero(rows[1].cpu()[~live]).item() == 0


def test_fused_linear_grpo_upstream_grad_module_and_no_grad():
    B, L, H, V = 2, 14, 64, 800
    h, w, ids, adv, old, ref, mask = _case(B, L, H, V, torch.bfloat16, 5)
    outs, (dh_ref, dw_ref) = _oracle(h, w, ids, adv, old, ref, mask, 1.0, 0.1, 0.2, 0.2)
    dev = gpu()
    hg = h.to(dev).requires_grad_(True)
    wg = w.to(dev).requires_grad_(True)
    args = (ids.to(dev), adv.to(dev), old.to(dev), ref.to(dev), mask.to(dev))
    loss, kl, clip = FusedLinearGRPOLoss(beta=0.1)(hg, wg, *args)
    (2.5 * loss).backward()
    assert rel_fro(hg.grad, 2.5 * dh_ref) < 1e-2 and rel_fro(wg.grad, 2.5 * dw_ref) < 1e-2
    with torch.no_grad():
        l_ng, kl_ng, clip_ng = hilda_fused_linear_grpo_loss(hg.detach(), wg.detach(), *args, beta=0.1)
    assert torch.equal(l_ng, loss.detach()) and torch.equal(kl_ng, kl) and torch.equal(clip_ng, clip)


def test_fused_linear_grpo_on_policy_closed_form():
    """old = logp, beta = 0: loss = -mean(A) whatever the lm_head."""
    B, L, H, V = 3, 10, 128, 2048
    h, w, ids, adv, _, _, mask = _case(B, L, H, V, torch.bfloat16, 3, "int32", 0.0, False)
    dev = gpu()
    loss, kl, clip = hilda_fused_linear_grpo_loss(h.to(dev), w.to(dev), ids.to(dev), adv.to(dev),
                                                  completion_mask=mask.to(dev))
    assert math.isclose(loss.item(), -adv.mean().item(), rel_tol=1e-5, abs_tol=1e-6)
    assert kl is None and clip.item() == 0.0


def test_fused_linear_grpo_rejects():
    dev = gpu()
    h = torch.randn(2, 5, 64, device=dev, dtype=torch.bfloat16)
    w = torch.randn(100, 64, device=dev, dtype=torch.bfloat16)
    ids = torch.zeros(2, 4, dtype=torch.int64, device=dev)
    adv = torch.zeros(2, device=dev)
    with pytest.raises(TypeError):
        hilda_fused_linear_grpo_loss(h.double(), w.double(), ids, adv)
    with pytest.raises(RuntimeError, match="workspace budget"):  # below the smallest plan
        hilda_fused_linear_grpo_loss(h, w[:99], ids, adv, workspace_budget=1024)
    with pytest.raises(ValueError):
        hilda_fused_linear_grpo_loss(h, w[:96], ids, adv, beta=0.1)


def test_fused_linear_grpo_f3_config():
    """B 16, L+1 1024, H 4096, V 151936 bf16, beta 0.1, C4's prefix masks: zero rows, the reductions against
    the per-token rows, the vocabulary sum of dW, and a sample of tokens (lse, per-token loss, dhidden row)
    against the oracle on CPU."""
    import workloads
    dev = gpu()

    def logp_fn(h, w, ids):
        _, _, _, _, _, rows = flg.fused_linear_grpo_forward(h, w, ids, torch.zeros(h.shape[0], device=dev),
                                                            compute_grad=False)
        return (h[:, :-1].float() * w[ids].float()).sum(-1) - rows[0]

    c = workloads.f3_fused_linear_grpo(logp_fn, device=dev)
    h, w, ids, adv, old, ref, mask = (c[k] for k in ("hidden", "weight", "completion_ids", "advantages", "old_logp",
                                                     "ref_logp", "completion_mask"))
    B, L = ids.shape
    print(f"f3 config B={B} L={L} H={h.shape[2]} V={w.shape[0]}", flush=True)
    loss, kl, clip, gh, gw, rows = flg.fused_linear_grpo_forward(h, w, ids, adv, old, ref, mask, 1.0, 0.1, 0.2, 0.2)
    live = mask != 0
    assert torch.count_nonzero(gh[:, -1]).item() == 0
    assert torch.count_nonzero(gh[:, :-1][~live]).item() == 0
    m = mask.double()
    lens = m.sum(-1).clamp(min=1)
    assert math.isclose(loss.item(), ((rows[1].double() * m).sum(-1) / lens).mean().item(), rel_tol=1e-5)
    assert math.isclose(kl.item(), (rows[2].double() * m).sum().item() / m.sum().item(), rel_tol=1e-5)
    # each dlogits row sums to zero over the vocabulary, so does dW (relative to its L1 mass)
    g32 = gw.float()
    assert (g32.sum(0).abs() / g32.abs().sum(0)).max().item() < 1e-2
    # a sample of live tokens against the oracle
    wc = w.cpu().float()
    torch.manual_seed(0)
    bl = live.nonzero().cpu()
    pick = bl[torch.randperm(bl.shape[0])[:24]]
    for b, l in pick.tolist():
        lg = (h[b, l].cpu().float() @ wc.T).to(torch.bfloat16).double()
        z = torch.stack([lg, torch.zeros_like(lg)])[None].requires_grad_(True)  # (1, 2, V): position 1 unused
        tl, _, _ = oracle.grpo_loss_ref(z, ids[b:b + 1, l:l + 1].cpu(), adv[b:b + 1].cpu().double(),
                                        old[b:b + 1, l:l + 1].cpu().double(), ref[b:b + 1, l:l + 1].cpu().double(),
                                        None, 1.0, 0.1, 0.2, 0.2)
        tl.backward()
        assert math.isclose(rows[1][b, l].item(), tl.item(), rel_tol=2e-3, abs_tol=2e-3), (b, l)
        assert math.isclose(rows[0][b, l].item(), torch.logsumexp(lg, 0).item(), rel_tol=1e-4, abs_tol=1e-3), (b, l)
        d = z.grad[0, 0] / (lens[b].item() * B)
        dh_ref = d.to(torch.bfloat16).float() @ wc
        assert rel_fro(gh[b, l].float().cpu(), dh_ref) < 1e-2, (b, l)


@pytest.mark.parametrize("chunk", [16, 8192])
def test_fused_linear_grpo_masked_sequences(chunk):
    """A wholly masked sequence and masks that leave later chunks empty: only the live positions reach the
    GEMMs, the rest get zero dhidden rows, and the loss matches the oracle."""
    B, L, H, V = 4, 11, 64, 512
    dtype = torch.bfloat16
    h, w, ids, adv, old, ref, mask = _case(B, L, H, V, dtype, 91)
    mask[1] = 0   # a sequence with no live token
    mask[2:] = 0  # and everything after it
    mask[0, 5:] = 0
    outs, (dh_ref, dw_ref) = _oracle(h, w, ids, adv, old, ref, mask, 1.0, 0.1, 0.2, 0.2)
    dev = gpu()
    args = (ids.to(dev), adv.to(dev), old.to(dev), ref.to(dev), mask.to(dev), 1.0, 0.1, 0.2, 0.2)
    loss, kl, clip, gh, gw, rows = flg.fused_linear_grpo_forward(h.to(dev), w.to(dev), *args, chunk=chunk)
    assert_close(loss, outs[0], name="loss", rtol=2e-3, atol=2e-3)
    assert_close(kl, outs[1], name="kl_mean", rtol=2e-3, atol=2e-3)
    assert rel_fro(gh, dh_ref) < 1e-2 and rel_fro(gw, dw_ref) < 1e-2
    live = torch.zeros(B, L + 1, dtype=torch.bool)
    live[:, :L] = mask.bool()
    assert torch.count_nonzero(gh.cpu()[~live]).item() == 0
    assert torch.count_nonzero(rows[1].cpu()[~mask.bool()]).item() == 0


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("budget", [None, -1])
def test_fused_linear_grpo_any_shape(dtype, budget):
    """H = 133 and V = 1001 (not multiples of 8): the GRPO row kernel reads rows padded with -inf logits to the
    next 16-byte multiple (probability and gradient 0 there); default and unlimited plans against the oracle."""
    B, L, H, V = 3, 20, 133, 1001
    beta, T, el, eh = 0.1, 1.0, 0.2, 0.2
    h, w, ids, adv, old, ref, mask = _case(B, L, H, V, dtype, 123)
    outs, (dh_ref, dw_ref) = _oracle(h, w, ids, adv, old, ref, mask, T, beta, el, eh)
    dev = gpu()
    print(f"FL-GRPO any shape {dtype} budget={budget}", flush=True)
    args = (ids.to(dev), adv.to(dev), _dev(old), _dev(ref), _dev(mask), T, beta, el, eh)
    loss, kl, clip, gh, gw, _ = flg.fused_linear_grpo_forward(h.to(dev), w.to(dev), *args, chunk=16,
                                                              workspace_budget=budget)
    lt = tol(dtype) if dtype == torch.float32 else dict(rtol=2e-3, atol=2e-3)
    assert_close(loss, outs[0], name="loss", **lt)
    assert_close(kl, outs[1], name="kl_mean", **lt)
    scale = B * L
    assert_close(gh.float() * scale, dh_ref * scale, name="dhidden*B*L", **tol(dtype))
    assert_close(gw.float() * scale, dw_ref * scale, name="dweight*B*L", **tol(dtype))
    assert torch.count_nonzero(gh[:, -1]).item() == 0


@pytest.mark.parametrize("form", ["out,wmn,dmn", "acc,wmn,dt", "defer,wt,dt"])
def test_fused_linear_grpo_plan_forms(form, monkeypatch):
    B, L, H, V = 4, 30, 64, 1500
    dtype = torch.bfloat16
    h, w, ids, adv, old, ref, mask = _case(B, L, H, V, dtype, 321)
    outs, (dh_ref, dw_ref) = _oracle(h, w, ids, adv, old, ref, mask, 1.0, 0.1, 0.2, 0.2)
    monkeypatch.setenv("HILDA_FL_FORM", form)
    dev = gpu()
    args = (ids.to(dev), adv.to(dev), old.to(dev), ref.to(dev), mask.to(dev), 1.0, 0.1, 0.2, 0.2)
    loss, kl, clip, gh, gw, _ = flg.fused_linear_grpo_forward(h.to(dev), w.to(dev), *args, chunk=24,
                                                              workspace_budget=-1)
    assert_close(loss, outs[0], name="loss", rtol=2e-3, atol=2e-3)
    assert rel_fro(gh, dh_ref) < 1e-2 and rel_fro(gw, dw_ref) < 1e-2
    assert_close(gw.float() * B * L, dw_ref * B * L, name="dweight*B*L", **tol(dtype))
