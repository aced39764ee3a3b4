"""CPU restatements of the reference's PyTorch implementations (test infrastructure).

Each function follows the reference file:line named in its docstring
(paths relative to /root/reference/triton-kernels/). They are used only as
the checker in tests, in ``__graft_entry__.smoke()`` and as the timed CPU
baseline in ``bench.py``; the product never calls them.

How each function is pinned (tests/test_oracle.py), independently of
retyping its formula:
  rms_norm_ref            torch.nn.functional.rms_norm (library); zeros -> zeros;
                          scale invariance; fp64 gradcheck of rms_norm_bwd_closed_form
  fused_add_rms_norm_ref  S bit-exact against bf16 addition; Y against rms_norm_ref of S
  rope_ref                complex-number rotation (x1 + i x2) * e^{i theta} (independent form);
                          position-0 identity; norm preservation; all-ones backward
                          known answer [cos+sin, cos-sin] (benchmarks/bench_rope.py:133-146)
  swiglu_ref              x * sigmoid(x) from torch.sigmoid; a = 0 -> da = 0.5*dc*b
  geglu_ref               odd-tanh identity gelu(x) - gelu(-x) = x; gelu(0) = 0, gelu'(0) = 1/2;
                          within 1e-3 of the exact (erf) GELU; tails x -> x and -> 0; fp64
                          gradcheck; a dropped cubic term or sqrt(2/pi) factor fails the erf check
  kl_div_ref              torch.nn.functional.kl_div (library) for every reduction and log_target;
                          identical distributions -> 0; Gibbs' inequality (>= 0)
  jsd_ref                 beta = 0 and beta = 1 against torch.nn.functional.kl_div (library);
                          beta = 1/2 symmetric and within [0, ln 2]; identical rows -> 0;
                          brute-force python loop (masked rows) on tiny inputs; fp64 gradcheck
  fused_linear_jsd_ref    fp64 brute force (explicit dot products, log-sum-exp and JSD by hand) on
                          tiny shapes with labels and temperature; fp64 gradcheck
  attn_res_ref            N = 1 -> h = v exactly (alpha = 1); equal blocks -> h = v; a w_query that
                          singles out one block (large score) -> h = that block; brute-force python
                          loop on tiny inputs (RMSNorm, dot, softmax, weighted sum); fp64 gradcheck
  cross_entropy_ref       torch.nn.functional.cross_entropy (library); uniform logits -> log V;
                          shift invariance; brute-force python loop on tiny inputs
  selective_log_softmax_ref  brute-force python loop (log-sum-exp by hand) on tiny inputs
  grpo_loss_ref           closed forms: old = logp, beta = 0 -> loss = -mean(A) and
                          dlogits = -A_b/(len_b*B) * (onehot - p); ref = logp -> kl = 0;
                          brute-force python loop of the per-token objective
  linear_ce_ref           fp64 brute force (explicit dot products) on tiny shapes
  exact_target_grad       equals fp64 autograd on ordinary rows; on a peaked row it matches the closed form
                          -(e^-a + e^-b) / (1 + e^-a + e^-b) of a 3-logit row [0, -a, -b] written out by hand,
                          where autograd's p_t - 1 is exactly 0
  fused_linear_grpo_ref   fp64 brute force: grpo_loss_ref on logits from explicit dot products; the
                          on-policy closed form (loss = -mean(A), dlogits = -A_b/(len_b*B) * (onehot - p) / T)
                          carried through the lm_head by explicit loops for dhidden and dweight
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F

__all__ = [
    "exact_target_grad",
    "rms_norm_ref", "rms_norm_bwd_closed_form", "fused_add_rms_norm_ref", "rope_tables", "rotate_half",
    "rope_ref", "swiglu_ref", "geglu_ref", "kl_div_ref", "jsd_ref", "fused_linear_jsd_ref", "attn_res_ref", "cross_entropy_ref", "selective_log_softmax_ref", "grpo_loss_ref",
    "linear_ce_ref", "fused_linear_grpo_ref", "fwd_bwd",
]


# ---------------------------------------------------------------------------
# RMSNorm / FusedAddRMSNorm
# ---------------------------------------------------------------------------
def _wide(t):
    """The reference's ``.float()``: at least fp32 (fp64 inputs stay fp64 so tests can run the oracle in fp64)."""
    return t if t.dtype == torch.float64 else t.float()


def rms_norm_ref(x, weight, eps=1e-6):
    """tests/test_rms_norm.py:22-28: everything in fp32, one cast at the end."""
    x_f32 = _wide(x)
    variance = x_f32.pow(2).mean(-1, keepdim=True)
    x_normed = x_f32 * torch.rsqrt(variance + eps)
    return (x_normed * _wide(weight)).to(x.dtype)


def rms_norm_bwd_closed_form(dy, x, w, eps=1e-6):
    """Closed-form RMSNorm gradients in fp64 (the formula of kernels/rms_norm.py:186-193).

    dx = rstd*(dy*w) - rstd^3 * mean(dy*w*x) * x ;  dw = sum_rows dy * x * rstd
    """
    x, dy, w = x.double(), dy.double(), w.double()
    rstd = torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps)
    m = dy * w
    dx = rstd * m - rstd.pow(3) * (m * x).mean(-1, keepdim=True) * x
    dw = (dy * x * rstd).reshape(-1, x.shape[-1]).sum(0)
    return dx, dw


def fused_add_rms_norm_ref(X, R, W, eps=1e-6):
    """benchmarks/bench_fused_add_rms_norm.py:37-41: S = X + R; Y = (S/rms).to(S.dtype) * W."""
    S = X + R
    rms = torch.sqrt(torch.mean(_wide(S) ** 2, dim=-1, keepdim=True) + eps)
    Y = (_wide(S) / rms).to(S.dtype) * W
    return Y, S


# ---------------------------------------------------------------------------
# RoPE
# ---------------------------------------------------------------------------
def rope_tables(dim, max_position_embeddings=2048, base=10000.0, dtype=torch.float32):
    """cos/sin tables of shape (1, max_pos, dim//2), as kernels/rope.py:209-222 builds them."""
    inv_freq = 1.0 / (base ** (torch.arange(0, dim, 2, dtype=torch.float32) / dim))
    t = torch.arange(max_position_embeddings, dtype=torch.float32)
    freqs = torch.outer(t, inv_freq)
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos()[None, :, : dim // 2].to(dtype), emb.sin()[None, :, : dim // 2].to(dtype)


def rotate_half(x):
    """benchmarks/bench_rope.py:40-43."""
    x1 = x[..., : x.shape[-1] // 2]
    x2 = x[..., x.shape[-1] // 2:]
    return torch.cat((-x2, x1), dim=-1)


def rope_ref(q, k, cos, sin):
    """benchmarks/bench_rope.py:46-58 (HuggingFace rotate-half RoPE).

    q, k: (B, H, T, D) logical layout (any strides); cos, sin: (1 or B, T, D//2).
    """
    cos_full = torch.cat([cos, cos], dim=-1).unsqueeze(1)
    sin_full = torch.cat([sin, sin], dim=-1).unsqueeze(1)
    q_embed = (q * cos_full) + (rotate_half(q) * sin_full)
    k_embed = (k * cos_full) + (rotate_half(k) * sin_full)
    return q_embed, k_embed


# ---------------------------------------------------------------------------
# SwiGLU
# ---------------------------------------------------------------------------
def swiglu_ref(a, b):
    """benchmarks/bench_swiglu.py:46-47: F.silu(a) * b."""
    return F.silu(a) * b


# ---------------------------------------------------------------------------
# GeGLU
# ---------------------------------------------------------------------------
def geglu_ref(a, b):
    """benchmarks/bench_geglu.py:43-44: F.gelu(a, approximate='tanh') * b (the library's tanh GELU)."""
    return F.gelu(a, approximate="tanh") * b


# ---------------------------------------------------------------------------
# KL divergence / JSD
# ---------------------------------------------------------------------------
def kl_div_ref(y_pred, y_true, reduction="batchmean", log_target=False, eps=1e-10):
    """kernels/kl_div.py:40-67 and :130-138: per-row sums of t (log max(t, eps) - y)
    (or e^t (t - y)); 'none' returns the per-row sums, 'mean' divides by rows * cols."""
    cols = y_pred.shape[-1]
    yp = y_pred.reshape(-1, cols)
    yt = y_true.reshape(-1, cols)
    if log_target:
        per = (torch.exp(yt) * (yt - yp)).sum(-1)
    else:
        per = (yt * (torch.log(torch.clamp(yt, min=eps)) - yp)).sum(-1)
    rows = yp.shape[0]
    if reduction == "none":
        return per
    if reduction == "sum":
        return per.sum()
    if reduction == "mean":
        return per.sum() / (rows * cols)
    return per.sum() / rows


def jsd_ref(X, Y, beta=0.5, labels=None, ignore_index=-100):
    """benchmarks/bench_jsd.py:30-44 (pytorch_jsd) with kernels/jsd.py's label masking
    (:48-58, :113-117): the per-row JSD(beta) summed over rows whose label is not
    ignore_index, divided by max(their count, 1) (all rows without labels)."""
    Q = X.exp()
    P = Y.exp()
    if beta == 0.0:
        per = (P * (Y - X)).sum(-1)
    elif beta == 1.0:
        per = (Q * (X - Y)).sum(-1)
    else:
        M = beta * P + (1 - beta) * Q
        log_M = M.log()
        per = beta * (P * (Y - log_M)).sum(-1) + (1 - beta) * (Q * (X - log_M)).sum(-1)
    if labels is None:
        return per.sum() / X.shape[0]
    keep = labels != ignore_index
    n = max(int(keep.sum()), 1)
    return torch.where(keep, per, torch.zeros_like(per)).sum() / n


def fused_linear_jsd_ref(s_input, s_weight, t_input, t_weight, labels=None, beta=0.5, temperature=1.0,
                         ignore_index=-100):
    """benchmarks/bench_fused_linear_jsd.py:30-41 (pytorch_linear_jsd: logits / T, log_softmax, JSD) with
    jsd_ref's beta end points and label masking (kernels/fused_linear_jsd.py:137-141,180-190); the teacher
    side is detached (:5-12)."""
    X = torch.log_softmax((s_input @ s_weight.T) / temperature, -1)
    Y = torch.log_softmax((t_input @ t_weight.T) / temperature, -1).detach()
    return jsd_ref(X, Y, beta, labels, ignore_index)


# ---------------------------------------------------------------------------
# AttnRes
# ---------------------------------------------------------------------------
def attn_res_ref(V, w_query, w_norm, eps=1e-6, key_dtype=None):
    """benchmarks/bench_attn_res.py:33-50 (pytorch_attn_res): V [N, ..., D];
    K = (V / rms(V)).to(V.dtype) * w_norm, scores <w_query, K>, softmax over N, h = sum alpha V.

    key_dtype (default V.dtype) is the dtype the keys are rounded to, twice, as the
    reference does (bench_attn_res.py:43, kernels/attn_res.py:70): pass the 16-bit
    dtype when V has been widened for the computation."""
    kd = V.dtype if key_dtype is None else key_dtype
    Vf = V.float() if V.dtype in (torch.float16, torch.bfloat16) else V
    rms = torch.sqrt(Vf.pow(2).mean(dim=-1, keepdim=True) + eps)
    K = ((Vf / rms).to(kd) * w_norm.to(kd)).to(Vf.dtype)
    scores = (K * w_query.to(Vf.dtype)).sum(-1)
    alpha = scores.softmax(dim=0)
    return (alpha.unsqueeze(-1) * Vf).sum(0).to(V.dtype)


# ---------------------------------------------------------------------------
# CrossEntropy
# ---------------------------------------------------------------------------
def cross_entropy_ref(logits, targets, ignore_index=-100, reduction="mean"):
    """benchmarks/bench_cross_entropy.py:77-79,101-103: F.cross_entropy.

    Restates two behaviours of kernels/cross_entropy.py that differ from
    torch: ``ignore_index == -1`` means "ignore nothing" (:197-198,219-225),
    and a mean over zero valid rows is 0, not NaN (:141,248).
    """
    if ignore_index == -1:
        return F.cross_entropy(logits, targets, reduction=reduction)
    if reduction == "mean":
        n_valid = (targets != ignore_index).sum()
        total = F.cross_entropy(logits, targets, ignore_index=ignore_index, reduction="sum")
        return total / n_valid.clamp(min=1).to(total.dtype)
    return F.cross_entropy(logits, targets, ignore_index=ignore_index, reduction=reduction)


# ---------------------------------------------------------------------------
# GRPO
# ---------------------------------------------------------------------------
def selective_log_softmax_ref(logits, input_ids, temperature=1.0, mask=None):
    """kernels/grpo_loss.py:65-80 semantics (log_softmax(logits/T).gather, benchmarks/bench_grpo.py:37-40).

    logits (B, L+1, V) -> logp (B, L) fp32 for the first L positions;
    ids = input_ids[:, -L:], mask = mask[:, -L:]; masked positions are 0.
    """
    B, L1, V = logits.shape
    L = L1 - 1
    ids = input_ids[:, -L:]
    logp = (_wide(logits[:, :-1, :]) / temperature).log_softmax(-1).gather(-1, ids.unsqueeze(-1)).squeeze(-1)
    if mask is not None:
        logp = torch.where(mask[:, -L:] != 0, logp, torch.zeros_like(logp))
    return logp


def grpo_loss_ref(logits, completion_ids, advantages, old_logp=None, ref_logp=None, completion_mask=None,
                  temperature=1.0, beta=0.0, eps_low=0.2, eps_high=0.2):
    """benchmarks/bench_grpo.py:30-57 for the loss; kl_mean and clip_ratio restated
    from kernels/grpo_loss.py:129-134,290-292 (the bench has no reference for them).

    Returns (loss, kl_mean or None, clip_ratio).
    """
    B, L_plus_1, V = logits.shape
    L = L_plus_1 - 1
    logits_shifted = logits[:, :-1, :] / temperature
    log_probs = logits_shifted.log_softmax(dim=-1)
    ids = completion_ids[:, -L:].unsqueeze(-1)
    logp = log_probs.gather(-1, ids).squeeze(-1)

    if old_logp is None:
        old_logp = logp.detach()
    ratio = torch.exp(logp - old_logp)
    ratio_clipped = torch.clamp(ratio, 1 - eps_low, 1 + eps_high)
    adv = advantages.unsqueeze(-1)
    loss1 = ratio * adv
    loss2 = ratio_clipped * adv
    per_token_loss = -torch.min(loss1, loss2)

    kl = None
    if beta != 0.0 and ref_logp is not None:
        kl = torch.exp(ref_logp - logp) - (ref_logp - logp) - 1
        per_token_loss = per_token_loss + beta * kl

    mask = completion_mask.float() if completion_mask is not None else torch.ones_like(per_token_loss)
    seq_lens = mask.sum(-1).clamp(min=1.0)
    loss = ((per_token_loss * mask).sum(-1) / seq_lens).mean()

    mask_sum = mask.sum().clamp(min=1.0)
    kl_mean = (kl * mask).sum() / mask_sum if kl is not None else None
    with torch.no_grad():
        r = ratio.detach()
        is_clipped = ((r < 1 - eps_low) & (adv < 0)) | ((r > 1 + eps_high) & (adv > 0))
        clip_ratio = (is_clipped.float() * mask).sum() / mask_sum
    return loss, kl_mean, clip_ratio


# ---------------------------------------------------------------------------
# FusedLinearCrossEntropy
# ---------------------------------------------------------------------------
def linear_ce_ref(hidden, weight, targets, ignore_index=-100, reduction="mean"):
    """benchmarks/bench_fused_linear_ce.py:36-38: logits = hidden @ weight.T, then CE.

    Keeps the reference's "mean over zero valid rows is 0" rule
    (kernels/fused_linear_cross_entropy.py:124-127,164-165).
    """
    logits = hidden @ weight.T
    return cross_entropy_ref(logits, targets, ignore_index=ignore_index, reduction=reduction)


# ---------------------------------------------------------------------------
# FusedLinear-GRPO (no counterpart in the reference)
# ---------------------------------------------------------------------------
def fused_linear_grpo_ref(hidden, weight, completion_ids, advantages, old_logp=None, ref_logp=None,
                          completion_mask=None, temperature=1.0, beta=0.0, eps_low=0.2, eps_high=0.2,
                          logits_dtype=None):
    """The reference's GRPO loss (grpo_loss_ref, benchmarks/bench_grpo.py:30-57) on the lm_head
    logits hidden @ weight.T (the linear of benchmarks/bench_fused_linear_ce.py:36-38).

    hidden (B, L+1, H), weight (V, H). logits_dtype rounds the logits to that dtype, as an lm_head
    GEMM that returns 16-bit logits does. Returns (loss, kl_mean or None, clip_ratio)."""
    logits = hidden @ weight.T
    if logits_dtype is not None:
        logits = logits.to(logits_dtype).to(hidden.dtype)
    return grpo_loss_ref(logits, completion_ids, advantages, old_logp, ref_logp, completion_mask, temperature,
                         beta, eps_low, eps_high)


# ---------------------------------------------------------------------------
# helpers
# ---------------------------------------------------------------------------
def exact_target_grad(d, targets, ignore_index=-100):
    """The gradient of a per-row log-softmax loss with each row's target entry formed exactly.

    For rows of the form g * (p - onehot(t)) (the CrossEntropy and GRPO gradients of
    kernels/cross_entropy.py:159-166 and kernels/grpo_loss.py:229-234) the entries sum to zero,
    so the target entry is -(sum of the row's other entries). Autograd forms it as (p_t - 1) * g,
    which cancels to 0 even in fp64 once 1 - p_t < 1e-16 (a logit 40 above the rest). d (..., V)
    and targets (...): rows whose target is ignore_index or out of range are left as they are.
    Returns a new tensor.
    """
    out = d.clone()
    V = d.shape[-1]
    flat = out.reshape(-1, V)
    t = targets.reshape(-1)
    for r in torch.nonzero((t != ignore_index) & (t >= 0) & (t < V)).flatten().tolist():
        c = int(t[r])
        row = flat[r]
        flat[r, c] = -(row[:c].sum() + row[c + 1:].sum())
    return out


def fwd_bwd(fn, inputs, grads=None, dtype=torch.float32, differentiable=None):
    """Run ``fn`` on fp32 (or ``dtype``) CPU copies of ``inputs`` and backprop.

    inputs: list of tensors (or None); entries with ``differentiable[i]`` True
    become leaves requiring grad. grads: upstream gradients for the outputs
    (None -> the outputs are scalars and backward() uses 1.0).
    Returns (outputs tuple, list of input grads).
    """
    if differentiable is None:
        differentiable = [t is not None and t.is_floating_point() for t in inputs]
    leaves = []
    for t, d in zip(inputs, differentiable):
        if t is None:
            leaves.append(None)
            continue
        c = t.detach().cpu()
        if c.is_floating_point():
            c = c.to(dtype)
        if d:
            c.requires_grad_(True)
        leaves.append(c)
    outs = fn(*leaves)
    if not isinstance(outs, (tuple, list)):
        outs = (outs,)
    diff_outs = [o for o in outs if o is not None and o.requires_grad]
    if grads is None:
        torch.autograd.backward(diff_outs[0])
    else:
        gl = [g.detach().cpu().to(o.dtype) for g, o in zip(grads, diff_outs)]
        torch.autograd.backward(diff_outs[: len(gl)], gl)
    return tuple(outs), [None if (t is None or not d) else t.grad for t, d in zip(leaves, differentiable)]


def log_v(v: int) -> float:
    return math.log(v)
