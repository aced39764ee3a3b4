"""Seeded synthetic inputs of the benchmark configurations C1-C5.

Shared by bench.py, the tests and smoke(); it holds workload definitions
only (no reference arithmetic). Every generator draws from
``torch.Generator(device).manual_seed(seed)`` in a fixed order, so the same
call on the same device gives the same tensors.
bf16 tensors are drawn in fp32 and then cast. Shapes default to the full
configuration; tests pass smaller sizes. The draws follow the descriptions
in BASELINE.json ``configs``.
"""
from __future__ import annotations

import torch

SEEDS = {"c1": 1, "c2": 2, "c3": 3, "c4": 4, "c5": 5, "f3": 6}


def rope_tables(dim, max_position_embeddings=2048, base=10000.0):
    """fp32 cos/sin tables (1, max_pos, dim//2) of RotaryEmbedding (kernels/rope.py:209-222)."""
    inv_freq = 1.0 / (base ** (torch.arange(0, dim, 2, dtype=torch.float32) / dim))
    t = torch.arange(max_position_embeddings, dtype=torch.float32)
    freqs = torch.outer(t, inv_freq)
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos()[None, :, : dim // 2].contiguous(), emb.sin()[None, :, : dim // 2].contiguous()


def _gen(device, seed):
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def _randn(g, shape, device, scale=1.0, dtype=torch.float32):
    t = torch.randn(*shape, generator=g, device=device, dtype=torch.float32)
    if scale != 1.0:
        t.mul_(scale)
    return t.to(dtype)


def c1_rms_norm(rows=4096, hidden=4096, device="cpu", seed=SEEDS["c1"]):
    """C1: RMSNorm fp32, x ~ N(0,1), w = 1 + N(0, 0.02), dy ~ N(0,1), eps = 1e-6."""
    g = _gen(device, seed)
    x = _randn(g, (rows, hidden), device)
    w = 1.0 + _randn(g, (hidden,), device, 0.02)
    dy = _randn(g, (rows, hidden), device)
    return {"x": x, "w": w, "dy": dy, "eps": 1e-6}


def c2_fused_add_rms_norm(rows=8192, hidden=4096, device="cpu", seed=SEEDS["c2"]):
    """C2 FusedAddRMSNorm bf16: x, r ~ N(0,1); w = 1 + N(0,0.02) (bf16); dy, ds ~ N(0,1)."""
    g = _gen(device, seed)
    bf = torch.bfloat16
    x = _randn(g, (rows, hidden), device, dtype=bf)
    r = _randn(g, (rows, hidden), device, dtype=bf)
    w = (1.0 + _randn(g, (hidden,), device, 0.02)).to(bf)
    dy = _randn(g, (rows, hidden), device, dtype=bf)
    ds = _randn(g, (rows, hidden), device, dtype=bf)
    return {"x": x, "r": r, "w": w, "dy": dy, "ds": ds, "eps": 1e-6}


def c2_rope(B=4, T=2048, Hq=32, Hk=8, D=128, theta=500000.0, device="cpu", seed=SEEDS["c2"] + 100):
    """C2 RoPE bf16: q [B,T,Hq,D], k [B,T,Hk,D] ~ N(0,1) stored [B,T,H,D] and
    returned as the (B,H,T,D) transposed views the reference API takes;
    fp32 cos/sin [1,T,D/2] for positions 0..T-1 at base theta; dq, dk ~ N(0,1)
    in the same layout."""
    g = _gen(device, seed)
    bf = torch.bfloat16
    q = _randn(g, (B, T, Hq, D), device, dtype=bf).transpose(1, 2)
    k = _randn(g, (B, T, Hk, D), device, dtype=bf).transpose(1, 2)
    cos, sin = rope_tables(D, T, theta)
    cos, sin = cos.to(device), sin.to(device)
    dq = _randn(g, (B, T, Hq, D), device, dtype=bf).transpose(1, 2)
    dk = _randn(g, (B, T, Hk, D), device, dtype=bf).transpose(1, 2)
    return {"q": q, "k": k, "cos": cos, "sin": sin, "dq": dq, "dk": dk}


def c2_swiglu(rows=8192, inter=14336, device="cpu", seed=SEEDS["c2"] + 200):
    """C2 SwiGLU bf16: gate, up ~ N(0,1) [rows, inter]; dc ~ N(0,1)."""
    g = _gen(device, seed)
    bf = torch.bfloat16
    a = _randn(g, (rows, inter), device, dtype=bf)
    b = _randn(g, (rows, inter), device, dtype=bf)
    dc = _randn(g, (rows, inter), device, dtype=bf)
    return {"a": a, "b": b, "dc": dc}


def c3_cross_entropy(rows=8192, vocab=128256, ignore_frac=0.10, device="cpu", seed=SEEDS["c3"]):
    """C3: logits = (2 N(0,1)).bf16 [rows, V]; targets uniform in [0,V); Bernoulli(0.1) -> -100."""
    g = _gen(device, seed)
    logits = _randn(g, (rows, vocab), device, 2.0, torch.bfloat16)
    targets = torch.randint(0, vocab, (rows,), generator=g, device=device)
    drop = torch.rand(rows, generator=g, device=device) < ignore_frac
    targets[drop] = -100
    return {"logits": logits, "targets": targets, "ignore_index": -100, "reduction": "mean"}


def c4_grpo(logp_fn, B=16, T=1024, vocab=151936, device="cpu", seed=SEEDS["c4"]):
    """C4: logits = (2 N(0,1)).bf16 [B, T, V] read as (B, L+1, V), L = T-1;
    ids uniform [0,V) (B,L); advantages N(0,1) (B,); valid lengths uniform in
    [256, T) clamped to L (prefix mask, int32); old = logp + 0.05 N, ref =
    logp + 0.1 N with logp the fp32 selective log-softmax of the logits;
    beta = 0.1, eps = 0.2, temperature = 1.

    ``logp_fn(logits, ids)`` computes logp: the tests pass the CPU oracle,
    the GPU bench passes the library's selective log-softmax (the values only
    shape the synthetic old/ref log-probs)."""
    g = _gen(device, seed)
    L = T - 1
    logits = _randn(g, (B, T, vocab), device, 2.0, torch.bfloat16)
    ids = torch.randint(0, vocab, (B, L), generator=g, device=device)
    adv = _randn(g, (B,), device)
    lo = min(256, L)
    lengths = torch.randint(lo, max(T, lo + 1), (B,), generator=g, device=device).clamp(max=L)
    mask = (torch.arange(L, device=device)[None, :] < lengths[:, None]).to(torch.int32)
    logp = logp_fn(logits, ids).float()
    old = logp + _randn(g, (B, L), device, 0.05)
    ref = logp + _randn(g, (B, L), device, 0.1)
    return {"logits": logits, "completion_ids": ids, "advantages": adv, "old_logp": old, "ref_logp": ref,
            "completion_mask": mask, "temperature": 1.0, "beta": 0.1, "eps_low": 0.2, "eps_high": 0.2}


def c5_fused_linear_ce(bt=16384, hidden=4096, vocab=128256, ignore_frac=0.05, device="cpu", seed=SEEDS["c5"]):
    """C5: hidden = N(0,1).bf16 [BT,H]; weight = (0.02 N(0,1)).bf16 [V,H];
    targets uniform [0,V) with Bernoulli(0.05) -> -100; reduction mean."""
    g = _gen(device, seed)
    h = _randn(g, (bt, hidden), device, dtype=torch.bfloat16)
    w = _randn(g, (vocab, hidden), device, 0.02, torch.bfloat16)
    targets = torch.randint(0, vocab, (bt,), generator=g, device=device)
    drop = torch.rand(bt, generator=g, device=device) < ignore_frac
    targets[drop] = -100
    return {"hidden": h, "weight": w, "targets": targets, "ignore_index": -100, "reduction": "mean"}


def f3_fused_linear_grpo(logp_fn, B=16, T=1024, hidden=4096, vocab=151936, device="cpu", seed=SEEDS["f3"]):
    """FusedLinear-GRPO (no counterpart in the reference): C4's GRPO batch behind an lm_head.
    hidden = N(0,1).bf16 (B, T, H) read as (B, L+1, H), L = T-1; weight = (0.02 N(0,1)).bf16 [V, H];
    ids, advantages and prefix masks drawn as in C4; old = logp + 0.05 N, ref = logp + 0.1 N with
    ``logp_fn(hidden, weight, ids)`` the fp32 log-probs of the ids under the lm_head logits."""
    g = _gen(device, seed)
    L = T - 1
    h = _randn(g, (B, T, hidden), device, dtype=torch.bfloat16)
    w = _randn(g, (vocab, hidden), device, 0.02, torch.bfloat16)
    ids = torch.randint(0, vocab, (B, L), generator=g, device=device)
    adv = _randn(g, (B,), device)
    lo = min(256, L)
    lengths = torch.randint(lo, max(T, lo + 1), (B,), generator=g, device=device).clamp(max=L)
    mask = (torch.arange(L, device=device)[None, :] < lengths[:, None]).to(torch.int32)
    logp = logp_fn(h, w, ids).float()
    old = logp + _randn(g, (B, L), device, 0.05)
    ref = logp + _randn(g, (B, L), device, 0.1)
    return {"hidden": h, "weight": w, "completion_ids": ids, "advantages": adv, "old_logp": old, "ref_logp": ref,
            "completion_mask": mask, "temperature": 1.0, "beta": 0.1, "eps_low": 0.2, "eps_high": 0.2}
