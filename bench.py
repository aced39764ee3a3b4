"""Benchmark of the hilda-kernel_amd hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--ops all|c2|none] [--no-cpu]

Headline (``value``): fwd+bwd throughput of the BASELINE.json configs[1]
workload, the Llama-3-8B layer ops in bf16 — FusedAddRMSNorm [8192,4096],
RoPE q[4,2048,32,128] + k[4,2048,8,128] ([B,T,H,D] storage), SwiGLU
[8192,14336] — as algorithmic HBM GB/s. One step = one fwd+bwd of the three
ops (inputs resident in HBM, grads via torch.autograd.grad so nothing is
accumulated). ``ops`` adds each configuration's op on its own (C1-C5), timed
with HIP events and a 512 MiB cache flush between reps; C5 (FusedLinearCE)
is reported in TFLOP/s of 6*n_valid*H*V. ``roofline`` is the
dominant kernel of the step (SwiGLU backward), timed per launch with HIP
events on its stream inside the timed region. ``cpu_baseline`` times the CPU
PyTorch reference path (the oracle) on the full C2 step, repeated for about
10 s of CPU work.

Prints one JSON line on stdout; progress goes to stderr.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "hilda-kernel_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import torch  # noqa: E402

import workloads  # noqa: E402

METRIC = "fwd+bwd HBM GB/s & % roofline per op; FusedLinearCE TFLOP/s (1 GPU)"
HBM_PEAK_GBPS = 8000.0
BF16_PEAK_TFLOPS = 2500.0


def log(*a):
    print(*a, file=sys.stderr, flush=True)


class TimingEvent:
    """A HIP timing event. By default created with hipEventDisableSystemFence, the flag HIP documents for
    events used only to time: recording it takes no system-scope release/acquire (no L2 write-back and
    invalidate between the kernels it sits between), so markers inside a timed region perturb it least. The
    elapsed time between two such events spans the launches between them, as rocprofv3's kernel timestamps do.
    fence=True gives a default event (the system-scope release that torch's timing events take): recorded at
    the end of a timed region, the region then includes writing the op's dirty L2 lines back to HBM."""
    _hip = None
    _FLAGS = 0x20000000  # hipEventDisableSystemFence

    @classmethod
    def _lib(cls):
        if cls._hip is None:
            import ctypes
            hip = ctypes.CDLL("libamdhip64.so")
            hip.hipEventCreateWithFlags.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_uint]
            hip.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
            hip.hipEventSynchronize.argtypes = [ctypes.c_void_p]
            hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
            hip.hipEventDestroy.argtypes = [ctypes.c_void_p]
            cls._hip = hip
        return cls._hip

    def __init__(self, fence=False):
        import ctypes
        self._ct = ctypes
        self.ev = ctypes.c_void_p()
        rc = self._lib().hipEventCreateWithFlags(ctypes.byref(self.ev), 0 if fence else self._FLAGS)
        if rc != 0:
            raise RuntimeError(f"hipEventCreateWithFlags failed ({rc})")

    def record(self, stream):
        rc = self._lib().hipEventRecord(self.ev, stream.cuda_stream)
        if rc != 0:
            raise RuntimeError(f"hipEventRecord failed ({rc})")

    def elapsed_time(self, end) -> float:
        hip = self._lib()
        if hip.hipEventSynchronize(end.ev) != 0:
            raise RuntimeError("hipEventSynchronize failed")
        ms = self._ct.c_float()
        rc = hip.hipEventElapsedTime(self._ct.byref(ms), self.ev, end.ev)
        if rc != 0:
            raise RuntimeError(f"hipEventElapsedTime failed ({rc})")
        return ms.value

    def __del__(self):
        if self._hip is not None and self.ev:
            self._hip.hipEventDestroy(self.ev)


# ---------------------------------------------------------------------------
# algorithmic work (each required input read once, each output written once)
# ---------------------------------------------------------------------------
def bytes_fused_add(rows, hidden, es=2):
    # fwd: X, R read; S, Y write; bwd: dY, dS, S read; dX write; plus W, RSTD, dW
    return 8 * rows * hidden * es + 3 * hidden * es + 2 * rows * 4


def bytes_rms_norm(rows, hidden, es=4):
    # fwd: X read, Y write; bwd: dY, X read, dX write; plus W, RSTD, dW
    return 5 * rows * hidden * es + 3 * hidden * es + 2 * rows * 4


def bytes_rope(q_elems, k_elems, T, D, es=2):
    # each direction reads q,k and writes q',k'; cos/sin fp32 [T, D/2] read per direction
    return 4 * (q_elems + k_elems) * es + 2 * 2 * T * (D // 2) * 4


def bytes_swiglu(rows, inter, es=2):
    # fwd: a, b read, c write; bwd: a, b, dc read, da, db write
    return 8 * rows * inter * es


def bytes_swiglu_bwd(rows, inter, es=2):
    return 5 * rows * inter * es


# ---------------------------------------------------------------------------
# the C2 step
# ---------------------------------------------------------------------------
class C2Step:
    def __init__(self, K, dev, scale=1):
        fa = workloads.c2_fused_add_rms_norm(rows=8192 // scale, device=dev)
        rp = workloads.c2_rope(B=max(1, 4 // scale), device=dev)
        sw = workloads.c2_swiglu(rows=8192 // scale, device=dev)
        self.K = K
        self.x = fa["x"].requires_grad_(True)
        self.r = fa["r"].requires_grad_(True)
        self.w = fa["w"].requires_grad_(True)
        self.dy, self.ds = fa["dy"], fa["ds"]
        self.q = rp["q"].detach().requires_grad_(True)   # (B,H,T,D) view of [B,T,H,D] storage
        self.k = rp["k"].detach().requires_grad_(True)
        self.cos, self.sin = rp["cos"], rp["sin"]
        self.dq, self.dk = rp["dq"], rp["dk"]
        self.a = sw["a"].requires_grad_(True)
        self.b = sw["b"].requires_grad_(True)
        self.dc = sw["dc"]
        rows, hidden = self.x.shape
        self.bytes = {
            "fused_add_rms_norm": bytes_fused_add(rows, hidden),
            "rope": bytes_rope(self.q.numel(), self.k.numel(), self.q.shape[2], self.q.shape[3]),
            "swiglu": bytes_swiglu(*self.a.shape),
        }
        self.swiglu_bwd_bytes = bytes_swiglu_bwd(*self.a.shape)

    def fused_add(self):
        K = self.K
        y, s = K.hilda_fused_add_rms_norm(self.x, self.r, self.w)
        return torch.autograd.grad([y, s], [self.x, self.r, self.w], [self.dy, self.ds])

    def rope(self):
        K = self.K
        qo, ko = K.hilda_rope(self.q, self.k, self.cos, self.sin)
        return torch.autograd.grad([qo, ko], [self.q, self.k], [self.dq, self.dk])

    def swiglu(self):
        K = self.K
        c = K.hilda_swiglu(self.a, self.b)
        return torch.autograd.grad([c], [self.a, self.b], [self.dc])

    def step(self):
        # each op's backward right after its forward (one autograd pass over all three outputs measured
        # 2% slower on the GPU: its reverse order re-reads the earlier ops' inputs after they left the
        # Infinity Cache, while it saved 100 us of host time a step that the GPU hides anyway)
        self.fused_add()
        self.rope()
        self.swiglu()

    def total_bytes(self):
        return sum(self.bytes.values())


# ---------------------------------------------------------------------------
# per-op timing with HIP events and a cache flush between reps
# ---------------------------------------------------------------------------
class Flusher:
    """Reads a 512 MiB buffer so MI355X's 256 MB MALL and the L2s hold none of the op's data.

    A read, not a write: a written flush buffer leaves up to 256 MB of dirty lines in the
    caches, and writing them back would be charged to the timed op (it halves the apparent
    bandwidth of a 64 MB copy). Earlier dirty lines are written back during the flush itself.
    """

    def __init__(self, dev):
        # fp32, so the sum reads the buffer directly (an integer sum widens it through a copy first)
        self.buf = torch.ones(128 << 20, dtype=torch.float32, device=dev)

    def __call__(self):
        self.sink = torch.sum(self.buf)


def time_events(fn, reps, flush=None, warmup=2):
    # Each rep starts after a flush (a read of 512 MiB: the op's inputs come from HBM). The start event is
    # fence-free: after a read-only flush the L2 holds nothing dirty, and a fenced record's write-back and
    # invalidate (about 5 us) would be charged to the op. The end event is fenced, so the op is charged for
    # writing all of its dirty L2 lines back to HBM.
    for _ in range(warmup):
        fn()
    stream = torch.cuda.current_stream()
    starts = [TimingEvent() for _ in range(reps)]
    ends = [TimingEvent(fence=True) for _ in range(reps)]
    for i in range(reps):
        if flush is not None:
            flush()
        starts[i].record(stream)
        fn()
        ends[i].record(stream)
    torch.cuda.synchronize()
    return [s.elapsed_time(e) for s, e in zip(starts, ends)]


def op_entry(config, ms_list, work, unit, peak):
    ms = statistics.median(ms_list)
    rate = work / (ms * 1e-3) / (1e9 if unit == "GB/s" else 1e12)
    return {"config": config, "ms": round(ms, 5), "value": round(rate, 2), "unit": unit,
            "frac": round(rate / peak, 4), "work": work, "reps": len(ms_list)}


def bench_c2_ops(c2, reps, flush):
    out = {}
    for name, fn in (("fused_add_rms_norm", c2.fused_add), ("rope", c2.rope), ("swiglu", c2.swiglu)):
        out[name] = op_entry("C2", time_events(fn, reps, flush), c2.bytes[name], "GB/s", HBM_PEAK_GBPS)
        log(f"  {name}: {out[name]['ms']:.4f} ms  {out[name]['value']:.0f} GB/s  ({out[name]['frac']:.1%})")
    return out


def bench_c1(K, dev, reps, flush, cpu=False):
    c = workloads.c1_rms_norm(device=dev)
    x = c["x"].requires_grad_(True)
    w = c["w"].requires_grad_(True)
    dy = c["dy"]

    def fn():
        y = K.hilda_rms_norm(x, w, c["eps"])
        return torch.autograd.grad([y], [x, w], [dy])

    work = bytes_rms_norm(*x.shape)
    e = op_entry("C1", time_events(fn, reps, flush), work, "GB/s", HBM_PEAK_GBPS)
    log(f"  rms_norm (C1 fp32): {e['ms']:.4f} ms  {e['value']:.0f} GB/s  ({e['frac']:.1%})")
    if cpu:
        import oracle
        xc, wc, dyc = (t.detach().cpu().requires_grad_(t is not dy) for t in (x, w, dy))

        def step():
            y = oracle.rms_norm_ref(xc, wc, c["eps"])
            torch.autograd.grad([y], [xc, wc], [dyc])

        e["cpu_baseline"] = cpu_entry(step, work, "GB/s", 1.0, "the full C1 input (x [4096,4096] fp32), the "
                                      "PyTorch reference path fwd+bwd", False)
    return e


def bench_geglu(K, dev, reps, flush):
    """GeGLU (next row beyond the C1-C5 configs): bf16 [8192, 14336], the reference benchmark's Mistral-7B row
    (benchmarks/bench_geglu.py:185-190), on the C2 SwiGLU inputs."""
    c = workloads.c2_swiglu(device=dev)
    a = c["a"].requires_grad_(True)
    b = c["b"].requires_grad_(True)
    dc = c["dc"]

    def fn():
        out = K.hilda_geglu(a, b)
        return torch.autograd.grad([out], [a, b], [dc])

    e = op_entry("geglu [8192,14336] bf16", time_events(fn, reps, flush), bytes_swiglu(*a.shape), "GB/s",
                 HBM_PEAK_GBPS)
    log(f"  geglu: {e['ms']:.4f} ms  {e['value']:.0f} GB/s  ({e['frac']:.1%})")
    return e


def _logprobs(rows, V, dev, seed):
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    x = torch.randn(rows, V, generator=g, device=dev, dtype=torch.float32)
    return torch.log_softmax(x, -1).to(torch.bfloat16)


def bench_kl_div(K, dev, reps, flush, rows=8192, V=128256):
    """KLDiv (next row): bf16 [8192, 128256] log-probabilities vs probabilities, 'batchmean', fwd+bwd
    (benchmarks/bench_kl_div.py:156-160 sizes)."""
    yp = _logprobs(rows, V, dev, 11).requires_grad_(True)
    yt = _logprobs(rows, V, dev, 12).float().exp().to(torch.bfloat16)

    def fn():
        loss = K.hilda_kl_div(yp, yt)
        return torch.autograd.grad([loss], [yp])

    # fwd reads y_pred and y_true; bwd reads y_true and writes dy_pred
    e = op_entry(f"kl_div [{rows},{V}] bf16", time_events(fn, reps, flush), 4 * 2 * rows * V, "GB/s", HBM_PEAK_GBPS)
    log(f"  kl_div: {e['ms']:.4f} ms  {e['value']:.0f} GB/s  ({e['frac']:.1%})")
    return e


def bench_jsd(K, dev, reps, flush, rows=8192, V=128256):
    """JSD(beta = 1/2) (next row): bf16 [8192, 128256] student and teacher log-probabilities, fwd+bwd
    (benchmarks/bench_jsd.py sizes)."""
    X = _logprobs(rows, V, dev, 13).requires_grad_(True)
    Y = _logprobs(rows, V, dev, 14)

    def fn():
        loss = K.hilda_jsd(X, Y, 0.5)
        return torch.autograd.grad([loss], [X])

    # one pass reads X and Y and writes dX; a unit upstream gradient leaves dX as is
    e = op_entry(f"jsd [{rows},{V}] bf16", time_events(fn, reps, flush), 3 * 2 * rows * V, "GB/s", HBM_PEAK_GBPS)
    log(f"  jsd: {e['ms']:.4f} ms  {e['value']:.0f} GB/s  ({e['frac']:.1%})")
    return e


def bench_fljsd(K, dev, reps, flush, BT=8192, H=4096, V=128256):
    """FusedLinearJSD (next row): student and teacher hidden [8192, 4096] ~ N(0,1), lm_heads [128256, 4096]
    ~ N(0, 0.02), beta = 1/2, bf16, fwd+bwd; in TFLOP/s of its four GEMMs, 8 BT H V."""
    g = torch.Generator(device=dev)
    g.manual_seed(21)
    bf = torch.bfloat16
    si = torch.randn(BT, H, generator=g, device=dev).to(bf).requires_grad_(True)
    sw = (0.02 * torch.randn(V, H, generator=g, device=dev)).to(bf).requires_grad_(True)
    ti = torch.randn(BT, H, generator=g, device=dev).to(bf)
    tw = (0.02 * torch.randn(V, H, generator=g, device=dev)).to(bf)

    def run(budget):
        def fn():
            loss = K.hilda_fused_linear_jsd(si, sw, ti, tw, workspace_budget=budget)
            return torch.autograd.grad([loss], [si, sw])
        return fn

    work = 8 * BT * H * V
    e = op_entry(f"fused_linear_jsd BT={BT} H={H} V={V} bf16 (workspace_budget='fastest')",
                 time_events(run("fastest"), reps, flush, warmup=1), work, "TFLOP/s", BF16_PEAK_TFLOPS)
    d_ms = statistics.median(time_events(run(None), max(3, reps // 2), flush, warmup=1))
    e["default_plan"] = {"ms": round(d_ms, 3), "value": round(work / (d_ms * 1e-3) / 1e12, 2), "unit": "TFLOP/s"}
    # fwd+bwd peak above the resident inputs, as for FusedLinearCE
    e["peak_mib"] = {"fastest": peak_mib(run("fastest"), dev), "default": peak_mib(run(None), dev)}
    log(f"  fused_linear_jsd: fastest plan {e['ms']:.3f} ms  {e['value']:.1f} TFLOP/s  ({e['frac']:.1%}), peak "
        f"{e['peak_mib']['fastest']} MiB; default plan {d_ms:.3f} ms, peak {e['peak_mib']['default']} MiB")
    del si, sw, ti, tw
    torch.cuda.empty_cache()
    # the reference's memory configs (bench_fused_linear_jsd.py:163-165,180), default plan
    e["reference_memory_configs"] = []
    for N_, V_ in ((4096, 32000), (2048, 128256)):
        r = fljsd_memory(K, dev, N_, H, V_, torch.float16, reps=3, flush=flush)
        e["reference_memory_configs"].append(r)
        log(f"    {r['config']}: torch fp32 {r['torch_fp32']['peak_mib']} MiB {r['torch_fp32']['ms']} ms; default "
            f"{r['default']['peak_mib']} MiB ({r['default']['saving']:.1%} less) {r['default']['ms']} ms")
    return e


def bench_attn_res(K, dev, reps, flush, N=8, B=4, T=2048, D=4096):
    """AttnRes (next row): N=8 blocks [4, 2048, 4096] bf16 ~ N(0,1), w_query 0.02 N(0,1), w_norm 1, fwd+bwd
    (benchmarks/bench_attn_res.py:205-211, its bf16 row)."""
    g = torch.Generator(device=dev)
    g.manual_seed(31)
    bf = torch.bfloat16
    V = torch.randn(N, B, T, D, generator=g, device=dev).to(bf).requires_grad_(True)
    wq = (0.02 * torch.randn(D, generator=g, device=dev)).to(bf).requires_grad_(True)
    wn = torch.ones(D, device=dev, dtype=bf).requires_grad_(True)
    dh = torch.randn(B, T, D, generator=g, device=dev).to(bf)

    def fn():
        h = K.hilda_attn_res(V, wq, wn)
        return torch.autograd.grad([h], [V, wq, wn], [dh])

    # fwd reads V, writes h; bwd reads dh and V, writes dV
    e = op_entry(f"attn_res N={N} [{B},{T},{D}] bf16", time_events(fn, reps, flush), (3 * N + 2) * B * T * D * 2,
                 "GB/s", HBM_PEAK_GBPS)
    log(f"  attn_res: {e['ms']:.4f} ms  {e['value']:.0f} GB/s  ({e['frac']:.1%})")
    return e


def bench_c3(K, dev, reps, flush, cpu=False):
    c = workloads.c3_cross_entropy(device=dev)
    logits = c["logits"].requires_grad_(True)
    t = c["targets"]
    N, V = logits.shape
    n_valid = int((t != -100).sum())

    def fn():
        loss = K.hilda_cross_entropy(logits, t)
        return torch.autograd.grad([loss], [logits])

    # read the contributing rows once, write every gradient row, targets + per-row loss
    work = 2 * V * n_valid + 2 * V * N + 12 * N
    e = op_entry("C3", time_events(fn, reps, flush), work, "GB/s", HBM_PEAK_GBPS)
    e["n_valid"] = n_valid
    e["row_bytes"] = V * logits.element_size()
    log(f"  cross_entropy (C3): {e['ms']:.4f} ms  {e['value']:.0f} GB/s  ({e['frac']:.1%})")
    if cpu:
        import oracle
        rows = 512
        lc = logits[:rows].detach().cpu().requires_grad_(True)
        tc = t[:rows].cpu()

        def step():
            loss = oracle.cross_entropy_ref(lc, tc)
            torch.autograd.grad([loss], [lc])

        e["cpu_baseline"] = cpu_entry(step, work, "GB/s", N / rows, f"the first {rows} of the 8192 C3 rows (bf16 "
                                      "logits, F.cross_entropy fwd+bwd), time scaled by 8192/512", True)
    return e


def bench_c4(K, dev, reps, flush, cpu=False):
    sls = K.fused_selective_log_softmax
    c = workloads.c4_grpo(lambda lg, ids: sls(lg, torch.cat([torch.zeros_like(ids[:, :1]), ids], 1)), device=dev)
    logits = c["logits"].requires_grad_(True)
    args = [c[k] for k in ("completion_ids", "advantages", "old_logp", "ref_logp", "completion_mask")]
    B, L1, V = logits.shape
    L = L1 - 1
    n_valid = int(c["completion_mask"].sum())

    def fn():
        loss, _, _ = K.hilda_grpo_loss(logits, *args, c["temperature"], c["beta"], c["eps_low"], c["eps_high"])
        return torch.autograd.grad([loss], [logits])

    work = 2 * V * n_valid + 2 * V * B * (L + 1) + 36 * B * L
    e = op_entry("C4", time_events(fn, reps, flush), work, "GB/s", HBM_PEAK_GBPS)
    e["row_bytes"] = V * logits.element_size()
    e["n_valid"] = n_valid
    log(f"  grpo_loss (C4): {e['ms']:.4f} ms  {e['value']:.0f} GB/s  ({e['frac']:.1%})")
    if cpu:
        import oracle
        lc = logits[:1].detach().cpu().requires_grad_(True)
        ac = [a[:1].cpu() for a in args]

        def step():
            # benchmarks/bench_grpo.py:80,158: the reference path runs on logits.float()
            loss, _, _ = oracle.grpo_loss_ref(lc.float(), *ac, c["temperature"], c["beta"], c["eps_low"],
                                              c["eps_high"])
            torch.autograd.grad([loss], [lc])

        e["cpu_baseline"] = cpu_entry(step, work, "GB/s", B, f"sequence 0 of the 16 C4 sequences (logits "
                                      f"[1,1024,151936] bf16, the reference path on logits.float()), time scaled "
                                      f"by 16", True)
    return e


def peak_mib(fn, dev):
    """Peak device memory of one call of fn above what was allocated before it, in MiB, measured as the
    reference's benchmark measures it (bench_fused_linear_ce.py:171-178): after a warm-up call, reset the peak
    statistics, run, read torch.cuda.max_memory_allocated."""
    fn()
    torch.cuda.synchronize(dev)
    torch.cuda.reset_peak_memory_stats(dev)
    base = torch.cuda.memory_allocated(dev)
    fn()
    torch.cuda.synchronize(dev)
    return round((torch.cuda.max_memory_allocated(dev) - base) / 2**20, 1)


def torch_gemms_c5(dev, H, V, n_live, reps, flush, chunk=8192):
    """torch.mm (hipBLASLt) on the three GEMM shapes of C5's fastest plan, bf16 in, bf16 out: a full chunk's
    logits X W^T and dX = D W, and the one dW = D^T X over the live rows. The library's own GEMMs on these
    shapes are the rows of a kernel trace of the same run; this is the vendor library's time beside them."""
    g = torch.Generator(device=dev).manual_seed(7)
    bf = torch.bfloat16
    x = torch.randn(chunk, H, generator=g, device=dev).to(bf)
    w = (0.02 * torch.randn(V, H, generator=g, device=dev)).to(bf)
    d = (1e-3 * torch.randn(chunk, V, generator=g, device=dev)).to(bf)
    out = {}
    lg = torch.empty(chunk, V, dtype=bf, device=dev)
    dx = torch.empty(chunk, H, dtype=bf, device=dev)
    shapes = [("logits", lambda: torch.mm(x, w.t(), out=lg), 2 * chunk * H * V, [chunk, V, H]),
              ("dx", lambda: torch.mm(d, w, out=dx), 2 * chunk * H * V, [chunk, H, V])]
    for name, fn, flops, mnk in shapes:
        ms = statistics.median(time_events(fn, reps, flush, warmup=1))
        out[name] = {"mnk": mnk, "ms": round(ms, 3), "tflops": round(flops / (ms * 1e-3) / 1e12, 1)}
    del lg, dx, d, x
    dt = (1e-3 * torch.randn(V, n_live, generator=g, device=dev)).to(bf)
    xk = torch.randn(n_live, H, generator=g, device=dev).to(bf)
    dw = torch.empty(V, H, dtype=bf, device=dev)
    ms = statistics.median(time_events(lambda: torch.mm(dt, xk, out=dw), reps, flush, warmup=1))
    out["dw"] = {"mnk": [V, H, n_live], "ms": round(ms, 3), "tflops": round(2 * n_live * H * V / (ms * 1e-3) / 1e12, 1)}
    del dt, xk, dw, w
    torch.cuda.empty_cache()
    return out


def flce_memory(K, dev, N, H, V, dtype, budgets=(None,), reps=3, flush=None, seed=0):
    """fwd+bwd peak memory and time of FusedLinearCE against torch's unfused hidden @ W.T + cross_entropy on
    the same GPU. Peak: leaves allocated inside the measured function, as the reference's bench_memory does
    (bench_fused_linear_ce.py:181-214). Time: resident leaves, flushed cache, median of reps. budgets: None (the
    default), 'fastest', bytes, or 'reference_form' (16-bit only): the reference's own memory and dW arithmetic."""
    from kernels import fused_linear_cross_entropy as fl
    g = torch.Generator(device=dev).manual_seed(seed)
    tg = torch.randint(0, V, (N,), device=dev, generator=g)

    def fresh(f):
        def fn():
            h = torch.randn(N, H, device=dev, dtype=dtype, requires_grad=True)
            w = torch.randn(V, H, device=dev, dtype=dtype, requires_grad=True)
            f(h, w).backward()
        return fn

    hs = torch.randn(N, H, device=dev, dtype=dtype, generator=g).requires_grad_(True)
    ws = (0.02 * torch.randn(V, H, device=dev, dtype=dtype, generator=g)).requires_grad_(True)

    def resident(f):
        def fn():
            return torch.autograd.grad([f(hs, ws)], [hs, ws])
        return fn

    def unfused(h, w):
        return torch.nn.functional.cross_entropy(h @ w.T, tg)

    out = {"config": f"N={N} H={H} V={V} {str(dtype).replace('torch.', '')}"}
    pu = peak_mib(fresh(unfused), dev)
    tu = statistics.median(time_events(resident(unfused), reps, flush, warmup=1))
    out["unfused_torch"] = {"peak_mib": pu, "ms": round(tu, 3)}
    torch.cuda.empty_cache()
    for b in budgets:
        key = "default" if b is None else str(b)
        forced = b == "reference_form"
        if forced:
            # the reference's footprint and dW arithmetic: a workspace of what its chunk loop holds at once (the
            # chunk's logits and the [V, H] product dlogits^T X, fused_linear_cross_entropy.py:113-161) and dW summed
            # in the weight dtype over row chunks (fewer than its chunks), through the planner's debugging override
            inc = -(-V // H)
            per = -(-N // inc)
            b = min(1 << (per - 1).bit_length(), N) * V * 2 + V * H * 2
            os.environ["HILDA_FL_FORM"] = "out,wmn,dmn"
        try:
            f = (lambda h, w, b=b: K.hilda_fused_linear_cross_entropy(h, w, tg, workspace_budget=b))
            p = peak_mib(fresh(f), dev)
            t = statistics.median(time_events(resident(f), reps, flush, warmup=1))
            plan = fl.fused_linear_cross_entropy_plan(N, H, V, dtype, workspace_budget=b)
        finally:
            if forced:
                del os.environ["HILDA_FL_FORM"]
        out[key] = {
            "peak_mib": p, "saving": round(1 - p / pu, 4), "ms": round(t, 3), "speed_vs_unfused": round(tu / t, 3),
            "plan": {k: plan[k] for k in ("chunk", "chunks", "dw", "w_transposed", "d_transposed")},
            "workspace_mib": round(plan["workspace_bytes"] / 2**20, 1)}
        torch.cuda.empty_cache()
    del hs, ws
    torch.cuda.empty_cache()
    return out


def fljsd_memory(K, dev, N, H, V, dtype, reps=3, flush=None, seed=0):
    """FusedLinearJSD's fwd+bwd peak memory and time against the reference's PyTorch path, the way the reference's
    benchmark measures them (bench_fused_linear_jsd.py:30-41,180-206): linear + log_softmax + JSD on fp32 copies of
    all four inputs, leaves allocated inside the measured function. Time: resident leaves, flushed cache."""
    g = torch.Generator(device=dev).manual_seed(seed)

    def torch_jsd(si, sw, ti, tw, beta=0.5, temperature=1.0):
        # every intermediate named, so each lives as long as in the reference's function: its peak memory
        s_logits = (si @ sw.t()) / temperature
        t_logits = (ti @ tw.t()) / temperature
        x = s_logits.log_softmax(dim=-1)
        y = t_logits.log_softmax(dim=-1)
        q = x.exp()
        p = y.exp()
        m = beta * p + (1 - beta) * q
        log_m = m.log()
        loss = beta * (p * (y - log_m)).sum(-1) + (1 - beta) * (q * (x - log_m)).sum(-1)
        return loss.mean()

    def ours(si, sw, ti, tw):
        return K.hilda_fused_linear_jsd(si, sw, ti, tw)

    def upcast(si, sw, ti, tw):
        return torch_jsd(si.float(), sw.float(), ti.float(), tw.float())

    def fresh(f):
        def fn():
            si = torch.randn(N, H, device=dev, dtype=dtype, requires_grad=True)
            sw = torch.randn(V, H, device=dev, dtype=dtype, requires_grad=True)
            ti = torch.randn(N, H, device=dev, dtype=dtype)
            tw = torch.randn(V, H, device=dev, dtype=dtype)
            f(si, sw, ti, tw).backward()
        return fn

    si = torch.randn(N, H, device=dev, dtype=dtype, generator=g).requires_grad_(True)
    sw = (0.02 * torch.randn(V, H, device=dev, dtype=dtype, generator=g)).requires_grad_(True)
    ti = torch.randn(N, H, device=dev, dtype=dtype, generator=g)
    tw = 0.02 * torch.randn(V, H, device=dev, dtype=dtype, generator=g)

    def resident(f):
        return lambda: torch.autograd.grad([f(si, sw, ti, tw)], [si, sw])

    out = {"config": f"N={N} H={H} V={V} {str(dtype).replace('torch.', '')}"}
    pu = peak_mib(fresh(upcast), dev)
    tu = statistics.median(time_events(resident(upcast), reps, flush, warmup=1))
    out["torch_fp32"] = {"peak_mib": pu, "ms": round(tu, 3)}
    torch.cuda.empty_cache()
    p = peak_mib(fresh(ours), dev)
    t = statistics.median(time_events(resident(ours), reps, flush, warmup=1))
    out["default"] = {"peak_mib": p, "saving": round(1 - p / pu, 4), "ms": round(t, 3),
                      "speed_vs_torch": round(tu / t, 2)}
    del si, sw, ti, tw
    torch.cuda.empty_cache()
    return out


def bench_c5(K, dev, reps, flush, cpu=False):
    """C5 in two memory plans: the unlimited workspace budget ('fastest': two 8192-row chunks, every chunk's
    D^T kept and one dW GEMM) is the entry's headline time; the default plan (the reference's memory class)
    beside it, each with its fwd+bwd peak memory against torch's unfused path."""
    from kernels import fused_linear_cross_entropy as fl
    c = workloads.c5_fused_linear_ce(device=dev)
    h = c["hidden"].requires_grad_(True)
    w = c["weight"].requires_grad_(True)
    t = c["targets"]
    BT, H = h.shape
    V = w.shape[0]
    n_valid = int((t != -100).sum())
    work = 6 * n_valid * H * V  # conservative: ignored rows need no FLOPs

    def run(budget):
        def fn():
            loss = K.hilda_fused_linear_cross_entropy(h, w, t, workspace_budget=budget)
            return torch.autograd.grad([loss], [h, w])
        return fn

    e = op_entry("C5 (workspace_budget='fastest')", time_events(run("fastest"), reps, flush, warmup=1), work,
                 "TFLOP/s", BF16_PEAK_TFLOPS)
    dense = 6 * BT * H * V
    e["dense_equivalent_tflops"] = round(dense / (e["ms"] * 1e-3) / 1e12, 2)
    e["n_valid"] = n_valid
    e["plan"] = fl.fused_linear_cross_entropy_plan(BT, H, V, torch.bfloat16, workspace_budget="fastest")
    d_ms = statistics.median(time_events(run(None), max(3, reps // 2), flush, warmup=1))
    e["default_plan"] = {"ms": round(d_ms, 3), "value": round(work / (d_ms * 1e-3) / 1e12, 2), "unit": "TFLOP/s",
                         "plan": fl.fused_linear_cross_entropy_plan(BT, H, V, torch.bfloat16)}
    log(f"  fused_linear_cross_entropy (C5): fastest plan {e['ms']:.3f} ms  {e['value']:.1f} TFLOP/s  "
        f"({e['frac']:.1%}); default plan {d_ms:.3f} ms")
    del h, w, c
    torch.cuda.empty_cache()
    e["torch_gemms"] = torch_gemms_c5(dev, H, V, n_valid, max(3, reps // 2), flush)
    tg = e["torch_gemms"]
    log(f"    hipBLASLt (torch.mm) on the same GEMMs: logits {tg['logits']['ms']} ms, dX {tg['dx']['ms']} ms, "
        f"dW {tg['dw']['ms']} ms")
    # peak memory at C5 (fresh leaves of the same shapes) and at the reference's memory configs
    # (bench_fused_linear_ce.py:270-274, fp16), default plan
    e["memory"] = flce_memory(K, dev, BT, H, V, torch.bfloat16, budgets=(None, "fastest", "reference_form"), reps=3,
                              flush=flush)
    m = e["memory"]
    log(f"    C5 peak: unfused {m['unfused_torch']['peak_mib']} MiB ({m['unfused_torch']['ms']} ms), default "
        f"{m['default']['peak_mib']} MiB ({m['default']['saving']:.1%} less), fastest {m['fastest']['peak_mib']} "
        f"MiB ({m['fastest']['saving']:.1%} less); the reference's footprint and dW arithmetic "
        f"{m['reference_form']['peak_mib']} MiB, {m['reference_form']['ms']} ms")
    e["reference_memory_configs"] = []
    for N_, H_, V_ in ((8192, 4096, 32000), (8192, 4096, 128256), (4096, 4096, 128256)):
        r = flce_memory(K, dev, N_, H_, V_, torch.float16, budgets=(None, "reference_form"), reps=3, flush=flush)
        e["reference_memory_configs"].append(r)
        log(f"    {r['config']}: unfused {r['unfused_torch']['peak_mib']} MiB {r['unfused_torch']['ms']} ms; "
            f"default {r['default']['peak_mib']} MiB ({r['default']['saving']:.1%} less) {r['default']['ms']} ms; "
            f"reference form {r['reference_form']['peak_mib']} MiB ({r['reference_form']['saving']:.1%} less) "
            f"{r['reference_form']['ms']} ms")
    if cpu:
        import oracle
        rows = 128
        c = workloads.c5_fused_linear_ce(device=dev)
        hc = c["hidden"][:rows].detach().cpu().requires_grad_(True)
        wc = c["weight"].detach().cpu().requires_grad_(True)
        tc = c["targets"][:rows].cpu()
        del c
        torch.cuda.empty_cache()

        def step():
            loss = oracle.linear_ce_ref(hc, wc, tc)
            torch.autograd.grad([loss], [hc, wc])

        e["cpu_baseline"] = cpu_entry(step, work, "TFLOP/s", BT / rows, f"the first {rows} of the 16384 C5 rows "
                                      "(bf16 hidden @ weight.T [128256,4096], then F.cross_entropy, fwd+bwd), time "
                                      "scaled by 16384/128", True, min_reps=1)
    return e


def bench_flgrpo(K, dev, reps, flush):
    """FusedLinear-GRPO (no counterpart in the reference): C4's batch (B 16, L+1 1024, V 151936, beta 0.1)
    behind an H = 4096 bf16 lm_head, fwd+bwd."""
    from kernels import fused_linear_grpo as flg

    def logp_fn(h, w, ids):
        # lse from a no-grad pass of the op itself, the id logits by a gather
        _, _, _, _, _, rows = flg.fused_linear_grpo_forward(h, w, ids, torch.zeros(h.shape[0], device=dev),
                                                            compute_grad=False)
        return (h[:, :-1].float() * w[ids].float()).sum(-1) - rows[0]

    c = workloads.f3_fused_linear_grpo(logp_fn, device=dev)
    h = c["hidden"].requires_grad_(True)
    w = c["weight"].requires_grad_(True)
    args = [c[k] for k in ("completion_ids", "advantages", "old_logp", "ref_logp", "completion_mask", "temperature",
                           "beta", "eps_low", "eps_high")]
    B, T, H = h.shape
    V = w.shape[0]
    n_live = int(c["completion_mask"].sum())

    def run(budget):
        def fn():
            loss, _, _ = K.hilda_fused_linear_grpo_loss(h, w, *args, workspace_budget=budget)
            return torch.autograd.grad([loss], [h, w])
        return fn

    work = 6 * n_live * H * V  # conservative: masked tokens and position L need no FLOPs
    e = op_entry(f"fused_linear_grpo B={B} L+1={T} H={H} V={V} bf16 (workspace_budget='fastest')",
                 time_events(run("fastest"), reps, flush, warmup=1), work, "TFLOP/s", BF16_PEAK_TFLOPS)
    e["dense_equivalent_tflops"] = round(6 * B * T * H * V / (e["ms"] * 1e-3) / 1e12, 2)
    e["n_live_tokens"] = n_live
    d_ms = statistics.median(time_events(run(None), max(3, reps // 2), flush, warmup=1))
    e["default_plan"] = {"ms": round(d_ms, 3), "value": round(work / (d_ms * 1e-3) / 1e12, 2), "unit": "TFLOP/s"}
    e["peak_mib"] = {"fastest": peak_mib(run("fastest"), dev), "default": peak_mib(run(None), dev)}
    log(f"  fused_linear_grpo: fastest plan {e['ms']:.3f} ms  {e['value']:.1f} TFLOP/s  ({e['frac']:.1%}), peak "
        f"{e['peak_mib']['fastest']} MiB; default plan {d_ms:.3f} ms, peak {e['peak_mib']['default']} MiB")
    return e


# ---------------------------------------------------------------------------
# CPU baseline: the oracle (the reference's PyTorch path) on the host cores
# ---------------------------------------------------------------------------
def cpu_model_name():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return ""


def cpu_entry(step, work, unit, scale, sample, extrapolated, seconds=3.0, min_reps=2):
    """A config's CPU baseline: `step` (the oracle, the reference's PyTorch path, on a slice of the config's own
    inputs) on every host core, one warm-up, then repeated for `seconds` of CPU work (at least `min_reps`); the
    median time times `scale` (the config over the slice) against the config's whole algorithmic work."""
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    step()
    times = []
    while len(times) < min_reps or sum(times) < seconds:
        t0 = time.perf_counter()
        step()
        times.append(time.perf_counter() - t0)
    t = statistics.median(times) * scale
    rate = work / t / (1e9 if unit == "GB/s" else 1e12)
    log(f"    CPU: {rate:.3f} {unit} ({t:.3f} s for the config, {len(times)} reps)")
    return {"value": round(rate, 4), "unit": unit, "cores": cores, "kind": "port", "sample": sample,
            "extrapolated": extrapolated, "seconds_per_config": round(t, 4), "reps": len(times),
            "cpu_model": cpu_model_name()}


def cpu_baseline(seconds=10.0):
    """The oracle (the reference's PyTorch path) on the full C2 step, fwd+bwd, on every host core: one warm-up
    step, then whole steps until `seconds` of CPU work (at least 3); throughput over all of them."""
    import oracle

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    fa = workloads.c2_fused_add_rms_norm(device="cpu")
    rp = workloads.c2_rope(device="cpu")
    sw = workloads.c2_swiglu(device="cpu")
    x, r, w = (fa[k].clone().requires_grad_(True) for k in ("x", "r", "w"))
    q = rp["q"].detach().requires_grad_(True)
    k = rp["k"].detach().requires_grad_(True)
    a, b = (sw[n].clone().requires_grad_(True) for n in ("a", "b"))
    work = (bytes_fused_add(*x.shape) + bytes_rope(q.numel(), k.numel(), q.shape[2], q.shape[3])
            + bytes_swiglu(*a.shape))

    def step():
        y, s = oracle.fused_add_rms_norm_ref(x, r, w)
        torch.autograd.grad([y, s], [x, r, w], [fa["dy"], fa["ds"]])
        qo, ko = oracle.rope_ref(q, k, rp["cos"], rp["sin"])
        torch.autograd.grad([qo, ko], [q, k], [rp["dq"].float(), rp["dk"].float()])
        c = oracle.swiglu_ref(a, b)
        torch.autograd.grad([c], [a, b], [sw["dc"]])

    step()
    times = []
    while len(times) < 3 or sum(times) < seconds:
        t0 = time.perf_counter()
        step()
        times.append(time.perf_counter() - t0)
    t = sum(times) / len(times)
    cpu_model = cpu_model_name()
    return {"value": round(work / t / 1e9, 3), "unit": "GB/s", "cores": cores, "kind": "port",
            "sample": f"the full C2 step (FusedAddRMSNorm [8192,4096], RoPE q[4,2048,32,128] k[4,2048,8,128], "
                      f"SwiGLU [8192,14336]), bf16 PyTorch reference path fwd+bwd: {len(times)} steps in "
                      f"{sum(times):.1f} s after one warm-up step",
            "seconds_per_step": round(t, 4), "cpu_model": cpu_model}


def copy_ceiling(work, dev, reps, flush, row_bytes=None):
    """A device copy moving the same bytes (work/2 read, work/2 written), timed like the ops: the practical
    ceiling for an HBM-bound op (at a few GB it sits well below the 8 TB/s peak: read/write turnaround,
    refresh, open pages).

    The copy is the library's hand-written streaming kernel (hk_stream_copy): by default the flat order, the
    whole GPU sweeping one contiguous front (the fastest order measured, faster than hipMemcpy); with
    row_bytes, one row of that size per CU at a time in the order of the register-resident row kernels.
    Returns GB/s.
    """
    from kernels import _lib
    if row_bytes:
        rows = max(1, (work // 2) // row_bytes)
        n = rows * row_bytes
        mode = _lib.COPY_ROWS
    else:
        n = (work // 2 + 4095) // 4096 * 4096
        rows, mode = 1, _lib.COPY_FLAT
    src = torch.empty(n, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)
    st = _lib.stream_of(dev)

    def fn():
        _lib.call("hk_stream_copy", dst.data_ptr(), src.data_ptr(), rows, n // rows, mode, st)

    fn()
    torch.cuda.synchronize()
    if not torch.equal(dst, src):
        raise RuntimeError("hk_stream_copy produced a wrong copy")
    ms = statistics.median(time_events(fn, reps, flush))
    del src, dst
    torch.cuda.empty_cache()
    return 2 * n / (ms * 1e-3) / 1e9


# Each op's kernels as (streams read, streams written, bytes per stream), the large operands only: the byte
# mix the op's own kernels move, which HBM serves at its own rate (more reads than writes runs faster than a
# copy, eight read streams slower).
_C1 = 4096 * 4096 * 4
_C2 = 8192 * 4096 * 2
_SW = 8192 * 14336 * 2
_AR = 4 * 2048 * 4096 * 2
MIX_PATTERNS = {
    "rms_norm": [(1, 1, _C1), (2, 1, _C1)],                  # fwd x -> y; bwd dy, x -> dx
    "fused_add_rms_norm": [(2, 2, _C2), (3, 1, _C2)],        # fwd x, r -> y, s; bwd dy, dS, s -> dx
    "swiglu": [(2, 1, _SW), (3, 2, _SW)],                    # fwd a, b -> c; bwd a, b, dc -> da, db
    "geglu": [(2, 1, _SW), (3, 2, _SW)],
    "attn_res": [(8, 1, _AR), (9, 8, _AR)],                  # fwd 8 blocks -> h; bwd 8 blocks, dh -> 8 dV
    "jsd": [(2, 1, 8192 * 128256 * 2)],                      # X, Y -> dX
}


MIX_PAD = 4352  # bytes between streams beyond their length: 64 MiB-spaced streams ran up to 8% slower


def mix_ceiling(parts, dev, reps, flush):
    """hk_stream_mix over every (reads, writes, bytes) part, the parts launched back to back in one timed call
    as an op's kernels are (each part on buffers of its own, streams MIX_PAD bytes apart), timed like the ops;
    median ms."""
    from kernels import _lib
    st = _lib.stream_of(dev)
    bufs = [(torch.empty(r * (nbytes + MIX_PAD), dtype=torch.uint8, device=dev).fill_(1),
             torch.empty(w * (nbytes + MIX_PAD), dtype=torch.uint8, device=dev), r, w, nbytes) for r, w, nbytes in parts]

    def fn():
        for src, dst, r, w, nbytes in bufs:
            _lib.call("hk_stream_mix", dst.data_ptr(), src.data_ptr(), nbytes, nbytes + MIX_PAD, r, w, st)

    fn()
    torch.cuda.synchronize()
    for src, dst, r, w, nbytes in bufs:
        expect = (0x01010101 if r % 2 else 0) + w - 1  # every word of the last stream
        last = (w - 1) * (nbytes + MIX_PAD) + nbytes
        if int(dst[last - 4:last].view(torch.int32).item()) != expect:
            raise RuntimeError("hk_stream_mix produced a wrong result")
    ms = statistics.median(time_events(fn, reps, flush))
    del bufs
    torch.cuda.empty_cache()
    return ms


def attach_copy(e, dev, reps, flush, name=None):
    """e["copy_same_bytes"] (flat copy) and, for the row kernels' entries (e["row_bytes"]),
    e["copy_rows_same_bytes"]: the op against copies of its own bytes; for the ops in MIX_PATTERNS,
    e["mix_same_pattern"]: against streaming kernels of its own kernels' read/write mix."""
    cc = copy_ceiling(e["work"], dev, reps, flush)
    e["copy_same_bytes"] = {"value": round(cc, 1), "unit": "GB/s", "op_over_copy": round(e["value"] / cc, 3),
                            "kernel": "hk_stream_copy flat"}
    if e.get("row_bytes"):
        cr = copy_ceiling(e["work"], dev, reps, flush, e["row_bytes"])
        e["copy_rows_same_bytes"] = {"value": round(cr, 1), "unit": "GB/s", "op_over_copy": round(e["value"] / cr, 3),
                                     "kernel": "hk_stream_copy rows of %d bytes" % e["row_bytes"]}
    if name in MIX_PATTERNS:
        t = mix_ceiling(MIX_PATTERNS[name], dev, reps, flush)
        e["mix_same_pattern"] = {"ms": round(t, 5), "value": round(e["work"] / (t * 1e-3) / 1e9, 1), "unit": "GB/s",
                                 "op_over_mix": round(t / e["ms"], 3),
                                 "streams": ["%dR%dW x %d MB" % (r, w, b >> 20) for r, w, b in MIX_PATTERNS[name]],
                                 "kernel": "hk_stream_mix"}
    return e


# ---------------------------------------------------------------------------
# the reference's own benchmark shapes, each op against a copy of its bytes
# ---------------------------------------------------------------------------
def dw_sweep(dev, reps):
    """RMSNorm backward with the weight gradient by fp64 atomics on one row against fp32 partial rows summed in a
    second pass, over rows x H, fp32 and bf16: the sweep behind HK_DW_AUTO's choice (the reference switches to
    atomics when rows <= 8 x CU count, rms_norm.py:325-326). Median call time with a cache flush between calls, as
    a markdown table on stdout."""
    from kernels import rms_norm as rn, _lib
    flush = Flusher(dev)
    cu = torch.cuda.get_device_properties(dev).multi_processor_count
    gen = torch.Generator(device=dev).manual_seed(0)
    print(f"| dtype | rows | H | partial rows (us) | fp64 atomics (us) | atomics / partial |")
    print("|---|---|---|---|---|---|")
    for dt in (torch.float32, torch.bfloat16):
        for H in (1024, 4096, 8192):
            for rows in sorted({16, 64, 256, 1024, 2048, 8 * cu, 16384}):
                x = torch.randn(rows, H, generator=gen, device=dev).to(dt)
                w = torch.randn(H, generator=gen, device=dev).to(dt)
                dy = torch.randn(rows, H, generator=gen, device=dev).to(dt)
                _, xf, rs = rn.rms_norm_forward(x, w)
                t = {}
                for mode in (_lib.DW_PARTIAL, _lib.DW_ATOMIC):
                    t[mode] = statistics.median(time_events(lambda: rn.rms_norm_backward(dy, xf, w, rs, mode), reps,
                                                            flush)) * 1e3
                print(f"| {str(dt).split('.')[-1]} | {rows} | {H} | {t[_lib.DW_PARTIAL]:.1f} | {t[_lib.DW_ATOMIC]:.1f} "
                      f"| {t[_lib.DW_ATOMIC] / t[_lib.DW_PARTIAL]:.2f} |", flush=True)
                del x, w, dy, xf, rs


# The shapes the reference's benchmarks time (triton-kernels/benchmarks/), shared by --reference-configs and
# --vs-torch; dtypes by name (torch.float16 / torch.bfloat16).
REF_SHAPES = {
    "rms_norm": ((4, 512, 4096, "float16"), (8, 1024, 4096, "float16"), (4, 2048, 4096, "float16"),
                 (8, 2048, 4096, "float16"), (4, 1024, 8192, "float16"), (4, 1024, 4096, "bfloat16")),  # :169-177
    "fused_add_rms_norm": ((4, 2048, 4096, "float16"), (4, 2048, 5120, "float16"), (4, 2048, 8192, "float16"),
                           (4, 2048, 4096, "bfloat16"), (2, 1024, 4096, "float16")),  # :198-204
    "rope": ((4, 2048, 32, 8, 128, "float16"), (4, 2048, 32, 32, 128, "float16"), (4, 2048, 64, 8, 128, "float16"),
             (8, 2048, 32, 8, 128, "float16"), (4, 2048, 32, 8, 128, "bfloat16"),
             (4, 512, 32, 8, 128, "float16")),  # :263-271
    "glu": ((8192, 11008, "float16"), (8192, 14336, "float16"), (8192, 28672, "float16"), (8192, 14336, "bfloat16"),
            (2048, 14336, "float16")),  # bench_swiglu.py:196-203, bench_geglu.py:191-198
    "cross_entropy": ((8192, 32000, "float16"), (8192, 128256, "float16"), (8192, 32000, "bfloat16"),
                      (8192, 128256, "bfloat16"), (2048, 32000, "float16")),  # :257-264
    "grpo": ((8, 512, 32000, 0.0), (8, 512, 32000, 0.1), (4, 1024, 32000, 0.0), (4, 512, 128256, 0.0)),  # :204-209
    "kl_div": ((8192, 32000, "float16"), (8192, 128256, "float16"), (8192, 32000, "bfloat16"),
               (2048, 32000, "float16")),  # :156-161
    "jsd": ((8192, 32000, "float16"), (4096, 128256, "float16"), (8192, 32000, "bfloat16")),  # :173-177
    "attn_res": ((4, 4096, "float16"), (8, 4096, "float16"), (8, 8192, "float16"), (16, 4096, "float16"),
                 (8, 4096, "bfloat16")),  # :205-211, B 4, T 2048
}


def _dt(name):
    return getattr(torch, name)


def reference_configs(dev, reps):
    """Every HBM-bound op on the shapes the reference's benchmarks time, fwd and bwd separately, with the
    algorithmic bytes of each call over a device copy of the same bytes; the fused-linear ops in TFLOP/s.
    Prints a markdown table. Shapes from triton-kernels/benchmarks: bench_rms_norm.py:169,
    bench_fused_add_rms_norm.py:198, bench_rope.py:263, bench_swiglu.py:196, bench_geglu.py:191,
    bench_cross_entropy.py:257, bench_grpo.py:204, bench_kl_div.py:156, bench_jsd.py:173,
    bench_attn_res.py:205, bench_fused_linear_ce.py:245, bench_fused_linear_jsd.py:163."""
    from kernels import (rms_norm as rn, fused_add_rms_norm as fa, rope, swiglu as sw, geglu as gg,
                         cross_entropy as ce, grpo_loss as gl, kl_div as kl, jsd as js, attn_res as ar,
                         fused_linear_cross_entropy as flce, fused_linear_jsd as fljsd)
    flush = Flusher(dev)
    F16, BF16, F32 = torch.float16, torch.bfloat16, torch.float32
    gen = torch.Generator(device=dev).manual_seed(0)
    rnd = lambda *shape, dt=F32: torch.randn(*shape, generator=gen, device=dev).to(dt)  # noqa: E731
    dname = {F16: "fp16", BF16: "bf16", F32: "fp32"}
    rows = []

    def hbm(op, shape, dt, fn, nbytes):
        ms = statistics.median(time_events(fn, reps, flush))
        cc = copy_ceiling(nbytes, dev, reps, flush)
        gbs = nbytes / (ms * 1e-3) / 1e9
        rows.append(f"| {op} | {shape} | {dname[dt]} | {ms * 1e3:.1f} us | {gbs:.0f} GB/s | {cc:.0f} GB/s | "
                    f"{gbs / cc:.0%} |")
        log(rows[-1])

    for B, T, H, dt in REF_SHAPES["rms_norm"]:
        dt = _dt(dt)
        R, es = B * T, torch.tensor([], dtype=dt).element_size()
        x, w, dy = rnd(R, H, dt=dt), rnd(H, dt=dt), rnd(R, H, dt=dt)
        _, xf, rs = rn.rms_norm_forward(x, w)
        hbm("RMSNorm fwd", f"{B}x{T}x{H}", dt, lambda: rn.rms_norm_forward(x, w), 2 * R * H * es)
        hbm("RMSNorm bwd", f"{B}x{T}x{H}", dt, lambda: rn.rms_norm_backward(dy, xf, w, rs), 3 * R * H * es)
        del x, dy, xf
    for B, T, H, dt in REF_SHAPES["fused_add_rms_norm"]:
        dt = _dt(dt)
        R, es = B * T, torch.tensor([], dtype=dt).element_size()
        x, r, w, dy, ds = rnd(R, H, dt=dt), rnd(R, H, dt=dt), rnd(H, dt=dt), rnd(R, H, dt=dt), rnd(R, H, dt=dt)
        _, s_, rs = fa.fused_add_rms_norm_forward(x, r, w)
        hbm("FusedAddRMSNorm fwd", f"{B}x{T}x{H}", dt, lambda: fa.fused_add_rms_norm_forward(x, r, w), 4 * R * H * es)
        hbm("FusedAddRMSNorm bwd", f"{B}x{T}x{H}", dt, lambda: fa.fused_add_rms_norm_backward(dy, ds, s_, w, rs),
            4 * R * H * es)
        del x, r, dy, ds, s_
    for B, T, nq, nk, hd, dt in REF_SHAPES["rope"]:
        dt = _dt(dt)
        q, k = rnd(B, nq, T, hd, dt=dt), rnd(B, nk, T, hd, dt=dt)
        cos, sin = rnd(1, T, hd // 2, dt=dt), rnd(1, T, hd // 2, dt=dt)
        nb = 2 * (q.numel() + k.numel()) * q.element_size()
        hbm("RoPE fwd", f"{B}x{T} q{nq} k{nk}", dt, lambda: rope.rope_forward(q, k, cos, sin), nb)
        hbm("RoPE bwd", f"{B}x{T} q{nq} k{nk}", dt, lambda: rope.rope_backward(q, k, cos, sin), nb)
        del q, k
    for name, mod in (("SwiGLU", sw), ("GeGLU", gg)):
        fwd = mod.swiglu_forward if mod is sw else mod.geglu_forward
        bwd = mod.swiglu_backward if mod is sw else mod.geglu_backward
        for N, D, dt in REF_SHAPES["glu"]:
            dt = _dt(dt)
            a, b, dc = rnd(N, D, dt=dt), rnd(N, D, dt=dt), rnd(N, D, dt=dt)
            hbm(f"{name} fwd", f"{N}x{D}", dt, lambda: fwd(a, b), 3 * N * D * 2)
            hbm(f"{name} bwd", f"{N}x{D}", dt, lambda: bwd(a, b, dc), 5 * N * D * 2)
            del a, b, dc
    for N, V, dt in REF_SHAPES["cross_entropy"]:
        dt = _dt(dt)
        x = rnd(N, V, dt=dt)
        t = torch.randint(0, V, (N,), generator=gen, device=dev)
        es = x.element_size()
        hbm("CrossEntropy fwd+grad", f"{N}x{V}", dt, lambda: ce.cross_entropy_forward(x, t, needs_grad=True),
            2 * N * V * es)
        hbm("CrossEntropy fwd", f"{N}x{V}", dt, lambda: ce.cross_entropy_forward(x, t), N * V * es)
        del x
    for B, L, V, beta in REF_SHAPES["grpo"]:
        x = rnd(B, L + 1, V, dt=BF16)
        ids = torch.randint(0, V, (B, L), generator=gen, device=dev)
        adv, old, ref = rnd(B), rnd(B, L) - 5, rnd(B, L) - 5
        mask = torch.ones(B, L, dtype=torch.int32, device=dev)
        kw = dict(old_logp=old, ref_logp=ref if beta else None, completion_mask=mask, beta=beta)
        nb = B * L * V * 2
        hbm("GRPO fwd+grad", f"{B}x{L}x{V} beta {beta}", BF16,
            lambda: gl.grpo_loss_forward(x, ids, adv, compute_grad=True, **kw), 2 * nb)
        hbm("GRPO fwd", f"{B}x{L}x{V} beta {beta}", BF16, lambda: gl.grpo_loss_forward(x, ids, adv, **kw), nb)
        hbm("selective log-softmax", f"{B}x{L}x{V}", BF16,
            lambda: gl.fused_selective_log_softmax(x, ids, 1.0, mask), nb)
        del x
    for N, V, dt in REF_SHAPES["kl_div"]:
        dt = _dt(dt)
        yp, yt = rnd(N, V).log_softmax(-1).to(dt), rnd(N, V).softmax(-1).to(dt)
        g1 = torch.ones((), device=dev)
        es = yp.element_size()
        hbm("KLDiv fwd", f"{N}x{V}", dt, lambda: kl.kl_div_forward(yp, yt), 2 * N * V * es)
        hbm("KLDiv bwd", f"{N}x{V}", dt, lambda: kl.kl_div_backward(yt, g1), 2 * N * V * es)
        del yp, yt
    for N, V, dt in REF_SHAPES["jsd"]:
        dt = _dt(dt)
        X, Y = rnd(N, V).log_softmax(-1).to(dt), rnd(N, V).log_softmax(-1).to(dt)
        hbm("JSD fwd+grad", f"{N}x{V}", dt, lambda: js.jsd_forward(X, Y, 0.5), 3 * N * V * X.element_size())
        del X, Y
    for n, D, dt in REF_SHAPES["attn_res"]:
        dt = _dt(dt)
        ntok = 4 * 2048
        Vb, wq, wn, dh = rnd(n, ntok, D, dt=dt), (0.02 * rnd(D)).to(dt), rnd(D, dt=dt), rnd(ntok, D, dt=dt)
        _, V3, alpha, rs = ar.attn_res_forward(Vb, wq, wn)
        hbm("AttnRes fwd", f"N {n}, 4x2048x{D}", dt, lambda: ar.attn_res_forward(Vb, wq, wn), (n + 1) * ntok * D * 2)
        hbm("AttnRes bwd", f"N {n}, 4x2048x{D}", dt, lambda: ar.attn_res_backward(dh, V3, wq, wn, alpha, rs),
            (2 * n + 1) * ntok * D * 2)
        del Vb, dh, V3
    mm = []
    for N, H, V, dt in ((8192, 4096, 32000, F16), (8192, 4096, 128256, F16), (8192, 4096, 32000, BF16),
                        (2048, 4096, 32000, F16)):
        x, w = (0.5 * rnd(N, H)).to(dt), (0.02 * rnd(V, H)).to(dt)
        t = torch.randint(0, V, (N,), generator=gen, device=dev)
        cells = []
        for budget in (None, "fastest"):
            ms = statistics.median(time_events(
                lambda: flce.fused_linear_cross_entropy_forward(x, w, t, workspace_budget=budget), 4, flush))
            tf = 6 * N * H * V / (ms * 1e-3) / 1e12
            cells.append(f"{ms:.2f} ms, {tf:.0f} TFLOP/s ({tf / BF16_PEAK_TFLOPS:.1%})")
        mm.append(f"| FusedLinearCE fwd+grad | {N}x{H}x{V} | {dname[dt]} | {cells[0]} | {cells[1]} |")
        log(mm[-1])
        del x, w
    for N, H, V, dt in ((4096, 4096, 32000, F16), (2048, 4096, 128256, F16), (4096, 4096, 32000, BF16)):
        xs, xt = (0.5 * rnd(N, H)).to(dt), (0.5 * rnd(N, H)).to(dt)
        ws, wt = (0.02 * rnd(V, H)).to(dt), (0.02 * rnd(V, H)).to(dt)
        cells = []
        for budget in (None, "fastest"):
            ms = statistics.median(time_events(
                lambda: fljsd.fused_linear_jsd_forward(xs, ws, xt, wt, workspace_budget=budget), 4, flush))
            tf = 8 * N * H * V / (ms * 1e-3) / 1e12
            cells.append(f"{ms:.2f} ms, {tf:.0f} TFLOP/s ({tf / BF16_PEAK_TFLOPS:.1%})")
        mm.append(f"| FusedLinearJSD fwd+grad | {N}x{H}x{V} | {dname[dt]} | {cells[0]} | {cells[1]} |")
        log(mm[-1])
        del xs, ws, xt, wt
    print("| Op | Shape | dtype | Time | Achieved | Copy of the same bytes | Op / copy |")
    print("|---|---|---|---|---|---|---|")
    print("\n".join(rows))
    print()
    print("| Op | Shape | dtype | default workspace budget | `'fastest'` (no limit) |")
    print("|---|---|---|---|---|")
    print("\n".join(mm))


def vs_torch(dev, reps):
    """The reference's published metric (README.md:13-49: fwd+bwd speedup over PyTorch eager, RoPE forward only) on
    this GPU: each op through the library's autograd API against the PyTorch baseline of the reference's own
    benchmark (the bench_*.py line each row cites), on the same shapes and inputs. The reference's lambdas draw
    their inputs with torch.randn inside the timed region; here the inputs are resident, upstream gradients random
    and each rep starts after a cache flush, so the ratio is of the ops alone. Prints a markdown table."""
    import kernels as K
    flush = Flusher(dev)
    F = torch.nn.functional
    gen = torch.Generator(device=dev).manual_seed(0)
    rnd = lambda *shape, dt=torch.float32: torch.randn(*shape, generator=gen, device=dev).to(dt)  # noqa: E731
    dname = {torch.float16: "fp16", torch.bfloat16: "bf16"}
    rows = []

    def pair(op, shape, dt, claim, base, ours, wrt, fwd_only=False):
        """base, ours: () -> output tensor or tuple; wrt: the tensors whose gradients both compute."""
        def run(f):
            if fwd_only:
                def fn():
                    with torch.no_grad():
                        return f()
                return fn
            outs = f()
            outs = outs if isinstance(outs, tuple) else (outs,)
            outs = [o for o in outs if o is not None and o.requires_grad]
            g = [None if o.dim() == 0 else torch.randn(o.shape, generator=gen, device=dev).to(o.dtype) for o in outs]
            del outs

            def fn():
                o = f()
                o = o if isinstance(o, tuple) else (o,)
                o = [t for t in o if t is not None and t.requires_grad]
                return torch.autograd.grad(o, wrt, g)
            return fn
        tb = statistics.median(time_events(run(base), reps, flush, warmup=2))
        to = statistics.median(time_events(run(ours), reps, flush, warmup=2))
        rows.append(f"| {op} | {shape} | {dname[dt]} | {tb * 1e3:.1f} us | {to * 1e3:.1f} us | {tb / to:.2f}x | "
                    f"{claim} |")
        log(rows[-1])

    def t_rms(x, w, eps=1e-6):  # bench_rms_norm.py:37-41 (its output promotes to fp32, as there)
        return x * torch.rsqrt(x.float().pow(2).mean(-1, keepdim=True) + eps) * w

    def t_fadd(x, r, w, eps=1e-6):  # bench_fused_add_rms_norm.py:37-41
        s_ = x + r
        rms = torch.sqrt(torch.mean(s_.float() ** 2, dim=-1, keepdim=True) + eps)
        return (s_.float() / rms).to(s_.dtype) * w, s_

    def t_rope(q, k, cos, sin):  # bench_rope.py:40-59 (HuggingFace rotate-half)
        c = torch.cat([cos, cos], dim=-1).unsqueeze(1)
        s_ = torch.cat([sin, sin], dim=-1).unsqueeze(1)

        def rot(x):
            h = x.shape[-1] // 2
            return torch.cat((-x[..., h:], x[..., :h]), dim=-1)
        return q * c + rot(q) * s_, k * c + rot(k) * s_

    def t_grpo(logits, ids, adv, old, ref, beta, eps=0.2):  # bench_grpo.py:30-57, on logits.float() (:157)
        L = logits.shape[1] - 1
        logp = logits[:, :-1, :].log_softmax(dim=-1).gather(-1, ids[:, -L:].unsqueeze(-1)).squeeze(-1)
        ratio = torch.exp(logp - old)
        a = adv.unsqueeze(-1)
        per_token = -torch.min(ratio * a, torch.clamp(ratio, 1 - eps, 1 + eps) * a)
        if beta != 0.0:
            per_token = per_token + beta * (torch.exp(ref - logp) - (ref - logp) - 1)
        mask = torch.ones_like(per_token)
        return ((per_token * mask).sum(-1) / mask.sum(-1).clamp(min=1.0)).mean()

    def t_jsd(x, y, beta=0.5):  # bench_jsd.py:30-45, on fp32 copies (:129)
        q, p = x.exp(), y.exp()
        log_m = (beta * p + (1 - beta) * q).log()
        return (beta * (p * (y - log_m)).sum(-1) + (1 - beta) * (q * (x - log_m)).sum(-1)).mean()

    def t_attn_res(v, wq, wn, eps=1e-6):  # bench_attn_res.py:33-51; its einsums as fp32 matmuls on contiguous operands
        vf = v.float()
        k = (vf / torch.sqrt(vf.pow(2).mean(dim=-1, keepdim=True) + eps)).to(v.dtype) * wn
        alpha = torch.matmul(k.float(), wq.float()).softmax(dim=0)  # [N, B, T]
        h = torch.matmul(alpha.permute(1, 2, 0).unsqueeze(-2).contiguous(), vf.permute(1, 2, 0, 3).contiguous())
        return h.squeeze(-2).to(v.dtype)

    for B, T, H, dt in REF_SHAPES["rms_norm"]:
        dt = _dt(dt)
        x, w = rnd(B, T, H, dt=dt).requires_grad_(True), torch.ones(H, device=dev, dtype=dt, requires_grad=True)
        pair("RMSNorm fwd+bwd", f"{B}x{T}x{H}", dt, "1.18-8.21x", lambda: t_rms(x, w), lambda: K.hilda_rms_norm(x, w),
             [x, w])
        del x
    for B, T, H, dt in REF_SHAPES["fused_add_rms_norm"]:
        dt = _dt(dt)
        x, r = rnd(B, T, H, dt=dt).requires_grad_(True), rnd(B, T, H, dt=dt).requires_grad_(True)
        w = torch.ones(H, device=dev, dtype=dt)
        pair("FusedAddRMSNorm fwd+bwd", f"{B}x{T}x{H}", dt, "4.15-5.66x", lambda: t_fadd(x, r, w),
             lambda: K.hilda_fused_add_rms_norm(x, r, w), [x, r])
        del x, r
    for B, T, nq, nk, hd, dt in REF_SHAPES["rope"]:
        dt = _dt(dt)
        q, k = rnd(B, nq, T, hd, dt=dt).requires_grad_(True), rnd(B, nk, T, hd, dt=dt).requires_grad_(True)
        cos, sin = rnd(1, T, hd // 2, dt=dt), rnd(1, T, hd // 2, dt=dt)
        pair("RoPE fwd", f"{B}x{T} q{nq} k{nk}", dt, "1.27-1.34x", lambda: t_rope(q, k, cos, sin),
             lambda: K.hilda_rope(q, k, cos, sin), [q, k], fwd_only=True)
        pair("RoPE fwd+bwd", f"{B}x{T} q{nq} k{nk}", dt, "-", lambda: t_rope(q, k, cos, sin),
             lambda: K.hilda_rope(q, k, cos, sin), [q, k])
        del q, k
    for name, base, ours, claim in (("SwiGLU", lambda a, b: F.silu(a) * b, K.hilda_swiglu, "1.26-1.68x"),
                                    ("GeGLU", lambda a, b: F.gelu(a, approximate="tanh") * b, K.hilda_geglu,
                                     "1.25-1.68x")):
        for N, D, dt in REF_SHAPES["glu"]:  # bench_swiglu.py:46-47, bench_geglu.py:42-43
            dt = _dt(dt)
            a, b = rnd(N, D, dt=dt).requires_grad_(True), rnd(N, D, dt=dt).requires_grad_(True)
            pair(f"{name} fwd+bwd", f"{N}x{D}", dt, claim, lambda: base(a, b), lambda: ours(a, b), [a, b])
            del a, b
    for N, V, dt in REF_SHAPES["cross_entropy"]:  # bench_cross_entropy.py:217-228, 10% ignored
        dt = _dt(dt)
        x = rnd(N, V, dt=dt).requires_grad_(True)
        t = torch.randint(0, V, (N,), generator=gen, device=dev)
        t[torch.rand(N, generator=gen, device=dev) < 0.1] = -100
        pair("CrossEntropy fwd+bwd", f"{N}x{V}", dt, "1.66-2.55x", lambda: F.cross_entropy(x, t, ignore_index=-100),
             lambda: K.hilda_cross_entropy(x, t), [x])
        del x
    for B, L, V, beta in REF_SHAPES["grpo"]:  # bench_grpo.py:150-166, bf16 logits
        x = (0.1 * rnd(B, L + 1, V)).to(torch.bfloat16).requires_grad_(True)
        ids = torch.randint(0, V, (B, L), generator=gen, device=dev)
        adv, old = rnd(B), 0.01 * rnd(B, L)
        # with beta != 0 both get reference log-probs: the reference's bench passes none (its kernel then reads a
        # one-element dummy at every token's offset, grpo_loss.py:150-153,277), which this library rejects
        ref = old + 0.1 * rnd(B, L) if beta else None
        pair("GRPO fwd+bwd", f"{B}x{L}x{V} beta {beta}", torch.bfloat16, "6.10-6.61x",
             lambda: t_grpo(x.float(), ids, adv, old, ref, beta),
             lambda: K.hilda_grpo_loss(x, ids, adv, old, ref, beta=beta)[0], [x])
        del x
    for N, V, dt in REF_SHAPES["kl_div"]:  # bench_kl_div.py:108-116
        dt = _dt(dt)
        yp = rnd(N, V, dt=dt).log_softmax(dim=-1).requires_grad_(True)
        yt = rnd(N, V, dt=dt).softmax(dim=-1)
        pair("KLDiv fwd+bwd", f"{N}x{V}", dt, "1.71-1.84x", lambda: F.kl_div(yp, yt, reduction="batchmean"),
             lambda: K.hilda_kl_div(yp, yt, reduction="batchmean"), [yp])
        del yp, yt
    for N, V, dt in REF_SHAPES["jsd"]:  # bench_jsd.py:124-132
        dt = _dt(dt)
        xj = rnd(N, V, dt=dt).log_softmax(dim=-1).requires_grad_(True)
        yj = rnd(N, V, dt=dt).log_softmax(dim=-1)
        pair("JSD fwd+bwd", f"{N}x{V}", dt, "9.18-11.02x", lambda: t_jsd(xj.float(), yj.float()),
             lambda: K.hilda_jsd(xj, yj, beta=0.5), [xj])
        del xj, yj
    for n, D, dt in REF_SHAPES["attn_res"]:  # bench_attn_res.py:168-181
        dt = _dt(dt)
        v = rnd(n, 4, 2048, D, dt=dt).requires_grad_(True)
        wq, wn = (0.02 * rnd(D)).to(dt), torch.ones(D, device=dev, dtype=dt)
        pair("AttnRes fwd+bwd", f"N {n}, 4x2048x{D}", dt, "20.55-24.01x", lambda: t_attn_res(v, wq, wn),
             lambda: K.hilda_attn_res(v, wq, wn), [v])
        del v
    print("| Op | Shape | dtype | PyTorch eager | this library | speedup | reference's claim (RTX 5090) |")
    print("|---|---|---|---|---|---|---|")
    print("\n".join(rows))


C2_OPS = ("fused_add_rms_norm", "rope", "swiglu")


def op_table():
    """(name, (bench function, full reps)) of the per-op entries after the C2 ops; the large-vocabulary ops run
    half the reps."""
    return (("rms_norm", (bench_c1, True)), ("geglu", (bench_geglu, True)), ("attn_res", (bench_attn_res, True)),
            ("cross_entropy", (bench_c3, False)), ("grpo_loss", (bench_c4, False)),
            ("fused_linear_cross_entropy", (bench_c5, False)), ("kl_div", (bench_kl_div, False)),
            ("jsd", (bench_jsd, False)), ("fused_linear_jsd", (bench_fljsd, False)),
            ("fused_linear_grpo", (bench_flgrpo, False)))


def load_traffic(kernel):
    """HBM bytes per launch from the committed rocprofv3 --pmc summary, if present."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            data = json.load(f)
        e = data["kernels"][kernel]
        return int(e["hbm_bytes_per_launch"])
    except (OSError, KeyError, ValueError):
        return None


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--ops", default="all",
                    help="all | c2 | none | a comma list of op names (e.g. attn_res,jsd) after the C2 ops")
    ap.add_argument("--op-reps", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="finish with three plain 1 GiB device-to-device copies (reference kernel of known "
                         "traffic for rocprofv3 FETCH_SIZE/WRITE_SIZE scaling)")
    ap.add_argument("--dw-sweep", action="store_true",
                    help="instead of the step: RMSNorm backward, dW by fp64 atomics against partial rows over rows x H, "
                         "as a markdown table")
    ap.add_argument("--vs-torch", action="store_true",
                    help="instead of the step: every op's fwd+bwd against the reference benchmarks' PyTorch "
                         "baselines on their shapes, the reference's published speedup metric, as a markdown table")
    ap.add_argument("--reference-configs", action="store_true",
                    help="instead of the step: every op on the reference benchmarks' own shapes, as a markdown table")
    ap.add_argument("--only-copy", action="store_true",
                    help="with --only: after each op, a device copy of the same bytes timed the same way (its "
                         "copyBuffer launches sit beside the op's kernels in a rocprofv3 trace)")
    ap.add_argument("--only", default=None,
                    help="comma list of op names: time only these (op-reps each, cache flushed between reps), with "
                         "no C2 headline step, copy ceilings or CPU baseline, and print their entries as JSON; "
                         "the command the per-config rocprofv3 summaries in profiles/ are taken from. copy_1g alone: "
                         "three 1 GiB device copies (the counter calibration)")
    args = ap.parse_args(argv)

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(run with --gpus 1)", file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 2

    import kernels as K
    from kernels import swiglu as swiglu_mod

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.reference_configs:
        reference_configs(dev, max(3, args.op_reps // 2))
        return 0
    if args.vs_torch:
        vs_torch(dev, max(3, args.op_reps // 2))
        return 0
    if args.dw_sweep:
        dw_sweep(dev, args.op_reps)
        return 0
    if args.only:
        table = dict(op_table())
        names = args.only.split(",")
        if names == ["copy_1g"]:
            # the counter calibration alone: three plain 1 GiB device-to-device copies
            src = torch.empty(1 << 30, dtype=torch.uint8, device=dev).fill_(1)
            dst = torch.empty_like(src)
            for _ in range(3):
                dst.copy_(src)
            torch.cuda.synchronize()
            return 0
        unknown = set(names) - set(table) - set(C2_OPS)
        if unknown:
            raise SystemExit(f"unknown op(s) {sorted(unknown)}; known: {sorted(table)}")
        flush = Flusher(dev)
        c2 = C2Step(K, dev) if any(n in C2_OPS for n in names) else None
        out = {}
        for name in names:
            if name in C2_OPS:
                fn = {"fused_add_rms_norm": c2.fused_add, "rope": c2.rope, "swiglu": c2.swiglu}[name]
                out[name] = op_entry("C2", time_events(fn, args.op_reps, flush), c2.bytes[name], "GB/s",
                                     HBM_PEAK_GBPS)
            else:
                out[name] = table[name][0](K, dev, args.op_reps, flush)
            torch.cuda.empty_cache()
            if args.only_copy and out[name].get("unit") == "GB/s":
                attach_copy(out[name], dev, args.op_reps, flush, name)
        print(json.dumps(out), flush=True)
        return 0
    log(f"device: {torch.cuda.get_device_name(dev)}")
    c2 = C2Step(K, dev)

    # fence-free HIP events around every SwiGLU backward launch inside the timed region (torch's default events
    # write back and invalidate L2 at each record: 5.7 us a step against 2.3 us for these)
    sw_events = []
    recording = {"on": False}
    orig_bwd = swiglu_mod.swiglu_backward

    def timed_bwd(a, b, dc):
        if not recording["on"]:
            return orig_bwd(a, b, dc)
        s, e = TimingEvent(), TimingEvent()
        s.record(torch.cuda.current_stream(a.device))
        out = orig_bwd(a, b, dc)
        e.record(torch.cuda.current_stream(a.device))
        sw_events.append((s, e))
        return out

    swiglu_mod.swiglu_backward = timed_bwd

    for _ in range(args.warmup):
        c2.step()
    torch.cuda.synchronize()
    recording["on"] = True
    t0 = time.perf_counter()
    for _ in range(args.steps):
        c2.step()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    recording["on"] = False
    swiglu_mod.swiglu_backward = orig_bwd

    ms_per_step = (t1 - t0) * 1e3 / args.steps
    total_bytes = c2.total_bytes()
    value = total_bytes / (ms_per_step * 1e-3) / 1e9

    # the same step captured once in a HIP graph and replayed (the library allocates and
    # synchronises nothing, so the whole fwd+bwd step is capturable): launch gaps removed
    graph = None
    try:
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(2):
                c2.step()
        torch.cuda.current_stream().wait_stream(side)
        cg = torch.cuda.CUDAGraph()
        with torch.cuda.graph(cg):
            c2.step()
        for _ in range(args.warmup):
            cg.replay()
        torch.cuda.synchronize()
        g0 = time.perf_counter()
        for _ in range(args.steps):
            cg.replay()
        torch.cuda.synchronize()
        g_ms = (time.perf_counter() - g0) * 1e3 / args.steps
        graph = {"ms_per_step": round(g_ms, 5), "value": round(total_bytes / (g_ms * 1e-3) / 1e9, 2),
                 "unit": "GB/s", "note": "the same C2 step replayed from one HIP graph capture"}
        log(f"C2 step as a HIP graph: {g_ms:.4f} ms/step, {graph['value']:.0f} GB/s")
        del cg
    except Exception as exc:  # reported, not fatal: the eager step is the headline
        log(f"C2 graph replay unavailable: {exc}")
    sw_ms = statistics.mean(s.elapsed_time(e) for s, e in sw_events)
    achieved = c2.swiglu_bwd_bytes / (sw_ms * 1e-3) / 1e9
    log(f"C2 step: {ms_per_step:.4f} ms/step, {value:.0f} GB/s; swiglu bwd {sw_ms * 1e3:.1f} us "
        f"-> {achieved:.0f} GB/s")

    roofline = {"bound": "hbm", "kernel": "swiglu_bwd_kernel", "achieved": round(achieved, 1),
                "peak": HBM_PEAK_GBPS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4),
                "traffic": load_traffic("swiglu_bwd_kernel"),
                "algorithmic_bytes_per_launch": c2.swiglu_bwd_bytes, "avg_launch_us": round(sw_ms * 1e3, 2),
                "launches": len(sw_events)}

    ops = {}
    if args.ops != "none":
        flush = Flusher(dev)
        log("per-op fwd+bwd (median, cache flushed between reps):")
        ops.update(bench_c2_ops(c2, args.op_reps, flush))
        table = op_table()
        wanted = [n for n, _ in table] if args.ops == "all" else \
            [] if args.ops == "c2" else args.ops.split(",")
        unknown = set(wanted) - {n for n, _ in table}
        if unknown:
            raise SystemExit(f"unknown op(s) {sorted(unknown)}; known: {[n for n, _ in table]}")
        del c2
        torch.cuda.empty_cache()
        c2 = None
        for name, (fn, full) in table:
            if name in wanted:
                reps = args.op_reps if full else max(3, args.op_reps // 2)
                if fn in (bench_c1, bench_c3, bench_c4, bench_c5):
                    # the config's own CPU baseline (a slice of the same inputs, scaled) unless --no-cpu
                    ops[name] = fn(K, dev, reps, flush, cpu=not args.no_cpu)
                else:
                    ops[name] = fn(K, dev, reps, flush)
                torch.cuda.empty_cache()
        log("device copy of the same bytes (practical HBM ceiling per op):")
        for name, e in ops.items():
            if e["unit"] != "GB/s":
                continue
            attach_copy(e, dev, max(3, args.op_reps // 2), flush, name)
            cc = e["copy_same_bytes"]["value"]
            extra = ""
            if "copy_rows_same_bytes" in e:
                cr = e["copy_rows_same_bytes"]["value"]
                extra = f"; row-order copy {cr:.0f} GB/s, op at {e['value'] / cr:.1%} of it"
            if "mix_same_pattern" in e:
                extra += f"; its stream mix {e['mix_same_pattern']['ms']:.4f} ms, op at " \
                         f"{e['mix_same_pattern']['op_over_mix']:.1%} of it"
            log(f"  {name}: copy {cc:.0f} GB/s, op at {e['value'] / cc:.1%} of it{extra}")
        del flush

    del c2
    torch.cuda.empty_cache()
    if args.calibrate_copy:
        src = torch.empty(1 << 30, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
        torch.cuda.empty_cache()
    cpu = None
    if not args.no_cpu:
        log("CPU baseline ...")
        cpu = cpu_baseline()
        log(f"  CPU: {cpu['value']} GB/s on {cpu['cores']} cores")

    line = {
        "metric": METRIC, "value": round(value, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_per_step, 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic: seeded N(0,1) inputs and upstream grads of BASELINE.json configs[1]",
        "config": {"workload": "C2 Llama-3-8B layer ops fwd+bwd: FusedAddRMSNorm x,r[8192,4096]; "
                               "RoPE q[4,2048,32,128] k[4,2048,8,128] theta=500000 ([B,T,H,D] storage); "
                               "SwiGLU gate,up[8192,14336]",
                   "bytes_per_step": total_bytes, "parallelism": "single GPU"},
        "roofline": roofline, "cpu_baseline": cpu, "graph_replay": graph, "ops": ops,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
