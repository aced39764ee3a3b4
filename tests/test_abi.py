"""CPU tier: the C-ABI library loads, exports every symbol include/*.h declares,
matches the Python binding table, and rejects bad arguments before touching
the GPU (so these run without a device). Also checks the Python layer's
no-CPU-fallback rule."""
import ctypes
import glob
import os
import re

import pytest
import torch

from kernels import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = glob.glob(os.path.join(ROOT, "include", "*.h"))

needs_lib = pytest.mark.skipif(not os.path.exists(_lib.LIB_PATH), reason="library not built")


def declared_symbols():
    names = set()
    for h in HEADERS:
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names.update(re.findall(r"\b(hk_[a-z0-9_]+)\s*\(", text))
    return names


def test_header_and_binding_table_agree():
    assert declared_symbols() == set(_lib.SIGNATURES), \
        f"header-only: {declared_symbols() - set(_lib.SIGNATURES)}; binding-only: {set(_lib.SIGNATURES) - declared_symbols()}"
    hdr = open(os.path.join(ROOT, "include", "hilda_kernel_amd.h")).read()
    assert f"#define HK_ABI_VERSION {_lib.ABI_VERSION}" in hdr


@needs_lib
def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(_lib.LIB_PATH)
    missing = [n for n in sorted(declared_symbols()) if not hasattr(lib, n)]
    assert not missing, f"not exported: {missing}"
    assert _lib.load().hk_abi_version() == _lib.ABI_VERSION


def _expect_einval(status, fragment):
    assert status == -1, f"expected HK_EINVAL, got {status}"
    msg = _lib.last_error()
    assert fragment in msg, f"error text {msg!r} lacks {fragment!r}"


@needs_lib
def test_argument_validation_without_gpu():
    lib = _lib.load()
    p = ctypes.c_void_p(16)  # never dereferenced: validation fails first
    _expect_einval(lib.hk_rms_norm_fwd(p, p, p, p, 4, 8, 8, 8, 7, 0, 1e-6, None), "dtype")
    _expect_einval(lib.hk_rms_norm_fwd(p, p, p, p, -1, 8, 8, 8, 0, 0, 1e-6, None), "shape")
    _expect_einval(lib.hk_rms_norm_fwd(p, p, p, p, 4, 8, 4, 8, 0, 0, 1e-6, None), "stride")
    _expect_einval(lib.hk_rms_norm_fwd(None, p, p, p, 4, 8, 8, 8, 0, 0, 1e-6, None), "null")
    _expect_einval(lib.hk_rms_norm_fwd(p, p, p, p, 4, 8, 8, 8, 1, 2, 1e-6, None), "dtype pair")
    _expect_einval(lib.hk_rms_norm_bwd(p, p, p, p, p, p, 4, 8, 8, 8, 8, 0, 0, 9, p, 64, None), "dw_mode")
    _expect_einval(lib.hk_fused_add_rms_norm_fwd(p, p, p, p, None, p, 4, 8, 8, 0, 0, 1e-6, None), "null")
    _expect_einval(lib.hk_rope(p, p, p, p, 1, 1, 1, 7, 7, 7, 7, 7, 7, 7, 1, 0, 3, 0, 0, 0, None), "even")
    _expect_einval(lib.hk_rope(p, p, p, p, 2, 1, 1, 8, 8, 8, 8, 8, 8, 8, 3, 0, 4, 0, 0, 0, None), "batch")
    _expect_einval(lib.hk_swiglu_fwd(p, p, p, -5, 2, None), "element count")
    _expect_einval(lib.hk_swiglu_bwd(p, p, p, p, p, 10, 5, None), "dtype")


@needs_lib
def test_argument_validation_losses_without_gpu():
    """The loss-family, fused-linear and AttnRes entry points reject bad arguments before any HIP call."""
    lib = _lib.load()
    p = ctypes.c_void_p(256)  # never dereferenced: validation fails first
    ws = ctypes.c_void_p(1 << 20)
    # CrossEntropy / GRPO
    _expect_einval(lib.hk_cross_entropy_fwd_grad(p, p, p, p, p, 4, 8, 8, 8, -100, 1, 7, ws, 1 << 20, None), "dtype")
    grpo = [p, p, None, p, p, p, p, p, p, p, 8, 1, p, None, 0, 0, None, 0, 0, None, 0, 0, 0, 2, 8, 16]
    _expect_einval(lib.hk_grpo_loss_fwd(*grpo, 1.0, 0.1, 0.2, 0.2, 2, ws, 1 << 20, None), "ref_logp")
    _expect_einval(lib.hk_grpo_loss_fwd(*grpo, 0.0, 0.0, 0.2, 0.2, 2, ws, 1 << 20, None), "temperature")
    # KLDiv / JSD / GeGLU
    _expect_einval(lib.hk_kl_div_fwd(p, p, p, p, 4, 8, 8, 8, 0, 1e-10, 9, 2, None), "reduction")
    _expect_einval(lib.hk_kl_div_fwd(p, p, p, p, 4, 8, 4, 8, 0, 1e-10, 1, 2, None), "shape")
    _expect_einval(lib.hk_jsd_fwd(p, p, p, p, p, None, -100, 1.5, 4, 8, 8, 8, 8, 2, ws, 1 << 20, None), "beta")
    _expect_einval(lib.hk_geglu_fwd(p, p, p, -1, 2, None), "element count")
    # FusedLinearCE: hidden [BT, H], weight [V, H] (any H and V); chunk, budget, workspace
    flce = [p, p, p, p, p, p, p, None]
    _expect_einval(lib.hk_fused_linear_cross_entropy(*flce, 64, 64, 128, -100, 1, 5, 0, 0, ws, 1 << 20, None),
                   "fp32, bf16 and fp16")
    _expect_einval(lib.hk_fused_linear_cross_entropy(*flce, 64, 0, 128, -100, 1, 2, 0, 0, ws, 1 << 20, None),
                   "invalid shape")
    _expect_einval(lib.hk_fused_linear_cross_entropy(*flce, 64, 64, 128, -100, 5, 2, 0, 0, ws, 1 << 20, None),
                   "reduction")
    _expect_einval(lib.hk_fused_linear_cross_entropy(*flce, 64, 64, 128, -100, 1, 2, 0, 0, ws, 64, None),
                   "workspace too small")
    _expect_einval(lib.hk_fused_linear_cross_entropy(*flce, 64, 64, 128, -100, 1, 2, 0, 4096, ws, 1 << 20, None),
                   "below the smallest plan")
    _expect_einval(lib.hk_fused_linear_cross_entropy(p, p, p, None, p, p, p, None, 64, 64, 128, -100, 1, 2, 0, 0, ws,
                                                     1 << 20, None), "computed together")
    _expect_einval(lib.hk_fused_linear_cross_entropy(*flce[:4], ctypes.c_void_p(257), *flce[5:], 64, 64, 128, -100,
                                                     1, 2, 0, 0, ws, 1 << 20, None), "element size")
    # FusedLinear-GRPO: hidden (B, L+1, H), weight [V, H]
    head = [p, p, p, p, p, p, p, p, p, p, p, p, 8, 1, p, None, 0, 0, None, 0, 0, None, 0, 0, 0, 2, 7]
    _expect_einval(lib.hk_fused_linear_grpo(*head, 64, 128, 1.0, 0.0, 0.2, 0.2, 3, 0, 0, ws, 1 << 30, None),
                   "fp32, bf16 and fp16")
    _expect_einval(lib.hk_fused_linear_grpo(*head, 0, 128, 1.0, 0.0, 0.2, 0.2, 2, 0, 0, ws, 1 << 30, None),
                   "invalid shape")
    _expect_einval(lib.hk_fused_linear_grpo(*head, 64, 128, 1.0, 0.1, 0.2, 0.2, 2, 0, 0, ws, 1 << 30, None),
                   "ref_logp")
    _expect_einval(lib.hk_fused_linear_grpo(*head, 64, 128, -1.0, 0.0, 0.2, 0.2, 2, 0, 0, ws, 1 << 30, None),
                   "temperature")
    _expect_einval(lib.hk_fused_linear_grpo(*head, 64, 128, 1.0, 0.0, 0.2, 0.2, 2, 0, 0, ws, 64, None),
                   "workspace too small")
    # FusedLinearJSD
    jsd = [p, p, p, p, p, p, p, None]
    _expect_einval(lib.hk_fused_linear_jsd(*jsd, 64, 64, 64, 128, -100, 1.5, 1.0, 2, 0, 0, ws, 1 << 30, None), "beta")
    _expect_einval(lib.hk_fused_linear_jsd(*jsd, 64, 64, 0, 128, -100, 0.5, 1.0, 2, 0, 0, ws, 1 << 30, None),
                   "teacher hidden size")
    # AttnRes
    _expect_einval(lib.hk_attn_res_fwd(p, p, p, p, p, p, 33, 16, 64, 1e-6, 2, None), "1..32 blocks")
    _expect_einval(lib.hk_attn_res_fwd(p, p, p, p, p, p, 4, 16, 12, 1e-6, 2, None), "multiple of 8")
    _expect_einval(lib.hk_attn_res_fwd(p, p, p, p, p, p, 4, 16, 8 * 256 * 8 + 8, 1e-6, 2, None), "at most")
    _expect_einval(lib.hk_attn_res_bwd(p, p, p, p, p, p, p, p, p, 4, 16, 64, 2, ws, 8, None), "workspace too small")
    _expect_einval(lib.hk_stream_copy(p, p, 4, 64, 7, None), "copy mode")
    _expect_einval(lib.hk_stream_copy(p, p, 4, 24, _lib.COPY_FLAT, None), "16-byte")
    _expect_einval(lib.hk_stream_copy(p, p, 4, 24 * 1024 * 16 + 16, _lib.COPY_ROWS, None), "at most")
    _expect_einval(lib.hk_stream_mix(p, p, 64, 64, 0, 1, None), "streams read")
    _expect_einval(lib.hk_stream_mix(p, p, 64, 64, 10, 1, None), "streams read")
    _expect_einval(lib.hk_stream_mix(p, p, 64, 64, 2, 9, None), "streams read")
    _expect_einval(lib.hk_stream_mix(p, p, 24, 32, 2, 1, None), "16-byte")
    _expect_einval(lib.hk_stream_mix(p, p, 64, 48, 2, 1, None), "stride")
    _expect_einval(lib.hk_stream_mix(p, p, 64, 72, 2, 1, None), "stride")


def _flce_ws(BT, H, V, budget=0, dtype=2, grad=1, chunk=0):
    return _lib.load().hk_fused_linear_cross_entropy_workspace_size(BT, H, V, chunk, budget, dtype, grad, None, None)


def _flce_plan(BT, H, V, budget=0, dtype=2, grad=1, chunk=0):
    info = (ctypes.c_int64 * 8)()
    _lib.check(_lib.load().hk_fused_linear_cross_entropy_plan(BT, H, V, chunk, budget, dtype, grad, None, None, info),
               "plan")
    return list(info)


@needs_lib
def test_fused_linear_workspace_queries():
    lib = _lib.load()
    MiB = 2**20
    # an unknown dtype needs no workspace; with no limit a gradient call needs more than a loss-only call
    assert _flce_ws(16384, 4096, 128256, dtype=5) == 0
    assert 0 < _flce_ws(16384, 4096, 128256, grad=0, budget=-1) < _flce_ws(16384, 4096, 128256, budget=-1)
    # the default plan costs what the reference's chunk costs (fused_linear_cross_entropy.py:112-114):
    # chunk logits about the size of the hidden states, plus the gathered rows, their transpose and a quarter
    # of the chunk for split partials; nothing grows with BT x V
    for BT, H, V, rows in ((4096, 4096, 128256, 128), (8192, 4096, 128256, 256), (8192, 4096, 32000, 1024),
                           (16384, 4096, 128256, 512)):
        chunk_bytes = rows * ((V + 63) // 64 * 64) * 2
        ws = _flce_ws(BT, H, V)
        assert 0 < ws <= 1.25 * chunk_bytes + 2 * rows * H * 2 + 16 * BT + MiB, (BT, H, V, ws)
        C, nch, dw, wt, dt, _, total, _ = _flce_plan(BT, H, V)
        assert total == ws and not wt and not dt  # nothing weight- or logits-sized
        # row chunks with dW in the output (C rows a chunk), or vocabulary tiles (C columns a tile)
        assert (dw == 2 and C * nch >= BT) or (dw in (3, 4) and C * nch >= V)
    # 47.7% below the unfused path's peak at the reference's tightest memory config (N 4096, V 128256,
    # fp16): h + w + logits + log-softmax + their two gradients at most, against h, w, both gradients and
    # the workspace here
    BT, H, V = 4096, 4096, 128256
    unfused = 2 * (BT * H + V * H + 3 * BT * V)
    ours = 2 * 2 * (BT * H + V * H) + _flce_ws(BT, H, V, dtype=1)
    assert ours <= (1 - 0.477) * unfused
    # no limit: C5 takes the fastest plan, every chunk's D^T kept and one dW GEMM (GBs of workspace)
    C, nch, dw, wt, dt, _, total, model = _flce_plan(16384, 4096, 128256, budget=-1)
    assert (C, nch, dw, wt, dt) == (8192, 2, 0, 1, 1) and total > 4 * 2**30
    # each plan fits its budget; a larger budget never gives up fp32 dW/dX sums once they fit, and never gives
    # a slower modelled plan of the same kind (16-bit accumulation over several chunks or tiles is taken only
    # while no fp32-summing plan fits)
    prev = None
    for b in (64 * MiB, 256 * MiB, 1 << 30, 4 << 30, 16 << 30):
        C, nch, dw, wt, dt, _, total, model = _flce_plan(16384, 4096, 128256, budget=b)
        assert total <= b
        exact = dw in (0, 1, 3) or nch <= 1
        if prev is not None:
            assert exact >= prev[0]
            assert exact > prev[0] or model <= prev[1]
        prev = (exact, model)
    # a budget below the smallest plan: no workspace size (and the op rejects the call)
    assert _flce_ws(64, 64, 128, budget=4096) == 0
    # fp32 has no MN-contiguous operand form: W^T and D^T are always materialised
    _, _, _, wt, dt, _, _, _ = _flce_plan(256, 4096, 32000, dtype=0)
    assert wt and dt
    # any H and V: an odd hidden size pads the weight into a copy (weight-sized workspace)
    assert _flce_ws(512, 4099, 32001) > 32001 * 4104 * 2
    # a misaligned weight is copied too
    assert (lib.hk_fused_linear_cross_entropy_workspace_size(512, 4096, 32000, 0, 0, 2, 1, None, ctypes.c_void_p(18))
            > 32000 * 4096 * 2)
    assert lib.hk_fused_linear_grpo_workspace_size(16, 1023, 4096, 151936, 0, 0, 2, 1, None, None) > 0
    assert lib.hk_fused_linear_grpo_workspace_size(0, 1023, 4096, 151936, 0, 0, 2, 1, None, None) == 0
    assert lib.hk_fused_linear_jsd_workspace_size(8192, 4096, 4096, 128256, 0, 0, 2, 1, 1, None, None, None,
                                                  None) > 0
    assert lib.hk_attn_res_bwd_workspace_size(8192, 4096) % (2 * 4096 * 4) == 0


@needs_lib
def test_cross_entropy_workspace_query():
    lib = _lib.load()
    # 256 bytes of counters, then the launch plan's row list (4 bytes a row, whole 256-byte blocks)
    assert lib.hk_cross_entropy_workspace_size(0) == 256
    assert lib.hk_cross_entropy_workspace_size(1) == 512
    assert lib.hk_cross_entropy_workspace_size(64) == 512
    assert lib.hk_cross_entropy_workspace_size(65) == 768
    assert lib.hk_cross_entropy_workspace_size(8192) == 256 + 8192 * 4


@needs_lib
def test_workspace_query_is_pure():
    lib = _lib.load()
    # atomic path: one [cols] fp64 row; partial path (bf16 -> fp32 accumulators): one row per row group
    part = lib.hk_rms_norm_bwd_workspace_size(8192, 4096, 2, 2, _lib.DW_PARTIAL, 0)
    atom = lib.hk_rms_norm_bwd_workspace_size(8192, 4096, 2, 2, _lib.DW_ATOMIC, 0)
    assert atom == 4096 * 8
    assert part >= 4096 * 4 and part % (4096 * 4) == 0
    # fp32 inputs accumulate in fp64 registers but store fp32 partial rows too, one per row group (16-bit
    # inputs sum a 1024-lane block's groups in LDS first, so they store fewer rows)
    part32 = lib.hk_rms_norm_bwd_workspace_size(8192, 4096, 0, 0, _lib.DW_PARTIAL, 0)
    assert part32 % (4096 * 4) == 0 and part32 >= part
    assert lib.hk_rms_norm_bwd_workspace_size(-1, 4096, 2, 2, 0, 0) == 0
    # the default mode takes the partial rows at every row count (no atomics for few rows)
    for rows in (16, 2048, 8192):
        assert (lib.hk_rms_norm_bwd_workspace_size(rows, 4096, 2, 2, _lib.DW_AUTO, 0) ==
                lib.hk_rms_norm_bwd_workspace_size(rows, 4096, 2, 2, _lib.DW_PARTIAL, 0))


def test_ops_refuse_cpu_tensors():
    """No CPU path: every op raises on host tensors instead of computing there."""
    from kernels import (hilda_rms_norm, hilda_swiglu, hilda_rope, hilda_fused_add_rms_norm, hilda_geglu,
                         hilda_cross_entropy, hilda_grpo_loss, hilda_kl_div, hilda_jsd, hilda_attn_res,
                         hilda_fused_linear_cross_entropy, hilda_fused_linear_jsd, hilda_fused_linear_grpo_loss)
    bf = torch.bfloat16
    lg = torch.randn(4, 16)
    t = torch.zeros(4, dtype=torch.int64)
    for call in (lambda: hilda_geglu(lg, lg), lambda: hilda_cross_entropy(lg, t),
                 lambda: hilda_kl_div(lg, lg), lambda: hilda_jsd(lg, lg),
                 lambda: hilda_grpo_loss(torch.randn(2, 3, 16), torch.zeros(2, 2, dtype=torch.int64),
                                         torch.zeros(2)),
                 lambda: hilda_attn_res(torch.randn(2, 1, 4, 16), torch.ones(16), torch.ones(16)),
                 lambda: hilda_fused_linear_cross_entropy(lg.to(bf), lg.to(bf), t),
                 lambda: hilda_fused_linear_jsd(lg.to(bf), lg.to(bf), lg.to(bf), lg.to(bf)),
                 lambda: hilda_fused_linear_grpo_loss(torch.randn(2, 3, 16).to(bf), lg.to(bf),
                                                      torch.zeros(2, 2, dtype=torch.int64), torch.zeros(2))):
        with pytest.raises(RuntimeError, match="ROCm GPU"):
            call()
    x = torch.randn(4, 8)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        hilda_rms_norm(x, torch.ones(8))
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        hilda_fused_add_rms_norm(x, x, torch.ones(8))
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        hilda_swiglu(x, x)
    q = torch.randn(1, 2, 4, 8)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        hilda_rope(q, q, torch.ones(1, 4, 4), torch.zeros(1, 4, 4))


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "LIB_PATH", str(tmp_path / "absent.so"))
    with pytest.raises(RuntimeError, match="not built"):
        _lib.load()


def test_fl_budget_argument(monkeypatch):
    """workspace_budget as the C ABI takes it: None reads $HILDA_FL_WORKSPACE_BUDGET (unset: the default, 0),
    'default' 0, 'fastest' / 'unlimited' -1, bytes as an int or a numeric string, negatives -1; other strings raise."""
    monkeypatch.delenv(_lib.BUDGET_ENV, raising=False)
    assert _lib.fl_budget(None) == 0
    monkeypatch.setenv(_lib.BUDGET_ENV, "fastest")
    assert _lib.fl_budget(None) == -1
    monkeypatch.setenv(_lib.BUDGET_ENV, "1.5e9")
    assert _lib.fl_budget(None) == 1_500_000_000
    assert _lib.fl_budget("default") == 0 and _lib.fl_budget("Unlimited") == -1
    assert _lib.fl_budget(64 << 20) == 64 << 20 and _lib.fl_budget(-7) == -1 and _lib.fl_budget(0) == 0
    with pytest.raises(ValueError):
        _lib.fl_budget("lots")


@needs_lib
def test_fl_budget_env_selects_the_plan(monkeypatch):
    """The environment variable reaches the plan when the call leaves workspace_budget None."""
    from kernels.fused_linear_cross_entropy import fused_linear_cross_entropy_plan as plan
    import torch
    shape = (16384, 4096, 128256, torch.bfloat16)
    monkeypatch.delenv(_lib.BUDGET_ENV, raising=False)
    default = plan(*shape)
    fastest = plan(*shape, workspace_budget="fastest")
    assert default != fastest
    monkeypatch.setenv(_lib.BUDGET_ENV, "fastest")
    assert plan(*shape) == fastest
    monkeypatch.setenv(_lib.BUDGET_ENV, str(default["workspace_bytes"]))
    assert plan(*shape)["workspace_bytes"] <= default["workspace_bytes"]


def _reference_jsd_transient(BT, H, V, es):
    """Bytes fused_linear_jsd_forward (fused_linear_jsd.py:133-203) holds at once beside its inputs and outputs, at
    its dW product: the chunk's tensors, each named, and the [V, H] product dlogits_compute.t() @ s_chunk."""
    inc = -(-V // H)
    per = -(-BT // inc)
    cs = min(1 << (per - 1).bit_length(), BT)  # triton.next_power_of_2, the last chunk may be shorter
    cell = cs * V
    upcast = es != 4  # .float() / .to() of an fp32 tensor return the tensor itself
    tensors = {
        "s_logits": cell * es, "t_logits": cell * es,
        "s_logprobs": cell * 4 if upcast else 0, "t_logprobs": cell * 4 if upcast else 0,
        "dX": cell * 4, "dlogits": cell * 4, "dlogits_compute": cell * es if upcast else 0,
        "loss_per_row": cs * 4,
    }
    return sum(tensors.values()) + V * H * es


@needs_lib
def test_fused_jsd_grpo_default_budget_floor():
    """FusedLinearJSD's default workspace is at most what the reference's own chunk loop holds at once (so, with the
    same outputs, its peak memory is at most the reference's) and uses that room: more than a 256 MiB plan, no more
    than the unlimited one. FusedLinear-GRPO (no reference) takes at least twice the weight's bytes. Both beat the
    reference-chunk budget FusedLinearCE's default gets."""
    lib = _lib.load()
    jsd = lambda BT, H, V, dt, budget: lib.hk_fused_linear_jsd_workspace_size(BT, H, H, V, 0, budget, dt, 1, 0, None,
                                                                              None, None, None)
    # the reference's memory configs (bench_fused_linear_jsd.py:163-166,180) and the benchmark shape
    for BT, H, V, dt, es in [(4096, 4096, 32000, 1, 2), (2048, 4096, 128256, 1, 2), (8192, 4096, 128256, 2, 2),
                             (2048, 4096, 32000, 0, 4)]:
        ref = _reference_jsd_transient(BT, H, V, es)
        d, f = jsd(BT, H, V, dt, 0), jsd(BT, H, V, dt, -1)
        assert 0 < d <= ref, (BT, H, V, dt, d, ref)
        assert d <= f
        if f > d:
            assert d > jsd(BT, H, V, dt, 256 << 20) or jsd(BT, H, V, dt, 256 << 20) == 0
    assert _flce_ws(8192, 4096, 128256) < jsd(8192, 4096, 128256, 2, 0)
    H = 4096
    grpo = lambda budget: lib.hk_fused_linear_grpo_workspace_size(16, 1023, H, 151936, 0, budget, 2, 1, None, None)
    g_floor = 2 * 151936 * H * 2
    d_grpo, f_grpo = grpo(0), grpo(-1)
    assert _flce_ws(16 * 1024, H, 151936) < d_grpo <= g_floor + (64 << 20) and d_grpo < f_grpo
    # an explicit budget is still honoured below the floor
    assert 0 < jsd(8192, H, 128256, 2, 256 << 20) <= 256 << 20


@needs_lib
def test_fused_linear_plans_property_sweep():
    """Over many shapes, dtypes and budgets the planner's answer is self-consistent: a plan that fits reports the
    bytes the size query returns, within any positive budget; its rows per chunk (or vocabulary columns per
    tile) and chunk (tile) count cover BT (V); the chunk cap is honoured; a budget of 0 bytes more than the
    answer gives the same plan; and loss-only calls never need more than gradient calls."""
    import random
    rnd = random.Random(7)
    lib = _lib.load()
    cases = 0
    for _ in range(300):
        BT = rnd.choice([1, 7, 64, 300, 1000, 4096, 8192, 16384, 50000])
        H = rnd.choice([8, 64, 264, 1000, 4096, 4099])
        V = rnd.choice([8, 1000, 2001, 32000, 50257, 128256])
        dt = rnd.choice([0, 1, 2])
        chunk = rnd.choice([0, 0, 64, 1000])
        budget = rnd.choice([0, 0, -1, 1 << 20, 64 << 20, 1 << 30])
        info = (ctypes.c_int64 * 8)()
        rc = lib.hk_fused_linear_cross_entropy_plan(BT, H, V, chunk, budget, dt, 1, None, None, info)
        ws = lib.hk_fused_linear_cross_entropy_workspace_size(BT, H, V, chunk, budget, dt, 1, None, None)
        if rc != 0:
            assert ws == 0 and budget > 0, (BT, H, V, dt, chunk, budget)
            continue
        cases += 1
        rows_or_cols, n, mode, wt, dtr, splits, total, model_ns = list(info)
        assert total == ws > 0
        if budget > 0:
            assert total <= budget
        assert model_ns > 0 and splits >= 1
        if mode in (3, 4):  # vocabulary tiles: columns a tile, tiles
            assert dt != 0 and chunk == 0 and rows_or_cols % 256 == 0 and rows_or_cols * n >= V
        else:
            assert rows_or_cols * n >= BT and rows_or_cols <= 8192
            if chunk > 0:
                assert rows_or_cols <= max(8, chunk)
            if dt == 0:
                assert wt and dtr  # fp32 reads no MN-contiguous operand
        # the same plan under a budget of exactly its bytes
        info2 = (ctypes.c_int64 * 8)()
        assert lib.hk_fused_linear_cross_entropy_plan(BT, H, V, chunk, total, dt, 1, None, None, info2) == 0
        assert info2[6] <= total
        # a loss-only call never needs more
        assert lib.hk_fused_linear_cross_entropy_workspace_size(BT, H, V, chunk, -1, dt, 0, None, None) <= \
            lib.hk_fused_linear_cross_entropy_workspace_size(BT, H, V, chunk, -1, dt, 1, None, None)
    assert cases > 150


@needs_lib
def test_fused_jsd_grpo_plans_property_sweep():
    """FusedLinearJSD's and FusedLinear-GRPO's plan queries agree with their size queries over many shapes, dtypes
    and budgets: the reported bytes are the size query's and fit a positive budget, the chunks cover the rows
    (GRPO: B*(L+1) positions), the chunk cap holds, no vocabulary tiles, and fp32 reads no MN-contiguous operand."""
    import random
    rnd = random.Random(11)
    lib = _lib.load()
    cases = 0
    for _ in range(200):
        H = rnd.choice([8, 64, 264, 1000, 4096, 4099])
        V = rnd.choice([8, 1000, 2001, 32000, 50257, 128256])
        dt = rnd.choice([0, 1, 2])
        chunk = rnd.choice([0, 0, 64, 1000])
        budget = rnd.choice([0, 0, -1, 1 << 20, 64 << 20, 1 << 30])
        info = (ctypes.c_int64 * 8)()
        if rnd.random() < 0.5:
            BT = rnd.choice([1, 7, 64, 300, 1000, 4096, 8192])
            Ht = rnd.choice([H, 8, 1000])
            labels = rnd.choice([0, 1])
            rc = lib.hk_fused_linear_jsd_plan(BT, H, Ht, V, chunk, budget, dt, 1, labels, None, None, None, None,
                                              info)
            ws = lib.hk_fused_linear_jsd_workspace_size(BT, H, Ht, V, chunk, budget, dt, 1, labels, None, None, None,
                                                        None)
            rows = BT
        else:
            B, L = rnd.choice([1, 3, 16]), rnd.choice([0, 5, 127, 1023])
            rc = lib.hk_fused_linear_grpo_plan(B, L, H, V, chunk, budget, dt, 1, None, None, info)
            ws = lib.hk_fused_linear_grpo_workspace_size(B, L, H, V, chunk, budget, dt, 1, None, None)
            rows = B * (L + 1)
        if rc != 0:
            assert ws == 0 and budget > 0
            continue
        cases += 1
        c, n, mode, wt, dtr, splits, total, model_ns = list(info)
        assert total == ws > 0 and mode in (0, 1, 2) and splits >= 1 and model_ns > 0
        if budget > 0:
            assert total <= budget
        assert c * n >= rows and c <= 8192
        if chunk > 0:
            assert c <= max(8, chunk)
        if dt == 0:
            assert wt and dtr
    assert cases > 100
    # argument checks run before any HIP call
    assert lib.hk_fused_linear_jsd_plan(8, 8, 8, 8, 0, 0, 2, 1, 0, None, None, None, None, None) == -1
    assert lib.hk_fused_linear_grpo_plan(0, 5, 8, 8, 0, 0, 2, 1, None, None, info) == -1
