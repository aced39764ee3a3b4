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
def test_workspace_query_is_pure():
    lib = _lib.load()
    # atomic path: one [cols] fp64 row; partial path (bf16 -> fp32 accumulators): one row per row group
    part = lib.hk_rms_norm_bwd_workspace_size(8192, 4096, 2, 2, _lib.DW_PARTIAL, 0)
    atom = lib.hk_rms_norm_bwd_workspace_size(8192, 4096, 2, 2, _lib.DW_ATOMIC, 0)
    assert atom == 4096 * 8
    assert part >= 4096 * 4 and part % (4096 * 4) == 0
    # fp32 inputs accumulate in fp64 registers but store fp32 partial rows too
    part32 = lib.hk_rms_norm_bwd_workspace_size(8192, 4096, 0, 0, _lib.DW_PARTIAL, 0)
    assert part32 == part
    assert lib.hk_rms_norm_bwd_workspace_size(-1, 4096, 2, 2, 0, 0) == 0


def test_ops_refuse_cpu_tensors():
    """No CPU path: every op raises on host tensors instead of computing there."""
    from kernels import hilda_rms_norm, hilda_swiglu, hilda_rope, hilda_fused_add_rms_norm
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
