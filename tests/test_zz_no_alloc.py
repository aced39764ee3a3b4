"""GPU: the allocation-free RMSNorm backward (hk_rms_norm_bwd_noalloc) against hk_rms_norm_bwd.

Both entry points run the same kernels, the second with its dW scratch in
caller workspace and the first in the library's per-device array, so their
results must be bitwise equal. Two calls in a row, the second on a smaller
input (the array keeps the first call's partial rows, which must not leak
into the second's dW), in both dW modes and for fp32 and bf16 inputs. A call
whose scratch need exceeds the array is rejected before any launch.
"""
import pytest
import torch

from _util import gpu
from kernels import _lib

pytestmark = pytest.mark.gpu


def _inputs(rows, cols, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(rows, cols, generator=g).to(dtype)
    w = (1 + 0.02 * torch.randn(cols, generator=g)).to(dtype)
    dy = torch.randn(rows, cols, generator=g).to(dtype)
    x, w, dy = x.to(gpu()), w.to(gpu()), dy.to(gpu())
    rstd = torch.rsqrt(x.float().pow(2).mean(-1) + 1e-6).contiguous()
    return x, w, dy, rstd


def _bwd(x, w, dy, rstd, dw_mode, noalloc):
    rows, cols = x.shape
    dev = x.device
    dx = torch.empty_like(x)
    dw = torch.empty_like(w)
    code_x, code_w = _lib.dtype_code(x), _lib.dtype_code(w)
    stream = _lib.stream_of(dev)
    if noalloc:
        _lib.call("hk_rms_norm_bwd_noalloc", dx.data_ptr(), dw.data_ptr(), dy.data_ptr(), x.data_ptr(), w.data_ptr(),
                  rstd.data_ptr(), rows, cols, cols, cols, cols, code_x, code_w, dw_mode, stream)
    else:
        lib = _lib.load()
        n = lib.hk_rms_norm_bwd_workspace_size(rows, cols, code_x, code_w, dw_mode, dev.index)
        ws = torch.empty(max(n, 16), dtype=torch.uint8, device=dev)
        _lib.call("hk_rms_norm_bwd", dx.data_ptr(), dw.data_ptr(), dy.data_ptr(), x.data_ptr(), w.data_ptr(),
                  rstd.data_ptr(), rows, cols, cols, cols, cols, code_x, code_w, dw_mode, ws.data_ptr(), ws.numel(),
                  stream)
    return dx, dw


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("dw_mode", [_lib.DW_AUTO, _lib.DW_ATOMIC])
def test_noalloc_matches_workspace_entry_point(dtype, dw_mode):
    # register-form rows, and fp32 rows too wide for registers (the streaming plan: per-row coefficients
    # placed after the partial rows in the scratch array)
    shapes = ((4096, 4096, 1), (300, 1024, 2)) + (((3, 40000, 4),) if dtype == torch.float32 else ())
    for rows, cols, seed in shapes:
        print(f"noalloc rms_norm_bwd {dtype} mode={dw_mode} rows={rows} cols={cols}", flush=True)
        x, w, dy, rstd = _inputs(rows, cols, dtype, seed)
        dx_a, dw_a = _bwd(x, w, dy, rstd, dw_mode, noalloc=True)
        dx_b, dw_b = _bwd(x, w, dy, rstd, dw_mode, noalloc=False)
        torch.cuda.synchronize()
        assert torch.equal(dx_a, dx_b), "dx differs from hk_rms_norm_bwd"
        assert torch.equal(dw_a, dw_b), "dw differs from hk_rms_norm_bwd"


def test_noalloc_rejects_oversized_scratch():
    # fp32 rows of 16384 columns: two partial rows a CU of 64 KiB each, beyond the 16 MiB array
    x, w, dy, rstd = _inputs(4096, 16384, torch.float32, 3)
    lib = _lib.load()
    need = lib.hk_rms_norm_bwd_workspace_size(4096, 16384, _lib.F32, _lib.F32, _lib.DW_AUTO, x.device.index)
    if need <= 16 << 20:
        pytest.skip(f"this GPU needs only {need} bytes of scratch here")
    dx, dw = torch.empty_like(x), torch.empty_like(w)
    status = lib.hk_rms_norm_bwd_noalloc(dx.data_ptr(), dw.data_ptr(), dy.data_ptr(), x.data_ptr(), w.data_ptr(),
                                         rstd.data_ptr(), 4096, 16384, 16384, 16384, 16384, _lib.F32, _lib.F32,
                                         _lib.DW_AUTO, _lib.stream_of(x.device))
    assert status == -1 and "dW scratch" in _lib.last_error()
