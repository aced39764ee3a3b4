"""ctypes binding of the gfx950 C-ABI library (``libhilda_kernel_amd.so``).

The library is built in-tree by ``hilda-kernel_amd/build.py``. There is no
fallback: if the library is missing, or a tensor is not on a ROCm device,
the ops raise instead of computing anything elsewhere.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch

LIB_NAME = "libhilda_kernel_amd.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)

F32, F16, BF16, U8, I32, I64 = 0, 1, 2, 3, 4, 5
DW_AUTO, DW_ATOMIC, DW_PARTIAL = 0, 1, 2
COPY_FLAT, COPY_ROWS = 0, 1
REDUCTION = {"none": 0, "mean": 1, "sum": 2}

_DTYPE_CODE = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16}
_MASK_CODE = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16, torch.bool: U8, torch.uint8: U8,
              torch.int32: I32, torch.int64: I64}

_i32, _i64, _f32, _p, _sz = ctypes.c_int, ctypes.c_int64, ctypes.c_float, ctypes.c_void_p, ctypes.c_size_t

# name -> (restype, argtypes); mirrors include/hilda_kernel_amd.h
SIGNATURES = {
    "hk_abi_version": (_i32, []),
    "hk_last_error": (ctypes.c_char_p, []),
    "hk_device_cu_count": (_i32, [_i32]),
    "hk_rms_norm_fwd": (_i32, [_p, _p, _p, _p, _i64, _i64, _i64, _i64, _i32, _i32, _f32, _p]),
    "hk_rms_norm_bwd_workspace_size": (_sz, [_i64, _i64, _i32, _i32, _i32, _i32]),
    "hk_rms_norm_bwd": (_i32, [_p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i32, _i32, _i32, _p, _sz, _p]),
    "hk_rms_norm_bwd_noalloc": (_i32, [_p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i32, _i32, _i32, _p]),
    "hk_stream_copy": (_i32, [_p, _p, _i64, _i64, _i32, _p]),
    "hk_stream_mix": (_i32, [_p, _p, _i64, _i64, _i32, _i32, _p]),
    "hk_fused_add_rms_norm_fwd": (_i32, [_p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i32, _i32, _f32, _p]),
    "hk_fused_add_rms_norm_bwd": (_i32, [_p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i32, _i32, _i32, _p, _sz, _p]),
    "hk_rope": (_i32, [_p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                       _i32, _i32, _i32, _p]),
    "hk_rope_qk": (_i32, [_p, _p] + [_i64] * 7 + [_p, _p] + [_i64] * 7 + [_p, _p] + [_i64] * 6 + [_i32, _i32, _i32, _p]),
    "hk_swiglu_fwd": (_i32, [_p, _p, _p, _i64, _i32, _p]),
    "hk_swiglu_bwd": (_i32, [_p, _p, _p, _p, _p, _i64, _i32, _p]),
    "hk_geglu_fwd": (_i32, [_p, _p, _p, _i64, _i32, _p]),
    "hk_geglu_bwd": (_i32, [_p, _p, _p, _p, _p, _i64, _i32, _p]),
    "hk_kl_div_fwd": (_i32, [_p, _p, _p, _p, _i64, _i64, _i64, _i64, _i32, _f32, _i32, _i32, _p]),
    "hk_kl_div_bwd": (_i32, [_p, _p, _p, _i32, _f32, _i64, _i64, _i64, _i64, _i32, _i32, _p]),
    "hk_jsd_workspace_size": (_sz, []),
    "hk_jsd_fwd": (_i32, [_p, _p, _p, _p, _p, _p, _i64, _f32, _i64, _i64, _i64, _i64, _i64, _i32, _p, _sz, _p]),
    "hk_attn_res_fwd": (_i32, [_p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _f32, _i32, _p]),
    "hk_attn_res_bwd_workspace_size": (_sz, [_i64, _i64]),
    "hk_attn_res_bwd": (_i32, [_p, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i32, _p, _sz, _p]),
    "hk_fused_linear_jsd_workspace_size": (_sz, [_i64] * 6 + [_i32, _i32, _i32, _p, _p, _p, _p]),
    "hk_fused_linear_jsd_plan": (_i32, [_i64] * 6 + [_i32, _i32, _i32, _p, _p, _p, _p, _p]),
    "hk_fused_linear_jsd": (_i32, [_p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _f32, _f32, _i32,
                                   _i64, _i64, _p, _sz, _p]),
    "hk_cross_entropy_workspace_size": (_sz, [_i64]),
    "hk_cross_entropy_fwd_grad": (_i32, [_p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i32, _i32, _p, _sz, _p]),
    "hk_cross_entropy_fwd": (_i32, [_p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i32, _i32, _p, _sz, _p]),
    "hk_scale_rows": (_i32, [_p, _p, _p, _p, _i32, _i32, _i64, _i64, _i64, _i64, _i32, _p]),
    "hk_selective_log_softmax": (_i32, [_p, _p, _p, _i64, _i64, _p, _i32, _i64, _i64, _i64, _i64, _i64, _f32, _i32,
                                        _p]),
    "hk_grpo_workspace_size": (_sz, [_i64, _i64]),
    "hk_fused_linear_cross_entropy_workspace_size": (_sz, [_i64] * 5 + [_i32, _i32, _p, _p]),
    "hk_fused_linear_cross_entropy_plan": (_i32, [_i64] * 5 + [_i32, _i32, _p, _p, _p]),
    "hk_fused_linear_cross_entropy": (_i32, [_p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i32, _i32,
                                             _i64, _i64, _p, _sz, _p]),
    "hk_grpo_loss_fwd": (_i32, [_p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _p, _p, _i64, _i64, _p, _i64, _i64, _p,
                                _i32, _i64, _i64, _i64, _i64, _i64, _f32, _f32, _f32, _f32, _i32, _p, _sz, _p]),
    "hk_fused_linear_grpo_workspace_size": (_sz, [_i64] * 6 + [_i32, _i32, _p, _p]),
    "hk_fused_linear_grpo_plan": (_i32, [_i64] * 6 + [_i32, _i32, _p, _p, _p]),
    "hk_fused_linear_grpo": (_i32, [_p] * 7 + [_p, _p, _p, _p, _p, _i64, _i64, _p, _p, _i64, _i64, _p, _i64, _i64,
                                               _p, _i32, _i64, _i64, _i64, _i64, _i64, _i64, _f32, _f32, _f32, _f32,
                                               _i32, _i64, _i64, _p, _sz, _p]),
}

ABI_VERSION = 2

_lib = None
_lock = threading.Lock()


def load() -> ctypes.CDLL:
    """Load (once) and return the C-ABI library; raise if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(
                    f"{LIB_NAME} is not built (expected at {LIB_PATH}); "
                    "run `python hilda-kernel_amd/build.py` first")
            lib = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            got = lib.hk_abi_version()
            if got != ABI_VERSION:
                raise RuntimeError(f"{LIB_NAME} ABI version {got}, expected {ABI_VERSION}; rebuild it")
            _lib = lib
    return _lib


def last_error() -> str:
    return load().hk_last_error().decode(errors="replace")


def check(status: int, what: str) -> None:
    if status != 0:
        raise RuntimeError(f"{what} failed (status {status}): {last_error()}")


def call(name: str, *args) -> None:
    """Call an int-returning entry point and raise RuntimeError on failure."""
    check(getattr(load(), name)(*args), name)


def dtype_code(t: torch.Tensor) -> int:
    try:
        return _DTYPE_CODE[t.dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype {t.dtype}; expected float32, float16 or bfloat16") from None


def require_device(*tensors: torch.Tensor) -> torch.device:
    """All tensors must live on one ROCm device; there is no CPU path."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise RuntimeError(
                f"hilda-kernel_amd ops run only on a ROCm GPU; got a tensor on {t.device}")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"tensors on different devices: {dev} and {t.device}")
    return dev


def mask_code(t: torch.Tensor) -> int:
    try:
        return _MASK_CODE[t.dtype]
    except KeyError:
        raise TypeError(f"unsupported mask dtype {t.dtype}") from None


def stream_of(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t) -> int | None:
    return None if t is None else t.data_ptr()


_cu_cache: dict[int, int] = {}


def cu_count(device: torch.device) -> int:
    idx = device.index if device.index is not None else torch.cuda.current_device()
    if idx not in _cu_cache:
        n = load().hk_device_cu_count(idx)
        check(0 if n > 0 else n, "hk_device_cu_count")
        _cu_cache[idx] = n
    return _cu_cache[idx]


# Workspace budget of the fused-linear ops (hk_fused_linear_cross_entropy_workspace_size):
# 0 the default plan (the reference's chunk, fused_linear_cross_entropy.py:112-114),
# -1 no limit (the fastest plan), > 0 a byte budget.
BUDGET_ENV = "HILDA_FL_WORKSPACE_BUDGET"


def fl_budget(budget) -> int:
    """A workspace budget argument as the C ABI takes it: None reads $HILDA_FL_WORKSPACE_BUDGET (unset: 0);
    'default' 0; 'fastest' -1; an int is bytes (0 default, negative no limit)."""
    if budget is None:
        budget = os.environ.get(BUDGET_ENV, "0")
    if isinstance(budget, str):
        b = budget.strip().lower()
        if b in ("", "default"):
            return 0
        if b in ("fastest", "unlimited", "none"):
            return -1
        try:
            budget = int(float(b))
        except ValueError:
            raise ValueError(f"workspace budget {budget!r}: expected bytes, 'default' or 'fastest'") from None
    budget = int(budget)
    return -1 if budget < 0 else budget


def workspace(nbytes: int, what: str, device: torch.device) -> torch.Tensor:
    """A device workspace of nbytes (0 from a size query means no plan fits the budget)."""
    if int(nbytes) == 0:
        raise RuntimeError(f"{what}: no memory plan fits the workspace budget (or the shape is invalid): "
                           f"{last_error()}")
    return torch.empty(int(nbytes), dtype=torch.uint8, device=device)
