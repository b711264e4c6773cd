"""ctypes binding of ``libpackbalance_amd.so`` (declared in ``include/packbalance_amd.h``).

This module is the only place that touches the C ABI.  It loads the in-tree
library, declares every entry point's signature, and turns status codes into
the exception types the reference raises (``ValueError`` for bad arguments,
``RuntimeError`` for unsupported sizes and launch failures).

There is no fallback: if the library is missing, every hot-path call raises.
"""

from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "libpackbalance_amd.so"

PB_OK = 0
PB_EINVAL = -1
PB_EUNSUPPORTED = -2
PB_EHIP = -3

PB_F32 = 0
PB_BF16 = 1
PB_F16 = 2

_DTYPES = {torch.float32: PB_F32, torch.bfloat16: PB_BF16, torch.float16: PB_F16}

_p = C.c_void_p
_i64 = C.c_int64
_i32 = C.c_int
_f32 = C.c_float


class BHSD(C.Structure):
    """``pb_bhsd``: a [B, H, S, D] view (element strides; D has unit stride)."""

    _fields_ = [("data", C.c_void_p), ("stride_b", C.c_int64), ("stride_h", C.c_int64),
                ("stride_s", C.c_int64)]

    @classmethod
    def of(cls, t: torch.Tensor) -> "BHSD":
        if t.dim() != 4 or t.stride(-1) != 1:
            raise ValueError("expected a [B, H, S, D] tensor with unit stride on D")
        return cls(t.data_ptr(), t.stride(0), t.stride(1), t.stride(2))


_pv = C.POINTER(BHSD)

# name -> (restype, argtypes).  Kept in the order of the header.
SIGNATURES: dict[str, tuple] = {
    "pb_last_error": (C.c_char_p, []),
    "pb_abi_version": (_i32, []),
    "pb_rmsnorm_fwd": (_i32, [_p, _i64, _i32, _p, _i32, _p, _i64, _p, _i64, _i64, _f32, _p]),
    "pb_rmsnorm_bwd_workspace_bytes": (_i64, [_i64, _i64]),
    "pb_rmsnorm_bwd": (
        _i32,
        [_p, _i64, _p, _i64, _i32, _p, _i32, _p, _p, _i64, _p, _p, _i64, _i64, _p],
    ),
    "pb_rmsnorm_bwd_noalloc": (
        _i32,
        [_p, _i64, _p, _i64, _i32, _p, _i32, _p, _p, _i64, _p, _i64, _i64, _p],
    ),
    "pb_swiglu_fwd": (_i32, [_p, _p, _p, _i64, _i32, _p]),
    "pb_swiglu_bwd": (_i32, [_p, _p, _p, _p, _p, _i64, _i32, _p]),
    "pb_swiglu_fwd_rows": (_i32, [_p, _i64, _p, _i64, _p, _i64, _i64, _i64, _i32, _p]),
    "pb_swiglu_bwd_rows": (_i32, [_p, _i64, _p, _i64, _p, _i64, _p, _i64, _p, _i64, _i64, _i64,
                                  _i32, _p]),
    "pb_ce_rows": (_i32, [_p, _i64, _i64, _i32, _p, _p, _p, _p, _i64, _i64, _i64, _f32, _p]),
    "pb_ce_rows_dl": (_i32, [_p, _i64, _i64, _i32, _p, _p, _p, _p, _i64, _i64, _i32, _i64, _i64,
                             _i64, _f32, _p]),
    "pb_doc_block_tables": (
        _i32,
        [_p, _i64, _i64, _i64, _i64, _i64, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p],
    ),
    "pb_attn_config": (_i32, [_i64, _i64, _i64, _i64, _i64, _p]),
    "pb_attn_plan": (_i32, [_p, _i64, _i64, _i64, _i64, _i64, _i32, _p, _p, _p, _p]),
    "pb_attn_fwd": (
        _i32,
        [_pv, _pv, _pv, _pv, _p, _p, _p, _i64, _p, _p, _i64, _i64, _i64, _i64, _i64, _f32, _i32,
         _p],
    ),
    "pb_attn_bwd": (
        _i32,
        [_pv, _pv, _pv, _pv, _pv, _pv, _pv, _pv, _p, _p, _p, _i64, _p, _p, _p, _p,
         _i64, _i64, _i64, _i64, _i64, _f32, _i32, _p],
    ),
    "pb_attn_bwd_f32_workspace_bytes": (_i64, [_i64, _i64, _i64, _i64, _i64]),
    "pb_attn_fwd_f32": (
        _i32, [_pv, _pv, _pv, _pv, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _f32, _p],
    ),
    "pb_attn_bwd_f32": (
        _i32,
        [_pv, _pv, _pv, _pv, _pv, _pv, _pv, _pv, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64,
         _f32, _p],
    ),
    "pb_lmhead_ce_workspace_bytes": (_i64, [_i64, _i64]),
    "pb_lmhead_ce_fwd": (
        _i32, [_p, _i64, _p, _i64, _i64, _i64, _i64, _p, _i64, _f32, _p, _p, _p, _p, _p],
    ),
    "pb_lmhead_ce_fwd_logits": (
        _i32,
        [_p, _i64, _p, _i64, _i64, _i64, _i64, _p, _i64, _f32, _p, _p, _p, _p, _i32, _p, _i64,
         _p],
    ),
    "pb_lmhead_ce_bwd_workspace_bytes": (_i64, [_i64, _i64, _i64, _i64]),
    "pb_lmhead_ce_bwd": (
        _i32,
        [_p, _i64, _p, _i64, _p, _i64, _p, _i64, _i64, _i64, _i64, _p, _i64, _f32, _p, _p,
         _i64, _p, _p, _i32, _i64, _p, _i32, _i64, _i32, _p],
    ),
    "pb_lmhead_ce_bwd_logits": (
        _i32,
        [_p, _i64, _p, _i64, _p, _i64, _p, _i64, _i64, _i64, _i64, _p, _i64, _f32, _p, _p,
         _i64, _p, _p, _i32, _i64, _p, _i32, _i64, _i32, _i32, _p, _i64, _p],
    ),
    "pb_lmhead_ce_dlogits": (
        _i32,
        [_p, _i64, _p, _i64, _i64, _i64, _i64, _p, _i64, _f32, _p, _p, _i64, _i64, _p, _i64, _p,
         _i64, _i32, _p, _i64, _p],
    ),
    "pb_pack_bf16": (_i32, [_p, _i32, _i64, _i64, _i64, _p, _i64, _i64, _i64, _i32, _p]),
    "pb_add_rmsnorm_fwd": (
        _i32,
        [_p, _i64, _i32, _p, _i64, _i32, _p, _i64, _p, _i32, _p, _i64, _i32, _p, _i64, _i64, _f32,
         _p],
    ),
    "pb_add_rmsnorm_bwd_workspace_bytes": (_i64, [_i64, _i64]),
    "pb_add_rmsnorm_bwd": (
        _i32,
        [_p, _i64, _i32, _p, _i64, _i32, _p, _i32, _p, _p, _i64, _p, _i64, _p, _i64, _i32, _p, _i32,
         _p, _i64, _i64, _p],
    ),
    "pb_add_rmsnorm_bwd_partials": (
        _i32,
        [_p, _i64, _i32, _p, _i64, _i32, _p, _i32, _p, _p, _i64, _p, _i64, _p, _i64, _i32, _p,
         _i64, _i64, _p],
    ),
    "pb_rmsnorm_dw_reduce_batched": (_i32, [_p, _i64, _p, _i64, _i64, _i64, _p]),
    "pb_pack_tensors": (
        _i32,
        [_p, _i32, _i64, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _p, _p, _p, _p, _p],
    ),
    "pb_clip_adamw_workspace_bytes": (_i64, [_i64]),
    "pb_clip_adamw_step": (
        _i32,
        [_p, _p, _i32, _i64, _p, _p, _p, _i32, _i64, _f32, _f32, _f32, _f32, _f32, _f32, _p, _p, _p,
         _p],
    ),
    "pb_rope_qk": (
        _i32,
        [_pv, _pv, _pv, _pv, _p, _i64, _i64, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i32,
         _i32, _p],
    ),
    "pb_transpose_batched": (_i32, [_p, _i64, _i64, _p, _i64, _i64, _i64, _i32, _p]),
}

ABI_VERSION = 4

_lib: C.CDLL | None = None
_load_error: str | None = None


def _load() -> C.CDLL | None:
    global _lib, _load_error
    if _lib is not None or _load_error is not None:
        return _lib
    if not LIB_PATH.exists():
        _load_error = (
            f"{LIB_PATH} is not built; run `python -m packbalance_amd.build` "
            "(or __graft_entry__.build())"
        )
        return None
    try:
        lib = C.CDLL(os.fspath(LIB_PATH))
    except OSError as exc:  # pragma: no cover - depends on the ROCm install
        _load_error = f"cannot load {LIB_PATH}: {exc}"
        return None
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if lib.pb_abi_version() != ABI_VERSION:
        _load_error = f"{LIB_PATH} has ABI {lib.pb_abi_version()}, expected {ABI_VERSION}; rebuild it"
        return None
    _lib = lib
    return _lib


def available() -> bool:
    """True when the native library is built and loadable (no GPU needed)."""
    return _load() is not None


def lib() -> C.CDLL:
    """The loaded library; raises RuntimeError when it is missing."""
    handle = _load()
    if handle is None:
        raise RuntimeError(f"packbalance_amd native library unavailable: {_load_error}")
    return handle


def check(status: int, what: str) -> None:
    if status == PB_OK:
        return
    msg = lib().pb_last_error().decode(errors="replace") or what
    if status == PB_EINVAL:
        raise ValueError(msg)
    raise RuntimeError(msg)


def call(name: str, *args) -> None:
    check(getattr(lib(), name)(*args), name)


def dtype_code(t: torch.Tensor) -> int:
    try:
        return _DTYPES[t.dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype {t.dtype}; expected float32, bfloat16 or float16") from None


def require_device(*tensors: torch.Tensor, op: str) -> None:
    """Hot-path ops run only on ROCm device tensors; anything else is an error."""
    for t in tensors:
        if not t.is_cuda:
            raise RuntimeError(
                f"{op}: packbalance_amd kernels need ROCm device tensors (got {t.device}); "
                "there is no CPU path"
            )
    lib()


def stream_ptr(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()
