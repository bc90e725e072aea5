"""ctypes binding of libtabicl_attn.so (the C ABI declared in include/tabicl_attn.h).

The library is the only compute path: if it is missing or fails to load, every op raises
NativeLibraryError; nothing falls back to a CPU or pure-PyTorch implementation.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch

LIB_PATH = Path(os.environ.get("TABICL_ATTN_LIB", Path(__file__).resolve().parent / "libtabicl_attn.so"))

DTYPE_BF16 = 0
DTYPE_F32 = 1
OP_HX, OP_HXQ, OP_PK_SELF, OP_PK_CROSS, OP_ICL = range(5)

_c_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32
_f32 = ctypes.c_float

# name -> argtypes, in the order of include/tabicl_attn.h
SIGNATURES = {
    "tabicl_hx_fwd": [_c_p, _c_p, _c_p, _c_p, _i64, _c_p, _i64, _i64, _i64, _i64, _i32, _i32, _c_p],
    "tabicl_hxq_fwd": [_c_p, _i64, _c_p, _c_p, _c_p, _i64, _i64, _i64, _i64, _i32, _i32, _c_p, _i64, _c_p],
    "tabicl_hxq_workspace_bytes": [_i64, _i64, _i64, _i64, _i32, _i32],
    "tabicl_hxq_fwd_masked": [_c_p, _i64, _c_p, _i64, _c_p, _c_p, _c_p, _i64, _i64, _i64, _i64, _i32, _i32, _c_p,
                              _i64, _c_p],
    "tabicl_pk_self_fwd": [_c_p, _c_p, _i64, _c_p, _c_p, _c_p, _i64, _i64, _i64, _i32, _i32, _i32, _i32,
                           _f32, _i32, _c_p],
    "tabicl_pk_cross_fwd": [_c_p, _i64, _c_p, _c_p, _i64, _c_p, _c_p, _c_p, _c_p, _c_p, _i64, _i64, _i64,
                            _i64, _i32, _i32, _i32, _i32, _f32, _i32, _c_p],
    "tabicl_pk_cross_fwd_ragged": [_c_p, _i64, _c_p, _c_p, _i64, _c_p, _c_p, _c_p, _c_p, _c_p, _i64, _i64, _i64,
                                   _i64, _i32, _i32, _i32, _i32, _f32, _i32, _c_p, _i64, _c_p],
    "tabicl_hxf_fwd": [_c_p, _i64, _c_p, _i64, _c_p, _c_p, _i64, _i64, _i64, _i64, _i32, _c_p, _i64, _c_p],
    "tabicl_hxf_fwd_masked": [_c_p, _i64, _c_p, _i64, _c_p, _i64, _c_p, _c_p, _i64, _i64, _i64, _i64, _i32, _c_p,
                              _i64, _c_p],
    "tabicl_hxf_workspace_bytes": [_i64, _i64, _i64, _i64, _i32],
    "tabicl_smallhead_bwd_workspace_bytes": [_i64, _i64, _i64, _i32],
    "tabicl_hx_bwd": [_c_p, _c_p, _c_p, _c_p, _i64, _c_p, _c_p, _c_p, _c_p, _c_p, _i64, _i64, _i64, _i64, _i32,
                      _i32, _c_p, _i64, _c_p],
    "tabicl_pk_self_bwd": [_c_p, _c_p, _i64, _c_p, _c_p, _c_p, _c_p, _c_p, _i64, _i64, _i64, _i32, _i32, _i32,
                           _i32, _f32, _i32, _c_p, _i64, _c_p],
    "tabicl_pk_cross_bwd": [_c_p, _i64, _c_p, _c_p, _i64, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _i64,
                            _i64, _i64, _i64, _i32, _i32, _i32, _i32, _f32, _i32, _c_p, _i64, _c_p],
    "tabicl_icl_fwd": [_c_p, _c_p, _c_p, _c_p, _i64, _c_p, _i64, _i64, _i64, _i64, _i64] + [_i64] * 12
                      + [_f32, _i32, _c_p, _i64, _c_p],
    "tabicl_icl_fwd_ragged": [_c_p, _c_p, _c_p, _c_p, _i64, _c_p, _i64, _c_p, _i64, _i64, _i64, _i64, _i64]
                             + [_i64] * 12 + [_f32, _i32, _c_p, _i64, _c_p],
    "tabicl_icl_fwd_ragged_listed": [_c_p, _c_p, _c_p, _c_p, _i64, _c_p, _i64, _c_p, _i64, _i64, _i64, _i64, _i64]
                                    + [_i64] * 12 + [_f32, _i32, _c_p, _i64, _c_p],
    "tabicl_icl_ragged_plan": [_c_p, _i64, _i64, _i64, _i64, _i64, _i64, _i32, _c_p, _i64, _c_p],
    "tabicl_layer_norm": [_c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _i64, _i64, _f32, _i32, _i32, _c_p],
    "tabicl_icl_fwd_masked": [_c_p, _c_p, _c_p, _c_p, _i64, _c_p, _i64, _i64, _c_p, _i64, _c_p, _i64, _i64, _i64,
                              _i64, _i64] + [_i64] * 12 + [_f32, _i32, _c_p, _i64, _c_p],
    "tabicl_icl_bwd_workspace_bytes": [_i64, _i64, _i64],
    "tabicl_icl_bwd": [_c_p, _c_p, _c_p, _c_p, _i64, _c_p, _i64, _i64, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _i64,
                       _i64, _i64, _i64, _i64, _f32, _i32, _c_p, _i64, _c_p],
    "tabicl_icl_fwd_stats": [_c_p, _c_p, _c_p, _c_p, _i64, _c_p, _c_p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                             _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _f32, _i32, _c_p, _i64, _c_p],
    "tabicl_icl_fwd_noalloc": [_c_p, _c_p, _c_p, _c_p, _i64, _c_p, _i64, _i64, _c_p, _i64, _c_p, _i64, _i64, _i64,
                               _i64, _i64] + [_i64] * 12 + [_f32, _i32, _c_p],
    "tabicl_icl_noalloc_scratch_bytes": [],
    "tabicl_icl_workspace_bytes": [_i64, _i64, _i64, _i64, _i64, _i32],
    "tabicl_icl_cache_append": [_c_p, _c_p, _i64, _i64, _i64, _i64, _c_p, _c_p, _i64, _i64, _i64, _i64, _i64,
                                _i64, _i64, _i32, _c_p],
    "tabicl_attn_supported": [_i32, _i64, _i64, _i64, _i32, _i32],
    "tabicl_attn_last_error": [],
    "tabicl_attn_version": [],
}
_RESTYPES = {"tabicl_attn_last_error": ctypes.c_char_p, "tabicl_attn_version": ctypes.c_char_p,
             "tabicl_icl_workspace_bytes": ctypes.c_int64, "tabicl_hxq_workspace_bytes": ctypes.c_int64,
             "tabicl_smallhead_bwd_workspace_bytes": ctypes.c_int64, "tabicl_hxf_workspace_bytes": ctypes.c_int64,
             "tabicl_icl_noalloc_scratch_bytes": ctypes.c_int64, "tabicl_icl_bwd_workspace_bytes": ctypes.c_int64}


class NativeLibraryError(RuntimeError):
    """libtabicl_attn.so is missing or failed to load (there is no fallback compute path)."""


class UnsupportedShapeError(ValueError):
    """The library rejected the arguments (status > 0)."""


_LIB = None
_LOAD_ERROR: Exception | None = None


def load() -> ctypes.CDLL:
    """Load (once) and return the library; raises NativeLibraryError if it cannot be loaded."""
    global _LIB, _LOAD_ERROR
    if _LIB is not None:
        return _LIB
    if not LIB_PATH.exists():
        raise NativeLibraryError(f"{LIB_PATH} not found: build it with build_lib.py (hipcc, gfx950)")
    try:
        lib = ctypes.CDLL(str(LIB_PATH))
    except OSError as exc:  # pragma: no cover - depends on the host
        _LOAD_ERROR = exc
        raise NativeLibraryError(f"cannot load {LIB_PATH}: {exc}") from exc
    for name, argtypes in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = _RESTYPES.get(name, ctypes.c_int)
    _LIB = lib
    return lib


def available() -> bool:
    try:
        load()
        return True
    except NativeLibraryError:
        return False


def last_error() -> str:
    return load().tabicl_attn_last_error().decode()


def version() -> str:
    return load().tabicl_attn_version().decode()


def dtype_code(dt: torch.dtype) -> int:
    if dt == torch.bfloat16:
        return DTYPE_BF16
    if dt == torch.float32:
        return DTYPE_F32
    raise UnsupportedShapeError(f"dtype {dt} is not supported (bfloat16 or float32)")


def stream_of(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def aligned16(t: torch.Tensor) -> torch.Tensor:
    """t when it is contiguous and starts on a 16-byte boundary (what the entry points require of a
    key bias), else a contiguous copy in a fresh allocation (the caching allocator aligns those).
    `.contiguous()` alone returns a contiguous view that starts off the boundary unchanged. Under
    torch.compile (no storage address to test) always the copy."""
    if not torch.compiler.is_compiling() and t.is_contiguous() and t.data_ptr() % 16 == 0:
        return t
    return t.clone(memory_format=torch.contiguous_format)


def check(status: int, what: str) -> None:
    if status == 0:
        return
    msg = last_error()
    if status > 0:
        raise UnsupportedShapeError(f"{what}: {msg}")
    raise RuntimeError(f"{what}: HIP error {-status}: {msg}")


def call(name: str, *args) -> None:
    lib = load()
    check(getattr(lib, name)(*args), name)


@torch.compiler.assume_constant_result
def supported(op: int, Lq: int, Lk: int, E: int, h: int, dt: torch.dtype) -> bool:
    """Shape predicate of the library (pure host logic; needs the library loaded, no GPU). A trace
    (torch.compile) takes its value for the traced shapes as a constant, as the reference's pure-Python
    predicates are."""
    try:
        code = dtype_code(dt)
    except UnsupportedShapeError:
        return False
    return bool(load().tabicl_attn_supported(op, Lq, Lk, E, h, code))


def require_device(*ts: torch.Tensor | None) -> None:
    for t in ts:
        if t is not None and t.device.type != "cuda":
            raise NativeLibraryError(f"tensor on {t.device}: the HIP kernels need GPU tensors (no CPU path)")
