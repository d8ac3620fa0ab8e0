"""ctypes binding of libxk_moe.so (the C ABI declared in include/xk_moe.h).

The library is loaded once, on first use; a missing or unloadable library raises
``RuntimeError`` — there is no fallback path. Every call goes through
``call(name, *args)``, which turns a nonzero status into ``RuntimeError`` carrying
``xk_last_error()``.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

ROOT_CSRC = Path(__file__).resolve().parent / "csrc"
LIB_PATH = Path(os.environ.get("XK_MOE_LIB", Path(__file__).resolve().parent / "_lib" / "libxk_moe.so"))

XK_OK = 0
XK_ERR_INVALID = 1
XK_ERR_WORKSPACE = 2
XK_ERR_LAUNCH = 3
XK_DT_BF16 = 0
XK_DT_FP32 = 1
XK_DT_FP16 = 2
XK_DT_NONE = -1
# Test-only bits of the int4 flags (csrc/int4_flags.h; not part of the ABI):
# pick the tile or the stream kernel where the shapes allow both.
_XK_INT4_TEST_FORCE_TILE = 1 << 8
_XK_INT4_TEST_FORCE_STREAM = 1 << 9

_p = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_f32 = ctypes.c_float

# name -> (restype, argtypes); must match include/xk_moe.h exactly.
SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "xk_last_error": (ctypes.c_char_p, []),
    "xk_abi_version": (ctypes.c_int, []),
    "xk_moe_align_workspace_bytes": (_i64, [_i64, _i32]),
    "xk_moe_align_block_size": (
        ctypes.c_int,
        [_p, _i64, _i32, _i32, _p, _i32, _p, _p, _p, _p, _p, _i64, _p],
    ),
    "xk_moe_sum_reduce": (ctypes.c_int, [_p, _i32, _i64, _i64, _i64, _p, _i32, _f32, _p, _p]),
    "xk_moe_int4_w4a16_workspace_bytes": (_i64, [_i64, _i64, _i64, _i64, _i64]),
    "xk_moe_int4_w4a16_ep_workspace_bytes": (_i64, [_i64, _i64, _i64, _i64, _i64, _i32]),
    "xk_moe_int4_w4a16": (
        ctypes.c_int,
        [_p, _i32, _i64, _i64, _p, _p, _i64, _i64, _i32, _p, _p, _i64, _p, _i32, _i32, _i32, _p,
         _p, _i64, _p],
    ),
    "xk_moe_topk_softmax": (ctypes.c_int, [_p, _i32, _i64, _i64, _i64, _i32, _p, _p, _p]),
    "xk_moe_int4_w4a16_noalloc_max_bytes": (_i64, []),
    "xk_moe_int4_w4a16_noalloc": (
        ctypes.c_int,
        [_p, _i32, _i64, _i64, _p, _p, _i64, _i64, _i32, _p, _p, _i64, _p, _i32, _i32, _i32, _p, _p],
    ),
    "xk_moe_int4_block_size": (_i32, [_i64, _i64, _i64]),
    "xk_moe_int4_w4a16_gemm": (
        ctypes.c_int,
        [_p, _i32, _i64, _i64, _p, _p, _i64, _i64, _i32, _p, _i64, _p, _i32, _p, _p, _p, _i32, _p,
         _i64, _p],
    ),
    "xk_moe_int4_gemm_workspace_bytes": (_i64, [_i64, _i64]),
    "xk_moe_topk_combine": (
        ctypes.c_int,
        [_p, _i64, _i64, _i64, _p, _i32, _p, _i32, _p, _i32, _p, _i32, _i32, _p],
    ),
    "xk_moe_int4_gemm_parts": (_i32, [_i64, _i64, _i64, _i64, _i64, _i32, _i32, _i32]),
    "xk_moe_int4_kernel": (_i32, [_i64, _i64, _i64, _i64, _i64, _i32, _i32, _i32, _i32]),
    "xk_moe_mxfp4_workspace_bytes": (_i64, [_i64, _i64, _i64, _i64, _i64]),
    "xk_moe_mxfp4": (
        ctypes.c_int,
        [_p, _i32, _i64, _i64, _p, _p, _p, _p, _i64, _i64, _p, _p, _f32, _i32, _p, _p, _i64, _p,
         _i32, _i32, _p, _p, _i64, _p],
    ),
}

_LIB: ctypes.CDLL | None = None


def load() -> ctypes.CDLL:
    """Load libxk_moe.so and declare every exported signature."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not LIB_PATH.exists():
        raise RuntimeError(
            f"libxk_moe.so not built at {LIB_PATH}; run `python -m xkernels_amd.build` "
            "(hipcc, gfx950)"
        )
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _LIB = lib
    return lib


def last_error() -> str:
    return (load().xk_last_error() or b"").decode(errors="replace")


def call(name: str, *args) -> None:
    """Invoke an entry point that returns a status; raise on failure."""
    rc = getattr(load(), name)(*args)
    if rc != XK_OK:
        raise RuntimeError(f"{name} failed (status {rc}): {last_error()}")


def query(name: str, *args) -> int:
    """Invoke a size query (no status)."""
    return int(getattr(load(), name)(*args))
