"""ctypes binding of the in-tree gfx950 library ``_lib/libfireprot_amd.so``.

Loading is lazy, guarded by a module ``threading.RLock`` and sticky on error,
as the reference's loaders are (python/fireprot/backends/amd/ck_attention.py:
27-78; extension.py:24-66).  Unlike the reference there is no build-on-demand
and no silent fallback here: ``library()`` raises when the library is absent,
so a GPU run without the native code fails loudly.  The capability predicates
in ``fireprot_amd.triangle_attention`` turn the same condition into a
registry rejection ("extension unavailable"), which falls back to the
*caller's* native function, exactly like the reference registry.
"""
from __future__ import annotations

import ctypes
import pathlib
import threading
from typing import Any

LIB_PATH = pathlib.Path(__file__).resolve().parent / "_lib" / "libfireprot_amd.so"
ABI_VERSION = 1

FPX_OK = 0
FPX_ERR_DIMS = 2
FPX_ERR_POINTER = 3
FPX_ERR_WORKSPACE = 4
FPX_F32 = 0
FPX_BF16 = 1

_p = ctypes.c_void_p
_i = ctypes.c_int
_i64 = ctypes.c_int64
_f = ctypes.c_float
_sz = ctypes.c_size_t

# name -> (restype, argtypes); mirrors include/fireprot_amd.h
SIGNATURES: dict[str, tuple[Any, list[Any]]] = {
    "fpx_abi_version": (_i, []),
    "fpx_tri_attn_workspace_bytes": (_sz, [_i, _i, _i, _i, _i]),
    "fpx_tri_attn_block": (_i, [
        _i, _p, _i64, _i64,          # dtype, z, z strides
        _p, _i64, _i64,              # mask, mask strides
        _p, _p, _f,                  # ln_w, ln_b, eps
        _p, _p, _p, _p, _p,          # w_qkvg, b_g, w_bias, w_o, b_o
        _f, _i, _i, _i, _i, _i,      # mask_inf, n, c, heads, head_dim, ending
        _p, _i64, _i64,              # dz, dz strides
        _p, _sz, _p,                 # workspace, bytes, stream
    ]),
    "fpx_tri_attn_block_residual": (_i, [
        _i, _p, _i64, _i64,          # dtype, z, z strides
        _p, _i64, _i64,              # mask, mask strides
        _p, _p, _f,                  # ln_w, ln_b, eps
        _p, _p, _p, _p, _p,          # w_qkvg, b_g, w_bias, w_o, b_o
        _f, _i, _i, _i, _i, _i,      # mask_inf, n, c, heads, head_dim, ending
        _p, _i64, _i64,              # z_out (may be z), strides
        _p, _sz, _p,                 # workspace, bytes, stream
    ]),
    "fpx_tri_attn_block_noalloc": (_i, [
        _i, _p, _i64, _i64,          # dtype, z, z strides
        _p, _i64, _i64,              # mask, mask strides
        _p, _p, _f,                  # ln_w, ln_b, eps
        _p, _p, _p, _p, _p,          # w_qkvg, b_g, w_bias, w_o, b_o
        _f, _i, _i, _i, _i, _i,      # mask_inf, n, c, heads, head_dim, ending
        _p, _i64, _i64,              # dz, dz strides
        _p,                          # stream (no workspace)
    ]),
    "fpx_tri_attn_prepare": (_i, [
        _i, _p, _i64, _i64, _p, _i64, _i64,   # dtype, z, strides, mask, strides
        _p, _p, _f, _p, _p, _p,               # ln_w, ln_b, eps, w_qkvg, b_g, w_bias
        _f, _i, _i, _p, _sz, _p,              # mask_inf, n, ending, workspace, bytes, stream
    ]),
    "fpx_tri_attn_attend": (_i, [_i, _i, _p, _sz, _p]),
    "fpx_tri_attn_finish": (_i, [_i, _p, _p, _i, _i, _p, _i64, _i64, _p, _sz, _p]),
    "fpx_attn_core": (_i, [_p, _p, _p, _p, _p, _i, _i, _p]),
    "ck_attention": (_i, [_p, _p, _p, _p, _p, _i, _i, _p]),
    "ck_attention_exact1536": (_i, [_p, _p, _p, _p, _p, _i, _i, _p]),
    "ck_attention_vector_bias1000": (_i, [_p, _p, _p, _p, _p, _i, _i, _p]),
    "fpx_attn_core_masked": (_i, [_p, _p, _p, _p, _i64, _p, _i64, _p, _i, _i, _p]),
    "fpx_attn_strided_workspace_bytes": (_sz, [_i, _i]),
    "fpx_attn_strided": (_i, [
        _p, _i64, _i64, _i64,        # q, strides (batch, head, row)
        _p, _i64, _i64, _i64,        # k
        _p, _i64, _i64, _i64,        # v
        _p, _i64, _i64,              # mask bias, strides (batch, key)
        _p, _i64, _i64, _i64,        # triangle bias, strides (head, query, key)
        _p, _i64, _i64, _i64,        # out
        _i, _i, _p, _sz, _p,         # batch, n, workspace, bytes, stream
    ]),
    "fpx_tri_mul_workspace_bytes": (_sz, [_i, _i, _i]),
    "fpx_tri_mul": (_i, [
        _p, _i64, _i64,              # z, strides
        _p, _i64, _i64,              # mask, strides
        _p, _p, _f,                  # ln_in_w, ln_in_b, eps_in
        _p, _p,                      # w_abpg [4][128][128], b_abpg [4][128]
        _p, _p, _f,                  # ln_out_w, ln_out_b, eps_out
        _p, _p, _p, _p,              # w_z, b_z, w_g, b_g
        _i, _i, _i, _i, _i,          # n, c_z, c_hidden, outgoing, accumulate
        _p, _i64, _i64,              # out (may be z), strides
        _p, _sz, _p,                 # workspace, bytes, stream
    ]),
    "fpx_transition_workspace_bytes": (_sz, [_i64, _i64, _i, _i]),
    "fpx_transition": (_i, [
        _p, _i64, _i64, _i64, _i64,  # x, rows_i, rows_j, strides
        _p, _p, _f,                  # ln_w, ln_b, eps
        _p, _p, _p,                  # w_a, w_b [512][128], w_o [128][512]
        _i, _i, _i,                  # c, expansion, accumulate
        _p, _i64, _i64,              # out (may be x), strides
        _p, _sz, _p,                 # workspace, bytes, stream
    ]),
    "fpx_layer_norm_c128": (_i, [_p, _i64, _i64, _i64, _i64, _p, _p, _f, _p, _p]),
    "fpx_qkv_projection": (_i, [_p, _i64, _p, _p, _p, _p, _p]),
    "fpx_sigmoid_mul_out": (_i, [_p, _p, _p, _i64, _p]),
    "fpx_split_planes": (_i, [_p, _i64, _p, _p]),
}

_lock = threading.RLock()
_library: ctypes.CDLL | None = None
_error: str | None = None


def library() -> ctypes.CDLL:
    """Return the loaded library, or raise ``RuntimeError`` saying why not."""
    global _library, _error
    with _lock:
        if _library is not None:
            return _library
        if _error is not None:
            raise RuntimeError(_error)
        try:
            if not LIB_PATH.exists():
                raise FileNotFoundError(
                    f"{LIB_PATH} is not built (run `python -m fireprot_amd.build`)")
            lib = ctypes.CDLL(str(LIB_PATH))
            for name, (restype, argtypes) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = restype
                fn.argtypes = argtypes
            if lib.fpx_abi_version() != ABI_VERSION:
                raise RuntimeError(
                    f"ABI mismatch: library {lib.fpx_abi_version()}, bindings {ABI_VERSION}")
        except Exception as error:  # sticky, like the reference loaders
            _error = f"fireprot_amd native library unavailable: {type(error).__name__}: {error}"
            raise RuntimeError(_error) from error
        _library = lib
        return lib


def available() -> bool:
    try:
        library()
        return True
    except RuntimeError:
        return False


def status() -> dict[str, Any]:
    with _lock:
        return {"path": str(LIB_PATH), "loaded": _library is not None, "error": _error}


def check(code: int, what: str) -> None:
    """Raise ``RuntimeError`` for a nonzero status, as ck_attention.py:139-140 does."""
    if code != FPX_OK:
        names = {FPX_ERR_DIMS: "unsupported sizes or layout",
                 FPX_ERR_POINTER: "null or misaligned pointer",
                 FPX_ERR_WORKSPACE: "workspace too small"}
        raise RuntimeError(f"{what} failed with status {code} ({names.get(code, 'HIP error')})")
