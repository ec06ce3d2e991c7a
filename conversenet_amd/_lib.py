"""ctypes binding of the C ABI in include/converse2d.h (libcvn_hip.so, built in-tree).

The library shares the HIP runtime already loaded by torch (same SONAME), so device pointers and
streams from torch tensors are valid arguments.  Loading fails loudly: there is no fallback.
"""
from __future__ import annotations

import ctypes
import os

import torch  # noqa: F401  (loads the HIP runtime the library binds to)

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("CVN_LIB", os.path.join(_HERE, "lib", "libcvn_hip.so"))

CVN_OK = 0
CVN_ERR_ARG = -1
CVN_ERR_UNSUPPORTED = -2
CVN_ERR_WORKSPACE = -3
CVN_ERR_HIP = -4

PAD_MODES = {"constant": 0, "zeros": 0, "reflect": 1, "replicate": 2, "circular": 3}
ROUTE_AUTO, ROUTE_FUSED, ROUTE_PFA268, ROUTE_GENERIC = 0, 1, 2, 3
ROUTE_OP_PLANNED = 4  # operator path on compile-time plans (cvn_converse2d_op_route)
NOALLOC_SCRATCH_BYTES = 64 << 20  # CVN_NOALLOC_SCRATCH_BYTES
ACT_NONE = 0
ACT_GELU = 1

_i64 = ctypes.c_int64
_int = ctypes.c_int
_f32 = ctypes.c_float
_ptr = ctypes.c_void_p
_size = ctypes.c_size_t

# name -> (restype, argtypes); mirrors include/converse2d.h
SIGNATURES = {
    "cvn_version": (ctypes.c_char_p, []),
    "cvn_last_error": (ctypes.c_char_p, []),
    "cvn_converse2d_fwd_workspace": (_size, [_i64, _i64, _i64, _i64, _i64, _int, _int, _int, _int]),
    "cvn_converse2d_fwd_f32": (_int, [_ptr, _i64, _i64, _i64, _i64, _ptr, _i64, _int, _int, _ptr, _f32, _int,
                                      _int, _int, _int, _ptr, _ptr, _size, _ptr]),
    "cvn_converse2d_fwd_noalloc_f32": (_int, [_ptr, _i64, _i64, _i64, _i64, _ptr, _i64, _int, _int, _ptr, _f32,
                                              _int, _int, _int, _int, _ptr, _ptr]),
    "cvn_converse2d_route": (_int, [_i64, _i64, _i64, _i64, _i64, _int, _int, _int, _int]),
    "cvn_converse2d_supported": (_int, [_i64, _i64, _i64, _i64, _i64, _int, _int, _int, _int, _int, _int]),
    "cvn_converse2d_table_bytes": (_size, [_i64, _i64, _i64, _i64, _i64, _int, _int, _int, _int, _int]),
    "cvn_converse2d_scratch_bytes": (_size, [_i64, _i64, _i64, _i64, _i64, _int, _int, _int, _int, _int]),
    "cvn_converse2d_table_f32": (_int, [_ptr, _i64, _int, _int, _ptr, _f32, _i64, _i64, _i64, _i64, _int, _int,
                                        _int, _ptr, _size, _ptr]),
    "cvn_converse2d_apply_f32": (_int, [_ptr, _i64, _i64, _i64, _i64, _i64, _int, _int, _int, _int, _int, _int,
                                        _int, _ptr, _size, _ptr, _size, _ptr, _ptr]),
    "cvn_converse2d_op_workspace": (_size, [_i64, _i64, _i64, _i64, _int, _int, _int]),
    "cvn_converse2d_op_f32": (_int, [_ptr, _ptr, _i64, _i64, _i64, _i64, _ptr, _int, _int, _ptr, _f32, _int, _ptr,
                                     _ptr, _size, _ptr]),
    "cvn_converse2d_op_route": (_int, [_i64, _i64, _int]),
    "cvn_converse2d_op_table_bytes": (_size, [_i64, _i64, _i64, _int, _int, _int]),
    "cvn_converse2d_op_scratch_bytes": (_size, [_i64, _i64, _i64, _i64, _int]),
    "cvn_converse2d_op_table_f32": (_int, [_ptr, _int, _int, _ptr, _f32, _i64, _i64, _i64, _int, _ptr, _size, _ptr]),
    "cvn_converse2d_op_apply_f32": (_int, [_ptr, _ptr, _i64, _i64, _i64, _i64, _int, _ptr, _size, _ptr, _size, _ptr,
                                           _ptr]),
    "cvn_converse2d_bwd_workspace": (_size, [_i64, _i64, _i64, _i64, _i64, _int, _int, _int, _int]),
    "cvn_converse2d_bwd_f32": (_int, [_ptr, _ptr, _i64, _i64, _i64, _i64, _ptr, _i64, _int, _int, _ptr, _f32, _int,
                                      _int, _int, _ptr, _ptr, _ptr, _ptr, _size, _ptr]),
    "cvn_clear_cache": (_int, []),
    "cvn_layernorm_cf_f32": (_int, [_ptr, _i64, _i64, _i64, _ptr, _ptr, _f32, _ptr, _ptr]),
    "cvn_conv1x1_f32": (_int, [_ptr, _i64, _i64, _i64, _ptr, _ptr, _i64, _int, _ptr, _ptr, _ptr, _ptr]),
    "cvn_ln_conv1x1_f32": (_int, [_ptr, _i64, _i64, _i64, _ptr, _ptr, _f32, _ptr, _ptr, _i64, _int, _ptr, _ptr,
                                  _ptr, _ptr]),
    "cvn_ln_mlp_residual_f32": (_int, [_ptr, _i64, _i64, _i64, _ptr, _ptr, _f32, _ptr, _ptr, _i64, _ptr, _ptr,
                                       _ptr, _ptr, _ptr]),
    "cvn_conv_ln_mlp_residual_f32": (_int, [_ptr, _int, _i64, _i64, _i64, _ptr, _ptr, _ptr, _ptr, _i64, _ptr,
                                            _ptr, _f32, _ptr, _ptr, _i64, _ptr, _ptr, _ptr, _ptr, _ptr]),
    "cvn_conv_ln_mlp_head_f32": (_int, [_ptr, _int, _i64, _i64, _i64, _ptr, _ptr, _ptr, _ptr, _i64, _ptr, _ptr, _f32,
                                        _ptr, _ptr, _i64, _ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _f32, _ptr, _ptr,
                                        _ptr, _ptr]),
    "cvn_copy_f32": (_int, [_ptr, _ptr, _i64, _ptr]),
}

_lib = None


def load():
    """Load libcvn_hip.so once and attach the C signatures.  Raises ImportError if it is missing."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"conversenet_amd: HIP library not found at {LIB_PATH}; build it with "
            "`python -m conversenet_amd.build` (or __graft_entry__.build())")
    lib = ctypes.CDLL(LIB_PATH, mode=ctypes.RTLD_GLOBAL)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def available() -> bool:
    try:
        load()
        return True
    except (ImportError, OSError):
        return False


def check(rc: int, what: str):
    if rc != CVN_OK:
        msg = _lib.cvn_last_error().decode(errors="replace")
        kind = {CVN_ERR_ARG: "invalid argument", CVN_ERR_UNSUPPORTED: "unsupported",
                CVN_ERR_WORKSPACE: "workspace", CVN_ERR_HIP: "HIP error"}.get(rc, f"error {rc}")
        raise RuntimeError(f"{what}: {kind}: {msg}")
