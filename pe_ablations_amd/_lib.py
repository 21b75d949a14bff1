"""ctypes binding of libpe_attn.so (include/pe_attn.h).

The library is loaded lazily from this package directory.  There is no fallback: when the library
is missing every entry point raises, so a run can never silently compute on another path.
"""

from __future__ import annotations

import ctypes
import os
import threading

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG_DIR, "libpe_attn.so")

PE_MODE_POPE, PE_MODE_ROPE, PE_MODE_NONE = 0, 1, 2
PE_DTYPE_BF16, PE_DTYPE_FP32, PE_DTYPE_FP16 = 0, 1, 2
PE_DTYPE_BOOL = 3  # explicit attention masks only
PE_CAUSAL_NONE, PE_CAUSAL_TOP_LEFT, PE_CAUSAL_BOTTOM_RIGHT = 0, 1, 2
PE_POS_EXACT, PE_POS_BF16, PE_POS_FP16 = 0, 1, 2

ERRORS = {
    "PE_OK": 0, "PE_ERR_NULL": -1, "PE_ERR_SHAPE": -2, "PE_ERR_HEAD_DIM": -3, "PE_ERR_MODE": -4,
    "PE_ERR_STRIDE": -5, "PE_ERR_WORKSPACE": -6, "PE_ERR_LAUNCH": -7, "PE_ERR_NO_DEVICE": -8,
    "PE_ERR_SCRATCH_LIMIT": -9,
}

# every symbol include/pe_attn.h declares
EXPORTED = [
    "pe_attn_check", "pe_attn_fwd_workspace_bytes", "pe_attn_bwd_workspace_bytes", "pe_attn_fwd",
    "pe_attn_bwd", "pe_attn_transform", "pe_attn_operand_width", "pe_attn_strerror", "pe_attn_version",
    "pe_attn_set_stage_events", "pe_attn_transform_bwd_workspace_bytes", "pe_attn_transform_bwd",
    "pe_attn_fwd_normed", "pe_rmsnorm_fwd", "pe_attn_fwd_noalloc", "pe_attn_noalloc_scratch_bytes",
    "pe_attn_value_width", "pe_attn_cache_append", "pe_attn_decode_workspace_bytes", "pe_attn_decode",
    "pe_swiglu_fwd", "pe_rmsnorm_bwd_workspace_bytes", "pe_rmsnorm_bwd", "pe_attn_fwd_masked",
    "pe_attn_bwd_masked", "pe_attn_bwd_masked_workspace_bytes",
]

# kernel stages bracketed by pe_attn_set_stage_events
STAGES = ["fwd_prep", "fwd_core", "bwd_pre", "bwd_dkdv", "bwd_dq", "bwd_inv"]


class PeTensor(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("dtype", ctypes.c_int32), ("reserved", ctypes.c_int32),
                ("stride", ctypes.c_int64 * 4)]


class PeParams(ctypes.Structure):
    _fields_ = [("B", ctypes.c_int32), ("Hq", ctypes.c_int32), ("Hkv", ctypes.c_int32),
                ("Sq", ctypes.c_int32), ("Sk", ctypes.c_int32),
                ("Dc", ctypes.c_int32), ("Dr", ctypes.c_int32), ("Dv", ctypes.c_int32),
                ("mode", ctypes.c_int32), ("dtype", ctypes.c_int32), ("causal", ctypes.c_int32),
                ("start_pos_q", ctypes.c_int32), ("start_pos_k", ctypes.c_int32),
                ("qk_l2norm", ctypes.c_int32),
                ("scale", ctypes.c_float), ("rope_mscale", ctypes.c_float),
                ("delta_head_stride", ctypes.c_int64),
                ("position_rounding", ctypes.c_int32), ("reserved", ctypes.c_int32)]


class PeNormParams(ctypes.Structure):
    _fields_ = [("q_weight", ctypes.c_void_p), ("k_weight", ctypes.c_void_p),
                ("weight_dtype", ctypes.c_int32), ("eps", ctypes.c_float)]


_lib = None
_lock = threading.Lock()


class PEAttnError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"{msg} (code {code})")
        self.code = code


def available() -> bool:
    return os.path.exists(LIB_PATH)


def lib():
    """The loaded library; raises when it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(
                    f"{LIB_PATH} is missing: build it with `python -m pe_ablations_amd.build` "
                    "(the fused PE attention has no non-HIP fallback)")
            L = ctypes.CDLL(LIB_PATH)
            P, T = ctypes.POINTER(PeParams), ctypes.POINTER(PeTensor)
            vp, fp, sz = ctypes.c_void_p, ctypes.POINTER(ctypes.c_float), ctypes.c_size_t
            L.pe_attn_check.argtypes = [P]
            L.pe_attn_check.restype = ctypes.c_int
            L.pe_attn_fwd_workspace_bytes.argtypes = [P]
            L.pe_attn_fwd_workspace_bytes.restype = sz
            L.pe_attn_bwd_workspace_bytes.argtypes = [P]
            L.pe_attn_bwd_workspace_bytes.restype = sz
            L.pe_attn_operand_width.argtypes = [P]
            L.pe_attn_operand_width.restype = ctypes.c_int
            L.pe_attn_fwd.argtypes = [P, T, T, T, T, T, vp, vp, T, vp, vp, sz, vp]
            L.pe_attn_fwd.restype = ctypes.c_int
            L.pe_attn_bwd.argtypes = [P, T, T, T, T, T, vp, vp, T, vp, T, T, T, T, T, T, vp, vp,
                                      vp, sz, vp, sz, vp]
            L.pe_attn_bwd.restype = ctypes.c_int
            L.pe_attn_fwd_masked.argtypes = [P, T, T, T, T, T, vp, vp, T, T, vp, vp, sz, vp]
            L.pe_attn_fwd_masked.restype = ctypes.c_int
            L.pe_attn_bwd_masked.argtypes = [P, T, T, T, T, T, vp, vp, T, T, vp, T, T, T, T, T, T, vp, vp,
                                             vp, sz, vp, sz, vp]
            L.pe_attn_bwd_masked.restype = ctypes.c_int
            L.pe_attn_bwd_masked_workspace_bytes.argtypes = [P]
            L.pe_attn_bwd_masked_workspace_bytes.restype = sz
            L.pe_attn_transform.argtypes = [P, ctypes.c_int, T, T, vp, vp, vp, vp]
            L.pe_attn_transform.restype = ctypes.c_int
            L.pe_attn_strerror.argtypes = [ctypes.c_int]
            L.pe_attn_strerror.restype = ctypes.c_char_p
            L.pe_attn_version.argtypes = []
            L.pe_attn_version.restype = ctypes.c_int
            L.pe_attn_transform_bwd_workspace_bytes.argtypes = [P, ctypes.c_int]
            L.pe_attn_transform_bwd_workspace_bytes.restype = sz
            L.pe_attn_transform_bwd.argtypes = [P, ctypes.c_int, vp, T, vp, vp, T, T, vp, vp, vp, sz, vp]
            L.pe_attn_transform_bwd.restype = ctypes.c_int
            L.pe_attn_fwd_normed.argtypes = [P, ctypes.POINTER(PeNormParams), T, T, T, T, T, vp, vp, T, vp,
                                             vp, sz, vp]
            L.pe_attn_fwd_normed.restype = ctypes.c_int
            i32, i64 = ctypes.c_int32, ctypes.c_int64
            L.pe_rmsnorm_fwd.argtypes = [vp, i32, i64, i64, i32, vp, i32, ctypes.c_float, vp, i32, i64, vp]
            L.pe_rmsnorm_fwd.restype = ctypes.c_int
            L.pe_rmsnorm_bwd_workspace_bytes.argtypes = [i64, i32]
            L.pe_rmsnorm_bwd_workspace_bytes.restype = sz
            L.pe_rmsnorm_bwd.argtypes = [vp, i32, i64, i64, i32, vp, i32, ctypes.c_float, vp, i64, vp, i64, vp,
                                         vp, sz, vp]
            L.pe_rmsnorm_bwd.restype = ctypes.c_int
            L.pe_swiglu_fwd.argtypes = [vp, vp, vp, i64, vp]
            L.pe_swiglu_fwd.restype = ctypes.c_int
            L.pe_attn_fwd_noalloc.argtypes = [P, T, T, T, T, T, vp, vp, T, vp, vp]
            L.pe_attn_fwd_noalloc.restype = ctypes.c_int
            L.pe_attn_noalloc_scratch_bytes.argtypes = []
            L.pe_attn_noalloc_scratch_bytes.restype = sz
            L.pe_attn_value_width.argtypes = [P]
            L.pe_attn_value_width.restype = ctypes.c_int
            L.pe_attn_cache_append.argtypes = [P, T, T, T, vp, vp, vp, vp, ctypes.c_int32, vp]
            L.pe_attn_cache_append.restype = ctypes.c_int
            L.pe_attn_decode_workspace_bytes.argtypes = [P]
            L.pe_attn_decode_workspace_bytes.restype = sz
            L.pe_attn_decode.argtypes = [P, T, T, vp, vp, ctypes.c_int32, vp, T, vp, vp, sz, vp]
            L.pe_attn_decode.restype = ctypes.c_int
            L.pe_attn_set_stage_events.argtypes = [vp]
            L.pe_attn_set_stage_events.restype = ctypes.c_int
            _lib = L
    return _lib


def check(code: int) -> None:
    if code != 0:
        raise PEAttnError(code, lib().pe_attn_strerror(code).decode())
