"""ctypes binding of libmx_qlinear.so (the C ABI declared in include/mx_qlinear.h).

The library is loaded lazily from this package directory. There is no fallback: if the
library is missing or a call fails, a RuntimeError (or ValueError for bad arguments)
is raised.
"""

from __future__ import annotations

import ctypes
import pathlib
import threading

LIB_PATH = pathlib.Path(__file__).resolve().parent / "libmx_qlinear.so"

MXQ_OK = 0
MXQ_ERR_INVALID = -1
MXQ_ERR_UNSUPPORTED = -2
MXQ_ERR_HIP = -3

DTYPE_F32, DTYPE_F16, DTYPE_BF16, DTYPE_E4M3 = 0, 1, 2, 5
ABI_VERSION = 5
# MXQ_GEMM_WORKSPACE_BYTES: the INT8 GEMMs' tile-queue workspace (counters)
GEMM_WORKSPACE_BYTES = 4096
ACT_NONE, ACT_GELU_TANH, ACT_SWIGLU = 0, 1, 2

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I = ctypes.c_int
_F = ctypes.c_float

# name -> argument types (every function returns int)
SIGNATURES: dict[str, list] = {
    "mxq_quantize_int8_rowwise": [_P, _I, _P, _P, _I64, _I64, _I, _P],
    "mxq_quantize_int8_rowwise_stochastic": [_P, _I, _P, _P, _P, _I64, _I64, _P],
    "mxq_quantize_int8_rowwise_absmax": [_P, _P, _P, _P, _I64, _I64, _P],
    "mxq_quantize_int8_rowwise_gelu": [_P, _P, _P, _P, _I64, _I64, _P],
    "mxq_adaln": [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _F, _P],
    "mxq_adaln_quantize_int8": [_P, _P, _P, _I64, _I64, _F, _P, _P, _P, _I64, _I64, _P],
    "mxq_int8_gemm_plan": [_I64, _I64, _I64, _I, _I64, _P],
    "mxq_int8_gemm_i32": [_P, _P, _P, _I64, _I64, _I64, _I64, _P, _I64, _P],
    "mxq_int8_gemm_dequant": [_P, _P, _P, _P, _I64, _P, _P, _I64, _I64, _I64, _I64, _I, _P, _I64, _P],
    "mxq_int8_gemm_dequant_gelu_absmax": [_P, _P, _P, _P, _I64, _P, _P, _P, _I64, _I64, _I64, _I64, _P, _I64,
                                          _P],
    "mxq_int8_gemm_dequant_swiglu": [_P, _P, _P, _P, _I64, _P, _P, _I64, _I64, _I64, _I64, _P, _I64, _P],
    "mxq_int8_gemm_gated_residual": [_P, _P, _P, _P, _I64, _P, _P, _I64, _P, _I64, _I64, _P, _I64, _I64, _I64,
                                     _P, _I64, _P],
    "mxq_fill_f32": [_P, _F, _I64, _P],
    "mxq_quantize_int8_rowwise_convrot": [_P, _I, _P, _P, _I64, _I64, _I64, _I, _P],
    "mxq_swiglu_bf16": [_P, _P, _I64, _I64, _P],
    "mxq_input_act_f16": [_P, _P, _I64, _I64, _I, _P],
    "mxq_adaln_quantize_int8_f16": [_P, _P, _P, _I64, _I64, _F, _P, _P, _P, _I64, _I64, _P],
    "mxq_int8_linear_m1": [_P, _P, _P, _I64, _P, _P, _I64, _I64, _I64, _I, _I, _P, _P, _P],
    "mxq_int8_gemv_dequant": [_P, _P, _P, _P, _I64, _P, _P, _I64, _I64, _I, _P],
    "mxq_rms_adaln_quantize_int8": [_P, _P, _P, _P, _I64, _I64, _P, _F, _P, _P, _P, _I64, _I64, _I64, _P, _I64, _P],
    "mxq_rms_adaln_quantize_int8_f16": [_P, _P, _P, _P, _I64, _I64, _P, _F, _P, _P, _P, _I64, _I64, _I64, _P],
    "mxq_gelu_tanh_bf16": [_P, _P, _I64, _P],
    "mxq_dequant_int4_grouped_to_int8": [_P, _P, _I, _P, _P, _I64, _I64, _I64, _P],
    "mxq_w4a8_codebook_gemm": [_P, _P, _P, _I, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I, _P, _I64,
                               _P],
    "mxq_w4a8_codebook_gemm_noalloc": [_P, _P, _P, _I, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I, _P],
    "mxq_w4a8_gemm_grouped": [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I, _P],
    "mxq_w4a8_gemm_grouped_prepared": [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I, _P],
    "mxq_w4a8_prepare_grouped": [_P, _P, _I64, _I64, _P],
    "mxq_probe_mfma_i8": [_P, _I64, _P, _I64, _P, _P, _I64, _I64, _P],
    "mxq_probe_lane_exchange": [_P, _P, _P, _P, _P],
    "mxq_w4a8_quantize_weight": [_P, _I, _I64, _I64, _I64, _I64, _I, _P, _I, _P, _P, _P, _P, _P, _P],
    "mxq_int8_group_sums": [_P, _P, _P, _I64, _I64, _I64, _I, _P],
}

_lib = None
_lock = threading.Lock()


class MxqError(RuntimeError):
    """A libmx_qlinear call failed (HIP error or unsupported request)."""


def load() -> ctypes.CDLL:
    """Load libmx_qlinear.so once; raise RuntimeError if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"{LIB_PATH} is missing: build it with __graft_entry__.build() or "
                    "`python -m mx_qlinear.build`; mx_qlinear has no CPU fallback"
                )
            lib = ctypes.CDLL(str(LIB_PATH))
            lib.mxq_last_error.restype = ctypes.c_char_p
            lib.mxq_last_error.argtypes = []
            lib.mxq_abi_version.restype = ctypes.c_int
            lib.mxq_abi_version.argtypes = []
            for name, args in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = ctypes.c_int
                fn.argtypes = args
            _lib = lib
    return _lib


def gemm_plan(m: int, n: int, k: int, table: int = 0, workspace_bytes: int = GEMM_WORKSPACE_BYTES) -> dict:
    """The INT8 GEMM launch plan (mxq_int8_gemm_plan): tile rows, workgroups, tiles, tiles per XCD
    claimed at run time (0: static order), workgroups per XCD, operand stages requested ahead,
    tile-rows per group of the tile order, whether the workgroups loop over tiles, tile columns.
    ``table``: 0 plain epilogues, 1 (or True) the GELU epilogue, 2 the SwiGLU one."""
    out = (ctypes.c_int64 * 9)()
    call("mxq_int8_gemm_plan", m, n, k, int(table), workspace_bytes, out)
    return {"tile": out[0], "grid": out[1], "tiles": out[2], "pool": out[3], "wg_per_xcd": out[4],
            "ahead": out[5], "group_m": out[6], "persistent": bool(out[7]), "tile_n": out[8]}


def call(name: str, *args) -> None:
    """Call ``name``; translate a non-zero return code into an exception."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != MXQ_OK:
        msg = lib.mxq_last_error().decode(errors="replace")
        if rc == MXQ_ERR_INVALID:
            raise ValueError(f"{name}: {msg}")
        raise MxqError(f"{name} failed ({rc}): {msg}")
