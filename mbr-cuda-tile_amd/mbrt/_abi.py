"""ctypes declarations of include/mbrt.h.

Loads lib/libmbrt.so from this package's source tree.  There is no fallback: if the
library is missing, importing raises (build it with `python mbr-cuda-tile_amd/build.py`).
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent.parent
LIB_PATH = PKG_DIR / "lib" / "libmbrt.so"

MAX_DIMS = 8

# dtype codes (src/tensor.h:17 values, plus I32)
F32, F16, I64, BF16, I32 = 0, 1, 2, 3, 4
# binary ops
ADD, SUB, MUL, DIV = 0, 1, 2, 3
SCALAR_ADD, SCALAR_MUL, SCALAR_CLAMP = 0, 1, 2
UNARY_NEG, UNARY_GT = 0, 1
REDUCE_SUM, REDUCE_MAX = 0, 1
ACT_NONE, ACT_GELU_REF, ACT_GELU_STD, ACT_SIGMOID, ACT_TANH = 0, 1, 2, 3, 4
LAYOUT_BHND, LAYOUT_BNHD = 0, 1
# arithmetic flags (mbrt_set_arith_flags)
ARITH_BF16_INTERMEDIATES = 1

STATUS_NAMES = {
    0: "MBRT_OK",
    1: "MBRT_E_INVALID_ARG",
    2: "MBRT_E_UNSUPPORTED_DTYPE",
    3: "MBRT_E_SHAPE",
    4: "MBRT_E_ALIGN",
    5: "MBRT_E_HIP",
}


class StridedMeta(C.Structure):
    _fields_ = [("src_strides", C.c_int64 * MAX_DIMS), ("dst_shape", C.c_int64 * MAX_DIMS), ("ndim", C.c_int32)]


class BroadcastMeta(C.Structure):
    _fields_ = [
        ("out_shape", C.c_int64 * MAX_DIMS),
        ("a_strides", C.c_int64 * MAX_DIMS),
        ("b_strides", C.c_int64 * MAX_DIMS),
        ("ndim", C.c_int32),
    ]


class PadMeta(C.Structure):
    _fields_ = [
        ("src_shape", C.c_int64 * MAX_DIMS),
        ("dst_shape", C.c_int64 * MAX_DIMS),
        ("pad_before", C.c_int64 * MAX_DIMS),
        ("ndim", C.c_int32),
    ]


class CatSrc(C.Structure):
    _fields_ = [("ptr", C.c_void_p), ("dim_size", C.c_int64), ("dim_offset", C.c_int64)]


P = C.c_void_p
I = C.c_int
L = C.c_int64
Fl = C.c_float
D = C.c_double

# name -> argtypes (all return int unless listed in _RESTYPE)
SIGNATURES: dict[str, list] = {
    "mbrt_last_error": [],
    "mbrt_version": [],
    "mbrt_stream_sync": [P],
    "mbrt_set_arith_flags": [C.c_uint32],
    "mbrt_get_arith_flags": [],
    "mbrt_fill": [P, I, L, D, P],
    "mbrt_arange": [P, I, L, L, P],
    "mbrt_convert": [P, I, P, I, L, P],
    "mbrt_scalar_op": [P, I, L, I, Fl, Fl, P],
    "mbrt_unary": [P, P, I, L, I, Fl, P],
    "mbrt_binary": [P, P, P, I, L, I, P],
    "mbrt_binary_broadcast": [P, P, P, I, C.POINTER(BroadcastMeta), I, P],
    "mbrt_strided_copy": [P, P, I, C.POINTER(StridedMeta), P],
    "mbrt_index_select": [P, P, I, P, I, L, L, C.POINTER(StridedMeta), I, P],
    "mbrt_pad_const": [P, P, I, C.POINTER(PadMeta), Fl, P],
    "mbrt_pad_reflect": [P, P, I, C.POINTER(PadMeta), P],
    "mbrt_cat": [P, C.POINTER(CatSrc), I, L, L, L, P],
    "mbrt_reduce_last_dim": [P, P, L, L, I, P],
    "mbrt_reduce_general": [P, P, L, L, L, I, P],
    "mbrt_rms_norm": [P, I, P, I, P, I, L, L, Fl, Fl, P],
    "mbrt_residual_add_rms_norm": [P, P, I, P, I, P, I, P, I, L, L, Fl, Fl, P],
    "mbrt_bias_act": [P, I, P, I, P, I, L, L, I, P],
    "mbrt_glu_last_dim": [P, I, P, I, L, L, P],
    "mbrt_sigmoid_gate_merge": [P, I, P, I, I, P, I, L, L, L, L, I, P],
    "mbrt_softmax_rows": [P, I, P, I, L, L, Fl, P],
    "mbrt_rotary_inplace": [P, P, I, P, P, I, L, L, L, L, I, P],
    "mbrt_split_qkv_heads_rotary": [P, I, P, P, I, P, P, P, I, L, L, L, L, L, P],
    "mbrt_band_gather": [P, P, I, P, I, L, L, L, L, P],
    "mbrt_band_mask_merge": [P, C.POINTER(P), I, I, P, P, I, P, I, P, I, L, L, L, L, L, P],
    "mbrt_zero_dc": [P, I, L, L, L, P],
    "mbrt_attention": [P, P, P, I, P, I, L, L, L, L, Fl, P],
    "mbrt_attention_strided": [P, P, P, I, L, L, L, L, L, L, L, L, L, L, L, P, P, I, P, I, I, P, I, Fl, P],
    "mbrt_attention_ex": [P, P, P, I, L, L, L, L, L, L, L, L, L, L, L, P, P, I, P, I, I, P, I, Fl, I, P],
    "mbrt_hann_window": [P, L, P],
    "mbrt_stft_num_frames": [L, L, I],
    "mbrt_stft": [P, P, P, L, L, L, L, L, L, I, I, P],
    "mbrt_istft_output_length": [L, L, I, L],
    "mbrt_istft_workspace_bytes": [L, L, L],
    "mbrt_istft": [P, I, P, P, L, L, L, L, L, L, L, I, I, L, P, L, P],
    "mbrt_istft_noalloc": [P, I, P, P, L, L, L, L, L, L, L, I, I, L, P],
    "mbrt_chunk_accumulate": [P, P, P, P, L, L, L, L, P],
    "mbrt_chunk_normalize": [P, P, L, L, P],
    "mbrt_chunk_fade_window": [P, L, L, I, I],
    "mbrt_mel_band_layout": [D, I, I, I, P, L, C.POINTER(C.c_int64), P],
    "mbrt_band_csr": [P, L, L, P, P, P, P],
    "mbrt_rotary_tables": [P, P, L, L, Fl],
}
_RESTYPE = {
    "mbrt_last_error": C.c_char_p,
    "mbrt_get_arith_flags": C.c_uint32,
    "mbrt_stft_num_frames": C.c_int64,
    "mbrt_istft_output_length": C.c_int64,
    "mbrt_istft_workspace_bytes": C.c_int64,
}


class MbrtError(RuntimeError):
    def __init__(self, fn: str, status: int, msg: str):
        super().__init__(f"{fn} -> {STATUS_NAMES.get(status, status)}: {msg}")
        self.status = status


def load(path: Path | str = LIB_PATH) -> C.CDLL:
    path = Path(path)
    if not path.exists():
        raise ImportError(f"mbrt: {path} is not built (run python mbr-cuda-tile_amd/build.py)")
    lib = C.CDLL(str(path))
    for name, argtypes in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = _RESTYPE.get(name, C.c_int)
    return lib


_LIB: C.CDLL | None = None


def lib() -> C.CDLL:
    global _LIB
    if _LIB is None:
        _LIB = load()
    return _LIB


def call(name: str, *args) -> None:
    """Call an entry point and raise MbrtError on a non-zero status."""
    lb = lib()
    st = getattr(lb, name)(*args)
    if st != 0:
        msg = lb.mbrt_last_error()
        raise MbrtError(name, st, msg.decode() if msg else "")
