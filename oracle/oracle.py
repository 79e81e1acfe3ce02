"""numpy wrapper of liboracle.so — TEST INFRASTRUCTURE ONLY (the oracle the GPU kernels
are held to; see oracle.h).  Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg import it.

Storage conventions: f32 -> np.float32; bf16 and f16 -> np.uint16 bit patterns;
indices -> np.int32 / np.int64.  Dtype codes match the C-ABI (F32=0, F16=1, I64=2,
BF16=3, I32=4).
"""
from __future__ import annotations

import ctypes as C
import math
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "liboracle.so"

F32, F16, I64, BF16, I32 = 0, 1, 2, 3, 4
EXACT, FAST, BF16I = 0, 1, 2

_NP = {F32: np.float32, F16: np.uint16, BF16: np.uint16, I64: np.int64, I32: np.int32}

_lib: C.CDLL | None = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB.exists():
            raise ImportError(f"oracle: {LIB} is not built (make -C oracle)")
        _lib = C.CDLL(str(LIB))
        _lib.orc_mel_bands.restype = C.c_int64
        _lib.orc_get_threads.restype = C.c_int
    return _lib


def _p(a):
    if a is None:
        return C.c_void_p(0)
    return a.ctypes.data_as(C.c_void_p)


def _i64arr(xs):
    return (C.c_int64 * max(len(xs), 1))(*xs)


L = C.c_int64


def set_threads(n: int) -> None:
    lib().orc_set_threads(int(n))


def empty(shape, dt) -> np.ndarray:
    return np.empty(shape, dtype=_NP[dt])


# ---- inputs / conversions ---------------------------------------------------------------

def randn(shape, seed: int, stream: int = 0, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    out = np.empty(shape, dtype=np.float32)
    lib().orc_randn(_p(out), L(out.size), C.c_uint64(seed), C.c_uint64(stream), C.c_double(mean), C.c_double(std))
    return out


def randu64(n: int, seed: int, stream: int = 0) -> np.ndarray:
    out = np.empty(n, dtype=np.uint64)
    lib().orc_randu64(_p(out), L(n), C.c_uint64(seed), C.c_uint64(stream))
    return out


def f32_to_bf16(a: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    out = np.empty(a.shape, dtype=np.uint16)
    lib().orc_f32_to_bf16(_p(a), _p(out), L(a.size))
    return out


def bf16_to_f32(a: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.uint16)
    out = np.empty(a.shape, dtype=np.float32)
    lib().orc_bf16_to_f32(_p(a), _p(out), L(a.size))
    return out


def f32_to_f16(a: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    out = np.empty(a.shape, dtype=np.uint16)
    lib().orc_f32_to_f16(_p(a), _p(out), L(a.size))
    return out


def f16_to_f32(a: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.uint16)
    out = np.empty(a.shape, dtype=np.float32)
    lib().orc_f16_to_f32(_p(a), _p(out), L(a.size))
    return out


def f64_to_bf16(a: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float64)
    out = np.empty(a.shape, dtype=np.uint16)
    lib().orc_f64_to_bf16(_p(a), _p(out), L(a.size))
    return out


def to_f32(a: np.ndarray, dt: int) -> np.ndarray:
    if dt == F32:
        return np.asarray(a, dtype=np.float32)
    if dt == BF16:
        return bf16_to_f32(a)
    if dt == F16:
        return f16_to_f32(a)
    return np.asarray(a, dtype=np.float32)


def from_f32(a: np.ndarray, dt: int) -> np.ndarray:
    if dt == F32:
        return np.ascontiguousarray(a, dtype=np.float32)
    if dt == BF16:
        return f32_to_bf16(a)
    if dt == F16:
        return f32_to_f16(a)
    raise ValueError(dt)


def convert(src: np.ndarray, sdt: int, ddt: int) -> np.ndarray:
    out = empty(src.shape, ddt)
    lib().orc_convert(_p(src), sdt, _p(out), ddt, L(src.size))
    return out


# ---- tensor library -----------------------------------------------------------------------

def binary(a, b, dt, op):
    out = empty(a.shape, dt)
    lib().orc_binary(_p(a), _p(b), _p(out), dt, L(a.size), op)
    return out


def binary_broadcast(a, b, dt, out_shape, a_strides, b_strides, op):
    out = empty(out_shape, dt)
    nd = len(out_shape)
    lib().orc_binary_broadcast(_p(a), _p(b), _p(out), dt, nd, _i64arr(out_shape), _i64arr(a_strides),
                               _i64arr(b_strides), op)
    return out


def strided_copy(src: np.ndarray, shape, strides) -> np.ndarray:
    """src: flat contiguous storage; returns the contiguous tensor of the strided view."""
    out = np.empty(shape, dtype=src.dtype)
    lib().orc_strided_copy(_p(src), _p(out), src.itemsize, len(shape), _i64arr(shape), _i64arr(strides))
    return out


def index_select(src: np.ndarray, out_shape, strides, sel: int, idx: np.ndarray) -> np.ndarray:
    idx = np.ascontiguousarray(idx, dtype=np.int64)
    out = np.empty(out_shape, dtype=src.dtype)
    lib().orc_index_select(_p(src), _p(out), src.itemsize, len(out_shape), _i64arr(out_shape), _i64arr(strides), sel,
                           _p(idx))
    return out


def pad(src, dt, dst_shape, before, value=0.0, reflect=False):
    out = empty(dst_shape, dt)
    lib().orc_pad(_p(src), _p(out), dt, src.ndim, _i64arr(src.shape), _i64arr(dst_shape), _i64arr(before),
                  C.c_float(value), 1 if reflect else 0)
    return out


def reduce_last(src, op, mode=EXACT):
    src = np.ascontiguousarray(src, dtype=np.float32)
    inner = src.shape[-1]
    out = np.empty(src.shape[:-1], dtype=np.float32)
    lib().orc_reduce_last(_p(src), _p(out), L(src.size // max(inner, 1)), L(inner), op, mode)
    return out


def reduce_general(src, dim, op):
    src = np.ascontiguousarray(src, dtype=np.float32)
    dim = dim % src.ndim
    outer = int(np.prod(src.shape[:dim], dtype=np.int64))
    inner = int(np.prod(src.shape[dim + 1:], dtype=np.int64))
    out = np.empty(src.shape[:dim] + src.shape[dim + 1:], dtype=np.float32)
    lib().orc_reduce_general(_p(src), _p(out), L(outer), L(src.shape[dim]), L(inner), op)
    return out


# ---- hot-path ops -------------------------------------------------------------------------

def rms_norm(x, xdt, gamma, gdt, odt, scale, eps, res=None, sdt=F32, mode=EXACT, want_sum=False):
    dim = x.shape[-1]
    rows = x.size // dim
    out = empty(x.shape, odt)
    sum_out = empty(x.shape, sdt) if (res is not None and want_sum) else None
    lib().orc_rms_norm(_p(x), xdt, _p(res), _p(gamma), gdt, _p(sum_out), sdt, _p(out), odt, L(rows), L(dim),
                       C.c_float(scale), C.c_float(eps), mode)
    return (out, sum_out) if want_sum else out


def bias_act(x, xdt, bias, bdt, odt, act, mode=EXACT):
    cols = x.shape[-1]
    out = empty(x.shape, odt)
    lib().orc_bias_act(_p(x), xdt, _p(bias), bdt, _p(out), odt, L(x.size // cols), L(cols), act, mode)
    return out


def glu(x, xdt, odt, mode=EXACT):
    full = x.shape[-1]
    out = empty(x.shape[:-1] + (full // 2,), odt)
    lib().orc_glu(_p(x), xdt, _p(out), odt, L(x.size // full), L(full // 2), mode)
    return out


def gate_merge(attn, adt, gate, gdt, odt, B, H, N, D, layout=0, logit=True, mode=EXACT):
    out = empty((B, N, H * D), odt)
    lib().orc_gate_merge(_p(attn), adt, _p(gate), gdt, 1 if logit else 0, _p(out), odt, L(B), L(H), L(N), L(D),
                         layout, mode)
    return out


def softmax(x, idt, odt, scale=1.0, mode=EXACT):
    cols = x.shape[-1]
    out = empty(x.shape, odt)
    lib().orc_softmax(_p(x), idt, _p(out), odt, L(x.size // cols), L(cols), C.c_float(scale), mode)
    return out


def rotary_tables(seq: int, dim_head: int, theta: float = 10000.0):
    cos = np.empty((seq, dim_head // 2), dtype=np.float32)
    sin = np.empty((seq, dim_head // 2), dtype=np.float32)
    lib().orc_rotary_tables(_p(cos), _p(sin), L(seq), L(dim_head), C.c_float(theta))
    return cos, sin


def rotary(q, k, dt, cos, sin, tdt, n_pos, heads, layout=0, mode=EXACT):
    """Returns rotated copies of q (and k)."""
    q = q.copy()
    k = k.copy() if k is not None else None
    D = q.shape[-1]
    lib().orc_rotary(_p(q), _p(k), dt, _p(cos), _p(sin), tdt, L(q.size // D), L(n_pos), L(heads), L(D), layout, mode)
    return q, k


def split_qkv(qkv, idt, cos, sin, tdt, odt, B, N, H, D, out_n, mode=EXACT):
    q = empty((B, H, out_n, D), odt)
    k = empty((B, H, out_n, D), odt)
    v = empty((B, H, out_n, D), odt)
    lib().orc_split_qkv(_p(qkv), idt, _p(cos), _p(sin), tdt, _p(q), _p(k), _p(v), odt, L(B), L(N), L(H), L(D),
                        L(out_n), mode)
    return q, k, v


def mel_bands(sr=44100.0, n_fft=2048, n_bands=60, channels=2):
    """Returns dict(freq_indices, freqs_per_band, bands_per_freq, csr_offsets, csr_indices) (int32)."""
    J = lib().orc_mel_bands(C.c_double(sr), n_fft, n_bands, channels, None, None, None, None, None)
    F = (n_fft // 2 + 1) * channels
    fi = np.empty(J, dtype=np.int32)
    fpb = np.empty(n_bands, dtype=np.int32)
    bpf = np.empty(F, dtype=np.int32)
    off = np.empty(F + 1, dtype=np.int32)
    ind = np.empty(J, dtype=np.int32)
    lib().orc_mel_bands(C.c_double(sr), n_fft, n_bands, channels, _p(fi), _p(fpb), _p(bpf), _p(off), _p(ind))
    return dict(freq_indices=fi, freqs_per_band=fpb, bands_per_freq=bpf, csr_offsets=off, csr_indices=ind)


def band_gather(stft, idx, odt, B, F, T):
    # indices outside [0, F) read the nearest valid row; clip before narrowing to int32
    idx = np.ascontiguousarray(np.clip(np.asarray(idx, dtype=np.int64), -1, F), dtype=np.int32)
    J = idx.size
    out = empty((B, T, J * 2), odt)
    lib().orc_band_gather(_p(stft), _p(idx), _p(out), odt, L(B), L(F), L(T), L(J))
    return out


def band_mask_merge(stft, masks, mdt, off, ind, cnt, cdt, odt, B, F, T, C_ch, mode=EXACT):
    off = np.ascontiguousarray(off, dtype=np.int32)
    ind = np.ascontiguousarray(ind, dtype=np.int32)
    S = len(masks)
    J = ind.size
    out = empty((B * S * C_ch, F // C_ch, T, 2), odt)
    arr = (C.c_void_p * S)(*[m.ctypes.data for m in masks])
    lib().orc_band_mask_merge(_p(stft), arr, mdt, S, _p(off), _p(ind), _p(cnt), cdt, _p(out), odt, L(B), L(F), L(T),
                              L(J), L(C_ch), mode)
    return out


def zero_dc(spec, dt):
    spec = spec.copy()
    outer, bins, T, _ = spec.shape
    lib().orc_zero_dc(_p(spec), dt, L(outer), L(bins), L(T))
    return spec


def attention(q, k, v, dt, odt, scale=0.0, mode=EXACT):
    """q [BH, nq, D], k and v [BH, nk, D] -> softmax(scale q k^T) v [BH, nq, D]."""
    BH, nq, D = q.shape
    nk = k.shape[1]
    out = empty((BH, nq, D), odt)
    lib().orc_attention(_p(q), _p(k), _p(v), dt, _p(out), odt, L(BH), L(nq), L(nk), L(D), C.c_float(scale), mode)
    return out


def attention_ref_p(q, k, v, dt, odt, scale=0.0, lazy=0.0, sum_rounded=False):
    """The attention with the reference's P arithmetic: running max per 64-key tile, P
    rounded once to bf16 for P V, row sum over the unrounded P (double elsewhere).  With
    lazy > 0 the running max moves only when a tile's max exceeds it by more than `lazy`
    (natural-log units); sum_rounded adds the rounded P to the row sum."""
    BH, nq, D = q.shape
    nk = k.shape[1]
    out = empty((BH, nq, D), odt)
    if lazy == 0.0 and not sum_rounded:
        lib().orc_attention_ref_p(_p(q), _p(k), _p(v), dt, _p(out), odt, L(BH), L(nq), L(nk), L(D), C.c_float(scale))
    else:
        lib().orc_attention_ref_p_ex(_p(q), _p(k), _p(v), dt, _p(out), odt, L(BH), L(nq), L(nk), L(D),
                                     C.c_float(scale), C.c_double(lazy), int(sum_rounded))
    return out


# the library's fast bf16-P mode: the running max moves by more than 8 in log2 units
ATTN_FAST_LAZY = 8.0 * math.log(2.0)


# ---- STFT / iSTFT, n_fft = win_length = 2048 (src/stft_cuda_tile.cu) ----------------------
# Restated in numpy float64: the frame DFT is evaluated with numpy's FFT (an exact-maths
# evaluator, pinned in tests against a direct O(N^2) DFT and torch.stft / torch.istft).

N_FFT = 2048
N_BINS = N_FFT // 2 + 1


def hann_window(size: int) -> np.ndarray:
    """src/stft_cuda_tile.cu:503-528: w[n] = 0.5 (1 - cos(n * (2 pi / size))), formed in f32
    (phase step and product rounded to f32 as the kernel does; cos rounded once)."""
    if size <= 0:
        return np.empty(0, np.float32)
    if size == 1:
        return np.ones(1, np.float32)
    step = np.float32(np.float32(6.28318530717958647692) / np.float32(size))
    phase = np.arange(size, dtype=np.float32) * step
    c = np.cos(phase.astype(np.float64)).astype(np.float32)
    return (np.float32(0.5) * (np.float32(1.0) - c)).astype(np.float32)


def hann_den(size: int) -> np.ndarray:
    """0.5 (1 + |cos|): the magnitude 1 - cos is a difference of."""
    if size <= 1:
        return np.ones(max(size, 0))
    step = np.float32(np.float32(6.28318530717958647692) / np.float32(size))
    phase = np.arange(size, dtype=np.float32) * step
    return 0.5 * (1.0 + np.abs(np.cos(phase.astype(np.float64))))


def stft_num_frames(length: int, hop: int, center: bool = True) -> int:
    """src/stft_cuda_tile.cu:544-551: T = (padded - n_fft) / hop + 1."""
    padded = length + (N_FFT if center else 0)
    return 0 if padded < N_FFT else (padded - N_FFT) // hop + 1


def stft_frames(x, hop: int, center: bool = True) -> np.ndarray:
    """Frames [B, T, 2048] (float64) of the signal, reflect-padded by n_fft/2 when centred
    (src/stft_cuda_tile.cu:544-548 with Tensor::pad_reflect's index rule,
    src/tensor_cuda_glue.cu:462-490: reflect once about the end samples, then clamp)."""
    x = np.asarray(x, np.float32)
    x = x.reshape(1, -1) if x.ndim == 1 else x
    B, Ls = x.shape
    off = N_FFT // 2 if center else 0
    T = stft_num_frames(Ls, hop, center)
    if T < 1:
        raise ValueError("signal shorter than n_fft")
    c = np.arange(T, dtype=np.int64)[:, None] * hop + np.arange(N_FFT, dtype=np.int64)[None, :] - off
    c = np.where(c < 0, -c, c)
    c = np.where(c >= Ls, 2 * (Ls - 1) - c, c)
    c = np.clip(c, 0, Ls - 1)
    return x[:, c].astype(np.float64)


def _stft_norm() -> float:
    return float(np.float32(1.0) / np.sqrt(np.float32(N_FFT)))


def stft(x, window, hop: int, center: bool = True, normalized: bool = False) -> np.ndarray:
    """src/stft_cuda_tile.cu:530-598: out[b, f, t] = sum_n frame_t[n] w[n] exp(-2 pi i f n / 2048)
    for f = 0..1024, as [B, 1025, T, 2] f32 (re, im), times the f32 1/sqrtf(2048) when
    normalized.  Exact in double, rounded once to f32."""
    fr = stft_frames(x, hop, center) * np.asarray(window, np.float64)[None, None, :]
    X = np.fft.rfft(fr, axis=-1)
    if normalized:
        X = X * _stft_norm()
    out = np.stack([X.real, X.imag], axis=-1).transpose(0, 2, 1, 3)
    return np.ascontiguousarray(out.astype(np.float32))


def stft_den(x, window, hop: int, center: bool = True, normalized: bool = False) -> np.ndarray:
    """sum_n |frame_t[n] w[n]| for every output of stft(): the magnitude each bin's sum of
    products is taken from, broadcast over bins and (re, im)."""
    fr = stft_frames(x, hop, center) * np.asarray(window, np.float64)[None, None, :]
    d = np.abs(fr).sum(-1) * (_stft_norm() if normalized else 1.0)  # [B, T]
    B, T = d.shape
    return np.broadcast_to(d[:, None, :, None], (B, N_BINS, T, 2))


def istft_output_length(frames: int, hop: int, center: bool = True, length: int = -1) -> int:
    """src/stft_cuda_tile.cu:623, 700-716."""
    if length > 0:
        return length
    full = N_FFT + (frames - 1) * hop
    return full - N_FFT if center else full


def _istft_frames(spec, dt, window, normalized):
    S = to_f32(np.asarray(spec), dt).astype(np.float64)
    if normalized:
        S = S * float(np.sqrt(np.float32(N_FFT)))
    X = (S[..., 0] + 1j * S[..., 1]).transpose(0, 2, 1)  # [B, T, 1025]
    return X


def _window_sum_f32(window, T: int, hop: int) -> np.ndarray:
    """src/stft_cuda_tile.cu:462-483: sum_t w[s - t hop]^2 in f32, frames in ascending order."""
    w = np.asarray(window, np.float32)
    ww = (w * w).astype(np.float32)
    full = N_FFT + (T - 1) * hop
    ws = np.zeros(full, np.float32)
    for t in range(T):
        sl = slice(t * hop, t * hop + N_FFT)
        ws[sl] = (ws[sl] + ww).astype(np.float32)
    return ws


def _finish(y, ws, T, hop, center, length):
    div = np.broadcast_to(ws[None, :] > np.float32(1e-8), y.shape)
    y = np.divide(y, np.broadcast_to(ws[None, :].astype(np.float64), y.shape), out=y.copy(), where=div)
    full = N_FFT + (T - 1) * hop
    if center:
        y = y[:, N_FFT // 2: full - N_FFT // 2]
    if length > 0:
        if length <= y.shape[1]:
            y = y[:, :length]
        else:
            y = np.concatenate([y, np.zeros((y.shape[0], length - y.shape[1]))], axis=1)
    return y


def istft(spec, dt, window, hop: int, center: bool = True, normalized: bool = False, length: int = -1) -> np.ndarray:
    """src/stft_cuda_tile.cu:600-717: per frame the real inverse DFT of the Hermitian
    extension (so the imaginary parts of bins 0 and 1024 drop out) divided by 2048, times
    the window; overlap-added at hop spacing; divided by the f32 window sum of squares where
    that exceeds 1e-8; centre trim of n_fft/2 at each end; `length` trims or zero-fills.
    Exact in double (except the f32 window sum, whose threshold test must match), rounded
    once to f32.  spec [B, 1025, T, 2] in dtype dt (F32 or BF16)."""
    X = _istft_frames(spec, dt, window, normalized)
    B, T, _ = X.shape
    fr = np.fft.irfft(X, n=N_FFT, axis=-1) * np.asarray(window, np.float64)[None, None, :]
    full = N_FFT + (T - 1) * hop
    y = np.zeros((B, full))
    for t in range(T):
        y[:, t * hop: t * hop + N_FFT] += fr[:, t]
    ws = _window_sum_f32(window, T, hop)
    return _finish(y, ws, T, hop, center, length).astype(np.float32)


def istft_den(spec, dt, window, hop: int, center: bool = True, normalized: bool = False,
              length: int = -1) -> np.ndarray:
    """Per output sample sum_t w[n_t] (|X_t[0]| + 2 sum_k |X_t[k]| + |X_t[1024]|) / 2048 (real
    parts at bins 0 and 1024), normalised and trimmed like istft(): the magnitude of the
    terms each sample is a sum of."""
    X = _istft_frames(spec, dt, window, normalized)
    B, T, _ = X.shape
    M = (np.abs(X[..., 0].real) + 2 * np.abs(X[..., 1:-1]).sum(-1) + np.abs(X[..., -1].real)) / N_FFT  # [B, T]
    w = np.abs(np.asarray(window, np.float64))
    full = N_FFT + (T - 1) * hop
    d = np.zeros((B, full))
    for t in range(T):
        d[:, t * hop: t * hop + N_FFT] += M[:, t:t + 1] * w[None, :]
    ws = _window_sum_f32(window, T, hop)
    return _finish(d, ws, T, hop, center, length)


# ---- chunk overlap-add (src/chunk_cuda_tile.cu, src/inference_app.cpp:72-232) --------------
# Restated in numpy float32 with the reference's rounding steps (a rounded product added to
# a rounded sum), so an ordered evaluation is reproduced bit for bit.

def chunk_fade_window(chunk_size: int, fade_size: int, first: bool = False, last: bool = False) -> np.ndarray:
    """src/inference_app.cpp:135-148, 201-210: ones with linear ramps i / (fade - 1) (f32)."""
    w = np.ones(chunk_size, np.float32)
    if fade_size == 1:
        if not first:
            w[0] = 0.0
        if not last:
            w[-1] = 0.0
    elif fade_size > 1:
        alpha = (np.arange(fade_size, dtype=np.float32) / np.float32(fade_size - 1)).astype(np.float32)
        if not first:
            w[:fade_size] = alpha
        if not last:
            w[chunk_size - fade_size:] = (np.float32(1.0) - alpha).astype(np.float32)
    return w


def chunk_accumulate(dest: np.ndarray, wsum: np.ndarray, src: np.ndarray, win: np.ndarray, offset: int) -> None:
    """src/chunk_cuda_tile.cu:18-42, in place: dest[c, off + i] += src[c, i] w[i]; wsum += w."""
    n = src.shape[-1]
    d = dest.reshape(-1, dest.shape[-1])
    s = np.asarray(src, np.float32).reshape(-1, n)
    w = np.asarray(win, np.float32)
    d[:, offset:offset + n] = (d[:, offset:offset + n] + (s * w).astype(np.float32)).astype(np.float32)
    wsum[offset:offset + n] = (wsum[offset:offset + n] + w).astype(np.float32)


def chunk_normalize(data: np.ndarray, wsum: np.ndarray) -> None:
    """src/chunk_cuda_tile.cu:44-58, in place: data /= wsum where wsum > 1e-8 (f32 division)."""
    d = data.reshape(-1, data.shape[-1])
    ok = wsum > np.float32(1e-8)
    q = np.divide(d, np.where(ok, wsum, np.float32(1.0))[None, :]).astype(np.float32)
    d[:] = np.where(ok[None, :], q, d)


def _reflect_pad_last(x: np.ndarray, before: int, after: int) -> np.ndarray:
    L = x.shape[-1]
    c = np.arange(-before, L + after)
    c = np.where(c < 0, -c, c)
    c = np.where(c >= L, 2 * (L - 1) - c, c)
    return x[..., np.clip(c, 0, L - 1)]


def process_chunked(audio: np.ndarray, chunk_size: int, step: int, chunk_batch_size: int, model_forward):
    """src/inference_app.cpp:72-232 step for step (model_forward: numpy [G, C, chunk] ->
    [G, ..., chunk]); audio [1, C, L] f32."""
    mix = np.asarray(audio, np.float32)
    length_init = mix.shape[-1]
    fade_size = chunk_size // 10
    border = chunk_size - step
    padded = length_init > 2 * border and border > 0
    if padded:
        mix = _reflect_pad_last(mix, border, border)
    total = mix.shape[-1]
    starts = list(range(0, total, step))
    count = len(starts)
    eff = max(1, min(chunk_batch_size, count))

    def prep(start, end):
        ch = mix[..., start:end]
        n = end - start
        if n < chunk_size:
            if n > chunk_size // 2:
                ch = _reflect_pad_last(ch, 0, chunk_size - n)
            else:
                ch = np.concatenate([ch, np.zeros(ch.shape[:-1] + (chunk_size - n,), np.float32)], axis=-1)
        return ch

    def group(g0, gs):
        ins = [prep(s, min(s + chunk_size, total)) for s in starts[g0:g0 + gs]]
        return np.asarray(model_forward(np.concatenate(ins, axis=0)), np.float32)

    first = group(0, min(eff, count))
    out_shape = (1,) + first.shape[1:-1] + (total,)
    fade = chunk_fade_window(chunk_size, fade_size)
    out = np.zeros(out_shape, np.float32)
    wsum = np.zeros(total, np.float32)
    C = out.size // total
    out2 = out.reshape(C, total)
    for g0 in range(0, count, eff):
        gs = min(eff, count - g0)
        bo = first if g0 == 0 else group(g0, gs)
        for local in range(gs):
            s = starts[g0 + local]
            e = min(s + chunk_size, total)
            n = e - s
            last = e >= total
            co = bo[local:local + 1][..., :n].reshape(C, n)
            win = fade
            if fade_size > 0 and (s == 0 or last):
                win = chunk_fade_window(chunk_size, fade_size, s == 0, last)
            chunk_accumulate(out2, wsum, co, win[:n], s)
    chunk_normalize(out2, wsum)
    out = out2.reshape(out_shape)
    if padded:
        out = out[..., border:border + length_init]
    return np.ascontiguousarray(out)
