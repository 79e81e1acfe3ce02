"""Python binding of the mbrt C-ABI (include/mbrt.h) over torch device tensors.

torch provides device memory and the stream only; every computation is a call into
lib/libmbrt.so.  Each function enqueues on torch's current HIP stream (or `stream`).
"""
from __future__ import annotations

import ctypes as C
from typing import Sequence

import torch

from . import _abi
from ._abi import (  # noqa: F401
    ACT_GELU_REF, ACT_GELU_STD, ACT_NONE, ACT_SIGMOID, ACT_TANH, ADD, ARITH_BF16_INTERMEDIATES, BF16, DIV, F16, F32,
    I32, I64,
    LAYOUT_BHND, LAYOUT_BNHD, MUL, REDUCE_MAX, REDUCE_SUM, SCALAR_ADD, SCALAR_CLAMP, SCALAR_MUL, SUB,
    UNARY_GT, UNARY_NEG, MbrtError, lib, LIB_PATH,
)

_DT = {torch.float32: F32, torch.float16: F16, torch.int64: I64, torch.bfloat16: BF16, torch.int32: I32}


def dtype_code(t: torch.Tensor) -> int:
    try:
        return _DT[t.dtype]
    except KeyError as e:
        raise TypeError(f"mbrt: unsupported dtype {t.dtype}") from e


def _s(stream) -> C.c_void_p:
    if stream is None:
        stream = torch.cuda.current_stream()
    return C.c_void_p(stream.cuda_stream if hasattr(stream, "cuda_stream") else int(stream))


def _p(t: torch.Tensor | None) -> C.c_void_p:
    return C.c_void_p(t.data_ptr() if t is not None else 0)


def _contig(*ts: torch.Tensor) -> None:
    for t in ts:
        if t is not None and not t.is_contiguous():
            raise ValueError("mbrt: expected a contiguous tensor")


def version() -> int:
    return lib().mbrt_version()


def sync(stream=None) -> None:
    _abi.call("mbrt_stream_sync", _s(stream))


def get_arith_flags() -> int:
    return int(lib().mbrt_get_arith_flags())


def set_arith_flags(flags: int) -> None:
    """Arithmetic flags for later calls from this thread (ARITH_BF16_INTERMEDIATES: the
    reference's full-bf16 experiment mode, src/mbr_cuda_tile.cu:190-192)."""
    _abi.call("mbrt_set_arith_flags", int(flags))


class arith_flags:
    """Context manager: `with mbrt.arith_flags(mbrt.ARITH_BF16_INTERMEDIATES): ...`"""

    def __init__(self, flags: int):
        self.flags = flags

    def __enter__(self):
        self.prev = get_arith_flags()
        set_arith_flags(self.flags)
        return self

    def __exit__(self, *exc):
        set_arith_flags(self.prev)
        return False


# ---- tensor library --------------------------------------------------------------------

def fill_(t: torch.Tensor, value: float, stream=None) -> torch.Tensor:
    _contig(t)
    _abi.call("mbrt_fill", _p(t), dtype_code(t), t.numel(), float(value), _s(stream))
    return t


def arange_(t: torch.Tensor, start: int, stream=None) -> torch.Tensor:
    _contig(t)
    _abi.call("mbrt_arange", _p(t), dtype_code(t), t.numel(), int(start), _s(stream))
    return t


def convert(src: torch.Tensor, dst: torch.Tensor, stream=None) -> torch.Tensor:
    _contig(src, dst)
    _abi.call("mbrt_convert", _p(src), dtype_code(src), _p(dst), dtype_code(dst), src.numel(), _s(stream))
    return dst


def scalar_(t: torch.Tensor, op: int, a: float, b: float = 0.0, stream=None) -> torch.Tensor:
    _contig(t)
    _abi.call("mbrt_scalar_op", _p(t), dtype_code(t), t.numel(), op, a, b, _s(stream))
    return t


def unary(src: torch.Tensor, dst: torch.Tensor, op: int, value: float = 0.0, stream=None) -> torch.Tensor:
    _contig(src, dst)
    _abi.call("mbrt_unary", _p(src), _p(dst), dtype_code(src), src.numel(), op, value, _s(stream))
    return dst


def binary(a: torch.Tensor, b: torch.Tensor, out: torch.Tensor, op: int, stream=None) -> torch.Tensor:
    _contig(a, b, out)
    _abi.call("mbrt_binary", _p(a), _p(b), _p(out), dtype_code(a), a.numel(), op, _s(stream))
    return out


def broadcast_meta(a_shape, a_strides, b_shape, b_strides):
    """Right-aligned broadcasting metadata (src/tensor.cu:548-580)."""
    nd = max(len(a_shape), len(b_shape))
    m = _abi.BroadcastMeta()
    m.ndim = nd
    out_shape = []
    for d in range(nd):
        ai, bi = len(a_shape) - nd + d, len(b_shape) - nd + d
        sa = a_shape[ai] if ai >= 0 else 1
        sb = b_shape[bi] if bi >= 0 else 1
        if sa != sb and sa != 1 and sb != 1:
            raise ValueError("broadcast: incompatible shapes")
        out_shape.append(max(sa, sb))
        m.out_shape[d] = out_shape[-1]
        m.a_strides[d] = a_strides[ai] if (ai >= 0 and sa != 1) else 0
        m.b_strides[d] = b_strides[bi] if (bi >= 0 and sb != 1) else 0
    return m, out_shape


def binary_broadcast(a: torch.Tensor, b: torch.Tensor, out: torch.Tensor, op: int, stream=None) -> torch.Tensor:
    m, shape = broadcast_meta(list(a.shape), list(a.stride()), list(b.shape), list(b.stride()))
    if list(out.shape) != shape or not out.is_contiguous():
        raise ValueError("binary_broadcast: out must be contiguous with the broadcast shape")
    _abi.call("mbrt_binary_broadcast", _p(a), _p(b), _p(out), dtype_code(out), C.byref(m), op, _s(stream))
    return out


def strided_meta(shape: Sequence[int], strides: Sequence[int]) -> _abi.StridedMeta:
    m = _abi.StridedMeta()
    m.ndim = len(shape)
    for d, (n, s) in enumerate(zip(shape, strides)):
        m.dst_shape[d] = n
        m.src_strides[d] = s
    return m


def strided_copy(src: torch.Tensor, dst: torch.Tensor, stream=None) -> torch.Tensor:
    """dst (contiguous) = src (any strided view), e.g. x.permute(...) -> contiguous."""
    _contig(dst)
    if list(dst.shape) != list(src.shape):
        raise ValueError("strided_copy: shape mismatch")
    m = strided_meta(src.shape, src.stride())
    _abi.call("mbrt_strided_copy", _p(src), _p(dst), dtype_code(src), C.byref(m), _s(stream))
    return dst


def index_select(src: torch.Tensor, dim: int, idx: torch.Tensor, out: torch.Tensor, stream=None) -> torch.Tensor:
    _contig(idx, out)
    dim = dim % src.dim()
    m = strided_meta(out.shape, src.stride())
    _abi.call("mbrt_index_select", _p(src), _p(out), dtype_code(src), _p(idx), dtype_code(idx), idx.numel(),
              src.shape[dim], C.byref(m), dim, _s(stream))
    return out


def pad(src: torch.Tensor, out: torch.Tensor, before: Sequence[int], value: float = 0.0, reflect: bool = False,
        stream=None) -> torch.Tensor:
    _contig(src, out)
    m = _abi.PadMeta()
    m.ndim = src.dim()
    for d in range(src.dim()):
        m.src_shape[d] = src.shape[d]
        m.dst_shape[d] = out.shape[d]
        m.pad_before[d] = before[d]
    if reflect:
        _abi.call("mbrt_pad_reflect", _p(src), _p(out), dtype_code(src), C.byref(m), _s(stream))
    else:
        _abi.call("mbrt_pad_const", _p(src), _p(out), dtype_code(src), C.byref(m), float(value), _s(stream))
    return out


def cat(srcs: Sequence[torch.Tensor], dim: int, out: torch.Tensor, stream=None) -> torch.Tensor:
    _contig(out, *srcs)
    dim = dim % out.dim()
    outer = 1
    for d in range(dim):
        outer *= out.shape[d]
    inner = 1
    for d in range(dim + 1, out.dim()):
        inner *= out.shape[d]
    arr = (_abi.CatSrc * len(srcs))()
    off = 0
    for i, s in enumerate(srcs):
        arr[i].ptr = s.data_ptr()
        arr[i].dim_size = s.shape[dim]
        arr[i].dim_offset = off
        off += s.shape[dim]
    _abi.call("mbrt_cat", _p(out), arr, len(srcs), outer, out.shape[dim], inner * out.element_size(), _s(stream))
    return out


def reduce_last(src: torch.Tensor, dst: torch.Tensor, op: int, stream=None) -> torch.Tensor:
    _contig(src, dst)
    inner = src.shape[-1]
    outer = src.numel() // max(inner, 1)
    _abi.call("mbrt_reduce_last_dim", _p(src), _p(dst), outer, inner, op, _s(stream))
    return dst


def reduce_general(src: torch.Tensor, dst: torch.Tensor, dim: int, op: int, stream=None) -> torch.Tensor:
    _contig(src, dst)
    dim = dim % src.dim()
    outer = 1
    for d in range(dim):
        outer *= src.shape[d]
    inner = 1
    for d in range(dim + 1, src.dim()):
        inner *= src.shape[d]
    _abi.call("mbrt_reduce_general", _p(src), _p(dst), outer, src.shape[dim], inner, op, _s(stream))
    return dst


# ---- hot-path ops -----------------------------------------------------------------------

def rms_norm(x: torch.Tensor, gamma: torch.Tensor, out: torch.Tensor, scale: float, eps: float = 1e-12,
             stream=None) -> torch.Tensor:
    _contig(x, gamma, out)
    dim = x.shape[-1]
    _abi.call("mbrt_rms_norm", _p(x), dtype_code(x), _p(gamma), dtype_code(gamma), _p(out), dtype_code(out),
              x.numel() // dim, dim, scale, eps, _s(stream))
    return out


def residual_add_rms_norm(residual: torch.Tensor, update: torch.Tensor, gamma: torch.Tensor,
                          sum_out: torch.Tensor | None, normed: torch.Tensor, scale: float, eps: float = 1e-12,
                          stream=None) -> torch.Tensor:
    _contig(residual, update, gamma, sum_out, normed)
    dim = residual.shape[-1]
    sdt = dtype_code(sum_out) if sum_out is not None else dtype_code(residual)
    _abi.call("mbrt_residual_add_rms_norm", _p(residual), _p(update), dtype_code(residual), _p(gamma),
              dtype_code(gamma), _p(sum_out), sdt, _p(normed), dtype_code(normed), residual.numel() // dim, dim,
              scale, eps, _s(stream))
    return normed


def bias_act(x: torch.Tensor, bias: torch.Tensor | None, out: torch.Tensor, act: int, stream=None) -> torch.Tensor:
    _contig(x, bias, out)
    cols = x.shape[-1]
    _abi.call("mbrt_bias_act", _p(x), dtype_code(x), _p(bias), dtype_code(bias) if bias is not None else F32, _p(out),
              dtype_code(out), x.numel() // cols, cols, act, _s(stream))
    return out


def glu(x: torch.Tensor, out: torch.Tensor, stream=None) -> torch.Tensor:
    _contig(x, out)
    full = x.shape[-1]
    if full % 2:
        raise ValueError("glu_last_dim: last dimension must be even")
    _abi.call("mbrt_glu_last_dim", _p(x), dtype_code(x), _p(out), dtype_code(out), x.numel() // full, full // 2,
              _s(stream))
    return out


def gate_merge(attn: torch.Tensor, gate: torch.Tensor, out: torch.Tensor, layout: int = LAYOUT_BHND,
               gate_is_logit: bool = True, stream=None) -> torch.Tensor:
    """attn [B,H,N,D] (BHND) or [B,N,H,D] (BNHD); gate [B,N,H]; out [B,N,H*D]."""
    _contig(attn, gate, out)
    if layout == LAYOUT_BHND:
        B, H, N, D = attn.shape
    else:
        B, N, H, D = attn.shape
    _abi.call("mbrt_sigmoid_gate_merge", _p(attn), dtype_code(attn), _p(gate), dtype_code(gate),
              1 if gate_is_logit else 0, _p(out), dtype_code(out), B, H, N, D, layout, _s(stream))
    return out


def softmax(x: torch.Tensor, out: torch.Tensor, scale: float = 1.0, stream=None) -> torch.Tensor:
    _contig(x, out)
    cols = x.shape[-1]
    _abi.call("mbrt_softmax_rows", _p(x), dtype_code(x), _p(out), dtype_code(out), x.numel() // cols, cols, scale,
              _s(stream))
    return out


def rotary_(q: torch.Tensor, k: torch.Tensor | None, cos: torch.Tensor, sin: torch.Tensor,
            layout: int = LAYOUT_BHND, heads: int = 1, stream=None) -> None:
    """In place. BHND: q [B*H, N, D]; BNHD: q [B, N, H, D]; cos/sin [N, D/2]."""
    _contig(q, k, cos, sin)
    D = q.shape[-1]
    n_pos = cos.shape[0]
    _abi.call("mbrt_rotary_inplace", _p(q), _p(k), dtype_code(q), _p(cos), _p(sin), dtype_code(cos),
              q.numel() // D, n_pos, heads, D, layout, _s(stream))


def split_qkv_rotary(qkv: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, q: torch.Tensor, k: torch.Tensor,
                     v: torch.Tensor, heads: int, stream=None) -> None:
    _contig(qkv, cos, sin, q, k, v)
    B, N, three_hd = qkv.shape
    D = three_hd // (3 * heads)
    out_n = q.shape[2]
    _abi.call("mbrt_split_qkv_heads_rotary", _p(qkv), dtype_code(qkv), _p(cos), _p(sin), dtype_code(cos), _p(q),
              _p(k), _p(v), dtype_code(q), B, N, heads, D, out_n, _s(stream))


def band_gather(stft: torch.Tensor, idx: torch.Tensor, out: torch.Tensor, stream=None) -> torch.Tensor:
    """stft [B, F, T, 2] f32; idx [J]; out [B, T, J*2]."""
    _contig(stft, idx, out)
    B, F, T, _ = stft.shape
    _abi.call("mbrt_band_gather", _p(stft), _p(idx), dtype_code(idx), _p(out), dtype_code(out), B, F, T, idx.numel(),
              _s(stream))
    return out


def band_mask_merge(stft: torch.Tensor, masks: Sequence[torch.Tensor], offsets: torch.Tensor,
                    indices: torch.Tensor, counts: torch.Tensor, out: torch.Tensor, channels: int,
                    stream=None) -> torch.Tensor:
    """stft [B, F, T, 2] f32; masks: 1-2 of [B, T, J*2]; out [B*S*C, F/C, T, 2]."""
    _contig(stft, offsets, indices, counts, out, *masks)
    B, F, T, _ = stft.shape
    J = indices.numel()
    arr = (C.c_void_p * 2)(*[m.data_ptr() for m in masks], *([0] * (2 - len(masks))))
    _abi.call("mbrt_band_mask_merge", _p(stft), arr, dtype_code(masks[0]), len(masks), _p(offsets), _p(indices),
              dtype_code(offsets), _p(counts), dtype_code(counts), _p(out), dtype_code(out), B, F, T, J, channels,
              _s(stream))
    return out


def zero_dc(spec: torch.Tensor, stream=None) -> torch.Tensor:
    """spec [outer, bins, T, 2]: bin 0 := 0 in place."""
    _contig(spec)
    outer, bins, T, _ = spec.shape
    _abi.call("mbrt_zero_dc", _p(spec), dtype_code(spec), outer, bins, T, _s(stream))
    return spec


ATTN_P_PAIR, ATTN_P_BF16, ATTN_P_BF16_FAST = 0, 1, 2  # enum mbrt_attn_precision


def _p_precision(p_bf16: bool, p_precision: int | None) -> int:
    if p_precision is None:
        return ATTN_P_BF16 if p_bf16 else ATTN_P_PAIR
    if p_bf16 and p_precision != ATTN_P_BF16:
        raise ValueError("attention: p_bf16 and p_precision disagree")
    return int(p_precision)


def attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, out: torch.Tensor, scale: float = 0.0,
              p_bf16: bool = False, stream=None, p_precision: int | None = None) -> torch.Tensor:
    """Fused attention: q [BH, nq, 64], k, v [BH, nk, 64] bf16 -> out [BH, nq, 64] (bf16/f32).
    p_bf16 selects the reference's arithmetic (P rounded once to bf16 for P V);
    p_precision one of ATTN_P_PAIR / ATTN_P_BF16 / ATTN_P_BF16_FAST."""
    for t in (q, k, v, out):
        _contig(t)
    BH, nq, D = q.shape
    nk = k.shape[1]
    pm = _p_precision(p_bf16, p_precision)
    if pm == ATTN_P_PAIR:
        _abi.call("mbrt_attention", _p(q), _p(k), _p(v), dtype_code(q), _p(out), dtype_code(out), BH, nq, nk, D,
                  float(scale), _s(stream))
    else:
        _abi.call("mbrt_attention_ex", _p(q), _p(k), _p(v), dtype_code(q), BH, 1, nq, nk, D, nq * D, 0, D,
                  nk * D, 0, D, None, None, F32, None, F32, 0, _p(out), dtype_code(out), float(scale),
                  pm, _s(stream))
    return out


def attention_bnhd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, out: torch.Tensor | None = None,
                   scale: float = 0.0, cos: torch.Tensor | None = None, sin: torch.Tensor | None = None,
                   gate: torch.Tensor | None = None, gate_is_logit: bool = True, out_dtype=None,
                   p_bf16: bool = False, stream=None, p_precision: int | None = None) -> torch.Tensor:
    """Fused attention over [B, N, H, 64] bf16 views (any strides with a unit last dim, e.g.
    slices of a fused qkv projection).  cos, sin [n_q, 32] rotate q in-kernel.  Without a
    gate the result is [B, H, n_q, 64]; with gate [B, n_q, H] it is the gated head merge
    [B, n_q, H*64].  out_dtype defaults to bf16."""
    B, nq, H, D = q.shape
    nk = k.shape[1]
    if k.shape != (B, nk, H, D) or v.shape != k.shape:
        raise ValueError("attention_bnhd: expected q [B, N, H, D] and k, v [B, N_k, H, D]")
    if q.stride(3) != 1 or k.stride(3) != 1 or v.stride(3) != 1 or k.stride() != v.stride():
        raise ValueError("attention_bnhd: the last dim must be contiguous and k, v strided alike")
    odt = out_dtype if out_dtype is not None else (out.dtype if out is not None else torch.bfloat16)
    if out is None:
        shape = (B, nq, H * D) if gate is not None else (B, H, nq, D)
        out = torch.empty(shape, dtype=odt, device=q.device)
    _contig(out)
    for t in (cos, sin, gate):
        if t is not None:
            _contig(t)
    _abi.call("mbrt_attention_ex", _p(q), _p(k), _p(v), dtype_code(q), B, H, nq, nk, D,
              q.stride(0), q.stride(2), q.stride(1), k.stride(0), k.stride(2), k.stride(1),
              _p(cos) if cos is not None else None, _p(sin) if sin is not None else None,
              dtype_code(cos) if cos is not None else F32,
              _p(gate) if gate is not None else None, dtype_code(gate) if gate is not None else F32,
              int(gate_is_logit), _p(out), dtype_code(out), float(scale), _p_precision(p_bf16, p_precision),
              _s(stream))
    return out


N_FFT = 2048


def hann_window(size: int = N_FFT, out: torch.Tensor | None = None, stream=None) -> torch.Tensor:
    """Periodic Hann window [size] f32 on the current device."""
    if out is None:
        out = torch.empty(size, dtype=torch.float32, device="cuda")
    _contig(out)
    _abi.call("mbrt_hann_window", _p(out), out.numel(), _s(stream))
    return out


def stft_num_frames(length: int, hop: int, center: bool = True) -> int:
    return int(_abi.lib().mbrt_stft_num_frames(length, hop, int(center)))


def stft(signal: torch.Tensor, window: torch.Tensor, hop: int, center: bool = True, normalized: bool = False,
         out: torch.Tensor | None = None, n_fft: int = N_FFT, win_length: int = N_FFT, stream=None) -> torch.Tensor:
    """signal [B, L] (or [L]) f32 -> complex spectrogram [B, 1025, T, 2] f32."""
    x = signal.reshape(1, -1) if signal.dim() == 1 else signal
    _contig(x, window)
    B, L = x.shape
    T = stft_num_frames(L, hop, center)
    if out is None:
        out = torch.empty((B, n_fft // 2 + 1, max(T, 0), 2), dtype=torch.float32, device=x.device)
    _contig(out)
    _abi.call("mbrt_stft", _p(x), _p(window), _p(out), B, L, n_fft, hop, win_length, window.numel(), int(center),
              int(normalized), _s(stream))
    return out


def istft_output_length(frames: int, hop: int, center: bool = True, length: int = -1) -> int:
    return int(_abi.lib().mbrt_istft_output_length(frames, hop, int(center), length))


def istft_workspace_bytes(batch: int, frames: int, hop: int) -> int:
    return int(_abi.lib().mbrt_istft_workspace_bytes(batch, frames, hop))


def istft(spec: torch.Tensor, window: torch.Tensor, hop: int, center: bool = True, normalized: bool = False,
          length: int = -1, out: torch.Tensor | None = None, workspace: torch.Tensor | None = None,
          n_fft: int = N_FFT, win_length: int = N_FFT, stream=None) -> torch.Tensor:
    """spec [B, 1025, T, 2] f32/bf16 -> waveform [B, istft_output_length(T, hop, center, length)] f32."""
    _contig(spec, window)
    B, F, T, _ = spec.shape
    n_out = istft_output_length(T, hop, center, length)
    if out is None:
        out = torch.empty((B, max(n_out, 0)), dtype=torch.float32, device=spec.device)
    _contig(out)
    need = int(_abi.lib().mbrt_istft_workspace_bytes(B, T, hop))
    if workspace is None:
        workspace = torch.empty(max(need, 0) // 4, dtype=torch.float32, device=spec.device)
    _abi.call("mbrt_istft", _p(spec), dtype_code(spec), _p(window), _p(out), B, F, T, n_fft, hop, win_length,
              window.numel(), int(center), int(normalized), length, _p(workspace),
              workspace.numel() * workspace.element_size(), _s(stream))
    return out


ISTFT_SCRATCH_BYTES = 32 * 1024 * 1024  # MBRT_ISTFT_SCRATCH_BYTES


def istft_noalloc(spec: torch.Tensor, window: torch.Tensor, hop: int, out: torch.Tensor, center: bool = True,
                  normalized: bool = False, length: int = -1, n_fft: int = N_FFT, win_length: int = N_FFT,
                  stream=None) -> torch.Tensor:
    """istft into a caller-provided `out` through mbrt_istft_noalloc: no workspace, no
    allocation (the block partials use the library's scratch array on this GPU)."""
    _contig(spec, window, out)
    B, F, T, _ = spec.shape
    _abi.call("mbrt_istft_noalloc", _p(spec), dtype_code(spec), _p(window), _p(out), B, F, T, n_fft, hop,
              win_length, window.numel(), int(center), int(normalized), length, _s(stream))
    return out


def chunk_accumulate(dest: torch.Tensor, weight_sum: torch.Tensor, src: torch.Tensor, window: torch.Tensor,
                     offset: int, stream=None) -> torch.Tensor:
    """dest [.., L] += src [.., n] * window at `offset` (channels = src.numel() / n); weight_sum += window."""
    _contig(dest, weight_sum, src, window)
    n, L = src.shape[-1], dest.shape[-1]
    _abi.call("mbrt_chunk_accumulate", _p(dest), _p(weight_sum), _p(src), _p(window), src.numel() // max(n, 1), n, L,
              offset, _s(stream))
    return dest


def chunk_normalize(data: torch.Tensor, weight_sum: torch.Tensor, stream=None) -> torch.Tensor:
    _contig(data, weight_sum)
    L = data.shape[-1]
    _abi.call("mbrt_chunk_normalize", _p(data), _p(weight_sum), data.numel() // max(L, 1), L, _s(stream))
    return data


def chunk_fade_window(chunk_size: int, fade_size: int, first: bool = False, last: bool = False):
    """Host fade window (numpy f32 [chunk_size])."""
    import numpy as np

    w = np.empty(chunk_size, dtype=np.float32)
    _abi.call("mbrt_chunk_fade_window", w.ctypes.data_as(C.c_void_p), chunk_size, fade_size, int(first), int(last))
    return w


# ---- host-side tables -----------------------------------------------------------------------

def mel_band_layout(sample_rate: float = 44100.0, n_fft: int = 2048, n_bands: int = 60, channels: int = 2):
    """(freq_indices int32 [J], freqs_per_band int32 [n_bands]) on the host (numpy)."""
    import numpy as np

    n = C.c_int64(0)
    fpb = np.empty(n_bands, dtype=np.int32)
    _abi.call("mbrt_mel_band_layout", sample_rate, n_fft, n_bands, channels, None, 0, C.byref(n),
              fpb.ctypes.data_as(C.c_void_p))
    fi = np.empty(n.value, dtype=np.int32)
    _abi.call("mbrt_mel_band_layout", sample_rate, n_fft, n_bands, channels, fi.ctypes.data_as(C.c_void_p), fi.size,
              C.byref(n), None)
    return fi, fpb


def band_csr(freq_indices, total_freq: int):
    """(offsets [F+1], indices [J], counts f32 [F], max bands per freq) on the host."""
    import numpy as np

    fi = np.ascontiguousarray(freq_indices, dtype=np.int32)
    off = np.empty(total_freq + 1, dtype=np.int32)
    ind = np.empty(fi.size, dtype=np.int32)
    cnt = np.empty(total_freq, dtype=np.float32)
    mx = C.c_int32(0)
    _abi.call("mbrt_band_csr", fi.ctypes.data_as(C.c_void_p), fi.size, total_freq, off.ctypes.data_as(C.c_void_p),
              ind.ctypes.data_as(C.c_void_p), cnt.ctypes.data_as(C.c_void_p), C.byref(mx))
    return off, ind, cnt, mx.value


def rotary_tables(seq_len: int, dim_head: int, theta: float = 10000.0):
    """(cos, sin) f32 [seq_len, dim_head/2] on the host (numpy)."""
    import numpy as np

    cos = np.empty((seq_len, dim_head // 2), dtype=np.float32)
    sin = np.empty((seq_len, dim_head // 2), dtype=np.float32)
    _abi.call("mbrt_rotary_tables", cos.ctypes.data_as(C.c_void_p), sin.ctypes.data_as(C.c_void_p), seq_len, dim_head,
              theta)
    return cos, sin
