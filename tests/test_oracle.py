"""Pins the CPU oracle (oracle/) before it is trusted as the GPU kernels' checker.

Each oracle function is checked against something that does not share its code:
closed forms and invariants, brute force, numpy / torch (CPU, float64) formulations of
the same maths, and the reference's own recorded band layout (tests/golden/).  Each
check is chosen so that a plausible mistake (a dropped term, a wrong sign or index, a
transposed operand, a wrong rounding) fails it.
"""
from __future__ import annotations

import json
from fractions import Fraction
from pathlib import Path

import numpy as np
import pytest
import torch

from parity import BF16, F16, F32, assert_bitexact, assert_close

GOLDEN = Path(__file__).resolve().parent / "golden"
I64, I32 = 2, 4  # the oracle's integer dtype ids


# ---- rounding ----------------------------------------------------------------------------

def test_bf16_roundtrip_all_patterns(orc):
    bits = np.arange(65536, dtype=np.uint16)
    f = orc.bf16_to_f32(bits)
    assert np.array_equal(f.view(np.uint32) >> 16, bits.astype(np.uint32))
    back = orc.f32_to_bf16(f)
    nan = np.isnan(f)
    assert np.array_equal(back[~nan], bits[~nan])
    assert np.all(np.isnan(orc.bf16_to_f32(back[nan])))


def test_f32_to_bf16_matches_torch(orc):
    rng = np.random.default_rng(1)
    u = rng.integers(0, 2**32, size=200_000, dtype=np.uint64).astype(np.uint32)
    # crafted ties: low 16 bits exactly 0x8000 with even and odd kept halves
    ties = (rng.integers(0, 2**16, size=2000, dtype=np.uint32) << 16) | 0x8000
    u = np.concatenate([u, ties, np.array([0x7f7fffff, 0x7f7f8000, 0xff7f8000, 0x00008000, 0x80018000],
                                          dtype=np.uint32)])
    f = u.view(np.float32)
    f = f[~np.isnan(f)]
    ours = orc.f32_to_bf16(f)
    ref = torch.from_numpy(f.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert_bitexact(ours, ref, "f32->bf16")


def test_f16_conversions_match_numpy(orc):
    bits = np.arange(65536, dtype=np.uint16)
    ours = orc.f16_to_f32(bits)
    ref = bits.view(np.float16).astype(np.float32)
    ok = ~np.isnan(ref)
    assert_bitexact(ours[ok], ref[ok], "f16->f32")
    rng = np.random.default_rng(2)
    f = np.concatenate([
        rng.standard_normal(100_000).astype(np.float32) * np.float32(1000),
        rng.standard_normal(20_000).astype(np.float32) * np.float32(1e-5),  # subnormal range
        np.array([65504, 65519.99, 65520, 1e6, 2**-24, 2**-25, 2**-25 * 1.0000001, 3 * 2**-26], np.float32),
    ])
    assert_bitexact(orc.f32_to_f16(f), f.astype(np.float16).view(np.uint16), "f32->f16")


def _nearest_bf16_exact(v: float) -> int:
    """Brute force: nearest bf16 to a double by exact rational comparison, ties to even."""
    f = np.float32(v)
    cands = set()
    for base in (np.float32(f),):
        b = int(np.array([base], np.float32).view(np.uint32)[0]) >> 16
        for d in range(-2, 3):
            cands.add((b + d) & 0xFFFF)
    best = None
    for c in cands:
        cv = float(np.array([c << 16], np.uint32).view(np.float32)[0])
        if not np.isfinite(cv):
            continue
        d = abs(Fraction(cv) - Fraction(v))
        key = (d, c & 1)
        if best is None or key < best[0]:
            best = (key, c)
    return best[1]


def test_f64_to_bf16_single_rounding(orc):
    rng = np.random.default_rng(3)
    vals = list(rng.standard_normal(400) * 10.0 ** rng.integers(-30, 30, 400))
    # exact midpoints between adjacent bf16 values, and a hair above/below them: a value
    # rounded to f32 first would land on the midpoint and round to even wrongly.
    for c in rng.integers(0x0080, 0x7f00, 200):
        lo = float(np.array([int(c) << 16], np.uint32).view(np.float32)[0])
        hi = float(np.array([(int(c) + 1) << 16], np.uint32).view(np.float32)[0])
        mid = (lo + hi) / 2
        vals += [mid, np.nextafter(mid, np.inf), np.nextafter(mid, -np.inf), -mid]
    vals = np.array(vals, dtype=np.float64)
    ours = orc.f64_to_bf16(vals)
    ref = np.array([_nearest_bf16_exact(v) if v >= 0 else _nearest_bf16_exact(-v) | 0x8000 for v in vals],
                   dtype=np.uint16)
    assert_bitexact(ours, ref, "f64->bf16")


def _as_dtype(x: np.ndarray, dt: int) -> np.ndarray:
    """numpy / torch conversion of float32 or integer values to oracle dtype `dt`."""
    if dt == F32:
        return x.astype(np.float32)
    if dt == F16:
        with np.errstate(over="ignore"):   # beyond 65504 rounds to inf, as intended
            return x.astype(np.float32).astype(np.float16).view(np.uint16)
    if dt == BF16:
        return torch.from_numpy(x.astype(np.float32)).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    return x.astype(np.int64 if dt == I64 else np.int32)


def test_convert_every_dtype_pair_matches_numpy_and_torch(orc):
    """convert_dtype (src/tensor_cuda_tile.cu:442-472): floats round to nearest even,
    float -> integer truncates toward zero, integer -> float goes through f32 (RNE), and
    i64 -> i32 keeps the low 32 bits.  Every pair against numpy / torch casts."""
    rng = np.random.default_rng(4)
    f = np.concatenate([rng.standard_normal(20_000) * 300.0, rng.standard_normal(2000) * 1e-3,
                        np.array([-2.75, -2.5, -0.5, 0.0, 0.5, 2.5, 2.75, 65504.0, -65504.0, 1e6, -7.9999])])
    f = f.astype(np.float32)
    ints = np.concatenate([rng.integers(-2**40, 2**40, 5000), rng.integers(-70000, 70000, 5000),
                           np.array([0, 1, -1, 2**24 + 1, -(2**24 + 1), 2**31 - 1, -2**31, 2**33 + 7])])
    floats = (F32, F16, BF16)
    for sdt in floats + (I64, I32):
        for ddt in floats + (I64, I32):
            if sdt in floats:
                src = _as_dtype(f, sdt)
                vals = orc.to_f32(src, sdt) if sdt != F32 else src   # the value the source holds
                if ddt in floats:
                    want = _as_dtype(vals, ddt)
                else:
                    small = np.abs(vals) < 2**31 - 128                  # in range of both integer types
                    src, vals = _as_dtype(vals[small], sdt), vals[small]
                    want = np.trunc(vals.astype(np.float64)).astype(np.int64 if ddt == I64 else np.int32)
            else:
                src = ints.astype(np.int64 if sdt == I64 else np.int32)
                if ddt in floats:
                    want = _as_dtype(src.astype(np.float32), ddt)     # through f32, then the float rule
                else:
                    want = src.astype(np.int64 if ddt == I64 else np.int32)
            got = orc.convert(src, sdt, ddt)
            assert_bitexact(np.asarray(got).view(want.dtype), want, f"convert {sdt}->{ddt}")


@pytest.mark.parametrize("center", [True, False])
def test_stft_num_frames_matches_torch(orc, center):
    """Frame count of src/stft_cuda_tile.cu:544-551 against torch.stft's own output shape."""
    w = torch.ones(2048, dtype=torch.float64)
    for L in [2048, 2049, 3000, 4095, 4096, 9001, 20000] + ([1, 700, 1024, 2047] if center else []):
        for hop in [1, 7, 441, 512, 1024, 2048, 3000]:
            x = torch.zeros(L, dtype=torch.float64)
            spec = torch.stft(x, 2048, hop, window=w, center=center, pad_mode="constant", return_complex=True)
            assert orc.stft_num_frames(L, hop, center) == spec.shape[-1], (L, hop, center)
    assert orc.stft_num_frames(2047, 441, False) == 0


def test_rng_deterministic_and_normal(orc):
    a = orc.randn(1_000_001, seed=0x4D42520001, stream=3)
    b = orc.randn(1_000_001, seed=0x4D42520001, stream=3)
    c = orc.randn(1_000_001, seed=0x4D42520001, stream=4)
    assert_bitexact(a, b, "rng determinism")
    assert not np.array_equal(a, c)
    assert abs(float(a.mean())) < 5e-3 and abs(float(a.std()) - 1.0) < 5e-3
    s = orc.randn(200_000, seed=7, mean=1.0, std=0.02)
    assert abs(float(s.mean()) - 1.0) < 5e-4 and abs(float(s.std()) - 0.02) < 5e-4


# ---- tensor library --------------------------------------------------------------------

@pytest.mark.parametrize("op", [0, 1, 2, 3])
def test_binary_f32_matches_numpy_bitexact(orc, op):
    a = orc.randn(10_001, seed=11)
    b = orc.randn(10_001, seed=12) + np.float32(3.0)
    ref = [np.add, np.subtract, np.multiply, np.divide][op](a, b)
    assert_bitexact(orc.binary(a, b, F32, op), ref, f"binary op {op}")


def test_binary_bf16_is_f32_op_then_rne(orc):
    a = orc.f32_to_bf16(orc.randn(5000, seed=13))
    b = orc.f32_to_bf16(orc.randn(5000, seed=14))
    ref = torch.from_numpy((orc.bf16_to_f32(a) * orc.bf16_to_f32(b))).to(torch.bfloat16)
    assert_bitexact(orc.binary(a, b, BF16, 2), ref.view(torch.int16).numpy().view(np.uint16), "bf16 mul")


def test_broadcast_binary_matches_numpy(orc):
    a = orc.randn((3, 1, 5, 7), seed=15)
    b = orc.randn((4, 1, 7), seed=16) + np.float32(3.0)
    out_shape = (3, 4, 5, 7)
    sa = [35, 0, 7, 1]
    sb = [0, 7, 0, 1]
    for op, f in enumerate((np.add, np.subtract, np.multiply, np.divide)):
        assert_bitexact(orc.binary_broadcast(a, b, F32, out_shape, sa, sb, op), f(a, b), f"broadcast op {op}")
        # bf16: the f32 result of the widened operands, rounded once
        ab, bb = orc.from_f32(a, BF16), orc.from_f32(b, BF16)
        want = orc.from_f32(f(orc.bf16_to_f32(ab), orc.bf16_to_f32(bb)).astype(np.float32), BF16)
        assert_bitexact(orc.binary_broadcast(ab, bb, BF16, out_shape, sa, sb, op), want, f"broadcast bf16 op {op}")
    # a transposed (strided) operand
    base = orc.randn((7, 5), seed=17)
    c = orc.randn((3, 1, 7), seed=18)
    assert_bitexact(orc.binary_broadcast(base, c, F32, (3, 5, 7), [0, 1, 5], [7, 0, 1], 1), base.T[None] - c,
                    "broadcast strided")


def test_strided_copy_permute_matches_numpy(orc):
    x = orc.randn((4, 7, 6, 5), seed=17)
    for perm in [(0, 2, 1, 3), (2, 0, 1, 3), (3, 1, 0, 2)]:
        v = x.transpose(perm)
        strides = [s // 4 for s in v.strides]
        assert_bitexact(orc.strided_copy(x.reshape(-1), v.shape, strides), np.ascontiguousarray(v), str(perm))


def test_index_select_and_pads(orc):
    x = orc.randn((5, 9), seed=18)
    idx = np.array([4, 0, 0, 8, 3], dtype=np.int64)
    assert_bitexact(orc.index_select(x.reshape(-1), (5, 5), [9, 1], 1, idx), np.take(x, idx, axis=1), "take")
    y = orc.pad(x, F32, (5, 14), [0, 2], value=-1.5)
    assert_bitexact(y, np.pad(x, ((0, 0), (2, 3)), constant_values=-1.5), "pad const")
    y = orc.pad(x, F32, (5, 14), [0, 3], reflect=True)
    assert_bitexact(y, np.pad(x, ((0, 0), (3, 2)), mode="reflect"), "pad reflect")


def test_reductions(orc):
    x = orc.randn((6, 33, 10), seed=19)
    got = orc.reduce_general(x, 1, 0)
    acc = np.zeros((6, 10), np.float32)
    for r in range(33):  # sequential f32 accumulation, the reference's loop order
        acc = (acc + x[:, r, :]).astype(np.float32)
    assert_bitexact(got, acc, "sequential sum")
    assert_bitexact(orc.reduce_general(x, 1, 1), x.max(axis=1), "max")
    assert_close(orc.reduce_last(x, 0), x.astype(np.float64).sum(-1).astype(np.float32), F32, "sum last")


# ---- hot-path ops -------------------------------------------------------------------------

def test_rms_norm_closed_forms_and_torch(orc):
    D = 384
    x = orc.randn((32, D), seed=21)
    gamma_one = np.ones(D, np.float32)
    y = orc.rms_norm(x, F32, gamma_one, F32, F32, scale=float(np.sqrt(D)), eps=0.0)
    assert np.allclose(np.linalg.norm(y.astype(np.float64), axis=1), np.sqrt(D), rtol=1e-6)
    y2 = orc.rms_norm(x * np.float32(8.0), F32, gamma_one, F32, F32, scale=float(np.sqrt(D)), eps=0.0)
    assert_close(y2, y, F32, "scale invariance")
    gamma = orc.randn(D, seed=22, mean=1.0, std=0.02)
    y = orc.rms_norm(x, F32, gamma, F32, F32, scale=float(np.sqrt(D)), eps=1e-8)
    xt = torch.from_numpy(x).double()
    ref = xt * torch.rsqrt((xt * xt).sum(-1, keepdim=True) + 1e-8) * torch.from_numpy(gamma).double() * np.sqrt(D)
    assert_close(y, ref.float().numpy(), F32, "rms vs torch")
    # F.normalize form of the reference (src/mbr_cuda_tile.cu:4806-4812)
    ref2 = torch.nn.functional.normalize(xt, dim=-1) * np.sqrt(D) * torch.from_numpy(gamma).double()
    assert_close(y, ref2.float().numpy(), F32, "rms vs F.normalize")


def test_residual_rms_sum_is_f32_add(orc):
    D = 384
    x = orc.randn((16, D), seed=23)
    r = orc.randn((16, D), seed=24)
    g = orc.randn(D, seed=25, mean=1.0, std=0.02)
    out, s = orc.rms_norm(x, F32, g, F32, F32, scale=float(np.sqrt(D)), eps=1e-8, res=r, sdt=F32, want_sum=True)
    assert_bitexact(s, x + r, "residual sum")
    assert_close(out, orc.rms_norm(x + r, F32, g, F32, F32, float(np.sqrt(D)), 1e-8), F32, "normed")
    xb, rb = orc.f32_to_bf16(x), orc.f32_to_bf16(r)
    _, sb = orc.rms_norm(xb, BF16, g, F32, BF16, float(np.sqrt(D)), 1e-8, res=rb, sdt=BF16, want_sum=True)
    assert_bitexact(sb, orc.f32_to_bf16(orc.bf16_to_f32(xb) + orc.bf16_to_f32(rb)), "bf16 residual sum")


def test_activations_vs_torch(orc):
    x = orc.randn((64, 96), seed=26, std=1.5)
    xt = torch.from_numpy(x).double()
    ref = {
        1: 0.5 * xt * (1 + torch.erf(xt)),
        2: torch.nn.functional.gelu(xt),
        3: torch.sigmoid(xt),
        4: torch.tanh(xt),
    }
    for act, r in ref.items():
        assert_close(orc.bias_act(x, F32, None, F32, F32, act), r.float().numpy(), F32, f"act {act}")
    # GELU(x) - GELU(-x) = x for both forms; GELU(0) = 0
    for act in (1, 2):
        z = np.array([0.0], np.float32)
        assert orc.bias_act(z, F32, None, F32, F32, act)[0] == 0.0
        d = orc.bias_act(x, F32, None, F32, F32, act).astype(np.float64) - \
            orc.bias_act(-x, F32, None, F32, F32, act).astype(np.float64)
        assert np.allclose(d, x, rtol=0, atol=1e-5)
    # bias is added per column
    b = orc.randn(96, seed=27)
    assert_close(orc.bias_act(x, F32, b, F32, F32, 3), torch.sigmoid(xt + torch.from_numpy(b).double()).float().numpy(),
                 F32, "bias sigmoid")


def test_glu_and_gate_merge(orc):
    x = orc.randn((10, 2 * 48), seed=28, std=1.5)
    ref = torch.nn.functional.glu(torch.from_numpy(x).double(), dim=-1)
    assert_close(orc.glu(x, F32, F32), ref.float().numpy(), F32, "glu")
    x0 = x.copy()
    x0[:, 48:] = 0
    assert_bitexact(orc.glu(x0, F32, F32), x0[:, :48] * np.float32(0.5), "glu gate 0")
    B, H, N, D = 2, 8, 5, 16
    attn = orc.randn((B, H, N, D), seed=29)
    gate = orc.randn((B, N, H), seed=30, std=2.0)
    ref = torch.from_numpy(attn).double().permute(0, 2, 1, 3) * torch.sigmoid(torch.from_numpy(gate).double())[..., None]
    got = orc.gate_merge(attn, F32, gate, F32, F32, B, H, N, D, layout=0)
    assert_close(got, ref.reshape(B, N, H * D).float().numpy(), F32, "gate merge BHND")
    attn_t = np.ascontiguousarray(attn.transpose(0, 2, 1, 3))
    got2 = orc.gate_merge(attn_t, F32, gate, F32, F32, B, H, N, D, layout=1)
    assert_bitexact(got2, got, "gate merge BNHD == BHND")


def test_softmax(orc):
    for cols in (801, 60, 7):
        x = orc.randn((9, cols), seed=31 + cols, std=3.0)
        for scale in (1.0, 0.125):
            ref = torch.softmax(torch.from_numpy(x).double() * scale, dim=-1)
            got = orc.softmax(x, F32, F32, scale)
            assert_close(got, ref.float().numpy(), F32, f"softmax {cols} {scale}")
            assert np.allclose(got.astype(np.float64).sum(-1), 1.0, atol=1e-6)
        assert_close(orc.softmax(x + np.float32(5.0), F32, F32), orc.softmax(x, F32, F32), F32, "shift invariance",
                     rtol=1e-4)


def test_rotary_tables_and_apply(orc):
    cos, sin = orc.rotary_tables(801, 64)
    n = np.arange(801)[:, None].astype(np.float64)
    i = np.arange(32)[None, :].astype(np.float64)
    ang = n * 10000.0 ** (-2 * i / 64)
    # the reference forms the angle in f32: |error| grows ~ n * 2^-24
    assert np.max(np.abs(cos - np.cos(ang))) < 1e-4 and np.max(np.abs(sin - np.sin(ang))) < 1e-4
    assert np.all(cos[0] == 1.0) and np.all(sin[0] == 0.0)
    BH, N, D = 6, 801, 64
    q = orc.randn((BH, N, D), seed=41)
    k = orc.randn((BH, N, D), seed=42)
    rq, rk = orc.rotary(q, k, F32, cos, sin, F32, N, 1, layout=0)
    # complex formulation: (x0 + i x1) * (c + i s)
    zc = torch.from_numpy(q).double().reshape(BH, N, 32, 2)
    z = torch.complex(zc[..., 0], zc[..., 1]) * torch.complex(torch.from_numpy(cos).double(),
                                                              torch.from_numpy(sin).double())
    ref = torch.stack([z.real, z.imag], -1).reshape(BH, N, D)
    assert_close(rq, ref.float().numpy(), F32, "rotary vs complex")
    assert np.allclose(np.linalg.norm(rq.reshape(BH, N, 32, 2), axis=-1), np.linalg.norm(q.reshape(BH, N, 32, 2), axis=-1),
                       rtol=1e-6)
    assert_bitexact(rq[:, 0], q[:, 0], "identity at n=0")
    # [B, N, H, D] layout rotates by position n = (row / H) % N
    qb = np.ascontiguousarray(q.reshape(2, 3, N, D).transpose(0, 2, 1, 3))
    rqb, _ = orc.rotary(qb, None, F32, cos, sin, F32, N, 3, layout=1)
    assert_bitexact(rqb, np.ascontiguousarray(rq.reshape(2, 3, N, D).transpose(0, 2, 1, 3)), "BNHD == BHND")


def test_split_qkv_matches_rotary(orc):
    B, N, H, D = 2, 60, 8, 64
    qkv = orc.randn((B, N, 3 * H * D), seed=43)
    cos, sin = orc.rotary_tables(N, D)
    q, k, v = orc.split_qkv(qkv, F32, cos, sin, F32, F32, B, N, H, D, 64)
    parts = qkv.reshape(B, N, 3, H, D)
    q_ref = np.ascontiguousarray(parts[:, :, 0].transpose(0, 2, 1, 3)).reshape(B * H, N, D)
    rq, _ = orc.rotary(q_ref, None, F32, cos, sin, F32, N, 1)
    assert_bitexact(q[:, :, :N].reshape(B * H, N, D), rq, "split q == rotary(q)")
    assert_bitexact(v[:, :, :N], np.ascontiguousarray(parts[:, :, 2].transpose(0, 2, 1, 3)), "v copied")
    assert np.all(q[:, :, N:] == 0) and np.all(k[:, :, N:] == 0) and np.all(v[:, :, N:] == 0)


# ---- mel bands -----------------------------------------------------------------------------

def test_mel_bands_match_reference_layout(orc):
    gold = json.loads((GOLDEN / "mel_band_widths.json").read_text())
    mb = orc.mel_bands(44100.0, 2048, 60, 2)
    fpb = mb["freqs_per_band"]
    widths = 4 * fpb
    stems = gold["config"]["stems"]
    want = {w: c // stems for w, c in gold["width_counts"]}
    got = {}
    for w in widths.tolist():
        got[w] = got.get(w, 0) + 1
    assert got == want, "band widths differ from the reference's recorded layout"
    assert int(widths.sum()) == gold["mask_stride"] == 2 * mb["freq_indices"].size
    assert mb["freq_indices"].size == 3958
    bpf = mb["bands_per_freq"]
    assert bpf.min() == 1 and bpf.max() == 2 and int((bpf[::2] == 1).sum()) == 71
    # CSR: every band-bin appears once, ascending within a freq, pointing back at its freq
    off, ind, fi = mb["csr_offsets"], mb["csr_indices"], mb["freq_indices"]
    assert off[0] == 0 and off[-1] == ind.size and np.all(np.diff(off) == bpf)
    assert np.array_equal(np.sort(ind), np.arange(ind.size))
    for f in range(bpf.size):
        seg = ind[off[f]:off[f + 1]]
        assert np.all(np.diff(seg) > 0) and np.all(fi[seg] == f)
    # stereo interleave 2*bin + ch, bands are contiguous bin ranges, DC and Nyquist covered
    assert np.array_equal(fi[0::2] % 2, np.zeros(fi.size // 2)) and np.array_equal(fi[1::2], fi[0::2] + 1)
    assert fi[0] == 0 and fi[-1] == 2049


def test_band_gather_matches_numpy(orc):
    B, F, T = 2, 2050, 37
    stft = orc.randn((B, F, T, 2), seed=51)
    idx = orc.mel_bands()["freq_indices"]
    got = orc.band_gather(stft, idx, F32, B, F, T)
    ref = stft[:, idx].transpose(0, 2, 1, 3).reshape(B, T, -1)
    assert_bitexact(got, np.ascontiguousarray(ref), "gather")


def test_band_gather_clamps_out_of_range_indices(orc):
    # an index outside [0, F) reads the nearest valid row: numpy's take(mode="clip")
    B, F, T = 2, 50, 9
    stft = orc.randn((B, F, T, 2), seed=53)
    idx = np.array([0, -1, -7, 49, 50, 51, 10**6, -(2**40), 2**40, 3], dtype=np.int64)
    got = orc.band_gather(stft, idx, F32, B, F, T)
    ref = np.take(stft, idx, axis=1, mode="clip").transpose(0, 2, 1, 3).reshape(B, T, -1)
    assert_bitexact(got, np.ascontiguousarray(ref), "gather clamp")


def test_band_merge_kat_and_numpy(orc):
    B, F, T = 2, 2050, 19
    mb = orc.mel_bands()
    stft = orc.randn((B, F, T, 2), seed=52)
    J = mb["freq_indices"].size
    cnt = mb["bands_per_freq"].astype(np.float32)
    ones = np.zeros((B, T, J, 2), np.float32)
    ones[..., 0] = 1.0
    out = orc.band_mask_merge(stft, [ones], F32, mb["csr_offsets"], mb["csr_indices"], cnt, F32, F32, B, F, T, 2)
    # mask == 1+0j: sum over the freq's bands of s, divided by their count, is s exactly
    ref = stft.reshape(B, F // 2, 2, T, 2).transpose(0, 2, 1, 3, 4).reshape(B * 2, F // 2, T, 2)
    assert_bitexact(out, np.ascontiguousarray(ref), "merge KAT")
    # general masks: scatter-add per band-bin with np.add.at in complex128, then / count
    m = orc.randn((B, T, J, 2), seed=53, std=0.5)
    m2 = orc.randn((B, T, J, 2), seed=54, std=0.5)
    out = orc.band_mask_merge(stft, [m, m2], F32, mb["csr_offsets"], mb["csr_indices"], cnt, F32, F32, B, F, T, 2)
    sc = stft[..., 0].astype(np.float64) + 1j * stft[..., 1]
    for s, mm in enumerate([m, m2]):
        mc = mm[..., 0].astype(np.float64) + 1j * mm[..., 1]            # [B, T, J]
        acc = np.zeros((B, F, T), np.complex128)
        prod = sc[:, mb["freq_indices"], :] * mc.transpose(0, 2, 1)      # [B, J, T]
        np.add.at(acc, (slice(None), mb["freq_indices"]), prod)
        acc /= cnt[None, :, None]
        ref = np.stack([acc.real, acc.imag], -1).reshape(B, F // 2, 2, T, 2).transpose(0, 2, 1, 3, 4)
        got = out.reshape(B, 2, 2, F // 2, T, 2)[:, s]
        assert_close(np.ascontiguousarray(got), np.ascontiguousarray(ref).astype(np.float32), F32, f"merge stem {s}")


def test_zero_dc(orc):
    x = orc.randn((3, 5, 4, 2), seed=55)
    y = orc.zero_dc(x, F32)
    assert np.all(y[:, 0] == 0) and np.array_equal(y[:, 1:], x[:, 1:])


# ---- attention -------------------------------------------------------------------------------

def test_attention_matches_numpy_and_closed_forms(orc):
    """Double oracle vs a numpy float64 einsum formulation; equal keys give the mean of v;
    constant v gives v; the FAST (f32, bf16-probability) pipeline stays within 5e-3."""
    for (BH, nq, nk, scale) in [(2, 5, 7, 0.0), (3, 33, 70, 0.3), (1, 64, 64, 0.125)]:
        q = orc.randn((BH, nq, 64), seed=11, stream=nq)
        k = orc.randn((BH, nk, 64), seed=12, stream=nk)
        v = orc.randn((BH, nk, 64), seed=13, stream=nk)
        out = orc.attention(q, k, v, F32, F32, scale)
        sc = scale or 1.0 / 8.0
        s = np.einsum("bid,bjd->bij", q.astype(np.float64), k.astype(np.float64)) * sc
        p = np.exp(s - s.max(-1, keepdims=True))
        p /= p.sum(-1, keepdims=True)
        ref = np.einsum("bij,bjd->bid", p, v.astype(np.float64))
        assert np.abs(out - ref).max() < 1e-6
        fast = orc.attention(q, k, v, F32, F32, scale, mode=orc.FAST)
        assert np.linalg.norm(fast - ref) / np.linalg.norm(ref) < 5e-3
    q = orc.randn((1, 4, 64), seed=14)
    k = np.repeat(orc.randn((1, 1, 64), seed=15), 9, axis=1)
    v = orc.randn((1, 9, 64), seed=16)
    out = orc.attention(q, k, v, F32, F32, 0.0)
    assert np.allclose(out, np.broadcast_to(v.mean(axis=1, keepdims=True), out.shape), atol=1e-6)
    ones = np.ones((1, 9, 64), np.float32) * 3.0
    assert np.allclose(orc.attention(q, orc.randn((1, 9, 64), seed=17), ones, F32, F32, 0.0), 3.0, atol=1e-6)


def _bf16_round(x):
    """float64 -> nearest bf16 (ties to even) by bit manipulation of the f32 value; the
    inputs here are f32-exact products of exp, so one rounding of their f32 value is the
    rounding of the value itself except at exact ties."""
    f = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    f = (f + 0x7FFF + ((f >> 16) & 1)) >> 16 << 16
    return f.astype(np.uint32).view(np.float32).astype(np.float64)


def test_attention_ref_p_pins(orc):
    """The reference-P variant: (1) q = 0 makes every P exactly 1 (a bf16 value), so it
    equals exact attention, the mean of v; (2) v = 1 gives sum bf16(p) / sum p per row,
    rebuilt here from numpy scores with the same 64-key running max (0 if P or the row sum
    were both rounded, or neither); (3) it stays within a bf16 rounding of every P of exact
    attention, and is not equal to it."""
    BH, nq, nk = 2, 9, 150
    k = orc.randn((BH, nk, 64), seed=21)
    v = orc.randn((BH, nk, 64), seed=22)
    q0 = np.zeros((BH, nq, 64), np.float32)
    assert_bitexact(orc.attention_ref_p(q0, k, v, F32, F32), orc.attention(q0, k, v, F32, F32), "q = 0")
    q = orc.randn((BH, nq, 64), seed=23, std=2.0)
    ones = np.ones((BH, nk, 64), np.float32)
    got = orc.attention_ref_p(q, k, ones, F32, F32, 0.125)
    s = np.einsum("bid,bjd->bij", q.astype(np.float64), k.astype(np.float64)) * 0.125
    num = np.zeros((BH, nq))
    den = np.zeros((BH, nq))
    m = np.full((BH, nq), -np.inf)
    for k0 in range(0, nk, 64):
        st = s[..., k0:k0 + 64]
        mn = np.maximum(m, st.max(-1))
        a = np.exp(m - mn)
        p = np.exp(st - mn[..., None])
        num = num * a + _bf16_round(p).sum(-1)
        den = den * a + p.sum(-1)
        m = mn
    ratio = num / den
    assert np.abs(ratio - 1).max() > 1e-5  # the rounding is visible
    assert np.allclose(got, np.broadcast_to(ratio[..., None], got.shape), rtol=0, atol=2e-7)
    exact = orc.attention(q, k, v, F32, F32, 0.125)
    refp = orc.attention_ref_p(q, k, v, F32, F32, 0.125)
    rel = np.linalg.norm(refp - exact) / np.linalg.norm(exact)
    assert 1e-5 < rel < 2.0 ** -8


def test_attention_ref_p_fast_pins(orc):
    """The fast bf16-P variant (running max moved only past 8 log2 units, row sum over the
    rounded P): (1) v = 1 gives exactly 1, the row sum and the output adding the same
    rounded values; (2) when every query's largest score lies in the first 64-key tile the
    running max never moves in either rule, so it equals the every-tile rule with the
    rounded row sum bit for bit; (3) with later tiles that outgrow the first by more than
    8 log2 units (the max must move), it stays within a bf16 rounding of every P of exact
    attention, and differs from the every-tile rule."""
    lazy = orc.ATTN_FAST_LAZY
    assert abs(lazy - 8 * np.log(2)) < 1e-15
    BH, nq, nk = 2, 9, 200
    k = orc.randn((BH, nk, 64), seed=31)
    v = orc.randn((BH, nk, 64), seed=32)
    q = orc.randn((BH, nq, 64), seed=33, std=2.0)
    ones = np.ones((BH, nk, 64), np.float32)
    got = orc.attention_ref_p(q, k, ones, F32, F32, 0.125, lazy=lazy, sum_rounded=True)
    assert_bitexact(got, np.ones_like(got), "v = 1")
    k1 = k.copy()
    k1[:, :nq] = 3.0 * q  # each query's largest score is its own key, in the first tile
    a = orc.attention_ref_p(q, k1, v, F32, F32, 0.125, lazy=lazy, sum_rounded=True)
    b = orc.attention_ref_p(q, k1, v, F32, F32, 0.125, lazy=0.0, sum_rounded=True)
    assert_bitexact(a, b, "max in the first tile")
    k2 = k.copy()
    k2[:, 130:130 + nq] = 0.5 * q  # the largest scores in the third tile, 7 to 16 above the first
    s = np.einsum("bid,bjd->bij", q.astype(np.float64), k2.astype(np.float64)) * 0.125
    assert (s[..., 128:].max(-1) - s[..., :64].max(-1)).min() > lazy  # every row's max moves
    a = orc.attention_ref_p(q, k2, v, F32, F32, 0.125, lazy=lazy, sum_rounded=True)
    b = orc.attention_ref_p(q, k2, v, F32, F32, 0.125, lazy=0.0, sum_rounded=True)
    exact = orc.attention(q, k2, v, F32, F32, 0.125)
    assert np.linalg.norm(a - exact) / np.linalg.norm(exact) < 2.0 ** -8
    assert np.abs(a - b).max() > 0


# ---- STFT / iSTFT --------------------------------------------------------------------------

def _direct_stft(x, w, hop, center, norm):
    """O(N^2) DFT of frames cut with numpy's own reflect padding (not the oracle's rule)."""
    xp = np.pad(x.astype(np.float64), ((0, 0), (1024, 1024)), mode="reflect") if center else x.astype(np.float64)
    T = (xp.shape[1] - 2048) // hop + 1
    n = np.arange(2048)
    M = np.exp(-2j * np.pi * np.outer(np.arange(1025), n) / 2048)  # [1025, 2048]
    fr = np.stack([xp[:, t * hop: t * hop + 2048] for t in range(T)], axis=1) * w.astype(np.float64)
    X = fr @ M.T  # [B, T, 1025]
    return (X * norm).transpose(0, 2, 1)


def test_hann_window_closed_form_and_torch(orc):
    for size in (2048, 1000, 7, 2):
        w = orc.hann_window(size)
        th = torch.hann_window(size, periodic=True, dtype=torch.float64).numpy()
        # the f32 phase (step and product rounded) and the f32 difference 1 - cos move w by
        # a few 1e-8 at most
        assert np.all(np.abs(w - th) <= 4e-7 * orc.hann_den(size)), size
    assert np.array_equal(orc.hann_window(1), np.ones(1, np.float32))
    w = orc.hann_window(2048)
    assert w[0] == 0.0 and w[1024] == 1.0 and np.abs(w[1:1024] - w[2047:1024:-1]).max() < 4e-7


def test_stft_oracle_matches_direct_dft(orc):
    rng = np.random.default_rng(11)
    w = orc.hann_window(2048)
    for (B, L, hop, center, normalized) in [(2, 3000, 441, True, False), (1, 5000, 512, False, True),
                                             (1, 2100, 300, True, True)]:
        x = rng.standard_normal((B, L)).astype(np.float32)
        norm = float(np.float32(1.0) / np.sqrt(np.float32(2048))) if normalized else 1.0
        want = _direct_stft(x, w, hop, center, norm)
        got = orc.stft(x, w, hop, center, normalized)
        assert got.shape == (B, 1025, want.shape[2], 2)
        den = orc.stft_den(x, w, hop, center, normalized)
        err = np.abs(got[..., 0] + 1j * got[..., 1] - want) / den[..., 0]
        assert err.max() < 1e-7, (B, L, hop, center, normalized, err.max())


def test_stft_oracle_reflect_rule(orc):
    """The oracle's reflect-then-clamp rule equals numpy's reflect padding whenever the
    signal is longer than the pad, and clamps for shorter ones (Tensor::pad_reflect)."""
    x = np.arange(3000, dtype=np.float32)[None, :]
    fr = orc.stft_frames(x, 441, True)
    xp = np.pad(x[0].astype(np.float64), (1024, 1024), mode="reflect")
    for t in range(fr.shape[1]):
        assert np.array_equal(fr[0, t], xp[t * 441: t * 441 + 2048])
    for L in (5, 700, 1024):   # pad 1024 >= length: reflect about each end once, then clamp
        short = np.arange(L, dtype=np.float32)[None, :]
        fr = orc.stft_frames(short, 441, True)
        for t in range(fr.shape[1]):
            for n in range(0, 2048, 7):
                c = t * 441 + n - 1024
                if c < 0:
                    c = -c
                if c >= L:
                    c = 2 * (L - 1) - c
                c = min(max(c, 0), L - 1)
                assert fr[0, t, n] == c, (L, t, n)


def test_stft_oracle_matches_torch(orc):
    rng = np.random.default_rng(12)
    w = orc.hann_window(2048)
    x = rng.standard_normal((2, 30000)).astype(np.float32)
    for normalized in (False, True):
        t = torch.stft(torch.from_numpy(x).double(), 2048, 441, 2048, torch.from_numpy(w).double(), center=True,
                       pad_mode="reflect", normalized=normalized, onesided=True, return_complex=True).numpy()
        got = orc.stft(x, w, 441, True, normalized)
        den = orc.stft_den(x, w, 441, True, normalized)
        assert (np.abs(got[..., 0] + 1j * got[..., 1] - t) / den[..., 0]).max() < 1e-7


def test_istft_oracle_matches_torch_and_round_trips(orc):
    rng = np.random.default_rng(13)
    w = orc.hann_window(2048)
    x = rng.standard_normal((2, 30000)).astype(np.float32)
    S = orc.stft(x, w, 441, True, False)
    T = S.shape[2]
    n = orc.istft_output_length(T, 441, True)
    assert n == (T - 1) * 441
    # perfect reconstruction where frames cover the signal
    y = orc.istft(S, F32, w, 441, True, False, length=30000)
    assert y.shape == (2, 30000)
    assert np.abs(y[:, :n] - x[:, :n]).max() < 1e-5 and np.all(y[:, n:] == 0)
    # an arbitrary (inconsistent) spectrum, with DC / Nyquist imaginary parts set
    R = rng.standard_normal(S.shape).astype(np.float32)
    for normalized, length in ((False, -1), (True, 25000)):
        got = orc.istft(R, F32, w, 441, True, normalized, length)
        ti = torch.istft(torch.from_numpy(R[..., 0] + 1j * R[..., 1]).to(torch.complex128), 2048, 441, 2048,
                         torch.from_numpy(w).double(), center=True, normalized=normalized, onesided=True,
                         length=None if length < 0 else length).numpy()
        den = orc.istft_den(R, F32, w, 441, True, normalized, length)
        assert got.shape == ti.shape
        assert (np.abs(got - ti) / np.maximum(den, 1e-30)).max() < 1e-6


def test_istft_oracle_gaps_and_bf16(orc):
    """hop > n_fft leaves samples no frame covers: window sum 0, output 0 (no division).
    A bf16 spectrum is read as its f32 values."""
    rng = np.random.default_rng(14)
    w = orc.hann_window(2048)
    R = rng.standard_normal((1, 1025, 4, 2)).astype(np.float32)
    y = orc.istft(R, F32, w, 3000, False, False)
    assert y.shape == (1, 2048 + 3 * 3000)
    assert np.all(y[0, 2048:3000] == 0) and np.all(y[0, 5048:6000] == 0)
    # single frame, not centred: x = irfft(X) w / w^2 = irfft(X) / w where w^2 > 1e-8
    y0 = orc.istft(R[:, :, :1], F32, w, 3000, False, False)[0]
    ref = np.fft.irfft(R[0, :, 0, 0] + 1j * R[0, :, 0, 1], 2048)
    ww = (w * w).astype(np.float32)
    ok = ww > np.float32(1e-8)
    want = np.where(ok, ref / np.where(ok, w, 1).astype(np.float64), ref * w)
    den = orc.istft_den(R[:, :, :1], F32, w, 3000, False, False)[0]
    assert np.all(np.abs(y0 - want) <= 1e-6 * den)
    Rb = orc.f32_to_bf16(R)
    assert np.array_equal(orc.istft(Rb, BF16, w, 441, True), orc.istft(orc.bf16_to_f32(Rb), F32, w, 441, True))


# ---- chunk overlap-add ---------------------------------------------------------------------

def test_chunk_fade_window_closed_form(orc):
    w = orc.chunk_fade_window(100, 10)
    assert np.array_equal(w[:10], np.arange(10, dtype=np.float32) / np.float32(9))
    assert np.array_equal(w[90:], np.float32(1) - np.arange(10, dtype=np.float32) / np.float32(9))
    assert np.all(w[10:90] == 1) and w[0] == 0 and w[9] == 1 and w[-1] == 0
    assert np.all(orc.chunk_fade_window(100, 10, first=True)[:90] == 1)
    assert np.all(orc.chunk_fade_window(100, 10, last=True)[10:] == 1)
    w1 = orc.chunk_fade_window(7, 1)
    assert w1[0] == 0 and w1[-1] == 0 and np.all(w1[1:-1] == 1)
    assert np.all(orc.chunk_fade_window(7, 0) == 1)


def test_chunk_overlap_add_reconstructs_and_matches_float64(orc):
    """Identity model: the weighted overlap-add divided by the weight sum gives the input
    back (to f32 rounding); a two-stem model gives (2x, -x); and the f32 restatement agrees
    with an independent float64 evaluation of sum_k m(x)_k w_k / sum_k w_k."""
    rng = np.random.default_rng(21)
    for L, chunk, step, batch in [(16000, 4000, 3000, 1), (17001, 4000, 3200, 3), (1500, 4000, 3000, 2)]:
        x = rng.standard_normal((1, 2, L)).astype(np.float32)
        y = orc.process_chunked(x, chunk, step, batch, lambda a: a.copy())
        assert y.shape == x.shape
        assert np.abs(y - x).max() <= 4e-7 * np.abs(x).max(), (L, chunk, step)
        y2 = orc.process_chunked(x, chunk, step, batch, lambda a: np.stack([2 * a, -a], axis=1))
        assert y2.shape == (1, 2, 2, L)
        assert np.abs(y2[0, 0] - 2 * x[0]).max() <= 1e-6 * np.abs(x).max()
        assert np.abs(y2[0, 1] + x[0]).max() <= 1e-6 * np.abs(x).max()
    # no overlap (step = chunk): the fades reach 0 at inner chunk edges, where the weight sum
    # is 0 and the output stays 0; everywhere else x w / w = x
    x = rng.standard_normal((1, 2, 9000)).astype(np.float32)
    y = orc.process_chunked(x, 1000, 1000, 4, lambda a: a.copy())
    edge = np.zeros(9000, bool)
    edge[1000::1000] = True
    edge[999:8999:1000] = True
    assert np.all(y[..., edge] == 0)
    assert np.abs(y[..., ~edge] - x[..., ~edge]).max() <= 4e-7 * np.abs(x).max()
    # accumulate / normalize against float64 with overlapping random chunks
    dest = np.zeros((3, 50), np.float32)
    ws = np.zeros(50, np.float32)
    acc64 = np.zeros((3, 50))
    ws64 = np.zeros(50)
    for off, n in [(0, 20), (10, 25), (30, 20), (5, 40)]:
        s = rng.standard_normal((3, n)).astype(np.float32)
        w = rng.random(n).astype(np.float32)
        orc.chunk_accumulate(dest, ws, s, w, off)
        acc64[:, off:off + n] += s.astype(np.float64) * w
        ws64[off:off + n] += w
    assert np.abs(dest - acc64).max() <= 1e-6 * np.abs(acc64).max()
    orc.chunk_normalize(dest, ws)
    assert np.abs(dest - acc64 / ws64).max() <= 1e-5 * np.abs(acc64 / ws64).max()
