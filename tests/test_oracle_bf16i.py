"""Pins the oracle's bf16-intermediates mode (ORC_BF16I), the reference's full-bf16
experiment mode (full_bf16_arith_enabled, src/mbr_cuda_tile.cu:190-192).

The rounding points themselves are the reference's (each test cites its kernel).  What
these tests pin is the oracle's arithmetic around them:
  * known answers worked out by hand for single elements, where one rounding point
    decides the result;
  * an independent restatement in exact rational arithmetic (fractions.Fraction, with
    exp / sqrt evaluated by `decimal` to 50 digits), compared bit for bit on small
    seeded inputs; every case set also contains inputs on which the mode changes the
    result against ORC_EXACT, so a rounding point that the oracle dropped fails it;
  * identities: where every intermediate is already a bf16 value the mode must equal
    ORC_EXACT bit for bit.
"""
from __future__ import annotations

import math
from decimal import Decimal, getcontext
from fractions import Fraction

import numpy as np

from parity import BF16, F32, assert_bitexact

getcontext().prec = 50
BF16I, EXACT = 2, 0


# ---- exact restatement helpers ---------------------------------------------------------

def fr(x) -> Fraction:
    return Fraction(float(x))


def rb(x: Fraction) -> Fraction:
    """Nearest bf16 (8 significant bits), ties to even; the values here are normal."""
    if x == 0:
        return Fraction(0)
    sign = -1 if x < 0 else 1
    ax = abs(x)
    e = ax.numerator.bit_length() - ax.denominator.bit_length()
    while Fraction(2) ** e > ax:
        e -= 1
    while Fraction(2) ** (e + 1) <= ax:
        e += 1
    ulp = Fraction(2) ** (e - 7)
    q = ax / ulp
    n = math.floor(q)
    rem = q - n
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and n % 2 == 1):
        n += 1
    return sign * n * ulp


def r32(x: Fraction) -> float:
    """Nearest f32 of an exact value (rounded once, in exact arithmetic)."""
    return _round_bits(x, 24)


def _round_bits(x: Fraction, p: int) -> float:
    if x == 0:
        return 0.0
    sign = -1 if x < 0 else 1
    ax = abs(x)
    e = ax.numerator.bit_length() - ax.denominator.bit_length()
    while Fraction(2) ** e > ax:
        e -= 1
    while Fraction(2) ** (e + 1) <= ax:
        e += 1
    ulp = Fraction(2) ** (e - (p - 1))
    q = ax / ulp
    n = math.floor(q)
    rem = q - n
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and n % 2 == 1):
        n += 1
    return float(sign * n * ulp)


def dexp(x: Fraction) -> Fraction:
    return Fraction((Decimal(x.numerator) / Decimal(x.denominator)).exp())


def dsqrt(x: Fraction) -> Fraction:
    return Fraction((Decimal(x.numerator) / Decimal(x.denominator)).sqrt())


def bf16_bits(vals) -> np.ndarray:
    """bf16 bit patterns of values that are exactly bf16."""
    a = np.array([float(v) for v in vals], dtype=np.float32)
    bits = a.view(np.uint32)
    assert np.all(bits & 0xFFFF == 0), "value is not a bf16"
    return (bits >> 16).astype(np.uint16)


def bf16_inputs(rng, shape, scale=1.0) -> np.ndarray:
    """Random bf16 bit patterns (normal values)."""
    f = (rng.standard_normal(shape) * scale).astype(np.float32)
    f[f == 0] = 0.5
    return (f.view(np.uint32) >> 16).astype(np.uint16)


def as_fr(bits) -> list[Fraction]:
    f = (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)
    return [Fraction(float(v)) for v in f.reshape(-1)]


# ---- RMSNorm (src/mbr_cuda_tile.cu:4815-4843, 4870-4905) ----------------------------------

def rms_exact(x, gamma, scale, eps):
    v = [rb(fr(t)) for t in x]
    ss = rb(sum(t * t for t in v))
    inv = rb(1 / dsqrt(ss + fr(np.float32(eps))))
    return [rb(t * inv * rb(fr(g)) * fr(np.float32(scale))) for t, g in zip(v, gamma)]


def test_rms_norm_bf16i_known_answer(orc):
    # x = [3, 4] (f32), gamma 1, scale 1: ss = 25, 1/sqrt(25) = 0.2 -> bf16 0.2001953125
    # (205 * 2^-10); y = [0.6005859375 -> 0.6015625 (154 * 2^-8), 0.80078125 (exact)].
    y = orc.rms_norm(np.array([[3.0, 4.0]], np.float32), F32, np.ones(2, np.float32), F32, BF16, 1.0, 1e-12,
                     mode=BF16I)
    assert_bitexact(y.reshape(-1), bf16_bits([0.6015625, 0.80078125]), "rms known answer 1")
    # x = [1, 0], gamma = [1.001, 1] (f32), scale 1.003: v = 1, ss = 1, inv = 1, bf16(gamma)
    # = 1.0, y0 = bf16(1 * 1 * 1 * 1.003) = 1.0; exact maths: 1.001 * 1.003 = 1.004003 ->
    # bf16 1.0078125 (ulp 2^-7: 128.51 * 2^-7), so the gamma rounding decides the result.
    x = np.array([[1.0, 0.0]], np.float32)
    gamma = np.array([1.001, 1.0], np.float32)
    y = orc.rms_norm(x, F32, gamma, F32, BF16, 1.003, 1e-12, mode=BF16I)
    assert_bitexact(y.reshape(-1), bf16_bits([1.0, 0.0]), "rms known answer 2 (gamma rounded)")
    y = orc.rms_norm(x, F32, gamma, F32, BF16, 1.003, 1e-12, mode=EXACT)
    assert_bitexact(y.reshape(-1), bf16_bits([1.0078125, 0.0]), "rms known answer 2, exact mode")


def test_rms_norm_bf16i_matches_exact_rationals(orc):
    rng = np.random.default_rng(11)
    differs = 0
    for case in range(12):
        dim = int(rng.integers(2, 9))
        x = (rng.standard_normal((1, dim)) * 3).astype(np.float32)
        gamma = (1 + 0.1 * rng.standard_normal(dim)).astype(np.float32)
        scale = float(np.float32(math.sqrt(dim)))
        want = rms_exact(x[0], gamma, scale, 1e-12)
        got = orc.rms_norm(x, F32, gamma, F32, BF16, scale, 1e-12, mode=BF16I)
        assert_bitexact(got.reshape(-1), bf16_bits(want), f"rms case {case}")
        differs += not np.array_equal(got, orc.rms_norm(x, F32, gamma, F32, BF16, scale, 1e-12, mode=EXACT))
    assert differs >= 3, "inputs never exercise the bf16 rounding points"


def test_residual_rms_norm_bf16i_rounds_the_sum(orc):
    # with an f32 residual the stored sum keeps f32; the norm reads it rounded to bf16
    rng = np.random.default_rng(12)
    x = rng.standard_normal((3, 8)).astype(np.float32)
    u = rng.standard_normal((3, 8)).astype(np.float32)
    gamma = np.ones(8, np.float32)
    y, s = orc.rms_norm(x, F32, gamma, F32, BF16, 2.0, 1e-12, res=u, sdt=F32, mode=BF16I, want_sum=True)
    assert_bitexact(s, (x + u).astype(np.float32), "residual sum")
    for r in range(3):
        assert_bitexact(y[r], bf16_bits(rms_exact(x[r] + u[r], gamma, 2.0, 1e-12)), f"residual row {r}")


# ---- softmax (src/mbr_cuda_tile.cu:5224-5252) ----------------------------------------------

def softmax_exact(xb, scale):
    z = [rb(v * fr(np.float32(scale))) for v in as_fr(xb)]
    m = max(z)
    e = [rb(dexp(t - m)) for t in z]
    d = rb(sum(e))
    return [rb(t / d) for t in e]


def test_softmax_bf16i_known_answer(orc):
    # row [1, 0, 0], scale 3: z = [3, 0, 0], max 3, e = [1, bf16(e^-3 = 0.049787..) =
    # 0.0498046875 (204 * 2^-12), the same], sum 1.099609375 -> bf16 1.1015625 (141 * 2^-7),
    # p0 = 1 / 1.1015625 = 0.907801.. -> 0.90625 (232 * 2^-8), p1 = 0.0498046875 / 1.1015625
    # = 0.045213.. -> 0.045166015625 (185 * 2^-12).  Exact maths: p0 = 1 / (1 + 2 e^-3) =
    # 0.909443.. -> 0.91015625 (233 * 2^-8), p1 = 0.0452785.. -> 0.045166015625.
    x = bf16_bits([1.0, 0.0, 0.0])
    assert_bitexact(orc.softmax(x[None], BF16, BF16, 3.0, mode=BF16I)[0],
                    bf16_bits([0.90625, 0.045166015625, 0.045166015625]), "softmax scale 3")
    assert_bitexact(orc.softmax(x[None], BF16, BF16, 3.0, mode=EXACT)[0],
                    bf16_bits([0.91015625, 0.045166015625, 0.045166015625]), "softmax scale 3 exact mode")


def test_softmax_bf16i_matches_exact_rationals(orc):
    rng = np.random.default_rng(13)
    differs = 0
    for case in range(10):
        cols = int(rng.integers(2, 24))
        x = bf16_inputs(rng, (1, cols), 2.0)
        scale = float(np.float32(0.125 if case % 2 else 1.0))
        got = orc.softmax(x, BF16, BF16, scale, mode=BF16I)
        assert_bitexact(got[0], bf16_bits(softmax_exact(x[0], scale)), f"softmax case {case}")
        differs += not np.array_equal(got, orc.softmax(x, BF16, BF16, scale, mode=EXACT))
    assert differs >= 3


# ---- GLU (src/mbr_cuda_tile.cu:5918-5940) ----------------------------------------------------

def test_glu_bf16i_known_answer_and_rationals(orc):
    # a = 3, b = 1: sigmoid(1) = 0.7310585.. -> bf16 0.73046875 (187 * 2^-8);
    # 3 * 0.73046875 = 2.19140625 -> 2.1875 (140 * 2^-6); exact 2.19317.. -> 2.1875.
    # a = 0.28125, b = 1: 0.28125 * 0.73046875 = 0.2054443359375 -> 0.205078125
    # (210 * 2^-10, 210.375 rounded down); exact 0.205610.. -> 0.2060546875 (211 * 2^-10).
    x = bf16_bits([3.0, 0.28125, 1.0, 1.0])[None]
    assert_bitexact(orc.glu(x, BF16, BF16, mode=BF16I)[0], bf16_bits([2.1875, 0.205078125]), "glu known answer")
    assert_bitexact(orc.glu(x, BF16, BF16, mode=EXACT)[0], bf16_bits([2.1875, 0.2060546875]), "glu exact mode")
    rng = np.random.default_rng(14)
    x = bf16_inputs(rng, (4, 16), 3.0)
    got = orc.glu(x, BF16, BF16, mode=BF16I)
    for r in range(4):
        a, b = as_fr(x[r, :8]), as_fr(x[r, 8:])
        want = [rb(ai * rb(1 / (1 + dexp(-bi)))) for ai, bi in zip(a, b)]
        assert_bitexact(got[r], bf16_bits(want), f"glu row {r}")
    assert not np.array_equal(got, orc.glu(x, BF16, BF16, mode=EXACT))


# ---- gate merge (src/mbr_cuda_tile.cu:4718-4750) ----------------------------------------------

def test_gate_merge_bf16i(orc):
    rng = np.random.default_rng(15)
    B, H, N, D = 1, 2, 3, 4
    attn = bf16_inputs(rng, (B, H, N, D), 2.0)
    gl = rng.standard_normal((B, N, H)).astype(np.float32)
    for odt in (BF16, F32):
        for logit in (True, False):
            got = orc.gate_merge(attn, BF16, gl, F32, odt, B, H, N, D, logit=logit, mode=BF16I)
            a = np.array(as_fr(attn)).reshape(B, H, N, D)
            want = []
            for n in range(N):
                for h in range(H):
                    g = fr(gl[0, n, h])
                    g = rb(1 / (1 + dexp(-g))) if logit else rb(g)
                    want += [rb(a[0, h, n, d] * g) for d in range(D)]
            want_arr = bf16_bits(want) if odt == BF16 else np.array([float(w) for w in want], np.float32)
            assert_bitexact(got.reshape(-1), want_arr, f"gate merge odt={odt} logit={logit}")
    # bf16 gates without a sigmoid and bf16 output: every intermediate is a bf16 product
    # rounded once, the same as the default mode
    gb = bf16_inputs(rng, (B, N, H))
    assert_bitexact(orc.gate_merge(attn, BF16, gb, BF16, BF16, B, H, N, D, logit=False, mode=BF16I),
                    orc.gate_merge(attn, BF16, gb, BF16, BF16, B, H, N, D, logit=False, mode=EXACT), "identity")


# ---- rotary and split (src/mbr_cuda_tile.cu:4000-4068) -----------------------------------------

def test_rotary_bf16i_rounds_the_tables(orc):
    rng = np.random.default_rng(16)
    n_pos, heads, D = 5, 2, 8
    cos, sin = orc.rotary_tables(n_pos, D)
    q = bf16_inputs(rng, (1, n_pos, heads, D))
    k = bf16_inputs(rng, (1, n_pos, heads, D))
    qr, kr = orc.rotary(q, k, BF16, cos, sin, F32, n_pos, heads, layout=1, mode=BF16I)
    # the same as the default mode with bf16-rounded tables, and different from it with f32 ones
    cb, sb = orc.f32_to_bf16(cos), orc.f32_to_bf16(sin)
    qe, ke = orc.rotary(q, k, BF16, cb, sb, BF16, n_pos, heads, layout=1, mode=EXACT)
    assert_bitexact(qr, qe, "rotary q")
    assert_bitexact(kr, ke, "rotary k")
    assert not np.array_equal(qr, orc.rotary(q, k, BF16, cos, sin, F32, n_pos, heads, layout=1, mode=EXACT)[0])
    # one pair by hand: x = (1, 1), cos = sin = 0.70710678 (f32) -> bf16 0.70703125;
    # y0 = 0, y1 = 2 * 0.70703125 = 1.4140625 (exact) against exact maths 1.41421.. -> 1.4140625,
    # and x = (3, 1): y0 = 2 * 0.70703125 = 1.4140625, y1 = 4 * 0.70703125 = 2.828125
    # against 2.8284.. -> 2.828125; x = (5, 0): y = (3.53515625, 3.53515625) -> bf16
    # 3.53125 (ulp 2^-6: 226.25 * 2^-6) against 3.5355.. -> 3.53125 (226.27)
    c = np.full((1, 1), 0.70710678, np.float32)
    qq = bf16_bits([1.0, 1.0])[None, None, None]
    out, _ = orc.rotary(qq, None, BF16, c, c, F32, 1, 1, layout=1, mode=BF16I)
    assert_bitexact(out.reshape(-1), bf16_bits([0.0, 1.4140625]), "rotary pair by hand")


def test_split_qkv_bf16i_rounds_the_tables(orc):
    rng = np.random.default_rng(17)
    B, N, H, D = 1, 4, 2, 8
    cos, sin = orc.rotary_tables(N, D)
    qkv = bf16_inputs(rng, (B, N, 3 * H * D))
    q, k, v = orc.split_qkv(qkv, BF16, cos, sin, F32, BF16, B, N, H, D, N, mode=BF16I)
    cb, sb = orc.f32_to_bf16(cos), orc.f32_to_bf16(sin)
    qe, ke, ve = orc.split_qkv(qkv, BF16, cb, sb, BF16, BF16, B, N, H, D, N, mode=EXACT)
    for a, b, name in ((q, qe, "q"), (k, ke, "k"), (v, ve, "v")):
        assert_bitexact(a, b, f"split {name}")


# ---- band mask merge (src/mbr_cuda_tile.cu:5650-5797) -------------------------------------------

def _tiny_bands():
    # F = 3 freqs (C = 1), J = 4 band-bins: freq 0 <- bins {0, 1}, freq 1 <- {2}, freq 2 <- {3}
    off = np.array([0, 2, 3, 4], np.int32)
    ind = np.array([0, 1, 2, 3], np.int32)
    cnt = np.array([2.0, 1.0, 1.0], np.float32)
    return off, ind, cnt


def test_band_merge_bf16i_reduce_and_scatter_forms(orc):
    rng = np.random.default_rng(18)
    off, ind, cnt = _tiny_bands()
    B, F, T, J, S = 1, 3, 5, 4, 2
    stft = rng.standard_normal((B, F, T, 2)).astype(np.float32)
    masks = [bf16_inputs(rng, (B, T, 2 * J)) for _ in range(S)]
    got_b = orc.band_mask_merge(stft, masks, BF16, off, ind, cnt, F32, BF16, B, F, T, 1, mode=BF16I)
    got_f = orc.band_mask_merge(stft, masks, BF16, off, ind, cnt, F32, F32, B, F, T, 1, mode=BF16I)
    for s in range(S):
        m = np.array(as_fr(masks[s])).reshape(B, T, J, 2)
        for f in range(F):
            for t in range(T):
                sr, si = fr(stft[0, f, t, 0]), fr(stft[0, f, t, 1])
                den = fr(cnt[f])
                # reduce form (BF16 output): masks summed with a rounding per add
                ar = ai = Fraction(0)
                for e in range(off[f], off[f + 1]):
                    ar, ai = rb(ar + m[0, t, ind[e], 0]), rb(ai + m[0, t, ind[e], 1])
                want = bf16_bits([rb((sr * ar - si * ai) / den), rb((sr * ai + si * ar) / den)])
                assert_bitexact(got_b[s, f, t], want, f"reduce form s={s} f={f} t={t}")
                # scatter form (F32 output): each entry's value rounded, then added
                vr = vi = Fraction(0)
                for e in range(off[f], off[f + 1]):
                    mr, mi = m[0, t, ind[e], 0], m[0, t, ind[e], 1]
                    vr += rb((sr * mr - si * mi) / den)
                    vi += rb((sr * mi + si * mr) / den)
                want = np.array([r32(vr), r32(vi)], np.float32)
                assert_bitexact(got_f[s, f, t], want, f"scatter form s={s} f={f} t={t}")
    assert not np.array_equal(got_b, orc.band_mask_merge(stft, masks, BF16, off, ind, cnt, F32, BF16, B, F, T, 1))
    assert not np.array_equal(got_f, orc.band_mask_merge(stft, masks, BF16, off, ind, cnt, F32, F32, B, F, T, 1))
