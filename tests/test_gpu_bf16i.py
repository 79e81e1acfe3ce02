"""GPU parity of the bf16-intermediates mode (MBRT_ARITH_BF16_INTERMEDIATES, the
reference's full-bf16 experiment mode) against the oracle's ORC_BF16I.

Rule: the kernels evaluate each step in f32 and round it to bf16 where the reference does;
the oracle evaluates each step exactly (double) and rounds once.  The two agree except
where a step's f32 value lies within an f32 rounding of a bf16 tie, and such a step moves
its output by one bf16 ulp (two where it feeds a later rounded step, e.g. a row sum).  So
every element must lie within 2 bf16 ulps of the oracle and at least 98 % must be
identical.  F32 outputs built from rounded terms (the band merge's scatter form) are held
to 2^-7 of the magnitude they are summed from.  Each case also checks that the flag
reaches the kernels: the outputs differ from the default mode's on these inputs.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import mbrt
from gpu_util import empty, say, to_dev, to_host
from parity import BF16, F32, I32, RTOL_F32, _f32, _ulp, assert_bitexact, merge_den

pytestmark = pytest.mark.gpu

BF16I = 2
FB = mbrt.ARITH_BF16_INTERMEDIATES


@pytest.fixture(scope="module", autouse=True)
def _threads(orc):
    orc.set_threads(8)


def inp(orc, shape, seed, stream, dt=F32, mean=0.0, std=1.0):
    x = orc.randn(shape, seed=seed, stream=stream, mean=mean, std=std)
    return x if dt == F32 else orc.from_f32(x, dt)


def assert_bf16i(y, ref, dt, what, max_ulp=2.0, min_exact=0.98, den=None):
    """`den`: magnitude of the terms an output is a difference of (complex products); the
    f32 evaluation of such a difference may then also be off by 1e-5 of it."""
    a, b = _f32(y, dt).reshape(-1), _f32(ref, dt).reshape(-1)
    assert np.isfinite(a).all() and np.isfinite(b).all(), what
    ulp = _ulp(np.maximum(np.abs(b), 1e-30), BF16)
    err = np.abs(a - b) / ulp
    if den is not None:
        err = err - RTOL_F32 * np.asarray(den, np.float64).reshape(-1) / ulp
    worst = int(np.argmax(err))
    assert err[worst] <= max_ulp, f"{what}: {err[worst]:.2f} bf16 ulp off at {worst}: got {a[worst]} want {b[worst]}"
    exact = float(np.mean(a == b))
    assert exact >= min_exact, f"{what}: only {exact:.4f} of the elements equal the oracle's"


def both_modes(run):
    """Runs `run()` (which returns a host array) with the flag set and with it clear."""
    with mbrt.arith_flags(FB):
        y = run()
    assert mbrt.get_arith_flags() == 0
    return y, run()


@pytest.mark.parametrize("D,xdt", [(384, BF16), (384, F32), (256, F32), (101, F32), (5000, BF16)])
def test_rms_norm_bf16i(orc, dev, D, xdt):
    say(f"bf16i rms_norm D={D} x={xdt}")
    rows = 64
    scale = float(np.sqrt(D))
    x = inp(orc, (rows, D), 301, D, xdt)
    g = inp(orc, (D,), 302, D, F32, mean=1.0, std=0.05)
    xd, gd = to_dev(x, xdt), to_dev(g, F32)

    def run():
        y = empty((rows, D), BF16)
        mbrt.rms_norm(xd, gd, y, scale=scale, eps=1e-12)
        torch.cuda.synchronize()
        return to_host(y, BF16)

    yf, yd = both_modes(run)
    assert_bf16i(yf, orc.rms_norm(x, xdt, g, F32, BF16, scale, 1e-12, mode=BF16I), BF16, "rms")
    assert not np.array_equal(yf, yd)


@pytest.mark.parametrize("D,xdt", [(384, BF16), (384, F32), (101, F32)])
def test_residual_rms_norm_bf16i(orc, dev, D, xdt):
    say(f"bf16i residual rms_norm D={D} x={xdt}")
    rows = 48
    scale = float(np.sqrt(D))
    x = inp(orc, (rows, D), 303, D, xdt)
    r = inp(orc, (rows, D), 304, D, xdt)
    g = inp(orc, (D,), 305, D, F32, mean=1.0, std=0.05)
    xd, rd, gd = to_dev(x, xdt), to_dev(r, xdt), to_dev(g, F32)

    def run():
        s, y = empty((rows, D), xdt), empty((rows, D), BF16)
        mbrt.residual_add_rms_norm(xd, rd, gd, s, y, scale, 1e-12)
        torch.cuda.synchronize()
        return np.concatenate([to_host(y, BF16).view(np.uint8).reshape(-1), to_host(s, xdt).view(np.uint8).reshape(-1)])

    with mbrt.arith_flags(FB):
        s, y = empty((rows, D), xdt), empty((rows, D), BF16)
        mbrt.residual_add_rms_norm(xd, rd, gd, s, y, scale, 1e-12)
        torch.cuda.synchronize()
    ry, rs = orc.rms_norm(x, xdt, g, F32, BF16, scale, 1e-12, res=r, sdt=xdt, mode=BF16I, want_sum=True)
    assert_bitexact(to_host(s, xdt), rs, "residual sum (the stored sum is not rounded further)")
    assert_bf16i(to_host(y, BF16), ry, BF16, "residual normed")
    fb, default = both_modes(run)
    assert not np.array_equal(fb, default)


# 960x60 and 64x64: staged short rows; 96x801: staged long rows; 41x801: the register
# kernel (the span is not whole 16-byte vectors); 16x3000: the loop kernel
@pytest.mark.parametrize("rows,cols", [(960, 60), (64, 64), (96, 801), (41, 801), (16, 3000)])
def test_softmax_bf16i(orc, dev, rows, cols):
    say(f"bf16i softmax {rows}x{cols}")
    x = inp(orc, (rows, cols), 306, cols, BF16, std=3.0)
    xd = to_dev(x, BF16)

    def run():
        y = empty((rows, cols), BF16)
        mbrt.softmax(xd, y, 0.125)
        torch.cuda.synchronize()
        return to_host(y, BF16)

    yf, yd = both_modes(run)
    assert_bf16i(yf, orc.softmax(x, BF16, BF16, 0.125, mode=BF16I), BF16, "softmax")
    assert not np.array_equal(yf, yd)
    # in place
    with mbrt.arith_flags(FB):
        xi = to_dev(x, BF16)
        mbrt.softmax(xi, xi, 0.125)
        torch.cuda.synchronize()
    assert np.array_equal(to_host(xi, BF16), yf), "in-place differs from out-of-place"


def test_softmax_bf16i_leaves_other_dtypes(orc, dev):
    # the reference rounds intermediates only in its bf16 -> bf16 kernels
    say("bf16i softmax f32 -> bf16 unchanged")
    x = inp(orc, (64, 801), 307, 1, F32, std=3.0)
    xd = to_dev(x, F32)

    def run():
        y = empty((64, 801), BF16)
        mbrt.softmax(xd, y, 0.125)
        torch.cuda.synchronize()
        return to_host(y, BF16)

    yf, yd = both_modes(run)
    assert np.array_equal(yf, yd)


@pytest.mark.parametrize("half", [256, 64, 33])
def test_glu_bf16i(orc, dev, half):
    say(f"bf16i glu half={half}")
    rows = 200
    x = inp(orc, (rows, 2 * half), 308, half, BF16, std=2.0)
    xd = to_dev(x, BF16)

    def run():
        y = empty((rows, half), BF16)
        mbrt.glu(xd, y)
        torch.cuda.synchronize()
        return to_host(y, BF16)

    yf, yd = both_modes(run)
    assert_bf16i(yf, orc.glu(x, BF16, BF16, mode=BF16I), BF16, "glu")
    assert not np.array_equal(yf, yd)


@pytest.mark.parametrize("D", [64, 6])
@pytest.mark.parametrize("odt", [BF16, F32])
@pytest.mark.parametrize("logit", [True, False])
def test_gate_merge_bf16i(orc, dev, D, odt, logit):
    say(f"bf16i gate merge D={D} out={odt} logit={logit}")
    B, H, N = 2, 8, 61
    attn = inp(orc, (B, H, N, D), 309, D, BF16)
    gate = inp(orc, (B, N, H), 310, D, F32, std=2.0)
    ad, gd = to_dev(attn, BF16), to_dev(gate, F32)

    def run():
        y = empty((B, N, H * D), odt)
        mbrt.gate_merge(ad, gd, y, mbrt.LAYOUT_BHND, gate_is_logit=logit)
        torch.cuda.synchronize()
        return to_host(y, odt)

    yf, yd = both_modes(run)
    ref = orc.gate_merge(attn, BF16, gate, F32, odt, B, H, N, D, layout=0, logit=logit, mode=BF16I)
    if logit:  # the f32 sigmoid may round to the other side of a bf16 tie
        assert_bf16i(yf, ref, odt, "gate merge", max_ulp=1.0, min_exact=0.99)
    else:  # one exact product of two bf16 values, rounded once: identical
        assert_bf16i(yf, ref, odt, "gate merge", max_ulp=0.0, min_exact=1.0)
    assert not np.array_equal(yf, yd)


@pytest.mark.parametrize("layout,D", [(mbrt.LAYOUT_BNHD, 64), (mbrt.LAYOUT_BHND, 64), (mbrt.LAYOUT_BNHD, 6)])
def test_rotary_bf16i(orc, dev, layout, D):
    say(f"bf16i rotary layout={layout} D={D}")
    B, N, H = 2, 801, 8
    cos, sin = orc.rotary_tables(N, D)
    shape = (B, N, H, D) if layout == mbrt.LAYOUT_BNHD else (B * H, N, D)
    q = inp(orc, shape, 311, D, BF16)
    k = inp(orc, shape, 312, D, BF16)
    cd, sd = to_dev(cos, F32), to_dev(sin, F32)

    def run():
        qd, kd = to_dev(q, BF16), to_dev(k, BF16)
        mbrt.rotary_(qd, kd, cd, sd, layout, heads=H)
        torch.cuda.synchronize()
        return np.stack([to_host(qd, BF16), to_host(kd, BF16)])

    yf, yd = both_modes(run)
    rq, rk = orc.rotary(q, k, BF16, cos, sin, F32, N, H, layout=layout, mode=BF16I)
    # exact bf16 products; their f32 sum is rounded to bf16 (a second rounding where the
    # sum needs more than 24 bits, which the oracle's double sum does not)
    assert_bf16i(yf, np.stack([rq, rk]), BF16, "rotary", max_ulp=1.0, min_exact=0.999)
    assert not np.array_equal(yf, yd)


@pytest.mark.parametrize("D", [64, 6])
def test_split_qkv_bf16i(orc, dev, D):
    say(f"bf16i split qkv D={D}")
    B, N, H, out_n = 2, 60, 8, 64
    cos, sin = orc.rotary_tables(N, D)
    qkv = inp(orc, (B, N, 3 * H * D), 313, D, BF16)
    xd, cd, sd = to_dev(qkv, BF16), to_dev(cos, F32), to_dev(sin, F32)

    def run():
        q, k, v = (empty((B, H, out_n, D), BF16) for _ in range(3))
        mbrt.split_qkv_rotary(xd, cd, sd, q, k, v, H)
        torch.cuda.synchronize()
        return np.stack([to_host(t, BF16) for t in (q, k, v)])

    yf, yd = both_modes(run)
    ref = np.stack(orc.split_qkv(qkv, BF16, cos, sin, F32, BF16, B, N, H, D, out_n, mode=BF16I))
    assert_bf16i(yf, ref, BF16, "split qkv", max_ulp=1.0, min_exact=0.999)
    assert not np.array_equal(yf, yd)


@pytest.mark.parametrize("odt", [BF16, F32])
def test_band_merge_bf16i(orc, dev, odt):
    say(f"bf16i band merge out={odt}")
    B, F, T, S = 1, 2050, 77, 2
    mb = orc.mel_bands(44100.0, 2048, 60, 2)
    J = mb["freq_indices"].size
    stft = inp(orc, (B, F, T, 2), 314, 1)
    masks = [inp(orc, (B, T, J * 2), 315, s, BF16, std=0.5) for s in range(S)]
    cnt = mb["bands_per_freq"].astype(np.float32)
    sd = to_dev(stft, F32)
    md = [to_dev(m, BF16) for m in masks]
    offd, indd, cntd = to_dev(mb["csr_offsets"], I32), to_dev(mb["csr_indices"], I32), to_dev(cnt, F32)

    def run():
        out = empty((B * S * 2, F // 2, T, 2), odt)
        mbrt.band_mask_merge(sd, md, offd, indd, cntd, out, 2)
        torch.cuda.synchronize()
        return to_host(out, odt)

    yf, yd = both_modes(run)
    ref = orc.band_mask_merge(stft, [m.reshape(B, T, J, 2) for m in masks], BF16, mb["csr_offsets"],
                              mb["csr_indices"], cnt, F32, odt, B, F, T, 2, mode=BF16I)
    den = merge_den(orc, stft, [orc.to_f32(m, BF16) for m in masks], mb, B, F, T, 2)
    if odt == BF16:
        assert_bf16i(yf, ref, BF16, "merge reduce form", den=den)
    else:
        err = np.abs(yf.astype(np.float64) - ref) / np.maximum(den, 1e-30)
        assert float(err.max()) <= 2.0 ** -7, f"merge scatter form: {err.max():.3e} of the summed magnitude"
        assert float(np.mean(yf == ref)) >= 0.9
    assert not np.array_equal(yf, yd)
