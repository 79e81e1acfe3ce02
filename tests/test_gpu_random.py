"""Seeded random-shape parity sweep: the row softmax, the sigmoid gate merge, RMSNorm and
GLU over random shapes, dtypes and layouts (every kernel form their launchers pick), and
the widened entry points: the fused attention in its strided / q-rotary / gated forms, the
attention with n_q != n_k, and the STFT / iSTFT over random lengths, hops, centring,
normalisation and windows.  Every case is drawn from a
fixed seed at import, so a failure names a reproducible shape; the sizes stay small
enough for the float64 oracle.

The fused attention is compared bit for bit with the separate GPU ops (rotary, attention,
gate merge) and, stage by stage, with the oracle; the rest with the oracle under
parity.py's rules.  A centred f32 STFT with hop <= n_fft/2 is also inverted back to its
signal.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import mbrt
from gpu_util import empty, say, to_dev, to_host
from parity import BF16, F16, F32, assert_bitexact, assert_close

pytestmark = pytest.mark.gpu

N_FFT = 2048


def _cases():
    rng = np.random.default_rng(0x4D42520F)
    pick = lambda lo, hi: int(rng.integers(lo, hi))  # noqa: E731
    attn = [(pick(1, 4), pick(1, 300), pick(1, 7), bool(pick(0, 2)), bool(pick(0, 2)), [BF16, F32][pick(0, 2)],
             [F32, BF16][pick(0, 2)]) for _ in range(10)]
    cross = [(pick(1, 5), pick(1, 260), pick(1, 260)) for _ in range(6)]
    stft = []
    while len(stft) < 8:
        B, L, center = pick(1, 4), pick(50, 30000), bool(pick(0, 2))
        hop = int(np.exp(rng.uniform(0.0, np.log(2600.0))))   # log-uniform: small hops too
        normalized, win, dt = bool(pick(0, 2)), ["hann", "rand"][pick(0, 2)], [F32, BF16][pick(0, 2)]
        if not center and L < N_FFT:
            continue
        frames = L // hop + 1 if center else (L - N_FFT) // hop + 1
        if frames <= 1500:   # keeps the oracle's O(frames * n_fft log n_fft) work in seconds
            stft.append((B, L, hop, center, normalized, win, dt))
    return attn, cross, stft


ATTN_CASES, CROSS_CASES, STFT_CASES = _cases()

SM_DTYPES = [(F32, F32), (BF16, BF16), (F32, BF16), (BF16, F32), (F16, F16)]


def _op_cases():
    rng = np.random.default_rng(0x4D425210)
    pick = lambda lo, hi: int(rng.integers(lo, hi))  # noqa: E731
    # row counts and lengths spread over every softmax form: short rows in groups of 4-16
    # lanes, the 2-byte row pairs (33..64, a multiple of 4, even row counts), the staged
    # spans of 129..1024 and the unaligned and long-row kernels
    softmax = []
    for _ in range(24):
        cols = [pick(1, 33), 4 * pick(9, 17), pick(33, 129), pick(129, 1025), pick(1025, 3000)][pick(0, 5)]
        rows = pick(1, 2500) * [1, 2][pick(0, 2)]
        softmax.append((rows, cols, SM_DTYPES[pick(0, 5)], round(float(rng.uniform(0.05, 2.0)), 3)))
    gate = [(pick(1, 5), pick(1, 10), pick(1, 200), [4, 5, 8, 12, 16, 32, 64, 128][pick(0, 8)],
             [(BF16, BF16, BF16), (F32, F32, F32), (BF16, F32, BF16), (F16, F16, F16), (BF16, BF16, F32)][pick(0, 5)],
             bool(pick(0, 2)), bool(pick(0, 2))) for _ in range(12)]
    rms = [(pick(1, 400), pick(1, 5000), [(F32, F32, F32), (BF16, F32, BF16), (BF16, BF16, BF16), (F16, F32, F16)][pick(0, 4)])
           for _ in range(8)]
    glu = [(pick(1, 300), pick(1, 700), [(F32, F32), (BF16, BF16), (F32, BF16), (F16, F16)][pick(0, 4)])
           for _ in range(8)]
    return softmax, gate, rms, glu


SM_CASES, GATE_CASES, RMS_CASES, GLU_CASES = _op_cases()


def _inp(orc, shape, seed, stream, dt, std=1.0):
    x = orc.randn(shape, seed=seed, stream=stream, std=std)
    return x if dt == F32 else orc.from_f32(x, dt)


@pytest.mark.parametrize("rows,cols,dts,scale", SM_CASES)
def test_random_softmax(orc, dev, rows, cols, dts, scale):
    idt, odt = dts
    say(f"random softmax rows={rows} cols={cols} {idt}->{odt} scale={scale}")
    x = _inp(orc, (rows, cols), 0x4D425200D1, rows * 7 + cols, idt, std=3.0)
    xd = to_dev(x, idt)
    y = empty((rows, cols), odt)
    mbrt.softmax(xd, y, scale)
    torch.cuda.synchronize()
    assert_close(to_host(y, odt), orc.softmax(x, idt, odt, scale), odt, "softmax")
    if idt == odt:
        mbrt.softmax(xd, xd, scale)
        torch.cuda.synchronize()
        assert_bitexact(to_host(xd, odt), to_host(y, odt), "softmax in place")


@pytest.mark.parametrize("B,H,N,D,dts,logit,bnhd", GATE_CASES)
def test_random_gate_merge(orc, dev, B, H, N, D, dts, logit, bnhd):
    adt, gdt, odt = dts
    say(f"random gate merge B={B} H={H} N={N} D={D} {adt},{gdt}->{odt} logit={logit} bnhd={bnhd}")
    attn = _inp(orc, (B, H, N, D), 0x4D425200D2, N * 13 + D, adt)
    gate = _inp(orc, (B, N, H), 0x4D425200D3, N * 13 + D, gdt, std=2.0)
    ref = orc.gate_merge(attn, adt, gate, gdt, odt, B, H, N, D, layout=0, logit=logit)
    y = empty((B, N, H * D), odt)
    if bnhd:
        mbrt.gate_merge(to_dev(np.ascontiguousarray(attn.transpose(0, 2, 1, 3)), adt), to_dev(gate, gdt), y,
                        mbrt.LAYOUT_BNHD, gate_is_logit=logit)
    else:
        mbrt.gate_merge(to_dev(attn, adt), to_dev(gate, gdt), y, mbrt.LAYOUT_BHND, gate_is_logit=logit)
    torch.cuda.synchronize()
    assert_close(to_host(y, odt), ref, odt, "gate merge")


@pytest.mark.parametrize("rows,D,dts", RMS_CASES)
def test_random_rmsnorm(orc, dev, rows, D, dts):
    xdt, gdt, odt = dts
    say(f"random rms_norm rows={rows} D={D} {xdt},{gdt}->{odt}")
    x = _inp(orc, (rows, D), 0x4D425200D4, rows + D, xdt)
    g = orc.randn((D,), seed=0x4D425200D5, stream=D, mean=1.0, std=0.02)
    g = g if gdt == F32 else orc.from_f32(g, gdt)
    y = empty((rows, D), odt)
    mbrt.rms_norm(to_dev(x, xdt), to_dev(g, gdt), y, scale=float(np.sqrt(D)), eps=1e-8)
    torch.cuda.synchronize()
    assert_close(to_host(y, odt), orc.rms_norm(x, xdt, g, gdt, odt, float(np.sqrt(D)), 1e-8), odt, "rms")


@pytest.mark.parametrize("rows,half,dts", GLU_CASES)
def test_random_glu(orc, dev, rows, half, dts):
    xdt, odt = dts
    say(f"random glu rows={rows} half={half} {xdt}->{odt}")
    x = _inp(orc, (rows, 2 * half), 0x4D425200D6, rows + half, xdt, std=1.5)
    y = empty((rows, half), odt)
    mbrt.glu(to_dev(x, xdt), y)
    torch.cuda.synchronize()
    assert_close(to_host(y, odt), orc.glu(x, xdt, odt), odt, "glu")


@pytest.mark.parametrize("B,N,H,rot,gate,odt,tdt", ATTN_CASES)
def test_random_attention_bnhd(orc, dev, B, N, H, rot, gate, odt, tdt):
    say(f"random attention_bnhd B={B} N={N} H={H} rot={rot} gate={gate} out={odt} trig={tdt}")
    qkv = to_dev(_inp(orc, (B, N, 3 * H * 64), 0x4D425200C0, N * 8 + H, BF16), BF16)
    v5 = qkv.view(B, N, 3, H, 64)
    q, k, v = v5[:, :, 0], v5[:, :, 1], v5[:, :, 2]
    cos_h, sin_h = orc.rotary_tables(N, 64)
    if tdt == BF16:
        cos_h, sin_h = orc.from_f32(cos_h, BF16), orc.from_f32(sin_h, BF16)
    cos, sin = to_dev(cos_h, tdt), to_dev(sin_h, tdt)
    g_h = _inp(orc, (B, N, H), 0x4D425200C1, N, BF16, std=2.0)
    g = to_dev(g_h, BF16)
    fused = mbrt.attention_bnhd(q, k, v, cos=cos if rot else None, sin=sin if rot else None,
                                gate=g if gate else None, out_dtype=torch.float32 if odt == F32 else torch.bfloat16)
    qc, kc, vc = (t.permute(0, 2, 1, 3).contiguous().view(B * H, N, 64) for t in (q, k, v))
    if rot:
        mbrt.rotary_(qc, None, cos, sin)
    att = empty((B, H, N, 64), odt)
    mbrt.attention(qc, kc, vc, att.view(B * H, N, 64), 0.0)
    sep = att
    if gate:
        sep = empty((B, N, H * 64), odt)
        mbrt.gate_merge(att, g, sep)
    torch.cuda.synchronize()
    assert tuple(fused.shape) == tuple(sep.shape)
    assert_bitexact(to_host(fused, odt), to_host(sep, odt), "attention_bnhd = separate ops")
    qh, kh, vh = (to_host(t, BF16) for t in (qc, kc, vc))
    ref = orc.attention(qh, kh, vh, BF16, odt, 0.0).reshape(B, H, N, 64)
    den = orc.attention(orc.to_f32(qh, BF16), orc.to_f32(kh, BF16), np.abs(orc.to_f32(vh, BF16)), F32, F32,
                        0.0).reshape(B, H, N, 64)
    assert_close(to_host(att, odt), ref, odt, "attention", den=den)
    if gate:
        gref = orc.gate_merge(to_host(att, odt), odt, g_h, BF16, odt, B, H, N, 64)
        assert_close(to_host(fused, odt), gref, odt, "gate merge")


@pytest.mark.parametrize("BH,nq,nk", CROSS_CASES)
def test_random_attention_cross(orc, dev, BH, nq, nk):
    say(f"random attention BH={BH} nq={nq} nk={nk}")
    q = _inp(orc, (BH, nq, 64), 0x4D425200C2, nq, BF16)
    k = _inp(orc, (BH, nk, 64), 0x4D425200C3, nk, BF16)
    v = _inp(orc, (BH, nk, 64), 0x4D425200C4, nk, BF16)
    out = empty((BH, nq, 64), F32)
    mbrt.attention(to_dev(q, BF16), to_dev(k, BF16), to_dev(v, BF16), out, 0.0)
    torch.cuda.synchronize()
    ref = orc.attention(q, k, v, BF16, F32, 0.0)
    den = orc.attention(orc.to_f32(q, BF16), orc.to_f32(k, BF16), np.abs(orc.to_f32(v, BF16)), F32, F32, 0.0)
    assert_close(to_host(out, F32), ref, F32, "attention", den=den)


@pytest.mark.parametrize("B,L,hop,center,normalized,win,dt", STFT_CASES)
def test_random_stft_istft(orc, dev, B, L, hop, center, normalized, win, dt):
    say(f"random stft/istft B={B} L={L} hop={hop} center={center} normalized={normalized} window={win} "
        f"spec={dt}")
    x = orc.randn((B, L), seed=0x4D425200C5, stream=L)
    w = orc.hann_window(N_FFT) if win == "hann" else \
        (np.random.default_rng(L).random(N_FFT) * 0.9 + 0.1).astype(np.float32)
    wd = to_dev(w, F32)
    spec = mbrt.stft(to_dev(x, F32), wd, hop, center, normalized)
    torch.cuda.synchronize()
    assert_close(to_host(spec, F32), orc.stft(x, w, hop, center, normalized), F32, "stft",
                 den=orc.stft_den(x, w, hop, center, normalized))
    if dt == BF16:
        spec = spec.to(torch.bfloat16)
    y = mbrt.istft(spec, wd, hop, center, normalized, L)
    torch.cuda.synchronize()
    sh = to_host(spec, dt)
    yh = to_host(y, F32)
    assert_close(yh, orc.istft(sh, dt, w, hop, center, normalized, L), F32, "istft",
                 den=orc.istft_den(sh, dt, w, hop, center, normalized, L))
    if dt == F32 and center and win == "hann" and hop <= N_FFT // 2:
        n = min(L, mbrt.istft_output_length(spec.shape[2], hop, True))
        assert np.abs(yh[:, :n] - x[:, :n]).max() <= 1e-5 * np.abs(x).max(), "istft(stft(x)) != x"
