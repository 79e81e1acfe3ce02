"""GPU parity of the STFT / iSTFT entry points (mbrt_hann_window, mbrt_stft, mbrt_istft)
against the oracle's float64 restatement of src/stft_cuda_tile.cu.

f32 outputs follow parity.py's rule with `den` = the magnitude each output's sum of
products is taken from (sum |x w| over the frame for a bin; sum_t w |X_t| / 2048 for a
sample), which is what an f32 evaluation's rounding scales with.  The full chunk shape
(8 signals x 352800 samples, 801 frames) is compared in full, plus the round trip
istft(stft(x)) = x.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import mbrt
from gpu_util import say, to_dev, to_host
from parity import BF16, F32, assert_close

pytestmark = pytest.mark.gpu


def _window(orc, kind: str):
    if kind == "hann":
        return orc.hann_window(2048)
    return (np.random.default_rng(3).random(2048) * 0.9 + 0.1).astype(np.float32)


@pytest.mark.parametrize("size", [2048, 1000, 7, 2, 1])
def test_hann_window(orc, dev, size):
    say(f"hann_window {size}")
    out = mbrt.hann_window(size)
    torch.cuda.synchronize()
    assert_close(to_host(out, F32), orc.hann_window(size), F32, "hann", den=orc.hann_den(size))


@pytest.mark.parametrize("B,L,hop,center,normalized,win", [
    (1, 3000, 441, True, False, "hann"),
    (2, 20000, 441, True, True, "hann"),
    (3, 4000, 441, True, False, "rand"),     # 30 frames: workgroups span signals
    (3, 2048, 512, False, False, "hann"),    # one frame per signal
    (1, 700, 441, True, False, "hann"),      # shorter than the pad: reflect, then clamp
    (1, 5000, 7, True, False, "rand"),       # small hop: 715 frames
    (2, 10000, 3000, False, True, "hann"),   # hop > n_fft
    (3, 9001, 441, True, False, "rand"),     # signal rows start at every 4-byte alignment
    (2, 20000, 1910, True, False, "hann"),   # largest hop whose 8-frame span is staged in LDS
    (2, 20000, 1911, True, False, "hann"),   # smallest hop read frame by frame
])
def test_stft_shapes(orc, dev, B, L, hop, center, normalized, win):
    say(f"stft B={B} L={L} hop={hop} center={center} normalized={normalized} window={win}")
    x = orc.randn((B, L), seed=0x4D425200B0, stream=L)
    w = _window(orc, win)
    out = mbrt.stft(to_dev(x, F32), to_dev(w, F32), hop, center, normalized)
    torch.cuda.synchronize()
    ref = orc.stft(x, w, hop, center, normalized)
    den = orc.stft_den(x, w, hop, center, normalized)
    print("stft errors", assert_close(to_host(out, F32), ref, F32, "stft", den=den))


@pytest.mark.parametrize("shift", [1, 2, 3])
def test_stft_unaligned_buffers(orc, dev, shift):
    """Signal and window that start off a 16-byte (window: 8-byte) boundary."""
    say(f"stft unaligned by {shift} floats")
    B, L, hop = 2, 6000, 441
    x = orc.randn((B, L), seed=0x4D425200B2, stream=shift)
    w = _window(orc, "rand")
    xbuf = torch.zeros(B * L + shift, device=dev)
    xbuf[shift:] = to_dev(x, F32).reshape(-1)
    wbuf = torch.zeros(2048 + shift, device=dev)
    wbuf[shift:] = to_dev(w, F32)
    out = mbrt.stft(xbuf[shift:].view(B, L), wbuf[shift:], hop, True, False)
    torch.cuda.synchronize()
    ref = orc.stft(x, w, hop, True, False)
    den = orc.stft_den(x, w, hop, True, False)
    print("stft unaligned errors", assert_close(to_host(out, F32), ref, F32, "stft unaligned", den=den))


def test_stft_full_shape(orc, dev):
    """4 x 2 channels x 352800 samples (8 s at 44.1 kHz): [8, 1025, 801, 2]."""
    say("stft full [8, 352800] hop 441")
    x = orc.randn((8, 352800), seed=0x4D425200B1, stream=0)
    w = orc.hann_window(2048)
    out = mbrt.stft(to_dev(x, F32), to_dev(w, F32), 441, True, False)
    torch.cuda.synchronize()
    assert out.shape == (8, 1025, 801, 2)
    ref = orc.stft(x, w, 441, True, False)
    den = orc.stft_den(x, w, 441, True, False)
    print("stft full errors", assert_close(to_host(out, F32), ref, F32, "stft full", den=den))


@pytest.mark.parametrize("B,T,hop,center,normalized,length,dt,win", [
    (1, 7, 441, True, False, -1, F32, "hann"),
    (2, 46, 441, True, True, 20000, F32, "hann"),     # length beyond the signal: zero fill
    (3, 10, 441, True, False, 1500, BF16, "hann"),    # length trims
    (2, 9, 512, False, False, -1, F32, "rand"),
    (1, 1, 441, False, False, -1, BF16, "hann"),      # one frame: window sum w^2 with its 1e-8 cut
    (2, 5, 3000, False, True, -1, F32, "hann"),       # hop > n_fft: uncovered samples are 0
    (1, 300, 7, True, False, -1, F32, "rand"),        # small hop: 293 frames per sample
])
def test_istft_shapes(orc, dev, B, T, hop, center, normalized, length, dt, win):
    say(f"istft B={B} T={T} hop={hop} center={center} normalized={normalized} length={length} dt={dt} window={win}")
    spec = orc.randn((B, 1025, T, 2), seed=0x4D425200B2, stream=T)
    if dt == BF16:
        spec = orc.from_f32(spec, BF16)
    w = _window(orc, win)
    out = mbrt.istft(to_dev(spec, dt), to_dev(w, F32), hop, center, normalized, length)
    torch.cuda.synchronize()
    ref = orc.istft(spec, dt, w, hop, center, normalized, length)
    den = orc.istft_den(spec, dt, w, hop, center, normalized, length)
    assert out.shape == ref.shape
    print("istft errors", assert_close(to_host(out, F32), ref, F32, "istft", den=den))


@pytest.mark.parametrize("dt", [F32, BF16])
def test_istft_full_shape_and_round_trip(orc, dev, dt):
    """[8, 1025, 801, 2] spectra from the GPU STFT: the iSTFT matches the oracle on the same
    spectrum, and (f32) reconstructs the signal."""
    say(f"istft full [8, 1025, 801, 2] dt={dt}")
    L = 352800
    x = orc.randn((8, L), seed=0x4D425200B3, stream=0)
    w = orc.hann_window(2048)
    wd = to_dev(w, F32)
    spec = mbrt.stft(to_dev(x, F32), wd, 441, True, False)
    if dt == BF16:
        spec = spec.to(torch.bfloat16)
    y = mbrt.istft(spec, wd, 441, True, False, length=L)
    torch.cuda.synchronize()
    s = to_host(spec, dt)
    ref = orc.istft(s, dt, w, 441, True, False, L)
    den = orc.istft_den(s, dt, w, 441, True, False, L)
    yh = to_host(y, F32)
    print("istft full errors", assert_close(yh, ref, F32, "istft full", den=den))
    n = mbrt.istft_output_length(801, 441, True)
    assert n == 800 * 441 and np.all(yh[:, n:] == 0)
    if dt == F32:
        assert np.abs(yh[:, :n] - x[:, :n]).max() <= 1e-5 * np.abs(x).max()


def test_stft_istft_reject_bad_arguments(dev):
    w = torch.ones(2048, device="cuda")
    x = torch.zeros((1, 4096), device="cuda")
    with pytest.raises(mbrt.MbrtError):
        mbrt.stft(x, w, 441, n_fft=1024)
    with pytest.raises(mbrt.MbrtError):
        mbrt.stft(x, torch.ones(1024, device="cuda"), 441)
    with pytest.raises(mbrt.MbrtError):
        mbrt.stft(torch.zeros((1, 2000), device="cuda"), w, 441, center=False)   # shorter than n_fft
    with pytest.raises(mbrt.MbrtError):
        mbrt.stft(x, w, 0)
    spec = torch.zeros((1, 1025, 4, 2), device="cuda")
    with pytest.raises(mbrt.MbrtError):
        mbrt.istft(torch.zeros((1, 1024, 4, 2), device="cuda"), w, 441)
    with pytest.raises(mbrt.MbrtError):
        mbrt.istft(spec.half(), w, 441)
    with pytest.raises(mbrt.MbrtError):
        mbrt.istft(spec, w, 441, workspace=torch.empty(16, device="cuda"))
    with pytest.raises(mbrt.MbrtError):
        mbrt.istft(spec, w, 441, win_length=1024)
