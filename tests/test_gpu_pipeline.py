"""The MelBandRoformer forward skeleton without its transformer, end to end on the GPU
(src/model_mel_band_roformer.cu:699-830): STFT of every channel, the stereo interleave
'b s f t c -> b (f s) t c', the band gather, the mask merge, the iSTFT, and the chunk
overlap-add around it (src/inference_app.cpp:72-232).  With unit masks (1 + 0j) the merge
returns the spectrum itself (overlapping bands are divided by their count), so the chain
reconstructs the audio."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import mbrt
from gpu_util import say, to_host
from parity import F32

pytestmark = pytest.mark.gpu


def _bands(dev):
    fi, _ = mbrt.mel_band_layout(44100.0, 2048, 60, 2)
    off, ind, cnt, _ = mbrt.band_csr(fi, 2050)
    t = lambda a: torch.from_numpy(a).to(dev)
    return t(fi), t(off), t(ind), t(cnt)


def _skeleton(x, w, bands, hop=441):
    """x [B, C, L] f32 -> reconstructed [B, C, L] through every tensor op of the forward."""
    B, C, L = x.shape
    fi, off, ind, cnt = bands
    J = fi.numel()
    spec = mbrt.stft(x.reshape(B * C, L), w, hop)                      # [B*C, 1025, T, 2]
    T = spec.shape[2]
    fs = torch.empty((B, 1025, C, T, 2), device=x.device)
    mbrt.strided_copy(spec.view(B, C, 1025, T, 2).permute(0, 2, 1, 3, 4), fs)
    fs = fs.view(B, 1025 * C, T, 2)                                     # freq 2 bin + ch
    bands_t = torch.empty((B, T, J * 2), device=x.device)
    mbrt.band_gather(fs, fi, bands_t)
    mask = torch.zeros_like(bands_t)
    mask[..., 0::2] = 1.0                                               # 1 + 0j per band-bin
    merged = torch.empty((B * C, 1025, T, 2), device=x.device)
    mbrt.band_mask_merge(fs, [mask], off, ind, cnt, merged, C)
    y = mbrt.istft(merged, w, hop, length=L).view(B, C, L)
    return spec, merged, y


def test_forward_skeleton_reconstructs_audio(dev):
    say("pipeline stft -> interleave -> gather -> merge(1) -> istft, [2, 2, 88200]")
    g = torch.Generator(device="cuda").manual_seed(7)
    x = torch.randn((2, 2, 88200), generator=g, device="cuda")
    w = mbrt.hann_window(2048)
    spec, merged, y = _skeleton(x, w, _bands("cuda"))
    torch.cuda.synchronize()
    # unit masks: every complex product is exact and a count of equal terms divided by the
    # count is exact, so the merge gives the STFT back exactly (as values: s * 1 + (-0) * 0
    # turns a -0 imaginary part into +0)
    assert np.array_equal(to_host(merged, F32), to_host(spec, F32)), "merge with unit masks"
    n = mbrt.istft_output_length(spec.shape[2], 441, True)
    xh, yh = to_host(x, F32), to_host(y, F32)
    assert np.abs(yh[..., :n] - xh[..., :n]).max() <= 2e-6 * np.abs(xh).max()
    assert np.all(yh[..., n:] == 0)


def test_chunked_skeleton_reconstructs_a_song(orc, dev):
    """Chunks of 2 s with 25 % overlap, each through the skeleton, overlap-added with fade
    windows (chunk_fade_window / chunk_accumulate / chunk_normalize, the reference's loop)."""
    say("pipeline chunked: 7 s stereo, chunk 88200, step 66150")
    g = torch.Generator(device="cuda").manual_seed(8)
    L, chunk, step = 308700, 88200, 66150
    audio = torch.randn((1, 2, L), generator=g, device="cuda")
    w = mbrt.hann_window(2048)
    bands = _bands("cuda")
    border = chunk - step
    mix = torch.empty((1, 2, L + 2 * border), device="cuda")
    mbrt.pad(audio, mix, [0, 0, border], reflect=True)
    total = mix.shape[-1]
    out = torch.zeros((2, total), device="cuda")
    wsum = torch.zeros(total, device="cuda")
    starts = list(range(0, total, step))
    fade = chunk // 10
    for k, s in enumerate(starts):
        e = min(s + chunk, total)
        n = e - s
        piece = mix[..., s:e]
        if n < chunk:
            padded = torch.empty((1, 2, chunk), device="cuda")
            mbrt.pad(piece.contiguous(), padded, [0, 0, 0], reflect=n > chunk // 2)  # reflect or zeros
            piece = padded
        _, _, y = _skeleton(piece.contiguous(), w, bands)
        win = torch.from_numpy(mbrt.chunk_fade_window(chunk, fade, s == 0, e >= total)).to("cuda")
        mbrt.chunk_accumulate(out, wsum, y[..., :n].reshape(2, n).contiguous(), win[:n].contiguous(), s)
    mbrt.chunk_normalize(out, wsum)
    torch.cuda.synchronize()
    rec = to_host(out, F32)[:, border:border + L]
    a = to_host(audio, F32)[0]
    assert np.abs(rec - a).max() <= 4e-6 * np.abs(a).max()


def test_side_stream_matches_default_stream(orc, dev):
    """Every call launches on the caller's current stream: the same ops on a second
    (default-priority) stream give the same bits as on the default stream."""
    say("softmax / attention / stft / istft / band chain on a side stream")
    x = torch.from_numpy(orc.randn((300, 801), seed=0x4D425200A7, std=3.0)).to(dev)
    q, k, v = (torch.from_numpy(orc.randn((8, 801, 64), seed=0x4D425200A8, stream=i)).to(dev).to(torch.bfloat16)
               for i in range(3))
    sig = torch.from_numpy(orc.randn((2, 2, 20000), seed=0x4D425200A9)).to(dev)
    w = mbrt.hann_window(2048)
    bands = _bands(dev)

    def run():
        y = torch.empty_like(x)
        mbrt.softmax(x, y, 1.0)
        o = torch.empty((8, 801, 64), dtype=torch.bfloat16, device=dev)
        mbrt.attention(q, k, v, o, 0.0)
        spec = mbrt.stft(sig.view(4, 20000), w, 441, True, False)
        back = mbrt.istft(spec, w, 441, True, False, 20000)
        return (y, o, spec, back, *_skeleton(sig, w, bands))

    ref = run()
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        got = run()
    side.synchronize()
    names = ("softmax", "attention", "stft", "istft", "chain stft", "chain merge", "chain istft")
    assert len(ref) == len(names)
    for name, a, b in zip(names, ref, got):
        assert torch.equal(a, b), f"{name} differs on a side stream"
