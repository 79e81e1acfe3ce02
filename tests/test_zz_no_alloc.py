"""The allocation-free iSTFT (mbrt_istft_noalloc) against mbrt_istft with a caller
workspace: the same kernels, so the outputs must agree bit for bit.  Two calls in a row,
the second smaller, show that the shared scratch array keeps nothing from the previous
call that the next one reads; a call beyond the scratch size fails before any launch.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import mbrt
from gpu_util import say, to_host
from parity import F32, assert_bitexact

pytestmark = pytest.mark.gpu


def _pair(B, T, hop, dtype, center, length, seed):
    say(f"istft_noalloc B={B} T={T} hop={hop} dtype={dtype} center={center} length={length}")
    g = torch.Generator(device="cuda").manual_seed(seed)
    spec = torch.randn((B, 1025, T, 2), generator=g, device="cuda").to(dtype)
    win = mbrt.hann_window(2048)
    ref = mbrt.istft(spec, win, hop, center=center, length=length)
    out = torch.full_like(ref, float("nan"))
    mbrt.istft_noalloc(spec, win, hop, out, center=center, length=length)
    torch.cuda.synchronize()
    assert_bitexact(to_host(out, F32), to_host(ref, F32), "istft_noalloc = istft")
    return out


def test_istft_noalloc_matches_istft(dev):
    # the chunk shape (8 signals, 801 frames at hop 441: 16.6 MB of block partials), then a
    # smaller call whose partials cover only the start of the scratch array
    _pair(8, 801, 441, torch.float32, True, 352800, 0x4D425200C0)
    _pair(2, 37, 300, torch.bfloat16, False, -1, 0x4D425200C1)
    # and the chunk shape again after the small call
    _pair(8, 801, 441, torch.bfloat16, True, -1, 0x4D425200C2)


def test_istft_noalloc_rejects_calls_beyond_the_scratch(dev):
    say("istft_noalloc beyond the scratch size")
    B, T, hop = 17, 801, 441
    assert mbrt.istft_workspace_bytes(B, T, hop) > mbrt.ISTFT_SCRATCH_BYTES
    spec = torch.zeros((B, 1025, T, 2), device="cuda")
    out = torch.zeros((B, mbrt.istft_output_length(T, hop, True, -1)), device="cuda")
    with pytest.raises(mbrt.MbrtError) as e:
        mbrt.istft_noalloc(spec, mbrt.hann_window(2048), hop, out)
    assert "scratch" in str(e.value)
    torch.cuda.synchronize()
    assert float(out.abs().max()) == 0.0  # nothing ran


def test_istft_noalloc_under_graph_capture(dev):
    # The first call on a GPU resolves the scratch array's device address (a runtime call
    # that is not a stream operation), so it is made outside the capture.  After that a
    # call allocates nothing and issues only kernel launches, and a captured call replays
    # with whatever the spectrum holds at replay time.  Each replay follows eager work
    # (new spectrum data, the workspace form into another buffer) and is checked bit for
    # bit against it.
    B, T, hop = 2, 64, 441
    say(f"istft_noalloc under graph capture B={B} T={T} hop={hop}")
    g = torch.Generator(device="cuda").manual_seed(0x4D425200C3)
    spec = torch.randn((B, 1025, T, 2), generator=g, device="cuda")
    win = mbrt.hann_window(2048)
    out = torch.empty((B, mbrt.istft_output_length(T, hop, True, -1)), device="cuda")
    mbrt.istft_noalloc(spec, win, hop, out)  # warm-up on this GPU, outside the capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        mbrt.istft_noalloc(spec, win, hop, out)
    torch.cuda.synchronize()
    for rep in range(3):
        spec.copy_(torch.randn((B, 1025, T, 2), generator=g, device="cuda"))
        ref = mbrt.istft(spec, win, hop)
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert_bitexact(to_host(out, F32), to_host(ref, F32), f"graph replay {rep} = istft")
