"""GPU parity of the chunk overlap-add entry points (mbrt_chunk_accumulate,
mbrt_chunk_normalize) against the oracle's f32 restatement of src/chunk_cuda_tile.cu.
The kernels round the product and the sum separately and run each call's writes once, so
a sequence of calls equals the ordered f32 evaluation bit for bit."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import mbrt
from gpu_util import say, to_dev, to_host
from parity import F32, assert_bitexact

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("C,L,calls", [
    (2, 18000, [(0, 4000), (3000, 4000), (6000, 4000), (9000, 4000), (12000, 4000), (15000, 3000)]),  # float4 path
    (3, 18601, [(0, 4000), (3200, 4000), (6400, 4000), (9600, 4000), (12800, 4000), (16000, 2601)]),  # scalar path
    (8, 1058400, [(0, 352800), (264600, 352800), (529200, 352800), (705600, 352800)]),  # 8 channels, 8 s chunks
    (1, 7, [(0, 3), (2, 5), (6, 1)]),
    (12, 8000, [(0, 4000), (2000, 4000), (4000, 4000)]),  # float4, 4 channels per thread, 3 groups
    (5, 8000, [(0, 4000), (4000, 4000)]),  # float4, 1 channel per thread, 5 groups
])
def test_chunk_accumulate_and_normalize_bitexact(orc, dev, C, L, calls):
    say(f"chunk accumulate C={C} L={L} calls={len(calls)}")
    rng = np.random.default_rng(C * 1000 + L)
    dest = torch.zeros((C, L), device="cuda")
    ws = torch.zeros(L, device="cuda")
    dref = np.zeros((C, L), np.float32)
    wref = np.zeros(L, np.float32)
    for k, (off, n) in enumerate(calls):
        src = rng.standard_normal((C, n)).astype(np.float32)
        win = orc.chunk_fade_window(n, n // 10, first=(k == 0), last=(k == len(calls) - 1))
        mbrt.chunk_accumulate(dest, ws, to_dev(src, F32), to_dev(win, F32), off)
        orc.chunk_accumulate(dref, wref, src, win, off)
    torch.cuda.synchronize()
    assert_bitexact(to_host(dest, F32), dref, "accumulate")
    assert_bitexact(to_host(ws, F32), wref, "weight sum")
    mbrt.chunk_normalize(dest, ws)
    torch.cuda.synchronize()
    orc.chunk_normalize(dref, wref)
    assert_bitexact(to_host(dest, F32), dref, "normalize")


def test_chunk_unaligned_views(orc, dev):
    """Offsets views into larger buffers: the scalar path handles any alignment."""
    say("chunk accumulate unaligned views")
    rng = np.random.default_rng(5)
    big = torch.zeros(2 * 1001 + 1, device="cuda")
    dest = big[1:].view(2, 1001)
    wbig = torch.zeros(1002, device="cuda")
    ws = wbig[1:]
    src = rng.standard_normal((2, 500)).astype(np.float32)
    win = rng.random(500).astype(np.float32)
    mbrt.chunk_accumulate(dest, ws, to_dev(src, F32), to_dev(win, F32), 301)
    torch.cuda.synchronize()
    dref = np.zeros((2, 1001), np.float32)
    wref = np.zeros(1001, np.float32)
    orc.chunk_accumulate(dref, wref, src, win, 301)
    assert_bitexact(to_host(dest, F32), dref, "unaligned accumulate")
    assert_bitexact(to_host(ws, F32), wref, "unaligned weight sum")
    assert float(big[0]) == 0.0 and float(wbig[0]) == 0.0


def test_chunk_rejects_bad_arguments(dev):
    dest = torch.zeros((2, 100), device="cuda")
    ws = torch.zeros(100, device="cuda")
    src = torch.zeros((2, 50), device="cuda")
    win = torch.ones(50, device="cuda")
    with pytest.raises(mbrt.MbrtError):
        mbrt.chunk_accumulate(dest, ws, src, win, 60)   # past the end
    with pytest.raises(mbrt.MbrtError):
        mbrt.chunk_accumulate(dest, ws, src, win, -1)
