"""Host <-> device helpers for the GPU tests (torch supplies memory only)."""
from __future__ import annotations

import sys

import numpy as np
import torch

from parity import BF16, F16, F32, I32, I64

TORCH_DT = {F32: torch.float32, F16: torch.float16, BF16: torch.bfloat16, I32: torch.int32, I64: torch.int64}


def to_dev(a: np.ndarray, dt: int) -> torch.Tensor:
    a = np.ascontiguousarray(a)
    if dt in (BF16, F16):
        t = torch.from_numpy(a.view(np.int16)).view(TORCH_DT[dt])
    else:
        t = torch.from_numpy(a)
    return t.to("cuda")


def to_host(t: torch.Tensor, dt: int) -> np.ndarray:
    t = t.detach().contiguous().cpu()
    if dt in (BF16, F16):
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def empty(shape, dt: int) -> torch.Tensor:
    return torch.empty(shape, dtype=TORCH_DT[dt], device="cuda")


def say(msg: str) -> None:
    """Name the GPU case before running it (flushed, so it survives a crash)."""
    print(f"[gpu-case] {msg}", file=sys.stderr, flush=True)
