""".csm model files (the reference's weight format, src/weights.h:82-96) on the host.

write_csm / read_csm move a config dict and named numpy arrays to and from the file:
  "CSM\\0" | u32 version 1 | u32 config_len | config JSON | u32 n_tensors |
  per tensor: u32 name_len | name (UTF-8) | u32 ndim | i64 shape[ndim] | u32 dtype | data
with dtype 0 f32, 1 f16, 2 i64, 3 bf16 (bf16 arrays are carried as uint16 bit patterns).
Nothing in a file is executed: the config is JSON and the tensors are raw bytes.

precomputed_band_tensors builds the __precomputed__.* tensors a MelBandRoformer file
carries (freq_indices, num_freqs_per_band, num_bands_per_freq; int64) from the library's
mel band layout.
"""
from __future__ import annotations

import json
import struct
from pathlib import Path

import numpy as np

F32, F16, I64, BF16 = 0, 1, 2, 3
_NP = {F32: np.float32, F16: np.float16, I64: np.int64, BF16: np.uint16}
_MAGIC = b"CSM\x00"


def _code(arr: np.ndarray, dtype: int | None) -> int:
    if dtype is not None:
        return dtype
    for code, t in ((F32, np.float32), (F16, np.float16), (I64, np.int64)):
        if arr.dtype == t:
            return code
    raise ValueError(f"csm: no dtype code for {arr.dtype} (pass dtype=BF16 for uint16 bf16 bits)")


def write_csm(path, config: dict, tensors, dtypes: dict | None = None) -> None:
    """tensors: mapping or (name, array) pairs, written in that order; dtypes: name -> code."""
    dtypes = dtypes or {}
    items = list(tensors.items()) if isinstance(tensors, dict) else list(tensors)
    cfg = json.dumps(config).encode("utf-8")
    with open(path, "wb") as f:
        f.write(_MAGIC)
        f.write(struct.pack("<II", 1, len(cfg)))
        f.write(cfg)
        f.write(struct.pack("<I", len(items)))
        for name, arr in items:
            arr = np.asarray(arr)
            code = _code(arr, dtypes.get(name))
            data = np.array(arr, dtype=_NP[code], order="C")  # keeps 0-d arrays 0-d
            nb = name.encode("utf-8")
            f.write(struct.pack("<I", len(nb)))
            f.write(nb)
            f.write(struct.pack("<I", data.ndim))
            f.write(struct.pack(f"<{data.ndim}q", *data.shape))
            f.write(struct.pack("<I", code))
            f.write(data.astype(data.dtype.newbyteorder("<"), copy=False).tobytes())


def read_csm(path):
    """(config dict, {name: (dtype code, array)}), the file read in full on the host."""
    buf = Path(path).read_bytes()
    p = 0

    def take(n):
        nonlocal p
        if p + n > len(buf):
            raise ValueError("csm: unexpected end of file")
        b = buf[p:p + n]
        p += n
        return b

    if take(4) != _MAGIC:
        raise ValueError("csm: invalid magic")
    version, clen = struct.unpack("<II", take(8))
    if version != 1:
        raise ValueError(f"csm: unsupported version {version}")
    config = json.loads(take(clen).decode("utf-8"))
    (n,) = struct.unpack("<I", take(4))
    out = {}
    for _ in range(n):
        (ln,) = struct.unpack("<I", take(4))
        name = take(ln).decode("utf-8")
        (nd,) = struct.unpack("<I", take(4))
        shape = struct.unpack(f"<{nd}q", take(8 * nd))
        (code,) = struct.unpack("<I", take(4))
        if code not in _NP:
            raise ValueError(f"csm: unknown dtype {code} for tensor {name}")
        dt = np.dtype(_NP[code]).newbyteorder("<")
        count = int(np.prod(shape, dtype=np.int64)) if nd else 1
        arr = np.frombuffer(take(count * dt.itemsize), dtype=dt).reshape(shape).astype(_NP[code])
        out[name] = (code, arr)
    return config, out


def precomputed_band_tensors(sample_rate: float = 44100.0, n_fft: int = 2048, num_bands: int = 60,
                             stereo: bool = True) -> dict:
    """The three __precomputed__ int64 tensors of a MelBandRoformer file."""
    from . import mel_band_layout

    channels = 2 if stereo else 1
    fi, fpb = mel_band_layout(sample_rate, n_fft, num_bands, channels)
    bins = n_fft // 2 + 1
    per_bin = np.bincount(fi[fi % channels == 0] // channels, minlength=bins).astype(np.int64)
    return {
        "__precomputed__.freq_indices": fi.astype(np.int64),
        "__precomputed__.num_freqs_per_band": fpb.astype(np.int64),
        "__precomputed__.num_bands_per_freq": per_bin,
    }
