"""The .csm model-file format (src/weights.h:82-96) on the host: the Python writer and
reader round-trip, the byte layout matches the reference's specification field by field,
and the __precomputed__ band tensors agree with the oracle's band layout and the
reference's recorded band widths."""
from __future__ import annotations

import json
import struct
from pathlib import Path

import numpy as np
import pytest

from mbrt import csm

GOLDEN = Path(__file__).resolve().parent / "golden"


def test_byte_layout_of_a_small_file(tmp_path):
    p = tmp_path / "a.csm"
    csm.write_csm(p, {"k": 1}, [("w", np.array([[1.5, -2.0]], np.float32)), ("i", np.array([7], np.int64))])
    b = p.read_bytes()
    cfg = b'{"k": 1}'
    want = (b"CSM\x00" + struct.pack("<II", 1, len(cfg)) + cfg + struct.pack("<I", 2)
            + struct.pack("<I", 1) + b"w" + struct.pack("<I", 2) + struct.pack("<qq", 1, 2) + struct.pack("<I", 0)
            + struct.pack("<ff", 1.5, -2.0)
            + struct.pack("<I", 1) + b"i" + struct.pack("<I", 1) + struct.pack("<q", 1) + struct.pack("<I", 2)
            + struct.pack("<q", 7))
    assert b == want


def test_round_trip_all_dtypes(tmp_path):
    rng = np.random.default_rng(0)
    bf = (rng.integers(0, 2**16, size=(3, 4))).astype(np.uint16)
    items = [("f32", rng.standard_normal((2, 3)).astype(np.float32)), ("f16", rng.standard_normal(5).astype(np.float16)),
             ("i64", np.arange(-3, 3, dtype=np.int64)), ("bf16", bf), ("scalar", np.array(2.5, np.float32)),
             ("empty", np.zeros((0, 4), np.float32)), ("naïve.weight", np.ones(2, np.float32))]
    cfg = {"num_bands": 60, "nested": {"a": [1, 2.5, None, True, "s\"q\\u00e9"]}}
    p = tmp_path / "m.csm"
    csm.write_csm(p, cfg, items, dtypes={"bf16": csm.BF16})
    c2, t2 = csm.read_csm(p)
    assert c2 == cfg
    assert list(t2) == [n for n, _ in items]
    for n, a in items:
        code, b = t2[n]
        assert b.shape == a.shape and b.dtype == a.dtype and np.array_equal(a, b), n
    assert t2["bf16"][0] == csm.BF16 and t2["i64"][0] == csm.I64 and t2["f16"][0] == csm.F16


def test_reader_rejects_malformed_files(tmp_path):
    good = tmp_path / "g.csm"
    csm.write_csm(good, {}, {"w": np.ones(4, np.float32)})
    b = good.read_bytes()
    for name, data in (("magic", b"CSX\x00" + b[4:]), ("version", b[:4] + struct.pack("<I", 2) + b[8:]),
                       ("trunc", b[:-3])):
        q = tmp_path / f"{name}.csm"
        q.write_bytes(data)
        with pytest.raises(ValueError):
            csm.read_csm(q)


def test_precomputed_band_tensors_match_oracle_and_golden(orc):
    t = csm.precomputed_band_tensors(44100.0, 2048, 60, True)
    mb = orc.mel_bands(44100.0, 2048, 60, 2)
    assert np.array_equal(t["__precomputed__.freq_indices"], mb["freq_indices"].astype(np.int64))
    assert np.array_equal(t["__precomputed__.num_freqs_per_band"], mb["freqs_per_band"].astype(np.int64))
    assert np.array_equal(np.repeat(t["__precomputed__.num_bands_per_freq"], 2), mb["bands_per_freq"].astype(np.int64))
    gold = json.loads((GOLDEN / "mel_band_widths.json").read_text())
    widths = t["__precomputed__.num_freqs_per_band"]
    assert 2 * 2 * int(widths.sum()) == gold["mask_stride"]   # 2 channels x (re, im) per band bin
    # recorded as [mask-estimator width 4 x bins (stereo x complex), calls per chunk = stems x bands]
    stems = gold["config"]["stems"]
    hist = [[4 * int(w), stems * int(n)] for w, n in zip(*np.unique(widths, return_counts=True))]
    assert hist == gold["width_counts"]
