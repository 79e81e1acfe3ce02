"""CPU checks of the C-ABI library: it loads, exports exactly what include/mbrt.h
declares, is valid C, and rejects bad arguments before touching the GPU."""
from __future__ import annotations

import ctypes as C
import re
import subprocess
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent
HEADER = REPO / "include" / "mbrt.h"
LIB = REPO / "mbr-cuda-tile_amd" / "lib" / "libmbrt.so"


def declared() -> set[str]:
    return set(re.findall(r"^MBRT_API\s+[\w\s\*]+?\b(mbrt_\w+)\s*\(", HEADER.read_text(), flags=re.M))


@pytest.fixture(scope="module")
def lib():
    if not LIB.exists():
        pytest.skip("libmbrt.so not built")
    import mbrt

    return mbrt.lib()


def test_exports_match_header(lib):
    names = declared()
    assert len(names) >= 28
    out = subprocess.run(["nm", "-D", "--defined-only", str(LIB)], capture_output=True, text=True, check=True).stdout
    exported = {l.split()[-1] for l in out.splitlines() if " T " in l}
    assert names <= exported, f"declared but not exported: {sorted(names - exported)}"
    assert {e for e in exported if e.startswith("mbrt_")} == names, "exported symbols not in the header"
    for n in names:
        assert hasattr(lib, n)


def test_binding_covers_header():
    from mbrt import _abi

    assert set(_abi.SIGNATURES) == declared()


def test_version(lib):
    assert lib.mbrt_version() == 10100


def test_header_is_c99(tmp_path):
    src = tmp_path / "use.c"
    src.write_text('#include "mbrt.h"\n#include <stdio.h>\n'
                   "int main(void) { mbrt_strided_meta m = {{0}, {0}, 0}; (void)m;\n"
                   "  printf(\"%d\\n\", mbrt_version()); return mbrt_last_error()[0] != 0; }\n")
    exe = tmp_path / "use"
    subprocess.run(["gcc", "-std=c99", "-Wall", "-Wextra", "-Werror", "-pedantic", f"-I{REPO / 'include'}",
                    str(src), "-o", str(exe), f"-L{LIB.parent}", "-lmbrt", f"-Wl,-rpath,{LIB.parent}"], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True)
    assert r.returncode == 0 and r.stdout.strip() == "10100"


def test_arith_flags_are_per_thread_and_validated(lib):
    import threading

    import mbrt

    seen = []
    with mbrt.arith_flags(mbrt.ARITH_BF16_INTERMEDIATES):
        t = threading.Thread(target=lambda: seen.append(mbrt.get_arith_flags()))
        t.start()
        t.join()
        assert mbrt.get_arith_flags() == mbrt.ARITH_BF16_INTERMEDIATES
    assert seen == [0] and mbrt.get_arith_flags() == 0
    assert lib.mbrt_set_arith_flags(0x80) == 1 and "unknown flags" in _err(lib)
    assert mbrt.get_arith_flags() == 0


def _err(lib) -> str:
    return lib.mbrt_last_error().decode()


def test_argument_errors_without_gpu(lib):
    from mbrt import _abi

    null = C.c_void_p(0)
    # unsupported dtype
    assert lib.mbrt_rms_norm(null, 2, null, 0, null, 0, 10, 384, 1.0, 1e-12, null) == 2
    assert "unsupported dtype" in _err(lib)
    assert lib.mbrt_softmax_rows(null, 0, null, 4, 1, 8, 1.0, null) == 2
    # bad shapes / arguments
    assert lib.mbrt_glu_last_dim(null, 0, null, 0, 4, 0, null) == 3
    assert lib.mbrt_rotary_inplace(null, null, 3, null, null, 0, 5, 5, 1, 7, 0, null) == 3
    assert "even" in _err(lib)
    assert lib.mbrt_strided_copy(null, null, 0, None, null) == 1
    assert lib.mbrt_band_mask_merge(null, None, 0, 3, null, null, 4, null, 0, null, 0, 1, 10, 10, 10, 2, null) == 1
    assert "stems" in _err(lib)
    assert lib.mbrt_band_mask_merge(null, None, 0, 1, null, null, 4, null, 0, null, 0, 1, 11, 10, 10, 2, null) == 3
    assert "channel" in _err(lib)
    assert lib.mbrt_arange(null, 3, 10, 0, null) == 2  # bf16 arange is rejected, as in the reference
    assert lib.mbrt_binary(null, null, null, 0, 100, 9, null) == 1
    m = _abi.StridedMeta()
    m.ndim = 9
    assert lib.mbrt_strided_copy(null, null, 0, C.byref(m), null) == 1
    # rms_norm with rows > 0 and NULL pointers
    assert lib.mbrt_rms_norm(null, 0, null, 0, null, 0, 10, 384, 1.0, 1e-12, null) == 1


def test_widened_entry_points_reject_bad_arguments_without_gpu(lib):
    """Attention, STFT / iSTFT and chunk entry points: each check fires before any launch.
    Non-NULL pointers are fake 16-byte-aligned addresses that are never dereferenced."""
    p = 0x10000   # aligned stand-in address
    bf16, f32, f16 = 3, 0, 1

    def strided(dtype=bf16, B=1, H=2, nq=8, nk=8, hd=64, q=(8 * 192, 64, 192), kv=(8 * 192, 64, 192),
                cos=None, sin=None, gate=None, out_dtype=f32):
        return lib.mbrt_attention_strided(p, p, p, dtype, B, H, nq, nk, hd, *q, *kv, cos, sin, f32, gate, bf16, 1,
                                          p, out_dtype, 0.0, None)

    assert strided(dtype=f32) == 2 and "BF16" in _err(lib)
    assert strided(out_dtype=f16) == 2
    assert strided(hd=32) == 3 and "head_dim" in _err(lib)
    assert strided(B=0) == 0 and strided(nq=0) == 0          # nothing to do
    assert strided(nk=0) == 3 and "zero keys" in _err(lib)
    assert strided(q=(8 * 192, 64, 68)) == 4 and "multiples of 8" in _err(lib)
    assert strided(kv=(8 * 192, 64, 32)) == 3 and "row stride" in _err(lib)
    assert strided(cos=p) == 1 and "cos and sin" in _err(lib)
    assert lib.mbrt_attention(p, p, p, bf16, p, f32, 4, 8, 8, 32, 0.0, None) == 3
    assert lib.mbrt_attention_ex(p, p, p, bf16, 1, 2, 8, 8, 64, 8 * 192, 64, 192, 8 * 192, 64, 192, None, None, f32,
                                 None, bf16, 1, p, f32, 0.0, 3, None) == 1 and "precision" in _err(lib)

    def stft(batch=1, length=4096, n_fft=2048, hop=441, win=2048, numel=2048, center=1, sig=p, out=p):
        return lib.mbrt_stft(sig, p, out, batch, length, n_fft, hop, win, numel, center, 0, None)

    assert stft(n_fft=1024, win=1024, numel=1024) == 3
    assert stft(hop=0) == 3
    assert stft(length=2000, center=0) == 3 and "shorter than n_fft" in _err(lib)
    assert stft(batch=0) == 0
    assert stft(sig=None) == 1
    assert stft(out=p + 4) == 4
    assert lib.mbrt_stft_num_frames(4096, 441, 1) == 4096 // 441 + 1
    assert lib.mbrt_stft_num_frames(4096, 441, 0) == (4096 - 2048) // 441 + 1

    def istft(dtype=f32, bins=1025, frames=10, hop=441, batch=1, ws=None, ws_bytes=None):
        need = lib.mbrt_istft_workspace_bytes(batch, frames, hop)
        return lib.mbrt_istft(p, dtype, p, p, batch, bins, frames, 2048, hop, 2048, 2048, 1, 0, -1,
                              p if ws is None else ws, need if ws_bytes is None else ws_bytes, None)

    assert istft(bins=1024) == 3 and "1025" in _err(lib)
    assert istft(dtype=f16) == 2
    assert istft(hop=0) == 3
    assert istft(batch=0) == 0
    assert istft(ws_bytes=16) == 1 and "workspace" in _err(lib)
    assert istft(ws=0) == 1

    assert lib.mbrt_chunk_accumulate(p, p, p, p, 2, 100, 150, 60, None) == 3   # chunk past the end
    assert lib.mbrt_chunk_accumulate(p, p, p, p, 0, 100, 150, 0, None) == 0
    assert lib.mbrt_chunk_accumulate(p, None, p, p, 2, 100, 150, 0, None) == 1
    assert lib.mbrt_chunk_normalize(None, p, 2, 100, None) == 1
    assert lib.mbrt_chunk_fade_window(None, 100, 51, 0, 0) == 3               # fades overlap
    assert lib.mbrt_hann_window(None, -1, None) == 3


def test_empty_sizes_are_noops(lib):
    null = C.c_void_p(0)
    assert lib.mbrt_fill(null, 0, 0, 1.0, null) == 0
    assert lib.mbrt_softmax_rows(null, 0, null, 0, 0, 801, 1.0, null) == 0
    assert lib.mbrt_rms_norm(null, 0, null, 0, null, 0, 0, 384, 1.0, 1e-12, null) == 0
    assert lib.mbrt_band_gather(null, null, 4, null, 0, 0, 2050, 801, 3958, null) == 0
    assert lib.mbrt_binary(null, null, null, 3, 0, 0, null) == 0


def test_host_tables_match_oracle(lib, orc):
    import numpy as np

    import mbrt

    fi, fpb = mbrt.mel_band_layout(44100.0, 2048, 60, 2)
    mb = orc.mel_bands(44100.0, 2048, 60, 2)
    assert np.array_equal(fi, mb["freq_indices"]) and np.array_equal(fpb, mb["freqs_per_band"])
    off, ind, cnt, mx = mbrt.band_csr(fi, 2050)
    assert np.array_equal(off, mb["csr_offsets"]) and np.array_equal(ind, mb["csr_indices"])
    assert np.array_equal(cnt, mb["bands_per_freq"].astype(np.float32)) and mx == 2
    for sr, nfft, nb, ch in [(44100.0, 2048, 60, 1), (48000.0, 2048, 64, 2), (44100.0, 4096, 128, 2)]:
        fi, fpb = mbrt.mel_band_layout(sr, nfft, nb, ch)
        mb = orc.mel_bands(sr, nfft, nb, ch)
        assert np.array_equal(fi, mb["freq_indices"]) and np.array_equal(fpb, mb["freqs_per_band"])
    c, s = mbrt.rotary_tables(801, 64)
    oc, os_ = orc.rotary_tables(801, 64)
    assert np.array_equal(c, oc) and np.array_equal(s, os_)
    with pytest.raises(mbrt.MbrtError):
        mbrt.band_csr(np.array([0, 5000], np.int32), 2050)


def test_chunk_fade_window_matches_oracle(lib, orc):
    import numpy as np

    import mbrt

    for n, f in ((524288, 52428), (4000, 400), (7, 1), (7, 0), (10, 5)):
        for first in (False, True):
            for last in (False, True):
                assert np.array_equal(mbrt.chunk_fade_window(n, f, first, last), orc.chunk_fade_window(n, f, first, last))
    null = C.c_void_p(0)
    assert lib.mbrt_chunk_fade_window(null, 10, 6, 0, 0) == 3   # fades overlap



def test_last_error_is_per_thread(lib):
    """Two threads making different bad calls each read back their own message (ctypes
    drops the GIL around foreign calls, so the calls interleave)."""
    import threading

    null = C.c_void_p(0)
    seen = {"glu": set(), "rotary": set()}

    def glu():
        for _ in range(3000):
            assert lib.mbrt_glu_last_dim(null, 0, null, 0, 4, 0, null) == 3
            seen["glu"].add(lib.mbrt_last_error().decode())

    def rotary():
        for _ in range(3000):
            assert lib.mbrt_rotary_inplace(null, null, 3, null, null, 0, 5, 5, 1, 7, 0, null) == 3
            seen["rotary"].add(lib.mbrt_last_error().decode())

    threads = [threading.Thread(target=glu), threading.Thread(target=rotary)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert len(seen["glu"]) == 1 and len(seen["rotary"]) == 1
    assert seen["glu"] != seen["rotary"] and all("even" in m for m in seen["rotary"])
