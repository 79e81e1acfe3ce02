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
    assert lib.mbrt_version() == 10000


def test_header_is_c99(tmp_path):
    src = tmp_path / "use.c"
    src.write_text('#include "mbrt.h"\n#include <stdio.h>\n'
                   "int main(void) { mbrt_strided_meta m = {{0}, {0}, 0}; (void)m;\n"
                   "  printf(\"%d\\n\", mbrt_version()); return mbrt_last_error()[0] != 0; }\n")
    exe = tmp_path / "use"
    subprocess.run(["gcc", "-std=c99", "-Wall", "-Wextra", "-Werror", "-pedantic", f"-I{REPO / 'include'}",
                    str(src), "-o", str(exe), f"-L{LIB.parent}", "-lmbrt", f"-Wl,-rpath,{LIB.parent}"], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True)
    assert r.returncode == 0 and r.stdout.strip() == "10000"


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

