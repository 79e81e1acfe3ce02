"""Regenerates mel_band_widths.json from the reference's mask-GLU benchmark.

bench/bf16_mask_final_glu_cutile.cu runs the mask-estimator output layer once per
(stem, band) of its two-stem, 60-band stereo model: `run_model_width<NOut, Count>` lists
each distinct per-band output width NOut = 2 (re/im) * 2 (channels) * freqs_in_band with
Count = calls per chunk, and kMaskStride is the width of the full mask row.  Those
numbers are the reference's own record of the mel band layout at sr 44100, n_fft 2048,
60 bands.  Run in the container that has the reference mounted:
    python tests/golden/extract_mel_widths.py /root/reference
"""
import json
import re
import sys
from pathlib import Path

src = Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference") / "bench" / "bf16_mask_final_glu_cutile.cu"
text = src.read_text()
stride = int(re.search(r"constexpr int kMaskStride = (\d+);", text).group(1))
pairs = [(int(a), int(b)) for a, b in re.findall(r"run_model_width<(\d+), (\d+)>\(opts", text)]
lines = [i + 1 for i, l in enumerate(text.splitlines()) if "run_model_width<" in l and "(opts" in l]
out = {
    "source": f"bench/bf16_mask_final_glu_cutile.cu:{text[:text.index('kMaskStride =')].count(chr(10)) + 1} "
              f"(kMaskStride), :{lines[0]}-{lines[-1]} (run_model_width<NOut, Count>)",
    "meaning": "per-band mask-estimator output width NOut = 4 * freqs_per_band (complex x stereo); "
               "Count = calls per chunk = 2 stems x bands of that width",
    "config": {"sr": 44100, "n_fft": 2048, "n_bands": 60, "channels": 2, "stems": 2},
    "mask_stride": stride,
    "width_counts": [[w, c] for w, c in pairs],
}
dst = Path(__file__).with_name("mel_band_widths.json")
dst.write_text(json.dumps(out, indent=1) + "\n")
print(dst, len(pairs), "widths")
