"""Build the gfx950 libraries in-tree with hipcc (no cmake/ninja needed).

Outputs (git-ignored, shipped with the source tree):
  mbr-cuda-tile_amd/lib/libmbrt.so        C-ABI + HIP kernels (include/mbrt.h)
  mbr-cuda-tile_amd/lib/libmbrt_tensor.so C++ Tensor / tensor_tile:: / mbr_tile:: layer

Usage: python mbr-cuda-tile_amd/build.py [-j N] [-v] [-D NAME=VALUE ...] [--out DIR]

-D passes a preprocessor definition to every HIP translation unit (the kernels' launch
shapes can be overridden this way); --out puts objects and libraries under DIR instead of
the package tree, so that such variants never replace the in-tree build.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shlex
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
REPO = PKG.parent
CSRC = PKG / "csrc"
HOST = PKG / "host"
BUILD = PKG / "_build"
LIB = PKG / "lib"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

# Packed-FP32 VALU forms are disabled for every HIP translation unit.
COMMON = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-fvisibility=hidden",
    "-std=c++17",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-command-line-argument",
    f"-I{REPO / 'include'}",
    f"-I{CSRC}",
    f"-I{HOST}",
]

KERNEL_SOURCES = [
    "abi_common.cpp",
    "k_elementwise.hip",
    "k_layout.hip",
    "k_reduce.hip",
    "k_norm.hip",
    "k_act.hip",
    "k_softmax.hip",
    "k_rotary.hip",
    "k_band.hip",
    "k_attention.hip",
    "k_stft.hip",
    "k_chunk.hip",
    "host_tables.cpp",
]

# Per-file compiler options.  The attention kernel keeps its MFMA accumulators in ordinary
# VGPRs (gfx950 MFMA reads and writes them directly), so the online softmax and the
# accumulator rescale need no AGPR <-> VGPR copies.  Its device code is also built without
# NaN-preserving float semantics: the score max then needs no quieting v_max per MFMA
# result (a NaN score still reaches the output through exp2 and the P V product).
EXTRA_FLAGS = {
    "k_attention.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form", "-Xarch_device", "-fno-honor-nans"],
}

TENSOR_SOURCES = [
    "hip_context.cpp",
    "memory_pool.cpp",
    "tensor.cpp",
    "tensor_tile.cpp",
    "mbr_tile.cpp",
    "stft_tile.cpp",
    "chunk_tile.cpp",
    "weights.cpp",
]


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(shlex.quote(c) for c in cmd), flush=True)
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(
        line for line in res.stdout.splitlines()
        if "packed-fp32-ops" not in line and "feature flag" not in line
    )
    if res.returncode != 0:
        raise RuntimeError(f"command failed ({res.returncode}): {' '.join(cmd)}\n{out}")
    if verbose and out.strip():
        print(out)


def _compile(src: Path, obj: Path, defines: list[str], verbose: bool, extra: list[str] | None = None) -> Path:
    lang = ["-x", "hip"] if src.suffix in (".hip", ".cpp") else []
    _run([HIPCC, *COMMON, *(extra or []), *[f"-D{d}" for d in defines], *lang, "-c", str(src), "-o", str(obj)],
         verbose)
    return obj


def _objects(srcdir: Path, names: list[str], tag: str, build_dir: Path, defines: list[str], jobs: int,
             verbose: bool) -> list[Path]:
    build_dir.mkdir(parents=True, exist_ok=True)
    objs = []
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        futs = []
        for n in names:
            src = srcdir / n
            obj = build_dir / f"{tag}_{Path(n).stem}.o"
            # the C-ABI library exports only its MBRT_API symbols; the C++ tensor layer
            # exports its whole API
            extra = ["-fvisibility=default"] if tag == "t" else EXTRA_FLAGS.get(n)
            futs.append(ex.submit(_compile, src, obj, defines, verbose, extra))
        for f in futs:
            objs.append(f.result())
    return objs


def build(jobs: int | None = None, verbose: bool = False, defines: list[str] | None = None,
          out_dir: Path | str | None = None) -> dict[str, Path]:
    """Compile every source and link both libraries; returns their paths."""
    jobs = jobs or min(8, os.cpu_count() or 4)
    defines = list(defines or [])
    lib_dir = Path(out_dir) if out_dir else LIB
    build_dir = lib_dir / "_build" if out_dir else BUILD
    lib_dir.mkdir(parents=True, exist_ok=True)
    kobjs = _objects(CSRC, KERNEL_SOURCES, "k", build_dir, defines, jobs, verbose)
    libmbrt = lib_dir / "libmbrt.so"
    tmp = libmbrt.with_suffix(".so.tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, kobjs)], verbose)
    os.replace(tmp, libmbrt)
    out = {"libmbrt": libmbrt}
    tsrc = [n for n in TENSOR_SOURCES if (HOST / n).exists()]
    if tsrc:
        tobjs = _objects(HOST, tsrc, "t", build_dir, defines, jobs, verbose)
        libt = lib_dir / "libmbrt_tensor.so"
        tmp = libt.with_suffix(".so.tmp")
        _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, tobjs),
              f"-L{lib_dir}", "-lmbrt", "-Wl,-rpath,$ORIGIN"], verbose)
        os.replace(tmp, libt)
        out["libmbrt_tensor"] = libt
    return out


def build_selftest(verbose: bool = False, out_dir: Path | str | None = None) -> Path:
    """Link tests/cpp/tensor_selftest.cpp against the libraries (test infrastructure: the
    C++ layer's self-test, run by tests/test_cpp_layer.py on a GPU)."""
    lib_dir = Path(out_dir) if out_dir else LIB
    exe = lib_dir / "tensor_selftest"
    src = REPO / "tests" / "cpp" / "tensor_selftest.cpp"
    tmp = exe.with_suffix(".tmp")
    _run([HIPCC, *COMMON, "-x", "hip", str(src), "-o", str(tmp), f"-L{lib_dir}", "-lmbrt_tensor", "-lmbrt",
          "-Wl,-rpath,$ORIGIN"], verbose)
    os.replace(tmp, exe)
    return exe


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("-j", type=int, default=None)
    ap.add_argument("-v", action="store_true")
    ap.add_argument("-D", dest="defines", action="append", default=[], metavar="NAME=VALUE")
    ap.add_argument("--out", default=None, help="output directory (default: the package's lib/)")
    ap.add_argument("--selftest", action="store_true", help="also link the C++ layer's self-test binary")
    a = ap.parse_args(argv)
    paths = build(a.j, a.v, a.defines, a.out)
    if a.selftest and "libmbrt_tensor" in paths:
        paths["tensor_selftest"] = build_selftest(a.v, a.out)
    for k, p in paths.items():
        print(f"{k}: {p}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
