"""Tests of the C++ tensor layer (cudasep::Tensor, tensor_tile::, mbr_tile::) that callers
of the reference's C++ API link against (mbr-cuda-tile_amd/lib/libmbrt_tensor.so).

CPU: the library exports the reference's C++ API.  GPU: tensor_selftest checks Tensor
semantics against host expectations, then runs the mbr_tile ops on inputs written here
and their outputs are compared with the oracle."""
from __future__ import annotations

import os
import subprocess
from pathlib import Path

import numpy as np
import pytest

from parity import BF16, F32, I64, assert_bitexact, assert_close, merge_den

REPO = Path(__file__).resolve().parent.parent
LIB = REPO / "mbr-cuda-tile_amd" / "lib"
SELFTEST = LIB / "tensor_selftest"
TENSOR_LIB = LIB / "libmbrt_tensor.so"

# Reference C++ entry points (src/tensor.h, src/tensor_cuda_tile.h, src/mbr_cuda_tile.h)
# the layer must define.
API = [
    "cudasep::Tensor::empty(", "cudasep::Tensor::zeros(", "cudasep::Tensor::ones(", "cudasep::Tensor::full(",
    "cudasep::Tensor::arange(", "cudasep::Tensor::from_cpu_f32(", "cudasep::Tensor::from_cpu_f16(",
    "cudasep::Tensor::from_cpu_i64(", "cudasep::Tensor::reshape(", "cudasep::Tensor::permute(",
    "cudasep::Tensor::transpose(", "cudasep::Tensor::contiguous() const", "cudasep::Tensor::unsqueeze(",
    "cudasep::Tensor::squeeze(", "cudasep::Tensor::expand(", "cudasep::Tensor::slice(",
    "cudasep::Tensor::index_select(", "cudasep::Tensor::cat(", "cudasep::Tensor::stack(", "cudasep::Tensor::split(",
    "cudasep::Tensor::unbind(", "cudasep::Tensor::pad(", "cudasep::Tensor::pad_reflect(", "cudasep::Tensor::to_dtype(",
    "cudasep::Tensor::operator+(", "cudasep::Tensor::operator-(", "cudasep::Tensor::operator*(",
    "cudasep::Tensor::operator/(", "cudasep::Tensor::add_(", "cudasep::Tensor::mul_(", "cudasep::Tensor::add_scalar_(",
    "cudasep::Tensor::mul_scalar_(", "cudasep::Tensor::clamp_(", "cudasep::Tensor::fill_(", "cudasep::Tensor::sum(",
    "cudasep::Tensor::mean(", "cudasep::Tensor::max(", "cudasep::Tensor::operator>(", "cudasep::Tensor::clone() const",
    "cudasep::Tensor::copy_from(", "cudasep::Tensor::to_cpu_f32() const", "cudasep::Tensor::copy_from_cpu(",
    "cudasep::Tensor::copy_to_cpu(", "cudasep::Tensor::is_contiguous() const", "cudasep::Tensor::print(",
    "cudasep::tensor_tile::fill(", "cudasep::tensor_tile::arange(", "cudasep::tensor_tile::convert_dtype(",
    "cudasep::tensor_tile::add_scalar(", "cudasep::tensor_tile::mul_scalar(", "cudasep::tensor_tile::clamp(",
    "cudasep::tensor_tile::negate(", "cudasep::tensor_tile::greater_than(", "cudasep::tensor_tile::binary_same_shape(",
    "cudasep::tensor_tile::binary_inplace_same_shape(", "cudasep::tensor_tile::binary_glue(",
    "cudasep::tensor_tile::binary_inplace_glue(", "cudasep::tensor_tile::index_select_glue(",
    "cudasep::tensor_tile::strided_copy_glue(", "cudasep::tensor_tile::pad_const_glue(",
    "cudasep::tensor_tile::pad_reflect_glue(", "cudasep::tensor_tile::cat_glue(",
    "cudasep::tensor_tile::sum_reduce_last_dim(", "cudasep::tensor_tile::max_reduce_last_dim(",
    "cudasep::tensor_tile::sum_reduce_general_glue(", "cudasep::tensor_tile::max_reduce_general_glue(",
    "cudasep::mbr_tile::rms_norm(", "cudasep::mbr_tile::try_residual_add_rms_norm(",
    "cudasep::mbr_tile::residual_rms_norm_fused_path_enabled(", "cudasep::mbr_tile::apply_gates_and_merge_heads(",
    "cudasep::mbr_tile::split_qkv_heads_rotary(", "cudasep::mbr_tile::apply_rotary_time_split_contig_inplace(",
    "cudasep::mbr_tile::apply_rotary_time_split_contig_k_only_inplace(",
    "cudasep::mbr_tile::gather_freqs_fold_complex(", "cudasep::mbr_tile::apply_mask_and_scatter(",
    "cudasep::mbr_tile::glu_last_dim(", "cudasep::mbr_tile::tanh_act(", "cudasep::mbr_tile::zero_dc(",
    "cudasep::mbr_tile::residual_bf16_enabled(", "cudasep::mbr_tile::bias_bf16_enabled(",
    "cudasep::mbr_tile::norm_gamma_bf16_enabled(", "cudasep::mbr_tile::bands_per_freq_bf16_enabled(",
    "cudasep::mbr_tile::rotary_freqs_bf16_enabled(", "cudasep::mbr_tile::scaled_dot_product_attention(",
    "cudasep::mbr_tile::scaled_dot_product_attention_time_split_contig(",
    "cudasep::mbr_tile::scaled_dot_product_attention_time_split_contig_q_rotary(",
    "cudasep::mbr_tile::set_time_attention_context_chunk(", "cudasep::mbr_tile::set_time_attention_context_depth(",
    "cudasep::stft_tile::hann_window(", "cudasep::stft_tile::stft(", "cudasep::stft_tile::istft(",
    "cudasep::chunk_tile::accumulate_chunk(", "cudasep::chunk_tile::normalize_by_weights(",
    "cudasep::chunk_tile::process_chunked(",
    "cudasep::HipMemoryPool::allocate(",
    "cudasep::HipMemoryPool::deallocate(", "cudasep::HipMemoryPool::trim_cached_memory(",
]


def test_tensor_layer_exports_reference_api():
    assert TENSOR_LIB.exists(), "run python mbr-cuda-tile_amd/build.py"
    out = subprocess.run(["nm", "-DC", "--defined-only", str(TENSOR_LIB)], capture_output=True, text=True,
                         check=True).stdout
    missing = [name for name in API if name not in out]
    assert not missing, f"missing C++ entry points: {missing}"


def test_tensor_layer_links_only_the_c_abi():
    """The C++ layer reaches the GPU kernels through libmbrt's C-ABI only."""
    out = subprocess.run(["nm", "-DC", "--undefined-only", str(TENSOR_LIB)], capture_output=True, text=True,
                         check=True).stdout
    used = sorted({ln.split()[-1] for ln in out.splitlines() if "mbrt_" in ln})
    assert used and all(u.startswith("mbrt_") for u in used), used
    assert SELFTEST.exists()


def _selftest(*args, timeout=120):
    return subprocess.run([str(SELFTEST), *args], capture_output=True, text=True, timeout=timeout)


@pytest.mark.gpu
def test_tensor_unit_semantics(dev):
    r = _selftest("unit")
    print(r.stdout)
    fails = [ln for ln in r.stdout.splitlines() if ln.startswith("FAIL")]
    assert r.returncode == 0 and not fails, (r.returncode, fails, r.stderr[-2000:])


def _write(dirp: Path, manifest: list, name: str, arr: np.ndarray, dt: int):
    arr = np.ascontiguousarray(arr)
    (dirp / f"{name}.bin").write_bytes(arr.tobytes())
    manifest.append(f"{name} {dt} {arr.ndim} {' '.join(str(s) for s in arr.shape)}")


def _read(dirp: Path, name: str):
    meta = (dirp / f"{name}.meta").read_text().split()
    dt, shape = int(meta[0]), tuple(int(s) for s in meta[1:])
    np_dt = {F32: np.float32, BF16: np.uint16, 1: np.uint16, I64: np.int64}[dt]
    return dt, np.fromfile(dirp / f"{name}.out", dtype=np_dt).reshape(shape)


@pytest.mark.gpu
def test_mbr_tile_ops_match_oracle(orc, dev, tmp_path):
    rng_seed = 0x4D425200C0
    R, D = 300, 384
    x = orc.randn((R, D), seed=rng_seed, stream=1)
    res = orc.randn((R, D), seed=rng_seed, stream=2)
    gamma = orc.randn((D,), seed=rng_seed, stream=3, mean=1.0, std=0.02)
    scores = orc.randn((97, 60), seed=rng_seed, stream=4, std=3.0)
    h = orc.randn((64, 1536), seed=rng_seed, stream=5, std=1.5)
    bias = orc.randn((1536,), seed=rng_seed, stream=6, std=0.1)
    g = orc.from_f32(orc.randn((50, 3072), seed=rng_seed, stream=7, std=1.5), BF16)
    B, H, N, Dh = 2, 8, 60, 64
    attn = orc.from_f32(orc.randn((B, H, N, Dh), seed=rng_seed, stream=8), BF16)
    logits = orc.randn((B, N, H), seed=rng_seed, stream=9, std=2.0)
    gates = 1.0 / (1.0 + np.exp(-logits.astype(np.float64)))
    gates = gates.astype(np.float32)
    q = orc.from_f32(orc.randn((B, N, H, Dh), seed=rng_seed, stream=10), BF16)
    k = orc.from_f32(orc.randn((B, N, H, Dh), seed=rng_seed, stream=11), BF16)
    cos, sin = orc.rotary_tables(N, Dh)
    qkv = orc.from_f32(orc.randn((B, N, 3 * H * Dh), seed=rng_seed, stream=12), BF16)
    mb = orc.mel_bands(44100.0, 2048, 60, 2)
    Bb, F, T = 2, 2050, 37
    J = mb["freq_indices"].size
    stft = orc.randn((Bb, F, T, 2), seed=rng_seed, stream=13)
    m0 = orc.randn((Bb, T, J * 2), seed=rng_seed, stream=14, std=0.5)
    m1 = orc.randn((Bb, T, J * 2), seed=rng_seed, stream=15, std=0.5)
    signal = orc.randn((2, 5000), seed=rng_seed, stream=16)
    audio_a = orc.randn((1, 2, 16000), seed=rng_seed, stream=17)
    audio_b = orc.randn((1, 2, 17001), seed=rng_seed, stream=18)
    audio_c = orc.randn((1, 2, 1500), seed=rng_seed, stream=19)
    cnt = mb["bands_per_freq"].astype(np.float32)

    man: list[str] = []
    for name, arr, dt in [("x", x, F32), ("res", res, F32), ("gamma", gamma, F32), ("scores", scores, F32),
                          ("h", h, F32), ("bias", bias, F32), ("g", g, BF16), ("attn", attn, BF16),
                          ("logits", logits, F32), ("gates", gates, F32), ("q", q, BF16), ("k", k, BF16),
                          ("cos", cos, F32), ("sin", sin, F32), ("qkv", qkv, BF16), ("stft", stft, F32),
                          ("mask0", m0, F32), ("mask1", m1, F32), ("counts", cnt, F32), ("signal", signal, F32),
                          ("audio_a", audio_a, F32), ("audio_b", audio_b, F32), ("audio_c", audio_c, F32),
                          ("freq_indices", mb["freq_indices"].astype(np.int64), I64),
                          ("csr_off", mb["csr_offsets"].astype(np.int64), I64),
                          ("csr_ind", mb["csr_indices"].astype(np.int64), I64)]:
        _write(tmp_path, man, name, arr, dt)
    (tmp_path / "manifest.txt").write_text("\n".join(man) + "\n")
    r = _selftest("ops", str(tmp_path))
    print(r.stdout)
    assert r.returncode == 0, (r.returncode, r.stdout[-2000:], r.stderr[-2000:])

    scale = float(np.float32(np.sqrt(np.float32(384.0))))
    dt, y = _read(tmp_path, "rms_norm")
    assert dt == F32
    assert_close(y, orc.rms_norm(x, F32, gamma, F32, F32, scale, 1e-12), F32, "rms_norm")
    ref_n, ref_s = orc.rms_norm(x, F32, gamma, F32, F32, scale, 1e-12, res=res, sdt=F32, want_sum=True)
    assert_close(_read(tmp_path, "resid_sum")[1], ref_s, F32, "residual sum")
    assert_close(_read(tmp_path, "resid_normed")[1], ref_n, F32, "residual normed")
    ref_sm = orc.softmax(scores, F32, F32, 0.125)
    assert_close(_read(tmp_path, "softmax")[1], ref_sm, F32, "softmax")
    assert_bitexact(_read(tmp_path, "softmax_inplace")[1], _read(tmp_path, "softmax")[1], "softmax in place")
    dt, y = _read(tmp_path, "gelu_ref")
    assert dt == BF16
    assert_close(y, orc.bias_act(h, F32, bias, F32, BF16, 1), BF16, "gelu ref")
    dt, y = _read(tmp_path, "gather")
    assert dt == F32
    assert_bitexact(y, orc.band_gather(stft, mb["freq_indices"], F32, Bb, F, T), "gather")
    ref_m = orc.band_mask_merge(stft, [m0.reshape(Bb, T, J, 2), m1.reshape(Bb, T, J, 2)], F32, mb["csr_offsets"],
                                mb["csr_indices"], cnt, F32, F32, Bb, F, T, 2)
    assert_close(_read(tmp_path, "merge")[1], ref_m, F32, "merge",
                 den=merge_den(orc, stft, [m0, m1], mb, Bb, F, T, 2))
    ref_m1 = orc.band_mask_merge(stft, [m0.reshape(Bb, T, J, 2)], F32, mb["csr_offsets"], mb["csr_indices"], cnt,
                                 F32, F32, Bb, F, T, 2)
    assert_close(_read(tmp_path, "merge_rebuilt_csr")[1], ref_m1, F32, "merge (CSR rebuilt from freq_indices)",
                 den=merge_den(orc, stft, [m0], mb, Bb, F, T, 2))
    spec = stft.reshape(Bb * 2, F // 2, T, 2)
    assert_bitexact(_read(tmp_path, "zero_dc")[1], orc.zero_dc(spec, F32), "zero_dc")
    dt, y = _read(tmp_path, "glu_bf16")
    assert dt == BF16
    assert_close(y, orc.glu(g, BF16, BF16), BF16, "glu bf16")
    assert_close(_read(tmp_path, "gates_merge")[1], orc.gate_merge(attn, BF16, gates, F32, BF16, B, H, N, Dh,
                                                                   logit=False), BF16, "gate merge")
    assert_close(_read(tmp_path, "gate_logits_merge")[1], orc.gate_merge(attn, BF16, logits, F32, BF16, B, H, N, Dh,
                                                                         logit=True), BF16, "gate logits merge")
    # CUDASEP_FULL_BF16_ARITH_EXPERIMENTS: the oracle's bf16-intermediates mode, within the
    # rule of tests/test_gpu_bf16i.py (2 bf16 ulps, 98 % identical; the merge's f32 scatter
    # form to 2^-7 of its summed magnitude)
    from test_gpu_bf16i import assert_bf16i
    BF16I = 2
    assert_bf16i(_read(tmp_path, "full_rms_norm")[1], orc.rms_norm(x, F32, gamma, F32, BF16, scale, 1e-12, mode=BF16I),
                 BF16, "full-bf16 rms_norm")
    assert_bf16i(_read(tmp_path, "full_glu")[1], orc.glu(g, BF16, BF16, mode=BF16I), BF16, "full-bf16 glu")
    sb = orc.from_f32(scores, BF16)
    assert_bf16i(_read(tmp_path, "full_softmax")[1], orc.softmax(sb, BF16, BF16, 0.125, mode=BF16I), BF16,
                 "full-bf16 softmax")
    assert_bf16i(_read(tmp_path, "full_gate_logits_merge")[1],
                 orc.gate_merge(attn, BF16, logits, F32, BF16, B, H, N, Dh, logit=True, mode=BF16I), BF16,
                 "full-bf16 gate logits merge", max_ulp=1.0, min_exact=0.99)
    mb16 = [orc.from_f32(m, BF16) for m in (m0, m1)]
    dt, y = _read(tmp_path, "full_merge")
    assert dt == F32
    ref_fm = orc.band_mask_merge(stft, [m.reshape(Bb, T, J, 2) for m in mb16], BF16, mb["csr_offsets"],
                                 mb["csr_indices"], cnt, F32, F32, Bb, F, T, 2, mode=BF16I)
    den_fm = merge_den(orc, stft, [orc.to_f32(m, BF16) for m in mb16], mb, Bb, F, T, 2)
    assert float((np.abs(y.astype(np.float64) - ref_fm) / np.maximum(den_fm, 1e-30)).max()) <= 2.0 ** -7
    rq, rk = orc.rotary(q, k, BF16, cos, sin, F32, N, H, layout=1)
    assert_close(_read(tmp_path, "rot_q")[1], rq, BF16, "rotary q")
    assert_close(_read(tmp_path, "rot_k")[1], rk, BF16, "rotary k")
    qa = np.ascontiguousarray(q.reshape(B, N, H, Dh).transpose(0, 2, 1, 3)).reshape(B * H, N, Dh)
    ka = np.ascontiguousarray(k.reshape(B, N, H, Dh).transpose(0, 2, 1, 3)).reshape(B * H, N, Dh)
    dt, y = _read(tmp_path, "attention")
    assert dt == BF16 and y.shape == (B, H, N, Dh)
    ref = orc.attention(qa, ka, ka, BF16, BF16, 0.0).reshape(B, H, N, Dh)
    den = orc.attention(orc.to_f32(qa, BF16), orc.to_f32(ka, BF16), np.abs(orc.to_f32(ka, BF16)), F32, F32,
                        0.0).reshape(B, H, N, Dh)
    assert_close(y, ref, BF16, "scaled_dot_product_attention", den=den)
    # split-contig forms: the [B, N, H, D] views give the contiguous-heads result bit for bit,
    # and the in-kernel q rotary equals rotating q first
    dt, ys = _read(tmp_path, "attention_split_contig")
    assert dt == BF16 and ys.shape == (B, H, N, Dh)
    assert_bitexact(ys, y, "scaled_dot_product_attention_time_split_contig")
    dt, yr = _read(tmp_path, "attention_split_contig_qrot")
    assert dt == BF16 and yr.shape == (B, H, N, Dh)
    assert_bitexact(yr, _read(tmp_path, "attention_rotated")[1], "scaled_dot_product_attention_time_split_contig_q_rotary")
    gq, gk = _read(tmp_path, "rot_q")[1], _read(tmp_path, "rot_k")[1]
    rqa = np.ascontiguousarray(gq.reshape(B, N, H, Dh).transpose(0, 2, 1, 3)).reshape(B * H, N, Dh)
    rka = np.ascontiguousarray(gk.reshape(B, N, H, Dh).transpose(0, 2, 1, 3)).reshape(B * H, N, Dh)
    ref_r = orc.attention(rqa, rka, rka, BF16, BF16, 0.0).reshape(B, H, N, Dh)
    den_r = orc.attention(orc.to_f32(rqa, BF16), orc.to_f32(rka, BF16), np.abs(orc.to_f32(rka, BF16)), F32, F32,
                          0.0).reshape(B, H, N, Dh)
    assert_close(yr, ref_r, BF16, "split-contig q-rotary attention", den=den_r)
    sq, sk, sv = orc.split_qkv(qkv, BF16, cos, sin, F32, BF16, B, N, H, Dh, 64)
    for name, ref in (("split_q", sq), ("split_k", sk), ("split_v", sv)):
        dt, y = _read(tmp_path, name)
        assert dt == BF16 and y.shape == (B, H, 64, Dh), (name, y.shape)
        assert_close(y, ref, BF16, name)
    hann = orc.hann_window(2048)
    assert_close(_read(tmp_path, "hann")[1], hann, F32, "stft_tile::hann_window", den=orc.hann_den(2048))
    hw = _read(tmp_path, "hann")[1]
    dt, spec = _read(tmp_path, "stft")
    assert dt == F32 and spec.shape == (2, 1025, 12, 2)
    assert_close(spec, orc.stft(signal, hw, 441), F32, "stft_tile::stft", den=orc.stft_den(signal, hw, 441))
    dt, y = _read(tmp_path, "istft")
    assert dt == F32 and y.shape == (2, 5000)
    assert_close(y, orc.istft(spec, F32, hw, 441, length=5000), F32, "stft_tile::istft",
                 den=orc.istft_den(spec, F32, hw, 441, length=5000))
    sb = orc.from_f32(spec, BF16)
    dt, y = _read(tmp_path, "istft_bf16")
    assert dt == F32 and y.shape == (2, 11 * 441)
    assert_close(y, orc.istft(sb, BF16, hw, 441), F32, "stft_tile::istft bf16", den=orc.istft_den(sb, BF16, hw, 441))
    ident = lambda a: a.copy()
    for name, ref in (("chunk_a_b1", orc.process_chunked(audio_a, 4000, 3000, 1, ident)),
                      ("chunk_a_b4", orc.process_chunked(audio_a, 4000, 3000, 4, ident)),
                      ("chunk_b_2stem", orc.process_chunked(audio_b, 4000, 3200, 2,
                                                            lambda a: np.stack([2 * a, -a], axis=1))),
                      ("chunk_c_short", orc.process_chunked(audio_c, 4000, 3000, 3, ident))):
        dt, y = _read(tmp_path, name)
        assert dt == F32
        assert_bitexact(y, ref, f"chunk_tile::process_chunked {name}")


JSON_CASES = [
    '{"a": 1, "b": [1, 2.5e-3, -0.0, 1E+2], "c": {"d": null, "e": true, "f": false}}',
    '"esc \\" \\\\ \\/ \\b\\f\\n\\r\\t \\u00e9 \\ud83d\\ude00"',
    '[]', '{}', '  [ 0 , -1 , 123456789012 ]  ', '3.141592653589793', '"naïve"',
    '{"a": 1,}', '[1 2]', '{"a" 1}', 'tru', '"unterminated', '01', '[1] x', '',
]


@pytest.mark.gpu
def test_csm_loader_json_and_band_tables(orc, dev, tmp_path):
    """ModelWeights::load against files written by mbrt.csm: every tensor bit-exact (all
    dtypes, 0-d, empty, a repeated name whose last copy wins), the config through the JSON
    parser, the bf16 conversion of 2-D f32 tensors, the band tables MelBandRoformer::load
    builds from __precomputed__ tensors, and the reference's errors for malformed files."""
    import json
    import struct

    from mbrt import csm

    rng = np.random.default_rng(31)
    cfg = {"num_bands": 60, "stft_n_fft": 2048, "stereo": True, "stft_hop_length": 441,
           "model_type": "mel_band_roformer", "dims": [384, 1536], "nested": {"x": [1.5, None, "s"]}}
    items = [("layers.0.w", rng.standard_normal((384, 1536)).astype(np.float32)),
             ("layers.0.b", rng.standard_normal(1536).astype(np.float32)),
             ("half", rng.standard_normal((7, 3)).astype(np.float16)),
             ("bf", rng.integers(0, 2**16, size=(5, 9)).astype(np.uint16)),
             ("idx", np.arange(-5, 6, dtype=np.int64)),
             ("scalar", np.array(-3.25, np.float32)), ("empty", np.zeros((0, 8), np.float32)),
             ("dup", np.zeros(3, np.float32)), ("dup", np.arange(3, dtype=np.float32))]
    items += list(csm.precomputed_band_tensors(44100.0, 2048, 60, True).items())
    csm.write_csm(tmp_path / "model.csm", cfg, items, dtypes={"bf": csm.BF16})
    good = (tmp_path / "model.csm").read_bytes()
    (tmp_path / "bad_magic.csm").write_bytes(b"CSN\x00" + good[4:])
    (tmp_path / "bad_version.csm").write_bytes(good[:4] + struct.pack("<I", 3) + good[8:])
    (tmp_path / "truncated.csm").write_bytes(good[:-10])
    csm.write_csm(tmp_path / "bad_dtype.csm", {}, [("w", np.ones(2, np.float32))])
    bd = bytearray((tmp_path / "bad_dtype.csm").read_bytes())
    struct.pack_into("<I", bd, len(bd) - 8 - 4, 9)  # dtype field of the only tensor
    (tmp_path / "bad_dtype.csm").write_bytes(bytes(bd))
    # shapes whose element count (huge_numel) or byte count (huge_bytes) overflows int64:
    # the header alone says so, before any allocation or read
    csm.write_csm(tmp_path / "huge_bytes.csm", {}, [("w", np.ones(2, np.float32))])
    hb = bytearray((tmp_path / "huge_bytes.csm").read_bytes())
    struct.pack_into("<q", hb, len(hb) - 8 - 4 - 8, 2**62)  # the only dim: 2^62 f32 = 2^64 bytes
    (tmp_path / "huge_bytes.csm").write_bytes(bytes(hb))
    csm.write_csm(tmp_path / "huge_numel.csm", {}, [("w", np.ones((1, 2), np.float32))])
    hn = bytearray((tmp_path / "huge_numel.csm").read_bytes())
    struct.pack_into("<qq", hn, len(hn) - 8 - 4 - 16, 2**33, 2**33)  # 2^66 elements
    (tmp_path / "huge_numel.csm").write_bytes(bytes(hn))
    (tmp_path / "json_cases.txt").write_text("\n".join(JSON_CASES) + "\n", encoding="utf-8")

    r = _selftest("csm", str(tmp_path))
    print(r.stdout[-3000:])
    assert r.returncode == 0, (r.returncode, r.stdout[-2000:], r.stderr[-2000:])

    want = {}
    for n, a in items:
        want[n] = a
    names = (tmp_path / "names.txt").read_text(encoding="utf-8").splitlines()
    assert names == sorted(want)
    for i, n in enumerate(names):
        dt, y = _read(tmp_path, f"t{i}")
        assert y.shape == want[n].shape, n
        assert_bitexact(y, want[n].view(y.dtype) if want[n].dtype.itemsize == y.dtype.itemsize else want[n], n)
        # after convert_linear_weights_to_bf16: 2-D f32 -> bf16 (RNE), the rest unchanged
        cdt, c = _read(tmp_path, f"c{i}")
        if want[n].ndim == 2 and want[n].dtype == np.float32:
            assert cdt == BF16
            assert_bitexact(c, orc.f32_to_bf16(want[n]), f"{n} as bf16")
        else:
            assert cdt == dt
            assert_bitexact(c, y, f"{n} unchanged")
    lines = (tmp_path / "config_out.txt").read_text(encoding="utf-8").splitlines()
    assert json.loads(lines[0]) == cfg
    assert lines[1].split() == ["60", "7", "441", "1", "mel_band_roformer"]
    mb = orc.mel_bands(44100.0, 2048, 60, 2)
    assert_bitexact(_read(tmp_path, "band_offsets")[1], mb["csr_offsets"].astype(np.int64), "band CSR offsets")
    assert_bitexact(_read(tmp_path, "band_indices")[1], mb["csr_indices"].astype(np.int64), "band CSR indices")
    assert_bitexact(_read(tmp_path, "band_counts")[1], mb["bands_per_freq"].astype(np.float32), "bands per freq")
    dims = [int(v) for v in (tmp_path / "band_dims.txt").read_text().split()]
    assert dims[0] == 2 and dims[1:] == (4 * mb["freqs_per_band"]).tolist()
    errs = dict(ln.split(" ", 1) for ln in (tmp_path / "errors.txt").read_text().splitlines())
    assert errs["bad_magic"] == "ModelWeights: invalid magic (expected CSM\\0)"
    assert errs["bad_version"] == "ModelWeights: unsupported version 3"
    assert errs["truncated"].startswith("ModelWeights: unexpected EOF")
    assert errs["huge_bytes"] == "ModelWeights: tensor too large: w"
    assert errs["huge_numel"] == "ModelWeights: tensor too large: w"
    assert errs["bad_dtype"] == "ModelWeights: unknown dtype 9 for tensor w"
    assert errs["missing"].startswith("ModelWeights: cannot open file: ")
    outs = (tmp_path / "json_out.txt").read_text(encoding="utf-8").splitlines()
    assert len(outs) == len(JSON_CASES)
    for case, out in zip(JSON_CASES, outs):
        try:
            ref = json.loads(case)
        except ValueError:
            assert out.startswith("ERR JSON parse error at position"), (case, out)
            continue
        assert not out.startswith("ERR"), (case, out)
        assert json.loads(out) == ref, (case, out)

