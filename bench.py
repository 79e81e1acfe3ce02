"""Benchmark of the MelBandRoformer tensor-op hot path on one MI355X.

One step = one pass of every op of the MelBandRoformer tensor path at its full chunk
shape (BL-1 .. BL-5), each on synthetic inputs already resident in HBM:
  BL-1  residual add + RMSNorm f32 [48060, 384] (writes the sum and the normed rows)
  BL-2  GELU bf16 [48060, 1536]; GLU bf16 [48060, 3072]; sigmoid gate x head merge bf16
        attn [60, 8, 801, 64] + logits [48060, 8]
  BL-3  row softmax, f32 and bf16: time [480*801, 801] and freq [6408*60, 60]
  BL-4  rotary in place bf16 q, k [480, 801, 64] with f32 cos/sin [801, 32];
        permute bf16 [4, 801, 60, 384] -> [4, 60, 801, 384] and back
  BL-5  band gather and mask merge, batch 4, 60 mel bands (3958 stereo band-bins)
value = sum of algorithmic bytes / sum of op times (GB/s, all ops); per-op GB/s and the
fraction of the 8 TB/s HBM peak are in config.per_op.  The K steps are timed op-major:
each op's K calls run back to back, bracketed by one pair of HIP events on the stream the
kernels run on, so every op pays for its own cache write-backs and an op's time is that
span over K.  Each op cycles through enough buffer sets that the working set between two
uses of a set exceeds 1 GB, so the 256 MB MALL cannot serve repeats.  Algorithmic bytes
count every input read once and every output written once.

cpu_baseline: the oracle's float pipeline (oracle/, OpenMP) on a row sample of every op,
timed on this host's cores.

  python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu]
"""
from __future__ import annotations

import argparse
import gc
import json
import math
import os
import re
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO / "mbr-cuda-tile_amd"))

METRIC = "achieved HBM GB/s (% of MI355X peak) per op; ms of tensor ops per chunk"
HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0  # dense bf16
MALL_DEFEAT_BYTES = 1.1e9
TRAFFIC_SUMMARY = REPO / "profiles" / "traffic_all_ops.md"


def parse_args():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-copy", action="store_true", help="skip the same-size copy timed beside every op")
    ap.add_argument("--copy-ceiling", action="store_true",
                    help="only measure the copy rate by size and the one-element launch time")
    ap.add_argument("--cpu-threads", type=int, default=None,
                    help="threads of the CPU baseline (default: the CPUs available, capped by OMP_NUM_THREADS)")
    ap.add_argument("--only", default=None,
                    help="comma-separated op-name substrings: time only those ops (tuning runs; "
                         "value then covers the selected ops only)")
    return ap.parse_args()


class Op:
    def __init__(self, name, nbytes, make, kernel):
        self.name = name
        self.bytes = nbytes      # algorithmic bytes per call
        self.make = make         # () -> buffer set (dict)
        self.kernel = kernel     # kernel symbol substring (for the rocprof cross-check)
        self.sets = []
        self.flops = 0.0
        self.next = False
        self.run = None          # (buffer set) -> None
        self.ms = 0.0            # mean GPU time per call over the timed calls
        self.retimed = 0         # timings redone because the host enqueue outlasted the hold
        self.copy_ms = 0.0       # a plain copy of the same bytes, timed the same way
        self.mix = None          # "r1w2": also compared with a contiguous kernel of the same read/write mix
        self.mix_ms = 0.0


def build_ops(torch, mbrt, bands):
    dev = "cuda"
    g = torch.Generator(device=dev).manual_seed(0x4D42520000)

    def randn(shape, dtype=torch.float32, std=1.0, mean=0.0):
        return (torch.randn(shape, generator=g, device=dev) * std + mean).to(dtype)

    bf16, f32 = torch.bfloat16, torch.float32
    ops = []

    # BL-1 residual + RMSNorm f32
    R, D = 48060, 384
    gamma = randn((D,), mean=1.0, std=0.02)
    op = Op("bl1_residual_rmsnorm_f32", 4 * R * D * 4 + D * 4,
            lambda: dict(x=randn((R, D)), r=randn((R, D)), s=torch.empty((R, D), device=dev),
                         y=torch.empty((R, D), device=dev)), "rms_fast_kernel")
    op.run = lambda b: mbrt.residual_add_rms_norm(b["x"], b["r"], gamma, b["s"], b["y"], math.sqrt(D), 1e-8)
    ops.append(op)

    # BL-2a GELU bf16
    op = Op("bl2a_gelu_bf16", 2 * 48060 * 1536 * 2,
            lambda: dict(x=randn((48060, 1536), bf16, 1.5), y=torch.empty((48060, 1536), dtype=bf16, device=dev)),
            "bias_act_vec_kernel")
    op.run = lambda b: mbrt.bias_act(b["x"], None, b["y"], mbrt.ACT_GELU_REF)
    ops.append(op)

    # BL-2b GLU bf16
    op = Op("bl2b_glu_bf16", 48060 * 3072 * 2 + 48060 * 1536 * 2,
            lambda: dict(x=randn((48060, 3072), bf16, 1.5), y=torch.empty((48060, 1536), dtype=bf16, device=dev)),
            "glu_vec_kernel")
    op.run = lambda b: mbrt.glu(b["x"], b["y"])
    ops.append(op)

    # BL-2c sigmoid gate x head merge bf16, attention output head-major [B, H, N, D]
    B, H, N, Dh = 60, 8, 801, 64
    op = Op("bl2c_gate_merge_bf16", 2 * B * H * N * Dh * 2 + B * N * H * 2,
            lambda B=B, H=H, N=N, Dh=Dh: dict(a=randn((B, H, N, Dh), bf16), gl=randn((B, N, H), bf16, 2.0),
                                              y=torch.empty((B, N, H * Dh), dtype=bf16, device=dev)),
            "gate_merge_vec_kernel")
    op.run = lambda b: mbrt.gate_merge(b["a"], b["gl"], b["y"], mbrt.LAYOUT_BHND)
    ops.append(op)

    # BL-3 softmax
    for tag, rows, cols in (("time", 480 * 801, 801), ("freq", 6408 * 60, 60)):
        for dt, dname in ((f32, "f32"), (bf16, "bf16")):
            es = 4 if dt == f32 else 2
            op = Op(f"bl3_softmax_{tag}_{dname}", 2 * rows * cols * es,
                    (lambda rows=rows, cols=cols, dt=dt: dict(x=randn((rows, cols), dt, 3.0),
                                                              y=torch.empty((rows, cols), dtype=dt, device=dev))),
                    # rows of up to 1024 elements are staged through LDS; 2-byte rows of 60 go
                    # in register row pairs
                    "softmax_pair_kernel" if (tag, dname) == ("freq", "bf16") else "softmax_staged_kernel")
            op.run = lambda b: mbrt.softmax(b["x"], b["y"], 1.0)
            ops.append(op)

    # BL-4a rotary in place, bf16 q/k [480, 801, 64], f32 tables [801, 32]
    cos_h, sin_h = mbrt.rotary_tables(801, 64, 10000.0)
    cos, sin = torch.from_numpy(cos_h).to(dev), torch.from_numpy(sin_h).to(dev)
    op = Op("bl4a_rotary_bf16", 4 * 480 * 801 * 64 * 2 + 2 * 801 * 32 * 4,
            lambda: dict(q=randn((480, 801, 64), bf16), k=randn((480, 801, 64), bf16)), "rotary_vec_kernel")
    op.run = lambda b: mbrt.rotary_(b["q"], b["k"], cos, sin, mbrt.LAYOUT_BHND)
    ops.append(op)

    # BL-4b permutes [4, 801, 60, 384] <-> [4, 60, 801, 384] bf16
    n_el = 4 * 801 * 60 * 384
    op = Op("bl4b_permute_btf_to_bft_bf16", 2 * n_el * 2,
            lambda: dict(x=randn((4, 801, 60, 384), bf16), y=torch.empty((4, 60, 801, 384), dtype=bf16, device=dev)),
            "row_copy_kernel")
    op.run = lambda b: mbrt.strided_copy(b["x"].permute(0, 2, 1, 3), b["y"])
    ops.append(op)
    op = Op("bl4b_permute_bft_to_btf_bf16", 2 * n_el * 2,
            lambda: dict(x=randn((4, 60, 801, 384), bf16), y=torch.empty((4, 801, 60, 384), dtype=bf16, device=dev)),
            "row_copy_kernel")
    op.run = lambda b: mbrt.strided_copy(b["x"].permute(0, 2, 1, 3), b["y"])
    ops.append(op)

    # BL-5 band split / merge, batch 4, stereo, 60 mel bands
    fi, off, ind, cnt = bands
    Bb, F, T = 4, 2050, 801
    J = fi.numel()
    op = Op("bl5a_band_gather_f32", Bb * F * T * 2 * 4 + Bb * T * J * 2 * 4 + J * 4,
            lambda: dict(s=randn((Bb, F, T, 2)), y=torch.empty((Bb, T, J * 2), device=dev)), "band_gather_pipe_kernel")
    op.run = lambda b: mbrt.band_gather(b["s"], fi, b["y"])
    op.mix = "r1w2"  # reads the stft once (52.5 MB), writes twice as much (101.4 MB)
    ops.append(op)
    op = Op("bl5b_band_mask_merge_f32",
            Bb * T * J * 2 * 4 + Bb * F * T * 2 * 4 + Bb * 2 * (F // 2) * T * 2 * 4 + (off.numel() + J) * 4 + F * 4,
            lambda: dict(s=randn((Bb, F, T, 2)), m=randn((Bb, T, J * 2), std=0.5),
                         y=torch.empty((Bb * 2, F // 2, T, 2), device=dev)), "band_merge_kernel")
    op.run = lambda b: mbrt.band_mask_merge(b["s"], [b["m"]], off, ind, cnt, b["y"], 2)
    ops.append(op)
    # Fused attention (MFMA), the first widening beyond the tensor-op path: q, k, v bf16
    # [BH, N, 64] for the time (480 x 801) and frequency (6408 x 60) attention.  Reported in
    # config.next_ops with TFLOP/s (4 BH N^2 64 flop); not part of `value`.
    P_SUFFIX = {mbrt.ATTN_P_PAIR: "", mbrt.ATTN_P_BF16: "_p_bf16", mbrt.ATTN_P_BF16_FAST: "_p_bf16_fast"}
    for atag, abh, an, pb in (("time", 480, 801, mbrt.ATTN_P_PAIR), ("freq", 6408, 60, mbrt.ATTN_P_PAIR),
                              ("time", 480, 801, mbrt.ATTN_P_BF16), ("freq", 6408, 60, mbrt.ATTN_P_BF16),
                              ("time", 480, 801, mbrt.ATTN_P_BF16_FAST), ("freq", 6408, 60, mbrt.ATTN_P_BF16_FAST)):
        op = Op(f"attention_{atag}_bf16" + P_SUFFIX[pb], 4 * abh * an * 64 * 2,
                (lambda abh=abh, an=an: dict(q=randn((abh, an, 64), bf16), k=randn((abh, an, 64), bf16),
                                             v=randn((abh, an, 64), bf16),
                                             y=torch.empty((abh, an, 64), dtype=bf16, device=dev))),
                "attention_kernel")
        op.flops = 4.0 * abh * an * an * 64
        op.next = True
        op.run = lambda b, pb=pb: mbrt.attention(b["q"], b["k"], b["v"], b["y"], 0.125, p_precision=pb)
        ops.append(op)
    # The time attention as the reference's split-contig q-rotary form plus the gate: q, k, v
    # read in place from the fused qkv projection [60, 801, 3*8*64], q rotated in the kernel,
    # the sigmoid gate [60, 801, 8] and the head merge applied in the epilogue -> [60, 801, 512].
    # It replaces rotary-on-q + the split + attention + gate merge.
    Bq, Nq, Hq = 60, 801, 8
    cos_t, sin_t = (torch.from_numpy(t).to(dev) for t in mbrt.rotary_tables(Nq, 64))
    op = Op("attention_time_fused_qrot_gate_bf16", Bq * Nq * 3 * Hq * 64 * 2 + Bq * Nq * Hq * 2 + Bq * Nq * Hq * 64 * 2,
            lambda: dict(qkv=randn((Bq, Nq, 3 * Hq * 64), bf16), g=randn((Bq, Nq, Hq), bf16, std=2.0),
                         y=torch.empty((Bq, Nq, Hq * 64), dtype=bf16, device=dev)),
            "attention_kernel")
    op.flops = 4.0 * Bq * Hq * Nq * Nq * 64
    op.next = True

    def run_fused(b):
        q5 = b["qkv"].view(Bq, Nq, 3, Hq, 64)
        mbrt.attention_bnhd(q5[:, :, 0], q5[:, :, 1], q5[:, :, 2], b["y"], 0.125, cos=cos_t, sin=sin_t, gate=b["g"])
    op.run = run_fused
    ops.append(op)
    # STFT / iSTFT (n_fft 2048, hop 441, Hann, centred) of the chunk: 4 x 2 channels x 352800
    # samples <-> [8, 1025, 801, 2].  Memory-bound; reported in config.next_ops with GB/s of
    # algorithmic bytes (signal + spectrum; the iSTFT's frame workspace is not counted).
    win = mbrt.hann_window(2048)
    Bs, Ls, Ts = 8, 352800, 801
    sb = Bs * Ls * 4 + 2048 * 4 + Bs * 1025 * Ts * 2 * 4
    op = Op("stft_chunk_f32", sb, lambda: dict(x=randn((Bs, Ls)), y=torch.empty((Bs, 1025, Ts, 2), device=dev)),
            "stft_kernel")
    op.next = True
    op.run = lambda b: mbrt.stft(b["x"], win, 441, out=b["y"])
    ops.append(op)
    for stag, sdt, ssz in (("f32", torch.float32, 4), ("bf16", bf16, 2)):
        op = Op(f"istft_chunk_{stag}", Bs * 1025 * Ts * 2 * ssz + 2048 * 4 + Bs * Ls * 4,
                (lambda sdt=sdt: dict(s=randn((Bs, 1025, Ts, 2), sdt), y=torch.empty((Bs, Ls), device=dev),
                                      w=torch.empty(mbrt.istft_workspace_bytes(Bs, Ts, 441) // 4, device=dev))),
                "istft_block_kernel")
        op.next = True
        op.run = lambda b: mbrt.istft(b["s"], win, 441, length=Ls, out=b["y"], workspace=b["w"])
        ops.append(op)
    # Chunk overlap-add: one 8 s chunk of 8 channels (4 stems x stereo) added at its offset into
    # a 24 s output with its fade window, and the final divide by the weight sum.
    Cc, Nc, Lc, off_c = 8, 352800, 1058400, 264600
    fade = torch.from_numpy(mbrt.chunk_fade_window(Nc, Nc // 10)).to(dev)
    op = Op("chunk_accumulate_8ch", Cc * Nc * 4 + Nc * 4 + 2 * Cc * Nc * 4 + 2 * Nc * 4,
            lambda: dict(s=randn((Cc, Nc)), d=randn((Cc, Lc)), w=torch.rand(Lc, device=dev) + 1.0),
            "accumulate_cw_kernel")
    op.next = True
    op.run = lambda b: mbrt.chunk_accumulate(b["d"], b["w"], b["s"], fade, off_c)
    ops.append(op)
    op = Op("chunk_normalize_8ch", 2 * Cc * Lc * 4 + Lc * 4,
            lambda: dict(d=randn((Cc, Lc)), w=torch.rand(Lc, device=dev) + 1.0), "normalize_vec_kernel")
    op.next = True
    op.run = lambda b: mbrt.chunk_normalize(b["d"], b["w"])
    ops.append(op)
    return ops


def make_sets(op):
    """Enough buffer sets that the working set between two uses of one set exceeds the
    MALL-defeat size, so that the 256 MB MALL cannot serve a repeat."""
    first = op.make()
    ws = sum(t.numel() * t.element_size() for t in first.values())
    nsets = 1 if ws >= MALL_DEFEAT_BYTES else max(2, math.ceil(MALL_DEFEAT_BYTES / ws) + 1)
    op.sets = [first] + [op.make() for _ in range(nsets - 1)]


def make_timer(torch, stream, steps, warmup):
    """Returns time_op(op): warm calls, then K back-to-back calls bracketed by one HIP event
    pair on `stream`; op.ms = span / K.

    The host enqueues the K calls while the stream is held by a spin kernel, so that they
    run back to back on the GPU and the events time the kernels, not the Python launch path
    (a ctypes call costs ~10 us, as long as the smaller ops).  Python's garbage collector is
    off meanwhile, and should the enqueue still take more than half the hold, the op is
    timed again with a longer hold: no GPU idle time can then fall inside the span."""
    c0, c1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda._sleep(1 << 20)
    c0.record(stream)
    torch.cuda._sleep(1 << 20)
    c1.record(stream)
    torch.cuda.synchronize()
    ms_per_unit = max(c0.elapsed_time(c1), 1e-3)  # GPU ms of a 2^20-cycle spin

    def time_op(op):
        for i in range(warmup):
            op.run(op.sets[i % len(op.sets)])
        torch.cuda.synchronize()
        hold_ms = 2.0 + 0.3 * steps
        for attempt in range(4):
            a0, a1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            gc.disable()
            try:
                torch.cuda._sleep(int((1 << 20) * max(1.0, hold_ms / ms_per_unit)))
                h0 = time.perf_counter()
                a0.record(stream)
                for i in range(steps):
                    op.run(op.sets[(warmup + i) % len(op.sets)])
                a1.record(stream)
                enqueue_ms = (time.perf_counter() - h0) * 1e3
            finally:
                gc.enable()
            torch.cuda.synchronize()
            if enqueue_ms < 0.5 * hold_ms:
                op.ms = a0.elapsed_time(a1) / steps
                op.retimed = attempt
                return
            hold_ms *= 4
        raise RuntimeError(f"bench.py: the host could not enqueue {op.name} within the stream hold")

    return time_op


def copy_op(torch, mbrt, nbytes):
    """A plain contiguous copy that moves `nbytes` (half read, half written) with the
    library's row-copy kernel: the ceiling an HBM-bound op of that size is compared with."""
    n = max(4, int(nbytes) // 32 * 4)  # whole 16-byte vectors per buffer: the vector copy path
    op = Op(f"copy_{nbytes}", n * 8, lambda: dict(x=torch.empty(n, device="cuda"), y=torch.empty(n, device="cuda")),
            "row_copy_kernel")
    op.run = lambda b: mbrt.strided_copy(b["x"], b["y"])
    return op


def mix_op(torch, mbrt, nbytes):
    """A contiguous kernel that reads one third and writes two thirds of `nbytes`: the
    library's bf16 -> f32 conversion.  The ceiling for ops with that read/write mix."""
    n = max(8, int(nbytes) // 6 // 8 * 8)
    op = Op(f"mix_r1w2_{nbytes}", n * 6,
            lambda: dict(x=torch.empty(n, dtype=torch.bfloat16, device="cuda"), y=torch.empty(n, device="cuda")),
            "convert_vec_kernel")
    op.run = lambda b: mbrt.convert(b["x"], b["y"])
    return op


def copy_ceiling(torch, mbrt, args):
    """--copy-ceiling: copy rate by size, and the time of a one-element launch (the fixed
    cost every kernel pays between back-to-back calls on one stream)."""
    stream = torch.cuda.current_stream()
    time_op = make_timer(torch, stream, args.steps, args.warmup)
    tiny = Op("launch_1_element", 8, lambda: dict(x=torch.empty(1, device="cuda")), "fill_kernel")
    tiny.run = lambda b: mbrt.fill_(b["x"], 1.0)
    tiny.sets = [tiny.make()]
    time_op(tiny)
    rows = []
    for mb in (12.5, 25, 50, 75, 100, 150, 200, 300, 400, 600, 1000, 2000):
        op = copy_op(torch, mbrt, int(mb * 1e6))
        make_sets(op)
        time_op(op)
        rows.append({"bytes_moved": op.bytes, "us": round(op.ms * 1e3, 2),
                     "gbs": round(op.bytes / (op.ms * 1e-3) / 1e9, 1)})
        print(f"copy {op.bytes / 1e6:8.1f} MB moved: {op.ms * 1e3:8.2f} us  {rows[-1]['gbs']:7.1f} GB/s",
              file=sys.stderr, flush=True)
        op.sets = []
        torch.cuda.empty_cache()
    mix_rows = []
    for mb in (50, 100, 150, 200, 400):
        op = mix_op(torch, mbrt, int(mb * 1e6))
        make_sets(op)
        time_op(op)
        mix_rows.append({"bytes_moved": op.bytes, "us": round(op.ms * 1e3, 2),
                         "gbs": round(op.bytes / (op.ms * 1e-3) / 1e9, 1)})
        print(f"read 1 : write 2 {op.bytes / 1e6:8.1f} MB moved: {op.ms * 1e3:8.2f} us  {mix_rows[-1]['gbs']:7.1f} GB/s",
              file=sys.stderr, flush=True)
        op.sets = []
        torch.cuda.empty_cache()
    print(json.dumps({"copy_ceiling": rows, "read1_write2_ceiling": mix_rows,
                      "read1_write2_kernel": "bf16 -> f32 convert_vec_kernel",
                      "launch_1_element_us": round(tiny.ms * 1e3, 3),
                      "kernel": "row_copy_kernel<16, 1>", "steps": args.steps,
                      "mall_defeat": f"buffer sets cycled past {MALL_DEFEAT_BYTES / 1e9:.1f} GB"}), flush=True)


def band_tables(torch, mbrt):
    """60-band stereo layout (sr 44100, n_fft 2048) and its per-freq CSR, built on the
    host by the library (as the reference's loader does) and uploaded once."""
    fi, _ = mbrt.mel_band_layout(44100.0, 2048, 60, 2)
    off, ind, cnt, _ = mbrt.band_csr(fi, 2050)
    t = lambda a: torch.from_numpy(a).to("cuda")
    return t(fi), t(off), t(ind), t(cnt)


def read_traffic() -> dict:
    """HBM bytes per launch of every op, from the committed rocprofv3 --pmc summary
    (FETCH_SIZE + WRITE_SIZE, calibrated with a copy of known size); {} if absent."""
    if not TRAFFIC_SUMMARY.exists():
        return {}
    return {m.group(1): float(m.group(2)) for m in
            re.finditer(r"^traffic_bytes_per_launch\[(\w+)\]:\s*([0-9.eE+]+)", TRAFFIC_SUMMARY.read_text(), flags=re.M)}


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform
    return platform.processor() or "unknown"


def cpu_threads_available() -> tuple[int, int]:
    """(threads to use, CPUs visible to this process).  The threads are the CPUs this
    process may run on, capped by OMP_NUM_THREADS when the host sets it: a shared host
    gives each GPU a share of its cores and says so there."""
    visible = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    env = os.environ.get("OMP_NUM_THREADS", "")
    use = min(visible, int(env)) if env.isdigit() and int(env) > 0 else visible
    return use, visible


def cpu_baseline(threads: int | None):
    """The oracle's float pipeline (f32 arithmetic, bf16 RNE on store, OpenMP over rows) on
    a sample of every BL op, timed on this host: 1 warm run, then the median of 5 timed runs
    per op, once on all the threads available and once on 1 thread."""
    import statistics

    import numpy as np

    sys.path.insert(0, str(REPO / "oracle"))
    import oracle as O

    if not O.LIB.exists():
        O.build()
    use, visible = cpu_threads_available()
    nthreads = threads or use
    rng = np.random.default_rng(0x4D42520000)
    frac = 2  # half of the rows (or frames) of every op
    rnd = lambda shape, std=1.0: (rng.standard_normal(shape, dtype=np.float32) * np.float32(std))
    bf = O.f32_to_bf16
    jobs = []
    R, D = 48060 // frac, 384
    x, r, gm = rnd((R, D)), rnd((R, D)), rnd(D) * np.float32(0.02) + np.float32(1.0)
    jobs.append(("bl1", 4 * R * D * 4, lambda: O.rms_norm(x, O.F32, gm, O.F32, O.F32, math.sqrt(D), 1e-8, res=r,
                                                         sdt=O.F32, mode=O.FAST, want_sum=True)))
    h = bf(rnd((48060 // frac, 1536), 1.5))
    jobs.append(("bl2a", 2 * h.size * 2, lambda: O.bias_act(h, O.BF16, None, O.F32, O.BF16, 1, mode=O.FAST)))
    h2 = bf(rnd((48060 // frac, 3072), 1.5))
    jobs.append(("bl2b", h2.size * 2 * 3 // 2, lambda: O.glu(h2, O.BF16, O.BF16, mode=O.FAST)))
    nb = 60 // frac
    at, gl = bf(rnd((nb, 8, 801, 64))), bf(rnd((nb, 801, 8), 2.0))
    jobs.append(("bl2c", 2 * at.size * 2 + gl.size * 2,
                 lambda: O.gate_merge(at, O.BF16, gl, O.BF16, O.BF16, nb, 8, 801, 64, mode=O.FAST)))
    for rows, cols in ((480 * 801 // frac, 801), (6408 * 60 // frac, 60)):
        s32 = rnd((rows, cols), 3.0)
        s16 = bf(s32)
        jobs.append((f"bl3_{cols}_f32", 2 * s32.size * 4, lambda s32=s32: O.softmax(s32, O.F32, O.F32, 1.0, O.FAST)))
        jobs.append((f"bl3_{cols}_bf16", 2 * s16.size * 2, lambda s16=s16: O.softmax(s16, O.BF16, O.BF16, 1.0, O.FAST)))
    q, k = bf(rnd((480 // frac, 801, 64))), bf(rnd((480 // frac, 801, 64)))
    cs, sn = O.rotary_tables(801, 64)
    jobs.append(("bl4a", 4 * q.size * 2, lambda: O.rotary(q, k, O.BF16, cs, sn, O.F32, 801, 1, mode=O.FAST)))
    p = bf(rnd((4, 801, 60 // frac, 384)))
    pv = p.reshape(-1)
    fb = 60 // frac
    shp, strd = (4, fb, 801, 384), (801 * fb * 384, 384, fb * 384, 1)
    jobs.append(("bl4b", 2 * p.size * 2, lambda: O.strided_copy(pv, shp, strd)))
    mb = O.mel_bands()
    J = mb["freq_indices"].size
    T = 801 // frac
    st = rnd((4, 2050, T, 2))
    jobs.append(("bl5a", st.size * 4 + 4 * T * J * 2 * 4, lambda: O.band_gather(st, mb["freq_indices"], O.F32, 4, 2050, T)))
    mk = rnd((4, T, J, 2), 0.5)
    cnt = mb["bands_per_freq"].astype(np.float32)
    jobs.append(("bl5b", mk.size * 4 + 2 * st.size * 4,
                 lambda: O.band_mask_merge(st, [mk], O.F32, mb["csr_offsets"], mb["csr_indices"], cnt, O.F32, O.F32, 4,
                                           2050, T, 2, mode=O.FAST)))

    def run_all(n):
        O.set_threads(n)
        per, tot_s = {}, 0.0
        for name, nbytes, fn in jobs:
            fn()  # warm
            ts = []
            for _ in range(5):
                t0 = time.perf_counter()
                fn()
                ts.append(time.perf_counter() - t0)
            med = statistics.median(ts)
            per[name] = round(nbytes / med / 1e9, 2)
            tot_s += med
        return per, tot_s

    tot_b = sum(nb for _, nb, _ in jobs)
    wall0 = time.perf_counter()
    per_all, s_all = run_all(nthreads)
    per_one, s_one = run_all(1)
    wall = time.perf_counter() - wall0
    return {
        "value": round(tot_b / s_all / 1e9, 3),
        "unit": "GB/s",
        "cores": nthreads,
        "kind": "port",
        "sample": f"1/{frac} of the rows (or frames) of every BL-1..BL-5 op ({tot_b / 1e9:.2f} GB of algorithmic "
                  f"bytes per pass), oracle float pipeline (oracle/oracle.cpp, ORC_FAST, OpenMP static over rows, "
                  f"-O3 -march=native); per op 1 warm run then the median of 5 timed runs; value = bytes / sum of "
                  f"per-op medians on {nthreads} threads; {wall:.1f} s wall for both thread counts",
        "cpu_model": cpu_model(),
        "cpus_visible": visible,
        "threads_available": use,
        "threads_1_gbs": round(tot_b / s_one / 1e9, 3),
        "per_op_gbs": per_all,
        "per_op_gbs_1_thread": per_one,
    }


def main():
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py: measures one GPU only (got --gpus {args.gpus}); "
              "the ops shard per row with no exchange, so run one process per GPU.", file=sys.stderr)
        sys.exit(2)
    import torch

    import mbrt

    torch.cuda.set_device(0)
    if args.copy_ceiling:
        copy_ceiling(torch, mbrt, args)
        return
    bands = band_tables(torch, mbrt)
    ops = build_ops(torch, mbrt, bands)
    if args.only:
        keys = [k for k in args.only.split(",") if k]
        ops = [op for op in ops if any(k in op.name for k in keys)]
    for op in ops:
        make_sets(op)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()

    # Op-major order: every op runs its K calls back to back, so an op's time includes the
    # write-back of the dirty lines its own previous call left in the MALL, not those of a
    # different op.  One HIP event pair on the kernels' stream brackets an op's K calls and
    # the op's time is that span over K: no events sit between the calls, as in a pipeline
    # (the reference's own benchmark reports time over N calls the same way).
    time_op = make_timer(torch, stream, args.steps, args.warmup)
    t0 = time.perf_counter()
    for op in ops:
        time_op(op)
    wall = time.perf_counter() - t0
    # the ceiling each op is held against: a plain copy moving the same bytes, timed the same way
    if not args.no_copy:
        for op in ops:
            if op.next:
                continue
            c = copy_op(torch, mbrt, op.bytes)
            make_sets(c)
            time_op(c)
            op.copy_ms = c.ms
            c.sets = []
            if op.mix == "r1w2":
                c = mix_op(torch, mbrt, op.bytes)
                make_sets(c)
                time_op(c)
                op.mix_ms = c.ms
                c.sets = []
        torch.cuda.empty_cache()

    per_op = {}
    next_ops = {}
    tot_bytes = 0
    tot_ms = 0.0
    traffic = read_traffic()

    def with_traffic(entry, op):
        if op.name in traffic:
            entry["traffic"] = traffic[op.name]
            entry["traffic_over_algorithmic"] = round(traffic[op.name] / op.bytes, 4)
        return entry

    for op in [o for o in ops if o.next]:
        ms = op.ms
        gbs = op.bytes / (ms * 1e-3) / 1e9
        if op.flops > 0:
            tf = op.flops / (ms * 1e-3) / 1e12
            # the roof that bounds it: MFMA above the ridge point (peak flop/s over peak B/s)
            mfma = op.flops / op.bytes > MFMA_BF16_PEAK_TFLOPS * 1e12 / (HBM_PEAK_GBS * 1e9)
            next_ops[op.name] = {"flops": op.flops, "bytes": op.bytes, "ms": round(ms, 5), "tflops": round(tf, 1),
                                 "frac_mfma_bf16_peak": round(tf / MFMA_BF16_PEAK_TFLOPS, 4),
                                 "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4), "bound": "mfma" if mfma else "hbm"}
        else:
            next_ops[op.name] = {"bytes": op.bytes, "ms": round(ms, 5), "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4)}
        with_traffic(next_ops[op.name], op)
        next_ops[op.name].pop("traffic", None)  # the ratio is kept; the line stays short
    ops = [o for o in ops if not o.next]
    for op in ops:
        ms = op.ms
        gbs = op.bytes / (ms * 1e-3) / 1e9
        per_op[op.name] = {"bytes": op.bytes, "ms": round(ms, 5),
                           "gbs": round(gbs, 1), "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4), "kernel": op.kernel}
        if op.copy_ms:
            per_op[op.name]["frac_of_same_size_copy"] = round(op.copy_ms / ms, 4)
        if op.mix_ms:
            per_op[op.name]["frac_of_same_mix_kernel"] = round(op.mix_ms / ms, 4)
        with_traffic(per_op[op.name], op)
        per_op[op.name].pop("traffic", None)
        if op.retimed:
            per_op[op.name]["retimed"] = op.retimed
        if gbs > HBM_PEAK_GBS:  # inputs are cycled past the MALL: this can only be a measurement error
            print(f"bench.py: {op.name} reports {gbs:.0f} GB/s, above the HBM peak", file=sys.stderr)
            per_op[op.name]["suspect"] = True
        tot_bytes += op.bytes
        tot_ms += ms
    if not ops:  # a tuning run of next_ops only
        print(json.dumps({"config": {"next_ops": next_ops}}), flush=True)
        return
    dom = max(ops, key=lambda o: o.ms)
    dom_ms = dom.ms
    achieved = dom.bytes / (dom_ms * 1e-3) / 1e9
    value = tot_bytes / (tot_ms * 1e-3) / 1e9

    # plain copy of known size, outside the timed region: calibrates FETCH_SIZE/WRITE_SIZE
    cal = torch.empty(1 << 28, dtype=torch.float32, device="cuda")
    cal_out = torch.empty_like(cal)
    mbrt.strided_copy(cal, cal_out)
    torch.cuda.synchronize()
    del cal, cal_out

    line = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(tot_ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": "mbr_chunk_tensor_ops: BL-1..BL-5 at full MelBandRoformer chunk shape "
                        "(T=801 frames, 60 bands, D=384, batch 4 band split), one pass per step",
            "ms_tensor_ops_per_step": round(tot_ms, 4),
            "ms_per_step_note": "sum of per-op means, each one HIP event pair over the op's K "
                                "back-to-back calls; wall_ms_per_step adds the holds and syncs",
            "wall_ms_per_step": round(wall * 1e3 / args.steps, 4),
            "frac_hbm_peak_all_ops": round(value / HBM_PEAK_GBS, 4),
            "storage_dtypes": "f32 and bf16 per op name; all arithmetic in f32",
            "mall_defeat": f"each op cycles >= {MALL_DEFEAT_BYTES / 1e9:.1f} GB of buffer sets",
            "per_op_fields": "traffic_over_algorithmic: rocprofv3 FETCH_SIZE + WRITE_SIZE per launch "
                             "(profiles/traffic_all_ops.md) over bytes; frac_of_same_size_copy: a plain "
                             "copy of the same bytes timed beside the op, over the op's time",
            "per_op": per_op,
            "next_ops": next_ops,
        },
        "roofline": {
            "bound": "hbm",
            "kernel": dom.kernel,
            "op": dom.name,
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic.get(dom.name),
            "algorithmic_bytes": dom.bytes,
            "avg_ms": round(dom_ms, 5),
        },
        "cpu_baseline": None if args.no_cpu else cpu_baseline(args.cpu_threads),
        # the same fractions in two short maps, last on the line: BL ops of the HBM peak, the
        # widened ops of the roof that bounds each (bf16 MFMA or HBM)
        "frac_hbm_peak_per_op": {k: v["frac_hbm_peak"] for k, v in per_op.items()},
        "frac_of_roof_next_ops": {k: v["frac_mfma_bf16_peak" if v.get("bound") == "mfma" else "frac_hbm_peak"]
                                  for k, v in next_ops.items()},
    }
    print(json.dumps(line, separators=(",", ":")), flush=True)


if __name__ == "__main__":
    main()
