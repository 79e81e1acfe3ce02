"""GPU parity of every C-ABI entry point against the CPU oracle.

Inputs are seeded (oracle RNG) and copied to the device; outputs come back through the
C-ABI (mbrt ctypes binding) and are compared with the oracle on the same inputs under
the rules in parity.py: bit-exact for copies, gathers and integer work; 1e-5 relative
(f32) or 1 ulp + 2e-3 norm-wise (bf16/f16) for float math.  The MelBandRoformer chunk
shapes run at full size where the oracle finishes in seconds, otherwise on a sampled set
of rows plus size-independent properties over the whole tensor.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import mbrt
from gpu_util import empty, say, to_dev, to_host
from parity import BF16, F16, F32, I32, I64, assert_bitexact, assert_close, merge_den, pair_den

pytestmark = pytest.mark.gpu

SEED = {1: 0x4D42520001, 2: 0x4D42520002, 3: 0x4D42520003, 4: 0x4D42520004, 5: 0x4D42520005}


def inp(orc, shape, seed, stream, dt=F32, mean=0.0, std=1.0):
    x = orc.randn(shape, seed=seed, stream=stream, mean=mean, std=std)
    return x if dt == F32 else orc.from_f32(x, dt)


@pytest.fixture(scope="module", autouse=True)
def _threads(orc):
    orc.set_threads(8)


# ---- layout ---------------------------------------------------------------------------------

def test_permute_btfd_bftd_full_bitexact(orc, dev):
    say("permute bf16 [4,801,60,384] <-> [4,60,801,384]")
    x = inp(orc, (4, 801, 60, 384), SEED[4], 1, BF16)
    xd = to_dev(x, BF16)
    y = empty((4, 60, 801, 384), BF16)
    mbrt.strided_copy(xd.permute(0, 2, 1, 3), y)
    back = empty((4, 801, 60, 384), BF16)
    mbrt.strided_copy(y.permute(0, 2, 1, 3), back)
    torch.cuda.synchronize()
    assert_bitexact(to_host(y, BF16), np.ascontiguousarray(x.transpose(0, 2, 1, 3)), "permute")
    assert_bitexact(to_host(back, BF16), x, "permute round trip")


@pytest.mark.parametrize("dt", [F32, BF16, I64, I32, F16])
@pytest.mark.parametrize("perm,shape", [
    ((0, 2, 1, 3), (3, 17, 5, 24)),       # inner dim kept: row copies
    ((0, 2, 1, 3), (2, 9, 7, 3)),         # odd runs: narrow vectors
    ((1, 0), (67, 130)),                  # true transpose: LDS tiles
    ((0, 2, 1), (3, 70, 129)),            # batched transpose
    ((2, 1, 0), (5, 3, 4)),               # small: element path
    ((0, 2, 1, 3, 4), (2, 2, 9, 11, 2)),  # stft [B,S,F,T,2] -> [B,F,S,T,2]
])
def test_strided_copy_generic(orc, dev, dt, perm, shape):
    say(f"strided_copy dt={dt} perm={perm} shape={shape}")
    rng = np.random.default_rng(hash((dt, perm, shape)) % 2**32)
    npdt = {F32: np.float32, BF16: np.uint16, F16: np.uint16, I64: np.int64, I32: np.int32}[dt]
    x = rng.integers(0, 2**15, size=shape).astype(npdt)
    xd = to_dev(x, dt)
    v = xd.permute(*perm)
    y = empty(v.shape, dt)
    mbrt.strided_copy(v, y)
    torch.cuda.synchronize()
    assert_bitexact(to_host(y, dt), np.ascontiguousarray(x.transpose(perm)), "strided copy")


def test_strided_copy_sliced_views(orc, dev):
    say("strided_copy of sliced, offset views")
    x = orc.randn((8, 33, 20), seed=5)
    xd = to_dev(x, F32)
    for v, ref in [(xd[:, 1:30, 3:17], x[:, 1:30, 3:17]), (xd[2:7, :, 1:], x[2:7, :, 1:]),
                   (xd[:, ::2, :], x[:, ::2, :]), (xd.permute(2, 0, 1)[5:9], x.transpose(2, 0, 1)[5:9])]:
        y = empty(v.shape, F32)
        mbrt.strided_copy(v, y)
        torch.cuda.synchronize()
        assert_bitexact(to_host(y, F32), np.ascontiguousarray(ref), "sliced view")


def test_index_select_pad_cat(orc, dev):
    say("index_select / pad / cat")
    x = orc.randn((6, 50, 8), seed=6)
    xd = to_dev(x, F32)
    for idt in (I64, I32):
        idx = np.array([3, 0, 49, 7, 7, 12], dtype=np.int64 if idt == I64 else np.int32)
        out = empty((6, 6, 8), F32)
        mbrt.index_select(xd, 1, to_dev(idx, idt), out)
        torch.cuda.synchronize()
        assert_bitexact(to_host(out, F32), np.take(x, idx, axis=1), "index_select")
    for reflect in (False, True):
        out = empty((6, 50, 15), F32)
        mbrt.pad(xd, out, [0, 0, 4], value=2.5, reflect=reflect)
        torch.cuda.synchronize()
        ref = np.pad(x, ((0, 0), (0, 0), (4, 3)), mode="reflect") if reflect else \
            np.pad(x, ((0, 0), (0, 0), (4, 3)), constant_values=2.5)
        assert_bitexact(to_host(out, F32), ref, f"pad reflect={reflect}")
    parts = [orc.randn((4, n, 6), seed=60 + n) for n in (3, 1, 5)]
    out = empty((4, 9, 6), F32)
    mbrt.cat([to_dev(p, F32) for p in parts], 1, out)
    torch.cuda.synchronize()
    assert_bitexact(to_host(out, F32), np.concatenate(parts, axis=1), "cat")


# ---- element-wise ----------------------------------------------------------------------------

@pytest.mark.parametrize("n", [0, 1, 7, 8, 1000, 4099])
def test_fill_arange_convert(orc, dev, n):
    say(f"fill/arange/convert n={n}")
    for dt in (F32, BF16, F16, I64, I32):
        t = empty((n,), dt)
        mbrt.fill_(t, 3.25 if dt not in (I64, I32) else 7)
        torch.cuda.synchronize()
        want = {F32: 3.25, BF16: 3.25, F16: 3.25, I64: 7, I32: 7}[dt]
        assert np.all(to_host(t, dt) == (orc.from_f32(np.full(n, want, np.float32), dt) if dt in (BF16, F16) else want))
    for dt in (F32, I64, I32, F16):
        t = empty((n,), dt)
        mbrt.arange_(t, -3)
        torch.cuda.synchronize()
        ref = np.arange(-3, n - 3)
        ref = orc.from_f32(ref.astype(np.float32), dt) if dt in (F32, F16) else ref.astype(t.cpu().numpy().dtype)
        assert_bitexact(to_host(t, dt), ref, f"arange dt={dt}")
    x = orc.randn(n, seed=7, std=100.0)
    for sdt, ddt in [(F32, BF16), (BF16, F32), (F32, F16), (F16, F32), (BF16, F16), (F32, I64), (I64, F32),
                     (F32, I32), (I32, BF16)]:
        src = orc.convert(x, F32, sdt) if sdt != F32 else x
        out = empty((n,), ddt)
        mbrt.convert(to_dev(src, sdt), out)
        torch.cuda.synchronize()
        assert_bitexact(to_host(out, ddt), orc.convert(src, sdt, ddt), f"convert {sdt}->{ddt}")


def test_convert_bf16_specials(orc, dev):
    say("convert f32->bf16 special values and ties")
    u = np.array([0x7f7fffff, 0x7f7f8000, 0x7f7f7fff, 0x3f808000, 0x3f818000, 0x00008000, 0x80018000, 0x7f800000,
                  0xff800000, 0x00000001, 0x80000000, 0x3f800000], dtype=np.uint32)
    rng = np.random.default_rng(8)
    u = np.concatenate([u, (rng.integers(0, 2**16, 5000).astype(np.uint32) << 16) | 0x8000,
                        rng.integers(0, 2**32, 20000, dtype=np.uint64).astype(np.uint32)])
    f = u.view(np.float32)
    f = f[~np.isnan(f)]
    out = empty(f.shape, BF16)
    mbrt.convert(to_dev(f, F32), out)
    torch.cuda.synchronize()
    assert_bitexact(to_host(out, BF16), orc.f32_to_bf16(f), "f32->bf16 RNE")
    nan = np.array([np.nan, -np.nan], np.float32)
    out = empty((2,), BF16)
    mbrt.convert(to_dev(nan, F32), out)
    torch.cuda.synchronize()
    assert np.all(np.isnan(orc.bf16_to_f32(to_host(out, BF16))))


@pytest.mark.parametrize("dt", [F32, BF16, F16])
@pytest.mark.parametrize("n", [5, 4096, 100_003])
def test_binary_same_shape_bitexact(orc, dev, dt, n):
    say(f"binary dt={dt} n={n}")
    a = orc.from_f32(orc.randn(n, seed=9), dt)
    b = orc.from_f32(orc.randn(n, seed=10) + np.float32(4.0), dt)
    ad, bd = to_dev(a, dt), to_dev(b, dt)
    for op in range(4):
        out = empty((n,), dt)
        mbrt.binary(ad, bd, out, op)
        torch.cuda.synchronize()
        assert_bitexact(to_host(out, dt), orc.binary(a, b, dt, op), f"binary op {op}")
    # in place a += b (residual add) and an unaligned (offset) view: scalar path
    mbrt.binary(ad, bd, ad, 0)
    torch.cuda.synchronize()
    assert_bitexact(to_host(ad, dt), orc.binary(a, b, dt, 0), "in-place add")
    if n > 1:
        out = empty((n - 1,), dt)
        mbrt.binary(to_dev(a, dt)[1:], to_dev(b, dt)[1:], out, 2)
        torch.cuda.synchronize()
        assert_bitexact(to_host(out, dt), orc.binary(a[1:].copy(), b[1:].copy(), dt, 2), "unaligned mul")


def test_broadcast_and_scalar_ops(orc, dev):
    say("broadcast binary / scalar / unary")
    a = orc.randn((3, 1, 5, 7), seed=11)
    b = orc.randn((4, 1, 7), seed=12)
    out = empty((3, 4, 5, 7), F32)
    mbrt.binary_broadcast(to_dev(a, F32), to_dev(b, F32), out, mbrt.MUL)
    torch.cuda.synchronize()
    assert_bitexact(to_host(out, F32), a * b, "broadcast mul")
    x = orc.randn(1003, seed=13)
    for op, a_, b_, ref in [(mbrt.SCALAR_ADD, 1.5, 0, x + np.float32(1.5)), (mbrt.SCALAR_MUL, -0.25, 0, x * np.float32(-0.25)),
                            (mbrt.SCALAR_CLAMP, -0.5, 0.75, np.clip(x, -0.5, 0.75))]:
        t = to_dev(x, F32)
        mbrt.scalar_(t, op, a_, b_)
        torch.cuda.synchronize()
        assert_bitexact(to_host(t, F32), ref.astype(np.float32), f"scalar {op}")
    out = empty((1003,), F32)
    mbrt.unary(to_dev(x, F32), out, mbrt.UNARY_GT, 0.1)
    torch.cuda.synchronize()
    assert_bitexact(to_host(out, F32), (x > np.float32(0.1)).astype(np.float32), "gt")
    mbrt.unary(to_dev(x, F32), out, mbrt.UNARY_NEG)
    torch.cuda.synchronize()
    assert_bitexact(to_host(out, F32), -x, "neg")


def _bstrides(shape, strides, out_shape):
    """Element strides of an operand addressed at the broadcast output's coordinates
    (right-aligned; 0 on broadcast and missing dims)."""
    nd, k = len(out_shape), len(out_shape) - len(shape)
    return [0 if d < k or shape[d - k] == 1 else strides[d - k] for d in range(nd)]


# (a shape, b shape): size-1 middle dims on both sides, a missing leading dim, the bias-add shape
BCAST_CASES = [((3, 1, 5, 7), (4, 1, 7)), ((2, 6, 1, 9), (6, 8, 1)), ((48060, 384), (384,)), ((1,), (17, 3))]


@pytest.mark.parametrize("dt", [F32, BF16, F16])
@pytest.mark.parametrize("op", [0, 1, 2, 3])
def test_broadcast_binary_ops(orc, dev, dt, op):
    """Every op and dtype of the broadcast binary against the oracle on the same strides:
    out-of-place, with a strided (transposed) operand, and in place (a op= b)."""
    say(f"broadcast binary op={op} dt={dt}")
    for ci, (sa, sb) in enumerate(BCAST_CASES):
        a = orc.from_f32(orc.randn(sa, seed=70 + ci), dt)
        b = orc.from_f32(orc.randn(sb, seed=80 + ci) + np.float32(3.0 if op == 3 else 0.0), dt)
        out_shape = list(np.broadcast_shapes(sa, sb))
        out = empty(out_shape, dt)
        mbrt.binary_broadcast(to_dev(a, dt), to_dev(b, dt), out, op)
        torch.cuda.synchronize()
        ca = [int(x) for x in np.array(np.zeros(sa).strides) // 8]
        cb = [int(x) for x in np.array(np.zeros(sb).strides) // 8]
        ref = orc.binary_broadcast(a.reshape(-1), b.reshape(-1), dt, out_shape, _bstrides(sa, ca, out_shape),
                                   _bstrides(sb, cb, out_shape), op)
        assert_bitexact(to_host(out, dt), ref, f"broadcast op {op} case {ci}")
    # strided operand: a is the transposed view of a contiguous [7, 5] tensor
    base = orc.from_f32(orc.randn((7, 5), seed=90), dt)
    b = orc.from_f32(orc.randn((3, 1, 7), seed=91) + np.float32(3.0 if op == 3 else 0.0), dt)
    at = to_dev(base, dt).t()  # [5, 7], strides (1, 5)
    out = empty((3, 5, 7), dt)
    mbrt.binary_broadcast(at, to_dev(b, dt), out, op)
    torch.cuda.synchronize()
    ref = orc.binary_broadcast(base.reshape(-1), b.reshape(-1), dt, [3, 5, 7], [0, 1, 5], [7, 0, 1], op)
    assert_bitexact(to_host(out, dt), ref, f"broadcast op {op} strided operand")
    # in place: a [8, 5, 64] op= b [5, 1]
    a = orc.from_f32(orc.randn((8, 5, 64), seed=92), dt)
    b = orc.from_f32(orc.randn((5, 1), seed=93) + np.float32(3.0 if op == 3 else 0.0), dt)
    ad = to_dev(a, dt)
    mbrt.binary_broadcast(ad, to_dev(b, dt), ad, op)
    torch.cuda.synchronize()
    ref = orc.binary_broadcast(a.reshape(-1), b.reshape(-1), dt, [8, 5, 64], [320, 64, 1], [0, 1, 0], op)
    assert_bitexact(to_host(ad, dt), ref, f"broadcast op {op} in place")


def test_reductions(orc, dev):
    say("reductions")
    for shape in [(7, 801), (3, 5000), (100, 1)]:
        x = orc.randn(shape, seed=14)
        out = empty(shape[:-1], F32)
        mbrt.reduce_last(to_dev(x, F32), out, mbrt.REDUCE_SUM)
        torch.cuda.synchronize()
        assert_close(to_host(out, F32), orc.reduce_last(x, 0), F32, "sum last", den=np.abs(x).sum(-1))
        mbrt.reduce_last(to_dev(x, F32), out, mbrt.REDUCE_MAX)
        torch.cuda.synchronize()
        assert_bitexact(to_host(out, F32), x.max(-1), "max last")
    x = orc.randn((6, 33, 10), seed=15)
    for op in (0, 1):
        out = empty((6, 10), F32)
        mbrt.reduce_general(to_dev(x, F32), out, 1, op)
        torch.cuda.synchronize()
        assert_bitexact(to_host(out, F32), orc.reduce_general(x, 1, op), f"general reduce {op}")


# ---- normalisation ------------------------------------------------------------------------

def test_residual_rmsnorm_bl1_full(orc, dev):
    say("BL-1 residual + RMSNorm f32 [48060,384]")
    D = 384
    x = inp(orc, (48060, D), SEED[1], 1)
    r = inp(orc, (48060, D), SEED[1], 2)
    g = inp(orc, (D,), SEED[1], 3, mean=1.0, std=0.02)
    xd, rd, gd = to_dev(x, F32), to_dev(r, F32), to_dev(g, F32)
    s, y = empty((48060, D), F32), empty((48060, D), F32)
    mbrt.residual_add_rms_norm(xd, rd, gd, s, y, scale=float(np.sqrt(D)), eps=1e-8)
    torch.cuda.synchronize()
    ref_y, ref_s = orc.rms_norm(x, F32, g, F32, F32, float(np.sqrt(D)), 1e-8, res=r, sdt=F32, want_sum=True)
    assert_bitexact(to_host(s, F32), ref_s, "residual sum")
    err = assert_close(to_host(y, F32), ref_y, F32, "normed")
    print("BL-1 errors", err)
    # in place: residual <- residual + update
    mbrt.residual_add_rms_norm(xd, rd, gd, xd, y, scale=float(np.sqrt(D)), eps=1e-8)
    torch.cuda.synchronize()
    assert_bitexact(to_host(xd, F32), ref_s, "in-place residual")
    assert_close(to_host(y, F32), ref_y, F32, "in-place normed")


@pytest.mark.parametrize("D", [8, 96, 256, 384, 1024, 4096, 100, 5000])
@pytest.mark.parametrize("xdt,gdt,odt", [(F32, F32, F32), (BF16, F32, BF16), (BF16, BF16, BF16), (F32, F32, BF16),
                                         (F16, F32, F16), (BF16, F32, F32)])
def test_rmsnorm_shapes_dtypes(orc, dev, D, xdt, gdt, odt):
    say(f"rms_norm D={D} {xdt},{gdt}->{odt}")
    rows = 37
    x = inp(orc, (rows, D), 99, D, xdt)
    g = inp(orc, (D,), 98, D, gdt, mean=1.0, std=0.02)
    y = empty((rows, D), odt)
    mbrt.rms_norm(to_dev(x, xdt), to_dev(g, gdt), y, scale=float(np.sqrt(D)), eps=1e-12)
    torch.cuda.synchronize()
    assert_close(to_host(y, odt), orc.rms_norm(x, xdt, g, gdt, odt, float(np.sqrt(D)), 1e-12), odt, "rms")
    if xdt == BF16:  # bf16 residual path: the sum is rounded to bf16 before normalising
        r = inp(orc, (rows, D), 97, D, xdt)
        s, y = empty((rows, D), BF16), empty((rows, D), odt)
        mbrt.residual_add_rms_norm(to_dev(x, xdt), to_dev(r, xdt), to_dev(g, gdt), s, y, float(np.sqrt(D)), 1e-12)
        torch.cuda.synchronize()
        ry, rs = orc.rms_norm(x, xdt, g, gdt, odt, float(np.sqrt(D)), 1e-12, res=r, sdt=BF16, want_sum=True)
        assert_bitexact(to_host(s, BF16), rs, "bf16 residual sum")
        assert_close(to_host(y, odt), ry, odt, "bf16 residual normed")


# ---- activations ---------------------------------------------------------------------------

@pytest.mark.parametrize("act", [mbrt.ACT_GELU_REF, mbrt.ACT_GELU_STD])
def test_gelu_bl2a_full(orc, dev, act):
    say(f"BL-2a GELU act={act} bf16 [48060,1536]")
    x = inp(orc, (48060, 1536), SEED[2], 1, BF16, std=1.5)
    y = empty((48060, 1536), BF16)
    mbrt.bias_act(to_dev(x, BF16), None, y, act)
    torch.cuda.synchronize()
    err = assert_close(to_host(y, BF16), orc.bias_act(x, BF16, None, F32, BF16, act), BF16, "gelu")
    print("BL-2a errors", err)


@pytest.mark.parametrize("act", [0, 1, 2, 3, 4])
@pytest.mark.parametrize("xdt,odt", [(F32, F32), (BF16, BF16), (F32, BF16), (F16, F16)])
def test_bias_act(orc, dev, act, xdt, odt):
    say(f"bias_act act={act} {xdt}->{odt}")
    x = inp(orc, (129, 264), 21, act, xdt, std=2.0)
    b = inp(orc, (264,), 22, act)
    for bias in (None, b):
        y = empty((129, 264), odt)
        mbrt.bias_act(to_dev(x, xdt), to_dev(bias, F32) if bias is not None else None, y, act)
        torch.cuda.synchronize()
        assert_close(to_host(y, odt), orc.bias_act(x, xdt, bias, F32, odt, act), odt, f"act {act} bias={bias is not None}")
    xo = inp(orc, (1001,), 23, act, xdt)  # n % 8 != 0, no bias: vector body + tail
    y = empty((1001,), odt)
    mbrt.bias_act(to_dev(xo, xdt), None, y, act)
    torch.cuda.synchronize()
    assert_close(to_host(y, odt), orc.bias_act(xo, xdt, None, F32, odt, act), odt, "tail")


def test_glu_bl2b_full(orc, dev):
    say("BL-2b GLU bf16 [48060,3072]")
    x = inp(orc, (48060, 3072), SEED[2], 2, BF16, std=1.5)
    y = empty((48060, 1536), BF16)
    mbrt.glu(to_dev(x, BF16), y)
    torch.cuda.synchronize()
    print("BL-2b errors", assert_close(to_host(y, BF16), orc.glu(x, BF16, BF16), BF16, "glu"))


@pytest.mark.parametrize("half,xdt,odt", [(20, F32, F32), (7, BF16, BF16), (64, F32, BF16), (24, F16, F16)])
def test_glu_shapes(orc, dev, half, xdt, odt):
    say(f"glu half={half}")
    x = inp(orc, (33, 2 * half), 24, half, xdt, std=1.5)
    y = empty((33, half), odt)
    mbrt.glu(to_dev(x, xdt), y)
    torch.cuda.synchronize()
    assert_close(to_host(y, odt), orc.glu(x, xdt, odt), odt, "glu")


def test_gate_merge_bl2c_full(orc, dev):
    say("BL-2c sigmoid gate merge bf16 attn [60,8,801,64]")
    B, H, N, D = 60, 8, 801, 64
    attn = inp(orc, (B, H, N, D), SEED[2], 3, BF16)
    gate = inp(orc, (B, N, H), SEED[2], 4, BF16, std=2.0)
    y = empty((B, N, H * D), BF16)
    mbrt.gate_merge(to_dev(attn, BF16), to_dev(gate, BF16), y, mbrt.LAYOUT_BHND)
    torch.cuda.synchronize()
    ref = orc.gate_merge(attn, BF16, gate, BF16, BF16, B, H, N, D, layout=0)
    print("BL-2c errors", assert_close(to_host(y, BF16), ref, BF16, "gate merge"))
    attn_t = np.ascontiguousarray(attn.transpose(0, 2, 1, 3))
    mbrt.gate_merge(to_dev(attn_t, BF16), to_dev(gate, BF16), y, mbrt.LAYOUT_BNHD)
    torch.cuda.synchronize()
    assert_close(to_host(y, BF16), ref, BF16, "gate merge token-major")


@pytest.mark.parametrize("D,adt,gdt,odt,logit", [(64, F32, F32, F32, True), (12, BF16, F32, BF16, True),
                                                 (16, F32, BF16, F32, False), (64, F16, F16, F16, True)])
@pytest.mark.parametrize("B,N", [(3, 19), (4, 21)])
def test_gate_merge_variants(orc, dev, D, adt, gdt, odt, logit, B, N):
    """B*N = 57 takes the token-row order of the head-major input; B*N = 84, a multiple
    of 4, the order that walks 4 tokens x all heads per step."""
    say(f"gate merge D={D} B={B} N={N}")
    H = 4
    attn = inp(orc, (B, H, N, D), 25, D, adt)
    gate = inp(orc, (B, N, H), 26, D, gdt, std=2.0)
    y = empty((B, N, H * D), odt)
    mbrt.gate_merge(to_dev(attn, adt), to_dev(gate, gdt), y, mbrt.LAYOUT_BHND, gate_is_logit=logit)
    torch.cuda.synchronize()
    ref = orc.gate_merge(attn, adt, gate, gdt, odt, B, H, N, D, layout=0, logit=logit)
    assert_close(to_host(y, odt), ref, odt, "gate merge")


# ---- softmax -------------------------------------------------------------------------------

_bl3_cache = {}


def _bl3_input(orc, rows, cols):
    """The f32 draw of one BL-3 shape (308M values for the time shape), made once for both
    dtypes."""
    if (rows, cols) not in _bl3_cache:
        _bl3_cache.clear()
        _bl3_cache[(rows, cols)] = orc.randn((rows, cols), seed=SEED[3], stream=0, std=3.0)
    return _bl3_cache[(rows, cols)]


@pytest.mark.parametrize("dt", [F32, BF16])
@pytest.mark.parametrize("shape", [(480, 801, 801), (6408, 60, 60)])
def test_softmax_bl3_full(orc, dev, shape, dt):
    say(f"BL-3 softmax {shape} dt={dt}")
    rows, cols = shape[0] * shape[1], shape[2]
    # the configuration's own inputs: N(0, 3) from the BL-3 stream, rounded to the dtype
    x32 = _bl3_input(orc, rows, cols)
    x = to_dev(x32 if dt == F32 else orc.from_f32(x32, dt), dt)
    y = torch.empty_like(x)
    mbrt.softmax(x, y, 1.0)
    torch.cuda.synchronize()
    # every row sums to 1: f32 to 1e-5; bf16 to 2^-8, the unit roundoff (one RNE rounding
    # per element moves a row's sum by at most 2^-8 of it), plus the f32 sum's own error
    sums = y.float().sum(-1, dtype=torch.float64)
    tol = 1e-5 if dt == F32 else 2.0 ** -8 + 1e-5
    assert float((sums - 1).abs().max()) < tol
    # every row against the oracle, in chunks of rows (bounded host memory)
    chunk = max(1, (48 << 20) // cols)
    worst = {"max_rel": 0.0, "norm_rel": 0.0}
    for r0 in range(0, rows, chunk):
        xs, ys = to_host(x[r0:r0 + chunk], dt), to_host(y[r0:r0 + chunk], dt)
        e = assert_close(ys, orc.softmax(xs, dt, dt, 1.0), dt, f"softmax rows {r0}..")
        worst = {k: max(worst[k], e[k]) for k in worst}
    print("BL-3 errors (all rows)", worst)
    # in place (same dtype) gives identical bits
    mbrt.softmax(x, x, 1.0)
    torch.cuda.synchronize()
    assert torch.equal(x.view(torch.int16 if dt != F32 else torch.int32), y.view(torch.int16 if dt != F32 else torch.int32))


@pytest.mark.parametrize("cols", [1, 5, 8, 60, 63, 64, 65, 127, 801, 1301, 2048, 4096, 9000])
@pytest.mark.parametrize("idt,odt", [(F32, F32), (BF16, BF16), (F32, BF16), (BF16, F32), (F16, F16)])
def test_softmax_shapes(orc, dev, cols, idt, odt):
    say(f"softmax cols={cols} {idt}->{odt}")
    rows = 23
    x = inp(orc, (rows, cols), 31, cols, idt, std=3.0)
    y = empty((rows, cols), odt)
    mbrt.softmax(to_dev(x, idt), y, 0.125)
    torch.cuda.synchronize()
    assert_close(to_host(y, odt), orc.softmax(x, idt, odt, 0.125), odt, "softmax")


@pytest.mark.parametrize("rows,cols", [(1000, 16), (1000, 17), (1000, 32), (1000, 60), (1000, 100), (1000, 128),
                                       (2008, 60), (8, 60), (1000, 200), (96, 513), (1000, 801), (24, 801),
                                       (1000, 1024), (1001, 516), (7000, 516), (13001, 520)])
@pytest.mark.parametrize("idt,odt", [(F32, F32), (BF16, BF16), (F32, BF16), (BF16, F32), (F16, F16)])
def test_softmax_short_rows(orc, dev, rows, cols, idt, odt):
    """Row counts whose spans are whole 16-byte vectors (the LDS-staged path, up to 1024
    columns), with a partial last block (1001 and 13001 rows end in a one-row block), then
    the same call in place."""
    say(f"softmax short rows={rows} cols={cols} {idt}->{odt}")
    x = inp(orc, (rows, cols), 37, cols, idt, std=3.0)
    xd = to_dev(x, idt)
    y = empty((rows, cols), odt)
    mbrt.softmax(xd, y, 0.5)
    torch.cuda.synchronize()
    assert_close(to_host(y, odt), orc.softmax(x, idt, odt, 0.5), odt, "softmax short")
    if idt == odt:
        mbrt.softmax(xd, xd, 0.5)
        torch.cuda.synchronize()
        assert_bitexact(to_host(xd, odt), to_host(y, odt), "softmax short in place")


@pytest.mark.parametrize("cols", [36, 40, 44, 52, 56, 60, 64])
@pytest.mark.parametrize("rows", [2, 34, 1000, 6406])
@pytest.mark.parametrize("dt", [BF16, F16])
def test_softmax_row_pairs(orc, dev, rows, cols, dt):
    """Two-byte rows of 33..64 columns (a multiple of 4) in an even count: the register
    kernel that gives each pair of rows to 16 lanes, where a lane's 8 elements may straddle
    the two rows (cols = 4 mod 8).  Then the same call in place."""
    say(f"softmax row pairs rows={rows} cols={cols} dt={dt}")
    x = inp(orc, (rows, cols), 43, cols, dt, std=4.0)
    xd = to_dev(x, dt)
    y = empty((rows, cols), dt)
    mbrt.softmax(xd, y, 0.7)
    torch.cuda.synchronize()
    assert_close(to_host(y, dt), orc.softmax(x, dt, dt, 0.7), dt, "softmax row pairs")
    mbrt.softmax(xd, xd, 0.7)
    torch.cuda.synchronize()
    assert_bitexact(to_host(xd, dt), to_host(y, dt), "softmax row pairs in place")


@pytest.mark.parametrize("rows,cols", [(96, 801), (96, 60), (96, 16), (23, 801), (23, 60), (5, 3000), (96, 44)])
@pytest.mark.parametrize("dt", [F32, BF16])
def test_softmax_special_values(orc, dev, rows, cols, dt):
    """Masked scores on every softmax path (LDS-staged long and short rows, the unaligned
    rows kernel, the long-row loop): -inf entries get probability 0 and the row still sums
    to 1, a fully masked row and a row holding +inf become NaN, as in the oracle."""
    say(f"softmax special values rows={rows} cols={cols} dt={dt}")
    x = orc.to_f32(inp(orc, (rows, cols), 41, cols, dt, std=3.0), dt).copy()
    x[1, ::7] = -np.inf
    x[2, :] = -np.inf
    x[3, cols // 2] = np.inf
    x[4, : cols - 1] = -np.inf  # one live element: probability 1
    x = orc.from_f32(x, dt)
    xd = to_dev(x, dt)
    y = empty((rows, cols), dt)
    mbrt.softmax(xd, y, 0.5)
    torch.cuda.synchronize()
    want = orc.softmax(x, dt, dt, 0.5)
    got = to_host(y, dt)
    assert_close(got, want, dt, "softmax special values")
    g = orc.to_f32(got, dt)
    assert np.all(g[1, ::7] == 0.0) and abs(float(g[1].sum(dtype=np.float64)) - 1.0) < 1e-2
    assert np.isnan(g[2]).all() and np.isnan(g[3]).all()
    assert g[4, cols - 1] == 1.0
    mbrt.softmax(xd, xd, 0.5)
    torch.cuda.synchronize()
    assert_bitexact(to_host(xd, dt), got, "softmax special values in place")


# ---- rotary --------------------------------------------------------------------------------

def test_rotary_bl4a_full(orc, dev):
    say("BL-4a rotary bf16 q,k [480,801,64], f32 tables [801,32]")
    BH, N, D = 480, 801, 64
    q = inp(orc, (BH, N, D), SEED[4], 2, BF16)
    k = inp(orc, (BH, N, D), SEED[4], 3, BF16)
    cos, sin = orc.rotary_tables(N, D)
    qd, kd = to_dev(q, BF16), to_dev(k, BF16)
    mbrt.rotary_(qd, kd, to_dev(cos, F32), to_dev(sin, F32), mbrt.LAYOUT_BHND)
    torch.cuda.synchronize()
    rq, rk = orc.rotary(q, k, BF16, cos, sin, F32, N, 1, layout=0)
    print("BL-4a errors", assert_close(to_host(qd, BF16), rq, BF16, "rotary q"))
    assert_close(to_host(kd, BF16), rk, BF16, "rotary k")


@pytest.mark.parametrize("layout", [0, 1])
@pytest.mark.parametrize("dt,tdt,D", [(F32, F32, 64), (BF16, BF16, 64), (F32, F32, 6), (F16, F32, 32)])
def test_rotary_variants(orc, dev, layout, dt, tdt, D):
    say(f"rotary layout={layout} dt={dt} tdt={tdt} D={D}")
    B, H, N = 2, 3, 61
    shape = (B * H, N, D) if layout == 0 else (B, N, H, D)
    q = inp(orc, shape, 32, D, dt)
    cos, sin = orc.rotary_tables(N, D)
    if tdt == BF16:
        cos, sin = orc.f32_to_bf16(cos), orc.f32_to_bf16(sin)
    qd = to_dev(q, dt)
    mbrt.rotary_(qd, None, to_dev(cos, tdt), to_dev(sin, tdt), layout, heads=H)
    torch.cuda.synchronize()
    rq, _ = orc.rotary(q, None, dt, cos, sin, tdt, N, H, layout=layout)
    assert_close(to_host(qd, dt), rq, dt, "rotary", den=pair_den(orc.to_f32(q, dt)))


@pytest.mark.parametrize("N,out_n,idt,odt", [(60, 64, BF16, BF16), (801, 801, BF16, BF16), (17, 17, F32, F32),
                                             (60, 60, F32, BF16)])
def test_split_qkv_rotary(orc, dev, N, out_n, idt, odt):
    say(f"split_qkv N={N} out_n={out_n}")
    B, H, D = 2, 8, 64
    qkv = inp(orc, (B, N, 3 * H * D), 33, N, idt)
    cos, sin = orc.rotary_tables(N, D)
    q, k, v = (empty((B, H, out_n, D), odt) for _ in range(3))
    for t in (q, k, v):
        t.fill_(float("nan"))
    mbrt.split_qkv_rotary(to_dev(qkv, idt), to_dev(cos, F32), to_dev(sin, F32), q, k, v, H)
    torch.cuda.synchronize()
    rq, rk, rv = orc.split_qkv(qkv, idt, cos, sin, F32, odt, B, N, H, D, out_n)
    assert_close(to_host(q, odt), rq, odt, "q", den=pair_den(orc.to_f32(rq, odt)))
    assert_close(to_host(k, odt), rk, odt, "k", den=pair_den(orc.to_f32(rk, odt)))
    assert_bitexact(to_host(v, odt), rv, "v")


# ---- band split / merge ----------------------------------------------------------------------

def _bands(orc):
    return orc.mel_bands(44100.0, 2048, 60, 2)


@pytest.mark.parametrize("idt,odt", [(I32, F32), (I64, F32), (I32, BF16)])
def test_band_gather_bl5a_full(orc, dev, idt, odt):
    say(f"BL-5a band gather B=4 idx={idt} out={odt}")
    B, F, T = 4, 2050, 801
    mb = _bands(orc)
    stft = inp(orc, (B, F, T, 2), SEED[5], 1)
    idx = mb["freq_indices"].astype(np.int64 if idt == I64 else np.int32)
    out = empty((B, T, idx.size * 2), odt)
    mbrt.band_gather(to_dev(stft, F32), to_dev(idx, idt), out)
    torch.cuda.synchronize()
    ref = orc.band_gather(stft, mb["freq_indices"], odt, B, F, T)
    assert_bitexact(to_host(out, odt), ref, "gather")


# Ragged shapes and every length of the gather's persistent tile walk (1, 2, 3 and more
# tiles per block on a 256-CU device): random indices with repeats, every output dtype,
# two frames, and 16000 band-bins (250 band-bin tiles).
@pytest.mark.parametrize("B,F,T,J,idt,odt,seed", [
    (1, 2050, 801, 3958, I32, F32, 1),
    (3, 70, 1, 5, I32, F32, 2),
    (2, 300, 33, 64, I64, F16, 3),
    (5, 513, 130, 200, I32, BF16, 4),
    (16, 2050, 97, 3958, I32, F32, 5),
    (2, 100, 64, 1, I32, F32, 6),
    (8, 2050, 64, 3958, I64, F32, 7),
    (12, 2050, 64, 3958, I32, F32, 8),
    (1, 7, 200, 129, I32, F32, 9),
    (2, 300, 2, 100, I64, BF16, 10),
    (1, 500, 45, 16000, I32, F32, 11)])
def test_band_gather_shapes(orc, dev, B, F, T, J, idt, odt, seed):
    say(f"band gather B={B} F={F} T={T} J={J} idx={idt} out={odt}")
    rng = np.random.default_rng(seed)
    idx = rng.integers(0, F, size=J).astype(np.int64 if idt == I64 else np.int32)
    stft = inp(orc, (B, F, T, 2), 50 + seed, 0)
    out = empty((B, T, J * 2), odt)
    mbrt.band_gather(to_dev(stft, F32), to_dev(idx, idt), out)
    torch.cuda.synchronize()
    assert_bitexact(to_host(out, odt), orc.band_gather(stft, idx, odt, B, F, T), "gather")


# The gather starts every output run on a line of the output row, which depends on the
# output's address: outputs placed 1..15 complex values past an aligned address, with
# guard values around them that must stay untouched.
@pytest.mark.parametrize("B,F,T,J,idt,odt", [(2, 2050, 70, 3958, I32, F32), (1, 300, 33, 100, I64, F32),
                                             (3, 70, 5, 17, I32, BF16), (1, 513, 130, 200, I32, F16)])
@pytest.mark.parametrize("shift", [1, 3, 8, 15])
def test_band_gather_output_offsets(orc, dev, B, F, T, J, idt, odt, shift):
    say(f"band gather into an output {shift} complex values past alignment B={B} T={T} J={J} out={odt}")
    rng = np.random.default_rng(shift * 131 + J)
    idx = rng.integers(0, F, size=J).astype(np.int64 if idt == I64 else np.int32)
    stft = inp(orc, (B, F, T, 2), 70 + shift, 0)
    n = B * T * J * 2  # output scalars
    buf = empty((n + 64,), odt)
    buf.fill_(-3.0)
    out = buf[2 * shift: 2 * shift + n].view(B, T, J * 2)
    mbrt.band_gather(to_dev(stft, F32), to_dev(idx, idt), out)
    torch.cuda.synchronize()
    assert_bitexact(to_host(out, odt), orc.band_gather(stft, idx, odt, B, F, T), "gather at an offset")
    host = to_host(buf, odt)
    guard = to_host(torch.full((1,), -3.0, dtype=buf.dtype, device="cuda"), odt)[0]
    assert (host[:2 * shift] == guard).all() and (host[2 * shift + n:] == guard).all(), "gather wrote outside its output"


@pytest.mark.parametrize("idt", [I32, I64])
def test_band_gather_out_of_range_indices_clamp(orc, dev, idt):
    say(f"band gather with out-of-range indices idx={idt}")
    B, F, T = 2, 50, 70
    vals = [0, -1, -7, 49, 50, 51, 10**6, 3] + ([-(2**40), 2**40, 2**32 + 5] if idt == I64 else [-(2**31)])
    idx = np.array(vals * 9, dtype=np.int64 if idt == I64 else np.int32)
    stft = inp(orc, (B, F, T, 2), 60, 0)
    out = empty((B, T, idx.size * 2), F32)
    mbrt.band_gather(to_dev(stft, F32), to_dev(idx, idt), out)
    torch.cuda.synchronize()
    ref = np.take(stft, idx, axis=1, mode="clip").transpose(0, 2, 1, 3).reshape(B, T, -1)
    assert_bitexact(to_host(out, F32), np.ascontiguousarray(ref), "gather clamp")


def test_band_merge_bl5b_full(orc, dev):
    say("BL-5b mask merge B=4, 1 stem, f32")
    B, F, T = 4, 2050, 801
    mb = _bands(orc)
    J = mb["freq_indices"].size
    stft = inp(orc, (B, F, T, 2), SEED[5], 1)
    mask = inp(orc, (B, T, J * 2), SEED[5], 2, std=0.5)
    cnt = mb["bands_per_freq"].astype(np.float32)
    out = empty((B * 2, F // 2, T, 2), F32)
    sd = to_dev(stft, F32)
    offd, indd, cntd = to_dev(mb["csr_offsets"], I32), to_dev(mb["csr_indices"], I32), to_dev(cnt, F32)
    mbrt.band_mask_merge(sd, [to_dev(mask, F32)], offd, indd, cntd, out, 2)
    torch.cuda.synchronize()
    ref = orc.band_mask_merge(stft, [mask.reshape(B, T, J, 2)], F32, mb["csr_offsets"], mb["csr_indices"], cnt, F32, F32,
                              B, F, T, 2)
    den = merge_den(orc, stft, [mask], mb, B, F, T, 2)
    print("BL-5b errors", assert_close(to_host(out, F32), ref, F32, "merge", den=den))
    # gather then merge with mask 1+0j is the identity on every bin (bit-exact, counts 1 and 2)
    g = empty((B, T, J * 2), F32)
    mbrt.band_gather(sd, to_dev(mb["freq_indices"], I32), g)
    ones = torch.zeros((B, T, J, 2), device="cuda")
    ones[..., 0] = 1
    mbrt.band_mask_merge(sd, [ones.reshape(B, T, J * 2)], offd, indd, cntd, out, 2)
    torch.cuda.synchronize()
    ident = stft.reshape(B, F // 2, 2, T, 2).transpose(0, 2, 1, 3, 4).reshape(B * 2, F // 2, T, 2)
    assert_bitexact(to_host(out, F32), np.ascontiguousarray(ident), "merge(mask=1) identity")


@pytest.mark.parametrize("mdt,cdt,odt,S,idt", [(F32, F32, F32, 2, I32), (BF16, BF16, BF16, 2, I64),
                                               (BF16, F32, F32, 1, I32)])
def test_band_merge_variants(orc, dev, mdt, cdt, odt, S, idt):
    say(f"band merge mdt={mdt} cdt={cdt} odt={odt} S={S}")
    B, F, T = 2, 2050, 77
    mb = _bands(orc)
    J = mb["freq_indices"].size
    stft = inp(orc, (B, F, T, 2), 41, S)
    masks = [inp(orc, (B, T, J * 2), 42, s, mdt, std=0.5) for s in range(S)]
    cnt = orc.from_f32(mb["bands_per_freq"].astype(np.float32), cdt)
    out = empty((B * S * 2, F // 2, T, 2), odt)
    ity = np.int64 if idt == I64 else np.int32
    mbrt.band_mask_merge(to_dev(stft, F32), [to_dev(m, mdt) for m in masks], to_dev(mb["csr_offsets"].astype(ity), idt),
                         to_dev(mb["csr_indices"].astype(ity), idt), to_dev(cnt, cdt), out, 2)
    torch.cuda.synchronize()
    ref = orc.band_mask_merge(stft, [m.reshape(B, T, J, 2) for m in masks], mdt, mb["csr_offsets"], mb["csr_indices"],
                              cnt, cdt, odt, B, F, T, 2)
    den = merge_den(orc, stft, [orc.to_f32(m, mdt) for m in masks], mb, B, F, T, 2) if odt == F32 else None
    assert_close(to_host(out, odt), ref, odt, "merge", den=den)


def test_band_merge_many_bands_per_freq(orc, dev):
    say("band merge with up to 70 bands per freq (chunked CSR)")
    # synthetic layout: 3 wide overlapping "bands" over a few freqs -> long CSR lists
    B, F, T, C = 1, 40, 70, 1
    fi = np.concatenate([np.arange(0, 40), np.arange(5, 35), np.repeat(np.arange(10, 12), 35)]).astype(np.int32)
    J = fi.size
    by = [[] for _ in range(F)]
    for j, f in enumerate(fi):
        by[f].append(j)
    off = np.zeros(F + 1, np.int32)
    off[1:] = np.cumsum([len(b) for b in by])
    ind = np.array([j for b in by for j in b], np.int32)
    cnt = np.array([len(b) for b in by], np.float32)
    stft = inp(orc, (B, F, T, 2), 43, 0)
    mask = inp(orc, (B, T, J * 2), 43, 1)
    out = empty((B * C, F, T, 2), F32)
    mbrt.band_mask_merge(to_dev(stft, F32), [to_dev(mask, F32)], to_dev(off, I32), to_dev(ind, I32), to_dev(cnt, F32),
                         out, C)
    torch.cuda.synchronize()
    ref = orc.band_mask_merge(stft, [mask.reshape(B, T, J, 2)], F32, off, ind, cnt, F32, F32, B, F, T, C)
    mbd = dict(bands_per_freq=cnt.astype(np.int32), csr_offsets=off, csr_indices=ind)
    assert_close(to_host(out, F32), ref, F32, "merge chunked", den=merge_den(orc, stft, [mask], mbd, B, F, T, C))


def test_band_merge_freqs_without_bands(orc, dev):
    """Freqs that no band covers (count 0: nothing to sum, divided by max(count, 1e-8))
    give 0; with no band freqs at all (empty CSR, no index array) every output is 0."""
    say("band merge with uncovered freqs and with no band freqs")
    B, F, T, C = 2, 40, 70, 2
    fi = np.concatenate([np.arange(4, 20), np.arange(12, 30)]).astype(np.int32)  # freqs 0-3 and 30-39 uncovered
    J = fi.size
    by = [[] for _ in range(F)]
    for j, f in enumerate(fi):
        by[f].append(j)
    off = np.zeros(F + 1, np.int32)
    off[1:] = np.cumsum([len(b) for b in by])
    ind = np.array([j for b in by for j in b], np.int32)
    cnt = np.array([len(b) for b in by], np.float32)
    stft = inp(orc, (B, F, T, 2), 45, 0)
    mask = inp(orc, (B, T, J * 2), 45, 1)
    out = empty((B * C, F // C, T, 2), F32)
    mbrt.band_mask_merge(to_dev(stft, F32), [to_dev(mask, F32)], to_dev(off, I32), to_dev(ind, I32), to_dev(cnt, F32),
                         out, C)
    torch.cuda.synchronize()
    ref = orc.band_mask_merge(stft, [mask.reshape(B, T, J, 2)], F32, off, ind, cnt, F32, F32, B, F, T, C)
    got = to_host(out, F32)
    mbd = dict(bands_per_freq=cnt.astype(np.int32), csr_offsets=off, csr_indices=ind)
    assert_close(got, ref, F32, "merge with uncovered freqs", den=merge_den(orc, stft, [mask], mbd, B, F, T, C))
    per_freq = got.reshape(B, C, F // C, T, 2).transpose(0, 2, 1, 3, 4).reshape(B, F, T, 2)
    assert (per_freq[:, :4] == 0).all() and (per_freq[:, 30:] == 0).all()
    # no band freqs: the offsets are all 0, the index array is empty and no mask value is read
    out0 = empty((B * C, F // C, T, 2), F32)
    out0.fill_(7.0)
    mbrt.band_mask_merge(to_dev(stft, F32), [torch.zeros(2, device="cuda")], to_dev(np.zeros(F + 1, np.int32), I32),
                         torch.empty(0, dtype=torch.int32, device="cuda"), to_dev(np.zeros(F, np.float32), F32), out0, C)
    torch.cuda.synchronize()
    assert (to_host(out0, F32) == 0).all()


def test_zero_dc(orc, dev):
    say("zero_dc")
    for dt in (F32, BF16):
        x = inp(orc, (8, 1025, 33, 2), 44, dt, dt)
        xd = to_dev(x, dt)
        mbrt.zero_dc(xd)
        torch.cuda.synchronize()
        assert_bitexact(to_host(xd, dt), orc.zero_dc(x, dt), "zero_dc")


# ---- fused attention -------------------------------------------------------------------------

@pytest.mark.parametrize("BH,nq,nk", [(3, 1, 1), (3, 5, 5), (2, 60, 60), (2, 64, 64), (2, 65, 65), (2, 130, 130),
                                      (2, 801, 801), (2, 37, 200), (2, 200, 37),
                                      # 128-query workgroups whose last one holds 1 or 33 queries (its
                                      # other waves only load and sync), and one query or one key
                                      (2, 129, 129), (1, 161, 70), (2, 1, 801), (2, 801, 1),
                                      # keys in whole 64-key tiles only (every tile through the
                                      # buffer-resource loads, the last one too)
                                      (2, 100, 128), (1, 70, 768)])
@pytest.mark.parametrize("odt", [BF16, F32])
def test_attention_shapes(orc, dev, BH, nq, nk, odt):
    say(f"attention BH={BH} nq={nq} nk={nk} out={odt}")
    q = inp(orc, (BH, nq, 64), 0x4D425200A0, nq, BF16)
    k = inp(orc, (BH, nk, 64), 0x4D425200A1, nk, BF16)
    v = inp(orc, (BH, nk, 64), 0x4D425200A2, nk, BF16)
    out = empty((BH, nq, 64), odt)
    mbrt.attention(to_dev(q, BF16), to_dev(k, BF16), to_dev(v, BF16), out, 0.0)
    torch.cuda.synchronize()
    ref = orc.attention(q, k, v, BF16, odt, 0.0)
    # outputs are sums of p v of either sign: the magnitude they cancel from is sum p |v|
    den = orc.attention(orc.to_f32(q, BF16), orc.to_f32(k, BF16), np.abs(orc.to_f32(v, BF16)), F32, F32, 0.0)
    print("attention errors", assert_close(to_host(out, odt), ref, odt, "attention", den=den))


def _pmax_v(q, k, v, scale):
    """max_j p_ij |v_jd| for every (query i, d), p the exact softmax (double): the size of
    the largest single term of an output, i.e. what one bf16 step of one P moves it by
    / 2^-8."""
    qd, kd, vd = (np.asarray(t, np.float64) for t in (q, k, v))
    out = np.empty(qd.shape[:2] + (vd.shape[2],))
    for b in range(qd.shape[0]):  # one head at a time: [N, N_k, 64] doubles of temporaries
        s = (qd[b] @ kd[b].T) * (scale or 1.0 / 8.0)
        p = np.exp(s - s.max(-1, keepdims=True))
        p /= p.sum(-1, keepdims=True)
        out[b] = np.max(p[:, :, None] * np.abs(vd[b])[None, :, :], axis=1)
    return out


def _assert_ref_p(orc, y, q, k, v, odt, scale, what, fast=False, flips=2):
    """The reference-P attention against the oracle variant that restates its rounding.  The
    kernel's P (f32 exp2) and the oracle's (double exp) round to different bf16 neighbours
    only within a few f32 ulps of a rounding boundary; each such flip moves an output by at
    most 2^-8 of its largest term, so the elementwise bound is 2^-7 max_j p|v| (two flips)
    plus the f32 rule on sum p|v| (plus 1 ulp for bf16 outputs); norm-wise it is 2e-4
    (2e-3 for bf16 outputs, the usual rule).  Against exact attention it is within one
    bf16 rounding of every P: norm-wise 2^-8."""
    qf, kf, vf = (orc.to_f32(t, BF16) for t in (q, k, v))
    if fast:  # the fast mode's rounding: lazy running max, row sum over the rounded P
        ref = orc.attention_ref_p(q, k, v, BF16, odt, scale, lazy=orc.ATTN_FAST_LAZY, sum_rounded=True)
    else:
        ref = orc.attention_ref_p(q, k, v, BF16, odt, scale)
    den = orc.attention(qf, kf, np.abs(vf), F32, F32, scale).astype(np.float64)
    pm = _pmax_v(qf, kf, vf, scale)
    a, b = orc.to_f32(y, odt).astype(np.float64), orc.to_f32(ref, odt).astype(np.float64)
    bound = flips * 2.0 ** -8 * pm + 1e-5 * den
    if odt == BF16:
        bound = bound + 2.0 ** (np.floor(np.log2(np.maximum(np.abs(b), 1e-30))) - 7)
    excess = np.abs(a - b) - bound
    worst = np.unravel_index(np.argmax(excess), excess.shape)
    assert excess[worst] <= 0, f"{what}: {a[worst]} vs {b[worst]} (bound {bound[worst]:.3e})"
    norm = np.linalg.norm(a - b) / np.linalg.norm(b)
    assert norm <= (2e-3 if odt == BF16 else 2e-4), f"{what}: norm-wise {norm:.3e}"
    exact = orc.attention(q, k, v, BF16, F32, scale).astype(np.float64)
    assert np.linalg.norm(a - exact) / np.linalg.norm(exact) <= 2.0 ** -8, f"{what}: vs exact attention"
    return norm


@pytest.mark.parametrize("BH,nq,nk", [(3, 1, 1), (2, 65, 65), (2, 801, 801), (2, 37, 200), (2, 129, 129),
                                      (2, 801, 1), (1, 161, 70), (2, 64, 64), (2, 96, 128)])
@pytest.mark.parametrize("odt", [BF16, F32])
def test_attention_p_bf16(orc, dev, BH, nq, nk, odt):
    say(f"attention P-bf16 BH={BH} nq={nq} nk={nk} out={odt}")
    q = inp(orc, (BH, nq, 64), 0x4D425200B0, nq, BF16)
    k = inp(orc, (BH, nk, 64), 0x4D425200B1, nk, BF16)
    v = inp(orc, (BH, nk, 64), 0x4D425200B2, nk, BF16)
    out = empty((BH, nq, 64), odt)
    mbrt.attention(to_dev(q, BF16), to_dev(k, BF16), to_dev(v, BF16), out, 0.0, p_bf16=True)
    torch.cuda.synchronize()
    print("P-bf16 norm-wise", _assert_ref_p(orc, to_host(out, odt), q, k, v, odt, 0.0, "attention P-bf16"))


def test_attention_p_bf16_known_answer(orc, dev):
    """v = 1: out = sum bf16(p) / sum p per query, not 1 (the reference rounds P but not the
    row sum); the oracle variant is pinned to that ratio on the CPU."""
    say("attention P-bf16 with v = 1")
    BH, nq, nk = 2, 40, 300
    q = inp(orc, (BH, nq, 64), 0x4D425200B3, 0, BF16, std=2.0)
    k = inp(orc, (BH, nk, 64), 0x4D425200B4, 0, BF16)
    v = orc.from_f32(np.ones((BH, nk, 64), np.float32), BF16)
    out = empty((BH, nq, 64), F32)
    mbrt.attention(to_dev(q, BF16), to_dev(k, BF16), to_dev(v, BF16), out, 0.125, p_bf16=True)
    torch.cuda.synchronize()
    y = to_host(out, F32)
    ref = orc.attention_ref_p(q, k, v, BF16, F32, 0.125)
    assert np.abs(ref - 1).max() > 1e-5
    assert np.abs(y - ref).max() <= 2.0 ** -7 / nk * 8 + 1e-6


@pytest.mark.parametrize("BH,nq,nk", [(3, 1, 1), (2, 65, 65), (2, 801, 801), (2, 37, 200), (2, 129, 129),
                                      (2, 801, 1), (1, 161, 70), (2, 300, 700), (2, 64, 64), (2, 96, 128)])
@pytest.mark.parametrize("odt", [BF16, F32])
def test_attention_p_bf16_fast(orc, dev, BH, nq, nk, odt):
    say(f"attention P-bf16 fast BH={BH} nq={nq} nk={nk} out={odt}")
    q = inp(orc, (BH, nq, 64), 0x4D425200C0, nq, BF16, std=1.5)
    k = inp(orc, (BH, nk, 64), 0x4D425200C1, nk, BF16)
    v = inp(orc, (BH, nk, 64), 0x4D425200C2, nk, BF16)
    if nk >= 700:
        # keys aligned with the queries far down the sequence: the running max has to move
        kq = orc.to_f32(k, BF16)
        kq[:, nk - 100:nk - 100 + min(nq, 100)] = 0.6 * orc.to_f32(q, BF16)[:, :min(nq, 100)]
        k = orc.from_f32(kq, BF16)
    out = empty((BH, nq, 64), odt)
    mbrt.attention(to_dev(q, BF16), to_dev(k, BF16), to_dev(v, BF16), out, 0.0, p_precision=mbrt.ATTN_P_BF16_FAST)
    torch.cuda.synchronize()
    print("P-bf16 fast norm-wise", _assert_ref_p(orc, to_host(out, odt), q, k, v, odt, 0.0, "attention P-bf16 fast",
                                                 fast=True))


# Heads of at most 64 queries and 64 keys run on persistent workgroups, each
# walking heads with the next head's K, V and Q loading while it computes: more heads than
# workgroups, waves without queries (n_q <= 48), one query, one key, every P precision.
@pytest.mark.parametrize("BH,nq,nk", [(2000, 60, 60), (1601, 17, 64), (1000, 64, 5), (900, 1, 33), (777, 33, 1)])
@pytest.mark.parametrize("pm", [mbrt.ATTN_P_PAIR, mbrt.ATTN_P_BF16, mbrt.ATTN_P_BF16_FAST])
@pytest.mark.parametrize("odt", [BF16, F32])
def test_attention_short_heads_persistent(orc, dev, BH, nq, nk, pm, odt):
    say(f"attention persistent heads BH={BH} nq={nq} nk={nk} pm={pm} out={odt}")
    q = inp(orc, (BH, nq, 64), 0x4D425200D0, nq, BF16, std=1.5)
    k = inp(orc, (BH, nk, 64), 0x4D425200D1, nk, BF16)
    v = inp(orc, (BH, nk, 64), 0x4D425200D2, nk, BF16)
    out = empty((BH, nq, 64), odt)
    mbrt.attention(to_dev(q, BF16), to_dev(k, BF16), to_dev(v, BF16), out, 0.125, p_precision=pm)
    torch.cuda.synchronize()
    y = to_host(out, odt)
    if pm == mbrt.ATTN_P_PAIR:
        ref = orc.attention(q, k, v, BF16, odt, 0.125)
        den = orc.attention(orc.to_f32(q, BF16), orc.to_f32(k, BF16), np.abs(orc.to_f32(v, BF16)), F32, F32, 0.125)
        # the pair hi + lo holds each P to 2^-15 of itself (hi is P truncated to bf16, lo the
        # rest rounded to bf16), so with a handful of keys and one P dominating, an f32
        # output can miss the 1e-5 rule by that much: the bound here is 2^-15 of sum p|v|
        assert_close(y, ref, odt, "attention persistent", den=den, rtol=2.0 ** -15 if odt == F32 else None)
    else:
        # millions of outputs: a row where three or four P round to the other bf16 neighbour
        # than in the oracle turns up, so four flips of the largest term are allowed
        _assert_ref_p(orc, y, q, k, v, odt, 0.125, "attention persistent", fast=pm == mbrt.ATTN_P_BF16_FAST,
                      flips=4)


def test_attention_p_bf16_fast_known_answer(orc, dev):
    """v = 1: the output and the row sum add the same rounded P in the same order, so every
    output is 1 up to the final division (one f32 rounding)."""
    say("attention P-bf16 fast with v = 1")
    BH, nq, nk = 2, 40, 300
    q = inp(orc, (BH, nq, 64), 0x4D425200C3, 0, BF16, std=2.0)
    k = inp(orc, (BH, nk, 64), 0x4D425200C4, 0, BF16)
    v = orc.from_f32(np.ones((BH, nk, 64), np.float32), BF16)
    out = empty((BH, nq, 64), F32)
    mbrt.attention(to_dev(q, BF16), to_dev(k, BF16), to_dev(v, BF16), out, 0.125, p_precision=mbrt.ATTN_P_BF16_FAST)
    torch.cuda.synchronize()
    assert np.abs(to_host(out, F32) - 1.0).max() <= 2.0 ** -23


def test_attention_p_bf16_fast_full_time_shape(orc, dev):
    """The time attention [480, 801, 64] in the fast bf16-P mode; every query of a sample
    of heads against the oracle variant."""
    say("attention P-bf16 fast full BH=480 N=801")
    BH, N = 480, 801
    g = torch.Generator(device="cuda").manual_seed(SEED[3] + 9)
    q, k, v = (torch.randn((BH, N, 64), generator=g, device="cuda").to(torch.bfloat16) for _ in range(3))
    out = torch.empty((BH, N, 64), dtype=torch.bfloat16, device="cuda")
    mbrt.attention(q, k, v, out, 0.125, p_precision=mbrt.ATTN_P_BF16_FAST)
    torch.cuda.synchronize()
    sel = torch.tensor(sorted(np.random.default_rng(7).choice(BH, 8, replace=False)), device="cuda")
    qs, ks, vs = (to_host(t[sel], BF16) for t in (q, k, v))
    _assert_ref_p(orc, to_host(out[sel], BF16), qs, ks, vs, BF16, 0.125, "attention P-bf16 fast full", fast=True)


def test_attention_p_bf16_full_time_shape(orc, dev):
    """The time attention [480, 801, 64] in the reference's arithmetic; every query of a
    sample of heads against the oracle variant."""
    say("attention P-bf16 full BH=480 N=801")
    BH, N = 480, 801
    g = torch.Generator(device="cuda").manual_seed(SEED[3] + 7)
    q, k, v = (torch.randn((BH, N, 64), generator=g, device="cuda").to(torch.bfloat16) for _ in range(3))
    out = torch.empty((BH, N, 64), dtype=torch.bfloat16, device="cuda")
    mbrt.attention(q, k, v, out, 0.125, p_bf16=True)
    torch.cuda.synchronize()
    sel = torch.tensor(sorted(np.random.default_rng(6).choice(BH, 8, replace=False)), device="cuda")
    qs, ks, vs = (to_host(t[sel], BF16) for t in (q, k, v))
    _assert_ref_p(orc, to_host(out[sel], BF16), qs, ks, vs, BF16, 0.125, "attention P-bf16 full")


@pytest.mark.parametrize("BH,N,scale", [(480, 801, 0.125), (6408, 60, 0.125)])
def test_attention_full_shapes(orc, dev, BH, N, scale):
    """Time (480 heads x 801) and frequency (6408 x 60) attention at full chunk shape: every
    query of every head against the oracle."""
    say(f"attention full BH={BH} N={N}")
    g = torch.Generator(device="cuda").manual_seed(SEED[3] + N)
    q, k, v = (torch.randn((BH, N, 64), generator=g, device="cuda").to(torch.bfloat16) for _ in range(3))
    out = torch.empty((BH, N, 64), dtype=torch.bfloat16, device="cuda")
    mbrt.attention(q, k, v, out, scale)
    torch.cuda.synchronize()
    qs, ks, vs, ys = (to_host(t, BF16) for t in (q, k, v, out))
    ref = orc.attention(qs, ks, vs, BF16, BF16, scale)
    den = orc.attention(orc.to_f32(qs, BF16), orc.to_f32(ks, BF16), np.abs(orc.to_f32(vs, BF16)), F32, F32, scale)
    print("attention full errors", assert_close(ys, ref, BF16, "attention", den=den))


# Attention over [B, N, H, 64] views of a fused qkv projection, with the in-kernel q rotary
# (the reference's split-contig _q_rotary form) and the gated head-merge epilogue: bit for
# bit the separate GPU ops (rotary, attention, gate merge), and close to the oracle chain.
@pytest.mark.parametrize("B,N,H,rot,gate,odt,tdt", [
    (2, 801, 8, False, False, BF16, F32),
    (2, 801, 8, True, False, BF16, F32),
    (2, 70, 3, True, True, BF16, BF16),
    (1, 60, 4, False, True, F32, F32),
    (3, 130, 2, True, True, F32, F32),
])
def test_attention_bnhd_fusions(orc, dev, B, N, H, rot, gate, odt, tdt):
    say(f"attention_bnhd B={B} N={N} H={H} rot={rot} gate={gate} out={odt} trig={tdt}")
    tdt_torch = {F32: torch.float32, BF16: torch.bfloat16}
    qkv = to_dev(inp(orc, (B, N, 3 * H * 64), 0x4D425200A3, N + H, BF16), BF16)
    v5 = qkv.view(B, N, 3, H, 64)
    q, k, v = v5[:, :, 0], v5[:, :, 1], v5[:, :, 2]  # strided views, read in place
    cos_h, sin_h = orc.rotary_tables(N, 64)
    if tdt == BF16:
        cos_h, sin_h = orc.from_f32(cos_h, BF16), orc.from_f32(sin_h, BF16)
    cos, sin = to_dev(cos_h, tdt), to_dev(sin_h, tdt)
    g_h = inp(orc, (B, N, H), 0x4D425200A4, N, BF16, std=2.0)
    g = to_dev(g_h, BF16)
    fused = mbrt.attention_bnhd(q, k, v, cos=cos if rot else None, sin=sin if rot else None,
                                gate=g if gate else None, out_dtype=tdt_torch[F32] if odt == F32 else torch.bfloat16)
    # the separate ops on contiguous heads
    qc, kc, vc = (t.permute(0, 2, 1, 3).contiguous().view(B * H, N, 64) for t in (q, k, v))
    if rot:
        mbrt.rotary_(qc, None, cos, sin)
    att = empty((B, H, N, 64), odt)
    mbrt.attention(qc, kc, vc, att.view(B * H, N, 64), 0.0)
    sep = att
    if gate:
        sep = empty((B, N, H * 64), odt)
        mbrt.gate_merge(att, g, sep)
    torch.cuda.synchronize()
    assert tuple(fused.shape) == tuple(sep.shape)
    assert_bitexact(to_host(fused, odt), to_host(sep, odt), "attention_bnhd = separate ops")
    # each stage against the oracle: the attention on the rotated q the rotary op produced
    # (that op is pinned to the oracle itself), then the gate on that attention output (the
    # two roundings of a chain may add up past one ulp of the final value)
    qh, kh, vh = (to_host(t, BF16) for t in (qc, kc, vc))
    ref = orc.attention(qh, kh, vh, BF16, odt, 0.0).reshape(B, H, N, 64)
    den = orc.attention(orc.to_f32(qh, BF16), orc.to_f32(kh, BF16), np.abs(orc.to_f32(vh, BF16)), F32, F32,
                        0.0).reshape(B, H, N, 64)
    print("attention_bnhd errors", assert_close(to_host(att, odt), ref, odt, "attention_bnhd attention", den=den))
    if gate:
        gref = orc.gate_merge(to_host(att, odt), odt, g_h, BF16, odt, B, H, N, 64)
        assert_close(to_host(fused, odt), gref, odt, "attention_bnhd gate merge")


@pytest.mark.parametrize("fast", [False, True])
def test_attention_bnhd_p_bf16_fusion(orc, dev, fast):
    """The reference's split-contig q-rotary time attention with the gate, in the
    reference's P arithmetic (and in the fast bf16-P mode): bit for bit rotary ->
    attention -> gate merge."""
    say(f"attention_bnhd P-bf16 rot+gate fast={fast}")
    pm = mbrt.ATTN_P_BF16_FAST if fast else mbrt.ATTN_P_BF16
    B, N, H = 2, 801, 8
    qkv = to_dev(inp(orc, (B, N, 3 * H * 64), 0x4D425200B5, 0, BF16), BF16)
    v5 = qkv.view(B, N, 3, H, 64)
    q, k, v = v5[:, :, 0], v5[:, :, 1], v5[:, :, 2]
    cos_h, sin_h = orc.rotary_tables(N, 64)
    cos, sin = to_dev(cos_h, F32), to_dev(sin_h, F32)
    g = to_dev(inp(orc, (B, N, H), 0x4D425200B6, 0, BF16, std=2.0), BF16)
    fused = mbrt.attention_bnhd(q, k, v, cos=cos, sin=sin, gate=g, p_precision=pm)
    qc, kc, vc = (t.permute(0, 2, 1, 3).contiguous().view(B * H, N, 64) for t in (q, k, v))
    mbrt.rotary_(qc, None, cos, sin)
    att = empty((B, H, N, 64), BF16)
    mbrt.attention(qc, kc, vc, att.view(B * H, N, 64), 0.0, p_precision=pm)
    sep = empty((B, N, H * 64), BF16)
    mbrt.gate_merge(att, g, sep)
    torch.cuda.synchronize()
    assert_bitexact(to_host(fused, BF16), to_host(sep, BF16), "attention_bnhd P-bf16 = separate ops")
    qh, kh, vh = (to_host(t[:2], BF16) for t in (qc, kc, vc))
    _assert_ref_p(orc, to_host(att.view(B * H, N, 64)[:2], BF16), qh, kh, vh, BF16, 0.0, "bnhd P-bf16 attention",
                  fast=fast)


@pytest.mark.parametrize("gdt,logit,odt", [(F32, True, BF16), (F16, True, F32), (BF16, False, BF16),
                                           (F32, False, F32)])
def test_attention_bnhd_gate_forms(orc, dev, gdt, logit, odt):
    """The gated epilogue for every gate dtype, as logits or as probabilities, with a
    non-default scale: bit for bit attention followed by the separate gate merge."""
    say(f"attention_bnhd gate dtype={gdt} logit={logit} out={odt}")
    B, N, H, scale = 2, 97, 3, 0.3
    qkv = to_dev(inp(orc, (B, N, 3 * H * 64), 0x4D425200A5, N, BF16), BF16)
    v5 = qkv.view(B, N, 3, H, 64)
    q, k, v = v5[:, :, 0], v5[:, :, 1], v5[:, :, 2]
    g_h = inp(orc, (B, N, H), 0x4D425200A6, N, gdt, std=2.0)
    if not logit:   # probabilities in [0, 1]
        g_h = orc.from_f32(np.abs(orc.to_f32(g_h, gdt)) / 6.0, gdt) if gdt != F32 else np.abs(g_h) / np.float32(6.0)
    g = to_dev(g_h, gdt)
    fused = mbrt.attention_bnhd(q, k, v, scale=scale, gate=g, gate_is_logit=logit,
                                out_dtype=torch.float32 if odt == F32 else torch.bfloat16)
    qc, kc, vc = (t.permute(0, 2, 1, 3).contiguous().view(B * H, N, 64) for t in (q, k, v))
    att = empty((B, H, N, 64), odt)
    mbrt.attention(qc, kc, vc, att.view(B * H, N, 64), scale)
    sep = empty((B, N, H * 64), odt)
    mbrt.gate_merge(att, g, sep, mbrt.LAYOUT_BHND, gate_is_logit=logit)
    torch.cuda.synchronize()
    assert_bitexact(to_host(fused, odt), to_host(sep, odt), "gated attention_bnhd = attention + gate merge")
    gref = orc.gate_merge(to_host(att, odt), odt, g_h, gdt, odt, B, H, N, 64, layout=0, logit=logit)
    assert_close(to_host(fused, odt), gref, odt, "gated attention_bnhd gate stage")


def test_attention_bnhd_rejects_bad_strides(dev):
    t = torch.zeros((1, 16, 1, 68), dtype=torch.bfloat16, device="cuda")
    q = t[..., :64]  # rows 68 elements apart: not 16-byte pieces
    with pytest.raises(mbrt.MbrtError):
        mbrt.attention_bnhd(q, q, q)
    ok = torch.zeros((1, 16, 1, 64), dtype=torch.bfloat16, device="cuda")
    cos = torch.zeros((16, 32), device="cuda")
    with pytest.raises(mbrt.MbrtError):
        mbrt.attention_bnhd(ok, ok, ok, cos=cos, sin=None)  # cos without sin


def test_attention_rejects_bad_arguments(dev):
    q = torch.zeros((2, 8, 32), dtype=torch.bfloat16, device="cuda")
    out = torch.empty_like(q)
    with pytest.raises(mbrt.MbrtError):
        mbrt.attention(q, q, q, out)  # head_dim 32 is not built
    q64 = torch.zeros((2, 8, 64), dtype=torch.float32, device="cuda")
    with pytest.raises(mbrt.MbrtError):
        mbrt.attention(q64, q64, q64, torch.empty_like(q64))  # f32 inputs
    qb = q64.to(torch.bfloat16)
    with pytest.raises(mbrt.MbrtError):
        mbrt.attention(qb, qb, qb, torch.empty_like(qb), -0.5)  # negative scale
