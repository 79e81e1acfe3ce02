"""Parity rules shared by the tests.

* Integer / byte / index work and pure copies: bit-exact.
* f32 outputs: max_i |y_i - yhat_i| / max(|yhat_i|, tau) <= 1e-5, tau = 1e-3 * RMS(yhat),
  where yhat is the oracle's double-precision value rounded once to f32.  For outputs
  that are sums or differences of products (rotary pairs, complex mask products,
  reductions) the denominator also includes the magnitude of those terms (`den`).
* bf16 / f16 outputs: one correct rounding alone can move a value by 2^-8 (bf16), which
  exceeds 2e-3, so the rule compares against yhat = the double-precision value rounded
  once to the output format: |y_i - yhat_i| <= 1 ulp(max(|yhat_i|, tau)) elementwise,
  and ||y - yhat||_2 / ||yhat||_2 <= 2e-3 norm-wise.
NaN positions must agree; infinities must agree exactly.
"""
from __future__ import annotations

import numpy as np

F32, F16, I64, BF16, I32 = 0, 1, 2, 3, 4

RTOL_F32 = 1e-5
NORM_RTOL_LOWP = 2e-3
TAU_REL = 1e-3


def _f32(a: np.ndarray, dt: int) -> np.ndarray:
    if dt == F32:
        return np.asarray(a, dtype=np.float32).astype(np.float64)
    if dt == BF16:
        return (np.asarray(a, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    if dt == F16:
        return np.asarray(a, dtype=np.uint16).view(np.float16).astype(np.float64)
    raise ValueError(dt)


def _check_specials(y: np.ndarray, yh: np.ndarray, what: str) -> np.ndarray | None:
    """Mask of the finite positions after checking that NaNs and infinities agree; None
    when every element of both is finite (the common case, which skips the masking)."""
    if np.isfinite(y).all() and np.isfinite(yh).all():
        return None
    ny, nh = np.isnan(y), np.isnan(yh)
    assert np.array_equal(ny, nh), f"{what}: NaN positions differ ({int((ny != nh).sum())} elements)"
    iy, ih = np.isinf(y), np.isinf(yh)
    assert np.array_equal(iy, ih) and np.array_equal(y[iy], yh[ih]), f"{what}: infinities differ"
    return ~(ny | iy)


def assert_bitexact(y: np.ndarray, yhat: np.ndarray, what: str = "") -> None:
    y = np.ascontiguousarray(y)
    yhat = np.ascontiguousarray(yhat)
    assert y.shape == yhat.shape, f"{what}: shape {y.shape} != {yhat.shape}"
    assert y.dtype.itemsize == yhat.dtype.itemsize, f"{what}: element sizes differ"
    if y.size == 0:
        return
    fy, fh = y.reshape(-1), yhat.reshape(-1)
    by, bh = fy.view(np.uint8).reshape(fy.size, -1), fh.view(np.uint8).reshape(fh.size, -1)
    diff = np.nonzero((by != bh).any(axis=1))[0]
    if diff.size:
        raise AssertionError(f"{what}: {diff.size} of {fy.size} elements differ; first at {diff[:5]}: "
                             f"{fy[diff[:5]]} vs {fh[diff[:5]]}")


def rel_errors(y: np.ndarray, yhat: np.ndarray, dt: int) -> tuple[float, float]:
    """(max elementwise error relative to max(|yhat|, tau), norm-wise relative error)."""
    a, b = _f32(y, dt).reshape(-1), _f32(yhat, dt).reshape(-1)
    ok = np.isfinite(a) & np.isfinite(b)
    a, b = a[ok], b[ok]
    if b.size == 0:
        return 0.0, 0.0
    tau = TAU_REL * float(np.sqrt(np.mean(b * b)))
    den = np.maximum(np.abs(b), tau if tau > 0 else 1e-30)
    elem = float(np.max(np.abs(a - b) / den))
    nb = float(np.linalg.norm(b))
    norm = float(np.linalg.norm(a - b) / nb) if nb > 0 else float(np.linalg.norm(a - b))
    return elem, norm


def _ulp(x: np.ndarray, dt: int) -> np.ndarray:
    p, emin = (8, -126) if dt == BF16 else (11, -14)
    ax = np.maximum(np.abs(x), np.finfo(np.float64).tiny)
    _, e = np.frexp(ax)  # ax = m 2^e, m in [0.5, 1): floor(log2 ax) = e - 1
    e = np.maximum(e - 1, emin)
    return np.ldexp(1.0, e - (p - 1))


def assert_close(y: np.ndarray, yhat: np.ndarray, dt: int, what: str = "", rtol: float | None = None,
                 den: np.ndarray | None = None) -> dict:
    """Apply the rule for output dtype `dt` (F32 / BF16 / F16); returns the measured errors.

    `den`: per-element magnitude of the terms that the exact result is a sum or
    difference of, for ops whose outputs cancel (rotations, complex products, reductions,
    attention's sum of p v).  The f32 error is then measured relative to
    max(|yhat|, den, tau): an f32 evaluation of a - b carries ~2^-24 (|a| + |b|) absolute
    error however small a - b is, in the reference's kernels as in these.  For bf16/f16
    outputs the elementwise bound becomes 1 ulp(max(|yhat|, tau)) + 1e-5 den: the output
    rounding plus the f32 rule on the cancelled magnitude.
    """
    assert y.shape == yhat.shape, f"{what}: shape {y.shape} != {yhat.shape}"
    a, b = _f32(y, dt), _f32(yhat, dt)
    ok = _check_specials(a, b, what)
    a, b = (a.reshape(-1), b.reshape(-1)) if ok is None else (a[ok], b[ok])
    if den is not None:
        den = np.asarray(den, np.float64).reshape(-1)
        den = (den if ok is None else den[ok.reshape(-1)]).reshape(b.shape)
    if b.size == 0:
        return {"max_rel": 0.0, "norm_rel": 0.0}
    tau = TAU_REL * float(np.sqrt(np.mean(b * b)))
    if dt == F32:
        tol = RTOL_F32 if rtol is None else rtol
        den = np.maximum(np.abs(b), tau if tau > 0 else 1e-30) if den is None else \
            np.maximum(np.maximum(np.abs(b), den), tau if tau > 0 else 1e-30)
        err = np.abs(a - b) / den
        worst = int(np.argmax(err))
        assert err[worst] <= tol, (f"{what}: f32 max rel err {err[worst]:.3e} > {tol:.0e} at {worst}: "
                                   f"got {a[worst]!r} want {b[worst]!r}")
        elem = float(err[worst])
    else:
        ulp = _ulp(np.maximum(np.abs(b), tau), dt)
        if den is not None:
            ulp = ulp + RTOL_F32 * den
        err = np.abs(a - b) / ulp
        worst = int(np.argmax(err))
        assert err[worst] <= 1.0 + 1e-9, (f"{what}: {err[worst]:.2f} ulp off at {worst}: got {a[worst]!r} "
                                          f"want {b[worst]!r}")
        elem = float(np.max(np.abs(a - b) / np.maximum(np.abs(b), tau if tau > 0 else 1e-30)))
    nb = float(np.linalg.norm(b))
    norm = float(np.linalg.norm(a - b) / nb) if nb > 0 else float(np.linalg.norm(a - b))
    if dt != F32:
        assert norm <= NORM_RTOL_LOWP, f"{what}: norm-wise rel err {norm:.3e} > {NORM_RTOL_LOWP}"
    return {"max_rel": elem, "norm_rel": norm}


def pair_den(x: np.ndarray) -> np.ndarray:
    """Per-element |(x0, x1)| of interleaved pairs (last dim), for rotations."""
    x = np.asarray(x, np.float64)
    pr = x.reshape(x.shape[:-1] + (x.shape[-1] // 2, 2))
    n = np.sqrt((pr * pr).sum(-1, keepdims=True))
    return np.broadcast_to(n, pr.shape).reshape(x.shape)


def merge_den(orc, stft, masks, mb, B, F, T, C):
    """sum_e |stft| |mask_e| / count for every complex output of the band merge (f32),
    repeated for the re and im parts: the magnitude its f32 products cancel from."""
    s_abs = np.zeros_like(stft)
    s_abs[..., 0] = np.hypot(stft[..., 0], stft[..., 1])
    m_abs = []
    for m in masks:
        m = np.asarray(m, np.float32).reshape(B, T, -1, 2)
        a = np.zeros_like(m)
        a[..., 0] = np.hypot(m[..., 0], m[..., 1])
        m_abs.append(a)
    cnt = mb["bands_per_freq"].astype(np.float32)
    out = orc.band_mask_merge(s_abs, m_abs, F32, mb["csr_offsets"], mb["csr_indices"], cnt, F32, F32, B, F, T, C)
    return np.repeat(out[..., :1], 2, axis=-1)

