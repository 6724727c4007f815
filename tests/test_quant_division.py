"""The FP8 group quantisers (the prefill gate_up epilogue, and the
per-token-group quantiser of hidden rows used by routing, the standalone
quantiser and the decode kernels' staging) divide by the group scale as
y = x * r, r = 1/scale (IEEE), then y + fma(-y, scale, x) * r.  This checks,
in emulated fp32 (products of two fp32 values are exact in float64, as the
FMA's are), that the corrected quotient equals IEEE fp32 division for the
values the epilogue sees: |x| <= amax, scale = max(amax, 1e-10) / 448."""
import numpy as np


def _f32(x):
    return np.asarray(x, dtype=np.float64).astype(np.float32)


def test_reciprocal_with_one_correction_equals_ieee_division():
    rng = np.random.default_rng(7)
    n = 2_000_000
    mag = rng.choice(np.array([1e-6, 1e-3, 1.0, 40.0, 3e3], dtype=np.float64), n)
    x = _f32(rng.standard_normal(n) * mag)
    amax = _f32(np.abs(x).astype(np.float64) * (1.0 + rng.random(n) * 4.0))
    scale = _f32(np.maximum(amax, np.float32(1e-10)).astype(np.float64) / 448.0)
    x64, s64 = x.astype(np.float64), scale.astype(np.float64)
    ieee = _f32(x64 / s64)
    r = _f32(1.0 / s64).astype(np.float64)
    y = _f32(x64 * r).astype(np.float64)
    resid = _f32(x64 - y * s64).astype(np.float64)   # fma(-y, scale, x), one rounding
    corrected = _f32(resid * r + y)                   # fma(resid, r, y), one rounding
    assert np.array_equal(corrected, ieee)
    # the plain product alone is not enough (so the test can fail)
    assert not np.array_equal(_f32(x64 * r), ieee)
