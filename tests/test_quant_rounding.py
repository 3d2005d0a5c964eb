"""The quantizers' division-free rounding (csrc/common.hpp rint_quot_n), restated in numpy float32
(IEEE-rounded multiply and divide, ties-to-even rint, as the kernels' __fmul_rn / __fdiv_rn /
rintf): rint(v * fl(1/s)), falling back to rint(fl(v / s)) where frac(v * fl(1/s)) lies within
2^-15 of 1/2, equals rint(fl(v / s)) for every scale rule the kernels use (per-token / block-32
int8: amax * fl(1/127); int4: amax / 7 and amax * fl(1/7)). Random rows over 60 decades, rows of
integer ratios, and values placed on, and one ulp either side of, every half-integer quotient.
A threshold much below the error bound (2^-22) must fail, so the check is not vacuous."""
import numpy as np
import pytest

f32 = np.float32


def _fast(v, s, r, thr):
    y = (v * r).astype(f32)
    f = (y - np.floor(y)).astype(f32)
    near = ~(np.abs((f - f32(0.5)).astype(f32)) > f32(thr))
    out = np.rint(y)
    out[near] = np.rint((v[near] / s).astype(f32))
    return out


def _mismatches(thr, trials=120):
    rng = np.random.default_rng(0)
    bad = 0
    for trial in range(trials):
        K = 2048
        kind = trial % 4
        if kind == 0:
            v = rng.standard_normal(K).astype(f32)
        elif kind == 1:
            v = (rng.standard_normal(K) * 10.0 ** rng.uniform(-30, 30)).astype(f32)
        elif kind == 2:
            v = rng.integers(-1000, 1000, K).astype(f32) / f32(rng.integers(1, 50))
        else:
            v = (rng.uniform(-1, 1, K) ** 3 * rng.uniform(1e-3, 1e3)).astype(f32)
        amax = np.max(np.abs(v)).astype(f32)
        for rule in ("i8", "i4div", "i4mul"):
            a = np.maximum(amax, f32(1e-8))
            s = (a * f32(1.0 / 127.0) if rule == "i8" else a / f32(7.0) if rule == "i4div" else a * f32(1.0 / 7.0)).astype(f32)
            r = (f32(1.0) / s).astype(f32)
            lim = 127 if rule == "i8" else 8
            h = (rng.integers(-lim, lim, 256) + f32(0.5)).astype(f32)
            hs = (h * s).astype(f32)
            vv = np.clip(np.concatenate([v, hs, np.nextafter(hs, f32(np.inf)), np.nextafter(hs, -f32(np.inf))]), -amax, amax)
            bad += int(np.sum(_fast(vv, s, r, thr) != np.rint((vv / s).astype(f32))))
    return bad


def test_reciprocal_rounding_equals_exact_division():
    assert _mismatches(2.0 ** -15) == 0


def test_too_small_threshold_is_caught():
    assert _mismatches(2.0 ** -22) > 0
