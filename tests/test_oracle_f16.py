"""Pins the oracle's binary16 conversions.

- f16 -> f32 (exact, Q8_0 and FTZ variants) exhaustively over all 65,536
  patterns against numpy's IEEE conversion, with each variant's special
  cases (gemm_q8_0.wgsl:33-60, gemm_q4_k.wgsl:30-43) stated independently.
- f32 -> f16 round-to-nearest-even (the `half` crate used by
  compute/engine.rs:133-136) against numpy's float16 cast on every f16
  rounding boundary and a large random sample of binary32 patterns.
"""
import numpy as np
import pytest

from oracle import oracle as O

ALL16 = np.arange(65536, dtype=np.uint32).astype(np.uint16)


def _bits(x):
    return np.asarray(x, dtype=np.float32).view(np.uint32)


def test_f16_exact_matches_ieee():
    ref = ALL16.view(np.float16).astype(np.float32)
    got = O.f16_to_f32(ALL16, "exact")
    nan = np.isnan(ref)
    assert np.array_equal(_bits(got)[~nan], _bits(ref)[~nan])
    assert np.isnan(got[nan]).all()
    # subnormals are exact multiples of 2^-24
    sub = (ALL16 & 0x7C00) == 0
    assert np.array_equal(np.abs(got[sub]), (ALL16[sub] & 0x3FF).astype(np.float32) * np.float32(2.0 ** -24))


def test_f16_ftz_flushes_subnormals_only():
    got = O.f16_to_f32(ALL16, "ftz")
    exact = O.f16_to_f32(ALL16, "exact")
    sub = (ALL16 & 0x7C00) == 0
    # subnormals (and zeros) become zero with the input's sign
    assert np.all(got[sub] == 0)
    assert np.array_equal(np.signbit(got[sub]), (ALL16[sub] & 0x8000) != 0)
    rest = ~sub & ~np.isnan(exact)
    assert np.array_equal(_bits(got[rest]), _bits(exact[rest]))


def test_f16_q8_maps_exponent31_to_1e38():
    got = O.f16_to_f32(ALL16, "q8")
    exact = O.f16_to_f32(ALL16, "exact")
    e31 = (ALL16 & 0x7C00) == 0x7C00
    neg = (ALL16 & 0x8000) != 0
    assert np.all(got[e31 & ~neg] == np.float32(1e38))
    assert np.all(got[e31 & neg] == np.float32(-1e38))
    assert np.array_equal(_bits(got[~e31]), _bits(exact[~e31]))


def _rne_reference(x: np.ndarray) -> np.ndarray:
    return x.astype(np.float16).view(np.uint16)


def test_f32_to_f16_rounding_boundaries():
    # every finite f16 value, the midpoints between neighbours and one ulp of
    # f32 either side of each midpoint: the cases a wrong tie rule would miss
    vals = ALL16.view(np.float16).astype(np.float64)
    fin = np.isfinite(vals)
    v = np.sort(np.unique(vals[fin]))
    mids = (v[:-1] + v[1:]) / 2
    cand = np.concatenate([v, mids, [65504.0, 65519.99, 65520.0, 65536.0, 1e6, 2.0 ** -25, 2.0 ** -26]])
    cand = np.concatenate([cand, -cand]).astype(np.float32)
    cand = np.concatenate([cand, np.nextafter(cand, np.float32(np.inf)), np.nextafter(cand, np.float32(-np.inf))])
    got = O.f32_to_f16_rne(cand)
    assert np.array_equal(got, _rne_reference(cand))


def test_f32_to_f16_random_patterns():
    rng = np.random.default_rng(7)
    pats = rng.integers(0, 2 ** 32, size=2_000_000, dtype=np.uint64).astype(np.uint32)
    x = pats.view(np.float32)
    got = O.f32_to_f16_rne(x)
    ref = _rne_reference(x)
    nan = np.isnan(x)
    assert np.array_equal(got[~nan], ref[~nan])
    assert np.all((got[nan] & 0x7C00) == 0x7C00) and np.all((got[nan] & 0x3FF) != 0)


@pytest.mark.parametrize("val,bits", [(1.0, 0x3C00), (-2.0, 0xC000), (65504.0, 0x7BFF), (1e9, 0x7C00),
                                      (2.0 ** -24, 0x0001), (2.0 ** -25, 0x0000), (3 * 2.0 ** -26, 0x0001)])
def test_f32_to_f16_known_values(val, bits):
    assert O.f32_to_f16_rne([val])[0] == bits
