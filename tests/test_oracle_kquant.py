"""Pins the oracle's Q5_K and Q6_K dequantisation.

Q5_K (GGML block_q5_K, 176 bytes) is pinned by reduction and brute force:
with every qh bit clear it must equal the already-pinned Q4_K dequantisation
of the same header and nibbles; setting any single one of the 256 qh bits
must change exactly one element, by exactly 16 * d * sc of that element's
sub-block, and the 256 bits must reach 256 distinct elements at the places
GGML's layout gives (bit 2j + h of qh[t] -> element 64j + 32h + t). The
build's quantiser round-trips through it within the quantisation step.

Q6_K (GGML block_q6_K, 210 bytes) is pinned by special values (all-zero and
all-one bit patterns fix the -32 offset and the sign of the int8 scales), by
brute force over single nibbles and single 2-bit fields (each must reach a
distinct element, in both element orders), by a hand-worked known answer for
the reference loader's order (compute/engine.rs:221-241), and by the
quantiser round trip in GGML order.
"""
import ctypes as C

import numpy as np
import pytest

from janus_amd import synth
from oracle import oracle as O

Q4_K, Q5_K, Q6_K = 12, 13, 14


def _q5_block(rng, d=1.0, dmin=0.5):
    blk = np.zeros(176, dtype=np.uint8)
    blk[0:2] = np.array([d], dtype=np.float16).view(np.uint8)
    blk[2:4] = np.array([dmin], dtype=np.float16).view(np.uint8)
    blk[4:16] = rng.integers(0, 256, 12, dtype=np.uint8)
    return blk


def _scale_min(s12: np.ndarray, j: int):
    a, b = C.c_uint8(), C.c_uint8()
    O.lib().jo_q4_k_scale_min(np.ascontiguousarray(s12), j, C.byref(a), C.byref(b))
    return a.value, b.value


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_q5_k_without_high_bits_is_q4_k(seed):
    rng = np.random.default_rng(seed)
    nb = 16
    raw = rng.integers(0, 256, (nb, 176), dtype=np.uint8)
    raw[:, 16:48] = 0
    d = np.abs(rng.standard_normal((nb, 2))).astype(np.float16) * np.float16(0.01)
    raw[:, 0:4] = d.view(np.uint8).reshape(nb, 4)
    q4 = np.concatenate([raw[:, 0:16], raw[:, 48:]], axis=1)
    got = O.dequant(Q5_K, raw.reshape(-1), nb, 256)
    want = O.dequant(Q4_K, q4.reshape(-1), nb, 256)
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


def test_q5_k_every_high_bit_reaches_one_element():
    rng = np.random.default_rng(5)
    blk = _q5_block(rng, d=0.5, dmin=0.25)
    blk[48:] = rng.integers(0, 256, 128, dtype=np.uint8)
    base = O.dequant(Q5_K, blk, 1, 256)[0]
    d = 0.5
    seen = set()
    for t in range(32):
        for bit in range(8):
            b2 = blk.copy()
            b2[16 + t] = 1 << bit
            w = O.dequant(Q5_K, b2, 1, 256)[0]
            diff = np.nonzero(w != base)[0]
            j, h = bit // 2, bit % 2
            want_el = 64 * j + 32 * h + t
            sc, _ = _scale_min(blk[4:16], 2 * j + h)
            if sc == 0:
                assert diff.size == 0
                continue
            assert diff.tolist() == [want_el], (t, bit, diff)
            assert w[want_el] - base[want_el] == np.float32(16 * d * sc)
            seen.add(want_el)
    assert len(seen) == sum(1 for e in range(256) if _scale_min(blk[4:16], e // 32)[0])


def test_q5_k_quantizer_round_trip():
    rng = np.random.default_rng(7)
    n, k = 8, 512
    w = rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02)
    raw = synth.quantize_q5_k(w)
    back = O.dequant(Q5_K, raw, n, k)
    sb = w.reshape(-1, 8, 32)
    step = (sb.max(axis=2) - np.minimum(sb.min(axis=2), 0)) / 31.0
    err = np.abs(back.reshape(-1, 8, 32) - sb)
    # half a step from rounding plus the 6-bit scale/min quantisation
    assert np.all(err <= 0.5 * step[:, :, None] * 1.2 + 0.04 * np.abs(sb).max())
    assert np.abs(back - w).mean() < 0.1 * np.abs(w).mean()


def _q6_block(d=1.0, scales=None):
    blk = np.zeros(210, dtype=np.uint8)
    blk[192:208] = (np.ones(16, np.int8) if scales is None else np.asarray(scales, np.int8)).view(np.uint8)
    blk[208:210] = np.array([d], dtype=np.float16).view(np.uint8)
    return blk


@pytest.mark.parametrize("ref_order", [False, True])
def test_q6_k_special_values(ref_order):
    scales = np.arange(-8, 8, dtype=np.int8)
    blk = _q6_block(0.25, scales)
    w0 = O.dequant(Q6_K, blk, 1, 256, q6k_ref_order=ref_order)[0]
    blk[:192] = 0xFF
    w1 = O.dequant(Q6_K, blk, 1, 256, q6k_ref_order=ref_order)[0]
    # every element's scale is one of the 16 groups' in both orders, so the
    # all-zero / all-one patterns give -32 and +31 units of d * scale
    assert sorted(np.unique(w0 / np.float32(-32 * 0.25)).tolist()) == sorted(set(scales.astype(float).tolist()))
    np.testing.assert_array_equal(w1 * np.float32(-32), w0 * np.float32(31))
    if ref_order:
        # engine.rs:236: scales[i / 16] -- contiguous 16-element groups
        np.testing.assert_array_equal(w0, np.repeat(scales, 16).astype(np.float32) * np.float32(-8.0))


@pytest.mark.parametrize("ref_order", [False, True])
def test_q6_k_every_nibble_and_high_pair_reaches_one_element(ref_order):
    blk = _q6_block(1.0)
    base = O.dequant(Q6_K, blk, 1, 256, q6k_ref_order=ref_order)[0]
    hit_lo, hit_hi = set(), set()
    for byte in range(128):
        for nib in range(2):
            b2 = blk.copy()
            b2[byte] = 1 << (4 * nib)
            diff = np.nonzero(O.dequant(Q6_K, b2, 1, 256, q6k_ref_order=ref_order)[0] != base)[0]
            assert diff.size == 1
            hit_lo.add(int(diff[0]))
    for byte in range(64):
        for pair in range(4):
            b2 = blk.copy()
            b2[128 + byte] = 1 << (2 * pair)
            w = O.dequant(Q6_K, b2, 1, 256, q6k_ref_order=ref_order)[0]
            diff = np.nonzero(w != base)[0]
            assert diff.size == 1 and w[diff[0]] - base[diff[0]] == 16.0
            hit_hi.add(int(diff[0]))
    assert hit_lo == set(range(256)) and hit_hi == set(range(256))
    if not ref_order:
        # GGML: the low nibble of ql[l] and bits 0-1 of qh[l] are both element l
        for l in range(32):
            b2 = blk.copy()
            b2[l] = 1
            assert np.nonzero(O.dequant(Q6_K, b2, 1, 256)[0] != base)[0].tolist() == [l]
            b2 = blk.copy()
            b2[128 + l] = 1 << 6     # bits 6-7 of qh[l]: element l + 96
            assert np.nonzero(O.dequant(Q6_K, b2, 1, 256)[0] != base)[0].tolist() == [l + 96]


def test_q6_k_reference_order_known_answer():
    """compute/engine.rs:221-241 worked by hand: element i takes nibble i % 2
    of ql[i / 2] and bits 2 (i % 4) of qh[i / 4]."""
    blk = _q6_block(0.5)
    blk[0] = 0x21          # elements 0, 1: low nibbles 1, 2
    blk[1] = 0x43          # elements 2, 3: low nibbles 3, 4
    blk[128] = 0b11100100  # elements 0..3: high pairs 0, 1, 2, 3
    w = O.dequant(Q6_K, blk, 1, 256, q6k_ref_order=True)[0]
    want = [0.5 * (q - 32) for q in (0 * 16 + 1, 1 * 16 + 2, 2 * 16 + 3, 3 * 16 + 4)]
    np.testing.assert_array_equal(w[:4], np.array(want, np.float32))
    assert np.all(w[4:] == np.float32(-16.0))


def test_q6_k_quantizer_round_trip():
    rng = np.random.default_rng(9)
    n, k = 8, 512
    w = rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02)
    raw = synth.quantize_q6_k(w)
    back = O.dequant(Q6_K, raw, n, k)
    g = w.reshape(-1, 16)
    step = np.abs(g).max(axis=1) / 31.0
    err = np.abs(back.reshape(-1, 16) - g)
    assert np.all(err <= 0.5 * step[:, None] * 1.1 + 0.01 * np.abs(g).max())
    assert np.abs(back - w).mean() < 0.05 * np.abs(w).mean()
    # the reference loader's order reads the same bytes as another permutation
    assert not np.array_equal(O.dequant(Q6_K, raw, n, k, q6k_ref_order=True), back)


def test_q5_k_gemv_close_to_f64():
    rng = np.random.default_rng(11)
    n, k = 64, 1024
    raw = synth.random_q5_k(rng, n, k)
    x = rng.standard_normal(k, dtype=np.float32)
    y = O.gemm_auto(x, Q5_K, raw, n, k)
    wf = O.dequant(Q5_K, raw, n, k)
    ref = wf.astype(np.float64) @ x.astype(np.float64)
    bound = 1e-5 * (np.abs(wf) @ np.abs(x))
    assert np.all(np.abs(y - ref) <= bound)


def _q6_k_ggml_numpy(raw: np.ndarray) -> np.ndarray:
    """GGML's published block_q6_K placement, restated element by element in
    numpy (independent of the oracle's loop): element e = 128 h + 32 j + l of a
    block (h < 2, j < 4, l < 32) takes the low (j < 2) or high (j >= 2) nibble
    of ql[64 h + l + 32 (j % 2)], bits 2 j..2 j + 1 of qh[32 h + l], and the
    int8 scale sc[8 h + l // 16 + 2 j]; w = d * sc * (q - 32) in binary32."""
    blk = raw.reshape(-1, 210)
    e = np.arange(256)
    h, j, l = e // 128, (e % 128) // 32, e % 32
    ql = blk[:, 64 * h + l + 32 * (j % 2)]
    lo = np.where(j < 2, ql & 15, ql >> 4).astype(np.int32)
    hi = ((blk[:, 128 + 32 * h + l] >> (2 * j)) & 3).astype(np.int32)
    sc = blk[:, 192:208].view(np.int8)[:, 8 * h + l // 16 + 2 * j].astype(np.float32)
    d = blk[:, 208:210].copy().view(np.float16).astype(np.float32)
    q = ((hi << 4) | lo) - 32
    return ((d * sc) * q.astype(np.float32)).reshape(-1)


def test_q6_k_ggml_order_matches_independent_numpy_dequant():
    """Every element and every scale group of random blocks: the oracle's GGML
    order equals the numpy restatement bit for bit (a swapped l + 32 / l + 64
    placement or scale group would differ on random bytes)."""
    rng = np.random.default_rng(61)
    nb = 64
    raw = rng.integers(0, 256, nb * 210, dtype=np.uint8).reshape(nb, 210)
    # finite binary16 scales d spanning several binades, some negative
    raw[:, 208:210] = (rng.uniform(-2.0, 2.0, nb) * 2.0 ** rng.integers(-14, 4, nb)).astype(np.float16).reshape(nb, 1).view(np.uint8)
    raw = raw.reshape(-1)
    got = O.dequant(Q6_K, raw, nb, 256).reshape(-1)
    want = _q6_k_ggml_numpy(raw)
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
    # and the two placements are not the same function (the test can fail)
    ref = O.dequant(Q6_K, raw, nb, 256, q6k_ref_order=True).reshape(-1)
    assert np.count_nonzero(ref != want) > 200 * nb
