"""Pins the oracle's block dequantisation and reference-order products.

Each format is checked against an independent numpy statement of its GGML
closed form (written from the block layout, not from the oracle's loops):
Q4_0 (w = d*(q-8), nibble j / j+16), Q8_0 (w = d*q with the shader's scale
decode), Q4_K (GGML dequantize_row_q4_K with get_scale_min_k4, which the
shader restates in gemm_q4_k.wgsl:82-147). Brute force covers every nibble
value for Q4_0 and every value of every scale byte for Q4_K's 6-bit unpack.
"""
import numpy as np
import pytest

from janus_amd import synth
from oracle import oracle as O


def np_q4_0(raw: np.ndarray) -> np.ndarray:
    b = raw.reshape(-1, 18)
    d = b[:, :2].copy().view(np.float16).astype(np.float32)          # [nb, 1]
    qs = b[:, 2:]
    q = np.concatenate([qs & 15, qs >> 4], axis=1).astype(np.int32) - 8
    return (d * q.astype(np.float32)).reshape(-1)


def np_q8_0(raw: np.ndarray) -> np.ndarray:
    b = raw.reshape(-1, 34)
    dbits = b[:, :2].copy().view(np.uint16)[:, 0]
    d = dbits.view(np.float16).astype(np.float32)
    inf = (dbits & 0x7C00) == 0x7C00
    d = np.where(inf, np.where(dbits & 0x8000, np.float32(-1e38), np.float32(1e38)), d).astype(np.float32)
    q = b[:, 2:].view(np.int8).astype(np.float32)
    return (d[:, None] * q).reshape(-1)


def np_scale_min_k4(s: np.ndarray, j: int):
    """GGML get_scale_min_k4 on a [nb, 12] array."""
    s = s.astype(np.int32)
    if j < 4:
        return s[:, j] & 63, s[:, j + 4] & 63
    return (s[:, j + 4] & 0xF) | ((s[:, j - 4] >> 6) << 4), (s[:, j + 4] >> 4) | ((s[:, j] >> 6) << 4)


def np_q4_k(raw: np.ndarray, ftz: bool) -> np.ndarray:
    b = raw.reshape(-1, 144)
    dbits = b[:, 0:2].copy().view(np.uint16)[:, 0]
    mbits = b[:, 2:4].copy().view(np.uint16)[:, 0]
    if ftz:
        dbits = np.where((dbits & 0x7C00) == 0, dbits & 0x8000, dbits).astype(np.uint16)
        mbits = np.where((mbits & 0x7C00) == 0, mbits & 0x8000, mbits).astype(np.uint16)
    d = dbits.view(np.float16).astype(np.float32)
    dmin = mbits.view(np.float16).astype(np.float32)
    sc, qs = b[:, 4:16], b[:, 16:]
    out = np.empty((b.shape[0], 256), dtype=np.float32)
    for j in range(4):
        for half in range(2):
            s, m = np_scale_min_k4(sc, 2 * j + half)
            scale = d * s.astype(np.float32)
            mn = dmin * m.astype(np.float32)
            q = (qs[:, 32 * j:32 * j + 32] >> (4 * half)) & 15
            out[:, 64 * j + 32 * half: 64 * j + 32 * half + 32] = (scale[:, None] * q.astype(np.float32)
                                                                    - mn[:, None])
    return out.reshape(-1)


def _bits_equal(a, b):
    a = np.ascontiguousarray(a, np.float32).reshape(-1)
    b = np.ascontiguousarray(b, np.float32).reshape(-1)
    return np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_q4_0_closed_form():
    rng = np.random.default_rng(0)
    raw = synth.random_q4_0(rng, 64, 256)
    assert _bits_equal(O.dequant(2, raw, 64, 256), np_q4_0(raw))


def test_q4_0_every_nibble_and_special_scales():
    # one block per (scale pattern): all 16 nibble values in both halves
    scales = np.array([0x3C00, 0x0001, 0x03FF, 0x8400, 0x7BFF, 0x2E66, 0x0000, 0x8001], dtype=np.uint16)
    raw = np.zeros((len(scales), 18), dtype=np.uint8)
    raw[:, :2] = scales.view(np.uint8).reshape(-1, 2)
    nib = np.arange(16, dtype=np.uint8)
    raw[:, 2:] = nib | (nib[::-1] << 4)
    got = O.dequant(2, raw.reshape(-1), len(scales), 32)
    assert _bits_equal(got.reshape(-1), np_q4_0(raw.reshape(-1)))
    d = scales.view(np.float16).astype(np.float32)
    assert np.array_equal(got[:, :16], d[:, None] * (np.arange(16) - 8).astype(np.float32))


def test_q8_0_closed_form_with_subnormal_and_inf_scales():
    rng = np.random.default_rng(1)
    raw = synth.random_q8_0(rng, 32, 256).reshape(-1, 34)
    special = np.array([0x0001, 0x03FF, 0x7C00, 0xFC00, 0x7E00, 0x8002], dtype=np.uint16)
    raw[: len(special), :2] = special.view(np.uint8).reshape(-1, 2)
    raw = raw.reshape(-1)
    got = O.dequant(8, raw, 32, 256)
    assert _bits_equal(got, np_q8_0(raw))
    assert got[0, 1] == np.float32(2.0 ** -24) * np.float32(raw.reshape(-1, 34)[0, 3].view(np.int8))


@pytest.mark.parametrize("ftz", [False, True])
def test_q4_k_closed_form(ftz):
    rng = np.random.default_rng(2)
    raw = synth.random_q4_k(rng, 8, 512).reshape(-1, 144)
    # force some subnormal d / dmin so the FTZ branch matters
    raw[0, 0:2] = np.array([0x0123], np.uint16).view(np.uint8)
    raw[1, 2:4] = np.array([0x8011], np.uint16).view(np.uint8)
    raw = raw.reshape(-1)
    assert _bits_equal(O.dequant(12, raw, 8, 512, ftz=ftz), np_q4_k(raw, ftz))


def test_q4_k_scale_unpack_every_byte_value():
    # vary each of the 12 scale bytes through all 256 values (others random)
    rng = np.random.default_rng(3)
    L = O.lib()
    import ctypes as C
    for byte in range(12):
        base = rng.integers(0, 256, 12, dtype=np.uint8)
        blocks = np.repeat(base[None, :], 256, axis=0)
        blocks[:, byte] = np.arange(256, dtype=np.uint8)
        for j in range(8):
            want_s, want_m = np_scale_min_k4(blocks, j)
            sc, mn = C.c_uint8(), C.c_uint8()
            for r in range(0, 256, 17):
                L.jo_q4_k_scale_min(np.ascontiguousarray(blocks[r]), j, C.byref(sc), C.byref(mn))
                assert (sc.value, mn.value) == (want_s[r], want_m[r])


def test_q4_k_quantizer_round_trip():
    rng = np.random.default_rng(4)
    w = rng.standard_normal((16, 512), dtype=np.float32) * np.float32(0.02)
    raw = synth.quantize_q4_k(w)
    back = O.dequant(12, raw, 16, 512)
    # 4-bit sub-block quantisation with 6-bit scales: error well under a step
    step = (w.reshape(-1, 32).max(1) - np.minimum(w.reshape(-1, 32).min(1), 0)) / 15
    err = np.abs(back - w).reshape(-1, 32).max(1)
    assert np.all(err <= step * 1.5 + 1e-4)


@pytest.mark.parametrize("ggml_type,gen", [(2, synth.random_q4_0), (8, synth.random_q8_0), (12, synth.random_q4_k)])
def test_reference_order_gemv_close_to_f64(ggml_type, gen):
    rng = np.random.default_rng(5)
    n, k = 48, 512
    raw = gen(rng, n, k)
    x = rng.standard_normal(k, dtype=np.float32)
    y = O.gemm_auto(x, ggml_type, raw, n, k)
    w = O.dequant(ggml_type, raw, n, k, ftz=(ggml_type == 12))
    y64 = O.gemv_f64(w, x)
    bound = 1e-5 * (np.abs(w) @ np.abs(x)) + 1e-30
    assert np.all(np.abs(y - y64) <= bound)


def test_reference_order_matches_sequential_sum():
    # Q8_0 order: per block sum of (d*q)*x, then row += block (gemm_q8_0.wgsl:95-123)
    rng = np.random.default_rng(6)
    raw = synth.random_q8_0(rng, 4, 96)
    x = rng.standard_normal(96, dtype=np.float32)
    w = np_q8_0(raw).reshape(4, 96)
    want = np.zeros(4, dtype=np.float32)
    for r in range(4):
        row = np.float32(0)
        for b in range(3):
            s = np.float32(0)
            for i in range(32):
                s = np.float32(s + np.float32(w[r, 32 * b + i] * x[32 * b + i]))
            row = np.float32(row + s)
        want[r] = row
    assert _bits_equal(O.gemm_auto(x, 8, raw, 4, 96), want)
