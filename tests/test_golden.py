"""The oracle against the committed golden fixtures (tests/golden/*.npz,
written by tests/golden/make_golden.py) and, where the fixture allows, against
independent closed forms, so a change to the oracle or the generators that
moves any stored bit fails here."""
from pathlib import Path

import numpy as np

from janus_amd import synth
from oracle import oracle as O
from tests.test_oracle_dequant import np_q4_0, np_q4_k, np_q8_0

G = Path(__file__).resolve().parent / "golden"


def _bits(a):
    return np.ascontiguousarray(a, np.float32).reshape(-1).view(np.uint32)


def _load(name):
    return np.load(G / f"{name}.npz")


def test_blocks_dequant_golden_and_closed_form():
    d = _load("blocks")
    assert np.array_equal(_bits(O.dequant(2, d["q4_0"], 4, 64)), d["q4_0_deq"])
    assert np.array_equal(_bits(O.dequant(8, d["q8_0"], 4, 64)), d["q8_0_deq"])
    assert np.array_equal(_bits(O.dequant(12, d["q4_k"], 2, 512, ftz=True)), d["q4_k_deq_ftz"])
    assert np.array_equal(_bits(O.dequant(12, d["q4_k"], 2, 512, ftz=False)), d["q4_k_deq_exact"])
    # independent numpy closed forms (nan scales excluded: payloads are not compared)
    for got, want in ((d["q4_0_deq"], np_q4_0(d["q4_0"])), (d["q8_0_deq"], np_q8_0(d["q8_0"])),
                      (d["q4_k_deq_ftz"], np_q4_k(d["q4_k"], True)), (d["q4_k_deq_exact"], np_q4_k(d["q4_k"], False))):
        w = np.ascontiguousarray(want, np.float32)
        ok = ~np.isnan(w)
        assert np.array_equal(got[ok], _bits(w)[ok])


def test_gemv_golden():
    d = _load("gemv")
    x = d["x"]
    for name, t in (("q4_0", 2), ("q8_0", 8), ("q4_k", 12), ("f16", 1)):
        y = O.gemm_auto(x, t, d[name], 64, 256)
        assert np.array_equal(_bits(y), _bits(d[name + "_y"])), name
        wf = O.dequant(t, d[name], 64, 256, ftz=(t in (1, 12)))
        bound = 1e-5 * (np.abs(wf.astype(np.float64)) @ np.abs(x.astype(np.float64))) + 1e-30
        assert np.all(np.abs(d[name + "_y"] - d[name + "_y64"]) <= bound), name


def test_kquant_golden():
    d = _load("kquant")
    assert np.array_equal(_bits(O.dequant(13, d["q5_k"], 2, 512)), d["q5_k_deq_exact"])
    assert np.array_equal(_bits(O.dequant(13, d["q5_k"], 2, 512, ftz=True)), d["q5_k_deq_ftz"])
    assert np.array_equal(_bits(O.dequant(14, d["q6_k"], 2, 512)), d["q6_k_deq_ggml"])
    assert np.array_equal(_bits(O.dequant(14, d["q6_k"], 2, 512, q6k_ref_order=True)), d["q6_k_deq_ref"])
    # Q5_K with its high bits cleared is the independent numpy Q4_K closed form
    # of the same header and nibbles
    b = d["q5_k"].reshape(-1, 176).copy()
    q4 = np.ascontiguousarray(np.concatenate([b[:, :16], b[:, 48:]], axis=1)).reshape(-1)
    b[:, 16:48] = 0
    for ftz in (False, True):
        assert np.array_equal(_bits(O.dequant(13, b.reshape(-1), 2, 512, ftz=ftz)), _bits(np_q4_k(q4, ftz)))
    x = d["x"]
    for name, t in (("q5_k", 13), ("q6_k", 14)):
        y = O.gemm_auto(x, t, d["gemv_" + name], 64, 256)
        assert np.array_equal(_bits(y), _bits(d["gemv_" + name + "_y"])), name
        wf = O.dequant(t, d["gemv_" + name], 64, 256)
        bound = 1e-5 * (np.abs(wf.astype(np.float64)) @ np.abs(x.astype(np.float64))) + 1e-30
        assert np.all(np.abs(d["gemv_" + name + "_y"] - d["gemv_" + name + "_y64"]) <= 2 * bound), name


def test_rope_golden_and_closed_form():
    d = _load("rope")
    for key, hd, theta in (("hd64_theta1e4", 64, 10000.0), ("hd128_theta5e5", 128, 500000.0)):
        t = O.rope_table(64, hd, theta)
        assert np.array_equal(_bits(t), _bits(d[key])), key
        pos = np.arange(64, dtype=np.float64)[:, None]
        inv = np.float64(theta) ** (-2.0 * np.arange(hd // 2, dtype=np.float64) / hd)
        ang = pos * inv
        want = np.stack([np.cos(ang), np.sin(ang)], axis=-1).reshape(-1)
        assert np.allclose(d[key], want, atol=2e-5 * 64, rtol=0), key   # f32 angle rounding grows with pos


def test_f16_golden_against_ieee():
    d = _load("f16")
    bits = d["bits"]
    assert np.array_equal(_bits(O.f16_to_f32(bits, "exact")), d["exact"])
    assert np.array_equal(_bits(O.f16_to_f32(bits, "q8")), d["q8"])
    assert np.array_equal(_bits(O.f16_to_f32(bits, "ftz")), d["ftz"])
    ieee = bits.view(np.float16).astype(np.float32)
    finite = np.isfinite(ieee)
    assert np.array_equal(d["exact"][finite], _bits(ieee)[finite])
    sub = (bits & 0x7C00) == 0
    assert np.all(d["ftz"][sub] & 0x7FFFFFFF == 0)


def test_config1_greedy_golden():
    d = _load("greedy_c1")
    spec = synth.tiny_config1(1)
    prompt = d["prompt"].tolist()
    assert prompt == np.random.default_rng(101).integers(0, spec.vocab, 32).tolist()
    toks, logits = O.OracleModel(spec, 64).generate(prompt, 16, return_logits=True)
    assert toks == d["tokens"].tolist()
    assert np.array_equal(_bits(logits[0]), _bits(d["logits0"]))
