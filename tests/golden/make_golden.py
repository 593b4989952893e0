"""Writes the golden fixtures in this directory (run from the repository root:
`python tests/golden/make_golden.py [fixture ...]`).

The reference (Rust + WGSL on wgpu) cannot be built or run in this image, so
these vectors come from the build's own seeded generators and the CPU oracle
(oracle/), whose functions are pinned independently by the closed-form, brute
force and reference-KAT tests in tests/test_oracle_*.py. The fixtures freeze
those pinned results so the oracle and the HIP path are both checked against
the same stored bytes from now on:

  blocks.npz    Q4_0 / Q8_0 / Q4_K GGUF blocks (with subnormal, zero, inf and
                nan scales planted) and their dequantised f32 bit patterns
                (Q4_K both with and without the shader's f16 flush-to-zero).
  gemv.npz      64x256 products for Q4_0, Q8_0, Q4_K and F16 weights: raw
                bytes, x, the reference-order f32 result and an f64 result.
  rope.npz      RoPE tables [max_seq][hd/2][cos, sin] for hd 64 / theta 1e4
                and hd 128 / theta 5e5 (model/transformer/constructor.rs:454-489).
  f16.npz       binary16 -> binary32 decodes of chosen bit patterns in the
                three reference variants (exact, Q8_0 scale, flush-to-zero).
  kquant.npz    Q5_K blocks (subnormal d / dmin, every scale bit and every
                high bit in use) with their dequantised bits (exact and
                flush-to-zero), Q6_K blocks with their dequantised bits in
                GGML and in the reference loader's element order
                (compute/engine.rs:198-248), and 64x256 Q5_K / Q6_K products.
  greedy_c1.npz benchmark configuration 1 (synth.tiny_config1(1)): the 32-token prompt,
                the 16 greedy tokens under the reference loop and sampler
                (generation.rs:129-323, sampler.rs:146-209) and the first
                decode step's logits.
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
sys.path.insert(0, str(ROOT))

from janus_amd import synth  # noqa: E402
from oracle import oracle as O  # noqa: E402


def _bits(a) -> np.ndarray:
    return np.ascontiguousarray(a, np.float32).reshape(-1).view(np.uint32)


def blocks() -> dict:
    rng = np.random.default_rng(1001)
    q40 = synth.random_q4_0(rng, 4, 64).reshape(-1, 18)           # 8 blocks
    special = np.array([0x0000, 0x0001, 0x03FF, 0x0400, 0x7BFF, 0x7C00, 0xFC00, 0x7E01], np.uint16)
    q40[:, :2] = special.view(np.uint8).reshape(-1, 2)
    q80 = synth.random_q8_0(rng, 4, 64).reshape(-1, 34)
    q80[:, :2] = special.view(np.uint8).reshape(-1, 2)
    q4k = synth.random_q4_k(rng, 2, 512).reshape(-1, 144)          # 4 super-blocks
    q4k[0, 0:2] = np.array([0x0003], np.uint16).view(np.uint8)     # subnormal d
    q4k[1, 2:4] = np.array([0x0200], np.uint16).view(np.uint8)     # subnormal dmin
    q4k[2, 4:16] = np.arange(12, dtype=np.uint8) * 21              # every bit of the 6-bit packing in use
    q40, q80, q4k = q40.reshape(-1), q80.reshape(-1), q4k.reshape(-1)
    return {
        "q4_0": q40, "q4_0_deq": _bits(O.dequant(2, q40, 4, 64)),
        "q8_0": q80, "q8_0_deq": _bits(O.dequant(8, q80, 4, 64)),
        "q4_k": q4k, "q4_k_deq_ftz": _bits(O.dequant(12, q4k, 2, 512, ftz=True)),
        "q4_k_deq_exact": _bits(O.dequant(12, q4k, 2, 512, ftz=False)),
    }


def gemv() -> dict:
    rng = np.random.default_rng(1002)
    n, k = 64, 256
    out = {"x": rng.standard_normal(k, dtype=np.float32)}
    gens = {"q4_0": (2, synth.random_q4_0), "q8_0": (8, synth.random_q8_0), "q4_k": (12, synth.random_q4_k)}
    for name, (t, gen) in gens.items():
        raw = gen(rng, n, k)
        out[name] = raw
        out[name + "_y"] = O.gemm_auto(out["x"], t, raw, n, k)
        out[name + "_y64"] = O.gemv_f64(O.dequant(t, raw, n, k, ftz=(t == 12)), out["x"])
    f16 = synth.f16_bits(rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02))
    out["f16"] = f16
    out["f16_y"] = O.gemm_auto(out["x"], 1, f16, n, k)
    out["f16_y64"] = O.gemv_f64(O.dequant(1, f16, n, k, ftz=True), out["x"])
    return out


def rope() -> dict:
    return {"hd64_theta1e4": O.rope_table(64, 64, 10000.0), "hd128_theta5e5": O.rope_table(64, 128, 500000.0)}


def f16() -> dict:
    pats = np.array([0x0000, 0x8000, 0x0001, 0x8001, 0x03FF, 0x0400, 0x3C00, 0xC000, 0x7BFF, 0xFBFF,
                     0x7C00, 0xFC00, 0x7E00, 0x7C01, 0x3555, 0x1234], np.uint16)
    return {"bits": pats, "exact": _bits(O.f16_to_f32(pats, "exact")), "q8": _bits(O.f16_to_f32(pats, "q8")),
            "ftz": _bits(O.f16_to_f32(pats, "ftz"))}


def greedy_c1() -> dict:
    spec = synth.tiny_config1(1)
    prompt = np.random.default_rng(101).integers(0, spec.vocab, 32)
    m = O.OracleModel(spec, 64)
    toks, logits = m.generate(prompt.tolist(), 16, return_logits=True)
    return {"prompt": prompt.astype(np.int32), "tokens": np.array(toks, np.int32),
            "logits0": np.asarray(logits[0], np.float32)}


def kquant() -> dict:
    rng = np.random.default_rng(1003)
    q5k = synth.random_q5_k(rng, 2, 512).reshape(-1, 176)          # 4 super-blocks
    q5k[0, 0:2] = np.array([0x0003], np.uint16).view(np.uint8)     # subnormal d
    q5k[1, 2:4] = np.array([0x0200], np.uint16).view(np.uint8)     # subnormal dmin
    q5k[2, 4:16] = np.arange(12, dtype=np.uint8) * 21              # every bit of the 6-bit packing in use
    q5k[3, 16:48] = 0xFF                                           # every fifth bit set
    q6k = synth.random_q6_k(rng, 2, 512).reshape(-1, 210)
    q6k[0, 192:208] = np.array([-128, 127] * 8, np.int8).view(np.uint8)   # extreme scales
    q6k[1, 208:210] = np.array([0x0001], np.uint16).view(np.uint8)        # subnormal d
    q5k, q6k = q5k.reshape(-1), q6k.reshape(-1)
    out = {
        "q5_k": q5k, "q5_k_deq_exact": _bits(O.dequant(13, q5k, 2, 512)),
        "q5_k_deq_ftz": _bits(O.dequant(13, q5k, 2, 512, ftz=True)),
        "q6_k": q6k, "q6_k_deq_ggml": _bits(O.dequant(14, q6k, 2, 512)),
        "q6_k_deq_ref": _bits(O.dequant(14, q6k, 2, 512, q6k_ref_order=True)),
    }
    n, k = 64, 256
    out["x"] = rng.standard_normal(k, dtype=np.float32)
    for name, t, gen in (("q5_k", 13, synth.random_q5_k), ("q6_k", 14, synth.random_q6_k)):
        raw = gen(rng, n, k)
        out["gemv_" + name] = raw
        out["gemv_" + name + "_y"] = O.gemm_auto(out["x"], t, raw, n, k)
        wf = O.dequant(t, raw, n, k)
        if t == 14:   # the reference runs Q6_K as flush-to-zero binary16 weights
            wf = O.f16_to_f32(O.f32_to_f16_rne(wf), "ftz").reshape(n, k)
        out["gemv_" + name + "_y64"] = O.gemv_f64(wf, out["x"])
    return out


FIXTURES = {"blocks": blocks, "gemv": gemv, "rope": rope, "f16": f16, "kquant": kquant, "greedy_c1": greedy_c1}


def main(names: list[str]) -> None:
    """Writes every fixture, or only the named ones (an existing file is
    rewritten only when asked for, so unrelated fixtures keep their bytes)."""
    for name in names or list(FIXTURES):
        np.savez_compressed(HERE / f"{name}.npz", **FIXTURES[name]())
        print(f"wrote tests/golden/{name}.npz")


if __name__ == "__main__":
    main(sys.argv[1:])
