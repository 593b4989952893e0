"""The HIP path against the committed golden fixtures (tests/golden/*.npz)."""
from pathlib import Path

import numpy as np
import pytest
import torch

from janus_amd import ops, synth
from janus_amd.model import Model

pytestmark = pytest.mark.gpu
G = Path(__file__).resolve().parent / "golden"
DEV = "cuda:0"


def _bits(a):
    return np.ascontiguousarray(a, np.float32).reshape(-1).view(np.uint32)


def test_gpu_dequant_matches_golden_bits(engine):
    d = np.load(G / "blocks.npz")
    for key, t, n, k, flags in (("q4_0", 2, 4, 64, 0), ("q8_0", 8, 4, 64, 0), ("q4_k", 12, 2, 512, 1),
                                ("q4_k", 12, 2, 512, 0)):
        w = ops.GpuTensor(engine, t, n, k, d[key], flags)
        got = _bits(w.dequant().cpu().numpy())
        want = d[key + "_deq" + ("" if t != 12 else ("_ftz" if flags else "_exact"))]
        ok = ~np.isnan(want.view(np.float32))
        assert np.array_equal(got[ok], want[ok]), key


def test_gpu_gemv_matches_golden(engine):
    d = np.load(G / "gemv.npz")
    x = torch.from_numpy(d["x"]).to(DEV)
    for name, t in (("q4_0", 2), ("q8_0", 8), ("q4_k", 12), ("f16", 1)):
        w = ops.GpuTensor(engine, t, 64, 256, d[name], 1 if t in (1, 12) else 0)
        y = torch.empty(64, device=DEV)
        ops.gemm_auto(engine, x, w, y, 1, 1, 256, 64)
        wf = w.dequant().cpu().numpy().astype(np.float64)
        bound = 1e-5 * (np.abs(wf) @ np.abs(d["x"].astype(np.float64))) + 1e-30
        assert np.all(np.abs(y.cpu().numpy() - d[name + "_y64"]) <= bound), name


def test_gpu_kquant_matches_golden(engine):
    d = np.load(G / "kquant.npz")
    from oracle import oracle as O
    for flags, key in ((0, "q5_k_deq_exact"), (1, "q5_k_deq_ftz")):
        w = ops.GpuTensor(engine, 13, 2, 512, d["q5_k"], flags)
        assert np.array_equal(_bits(w.dequant().cpu().numpy()), d[key]), key
    # Q6_K is stored as the binary16 rounding of its dequantisation
    for flags, key in ((0, "q6_k_deq_ggml"), (2, "q6_k_deq_ref")):
        w = ops.GpuTensor(engine, 14, 2, 512, d["q6_k"], flags)
        want = O.f16_to_f32(O.f32_to_f16_rne(d[key].view(np.float32)), "exact")
        assert np.array_equal(_bits(w.dequant().cpu().numpy()), _bits(want)), key
    x = torch.from_numpy(d["x"]).to(DEV)
    for name, t, flags in (("q5_k", 13, 0), ("q6_k", 14, 1)):
        w = ops.GpuTensor(engine, t, 64, 256, d["gemv_" + name], flags)
        y = torch.empty(64, device=DEV)
        ops.gemm_auto(engine, x, w, y, 1, 1, 256, 64)
        wf = w.dequant().cpu().numpy().astype(np.float64)
        bound = 1e-5 * (np.abs(wf) @ np.abs(d["x"].astype(np.float64))) + 1e-30
        assert np.all(np.abs(y.cpu().numpy() - d["gemv_" + name + "_y64"]) <= bound), name


def test_gpu_rope_table_matches_golden(engine):
    d = np.load(G / "rope.npz")
    for key, hd, theta in (("hd64_theta1e4", 64, 10000.0), ("hd128_theta5e5", 128, 500000.0)):
        t = ops.create_rope_cache(engine, 64, hd, theta)
        assert np.array_equal(_bits(t.cpu().numpy()), _bits(d[key])), key


def test_gpu_config1_greedy_matches_golden(engine):
    d = np.load(G / "greedy_c1.npz")
    m = Model(engine, synth.tiny_config1(1), max_seq_len=64)
    assert m.generate(d["prompt"].tolist(), 16) == d["tokens"].tolist()
    m.forward([int(d["prompt"][-1])], [32])
    got = m.logits()[0]
    assert float(np.max(np.abs(got - d["logits0"])) / np.max(np.abs(d["logits0"]))) <= 2e-3
    m.close()
