"""GPU parity of the K-quant weight formats.

- Q4_K / Q5_K: the scale fields the upload rewrites decode every byte value
  of the GGML scale bytes as get_scale_min_k4 does.
- Q6_K: the upload dequantises on the host to binary16 as the reference's
  loader does (compute/engine.rs:800-831) and the handle reports F16; the
  stored weights are bit-exact against the oracle's dequantisation rounded
  to binary16, in GGML order and, with JANUS_WEIGHT_Q6K_REF_ORDER, in the
  reference's own order (engine.rs:198-248).
- Models mixing formats the way Q4_K_M / Q5_K_M GGUF files do (Q4_K or Q5_K
  blocks with Q6_K value / down projections and a Q6_K LM head) match the
  oracle's logits on the f32 and the fused binary16 paths, and the batched
  path equals single-sequence runs.
"""
import numpy as np
import pytest
import torch

from janus_amd import _lib, ops, synth
from janus_amd.model import Model
from oracle import oracle as O

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
REL = 2e-3


def _rel_err(a, b):
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))


@pytest.mark.parametrize("flags", [0, _lib.WEIGHT_Q6K_REF_ORDER, _lib.WEIGHT_FTZ_F16])
def test_q6_k_upload_is_the_binary16_rounded_dequant(engine, flags):
    n, k = 40, 768
    raw = synth.random_q6_k(np.random.default_rng(3), n, k)
    w = ops.GpuTensor(engine, _lib.DT_Q6_K, n, k, raw, flags)
    assert w.ggml_type == _lib.DT_F16
    got = w.dequant().cpu().numpy()
    wf = O.dequant(_lib.DT_Q6_K, raw, n, k, q6k_ref_order=bool(flags & _lib.WEIGHT_Q6K_REF_ORDER))
    bits = O.f32_to_f16_rne(wf)
    want = O.f16_to_f32(bits, "ftz" if flags & _lib.WEIGHT_FTZ_F16 else "exact").reshape(n, k)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_q6_k_rejects_bad_sizes(engine):
    raw = synth.random_q6_k(np.random.default_rng(4), 2, 256)
    with pytest.raises(_lib.JanusError):
        ops.GpuTensor(engine, _lib.DT_Q6_K, 2, 256, raw[:-1])
    with pytest.raises(_lib.JanusError):
        ops.GpuTensor(engine, _lib.DT_Q5_K, 2, 200, np.zeros(352, np.uint8))


def test_q6_k_gemv_matches_oracle(engine):
    n, k = 300, 1024
    raw = synth.random_q6_k(np.random.default_rng(5), n, k)
    w = ops.GpuTensor(engine, _lib.DT_Q6_K, n, k, raw, _lib.WEIGHT_FTZ_F16)
    x = np.random.default_rng(6).standard_normal(k, dtype=np.float32)
    y = torch.empty(n, device=DEV)
    ops.gemm_auto(engine, torch.from_numpy(x).to(DEV), w, y, 1, 1, k, n)
    want = O.gemm_auto(x, _lib.DT_Q6_K, raw, n, k)
    wf = w.dequant().cpu().numpy()
    bound = 2e-5 * (np.abs(wf) @ np.abs(x)) + 1e-30
    assert np.all(np.abs(y.cpu().numpy() - want) <= bound)


def _k_mixed(seed, block_type, ffn=1024):
    """2-layer Llama-3-shaped model: block matrices in block_type, attn_v and
    ffn_down in Q6_K, Q6_K LM head (the Q4_K_M / Q5_K_M recipe)."""
    spec = synth.make_model(seed, 512, 4, 1, ffn, 1024, 2, block_type, 1e-5, 500000.0,
                            embed_type=synth.F16, head_type=synth.Q6_K, down_type=synth.Q6_K)
    rng = np.random.default_rng(seed + 1)
    for i, t in enumerate(spec.tensors):
        if t.name.endswith("attn_v.weight"):
            spec.tensors[i] = synth.Tensor(t.name, synth.Q6_K, t.n, t.k, synth.random_q6_k(rng, t.n, t.k))
    return spec


@pytest.mark.parametrize("block_type", [synth.Q5_K, synth.Q4_K])
@pytest.mark.parametrize("act_dtype", [_lib.DT_F32, _lib.DT_F16])
def test_k_quant_mixed_model_matches_oracle(engine, block_type, act_dtype):
    spec = _k_mixed(21, block_type)
    prompt = np.random.default_rng(22).integers(0, spec.vocab, 12).tolist()
    ref = O.OracleModel(spec, 32, kv_f16=True)
    m = Model(engine, spec, max_seq_len=32, kv_dtype=_lib.DT_F16, act_dtype=act_dtype)
    worst = 0.0
    for p, t in enumerate(prompt):
        want = ref.forward(t, p)
        m.forward([t], [p])
        worst = max(worst, _rel_err(m.logits()[0], want))
    assert worst <= REL, worst
    m.close()


def test_q5_k_model_fused_and_batched_paths(engine):
    """All-Q5_K blocks take the fused single-sequence path (paired QKV and
    gate/up GEMVs with RMSNorm prologues) and the batched MFMA path; both
    must match the oracle and each other."""
    spec = synth.make_model(31, 512, 4, 1, 1024, 1000, 2, synth.Q5_K, 1e-5, 500000.0,
                            embed_type=synth.F16, head_type=synth.F16)
    rng = np.random.default_rng(32)
    lens = [6, 11, 9]
    prompts = [rng.integers(0, spec.vocab, n).tolist() for n in lens]
    singles = []
    for pr in prompts:
        m = Model(engine, spec, max_seq_len=32, kv_dtype=_lib.DT_F16, act_dtype=_lib.DT_F16)
        for p, t in enumerate(pr):
            m.forward([t], [p])
        singles.append(m.logits()[0])
        m.close()
    mb = Model(engine, spec, max_seq_len=32, max_batch=3, kv_dtype=_lib.DT_F16, act_dtype=_lib.DT_F16)
    for step in range(max(lens)):
        mb.forward([pr[min(step, len(pr) - 1)] for pr in prompts], [min(step, len(pr) - 1) for pr in prompts])
    out = mb.logits(3)
    for s in range(3):
        assert _rel_err(out[s], singles[s]) <= 1e-3
    ref = O.OracleModel(spec, 32, kv_f16=True)
    for p, t in enumerate(prompts[1]):
        want = ref.forward(t, p)
    assert _rel_err(singles[1], want) <= REL
    assert _rel_err(out[1], want) <= REL
    mb.close()


def _every_scale_byte(ggml_type, seed):
    """Q4_K / Q5_K bytes over 8 rows of 32 super-blocks in which scale byte i
    (bytes 4..15) of super-block b is (b + 97 i) % 256: every position takes
    every byte value once, so every 6-bit sc and m of every sub-block, with
    its top bits from the shared bytes of sub-blocks 4..7, is decoded."""
    n, k = 8, 32 * 256
    rng = np.random.default_rng(seed)
    bb = 144 if ggml_type == _lib.DT_Q4_K else 176
    nsb = n * k // 256
    raw = np.frombuffer(rng.bytes(nsb * bb), np.uint8).reshape(nsb, bb).copy()
    dd = np.abs(rng.standard_normal((nsb, 2), dtype=np.float32)) * np.float32(0.02 / 128)
    raw[:, 0:4] = synth.f16_bits(dd).view(np.uint8).reshape(nsb, 4)
    b = np.arange(nsb)[:, None]
    raw[:, 4:16] = ((b + 97 * np.arange(12)[None, :]) % 256).astype(np.uint8)
    return n, k, raw.reshape(-1)


@pytest.mark.parametrize("ggml_type", [_lib.DT_Q4_K, _lib.DT_Q5_K])
def test_k_scale_fields_every_byte_value(engine, ggml_type):
    """The upload rewrites the 12 scale bytes as one 24-bit field per chunk
    pair; dequantisation is bit-exact against the oracle's GGML decode
    (get_scale_min_k4) for every byte value in every position, and the M = 1
    product and the 4-row MFMA product stay within 2e-5 * sum |w x| of the
    f64 product over those weights."""
    n, k, raw = _every_scale_byte(ggml_type, 40 + ggml_type)
    w = ops.GpuTensor(engine, ggml_type, n, k, raw)
    got = w.dequant().cpu().numpy()
    want = O.dequant(ggml_type, raw, n, k)
    assert np.array_equal(got.reshape(-1).view(np.uint32), want.reshape(-1).view(np.uint32))
    wf = want.reshape(n, k).astype(np.float64)
    x = np.random.default_rng(7).standard_normal(k, dtype=np.float32)
    y = torch.empty(n, device=DEV)
    ops.gemm_auto(engine, torch.from_numpy(x).to(DEV), w, y, 1, 1, k, n)
    bound = 2e-5 * (np.abs(wf) @ np.abs(x.astype(np.float64))) + 1e-30
    assert np.all(np.abs(y.cpu().numpy() - wf @ x.astype(np.float64)) <= bound)
    a16 = torch.from_numpy(np.random.default_rng(8).standard_normal((4, k), dtype=np.float32)).to(torch.float16)
    c = torch.empty(4, n, device=DEV)
    ops.gemm_auto(engine, a16.to(DEV), w, c, 4, 1, k, n)
    xa = a16.float().numpy().astype(np.float64)
    bound = 2e-5 * (np.abs(xa) @ np.abs(wf).T) + 1e-30
    assert np.all(np.abs(c.cpu().numpy() - xa @ wf.T) <= bound)
