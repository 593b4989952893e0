"""GPU parity of weight upload, dequantisation and the matrix products.

- janus_weight_dequant is bit-exact against the oracle's dequantisation for
  every format, including subnormal and inf/nan binary16 scales.
- GEMV outputs match the oracle (the reference's accumulation order) and an
  f64 product of the dequantised weights within
  |y - y64| <= 1e-5 * sum_i |w_i x_i|   (fp32 accumulation, any order).
- Config-2 shapes (Llama-3-8B Q4_0 GEMV, x fp16 N(0,1), fp16 output) are
  checked against a float64 GPU product of the dequantised weights.
"""
import numpy as np
import pytest
import torch

from janus_amd import ops, synth
from oracle import oracle as O

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
GEN = {2: synth.random_q4_0, 8: synth.random_q8_0, 12: synth.random_q4_k, 13: synth.random_q5_k}


def _weight(engine, ggml_type, n, k, seed, flags=0):
    rng = np.random.default_rng(seed)
    if ggml_type in GEN:
        raw = GEN[ggml_type](rng, n, k)
    elif ggml_type == 1:
        raw = synth.f16_bits(rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02))
    else:
        raw = rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02)
    return raw, ops.GpuTensor(engine, ggml_type, n, k, raw, flags)


def _bits(a):
    return np.ascontiguousarray(a, np.float32).reshape(-1).view(np.uint32)


@pytest.mark.parametrize("ggml_type,flags", [(2, 0), (8, 0), (12, 0), (12, 1), (13, 0), (13, 1), (1, 0), (1, 1), (0, 1)])
def test_dequant_bit_exact(engine, ggml_type, flags):
    n, k = 24, 512
    raw, w = _weight(engine, ggml_type, n, k, 10 + ggml_type, flags)
    if ggml_type in (2, 8):   # plant subnormal / inf / nan scales
        bb = 18 if ggml_type == 2 else 34
        r = raw.reshape(-1, bb)
        r[:5, :2] = np.array([0x0001, 0x03FF, 0x7C00, 0xFC00, 0x7E01], np.uint16).view(np.uint8).reshape(-1, 2)
        w = ops.GpuTensor(engine, ggml_type, n, k, raw, flags)
    if ggml_type in (12, 13):
        r = raw.reshape(-1, 144 if ggml_type == 12 else 176)
        r[0, 0:2] = np.array([0x0005], np.uint16).view(np.uint8)
        w = ops.GpuTensor(engine, ggml_type, n, k, raw, flags)
    got = w.dequant().cpu().numpy()
    want = O.dequant(ggml_type, raw, n, k, ftz=bool(flags))
    nan = np.isnan(want.reshape(-1))
    assert np.array_equal(_bits(got)[~nan], _bits(want)[~nan])


def _bound(wf, x):
    return 1e-5 * (np.abs(wf.astype(np.float64)) @ np.abs(x.astype(np.float64))) + 1e-30


# the reference decodes F16 weights and Q4_K d/dmin with f16_to_f32_safe
FTZ = {0: 1, 1: 1, 2: 0, 8: 0, 12: 1, 13: 0}


@pytest.mark.parametrize("ggml_type", [2, 8, 12, 13, 1])
@pytest.mark.parametrize("n,k", [(1, 256), (7, 256), (64, 256), (130, 512), (256, 4096), (96, 14336)])
def test_gemv_f32_matches_oracle(engine, ggml_type, n, k):
    raw, w = _weight(engine, ggml_type, n, k, n + k, FTZ[ggml_type])
    rng = np.random.default_rng(k)
    x = rng.standard_normal(k, dtype=np.float32)
    y = torch.empty(n, dtype=torch.float32, device=DEV)
    ops.gemm_auto(engine, torch.from_numpy(x).to(DEV), w, y, 1, 1, k, n)
    got = y.cpu().numpy()
    want = O.gemm_auto(x, ggml_type, raw, n, k)
    wf = O.dequant(ggml_type, raw, n, k, ftz=bool(FTZ[ggml_type]))
    y64 = O.gemv_f64(wf, x)
    b = _bound(wf, x)
    assert np.all(np.abs(got - y64) <= b)
    assert np.all(np.abs(got - want) <= 2 * b)


@pytest.mark.parametrize("ggml_type", [2, 8, 12, 13, 1])
@pytest.mark.parametrize("n,k", [(33, 256), (512, 4096), (64, 11008), (1003, 8704), (1003, 4096), (8200, 4096),
                                 (2500, 4096)])
def test_gemv_f16_activations(engine, ggml_type, n, k):
    """Every binary16 product of 64+ units per row runs the LDS-staged kernel.
    (1003, 8704): five units per lane,
    single-buffered (Q4_0 / Q8_0 with x requested first, K-quants re-reading x
    from LDS; F16 rows of 1088 units take the register kernel), a last
    workgroup with five idle wavefronts that stream a real row group and
    discard it. (1003, 4096): F16 with eight units per lane on the
    double-buffered body, five idle wavefronts; the quantised formats two
    units per lane, one row per step (Q4_0 in one 512-thread workgroup per
    CU, the K-quants and Q8_0 in two), idle wavefronts in the last workgroup.
    (8200, 4096): 8200 row groups of one row (quantised formats, 512-thread
    workgroups two per CU), whose persistent grid gives wavefronts a second
    and third group. (2500, 4096): Q4_0 with ten groups per CU on a 256-CU
    device, one 512-thread workgroup per CU whose wavefronts own one or two
    groups."""
    _check_gemv_f16(engine, ggml_type, n, k)


def _check_gemv_f16(engine, ggml_type, n, k):
    raw, w = _weight(engine, ggml_type, n, k, 3 * n + k, FTZ[ggml_type])
    rng = np.random.default_rng(n)
    xh = rng.standard_normal(k).astype(np.float16)
    y = torch.empty(n, dtype=torch.float16, device=DEV)
    ops.gemm_auto(engine, torch.from_numpy(xh).to(DEV), w, y, 1, 1, k, n)
    got = y.float().cpu().numpy()
    x = xh.astype(np.float32)
    wf = O.dequant(ggml_type, raw, n, k, ftz=bool(FTZ[ggml_type]))
    y64 = O.gemv_f64(wf, x)
    # fp32 accumulation then one binary16 rounding of the output
    assert np.all(np.abs(got - y64) <= _bound(wf, x) + np.abs(y64) * 2.0 ** -11 + 2.0 ** -24)


@pytest.fixture(scope="module")
def wide_engine():
    """A context whose LDS-staged GEMV takes 1024-thread workgroups wherever
    the body fits (JANUS_GEMV_LDS_THREADS=1024 is read when the context is
    made)."""
    import os
    from janus_amd.ops import ComputeEngine
    old = os.environ.get("JANUS_GEMV_LDS_THREADS")
    os.environ["JANUS_GEMV_LDS_THREADS"] = "1024"
    try:
        eng = ComputeEngine(0)
    finally:
        if old is None:
            del os.environ["JANUS_GEMV_LDS_THREADS"]
        else:
            os.environ["JANUS_GEMV_LDS_THREADS"] = old
    yield eng
    eng.sync()
    eng.close()


@pytest.mark.parametrize("ggml_type", [2, 1])
@pytest.mark.parametrize("n,k", [(1003, 4096), (8200, 4096)])
def test_gemv_f16_activations_1024_thread_workgroups(wide_engine, ggml_type, n, k):
    """1024-thread workgroups for every LDS-staged body that fits them (Q4_0
    and F16 rows of two units per lane), also where the default takes 512:
    a last workgroup with idle wavefronts, and a persistent grid."""
    _check_gemv_f16(wide_engine, ggml_type, n, k if ggml_type == 2 else k // 4)


@pytest.mark.parametrize("n,threads", [(2500, None), (3000, None), (2500, "640"), (3000, "768")])
def test_gemv_f16_rows_one_workgroup_per_cu(engine, monkeypatch, n, threads):
    """F16 rows of two units per lane (k = 1024), one row per step: 2500 and
    3000 groups run one 512-thread workgroup per CU on a 256-CU device (its
    wavefronts own one or two groups); with JANUS_GEMV_LDS_THREADS at 640 or
    768, one such workgroup per CU with about one group per wavefront."""
    if threads is None:
        _check_gemv_f16(engine, 1, n, 1024)
        return
    from janus_amd.ops import ComputeEngine
    monkeypatch.setenv("JANUS_GEMV_LDS_THREADS", threads)
    monkeypatch.setenv("JANUS_GEMV_LDS_WPC", str(int(threads) // 64))
    eng = ComputeEngine(0)
    try:
        _check_gemv_f16(eng, 1, n, 1024)
    finally:
        eng.sync()
        eng.close()


def test_gemv_f16_odd_k_generic_path(engine):
    # ffn_down of the tiny model: k = 688 is not a multiple of 32 -> F16 path
    n, k = 256, 688
    raw, w = _weight(engine, 0, n, k, 77, flags=1)
    x = np.random.default_rng(1).standard_normal(k, dtype=np.float32)
    y = torch.empty(n, dtype=torch.float32, device=DEV)
    ops.gemm_auto(engine, torch.from_numpy(x).to(DEV), w, y, 1, 1, k, n)
    want = O.gemm_auto(x, 0, raw, n, k)
    wf = O.dequant(0, raw, n, k, ftz=True)
    assert np.all(np.abs(y.cpu().numpy() - want) <= 2 * _bound(wf, x))


def test_gemv_residual_epilogue(engine):
    n, k = 4096, 4096
    raw, w = _weight(engine, 2, n, k, 5)
    rng = np.random.default_rng(2)
    x = torch.from_numpy(rng.standard_normal(k, dtype=np.float32)).to(DEV)
    r = torch.from_numpy(rng.standard_normal(n, dtype=np.float32)).to(DEV)
    plain = torch.empty(n, device=DEV)
    ops.gemm_auto(engine, x, w, plain, 1, 1, k, n)
    out = r.clone()
    ops.gemm_residual(engine, x, w, out, out, 1)   # residual aliases the output
    torch.cuda.synchronize()
    assert torch.equal(out, plain + r)


@pytest.mark.parametrize("n,k", [(14336, 4096), (4096, 14336), (4096, 4096)])
def test_config2_q4_0_gemv_full_shapes(engine, n, k):
    """benchmark configuration 2: Q4_0, x fp16 N(0,1), fp32 accumulate, fp16 output."""
    rng = np.random.default_rng(2)
    raw = synth.random_q4_0(rng, n, k)
    w = ops.GpuTensor(engine, 2, n, k, raw)
    xh = torch.from_numpy(rng.standard_normal(k).astype(np.float16)).to(DEV)
    y = torch.empty(n, dtype=torch.float16, device=DEV)
    ops.gemm_auto(engine, xh, w, y, 1, 1, k, n)
    wf = w.dequant()
    ref = (wf.double() @ xh.double()).float()
    bound = 1e-5 * (wf.abs().double() @ xh.abs().double()).float() + ref.abs() * 2.0 ** -11 + 2.0 ** -24
    assert bool(((y.float() - ref).abs() <= bound).all())
    del wf


def test_dims_must_match_weight(engine):
    _, w = _weight(engine, 2, 64, 256, 1)
    x = torch.zeros(256, device=DEV)
    y = torch.zeros(64, device=DEV)
    with pytest.raises(ops.JanusError) as e:
        ops.gemm_auto(engine, x, w, y, 1, 1, 256, 65)
    assert e.value.status == 2


@pytest.mark.parametrize("ggml_type", [2, 8, 12, 13, 1])
@pytest.mark.parametrize("xdt,m", [(torch.float16, 1), (torch.float32, 1), (torch.float16, 8)])
def test_gemv_error_is_unbiased_across_rows(engine, ggml_type, xdt, m):
    """The products' rounding errors are independent across rows, as the
    reference's per-element fp32 sums are: over 4096 rows of one product the
    mean of (y - y64) / sum|w x| stays a small fraction of its spread, and the
    spread stays at fp32 rounding level. An error shared by every row (a
    biased instruction, an offset term rounded once per block and reused by
    all rows) is what amplifies through the layers; the binary16 path once
    measured a mean of -1.8e-7 there (v_dot2_f32_f16 on subnormal operands).
    m = 8: the small-M MFMA product, per activation row."""
    n, k = 4096, 4096
    raw, w = _weight(engine, ggml_type, n, k, 77 + ggml_type, FTZ[ggml_type])
    wf = w.dequant().double()
    rng = np.random.default_rng(ggml_type)
    means, rmss = [], []
    for _ in range(3):
        x = torch.from_numpy(rng.standard_normal((m, k)).astype(np.float16).astype(np.float32)).to(DEV)
        y = torch.empty(m, n, device=DEV)
        ops.gemm_auto(engine, x.to(xdt), w, y, m, 1, k, n)
        xd = x.double()
        e = (y.double() - xd @ wf.T) / (xd.abs() @ wf.abs().T)
        means.extend(e.mean(dim=1).tolist())
        rmss.extend(e.pow(2).mean(dim=1).sqrt().tolist())
    mean, rms = float(np.mean(np.abs(means))), float(np.mean(rmss))
    assert rms < 2e-8, (means, rmss)
    assert mean < 0.25 * rms + 1e-10, (means, rmss)
