"""GPU parity of the small-M MFMA GEMM (janus_gemm_auto with 2..64 rows of
binary16 activations).

The reference has no correct quantised product for M > 1 (it hands quantised
bytes to its f16 GEMM, crates/janus-engine/src/compute/ops/quantized.rs:77-90),
so parity is the invariant "GEMM(M) == M stacked GEMV(1)": every row must
match the M=1 kernel on the same binary16 row, and both must match an f64
product of the bit-exact dequantised weights within
|y - y64| <= 2e-5 * sum_i |w_i x_i|   (exact products, fp32 accumulation).
"""
import numpy as np
import pytest
import torch

from janus_amd import ops, synth
from oracle import oracle as O

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
GEN = {2: synth.random_q4_0, 8: synth.random_q8_0, 12: synth.random_q4_k, 13: synth.random_q5_k}


def _weight(engine, ggml_type, n, k, seed):
    rng = np.random.default_rng(seed)
    if ggml_type in GEN:
        raw = GEN[ggml_type](rng, n, k)
    else:
        raw = synth.f16_bits(rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02))
    return raw, ops.GpuTensor(engine, ggml_type, n, k, raw)


def _acts(rows, k, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(rows, k, generator=g).to(torch.float16)


def _check_against_f64(y, wf, a16):
    x = a16.float().numpy().astype(np.float64)
    w = wf.astype(np.float64)
    ref = x @ w.T
    bound = 2e-5 * (np.abs(x) @ np.abs(w).T) + 1e-30
    err = np.abs(y.astype(np.float64) - ref)
    assert np.all(err <= bound), float(np.max(err / bound))


@pytest.mark.parametrize("ggml_type", [2, 8, 12, 13, 1])
@pytest.mark.parametrize("rows", [2, 7, 32, 33, 64])
@pytest.mark.parametrize("n,k", [(96, 256), (200, 512), (4096, 4096), (1024, 14336)])
def test_mfma_gemm_matches_stacked_gemv_and_f64(engine, ggml_type, rows, n, k):
    raw, w = _weight(engine, ggml_type, n, k, 100 + ggml_type + n)
    a16 = _acts(rows, k, rows + n)
    a = a16.to(DEV)
    c = torch.empty(rows, n, device=DEV)
    ops.gemm_auto(engine, a, w, c, rows, 1, k, n)
    stacked = torch.empty(rows, n, device=DEV)
    for r in range(rows):
        ops.gemm_auto(engine, a[r].contiguous(), w, stacked[r], 1, 1, k, n)
    torch.cuda.synchronize()
    got = c.cpu().numpy()
    wf = w.dequant().cpu().numpy()
    _check_against_f64(got, wf, a16)
    _check_against_f64(stacked.cpu().numpy(), wf, a16)


@pytest.mark.parametrize("ggml_type", [2, 8, 12, 13])
@pytest.mark.parametrize("rows", [32, 48, 64])
@pytest.mark.parametrize("n,k", [(6144, 4096), (4096, 14336)])
def test_pipelined_gemm_shapes_match_f64(engine, ggml_type, rows, n, k):
    """Shapes whose workgroups run several K passes take the cross-pass
    pipelined kernel (A double-buffered in LDS, next-pass weights in flight):
    one and two 32-row M tiles, every quantised format, K split over
    workgroups. Repeated calls are bitwise equal."""
    raw, w = _weight(engine, ggml_type, n, k, 300 + ggml_type + rows)
    a16 = _acts(rows, k, 7 * rows + n)
    a = a16.to(DEV)
    outs = []
    for _ in range(2):
        c = torch.empty(rows, n, device=DEV)
        ops.gemm_auto(engine, a, w, c, rows, 1, k, n)
        outs.append(c.cpu())
    assert torch.equal(outs[0], outs[1])
    _check_against_f64(outs[0].numpy(), w.dequant().cpu().numpy(), a16)


@pytest.mark.parametrize("ggml_type", [2, 8])
@pytest.mark.parametrize("rows", [32, 40])
def test_pipelined_gemm_ragged_k_and_partial_tile(engine, ggml_type, rows):
    """k = 4160 leaves a 64-wide last pass (K-tail chunks clamped, not computed)
    and n = 6176 leaves a last tile with one active row group of four (the
    others stream a real group and discard it)."""
    n, k = 6176, 4160
    raw, w = _weight(engine, ggml_type, n, k, 500 + ggml_type + rows)
    a16 = _acts(rows, k, 11 * rows)
    a = a16.to(DEV)
    c = torch.empty(rows, n, device=DEV)
    ops.gemm_auto(engine, a, w, c, rows, 1, k, n)
    torch.cuda.synchronize()
    _check_against_f64(c.cpu().numpy(), w.dequant().cpu().numpy(), a16)


@pytest.mark.parametrize("ggml_type", [2, 12])
def test_mfma_gemm_is_deterministic_under_split_k(engine, ggml_type):
    n, k, rows = 4096, 4096, 32          # few row tiles: the product is split over K
    _, w = _weight(engine, ggml_type, n, k, 7)
    a = _acts(rows, k, 3).to(DEV)
    outs = []
    for _ in range(3):
        c = torch.empty(rows, n, device=DEV)
        ops.gemm_auto(engine, a, w, c, rows, 1, k, n)
        outs.append(c.cpu())
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[1], outs[2])


def test_mfma_gemm_residual_and_f16_output(engine):
    n, k, rows = 640, 1024, 5
    _, w = _weight(engine, 2, n, k, 21)
    a16 = _acts(rows, k, 4)
    a = a16.to(DEV)
    base = torch.empty(rows, n, device=DEV)
    ops.gemm_auto(engine, a, w, base, rows, 1, k, n)
    resid = torch.randn(rows, n, device=DEV)
    out = torch.empty(rows, n, device=DEV)
    ops.gemm_residual(engine, a, w, resid, out, rows)
    torch.cuda.synchronize()
    assert torch.equal(out, base + resid)
    inplace = resid.clone()
    ops.gemm_residual(engine, a, w, inplace, inplace, rows)
    assert torch.equal(inplace, base + resid)
    h = torch.empty(rows, n, device=DEV, dtype=torch.float16)
    ops.gemm_auto(engine, a, w, h, rows, 1, k, n)
    assert torch.equal(h, base.to(torch.float16))


def test_mfma_gemm_q4_0_odd_block_count(engine):
    # k / 32 odd: the last 64-wide tile chunk carries one zero block
    n, k, rows = 70, 96, 3
    raw, w = _weight(engine, 2, n, k, 5)
    a16 = _acts(rows, k, 6)
    c = torch.empty(rows, n, device=DEV)
    ops.gemm_auto(engine, a16.to(DEV), w, c, rows, 1, k, n)
    torch.cuda.synchronize()
    _check_against_f64(c.cpu().numpy(), O.dequant(2, raw, n, k), a16)


def test_f32_activations_keep_the_reference_dtype(engine):
    # f32 rows go through the M=1 kernels row by row: bit-identical to single calls
    n, k, rows = 128, 512, 3
    _, w = _weight(engine, 8, n, k, 8)
    a = torch.randn(rows, k, device=DEV)
    c = torch.empty(rows, n, device=DEV)
    ops.gemm_auto(engine, a, w, c, rows, 1, k, n)
    for r in range(rows):
        y = torch.empty(n, device=DEV)
        ops.gemm_auto(engine, a[r].contiguous(), w, y, 1, 1, k, n)
        assert torch.equal(y, c[r])
