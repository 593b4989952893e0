"""The reference's own known-answer tests, restated against the oracle.

Sources (crates/janus-engine/src/compute/ops/tests.rs):
  :104-136  f16 GEMV [1..6]x[1,2,3] = [14, 32] (eps 1e-3)
  :138-193  f16 GEMM A[2x3] . B[2x3]^T = [58, 64, 139, 154] (eps 1e-2)
  :274-331  add [11,22,33,44], mul [10,40,90,160] (eps 1e-5)
  :333-390  RoPE at position 0 is the identity; table row 1 for hd=4, base 1e4
            = (0.5403023, 0.84147096, 0.99995, 0.009999833)
  :392-428  argmax([-1, .5, 4.2, 3.9, 2]) = 2
  :195-272  silu / rmsnorm of [1, -1, .5, -.5] are finite
"""
import numpy as np

from oracle import oracle as O


def test_f16_gemv_kat():
    w = O.f32_to_f16_rne([1, 2, 3, 4, 5, 6])
    x = np.array([1, 2, 3], np.float32)
    y = np.empty(2, np.float32)
    O.lib().jo_gemm_f16(x, w, y, 1, 1, 3, 2)
    assert np.allclose(y, [14, 32], atol=1e-3)


def test_f16_gemm_kat():
    a = np.array([1, 2, 3, 4, 5, 6], np.float32)
    b = O.f32_to_f16_rne([7, 9, 11, 8, 10, 12])
    c = np.empty(4, np.float32)
    O.lib().jo_gemm_f16(a, b, c, 1, 2, 3, 2)
    assert np.allclose(c, [58, 64, 139, 154], atol=1e-2)


def test_add_mul_kat():
    a = np.array([1, 2, 3, 4], np.float32)
    b = np.array([10, 20, 30, 40], np.float32)
    assert np.allclose(O.add(a, b), [11, 22, 33, 44], atol=1e-5)
    assert np.allclose(O.mul(a, b), [10, 40, 90, 160], atol=1e-5)


def test_rope_kat():
    table = np.array([1, 0, 1, 0, 0.5403023, 0.84147096, 0.99995, 0.009999833], np.float32)
    x = np.array([1, 0, 1, 0], np.float32)
    assert np.allclose(O.rope(x, table, 1, 4, 0), x, atol=1e-4)
    t = O.rope_table(2, 4, 10000.0)
    assert np.allclose(t, table, atol=1e-6)


def test_argmax_kat():
    l = np.array([-1.0, 0.5, 4.2, 3.9, 2.0], np.float32)
    assert O.argmax_wgsl(l) == 2
    assert O.argmax_last(l) == 2


def test_silu_rmsnorm_finite_kat():
    x = np.array([1.0, -1.0, 0.5, -0.5], np.float32)
    assert np.isfinite(O.silu(x)).all()
    assert np.isfinite(O.rmsnorm(x, np.ones(4, np.float32), 1e-5)).all()
