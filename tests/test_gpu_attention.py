"""GPU parity of split-K decode attention.

Against the oracle (attention.wgsl:62-186 + softmax.wgsl:18-51 restated)
with f32 K/V, and against the oracle fed binary16-rounded K/V for an f16
cache; the invariant split-K == single pass is covered by lengths that span
one and many splits. The ragged case packs sequences via a prefix-sum
offset table into one launch (benchmark configuration 4 shape, reduced lengths).
"""
import numpy as np
import pytest
import torch

from janus_amd import ops
from oracle import oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _close(got, want):
    assert np.allclose(got, want, rtol=2e-5, atol=2e-6), np.max(np.abs(got - want))


@pytest.mark.parametrize("kv", [torch.float32, torch.float16])
@pytest.mark.parametrize("H,KVH,D", [(4, 2, 64), (32, 8, 128), (32, 32, 128), (8, 1, 64), (64, 8, 128)])
@pytest.mark.parametrize("L", [1, 63, 64, 65, 700, 3000])
def test_attention_single_sequence(engine, kv, H, KVH, D, L):
    rng = np.random.default_rng(L * H + D)
    q = rng.standard_normal(H * D).astype(np.float32)
    k = rng.standard_normal((L, KVH, D)).astype(np.float32)
    v = rng.standard_normal((L, KVH, D)).astype(np.float32)
    if kv == torch.float16:
        k, v = k.astype(np.float16).astype(np.float32), v.astype(np.float16).astype(np.float32)
    cap = L + 5
    kc = torch.zeros(cap, KVH, D, device=DEV, dtype=kv)
    vc = torch.zeros_like(kc)
    kc[:L] = torch.from_numpy(k).to(DEV, kv)
    vc[:L] = torch.from_numpy(v).to(DEV, kv)
    out = torch.empty(H * D, device=DEV)
    ops.compute_attention(engine, torch.from_numpy(q).to(DEV), kc, vc, out, 1, L, cap, H, KVH, D)
    _close(out.cpu().numpy(), O.attention(q, k, v, H, KVH, D))


def test_attention_zero_length_is_zero(engine):
    H, KVH, D = 4, 2, 64
    kc = torch.randn(8, KVH, D, device=DEV)
    out = torch.full((H * D,), 7.0, device=DEV)
    ops.compute_attention(engine, torch.randn(H * D, device=DEV), kc, kc, out, 1, 0, 8, H, KVH, D)
    assert torch.count_nonzero(out).item() == 0


@pytest.mark.parametrize("kv", [torch.float32, torch.float16])
def test_attention_ragged_prefix_sum_offsets(engine, kv):
    H, KVH, D = 32, 8, 128
    rng = np.random.default_rng(44)
    lens = rng.integers(1, 1500, 16).tolist()
    lens[3] = 1
    lens[7] = 64
    offs = np.concatenate([[0], np.cumsum(lens)[:-1]]).astype(np.int32)
    total = int(sum(lens))
    k = rng.standard_normal((total, KVH, D)).astype(np.float32)
    v = rng.standard_normal((total, KVH, D)).astype(np.float32)
    if kv == torch.float16:
        k, v = k.astype(np.float16).astype(np.float32), v.astype(np.float16).astype(np.float32)
    q = rng.standard_normal((16, H * D)).astype(np.float32)
    kc, vc = torch.from_numpy(k).to(DEV, kv), torch.from_numpy(v).to(DEV, kv)
    out = torch.empty(16, H * D, device=DEV)
    ops.compute_attention(engine, torch.from_numpy(q).to(DEV), kc, vc, out, 16, 0, max(lens), H, KVH, D,
                          row_base=torch.from_numpy(offs).to(DEV), seq_lens=torch.tensor(lens, dtype=torch.int32,
                                                                                          device=DEV),
                          max_len_hint=max(lens))
    got = out.cpu().numpy()
    for b in range(16):
        sl = slice(offs[b], offs[b] + lens[b])
        _close(got[b], O.attention(q[b], k[sl], v[sl], H, KVH, D))


@pytest.mark.parametrize("H,KVH,D", [(8, 1, 64), (32, 32, 128), (64, 8, 128), (8, 4, 64)])
def test_attention_ragged_task_list_edges(engine, H, KVH, D):
    """Binary16 ragged batches run as a device-built task list: empty
    sequences must come out as zeros, and lengths on either side of a piece
    boundary (planned piece length is a multiple of 16) must merge exactly."""
    rng = np.random.default_rng(H * 7 + D)
    lens = [0, 1, 15, 16, 17, 255, 256, 257, 1023, 1025, 2500, 3]
    B = len(lens)
    offs = np.concatenate([[0], np.cumsum(lens)[:-1]]).astype(np.int32)
    total = int(sum(lens))
    k = rng.standard_normal((total, KVH, D)).astype(np.float16).astype(np.float32)
    v = rng.standard_normal((total, KVH, D)).astype(np.float16).astype(np.float32)
    q = rng.standard_normal((B, H * D)).astype(np.float32)
    kc = torch.from_numpy(k).to(DEV, torch.float16)
    vc = torch.from_numpy(v).to(DEV, torch.float16)
    out = torch.full((B, H * D), 7.0, device=DEV)
    ops.compute_attention(engine, torch.from_numpy(q).to(DEV), kc, vc, out, B, 0, max(lens), H, KVH, D,
                          row_base=torch.from_numpy(offs).to(DEV),
                          seq_lens=torch.tensor(lens, dtype=torch.int32, device=DEV), max_len_hint=max(lens))
    got = out.cpu().numpy()
    for b in range(B):
        if lens[b] == 0:
            assert np.count_nonzero(got[b]) == 0
            continue
        sl = slice(offs[b], offs[b] + lens[b])
        _close(got[b], O.attention(q[b], k[sl], v[sl], H, KVH, D))


def test_attention_large_q_prescale(engine):
    """q components beyond the binary16 range are scaled by a power of two
    before the MFMA split; the result must still match the f64 oracle."""
    H, KVH, D = 32, 8, 128
    rng = np.random.default_rng(9)
    lens = [40, 300]
    offs = np.array([0, 40], np.int32)
    # scores stay O(1) (the tolerance is that of fp32 scores of moderate size)
    k = (rng.standard_normal((340, KVH, D)) * 2e-5).astype(np.float16).astype(np.float32)
    v = rng.standard_normal((340, KVH, D)).astype(np.float16).astype(np.float32)
    q = (rng.standard_normal((2, H * D)) * 2e5).astype(np.float32)
    out = torch.empty(2, H * D, device=DEV)
    ops.compute_attention(engine, torch.from_numpy(q).to(DEV), torch.from_numpy(k).to(DEV, torch.float16),
                          torch.from_numpy(v).to(DEV, torch.float16), out, 2, 0, 300, H, KVH, D,
                          row_base=torch.from_numpy(offs).to(DEV),
                          seq_lens=torch.tensor(lens, dtype=torch.int32, device=DEV), max_len_hint=300)
    got = out.cpu().numpy()
    for b in range(2):
        sl = slice(offs[b], offs[b] + lens[b])
        # scores reach ~10 here, where fp32 arithmetic itself (a numpy fp32
        # restatement) is off by ~6e-6: the bound is set at that level; an
        # overflow of the binary16 q parts would give inf / nan instead
        want = O.attention(q[b], k[sl], v[sl], H, KVH, D)
        assert np.allclose(got[b], want, rtol=1e-4, atol=1e-5), np.max(np.abs(got[b] - want))
