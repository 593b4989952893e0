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


@pytest.mark.parametrize("H,KVH,D", [(32, 8, 128), (32, 32, 128), (8, 1, 64)])
@pytest.mark.parametrize("L,hint", [(65, 256), (300, 512), (700, 1024), (1500, 2048), (3000, 8192)])
def test_attention_planned_for_a_longer_length(engine, H, KVH, D, L, hint):
    """Captured decode steps plan attention for the length bucket above the
    live context: the length read from the device, the plan made for
    max_len_hint (one workgroup per head, per-query-head splits or KV-head
    splits with a merge), fp16 cache, against the oracle."""
    rng = np.random.default_rng(L + H + D)
    q = rng.standard_normal(H * D).astype(np.float32)
    k = rng.standard_normal((L, KVH, D)).astype(np.float16).astype(np.float32)
    v = rng.standard_normal((L, KVH, D)).astype(np.float16).astype(np.float32)
    kc = torch.zeros(hint, KVH, D, device=DEV, dtype=torch.float16)
    vc = torch.zeros_like(kc)
    kc[:L] = torch.from_numpy(k).to(DEV, torch.float16)
    vc[:L] = torch.from_numpy(v).to(DEV, torch.float16)
    lens = torch.tensor([L], dtype=torch.int32, device=DEV)
    out = torch.empty(H * D, device=DEV)
    ops.compute_attention(engine, torch.from_numpy(q).to(DEV), kc, vc, out, 1, 0, hint, H, KVH, D, seq_lens=lens,
                          max_len_hint=hint)
    _close(out.cpu().numpy(), O.attention(q, k, v, H, KVH, D))


@pytest.mark.parametrize("kv", [torch.float32, torch.float16])
@pytest.mark.parametrize("B", [2, 4, 8])
@pytest.mark.parametrize("hint", [1024, 2048])
def test_attention_small_batches_planned_lengths(engine, kv, B, hint):
    """2, 4 and 8 sequences of 32 query / 8 KV heads, lengths up to the
    plan's length (as in a captured step's bucket). Up to 1024 positions the
    per-query-head launch: one workgroup per head when 4 or 8 sequences fill
    half the CUs, splits with the merge kernel for 2. Beyond 1024 the KV-head
    splits (f32 cache) or the task list (fp16 cache). Against the oracle."""
    H, KVH, D = 32, 8, 128
    rng = np.random.default_rng(B * 10 + hint)
    lens = rng.integers(hint // 2 + 1, hint + 1, B).tolist()
    lens[0] = hint
    lens[-1] = hint // 2 + 1
    offs = np.concatenate([[0], np.cumsum(lens)[:-1]]).astype(np.int32)
    total = int(sum(lens))
    k = rng.standard_normal((total, KVH, D)).astype(np.float32)
    v = rng.standard_normal((total, KVH, D)).astype(np.float32)
    if kv == torch.float16:
        k, v = k.astype(np.float16).astype(np.float32), v.astype(np.float16).astype(np.float32)
    q = rng.standard_normal((B, H * D)).astype(np.float32)
    out = torch.full((B, H * D), 7.0, device=DEV)
    ops.compute_attention(engine, torch.from_numpy(q).to(DEV), torch.from_numpy(k).to(DEV, kv),
                          torch.from_numpy(v).to(DEV, kv), out, B, 0, hint, H, KVH, D,
                          row_base=torch.from_numpy(offs).to(DEV),
                          seq_lens=torch.tensor(lens, dtype=torch.int32, device=DEV), max_len_hint=hint)
    got = out.cpu().numpy()
    for b in range(B):
        sl = slice(offs[b], offs[b] + lens[b])
        _close(got[b], O.attention(q[b], k[sl], v[sl], H, KVH, D))


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


@pytest.fixture(scope="module")
def rows_engine():
    """A context whose planner takes the row-streaming kernel whenever the
    shape allows it (JANUS_ATTN_ROWS=1 is read when the context is made)."""
    import os
    from janus_amd.ops import ComputeEngine
    old = os.environ.get("JANUS_ATTN_ROWS")
    os.environ["JANUS_ATTN_ROWS"] = "1"
    try:
        eng = ComputeEngine(0)
    finally:
        if old is None:
            del os.environ["JANUS_ATTN_ROWS"]
        else:
            os.environ["JANUS_ATTN_ROWS"] = old
    yield eng
    eng.sync()
    eng.close()


def _ragged_f16(rng, lens, H, KVH, D, qscale=1.0):
    offs = np.concatenate([[0], np.cumsum(lens)[:-1]]).astype(np.int32)
    total = max(int(sum(lens)), 1)
    k = rng.standard_normal((total, KVH, D)).astype(np.float16).astype(np.float32)
    v = rng.standard_normal((total, KVH, D)).astype(np.float16).astype(np.float32)
    q = (rng.standard_normal((len(lens), H * D)) * qscale).astype(np.float32)
    dev = dict(q=torch.from_numpy(q).to(DEV), kc=torch.from_numpy(k).to(DEV, torch.float16),
               vc=torch.from_numpy(v).to(DEV, torch.float16), offs=torch.from_numpy(offs).to(DEV),
               lens=torch.tensor(lens, dtype=torch.int32, device=DEV))
    return q, k, v, offs, dev


def _run_ragged(eng, dev, lens, H, KVH, D):
    B = len(lens)
    out = torch.full((B, H * D), 7.0, device=DEV)
    mx = max(max(lens), 1)
    ops.compute_attention(eng, dev["q"], dev["kc"], dev["vc"], out, B, 0, mx, H, KVH, D, row_base=dev["offs"],
                          seq_lens=dev["lens"], max_len_hint=mx)
    return out.cpu().numpy()


@pytest.mark.parametrize("H,KVH,D", [(32, 8, 128), (16, 8, 128), (8, 8, 128), (32, 4, 128), (16, 4, 128),
                                     (4, 4, 128)])
def test_attention_rows_ragged_edges(rows_engine, H, KVH, D):
    """Row streaming (whole cache rows of a 16-position block through LDS,
    workgroup ranges of blocks across sequences): empty sequences give zeros,
    and lengths on either side of block and range boundaries match the f64
    oracle, including sequences split over several workgroups and runs of
    one-block sequences inside one workgroup."""
    rng = np.random.default_rng(H * 11 + KVH)
    lens = [0, 1, 15, 16, 17, 255, 256, 257, 1023, 1025, 2500, 3, 0, 16, 1, 31]
    q, k, v, offs, dev = _ragged_f16(rng, lens, H, KVH, D)
    got = _run_ragged(rows_engine, dev, lens, H, KVH, D)
    for b in range(len(lens)):
        if lens[b] == 0:
            assert np.count_nonzero(got[b]) == 0
            continue
        sl = slice(offs[b], offs[b] + lens[b])
        _close(got[b], O.attention(q[b], k[sl], v[sl], H, KVH, D))


@pytest.mark.parametrize("lens_kind", ["short64", "mixed64", "two_long"])
def test_attention_rows_batches(rows_engine, lens_kind):
    """Row streaming at the batch limits: 64 one-block sequences (every
    block starts a segment), 64 mixed lengths, and two long sequences (each
    spread over many workgroups, merged)."""
    H, KVH, D = 32, 8, 128
    rng = np.random.default_rng({"short64": 1, "mixed64": 2, "two_long": 3}[lens_kind])
    if lens_kind == "short64":
        lens = rng.integers(1, 17, 64).tolist()
    elif lens_kind == "mixed64":
        lens = rng.integers(0, 2000, 64).tolist()
    else:
        lens = [6000, 4500]
    q, k, v, offs, dev = _ragged_f16(rng, lens, H, KVH, D)
    got = _run_ragged(rows_engine, dev, lens, H, KVH, D)
    for b in range(len(lens)):
        if lens[b] == 0:
            assert np.count_nonzero(got[b]) == 0
            continue
        sl = slice(offs[b], offs[b] + lens[b])
        _close(got[b], O.attention(q[b], k[sl], v[sl], H, KVH, D))


def test_attention_rows_large_q_prescale(rows_engine):
    """q beyond the binary16 range through the row-streaming kernel (q is
    staged through LDS there): power-of-two prescale as in the other kernels."""
    H, KVH, D = 32, 8, 128
    rng = np.random.default_rng(19)
    lens = [40, 300, 17]
    offs = np.array([0, 40, 340], np.int32)
    k = (rng.standard_normal((357, KVH, D)) * 2e-5).astype(np.float16).astype(np.float32)
    v = rng.standard_normal((357, KVH, D)).astype(np.float16).astype(np.float32)
    q = (rng.standard_normal((3, H * D)) * 2e5).astype(np.float32)
    out = torch.empty(3, H * D, device=DEV)
    ops.compute_attention(rows_engine, torch.from_numpy(q).to(DEV), torch.from_numpy(k).to(DEV, torch.float16),
                          torch.from_numpy(v).to(DEV, torch.float16), out, 3, 0, 300, H, KVH, D,
                          row_base=torch.from_numpy(offs).to(DEV),
                          seq_lens=torch.tensor(lens, dtype=torch.int32, device=DEV), max_len_hint=300)
    got = out.cpu().numpy()
    for b in range(3):
        sl = slice(offs[b], offs[b] + lens[b])
        want = O.attention(q[b], k[sl], v[sl], H, KVH, D)
        assert np.allclose(got[b], want, rtol=1e-4, atol=1e-5), np.max(np.abs(got[b] - want))


def test_attention_rows_matches_default_plan_at_config4_shape(engine, rows_engine):
    """At the 32-sequence benchmark shape the default planner and the forced
    row-streaming plan agree to fp32 rounding (different split points)."""
    H, KVH, D = 32, 8, 128
    rng = np.random.default_rng(32)
    lens = rng.integers(1024, 4097, 32).tolist()
    q, k, v, offs, dev = _ragged_f16(rng, lens, H, KVH, D)
    a = _run_ragged(engine, dev, lens, H, KVH, D)
    b = _run_ragged(rows_engine, dev, lens, H, KVH, D)
    assert np.allclose(a, b, rtol=2e-5, atol=2e-6), np.max(np.abs(a - b))
    for i in (0, 17, 31):
        sl = slice(offs[i], offs[i] + lens[i])
        _close(b[i], O.attention(q[i], k[sl], v[sl], H, KVH, D))


def test_attention_rows_merge_ignores_stale_workspace(rows_engine):
    """The merge of a sequence split over several workgroups reads only
    partials written by the same launch. The first launch leaves non-finite
    partials in workgroup 0's first slot (its first sequence has infinite V
    and spans several workgroups); in the second, the first sequence lies
    inside workgroup 0 (so that slot is not rewritten) while the next one is
    split over fewer than 32 segments, whose merge has idle lanes. Every
    output must be finite and equal the oracle."""
    H, KVH, D = 32, 8, 128
    rng = np.random.default_rng(77)
    lens = [2000, 2000, 500]
    q, k, v, offs, dev = _ragged_f16(rng, lens, H, KVH, D)
    dev["vc"][: lens[0]] = float("inf")
    _run_ragged(rows_engine, dev, lens, H, KVH, D)
    lens = [1, 3000, 3000]
    q, k, v, offs, dev = _ragged_f16(rng, lens, H, KVH, D)
    got = _run_ragged(rows_engine, dev, lens, H, KVH, D)
    assert np.isfinite(got).all()
    for b in range(len(lens)):
        sl = slice(offs[b], offs[b] + lens[b])
        _close(got[b], O.attention(q[b], k[sl], v[sl], H, KVH, D))
