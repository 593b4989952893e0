"""janus_attention_noalloc: the allocation-free variant of janus_attention
(fixed per-device scratch for the split partials).

On the GPU it must give exactly janus_attention's output (same kernels, same
split plan) on two calls in a row, the second smaller than the first, with
contexts long enough that the partials really go through the scratch. On the
host it must reject shapes whose partials exceed the scratch before anything
is enqueued.
"""
import ctypes as C

import numpy as np
import pytest
import torch

from janus_amd import _lib, ops

DEV = "cuda:0"


def _case(rng, lens, H, KVH, D, kv):
    offs = np.concatenate([[0], np.cumsum(lens)[:-1]]).astype(np.int32)
    total = int(sum(lens))
    k = torch.from_numpy(rng.standard_normal((total, KVH, D), dtype=np.float32)).to(DEV, kv)
    v = torch.from_numpy(rng.standard_normal((total, KVH, D), dtype=np.float32)).to(DEV, kv)
    q = torch.from_numpy(rng.standard_normal((len(lens), H * D), dtype=np.float32)).to(DEV)
    return q, k, v, torch.from_numpy(offs).to(DEV), torch.tensor(lens, dtype=torch.int32, device=DEV)


@pytest.mark.gpu
@pytest.mark.parametrize("kv", [torch.float16, torch.float32])
def test_noalloc_equals_attention_twice_second_smaller(engine, kv):
    rng = np.random.default_rng(123)
    H, KVH, D = 32, 8, 128
    for lens in ([4096, 300, 7000, 1, 2500, 8192], [3000, 17]):
        q, k, v, offs, dl = _case(rng, lens, H, KVH, D, kv)
        B, mx = len(lens), max(lens)
        assert mx > 1024   # long enough for split partials
        want = torch.full((B, H * D), 7.0, device=DEV)
        got = torch.full((B, H * D), -7.0, device=DEV)
        ops.compute_attention(engine, q, k, v, want, B, 0, mx, H, KVH, D, row_base=offs, seq_lens=dl,
                              max_len_hint=mx)
        ops.compute_attention_noalloc(engine, q, k, v, got, B, 0, mx, H, KVH, D, row_base=offs, seq_lens=dl,
                                      max_len_hint=mx)
        torch.cuda.synchronize()
        assert torch.equal(got, want), float((got - want).abs().max())


@pytest.mark.gpu
def test_noalloc_allocates_no_workspace():
    """On a fresh context, calls of every split plan (row streaming, the
    piece list, and a single sequence split over workgroups) leave the
    context's workspaces unallocated; the regular entry point on the same
    context then gives the same outputs (and does allocate)."""
    from janus_amd.ops import ComputeEngine
    eng = ComputeEngine(0)
    try:
        rng = np.random.default_rng(5)
        cases = [([3000, 2500, 4096, 100], 32, 8, 128, torch.float16),   # rows plan
                 ([3000, 2500, 900], 16, 4, 64, torch.float16),          # piece list
                 ([6000], 32, 8, 128, torch.float32)]                    # split + merge
        outs = []
        for lens, H, KVH, D, kv in cases:
            q, k, v, offs, dl = _case(rng, lens, H, KVH, D, kv)
            B, mx = len(lens), max(lens)
            got = torch.full((B, H * D), -7.0, device=DEV)
            ops.compute_attention_noalloc(eng, q, k, v, got, B, 0, mx, H, KVH, D, row_base=offs, seq_lens=dl,
                                          max_len_hint=mx)
            torch.cuda.synchronize()
            assert eng.workspace_bytes() == (0, 0), (lens, eng.workspace_bytes())
            outs.append((q, k, v, offs, dl, got))
        for (lens, H, KVH, D, kv), (q, k, v, offs, dl, got) in zip(cases, outs):
            B, mx = len(lens), max(lens)
            want = torch.full((B, H * D), 7.0, device=DEV)
            ops.compute_attention(eng, q, k, v, want, B, 0, mx, H, KVH, D, row_base=offs, seq_lens=dl,
                                  max_len_hint=mx)
            torch.cuda.synchronize()
            assert torch.equal(got, want), (lens, float((got - want).abs().max()))
        assert eng.workspace_bytes()[0] > 0
    finally:
        eng.sync()
        eng.close()


@pytest.mark.gpu
def test_noalloc_single_sequence_gqa(engine):
    """Batch 1 with a long context (the per-query-head split plan)."""
    rng = np.random.default_rng(7)
    for L in (6000, 700):
        q, k, v, _, _ = _case(rng, [L], 32, 8, 128, torch.float16)
        want = torch.empty(32 * 128, device=DEV)
        got = torch.empty(32 * 128, device=DEV)
        ops.compute_attention(engine, q[0], k, v, want, 1, L, L, 32, 8, 128)
        ops.compute_attention_noalloc(engine, q[0], k, v, got, 1, L, L, 32, 8, 128)
        torch.cuda.synchronize()
        assert torch.equal(got, want)


def test_noalloc_rejects_partials_above_scratch():
    lib = _lib.load()
    h = C.c_void_p()
    assert lib.janus_create(-1, C.byref(h)) == _lib.OK
    try:
        buf = (C.c_float * 4)()
        lens = (C.c_int32 * 64)()
        p = C.cast(buf, C.c_void_p)
        # 64 sequences up to 2^20 positions with 64-dim heads (the piece plan,
        # partials per sequence and piece): far more than the scratch holds
        st = lib.janus_attention_noalloc(h, p, p, p, _lib.DT_F16, p, 64, 32, 8, 64, 0, 1 << 20, None,
                                         C.cast(lens, C.c_void_p), 1 << 20, 0.0)
        assert st == _lib.E_INVALID_DIM
        assert b"fixed scratch" in lib.janus_last_error(h)
        # the same batch with 128-dim heads streams whole rows, whose partials
        # are per workgroup (two slots) whatever the lengths: within the scratch
        st = lib.janus_attention_noalloc(h, p, p, p, _lib.DT_F16, p, 64, 32, 8, 128, 0, 1 << 20, None,
                                         C.cast(lens, C.c_void_p), 1 << 20, 0.0)
        assert st == _lib.E_NO_DEVICE
        # a shape within the scratch passes the host checks and then needs a device
        st = lib.janus_attention_noalloc(h, p, p, p, _lib.DT_F16, p, 1, 32, 8, 128, 100, 128, None, None, 0, 0.0)
        assert st == _lib.E_NO_DEVICE
    finally:
        lib.janus_destroy(h)
