"""GPU parity of the glue kernels against the oracle and the reference KATs
(crates/janus-engine/src/compute/ops/tests.rs:195-479)."""
import numpy as np
import pytest
import torch

from janus_amd import ops, synth
from oracle import oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def T(a, dtype=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV, dtype)


def test_add_mul_kat(engine):
    a, b = T([1, 2, 3, 4.0]), T([10, 20, 30, 40.0])
    out = torch.empty(4, device=DEV)
    ops.add_tensors(engine, a, b, out, 4)
    assert torch.allclose(out.cpu(), torch.tensor([11, 22, 33, 44.0]), atol=1e-5)
    ops.elementwise_mul(engine, a, b, out, 4)
    assert torch.allclose(out.cpu(), torch.tensor([10, 40, 90, 160.0]), atol=1e-5)


@pytest.mark.parametrize("batch,hidden", [(1, 4), (1, 256), (3, 4096), (32, 4096), (2, 300)])
def test_rmsnorm(engine, batch, hidden):
    rng = np.random.default_rng(hidden)
    x = rng.standard_normal((batch, hidden)).astype(np.float32) * 3
    g = (1 + 0.02 * rng.standard_normal(hidden)).astype(np.float32)
    out = torch.empty(batch, hidden, device=DEV)
    ops.rmsnorm(engine, T(x), out, T(g), batch, hidden, 1e-5)
    want = O.rmsnorm(x, g, 1e-5)
    assert np.allclose(out.cpu().numpy(), want, rtol=3e-6, atol=1e-7)
    out16 = torch.empty(batch, hidden, device=DEV, dtype=torch.float16)
    ops.rmsnorm(engine, T(x), out16, T(g), batch, hidden, 1e-5)
    assert np.allclose(out16.float().cpu().numpy(), want, rtol=1e-3, atol=1e-6)


def test_silu_swiglu(engine):
    x = np.linspace(-20, 20, 4097).astype(np.float32)
    u = np.random.default_rng(0).standard_normal(4097).astype(np.float32)
    out = torch.empty(4097, device=DEV)
    ops.silu(engine, T(x), out, 4097)
    assert np.allclose(out.cpu().numpy(), O.silu(x), rtol=2e-6, atol=1e-30)
    ops.swiglu(engine, T(x), T(u), out, 4097)
    assert np.allclose(out.cpu().numpy(), O.mul(O.silu(x), u), rtol=3e-6, atol=1e-30)


def test_rope_kat_and_table(engine):
    table = T([1, 0, 1, 0, 0.5403023, 0.84147096, 0.99995, 0.009999833])
    x = T([1, 0, 1, 0.0])
    out = torch.empty(4, device=DEV)
    ops.rope(engine, x, out, table, 1, 1, 4, 0)
    assert torch.allclose(out.cpu(), x.cpu(), atol=1e-4)
    # the library's host-computed table equals the oracle's bit for bit
    for hd, base in [(64, 10000.0), (128, 500000.0)]:
        t = ops.create_rope_cache(engine, 512, hd, base)
        assert np.array_equal(t.cpu().numpy().view(np.uint32), O.rope_table(512, hd, base).view(np.uint32))


def test_rope_matches_oracle_and_per_sequence_positions(engine):
    hd, H = 128, 8
    table_np = O.rope_table(100, hd, 500000.0)
    table = T(table_np)
    rng = np.random.default_rng(5)
    x = rng.standard_normal((3, H * hd)).astype(np.float32)
    out = torch.empty(3, H * hd, device=DEV)
    pos = [4, 50, 99]
    ops.rope(engine, T(x), out, table, 3, H, hd, 0, T(pos, torch.int32))
    for b, p in enumerate(pos):
        want = O.rope(x[b], table_np, H, hd, p)
        assert np.allclose(out[b].cpu().numpy(), want, rtol=1e-6, atol=1e-6)


def test_kv_cache_update_kat(engine):
    cache = ops.KVCache(engine, 1, 1, 16, 2, 4)
    k, v = torch.full((8,), 0.1, device=DEV), torch.full((8,), 0.2, device=DEV)
    cache.update(k, v, 0, 0)
    assert cache.current_position() == 1
    kc, vc = cache.buffers()
    assert torch.equal(kc[0, 0].reshape(-1), k) and torch.equal(vc[0, 0].reshape(-1), v)
    with pytest.raises(ops.JanusError) as e:
        cache.update(k, v, 0, 16)
    assert e.value.status == 4


def test_kv_update_f16_ragged(engine):
    kvh, hd, cap = 8, 128, 32
    kc = torch.zeros(3 * cap, kvh, hd, device=DEV, dtype=torch.float16)
    vc = torch.zeros_like(kc)
    rng = np.random.default_rng(1)
    kn, vn = T(rng.standard_normal((3, kvh * hd))), T(rng.standard_normal((3, kvh * hd)))
    base, pos = T([0, 32, 64], torch.int32), T([5, 0, 31], torch.int32)
    ops.kv_update(engine, kn, vn, kc, vc, 3, kvh, hd, 0, cap, base, pos)
    for b, (rb, p) in enumerate([(0, 5), (32, 0), (64, 31)]):
        assert torch.equal(kc[rb + p].reshape(-1), kn[b].half())
        assert torch.equal(vc[rb + p].reshape(-1), vn[b].half())
    assert int((kc != 0).sum()) == 3 * kvh * hd


def test_embed(engine):
    vocab, hidden = 512, 256
    rng = np.random.default_rng(2)
    emb = rng.standard_normal((vocab, hidden)).astype(np.float32)
    emb[0, :4] = [1e-6, -3e-7, 6e-5, 7e-5]   # f16 subnormals flush to zero
    table = ops.GpuTensor(engine, 0, vocab, hidden, emb, ops.WEIGHT_FTZ_F16)
    ids = [0, 511, 17, 17]
    out = torch.empty(len(ids), hidden, device=DEV)
    ops.embed_tokens(engine, table, ids, out)
    bits = O.f32_to_f16_rne(emb).reshape(vocab, hidden)
    want = np.stack([O.f16_to_f32(bits[i], "ftz") for i in ids])
    assert np.array_equal(out.cpu().numpy(), want)
    assert out[0, 0].item() == 0.0 and out[0, 2].item() == 0.0
    with pytest.raises(ops.JanusError) as e:
        ops.embed_tokens(engine, table, [512], out)
    assert e.value.status == 5


def test_argmax_kat_and_tie_rules(engine):
    out = torch.zeros(4, dtype=torch.int32, device=DEV)
    l = T([-1.0, 0.5, 4.2, 3.9, 2.0])
    ops.argmax(engine, l, out, 5, 1, ops.TIE_WGSL)
    assert out[0].item() == 2
    rng = np.random.default_rng(3)
    for trial in range(40):
        v = int(rng.integers(1, 140000)) if trial % 4 == 0 else int(rng.integers(1, 3000))
        logits = rng.integers(-4, 5, (2, v)).astype(np.float32)
        lt = T(logits)
        ops.argmax(engine, lt, out, v, 2, ops.TIE_LAST)
        got_last = out[:2].cpu().tolist()
        ops.argmax(engine, lt, out, v, 2, ops.TIE_WGSL)
        got_wgsl = out[:2].cpu().tolist()
        for b in range(2):
            assert got_last[b] == O.argmax_last(logits[b])
            assert got_wgsl[b] == O.argmax_wgsl(logits[b])


def test_repetition_penalty(engine):
    rng = np.random.default_rng(4)
    logits = rng.standard_normal(1000).astype(np.float32)
    ctxt = [3, 3, 999, 3, 0, 500, 500]
    lt = T(logits)
    ops.repetition_penalty(engine, lt, 1000, T(ctxt, torch.int32), 1.15)
    want = logits.copy()
    O.lib().jo_repetition_penalty(want, 1000, np.array(ctxt, np.uint32), len(ctxt), 1.15)
    assert np.array_equal(lt.cpu().numpy(), want)
