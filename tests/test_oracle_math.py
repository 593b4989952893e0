"""Pins the oracle's floating-point glue against f64 closed forms, invariants
and brute force (the reference's own tests only check these for finiteness).

- RMSNorm, SiLU, RoPE rotation and attention against f64 numpy statements.
- Attention invariants: one position returns V; GQA equals MHA with
  repeated KV heads; permuting positions leaves the output unchanged.
- RoPE table: closed form pos / base^(2i/hd) in f64; rotation keeps norms.
- argmax tie rules by brute force: last-max (model/sampler.rs:784-795) and
  the 256-lane scan (argmax.wgsl:26-126) = min (bitrev8(i % 256), i) among ties.
- Greedy sampling: penalty compounds per occurrence (sampler.rs:599-613).
"""
import numpy as np
import pytest

from janus_amd import synth
from oracle import oracle as O


def test_rmsnorm_vs_f64():
    rng = np.random.default_rng(0)
    for h in (1, 4, 256, 300, 4096):
        x = rng.standard_normal((3, h)).astype(np.float32)
        g = (1 + 0.1 * rng.standard_normal(h)).astype(np.float32)
        y = O.rmsnorm(x, g, 1e-5)
        x64 = x.astype(np.float64)
        ref = x64 / np.sqrt((x64 ** 2).mean(axis=1, keepdims=True) + 1e-5) * g
        assert np.allclose(y, ref, rtol=2e-6, atol=1e-7)


def test_silu_vs_f64():
    x = np.linspace(-30, 30, 10001).astype(np.float32)
    ref = x.astype(np.float64) / (1 + np.exp(-x.astype(np.float64)))
    assert np.allclose(O.silu(x), ref, rtol=1e-6, atol=1e-30)


def test_rope_table_closed_form_and_rotation():
    hd, base, n = 64, 500000.0, 300
    t = O.rope_table(n, hd, base).reshape(n, hd // 2, 2)
    i = np.arange(hd // 2)
    ang = np.arange(n)[:, None] / base ** (2 * i / hd)[None, :]
    # binary32 powf/cosf/sinf: within a few ulp of the f64 angle's cos/sin
    # plus the angle's own f32 rounding (relative 2^-24 of pos/theta)
    tol = 4e-7 * np.maximum(1, ang)
    assert np.all(np.abs(t[..., 0] - np.cos(ang)) <= tol)
    assert np.all(np.abs(t[..., 1] - np.sin(ang)) <= tol)
    rng = np.random.default_rng(1)
    x = rng.standard_normal(4 * hd).astype(np.float32)
    y = O.rope(x, t.reshape(-1), 4, hd, 123)
    xr, yr = x.reshape(4, 2, hd // 2), y.reshape(4, 2, hd // 2)
    # each (i, i + hd/2) pair keeps its length
    assert np.allclose(np.hypot(xr[:, 0], xr[:, 1]), np.hypot(yr[:, 0], yr[:, 1]), rtol=1e-5)
    c, s = t[123, :, 0], t[123, :, 1]
    assert np.allclose(yr[:, 0], xr[:, 0] * c - xr[:, 1] * s, atol=1e-6)


def np_attention(q, k, v, H, KVH, D):
    q = q.reshape(H, D).astype(np.float64)
    k = k.reshape(-1, KVH, D).astype(np.float64)
    v = v.reshape(-1, KVH, D).astype(np.float64)
    out = np.zeros((H, D))
    for h in range(H):
        g = h * KVH // H
        s = k[:, g, :] @ q[h] / np.sqrt(D)
        p = np.exp(s - s.max())
        out[h] = (p / p.sum()) @ v[:, g, :]
    return out.reshape(-1)


@pytest.mark.parametrize("L,H,KVH,D", [(1, 4, 2, 64), (37, 4, 2, 64), (300, 32, 8, 128), (129, 8, 8, 128)])
def test_attention_vs_f64(L, H, KVH, D):
    rng = np.random.default_rng(L)
    q = rng.standard_normal(H * D).astype(np.float32)
    k = rng.standard_normal((L, KVH, D)).astype(np.float32)
    v = rng.standard_normal((L, KVH, D)).astype(np.float32)
    out = O.attention(q, k, v, H, KVH, D)
    assert np.allclose(out, np_attention(q, k, v, H, KVH, D), rtol=1e-4, atol=1e-5)


def test_attention_invariants():
    rng = np.random.default_rng(9)
    H, KVH, D, L = 8, 2, 64, 50
    q = rng.standard_normal(H * D).astype(np.float32)
    k = rng.standard_normal((L, KVH, D)).astype(np.float32)
    v = rng.standard_normal((L, KVH, D)).astype(np.float32)
    # single position -> V of the mapped head
    one = O.attention(q, k[:1], v[:1], H, KVH, D).reshape(H, D)
    assert np.allclose(one, v[0][np.arange(H) * KVH // H], atol=1e-6)
    # GQA == MHA with KV heads repeated
    gqa = O.attention(q, k, v, H, KVH, D)
    rep = np.arange(H) * KVH // H
    mha = O.attention(q, k[:, rep, :].copy(), v[:, rep, :].copy(), H, H, D)
    assert np.array_equal(gqa, mha)
    # permuting positions only reorders the sums
    perm = rng.permutation(L)
    assert np.allclose(O.attention(q, k[perm].copy(), v[perm].copy(), H, KVH, D), gqa, atol=1e-5)


def _bitrev8(t):
    return int(f"{t:08b}"[::-1], 2)


def _wgsl_rule(l):
    # the tree merges slot t + stride into slot t for stride 128 .. 1 and keeps
    # the lower slot on ties, so among tied lanes the one whose lane id has the
    # smallest bit-reversed value wins; within a lane the scan keeps the first
    m = l.max()
    ties = np.flatnonzero(l == m)
    return int(min(ties, key=lambda i: (_bitrev8(i % 256), i)))


def test_argmax_tie_rules_brute_force():
    rng = np.random.default_rng(11)
    for trial in range(300):
        v = int(rng.integers(1, 1200))
        l = rng.integers(-3, 4, v).astype(np.float32)   # many ties
        assert O.argmax_last(l) == int(np.flatnonzero(l == l.max())[-1])
        assert O.argmax_wgsl(l) == _wgsl_rule(l)


def test_greedy_penalty_compounds_per_occurrence():
    logits = np.array([2.0, 1.9, -1.0, 0.5], np.float32)
    # token 0 penalised twice: 2 / 1.15 / 1.15 = 1.512 < 1.9 -> 1 wins
    assert O.greedy_sample(logits, [0, 0]) == 1
    # once: 2/1.15 = 1.739 < 1.9 -> 1 wins too; none: 0 wins
    assert O.greedy_sample(logits, []) == 0
    # negative logits are multiplied
    l2 = np.array([-1.0, -1.1], np.float32)
    assert O.greedy_sample(l2, [0]) == 1
    # sequential division, not division by p^2
    x = np.array([3.0, 0.0], np.float32)
    y = x.copy()
    O.lib().jo_repetition_penalty(y, 2, np.array([0, 0, 0], np.uint32), 3, 1.15)
    assert y[0] == np.float32(np.float32(np.float32(3.0 / np.float32(1.15)) / np.float32(1.15)) / np.float32(1.15))
    with pytest.raises(FloatingPointError):
        O.greedy_sample(np.array([np.nan, 1.0], np.float32), [])


def test_model_oracle_fp16_kv_close_to_f32_kv():
    spec = synth.tiny_config1(3)
    a = O.OracleModel(spec, 48)
    b = O.OracleModel(spec, 48, kv_f16=True)
    rng = np.random.default_rng(3)
    prompt = rng.integers(0, spec.vocab, 8)
    for p, t in enumerate(prompt):
        la, lb = a.forward(int(t), p), b.forward(int(t), p)
    assert np.max(np.abs(la - lb)) <= 2e-3 * np.max(np.abs(la))


def test_model_oracle_generate_refeeds_last_prompt_token():
    spec = synth.tiny_config1(4)
    m = O.OracleModel(spec, 64)
    prompt = [5, 17, 300]
    toks, logits = m.generate(prompt, 2, return_logits=True)
    # step 0 logits == forward(last prompt token, position n) after a prefill
    m2 = O.OracleModel(spec, 64)
    for p, t in enumerate(prompt):
        m2.forward(t, p)
    assert np.array_equal(m2.forward(prompt[-1], len(prompt)), logits[0])


def test_model_oracle_act_f16_rounds_exactly_the_product_inputs():
    """act_f16 feeds every product (q/k/v, o, gate/up, down, LM head) a
    binary16-representable input and leaves the residual stream alone: the
    default mode feeds f32 values that binary16 does not hold, and with
    act_f16 off the logits are unchanged by the new flag."""
    spec = synth.tiny_config1(5)
    prompt = np.random.default_rng(5).integers(0, spec.vocab, 6)

    def run(act_f16):
        m = O.OracleModel(spec, 32, kv_f16=True, act_f16=act_f16)
        seen = []
        mm = m._mm

        def rec(name, x):
            seen.append((name, np.array(x, dtype=np.float32)))
            return mm(name, x)

        m._mm = rec
        out = [m.forward(int(t), p) for p, t in enumerate(prompt)]
        return out, seen

    base, _ = run(False)
    ref = O.OracleModel(spec, 32, kv_f16=True)
    for p, t in enumerate(prompt):
        assert np.array_equal(ref.forward(int(t), p), base[p])
    h, seen16 = run(True)
    _, seen32 = run(False)
    names = {n.split(".")[-2] if n.startswith("blk.") else n.split(".")[0] for n, _ in seen16}
    assert names == {"attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down", "output"}
    for name, x in seen16:
        assert np.array_equal(x, x.astype(np.float16).astype(np.float32)), name
    assert any(not np.array_equal(x, x.astype(np.float16).astype(np.float32)) for _, x in seen32)
    # binary16 storage of activations moves the logits by a rounding-sized amount
    for a, b in zip(base, h):
        assert 0 < np.max(np.abs(a - b)) <= 1e-2 * np.max(np.abs(a))
