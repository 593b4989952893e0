"""GPU parity of streaming generation, janus_model_generate_stream
(Model::generate_with_callback, generation.rs:340-604, on token ids).

- the streamed tokens, in callback order with indices 0, 1, ..., equal
  janus_model_generate's and the oracle's Model::generate, for both sampler
  rules and both activation dtypes (binary16 activations against the oracle's
  act_f16 mode: identical or parted only at a certified near tie);
- a callback returning false ends generation with that token kept
  (generation.rs:481-509), and the model generates normally afterwards;
- a stop token (128009) is neither returned nor passed to the callback;
- max_seq_len bounds the stream as it bounds generate;
- NaN logits under the penalty rule return JANUS_E_NAN_LOGITS;
- an exception in a Python callback stops generation and is re-raised;
- after generation ends the KV rows of every consumed position hold what
  eager steps write (replays behind a finished row recompute its last step),
  so a caller can continue from the cache as the reference's can.
"""
import numpy as np
import pytest
import torch

import decode_models as DM
from greedy import assert_same_or_near_tie
from janus_amd import _lib, ops, synth
from janus_amd.model import Model
from oracle import oracle as O


pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def spec():
    return synth.tiny_config1(1)


def _collect(m, prompt, n, penalty, stop_after=None):
    seen = []

    def cb(tok):
        seen.append(tok)
        return stop_after is None or len(seen) < stop_after

    got = m.generate_with_callback(prompt, n, cb, repetition_penalty=penalty)
    return got, seen


@pytest.mark.parametrize("act", [_lib.DT_F32, _lib.DT_F16])
@pytest.mark.parametrize("penalty", [1.0, 1.15])
def test_stream_equals_generate_and_oracle(engine, spec, act, penalty):
    prompt = DM.prompt(301, 24, spec.vocab)
    want, logits = O.OracleModel(spec, 128, act_f16=(act == _lib.DT_F16)).generate(prompt, 60, penalty,
                                                                                    return_logits=True)
    m = Model(engine, spec, max_seq_len=128, act_dtype=act)
    got, seen = _collect(m, prompt, 60, penalty)
    plain = m.generate(prompt, 60, repetition_penalty=penalty)
    again, _ = _collect(m, prompt, 60, penalty)
    m.close()
    assert len(got) == 60
    assert got == seen == plain == again
    if act == _lib.DT_F32:
        assert got == want
    else:
        assert_same_or_near_tie(got, want, logits, penalty)


def test_callback_stop_keeps_the_token_and_model_recovers(engine, spec):
    prompt = DM.prompt(302, 12, spec.vocab)
    m = Model(engine, spec, max_seq_len=96)
    full = m.generate(prompt, 20, repetition_penalty=1.15)
    for k in (1, 2, 7):
        got, seen = _collect(m, prompt, 20, 1.15, stop_after=k)
        assert got == seen == full[:k], k
    # indices arrive 0, 1, 2, ... and a NULL callback streams the same tokens
    idx = []
    lib = m.lib
    cb = _lib.TOKEN_CALLBACK(lambda _u, _t, i: idx.append(i) or 1)
    out = np.zeros(20, np.uint32)
    n = _lib.U32()
    p = np.asarray(prompt, np.uint32)
    m._check(lib.janus_model_generate_stream(m.handle, p.ctypes.data, len(p), 20, 1.15, cb, None,
                                             out.ctypes.data, _lib.C.byref(n)))
    assert idx == list(range(20)) and out[: n.value].tolist() == full
    m._check(lib.janus_model_generate_stream(m.handle, p.ctypes.data, len(p), 20, 1.15, _lib.TOKEN_CALLBACK(),
                                             None, out.ctypes.data, _lib.C.byref(n)))
    assert out[: n.value].tolist() == full
    assert m.generate(prompt, 20, repetition_penalty=1.15) == full
    m.close()


def test_stream_capacity_zero_tokens_and_bad_prompts(engine, spec):
    m = Model(engine, spec, max_seq_len=16)
    prompt = DM.prompt(303, 12, spec.vocab)
    # positions 12..15 are left: the reference stops at seq_pos == max_seq_len
    got, seen = _collect(m, prompt, 10, 1.15)
    assert got == seen == m.generate(prompt, 10, repetition_penalty=1.15)
    assert len(got) == 4
    assert got == O.OracleModel(spec, 16).generate(prompt, 10, 1.15)
    full = DM.prompt(304, 16, spec.vocab)
    assert _collect(m, full, 5, 1.15) == ([], [])
    assert _collect(m, prompt, 0, 1.15) == ([], [])
    with pytest.raises(ops.JanusError) as ei:
        m.generate_with_callback([], 4, lambda t: True)
    assert ei.value.status == _lib.E_INVALID_ARG
    with pytest.raises(ops.JanusError) as ei:
        m.generate_with_callback([spec.vocab], 4, lambda t: True)
    assert ei.value.status == _lib.E_TOKEN_RANGE
    with pytest.raises(ops.JanusError) as ei:
        m.generate_with_callback(DM.prompt(305, 17, spec.vocab), 4, lambda t: True)
    assert ei.value.status == _lib.E_KV_OVERFLOW
    m.close()


def test_stream_stop_token_not_returned(engine):
    """A head that makes 128009 the first choice of prompt pa: nothing is
    streamed or returned; another prompt streams the oracle's tokens."""
    pa = [11, 22, 33]
    s = DM.eos_model(pa)
    assert O.OracleModel(s, 16).generate(pa, 5, 1.15) == []
    m = Model(engine, s, max_seq_len=16)
    assert _collect(m, pa, 5, 1.15) == ([], [])
    pb = [5, 6, 7, 8]
    got, seen = _collect(m, pb, 5, 1.15)
    assert got == seen == O.OracleModel(s, 16).generate(pb, 5, 1.15)
    m.close()


def test_stream_nan_logits_refused_and_callback_errors_reraised(engine, spec):
    s = DM.nan_head_model()
    prompt = DM.prompt(98, 5, s.vocab)
    m = Model(engine, s, max_seq_len=32)
    with pytest.raises(ops.JanusError) as ei:
        m.generate_with_callback(prompt, 4, lambda t: True, repetition_penalty=1.15)
    assert ei.value.status == _lib.E_NAN_LOGITS
    got, _ = _collect(m, prompt, 6, 1.0)
    assert got == O.OracleModel(s, 32).generate(prompt, 6, 1.0)
    m.close()

    m = Model(engine, spec, max_seq_len=64)
    prompt = DM.prompt(306, 8, spec.vocab)

    def boom(tok):
        raise KeyError(tok)

    with pytest.raises(KeyError):
        m.generate_with_callback(prompt, 10, boom)
    assert m.generate_with_callback(prompt, 10) == m.generate(prompt, 10)
    m.close()


def _kv_rows(k, v, rows):
    torch.cuda.synchronize()
    return k[:, :rows].cpu().numpy().copy(), v[:, :rows].cpu().numpy().copy()


@pytest.mark.parametrize("how", ["generate", "stream", "stream_stop"])
def test_kv_rows_after_generation_equal_eager(engine, how):
    """Prompt pa's first choice is the stop token 128009: generate(pa, 5)
    stops at position 3 while the replays of its chunk go on (4 more). The
    K/V rows 0..3 of both layers must equal bit for bit those of
    generate(pa, 1), whose chunk ends with that step, and be close to eager
    forwards of pa and the re-fed last token (the captured step plans its
    attention for max_seq_len, eager steps for the current length). A
    callback stop on prompt pc leaves rows 0..3 as generate(pc, 1) does (the
    step queued behind it writes position 4)."""
    pa, pc = [11, 22, 33], [40, 41, 42]
    s = DM.eos_model(pa, layers=2)
    shape = (2, 2 * 16, 2, 64)

    def model():
        m = Model(engine, s, max_seq_len=16, max_batch=2)
        k = torch.full(shape, 7.0, device="cuda:0", dtype=torch.float32)
        v = torch.full(shape, 7.0, device="cuda:0", dtype=torch.float32)
        m.set_kv_cache(k, v)
        return m, k, v

    prompt = pc if how == "stream_stop" else pa
    ref, rk, rv = model()
    for p, t in enumerate(prompt + [prompt[-1]]):
        ref.forward([t], [p])
    eager = _kv_rows(rk, rv, 4)
    ref.close()
    ref, rk, rv = model()
    first = ref.generate(prompt, 1, 1.15)
    want = _kv_rows(rk, rv, 4)
    ref.close()
    m, k, v = model()
    if how == "generate":
        assert first == [] and m.generate(pa, 5, 1.15) == []
    elif how == "stream":
        assert first == [] and m.generate_with_callback(pa, 5, lambda t: True) == []
    else:
        assert len(first) == 1 and first[0] != 128009
        assert m.generate_with_callback(pc, 5, lambda t: False) == first
    got = _kv_rows(k, v, 4)
    m.close()
    for g, w, e in zip(got, want, eager):
        assert np.array_equal(g, w)
        assert np.max(np.abs(g - e)) <= 1e-5 * np.max(np.abs(e))
