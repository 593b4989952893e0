"""End-to-end parity of the decode driver on benchmark configuration 1.

Tiny random-init Llama (2 layers, hidden 256, 4 heads x 64, 2 KV heads,
FFN 688, vocab 512, Q8_0 blocks, F32 ffn_down, eps 1e-5, theta 1e4):
a 32-token seeded prompt, then 16 greedy tokens with the reference's loop
(re-fed last prompt token) and sampler (penalty 1.15, last-max argmax).

- logits at every decode step within 2e-3 relative (max-abs error divided
  by max-abs logit) of the oracle;
- the greedy token stream identical to the oracle's;
- fp16 KV against the oracle with binary16-rounded K/V;
- HIP-graph decode == eager decode; a ragged batch == per-sequence runs.
"""
import numpy as np
import pytest

from janus_amd import _lib, synth
from janus_amd.model import Model
from oracle import oracle as O

pytestmark = pytest.mark.gpu
REL = 2e-3


def _prompt(seed=101, n=32, vocab=512):
    return np.random.default_rng(seed).integers(0, vocab, n).tolist()


@pytest.fixture(scope="module")
def spec():
    return synth.tiny_config1(1)


def _rel_err(a, b):
    return float(np.max(np.abs(a - b)) / np.max(np.abs(b)))


@pytest.mark.parametrize("kv_dtype", [_lib.DT_F32, _lib.DT_F16])
def test_config1_logits_every_step(engine, spec, kv_dtype):
    prompt = _prompt()
    ref = O.OracleModel(spec, 64, kv_f16=(kv_dtype == _lib.DT_F16))
    m = Model(engine, spec, max_seq_len=64, kv_dtype=kv_dtype)
    worst = 0.0
    for p, t in enumerate(prompt):
        want = ref.forward(t, p)
        m.forward([t], [p])
        worst = max(worst, _rel_err(m.logits()[0], want))
    assert worst <= REL, worst
    m.close()


def test_config1_greedy_tokens_identical(engine, spec):
    prompt = _prompt()
    ref_tokens, ref_logits = O.OracleModel(spec, 64).generate(prompt, 16, return_logits=True)
    m = Model(engine, spec, max_seq_len=64)
    got = m.generate(prompt, 16, repetition_penalty=1.15)
    assert got == ref_tokens
    assert len(got) == 16
    m.close()


def test_config1_generate_stops_at_capacity(engine, spec):
    m = Model(engine, spec, max_seq_len=40)
    got = m.generate(_prompt(), 16)
    assert len(got) == 8   # positions 32..39
    m.close()


def test_graph_decode_matches_eager(engine, spec):
    prompt = _prompt(7, 12)
    m = Model(engine, spec, max_seq_len=64)
    for p, t in enumerate(prompt):
        m.forward([t], [p])
    # eager greedy (plain argmax) continuation
    eager, last, pos = [], prompt[-1], len(prompt)
    for _ in range(10):
        m.forward([last], [pos])
        last = O.argmax_last(m.logits()[0])
        eager.append(last)
        pos += 1
    m2 = Model(engine, spec, max_seq_len=64)
    for p, t in enumerate(prompt):
        m2.forward([t], [p])
    m2.graph_begin([prompt[-1]], [len(prompt)])
    graph = []
    for _ in range(10):
        m2.graph_run(1)
        graph.append(m2.graph_tokens(1)[0])
    assert graph == eager
    m.close()
    m2.close()


def test_ragged_batch_equals_single_sequences(engine, spec):
    rng = np.random.default_rng(9)
    lens = [3, 17, 9, 30]
    prompts = [rng.integers(0, 512, n).tolist() for n in lens]
    singles = []
    for pr in prompts:
        m = Model(engine, spec, max_seq_len=64)
        for p, t in enumerate(pr):
            m.forward([t], [p])
        singles.append(m.logits()[0])
        m.close()
    mb = Model(engine, spec, max_seq_len=64, max_batch=4)
    # feed all sequences together, each at its own position
    for step in range(max(lens)):
        toks, poss, rows = [], [], []
        for s, pr in enumerate(prompts):
            toks.append(pr[min(step, len(pr) - 1)])
            poss.append(min(step, len(pr) - 1))
        mb.forward(toks, poss)
        if step == max(lens) - 1:
            out = mb.logits(4)
    for s in range(4):
        assert _rel_err(out[s], singles[s]) <= 1e-5
    mb.close()


def _mini_llama3(seed=11, qtype=synth.Q4_0, ffn=1024):
    """A 2-layer Llama-3-shaped model (head_dim 128, GQA 4:1, theta 5e5) small
    enough for the oracle: exercises the fused single-sequence path."""
    return synth.make_model(seed, 512, 4, 1, ffn, 1000, 2, qtype, 1e-5, 500000.0,
                            embed_type=synth.F16, head_type=synth.F16)


@pytest.mark.parametrize("qtype", [synth.Q4_0, synth.Q8_0, synth.Q4_K])
@pytest.mark.parametrize("kv_dtype", [_lib.DT_F16, _lib.DT_F32])
def test_fused_f16_activation_path_matches_oracle(engine, qtype, kv_dtype):
    spec = _mini_llama3(qtype=qtype)
    prompt = _prompt(5, 24, spec.vocab)
    ref = O.OracleModel(spec, 64, kv_f16=(kv_dtype == _lib.DT_F16))
    m = Model(engine, spec, max_seq_len=64, kv_dtype=kv_dtype, act_dtype=_lib.DT_F16)
    worst = 0.0
    for p, t in enumerate(prompt):
        want = ref.forward(t, p)
        m.forward([t], [p])
        worst = max(worst, _rel_err(m.logits()[0], want))
    assert worst <= REL, worst
    m.close()


def test_fused_path_config1_greedy_tokens(engine, spec):
    prompt = _prompt()
    ref_tokens = O.OracleModel(spec, 64).generate(prompt, 16)
    m = Model(engine, spec, max_seq_len=64, act_dtype=_lib.DT_F16)
    assert m.generate(prompt, 16) == ref_tokens
    m.close()


def test_fused_graph_matches_fused_eager(engine):
    spec = _mini_llama3(13)
    prompt = _prompt(8, 10, spec.vocab)
    outs = []
    for use_graph in (False, True):
        m = Model(engine, spec, max_seq_len=64, kv_dtype=_lib.DT_F16, act_dtype=_lib.DT_F16)
        for p, t in enumerate(prompt):
            m.forward([t], [p])
        toks, last, pos = [], prompt[-1], len(prompt)
        if use_graph:
            m.graph_begin([last], [pos])
            for _ in range(12):
                m.graph_run(1)
                toks.append(m.graph_tokens(1)[0])
        else:
            for _ in range(12):
                m.forward([last], [pos])
                last = O.argmax_last(m.logits()[0])
                toks.append(last)
                pos += 1
        outs.append(toks)
        m.close()
    assert outs[0] == outs[1]


@pytest.mark.parametrize("qtype,kv_dtype,ffn", [(synth.Q4_0, _lib.DT_F16, 1024), (synth.Q4_K, _lib.DT_F16, 1024),
                                                 (synth.Q8_0, _lib.DT_F32, 1024), (synth.Q4_0, _lib.DT_F16, 12288)])
def test_batched_f16_path_equals_single_sequences(engine, qtype, kv_dtype, ffn):
    """Ragged batch with binary16 activations (fused batched step: MFMA
    products with RoPE/KV-append, residual+RMSNorm and SwiGLU epilogues,
    per-sequence positions) against each sequence run alone on the fused
    single-sequence GEMV path, and against the oracle. FFN 12288 gives the
    gate/up product enough row tiles to run unsplit with SwiGLU applied in
    the product's own store."""
    spec = _mini_llama3(17, qtype, ffn)
    rng = np.random.default_rng(19)
    lens = [5, 12, 8]
    prompts = [rng.integers(0, spec.vocab, n).tolist() for n in lens]
    singles = []
    for pr in prompts:
        m = Model(engine, spec, max_seq_len=32, kv_dtype=kv_dtype, act_dtype=_lib.DT_F16)
        for p, t in enumerate(pr):
            m.forward([t], [p])
        singles.append(m.logits()[0])
        m.close()
    mb = Model(engine, spec, max_seq_len=32, max_batch=3, kv_dtype=kv_dtype, act_dtype=_lib.DT_F16)
    for step in range(max(lens)):
        mb.forward([pr[min(step, len(pr) - 1)] for pr in prompts], [min(step, len(pr) - 1) for pr in prompts])
    out = mb.logits(3)
    for s in range(3):
        assert _rel_err(out[s], singles[s]) <= 1e-3
    ref = O.OracleModel(spec, 32, kv_f16=(kv_dtype == _lib.DT_F16))
    for p, t in enumerate(prompts[1]):
        want = ref.forward(t, p)
    assert _rel_err(out[1], want) <= REL
    mb.close()


def test_batched_graph_matches_batched_eager(engine):
    """Graph replays of the fused batched step (device positions, in-graph
    argmax) give the token streams of eager batched steps."""
    spec = _mini_llama3(23)
    rng = np.random.default_rng(29)
    lens = [6, 3, 9, 4]
    prompts = [rng.integers(0, spec.vocab, n).tolist() for n in lens]
    outs = []
    for use_graph in (False, True):
        m = Model(engine, spec, max_seq_len=48, max_batch=4, kv_dtype=_lib.DT_F16, act_dtype=_lib.DT_F16)
        for step in range(max(lens)):
            m.forward([pr[min(step, len(pr) - 1)] for pr in prompts], [min(step, len(pr) - 1) for pr in prompts])
        last = [pr[-1] for pr in prompts]
        pos = [len(pr) for pr in prompts]
        toks = []
        if use_graph:
            m.graph_begin(last, pos)
            for _ in range(10):
                m.graph_run(1)
                toks.append(m.graph_tokens(4))
        else:
            for _ in range(10):
                m.forward(last, pos)
                logits = m.logits(4)
                last = [O.argmax_last(logits[s]) for s in range(4)]
                toks.append(list(last))
                pos = [p + 1 for p in pos]
        outs.append([list(map(int, t)) for t in toks])
        m.close()
    assert outs[0] == outs[1]


def test_batched_40_sequences_two_m_tiles(engine):
    """40 sequences: the fused batched step runs its products with two 32-row
    MFMA tiles; every sequence must match its own single-sequence run."""
    spec = _mini_llama3(31)
    rng = np.random.default_rng(37)
    B = 40
    lens = rng.integers(1, 9, B).tolist()
    prompts = [rng.integers(0, spec.vocab, n).tolist() for n in lens]
    mb = Model(engine, spec, max_seq_len=16, max_batch=B, kv_dtype=_lib.DT_F16, act_dtype=_lib.DT_F16)
    for step in range(max(lens)):
        mb.forward([pr[min(step, len(pr) - 1)] for pr in prompts], [min(step, len(pr) - 1) for pr in prompts])
    out = mb.logits(B)
    mb.close()
    for s in (0, 17, 31, 32, 39):
        m = Model(engine, spec, max_seq_len=16, kv_dtype=_lib.DT_F16, act_dtype=_lib.DT_F16)
        for p, t in enumerate(prompts[s]):
            m.forward([t], [p])
        assert _rel_err(out[s], m.logits()[0]) <= 1e-3, s
        m.close()


def test_batched_residual_norm_split_matches_single_workgroup_form(monkeypatch):
    """The batched residual + RMSNorm epilogue spread over (512-column
    slice, row) workgroups in two launches against the one-workgroup-per-row
    kernel (JANUS_EPI_SPLIT=0), at hidden 1152 (three slices, the last one a
    quarter full), and both against each sequence run alone."""
    from janus_amd.ops import ComputeEngine
    spec = synth.make_model(31, 1152, 9, 9, 1024, 1000, 2, synth.Q4_0, 1e-5, 500000.0,
                            embed_type=synth.F16, head_type=synth.F16)
    rng = np.random.default_rng(37)
    lens = [6, 11, 9]
    prompts = [rng.integers(0, spec.vocab, n).tolist() for n in lens]
    outs = {}
    for split in ("0", "1"):
        monkeypatch.setenv("JANUS_EPI_SPLIT", split)
        eng = ComputeEngine(0)
        mb = Model(eng, spec, max_seq_len=32, max_batch=3, kv_dtype=_lib.DT_F16, act_dtype=_lib.DT_F16)
        for step in range(max(lens)):
            mb.forward([pr[min(step, len(pr) - 1)] for pr in prompts], [min(step, len(pr) - 1) for pr in prompts])
        outs[split] = mb.logits(3)
        mb.close()
        if split == "1":
            for s in range(3):
                m = Model(eng, spec, max_seq_len=32, kv_dtype=_lib.DT_F16, act_dtype=_lib.DT_F16)
                for p, t in enumerate(prompts[s]):
                    m.forward([t], [p])
                assert _rel_err(outs["1"][s], m.logits()[0]) <= 1e-3
                m.close()
        eng.sync()
        eng.close()
    for s in range(3):
        assert _rel_err(outs["1"][s], outs["0"][s]) <= 1e-3
