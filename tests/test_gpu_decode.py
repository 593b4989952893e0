"""GPU parity of the device-side decode loop (include/janus_model.h).

- generate runs on captured-step replays with the penalty's context kept as
  occurrence counts on the device: its tokens equal the oracle's
  Model::generate (generation.rs:129-323, sampler.rs:146-209) and a host
  loop that samples the GPU's own logits with the oracle's sampler, over
  200+ tokens and with both sampler rules (penalty + last max; the
  |penalty - 1| < 0.01 fast path with argmax.wgsl's tie rule, planted ties);
- graph decode with the penalty equals eager decode with the host sampler;
- KV slots: a sequence gives the same logits in any slot;
- generate_batch (continuous batching, requests admitted into freed slots)
  gives every request the tokens it gets alone and the oracle's;
- a workspace that grows after a capture does not invalidate the captured
  step (the old buffer stays alive);
- captured steps per context-length bucket: graph_run, generate,
  generate_with_callback and generate_batch across bucket edges give the
  tokens of eager steps, with the buckets and with one step planned for
  max_seq_len.
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
DEV = "cuda:0"


_prompt = DM.prompt


def _rel_err(a, b):
    return float(np.max(np.abs(a - b)) / np.max(np.abs(b)))


@pytest.fixture(scope="module")
def spec():
    return synth.tiny_config1(1)


def _host_loop(m, prompt, steps, penalty):
    """Eager decode on the GPU with the oracle's sampler on the GPU's logits."""
    for p, t in enumerate(prompt):
        m.forward([t], [p])
    last, pos, gen = prompt[-1], len(prompt), []
    for _ in range(steps):
        m.forward([last], [pos])
        last = O.greedy_sample(m.logits()[0], gen, penalty)
        gen.append(last)
        pos += 1
    return gen


@pytest.mark.parametrize("act", [_lib.DT_F32, _lib.DT_F16])
def test_generate_200_tokens_penalty_matches_oracle_and_host_loop(engine, spec, act):
    """200 tokens with the reference's default sampler, against the oracle
    in the same activation dtype (binary16 activations: the oracle's act_f16
    mode), identical or parted only at a certified near tie."""
    prompt = _prompt(101, 32, spec.vocab)
    want, logits = O.OracleModel(spec, 256, act_f16=(act == _lib.DT_F16)).generate(prompt, 200, 1.15,
                                                                                    return_logits=True)
    m = Model(engine, spec, max_seq_len=256, act_dtype=act)
    got = m.generate(prompt, 200, repetition_penalty=1.15)
    host = _host_loop(m, prompt, 200, 1.15)
    m.close()
    assert len(got) == 200
    assert got == host
    if act == _lib.DT_F32:
        assert got == want
    else:
        assert_same_or_near_tie(got, want, logits, 1.15)


def _tied_head_spec(vocab=512):
    """Config-1 architecture whose LM head is zero except rows 4 and 12 (equal
    to w) and rows 20 and 28 (equal to -w): whatever the sign of w . x, the
    largest logit is a tie between two rows that are equal mod 8, so both take
    the same reduction path and tie exactly. argmax.wgsl prefers the smaller
    bitrev8(i % 256) (4 over 12, 20 over 28), the last-max argmax the later
    index; the zero logits tie as well (argmax.wgsl: 0, last-max: vocab-1)."""
    s = synth.tiny_config1(3)
    rng = np.random.default_rng(5)
    head = np.zeros((vocab, s.hidden), np.float32)
    row = rng.standard_normal(s.hidden).astype(np.float32) * np.float32(0.05)
    head[4] = head[12] = row
    head[20] = head[28] = -row
    s.tensors = [t for t in s.tensors if t.name != "output.weight"]
    s.tensors.append(synth.Tensor("output.weight", synth.F32, vocab, s.hidden, head))
    return s


@pytest.mark.parametrize("act", [_lib.DT_F32, _lib.DT_F16])
@pytest.mark.parametrize("penalty", [1.0, 1.005, 1.15])
def test_generate_sampler_rules_with_planted_ties(engine, act, penalty):
    s = _tied_head_spec()
    for seed in range(3):
        prompt = _prompt(200 + seed, 6, s.vocab)
        want = O.OracleModel(s, 32).generate(prompt, 6, penalty)
        m = Model(engine, s, max_seq_len=32, act_dtype=act)
        got = m.generate(prompt, 6, repetition_penalty=penalty)
        m.close()
        assert got == want, (seed, got, want)
        # the first choice is decided by a tie rule
        assert want[0] in ((4, 20) if penalty < 1.01 else (12, 28)), want


def test_graph_penalty_decode_matches_eager(engine):
    """The captured step with the penalty sampler (counts kept on the device)
    against eager steps sampled on the host, for a batch of 3 and for 1."""
    s = synth.make_model(41, 512, 4, 1, 1024, 1000, 2, synth.Q4_0, 1e-5, 500000.0,
                         embed_type=synth.F16, head_type=synth.F16)
    for nseq in (1, 3):
        prompts = [_prompt(50 + i, 7 + i, s.vocab) for i in range(nseq)]
        outs = []
        for use_graph in (False, True):
            m = Model(engine, s, max_seq_len=64, max_batch=3, kv_dtype=_lib.DT_F16, act_dtype=_lib.DT_F16)
            n = max(len(p) for p in prompts)
            for step in range(n):
                m.forward([p[min(step, len(p) - 1)] for p in prompts], [min(step, len(p) - 1) for p in prompts])
            last = [p[-1] for p in prompts]
            pos = [len(p) for p in prompts]
            gens = [[] for _ in prompts]
            if use_graph:
                m.set_sampler(_lib.SAMPLER_PENALTY, 1.15)
                m.graph_begin(last, pos)
                m.graph_run(12)
                gens = [m.generated(r) for r in range(nseq)]
            else:
                for _ in range(12):
                    m.forward(last, pos)
                    lg = m.logits(nseq)
                    last = [O.greedy_sample(lg[r], gens[r], 1.15) for r in range(nseq)]
                    for r in range(nseq):
                        gens[r].append(last[r])
                    pos = [p + 1 for p in pos]
            outs.append(gens)
            m.close()
        assert outs[0] == outs[1], nseq


@pytest.mark.parametrize("hidden", [1024, 2048, 4096])
def test_folded_lm_head_two_rows_per_step(engine, hidden):
    """The greedy choice folded into the F16 LM head at 2, 4 and 8 units per
    lane, where the LDS kernel takes two rows per wavefront step: the key
    epilogue is the per-row store, not the paired QKV / SwiGLU one (which
    would write K/V rows through the head's null cache pointers). Graph
    decode under both sampler rules against eager steps with the host
    sampler."""
    s = synth.make_model(57 + hidden, hidden, hidden // 128, hidden // 512, 512, 1000, 1, synth.Q4_0, 1e-5, 500000.0,
                         embed_type=synth.F16, head_type=synth.F16)
    prompt = _prompt(hidden, 6, s.vocab)
    for mode, penalty in ((_lib.SAMPLER_ARGMAX, 1.0), (_lib.SAMPLER_PENALTY, 1.15)):
        outs = []
        for use_graph in (False, True):
            m = Model(engine, s, max_seq_len=32, kv_dtype=_lib.DT_F16, act_dtype=_lib.DT_F16)
            for p_, t in enumerate(prompt):
                m.forward([t], [p_])
            last, pos, gen = prompt[-1], len(prompt), []
            if use_graph:
                m.set_sampler(mode, penalty)
                m.graph_begin([last], [pos])
                m.graph_run(8)
                gen = m.generated(0)
            else:
                for _ in range(8):
                    m.forward([last], [pos])
                    lg = m.logits()[0]
                    last = O.argmax_last(lg) if mode == _lib.SAMPLER_ARGMAX else O.greedy_sample(lg, gen, penalty)
                    gen.append(last)
                    pos += 1
            outs.append(list(gen))
            m.close()
        assert outs[0] == outs[1], (hidden, mode, outs)


def test_kv_slots_equal_logits(engine, spec):
    prompt = _prompt(61, 9, spec.vocab)
    m = Model(engine, spec, max_seq_len=32, max_batch=4)
    out = []
    for slot in (0, 2, 3):
        for p, t in enumerate(prompt):
            m.forward([t], [p], slots=[slot])
        out.append(m.logits()[0])
    # two sequences in swapped slots in one batch
    other = _prompt(62, 9, spec.vocab)
    for p in range(9):
        m.forward([other[p], prompt[p]], [p, p], slots=[3, 1])
    both = m.logits(2)
    m.close()
    assert np.array_equal(out[0], out[1]) and np.array_equal(out[0], out[2])
    assert _rel_err(both[1], out[0]) <= 1e-5


def test_kv_slots_rejects_bad_slots(engine, spec):
    m = Model(engine, spec, max_seq_len=32, max_batch=2)
    with pytest.raises(ops.JanusError):
        m.forward([1, 2], [0, 0], slots=[1, 1])
    with pytest.raises(ops.JanusError):
        m.forward([1], [0], slots=[2])
    m.close()


@pytest.mark.parametrize("act,kv", [(_lib.DT_F32, _lib.DT_F32), (_lib.DT_F16, _lib.DT_F16)])
def test_generate_batch_continuous_matches_alone_and_oracle(engine, spec, act, kv):
    """7 requests of different lengths through 3 slots: requests finish at
    different steps and waiting ones take their slots mid-run."""
    rng = np.random.default_rng(71)
    lens = [5, 12, 3, 9, 1, 7, 4]
    maxt = 9
    prompts = [rng.integers(0, spec.vocab, n).tolist() for n in lens]
    m = Model(engine, spec, max_seq_len=48, max_batch=3, kv_dtype=kv, act_dtype=act)
    got = m.generate_batch(prompts, maxt, 1.15)
    alone = [m.generate_batch([p], maxt, 1.15)[0] for p in prompts]
    m.close()
    assert all(len(g) == maxt for g in got)
    for p, g, a in zip(prompts, got, alone):
        want, logits = O.OracleModel(spec, 48, kv_f16=(kv == _lib.DT_F16), act_f16=(act == _lib.DT_F16)).generate(
            p, maxt, 1.15, return_logits=True, batch_rules=True)
        if act == _lib.DT_F32:
            # f32 activations: batched rows run the per-row products of a
            # single sequence, so only attention's split plan differs
            assert g == a
            assert g == want
        else:
            # binary16 activations: batched rows take the MFMA products,
            # alone the GEMV ones (fp32 sums in another order); both against
            # the oracle's binary16-activation mode
            assert_same_or_near_tie(g, want, logits, 1.15)
            assert_same_or_near_tie(a, want, logits, 1.15)


def test_generate_batch_capacity_and_empty_prompt(engine, spec):
    m = Model(engine, spec, max_seq_len=16, max_batch=2)
    out = m.generate_batch([[1, 2, 3], list(range(14)), [5]], 8, 1.15)
    assert [len(o) for o in out] == [8, 2, 8]   # positions 14 and 15 only for the long prompt
    with pytest.raises(ops.JanusError):
        m.generate_batch([[1], []], 4, 1.15)
    m.close()


def test_stop_token_generate_drops_batch_keeps(engine):
    pa = [11, 22, 33]
    s = DM.eos_model(pa)
    want_single = O.OracleModel(s, 16).generate(pa, 5, 1.15)
    want_batch = O.OracleModel(s, 16).generate(pa, 5, 1.15, batch_rules=True)
    assert want_single == [] and want_batch == [128009]
    pb = [5, 6, 7, 8]
    want_b = O.OracleModel(s, 16).generate(pb, 5, 1.15, batch_rules=True)
    m = Model(engine, s, max_seq_len=16, max_batch=2)
    assert m.generate(pa, 5, 1.15) == want_single
    assert m.generate_batch([pa, pb], 5, 1.15) == [want_batch, want_b]
    m.close()


def test_workspace_growth_keeps_captured_step():
    """Capture with fewer sequences than max_batch, grow the GEMM workspace
    with a large standalone product, then replay: the captured step must
    still give the eager tokens (its workspace was retired, not freed). A
    context of its own, so the workspace starts at this test's sizes."""
    engine = ops.ComputeEngine(0)
    s = synth.make_model(91, 512, 4, 1, 1024, 1000, 2, synth.Q4_0, 1e-5, 500000.0,
                         embed_type=synth.F16, head_type=synth.F16)
    prompts = [_prompt(92, 6, s.vocab), _prompt(93, 6, s.vocab)]
    outs = []
    for grow in (False, True):
        m = Model(engine, s, max_seq_len=48, max_batch=4, kv_dtype=_lib.DT_F16, act_dtype=_lib.DT_F16)
        for step in range(6):
            m.forward([p[step] for p in prompts], [step, step])
        m.graph_begin([p[-1] for p in prompts], [6, 6])
        m.graph_run(3)
        if grow:
            _, before = engine.workspace_bytes()
            n, k = 32768, 4096
            w = ops.GpuTensor(engine, 1, n, k, synth.f16_bits(np.full((n, k), 0.01, np.float32)))
            a = torch.ones(64, k, device=DEV, dtype=torch.float16)
            c = torch.empty(64, n, device=DEV)
            ops.gemm_auto(engine, a, w, c, 64, 1, k, n)
            engine.sync()
            _, after = engine.workspace_bytes()
            assert after > before
            # eager steps with every row in between (another plan, same buffers)
            m2 = Model(engine, s, max_seq_len=48, max_batch=4, kv_dtype=_lib.DT_F16, act_dtype=_lib.DT_F16)
            m2.forward([1, 2, 3, 4], [0, 0, 0, 0])
            m2.close()
            del w
        m.graph_run(6)
        outs.append([m.generated(r) for r in range(2)])
        m.close()
    assert outs[0] == outs[1]
    assert all(len(g) == 9 for g in outs[0])
    engine.sync()
    engine.close()


def test_nan_logits_refused_under_cpu_sampler_rules(engine):
    """NaN logits: the reference's CPU sampler (penalty != 1, and every batch)
    panics (sampler.rs:191-193, 397-399), so generate, generate_batch and a
    graph run under the penalty or plain last-max rule return
    JANUS_E_NAN_LOGITS, and no token is chosen at that step. The GPU-argmax
    rule (|penalty - 1| < 0.01) ignores NaN as argmax.wgsl does and follows
    the oracle."""
    s = DM.nan_head_model()
    prompt = _prompt(98, 5, s.vocab)
    m = Model(engine, s, max_seq_len=32, max_batch=2)
    m.forward([prompt[0]], [0])
    assert np.isnan(m.logits()[0][321])
    with pytest.raises(ops.JanusError) as ei:
        m.generate(prompt, 4, repetition_penalty=1.15)
    assert ei.value.status == _lib.E_NAN_LOGITS
    with pytest.raises(ops.JanusError) as ei:
        m.generate_batch([prompt, prompt[:3]], 4, 1.15)
    assert ei.value.status == _lib.E_NAN_LOGITS
    for mode, pen in ((_lib.SAMPLER_ARGMAX, 1.0), (_lib.SAMPLER_PENALTY, 1.15)):
        m.set_sampler(mode, pen)
        m.graph_begin([prompt[-1]], [len(prompt)])
        with pytest.raises(ops.JanusError) as ei:
            m.graph_run(3)
        assert ei.value.status == _lib.E_NAN_LOGITS
        assert m.generated(0) == []
    # the GPU-argmax rule: NaN never wins, the stream equals the oracle's
    got = m.generate(prompt, 6, repetition_penalty=1.0)
    m.close()
    assert got == O.OracleModel(s, 32).generate(prompt, 6, 1.0)
    with pytest.raises(FloatingPointError):
        O.OracleModel(s, 32).generate(prompt, 2, 1.15)


def _eager_tokens(m, prompt, steps, penalty):
    """Eager steps after an eager prefill, sampled on the host from the GPU's
    logits (penalty None: last-max argmax); returns the tokens and each
    step's logits."""
    for p, t in enumerate(prompt):
        m.forward([t], [p])
    last, pos, gen, logits = prompt[-1], len(prompt), [], []
    for _ in range(steps):
        m.forward([last], [pos])
        lg = m.logits()[0]
        logits.append(lg)
        last = O.argmax_last(lg) if penalty is None else O.greedy_sample(lg, gen, penalty)
        gen.append(last)
        pos += 1
    return gen, logits


def test_captured_steps_cross_length_buckets(monkeypatch):
    """Captured steps are planned per context-length bucket (256, 512, ...,
    the last one max_seq_len): each replay runs the smallest bucket that
    covers its longest row. With max_seq_len 600 the buckets are 256, 512
    and 600. Graph decode from position 240 over two graph_run calls (the
    second starting mid-bucket) crosses both edges; generate and
    generate_with_callback cross 256 while prefilling and 512 while
    decoding; generate_batch crosses them with its rows at different
    positions. Each loop's tokens against eager steps sampled on the host
    (identical, or parted only at a certified near tie), with the buckets and
    with one step planned for max_seq_len (JANUS_GRAPH_BUCKETS=0)."""
    s = synth.make_model(97, 512, 4, 1, 1024, 1000, 2, synth.Q4_0, 1e-5, 500000.0,
                         embed_type=synth.F16, head_type=synth.F16)
    prompt = _prompt(98, 240, s.vocab)
    short = prompt[:100]
    steps = 300   # positions 240..539
    eng = ops.ComputeEngine(0)
    m = Model(eng, s, max_seq_len=600, kv_dtype=_lib.DT_F16, act_dtype=_lib.DT_F16)
    want_arg, lg_arg = _eager_tokens(m, prompt, steps, None)
    want_pen, lg_pen = _eager_tokens(m, prompt, steps, 1.15)
    want_short, lg_short = _eager_tokens(m, short, steps, 1.15)
    m.close()
    eng.close()
    for buckets in ("1", "0"):
        monkeypatch.setenv("JANUS_GRAPH_BUCKETS", buckets)
        eng = ops.ComputeEngine(0)
        m = Model(eng, s, max_seq_len=600, max_batch=2, kv_dtype=_lib.DT_F16, act_dtype=_lib.DT_F16)
        for p, t in enumerate(prompt):
            m.forward([t], [p])
        m.set_sampler(_lib.SAMPLER_ARGMAX)
        m.graph_begin([prompt[-1]], [len(prompt)])
        m.graph_run(100)
        m.graph_run(steps - 100)
        graph = m.generated(0)
        gen = m.generate(prompt, steps, 1.15)
        stream = m.generate_with_callback(prompt, steps, None, 1.15)
        batch = m.generate_batch([prompt, short], steps, 1.15)
        m.close()
        eng.close()
        assert len(graph) == len(gen) == len(stream) == steps and [len(b) for b in batch] == [steps, steps]
        assert_same_or_near_tie(graph, want_arg, lg_arg, 1.0)
        for got in (gen, stream, batch[0]):
            assert_same_or_near_tie(got, want_pen, lg_pen, 1.15)
        assert_same_or_near_tie(batch[1], want_short, lg_short, 1.15)
