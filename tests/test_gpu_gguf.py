"""Decode from a GGUF file: Model.from_gguf (constructor.rs:23-437 with the
config of model/config.rs:377-446) against the committed config-1 golden
stream, and quantised embeddings against the oracle's dequantisation."""
from pathlib import Path

import numpy as np
import pytest

from janus_amd import synth
from janus_amd.model import Model
from oracle import oracle as O

pytestmark = pytest.mark.gpu

G = Path(__file__).resolve().parent / "golden"


@pytest.mark.parametrize("alignment", [32, 128])
def test_gguf_config1_greedy_matches_golden(engine, tmp_path, alignment):
    d = np.load(G / "greedy_c1.npz")
    path = tmp_path / "c1.gguf"
    synth.write_gguf(synth.tiny_config1(1), path, context_length=64, alignment=alignment)
    m = Model.from_gguf(engine, path)
    assert m.cfg.max_seq_len == 64
    assert m.generate(d["prompt"].tolist(), 16) == d["tokens"].tolist()
    m.forward([int(d["prompt"][-1])], [32])
    got = m.logits()[0]
    assert float(np.max(np.abs(got - d["logits0"])) / np.max(np.abs(d["logits0"]))) <= 2e-3
    m.close()


@pytest.mark.parametrize("qtype,gen", [(8, synth.random_q8_0), (2, synth.random_q4_0), (12, synth.random_q4_k),
                                       (13, synth.random_q5_k), (14, synth.random_q6_k)])
def test_gguf_quantised_embedding_is_the_f16_rounded_dequant(engine, tmp_path, qtype, gen):
    """A quantised token_embd.weight is loaded as the binary16 rounding of its
    GGML-order dequantisation: the model built from the file and one built
    from the oracle's table rounded with numpy give bitwise equal logits."""
    spec = synth.tiny_config1(2)
    emb = next(t for t in spec.tensors if t.name == "token_embd.weight")
    raw = gen(np.random.default_rng(40 + qtype), emb.n, emb.k)
    emb.ggml_type, emb.data = qtype, raw
    path = tmp_path / "q.gguf"
    synth.write_gguf(spec, path, context_length=64)
    a = Model.from_gguf(engine, path)
    table = O.dequant(qtype, raw.reshape(-1), emb.n, emb.k, ftz=False).reshape(emb.n, emb.k)
    emb.ggml_type, emb.data = 1, table.astype(np.float16).view(np.uint16)
    b = Model(engine, spec, max_seq_len=64)
    for pos, tok in enumerate([3, 500, 17, 3]):
        a.forward([tok], [pos])
        b.forward([tok], [pos])
        assert np.array_equal(a.logits(), b.logits()), (pos, tok)
    a.close()
    b.close()
