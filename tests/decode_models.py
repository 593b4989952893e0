"""Small models with planted LM heads shared by the decode-loop GPU tests
(built on the CPU; the oracle supplies the hidden state a head is aimed at)."""
import numpy as np

from janus_amd import synth
from oracle import oracle as O


def prompt(seed, n, vocab):
    return np.random.default_rng(seed).integers(0, vocab, n).tolist()


def eos_model(pa=(11, 22, 33), layers=1):
    """Vocabulary of 128256 with an LM head that is zero except row 128009, set
    to the sign pattern of the normalised hidden state of prompt pa's first
    decode step (the re-fed last prompt token at position len(pa), computed by
    the oracle), and a weaker row 77: pa's first sampled token is the stop
    token 128009; for other prompts the oracle decides."""
    s = synth.make_model(83, 256, 4, 2, 512, 128256, layers, synth.Q8_0, 1e-5, 10000.0,
                         embed_type=synth.F16, head_type=synth.F16)
    ref = O.OracleModel(s, 16)
    for p, t in enumerate(pa):
        ref.forward(t, p)
    xs = {}
    orig = O.rmsnorm

    def spy(x, gamma, eps):
        xs["last"] = np.array(x, copy=True)
        return orig(x, gamma, eps)

    O.rmsnorm = spy
    try:
        ref.forward(pa[-1], len(pa))
    finally:
        O.rmsnorm = orig
    xn = O.rmsnorm(xs["last"], [t for t in s.tensors if t.name == "output_norm.weight"][0].data, s.rms_eps)
    head = np.zeros((s.vocab, s.hidden), np.float32)
    head[128009] = np.sign(xn) * np.float32(0.05)
    head[77] = np.sign(xn) * np.float32(0.01)
    s.tensors = [t for t in s.tensors if t.name != "output.weight"]
    s.tensors.append(synth.Tensor("output.weight", synth.F16, s.vocab, s.hidden, synth.f16_bits(head)))
    return s


def nan_head_model():
    """A one-layer model whose F16 LM head holds a NaN in row 321, so every
    step's logit 321 is NaN."""
    s = synth.make_model(97, 256, 4, 2, 512, 1000, 1, synth.Q8_0, 1e-5, 10000.0,
                         embed_type=synth.F16, head_type=synth.F16)
    head = [t for t in s.tensors if t.name == "output.weight"][0]
    bits = np.array(head.data, dtype=np.uint16, copy=True).reshape(s.vocab, s.hidden)
    bits[321, 17] = 0x7E00
    s.tensors = [t for t in s.tensors if t.name != "output.weight"]
    s.tensors.append(synth.Tensor("output.weight", synth.F16, s.vocab, s.hidden, bits.reshape(-1)))
    return s
