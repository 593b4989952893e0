"""Synthetic GGUF tensors for tests and benchmarks (no checkpoints are used).

Every generator returns bytes laid out exactly as a GGUF file stores the
tensor (GGML block formats), so they go through the same upload path as real
weights. Shapes follow PyTorch's [out][in] order: n rows of k columns.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

QK = 32       # Q4_0 / Q8_0 block width
QK_K = 256    # K-quant super-block width


def f16_bits(x: np.ndarray) -> np.ndarray:
    """binary16 bit patterns of x, round to nearest even (numpy's float16)."""
    return np.asarray(x, dtype=np.float32).astype(np.float16).view(np.uint16)


def random_q4_0(rng: np.random.Generator, n: int, k: int, scale_sigma: float = 0.02) -> np.ndarray:
    """Q4_0 blocks: 16 bytes of nibbles uniform in 0..15, d = f16(|N(0, sigma)| / 8)."""
    assert k % QK == 0
    nb = n * (k // QK)
    out = np.empty((nb, 18), dtype=np.uint8)
    out[:, 2:] = np.frombuffer(rng.bytes(nb * 16), dtype=np.uint8).reshape(nb, 16)
    d = np.abs(rng.standard_normal(nb, dtype=np.float32)) * np.float32(scale_sigma / 8.0)
    out[:, :2] = f16_bits(d).view(np.uint8).reshape(nb, 2)
    return out.reshape(-1)


def random_q8_0(rng: np.random.Generator, n: int, k: int, scale_sigma: float = 0.02) -> np.ndarray:
    """Q8_0 blocks: 32 int8 uniform in [-127, 127], d = f16(|N(0, sigma)| / 127)."""
    assert k % QK == 0
    nb = n * (k // QK)
    out = np.empty((nb, 34), dtype=np.uint8)
    out[:, 2:] = rng.integers(-127, 128, size=(nb, 32), dtype=np.int8).view(np.uint8)
    d = np.abs(rng.standard_normal(nb, dtype=np.float32)) * np.float32(scale_sigma / 127.0)
    out[:, :2] = f16_bits(d).view(np.uint8).reshape(nb, 2)
    return out.reshape(-1)


def quantize_q4_k(w: np.ndarray) -> np.ndarray:
    """Quantise f32 weights [n, k] to GGML block_q4_K bytes.

    Per 32-weight sub-block: scale = (max - min) / 15, offset m = max(-min, 0);
    the eight scales and mins are then quantised to 6 bits against d =
    max(scale)/63 and dmin = max(m)/63 (binary16), and the nibbles rounded
    against the 6-bit values actually stored. Parity is judged on the stored
    bytes, so this quantiser's choices do not affect any comparison.
    """
    w = np.asarray(w, dtype=np.float32)
    n, k = w.shape
    assert k % QK_K == 0
    sb = w.reshape(-1, 8, 32)                       # [super-blocks, sub-blocks, 32]
    mn = np.minimum(sb.min(axis=2), 0.0)
    mx = sb.max(axis=2)
    scale = (mx - mn) / 15.0
    moff = -mn
    d = f16_bits(scale.max(axis=1) / 63.0)
    dmin = f16_bits(moff.max(axis=1) / 63.0)
    df = d.view(np.float16).astype(np.float32)
    dminf = dmin.view(np.float16).astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        sc = np.where(df[:, None] > 0, np.rint(scale / df[:, None]), 0).clip(0, 63).astype(np.uint8)
        mq = np.where(dminf[:, None] > 0, np.rint(moff / dminf[:, None]), 0).clip(0, 63).astype(np.uint8)
        eff_s = df[:, None] * sc.astype(np.float32)
        eff_m = dminf[:, None] * mq.astype(np.float32)
        q = np.where(eff_s[:, :, None] > 0, np.rint((sb + eff_m[:, :, None]) / eff_s[:, :, None]), 0)
    q = q.clip(0, 15).astype(np.uint8).reshape(-1, 4, 2, 32)   # [sb, j, lo/hi, t]
    nsb = sb.shape[0]
    scales = np.zeros((nsb, 12), dtype=np.uint8)
    scales[:, 0:4] = sc[:, 0:4] & 63
    scales[:, 4:8] = mq[:, 0:4] & 63
    scales[:, 8:12] = (sc[:, 4:8] & 15) | ((mq[:, 4:8] & 15) << 4)
    scales[:, 0:4] |= (sc[:, 4:8] >> 4) << 6
    scales[:, 4:8] |= (mq[:, 4:8] >> 4) << 6
    qs = (q[:, :, 0, :] | (q[:, :, 1, :] << 4)).reshape(nsb, 128)
    out = np.empty((nsb, 144), dtype=np.uint8)
    out[:, 0:2] = d.view(np.uint8).reshape(nsb, 2)
    out[:, 2:4] = dmin.view(np.uint8).reshape(nsb, 2)
    out[:, 4:16] = scales
    out[:, 16:] = qs
    return out.reshape(-1)


def random_q4_k(rng: np.random.Generator, n: int, k: int, sigma: float = 0.02) -> np.ndarray:
    return quantize_q4_k(rng.standard_normal((n, k), dtype=np.float32) * np.float32(sigma))


def random_q4_k_bytes(rng: np.random.Generator, n: int, k: int, sigma: float = 0.02) -> np.ndarray:
    """block_q4_K bytes drawn directly (no quantiser; ~100x faster for
    billion-weight models): nibbles and the twelve 6-bit scale bytes uniform,
    d and dmin = f16(|N(0, 1)| * sigma / 128), which puts the weights
    (d*sc)*q - dmin*m at the scale of N(0, sigma). Parity is judged on the
    stored bytes, so any valid bytes serve."""
    assert k % QK_K == 0
    nsb = n * (k // QK_K)
    out = np.empty((nsb, 144), dtype=np.uint8)
    out[:, 4:] = np.frombuffer(rng.bytes(nsb * 140), dtype=np.uint8).reshape(nsb, 140)
    dd = np.abs(rng.standard_normal((nsb, 2), dtype=np.float32)) * np.float32(sigma / 128.0)
    out[:, 0:4] = f16_bits(dd).view(np.uint8).reshape(nsb, 4)
    return out.reshape(-1)


def _k_scales(sc: np.ndarray, mq: np.ndarray) -> np.ndarray:
    """The 12-byte 6-bit scale/min packing shared by block_q4_K and block_q5_K."""
    scales = np.zeros((sc.shape[0], 12), dtype=np.uint8)
    scales[:, 0:4] = sc[:, 0:4] & 63
    scales[:, 4:8] = mq[:, 0:4] & 63
    scales[:, 8:12] = (sc[:, 4:8] & 15) | ((mq[:, 4:8] & 15) << 4)
    scales[:, 0:4] |= (sc[:, 4:8] >> 4) << 6
    scales[:, 4:8] |= (mq[:, 4:8] >> 4) << 6
    return scales


def quantize_q5_k(w: np.ndarray) -> np.ndarray:
    """Quantise f32 weights [n, k] to GGML block_q5_K bytes {d, dmin, scales[12],
    qh[32], qs[128]}: the Q4_K scheme with 5-bit values (scale = range / 31);
    bit 4 of the value for element 64j + 32h + t sits in bit 2j + h of qh[t]."""
    w = np.asarray(w, dtype=np.float32)
    n, k = w.shape
    assert k % QK_K == 0
    sb = w.reshape(-1, 8, 32)
    mn = np.minimum(sb.min(axis=2), 0.0)
    scale = (sb.max(axis=2) - mn) / 31.0
    moff = -mn
    d = f16_bits(scale.max(axis=1) / 63.0)
    dmin = f16_bits(moff.max(axis=1) / 63.0)
    df = d.view(np.float16).astype(np.float32)
    dminf = dmin.view(np.float16).astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        sc = np.where(df[:, None] > 0, np.rint(scale / df[:, None]), 0).clip(0, 63).astype(np.uint8)
        mq = np.where(dminf[:, None] > 0, np.rint(moff / dminf[:, None]), 0).clip(0, 63).astype(np.uint8)
        eff_s = df[:, None] * sc.astype(np.float32)
        eff_m = dminf[:, None] * mq.astype(np.float32)
        q = np.where(eff_s[:, :, None] > 0, np.rint((sb + eff_m[:, :, None]) / eff_s[:, :, None]), 0)
    q = q.clip(0, 31).astype(np.uint8).reshape(-1, 4, 2, 32)   # [sb, j, lo/hi, t]
    nsb = sb.shape[0]
    qs = ((q[:, :, 0, :] & 15) | ((q[:, :, 1, :] & 15) << 4)).reshape(nsb, 128)
    qh = np.zeros((nsb, 32), dtype=np.uint8)
    for j in range(4):
        qh |= ((q[:, j, 0, :] >> 4) << (2 * j)).astype(np.uint8)
        qh |= ((q[:, j, 1, :] >> 4) << (2 * j + 1)).astype(np.uint8)
    out = np.empty((nsb, 176), dtype=np.uint8)
    out[:, 0:2] = d.view(np.uint8).reshape(nsb, 2)
    out[:, 2:4] = dmin.view(np.uint8).reshape(nsb, 2)
    out[:, 4:16] = _k_scales(sc, mq)
    out[:, 16:48] = qh
    out[:, 48:] = qs
    return out.reshape(-1)


def random_q5_k(rng: np.random.Generator, n: int, k: int, sigma: float = 0.02) -> np.ndarray:
    return quantize_q5_k(rng.standard_normal((n, k), dtype=np.float32) * np.float32(sigma))


def quantize_q6_k(w: np.ndarray) -> np.ndarray:
    """Quantise f32 weights [n, k] to GGML block_q6_K bytes {ql[128], qh[64],
    scales[16] (int8), d}: per 16-element group an int8 scale against d =
    max(group scale) / 127, values q + 32 in 0..63. Element 128h + 32p + l
    keeps its low nibble in nibble p // 2 of ql[64h + l + 32 (p % 2)] and its
    two high bits in bits 2p of qh[32h + l]."""
    w = np.asarray(w, dtype=np.float32)
    n, k = w.shape
    assert k % QK_K == 0
    g = w.reshape(-1, 16, 16)
    nsb = g.shape[0]
    gs = np.abs(g).max(axis=2) / 31.0
    d = f16_bits(gs.max(axis=1) / 127.0)
    df = d.view(np.float16).astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        sc = np.where(df[:, None] > 0, np.rint(gs / df[:, None]), 0).clip(-128, 127).astype(np.int8)
        eff = df[:, None] * sc.astype(np.float32)
        q = np.where(eff[:, :, None] != 0, np.rint(g / eff[:, :, None]), 0)
    q = (q.clip(-32, 31) + 32).astype(np.uint8).reshape(nsb, 2, 4, 32)   # [sb, h, p, l]
    ql = np.zeros((nsb, 2, 64), dtype=np.uint8)
    qh = np.zeros((nsb, 2, 32), dtype=np.uint8)
    for p in range(4):
        ql[:, :, 32 * (p % 2):32 * (p % 2) + 32] |= ((q[:, :, p, :] & 15) << (4 * (p // 2))).astype(np.uint8)
        qh |= ((q[:, :, p, :] >> 4) << (2 * p)).astype(np.uint8)
    out = np.empty((nsb, 210), dtype=np.uint8)
    out[:, 0:128] = ql.reshape(nsb, 128)
    out[:, 128:192] = qh.reshape(nsb, 64)
    out[:, 192:208] = sc.view(np.uint8)
    out[:, 208:210] = d.view(np.uint8).reshape(nsb, 2)
    return out.reshape(-1)


def random_q6_k(rng: np.random.Generator, n: int, k: int, sigma: float = 0.02) -> np.ndarray:
    return quantize_q6_k(rng.standard_normal((n, k), dtype=np.float32) * np.float32(sigma))


@dataclass
class Tensor:
    """One GGUF tensor: GGML type id, logical shape (n, k) (k = 0 for 1-D) and bytes."""
    name: str
    ggml_type: int
    n: int
    k: int
    data: np.ndarray


@dataclass
class ModelSpec:
    hidden: int
    heads: int
    kv_heads: int
    ffn: int
    vocab: int
    layers: int
    rms_eps: float = 1e-5
    rope_theta: float = 10000.0
    tensors: list = field(default_factory=list)

    @property
    def head_dim(self) -> int:
        return self.hidden // self.heads


F32, F16, Q4_0, Q8_0, Q4_K, Q5_K, Q6_K = 0, 1, 2, 8, 12, 13, 14


def _mat(rng, name, qtype, n, k, kquant_bytes=False):
    if qtype == Q4_0:
        return Tensor(name, Q4_0, n, k, random_q4_0(rng, n, k))
    if qtype == Q8_0:
        return Tensor(name, Q8_0, n, k, random_q8_0(rng, n, k))
    if qtype == Q4_K:
        return Tensor(name, Q4_K, n, k, random_q4_k_bytes(rng, n, k) if kquant_bytes else random_q4_k(rng, n, k))
    if qtype == Q5_K:
        return Tensor(name, Q5_K, n, k, random_q5_k(rng, n, k))
    if qtype == Q6_K:
        return Tensor(name, Q6_K, n, k, random_q6_k(rng, n, k))
    if qtype == F16:
        return Tensor(name, F16, n, k, f16_bits(rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02)))
    return Tensor(name, F32, n, k, rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02))


def make_model(seed: int, hidden: int, heads: int, kv_heads: int, ffn: int, vocab: int, layers: int,
               qtype: int, rms_eps: float = 1e-5, rope_theta: float = 10000.0, embed_type: int = F32,
               head_type: int = F32, down_type: int | None = None, kquant_bytes: bool = False) -> ModelSpec:
    """Random-init Llama-architecture tensors with GGUF names.

    Embeddings ~ N(0, 1); norms ~ 1 + N(0, 0.02); the LM head ~ N(0, 0.02) in
    F32 or F16 (the reference only runs the LM head as an f16 GEMM); block
    matrices in `qtype`, ffn_down in `down_type` when given (a Q8_0 ffn_down
    with ffn % 32 != 0 is rejected by the reference, ops/quantized.rs:327-332).
    kquant_bytes draws Q4_K blocks directly (random_q4_k_bytes) instead of
    quantising N(0, 0.02) weights.
    """
    rng = np.random.default_rng(seed)
    spec = ModelSpec(hidden, heads, kv_heads, ffn, vocab, layers, rms_eps, rope_theta)
    kvd = kv_heads * (hidden // heads)
    emb = rng.standard_normal((vocab, hidden), dtype=np.float32)
    spec.tensors.append(Tensor("token_embd.weight", embed_type, vocab, hidden,
                               emb if embed_type == F32 else f16_bits(emb)))
    for l in range(layers):
        p = f"blk.{l}."
        spec.tensors.append(Tensor(p + "attn_norm.weight", F32, hidden, 0,
                                   1 + rng.standard_normal(hidden, dtype=np.float32) * np.float32(0.02)))
        kb = kquant_bytes
        spec.tensors.append(_mat(rng, p + "attn_q.weight", qtype, hidden, hidden, kb))
        spec.tensors.append(_mat(rng, p + "attn_k.weight", qtype, kvd, hidden, kb))
        spec.tensors.append(_mat(rng, p + "attn_v.weight", qtype, kvd, hidden, kb))
        spec.tensors.append(_mat(rng, p + "attn_output.weight", qtype, hidden, hidden, kb))
        spec.tensors.append(Tensor(p + "ffn_norm.weight", F32, hidden, 0,
                                   1 + rng.standard_normal(hidden, dtype=np.float32) * np.float32(0.02)))
        spec.tensors.append(_mat(rng, p + "ffn_gate.weight", qtype, ffn, hidden, kb))
        spec.tensors.append(_mat(rng, p + "ffn_up.weight", qtype, ffn, hidden, kb))
        spec.tensors.append(_mat(rng, p + "ffn_down.weight", down_type if down_type is not None else qtype,
                                 hidden, ffn, kb))
    spec.tensors.append(Tensor("output_norm.weight", F32, hidden, 0,
                               1 + rng.standard_normal(hidden, dtype=np.float32) * np.float32(0.02)))
    spec.tensors.append(_mat(rng, "output.weight", head_type, vocab, hidden))
    return spec


def tiny_config1(seed: int = 1) -> ModelSpec:
    """benchmark configuration 1: 2 layers, hidden 256, 4 heads x 64, 2 KV heads, FFN 688,
    vocab 512, eps 1e-5, theta 1e4, Q8_0 blocks; ffn_down F32 because 688 % 32 != 0."""
    return make_model(seed, 256, 4, 2, 688, 512, 2, Q8_0, 1e-5, 10000.0, F32, F32, down_type=F32)


def write_gguf(spec: ModelSpec, path, context_length: int = 4096, alignment: int = 32) -> None:
    """Write a spec as a Llama-architecture GGUF file: the metadata keys
    model_config_from_gguf_metadata reads (model/config.rs:377-446) and every
    tensor with its dimensions innermost first ([k, n] for a 2-D [n][k] weight)."""
    from . import gguf as G
    md = {"general.architecture": G.Value(G.STRING, "llama"),
          "llama.embedding_length": G.Value(G.UINT32, spec.hidden),
          "llama.block_count": G.Value(G.UINT32, spec.layers),
          "llama.attention.head_count": G.Value(G.UINT32, spec.heads),
          "llama.attention.head_count_kv": G.Value(G.UINT32, spec.kv_heads),
          "llama.feed_forward_length": G.Value(G.UINT32, spec.ffn),
          "llama.context_length": G.Value(G.UINT32, context_length),
          "llama.attention.layer_norm_rms_epsilon": G.Value(G.FLOAT32, spec.rms_eps),
          "llama.rope.freq_base": G.Value(G.FLOAT32, spec.rope_theta),
          "llama.vocab_size": G.Value(G.UINT32, spec.vocab)}
    tensors = [(t.name, [t.k, t.n] if t.k else [t.n], t.ggml_type, t.data) for t in spec.tensors]
    G.write(path, md, tensors, alignment=alignment)
