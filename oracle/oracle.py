"""numpy/ctypes front end of the CPU oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY. This module restates janus-engine's decode
arithmetic on the CPU so tests can check the HIP path against it. Only
tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
it, and only as the checker or the CPU baseline -- never as the product path.

The element-level arithmetic lives in janus_oracle.c (each function cites its
reference file:line). The model-level driver below follows
crates/janus-engine/src/model/block.rs:190-458 (per-layer op order),
model/transformer/forward.rs:25-119 (embed -> blocks -> norm -> LM head) and
model/transformer/generation.rs:129-323 with model/sampler.rs:146-209
(prefill, re-fed last prompt token, penalty 1.15 over generated tokens,
last-max argmax).
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
# JANUS_ORACLE_LIB: another build of the oracle (the sanitised one of `make asan`)
LIB_PATH = Path(os.environ.get("JANUS_ORACLE_LIB") or HERE / "liboracle.so")

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(dtype=np.float64, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(dtype=np.uint8, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(dtype=np.uint16, flags="C_CONTIGUOUS")
_u32p = np.ctypeslib.ndpointer(dtype=np.uint32, flags="C_CONTIGUOUS")
U32, SZ, F32, I32 = C.c_uint32, C.c_size_t, C.c_float, C.c_int

_SIG = {
    "jo_f16_to_f32_exact": (F32, [C.c_uint16]),
    "jo_f16_to_f32_q8": (F32, [C.c_uint16]),
    "jo_f16_to_f32_ftz": (F32, [C.c_uint16]),
    "jo_f32_to_f16_rne": (C.c_uint16, [F32]),
    "jo_f32_to_f16_rne_n": (None, [_f32p, _u16p, SZ]),
    "jo_f16_to_f32_n": (None, [_u16p, _f32p, SZ, I32]),
    "jo_dequant_q8_0": (None, [_u8p, SZ, _f32p]),
    "jo_dequant_q4_0": (None, [_u8p, SZ, _f32p]),
    "jo_dequant_q4_k": (None, [_u8p, SZ, I32, _f32p]),
    "jo_q4_k_scale_min": (None, [_u8p, I32, C.POINTER(C.c_uint8), C.POINTER(C.c_uint8)]),
    "jo_dequant_q5_k": (None, [_u8p, SZ, I32, _f32p]),
    "jo_gemv_q5_k": (None, [_u8p, _f32p, _f32p, U32, U32, I32]),
    "jo_dequant_q6_k": (None, [_u8p, SZ, I32, _f32p]),
    "jo_gemv_q8_0": (None, [_u8p, _f32p, _f32p, U32, U32]),
    "jo_gemv_q4_k": (None, [_u8p, _f32p, _f32p, U32, U32, I32]),
    "jo_gemv_q4_0": (None, [_u8p, _f32p, _f32p, U32, U32]),
    "jo_gemv_q4_0_mt": (None, [_u8p, _f32p, _f32p, U32, U32]),
    "jo_gemm_f16": (None, [_f32p, _u16p, _f32p, U32, U32, U32, U32]),
    "jo_gemv_f64": (None, [_f32p, _f32p, _f64p, U32, U32]),
    "jo_rmsnorm": (None, [_f32p, _f32p, _f32p, U32, U32, F32]),
    "jo_silu": (None, [_f32p, _f32p, SZ]),
    "jo_mul": (None, [_f32p, _f32p, _f32p, SZ]),
    "jo_add": (None, [_f32p, _f32p, _f32p, SZ]),
    "jo_rope_table": (None, [_f32p, U32, U32, F32]),
    "jo_rope": (None, [_f32p, _f32p, _f32p, U32, U32, U32, U32]),
    "jo_attention": (None, [_f32p, _f32p, _f32p, _f32p, U32, U32, U32, U32, F32]),
    "jo_embed": (I32, [_u16p, _u32p, _f32p, U32, U32, U32]),
    "jo_repetition_penalty": (None, [_f32p, U32, _u32p, SZ, F32]),
    "jo_argmax_last": (U32, [_f32p, U32]),
    "jo_argmax_wgsl": (U32, [_f32p, U32]),
    "jo_num_threads": (I32, []),
}

_lib = None


def lib():
    """Load liboracle.so, building it with oracle/Makefile if it is missing."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            subprocess.run(["make", "-s", "-C", str(HERE), "liboracle.so"], check=True)
        L = C.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIG.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


# ---- binary16 --------------------------------------------------------------

def f32_to_f16_rne(x) -> np.ndarray:
    x = _f32(x).reshape(-1)
    out = np.empty(x.size, dtype=np.uint16)
    lib().jo_f32_to_f16_rne_n(x, out, x.size)
    return out


def f16_to_f32(bits, mode: str = "exact") -> np.ndarray:
    b = np.ascontiguousarray(bits, dtype=np.uint16).reshape(-1)
    out = np.empty(b.size, dtype=np.float32)
    lib().jo_f16_to_f32_n(b, out, b.size, {"exact": 0, "q8": 1, "ftz": 2}[mode])
    return out


# ---- dequantisation and products ------------------------------------------------

def dequant(ggml_type: int, data: np.ndarray, n: int, k: int, ftz: bool = False,
            q6k_ref_order: bool = False) -> np.ndarray:
    """Reference dequantisation of GGUF bytes (or F32/F16 values) to f32 [n, k].
    Q6_K uses GGML's element order unless q6k_ref_order selects the
    reference loader's (compute/engine.rs:198-248)."""
    L = lib()
    out = np.empty(n * k, dtype=np.float32)
    if ggml_type == 8:
        L.jo_dequant_q8_0(np.ascontiguousarray(data, dtype=np.uint8), n * k // 32, out)
    elif ggml_type == 2:
        L.jo_dequant_q4_0(np.ascontiguousarray(data, dtype=np.uint8), n * k // 32, out)
    elif ggml_type == 12:
        L.jo_dequant_q4_k(np.ascontiguousarray(data, dtype=np.uint8), n * k // 256, int(ftz), out)
    elif ggml_type == 13:
        L.jo_dequant_q5_k(np.ascontiguousarray(data, dtype=np.uint8), n * k // 256, int(ftz), out)
    elif ggml_type == 14:
        L.jo_dequant_q6_k(np.ascontiguousarray(data, dtype=np.uint8), n * k // 256, int(q6k_ref_order), out)
    elif ggml_type == 1:
        out = f16_to_f32(np.asarray(data).view(np.uint16), "ftz" if ftz else "exact")
    elif ggml_type == 0:
        bits = f32_to_f16_rne(np.asarray(data, dtype=np.float32))
        out = f16_to_f32(bits, "ftz" if ftz else "exact")
    else:
        raise ValueError(ggml_type)
    return out.reshape(n, k)


def weight_f16_bits(ggml_type: int, data: np.ndarray) -> np.ndarray:
    """Packed binary16 storage of a 2-D float tensor (compute/engine.rs:471-566)."""
    if ggml_type == 0:
        return f32_to_f16_rne(np.asarray(data, dtype=np.float32))
    return np.ascontiguousarray(np.asarray(data).view(np.uint16)).reshape(-1)


def gemm_auto(x: np.ndarray, ggml_type: int, data: np.ndarray, n: int, k: int) -> np.ndarray:
    """gemm_auto at M=1 for one f32 row x [k] (ops/quantized.rs:63-186)."""
    L = lib()
    x = _f32(x).reshape(-1)
    y = np.empty(n, dtype=np.float32)
    if ggml_type == 8:
        L.jo_gemv_q8_0(np.ascontiguousarray(data, dtype=np.uint8), x, y, n, k)
    elif ggml_type == 12:
        L.jo_gemv_q4_k(np.ascontiguousarray(data, dtype=np.uint8), x, y, n, k, 1)
    elif ggml_type == 13:
        L.jo_gemv_q5_k(np.ascontiguousarray(data, dtype=np.uint8), x, y, n, k, 0)
    elif ggml_type == 14:
        # the reference loads Q6_K as binary16 weights (engine.rs:800-831)
        bits = f32_to_f16_rne(dequant(14, data, n, k))
        L.jo_gemm_f16(x, bits, y, 1, 1, k, n)
    elif ggml_type == 2:
        L.jo_gemv_q4_0(np.ascontiguousarray(data, dtype=np.uint8), x, y, n, k)
    elif ggml_type in (0, 1):
        L.jo_gemm_f16(x, weight_f16_bits(ggml_type, data), y, 1, 1, k, n)
    else:
        raise ValueError(ggml_type)
    return y


def gemv_f64(w_f32: np.ndarray, x: np.ndarray) -> np.ndarray:
    n, k = w_f32.shape
    y = np.empty(n, dtype=np.float64)
    lib().jo_gemv_f64(_f32(w_f32), _f32(x), y, n, k)
    return y


def rmsnorm(x: np.ndarray, gamma: np.ndarray, eps: float) -> np.ndarray:
    x = _f32(x)
    b, h = (1, x.size) if x.ndim == 1 else x.shape
    out = np.empty_like(x)
    lib().jo_rmsnorm(x, out, _f32(gamma), b, h, eps)
    return out


def silu(x) -> np.ndarray:
    x = _f32(x)
    out = np.empty_like(x)
    lib().jo_silu(x, out, x.size)
    return out


def mul(a, b) -> np.ndarray:
    a, b = _f32(a), _f32(b)
    out = np.empty_like(a)
    lib().jo_mul(a, b, out, a.size)
    return out


def add(a, b) -> np.ndarray:
    a, b = _f32(a), _f32(b)
    out = np.empty_like(a)
    lib().jo_add(a, b, out, a.size)
    return out


def rope_table(max_seq: int, head_dim: int, base: float) -> np.ndarray:
    t = np.empty(max_seq * head_dim, dtype=np.float32)
    lib().jo_rope_table(t, max_seq, head_dim, base)
    return t


def rope(x: np.ndarray, table: np.ndarray, heads: int, head_dim: int, position: int, batch: int = 1) -> np.ndarray:
    x = _f32(x)
    out = np.empty_like(x)
    lib().jo_rope(x, out, _f32(table), batch, heads, head_dim, position)
    return out


def attention(q, k, v, heads: int, kv_heads: int, head_dim: int, scale: float | None = None) -> np.ndarray:
    """One sequence: q [H*hd], k/v [len, kvh, hd] f32 -> out [H*hd]."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    length = k.size // (kv_heads * head_dim)
    if scale is None:
        scale = float(np.float32(1.0) / np.sqrt(np.float32(head_dim)))
    out = np.empty(heads * head_dim, dtype=np.float32)
    lib().jo_attention(q.reshape(-1), k.reshape(-1) if length else np.zeros(1, np.float32),
                       v.reshape(-1) if length else np.zeros(1, np.float32), out, length, heads, kv_heads,
                       head_dim, scale)
    return out


def argmax_last(logits) -> int:
    l = _f32(logits)
    return int(lib().jo_argmax_last(l, l.size))


def argmax_wgsl(logits) -> int:
    l = _f32(logits)
    return int(lib().jo_argmax_wgsl(l, l.size))


def greedy_sample(logits, context, penalty: float = 1.15, batch: bool = False) -> int:
    """Sampler::sample with temperature 0 (model/sampler.rs:146-209): with
    |penalty - 1| < 0.01 the GPU argmax of argmax.wgsl (no penalty, its tie
    rule, :154-160), otherwise the penalty over the context and the last-max
    argmax. batch=True is Sampler::sample_batch (:379-428), which always
    applies the penalty and the last-max argmax."""
    l = _f32(logits).copy()
    if not batch and abs(np.float32(penalty) - np.float32(1.0)) < np.float32(0.01):
        return argmax_wgsl(l)
    if np.isnan(l).any():
        raise FloatingPointError("NaN logits")
    ctx = np.ascontiguousarray(np.asarray(context, dtype=np.uint32))
    lib().jo_repetition_penalty(l, l.size, ctx, ctx.size, penalty)
    return argmax_last(l)


# ---- model-level driver -------------------------------------------------------------

class OracleModel:
    """CPU restatement of Model::forward / generate for a synth.ModelSpec.

    kv_f16=True rounds K and V to binary16 on append (the fp16-KV parity mode);
    otherwise the cache is f32 like the reference's (compute/cache/core.rs:60-88).

    act_f16=True also rounds to binary16 every product input that the build's
    binary16-activation decode path holds in binary16: the attention RMSNorm
    output, the attention output, the FFN RMSNorm output, the SwiGLU output
    and the final RMSNorm output (the residual stream, q and the logits stay
    f32). The reference keeps these in f32; this mode separates the build's
    storage choice from its arithmetic, so a step whose logits are sensitive
    to activation rounding is compared with the same rounding applied.
    """

    def __init__(self, spec, max_seq_len: int = 256, kv_f16: bool = False, act_f16: bool = False):
        self.spec = spec
        self.max_seq_len = max_seq_len
        self.kv_f16 = kv_f16
        self.act_f16 = act_f16
        self.t = {t.name: t for t in spec.tensors}
        self.table = rope_table(max_seq_len, spec.head_dim, spec.rope_theta)
        emb = self.t["token_embd.weight"]
        self.embed_bits = weight_f16_bits(emb.ggml_type, emb.data).reshape(spec.vocab, spec.hidden)
        kvd = spec.kv_heads * spec.head_dim
        self.k = np.zeros((spec.layers, max_seq_len, kvd), dtype=np.float32)
        self.v = np.zeros((spec.layers, max_seq_len, kvd), dtype=np.float32)

    def _mm(self, name: str, x: np.ndarray) -> np.ndarray:
        t = self.t[name]
        return gemm_auto(x, t.ggml_type, t.data, t.n, t.k)

    def _vec(self, name: str) -> np.ndarray:
        return _f32(self.t[name].data)

    def reset(self) -> None:
        self.k[:] = 0
        self.v[:] = 0

    def forward(self, token: int, pos: int) -> np.ndarray:
        s = self.spec
        if token >= s.vocab:
            raise IndexError("token id exceeds vocab")
        if pos >= self.max_seq_len:
            raise IndexError("KV cache position exceeds max_seq_len")
        h16 = (lambda a: a.astype(np.float16).astype(np.float32)) if self.act_f16 else (lambda a: a)
        x = f16_to_f32(self.embed_bits[token], "ftz")                        # embed.wgsl
        for l in range(s.layers):
            p = f"blk.{l}."
            xn = h16(rmsnorm(x, self._vec(p + "attn_norm.weight"), s.rms_eps))
            q = self._mm(p + "attn_q.weight", xn)
            k = self._mm(p + "attn_k.weight", xn)
            v = self._mm(p + "attn_v.weight", xn)
            q = rope(q, self.table, s.heads, s.head_dim, pos)
            k = rope(k, self.table, s.kv_heads, s.head_dim, pos)
            if self.kv_f16:
                k = k.astype(np.float16).astype(np.float32)
                v = v.astype(np.float16).astype(np.float32)
            self.k[l, pos] = k
            self.v[l, pos] = v
            att = h16(attention(q, self.k[l, : pos + 1], self.v[l, : pos + 1], s.heads, s.kv_heads, s.head_dim))
            h1 = add(x, self._mm(p + "attn_output.weight", att))
            fn = h16(rmsnorm(h1, self._vec(p + "ffn_norm.weight"), s.rms_eps))
            g = self._mm(p + "ffn_gate.weight", fn)
            u = self._mm(p + "ffn_up.weight", fn)
            act = h16(mul(silu(g), u))
            x = add(h1, self._mm(p + "ffn_down.weight", act))
        xn = h16(rmsnorm(x, self._vec("output_norm.weight"), s.rms_eps))
        return self._mm("output.weight", xn)

    def generate(self, prompt, max_tokens: int, penalty: float = 1.15, return_logits: bool = False,
                 batch_rules: bool = False):
        """Model::generate (generation.rs:129-323): prefill, re-feed the last
        prompt token at position n, then sample until max_tokens, max_seq_len
        or 128001/128009, which is not pushed (:241-260).

        batch_rules=True follows one sequence of Model::generate_batch
        (generation.rs:765-833) as the build's continuous batching runs it:
        Sampler::sample_batch's rules, and the stop token is pushed before the
        check."""
        self.reset()
        pos = 0
        for tok in prompt:
            self.forward(int(tok), pos)
            pos += 1
        last = int(prompt[-1])
        generated, all_logits = [], []
        for _ in range(max_tokens):
            if pos >= self.max_seq_len:
                break
            logits = self.forward(last, pos)
            all_logits.append(logits)
            nxt = greedy_sample(logits, generated, penalty, batch=batch_rules)
            if nxt in (128001, 128009):
                if batch_rules:
                    generated.append(nxt)
                break
            generated.append(nxt)
            last = nxt
            pos += 1
        return (generated, all_logits) if return_logits else generated
