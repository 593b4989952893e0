"""Python mirror of janus-engine's operator layer over libjanus_hip.

Names, argument order and error behaviour follow the reference's
`compute::ops` functions (crates/janus-engine/src/compute/ops/mod.rs:31-43)
with the engine/encoder/pipeline-cache arguments folded into one
`ComputeEngine`. Buffers are torch tensors on the GPU (torch provides the
device memory and the stream; all arithmetic runs in the HIP kernels).
Errors raise `JanusError` carrying the reference-equivalent status code.
"""
from __future__ import annotations

import ctypes as C
from typing import Optional, Sequence

import numpy as np
import torch

from . import _lib
from ._lib import (DT_F16, DT_F32, DT_Q4_0, DT_Q4_K, DT_Q5_K, DT_Q6_K, DT_Q8_0, TIE_LAST,  # noqa: F401
                   TIE_WGSL, WEIGHT_FTZ_F16, JanusError, check)

_TORCH_DT = {torch.float32: DT_F32, torch.float16: DT_F16}


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    if t is None:
        return None
    if not t.is_cuda:
        raise ValueError("janus_amd ops take GPU tensors")
    if not t.is_contiguous():
        raise ValueError("janus_amd ops take contiguous tensors")
    return t.data_ptr()


def _dt(t: torch.Tensor) -> int:
    try:
        return _TORCH_DT[t.dtype]
    except KeyError:
        raise ValueError(f"unsupported activation dtype {t.dtype}") from None


class ComputeEngine:
    """ComputeEngine::new (compute/engine.rs:27-83).

    Owns a janus context on `device`, bound to torch's current stream so
    ordering with torch allocations and copies is implicit. `device=-1`
    creates a validation-only context (host-side argument checks, no GPU).
    """

    def __init__(self, device: int = 0):
        self.lib = _lib.load()
        self.device = device
        h = C.c_void_p()
        check(self.lib.janus_create(device, C.byref(h)))
        self.ctx = h
        if device >= 0:
            self.bind_stream()

    def bind_stream(self, stream: Optional[torch.cuda.Stream] = None) -> None:
        s = stream if stream is not None else torch.cuda.current_stream(self.device)
        check(self.lib.janus_set_stream(self.ctx, C.c_void_p(s.cuda_stream)), self.ctx)

    def sync(self) -> None:
        check(self.lib.janus_sync(self.ctx), self.ctx)

    def workspace_bytes(self) -> tuple[int, int]:
        """(attention, small-M GEMM) workspace sizes of the context."""
        a, g = C.c_size_t(), C.c_size_t()
        check(self.lib.janus_workspace_bytes(self.ctx, C.byref(a), C.byref(g)), self.ctx)
        return a.value, g.value

    def close(self) -> None:
        if self.ctx:
            self.lib.janus_destroy(self.ctx)
            self.ctx = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _check(self, status: int) -> None:
        check(status, self.ctx)


class GpuTensor:
    """GpuTensor (compute/tensor.rs:4-7): an uploaded, library-owned weight.

    `data` holds the tensor exactly as a GGUF file stores it (F32/F16 values,
    or Q4_0/Q8_0/Q4_K/Q5_K/Q6_K blocks) for logical shape [n rows][k cols].
    A Q6_K upload reports F16 afterwards, as the reference's loader does.
    """

    def __init__(self, engine: ComputeEngine, ggml_type: int, n: int, k: int, data, flags: int = 0):
        self.engine = engine
        self.ggml_type = ggml_type
        self.n, self.k = n, k
        buf = np.ascontiguousarray(data).view(np.uint8).reshape(-1)
        h = C.c_void_p()
        engine._check(engine.lib.janus_weight_upload(engine.ctx, ggml_type, n, k, buf.ctypes.data,
                                                     buf.nbytes, flags, C.byref(h)))
        self.handle = h
        # Q6_K is stored as binary16 after upload (compute/engine.rs:800-831)
        t = C.c_int()
        engine._check(engine.lib.janus_weight_info(h, C.byref(t), None, None, None))
        self.ggml_type = t.value

    def dequant(self) -> torch.Tensor:
        out = torch.empty(self.n, self.k, dtype=torch.float32, device=f"cuda:{self.engine.device}")
        self.engine._check(self.engine.lib.janus_weight_dequant(self.engine.ctx, self.handle, _ptr(out)))
        return out

    def free(self) -> None:
        if self.handle:
            self.engine.lib.janus_weight_free(self.engine.ctx, self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


# ---- matrix products (ops/quantized.rs:63-186) -----------------------------

def gemm_auto(engine: ComputeEngine, matrix_a: torch.Tensor, matrix_b: GpuTensor, output: torch.Tensor,
              batch_size: int, m: int, k: int, n: int) -> None:
    engine._check(engine.lib.janus_gemm_auto(engine.ctx, _ptr(matrix_a), _dt(matrix_a), matrix_b.handle,
                                             _ptr(output), _dt(output), batch_size, m, k, n))


def gemm_residual(engine: ComputeEngine, a: torch.Tensor, w: GpuTensor, residual: torch.Tensor,
                  output: torch.Tensor, rows: int) -> None:
    engine._check(engine.lib.janus_gemm_residual(engine.ctx, _ptr(a), _dt(a), w.handle, _ptr(residual),
                                                 _ptr(output), rows, w.k, w.n))


# ---- activations / elementwise (ops/activation.rs, ops/elementwise.rs) -------

def rmsnorm(engine, input, output, weights, batch_size: int, hidden_dim: int, epsilon: float) -> None:
    engine._check(engine.lib.janus_rmsnorm(engine.ctx, _ptr(input), _ptr(output), _dt(output), _ptr(weights),
                                           batch_size, hidden_dim, epsilon))


def silu(engine, input, output, size: int) -> None:
    engine._check(engine.lib.janus_silu(engine.ctx, _ptr(input), _ptr(output), size))


def elementwise_mul(engine, tensor_a, tensor_b, output, size: int) -> None:
    engine._check(engine.lib.janus_elementwise_mul(engine.ctx, _ptr(tensor_a), _ptr(tensor_b), _ptr(output), size))


def add_tensors(engine, tensor_a, tensor_b, output, size: int) -> None:
    engine._check(engine.lib.janus_add_tensors(engine.ctx, _ptr(tensor_a), _ptr(tensor_b), _ptr(output), size))


def swiglu(engine, gate, up, output, size: int) -> None:
    engine._check(engine.lib.janus_swiglu(engine.ctx, _ptr(gate), _ptr(up), _ptr(output), _dt(output), size))


# ---- RoPE (ops/rope.rs:48-115) -----------------------------------------------

def create_rope_cache(engine, max_seq_len: int, head_dim: int, theta_base: float) -> torch.Tensor:
    """Model::create_rope_cache (model/transformer/constructor.rs:454-489)."""
    t = torch.empty(max_seq_len * head_dim, dtype=torch.float32, device=f"cuda:{engine.device}")
    engine._check(engine.lib.janus_rope_table(engine.ctx, _ptr(t), max_seq_len, head_dim, theta_base))
    return t


def rope(engine, input, output, rope_cache, batch_size: int, num_heads: int, head_dim: int, position: int,
         positions: Optional[torch.Tensor] = None) -> None:
    engine._check(engine.lib.janus_rope(engine.ctx, _ptr(input), _ptr(output), _ptr(rope_cache), batch_size,
                                        num_heads, head_dim, position, _ptr(positions)))


# ---- KV cache (compute/cache/core.rs) -------------------------------------------

class KVCache:
    """KVCache::new / update / buffers (compute/cache/core.rs:60-324).

    Layout per cache: [num_layers][batch_size * max_seq_len][num_kv_heads][head_dim];
    sequence b owns rows [b * max_seq_len, (b + 1) * max_seq_len) of each layer.
    """

    def __init__(self, engine, batch_size: int, num_layers: int, max_seq_len: int, num_kv_heads: int,
                 head_dim: int, dtype: torch.dtype = torch.float32):
        self.engine = engine
        self.batch_size, self.num_layers, self.max_seq_len = batch_size, num_layers, max_seq_len
        self.num_kv_heads, self.head_dim = num_kv_heads, head_dim
        self.dtype = dtype
        shape = (num_layers, batch_size * max_seq_len, num_kv_heads, head_dim)
        dev = f"cuda:{engine.device}"
        self.key_cache = torch.zeros(shape, dtype=dtype, device=dev)
        self.value_cache = torch.zeros(shape, dtype=dtype, device=dev)
        self.position = 0

    def update(self, new_key, new_value, layer_idx: int, position: int) -> None:
        engine = self.engine
        engine._check(engine.lib.janus_kv_update(
            engine.ctx, _ptr(new_key), _ptr(new_value), _ptr(self.key_cache[layer_idx]),
            _ptr(self.value_cache[layer_idx]), _dt(self.key_cache), self.batch_size, self.num_kv_heads,
            self.head_dim, position, self.max_seq_len, None, None))
        self.position = position + 1

    def current_position(self) -> int:
        return self.position

    def buffers(self):
        return self.key_cache, self.value_cache

    def reset(self) -> None:
        self.position = 0


def kv_update(engine, k_new, v_new, k_cache, v_cache, batch: int, kv_heads: int, head_dim: int, position: int,
              max_seq_len: int, row_base=None, positions=None) -> None:
    engine._check(engine.lib.janus_kv_update(engine.ctx, _ptr(k_new), _ptr(v_new), _ptr(k_cache), _ptr(v_cache),
                                             _dt(k_cache), batch, kv_heads, head_dim, position, max_seq_len,
                                             _ptr(row_base), _ptr(positions)))


# ---- attention (ops/attention.rs:78-235) ------------------------------------------

def compute_attention(engine, query, key_cache, value_cache, output, batch_size: int, seq_len: int,
                      max_seq_len: int, num_heads: int, num_kv_heads: int, head_dim: int,
                      row_base: Optional[torch.Tensor] = None, seq_lens: Optional[torch.Tensor] = None,
                      max_len_hint: int = 0, scale: float = 0.0) -> None:
    """One decode query per sequence against one layer's cache slice."""
    engine._check(engine.lib.janus_attention(
        engine.ctx, _ptr(query), _ptr(key_cache), _ptr(value_cache), _dt(key_cache), _ptr(output), batch_size,
        num_heads, num_kv_heads, head_dim, seq_len, max_seq_len, _ptr(row_base), _ptr(seq_lens), max_len_hint,
        scale))


def compute_attention_noalloc(engine, query, key_cache, value_cache, output, batch_size: int, seq_len: int,
                              max_seq_len: int, num_heads: int, num_kv_heads: int, head_dim: int,
                              row_base: Optional[torch.Tensor] = None, seq_lens: Optional[torch.Tensor] = None,
                              max_len_hint: int = 0, scale: float = 0.0) -> None:
    """compute_attention through the allocation-free entry point (fixed
    per-device scratch; janus_attention_noalloc in include/janus_hip.h)."""
    engine._check(engine.lib.janus_attention_noalloc(
        engine.ctx, _ptr(query), _ptr(key_cache), _ptr(value_cache), _dt(key_cache), _ptr(output), batch_size,
        num_heads, num_kv_heads, head_dim, seq_len, max_seq_len, _ptr(row_base), _ptr(seq_lens), max_len_hint,
        scale))


# ---- embedding and sampling ---------------------------------------------------------

def embed_tokens(engine, table: GpuTensor, token_ids: Sequence[int], output) -> None:
    """Model::embed_tokens (model/transformer/embedding.rs:16-198)."""
    ids = np.ascontiguousarray(np.asarray(token_ids, dtype=np.uint32))
    engine._check(engine.lib.janus_embed(engine.ctx, table.handle, ids.ctypes.data, len(ids), _ptr(output)))


def argmax(engine, logits, output, vocab_size: int, batch_size: int, tie_rule: int = TIE_WGSL) -> None:
    """ops::argmax (ops/argmax.rs:50-107); tie_rule TIE_LAST gives Sampler::argmax."""
    engine._check(engine.lib.janus_argmax(engine.ctx, _ptr(logits), _ptr(output), vocab_size, batch_size, tie_rule))


def repetition_penalty(engine, logits, vocab_size: int, context: torch.Tensor, penalty: float) -> None:
    engine._check(engine.lib.janus_repetition_penalty(engine.ctx, _ptr(logits), vocab_size, _ptr(context),
                                                      context.numel(), penalty))
