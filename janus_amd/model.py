"""Python handle on the C++ decode driver (include/janus_model.h).

Mirrors the reference's Model API shape: construct from a config and GGUF
tensors (Model::new, model/transformer/constructor.rs:23-437), run
`forward(token, pos)` (forward.rs:25-119) and `generate` with the reference's
loop and greedy-sampler semantics (generation.rs:129-323).
"""
from __future__ import annotations

import ctypes as C
from typing import Callable, Sequence

import numpy as np

from . import _lib, gguf, ops
from ._lib import DT_F16, DT_F32, DT_Q4_0, DT_Q4_K, DT_Q5_K, DT_Q6_K, DT_Q8_0, ModelConfig, check
from .ops import ComputeEngine
from .synth import ModelSpec, Tensor


class Model:
    def __init__(self, engine: ComputeEngine, spec: ModelSpec, max_seq_len: int = 256, max_batch: int = 1,
                 kv_dtype: int = DT_F32, act_dtype: int = DT_F32):
        self.engine = engine
        self.lib = engine.lib
        self.spec = spec
        cfg = ModelConfig(spec.hidden, spec.heads, spec.kv_heads, spec.head_dim, spec.ffn, spec.vocab,
                          spec.layers, max_seq_len, max_batch, spec.rms_eps, spec.rope_theta, kv_dtype, act_dtype)
        self.cfg = cfg
        h = C.c_void_p()
        self._check(self.lib.janus_model_create(engine.ctx, C.byref(cfg), C.byref(h)))
        self.handle = h
        for t in spec.tensors:
            buf = np.ascontiguousarray(t.data).view(np.uint8).reshape(-1)
            self._check(self.lib.janus_model_set_tensor(h, t.name.encode(), t.ggml_type, t.n, t.k,
                                                        buf.ctypes.data, buf.nbytes))
        self._check(self.lib.janus_model_validate(h))

    @classmethod
    def from_gguf(cls, engine: ComputeEngine, path, max_seq_len: int | None = None, max_batch: int = 1,
                  kv_dtype: int = DT_F32, act_dtype: int = DT_F32) -> "Model":
        """Model::new from a GGUF file (model/transformer/constructor.rs:23-437):
        the config from the file's metadata (model/config.rs:377-446; max_seq_len
        defaults to its clamped context_length) and every tensor handed to the
        weight upload as the file stores it, read through the memory map.

        A quantised token_embd.weight (Q4_0 / Q8_0 / Q4_K / Q5_K / Q6_K) becomes a binary16
        table as allocate_tensors does (compute/engine.rs:635-771), but in GGML
        element order for every format: the blocks are dequantised on the GPU by
        the weight upload's closed form and rounded to binary16 (RNE). The
        reference's own Q4_K embedding path uses a non-GGML order
        (engine.rs:267-316) and is not followed."""
        f = gguf.GgufFile(path)
        try:
            c = gguf.config_from_metadata(f.meta.metadata)
            m = cls(engine, ModelSpec(c.hidden, c.heads, c.kv_heads, c.ffn, c.vocab, c.layers, c.rms_eps,
                                      c.rope_theta, [_gguf_tensor(engine, f, t) for t in f.tensors]),
                    max_seq_len or c.max_seq_len, max_batch, kv_dtype, act_dtype)
            # the weights are uploaded: drop the views into the mapping
            m.spec = ModelSpec(c.hidden, c.heads, c.kv_heads, c.ffn, c.vocab, c.layers, c.rms_eps, c.rope_theta)
            return m
        finally:
            f.close()

    def _check(self, status: int) -> None:
        check(status, self.engine.ctx)

    def close(self) -> None:
        if getattr(self, "handle", None):
            self.lib.janus_model_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def forward(self, tokens: Sequence[int], positions: Sequence[int], slots: Sequence[int] | None = None) -> None:
        """One decode step (Model::forward / forward_batch); sequence s uses KV
        slot slots[s] (default s)."""
        t = np.ascontiguousarray(np.asarray(tokens, dtype=np.uint32))
        p = np.ascontiguousarray(np.asarray(positions, dtype=np.uint32))
        if slots is None:
            self._check(self.lib.janus_model_forward(self.handle, t.ctypes.data, p.ctypes.data, len(t)))
        else:
            s = np.ascontiguousarray(np.asarray(slots, dtype=np.uint32))
            self._check(self.lib.janus_model_forward_slots(self.handle, t.ctypes.data, p.ctypes.data,
                                                           s.ctypes.data, len(t)))

    def logits(self, nseq: int = 1) -> np.ndarray:
        out = np.empty((nseq, self.spec.vocab), dtype=np.float32)
        self._check(self.lib.janus_model_read_logits(self.handle, out.ctypes.data, nseq))
        return out

    def logits_ptr(self) -> int:
        return self.lib.janus_model_logits(self.handle)

    def generate(self, prompt: Sequence[int], max_tokens: int, repetition_penalty: float = 1.15) -> list[int]:
        p = np.ascontiguousarray(np.asarray(prompt, dtype=np.uint32))
        out = np.zeros(max(1, max_tokens), dtype=np.uint32)
        n = C.c_uint32()
        self._check(self.lib.janus_model_generate(self.handle, p.ctypes.data, len(p), max_tokens,
                                                  repetition_penalty, out.ctypes.data, C.byref(n)))
        return out[: n.value].tolist()

    def generate_with_callback(self, prompt: Sequence[int], max_tokens: int,
                               callback: Callable[[int], bool] | None = None,
                               repetition_penalty: float = 1.15) -> list[int]:
        """Model::generate_with_callback (generation.rs:340-604) on token ids:
        `callback(token)` runs for each generated token as its step finishes
        and stops generation, with that token kept, by returning False. An
        exception raised by the callback stops generation and is re-raised."""
        p = np.ascontiguousarray(np.asarray(prompt, dtype=np.uint32))
        out = np.zeros(max(1, max_tokens), dtype=np.uint32)
        n = C.c_uint32()
        raised: list[BaseException] = []

        def trampoline(_user, token, _index):
            try:
                return 1 if callback(int(token)) else 0
            except BaseException as exc:   # never unwind through the C frames
                raised.append(exc)
                return 0

        cb = _lib.TOKEN_CALLBACK(trampoline) if callback is not None else _lib.TOKEN_CALLBACK()
        status = self.lib.janus_model_generate_stream(self.handle, p.ctypes.data, len(p), max_tokens,
                                                      repetition_penalty, cb, None, out.ctypes.data, C.byref(n))
        if raised:
            raise raised[0]
        self._check(status)
        return out[: n.value].tolist()

    def generate_batch(self, prompts: Sequence[Sequence[int]], max_tokens: int,
                       repetition_penalty: float = 1.15) -> list[list[int]]:
        """Model::generate_batch with continuous batching (include/janus_model.h)."""
        lens = np.ascontiguousarray(np.asarray([len(p) for p in prompts], dtype=np.uint32))
        flat = np.ascontiguousarray(np.concatenate([np.asarray(p, dtype=np.uint32) for p in prompts])
                                    if len(prompts) else np.zeros(1, np.uint32))
        out = np.zeros((max(1, len(prompts)), max(1, max_tokens)), dtype=np.uint32)
        n = np.zeros(max(1, len(prompts)), dtype=np.uint32)
        self._check(self.lib.janus_model_generate_batch(self.handle, flat.ctypes.data, lens.ctypes.data,
                                                        len(prompts), max_tokens, repetition_penalty,
                                                        out.ctypes.data, n.ctypes.data))
        return [out[i, : n[i]].tolist() for i in range(len(prompts))]

    def set_sampler(self, mode: int, repetition_penalty: float = 1.0) -> None:
        self._check(self.lib.janus_model_set_sampler(self.handle, mode, repetition_penalty))

    def graph_begin(self, tokens: Sequence[int], positions: Sequence[int], slots: Sequence[int] | None = None) -> None:
        t = np.ascontiguousarray(np.asarray(tokens, dtype=np.uint32))
        p = np.ascontiguousarray(np.asarray(positions, dtype=np.uint32))
        if slots is None:
            self._check(self.lib.janus_model_graph_begin(self.handle, t.ctypes.data, p.ctypes.data, len(t)))
        else:
            s = np.ascontiguousarray(np.asarray(slots, dtype=np.uint32))
            self._check(self.lib.janus_model_graph_begin_slots(self.handle, t.ctypes.data, p.ctypes.data,
                                                               s.ctypes.data, len(t)))

    def generated(self, row: int = 0, cap: int = 1 << 16) -> list[int]:
        """Tokens generated by batch row `row` since its graph_begin or admission."""
        out = np.zeros(max(1, cap), dtype=np.uint32)
        n = C.c_uint32()
        self._check(self.lib.janus_model_read_generated(self.handle, row, out.ctypes.data, cap, C.byref(n)))
        return out[: min(n.value, cap)].tolist()

    def graph_run(self, steps: int) -> None:
        self._check(self.lib.janus_model_graph_run(self.handle, steps))

    def graph_tokens(self, nseq: int) -> list[int]:
        out = np.zeros(nseq, dtype=np.uint32)
        self._check(self.lib.janus_model_graph_read_tokens(self.handle, out.ctypes.data, nseq))
        return out.tolist()

    def set_kv_cache(self, k, v) -> None:
        """Use caller-owned cache tensors [layers, max_batch * max_seq_len, kv_heads, head_dim]."""
        self._k_ext, self._v_ext = k, v   # keep them alive
        self._check(self.lib.janus_model_set_kv_cache(self.handle, k.data_ptr(), v.data_ptr(),
                                                      k.numel() * k.element_size()))

    def kv_cache_ptr(self, which: int) -> int:
        return self.lib.janus_model_kv_cache(self.handle, which)


def _gguf_tensor(engine: ComputeEngine, f, t) -> Tensor:
    n, k = t.shape_nk()
    if t.name == "token_embd.weight" and t.ggml_type in (DT_Q4_0, DT_Q8_0, DT_Q4_K, DT_Q5_K, DT_Q6_K):
        return Tensor(t.name, DT_F16, n, k, _embedding_f16(engine, t.ggml_type, n, k, f.tensor_data(t)))
    return Tensor(t.name, t.ggml_type, n, k, f.tensor_data(t))


def _embedding_f16(engine: ComputeEngine, ggml_type: int, n: int, k: int, raw) -> np.ndarray:
    """Quantised embedding blocks -> binary16 [n][k] (GGML element order): the
    GPU weight dequant's exact f32 values, rounded to nearest-even binary16."""
    w = ops.GpuTensor(engine, ggml_type, n, k, raw)
    try:
        h = w.dequant().half().cpu().numpy()
    finally:
        w.free()
    return h.view(np.uint16)
