"""ctypes binding of libjanus_hip.so (declarations: include/janus_hip.h,
include/janus_model.h).

The library is loaded from this package directory (JANUS_LIB names another
build of it, such as the host-sanitised one of `python -m janus_amd.build
--sanitize`). There is no fallback: if the shared object is missing the
import fails loudly with the build command.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

LIB_PATH = Path(os.environ.get("JANUS_LIB") or Path(__file__).resolve().parent / "libjanus_hip.so")

# status codes (janus_status)
OK = 0
E_INVALID_ARG = 1
E_INVALID_DIM = 2
E_UNSUPPORTED_DTYPE = 3
E_KV_OVERFLOW = 4
E_TOKEN_RANGE = 5
E_HIP = 6
E_OOM = 7
E_NO_DEVICE = 8
E_NAN_LOGITS = 9

# GGML type ids (janus_dtype)
DT_F32 = 0
DT_F16 = 1
DT_Q4_0 = 2
DT_Q8_0 = 8
DT_Q4_K = 12
DT_Q5_K = 13
DT_Q6_K = 14

WEIGHT_FTZ_F16 = 0x1
WEIGHT_Q6K_REF_ORDER = 0x2
TIE_LAST = 0
TIE_WGSL = 1
SAMPLER_ARGMAX = 0
SAMPLER_PENALTY = 1
SAMPLER_WGSL = 2
ATTN_SCRATCH_BYTES = 16 << 20

P = C.c_void_p
U32 = C.c_uint32
I32 = C.c_int
F32 = C.c_float
SZ = C.c_size_t


class ModelConfig(C.Structure):
    """janus_model_config (include/janus_model.h)."""

    _fields_ = [
        ("hidden", U32), ("heads", U32), ("kv_heads", U32), ("head_dim", U32),
        ("ffn", U32), ("vocab", U32), ("layers", U32), ("max_seq_len", U32),
        ("max_batch", U32), ("rms_eps", F32), ("rope_theta", F32),
        ("kv_dtype", I32), ("act_dtype", I32),
    ]


# janus_token_callback (include/janus_model.h); TOKEN_CALLBACK() is NULL
TOKEN_CALLBACK = C.CFUNCTYPE(I32, P, U32, U32)

# name -> (restype, argtypes)
_SIGNATURES = {
    # context / buffers
    "janus_create": (I32, [I32, C.POINTER(P)]),
    "janus_destroy": (None, [P]),
    "janus_last_error": (C.c_char_p, [P]),
    "janus_status_string": (C.c_char_p, [I32]),
    "janus_abi_version": (I32, []),
    "janus_set_stream": (I32, [P, P]),
    "janus_get_stream": (P, [P]),
    "janus_sync": (I32, [P]),
    "janus_workspace_bytes": (I32, [P, C.POINTER(SZ), C.POINTER(SZ)]),
    "janus_device_count": (I32, [C.POINTER(I32)]),
    "janus_alloc": (I32, [P, SZ, C.POINTER(P)]),
    "janus_free": (I32, [P, P]),
    "janus_h2d": (I32, [P, P, P, SZ]),
    "janus_d2h": (I32, [P, P, P, SZ]),
    # weights
    "janus_weight_upload": (I32, [P, I32, U32, U32, P, SZ, U32, C.POINTER(P)]),
    "janus_weight_free": (I32, [P, P]),
    "janus_weight_info": (I32, [P, C.POINTER(I32), C.POINTER(U32), C.POINTER(U32), C.POINTER(SZ)]),
    "janus_weight_dequant": (I32, [P, P, P]),
    # operators
    "janus_gemm_auto": (I32, [P, P, I32, P, P, I32, U32, U32, U32, U32]),
    "janus_gemm_residual": (I32, [P, P, I32, P, P, P, U32, U32, U32]),
    "janus_rmsnorm": (I32, [P, P, P, I32, P, U32, U32, F32]),
    "janus_silu": (I32, [P, P, P, U32]),
    "janus_elementwise_mul": (I32, [P, P, P, P, U32]),
    "janus_add_tensors": (I32, [P, P, P, P, U32]),
    "janus_swiglu": (I32, [P, P, P, P, I32, U32]),
    "janus_rope_table": (I32, [P, P, U32, U32, F32]),
    "janus_rope": (I32, [P, P, P, P, U32, U32, U32, U32, P]),
    "janus_kv_update": (I32, [P, P, P, P, P, I32, U32, U32, U32, U32, U32, P, P]),
    "janus_attention": (I32, [P, P, P, P, I32, P, U32, U32, U32, U32, U32, U32, P, P, U32, F32]),
    "janus_attention_noalloc": (I32, [P, P, P, P, I32, P, U32, U32, U32, U32, U32, U32, P, P, U32, F32]),
    "janus_embed": (I32, [P, P, P, U32, P]),
    "janus_embed_device": (I32, [P, P, P, U32, P]),
    "janus_argmax": (I32, [P, P, P, U32, U32, I32]),
    "janus_repetition_penalty": (I32, [P, P, U32, P, U32, F32]),
    # decode driver
    "janus_model_create": (I32, [P, C.POINTER(ModelConfig), C.POINTER(P)]),
    "janus_model_destroy": (None, [P]),
    "janus_model_set_tensor": (I32, [P, C.c_char_p, I32, U32, U32, P, SZ]),
    "janus_model_validate": (I32, [P]),
    "janus_model_reset": (I32, [P]),
    "janus_model_set_kv_cache": (I32, [P, P, P, SZ]),
    "janus_model_forward": (I32, [P, P, P, U32]),
    "janus_model_forward_slots": (I32, [P, P, P, P, U32]),
    "janus_model_logits": (P, [P]),
    "janus_model_kv_cache": (P, [P, I32]),
    "janus_model_read_logits": (I32, [P, P, U32]),
    "janus_model_generate": (I32, [P, P, U32, U32, F32, P, P]),
    "janus_model_generate_stream": (I32, [P, P, U32, U32, F32, TOKEN_CALLBACK, P, P, P]),
    "janus_model_generate_batch": (I32, [P, P, P, U32, U32, F32, P, P]),
    "janus_model_set_sampler": (I32, [P, I32, F32]),
    "janus_model_graph_begin": (I32, [P, P, P, U32]),
    "janus_model_graph_begin_slots": (I32, [P, P, P, P, U32]),
    "janus_model_graph_run": (I32, [P, U32]),
    "janus_model_graph_read_tokens": (I32, [P, P, U32]),
    "janus_model_read_generated": (I32, [P, U32, P, U32, P]),
}

EXPORTED = tuple(_SIGNATURES)

_lib: C.CDLL | None = None


def load() -> C.CDLL:
    """Load libjanus_hip.so and declare every entry point; raises if absent."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(
            f"{LIB_PATH} is not built; run `python -m janus_amd.build` "
            "(there is no CPU fallback for the HIP path)")
    lib = C.CDLL(str(LIB_PATH))
    for name, (res, args) in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


class JanusError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"janus status {status}: {message}")
        self.status = status


def check(status: int, ctx=None) -> None:
    if status != OK:
        lib = load()
        msg = lib.janus_last_error(ctx).decode() if ctx else lib.janus_status_string(status).decode()
        raise JanusError(status, msg or lib.janus_status_string(status).decode())
