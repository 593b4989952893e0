"""C-ABI checks that need no GPU: the library loads, exports every function
declared in include/*.h, and rejects bad arguments on the host with the
status codes that stand in for the reference's errors
(crates/janus-engine/src/compute/error.rs:5-35).
"""
import ctypes as C
import re
from pathlib import Path

import numpy as np
import pytest

from janus_amd import _lib, synth

ROOT = Path(__file__).resolve().parent.parent


def _declared_functions():
    names = set()
    for h in (ROOT / "include").glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        for m in re.finditer(r"\b(janus_\w+)\s*\(", text):
            names.add(m.group(1))
    return sorted(names)


def test_exports_every_declared_symbol():
    lib = _lib.load()
    declared = _declared_functions()
    assert len(declared) >= 40
    missing = [n for n in declared if not hasattr(lib, n)]
    assert not missing, missing
    # and the Python binding declares a prototype for each of them
    assert set(declared) <= set(_lib.EXPORTED)


def test_abi_version_and_status_strings():
    lib = _lib.load()
    assert lib.janus_abi_version() == 1
    assert lib.janus_status_string(_lib.E_KV_OVERFLOW) == b"kv cache overflow"


@pytest.fixture()
def vctx():
    lib = _lib.load()
    h = C.c_void_p()
    assert lib.janus_create(-1, C.byref(h)) == _lib.OK
    yield lib, h
    lib.janus_destroy(h)


def _upload(lib, ctx, ggml_type, n, k, data, flags=0):
    buf = np.ascontiguousarray(data).view(np.uint8).reshape(-1)
    w = C.c_void_p()
    return lib.janus_weight_upload(ctx, ggml_type, n, k, buf.ctypes.data, buf.nbytes, flags, C.byref(w))


def test_weight_upload_validation(vctx):
    lib, ctx = vctx
    rng = np.random.default_rng(0)
    # k not a multiple of the block width -> InvalidDimensions (quantized.rs:327-332)
    raw = synth.random_q8_0(rng, 4, 64)
    assert _upload(lib, ctx, _lib.DT_Q8_0, 4, 48, raw) == _lib.E_INVALID_DIM
    assert b"multiple of 32" in lib.janus_last_error(ctx)
    assert _upload(lib, ctx, _lib.DT_Q4_K, 4, 128, np.zeros(4 * 72, np.uint8)) == _lib.E_INVALID_DIM
    # byte size mismatch
    assert _upload(lib, ctx, _lib.DT_Q4_0, 4, 64, np.zeros(10, np.uint8)) == _lib.E_INVALID_DIM
    assert _upload(lib, ctx, _lib.DT_Q5_K, 4, 128, np.zeros(4 * 88, np.uint8)) == _lib.E_INVALID_DIM
    assert _upload(lib, ctx, _lib.DT_Q5_K, 4, 256, np.zeros(4 * 176 - 1, np.uint8)) == _lib.E_INVALID_DIM
    assert _upload(lib, ctx, _lib.DT_Q6_K, 4, 256, np.zeros(4 * 210 + 2, np.uint8)) == _lib.E_INVALID_DIM
    assert b"blocks of 210" in lib.janus_last_error(ctx)
    # unsupported GGML type (Q2_K = 10) -> error instead of panic (quantized.rs:181)
    assert _upload(lib, ctx, 10, 4, 256, np.zeros(4 * 84, np.uint8)) == _lib.E_UNSUPPORTED_DTYPE
    # a valid tensor passes every host check and then needs the device
    assert _upload(lib, ctx, _lib.DT_Q8_0, 4, 64, raw) == _lib.E_NO_DEVICE
    assert _upload(lib, ctx, _lib.DT_Q5_K, 4, 256, np.zeros(4 * 176, np.uint8)) == _lib.E_NO_DEVICE
    assert _upload(lib, ctx, _lib.DT_Q6_K, 4, 256, np.zeros(4 * 210, np.uint8)) == _lib.E_NO_DEVICE


def test_op_validation(vctx):
    lib, ctx = vctx
    dummy = C.c_void_p(0x1000)
    # KV overflow: position >= max_seq_len (compute/cache/core.rs:283-288)
    st = lib.janus_kv_update(ctx, dummy, dummy, dummy, dummy, _lib.DT_F16, 1, 2, 64, 16, 16, None, None)
    assert st == _lib.E_KV_OVERFLOW and b"exceeds max_seq_len" in lib.janus_last_error(ctx)
    assert lib.janus_kv_update(ctx, dummy, dummy, dummy, dummy, 5, 1, 2, 64, 0, 16, None, None) == \
        _lib.E_UNSUPPORTED_DTYPE
    # attention shape checks
    assert lib.janus_attention(ctx, dummy, dummy, dummy, _lib.DT_F16, dummy, 1, 6, 4, 64, 1, 8, None, None, 0,
                               0.0) == _lib.E_INVALID_DIM
    assert lib.janus_attention(ctx, dummy, dummy, dummy, _lib.DT_F16, dummy, 1, 8, 2, 96, 1, 8, None, None, 0,
                               0.0) == _lib.E_INVALID_DIM
    assert lib.janus_attention(ctx, dummy, dummy, dummy, _lib.DT_F16, dummy, 1, 8, 2, 64, 9, 8, None, None, 0,
                               0.0) == _lib.E_KV_OVERFLOW
    # rope needs an even head_dim; argmax a tie rule it knows
    assert lib.janus_rope(ctx, dummy, dummy, dummy, 1, 1, 5, 0, None) == _lib.E_INVALID_DIM
    assert lib.janus_argmax(ctx, dummy, dummy, 10, 1, 7) == _lib.E_INVALID_ARG
    # null buffers
    assert lib.janus_rmsnorm(ctx, None, dummy, _lib.DT_F32, dummy, 1, 4, 1e-5) == _lib.E_INVALID_ARG
    # well-formed calls reach the device check
    assert lib.janus_rmsnorm(ctx, dummy, dummy, _lib.DT_F32, dummy, 1, 4, 1e-5) == _lib.E_NO_DEVICE
    assert lib.janus_sync(ctx) == _lib.E_NO_DEVICE


def test_create_rejects_bad_device():
    lib = _lib.load()
    h = C.c_void_p()
    st = lib.janus_create(1 << 20, C.byref(h))
    assert st in (_lib.E_INVALID_ARG, _lib.E_NO_DEVICE)


def test_model_config_validation(vctx):
    lib, ctx = vctx
    cfg = _lib.ModelConfig(256, 4, 3, 64, 688, 512, 2, 64, 1, 1e-5, 1e4, _lib.DT_F32, _lib.DT_F32)
    m = C.c_void_p()
    assert lib.janus_model_create(ctx, C.byref(cfg), C.byref(m)) == _lib.E_INVALID_DIM   # 4 % 3 != 0
    cfg.kv_heads = 2
    cfg.max_batch = 65
    assert lib.janus_model_create(ctx, C.byref(cfg), C.byref(m)) == _lib.E_INVALID_DIM
    cfg.max_batch = 1
    assert lib.janus_model_create(ctx, C.byref(cfg), C.byref(m)) == _lib.E_NO_DEVICE
