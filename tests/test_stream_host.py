"""Host side of streaming generation (Model.generate_with_callback over
janus_model_generate_stream), without a GPU: the library entry point is
replaced by a stand-in that follows the C contract of include/janus_model.h
(each token goes to the callback in order with its index; a callback
returning 0 ends generation with that token kept; a NULL callback streams
nothing). What is checked is the wrapper: the trampoline's return values, an
exception raised by a Python callback stopping generation and reaching the
caller, and the output slice. The GPU behaviour is tests/test_gpu_stream.py.
"""
import ctypes as C

import pytest

from janus_amd import _lib
from janus_amd.model import Model


class _FakeLib:
    """janus_model_generate_stream over a fixed token list."""

    def __init__(self, tokens):
        self.tokens = tokens
        self.calls = []

    def janus_model_generate_stream(self, handle, prompt_ptr, n_prompt, max_tokens, penalty, cb, user, out_ptr, n_out):
        assert isinstance(cb, _lib.TOKEN_CALLBACK)
        self.calls.append((n_prompt, max_tokens, round(penalty, 4), bool(cb)))
        out = (C.c_uint32 * max(1, max_tokens)).from_address(out_ptr)
        n = 0
        for t in self.tokens[:max_tokens]:
            out[n] = t
            n += 1
            if cb and not cb(user, t, n - 1):
                break
        n_out._obj.value = n
        return _lib.OK


def _model(tokens):
    m = Model.__new__(Model)
    m.lib = _FakeLib(tokens)
    m.handle = C.c_void_p(1)

    class _Engine:
        ctx = None

    m.engine = _Engine()
    return m


def test_tokens_stream_in_order_and_false_stops_with_the_token_kept():
    m = _model([7, 3, 9, 9, 2])
    seen = []
    assert m.generate_with_callback([1, 2], 5, lambda t: seen.append(t) or True) == [7, 3, 9, 9, 2]
    assert seen == [7, 3, 9, 9, 2]
    seen.clear()
    assert m.generate_with_callback([1, 2], 5, lambda t: seen.append(t) or len(seen) < 3) == [7, 3, 9]
    assert seen == [7, 3, 9]
    assert m.lib.calls[0] == (2, 5, 1.15, True)


def test_no_callback_passes_null_and_max_tokens_bounds_the_output():
    m = _model([4, 5, 6])
    assert m.generate_with_callback([1], 2, None, repetition_penalty=1.0) == [4, 5]
    assert m.lib.calls == [(1, 2, 1.0, False)]


def test_callback_exception_stops_generation_and_is_reraised():
    m = _model([4, 5, 6, 7])
    seen = []

    def cb(t):
        seen.append(t)
        if len(seen) == 2:
            raise ValueError("stop here")
        return True

    with pytest.raises(ValueError, match="stop here"):
        m.generate_with_callback([1], 4, cb)
    assert seen == [4, 5]   # no token after the one that raised


def test_token_callback_prototype():
    assert _lib.TOKEN_CALLBACK._restype_ is C.c_int32 or _lib.TOKEN_CALLBACK._restype_ is C.c_int
    assert list(_lib.TOKEN_CALLBACK._argtypes_) == [C.c_void_p, C.c_uint32, C.c_uint32]
    sig = dict(zip(("res", "args"), _lib._SIGNATURES["janus_model_generate_stream"]))
    assert sig["args"][5] is _lib.TOKEN_CALLBACK
    assert len(sig["args"]) == 9
