"""GGUF reader, writer and config extraction (no GPU).

Mirrors the reference's parser tests (formats/gguf/parser.rs:483-529: magic
and version of an empty file) and covers what they leave open with
hand-built byte strings: every metadata value type, arrays, alignment and the
tensor data offsets, the error cases, and the config rules of
model/config.rs:377-446.
"""
import struct

import numpy as np
import pytest

from janus_amd import gguf as G
from janus_amd import synth


def _kv(key, vtype, payload):
    k = key.encode()
    return struct.pack("<Q", len(k)) + k + struct.pack("<I", vtype) + payload


def _header(version=3, n_tensors=0, kvs=b"", n_kv=0):
    return b"GGUF" + struct.pack("<IQQ", version, n_tensors, n_kv) + kvs


def test_empty_file_header():
    # parser.rs test_parse_magic_and_version: magic, version 2, zero counts
    md = G.parse_header(_header(version=2))
    assert md.version == 2 and md.tensors == [] and md.metadata == {}
    assert md.alignment == 32 and md.data_offset == 32   # 24 header bytes rounded up


@pytest.mark.parametrize("bad", [b"GGUG", b"FUGG", b"\0\0\0\0"])
def test_bad_magic(bad):
    with pytest.raises(G.InvalidMagic):
        G.parse_header(bad + _header()[4:])


@pytest.mark.parametrize("version", [0, 1, 4, 0xFFFFFFFF])
def test_unsupported_versions(version):
    with pytest.raises(G.UnsupportedVersion):
        G.parse_header(_header(version=version))


def test_truncated_header_and_string():
    full = _header(kvs=_kv("a.b", G.STRING, struct.pack("<Q", 5) + b"hello"), n_kv=1)
    G.parse_header(full)
    for cut in (3, 7, 15, 23, len(full) - 1):
        with pytest.raises(G.IncompleteData):
            G.parse_header(full[:cut])


def test_every_scalar_type_and_arrays_parse():
    cases = [(G.UINT8, "<B", 200), (G.INT8, "<b", -5), (G.UINT16, "<H", 60000), (G.INT16, "<h", -300),
             (G.UINT32, "<I", 4000000000), (G.INT32, "<i", -7), (G.FLOAT32, "<f", 1.5), (G.UINT64, "<Q", 2**40),
             (G.INT64, "<q", -2**40), (G.FLOAT64, "<d", 0.1)]
    kvs = b"".join(_kv(f"k{i}", t, struct.pack(f, v)) for i, (t, f, v) in enumerate(cases))
    kvs += _kv("flag", G.BOOL, b"\x02")                                   # any non-zero byte is true
    kvs += _kv("name", G.STRING, struct.pack("<Q", 3) + b"abc")
    kvs += _kv("arr", G.ARRAY, struct.pack("<IQ", G.INT32, 3) + struct.pack("<3i", 1, -2, 3))
    kvs += _kv("toks", G.ARRAY, struct.pack("<IQ", G.STRING, 2) + struct.pack("<Q", 1) + b"x"
               + struct.pack("<Q", 2) + b"yz")
    md = G.parse_header(_header(kvs=kvs, n_kv=len(cases) + 4)).metadata
    for i, (t, _, v) in enumerate(cases):
        assert md[f"k{i}"].type == t and md[f"k{i}"].value == pytest.approx(v)
    assert md["flag"] == G.Value(G.BOOL, True)
    assert md["name"] == G.Value(G.STRING, b"abc")
    assert [x.value for x in md["arr"].value] == [1, -2, 3]
    assert [x.value for x in md["toks"].value] == [b"x", b"yz"]


def test_nested_array_and_bad_types_are_rejected():
    nested = _kv("n", G.ARRAY, struct.pack("<IQ", G.ARRAY, 1) + struct.pack("<IQ", G.UINT8, 0))
    with pytest.raises(G.ParseError):
        G.parse_header(_header(kvs=nested, n_kv=1))
    # an empty array of arrays has no element to reject (parse_array_element runs per element)
    G.parse_header(_header(kvs=_kv("n", G.ARRAY, struct.pack("<IQ", G.ARRAY, 0)), n_kv=1))
    with pytest.raises(G.ParseError):
        G.parse_header(_header(kvs=_kv("v", 13, b""), n_kv=1))
    info = struct.pack("<Q", 1) + b"t" + struct.pack("<IQIQ", 1, 32, 4, 0)   # GGML type 4 does not exist
    with pytest.raises(G.InvalidTensorType):
        G.parse_header(_header(n_tensors=1) + info)


@pytest.mark.parametrize("alignment", [32, 64, 256])
def test_writer_reader_round_trip(tmp_path, alignment):
    rng = np.random.default_rng(3)
    q40 = synth.random_q4_0(rng, 8, 64)
    f32 = rng.standard_normal(24).astype(np.float32)
    f16 = synth.f16_bits(rng.standard_normal((5, 16)).astype(np.float32))
    md = {"general.architecture": G.Value(G.STRING, "llama"), "llama.block_count": G.Value(G.UINT32, 2),
          "pi": G.Value(G.FLOAT32, 3.25), "ids": G.Value(G.ARRAY, [G.Value(G.UINT16, 7), G.Value(G.UINT16, 9)])}
    path = tmp_path / "t.gguf"
    G.write(path, md, [("a", [64, 8], 2, q40), ("b", [24], 0, f32), ("c", [16, 5], 1, f16)], alignment=alignment)
    f = G.GgufFile(path)
    try:
        assert f.meta.data_offset % alignment == 0 and f.meta.alignment == alignment
        assert f.get("llama.block_count") == 2 and f.get("pi") == 3.25
        assert f.get("general.architecture") == b"llama"
        names = [t.name for t in f.tensors]
        assert names == ["a", "b", "c"]
        a, b, c = f.tensors
        assert all(t.offset % alignment == 0 for t in f.tensors)
        assert a.shape_nk() == (8, 64) and b.shape_nk() == (24, 0) and c.shape_nk() == (5, 16)
        assert a.size_bytes() == 8 * 2 * 18 and b.size_bytes() == 96 and c.size_bytes() == 160
        assert np.array_equal(f.tensor_data(a), q40.reshape(-1).view(np.uint8))
        assert np.array_equal(f.tensor_data(b).view(np.float32), f32)
        assert np.array_equal(f.tensor_data(c).view(np.uint16), f16.reshape(-1))
    finally:
        f.close()


def test_block_sizes_of_the_path_formats():
    def size(t, dims):
        return G.TensorInfo("x", dims, t, 0).size_bytes()
    assert size(0, [4096]) == 16384
    assert size(1, [4096, 2]) == 16384
    assert size(2, [4096, 4096]) == 4096 * 128 * 18        # Q4_0: 32 per 18 B
    assert size(8, [4096, 4096]) == 4096 * 128 * 34        # Q8_0: 32 per 34 B (GGML, not the shader's 36)
    assert size(12, [11008, 4096]) == 4096 * 43 * 144      # Q4_K: 256 per 144 B


def test_tensor_data_past_the_end_is_an_error(tmp_path):
    path = tmp_path / "short.gguf"
    G.write(path, {}, [("w", [32, 2], 2, np.zeros(36, np.uint8))])
    data = path.read_bytes()
    path.write_bytes(data[:-10])
    f = G.GgufFile(path)
    try:
        with pytest.raises(G.IncompleteData):
            f.tensor_data(f.tensors[0])
    finally:
        f.close()


def _llama_md(**over):
    md = {"general.architecture": G.Value(G.STRING, "llama"),
          "llama.embedding_length": G.Value(G.UINT32, 4096), "llama.block_count": G.Value(G.UINT32, 32),
          "llama.attention.head_count": G.Value(G.UINT32, 32),
          "llama.attention.head_count_kv": G.Value(G.UINT32, 8),
          "llama.feed_forward_length": G.Value(G.UINT32, 14336),
          "llama.context_length": G.Value(G.UINT32, 8192),
          "llama.attention.layer_norm_rms_epsilon": G.Value(G.FLOAT32, 1e-5),
          "llama.rope.freq_base": G.Value(G.FLOAT32, 500000.0),
          "llama.vocab_size": G.Value(G.UINT32, 128256)}
    for k, v in over.items():
        key = k.replace("__", ".")
        if v is None:
            md.pop(key)
        else:
            md[key] = v
    return md


def test_config_llama3_shape():
    c = G.config_from_metadata(_llama_md())
    assert (c.hidden, c.layers, c.heads, c.kv_heads, c.head_dim, c.ffn, c.vocab) == (4096, 32, 32, 8, 128, 14336,
                                                                                    128256)
    assert c.max_seq_len == 4096                       # 8192 clamped to the engine limit
    assert c.rms_eps == np.float32(1e-5) and c.rope_theta == 500000.0


def test_config_fallbacks():
    md = _llama_md(**{"llama__attention__head_count_kv": None, "llama__rope__freq_base": None,
                      "llama__vocab_size": None})
    c = G.config_from_metadata(md)
    assert c.kv_heads == 32 and c.rope_theta == 500000.0 and c.vocab == 0
    md["rope.freq_base"] = G.Value(G.FLOAT64, 10000.0)
    md["tokenizer.ggml.tokens"] = G.Value(G.ARRAY, [G.Value(G.STRING, b"a")] * 5)
    c = G.config_from_metadata(md)
    assert c.rope_theta == 10000.0 and c.vocab == 5
    assert G.config_from_metadata(md, tokenizer_vocab_size=9).vocab == 5
    md.pop("tokenizer.ggml.tokens")
    assert G.config_from_metadata(md, tokenizer_vocab_size=9).vocab == 9
    # other architectures use their own prefix
    other = {k.replace("llama.", "mistral."): v for k, v in _llama_md().items()}
    other["general.architecture"] = G.Value(G.STRING, "mistral")
    assert G.config_from_metadata(other).ffn == 14336


def test_config_integer_and_float_types():
    md = _llama_md(llama__block_count=G.Value(G.INT16, 32), llama__feed_forward_length=G.Value(G.UINT64, 14336),
                   llama__attention__layer_norm_rms_epsilon=G.Value(G.FLOAT64, 1e-6),
                   llama__rope__freq_base=G.Value(G.UINT32, 10000))
    c = G.config_from_metadata(md)
    assert c.layers == 32 and c.ffn == 14336 and c.rms_eps == np.float32(1e-6) and c.rope_theta == 10000.0
    with pytest.raises(G.ConfigError):
        G.config_from_metadata(_llama_md(llama__block_count=G.Value(G.INT32, -1)))
    with pytest.raises(G.ConfigError):
        G.config_from_metadata(_llama_md(llama__block_count=G.Value(G.UINT64, 2**32)))
    with pytest.raises(G.ConfigError):
        G.config_from_metadata(_llama_md(llama__block_count=G.Value(G.FLOAT32, 32.0)))
    with pytest.raises(G.ConfigError):
        G.config_from_metadata(_llama_md(llama__rope__freq_base=G.Value(G.STRING, b"1e4")))
    with pytest.raises(G.MissingGgufMetadata):
        G.config_from_metadata(_llama_md(llama__feed_forward_length=None))
