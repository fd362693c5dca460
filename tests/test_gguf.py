"""GGUF reader and writer (include/inferi_hip.h ifr_gguf_*), CPU only.

The reader is pinned by the reference's own parser fixture, dummy.gguf
(tests/golden/, from the reference's assets; its test gguf.rs:776-785 only
parses it, so the expected values here are the ones llama.cpp's llama-gguf
writes: one metadata value of each type and tensors filled with 100 + i).
The writer is pinned by re-serializing that file's content byte for byte.
"""

import os

import numpy as np
import pytest

import inferi_amd as I

HERE = os.path.dirname(os.path.abspath(__file__))
DUMMY = os.path.join(HERE, "golden", "dummy.gguf")

# GGUF stores dims in its own order (ne0 first); the reference reverses them.
DUMMY_NE = [[7, 8, 6, 4], [7, 3, 10, 2], [8, 1, 10], [7, 1, 7, 3], [2], [8], [3], [4, 8, 6], [3, 3], [10, 8, 4]]
DUMMY_META = [
    ("some.parameter.uint8", I.GGUF_U8, 0x12), ("some.parameter.int8", I.GGUF_I8, -0x13),
    ("some.parameter.uint16", I.GGUF_U16, 0x1234), ("some.parameter.int16", I.GGUF_I16, -0x1235),
    ("some.parameter.uint32", I.GGUF_U32, 0x12345678), ("some.parameter.int32", I.GGUF_I32, -0x12345679),
    ("some.parameter.float32", I.GGUF_F32, float(np.float32(0.123456789))),
    ("some.parameter.uint64", I.GGUF_U64, 0x123456789ABCDEF0),
    ("some.parameter.int64", I.GGUF_I64, -0x123456789ABCDEF1),
    ("some.parameter.float64", I.GGUF_F64, 0.1234567890123456789), ("some.parameter.bool", I.GGUF_BOOL, True),
    ("some.parameter.string", I.GGUF_STRING, "hello world"),
]


def test_dummy_gguf_known_answers():
    g = I.Gguf(DUMMY)
    assert g.version == 3 and g.alignment == 32
    keys = g.keys()
    assert keys == [k for k, _, _ in DUMMY_META] + ["some.parameter.arr.i16", "some.parameter.arr.f32",
                                                    "some.parameter.arr.str"]
    for k, t, v in DUMMY_META:
        assert g.type_of(k)[0] == t
        assert g.get(k) == v, k
    assert g.type_of("some.parameter.arr.i16") == (I.GGUF_ARRAY, I.GGUF_I16, 4)
    assert g.get("some.parameter.arr.i16").tolist() == [1, 2, 3, 4]
    assert np.array_equal(g.get("some.parameter.arr.f32"), np.array([3.145, 2.718, 1.414], np.float32))
    assert g.get("some.parameter.arr.str") == ["hello", "world", "!"]
    names = g.tensor_names()
    assert names == [f"tensor_{i}" for i in range(10)]
    for i, ne in enumerate(DUMMY_NE):
        t = g.tensor(f"tensor_{i}")
        assert t.dtype == 0 and t.rank == len(ne)
        assert t.dims == tuple(list(reversed(ne)) + [1] * (4 - len(ne)))  # gguf.rs:620-626
        vals = t.data.view(np.float32)
        assert vals.size == int(np.prod(ne)) and np.all(vals == 100 + i)
    with pytest.raises(KeyError):
        g.get("missing.key")
    with pytest.raises(I.HipError):
        g.tensor("tensor_10")
    g.close()


def write_dummy(path):
    w = I.GgufWriter()
    for k, t, v in DUMMY_META:
        w.set(k, t, v)
    w.set_array("some.parameter.arr.i16", I.GGUF_I16, [1, 2, 3, 4])
    w.set_array("some.parameter.arr.f32", I.GGUF_F32, [3.145, 2.718, 1.414])
    w.set_array("some.parameter.arr.str", I.GGUF_STRING, ["hello", "world", "!"])
    for i, ne in enumerate(DUMMY_NE):
        w.add_tensor(f"tensor_{i}", 0, list(reversed(ne)), np.full(int(np.prod(ne)), 100 + i, np.float32))
    w.save(path)
    w.close()


def test_writer_reproduces_dummy_gguf_byte_for_byte(tmp_path):
    p = tmp_path / "again.gguf"
    write_dummy(str(p))
    assert p.read_bytes() == open(DUMMY, "rb").read()


def test_from_bytes_matches_open():
    data = open(DUMMY, "rb").read()
    a, b = I.Gguf(DUMMY), I.Gguf(data=data)
    assert a.metadata.keys() == b.metadata.keys()
    for n in a.tensor_names():
        assert np.array_equal(a.tensor(n).data, b.tensor(n).data)


def test_round_trip_all_types_and_alignment(tmp_path):
    rng = np.random.default_rng(3)
    w = I.GgufWriter()
    w.set("general.alignment", I.GGUF_U32, 64)
    w.set("empty", I.GGUF_STRING, "")
    w.set("unicode", I.GGUF_STRING, "héllo 世界")
    w.set("neg", I.GGUF_I64, -(2 ** 63))
    w.set("big", I.GGUF_U64, 2 ** 64 - 1)
    w.set("f", I.GGUF_F64, -1e300)
    w.set("b", I.GGUF_BOOL, False)
    w.set("b", I.GGUF_BOOL, True)  # replaced in place
    w.set_array("empty_arr", I.GGUF_U32, [])
    w.set_array("bools", I.GGUF_BOOL, [True, False, True])
    w.set_array("u64s", I.GGUF_U64, [0, 2 ** 64 - 1])
    tensors = {
        "q4k": (12, [3, 512], rng.integers(0, 256, 3 * 2 * 144, dtype=np.uint8)),
        "q6k": (14, [2, 256], rng.integers(0, 256, 2 * 210, dtype=np.uint8)),
        "q8_0": (8, [5, 64], rng.integers(0, 256, 5 * 2 * 34, dtype=np.uint8)),
        "f16": (1, [7], rng.integers(0, 256, 14, dtype=np.uint8)),
        "f32": (0, [2, 3, 4, 5], rng.standard_normal(120).astype(np.float32).view(np.uint8)),
    }
    for n, (dt, dims, data) in tensors.items():
        w.add_tensor(n, dt, dims, data)
    p = str(tmp_path / "rt.gguf")
    w.save(p)
    w.close()
    g = I.Gguf(p)
    assert g.alignment == 64
    assert g.keys()[:2] == ["general.alignment", "empty"] and g.keys().count("b") == 1
    assert g.get("empty") == "" and g.get("unicode") == "héllo 世界"
    assert g.get("neg") == -(2 ** 63) and g.get("big") == 2 ** 64 - 1 and g.get("f") == -1e300
    assert g.get("b") is True
    assert g.get("empty_arr").size == 0 and g.get("bools").tolist() == [True, False, True]
    assert g.get("u64s").tolist() == [0, 2 ** 64 - 1]
    raw = open(p, "rb").read()
    for n, (dt, dims, data) in tensors.items():
        t = g.tensor(n)
        assert t.dtype == dt and t.rank == len(dims) and t.dims[: len(dims)] == tuple(dims)
        assert np.array_equal(t.data, data.view(np.uint8))
        off = raw.find(data.view(np.uint8).tobytes())
        assert off % 64 == 0  # every tensor's data on the alignment
    assert len(raw) % 64 == 0


def test_writer_rejects_bad_tensors():
    w = I.GgufWriter()
    with pytest.raises(I.HipError):
        w.add_tensor("x", 12, [2, 100], np.zeros(10, np.uint8))  # 100 not a multiple of 256
    with pytest.raises(I.HipError):
        w.add_tensor("x", 0, [2, 2], np.zeros(15, np.uint8))  # wrong byte count
    with pytest.raises(I.HipError):
        w.add_tensor("x", 0, [1, 1, 1, 1, 1], np.zeros(4, np.uint8))  # rank 5
    w.add_tensor("x", 0, [1], np.zeros(4, np.uint8))
    with pytest.raises(I.HipError):
        w.add_tensor("x", 0, [1], np.zeros(4, np.uint8))  # twice
    w.close()


def test_truncated_and_malformed_files_fail_cleanly():
    data = open(DUMMY, "rb").read()
    for n in list(range(0, 1300)) + list(range(1300, len(data), 97)) + [len(data) - 1]:
        with pytest.raises(I.HipError):
            I.Gguf(data=data[:n])
    with pytest.raises(I.HipError, match="magic"):
        I.Gguf(data=b"GGUX" + data[4:])
    assert I.Gguf(data=b"FUGG" + data[4:]).version == 3  # the other byte order is accepted (gguf.rs:19-20)

    def one_tensor(rank=1, ttype=0, meta_type=None, dims=None):
        dims = dims or [1] * rank
        b = bytearray(b"GGUF") + (3).to_bytes(4, "little") + (1).to_bytes(8, "little")
        b += (1 if meta_type is not None else 0).to_bytes(8, "little")
        if meta_type is not None:
            b += (1).to_bytes(8, "little") + b"k" + meta_type.to_bytes(4, "little") + (0).to_bytes(8, "little")
        b += (1).to_bytes(8, "little") + b"t" + rank.to_bytes(4, "little")
        b += b"".join(int(d).to_bytes(8, "little") for d in dims)
        b += ttype.to_bytes(4, "little") + (0).to_bytes(8, "little")
        b += bytes((-len(b)) % 32) + bytes(32)
        return bytes(b)

    assert I.Gguf(data=one_tensor()).tensor("t").dims == (1, 1, 1, 1)
    with pytest.raises(I.HipError, match="rank"):
        I.Gguf(data=one_tensor(rank=5))
    with pytest.raises(I.HipError, match="type 4"):
        I.Gguf(data=one_tensor(ttype=4))  # Q4_2 was removed from the format
    with pytest.raises(I.HipError, match="value type 13"):
        I.Gguf(data=one_tensor(meta_type=13))
    g = I.Gguf(data=one_tensor(ttype=10))  # Q2_K: listed, data not read (as the reference)
    assert g.tensor("t").data is None
    # dims whose product wraps 64 bits (four dims of 2^32: 2^128) or exceeds
    # 2^62, and element counts that are not whole blocks, are rejected before
    # any byte count is formed from them
    with pytest.raises(I.HipError, match="too large"):
        I.Gguf(data=one_tensor(rank=4, dims=[1 << 32] * 4))
    with pytest.raises(I.HipError, match="too large"):
        I.Gguf(data=one_tensor(rank=2, dims=[1 << 31, 1 << 31]))
    with pytest.raises(I.HipError, match="not a multiple"):
        I.Gguf(data=one_tensor(rank=1, ttype=12, dims=[300]))  # Q4_K blocks are 256 elements
    with pytest.raises(I.HipError, match="past the end"):
        I.Gguf(data=one_tensor(rank=2, ttype=0, dims=[1 << 20, 1 << 20]))  # 4 TiB of F32 in a small file


def llama_file(path, meta, tokens=8, drop=()):
    w = I.GgufWriter()
    w.set("general.architecture", I.GGUF_STRING, meta.pop("arch", "llama"))
    for k, (t, v) in meta.items():
        if k not in drop:
            w.set(k, t, v)
    if tokens is not None:
        w.set_array("tokenizer.ggml.tokens", I.GGUF_STRING, [f"t{i}" for i in range(tokens)])
    w.save(path)
    w.close()


BASE = {"llama.embedding_length": (I.GGUF_U32, 256), "llama.feed_forward_length": (I.GGUF_U32, 512),
        "llama.block_count": (I.GGUF_U32, 2), "llama.attention.head_count": (I.GGUF_U32, 4),
        "llama.attention.head_count_kv": (I.GGUF_U32, 2), "llama.context_length": (I.GGUF_U32, 48),
        "llama.rope.freq_base": (I.GGUF_F32, 500000.0),
        "llama.attention.layer_norm_rms_epsilon": (I.GGUF_F32, 1e-5)}


def test_config_from_gguf(tmp_path):
    p = str(tmp_path / "m.gguf")
    llama_file(p, dict(BASE), tokens=1000)
    c = I.Llama2Config.from_gguf(I.Gguf(p))
    assert (c.n_layers, c.hidden, c.ffn, c.n_heads, c.n_kv_heads, c.vocab, c.max_pos) == (2, 256, 512, 4, 2, 1000, 48)
    assert c.rope_theta == 500000.0 and c.rms_eps == np.float32(1e-5) and c.kv_dtype == I.F32
    # optional keys default as in cpu.rs:97-106
    llama_file(p, dict(BASE), drop=("llama.rope.freq_base", "llama.attention.layer_norm_rms_epsilon"))
    c = I.Llama2Config.from_gguf(I.Gguf(p))
    assert c.rope_theta == 10000.0 and c.rms_eps == np.float32(1e-6)
    # strict types, as unwrap_u32 / as_f32
    bad = dict(BASE)
    bad["llama.block_count"] = (I.GGUF_U64, 2)
    llama_file(p, bad)
    with pytest.raises(I.HipError, match="block_count"):
        I.Llama2Config.from_gguf(I.Gguf(p))
    bad = dict(BASE)
    bad["llama.rope.freq_base"] = (I.GGUF_F64, 1e4)
    llama_file(p, bad)
    with pytest.raises(I.HipError, match="freq_base"):
        I.Llama2Config.from_gguf(I.Gguf(p))
    llama_file(p, dict(BASE), tokens=None)
    with pytest.raises(I.HipError, match="tokens"):
        I.Llama2Config.from_gguf(I.Gguf(p))
    # qwen2: the keys carry its prefix and the RoPE pairing is NeoX (models/llama2/mod.rs:18-30)
    q = {k.replace("llama.", "qwen2."): v for k, v in BASE.items()}
    q["arch"] = "Qwen2"
    llama_file(p, q, tokens=100)
    c = I.Llama2Config.from_gguf(I.Gguf(p))
    assert c.rope_variant == I.ROPE_NEOX and c.n_layers == 2 and c.vocab == 100 and c.rope_theta == 500000.0
    llama_file(p, dict(BASE, arch="qwen2"))  # llama.* keys under a qwen2 architecture are not read
    with pytest.raises(I.HipError, match="qwen2.embedding_length"):
        I.Llama2Config.from_gguf(I.Gguf(p))
