"""GGUF v3 reader (yule_hip_gguf_*, a host-only parser in libyule_hip.so) and
the Python writer.  The first block restates the reference parser's own tests
(yule-core/src/gguf.rs:625-790) byte for byte; the rest covers what they
leave open: tensor bounds and overlaps (gguf.rs:380-421), the alignment key,
typed metadata lookups with as_u32 / as_f64 semantics (gguf.rs:50-80), and a
writer -> reader round trip of a whole synthetic model."""
import struct

import numpy as np
import pytest

from yule_amd.backend import YuleGpuError
from yule_amd.formats import DType, matrix_bytes
from yule_amd.gguf import (GGUF_MAGIC, MAX_KV_COUNT, MAX_STRING_LEN, MAX_TENSOR_COUNT, GgufFile, TensorEntry, Value,
                           ValueType, encode_kv, write_gguf)
from yule_amd.model import TINY_TEST, SyntheticModel

ERR_INVALID, ERR_PARSE, ERR_IO = 1, 6, 7


def minimal() -> bytearray:
    return bytearray(struct.pack("<IIQQ", GGUF_MAGIC, 3, 0, 0))


def parse(tmp_path, data: bytes, name="f.gguf") -> GgufFile:
    p = tmp_path / name
    p.write_bytes(bytes(data))
    return GgufFile(p)


def parse_err(tmp_path, data: bytes) -> YuleGpuError:
    with pytest.raises(YuleGpuError) as e:
        parse(tmp_path, data)
    return e.value


def tensor_info(name: str, dims, dtype: int, offset: int) -> bytes:
    b = name.encode()
    return (struct.pack("<Q", len(b)) + b + struct.pack("<I", len(dims)) + struct.pack(f"<{len(dims)}Q", *dims) +
            struct.pack("<IQ", dtype, offset))


def with_tensors(infos, kvs=b"", n_kv=0, align=32, data_len=0) -> bytes:
    head = struct.pack("<IIQQ", GGUF_MAGIC, 3, len(infos), n_kv) + kvs + b"".join(infos)
    pad = (-len(head)) % align
    return head + b"\0" * pad + b"\0" * data_len


# ---- gguf.rs tests ---------------------------------------------------------

def test_parse_minimal_gguf(tmp_path):
    with parse(tmp_path, minimal()) as g:
        assert g.version == 3 and len(g.tensors) == 0 and g.n_kv == 0


def test_reject_bad_magic(tmp_path):
    d = minimal()
    d[0] = 0xFF
    e = parse_err(tmp_path, d)
    assert e.code == ERR_PARSE and "magic" in str(e)


def test_reject_bad_version(tmp_path):
    d = minimal()
    d[4:8] = struct.pack("<I", 99)
    e = parse_err(tmp_path, d)
    assert e.code == ERR_PARSE and "version 99" in str(e)


def test_reject_excessive_tensor_count(tmp_path):
    d = minimal()
    d[8:16] = struct.pack("<Q", MAX_TENSOR_COUNT + 1)
    assert "tensor count" in str(parse_err(tmp_path, d))


def test_reject_excessive_kv_count(tmp_path):
    d = minimal()
    d[16:24] = struct.pack("<Q", MAX_KV_COUNT + 1)
    assert "KV count" in str(parse_err(tmp_path, d))


def test_reject_truncated_file(tmp_path):
    assert parse_err(tmp_path, bytes(8)).code == ERR_PARSE


def test_parse_with_metadata(tmp_path):
    d = struct.pack("<IIQQ", GGUF_MAGIC, 3, 0, 1) + encode_kv("general.architecture", "llama")
    # the encoding is the one the reference test spells out by hand
    key, val = b"general.architecture", b"llama"
    assert d[24:] == struct.pack("<Q", len(key)) + key + struct.pack("<I", 8) + struct.pack("<Q", len(val)) + val
    with parse(tmp_path, d) as g:
        assert g.get_str("general.architecture") == "llama"


def test_parse_with_tensor(tmp_path):
    """4096 x 4096 F32 at offset 0: the data region (64 MiB) is left as a
    file hole, which the mapping reads as zeros."""
    head = with_tensors([tensor_info("output.weight", (4096, 4096), 0, 0)])
    p = tmp_path / "t.gguf"
    with open(p, "wb") as f:
        f.write(head)
        f.truncate(len(head) + 4096 * 4096 * 4)
    with GgufFile(p) as g:
        assert len(g.tensors) == 1
        t = g.tensors[0]
        assert (t.name, t.dims, t.dtype, t.num_elements) == ("output.weight", (4096, 4096), 0, 4096 * 4096)
        assert t.size_bytes == 4096 * 4096 * 4 and g.data_offset == len(head)


def test_reject_string_too_long(tmp_path):
    d = struct.pack("<IIQQ", GGUF_MAGIC, 3, 0, 1) + struct.pack("<Q", MAX_STRING_LEN + 1)
    assert "string length" in str(parse_err(tmp_path, d))


# ---- beyond the reference's tests ------------------------------------------

def test_missing_file_is_io_error(tmp_path):
    with pytest.raises(YuleGpuError) as e:
        GgufFile(tmp_path / "absent.gguf")
    assert e.value.code == ERR_IO


@pytest.mark.parametrize("cut", [25, 40, 60])
def test_reject_truncated_header(tmp_path, cut):
    d = with_tensors([tensor_info("a", (32,), 0, 0)], data_len=128)
    assert parse_err(tmp_path, d[:cut]).code == ERR_PARSE


def test_reject_tensor_out_of_bounds(tmp_path):
    # Q4_K 256 x 2 needs 288 bytes; only 287 follow the header
    d = with_tensors([tensor_info("w", (256, 2), 12, 0)], data_len=287)
    assert "out of bounds" in str(parse_err(tmp_path, d))
    with parse(tmp_path, with_tensors([tensor_info("w", (256, 2), 12, 0)], data_len=288)) as g:
        assert g.tensors[0].size_bytes == 288


def test_reject_overlapping_tensors(tmp_path):
    infos = [tensor_info("a", (64,), 0, 0), tensor_info("b", (64,), 0, 256)]   # a spans [0, 256)
    with parse(tmp_path, with_tensors(infos, data_len=512)):
        pass
    infos[1] = tensor_info("b", (64,), 0, 255)
    assert "overlapping" in str(parse_err(tmp_path, with_tensors(infos, data_len=512)))


def test_reject_unknown_dtype_and_too_many_dims(tmp_path):
    assert "dtype" in str(parse_err(tmp_path, with_tensors([tensor_info("a", (32,), 99, 0)], data_len=64)))
    assert "dimensions" in str(parse_err(tmp_path, with_tensors([tensor_info("a", (1,) * 9, 0, 0)], data_len=64)))


def test_reject_unknown_value_type(tmp_path):
    d = struct.pack("<IIQQ", GGUF_MAGIC, 3, 0, 1) + struct.pack("<Q", 1) + b"k" + struct.pack("<I", 13)
    assert "value type" in str(parse_err(tmp_path, d))


def test_quantized_size_rounds_up_blocks(tmp_path):
    """size = ceil(n / block) * block_bytes (tensor.rs size_bytes)."""
    infos = [tensor_info("q8", (33,), 8, 0)]     # two Q8_0 blocks
    with parse(tmp_path, with_tensors(infos, data_len=68)) as g:
        assert g.tensors[0].size_bytes == 68


@pytest.mark.parametrize("align", [32, 64, 256])
def test_alignment_key(tmp_path, align):
    kvs = encode_kv("general.alignment", Value(ValueType.U32, align))
    d = with_tensors([tensor_info("a", (8,), 0, 0)], kvs, 1, align=align, data_len=32)
    with parse(tmp_path, d) as g:
        assert g.alignment == align and g.data_offset % align == 0
        assert g.data_offset == (len(d) - 32)


def test_metadata_types(tmp_path):
    md = {"u8": Value(ValueType.U8, 7), "u16": Value(ValueType.U16, 700), "u32": Value(ValueType.U32, 70000),
          "i32": Value(ValueType.I32, 5), "neg": Value(ValueType.I32, -5), "u64": Value(ValueType.U64, 2**40),
          "f32": Value(ValueType.F32, 1e-5), "f64": Value(ValueType.F64, 0.1), "b": True, "s": "héllo",
          "arr": ["a", "bb", "ccc"], "nums": Value(ValueType.ARRAY, [1.0, 2.0], ValueType.F32),
          "nested": Value(ValueType.ARRAY, [[1, 2], [3]], ValueType.ARRAY)}
    p = tmp_path / "m.gguf"
    write_gguf(p, md, [])
    with GgufFile(p) as g:
        assert g.n_kv == len(md)
        # as_u32: u8 / u16 / u32 and non-negative i32 only (gguf.rs:52-60)
        assert [g.get_u32(k) for k in ("u8", "u16", "u32", "i32")] == [7, 700, 70000, 5]
        assert g.get_u32("neg") is None and g.get_u32("u64") is None and g.get_u32("f32") is None
        # as_f64: f32 widened, f64 as is (gguf.rs:73-79)
        assert g.get_f64("f32") == float(np.float32(1e-5)) and g.get_f64("f64") == 0.1
        assert g.get_f64("u32") is None
        assert g.get_str("s") == "héllo" and g.get_str("u32") is None
        assert g.get_array_len("arr") == 3 and g.get_array_len("nums") == 2 and g.get_array_len("nested") == 2
        assert g.get_u32("absent") is None


def test_model_round_trip(tmp_path):
    """SyntheticModel -> GGUF -> parser: every tensor's name, dtype, dims and
    bytes survive, each sits on a 32-byte boundary, and the metadata reads
    back the configuration."""
    m = SyntheticModel.generate(TINY_TEST, seed=5, scheme="Q4_K_M")
    p = tmp_path / "model.gguf"
    m.to_gguf(p)
    c = m.cfg
    with GgufFile(p) as g:
        assert g.get_str("general.architecture") == "llama"
        assert g.get_u32("llama.block_count") == c.n_layers and g.get_u32("llama.embedding_length") == c.dim
        assert g.get_u32("llama.attention.head_count_kv") == c.n_kv_heads
        assert g.get_u32("tokenizer.ggml.vocab_size") == c.vocab
        assert g.get_f64("llama.attention.layer_norm_rms_epsilon") == float(np.float32(c.norm_eps))
        assert len(g.tensors) == len(m.tensors)
        for t in g.tensors:
            src = m[t.name]
            assert t.dtype == int(src.dtype) and t.dims == tuple(src.shape)
            assert (g.data_offset + t.offset) % 32 == 0
            if src.dtype != DType.F32:
                assert t.size_bytes == matrix_bytes(src.dtype, src.shape[1], src.shape[0])
            assert np.array_equal(g.tensor_data(t.name), np.ascontiguousarray(src.data).view(np.uint8).ravel())


def test_find_missing_tensor(tmp_path):
    p = tmp_path / "e.gguf"
    write_gguf(p, {}, [TensorEntry("a", 0, (4,), np.zeros(4, np.float32))])
    with GgufFile(p) as g:
        with pytest.raises(YuleGpuError) as e:
            g.tensor_data("b")
        assert e.value.code == ERR_INVALID
        assert np.array_equal(g.tensor_data("a"), np.zeros(16, np.uint8))


def test_fuzz_corrupted_files_never_crash(tmp_path):
    """Random byte flips, truncations and length-field overwrites of a valid
    model file: the parser either accepts the file (then every tensor lies
    inside it) or raises a parse error; it never reads out of bounds."""
    from yule_amd.model import LlamaConfig
    cfg = LlamaConfig(n_layers=1, dim=256, n_heads=4, n_kv_heads=2, ff_dim=256, vocab=64, max_seq=16)
    p = tmp_path / "base.gguf"
    SyntheticModel.generate(cfg, seed=1, scheme="Q4_K_M").to_gguf(p)
    base = bytearray(p.read_bytes())
    with GgufFile(p) as g:
        header_end = g.data_offset
    rng = np.random.default_rng(7)
    q = tmp_path / "fuzz.gguf"
    outcomes = {"ok": 0, "err": 0}
    for it in range(300):
        d = bytearray(base)
        kind = it % 3
        if kind == 0:      # flip bytes in the header region
            for _ in range(int(rng.integers(1, 8))):
                d[int(rng.integers(0, header_end))] ^= int(rng.integers(1, 256))
        elif kind == 1:    # truncate anywhere
            d = d[: int(rng.integers(0, len(d)))]
        else:              # overwrite an aligned u64 in the header with an extreme value
            pos = int(rng.integers(0, max(1, header_end - 8)))
            extremes = [0, 1, 2**31, 2**32 - 1, 2**63, 2**64 - 1]
            d[pos:pos + 8] = struct.pack("<Q", extremes[int(rng.integers(0, len(extremes)))])
        q.write_bytes(bytes(d))
        try:
            with GgufFile(q) as g:
                for t in g.tensors:
                    assert g.data_offset + t.offset + t.size_bytes <= len(d)
                outcomes["ok"] += 1
        except YuleGpuError as e:
            assert e.code in (ERR_PARSE, ERR_IO)
            outcomes["err"] += 1
    assert outcomes["err"] > 100


@pytest.mark.parametrize("raw,ok", [(b"llama", True), ("héllo 世\U0001F600".encode(), True),
                                     (b"\xff", False), (b"\xc0\xaf", False), (b"\xed\xa0\x80", False),
                                     (b"\xf4\x90\x80\x80", False), (b"\xe2\x82", False)])
def test_strings_must_be_utf8(tmp_path, raw, ok):
    """Keys, string values and tensor names are UTF-8 (gguf.rs:226-243):
    overlong forms, surrogates, code points past U+10FFFF and truncated
    sequences are parse errors."""
    d = struct.pack("<IIQQ", GGUF_MAGIC, 3, 0, 1) + struct.pack("<Q", 1) + b"k" + struct.pack("<I", 8) + \
        struct.pack("<Q", len(raw)) + raw
    if ok:
        with parse(tmp_path, d) as g:
            assert g.get_str("k") == raw.decode()
    else:
        assert "UTF-8" in str(parse_err(tmp_path, d))
