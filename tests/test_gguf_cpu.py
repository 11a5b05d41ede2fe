"""The GGUF reader (thq_gguf_*), on the CPU, against files written by
tests/gguf_writer.py from the file format.

The reader restates [ext] candle-core 0.11 gguf_file::Content::read, the
parser the loader runs first (engine/src/model.rs:526-562). The reference
tree holds no GGUF file, so these checks pin its rules:
  - versions 1-3 parse to the same content, and both byte orders of the magic
    are accepted;
  - dims come back row-major (GGUF's ne reversed) and tensor data starts at
    the alignment Content::read computes;
  - general.alignment counts when it is U8/U16/U32 or a non-negative
    I8/I16/I32, and otherwise the default of 32 applies;
  - strings lose trailing NULs, and invalid UTF-8 becomes U+FFFD exactly as
    Python's decode(errors="replace") does; both follow Unicode's
    maximal-subpart rule, as Rust's from_utf8_lossy does;
  - the typed lookups are as strict as Value::to_u32 / to_f32 / to_string;
  - a repeated key or tensor name replaces the earlier one;
  - a malformed file fails with THQ_EFORMAT at every truncation point and
    never reads out of bounds.
"""
import os
import struct

import numpy as np
import pytest

import gguf_writer as G

thq = pytest.importorskip("thq")


def rng_bytes(n, seed):
    return np.random.default_rng(seed).integers(0, 256, n, dtype=np.uint8).tobytes()


# the metadata a Qwen3 Q4_K_M file carries (a subset) and one tensor per type
KV = [
    ("general.architecture", G.STRING, "qwen3"),
    ("general.name", G.STRING, "Qwen3 8B"),
    ("qwen3.context_length", G.U32, 40960),
    ("qwen3.block_count", G.U32, 36),
    ("qwen3.rope.freq_base", G.F32, 1000000.0),
    ("qwen3.attention.layer_norm_rms_epsilon", G.F32, 1e-6),
    ("tokenizer.ggml.eos_token_id", G.U32, 151645),
    ("tokenizer.ggml.add_bos_token", G.BOOL, 0),
    ("tokenizer.ggml.tokens", G.ARRAY, (G.STRING, ["<|im_start|>", "hello", "world", ""])),
    ("tokenizer.ggml.token_type", G.ARRAY, (G.I32, [3, 1, 1, 1])),
    ("misc.u8", G.U8, 7),
    ("misc.i16", G.I16, -3),
    ("misc.u64", G.U64, 1 << 40),
    ("misc.i64", G.I64, -(1 << 40)),
    ("misc.f64", G.F64, 0.125),
    ("misc.nested", G.ARRAY, (G.ARRAY, [(G.U8, [1, 2]), (G.U16, [3])])),
]
TENSORS = [
    ("blk.0.ffn_down.weight", 14, (16, 512), rng_bytes(16 * 2 * 210, 1)),   # Q6_K [16, 512]
    ("blk.0.ffn_gate.weight", 12, (8, 256), rng_bytes(8 * 144, 2)),         # Q4_K
    ("blk.0.attn_q.weight", 8, (4, 64), rng_bytes(4 * 2 * 34, 3)),          # Q8_0
    ("blk.0.attn_norm.weight", 0, (256,), rng_bytes(256 * 4, 4)),           # F32, 1-D
    ("token_embd.weight", 1, (3, 5, 7), rng_bytes(3 * 5 * 7 * 2, 5)),       # F16, 3-D
]


def write(tmp_path, name, data):
    p = tmp_path / name
    p.write_bytes(data)
    return str(p)


def check_content(f: "thq.GGUFFile", start, offs, tensors=TENSORS):
    assert f.tensor_names() == [t[0] for t in tensors]
    for (name, gt, shape, data), off in zip(tensors, offs):
        info = f.tensor_info(name)
        assert info["type"] == gt and info["shape"] == tuple(shape)
        assert info["offset"] == start + off
        assert info["nbytes"] == len(data)
        assert f.tensor_bytes(name).tobytes() == data
    assert f.string("general.architecture") == "qwen3"
    assert f.u32("qwen3.context_length") == 40960
    assert f.u32("tokenizer.ggml.eos_token_id") == 151645
    assert f.f32("qwen3.rope.freq_base") == 1000000.0
    assert f.f32("qwen3.attention.layer_norm_rms_epsilon") == np.float32(1e-6)
    assert f.array("tokenizer.ggml.tokens") == (G.STRING, 4)
    assert f.array("tokenizer.ggml.token_type") == (G.I32, 4)
    assert f.array("misc.nested") == (G.ARRAY, 2)
    assert f.metadata_keys() == {k: t for k, t, _ in KV}


@pytest.mark.parametrize("version", [1, 2, 3])
def test_versions_parse_to_the_same_content(tmp_path, version):
    data, start, offs = G.build(KV, TENSORS, version=version)
    assert start % 32 == 0
    with thq.GGUFFile(write(tmp_path, f"v{version}.gguf", data)) as f:
        assert f.version == version
        check_content(f, start, offs)


def test_byte_swapped_magic_is_accepted(tmp_path):
    data, start, offs = G.build(KV, TENSORS, magic=b"FUGG")
    with thq.GGUFFile(write(tmp_path, "m.gguf", data)) as f:
        check_content(f, start, offs)


@pytest.mark.parametrize("typ,val,align", [
    (G.U32, 64, 64), (G.U8, 16, 16), (G.U16, 256, 256), (G.I8, 8, 8), (G.I32, 128, 128),
    (G.I32, -1, 32),      # negative: default
    (G.U64, 128, 32),     # U64 is not read: default
    (G.F32, 64.0, 32),    # nor a float
    (G.STRING, "64", 32),
    (G.U32, 1, 1),        # unaligned data section
    (G.U32, 7, 7),
])
def test_general_alignment(tmp_path, typ, val, align):
    kv = [("general.alignment", typ, val)] + KV
    assert G.effective_alignment(kv) == align
    data, start, offs = G.build(kv, TENSORS)
    assert start % align == 0
    with thq.GGUFFile(write(tmp_path, "a.gguf", data)) as f:
        for (name, _, _, blob), off in zip(TENSORS, offs):
            assert f.tensor_info(name)["offset"] == start + off
            assert f.tensor_bytes(name).tobytes() == blob


STRINGS = [b"abc\x00\x00", b"\xff", b"a\xe2\x82b", b"\xf0\x80\x80", b"\xed\xa0\x80", b"\xf4\x90\x80\x80",
           b"\xc0\xaf", b"\xe0\x9f\xbf", "héllo → \U0001F600".encode(), b"\xf0\x9f\x98", b"\x80\x80x",
           b"mid\x00nul", b""]


def test_strings_are_utf8_lossy_without_trailing_nuls(tmp_path):
    kv = [(f"s{i}", G.STRING, s) for i, s in enumerate(STRINGS)]
    # tensor names and keys take the same path
    tensors = [(b"t\xff\x00", 0, (1,), b"\x00\x00\x80\x3f")]
    data, _, _ = G.build(kv, tensors)
    with thq.GGUFFile(write(tmp_path, "s.gguf", data)) as f:
        for i, s in enumerate(STRINGS):
            want = s.rstrip(b"\x00").decode("utf-8", "replace")
            assert f.string(f"s{i}") == want, (s, f.string(f"s{i}"))
        assert f.tensor_names() == ["t�"]


def test_repeated_keys_and_tensor_names_keep_the_last(tmp_path):
    kv = [("a", G.U32, 1), ("b", G.STRING, "x"), ("a", G.U32, 2)]
    t1, t2 = rng_bytes(34, 6), rng_bytes(68, 7)
    data, start, offs = G.build(kv, [("w", 8, (1, 32), t1), ("w", 8, (2, 32), t2)])
    with thq.GGUFFile(write(tmp_path, "d.gguf", data)) as f:
        assert f.u32("a") == 2
        assert f.metadata_keys() == {"a": G.U32, "b": G.STRING}
        assert f.tensor_names() == ["w"]
        info = f.tensor_info("w")
        assert info["shape"] == (2, 32) and info["offset"] == start + offs[1]
        assert f.tensor_bytes("w").tobytes() == t2


def test_typed_lookups_are_strict(tmp_path):
    data, _, _ = G.build(KV, TENSORS)
    with thq.GGUFFile(write(tmp_path, "t.gguf", data)) as f:
        for fn, key in [(f.u32, "misc.u8"), (f.u32, "misc.u64"), (f.u32, "qwen3.rope.freq_base"),
                        (f.f32, "misc.f64"), (f.f32, "qwen3.context_length"), (f.string, "misc.u8"),
                        (f.array, "general.name")]:
            with pytest.raises(thq.ThqError) as e:
                fn(key)
            assert e.value.code == thq.EDTYPE
        for fn in (f.u32, f.f32, f.string, f.array):
            with pytest.raises(thq.ThqError) as e:
                fn("no.such.key")
            assert e.value.code == thq.ENOTFOUND
        assert f.find("no.such.tensor") == -1


def test_tensor_data_errors(tmp_path):
    t_ok = rng_bytes(144, 8)
    tensors = [("ok", 12, (1, 256), t_ok),
               ("ragged", 12, (1, 100), b""),                  # 100 elements: not whole Q4_K blocks
               ("past_eof", 8, (1, 32), b"", 1 << 20)]          # offset past the end
    data, _, _ = G.build([], tensors)
    with thq.GGUFFile(write(tmp_path, "e.gguf", data)) as f:
        assert f.tensor_bytes("ok").tobytes() == t_ok
        with pytest.raises(thq.ThqError) as e:
            f.tensor_bytes("ragged")
        assert e.value.code == thq.ESHAPE
        with pytest.raises(thq.ThqError) as e:
            f.tensor_bytes("past_eof")
        assert e.value.code == thq.EFORMAT


def build_raw_kv(value_type: int, payload: bytes) -> bytes:
    """a v3 header with one metadata entry of an arbitrary type id"""
    w = G._W(3)
    w.buf += b"GGUF"
    w.u32(3)
    w.length(0)
    w.length(1)
    w.string("k")
    w.u32(value_type)
    w.buf += payload
    return bytes(w.buf)


def test_malformed_headers(tmp_path):
    base = G.build(KV[:3], TENSORS[:2])[0]
    cases = {"magic": b"GGML" + base[4:]}
    for v in (0, 4):
        b = bytearray(base)
        b[4:8] = struct.pack("<I", v)
        cases[f"version {v}"] = bytes(b)
    cases["value type 13"] = build_raw_kv(13, b"\x00" * 8)
    cases["bool 2"] = build_raw_kv(G.BOOL, b"\x02")
    cases["array of type 99"] = build_raw_kv(G.ARRAY, struct.pack("<IQ", 99, 1) + b"\x00" * 8)
    cases["unknown ggml type 16"] = G.build([], [("w", 16, (1, 256), b"")])[0]
    cases["ggml type 4 (removed Q4_2)"] = G.build([], [("w", 4, (1, 32), b"")])[0]
    # GGML tensors have at most 4 dims; the reader rejects more
    cases["5 dims"] = G.build([], [("w", 0, (1, 1, 1, 1, 1), b"\x00" * 4)])[0]
    cases["string past the end"] = build_raw_kv(G.STRING, struct.pack("<Q", 1 << 40) + b"abc")
    cases["alignment 0"] = G.build([("general.alignment", G.U32, 0)], [], data_align=32)[0]
    cases["empty file"] = b""
    for name, data in cases.items():
        with pytest.raises(thq.ThqError) as e:
            thq.GGUFFile(write(tmp_path, "bad.gguf", data))
        assert e.value.code == thq.EFORMAT, name


def test_every_truncation_of_the_header_fails_cleanly(tmp_path):
    data, _, _ = G.build(KV, TENSORS[:3])
    # the header proper ends before the alignment padding: its length is the
    # data start of the same file laid out with alignment 1
    header_end = G.build(KV, TENSORS[:3], data_align=1)[1]
    p = tmp_path / "cut.gguf"
    for cut in range(0, header_end):
        p.write_bytes(data[:cut])
        with pytest.raises(thq.ThqError) as e:
            thq.GGUFFile(str(p))
        assert e.value.code == thq.EFORMAT, cut
    # the full header alone (no data) opens; the tensors' bytes are missing
    p.write_bytes(data[:header_end])
    with thq.GGUFFile(str(p)) as f:
        with pytest.raises(thq.ThqError) as e:
            f.tensor_bytes(TENSORS[0][0])
        assert e.value.code == thq.EFORMAT


def test_missing_file_and_null_handles(tmp_path):
    with pytest.raises(thq.ThqError) as e:
        thq.GGUFFile(str(tmp_path / "absent.gguf"))
    assert e.value.code == thq.EIO
    L = thq.lib
    assert L.thq_gguf_tensor_count(None) == -1
    assert L.thq_gguf_find_tensor(None, b"x") == -1
    assert L.thq_gguf_open(None, None) == thq.EINVAL
    L.thq_gguf_close(None)  # no-op


def raw_header(n_tensors: int, n_kv: int, body: bytes = b"") -> bytes:
    return b"GGUF" + struct.pack("<IQQ", 3, n_tensors, n_kv) + body


def raw_tensor_info(name: str, ne, ggml_type: int, offset: int) -> bytes:
    """one tensor info as GGUF stores it (ne fastest dimension first)"""
    b = struct.pack("<Q", len(name)) + name.encode() + struct.pack("<I", len(ne))
    for d in ne:
        b += struct.pack("<Q", d)
    return b + struct.pack("<IQ", ggml_type, offset)


def test_hostile_counts_and_sizes_fail_cleanly(tmp_path):
    """Counts and sizes near the integer limits are format errors: the reader
    neither reserves memory for them nor lets a size or offset wrap."""
    cases = {
        "tensor count 2^40": raw_header(1 << 40, 0),
        "tensor count 2^63": raw_header(1 << 63, 0),
        "metadata count 2^40": raw_header(0, 1 << 40),
        "metadata count 2^64-1": raw_header(0, (1 << 64) - 1),
        "array of 2^62 u8": build_raw_kv(G.ARRAY, struct.pack("<IQ", G.U8, 1 << 62)),
        "array of 2^40 strings": build_raw_kv(G.ARRAY, struct.pack("<IQ", G.STRING, 1 << 40)),
        "array of 2^61 u64": build_raw_kv(G.ARRAY, struct.pack("<IQ", G.U64, 1 << 61)),
        "tensor name length 2^63": raw_header(1, 0, struct.pack("<Q", 1 << 63) + b"w"),
        "element count overflows": raw_header(1, 0, raw_tensor_info("w", (1 << 33, 1 << 33), 0, 0)),
        "byte size overflows": raw_header(1, 0, raw_tensor_info("w", (1 << 62,), 0, 0)),
    }
    for name, data in cases.items():
        with pytest.raises(thq.ThqError) as e:
            thq.GGUFFile(write(tmp_path, "bad.gguf", data))
        assert e.value.code == thq.EFORMAT, name
    # an offset that wraps past 2^64 with the tensor's size: no data, never a pointer
    data = raw_header(1, 0, raw_tensor_info("w", (4,), 0, (1 << 64) - 8))
    try:
        f = thq.GGUFFile(write(tmp_path, "off.gguf", data))
    except thq.ThqError as e:
        assert e.code == thq.EFORMAT
    else:
        with f:
            with pytest.raises(thq.ThqError) as e:
                f.tensor_bytes("w")
            assert e.value.code == thq.EFORMAT


def test_random_corruption_never_reads_out_of_bounds(tmp_path):
    """Bit flips and 8-byte overwrites anywhere in a valid header give either a
    parse or THQ_EFORMAT; every string and tensor the parse returns lies inside
    the file (each is read here in full)."""
    import ctypes as C
    data, _, _ = G.build(KV, TENSORS)
    header_end = G.build(KV, TENSORS, data_align=1)[1]
    rng = np.random.default_rng(11)
    p = tmp_path / "x.gguf"
    L = thq.lib
    opened = 0
    for trial in range(1500):
        b = bytearray(data)
        pos = int(rng.integers(0, header_end))
        if trial % 3 == 0:
            b[pos:pos + 8] = rng_bytes(8, trial)[: len(b[pos:pos + 8])]
        else:
            b[pos] ^= 1 << int(rng.integers(0, 8))
        p.write_bytes(bytes(b))
        h = C.c_void_p()
        rc = L.thq_gguf_open(str(p).encode(), C.byref(h))
        if rc != 0:
            assert rc == thq.EFORMAT, (trial, pos, rc)
            continue
        opened += 1
        try:
            for i in range(L.thq_gguf_metadata_count(h)):
                key, vt = C.c_char_p(), C.c_uint32()
                assert L.thq_gguf_metadata_key(h, i, C.byref(key), C.byref(vt)) == 0
                if vt.value == G.STRING:
                    s, n = C.c_void_p(), C.c_uint64()
                    assert L.thq_gguf_metadata_str(h, key.value, C.byref(s), C.byref(n)) == 0
                    assert n.value <= len(b)
                    C.string_at(s.value, n.value) if n.value else b""
            for i in range(L.thq_gguf_tensor_count(h)):
                d, n = C.c_void_p(), C.c_uint64()
                rc = L.thq_gguf_tensor_data(h, i, C.byref(d), C.byref(n))
                assert rc in (0, thq.EFORMAT, thq.ESHAPE), (trial, rc)  # ESHAPE: elements not whole blocks
                if rc == 0 and n.value:
                    assert n.value <= len(b)
                    C.string_at(d.value, n.value)
        finally:
            L.thq_gguf_close(h)
    assert opened > 0
