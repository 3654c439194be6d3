"""GGUF container: the library's native reader (frq_gguf_*, through
fuel_amd.GgufFile) and the oracle's Python restatement of
fuel_formats::gguf::Content::read (fuel-formats/src/gguf.rs:378-461), both
against files assembled field by field here with struct.pack (known answers),
then against each other on written files.  The last test uploads tensors of a
file to the GPU (load_quantized) and runs QMatMul on them."""
import struct

import numpy as np
import pytest

import fuel_amd as F
import oracle as O
from oracle import gguf as G


def s64(x: bytes) -> bytes:  # v2/v3 string
    return struct.pack("<Q", len(x)) + x


def s32(x: bytes) -> bytes:  # v1 string
    return struct.pack("<I", len(x)) + x


def kv(key: bytes, vt: int, payload: bytes, v1=False) -> bytes:
    return (s32(key) if v1 else s64(key)) + struct.pack("<I", vt) + payload


def hand_file(version=3, align_entry=None, extra_kv=b"", extra_kv_count=0):
    """Metadata of every scalar type, a string, a nested array; two tensors."""
    v1 = version == 1
    S = s32 if v1 else s64
    cnt = (lambda n: struct.pack("<I", n)) if v1 else (lambda n: struct.pack("<Q", n))
    kvs = [
        kv(b"u8", 0, struct.pack("<B", 200), v1),
        kv(b"i8", 1, struct.pack("<b", -5), v1),
        kv(b"u16", 2, struct.pack("<H", 65000), v1),
        kv(b"i16", 3, struct.pack("<h", -30000), v1),
        kv(b"u32", 4, struct.pack("<I", 4000000000), v1),
        kv(b"i32", 5, struct.pack("<i", -2000000000), v1),
        kv(b"f32", 6, struct.pack("<f", 0.1), v1),
        kv(b"bool", 7, struct.pack("<B", 1), v1),
        kv(b"str", 8, S(b"llama\0\0"), v1),
        kv(b"arr", 9, struct.pack("<I", 9) + cnt(2)
           + struct.pack("<I", 4) + cnt(2) + struct.pack("<II", 1, 2)
           + struct.pack("<I", 4) + cnt(0), v1),
        kv(b"u64", 10, struct.pack("<Q", 2 ** 63 + 7), v1),
        kv(b"i64", 11, struct.pack("<q", -(2 ** 62)), v1),
        kv(b"f64", 12, struct.pack("<d", -2.5), v1),
    ]
    if align_entry is not None:
        kvs.append(kv(b"general.alignment", align_entry[0], align_entry[1], v1))
    dimw = (lambda d: struct.pack("<I", d)) if v1 else (lambda d: struct.pack("<Q", d))
    # tensor "w": file dims (512, 3) = ne0 512 (inner), ne1 3 -> fuel shape (3, 512), Q4_K
    # tensor "g": file dims (256,) F32 at offset 1024
    tens = (S(b"w") + struct.pack("<I", 2) + dimw(512) + dimw(3) + struct.pack("<IQ", 12, 0)
            + S(b"g") + struct.pack("<I", 1) + dimw(256) + struct.pack("<IQ", 0, 1024))
    head = struct.pack("<II", 0x46554747, version) + cnt(2) + cnt(len(kvs) + extra_kv_count)
    return head + b"".join(kvs) + extra_kv + tens


def check_known(c, version, header_len, align=32):
    md = {k: G.plain(v) for k, v in c["meta"].items()}
    assert md["u8"] == 200 and md["i8"] == -5 and md["u16"] == 65000 and md["i16"] == -30000
    assert md["u32"] == 4000000000 and md["i32"] == -2000000000
    assert md["f32"] == float(np.float32(0.1)) and md["bool"] is True
    assert md["str"] == "llama"                       # trailing NULs dropped
    assert md["arr"] == [[1, 2], []]
    assert md["u64"] == 2 ** 63 + 7 and md["i64"] == -(2 ** 62) and md["f64"] == -2.5
    assert c["types"]["arr"] == G.VT_ARRAY and c["types"]["f32"] == G.VT_F32
    assert c["version"] == version
    w, g = c["tensors"]["w"], c["tensors"]["g"]
    assert (w.dtype, tuple(w.dims), w.offset, w.nbytes) == (12, (3, 512), 0, 3 * 2 * 144)
    assert (g.dtype, tuple(g.dims), g.offset, g.nbytes) == (0, (256,), 1024, 1024)
    assert c["data_offset"] == (header_len + align - 1) // align * align


def parse_both(tmp_path, data: bytes):
    p = tmp_path / "t.gguf"
    p.write_bytes(data)
    o = G.read(data)
    n = F.GgufFile(str(p))
    oc = {"meta": o.metadata, "types": {k: v.type for k, v in o.metadata.items()}, "version": o.version,
          "tensors": o.tensors, "data_offset": o.tensor_data_offset}
    nc = {"meta": {k: G.Value(v.type, _conv(v)) for k, v in n.values.items()},
          "types": {k: v.type for k, v in n.values.items()}, "version": n.version,
          "tensors": n.tensors, "data_offset": n.tensor_data_offset}
    return oc, nc, n


def _conv(v):
    # fuel_amd.gguf.Value -> oracle Value tree (same field names)
    if v.type == G.VT_ARRAY:
        return [G.Value(e.type, _conv(e)) for e in v.value]
    return v.value


@pytest.mark.parametrize("version", [1, 2, 3])
def test_known_answer_versions(tmp_path, version):
    data = hand_file(version)
    oc, nc, _ = parse_both(tmp_path, data)
    check_known(oc, version, len(data))
    check_known(nc, version, len(data))


@pytest.mark.parametrize("entry,align", [
    ((4, struct.pack("<I", 64)), 64),      # u32
    ((0, struct.pack("<B", 16)), 16),      # u8
    ((2, struct.pack("<H", 128)), 128),    # u16
    ((5, struct.pack("<i", 8)), 8),        # non-negative i32
    ((5, struct.pack("<i", -1)), 32),      # negative i32: default
    ((10, struct.pack("<Q", 64)), 32),     # u64 is not among the accepted types: default
    ((8, s64(b"64")), 32),                 # a string: default
])
def test_alignment_rules(tmp_path, entry, align):
    data = hand_file(3, entry)
    oc, nc, _ = parse_both(tmp_path, data)
    check_known(oc, 3, len(data), align)
    check_known(nc, 3, len(data), align)


def test_zero_alignment_is_an_error(tmp_path):
    data = hand_file(3, (4, struct.pack("<I", 0)))
    with pytest.raises(G.GgufError):
        G.read(data)
    p = tmp_path / "z.gguf"
    p.write_bytes(data)
    with pytest.raises(F.FuelRocmError, match="alignment"):
        F.GgufFile(str(p))


def test_byte_swapped_magic_and_repeated_key(tmp_path):
    data = bytearray(hand_file(3, extra_kv=kv(b"u8", 4, struct.pack("<I", 7)), extra_kv_count=1))
    data[0:4] = struct.pack("<I", 0x47475546)
    oc, nc, n = parse_both(tmp_path, bytes(data))
    for c in (oc, nc):
        assert G.plain(c["meta"]["u8"]) == 7 and c["types"]["u8"] == G.VT_U32  # the last value wins
        assert list(c["meta"])[0] == "u8"                                      # at its first position


@pytest.mark.parametrize("raw,want", [
    (b"a\0b", "a\0b"),                                  # embedded NUL kept
    (b"caf\xc3\xa9", "café"),
    (b"\xe0\x80x", "��x"),                    # E0 needs A0..BF next
    (b"\xf0\x9f\x98", "�"),                        # truncated 4-byte sequence: one replacement
    (b"\xed\xa0\x80", "���"),            # surrogate range
    (b"\xff\xc2", "��"),
])
def test_string_cleanup(tmp_path, raw, want):
    data = (struct.pack("<II", 0x46554747, 3) + struct.pack("<QQ", 0, 1) + kv(b"s", 8, s64(raw + b"\0")))
    oc, nc, _ = parse_both(tmp_path, data)
    assert oc["meta"]["s"].value == want
    assert nc["meta"]["s"].value == want


@pytest.mark.parametrize("mutate,msg", [
    (lambda d: b"GGML" + d[4:], "unknown magic"),
    (lambda d: d[:4] + struct.pack("<I", 4) + d[8:], "unsupported magic/version"),
    (lambda d: d.replace(kv(b"bool", 7, b"\x01"), kv(b"bool", 7, b"\x02")), "unexpected bool value 2"),
    (lambda d: d.replace(kv(b"bool", 7, b"\x01"), kv(b"bool", 13, b"\x01")), "unrecognized value-type"),
    (lambda d: d.replace(struct.pack("<IQ", 12, 0), struct.pack("<IQ", 4, 0)), "unknown dtype for tensor 4"),
    (lambda d: d[:-5], "end of file"),
])
def test_errors(tmp_path, mutate, msg):
    data = mutate(hand_file(3))
    with pytest.raises(G.GgufError):
        G.read(data)
    p = tmp_path / "e.gguf"
    p.write_bytes(data)
    with pytest.raises(F.FuelRocmError, match=msg):
        F.GgufFile(str(p))


@pytest.mark.parametrize("version", [1, 3])
def test_written_file_round_trip(tmp_path, version):
    rng = np.random.default_rng(version)
    w = O.quantize(O.Q4K, O.normal((4, 512), seed=3, stream=1, std=0.02))
    q6 = O.quantize(O.Q6K, O.normal((2, 256), seed=3, stream=2, std=0.02))
    g = rng.standard_normal(512).astype(np.float32)
    md = [("general.architecture", G.Value(G.VT_STRING, "llama")),
          ("general.alignment", G.Value(G.VT_U32, 64)),
          ("llama.block_count", G.Value(G.VT_U32, 2)),
          ("tokenizer.ggml.tokens", G.Value(G.VT_ARRAY, [G.Value(G.VT_STRING, t) for t in ("<s>", "a", "é")])),
          ("llama.rope.freq_base", G.Value(G.VT_F32, 10000.0))]
    tens = [("blk.0.attn_q.weight", 12, (4, 512), w.tobytes()),
            ("blk.0.attn_v.weight", 14, (2, 256), q6.tobytes()),
            ("blk.0.attn_norm.weight", 0, (512,), g.tobytes())]
    data = G.write(md, tens, version=version, alignment=64)
    p = tmp_path / "m.gguf"
    p.write_bytes(data)
    o, n = G.read(data), F.GgufFile(str(p))
    assert n.tensor_data_offset == o.tensor_data_offset and n.tensor_data_offset % 64 == 0
    assert n.metadata == {k: G.plain(v) for k, v in o.metadata.items()}
    for name, dt, dims, raw in tens:
        ti = n.tensors[name]
        assert (ti.dtype, ti.dims, ti.nbytes) == (dt, dims, len(raw)) and ti == n.tensors[name]
        assert (o.tensors[name].offset, o.tensors[name].nbytes) == (ti.offset, ti.nbytes)
        assert n.tensor_bytes(name).tobytes() == raw
    with pytest.raises(F.FuelRocmError, match="missing tensor"):
        n.tensor_bytes("nope")


def test_tensor_outside_file_is_an_error(tmp_path):
    data = G.write([], [("w", 12, (1, 256), bytes(144))])
    data = data[:-10]  # the tensor's bytes run past the end
    p = tmp_path / "s.gguf"
    p.write_bytes(data)
    n = F.GgufFile(str(p))
    with pytest.raises(F.FuelRocmError, match="outside"):
        n.tensor_bytes("w")


@pytest.mark.gpu
def test_load_quantized_and_matmul(tmp_path, dev):
    """Tensors of a file uploaded verbatim (load_quantized) and used by QMatMul."""
    k, n = 1024, 96
    tens, mats = [], {}
    for dt in (O.Q4K, O.Q6K, O.Q8_0):
        wq = O.quantize(dt, O.normal((n, k), seed=7, stream=dt, std=0.02))
        name = f"w{dt}"
        tens.append((name, dt, (n, k), wq.tobytes()))
        mats[name] = (dt, wq)
    p = tmp_path / "q.gguf"
    p.write_bytes(G.write([("general.alignment", G.Value(G.VT_U32, 32))], tens))
    f = F.GgufFile(str(p))
    x = O.normal((3, k), seed=7, stream=99)
    for name, (dt, wq) in mats.items():
        qs = f.load_quantized(dev, name)
        assert qs.dtype() == dt and qs.data() == wq.tobytes()
        y, shape = qs.fwd((n, k), dev.from_numpy(x))
        assert shape == (3, n)
        from blockref import rel_err
        assert rel_err(y.numpy(), O.matmul(dt, x, wq)) <= 1e-3
