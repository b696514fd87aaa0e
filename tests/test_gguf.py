"""GGUF model store (include/si_hip_gguf.h) against the reference's own GGUF
fixture and assertions (src/model.rs:1913-2008), against a GGUF writer in
this file that shares no code with the reader, and against Python's UTF-8
decoder for the string errors.  Everything here but the last tests runs on
the CPU; the `gpu` tests upload tensors from a store and check the kernels
see exactly the bytes a direct upload gives them."""
from __future__ import annotations

import math
import random
import struct
from pathlib import Path

import numpy as np
import pytest

import si_hip
from si_hip import GgufFile, GgufValue, HipError

GOLDEN = Path(__file__).resolve().parent / "golden"
TINY = GOLDEN / "tiny_qwen35.gguf"

U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
Q4K, Q5K, Q6K = si_hip.GGML_TYPE_Q4_K, si_hip.GGML_TYPE_Q5_K, si_hip.GGML_TYPE_Q6_K
BLOCK_BYTES = {Q4K: 144, Q5K: 176, Q6K: 210}


# ---- an independent writer ----------------------------------------------------

_SCALAR = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f",
           U64: "<Q", I64: "<q", F64: "<d"}


def _str(s: str | bytes) -> bytes:
    raw = s.encode("utf-8") if isinstance(s, str) else s
    return struct.pack("<Q", len(raw)) + raw


class Raw(bytes):
    """Bytes written as a value's payload whatever its declared type."""


def _val(t: int, v) -> bytes:
    """GGUF value payload; arrays are (element_type, [items])."""
    if isinstance(v, Raw):
        return bytes(v)
    if t in _SCALAR:
        return struct.pack(_SCALAR[t], v)
    if t == BOOL:
        return struct.pack("<B", v)
    if t == STR:
        return _str(v)
    if t == ARR:
        et, items = v
        return struct.pack("<IQ", et, len(items)) + b"".join(_val(et, x) for x in items)
    raise ValueError(t)


def write_gguf(metadata, tensors, alignment=32, version=3, data_tail=b""):
    """metadata: [(key, type, value)]; tensors: [(name, shape, ggml_type,
    offset, payload bytes)].  Payloads are placed at data base + offset
    (empty ones take no room, whatever their offset); returns the file bytes
    and the data base."""
    b = bytearray(b"GGUF")
    b += struct.pack("<IQQ", version, len(tensors), len(metadata))
    for key, t, v in metadata:
        b += _str(key) + struct.pack("<I", t) + _val(t, v)
    for name, shape, gt, off, _ in tensors:
        b += _str(name) + struct.pack("<I", len(shape))
        b += b"".join(struct.pack("<Q", d) for d in shape)
        b += struct.pack("<IQ", gt, off)
    base = -(-len(b) // alignment) * alignment
    size = max([off + len(p) for _, _, _, off, p in tensors if p], default=0)
    out = bytearray(b) + bytearray(base - len(b) + size)
    for _, _, _, off, p in tensors:
        if p:
            out[base + off: base + off + len(p)] = p
    return bytes(out) + data_tail, base


def _err(data: bytes) -> str:
    with pytest.raises(HipError) as e:
        GgufFile(data=data)
    return str(e.value).split(": ", 1)[1]


# ---- the reference's fixture and assertions ----------------------------------

def test_committed_fixture_is_what_its_script_writes():
    import importlib.util
    spec = importlib.util.spec_from_file_location("make_gguf_fixture",
                                                  GOLDEN / "make_gguf_fixture.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    assert TINY.read_bytes() == mod.tiny_fixture()


@pytest.mark.parametrize("source", ["path", "bytes"])
def test_parses_reference_fixture(source):
    """parses_gguf_metadata_and_tensor_index (src/model.rs:1913-1928)."""
    g = GgufFile(path=TINY) if source == "path" else GgufFile(data=TINY.read_bytes())
    assert g.metadata["general.architecture"] == GgufValue(STR, "qwen35")
    assert g.metadata["general.alignment"] == GgufValue(U32, 32)
    assert len(g.tensor_list) == 1
    t = g.tensor_list[0]
    assert t.name == "blk.0.attn_q.weight"
    assert t.shape == (4, 2)
    assert t.ggml_type == 0
    assert t.data_start % 32 == 0
    # and what the fixture's layout fixes beyond those assertions
    assert (g.version, g.alignment, g.data_base) == (3, 32, 192)
    assert (t.data_start, t.data_end) == (192, 200)
    info, data = g.tensor("blk.0.attn_q.weight")
    assert data.tolist() == [1, 2, 3, 4, 5, 6, 7, 8]
    assert g.element_count("blk.0.attn_q.weight") == 8
    assert g.expected_payload_bytes("blk.0.attn_q.weight") == 32
    g.close()


def test_rejects_invalid_magic_and_truncation():
    """rejects_invalid_gguf_magic_and_truncation (src/model.rs:1974-1979)."""
    assert _err(b"NOPE") == "GGUF header has invalid magic"
    assert _err(TINY.read_bytes()[:20]) == "GGUF header is truncated"


def test_every_prefix_of_the_fixture():
    """The index ends at byte 162 and its data base is 192: every shorter
    prefix is truncated, the padding-only ones put the tensor past the end,
    and from 192 on the one tensor runs to the end of whatever is there."""
    full = TINY.read_bytes()
    for n in range(len(full) + 1):
        if n < 162:
            assert _err(full[:n]) == "GGUF header is truncated", n
        elif n < 192:
            assert _err(full[:n]) == "GGUF tensor blk.0.attn_q.weight exceeds file size", n
        else:
            g = GgufFile(data=full[:n])
            t = g.tensor_list[0]
            assert (t.data_start, t.data_end) == (192, n)
            assert g.tensor(t.name)[1].tolist() == list(range(1, n - 191))


def test_inspect_of_reference_fixture():
    """si-gguf-inspect (src/bin/si-gguf-inspect.rs:11-60) on the fixture."""
    g = GgufFile(path=TINY)
    assert g.inspect("tiny.gguf").splitlines() == [
        "model=tiny.gguf",
        "tensors=1",
        "tensor_type_counts={0: 1}",
        "non_q4_tensor=blk.0.attn_q.weight type=0 shape=[4, 2] bytes=8",
        "metadata.general.alignment=U32(32)",
        'metadata.general.architecture=string("qwen35")',
    ]


# ---- header and metadata rules -----------------------------------------------

def _with_header(version=3):
    return write_gguf([("general.architecture", STR, "qwen35")], [], version=version)[0]


@pytest.mark.parametrize("version,ok", [(0, False), (1, False), (2, True), (3, True), (4, False),
                                        (0xffffffff, False)])
def test_versions(version, ok):
    data = _with_header(version)
    if ok:
        assert GgufFile(data=data).version == version
    else:
        assert _err(data) == f"unsupported GGUF version {version}"


def test_duplicate_metadata_keys_rejected():
    data, _ = write_gguf([("a", U32, 1), ("b", U32, 2), ("a", U8, 3)], [])
    assert _err(data) == "GGUF metadata contains duplicate keys"


def test_unsupported_metadata_type():
    data, _ = write_gguf([("a", U32, 1), ("b", 13, Raw(b"\1\0\0\0"))], [])
    assert _err(data) == "unsupported GGUF metadata type 13"
    # an array of an unknown type is read only item by item: empty is fine
    data, _ = write_gguf([("e", ARR, (99, []))], [])
    g = GgufFile(data=data)
    assert g.metadata["e"] == GgufValue(ARR, [])
    data, _ = write_gguf([("e", ARR, Raw(struct.pack("<IQB", 99, 1, 1)))], [])
    assert _err(data) == "unsupported GGUF metadata type 99"


def test_counts_past_the_end_are_truncation():
    data, _ = write_gguf([("e", ARR, Raw(struct.pack("<IQQQ", U64, 1 << 62, 1, 2)))], [])
    assert _err(data) == "GGUF header is truncated"
    data, _ = write_gguf([("k", STR, Raw(struct.pack("<Q", (1 << 64) - 1) + b"v"))], [])
    assert _err(data) == "GGUF offset overflows"
    data, _ = write_gguf([("k", STR, Raw(struct.pack("<Q", 1 << 40) + b"v"))], [])
    assert _err(data) == "GGUF header is truncated"
    hdr = b"GGUF" + struct.pack("<IQQ", 3, 1 << 60, 0)
    assert _err(hdr + bytes(64)) == "GGUF header is truncated"
    hdr = b"GGUF" + struct.pack("<IQQ", 3, 0, 1 << 60)
    assert _err(hdr + _str("k") + struct.pack("<IB", U8, 1) + bytes(5)) == \
        "GGUF header is truncated"
    rank = _str("w") + struct.pack("<I", 0xffffffff) + struct.pack("<Q", 1)
    assert _err(b"GGUF" + struct.pack("<IQQ", 3, 1, 0) + rank) == "GGUF header is truncated"


def test_deep_array_nesting_is_bounded():
    v = (U8, [7])
    for _ in range(200):
        v = (ARR, [v])
    data, _ = write_gguf([("deep", ARR, v)], [])
    g = GgufFile(data=data)
    x = g.metadata["deep"]
    for _ in range(200):
        x = x.value[0]
    assert x == GgufValue(ARR, [GgufValue(U8, 7)])
    for _ in range(100):
        v = (ARR, [v])
    data, _ = write_gguf([("deep", ARR, v)], [])
    assert _err(data) == "GGUF metadata arrays nest too deeply"


@pytest.mark.parametrize("key,t,v,expect", [
    ("general.alignment", U32, 64, 64),
    ("general.alignment", U64, 4096, 4096),
    ("general.alignment", U32, 1, 1),
    ("general.alignment", I32, 64, 32),     # only U32/U64 count
    ("general.alignment", STR, "64", 32),
    ("other.alignment", U32, 64, 32),
])
def test_alignment_sources(key, t, v, expect):
    data, base = write_gguf([(key, t, v)], [("w", [4], 0, 0, bytes(16))], alignment=expect)
    g = GgufFile(data=data)
    assert g.alignment == expect and g.data_base == base
    assert g.data_base % expect == 0
    assert g.tensor_list[0].data_start == base


@pytest.mark.parametrize("t,v", [(U32, 0), (U32, 48), (U64, 3), (U64, 1 << 63 | 1), (U64, 0)])
def test_bad_alignment_rejected(t, v):
    data, _ = write_gguf([("general.alignment", t, v)], [])
    assert _err(data) == "GGUF alignment must be a non-zero power of two"


def test_largest_alignment():
    """2^63 still aligns a small offset (to 2^63) without overflowing; a
    tensor then lies past the end of any file."""
    data, _ = write_gguf([("general.alignment", U64, 1 << 63)], [])
    assert GgufFile(data=data).data_base == 1 << 63
    data, _ = write_gguf([("general.alignment", U64, 1 << 63)], [("w", [4], 0, 0, b"")],
                         alignment=64)
    assert _err(data) == "GGUF tensor w exceeds file size"


def test_tensor_past_end_of_file():
    data, base = write_gguf([], [("b", [4], 0, 64, bytes(16)), ("a", [4], 0, 0, bytes(16))])
    g = GgufFile(data=data)
    assert g.tensors["b"].data_end == len(data) == base + 80
    # the ranges are checked in offset order: a's end (b's start) fails first
    assert _err(data[:base + 63]) == "GGUF tensor a exceeds file size"
    assert GgufFile(data=data[:base + 64]).tensors["b"].byte_len() == 0


def test_offset_overflow_messages():
    data, _ = write_gguf([], [("a", [4], 0, (1 << 64) - 8, b"")])
    assert _err(data) == "GGUF tensor a start overflows"
    data, _ = write_gguf([], [("a", [4], 0, 0, bytes(16)), ("b", [4], 0, (1 << 64) - 8, b"")])
    assert _err(data) == "GGUF tensor a end overflows"


# ---- UTF-8: the position and length core::str::from_utf8 reports ------------

def _python_utf8_message(raw: bytes) -> str | None:
    try:
        raw.decode("utf-8")
        return None
    except UnicodeDecodeError as e:
        if e.reason == "unexpected end of data":
            return f"incomplete utf-8 byte sequence from index {e.start}"
        return f"invalid utf-8 sequence of {e.end - e.start} bytes from index {e.start}"


def test_utf8_errors_match_the_decoder():
    rng = random.Random(7)
    edge = [b"\x80", b"\xc0\x80", b"\xc1\xbf", b"\xc2", b"\xe0\x80\x80", b"\xe0\x9f\xbf",
            b"\xe0\xa0", b"\xed\xa0\x80", b"\xed\x9f\xbf", b"\xef\xbf\xbf", b"\xf0\x8f\xbf\xbf",
            b"\xf0\x90\x80", b"\xf0\x90\x80A", b"\xf4\x90\x80\x80", b"\xf4\x8f\xbf\xbf",
            b"\xf5\x80\x80\x80", b"\xff", b"a\xe1\x80b", "héllo ✓ 🚀".encode()]
    cases = list(edge)
    alphabet = [0x41, 0x7f, 0x80, 0x8f, 0x90, 0x9f, 0xa0, 0xbf, 0xc0, 0xc2, 0xdf, 0xe0, 0xe1,
                0xed, 0xee, 0xef, 0xf0, 0xf1, 0xf4, 0xf5, 0xff]
    for _ in range(1500):
        cases.append(bytes(rng.choice(alphabet) for _ in range(rng.randint(1, 7))))
    for raw in cases:
        data, _ = write_gguf([("k", STR, raw)], [])
        expect = _python_utf8_message(raw)
        if expect is None:
            assert GgufFile(data=data).metadata["k"].value == raw.decode("utf-8")
        else:
            assert _err(data) == "GGUF string is not UTF-8: " + expect, raw


# ---- a file with every value type, several tensors, unsorted offsets --------

def _everything():
    rng = np.random.default_rng(11)
    q4 = rng.integers(0, 256, 2 * 2 * 144, dtype=np.uint8).tobytes()
    q6 = rng.integers(0, 256, 3 * 210, dtype=np.uint8).tobytes()
    f32 = np.arange(6, dtype=np.float32).tobytes()
    md = [
        ("general.alignment", U64, 64),
        ("u8", U8, 255), ("i8", I8, -128), ("u16", U16, 65535), ("i16", I16, -32768),
        ("u32", U32, 0xffffffff), ("i32", I32, -(1 << 31)), ("f32", F32, -1.5e-7),
        ("bool", BOOL, 2), ("bool0", BOOL, 0), ("s", STR, "Grüße 🚀"), ("empty", STR, ""),
        ("u64", U64, (1 << 64) - 1), ("i64", I64, -(1 << 63)), ("f64", F64, math.pi),
        ("nested", ARR, (ARR, [(STR, ["a", "bc"]), (I16, [-1, 2, -3]), (ARR, [])])),
        ("floats", ARR, (F32, [0.1, float("inf"), -0.0])),
    ]
    tensors = [  # index order differs from offset order
        ("blk.1.ffn_down.weight", [256, 3], Q6K, 768, q6),
        ("blk.0.ffn_up.weight", [512, 2], Q4K, 0, q4),
        ("output_norm.weight", [6], 0, 640, f32),
        ("zz.empty", [0], 1, 704, b""),
    ]
    return md, tensors


def test_round_trip_of_every_value_type():
    md, tensors = _everything()
    data, base = write_gguf(md, tensors, alignment=64)
    g = GgufFile(data=data)
    assert (g.alignment, g.data_base) == (64, base)
    m = g.metadata
    assert sorted(m) == sorted(k for k, _, _ in md)
    assert list(m) == sorted(m, key=lambda k: k.encode())      # byte order, as a BTreeMap
    assert m["u8"] == GgufValue(U8, 255) and m["i8"] == GgufValue(I8, -128)
    assert m["u16"] == GgufValue(U16, 65535) and m["i16"] == GgufValue(I16, -32768)
    assert m["u32"] == GgufValue(U32, 0xffffffff) and m["i32"] == GgufValue(I32, -(1 << 31))
    assert m["f32"] == GgufValue(F32, float(np.float32(-1.5e-7)))
    assert m["bool"] == GgufValue(BOOL, True) and m["bool0"] == GgufValue(BOOL, False)
    assert m["s"] == GgufValue(STR, "Grüße 🚀") and m["empty"] == GgufValue(STR, "")
    assert m["u64"] == GgufValue(U64, (1 << 64) - 1) and m["i64"] == GgufValue(I64, -(1 << 63))
    assert m["f64"] == GgufValue(F64, math.pi)
    assert m["nested"] == GgufValue(ARR, [
        GgufValue(ARR, [GgufValue(STR, "a"), GgufValue(STR, "bc")]),
        GgufValue(ARR, [GgufValue(I16, -1), GgufValue(I16, 2), GgufValue(I16, -3)]),
        GgufValue(ARR, [])])
    fl = m["floats"].value
    assert fl[0] == GgufValue(F32, float(np.float32(0.1)))
    assert fl[1].value == math.inf and math.copysign(1, fl[2].value) < 0
    # the tensor index, in file order, with ranges running to the next offset
    assert [t.name for t in g.tensor_list] == [t[0] for t in tensors]
    ends = {0: base + 640, 640: base + 704, 704: base + 768, 768: len(data)}
    for t, (name, shape, gt, off, payload) in zip(g.tensor_list, tensors):
        assert (t.shape, t.ggml_type, t.offset) == (tuple(shape), gt, off)
        assert (t.data_start, t.data_end) == (base + off, ends[off])
        _, got = g.tensor(name)
        assert got.tobytes()[:len(payload)] == payload
        assert set(got.tobytes()[len(payload):]) <= {0}
    assert g.expected_payload_bytes("blk.0.ffn_up.weight") == 2 * 2 * 144
    assert g.expected_payload_bytes("blk.1.ffn_down.weight") == 3 * 210
    assert g.expected_payload_bytes("output_norm.weight") == 24
    assert g.expected_payload_bytes("zz.empty") == 0
    assert g.element_count("blk.0.ffn_up.weight") == 1024


def test_open_maps_the_same_store(tmp_path):
    md, tensors = _everything()
    data, _ = write_gguf(md, tensors, alignment=64)
    p = tmp_path / "m.gguf"
    p.write_bytes(data)
    a, b = GgufFile(path=p), GgufFile(data=data)
    assert a.metadata == b.metadata
    for ta, tb in zip(a.tensor_list, b.tensor_list):
        assert (ta.name, ta.shape, ta.ggml_type, ta.data_start, ta.data_end) == \
               (tb.name, tb.shape, tb.ggml_type, tb.data_start, tb.data_end)
        assert a.tensor(ta.name)[1].tobytes() == b.tensor(tb.name)[1].tobytes()
    assert a.inspect("m") == b.inspect("m")
    missing = tmp_path / "missing.gguf"
    with pytest.raises(HipError) as e:
        GgufFile(path=missing)
    assert str(e.value).endswith(f"open GGUF model {missing}: No such file or directory "
                                 "(os error 2)")
    empty = tmp_path / "empty.gguf"
    empty.write_bytes(b"")
    with pytest.raises(HipError, match="GGUF header is truncated"):
        GgufFile(path=empty)


def test_duplicate_tensor_names_resolve_to_the_last():
    data, base = write_gguf([], [("w", [4], 0, 0, b"\x01" * 16), ("w", [8], 0, 32, b"\x02" * 32)])
    g = GgufFile(data=data)
    assert len(g.tensor_list) == 2 and len(g.tensors) == 1
    info, got = g.tensor("w")
    assert info.shape == (8,) and got.tobytes() == b"\x02" * 32


def test_equal_offsets_give_an_empty_first_range():
    data, base = write_gguf([], [("a", [4], 0, 0, bytes(16)), ("b", [4], 0, 0, bytes(16))])
    g = GgufFile(data=data)
    a, b = g.tensor_list
    assert (a.data_start, a.data_end) == (base, base)          # stable order: a, then b
    assert (b.data_start, b.data_end) == (base, len(data))


def test_lookup_and_payload_errors():
    big = [(1 << 32), (1 << 32)]
    data, _ = write_gguf([], [
        ("q", [100], Q4K, 0, bytes(64)),
        ("q5", [257], Q5K, 64, bytes(64)),
        ("q6", [255, 3], Q6K, 128, bytes(64)),
        ("huge", big + [1 << 2], 0, 192, bytes(16)),
        ("q4_0", [32], 2, 224, bytes(18)),
    ])
    g = GgufFile(data=data)
    with pytest.raises(HipError, match="unknown GGUF tensor nope$"):
        g.tensor("nope")
    with pytest.raises(HipError, match="GGUF Q4_K tensor q has 100 elements; expected a multiple "
                                       "of 256"):
        g.expected_payload_bytes("q")
    with pytest.raises(HipError, match="GGUF Q5_K tensor q5 has 257 elements"):
        g.expected_payload_bytes("q5")
    with pytest.raises(HipError, match="GGUF Q6_K tensor q6 has 765 elements"):
        g.expected_payload_bytes("q6")
    with pytest.raises(HipError, match="GGUF tensor huge element count overflows"):
        g.element_count("huge")
    assert g.tensors["huge"].element_count() is None
    assert g.expected_payload_bytes("q4_0") is None
    # F32 whose byte count overflows: unknown, not an error
    data, _ = write_gguf([], [("f", [1 << 31, 1 << 31, 2], 0, 0, bytes(8))])
    assert GgufFile(data=data).expected_payload_bytes("f") is None
    with pytest.raises(HipError, match="GGUF metadata is missing general.name"):
        v = si_hip.GgufValueC()
        si_hip._check(si_hip.lib().si_hip_gguf_metadata_get(g.handle, b"general.name",
                                                            si_hip.C.byref(v)))


def test_upload_checks_fire_before_the_device():
    """Type and length checks of a store upload (src/model.rs:790-850)
    reject before any device call, so a null context is enough."""
    C = si_hip.C
    q4 = bytes(2 * 144)
    data, _ = write_gguf([], [("f", [4], 0, 0, bytes(16)), ("short", [512], Q4K, 32, q4[:200]),
                              ("bad", [100], Q4K, 256, bytes(144))])
    g = GgufFile(data=data)
    w = C.c_void_p()
    for name, msg in [("f", "GGUF tensor f has type 0; expected 12, 13 or 14"),
                      ("short", "GGUF tensor short has 224 bytes; expected at least 288"),
                      ("bad", "GGUF Q4_K tensor bad has 100 elements; expected a multiple of "
                              "256")]:
        for fn in (si_hip.lib().si_hip_gguf_upload_tensor,
                   si_hip.lib().si_hip_gguf_bind_tensor_mapped):
            rc = fn(None, g.handle, g._index(name), C.byref(w))
            assert rc < 0 and si_hip.last_error() == msg
            assert w.value is None


def test_inspect_lists_like_the_reference_tool():
    md, tensors = _everything()
    tensors = tensors + [("output.weight", [256, 4], Q6K, 1408, bytes(4 * 210)),
                         ("token_embd.weight", [256, 4], Q4K, 2304, bytes(4 * 144))]
    md = md + [("long", STR, "x" * 170)]
    data, base = write_gguf(md, tensors, alignment=64)
    g = GgufFile(data=data)
    lines = g.inspect("m.gguf").splitlines()
    assert lines[:3] == ["model=m.gguf", "tensors=6",
                         "q4_k_tensor=blk.0.ffn_up.weight shape=[512, 2] bytes=640 elements=1024"]
    assert lines[3].startswith("q4_k_tensor=token_embd.weight shape=[256, 4] bytes=")
    assert lines[4] == "tensor_type_counts={0: 1, 1: 1, 12: 2, 14: 2}"
    assert lines[5].startswith("special_tensor=token_embd.weight type=12 shape=[256, 4] bytes=")
    assert lines[6] == "special_tensor=output.weight type=14 shape=[256, 4] bytes=896"
    assert lines[7] == "special_tensor=output_norm.weight type=0 shape=[6] bytes=64"
    assert [ln.split(" ")[0] for ln in lines[8:12]] == [
        "non_q4_tensor=blk.1.ffn_down.weight", "non_q4_tensor=output.weight",
        "non_q4_tensor=output_norm.weight", "non_q4_tensor=zz.empty"]
    meta = dict(ln[len("metadata."):].split("=", 1) for ln in lines[12:])
    assert meta["u8"] == "U8(255)" and meta["i8"] == "I8(-128)"
    assert meta["f32"] == "F32(-1.5e-7)" and meta["f64"] == "F64(3.141592653589793)"
    assert meta["bool"] == "Bool(true)"
    assert meta["s"] == 'string("Grüße 🚀")'
    assert meta["long"] == 'string(len=170, prefix="' + "x" * 160 + '")'
    assert meta["nested"] == ('array(len=3, first=[array(len=2, first=[string("a"), '
                              'string("bc")]), array(len=3, first=[I16(-1), I16(2), I16(-3)]), '
                              'array(len=0, first=[])])')
    assert meta["floats"] == "array(len=3, first=[F32(0.1), F32(inf), F32(-0.0)])"
    assert meta["general.alignment"] == "U64(64)"


# ---- uploads to HBM -----------------------------------------------------------

def _kquant_file(seed=5):
    rows, cols = 96, 1024
    q4 = si_hip.synth_matrix(Q4K, seed, rows, cols)
    q5 = si_hip.synth_matrix(Q5K, seed + 1, rows, cols)
    q6 = si_hip.synth_matrix(Q6K, seed + 2, rows, cols)
    off5 = -(-q4.size // 32) * 32 + 32
    off6 = -(-(off5 + q5.size) // 32) * 32
    data, _ = write_gguf([("general.architecture", STR, "qwen35")], [
        ("q6", [cols, rows], Q6K, off6, q6.tobytes()),
        ("q4", [cols, rows], Q4K, 0, q4.tobytes()),
        ("q5", [cols, rows], Q5K, off5, q5.tobytes()),
    ], data_tail=bytes(48))
    return rows, cols, {"q4": q4, "q5": q5, "q6": q6}, data


@pytest.mark.gpu
@pytest.mark.parametrize("mapped", [False, True])
def test_store_upload_matches_direct_upload(hip_ctx, tmp_path, mapped):
    rows, cols, mats, data = _kquant_file()
    p = tmp_path / "k.gguf"
    p.write_bytes(data)
    g = GgufFile(path=p)
    x = si_hip.synth_normal(3, cols)
    types = {"q4": Q4K, "q5": Q5K, "q6": Q6K}
    for name, raw in mats.items():
        w = g.upload(hip_ctx, name, mapped=mapped)
        assert w.byte_len() == raw.size and w.ggml_type() == types[name]
        assert w.is_mapped() == mapped
        ref = hip_ctx.upload_quant_weight_private(raw, types[name])
        y = hip_ctx.gguf_quant_matvec_weight(w, rows, cols, x)
        y_ref = hip_ctx.gguf_quant_matvec_weight(ref, rows, cols, x)
        assert np.array_equal(y.view(np.uint32), y_ref.view(np.uint32)), name
        w.free()
        ref.free()
    g.close()


def test_store_quant_group_rejections(tmp_path):
    """gguf_quant_matvec_many_tensors's checks (metal.rs:4537-4576), before any
    device work (a null context)."""
    rows, cols, mats, data = _kquant_file()
    p = tmp_path / "k.gguf"
    p.write_bytes(data)
    g = GgufFile(path=p)

    class NoCtx:
        handle = None

    with pytest.raises(si_hip.HipError) as e:
        g.quant_matvec_many(NoCtx(), ["q4", "q5"], np.zeros(cols + 1, np.float32))
    assert e.value.message == "quantized matvec group input length is invalid"
    with pytest.raises(si_hip.HipError) as e:
        g.quant_matvec_many(NoCtx(), [], np.zeros(cols, np.float32))
    assert e.value.message == "quantized matvec group requires at least one tensor"
    g.close()


def test_store_tensor_rows_rejections():
    """q4_k_matvec_tensor_rows / quant_k_matvec_tensor_rows checks
    (metal.rs:4353-4376, 4407-4430), before any device work."""
    rows, cols, mats, data = _kquant_file()
    g = GgufFile(data=data)

    class NoCtx:
        handle = None

    for name, label in (("q4", "Q4_K"), ("q5", "Q5_K"), ("q6", "Q6_K")):
        for start, count in ((0, 0), (rows, 1), (rows - 1, 2)):
            with pytest.raises(si_hip.HipError) as e:
                g.matvec_tensor_rows(NoCtx(), name, start, count, np.zeros(cols, np.float32))
            assert e.value.message == f"{label} row range is invalid"
        with pytest.raises(si_hip.HipError) as e:
            g.matvec_tensor_rows(NoCtx(), name, 0, 1, np.zeros(cols - 1, np.float32))
        assert e.value.message == f"{label} tensor columns or input length is invalid"
    g.close()


@pytest.mark.gpu
def test_store_tensor_rows_match_the_oracle(hip_ctx):
    """gguf_matvec_tensor_rows over row ranges of the store's Q4_K, Q5_K and
    Q6_K tensors: within the oracle's bound over the same rows."""
    import oracle_lib as O
    rows, cols, mats, data = _kquant_file(11)
    g = GgufFile(data=data)
    x = si_hip.synth_normal(12, cols)
    types = {"q4": Q4K, "q5": Q5K, "q6": Q6K}
    rb = {Q4K: 144, Q5K: 176, Q6K: 210}
    for name, (start, count) in (("q4", (5, 37)), ("q5", (0, rows)), ("q6", (rows - 3, 3))):
        t = types[name]
        y = g.matvec_tensor_rows(hip_ctx, name, start, count, x)
        b = cols // 256 * rb[t]
        part = mats[name][start * b:(start + count) * b]
        _, y64, ab = O.matvec(t, part, count, cols, x)
        err = np.max(np.abs(y.astype(np.float64) - y64) / (2e-5 * ab + 1e-30))
        assert err <= 1.0, (name, err)
    g.close()


@pytest.mark.gpu
def test_store_quant_group_matches_single_calls(hip_ctx, tmp_path):
    """gguf_quant_matvec_many_tensors over the store's Q4_K, Q5_K and Q6_K
    tensors, and gguf_quant_matvec_many_bytes over the same bytes (an
    all-Q4_K group runs as one launch): each output within the oracle's
    bound, and both entry points bit-identical."""
    import oracle_lib as O
    rows, cols, mats, data = _kquant_file()
    p = tmp_path / "k.gguf"
    p.write_bytes(data)
    g = GgufFile(path=p)
    x = si_hip.synth_normal(9, cols)
    types = {"q4": Q4K, "q5": Q5K, "q6": Q6K}
    for names in (["q4", "q5", "q6"], ["q4", "q4", "q4"], ["q6", "q6"]):
        outs = g.quant_matvec_many(hip_ctx, names, x)
        again = hip_ctx.gguf_quant_matvec_many_bytes(
            [(types[n], mats[n], rows, cols) for n in names], x)
        for n, y, y2 in zip(names, outs, again):
            _, y64, ab = O.matvec(types[n], mats[n], rows, cols, x)
            err = np.max(np.abs(y.astype(np.float64) - y64) / (2e-5 * ab + 1e-30))
            assert err <= 1.0, (names, n, err)
            assert np.array_equal(y.view(np.uint32), y2.view(np.uint32))
    g.close()


@pytest.mark.gpu
def test_store_embedding_rows_are_the_packed_rows(hip_ctx):
    import oracle_lib
    rows, cols, mats, data = _kquant_file(9)
    g = GgufFile(data=data)
    table = g.upload(hip_ctx, "q4")
    for token in (0, 1, rows - 1):
        got = hip_ctx.q4_k_embedding_tensor(table, (cols, rows), token)
        row_bytes = mats["q4"][token * (cols // 256) * 144:(token + 1) * (cols // 256) * 144]
        want = oracle_lib.dequantize(Q4K, row_bytes, cols)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    table.free()


# ---- the inspect command ------------------------------------------------------

def _run_inspect(*args):
    import os
    import subprocess
    import sys
    pkg = str(Path(__file__).resolve().parent.parent / "memory-aware-inference_amd")
    env = dict(os.environ, PYTHONPATH=pkg + os.pathsep + os.environ.get("PYTHONPATH", ""))
    return subprocess.run([sys.executable, "-m", "si_hip.gguf_inspect", *args],
                          capture_output=True, text=True, env=env, timeout=120)


def test_inspect_command(tmp_path):
    r = _run_inspect("--model", str(TINY))
    assert r.returncode == 0 and r.stderr == ""
    assert r.stdout.splitlines()[0] == f"model={TINY}"
    assert r.stdout.splitlines()[1:] == GgufFile(path=TINY).inspect("x").splitlines()[1:]
    for bad in ([], ["--model"], ["--mode", "x"], ["--model", str(TINY), "extra"]):
        r = _run_inspect(*bad)
        assert (r.returncode, r.stdout, r.stderr) == (2, "", "Usage: si-gguf-inspect --model PATH\n")
    nope = tmp_path / "nope.gguf"
    nope.write_bytes(b"NOPE")
    r = _run_inspect("--model", str(nope))
    assert (r.returncode, r.stdout, r.stderr) == (1, "", "error: GGUF header has invalid magic\n")


# ---- a real model file, when SI_GGUF_MODEL names one --------------------------
# The reference runs these only when the variable is set (src/model.rs:2184-2245,
# src/metal.rs:7605-7768); no model file ships with this repository.

def _real_store():
    import os
    path = os.environ.get("SI_GGUF_MODEL")
    if not path:
        pytest.skip("SI_GGUF_MODEL is not set")
    return GgufFile(path=path)


def test_opens_real_gguf_when_si_gguf_model_is_set():
    import oracle_lib
    g = _real_store()
    assert g.metadata["general.architecture"] == GgufValue(STR, "qwen35")
    assert g.tensor_list
    assert "output.weight" in g.tensors or "token_embd.weight" in g.tensors
    for gt in (Q4K, Q5K, Q6K):
        info = next(t for t in g.tensors.values() if t.ggml_type == gt)
        _, raw = g.tensor(info.name)
        assert np.isfinite(oracle_lib.dequantize(gt, raw[:BLOCK_BYTES[gt]], 256)).all()


@pytest.mark.gpu
@pytest.mark.parametrize("gt,period,shift,div", [(Q4K, 17, 8.0, 7.0), (Q5K, 19, 9.0, 8.0),
                                                  (Q6K, 19, 9.0, 8.0)])
def test_matvec_against_real_gguf_row(hip_ctx, gt, period, shift, div):
    """q4_k_matvec_runs_against_real_gguf_row / q5_and_q6_k_matvec_run_against_
    real_gguf_rows (src/metal.rs:7605-7703): row 0 of the first rank-2 tensor
    of the type, x[i] = ((i % p) - s) / d, within 1e-2 of the decoded row's
    sequential f32 dot -- and within the 2e-5 * sum|w*x| bound of its f64 dot."""
    import oracle_lib
    g = _real_store()
    info = next(t for t in g.tensors.values() if t.ggml_type == gt and len(t.shape) == 2)
    cols = info.shape[0]
    assert cols % 256 == 0
    x = ((np.arange(cols) % period).astype(np.float32) - np.float32(shift)) / np.float32(div)
    _, raw = g.tensor(info.name)
    row = raw[:cols // 256 * BLOCK_BYTES[gt]]
    w = oracle_lib.dequantize(gt, row, cols)
    seq = np.float32(0)
    for a, b in zip(w, x):
        seq = np.float32(seq + np.float32(a * b))
    exact = float(np.dot(w.astype(np.float64), x.astype(np.float64)))
    bound = 2e-5 * float(np.abs(w.astype(np.float64) * x).sum())
    weight = g.upload(hip_ctx, info.name)
    y = hip_ctx.gguf_quant_matvec_tensor_rows(weight, info.shape, 0, 1, x)[0]
    assert abs(y - seq) < 1e-2
    assert abs(y - exact) <= bound
    weight.free()


@pytest.mark.gpu
def test_embedding_against_real_gguf_token(hip_ctx):
    """q4_k_embedding_runs_against_real_gguf_token (src/metal.rs:7733-7768),
    held to bit equality with the decoded row."""
    import oracle_lib
    g = _real_store()
    info = g.tensors["token_embd.weight"]
    assert info.ggml_type == Q4K
    cols = info.shape[0]
    _, raw = g.tensor(info.name)
    want = oracle_lib.dequantize(Q4K, raw[:cols // 256 * 144], cols)
    table = g.upload(hip_ctx, info.name)
    got = hip_ctx.q4_k_embedding_tensor(table, info.shape, 0)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    table.free()
