"""Write tests/golden/tiny_qwen35.gguf: the GGUF file the reference's model
tests build in memory (tiny_gguf_fixture, src/model.rs:1981-2008), byte for
byte -- GGUF v3, two metadata entries (general.architecture = String
"qwen35", general.alignment = U32 32), one tensor "blk.0.attn_q.weight" of
shape [4, 2], ggml type 0, offset 0, the index padded with zeros to a
multiple of 32, then the eight data bytes 1..8.

The reference's tests assert (src/model.rs:1913-1979): the two metadata
values, one tensor with that name, shape and type, data_start % 32 == 0,
and that b"NOPE" and the first 20 bytes of this file are both rejected.

Run from the repository root: python tests/golden/make_gguf_fixture.py
"""
from __future__ import annotations

import struct
from pathlib import Path

OUT = Path(__file__).resolve().parent / "tiny_qwen35.gguf"


def gguf_string(value: str) -> bytes:
    raw = value.encode("utf-8")
    return struct.pack("<Q", len(raw)) + raw


def tiny_fixture() -> bytes:
    b = bytearray(b"GGUF")
    b += struct.pack("<IQQ", 3, 1, 2)          # version, tensor count, metadata count
    b += gguf_string("general.architecture") + struct.pack("<I", 8) + gguf_string("qwen35")
    b += gguf_string("general.alignment") + struct.pack("<II", 4, 32)
    b += gguf_string("blk.0.attn_q.weight") + struct.pack("<IQQ", 2, 4, 2)
    b += struct.pack("<IQ", 0, 0)              # ggml type, offset
    b += bytes(-len(b) % 32)
    b += bytes(range(1, 9))
    return bytes(b)


if __name__ == "__main__":
    data = tiny_fixture()
    OUT.write_bytes(data)
    print(f"wrote {OUT} ({len(data)} bytes)")
