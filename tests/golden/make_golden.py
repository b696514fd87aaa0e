"""Write the committed fixtures under tests/golden/.

  quant_kats.json     the four known-answer tests of src/quant.rs:209-280,
                      as block bytes plus the values those tests assert, and
                      the byte-length rejection cases of quant.rs:233-238.
  blocks_q{4,5,6}_k.json
                      random and edge-case blocks with their expected f32
                      bit patterns from tests/numpy_ref.py, checked here
                      against the C oracle before they are written.

Run from the repository root: python tests/golden/make_golden.py
"""
from __future__ import annotations

import json
import struct
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
REPO = HERE.parent.parent
sys.path.insert(0, str(REPO / "tests"))
sys.path.insert(0, str(REPO / "memory-aware-inference_amd"))

import numpy_ref  # noqa: E402
import oracle_lib  # noqa: E402
import si_hip  # noqa: E402

ONE = struct.pack("<H", 0x3C00)


def kats() -> dict:
    # quant.rs:213-231
    q4 = bytearray(144)
    q4[0:2] = ONE
    q4[4:16] = bytes([1] * 12)
    q4[16:] = bytes([0x10] * 128)
    q4_expect = ([0.0] * 32 + [1.0] * 32) * 4
    # quant.rs:240-259
    q5 = bytearray(176)
    q5[0:2] = ONE
    q5[4:16] = bytes([1] * 12)
    q5[48:] = bytes([0x10] * 128)
    q5[16:48] = bytes([0xFF] * 32)
    q5_expect = ([16.0] * 32 + [17.0] * 32) * 4
    # quant.rs:261-280
    q6 = bytearray(210)
    q6[208:210] = ONE
    q6[:128] = bytes([0x21] * 128)
    q6[128:192] = bytes([0xE4] * 64)
    q6[192:208] = bytes([1] * 16)
    q6_expect = ([-31.0] * 32 + [-15.0] * 32 + [2.0] * 32 + [18.0] * 32) * 2
    return {
        "source": "super-inference src/quant.rs:209-280",
        "kats": [
            {"name": "decodes_one_q4_k_block", "ggml_type": 12, "elements": 256,
             "bytes": q4.hex(), "expected": q4_expect},
            {"name": "decodes_one_q5_k_block_with_high_bits", "ggml_type": 13, "elements": 256,
             "bytes": q5.hex(), "expected": q5_expect},
            {"name": "decodes_one_q6_k_block_with_high_bits_and_scales", "ggml_type": 14,
             "elements": 256, "bytes": q6.hex(), "expected": q6_expect},
        ],
        # rejects_q4_k_shape_and_byte_mismatches (quant.rs:233-238)
        "rejections": [
            {"ggml_type": 12, "byte_len": 144, "elements": 255},
            {"ggml_type": 12, "byte_len": 143, "elements": 256},
            {"ggml_type": 12, "byte_len": 145, "elements": 256},
        ],
    }


def edge_blocks(ggml_type: int, rng: np.random.Generator) -> list[bytes]:
    bb = numpy_ref.BLOCK[ggml_type]
    halves = [0x0001, 0x03FF, 0x0400, 0x8001, 0x7BFF, 0xFBFF, 0x0000, 0x8000, 0x7C00, 0xFC00,
              0x7E00, 0x7C01, 0x3555, 0x1234]
    out = []
    for h in halves:
        b = bytearray(rng.integers(0, 256, bb, dtype=np.uint8).tobytes())
        if ggml_type == 14:
            b[208:210] = struct.pack("<H", h)
        else:
            b[0:2] = struct.pack("<H", h)
            b[2:4] = struct.pack("<H", halves[(halves.index(h) + 3) % len(halves)])
        out.append(bytes(b))
    # all-ones / all-zeros bytes
    out.append(bytes([0xFF] * bb))
    out.append(bytes([0x00] * bb))
    return out


def same_bits(a: np.ndarray, b: np.ndarray) -> bool:
    nan = np.isnan(a) & np.isnan(b)
    return bool(np.all(nan | (a.view(np.uint32) == b.view(np.uint32))))


def block_fixture(ggml_type: int) -> dict:
    rng = np.random.default_rng(1000 + ggml_type)
    rand = si_hip.synth_blocks(ggml_type, seed=4242 + ggml_type, n_blocks=16).tobytes()
    bb = numpy_ref.BLOCK[ggml_type]
    blocks = [rand[i * bb:(i + 1) * bb] for i in range(16)] + edge_blocks(ggml_type, rng)
    data = b"".join(blocks)
    expect = numpy_ref.dequant(ggml_type, data)
    oracle = oracle_lib.dequantize(ggml_type, data, len(blocks) * 256)
    if not same_bits(expect, oracle):
        raise SystemExit(f"numpy and C restatements disagree for type {ggml_type}")
    return {
        "ggml_type": ggml_type,
        "n_blocks": len(blocks),
        "bytes": data.hex(),
        "expected_bits": expect.view(np.uint32).tolist(),
        "note": "expected from tests/numpy_ref.py, equal to the C oracle (NaN-aware)",
    }


def main() -> None:
    (HERE / "quant_kats.json").write_text(json.dumps(kats(), indent=1) + "\n")
    for t, name in ((12, "q4_k"), (13, "q5_k"), (14, "q6_k")):
        (HERE / f"blocks_{name}.json").write_text(json.dumps(block_fixture(t)) + "\n")
    print("fixtures written to", HERE)


if __name__ == "__main__":
    main()
