"""Writes tests/golden/known_answers.json: the known-answer vectors that the
reference's own tests hold for the GGUF dequant path, re-encoded as GGUF
block streams.

Sources (asqrzk/CombsEngine):
  q8_0_gguf_roundtrip  engine/core/combs-formats/tests/gguf.rs:75-81, 113-120
                       16 Q8_0 blocks, d = 0.5 (f16 0x3800), bytes alternating
                       2 / 254 (= -2 as i8)  ->  values +1.0 / -1.0.
  q4_0_reference_block engine/core/combs-core/src/quant.rs:81-111
                       packed bytes (i*37 + 11) % 256, i < 64 (2 rows x 2
                       groups x 16 bytes), scales [0.5, -1.25, 2.0, 0.75]
                       (all exact in f16); expected value j of a group is
                       ((byte[j] & 15) - 8) * scale, value j+16 is
                       ((byte[j] >> 4) - 8) * scale (reference_block).
  q4_0_all_eights      quant.rs:122-133: bytes 0x88, scale 3.5 -> 32 zeros.

No value here is produced by this repository's oracle; they come from the
constants and formulas written in those tests.
"""
import json
import os
import struct

HERE = os.path.dirname(os.path.abspath(__file__))


def f16_bits(v):
    return struct.unpack("<H", struct.pack("<e", v))[0]


def main():
    out = {}
    # gguf.rs:113-120
    blk = struct.pack("<H", f16_bits(0.5)) + bytes(2 if j % 2 == 0 else 254 for j in range(32))
    out["q8_0_gguf_roundtrip"] = {
        "format": 8, "hex": (blk * 16).hex(), "n": 512,
        "expect": [1.0 if j % 2 == 0 else -1.0 for j in range(32)] * 16,
    }
    # quant.rs:81-111
    packed = [(i * 37 + 11) % 256 for i in range(64)]
    scales = [0.5, -1.25, 2.0, 0.75]
    stream, expect = b"", []
    for row in range(2):
        for g in range(2):
            bs = packed[row * 32 + g * 16: row * 32 + g * 16 + 16]
            sc = scales[row * 2 + g]
            stream += struct.pack("<H", f16_bits(sc)) + bytes(bs)
            vals = [0.0] * 32
            for j in range(16):
                vals[j] = ((bs[j] & 0x0F) - 8.0) * sc
                vals[j + 16] = ((bs[j] >> 4) - 8.0) * sc
            expect += vals
    out["q4_0_reference_block"] = {"format": 2, "hex": stream.hex(), "n": 128, "expect": expect}
    # quant.rs:122-133
    blk = struct.pack("<H", f16_bits(3.5)) + bytes([0x88] * 16)
    out["q4_0_all_eights"] = {"format": 2, "hex": blk.hex(), "n": 32, "expect": [0.0] * 32}
    with open(os.path.join(HERE, "known_answers.json"), "w") as f:
        json.dump(out, f, indent=1)


if __name__ == "__main__":
    main()
