"""Writes tests/golden/iq4xs_kat_blocks.json: the five synthetic IQ4_XS
known-answer blocks whose raw_sha256 the reference records in
kernels/fixtures/manifest.json:3-81 (recipe: tools/dump_gguf_fixtures.py:50-136,
restated here from its description: d, scales_h, scales_l, qs per case).

The block bytes are built independently of the oracle library, hashed, and
checked against the manifest's values when the reference is mounted; the
fixture records bytes, hashes and hand-derived dequantised values.
Run: python tests/golden/make_kat_fixtures.py
"""
import hashlib
import json
import os
import struct

import numpy as np

MANIFEST = "/root/reference/kernels/fixtures/manifest.json"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "iq4xs_kat_blocks.json")


def block(d: float, scales_h: int, scales_l: bytes, qs: bytes) -> bytes:
    assert len(scales_l) == 4 and len(qs) == 128
    return np.float16(d).tobytes() + struct.pack("<H", scales_h) + scales_l + qs


def cases() -> dict:
    ramp = bytes([(i & 0xF) | (((15 - i) & 0xF) << 4) for i in range(128)])
    split = bytes([((2 * s + 1) % 16) | (((2 * s + 2) % 16) << 4) for s in range(8) for _ in range(16)])
    iso_qs = bytearray(128)
    iso_qs[48:64] = bytes([0x79] * 16)
    return {
        "synthetic_zero": [block(0.0, 0, bytes(4), bytes(128))],
        "synthetic_max_scale": [block(0.5, 0xFFFF, bytes([0xFF] * 4), ramp),
                                block(0.5, 0x0000, bytes(4), ramp)],
        "synthetic_split_half": [block(1.25, 0b1110010011100100, bytes([0x21, 0x43, 0x65, 0x87]), split)],
        "synthetic_nibble_extremes": [block(1.0, 0x5555, bytes([0x33] * 4), bytes(128)),
                                      block(1.0, 0x5555, bytes([0x33] * 4), bytes([0xFF] * 128)),
                                      block(1.0, 0x5555, bytes([0x33] * 4),
                                            bytes([0x0F if i % 2 == 0 else 0xF0 for i in range(128)]))],
        "synthetic_subblock_isolated": [block(2.0, 0b0000000010000000, bytes([0, 0x50, 0, 0]), bytes(iso_qs))],
    }


# Hand-derived dequantised weights (value = d * (ls - 32) * kvalues[nibble]),
# listed as (block, element, value).  ls = (scales_l nibble) | (scales_h bits << 4).
HAND_VALUES = {
    "synthetic_zero": [(0, 0, 0.0), (0, 255, 0.0)],
    # ls = 63 -> +31; block 0 qs[0] = 0xF0: lo nibble 0 (kv -127) at element 0,
    # hi nibble 15 (kv 113) at element 16.  Block 1: ls = 0 -> -32.
    "synthetic_max_scale": [(0, 0, 0.5 * 31 * -127), (0, 16, 0.5 * 31 * 113),
                            (1, 0, 0.5 * -32 * -127), (1, 16, 0.5 * -32 * 113)],
    # sub-block 0: ls = 0x1 | (0 << 4) = 1 -> -31; nibbles lo 1 (kv -104), hi 2 (kv -83).
    # sub-block 3: ls = 0x4 | (3 << 4) = 52 -> +20; nibbles lo 7 (kv -10), hi 8 (kv 1).
    "synthetic_split_half": [(0, 0, 1.25 * -31 * -104), (0, 16, 1.25 * -31 * -83),
                             (0, 96, 1.25 * 20 * -10), (0, 112, 1.25 * 20 * 1)],
    # ls = 3 | (1 << 4) = 19 -> -13 for every sub-block.
    "synthetic_nibble_extremes": [(0, 0, -13 * -127.0), (1, 0, -13 * 113.0),
                                  (2, 0, -13 * 113.0), (2, 16, -13 * -127.0),
                                  (2, 1, -13 * -127.0), (2, 17, -13 * 113.0)],
    # sub-block 3: ls = 5 | (2 << 4) = 37 -> +5; qs 0x79: lo 9 (kv 13), hi 7 (kv -10).
    # The other sub-blocks are NOT zero: scale bits 0 mean ls - 32 = -32 and
    # code 0 means kvalue -127, so each of their weights is 2 * -32 * -127.
    "synthetic_subblock_isolated": [(0, 96, 2.0 * 5 * 13), (0, 112, 2.0 * 5 * -10),
                                    (0, 0, 2.0 * -32 * -127), (0, 128, 2.0 * -32 * -127)],
}


def main() -> None:
    manifest = {}
    if os.path.exists(MANIFEST):
        with open(MANIFEST) as f:
            manifest = {e["name"]: e["raw_sha256"] for e in json.load(f) if e.get("synthetic")}
    out = []
    for name, blocks in cases().items():
        raw = b"".join(blocks)
        sha = hashlib.sha256(raw).hexdigest()
        if manifest:
            assert manifest[name] == sha, (name, sha, manifest[name])
        out.append({"name": name, "n_blocks": len(blocks), "raw_hex": raw.hex(),
                    "raw_sha256_reference": manifest.get(name, sha),
                    "hand_values": [list(v) for v in HAND_VALUES[name]]})
    with open(OUT, "w") as f:
        json.dump({"source": "kernels/fixtures/manifest.json:3-81", "cases": out}, f, indent=1)
    print(f"wrote {OUT}: {len(out)} cases, sha256 {'verified against manifest' if manifest else 'NOT verified'}")


if __name__ == "__main__":
    main()
