"""Writes tests/golden/matmul_fixtures/: a small synthetic GGUF holding two
IQ4_XS projection tensors, and matmul cases cut from it in the reference's
fixture format (tools/dump_matmul_fixtures.py:183-247: W.bin, x/X.bin,
y_ref/Y_ref.bin, manifest_matmul.json), through this package's GGUF reader
and extraction rules.  Weights follow the seeded generator of the oracle
(d ~ U(0.005, 0.02), 6-bit scales and 4-bit codes uniform); activations are
N(0, 1) from numpy's default_rng(42) as in the reference; y_ref is the
float32 product of the dequantised weights and the raw activations, as the
reference computes it.  The reference's model file is not available here, so
these are not real-weight statistics.

    python tests/golden/make_matmul_fixtures.py
"""
import json
import os
import struct
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from __graft_entry__ import load_package  # noqa: E402
from oracle.oracle import Oracle  # noqa: E402

OUT = os.path.join(HERE, "matmul_fixtures")
TENSORS = [("blk.0.attn_q.weight", 1024, 96, 11), ("blk.0.ffn_down.weight", 2048, 64, 12)]  # name, K_t, N_t, seed
CASES = [("attn_q", "blk.0.attn_q.weight", 1024, 64), ("ffn_down", "blk.0.ffn_down.weight", 1536, 48)]
MS = (1, 16)
SEED = 42


def gguf_bytes(tensors, alignment=32) -> bytes:
    def s(x):
        b = x.encode()
        return struct.pack("<Q", len(b)) + b
    kvs = [s("general.architecture") + struct.pack("<I", 8) + s("qwen35"),
           s("general.file_type") + struct.pack("<I", 4) + struct.pack("<I", 30),
           s("general.alignment") + struct.pack("<I", 4) + struct.pack("<I", alignment)]
    infos, blobs, off = [], [], 0
    for name, K, N, W in tensors:
        off = (off + alignment - 1) // alignment * alignment
        infos.append(s(name) + struct.pack("<I", 2) + struct.pack("<QQ", K, N) + struct.pack("<IQ", 23, off))
        blobs.append((off, W.tobytes()))
        off += W.nbytes
    head = b"GGUF" + struct.pack("<IQQ", 3, len(tensors), len(kvs)) + b"".join(kvs) + b"".join(infos)
    start = (len(head) + alignment - 1) // alignment * alignment
    out = bytearray(head + bytes(start - len(head)))
    for o, b in blobs:
        out += bytes(start + o - len(out)) + b
    return bytes(out)


def main() -> None:
    os.makedirs(OUT, exist_ok=True)
    orc = Oracle()
    pkg = load_package()
    import importlib
    gg = importlib.import_module(pkg.__name__ + ".gguf")
    fx = importlib.import_module(pkg.__name__ + ".fixtures")
    mats = [(n, K, N, orc.gen_weights(K, N, seed=sd)) for n, K, N, sd in TENSORS]
    gpath = os.path.join(OUT, "synthetic_layer.gguf")
    with open(gpath, "wb") as f:
        f.write(gguf_bytes(mats))
    rng = np.random.default_rng(SEED)
    entries = []
    with gg.GGUFReader(gpath) as r:
        for name, tname, K, N in CASES:
            W = fx.extract_projection(r, tname, K, N)
            prefix = f"matmul_{name}_{K}x{N}"
            W.tofile(os.path.join(OUT, prefix + "_W.bin"))
            Wf = orc.dequant(W, K, N).astype(np.float32)
            for M in MS:
                X = rng.standard_normal(size=(K, M)).astype(np.float32)
                Y = (Wf @ X).astype(np.float32)
                e = fx.matmul_entry(name, K, N, M, W, tname, SEED, prefix)
                if M == 1:
                    X[:, 0].tofile(os.path.join(OUT, e["x_bin"]))
                    Y[:, 0].tofile(os.path.join(OUT, e["y_ref_bin"]))
                else:
                    X.tofile(os.path.join(OUT, e["X_bin"]))
                    Y.tofile(os.path.join(OUT, e["Y_ref_bin"]))
                entries.append(e)
    with open(os.path.join(OUT, "manifest_matmul.json"), "w", encoding="utf-8") as f:
        json.dump(entries, f, indent=2)
    print(f"wrote {len(entries)} cases to {OUT}")


if __name__ == "__main__":
    main()
