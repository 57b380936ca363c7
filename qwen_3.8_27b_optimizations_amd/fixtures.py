"""Matmul fixtures in the reference's format, and weight extraction from a
GGUF model for the projection shapes.

Format (tools/dump_matmul_fixtures.py:183-247 of the reference; the entries
of kernels/fixtures/manifest_matmul.json): per case a JSON entry with K, N,
M, W_shape [N, K], W_blocks, W_source, W_sha256, the file names, dtype
"IQ4_XS" and the activation seed, and raw little-endian files
    W_bin                   uint8   [N * K/256][136]   IQ4_XS super-blocks
    x_bin / X_bin           float32 [K] / [K][M]      (X[k*M + m])
    y_ref_bin / Y_ref_bin   float32 [N] / [N][M]      (Y[n*M + m])
The M = 1 cases use the lower-case keys, the others the upper-case ones.
Their y_ref is float32 (dequantised W) @ X on the unquantised activations.
"""
from __future__ import annotations

import hashlib
import json
import os

import numpy as np

from .gguf import GGUFReader

BLOCK_BYTES = 136
QK_K = 256


def load_manifest(directory: str, name: str = "manifest_matmul.json") -> list:
    with open(os.path.join(directory, name), encoding="utf-8") as f:
        entries = json.load(f)
    if not isinstance(entries, list):
        raise ValueError(f"{name}: expected a list of cases")
    return entries


def _read(directory: str, fname: str, dtype, count: int) -> np.ndarray:
    path = os.path.join(directory, fname)
    a = np.fromfile(path, dtype=dtype)
    if a.size != count:
        raise ValueError(f"{fname}: {a.size} elements, the manifest implies {count}")
    return a


def load_matmul_case(directory: str, entry: dict, check_sha: bool = True) -> dict:
    """{"W": uint8 [N*K/256*136], "X": float32 [K, M], "Y_ref": float32 [N, M], "K", "N", "M", "entry"}."""
    K, N, M = int(entry["K"]), int(entry["N"]), int(entry["M"])
    if K % QK_K or K <= 0 or N <= 0 or M <= 0:
        raise ValueError(f"case {entry.get('name')}: bad shape K={K} N={N} M={M}")
    if entry.get("dtype", "IQ4_XS") != "IQ4_XS":
        raise ValueError(f"case {entry.get('name')}: dtype {entry.get('dtype')}")
    n_blocks = N * (K // QK_K)
    if "W_blocks" in entry and int(entry["W_blocks"]) != n_blocks:
        raise ValueError(f"case {entry.get('name')}: W_blocks {entry['W_blocks']} != N*K/256 = {n_blocks}")
    W = _read(directory, entry["W_bin"], np.uint8, n_blocks * BLOCK_BYTES)
    if check_sha and "W_sha256" in entry:
        got = hashlib.sha256(W.tobytes()).hexdigest()
        if got != entry["W_sha256"]:
            raise ValueError(f"case {entry.get('name')}: W sha256 {got[:12]}... != manifest {entry['W_sha256'][:12]}...")
    x_key, y_key = ("x_bin", "y_ref_bin") if M == 1 else ("X_bin", "Y_ref_bin")
    X = _read(directory, entry[x_key], np.float32, K * M).reshape(K, M)
    Y = _read(directory, entry[y_key], np.float32, N * M).reshape(N, M)
    return {"W": W, "X": X, "Y_ref": Y, "K": K, "N": N, "M": M, "entry": entry}


def extract_projection(reader: GGUFReader, name: str, K: int, N: int) -> np.ndarray:
    """Raw IQ4_XS blocks of an N x K slice of a 2-D IQ4_XS tensor of shape
    (K_t, N_t) (ggml order), by the reference's rules
    (tools/dump_matmul_fixtures.py:75-104):
      K == K_t, N <= N_t : the first N rows, whole;
      K <= K_t, N <= N_t : the first N rows, each cut to its first K/256
                           super-blocks.
    Returns a new uint8 array [N * K/256 * 136]."""
    data, K_t, N_t = reader.iq4xs_matrix(name)
    if K % QK_K or K <= 0 or N <= 0 or K > K_t or N > N_t:
        raise ValueError(f"{name} is {K_t} x {N_t}; cannot take K={K}, N={N}")
    bpr_t, bpr = K_t // QK_K, K // QK_K
    rows = data[: N * bpr_t * BLOCK_BYTES].reshape(N, bpr_t, BLOCK_BYTES)
    return np.array(rows[:, :bpr, :], dtype=np.uint8, copy=True).reshape(-1)


def matmul_entry(name: str, K: int, N: int, M: int, W: np.ndarray, source: str, seed: int, prefix: str) -> dict:
    """A manifest entry in the reference's key layout for files named `prefix*`."""
    e = {"name": name, "K": K, "N": N, "M": M, "W_shape": [N, K], "W_blocks": N * (K // QK_K), "W_source": source,
         "W_sha256": hashlib.sha256(W.tobytes()).hexdigest(), "W_bin": f"{prefix}_W.bin",
         "X_shape": [K, M], "Y_shape": [N, M]}
    if M == 1:
        e.update({"x_bin": f"{prefix}_M1_x.bin", "y_ref_bin": f"{prefix}_M1_y_ref.bin"})
    else:
        e.update({"X_bin": f"{prefix}_M{M}_X.bin", "Y_ref_bin": f"{prefix}_M{M}_Y_ref.bin"})
    e.update({"dtype": "IQ4_XS", "seed": seed})
    return e
