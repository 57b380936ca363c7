"""GGUF reader and fixture loader (CPU).  The reader is pinned by files
assembled here field by field from the published GGUF layout (independent of
any writer in this repository), by the facts the reference's own llama.cpp
log states about its model file (benchmarks/environment/startup-log.txt:
24-73: GGUF V3, typed key-values, per-type tensor counts, file type 30 =
"IQ4_XS - 4.25 bpw"), and by the reference's slicing rules for projection
fixtures (tools/dump_matmul_fixtures.py:75-104)."""
import hashlib
import json
import os
import struct

import numpy as np
import pytest


def S(s: str) -> bytes:
    b = s.encode("utf-8")
    return struct.pack("<Q", len(b)) + b


def kv(key, vtype, payload: bytes) -> bytes:
    return S(key) + struct.pack("<I", vtype) + payload


def tinfo(name, ne, gtype, offset) -> bytes:
    return S(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", d) for d in ne) + \
        struct.pack("<IQ", gtype, offset)


def assemble(kvs, tensors, blobs, alignment=32, version=3) -> bytes:
    """tensors: (name, ne, type); blobs: their bytes, laid out in order at aligned offsets."""
    offs, pos = [], 0
    for b in blobs:
        pos = (pos + alignment - 1) // alignment * alignment
        offs.append(pos)
        pos += len(b)
    head = b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(kvs)) + b"".join(kvs)
    head += b"".join(tinfo(n, ne, t, o) for (n, ne, t), o in zip(tensors, offs))
    data_start = (len(head) + alignment - 1) // alignment * alignment
    out = bytearray(head + b"\0" * (data_start - len(head)))
    for b, o in zip(blobs, offs):
        out += b"\0" * (data_start + o - len(out))
        out += b
    return bytes(out)


@pytest.fixture(scope="module")
def gg(pkg):
    import importlib

    return importlib.import_module(pkg.__name__ + ".gguf")


@pytest.fixture(scope="module")
def fx(pkg):
    import importlib

    return importlib.import_module(pkg.__name__ + ".fixtures")


ALL_KVS = [
    kv("general.architecture", 8, S("qwen35")),
    kv("t.u8", 0, struct.pack("<B", 200)), kv("t.i8", 1, struct.pack("<b", -5)),
    kv("t.u16", 2, struct.pack("<H", 60000)), kv("t.i16", 3, struct.pack("<h", -30000)),
    kv("qwen35.embedding_length", 4, struct.pack("<I", 5120)), kv("general.sampling.top_k", 5, struct.pack("<i", 20)),
    kv("qwen35.attention.layer_norm_rms_epsilon", 6, struct.pack("<f", 1e-6)), kv("t.bool", 7, b"\x01"),
    kv("qwen35.rope.dimension_sections", 9, struct.pack("<IQ", 5, 4) + struct.pack("<4i", 11, 11, 10, 0)),
    kv("tokenizer.ggml.tokens", 9, struct.pack("<IQ", 8, 3) + S("!") + S("\"") + S("Ġ Ġ")),
    kv("t.u64", 10, struct.pack("<Q", 2 ** 40 + 3)), kv("t.i64", 11, struct.pack("<q", -(2 ** 40))),
    kv("t.f64", 12, struct.pack("<d", 0.1)),
    kv("t.nested", 9, struct.pack("<IQ", 9, 2) + struct.pack("<IQ", 4, 2) + struct.pack("<2I", 1, 2)
       + struct.pack("<IQ", 4, 1) + struct.pack("<I", 3)),
    kv("general.file_type", 4, struct.pack("<I", 30)),
]


def write(tmp_path, name, data):
    p = tmp_path / name
    p.write_bytes(data)
    return str(p)


def test_reader_hand_assembled_file(gg, orc, tmp_path):
    W = orc.gen_weights(512, 3, seed=5)                          # 3 rows x 2 super-blocks
    f32 = np.arange(5, dtype="<f4") * np.float32(0.5)
    q5k = bytes(range(176)) * 2                                   # 2 blocks of 176 B
    tensors = [("blk.0.ffn_down.weight", (512, 3), 23), ("blk.0.attn_norm.weight", (5,), 0),
               ("token_embd.weight", (256, 2), 13)]
    blobs = [W.tobytes(), f32.tobytes(), q5k]
    for align, version in ((32, 3), (64, 3), (32, 2)):
        kvs = list(ALL_KVS) + ([kv("general.alignment", 4, struct.pack("<I", align))] if align != 32 else [])
        path = write(tmp_path, f"a{align}_{version}.gguf", assemble(kvs, tensors, blobs, align, version))
        with gg.GGUFReader(path) as r:
            assert r.version == version and r.alignment == align and r.data_offset % align == 0
            m = r.metadata
            assert m["general.architecture"] == "qwen35" and m["t.u8"] == 200 and m["t.i8"] == -5
            assert m["t.u16"] == 60000 and m["t.i16"] == -30000 and m["qwen35.embedding_length"] == 5120
            assert m["general.sampling.top_k"] == 20 and m["t.bool"] is True
            assert m["qwen35.attention.layer_norm_rms_epsilon"] == np.float32(1e-6)
            assert list(m["qwen35.rope.dimension_sections"]) == [11, 11, 10, 0]
            assert m["tokenizer.ggml.tokens"] == ["!", "\"", "Ġ Ġ"]
            assert m["t.u64"] == 2 ** 40 + 3 and m["t.i64"] == -(2 ** 40) and m["t.f64"] == 0.1
            assert [list(a) for a in m["t.nested"]] == [[1, 2], [3]]
            assert r.metadata_types["qwen35.rope.dimension_sections"] == (9, 5)
            assert [t.name for t in r.tensors] == [n for n, _, _ in tensors]
            blocks, K, N = r.iq4xs_matrix("blk.0.ffn_down.weight")
            assert (K, N) == (512, 3) and np.array_equal(blocks, W)
            assert np.array_equal(r.tensor("blk.0.attn_norm.weight").data.view("<f4"), f32)
            t = r.tensor("token_embd.weight")
            assert t.type_name == "q5_K" and t.nbytes == 352 and bytes(t.data) == q5k
            for t, b in zip(r.tensors, blobs):
                assert t.offset % align == 0 and t.nbytes == len(b)


def test_reader_reproduces_the_reference_log_facts(gg, tmp_path):
    """llama.cpp's listing of the reference's model: tensors of types f32,
    q5_K, q6_K and iq4_xs (startup-log.txt:68-71) and file type 30 printed
    as 'IQ4_XS - 4.25 bpw' (:37, :73)."""
    tensors, blobs = [], []
    for i, (t, blk, bb) in enumerate(((0, 1, 4), (13, 256, 176), (14, 256, 210), (23, 256, 136), (23, 256, 136))):
        tensors.append((f"t{i}", (256, 1), t))
        blobs.append(bytes(256 // blk * bb))
    path = write(tmp_path, "log.gguf", assemble(ALL_KVS, tensors, blobs))
    with gg.GGUFReader(path) as r:
        assert r.type_counts() == {"f32": 1, "q5_K": 1, "q6_K": 1, "iq4_xs": 2}
        assert r.file_type() == "IQ4_XS - 4.25 bpw"
        assert gg.TYPE_NAMES[r.metadata_types["qwen35.embedding_length"][0]] == "u32"
        assert gg.TYPE_NAMES[r.metadata_types["qwen35.attention.layer_norm_rms_epsilon"][0]] == "f32"


def test_reader_rejects_malformed_files(gg, tmp_path):
    good = assemble(ALL_KVS, [("w", (256, 1), 23)], [bytes(136)])
    cases = {
        "magic": b"GGUX" + good[4:],
        "version": good[:4] + struct.pack("<I", 1) + good[8:],
        "truncated_kv": good[:40],
        "truncated_tail": good[:len(good) - 200],
        "truncated_data": good[:-10],
        "bad_kv_type": assemble([kv("k", 13, b"")], [], []),
        "misaligned": b"GGUF" + struct.pack("<IQQ", 3, 1, 0) + tinfo("w", (256, 1), 23, 7) + bytes(200),
        "ragged_row": assemble([], [("w", (200, 1), 23)], [bytes(136)]),
        "tiny": b"GGUF",
    }
    for name, data in cases.items():
        with pytest.raises(gg.GGUFError):
            gg.GGUFReader(write(tmp_path, name + ".gguf", data))
    path = write(tmp_path, "f32.gguf", assemble([], [("w", (4,), 0)], [bytes(16)]))
    with gg.GGUFReader(path) as r:
        with pytest.raises(gg.GGUFError):
            r.iq4xs_matrix("w")
        with pytest.raises(KeyError):
            r.tensor("missing")


def test_extract_projection_follows_the_reference_rules(gg, fx, orc, tmp_path):
    K_t, N_t = 1024, 6
    W = orc.gen_weights(K_t, N_t, seed=9)
    path = write(tmp_path, "p.gguf", assemble([], [("blk.0.ffn_up.weight", (K_t, N_t), 23)], [W.tobytes()]))
    rows = W.reshape(N_t, K_t // 256, 136)
    with gg.GGUFReader(path) as r:
        assert np.array_equal(fx.extract_projection(r, "blk.0.ffn_up.weight", 1024, 4), rows[:4].ravel())
        assert np.array_equal(fx.extract_projection(r, "blk.0.ffn_up.weight", 512, 6), rows[:, :2].ravel())
        with pytest.raises(ValueError):
            fx.extract_projection(r, "blk.0.ffn_up.weight", 2048, 1)
        with pytest.raises(ValueError):
            fx.extract_projection(r, "blk.0.ffn_up.weight", 1024, 7)


def test_committed_fixtures_load_and_check(fx, orc):
    d = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "matmul_fixtures")
    entries = fx.load_manifest(d)
    assert {e["M"] for e in entries} >= {1, 16}
    for e in entries:
        c = fx.load_matmul_case(d, e)
        K, N, M = c["K"], c["N"], c["M"]
        assert c["W"].size == N * K // 256 * 136 and c["X"].shape == (K, M) and c["Y_ref"].shape == (N, M)
        # y_ref is the float32 product of the dequantised weights and the raw activations
        Wf = orc.dequant(c["W"], K, N).astype(np.float64)
        y64 = Wf @ c["X"].astype(np.float64)
        err = np.linalg.norm(c["Y_ref"] - y64) / np.linalg.norm(y64)
        assert err < 1e-5, (e["name"], err)
    bad = dict(entries[0], W_sha256="0" * 64)
    with pytest.raises(ValueError):
        fx.load_matmul_case(d, bad)
    short = dict(entries[0], K=entries[0]["K"] + 256, W_blocks=None)
    short.pop("W_blocks")
    with pytest.raises(ValueError):
        fx.load_matmul_case(d, short, check_sha=False)
