"""The GGUF tooling of the end-to-end configuration (CPU): the v3 writer / reader against the
published layout (a byte-exact known answer and round trips of every metadata and tensor type
the writer emits), its rejections, the random-init Llama-3 writer (llama.cpp's metadata keys,
tensor names and shapes, vocab, decoded weight ranges through the oracle), and the llama-bench
harness's commands (llama.cpp exists on neither machine, so only its dry run runs here)."""
import json
import os
import struct
import subprocess
import sys

import numpy as np
import pytest

import gguf_io as G
import llama3_gguf as L
from oracle import oracle as O

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(HERE, "..", "ggml-rocket_amd")


def test_known_answer_bytes(tmp_path):
    """One u32 pair and one F32 [4] tensor, laid out by hand from the specification."""
    p = tmp_path / "ka.gguf"
    w = G.Writer(str(p))
    w.add("a", 7)
    w.add_tensor("t", 0, [4])
    w.write_data(np.arange(4, dtype=np.float32))
    w.close()
    head = (b"GGUF" + struct.pack("<IQQ", 3, 1, 1)
            + struct.pack("<Q", 1) + b"a" + struct.pack("<II", 4, 7)
            + struct.pack("<Q", 1) + b"t" + struct.pack("<IQ", 1, 4) + struct.pack("<IQ", 0, 0))
    head += b"\0" * ((-len(head)) % 32)
    assert p.read_bytes() == head + np.arange(4, dtype=np.float32).tobytes()


def test_round_trip_every_type(tmp_path):
    p = tmp_path / "rt.gguf"
    w = G.Writer(str(p), alignment=64)
    w.add("u32", 4000000000)
    w.add("i64", -5)
    w.add("f32", 1.5)
    w.add("str", "μ-text")
    w.add("flag", True)
    w.add("u8", 255, G.UINT8)
    w.add("f64", 2.25, G.FLOAT64)
    w.add("ints", (G.INT32, [1, -2, 3]), G.ARRAY)
    w.add("floats", (G.FLOAT32, np.array([0.5, -1.0], np.float32)), G.ARRAY)
    w.add("words", (G.STRING, ["x", "", "yz"]), G.ARRAY)
    rng = np.random.default_rng(5)
    tensors = [("f32", 0, [8, 3]), ("f16", 1, [5]), ("q4k", 12, [512, 2]), ("q6k", 14, [256, 3]),
               ("q8", 8, [64, 1]), ("q40", 2, [32, 2]), ("q5k", 13, [256, 1])]
    data = {}
    for name, t, ne in tensors:
        w.add_tensor(name, t, ne)
        data[name] = rng.integers(0, 256, G.tensor_nbytes(t, ne), dtype=np.uint8)
    for name, _, _ in tensors:
        w.write_data(data[name])
    w.close()
    r = G.Reader(str(p))
    assert r.kv["u32"] == 4000000000 and r.kv["i64"] == -5 and r.kv["f32"] == 1.5
    assert r.kv["str"] == "μ-text" and r.kv["flag"] is True and r.kv["u8"] == 255 and r.kv["f64"] == 2.25
    assert r.kv["general.alignment"] == 64
    assert list(r.kv["ints"]) == [1, -2, 3] and list(r.kv["floats"]) == [0.5, -1.0]
    assert r.kv["words"] == ["x", "", "yz"]
    assert r.data_offset % 64 == 0
    for name, t, ne in tensors:
        tt, nn, off, nb = r.tensors[name]
        assert (tt, nn) == (t, ne) and (off - r.data_offset) % 64 == 0
        assert np.array_equal(r.data(name), data[name])
    assert G.tensor_nbytes(12, [512, 2]) == 4 * 144 and G.tensor_nbytes(2, [32, 2]) == 36


def test_reader_rejects(tmp_path):
    good = tmp_path / "g.gguf"
    w = G.Writer(str(good))
    w.add_tensor("t", 0, [4])
    w.write_data(np.zeros(4, np.float32))
    w.close()
    b = good.read_bytes()
    for name, blob in (("magic", b"GGUX" + b[4:]), ("version", b[:4] + struct.pack("<I", 2) + b[8:]),
                       ("truncated", b[:30]), ("short data", b[:-4])):
        p = tmp_path / f"{name}.gguf"
        p.write_bytes(blob)
        with pytest.raises(G.GGUFError):
            G.Reader(str(p))
    with pytest.raises(G.GGUFError):
        G.tensor_nbytes(12, [100])          # not a whole Q4_K block
    w = G.Writer(str(tmp_path / "n.gguf"))
    w.add_tensor("t", 0, [4])
    with pytest.raises(G.GGUFError):
        w.write_data(np.zeros(3, np.float32))   # size differs from the declaration


def test_llama3_tiny_model(tmp_path):
    p = str(tmp_path / "tiny.gguf")
    info = L.write_llama3(p, layers=2, d=256, ffn=512, heads=4, kv_heads=2, vocab=1024)
    r = G.Reader(p)
    kv = r.kv
    assert kv["general.architecture"] == "llama" and kv["llama.block_count"] == 2
    assert kv["llama.embedding_length"] == 256 and kv["llama.feed_forward_length"] == 512
    assert kv["llama.attention.head_count"] == 4 and kv["llama.attention.head_count_kv"] == 2
    assert kv["llama.rope.dimension_count"] == 64 and kv["llama.vocab_size"] == 1024
    toks, tt = kv["tokenizer.ggml.tokens"], kv["tokenizer.ggml.token_type"]
    assert len(toks) == 1024 and toks[:3] == ["<unk>", "<s>", "</s>"] and toks[3 + 0x0A] == "<0x0A>"
    assert list(tt[:4]) == [2, 3, 3, 6] and int(tt[259]) == 1 and len(kv["tokenizer.ggml.scores"]) == 1024
    assert info["tensors"] == len(r.tensors) == 2 + 9 * 2 + 1
    shapes = {"attn_q": [256, 256], "attn_k": [256, 128], "attn_v": [256, 128], "attn_output": [256, 256],
              "ffn_gate": [256, 512], "ffn_up": [256, 512], "ffn_down": [512, 256]}
    for li in range(2):
        for n, ne in shapes.items():
            t, got, _, _ = r.tensors[f"blk.{li}.{n}.weight"]
            assert t == 12 and got == ne
        assert r.tensors[f"blk.{li}.attn_norm.weight"][:2] == (0, [256])
    assert r.tensors["token_embd.weight"][:2] == (12, [256, 1024])
    assert r.tensors["output.weight"][:2] == (14, [256, 1024])
    assert np.all(r.data("output_norm.weight").view(np.float32) == 1.0)
    # weights decode to finite values within +-0.05, layers distinct
    y = O.dequantize(O.Q4_K, np.array(r.data("blk.1.ffn_down.weight")), 512)
    assert np.isfinite(y).all() and np.abs(y).max() <= 0.0502 and y.std() > 0.005
    assert not np.array_equal(r.data("blk.0.attn_q.weight"), r.data("blk.1.attn_q.weight"))
    y6 = O.dequantize(O.Q6_K, np.array(r.data("output.weight")), 256)
    assert np.isfinite(y6).all() and np.abs(y6).max() <= 0.0502


def test_llama_bench_dry_run(tmp_path):
    out = subprocess.run([sys.executable, os.path.join(PKG, "llama_bench.py"), "--llama-cpp", str(tmp_path),
                          "--gguf", str(tmp_path / "m.gguf"), "--dry-run"], capture_output=True, text=True, check=True)
    cmds = json.loads(out.stdout)
    assert "-p 2048 -n 0 -b 512 -ub 512 -nr 1" in cmds["device"]
    assert "GGML_BACKEND_PATH=" in cmds["device"] and "MI355X_QUANT_RESIDENT=1" in cmds["device"]
    assert "-nr 0" in cmds["cpu"] and "GGML_BACKEND_PATH" not in cmds["cpu"]
    assert cmds["gguf"] and "llama3_gguf.py" in cmds["gguf"]
    # without a llama.cpp build it declines with status 2
    r = subprocess.run([sys.executable, os.path.join(PKG, "llama_bench.py"), "--llama-cpp", str(tmp_path)],
                       capture_output=True, text=True)
    assert r.returncode == 2 and "llama-bench" in r.stderr
