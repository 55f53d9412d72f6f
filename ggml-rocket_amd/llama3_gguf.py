"""A random-init Llama-3-8B GGUF: the model file of the end-to-end prefill configuration
(Q4_K projections and token embedding, Q6_K output, F32 norms), written with `gguf_io`.

    python ggml-rocket_amd/llama3_gguf.py OUT.gguf [--layers 32] [--d 4096] [--ffn 14336]
                                          [--heads 32] [--kv-heads 8] [--vocab 128256]

Metadata follows llama.cpp's `llama` architecture keys (general.architecture, llama.block_count,
llama.embedding_length, llama.feed_forward_length, llama.attention.head_count /
head_count_kv / layer_norm_rms_epsilon, llama.rope.freq_base / dimension_count,
llama.context_length, llama.vocab_size, general.file_type, general.quantization_version) and a
SentencePiece-style vocab (`tokenizer.ggml.model` "llama": <unk>, <s>, </s>, the 256 byte tokens
<0x00>..<0xFF> a loader looks up for byte fallback and the newline, then filler tokens, with
scores and token types). Tensor names and shapes are llama.cpp's (`token_embd`, `blk.N.attn_q` /
`attn_k` / `attn_v` / `attn_output` / `ffn_gate` / `ffn_up` / `ffn_down`, the norms, `output`;
ne0 = the input width). The weights are random codes under block headers that keep the decoded
values within about +-0.05: a timing model, not a language model (the prefill benchmark times
the same work for any weights). Smaller dims make the tiny models the tests use.
"""
import argparse
import os
import sys

import numpy as np

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
import gguf_io as G   # noqa: E402

F32, F16, Q4_K, Q6_K = 0, 1, 12, 14
FTYPE_MOSTLY_Q4_K_S = 14   # llama_ftype: Q4_K weights, Q6_K output


def _f16_bits(x: float) -> int:
    return int(np.array([x], dtype=np.float16).view(np.uint16)[0])


class _Pool:
    """Random bytes cycled from one pool: fast enough for gigabytes of codes."""

    def __init__(self, seed: int, size: int = 64 << 20):
        self.buf = np.random.default_rng(seed).integers(0, 256, size, dtype=np.uint8)
        self.pos = 0

    def take(self, n: int) -> np.ndarray:
        out = np.empty(n, dtype=np.uint8)
        done = 0
        while done < n:
            k = min(n - done, self.buf.size - self.pos)
            out[done:done + k] = self.buf[self.pos:self.pos + k]
            done += k
            self.pos = (self.pos + k + 4099) % self.buf.size   # a prime stride: tensors differ
        return out


def q4k_blocks(pool: _Pool, n_blocks: int) -> np.ndarray:
    """n Q4_K blocks: d, dmin fp16, random 6-bit scales / mins (any 12 bytes are a valid
    packing), random nibbles; |y| = |d sc q - dmin m| <= 0.05."""
    b = pool.take(n_blocks * 144).reshape(n_blocks, 144)
    hdr = np.array([_f16_bits(0.05 / (63 * 15)), _f16_bits(0.05 / 63)], dtype=np.uint16)
    b[:, 0:4] = hdr.view(np.uint8)
    return b.reshape(-1)


def q6k_blocks(pool: _Pool, n_blocks: int) -> np.ndarray:
    """n Q6_K blocks: random 6-bit codes, int8 scales in [-64, 63], d so |y| <= 0.05."""
    b = pool.take(n_blocks * 210).reshape(n_blocks, 210)
    b[:, 192:208] = (b[:, 192:208] & 0x7F) - 64 & 0xFF
    b[:, 208:210] = np.array([_f16_bits(0.05 / (64 * 32))], dtype=np.uint16).view(np.uint8)
    return b.reshape(-1)


def write_llama3(path: str, layers: int = 32, d: int = 4096, ffn: int = 14336, heads: int = 32,
                 kv_heads: int = 8, vocab: int = 128256, ctx: int = 8192, seed: int = 0x5EED) -> dict:
    hd = d // heads
    w = G.Writer(path)
    w.add("general.architecture", "llama")
    w.add("general.name", f"random-init llama3 {layers}L d{d}")
    w.add("general.file_type", FTYPE_MOSTLY_Q4_K_S)
    w.add("general.quantization_version", 2)
    w.add("llama.context_length", ctx)
    w.add("llama.embedding_length", d)
    w.add("llama.block_count", layers)
    w.add("llama.feed_forward_length", ffn)
    w.add("llama.rope.dimension_count", hd)
    w.add("llama.rope.freq_base", 500000.0)
    w.add("llama.attention.head_count", heads)
    w.add("llama.attention.head_count_kv", kv_heads)
    w.add("llama.attention.layer_norm_rms_epsilon", 1e-5)
    w.add("llama.vocab_size", vocab)
    tokens = ["<unk>", "<s>", "</s>"] + [f"<0x{i:02X}>" for i in range(256)]
    tokens += [f"▁t{i}" for i in range(vocab - len(tokens))]
    ttype = np.full(vocab, 1, dtype=np.int32)   # normal
    ttype[0], ttype[1], ttype[2] = 2, 3, 3       # unknown, control, control
    ttype[3:259] = 6                             # byte
    scores = -np.arange(vocab, dtype=np.float32)
    w.add("tokenizer.ggml.model", "llama")
    w.add("tokenizer.ggml.tokens", (G.STRING, tokens), G.ARRAY)
    w.add("tokenizer.ggml.scores", (G.FLOAT32, scores), G.ARRAY)
    w.add("tokenizer.ggml.token_type", (G.INT32, ttype), G.ARRAY)
    w.add("tokenizer.ggml.bos_token_id", 1)
    w.add("tokenizer.ggml.eos_token_id", 2)
    w.add("tokenizer.ggml.unknown_token_id", 0)

    plan = [("token_embd.weight", Q4_K, [d, vocab])]
    for i in range(layers):
        plan += [(f"blk.{i}.attn_norm.weight", F32, [d]),
                 (f"blk.{i}.attn_q.weight", Q4_K, [d, d]),
                 (f"blk.{i}.attn_k.weight", Q4_K, [d, kv_heads * hd]),
                 (f"blk.{i}.attn_v.weight", Q4_K, [d, kv_heads * hd]),
                 (f"blk.{i}.attn_output.weight", Q4_K, [d, d]),
                 (f"blk.{i}.ffn_norm.weight", F32, [d]),
                 (f"blk.{i}.ffn_gate.weight", Q4_K, [d, ffn]),
                 (f"blk.{i}.ffn_up.weight", Q4_K, [d, ffn]),
                 (f"blk.{i}.ffn_down.weight", Q4_K, [ffn, d])]
    plan += [("output_norm.weight", F32, [d]), ("output.weight", Q6_K, [d, vocab])]
    for name, t, ne in plan:
        w.add_tensor(name, t, ne)
    pool = _Pool(seed)
    total = 0
    for name, t, ne in plan:
        nb = G.tensor_nbytes(t, ne)
        if t == F32:
            data = np.ones(int(np.prod(ne)), dtype=np.float32)
        elif t == Q4_K:
            data = q4k_blocks(pool, nb // 144)
        else:
            data = q6k_blocks(pool, nb // 210)
        w.write_data(data)
        total += nb
    w.close()
    return {"path": path, "tensors": len(plan), "data_bytes": total, "file_bytes": os.path.getsize(path)}


def main():
    p = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    p.add_argument("out")
    p.add_argument("--layers", type=int, default=32)
    p.add_argument("--d", type=int, default=4096)
    p.add_argument("--ffn", type=int, default=14336)
    p.add_argument("--heads", type=int, default=32)
    p.add_argument("--kv-heads", type=int, default=8)
    p.add_argument("--vocab", type=int, default=128256)
    a = p.parse_args()
    info = write_llama3(a.out, a.layers, a.d, a.ffn, a.heads, a.kv_heads, a.vocab)
    print(info)


if __name__ == "__main__":
    main()
