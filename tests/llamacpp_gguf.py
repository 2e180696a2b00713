"""Writes GGUF files laid out the way llama.cpp's converter writes a Llama-3.2
model (test infrastructure).

Real files cannot be fetched here, so the tests rewrite a synthetic model in
that layout: llama.cpp's metadata set and key order (general.* strings and
string arrays, llama.attention.key_length / value_length, general.file_type,
the tokenizer.ggml.* arrays, general.quantization_version), its tensor order
(token_embd, then each block's tensors, then output_norm and the
rope_freqs.weight table llama.cpp stores for llama3 RoPE), and padding of the
data section and of every tensor to general.alignment.  The reference reads
the fields it needs and ignores the rest (src/models/llama/config.rs:29-73,
src/models/llama/weights.rs:50-97); with general.alignment other than 32 only
a reader that honours the key finds the tensors.
"""
from __future__ import annotations

import struct

import numpy as np

from oracle.gguf_reader import ARRAY, BOOL, F32, I32, STRING, U32, GGUFFile

GGUF_MAGIC = 0x46554747


def _str(s: str) -> bytes:
    b = s.encode("utf-8")
    return struct.pack("<Q", len(b)) + b


def _value(t: int, v) -> bytes:
    if t == STRING:
        return _str(v)
    if t == BOOL:
        return struct.pack("<B", 1 if v else 0)
    if t == ARRAY:
        at, items = v
        return struct.pack("<IQ", at, len(items)) + b"".join(_value(at, x) for x in items)
    fmt = {U32: "<I", I32: "<i", F32: "<f"}[t]
    return struct.pack(fmt, v)


def write_gguf(path: str, kvs: list, tensors: list, alignment: int = 32) -> None:
    """kvs: [(key, type, value)]; tensors: [(name, dims, ggml_type, bytes)]."""
    out = bytearray(struct.pack("<IIQQ", GGUF_MAGIC, 3, len(tensors), len(kvs)))
    for k, t, v in kvs:
        out += _str(k) + struct.pack("<I", t) + _value(t, v)
    off, blobs = 0, []
    for name, dims, typ, data in tensors:
        out += _str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        out += struct.pack("<IQ", typ, off)
        pad = b"\0" * ((-len(data)) % alignment)
        blobs.append(bytes(data) + pad)
        off += len(blobs[-1])
    out += b"\0" * ((-len(out)) % alignment)
    with open(path, "wb") as fh:
        fh.write(bytes(out))
        for b in blobs:
            fh.write(b)


def llama3_rope_freqs(head_dim: int, base: float, factor=32.0, low=1.0, high=4.0, orig=8192) -> np.ndarray:
    """The per-frequency divisors llama.cpp stores as rope_freqs.weight."""
    inv = base ** (-np.arange(0, head_dim, 2, dtype=np.float64) / head_dim)
    wl = 2 * np.pi / inv
    f = np.ones_like(inv)
    f[wl > orig / low] = factor
    mid = (wl <= orig / low) & (wl >= orig / high)
    smooth = (orig / wl[mid] - low) / (high - low)
    f[mid] = 1.0 / ((1 - smooth) / factor + smooth)
    return f.astype(np.float32)


def token_strings(vocab: int) -> list:
    """Byte-level BPE style token strings: the 256 byte symbols, then merges."""
    base = [chr(0x100 + b) if b < 0x21 or 0x7E < b < 0xA1 or b == 0xAD else chr(b) for b in range(256)]
    toks = base[:vocab]
    i = 0
    while len(toks) < vocab:
        toks.append(base[97 + i % 26] + base[97 + (i // 26) % 26] + str(i))
        i += 1
    return toks


def rewrite_llamacpp(src: str, dst: str, alignment: int = 32, alignment_key: bool = True,
                     vocab_size_key: bool = False, rope_freqs: bool = True, rope_scaling_keys: bool = False,
                     head_dim_key: bool = True) -> None:
    """Re-emits the synthetic model at src in llama.cpp's layout at dst."""
    g = GGUFFile(src)
    md = {k: v for k, (t, v) in g.metadata.items()}
    D = md["llama.embedding_length"]
    H = md["llama.attention.head_count"]
    hd = md.get("llama.rope.dimension_count", D // H)
    vocab = md["llama.vocab_size"]
    ftype = {8: 7, 2: 2, 30: 32}[g.tensors["blk.0.attn_q.weight"].ggml_type]
    toks = token_strings(vocab)
    kvs = [("general.architecture", STRING, "llama"),
           ("general.type", STRING, "model"),
           ("general.name", STRING, "Llama 3.2 1B Instruct"),
           ("general.finetune", STRING, "Instruct"),
           ("general.basename", STRING, "Llama-3.2"),
           ("general.size_label", STRING, "1B"),
           ("general.license", STRING, "llama3.2"),
           ("general.tags", ARRAY, (STRING, ["facebook", "meta", "pytorch", "llama", "llama-3"])),
           ("general.languages", ARRAY, (STRING, ["en", "de", "fr"])),
           ("llama.block_count", U32, md["llama.block_count"]),
           ("llama.context_length", U32, md["llama.context_length"]),
           ("llama.embedding_length", U32, D),
           ("llama.feed_forward_length", U32, md["llama.feed_forward_length"]),
           ("llama.attention.head_count", U32, H),
           ("llama.attention.head_count_kv", U32, md["llama.attention.head_count_kv"]),
           ("llama.rope.freq_base", F32, md["llama.rope.freq_base"]),
           ("llama.attention.layer_norm_rms_epsilon", F32, md["llama.attention.layer_norm_rms_epsilon"]),
           ("llama.attention.key_length", U32, hd),
           ("llama.attention.value_length", U32, hd)]
    if vocab_size_key:
        kvs.append(("llama.vocab_size", U32, vocab))
    if head_dim_key:
        kvs.append(("llama.rope.dimension_count", U32, hd))
    if rope_scaling_keys:
        kvs += [("llama.rope.scaling.factor", F32, 32.0), ("llama.rope.scaling.low_freq_factor", F32, 1.0),
                ("llama.rope.scaling.high_freq_factor", F32, 4.0),
                ("llama.rope.scaling.original_context_length", U32, 8192)]
    kvs += [("general.file_type", U32, ftype),
            ("tokenizer.ggml.model", STRING, "gpt2"),
            ("tokenizer.ggml.pre", STRING, "llama-bpe"),
            ("tokenizer.ggml.tokens", ARRAY, (STRING, toks)),
            ("tokenizer.ggml.token_type", ARRAY, (I32, [1] * vocab)),
            ("tokenizer.ggml.merges", ARRAY, (STRING, [f"{toks[97]} {toks[98]}", f"{toks[99]} {toks[100]}"])),
            ("tokenizer.ggml.bos_token_id", U32, md["tokenizer.ggml.bos_token_id"]),
            ("tokenizer.ggml.eos_token_id", U32, md["tokenizer.ggml.eos_token_id"]),
            ("tokenizer.ggml.padding_token_id", U32, md["tokenizer.ggml.eos_token_id"]),
            ("tokenizer.chat_template", STRING, "{% for m in messages %}{{ m['content'] }}{% endfor %}"),
            ("general.quantization_version", U32, 2)]
    if alignment_key:
        kvs.insert(1, ("general.alignment", U32, alignment))
    names = ["token_embd.weight"]
    for i in range(md["llama.block_count"]):
        names += [f"blk.{i}.{n}.weight" for n in ("attn_norm", "attn_q", "attn_k", "attn_v", "attn_output",
                                                  "ffn_norm", "ffn_gate", "ffn_up", "ffn_down")]
    names += [n for n in ("output.weight",) if n in g.tensors]
    names.append("output_norm.weight")
    tensors = []
    for n in names:
        ti = g.tensors[n]
        tensors.append((n, list(ti.dims), ti.ggml_type, g.tensor_bytes(n).tobytes()))
    if rope_freqs:
        rf = llama3_rope_freqs(hd, md["llama.rope.freq_base"])
        tensors.append(("rope_freqs.weight", [hd // 2], 0, rf.tobytes()))
    write_gguf(dst, kvs, tensors, alignment)
