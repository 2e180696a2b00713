"""Host-side logic on the CPU: the C ABI's exports, the GGUF reader/writer,
the config reader, error mapping and the synthetic model generator.  Nothing
here launches a kernel."""
import ctypes as C
import os
import re
import struct

import numpy as np
import pytest

from oracle import oracle as O
from oracle.gguf_reader import GGUFError, GGUFFile

import sqhip
from sqhip._lib import ModelInfo, lib

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include",
                      "squirrel_hip.h")
SMALL = dict(n_layers=2, dim=128, ffn_dim=256, n_heads=2, n_kv_heads=1, vocab=300,
             context_length=512)


def test_every_declared_symbol_is_exported():
    text = open(HEADER).read()
    names = set(re.findall(r"\b(sq_[a-z0-9_]+)\s*\(", text))
    assert len(names) > 30
    L = C.CDLL(sqhip._lib.LIB_PATH)
    missing = [n for n in sorted(names) if not hasattr(L, n)]
    assert not missing, missing


def test_integration_binding_lists_every_declaration():
    """The Rust -sys binding shown for maintainers binds every function the
    header declares, and nothing else."""
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    declared = set(re.findall(r"\b(sq_[a-z0-9_]+)\s*\(", text))
    doc = open(os.path.join(os.path.dirname(HEADER), "..", "INTEGRATION.md")).read()
    block = doc[doc.index('extern "C" {'):]
    block = block[:block.index("\n}\n")]
    bound = set(re.findall(r"pub fn (sq_[a-z0-9_]+)\(", block))
    assert bound == declared, (sorted(declared - bound), sorted(bound - declared))


def inspect(path):
    info = ModelInfo()
    inv = np.zeros(64, np.float32)
    code = lib().sq_gguf_inspect(os.fsencode(path), C.byref(info), inv.ctypes.data, inv.size)
    return code, info, inv


@pytest.mark.parametrize("wtype", ["Q8_0", "Q4_0", "BF16"])
def test_synth_gguf_round_trip(tmp_path, wtype):
    p = str(tmp_path / "m.gguf")
    sqhip.write_synthetic_gguf(p, wtype, seed=5, **SMALL)
    g = GGUFFile(p)
    assert g.magic == 0x46554747 and g.version == 3
    md = g.metadata
    assert md["llama.block_count"] == (4, 2) and md["llama.embedding_length"] == (4, 128)
    assert md["llama.rope.freq_base"][0] == 6 and md["llama.rope.freq_base"][1] == 500000.0
    assert md["general.architecture"] == (8, "llama")
    names = {f"blk.{i}.{n}.weight" for i in range(2) for n in O.LAYER_NAMES}
    names |= {"token_embd.weight", "output_norm.weight"}
    assert set(g.tensors) == names  # tied: no output.weight
    t = g.tensors["blk.1.ffn_down.weight"]
    assert t.dims == (256, 128) and t.ggml_type == {"Q8_0": 8, "Q4_0": 2, "BF16": 30}[wtype]
    assert all(ti.offset % 32 == 0 for ti in g.tensors.values())
    assert g.data_offset % 32 == 0
    norm = np.frombuffer(g.tensor_bytes("blk.0.ffn_norm.weight").tobytes(), np.float32)
    assert np.all(norm == 1.0)
    code, info, inv = inspect(p)
    assert code == 0
    assert (info.n_layers, info.dim, info.ffn_dim, info.n_heads, info.n_kv_heads, info.head_dim,
            info.vocab, info.tied_output) == (2, 128, 256, 2, 1, 64, 300, 1)
    cfg = O.LlamaConfig(g)
    assert np.array_equal(inv[:32], cfg.inv_freq)


def test_synth_is_deterministic_and_seeded(tmp_path):
    a, b, c = (str(tmp_path / f"{n}.gguf") for n in "abc")
    sqhip.write_synthetic_gguf(a, "Q8_0", seed=1, **SMALL)
    sqhip.write_synthetic_gguf(b, "Q8_0", seed=1, **SMALL)
    sqhip.write_synthetic_gguf(c, "Q8_0", seed=2, **SMALL)
    assert open(a, "rb").read() == open(b, "rb").read()
    assert open(a, "rb").read() != open(c, "rb").read()


def test_synth_weights_statistics_and_q8_idempotence(tmp_path):
    p = str(tmp_path / "m.gguf")
    sqhip.write_synthetic_gguf(p, "Q8_0", seed=3, **SMALL)
    g = GGUFFile(p)
    blocks = np.frombuffer(g.tensor_bytes("token_embd.weight").tobytes(), O.BLOCK_Q8_0)
    x = O.dequantize(O.Q8_0, blocks, blocks.size * 32)
    assert abs(x.mean()) < 1e-3 and abs(x.std() - 0.02) < 1e-3
    # Requantizing dequantized Q8_0 blocks reproduces them (the writer used
    # the reference quantizer).
    re_q = O.quantize_row_q8_0(x)
    assert np.array_equal(re_q["d"], blocks["d"]) and np.array_equal(re_q["qs"], blocks["qs"])


def test_synth_q4_0_convention(tmp_path):
    p = str(tmp_path / "m.gguf")
    sqhip.write_synthetic_gguf(p, "Q4_0", seed=3, **SMALL)
    blocks = np.frombuffer(GGUFFile(p).tensor_bytes("blk.0.attn_q.weight").tobytes(), O.BLOCK_Q4_0)
    lo, hi = blocks["qs"] & 15, blocks["qs"] >> 4
    q = np.concatenate([lo, hi], axis=1).astype(np.int32)
    # d = m / -8 with m the signed extreme value: that element decodes to -8.
    assert np.all((q == 0).any(axis=1))
    d = blocks["d"].view(np.float16).astype(np.float32)
    x = (q - 8) * d[:, None]
    assert np.all(np.abs(x).max(axis=1) <= 8 * np.abs(d) + 1e-12)


# ----------------------------------------------------------- crafted files

class Writer:
    """A minimal independent GGUF writer for crafting malformed files."""

    def __init__(self):
        self.kv = []
        self.t = []

    def u32(self, k, v):
        self.kv.append((k, struct.pack("<II", 4, v)))
        return self

    def f32(self, k, v):
        self.kv.append((k, struct.pack("<If", 6, v)))
        return self

    def raw(self, k, typ, payload):
        self.kv.append((k, struct.pack("<I", typ) + payload))
        return self

    def tensor(self, name, dims, typ, data):
        self.t.append((name, dims, typ, data))
        return self

    def bytes(self):
        s = lambda x: struct.pack("<Q", len(x)) + x.encode()  # noqa: E731
        out = struct.pack("<IIQQ", 0x46554747, 3, len(self.t), len(self.kv))
        for k, v in self.kv:
            out += s(k) + v
        off, infos, blobs = 0, b"", []
        for name, dims, typ, data in self.t:
            infos += s(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
            infos += struct.pack("<IQ", typ, off)
            blobs.append(data + b"\0" * ((-len(data)) % 32))
            off += len(blobs[-1])
        out += infos
        out += b"\0" * ((-len(out)) % 32)
        return out + b"".join(blobs)


def base_meta(w):
    for k, v in [("llama.block_count", 1), ("llama.embedding_length", 64), ("llama.feed_forward_length", 64),
                 ("llama.attention.head_count", 1), ("llama.attention.head_count_kv", 1),
                 ("llama.context_length", 128), ("tokenizer.ggml.bos_token_id", 1),
                 ("tokenizer.ggml.eos_token_id", 2), ("llama.vocab_size", 32)]:
        w.u32(k, v)
    w.f32("llama.rope.freq_base", 10000.0).f32("llama.attention.layer_norm_rms_epsilon", 1e-5)
    return w


def q8(k, n):
    return np.zeros(n * k // 32, O.BLOCK_Q8_0).tobytes()


def full_model(w, skip=()):
    f = np.ones(64, np.float32).tobytes()
    names = [("blk.0.attn_norm.weight", [64], 0, f), ("blk.0.attn_q.weight", [64, 64], 8, q8(64, 64)),
             ("blk.0.attn_k.weight", [64, 64], 8, q8(64, 64)), ("blk.0.attn_v.weight", [64, 64], 8, q8(64, 64)),
             ("blk.0.attn_output.weight", [64, 64], 8, q8(64, 64)), ("blk.0.ffn_norm.weight", [64], 0, f),
             ("blk.0.ffn_gate.weight", [64, 64], 8, q8(64, 64)), ("blk.0.ffn_up.weight", [64, 64], 8, q8(64, 64)),
             ("blk.0.ffn_down.weight", [64, 64], 8, q8(64, 64)), ("token_embd.weight", [64, 32], 8, q8(64, 32)),
             ("output_norm.weight", [64], 0, f)]
    for n, d, t, data in names:
        if n not in skip:
            w.tensor(n, d, t, data)
    return w


def write(tmp_path, data, name="x.gguf"):
    p = str(tmp_path / name)
    with open(p, "wb") as fh:
        fh.write(data)
    return p


def test_crafted_valid_model_inspects(tmp_path):
    p = write(tmp_path, full_model(base_meta(Writer())).bytes())
    code, info, inv = inspect(p)
    assert code == 0 and info.head_dim == 64 and info.vocab == 32
    assert inv[0] == 1.0


@pytest.mark.parametrize("case,code", [
    ("missing_file", 16), ("truncated", 17), ("bad_bool", 17), ("bad_value_type", 17),
    ("unknown_ggml_type", 17), ("missing_metadata", 18), ("wrong_metadata_type", 18),
    ("missing_tensor", 19), ("unsupported_quant", 20), ("vocab_from_tokens", 0),
])
def test_load_path_errors(tmp_path, case, code):
    w = full_model(base_meta(Writer()))
    if case == "missing_file":
        p = str(tmp_path / "nope.gguf")
    elif case == "truncated":
        p = write(tmp_path, w.bytes()[:100])
    elif case == "bad_bool":
        w.raw("some.flag", 7, b"\x02")
        p = write(tmp_path, w.bytes())
    elif case == "bad_value_type":
        w.raw("weird", 13, b"")
        p = write(tmp_path, w.bytes())
    elif case == "unknown_ggml_type":
        w.tensor("extra", [32], 4, b"\0" * 64)
        p = write(tmp_path, w.bytes())
    elif case == "missing_metadata":
        w.kv = [kv for kv in w.kv if kv[0] != "llama.context_length"]
        p = write(tmp_path, w.bytes())
    elif case == "wrong_metadata_type":
        w.kv = [kv for kv in w.kv if kv[0] != "llama.block_count"]
        w.f32("llama.block_count", 1.0)
        p = write(tmp_path, w.bytes())
    elif case == "missing_tensor":
        w = full_model(base_meta(Writer()), skip=("blk.0.ffn_up.weight",))
        p = write(tmp_path, w.bytes())
    elif case == "unsupported_quant":
        w = full_model(base_meta(Writer()), skip=("blk.0.attn_q.weight",))
        w.tensor("blk.0.attn_q.weight", [64, 64], 12, b"\0" * (64 * 64 // 256 * 144))
        p = write(tmp_path, w.bytes())
    else:  # vocab from tokenizer.ggml.tokens when llama.vocab_size is absent
        w.kv = [kv for kv in w.kv if kv[0] != "llama.vocab_size"]
        toks = struct.pack("<IQ", 8, 32) + b"".join(struct.pack("<Q", 1) + b"t" for _ in range(32))
        w.raw("tokenizer.ggml.tokens", 9, toks)
        p = write(tmp_path, w.bytes())
    got, info, _ = inspect(p)
    assert got == code, lib().sq_last_error()
    if code == 0:
        assert info.vocab == 32
    # The independent Python reader agrees on which files are malformed.
    if code in (16, 17):
        with pytest.raises((GGUFError, OSError, ValueError)):
            GGUFFile(p)
    elif code == 18:
        with pytest.raises(O.ConfigError):
            O.LlamaConfig(GGUFFile(p))


# ----------------------------------------------------------- llama.cpp layout

LLAMACPP_VARIANTS = {
    # alignment, write the key, llama.vocab_size, rope scaling keys, rope.dimension_count
    "align32": dict(alignment=32),
    "align64": dict(alignment=64),
    "align256": dict(alignment=256),
    "no_alignment_key": dict(alignment=32, alignment_key=False),
    "vocab_size_key": dict(alignment=32, vocab_size_key=True),
    "rope_scaling_keys": dict(alignment=32, rope_scaling_keys=True),
    "no_head_dim_key": dict(alignment=32, head_dim_key=False),
}


@pytest.mark.parametrize("wtype", ["Q8_0", "Q4_0"])
@pytest.mark.parametrize("variant", sorted(LLAMACPP_VARIANTS))
def test_llamacpp_layout_inspects(tmp_path, wtype, variant):
    """Files in llama.cpp's layout (its metadata set, token and merge arrays,
    rope_freqs.weight, general.alignment padding) read to the same config as
    the synthetic model they were rewritten from (config.rs:29-73): the
    vocabulary comes from tokenizer.ggml.tokens when llama.vocab_size is
    absent, head_dim from dim / heads when rope.dimension_count is absent, and
    the llama3 RoPE table from the defaults or equal keys."""
    from llamacpp_gguf import rewrite_llamacpp
    src = str(tmp_path / "src.gguf")
    sqhip.write_synthetic_gguf(src, wtype, seed=3, **SMALL)
    dst = str(tmp_path / "llamacpp.gguf")
    rewrite_llamacpp(src, dst, **LLAMACPP_VARIANTS[variant])
    code0, want, inv0 = inspect(src)
    code, got, inv = inspect(dst)
    assert code0 == 0 and code == 0, lib().sq_last_error()
    for f in ("n_layers", "dim", "ffn_dim", "n_heads", "n_kv_heads", "head_dim", "vocab", "context_length",
              "bos", "eos", "wtype", "tied_output", "rope_base", "rms_eps", "weight_bytes"):
        assert getattr(got, f) == getattr(want, f), f
    assert np.array_equal(inv, inv0)
    # the fixture itself: every tensor at data_start + offset, aligned as declared
    if variant != "no_alignment_key":
        a = LLAMACPP_VARIANTS[variant]["alignment"]
        raw = np.fromfile(dst, np.uint8)
        g = GGUFFile(src)
        if a == 32:  # the fixed-32 reader restating the reference finds the same bytes
            d = GGUFFile(dst)
            for n in g.tensors:
                assert np.array_equal(d.tensor_bytes(n), g.tensor_bytes(n)), n
        assert len(raw) % a == 0


@pytest.mark.parametrize("bad", [("u32", 48), ("u32", 0), ("f32", 32.0)])
def test_llamacpp_bad_alignment_is_a_format_error(tmp_path, bad):
    """general.alignment must be a power-of-two u32 (as llama.cpp requires)."""
    w = full_model(base_meta(Writer()))
    if bad[0] == "u32":
        w.u32("general.alignment", bad[1])
    else:
        w.f32("general.alignment", bad[1])
    code, _, _ = inspect(write(tmp_path, w.bytes()))
    assert code == 17 and "alignment" in lib().sq_last_error().decode()


# ----------------------------------------------------------- argument checks

def test_operator_shape_errors_without_device():
    L = lib()
    assert L.sq_sdpa(None, None, None, None, 1, 1, 3, 2, 2) == 1           # bad group ratio
    assert L.sq_sdpa(None, None, None, None, 2, 1, 1, 1, 2) == 1           # seq_k < seq_q
    assert L.sq_sdpa(None, None, None, None, 1, 1, 1, 0, 2) == 1           # no kv heads
    assert L.sq_softmax(None, None, 0) == 3                                 # EmptyInput
    assert L.sq_rms_norm(None, None, None, 1, 0, 1e-5) == 1
    assert L.sq_rope_rows(None, 1, 96, 0, None, 32) == 1                    # 96 % 64
    assert L.sq_rope_rows(None, 1, 64, 0, None, 0) == 1                     # empty table
    assert L.sq_quantize_row_q8_0(None, 33, None) == 1
    blk = np.zeros(2, O.BLOCK_Q8_0)
    h = C.c_void_p()
    assert L.sq_weight_upload(8, blk.ctypes.data, 1, 40, C.byref(h)) == 1   # k not a block multiple
    assert L.sq_weight_upload(0, blk.ctypes.data, 1, 64, C.byref(h)) == 2   # F32 is not a weight type
    assert L.sq_forward(None, None, None, 0) == 22
    assert b"ShapeMismatch" in L.sq_last_error() or L.sq_last_error()


def test_bench_refuses_more_than_one_gpu():
    import subprocess
    import sys
    repo = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, os.path.join(repo, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2 and "one GPU" in r.stderr
