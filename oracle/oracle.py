"""ctypes front end of the oracle (CPU restatement of the reference).

TEST INFRASTRUCTURE ONLY.  Imported by tests/, the smoke() entry and the
bench's cpu_baseline leg, never by the product.  liboracle.so is built by
`make -C oracle` (the build entry point does it).

Model loading restates src/models/llama/config.rs:29-149 (metadata keys,
types and defaults) and src/models/llama/weights.rs:50-97 (tensor names, tied
LM head).
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

from .gguf_reader import F32, U32, ARRAY, GGUFFile

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "liboracle.so")

Q8_0, Q4_0, BF16, F32_T = 8, 2, 30, 0
W8A32, W8A8, W8A8_NEON = 0, 1, 2
OK, SHAPE, INVALID_TYPE, EMPTY, ALIGN = 0, 1, 2, 3, 4

BLOCK_Q8_0 = np.dtype([("d", "<u2"), ("qs", "i1", (32,))])
BLOCK_Q4_0 = np.dtype([("d", "<u2"), ("qs", "u1", (16,))])
assert BLOCK_Q8_0.itemsize == 34 and BLOCK_Q4_0.itemsize == 18


def build() -> str:
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        vp, sz, f32p = C.c_void_p, C.c_size_t, C.POINTER(C.c_float)
        L.or_f32_to_f16.argtypes = [C.c_float]
        L.or_f32_to_f16.restype = C.c_uint16
        L.or_f16_to_f32.argtypes = [C.c_uint16]
        L.or_f16_to_f32.restype = C.c_float
        L.or_f32_to_f16_array.argtypes = [vp, sz, vp]
        L.or_set_threads.argtypes = [C.c_int]
        L.or_quantize_row_q8_0.argtypes = [vp, sz, vp]
        for n in ("or_dot_f32_q8_0", "or_dot_f32_q4_0", "or_dot_f32_bf16", "or_dot_q8_0_q8_0",
                  "or_dot_q8_0_q4_0", "or_dot_q8_0_q8_0_neon", "or_dot_q8_0_q4_0_neon"):
            getattr(L, n).argtypes = [vp, vp, sz]
            getattr(L, n).restype = C.c_float
        L.or_linear.argtypes = [vp, sz, sz, C.c_int, vp, sz, vp, C.c_int]
        L.or_block_isums.argtypes = [vp, C.c_int, vp, sz, vp]
        L.or_softmax.argtypes = [vp, vp, sz]
        L.or_rms_norm_rows.argtypes = [vp, vp, vp, sz, sz, C.c_float]
        L.or_rope_rows.argtypes = [vp, sz, sz, sz, vp, sz]
        L.or_sigmoid.argtypes = [C.c_float]
        L.or_sigmoid.restype = C.c_float
        L.or_silu.argtypes = [vp, sz]
        L.or_rope_inv_freq.argtypes = [sz, C.c_float, C.c_float, C.c_float, C.c_float,
                                       C.c_float, vp]
        L.or_sdpa.argtypes = [vp, vp, vp, vp, sz, sz, sz, sz, sz]
        L.or_greedy.argtypes = [vp, sz]
        L.or_greedy.restype = C.c_int64
        L.or_embed.argtypes = [vp, sz, C.c_int, vp, sz, sz, vp]
        L.or_dot_f32_f32.argtypes = [vp, sz, vp, sz, f32p]
        L.or_ctx_new.argtypes = [vp, sz, C.c_int]
        L.or_ctx_new.restype = vp
        L.or_ctx_free.argtypes = [vp]
        L.or_ctx_reset.argtypes = [vp]
        L.or_ctx_seq_len.argtypes = [vp]
        L.or_ctx_seq_len.restype = sz
        L.or_forward.argtypes = [vp, vp, vp, sz]
        L.or_forward_locked.argtypes = [vp, vp, vp, sz, C.POINTER(OrLock)]
        L.or_ctx_logits.argtypes = [vp]
        L.or_ctx_logits.restype = f32p
        L.or_ctx_last_hidden.argtypes = [vp]
        L.or_ctx_last_hidden.restype = f32p
        _lib = L
    return _lib


def _p(a: np.ndarray):
    return a.ctypes.data_as(C.c_void_p)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def set_threads(n: int) -> int:
    return lib().or_set_threads(int(n))


# ---------------------------------------------------------------- scalars
def f32_to_f16(x: float) -> int:
    return lib().or_f32_to_f16(float(x))


def f16_to_f32(h: int) -> float:
    return lib().or_f16_to_f32(int(h))


def f32_to_f16_array(x: np.ndarray) -> np.ndarray:
    x = _f32(x).ravel()
    out = np.zeros(x.size, dtype=np.uint16)
    lib().or_f32_to_f16_array(_p(x), x.size, _p(out))
    return out


# ---------------------------------------------------------------- blocks
def quantize_row_q8_0(x) -> np.ndarray:
    x = _f32(x).ravel()
    out = np.zeros(x.size // 32, dtype=BLOCK_Q8_0)
    lib().or_quantize_row_q8_0(_p(x), x.size, _p(out))
    return out


def dot_f32(a, w: np.ndarray, wtype: int) -> float:
    a = _f32(a)
    L = lib()
    if wtype == Q8_0:
        return L.or_dot_f32_q8_0(_p(a), _p(w), w.size)
    if wtype == Q4_0:
        return L.or_dot_f32_q4_0(_p(a), _p(w), w.size)
    w = np.ascontiguousarray(w, dtype=np.uint16)
    return L.or_dot_f32_bf16(_p(a), _p(w), w.size)


def dot_q8(aq: np.ndarray, w: np.ndarray, wtype: int, neon: bool = False) -> float:
    L = lib()
    fn = {(Q8_0, False): L.or_dot_q8_0_q8_0, (Q4_0, False): L.or_dot_q8_0_q4_0,
          (Q8_0, True): L.or_dot_q8_0_q8_0_neon, (Q4_0, True): L.or_dot_q8_0_q4_0_neon}
    return fn[(wtype, neon)](_p(aq), _p(w), w.size)


def block_isums(aq: np.ndarray, w_row: np.ndarray, wtype: int) -> np.ndarray:
    out = np.zeros(aq.size, dtype=np.int32)
    st = lib().or_block_isums(_p(aq), wtype, _p(w_row), aq.size, _p(out))
    if st:
        raise ValueError(f"status {st}")
    return out


def dequantize(wtype: int, blocks: np.ndarray, n: int) -> np.ndarray:
    out = np.zeros(n, dtype=np.float32)
    lib_fn = lib().or_embed  # reuse the row dequantizer through a 1-token embed
    st = lib_fn(_p(np.zeros(1, np.uint32)), 1, wtype, _p(np.ascontiguousarray(blocks)), n, 1,
                _p(out))
    if st:
        raise ValueError(f"status {st}")
    return out


def linear(x, wtype: int, w: np.ndarray, n_out: int, mode: int = W8A32) -> np.ndarray:
    """linear (src/ops/linear.rs:26-70): x [m, k] f32, w = n_out rows of blocks."""
    x = _f32(x)
    if x.ndim == 1:
        x = x[None, :]
    m, k = x.shape
    out = np.zeros((m, n_out), dtype=np.float32)
    st = lib().or_linear(_p(x), m, k, wtype, _p(np.ascontiguousarray(w)), n_out, _p(out), mode)
    if st:
        raise ValueError(f"status {st}")
    return out


# ---------------------------------------------------------------- pointwise
def softmax(a) -> tuple[int, np.ndarray]:
    a = _f32(a)
    out = np.zeros_like(a)
    st = lib().or_softmax(_p(a), _p(out), a.size)
    return st, out


def rms_norm(x, w, eps: float) -> np.ndarray:
    x = _f32(x)
    if x.ndim == 1:
        x = x[None, :]
    w = _f32(w)
    out = np.zeros_like(x)
    lib().or_rms_norm_rows(_p(x), _p(w), _p(out), x.shape[0], x.shape[1], eps)
    return out


def rope_rows(t, base_pos: int, inv_freq) -> tuple[int, np.ndarray]:
    t = _f32(t).copy()
    if t.ndim == 1:
        t = t[None, :]
    inv = _f32(inv_freq)
    st = lib().or_rope_rows(_p(t), t.shape[0], t.shape[1], base_pos, _p(inv), inv.size)
    return st, t


def sigmoid(x: float) -> float:
    return lib().or_sigmoid(float(x))


def silu(x) -> np.ndarray:
    x = _f32(x).copy()
    lib().or_silu(_p(x), x.size)
    return x


def rope_inv_freq(head_dim: int, base: float, factor=32.0, low=1.0, high=4.0,
                  orig_ctx=8192.0) -> np.ndarray:
    out = np.zeros(head_dim // 2, dtype=np.float32)
    lib().or_rope_inv_freq(head_dim, base, factor, low, high, orig_ctx, _p(out))
    return out


def sdpa(q, k, v, seq_q, seq_k, n_heads, n_kv_heads, head_dim) -> tuple[int, np.ndarray]:
    q, k, v = _f32(q), _f32(k), _f32(v)
    out = np.zeros(seq_q * n_heads * head_dim, dtype=np.float32)
    if q.size != out.size or k.size != seq_k * n_kv_heads * head_dim or v.size != k.size:
        return SHAPE, out
    st = lib().or_sdpa(_p(q), _p(k), _p(v), _p(out), seq_q, seq_k, n_heads, n_kv_heads,
                       head_dim)
    return st, out


def greedy(logits) -> int:
    a = _f32(logits)
    return int(lib().or_greedy(_p(a), a.size))


def embed(tokens, wtype: int, table: np.ndarray, dim: int, vocab: int) -> np.ndarray:
    t = np.ascontiguousarray(tokens, dtype=np.uint32)
    out = np.zeros((t.size, dim), dtype=np.float32)
    st = lib().or_embed(_p(t), t.size, wtype, _p(np.ascontiguousarray(table)), dim, vocab,
                        _p(out))
    if st:
        raise ValueError(f"status {st}")
    return out


# ---------------------------------------------------------------- the model
class ConfigError(Exception):
    pass


def _read_u32(g: GGUFFile, key: str) -> int:
    """read_u32 (config.rs:129-138): missing -> MissingMetadata, other type ->
    WrongMetadataType."""
    if key not in g.metadata:
        raise ConfigError(f"MissingMetadata({key})")
    t, v = g.metadata[key]
    if t != U32:
        raise ConfigError(f"WrongMetadataType({key}, u32)")
    return v


def _read_f32(g: GGUFFile, key: str) -> float:
    if key not in g.metadata:
        raise ConfigError(f"MissingMetadata({key})")
    t, v = g.metadata[key]
    if t != F32:
        raise ConfigError(f"WrongMetadataType({key}, f32)")
    return v


def _opt(fn, g, key, default):
    try:
        return fn(g, key)
    except ConfigError:
        return default


class LlamaConfig:
    """LlamaConfig::from_gguf (src/models/llama/config.rs:29-73)."""

    def __init__(self, g: GGUFFile):
        self.n_blocks = _read_u32(g, "llama.block_count")
        self.embed_dim = _read_u32(g, "llama.embedding_length")
        self.ffn_dim = _read_u32(g, "llama.feed_forward_length")
        self.n_heads = _read_u32(g, "llama.attention.head_count")
        self.n_kv_heads = _read_u32(g, "llama.attention.head_count_kv")
        self.head_dim = _opt(_read_u32, g, "llama.rope.dimension_count",
                             self.embed_dim // self.n_heads)
        self.rope_base = _read_f32(g, "llama.rope.freq_base")
        self.rms_eps = _read_f32(g, "llama.attention.layer_norm_rms_epsilon")
        self.context_length = _read_u32(g, "llama.context_length")
        self.bos = _read_u32(g, "tokenizer.ggml.bos_token_id")
        self.eos = _read_u32(g, "tokenizer.ggml.eos_token_id")
        try:
            self.vocab = _read_u32(g, "llama.vocab_size")
        except ConfigError:
            tok = g.metadata.get("tokenizer.ggml.tokens")
            if tok is None or tok[0] != ARRAY:
                raise ConfigError("MissingMetadata(llama.vocab_size / tokenizer.ggml.tokens)")
            self.vocab = len(tok[1][1])
        factor = _opt(_read_f32, g, "llama.rope.scaling.factor", 32.0)
        low = _opt(_read_f32, g, "llama.rope.scaling.low_freq_factor", 1.0)
        high = _opt(_read_f32, g, "llama.rope.scaling.high_freq_factor", 4.0)
        orig = float(_opt(_read_u32, g, "llama.rope.scaling.original_context_length", 8192))
        self.inv_freq = rope_inv_freq(self.head_dim, self.rope_base, factor, low, high, orig)


LAYER_NAMES = ("attn_norm", "attn_q", "attn_k", "attn_v", "attn_output", "ffn_norm",
               "ffn_gate", "ffn_up", "ffn_down")


class _Llama(C.Structure):
    _fields_ = [("n_layers", C.c_int), ("dim", C.c_int), ("ffn_dim", C.c_int),
                ("n_heads", C.c_int), ("n_kv_heads", C.c_int), ("head_dim", C.c_int),
                ("vocab", C.c_int), ("eps", C.c_float), ("wtype", C.c_int),
                ("tok_embd", C.c_void_p), ("output", C.c_void_p),
                ("output_norm", C.c_void_p), ("layer", C.POINTER(C.c_void_p)),
                ("inv_freq", C.c_void_p)]


class OrLock(C.Structure):
    """or_lock (oracle.h): the phase lock of a forward's quantization sites."""
    _fields_ = [("blocks", C.c_void_p), ("tol", C.c_float), ("values", C.c_uint64),
                ("flips", C.c_uint64), ("scale_flips", C.c_uint64), ("bad", C.c_uint64),
                ("first_bad_layer", C.c_int), ("first_bad_site", C.c_int),
                ("first_bad_index", C.c_size_t), ("first_bad_dist", C.c_float),
                ("max_flip_dist", C.c_float), ("max_scale_rel", C.c_float),
                ("site_values", C.c_uint64 * 5), ("site_flips", C.c_uint64 * 5),
                ("plant_layer", C.c_int), ("plant_site", C.c_int), ("plant_quanta", C.c_float)]


class OracleModel:
    """Llama3_2 over a GGUF file (model.rs:20-110, weights.rs:50-97)."""

    def __init__(self, path: str):
        self.g = GGUFFile(path)
        self.cfg = c = LlamaConfig(self.g)

        def get(name):
            if name not in self.g.tensors:
                raise KeyError(f"MissingTensor({name})")
            return self.g.tensor_bytes(name)

        self._keep = []
        ptrs = []
        wtype = None
        for i in range(c.n_blocks):
            for nm in LAYER_NAMES:
                t = get(f"blk.{i}.{nm}.weight")
                self._keep.append(t)
                ptrs.append(t.ctypes.data)
                if nm == "attn_q":
                    wtype = self.g.tensors[f"blk.{i}.{nm}.weight"].ggml_type
        emb = get("token_embd.weight")
        norm = get("output_norm.weight")
        out = get("output.weight") if "output.weight" in self.g.tensors else emb
        self.tied = "output.weight" not in self.g.tensors
        self.wtype = wtype
        self._keep += [emb, norm, out]
        self._layer_arr = (C.c_void_p * len(ptrs))(*ptrs)
        self._inv = np.ascontiguousarray(c.inv_freq)
        self.s = _Llama(c.n_blocks, c.embed_dim, c.ffn_dim, c.n_heads, c.n_kv_heads,
                        c.head_dim, c.vocab, c.rms_eps, wtype, emb.ctypes.data,
                        out.ctypes.data, norm.ctypes.data,
                        C.cast(self._layer_arr, C.POINTER(C.c_void_p)), self._inv.ctypes.data)

    def new_context(self, max_positions: int, mode: int = W8A32) -> "OracleContext":
        return OracleContext(self, max_positions, mode)


class OracleContext:
    def __init__(self, model: OracleModel, max_positions: int, mode: int):
        self.m = model
        self.h = lib().or_ctx_new(C.byref(model.s), max_positions, mode)

    def forward(self, ids, lock=None, tol: float = 0.02, plant=None):
        """One Llama3_2::forward.  With `lock` (an implementation's Q8_0
        blocks of every quantization site, oracle.h or_lock order) the
        integer path checks each site against its own quantization and then
        continues with the given blocks; returns the lock's counts.  `plant`
        = (layer, site, quanta) replaces that site's given blocks by the
        oracle's own quantization with every scaled value moved by `quanta`
        (a planted systematic error, for tests of the lock)."""
        ids = np.ascontiguousarray(ids, dtype=np.uint32)
        if lock is None:
            st = lib().or_forward(C.byref(self.m.s), self.h, _p(ids), ids.size)
            if st:
                raise RuntimeError(f"oracle forward status {st}")
            return None
        blocks = np.ascontiguousarray(lock)
        c = self.m.cfg
        width = 2 * c.embed_dim + c.n_heads * c.head_dim + c.ffn_dim
        need = (ids.size * c.n_blocks * width + c.embed_dim) // 32
        if blocks.dtype != BLOCK_Q8_0 or blocks.size != need:
            raise ValueError(f"lock needs {need} Q8_0 blocks, got {blocks.size}")
        lk = OrLock(blocks.ctypes.data, tol)
        if plant is not None:
            lk.plant_layer, lk.plant_site, lk.plant_quanta = int(plant[0]), int(plant[1]), float(plant[2])
        st = lib().or_forward_locked(C.byref(self.m.s), self.h, _p(ids), ids.size, C.byref(lk))
        if st:
            raise RuntimeError(f"oracle forward status {st}")
        return {"values": lk.values, "flips": lk.flips, "scale_flips": lk.scale_flips, "bad": lk.bad,
                "first_bad": (lk.first_bad_layer, lk.first_bad_site, lk.first_bad_index, lk.first_bad_dist)
                if lk.bad else None,
                "max_flip_dist": float(lk.max_flip_dist), "max_scale_rel": float(lk.max_scale_rel),
                "site_values": list(lk.site_values), "site_flips": list(lk.site_flips)}

    def logits(self) -> np.ndarray:
        p = lib().or_ctx_logits(self.h)
        return np.ctypeslib.as_array(p, shape=(self.m.cfg.vocab,)).copy()

    def last_hidden(self) -> np.ndarray:
        p = lib().or_ctx_last_hidden(self.h)
        return np.ctypeslib.as_array(p, shape=(self.m.cfg.embed_dim,)).copy()

    def seq_len(self) -> int:
        return lib().or_ctx_seq_len(self.h)

    def reset(self) -> None:
        lib().or_ctx_reset(self.h)

    def close(self) -> None:
        if self.h:
            lib().or_ctx_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
