"""Model-level API, mirroring the reference's Model / ModelContext /
GreedySampler / TextTokenGenerator (src/models/common/model.rs:6-26,
context.rs:9-27, src/samplers/greedy.rs, src/text_generator.rs) on token ids.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

from ._lib import (SQ_CTX_F32_ACTS, SQ_CTX_MULTI_KERNEL, SQ_CTX_NO_GRAPH, SQ_GEN_IGNORE_EOS, SQ_GEN_NO_KV_CACHE,
                   ModelInfo, SynthSpec, check, lib)
from .ops import BLOCK_Q8_0

WTYPES = {"Q8_0": 8, "Q4_0": 2, "BF16": 30}

# Llama-3.2-1B architecture (the benchmark workloads).
LLAMA_1B = dict(n_layers=16, dim=2048, ffn_dim=8192, n_heads=32, n_kv_heads=8, vocab=128256,
                context_length=131072)


def write_synthetic_gguf(path: str, wtype="Q8_0", seed: int = 0, std_dev: float = 0.02,
                         rope_base: float = 500000.0, rms_eps: float = 1e-5, bos: int = 128000,
                         eos: int = 128009, **dims) -> str:
    """Seeded random-init Llama GGUF (tied embeddings, norm gains 1.0)."""
    d = dict(LLAMA_1B)
    d.update(dims)
    wt = WTYPES[wtype] if isinstance(wtype, str) else int(wtype)
    spec = SynthSpec(d["n_layers"], d["dim"], d["ffn_dim"], d["n_heads"], d["n_kv_heads"],
                     d["vocab"], d["context_length"], wt, seed, std_dev, rope_base, rms_eps, bos,
                     eos)
    check(lib().sq_synth_write_gguf(os.fsencode(path), C.byref(spec)))
    return path


class GreedySampler:
    """GreedySampler::sample (src/samplers/greedy.rs:6-15) on host logits:
    Iterator::max_by with NaN compared as Equal (ties go to the last index)."""

    @staticmethod
    def sample(logits) -> int:
        best = 0
        for i in range(1, len(logits)):
            a, b = logits[best], logits[i]
            if not (a > b):
                best = i
        return best


class Llama3_2:
    """Llama3_2::from_gguf (src/models/llama/model.rs:20-32), weights in HBM."""

    def __init__(self, path: str):
        h = C.c_void_p()
        check(lib().sq_model_load_gguf(os.fsencode(path), C.byref(h)))
        self.h = h.value
        info = ModelInfo()
        check(lib().sq_model_info_get(self.h, C.byref(info)))
        self.info = info
        self.vocab = info.vocab
        self.dim = info.dim

    @classmethod
    def from_gguf(cls, path: str) -> "Llama3_2":
        return cls(path)

    def rope_inv_freq(self) -> np.ndarray:
        out = np.zeros(self.info.head_dim // 2, np.float32)
        check(lib().sq_model_rope_inv_freq(self.h, out.ctypes.data, out.size))
        return out

    def new_context(self, max_positions: int = 4096, f32_acts: bool = False,
                    graph: bool = True, persistent: bool = True) -> "ModelContext":
        """persistent=False selects the one-kernel-per-op decode step."""
        return ModelContext(self, max_positions, f32_acts, graph, persistent)

    def forward(self, token_ids, ctx: "ModelContext") -> None:
        ctx.forward(token_ids)

    def eos_token_id(self) -> int:
        return self.info.eos

    def bos_token_id(self) -> int:
        return self.info.bos

    def close(self) -> None:
        if self.h:
            lib().sq_model_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class ModelContext:
    """KV cache + workspace on the device (src/models/common/context.rs)."""

    def __init__(self, model: Llama3_2, max_positions: int, f32_acts: bool, graph: bool,
                 persistent: bool = True):
        self.model = model
        flags = ((SQ_CTX_F32_ACTS if f32_acts else 0) | (0 if graph else SQ_CTX_NO_GRAPH)
                 | (0 if persistent else SQ_CTX_MULTI_KERNEL))
        h = C.c_void_p()
        check(lib().sq_ctx_new(model.h, max_positions, flags, C.byref(h)))
        self.h = h.value
        self.max_positions = max_positions

    def forward(self, token_ids) -> None:
        ids = np.ascontiguousarray(token_ids, dtype=np.uint32)
        check(lib().sq_forward(self.model.h, self.h, ids.ctypes.data, ids.size))
        self._last_rows = ids.size

    def act_taps(self, enable: bool = True) -> None:
        """Record the quantized activations of every site of each forward."""
        check(lib().sq_ctx_act_taps(self.h, 1 if enable else 0))

    def act_tap_blocks(self) -> np.ndarray:
        """Q8_0 blocks of every quantization site of the most recent forward
        (the order of sq_ctx_act_tap_read)."""
        i = self.model.info
        rows = self._last_rows
        width = 2 * i.dim + i.n_heads * i.head_dim + i.ffn_dim
        n = (rows * i.n_layers * width + i.dim) // 32
        out = np.zeros(n, BLOCK_Q8_0)
        check(lib().sq_ctx_act_tap_read(self.h, out.ctypes.data, n))
        return out

    def logits(self) -> np.ndarray:
        out = np.empty(self.model.vocab, np.float32)
        check(lib().sq_logits(self.h, out.ctypes.data, out.size))
        return out

    def argmax(self) -> int:
        t = C.c_uint32()
        check(lib().sq_argmax(self.h, C.byref(t)))
        return t.value

    def last_hidden(self) -> np.ndarray:
        out = np.empty(self.model.dim, np.float32)
        check(lib().sq_ctx_last_hidden(self.h, out.ctypes.data, out.size))
        return out

    def debug_act(self) -> tuple[np.ndarray, np.ndarray]:
        normed = np.empty(self.model.dim, np.float32)
        blocks = np.zeros(self.model.dim // 32, BLOCK_Q8_0)
        check(lib().sq_ctx_debug_act(self.h, normed.ctypes.data, blocks.ctypes.data))
        return normed, blocks

    def reset_cache(self) -> None:
        check(lib().sq_ctx_reset(self.h))

    def seq_len(self) -> int:
        return lib().sq_ctx_seq_len(self.h)

    def step_trace(self, enable: bool = True) -> None:
        """Record a per-workgroup timeline of each persistent decode step."""
        check(lib().sq_ctx_step_trace(self.h, 1 if enable else 0))

    def step_trace_read(self) -> np.ndarray:
        """[workgroups, stamps] wall-clock ticks of the most recent step."""
        g, st = C.c_int(), C.c_int()
        check(lib().sq_ctx_step_trace_read(self.h, None, 0, C.byref(g), C.byref(st)))
        out = np.zeros((g.value, st.value), np.uint64)
        check(lib().sq_ctx_step_trace_read(self.h, out.ctypes.data, out.size, C.byref(g), C.byref(st)))
        return out

    @property
    def persistent(self) -> bool:
        """True when decode steps run as one persistent kernel per token."""
        return lib().sq_ctx_decode_kernel(self.h) == 1

    def time_kernel(self, which: int, iters: int) -> tuple[float, int]:
        us = C.c_double()
        b = C.c_uint64()
        check(lib().sq_ctx_time_kernel(self.h, which, iters, C.byref(us), C.byref(b)))
        return us.value, b.value

    def prefill_phases(self, prompt_ids) -> dict:
        """Milliseconds of one batched prefill by phase (sq_ctx_prefill_phases)."""
        ids = np.ascontiguousarray(prompt_ids, dtype=np.uint32)
        ms = np.zeros(4, np.float64)
        check(lib().sq_ctx_prefill_phases(self.h, ids.ctypes.data, ids.size, ms.ctypes.data))
        self._last_rows = ids.size
        return {"matmul": float(ms[0]), "attention": float(ms[1]), "other": float(ms[2]), "total": float(ms[3])}

    def score(self, window_ids, burn: int) -> np.ndarray:
        """One perplexity window (sq_ctx_score, perplexity.rs:61-110): resets
        the cache, prefills window[:burn], then teacher-forces the rest and
        returns log p(window[i]) for i in [burn, len) as float64."""
        ids = np.ascontiguousarray(window_ids, dtype=np.uint32)
        out = np.zeros(max(0, ids.size - burn), np.float64)
        check(lib().sq_ctx_score(self.h, ids.ctypes.data, ids.size, burn, out.ctypes.data))
        self._last_rows = 1
        return out

    def close(self) -> None:
        if self.h:
            lib().sq_ctx_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class TextTokenGenerator:
    """TextTokenGenerator::generate (src/text_generator.rs:38-101) on ids."""

    def __init__(self, model: Llama3_2, ctx: ModelContext):
        self.model, self.ctx = model, ctx

    def generate(self, prompt_ids, max_tokens: int, ignore_eos: bool = False,
                 no_kv_cache: bool = False) -> tuple[list[int], np.ndarray]:
        p = np.ascontiguousarray(prompt_ids, dtype=np.uint32)
        out = np.zeros(max(max_tokens, 1), np.uint32)
        ms = np.zeros(max(max_tokens, 1), np.float64)
        n = C.c_size_t()
        flags = (SQ_GEN_IGNORE_EOS if ignore_eos else 0) | (SQ_GEN_NO_KV_CACHE if no_kv_cache else 0)
        check(lib().sq_generate(self.model.h, self.ctx.h, p.ctypes.data, p.size, max_tokens, flags,
                                out.ctypes.data, C.byref(n), ms.ctypes.data))
        return [int(t) for t in out[:n.value]], ms[:max(n.value, 1 if max_tokens else 0)]
