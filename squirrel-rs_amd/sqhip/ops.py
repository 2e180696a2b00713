"""Operator-level API on device buffers, mirroring src/ops/ of the reference.

Each function takes DeviceArray arguments (HBM), validates shapes the way the
reference's op does and raises KernelError with the same kind on failure.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from ._lib import SQ_CTX_F32_ACTS, check, lib

BLOCK_Q8_0 = np.dtype([("d", "<u2"), ("qs", "i1", (32,))])
BLOCK_Q4_0 = np.dtype([("d", "<u2"), ("qs", "u1", (16,))])


class DeviceArray:
    """A device allocation with a numpy dtype and shape (plumbing only)."""

    def __init__(self, shape, dtype=np.float32):
        self.shape = tuple(int(s) for s in (shape if isinstance(shape, (tuple, list)) else (shape,)))
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape, dtype=np.int64)) * self.dtype.itemsize
        p = C.c_void_p()
        check(lib().sq_malloc(C.byref(p), max(self.nbytes, 1)))
        self.ptr = p.value

    @classmethod
    def from_numpy(cls, a: np.ndarray) -> "DeviceArray":
        a = np.ascontiguousarray(a)
        d = cls(a.shape, a.dtype)
        if a.nbytes:
            check(lib().sq_memcpy_h2d(d.ptr, a.ctypes.data, a.nbytes))
        return d

    def numpy(self) -> np.ndarray:
        out = np.empty(self.shape, self.dtype)
        if self.nbytes:
            check(lib().sq_memcpy_d2h(out.ctypes.data, self.ptr, self.nbytes))
        return out

    @property
    def size(self) -> int:
        return int(np.prod(self.shape, dtype=np.int64))

    def free(self) -> None:
        if self.ptr:
            lib().sq_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Weight:
    """A weight matrix in the device layout: `rows` rows of k/32 GGUF blocks
    (the WeightBlock extension point, src/kernels/tensor.rs:37-69)."""

    def __init__(self, wtype: int, blocks: np.ndarray, rows: int, k: int):
        self.wtype, self.rows, self.k = wtype, rows, k
        b = np.ascontiguousarray(blocks)
        h = C.c_void_p()
        check(lib().sq_weight_upload(wtype, b.ctypes.data, rows, k, C.byref(h)))
        self.h = h.value

    def __del__(self):
        try:
            if self.h:
                lib().sq_weight_free(self.h)
                self.h = None
        except Exception:
            pass


def quantize_row_q8_0(x: DeviceArray) -> np.ndarray:
    """quantize_row_q8_0 (src/kernels/dot_prod.rs:10-31); returns GGUF blocks."""
    out = DeviceArray((x.size // 32,), BLOCK_Q8_0)
    check(lib().sq_quantize_row_q8_0(x.ptr, x.size, out.ptr))
    return out.numpy()


def linear(x: DeviceArray, w: Weight, out: DeviceArray, f32_acts: bool = False) -> None:
    """linear (src/ops/linear.rs:26-70): out[m, rows] = x[m, k] @ W."""
    if len(x.shape) != 2 or len(out.shape) != 2 or x.shape[1] != w.k or out.shape != (x.shape[0], w.rows):
        _shape_error()
    check(lib().sq_linear(x.ptr, x.shape[0], x.shape[1], w.h, out.ptr,
                          SQ_CTX_F32_ACTS if f32_acts else 0))


def _shape_error() -> int:
    from ._lib import KernelError
    raise KernelError(1, "ShapeMismatch")


def linear_shared(x: DeviceArray, weights: list[Weight], outs: list[DeviceArray],
                  f32_acts: bool = False) -> None:
    """linear_shared (src/ops/linear.rs:73-168)."""
    if len(weights) != len(outs) or not weights:
        _shape_error()
    for w, o in zip(weights, outs):
        if o.shape != (x.shape[0], w.rows):
            _shape_error()
    ws = (C.c_void_p * len(weights))(*[w.h for w in weights])
    os_ = (C.c_void_p * len(outs))(*[o.ptr for o in outs])
    check(lib().sq_linear_shared(x.ptr, x.shape[0], x.shape[1], ws, os_, len(weights),
                                 SQ_CTX_F32_ACTS if f32_acts else 0))


def block_isums(act_blocks: DeviceArray, w: Weight, row: int) -> np.ndarray:
    out = DeviceArray((w.k // 32,), np.int32)
    check(lib().sq_block_isums(act_blocks.ptr, w.h, row, out.ptr))
    return out.numpy()


def embed(tokens: DeviceArray, table: Weight, out: DeviceArray) -> None:
    """embed (src/ops/embedding.rs:10-52)."""
    check(lib().sq_embed(tokens.ptr, tokens.size, table.h, out.ptr))


def rms_norm(x: DeviceArray, w: DeviceArray, out: DeviceArray, eps: float) -> None:
    """rms_norm (src/ops/rms_norm.rs:13-43): normalizes along the last axis."""
    if x.shape != out.shape or not x.shape or w.shape != (x.shape[-1],):
        _shape_error()
    dim = x.shape[-1]
    check(lib().sq_rms_norm(x.ptr, w.ptr, out.ptr, x.size // dim if dim else 0, dim, eps))


def rope_rows(t: DeviceArray, base_position: int, inv_freq: np.ndarray) -> None:
    """rope_rows (src/ops/rope.rs:6-32), in place."""
    inv = np.ascontiguousarray(inv_freq, dtype=np.float32)
    if not t.shape:
        _shape_error()
    rows = t.shape[0]
    row_dim = t.size // rows if rows else 0
    check(lib().sq_rope_rows(t.ptr, rows, row_dim, base_position, inv.ctypes.data, inv.size))


def sdpa_cached(q: DeviceArray, k: DeviceArray, v: DeviceArray, out: DeviceArray, n_heads: int,
                n_kv_heads: int, head_dim: int) -> None:
    """sdpa_cached (src/ops/sdpa.rs:8-38): seq lengths derived from sizes."""
    if n_kv_heads == 0 or head_dim == 0:
        _shape_error()
    qpt, kvpt = n_heads * head_dim, n_kv_heads * head_dim
    if q.size % qpt or k.size % kvpt or v.size != k.size or out.size != q.size:
        _shape_error()
    check(lib().sq_sdpa(q.ptr, k.ptr, v.ptr, out.ptr, q.size // qpt, k.size // kvpt, n_heads,
                        n_kv_heads, head_dim))


def silu(t: DeviceArray) -> None:
    check(lib().sq_silu(t.ptr, t.size))


def elementwise_mul(a: DeviceArray, b: DeviceArray, out: DeviceArray) -> None:
    if a.shape != b.shape or a.shape != out.shape:
        _shape_error()
    check(lib().sq_elementwise_mul(a.ptr, b.ptr, out.ptr, a.size))


def elementwise_add(a: DeviceArray, b: DeviceArray) -> None:
    if a.shape != b.shape:
        _shape_error()
    check(lib().sq_elementwise_add(a.ptr, b.ptr, a.size))


def softmax(a: DeviceArray, out: DeviceArray) -> None:
    if a.size != out.size:
        _shape_error()
    check(lib().sq_softmax(a.ptr, out.ptr, a.size))


def gemm_counters(reset: bool = False) -> dict:
    """Matrix-core matmul launches since the last reset (sq_gemm_counters)."""
    out = np.zeros(6, np.uint64)
    check(lib().sq_gemm_counters(1 if reset else 0, out.ctypes.data))
    return {"launches": int(out[0]), "split_launches": int(out[1]), "tile128_launches": int(out[2]),
            "max_splits": int(out[3]), "tile128x64_launches": int(out[4]), "rows_launches": int(out[5])}


def log_softmax_at(logits: DeviceArray, idx: int) -> float:
    """log p(idx) under softmax(logits) in f64 (perplexity.rs:112-117)."""
    v = C.c_double()
    check(lib().sq_log_softmax_at(logits.ptr, logits.size, idx, C.byref(v)))
    return v.value


def greedy(logits: DeviceArray) -> int:
    """GreedySampler::sample (src/samplers/greedy.rs:6-15) on the device."""
    t = C.c_uint32()
    check(lib().sq_greedy(logits.ptr, logits.size, C.byref(t)))
    return t.value
