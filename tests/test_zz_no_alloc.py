"""sq_linear_noalloc (static per-GPU scratch, no hipMalloc) against sq_linear.

Both entry points run the same kernels with the same K-split workspace size,
so their outputs must be bit-identical.  Two calls in a row, the second with
a smaller input, check that the shared scratch carries nothing from one call
to the next; a third call takes the single-row matvec path.  Inputs beyond
the scratch's size are refused on the host before any kernel runs.
"""
import ctypes as C

import numpy as np
import pytest

from oracle import oracle as O

pytestmark = pytest.mark.gpu

sq = pytest.importorskip("sqhip")
from sqhip import ops  # noqa: E402
from sqhip._lib import SQ_ERR_SHAPE, check, lib  # noqa: E402
from sqhip.ops import DeviceArray  # noqa: E402


def weights(wtype, rows, k, seed):
    x = (np.random.default_rng(seed).standard_normal((rows, k)) * 0.02).astype(np.float32)
    if wtype == O.Q8_0:
        return O.quantize_row_q8_0(x).reshape(rows, k // 32)
    xb = x.reshape(-1, 32)
    idx = np.argmax(np.abs(xb), axis=1)
    mx = xb[np.arange(xb.shape[0]), idx]
    d = (mx / np.float32(-8)).astype(np.float32)
    inv = np.where(d != 0, np.float32(1) / np.where(d != 0, d, 1), 0).astype(np.float32)
    q = np.minimum(15, np.trunc(xb * inv[:, None] + np.float32(8.5)).astype(np.int32))
    blk = np.zeros(xb.shape[0], O.BLOCK_Q4_0)
    blk["d"] = d.astype(np.float16).view(np.uint16)
    blk["qs"] = (q[:, :16] | (q[:, 16:] << 4)).astype(np.uint8)
    return blk.reshape(rows, k // 32)


def both(W, x, n):
    m, k = x.shape
    dx = DeviceArray.from_numpy(x)
    a, b = DeviceArray((m, n)), DeviceArray((m, n))
    check(lib().sq_linear(dx.ptr, m, k, W.h, a.ptr, 0))
    check(lib().sq_linear_noalloc(dx.ptr, m, k, W.h, b.ptr, 0))
    return a.numpy(), b.numpy()


@pytest.mark.parametrize("wtype", [O.Q8_0, O.Q4_0])
def test_noalloc_matches_linear_on_consecutive_calls(wtype):
    k, n = 2048, 512
    W = ops.Weight(wtype, weights(wtype, n, k, seed=5 + wtype), n, k)
    rng = np.random.default_rng(11)
    for m in (67, 5, 1):  # each call smaller than the one before
        x = (rng.standard_normal((m, k)) * 1.5).astype(np.float32)
        ref, got = both(W, x, n)
        print(f"wtype {wtype} m {m}: max|diff| {float(np.abs(ref - got).max()):.3e}")
        assert np.array_equal(ref.view(np.uint32), got.view(np.uint32)), f"m={m}"


def test_noalloc_refuses_inputs_beyond_its_scratch():
    k, n = 2048, 64
    W = ops.Weight(O.Q8_0, weights(O.Q8_0, n, k, seed=3), n, k)
    m = (4 << 20) // k + 1
    dx = DeviceArray((m, k))
    out = DeviceArray((m, n))
    code = lib().sq_linear_noalloc(dx.ptr, m, k, W.h, out.ptr, 0)
    assert code == SQ_ERR_SHAPE
    assert b"static scratch" in lib().sq_last_error()
