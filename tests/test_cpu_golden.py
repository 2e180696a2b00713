"""The golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py
from the oracle) against the oracle and against independent restatements.

The oracle must reproduce each fixture bit for bit (it is deterministic C code
built without FMA contraction), so a later edit of the oracle that changes any
result fails here.  The integer parts are also recomputed by brute force in
numpy, and the float parts by float64 numpy closed forms within a stated
tolerance, so a fixture cannot simply freeze an oracle mistake.
"""
import os

import numpy as np
import pytest

from oracle import oracle as O

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    return np.load(os.path.join(GOLDEN, name), allow_pickle=False)


def test_quantizer_fixture():
    f = load("quantize_q8_0.npz")
    for i in range(int(f["n"])):
        x = f[f"x{i}"]
        b = O.quantize_row_q8_0(x)
        assert np.array_equal(b["qs"].reshape(-1), f[f"qs{i}"])
        assert np.array_equal(b["d"], f[f"d{i}"])
        # independent restatement of dot_prod.rs:21-31 in numpy (f32 steps)
        with np.errstate(all="ignore"):  # the f32::MAX/2 block overflows the f16 scale on purpose
            xb = x.reshape(-1, 32)
            amax = np.max(np.abs(xb), axis=1).astype(np.float32)
            scale = (amax / np.float32(127.0)).astype(np.float32)
            inv = np.where(scale > 0, np.float32(1.0) / np.where(scale > 0, scale, 1), 0).astype(np.float32)
            v = (xb * inv[:, None]).astype(np.float32)
            r = np.sign(v) * np.floor(np.abs(v) + np.float32(0.5))  # round half away from zero
            qs = np.clip(r, -127, 127).astype(np.int8)
            d = scale.astype(np.float16).view(np.uint16)
        assert np.array_equal(qs.reshape(-1), f[f"qs{i}"])
        assert np.array_equal(d, f[f"d{i}"])


def unpack(wtype, wbytes, k):
    """Blocks -> (per-block integer weights [kb, 32], per-block f16 scales)."""
    if wtype == O.Q8_0:
        blk = wbytes.view(O.BLOCK_Q8_0)
        return blk["qs"].astype(np.int64), blk["d"].view(np.float16).astype(np.float64)
    blk = wbytes.view(O.BLOCK_Q4_0)
    lo = (blk["qs"] & 15).astype(np.int64) - 8
    hi = (blk["qs"] >> 4).astype(np.int64) - 8
    return np.concatenate([lo, hi], axis=1), blk["d"].view(np.float16).astype(np.float64)


@pytest.mark.parametrize("wtype,name", [(O.Q8_0, "q8_0"), (O.Q4_0, "q4_0")])
@pytest.mark.parametrize("k", [2048, 8192])
def test_row_fixture(wtype, name, k):
    f = load("rows.npz")
    tag = f"{name}_{k}"
    w = f[f"{tag}_w"].view(O.BLOCK_Q8_0 if wtype == O.Q8_0 else O.BLOCK_Q4_0)
    x = f[f"{tag}_x"]
    aq = O.quantize_row_q8_0(x)
    # the oracle reproduces the fixture exactly
    assert np.array_equal(O.block_isums(aq, w, wtype), f[f"{tag}_isums"])
    assert np.float32(O.dot_q8(aq, w, wtype)) == f[f"{tag}_dot_w8a8"]
    assert np.float32(O.dot_f32(x, w, wtype)) == f[f"{tag}_dot_w8a32"]
    # brute-force integer sums and a float64 combine
    qw, dw = unpack(wtype, f[f"{tag}_w"], k)
    qa = aq["qs"].astype(np.int64)
    isums = (qa * qw).sum(axis=1)
    assert np.array_equal(isums, f[f"{tag}_isums"].astype(np.int64))
    da = aq["d"].view(np.float16).astype(np.float64)
    ref = float((isums * da * dw).sum())
    mag = float((np.abs(isums) * np.abs(da) * np.abs(dw)).sum())
    assert abs(float(f[f"{tag}_dot_w8a8"]) - ref) <= 1e-6 * mag
    ref32 = float((x.astype(np.float64).reshape(-1, 32) * qw * dw[:, None]).sum())
    mag32 = float((np.abs(x.astype(np.float64).reshape(-1, 32)) * np.abs(qw) * np.abs(dw[:, None])).sum())
    assert abs(float(f[f"{tag}_dot_w8a32"]) - ref32) <= 1e-6 * mag32


def test_rope_fixture():
    f = load("rope_inv_freq.npz")
    got = O.rope_inv_freq(64, 500000.0, 32.0, 1.0, 4.0, 8192.0)
    assert np.array_equal(got, f["inv_freq"])
    # the HF llama3 scaling formula in float64
    base, factor, low, high, orig = 500000.0, 32.0, 1.0, 4.0, 8192.0
    inv = base ** (-np.arange(0, 64, 2, dtype=np.float64) / 64)
    wl = 2 * np.pi / inv
    smooth = (orig / wl - low) / (high - low)
    want = np.where(wl > orig / low, inv / factor,
                    np.where(wl < orig / high, inv, (1 - smooth) * inv / factor + smooth * inv))
    assert np.allclose(f["inv_freq"], want, rtol=2e-6, atol=0)


def test_sdpa_fixture():
    f = load("sdpa.npz")
    for i in range(int(f["n"])):
        sq_, sk, nh, nkv = (int(v) for v in f[f"case{i}"])
        q, k, v = f[f"q{i}"], f[f"k{i}"], f[f"v{i}"]
        st, out = O.sdpa(q, k, v, sq_, sk, nh, nkv, 64)
        assert st == 0 and np.array_equal(out, f[f"out{i}"])
        # float64 causal GQA attention, bottom-right aligned (attention.rs:11-70)
        Q = q.astype(np.float64).reshape(sq_, nh, 64)
        K = k.astype(np.float64).reshape(sk, nkv, 64)
        V = v.astype(np.float64).reshape(sk, nkv, 64)
        ref = np.zeros((sq_, nh, 64))
        for t in range(sq_):
            n = sk - sq_ + t + 1
            for h in range(nh):
                s = K[:n, h // (nh // nkv)] @ Q[t, h] / 8.0
                p = np.exp(s - s.max())
                ref[t, h] = (p / p.sum()) @ V[:n, h // (nh // nkv)]
        assert np.allclose(out.reshape(sq_, nh, 64), ref, rtol=1e-5, atol=1e-6)


def test_tiny_model_fixture(tmp_path):
    sq = pytest.importorskip("sqhip")
    f = load("tiny_model.npz")
    keys = ("n_layers", "dim", "ffn_dim", "n_heads", "n_kv_heads", "vocab", "context_length")
    dims = {k: int(v) for k, v in zip(keys, f["dims"])}
    path = str(tmp_path / "tiny.gguf")
    sq.write_synthetic_gguf(path, "Q8_0", seed=int(f["model_seed"]), **dims)
    m = O.OracleModel(path)
    for mode, name in ((O.W8A8, "w8a8"), (O.W8A32, "w8a32")):
        c = m.new_context(64, mode)
        c.forward(f["prompt"])
        got = [c.logits()]
        for t in f["steps"]:
            c.forward([int(t)])
            got.append(c.logits())
        assert np.array_equal(np.stack(got), f[f"logits_{name}"])
        assert [O.greedy(x) for x in got] == list(f[f"greedy_{name}"])
