"""The device path against the golden fixtures (tests/golden/*.npz, written
from the oracle by tests/golden/make_golden.py), through the C ABI.

Bars: bit-exact for the quantizer and the per-block i32 sums; the row dot
within 4e-6 of the sum of |terms| (summation order differs from the
reference's sequential fold); attention within rtol 1e-5 / atol 2e-6; the
tiny model's logits phase-locked (tests/lock_bar.py): the oracle, locked to
the device's quantized activations, is within 1e-5 relative L2 of the
device's logits at every step, and until the first step at which the lock
accepted a flip the locked oracle's logits equal the fixture's W8A8 logits
bit for bit (before any flip the locked run is the run that wrote them).
"""
import os

import numpy as np
import pytest

from oracle import oracle as O

pytestmark = pytest.mark.gpu

sq = pytest.importorskip("sqhip")
from sqhip import ops  # noqa: E402
from sqhip.ops import DeviceArray  # noqa: E402

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    return np.load(os.path.join(GOLDEN, name), allow_pickle=False)


def test_quantizer_matches_fixture():
    f = load("quantize_q8_0.npz")
    for i in range(int(f["n"])):
        got = ops.quantize_row_q8_0(DeviceArray.from_numpy(f[f"x{i}"]))
        assert np.array_equal(got["qs"].reshape(-1), f[f"qs{i}"]), f"row {i}: quants"
        assert np.array_equal(got["d"], f[f"d{i}"]), f"row {i}: scales"


@pytest.mark.parametrize("wtype,name", [(O.Q8_0, "q8_0"), (O.Q4_0, "q4_0")])
@pytest.mark.parametrize("k", [2048, 8192])
def test_row_matches_fixture(wtype, name, k):
    f = load("rows.npz")
    tag = f"{name}_{k}"
    w = f[f"{tag}_w"].view(O.BLOCK_Q8_0 if wtype == O.Q8_0 else O.BLOCK_Q4_0).reshape(1, k // 32)
    x = f[f"{tag}_x"]
    aq = O.quantize_row_q8_0(x)
    W = ops.Weight(wtype, w, 1, k)
    got = ops.block_isums(DeviceArray.from_numpy(aq), W, 0)
    assert np.array_equal(got, f[f"{tag}_isums"])
    out = DeviceArray((1, 1))
    ops.linear(DeviceArray.from_numpy(x.reshape(1, k)), W, out)
    y = float(out.numpy().reshape(-1)[0])
    isums = f[f"{tag}_isums"].astype(np.float64)
    mag = float(np.sum(np.abs(isums) * np.abs(aq["d"].view(np.float16).astype(np.float64))
                       * np.abs(w["d"].view(np.float16).astype(np.float64).reshape(-1))))
    assert abs(y - float(f[f"{tag}_dot_w8a8"])) <= 4e-6 * mag + 1e-6


def test_sdpa_matches_fixture():
    f = load("sdpa.npz")
    for i in range(int(f["n"])):
        sq_, sk, nh, nkv = (int(v) for v in f[f"case{i}"])
        out = DeviceArray(f[f"q{i}"].size)
        ops.sdpa_cached(DeviceArray.from_numpy(f[f"q{i}"]), DeviceArray.from_numpy(f[f"k{i}"]),
                        DeviceArray.from_numpy(f[f"v{i}"]), out, nh, nkv, 64)
        assert np.allclose(out.numpy(), f[f"out{i}"], rtol=1e-5, atol=2e-6), f"case {i}"


def rel_l2(a, b):
    return float(np.linalg.norm(a.astype(np.float64) - b) / np.linalg.norm(b))


@pytest.mark.parametrize("persistent", [True, False])
def test_tiny_model_matches_fixture(tmp_path, persistent):
    from lock_bar import LOCK_TOL
    f = load("tiny_model.npz")
    keys = ("n_layers", "dim", "ffn_dim", "n_heads", "n_kv_heads", "vocab", "context_length")
    dims = {k: int(v) for k, v in zip(keys, f["dims"])}
    path = str(tmp_path / "tiny.gguf")
    sq.write_synthetic_gguf(path, "Q8_0", seed=int(f["model_seed"]), **dims)
    m = sq.Llama3_2(path)
    c = m.new_context(64, persistent=persistent)
    assert c.persistent == persistent
    c.act_taps(True)
    oc = O.OracleModel(path).new_context(64, O.W8A8)
    flipped = False
    for step, ids in enumerate([f["prompt"]] + [[int(t)] for t in f["steps"]]):
        c.forward(ids)
        g = c.logits()
        st = oc.forward(ids, lock=c.act_tap_blocks(), tol=LOCK_TOL)
        w = oc.logits()
        flipped = flipped or st["flips"] > 0 or st["scale_flips"] > 0
        print(f"step {step}: rel_l2 vs locked oracle {rel_l2(g, w):.2e}, flips {st['flips']}")
        assert st["bad"] == 0, f"step {step}: {st['first_bad']}"
        assert rel_l2(g, w) <= 1e-5, f"step {step}"
        if not flipped:
            assert np.array_equal(w, f["logits_w8a8"][step]), f"step {step}: locked oracle vs fixture"
