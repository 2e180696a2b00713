"""The oracle pinned against the reference's own tests and independent maths.

Every check here is independent of the oracle's code: the reference's
known-answer tests (values and inputs copied from its #[test] functions),
closed forms, numpy/float64 recomputations, brute force on small inputs and
library routines (numpy float16 RNE, torch SDPA).  A plausible mistake in the
restatement (a dropped term, a wrong sign or index, round-half-even instead
of half-away, a first-index argmax tie, half-split RoPE pairs) fails one of
them.
"""
import math

import numpy as np
import pytest

from oracle import oracle as O

F32 = np.float32


def rng(s):
    return np.random.default_rng(s)


# ------------------------------------------------------------- f16 / bf16

def test_f32_to_f16_is_ieee_rne():
    """half 2.7.1 f16::from_f32 is IEEE round-to-nearest-even: checked against
    numpy's float16 conversion on every exponent and on the rounding
    boundaries of every f16 value, plus a random sample of all bit patterns."""
    r = rng(0)
    pats = [r.integers(0, 2**32, 2**21, dtype=np.uint64).astype(np.uint32)]
    # all f16 values, and midpoints +-1 f32 ulp between neighbours
    h = np.arange(0, 2**16, dtype=np.uint32).astype(np.uint16)
    hv = h.view(np.float16).astype(np.float32)
    hv = hv[np.isfinite(hv)]
    pats.append(hv.view(np.uint32))
    with np.errstate(over="ignore"):
        nxt = np.nextafter(hv.astype(np.float16), np.float16(np.inf)).astype(np.float32)
    mid = ((hv.astype(np.float64) + nxt.astype(np.float64)) / 2).astype(np.float32)
    for d in (-1, 0, 1):
        pats.append(mid.view(np.uint32).astype(np.int64).__add__(d).astype(np.uint32))
    # subnormal / overflow neighbourhoods
    for e in range(0x60, 0x90):
        base = np.uint32(e << 23)
        pats.append(base + r.integers(0, 2**23, 4096, dtype=np.uint32))
        pats.append((base | np.uint32(0x80000000)) + r.integers(0, 2**23, 1024, dtype=np.uint32))
    x = np.concatenate(pats).view(np.float32)
    x = x[~np.isnan(x)]
    got = O.f32_to_f16_array(x)
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, f"{bad.size} mismatches, first {x[bad[:5]]}"


def test_f16_and_bf16_widening_exact():
    for h in (0x0000, 0x8000, 0x0001, 0x03FF, 0x0400, 0x3C00, 0x7BFF, 0x7C00, 0xFC00, 0xC000):
        assert O.f16_to_f32(h) == float(np.array(h, np.uint16).view(np.float16))


# ------------------------------------------------------------- quantizer

def quantize_numpy(x):
    """quantize_row_q8_0_scalar (dot_prod.rs:21-31) written independently:
    f32 arithmetic via numpy scalars, round half away from zero done in
    float64 on the exact f32 product."""
    x = x.astype(np.float32).reshape(-1, 32)
    with np.errstate(all="ignore"):
        amax = np.nanmax(np.abs(x), axis=1, initial=0.0).astype(np.float32)
        amax = np.where(np.isnan(amax), F32(0), amax)
        scale = (amax / F32(127)).astype(np.float32)
        inv = np.where(scale > 0, F32(1) / np.where(scale > 0, scale, F32(1)), F32(0)).astype(np.float32)
        prod = (x * inv[:, None]).astype(np.float32).astype(np.float64)
        rnd = np.sign(prod) * np.floor(np.abs(prod) + 0.5)
        q = np.clip(rnd, -127, 127)
        q = np.where(np.isnan(q), 0, q).astype(np.int8)
        d = scale.astype(np.float16).view(np.uint16)
    return d, q


def test_quantizer_reference_edge_cases():
    """neon_quantize_matches_scalar (dot_prod.rs:629-654) inputs: all-zero
    block, negative absmax, +-0.5 ties, f32::MAX/2 (scale overflows to inf)."""
    src = (np.sin(np.arange(32 * 6, dtype=F32) * F32(0.37)) * F32(4) - F32(0.5)).astype(F32)
    src[32:64] = 0
    src[64] = -100
    src[96] = 0.5
    src[97] = -0.5
    src[128] = np.finfo(F32).max / 2
    got = O.quantize_row_q8_0(src)
    d, q = quantize_numpy(src)
    assert np.array_equal(got["d"], d) and np.array_equal(got["qs"], q)
    assert got["d"][1] == 0 and not got["qs"][1].any()          # all-zero block
    assert got["qs"][2][0] == -127                                # negative absmax
    # scale = MAX/2/127 is finite in f32 (inv too), but its f16 overflows
    assert got["d"][4] == 0x7C00 and got["qs"][4][0] == 127 and not got["qs"][4][1:].any()


def test_quantizer_ties_round_away_from_zero():
    # amax 127 -> scale 1 -> inv 1: x*inv lands exactly on .5 values
    x = np.zeros(32, F32)
    x[0] = 127
    x[1:9] = [0.5, -0.5, 1.5, -1.5, 2.5, -2.5, 126.5, -126.5]
    q = O.quantize_row_q8_0(x)["qs"][0]
    assert list(q[1:9]) == [1, -1, 2, -2, 3, -3, 127, -127]


@pytest.mark.parametrize("seed", range(4))
def test_quantizer_random_and_special_values(seed):
    r = rng(seed)
    x = (r.standard_normal(32 * 64) * 10 ** r.uniform(-8, 4, 32 * 64)).astype(F32)
    x[::97] = np.nan
    x[5::131] = np.inf
    x[7::173] = -np.inf
    x[40:72] = np.float32(1e-40)
    got = O.quantize_row_q8_0(x)
    d, q = quantize_numpy(x)
    assert np.array_equal(got["d"], d) and np.array_equal(got["qs"], q)


# ------------------------------------------------------------- dot products

def q8_blocks(n, mul, add, scale_step):
    """Deterministic blocks of the reference's tests (dot_prod.rs:560-572)."""
    b = np.zeros(n, O.BLOCK_Q8_0)
    for blk in range(n):
        b["qs"][blk] = [(((i * mul + blk * add) % 251) - 125) for i in range(32)]
        b["d"][blk] = np.float16(scale_step * (blk + 1)).view(np.uint16)
    return b


def q4_blocks(n):
    """test_q4_blocks (dot_prod.rs:702-718)."""
    b = np.zeros(n, O.BLOCK_Q4_0)
    for blk in range(n):
        b["qs"][blk] = [(((i * 7 + blk * 5) % 16) << 4) | ((i + blk * 3) % 16) for i in range(16)]
        b["d"][blk] = np.float16(0.003 * (blk + 1)).view(np.uint16)
    return b


def deq(wtype, blocks):
    return O.dequantize(wtype, blocks, blocks.size * 32)


def test_dot_f32_q8_matches_float64():
    b = q8_blocks(4, 7, 13, 0.001)
    a = (np.sin(np.arange(128, dtype=F32) * F32(0.013)) * F32(3) - F32(1)).astype(F32)
    got = O.dot_f32(a, b, O.Q8_0)
    want = float(a.astype(np.float64) @ deq(O.Q8_0, b).astype(np.float64))
    assert abs(got - want) <= 1e-5 * max(abs(want), 1)


def test_int_dot_close_to_f32():
    """int_dot_close_to_f32 (dot_prod.rs:589-625), scalar twin."""
    b = q8_blocks(8, 5, 11, 0.002)
    a = (np.cos(np.arange(256, dtype=F32) * F32(0.017)) * F32(2.5)).astype(F32)
    ref = O.dot_f32(a, b, O.Q8_0)
    got = O.dot_q8(O.quantize_row_q8_0(a), b, O.Q8_0)
    assert abs(got - ref) <= 1e-2 * max(abs(ref), 1)


def test_q8_int_dot_scalar_vs_neon_order():
    """q8_int_dot_scalar_matches_neon (dot_prod.rs:675-686)."""
    acts = q8_blocks(4, 11, 17, 0.002)
    w = q8_blocks(4, 11, 17, 0.002)
    s, n = O.dot_q8(acts, w, O.Q8_0), O.dot_q8(acts, w, O.Q8_0, neon=True)
    assert abs(n - s) <= abs(n) * 1e-5 + 1e-6


def test_q4_int_dot_scalar_vs_neon_order():
    acts = q8_blocks(4, 11, 17, 0.002)
    w = q4_blocks(4)
    s, n = O.dot_q8(acts, w, O.Q4_0), O.dot_q8(acts, w, O.Q4_0, neon=True)
    assert abs(n - s) <= abs(n) * 1e-5 + 1e-6


def test_q4_dequant_matches_dot():
    """q4_dequant_matches_dot (dot_prod.rs:722-742): one-hot activations."""
    b = q4_blocks(2)
    dq = deq(O.Q4_0, b)
    for pos in (0, 1, 15, 16, 17, 31, 32, 63):
        oh = np.zeros(64, F32)
        oh[pos] = 1
        assert abs(O.dot_f32(oh, b, O.Q4_0) - dq[pos]) < 1e-6
    # nibble layout: low nibble is element j, high nibble element j+16
    s = np.float16(b["d"][0].view(np.float16)).astype(np.float32)
    assert dq[3] == s * ((int(b["qs"][0][3]) & 15) - 8)
    assert dq[19] == s * ((int(b["qs"][0][3]) >> 4) - 8)


def test_q4_int_dot_close_to_f32():
    b = q4_blocks(8)
    a = (np.sin(np.arange(256, dtype=F32) * F32(0.019)) * F32(2) + F32(0.3)).astype(F32)
    ref = O.dot_f32(a, b, O.Q4_0)
    got = O.dot_q8(O.quantize_row_q8_0(a), b, O.Q4_0)
    assert abs(got - ref) <= 1e-2 * max(abs(ref), 1)


def test_q4_int_dot_exact_on_integers():
    """q4_int_dot_exact_on_integers (dot_prod.rs:774-803)."""
    qs = np.array([((i % 16) << 4) | (15 - i % 16) for i in range(16)], np.uint8)
    w = np.zeros(1, O.BLOCK_Q4_0)
    w["d"] = np.float16(1.0).view(np.uint16)
    w["qs"][0] = qs
    a = np.zeros(1, O.BLOCK_Q8_0)
    a["d"] = np.float16(1.0).view(np.uint16)
    a["qs"][0] = np.arange(32) - 16
    expected = sum(int(a["qs"][0][j]) * ((int(qs[j]) & 15) - 8) +
                   int(a["qs"][0][j + 16]) * ((int(qs[j]) >> 4) - 8) for j in range(16))
    assert O.dot_q8(a, w, O.Q4_0) == float(expected)
    assert O.dot_q8(a, w, O.Q4_0, neon=True) == float(expected)


@pytest.mark.parametrize("wtype", [O.Q8_0, O.Q4_0])
def test_block_isums_brute_force(wtype):
    r = rng(wtype)
    a = O.quantize_row_q8_0(r.standard_normal(256).astype(F32))
    if wtype == O.Q8_0:
        w = O.quantize_row_q8_0(r.standard_normal(256).astype(F32))
        wq = w["qs"].astype(np.int64)
    else:
        w = q4_blocks(8)
        wq = np.concatenate([(w["qs"] & 15).astype(np.int64) - 8, (w["qs"] >> 4).astype(np.int64) - 8], axis=1)
    want = (a["qs"].astype(np.int64) * wq).sum(axis=1)
    assert np.array_equal(O.block_isums(a, w, wtype), want)


def test_bf16_dequant_matches_dot():
    """bf16_dequant_matches_dot (dot_prod.rs:836-856)."""
    vals = np.array([math.sin(i * 0.11 + blk) * 2.5 for blk in range(2) for i in range(32)], F32)
    u = vals.view(np.uint32)
    b = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    dq = deq(O.BF16, b)
    for pos in (0, 1, 15, 16, 31, 32, 63):
        oh = np.zeros(64, F32)
        oh[pos] = 1
        assert abs(O.dot_f32(oh, b, O.BF16) - dq[pos]) < 1e-6


# ------------------------------------------------------------- matmul

def bf16_weights(b_cols, a_cols):
    """bf16_weights (matmul.rs:187-197)."""
    v = np.array([math.cos((blk * 32 + i) * 0.011) * 0.4 for blk in range(b_cols * a_cols // 32)
                  for i in range(32)], F32)
    u = v.view(np.uint32)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16).reshape(b_cols, a_cols)


def acts(a_rows, a_cols):
    return (np.sin(np.arange(a_rows * a_cols, dtype=F32) * F32(0.037)) * F32(2) - F32(0.5)).reshape(a_rows, a_cols)


@pytest.mark.parametrize("shape", [(1, 128, 7), (5, 96, 9)])
def test_matmul_matches_naive(shape):
    """matches_naive_single_row / multi_row (matmul.rs:234-253)."""
    m, k, n = shape
    w = bf16_weights(n, k)
    a = acts(m, k)
    got = O.linear(a, O.BF16, w, n, O.W8A32)
    wf = (w.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    want = a.astype(np.float64) @ wf.T
    assert np.all(np.abs(got - want) <= 1e-4 * np.maximum(np.abs(want), 1))


def test_prequant_path_close_to_f32_path():
    """prequant_path_close_to_f32_path (matmul.rs:283-336): error bounded by
    5e-3 of the magnitude of the terms."""
    a_rows, a_cols, b_cols = 2, 128, 6
    a = acts(a_rows, a_cols)
    w = q8_blocks(b_cols * (a_cols // 32), 7, 13, 0.001).reshape(b_cols, a_cols // 32)
    want = O.linear(a, O.Q8_0, w, b_cols, O.W8A32)
    got = O.linear(a, O.Q8_0, w, b_cols, O.W8A8)
    wf = np.stack([deq(O.Q8_0, w[c]) for c in range(b_cols)])
    mag = np.abs(a.astype(np.float64)) @ np.abs(wf.astype(np.float64)).T
    assert np.all(np.abs(got - want) <= 5e-3 * mag)


# ------------------------------------------------------------- pointwise

def test_softmax_reference_tests():
    """softmax.rs:39-85."""
    st, out = O.softmax([1, 2, 3])
    assert st == 0 and abs(out.sum() - 1) < 1e-6 and np.all(out > 0)
    assert np.allclose(out, [0.09003057, 0.24472847, 0.66524096], atol=1e-6)
    st, out = O.softmax([100, 101])
    assert np.all(np.isfinite(out)) and abs(out.sum() - 1) < 1e-6 and out[1] > out[0]
    st, out = O.softmax([0.1, -5.0, 3.7, 2.0])
    assert int(np.argmax(out)) == 2
    assert O.softmax(np.zeros(0, F32))[0] == O.EMPTY


def test_rms_norm_reference_tests():
    """rms_norm.rs:86-141."""
    x = np.array([1, 2, 3, 4], F32)
    out = O.rms_norm(x, np.ones(4, F32), 0.0)[0]
    assert np.allclose(out, x / np.sqrt(7.5), atol=1e-5)
    z = O.rms_norm(np.zeros(4, F32), np.ones(4, F32), 1e-5)[0]
    assert np.all(np.isfinite(z)) and np.all(z == 0)
    assert np.allclose(O.rms_norm(x, np.full(4, 2, F32), 0.0)[0], 2 * out, atol=1e-5)
    w = np.array([0.5, 1.0, 1.5, 2.0], F32)
    want = x * w / np.sqrt((x.astype(np.float64) ** 2).mean() + 1e-5)
    assert np.allclose(O.rms_norm(x, w, 1e-5)[0], want, atol=1e-5)


def test_sigmoid_silu():
    for x in (-100.0, -20.0, -1.0, -0.0, 0.0, 0.5, 3.0, 30.0, 100.0):
        want = 1 / (1 + math.exp(-x)) if x > -700 else 0.0
        assert abs(O.sigmoid(x) - want) <= 2e-7 * want + 1e-40
    x = np.linspace(-30, 30, 601).astype(F32)
    want = x.astype(np.float64) / (1 + np.exp(-x.astype(np.float64)))
    assert np.allclose(O.silu(x), want, rtol=1e-6, atol=1e-30)
    assert O.silu(np.array([-100.0], F32))[0] < 0  # stable branch keeps the tiny value


def test_rope_interleaved_pairs():
    """rope_f32_interleaved (rope.rs:7-36) against a float64 rotation of
    adjacent pairs; half-split pairing or a sign flip fails."""
    inv = O.rope_inv_freq(64, 500000.0)
    t = rng(2).standard_normal((3, 128)).astype(F32)
    st, got = O.rope_rows(t, 7, inv)
    assert st == 0
    want = t.astype(np.float64).copy()
    for r in range(3):
        for h in range(2):
            for j in range(32):
                th = np.float64(F32(7 + r) * inv[j])
                a, b = want[r, h * 64 + 2 * j], want[r, h * 64 + 2 * j + 1]
                want[r, h * 64 + 2 * j] = a * math.cos(th) - b * math.sin(th)
                want[r, h * 64 + 2 * j + 1] = a * math.sin(th) + b * math.cos(th)
    assert np.allclose(got, want, atol=2e-6)
    assert O.rope_rows(np.zeros((1, 96), F32), 0, inv)[0] == O.SHAPE


def test_rope_inv_freq_llama3():
    """compute_rope_inv_freq (config.rs:83-127) against the HF llama3 formula
    in float64; inv_freq[0] = 1 exactly; low frequencies are divided by 32."""
    got = O.rope_inv_freq(64, 500000.0)
    base = 500000.0 ** (-np.arange(0, 64, 2) / 64.0)
    lw, hw = 8192 / 1.0, 8192 / 4.0
    want = []
    for f in base:
        wl = 2 * math.pi / f
        if wl > lw:
            want.append(f / 32)
        elif wl >= hw:
            s = (8192 / wl - 1) / (4 - 1)
            want.append((1 - s) * f / 32 + s * f)
        else:
            want.append(f)
    want = np.array(want)
    assert got[0] == 1.0
    assert np.allclose(got, want, rtol=2e-6, atol=0)
    assert got[-1] < base[-1] / 31  # scaled


# ------------------------------------------------------------- attention

def sdpa(q, k, v, sq_, sk, nh, nkv, hd):
    st, out = O.sdpa(np.array(q, F32), np.array(k, F32), np.array(v, F32), sq_, sk, nh, nkv, hd)
    return st, out


def test_attention_reference_tests():
    """attention.rs:84-171."""
    st, out = sdpa([0.5, -1.0, 2.0, 0.25], [0.5, -1.0, 2.0, 0.25], [7, 8, 9, 10], 1, 1, 1, 1, 4)
    assert st == 0 and np.allclose(out, [7, 8, 9, 10], atol=1e-5)
    q, k = [1.0, 0.0, 0.5, 0.5], [1.0, 0.0, 0.0, 1.0]
    _, a = sdpa(q, k, [3, 4, 99, -99], 2, 2, 1, 1, 2)
    _, b = sdpa(q, k, [3, 4, -42, 1234], 2, 2, 1, 1, 2)
    assert np.allclose(a[:2], b[:2], atol=1e-5) and np.allclose(a[:2], [3, 4], atol=1e-5)
    _, o = sdpa([1, 0, 1, 0, 0, 1, 0, 1], [1, 1, 0.5, -0.5], [10, 20, 30, 40], 1, 1, 4, 2, 2)
    assert np.allclose(o[0:2], o[2:4]) and np.allclose(o[4:6], o[6:8])
    _, o = sdpa([0.1, 0.2, 0.3, 0.4], [1, 0, -1, 2], [5, 6, 7, 8], 1, 1, 2, 2, 2)
    assert np.allclose(o, [5, 6, 7, 8], atol=1e-5)
    assert sdpa(np.zeros(6), np.zeros(6), np.zeros(6), 1, 1, 3, 2, 2)[0] == O.SHAPE


def test_attention_matches_torch():
    """Causal GQA with bottom-right alignment (seq_q < seq_k) vs torch SDPA
    in float64 with an explicit mask."""
    torch = pytest.importorskip("torch")
    sq_, sk, nh, nkv, hd = 5, 9, 8, 2, 16
    r = rng(4)
    q = r.standard_normal((sq_, nh, hd)).astype(F32)
    k = r.standard_normal((sk, nkv, hd)).astype(F32)
    v = r.standard_normal((sk, nkv, hd)).astype(F32)
    st, got = sdpa(q.ravel(), k.ravel(), v.ravel(), sq_, sk, nh, nkv, hd)
    assert st == 0
    tq = torch.tensor(q, dtype=torch.float64).permute(1, 0, 2)
    tk = torch.tensor(k, dtype=torch.float64).permute(1, 0, 2).repeat_interleave(nh // nkv, 0)
    tv = torch.tensor(v, dtype=torch.float64).permute(1, 0, 2).repeat_interleave(nh // nkv, 0)
    mask = torch.ones(sq_, sk, dtype=torch.bool).tril(diagonal=sk - sq_)
    want = torch.nn.functional.scaled_dot_product_attention(tq, tk, tv, attn_mask=mask)
    want = want.permute(1, 0, 2).reshape(-1).numpy()
    assert np.allclose(got, want, atol=2e-6)


# ------------------------------------------------------------- greedy

def test_greedy_reference_semantics():
    """greedy.rs:21-31 plus the Iterator::max_by rules: ties go to the last
    index; a NaN comparison hands the lead to the later element."""
    nan = float("nan")
    assert O.greedy([0.1, -2.3, 5.7, 4.0]) == 2
    assert O.greedy([1.0, nan, 3.0, 2.0]) == 2
    assert O.greedy([3.0, 1.0, 3.0, 2.0]) == 2
    assert O.greedy([5.0, nan, 1.0]) == 2
    assert O.greedy([1.0, 3.0, nan]) == 2
    assert O.greedy([-0.0, 0.0, -0.0]) == 2


def max_by_reference(xs):
    """Rust's Iterator::max_by(partial_cmp, NaN -> Equal) spelled out."""
    best = 0
    for i in range(1, len(xs)):
        a, b = xs[best], xs[i]
        greater = (not math.isnan(a)) and (not math.isnan(b)) and a > b
        if not greater:
            best = i
    return best


@pytest.mark.parametrize("seed", range(20))
def test_greedy_random_with_nans(seed):
    r = rng(seed)
    x = np.round(r.standard_normal(50) * 2).astype(F32)
    if seed % 2:
        x[r.integers(0, 50, 3)] = np.nan
    assert O.greedy(x) == max_by_reference(list(map(float, x)))


# ------------------------------------------------------------- full model

def numpy_llama(path, ids_steps):
    """Independent float64 Llama forward over dequantized weights: checks the
    oracle's model wiring (embed, pre-norms, interleaved RoPE, GQA causal
    attention, SwiGLU, residuals, final norm, tied head)."""
    from oracle.gguf_reader import GGUFFile
    g = GGUFFile(path)
    cfg = O.LlamaConfig(g)
    D, H, KV, hd, L = cfg.embed_dim, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim, cfg.n_blocks

    def mat(name):
        info = g.tensors[name]
        k, n = info.dims
        raw = g.tensor_bytes(name)
        blocks = np.frombuffer(raw.tobytes(), O.BLOCK_Q8_0).reshape(n, k // 32)
        return np.stack([O.dequantize(O.Q8_0, blocks[i], k) for i in range(n)]).astype(np.float64)

    def vec(name):
        return np.frombuffer(g.tensor_bytes(name).tobytes(), np.float32).astype(np.float64)

    emb = mat("token_embd.weight")
    W = [{n: (vec if "norm" in n else mat)(f"blk.{i}.{n}.weight") for n in O.LAYER_NAMES} for i in range(L)]
    inv = cfg.inv_freq.astype(np.float64)

    def norm(x, w):
        return x / np.sqrt((x * x).mean(-1, keepdims=True) + cfg.rms_eps) * w

    def rope(x, pos):
        x = x.copy()
        for j in range(hd // 2):
            th = pos[:, None] * inv[j]
            a, b = x[..., 2 * j].copy(), x[..., 2 * j + 1].copy()
            x[..., 2 * j] = a * np.cos(th) - b * np.sin(th)
            x[..., 2 * j + 1] = a * np.sin(th) + b * np.cos(th)
        return x

    kc = [np.zeros((0, KV, hd)) for _ in range(L)]
    vc = [np.zeros((0, KV, hd)) for _ in range(L)]
    outs, p0 = [], 0
    for ids in ids_steps:
        ids = np.atleast_1d(ids)
        n = len(ids)
        pos = np.arange(p0, p0 + n, dtype=np.float64)
        h = emb[ids]
        for i in range(L):
            w = W[i]
            x = norm(h, w["attn_norm"])
            q = rope((x @ w["attn_q"].T).reshape(n, H, hd), pos)
            k = rope((x @ w["attn_k"].T).reshape(n, KV, hd), pos)
            v = (x @ w["attn_v"].T).reshape(n, KV, hd)
            kc[i] = np.concatenate([kc[i], k])
            vc[i] = np.concatenate([vc[i], v])
            att = np.zeros((n, H, hd))
            for t in range(n):
                for hh in range(H):
                    g_ = hh // (H // KV)
                    s = kc[i][: p0 + t + 1, g_] @ q[t, hh] / math.sqrt(hd)
                    p = np.exp(s - s.max())
                    att[t, hh] = (p / p.sum()) @ vc[i][: p0 + t + 1, g_]
            h = h + att.reshape(n, -1) @ w["attn_output"].T
            x = norm(h, w["ffn_norm"])
            gte, up = x @ w["ffn_gate"].T, x @ w["ffn_up"].T
            h = h + (gte / (1 + np.exp(-gte)) * up) @ w["ffn_down"].T
        p0 += n
        outs.append(norm(h[-1], vec("output_norm.weight")) @ emb.T)
    return outs


def test_oracle_model_matches_float64_llama(tmp_path):
    import sqhip
    path = str(tmp_path / "m.gguf")
    sqhip.write_synthetic_gguf(path, "Q8_0", seed=11, n_layers=2, dim=128, ffn_dim=256, n_heads=4,
                               n_kv_heads=2, vocab=300, context_length=256)
    steps = [np.array([3, 250, 17, 99, 5], np.uint32), 42, 7]
    want = numpy_llama(path, steps)
    m = O.OracleModel(path)
    c = m.new_context(64, O.W8A32)
    for ids, w in zip(steps, want):
        c.forward(np.atleast_1d(ids))
        got = c.logits()
        assert np.allclose(got, w, rtol=1e-4, atol=2e-5), float(np.abs(got - w).max())
