"""The error bound of the prefill attention's split-f16 products, on the CPU.

The split-f16 attention kernel forms every f32 operand x as two binary16
halves, hi = f16(x * 2^-8) (round to nearest even) and
lo = f16((x * 2^-8 - hi) * 2^11), and every product a * b as
hi_a hi_b + 2^-11 (hi_a lo_b + lo_a hi_b) accumulated in f32.  The claim
the kernel rests on: each half pair carries x to about 2^-22 relative (an
absolute 2^-33 floor below f16's normal range), and each three-product term
is within about 3 * 2^-22 of the exact product.  numpy's float16 rounds to
nearest even, as the device conversion does; products and sums are formed in
float64 here (the device's products of halves are exact in f32), so this
checks the decomposition's arithmetic, and tests/test_gpu_ops.py checks the
kernel itself against the oracle.
"""
import numpy as np

PRE = np.float32(2.0 ** -8)
UP = np.float32(2.0 ** 11)


def split(x):
    xs = (x.astype(np.float32) * PRE).astype(np.float32)
    hi = xs.astype(np.float16)
    lo = ((xs - hi.astype(np.float32)) * UP).astype(np.float32).astype(np.float16)
    return xs, hi, lo


def test_split_reconstructs_to_2_pow_minus_22():
    rng = np.random.default_rng(7)
    mags = 10.0 ** rng.uniform(-6, 6, 200000)
    x = (mags * rng.choice([-1.0, 1.0], mags.size)).astype(np.float32)
    xs, hi, lo = split(x)
    back = hi.astype(np.float64) + lo.astype(np.float64) * 2.0 ** -11
    err = np.abs(back - xs.astype(np.float64))
    normal = np.abs(xs) >= 2.0 ** -14  # hi a normal f16
    assert np.all(err[normal] <= 2.0 ** -22 * np.abs(xs[normal]).astype(np.float64))
    assert np.all(err[~normal] <= 2.0 ** -35)  # f16 subnormal lo spacing 2^-24, scaled by 2^-11
    assert np.isfinite(hi).all() and np.isfinite(lo).all()


def test_three_products_within_3_pow_minus_22():
    rng = np.random.default_rng(11)
    a = (rng.standard_normal(100000) * 10.0 ** rng.uniform(-3, 3, 100000)).astype(np.float32)
    b = (rng.standard_normal(100000) * 10.0 ** rng.uniform(-3, 3, 100000)).astype(np.float32)
    xa, ha, la = split(a)
    xb, hb, lb = split(b)
    f = lambda h: h.astype(np.float64)  # noqa: E731
    prod = f(ha) * f(hb) + 2.0 ** -11 * (f(ha) * f(lb) + f(la) * f(hb))
    exact = xa.astype(np.float64) * xb.astype(np.float64)
    both_normal = (np.abs(xa) >= 2.0 ** -14) & (np.abs(xb) >= 2.0 ** -14)
    rel = np.abs(prod - exact)[both_normal] / np.abs(exact[both_normal])
    assert rel.max() <= 3 * 2.0 ** -22, rel.max()
    # with the dropped lo * lo term added back (a fourth product) only the
    # halves' own rounding remains, at most 2 * 2^-22
    prod4 = prod + 2.0 ** -22 * f(la) * f(lb)
    rel4 = np.abs(prod4 - exact)[both_normal] / np.abs(exact[both_normal])
    assert rel4.max() <= 2 * 2.0 ** -22, rel4.max()


def test_hi_finite_for_the_kernel_operand_range():
    # |x| < 2^23 keeps hi = f16(x * 2^-8) below f16's largest finite value
    x = np.array([2.0 ** 23 * 0.999, -(2.0 ** 23) * 0.999, 3e4, -65504.0], np.float32)
    _, hi, lo = split(x)
    assert np.isfinite(hi).all() and np.isfinite(lo).all()
    with np.errstate(over="ignore"):
        _, hi_big, _ = split(np.array([2.0 ** 24], np.float32))
    assert not np.isfinite(hi_big).all()  # the stated limit is real
