"""The fused penalty's division (vdx_kernels.hip: penalise_fast): for fp32 x
and p, RN32(RN64(x * RN64(1/p))) equals the IEEE fp32 quotient RN32(x / p)
whenever the quotient is >= 2^-125, so the kernel may divide by multiplying
with a double reciprocal and still reproduce the reference's Single division
(Sampler.pas:295-300) bit for bit.

The argument (x / p is never within 2^-49 relative of a midpoint of two fp32
values, while the double product is within 2^-52 of x / p) is checked here
on the cases that stress it: random operands over the whole exponent range,
the penalties the tests and the bench use, and quotients constructed to lie as
close to a midpoint as fp32 operands allow.
"""
import numpy as np

TINY = 2.0 ** -125


def fast_div(x, p):
    ip = 1.0 / np.float64(p)
    return (x.astype(np.float64) * ip).astype(np.float32)


def check(x, p):
    x = np.asarray(x, dtype=np.float32)
    p = np.float32(p)
    want = x / p
    got = fast_div(x, p)
    ok = np.abs(x.astype(np.float64) / np.float64(p)) >= TINY
    bad = ok & (got.view(np.uint32) != want.view(np.uint32))
    assert not bad.any(), (p, x[bad][:5], got[bad][:5], want[bad][:5])
    return int(ok.sum())


def test_random_operands_all_exponents():
    rng = np.random.default_rng(11)
    n = 0
    for _ in range(40):
        p = np.float32(1.0 + rng.random() * 20.0)
        bits = rng.integers(0x00800000, 0x7F800000, 200_000, dtype=np.uint32)
        n += check(bits.view(np.float32), p)
    assert n > 7_000_000


def test_bench_and_test_penalties():
    rng = np.random.default_rng(12)
    for p in (1.1, 1.3, 1.5, 2.0, 3.0, 1.0001, 7.25, 1e3, 65504.0):
        x = (rng.standard_normal(500_000) * 10.0 ** rng.integers(-30, 30, 500_000)).astype(np.float32)
        x = np.abs(x)
        check(x, p)


def test_quotients_next_to_midpoints():
    # y = a fp32 midpoint (odd multiple of half an ulp); x = RN32(y * p) puts
    # x / p within about an ulp of x of that midpoint
    rng = np.random.default_rng(13)
    for p in (1.1, 3.0, 1.3, 2.7182817, 1.0000001):
        p32 = np.float32(p)
        m = rng.integers(1 << 23, 1 << 24, 300_000).astype(np.float64)
        e = rng.integers(-100, 100, m.size).astype(np.float64)
        y = (2.0 * m + 1.0) * 2.0 ** (e - 24)
        x = (y * np.float64(p32)).astype(np.float32)
        for d in (-1, 0, 1):  # and the neighbouring fp32 values of x
            xi = (x.view(np.uint32).astype(np.int64) + d).astype(np.uint32).view(np.float32)
            check(xi, p32)


def test_special_values_follow_the_kernel_rule():
    # +inf stays +inf; quotients below 2^-125 are left to the IEEE division
    p = np.float32(1.1)
    assert fast_div(np.array([np.inf], np.float32), p)[0] == np.inf
    small = np.array([2.0 ** -124, 2.0 ** -126, 1e-45], dtype=np.float32)
    q = np.abs(small.astype(np.float64) / np.float64(p))
    assert (q[1:] < TINY).all() and q[0] >= TINY
