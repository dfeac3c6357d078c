"""The kernels temper a logit under an additive f32 mask (tempered_logits, rl.rs:477-484: x / T in
f32, then the mask) as f32(f64(x) * rt), rt = 1 / f64(T) rounded to f64, wherever that product
is at least 2^-126 in magnitude or x is zero, and by the f32 division itself elsewhere (a wave
holding such an element divides it). This checks that rule against IEEE f32 division (numpy's),
so that the kernels' tempered values are the reference's to the bit:
- every f32 significand at two exponents for each temperature (normal quotients both sides of
  1), so every numerator's distance to a rounding midpoint is covered;
- the numerators whose quotients lie closest to a midpoint, found by exact integer search, at
  exponents from the subnormal range to the overflow threshold;
- special values: zeros, infinities, NaN, subnormal numerators and the largest finite values.
Wherever the product and the division differ, the kernel must be on its division path."""
import numpy as np
import pytest

TAUS = [0.7, 0.8, 0.9, 1.3, 0.6, 0.5, 2.0, 3.0, 1e-3, 7.25, 0.30000001, 1.9999999]


def by_product(x, tau):
    """The kernels' rule: (product, whether the kernel divides instead)."""
    x = np.asarray(x, np.float32)
    rt = np.float64(1.0) / np.float64(np.float32(tau))
    with np.errstate(over="ignore", invalid="ignore"):
        q = (x.astype(np.float64) * rt).astype(np.float32)
    divides = (np.abs(q) < np.float32(2.0 ** -126)) & (x != 0)
    return q, divides


def by_division(x, tau):
    with np.errstate(over="ignore", invalid="ignore", divide="ignore", under="ignore"):
        return np.asarray(x, np.float32) / np.float32(tau)


def check(x, tau):
    q, divides = by_product(x, tau)
    d = by_division(x, tau)
    same = (q.view(np.uint32) == d.view(np.uint32)) | (np.isnan(q) & np.isnan(d))
    bad = ~same & ~divides
    assert not bad.any(), (f"tau {tau}: {int(bad.sum())} quotients differ from f32 division, e.g. "
                           f"x = {x[bad][:4]!r}")
    return int((~same).sum())


def significands():
    """Every f32 significand, as integers in [2^23, 2^24)."""
    return np.arange(1 << 23, 1 << 24, dtype=np.int64)


def with_exponent(X, e):
    """X * 2^e as f32 (exact for 24-bit X while in range)."""
    return np.ldexp(X.astype(np.float64), e).astype(np.float32)


def nearest_to_midpoints(tau, count):
    """The significands X whose quotient X / tau lies closest to an f32 rounding midpoint (exact
    integer arithmetic on tau's significand T: the scaled quotient Y = X 2^j / T in [2^23, 2^24)
    is |2 ((X 2^j) mod T) - T| / (2 T) from a midpoint)."""
    m, e = np.frexp(np.float64(np.float32(tau)))
    T = int(np.ldexp(m, 24))
    X = significands()
    j = np.where(X >= T, 23, 24)
    rem = (X << j) % T
    dist = np.abs(2 * rem - T)
    return X[np.argsort(dist, kind="stable")[:count]]


@pytest.mark.parametrize("tau", TAUS)
def test_every_significand(tau):
    X = significands()
    for e in (-23, -20, 0, 40):  # numerators in [1, 2), [8, 16), [2^23, 2^24), [2^63, 2^64)
        check(with_exponent(X, e), tau)
        check(-with_exponent(X, e), tau)


@pytest.mark.parametrize("tau", TAUS)
def test_quotients_nearest_to_a_midpoint_at_every_exponent(tau):
    X = nearest_to_midpoints(tau, 256)
    for e in range(-172, 105, 3):  # subnormal quotients up to the overflow threshold and past it
        x = with_exponent(X, e)
        check(x, tau)
        check(-x, tau)


def test_overflow_threshold():
    for tau in TAUS:
        if tau >= 1.0:
            continue
        # numerators whose quotient straddles the overflow threshold (2^128 - 2^103)
        top = np.float64(np.finfo(np.float32).max) * np.float64(np.float32(tau))
        x = np.float32(top)
        xs = [x]
        for _ in range(64):
            xs.append(np.nextafter(xs[-1], np.float32(np.inf)))
        xs = np.array(xs[::-1] + [np.nextafter(x, np.float32(0))], np.float32)
        q, divides = by_product(xs, tau)
        d = by_division(xs, tau)
        assert np.array_equal(q.view(np.uint32), d.view(np.uint32)), f"tau {tau}: overflow threshold"
        assert not divides.any()
        assert np.isinf(d).any() and np.isfinite(d).any(), f"tau {tau}: the cases straddle the threshold"


def test_special_values():
    sub = np.array([2.0 ** -149, 3 * 2.0 ** -149, 2.0 ** -127, 1.5 * 2.0 ** -126], np.float32)
    x = np.concatenate([np.array([0.0, -0.0, np.inf, -np.inf, np.nan, np.finfo(np.float32).max,
                                  -np.finfo(np.float32).max, np.finfo(np.float32).tiny], np.float32), sub, -sub])
    for tau in TAUS + [6.0]:
        check(x, tau)
        q, divides = by_product(x, tau)
        # zeros keep their sign on the product path
        assert np.signbit(q[1]) and not np.signbit(q[0]) and not divides[:2].any()


def test_exact_subnormal_ties_take_the_division():
    # 5 2^-149 / 10 and 3 2^-149 / 6 are 2^-150 exactly, the midpoint between 0 and 2^-149 (ties
    # to even: 0), and 3 2^-149 / 2 is the midpoint 1.5 2^-149 (to 2^-148). The proof that the
    # product rounds like the division needs quotients of at least 2^-126, so the kernel divides
    # these.
    for x, tau, want in ((5 * 2.0 ** -149, 10.0, 0.0), (3 * 2.0 ** -149, 6.0, 0.0), (3 * 2.0 ** -149, 2.0, 2.0 ** -148)):
        xs = np.array([x, -x], np.float32)
        q, divides = by_product(xs, tau)
        assert np.array_equal(by_division(xs, tau), np.array([want, -want], np.float32))
        assert divides.all()
        check(xs, tau)


@pytest.mark.parametrize("rule", ["f32 reciprocal", "f64 reciprocal rounded to f32"])
def test_a_cruder_rule_fails_these_checks(rule, monkeypatch):
    def crude(x, tau):
        x = np.asarray(x, np.float32)
        if rule == "f32 reciprocal":
            q = x * (np.float32(1.0) / np.float32(tau))
        else:
            r = np.float64(np.float32(np.float64(1.0) / np.float64(np.float32(tau))))
            q = (x.astype(np.float64) * r).astype(np.float32)
        return q, (np.abs(q) < np.float32(2.0 ** -126)) & (x != 0)

    monkeypatch.setitem(globals(), "by_product", crude)
    with pytest.raises(AssertionError, match="quotients differ"):
        check(with_exponent(nearest_to_midpoints(0.7, 256), 0), 0.7)
