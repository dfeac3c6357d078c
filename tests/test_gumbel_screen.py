"""The Gumbel sampler's screen (rl_gumbel.hip, gumbel_screen), as a method: its f32 evaluation of
g = -ln(-ln u), u = ((k >> 11) + 0.5) / 2^53 (src/nn/rl.rs:490-498), stays within a small bound of
the exact value rounded to f32 over the whole range of k, and is infinite exactly where g is. The
kernel keeps every element within a margin of at least 1e-3 of the row's largest screened value, so
the bound must sit far below that margin. numpy's f32 logarithm stands in for the hardware's here (both within about
an ulp); the device code itself is checked against Cpu(Reference)'s tokens in test_gumbel_gpu.py.
The margin (rl_gumbel_kernels.hpp, screen_floor) is checked at every magnitude: an element it
leaves out cannot reach the largest exactly, once the f32 rounding of z + g is counted."""
import numpy as np

MARGIN = 1e-3


def _fma(a, b, c):
    """f32 fused multiply-add: the f64 product of two f32 values is exact; the sum is rounded to
    f64, then to f32 (a double rounding that can differ from one rounding by an ulp at most)."""
    return (np.asarray(a, np.float32).astype(np.float64) * np.asarray(b, np.float32).astype(np.float64)
            + np.asarray(c, np.float32).astype(np.float64)).astype(np.float32)


def screen(k):
    k = k.astype(np.uint64)
    hi = (k >> np.uint64(21)).astype(np.uint32)           # the u64's high word
    kl = (k & np.uint64(2**21 - 1)).astype(np.uint32)     # k's low 21 bits (the low word >> 11)
    ln2 = np.float32(np.log(2.0))
    with np.errstate(divide="ignore"):
        u = _fma(hi.astype(np.float32), 2.0**-32, _fma(kl.astype(np.float32), 2.0**-53, 2.0**-54))
        tl = np.log2(u).astype(np.float32) * -ln2
        # 2^53 d = (2^32 - hi) 2^21 - kl - (kl & 1), in one fused multiply-add
        nh = (np.uint32(0) - hi).astype(np.uint32)
        d = _fma((kl + (kl & np.uint32(1))).astype(np.float32), -(2.0**-53),
                 nh.astype(np.float32) * np.float32(2.0**-32))
        ser = _fma(d, 1 / 6, 1 / 5)
        for c in (1 / 4, 1 / 3, 0.5, 1.0):
            ser = _fma(ser, d, c)
        t = np.where(hi >= np.uint32(0xF0000000), (d * ser).astype(np.float32), tl).astype(np.float32)
        return (np.log2(t).astype(np.float32) * -ln2).astype(np.float32)


def exact(k):
    with np.errstate(divide="ignore"):
        u = (k.astype(np.float64) + 0.5) * 2.0**-53
        return (-np.log(-np.log(u))).astype(np.float32)


def test_screen_bound_over_the_range_of_k():
    rng = np.random.default_rng(5)
    k = np.concatenate([
        rng.integers(0, 2**53, 1_000_000, dtype=np.uint64),
        np.uint64(2**53 - 1) - rng.integers(0, 2**20, 200_000, dtype=np.uint64),  # u -> 1
        rng.integers(0, 2**20, 200_000, dtype=np.uint64),                         # u -> 0
        np.arange(2**52 - 2**15, 2**52 + 2**15, dtype=np.uint64),                 # u = 1/2
        np.arange(15 * 2**49 - 2**15, 15 * 2**49 + 2**15, dtype=np.uint64),       # u = 1 - 2^-4
        np.array([0, 1, 2**52 - 1, 2**52, 2**53 - 2, 2**53 - 1], dtype=np.uint64),
    ])
    g, a = exact(k), screen(k)
    fin = np.isfinite(g)
    assert np.array_equal(fin, np.isfinite(a)), "infinite where the exact value is not, or the other way"
    assert np.array_equal(g[~fin], a[~fin])
    assert int((~fin).sum()) == 1  # k = 2^53 - 1: u rounds to 1
    err = np.abs(a[fin].astype(np.float64) - g[fin].astype(np.float64))
    assert err.max() < 1e-5 and err.max() * 50 < MARGIN, err.max()


SCREEN_ERR = 3.9e-6  # above the bound the sweep above asserts for the screen (3.81e-6)


def floor_of(x, rel):
    """The kernel's screen_floor in f32: x less max(1e-3, |x| rel); +inf for x = +inf."""
    x = np.asarray(x, np.float32)
    with np.errstate(invalid="ignore"):
        m = np.maximum(np.float32(MARGIN), np.abs(x) * np.float32(rel)).astype(np.float32)
        return np.where(x == np.inf, x, (x - m).astype(np.float32))


def _uncovered(amx, rel):
    """For each largest screened value amx: can the largest f32 below the row's floor still reach
    amx's element exactly? A screened sum a and its exact one differ by the screen's error plus at
    most an ulp of the sum (the f32 rounding of z + g), on either side."""
    lo = floor_of(amx, rel)
    below = np.nextafter(lo, np.float32(-np.inf))   # the largest value the row leaves out
    d_y = SCREEN_ERR + np.spacing(np.abs(below)).astype(np.float64)
    d_x = SCREEN_ERR + np.spacing(np.abs(amx)).astype(np.float64)
    return below.astype(np.float64) + d_y >= amx.astype(np.float64) - d_x


def _largest_values():
    rng = np.random.default_rng(11)
    mags = np.float32(2.0) ** rng.uniform(-20, 100, 200_000).astype(np.float32)
    edges = np.float32(2.0) ** np.arange(-20, 101, dtype=np.float32)
    x = np.concatenate([mags, edges, np.nextafter(edges, np.float32(0)), np.nextafter(edges, np.float32(np.inf))])
    return np.concatenate([x, -x]).astype(np.float32)


def test_row_margin_leaves_out_only_elements_that_cannot_win():
    # an element the row's floor (rel 2^-21) leaves out lies below the largest one exactly, at
    # every magnitude, so candidates within it decide the row and a single one is the answer
    amx = _largest_values()
    assert not _uncovered(amx, 2.0**-21).any()
    # planted mistake: the absolute margin alone is too narrow once an ulp of the sum nears it
    bad = _uncovered(amx, 0.0)
    assert bad.any() and np.abs(amx[bad]).min() >= 4096


def test_thread_floor_keeps_a_superset_of_the_row_candidates():
    # a thread's largest screened value t lies between the row's floor and the row's largest x
    # when it holds a row candidate; the thread's floor (rel 2^-20) at t is then at or below the row's
    x = _largest_values()
    lo = floor_of(x, 2.0**-21)
    rng = np.random.default_rng(12)
    t = (lo.astype(np.float64) + rng.random(x.size) * (x.astype(np.float64) - lo)).astype(np.float32)
    t = np.clip(t, lo, x)
    assert (floor_of(t, 2.0**-20) <= lo).all()
    assert (floor_of(lo, 2.0**-20) <= lo).all() and (floor_of(x, 2.0**-20) <= lo).all()
    # +inf: the infinite values only
    assert floor_of(np.float32(np.inf), 2.0**-21) == np.inf
