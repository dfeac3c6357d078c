"""The Gumbel sampler's screen (rl_gumbel.hip, gumbel_screen), as a method: its f32 evaluation of
g = -ln(-ln u), u = ((k >> 11) + 0.5) / 2^53 (src/nn/rl.rs:490-498), stays within a small bound of
the exact value rounded to f32 over the whole range of k, and is infinite exactly where g is. The
kernel keeps every element within 1e-3 of the row's largest screened value, so the bound must sit
far below that margin. numpy's f32 logarithm stands in for the hardware's here (both within about
an ulp); the device code itself is checked against Cpu(Reference)'s tokens in test_gumbel_gpu.py."""
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
