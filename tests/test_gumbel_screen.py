"""The Gumbel sampler's screen (rl_gumbel.hip, gumbel_screen), as a method: its f32 evaluation of
g = -ln(-ln u), u = ((k >> 11) + 0.5) / 2^53 (src/nn/rl.rs:490-498), stays within a small bound of
the exact value rounded to f32 over the whole range of k, and is infinite exactly where g is. The
kernel keeps every element within 1e-3 of the row's largest screened value, so the bound must sit
far below that margin. numpy's f32 logarithm stands in for the hardware's here (both within about
an ulp); the device code itself is checked against Cpu(Reference)'s tokens in test_gumbel_gpu.py."""
import numpy as np

MARGIN = 1e-3


def screen(k):
    k = k.astype(np.uint64)
    ln2 = np.float32(np.log(2.0))
    with np.errstate(divide="ignore"):
        # u < 1/2: from u in f32
        u = k.astype(np.float32) * np.float32(2.0**-53) + np.float32(2.0**-54)
        t_small = -(np.log2(u).astype(np.float32) * ln2)
        # u >= 1/2: 1 - u from the integer, with the f64 sum k + 0.5 rounding to even from 2^52 on
        dint = np.uint64(2**53) - k - (k & np.uint64(1))
        d = dint.astype(np.float32) * np.float32(2.0**-53)
        w = d / (np.float32(2) - d)
        w2 = w * w
        ser = np.float32(1 / 15)
        for c in (1 / 13, 1 / 11, 1 / 9, 1 / 7, 1 / 5, 1 / 3, 1.0):
            ser = (ser * w2 + np.float32(c)).astype(np.float32)
        t_big = np.float32(2) * w * ser
        t = np.where(k < np.uint64(2**52), t_small, t_big).astype(np.float32)
        g = -(np.log2(t).astype(np.float32) * ln2)
    return np.where(dint == 0, np.float32(np.inf), g)


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
        np.array([0, 1, 2**52 - 1, 2**52, 2**53 - 2, 2**53 - 1], dtype=np.uint64),
    ])
    g, a = exact(k), screen(k)
    fin = np.isfinite(g)
    assert np.array_equal(fin, np.isfinite(a)), "infinite where the exact value is not, or the other way"
    assert np.array_equal(g[~fin], a[~fin])
    assert int((~fin).sum()) == 1  # k = 2^53 - 1: u rounds to 1
    err = np.abs(a[fin].astype(np.float64) - g[fin].astype(np.float64))
    assert err.max() < 1e-5 and err.max() * 50 < MARGIN, err.max()
