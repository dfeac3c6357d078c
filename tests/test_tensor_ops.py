"""CPU tests of the general ops' checker (oracle/tensor_ops.py) and host mirror (noetic_ops): the
binary16 conversions against numpy's IEEE conversions, the correctly rounded exp/ln/pow against
exact values and the f64 library, Layout's views against numpy's, and the C ABI's refusals before
any device call."""
import ctypes as C
import math

import numpy as np
import pytest

import noetic_ops as ops
import noetic_rl as nr
from oracle import oracle as O
from oracle import tensor_ops as T


def specials():
    v = [0.0, -0.0, 1.0, -1.0, np.inf, -np.inf, 65504.0, 65519.99, 65520.0, 2.0 ** -14, 2.0 ** -24, 2.0 ** -25,
         3 * 2.0 ** -26, 2.0 ** -24 * 1.5, 2.0 ** -24 * 2.5, 1e-45, 1e38, -3.1415926, 1 + 2.0 ** -11, 1 + 3 * 2.0 ** -11]
    return np.array(v, np.float32)


def test_f16_from_f32_is_numpys_ieee_rounding():
    rng = np.random.default_rng(1)
    x = np.concatenate([specials(), rng.normal(0, 1, 4000).astype(np.float32),
                        (rng.normal(0, 1, 4000) * 2.0 ** rng.integers(-30, 20, 4000)).astype(np.float32),
                        # exact ties between two binary16 values, normal and subnormal
                        ((np.arange(1, 500) * 2 + 1) * 2.0 ** -25).astype(np.float32),
                        ((np.arange(1024, 1500) * 2 + 1) * 2.0 ** -11).astype(np.float32)])
    ours = T.f16_from_f32(x)
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(ours, want)
    nan = T.f16_from_f32(np.array([np.nan, -np.nan], np.float32))
    assert np.all((nan & 0x7C00) == 0x7C00) and np.all(nan & 0x0200)  # quiet NaN


def test_f16_to_f32_is_exact_on_every_pattern():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ours = T.f16_to_f32(h)
    want = h.view(np.float16).astype(np.float32)
    fin = ~np.isnan(want)
    assert np.array_equal(ours[fin].view(np.uint32), want[fin].view(np.uint32))
    assert np.all(np.isnan(ours[~fin]))
    assert np.array_equal(T.f16_from_f32(ours[fin]), h[fin])  # round trip


def test_correctly_rounded_reference_values():
    assert T.correctly_rounded("exp", 0.0) == 1.0
    assert T.correctly_rounded("log", 1.0) == 0.0
    assert T.correctly_rounded("pow", 2.0, 10.0) == 1024.0 and T.correctly_rounded("pow", 4.0, 0.5) == 2.0
    assert T.correctly_rounded("exp", 100.0) == np.inf
    # e^-103 = 1.32 times the least subnormal, e^-104 = 0.49 times it: 2^-149 and 0
    assert T.correctly_rounded("exp", -103.0) == np.float32(2.0 ** -149) and T.correctly_rounded("exp", -104.0) == 0.0
    # exp(1) rounded to f32 is 0x402df854
    assert np.float32(T.correctly_rounded("exp", 1.0)).view(np.uint32) == 0x402DF854
    # against the f64 library rounded to f32: the same except rare double roundings
    rng = np.random.default_rng(2)
    xs = rng.uniform(-80, 80, 300).astype(np.float32)
    diff = sum(T.correctly_rounded("exp", float(x)) != np.float32(math.exp(float(x))) for x in xs)
    assert diff <= 3
    ls = np.abs(rng.normal(0, 100, 300)).astype(np.float32) + np.float32(1e-6)
    diff = sum(T.correctly_rounded("log", float(x)) != np.float32(math.log(float(x))) for x in ls)
    assert diff <= 3


def test_layout_views_match_numpy():
    base = np.arange(2 * 3 * 4, dtype=np.float32)
    l = ops.Layout([2, 3, 4])
    a = base.reshape(2, 3, 4)
    assert np.array_equal(T.view(base, l.shape, l.strides, l.offset), a)
    s = l.swapped(0, 2)
    assert np.array_equal(T.view(base, s.shape, s.strides, s.offset), a.transpose(2, 1, 0))
    n = l.narrowed([range(1, 2), range(0, 3), range(1, 3)])
    assert np.array_equal(T.view(base, n.shape, n.strides, n.offset), a[1:2, :, 1:3])
    b = ops.Layout([3, 1]).broadcast([2, 3, 4])
    assert b.strides == [0, 1, 0]
    assert ops.broadcast_shape([3, 1], [2, 1, 4]) == [2, 3, 4]
    with pytest.raises(ValueError):
        ops.broadcast_shape([3], [4])


def test_sum_dim_and_argmax_restatements():
    rng = np.random.default_rng(3)
    x = rng.normal(0, 1, (3, 5, 7)).astype(np.float32)
    s = T.sum_dim(x, x.shape, 2)
    assert np.array_equal(s.ravel(), np.array([O.unrolled_sum(r) for r in x.reshape(-1, 7)], np.float32))
    m = T.sum_dim(x, x.shape, 1)
    want = np.zeros((3, 7), np.float32)
    for k in range(5):
        want = want + x[:, k, :]
    assert np.array_equal(m.reshape(3, 7), want)
    x[1, 3, 2] = np.nan
    x[2, 1, 4] = x[2, 4, 4] = 99.0
    idx, val = T.argmax_dim(x, x.shape, 1)
    assert idx[1, 0, 2] == 3 and np.isnan(val[1, 0, 2]) and idx[2, 0, 4] == 1


def test_op_refusals_before_the_device():
    L = nr.lib()
    lay = ops.Layout([4]).c()
    buf = np.zeros(4, np.float32)
    p = buf.ctypes.data
    assert L.nt_hip_unary(99, 0.0, p, C.byref(lay), p) == -1
    assert "op" in L.nt_hip_last_error().decode()
    bad = ops.Layout([4]).c()
    bad.rank = 9
    assert L.nt_hip_copy(p, C.byref(bad), 4, p) == -1
    assert "rank" in L.nt_hip_last_error().decode()
    lb = ops.Layout([2, 2]).c()
    assert L.nt_hip_binary(0, p, C.byref(lay), p, C.byref(lb), p) == -1
    assert "broadcast" in L.nt_hip_last_error().decode()
    assert L.nt_hip_reduce_dim(1, p, 1, 0, 1, 1, p) == -1
    assert "empty dimension" in L.nt_hip_last_error().decode()
    assert L.nt_hip_reduce_all(2, p, 4, p) == -4  # NT_E_UNSUPPORTED: argmax over all elements
    # matmul: shapes that do not multiply, and batches that do not broadcast
    la, lb = ops.Layout([2, 3]).c(), ops.Layout([4, 2]).c()
    assert L.nt_hip_matmul(p, C.byref(la), p, C.byref(lb), p) == -1
    assert "multiply" in L.nt_hip_last_error().decode()
    la, lb = ops.Layout([2, 1, 2]).c(), ops.Layout([3, 2, 1]).c()
    assert L.nt_hip_matmul(p, C.byref(la), p, C.byref(lb), p) == -1
    assert "broadcast" in L.nt_hip_last_error().decode()


# ----------------------------------------------------------------------------------- matmul checker

def test_matmul_checker_small_integers_are_exact():
    """With small integer operands every partial sum is exact in f32, so any order gives the
    integer product: the checker equals numpy's int64 matmul, with and without chain closures
    (k up to 600), broadcast batches and transposed views."""
    rng = np.random.default_rng(3)
    for (ba, bb, m, k, n) in [((1,), (1,), 7, 5, 3), ((2,), (2,), 13, 256, 9), ((3,), (1,), 17, 600, 11),
                              ((2, 1), (1, 3), 5, 300, 4)]:
        a = rng.integers(-8, 9, ba + (m, k)).astype(np.float32)
        bt = rng.integers(-8, 9, bb + (n, k)).astype(np.float32)
        b = np.swapaxes(bt, -1, -2)  # a transposed view, read through its strides
        want = (a.astype(np.int64) @ b.astype(np.int64)).astype(np.float32)
        assert np.array_equal(O.matmul(a, b), want)


def test_matmul_checker_closes_the_chain_every_256():
    """k = 512: A's row is [2^24, 1 x 511] and B's column all ones. The first 256-long chain stays
    at 2^24 (each +1 rounds back to even), the second chain is 256, and the closure adds them:
    2^24 + 256. A single 512-long chain would stay at 2^24."""
    a = np.ones((1, 1, 512), np.float32)
    a[0, 0, 0] = 2.0 ** 24
    b = np.ones((1, 512, 1), np.float32)
    assert O.matmul(a, b)[0, 0, 0] == np.float32(2.0 ** 24 + 256)
    a[0, 0, 0], a[0, 0, 256] = 1.0, 2.0 ** 24  # 2^24 leads the second chain instead: 255 + 1 then 2^24
    assert O.matmul(a, b)[0, 0, 0] == np.float32(2.0 ** 24 + 256)


def test_matmul_checker_fuses_each_product_in_k_order():
    """[-1, 1 + 2^-12] . [1, 1 + 2^-12]: the chain is -1, then fma(1 + 2^-12, 1 + 2^-12, -1) =
    2^-11 + 2^-24 exactly. A rounded product (1 + 2^-11) or the reversed order (round the square
    first, then add -1) gives 2^-11."""
    e = np.float32(1 + 2.0 ** -12)
    a = np.array([[[-1.0, e]]], np.float32)
    b = np.array([[[1.0], [e]]], np.float32)
    assert O.matmul(a, b)[0, 0, 0] == np.float32(2.0 ** -11 + 2.0 ** -24)
    assert O.matmul(a[:, :, ::-1].copy(), b[:, ::-1, :].copy())[0, 0, 0] == np.float32(2.0 ** -11)


def test_matmul_checker_within_the_reference_error_bound():
    """Random [-1, 1] operands: within the reference's bound 2 k eps sum|a||b| of the f64 product
    (src/tensor/tests/gpu/cuda_only.rs:40-50), for k past several chain closures."""
    rng = np.random.default_rng(4)
    a = rng.uniform(-1, 1, (2, 33, 1000)).astype(np.float32)
    b = rng.uniform(-1, 1, (2, 1000, 17)).astype(np.float32)
    got = O.matmul(a, b).astype(np.float64)
    exact = a.astype(np.float64) @ b.astype(np.float64)
    bound = 2 * 1000 * np.finfo(np.float32).eps * (np.abs(a).astype(np.float64) @ np.abs(b).astype(np.float64))
    assert np.all(np.abs(got - exact) <= bound)


# ----------------------------------------------------------------------------------- sort checker

def _sort_order(a, b):
    """sort_order (kernels.rs:379-388) from the IEEE definitions: NaNs equal and above everything,
    else by value, and for equal values (only +-0 can differ) -0 below +0."""
    an, bn = math.isnan(a), math.isnan(b)
    if an or bn:
        return 0 if (an and bn) else (1 if an else -1)
    if a != b:
        return -1 if a < b else 1
    sa, sb = math.copysign(1.0, a) < 0, math.copysign(1.0, b) < 0
    return 0 if sa == sb else (-1 if sa else 1)


def test_sort_checker_is_the_stable_sort_order():
    """The checker's keyed numpy sort equals Python's stable sorted() under sort_order on lanes
    with ties, +-0, infinities and NaNs of both signs and several payloads."""
    import functools
    levels = np.array([-1e9, -0.5, 0.0, -0.0, 0.25, 1.0, np.nan, -1e-45, np.inf, -np.inf, 2.5], np.float32)
    nans = np.array([0xFFC00000, 0x7F800001, 0x7FC00001], np.uint32).view(np.float32)
    rng = np.random.default_rng(5)
    for n in (1, 2, 17, 300):
        lane = np.concatenate([levels, nans])[rng.integers(0, 14, n)]
        vals, pos = T.sort_desc(lane[None, :], [1, n], 1)
        want = sorted(range(n), key=functools.cmp_to_key(lambda i, j: -_sort_order(float(lane[i]), float(lane[j]))))
        assert list(pos[0]) == want
        assert np.array_equal(vals[0].view(np.uint32), lane[want].view(np.uint32))
