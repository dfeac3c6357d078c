"""The reference's device op bodies (src/tensor/tests/gpu/ops.rs:52-148) on this build's general
ops, through the tensor-level dispatch mirror (noetic_ops.DTensor):
- `body_exact_ops_match_cpu_ref_bit_for_bit`: every case, the three matmuls included, bit for bit
  against CpuRef;
- `body_transcendentals_within_4_ulp`: exp, log, sqrt, powf 0.5 and 3, sigmoid within 4 ulp, and
  softmax / log_softmax within 1e-6 relative;
- `body_nan_max_argmax_and_stable_sort_match_cpu_ref` (its sort half is in tests/test_sort_gpu.py)
  and `body_deterministic_twice` (ops.rs:183-234).
Inputs are the reference's own: `t(shape, seed)` = rnd(numel, seed, -2, 2) (ChaCha8 seeded from
the u64, rand 0.8's f32 gen_range; tests/mod.rs:28-31), restated by the oracle and pinned there
against the reference's fixture records. CpuRef's values are the checker's: IEEE f32 elementwise
arithmetic, the eight-partial sum along the last axis and in-order sums along others, the first
maximum, the binary16 / bfloat16 conversions, matmul's fma chains closed every 256 k.
"""
import numpy as np
import pytest

import noetic_ops as ops
import noetic_rl as nr
from noetic_ops import DTensor
from oracle import oracle as O
from oracle import tensor_ops as T

pytestmark = pytest.mark.gpu
F = np.float32


@pytest.fixture(scope="module", autouse=True)
def device():
    nr.claim(0)
    yield


def t(shape, seed):
    return O.reference_rnd_f32(seed, int(np.prod(shape)), -2.0, 2.0).astype(F).reshape(shape)


# CpuRef on host arrays
def c_sum(x):
    return np.array([O.unrolled_sum(np.ascontiguousarray(x, F).ravel())], F)


def c_sum_dim(x, d):
    return T.sum_dim(np.ascontiguousarray(x, F), list(x.shape), d)


def c_max_dim(x, d):
    return T.argmax_dim(np.ascontiguousarray(x, F), list(x.shape), d)[1].astype(F)


def c_sign(x):
    return np.where(x == 0, F(0), np.where(np.signbit(x), F(-1), F(1))).astype(F)


def c_mask_fill(x, m, v):
    return np.where(np.broadcast_to(m, x.shape), F(v), x).astype(F)


def c_clamp(x, lo, hi):
    y = c_mask_fill(x, x > F(hi), hi)
    return c_mask_fill(y, y < F(lo), lo)


def c_tril(h, w, off):
    p = np.arange(h * w)
    return ((p // w) - ((p % w) - off) < 0).reshape(h, w)


def exact_cases(a, b, c):
    """(name, device function of the DTensors, CpuRef function of the arrays)."""
    g_idx = (np.arange(3 * 5 * 4) * 5 % 7).reshape(3, 5, 4)
    long_lane = t([4, 1037], 9)
    return [
        ("add broadcast", lambda x: x[0].add(x[1]), lambda x: x[0] + x[1]),
        ("sub broadcast", lambda x: x[1].sub(x[0]), lambda x: x[1] - x[0]),
        ("mul", lambda x: x[0].mul(x[2]), lambda x: x[0] * x[2]),
        ("div", lambda x: x[0].div(x[2]), lambda x: x[0] / x[2]),
        ("add of views", lambda x: x[0].swap_dims(0, 2).add(x[2].swap_dims(0, 2)),
         lambda x: np.swapaxes(x[0], 0, 2) + np.swapaxes(x[2], 0, 2)),
        ("scalars", lambda x: x[0].add_scalar(0.3).mul_scalar(1.7).sub_scalar(0.1).div_scalar(3.0),
         lambda x: (((x[0] + F(0.3)) * F(1.7)) - F(0.1)) / F(3.0)),
        ("neg recip abs sign", lambda x: x[0].neg().recip().abs().add(x[0].sign()),
         lambda x: np.abs(F(1) / (-x[0])) + c_sign(x[0])),
        ("powi 2 and -2", lambda x: x[2].powf_scalar(2.0).add(x[2].powf_scalar(-2.0)),
         lambda x: (x[2] * x[2]) + (F(1) / (x[2] * x[2]))),
        ("clamp (compare + mask_fill)", lambda x: x[0].clamp(-0.5, 0.7), lambda x: c_clamp(x[0], -0.5, 0.7)),
        ("mask_fill broadcast mask", lambda x: x[0].mask_fill(x[1].greater_elem(0.0), -9.0),
         lambda x: c_mask_fill(x[0], x[1] > 0, -9.0)),
        ("mask_fill host mask",
         lambda x: x[0].slice([range(0, 3), range(0, 5), range(0, 5)]).mask_fill(
             DTensor.from_numpy(c_tril(5, 5, 0).astype(np.uint8), "bool").unsqueeze(0), -1e9),
         lambda x: c_mask_fill(x[0][0:3, 0:5, 0:5], c_tril(5, 5, 0)[None], -1e9)),
        ("sum", lambda x: x[0].sum(), lambda x: c_sum(x[0])),
        ("mean", lambda x: x[0].mean(), lambda x: c_sum(x[0]) / F(x[0].size)),
        ("sum_dim 0", lambda x: x[0].sum_dim(0), lambda x: c_sum_dim(x[0], 0)),
        ("sum_dim 1", lambda x: x[0].sum_dim(1), lambda x: c_sum_dim(x[0], 1)),
        ("sum_dim 2", lambda x: x[0].sum_dim(2), lambda x: c_sum_dim(x[0], 2)),
        ("sum_dim of a view", lambda x: x[0].swap_dims(1, 2).sum_dim(2),
         lambda x: c_sum_dim(np.ascontiguousarray(np.swapaxes(x[0], 1, 2)), 2)),
        ("sum_dim last, long lane", lambda x: DTensor.from_numpy(long_lane).sum_dim(1),
         lambda x: c_sum_dim(long_lane, 1)),
        ("mean_dim", lambda x: x[0].mean_dim(1).add(x[0].mean_dim(2).sum_dim(1)),
         lambda x: (c_sum_dim(x[0], 1) / F(5)) + c_sum_dim(c_sum_dim(x[0], 2) / F(7), 1)),
        ("max_dim", lambda x: x[0].max_dim(1).add(x[0].max_dim(2).sum_dim(1)),
         lambda x: c_max_dim(x[0], 1) + c_sum_dim(c_max_dim(x[0], 2), 1)),
        ("max", lambda x: x[0].max(), lambda x: np.array([T.max_all(x[0])], F)),
        ("argmax (as floats)", lambda x: DTensor.from_numpy(x[0].argmax(2).astype(F)),
         lambda x: T.argmax_dim(x[0], list(x[0].shape), 2)[0].astype(F)),
        ("reshape of a view", lambda x: x[0].swap_dims(0, 1).reshape([15, 7]),
         lambda x: np.ascontiguousarray(np.swapaxes(x[0], 0, 1)).reshape(15, 7)),
        ("slice", lambda x: x[0].slice([range(1, 3), range(0, 5), range(2, 6)]).mul_scalar(1.0),
         lambda x: x[0][1:3, 0:5, 2:6] * F(1.0)),
        ("slice_assign", lambda x: x[0].slice_assign([range(0, 2), range(1, 3), range(0, 7)],
                                                     x[2].slice([range(0, 2), range(0, 2), range(0, 7)])),
         lambda x: (lambda y: (y.__setitem__((slice(0, 2), slice(1, 3), slice(0, 7)), x[2][0:2, 0:2, 0:7]), y)[1])(
             x[0].copy())),
        ("cat", lambda x: DTensor.cat([x[0], x[2].swap_dims(0, 0), x[0]], 1),
         lambda x: np.concatenate([x[0], x[2], x[0]], axis=1)),
        ("expand", lambda x: x[1].expand([3, 4, 7]).mul_scalar(2.0),
         lambda x: np.broadcast_to(x[1], (3, 4, 7)) * F(2.0)),
        ("matmul batched", lambda x: x[0].matmul(x[2].swap_dims(1, 2)),
         lambda x: O.matmul(x[0], np.swapaxes(x[2], 1, 2))),
        ("matmul broadcast batch",
         lambda x: x[0].matmul(x[2].slice([range(0, 1), range(0, 5), range(0, 7)]).swap_dims(1, 2)),
         lambda x: O.matmul(x[0], np.swapaxes(x[2][0:1, 0:5, 0:7], 1, 2))),
        ("matmul rank 4 swapped", lambda x: x[0].reshape([3, 5, 1, 7]).matmul(x[2].reshape([3, 1, 7, 5])),
         lambda x: O.matmul(x[0].reshape(3, 5, 1, 7), x[2].reshape(3, 1, 7, 5))),
        ("gather", lambda x: x[0].gather(2, g_idx), lambda x: np.take_along_axis(x[0], g_idx, axis=2)),
        ("select", lambda x: x[0].select(1, [4, 0, 0, 2]), lambda x: x[0][:, [4, 0, 0, 2], :]),
        ("cast f16 round trip", lambda x: x[0].cast("f16").cast("f32"),
         lambda x: T.f16_to_f32(T.f16_from_f32(x[0]))),
        ("cast bf16 round trip", lambda x: x[0].mul_scalar(1e3).cast("bf16").cast("f32"),
         lambda x: O.bf16_to_f32(O.bf16_from_f32(x[0] * F(1e3))).reshape(x[0].shape)),
        ("f16 operand", lambda x: x[0].cast("f16").add(x[2].cast("f16")),
         lambda x: T.f16_to_f32(T.f16_from_f32(x[0])) + T.f16_to_f32(T.f16_from_f32(x[2]))),
    ]


def bits_equal(a, b):
    a, b = np.asarray(a, F), np.asarray(b, F)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_body_exact_ops_match_cpu_ref_bit_for_bit():
    a, b = t([3, 5, 7], 1), t([3, 1, 7], 2)
    c = (np.abs(t([3, 5, 7], 3)) + F(0.5)).astype(F)
    arrays = [a, b, c]
    devs = [DTensor.from_numpy(v) for v in arrays]
    cases = exact_cases(a, b, c)
    for name, on_device, on_cpu in cases:
        got = on_device(devs).to_numpy()
        want = np.asarray(on_cpu(arrays), F).reshape(got.shape) if np.asarray(on_cpu(arrays)).size == got.size \
            else np.asarray(on_cpu(arrays), F)
        assert bits_equal(got, want), f"{name}: {np.count_nonzero(got.ravel() != np.asarray(want).ravel())} differ"
    print(f"{len(cases)} op cases bit for bit against CpuRef")


def ulps(a, b):
    def key(x):
        i = x.view(np.int32).astype(np.int64)
        return np.where(i < 0, np.int64(-2 ** 31) - i, i)
    a, b = np.asarray(a, F), np.asarray(b, F)
    same = (a.view(np.uint32) == b.view(np.uint32)) | (np.isnan(a) & np.isnan(b))
    return np.where(same, 0, np.abs(key(a) - key(b)))


def test_body_transcendentals_within_4_ulp():
    x = t([64, 257], 5)
    pos = (np.abs(x) + F(1e-3)).astype(F)
    dx, dp = DTensor.from_numpy(x), DTensor.from_numpy(pos)
    with np.errstate(all="ignore"):
        # CpuRef: the platform libm in f32; the correctly rounded value stands in for it, and the
        # reference's bound (4 ulp) covers both
        cr = np.vectorize(lambda v, fn, s=0.0: T.correctly_rounded(fn, float(v), s), otypes=[F])
        sig = np.where(x >= 0, F(1) / (F(1) + cr(-x, "exp")), cr(x, "exp") / (F(1) + cr(x, "exp"))).astype(F)
        cases = [("exp", dx.exp(), cr(x, "exp")), ("log", dp.log(), cr(pos, "log")),
                 ("sqrt", dp.sqrt(), np.sqrt(pos)), ("powf 0.5", dp.powf_scalar(0.5), cr(pos, "pow", 0.5)),
                 ("powf 3", dp.powf_scalar(3.0), cr(pos, "pow", 3.0)), ("sigmoid", dx.sigmoid(), sig)]
    report = []
    for name, got, want in cases:
        u = ulps(got.to_numpy(), want)
        report.append(f"{name} max {int(u.max())} ulp")
        assert u.max() <= 4, f"{name}: {u.max()} ulp"
    for name, f, ref in (("softmax", ops.softmax, np.exp), ("log_softmax", ops.log_softmax, None)):
        got = f(dx, 1).to_numpy()
        z = x.astype(np.float64)
        lse = np.log(np.exp(z - z.max(1, keepdims=True)).sum(1, keepdims=True)) + z.max(1, keepdims=True)
        want = np.exp(z - lse) if name == "softmax" else z - lse
        d = np.max(np.abs(got - want) / (1.0 + np.abs(want)))
        report.append(f"{name} max rel {d:.1e}")
        assert d <= 1e-6, f"{name}: {d}"
    print("; ".join(report))


def test_body_nan_max_argmax_match_cpu_ref():
    """ops.rs:219-234 (the sort half is tests/test_sort_gpu.py's): NaN-propagating max and argmax."""
    nan = np.nan
    v = np.array([1.0, nan, 5.0, 2.0, nan, 3.0, 9.0, 0.0, 4.0, nan, nan, 1.0, 1.0, 7.0, 7.0, 2.0], F).reshape(4, 4)
    x = DTensor.from_numpy(v)
    for d in (0, 1):
        idx, val = T.argmax_dim(v, [4, 4], d)
        assert np.array_equal(x.argmax(d), idx), f"argmax {d}"
        assert ulps(x.max_dim(d).to_numpy(), val).max() == 0, f"max_dim {d}"
    for w in ([1.0, nan, 2.0], [nan, 1.0, 2.0], [1.0, 2.0, nan], [1.0, 3.0, 2.0]):
        w = np.array(w, F)
        assert ulps(DTensor.from_numpy(w).max().to_numpy(), np.array([T.max_all(w)], F)).max() == 0, "max"


def test_body_deterministic_twice():
    """ops.rs:183-196: a softmax's lane sums over a matmul and a sigmoid's means, computed twice,
    are the same bits."""
    def run():
        a = DTensor.from_numpy(t([8, 64, 96], 11))
        b = DTensor.from_numpy(t([8, 96, 64], 12))
        y = ops.softmax(a.matmul(b), 2).sum_dim(1).log()
        z = a.sigmoid().mean_dim(2)
        return y.to_numpy(), z.to_numpy()
    (y1, z1), (y2, z2) = run(), run()
    assert y1.tobytes() == y2.tobytes() and z1.tobytes() == z2.tobytes()
