"""GPU parity of nt_hip_sort_desc (GpuBackend::sort_desc) against CpuRef's stable descending sort
(oracle/tensor_ops.py `sort_desc`, pinned against a comparator sort in tests/test_tensor_ops.py):
values bit for bit (NaN payloads kept) and positions equal on every lane.

Cases: the reference's device bodies on its own inputs (`t(shape, seed)` = rnd(numel, seed, -2, 2),
tests/mod.rs:28-31) - `body_device_sort_matches_cpu_ref` (src/tensor/tests/gpu/kernels.rs:32-104:
distinct values along every axis, ties with +-0 and infinities, topk, a 5000-long lane) and the
sort half of `body_nan_max_argmax_and_stable_sort_match_cpu_ref` (src/tensor/tests/gpu/ops.rs:
219-246: NaNs of both signs and payloads, lanes of 16 to 5000) - plus lanes past one LDS run
(8193, 20000, a 128256-token vocabulary row) with inner lanes, and reruns.
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


def check(name, x, dim):
    v, i = DTensor.from_numpy(x).sort_descending_with_indices(dim)
    wv, wi = T.sort_desc(x, list(x.shape), dim)
    got = v.to_numpy()
    assert np.array_equal(got.view(np.uint32), wv.view(np.uint32)), f"{name}: values"
    assert np.array_equal(i, wi), f"{name}: positions ({np.count_nonzero(i != wi)} differ)"
    print(f"sort {name}: values and positions equal CpuRef's ({x.size} elements)", flush=True)
    return got, i


@pytest.mark.parametrize("shape,dim", [([4, 9], 1), ([3, 7, 5], 1), ([6, 5, 4], 0), ([2, 3, 1000], 2), ([2, 4096], 1),
                                       ([1, 1], 1)])
def test_body_device_sort_distinct_values(shape, dim):
    """kernels.rs:35-66: along each axis, the reference's inputs."""
    check(f"{shape} dim {dim}", t(shape, 11 + dim), dim)


def test_body_device_sort_ties_zeros_infinities_topk_long_lane():
    """kernels.rs:67-104: ties in first-index order with +-0 and infinities, topk, a 5000-long lane
    (the CUDA backend sends it through the host; it stays on the device here)."""
    lv = [1.0, -0.0, 0.0, 2.5, np.inf, -3.0, 1.0, -np.inf, 2.5]
    x = np.array([lv[(i * 7 + i // 33) % 9] for i in range(8 * 33)], F).reshape(8, 33)
    vals, pos = check("ties, +-0, infinities", x, 1)
    for lane in range(8):
        for p in range(32):
            if vals[lane, p].view(np.uint32) == vals[lane, p + 1].view(np.uint32):
                assert pos[lane, p] < pos[lane, p + 1], "ties in first-index order"
    x = t([5, 40], 3)
    tv, ti = DTensor.from_numpy(x).topk_with_indices(4, 1)
    wv, wi = T.sort_desc(x, [5, 40], 1)
    assert np.array_equal(tv.to_numpy().view(np.uint32), wv[:, :4].view(np.uint32)) and np.array_equal(ti, wi[:, :4])
    check("[2, 5000] long lane", t([2, 5000], 4), 1)


@pytest.mark.parametrize("n", [16, 300, 4096, 5000, 8192, 8193, 20000])
def test_body_stable_sort_with_nans(n):
    """ops.rs:235-246: lanes of the reference's levels (NaN, a sign-bit NaN, a signalling NaN,
    +-0, +-inf), values and positions exactly CpuRef's."""
    levels = np.array([-1e9, -0.5, 0.0, -0.0, 0.25, 1.0, np.nan, 0.0, -np.inf, 0.0, np.inf], F)
    levels[7] = np.array([0xFFC00000], np.uint32).view(F)[0]
    levels[9] = np.array([0x7F800001], np.uint32).view(F)[0]
    x = np.array([levels[(i * 7 + i // 3) % 11] for i in range(2 * n)], F).reshape(2, n)
    check(f"levels lanes of {n}", x, 1)


def test_long_lanes_with_inner_lanes_and_a_vocabulary_row():
    """Lanes past one LDS run merged on the device: an inner dimension (strided lanes), an odd
    run count, and four 128256-token vocabulary rows (the shape a top-p filter sorts)."""
    rng = np.random.default_rng(6)
    x = rng.normal(0, 1, (2, 10000, 3)).astype(F)
    x[0, ::7, 1] = x[0, 3, 1]  # ties across runs
    check("[2, 10000, 3] along 1", x, 1)
    x = (rng.normal(0, 2, (4, 128256)) * 8).round().astype(F) / F(8)  # many ties
    check("4 x 128256 vocabulary rows", x, 1)


def test_reruns_are_bit_identical():
    x = DTensor.from_numpy(t([3, 20000], 7))
    v1, i1 = x.sort_descending_with_indices(1)
    v2, i2 = x.sort_descending_with_indices(1)
    assert v1.to_numpy().tobytes() == v2.to_numpy().tobytes() and np.array_equal(i1, i2)


def test_trait_method_shapes_and_refusals():
    x = nr.Tensor.from_numpy(t([3, 4, 5], 8))
    vals, idx = ops.sort_desc(x, (3, 4, 5))
    assert vals.shape == (3, 4, 5) and idx.dtype == "i32"
    with pytest.raises(ValueError):
        ops.sort_desc(x, (3, 5, 5))
    with pytest.raises(ValueError):
        DTensor.from_numpy(t([7], 9)).sort_descending_with_indices(0)
