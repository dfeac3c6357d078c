"""GPU parity of nt_hip_matmul (GpuBackend::matmul) against CpuRef's arithmetic (oracle.c
`or_matmul_f32`: fma chains over k in order, closed every 256), bit for bit.

The cases are the reference's own device bodies on the reference's inputs (`t(shape, seed)` =
rnd(numel, seed, -2, 2), tests/mod.rs:28-31, restated by the oracle):
- `body_matmul_bit_exact_past_one_k_block` (src/tensor/tests/gpu/ops.rs:104-117);
- `body_matmul_large_tiles_and_split_k_bit_exact` (src/tensor/tests/gpu/kernels.rs:227-250);
plus this kernel's own edges: both tile sizes, every load orientation (A along k or m, B along n or
k), odd offsets and strides, k = 0 and k = 1, empty outputs, many batches, reruns.
"""
import ctypes as C

import numpy as np
import pytest

import noetic_ops as ops
import noetic_rl as nr
from noetic_ops import DTensor, Layout
from oracle import oracle as O

pytestmark = pytest.mark.gpu
F = np.float32


@pytest.fixture(scope="module", autouse=True)
def device():
    nr.claim(0)
    yield


def t(shape, seed):
    return O.reference_rnd_f32(seed, int(np.prod(shape)), -2.0, 2.0).astype(F).reshape(shape)


def bits(a, b):
    a, b = np.asarray(a, F), np.asarray(b, F)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


def check(name, a, b, dev_fn, cpu_fn):
    got = dev_fn(DTensor.from_numpy(a), DTensor.from_numpy(b)).to_numpy()
    want = cpu_fn(a, b)
    ndiff = int(np.count_nonzero(got.view(np.uint32) != want.view(np.uint32))) if got.shape == want.shape else -1
    print(f"matmul {name}: {got.size - max(ndiff, 0)} of {got.size} bit-equal", flush=True)
    assert bits(got, want), f"{name}: {ndiff} outputs differ"
    return got


@pytest.mark.parametrize("i,sh", list(enumerate([[1, 64, 1000, 33], [1, 300, 1000, 17], [2, 129, 513, 65],
                                                  [1, 512, 512, 512], [1, 1024, 1024, 1024]])))
def test_body_matmul_bit_exact_past_one_k_block(i, sh):
    """ops.rs:104-117: chains past one k block, bit for bit."""
    a = t([sh[0], sh[1], sh[2]], 40 + i)
    b = t([sh[0], sh[2], sh[3]], 50 + i)
    check(str(sh), a, b, lambda x, y: x.matmul(y), O.matmul)


SWAP = lambda x: np.swapaxes(x, 1, 2)  # noqa: E731


@pytest.mark.parametrize("i,case", list(enumerate([
    ("[2,130,300]x[2,300,257]", [2, 130, 300], [2, 300, 257], None, None),
    ("[1,128,64]x[1,64,128]", [1, 128, 64], [1, 64, 128], None, None),
    ("[3,200,513]x[1,513,140] broadcast", [3, 200, 513], [1, 513, 140], None, None),
    ("transposed views", [2, 300, 150], [2, 260, 300], "swap", "swap"),
    ("[1,1024,1024]x[1,1024,1024]", [1, 1024, 1024], [1, 1024, 1024], None, None),
    ("split-k [1,256,2048]x[1,2048,256]", [1, 256, 2048], [1, 2048, 256], None, None),
    ("split-k transposed rhs, k 1000", [2, 130, 1000], [2, 140, 1000], None, "swap"),
])))
def test_body_matmul_large_tiles_and_split_k_bit_exact(i, case):
    """kernels.rs:227-250: the reference's large-tile and split-k cases, bit for bit."""
    name, sa, sb, ta, tb = case
    a, b = t(sa, 60 + i), t(sb, 70 + i)
    dv = lambda x: x.swap_dims(1, 2)  # noqa: E731
    check(name, a, b,
          lambda x, y: (dv(x) if ta else x).matmul(dv(y) if tb else y),
          lambda x, y: O.matmul(SWAP(x) if ta else x, SWAP(y) if tb else y))


def test_unsplit_chains_closed_in_registers():
    """With 1024 tiles or more the workgroups close the 256-k chains themselves (no split-k):
    both tile sizes, k past one closure."""
    rng = np.random.default_rng(8)
    a, b = rng.uniform(-2, 2, (4, 1024, 300)).astype(F), rng.uniform(-2, 2, (4, 300, 1024)).astype(F)
    check("unsplit 64 tiles [4,1024,300]x[4,300,1024]", a, b, lambda x, y: x.matmul(y), O.matmul)
    a, b = rng.uniform(-2, 2, (1, 4096, 260)).astype(F), rng.uniform(-2, 2, (1, 260, 4096)).astype(F)
    check("unsplit 128 tiles [1,4096,260]x[1,260,4096]", a, b, lambda x, y: x.matmul(y), O.matmul)


def test_both_tiles_every_orientation_and_offsets():
    """The 128x128 tile (at least 512 tiles) and the 64x64 one, with A read along k and along m and
    B along n and along k, chains closed inside both (split over workgroups, then folded in
    order); views at odd offsets and strides."""
    rng = np.random.default_rng(7)
    big_a = rng.uniform(-2, 2, (2, 2048, 264)).astype(F)
    big_b = rng.uniform(-2, 2, (2, 264, 2048)).astype(F)
    check("128 tiles A.B [2,2048,264]x[2,264,2048]", big_a, big_b, lambda x, y: x.matmul(y), O.matmul)
    at = np.ascontiguousarray(SWAP(big_a[:, :1024, :]))  # [2, 264, 1024]
    bt = np.ascontiguousarray(SWAP(big_b[:, :, :1024]))  # [2, 1024, 264]
    for ta in (False, True):
        for tb in (False, True):
            a = at if ta else np.ascontiguousarray(big_a[:, :1024, :])
            b = bt if tb else np.ascontiguousarray(big_b[:, :, :1024])
            check(f"64 tiles A{'T' if ta else ''}.B{'T' if tb else ''}", a, b,
                  lambda x, y: (x.swap_dims(1, 2) if ta else x).matmul(y.swap_dims(1, 2) if tb else y),
                  lambda x, y: O.matmul(SWAP(x) if ta else x, SWAP(y) if tb else y))
    # views that start at an odd element and step by odd strides
    base = rng.uniform(-2, 2, (3, 101, 77)).astype(F)
    other = rng.uniform(-2, 2, (3, 77, 95)).astype(F)
    check("odd offsets and strides", base, other,
          lambda x, y: x.slice([range(0, 3), range(1, 100), range(3, 70)]).matmul(
              y.slice([range(0, 3), range(3, 70), range(2, 93)])),
          lambda x, y: O.matmul(x[:, 1:100, 3:70], y[:, 3:70, 2:93]))


def test_edges_k0_k1_empty_and_many_batches():
    a0, b0 = np.zeros((2, 3, 0), F), np.zeros((2, 0, 4), F)
    got = DTensor.from_numpy(np.ones((2, 3, 1), F)).slice([range(0, 2), range(0, 3), range(0, 0)]).matmul(
        DTensor.from_numpy(np.ones((2, 1, 4), F)).slice([range(0, 2), range(0, 0), range(0, 4)]))
    assert got.shape == [2, 3, 4] and bits(got.to_numpy(), O.matmul(a0, b0)), "k = 0 gives zeros"
    a, b = t([5, 7, 1], 1), t([5, 1, 9], 2)
    check("k = 1", a, b, lambda x, y: x.matmul(y), O.matmul)
    e = DTensor.from_numpy(t([2, 3, 4], 3)).slice([range(0, 2), range(0, 0), range(0, 4)]).matmul(
        DTensor.from_numpy(t([2, 4, 5], 4)))
    assert e.shape == [2, 0, 5]
    a, b = t([300, 9, 33], 5), t([1, 33, 13], 6)
    check("300 batches against one", a, b, lambda x, y: x.matmul(y), O.matmul)
    a, b = t([2, 1, 3, 40, 20], 7), t([1, 4, 1, 20, 24], 8)
    check("rank 5, batches broadcast both ways", a, b, lambda x, y: x.matmul(y), O.matmul)


def test_reruns_are_bit_identical():
    a, b = DTensor.from_numpy(t([4, 333, 700], 9)), DTensor.from_numpy(t([4, 700, 211], 10))
    y1, y2 = a.matmul(b).to_numpy(), a.matmul(b).to_numpy()
    assert y1.tobytes() == y2.tobytes()


def test_trait_method_returns_the_output_shape():
    """GpuBackend::matmul returns the storage and [batch..., m, n]."""
    a, b = nr.Tensor.from_numpy(t([3, 1, 6, 5], 11)), nr.Tensor.from_numpy(t([1, 2, 5, 4], 12))
    y, shape = ops.matmul(a, Layout([3, 1, 6, 5]), b, Layout([1, 2, 5, 4]))
    assert shape == [3, 2, 6, 4]
    assert bits(y.to_numpy().reshape(shape), O.matmul(a.to_numpy().reshape(3, 1, 6, 5),
                                                      b.to_numpy().reshape(1, 2, 5, 4)))
    with pytest.raises(ValueError):
        ops.matmul(a, Layout([3, 1, 6, 5]), b, Layout([1, 2, 4, 5]))
    assert nr.lib().nt_hip_matmul(C.c_void_p(a.ptr), C.byref(Layout([6, 5]).c()), C.c_void_p(b.ptr),
                                  C.byref(Layout([4, 5]).c()), C.c_void_p(b.ptr)) == -1
