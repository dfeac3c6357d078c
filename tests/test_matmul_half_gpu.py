"""GPU tests of nt_hip_matmul_half (GpuBackend::matmul_half: bf16 operands on the matrix cores, f32
accumulation), with the reference's stated tolerance rather than byte equality
(src/tensor/tests/gpu/half_gemm.rs:1-10, 73-104):
- on the reference's fixed shapes and inputs (`ht(shape, seed)` = rnd(numel, seed, -2, 2)), the
  largest |got - want| / sum|a||b| is within 2^-21 k of the bf16-rounded operands' exact f64
  product, and within 2u + 2^-21 k (u = 2^-8) of the f32 operands' product;
- small integer operands (exact in bf16, every partial sum exact in f32) give the integer product
  exactly: this pins the MFMA's operand and result lane layout independently of rounding;
- the same products twice give the same bits; the key part names the product.
"""
import numpy as np
import pytest

import noetic_ops as ops
import noetic_rl as nr
from noetic_ops import DTensor, MatmulPrecision as MP
from oracle import oracle as O

pytestmark = pytest.mark.gpu
F = np.float32
HALF = MP.HALF


@pytest.fixture(scope="module", autouse=True)
def device():
    nr.claim(0)
    yield


def ht(shape, seed):
    return O.reference_rnd_f32(seed, int(np.prod(shape)), -2.0, 2.0).astype(F).reshape(shape)


def bf16(x):
    return O.bf16_to_f32(O.bf16_from_f32(np.ascontiguousarray(x, F))).reshape(np.shape(x)).astype(np.float64)


SW = lambda x: np.swapaxes(x, 1, 2)  # noqa: E731
CASES = [("[1,64,64]x[1,64,64]", [1, 64, 64], [1, 64, 64], False),
         ("[1,256,256]x[1,256,256]", [1, 256, 256], [1, 256, 256], False),
         ("[2,130,300]x[2,300,257] ragged", [2, 130, 300], [2, 300, 257], False),
         ("[1,7,5]x[1,5,3] tiny", [1, 7, 5], [1, 5, 3], False),
         ("[1,64,2048]x[1,2048,64] long k", [1, 64, 2048], [1, 2048, 64], False),
         ("[3,100,96]x[1,96,70] broadcast", [3, 100, 96], [1, 96, 70], False),
         ("AT.BT views [2,150,300],[2,260,150]", [2, 150, 300], [2, 260, 150], True),
         ("[1,512,512]x[1,512,512]", [1, 512, 512], [1, 512, 512], False),
         ("[2,2048,96]x[2,96,2048] (128 tiles)", [2, 2048, 96], [2, 96, 2048], False)]


@pytest.mark.parametrize("i,case", list(enumerate(CASES)))
def test_body_half_matmul_error_against_f32_on_fixed_shapes(i, case):
    label, sa, sb, tr = case
    a, b = ht(sa, 80 + i), ht(sb, 90 + i)
    da, db = DTensor.from_numpy(a), DTensor.from_numpy(b)
    if tr:
        da, db, a, b = da.swap_dims(1, 2), db.swap_dims(1, 2), SW(a), SW(b)
    got = da.matmul_with(db, HALF).to_numpy().astype(np.float64)
    k = a.shape[-1]
    a64, b64 = a.astype(np.float64), b.astype(np.float64)
    want16 = bf16(a) @ bf16(b)
    s16 = np.abs(bf16(a)) @ np.abs(bf16(b))
    want32, s32 = a64 @ b64, np.abs(a64) @ np.abs(b64)
    e16 = np.max(np.abs(got - want16) / np.maximum(s16, np.finfo(np.float64).tiny))
    e32 = np.max(np.abs(got - want32) / np.maximum(s32, np.finfo(np.float64).tiny))
    acc = 2.0 ** -21 * k
    print(f"half matmul {label} (bf16, k {k}): {e16:.3e} against the rounded operands (bound {acc:.3e}), "
          f"{e32:.3e} against the f32 operands (bound {2 * 2.0 ** -8 + acc:.3e})", flush=True)
    assert got.shape == want32.shape
    assert e16 <= acc and e32 <= 2 * 2.0 ** -8 + acc and np.all(np.isfinite(got))


@pytest.mark.parametrize("shape", [(1, 32, 16, 32), (2, 128, 64, 128), (3, 200, 96, 130), (1, 257, 33, 300),
                                   (2, 2048, 64, 2048)])
def test_integer_operands_are_exact_and_pin_the_lane_layout(shape):
    """Integers in [-8, 8] are exact in bf16 and every partial sum is exact in f32, so the product
    equals numpy's integer product exactly whatever the summation order: a wrong operand or result
    lane mapping would show as wrong integers. Both orientations of each operand; both tile sizes
    (128x128 from 512 workgroups up, the last shape; 64x64 below)."""
    nb, m, k, n = shape
    rng = np.random.default_rng(m + k)
    a = rng.integers(-8, 9, (nb, m, k)).astype(F)
    b = rng.integers(-8, 9, (nb, k, n)).astype(F)
    want = (a.astype(np.float64) @ b.astype(np.float64)).astype(F)  # exact: |sums| <= 64 k
    for ta in (False, True):
        for tb in (False, True):
            da = DTensor.from_numpy(np.ascontiguousarray(SW(a))).swap_dims(1, 2) if ta else DTensor.from_numpy(a)
            db = DTensor.from_numpy(np.ascontiguousarray(SW(b))).swap_dims(1, 2) if tb else DTensor.from_numpy(b)
            got = da.matmul_with(db, HALF).to_numpy()
            assert np.array_equal(got, want), f"{shape} ta={ta} tb={tb}: {np.count_nonzero(got != want)} differ"


def test_half_matmul_is_run_to_run_identical_and_keyed():
    outs = []
    for _ in range(2):
        run = []
        for i, (_, sa, sb, tr) in enumerate(CASES):
            da, db = DTensor.from_numpy(ht(sa, 80 + i)), DTensor.from_numpy(ht(sb, 90 + i))
            if tr:
                da, db = da.swap_dims(1, 2), db.swap_dims(1, 2)
            run.append(da.matmul_with(db, HALF).to_numpy().tobytes())
        outs.append(run)
    assert outs[0] == outs[1]
    key = ops.half_gemm_key()
    assert key.startswith("gemm-bf16-mfma32x32x16-f32acc-kernels-") and len(key.split("-")[-1]) == 16
    f32 = DTensor.from_numpy(ht([1, 64, 64], 1)).matmul(DTensor.from_numpy(ht([1, 64, 64], 2))).to_numpy()
    half = DTensor.from_numpy(ht([1, 64, 64], 1)).matmul_with(DTensor.from_numpy(ht([1, 64, 64], 2)), HALF).to_numpy()
    assert not np.array_equal(f32, half), "the half product is a different product"


# ---- the packed-operand path (operands rounded to bf16 once into fragment order, 256 x 256 tiles
# through the MFMA pipeline). Products of at least 64 such tiles with k >= 256 take it by
# themselves; NOETIC_HIP_HALF_GEMM=packed|staged forces one path for any shape.

class _Path:
    def __init__(self, path):
        self.path = path

    def __enter__(self):
        import os
        self.old = os.environ.get("NOETIC_HIP_HALF_GEMM")
        os.environ["NOETIC_HIP_HALF_GEMM"] = self.path

    def __exit__(self, *exc):
        import os
        if self.old is None:
            os.environ.pop("NOETIC_HIP_HALF_GEMM", None)
        else:
            os.environ["NOETIC_HIP_HALF_GEMM"] = self.old


@pytest.mark.parametrize("shape", [(1, 32, 16, 32), (2, 256, 64, 256), (3, 200, 96, 130), (1, 257, 33, 300),
                                   (1, 300, 530, 513), (2, 512, 272, 257)])
def test_packed_path_integer_operands_are_exact(shape):
    """The packed path's lane layout (both packings, the pipeline's operand order, the tile
    stores) pinned by exact integer products, both orientations of each operand, ragged m, n
    and k (rows, columns and k past the ends packed as zeros)."""
    nb, m, k, n = shape
    rng = np.random.default_rng(m * 7 + k + n)
    a = rng.integers(-8, 9, (nb, m, k)).astype(F)
    b = rng.integers(-8, 9, (nb, k, n)).astype(F)
    want = (a.astype(np.float64) @ b.astype(np.float64)).astype(F)
    with _Path("packed"):
        for ta in (False, True):
            for tb in (False, True):
                da = DTensor.from_numpy(np.ascontiguousarray(SW(a))).swap_dims(1, 2) if ta else DTensor.from_numpy(a)
                db = DTensor.from_numpy(np.ascontiguousarray(SW(b))).swap_dims(1, 2) if tb else DTensor.from_numpy(b)
                got = da.matmul_with(db, HALF).to_numpy()
                assert np.array_equal(got, want), f"{shape} ta={ta} tb={tb}: {np.count_nonzero(got != want)} differ"


@pytest.mark.parametrize("i,case", list(enumerate(CASES)))
def test_packed_path_equals_the_staged_kernel(i, case):
    """Both paths run the same MFMA over the same k order from zero on the same bf16 operands,
    so every output is the same sum: the reference's fixed shapes through both, bit for bit."""
    label, sa, sb, tr = case
    outs = []
    for path in ("staged", "packed"):
        da, db = DTensor.from_numpy(ht(sa, 80 + i)), DTensor.from_numpy(ht(sb, 90 + i))
        if tr:
            da, db = da.swap_dims(1, 2), db.swap_dims(1, 2)
        with _Path(path):
            outs.append(da.matmul_with(db, HALF).to_numpy())
    assert outs[0].tobytes() == outs[1].tobytes(), f"{label}: {np.count_nonzero(outs[0] != outs[1])} outputs differ"


def test_large_product_takes_the_packed_path_within_the_bound():
    """2048 x 1024 x 2048 (64 tiles of 256 x 256: the packed path by itself) against the exact
    product of the rounded operands, and broadcast batches through the same path."""
    m, k, n = 2048, 1024, 2048
    a, b = ht([1, m, k], 5), ht([1, k, n], 6)
    got = DTensor.from_numpy(a).matmul_with(DTensor.from_numpy(b), HALF).to_numpy().astype(np.float64)
    want16 = bf16(a) @ bf16(b)
    s16 = np.abs(bf16(a)) @ np.abs(bf16(b))
    e16 = np.max(np.abs(got - want16) / np.maximum(s16, np.finfo(np.float64).tiny))
    print(f"packed half matmul {m}x{k}x{n}: {e16:.3e} against the rounded operands (bound {2.0 ** -21 * k:.3e})")
    assert e16 <= 2.0 ** -21 * k
    with _Path("staged"):
        staged = DTensor.from_numpy(a).matmul_with(DTensor.from_numpy(b), HALF).to_numpy().astype(np.float64)
    assert np.array_equal(got, staged)
    # broadcast: A [3, 300, 512] against B [1, 512, 260], every batch against the same B
    a3, b1 = ht([3, 300, 512], 7), ht([1, 512, 260], 8)
    with _Path("packed"):
        g3 = DTensor.from_numpy(a3).matmul_with(DTensor.from_numpy(b1), HALF).to_numpy().astype(np.float64)
    w3 = bf16(a3) @ bf16(b1)
    s3 = np.abs(bf16(a3)) @ np.abs(bf16(b1))
    assert np.max(np.abs(g3 - w3) / np.maximum(s3, np.finfo(np.float64).tiny)) <= 2.0 ** -21 * 512
