"""GPU parity of the general ops (include/noetic_ops.h) against the CPU checker on the same bytes.

Bit-exact: copies and writes through views (transposed, narrowed, broadcast, offset), casts
(bf16, f16 and bool; every f16 pattern), the IEEE operations (negate, abs, sign, +, -, *, /, sqrt,
1/x), comparisons, mask_fill, sums in CpuRef's order, the first maximum and its index, gather,
index_select, one_hot, scatter_add, index_add, fill. exp, ln and pow are checked against the
correctly rounded f32 (exact decimal evaluation): every sampled input within one ulp, and the
count of inputs off by one printed. `tempered_logits` built from these ops equals the oracle's
`tempered` to the bit.
"""
import numpy as np
import pytest

import noetic_ops as ops
import noetic_rl as nr
from noetic_ops import BinaryOp, CmpOp, Layout, ReduceOp, UnaryOp
from oracle import oracle as O
from oracle import tensor_ops as T

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def device():
    nr.claim(0)
    yield


def dev(a, dtype=None):
    return nr.Tensor.from_numpy(np.ascontiguousarray(a), dtype)


def bits(a):
    return np.asarray(a).view(np.uint32 if np.asarray(a).dtype.itemsize == 4 else np.uint16)


def specials():
    return np.array([0.0, -0.0, 1.0, -1.0, 2.5, -7.25, np.inf, -np.inf, np.nan, 1e-45, -1e-40, 3e38, 1e-30, 0.5,
                     65504.0, 1e30], np.float32)


def sample(n, seed):
    rng = np.random.default_rng(seed)
    x = (rng.normal(0, 1, n) * 2.0 ** rng.integers(-20, 20, n)).astype(np.float32)
    x[: len(specials())] = specials()
    return x


VIEWS = [
    # (base shape, view shape, strides, offset): contiguous, transposed, narrowed, broadcast, rank 5
    ((6, 7), (6, 7), (7, 1), 0),
    ((6, 7), (7, 6), (1, 7), 0),
    ((6, 7), (3, 4), (7, 1), 9),
    ((6, 7), (4, 6, 7), (0, 7, 1), 0),
    ((2, 3, 4, 5, 6), (2, 3, 4, 5, 6), (360, 120, 30, 6, 1), 0),
    ((2, 3, 4, 5, 6), (6, 5, 2, 4, 3), (1, 6, 360, 30, 120), 0),
    # transposes of several 64 x 64 tiles (ragged at both edges), one from an offset
    ((300, 130), (130, 300), (1, 130), 0),
    ((10, 9), (8, 9), (1, 9), 1),
]


@pytest.mark.parametrize("case", VIEWS)
@pytest.mark.parametrize("dtype", ["f32", "bf16", "u8", "i64"])
def test_copy_and_write_through_views(case, dtype):
    base_shape, shape, strides, off = case
    n = int(np.prod(base_shape))
    npd = {"f32": np.float32, "bf16": np.uint16, "u8": np.uint8, "i64": np.int64}[dtype]
    base = (np.arange(n) * 7 + 3).astype(npd)
    x = dev(base, dtype)
    l = Layout(shape, strides, off)
    want = T.view(base, shape, strides, off)
    got = ops.copy(x, l).to_numpy()
    assert np.array_equal(got, want)
    # write the view's elements into a narrowed view of a fresh destination; the rest is untouched
    if 0 not in strides:
        dst_full = np.zeros([s + 2 for s in shape], npd)
        d = dev(dst_full, dtype)
        dl = Layout(dst_full.shape).narrowed([range(1, s + 1) for s in shape])
        ops.write(d, dl, x, l)
        out = d.to_numpy()
        inner = tuple(slice(1, s + 1) for s in shape)
        assert np.array_equal(out[inner], want)
        out[inner] = 0
        assert not out.any()


def test_casts():
    x = sample(5000, 1)
    xt = dev(x)
    l = Layout([len(x)])
    assert np.array_equal(ops.cast(xt, l, "bf16").to_numpy(), O.bf16_from_f32(x))
    got16 = ops.cast(xt, l, "f16").to_numpy()
    want16 = T.f16_from_f32(x)
    assert np.array_equal(got16, want16)
    # every f16 and every bf16 high half widened exactly (strided: every other element)
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    h2 = np.repeat(h, 2)
    ht = dev(h2, "f16")
    wide = ops.cast(ht, Layout([65536], [2], 1), "f32").to_numpy()
    want = T.f16_to_f32(h)
    fin = ~np.isnan(want)
    assert np.array_equal(bits(wide[fin]), bits(want[fin])) and np.all(np.isnan(wide[~fin]))
    bt = dev(h, "bf16")
    wb = ops.cast(bt, Layout([65536]), "f32").to_numpy()
    assert np.array_equal(bits(wb), h.astype(np.uint32) << 16)
    # f16 -> bf16 through f32, and bool -> f32
    assert np.array_equal(ops.cast(dev(want16, "f16"), l, "bf16").to_numpy(), O.bf16_from_f32(T.f16_to_f32(want16)))
    b = np.array([0, 1, 1, 0, 1], np.uint8)
    assert np.array_equal(ops.cast(dev(b, "bool"), Layout([5]), "f32").to_numpy(), b.astype(np.float32))


def test_exact_unary_ops_through_a_transposed_view():
    x = sample(48 * 40, 2).reshape(48, 40)
    xt = dev(x)
    lt = Layout([40, 48], [1, 40])
    xv = x.T
    with np.errstate(all="ignore"):
        cases = {
            UnaryOp.NEG: (0.0, -xv), UnaryOp.ABS: (0.0, np.abs(xv)),
            UnaryOp.SIGN: (0.0, np.where(xv == 0, 0.0, np.where(np.signbit(xv), -1.0, 1.0)).astype(np.float32)),
            UnaryOp.SQRT: (0.0, np.sqrt(xv)), UnaryOp.RECIP: (0.0, np.float32(1.0) / xv),
            UnaryOp.ADD_SCALAR: (1.5, xv + np.float32(1.5)), UnaryOp.SUB_SCALAR: (-3.25, xv - np.float32(-3.25)),
            UnaryOp.MUL_SCALAR: (0.7, xv * np.float32(0.7)), UnaryOp.DIV_SCALAR: (0.7, xv / np.float32(0.7)),
        }
    for op, (s, want) in cases.items():
        got = ops.unary(op, xt, lt, s).to_numpy()
        same = (bits(got) == bits(np.asarray(want, np.float32))) | (np.isnan(got) & np.isnan(want))
        assert same.all(), f"{op.name}: {np.count_nonzero(~same)} elements differ"


def _ulps(a, b):
    a, b = np.float32(a), np.float32(b)
    if a == b or (np.isnan(a) and np.isnan(b)):
        return 0
    ia, ib = int(np.array(a).view(np.int32)), int(np.array(b).view(np.int32))
    ia = ia if ia >= 0 else -(ia & 0x7FFFFFFF)
    ib = ib if ib >= 0 else -(ib & 0x7FFFFFFF)
    return abs(ia - ib)


def test_exp_ln_pow_are_correctly_rounded_within_one_ulp():
    rng = np.random.default_rng(3)
    xe = np.concatenate([rng.uniform(-103, 88, 600), rng.normal(0, 1, 200), [0.0, -0.0, 1.0, 88.72, -103.9]])
    xe = xe.astype(np.float32)
    xl = np.concatenate([np.abs(rng.normal(0, 1, 400)) * 2.0 ** rng.integers(-140, 120, 400), [1.0, 2.0, 1e-45]])
    xl = xl.astype(np.float32)
    xp = np.abs(rng.normal(0, 3, 300)).astype(np.float32) + np.float32(1e-3)
    report = []
    for op, x, s, fn in ((UnaryOp.EXP, xe, 0.0, "exp"), (UnaryOp.LOG, xl, 0.0, "log"),
                         (UnaryOp.POW_SCALAR, xp, 2.3, "pow"), (UnaryOp.POW_SCALAR, xp, -0.5, "pow")):
        got = ops.unary(op, dev(x), Layout([len(x)]), s).to_numpy()
        s32 = float(np.float32(s))  # the exponent travels as f32 (PowScalar(p as f32), float.rs:565-569)
        u = [_ulps(g, T.correctly_rounded(fn, float(v), s32)) for g, v in zip(got, x)]
        assert max(u) <= 1, f"{fn}: {max(u)} ulp"
        report.append(f"{fn}{'' if fn != 'pow' else f'(s={s})'} {sum(1 for k in u if k)}/{len(u)} off by one")
    # special values (C99): exp(-inf) = 0, exp(inf) = inf, ln 0 = -inf, ln(-1) = NaN, ln inf = inf, x^0 = 1
    sp = np.array([-np.inf, np.inf, np.nan], np.float32)
    e = ops.unary(UnaryOp.EXP, dev(sp), Layout([3])).to_numpy()
    assert e[0] == 0.0 and e[1] == np.inf and np.isnan(e[2])
    lg = ops.unary(UnaryOp.LOG, dev(np.array([0.0, -1.0, np.inf], np.float32)), Layout([3])).to_numpy()
    assert lg[0] == -np.inf and np.isnan(lg[1]) and lg[2] == np.inf
    p0 = ops.unary(UnaryOp.POW_SCALAR, dev(np.array([np.nan, 0.0, -2.0], np.float32)), Layout([3]), 0.0).to_numpy()
    assert np.all(p0 == 1.0)
    print("; ".join(report))


def test_sigmoid_two_branch_form():
    x = np.concatenate([sample(1000, 4)[16:], [0.0, -0.0, 30.0, -30.0, -104.0, np.inf, -np.inf]]).astype(np.float32)
    got = ops.unary(UnaryOp.SIGMOID, dev(x), Layout([len(x)])).to_numpy()
    with np.errstate(all="ignore"):
        e = np.exp(-np.abs(x.astype(np.float64)))
        want = np.where(x >= 0, 1.0 / (1.0 + e), e / (1.0 + e))
    # f32 exp rounding, one add and one divide; an absolute floor where the value is subnormal
    assert np.all(np.abs(got - want) <= 4 * 2.0 ** -24 * want + 2.0 ** -148)
    assert got[-2] == 1.0 and got[-1] == 0.0


def test_compare_binary_and_mask_fill_with_broadcast():
    rng = np.random.default_rng(5)
    a = sample(8 * 33, 6).reshape(8, 33)
    b = rng.normal(0, 2, (1, 33)).astype(np.float32)
    b[0, 3] = np.nan
    out = [8, 33]
    al, bl = Layout(a.shape).broadcast(out), Layout(b.shape).broadcast(out)
    at, bt = dev(a), dev(b)
    with np.errstate(all="ignore"):
        for op, f in ((BinaryOp.ADD, np.add), (BinaryOp.SUB, np.subtract), (BinaryOp.MUL, np.multiply),
                      (BinaryOp.DIV, np.divide)):
            got = ops.binary(op, at, al, bt, bl).to_numpy()
            want = f(a, b).astype(np.float32)
            same = (bits(got) == bits(want)) | (np.isnan(got) & np.isnan(want))
            assert same.all(), op.name
        for op, f in ((CmpOp.GT, np.greater), (CmpOp.GE, np.greater_equal), (CmpOp.LT, np.less),
                      (CmpOp.LE, np.less_equal), (CmpOp.EQ, np.equal)):
            got = ops.compare(op, at, Layout(a.shape), 1.0).to_numpy()
            assert np.array_equal(got, f(a, np.float32(1.0)).astype(np.uint8)), op.name
    m = (rng.random((1, 33)) < 0.4).astype(np.uint8)
    got = ops.mask_fill(at, Layout(a.shape), dev(m, "bool"), Layout(m.shape).broadcast(out), -1e9).to_numpy()
    want = np.where(m != 0, np.float32(-1e9), a).astype(np.float32)
    assert np.array_equal(bits(got), bits(want))  # a select: NaN bits included


@pytest.mark.parametrize("shape,dim", [((64, 1000), 1), ((3, 50304), 1), ((5, 7, 9), 1), ((5, 7, 9), 0),
                                       ((4, 1, 13), 2), ((1, 1), 1), ((2, 17), 0), ((1, 129), 1)])
def test_reductions_in_cpurefs_order(shape, dim):
    rng = np.random.default_rng(sum(shape) + dim)
    x = (rng.normal(0, 1, shape) * 2.0 ** rng.integers(-10, 10, shape)).astype(np.float32)
    xt = dev(x)
    got = ops.reduce_dim(ReduceOp.SUM, xt, list(shape), dim).to_numpy()
    want = T.sum_dim(x, list(shape), dim)
    assert np.array_equal(bits(got), bits(want)), "sum"
    x.ravel()[:: max(1, x.size // 5)] = 40.0  # ties: the first maximum
    if x.size > 3:
        x.ravel()[3] = np.nan
    xt = dev(x)
    idx, val = T.argmax_dim(x, list(shape), dim)
    gi = ops.reduce_dim(ReduceOp.ARGMAX, xt, list(shape), dim).to_numpy()
    gv = ops.reduce_dim(ReduceOp.MAX, xt, list(shape), dim).to_numpy()
    assert np.array_equal(gi, idx.astype(np.int32))
    assert np.array_equal(np.isnan(gv), np.isnan(val)) and np.array_equal(gv[~np.isnan(gv)], val[~np.isnan(val)])


def test_reduce_all():
    rng = np.random.default_rng(7)
    for n in (1, 7, 8, 9, 1000, 65537):
        x = rng.normal(0, 1, n).astype(np.float32)
        s = ops.reduce_all(ReduceOp.SUM, dev(x), n).to_numpy()[0]
        assert np.float32(s).view(np.uint32) == np.float32(O.unrolled_sum(x)).view(np.uint32)
        m = ops.reduce_all(ReduceOp.MAX, dev(x), n).to_numpy()[0]
        assert m == T.max_all(x)
    x[500] = np.nan
    assert np.isnan(ops.reduce_all(ReduceOp.MAX, dev(x), len(x)).to_numpy()[0])


def test_indexing_ops():
    rng = np.random.default_rng(8)
    outer, n, inner, m = 3, 11, 4, 6
    x = rng.normal(0, 1, (outer, n, inner)).astype(np.float32)
    idx = rng.integers(0, n, (outer, m, inner)).astype(np.int32)
    got = ops.gather(dev(x), (outer, n, inner, m), dev(idx)).to_numpy()
    assert np.array_equal(got, np.take_along_axis(x, idx, axis=1))
    bad = idx.copy()
    bad[0, 0, 0], bad[1, 2, 3] = -1, n
    g2 = ops.gather(dev(x), (outer, n, inner, m), dev(bad)).to_numpy()
    assert np.isnan(g2[0, 0, 0]) and np.isnan(g2[1, 2, 3]) and np.isnan(g2).sum() == 2
    sel = rng.integers(0, n, m).astype(np.int32)
    got = ops.index_select(dev(x), (outer, n, inner, m), dev(sel)).to_numpy()
    assert np.array_equal(got, x[:, sel, :])
    oh = ops.one_hot(dev(sel), m, n).to_numpy()
    assert np.array_equal(oh, (sel[:, None] == np.arange(n)[None, :]).astype(np.float32))
    v = rng.normal(0, 1, (outer, m, inner)).astype(np.float32)
    got = ops.scatter_add(dev(idx), dev(v), (outer, n, inner, m)).to_numpy()
    want = np.zeros((outer, n, inner), np.float32)
    for o in range(outer):
        for k in range(m):  # ascending source order, in f32
            for i in range(inner):
                want[o, idx[o, k, i], i] = want[o, idx[o, k, i], i] + v[o, k, i]
    assert np.array_equal(bits(got), bits(want))
    got = ops.index_add(dev(sel), dev(v), (outer, n, inner, m)).to_numpy()
    want = np.zeros((outer, n, inner), np.float32)
    for k in range(m):
        want[:, sel[k], :] = want[:, sel[k], :] + v[:, k, :]
    assert np.array_equal(bits(got), bits(want))
    f = ops.fill((5, 3), -2.5).to_numpy()
    assert np.all(f == np.float32(-2.5))


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_tempered_logits_from_the_general_ops(dtype):
    rng = np.random.default_rng(9)
    x = rng.normal(0, 2, (2, 3, 4, 257)).astype(np.float32)
    mask = np.where(rng.random((1, 1, 1, 257)) < 0.2, -np.inf, 0.0).astype(np.float32)
    mask[..., 5] = -1e9
    if dtype == "bf16":
        xb = O.bf16_from_f32(x)
        x, xt = O.bf16_to_f32(xb), dev(xb, "bf16")
    else:
        xt = dev(x)
    for tau in (1.0, 0.7):
        if dtype == "bf16" and tau == 1.0:
            # not divided, bf16 logits meet the f32 mask in add's same_dtype check (rl.rs:476-483)
            with pytest.raises(nr.DTypeError, match=r"^add: bf16 and f32 \(casts are explicit\)$"):
                ops.tempered_logits(xt, tau, dev(mask))
            continue
        z = ops.tempered_logits(xt, tau, dev(mask)).to_numpy().reshape(-1, 257)
        want = O.tempered(x.reshape(-1, 257), tau, addmask=mask.reshape(1, 257))
        assert np.array_equal(bits(z), bits(want))
    assert ops.tempered_logits(xt, 1.0, None) is xt


def test_release_is_stream_ordered():
    """nt_hip_free only records the pointer; the next entry frees it on the stream after the work
    queued before it (the reference's deferred, stream-ordered free). A buffer released while a
    kernel that reads it is still queued, then memory taken again and filled, leaves that kernel's
    result intact."""
    import ctypes as C
    L = nr.lib()
    n = 1 << 24
    x = np.random.default_rng(10).normal(0, 1, n).astype(np.float32)
    for _ in range(3):
        xt = dev(x)
        y = nr.Tensor((n,), "f32")
        nr._check(L.nt_hip_unary(int(UnaryOp.EXP), 0.0, C.c_void_p(xt.ptr), C.byref(Layout([n]).c()), C.c_void_p(y.ptr)),
                  "exp")
        del xt  # released with the exp still queued
        z = ops.fill((n,), 7.0)  # new memory, possibly the same block, written on the stream
        got = y.to_numpy()
        assert np.array_equal(got, ops.unary(UnaryOp.EXP, dev(x), Layout([n])).to_numpy())
        assert np.all(z.to_numpy() == np.float32(7.0))


def test_key_and_platform_details():
    """`key` and `platform_details` (gpu/mod.rs:197-199), joined as `gpu_platform_key`
    (gpu/mod.rs:699-704): stable across calls, no spaces, and a buffer too small is an error."""
    import ctypes as C
    import re

    k, d = nr.key(), nr.platform_details()
    assert re.fullmatch(r"hip-gfx950[^ ]*-hiprt\d+-kernels-[0-9a-f]{16}", k), k
    assert re.fullmatch(r"hipdriver\d+-amdgpu-[^ ]+-clang-[^ ]+", d), d
    assert nr.platform_key() == f"{k}-{d}"
    assert (nr.key(), nr.platform_details()) == (k, d)
    small = C.create_string_buffer(8)
    assert nr.lib().nt_hip_platform_details(small, 8) != 0
    assert "too small" in nr.lib().nt_hip_last_error().decode()
    print("platform key:", nr.platform_key())
