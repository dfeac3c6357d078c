"""The reference's Gumbel-max sample_categorical on the device (nt_hip_rl_sample_gumbel, through
noetic_rl.sample_categorical) against Cpu(Reference)'s op sequence for the same stream (the
oracle's restatement, or_cpuref_sample_gumbel: tempered_logits, the max_dim refusal, one u64
per logit in row-major order, f32(-ln(-ln u)), z + g, the first argmax).

The reference's own contract (src/nn/tests/gpu/rl.rs:155-174): at most 1 token in 1000 may
differ from CpuRef for the same stream (two perturbed logits rounding differently), greedy equal,
none excluded, identical run to run; and (src/nn/tests/rl.rs:579-625) the stream advances by one
u64 per logit, greedy draws nothing, frequencies within 4.5 standard errors.
"""
import numpy as np
import pytest
from scipy.special import log_softmax

import noetic_rl as nr
import workloads as W
from oracle import oracle as O

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def device():
    nr.claim(0)
    yield


def both(x, tau, root, label, addmask=None, keep=None, dev_logits=None, dev_mask=None, pre_u32=0):
    """Device and CpuRef tokens for rows x [R, V] under the same stream."""
    R, V = x.shape
    if dev_logits is None:
        dev_logits = nr.Tensor.from_numpy(np.ascontiguousarray(x, np.float32))
    m = dev_mask
    if m is not None:
        pass
    elif addmask is not None:
        m = nr.Tensor.from_numpy(np.ascontiguousarray(addmask, np.float32))
    elif keep is not None:
        m = nr.Tensor.from_numpy(np.ascontiguousarray(keep, np.uint8), "u8")
    rd, rc = nr.Rng(root, label), O.Rng(root, label)
    for _ in range(pre_u32):
        rd.next_u32()
        rc.next_u32()
    dev = nr.sample_categorical(dev_logits, tau, m, rd).to_numpy().ravel().astype(np.int64)
    cpu = O.cpuref_sample_gumbel(x, tau, rc, addmask=addmask, keep=keep)
    # both streams have moved on by the same count
    assert rd.next_u64() == rc.next_u64(), "device and CpuRef streams advanced differently"
    return dev, cpu


def test_reference_sampler_body_on_the_device():
    # src/nn/tests/gpu/rl.rs:155-174 on the reference's own inputs: rnd(n * V, 960, -3, 3) as f32,
    # an additive [1, 1, V] mask with -inf at k % 7 == 3, temperatures 1 (root 11), 0.7 (root 12)
    # and 0 (root 13) of derive(root, "device sampler").
    shape = (4, 128, 96)
    n, V = shape[0] * shape[1], shape[2]
    x = O.reference_rnd_f64(960, n * V, -3.0, 3.0).astype(np.float32).reshape(n, V)
    mask = np.array([[-np.inf if k % 7 == 3 else 0.0 for k in range(V)]], np.float32)
    xt = nr.Tensor.from_numpy(x.reshape(shape))
    mt = nr.Tensor.from_numpy(mask.reshape(1, 1, V))
    dev, cpu = [], []
    for tau, root in [(1.0, 11), (0.7, 12), (0.0, 13)]:
        d = nr.sample_categorical(xt, tau, mt, nr.Rng(root, "device sampler")).to_numpy().ravel()
        c = O.cpuref_sample_gumbel(x, tau, O.Rng(root, "device sampler"), addmask=mask)
        assert d.shape == (n,)
        dev.append(d)
        cpu.append(c)
    differ = 0
    for d, c in zip(dev, cpu):
        assert np.all(d % 7 != 3), "an excluded token was drawn"
        differ += int(np.sum(d != c))
    assert np.array_equal(dev[2], cpu[2]), "greedy tokens differ from CpuRef"
    assert differ * 1000 <= 3 * n, f"{differ} of {3 * n} sampled tokens differ from CpuRef"
    again = [nr.sample_categorical(xt, tau, mt, nr.Rng(root, "device sampler")).to_numpy().ravel()
             for tau, root in [(1.0, 11), (0.7, 12), (0.0, 13)]]
    for a, d in zip(again, dev):
        assert np.array_equal(a, d), "sampler run to run"
    print(f"hip rl sampler: {differ} of {3 * n} tokens differ from CpuRef for the same stream (greedy equal), "
          f"none excluded, identical run to run")


def test_the_stream_advances_one_u64_per_logit():
    # tests/rl.rs:596-599 (one u64 per logit) and 624 (greedy draws nothing)
    rows, V = 37, 29
    x = nr.Tensor.from_numpy(np.random.default_rng(1).normal(0, 1, (rows, V)).astype(np.float32))
    rng = nr.Rng(5, "sampler test")
    copy = rng.clone()
    nr.sample_categorical(x, 0.7, None, rng)
    for _ in range(rows * V):
        copy.next_u64()
    assert rng.next_u64() == copy.next_u64(), "one u64 per logit"
    rng = nr.Rng(1, "greedy")
    copy = rng.clone()
    nr.sample_categorical(x, 0.0, None, rng)
    assert rng.next_u64() == copy.next_u64(), "greedy draws nothing"
    # a refused call draws nothing either (the reference panics before its draw, rl.rs:515-519)
    keep = np.ones((rows, V), np.uint8)
    keep[4] = 0
    rng = nr.Rng(2, "refused")
    copy = rng.clone()
    with pytest.raises(ValueError, match="position 4 has no allowed token"):
        nr.sample_categorical(x, 1.0, nr.Tensor.from_numpy(keep, "u8"), rng)
    assert rng.next_u64() == copy.next_u64(), "a refused call moved the stream"


def test_frequencies_and_streams():
    # tests/rl.rs:579-611: 40,000 copies of one row, mask [1, V], frequencies against
    # softmax(l/T + mask) within 4.5 standard errors, the same stream gives the same tokens, another
    # stream other tokens; and every token equal to CpuRef's for the same stream.
    row = np.array([0.4, -1.0, 1.2, 3.0, 0.0, -0.3], np.float32)
    maskrow = np.array([[0.0, 0.0, 0.0, -np.inf, 0.5, 0.0]], np.float32)
    n, v = 40_000, 6
    x = np.repeat(row[None, :], n, 0)
    xt, mt = nr.Tensor.from_numpy(x), nr.Tensor.from_numpy(maskrow)
    for tau in (0.7, 1.0, 2.5):
        tok, cpu = both(x, tau, 5, "sampler test", addmask=maskrow, dev_logits=xt)
        assert np.array_equal(tok, cpu), f"T={tau}: {int(np.sum(tok != cpu))} tokens differ from CpuRef"
        z = row.astype(np.float64) / tau + maskrow[0].astype(np.float64)
        p = np.exp(log_softmax(z))
        cnt = np.bincount(tok, minlength=v)
        assert cnt[3] == 0, "excluded token drawn"
        se = np.sqrt(p * (1 - p) / n)
        assert np.all(np.abs(cnt / n - p) <= 4.5 * se + 1e-12), f"T={tau}: {cnt / n} vs {p}"
        again = nr.sample_categorical(xt, tau, mt, nr.Rng(5, "sampler test")).to_numpy()
        assert np.array_equal(again, tok), "same stream, same tokens"
        other = nr.sample_categorical(xt, tau, mt, nr.Rng(6, "sampler test")).to_numpy()
        assert not np.array_equal(other, tok)


@pytest.mark.parametrize("pre_u32", [0, 1, 6, 15])
@pytest.mark.parametrize("V", [1, 7, 37, 1000, 4099])
def test_ragged_rows_at_every_stream_offset(V, pre_u32):
    # rows that start anywhere inside a keystream block, and odd word positions (a next_u32
    # before the call), so u64 draws straddle blocks: every token equal to CpuRef's
    rng = np.random.default_rng(V + 100 * pre_u32)
    rows = 41
    x = rng.normal(0, 2, (rows, V)).astype(np.float32)
    keep = (rng.random((rows, V)) < 0.7).astype(np.uint8)
    keep[np.arange(rows), rng.integers(0, V, rows)] = 1
    for tau in (1.0, 0.6):
        dev, cpu = both(x, tau, V, "ragged", keep=keep, pre_u32=pre_u32)
        assert np.array_equal(dev, cpu), f"V={V} +{pre_u32} words T={tau}: rows {np.nonzero(dev != cpu)[0][:8]}"
        assert keep[np.arange(rows), dev].all()


def test_c4_gumbel_against_cpuref():
    # C4's bf16 rows and grammar mask through the reference's sampler: the device noise against
    # CpuRef's for the same stream, all 256 rows (32.8 M draws)
    w = W.c4()
    rows, V = w["rows"], w["V"]
    x = W.bf16_to_f32(w["logits"].to_numpy().reshape(rows, V))
    keep = w["mask"].to_numpy().reshape(rows, V)
    dev, cpu = both(x, w["temperature"], 2024, "c4/gumbel", keep=keep, dev_logits=w["logits"], dev_mask=w["mask"])
    differ = int(np.sum(dev != cpu))
    assert keep[np.arange(rows), dev].all(), "an excluded token was drawn"
    assert differ * 1000 <= rows, f"c4: {differ} of {rows} tokens differ from CpuRef"
    print(f"c4 gumbel: {differ} of {rows} tokens differ from CpuRef for the same stream")


def test_additive_masks_nan_and_infinite_logits():
    # -1e9 and -inf masks give the same tokens (rl.rs:16-19); a NaN refuses its row whatever the
    # mask; +inf logits win over finite ones, the first +inf among several
    rng = np.random.default_rng(3)
    rows, V = 16, 53
    x = rng.normal(0, 1, (rows, V)).astype(np.float32)
    x[2, 7] = np.inf
    x[2, 31] = np.inf
    out = []
    for fill in (-1e9, -np.inf):
        m = np.zeros((1, V), np.float32)
        m[0, ::5] = fill
        d, c = both(x, 0.8, 9, "masks", addmask=m)
        assert np.array_equal(d, c)
        out.append(d)
    assert np.array_equal(out[0], out[1])
    assert out[0][2] == 7
    x[5, 11] = np.nan
    with pytest.raises(ValueError, match="position 5 has no allowed token"):
        nr.sample_categorical(nr.Tensor.from_numpy(x), 0.8, None, nr.Rng(9, "masks"))


@pytest.mark.parametrize("pre_u32", [0, 1])
def test_many_near_ties_take_the_exact_path(pre_u32):
    # logits near 1e9, 64 apart (f32's spacing there): z + g rounds back to z unless g passes 32,
    # so every block's elements of the largest z tie, the threads' candidate slots run out and
    # those rows take the exact evaluation of every element. The first maximum in index order
    # must still be CpuRef's, on an even and an odd stream position, beside rows (1e4 + noise)
    # that take the screen.
    rng = np.random.default_rng(17)
    rows, V = 12, 4099
    x = (1e9 + 64.0 * rng.integers(0, 3, (rows, V))).astype(np.float32)
    x[6:] = (1e4 + rng.normal(0, 0.01, (rows - 6, V))).astype(np.float32)
    d, c = both(x, 1.0, 21, "near ties", pre_u32=pre_u32)
    assert np.array_equal(d, c), f"tokens differ from CpuRef: {np.nonzero(d != c)[0]}"


@pytest.mark.parametrize("mask", ["none", "keep", "add"])
@pytest.mark.parametrize("tau", [1.0, 0.7])
@pytest.mark.parametrize("pre_u32", [0, 1])
def test_large_logits_where_an_ulp_of_the_sum_passes_the_absolute_margin(pre_u32, tau, mask):
    # At |z| of 2^16 and 1e6 an ulp of z + g (2^-7, 2^-4) is wider than the screen's 1e-3: the
    # screened and exact sums of two elements can order differently by an ulp, and exact sums tie
    # often. The margin grows with |z| (4 ulps), so the row's few candidates within it are
    # evaluated exactly (or the single one is the answer), and the first maximum is CpuRef's.
    rng = np.random.default_rng(23)
    rows, V = 24, 6007
    x = np.empty((rows, V), np.float32)
    x[:8] = 65536.0 + rng.normal(0, 1.0, (8, V))
    x[8:16] = 1e6 + rng.normal(0, 0.5, (8, V))
    x[16:] = -3e5 + rng.normal(0, 0.2, (8, V))
    # (a u8 keep-mask divides only the queued blocks by tau; an additive f32 mask divides first)
    keep = addmask = None
    if mask == "keep":
        keep = (rng.random((rows, V)) < 0.5).astype(np.uint8)
        keep[:, 0] = 1
    elif mask == "add":
        addmask = np.where(rng.random((1, V)) < 0.5, -np.inf, 0.0).astype(np.float32)
        addmask[0, 0] = 0.0
    d, c = both(x, tau, 29, "large logits", keep=keep, addmask=addmask, pre_u32=pre_u32)
    assert np.array_equal(d, c), f"tokens differ from CpuRef: {np.nonzero(d != c)[0]}"


def gumbel_call(xt, dtype, kind, rows, V, ld, mt, mask_ld, tau, rng):
    """nt_hip_rl_sample_gumbel through the C ABI at `rng`'s position: (ids, status); the stream
    is not moved."""
    import ctypes as C
    ids, st = nr.IntTensor((rows,)), nr.Tensor((rows,), "u8")
    block, word = rng.word_pos()
    a = nr.NtRlGumbelArgs(xt.ptr, dtype, kind, rows, V, ld, None if mt is None else mt.ptr, mask_ld, tau,
                          rng.key(), block, word, 0, ids.ptr, st.ptr)
    nr._check(nr.lib().nt_hip_rl_sample_gumbel(C.byref(a)), "sample_gumbel")
    return ids.to_numpy().ravel().astype(np.int64), st.to_numpy().ravel()


@pytest.mark.parametrize("pre_u32", [0, 1])
@pytest.mark.parametrize("V", [4096, 4099])
def test_u8_excluded_non_finite_logits_do_not_reach_the_row(V, pre_u32):
    """A u8 keep-mask selects: NaN and +inf at excluded tokens (inside blocks that keep a token
    and in blocks that keep none) leave the row to sample as Cpu(Reference)'s sequence does with
    the same rule; +inf at a kept token wins (the first one); NaN at a kept token refuses the row.
    V = 4096 at an even stream position takes the aligned path, the rest the element-wise one."""
    rng = np.random.default_rng(V + pre_u32)
    rows = 8
    x = rng.normal(0, 2, (rows, V)).astype(np.float32)
    keep = (rng.random((rows, V)) < 0.6).astype(np.uint8)
    keep[:, 100] = 1
    x[0, 5], keep[0, 5] = np.nan, 0
    x[1, 9], keep[1, 9] = np.inf, 0
    keep[2, 16:24] = 0
    x[2, 16:24] = np.nan  # a whole block excluded
    keep[3, 40:48] = [1, 0, 1, 0, 1, 1, 0, 1]
    x[3, 41], x[3, 43], x[3, 46] = np.nan, np.inf, -np.inf
    x[4, 200], keep[4, 200] = np.inf, 1
    x[4, 300], keep[4, 300] = np.inf, 1
    x[5, V - 1], keep[5, V - 1] = np.nan, 0
    for tau in (1.0, 0.7, 0.0):
        dev, cpu = both(x, tau, 31, "u8 non-finite", keep=keep, pre_u32=pre_u32)
        assert np.array_equal(dev, cpu), f"tau={tau}: rows {np.nonzero(dev != cpu)[0]}"
        assert keep[np.arange(rows), dev].all()
        assert dev[4] == 200
    # NaN at a kept token: that row alone is refused (status through the C ABI), nothing drawn
    x2 = x.copy()
    x2[6, 100] = np.nan
    rd = nr.Rng(31, "u8 non-finite")
    for _ in range(pre_u32):
        rd.next_u32()
    ids, st = gumbel_call(nr.Tensor.from_numpy(x2), nr.NT_F32, nr.NT_MASK_U8, rows, V, V,
                          nr.Tensor.from_numpy(keep, "u8"), V, 0.7, rd)
    assert st[6] == nr.NT_ROW_NAN and ids[6] == -1
    assert np.all(st[np.arange(rows) != 6] == nr.NT_ROW_OK)


@pytest.mark.parametrize("pre_u32", [0, 1])
@pytest.mark.parametrize("V", [4096, 4099])
@pytest.mark.parametrize("mask", ["none", "keep"])
def test_rows_below_minus_flt_max_tau_have_no_token(mask, V, pre_u32):
    """Every allowed logit at -3.3e38 with T = 0.7: the tempered values x / T are all -inf, so the
    reference's max_dim is -inf and the row is refused before any draw (rl.rs:515-519), even where
    the keep-mask excludes token 0. A row with only some of its allowed logits there samples
    among the others as Cpu(Reference) does."""
    rows = 4
    rng = np.random.default_rng(V)
    x = rng.normal(0, 1, (rows, V)).astype(np.float32)
    keep = np.ones((rows, V), np.uint8) if mask == "keep" else None
    x[1] = -3.3e38
    if keep is not None:
        keep[1, 0] = 0
    mt = None if keep is None else nr.Tensor.from_numpy(keep, "u8")
    kind = nr.NT_MASK_NONE if keep is None else nr.NT_MASK_U8
    rd = nr.Rng(41, "below -FLT_MAX T")
    for _ in range(pre_u32):
        rd.next_u32()
    ids, st = gumbel_call(nr.Tensor.from_numpy(x), nr.NT_F32, kind, rows, V, V, mt, 0 if mt is None else V, 0.7, rd)
    assert st[1] == nr.NT_ROW_NO_TOKEN and ids[1] == -1, (st, ids)
    assert np.all(st[[0, 2, 3]] == nr.NT_ROW_OK)
    copy = rd.clone()
    with pytest.raises(ValueError, match="position 1 has no allowed token"):
        nr.sample_categorical(nr.Tensor.from_numpy(x), 0.7, mt, rd)
    assert rd.next_u64() == copy.next_u64(), "a refused call moved the stream"
    # half of row 1's logits back to normal values: it samples among them
    x[1, ::2] = rng.normal(0, 1, (V + 1) // 2).astype(np.float32)
    dev, cpu = both(x, 0.7, 41, "below -FLT_MAX T", keep=keep, pre_u32=pre_u32)
    assert np.array_equal(dev, cpu) and dev[1] % 2 == 0


@pytest.mark.parametrize("pre_u32", [0, 1])
@pytest.mark.parametrize("V", [1001, 4096, 4099])
@pytest.mark.parametrize("mask", ["u8", "f32add"])
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_strided_rows_through_the_c_abi(dtype, mask, V, pre_u32):
    """Rows and mask rows with a padded stride (ld and mask_ld V rounded up to 8, and 16 more)
    whose padding holds NaN logits and keep bytes of 1 / NaN mask values: nothing past V is
    read. Every token equal to Cpu(Reference)'s on the unpadded rows, at an even and an odd
    stream position."""
    rows = 9
    rng = np.random.default_rng(V * 4 + pre_u32)
    x = rng.normal(0, 2, (rows, V)).astype(np.float32)
    ld = -(-V // 8) * 8 + 16
    if dtype == "bf16":
        xb = O.bf16_from_f32(x)
        x = O.bf16_to_f32(xb)
        pad = np.full((rows, ld), 0x7fc0, np.uint16)
        pad[:, :V] = xb
        xt, dt = nr.Tensor.from_numpy(pad, "bf16"), nr.NT_BF16
    else:
        pad = np.full((rows, ld), np.nan, np.float32)
        pad[:, :V] = x
        xt, dt = nr.Tensor.from_numpy(pad), nr.NT_F32
    keep = addmask = None
    if mask == "u8":
        keep = (rng.random((rows, V)) < 0.5).astype(np.uint8)
        keep[:, V // 2] = 1
        mpad = np.ones((rows, ld), np.uint8)
        mpad[:, :V] = keep
        mt, kind = nr.Tensor.from_numpy(mpad, "u8"), nr.NT_MASK_U8
    else:
        addmask = np.where(rng.random((rows, V)) < 0.5, -np.inf, 0.0).astype(np.float32)
        addmask[:, V // 2] = 0.0
        mpad = np.full((rows, ld), np.nan, np.float32)
        mpad[:, :V] = addmask
        mt, kind = nr.Tensor.from_numpy(mpad), nr.NT_MASK_F32
    for tau in (1.0, 0.7):
        rd, rc = nr.Rng(53, "strided"), O.Rng(53, "strided")
        for _ in range(pre_u32):
            rd.next_u32()
            rc.next_u32()
        ids, st = gumbel_call(xt, dt, kind, rows, V, ld, mt, ld, tau, rd)
        assert np.all(st == nr.NT_ROW_OK), st
        cpu = O.cpuref_sample_gumbel(x, tau, rc, addmask=addmask, keep=keep)
        assert np.array_equal(ids, cpu), f"tau={tau}: rows {np.nonzero(ids != cpu)[0]}"
