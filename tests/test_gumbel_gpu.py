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
