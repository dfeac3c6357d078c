"""The queued sampler (u8 keep-masks, one workgroup per row) against the oracle.

The kernel reads each wave's mask first and queues, in index order, the lane groups (8
consecutive elements) that keep a token; slot j of a stage holds queue entries [64 j, 64 j + 64)
and only their logits are read. A wave whose first stage keeps a token in more than 70% of its
lane groups takes the dense path instead (every group loaded in place). These cases put the draw
where the queue's levels meet:
- grammar-like masks of kept runs (the C4 workload's kind) at every chunks-per-wave K the kernel
  is built for (bf16 4, 8, 16; f32 4, 8), V just past a K boundary and just below the next;
- rows whose kept tokens are one run inside one wave, the row's last element only, its first
  element only; the row's maximum in its last element with every other logit 200 below; a peaked
  row; rows dense in some waves' first stage and sparse in others (both paths in one row);
- temperature 1, 0.7 and 0 (greedy: the first maximum in index order), with entropy;
- refusals: a NaN or +inf at a kept token refuses the row, a NaN or +inf at an excluded token
  (inside a queued lane group or in a group never read) does not, a row with nothing kept is
  refused with NT_ROW_NO_TOKEN;
- 1024 rows (four workgroups per compute unit, each starting on the LDS its predecessor left) and
  one shared mask row (mask_ld 0), against the register-resident sampler on the same inputs.
ids must equal the oracle's except for draws within 1e-6 of a CDF edge; logp and entropy hold
1e-5 relative / 1e-6 absolute (the bf16 inputs are exact in f32, and the kernel computes in f32
and f64).
"""
import ctypes as C

import numpy as np
import pytest

import noetic_rl as nr
import workloads as W
from oracle import oracle as O

pytestmark = pytest.mark.gpu

EDGE = 1e-6
CHUNK = 512
WAVES = 16


@pytest.fixture(scope="module", autouse=True)
def device():
    nr.claim(0)
    yield


def close(ours, want):
    ours, want = np.asarray(ours, np.float64), np.asarray(want, np.float64)
    return np.abs(ours - want) <= 1e-6 + 1e-5 * np.abs(want)


def runs(rng, n, kept_mean, gap_mean):
    """A keep-mask of n tokens: alternating excluded and kept runs, lengths uniform in
    [1, 2 mean - 1], starting with a gap of random phase."""
    out = np.zeros(n, np.uint8)
    pos = -int(rng.integers(0, 2 * gap_mean))
    while pos < n:
        pos += int(rng.integers(1, 2 * gap_mean))
        k = int(rng.integers(1, 2 * kept_mean))
        out[max(pos, 0):max(min(pos + k, n), 0)] = 1
        pos += k
    return out


def rows_for(V, K, rng):
    rows = 16
    x = rng.normal(0, 2, (rows, V)).astype(np.float32)
    keep = np.stack([runs(rng, V, 96, 224) for _ in range(rows)])
    keep[:, 0] |= rng.integers(0, 2, rows).astype(np.uint8)
    span = K * CHUNK  # elements per wave
    stage = span // (2 if K >= 8 else 1)  # a wave's first stage
    # row 1: one run inside wave 3's range (or the last wave holding elements)
    w = min(3, (V - 1) // span)
    keep[1] = 0
    keep[1, w * span + 100:min(V, w * span + 260)] = 1
    # rows 2 and 3: only the last element, only the first
    keep[2] = 0
    keep[2, V - 1] = 1
    keep[3] = 0
    keep[3, 0] = 1
    # row 4: the maximum in the last element, every other logit 200 below it
    x[4] -= 200.0
    x[4, V - 1] = 5.0
    keep[4, V - 1] = 1
    # row 5: peaked, the mass on one token of the middle wave's range
    mid = min(V - 1, (V // span // 2) * span + 7)
    x[5, mid] = 40.0
    keep[5, mid] = 1
    # rows 6 and 7: every wave's first stage dense (the dense path) over sparse runs elsewhere,
    # and the even waves dense, the odd ones sparse (both paths in one row)
    for r, waves in ((6, range(WAVES)), (7, range(0, WAVES, 2))):
        for wv in waves:
            a, b = wv * span, min(V, wv * span + stage)
            if a < V:
                keep[r, a:b] = (rng.random(b - a) < 0.95)
    # row 8: everything kept (dense everywhere)
    keep[8] = 1
    return x, keep


def cases():
    out = []
    for dtype, ks in (("bf16", (4, 8, 16)), ("f32", (4, 8))):
        for K in ks:
            out += [(dtype, K, WAVES * (K // 2) * CHUNK + 8), (dtype, K, WAVES * K * CHUNK - 40)]
    return out


def tensors(x, keep, dtype):
    if dtype == "bf16":
        xb = O.bf16_from_f32(x)
        return O.bf16_to_f32(xb), nr.Tensor.from_numpy(xb, "bf16"), nr.Tensor.from_numpy(keep)
    return x, nr.Tensor.from_numpy(x), nr.Tensor.from_numpy(keep)


@pytest.mark.parametrize("dtype,K,V", cases())
def test_queued_sampler_levels(dtype, K, V, monkeypatch):
    monkeypatch.setenv("NOETIC_HIP_SAMPLE_SEG", "off")  # one workgroup per row, whatever the row count
    rng = np.random.default_rng(V * 3 + K)
    x, keep = rows_for(V, K, rng)
    x, xt, mt = tensors(x, keep, dtype)
    rows = x.shape[0]
    u = np.random.default_rng(V + K).random(rows)
    u[0], u[6] = 0.0, np.nextafter(1.0, 0.0)  # the first and the last weight
    ut = nr.Tensor.from_numpy(u, "f64")
    for tau in (1.0, 0.7, 0.0):
        ids, lp, ent = nr.sample_logp(xt, tau, mt, None, entropy=True, uniforms=None if tau == 0.0 else ut)
        ids, lp, ent = ids.to_numpy(), lp.to_numpy(), ent.to_numpy()
        z = O.tempered(x, 1.0 if tau == 0.0 else tau, keep=keep)
        if tau == 0.0:
            zz = np.where(np.isfinite(z), z, -np.inf)
            assert np.array_equal(ids, np.argmax(zz, axis=1)), f"{dtype} K={K} V={V}: greedy ids"
        else:
            want, edges = O.sample_invcdf(z, u)
            differ = np.nonzero(ids != want)[0]
            assert np.all(edges[differ] < EDGE), f"{dtype} K={K} V={V} tau={tau}: rows {differ} differ"
            # the register-resident sampler on the same bytes: the same ids off the edges
            monkeypatch.setenv("NOETIC_HIP_SAMPLE_QUEUE", "off")
            rr = nr.sample_logp(xt, tau, mt, None, uniforms=ut)[0].to_numpy()
            monkeypatch.delenv("NOETIC_HIP_SAMPLE_QUEUE")
            d2 = np.nonzero(ids != rr)[0]
            assert np.all(edges[d2] < EDGE), f"{dtype} K={K} V={V} tau={tau}: rows {d2} differ from the rr kernel"
        assert keep[np.arange(rows), ids].all(), f"{dtype} K={K} V={V} tau={tau}: an excluded token was drawn"
        assert np.all(close(lp, O.token_logp(z, ids))), f"{dtype} K={K} V={V} tau={tau}: logp"
        assert np.all(close(ent, O.entropy(z))), f"{dtype} K={K} V={V} tau={tau}: entropy"
        assert ids[2] == V - 1 and ids[3] == 0 and ids[4] == V - 1


@pytest.mark.parametrize("dtype,V", [("bf16", WAVES * 16 * CHUNK - 8), ("bf16", WAVES * 4 * CHUNK - 8),
                                     ("f32", WAVES * 8 * CHUNK - 8)])
def test_queued_sampler_refusals(dtype, V):
    """Row by row: NaN at a kept token (first wave, a middle wave, the last element) or +inf at
    a kept token -> NT_ROW_NAN; nothing kept -> NT_ROW_NO_TOKEN; NaN and +inf at excluded tokens,
    inside a lane group that keeps a token and in groups that keep none (never read), leave the
    row to sample as the oracle does."""
    rows = 12
    rng = np.random.default_rng(V + 5)
    x = rng.normal(0, 2, (rows, V)).astype(np.float32)
    keep = np.stack([runs(rng, V, 96, 224) for _ in range(rows)])
    keep[:, 64] = 1
    span = V // WAVES
    for r, pos in ((0, 5), (1, 9 * span + 3), (2, V - 1)):
        x[r, pos] = np.nan
        keep[r, pos] = 1
    x[4, 7] = np.inf
    keep[4, 7] = 1
    keep[5] = 0
    # rows 6-9: non-finite logits at excluded tokens only
    keep[6, 64:72] = [1, 0, 1, 1, 1, 1, 1, 1]
    x[6, 65] = np.nan  # in a queued group
    keep[7, 1024:1032] = [1, 1, 1, 1, 1, 1, 1, 0]
    x[7, 1031] = np.inf
    keep[8, 2048:4096] = 0
    x[8, 2048:4096] = np.nan  # groups never read
    keep[9, 3000:3100] = 0
    x[9, 3000:3100:7] = np.inf
    x, xt, mt = tensors(x, keep, dtype)
    nan_rows, none_rows = {0, 1, 2, 4}, {5}
    u = np.random.default_rng(3).random(rows)
    ut = nr.Tensor.from_numpy(u, "f64")
    ids, lp, ent, st = nr.IntTensor((rows,)), nr.Tensor((rows,), "f32"), nr.Tensor((rows,), "f32"), nr.Tensor((rows,), "u8")
    a = nr.NtRlSampleArgs(xt.ptr, nr.NT_BF16 if dtype == "bf16" else nr.NT_F32, nr.NT_MASK_U8, rows, V, V, mt.ptr, V,
                          0.9, ut.ptr, ids.ptr, lp.ptr, ent.ptr, st.ptr)
    nr._check(nr.lib().nt_hip_rl_sample(C.byref(a)), "sample")
    ids, lp, ent, st = ids.to_numpy(), lp.to_numpy(), ent.to_numpy(), st.to_numpy()
    for r in range(rows):
        if r in nan_rows:
            assert st[r] == nr.NT_ROW_NAN and ids[r] == -1 and np.isnan(lp[r]), f"row {r}: {st[r]} {ids[r]}"
        elif r in none_rows:
            assert st[r] == nr.NT_ROW_NO_TOKEN and ids[r] == -1, f"row {r}: {st[r]}"
        else:
            assert st[r] == nr.NT_ROW_OK, f"row {r}: status {st[r]}"
    ok = np.array([r for r in range(rows) if r not in nan_rows | none_rows])
    z = O.tempered(x[ok], 0.9, keep=keep[ok])
    want, edges = O.sample_invcdf(z, u[ok])
    differ = np.nonzero(ids[ok] != want)[0]
    assert np.all(edges[differ] < EDGE), f"rows {ok[differ]} differ"
    assert np.all(close(lp[ok], O.token_logp(z, ids[ok])))
    assert np.all(close(ent[ok], O.entropy(z)))


def test_queued_sampler_many_rows_against_register_resident(monkeypatch):
    """1024 C4 rows: four workgroups per compute unit in turn, each starting on the LDS its
    predecessor left. Every id equals the register-resident sampler's off the CDF edges (the
    oracle decides the rows where they differ), and a rerun gives the same bits."""
    rows = 1024
    w = W.c4(seed=77, rows=rows)
    V = w["V"]
    u = nr.Rng(77, "c4/many-rows/uniforms").uniforms(rows)
    ut = nr.Tensor.from_numpy(u, "f64")
    ids, lp = nr.sample_logp(w["logits"], 0.7, w["mask"], None, uniforms=ut)
    ids2, lp2 = nr.sample_logp(w["logits"], 0.7, w["mask"], None, uniforms=ut)
    a, b = ids.to_numpy().ravel(), lp.to_numpy().ravel()
    assert np.array_equal(a, ids2.to_numpy().ravel()) and b.tobytes() == lp2.to_numpy().ravel().tobytes(), "rerun bits"
    monkeypatch.setenv("NOETIC_HIP_SAMPLE_QUEUE", "off")
    rr, lrr = nr.sample_logp(w["logits"], 0.7, w["mask"], None, uniforms=ut)
    monkeypatch.delenv("NOETIC_HIP_SAMPLE_QUEUE")
    rr, lrr = rr.to_numpy().ravel(), lrr.to_numpy().ravel()
    same = a == rr
    assert np.all(close(b[same], lrr[same])), "logp against the register-resident sampler"
    differ = np.nonzero(~same)[0]
    assert len(differ) <= 8, f"{len(differ)} rows differ from the register-resident sampler"
    if len(differ):
        x = W.bf16_to_f32(W.download_rows(w["logits"], differ, V))
        keep = W.download_rows(w["mask"], differ, V)
        z = O.tempered(x, 0.7, keep=keep)
        want, edges = O.sample_invcdf(z, u[differ])
        assert np.all(edges < EDGE), f"rows {differ[edges >= EDGE]} differ off a CDF edge"
        bad = np.nonzero(a[differ] != want)[0]
        assert np.all(edges[bad] < EDGE)


def test_queued_sampler_shared_mask(monkeypatch):
    """One grammar mask row for every logits row (mask_ld 0), C4's shape."""
    monkeypatch.setenv("NOETIC_HIP_SAMPLE_SEG", "off")
    w = W.c4(seed=9, rows=128, shared_mask=True)
    rows, V = w["rows"], w["V"]
    u = nr.Rng(9, "c4s/uniforms").uniforms(rows)
    ids, lp, ent = nr.sample_logp(w["logits"], 0.7, w["mask"], None, entropy=True, uniforms=nr.Tensor.from_numpy(u, "f64"))
    x = W.bf16_to_f32(w["logits"].to_numpy().reshape(rows, V))
    keep = np.broadcast_to(w["mask"].to_numpy().reshape(1, V), (rows, V))
    z = O.tempered(x, 0.7, keep=keep)
    want, edges = O.sample_invcdf(z, u)
    a = ids.to_numpy().ravel()
    differ = np.nonzero(a != want)[0]
    assert np.all(edges[differ] < EDGE), f"rows {differ} differ"
    assert np.all(close(lp.to_numpy().ravel(), O.token_logp(z, a)))
    assert np.all(close(ent.to_numpy().ravel(), O.entropy(z)))
