"""The register-resident and the segmented samplers at every shape they are built for, against
the oracle.

The kernel cuts a row into 512-element chunks and gives wave w (of 16) the K consecutive chunks
[w K, w K + K), K the smallest power of two with 16 K chunks covering the row (bf16 up to 16,
f32 up to 8, f32 additive mask up to 4). The crossing of u S is found in three levels: the wave
(an f64 scan over the 16 wave totals), the chunk (the wave's own prefix), the lane and element.
These cases put the crossing and the row's weight where those levels meet:
- V just past a K boundary (waves 9..15 hold no chunk at all, wave 8 one partial chunk) and V
  just below the next one (every wave full, the last chunk ragged);
- rows whose allowed tokens all lie in one wave's range, or in the row's last element only, or
  in its first element only (every other wave has no weight, so its reference is -inf);
- a row whose maximum sits in the last wave with every other wave far below it (their weights
  relative to the row's maximum underflow);
- temperature 1, 0.7 and 0 (greedy, the first maximum in index order).
ids must equal the oracle's except for draws within 1e-6 of a CDF edge; logp and entropy hold
the dtype's tolerance (1e-5 relative / 1e-6 absolute for f32, 2e-3 relative for bf16).
"""
import numpy as np
import pytest

import noetic_rl as nr
from oracle import oracle as O

pytestmark = pytest.mark.gpu

EDGE = 1e-6
CHUNK = 512
WAVES = 16


@pytest.fixture(scope="module", autouse=True)
def device():
    nr.claim(0)
    yield


def close(ours, want, bf16):
    ours, want = np.asarray(ours, np.float64), np.asarray(want, np.float64)
    tol = (1e-6 + 2e-3 * np.abs(want)) if bf16 else (1e-6 + 1e-5 * np.abs(want))
    return np.abs(ours - want) <= tol


def rows_for(V, rng, K):
    """16 rows of V logits in [-6, 6] (N(0, 2)) and their u8 keep-masks, with the special rows."""
    rows = 16
    x = rng.normal(0, 2, (rows, V)).astype(np.float32)
    keep = (rng.random((rows, V)) < 0.7).astype(np.uint8)
    keep[:, 0] = 1
    span = K * CHUNK  # elements per wave
    # row 1: only wave 3's range allowed (or the last wave holding elements)
    w = min(3, (V - 1) // span)
    keep[1] = 0
    keep[1, w * span:min(V, (w + 1) * span)] = 1
    # row 2: only the last element; row 3: only the first
    keep[2] = 0
    keep[2, V - 1] = 1
    keep[3] = 0
    keep[3, 0] = 1
    # row 4: the maximum in the row's last element, every other logit 200 below it
    x[4] -= 200.0
    x[4, V - 1] = 5.0
    keep[4, V - 1] = 1
    # row 5: a peaked row, the mass in one element of the middle wave's range
    mid = min(V - 1, (V // span // 2) * span + 7)
    x[5, mid] = 40.0
    keep[5, mid] = 1
    return x, keep


def cases():
    out = []
    for dtype, kmax in (("bf16", 16), ("f32", 8)):
        K = 1
        while K <= kmax:
            # (V a multiple of 8: rows the register-resident kernel takes)
            lo = WAVES * (K // 2) * CHUNK + 8 if K > 1 else 2 * CHUNK + 8
            hi = WAVES * K * CHUNK - 40
            out += [(dtype, "u8", K, lo), (dtype, "u8", K, hi)]
            K *= 2
    # the f32 additive mask (K at most 4 there) and no mask
    out += [("f32", "f32add", 4, WAVES * 4 * CHUNK - 8), ("bf16", "f32add", 2, WAVES * 2 * CHUNK),
            ("bf16", "none", 16, WAVES * 16 * CHUNK - 8), ("f32", "none", 1, 704)]
    return out


@pytest.mark.parametrize("dtype,mask,K,V", cases())
def test_register_resident_sampler_levels(dtype, mask, K, V, monkeypatch):
    """u8 rows of K >= 4 take the queued sampler by default (these masks keep 70% of the tokens,
    so its waves take its dense path); the test below runs them through the register-resident
    sampler itself."""
    monkeypatch.setenv("NOETIC_HIP_SAMPLE_SEG", "off")  # one workgroup per row, whatever the row count
    check_levels(dtype, mask, K, V)


@pytest.mark.parametrize("dtype,mask,K,V", [c for c in cases() if c[1] == "u8" and c[2] >= 4])
def test_register_resident_sampler_levels_without_queue(dtype, mask, K, V, monkeypatch):
    monkeypatch.setenv("NOETIC_HIP_SAMPLE_SEG", "off")
    monkeypatch.setenv("NOETIC_HIP_SAMPLE_QUEUE", "off")
    check_levels(dtype, mask, K, V)


def seg_cases():
    """(dtype, mask, NW, K, window, V) for the segmented sampler: every shape it is built for, V
    one element past a segment boundary (the last segment holds one partial chunk) and just below
    a whole number of segments, the f32 additive and no mask, both load windows."""
    out = []
    for dtype in ("bf16", "f32"):
        for nw, k in ((4, 4), (8, 4), (4, 8), (8, 8), (4, 16), (8, 16)):
            if dtype == "f32" and k > 8:
                continue
            seg = nw * k * CHUNK
            out += [(dtype, "u8", nw, k, "one", 2 * seg + 8), (dtype, "u8", nw, k, "one", 3 * seg - 40)]
            if k == 4:
                out += [(dtype, "u8", nw, k, "all", 5 * seg - 8)]
    out += [("f32", "f32add", 4, 4, "one", 4 * 4 * 4 * CHUNK - 8), ("bf16", "f32add", 8, 8, "one", 2 * 8 * 8 * CHUNK),
            ("bf16", "none", 8, 4, "all", 128256), ("f32", "none", 8, 8, "one", 50304)]
    return out


@pytest.mark.parametrize("dtype,mask,nw,K,window,V", seg_cases())
def test_segmented_sampler_levels(dtype, mask, nw, K, window, V, monkeypatch):
    """The same rows through the segmented sampler: the row cut into segments of nw waves of K
    chunks (one workgroup each); the last segment to arrive merges the wave records (phase 2 over
    up to 64 records), finds the crossing wave and chunk and reads that chunk again."""
    monkeypatch.setenv("NOETIC_HIP_SAMPLE_SEG", f"{nw},{K}")
    monkeypatch.setenv("NOETIC_HIP_SAMPLE_WINDOW", window)
    check_levels(dtype, mask, K, V)


def check_levels(dtype, mask, K, V):
    rng = np.random.default_rng(V * 7 + K)
    x, keep = rows_for(V, rng, K)
    rows = x.shape[0]
    bf16 = dtype == "bf16"
    if bf16:
        xb = O.bf16_from_f32(x)
        x = O.bf16_to_f32(xb)
        xt = nr.Tensor.from_numpy(xb, "bf16")
    else:
        xt = nr.Tensor.from_numpy(x)
    if mask == "u8":
        mt, kw = nr.Tensor.from_numpy(keep), dict(keep=keep)
    elif mask == "f32add":
        add = np.where(keep == 1, 0.0, -np.inf).astype(np.float32)
        add[:, 1::3] = np.where(keep[:, 1::3] == 1, -1.5, -np.inf)  # finite offsets too
        mt, kw = nr.Tensor.from_numpy(add), dict(addmask=add)
    else:
        mt, kw = None, {}
    u = np.random.default_rng(V + K).random(rows)
    u[0], u[6] = 0.0, np.nextafter(1.0, 0.0)  # the first and the last weight
    ut = nr.Tensor.from_numpy(u, "f64")
    for tau in (1.0, 0.7, 0.0):
        ids, lp, ent = nr.sample_logp(xt, tau, mt, None, entropy=True, uniforms=None if tau == 0.0 else ut)
        ids, lp, ent = ids.to_numpy(), lp.to_numpy(), ent.to_numpy()
        z = O.tempered(x, 1.0 if tau == 0.0 else tau, **kw)
        if tau == 0.0:
            zz = np.where(np.isfinite(z), z, -np.inf)
            assert np.array_equal(ids, np.argmax(zz, axis=1)), f"{dtype} {mask} K={K} V={V}: greedy ids"
        else:
            want, edges = O.sample_invcdf(z, u)
            differ = np.nonzero(ids != want)[0]
            assert np.all(edges[differ] < EDGE), f"{dtype} {mask} K={K} V={V} tau={tau}: rows {differ} differ"
        allowed = np.isfinite(z[np.arange(rows), ids])
        assert allowed.all(), f"{dtype} {mask} K={K} V={V} tau={tau}: an excluded token was drawn"
        assert np.all(close(lp, O.token_logp(z, ids), bf16)), f"{dtype} {mask} K={K} V={V} tau={tau}: logp"
        assert np.all(close(ent, O.entropy(z), bf16)), f"{dtype} {mask} K={K} V={V} tau={tau}: entropy"
        assert ids[4] == V - 1
        if mask != "none":
            assert ids[2] == V - 1 and ids[3] == 0


@pytest.mark.parametrize("seg", ["off", "8,4", "4,8"])
@pytest.mark.parametrize("dtype,mask,V", [("bf16", "u8", WAVES * 16 * CHUNK - 8), ("f32", "u8", WAVES * 4 * CHUNK - 8),
                                          ("f32", "f32add", WAVES * 2 * CHUNK), ("bf16", "none", 4096)])
def test_register_resident_sampler_refusals(dtype, mask, V, seg, monkeypatch):
    """Each row is refused on its own: a NaN in the first wave's range, in a middle wave's, in the
    row's last element, or a +inf logit (its weight is inf - inf) gives NT_ROW_NAN; a row with
    every token excluded gives NT_ROW_NO_TOKEN; the rows between them sample as the oracle does.
    A NaN at a token the u8 mask excludes does not reach the row; under an f32 mask's -inf it
    does (NaN + -inf), as in the reference's tempered_logits."""
    import ctypes as C
    monkeypatch.setenv("NOETIC_HIP_SAMPLE_SEG", seg)
    rows = 10
    rng = np.random.default_rng(V)
    x = rng.normal(0, 2, (rows, V)).astype(np.float32)
    keep = (rng.random((rows, V)) < 0.6).astype(np.uint8)
    keep[:, 0] = 1
    span = V // WAVES
    for r, pos in ((0, 5), (1, 9 * span + 3), (2, V - 1)):
        x[r, pos] = np.nan
        keep[r, pos] = 1
    x[4, 7] = np.inf
    keep[4, 7] = 1
    keep[5] = 0
    x[6, 11] = np.nan  # excluded below
    keep[6, 11] = 0
    if mask == "none":
        keep[:] = 1
        keep[6, 11] = 1  # no mask: the NaN stays in the row
        keep[5] = 1
    nan_rows = {0, 1, 2, 4} | ({6} if mask != "u8" else set())
    none_rows = {5} if mask != "none" else set()
    bf16 = dtype == "bf16"
    if bf16:
        xs = O.bf16_from_f32(x)
        x = O.bf16_to_f32(xs)
        xt = nr.Tensor.from_numpy(xs, "bf16")
    else:
        xt = nr.Tensor.from_numpy(x)
    if mask == "u8":
        mt, kind, kw = nr.Tensor.from_numpy(keep), nr.NT_MASK_U8, dict(keep=keep)
    elif mask == "f32add":
        add = np.where(keep == 1, 0.0, -np.inf).astype(np.float32)
        mt, kind, kw = nr.Tensor.from_numpy(add), nr.NT_MASK_F32, dict(addmask=add)
    else:
        mt, kind, kw = None, nr.NT_MASK_NONE, {}
    u = np.random.default_rng(1).random(rows)
    ut = nr.Tensor.from_numpy(u, "f64")
    ids, lp, ent, st = nr.IntTensor((rows,)), nr.Tensor((rows,), "f32"), nr.Tensor((rows,), "f32"), nr.Tensor((rows,), "u8")
    a = nr.NtRlSampleArgs(xt.ptr, nr.NT_BF16 if bf16 else nr.NT_F32, kind, rows, V, V, None if mt is None else mt.ptr,
                          0 if mt is None else V, 0.9, ut.ptr, ids.ptr, lp.ptr, ent.ptr, st.ptr)
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
    z = O.tempered(x[ok], 0.9, **({k: v[ok] for k, v in kw.items()}))
    want, edges = O.sample_invcdf(z, u[ok])
    differ = np.nonzero(ids[ok] != want)[0]
    assert np.all(edges[differ] < EDGE), f"rows {ok[differ]} differ"
    assert np.all(close(lp[ok], O.token_logp(z, ids[ok]), bf16))
    assert np.all(close(ent[ok], O.entropy(z), bf16))
