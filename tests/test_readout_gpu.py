"""The readout-fused sampler (nt_hip_rl_readout_sample) against the oracle.

Pass 1's logits (written by the debug pointer) are checked against an f64 product of the same
bf16 operands, within the accumulation bound of f32 sums (the reference's half-precision product
is judged by a bound, src/tensor/gpu/half_gemm.rs:73-104); the draw is then checked exactly as the
fused sampler's: the oracle's f64 inverse-CDF on those logits, ids equal except within 1e-6 of a
CDF edge, log-probabilities within 1e-5 relative / 1e-6 absolute (f32). The crossing block that
pass 2 recomputes must equal pass 1's logits bit for bit, and reruns are byte-identical."""
import numpy as np
import pytest

import noetic_ops as ops
import noetic_rl as nr
import workloads as W
from oracle import oracle as O

pytestmark = pytest.mark.gpu
EDGE = 1e-6


@pytest.fixture(scope="module", autouse=True)
def device():
    nr.claim(0)
    # the readout fusion is the reduced-precision product: it runs at MatmulPrecision::Half
    prev = nr.set_matmul_precision(nr.MatmulPrecision.HALF)
    yield
    nr.set_matmul_precision(prev)


def rounded(t):
    """A device tensor's values as the product reads them: bf16 as they are, f32 and f16 (widened
    exactly) rounded to nearest-even bf16 (precision.rs:4-8; the oracle's half.rs restatement), as
    f64."""
    a = t.to_numpy()
    if t.dtype == "bf16":
        return W.bf16_to_f32(a).astype(np.float64)
    if t.dtype == "f16":
        a = a.view(np.float16).astype(np.float32)
    return O.bf16_to_f32(O.bf16_from_f32(a)).astype(np.float64)


def normal(shape, dtype, seed, label, std):
    """W.normal's values; f16 ones drawn in f32 and rounded to f16 on the host."""
    if dtype != "f16":
        return W.normal(shape, dtype, seed, label, std=std)
    f = W.normal(shape, "f32", seed, label, std=std).to_numpy()
    return nr.Tensor.from_numpy(f.astype(np.float16).view(np.uint16), "f16")


def run_case(name, rows, V, d, tau, masked, seed, check_gemm_rows=None, dtype="bf16"):
    h = normal((rows, d), dtype, seed, f"readout/{name}/h", std=1.0)
    # the reference's Linear layout [d, V] (src/nn/linear.rs:1-3), packed once; also the
    # vocabulary-major layout, whose packing must give the same bytes
    w = normal((d, V), dtype, seed, f"readout/{name}/w", std=2.0 / np.sqrt(d))
    packed = nr.PackedReadout(w, "dv")
    wt = nr.Tensor.from_numpy(np.ascontiguousarray(w.to_numpy().T), dtype)
    packed_vd = nr.PackedReadout(wt, "vd")
    del wt
    nr.sync()
    assert packed.buf_bytes() == packed_vd.buf_bytes(), f"{name}: the two layouts pack differently"
    del packed_vd
    keep = None
    mt = None
    if masked:
        rng = np.random.default_rng(seed)
        keep = (rng.random((rows, V)) < 0.3).astype(np.uint8)
        keep[np.arange(rows), rng.integers(0, V, rows)] = 1
        mt = nr.Tensor.from_numpy(keep, "u8")
    u = nr.Rng(seed, f"readout/{name}/u").uniforms(rows)
    ut = nr.Tensor.from_numpy(u, "f64")
    ids, lp, logits, blk, bidx = nr.readout_sample_logp(h, packed, tau, mt, None, uniforms=ut if tau else None,
                                                        debug=True)
    ids, lp, logits = ids.to_numpy().ravel(), lp.to_numpy().ravel(), logits.to_numpy()
    blk, bidx = blk.to_numpy(), bidx.to_numpy().ravel()
    # the product against f64 on a row sample, within f32 accumulation's bound
    hb = rounded(h)
    sample = np.arange(rows) if check_gemm_rows is None else check_gemm_rows
    wb = rounded(w)  # [d, V]
    exact = hb[sample] @ wb
    scale = np.abs(hb[sample]) @ np.abs(wb)
    gerr = np.abs(logits[sample].astype(np.float64) - exact)
    bound = 2.0 ** -21 * d * scale
    assert np.all(gerr <= bound), f"{name}: product off by {np.max(gerr / np.maximum(scale, 1e-30)):.2e} of sum|a||b|"
    # the draw on those logits
    z = O.tempered(logits, 1.0 if tau == 0 else tau, keep=keep)
    if tau == 0:
        zz = np.where(np.isfinite(z), z, -np.inf)
        assert np.array_equal(ids, np.argmax(zz, axis=1)), f"{name}: greedy ids"
    else:
        want, edges = O.sample_invcdf(z, u)
        differ = np.nonzero(ids != want)[0]
        far = differ[edges[differ] >= EDGE]
        if len(far):
            # say which stage disagrees: the row's product, pass 2's recomputed block, or the draw
            notes = []
            for r in far[:4]:
                ex = hb[r] @ wb
                sc = np.abs(hb[r]) @ np.abs(wb)
                rel = float(np.max(np.abs(logits[r].astype(np.float64) - ex) / np.maximum(sc, 1e-30)))
                b = int(bidx[r])
                cols = np.arange(32 * b, min(32 * b + 32, V))
                same = blk[r, :len(cols)].tobytes() == logits[r, cols].tobytes()
                notes.append(f"row {r}: id {ids[r]} oracle {want[r]} edge {edges[r]:.2e}, product err {rel:.1e}, "
                             f"block {b} recomputed {'==' if same else '!='} pass 1")
            raise AssertionError(f"{name}: rows {far[:8]} differ away from a CDF edge; " + "; ".join(notes))
        # the recomputed crossing block is pass 1's, bit for bit
        for r in range(rows):
            b = int(bidx[r])
            cols = np.arange(32 * b, min(32 * b + 32, V))
            if blk[r, :len(cols)].tobytes() != logits[r, cols].tobytes():
                ex = hb[r] @ wb[:, cols]
                sc = np.abs(hb[r]) @ np.abs(wb[:, cols])
                e1 = float(np.max(np.abs(logits[r, cols].astype(np.float64) - ex) / sc))
                e2 = float(np.max(np.abs(blk[r, :len(cols)].astype(np.float64) - ex) / sc))
                nd = int(np.sum(blk[r, :len(cols)] != logits[r, cols]))
                raise AssertionError(f"{name}: row {r} block {b}: {nd} of {len(cols)} recomputed logits differ from "
                                     f"pass 1; error against f64, pass 1 {e1:.1e}, recomputed {e2:.1e}")
            assert 32 * b <= ids[r] < 32 * b + 32
        print(f"{name}: {rows} rows, {len(differ)} ids differ ({int(np.sum(edges < EDGE))} boundary draws), "
              f"product max err {np.max(gerr / np.maximum(scale, 1e-30)):.1e} of sum|a||b|", end="")
    want_lp = O.token_logp(z, ids)
    err = np.abs(lp.astype(np.float64) - want_lp)
    assert np.all(err <= 1e-6 + 1e-5 * np.abs(want_lp)), f"{name}: logp off by {err.max():.2e}"
    print(f", logp max |d| {err.max():.1e}")
    if keep is not None:
        assert keep[np.arange(rows), ids].all(), f"{name}: an excluded token was drawn"
    again = nr.readout_sample_logp(h, packed, tau, mt, None, uniforms=ut if tau else None)
    assert again[0].to_numpy().tobytes() == ids.astype(np.int32).tobytes(), f"{name}: rerun ids"
    assert again[1].to_numpy().tobytes() == lp.tobytes(), f"{name}: rerun logp"
    if dtype in ("f32", "f16"):
        # f32 and f16 operands are the device cast's bf16 operands: the same packed bytes, logits,
        # ids and log-probabilities, bit for bit
        lay = lambda t: ops.Layout.contiguous(t.shape)
        hc, wc = ops.cast(h, lay(h), "bf16"), ops.cast(w, lay(w), "bf16")
        pc = nr.PackedReadout(wc, "dv")
        del wc
        assert pc.buf_bytes() == packed.buf_bytes(), f"{name}: {dtype} packing differs from the bf16 cast's"
        ic, lc, zc = nr.readout_sample_logp(hc, pc, tau, mt, None, uniforms=ut if tau else None, debug=True)[:3]
        assert ic.to_numpy().tobytes() == ids.astype(np.int32).tobytes(), f"{name}: ids against the bf16 cast"
        assert lc.to_numpy().tobytes() == lp.tobytes(), f"{name}: logp against the bf16 cast"
        assert zc.to_numpy().tobytes() == logits.tobytes(), f"{name}: logits against the bf16 cast"


@pytest.mark.parametrize("rows,V,d", [(40, 1000, 256), (256, 4104, 512), (1, 300, 64), (97, 257, 16), (64, 600, 528)])
@pytest.mark.parametrize("tau,masked", [(0.7, True), (1.0, False), (0.0, True)])
def test_readout_sampler_small_shapes(rows, V, d, tau, masked):
    run_case(f"r{rows}v{V}d{d}t{tau}m{int(masked)}", rows, V, d, tau, masked, seed=rows + V + d)


@pytest.mark.parametrize("tau,masked", [(0.7, True), (0.0, True)])
def test_readout_sampler_above_131072_columns(tau, masked):
    # V 151936 (benchmark configuration 5's vocabulary): the resolve's larger per-thread arrays
    run_case(f"r24v151936d64t{tau}", 24, 151936, 64, tau, masked, seed=151936)


def test_readout_sampler_at_the_decode_shape():
    # C4's decode step: 256 rows, d 4096, V 128256, a 30% keep-mask, T 0.7
    run_case("c4 readout", 256, 128256, 4096, 0.7, True, seed=2024, check_gemm_rows=np.arange(0, 256, 16))


@pytest.mark.parametrize("rows,V,d", [(40, 1000, 256), (97, 257, 16)])
@pytest.mark.parametrize("tau,masked", [(0.7, True), (0.0, False)])
def test_readout_sampler_f32_operands_small_shapes(rows, V, d, tau, masked):
    run_case(f"f32 r{rows}v{V}d{d}t{tau}m{int(masked)}", rows, V, d, tau, masked, seed=rows + V + d + 1,
             dtype="f32")


def test_readout_sampler_f32_operands_at_the_decode_shape():
    # C4's decode step with the head's f32 weight [4096, 128256] and f32 hidden states, as the
    # reference's decoder holds them, rounded to bf16 as MatmulPrecision::Half rounds its operands
    run_case("c4 readout f32", 256, 128256, 4096, 0.7, True, seed=2025, check_gemm_rows=np.arange(3, 256, 16),
             dtype="f32")


@pytest.mark.parametrize("rows,V,d", [(40, 1000, 256), (97, 257, 16)])
@pytest.mark.parametrize("tau,masked", [(0.7, True), (0.0, False)])
def test_readout_sampler_f16_operands_small_shapes(rows, V, d, tau, masked):
    run_case(f"f16 r{rows}v{V}d{d}t{tau}m{int(masked)}", rows, V, d, tau, masked, seed=rows + V + d + 2,
             dtype="f16")


def test_readout_sampler_f16_operands_at_a_wide_head():
    # 256 rows against an f16 head of V 50304 (benchmark configuration 3's vocabulary), d 1024
    run_case("f16 r256v50304d1024", 256, 50304, 1024, 0.8, True, seed=2026, check_gemm_rows=np.arange(5, 256, 25),
             dtype="f16")


def test_f16_weights_pack_rounded_to_nearest_even():
    """f16 widens to f32 exactly, so packing rounds once to nearest-even bf16: ties between bf16
    neighbours (the low three of f16's ten fraction bits 100), their neighbours, subnormals, the
    largest finite value, signed zeros, infinities and NaNs give numpy's widened values rounded by
    the oracle's half.rs restatement, and the device cast f16 -> bf16's bytes."""
    d, V = 32, 300
    rng = np.random.default_rng(18)
    h = rng.normal(0, 1, (d, V)).astype(np.float16).view(np.uint16)
    special = np.array([0x3C04, 0x3C0C, 0x3C05, 0x3C03, 0xBC04, 0xBC0C, 0x0001, 0x0004, 0x000C, 0x03FF, 0x8003,
                        0x0400, 0x7BFF, 0x7BFC, 0xFBFF, 0x7C00, 0xFC00, 0x0000, 0x8000, 0x7E01, 0xFC01, 0x7D23],
                       np.uint16)
    pos = rng.choice(d * V, size=(8, special.size), replace=False)
    for k in range(8):
        h.ravel()[pos[k]] = special
    wide = h.view(np.float16).astype(np.float32)
    nan = np.isnan(wide)
    want = O.bf16_from_f32(wide)
    w = nr.Tensor.from_numpy(h, "f16")
    wc = ops.cast(w, ops.Layout.contiguous(w.shape), "bf16")
    cast = wc.to_numpy()
    assert np.array_equal(cast[~nan], want[~nan]), "the device cast f16 -> bf16 is not the widened value's RNE"
    assert np.all(np.isnan(W.bf16_to_f32(cast[nan])))
    ref = nr.Tensor.from_numpy(np.where(nan, np.uint16(0x7FC0), want).astype(np.uint16), "bf16")
    a = np.frombuffer(nr.PackedReadout(w, "dv").buf_bytes(), np.uint16)
    b = np.frombuffer(nr.PackedReadout(ref, "dv").buf_bytes(), np.uint16)
    c = np.frombuffer(nr.PackedReadout(wc, "dv").buf_bytes(), np.uint16)
    for other in (b, c):
        differ = np.nonzero(a != other)[0]
        # only NaNs may differ (in payload), and those stay NaNs
        assert np.all(np.isnan(W.bf16_to_f32(a[differ]))) and np.all(np.isnan(W.bf16_to_f32(other[differ])))
        assert len(differ) <= int(nan.sum())
    assert np.sum(np.isnan(W.bf16_to_f32(a))) == int(nan.sum())
    # the vocabulary-major layout packs to the same bytes
    wt = nr.Tensor.from_numpy(np.ascontiguousarray(h.T), "f16")
    assert nr.PackedReadout(wt, "vd").buf_bytes() == a.tobytes()


def test_f32_weights_pack_rounded_to_nearest_even():
    """Ties, their neighbours, subnormals, the overflow to infinity, signed zeros, infinities and
    NaNs: packing f32 gives the bytes of packing the device cast's bf16 (half.rs:16-23, itself
    checked against the oracle's restatement here), a NaN staying a NaN."""
    d, V = 32, 300
    rng = np.random.default_rng(8)
    bits = rng.normal(0, 1, (d, V)).astype(np.float32).view(np.uint32)
    special = np.array([0x3F808000, 0x3F818000, 0x3F808001, 0x3F807FFF, 0xBF808000, 0xBF818000,
                        0x00008000, 0x00018000, 0x0000FFFF, 0x80007FFF, 0x00000001, 0x807F8000,
                        0x7F7FFFFF, 0x7F7F7FFF, 0x7F7F8000, 0xFF7FFFFF, 0x7F800000, 0xFF800000,
                        0x00000000, 0x80000000, 0x7FC00001, 0xFF800001, 0x7F812345], np.uint32)
    pos = rng.choice(d * V, size=(8, special.size), replace=False)
    for k in range(8):
        bits.ravel()[pos[k]] = special
    wf = bits.view(np.float32)
    w = nr.Tensor.from_numpy(wf)
    wc = ops.cast(w, ops.Layout.contiguous(w.shape), "bf16")
    cast = wc.to_numpy()
    nan = np.isnan(wf)
    want = O.bf16_from_f32(wf)
    assert np.array_equal(cast[~nan], want[~nan]), "the device cast is not half.rs's rounding"
    assert np.all(np.isnan(W.bf16_to_f32(cast[nan])))
    a = np.frombuffer(nr.PackedReadout(w, "dv").buf_bytes(), np.uint16)
    b = np.frombuffer(nr.PackedReadout(wc, "dv").buf_bytes(), np.uint16)
    differ = np.nonzero(a != b)[0]
    # only NaNs may differ (in payload), and those stay NaNs
    assert np.all(np.isnan(W.bf16_to_f32(a[differ]))) and np.all(np.isnan(W.bf16_to_f32(b[differ])))
    assert np.sum(np.isnan(W.bf16_to_f32(a))) == int(nan.sum())
    assert len(differ) <= int(nan.sum())


def test_seed_batched_head():
    # the decoder's seed-batched head: hidden [S, N, d] . W [S, d, V] (linear.rs:1-12), N above
    # one call's 256 rows; each seed's rows equal the unbatched call on that seed's weight
    S, N, d, V, tau = 2, 300, 64, 1000, 0.8
    h = W.normal((S, N, d), "f32", 9, "readout/seeds/h")
    w = W.normal((S, d, V), "f32", 9, "readout/seeds/w", std=2.0 / np.sqrt(d))
    rng = np.random.default_rng(9)
    keep = (rng.random((S, N, V)) < 0.4).astype(np.uint8)
    keep[..., 7] = 1
    u = nr.Rng(9, "readout/seeds/u").uniforms(S * N)
    packed = nr.PackedReadout(w, "dv")
    ids, lp, logits = nr.readout_sample_logp(h, packed, tau, nr.Tensor.from_numpy(keep), None,
                                             uniforms=nr.Tensor.from_numpy(u, "f64"), debug=True)[:3]
    assert ids.shape == (S, N) and lp.shape == (S, N) and logits.shape == (S, N, V)
    ids, lp, logits = ids.to_numpy(), lp.to_numpy(), logits.to_numpy()
    hn, wn = h.to_numpy(), w.to_numpy()
    for k in range(S):
        hk, wk = nr.Tensor.from_numpy(hn[k]), nr.Tensor.from_numpy(wn[k])
        i1, l1, z1 = nr.readout_sample_logp(hk, nr.PackedReadout(wk, "dv"), tau, nr.Tensor.from_numpy(keep[k]), None,
                                            uniforms=nr.Tensor.from_numpy(u[k * N:(k + 1) * N], "f64"),
                                            debug=True)[:3]
        assert i1.to_numpy().tobytes() == ids[k].tobytes(), f"seed {k}: ids"
        assert l1.to_numpy().tobytes() == lp[k].tobytes(), f"seed {k}: logp"
        assert z1.to_numpy().tobytes() == logits[k].tobytes(), f"seed {k}: logits"
        hb, wb = rounded(hk), rounded(wk)
        exact, scale = hb @ wb, np.abs(hb) @ np.abs(wb)
        assert np.all(np.abs(logits[k].astype(np.float64) - exact) <= 2.0 ** -21 * d * scale), f"seed {k}: product"
        z = O.tempered(logits[k], tau, keep=keep[k])
        want, edges = O.sample_invcdf(z, u[k * N:(k + 1) * N])
        assert np.all((ids[k] == want) | (edges < EDGE)), f"seed {k}: draws"
        wl = O.token_logp(z, ids[k])
        assert np.all(np.abs(lp[k] - wl) <= 1e-6 + 1e-5 * np.abs(wl)), f"seed {k}: logp"
    # the scorer over the same batched head gives the sampler's log-probabilities
    slp, _ = nr.readout_score(h, packed, tau, nr.Tensor.from_numpy(keep), nr.Tensor.from_numpy(ids), entropy=False)
    assert slp.shape == (S, N) and slp.to_numpy().tobytes() == lp.tobytes()
    with pytest.raises(ValueError, match="2 seeds"):
        nr.readout_sample_logp(nr.Tensor.from_numpy(hn[0]), packed, tau, None, None,
                               uniforms=nr.Tensor.from_numpy(u[:N], "f64"))


def test_readout_masks_per_seed_and_broadcast():
    """A seed-batched head's mask with one row per seed ([S, 1, V], read in place: each seed's calls
    share its row) and a mask broadcast over a leading dimension ([B, 1, V] against hidden
    [B, T, d], broadcast on the device first) give the bits of the same mask materialised per
    row."""
    S, N, d, V, tau = 2, 300, 64, 1000, 0.8
    h = W.normal((S, N, d), "bf16", 21, "readout/seedmask/h")
    w = nr.PackedReadout(W.normal((S, d, V), "bf16", 21, "readout/seedmask/w", std=2.0 / np.sqrt(d)), "dv")
    rng = np.random.default_rng(21)
    m = (rng.random((S, 1, V)) < 0.4).astype(np.uint8)
    m[..., 9] = 1
    full = np.ascontiguousarray(np.broadcast_to(m, (S, N, V)))
    u = nr.Tensor.from_numpy(nr.Rng(21, "readout/seedmask/u").uniforms(S * N), "f64")
    a = nr.readout_sample_logp(h, w, tau, nr.Tensor.from_numpy(m), None, uniforms=u)
    b = nr.readout_sample_logp(h, w, tau, nr.Tensor.from_numpy(full), None, uniforms=u)
    assert all(x.to_numpy().tobytes() == y.to_numpy().tobytes() for x, y in zip(a, b)), "per-seed mask"
    sa = nr.readout_score(h, w, tau, nr.Tensor.from_numpy(m), a[0])
    sb = nr.readout_score(h, w, tau, nr.Tensor.from_numpy(full), a[0])
    assert all(x.to_numpy().tobytes() == y.to_numpy().tobytes() for x, y in zip(sa, sb)), "per-seed mask, scorer"
    assert sa[0].to_numpy().tobytes() == a[1].to_numpy().tobytes(), "scoring the draws gives their logp"
    # unbatched head, hidden [B, T, d], mask [B, 1, V]
    B, T = 6, 50
    h2 = W.normal((B, T, d), "bf16", 22, "readout/bcast/h")
    w2 = nr.PackedReadout(W.normal((d, V), "bf16", 22, "readout/bcast/w", std=2.0 / np.sqrt(d)), "dv")
    m2 = (rng.random((B, 1, V)) < 0.4).astype(np.uint8)
    m2[..., 4] = 1
    full2 = np.ascontiguousarray(np.broadcast_to(m2, (B, T, V)))
    u2 = nr.Tensor.from_numpy(nr.Rng(22, "readout/bcast/u").uniforms(B * T), "f64")
    a2 = nr.readout_sample_logp(h2, w2, tau, nr.Tensor.from_numpy(m2), None, uniforms=u2)
    b2 = nr.readout_sample_logp(h2, w2, tau, nr.Tensor.from_numpy(full2), None, uniforms=u2)
    assert all(x.to_numpy().tobytes() == y.to_numpy().tobytes() for x, y in zip(a2, b2)), "broadcast mask"
    with pytest.raises(ValueError, match="keep-mask"):
        nr.readout_sample_logp(h2, w2, tau, nr.Tensor.from_numpy(m2[:, :, :V - 1].copy()), None, uniforms=u2)


@pytest.mark.parametrize("rows,V,d", [(40, 1000, 256), (256, 4104, 64)])
def test_readout_shared_mask_row(rows, V, d):
    # one grammar mask [1, V] shared by every row (mask_ld 0) gives the materialised mask's results
    h = W.normal((rows, d), "bf16", 3, "readout/shared/h")
    w = nr.PackedReadout(W.normal((d, V), "bf16", 3, "readout/shared/w", std=2.0 / np.sqrt(d)), "dv")
    rng = np.random.default_rng(3)
    keep = (rng.random((1, V)) < 0.3).astype(np.uint8)
    keep[0, 11] = 1
    full = nr.Tensor.from_numpy(np.ascontiguousarray(np.broadcast_to(keep, (rows, V))))
    shared = nr.Tensor.from_numpy(keep)
    ut = nr.Tensor.from_numpy(nr.Rng(3, "readout/shared/u").uniforms(rows), "f64")
    a = nr.readout_sample_logp(h, w, 0.7, shared, None, uniforms=ut, debug=True)
    b = nr.readout_sample_logp(h, w, 0.7, full, None, uniforms=ut, debug=True)
    for x, y in zip(a, b):
        assert x.to_numpy().tobytes() == y.to_numpy().tobytes()
    assert keep[0, a[0].to_numpy()].all()
    sa = nr.readout_score(h, w, 0.7, shared, a[0], entropy=True)
    sb = nr.readout_score(h, w, 0.7, full, a[0], entropy=True)
    for x, y in zip(sa, sb):
        assert x.to_numpy().tobytes() == y.to_numpy().tobytes()


def test_readout_refuses_a_row_with_no_allowed_token():
    rows, V, d = 8, 512, 64
    h = W.normal((rows, d), "bf16", 1, "readout/refuse/h")
    w = nr.PackedReadout(W.normal((d, V), "bf16", 1, "readout/refuse/w"), "dv")
    keep = np.ones((rows, V), np.uint8)
    keep[5] = 0
    with pytest.raises(ValueError, match="position 5 has no allowed token"):
        nr.readout_sample_logp(h, w, 0.8, nr.Tensor.from_numpy(keep, "u8"), nr.Rng(1, "x"))
