"""The readout-fused sampler (nt_hip_rl_readout_sample) against the oracle.

Pass 1's logits (written by the debug pointer) are checked against an f64 product of the same
bf16 operands, within the accumulation bound of f32 sums (the reference's half-precision product
is judged by a bound, src/tensor/gpu/half_gemm.rs:73-104); the draw is then checked exactly as the
fused sampler's: the oracle's f64 inverse-CDF on those logits, ids equal except within 1e-6 of a
CDF edge, log-probabilities within 1e-5 relative / 1e-6 absolute (f32). The crossing block that
pass 2 recomputes must equal pass 1's logits bit for bit, and reruns are byte-identical."""
import numpy as np
import pytest

import noetic_rl as nr
import workloads as W
from oracle import oracle as O

pytestmark = pytest.mark.gpu
EDGE = 1e-6


@pytest.fixture(scope="module", autouse=True)
def device():
    nr.claim(0)
    yield


def run_case(name, rows, V, d, tau, masked, seed, check_gemm_rows=None):
    h = W.normal((rows, d), "bf16", seed, f"readout/{name}/h", std=1.0)
    # the reference's Linear layout [d, V] (src/nn/linear.rs:1-3), packed once; also the
    # vocabulary-major layout, whose packing must give the same bytes
    w = W.normal((d, V), "bf16", seed, f"readout/{name}/w", std=2.0 / np.sqrt(d))
    packed = nr.PackedReadout(w, "dv")
    wt = nr.Tensor.from_numpy(np.ascontiguousarray(w.to_numpy().T), "bf16")
    packed_vd = nr.PackedReadout(wt, "vd")
    nr.sync()
    assert packed.buf_bytes() == packed_vd.buf_bytes(), f"{name}: the two layouts pack differently"
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
    hb = W.bf16_to_f32(h.to_numpy()).astype(np.float64)
    sample = np.arange(rows) if check_gemm_rows is None else check_gemm_rows
    wb = W.bf16_to_f32(w.to_numpy()).astype(np.float64)  # [d, V]
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


def test_readout_refuses_a_row_with_no_allowed_token():
    rows, V, d = 8, 512, 64
    h = W.normal((rows, d), "bf16", 1, "readout/refuse/h")
    w = nr.PackedReadout(W.normal((d, V), "bf16", 1, "readout/refuse/w"), "dv")
    keep = np.ones((rows, V), np.uint8)
    keep[5] = 0
    with pytest.raises(ValueError, match="position 5 has no allowed token"):
        nr.readout_sample_logp(h, w, 0.8, nr.Tensor.from_numpy(keep, "u8"), nr.Rng(1, "x"))
