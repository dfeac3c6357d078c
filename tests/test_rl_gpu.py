"""GPU parity tests: the fused HIP kernels (through the C ABI) against the CPU oracle on the same
bytes, at the benchmark configurations' real shapes where the oracle finishes in seconds.

Tolerances: sampled ids exact except draws whose uniform lies within
1e-6 of a CDF edge (counted and printed); log-probabilities, KL and entropy within 1e-5 relative
/ 1e-6 absolute for f32 inputs and 2e-3 relative for bf16 inputs; reruns bit-identical.
"""
import math

import numpy as np
import pytest
from scipy.special import log_softmax

import noetic_rl as nr
import workloads as W
from oracle import oracle as O

pytestmark = pytest.mark.gpu

EDGE = 1e-6


@pytest.fixture(scope="module", autouse=True)
def device():
    nr.claim(0)
    yield


def close_f32(ours, want):
    """|Δ| <= 1e-6 + 1e-5 |ref| (f32 inputs)."""
    ours, want = np.asarray(ours, np.float64), np.asarray(want, np.float64)
    same_inf = np.isinf(ours) & (ours == want)
    err = np.where(same_inf, 0.0, np.abs(ours - want) - (1e-6 + 1e-5 * np.abs(want)))
    return err <= 0.0


def close_bf16(ours, want):
    """|Δ| <= 2e-3 |ref| (bf16 inputs; a 1e-6 floor for values at zero)."""
    ours, want = np.asarray(ours, np.float64), np.asarray(want, np.float64)
    same_inf = np.isinf(ours) & (ours == want)
    err = np.where(same_inf, 0.0, np.abs(ours - want) - (1e-6 + 2e-3 * np.abs(want)))
    return err <= 0.0


def rel_err(ours, want):
    ours, want = np.asarray(ours, np.float64), np.asarray(want, np.float64)
    fin = np.isfinite(want)
    return float(np.max(np.abs(ours[fin] - want[fin]) / (1.0 + np.abs(want[fin])))) if fin.any() else 0.0


def check_sample(name, z, u, ids, logp, ent=None, bf16=False):
    """ids vs the oracle (boundary draws counted), logp/entropy within the dtype's tolerance."""
    want_ids, edges = O.sample_invcdf(z, u)
    differ = np.nonzero(ids != want_ids)[0]
    boundary = int(np.sum(edges < EDGE))
    assert np.all(edges[differ] < EDGE), f"{name}: {len(differ)} ids differ away from a CDF edge: rows {differ[:8]}"
    ok = close_bf16 if bf16 else close_f32
    want_lp = O.token_logp(z, ids)
    assert np.all(ok(logp, want_lp)), f"{name}: logp off by {rel_err(logp, want_lp):.3e}"
    msg = f"{name}: {len(ids)} rows, {len(differ)} ids differ ({boundary} boundary draws), logp rel {rel_err(logp, want_lp):.2e}"
    if ent is not None:
        want_h = O.entropy(z)
        assert np.all(ok(ent, want_h)), f"{name}: entropy off by {rel_err(ent, want_h):.3e}"
        msg += f", entropy rel {rel_err(ent, want_h):.2e}"
    print(msg)
    return len(differ)


def test_c1_golden_fixture_on_device():
    import json, os
    with open(os.path.join(os.path.dirname(__file__), "golden", "c1_readme.json")) as f:
        fx = json.load(f)
    S, B, T, V = fx["shape"]
    x = np.stack([np.frombuffer(bytes.fromhex(h), dtype=np.float32) for h in fx["logits_f32_hex"]])
    keep = np.array(fx["keep_u8"], dtype=np.uint8)
    u = np.array(fx["uniforms"])
    xt = nr.Tensor.from_numpy(x.reshape(S, B, T, V))
    mt = nr.Tensor.from_numpy(keep.reshape(S, B, T, V))
    ut = nr.Tensor.from_numpy(u, "f64")
    ids, lp, ent = nr.sample_logp(xt, 1.0, mt, None, entropy=True, uniforms=ut)
    ids, lp, ent = ids.to_numpy().ravel(), lp.to_numpy().ravel(), ent.to_numpy().ravel()
    edges = np.array(fx["edge_distance"])
    differ = np.nonzero(ids != np.array(fx["ids"]))[0]
    assert np.all(edges[differ] < EDGE)
    assert np.all(close_f32(lp, fx["logp"])), rel_err(lp, fx["logp"])
    assert np.all(close_f32(ent, fx["entropy"])), rel_err(ent, fx["entropy"])


def test_c4_north_star_parity_and_rerun_bits():
    w = W.c4()
    rows, V = w["rows"], w["V"]
    u = nr.Rng(2024, "c4/uniforms").uniforms(rows)
    ut = nr.Tensor.from_numpy(u, "f64")
    ids, lp = nr.sample_logp(w["logits"], w["temperature"], w["mask"], None, uniforms=ut)
    ids2, lp2 = nr.sample_logp(w["logits"], w["temperature"], w["mask"], None, uniforms=ut)
    a, b = ids.to_numpy().ravel(), lp.to_numpy().ravel()
    assert np.array_equal(a, ids2.to_numpy().ravel()) and b.tobytes() == lp2.to_numpy().ravel().tobytes(), "rerun bits"
    x = W.bf16_to_f32(w["logits"].to_numpy().reshape(rows, V))
    keep = w["mask"].to_numpy().reshape(rows, V)
    assert keep[np.arange(rows), a].all(), "an excluded token was drawn"
    z = O.tempered(x, w["temperature"], keep=keep)
    # the f32 tolerance (the bf16 inputs are exact in f32; the kernel computes in f32 and f64)
    check_sample("c4", z, u, a, b, bf16=False)


def test_c2_decode_parity():
    w = W.c2()
    rows, V = w["rows"], w["V"]
    u = nr.Rng(2024, "c2/uniforms").uniforms(rows)
    ids, lp, ent = nr.sample_logp(w["logits"], w["temperature"], None, None, entropy=True,
                                  uniforms=nr.Tensor.from_numpy(u, "f64"))
    x = w["logits"].to_numpy().reshape(rows, V)
    z = O.tempered(x, w["temperature"])
    check_sample("c2", z, u, ids.to_numpy().ravel(), lp.to_numpy().ravel(), ent.to_numpy().ravel())


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("V", [1, 7, 1000, 1001, 1008, 4099])
def test_ragged_and_unaligned_rows(dtype, V):
    rng = np.random.default_rng(V)
    rows = 33
    x = rng.normal(0, 3, (rows, V)).astype(np.float32)
    if dtype == "bf16":
        xb = O.bf16_from_f32(x)
        x = O.bf16_to_f32(xb)
        xt = nr.Tensor.from_numpy(xb, "bf16")
    else:
        xt = nr.Tensor.from_numpy(x)
    keep = (rng.random((rows, V)) < 0.6).astype(np.uint8)
    keep[np.arange(rows), rng.integers(0, V, rows)] = 1
    u = nr.Rng(V, "ragged").uniforms(rows)
    for tau in (1.0, 0.45):
        ids, lp, ent = nr.sample_logp(xt, tau, nr.Tensor.from_numpy(keep), None, entropy=True,
                                      uniforms=nr.Tensor.from_numpy(u, "f64"))
        z = O.tempered(x, tau, keep=keep)
        check_sample(f"ragged {dtype} V={V} T={tau}", z, u, ids.to_numpy(), lp.to_numpy(), ent.to_numpy(),
                     bf16=dtype == "bf16")


def test_greedy_is_the_first_masked_argmax():
    # tests/rl.rs:617-625 plus ties: the first maximum wins
    row = np.array([0.4, -1.0, 1.2, 3.0, 0.0, -0.3], dtype=np.float32)
    x = nr.Tensor.from_numpy(np.stack([row, row, np.array([1, 5, 5, 2, 5, 0], np.float32)]))
    mask = nr.Tensor.from_numpy(np.array([[0.0, 0.0, 0.0, -np.inf, 2.0, 0.0]], np.float32))
    ids, lp = nr.sample_logp(x, 0.0, mask, None)
    assert ids.to_numpy().tolist() == [4, 4, 4]
    ids, lp = nr.sample_logp(x, 0.0, None, None)
    assert ids.to_numpy().tolist() == [3, 3, 1]
    z = O.tempered(np.stack([row, row, np.array([1, 5, 5, 2, 5, 0], np.float32)]), 1.0)
    assert np.all(close_f32(lp.to_numpy(), O.token_logp(z, [3, 3, 1])))


def test_rows_with_no_allowed_token_are_refused():
    x = nr.Tensor.from_numpy(np.zeros((2, 3), np.float32))
    keep = nr.Tensor.from_numpy(np.array([[1, 1, 1], [0, 0, 0]], np.uint8))
    nanrow = nr.Tensor.from_numpy(np.array([[0.0, np.nan, 1.0], [0.0, 1.0, 2.0]], np.float32))
    for sampler in (nr.sample_categorical, nr.sample_categorical_inv_cdf):
        with pytest.raises(ValueError, match="position 1 has no allowed token"):
            sampler(x, 1.0, keep, nr.Rng(0, "x"))
        with pytest.raises(ValueError, match="position 0"):
            sampler(nanrow, 1.0, None, nr.Rng(0, "x"))


def test_additive_minus_1e9_equals_minus_infinity_to_the_bit():
    # tests/rl.rs:773-813
    rng = np.random.default_rng(11)
    rows, V = 24, 37
    x = nr.Tensor.from_numpy(rng.uniform(-4, 4, (2, 3, 4, V)).astype(np.float32))
    refl = nr.Tensor.from_numpy(rng.uniform(-4, 4, (2, 3, 4, V)).astype(np.float32))
    tok = rng.integers(0, V, (2, 3, 4)).astype(np.int32)
    tok[tok == 3] = 1
    tok = nr.Tensor.from_numpy(tok)
    outs = []
    for fill in (-1e9, -np.inf):
        vm = nr.Tensor.from_numpy(np.array([[[[fill if k == 3 else 0.0 for k in range(V)]]]], np.float32))
        lp, rlp, kl, ent = nr.score(nr.tempered_logits(x, 0.8, vm), nr.tempered_logits(refl, 0.8, vm), tok)
        ids, slp = nr.sample_logp(x, 0.8, vm, nr.Rng(1, "m"))
        outs.append([a.to_numpy().tobytes() for a in (lp, rlp, kl, ent, ids, slp)])
    for a, b in zip(*outs):
        assert a == b


def test_inv_cdf_sampler_on_the_reference_body_inputs():
    # The inverse-CDF entry on the inputs of src/nn/tests/gpu/rl.rs:155-174 (rnd(n V, 960, -3, 3),
    # mask k%7==3 -> -inf, temperatures 1, 0.7 and 0), against the oracle's inverse-CDF draw for
    # the same uniforms (the reference's Gumbel sampler body itself runs in test_gumbel_gpu.py).
    shape = (4, 128, 96)
    n = 4 * 128
    x = O.reference_rnd_f64(960, n * 96, -3.0, 3.0).astype(np.float32).reshape(shape)
    mask = np.array([[[-np.inf if k % 7 == 3 else 0.0 for k in range(96)]]], np.float32)
    xt, mt = nr.Tensor.from_numpy(x), nr.Tensor.from_numpy(mask)
    for tau, root in [(1.0, 11), (0.7, 12), (0.0, 13)]:
        rng_s = nr.Rng(root, "device sampler")
        u = rng_s.clone().uniforms(n)
        ids, lp = nr.sample_logp(xt, tau, mt, rng_s)
        ids = ids.to_numpy().ravel()
        assert np.all(ids % 7 != 3)
        z = O.tempered(x.reshape(n, 96), 1.0 if tau == 0 else tau, addmask=mask.reshape(1, 96))
        if tau == 0:
            assert np.array_equal(ids, O.argmax_first(z))
        else:
            check_sample(f"sampler body T={tau}", z, u, ids, lp.to_numpy().ravel())
        again = nr.sample_logp(xt, tau, mt, nr.Rng(root, "device sampler"))[0].to_numpy().ravel()
        assert np.array_equal(again, ids), "run to run"


def test_frequencies_over_many_rows_on_device():
    # the reference's frequency check (tests/rl.rs:579-611) on the inverse-CDF entry; one u64 per
    # row consumed
    row = np.array([0.4, -1.0, 1.2, 3.0, 0.0, -0.3], np.float32)
    n = 40_000
    x = nr.Tensor.from_numpy(np.repeat(row[None, :], n, 0))
    mask = nr.Tensor.from_numpy(np.array([[0.0, 0.0, 0.0, -np.inf, 0.5, 0.0]], np.float32))
    for tau in (0.7, 2.5):
        rng = nr.Rng(5, "sampler test")
        copy = rng.clone()
        ids = nr.sample_categorical_inv_cdf(x, tau, mask, rng).to_numpy()
        copy.skip_u64(n)
        assert rng.next_u64() == copy.next_u64(), "one u64 per row"
        p = np.exp(log_softmax(row.astype(np.float64) / tau + np.array([0, 0, 0, -np.inf, 0.5, 0])))
        cnt = np.bincount(ids, minlength=6)
        assert cnt[3] == 0
        se = np.sqrt(p * (1 - p) / n)
        assert np.all(np.abs(cnt / n - p) <= 4.5 * se + 1e-12)


def _score_check(name, xf, yf, tok, lp, rlp, kl, ent, ok):
    want_lp = O.token_logp(xf, tok)
    want_rlp = O.token_logp(yf, tok)
    want_kl = O.kl(xf, yf)
    want_h = O.entropy(xf)
    for what, a, b in (("logp", lp, want_lp), ("ref_logp", rlp, want_rlp), ("kl", kl, want_kl), ("entropy", ent, want_h)):
        assert np.all(ok(a, b)), f"{name} {what}: rel {rel_err(a, b):.3e}; worst {np.asarray(a)[~ok(a, b)][:3]} vs {np.asarray(b)[~ok(a, b)][:3]}"
    print(f"{name}: logp {rel_err(lp, want_lp):.1e} ref {rel_err(rlp, want_rlp):.1e} kl {rel_err(kl, want_kl):.1e} "
          f"entropy {rel_err(ent, want_h):.1e}")


def test_c3_scoring_parity_on_a_row_slice():
    w = W.c3(rows=512)
    rows, V = w["rows"], w["V"]
    lp, rlp, kl, ent = nr.score(w["logits"], w["ref"], w["tokens"])
    lp2, rlp2, kl2, ent2 = nr.score(w["logits"], w["ref"], w["tokens"])
    for a, b in ((lp, lp2), (rlp, rlp2), (kl, kl2), (ent, ent2)):
        assert a.to_numpy().tobytes() == b.to_numpy().tobytes(), "rerun bits"
    xf = W.bf16_to_f32(w["logits"].to_numpy())
    yf = W.bf16_to_f32(w["ref"].to_numpy())
    tok = w["tokens"].to_numpy()
    _score_check("c3 slice", xf, yf, tok, lp.to_numpy(), rlp.to_numpy(), kl.to_numpy(), ent.to_numpy(), close_bf16)
    # per-sampled-token estimators and reductions on the device against the oracle
    S, B, T = 4, 8, 16
    shp = (S, B, T)
    lpt = nr.Tensor(shp, "f32", lp.buf)
    rlpt = nr.Tensor(shp, "f32", rlp.buf)
    m = (np.random.default_rng(3).random(shp) < 0.75).astype(np.float32)
    m[1, 2, :] = 0.0
    mt = nr.Tensor.from_numpy(m)
    for est in (nr.KlEstimator.K1, nr.KlEstimator.K2, nr.KlEstimator.K3):
        for clamp in (None, 20.0):
            per = O.kl_estimate(lp.to_numpy().astype(np.float64), rlp.to_numpy().astype(np.float64), int(est), clamp, m)
            for red in nr.TokenReduction:
                got = nr.kl_estimate(lpt, rlpt, est, clamp, mt, red).to_numpy().ravel()
                want = O.reduce_tokens(per, m, shp, red.name.lower())
                assert np.all(close_f32(got, want)), (est, clamp, red, rel_err(got, want))


def test_f32_scoring_with_temperature_and_mask():
    rng = np.random.default_rng(21)
    rows, V = 64, 5000
    x = rng.normal(0, 2, (rows, V)).astype(np.float32)
    y = (x + rng.normal(0, 0.3, (rows, V))).astype(np.float32)
    keep = (rng.random((1, V)) < 0.7).astype(np.uint8)
    tok = rng.integers(0, V, rows).astype(np.int32)
    tok = np.where(keep[0, tok] == 1, tok, np.argmax(keep[0])).astype(np.int32)
    tau = 0.8
    xt, yt, mt, tt = nr.Tensor.from_numpy(x), nr.Tensor.from_numpy(y), nr.Tensor.from_numpy(keep), nr.Tensor.from_numpy(tok)
    lp, rlp, kl, ent = nr.score(nr.tempered_logits(xt, tau, mt), nr.tempered_logits(yt, tau, mt), tt)
    xf, yf = O.tempered(x, tau, keep=keep), O.tempered(y, tau, keep=keep)
    _score_check("f32 scoring", xf, yf, tok, lp.to_numpy(), rlp.to_numpy(), kl.to_numpy(), ent.to_numpy(), close_f32)


def test_reference_losses_body_values():
    # src/nn/tests/gpu/rl.rs:38-68: SH [2,8,12], V 24, logits in [-6,6] with ±1e4 and −∞ (in both
    # distributions) at entries that are not the token, sequence 3 of seed 0 masked; values
    # within 1e-5 under |Δ|/(1+|ref|).
    SH, V = (2, 8, 12), 24
    n = 2 * 8 * 12
    rng = np.random.default_rng(950)
    logits = rng.uniform(-6, 6, (n, V))
    refl = rng.uniform(-6, 6, (n, V))
    tokens = rng.integers(0, V, n)
    for i in range(0, n, 5):
        t = tokens[i]
        a, b = (t + 1) % V, (t + 2) % V
        logits[i, a] = refl[i, a] = -np.inf
        logits[i, b] = 1e4 if i % 2 == 0 else -1e4
    mask = (rng.random(n) < 0.75).astype(np.float64)
    mask[3 * 12:4 * 12] = 0.0
    x32, r32 = logits.astype(np.float32), refl.astype(np.float32)
    xt = nr.Tensor.from_numpy(x32.reshape(*SH, V))
    rt = nr.Tensor.from_numpy(r32.reshape(*SH, V))
    tt = nr.Tensor.from_numpy(tokens.astype(np.int32).reshape(SH))
    mt = nr.Tensor.from_numpy(mask.astype(np.float32).reshape(SH))
    tol = 1e-5
    lp = nr.token_log_probs(xt, tt).to_numpy().ravel()
    want = O.token_logp(x32, tokens)
    assert rel_err(lp, want) <= tol and np.all(np.isfinite(lp))
    ent_want = O.entropy(x32)
    kl_want = O.kl(x32, r32)
    for red in nr.TokenReduction:
        got = nr.categorical_entropy(xt, mt, red).to_numpy().ravel()
        assert rel_err(got, O.reduce_tokens(ent_want * mask, mask, SH, red.name.lower())) <= tol, red
        got = nr.categorical_kl(xt, rt, mt, red).to_numpy().ravel()
        assert rel_err(got, O.reduce_tokens(kl_want * mask, mask, SH, red.name.lower())) <= tol, red
    # the reference KL under a −1e9 vocabulary mask at temperature 0.8
    vm = np.array([[[[-1e9 if k == 5 else 0.0 for k in range(V)]]]], np.float32)
    vmt = nr.Tensor.from_numpy(vm)
    got = nr.reference_kl(xt, rt, 0.8, vmt, mt, nr.TokenReduction.NONE).to_numpy().ravel()
    want = O.kl(O.tempered(x32, 0.8, addmask=vm.reshape(1, V)), O.tempered(r32, 0.8, addmask=vm.reshape(1, V))) * mask
    assert rel_err(got, want) <= tol
    again = nr.reference_kl(xt, rt, 0.8, vmt, mt, nr.TokenReduction.NONE).to_numpy().ravel()
    assert got.tobytes() == again.tobytes()


def _sample_rows(rows, n, seed):
    """The first, second and last rows plus n - 3 others, sorted."""
    rng = np.random.default_rng(seed)
    pick = {0, 1, rows - 1} | set(rng.choice(rows, n - 3, replace=False).tolist())
    return np.array(sorted(pick))


def test_c3_full_size_scoring():
    # benchmark configuration 3 at its real size: 2 x bf16 [8,16,512,50304] (13.2 GB). Rows spread over
    # the tensor against the oracle; every row through size-independent properties.
    w = W.c3()
    rows, V = w["rows"], w["V"]
    lp, rlp, kl, ent = nr.score(w["logits"], w["ref"], w["tokens"])
    lp2, rlp2, kl2, ent2 = nr.score(w["logits"], w["ref"], w["tokens"])
    outs = [t.to_numpy().ravel() for t in (lp, rlp, kl, ent)]
    for a, b in zip(outs, (lp2, rlp2, kl2, ent2)):
        assert a.tobytes() == b.to_numpy().ravel().tobytes(), "rerun bits"
    lpn, rlpn, kln, entn = outs
    assert np.all(np.isfinite(lpn)) and np.all(lpn <= 0.0) and np.all(rlpn <= 0.0)
    assert np.all(kln >= -1e-6), f"KL < 0 at {np.nonzero(kln < -1e-6)[0][:4]}"
    assert np.all(entn >= 0.0) and np.all(entn <= math.log(V) * (1 + 1e-6))
    sel = np.union1d(_sample_rows(rows, 48, 33), np.argsort(entn)[:16])
    xf = W.bf16_to_f32(W.download_rows(w["logits"], sel, V))
    yf = W.bf16_to_f32(W.download_rows(w["ref"], sel, V))
    tok = w["tokens"].to_numpy().ravel()[sel]
    _score_check("c3 full", xf, yf, tok, lpn[sel], rlpn[sel], kln[sel], entn[sel], close_f32)
    # k3 per sampled token over the whole batch against the oracle's closed form
    S, B, T = w["logits"].shape[:-1]
    k3 = nr.kl_estimate(nr.Tensor((S, B, T), "f32", lp.buf), nr.Tensor((S, B, T), "f32", rlp.buf),
                        nr.KlEstimator.K3, None, None, nr.TokenReduction.NONE).to_numpy().ravel()
    want = O.kl_estimate(lpn.astype(np.float64), rlpn.astype(np.float64), 3, None, None)
    assert np.all(close_f32(k3, want)), rel_err(k3, want)


def test_c5_full_size_scoring_and_group_advantages():
    # benchmark configuration 5 at its real size: f32 [4,32,1024,151936] (79.7 GB) + u8 mask (19.9 GB).
    w = W.c5()
    rows, V = w["rows"], w["V"]
    S, B, T = w["logits"].shape[:-1]
    lp, _, _, ent = nr._score(nr.tempered_logits(w["logits"], 1.0, w["mask"]), None, w["tokens"], True, False, False,
                              True)[:4]
    lpn, entn = lp.to_numpy().ravel(), ent.to_numpy().ravel()
    assert np.all(np.isfinite(lpn)) and np.all(lpn <= 0.0), "every scored token is kept"
    assert np.all(entn >= 0.0) and np.all(entn <= math.log(V) * (1 + 1e-6))
    # random rows, and the 16 of lowest entropy (where the 1e-6 absolute floor is what holds)
    sel = np.union1d(_sample_rows(rows, 32, 55), np.argsort(entn)[:16])
    x = W.download_rows(w["logits"], sel, V)
    keep = W.download_rows(w["mask"], sel, V)
    z = O.tempered(x, 1.0, keep=keep)
    tok = w["tokens"].to_numpy().ravel()[sel]
    want_lp, want_h = O.token_logp(z, tok), O.entropy(z)
    assert np.all(close_f32(lpn[sel], want_lp)), rel_err(lpn[sel], want_lp)
    assert np.all(close_f32(entn[sel], want_h)), rel_err(entn[sel], want_h)
    print(f"c5 full: logp rel {rel_err(lpn[sel], want_lp):.1e}, entropy rel {rel_err(entn[sel], want_h):.1e}")
    # rewards = each sequence's mean log-probability (device), advantages over groups of 8 along B
    rew = nr._reduce(nr.Tensor((S, B, T), "f32", lp.buf), None, nr.TokenReduction.PER_SEQUENCE)
    rewn = rew.to_numpy().astype(np.float64).ravel()
    want_rew = O.reduce_tokens(lpn.astype(np.float64), np.ones(S * B * T), (S, B, T), "per_sequence")
    assert np.all(close_f32(rewn, want_rew)), rel_err(rewn, want_rew)
    adv = nr.group_advantages_tensor(nr.Tensor.from_numpy(rewn.reshape(S, B // 8, 8).astype(np.float32)), "std",
                                     1e-6).to_numpy().astype(np.float64)
    want_adv = O.group_advantages(rewn.astype(np.float32).astype(np.float64), 8, "std", 1e-6)
    assert np.all(close_f32(adv.ravel(), want_adv)), rel_err(adv.ravel(), want_adv)
    assert np.all(np.abs(adv.reshape(-1, 8).sum(axis=1)) < 1e-4), "each group's advantages sum to zero"


@pytest.mark.parametrize("case", [
    # (dtype, mask kind, broadcast mask, V, temperature, entropy)
    ("bf16", "u8", True, 128256, 0.7, False),   # c4's shape with one shared [1, V] grammar mask
    ("bf16", "u8", False, 128256, 0.7, True),   # c4 with the entropy output (register-resident)
    ("f32", "f32", False, 32768, 0.8, True),    # additive f32 mask at the register-resident limit
    ("f32", "f32", True, 20000, 1.0, False),    # additive mask shared by every row, temperature 1
    ("f32", "u8", False, 65536, 1.3, False),    # f32 logits, u8 mask, the largest f32 row kept in VGPRs
    ("bf16", "none", False, 131072, 0.5, True), # no mask, the largest register-resident bf16 row
])
def test_sampler_mask_layouts_against_the_oracle(case):
    dtype, mk, shared, V, tau, want_ent = case
    rows = 48
    rng = np.random.default_rng(V + int(100 * tau))
    x = rng.normal(0, 2, (rows, V)).astype(np.float32)
    if dtype == "bf16":
        xb = O.bf16_from_f32(x)
        x = O.bf16_to_f32(xb)
        xt = nr.Tensor.from_numpy(xb, "bf16")
    else:
        xt = nr.Tensor.from_numpy(x)
    mrows = 1 if shared else rows
    keep = add = mt = None
    if mk == "u8":
        keep = (rng.random((mrows, V)) < 0.3).astype(np.uint8)
        keep[:, rng.integers(0, V)] = 1
        mt = nr.Tensor.from_numpy(keep)
    elif mk == "f32":
        add = np.where(rng.random((mrows, V)) < 0.5, 0.0, -np.inf).astype(np.float32)
        add[:, ::97] = -1e9
        add[:, rng.integers(0, V)] = 0.0
        mt = nr.Tensor.from_numpy(add)
    u = nr.Rng(V, "mask layouts").uniforms(rows)
    out = nr.sample_logp(xt, tau, mt, None, entropy=want_ent, uniforms=nr.Tensor.from_numpy(u, "f64"))
    ids, lp = out[0].to_numpy().ravel(), out[1].to_numpy().ravel()
    z = O.tempered(x, tau, addmask=add, keep=keep)
    ent = out[2].to_numpy().ravel() if want_ent else None
    check_sample(f"{case}", z, u, ids, lp, ent, bf16=False)



@pytest.mark.parametrize("case", [
    # (dtype, V, rows, one shared mask row, temperature, entropy, NOETIC_HIP_SAMPLE_RR)
    ("bf16", 128256, 96, False, 0.7, True, None),   # C4's vocabulary: 251 chunks, the last half full; 16 waves
    ("f16", 40000, 72, False, 1.0, False, None),    # 79 chunks
    ("bf16", 32776, 80, False, 0.0, False, None),   # greedy; 65 chunks, the last of 8 elements
    ("bf16", 33280, 2048, True, 0.9, True, None),   # 2048 rows: 4 waves per row; one mask row for all
    ("bf16", 4104, 40, False, 0.8, True, "off"),    # 9 chunks: 2 waves (the streaming kernel forced)
    ("f16", 1032, 24, False, 1.3, True, "off"),     # 3 chunks: 1 wave
])
def test_streaming_sampler_f32_masks_on_16_bit_rows(case, monkeypatch):
    """An additive f32 mask on aligned 16-bit rows longer than the register-resident kernel holds
    (V > 32768 there) takes the streaming sampler, which stages each wave's mask words through
    LDS, two chunks at a time. Masks mix -inf, -1e9 and finite values; rows, chunk counts and
    wave counts cover a partial last chunk, 1, 2, 4 and 16 waves per row and a shared mask row."""
    dtype, V, rows, shared, tau, want_ent, rr = case
    if rr:
        monkeypatch.setenv("NOETIC_HIP_SAMPLE_RR", rr)
    rng = np.random.default_rng(V + rows)
    x = rng.normal(0, 2, (rows, V)).astype(np.float32)
    if dtype == "bf16":
        xb = O.bf16_from_f32(x)
        x = O.bf16_to_f32(xb)
        xt = nr.Tensor.from_numpy(xb, "bf16")
    else:
        h = x.astype(np.float16)
        x = h.astype(np.float32)
        xt = nr.Tensor.from_numpy(h.view(np.uint16), "f16")
    mrows = 1 if shared else rows
    add = np.where(rng.random((mrows, V)) < 0.4, -np.inf, rng.normal(0, 0.5, (mrows, V))).astype(np.float32)
    add[:, ::97] = -1e9
    add[:, rng.integers(0, V)] = 0.0
    mt = nr.Tensor.from_numpy(add)
    u = nr.Rng(V, "streaming f32 masks").uniforms(rows)
    out = nr.sample_logp(xt, tau, mt, None, entropy=want_ent, uniforms=nr.Tensor.from_numpy(u, "f64"))
    ids, lp = out[0].to_numpy().ravel(), out[1].to_numpy().ravel()
    ent = out[2].to_numpy().ravel() if want_ent else None
    sel = np.arange(rows) if rows <= 96 else np.arange(0, rows, 64)
    xs = x[sel]
    am = add if shared else add[sel]
    z = O.tempered(xs, 1.0 if tau == 0 else tau, addmask=np.broadcast_to(am, xs.shape))
    if tau == 0.0:
        assert np.array_equal(ids[sel], O.argmax_first(z)), f"{case}: greedy ids"
        assert np.all(close_f32(lp[sel], O.token_logp(z, ids[sel]))), f"{case}: greedy logp"
    else:
        check_sample(f"{case}", z, u[sel], ids[sel], lp[sel], None if ent is None else ent[sel])
    again = nr.sample_logp(xt, tau, mt, None, entropy=want_ent, uniforms=nr.Tensor.from_numpy(u, "f64"))
    for a, b in zip(out, again):
        assert a.to_numpy().tobytes() == b.to_numpy().tobytes(), f"{case}: rerun bits"

def _peaked_rows(rows, V, seed, bf16):
    """N(0,1) rows with one dominant logit (+20 .. +60) placed late in the row (after every
    early reference has been set), at an index that differs per row; the tokens are the peaks,
    whose logp is near 0 (where only the 1e-6 absolute floor holds)."""
    rng = np.random.default_rng(seed)
    x = rng.normal(0, 1, (rows, V)).astype(np.float32)
    peak = (V - 1 - rng.integers(0, V // 3, rows)).astype(np.int64)
    x[np.arange(rows), peak] = rng.uniform(20, 60, rows).astype(np.float32)
    y = (x + rng.normal(0, 0.3, x.shape)).astype(np.float32)
    if bf16:
        xb, yb = O.bf16_from_f32(x), O.bf16_from_f32(y)
        return O.bf16_to_f32(xb), O.bf16_to_f32(yb), nr.Tensor.from_numpy(xb, "bf16"), nr.Tensor.from_numpy(yb, "bf16"), peak
    return x, y, nr.Tensor.from_numpy(x), nr.Tensor.from_numpy(y), peak


@pytest.mark.parametrize("dtype,V", [("f32", 151936), ("bf16", 50304), ("f32", 4099)])
def test_peaked_rows_scoring_keeps_the_tolerance(dtype, V):
    # A late dominant logit: entropy and KL near 0 and logp near 0, computed as differences of
    # log-sums (ln S - ln2 H / S, ln S - ln S_ref, (z - m) - ln S) that must not cancel.
    rows = 48
    x, y, xt, yt, peak = _peaked_rows(rows, V, V, dtype == "bf16")
    tok = peak.astype(np.int32)
    lp, rlp, kl, ent = nr.score(xt, yt, nr.Tensor.from_numpy(tok))
    _score_check(f"peaked {dtype} V{V}", x, y, tok, lp.to_numpy(), rlp.to_numpy(), kl.to_numpy(), ent.to_numpy(),
                 close_f32)
    assert np.max(ent.to_numpy()) < 1e-2, "the rows are peaked"


@pytest.mark.parametrize("dtype,V", [("bf16", 128256), ("f32", 32000), ("bf16", 1000), ("bf16", 151936)])
def test_peaked_rows_sampling_keeps_the_tolerance(dtype, V):
    # The sampler's logp of the (almost always drawn) peak, and its entropy, on the same rows.
    rows = 64
    x, _, xt, _, peak = _peaked_rows(rows, V, V + 1, dtype == "bf16")
    u = np.random.default_rng(V).random(rows)
    ids, lp, ent = nr.sample_logp(xt, 1.0, None, None, entropy=True, uniforms=nr.Tensor.from_numpy(u, "f64"))
    check_sample(f"peaked {dtype} V{V}", x, u, ids.to_numpy().ravel(), lp.to_numpy().ravel(), ent.to_numpy().ravel())
    assert np.mean(ids.to_numpy().ravel() == peak) > 0.9


@pytest.mark.parametrize("V,seg", [(4096, "off"), (50304, "off"), (128256, "off"), (4099, "off"), (128256, "8,4")])
@pytest.mark.parametrize("mask", ["none", "u8"])
def test_rows_below_minus_flt_max_tau_have_no_token(V, seg, mask, monkeypatch):
    """Every allowed logit at -3.3e38 with T = 0.7: the tempered values x / T are all -inf, so the
    row has no allowed token (the reference's max_dim is -inf, rl.rs:515-519) and every kernel
    refuses it with NT_ROW_NO_TOKEN: the samplers (register-resident, queued, streaming at an
    unaligned V, segmented) and the scorer. The other rows are unaffected."""
    import ctypes as C
    monkeypatch.setenv("NOETIC_HIP_SAMPLE_SEG", seg)
    rows = 4
    rng = np.random.default_rng(V)
    x = rng.normal(0, 1, (rows, V)).astype(np.float32)
    x[2] = -3.3e38
    keep = None
    if mask == "u8":
        keep = np.ones((rows, V), np.uint8)
        keep[:, ::3] = 0
        mt, kind = nr.Tensor.from_numpy(keep), nr.NT_MASK_U8
    else:
        mt, kind = None, nr.NT_MASK_NONE
    xt = nr.Tensor.from_numpy(x)
    u = nr.Tensor.from_numpy(np.full(rows, 0.5), "f64")
    ids, lp, st = nr.IntTensor((rows,)), nr.Tensor((rows,), "f32"), nr.Tensor((rows,), "u8")
    a = nr.NtRlSampleArgs(xt.ptr, nr.NT_F32, kind, rows, V, V, None if mt is None else mt.ptr, 0 if mt is None else V,
                          0.7, u.ptr, ids.ptr, lp.ptr, None, st.ptr)
    nr._check(nr.lib().nt_hip_rl_sample(C.byref(a)), "sample")
    s = st.to_numpy()
    assert s[2] == nr.NT_ROW_NO_TOKEN and ids.to_numpy()[2] == -1, s
    assert np.all(s[[0, 1, 3]] == nr.NT_ROW_OK), s
    tok = nr.Tensor.from_numpy(np.zeros(rows, np.int32))
    slp, sst = nr.Tensor((rows,), "f32"), nr.Tensor((rows,), "u8")
    b = nr.NtRlScoreArgs(xt.ptr, None, nr.NT_F32, kind, rows, V, V, None if mt is None else mt.ptr,
                         0 if mt is None else V, 0.7, tok.ptr, slp.ptr, None, None, None, sst.ptr, None, None, None, None)
    nr._check(nr.lib().nt_hip_rl_score(C.byref(b)), "score")
    assert sst.to_numpy()[2] == nr.NT_ROW_NO_TOKEN, sst.to_numpy()
