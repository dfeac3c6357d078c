"""The readout-fused scorer (nt_hip_rl_readout_score) against the oracle.

Pass 1's logits (written by the debug pointer) are the product the scorer saw; on them the
oracle's f64 token_log_probs and categorical_entropy (rl.rs:134-141, 405-414) of the tempered,
masked rows are the expected values, within the f32 tolerance (1e-5 relative / 1e-6 absolute).
The same rows through the unfused scorer (nt_hip_rl_score on the written logits) agree to the
same tolerance. Scoring the sampler's own draws gives the sampler's log-probabilities bit for bit
(the same records, merged in the same order, and the same recomputed block). Reruns are
byte-identical; excluded tokens give -inf, tokens out of range raise, and a row with nothing
allowed gives NaN, as the unfused scorer does."""
import numpy as np
import pytest

import noetic_rl as nr
import workloads as W
from oracle import oracle as O

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def device():
    nr.claim(0)
    # the readout fusion is the reduced-precision product: it runs at MatmulPrecision::Half
    prev = nr.set_matmul_precision(nr.MatmulPrecision.HALF)
    yield
    nr.set_matmul_precision(prev)


def close(name, got, want):
    got = np.asarray(got, np.float64)
    fin = np.isfinite(want)
    assert np.array_equal(np.isfinite(got), fin), f"{name}: finite pattern differs"
    assert np.array_equal(got[~fin], want[~fin]), f"{name}: non-finite values differ"
    err = np.abs(got[fin] - want[fin])
    assert np.all(err <= 1e-6 + 1e-5 * np.abs(want[fin])), f"{name}: off by {err.max():.2e}"
    return float(err.max()) if err.size else 0.0


def normal(shape, dtype, seed, label, std):
    """W.normal's values; f16 ones drawn in f32 and rounded to f16 on the host."""
    if dtype != "f16":
        return W.normal(shape, dtype, seed, label, std=std)
    f = W.normal(shape, "f32", seed, label, std=std).to_numpy()
    return nr.Tensor.from_numpy(f.astype(np.float16).view(np.uint16), "f16")


def make(name, rows, V, d, seed, masked, dtype="bf16"):
    h = normal((rows, d), dtype, seed, f"readout/{name}/h", std=1.0)
    w = normal((d, V), dtype, seed, f"readout/{name}/w", std=2.0 / np.sqrt(d))
    packed = nr.PackedReadout(w, "dv")
    rng = np.random.default_rng(seed)
    keep = mt = None
    if masked:
        keep = (rng.random((rows, V)) < 0.3).astype(np.uint8)
        keep[np.arange(rows), rng.integers(0, V, rows)] = 1
        mt = nr.Tensor.from_numpy(keep, "u8")
    return h, packed, keep, mt, rng


def run_case(name, rows, V, d, tau, masked, seed, dtype="bf16"):
    h, packed, keep, mt, rng = make(name, rows, V, d, seed, masked, dtype)
    tok = rng.integers(0, V, rows).astype(np.int32)
    if keep is not None:
        # mostly allowed tokens, and every fourth row's token as drawn (excluded ones among them)
        allowed = np.array([rng.choice(np.nonzero(keep[r])[0]) for r in range(rows)], np.int32)
        tok = np.where(np.arange(rows) % 4 == 0, tok, allowed).astype(np.int32)
    tt = nr.Tensor.from_numpy(tok)
    lp, ent, logits = nr.readout_score(h, packed, tau, mt, tt, entropy=True, debug=True)
    lp, ent, logits = lp.to_numpy().ravel(), ent.to_numpy().ravel(), logits.to_numpy()
    z = O.tempered(logits, tau, keep=keep)
    e1 = close(f"{name} logp", lp, O.token_logp(z, tok))
    e2 = close(f"{name} entropy", ent, O.entropy(z))
    if keep is not None:
        excl = keep[np.arange(rows), tok] == 0
        assert np.all(lp[excl] == -np.inf), f"{name}: an excluded token's logp"
    # the unfused scorer on the same (written) logits
    xt = nr.tempered_logits(nr.Tensor.from_numpy(logits), tau, mt)
    ulp, _, _, uent = nr.score(xt, None, tt, entropy=True, kl=False)
    close(f"{name} logp against the unfused scorer", lp, ulp.to_numpy().ravel().astype(np.float64))
    close(f"{name} entropy against the unfused scorer", ent, uent.to_numpy().ravel().astype(np.float64))
    # reruns, and the two halves asked for alone
    lp2, ent2 = nr.readout_score(h, packed, tau, mt, tt, entropy=True)
    assert lp2.to_numpy().tobytes() == lp.tobytes() and ent2.to_numpy().tobytes() == ent.tobytes(), f"{name}: rerun"
    lp3, none = nr.readout_score(h, packed, tau, mt, tt, entropy=False)
    assert none is None and lp3.to_numpy().tobytes() == lp.tobytes(), f"{name}: logp alone"
    none, ent3 = nr.readout_score(h, packed, tau, mt, None, entropy=True)
    assert none is None and ent3.to_numpy().tobytes() == ent.tobytes(), f"{name}: entropy alone"
    print(f"{name}: {rows} rows, logp max |d| {e1:.1e}, entropy max |d| {e2:.1e}")


@pytest.mark.parametrize("rows,V,d", [(40, 1000, 256), (256, 4104, 512), (1, 300, 64), (97, 257, 16), (64, 600, 528),
                                      (24, 151936, 64)])
@pytest.mark.parametrize("tau,masked", [(0.7, True), (1.0, False)])
def test_readout_scorer_small_shapes(rows, V, d, tau, masked):
    run_case(f"r{rows}v{V}d{d}t{tau}m{int(masked)}", rows, V, d, tau, masked, seed=rows + V + d + 1)


@pytest.mark.parametrize("tau,masked", [(0.7, True), (1.0, False)])
def test_readout_scorer_f16_operands(tau, masked):
    # an f16 head and f16 hidden rows, each rounded to bf16 as MatmulPrecision::Half loads them
    run_case(f"f16 r40v1000d256t{tau}m{int(masked)}", 40, 1000, 256, tau, masked, seed=1297, dtype="f16")


def test_readout_scorer_at_the_decode_shape():
    # C4's decode shape: 256 rows, d 4096, V 128256, a 30% keep-mask, T 0.7
    run_case("c4 readout score", 256, 128256, 4096, 0.7, True, seed=2025)


@pytest.mark.parametrize("tau,masked", [(0.7, True), (1.0, False)])
def test_scoring_the_samplers_draws_gives_its_logp_bit_for_bit(tau, masked):
    rows, V, d = 64, 5000, 256
    h, packed, keep, mt, rng = make("draws", rows, V, d, 31, masked)
    ut = nr.Tensor.from_numpy(nr.Rng(31, "readout/draws/u").uniforms(rows), "f64")
    ids, lp = nr.readout_sample_logp(h, packed, tau, mt, None, uniforms=ut)
    slp, _ = nr.readout_score(h, packed, tau, mt, ids, entropy=False)
    assert slp.to_numpy().tobytes() == lp.to_numpy().tobytes()


def test_readout_scorer_refusals():
    rows, V, d = 8, 512, 64
    h, packed, _, _, _ = make("refuse", rows, V, d, 5, False)
    keep = np.ones((rows, V), np.uint8)
    keep[3] = 0  # row 3 allows nothing
    mt = nr.Tensor.from_numpy(keep, "u8")
    tok = nr.Tensor.from_numpy(np.arange(rows, dtype=np.int32))
    lp, ent = nr.readout_score(h, packed, 1.0, mt, tok)
    lp, ent = lp.to_numpy().ravel(), ent.to_numpy().ravel()
    assert np.isnan(lp[3]) and np.isnan(ent[3])
    assert np.all(np.isfinite(np.delete(lp, 3))) and np.all(np.isfinite(np.delete(ent, 3)))
    # a token out of range: the unfused scorer's IndexError
    bad = nr.Tensor.from_numpy(np.array([0, 1, 2, 0, 4, V, 6, 7], np.int32))
    with pytest.raises(IndexError, match="gather index out of range"):
        nr.readout_score(h, packed, 1.0, None, bad)
    with pytest.raises(ValueError, match="must be positive"):
        nr.readout_score(h, packed, 0.0, None, tok)
