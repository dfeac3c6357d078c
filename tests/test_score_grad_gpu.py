"""GPU parity tests of the fused backward (nt_hip_rl_score_backward) against the CPU oracle's f64
gradient, on the same bytes.

The op sequence it replaces is the reference's autograd through tempered_logits (rl.rs:475-486),
log_softmax (activation.rs:36-41: g - exp(y) sum g), gather (rl.rs:134-141), categorical_kl
with the reference detached (rl.rs:327-338) and categorical_entropy (rl.rs:405-414).

Tolerance: each element of dL/dx is a sum of terms, [v == token] g_logp - pi_v (g_logp + g_kl KL
+ g_H H + (g_H - g_kl) log pi_v + g_kl log pi_ref,v), divided by T. The kernel's error is held to
1e-5 of the sum of those terms' magnitudes (the f32 relative tolerance, applied to the terms so
that cancellation inside an element does not loosen or tighten it), with a 1e-30 floor for
probabilities below f32's range. bf16 gradients must equal the f32 gradient rounded to nearest
even, bit for bit; reruns are bit-identical.
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


def term_scale(z, r, tok, glp, gkl, gh, kl, h, tau):
    """Per element, the sum of the magnitudes of the terms dL/dx_v adds up (f64)."""
    z = np.asarray(z, np.float64)
    R, V = z.shape
    with np.errstate(invalid="ignore", over="ignore"):
        lp = log_softmax(z, axis=1)
        pi = np.exp(lp)
        t = np.abs(glp)[:, None] + np.abs(gkl * kl)[:, None] + np.abs(gh * h)[:, None] + \
            np.abs(gh - gkl)[:, None] * np.abs(lp)
        if r is not None:
            t = t + np.abs(gkl)[:, None] * np.abs(log_softmax(np.asarray(r, np.float64), axis=1))
        s = np.where(pi > 0.0, pi * t, 0.0)
    if tok is not None:
        s[np.arange(R), np.asarray(tok, np.int64)] += np.abs(glp)
    return s / tau


def check_grad(name, got, want, scale):
    got = np.asarray(got, np.float64)
    err = np.abs(got - want)
    bad = ~(err <= 1e-5 * scale + 1e-30)
    worst = float(np.max(err / (scale + 1e-30)))
    assert not bad.any(), f"{name}: {int(bad.sum())} elements off; worst |Δ|/scale {worst:.2e}; " \
                          f"first at {np.argwhere(bad)[:3].tolist()}: {got[bad][:3]} vs {want[bad][:3]}"
    print(f"{name}: {got.size} elements, worst |Δ|/scale {worst:.2e}")


def upstream(rows, seed, kl=True, ent=True, lp=True):
    """Per-row upstream gradients like a PPO/GRPO loss's: advantages on logp, beta on KL, a small
    negative entropy bonus."""
    rng = np.random.default_rng(seed)
    g = {"g_lp": rng.normal(0, 1, rows).astype(np.float32) if lp else None,
         "g_kl": rng.uniform(0.01, 0.2, rows).astype(np.float32) if kl else None,
         "g_h": (-rng.uniform(0.0, 0.05, rows)).astype(np.float32) if ent else None}
    return g


def run_backward(pol, ref, tok_t, g, shape, grad_dtype):
    """Forward with the saved statistics, then the backward; returns (grad, kl, entropy) tensors."""
    lp, rlp, kl, ent, stats = nr.score_with_stats(pol, ref, tok_t, entropy=g["g_h"] is not None,
                                                  kl=g["g_kl"] is not None)
    gt = {k: (None if v is None else nr.Tensor.from_numpy(v.reshape(shape))) for k, v in g.items()}
    grad = nr.score_grad(pol, ref, tok_t if g["g_lp"] is not None else None, stats, kl=kl, entropy=ent,
                         g_logp=gt["g_lp"], g_kl=gt["g_kl"], g_entropy=gt["g_h"], grad_dtype=grad_dtype)
    return grad, kl, ent


def zeros_or(a, n):
    return np.zeros(n, np.float64) if a is None else np.asarray(a, np.float64).ravel()


def compare_to_oracle(name, z, r, tok, g, kl, ent, tau, grad_f32, grad_bf16=None):
    R = z.shape[0]
    glp, gkl, gh = (zeros_or(g[k], R) for k in ("g_lp", "g_kl", "g_h"))
    want = O.score_grad(z, tok, r, glp, gkl, gh, tau)
    scale = term_scale(z, r, tok, glp, gkl, gh, zeros_or(kl, R), zeros_or(ent, R), tau)
    check_grad(name, grad_f32, want, scale)
    if grad_bf16 is not None:
        assert np.array_equal(grad_bf16, O.bf16_from_f32(grad_f32)), f"{name}: bf16 grad is not RNE of the f32 grad"


def test_c3_backward_parity_on_a_row_slice():
    # benchmark configuration 3's rows (bf16, V 50304, the reference's logits beside the policy's):
    # d(g_lp logp + g_kl KL + g_H H)/dx in f32 and bf16.
    w = W.c3(rows=64)
    rows, V = w["rows"], w["V"]
    g = upstream(rows, 7)
    gf, kl, ent = run_backward(w["logits"], w["ref"], w["tokens"], g, (rows,), "f32")
    gb, _, _ = run_backward(w["logits"], w["ref"], w["tokens"], g, (rows,), "bf16")
    gf2, _, _ = run_backward(w["logits"], w["ref"], w["tokens"], g, (rows,), "f32")
    gfn = gf.to_numpy()
    assert gfn.tobytes() == gf2.to_numpy().tobytes(), "rerun bits"
    xf = W.bf16_to_f32(w["logits"].to_numpy())
    yf = W.bf16_to_f32(w["ref"].to_numpy())
    tok = w["tokens"].to_numpy()
    compare_to_oracle("c3 slice", xf, yf, tok, g, kl.to_numpy(), ent.to_numpy(), 1.0, gfn, gb.to_numpy())


def test_token_log_prob_gradient_is_onehot_minus_softmax():
    # tests/rl.rs:116-121 on the device: the gradient of sum(token_log_probs) is onehot - softmax.
    rng = np.random.default_rng(116)
    rows, V = 32, 3000
    x = rng.normal(0, 3, (rows, V)).astype(np.float32)
    tok = rng.integers(0, V, rows).astype(np.int32)
    xt, tt = nr.Tensor.from_numpy(x), nr.Tensor.from_numpy(tok)
    g = {"g_lp": np.ones(rows, np.float32), "g_kl": None, "g_h": None}
    grad, _, _ = run_backward(xt, None, tt, g, (rows,), "f32")
    want = -np.exp(log_softmax(x.astype(np.float64), axis=1))
    want[np.arange(rows), tok] += 1.0
    scale = term_scale(x, None, tok, g["g_lp"].astype(np.float64), np.zeros(rows), np.zeros(rows), np.zeros(rows),
                       np.zeros(rows), 1.0)
    check_grad("onehot - softmax", grad.to_numpy(), want, scale)
    assert np.all(np.abs(grad.to_numpy().sum(axis=1)) < 1e-5), "each row's gradient sums to zero"


@pytest.mark.parametrize("case", [
    # (logits dtype, mask kind, shared mask, V, temperature, objectives)
    ("f32", "u8", True, 5000, 0.8, "lp kl h"),     # one grammar mask for every row
    ("f32", "f32", False, 1001, 1.3, "lp kl h"),   # additive per-row mask, a row length not a multiple of 8
    ("bf16", "u8", False, 4099, 1.0, "kl h"),      # no token term (KL and entropy only), unaligned rows
    ("bf16", "none", False, 32768, 0.7, "lp h"),   # no reference: logp and entropy only
    ("f32", "none", False, 7, 1.0, "lp kl h"),     # a row shorter than one lane's eight elements
    ("f16", "u8", False, 4096, 0.9, "lp kl h"),    # f16 logits (aligned rows), f16 gradients too
    ("f16", "f32", True, 1003, 1.0, "lp kl h"),    # f16 logits, unaligned rows, a shared additive mask
])
def test_backward_masks_temperatures_and_objectives(case):
    dtype, mk, shared, V, tau, obj = case
    rows = 40
    rng = np.random.default_rng(V + int(10 * tau))
    x = rng.normal(0, 2, (rows, V)).astype(np.float32)
    y = (x + rng.normal(0, 0.3, (rows, V))).astype(np.float32)
    if dtype == "bf16":
        xb, yb = O.bf16_from_f32(x), O.bf16_from_f32(y)
        x, y = O.bf16_to_f32(xb), O.bf16_to_f32(yb)
        xt, yt = nr.Tensor.from_numpy(xb, "bf16"), nr.Tensor.from_numpy(yb, "bf16")
    elif dtype == "f16":
        xh, yh = x.astype(np.float16), y.astype(np.float16)
        x, y = xh.astype(np.float32), yh.astype(np.float32)
        xt, yt = nr.Tensor.from_numpy(xh.view(np.uint16), "f16"), nr.Tensor.from_numpy(yh.view(np.uint16), "f16")
    else:
        xt, yt = nr.Tensor.from_numpy(x), nr.Tensor.from_numpy(y)
    mrows = 1 if shared else rows
    keep = am = None
    mt = None
    if mk == "u8":
        keep = (rng.random((mrows, V)) < 0.6).astype(np.uint8)
        keep[:, 0] = 1
        mt = nr.Tensor.from_numpy(keep)
    elif mk == "f32":
        am = np.where(rng.random((mrows, V)) < 0.3, -1e9, rng.normal(0, 0.5, (mrows, V))).astype(np.float32)
        am[:, 0] = 0.0
        mt = nr.Tensor.from_numpy(am)
    tok = rng.integers(0, V, rows).astype(np.int32)
    if keep is not None:
        k = keep if not shared else np.repeat(keep, rows, 0)
        tok = np.where(k[np.arange(rows), tok] == 1, tok, 0).astype(np.int32)
    want_kl, want_h = "kl" in obj, "h" in obj
    g = upstream(rows, V, kl=want_kl, ent=want_h, lp="lp" in obj)
    # the fused (logits, τ, mask) triple: bf16 rows at τ 1 under a mask, widened exactly
    pol = nr.Tempered(xt, tau, mt)
    ref = nr.Tempered(yt, tau, mt) if want_kl else None
    tt = nr.Tensor.from_numpy(tok)
    gf, kl, ent = run_backward(pol, ref, tt, g, (rows,), "f32")
    gb, _, _ = run_backward(pol, ref, tt, g, (rows,), "bf16")
    z = O.tempered(x, tau, addmask=am, keep=keep)
    r = O.tempered(y, tau, addmask=am, keep=keep) if want_kl else None
    compare_to_oracle(f"{dtype} {mk} V{V} T{tau} {obj}", z, r, tok if "lp" in obj else None, g,
                      None if kl is None else kl.to_numpy(), None if ent is None else ent.to_numpy(), tau,
                      gf.to_numpy(), gb.to_numpy())
    if dtype == "f16":
        # the f16 gradient (the logits' own dtype, score_grad's default) is the f32 one rounded
        # to nearest even, as numpy's float16 cast rounds it
        gh16, _, _ = run_backward(pol, ref, tt, g, (rows,), None)
        assert gh16.dtype == "f16"
        assert np.array_equal(gh16.to_numpy(), gf.to_numpy().astype(np.float16).view(np.uint16)), \
            "f16 grad is not RNE of the f32 grad"
    if keep is not None:
        # excluded entries get no softmax term: only the token's own term could remain, and the
        # tokens are kept, so every excluded entry's gradient is exactly zero
        k = keep if not shared else np.repeat(keep, rows, 0)
        assert np.all(gf.to_numpy()[k == 0] == 0.0)


def test_backward_of_the_reference_losses_body():
    # src/nn/tests/gpu/rl.rs:38-68's inputs: ±1e4 and −∞ (in both distributions) at entries that
    # are not the token; logp, KL and entropy all weighted.
    n, V = 2 * 8 * 12, 24
    rng = np.random.default_rng(950)
    logits = rng.uniform(-6, 6, (n, V))
    refl = rng.uniform(-6, 6, (n, V))
    tokens = rng.integers(0, V, n)
    for i in range(0, n, 5):
        t = tokens[i]
        a, b = (t + 1) % V, (t + 2) % V
        logits[i, a] = refl[i, a] = -np.inf
        logits[i, b] = 1e4 if i % 2 == 0 else -1e4
    x32, r32 = logits.astype(np.float32), refl.astype(np.float32)
    xt, rt = nr.Tensor.from_numpy(x32), nr.Tensor.from_numpy(r32)
    tt = nr.Tensor.from_numpy(tokens.astype(np.int32))
    g = upstream(n, 38)
    gf, kl, ent = run_backward(xt, rt, tt, g, (n,), "f32")
    gfn = gf.to_numpy()
    compare_to_oracle("losses body", x32, r32, tokens, g, kl.to_numpy(), ent.to_numpy(), 1.0, gfn)
    assert np.all(np.isfinite(gfn))
    assert np.all(gfn[np.isneginf(x32)] == 0.0), "−∞ logits get a zero gradient"


def test_refused_rows_give_nan_gradients():
    # A row with no allowed token has no softmax: its gradient is NaN, as the op sequence's
    # log_softmax gives it; the other rows are unaffected.
    rows, V = 6, 512
    rng = np.random.default_rng(5)
    x = rng.normal(0, 1, (rows, V)).astype(np.float32)
    keep = np.ones((rows, V), np.uint8)
    keep[2] = 0
    xt, mt = nr.Tensor.from_numpy(x), nr.Tensor.from_numpy(keep)
    pol = nr.tempered_logits(xt, 1.0, mt)
    g = {"g_lp": None, "g_kl": None, "g_h": np.full(rows, -0.1, np.float32)}
    gf, _, ent = run_backward(pol, None, None, g, (rows,), "f32")
    gfn = gf.to_numpy()
    assert np.all(np.isnan(gfn[2])) and np.isnan(ent.to_numpy()[2])
    ok = np.array([0, 1, 3, 4, 5])
    compare_to_oracle("beside a refused row", x[ok], None, None, {k: (None if v is None else v[ok]) for k, v in g.items()},
                      None, ent.to_numpy()[ok], 1.0, gfn[ok])


def test_c3_full_size_backward():
    # benchmark configuration 3 at its real size (2 x bf16 [8,16,512,50304]): the f32 gradient of every
    # row sums to zero (each of the three objectives' gradients does: softmax sums to one), to
    # 1e-5 of the row's total term magnitude (the per-element scale summed over the row: with
    # sum pi |log pi| = H and sum pi |log pi_ref| = H + KL it is 2|g_lp| + |g_kl| KL + |g_H| H +
    # |g_H - g_kl| H + |g_kl| (H + KL)); rows spread over the tensor against the oracle; a second
    # run into bf16 equals the first rounded to nearest even, bit for bit, over the whole tensor.
    w = W.c3()
    rows, V = w["rows"], w["V"]
    shape = w["logits"].shape[:-1]
    g = upstream(rows, 2024)
    gf, kl, ent = run_backward(w["logits"], w["ref"], w["tokens"], g, shape, "f32")
    gb, _, _ = run_backward(w["logits"], w["ref"], w["tokens"], g, shape, "bf16")
    print(f"c3 full: backward done ({rows} rows)", flush=True)
    gfn = gf.to_numpy().reshape(rows, V)
    gbn = gb.to_numpy().reshape(rows, V)
    assert np.all(np.isfinite(gfn))
    assert np.array_equal(gbn[:64], O.bf16_from_f32(gfn[:64])), "bf16 != RNE(f32) in the first rows"
    glp, gkl, gh = (np.abs(g[k].astype(np.float64)) for k in ("g_lp", "g_kl", "g_h"))
    kln, hn = kl.to_numpy().ravel().astype(np.float64), ent.to_numpy().ravel().astype(np.float64)
    total = 2 * glp + gkl * kln + gh * hn + np.abs(g["g_h"].astype(np.float64) - g["g_kl"]) * hn + gkl * (hn + kln)
    chunk = 8192
    for r0 in range(0, rows, chunk):
        blk = gfn[r0:r0 + chunk]
        sums = blk.sum(axis=1, dtype=np.float64)
        bound = 1e-5 * total[r0:r0 + chunk]
        assert np.all(np.abs(sums) <= bound), f"row sums at {r0 + np.nonzero(np.abs(sums) > bound)[0][:4]}"
        # round to nearest even in 32-bit arithmetic (exact for finite values), to keep the pass short
        b = blk.view(np.uint32)
        rne = ((b + np.uint32(0x7FFF) + ((b >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)).astype(np.uint16)
        assert np.array_equal(gbn[r0:r0 + chunk], rne), f"bf16 != RNE(f32) in rows {r0}.."
    print("c3 full: row sums and bf16 rounding checked", flush=True)
    sel = np.array(sorted({0, 1, rows - 1} | set(np.random.default_rng(34).choice(rows, 21, replace=False).tolist())))
    xf = W.bf16_to_f32(W.download_rows(w["logits"], sel, V))
    yf = W.bf16_to_f32(W.download_rows(w["ref"], sel, V))
    tok = w["tokens"].to_numpy().ravel()[sel]
    gs = {k: v[sel] for k, v in g.items()}
    compare_to_oracle("c3 full", xf, yf, tok, gs, kl.to_numpy().ravel()[sel], ent.to_numpy().ravel()[sel], 1.0,
                      gfn[sel])
