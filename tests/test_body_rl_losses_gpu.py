"""The reference's device body test for nn::rl (src/nn/tests/gpu/rl.rs:1-140), on this build: each of
its eleven losses' value and logit gradient (the gradient of sum(loss * up) for a random upstream
up) with ±1e4 and −∞ logits and masked positions, against the CPU oracle; masked positions with
exactly zero gradient; byte-identical run to run. The reference compares with Cpu(Reference)
under |Δ|/(1+|ref|): values within 1e-5, gradients within 1e-4; the same bounds hold here against
the f64 oracle. Where a loss branches on the log-probabilities (PPO's selects, the k3 clamp), the
oracle takes the device's log-probabilities as its input, as the reference's Cpu(Reference) and
device runs start from the same f32 values; the log-probabilities themselves are the first case.

Data (gpu/rl.rs:38-68): [2, 8, 12] positions of V = 24 logits in [-6, 6]; at every fifth
position −∞ in both distributions after the token and ±1e4 two after it; a 75% mask with
sequence 3 masked; old log-probabilities in [-8, -0.5]; advantages in [-2, 2]; reference
log-probabilities of the tokens the policy's plus δ in [-1.5, 1.5]. The values come from numpy's
generator rather than the reference's ChaCha8 streams: parity is against the oracle on the same
bytes, so only the construction matters.
"""
import numpy as np
import pytest
from scipy.special import log_softmax

import noetic_rl as nr
from oracle import oracle as O

pytestmark = pytest.mark.gpu

SH = (2, 8, 12)
V = 24
TR = nr.TokenReduction


@pytest.fixture(scope="module", autouse=True)
def device():
    nr.claim(0)
    yield


def rel(a, b):
    a, b = np.asarray(a, np.float64).ravel(), np.asarray(b, np.float64).ravel()
    d = np.where(a == b, 0.0, np.abs(a - b) / (1.0 + np.abs(b)))
    return float(d.max()) if d.size else 0.0


def data():
    rng = np.random.default_rng(950)
    n = int(np.prod(SH))
    logits = rng.uniform(-6, 6, (n, V))
    refl = rng.uniform(-6, 6, (n, V))
    tokens = rng.integers(0, V, n)
    for i in range(0, n, 5):
        t = tokens[i]
        a, b = (t + 1) % V, (t + 2) % V
        logits[i, a] = refl[i, a] = -np.inf
        logits[i, b] = 1e4 if i % 2 == 0 else -1e4
    mask = (rng.random(n) < 0.75).astype(np.float64)
    mask[3 * SH[2]:4 * SH[2]] = 0.0
    old = rng.uniform(-8, -0.5, n)
    adv = rng.uniform(-2, 2, n)
    lsm = log_softmax(logits, axis=1)
    lr = lsm[np.arange(n), tokens] + rng.uniform(-1.5, 1.5, n)
    f32 = lambda a: np.asarray(a, np.float32)
    return {"x": f32(logits), "r": f32(refl), "tok": tokens.astype(np.int32), "m": f32(mask), "old": f32(old),
            "adv": f32(adv), "lr": f32(lr)}


def t(a, shape):
    return nr.Tensor.from_numpy(np.ascontiguousarray(np.asarray(a, np.float32).reshape(shape)))


def run(d):
    """Each case's (value, logit gradient) on the device, and the oracle's."""
    lsh = SH + (V,)
    xt, rt, mt = t(d["x"], lsh), t(d["r"], lsh), t(d["m"], SH)
    tok = nr.Tensor.from_numpy(d["tok"].reshape(SH))
    old, adv, lr = t(d["old"], SH), t(d["adv"], SH), t(d["lr"], SH)
    advs = t(d["adv"][:SH[0] * SH[1]], SH[:2])
    vm = np.array([-1e9 if k % 5 == 4 else 0.0 for k in range(V)], np.float32)
    vmt = t(vm, (1, 1, 1, V))
    m = d["m"].astype(np.float64)
    n = m.size
    up_rng = np.random.default_rng(9)
    pol, ref = xt, rt
    lp, rlp, kl, ent, stats = nr.score_with_stats(pol, ref, tok)
    lpn = lp.to_numpy().astype(np.float64).ravel()
    z, r = d["x"], d["r"]
    clip_a = nr.Clip.new(0.2, 0.28)
    clip_d = nr.Clip.symmetric(0.2).with_dual(3.0).with_log_ratio_clamp(None)
    out = []

    def grad(g_lp=None, g_kl=None, g_h=None, p=pol, q=ref, st=stats, k=kl, e=ent, tokens=tok):
        return nr.score_grad(p, q, tokens, st, kl=k, entropy=e, g_logp=g_lp, g_kl=g_kl, g_entropy=g_h,
                             grad_dtype="f32").to_numpy().reshape(n, V)

    def want_grad(zz, rr, g_lp=None, g_kl=None, g_h=None, tau=1.0):
        return O.score_grad(zz, d["tok"] if g_lp is not None else None, rr, g_lp, g_kl, g_h, tau)

    def up_for(value):
        return up_rng.uniform(-1, 1, value.shape).astype(np.float32)

    ob = lambda red, up, local: O.reduce_tokens_backward(m, SH, red, up, 1.0, local)
    RED = {TR.NONE: "none", TR.SUM: "sum", TR.TOKEN_MEAN: "token_mean", TR.PER_SEQUENCE: "per_sequence",
           TR.SEQUENCE_MEAN: "sequence_mean"}

    # 1. token_log_probs, masked positions filled with 0
    val = np.where(m != 0, lpn, 0.0)
    want_val = np.where(m != 0, O.token_logp(z, d["tok"]), 0.0)
    up = up_for(val)
    g = grad(g_lp=nr.reduce_tokens_backward(mt, SH, TR.NONE, t(up, SH)))
    out.append(("token_log_probs", val, want_val, g, want_grad(z, None, g_lp=np.where(m != 0, up, 0.0))))

    # 2-3, 4, 9: the policy losses
    for name, kind, w, wshape, clip, red in [
            ("pg token-mean", "pg", adv, SH, None, TR.TOKEN_MEAN),
            ("pg per-sequence weights, none", "pg", advs, SH[:2], None, TR.NONE),
            ("ppo sum", "ppo", adv, SH, clip_a, TR.SUM),
            ("ppo dual clip, no log-ratio clamp, token-mean", "ppo", adv, SH, clip_d, TR.TOKEN_MEAN)]:
        if kind == "pg":
            value = nr.policy_gradient_loss(lp, w, mt, red).to_numpy()
        else:
            value = nr.clipped_policy_loss(lp, old, w, mt, clip, red).to_numpy()
        up = up_for(value)
        ups = t(up, value.shape)
        if kind == "pg":
            g_lp = nr.policy_gradient_loss_backward(lp, w, mt, red, upstream=ups)
        else:
            g_lp = nr.clipped_policy_loss_backward(lp, old, w, mt, clip, red, upstream=ups)
        ckw = {} if clip is None else dict(low=clip.low, high=clip.high, dual=clip.dual, clamp=clip.log_ratio_clamp)
        per, dper, _ = O.policy_loss(kind, lpn, d["old"], w.to_numpy(), m, SH[2], per_seq=len(wshape) == 2, **ckw)
        want_val = O.reduce_tokens(per, m, SH, RED[red])
        out.append((name, value, want_val, grad(g_lp=g_lp), want_grad(z, None, g_lp=ob(RED[red], up, dper))))

    # 5. exact KL, sequence-mean
    value = nr.categorical_kl(xt, rt, mt, TR.SEQUENCE_MEAN).to_numpy()
    up = up_for(value)
    g_kl = nr.reduce_tokens_backward(mt, SH, TR.SEQUENCE_MEAN, t(up, value.shape))
    want_val = O.reduce_tokens(np.where(m != 0, O.kl(z, r), 0.0), m, SH, "sequence_mean")
    out.append(("kl sequence-mean", value, want_val, grad(g_kl=g_kl), want_grad(z, r, g_kl=ob("sequence_mean", up, None))))

    # 6-8. the estimators, per sequence
    for est, clamp in ((nr.KlEstimator.K1, None), (nr.KlEstimator.K2, None), (nr.KlEstimator.K3, nr.KL_DELTA_CLAMP)):
        value = nr.kl_estimate(lp, lr, est, clamp, mt, TR.PER_SEQUENCE).to_numpy()
        up = up_for(value)
        g_lp = nr.kl_estimate_backward(lp, lr, est, clamp, mt, TR.PER_SEQUENCE, upstream=t(up, value.shape))
        lrn = d["lr"].astype(np.float64)
        want_val = O.reduce_tokens(O.kl_estimate(lpn, lrn, int(est), clamp, m), m, SH, "per_sequence")
        local = O.kl_estimate_grad(lpn, lrn, int(est), clamp, m)
        out.append((f"k{int(est)} per-sequence", value, want_val, grad(g_lp=g_lp),
                    want_grad(z, None, g_lp=ob("per_sequence", up, local))))

    # 10. reference KL at τ 0.7 under a −1e9 vocabulary mask, token-mean
    value = nr.reference_kl(xt, rt, 0.7, vmt, mt, TR.TOKEN_MEAN).to_numpy()
    up = up_for(value)
    tp, tq = nr.tempered_logits(xt, 0.7, vmt), nr.tempered_logits(rt, 0.7, vmt)
    _, _, kl7, _, st7 = nr.score_with_stats(tp, tq, None, entropy=False, kl=True)
    g_kl = nr.reduce_tokens_backward(mt, SH, TR.TOKEN_MEAN, t(up, value.shape))
    z7, r7 = O.tempered(z, 0.7, addmask=vm), O.tempered(r, 0.7, addmask=vm)
    want_val = O.reduce_tokens(np.where(m != 0, O.kl(z7, r7), 0.0), m, SH, "token_mean")
    out.append(("reference kl τ 0.7 with a −1e9 vocabulary mask, token-mean", value, want_val,
                grad(g_kl=g_kl, p=tp, q=tq, st=st7, k=kl7, e=None, tokens=None),
                want_grad(z7, r7, g_kl=ob("token_mean", up, None), tau=0.7)))

    # 11. entropy, token-mean
    value = nr.categorical_entropy(xt, mt, TR.TOKEN_MEAN).to_numpy()
    up = up_for(value)
    g_h = nr.reduce_tokens_backward(mt, SH, TR.TOKEN_MEAN, t(up, value.shape))
    want_val = O.reduce_tokens(np.where(m != 0, O.entropy(z), 0.0), m, SH, "token_mean")
    out.append(("entropy token-mean", value, want_val, grad(g_h=g_h), want_grad(z, None, g_h=ob("token_mean", up, None))))
    return out


def test_body_rl_losses_on_the_device():
    d = data()
    first = run(d)
    assert len(first) == 11
    masked = d["m"] == 0
    worst = [0.0, 0.0]
    for name, value, want_value, g, want_g in first:
        assert np.all(np.isfinite(value)) and np.all(np.isfinite(g)), f"{name}: not finite"
        ev, eg = rel(value, want_value), rel(g, want_g)
        assert ev <= 1e-5, f"{name} value: {ev:.2e} from the oracle"
        assert eg <= 1e-4, f"{name} gradient: {eg:.2e} from the oracle"
        assert np.all(g[masked] == 0.0), f"{name}: a masked position has a gradient"
        worst = [max(worst[0], ev), max(worst[1], eg)]
    again = run(d)
    for (name, v1, _, g1, _), (_, v2, _, g2, _) in zip(first, again):
        assert np.asarray(v1).tobytes() == np.asarray(v2).tobytes() and g1.tobytes() == g2.tobytes(), f"{name}: rerun"
    print(f"rl losses: values within {worst[0]:.1e} and gradients within {worst[1]:.1e} of the oracle "
          f"(±1e4 and −∞ logits, masked positions zero), byte-identical run to run")
