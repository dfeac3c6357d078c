"""GPU parity tests of the policy losses (nt_hip_rl_policy_loss), the reduce_tokens backward and
kl_estimate's derivative against the CPU oracle, and of a whole PPO objective's gradient with
respect to the logits (losses, reductions and the fused scoring backward composed on the device)
against central differences of an f64 forward.

Tolerances: per-token values and derivatives within 1e-5 relative / 1e-6 absolute (the f32
tolerance); clip indicators exact; the reference's own f32 known answers (tests/rl.rs:725-750)
as it states them.
"""
import math

import numpy as np
import pytest
from scipy.special import log_softmax

import noetic_rl as nr
from oracle import oracle as O

pytestmark = pytest.mark.gpu

RED = {nr.TokenReduction.NONE: "none", nr.TokenReduction.SUM: "sum", nr.TokenReduction.TOKEN_MEAN: "token_mean",
       nr.TokenReduction.PER_SEQUENCE: "per_sequence", nr.TokenReduction.SEQUENCE_MEAN: "sequence_mean"}


@pytest.fixture(scope="module", autouse=True)
def device():
    nr.claim(0)
    yield


def close_f32(ours, want):
    ours, want = np.asarray(ours, np.float64), np.asarray(want, np.float64)
    same = (ours == want) | (np.isnan(ours) & np.isnan(want))
    return same | (np.abs(ours - want) <= 1e-6 + 1e-5 * np.abs(want))


def assert_close(name, ours, want):
    ok = close_f32(ours, want)
    assert ok.all(), f"{name}: {int((~ok).sum())} off, first {np.argwhere(~ok)[:3].ravel().tolist()}: " \
                     f"{np.asarray(ours).ravel()[~ok.ravel()][:3]} vs {np.asarray(want).ravel()[~ok.ravel()][:3]}"


def t(a, shape=None):
    a = np.ascontiguousarray(a, dtype=np.float32)
    return nr.Tensor.from_numpy(a.reshape(shape) if shape is not None else a)


def ppo_data(shape, seed, dual=False):
    """logp, old (offsets away from every clip edge: ratios 4.48, 1.65, 1.105, 0.95, 0.67, as
    tests/rl.rs:228-235 and 678-684 build them), advantages of both signs, an 80% mask with one
    empty sequence; all f32."""
    n = int(np.prod(shape))
    rng = np.random.default_rng(seed)
    lp = (-rng.uniform(0.05, 6.0, n)).astype(np.float32)
    offs = np.array([-1.5, -0.5, -0.1, 0.05, 0.4] if dual else [-0.5, -0.1, 0.05, 0.4])
    i = np.arange(n)
    old = (lp.astype(np.float64) + offs[(i * 7 + i // 3) % len(offs)]).astype(np.float32)
    adv = rng.uniform(-2.0, 2.0, n)
    adv = np.where(np.abs(adv) < 0.1, -0.5, adv).astype(np.float32)
    mask = (rng.random(n) < 0.8).astype(np.float32)
    S, B, T = shape
    mask[T:2 * T] = 0.0  # sequence (0, 1) has no scored token
    return lp, old, adv, mask


@pytest.mark.parametrize("shape", [(8, 16, 512), (4, 32, 1024)])
@pytest.mark.parametrize("variant", ["pg", "pg_per_seq", "ppo", "ppo_asym", "ppo_dual", "ppo_open"])
def test_policy_losses_per_token_against_the_oracle(shape, variant):
    # benchmark configurations 3 and 5's [S, B, T]; every clip setting of tests/rl.rs:251-317, 678-717
    S, B, T = shape
    clip = {"ppo": nr.Clip.symmetric(0.2), "ppo_asym": nr.Clip.new(0.2, 0.28),
            "ppo_dual": nr.Clip.symmetric(0.2).with_dual(3.0),
            "ppo_open": nr.Clip.symmetric(0.2).with_log_ratio_clamp(None)}.get(variant)
    lp, old, adv, mask = ppo_data(shape, 840 + len(variant), dual=variant == "ppo_dual")
    per_seq = variant == "pg_per_seq"
    w = adv.reshape(shape)[:, :, 0].copy() if per_seq else adv
    lpt, oldt, mt = t(lp, shape), t(old, shape), t(mask, shape)
    wt = t(w, (S, B) if per_seq else shape)
    kind = nr.NT_LOSS_PG if clip is None else nr.NT_LOSS_PPO
    loss, dloss, hit = nr._policy_loss(kind, variant, lpt, None if clip is None else oldt, wt, mt, clip)
    okw = dict(low=clip.low, high=clip.high, dual=clip.dual, clamp=clip.log_ratio_clamp) if clip else {}
    want_loss, want_d, want_hit = O.policy_loss("pg" if clip is None else "ppo", lp, old, w, mask, T, per_seq=per_seq,
                                                **okw)
    assert_close(f"{variant} loss", loss.to_numpy().ravel(), want_loss)
    assert_close(f"{variant} dloss", dloss.to_numpy().ravel(), want_d)
    assert np.array_equal(hit.to_numpy().ravel(), want_hit), f"{variant} clip indicator"
    if clip is not None:
        assert 0 < want_hit.sum() < mask.sum(), "the case clips some tokens"
        frac = nr.clip_fraction(lpt, oldt, wt, mt, clip).to_numpy()
        assert_close("clip fraction", frac, O.reduce_tokens(want_hit, mask, shape, "token_mean"))
    for red in nr.TokenReduction:
        want = O.reduce_tokens(want_loss, mask, shape, RED[red])
        got = (nr.policy_gradient_loss(lpt, wt, mt, red) if clip is None
               else nr.clipped_policy_loss(lpt, oldt, wt, mt, clip, red)).to_numpy().ravel()
        assert_close(f"{variant} {red.name}", got, want)


@pytest.mark.parametrize("reduction", list(nr.TokenReduction))
def test_reductions_forward_and_backward_against_the_oracle(reduction):
    S, B, T = 8, 16, 512
    rng = np.random.default_rng(int(reduction) + 5)
    mask = (rng.random(S * B * T) < 0.7).astype(np.float32)
    mask[3 * T:4 * T] = 0.0                  # an empty sequence
    mask[5 * B * T:6 * B * T] = 0.0          # an empty seed
    per = np.where(mask != 0, rng.normal(0, 1, S * B * T), 0.0).astype(np.float32)
    red = RED[reduction]
    want = O.reduce_tokens(per, mask, (S, B, T), red)
    got = nr._reduce(t(per, (S, B, T)), t(mask, (S, B, T)), reduction).to_numpy().ravel()
    assert_close(f"reduce {red}", got, want)
    up = rng.normal(0, 1, want.size).astype(np.float32)
    local = rng.normal(0, 1, S * B * T).astype(np.float32)
    ups = nr._reduced_shape((S, B, T), reduction)
    g = nr.reduce_tokens_backward(t(mask, (S, B, T)), (S, B, T), reduction, t(up, ups), -0.7, t(local, (S, B, T)))
    assert_close(f"reduce {red} backward", g.to_numpy().ravel(),
                 O.reduce_tokens_backward(mask, (S, B, T), red, up, -0.7, local))
    g1 = nr.reduce_tokens_backward(None, (S, B, T), reduction).to_numpy().ravel()
    assert_close(f"reduce {red} backward, no mask", g1, O.reduce_tokens_backward(None, (S, B, T), red))


def test_overflow_guards_on_the_device():
    # tests/rl.rs:725-750, in f32 as the reference states it: A = -1 with a log-ratio of 100
    lp, old, adv = t([-0.5, -1.0], (1, 1, 2)), t([-100.5, -1.0], (1, 1, 2)), t([-1.0, 1.0], (1, 1, 2))

    def run(clip):
        loss, dloss, _ = nr._policy_loss(nr.NT_LOSS_PPO, "clipped_policy_loss", lp, old, adv, None, clip)
        return loss.to_numpy().ravel(), dloss.to_numpy().ravel()

    open_, _ = run(nr.Clip.symmetric(0.2).with_log_ratio_clamp(None))
    assert open_[0] == np.inf
    clamped, g = run(nr.Clip.symmetric(0.2))
    want = float(np.exp(np.float32(20.0)))
    assert abs(clamped[0] - want) <= 1e-7 * want and g[0] == 0.0
    dual, g = run(nr.Clip.symmetric(0.2).with_dual(3.0))
    assert (dual[0], g[0]) == (3.0, 0.0)
    dual, g = run(nr.Clip.symmetric(0.2).with_dual(3.0).with_log_ratio_clamp(None))
    assert dual[0] == 3.0 and np.isnan(g[0]), "the unselected branch's 0 times an overflowed ratio's derivative"
    assert clamped[1] == -1.0 and g[1] == -1.0, "an on-policy token: -A r with r = 1"
    assert nr.clip_fraction(lp, old, adv, None, nr.Clip.symmetric(0.2)).to_numpy().tolist() == [0.5]


def test_masking_edges_all_masked_and_one_token():
    # tests/rl.rs:507-545: every position masked gives 0 and exactly zero gradient; one scored
    # token gives that token's loss under TokenMean, SequenceMean and Sum
    shape = (2, 3, 4)
    lp, old, adv, _ = ppo_data(shape, 910)
    lpt, oldt, at = t(lp, shape), t(old, shape), t(adv, shape)
    none = t(np.zeros(24), shape)
    one_np = np.zeros(24, np.float32)
    one_np[22] = 1.0
    one = t(one_np, shape)
    clip = nr.Clip.symmetric(0.2)
    for name, fwd, bwd in [
        ("PG", lambda m, r: nr.policy_gradient_loss(lpt, at, m, r),
         lambda m, r: nr.policy_gradient_loss_backward(lpt, at, m, r)),
        ("PPO", lambda m, r: nr.clipped_policy_loss(lpt, oldt, at, m, clip, r),
         lambda m, r: nr.clipped_policy_loss_backward(lpt, oldt, at, m, clip, r)),
        ("k3", lambda m, r: nr.kl_estimate(lpt, oldt, nr.KlEstimator.K3, nr.KL_DELTA_CLAMP, m, r),
         lambda m, r: nr.kl_estimate_backward(lpt, oldt, nr.KlEstimator.K3, nr.KL_DELTA_CLAMP, m, r)),
    ]:
        for r in nr.TokenReduction:
            assert np.all(fwd(none, r).to_numpy() == 0.0), (name, r)
            assert np.all(bwd(none, r).to_numpy() == 0.0), (name, r, "gradient")
        per = fwd(one, nr.TokenReduction.NONE).to_numpy().ravel()
        assert np.all(np.delete(per, 22) == 0.0)
        for r in (nr.TokenReduction.TOKEN_MEAN, nr.TokenReduction.SEQUENCE_MEAN, nr.TokenReduction.SUM):
            assert fwd(one, r).to_numpy().tolist() == [0.0, float(per[22])], (name, r)


def test_garbage_old_logp_at_masked_positions():
    # tests/rl.rs:319-333: old values of ±1e4 at masked positions leave loss and gradient finite
    # and unchanged, to the bit
    shape = (4, 8, 32)
    lp, old, adv, mask = ppo_data(shape, 860)
    garbage = np.where(mask == 0, np.where(np.arange(mask.size) % 2 == 0, -1e4, 1e4), old).astype(np.float32)
    clip = nr.Clip.symmetric(0.2)
    outs = []
    for o in (old, garbage):
        args = (t(lp, shape), t(o, shape), t(adv, shape), t(mask, shape), clip)
        outs.append((nr.clipped_policy_loss(*args).to_numpy(), nr.clipped_policy_loss_backward(*args).to_numpy()))
    assert all(np.all(np.isfinite(x)) for x in outs[1])
    assert outs[0][0].tobytes() == outs[1][0].tobytes() and outs[0][1].tobytes() == outs[1][1].tobytes()


@pytest.mark.parametrize("est", [nr.KlEstimator.K1, nr.KlEstimator.K2, nr.KlEstimator.K3])
def test_kl_estimate_backward_against_the_oracle(est):
    shape = (8, 16, 512)
    n = int(np.prod(shape))
    rng = np.random.default_rng(int(est))
    lp = (-rng.uniform(0.1, 8, n)).astype(np.float32)
    lr = (lp + rng.normal(0, 2, n)).astype(np.float32)
    lr[::97] = lp[::97] + 25.0  # beyond the clamp
    mask = (rng.random(n) < 0.8).astype(np.float32)
    for clamp in (None, nr.KL_DELTA_CLAMP):
        for red in (nr.TokenReduction.NONE, nr.TokenReduction.TOKEN_MEAN, nr.TokenReduction.SEQUENCE_MEAN):
            got = nr.kl_estimate_backward(t(lp, shape), t(lr, shape), est, clamp, t(mask, shape), red,
                                          scale=0.5).to_numpy().ravel()
            local = O.kl_estimate_grad(lp, lr, int(est), clamp, mask)
            want = O.reduce_tokens_backward(mask, shape, RED[red], None, 0.5, local)
            assert_close(f"k{int(est)} clamp {clamp} {red.name}", got, want)


def test_ppo_objective_gradient_through_the_logits_matches_finite_differences():
    # L = clipped_policy_loss + 0.02 k3 (clamped) + 0.05 KL - 0.01 H, each TokenMean over a masked
    # [1, 2, 3] batch of V = 11 logits; d L / d logits from the device pieces (score with saved
    # statistics, loss derivatives, reduce_tokens backward, the fused scoring backward) against
    # central differences of an f64 forward.
    S, B, T, V = 1, 2, 3, 11
    rng = np.random.default_rng(2024)
    x = rng.normal(0, 1.5, (S, B, T, V)).astype(np.float32)
    y = (x + rng.normal(0, 0.4, x.shape)).astype(np.float32)
    tok = rng.integers(0, V, (S, B, T)).astype(np.int32)
    mask = np.array([1, 1, 0, 1, 0, 1], np.float32).reshape(S, B, T)
    lp64 = np.take_along_axis(log_softmax(x.astype(np.float64), -1), tok[..., None].astype(np.int64), -1)[..., 0]
    offs = np.array([-0.5, -0.1, 0.05, 0.4, -0.1, 0.05]).reshape(S, B, T)
    old = (lp64 + offs).astype(np.float32)
    adv = np.array([1.3, -0.7, 0.4, -1.1, 0.9, -0.2], np.float32).reshape(S, B, T)
    clip = nr.Clip.symmetric(0.2)
    beta_k3, beta_kl, eta = 0.02, 0.05, 0.01
    TM = nr.TokenReduction.TOKEN_MEAN

    def objective(xx):  # f64 forward of the same op sequence
        lpx = log_softmax(xx, -1)
        lpy = log_softmax(y.astype(np.float64), -1)
        lp = np.take_along_axis(lpx, tok[..., None].astype(np.int64), -1)[..., 0].ravel()
        lr = np.take_along_axis(lpy, tok[..., None].astype(np.int64), -1)[..., 0].ravel()
        ppo, _, _ = O.policy_loss("ppo", lp, old, adv, mask, T, low=0.2, high=0.2, clamp=20.0)
        k3 = O.kl_estimate(lp, lr, 3, 20.0, mask)
        px = np.exp(lpx)
        kl = (px * (lpx - lpy)).sum(-1).ravel()
        h = -(px * lpx).sum(-1).ravel()
        m = mask.ravel()
        red = lambda v: O.reduce_tokens(np.where(m != 0, v, 0.0), m, (S, B, T), "token_mean")[0]
        return red(ppo) + beta_k3 * red(k3) + beta_kl * red(kl) - eta * red(h)

    xt, yt, tt, mt = nr.Tensor.from_numpy(x), nr.Tensor.from_numpy(y), nr.Tensor.from_numpy(tok), t(mask)
    lp, rlp, kl, ent, stats = nr.score_with_stats(xt, yt, tt)
    g_lp = (nr.clipped_policy_loss_backward(lp, t(old), t(adv), mt, clip, TM).to_numpy() +
            nr.kl_estimate_backward(lp, rlp, nr.KlEstimator.K3, nr.KL_DELTA_CLAMP, mt, TM, scale=beta_k3).to_numpy())
    g_kl = nr.reduce_tokens_backward(mt, (S, B, T), TM, scale=beta_kl)
    g_h = nr.reduce_tokens_backward(mt, (S, B, T), TM, scale=-eta)
    grad = nr.score_grad(xt, yt, tt, stats, kl=kl, entropy=ent, g_logp=t(g_lp), g_kl=g_kl, g_entropy=g_h,
                         grad_dtype="f32").to_numpy()
    h = 1e-5
    x64 = x.astype(np.float64)
    fd = np.zeros_like(x64)
    for idx in np.ndindex(x.shape):
        e = np.zeros_like(x64)
        e[idx] = h
        fd[idx] = (objective(x64 + e) - objective(x64 - e)) / (2 * h)
    err = np.abs(grad - fd)
    assert np.all(err <= 1e-6 + 1e-4 * np.abs(fd)), f"worst {err.max():.2e} at {np.unravel_index(err.argmax(), x.shape)}"
    assert np.all(grad[mask == 0] == 0.0), "masked positions get no gradient"
    print(f"PPO objective gradient: {x.size} logits, worst |Δ| {err.max():.2e}, max |grad| {np.abs(fd).max():.3e}")


def test_group_advantages_on_the_device():
    # tests/rl.rs:551-575 and 645-653 on the device: hand values, equal rewards give exact zeros
    # whatever the normalisation, groups of one; then many groups against the oracle to the bit
    # (f64 per group, rounded to f32)
    r = np.array([1.0, 0.0, 0.0, 1.0, 2.0, 2.0, 2.0, 2.0, 0.0, 0.0, 0.0, 3.0], np.float32)
    rt = t(r, (3, 4))
    s3 = 0.5 / math.sqrt(1.0 / 3.0)
    got = nr.group_advantages_tensor(rt, "std", 0.0, True).to_numpy().ravel()
    assert np.array_equal(got, np.float32([s3, -s3, -s3, s3, 0, 0, 0, 0, -0.5, -0.5, -0.5, 1.5]))
    p3 = math.sqrt(1.6875)
    got = nr.group_advantages_tensor(rt, "std", 0.0, False).to_numpy().ravel()
    assert np.array_equal(got, np.float32([1, -1, -1, 1, 0, 0, 0, 0, -0.75 / p3, -0.75 / p3, -0.75 / p3, 2.25 / p3]))
    got = nr.group_advantages_tensor(rt, "mean").to_numpy().ravel()
    assert got.tolist() == [0.5, -0.5, -0.5, 0.5, 0.0, 0.0, 0.0, 0.0, -0.75, -0.75, -0.75, 2.25]
    got = nr.group_advantages_tensor(rt, "std", 1e-2, True).to_numpy().ravel()
    assert np.array_equal(got[8:], np.float32([-0.75 / 1.51, -0.75 / 1.51, -0.75 / 1.51, 2.25 / 1.51]))
    assert nr.group_advantages_tensor(t([3.0, -1.0], (2, 1)), "std", 1e-6, False).to_numpy().ravel().tolist() == [0, 0]
    eq = t([0.1, 0.1, 0.1, 1.0, 0.0, 0.0], (2, 3))
    for norm, unb in (("std", True), ("std", False), ("mean", True)):
        a = nr.group_advantages_tensor(eq, norm, 0.0, unb).to_numpy().ravel()
        assert a[:3].tolist() == [0.0, 0.0, 0.0] and a[3] > 0 and a[4] < 0 and a[4] == a[5], (norm, unb)
    with pytest.raises(nr.HipError, match="at least 2"):
        nr.group_advantages_tensor(t([1.0, 2.0], (2, 1)), "std", 1e-6, True)
    rng = np.random.default_rng(465)
    for G, n in ((65536, 8), (1000, 1000), (4096, 2)):
        rw = rng.normal(0, 1, (G, n)).astype(np.float32)
        rw[::7] = rw[::7, :1]                       # equal-reward groups
        rw[1::5] = np.round(rw[1::5])               # binary-ish verifier rewards
        for norm, eps, unb in (("std", 1e-6, True), ("std", 0.0, False), ("mean", 0.0, True)):
            got = nr.group_advantages_tensor(t(rw, (G, n)), norm, eps, unb).to_numpy().ravel()
            want = O.group_advantages(rw.astype(np.float64).ravel(), n, norm, eps, unb).astype(np.float32)
            assert np.array_equal(got, want), (G, n, norm, int((got != want).sum()))
    # 16-bit rewards are read exactly widened, and the result is f32, as from_f64s stores a
    # 16-bit dtype (float.rs:256-260)
    rw = rng.normal(0, 1, (512, 8)).astype(np.float32)
    rb, rh = O.bf16_from_f32(rw), rw.astype(np.float16)
    for raw, dt, wide in ((rb, "bf16", O.bf16_to_f32(rb)), (rh.view(np.uint16), "f16", rh.astype(np.float32))):
        adv = nr.group_advantages_tensor(nr.Tensor.from_numpy(raw, dt), "std", 1e-6, True)
        assert adv.dtype == "f32"
        want = O.group_advantages(wide.astype(np.float64).ravel(), 8, "std", 1e-6, True).astype(np.float32)
        assert np.array_equal(adv.to_numpy().ravel(), want), dt


@pytest.mark.parametrize("dt", ["bf16", "f16"])
def test_16_bit_per_token_operands_are_widened(dt):
    """16-bit log-probabilities, weights and masks (one dtype where the reference's binary ops meet
    them; PPO's advantages f32, since its ratio is f32) give the widened f32 call's values bit for
    bit: the reference computes 16-bit storage in f32 (fdisp, float.rs:43-58)."""
    rng = np.random.default_rng(17)
    sh = (2, 4, 16)
    lp = -np.abs(rng.normal(1.0, 1.0, sh)).astype(np.float32)
    old = (lp + rng.normal(0, 0.3, sh)).astype(np.float32)
    w = rng.normal(0, 1, sh).astype(np.float32)
    m = (rng.random(sh) < 0.8).astype(np.float32)

    def pair(x):
        if dt == "bf16":
            r = O.bf16_from_f32(x)
            return nr.Tensor.from_numpy(r, dt), nr.Tensor.from_numpy(O.bf16_to_f32(r))
        r = x.astype(np.float16)
        return nr.Tensor.from_numpy(r.view(np.uint16), dt), nr.Tensor.from_numpy(r.astype(np.float32))

    (lp16, lp32), (old16, old32), (w16, w32), (m16, m32) = pair(lp), pair(old), pair(w), pair(m)
    a32 = w32  # PPO's advantages stay f32 (r · A, with r f32)
    clip = nr.Clip.symmetric(0.2).with_dual(3.0)
    same = lambda x, y, what: (x.dtype == "f32" and x.to_numpy().tobytes() == y.to_numpy().tobytes()) or \
        pytest.fail(f"{dt} {what}")
    for red in (nr.TokenReduction.NONE, nr.TokenReduction.TOKEN_MEAN, nr.TokenReduction.SEQUENCE_MEAN):
        same(nr.policy_gradient_loss(lp16, w16, m16, red), nr.policy_gradient_loss(lp32, w32, m32, red), f"pg {red}")
        same(nr.clipped_policy_loss(lp16, old16, a32, m16, clip, red),
             nr.clipped_policy_loss(lp32, old32, a32, m32, clip, red), f"ppo {red}")
        for est in (nr.KlEstimator.K1, nr.KlEstimator.K3):
            same(nr.kl_estimate(lp16, old16, est, 20.0, m16, red), nr.kl_estimate(lp32, old32, est, 20.0, m32, red),
                 f"kl {est} {red}")
            same(nr.kl_estimate_backward(lp16, old16, est, None, m16, red),
                 nr.kl_estimate_backward(lp32, old32, est, None, m32, red), f"kl backward {est} {red}")
        same(nr.policy_gradient_loss_backward(lp16, w16, m16, red),
             nr.policy_gradient_loss_backward(lp32, w32, m32, red), f"pg backward {red}")
    same(nr.clip_fraction(lp16, old16, w16, m16, clip), nr.clip_fraction(lp32, old32, w32, m32, clip), "clip_fraction")
    assert nr.check_scored_finite("t", lp16, m16) is None


def test_check_scored_finite_and_the_debug_refusal():
    # tests/rl.rs:836-855: a -inf at a scored position is named; at a masked position it passes
    lp = t([-1.0, -np.inf, -2.0], (1, 1, 3))
    e = nr.check_scored_finite("test", lp, None)
    assert e is not None and "position 1" in e and "not finite" in e
    assert nr.check_scored_finite("test", lp, t([1.0, 0.0, 1.0], (1, 1, 3))) is None
    assert nr.check_scored_finite("test", t([-1.0, -3.0, -2.0], (1, 1, 3)), None) is None
    saved = nr.DEBUG_CHECKS
    try:
        nr.DEBUG_CHECKS = True
        with pytest.raises(AssertionError, match="not finite"):
            nr.policy_gradient_loss(t([-1.0, -np.inf], (1, 1, 2)), t([1.0], (1, 1)), None, nr.TokenReduction.SUM)
    finally:
        nr.DEBUG_CHECKS = saved
