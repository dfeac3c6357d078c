"""CPU tests that pin the oracle (oracle/oracle.c) before it is trusted as the checker.

Each oracle function is checked against something other than its own formula: the reference's
known-answer tests (src/hash.rs:33-36, src/nn/tests/rl.rs), textbook vectors (RFC 8439),
independent library routines (hashlib, scipy, numpy's IEEE f32 arithmetic), closed forms,
invariants, and brute force on tiny inputs.
"""
import hashlib
import json
import math
import os
import struct

import numpy as np
import pytest
from scipy.special import log_softmax

from oracle import oracle as O

HERE = os.path.dirname(os.path.abspath(__file__))
NINF = float("-inf")


def f32(x):
    return np.asarray(x, dtype=np.float32)


def assert_close(what, ours, theirs, tol):
    """|a - b| <= tol * (1 + |b|) (src/nn/tests/mod.rs:104-109)."""
    ours, theirs = np.asarray(ours, dtype=np.float64), np.asarray(theirs, dtype=np.float64)
    assert ours.shape == theirs.shape, what
    bad = ~(np.abs(ours - theirs) <= tol * (1.0 + np.abs(theirs)))
    both_inf = np.isinf(ours) & np.isinf(theirs) & (np.sign(ours) == np.sign(theirs))
    bad &= ~both_inf
    assert not bad.any(), f"{what}: {ours[bad][:4]} vs {theirs[bad][:4]}"


# ------------------------------------------------------------------------ SHA-256, ChaCha20

def test_sha256_known_vectors():
    # src/hash.rs:33-36
    assert O.sha256(b"").hex() == "e3b0c44298fc1c149afbf4c8996fb92427ae41e4649b934ca495991b7852b855"
    assert O.sha256(b"abc").hex() == "ba7816bf8f01cfea414140de5dae2223b00361a396177a9cb410ff61f20015ad"
    rng = np.random.default_rng(1)
    for n in (1, 55, 56, 63, 64, 65, 119, 120, 128, 1000):
        data = rng.integers(0, 256, n, dtype=np.uint8).tobytes()
        assert O.sha256(data) == hashlib.sha256(data).digest(), n


# RFC 8439 Appendix A.1, test vectors #1 (counter 0) and #2 (counter 1): all-zero key and nonce.
TV1 = bytes.fromhex("76b8e0ada0f13d90405d6ae55386bd28bdd219b8a08ded1aa836efcc8b770dc7"
                    "da41597c5157488d7724e03fb8d84a376a43b8f41518a11cc387b669b2ee6586")
TV2_HEAD = bytes.fromhex("9f07e7be5551387a98ba977c732d080d")


def test_chacha20_rfc8439_vectors():
    b0 = struct.pack("<16I", *O.chacha_block([0] * 8, 0))
    b1 = struct.pack("<16I", *O.chacha_block([0] * 8, 1))
    assert b0 == TV1
    assert b1[:16] == TV2_HEAD


def test_rng_derive_is_sha256_seeded_chacha():
    # rng::derive(root, label) = ChaCha20Rng::from_seed(SHA-256(root_le || label)) (src/rng.rs:9-17)
    root, label = 5, "sampler test"
    seed = hashlib.sha256(struct.pack("<Q", root) + label.encode()).digest()
    key = list(struct.unpack("<8I", seed))
    r = O.Rng(root, label)
    words = [r.next_u32() for _ in range(40)]
    blocks = O.chacha_block(key, 0) + O.chacha_block(key, 1) + O.chacha_block(key, 2)
    assert words == blocks[:40]
    # next_u64 = lo | hi << 32 of the next two words, also across a block boundary after an odd
    # number of u32 draws (rand_core BlockRng).
    r1, r2 = O.Rng(root, label), O.Rng(root, label)
    r1.next_u32()
    r2.next_u32()
    w = [r2.next_u32() for _ in range(40)]
    u = [r1.next_u64() for _ in range(20)]
    assert u == [w[2 * i] | (w[2 * i + 1] << 32) for i in range(20)]


def test_uniform_mapping_endpoints():
    # u = ((k >> 11) + 0.5) / 2^53 (rl.rs:490-498). The reference calls it the open interval
    # (0, 1), but for k >> 11 = 2^53 - 1 the f64 sum 2^53 - 0.5 rounds (ties to even) to 2^53,
    # so u = 1.0 exactly with probability 2^-53; the inverse-CDF sampler then takes its "no
    # crossing" branch (the last token with weight).
    assert O.uniform_open01(0) == 0.5 / 2 ** 53
    assert O.uniform_open01(2 ** 64 - 1) == 1.0
    assert O.uniform_open01((2 ** 53 - 2) << 11) == (2 ** 53 - 1.5) / 2 ** 53 < 1.0
    z = f32([[0.0, 1.0, NINF, 2.0, NINF]])
    ids, _ = O.sample_invcdf(z, [1.0])
    assert ids[0] == 3
    assert O.uniform_open01(1 << 63) == 0.5 + 0.5 / 2 ** 53


def test_box_muller_normals_are_standard():
    z = O.Rng(9, "normals").normals(200_000)
    assert abs(z.mean()) < 0.01 and abs(z.std() - 1.0) < 0.01
    # the Box-Muller convention: u1 = gen_f64 (max 1e-300), u2 = gen_f64, cos branch
    r, s = O.Rng(9, "normals"), O.Rng(9, "normals")
    g = s.gen_f64(2)
    assert r.normals(1)[0] == math.sqrt(-2.0 * math.log(max(g[0], 1e-300))) * math.cos(2.0 * math.pi * g[1])


# ------------------------------------------------------------------------ bf16

def test_bf16_round_to_nearest_even():
    rng = np.random.default_rng(3)
    bits = rng.integers(0, 2 ** 32, 200_000, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    x = x[np.isfinite(x)]
    h = O.bf16_from_f32(x)
    # brute force: the nearest of the two bf16 neighbours, ties to the even one
    lo = (x.view(np.uint32) & 0xFFFF0000).view(np.float32)
    hi_bits = (x.view(np.uint32).astype(np.uint64) & 0xFFFF0000) + 0x10000
    for i in range(2000):
        xi = float(x[i])
        cands = [int(x[i].view(np.uint32) >> 16), int(hi_bits[i] >> 16) & 0xFFFF]
        vals = [float(O.bf16_to_f32(np.uint16(c))) for c in cands]
        d = [abs(v - xi) if math.isfinite(v) else math.inf for v in vals]
        if d[0] < d[1]:
            want = cands[0]
        elif d[1] < d[0]:
            want = cands[1]
        else:
            want = cands[0] if cands[0] % 2 == 0 else cands[1]
        assert int(h[i]) == want, (xi, h[i], cands)
    # the vectorised form equals the scalar C restatement (half.rs:16-23), NaN included
    special = f32([0.0, -0.0, 1.0, -1.0, np.inf, -np.inf, np.nan, 3.4e38, 1e-40, 1.00390625, 1.01171875])
    for v in list(special) + list(x[:500]):
        assert int(O.bf16_from_f32(f32([v]))[0]) == O.bf16_from_f32_scalar(float(v))
    assert np.all(O.bf16_to_f32(O.bf16_from_f32(lo)) == lo)


# ------------------------------------------------------------------------ row oracle

def test_tempered_logits_are_f32_divide_then_add():
    rng = np.random.default_rng(4)
    x = f32(rng.normal(0, 3, (3, 50)))
    add = f32(rng.normal(0, 1, (1, 50)))
    for tau in (0.7, 1.0, 2.5):
        z = O.tempered(x, tau, addmask=add)
        want = (x if tau == 1.0 else x / np.float32(tau)) + add  # numpy: IEEE f32 divide and add
        assert np.array_equal(z, want)
    keep = np.array([[1, 0] * 25], dtype=np.uint8)
    z = O.tempered(x, 0.8, keep=keep)
    assert np.all(np.isneginf(z[:, 1::2])) and np.array_equal(z[:, 0::2], x[:, 0::2] / np.float32(0.8))


def test_log_probs_entropy_kl_match_scipy():
    rng = np.random.default_rng(5)
    for V in (1, 2, 7, 64, 1000):
        z = f32(rng.normal(0, 3, (6, V)))
        r = f32(z + rng.normal(0, 0.5, (6, V)))
        ls = log_softmax(z.astype(np.float64), axis=1)
        lr = log_softmax(r.astype(np.float64), axis=1)
        tok = rng.integers(0, V, 6)
        assert_close("logp", O.token_logp(z, tok), ls[np.arange(6), tok], 1e-13)
        assert_close("entropy", O.entropy(z), -(np.exp(ls) * ls).sum(1), 1e-12)
        assert_close("kl", O.kl(z, r), (np.exp(ls) * (ls - lr)).sum(1), 1e-12)
        assert np.all(O.kl(z, r) >= -1e-15)
        assert np.all(np.abs(O.kl(z, z)) < 1e-15)  # KL(π ‖ π) = 0 (tests/rl.rs:363)


def test_reference_known_answers_large_and_excluded():
    # tests/rl.rs:134-150: ±1e4 logits stay finite; a −∞ token gives −∞
    lp = O.token_logp(f32([[1e4, -1e4, 0.0, 1e3], [-1e4, -1e4, 1e4, 1e4]]), [0, 2])
    assert abs(lp[0]) < 1e-6 and abs(lp[1] - math.log(0.5)) < 1e-6
    row = f32([[1.0, NINF, 0.0, 2.0]] * 2)
    lp = O.token_logp(row, [1, 3])
    assert lp[0] == NINF
    assert abs(lp[1] - log_softmax([1.0, 0.0, 2.0])[2]) < 1e-12
    # tests/rl.rs:392-407: −∞ entries give the KL / entropy of the kept tokens
    p = f32([[1.0, NINF, 0.5, -1.0], [2.0, 0.0, NINF, NINF]])
    q = f32([[0.0, NINF, 1.5, 0.5], [-1.0, 1.0, NINF, NINF]])
    assert_close("kl kept", O.kl(p, q), [O.kl(p[:1, [0, 2, 3]], q[:1, [0, 2, 3]])[0], O.kl(p[1:, :2], q[1:, :2])[0]], 1e-15)
    assert_close("entropy kept", O.entropy(p), [O.entropy(p[:1, [0, 2, 3]])[0], O.entropy(p[1:, :2])[0]], 1e-15)
    # uniform entropy = ln V (tests/rl.rs:369-370)
    assert_close("uniform", O.entropy(f32([[0.3] * 5])), [math.log(5)], 1e-15)
    # π > 0 where π_ref = 0 gives +∞ (tests/rl.rs:420-421)
    assert O.kl(f32([[0.0, 0.0]]), f32([[0.0, NINF]]))[0] == math.inf
    # one-sided −1e9 gives about 1e9 · p₂ (tests/rl.rs:807-811)
    one = f32([[0.0, 0.5, 1.0]])
    p2 = math.exp(log_softmax([0.0, 0.5, 1.0])[2])
    k = O.kl(one, one + f32([[0.0, 0.0, -1e9]]))[0]
    assert abs(k / (1e9 * p2) - 1.0) < 1e-6
    # rows refused by the sampler: every entry −∞, or a NaN (rl.rs:516-519)
    assert O.row_stats(f32([NINF, NINF])).status == 1
    assert O.row_stats(f32([0.0, np.nan, 1.0])).status == 2
    # first maximum, NaN-propagating (kernels.rs:184-209)
    assert O.row_stats(f32([1.0, 3.0, 3.0, 2.0])).argmax == 1
    assert O.row_stats(f32([1.0, np.nan, 5.0])).argmax == 1


# ------------------------------------------------------------------------ inverse-CDF sampler

def _numpy_invcdf(z, u):
    """The same definition by an independent route: f64 weights, cumsum, searchsorted."""
    m = np.max(z.astype(np.float64))
    w = np.exp(z.astype(np.float64) - m)
    c = np.cumsum(w)
    i = int(np.searchsorted(c, u * c[-1], side="right"))
    return i if i < len(z) else int(np.nonzero(w > 0)[0][-1])


def test_invcdf_matches_brute_force_on_tiny_rows():
    with open(os.path.join(HERE, "golden", "tiny_invcdf.json")) as f:
        fx = json.load(f)
    grid = np.arange(1, 1000) / 1000.0
    for case in fx["cases"]:
        x = np.frombuffer(bytes.fromhex(case["logits_f32_hex"]), dtype=np.float32)
        keep = np.array(case["keep_u8"], dtype=np.uint8)
        z = O.tempered(x[None, :], case["temperature"], keep=keep[None, :])
        ids, edges = O.sample_invcdf(np.repeat(z, grid.size, 0), grid)
        assert ids.tolist() == case["ids_on_grid"], "oracle drifted from the committed fixture"
        for u, i, e in zip(grid, ids, edges):
            if e > 1e-12:  # away from floating ties, cumsum order is the same
                assert i == _numpy_invcdf(z[0], u)
            assert keep[i] == 1, "an excluded token was drawn"
        # the step function: token v is drawn on an interval of length p_v
        p = np.exp(log_softmax(z[0].astype(np.float64)))
        counts = np.bincount(ids, minlength=len(x)) / grid.size
        assert np.all(np.abs(counts - p) <= 2.0 / grid.size + 1e-12)


def test_invcdf_frequencies_match_the_distribution():
    # the reference's frequency test (tests/rl.rs:579-611): 40,000 draws within 4.5 s.e.
    row = f32([0.4, -1.0, 1.2, 3.0, 0.0, -0.3])
    maskrow = f32([0.0, 0.0, 0.0, NINF, 0.5, 0.0])
    n = 40_000
    for tau in (0.7, 1.0, 2.5):
        z = O.tempered(row[None, :], tau, addmask=maskrow[None, :])
        u = O.Rng(5, "sampler test").uniforms(n)
        ids, _ = O.sample_invcdf(np.repeat(z, n, 0), u)
        p = np.exp(log_softmax((row.astype(np.float64) / tau) + maskrow))
        cnt = np.bincount(ids, minlength=6)
        assert cnt[3] == 0, "excluded token drawn"
        f = cnt / n
        se = np.sqrt(p * (1 - p) / n)
        assert np.all(np.abs(f - p) <= 4.5 * se + 1e-12), (tau, f, p)


def test_argmax_is_first_and_greedy_picks_masked_argmax():
    # tests/rl.rs:617-625: τ = 0 is the argmax of the masked logits (token 4)
    row = f32([0.4, -1.0, 1.2, 3.0, 0.0, -0.3])
    z = O.tempered(row[None, :], 1.0, addmask=f32([[0.0, 0.0, 0.0, NINF, 2.0, 0.0]]))
    assert O.argmax_first(z)[0] == 4


# ------------------------------------------------------------------------ estimators, reductions

def test_kl_estimators_closed_forms_and_enumeration():
    # δ = 100: clamped k3 = exp(20) − 21 (tests/rl.rs:753-768); masked positions give 0
    k = O.kl_estimate([-100.5, -1.0], [-0.5, -1.2], 3, clamp=20.0)
    assert abs(k[0] - (math.exp(20.0) - 21.0)) <= 1e-12 * k[0]
    assert abs(k[1] - (math.exp(-0.2) + 0.2 - 1.0)) < 1e-15
    assert O.kl_estimate([-1.0], [-3.0], 1, mask=[0.0])[0] == 0.0
    assert O.kl_estimate([-1.0], [-3.0], 2)[0] == 2.0
    # E_π[k1] = E_π[k3] = KL(π ‖ π_ref) by enumeration (tests/rl.rs:467-500)
    rng = np.random.default_rng(6)
    V = 6
    pl, rl = f32(rng.uniform(-2, 2, V)), f32(rng.uniform(-2, 2, V))
    lp, lr = log_softmax(pl.astype(np.float64)), log_softmax(rl.astype(np.float64))
    pi = np.exp(lp)
    kl = O.kl(pl[None, :], rl[None, :])[0]
    for est in (1, 3):
        assert abs(float((O.kl_estimate(lp, lr, est) * pi).sum()) - kl) < 1e-14
    assert np.all(O.kl_estimate(lp, lr, 2) >= 0) and np.all(O.kl_estimate(lp, lr, 3) >= 0)


def test_reductions_by_hand():
    # tests/rl.rs:163-179: per-token [1 2 0; 0 −10 0], mask [1 1 0; 0 1 0]
    per = [1.0, 2.0, 0.0, 0.0, -10.0, 0.0]
    m = [1.0, 1.0, 0.0, 0.0, 1.0, 0.0]
    sh = (1, 2, 3)
    assert O.reduce_tokens(per, m, sh, "sum").tolist() == [-7.0]
    assert abs(O.reduce_tokens(per, m, sh, "token_mean")[0] + 7.0 / 3.0) < 1e-15
    assert O.reduce_tokens(per, m, sh, "per_sequence").tolist() == [1.5, -10.0]
    assert O.reduce_tokens(per, m, sh, "sequence_mean").tolist() == [-4.25]
    assert O.reduce_tokens(per, m, sh, "none").tolist() == per
    # every position masked: exact zeros (tests/rl.rs:506-545)
    z = [0.0] * 6
    for red in ("sum", "token_mean", "per_sequence", "sequence_mean"):
        assert np.all(O.reduce_tokens(z, z, sh, red) == 0.0)


def test_group_advantages_by_hand():
    # tests/rl.rs:550-569
    r = [1.0, 0.0, 0.0, 1.0, 2.0, 2.0, 2.0, 2.0, 0.0, 0.0, 0.0, 3.0]
    s3 = 0.5 / math.sqrt(1.0 / 3.0)
    assert_close("unbiased", O.group_advantages(r, 4, "std", 0.0, True),
                 [s3, -s3, -s3, s3, 0, 0, 0, 0, -0.5, -0.5, -0.5, 1.5], 1e-15)
    p3 = math.sqrt(1.6875)
    assert_close("population", O.group_advantages(r, 4, "std", 0.0, False),
                 [1, -1, -1, 1, 0, 0, 0, 0, -0.75 / p3, -0.75 / p3, -0.75 / p3, 2.25 / p3], 1e-15)
    assert O.group_advantages(r, 4, "mean").tolist() == [0.5, -0.5, -0.5, 0.5, 0, 0, 0, 0, -0.75, -0.75, -0.75, 2.25]
    assert_close("eps", O.group_advantages(r, 4, "std", 1e-2, True)[8:], [-0.75 / 1.51] * 3 + [2.25 / 1.51], 1e-15)
    assert O.group_advantages([3.0, -1.0], 1, "std", 1e-6, False).tolist() == [0.0, 0.0]
    # equal rewards give exact zeros at ε = 0 (tests/rl.rs:644-653)
    a = O.group_advantages([0.1, 0.1, 0.1, 1.0, 0.0, 0.0], 3, "std", 0.0, True)
    assert a[:3].tolist() == [0.0, 0.0, 0.0] and a[3] > 0 > a[4] and a[4] == a[5]
    with pytest.raises(ValueError):
        O.group_advantages([1.0, 2.0], 1, "std", 1e-6, True)  # tests/rl.rs:571-575


# ------------------------------------------------------------------------ Cpu(Reference) restatement

def test_cpuref_log_softmax_in_f32():
    rng = np.random.default_rng(8)
    x = f32(rng.normal(0, 4, (5, 333)))
    y = O.cpuref_log_softmax(x)
    assert_close("cpuref log_softmax", y, log_softmax(x.astype(np.float64), axis=1), 1e-6)
    # the 8-partial order is exact on small integers
    v = f32(np.arange(1, 20))
    assert O.unrolled_sum(v) == float(v.sum())


def test_cpuref_gumbel_sampler_frequencies_and_consumption():
    row = f32([0.4, -1.0, 1.2, 3.0, 0.0, -0.3])
    keep = np.array([[1, 1, 1, 0, 1, 1]], dtype=np.uint8)
    n, tau = 20_000, 0.7
    rng = O.Rng(5, "gumbel")
    ids, lp = O.cpuref_sample_logp(np.repeat(row[None, :], n, 0), tau, keep, rng)
    # the stream advanced one u64 per logit (tests/rl.rs:596-599)
    copy = O.Rng(5, "gumbel")
    for _ in range(n * 6):
        copy.next_u64()
    assert rng.next_u64() == copy.next_u64()
    z = np.where(keep[0] == 1, row.astype(np.float64) / tau, -np.inf)
    p = np.exp(log_softmax(z))
    cnt = np.bincount(ids, minlength=6)
    assert cnt[3] == 0
    se = np.sqrt(p * (1 - p) / n)
    assert np.all(np.abs(cnt / n - p) <= 4.5 * se + 1e-12)
    assert_close("gumbel logp", lp, np.log(p[ids]), 1e-6)
    with pytest.raises(ValueError, match="no allowed token"):
        O.cpuref_sample_logp(f32(np.zeros((2, 3))), 1.0, np.array([[1, 1, 1], [0, 0, 0]], dtype=np.uint8),
                             O.Rng(0, "x"))


def test_cpuref_gumbel_with_additive_masks_is_the_references_sampler_test():
    # tests/rl.rs:579-625 on or_cpuref_sample_gumbel (the checker of the device's Gumbel sampler):
    # 40,000 copies of one row under an additive [1, V] mask, frequencies within 4.5 s.e., one u64
    # per logit, the same stream the same tokens and another stream other tokens; greedy is the
    # masked argmax [4, 4] and draws nothing; a refused row draws nothing.
    row = f32([0.4, -1.0, 1.2, 3.0, 0.0, -0.3])
    maskrow = f32([[0.0, 0.0, 0.0, -np.inf, 0.5, 0.0]])
    n, v = 40_000, 6
    x = np.repeat(row[None, :], n, 0)
    for tau in (0.7, 1.0, 2.5):
        rng, copy = O.Rng(5, "sampler test"), O.Rng(5, "sampler test")
        tok = O.cpuref_sample_gumbel(x, tau, rng, addmask=maskrow)
        for _ in range(n * v):
            copy.next_u64()
        assert rng.next_u64() == copy.next_u64(), "one u64 per logit"
        p = np.exp(log_softmax(row.astype(np.float64) / tau + maskrow[0].astype(np.float64)))
        cnt = np.bincount(tok, minlength=v)
        assert cnt[3] == 0
        se = np.sqrt(p * (1 - p) / n)
        assert np.all(np.abs(cnt / n - p) <= 4.5 * se + 1e-12), (tau, cnt / n, p)
        assert np.array_equal(O.cpuref_sample_gumbel(x, tau, O.Rng(5, "sampler test"), addmask=maskrow), tok)
        assert not np.array_equal(O.cpuref_sample_gumbel(x, tau, O.Rng(6, "sampler test"), addmask=maskrow), tok)
    # the keep-mask form gives the additive form's tokens (0 / -inf)
    keep = np.array([[1, 1, 1, 0, 1, 1]], np.uint8)
    zero_half = f32([[0.0, 0.0, 0.0, -np.inf, 0.0, 0.0]])
    assert np.array_equal(O.cpuref_sample_gumbel(x[:500], 0.9, O.Rng(1, "k"), keep=keep),
                          O.cpuref_sample_gumbel(x[:500], 0.9, O.Rng(1, "k"), addmask=zero_half))
    # greedy (tests/rl.rs:617-625)
    greedy_mask = f32([[0.0, 0.0, 0.0, -np.inf, 2.0, 0.0]])
    rng, copy = O.Rng(1, "greedy"), O.Rng(1, "greedy")
    assert O.cpuref_sample_gumbel(np.stack([row, row]), 0.0, rng, addmask=greedy_mask).tolist() == [4, 4]
    assert rng.next_u64() == copy.next_u64(), "greedy draws nothing"
    # a refused row draws nothing (the reference's check precedes its draw, rl.rs:515-519)
    rng, copy = O.Rng(0, "x"), O.Rng(0, "x")
    with pytest.raises(ValueError, match="position 1 has no allowed token"):
        O.cpuref_sample_gumbel(f32(np.zeros((2, 3))), 1.0, rng, addmask=f32([[0, 0, 0], [-np.inf] * 3]))
    assert rng.next_u64() == copy.next_u64()
    # V = 2 in closed form: P(token 0) = sigmoid(z0 - z1)
    n2 = 50_000
    tok = O.cpuref_sample_gumbel(np.repeat(f32([[0.3, -0.9]]), n2, 0), 1.0, O.Rng(8, "two"))
    p0 = 1.0 / (1.0 + math.exp(-(0.3 - -0.9)))
    assert abs(np.mean(tok == 0) - p0) <= 4.5 * math.sqrt(p0 * (1 - p0) / n2)


def test_u8_keep_mask_selects_in_every_checker():
    """A u8 keep-mask selects: an excluded token is -inf whatever its logit, so a NaN or +inf there
    does not reach the row (the device kernels' rule). The reference's additive -inf mask lets
    them through (NaN + -inf and +inf + -inf are NaN) and the row is refused. The three CPU
    checkers that take a keep-mask (the f64 row oracle's tempered, the Cpu(Reference) Gumbel
    sequence, the Cpu(Fast) inverse-CDF sequence) apply the same rule."""
    f32 = lambda a: np.asarray(a, np.float32)
    x = f32([[0.3, np.nan, 1.2, np.inf, -0.5, 0.8], [1.0, 2.0, np.nan, 0.0, np.inf, -1.0]])
    keep = np.array([[1, 0, 1, 0, 1, 1], [1, 1, 0, 1, 0, 1]], np.uint8)
    add = np.where(keep == 1, 0.0, -np.inf).astype(np.float32)
    z = O.tempered(x, 0.7, keep=keep)
    assert np.all(np.isneginf(z[keep == 0])) and np.all(np.isfinite(z[keep == 1]))
    for tau in (1.0, 0.7, 0.0):
        ids = O.cpuref_sample_gumbel(x, tau, O.Rng(3, "keep rule"), keep=keep)
        assert keep[np.arange(2), ids].all()
        # the same tokens as the finite rows with the excluded logits replaced
        xf = np.where(keep == 1, x, 0.0).astype(np.float32)
        assert np.array_equal(ids, O.cpuref_sample_gumbel(xf, tau, O.Rng(3, "keep rule"), keep=keep))
        with pytest.raises(ValueError, match="position 0 has no allowed token"):
            O.cpuref_sample_gumbel(x, tau, O.Rng(3, "keep rule"), addmask=add)
    ids, lp = O.cpufast_sample_logp(x, 0.7, keep, O.Rng(4, "keep rule"), 2)
    assert keep[np.arange(2), ids].all() and np.all(np.isfinite(lp))
    ids2, lp2 = O.cpufast_sample_logp(np.where(keep == 1, x, 0.0).astype(np.float32), 0.7, keep, O.Rng(4, "keep rule"), 2)
    assert np.array_equal(ids, ids2) and np.array_equal(lp, lp2)


def test_cpufast_restatement_against_cpuref_and_the_f64_oracle():
    # Cpu(Fast) (src/tensor/backend.rs:57-239) differs from Cpu(Reference) only in how maps, zips
    # and sums are split: above its thresholds (here 64 x 65536 = 2^22 elements) the tokens, whose
    # argmax runs the Reference kernel on the same noise, equal CpuRef's for the same stream; the
    # log-probabilities differ only in the sum order (16 accumulators against 8 partials) and hold
    # the f64 oracle's value within f32 tolerance; the stream advances one u64 per logit; threads
    # do not change the result. The sum order itself has no reference record (parity unpinned
    # below the tolerance).
    rng = np.random.default_rng(4)
    R, V = 64, 65536
    x = rng.normal(0, 2, (R, V)).astype(np.float32)
    keep = (rng.random((R, V)) < 0.4).astype(np.uint8)
    keep[:, 3] = 1
    a_ids, a_lp = O.cpuref_sample_logp(x, 0.7, keep, O.Rng(5, "fast"))
    outs = []
    for threads in (1, 3, 8):
        r = O.Rng(5, "fast")
        ids, lp = O.cpufast_sample_logp(x, 0.7, keep, r, threads)
        copy = O.Rng(5, "fast")
        for _ in range(R * V):
            copy.next_u64()
        assert r.next_u64() == copy.next_u64(), "one u64 per logit"
        assert np.array_equal(ids, a_ids)
        outs.append(lp.tobytes())
        z = O.tempered(x, 0.7, keep=keep)
        want = O.token_logp(z, ids)
        assert np.all(np.abs(lp - want) <= 1e-6 + 1e-5 * np.abs(want))
    assert outs[1] == outs[2], "threads change nothing above the thresholds"
    # below the thresholds every op is Reference's: bit-identical to CpuRef
    small = x[:4, :1024]
    b_ids, b_lp = O.cpufast_sample_logp(small, 0.7, keep[:4, :1024], O.Rng(6, "fast"), 8)
    c_ids, c_lp = O.cpuref_sample_logp(small, 0.7, keep[:4, :1024], O.Rng(6, "fast"))
    assert np.array_equal(b_ids, c_ids) and b_lp.tobytes() == c_lp.tobytes()


# ------------------------------------------------------------------------ golden C1 fixture

def test_c1_golden_fixture():
    with open(os.path.join(HERE, "golden", "c1_readme.json")) as f:
        fx = json.load(f)
    S, B, T, V = fx["shape"]
    x = np.stack([np.frombuffer(bytes.fromhex(h), dtype=np.float32) for h in fx["logits_f32_hex"]])
    keep = np.array(fx["keep_u8"], dtype=np.uint8)
    u = np.array(fx["uniforms"])
    assert x.shape == (S * B * T, V) and keep.min(axis=1).min() >= 0 and keep.sum(axis=1).min() >= 1
    # the fixture's inputs come from the seeded streams it names
    from tests.golden.make_golden import c1_inputs
    _, x2, keep2, u2 = c1_inputs()
    assert np.array_equal(x, x2) and np.array_equal(keep, keep2) and np.array_equal(u, u2)
    z = O.tempered(x, 1.0, keep=keep)
    ids, edges = O.sample_invcdf(z, u)
    assert ids.tolist() == fx["ids"]
    # independent check of the expected values: scipy's log_softmax over the kept tokens
    ls = log_softmax(np.where(keep == 1, x.astype(np.float64), -np.inf), axis=1)
    assert_close("c1 logp", fx["logp"], ls[np.arange(len(ids)), ids], 1e-13)
    ent = -np.where(keep == 1, np.exp(ls) * np.where(keep == 1, ls, 0.0), 0.0).sum(1)
    assert_close("c1 entropy", fx["entropy"], ent, 1e-13)
    for i, row_id in enumerate(ids):
        assert row_id == _numpy_invcdf(z[i], u[i])


# ------------------------------------------------------------------------ fused backward

def _fd_objective(z, zr, tok, g_lp, g_kl, g_h):
    """The forward objective in f64 from scipy (independent of the oracle's restatement)."""
    lp = log_softmax(z)
    val = g_lp * lp[tok] if tok >= 0 else 0.0
    pi = np.exp(lp)
    if g_kl:
        lr = log_softmax(zr)
        val += g_kl * float(np.sum(np.where(pi > 0, pi * (lp - lr), 0.0)))
    if g_h:
        val += g_h * float(-np.sum(np.where(pi > 0, pi * lp, 0.0)))
    return val


def test_score_grad_matches_finite_differences():
    # the reference checks its gradients by central differences (fd_input, eps 1e-6, tol 1e-7;
    # src/nn/tests/joint_embed.rs:19-33, used at tests/rl.rs:125-129 and 283-314); here against
    # scipy's log_softmax as the forward, for each term alone and all three together
    rng = np.random.default_rng(71)
    V = 12
    z = rng.uniform(-3, 3, V).astype(np.float32).astype(np.float64)
    zr = (z + rng.normal(0, 0.5, V)).astype(np.float32).astype(np.float64)
    tok = 5
    for g in [(1.0, 0.0, 0.0), (0.0, 1.0, 0.0), (0.0, 0.0, 1.0), (-0.7, 1.3, 0.4)]:
        got = O.score_grad(z.astype(np.float32), [tok], zr.astype(np.float32), [g[0]], [g[1]], [g[2]])[0]
        fd = np.empty(V)
        for j in range(V):
            zp, zm = z.copy(), z.copy()
            zp[j] += 1e-6
            zm[j] -= 1e-6
            fd[j] = (_fd_objective(zp, zr, tok, *g) - _fd_objective(zm, zr, tok, *g)) / 2e-6
        assert np.all(np.abs(fd - got) <= 1e-7 * (1 + np.abs(fd))), (g, np.max(np.abs(fd - got)))


def test_score_grad_of_token_log_probs_is_onehot_minus_softmax():
    # tests/rl.rs:116-121: d sum(token_log_probs)/dx = onehot - softmax (to 1e-14 in f64)
    rng = np.random.default_rng(72)
    x = rng.uniform(-6, 6, (5, 9)).astype(np.float32)
    tok = rng.integers(0, 9, 5)
    got = O.score_grad(x, tok, g_lp=np.ones(5))
    sm = np.exp(log_softmax(x.astype(np.float64), axis=1))
    want = np.eye(9)[tok] - sm
    assert np.max(np.abs(got - want)) <= 1e-14
    # the temperature's divide: z = x / T, dL/dx = dL/dz / T
    tau = 0.7
    z = O.tempered(x, tau)
    got = O.score_grad(z, tok, g_lp=np.ones(5), tau=tau)
    want = (np.eye(9)[tok] - np.exp(log_softmax(z.astype(np.float64), axis=1))) / tau
    assert np.max(np.abs(got - want)) <= 1e-14


def test_score_grad_large_and_excluded_logits():
    # tests/rl.rs:131-150: logits of +-1e4 stay finite; an entry excluded by -inf has gradient 0
    # (only the token term where the token itself is excluded)
    x = np.array([[1e4, -1e4, 0.0, 1e3], [-1e4, -1e4, 1e4, 1e4]], np.float32)
    got = O.score_grad(x, [0, 2], g_lp=[1.0, 1.0])
    assert np.all(np.isfinite(got))
    assert got[0, 0] == 0.0 and abs(got[1, 2] - 0.5) < 1e-15 and abs(got[1, 3] + 0.5) < 1e-15
    z = np.array([[0.5, -np.inf, 1.0, -np.inf]], np.float32)
    zr = np.array([[0.2, -np.inf, 0.9, 3.0]], np.float32)
    got = O.score_grad(z, [1], zr, [1.0], [0.3], [0.2])
    assert got[0, 3] == 0.0 and got[0, 1] == 1.0 and np.all(np.isfinite(got))


# ----------------------------------------------------------------------------- policy losses

def test_policy_gradient_reductions_by_hand():
    # tests/rl.rs:160-179: logp [-1..-6] as [1,2,3], per-sequence weights [1,-2], mask [1 1 0; 0 1 0]
    lp = np.array([-1.0, -2.0, -3.0, -4.0, -5.0, -6.0])
    w = np.array([1.0, -2.0])
    m = np.array([1.0, 1.0, 0.0, 0.0, 1.0, 0.0])
    per, dper, _ = O.policy_loss("pg", lp, None, w, m, 3, per_seq=True)
    assert per.tolist() == [1.0, 2.0, 0.0, 0.0, -10.0, 0.0]
    assert dper.tolist() == [-1.0, -1.0, 0.0, 0.0, 2.0, 0.0]
    red = lambda r: O.reduce_tokens(per, m, (1, 2, 3), r).tolist()
    assert red("sum") == [-7.0]
    assert abs(red("token_mean")[0] + 7.0 / 3.0) < 1e-15
    assert red("per_sequence") == [1.5, -10.0]
    assert red("sequence_mean") == [-4.25]
    per_all, _, _ = O.policy_loss("pg", lp, None, w, None, 3, per_seq=True)
    assert O.reduce_tokens(per_all, None, (1, 2, 3), "sum").tolist() == [6.0 - 30.0]


def test_clipped_policy_loss_overflow_guard_known_answers():
    # tests/rl.rs:725-750 in f64: A = -1 with a log-ratio of 100; an on-policy token with A = 1
    lp, old, adv = np.array([-0.5, -1.0]), np.array([-100.5, -1.0]), np.array([-1.0, 1.0])
    loss, dloss, hit = O.policy_loss("ppo", lp, old, adv, None, 2, low=0.2, high=0.2, clamp=20.0)
    assert abs(loss[0] - math.exp(20.0)) <= 1e-9 * math.exp(20.0) and dloss[0] == 0.0
    assert loss[1] == -1.0 and dloss[1] == -1.0
    loss, dloss, _ = O.policy_loss("ppo", lp, old, adv, None, 2, dual=3.0, clamp=20.0)
    assert (loss[0], dloss[0]) == (3.0, 0.0)
    loss, _, _ = O.policy_loss("ppo", lp, old, adv, None, 2, clamp=None)
    assert loss[0] == math.exp(100.0)  # f64 holds it; f32 overflows to +inf (tested on the device)
    assert O.reduce_tokens(hit, None, (1, 1, 2), "token_mean").tolist() == [0.5]


def _ppo_case(seed, n=60, T=5):
    # tests/rl.rs:228-235's construction: old = logp + offsets so every ratio exp(-o) is away from
    # the clip edges (1.65, 1.105, 0.95, 0.67, and 4.48 for a dual clip), advantages of both signs
    rng = np.random.default_rng(seed)
    lp = -rng.uniform(0.1, 4.0, n)
    offs = np.array([-1.5, -0.5, -0.1, 0.05, 0.4])
    old = lp + offs[(np.arange(n) * 7 + np.arange(n) // 3) % 5]
    adv = rng.uniform(-2.0, 2.0, n)
    adv = np.where(np.abs(adv) < 0.1, -0.5, adv)
    mask = (rng.random(n) < 0.8).astype(np.float64)
    return lp, old, adv, mask, T


@pytest.mark.parametrize("clip", [dict(low=0.2, high=0.2), dict(low=0.2, high=0.28),
                                  dict(low=0.2, high=0.2, dual=3.0), dict(low=0.1, high=0.3, clamp=None)])
def test_policy_loss_derivatives_match_finite_differences(clip):
    lp, old, adv, mask, T = _ppo_case(840)
    _, dloss, _ = O.policy_loss("ppo", lp, old, adv, mask, T, **clip)
    h = 1e-6
    for i in range(lp.size):
        e = np.zeros_like(lp)
        e[i] = h
        fd = (O.policy_loss("ppo", lp + e, old, adv, mask, T, **clip)[0][i] -
              O.policy_loss("ppo", lp - e, old, adv, mask, T, **clip)[0][i]) / (2 * h)
        assert abs(fd - dloss[i]) <= 1e-7 * (1 + abs(fd)), (i, fd, dloss[i])
    # PG: the derivative is -w, per token and per sequence
    w = np.random.default_rng(1).uniform(-2, 2, lp.size // T)
    _, d, _ = O.policy_loss("pg", lp, None, w, mask, T, per_seq=True)
    assert np.array_equal(d, np.where(mask != 0, -np.repeat(w, T), 0.0))


def test_ppo_on_policy_gradient_equals_pg_and_bounds_give_zero():
    # tests/rl.rs:297-313: at old = logp the PPO derivative is the PG one with the advantages as
    # weights; a clipped-and-active token (A > 0, r > 1.2 or A < 0, r < 0.8) gets zero, others -A r
    lp, old, adv, mask, T = _ppo_case(850)
    _, d_ppo, _ = O.policy_loss("ppo", lp, lp, adv, mask, T)
    _, d_pg, _ = O.policy_loss("pg", lp, None, adv, mask, T)
    assert np.array_equal(d_ppo, d_pg)
    _, d, hit = O.policy_loss("ppo", lp, old, adv, mask, T)
    r = np.exp(lp - old)
    clipped = ((adv > 0) & (r > 1.2)) | ((adv < 0) & (r < 0.8))
    want = np.where((mask == 0) | clipped, 0.0, -adv * r)
    assert np.allclose(d, want, rtol=1e-14, atol=0)
    assert np.array_equal(hit, np.where(mask != 0, clipped.astype(float), 0.0))
    # a dual clip c = 3 caps A < 0 tokens with r > 3 at -3A, with zero derivative
    loss, d, hit = O.policy_loss("ppo", lp, old, adv, mask, T, dual=3.0)
    capped = (mask != 0) & (adv < 0) & (r > 3.0)
    assert capped.any()
    assert np.array_equal(loss[capped], -3.0 * adv[capped]) and np.all(d[capped] == 0.0)
    assert np.all(hit[capped] == 1.0)


@pytest.mark.parametrize("reduction", ["none", "sum", "token_mean", "per_sequence", "sequence_mean"])
def test_reduce_tokens_backward_matches_finite_differences(reduction):
    S, B, T = 2, 3, 4
    rng = np.random.default_rng(7)
    per = rng.normal(0, 1, S * B * T)
    mask = (rng.random(S * B * T) < 0.6).astype(np.float64)
    mask[(0 * B + 1) * T:(0 * B + 2) * T] = 0.0  # an empty sequence
    mask[S * B * T // 2:] = 0.0                  # an empty seed
    per = np.where(mask != 0, per, 0.0)
    n_out = O.reduce_tokens(per, mask, (S, B, T), reduction).size
    up = rng.normal(0, 1, n_out)
    local = rng.normal(0, 1, S * B * T)
    got = O.reduce_tokens_backward(mask, (S, B, T), reduction, up, 0.5, local)
    h = 1e-6
    for i in range(S * B * T):
        e = np.zeros_like(per)
        e[i] = h
        f = lambda x: float(up @ O.reduce_tokens(np.where(mask != 0, x, 0.0), mask, (S, B, T), reduction))
        fd = 0.5 * local[i] * (f(per + e) - f(per - e)) / (2 * h)
        assert abs(fd - got[i]) <= 1e-8 * (1 + abs(fd)), (reduction, i, fd, got[i])


def test_kl_estimate_derivatives_match_finite_differences():
    rng = np.random.default_rng(9)
    lp = -rng.uniform(0.1, 5, 40)
    lr = lp + rng.normal(0, 1.5, 40)
    lr[3] = lp[3] + 30.0  # beyond a clamp of 20
    mask = (rng.random(40) < 0.8).astype(np.float64)
    h = 1e-6
    for est in (1, 2, 3):
        for clamp in (None, 20.0):
            g = O.kl_estimate_grad(lp, lr, est, clamp, mask)
            for i in range(40):
                e = np.zeros(40)
                e[i] = h
                fd = (O.kl_estimate(lp + e, lr, est, clamp, mask)[i] - O.kl_estimate(lp - e, lr, est, clamp, mask)[i]) / (2 * h)
                assert abs(fd - g[i]) <= 1e-6 * (1 + abs(fd)), (est, clamp, i, fd, g[i])


def test_chacha_stream_layout_matches_the_reference_fixtures():
    # The reference's recorded burn fixtures (src/tensor/tests/fixtures/burn021-windows-x86_64.txt
    # and burn021-macos-aarch64.txt, the same records on both platforms: add_scalar, mul_scalar,
    # sum_dim2 of src/tensor/tests/f64ops.rs:12-24) hash the bits of outputs whose inputs come from
    # ChaCha8Rng::seed_from_u64 and gen_range (src/tensor/tests/mod.rs:28-31). Reproducing them pins
    # the ChaCha block layout and word order the oracle's ChaCha20 stream shares (with RFC 8439
    # pinning the 20-round core), rand_core's seed expansion and rand's f32 range mapping.
    records = {"add_scalar": "cbe9c8a9adc29c2d425c260f055b10adbd6444714471aa97519b2a7e9b72ccdb",
               "mul_scalar": "19c77c93a882e0421e1e07d82a202d6f1633c7dce42085119519d85adf9ceef8",
               "sum_dim2": "9de56d8c8dae0c91245cd23e063c8bb7d5ddc74ca56c9e4b1100e05647cb8425"}
    x = O.reference_rnd_f32(1, 130, -3.0, 3.0)
    v = (x.astype(np.float64) * 1.37).astype(np.float32).astype(np.float64)  # `ours` (f64ops.rs:7)
    sha = lambda a: hashlib.sha256(np.ascontiguousarray(a, "<f8").tobytes()).hexdigest()
    assert sha(v + 1e-6) == records["add_scalar"]
    assert sha(v * 0.3) == records["mul_scalar"]
    s = v.reshape(2, 5, 13)
    assert sha([sum(list(s[i, j]), 0.0) for i in range(2) for j in range(5)]) == records["sum_dim2"]
    # the check discriminates: the textbook PCG increment (a plausible mix-up) misses every record
    bad = np.empty(130, dtype=np.float32)
    O.lib().or_reference_rnd_f32(1, 1442695040888963407, 130, -3.0, 3.0, bad.ctypes.data_as(O._c_float_p))
    vb = (bad.astype(np.float64) * 1.37).astype(np.float32).astype(np.float64)
    assert sha(vb + 1e-6) != records["add_scalar"]


def test_cpuref_log_softmax_order_matches_the_reference_fixture():
    # src/tensor/tests/f64ops.rs:21 records the reference's log_softmax (activation.rs:30-42) of
    # [2,5,13] inputs along the last axis in f64; the record (same on both platforms) fixes its
    # operation order, the unrolled lane sum of kernels.rs:120-151 included. A left-to-right sum
    # (a plausible restatement) misses it.
    record = "934eb3edd7b1924449a0c2b3f72727493eaee084a744c77a6dc69f820d8d36d9"
    x = O.reference_rnd_f32(1, 130, -3.0, 3.0)
    v = (x.astype(np.float64) * 1.37).astype(np.float32).astype(np.float64).reshape(10, 13)
    sha = lambda a: hashlib.sha256(np.ascontiguousarray(a, "<f8").tobytes()).hexdigest()
    assert sha(O.cpuref_log_softmax_f64(v)) == record
    seq = [[(t - r.max()) - math.log(sum((math.exp(u - r.max()) for u in r), 0.0)) for t in r] for r in v]
    assert sha(seq) != record
