"""Masks that broadcast over leading dimensions on the fused path (rl.rs:477-483: the mask has the
logits' rank, each dimension equal or 1), through NtMaskRows.

Each case runs the fused sampler (sample_logp with entropy), the scorer (logp, reference logp,
exact KL, entropy and the saved statistics), its fused backward, and, where the reference takes
the dtype, the Gumbel-max sample_categorical, once with the broadcast mask and once with the same
mask materialised to the logits' full shape: the results must be the same bits. They are then
checked against the oracle's f64 restatement on the materialised mask: ids equal except within
1e-6 of a CDF edge, values within 1e-5 relative / 1e-6 absolute. Shapes cover one, two and three
folded groups, four groups (the host broadcasts the mask on the device first), odd vocabularies
(the element-wise kernels), C4's vocabulary at 8 and 256 rows (the segmented and the queued
samplers), and masks of one value per position ([.., 1], broadcast along the vocabulary too,
which the host also broadcasts on the device first)."""
import zlib

import numpy as np
import pytest

import noetic_rl as nr
from oracle import oracle as O

pytestmark = pytest.mark.gpu
EDGE = 1e-6


@pytest.fixture(scope="module", autouse=True)
def device():
    nr.claim(0)
    yield


def close(name, got, want):
    got, want = np.asarray(got, np.float64).ravel(), np.asarray(want, np.float64).ravel()
    fin = np.isfinite(want)
    assert np.array_equal(np.isfinite(got), fin), f"{name}: finite pattern"
    assert np.array_equal(got[~fin], want[~fin]), f"{name}: non-finite values"
    err = np.abs(got[fin] - want[fin])
    assert np.all(err <= 1e-6 + 1e-5 * np.abs(want[fin])), f"{name}: off by {err.max():.2e}"


def to_dev(x, dtype):
    if dtype == "bf16":
        return nr.Tensor.from_numpy(O.bf16_from_f32(x), "bf16")
    if dtype == "f16":
        return nr.Tensor.from_numpy(x.astype(np.float16).view(np.uint16), "f16")
    return nr.Tensor.from_numpy(x)


def widened(x, dtype):
    if dtype == "bf16":
        return O.bf16_to_f32(O.bf16_from_f32(x))
    if dtype == "f16":
        return x.astype(np.float16).astype(np.float32)
    return x.astype(np.float32)


def make_mask(rng, mshape, kind):
    if kind == "u8":
        m = (rng.random(mshape) < 0.5).astype(np.uint8)
        m[..., 3] = 1
        return m
    if kind == "u8 position":
        return np.ones(mshape, np.uint8)  # [.., 1]: every position kept
    if kind == "f32 position":
        return rng.normal(0, 3, mshape).astype(np.float32)  # [.., 1]: a finite value per position
    m = np.where(rng.random(mshape) < 0.3, -np.inf, rng.normal(0, 0.5, mshape)).astype(np.float32)
    m[..., 5] = -1e9
    m[..., 3] = 0.0
    return m


CASES = [
    # name, logits shape, mask shape, mask kind, dtype, tau, oracle rows (None = all)
    ("[S,1,1,V] u8 f32", (3, 4, 5, 1000), (3, 1, 1, 1000), "u8", "f32", 0.8, None),
    ("[1,B,1,V] T>1 f32-mask bf16", (2, 3, 4, 777), (1, 3, 1, 777), "f32", "bf16", 0.7, None),
    ("[S,1,T,V] u8 bf16 tau 1", (2, 3, 4, 2048), (2, 1, 4, 2048), "u8", "bf16", 1.0, None),
    ("[1,B,1,V] f16", (1, 6, 3, 4104), (1, 6, 1, 4104), "u8", "f16", 0.9, None),
    ("four groups", (2, 2, 2, 2, 600), (2, 1, 2, 1, 600), "u8", "f32", 0.9, None),
    ("[1,B,1,V] C4 vocabulary, 8 rows", (1, 4, 2, 128256), (1, 4, 1, 128256), "u8", "bf16", 0.7, None),
    ("[1,B,1,V] C4 vocabulary, 256 rows", (1, 128, 2, 128256), (1, 128, 1, 128256), "u8", "bf16", 0.7,
     np.arange(0, 256, 17)),
    # a mask that broadcasts along the vocabulary axis too: one value per position (the host
    # broadcasts it to the logits' shape on the device first)
    ("[S,B,T,1] f32 value per position", (2, 3, 4, 777), (2, 3, 4, 1), "f32 position", "f32", 0.8, None),
    ("[S,1,T,1] f32 bf16 tau 1", (2, 3, 4, 1000), (2, 1, 4, 1), "f32 position", "bf16", 1.0, None),
    ("[1,B,1,1] u8", (1, 5, 2, 600), (1, 5, 1, 1), "u8 position", "f16", 0.9, None),
]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_broadcast_masks(case):
    name, shape, mshape, kind, dtype, tau, sel = case
    rng = np.random.default_rng(zlib.crc32(name.encode()))
    V = shape[-1]
    rows = int(np.prod(shape[:-1]))
    x = rng.normal(0, 2, shape).astype(np.float32)
    y = (x + rng.normal(0, 0.3, shape)).astype(np.float32)
    m = make_mask(rng, mshape, kind)
    full = np.ascontiguousarray(np.broadcast_to(m, shape))
    xt, yt = to_dev(x, dtype), to_dev(y, dtype)
    mdt = "u8" if kind.startswith("u8") else "f32"
    mt, ft = nr.Tensor.from_numpy(m, mdt), nr.Tensor.from_numpy(full, mdt)
    u = nr.Rng(7, name).uniforms(rows)
    ut = nr.Tensor.from_numpy(u, "f64")

    # the fused sampler
    a = nr.sample_logp(xt, tau, mt, None, entropy=True, uniforms=ut)
    b = nr.sample_logp(xt, tau, ft, None, entropy=True, uniforms=ut)
    for i, what in enumerate(("ids", "logp", "entropy")):
        assert a[i].to_numpy().tobytes() == b[i].to_numpy().tobytes(), f"{name}: sampler {what} differ"
    ids, lp, ent = (t.to_numpy().reshape(rows) for t in a)

    # the scorer and its saved statistics, then the fused backward
    tok = nr.Tensor.from_numpy(ids.reshape(shape[:-1]).astype(np.int32))
    sa = nr.score_with_stats(nr.Tempered(xt, tau, mt), nr.Tempered(yt, tau, mt), tok)
    sb = nr.score_with_stats(nr.Tempered(xt, tau, ft), nr.Tempered(yt, tau, ft), tok)
    for i in range(4):
        assert sa[i].to_numpy().tobytes() == sb[i].to_numpy().tobytes(), f"{name}: score output {i} differs"
    for f in ("lse_base", "lse_rest", "ref_lse_base", "ref_lse_rest"):
        assert getattr(sa[4], f).to_numpy().tobytes() == getattr(sb[4], f).to_numpy().tobytes(), f"{name}: {f}"
    g = {k: nr.Tensor.from_numpy(rng.normal(0, 1, shape[:-1]).astype(np.float32)) for k in ("lp", "kl", "h")}
    ga = nr.score_grad(nr.Tempered(xt, tau, mt), nr.Tempered(yt, tau, mt), tok, sa[4], kl=sa[2], entropy=sa[3],
                       g_logp=g["lp"], g_kl=g["kl"], g_entropy=g["h"], grad_dtype="f32")
    gb = nr.score_grad(nr.Tempered(xt, tau, ft), nr.Tempered(yt, tau, ft), tok, sb[4], kl=sb[2], entropy=sb[3],
                       g_logp=g["lp"], g_kl=g["kl"], g_entropy=g["h"], grad_dtype="f32")
    assert ga.to_numpy().tobytes() == gb.to_numpy().tobytes(), f"{name}: backward differs"

    # the reference's sampler, where the reference takes this dtype and temperature
    if not (dtype != "f32" and tau == 1.0):
        ga_ids = nr.sample_categorical(xt, tau, mt, nr.Rng(8, name)).to_numpy()
        gb_ids = nr.sample_categorical(xt, tau, ft, nr.Rng(8, name)).to_numpy()
        assert ga_ids.tobytes() == gb_ids.tobytes(), f"{name}: Gumbel ids differ"

    # the oracle on the materialised mask
    r = np.arange(rows) if sel is None else sel
    xw = widened(x, dtype).reshape(rows, V)[r]
    yw = widened(y, dtype).reshape(rows, V)[r]
    fm = full.reshape(rows, V)[r]
    kw = dict(keep=fm) if mdt == "u8" else dict(addmask=fm)
    z, zr = O.tempered(xw, tau, **kw), O.tempered(yw, tau, **kw)
    want, edges = O.sample_invcdf(z, u[r])
    differ = np.nonzero(ids[r] != want)[0]
    assert np.all(edges[differ] < EDGE), f"{name}: rows {r[differ][:8]} differ from the oracle away from a CDF edge"
    close(f"{name} logp", lp[r], O.token_logp(z, ids[r]))
    close(f"{name} entropy", ent[r], O.entropy(z))
    lps, rlps, kls, ents = (sa[i].to_numpy().reshape(rows)[r] for i in range(4))
    close(f"{name} score logp", lps, O.token_logp(z, ids[r]))
    close(f"{name} score ref logp", rlps, O.token_logp(zr, ids[r]))
    close(f"{name} score kl", kls, O.kl(z, zr))
    close(f"{name} score entropy", ents, O.entropy(z))
    print(f"{name}: {rows} rows, {len(differ)} boundary draws")
