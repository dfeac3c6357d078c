"""The drop-in's dtype and precision rules on the device.

Reference-named functions keep the reference's refusals of 16-bit logits (noetic-tensor 0.7.0:
`log_softmax`'s "sub: bf16 and f32", activation.rs:30-42 with float.rs:710-722; the Gumbel noise's
"add: bf16 and f32" at τ == 1, rl.rs:520-525 with float.rs:257-260), in the reference's order: the
row check precedes the noise, and a refused call leaves the stream where it was. Where the
reference takes 16-bit logits (τ ≠ 1, or greedy without a mask) the results are those of the
exactly widened f32 logits: the same ids, and values within the f32 tolerance (1e-5 relative /
1e-6 absolute; the kernels read bf16 and f32 rows in different lane orders, so sums may round
apart). The fused entries (`sample_logp`, `score` on a `Tempered` triple) take 16-bit logits at
every τ and give the widened logits' results to the same bar. The
platform key carries the reduced-precision product's part only at MatmulPrecision::Half
(gpu/mod.rs:690-704)."""
import numpy as np
import pytest

import noetic_ops as nops
import noetic_rl as nr
from oracle import oracle as O

pytestmark = pytest.mark.gpu

ADD = r"^add: bf16 and f32 \(casts are explicit\)$"
SUB = r"^sub: bf16 and f32 \(casts are explicit\)$"


@pytest.fixture(scope="module", autouse=True)
def device():
    nr.claim(0)
    yield


def close(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    fin = np.isfinite(b)
    assert np.array_equal(np.isfinite(a), fin) and np.array_equal(a[~fin], b[~fin])
    assert np.all(np.abs(a[fin] - b[fin]) <= 1e-6 + 1e-5 * np.abs(b[fin]))


def logits(rows=12, V=700, seed=3):
    rng = np.random.default_rng(seed)
    xb = O.bf16_from_f32(rng.normal(0, 2, (rows, V)).astype(np.float32))
    return xb, O.bf16_to_f32(xb)


def test_sample_categorical_on_bf16_follows_the_reference():
    xb, xf = logits()
    rows, V = xf.shape
    tb, tf = nr.Tensor.from_numpy(xb, "bf16"), nr.Tensor.from_numpy(xf)
    # τ == 1: refused by z + g, and the stream is not advanced
    rng = nr.Rng(11, "dtype/gumbel")
    before = rng.word_pos()
    with pytest.raises(nr.DTypeError, match=ADD):
        nr.sample_categorical(tb, 1.0, None, rng)
    assert rng.word_pos() == before
    # the row check comes first (rl.rs:516-519 before 520-525)
    dead = xb.copy()
    dead[4] = 0xFF80  # bf16 −∞
    with pytest.raises(ValueError, match="position 4 has no allowed token"):
        nr.sample_categorical(nr.Tensor.from_numpy(dead, "bf16"), 1.0, None, nr.Rng(11, "dtype/gumbel"))
    # greedy with a mask: tempered_logits' add
    keep = np.ones((rows, V), np.uint8)
    with pytest.raises(nr.DTypeError, match=ADD):
        nr.sample_categorical(tb, 0.0, nr.Tensor.from_numpy(keep), nr.Rng(11, "dtype/gumbel"))
    # where the reference samples bf16, the ids are the widened logits' ids, and the stream moves alike
    for tau, mask in ((0.7, nr.Tensor.from_numpy(keep)), (0.0, None), (1.3, None)):
        ra, rb = nr.Rng(12, "dtype/gumbel"), nr.Rng(12, "dtype/gumbel")
        a = nr.sample_categorical(tb, tau, mask, ra).to_numpy()
        b = nr.sample_categorical(tf, tau, mask, rb).to_numpy()
        assert np.array_equal(a, b), f"τ {tau}: bf16 and widened f32 ids differ"
        assert ra.word_pos() == rb.word_pos()


def test_log_softmax_functions_refuse_untempered_bf16():
    xb, xf = logits(rows=2 * 3, V=301, seed=4)
    tb = nr.Tensor.from_numpy(xb.reshape(1, 2, 3, 301), "bf16")
    tf = nr.Tensor.from_numpy(xf.reshape(1, 2, 3, 301))
    tok = nr.Tensor.from_numpy(np.arange(6, dtype=np.int32).reshape(1, 2, 3) * 17)
    with pytest.raises(nr.DTypeError, match=SUB):
        nr.token_log_probs(tb, tok)
    with pytest.raises(nr.DTypeError, match=SUB):
        nr.categorical_entropy(tb)
    with pytest.raises(nr.DTypeError, match=SUB):
        nr.categorical_kl(tb, tb)
    # the general ops' log_softmax refuses in the same place
    with pytest.raises(nr.DTypeError, match=SUB):
        nops.log_softmax(nops.DTensor(tb), 3)
    # tempered at τ ≠ 1 the reference computes in f32: the widened logits' values
    keep = nr.Tensor.from_numpy((np.random.default_rng(4).random((1, 2, 3, 301)) < 0.8).astype(np.uint8))
    close(nr.token_log_probs(nr.tempered_logits(tb, 0.7, keep), tok).to_numpy(),
          nr.token_log_probs(nr.tempered_logits(tf, 0.7, keep), tok).to_numpy())
    a = nr.reference_kl(tb, tb, 0.7, keep, None, nr.TokenReduction.NONE).to_numpy()
    b = nr.reference_kl(tf, tf, 0.7, keep, None, nr.TokenReduction.NONE).to_numpy()
    assert np.all(np.abs(a.astype(np.float64) - b) <= 1e-6 + 1e-5 * np.abs(b))


def test_fused_entries_take_bf16_at_every_temperature_as_widened_f32():
    xb, xf = logits(rows=16, V=1000, seed=5)
    tb, tf = nr.Tensor.from_numpy(xb, "bf16"), nr.Tensor.from_numpy(xf)
    keep = nr.Tensor.from_numpy((np.random.default_rng(5).random((16, 1000)) < 0.5).astype(np.uint8))
    u = nr.Tensor.from_numpy(nr.Rng(13, "dtype/u").uniforms(16), "f64")
    for tau, mask in ((1.0, None), (1.0, keep), (0.6, keep)):
        ia, la = nr.sample_logp(tb, tau, mask, None, uniforms=u)
        ib, lb = nr.sample_logp(tf, tau, mask, None, uniforms=u)
        assert np.array_equal(ia.to_numpy(), ib.to_numpy()), f"τ {tau}: ids"
        close(la.to_numpy(), lb.to_numpy())
        sa = nr.score(nr.Tempered(tb, tau, mask), None, ia, entropy=True, kl=False)
        sb = nr.score(nr.Tempered(tf, tau, mask), None, ib, entropy=True, kl=False)
        close(sa[0].to_numpy(), sb[0].to_numpy())
        close(sa[3].to_numpy(), sb[3].to_numpy())
        # scoring the sampler's draws gives its log-probabilities (two kernels: the f32 tolerance)
        d = np.abs(sa[0].to_numpy().astype(np.float64) - la.to_numpy())
        assert np.all(d <= 1e-6 + 1e-5 * np.abs(la.to_numpy()))


@pytest.mark.parametrize("dt", ["bf16", "f16"])
def test_16_bit_additive_masks_add_in_f32(dt):
    """A 16-bit additive mask of the logits' own dtype on untempered logits: the reference's add
    computes the sum in f32 into f32 storage (fdisp, float.rs:43-58; f32_operand on a GPU,
    gpu/mod.rs:336-342), so tempered_logits is f32 and the reference's functions and its sampler
    at τ == 1 take it. Every path gives the widened f32 inputs' results: the materialised sum bit
    for bit, the Gumbel and greedy ids with the stream moved alike, and the scorer's values within
    the f32 tolerance (bf16 and f32 rows are read in different lane orders)."""
    rows, V = 12, 700
    rng = np.random.default_rng(6)
    x = rng.normal(0, 2, (rows, V)).astype(np.float32)
    m = np.where(rng.random((rows, V)) < 0.3, -np.inf, rng.normal(0, 1, (rows, V))).astype(np.float32)
    m[:, 3] = 0.0
    if dt == "bf16":
        xr, mr = O.bf16_from_f32(x), O.bf16_from_f32(m)
        xw, mw = O.bf16_to_f32(xr), O.bf16_to_f32(mr)
    else:
        xr, mr = x.astype(np.float16).view(np.uint16), m.astype(np.float16).view(np.uint16)
        xw, mw = xr.view(np.float16).astype(np.float32), mr.view(np.float16).astype(np.float32)
    sh = (1, 3, 4, V)  # [S, B, T, V], as categorical_entropy takes it
    t16, m16 = nr.Tensor.from_numpy(xr.reshape(sh), dt), nr.Tensor.from_numpy(mr.reshape(sh), dt)
    t32, m32 = nr.Tensor.from_numpy(xw.reshape(sh)), nr.Tensor.from_numpy(mw.reshape(sh))
    z16, z32 = nops.tempered_logits(t16, 1.0, m16), nops.tempered_logits(t32, 1.0, m32)
    assert z16.dtype == "f32" and z16.to_numpy().tobytes() == z32.to_numpy().tobytes()
    assert np.array_equal(z16.to_numpy(), (xw + mw).reshape(sh))
    for tau in (1.0, 0.0, 0.8):
        if tau == 0.8:
            # divided logits are f32 and the mask is not: refused by add, before any draw
            with pytest.raises(nr.DTypeError, match=f"add: f32 and {dt}"):
                nr.sample_categorical(t16, tau, m16, nr.Rng(21, "m16"))
            continue
        ra, rb = nr.Rng(21, "m16"), nr.Rng(21, "m16")
        a = nr.sample_categorical(t16, tau, m16, ra).to_numpy()
        b = nr.sample_categorical(t32, tau, m32, rb).to_numpy()
        assert np.array_equal(a, b), f"τ {tau}: ids"
        assert ra.word_pos() == rb.word_pos()
    tok = nr.Tensor.from_numpy(((np.arange(rows, dtype=np.int32) * 31) % V).reshape(sh[:-1]))
    close(nr.token_log_probs(nr.tempered_logits(t16, 1.0, m16), tok).to_numpy(),
          nr.token_log_probs(nr.tempered_logits(t32, 1.0, m32), tok).to_numpy())
    close(nr.categorical_entropy(nr.tempered_logits(t16, 1.0, m16)).to_numpy(),
          nr.categorical_entropy(nr.tempered_logits(t32, 1.0, m32)).to_numpy())
    # the fused triple takes the 16-bit mask at every τ, widened
    u = nr.Tensor.from_numpy(nr.Rng(22, "m16/u").uniforms(rows), "f64")
    ia, la = nr.sample_logp(t16, 0.8, m16, None, uniforms=u)
    ib, lb = nr.sample_logp(t32, 0.8, m32, None, uniforms=u)
    assert np.array_equal(ia.to_numpy(), ib.to_numpy())
    close(la.to_numpy(), lb.to_numpy())


def test_platform_key_carries_the_half_product_part_only_at_half():
    base = nr.platform_key()
    assert "gemm-" not in base
    with nr.matmul_precision_scope(nr.MatmulPrecision.HALF):
        half = nr.platform_key()
        part = nops.half_gemm_key()
    assert half == f"{base}-{part}" and part.startswith("gemm-bf16-")
    assert nr.platform_key() == base
