"""f16 logits on the fused path (NT_F16): the kernels widen each value exactly, as the reference
computes 16-bit dtypes in f32 (src/tensor/float.rs:43-58; half.rs's F16).

At C2's decode shape (64 rows of V = 32000, tau 0.8, no mask; C2's own inputs rounded to f16),
C4's (256 rows of V = 128256 under a 30% runs mask, tau 0.7: the queued sampler) and an odd
vocabulary (the element-wise kernels), the sampler's ids equal the oracle's f64 inverse CDF on the
widened logits except within 1e-6 of a CDF edge, and its log-probabilities and entropies, the
scorer's values and the Gumbel-max sampler's draws are checked against the oracle and against
the same calls on the widened f32 logits. Special values (subnormals, the largest finite value,
-inf, NaN) widen exactly: a NaN row and an all -inf row are refused with their statuses."""
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


def close(name, got, want):
    got, want = np.asarray(got, np.float64).ravel(), np.asarray(want, np.float64).ravel()
    fin = np.isfinite(want)
    assert np.array_equal(np.isfinite(got), fin), f"{name}: finite pattern"
    assert np.array_equal(got[~fin], want[~fin]), f"{name}: non-finite values"
    err = np.abs(got[fin] - want[fin])
    assert np.all(err <= 1e-6 + 1e-5 * np.abs(want[fin])), f"{name}: off by {err.max():.2e}"


def f16_pair(x):
    """(device f16 tensor, the widened f32 values) of f32 x."""
    h = x.astype(np.float16)
    return nr.Tensor.from_numpy(h.view(np.uint16), "f16"), h.astype(np.float32)


def run(name, x, tau, keep=None, sel=None):
    rows, V = x.shape
    xt, xw = f16_pair(x)
    ft = nr.Tensor.from_numpy(xw)
    mt = None if keep is None else nr.Tensor.from_numpy(keep)
    u = nr.Rng(31, name).uniforms(rows)
    ut = nr.Tensor.from_numpy(u, "f64")
    ids, lp, ent = (t.to_numpy() for t in nr.sample_logp(xt, tau, mt, None, entropy=True, uniforms=ut))
    fids, flp, fent = (t.to_numpy() for t in nr.sample_logp(ft, tau, mt, None, entropy=True, uniforms=ut))
    r = np.arange(rows) if sel is None else sel
    z = O.tempered(xw[r], 1.0 if tau == 0 else tau, keep=None if keep is None else keep[r])
    if tau == 0.0:
        want, edges = O.argmax_first(z), np.ones(len(r))  # greedy: the first maximum, exactly
    else:
        want, edges = O.sample_invcdf(z, u[r])
    differ = np.nonzero(ids[r] != want)[0]
    assert np.all(edges[differ] < EDGE), f"{name}: rows {r[differ][:8]} differ from the oracle away from a CDF edge"
    fd = np.nonzero(ids != fids)[0]
    assert len(fd) <= 1, f"{name}: {len(fd)} ids differ from the widened f32 call's"
    close(f"{name} logp", lp[r], O.token_logp(z, ids[r]))
    close(f"{name} entropy", ent[r], O.entropy(z))
    close(f"{name} logp vs f32", lp, flp)
    close(f"{name} entropy vs f32", ent, fent)
    # the scorer on the drawn tokens
    tok = nr.Tensor.from_numpy(ids.astype(np.int32))
    slp, _, _, sent = nr.score(nr.Tempered(xt, 1.0 if tau == 0 else tau, mt), None, tok, entropy=True, kl=False)
    close(f"{name} score logp", slp.to_numpy()[r], O.token_logp(z, ids[r]))
    close(f"{name} score entropy", sent.to_numpy()[r], O.entropy(z))
    # the Gumbel-max sampler, where the reference takes f16 (tau not 1; greedy only unmasked):
    # the widened logits' draws
    if tau not in (0.0, 1.0) or (tau == 0.0 and keep is None):
        ga = nr.sample_categorical(xt, tau, mt, nr.Rng(32, name)).to_numpy()
        gb = nr.sample_categorical(ft, tau, mt, nr.Rng(32, name)).to_numpy()
        assert ga.tobytes() == gb.tobytes(), f"{name}: Gumbel draws differ from the widened f32 call's"
    else:
        with pytest.raises(nr.DTypeError, match="add: f16 and f32"):
            nr.sample_categorical(xt, tau, mt, nr.Rng(32, name))
    print(f"{name}: {len(differ)} boundary draws, {len(fd)} ids apart from the f32 call")


def test_f16_at_the_c2_decode_shape():
    w = W.c2()
    x = w["logits"].to_numpy().reshape(w["rows"], w["V"])
    run("c2 f16", x, w["temperature"])


def test_f16_at_the_c4_decode_shape():
    w = W.c4()
    x = W.bf16_to_f32(w["logits"].to_numpy().reshape(w["rows"], w["V"]))
    keep = w["mask"].to_numpy().reshape(w["rows"], w["V"])
    run("c4 f16", x, w["temperature"], keep=keep, sel=np.arange(0, 256, 9))


@pytest.mark.parametrize("tau", [0.0, 1.0, 0.6])
def test_f16_odd_vocabulary(tau):
    rng = np.random.default_rng(12)
    x = rng.normal(0, 3, (24, 1001)).astype(np.float32)
    keep = (rng.random((24, 1001)) < 0.6).astype(np.uint8)
    keep[:, 7] = 1
    run(f"odd f16 tau {tau}", x, tau, keep=keep)


def test_f16_special_values():
    rng = np.random.default_rng(13)
    V = 512
    x = rng.normal(0, 1, (6, V)).astype(np.float16)
    x[0, :8] = np.array([6.0e-8, -6.0e-8, 6.1e-5, 65504, -65504, -np.inf, 0.0, -0.0], np.float16)
    x[1, :] = np.float16(-np.inf)          # nothing allowed
    x[2, 5] = np.float16(np.nan)           # a NaN reaches the sum
    x[3, :] = np.float16(6.0e-8)           # subnormal only: uniform
    x[4, 100] = np.float16(65504)          # the largest finite value dominates
    xt = nr.Tensor.from_numpy(x.view(np.uint16), "f16")
    ft = nr.Tensor.from_numpy(x.astype(np.float32))
    u = nr.Tensor.from_numpy(nr.Rng(33, "special").uniforms(6), "f64")
    a = nr.sample_logp(xt, 0.9, None, None, uniforms=u, check=False)
    b = nr.sample_logp(ft, 0.9, None, None, uniforms=u, check=False)
    ia, ib = a[0].to_numpy(), b[0].to_numpy()
    assert ia[1] == -1 and ib[1] == -1 and ia[2] == -1 and ib[2] == -1
    assert ia[4] == 100 and a[1].to_numpy()[4] == 0.0
    ok = [0, 3, 4, 5]
    assert np.array_equal(ia[ok], ib[ok])
    close("special logp", a[1].to_numpy()[ok], b[1].to_numpy()[ok])
    with pytest.raises(ValueError, match="position 1 has no allowed token"):
        nr.sample_logp(xt, 0.9, None, None, uniforms=u)
