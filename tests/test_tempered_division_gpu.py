"""The kernels' tempered values under an additive f32 mask against IEEE f32 division, on the GPU.

The kernels take a row's maximum from their own tempered values (x / T computed as
f32(f64(x) * (1 / f64(T))), with the division itself for quotients below 2^-126) and the
scored token's value by the f32 division. A row whose only allowed token is token 0 therefore
scores log-probability (z_div - z_kernel) - ln 1, which is 0 exactly when the two agree to the
bit. The numerators are the f32 significands whose quotients by T lie closest to a rounding
midpoint (exact integer search), at exponents from subnormal quotients to past the overflow
threshold, both signs, at three temperatures, for aligned (V = 512) and unaligned (V = 1000)
rows. Rows whose quotient overflows (+inf: inf - inf, refused; -inf: nothing allowed, refused)
must be refused exactly where numpy's f32 division overflows."""
import numpy as np
import pytest

import noetic_rl as nr
from tests.test_tempered_division import by_division, nearest_to_midpoints, with_exponent

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def device():
    nr.claim(0)
    yield


def numerators(tau):
    X = nearest_to_midpoints(tau, 64)
    xs = [with_exponent(X, e) for e in range(-170, 105, 6)]
    # numerators whose quotients straddle the overflow threshold (below 1: the largest finite ones)
    fmax = np.float64(np.finfo(np.float32).max)
    top = np.float32(fmax * np.float64(np.float32(tau))) if tau < 1 else np.float32(fmax)
    near = [top]
    for _ in range(8):
        if tau < 1:
            near.append(np.nextafter(near[-1], np.float32(np.inf)))
        near.insert(0, np.nextafter(near[0], np.float32(0)))
    xs.append(np.array(near, np.float32))
    x = np.concatenate(xs)
    return np.concatenate([x, -x, np.array([0.0, -0.0, 5 * 2.0 ** -149, 3 * 2.0 ** -149, np.inf, -np.inf], np.float32)])


@pytest.mark.parametrize("V", [512, 1000])
@pytest.mark.parametrize("tau", [0.7, 0.9, 1.3])
def test_tempered_values_equal_f32_division(tau, V):
    x0 = numerators(tau)
    rows = len(x0)
    rng = np.random.default_rng(V)
    x = rng.normal(0, 2, (rows, V)).astype(np.float32)
    x[:, 0] = x0
    add = np.full((rows, V), -np.inf, np.float32)
    add[:, 0] = 0.0
    tok = nr.Tensor.from_numpy(np.zeros(rows, np.int32))
    lp, _, _, ent = nr.score(nr.Tempered(nr.Tensor.from_numpy(x), tau, nr.Tensor.from_numpy(add)), None, tok,
                             entropy=True, kl=False)
    lp, ent = lp.to_numpy().ravel(), ent.to_numpy().ravel()
    z = by_division(x0, tau)
    fin = np.isfinite(z)
    assert np.all(lp[fin] == 0.0), (f"tau {tau} V {V}: {int(np.sum(lp[fin] != 0))} rows whose maximum differs "
                                    f"from the division, e.g. x = {x0[fin][lp[fin] != 0][:4]!r}")
    assert np.all(ent[fin] == 0.0)
    assert np.all(np.isnan(lp[~fin])), f"tau {tau} V {V}: overflowed quotients must refuse their rows"
    assert (~fin).sum() >= (16 if tau < 1 else 2) and fin.sum() > 1000
