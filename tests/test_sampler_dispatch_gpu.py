"""nt_hip_rl_sample's default choice of kernel by shape, measured on MI355X and checked here
against the oracle at the shapes each choice serves:
- few rows with many chunks (a small-batch decode step at V = 128256): the segmented sampler,
  one row across 8 workgroups;
- unmasked f32 rows of 32768 < V <= 65536 (V = 50304): segments up to 256 rows, the streaming
  kernel beyond (the register-resident kernel would need 8 chunks per wave there and spill);
- C4's 256 rows: one workgroup per row.
Reruns are byte-identical whichever segment of a row happens to arrive last."""
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


def check(name, z, u, ids, lp, ent, bf16):
    want, edges = O.sample_invcdf(z, u)
    differ = np.nonzero(ids != want)[0]
    assert np.all(edges[differ] < EDGE), f"{name}: rows {differ[:8]} differ away from a CDF edge"
    tol = (lambda w: 1e-6 + 2e-3 * np.abs(w)) if bf16 else (lambda w: 1e-6 + 1e-5 * np.abs(w))
    wl, wh = O.token_logp(z, ids), O.entropy(z)
    assert np.all(np.abs(lp - wl) <= tol(wl)), f"{name}: logp"
    assert np.all(np.abs(ent - wh) <= tol(wh)), f"{name}: entropy"
    print(f"{name}: {len(ids)} rows, {len(differ)} ids differ ({int(np.sum(edges < EDGE))} boundary draws), "
          f"logp max |d| {np.max(np.abs(lp - wl)):.1e}, entropy max |d| {np.max(np.abs(ent - wh)):.1e}")


@pytest.mark.parametrize("rows", [1, 3, 16, 64])
def test_small_batch_decode_rows_take_segments(rows):
    w = W.c4(rows=rows)
    V = w["V"]
    u = nr.Rng(rows, "dispatch/c4").uniforms(rows)
    ut = nr.Tensor.from_numpy(u, "f64")
    out = [nr.sample_logp(w["logits"], 0.7, w["mask"], None, entropy=True, uniforms=ut) for _ in range(3)]
    ids, lp, ent = (t.to_numpy().ravel() for t in out[0])
    for again in out[1:]:
        assert all(a.to_numpy().tobytes() == b.to_numpy().tobytes() for a, b in zip(again, out[0])), "rerun bits"
    x = W.bf16_to_f32(w["logits"].to_numpy().reshape(rows, V))
    keep = w["mask"].to_numpy().reshape(rows, V)
    # the f32 tolerance: the bf16 inputs are exact in f32, and the kernel computes in f32 and f64
    check(f"c4 row shape, {rows} rows", O.tempered(x, 0.7, keep=keep), u, ids, lp, ent, bf16=False)


@pytest.mark.parametrize("rows", [8, 256, 1024])
def test_unmasked_f32_rows_of_50304(rows):
    V = 50304
    x = W.normal((rows, V), "f32", rows, "dispatch/f32", std=1.5)
    u = nr.Rng(rows, "dispatch/f32u").uniforms(rows)
    ut = nr.Tensor.from_numpy(u, "f64")
    a = nr.sample_logp(x, 0.8, None, None, entropy=True, uniforms=ut)
    b = nr.sample_logp(x, 0.8, None, None, entropy=True, uniforms=ut)
    assert all(p.to_numpy().tobytes() == q.to_numpy().tobytes() for p, q in zip(a, b)), "rerun bits"
    ids, lp, ent = (t.to_numpy().ravel() for t in a)
    pick = np.arange(rows) if rows <= 256 else np.arange(0, rows, 8)
    xs = W.download_rows(x, pick, V)
    check(f"f32 V=50304, {rows} rows", O.tempered(xs, 0.8), u[pick], ids[pick], lp[pick], ent[pick], bf16=False)


def test_greedy_through_segments():
    # temperature 0 in the segmented sampler: the first maximum in index order, across segments
    rows, V = 4, 128256
    x = np.random.default_rng(9).normal(0, 1, (rows, V)).astype(np.float32)
    x[0, [70000, 90000]] = 9.0          # a tie across segments: the earlier wins
    x[1, [17, 128255]] = 9.0
    x[2, 100000] = 9.0
    x[3, :] = 1.0                       # all equal: index 0
    xb = O.bf16_from_f32(x)
    xt = nr.Tensor.from_numpy(xb, "bf16")
    ids, lp = nr.sample_logp(xt, 0.0, None, None)
    assert ids.to_numpy().tolist() == [70000, 17, 100000, 0]
