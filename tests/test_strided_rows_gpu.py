"""Strided rows through the C ABI (ld > V, mask_ld > V, grad_ld > V), as a caller with padded rows
passes them: every kernel must read only the first V elements of each row and write only the first
V gradient elements. The pads hold NaN (inputs) or a sentinel (gradient), so a read or write of a
pad shows. With aligned strides the results equal the dense call's bit for bit; with unaligned
strides (the element-wise path) they hold the oracle's tolerances. Several host threads calling
the entry points at once get the results of calling them one after another.
"""
import ctypes as C

import numpy as np
import pytest

import noetic_rl as nr
from oracle import oracle as O

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def device():
    nr.claim(0)
    yield


def padded(a, ld, fill):
    rows, V = a.shape
    out = np.full((rows, ld), fill, dtype=a.dtype)
    out[:, :V] = a
    return out


def close_f32(ours, want):
    ours, want = np.asarray(ours, np.float64), np.asarray(want, np.float64)
    return np.abs(ours - want) <= 1e-6 + 1e-5 * np.abs(want)


CASES = [
    # (dtype, V, pad of the logits rows, pad of the mask rows) ; aligned when V and both strides are multiples of 8
    ("bf16", 50304, 64, 40),
    ("f32", 4099, 3, 5),
    ("bf16", 1000, 8, 8),
]


def make(dtype, V, rows, seed):
    rng = np.random.default_rng(seed)
    x = rng.normal(0, 2, (rows, V)).astype(np.float32)
    y = (x + rng.normal(0, 0.3, (rows, V))).astype(np.float32)
    keep = (rng.random((rows, V)) < 0.7).astype(np.uint8)
    keep[:, 0] = 1
    t = rng.integers(0, V, rows)
    tok = np.where(keep[np.arange(rows), t] == 1, t, 0).astype(np.int32)
    if dtype == "bf16":
        xb, yb = O.bf16_from_f32(x), O.bf16_from_f32(y)
        return O.bf16_to_f32(xb), O.bf16_to_f32(yb), xb, yb, keep, tok
    return x, y, x, y, keep, tok


def dev(a, dtype=None):
    return nr.Tensor.from_numpy(np.ascontiguousarray(a), dtype)


@pytest.mark.parametrize("case", CASES)
def test_sampler_reads_only_the_first_V_of_each_strided_row(case):
    dtype, V, xpad, mpad = case
    rows = 32
    x, _, xs, _, keep, _ = make(dtype, V, rows, V)
    nan = np.uint16(0x7fc0) if dtype == "bf16" else np.float32(np.nan)
    ld, mld = V + xpad, V + mpad
    xt = dev(padded(xs, ld, nan), dtype)
    mt = dev(padded(keep, mld, np.uint8(1)))  # a pad that "keeps" its NaN logits, were it read
    u = np.random.default_rng(1).random(rows)
    ut = dev(u, "f64")
    dt = nr.NT_BF16 if dtype == "bf16" else nr.NT_F32
    outs = []
    for stride_x, stride_m, xin, min_ in ((ld, mld, xt, mt), (V, V, dev(xs, dtype), dev(keep))):
        ids, lp, ent, st = nr.IntTensor((rows,)), nr.Tensor((rows,), "f32"), nr.Tensor((rows,), "f32"), nr.Tensor((rows,), "u8")
        a = nr.NtRlSampleArgs(xin.ptr, dt, nr.NT_MASK_U8, rows, V, stride_x, min_.ptr, stride_m, 0.7, ut.ptr, ids.ptr,
                              lp.ptr, ent.ptr, st.ptr)
        nr._check(nr.lib().nt_hip_rl_sample(C.byref(a)), "sample")
        outs.append([t.to_numpy() for t in (ids, lp, ent, st)])
    strided, dense = outs
    assert np.all(strided[3] == 0), "no row refused (a NaN pad read would refuse it)"
    z = O.tempered(x, 0.7, keep=keep)
    want_ids, edges = O.sample_invcdf(z, u)
    assert np.all((strided[0] == want_ids) | (edges < 1e-6))
    assert np.all(close_f32(strided[1], O.token_logp(z, strided[0])))
    assert np.all(close_f32(strided[2], O.entropy(z)))
    if V % 8 == 0 and ld % 8 == 0 and mld % 8 == 0:
        for s, d in zip(strided, dense):
            assert s.tobytes() == d.tobytes(), "aligned strides: the dense call's bits"


@pytest.mark.parametrize("case", CASES)
def test_scoring_and_backward_read_and_write_only_the_first_V(case):
    dtype, V, xpad, mpad = case
    rows = 24
    x, y, xs, ys, keep, tok = make(dtype, V, rows, V + 7)
    nan = np.uint16(0x7fc0) if dtype == "bf16" else np.float32(np.nan)
    ld, mld, gld = V + xpad, V + mpad, V + xpad + 8
    dt = nr.NT_BF16 if dtype == "bf16" else nr.NT_F32
    g = np.random.default_rng(V)
    g_lp, g_kl, g_h = (dev(g.normal(0, 1, rows).astype(np.float32)) for _ in range(3))
    tt = dev(tok)

    def run(stride, mstride, gstride, xin, yin, min_):
        f = lambda: nr.Tensor((rows,), "f32")
        lp, rlp, kl, ent, lb, lr, rlb, rlr = (f() for _ in range(8))
        st = nr.Tensor((rows,), "u8")
        a = nr.NtRlScoreArgs(xin.ptr, yin.ptr, dt, nr.NT_MASK_U8, rows, V, stride, min_.ptr, mstride, 1.3, tt.ptr,
                             lp.ptr, rlp.ptr, kl.ptr, ent.ptr, st.ptr, lb.ptr, lr.ptr, rlb.ptr, rlr.ptr)
        nr._check(nr.lib().nt_hip_rl_score(C.byref(a)), "score")
        grad = dev(np.full((rows, gstride), 7.5, np.float32))  # a sentinel the pads must keep
        b = nr.NtRlScoreGradArgs(xin.ptr, yin.ptr, dt, nr.NT_MASK_U8, rows, V, stride, min_.ptr, mstride, 1.3, tt.ptr,
                                 lb.ptr, lr.ptr, rlb.ptr, rlr.ptr, kl.ptr, ent.ptr, g_lp.ptr, g_kl.ptr, g_h.ptr,
                                 grad.ptr, nr.NT_F32, 0, gstride)
        nr._check(nr.lib().nt_hip_rl_score_backward(C.byref(b)), "score backward")
        return [t.to_numpy() for t in (lp, rlp, kl, ent, st)], grad.to_numpy().reshape(rows, gstride)

    s_out, s_grad = run(ld, mld, gld, dev(padded(xs, ld, nan), dtype), dev(padded(ys, ld, nan), dtype),
                        dev(padded(keep, mld, np.uint8(1))))
    d_out, d_grad = run(V, V, V, dev(xs, dtype), dev(ys, dtype), dev(keep))
    assert np.all(s_out[4] == 0), "no row refused (a NaN pad read would refuse it)"
    assert np.all(s_grad[:, V:] == 7.5), "the gradient's pads are untouched"
    assert np.all(np.isfinite(s_grad[:, :V]))
    z, r = O.tempered(x, 1.3, keep=keep), O.tempered(y, 1.3, keep=keep)
    for name, got, want in (("logp", s_out[0], O.token_logp(z, tok)), ("ref_logp", s_out[1], O.token_logp(r, tok)),
                            ("kl", s_out[2], O.kl(z, r)), ("entropy", s_out[3], O.entropy(z))):
        assert np.all(close_f32(got, want)), name
    want_g = O.score_grad(z, tok, r, g_lp.to_numpy(), g_kl.to_numpy(), g_h.to_numpy(), 1.3)
    scale = np.abs(want_g).max(axis=1, keepdims=True)
    assert np.all(np.abs(s_grad[:, :V] - want_g) <= 1e-5 * scale + 1e-12)
    if V % 8 == 0 and ld % 8 == 0 and mld % 8 == 0 and gld % 8 == 0:
        for s, d in zip(s_out, d_out):
            assert s.tobytes() == d.tobytes(), "aligned strides: the dense call's bits"
        assert s_grad[:, :V].tobytes() == d_grad.tobytes()


def test_entry_points_from_several_threads():
    """Every device entry point takes the one process-wide lock (the reference's Mutex<Ctx>), so
    host threads calling the sampler and the scorer at once get the results of calling them one
    after another."""
    import threading
    rng = np.random.default_rng(77)
    rows, V = 40, 5000
    jobs = []
    for k in range(6):
        x = rng.normal(0, 2, (rows, V)).astype(np.float32)
        tok = rng.integers(0, V, rows).astype(np.int32)
        jobs.append((dev(x), dev(tok), dev(rng.random(rows), "f64")))

    def run(job):
        xt, tt, ut = job
        ids, lp, ent = nr.sample_logp(xt, 0.9, None, None, entropy=True, uniforms=ut)
        slp, _, _, sent = nr.score(xt, None, tt)
        return [a.to_numpy().tobytes() for a in (ids, lp, ent, slp, sent)]

    want = [run(j) for j in jobs]
    got = [None] * len(jobs)

    def worker(i):
        for _ in range(5):
            got[i] = run(jobs[i])

    th = [threading.Thread(target=worker, args=(i,)) for i in range(len(jobs))]
    for t in th:
        t.start()
    for t in th:
        t.join()
    assert got == want
