"""GPU tests of the row kernels' run-time path: the same calls through the ahead-of-time code
objects and through hiprtc (compiled at first use from the embedded source, loaded with
hipModuleLoadData) give byte-identical ids, log-probabilities and entropies (C4 among them, with
its oracle parity), and byte-identical scores, saved statistics and gradients from the scorer and
its fused backward (C3's rows among them, the gradient with its oracle parity); the provenance key
names the path; a second process loads the compiled code objects from the disk cache instead of
compiling."""
import os
import subprocess
import sys
import time

import numpy as np
import pytest

import noetic_rl as nr
import workloads as W
from oracle import oracle as O
from tests.test_rl_gpu import check_sample
from tests.test_score_grad_gpu import compare_to_oracle, upstream

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module", autouse=True)
def device(tmp_path_factory):
    cache = str(tmp_path_factory.mktemp("rtc_cache"))
    old = os.environ.get("NOETIC_HIP_CACHE_DIR")
    os.environ["NOETIC_HIP_CACHE_DIR"] = cache
    nr.claim(0)
    prev = nr.set_kernel_path("aot")
    yield cache
    nr.set_kernel_path(prev)
    if old is None:
        os.environ.pop("NOETIC_HIP_CACHE_DIR", None)
    else:
        os.environ["NOETIC_HIP_CACHE_DIR"] = old


def both_paths(fn):
    """fn() through the ahead-of-time kernels, then twice through hiprtc (compile, then the
    process's cached function); returns the three results as byte strings."""
    out = []
    for path in ("aot", "rtc", "rtc"):
        nr.set_kernel_path(path)
        try:
            t = time.perf_counter()
            res = fn()
            nr.sync()
            print(f"  {path}: {1e3 * (time.perf_counter() - t):.1f} ms", flush=True)
        finally:
            nr.set_kernel_path("aot")
        out.append([r.to_numpy().tobytes() for r in res])
    return out


def test_c4_parity_and_rerun_bits_through_both_paths():
    w = W.c4()
    rows, V = w["rows"], w["V"]
    u = nr.Rng(2024, "c4/uniforms").uniforms(rows)
    ut = nr.Tensor.from_numpy(u, "f64")
    aot, rtc1, rtc2 = both_paths(lambda: nr.sample_logp(w["logits"], w["temperature"], w["mask"], None, uniforms=ut))
    assert rtc1 == aot and rtc2 == aot, "hiprtc and hipcc code objects disagree"
    ids, lp = nr.sample_logp(w["logits"], w["temperature"], w["mask"], None, uniforms=ut)
    ids, lp = ids.to_numpy().ravel(), lp.to_numpy().ravel()
    assert ids.tobytes() == aot[0] and lp.tobytes() == aot[1], "rerun bits"
    x = W.bf16_to_f32(w["logits"].to_numpy().reshape(rows, V))
    keep = w["mask"].to_numpy().reshape(rows, V)
    z = O.tempered(x, w["temperature"], keep=keep)
    check_sample("c4 (aot = rtc)", z, u, ids, lp, bf16=False)


@pytest.mark.parametrize("case", ["c2_f32_entropy", "seg_bf16_16rows", "stream_unaligned_f32", "queued_shared_mask",
                                  "stream_f32_mask_bf16"])
def test_each_sampler_kernel_is_byte_identical_through_both_paths(case):
    """One call per kernel family: the register-resident sampler with entropy (C2), the segmented
    sampler (16 rows of V = 128256), the streaming sampler (unaligned rows, and aligned bf16 rows
    under an f32 mask, whose words it stages through LDS), and the queued sampler's instance for a
    mask row shared by every row (C4's shape, 128 rows)."""
    rng = np.random.default_rng(7)
    if case == "c2_f32_entropy":
        w = W.c2()
        rows, xt, mt, tau = w["rows"], w["logits"], None, w["temperature"]
    elif case == "seg_bf16_16rows":
        rows, V = 16, 128256
        xt = nr.Tensor.from_numpy(O.bf16_from_f32(rng.normal(0, 2, (rows, V)).astype(np.float32)), "bf16")
        mt = nr.Tensor.from_numpy((rng.random((rows, V)) < 0.9).astype(np.uint8))
        tau = 0.7
    elif case == "queued_shared_mask":
        w = W.c4(seed=13, rows=128, shared_mask=True)
        rows, xt, mt, tau = w["rows"], w["logits"], w["mask"], w["temperature"]
    elif case == "stream_f32_mask_bf16":
        rows, V = 80, 40000
        xt = nr.Tensor.from_numpy(O.bf16_from_f32(rng.normal(0, 2, (rows, V)).astype(np.float32)), "bf16")
        add = np.where(rng.random((rows, V)) < 0.4, -np.inf, rng.normal(0, 0.5, (rows, V))).astype(np.float32)
        add[:, 3] = 0.0
        mt = nr.Tensor.from_numpy(add)
        tau = 0.8
    else:
        rows, V = 33, 1001
        xt = nr.Tensor.from_numpy(rng.normal(0, 3, (rows, V)).astype(np.float32))
        mt = None
        tau = 1.0
    u = nr.Tensor.from_numpy(nr.Rng(11, case).uniforms(rows), "f64")
    aot, rtc1, rtc2 = both_paths(lambda: nr.sample_logp(xt, tau, mt, None, entropy=True, uniforms=u))
    assert rtc1 == aot and rtc2 == aot, f"{case}: hiprtc and hipcc code objects disagree"
    if case == "queued_shared_mask":
        # the shared row read through the caches gives the bits of the same mask materialised per
        # row (each row's own mask, read non-temporal)
        full = nr.Tensor.from_numpy(np.ascontiguousarray(np.broadcast_to(mt.to_numpy(), (1, rows, 1, mt.shape[-1]))))
        got = nr.sample_logp(xt, tau, full, None, entropy=True, uniforms=u)
        assert [t.to_numpy().tobytes() for t in got] == aot, "shared and materialised masks differ"


@pytest.mark.parametrize("case", ["c3_bf16_aligned", "f32_masked_tempered_unaligned"])
def test_scorer_and_backward_are_byte_identical_through_both_paths(case):
    """k_score (logp, the reference's logp, exact KL, entropy and the log-sum-exp statistics it
    saves) and k_score_grad (f32 and bf16 gradients of g_logp logp + g_kl KL + g_H H): C3's bf16
    rows with the reference (the buffer-resource kernels), and f32 rows of V = 1001 under a u8 mask
    and a temperature (the general kernels)."""
    rng = np.random.default_rng(5)
    if case == "c3_bf16_aligned":
        w = W.c3(rows=64)
        rows, tau = w["rows"], 1.0
        pol, ref, tok = w["logits"], w["ref"], w["tokens"]
        z = W.bf16_to_f32(pol.to_numpy())
        r = W.bf16_to_f32(ref.to_numpy())
    else:
        rows, V, tau = 40, 1001, 0.8
        x = rng.normal(0, 3, (rows, V)).astype(np.float32)
        y = (x + rng.normal(0, 0.5, (rows, V))).astype(np.float32)
        keep = (rng.random((rows, V)) < 0.8).astype(np.uint8)
        keep[:, 0] = 1
        tokens = np.array([rng.choice(np.nonzero(keep[i])[0]) for i in range(rows)], np.int32)
        mt = nr.Tensor.from_numpy(keep)
        pol = nr.tempered_logits(nr.Tensor.from_numpy(x), tau, mt)
        ref = nr.tempered_logits(nr.Tensor.from_numpy(y), tau, mt)
        tok = nr.Tensor.from_numpy(tokens)
        z, r = O.tempered(x, tau, keep=keep), O.tempered(y, tau, keep=keep)
    g = upstream(rows, 9)
    gt = {k: nr.Tensor.from_numpy(v) for k, v in g.items()}

    def call():
        lp, rlp, kl, ent, st = nr.score_with_stats(pol, ref, tok)
        out = [lp, rlp, kl, ent, st.lse_base, st.lse_rest, st.ref_lse_base, st.ref_lse_rest]
        for gdt in ("f32", "bf16"):
            out.append(nr.score_grad(pol, ref, tok, st, kl=kl, entropy=ent, g_logp=gt["g_lp"], g_kl=gt["g_kl"],
                                     g_entropy=gt["g_h"], grad_dtype=gdt))
        return out

    aot, rtc1, rtc2 = both_paths(call)
    names = ["logp", "ref_logp", "kl", "entropy", "lse_base", "lse_rest", "ref_lse_base", "ref_lse_rest",
             "grad f32", "grad bf16"]
    for i, n in enumerate(names):
        assert rtc1[i] == aot[i] and rtc2[i] == aot[i], f"{case}: {n} differs between hiprtc and hipcc code objects"
    kl = np.frombuffer(aot[2], np.float32)
    ent = np.frombuffer(aot[3], np.float32)
    gf = np.frombuffer(aot[8], np.float32).reshape(z.shape)
    gb = np.frombuffer(aot[9], np.uint16).reshape(z.shape)
    compare_to_oracle(f"{case} (aot = rtc)", z, r, tok.to_numpy(), g, kl, ent, tau, gf, gb)


@pytest.mark.parametrize("pre_u32", [0, 1])
def test_gumbel_sampler_is_byte_identical_through_both_paths(pre_u32):
    """The reference's Gumbel-max sampler on C4's rows (the aligned, screened path at an even
    stream position; the element-wise path at an odd one), through both paths."""
    w = W.c4()

    def call():
        rng = nr.Rng(5, "rtc/gumbel")
        for _ in range(pre_u32):
            rng.next_u32()
        return [nr.sample_categorical(w["logits"], w["temperature"], w["mask"], rng)]

    aot, rtc1, rtc2 = both_paths(call)
    assert rtc1 == aot and rtc2 == aot, "hiprtc and hipcc code objects disagree"


def test_key_names_the_path():
    k_aot = nr.key()
    nr.set_kernel_path("rtc")
    try:
        k_rtc = nr.key()
    finally:
        nr.set_kernel_path("aot")
    assert "hiprtc" not in k_aot and "-hiprtc" in k_rtc, (k_aot, k_rtc)
    assert k_aot != k_rtc


CHILD = r"""
import os, sys, time
sys.path[:0] = [os.path.join(sys.argv[1], "noetic-tensor_amd"), sys.argv[1]]
import numpy as np
import noetic_rl as nr
import workloads as W
nr.claim(0)
nr.set_kernel_path("rtc")
w = W.c4()
ut = nr.Tensor.from_numpy(nr.Rng(2024, "c4/uniforms").uniforms(w["rows"]), "f64")
t = time.perf_counter()
ids, lp = nr.sample_logp(w["logits"], w["temperature"], w["mask"], None, uniforms=ut)
nr.sync()
dt = time.perf_counter() - t
sys.stdout.write(f"{dt:.4f} {ids.to_numpy().tobytes().hex()} {lp.to_numpy().tobytes().hex()}\n")
"""


def test_a_second_process_loads_the_code_objects_from_the_disk_cache(device):
    # the C4 test above compiled the C4 instance into the cache directory
    files = [f for f in os.listdir(device) if f.endswith(".co")]
    assert files, "no code object was written to the cache"
    w = W.c4()
    ut = nr.Tensor.from_numpy(nr.Rng(2024, "c4/uniforms").uniforms(w["rows"]), "f64")
    ids, lp = nr.sample_logp(w["logits"], w["temperature"], w["mask"], None, uniforms=ut)
    env = dict(os.environ, NOETIC_HIP_CACHE_DIR=device)
    r = subprocess.run([sys.executable, "-c", CHILD, ROOT], env=env, capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr[-2000:]
    dt, ids_hex, lp_hex = r.stdout.split()
    print(f"  second process, first C4 call from the cache: {1e3 * float(dt):.1f} ms")
    assert bytes.fromhex(ids_hex) == ids.to_numpy().tobytes()
    assert bytes.fromhex(lp_hex) == lp.to_numpy().tobytes()
    # compiling takes seconds; loading the cached code object takes well under one
    assert float(dt) < 1.0
    assert len([f for f in os.listdir(device) if f.endswith(".co")]) == len(files)
