"""CPU tests of the C ABI: libnoetic_hip.so loads, exports every symbol include/*.h declares,
fails cleanly without a GPU, and its host-side stream (the sampler's uniforms) equals the
oracle's restatement of rng::derive / ChaCha20Rng."""
import ctypes as C
import glob
import os
import re
import struct

import numpy as np
import pytest

import noetic_rl as nr
from oracle import oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"^\s*[A-Za-z_][\w\s\*]*?\b(nt_\w+)\s*\(", text, flags=re.M):
            names.add(m.group(1))
    return names


def test_library_exports_every_declared_symbol():
    names = declared_symbols()
    assert {"nt_hip_claim", "nt_hip_rl_sample", "nt_hip_rl_score", "nt_rng_derive"} <= names
    L = C.CDLL(nr.LIB_PATH)
    missing = [n for n in sorted(names) if not hasattr(L, n)]
    assert not missing, missing
    # the Python binding declares a signature for each of them
    assert names <= set(nr._SIGS), sorted(names - set(nr._SIGS))


def test_argument_struct_layouts_match_the_header():
    """The ctypes mirrors of the argument structs have the C header's sizes and field offsets
    (the header compiled by gcc on this host; a Rust #[repr(C)] binding asserts the same)."""
    import subprocess
    import tempfile
    fields = {"NtRlSampleArgs": [f[0] for f in nr.NtRlSampleArgs._fields_],
              "NtRlScoreArgs": [f[0] for f in nr.NtRlScoreArgs._fields_],
              "NtRlScoreGradArgs": [f[0] for f in nr.NtRlScoreGradArgs._fields_],
              "NtRlPolicyLossArgs": [f[0] for f in nr.NtRlPolicyLossArgs._fields_],
              "NtRlGumbelArgs": [f[0] for f in nr.NtRlGumbelArgs._fields_],
              "NtRlReadoutSampleArgs": [f[0] for f in nr.NtRlReadoutSampleArgs._fields_],
              "NtRlReadoutScoreArgs": [f[0] for f in nr.NtRlReadoutScoreArgs._fields_]}
    body = []
    for st, fs in fields.items():
        body.append(f'printf("{st} %zu\\n", sizeof({st}));')
        body += [f'printf("{st}.{f} %zu\\n", offsetof({st}, {f}));' for f in fs]
    src = ("#include <stdio.h>\n#include <stddef.h>\n#include \"noetic_hip.h\"\nint main(void) {\n"
           + "\n".join(body) + "\nreturn 0;\n}\n")
    with tempfile.TemporaryDirectory() as d:
        c, exe = os.path.join(d, "layout.c"), os.path.join(d, "layout")
        open(c, "w").write(src)
        subprocess.run(["gcc", "-I", os.path.join(ROOT, "include"), c, "-o", exe], check=True)
        out = subprocess.run([exe], check=True, capture_output=True, text=True).stdout.split("\n")
    got = dict(line.split() for line in out if line)
    for st, fs in fields.items():
        cls = getattr(nr, st)
        assert int(got[st]) == C.sizeof(cls), st
        for f in fs:
            assert int(got[f"{st}.{f}"]) == getattr(cls, f).offset, (st, f)
    assert int(got["NtRlSampleArgs"]) == 136 and int(got["NtRlScoreArgs"]) == 184
    assert int(got["NtRlScoreGradArgs"]) == 208 and int(got["NtRlPolicyLossArgs"]) == 120
    assert int(got["NtRlGumbelArgs"]) == 160 and int(got["NtRlReadoutSampleArgs"]) == 136
    assert int(got["NtRlReadoutScoreArgs"]) == 120


def test_without_a_claimed_device_calls_fail_cleanly():
    L = nr.lib()
    if L.nt_hip_device_count() > 0:
        pytest.skip("a GPU is visible: the no-device path is not reachable here")
    assert L.nt_hip_claim(0) != 0
    assert b"device" in L.nt_hip_last_error().lower()
    p = C.c_void_p()
    assert L.nt_hip_alloc(16, C.byref(p)) == -2  # NT_E_UNCLAIMED
    a = nr.NtRlSampleArgs()
    assert L.nt_hip_rl_sample(C.byref(a)) == -1  # NT_E_ARG: null logits / rows checked first
    with pytest.raises(nr.HipUnavailable):
        nr.claim(0)


def test_argument_validation_precedes_the_device():
    L = nr.lib()
    a = nr.NtRlSampleArgs(None, nr.NT_BF16, nr.NT_MASK_U8, 4, 16, 16, None, 0, 1.0, None, None, None, None, None)
    assert L.nt_hip_rl_sample(C.byref(a)) == -1  # a u8 mask kind without a mask
    assert b"mask" in L.nt_hip_last_error()
    a = nr.NtRlSampleArgs(None, nr.NT_F32, nr.NT_MASK_NONE, 4, 16, 16, None, 0, -1.0, None, None, None, None, None)
    assert L.nt_hip_rl_sample(C.byref(a)) == -1
    assert "temperature" in L.nt_hip_last_error().decode()
    # the backward: each upstream gradient needs the forward outputs it multiplies
    buf = np.zeros(64, np.float32)
    h = buf.ctypes.data
    g = nr.NtRlScoreGradArgs(logits=h, dtype=nr.NT_F32, mask_kind=nr.NT_MASK_NONE, rows=4, vocab=16, ld=16,
                             temperature=1.0, lse_base=h, lse_rest=h, g_logp=h, grad=h, grad_dtype=nr.NT_F32,
                             grad_ld=16)
    assert L.nt_hip_rl_score_backward(C.byref(g)) == -1
    assert "g_logp needs tokens" in L.nt_hip_last_error().decode()
    g.g_logp, g.g_kl, g.kl = None, h, h
    assert L.nt_hip_rl_score_backward(C.byref(g)) == -1
    assert "g_kl needs ref_logits" in L.nt_hip_last_error().decode()
    g.g_kl, g.grad_dtype = None, 7
    assert L.nt_hip_rl_score_backward(C.byref(g)) == -1
    assert "grad dtype" in L.nt_hip_last_error().decode()
    g.grad_dtype, g.grad_ld = nr.NT_BF16, 8
    assert L.nt_hip_rl_score_backward(C.byref(g)) == -1
    assert "grad_ld" in L.nt_hip_last_error().decode()
    # the policy losses check Clip::check's ranges (rl.rs:189-200) before the device
    pl = nr.NtRlPolicyLossArgs(logp=h, old_logp=h, weights=h, S=1, B=1, T=4, kind=nr.NT_LOSS_PPO, clip_low=1.0,
                               clip_high=0.2, log_ratio_clamp=20.0)
    assert L.nt_hip_rl_policy_loss(C.byref(pl)) == -1
    assert "need 0 ≤ low < 1" in L.nt_hip_last_error().decode()
    pl.clip_low, pl.dual = 0.2, 0.5
    assert L.nt_hip_rl_policy_loss(C.byref(pl)) == -1
    assert "dual clip 0.5 (need c > 1)" in L.nt_hip_last_error().decode()
    pl.dual, pl.log_ratio_clamp = 0.0, -1.0
    assert L.nt_hip_rl_policy_loss(C.byref(pl)) == -1
    assert "log-ratio clamp" in L.nt_hip_last_error().decode()
    pl.log_ratio_clamp, pl.old_logp = 20.0, None
    assert L.nt_hip_rl_policy_loss(C.byref(pl)) == -1
    with pytest.raises(ValueError, match="need c > 1"):
        nr.Clip.symmetric(0.2).with_dual(1.0).check()
    # group_advantages' refusals (rl.rs:437-441)
    assert L.nt_hip_rl_group_advantages(h, 2, 1, 1, 1e-6, 1, h) == -1
    assert "needs groups of at least 2" in L.nt_hip_last_error().decode()
    assert L.nt_hip_rl_group_advantages(h, 2, 2, 1, -1.0, 0, h) == -1
    assert "< 0" in L.nt_hip_last_error().decode()


def test_product_stream_equals_the_oracle_stream():
    for root, label in [(5, "sampler test"), (0, "x"), (2 ** 63 + 11, "device sampler"), (7, "")]:
        a, b = nr.Rng(root, label), O.Rng(root, label)
        assert [a.next_u64() for _ in range(100)] == [b.next_u64() for _ in range(100)]
        a.next_u32()
        b.next_u32()
        assert np.array_equal(a.uniforms(1000), b.uniforms(1000))
    # from_seed(0) is the RFC 8439 A.1 keystream
    r = nr.NtRng()
    assert nr.lib().nt_rng_from_seed(C.byref(r), bytes(32)) == 0
    words = [nr.lib().nt_rng_next_u32(C.byref(r)) for _ in range(16)]
    assert struct.pack("<16I", *words).hex().startswith("76b8e0ada0f13d90405d6ae55386bd28")
    out = C.create_string_buffer(32)
    nr.lib().nt_sha256(b"abc", 3, out)
    assert out.raw.hex() == "ba7816bf8f01cfea414140de5dae2223b00361a396177a9cb410ff61f20015ad"


def test_stream_positions_and_skips_equal_the_draws():
    # nt_rng_word_pos / set_word_pos / skip_u64 (rand_chacha's get_word_pos / set_word_pos): the
    # Gumbel sampler generates its draws at the stream's position and then advances the stream by
    # one u64 per logit (src/nn/tests/rl.rs:596-599); that must equal drawing them one by one,
    # from every word offset inside a block (odd offsets after a next_u32 included)
    for pre in range(0, 17):
        for n in (0, 1, 7, 8, 9, 63, 64, 65, 1000, 12345):
            a, b = nr.Rng(3, "skip"), nr.Rng(3, "skip")
            for _ in range(pre):
                a.next_u32()
                b.next_u32()
            blk, word = a.word_pos()
            assert 16 * blk + word == pre
            a.skip_u64(n)
            for _ in range(n):
                b.next_u64()
            assert a.word_pos() == b.word_pos()
            assert [a.next_u64() for _ in range(5)] == [b.next_u64() for _ in range(5)], (pre, n)
    r = nr.Rng(4, "pos")
    assert nr.lib().nt_rng_set_word_pos(C.byref(r.s), 1000, 5) == 0
    assert r.word_pos() == (1000, 5)
    w = O.chacha_block(list(r.s.key), 1000)
    assert r.next_u32() == w[5] and r.next_u64() == w[6] | (w[7] << 32)
    assert nr.lib().nt_rng_set_word_pos(C.byref(r.s), 0, 16) == -1


def test_gumbel_sampler_arguments_are_checked_before_the_device():
    L = nr.lib()
    a = nr.NtRlGumbelArgs(None, nr.NT_F32, nr.NT_MASK_NONE, 4, 16, 16, None, 0, 1.0)
    a.word = 16
    assert L.nt_hip_rl_sample_gumbel(C.byref(a)) == -1
    assert b"word" in L.nt_hip_last_error()
    a.word, a.temperature = 0, float("nan")
    assert L.nt_hip_rl_sample_gumbel(C.byref(a)) == -1
    assert "temperature" in L.nt_hip_last_error().decode()


def test_runs_mask_generator_host():
    rows, V = 16, 4096
    out = np.empty(rows * V, dtype=np.uint8)
    lab = b"c4/mask"
    rc = nr.lib().nt_synth_runs_mask_host(out.ctypes.data_as(C.c_void_p), rows, V, 2024, lab, len(lab), 96, 224)
    assert rc == 0
    m = out.reshape(rows, V)
    assert set(np.unique(m)) <= {0, 1} and m.sum(1).min() >= 1
    frac = m.mean()
    assert 0.2 < frac < 0.4, frac  # kept runs of mean 96 between gaps of mean 224: about 30%
    out2 = np.empty_like(out)
    nr.lib().nt_synth_runs_mask_host(out2.ctypes.data_as(C.c_void_p), rows, V, 2024, lab, len(lab), 96, 224)
    assert np.array_equal(out, out2)


def test_python_mirror_refuses_like_the_reference_without_a_device():
    with pytest.raises(ValueError, match="temperature"):
        nr.tempered_logits(None, 0.0, None)
    with pytest.raises(ValueError, match="at least 2"):
        nr.group_advantages([1.0, 2.0], 1, "std", 1e-6, True)
    assert nr.group_advantages([1, 0, 0, 1, 2, 2, 2, 2], 4).tolist() == [0.5, -0.5, -0.5, 0.5, 0, 0, 0, 0]


def test_group_norm_forms_agree():
    r = [1.0, 0.0, 0.0, 1.0, 2.0, 2.0, 2.0, 2.0, 0.0, 0.0, 0.0, 3.0]
    assert nr.group_advantages(r, 4, nr.GroupNorm.MEAN_ONLY).tolist() == nr.group_advantages(r, 4, "mean").tolist()
    a = nr.group_advantages(r, 4, nr.GroupNorm.std(1e-2, True))
    assert a.tolist() == nr.group_advantages(r, 4, "std", 1e-2, True).tolist()
    with pytest.raises(ValueError, match="at least 2"):
        nr.group_advantages([1.0, 2.0], 1, nr.GroupNorm.std(1e-6, True))


def test_bench_refuses_more_than_one_gpu_before_touching_a_device():
    import json
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    p = subprocess.run([sys.executable, os.path.join(root, "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert p.returncode == 2
    msg = json.loads(p.stdout.strip().splitlines()[-1])
    assert "one GPU" in msg["error"]


def test_mask_groups_fold():
    """The host's folding of a broadcast mask's leading dimensions into (rows, mask stride) groups,
    the rows -> mask-row map it hands the kernels (NtMaskRows)."""
    g = nr.mask_groups
    V = 10
    assert g((3, 4, 5, V), (3, 4, 5, V)) == [(60, V)]
    assert g((3, 4, 5, V), (1, 1, 1, V)) == [(60, 0)]
    assert g((3, 4, 5, V), (3, 1, 1, V)) == [(3, V), (20, 0)]
    assert g((2, 3, 4, V), (1, 3, 1, V)) == [(2, 0), (3, V), (4, 0)]
    assert g((2, 3, 4, V), (2, 1, 4, V)) == [(2, 4 * V), (3, 0), (4, V)]
    assert g((2, 2, 2, 2, V), (2, 1, 2, 1, V)) == [(2, 2 * V), (2, 0), (2, V), (2, 0)]
    assert g((1, 4, 1, V), (1, 4, 1, V)) == [(4, V)]


def test_broadcast_mask_map_is_checked_before_the_device():
    """NtMaskRows is validated before anything touches a device: rows a whole number of T B
    groups, each stride 0 or at least the vocabulary; a logits dtype outside f32, bf16 and f16
    is refused."""
    L = nr.lib()
    buf = np.zeros(64, np.uint8)
    h = buf.ctypes.data
    base = dict(logits=h, dtype=nr.NT_F32, mask_kind=nr.NT_MASK_U8, rows=12, vocab=16, ld=16, mask=h, mask_ld=16,
                temperature=1.0, uniforms=h, ids=h, status=h)
    cases = [
        (nr.NtMaskRows(5, 1, 0, 0), "rows a multiple"),   # 12 rows are not whole groups of 5
        (nr.NtMaskRows(3, 2, 8, 0), "strides 0 or at least vocab"),
        (nr.NtMaskRows(3, 2, 16, 8), "strides 0 or at least vocab"),
        (nr.NtMaskRows(0, 2, 16, 0), "mask rows T 0"),
    ]
    for mr, msg in cases:
        a = nr.NtRlSampleArgs(**base, mask_rows=mr)
        assert L.nt_hip_rl_sample(C.byref(a)) == -1, mr
        assert msg in L.nt_hip_last_error().decode()
        s = nr.NtRlScoreArgs(logits=h, dtype=nr.NT_F32, mask_kind=nr.NT_MASK_U8, rows=12, vocab=16, ld=16, mask=h,
                             mask_ld=16, temperature=1.0, status=h, mask_rows=mr)
        assert L.nt_hip_rl_score(C.byref(s)) == -1
        assert msg in L.nt_hip_last_error().decode()
    a = nr.NtRlSampleArgs(**dict(base, dtype=3))
    assert L.nt_hip_rl_sample(C.byref(a)) == -1
    assert "dtype 3" in L.nt_hip_last_error().decode()
