"""The allocation-free sampler entry point, nt_hip_rl_sample_noalloc, through the C ABI against
nt_hip_rl_sample on the same inputs: the same kernels, so every output byte is equal. Two calls
in a row, the second with a smaller input, at shapes that take the segmented sampler (whose
workspace is the fixed device array); the same with the library on its run-time (hiprtc) kernel
path, where the entry still launches the ahead-of-time code objects and the device's free memory
does not change over warm calls; and a launch needing more than that array is refused before
anything runs."""
import ctypes as C

import numpy as np
import pytest

import noetic_rl as nr
import workloads as W

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def device():
    nr.claim(0)
    yield


def run(entry, x, dt, mk, m, rows, V, tau, U, entropy):
    ids, lp, st = nr.IntTensor((rows,)), nr.Tensor((rows,), "f32"), nr.Tensor((rows,), "u8")
    ent = nr.Tensor((rows,), "f32") if entropy else None
    a = nr.NtRlSampleArgs(x.ptr, dt, mk, rows, V, V, None if m is None else m.ptr, 0 if m is None else V, tau,
                          U.ptr, ids.ptr, lp.ptr, None if ent is None else ent.ptr, st.ptr)
    rc = getattr(nr.lib(), entry)(C.byref(a))
    assert rc == 0, nr.lib().nt_hip_last_error()
    nr.sync()
    out = [ids.to_numpy().tobytes(), lp.to_numpy().tobytes(), st.to_numpy().tobytes()]
    if ent is not None:
        out.append(ent.to_numpy().tobytes())
    return out


def test_noalloc_equals_the_allocating_entry_on_two_calls():
    # call 1: C4's row shape at 64 rows (bf16 V = 128256, u8 grammar mask, T 0.7): segments of
    # 8 waves x 4 chunks; call 2, smaller: 8 unmasked f32 rows of V = 50304 with the entropy
    w = W.c4(rows=64)
    U = nr.Tensor.from_numpy(nr.Rng(1, "noalloc/u").uniforms(64), "f64")
    args = (w["logits"], nr.NT_BF16, nr.NT_MASK_U8, w["mask"], 64, w["V"], w["temperature"], U, False)
    first = [run(e, *args) for e in ("nt_hip_rl_sample_noalloc", "nt_hip_rl_sample")]
    assert first[0] == first[1]
    assert np.all(np.frombuffer(first[0][2], np.uint8) == 0)
    x2 = W.normal((8, 50304), "f32", 5, "noalloc/f32")
    U2 = nr.Tensor.from_numpy(nr.Rng(2, "noalloc/u").uniforms(8), "f64")
    args2 = (x2, nr.NT_F32, nr.NT_MASK_NONE, None, 8, 50304, 0.8, U2, True)
    second = [run(e, *args2) for e in ("nt_hip_rl_sample_noalloc", "nt_hip_rl_sample")]
    assert second[0] == second[1]
    assert np.all(np.frombuffer(second[0][2], np.uint8) == 0)
    # and the first shape again, after the smaller call: the workspace's counters were left at zero
    again = run("nt_hip_rl_sample_noalloc", *args)
    assert again == first[1]


def test_noalloc_refuses_a_launch_beyond_its_workspace(monkeypatch):
    # 4096 rows forced into segments of 8 waves x 4 chunks need 4096 x 64 records x 48 bytes of
    # workspace (12.6 MB), more than the fixed 2 MiB: refused before any launch. The buffers are
    # never read: the refusal comes first.
    monkeypatch.setenv("NOETIC_HIP_SAMPLE_SEG", "8,4")
    buf = nr.Buffer(1 << 20)
    a = nr.NtRlSampleArgs(buf.ptr, nr.NT_BF16, nr.NT_MASK_NONE, 4096, 128256, 128256, None, 0, 0.7, buf.ptr,
                          buf.ptr, buf.ptr, None, buf.ptr)
    before = nr.launches()
    assert nr.lib().nt_hip_rl_sample_noalloc(C.byref(a)) == -1  # NT_E_ARG
    assert "allocation-free maximum" in nr.lib().nt_hip_last_error().decode()
    assert nr.launches() == before


def test_noalloc_on_the_run_time_kernel_path_allocates_nothing():
    # with the library on the hiprtc path, the allocation-free entry still launches the
    # ahead-of-time code objects (a hiprtc instance's first launch compiles and loads a code
    # object, which allocates): its outputs equal the allocating entry's on that path, and after a
    # first call the device's free memory is the same across further calls
    hip = C.CDLL("libamdhip64.so")
    hip.hipMemGetInfo.argtypes = [C.POINTER(C.c_size_t), C.POINTER(C.c_size_t)]

    def free_bytes():
        nr.sync()
        f, t = C.c_size_t(), C.c_size_t()
        assert hip.hipMemGetInfo(C.byref(f), C.byref(t)) == 0
        return f.value

    prev = nr.lib().nt_hip_set_kernel_path(1)  # NT_KERNELS_RTC
    try:
        w = W.c4(seed=3, rows=48)
        U = nr.Tensor.from_numpy(nr.Rng(3, "noalloc/rtc").uniforms(48), "f64")
        x2 = W.normal((8, 50304), "f32", 6, "noalloc/rtc/f32")
        U2 = nr.Tensor.from_numpy(nr.Rng(4, "noalloc/rtc").uniforms(8), "f64")
        calls = [(w["logits"], nr.NT_BF16, nr.NT_MASK_U8, w["mask"], 48, w["V"], 0.7, U, False),
                 (x2, nr.NT_F32, nr.NT_MASK_NONE, None, 8, 50304, 0.8, U2, True)]
        outs = [run("nt_hip_rl_sample_noalloc", *c) for c in calls]  # first calls
        before = free_bytes()
        for _ in range(3):
            for c, o in zip(calls, outs):
                assert run("nt_hip_rl_sample_noalloc", *c) == o
        assert free_bytes() == before, "device memory allocated by warm allocation-free calls"
        for c, o in zip(calls, outs):
            assert run("nt_hip_rl_sample", *c) == o  # the allocating entry on the hiprtc path: the same bytes
    finally:
        nr.lib().nt_hip_set_kernel_path(prev)
