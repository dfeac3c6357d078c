"""CPU tests of the row kernels' run-time path (hiprtc: the samplers, the scorer and its backward):
the path switch needs no device, and hiprtc compiles the embedded device source into a gfx950 code
object here, without a GPU, with the program text and options the library passes (rtc.cpp)."""
import ctypes as C
import os

import pytest

import noetic_rl as nr

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "noetic-tensor_amd", "csrc")

# The files the library embeds, under the names the program includes them by (Makefile: RTC_SRC).
EMBEDDED = {
    "noetic_hip.h": os.path.join(ROOT, "include", "noetic_hip.h"),
    "nt_rows.hpp": os.path.join(CSRC, "nt_rows.hpp"),
    "rl_sample_kernels.hpp": os.path.join(CSRC, "rl_sample_kernels.hpp"),
    "rl_score_kernels.hpp": os.path.join(CSRC, "rl_score_kernels.hpp"),
    "nt_chacha.hpp": os.path.join(CSRC, "nt_chacha.hpp"),
    "rl_gumbel_kernels.hpp": os.path.join(CSRC, "rl_gumbel_kernels.hpp"),
}
PROGRAM = (b'#include "rl_sample_kernels.hpp"\n#include "rl_score_kernels.hpp"\n'
           b'#include "rl_gumbel_kernels.hpp"\n')
OPTIONS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-ffp-contract=off",
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def test_kernel_path_switch_needs_no_device():
    prev = nr.set_kernel_path("rtc")
    try:
        assert nr.kernel_path() == "rtc"
        assert nr.set_kernel_path("aot") == "rtc"
        assert nr.kernel_path() == "aot"
        assert nr.lib().nt_hip_set_kernel_path(7) == -1  # NT_E_ARG
        assert b"NT_KERNELS_AOT or NT_KERNELS_RTC" in nr.lib().nt_hip_last_error()
        with pytest.raises(ValueError):
            nr.set_kernel_path("jit")
    finally:
        nr.set_kernel_path(prev)


@pytest.mark.parametrize("expr, kernel", [
    # bf16 rows, u8 mask, 16 chunks per wave: C4's sampler
    (b"nt::k_sample_rr<1, 1, 16, false, 8, 1>", b"k_sample_rr"),
    # bf16 policy and reference rows, no mask, logp + KL + entropy, aligned: C3's scorer
    (b"nt::k_score<1, 0, true, true, true, true>", b"k_score"),
    # its backward with the KL term into a bf16 gradient
    (b"nt::k_score_grad<1, 0, true, 1, true>", b"k_score_grad"),
    # the reference's Gumbel-max sampler on C4's rows (bf16, u8 mask, an even stream position)
    (b"nt::k_sample_gumbel<1, 1, false, false>", b"k_sample_gumbel"),
])
def test_hiprtc_compiles_the_row_kernel_instances_on_the_cpu(expr, kernel):
    try:
        rtc = C.CDLL("libhiprtc.so")
    except OSError:
        rtc = C.CDLL("/opt/rocm/lib/libhiprtc.so")
    names = list(EMBEDDED)
    texts = [open(EMBEDDED[n], "rb").read() for n in names]
    Arr = C.c_char_p * len(names)
    prog = C.c_void_p()
    assert rtc.hiprtcCreateProgram(C.byref(prog), PROGRAM, b"nt_rtc.hip", len(names), Arr(*texts),
                                   Arr(*[n.encode() for n in names])) == 0
    assert rtc.hiprtcAddNameExpression(prog, expr) == 0
    opts = (C.c_char_p * len(OPTIONS))(*[o.encode() for o in OPTIONS])
    rc = rtc.hiprtcCompileProgram(prog, len(OPTIONS), opts)
    if rc != 0:
        n = C.c_size_t()
        rtc.hiprtcGetProgramLogSize(prog, C.byref(n))
        log = C.create_string_buffer(n.value + 1)
        rtc.hiprtcGetProgramLog(prog, log)
        pytest.fail(log.value.decode(errors="replace")[:4000])
    lowered = C.c_char_p()
    assert rtc.hiprtcGetLoweredName(prog, expr, C.byref(lowered)) == 0
    assert lowered.value.startswith(b"_ZN2nt") and kernel in lowered.value
    size = C.c_size_t()
    assert rtc.hiprtcGetCodeSize(prog, C.byref(size)) == 0 and size.value > 0
    code = C.create_string_buffer(size.value)
    assert rtc.hiprtcGetCode(prog, code) == 0
    assert code.raw[:4] == b"\x7fELF"
    rtc.hiprtcDestroyProgram(C.byref(prog))
