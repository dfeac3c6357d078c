"""Host-side mirror of noetic-tensor's `nn::rl` for a `Device::Hip(0)` tensor.

The reference (shyble/noetic-tensor 0.7.0) is a Rust crate; its `nn::rl` functions take
`Tensor`/`IntTensor` values and dispatch every op to the device's backend. This module keeps
those function names, argument meanings and refusal messages, and runs each call as the fused
kernels of libnoetic_hip.so through its C ABI (include/noetic_hip.h). There is no CPU fallback:
without the built library, or without a GPU, every call raises `HipUnavailable`.

Tensors live in device memory owned by this module (`Tensor`, `IntTensor`); `to_numpy()` is the
reference's `to_vec*` (a synchronising download).
"""
from __future__ import annotations

import ctypes as C
import enum
import math
import os
import threading
from typing import Optional, Sequence

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libnoetic_hip.so")

# include/noetic_hip.h
NT_F32, NT_BF16, NT_F16 = 0, 1, 2
NT_MASK_NONE, NT_MASK_U8, NT_MASK_F32 = 0, 1, 2
NT_ROW_OK, NT_ROW_NO_TOKEN, NT_ROW_NAN, NT_ROW_BAD_TOKEN = 0, 1, 2, 3


class HipUnavailable(RuntimeError):
    """libnoetic_hip.so is not built, or no HIP device can be claimed."""


class HipError(RuntimeError):
    """A failed call into libnoetic_hip.so (the reference's TensorError::Device)."""


class DTypeError(TypeError):
    """TensorError::DType (src/tensor/error.rs:8-9): a value of another dtype than the operation
    needs, with the reference's message (`same_dtype`, src/tensor/infer.rs:157-158)."""


def same_dtype(a: str, b: str, op: str):
    """infer::same_dtype (infer.rs:157-158): binary ops take one dtype; casts are explicit."""
    if a != b:
        raise DTypeError(f"{op}: {a} and {b} (casts are explicit)")


_HALF = ("bf16", "f16")


def tempered_dtype(dtype: str, temperature: float, mask_dtype: Optional[str]) -> str:
    """The dtype of the reference's materialised `tempered_logits(logits, τ, mask)` (rl.rs:475-486),
    or its DType refusal: `div_scalar` computes 16-bit values in f32 into f32 storage (`fdisp`,
    float.rs:43-58, 494-499), τ == 1 keeps the logits' own dtype, and the additive mask is added
    under `add`'s same_dtype check (float.rs:398-402), its sum of two 16-bit tensors computed in
    f32 into f32 storage as well (fdisp; on a GPU, f32_operand, gpu/mod.rs:336-342, 381-391). A u8
    keep-mask stands for the f32 0/−∞ mask it encodes."""
    z = dtype if temperature == 1.0 else ("f32" if dtype in _HALF else dtype)
    if mask_dtype is not None:
        same_dtype(z, "f32" if mask_dtype in ("u8", "bool") else mask_dtype, "add")
        z = "f32" if z in _HALF else z
    return z


def log_softmax_dtype(dtype: str) -> str:
    """`log_softmax` (activation.rs:30-42) on logits of `dtype`, or its DType refusal: `max_dim`
    returns f32 storage for 16-bit logits (fdisp, float.rs:710-722), so `x.sub(max)` of a bf16 or
    f16 x fails same_dtype ("sub: bf16 and f32"). The reference's `token_log_probs`,
    `categorical_kl` and `categorical_entropy` therefore take f32 logits, or 16-bit ones only
    after a divide (τ ≠ 1) or an explicit `cast` (float.rs:113)."""
    if dtype in _HALF:
        same_dtype(dtype, "f32", "sub")
    return dtype


class MatmulPrecision(enum.Enum):
    """precision::MatmulPrecision (src/tensor/precision.rs:27-38): F32 (the default: CpuRef's bits)
    or Half (bf16 operands rounded to nearest-even as they are loaded, f32 accumulation, on the
    matrix cores)."""
    F32 = "f32"
    HALF = "half"


_precision = threading.local()


def set_matmul_precision(p: MatmulPrecision) -> MatmulPrecision:
    """precision::set_matmul_precision (precision.rs:53-58): the calling thread's precision of
    GPU products; returns the previous setting."""
    prev = matmul_precision()
    _precision.value = MatmulPrecision(p)
    return prev


def matmul_precision() -> MatmulPrecision:
    """precision::matmul_precision (precision.rs:60-63): F32 unless set on this thread."""
    return getattr(_precision, "value", MatmulPrecision.F32)


class matmul_precision_scope:
    """`set_matmul_precision(p)` for a `with` block, the previous setting restored after it."""

    def __init__(self, p: MatmulPrecision):
        self.p = MatmulPrecision(p)

    def __enter__(self):
        self.prev = set_matmul_precision(self.p)
        return self

    def __exit__(self, *exc):
        set_matmul_precision(self.prev)
        return False


class NtMaskRows(C.Structure):
    """A mask broadcast over leading dimensions: logits row (s B + b) T + t reads the mask row at
    element s ld_s + b ld_b + t mask_ld (all zero: rows of mask_ld)."""
    _fields_ = [("t_rows", C.c_int64), ("b_rows", C.c_int64), ("ld_b", C.c_int64), ("ld_s", C.c_int64)]


class NtRlSampleArgs(C.Structure):
    _fields_ = [("logits", C.c_void_p), ("dtype", C.c_int32), ("mask_kind", C.c_int32),
                ("rows", C.c_int64), ("vocab", C.c_int64), ("ld", C.c_int64),
                ("mask", C.c_void_p), ("mask_ld", C.c_int64), ("temperature", C.c_double),
                ("uniforms", C.c_void_p), ("ids", C.c_void_p), ("logp", C.c_void_p),
                ("entropy", C.c_void_p), ("status", C.c_void_p), ("mask_rows", NtMaskRows)]


class NtRlGumbelArgs(C.Structure):
    _fields_ = [("logits", C.c_void_p), ("dtype", C.c_int32), ("mask_kind", C.c_int32),
                ("rows", C.c_int64), ("vocab", C.c_int64), ("ld", C.c_int64),
                ("mask", C.c_void_p), ("mask_ld", C.c_int64), ("temperature", C.c_double),
                ("key", C.c_uint32 * 8), ("block", C.c_uint64), ("word", C.c_int32), ("pad0", C.c_int32),
                ("ids", C.c_void_p), ("status", C.c_void_p), ("mask_rows", NtMaskRows)]


class NtRlReadoutSampleArgs(C.Structure):
    _fields_ = [("hidden", C.c_void_p), ("weight_packed", C.c_void_p), ("rows", C.c_int64), ("vocab", C.c_int64),
                ("dim", C.c_int64), ("ldh", C.c_int64), ("mask_kind", C.c_int32),
                ("hidden_dtype", C.c_int32), ("mask", C.c_void_p), ("mask_ld", C.c_int64),
                ("temperature", C.c_double), ("uniforms", C.c_void_p), ("ids", C.c_void_p), ("logp", C.c_void_p), ("status", C.c_void_p),
                ("logits", C.c_void_p), ("debug_block", C.c_void_p), ("debug_block_index", C.c_void_p)]


class NtRlReadoutScoreArgs(C.Structure):
    _fields_ = [("hidden", C.c_void_p), ("weight_packed", C.c_void_p), ("rows", C.c_int64), ("vocab", C.c_int64),
                ("dim", C.c_int64), ("ldh", C.c_int64), ("mask_kind", C.c_int32),
                ("hidden_dtype", C.c_int32), ("mask", C.c_void_p), ("mask_ld", C.c_int64),
                ("temperature", C.c_double), ("tokens", C.c_void_p), ("logp", C.c_void_p), ("entropy", C.c_void_p), ("status", C.c_void_p),
                ("logits", C.c_void_p)]


class NtRlScoreArgs(C.Structure):
    _fields_ = [("logits", C.c_void_p), ("ref_logits", C.c_void_p), ("dtype", C.c_int32),
                ("mask_kind", C.c_int32), ("rows", C.c_int64), ("vocab", C.c_int64), ("ld", C.c_int64),
                ("mask", C.c_void_p), ("mask_ld", C.c_int64), ("temperature", C.c_double),
                ("tokens", C.c_void_p), ("logp", C.c_void_p), ("ref_logp", C.c_void_p),
                ("kl", C.c_void_p), ("entropy", C.c_void_p), ("status", C.c_void_p),
                ("lse_base", C.c_void_p), ("lse_rest", C.c_void_p), ("ref_lse_base", C.c_void_p),
                ("ref_lse_rest", C.c_void_p), ("mask_rows", NtMaskRows)]


class NtRlScoreGradArgs(C.Structure):
    _fields_ = [("logits", C.c_void_p), ("ref_logits", C.c_void_p), ("dtype", C.c_int32),
                ("mask_kind", C.c_int32), ("rows", C.c_int64), ("vocab", C.c_int64), ("ld", C.c_int64),
                ("mask", C.c_void_p), ("mask_ld", C.c_int64), ("temperature", C.c_double),
                ("tokens", C.c_void_p), ("lse_base", C.c_void_p), ("lse_rest", C.c_void_p),
                ("ref_lse_base", C.c_void_p), ("ref_lse_rest", C.c_void_p), ("kl", C.c_void_p),
                ("entropy", C.c_void_p), ("g_logp", C.c_void_p), ("g_kl", C.c_void_p), ("g_entropy", C.c_void_p),
                ("grad", C.c_void_p), ("grad_dtype", C.c_int32), ("pad0", C.c_int32), ("grad_ld", C.c_int64),
                ("mask_rows", NtMaskRows)]


class NtRlPolicyLossArgs(C.Structure):
    _fields_ = [("logp", C.c_void_p), ("old_logp", C.c_void_p), ("weights", C.c_void_p), ("mask", C.c_void_p),
                ("S", C.c_int64), ("B", C.c_int64), ("T", C.c_int64), ("kind", C.c_int32),
                ("weights_per_sequence", C.c_int32), ("clip_low", C.c_double), ("clip_high", C.c_double),
                ("dual", C.c_double), ("log_ratio_clamp", C.c_double), ("loss", C.c_void_p), ("dloss", C.c_void_p),
                ("hit", C.c_void_p)]


NT_LOSS_PG, NT_LOSS_PPO = 0, 1


class NtLayout(C.Structure):
    """include/noetic_ops.h NtLayout: a view (element offset, shape, element strides)."""
    _fields_ = [("rank", C.c_int32), ("pad_", C.c_int32), ("offset", C.c_int64), ("shape", C.c_int64 * 8),
                ("strides", C.c_int64 * 8)]


class NtRng(C.Structure):
    _fields_ = [("key", C.c_uint32 * 8), ("counter", C.c_uint64), ("buf", C.c_uint32 * 16), ("idx", C.c_int32)]


class NtSynthNormal(C.Structure):
    _fields_ = [("out", C.c_void_p), ("dtype", C.c_int32), ("rows", C.c_int64), ("vocab", C.c_int64),
                ("key", C.c_uint32 * 8), ("mean", C.c_double), ("std", C.c_double), ("zipf_s", C.c_double),
                ("rot_key", C.c_uint32 * 8), ("base", C.c_void_p)]


# Every function the headers under include/ declare, with its ctypes signature.
_SIGS = {
    # noetic_hip.h
    "nt_hip_claim": (C.c_int, [C.c_int]),
    "nt_hip_device_count": (C.c_int, []),
    "nt_hip_last_error": (C.c_char_p, []),
    "nt_hip_key": (C.c_int, [C.c_char_p, C.c_size_t]),
    "nt_hip_platform_details": (C.c_int, [C.c_char_p, C.c_size_t]),
    "nt_hip_alloc": (C.c_int, [C.c_size_t, C.POINTER(C.c_void_p)]),
    "nt_hip_free": (C.c_int, [C.c_void_p]),
    "nt_hip_upload": (C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t]),
    "nt_hip_download": (C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t]),
    "nt_hip_memset": (C.c_int, [C.c_void_p, C.c_int, C.c_size_t]),
    "nt_hip_sync": (C.c_int, []),
    "nt_hip_stream": (C.c_int, [C.POINTER(C.c_void_p)]),
    "nt_hip_launches": (C.c_uint64, []),
    "nt_hip_set_kernel_path": (C.c_int, [C.c_int]),
    "nt_hip_kernel_path": (C.c_int, []),
    "nt_hip_rl_sample": (C.c_int, [C.POINTER(NtRlSampleArgs)]),
    "nt_hip_rl_sample_gumbel": (C.c_int, [C.POINTER(NtRlGumbelArgs)]),
    "nt_hip_rl_readout_sample": (C.c_int, [C.POINTER(NtRlReadoutSampleArgs)]),
    "nt_hip_rl_readout_score": (C.c_int, [C.POINTER(NtRlReadoutScoreArgs)]),
    "nt_hip_rl_readout_packed_bytes": (C.c_int64, [C.c_int64, C.c_int64]),
    "nt_hip_rl_readout_pack_weight": (C.c_int, [C.c_void_p, C.c_int32, C.c_int32, C.c_int64, C.c_int64, C.c_int64,
                                                C.c_void_p]),
    "nt_hip_rl_sample_noalloc": (C.c_int, [C.POINTER(NtRlSampleArgs)]),
    "nt_hip_rl_score": (C.c_int, [C.POINTER(NtRlScoreArgs)]),
    "nt_hip_rl_score_backward": (C.c_int, [C.POINTER(NtRlScoreGradArgs)]),
    "nt_hip_rl_kl_estimate": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int64, C.c_int32, C.c_double,
                                        C.c_void_p]),
    "nt_hip_rl_zero_masked": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int64, C.c_void_p]),
    "nt_hip_rl_reduce_tokens": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int64, C.c_int64, C.c_int64, C.c_int32,
                                          C.c_void_p]),
    "nt_hip_rl_reduce_tokens_backward": (C.c_int, [C.c_void_p, C.c_int64, C.c_int64, C.c_int64, C.c_int32,
                                                   C.c_void_p, C.c_double, C.c_void_p, C.c_void_p]),
    "nt_hip_rl_kl_estimate_backward": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int64, C.c_int32,
                                                 C.c_double, C.c_void_p]),
    "nt_hip_rl_policy_loss": (C.c_int, [C.POINTER(NtRlPolicyLossArgs)]),
    "nt_hip_rl_group_advantages": (C.c_int, [C.c_void_p, C.c_int64, C.c_int64, C.c_int32, C.c_double, C.c_int32,
                                             C.c_void_p]),
    # noetic_ops.h
    "nt_hip_copy": (C.c_int, [C.c_void_p, C.POINTER(NtLayout), C.c_int32, C.c_void_p]),
    "nt_hip_write": (C.c_int, [C.c_void_p, C.POINTER(NtLayout), C.c_void_p, C.POINTER(NtLayout), C.c_int32]),
    "nt_hip_cast": (C.c_int, [C.c_void_p, C.POINTER(NtLayout), C.c_int32, C.c_int32, C.c_void_p]),
    "nt_hip_unary": (C.c_int, [C.c_int32, C.c_float, C.c_void_p, C.POINTER(NtLayout), C.c_void_p]),
    "nt_hip_compare": (C.c_int, [C.c_int32, C.c_float, C.c_void_p, C.POINTER(NtLayout), C.c_void_p]),
    "nt_hip_binary": (C.c_int, [C.c_int32, C.c_void_p, C.POINTER(NtLayout), C.c_void_p, C.POINTER(NtLayout),
                                C.c_void_p]),
    "nt_hip_mask_fill": (C.c_int, [C.c_void_p, C.POINTER(NtLayout), C.c_void_p, C.POINTER(NtLayout), C.c_float,
                                   C.c_void_p]),
    "nt_hip_reduce_dim": (C.c_int, [C.c_int32, C.c_void_p, C.c_int64, C.c_int64, C.c_int64, C.c_int32, C.c_void_p]),
    "nt_hip_reduce_all": (C.c_int, [C.c_int32, C.c_void_p, C.c_int64, C.c_void_p]),
    "nt_hip_gather": (C.c_int, [C.c_void_p, C.c_int64, C.c_int64, C.c_int64, C.c_void_p, C.c_int64, C.c_void_p]),
    "nt_hip_index_select": (C.c_int, [C.c_void_p, C.c_int64, C.c_int64, C.c_int64, C.c_void_p, C.c_int64,
                                      C.c_void_p]),
    "nt_hip_one_hot": (C.c_int, [C.c_void_p, C.c_int64, C.c_int64, C.c_void_p]),
    "nt_hip_scatter_add": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int64, C.c_int64, C.c_int64, C.c_int64,
                                     C.c_void_p]),
    "nt_hip_index_add": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int64, C.c_int64, C.c_int64, C.c_int64, C.c_void_p]),
    "nt_hip_fill": (C.c_int, [C.c_void_p, C.c_int64, C.c_float]),
    "nt_hip_matmul": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p]),
    "nt_hip_matmul_half": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p]),
    "nt_hip_half_gemm_key": (C.c_int, [C.c_char_p, C.c_size_t]),
    "nt_hip_sort_desc": (C.c_int, [C.c_void_p, C.c_int64, C.c_int64, C.c_int64, C.c_void_p, C.c_void_p]),
    # noetic_rng.h
    "nt_rng_derive": (C.c_int, [C.POINTER(NtRng), C.c_uint64, C.c_char_p, C.c_size_t]),
    "nt_rng_from_seed": (C.c_int, [C.POINTER(NtRng), C.c_char_p]),
    "nt_rng_next_u32": (C.c_uint32, [C.POINTER(NtRng)]),
    "nt_rng_next_u64": (C.c_uint64, [C.POINTER(NtRng)]),
    "nt_rng_uniforms": (C.c_int, [C.POINTER(NtRng), C.c_size_t, C.c_void_p]),
    "nt_rng_word_pos": (C.c_int, [C.POINTER(NtRng), C.POINTER(C.c_uint64), C.POINTER(C.c_int32)]),
    "nt_rng_set_word_pos": (C.c_int, [C.POINTER(NtRng), C.c_uint64, C.c_int32]),
    "nt_rng_skip_u64": (C.c_int, [C.POINTER(NtRng), C.c_uint64]),
    "nt_sha256": (C.c_int, [C.c_char_p, C.c_size_t, C.c_char_p]),
    # noetic_synth.h
    "nt_synth_normal": (C.c_int, [C.POINTER(NtSynthNormal)]),
    "nt_synth_spikes": (C.c_int, [C.c_void_p, C.c_int32, C.c_int64, C.c_int64, C.c_int32, C.POINTER(C.c_uint32),
                                  C.c_double]),
    "nt_synth_bernoulli_mask": (C.c_int, [C.c_void_p, C.c_int64, C.POINTER(C.c_uint32), C.c_double]),
    "nt_synth_tokens": (C.c_int, [C.c_void_p, C.c_int64, C.POINTER(C.c_uint32), C.c_int64]),
    "nt_synth_keep_tokens": (C.c_int, [C.c_void_p, C.c_int64, C.c_int64, C.c_void_p]),
    "nt_synth_runs_mask_host": (C.c_int, [C.c_void_p, C.c_int64, C.c_int64, C.c_uint64, C.c_char_p, C.c_size_t,
                                          C.c_int32, C.c_int32]),
    "nt_measure_read": (C.c_int, [C.c_size_t, C.c_int32, C.POINTER(C.c_double)]),
    "nt_measure_launch_period": (C.c_int, [C.c_int32, C.c_int32, C.c_int32, C.POINTER(C.c_double)]),
    "nt_measure_shader_clock": (C.c_int, [C.c_int32, C.POINTER(C.c_double)]),
}

_lib = None
_claimed = False


def lib():
    """The loaded libnoetic_hip.so (no device claimed yet)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise HipUnavailable(f"{LIB_PATH} is not built (run __graft_entry__.build())")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def _check(rc, what):
    if rc != 0:
        raise HipError(f"{what}: {lib().nt_hip_last_error().decode(errors='replace')} (code {rc})")


def claim(device: int = 0):
    """Claim Hip(device) for this process (one device per process)."""
    global _claimed
    L = lib()
    if L.nt_hip_device_count() < 1:
        raise HipUnavailable("no HIP device visible")
    _check(L.nt_hip_claim(device), f"claim Hip({device})")
    _claimed = True


def _dev():
    if not _claimed:
        claim(0)
    return lib()


def sync():
    _check(_dev().nt_hip_sync(), "sync")


def key() -> str:
    buf = C.create_string_buffer(256)
    _check(_dev().nt_hip_key(buf, 256), "key")
    return buf.value.decode()


KERNELS_AOT, KERNELS_RTC = 0, 1


def set_kernel_path(path: str) -> str:
    """Choose how the sampler kernels are loaded for the rest of the process: "aot" (the code
    objects hipcc built into the library) or "rtc" (compiled by hiprtc from the embedded source at
    first use, as the reference compiles its CUDA kernels with NVRTC: cuda/mod.rs:169-218).
    Returns the previous choice. Needs no device."""
    code = {"aot": KERNELS_AOT, "rtc": KERNELS_RTC}.get(path)
    if code is None:
        raise ValueError(f"kernel path {path!r}: 'aot' or 'rtc'")
    prev = lib().nt_hip_set_kernel_path(code)
    if prev < 0:
        _check(prev, "set_kernel_path")
    return "rtc" if prev == KERNELS_RTC else "aot"


def kernel_path() -> str:
    return "rtc" if lib().nt_hip_kernel_path() == KERNELS_RTC else "aot"


def platform_details() -> str:
    """`GpuBackend::platform_details` (gpu/mod.rs:199): the HIP driver, the amdgpu kernel driver
    release and the compiler that built the code objects."""
    buf = C.create_string_buffer(512)
    _check(_dev().nt_hip_platform_details(buf, 512), "platform_details")
    return buf.value.decode()


def platform_key() -> str:
    """`gpu_platform_key` (gpu/mod.rs:690-704): `key()` followed by `platform_details()` and, when
    the calling thread's matmul precision is Half, the reduced-precision product's part
    (`half_gemm_key`, precision.rs:72-78): the kernels' source hash, which covers the readout
    fusion's product as well as `matmul_half`."""
    base = f"{key()}-{platform_details()}"
    if matmul_precision() == MatmulPrecision.HALF:
        buf = C.create_string_buffer(256)
        _check(_dev().nt_hip_half_gemm_key(buf, 256), "half_gemm_key")
        return f"{base}-{buf.value.decode()}"
    return base


def launches() -> int:
    return int(lib().nt_hip_launches())


# ----------------------------------------------------------------------------------- storage

_NP = {"f32": np.float32, "bf16": np.uint16, "f16": np.uint16, "u8": np.uint8, "bool": np.uint8, "i32": np.int32,
       "i64": np.int64, "f64": np.float64}


class Buffer:
    """A device allocation owned by Python (freed on garbage collection)."""

    def __init__(self, nbytes: int):
        L = _dev()
        self.nbytes = int(nbytes)
        p = C.c_void_p()
        _check(L.nt_hip_alloc(max(self.nbytes, 1), C.byref(p)), f"alloc {nbytes} B")
        self.ptr = p.value

    def __del__(self):
        try:
            if self.ptr and _lib is not None:
                _lib.nt_hip_free(C.c_void_p(self.ptr))
        except Exception:
            pass
        self.ptr = None


class Tensor:
    """Device storage with a shape and a dtype ("f32", "bf16" or "f16" bits, "u8", "bool" bytes, "i32",
    "i64", "f64")."""

    def __init__(self, shape: Sequence[int], dtype: str, buf: Optional[Buffer] = None):
        self.shape = tuple(int(s) for s in shape)
        self.dtype = dtype
        self.numel = int(np.prod(self.shape)) if self.shape else 1
        nbytes = self.numel * np.dtype(_NP[dtype]).itemsize
        self.buf = buf if buf is not None else Buffer(nbytes)
        self.nbytes = nbytes

    @property
    def ptr(self):
        return self.buf.ptr

    @staticmethod
    def from_numpy(a: np.ndarray, dtype: Optional[str] = None) -> "Tensor":
        if dtype is None:
            dtype = {np.dtype(np.float32): "f32", np.dtype(np.uint16): "bf16", np.dtype(np.uint8): "u8",
                     np.dtype(np.int32): "i32", np.dtype(np.float64): "f64"}[a.dtype]
        a = np.ascontiguousarray(a, dtype=_NP[dtype])
        t = Tensor(a.shape, dtype)
        _check(_dev().nt_hip_upload(C.c_void_p(t.ptr), a.ctypes.data_as(C.c_void_p), t.nbytes), "upload")
        return t

    def to_numpy(self) -> np.ndarray:
        out = np.empty(self.shape, dtype=_NP[self.dtype])
        _check(_dev().nt_hip_download(out.ctypes.data_as(C.c_void_p), C.c_void_p(self.ptr), self.nbytes), "download")
        return out

    def to_f64(self) -> np.ndarray:
        """`to_vec_f64` (a bf16 tensor widens exactly)."""
        a = self.to_numpy()
        if self.dtype == "bf16":
            return (a.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
        if self.dtype == "f16":
            return a.view(np.float16).astype(np.float64)
        return a.astype(np.float64)

    def dims(self):
        return self.shape


def IntTensor(shape, buf=None) -> Tensor:
    """Device I32 indices (the reference's device index dtype, src/tensor/gpu/mod.rs:355-357)."""
    return Tensor(shape, "i32", buf)


def _dtype_code(t: Tensor) -> int:
    code = {"f32": NT_F32, "bf16": NT_BF16, "f16": NT_F16}.get(t.dtype)
    if code is None:
        raise ValueError(f"logits of dtype {t.dtype} (f32, bf16 or f16)")
    return code


# ----------------------------------------------------------------------------------- rng

class Rng:
    """rng::derive(root, label) (src/rng.rs:9-17): the engine stream the sampler draws from."""

    def __init__(self, root: int, label: str):
        self.s = NtRng()
        b = label.encode()
        _check(lib().nt_rng_derive(C.byref(self.s), root, b, len(b)), "rng derive")

    def clone(self) -> "Rng":
        r = Rng.__new__(Rng)
        r.s = NtRng()
        C.memmove(C.byref(r.s), C.byref(self.s), C.sizeof(NtRng))
        return r

    def next_u64(self) -> int:
        return int(lib().nt_rng_next_u64(C.byref(self.s)))

    def next_u32(self) -> int:
        return int(lib().nt_rng_next_u32(C.byref(self.s)))

    def uniforms(self, n: int) -> np.ndarray:
        out = np.empty(n, dtype=np.float64)
        _check(lib().nt_rng_uniforms(C.byref(self.s), n, out.ctypes.data_as(C.c_void_p)), "uniforms")
        return out

    def key(self):
        return (C.c_uint32 * 8)(*self.s.key)

    def word_pos(self):
        """(block, word): the next unread keystream word (rand_chacha `get_word_pos`)."""
        b, w = C.c_uint64(), C.c_int32()
        _check(lib().nt_rng_word_pos(C.byref(self.s), C.byref(b), C.byref(w)), "rng word_pos")
        return int(b.value), int(w.value)

    def skip_u64(self, n: int):
        """The state after n next_u64 calls, without generating them."""
        _check(lib().nt_rng_skip_u64(C.byref(self.s), n), "rng skip")


# ----------------------------------------------------------------------------------- nn::rl

class TokenReduction(enum.IntEnum):
    """rl.rs:37-55."""
    NONE = 0
    SUM = 1
    TOKEN_MEAN = 2
    PER_SEQUENCE = 3
    SEQUENCE_MEAN = 4


class KlEstimator(enum.IntEnum):
    """rl.rs:356-366."""
    K1 = 1
    K2 = 2
    K3 = 3


KL_DELTA_CLAMP = 20.0  # rl.rs:150


class Tempered:
    """`tempered_logits(logits, temperature, mask)` (rl.rs:475-486), kept unmaterialised: the
    fused kernels apply the divide and the vocabulary mask while streaming the logits.
    mask: None, a u8 keep-mask (0 excludes) or an additive f32, bf16 or f16 mask (a 16-bit one
    widened exactly, as the reference's add computes it in f32) in the logits' rank, each
    dimension equal to the logits' or 1 (a mask whose leading dims are all 1 is shared by every
    row; one whose last dimension is 1 is a value per position).

    Built directly, it is the fused entries' (logits, τ, mask) triple: 16-bit logits are widened
    exactly to f32 at every τ, the values the reference's chain gives on `logits.cast(F32)`.
    Built by `tempered_logits`, it also keeps the reference's dtype rules (`dtype`): the
    reference-named functions refuse it where the materialised tensor would be refused."""

    def __init__(self, logits: Tensor, temperature: float, mask: Optional[Tensor]):
        if not (temperature > 0.0 and math.isfinite(temperature)):
            raise ValueError(f"tempered_logits: temperature {temperature} (must be positive)")
        self.logits, self.temperature, self.mask = logits, float(temperature), mask
        self.dtype = None  # the materialised tensor's dtype, when built by tempered_logits
        if mask is not None:
            if len(mask.shape) != len(logits.shape):
                raise ValueError("tempered_logits: mask rank")
            if not all(a == b or a == 1 for a, b in zip(mask.shape, logits.shape)):
                raise ValueError(f"tempered_logits: mask {list(mask.shape)} does not broadcast to the logits "
                                 f"{list(logits.shape)}")


def tempered_logits(logits: Tensor, temperature: float, mask: Optional[Tensor] = None) -> Tempered:
    """rl.rs:475-486, unmaterialised, with the reference's refusals: a 16-bit tensor at τ == 1 is
    not divided, so adding the (f32) mask fails same_dtype ("add: bf16 and f32")."""
    t = Tempered(logits, temperature, mask)
    t.dtype = tempered_dtype(logits.dtype, t.temperature, None if mask is None else mask.dtype)
    return t


def _logits_dtype(x) -> str:
    """The dtype the reference's op would see: a Tensor's own, a `tempered_logits` result's
    materialised one; a Tempered built directly (the fused triple) reads as f32."""
    if isinstance(x, Tempered):
        return x.dtype if x.dtype is not None else "f32"
    return x.dtype


def _as_tempered(x) -> Tempered:
    return x if isinstance(x, Tempered) else Tempered(x, 1.0, None)


def mask_groups(logits_shape, mask_shape):
    """The leading dimensions of a mask that broadcasts to the logits (rl.rs:477-483), folded into
    (rows, mask stride) groups, outermost first: the mask is contiguous, a dimension the mask has
    as 1 reads stride 0, and adjacent dimensions merge when the outer one's stride is the inner
    one's times its length (both broadcast, or both read in order). Dimensions of length 1 drop."""
    V = mask_shape[-1]
    stride, strides = V, []
    for d in reversed(mask_shape[:-1]):
        strides.append(stride if d > 1 else 0)
        stride *= d
    strides.reverse()
    groups = []
    for d, e in zip(logits_shape[:-1], strides):
        if d == 1:
            continue
        if groups and groups[-1][1] == e * d:
            groups[-1] = (groups[-1][0] * d, e)
        else:
            groups.append((d, e))
    return groups


def _mask_fields(t: Tempered, rows: int, V: int):
    """(kind, pointer, mask_ld, NtMaskRows, the tensor to keep alive) of a Tempered's mask: rows of
    mask_ld when its leading dimensions fold into one group, the (s, b, t) map for up to three; a
    mask of more groups, or one that broadcasts along the vocabulary axis too (a value per
    position, [.., 1]), is first broadcast to [rows, V] on the device (noetic_ops.copy)."""
    m = t.mask
    mr = NtMaskRows(0, 0, 0, 0)
    if m is None:
        return NT_MASK_NONE, None, 0, mr, None
    kind = {"u8": NT_MASK_U8, "f32": NT_MASK_F32, "bf16": NT_MASK_F32, "f16": NT_MASK_F32}.get(m.dtype)
    if kind is None:
        raise ValueError(f"vocabulary mask of dtype {m.dtype} (u8 keep-mask, or additive f32, bf16 or f16)")
    if m.dtype in _HALF:
        # a 16-bit additive mask is added in f32 (fdisp; f32_operand on a GPU): widened exactly
        import noetic_ops as ops  # (noetic_ops imports this module)
        m = ops.cast(m, ops.Layout.contiguous(m.shape), "f32")
    if m.shape[-1] != V:
        import noetic_ops as ops  # (noetic_ops imports this module)
        full = ops.copy(m, ops.Layout.contiguous(m.shape).broadcast(t.logits.shape))
        return kind, full.ptr, V, mr, full
    g = mask_groups(t.logits.shape, m.shape)
    if not g:
        return kind, m.ptr, 0, mr, m
    if len(g) == 1:
        return kind, m.ptr, g[0][1], mr, m
    if len(g) <= 3:
        g = [(1, 0)] * (3 - len(g)) + g
        (_, ls), (B, lb), (T, lt) = g
        return kind, m.ptr, lt, NtMaskRows(T, B, lb, ls), m
    import noetic_ops as ops  # (noetic_ops imports this module)
    full = ops.copy(m, ops.Layout.contiguous(m.shape).broadcast(t.logits.shape))
    return kind, full.ptr, V, mr, full


def _rows(x: Tensor):
    if len(x.shape) < 1:
        raise ValueError("logits of rank 0")
    V = x.shape[-1]
    return x.numel // V, V


def _row_arg(t: Optional[Tensor], rows: int, dtype: str, what: str) -> Optional[Tensor]:
    """A per-row device argument the kernels read `rows` values of `dtype` from: checked here,
    before any launch (16-bit floats where f32 is read are widened exactly on the device)."""
    if t is None:
        return None
    if t.numel != rows:
        raise ValueError(f"{what}: {t.numel} values for {rows} rows")
    if t.dtype == dtype:
        return t
    if dtype == "f32":
        return _f32_storage(t, what)
    raise ValueError(f"{what}: dtype {t.dtype} ({dtype})")


def sample_logp(logits: Tensor, temperature: float, mask: Optional[Tensor], rng: Optional[Rng],
                entropy: bool = False, uniforms: Optional[Tensor] = None, check: bool = True):
    """sample_categorical_inv_cdf with its log-probabilities, the fused path: (ids, logp[,
    entropy]) of the inverse-CDF sample of each row, drawing one uniform per row from `rng`
    (none at temperature 0). `uniforms` (device f64 [rows]) may be given instead of `rng`.
    `check` reads the per-row status and refuses a row with no allowed token, as
    sample_categorical does (rl.rs:516-519)."""
    if not (temperature >= 0.0 and math.isfinite(temperature)):
        raise ValueError(f"sample_categorical: temperature {temperature} (must be ≥ 0)")
    t = Tempered(logits, 1.0 if temperature == 0.0 else temperature, mask)
    rows, V = _rows(logits)
    out_shape = logits.shape[:-1]
    if temperature != 0.0 and uniforms is None:
        if rng is None:
            raise ValueError("sample_categorical: a stream is needed at temperature > 0")
        uniforms = Tensor.from_numpy(rng.uniforms(rows), "f64")
    uniforms = _row_arg(uniforms, rows, "f64", "sample_categorical: uniforms")
    ids = IntTensor(out_shape)
    lp = Tensor(out_shape, "f32")
    ent = Tensor(out_shape, "f32") if entropy else None
    status = Tensor(out_shape, "u8")
    kind, mptr, mld, mrows, _keep = _mask_fields(t, rows, V)
    a = NtRlSampleArgs(logits.ptr, _dtype_code(logits), kind, rows, V, V, mptr, mld, float(temperature),
                       None if uniforms is None else uniforms.ptr, ids.ptr, lp.ptr,
                       None if ent is None else ent.ptr, status.ptr, mrows)
    _check(lib().nt_hip_rl_sample(C.byref(a)), "sample")
    if check:
        st = status.to_numpy().ravel()
        bad = np.nonzero(st != NT_ROW_OK)[0]
        if bad.size:
            raise ValueError(f"sample_categorical: position {bad[0]} has no allowed token (every logit −∞ or a NaN)")
    return (ids, lp, ent) if entropy else (ids, lp)


def sample_categorical(logits: Tensor, temperature: float, mask: Optional[Tensor], rng: Rng) -> Tensor:
    """rl.rs:510-529, the reference's Gumbel-max sampler: argmax(z + g) with z the tempered logits
    and one Gumbel draw per logit from `rng` in row-major order, so the stream advances by one
    u64 per logit (none at temperature 0). The draws are generated on the device at the stream's
    position (nt_hip_rl_sample_gumbel); the stream is advanced here, after the rows are accepted:
    a row with no allowed token is refused with the reference's message and draws nothing.

    The reference's dtype rules hold, in its order: 16-bit logits at τ ∈ {0, 1} with a mask are
    refused by tempered_logits' add, and at τ == 1 (after the row check) by `z + g`, the noise
    being f32 (`from_f64s` computes 16-bit dtypes in f32, float.rs:257-260): "add: bf16 and f32".
    `sample_logp` takes them at every τ, widened exactly."""
    if not (temperature >= 0.0 and math.isfinite(temperature)):
        raise ValueError(f"sample_categorical: temperature {temperature} (must be ≥ 0)")
    t = Tempered(logits, 1.0 if temperature == 0.0 else temperature, mask)
    z = tempered_dtype(logits.dtype, t.temperature, None if mask is None else mask.dtype)
    rows, V = _rows(logits)
    out_shape = logits.shape[:-1]
    ids = IntTensor(out_shape)
    status = Tensor(out_shape, "u8")
    kind, mptr, mld, mrows, _keep = _mask_fields(t, rows, V)
    block, word = rng.word_pos()
    a = NtRlGumbelArgs(logits.ptr, _dtype_code(logits), kind, rows, V, V, mptr, mld, float(temperature),
                       rng.key(), block, word, 0, ids.ptr, status.ptr, mrows)
    _check(lib().nt_hip_rl_sample_gumbel(C.byref(a)), "sample_categorical")
    st = status.to_numpy().ravel()
    bad = np.nonzero(st != NT_ROW_OK)[0]
    if bad.size:
        raise ValueError(f"sample_categorical: position {bad[0]} has no allowed token (every logit −∞ or a NaN)")
    if temperature != 0.0:
        same_dtype(z, "f32" if z in _HALF else z, "add")
        rng.skip_u64(rows * V)
    return ids


def sample_categorical_inv_cdf(logits: Tensor, temperature: float, mask: Optional[Tensor], rng: Rng) -> Tensor:
    """A new nn::rl entry beside sample_categorical (rl.rs:510-529): the same distribution, drawn
    by the inverse CDF of one uniform per row (one u64 of `rng` per row, none at temperature 0)
    in one fused pass over the logits. `sample_logp` also returns the tokens' log-probabilities."""
    return sample_logp(logits, temperature, mask, rng)[0]


NT_READOUT_W_DV, NT_READOUT_W_VD = 0, 1
_ESIZE = {"f32": 4, "bf16": 2, "f16": 2}
_DTCODE = {"f32": NT_F32, "bf16": NT_BF16, "f16": NT_F16}
_READOUT_ROWS = 256  # rows per readout call (include/noetic_hip.h)


class PackedReadout:
    """The decoder head's weight (`Linear`, linear.rs:1-12: `x.matmul(w)` with w [in, out], or
    seed-batched [S, in, out]) packed once for the readout-fused entries, in the order the matrix
    cores read it: from [d, V] or [S, d, V] (`layout` "dv"), or a vocabulary-major [V, d] /
    [S, V, d] ("vd"). bf16 is packed as it is; f32 and f16 are rounded to bf16 to nearest-even as
    they are packed, the rounding MatmulPrecision::Half gives its operands as they are loaded
    (precision.rs:4-8; an f16 value widens to f32 exactly first). One packing kernel per seed."""

    def __init__(self, weight: Tensor, layout: str = "dv"):
        if weight.dtype not in _ESIZE or len(weight.shape) not in (2, 3):
            raise ValueError("readout weight: an f32, bf16 or f16 [d, V] or [S, d, V] matrix")
        sh = tuple(weight.shape) if len(weight.shape) == 3 else (1,) + tuple(weight.shape)
        self.seeds, self.batched, self.weight_dtype = sh[0], len(weight.shape) == 3, weight.dtype
        if layout == "dv":
            self.dim, self.vocab = sh[1], sh[2]
            code, ld = NT_READOUT_W_DV, self.vocab
        elif layout == "vd":
            self.vocab, self.dim = sh[1], sh[2]
            code, ld = NT_READOUT_W_VD, self.dim
        else:
            raise ValueError(f"readout weight layout {layout!r} (dv or vd)")
        nbytes = int(lib().nt_hip_rl_readout_packed_bytes(self.vocab, self.dim))
        if nbytes < 0:
            raise ValueError(f"readout weight [{self.vocab}, {self.dim}]: dim a multiple of 16")
        self.seed_bytes = nbytes
        self.buf = Buffer(nbytes * self.seeds)
        dt = _DTCODE[weight.dtype]
        step = sh[1] * sh[2] * _ESIZE[weight.dtype]
        for k in range(self.seeds):
            _check(lib().nt_hip_rl_readout_pack_weight(weight.ptr + k * step, dt, code, self.vocab, self.dim, ld,
                                                       self.seed_ptr(k)), "readout pack")

    def seed_ptr(self, seed: int) -> int:
        return self.buf.ptr + seed * self.seed_bytes

    def buf_bytes(self, seed: int = 0) -> bytes:
        """One seed's packed bytes (a synchronising download; for tests)."""
        out = (C.c_uint8 * self.seed_bytes)()
        _check(lib().nt_hip_download(out, C.c_void_p(self.seed_ptr(seed)), self.seed_bytes), "download packed")
        return bytes(out)


def _readout_gate(who: str):
    """The readout fusion's product has bf16 operands and f32 accumulation on the matrix cores, the
    reduced-precision product: it stands for the head's `x.matmul(w)` only when the calling
    thread's matmul precision is Half (`Tensor::matmul` reads it for a GPU tensor,
    float.rs:924-930; precision.rs:59-63). At the default F32 the head's product is the f32 one:
    multiply with `noetic_ops.DTensor.matmul` and sample or score the written logits."""
    if matmul_precision() != MatmulPrecision.HALF:
        raise ValueError(f"{who}: the readout fusion computes the MatmulPrecision::Half product; at this "
                         "thread's f32 precision multiply with matmul and use the written logits")


def _readout_shape(hidden: Tensor, weight: PackedReadout, who: str):
    """(seeds, rows per seed, d) of the head's input: [.., d] against a [d, V] weight (the weight
    broadcast over the leading dims, as `to_rank` does, linear.rs:52-58), [S, N, d] against a
    seed-batched one."""
    if hidden.dtype not in _ESIZE or len(hidden.shape) < 2:
        raise ValueError(f"{who}: hidden [.., d] in f32, bf16 or f16")
    d = hidden.shape[-1]
    if weight.batched:
        if len(hidden.shape) != 3 or hidden.shape[0] != weight.seeds:
            raise ValueError(f"{who}: hidden {list(hidden.shape)} against a weight of {weight.seeds} seeds "
                             "(hidden [S, N, d])")
        S, N = hidden.shape[0], hidden.shape[1]
    else:
        S, N = 1, hidden.numel // d
    if d != weight.dim:
        raise ValueError(f"{who}: hidden's d {d} against the weight's {weight.dim}")
    # the head's x.matmul(w) takes one dtype (float.rs:946-949: "matmul: f32 and bf16 (casts are
    # explicit)"), after the shape checks
    same_dtype(hidden.dtype, weight.weight_dtype, "matmul")
    return S, N, d


def _readout_mask_ld(mask: Optional[Tensor], rows: int, V: int, seeds: int = 1):
    """(row stride, stride between seeds) of the readout's u8 keep-mask [.., V]: one row per
    logits row (V, rows / seeds V), one row per seed shared by that seed's rows (0, V; the
    seed-batched head's [S, 1, V]), or one row shared by every row (0, 0)."""
    if mask is None:
        return 0, 0
    if mask.dtype != "u8" or mask.shape[-1] != V:
        raise ValueError("readout: a u8 keep-mask [.., V]")
    if mask.numel == rows * V and rows > 1:
        return V, (rows // seeds) * V
    if mask.numel == V:
        return 0, 0
    if seeds > 1 and mask.numel == seeds * V:
        return 0, V
    raise ValueError("readout: a u8 keep-mask with one row per logits row, one per seed, or one shared row "
                     "(or one that broadcasts to the logits' shape)")


def _readout_mask(mask: Optional[Tensor], logits_shape, rows: int, V: int, seeds: int):
    """The readout's mask and its (row, seed) strides: the forms _readout_mask_ld reads in place,
    or a mask of the logits' rank that broadcasts to them (rl.rs:477-483), broadcast on the
    device first."""
    if mask is not None and mask.dtype == "u8" and mask.shape[-1] == V and len(mask.shape) == len(logits_shape) \
            and mask.numel not in (V, rows * V) and not (seeds > 1 and mask.numel == seeds * V) \
            and all(a == b or a == 1 for a, b in zip(mask.shape, logits_shape)):
        import noetic_ops as ops  # (noetic_ops imports this module)
        mask = ops.copy(mask, ops.Layout.contiguous(mask.shape).broadcast(tuple(logits_shape)))
    return (mask,) + _readout_mask_ld(mask, rows, V, seeds)


def _readout_chunks(S: int, N: int):
    """(seed, first row of the call over all rows, rows) of each call: one seed's rows, at most
    256 per call."""
    for k in range(S):
        for r0 in range(0, N, _READOUT_ROWS):
            yield k, k * N + r0, min(_READOUT_ROWS, N - r0)


def readout_sample_logp(hidden: Tensor, weight: PackedReadout, temperature: float, mask: Optional[Tensor],
                        rng: Optional[Rng], uniforms: Optional[Tensor] = None, debug: bool = False,
                        check: bool = True):
    """One decode step fused at MatmulPrecision::Half: logits = hidden . W (the decoder's head,
    decoder.rs:272,286; linear.rs:52-58) with bf16 operands (an f32 hidden rounded to nearest-even
    first) and f32 accumulation, then sample_logp's inverse-CDF draw and log-probability on them
    (rl.rs:134-141, 475-529), the logits never written. `weight` is the head's weight packed once
    (PackedReadout); hidden is [.., d], or [S, N, d] for a seed-batched weight. Returns (ids, logp)
    shaped like hidden without d, plus with `debug` the f32 logits [.., V], the recomputed crossing
    block [.., 32] and its index."""
    _readout_gate("readout_sample_logp")
    if not (temperature >= 0.0 and math.isfinite(temperature)):
        raise ValueError(f"sample_categorical: temperature {temperature} (must be ≥ 0)")
    S, N, d = _readout_shape(hidden, weight, "readout")
    rows, V, es = S * N, weight.vocab, _ESIZE[hidden.dtype]
    out_shape = hidden.shape[:-1]
    mask, mld, msd = _readout_mask(mask, tuple(out_shape) + (V,), rows, V, S)
    if temperature != 0.0 and uniforms is None:
        if rng is None:
            raise ValueError("sample_categorical: a stream is needed at temperature > 0")
        uniforms = Tensor.from_numpy(rng.uniforms(rows), "f64")
    uniforms = _row_arg(uniforms, rows, "f64", "sample_categorical: uniforms")
    ids, lp, status = IntTensor(out_shape), Tensor(out_shape, "f32"), Tensor(out_shape, "u8")
    dbg = ((Tensor(out_shape + (V,), "f32"), Tensor(out_shape + (32,), "f32"), IntTensor(out_shape)) if debug
           else (None, None, None))
    for k, g0, n in _readout_chunks(S, N):
        at = lambda t, w: None if t is None else t.ptr + g0 * w
        # this call's first mask row: its seed's rows, then its place among them
        mask_at = lambda k, g0: None if mask is None else mask.ptr + k * msd + (g0 - k * N) * mld
        a = NtRlReadoutSampleArgs(at(hidden, d * es), weight.seed_ptr(k if weight.batched else 0), n, V, d, d,
                                  NT_MASK_U8 if mask is not None else NT_MASK_NONE,
                                  _DTCODE[hidden.dtype], mask_at(k, g0),
                                  mld, float(temperature), at(uniforms, 8), at(ids, 4),
                                  at(lp, 4), at(status, 1), at(dbg[0], V * 4), at(dbg[1], 32 * 4), at(dbg[2], 4))
        _check(lib().nt_hip_rl_readout_sample(C.byref(a)), "readout sample")
    if check:
        st = status.to_numpy().ravel()
        bad = np.nonzero(st != NT_ROW_OK)[0]
        if bad.size:
            raise ValueError(f"sample_categorical: position {bad[0]} has no allowed token (every logit −∞ or a NaN)")
    return (ids, lp, *dbg) if debug else (ids, lp)


def readout_score(hidden: Tensor, weight: PackedReadout, temperature: float, mask: Optional[Tensor],
                  tokens: Optional[Tensor], entropy: bool = True, debug: bool = False):
    """The scoring pass fused with the head at MatmulPrecision::Half: logits = hidden . W
    (decoder.rs:272,286) tempered and masked (rl.rs:475-486), then token_log_probs (rl.rs:134-141)
    of `tokens` and, with `entropy`, categorical_entropy (rl.rs:405-414) per row, as `score` gives
    them on written logits, the logits never written. Shapes as readout_sample_logp; tokens are
    shaped like hidden without d. Returns (logp or None, entropy or None), plus with `debug` the f32
    logits [.., V]."""
    _readout_gate("readout_score")
    if not (temperature > 0.0 and math.isfinite(temperature)):
        raise ValueError(f"tempered_logits: temperature {temperature} (must be positive)")
    S, N, d = _readout_shape(hidden, weight, "readout")
    rows, V, es = S * N, weight.vocab, _ESIZE[hidden.dtype]
    out_shape = hidden.shape[:-1]
    if tokens is not None and (tokens.dtype != "i32" or tokens.numel != rows):
        raise ValueError("token_log_probs: tokens shape (the logits' without the vocabulary axis)")
    if tokens is None and not entropy:
        raise ValueError("readout_score: neither log-probabilities nor the entropy asked for")
    mask, mld, msd = _readout_mask(mask, tuple(out_shape) + (V,), rows, V, S)
    lp = Tensor(out_shape, "f32") if tokens is not None else None
    ent = Tensor(out_shape, "f32") if entropy else None
    status = Tensor(out_shape, "u8")
    logits = Tensor(out_shape + (V,), "f32") if debug else None
    for k, g0, n in _readout_chunks(S, N):
        at = lambda t, w: None if t is None else t.ptr + g0 * w
        # this call's first mask row: its seed's rows, then its place among them
        mask_at = lambda k, g0: None if mask is None else mask.ptr + k * msd + (g0 - k * N) * mld
        a = NtRlReadoutScoreArgs(at(hidden, d * es), weight.seed_ptr(k if weight.batched else 0), n, V, d, d,
                                 NT_MASK_U8 if mask is not None else NT_MASK_NONE,
                                 _DTCODE[hidden.dtype], mask_at(k, g0),
                                 mld, float(temperature), at(tokens, 4), at(lp, 4),
                                 at(ent, 4), at(status, 1), at(logits, V * 4))
        _check(lib().nt_hip_rl_readout_score(C.byref(a)), "readout score")
    if tokens is not None:
        st = status.to_numpy().ravel()
        bad = np.nonzero(st == NT_ROW_BAD_TOKEN)[0]
        if bad.size:
            raise IndexError(f"gather index out of range {V} at position {bad[0]}")
    return (lp, ent, logits) if debug else (lp, ent)


def _score(policy, ref, tokens, want_logp, want_ref_logp, want_kl, want_ent, want_stats=False):
    p = _as_tempered(policy)
    rows, V = _rows(p.logits)
    if ref is not None:
        r = _as_tempered(ref)
        if r.logits.shape != p.logits.shape or r.logits.dtype != p.logits.dtype:
            raise ValueError("categorical_kl: reference logits shape")
        if r.temperature != p.temperature or r.mask is not p.mask:
            raise ValueError("the fused scorer takes both sides under one temperature and one vocabulary mask "
                             "(reference_kl)")
    out_shape = p.logits.shape[:-1]
    if tokens is not None and tokens.shape != out_shape:
        raise ValueError("token_log_probs: tokens shape (the logits' without the vocabulary axis)")
    tokens = _row_arg(tokens, rows, "i32", "token_log_probs: tokens")
    mk = lambda want: Tensor(out_shape, "f32") if want else None
    lp, rlp, kl, ent = mk(want_logp), mk(want_ref_logp), mk(want_kl), mk(want_ent)
    stats = None
    if want_stats:
        stats = RowStats(mk(True), mk(True), mk(ref is not None), mk(ref is not None))
    status = Tensor(out_shape, "u8")
    kind, mptr, mld, mrows, _keep = _mask_fields(p, rows, V)
    ptr = lambda t: None if t is None else t.ptr
    sp = (lambda f: ptr(getattr(stats, f))) if stats is not None else (lambda f: None)
    a = NtRlScoreArgs(p.logits.ptr, None if ref is None else _as_tempered(ref).logits.ptr, _dtype_code(p.logits),
                      kind, rows, V, V, mptr, mld, p.temperature, ptr(tokens), ptr(lp), ptr(rlp), ptr(kl), ptr(ent),
                      status.ptr, sp("lse_base"), sp("lse_rest"), sp("ref_lse_base"), sp("ref_lse_rest"), mrows)
    _check(lib().nt_hip_rl_score(C.byref(a)), "score")
    if tokens is not None:
        st = status.to_numpy().ravel()
        bad = np.nonzero(st == NT_ROW_BAD_TOKEN)[0]
        if bad.size:
            raise IndexError(f"gather index out of range {V} at position {bad[0]}")
    if want_stats:
        return lp, rlp, kl, ent, status, stats
    return lp, rlp, kl, ent, status


class RowStats:
    """A scoring pass's per-row log-sum-exp (lse = base + rest, z units), saved for the backward
    in place of the reference's materialised log_softmax output (activation.rs:36-41)."""

    def __init__(self, lse_base, lse_rest, ref_lse_base=None, ref_lse_rest=None):
        self.lse_base, self.lse_rest = lse_base, lse_rest
        self.ref_lse_base, self.ref_lse_rest = ref_lse_base, ref_lse_rest


def score_with_stats(logits, ref_logits, tokens: Optional[Tensor], entropy=True, kl=True):
    """`score` that also returns the RowStats its backward (`score_grad`) needs."""
    lp, rlp, k, ent, _, stats = _score(logits, ref_logits, tokens, tokens is not None,
                                       tokens is not None and ref_logits is not None, kl and ref_logits is not None,
                                       entropy, want_stats=True)
    return lp, rlp, k, ent, stats


def score_grad(logits, ref_logits, tokens: Optional[Tensor], stats: RowStats, kl: Optional[Tensor] = None,
               entropy: Optional[Tensor] = None, g_logp: Optional[Tensor] = None, g_kl: Optional[Tensor] = None,
               g_entropy: Optional[Tensor] = None, grad_dtype: Optional[str] = None) -> Tensor:
    """The fused backward of `score`: d(sum_r g_logp[r] logp[r] + g_kl[r] kl[r] + g_entropy[r]
    entropy[r]) / d logits (the raw logits under `tempered_logits`), in one pass. It follows the
    reference's autograd through log_softmax (activation.rs:36-41), gather, categorical_kl
    (rl.rs:327-338, the reference detached), categorical_entropy (rl.rs:405-414) and the
    temperature's divide. `grad_dtype` defaults to the logits' dtype."""
    p = _as_tempered(logits)
    rows, V = _rows(p.logits)
    if ref_logits is not None and (tuple(_as_tempered(ref_logits).logits.shape) != tuple(p.logits.shape) or
                                   _as_tempered(ref_logits).logits.dtype != p.logits.dtype):
        raise ValueError("categorical_kl: reference logits shape")
    tokens = _row_arg(tokens, rows, "i32", "token_log_probs: tokens")
    kl, entropy = _row_arg(kl, rows, "f32", "score backward: kl"), _row_arg(entropy, rows, "f32", "score backward: entropy")
    g_logp = _row_arg(g_logp, rows, "f32", "score backward: g_logp")
    g_kl = _row_arg(g_kl, rows, "f32", "score backward: g_kl")
    g_entropy = _row_arg(g_entropy, rows, "f32", "score backward: g_entropy")
    for f in ("lse_base", "lse_rest", "ref_lse_base", "ref_lse_rest"):
        _row_arg(getattr(stats, f), rows, "f32", f"score backward: {f}")
    kind, mptr, mld, mrows, _keep = _mask_fields(p, rows, V)
    gdt = grad_dtype or p.logits.dtype
    gcode = {"f32": NT_F32, "bf16": NT_BF16, "f16": NT_F16}.get(gdt)
    if gcode is None:
        raise ValueError(f"gradient dtype {gdt}")
    grad = Tensor(p.logits.shape, gdt)
    ptr = lambda t: None if t is None else t.ptr
    ref = None if ref_logits is None else _as_tempered(ref_logits)
    a = NtRlScoreGradArgs(p.logits.ptr, None if ref is None else ref.logits.ptr, _dtype_code(p.logits), kind, rows,
                          V, V, mptr, mld, p.temperature, ptr(tokens), ptr(stats.lse_base), ptr(stats.lse_rest),
                          ptr(stats.ref_lse_base), ptr(stats.ref_lse_rest), ptr(kl), ptr(entropy), ptr(g_logp),
                          ptr(g_kl), ptr(g_entropy), grad.ptr, gcode, 0, V, mrows)
    _check(lib().nt_hip_rl_score_backward(C.byref(a)), "score backward")
    return grad


def token_log_probs(logits, tokens: Tensor) -> Tensor:
    """rl.rs:134-141: log_softmax(logits)[…, tokens[…]]; `logits` may be a `tempered_logits`.
    16-bit logits are refused as the reference's log_softmax refuses them (at τ == 1, or
    untempered: "sub: bf16 and f32 (casts are explicit)"); `score` with a Tempered triple takes
    them, widened exactly."""
    x = _as_tempered(logits)
    if len(x.logits.shape) < 1:
        raise ValueError("token_log_probs: logits of rank 0")
    if tuple(tokens.shape) != tuple(x.logits.shape[:-1]):
        raise ValueError("token_log_probs: tokens shape (the logits' without the vocabulary axis)")
    log_softmax_dtype(_logits_dtype(logits))
    return _score(logits, None, tokens, True, False, False, False)[0]


def score(logits, ref_logits, tokens: Optional[Tensor], entropy=True, kl=True):
    """The fused scoring pass: (logp, ref_logp, exact KL, entropy) per position in one read of
    both logits (token_log_probs x2, categorical_kl / reference_kl, categorical_entropy)."""
    lp, rlp, k, ent, _ = _score(logits, ref_logits, tokens, tokens is not None,
                                tokens is not None and ref_logits is not None, kl and ref_logits is not None, entropy)
    return lp, rlp, k, ent


def _f32_storage(t: Optional[Tensor], what: str) -> Optional[Tensor]:
    """A per-token float argument as the f32 values the kernels read: f32 as it is, bf16 and f16
    widened exactly on the device (the reference computes 16-bit storage in f32, fdisp,
    float.rs:43-58); any other dtype is refused (the reference's float Tensor has no other)."""
    if t is None or t.dtype == "f32":
        return t
    if t.dtype in _HALF:
        import noetic_ops as ops  # (noetic_ops imports this module)
        return ops.cast(t, ops.Layout.contiguous(t.shape), "f32")
    raise ValueError(f"{what}: a float tensor (f32, bf16 or f16), not {t.dtype}")


def _reduce(per: Tensor, mask: Optional[Tensor], reduction: TokenReduction) -> Tensor:
    if len(per.shape) != 3:
        raise ValueError("per-token values [S, B, T]")
    if mask is not None and tuple(mask.shape) != tuple(per.shape):
        raise AssertionError("rl: mask shape")
    per, mask = _f32_storage(per, "reduce_tokens"), _f32_storage(mask, "rl: mask")
    S, B, T = per.shape
    reduction = TokenReduction(reduction)
    if reduction == TokenReduction.NONE:
        return per
    out = Tensor((S, B) if reduction == TokenReduction.PER_SEQUENCE else (S,), "f32")
    _check(lib().nt_hip_rl_reduce_tokens(per.ptr, None if mask is None else mask.ptr, S, B, T, int(reduction),
                                         out.ptr), "reduce_tokens")
    return out


def _zero_masked(per: Tensor, mask: Optional[Tensor]) -> Tensor:
    """zero_masked (rl.rs:100-102): a select, so a non-finite value at a masked position does
    not leak."""
    if mask is None:
        return per
    if mask.shape != per.shape:
        raise AssertionError("rl: mask shape")
    per, mask = _f32_storage(per, "zero_masked"), _f32_storage(mask, "rl: mask")
    out = Tensor(per.shape, "f32")
    _check(lib().nt_hip_rl_zero_masked(per.ptr, mask.ptr, per.numel, out.ptr), "zero_masked")
    return out


def categorical_kl(logits, ref_logits, mask: Optional[Tensor] = None,
                   reduction: TokenReduction = TokenReduction.TOKEN_MEAN) -> Tensor:
    """rl.rs:327-338 (exact KL per position, reduced per seed); both sides' log_softmax keep the
    reference's dtype refusal (as token_log_probs)."""
    x = _as_tempered(logits)
    if len(x.logits.shape) != 4:
        raise ValueError("categorical_kl: logits [S, B, T, V]")
    if tuple(_as_tempered(ref_logits).logits.shape) != tuple(x.logits.shape):
        raise ValueError("categorical_kl: reference logits shape")
    log_softmax_dtype(_logits_dtype(logits))
    log_softmax_dtype(_logits_dtype(ref_logits))
    kl = _score(logits, ref_logits, None, False, False, True, False)[2]
    return _reduce(_zero_masked(kl, mask), mask, reduction)


def reference_kl(logits: Tensor, ref_logits: Tensor, temperature: float, vocab_mask: Optional[Tensor],
                 mask: Optional[Tensor] = None, reduction: TokenReduction = TokenReduction.TOKEN_MEAN) -> Tensor:
    """rl.rs:347-351."""
    return categorical_kl(tempered_logits(logits, temperature, vocab_mask),
                          tempered_logits(ref_logits, temperature, vocab_mask), mask, reduction)


def categorical_entropy(logits, mask: Optional[Tensor] = None,
                        reduction: TokenReduction = TokenReduction.TOKEN_MEAN) -> Tensor:
    """rl.rs:405-414; log_softmax's dtype refusal as token_log_probs."""
    x = _as_tempered(logits)
    if len(x.logits.shape) != 4:
        raise ValueError("categorical_entropy: logits [S, B, T, V]")
    log_softmax_dtype(_logits_dtype(logits))
    ent = _score(logits, None, None, False, False, False, True)[3]
    return _reduce(_zero_masked(ent, mask), mask, reduction)


def kl_estimate(logp: Tensor, ref_logp: Tensor, estimator: KlEstimator, delta_clamp: Optional[float] = None,
                mask: Optional[Tensor] = None, reduction: TokenReduction = TokenReduction.TOKEN_MEAN) -> Tensor:
    """rl.rs:380-400."""
    if len(logp.shape) != 3:
        raise ValueError("kl_estimate: logp [S, B, T]")
    if logp.shape != ref_logp.shape:
        raise ValueError("kl_estimate: reference log-probabilities shape")
    if delta_clamp is not None and not delta_clamp > 0.0:
        raise ValueError(f"kl_estimate: δ clamp {delta_clamp} (need b > 0)")
    if mask is not None and mask.shape != logp.shape:
        raise AssertionError("rl: mask shape")
    same_dtype(ref_logp.dtype, logp.dtype, "sub")  # δ = ref_logp − logp (rl.rs:392)
    logp, ref_logp = _f32_storage(logp, "kl_estimate"), _f32_storage(ref_logp, "kl_estimate")
    mask = _f32_storage(mask, "rl: mask")
    out = Tensor(logp.shape, "f32")
    _check(lib().nt_hip_rl_kl_estimate(logp.ptr, ref_logp.ptr, None if mask is None else mask.ptr, logp.numel,
                                       int(estimator), 0.0 if delta_clamp is None else float(delta_clamp), out.ptr),
           "kl_estimate")
    return _reduce(out, mask, reduction)


def _reduced_shape(shape, reduction: TokenReduction):
    S, B, _ = shape
    return {TokenReduction.NONE: tuple(shape), TokenReduction.PER_SEQUENCE: (S, B)}.get(TokenReduction(reduction), (S,))


def reduce_tokens_backward(mask: Optional[Tensor], shape, reduction: TokenReduction, upstream: Optional[Tensor] = None,
                           scale: float = 1.0, local: Optional[Tensor] = None) -> Tensor:
    """The gradient of reduce_tokens(zero_masked(per)) (rl.rs:69-102) with respect to per, times
    `scale` and the per-token derivative `local` (a loss's d per / d logp): [S, B, T], 0 at
    masked positions. `upstream` is the reduced output's gradient (None: ones)."""
    S, B, T = shape
    reduction = TokenReduction(reduction)
    if upstream is not None and tuple(upstream.shape) != _reduced_shape(shape, reduction):
        raise ValueError(f"reduce_tokens backward: upstream shape {upstream.shape} for {reduction.name}")
    if mask is not None and tuple(mask.shape) != (S, B, T):
        raise AssertionError("rl: mask shape")
    if local is not None and tuple(local.shape) != (S, B, T):
        raise ValueError("reduce_tokens backward: per-token derivative [S, B, T]")
    mask = _f32_storage(mask, "rl: mask")
    upstream = _f32_storage(upstream, "reduce_tokens backward")
    local = _f32_storage(local, "reduce_tokens backward")
    out = Tensor((S, B, T), "f32")
    _check(lib().nt_hip_rl_reduce_tokens_backward(None if mask is None else mask.ptr, S, B, T, int(reduction),
                                                  None if upstream is None else upstream.ptr, float(scale),
                                                  None if local is None else local.ptr, out.ptr),
           "reduce_tokens backward")
    return out


def kl_estimate_backward(logp: Tensor, ref_logp: Tensor, estimator: KlEstimator, delta_clamp: Optional[float] = None,
                         mask: Optional[Tensor] = None, reduction: TokenReduction = TokenReduction.TOKEN_MEAN,
                         upstream: Optional[Tensor] = None, scale: float = 1.0) -> Tensor:
    """d (scale * kl_estimate(...)) / d logp (rl.rs:380-400), [S, B, T]; the reference logp is
    detached."""
    if logp.shape != ref_logp.shape or len(logp.shape) != 3:
        raise ValueError("kl_estimate: logp and reference log-probabilities [S, B, T]")
    if delta_clamp is not None and not delta_clamp > 0.0:
        raise ValueError(f"kl_estimate: δ clamp {delta_clamp} (need b > 0)")
    if mask is not None and mask.shape != logp.shape:
        raise AssertionError("rl: mask shape")
    same_dtype(ref_logp.dtype, logp.dtype, "sub")  # δ = ref_logp − logp (rl.rs:392)
    logp, ref_logp = _f32_storage(logp, "kl_estimate"), _f32_storage(ref_logp, "kl_estimate")
    mask = _f32_storage(mask, "rl: mask")
    local = Tensor(logp.shape, "f32")
    _check(lib().nt_hip_rl_kl_estimate_backward(logp.ptr, ref_logp.ptr, None if mask is None else mask.ptr,
                                                logp.numel, int(estimator),
                                                0.0 if delta_clamp is None else float(delta_clamp), local.ptr),
           "kl_estimate backward")
    return reduce_tokens_backward(mask, logp.shape, reduction, upstream, scale, local)


LOG_RATIO_CLAMP = 20.0  # rl.rs:146


class Clip:
    """clipped_policy_loss's settings (rl.rs:161-201): the ratio clipped to [1 - low, 1 + high];
    `dual` (c > 1) caps a negative-advantage token's loss at -c A; `log_ratio_clamp` bounds
    logp - old_logp (None: unbounded)."""

    def __init__(self, low: float, high: float, dual: Optional[float] = None,
                 log_ratio_clamp: Optional[float] = LOG_RATIO_CLAMP):
        self.low, self.high, self.dual, self.log_ratio_clamp = float(low), float(high), dual, log_ratio_clamp

    @staticmethod
    def new(low: float, high: float) -> "Clip":
        return Clip(low, high)

    @staticmethod
    def symmetric(eps: float) -> "Clip":
        return Clip(eps, eps)

    def with_dual(self, c: float) -> "Clip":
        return Clip(self.low, self.high, c, self.log_ratio_clamp)

    def with_log_ratio_clamp(self, b: Optional[float]) -> "Clip":
        return Clip(self.low, self.high, self.dual, b)

    def check(self):
        if not (0.0 <= self.low < 1.0 and self.high >= 0.0 and math.isfinite(self.low) and math.isfinite(self.high)):
            raise ValueError(f"clip range [1 − {self.low}, 1 + {self.high}] (need 0 ≤ low < 1, 0 ≤ high)")
        if self.dual is not None and not (self.dual > 1.0 and math.isfinite(self.dual)):
            raise ValueError(f"dual clip {self.dual} (need c > 1)")
        if self.log_ratio_clamp is not None and not self.log_ratio_clamp > 0.0:
            raise ValueError(f"log-ratio clamp {self.log_ratio_clamp} (need b > 0)")


def check_scored_finite(what: str, logp: Tensor, mask: Optional[Tensor] = None) -> Optional[str]:
    """rl.rs:200-212: None when every scored log-probability (mask != 0) is finite, else the
    reference's message naming the first position that is not (a host read)."""
    v = logp.to_f64().ravel()
    m = None if mask is None else mask.to_f64().ravel()
    bad = ~np.isfinite(v) if m is None else (~np.isfinite(v)) & (m != 0.0)
    idx = np.nonzero(bad)[0]
    if idx.size == 0:
        return None
    i = int(idx[0])
    val = "inf" if v[i] == np.inf else ("-inf" if v[i] == -np.inf else "NaN")
    return f"{what}: the scored log-probability at flat position {i} is {val} (not finite)"


# The reference runs check_scored_finite in the losses in debug builds (rl.rs:214-221). Here it is
# opt-in, since it reads the log-probabilities back to the host: NOETIC_RL_DEBUG_CHECKS=1.
DEBUG_CHECKS = os.environ.get("NOETIC_RL_DEBUG_CHECKS") == "1"


def _debug_check(what: str, logp: Tensor, mask: Optional[Tensor]):
    if DEBUG_CHECKS:
        e = check_scored_finite(what, logp, mask)
        if e is not None:
            raise AssertionError(e)


def _policy_loss(kind: int, what: str, logp: Tensor, old_logp: Optional[Tensor], weights: Tensor,
                 mask: Optional[Tensor], clip: Optional[Clip]):
    """(loss, dloss, hit) per token from nt_hip_rl_policy_loss, with the reference's shape checks
    (token_weights rl.rs:106-122, mask_or_ones 58-66)."""
    if len(logp.shape) != 3:
        raise ValueError(f"{what}: logp [S, B, T]")
    S, B, T = logp.shape
    if len(weights.shape) == 2:
        if tuple(weights.shape) != (S, B):
            raise ValueError(f"{what}: per-sequence weights [S, B]")
        per_seq = 1
    elif len(weights.shape) == 3:
        if tuple(weights.shape) != (S, B, T):
            raise ValueError(f"{what}: per-token weights [S, B, T]")
        per_seq = 0
    else:
        raise ValueError(f"{what}: weights of rank {len(weights.shape)} (per-sequence [S, B] or per-token [S, B, T])")
    if mask is not None and mask.shape != logp.shape:
        raise ValueError("rl: mask shape")
    if old_logp is not None and old_logp.shape != logp.shape:
        raise ValueError("rl: old log-probabilities shape")
    if clip is not None:
        clip.check()
    # The reference's binary ops between them (same_dtype): PG's logp · w (rl.rs:232); PPO's
    # logp − old (rl.rs:240), then r · A with r = exp(log-ratio) computed in f32 (rl.rs:270);
    # clip_fraction compares A with 0 only (rl.rs:303-304). A mask meets no other operand.
    if kind == NT_LOSS_PG:
        same_dtype(logp.dtype, weights.dtype, "mul")
    else:
        same_dtype(logp.dtype, old_logp.dtype, "sub")
        if what != "clip_fraction":
            same_dtype("f32", weights.dtype, "mul")
    if what != "clip_fraction":
        _debug_check(what, logp, mask)
        if old_logp is not None:
            _debug_check(f"{what} (old log-probabilities)", old_logp, mask)
    logp, old_logp = _f32_storage(logp, what), _f32_storage(old_logp, what)
    weights, mask = _f32_storage(weights, what), _f32_storage(mask, "rl: mask")
    loss, dloss, hit = Tensor(logp.shape, "f32"), Tensor(logp.shape, "f32"), Tensor(logp.shape, "f32")
    a = NtRlPolicyLossArgs(logp.ptr, None if old_logp is None else old_logp.ptr, weights.ptr,
                           None if mask is None else mask.ptr, S, B, T, kind, per_seq,
                           clip.low if clip else 0.0, clip.high if clip else 0.0,
                           (clip.dual or 0.0) if clip else 0.0,
                           (clip.log_ratio_clamp or 0.0) if clip else 0.0, loss.ptr, dloss.ptr, hit.ptr)
    _check(lib().nt_hip_rl_policy_loss(C.byref(a)), what)
    return loss, dloss, hit


def policy_gradient_loss(logp: Tensor, weights: Tensor, mask: Optional[Tensor] = None,
                         reduction: TokenReduction = TokenReduction.TOKEN_MEAN) -> Tensor:
    """rl.rs:228-235: -w logp per scored token, reduced per seed."""
    loss, _, _ = _policy_loss(NT_LOSS_PG, "policy_gradient_loss", logp, None, weights, mask, None)
    return _reduce(loss, mask, reduction)


def policy_gradient_loss_backward(logp: Tensor, weights: Tensor, mask: Optional[Tensor] = None,
                                  reduction: TokenReduction = TokenReduction.TOKEN_MEAN,
                                  upstream: Optional[Tensor] = None, scale: float = 1.0) -> Tensor:
    """d (scale * policy_gradient_loss(...)) / d logp, [S, B, T] (the weights are detached)."""
    _, dloss, _ = _policy_loss(NT_LOSS_PG, "policy_gradient_loss", logp, None, weights, mask, None)
    return reduce_tokens_backward(mask, logp.shape, reduction, upstream, scale, dloss)


def clipped_policy_loss(logp: Tensor, old_logp: Tensor, advantages: Tensor, mask: Optional[Tensor], clip: Clip,
                        reduction: TokenReduction = TokenReduction.TOKEN_MEAN) -> Tensor:
    """rl.rs:265-287: PPO's clipped surrogate as a loss, reduced per seed."""
    loss, _, _ = _policy_loss(NT_LOSS_PPO, "clipped_policy_loss", logp, old_logp, advantages, mask, clip)
    return _reduce(loss, mask, reduction)


def clipped_policy_loss_backward(logp: Tensor, old_logp: Tensor, advantages: Tensor, mask: Optional[Tensor],
                                 clip: Clip, reduction: TokenReduction = TokenReduction.TOKEN_MEAN,
                                 upstream: Optional[Tensor] = None, scale: float = 1.0) -> Tensor:
    """d (scale * clipped_policy_loss(...)) / d logp, [S, B, T] (old_logp and the advantages are
    detached)."""
    _, dloss, _ = _policy_loss(NT_LOSS_PPO, "clipped_policy_loss", logp, old_logp, advantages, mask, clip)
    return reduce_tokens_backward(mask, logp.shape, reduction, upstream, scale, dloss)


def clip_fraction(logp: Tensor, old_logp: Tensor, advantages: Tensor, mask: Optional[Tensor], clip: Clip) -> Tensor:
    """rl.rs:293-317: per seed [S], the fraction of scored tokens a bound gives no gradient."""
    _, _, hit = _policy_loss(NT_LOSS_PPO, "clip_fraction", logp, old_logp, advantages, mask, clip)
    return _reduce(hit, mask, TokenReduction.TOKEN_MEAN)


class GroupNorm:
    """rl.rs:417-424: `GroupNorm.MEAN_ONLY` (r - mean) or `GroupNorm.std(eps, unbiased)`
    ((r - mean) / (std + eps)). The functions also take the strings "mean" and "std"."""

    def __init__(self, kind: str, eps: float = 0.0, unbiased: bool = True):
        self.kind, self.eps, self.unbiased = kind, float(eps), bool(unbiased)

    @staticmethod
    def std(eps: float, unbiased: bool) -> "GroupNorm":
        return GroupNorm("std", eps, unbiased)


GroupNorm.MEAN_ONLY = GroupNorm("mean")


def _norm(norm, eps, unbiased):
    if isinstance(norm, GroupNorm):
        return norm.kind, norm.eps, norm.unbiased
    return norm, eps, unbiased


def group_advantages(rewards: Sequence[float], n: int, norm="mean", eps: float = 0.0,
                     unbiased: bool = True) -> np.ndarray:
    """rl.rs:436-463, on the host in f64 as the reference computes it. norm: a GroupNorm, or
    "mean" (MeanOnly) / "std" (Std{eps, unbiased})."""
    norm, eps, unbiased = _norm(norm, eps, unbiased)
    r = np.asarray(rewards, dtype=np.float64).ravel()
    if not (n >= 1 and r.size % n == 0):
        raise ValueError(f"group_advantages: {r.size} rewards in groups of {n}")
    if norm == "std":
        if not eps >= 0.0:
            raise ValueError(f"group_advantages: ε {eps} < 0")
        if unbiased and n < 2:
            raise ValueError("group_advantages: the sample standard deviation needs groups of at least 2")
    out = np.empty_like(r)
    for g in range(0, r.size, n):
        grp = r[g:g + n]
        if grp.min() == grp.max():
            out[g:g + n] = 0.0
            continue
        mean = sum(grp.tolist()) / n
        scale = 1.0
        if norm == "std":
            ss = sum((x - mean) * (x - mean) for x in grp.tolist())
            scale = math.sqrt(ss / ((n - 1) if unbiased else n)) + eps
        out[g:g + n] = [(x - mean) / scale for x in grp.tolist()]
    return out


def group_advantages_tensor(rewards: Tensor, norm="mean", eps: float = 0.0, unbiased: bool = True) -> Tensor:
    """rl.rs:465-469: the last axis grouped, computed on the device (f64 per group, the
    reference's host arithmetic) with no host round trip; same shape, f32. The reference's result
    has the rewards' dtype through `from_f64s`, which stores 16-bit dtypes as f32 (fdisp,
    float.rs:256-260): bf16 and f16 rewards, read exactly widened, give f32 as well."""
    norm, eps, unbiased = _norm(norm, eps, unbiased)
    if len(rewards.shape) == 0:
        raise ValueError("group_advantages_tensor: rewards of rank 0")
    if rewards.dtype not in ("f32",) + _HALF:
        raise ValueError(f"group_advantages_tensor: rewards of dtype {rewards.dtype} (f32, bf16 or f16)")
    if norm not in ("mean", "std"):
        raise ValueError(f"group_advantages: norm {norm!r} (mean or std)")
    n = rewards.shape[-1]
    if rewards.dtype in _HALF:
        import noetic_ops as ops  # (noetic_ops imports this module)
        rewards = ops.cast(rewards, ops.Layout.contiguous(rewards.shape), "f32")  # exact
    out = Tensor(rewards.shape, "f32")
    _check(lib().nt_hip_rl_group_advantages(rewards.ptr, rewards.numel // max(n, 1), n, 1 if norm == "std" else 0,
                                            float(eps), 1 if unbiased else 0, out.ptr), "group_advantages")
    return out
