"""ctypes front of the CPU oracle (liboracle.so, built from oracle.c).

TEST INFRASTRUCTURE ONLY: tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use
it as the checker and as the timed CPU baseline. The product (noetic-tensor_amd/) never
imports it. Every function cites the reference (shyble/noetic-tensor 0.7.0) code it restates.
"""
import ctypes as C
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")

_c_double_p = C.POINTER(C.c_double)
_c_float_p = C.POINTER(C.c_float)
_c_int64_p = C.POINTER(C.c_int64)
_c_u8_p = C.POINTER(C.c_uint8)


class ChaCha(C.Structure):
    """rand_chacha 0.3.1 ChaCha20Rng state (oracle.h `or_chacha`)."""

    _fields_ = [("key", C.c_uint32 * 8), ("counter", C.c_uint64), ("buf", C.c_uint32 * 16),
                ("idx", C.c_int)]


class RowStats(C.Structure):
    _fields_ = [("m", C.c_double), ("S", C.c_double), ("lse", C.c_double),
                ("argmax", C.c_int64), ("status", C.c_int)]


def build():
    """Compile liboracle.so with the committed Makefile."""
    import subprocess
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = C.CDLL(_LIB_PATH)
        L.or_sha256.argtypes = [C.c_char_p, C.c_size_t, C.c_char_p]
        L.or_chacha_block.argtypes = [C.POINTER(C.c_uint32), C.c_uint64, C.c_uint64, C.POINTER(C.c_uint32)]
        L.or_rng_derive.argtypes = [C.POINTER(ChaCha), C.c_uint64, C.c_char_p, C.c_size_t]
        L.or_chacha_next_u32.argtypes = [C.POINTER(ChaCha)]
        L.or_chacha_next_u32.restype = C.c_uint32
        L.or_chacha_next_u64.argtypes = [C.POINTER(ChaCha)]
        L.or_chacha_next_u64.restype = C.c_uint64
        L.or_uniform_open01.argtypes = [C.c_uint64]
        L.or_uniform_open01.restype = C.c_double
        L.or_rng_uniforms.argtypes = [C.POINTER(ChaCha), C.c_size_t, _c_double_p]
        L.or_rng_normal.argtypes = [C.POINTER(ChaCha)]
        L.or_rng_normal.restype = C.c_double
        L.or_rng_gen_f64.argtypes = [C.POINTER(ChaCha)]
        L.or_rng_gen_f64.restype = C.c_double
        L.or_bf16_from_f32.argtypes = [C.c_float]
        L.or_bf16_from_f32.restype = C.c_uint16
        L.or_tempered_row.argtypes = [_c_float_p, C.c_int64, C.c_double, _c_float_p, _c_u8_p, _c_float_p]
        L.or_row_stats.argtypes = [_c_float_p, C.c_int64]
        L.or_row_stats.restype = RowStats
        L.or_token_logp.argtypes = [_c_float_p, C.c_int64, C.c_int64]
        L.or_token_logp.restype = C.c_double
        L.or_entropy.argtypes = [_c_float_p, C.c_int64]
        L.or_entropy.restype = C.c_double
        L.or_kl.argtypes = [_c_float_p, _c_float_p, C.c_int64]
        L.or_kl.restype = C.c_double
        L.or_score_grad_row.argtypes = [_c_float_p, _c_float_p, C.c_int64, C.c_int64, C.c_double, C.c_double,
                                        C.c_double, _c_double_p]
        L.or_score_grad_row.restype = C.c_int
        L.or_sample_invcdf.argtypes = [_c_float_p, C.c_int64, C.c_double, _c_double_p]
        L.or_sample_invcdf.restype = C.c_int64
        L.or_kl_estimate.argtypes = [_c_double_p, _c_double_p, _c_double_p, C.c_int64, C.c_int, C.c_double, _c_double_p]
        L.or_reduce_tokens.argtypes = [_c_double_p, _c_double_p, C.c_int64, C.c_int64, C.c_int64, C.c_int, _c_double_p]
        L.or_reduce_tokens.restype = C.c_int64
        L.or_reference_rnd_f32.argtypes = [C.c_uint64, C.c_uint64, C.c_int64, C.c_float, C.c_float, _c_float_p]
        L.or_reference_rnd_f64.argtypes = [C.c_uint64, C.c_uint64, C.c_int64, C.c_double, C.c_double, _c_double_p]
        L.or_policy_loss.argtypes = [C.c_int, C.c_int64, C.c_int64, _c_double_p, _c_double_p, _c_double_p, C.c_int,
                                     _c_double_p, C.c_double, C.c_double, C.c_double, C.c_double, _c_double_p,
                                     _c_double_p, _c_double_p]
        L.or_reduce_tokens_backward.argtypes = [_c_double_p, C.c_int64, C.c_int64, C.c_int64, C.c_int, _c_double_p,
                                                C.c_double, _c_double_p, _c_double_p]
        L.or_kl_estimate_grad.argtypes = [_c_double_p, _c_double_p, _c_double_p, C.c_int64, C.c_int, C.c_double,
                                          _c_double_p]
        L.or_group_advantages.argtypes = [_c_double_p, C.c_int64, C.c_int64, C.c_int, C.c_double, C.c_int, _c_double_p]
        L.or_group_advantages.restype = C.c_int
        L.or_cpuref_log_softmax_f64.argtypes = [_c_double_p, C.c_int64, C.c_int64, _c_double_p]
        L.or_unrolled_sum_f32.argtypes = [_c_float_p, C.c_int64]
        L.or_unrolled_sum_f32.restype = C.c_float
        L.or_cpuref_log_softmax.argtypes = [_c_float_p, C.c_int64, C.c_int64, _c_float_p]
        L.or_cpuref_sample_logp.argtypes = [_c_float_p, C.c_int64, C.c_int64, C.c_double, _c_u8_p, C.c_int64,
                                            C.POINTER(ChaCha), _c_int64_p, _c_float_p]
        L.or_cpuref_sample_logp.restype = C.c_int64
        L.or_cpuref_sample_gumbel.argtypes = [_c_float_p, C.c_int64, C.c_int64, C.c_double, _c_float_p, C.c_int64,
                                              _c_u8_p, C.c_int64, C.POINTER(ChaCha), _c_int64_p]
        L.or_cpuref_sample_gumbel.restype = C.c_int64
        L.or_cpufast_sample_logp.argtypes = [_c_float_p, C.c_int64, C.c_int64, C.c_double, _c_u8_p, C.c_int64,
                                             C.POINTER(ChaCha), C.c_int, _c_int64_p, _c_float_p]
        L.or_cpufast_sample_logp.restype = C.c_int64
        L.or_cpu_sample_logp_invcdf.argtypes = [_c_float_p, C.c_int64, C.c_int64, C.c_double, _c_u8_p, C.c_int64,
                                                _c_double_p, _c_int64_p, _c_float_p, C.c_int]
        L.or_cpu_sample_logp_invcdf.restype = C.c_int64
        L.or_matmul_f32.argtypes = [_c_float_p, C.c_int64, C.c_int64, _c_float_p, C.c_int64, C.c_int64, C.c_int64,
                                    C.c_int64, C.c_int64, _c_float_p]
        _lib = L
    return _lib


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _ptr(a, ty):
    return a.ctypes.data_as(ty)


# ----------------------------------------------------------------------------- hashing / rng

def sha256(data: bytes) -> bytes:
    out = C.create_string_buffer(32)
    lib().or_sha256(data, len(data), out)
    return out.raw


def chacha_block(key_words, counter, stream=0):
    key = (C.c_uint32 * 8)(*key_words)
    out = (C.c_uint32 * 16)()
    lib().or_chacha_block(key, counter, stream, out)
    return list(out)


class Rng:
    """rng::derive(root, label) (src/rng.rs:9-17) as the oracle restates it."""

    def __init__(self, root: int, label: str):
        self.s = ChaCha()
        b = label.encode()
        lib().or_rng_derive(C.byref(self.s), root, b, len(b))

    def next_u32(self):
        return lib().or_chacha_next_u32(C.byref(self.s))

    def next_u64(self):
        return lib().or_chacha_next_u64(C.byref(self.s))

    def uniforms(self, n):
        out = np.empty(n, dtype=np.float64)
        lib().or_rng_uniforms(C.byref(self.s), n, _ptr(out, _c_double_p))
        return out

    def normals(self, n):
        L = lib()
        return np.array([L.or_rng_normal(C.byref(self.s)) for _ in range(n)], dtype=np.float64)

    def gen_f64(self, n):
        L = lib()
        return np.array([L.or_rng_gen_f64(C.byref(self.s)) for _ in range(n)], dtype=np.float64)


def uniform_open01(k: int) -> float:
    return lib().or_uniform_open01(k)


# ----------------------------------------------------------------------------- bf16

def bf16_from_f32(x):
    """Vectorised restatement of half.rs:16-23 (checked against the C scalar in the tests)."""
    x = _f32(x)
    b = x.view(np.uint32).astype(np.uint64)
    nan = np.isnan(x)
    rounded = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16) & 0xFFFF
    quiet = ((b >> 16) | 0x0040) & 0xFFFF
    return np.where(nan, quiet, rounded).astype(np.uint16)


def bf16_to_f32(h):
    return (np.asarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def bf16_from_f32_scalar(x: float) -> int:
    return lib().or_bf16_from_f32(x)


# ----------------------------------------------------------------------------- row oracle

def tempered(x, tau, addmask=None, keep=None):
    """tempered_logits of rows [R, V] (rl.rs:475-486). keep: u8 [R or 1, V]; addmask: f32."""
    x = _f32(np.atleast_2d(x))
    R, V = x.shape
    z = np.empty_like(x)
    for r in range(R):
        am = None if addmask is None else _f32(np.atleast_2d(addmask)[r if np.atleast_2d(addmask).shape[0] > 1 else 0])
        kp = None if keep is None else np.ascontiguousarray(np.atleast_2d(keep)[r if np.atleast_2d(keep).shape[0] > 1 else 0], dtype=np.uint8)
        lib().or_tempered_row(_ptr(x[r], _c_float_p), V, tau,
                              None if am is None else _ptr(am, _c_float_p),
                              None if kp is None else _ptr(kp, _c_u8_p), _ptr(z[r], _c_float_p))
    return z


def row_stats(z):
    z = _f32(z)
    return lib().or_row_stats(_ptr(z, _c_float_p), z.shape[-1])


def token_logp(z, tokens):
    z = _f32(np.atleast_2d(z))
    return np.array([lib().or_token_logp(_ptr(z[r], _c_float_p), z.shape[1], int(tokens[r]))
                     for r in range(z.shape[0])])


def entropy(z):
    z = _f32(np.atleast_2d(z))
    return np.array([lib().or_entropy(_ptr(z[r], _c_float_p), z.shape[1]) for r in range(z.shape[0])])


def kl(z, r):
    z = _f32(np.atleast_2d(z))
    r = _f32(np.atleast_2d(r))
    return np.array([lib().or_kl(_ptr(z[i], _c_float_p), _ptr(r[i], _c_float_p), z.shape[1])
                     for i in range(z.shape[0])])


def score_grad(z, tokens=None, r=None, g_lp=None, g_kl=None, g_h=None, tau=1.0):
    """d(g_lp logp + g_kl KL + g_h H)/dx per row, in f64, for rows of tempered logits z (f32)
    with z = x / tau + mask: the z gradient (or_score_grad_row) divided by tau."""
    z = _f32(np.atleast_2d(z))
    R, V = z.shape
    rr = None if r is None else _f32(np.atleast_2d(r))
    out = np.empty((R, V), dtype=np.float64)
    col = lambda a, i: 0.0 if a is None else float(np.ravel(a)[i])
    for i in range(R):
        tok = -1 if tokens is None else int(np.ravel(tokens)[i])
        lib().or_score_grad_row(_ptr(z[i], _c_float_p), None if rr is None else _ptr(rr[i], _c_float_p), V, tok,
                                col(g_lp, i), col(g_kl, i), col(g_h, i), _ptr(out[i], _c_double_p))
    return out / tau


def sample_invcdf(z, u):
    """(ids, edge distances) of the inverse-CDF sampler on tempered rows z [R, V]."""
    z = _f32(np.atleast_2d(z))
    ids = np.empty(z.shape[0], dtype=np.int64)
    edges = np.empty(z.shape[0], dtype=np.float64)
    e = C.c_double()
    for r in range(z.shape[0]):
        ids[r] = lib().or_sample_invcdf(_ptr(z[r], _c_float_p), z.shape[1], float(u[r]), C.byref(e))
        edges[r] = e.value
    return ids, edges


def argmax_first(z):
    z = _f32(np.atleast_2d(z))
    return np.array([row_stats(z[r]).argmax for r in range(z.shape[0])], dtype=np.int64)


def kl_estimate(lp, lr, est, clamp=None, mask=None):
    lp = np.ascontiguousarray(lp, dtype=np.float64).ravel()
    lr = np.ascontiguousarray(lr, dtype=np.float64).ravel()
    m = None if mask is None else np.ascontiguousarray(mask, dtype=np.float64).ravel()
    out = np.empty_like(lp)
    lib().or_kl_estimate(_ptr(lp, _c_double_p), _ptr(lr, _c_double_p),
                         None if m is None else _ptr(m, _c_double_p), lp.size, est,
                         0.0 if clamp is None else float(clamp), _ptr(out, _c_double_p))
    return out


REDUCTIONS = {"none": 0, "sum": 1, "token_mean": 2, "per_sequence": 3, "sequence_mean": 4}


def reduce_tokens(per, mask, shape, reduction):
    S, B, T = shape
    per = np.ascontiguousarray(per, dtype=np.float64).ravel()
    m = None if mask is None else np.ascontiguousarray(mask, dtype=np.float64).ravel()
    out = np.empty(S * B * T, dtype=np.float64)
    n = lib().or_reduce_tokens(_ptr(per, _c_double_p), None if m is None else _ptr(m, _c_double_p),
                               S, B, T, REDUCTIONS[reduction], _ptr(out, _c_double_p))
    return out[:n]


# rand_core 0.6.4's seed_from_u64 increment for its PCG32 steps
PCG32_INC = 11634580027462260723


def reference_rnd_f32(seed, n, lo, hi):
    """The reference's test helper rnd (src/tensor/tests/mod.rs:28-31): ChaCha8Rng::seed_from_u64
    then gen_range(lo..hi) as f32 (or_reference_rnd_f32)."""
    out = np.empty(n, dtype=np.float32)
    lib().or_reference_rnd_f32(seed, PCG32_INC, n, lo, hi, _ptr(out, _c_float_p))
    return out


def reference_rnd_f64(seed, n, lo, hi):
    """The nn tests' helper rnd (src/nn/tests/mod.rs:35-38): ChaCha8Rng::seed_from_u64 then
    gen_range(lo..hi) as f64 (or_reference_rnd_f64)."""
    out = np.empty(n, dtype=np.float64)
    lib().or_reference_rnd_f64(seed, PCG32_INC, n, lo, hi, _ptr(out, _c_double_p))
    return out


def _d(a):
    return None if a is None else np.ascontiguousarray(a, dtype=np.float64).ravel()


def _dp(a):
    return None if a is None else _ptr(a, _c_double_p)


def policy_loss(kind, lp, old, w, mask, T, per_seq=False, low=0.2, high=0.2, dual=None, clamp=20.0):
    """(loss, dloss, hit) per token, f64 (or_policy_loss): kind "pg" or "ppo"; dual/clamp None
    for none."""
    lp, old, w, m = _d(lp), _d(old), _d(w), _d(mask)
    n = lp.size
    loss, dloss, hit = np.empty(n), np.empty(n), np.empty(n)
    lib().or_policy_loss(0 if kind == "pg" else 1, n, T, _dp(lp), _dp(old), _dp(w), 1 if per_seq else 0, _dp(m),
                         low, high, 0.0 if dual is None else float(dual), 0.0 if clamp is None else float(clamp),
                         _dp(loss), _dp(dloss), _dp(hit))
    return loss, dloss, hit


def reduce_tokens_backward(mask, shape, reduction, up=None, scale=1.0, local=None):
    S, B, T = shape
    m, u, loc = _d(mask), _d(up), _d(local)
    out = np.empty(S * B * T)
    lib().or_reduce_tokens_backward(_dp(m), S, B, T, REDUCTIONS[reduction], _dp(u), scale, _dp(loc), _dp(out))
    return out


def kl_estimate_grad(lp, lr, est, clamp=None, mask=None):
    lp, lr, m = _d(lp), _d(lr), _d(mask)
    out = np.empty_like(lp)
    lib().or_kl_estimate_grad(_dp(lp), _dp(lr), _dp(m), lp.size, est, 0.0 if clamp is None else float(clamp),
                              _dp(out))
    return out


def group_advantages(rewards, n, norm="mean", eps=0.0, unbiased=True):
    r = np.ascontiguousarray(rewards, dtype=np.float64).ravel()
    out = np.empty_like(r)
    rc = lib().or_group_advantages(_ptr(r, _c_double_p), r.size, n, 0 if norm == "mean" else 1,
                                   eps, 1 if unbiased else 0, _ptr(out, _c_double_p))
    if rc != 0:
        raise ValueError("group_advantages: invalid groups/eps/unbiased")
    return out


# ----------------------------------------------------------------------------- Cpu(Reference)

def cpuref_log_softmax_f64(x):
    x = np.ascontiguousarray(np.atleast_2d(x), dtype=np.float64)
    y = np.empty_like(x)
    lib().or_cpuref_log_softmax_f64(_ptr(x, _c_double_p), x.shape[0], x.shape[1], _ptr(y, _c_double_p))
    return y


def unrolled_sum(x):
    x = _f32(x)
    return lib().or_unrolled_sum_f32(_ptr(x, _c_float_p), x.size)


def matmul(a, b):
    """Tensor::matmul on Cpu(Reference) (float.rs:926-960, kernels.rs:415-450): a [..., m, k] and
    b [..., k, n] f32 of equal rank, batch dimensions broadcast where one side is 1; each batch
    is oracle.c `or_matmul_f32` (fmaf chains over k in order, closed every 256). Views are read
    through their strides."""
    a, b = np.asarray(a), np.asarray(b)
    assert a.dtype == np.float32 and b.dtype == np.float32 and a.ndim == b.ndim >= 2
    assert a.shape[-1] == b.shape[-2]
    batch = np.broadcast_shapes(a.shape[:-2], b.shape[:-2])
    m, k, n = a.shape[-2], a.shape[-1], b.shape[-1]
    ab = np.broadcast_to(a, batch + (m, k))
    bb = np.broadcast_to(b, batch + (k, n))
    out = np.empty(batch + (m, n), np.float32)
    L = lib()
    for z in np.ndindex(*batch):
        x, y = ab[z], bb[z]
        # the base of each view, with element strides (numpy strides are in bytes; a broadcast
        # batch has stride 0 and is already folded into the view's base)
        xs, ys = (s // 4 for s in x.strides), (s // 4 for s in y.strides)
        (ars, acs), (brs, bcs) = xs, ys
        xp = C.cast(x.__array_interface__["data"][0], _c_float_p)
        yp = C.cast(y.__array_interface__["data"][0], _c_float_p)
        L.or_matmul_f32(xp, ars, acs, yp, brs, bcs, m, k, n, _ptr(out[z], _c_float_p))
    return out


def cpuref_log_softmax(x):
    x = _f32(np.atleast_2d(x))
    y = np.empty_like(x)
    lib().or_cpuref_log_softmax(_ptr(x, _c_float_p), x.shape[0], x.shape[1], _ptr(y, _c_float_p))
    return y


def cpuref_sample_logp(x, tau, keep, rng: Rng):
    """The reference's Gumbel-max sample_categorical + token_log_probs on Cpu(Reference)."""
    x = _f32(np.atleast_2d(x))
    R, V = x.shape
    kp = None if keep is None else np.ascontiguousarray(np.atleast_2d(keep), dtype=np.uint8)
    ids = np.empty(R, dtype=np.int64)
    lp = np.empty(R, dtype=np.float32)
    rc = lib().or_cpuref_sample_logp(_ptr(x, _c_float_p), R, V, tau,
                                     None if kp is None else _ptr(kp, _c_u8_p),
                                     0 if kp is None or kp.shape[0] == 1 else V,
                                     C.byref(rng.s), _ptr(ids, _c_int64_p), _ptr(lp, _c_float_p))
    if rc:
        raise ValueError(f"sample_categorical: position {rc - 1} has no allowed token (every logit −∞ or a NaN)")
    return ids, lp


def cpufast_sample_logp(x, tau, keep, rng: Rng, threads):
    """sample_categorical + token_log_probs on the reference's Cpu(Fast) backend with `threads`
    workers (or_cpufast_sample_logp)."""
    x = _f32(np.atleast_2d(x))
    R, V = x.shape
    kp = None if keep is None else np.ascontiguousarray(np.atleast_2d(keep), dtype=np.uint8)
    ids = np.empty(R, dtype=np.int64)
    lp = np.empty(R, dtype=np.float32)
    rc = lib().or_cpufast_sample_logp(_ptr(x, _c_float_p), R, V, tau, None if kp is None else _ptr(kp, _c_u8_p),
                                      0 if kp is None or kp.shape[0] == 1 else V, C.byref(rng.s), threads,
                                      _ptr(ids, _c_int64_p), _ptr(lp, _c_float_p))
    if rc:
        raise ValueError(f"sample_categorical: position {rc - 1} has no allowed token (every logit −∞ or a NaN)")
    return ids, lp


def cpuref_sample_gumbel(x, tau, rng: Rng, addmask=None, keep=None):
    """The reference's sample_categorical (rl.rs:510-529) on Cpu(Reference): ids [R] of rows
    x [R, V] under an additive f32 mask [R or 1, V] or a u8 keep-mask; one u64 of `rng` per
    logit (none at tau 0 or when a row is refused)."""
    x = _f32(np.atleast_2d(x))
    R, V = x.shape
    am = None if addmask is None else _f32(np.atleast_2d(addmask))
    kp = None if keep is None else np.ascontiguousarray(np.atleast_2d(keep), dtype=np.uint8)
    ids = np.empty(R, dtype=np.int64)
    rc = lib().or_cpuref_sample_gumbel(_ptr(x, _c_float_p), R, V, tau,
                                       None if am is None else _ptr(am, _c_float_p),
                                       0 if am is None or am.shape[0] == 1 else V,
                                       None if kp is None else _ptr(kp, _c_u8_p),
                                       0 if kp is None or kp.shape[0] == 1 else V,
                                       C.byref(rng.s), _ptr(ids, _c_int64_p))
    if rc:
        raise ValueError(f"sample_categorical: position {rc - 1} has no allowed token (every logit −∞ or a NaN)")
    return ids


def cpu_sample_logp_invcdf(x, tau, keep, u, threads=1):
    x = _f32(np.atleast_2d(x))
    R, V = x.shape
    kp = None if keep is None else np.ascontiguousarray(np.atleast_2d(keep), dtype=np.uint8)
    u = np.ascontiguousarray(u, dtype=np.float64)
    ids = np.empty(R, dtype=np.int64)
    lp = np.empty(R, dtype=np.float32)
    rc = lib().or_cpu_sample_logp_invcdf(_ptr(x, _c_float_p), R, V, tau,
                                         None if kp is None else _ptr(kp, _c_u8_p),
                                         0 if kp is None or kp.shape[0] == 1 else V,
                                         _ptr(u, _c_double_p), _ptr(ids, _c_int64_p), _ptr(lp, _c_float_p), threads)
    if rc:
        raise ValueError(f"sample_categorical: position {rc - 1} has no allowed token (every logit −∞ or a NaN)")
    return ids, lp
