"""CPU restatement of the reference's general tensor ops, the checker of include/noetic_ops.h.

TEST INFRASTRUCTURE ONLY: tests/ import it as the checker; the product never does. Each function
cites the reference (shyble/noetic-tensor 0.7.0) code whose behaviour it restates.
"""
from decimal import Decimal, getcontext
from fractions import Fraction

import numpy as np

from oracle import oracle as O


def view(flat, shape, strides, offset=0):
    """The elements a Layout selects (src/tensor/layout.rs:8-12), as a numpy view."""
    flat = np.ascontiguousarray(flat).ravel()
    it = flat.itemsize
    return np.lib.stride_tricks.as_strided(flat[offset:], shape=tuple(shape), strides=tuple(s * it for s in strides),
                                           writeable=False)


def sum_dim(x, shape, dim):
    """`sum_dim` keeping the dimension (kernels.rs:153-174): along the last axis each lane is
    ndarray's eight-partial unrolled fold (oracle.c `or_unrolled_sum_f32`), along any other axis
    the slices are added in order from zero, in f32."""
    x = np.asarray(x, np.float32).reshape(shape)
    out_shape = list(shape)
    out_shape[dim] = 1
    if dim == len(shape) - 1:
        rows = x.reshape(-1, shape[-1])
        return np.array([O.unrolled_sum(r) for r in rows], np.float32).reshape(out_shape)
    outer, n, inner = int(np.prod(shape[:dim])), shape[dim], int(np.prod(shape[dim + 1:]))
    x3 = x.reshape(outer, n, inner)
    acc = np.zeros((outer, inner), np.float32)
    for k in range(n):
        acc = acc + x3[:, k, :]
    return acc.reshape(out_shape)


def argmax_dim(x, shape, dim):
    """`argmax_dim` (kernels.rs:184-209): the first NaN of a lane, else its first maximum."""
    x = np.asarray(x, np.float32).reshape(shape)
    outer, n, inner = int(np.prod(shape[:dim])), shape[dim], int(np.prod(shape[dim + 1:]))
    x3 = x.reshape(outer, n, inner)
    idx = np.zeros((outer, inner), np.int64)
    for o in range(outer):
        for i in range(inner):
            lane = x3[o, :, i]
            nan = np.nonzero(np.isnan(lane))[0]
            idx[o, i] = nan[0] if nan.size else int(np.argmax(lane))  # np.argmax: the first maximum
    out_shape = list(shape)
    out_shape[dim] = 1
    vals = np.take_along_axis(x3, idx[:, None, :], axis=1)
    return idx.reshape(out_shape), vals.reshape(out_shape)


def max_all(x):
    """CpuRef's max over every element, NaN-propagating (the first NaN's payload)."""
    x = np.asarray(x, np.float32).ravel()
    nan = np.nonzero(np.isnan(x))[0]
    return x[nan[0]] if nan.size else x.max()


def f16_from_f32(x):
    """F16::from_f32 (half.rs:30-60): round to nearest even, subnormals, overflow to inf, NaN kept
    quiet with its top payload bits. Written from the binary16 format; pinned against numpy's
    float16 conversion for every non-NaN input."""
    b = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    sign = ((b >> 16) & 0x8000).astype(np.uint64)
    ex = ((b >> 23) & 0xFF).astype(np.int64)
    man = (b & 0x7FFFFF).astype(np.uint64)
    out = np.zeros(b.shape, np.uint64)
    for k in np.ndindex(b.shape):
        s, e8, m = int(sign[k]), int(ex[k]), int(man[k])
        if e8 == 0xFF:
            out[k] = s | 0x7C00 | ((0x0200 | (m >> 13)) if m else 0)
            continue
        e = e8 - 127 + 15
        if e >= 0x1F:
            out[k] = s | 0x7C00
            continue
        if e <= 0:
            if e < -10:
                out[k] = s
                continue
            full = m | 0x800000
            sh = 14 - e
            q, rem, half = full >> sh, full & ((1 << sh) - 1), 1 << (sh - 1)
        else:
            q, rem, half = (e << 10) | (m >> 13), m & 0x1FFF, 0x1000
        q += 1 if (rem > half or (rem == half and q & 1)) else 0
        out[k] = s | q
    return out.astype(np.uint16)


def f16_to_f32(h):
    """F16::to_f32 (half.rs:62-90): exact (a NaN keeps its payload in the top mantissa bits)."""
    h = np.asarray(h, np.uint16).astype(np.uint32)
    sign = (h & 0x8000) << 16
    e = (h >> 10) & 0x1F
    m = h & 0x3FF
    normal = (sign | ((e + 112) << 23) | (m << 13)).view(np.float32)
    special = (sign | 0x7F800000 | (m << 13)).view(np.float32)
    sub = (m.astype(np.float32) * np.float32(2.0 ** -24)) * np.where(sign != 0, -1, 1).astype(np.float32)
    return np.where(e == 0x1F, special, np.where(e == 0, sub, normal)).astype(np.float32)


def _nearest_f32(q: Fraction) -> np.float32:
    """The f32 nearest to the exact rational q (ties to even), by exact arithmetic."""
    if q == 0:
        return np.float32(0.0)
    neg = q < 0
    a = -q if neg else q
    # the binade: 2^e <= a < 2^(e+1)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    if e > 127:
        return np.float32(-np.inf if neg else np.inf)
    lsb = max(e - 23, -149)
    scaled = a / (Fraction(2) ** lsb)
    n = scaled.numerator // scaled.denominator
    rem = scaled - n
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and n % 2 == 1):
        n += 1
    v = float(Fraction(n) * Fraction(2) ** lsb)  # exact in f64; 2^128 (a carry out of the top) is inf in f32
    with np.errstate(over="ignore"):
        r = np.float32(v)
    return -r if neg else r


def correctly_rounded(fn: str, x: float, s: float = 0.0) -> np.float32:
    """exp, ln or pow of f32 inputs to 60 significant digits (decimal's exp, ln and power are
    correctly rounded at the context precision), then rounded once to the nearest f32: the value
    an exact implementation returns. Special inputs (NaN, infinities, zero, negative) are left to
    the caller."""
    getcontext().prec = 60
    d = Decimal(float(x))
    if fn == "exp":
        r = d.exp()
    elif fn == "log":
        r = d.ln()
    else:
        r = d ** Decimal(float(s))
    return _nearest_f32(Fraction(r))


def sort_order_key(x):
    """CpuRef's sort_order (kernels.rs:374-388) as an unsigned key per element: every NaN
    (whatever its sign and payload) one key above +inf, otherwise total_cmp's order, -0 below +0."""
    b = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    k = np.where(b & 0x80000000, (~b) & 0xFFFFFFFF, b | 0x80000000)
    return np.where(np.isnan(np.asarray(x, np.float32)), np.uint64(0xFFFFFFFF), k).astype(np.uint64)


def sort_desc(x, shape, dim):
    """sort_desc_with_indices (kernels.rs:390-413): per lane a stable descending sort in
    sort_order; the values (the source elements, NaN payloads kept) and their int64 positions."""
    x = np.asarray(x, np.float32).reshape(shape)
    keys = sort_order_key(x).astype(np.int64)
    order = np.argsort(-keys, axis=dim, kind="stable")  # ascending -key = descending key, ties by position
    return np.take_along_axis(x, order, axis=dim), order.astype(np.int64)
