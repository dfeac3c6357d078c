"""Host mirror of the reference's general GPU ops (the `GpuBackend` trait, src/tensor/gpu/mod.rs:137-207)
for a `Device::Hip(0)` tensor, over libnoetic_hip.so's include/noetic_ops.h entry points.

These are the ops the nn::rl chain runs around the fused entry points: `tempered_logits`' divide
and mask add, casts of bf16 logits, comparisons and `mask_fill` for clamps and masks, lane
reductions, `gather` and its scatter. Each function keeps the trait method's name and argument
meaning (a `Layout` is a view read in place; outputs are fresh, contiguous and row-major), and
`Layout` keeps src/tensor/layout.rs's view operations. There is no CPU fallback: without the built
library every call raises `HipUnavailable`, as in `noetic_rl`.

`matmul` is the reference's f32 product bit for bit (a VALU kernel: the reference's order of fma
chains rules out the matrix cores), `matmul_half` its reduced-precision product on the matrix cores
(bf16 operands, f32 accumulation), and `sort_desc` CpuRef's stable descending order on the device
for every lane length.
"""
from __future__ import annotations

import ctypes as C
import enum
from typing import List, Optional, Sequence, Tuple

import numpy as np

import noetic_rl as nr
from noetic_rl import (MatmulPrecision, NtLayout, Tensor, _check, _dev, matmul_precision, matmul_precision_scope,
                       same_dtype, set_matmul_precision)

MAX_RANK = 8
_DT = {"f32": 0, "bf16": 1, "f16": 2, "bool": 3, "u8": 4, "i32": 5, "i64": 6}


class Unsupported(NotImplementedError):
    """TensorError::Unsupported: a valid request this backend does not implement."""


class UnaryOp(enum.IntEnum):
    """gpu/mod.rs:68-103 (`UnaryOp::code`)."""
    NEG = 0
    EXP = 1
    LOG = 2
    SQRT = 3
    RECIP = 4
    ABS = 5
    SIGN = 6
    SIGMOID = 7
    ADD_SCALAR = 8
    SUB_SCALAR = 9
    MUL_SCALAR = 10
    DIV_SCALAR = 11
    POW_SCALAR = 12


class CmpOp(enum.IntEnum):
    """gpu/mod.rs:107-114."""
    GT = 0
    GE = 1
    LT = 2
    LE = 3
    EQ = 4


class BinaryOp(enum.IntEnum):
    """gpu/mod.rs:116-122."""
    ADD = 0
    SUB = 1
    MUL = 2
    DIV = 3


class ReduceOp(enum.IntEnum):
    """gpu/mod.rs:124-133."""
    SUM = 0
    MAX = 1
    ARGMAX = 2


def _row_major(shape: Sequence[int]) -> List[int]:
    st, s = [0] * len(shape), 1
    for d in range(len(shape) - 1, -1, -1):
        st[d] = s
        s *= shape[d]
    return st


class Layout:
    """src/tensor/layout.rs:8-81: shape, element strides and element offset of a view."""

    def __init__(self, shape: Sequence[int], strides: Optional[Sequence[int]] = None, offset: int = 0):
        self.shape = [int(d) for d in shape]
        self.strides = [int(s) for s in (strides if strides is not None else _row_major(self.shape))]
        self.offset = int(offset)
        if len(self.shape) > MAX_RANK:
            raise ValueError(f"rank {len(self.shape)} (at most {MAX_RANK} on the device)")

    @staticmethod
    def contiguous(shape: Sequence[int]) -> "Layout":
        return Layout(shape)

    def numel(self) -> int:
        return int(np.prod(self.shape)) if self.shape else 1

    def is_contiguous(self) -> bool:
        return self.strides == _row_major(self.shape)

    def reshaped(self, shape: Sequence[int]) -> Optional["Layout"]:
        return Layout(shape, None, self.offset) if self.is_contiguous() else None

    def swapped(self, a: int, b: int) -> "Layout":
        sh, st = list(self.shape), list(self.strides)
        sh[a], sh[b] = sh[b], sh[a]
        st[a], st[b] = st[b], st[a]
        return Layout(sh, st, self.offset)

    def narrowed(self, ranges: Sequence[range]) -> "Layout":
        off = self.offset + sum(r.start * s for r, s in zip(ranges, self.strides))
        return Layout([r.stop - r.start for r in ranges], self.strides, off)

    def broadcast(self, out: Sequence[int]) -> "Layout":
        """Right-aligned, stride 0 on every expanded dimension (layout.rs:71-80)."""
        ni, no = len(self.shape), len(out)
        st = [0] * no
        for i in range(ni):
            o = no - ni + i
            st[o] = self.strides[i] if self.shape[i] == out[o] else 0
        return Layout(out, st, self.offset)

    def c(self) -> NtLayout:
        lay = NtLayout()
        lay.rank = len(self.shape)
        lay.offset = self.offset
        for d, (n, s) in enumerate(zip(self.shape, self.strides)):
            lay.shape[d] = n
            lay.strides[d] = s
        return lay


def broadcast_shape(a: Sequence[int], b: Sequence[int]) -> List[int]:
    """shape::broadcast: right-aligned, each pair equal or one of them 1."""
    n = max(len(a), len(b))
    a, b = [1] * (n - len(a)) + list(a), [1] * (n - len(b)) + list(b)
    out = []
    for x, y in zip(a, b):
        if x != y and 1 not in (x, y):
            raise ValueError(f"shapes {a} and {b} do not broadcast")
        out.append(max(x, y))
    return out


def _esize(dtype: str) -> int:
    return np.dtype(nr._NP[dtype]).itemsize


def _f32(x: Tensor, what: str):
    if x.dtype != "f32":
        raise TypeError(f"{what}: {x.dtype} storage in a float kernel (cast to f32 first)")


def _inside(t: Tensor, l: Layout, what: str):
    """The device reads a view in place with no bounds of its own: every element the view selects
    must lie in the tensor's buffer (the reference's Layout guarantees this by construction)."""
    if l.numel() == 0:
        return
    last = l.offset + sum((n - 1) * s for n, s in zip(l.shape, l.strides))
    if l.offset < 0 or min(l.strides, default=0) < 0 or last >= t.numel:
        raise IndexError(f"{what}: the view {l.shape} strides {l.strides} offset {l.offset} leaves the buffer "
                         f"of {t.numel} elements")


# ----------------------------------------------------------------------------------- trait methods

def alloc(dtype: str, shape: Sequence[int]) -> Tensor:
    """GpuBackend::alloc: uninitialised storage."""
    return Tensor(shape, dtype)


def copy(x: Tensor, xl: Layout) -> Tensor:
    """GpuBackend::copy: the elements the view selects, contiguous (any dtype)."""
    _inside(x, xl, "copy")
    y = Tensor(xl.shape, x.dtype)
    _check(_dev().nt_hip_copy(C.c_void_p(x.ptr), C.byref(xl.c()), _esize(x.dtype), C.c_void_p(y.ptr)), "copy")
    return y


def write(dst: Tensor, dl: Layout, src: Tensor, sl: Layout) -> None:
    """GpuBackend::write: the view sl of src into the view dl of dst (slice_assign, cat)."""
    if dst.dtype != src.dtype or dl.shape != sl.shape:
        raise ValueError(f"write of {src.dtype} {sl.shape} into {dst.dtype} {dl.shape}")
    _inside(dst, dl, "write")
    _inside(src, sl, "write")
    _check(_dev().nt_hip_write(C.c_void_p(dst.ptr), C.byref(dl.c()), C.c_void_p(src.ptr), C.byref(sl.c()),
                               _esize(src.dtype)), "write")


def cast(x: Tensor, xl: Layout, to: str) -> Tensor:
    """GpuBackend::cast: f16/bf16/bool -> f32, f32 -> f16/bf16 (RNE), f16 <-> bf16, same = copy."""
    if to not in ("f32", "f16", "bf16") and to != x.dtype:
        raise Unsupported(f"cast {x.dtype} → {to}")
    _inside(x, xl, "cast")
    y = Tensor(xl.shape, to)
    _check(_dev().nt_hip_cast(C.c_void_p(x.ptr), C.byref(xl.c()), _DT[x.dtype], _DT[to], C.c_void_p(y.ptr)), "cast")
    return y


def unary(op: UnaryOp, x: Tensor, xl: Layout, s: float = 0.0) -> Tensor:
    """GpuBackend::unary (f32): the op with its scalar (AddScalar .. PowScalar)."""
    _f32(x, "unary")
    _inside(x, xl, "unary")
    y = Tensor(xl.shape, "f32")
    _check(_dev().nt_hip_unary(int(op), s, C.c_void_p(x.ptr), C.byref(xl.c()), C.c_void_p(y.ptr)), "unary")
    return y


def compare(op: CmpOp, x: Tensor, xl: Layout, s: float) -> Tensor:
    """GpuBackend::compare: bool storage of x op s."""
    _f32(x, "compare")
    _inside(x, xl, "compare")
    y = Tensor(xl.shape, "bool")
    _check(_dev().nt_hip_compare(int(op), s, C.c_void_p(x.ptr), C.byref(xl.c()), C.c_void_p(y.ptr)), "compare")
    return y


def binary(op: BinaryOp, a: Tensor, al: Layout, b: Tensor, bl: Layout) -> Tensor:
    """GpuBackend::binary over the broadcast shape (al and bl already broadcast to it)."""
    _f32(a, "binary")
    _f32(b, "binary")
    _inside(a, al, "binary")
    _inside(b, bl, "binary")
    y = Tensor(al.shape, "f32")
    _check(_dev().nt_hip_binary(int(op), C.c_void_p(a.ptr), C.byref(al.c()), C.c_void_p(b.ptr), C.byref(bl.c()),
                                C.c_void_p(y.ptr)), "binary")
    return y


def mask_fill(x: Tensor, xl: Layout, mask: Tensor, ml: Layout, value: float) -> Tensor:
    """GpuBackend::mask_fill: value where the (bool) mask, broadcast by its layout, is true."""
    _f32(x, "mask_fill")
    if mask.dtype != "bool":
        raise TypeError(f"a mask of {mask.dtype} storage")
    _inside(x, xl, "mask_fill")
    _inside(mask, ml, "mask_fill")
    y = Tensor(xl.shape, "f32")
    _check(_dev().nt_hip_mask_fill(C.c_void_p(x.ptr), C.byref(xl.c()), C.c_void_p(mask.ptr), C.byref(ml.c()), value,
                                   C.c_void_p(y.ptr)), "mask_fill")
    return y


def reduce_dim(op: ReduceOp, x: Tensor, shape: Sequence[int], dim: int) -> Tensor:
    """GpuBackend::reduce_dim along `dim` of contiguous f32 x (the dimension kept, size 1): f32 values
    for Sum and Max, I32 indices for ArgMax."""
    _f32(x, "reduce_dim")
    shape = list(shape)
    outer, n, inner = int(np.prod(shape[:dim])), shape[dim], int(np.prod(shape[dim + 1:]))
    out_shape = shape[:dim] + [1] + shape[dim + 1:]
    if outer * n * inner != x.numel:
        raise ValueError(f"reduce_dim: shape {shape} against {x.numel} elements")
    y = Tensor(out_shape, "i32" if op == ReduceOp.ARGMAX else "f32")
    _check(_dev().nt_hip_reduce_dim(int(op), C.c_void_p(x.ptr), outer, n, inner, int(dim + 1 == len(shape)),
                                    C.c_void_p(y.ptr)), "reduce_dim")
    return y


def reduce_all(op: ReduceOp, x: Tensor, n: int) -> Tensor:
    """GpuBackend::reduce_all: Sum or Max of every element, one f32."""
    _f32(x, "reduce_all")
    if n > x.numel:
        raise ValueError(f"reduce_all: {n} elements of {x.numel}")
    y = Tensor((1,), "f32")
    _check(_dev().nt_hip_reduce_all(int(op), C.c_void_p(x.ptr), n, C.c_void_p(y.ptr)), "reduce_all")
    return y


def _lanes_fit(x: Optional[Tensor], nx: int, idx: Tensor, ni: int, what: str):
    if x is not None and (x.dtype != "f32" or x.numel < nx):
        raise ValueError(f"{what}: f32 storage of at least {nx} elements")
    if idx.dtype != "i32" or idx.numel < ni:
        raise ValueError(f"{what}: I32 indices of at least {ni} elements")


def gather(x: Tensor, lanes: Sequence[int], idx: Tensor) -> Tensor:
    """GpuBackend::gather of contiguous x [outer, n, inner] at I32 indices [outer, m, inner]."""
    outer, n, inner, m = (int(v) for v in lanes)
    _lanes_fit(x, outer * n * inner, idx, outer * m * inner, "gather")
    y = Tensor((outer, m, inner), "f32")
    _check(_dev().nt_hip_gather(C.c_void_p(x.ptr), outer, n, inner, C.c_void_p(idx.ptr), m, C.c_void_p(y.ptr)),
           "gather")
    return y


def index_select(x: Tensor, lanes: Sequence[int], idx: Tensor) -> Tensor:
    """GpuBackend::index_select of contiguous x [outer, n, inner] at m I32 indices."""
    outer, n, inner, m = (int(v) for v in lanes)
    _lanes_fit(x, outer * n * inner, idx, m, "index_select")
    y = Tensor((outer, m, inner), "f32")
    _check(_dev().nt_hip_index_select(C.c_void_p(x.ptr), outer, n, inner, C.c_void_p(idx.ptr), m,
                                      C.c_void_p(y.ptr)), "index_select")
    return y


def one_hot(idx: Tensor, count: int, n: int) -> Tensor:
    """GpuBackend::one_hot: f32 rows of width n for count I32 indices."""
    _lanes_fit(None, 0, idx, count, "one_hot")
    y = Tensor((count, n), "f32")
    _check(_dev().nt_hip_one_hot(C.c_void_p(idx.ptr), count, n, C.c_void_p(y.ptr)), "one_hot")
    return y


def scatter_add(idx: Tensor, vals: Tensor, lanes: Sequence[int]) -> Tensor:
    """GpuBackend::scatter_add of values [outer, m, inner] into zeros [outer, n, inner]."""
    outer, n, inner, m = (int(v) for v in lanes)
    _lanes_fit(vals, outer * m * inner, idx, outer * m * inner, "scatter_add")
    y = Tensor((outer, n, inner), "f32")
    _check(_dev().nt_hip_scatter_add(C.c_void_p(idx.ptr), C.c_void_p(vals.ptr), outer, n, inner, m,
                                     C.c_void_p(y.ptr)), "scatter_add")
    return y


def index_add(idx: Tensor, vals: Tensor, lanes: Sequence[int]) -> Tensor:
    """GpuBackend::index_add of value slices [outer, m, inner] into zeros [outer, n, inner]."""
    outer, n, inner, m = (int(v) for v in lanes)
    _lanes_fit(vals, outer * m * inner, idx, m, "index_add")
    y = Tensor((outer, n, inner), "f32")
    _check(_dev().nt_hip_index_add(C.c_void_p(idx.ptr), C.c_void_p(vals.ptr), outer, n, inner, m,
                                   C.c_void_p(y.ptr)), "index_add")
    return y


def fill(shape: Sequence[int], value: float) -> Tensor:
    """GpuBackend::fill: f32 elements equal to value, written on the device."""
    y = Tensor(shape, "f32")
    _check(_dev().nt_hip_fill(C.c_void_p(y.ptr), y.numel, value), "fill")
    return y


def sort_desc(x: Tensor, lanes: Sequence[int]) -> Tuple[Tensor, Tensor]:
    """GpuBackend::sort_desc: along the middle of contiguous f32 x [outer, n, inner], descending in
    CpuRef's order (NaN first, total_cmp, stable); the values and their I32 positions."""
    outer, n, inner = (int(v) for v in lanes)
    if x.dtype != "f32" or outer * n * inner > x.numel:
        raise ValueError(f"sort_desc of {x.dtype} storage of {x.numel} elements as {[outer, n, inner]}")
    vals, idx = Tensor((outer, n, inner), "f32"), Tensor((outer, n, inner), "i32")
    _check(_dev().nt_hip_sort_desc(C.c_void_p(x.ptr), outer, n, inner, C.c_void_p(vals.ptr), C.c_void_p(idx.ptr)),
           "sort_desc")
    return vals, idx


def matmul(a: Tensor, al: Layout, b: Tensor, bl: Layout,
           precision: MatmulPrecision = MatmulPrecision.F32) -> Tuple[Tensor, List[int]]:
    """GpuBackend::matmul (or matmul_half with MatmulPrecision.HALF): the batched product of two f32
    views (batch dimensions broadcast when 1) and the output shape; at F32 CpuRef's arithmetic bit
    for bit (nt_hip_matmul), at HALF bf16 operands with f32 accumulation (nt_hip_matmul_half)."""
    if a.dtype != "f32" or b.dtype != "f32":
        raise ValueError(f"matmul of {a.dtype} and {b.dtype} storage (f32 operands only)")
    ash, bsh = list(al.shape), list(bl.shape)
    r = len(ash)
    if r < 2 or len(bsh) != r or ash[r - 1] != bsh[r - 2]:
        raise ValueError(f"matmul {ash} × {bsh}")
    batch = list(broadcast_shape(ash[:-2], bsh[:-2]))
    _inside(a, al, "matmul")
    _inside(b, bl, "matmul")
    shape = batch + [ash[r - 2], bsh[r - 1]]
    y = Tensor(shape, "f32")
    fn = _dev().nt_hip_matmul_half if precision == MatmulPrecision.HALF else _dev().nt_hip_matmul
    _check(fn(C.c_void_p(a.ptr), C.byref(al.c()), C.c_void_p(b.ptr), C.byref(bl.c()), C.c_void_p(y.ptr)), "matmul")
    return y, shape


def half_gemm_key() -> str:
    """GpuBackend::half_gemm_key: the reduced-precision product's key part."""
    buf = C.create_string_buffer(256)
    _check(_dev().nt_hip_half_gemm_key(buf, 256), "half_gemm_key")
    return buf.value.decode()


# ----------------------------------------------------------------------------------- tensor level

def tempered_logits(logits: Tensor, temperature: float, mask: Optional[Tensor] = None) -> Tensor:
    """`tempered_logits` (rl.rs:475-486) materialised on the device with the general ops:
    `div_scalar(τ)` unless τ == 1 (16-bit logits come out f32), then `add(mask)` broadcast at rank
    under add's same_dtype check (an f32 mask on f32 or divided logits; at τ == 1 a 16-bit mask
    of the logits' own dtype, the sum computed in f32 into f32 storage; other pairs are refused
    there, as the reference's add refuses them). The fused entry points take the tempered logits without materialising them;
    this is the op sequence a caller gets when it asks for the tensor itself."""
    if not (temperature > 0.0 and np.isfinite(temperature)):
        raise ValueError(f"tempered_logits: temperature {temperature} (must be positive)")
    if temperature == 1.0 and mask is None:
        return logits  # rl.rs:476: no divide, no add
    lay = Layout.contiguous(logits.shape)
    z = logits
    if temperature != 1.0:  # div_scalar computes 16-bit logits in f32 (f32_operand)
        z = cast(logits, lay, "f32") if logits.dtype != "f32" else logits
        z = unary(UnaryOp.DIV_SCALAR, z, lay, float(np.float32(temperature)))
    if mask is not None:
        if len(mask.shape) != len(logits.shape):
            raise ValueError("tempered_logits: mask rank")
        if not all(a == b or a == 1 for a, b in zip(mask.shape, logits.shape)):
            raise ValueError(f"tempered_logits: mask {list(mask.shape)} does not broadcast to the logits "
                             f"{list(logits.shape)}")
        # add's same_dtype check on the reference's z: 16-bit logits are not divided at τ == 1
        same_dtype(logits.dtype if temperature == 1.0 else "f32", mask.dtype, "add")
        if mask.dtype not in ("f32", "bf16", "f16"):
            raise TypeError("tempered_logits: an additive float mask")
        # the sum computes 16-bit operands in f32 into f32 storage (f32_operand, gpu/mod.rs:336-342)
        m = cast(mask, Layout.contiguous(mask.shape), "f32") if mask.dtype != "f32" else mask
        if z.dtype != "f32":
            z = cast(z, lay, "f32")
        out = broadcast_shape(logits.shape, mask.shape)
        z = binary(BinaryOp.ADD, z, lay.broadcast(out), m, Layout.contiguous(mask.shape).broadcast(out))
    return z


# ----------------------------------------------------------------------------------- dispatch

class DTensor:
    """A tensor on the device: storage and the Layout it is read through. The methods are the
    reference's tensor-level dispatch onto the trait (src/tensor/gpu/mod.rs:327-700, the `gpu_*`
    functions) for the ops the rl chain uses: 16-bit operands are cast to f32 first
    (`f32_operand`), reductions and indexing read a contiguous f32 copy (`f32_contiguous`), binary
    ops broadcast both layouts to the output shape, and views (swap_dims, slice, expand, reshape of
    a row-major layout) are new layouts over the same storage (layout.rs)."""

    def __init__(self, storage: Tensor, layout: Optional[Layout] = None):
        self.storage = storage
        self.layout = layout if layout is not None else Layout.contiguous(storage.shape)
        self.dtype = storage.dtype

    @staticmethod
    def from_numpy(a, dtype: Optional[str] = None) -> "DTensor":
        return DTensor(Tensor.from_numpy(np.ascontiguousarray(a), dtype))

    @property
    def shape(self) -> List[int]:
        return list(self.layout.shape)

    def numel(self) -> int:
        return self.layout.numel()

    def contiguous(self) -> "DTensor":
        """gpu_copy: the view's elements, row-major (the same storage when already so)."""
        l = self.layout
        if l.is_contiguous() and l.offset == 0 and self.storage.numel == l.numel():
            return self
        return DTensor(copy(self.storage, l))

    def to_numpy(self) -> np.ndarray:
        return self.contiguous().storage.to_numpy().reshape(self.shape)

    # -- views (layout.rs)
    def swap_dims(self, a: int, b: int) -> "DTensor":
        return DTensor(self.storage, self.layout.swapped(a, b))

    def slice(self, ranges: Sequence[range]) -> "DTensor":
        return DTensor(self.storage, self.layout.narrowed(ranges))

    def expand(self, shape: Sequence[int]) -> "DTensor":
        return DTensor(self.storage, self.layout.broadcast(shape))

    def unsqueeze(self, d: int) -> "DTensor":
        sh, st = list(self.layout.shape), list(self.layout.strides)
        sh.insert(d, 1)
        st.insert(d, st[d] * sh[d + 1] if d < len(st) else 1)
        return DTensor(self.storage, Layout(sh, st, self.layout.offset))

    def reshape(self, shape: Sequence[int]) -> "DTensor":
        c = self.contiguous()
        return DTensor(c.storage, c.layout.reshaped(shape))

    # -- operands
    def _f32(self) -> "DTensor":
        """f32_operand (gpu/mod.rs:336-342): f16 and bf16 are cast to f32 first."""
        if self.dtype == "f32":
            return self
        if self.dtype in ("f16", "bf16"):
            return DTensor(cast(self.storage, self.layout, "f32"))
        raise TypeError(f"{self.dtype} storage in a float GPU kernel")

    def _f32_contiguous(self) -> "DTensor":
        return self._f32().contiguous()

    # -- products
    def matmul(self, rhs: "DTensor") -> "DTensor":
        """Tensor::matmul on the device (float.rs:924-930 -> gpu_matmul, gpu/mod.rs:458-470) at the
        calling thread's precision (`set_matmul_precision`): both operands as f32 views (16-bit
        ones cast first), batch dimensions broadcast."""
        return self.matmul_with(rhs, matmul_precision())

    def matmul_with(self, rhs: "DTensor", precision: MatmulPrecision) -> "DTensor":
        """Tensor::matmul_with (float.rs:934-944): the product at a named precision."""
        if self.dtype != rhs.dtype:
            raise TypeError(f"matmul of {self.dtype} and {rhs.dtype}")
        x, y = self._f32(), rhs._f32()
        st, shape = matmul(x.storage, x.layout, y.storage, y.layout, precision)
        return DTensor(st, Layout.contiguous(shape))

    # -- elementwise
    def unary(self, op: UnaryOp, s: float = 0.0) -> "DTensor":
        x = self._f32()
        return DTensor(unary(op, x.storage, x.layout, float(np.float32(s))))

    def neg(self):
        return self.unary(UnaryOp.NEG)

    def exp(self):
        return self.unary(UnaryOp.EXP)

    def log(self):
        return self.unary(UnaryOp.LOG)

    def sqrt(self):
        return self.unary(UnaryOp.SQRT)

    def recip(self):
        return self.unary(UnaryOp.RECIP)

    def abs(self):
        return self.unary(UnaryOp.ABS)

    def sign(self):
        return self.unary(UnaryOp.SIGN)

    def sigmoid(self):
        return self.unary(UnaryOp.SIGMOID)

    def add_scalar(self, s):
        return self.unary(UnaryOp.ADD_SCALAR, s)

    def sub_scalar(self, s):
        return self.unary(UnaryOp.SUB_SCALAR, s)

    def mul_scalar(self, s):
        return self.unary(UnaryOp.MUL_SCALAR, s)

    def div_scalar(self, s):
        return self.unary(UnaryOp.DIV_SCALAR, s)

    def powf_scalar(self, p: float) -> "DTensor":
        """float.rs:543-570: an integer exponent goes through powi (0 ones, 1 itself, 2 x·x, −1 recip,
        −2 recip(x·x)), any other through PowScalar(p as f32)."""
        if float(p).is_integer():
            k = int(p)
            if k == 0:
                return DTensor(fill(self.shape, 1.0))
            if k == 1:
                return self
            if k == 2:
                return self.mul(self)
            if k == -1:
                return self.recip()
            if k == -2:
                return self.mul(self).recip()
        return self.unary(UnaryOp.POW_SCALAR, p)

    def _binary(self, op: BinaryOp, other: "DTensor") -> "DTensor":
        """float.rs:398-460: shapes broadcast, then one dtype (same_dtype, infer.rs:157-158: a bf16
        tensor and an f32 one are refused, casts are explicit), then the f32 kernel."""
        out = broadcast_shape(self.shape, other.shape)
        same_dtype(self.dtype, other.dtype, op.name.lower())
        a, b = self._f32(), other._f32()
        return DTensor(binary(op, a.storage, a.layout.broadcast(out), b.storage, b.layout.broadcast(out)))

    def add(self, o):
        return self._binary(BinaryOp.ADD, o)

    def sub(self, o):
        return self._binary(BinaryOp.SUB, o)

    def mul(self, o):
        return self._binary(BinaryOp.MUL, o)

    def div(self, o):
        return self._binary(BinaryOp.DIV, o)

    def compare(self, op: CmpOp, s: float) -> "DTensor":
        x = self._f32()
        return DTensor(compare(op, x.storage, x.layout, float(np.float32(s))))

    def greater_elem(self, s):
        return self.compare(CmpOp.GT, s)

    def lower_elem(self, s):
        return self.compare(CmpOp.LT, s)

    def mask_fill(self, mask: "DTensor", value: float) -> "DTensor":
        x = self._f32()
        return DTensor(mask_fill(x.storage, x.layout, mask.storage, mask.layout.broadcast(self.shape),
                                 float(np.float32(value))))

    def clamp(self, lo: float, hi: float) -> "DTensor":
        """float.rs:576-595: clamp_min(clamp_max(x, hi), lo), each a mask_fill of a comparison."""
        x = self.mask_fill(self.greater_elem(hi), hi)
        return x.mask_fill(x.lower_elem(lo), lo)

    # -- reductions
    def sum(self) -> "DTensor":
        x = self._f32_contiguous()
        return DTensor(reduce_all(ReduceOp.SUM, x.storage, x.numel()))

    def mean(self) -> "DTensor":
        return self.sum().div_scalar(float(self.numel()))

    def max(self) -> "DTensor":
        x = self._f32_contiguous()
        return DTensor(reduce_all(ReduceOp.MAX, x.storage, x.numel()))

    def sum_dim(self, d: int) -> "DTensor":
        x = self._f32_contiguous()
        return DTensor(reduce_dim(ReduceOp.SUM, x.storage, self.shape, d))

    def mean_dim(self, d: int) -> "DTensor":
        return self.sum_dim(d).div_scalar(float(self.shape[d]))

    def max_dim(self, d: int) -> "DTensor":
        x = self._f32_contiguous()
        return DTensor(reduce_dim(ReduceOp.MAX, x.storage, self.shape, d))

    def argmax(self, d: int) -> np.ndarray:
        """gpu_argmax: I32 device indices read back as host i64 (int tensors live on the host)."""
        x = self._f32_contiguous()
        return reduce_dim(ReduceOp.ARGMAX, x.storage, self.shape, d).to_numpy().astype(np.int64)

    # -- indexing and casts
    def gather(self, d: int, idx: np.ndarray) -> "DTensor":
        x = self._f32_contiguous()
        sh = self.shape
        outer, n, inner = int(np.prod(sh[:d])), sh[d], int(np.prod(sh[d + 1:]))
        m = idx.shape[d]
        i = Tensor.from_numpy(np.ascontiguousarray(idx, np.int64).astype(np.int32))
        y = gather(x.storage, (outer, n, inner, m), i)
        return DTensor(y, Layout.contiguous(list(idx.shape)))

    def select(self, d: int, indices: Sequence[int]) -> "DTensor":
        x = self._f32_contiguous()
        sh = self.shape
        outer, n, inner = int(np.prod(sh[:d])), sh[d], int(np.prod(sh[d + 1:]))
        i = Tensor.from_numpy(np.asarray(indices, np.int32))
        y = index_select(x.storage, (outer, n, inner, len(indices)), i)
        out = list(sh)
        out[d] = len(indices)
        return DTensor(y, Layout.contiguous(out))

    def sort_descending_with_indices(self, d: int) -> Tuple["DTensor", np.ndarray]:
        """Tensor::sort_descending_with_indices on the device (float.rs:1032-1040 ->
        gpu_sort_desc, gpu/mod.rs:549-561): rank >= 2, a contiguous f32 copy sorted along d; the
        values and the positions (read back here as int64, as IntTensor::to_vec does)."""
        if len(self.shape) < 2:
            raise ValueError("sort needs rank 2 or more")
        x = self._f32_contiguous()
        sh = self.shape
        lanes = (int(np.prod(sh[:d])), sh[d], int(np.prod(sh[d + 1:])))
        vals, idx = sort_desc(x.storage, lanes)
        return DTensor(vals, Layout.contiguous(sh)), idx.to_numpy().reshape(sh).astype(np.int64)

    def topk_with_indices(self, k: int, d: int) -> Tuple["DTensor", np.ndarray]:
        """Tensor::topk_with_indices (float.rs:1070-1080): the first k of the descending sort
        along d."""
        v, i = self.sort_descending_with_indices(d)
        r = [range(0, s) for s in self.shape]
        r[d] = range(0, k)
        return DTensor(v.storage, v.layout.narrowed(r)).contiguous(), i[tuple(slice(q.start, q.stop) for q in r)]

    def cast(self, to: str) -> "DTensor":
        """gpu_cast: 16-bit through f32 (f32_operand), f32 to 16-bit by the cast kernel."""
        if to == "f32":
            return self._f32().contiguous()
        x = self._f32()
        return DTensor(cast(x.storage, x.layout, to))

    def float(self) -> "DTensor":
        """A bool tensor as f32 1.0 / 0.0 (gpu_bool_float)."""
        return DTensor(cast(self.storage, self.layout, "f32"))

    def slice_assign(self, ranges: Sequence[range], value: "DTensor") -> "DTensor":
        """gpu_slice_assign: a fresh copy of self with value written into ranges."""
        out = DTensor(copy(self._f32().storage, self._f32().layout))
        v = value._f32()
        write(out.storage, Layout.contiguous(self.shape).narrowed(ranges), v.storage, v.layout)
        return out

    @staticmethod
    def cat(parts: Sequence["DTensor"], d: int) -> "DTensor":
        """gpu_cat: each part written into its slice of one fresh f32 buffer."""
        out_sh = list(parts[0].shape)
        out_sh[d] = sum(p.shape[d] for p in parts)
        out = alloc("f32", out_sh)
        base = Layout.contiguous(out_sh)
        at = 0
        for p in parts:
            v = p._f32()
            r = [range(0, s) for s in out_sh]
            r[d] = range(at, at + p.shape[d])
            at += p.shape[d]
            write(out, base.narrowed(r), v.storage, v.layout)
        return DTensor(out)


def softmax(x: DTensor, d: int) -> DTensor:
    """activation.rs:13-25: exp(x − max) / Σ exp(x − max) along d."""
    e = x.sub(x.max_dim(d)).exp()
    return e.div(e.sum_dim(d))


def log_softmax(x: DTensor, d: int) -> DTensor:
    """activation.rs:27-42: (x − max) − log Σ exp(x − max) along d."""
    shifted = x.sub(x.max_dim(d))
    return shifted.sub(shifted.exp().sum_dim(d).log())
