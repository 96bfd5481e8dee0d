"""SpyreKernel: Inductor loop IR -> HIP source for gfx950.

Reference: SpyreKernel (torch_spyre/_inductor/spyre_kernel.py:85-369), which
records exactly ONE op per kernel (`record_compute_op` raises on a second,
:107-114) and summarises it as a KernelSpec for the Spyre SuperDSC emitter.
Here a kernel is a whole fused Inductor node group: every load, pointwise
op, reduction and store of the group is emitted as HIP C++ into one of two
hand-written templates (include/spyre_inductor_rt.h):

  pointwise  one thread per element of the flattened x range;
  reduction  one workgroup per x row; each reduction phase is a strided loop
             over the row (coalesced, fp32 accumulators) closed by a block
             reduction, and phases that depend on earlier reductions (softmax,
             norms) follow in the same kernel.

The kernel is compiled by hiprtc at compile time (runtime/async_compile.py)
and launched by torch_spyre._C.launch_kernel.  Static shapes only: dynamic
sizes raise Unsupported.
"""

from __future__ import annotations

import hashlib
import itertools
import math
import re
from typing import Any, Optional, Union

import sympy
import torch
from sympy.printing.precedence import PRECEDENCE

from torch._inductor.codegen.common import (
    is_buffer_removed,
    CSEVariable,
    DeferredLine,
    IndentedBuffer,
    OpOverrides,
)
from torch._inductor.codegen.simd import IterationRangesEntry, SIMDKernel
from torch._inductor.utils import get_bounds_index_expr
from torch._inductor.virtualized import OpsWrapper, V, ops
from torch.utils._sympy.functions import Identity
from torch.utils._sympy.printers import ExprPrinter
from torch.utils._sympy.value_ranges import ValueRanges, bound_sympy

from . import Unsupported

DTYPE_TO_HIP = {
    torch.float32: "float",
    torch.float64: "double",
    torch.float16: "_Float16",
    torch.bfloat16: "bfloat16",
    torch.bool: "bool",
    torch.int8: "int8_t",
    torch.uint8: "uint8_t",
    torch.int32: "int32_t",
    torch.int64: "int64_t",
}

# Values of these dtypes are widened to fp32 on load.
_FLOAT_LOAD = {torch.float16, torch.bfloat16, torch.float32, torch.float64}
_PRODUCT = re.compile(r"^(\w+) \* (\w+)$")
_SUM = re.compile(r"^(\w+) \+ (\w+)$")
_ERF = re.compile(r"^spy::erf_fast\((\w+)\)$")

MAX_BLOCK = 512
# Row loops of at most this many trips keep each loaded value in registers
# for the later phases of the row (softmax's sum and normalise, LayerNorm's
# normalise): the row is read from memory once.
MAX_CACHED_TRIPS = 8
# Row reductions over >= 512 elements give each thread VEC consecutive row
# elements per trip, emitted as VEC straight-line copies of the body: loads
# and stores of contiguous rows at consecutive indices merge into 16-byte
# accesses.  Pointwise kernels give each thread EPT elements strided by the
# block (every wave instruction stays one coalesced run; index expressions
# with broadcasts do not merge reliably into wide accesses, and partly merged
# ones lose the coalescing) once there are enough elements to keep ~1024
# workgroups: EPT independent loads in flight per thread instead of one.
PW_BLOCK = 256
VEC = 8
# Row elements per thread the row-reduction block is sized for.
ROW_EPT = 16
# Pointwise kernels whose direct (not gathered) accesses all walk their
# buffers contiguously give each thread GROUP consecutive elements: such a
# load is one 16-byte load of the group and such a store one 16-byte store
# (fp16 / bf16; two of each for fp32) instead of GROUP 2-byte accesses.
GROUP = 8
# Outputs of at least this many bytes are written with streaming stores: they
# do not fit in the caches for their consumer anyway, and the streaming form
# measured 3-5 % faster on the [8192, 4096] row kernels.  Smaller outputs
# (a decoder layer's activations) keep plain stores, so the next kernel can
# find them in the caches.
NT_STORE_BYTES = 64 << 20


_GROUP_DTYPES = (torch.float16, torch.bfloat16, torch.float32)
_XINDEX = re.compile(r"\bxindex\b")
_IDENT = re.compile(r"\b[A-Za-z_]\w*\b")
_TMP = re.compile(r"tmp\d+")


def _next_pow2(n: int) -> int:
    return 1 << max(0, (int(n) - 1).bit_length())


def hip_value(val: Any) -> str:
    if isinstance(val, bool):
        return "true" if val else "false"
    if isinstance(val, float):
        if val == math.inf:
            return "spy::inf()"
        if val == -math.inf:
            return "(-spy::inf())"
        if val != val:
            return '__builtin_nanf("")'
        return f"{val!r}f"
    if isinstance(val, int):
        return f"static_cast<int64_t>({val}LL)"
    return str(val)


class HipExprPrinter(ExprPrinter):
    """sympy index expressions -> int64 C++ expressions."""

    def _print_Symbol(self, expr):
        return str(expr)

    def _print_Integer(self, expr):
        return f"{int(expr)}LL"

    def _print_FloorDiv(self, expr):
        x, div = expr.args
        return f"spy::floordiv_i({self.doprint(x)}, {self.doprint(div)})"

    def _print_ModularIndexing(self, expr):
        x, div, mod = expr.args
        x = self.doprint(x)
        if div != 1:
            x = f"spy::floordiv_i({x}, {self.doprint(div)})"
        return f"spy::mod_i({x}, {self.doprint(mod)})"

    def _print_Mod(self, expr):
        return f"spy::mod_i({self.doprint(expr.args[0])}, {self.doprint(expr.args[1])})"

    def _print_PythonMod(self, expr):
        return self._print_Mod(expr)

    def _print_Min(self, expr):
        args = [self.doprint(a) for a in expr.args]
        out = args[0]
        for a in args[1:]:
            out = f"spy::min_i({out}, {a})"
        return out

    def _print_Max(self, expr):
        args = [self.doprint(a) for a in expr.args]
        out = args[0]
        for a in args[1:]:
            out = f"spy::max_i({out}, {a})"
        return out

    def _print_Where(self, expr):
        c, p, q = (self.parenthesize(a, PRECEDENCE["Atom"] - 0.5) for a in expr.args)
        return f"({c} ? {p} : {q})"

    def _print_Pow(self, expr):
        base, exp = expr.args
        if exp.is_Integer and int(exp) >= 0:
            b = self.parenthesize(base, PRECEDENCE["Mul"])
            return "*".join([b] * int(exp)) if int(exp) > 0 else "1LL"
        raise Unsupported(f"index expression {expr}")

    def _print_PowByNatural(self, expr):
        return self._print_Pow(sympy.Pow(*expr.args))

    def _print_Abs(self, expr):
        a = self.doprint(expr.args[0])
        return f"(({a}) < 0 ? -({a}) : ({a}))"

    def _print_ToFloat(self, expr):
        return f"static_cast<float>({self.doprint(expr.args[0])})"

    def _print_IntTrueDiv(self, expr):
        a, b = expr.args
        return f"(static_cast<float>({self.doprint(a)}) / static_cast<float>({self.doprint(b)}))"

    def _print_FloorToInt(self, expr):
        return f"static_cast<int64_t>(floorf({self.doprint(expr.args[0])}))"

    def _print_TruncToInt(self, expr):
        return f"static_cast<int64_t>(truncf({self.doprint(expr.args[0])}))"

    def _print_Float(self, expr):
        return f"{float(expr)!r}f"


_printer = HipExprPrinter()


def _defining_expr(v: Any) -> Optional[str]:
    """The expression a CSE variable of the current kernel was generated
    from (None for anything else)."""
    if not isinstance(v, CSEVariable):
        return None
    for key, var in V.kernel.cse._cache.items():
        if var is v and isinstance(key, str):
            return key
    return None


def _product(e: Optional[str]) -> Optional[tuple[str, str]]:
    m = _PRODUCT.match(e) if e is not None else None
    return (m.group(1), m.group(2)) if m else None


def _scaled_by(e: Optional[str], const: str) -> Optional[str]:
    """x when `e` is x * c or c * x with c a variable holding `const`."""
    p = _product(e)
    if p is None:
        return None
    for x, c in (p, p[::-1]):
        var = V.kernel.cse.try_get(const)
        if var is not None and str(var) == c:
            return x
    return None


def _gelu_input(half: Any, tail: Any) -> Optional[str]:
    """x when half * tail is the erf form of GELU that aten.gelu decomposes
    into: (x * 0.5) * (erf(x * M_SQRT1_2) + 1)."""
    x = _scaled_by(_defining_expr(half), hip_value(0.5))
    if x is None:
        return None
    t = _defining_expr(tail)
    m = _SUM.match(t) if t is not None else None
    if m is None:
        return None
    one = V.kernel.cse.try_get(hip_value(1.0))
    for e, c in ((m.group(1), m.group(2)), (m.group(2), m.group(1))):
        if one is None or str(one) != c:
            continue
        evar = next((v for k, v in V.kernel.cse._cache.items() if str(v) == e), None)
        f = _ERF.match(_defining_expr(evar) or "")
        if f is None:
            continue
        arg = next((v for k, v in V.kernel.cse._cache.items() if str(v) == f.group(1)), None)
        if _scaled_by(_defining_expr(arg), hip_value(math.sqrt(0.5))) == x:
            return x
    return None


class SpyreOverrides(OpOverrides):
    """Pointwise ops as HIP C++ expressions on fp32 (or native int) values."""

    @staticmethod
    def mul(a, b):
        # GELU's erf form collapses to one call (spy::gelu_erf): max(x, 0)
        # minus |x| times a Gaussian tail, about a third of the operations
        # of 0.5 x (1 + erf(x / sqrt 2)) through a general erf.
        for h, t in ((a, b), (b, a)):
            x = _gelu_input(h, t)
            if x is not None:
                return f"spy::gelu_erf({x})"
        return f"{a} * {b}"

    @staticmethod
    def to_dtype(x, dtype: torch.dtype, src_dtype: Optional[torch.dtype] = None,
                 use_compute_types: bool = True):
        if dtype == torch.float16:
            return f"spy::round_half({x})"
        if dtype == torch.bfloat16:
            return f"spy::round_bf16({x})"
        if dtype in (torch.float32, torch.float64):
            return f"static_cast<float>({x})"
        if dtype == torch.bool:
            return f"(({x}) != 0)"
        if dtype in DTYPE_TO_HIP:
            return f"static_cast<{DTYPE_TO_HIP[dtype]}>({x})"
        raise Unsupported(f"to_dtype {dtype}")

    @staticmethod
    def to_dtype_bitcast(x, dtype, src_dtype):
        raise Unsupported("bitcast")

    @staticmethod
    def constant(val, dtype: torch.dtype):
        if dtype.is_floating_point:
            return hip_value(float(val))
        if dtype == torch.bool:
            return hip_value(bool(val))
        return hip_value(int(val))

    @staticmethod
    def index_expr(expr: sympy.Expr, dtype: torch.dtype):
        idx = V.kernel.index_to_str(V.kernel.prepare_indexing(expr))
        var = V.kernel.cse.generate(V.kernel.compute, idx, bounds=get_bounds_index_expr(expr),
                                    dtype=torch.int64)
        return ops.to_dtype(var, dtype)

    @staticmethod
    def masked(mask, body, other):
        with V.kernel.mask_loads(mask, other) as new_mask:
            result = body()
        if isinstance(result, tuple):
            raise Unsupported("masked tuple")
        other_s = hip_value(other) if not isinstance(other, CSEVariable) else str(other)
        return V.kernel.cse.generate(V.kernel.compute,
                                     f"(({new_mask}) ? ({result}) : ({other_s}))",
                                     dtype=getattr(result, "dtype", None))

    @staticmethod
    def where(a, b, c):
        return f"(({a}) ? ({b}) : ({c}))"

    # comparisons / logic (C++ yields bool)
    @staticmethod
    def eq(a, b):
        return f"({a} == {b})"

    @staticmethod
    def ne(a, b):
        return f"({a} != {b})"

    @staticmethod
    def lt(a, b):
        return f"({a} < {b})"

    @staticmethod
    def le(a, b):
        return f"({a} <= {b})"

    @staticmethod
    def gt(a, b):
        return f"({a} > {b})"

    @staticmethod
    def ge(a, b):
        return f"({a} >= {b})"

    @staticmethod
    def logical_and(a, b):
        return f"({a} && {b})"

    @staticmethod
    def logical_or(a, b):
        return f"({a} || {b})"

    @staticmethod
    def logical_not(a):
        return f"(!{a})"

    @staticmethod
    def logical_xor(a, b):
        return f"(static_cast<bool>({a}) != static_cast<bool>({b}))"

    @staticmethod
    def bitwise_and(a, b):
        return f"({a} & {b})"

    @staticmethod
    def bitwise_or(a, b):
        return f"({a} | {b})"

    @staticmethod
    def bitwise_xor(a, b):
        return f"({a} ^ {b})"

    @staticmethod
    def bitwise_not(a):
        return f"(~{a})"

    # arithmetic
    @staticmethod
    def neg(x):
        return f"(-{x})"

    @staticmethod
    def reciprocal(x):
        return f"(1.0f / {x})"

    @staticmethod
    def square(x):
        return f"({x} * {x})"

    @staticmethod
    def floordiv(a, b):
        return f"spy::floordiv({a}, {b})"

    @staticmethod
    def truncdiv(a, b):
        return f"spy::truncdiv({a}, {b})"

    @staticmethod
    def remainder(a, b):
        return f"spy::remainder({a}, {b})"

    @staticmethod
    def mod(a, b):
        return f"spy::remainder({a}, {b})"

    @staticmethod
    def fmod(a, b):
        return f"fmodf({a}, {b})"

    @staticmethod
    def pow(a, b):
        return f"powf({a}, {b})"

    @staticmethod
    def maximum(a, b):
        return f"spy::maximum({a}, {b})"

    @staticmethod
    def minimum(a, b):
        return f"spy::minimum({a}, {b})"

    @staticmethod
    def abs(x):
        return f"fabsf({x})"

    @staticmethod
    def relu(x):
        return f"spy::relu({x})"

    @staticmethod
    def sigmoid(x):
        return f"spy::sigmoid({x})"

    @staticmethod
    def rsqrt(x):
        return f"spy::rsqrt({x})"

    @staticmethod
    def sign(x):
        return f"spy::sign({x})"

    @staticmethod
    def round(x):
        return f"rintf({x})"

    @staticmethod
    def isnan(x):
        return f"({x} != {x})"

    @staticmethod
    def isinf(x):
        return f"(spy::isinf_({x}) != 0.f)"

    @staticmethod
    def signbit(x):
        return f"signbit({x})"

    @staticmethod
    def fma(a, b, c):
        return f"fmaf({a}, {b}, {c})"


def _unary_fn(fn: str):
    return staticmethod(lambda x: f"{fn}({x})")


for _name, _fn in {
    "exp": "expf", "exp2": "exp2f", "expm1": "expm1f", "log": "logf", "log2": "log2f",
    "log10": "log10f", "log1p": "log1pf", "sqrt": "sqrtf", "sin": "sinf", "cos": "cosf",
    "tan": "tanf", "tanh": "tanhf", "asin": "asinf", "acos": "acosf", "atan": "atanf",
    "sinh": "sinhf", "cosh": "coshf", "asinh": "asinhf", "acosh": "acoshf", "atanh": "atanhf",
    "erf": "spy::erf_fast", "erfc": "erfcf", "floor": "floorf", "ceil": "ceilf", "trunc": "truncf",
    "lgamma": "lgammaf",
}.items():
    setattr(SpyreOverrides, _name, _unary_fn(_fn))

SpyreOverrides.atan2 = staticmethod(lambda a, b: f"atan2f({a}, {b})")
SpyreOverrides.copysign = staticmethod(lambda a, b: f"copysignf({a}, {b})")
SpyreOverrides.hypot = staticmethod(lambda a, b: f"hypotf({a}, {b})")


class SpyreKernel(SIMDKernel):
    """One generated HIP kernel (see module docstring)."""

    overrides = SpyreOverrides  # type: ignore[assignment]
    suffix = ";"
    newvar_prefix = "auto "
    kexpr = _printer.doprint

    def __init__(self, tiling: dict[str, sympy.Expr], **kwargs: Any) -> None:
        super().__init__(tiling, **kwargs)
        self._acc_ids = itertools.count()
        self._rloop_open = False
        self._pending_accum = False
        # kernel argument name -> max element extent (None = not checkable)
        self._extents: dict[str, Optional[int]] = {}
        # (argument, index) -> register array holding that load for each
        # trip of a short row loop
        self._row_cache: dict[tuple[str, str], str] = {}
        # Pointwise group form: the contiguous loads / stores (each emitted
        # through a macro that the kernel defines as an element access or as
        # the group's register array), the index variables of the x tree,
        # and whether some direct access rules the form out.
        self._grp_loads: dict[tuple[str, str, Optional[int]], int] = {}
        # (argument, index, dtype, span): span set for a masked load, whose
        # group is read only where it lies inside the buffer
        self._grp_load_info: list[tuple[str, sympy.Expr, torch.dtype, Optional[int]]] = []
        self._grp_stores: list[tuple[str, str, sympy.Expr, torch.dtype, bool]] = []
        self._grp_bad = False
        self._grp_gathered: set[int] = set()  # group loads with a gathered index
        self._x_entries: list[tuple[str, str, int, int]] = []

    # -- sizes ----------------------------------------------------------------
    def _static(self, e) -> int:
        if not isinstance(e, (int, sympy.Integer)):
            raise Unsupported(f"dynamic size {e}")
        return int(e)

    def _xnumel(self) -> int:
        n = 1
        for t in self.range_trees:
            if not t.is_reduction:
                n *= self._static(t.numel)
        return n

    def _rnumel(self) -> int:
        n = 1
        for t in self.range_trees:
            if t.is_reduction:
                n *= self._static(t.numel)
        return n

    def _block(self) -> int:
        # Row reductions: about 16 elements per thread (two VEC trips;
        # fewer, larger workgroups amortise the block reductions' barriers),
        # 64 .. 512.  Against 8 per thread, measured on the compiled c1 / c3
        # kernels (rows of 4096): GELU chain + row-sum 24.1 -> 22.1 us,
        # softmax 4.9 -> 4.5 us, add + RMSNorm / LayerNorm 0.5 % faster.
        if self.inside_reduction or self.features.is_reduction():
            return min(MAX_BLOCK, max(64, _next_pow2(self._rnumel()) // ROW_EPT))
        return PW_BLOCK

    def _rvec(self) -> int:
        return VEC if self._rnumel() >= 64 * VEC else 1

    def _trips(self) -> int:
        r, span = self._rnumel(), self._block() * self._rvec()
        return (r + span - 1) // span

    @staticmethod
    def _ept(xnumel: int) -> int:
        # keep at least ~1024 workgroups (4 per CU) before packing elements
        for ept in (8, 4, 2):
            if xnumel >= PW_BLOCK * ept * 1024:
                return ept
        return 1

    def dtype_to_str(self, dtype: torch.dtype) -> str:
        try:
            return DTYPE_TO_HIP[dtype]
        except KeyError:
            raise Unsupported(f"dtype {dtype}")

    def should_use_persistent_reduction(self) -> bool:
        return False  # reductions are strided loops over the row

    def should_use_cooperative_reduction(self) -> bool:
        return False

    # -- index ranges -----------------------------------------------------------
    def _record_extent(self, name: str, index: sympy.Expr, masked: bool) -> None:
        ext: Optional[int]
        if masked:
            ext = None
        else:
            ranges = {}
            for sym, entry in self.range_tree_nodes.items():
                ranges[sym] = ValueRanges(0, self._static(entry.length) - 1)
            free = index.free_symbols
            if any(s not in ranges for s in free):
                ext = None  # indirect (gathered) index
            else:
                vr = bound_sympy(index, {s: ranges[s] for s in free})
                lo, hi = vr.lower, vr.upper
                if not (lo.is_number and hi.is_number) or lo < 0:
                    raise Unsupported(f"cannot bound index {index}")
                ext = int(hi) + 1
        prev = self._extents.get(name, 0)
        if prev is None or ext is None:
            self._extents[name] = None
        else:
            self._extents[name] = max(prev, ext)

    def _open_rloop(self) -> None:
        if self._rloop_open:
            return
        r, b, v = self._rnumel(), self._block(), self._rvec()
        loops = self._trips()
        if loops <= MAX_CACHED_TRIPS:
            self.body.writeline("#pragma unroll")
        self.body.writeline(f"for (int64_t r0_cnt = 0; r0_cnt < {loops}LL; ++r0_cnt) {{")
        self.body.writeline("#pragma unroll")
        self.body.writeline(f"for (int spy_v = 0; spy_v < {v}; ++spy_v) {{")
        with self.body.indent():
            self.body.writeline(
                f"const int64_t r0_index = (r0_cnt * {b}LL + threadIdx.x) * {v}LL + spy_v;")
            if loops * b * v != r:
                self.body.writeline(f"if (r0_index >= {r}LL) break;")
        self._rloop_open = True

    def codegen_iteration_ranges_entry(self, entry: IterationRangesEntry) -> None:
        expr = self.kexpr(self.rename_indexing(entry.expr))
        if entry.is_reduction:
            self._open_rloop()
            with self.body.indent():
                self.body.writeline(f"const int64_t {entry.name} = {expr};")
        else:
            self.indexing_code.writeline(f"const int64_t {entry.name} = {expr};")
            try:
                div, length = int(entry.divisor), int(entry.length)
            except (TypeError, ValueError):
                div, length = 0, 0
            self._x_entries.append((entry.name, expr, div, length))

    # -- memory -------------------------------------------------------------------
    def _group_uniform(self, name: str, depth: int = 0) -> bool:
        """A value of the kernel body (a CSE variable) that is the same for
        GROUP consecutive elements whose first flat index is a multiple of
        GROUP: every name in its defining expression is such a value, an
        index variable with a divisor that is a multiple of GROUP, or a
        pointer, type or function name."""
        if depth > 32:
            return False
        expr = None
        for key, var in self.cse._cache.items():
            if isinstance(key, str) and str(var) == name:
                expr = key
                break
        if expr is None:
            return False
        entries = {str(s): e for s, e in self.range_tree_nodes.items()}
        for ident in _IDENT.findall(expr):
            if _TMP.fullmatch(ident):
                if not self._group_uniform(ident, depth + 1):
                    return False
            elif ident in entries:
                e = entries[ident]
                try:
                    div = int(e.divisor)
                except (TypeError, ValueError):
                    return False
                if e.is_reduction or div == 1 or div % GROUP:
                    return False
            elif ident == "xindex" or ident.startswith(("r0_", "spy_", "SPY_")):
                return False
        return True

    def _group_class(self, index: sympy.Expr) -> str:
        """How a pointwise access moves over GROUP consecutive elements whose
        first flat index is a multiple of GROUP: "vec" (the index advances
        by 1 and starts at a multiple of GROUP: one wide access), "bcast"
        (the index is the same for all of them) or "other"."""
        if self.features.is_reduction() or self.inside_reduction:
            return "other"
        index = index.replace(lambda e: isinstance(e, Identity), lambda e: e.args[0])
        entries = {}
        for sym in index.free_symbols:
            e = self.range_tree_nodes.get(sym)
            if e is None and self._group_uniform(str(sym)):
                entries[sym] = (GROUP, 0)  # a gathered index, the same for the group
                continue
            if e is None or e.is_reduction:
                return "other"  # gathered (indirect) index
            try:
                div, length = int(e.divisor), int(e.length)
            except (TypeError, ValueError):
                return "other"
            entries[sym] = (div, length)
        inner = [s for s, (d, ln) in entries.items() if d == 1]
        for s, (d, ln) in entries.items():
            # variables with divisor 1 step by one inside a group (their
            # range a multiple of GROUP, so a group never wraps them); the
            # others stay fixed (divisor a multiple of GROUP)
            if (d == 1 and ln % GROUP) or (d != 1 and d % GROUP):
                return "other"
        if not inner:
            return "bcast"
        total = 0
        rest = index
        for s in inner:
            c = sympy.diff(index, s)
            if not c.is_Integer:
                return "other"
            total += int(c)
            rest = rest - c * s
        if total != 1:
            return "other"
        rest = sympy.expand(rest)
        for term, coeff in rest.as_coefficients_dict().items():
            if not coeff.is_Integer or int(coeff) % GROUP:
                return "other"
            if not (term == 1 or (term.is_Symbol and term in entries)):
                return "other"
        return "vec"

    @staticmethod
    def _buffer_span(name: str) -> Optional[int]:
        """Elements of a buffer as laid out from the kernel's pointer,
        1 + sum (size - 1) * stride (None if unknown)."""
        try:
            layout = V.graph.get_buffer(name).get_layout()
            size = [int(n) for n in layout.size]
            stride = [int(st) for st in layout.stride]
        except Exception:
            return None
        if any(n <= 0 for n in size) or any(st < 0 for st in stride):
            return None
        return 1 + sum((n - 1) * st for n, st in zip(size, stride))

    def load(self, name: str, index: sympy.Expr) -> CSEVariable:
        var = self.args.input(name)
        index = self.prepare_indexing(index)
        dtype = V.graph.get_dtype(name)
        self.dtype_to_str(dtype)
        masked = bool(self._load_mask)
        grouped = False
        gathered = self.is_indirect_indexing(index)
        if not (self.features.is_reduction() or self.inside_reduction):
            cls = self._group_class(index)
            span = None
            if cls == "vec" and dtype in _GROUP_DTYPES:
                # A masked load reads its whole group where the group lies
                # inside the buffer (checked per group at run time; elements
                # outside it read 0), and the mask selects per element.
                if masked:
                    span = self._buffer_span(name)
                grouped = (not masked or span is not None) and not (masked and gathered)
            elif cls == "other":
                self._grp_bad = True
        if grouped and masked:
            # what the group form may read: the buffer's span, checked
            # against the storage at launch
            prev = self._extents.get(str(var), 0)
            self._extents[str(var)] = None if prev is None else max(prev, span)
        else:
            self._record_extent(str(var), index, masked)
        if grouped:
            key = (str(var), self.index_to_str(index), span)
            k = self._grp_loads.get(key)
            if k is None:
                k = len(self._grp_load_info)
                self._grp_loads[key] = k
                self._grp_load_info.append((str(var), index, dtype, span))
                if gathered:
                    # the gathered index is computed in the body: the group
                    # is read there, by its first element
                    self._grp_gathered.add(k)
                    self.compute.writeline(f"SPY_GLD{k};")
            if gathered:
                return self.cse.generate(self.compute, f"SPY_LD{k}", dtype=torch.float32)
            if not masked:
                return self.cse.generate(self.loads, f"SPY_LD{k}", dtype=torch.float32)
            other = self._load_other
            other_s = hip_value(other) if other is not None else "0"
            return self.cse.generate(self.compute, f"(({self._load_mask}) ? SPY_LD{k} : {other_s})",
                                     dtype=torch.float32)
        line = f"{var}[{self.index_to_str(index)}]"
        if dtype in _FLOAT_LOAD:
            line = f"spy::to_f({line})"
            out_dtype = torch.float32
        else:
            out_dtype = dtype
        buf = self.loads
        if masked:
            other = self._load_other
            other_s = hip_value(other) if other is not None else "0"
            line = f"(({self._load_mask}) ? {line} : {other_s})"
            buf = self.compute
        elif self.is_indirect_indexing(index):
            buf = self.compute
        elif self._cacheable_row_load(index):
            key = (str(var), self.index_to_str(index))
            arr = self._row_cache.get(key)
            if arr is None:
                arr = f"rc{len(self._row_cache)}"
                ctype = "float" if dtype in _FLOAT_LOAD else self.dtype_to_str(dtype)
                self.indexing_code.writeline(f"{ctype} {arr}[{self._trips() * self._rvec()}];")
                self._row_cache[key] = arr
                self.loads.writeline(f"{arr}[r0_cnt * {self._rvec()} + spy_v] = {line};")
            return self.cse.generate(buf, f"{arr}[r0_cnt * {self._rvec()} + spy_v]",
                                     dtype=out_dtype)
        return self.cse.generate(buf, line, dtype=out_dtype)

    def _cacheable_row_load(self, index: sympy.Expr) -> bool:
        """A load inside a short row loop whose index depends on the row
        position: later phases of the same row read it from registers."""
        if not (self.inside_reduction and self.features.is_reduction()):
            return False
        if self._trips() > MAX_CACHED_TRIPS:
            return False
        return any(e.is_reduction and sym in index.free_symbols
                   for sym, e in self.range_tree_nodes.items())

    def store(self, name: str, index: sympy.Expr, value: CSEVariable,
              mode: Any = None) -> None:
        if mode is not None:
            raise Unsupported(f"store mode {mode}")
        var = self.args.output(name)
        index = self.prepare_indexing(index)
        dtype = V.graph.get_dtype(name)
        self._record_extent(str(var), index, False)
        ctype = self.dtype_to_str(dtype)
        if self._streaming_output(name, dtype):
            line = (f"spy::store_nt(&{var}[{self.index_to_str(index)}], "
                    f"spy::cvt<{ctype}>({value}));")
        else:
            line = f"{var}[{self.index_to_str(index)}] = spy::cvt<{ctype}>({value});"
        if not (self.features.is_reduction() or self.inside_reduction):
            # A scatter (an index computed in the body) keeps the element
            # form: the grouped store is written after the element loop,
            # where the body's index variables are out of scope.
            if (self._group_class(index) == "vec" and dtype in _GROUP_DTYPES
                    and not self.is_indirect_indexing(index)):
                k = len(self._grp_stores)
                self._grp_stores.append((name, str(var), index, dtype,
                                         self._streaming_output(name, dtype)))
                line = f"SPY_ST{k}({value});"
            else:
                self._grp_bad = True
        if self.inside_reduction:
            self.compute.writeline(DeferredLine(name, line))
            if self._cacheable_row_load(index):
                # later phases of the row read the stored value (as rounded
                # to the buffer's dtype) from registers, not back from memory
                key = (str(var), self.index_to_str(index))
                arr = self._row_cache.get(key)
                fl = dtype in _FLOAT_LOAD
                if arr is None:
                    arr = f"rc{len(self._row_cache)}"
                    self.indexing_code.writeline(
                        f"{'float' if fl else ctype} {arr}[{self._trips() * self._rvec()}];")
                    self._row_cache[key] = arr
                stored = f"spy::cvt<{ctype}>({value})"
                self.compute.writeline(f"{arr}[r0_cnt * {self._rvec()} + spy_v] = "
                                       f"{f'spy::to_f({stored})' if fl else stored};")
        else:
            self.stores.writeline(DeferredLine(name, line))

    @staticmethod
    def _streaming_output(name: str, dtype: torch.dtype) -> bool:
        try:
            numel = int(V.graph.get_numel(name))
        except (TypeError, ValueError):
            return False
        return numel * dtype.itemsize >= NT_STORE_BYTES

    def store_reduction(self, name: str, index: sympy.Expr, value: CSEVariable) -> None:
        var = self.args.output(name)
        index = self.prepare_indexing(index)
        dtype = V.graph.get_dtype(name)
        self._record_extent(str(var), index, False)
        line = (f"if (threadIdx.x == 0) {var}[{self.index_to_str(index)}] = "
                f"spy::cvt<{self.dtype_to_str(dtype)}>({value});")
        self.stores.writeline(DeferredLine(name, line))

    def check_bounds(self, expr: sympy.Expr, size: sympy.Expr, lower: bool, upper: bool) -> None:
        # Indirect indices (gathers, scatters) are checked without a trap: an
        # out-of-range index is reported to the device error word (a kernel
        # parameter the launcher appends; the host raises IndexError at its
        # next synchronisation) and replaced by 0, so the access stays in
        # bounds.  Eager index_select / embedding report the same way.
        if not (lower or upper):
            return
        if not isinstance(expr, sympy.Symbol):
            raise Unsupported(f"bounds check on {expr}")
        e = str(expr)
        n = self.index_to_str(size)
        self._needs_error_word = True
        # Branch-free: the flag collects in a register and the error word is
        # written once at the end of the kernel.  (A store to the volatile
        # error word inside the row loop split every element into its own
        # block, so the row's loads and stores did not merge into 16-byte
        # accesses and the index was reloaded per element.)
        self.compute.writeline(f"{{ const bool spy_c = {e} < 0 || {e} >= {n}; "
                               f"spy_bad |= spy_c; {e} = spy_c ? 0 : {e}; }}")

    # -- reductions ---------------------------------------------------------------
    def _acc(self, decl: str) -> str:
        name = f"acc{next(self._acc_ids)}"
        self.indexing_code.writeline(decl.format(name=name))
        return name

    def reduction(self, dtype, src_dtype, reduction_type, value):
        key = (src_dtype, reduction_type, value)
        if key in self.cse.reduction_cache:
            return self.cse.reduction_cache[key]
        result = self._reduction(dtype, src_dtype, reduction_type, value)
        self.cse.reduction_cache[key] = result  # type: ignore[assignment]
        return result

    def _reduction(self, dtype, src_dtype, reduction_type, value):
        assert self.inside_reduction
        if self._load_mask:
            raise Unsupported("masked reduction")
        b = self._block()
        self._pending_accum = True
        ops_map = {"sum": "SumF", "prod": "ProdF", "max": "MaxF", "min": "MinF", "any": "AnyF"}
        if reduction_type in ops_map:
            op = ops_map[reduction_type]
            acc = self._acc(f"float {{name}} = spy::{op}::id();")
            self.compute.writeline(f"{acc} = spy::{op}::op({acc}, static_cast<float>({value}));")
            return self.cse.generate(
                self.stores, f"spy::block_reduce<spy::{op}, {b}>({acc}, spy_lds)",
                dtype=torch.float32)
        if reduction_type in ("argmax", "argmin"):
            is_max = "true" if reduction_type == "argmax" else "false"
            init = "-spy::inf()" if reduction_type == "argmax" else "spy::inf()"
            av = self._acc(f"float {{name}} = {init};")
            ai = self._acc("int64_t {name} = 0x7fffffffffffffffLL;")
            rvar = "r0_index"
            self.compute.writeline(
                f"spy::arg_combine<{is_max}>({av}, {ai}, static_cast<float>({value}), {rvar});")
            return self.cse.generate(
                self.stores, f"spy::block_arg<{is_max}, {b}>({av}, {ai}, spy_lds, spy_lds_i)",
                dtype=torch.int64)
        if reduction_type == "welford_reduce":
            acc = self._acc("spy::WelfordAcc {name} = {{0.f, 0.f, 0.f, 0.f}};")
            self.compute.writeline(
                f"{acc} = spy::welford_acc_add({acc}, static_cast<float>({value}));")
            res = self.cse.generate(
                self.stores, f"spy::block_welford<{b}>(spy::welford_finish({acc}), spy_lds)",
                dtype=torch.float32)
            return OpsWrapper._unwrap(
                tuple(CSEVariable(f"{res}.{f}", ValueRanges.unknown(), torch.float32)
                      for f in ("mean", "m2", "weight")))
        if reduction_type == "welford_combine":
            mean, m2, weight = value
            acc = self._acc("spy::Welford {name} = {{0.f, 0.f, 0.f}};")
            self.compute.writeline(
                f"{acc} = spy::welford_combine({acc}, spy::Welford{{static_cast<float>({mean}), "
                f"static_cast<float>({m2}), static_cast<float>({weight})}});")
            res = self.cse.generate(self.stores, f"spy::block_welford<{b}>({acc}, spy_lds)",
                                    dtype=torch.float32)
            return OpsWrapper._unwrap(
                tuple(CSEVariable(f"{res}.{f}", ValueRanges.unknown(), torch.float32)
                      for f in ("mean", "m2", "weight")))
        raise Unsupported(f"reduction {reduction_type}")

    # -- assembly -----------------------------------------------------------------
    def codegen_body(self) -> None:
        if self._pending_accum and not self._rloop_open and self.inside_reduction:
            self._open_rloop()
        if self._rloop_open:
            with self.body.indent():
                self.body.splice(self.loads)
                self.body.splice(self.compute)
            self.body.writeline("}}")
            self._rloop_open = False
            # values computed inside the loop die with it; reduction results
            # (made after the loop) stay available to later phases
            keep = set()
            for item in self.cse.reduction_cache.values():
                for v in (item if isinstance(item, tuple) else (item,)):
                    keep.add(v)
            from torch.utils._ordered_set import OrderedSet

            self.cse.invalidate(OrderedSet(keep))
            for entry in self.range_tree_nodes.values():
                if entry.is_reduction:
                    entry.cache_clear()
        else:
            self.body.splice(self.loads)
            self.body.splice(self.compute)
        self._pending_accum = False
        self.body.splice(self.stores)
        self.loads.clear()
        self.compute.clear()
        self.stores.clear()

    def _kernel_args(self):
        arg_defs, call_args, _, arg_types = self.args.python_argdefs()
        if self.args.sizevars or self.args.workspace_args:
            raise Unsupported("dynamic sizes / workspaces")
        outputs = {inner for inner in self.args.output_buffers.values() if isinstance(inner, str)}
        for inplaced in self.args.inplace_buffers.values():
            if hasattr(inplaced, "inner_name"):
                outputs.add(inplaced.inner_name)
        return arg_defs, call_args, arg_types, outputs

    def codegen_kernel(self, name: Optional[str] = None) -> str:
        self.codegen_body()
        is_red = self.features.is_reduction()
        xnumel, rnumel = self._xnumel(), (self._rnumel() if is_red else 1)
        block = self._block()
        arg_defs, call_args, arg_types, outputs = self._kernel_args()
        params = []
        spec_args = []
        for i, (ad, outer, dt) in enumerate(zip(arg_defs, call_args, arg_types)):
            inner = str(ad.name) if hasattr(ad, "name") else str(ad)
            ctype = self.dtype_to_str(dt)
            if inner in outputs or inner.startswith("in_out_ptr"):
                params.append(f"{ctype}* __restrict__ {inner}")
                is_input = False
            else:
                params.append(f"const {ctype}* __restrict__ {inner}")
                is_input = True
            # keyed by the kernel-side argument name, so buffers that are
            # mutated in place (passed under their graph-input name) keep
            # their bound; an argument the body never touched is unbounded
            ext = self._extents.get(inner)
            spec_args.append(f"TensorArg(is_input={is_input}, arg_index={i}, "
                             f"dtype={dt!r}, extent={ext!r})")
        if getattr(self, "_needs_error_word", False):
            # the device error word, appended by the launcher after the buffers
            params.append("volatile int* __restrict__ spy_err")
        code = IndentedBuffer()
        code.writeline('#include "spyre_inductor_rt.h"')
        n_index_lines = len([ln for ln in self.indexing_code.getvalue().splitlines() if ln.strip()])
        group = (not is_red and xnumel % GROUP == 0 and not self._grp_bad
                 and bool(self._grp_load_info or self._grp_stores)
                 and n_index_lines == len(self._x_entries))
        stores = [(name, var, index, dt, nt) for name, var, index, dt, nt in self._grp_stores
                  if not is_buffer_removed(name)]
        # the contiguous accesses: element accesses, or the group's arrays
        for k, (var, index, dt, _) in enumerate(self._grp_load_info):
            code.writeline(f"#define SPY_LD{k} spy_ld{k}[spy_v]" if group else
                           f"#define SPY_LD{k} spy::to_f({var}[{self.index_to_str(index)}])")
            if k in self._grp_gathered:
                code.writeline(f"#define SPY_GLD{k} if (spy_v == 0) spy::load8f({var} + "
                               f"({self._group_first(index)}), spy_al, spy_ld{k})" if group else
                               f"#define SPY_GLD{k}")
        for k, (name, var, index, dt, nt) in enumerate(self._grp_stores):
            ct = self.dtype_to_str(dt)
            if group:
                code.writeline(f"#define SPY_ST{k}(v_) spy_st{k}[spy_v] = spy::cvt<{ct}>(v_)")
            elif nt:
                code.writeline(f"#define SPY_ST{k}(v_) spy::store_nt(&{var}[{self.index_to_str(index)}], "
                               f"spy::cvt<{ct}>(v_))")
            else:
                code.writeline(f"#define SPY_ST{k}(v_) {var}[{self.index_to_str(index)}] = "
                               f"spy::cvt<{ct}>(v_)")
        code.writeline(f'extern "C" __global__ void __launch_bounds__({block}) spyre_kernel(')
        with code.indent():
            code.writeline(",\n".join(params) if params else "")
        code.writeline(") {")
        needs_err = getattr(self, "_needs_error_word", False)
        with code.indent():
            if needs_err:
                code.writeline("bool spy_bad = false;")
            if is_red:
                code.writeline(f"__shared__ float spy_lds[3 * {max(1, block // 64)}];")
                code.writeline(f"__shared__ int64_t spy_lds_i[{max(1, block // 64)}];")
                code.writeline("const int64_t xindex = blockIdx.x;")
                grid = xnumel
            elif group:
                grid = (xnumel // GROUP + block - 1) // block
            else:
                ept = self._ept(xnumel)
                span = block * ept
                grid = (xnumel + span - 1) // span
            if is_red:
                code.splice(self.indexing_code)
                code.splice(self.body)
            elif group:
                self._codegen_group(code, block, xnumel, stores)
            elif ept == 1:
                code.writeline(f"const int64_t xindex = static_cast<int64_t>(blockIdx.x) * {block}LL"
                               " + threadIdx.x;")
                code.writeline(f"if (xindex >= {xnumel}LL) return;")
                code.splice(self.indexing_code)
                code.splice(self.body)
            else:
                # Whole spans run EPT straight-line copies of the body (all
                # loads can be issued before the first store); the tail span
                # checks each element.
                code.writeline(f"const int64_t spy_base = static_cast<int64_t>(blockIdx.x) * {span}LL;")
                code.writeline(f"if (spy_base + {span}LL <= {xnumel}LL) {{")
                with code.indent():
                    code.writeline("#pragma unroll")
                    code.writeline(f"for (int spy_e = 0; spy_e < {ept}; ++spy_e) {{")
                    with code.indent():
                        code.writeline(f"const int64_t xindex = spy_base + spy_e * {block}LL + threadIdx.x;")
                        code.splice(self.indexing_code)
                        code.splice(self.body)
                    code.writeline("}")
                code.writeline("} else {")
                with code.indent():
                    code.writeline(f"for (int spy_e = 0; spy_e < {ept}; ++spy_e) {{")
                    with code.indent():
                        code.writeline(f"const int64_t xindex = spy_base + spy_e * {block}LL + threadIdx.x;")
                        code.writeline(f"if (xindex < {xnumel}LL) {{")
                        with code.indent():
                            code.splice(self.indexing_code)
                            code.splice(self.body)
                        code.writeline("}")
                    code.writeline("}")
                code.writeline("}")
            if needs_err:
                code.writeline("if (spy_bad) *spy_err = 1;")
        code.writeline("}")
        src = code.getvalue()
        if grid <= 0 or grid >= 2**31:
            raise Unsupported(f"grid {grid}")
        # a name of its own per kernel (kind + source hash), so profiles tell
        # generated kernels apart
        symbol = (f"spyre_{'red' if is_red else 'pw'}_"
                  f"{hashlib.sha1(src.encode()).hexdigest()[:10]}")
        src = src.replace(") spyre_kernel(\n", f") {symbol}(\n", 1)
        spec = IndentedBuffer()
        spec.writeline("KernelSpec(")
        with spec.indent():
            spec.writeline(f"op={'reduction' if is_red else 'pointwise'!r},")
            spec.writeline(f"is_reduction={is_red},")
            spec.writeline(f"dimensions={[xnumel, rnumel] if is_red else [xnumel]!r},")
            spec.writeline(f"grid={grid}, block={block},")
            if getattr(self, "_needs_error_word", False):
                spec.writeline("error_word=True,")
            spec.writeline("args=[")
            with spec.indent():
                for a in spec_args:
                    spec.writeline(a + ",")
            spec.writeline("],")
            spec.writeline(f"source={src!r},")
            spec.writeline(f"symbol={symbol!r},")
        spec.writeline(")")
        return spec.getvalue()

    def _group_first(self, index: sympy.Expr) -> str:
        """The index of a group's first element (index variables at their
        group base; a gathered index, the same for the group, as it is)."""
        return self.kexpr(index.subs({s: sympy.Symbol(f"spy_b_{s.name}", integer=True)
                                      for s in index.free_symbols
                                      if s in self.range_tree_nodes}))

    def _codegen_group(self, code: IndentedBuffer, block: int, xnumel: int, stores) -> None:
        """Pointwise body over GROUP consecutive elements per thread: the
        contiguous loads are read as whole groups before the element loop
        and the contiguous stores written as whole groups after it."""
        code.writeline(f"const int64_t spy_xb = (static_cast<int64_t>(blockIdx.x) * {block}LL"
                       f" + threadIdx.x) * {GROUP}LL;")
        code.writeline(f"if (spy_xb >= {xnumel}LL) return;")
        ptrs = sorted({var for var, _, _, _ in self._grp_load_info} | {var for _, var, _, _, _ in stores})
        ors = " | ".join(f"reinterpret_cast<unsigned long long>({v})" for v in ptrs)
        code.writeline(f"const bool spy_al = (({ors}) & 15ULL) == 0ULL;")
        for nm, expr, _, _ in self._x_entries:
            base = _XINDEX.sub("spy_xb", expr)
            code.writeline(f"const int64_t spy_b_{nm} = {base};")

        first = self._group_first
        for k, (var, index, dt, span) in enumerate(self._grp_load_info):
            code.writeline(f"float spy_ld{k}[{GROUP}];")
            if k in self._grp_gathered:
                continue  # read in the body (SPY_GLD)
            if span is None:
                code.writeline(f"spy::load8f({var} + ({first(index)}), spy_al, spy_ld{k});")
            else:
                code.writeline(f"spy::load8f_in({var}, {first(index)}, {span}LL, spy_al, spy_ld{k});")
        for k, (name, var, index, dt, nt) in enumerate(self._grp_stores):
            code.writeline(f"{self.dtype_to_str(dt)} spy_st{k}[{GROUP}];")
        code.writeline("#pragma unroll")
        code.writeline(f"for (int spy_v = 0; spy_v < {GROUP}; ++spy_v) {{")
        with code.indent():
            code.writeline("const int64_t xindex = spy_xb + spy_v;")
            code.writeline("(void)xindex;")
            for nm, expr, div, length in self._x_entries:
                if div == 1 and length % GROUP == 0:
                    code.writeline(f"const int64_t {nm} = spy_b_{nm} + spy_v;")
                elif div > 1 and div % GROUP == 0:
                    code.writeline(f"const int64_t {nm} = spy_b_{nm};")
                else:
                    code.writeline(f"const int64_t {nm} = {expr};")
            code.splice(self.body)
        code.writeline("}")
        for k, (name, var, index, dt, nt) in enumerate(self._grp_stores):
            if is_buffer_removed(name):
                continue
            code.writeline(f"spy::store8v<{self.dtype_to_str(dt)}, {'true' if nt else 'false'}>("
                           f"{var} + ({first(index)}), spy_al, spy_st{k});")

    def call_kernel(self, name: str, node: Any = None, deallocate_ws: bool = True) -> None:
        wrapper = V.graph.wrapper_code
        _, call_args, _, _ = self.args.python_argdefs()
        wrapper.writeline(f"{name}.run({', '.join(str(a) for a in call_args)})")
