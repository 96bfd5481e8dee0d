// Generic strided pointwise engine (all eager elementwise ops, casts,
// strided copies, fill) plus the small data-movement kernels: row gather,
// tril/triu and rotary embedding.
//
// Contiguous same-dtype floating operands take a vector path (8 elements per
// thread, 16-byte loads); everything else takes an N-d strided path with one
// element per thread.  Both are HBM-bound; the strided path is for views and
// broadcasts, the vector path for the activations of a model.
#include <algorithm>

#include "sph_common.h"

namespace sph {
namespace {

constexpr int kMaxOperands = 4;

struct PwArgs {
  void* ptr[kMaxOperands];
  int dtype[kMaxOperands];
  int64_t stride[kMaxOperands][SPH_MAX_DIMS];
  int64_t size[SPH_MAX_DIMS];
  int ndim;
  int nin;
  int op;
  double alpha, beta;
  int64_t numel;
};

// ---------------------------------------------------------------------------
// Typed element access by runtime dtype (uniform branches).
// ---------------------------------------------------------------------------
template <typename C>
__device__ inline C load_as(const void* base, int dt, int64_t off) {
  switch (dt) {
    case SPH_F16:
      return static_cast<C>(static_cast<float>(static_cast<const half_t*>(base)[off]));
    case SPH_BF16:
      return static_cast<C>(bf16_to_float(static_cast<const bf16_t*>(base)[off]));
    case SPH_F32:
      return static_cast<C>(static_cast<const float*>(base)[off]);
    case SPH_F64:
      return static_cast<C>(static_cast<const double*>(base)[off]);
    case SPH_I8:
      return static_cast<C>(static_cast<const int8_t*>(base)[off]);
    case SPH_U8:
      return static_cast<C>(static_cast<const uint8_t*>(base)[off]);
    case SPH_I16:
      return static_cast<C>(static_cast<const int16_t*>(base)[off]);
    case SPH_I32:
      return static_cast<C>(static_cast<const int32_t*>(base)[off]);
    case SPH_I64:
      return static_cast<C>(static_cast<const int64_t*>(base)[off]);
    case SPH_BOOL:
      return static_cast<C>(static_cast<const uint8_t*>(base)[off] != 0);
    default:
      return C(0);
  }
}

template <typename C>
__device__ inline void store_as(void* base, int dt, int64_t off, C v) {
  switch (dt) {
    case SPH_F16:
      static_cast<half_t*>(base)[off] = static_cast<half_t>(static_cast<float>(v));
      break;
    case SPH_BF16:
      static_cast<bf16_t*>(base)[off] = float_to_bf16(static_cast<float>(v));
      break;
    case SPH_F32:
      static_cast<float*>(base)[off] = static_cast<float>(v);
      break;
    case SPH_F64:
      static_cast<double*>(base)[off] = static_cast<double>(v);
      break;
    case SPH_I8:
      static_cast<int8_t*>(base)[off] = static_cast<int8_t>(static_cast<int64_t>(v));
      break;
    case SPH_U8:
      static_cast<uint8_t*>(base)[off] = static_cast<uint8_t>(static_cast<int64_t>(v));
      break;
    case SPH_I16:
      static_cast<int16_t*>(base)[off] = static_cast<int16_t>(static_cast<int64_t>(v));
      break;
    case SPH_I32:
      static_cast<int32_t*>(base)[off] = static_cast<int32_t>(static_cast<int64_t>(v));
      break;
    case SPH_I64:
      static_cast<int64_t*>(base)[off] = static_cast<int64_t>(v);
      break;
    case SPH_BOOL:
      static_cast<uint8_t*>(base)[off] = (v != C(0)) ? 1 : 0;
      break;
    default:
      break;
  }
}

// ---------------------------------------------------------------------------
// Op semantics.  C is float, double or int64_t.
// ---------------------------------------------------------------------------
template <typename C>
__device__ inline C m_exp(C x) { if constexpr (sizeof(C) == 8) return exp(x); else return expf(x); }
template <typename C>
__device__ inline C m_log(C x) { if constexpr (sizeof(C) == 8) return log(x); else return logf(x); }

template <typename C>
__device__ inline C eval_float(int op, C a, C b, C c, C alpha, C beta) {
  using std::isnan;
  switch (op) {
    case SPH_PW_COPY: return a;
    case SPH_PW_FILL: return alpha;
    case SPH_PW_ADD: return a + alpha * b;
    case SPH_PW_SUB: return a - alpha * b;
    case SPH_PW_MUL: return a * b;
    case SPH_PW_DIV: return a / b;
    case SPH_PW_ADD_SCALAR: return a + alpha;
    case SPH_PW_MUL_SCALAR: return a * alpha;
    case SPH_PW_RSUB_SCALAR: return alpha - a;
    case SPH_PW_DIV_SCALAR: return a / alpha;
    case SPH_PW_POW_SCALAR: return pow(a, alpha);
    case SPH_PW_RPOW_SCALAR: return pow(alpha, a);
    case SPH_PW_POW: return pow(a, b);
    case SPH_PW_MAXIMUM: return (isnan(a) || isnan(b)) ? a + b : (a > b ? a : b);
    case SPH_PW_MINIMUM: return (isnan(a) || isnan(b)) ? a + b : (a < b ? a : b);
    case SPH_PW_NEG: return -a;
    case SPH_PW_ABS: return fabs(a);
    case SPH_PW_EXP: return m_exp(a);
    case SPH_PW_LOG: return m_log(a);
    case SPH_PW_SQRT: return sqrt(a);
    case SPH_PW_RSQRT: return C(1) / sqrt(a);
    case SPH_PW_RECIPROCAL: return C(1) / a;
    case SPH_PW_SIGMOID: return C(1) / (C(1) + m_exp(-a));
    case SPH_PW_TANH: return tanh(a);
    case SPH_PW_RELU: return isnan(a) ? a : (a > C(0) ? a : C(0));
    case SPH_PW_GELU: return C(0.5) * a * (C(1) + erf(a * C(0.70710678118654752440)));
    case SPH_PW_GELU_TANH: {
      const C k = C(0.79788456080286535588);
      return C(0.5) * a * (C(1) + tanh(k * (a + C(0.044715) * a * a * a)));
    }
    case SPH_PW_SILU: return a / (C(1) + m_exp(-a));
    case SPH_PW_SIN: return sin(a);
    case SPH_PW_COS: return cos(a);
    case SPH_PW_ERF: return erf(a);
    case SPH_PW_LOG1P: return log1p(a);
    case SPH_PW_EXPM1: return expm1(a);
    case SPH_PW_MISH: {
      const C sp = (a > C(20)) ? a : log1p(m_exp(a));
      return a * tanh(sp);
    }
    case SPH_PW_LOGICAL_NOT: return a == C(0) ? C(1) : C(0);
    case SPH_PW_SIGN: return (a > C(0)) ? C(1) : ((a < C(0)) ? C(-1) : a);
    case SPH_PW_FLOOR: return floor(a);
    case SPH_PW_CEIL: return ceil(a);
    case SPH_PW_ROUND: return rint(a);
    case SPH_PW_TRUNC: return trunc(a);
    case SPH_PW_CLAMP: {
      if (isnan(a)) return a;
      C r = a < alpha ? alpha : a;
      return r > beta ? beta : r;
    }
    case SPH_PW_LEAKY_RELU: return a > C(0) ? a : a * alpha;
    case SPH_PW_SQUARE: return a * a;
    case SPH_PW_EQ: return a == b ? C(1) : C(0);
    case SPH_PW_NE: return a != b ? C(1) : C(0);
    case SPH_PW_LT: return a < b ? C(1) : C(0);
    case SPH_PW_LE: return a <= b ? C(1) : C(0);
    case SPH_PW_GT: return a > b ? C(1) : C(0);
    case SPH_PW_GE: return a >= b ? C(1) : C(0);
    case SPH_PW_EQ_SCALAR: return a == alpha ? C(1) : C(0);
    case SPH_PW_NE_SCALAR: return a != alpha ? C(1) : C(0);
    case SPH_PW_LT_SCALAR: return a < alpha ? C(1) : C(0);
    case SPH_PW_LE_SCALAR: return a <= alpha ? C(1) : C(0);
    case SPH_PW_GT_SCALAR: return a > alpha ? C(1) : C(0);
    case SPH_PW_GE_SCALAR: return a >= alpha ? C(1) : C(0);
    case SPH_PW_LOGICAL_AND: return (a != C(0) && b != C(0)) ? C(1) : C(0);
    case SPH_PW_LOGICAL_OR: return (a != C(0) || b != C(0)) ? C(1) : C(0);
    case SPH_PW_WHERE: return a != C(0) ? b : c;
    case SPH_PW_SILU_MUL: return a / (C(1) + m_exp(-a)) * b;
    case SPH_PW_ADDCMUL: return a + alpha * b * c;
    case SPH_PW_LERP: return a + alpha * (b - a);
    default: return C(0);
  }
}

__device__ inline int64_t eval_int(int op, int64_t a, int64_t b, int64_t c,
                                   int64_t alpha, int64_t beta) {
  switch (op) {
    case SPH_PW_COPY: return a;
    case SPH_PW_FILL: return alpha;
    case SPH_PW_ADD: return a + alpha * b;
    case SPH_PW_SUB: return a - alpha * b;
    case SPH_PW_MUL: return a * b;
    case SPH_PW_ADD_SCALAR: return a + alpha;
    case SPH_PW_MUL_SCALAR: return a * alpha;
    case SPH_PW_RSUB_SCALAR: return alpha - a;
    case SPH_PW_MAXIMUM: return a > b ? a : b;
    case SPH_PW_MINIMUM: return a < b ? a : b;
    case SPH_PW_NEG: return -a;
    case SPH_PW_ABS: return a < 0 ? -a : a;
    case SPH_PW_RELU: return a > 0 ? a : 0;
    case SPH_PW_SQUARE: return a * a;
    case SPH_PW_SIGN: return (a > 0) - (a < 0);
    case SPH_PW_CLAMP: { int64_t r = a < alpha ? alpha : a; return r > beta ? beta : r; }
    case SPH_PW_LOGICAL_NOT: return a == 0;
    case SPH_PW_BITWISE_NOT: return ~a;
    case SPH_PW_EQ: return a == b;
    case SPH_PW_NE: return a != b;
    case SPH_PW_LT: return a < b;
    case SPH_PW_LE: return a <= b;
    case SPH_PW_GT: return a > b;
    case SPH_PW_GE: return a >= b;
    case SPH_PW_EQ_SCALAR: return a == alpha;
    case SPH_PW_NE_SCALAR: return a != alpha;
    case SPH_PW_LT_SCALAR: return a < alpha;
    case SPH_PW_LE_SCALAR: return a <= alpha;
    case SPH_PW_GT_SCALAR: return a > alpha;
    case SPH_PW_GE_SCALAR: return a >= alpha;
    case SPH_PW_LOGICAL_AND: return a != 0 && b != 0;
    case SPH_PW_LOGICAL_OR: return a != 0 || b != 0;
    case SPH_PW_WHERE: return a != 0 ? b : c;
    default: return 0;
  }
}

template <typename C>
__device__ inline C eval_op(int op, C a, C b, C c, C alpha, C beta) {
  if constexpr (__is_same(C, int64_t)) return eval_int(op, a, b, c, alpha, beta);
  else return eval_float<C>(op, a, b, c, alpha, beta);
}

// bitwise_not on bool flips the truth value, not all bits.
template <typename C>
__device__ inline C fix_bool_not(int op, int out_dt, C v) {
  if constexpr (__is_same(C, int64_t)) {
    if (op == SPH_PW_BITWISE_NOT && out_dt == SPH_BOOL) return (v & 1) ? 1 : 0;
  }
  return v;
}

// N-d strided path: one element per thread, grid-stride.
template <typename C, typename IDX>
__global__ void __launch_bounds__(256) pw_strided(const PwArgs p) {
  const C alpha = static_cast<C>(p.alpha), beta = static_cast<C>(p.beta);
  for (IDX i = static_cast<IDX>(blockIdx.x) * 256 + threadIdx.x; i < static_cast<IDX>(p.numel);
       i += static_cast<IDX>(gridDim.x) * 256) {
    int64_t off[kMaxOperands] = {0, 0, 0, 0};
    IDX rem = i;
    for (int d = p.ndim - 1; d >= 0; --d) {
      const IDX sz = static_cast<IDX>(p.size[d]);
      const IDX q = rem / sz;
      const int64_t coord = static_cast<int64_t>(rem - q * sz);
      rem = q;
#pragma unroll
      for (int o = 0; o < kMaxOperands; ++o) off[o] += coord * p.stride[o][d];
    }
    C a = C(0), b = C(0), c = C(0);
    if (p.nin > 0) a = load_as<C>(p.ptr[1], p.dtype[1], off[1]);
    if (p.nin > 1) b = load_as<C>(p.ptr[2], p.dtype[2], off[2]);
    if (p.nin > 2) c = load_as<C>(p.ptr[3], p.dtype[3], off[3]);
    C v = eval_op<C>(p.op, a, b, c, alpha, beta);
    v = fix_bool_not<C>(p.op, p.dtype[0], v);
    store_as<C>(p.ptr[0], p.dtype[0], off[0], v);
  }
}

// Contiguous vector path for floating T: 8 elements per thread.
template <typename T>
__global__ void __launch_bounds__(256) pw_vec(const PwArgs p) {
  const float alpha = static_cast<float>(p.alpha), beta = static_cast<float>(p.beta);
  const int64_t nvec = (p.numel + 7) / 8;
  for (int64_t vi = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; vi < nvec;
       vi += static_cast<int64_t>(gridDim.x) * 256) {
    const int64_t e0 = vi * 8;
    const int n = (p.numel - e0) >= 8 ? 8 : static_cast<int>(p.numel - e0);
    float a[8] = {0, 0, 0, 0, 0, 0, 0, 0}, b[8] = {0, 0, 0, 0, 0, 0, 0, 0},
          c[8] = {0, 0, 0, 0, 0, 0, 0, 0}, o[8];
    if (n == 8) {
      if (p.nin > 0) load8<T>(static_cast<const T*>(p.ptr[1]) + e0, a);
      if (p.nin > 1) load8<T>(static_cast<const T*>(p.ptr[2]) + e0, b);
      if (p.nin > 2) load8<T>(static_cast<const T*>(p.ptr[3]) + e0, c);
    } else {
      if (p.nin > 0) load8_partial<T>(static_cast<const T*>(p.ptr[1]) + e0, n, 0.f, a);
      if (p.nin > 1) load8_partial<T>(static_cast<const T*>(p.ptr[2]) + e0, n, 0.f, b);
      if (p.nin > 2) load8_partial<T>(static_cast<const T*>(p.ptr[3]) + e0, n, 0.f, c);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) o[j] = eval_float<float>(p.op, a[j], b[j], c[j], alpha, beta);
    if (n == 8) store8<T>(static_cast<T*>(p.ptr[0]) + e0, o);
    else store8_partial<T>(static_cast<T*>(p.ptr[0]) + e0, n, o);
  }
}

bool op_is_int_exact(int op) {
  switch (op) {
    case SPH_PW_COPY: case SPH_PW_FILL: case SPH_PW_ADD: case SPH_PW_SUB:
    case SPH_PW_MUL: case SPH_PW_ADD_SCALAR: case SPH_PW_MUL_SCALAR:
    case SPH_PW_RSUB_SCALAR: case SPH_PW_MAXIMUM: case SPH_PW_MINIMUM:
    case SPH_PW_NEG: case SPH_PW_ABS: case SPH_PW_RELU: case SPH_PW_SQUARE:
    case SPH_PW_SIGN: case SPH_PW_CLAMP: case SPH_PW_LOGICAL_NOT:
    case SPH_PW_BITWISE_NOT: case SPH_PW_EQ: case SPH_PW_NE: case SPH_PW_LT:
    case SPH_PW_LE: case SPH_PW_GT: case SPH_PW_GE: case SPH_PW_EQ_SCALAR:
    case SPH_PW_NE_SCALAR: case SPH_PW_LT_SCALAR: case SPH_PW_LE_SCALAR:
    case SPH_PW_GT_SCALAR: case SPH_PW_GE_SCALAR: case SPH_PW_LOGICAL_AND:
    case SPH_PW_LOGICAL_OR: case SPH_PW_WHERE:
      return true;
    default:
      return false;
  }
}

int op_arity(int op) {
  switch (op) {
    case SPH_PW_FILL: return 0;
    case SPH_PW_ADD: case SPH_PW_SUB: case SPH_PW_MUL: case SPH_PW_DIV:
    case SPH_PW_POW: case SPH_PW_MAXIMUM: case SPH_PW_MINIMUM: case SPH_PW_EQ:
    case SPH_PW_NE: case SPH_PW_LT: case SPH_PW_LE: case SPH_PW_GT:
    case SPH_PW_GE: case SPH_PW_LOGICAL_AND: case SPH_PW_LOGICAL_OR:
    case SPH_PW_SILU_MUL: case SPH_PW_LERP:
      return 2;
    case SPH_PW_WHERE: case SPH_PW_ADDCMUL: return 3;
    default: return 1;
  }
}

// Drops size-1 dims and merges dims that are contiguous for every operand.
void coalesce(PwArgs& p, int nops) {
  int nd = 0;
  int64_t size[SPH_MAX_DIMS];
  int64_t stride[kMaxOperands][SPH_MAX_DIMS];
  for (int d = 0; d < p.ndim; ++d) {
    if (p.size[d] == 1) continue;
    if (nd > 0) {
      bool mergeable = true;
      for (int o = 0; o < nops; ++o)
        if (stride[o][nd - 1] != p.stride[o][d] * p.size[d]) mergeable = false;
      if (mergeable) {
        size[nd - 1] *= p.size[d];
        for (int o = 0; o < nops; ++o) stride[o][nd - 1] = p.stride[o][d];
        continue;
      }
    }
    size[nd] = p.size[d];
    for (int o = 0; o < nops; ++o) stride[o][nd] = p.stride[o][d];
    ++nd;
  }
  if (nd == 0) {  // scalar
    size[0] = 1;
    for (int o = 0; o < nops; ++o) stride[o][0] = 0;
    nd = 1;
  }
  p.ndim = nd;
  for (int d = 0; d < nd; ++d) {
    p.size[d] = size[d];
    for (int o = 0; o < nops; ++o) p.stride[o][d] = stride[o][d];
  }
  for (int d = nd; d < SPH_MAX_DIMS; ++d) {
    p.size[d] = 1;
    for (int o = 0; o < kMaxOperands; ++o) p.stride[o][d] = 0;
  }
}

inline unsigned grid_for(int64_t work, int64_t per_block) {
  int64_t g = (work + per_block - 1) / per_block;
  if (g > 65536) g = 65536;
  if (g < 1) g = 1;
  return static_cast<unsigned>(g);
}

}  // namespace
}  // namespace sph

using namespace sph;

extern "C" int sph_pointwise(int op, int nin, const sph_operand* operands,
                             int ndim, const int64_t* sizes, double alpha,
                             double beta, sph_stream_t stream) {
  SPH_REQUIRE(op >= 0 && op < SPH_PW_OP_COUNT_, SPH_ERR_INVALID_ARG, "pointwise: bad op");
  SPH_REQUIRE(nin == op_arity(op), SPH_ERR_INVALID_ARG, "pointwise: wrong number of inputs");
  SPH_REQUIRE(ndim >= 0 && ndim <= SPH_MAX_DIMS, SPH_ERR_INVALID_ARG, "pointwise: ndim > 8");
  PwArgs p{};
  p.ndim = ndim;
  p.nin = nin;
  p.op = op;
  p.alpha = alpha;
  p.beta = beta;
  const int nops = nin + 1;
  int64_t numel = 1;
  for (int d = 0; d < ndim; ++d) {
    SPH_REQUIRE(sizes[d] >= 0, SPH_ERR_INVALID_ARG, "pointwise: negative size");
    p.size[d] = sizes[d];
    numel *= sizes[d];
  }
  if (numel == 0) return SPH_OK;
  bool any_f64 = false, all_int = true;
  for (int o = 0; o < nops; ++o) {
    SPH_REQUIRE(dtype_size(operands[o].dtype) > 0, SPH_ERR_INVALID_ARG, "pointwise: bad dtype");
    p.ptr[o] = operands[o].data;
    p.dtype[o] = operands[o].dtype;
    for (int d = 0; d < ndim; ++d) p.stride[o][d] = operands[o].strides[d];
    if (operands[o].dtype == SPH_F64) any_f64 = true;
    if (is_float_dtype(operands[o].dtype)) all_int = false;
  }
  coalesce(p, nops);
  p.numel = numel;
  hipStream_t st = as_stream(stream);

  // Vector path: everything contiguous and of one floating dtype.
  bool vec = p.ndim == 1 && !any_f64;
  for (int o = 0; o < nops && vec; ++o) {
    vec = p.stride[o][0] == 1 && p.dtype[o] == p.dtype[0] &&
          (p.dtype[o] == SPH_F16 || p.dtype[o] == SPH_BF16 || p.dtype[o] == SPH_F32) &&
          (reinterpret_cast<uintptr_t>(p.ptr[o]) & 15u) == 0;
  }
  if (vec && op_is_int_exact(op) && op != SPH_PW_COPY && op != SPH_PW_FILL &&
      (op >= SPH_PW_EQ && op <= SPH_PW_GE_SCALAR))
    vec = false;  // comparisons produce bool outputs elsewhere
  if (vec) {
    const unsigned g = grid_for((numel + 7) / 8, 256);
    switch (p.dtype[0]) {
      case SPH_F16: pw_vec<half_t><<<g, 256, 0, st>>>(p); break;
      case SPH_BF16: pw_vec<bf16_t><<<g, 256, 0, st>>>(p); break;
      default: pw_vec<float><<<g, 256, 0, st>>>(p); break;
    }
    return check_launch("sph_pointwise");
  }
  const unsigned g = grid_for(numel, 256);
  const bool small = numel < (1LL << 31);
  if (any_f64) {
    if (small) pw_strided<double, uint32_t><<<g, 256, 0, st>>>(p);
    else pw_strided<double, uint64_t><<<g, 256, 0, st>>>(p);
  } else if (all_int && op_is_int_exact(op)) {
    if (small) pw_strided<int64_t, uint32_t><<<g, 256, 0, st>>>(p);
    else pw_strided<int64_t, uint64_t><<<g, 256, 0, st>>>(p);
  } else {
    SPH_REQUIRE(op != SPH_PW_BITWISE_NOT, SPH_ERR_UNSUPPORTED,
                "pointwise: bitwise_not needs integer operands");
    if (small) pw_strided<float, uint32_t><<<g, 256, 0, st>>>(p);
    else pw_strided<float, uint64_t><<<g, 256, 0, st>>>(p);
  }
  return check_launch("sph_pointwise");
}

// ---------------------------------------------------------------------------
// Row gather
// ---------------------------------------------------------------------------
namespace sph {
namespace {
template <typename V>
__global__ void __launch_bounds__(256)
gather_rows_kernel(const V* __restrict__ table, int64_t num_rows, int64_t row_v,
                   const void* __restrict__ idx, int idx64, int64_t n_idx,
                   V* __restrict__ out, int32_t* __restrict__ oob) {
  const int64_t i = blockIdx.x;
  const int64_t r = idx64 ? static_cast<const int64_t*>(idx)[i]
                          : static_cast<int64_t>(static_cast<const int32_t*>(idx)[i]);
  V* o = out + i * row_v;
  if (r < 0 || r >= num_rows) {
    for (int64_t c = threadIdx.x; c < row_v; c += 256) o[c] = V{};
    // one lane reports it (a plain vector store; any number of workgroups
    // may store the same 1)
    if (oob != nullptr && threadIdx.x == 0) *reinterpret_cast<volatile int32_t*>(oob) = 1;
    return;
  }
  const V* s = table + r * row_v;
  for (int64_t c = threadIdx.x; c < row_v; c += 256) o[c] = s[c];
}
}  // namespace
}  // namespace sph

extern "C" int sph_gather_rows(const void* table, int64_t num_rows,
                               int64_t row_elems, int elem_bytes,
                               const void* idx, int idx_is_i64, int64_t n_idx,
                               void* out, int32_t* oob_flag, sph_stream_t stream) {
  SPH_REQUIRE(num_rows >= 0 && row_elems >= 0 && n_idx >= 0, SPH_ERR_INVALID_ARG,
              "gather_rows: negative size");
  SPH_REQUIRE(elem_bytes == 1 || elem_bytes == 2 || elem_bytes == 4 || elem_bytes == 8,
              SPH_ERR_INVALID_ARG, "gather_rows: elem_bytes");
  SPH_REQUIRE(n_idx <= 0x7fffffffLL, SPH_ERR_TOO_LARGE, "gather_rows: too many indices");
  if (n_idx == 0 || row_elems == 0) return SPH_OK;
  hipStream_t st = as_stream(stream);
  const int64_t row_bytes = row_elems * elem_bytes;
  const bool v16 = (row_bytes % 16 == 0) && ((reinterpret_cast<uintptr_t>(table) & 15u) == 0) &&
                   ((reinterpret_cast<uintptr_t>(out) & 15u) == 0);
  const unsigned g = static_cast<unsigned>(n_idx);
  if (v16) {
    gather_rows_kernel<u32x4><<<g, 256, 0, st>>>(static_cast<const u32x4*>(table), num_rows,
                                                 row_bytes / 16, idx, idx_is_i64, n_idx,
                                                 static_cast<u32x4*>(out), oob_flag);
  } else if (elem_bytes == 2) {
    gather_rows_kernel<uint16_t><<<g, 256, 0, st>>>(static_cast<const uint16_t*>(table), num_rows,
                                                    row_elems, idx, idx_is_i64, n_idx,
                                                    static_cast<uint16_t*>(out), oob_flag);
  } else if (elem_bytes == 4) {
    gather_rows_kernel<uint32_t><<<g, 256, 0, st>>>(static_cast<const uint32_t*>(table), num_rows,
                                                    row_elems, idx, idx_is_i64, n_idx,
                                                    static_cast<uint32_t*>(out), oob_flag);
  } else if (elem_bytes == 8) {
    gather_rows_kernel<uint64_t><<<g, 256, 0, st>>>(static_cast<const uint64_t*>(table), num_rows,
                                                    row_elems, idx, idx_is_i64, n_idx,
                                                    static_cast<uint64_t*>(out), oob_flag);
  } else {
    gather_rows_kernel<uint8_t><<<g, 256, 0, st>>>(static_cast<const uint8_t*>(table), num_rows,
                                                   row_elems, idx, idx_is_i64, n_idx,
                                                   static_cast<uint8_t*>(out), oob_flag);
  }
  return check_launch("sph_gather_rows");
}

// ---------------------------------------------------------------------------
// Transposing copy: dst[b, v, u] = src[b, u, v] through 64 x 64 LDS tiles
// ---------------------------------------------------------------------------
namespace sph {
namespace {

constexpr int kTT = 64;  // tile edge (elements)

struct TransposeArgs {
  const void* src;
  void* dst;
  int64_t U, V;     // sizes of the dst-contiguous dim u and the src-contiguous dim v
  int64_t su, dv;   // stride of u in src, of v in dst (elements)
  int64_t nbatch, tiles_u, tiles_v;
  int nb;           // batch dims (<= 4), outermost first
  int64_t bsize[4], bsrc[4], bdst[4];
};

// One 256-thread workgroup per 64 x 64 tile of one batch entry: the load
// walks v (contiguous in src) across lanes, the store walks u (contiguous
// in dst) across lanes, so both sides are coalesced; the tile sits in LDS
// as [v][u] with one element of padding per row.
template <typename T>
__global__ void __launch_bounds__(256) transpose_tile_kernel(TransposeArgs a) {
  __shared__ T tile[kTT][kTT + 1];
  const int64_t tu = blockIdx.x % a.tiles_u, tv = blockIdx.x / a.tiles_u;
  const int64_t u0 = tu * kTT, v0 = tv * kTT;
  const int tx = threadIdx.x % kTT, ty = threadIdx.x / kTT;
  for (int64_t b = blockIdx.y; b < a.nbatch; b += gridDim.y) {
    int64_t rem = b, so = 0, doff = 0;
    for (int d = a.nb - 1; d >= 0; --d) {
      const int64_t i = rem % a.bsize[d];
      rem /= a.bsize[d];
      so += i * a.bsrc[d];
      doff += i * a.bdst[d];
    }
    const T* src = static_cast<const T*>(a.src) + so;
    T* dst = static_cast<T*>(a.dst) + doff;
    const int64_t v = v0 + tx;
#pragma unroll 4
    for (int i = ty; i < kTT; i += 4) {
      const int64_t u = u0 + i;
      if (u < a.U && v < a.V) tile[tx][i] = src[u * a.su + v];
    }
    __syncthreads();
    const int64_t u = u0 + tx;
#pragma unroll 4
    for (int i = ty; i < kTT; i += 4) {
      const int64_t vv = v0 + i;
      if (u < a.U && vv < a.V) dst[vv * a.dv + u] = tile[i][tx];
    }
    __syncthreads();
  }
}

// 2-byte elements with whole 64 x 64 tiles and 16-byte aligned rows: each
// thread loads two 16-byte chunks of src rows (8 consecutive v) and stores
// two 16-byte chunks of dst rows (8 consecutive u).  The tile sits in LDS as
// [u][v] with a 66-element row pitch: the store phase's column reads (8 rows
// of one v per thread, 8 threads per v) then fall on distinct banks.
__global__ void __launch_bounds__(256) transpose_tile16_kernel(TransposeArgs a) {
  constexpr int P = kTT + 2;  // row pitch (elements)
  __shared__ __attribute__((aligned(16))) uint16_t tile[kTT * P];
  const int64_t tu = blockIdx.x % a.tiles_u, tv = blockIdx.x / a.tiles_u;
  const int64_t u0 = tu * kTT, v0 = tv * kTT;
  const int t = threadIdx.x;
  for (int64_t b = blockIdx.y; b < a.nbatch; b += gridDim.y) {
    int64_t rem = b, so = 0, doff = 0;
    for (int d = a.nb - 1; d >= 0; --d) {
      const int64_t i = rem % a.bsize[d];
      rem /= a.bsize[d];
      so += i * a.bsrc[d];
      doff += i * a.bdst[d];
    }
    const uint16_t* src = static_cast<const uint16_t*>(a.src) + so;
    uint16_t* dst = static_cast<uint16_t*>(a.dst) + doff;
    u32x4 ld[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int c = t + 256 * k, u = c >> 3, j = c & 7;
      ld[k] = *reinterpret_cast<const u32x4*>(src + (u0 + u) * a.su + v0 + 8 * j);
    }
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int c = t + 256 * k, u = c >> 3, j = c & 7;
      uint32_t* row = reinterpret_cast<uint32_t*>(tile + u * P + 8 * j);
#pragma unroll
      for (int e = 0; e < 4; ++e) row[e] = ld[k][e];
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int c = t + 256 * k, v = c >> 3, i = c & 7;
      uint32_t w[4];
#pragma unroll
      for (int e = 0; e < 4; ++e)
        w[e] = static_cast<uint32_t>(tile[(8 * i + 2 * e) * P + v]) |
               (static_cast<uint32_t>(tile[(8 * i + 2 * e + 1) * P + v]) << 16);
      *reinterpret_cast<u32x4*>(dst + (v0 + v) * a.dv + u0 + 8 * i) = u32x4{w[0], w[1], w[2], w[3]};
    }
    __syncthreads();
  }
}

}  // namespace
}  // namespace sph

extern "C" int sph_transpose_copy(int elem_bytes, const void* src, void* dst, int64_t U, int64_t V,
                                  int64_t su, int64_t dv, int nb, const int64_t* bsizes,
                                  const int64_t* bsrc_strides, const int64_t* bdst_strides,
                                  sph_stream_t stream) {
  SPH_REQUIRE(elem_bytes == 1 || elem_bytes == 2 || elem_bytes == 4 || elem_bytes == 8,
              SPH_ERR_INVALID_ARG, "transpose_copy: elem_bytes");
  SPH_REQUIRE(U >= 0 && V >= 0 && nb >= 0 && nb <= 4, SPH_ERR_INVALID_ARG,
              "transpose_copy: negative size or more than 4 batch dims");
  TransposeArgs a{};
  a.src = src;
  a.dst = dst;
  a.U = U;
  a.V = V;
  a.su = su;
  a.dv = dv;
  a.nb = nb;
  a.nbatch = 1;
  for (int d = 0; d < nb; ++d) {
    SPH_REQUIRE(bsizes[d] >= 0, SPH_ERR_INVALID_ARG, "transpose_copy: negative batch size");
    a.bsize[d] = bsizes[d];
    a.bsrc[d] = bsrc_strides[d];
    a.bdst[d] = bdst_strides[d];
    a.nbatch *= bsizes[d];
  }
  if (U == 0 || V == 0 || a.nbatch == 0) return SPH_OK;
  a.tiles_u = ceil_div(U, kTT);
  a.tiles_v = ceil_div(V, kTT);
  SPH_REQUIRE(a.tiles_u * a.tiles_v < (int64_t(1) << 31), SPH_ERR_TOO_LARGE,
              "transpose_copy: too many tiles");
  dim3 grid(static_cast<unsigned>(a.tiles_u * a.tiles_v),
            static_cast<unsigned>(a.nbatch < 65535 ? a.nbatch : 65535));
  hipStream_t st = as_stream(stream);
  // whole tiles, rows and batch offsets of both sides 16-byte aligned
  bool wide = elem_bytes == 2 && U % kTT == 0 && V % kTT == 0 && su % 8 == 0 && dv % 8 == 0 &&
              (reinterpret_cast<uintptr_t>(src) & 15) == 0 && (reinterpret_cast<uintptr_t>(dst) & 15) == 0;
  for (int d = 0; d < nb && wide; ++d) wide = (a.bsize[d] == 1) || (a.bsrc[d] % 8 == 0 && a.bdst[d] % 8 == 0);
  if (wide) {
    transpose_tile16_kernel<<<grid, 256, 0, st>>>(a);
    return check_launch("sph_transpose_copy");
  }
  switch (elem_bytes) {
    case 1: transpose_tile_kernel<uint8_t><<<grid, 256, 0, st>>>(a); break;
    case 2: transpose_tile_kernel<uint16_t><<<grid, 256, 0, st>>>(a); break;
    case 4: transpose_tile_kernel<uint32_t><<<grid, 256, 0, st>>>(a); break;
    default: transpose_tile_kernel<uint64_t><<<grid, 256, 0, st>>>(a); break;
  }
  return check_launch("sph_transpose_copy");
}

// ---------------------------------------------------------------------------
// tril / triu
// ---------------------------------------------------------------------------
namespace sph {
namespace {
template <typename V>
__global__ void __launch_bounds__(256)
tri_kernel(const V* __restrict__ x, V* __restrict__ y, int64_t total, int64_t rows,
           int64_t cols, int upper, int64_t diag) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * 256) {
    const int64_t c = i % cols;
    const int64_t r = (i / cols) % rows;
    const bool keep = upper ? (c - r >= diag) : (c - r <= diag);
    y[i] = keep ? x[i] : V{};
  }
}
}  // namespace
}  // namespace sph

extern "C" int sph_tri(int upper, int64_t diagonal, int elem_bytes, const void* x,
                       void* y, int64_t batch, int64_t rows, int64_t cols,
                       sph_stream_t stream) {
  SPH_REQUIRE(batch >= 0 && rows >= 0 && cols >= 0, SPH_ERR_INVALID_ARG, "tri: negative size");
  const int64_t total = batch * rows * cols;
  if (total == 0) return SPH_OK;
  hipStream_t st = as_stream(stream);
  const unsigned g = grid_for(total, 256);
  switch (elem_bytes) {
    case 1:
      tri_kernel<uint8_t><<<g, 256, 0, st>>>(static_cast<const uint8_t*>(x), static_cast<uint8_t*>(y),
                                             total, rows, cols, upper, diagonal);
      break;
    case 2:
      tri_kernel<uint16_t><<<g, 256, 0, st>>>(static_cast<const uint16_t*>(x), static_cast<uint16_t*>(y),
                                              total, rows, cols, upper, diagonal);
      break;
    case 4:
      tri_kernel<uint32_t><<<g, 256, 0, st>>>(static_cast<const uint32_t*>(x), static_cast<uint32_t*>(y),
                                              total, rows, cols, upper, diagonal);
      break;
    case 8:
      tri_kernel<uint64_t><<<g, 256, 0, st>>>(static_cast<const uint64_t*>(x), static_cast<uint64_t*>(y),
                                              total, rows, cols, upper, diagonal);
      break;
    default:
      return set_error(SPH_ERR_INVALID_ARG, "tri: elem_bytes");
  }
  return check_launch("sph_tri");
}

// ---------------------------------------------------------------------------
// Rotary embedding (rotate-half)
// ---------------------------------------------------------------------------
namespace sph {
namespace {
template <typename T>
__global__ void __launch_bounds__(256)
rope_kernel(const T* __restrict__ x, T* __restrict__ y, const int64_t* __restrict__ pos,
            int64_t tokens, int64_t heads, int64_t half, float log2_theta) {
  const int64_t total = tokens * heads * half;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * 256) {
    const int64_t f = i % half;
    const int64_t th = i / half;  // token * heads + head
    const int64_t tok = th / heads;
    const float inv_freq = exp2f(-log2_theta * (2.0f * static_cast<float>(f)) /
                                 (2.0f * static_cast<float>(half)));
    const float ang = static_cast<float>(pos[tok]) * inv_freq;
    float sn, cs;
    sincosf(ang, &sn, &cs);
    const int64_t base = th * 2 * half;
    const float x1 = Num<T>::to_f(x[base + f]);
    const float x2 = Num<T>::to_f(x[base + f + half]);
    y[base + f] = Num<T>::from_f(x1 * cs - x2 * sn);
    y[base + f + half] = Num<T>::from_f(x2 * cs + x1 * sn);
  }
}
}  // namespace
}  // namespace sph

extern "C" int sph_rope(sph_dtype dtype, const void* x, void* y, const int64_t* positions,
                        int64_t tokens, int64_t heads, int64_t head_dim, float theta,
                        sph_stream_t stream) {
  SPH_REQUIRE(tokens >= 0 && heads >= 0 && head_dim >= 0 && head_dim % 2 == 0,
              SPH_ERR_INVALID_ARG, "rope: bad shape");
  SPH_REQUIRE(theta > 0.f, SPH_ERR_INVALID_ARG, "rope: theta must be > 0");
  const int64_t total = tokens * heads * (head_dim / 2);
  if (total == 0) return SPH_OK;
  hipStream_t st = as_stream(stream);
  const unsigned g = grid_for(total, 256);
  const float l2t = std::log2(theta);
  switch (dtype) {
    case SPH_F16:
      rope_kernel<half_t><<<g, 256, 0, st>>>(static_cast<const half_t*>(x), static_cast<half_t*>(y),
                                             positions, tokens, heads, head_dim / 2, l2t);
      break;
    case SPH_BF16:
      rope_kernel<bf16_t><<<g, 256, 0, st>>>(static_cast<const bf16_t*>(x), static_cast<bf16_t*>(y),
                                             positions, tokens, heads, head_dim / 2, l2t);
      break;
    case SPH_F32:
      rope_kernel<float><<<g, 256, 0, st>>>(static_cast<const float*>(x), static_cast<float*>(y),
                                            positions, tokens, heads, head_dim / 2, l2t);
      break;
    default:
      return set_error(SPH_ERR_UNSUPPORTED, "rope: dtype");
  }
  return check_launch("sph_rope");
}
