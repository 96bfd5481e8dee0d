// Generic strided reductions (sum, mean, max, min, argmax, argmin, prod,
// sum of squares, any, all) over any subset of up to 8 dims.
//
// The host reorders the iteration space as [kept dims..., reduced dims...].
// When the innermost reduced dim is contiguous in memory a wave reduces one
// output (lanes stride the reduced elements -> coalesced reads), or, for a
// few long rows (e.g. argmax over an LM head's logits), a whole 1024-thread
// workgroup reduces one output; otherwise one thread reduces one output and
// adjacent threads read adjacent kept elements.
#include <math.h>

#include "sph_common.h"

namespace sph {
namespace {

struct RedArgs {
  const void* in;
  void* out;
  int in_dt, out_dt;
  int op;
  int n_outer, n_inner;  // dims of each group
  int64_t outer_size[SPH_MAX_DIMS], outer_in_stride[SPH_MAX_DIMS], outer_out_stride[SPH_MAX_DIMS];
  int64_t inner_size[SPH_MAX_DIMS], inner_stride[SPH_MAX_DIMS];
  int64_t outer_numel, inner_numel;
};

template <typename A>
struct Acc {
  A v;
  int64_t idx;
};

template <typename A>
__device__ inline A load_val(const void* base, int dt, int64_t off) {
  switch (dt) {
    case SPH_F16: return static_cast<A>(static_cast<float>(static_cast<const half_t*>(base)[off]));
    case SPH_BF16: return static_cast<A>(bf16_to_float(static_cast<const bf16_t*>(base)[off]));
    case SPH_F32: return static_cast<A>(static_cast<const float*>(base)[off]);
    case SPH_F64: return static_cast<A>(static_cast<const double*>(base)[off]);
    case SPH_I8: return static_cast<A>(static_cast<const int8_t*>(base)[off]);
    case SPH_U8: return static_cast<A>(static_cast<const uint8_t*>(base)[off]);
    case SPH_I16: return static_cast<A>(static_cast<const int16_t*>(base)[off]);
    case SPH_I32: return static_cast<A>(static_cast<const int32_t*>(base)[off]);
    case SPH_I64: return static_cast<A>(static_cast<const int64_t*>(base)[off]);
    case SPH_BOOL: return static_cast<A>(static_cast<const uint8_t*>(base)[off] != 0);
    default: return A(0);
  }
}

template <typename A>
__device__ inline void store_val(void* base, int dt, int64_t off, A v) {
  switch (dt) {
    case SPH_F16: static_cast<half_t*>(base)[off] = static_cast<half_t>(static_cast<float>(v)); break;
    case SPH_BF16: static_cast<bf16_t*>(base)[off] = float_to_bf16(static_cast<float>(v)); break;
    case SPH_F32: static_cast<float*>(base)[off] = static_cast<float>(v); break;
    case SPH_F64: static_cast<double*>(base)[off] = static_cast<double>(v); break;
    case SPH_I8: static_cast<int8_t*>(base)[off] = static_cast<int8_t>(v); break;
    case SPH_U8: static_cast<uint8_t*>(base)[off] = static_cast<uint8_t>(v); break;
    case SPH_I16: static_cast<int16_t*>(base)[off] = static_cast<int16_t>(v); break;
    case SPH_I32: static_cast<int32_t*>(base)[off] = static_cast<int32_t>(v); break;
    case SPH_I64: static_cast<int64_t*>(base)[off] = static_cast<int64_t>(v); break;
    case SPH_BOOL: static_cast<uint8_t*>(base)[off] = (v != A(0)) ? 1 : 0; break;
    default: break;
  }
}

template <typename A>
__device__ inline bool is_nan_(A v) {
  if constexpr (__is_same(A, int64_t)) return false;
  else return v != v;
}

template <typename A>
__device__ inline Acc<A> init_acc(int op) {
  Acc<A> a;
  a.idx = -1;
  switch (op) {
    case SPH_RED_PROD: case SPH_RED_ALL: a.v = A(1); break;
    case SPH_RED_MAX: case SPH_RED_ARGMAX:
      if constexpr (__is_same(A, int64_t)) a.v = INT64_MIN; else a.v = -INFINITY;
      break;
    case SPH_RED_MIN: case SPH_RED_ARGMIN:
      if constexpr (__is_same(A, int64_t)) a.v = INT64_MAX; else a.v = INFINITY;
      break;
    default: a.v = A(0);
  }
  return a;
}

// Folds element (v, i) into acc.  For arg ops, NaN wins and ties keep the
// smaller index, as torch does.
template <typename A>
__device__ inline void fold(int op, Acc<A>& a, A v, int64_t i) {
  switch (op) {
    case SPH_RED_SUM: case SPH_RED_MEAN: a.v += v; break;
    case SPH_RED_SUMSQ: a.v += v * v; break;
    case SPH_RED_PROD: a.v *= v; break;
    case SPH_RED_ANY: a.v = (a.v != A(0) || v != A(0)) ? A(1) : A(0); break;
    case SPH_RED_ALL: a.v = (a.v != A(0) && v != A(0)) ? A(1) : A(0); break;
    case SPH_RED_MAX:
      if (is_nan_(v) || v > a.v) a.v = v;
      break;
    case SPH_RED_MIN:
      if (is_nan_(v) || v < a.v) a.v = v;
      break;
    case SPH_RED_ARGMAX: case SPH_RED_ARGMIN: {
      if (a.idx < 0) { a.v = v; a.idx = i; break; }
      if (is_nan_(a.v)) break;
      const bool better = is_nan_(v) || (op == SPH_RED_ARGMAX ? v > a.v : v < a.v);
      if (better) { a.v = v; a.idx = i; }
      break;
    }
    default: break;
  }
}

// Combines two partial accumulators (b covers later or earlier indices).
template <typename A>
__device__ inline void combine(int op, Acc<A>& a, const Acc<A>& b) {
  switch (op) {
    case SPH_RED_SUM: case SPH_RED_MEAN: case SPH_RED_SUMSQ: a.v += b.v; break;
    case SPH_RED_PROD: a.v *= b.v; break;
    case SPH_RED_ANY: a.v = (a.v != A(0) || b.v != A(0)) ? A(1) : A(0); break;
    case SPH_RED_ALL: a.v = (a.v != A(0) && b.v != A(0)) ? A(1) : A(0); break;
    case SPH_RED_MAX: if (is_nan_(b.v) || b.v > a.v) a.v = b.v; break;
    case SPH_RED_MIN: if (is_nan_(b.v) || b.v < a.v) a.v = b.v; break;
    case SPH_RED_ARGMAX: case SPH_RED_ARGMIN: {
      if (b.idx < 0) break;
      if (a.idx < 0) { a = b; break; }
      const bool an = is_nan_(a.v), bn = is_nan_(b.v);
      if (an && bn) { if (b.idx < a.idx) a = b; break; }
      if (an) break;
      if (bn) { a = b; break; }
      const bool better = (op == SPH_RED_ARGMAX) ? b.v > a.v : b.v < a.v;
      if (better || (b.v == a.v && b.idx < a.idx)) a = b;
      break;
    }
    default: break;
  }
}

template <typename A>
__device__ inline void finish(const RedArgs& p, int64_t out_off, const Acc<A>& a) {
  if (p.op == SPH_RED_ARGMAX || p.op == SPH_RED_ARGMIN) {
    static_cast<int64_t*>(p.out)[out_off] = a.idx < 0 ? 0 : a.idx;
    return;
  }
  A v = a.v;
  if (p.op == SPH_RED_MEAN) v = v / static_cast<A>(p.inner_numel);
  store_val<A>(p.out, p.out_dt, out_off, v);
}

__device__ inline void outer_offsets(const RedArgs& p, int64_t o, int64_t& in_off, int64_t& out_off) {
  in_off = 0;
  out_off = 0;
  for (int d = p.n_outer - 1; d >= 0; --d) {
    const int64_t c = o % p.outer_size[d];
    o /= p.outer_size[d];
    in_off += c * p.outer_in_stride[d];
    out_off += c * p.outer_out_stride[d];
  }
}

__device__ inline int64_t inner_offset(const RedArgs& p, int64_t i) {
  if (p.n_inner == 1) return i * p.inner_stride[0];
  int64_t off = 0;
  for (int d = p.n_inner - 1; d >= 0; --d) {
    const int64_t c = i % p.inner_size[d];
    i /= p.inner_size[d];
    off += c * p.inner_stride[d];
  }
  return off;
}

template <typename A>
__device__ inline Acc<A> shfl_acc(const Acc<A>& a, int off) {
  Acc<A> r;
  if constexpr (sizeof(A) == 8) {
    r.v = __shfl_xor(a.v, off, 64);
  } else {
    r.v = __shfl_xor(a.v, off, 64);
  }
  r.idx = __shfl_xor(a.idx, off, 64);
  return r;
}

// One wave per output; lanes stride over the reduced elements.
template <typename A>
__global__ void __launch_bounds__(256) reduce_wave(const RedArgs p) {
  const int lane = threadIdx.x & 63;
  const int64_t wave = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) >> 6;
  const int64_t nwaves = (static_cast<int64_t>(gridDim.x) * 256) >> 6;
  for (int64_t o = wave; o < p.outer_numel; o += nwaves) {
    int64_t in_off, out_off;
    outer_offsets(p, o, in_off, out_off);
    Acc<A> a = init_acc<A>(p.op);
    for (int64_t i = lane; i < p.inner_numel; i += 64) {
      const A v = load_val<A>(p.in, p.in_dt, in_off + inner_offset(p, i));
      fold<A>(p.op, a, v, i);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      Acc<A> b = shfl_acc<A>(a, off);
      combine<A>(p.op, a, b);
    }
    if (lane == 0) finish<A>(p, out_off, a);
  }
}

// One 1024-thread workgroup per output: threads stride over the reduced
// elements, waves combine with butterflies, the 16 wave results through LDS.
constexpr int kBlockRed = 1024;

template <typename A>
__global__ void __launch_bounds__(kBlockRed) reduce_block(const RedArgs p) {
  __shared__ A sv[kBlockRed / 64];
  __shared__ int64_t si[kBlockRed / 64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  for (int64_t o = blockIdx.x; o < p.outer_numel; o += gridDim.x) {
    int64_t in_off, out_off;
    outer_offsets(p, o, in_off, out_off);
    Acc<A> a = init_acc<A>(p.op);
    for (int64_t i = threadIdx.x; i < p.inner_numel; i += kBlockRed) {
      const A v = load_val<A>(p.in, p.in_dt, in_off + inner_offset(p, i));
      fold<A>(p.op, a, v, i);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      Acc<A> b = shfl_acc<A>(a, off);
      combine<A>(p.op, a, b);
    }
    if (lane == 0) {
      sv[wave] = a.v;
      si[wave] = a.idx;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      Acc<A> r{sv[0], si[0]};
      for (int w = 1; w < kBlockRed / 64; ++w) {
        Acc<A> b{sv[w], si[w]};
        combine<A>(p.op, r, b);
      }
      finish<A>(p, out_off, r);
    }
    __syncthreads();
  }
}

// One 1024-thread workgroup per output for contiguous rows of 16-bit or
// fp32 floats with the op fixed at compile time: every thread issues its
// 16-byte loads U at a time before folding them, so a long row (an LM
// head's 49155 logits) costs a few load round trips instead of one per
// element.  Elements before the row's first 16-byte boundary and after
// its last whole chunk are folded one by one.  A thread's elements come in
// increasing index order, so the fold's tie and NaN rules (first index
// wins) carry over unchanged.
template <typename T>
__device__ inline float as_f(T v) {
  if constexpr (__is_same(T, float)) return v;
  else return Num<T>::to_f(v);
}

template <typename T, int OP>
__global__ void __launch_bounds__(kBlockRed) reduce_rows_vec(const RedArgs p) {
  constexpr int VE = 16 / sizeof(T), U = 4;
  __shared__ float sv[kBlockRed / 64];
  __shared__ int64_t si[kBlockRed / 64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t n = p.inner_numel;
  for (int64_t o = blockIdx.x; o < p.outer_numel; o += gridDim.x) {
    int64_t in_off, out_off;
    outer_offsets(p, o, in_off, out_off);
    const T* row = static_cast<const T*>(p.in) + in_off;
    const int64_t mis = (reinterpret_cast<uintptr_t>(row) & 15) / sizeof(T);
    const int64_t head = mis == 0 ? 0 : (VE - mis < n ? VE - mis : n);
    const int64_t nchunks = (n - head) / VE;
    const int64_t tail0 = head + nchunks * VE;
    Acc<float> a = init_acc<float>(OP);
    if (threadIdx.x < head) fold<float>(OP, a, as_f<T>(row[threadIdx.x]), threadIdx.x);
    const u32x4* body = reinterpret_cast<const u32x4*>(row + head);
    for (int64_t c0 = threadIdx.x; c0 < nchunks; c0 += static_cast<int64_t>(kBlockRed) * U) {
      u32x4 v[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t c = c0 + static_cast<int64_t>(u) * kBlockRed;
        v[u] = body[c < nchunks ? c : c0];
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t c = c0 + static_cast<int64_t>(u) * kBlockRed;
        if (c < nchunks) {
          const T* e = reinterpret_cast<const T*>(&v[u]);
#pragma unroll
          for (int j = 0; j < VE; ++j) fold<float>(OP, a, as_f<T>(e[j]), head + c * VE + j);
        }
      }
    }
    if (tail0 + threadIdx.x < n)
      fold<float>(OP, a, as_f<T>(row[tail0 + threadIdx.x]), tail0 + threadIdx.x);
    // the head and tail elements may carry a larger index than the body's:
    // combine() orders ties by index, so the order of folding does not matter
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      Acc<float> b = shfl_acc<float>(a, off);
      combine<float>(OP, a, b);
    }
    if (lane == 0) {
      sv[wave] = a.v;
      si[wave] = a.idx;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      Acc<float> r{sv[0], si[0]};
      for (int w = 1; w < kBlockRed / 64; ++w) {
        Acc<float> b{sv[w], si[w]};
        combine<float>(OP, r, b);
      }
      finish<float>(p, out_off, r);
    }
    __syncthreads();
  }
}

template <typename T>
void launch_rows_vec(const RedArgs& p, unsigned g, hipStream_t st) {
  switch (p.op) {
    case SPH_RED_ARGMAX: reduce_rows_vec<T, SPH_RED_ARGMAX><<<g, kBlockRed, 0, st>>>(p); break;
    case SPH_RED_ARGMIN: reduce_rows_vec<T, SPH_RED_ARGMIN><<<g, kBlockRed, 0, st>>>(p); break;
    case SPH_RED_MAX: reduce_rows_vec<T, SPH_RED_MAX><<<g, kBlockRed, 0, st>>>(p); break;
    case SPH_RED_MIN: reduce_rows_vec<T, SPH_RED_MIN><<<g, kBlockRed, 0, st>>>(p); break;
    case SPH_RED_SUM: reduce_rows_vec<T, SPH_RED_SUM><<<g, kBlockRed, 0, st>>>(p); break;
    default: reduce_rows_vec<T, SPH_RED_MEAN><<<g, kBlockRed, 0, st>>>(p); break;
  }
}

// One thread per output.
template <typename A>
__global__ void __launch_bounds__(256) reduce_thread(const RedArgs p) {
  for (int64_t o = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; o < p.outer_numel;
       o += static_cast<int64_t>(gridDim.x) * 256) {
    int64_t in_off, out_off;
    outer_offsets(p, o, in_off, out_off);
    Acc<A> a = init_acc<A>(p.op);
    for (int64_t i = 0; i < p.inner_numel; ++i) {
      const A v = load_val<A>(p.in, p.in_dt, in_off + inner_offset(p, i));
      fold<A>(p.op, a, v, i);
    }
    finish<A>(p, out_off, a);
  }
}

}  // namespace
}  // namespace sph

using namespace sph;

extern "C" int sph_reduce(int op, const sph_operand* in, const sph_operand* out, int ndim,
                          const int64_t* sizes, uint32_t reduce_mask, sph_stream_t stream) {
  SPH_REQUIRE(op >= SPH_RED_SUM && op <= SPH_RED_ALL, SPH_ERR_INVALID_ARG, "reduce: bad op");
  SPH_REQUIRE(ndim >= 0 && ndim <= SPH_MAX_DIMS, SPH_ERR_INVALID_ARG, "reduce: ndim > 8");
  SPH_REQUIRE(dtype_size(in->dtype) > 0 && dtype_size(out->dtype) > 0, SPH_ERR_INVALID_ARG,
              "reduce: bad dtype");
  const bool arg = (op == SPH_RED_ARGMAX || op == SPH_RED_ARGMIN);
  SPH_REQUIRE(!arg || out->dtype == SPH_I64, SPH_ERR_INVALID_ARG, "reduce: arg ops write int64");
  RedArgs p{};
  p.in = in->data;
  p.out = out->data;
  p.in_dt = in->dtype;
  p.out_dt = out->dtype;
  p.op = op;
  p.outer_numel = 1;
  p.inner_numel = 1;
  int n_red = 0;
  for (int d = 0; d < ndim; ++d) {
    SPH_REQUIRE(sizes[d] >= 0, SPH_ERR_INVALID_ARG, "reduce: negative size");
    if (reduce_mask & (1u << d)) {
      ++n_red;
      if (sizes[d] == 1 && !arg) continue;
      p.inner_size[p.n_inner] = sizes[d];
      p.inner_stride[p.n_inner] = in->strides[d];
      p.inner_numel *= sizes[d];
      ++p.n_inner;
    } else {
      if (sizes[d] == 1) continue;
      p.outer_size[p.n_outer] = sizes[d];
      p.outer_in_stride[p.n_outer] = in->strides[d];
      p.outer_out_stride[p.n_outer] = out->strides[d];
      p.outer_numel *= sizes[d];
      ++p.n_outer;
    }
  }
  SPH_REQUIRE(!arg || n_red == 1, SPH_ERR_INVALID_ARG, "reduce: arg ops reduce exactly one dim");
  if (p.outer_numel == 0) return SPH_OK;
  SPH_REQUIRE(p.inner_numel > 0 || (op != SPH_RED_MAX && op != SPH_RED_MIN && !arg),
              SPH_ERR_INVALID_ARG, "reduce: max/min/arg over an empty dim");
  hipStream_t st = as_stream(stream);
  const bool inner_contig = p.n_inner > 0 && p.inner_stride[p.n_inner - 1] == 1 &&
                            p.inner_size[p.n_inner - 1] >= 16;
  const bool f64 = in->dtype == SPH_F64 || (out->dtype == SPH_F64 && !arg);
  const bool ints = !is_float_dtype(in->dtype) && !is_float_dtype(out->dtype) &&
                    op != SPH_RED_MEAN;
  auto grid = [](int64_t work) {
    int64_t g = (work + 255) / 256;
    if (g > 65536) g = 65536;
    return static_cast<unsigned>(g < 1 ? 1 : g);
  };
  // the vector path: one contiguous reduced dim of a 16-bit or fp32 float
  // input, an op whose fp32 accumulation matches the generic path's
  const bool vec_op = op == SPH_RED_ARGMAX || op == SPH_RED_ARGMIN || op == SPH_RED_MAX ||
                      op == SPH_RED_MIN || op == SPH_RED_SUM || op == SPH_RED_MEAN;
  const bool vec_in = in->dtype == SPH_F16 || in->dtype == SPH_BF16 || in->dtype == SPH_F32;
  const bool vec_out = arg || out->dtype == SPH_F16 || out->dtype == SPH_BF16 ||
                       out->dtype == SPH_F32;
  if (inner_contig && p.n_inner == 1 && vec_op && vec_in && vec_out &&
      p.inner_numel >= 8192 && p.outer_numel < 2048) {
    const unsigned g = static_cast<unsigned>(p.outer_numel);
    if (in->dtype == SPH_F16) launch_rows_vec<half_t>(p, g, st);
    else if (in->dtype == SPH_BF16) launch_rows_vec<bf16_t>(p, g, st);
    else launch_rows_vec<float>(p, g, st);
  } else if (inner_contig && p.inner_numel >= 8192 && p.outer_numel < 2048) {
    const unsigned g = static_cast<unsigned>(p.outer_numel < 65536 ? p.outer_numel : 65536);
    if (f64) reduce_block<double><<<g, kBlockRed, 0, st>>>(p);
    else if (ints) reduce_block<int64_t><<<g, kBlockRed, 0, st>>>(p);
    else reduce_block<float><<<g, kBlockRed, 0, st>>>(p);
  } else if (inner_contig) {
    const unsigned g = grid(p.outer_numel * 64);
    if (f64) reduce_wave<double><<<g, 256, 0, st>>>(p);
    else if (ints) reduce_wave<int64_t><<<g, 256, 0, st>>>(p);
    else reduce_wave<float><<<g, 256, 0, st>>>(p);
  } else {
    const unsigned g = grid(p.outer_numel);
    if (f64) reduce_thread<double><<<g, 256, 0, st>>>(p);
    else if (ints) reduce_thread<int64_t><<<g, 256, 0, st>>>(p);
    else reduce_thread<float><<<g, 256, 0, st>>>(p);
  }
  return check_launch("sph_reduce");
}
