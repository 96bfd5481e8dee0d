// Generated and scanned fills on the device: arange, cumsum, the random
// fills (uniform_, normal_, random_) and dropout.
//
// Reference: the reference runs cumsum on the CPU and copies the result
// (codegen/inputs/spyre_torch_ops.cpp:502-505); its random fills and arange
// take the CPU path as well, and its native_dropout is an identity stub
// (:180-186).  Here every one of them runs on the GPU.
//
// Random numbers: Philox4x32-10 (Salmon, Moraes, Dror and Shaw, "Parallel
// random numbers: as easy as 1, 2, 3", SC'11), a counter-based generator:
// block j of a fill is the 4 x 32-bit output for counter (lo(offset + j),
// hi(offset + j), 0, 0) and key (lo(seed), hi(seed)).  Element i of a fill
// of 32-bit draws takes word i % 4 of block i / 4; a fill of 64-bit draws
// (float64 values, integer ranges above 2^32) takes words 2(i % 2) and
// 2(i % 2) + 1 of block i / 2 as one 64-bit number (first word high).  So a
// fill's values depend only on (seed, offset, n, kind, dtype, parameters),
// not on the launch shape, and a host restatement reproduces them.
#include <type_traits>

#include "sph_common.h"

namespace sph {
namespace {

constexpr uint32_t kPhiloxM0 = 0xD2511F53u, kPhiloxM1 = 0xCD9E8D57u;  // round multipliers
constexpr uint32_t kPhiloxW0 = 0x9E3779B9u, kPhiloxW1 = 0xBB67AE85u;  // key increments

struct Words {
  uint32_t w[4];
};

// Ten rounds of Philox4x32 on counter (c0, c1, c2, c3) under key (k0, k1):
// each round multiplies c0 and c2 by the round multipliers, and the new
// counter is (hi(M1 c2) ^ c1 ^ k0, lo(M1 c2), hi(M0 c0) ^ c3 ^ k1, lo(M0 c0));
// the key advances by the Weyl increments between rounds.
__device__ inline Words philox10(uint64_t ctr, uint32_t k0, uint32_t k1) {
  uint32_t c0 = static_cast<uint32_t>(ctr), c1 = static_cast<uint32_t>(ctr >> 32), c2 = 0, c3 = 0;
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    const uint32_t lo0 = kPhiloxM0 * c0, hi0 = __umulhi(kPhiloxM0, c0);
    const uint32_t lo1 = kPhiloxM1 * c2, hi1 = __umulhi(kPhiloxM1, c2);
    c0 = hi1 ^ c1 ^ k0;
    c1 = lo1;
    c2 = hi0 ^ c3 ^ k1;
    c3 = lo0;
    k0 += kPhiloxW0;
    k1 += kPhiloxW1;
  }
  return {{c0, c1, c2, c3}};
}

// [0, 1) from the top 24 bits of a word / the top 53 bits of a 64-bit draw.
__device__ inline float unit_f(uint32_t w) { return static_cast<float>(w >> 8) * 0x1p-24f; }
__device__ inline double unit_d(uint64_t w) { return static_cast<double>(w >> 11) * 0x1p-53; }

template <typename T>
struct Put;
template <>
struct Put<half_t> {
  __device__ static void f(half_t* p, float v) { *p = static_cast<half_t>(v); }
  __device__ static float back(float v) { return static_cast<float>(static_cast<half_t>(v)); }
};
template <>
struct Put<bf16_t> {
  __device__ static void f(bf16_t* p, float v) { *p = float_to_bf16(v); }
  __device__ static float back(float v) { return bf16_to_float(float_to_bf16(v)); }
};
template <>
struct Put<float> {
  __device__ static void f(float* p, float v) { *p = v; }
  __device__ static float back(float v) { return v; }
};

constexpr int kFillBlock = 256;

inline unsigned fill_grid(int64_t units) {
  const int64_t g = ceil_div(units, kFillBlock);
  return static_cast<unsigned>(g < 65536 ? g : 65536);
}

// ---- uniform_ / normal_ on 2- and 4-byte floats (32-bit draws) ------------
// kind 0: from + u (to - from), u in [0, 1), a value that rounds up to `to`
// in the output type is replaced by `from` (the range stays half-open);
// kind 1: mean + std * n, n standard normal by Box-Muller on word pairs
// (u1 in (0, 1] from the first word, u2 in [0, 1) from the second):
// r = sqrt(-2 ln u1), n = r cos(2 pi u2) and r sin(2 pi u2).
template <typename T>
__global__ void __launch_bounds__(kFillBlock)
rng_f32_kernel(T* __restrict__ out, int64_t n, uint32_t k0, uint32_t k1, uint64_t offset,
               int kind, float a, float b) {
  const int64_t blocks = (n + 3) / 4;
  for (int64_t j = static_cast<int64_t>(blockIdx.x) * kFillBlock + threadIdx.x; j < blocks;
       j += static_cast<int64_t>(gridDim.x) * kFillBlock) {
    const Words r = philox10(offset + static_cast<uint64_t>(j), k0, k1);
    float v[4];
    if (kind == 0) {
      const float range = __fsub_rn(b, a);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float x = __fadd_rn(__fmul_rn(unit_f(r.w[e]), range), a);
        v[e] = Put<T>::back(x) >= b ? a : x;
      }
    } else {
#pragma unroll
      for (int e = 0; e < 4; e += 2) {
        const float u1 = static_cast<float>((r.w[e] >> 8) + 1u) * 0x1p-24f;
        const float u2 = unit_f(r.w[e + 1]);
        const float rad = sqrtf(-2.0f * logf(u1));
        float sn, cs;
        sincosf(6.283185307179586f * u2, &sn, &cs);
        v[e] = __fadd_rn(__fmul_rn(rad * cs, b), a);
        v[e + 1] = __fadd_rn(__fmul_rn(rad * sn, b), a);
      }
    }
    const int64_t i0 = j * 4;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (i0 + e < n) Put<T>::f(out + i0 + e, v[e]);
  }
}

// ---- uniform_ / normal_ on float64 (64-bit draws) ---------------------------
__global__ void __launch_bounds__(kFillBlock)
rng_f64_kernel(double* __restrict__ out, int64_t n, uint32_t k0, uint32_t k1, uint64_t offset,
               int kind, double a, double b) {
  const int64_t blocks = (n + 1) / 2;
  for (int64_t j = static_cast<int64_t>(blockIdx.x) * kFillBlock + threadIdx.x; j < blocks;
       j += static_cast<int64_t>(gridDim.x) * kFillBlock) {
    const Words r = philox10(offset + static_cast<uint64_t>(j), k0, k1);
    const uint64_t d0 = (static_cast<uint64_t>(r.w[0]) << 32) | r.w[1];
    const uint64_t d1 = (static_cast<uint64_t>(r.w[2]) << 32) | r.w[3];
    double v[2];
    if (kind == 0) {
      const double range = __dsub_rn(b, a);
      const double x0 = __dadd_rn(__dmul_rn(unit_d(d0), range), a);
      const double x1 = __dadd_rn(__dmul_rn(unit_d(d1), range), a);
      v[0] = x0 >= b ? a : x0;
      v[1] = x1 >= b ? a : x1;
    } else {
      const double u1 = static_cast<double>((d0 >> 11) + 1u) * 0x1p-53;
      const double u2 = unit_d(d1);
      const double rad = sqrt(-2.0 * log(u1));
      double sn, cs;
      sincos(6.283185307179586 * u2, &sn, &cs);
      v[0] = __dadd_rn(__dmul_rn(rad * cs, b), a);
      v[1] = __dadd_rn(__dmul_rn(rad * sn, b), a);
    }
    const int64_t i0 = j * 2;
    out[i0] = v[0];
    if (i0 + 1 < n) out[i0 + 1] = v[1];
  }
}

// ---- random_(from, to): from + draw % range --------------------------------
template <typename T, bool WIDE>
__global__ void __launch_bounds__(kFillBlock)
rng_int_kernel(T* __restrict__ out, int64_t n, uint32_t k0, uint32_t k1, uint64_t offset,
               int64_t from, uint64_t range) {
  constexpr int EPB = WIDE ? 2 : 4;
  const int64_t blocks = (n + EPB - 1) / EPB;
  for (int64_t j = static_cast<int64_t>(blockIdx.x) * kFillBlock + threadIdx.x; j < blocks;
       j += static_cast<int64_t>(gridDim.x) * kFillBlock) {
    const Words r = philox10(offset + static_cast<uint64_t>(j), k0, k1);
    const int64_t i0 = j * EPB;
#pragma unroll
    for (int e = 0; e < EPB; ++e) {
      if (i0 + e >= n) break;
      const uint64_t d = WIDE ? ((static_cast<uint64_t>(r.w[2 * e]) << 32) | r.w[2 * e + 1])
                              : static_cast<uint64_t>(r.w[e]);
      const int64_t val = static_cast<int64_t>(static_cast<uint64_t>(from) + d % range);
      if constexpr (std::is_same<T, half_t>::value || std::is_same<T, float>::value ||
                    std::is_same<T, double>::value)
        out[i0 + e] = static_cast<T>(static_cast<double>(val));
      else if constexpr (std::is_same<T, bf16_t>::value)
        out[i0 + e] = float_to_bf16(static_cast<float>(val));
      else
        out[i0 + e] = static_cast<T>(val);
    }
  }
}

// ---- dropout: keep with probability 1 - p (u >= p), kept values x * scale --
template <typename T>
__global__ void __launch_bounds__(kFillBlock)
dropout_kernel(const T* __restrict__ x, T* __restrict__ y, uint8_t* __restrict__ mask, int64_t n,
               float p, float scale, uint32_t k0, uint32_t k1, uint64_t offset) {
  const int64_t blocks = (n + 3) / 4;
  for (int64_t j = static_cast<int64_t>(blockIdx.x) * kFillBlock + threadIdx.x; j < blocks;
       j += static_cast<int64_t>(gridDim.x) * kFillBlock) {
    const Words r = philox10(offset + static_cast<uint64_t>(j), k0, k1);
    const int64_t i0 = j * 4;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if (i0 + e >= n) break;
      const bool keep = unit_f(r.w[e]) >= p;
      mask[i0 + e] = keep ? 1 : 0;
      Put<T>::f(y + i0 + e, keep ? Num<T>::to_f(x[i0 + e]) * scale : 0.0f);
    }
  }
}

// ---- arange: start + step * i in the accumulation type of the output -------
template <typename T, typename ACC>
__global__ void __launch_bounds__(kFillBlock)
arange_kernel(T* __restrict__ out, int64_t n, ACC start, ACC step) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kFillBlock + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * kFillBlock) {
    if constexpr (std::is_same<ACC, double>::value)
      out[i] = static_cast<T>(__dadd_rn(start, __dmul_rn(step, static_cast<double>(i))));
    else if constexpr (std::is_same<ACC, float>::value)
      Put<T>::f(out + i, __fadd_rn(start, __fmul_rn(step, static_cast<float>(i))));
    else
      out[i] = static_cast<T>(start + step * i);
  }
}

// ---- cumsum ----------------------------------------------------------------
// Sequential per column of a contiguous [outer, len, inner] tensor: thread
// (o, c) walks l = 0..len-1 accumulating in ACC, the order of torch's CPU
// kernel (so results are bit-identical to it); columns are adjacent across
// threads, so for inner >= 64 every load is one coalesced run.
template <typename T, typename ACC>
__global__ void __launch_bounds__(kFillBlock)
cumsum_cols_kernel(const T* __restrict__ x, T* __restrict__ y, int64_t outer, int64_t len,
                   int64_t inner) {
  const int64_t cols = outer * inner;
  for (int64_t c = static_cast<int64_t>(blockIdx.x) * kFillBlock + threadIdx.x; c < cols;
       c += static_cast<int64_t>(gridDim.x) * kFillBlock) {
    const int64_t o = c / inner, ci = c % inner;
    const T* xs = x + o * len * inner + ci;
    T* ys = y + o * len * inner + ci;
    ACC acc = 0;
    for (int64_t l = 0; l < len; ++l) {
      if constexpr (std::is_same<T, half_t>::value || std::is_same<T, bf16_t>::value) {
        acc += Num<T>::to_f(xs[l * inner]);
        Put<T>::f(ys + l * inner, acc);
      } else {
        acc += static_cast<ACC>(xs[l * inner]);
        ys[l * inner] = static_cast<T>(acc);
      }
    }
  }
}

template <typename ACC>
__device__ inline ACC shfl_up_acc(ACC v, int d) {
  if constexpr (sizeof(ACC) == 8) {
    int64_t b;
    __builtin_memcpy(&b, &v, 8);
    const int lo = __shfl_up(static_cast<int>(b), d, 64);
    const int hi = __shfl_up(static_cast<int>(b >> 32), d, 64);
    const int64_t r = (static_cast<int64_t>(hi) << 32) | static_cast<uint32_t>(lo);
    ACC out;
    __builtin_memcpy(&out, &r, 8);
    return out;
  } else {
    return __shfl_up(v, d, 64);
  }
}

// One 1024-thread workgroup per row (inner == 1, few long rows): tiles of
// 8192 elements, 8 consecutive per thread scanned in registers, the thread
// totals scanned across the workgroup (wave scans + one LDS pass over the
// 16 wave totals), a carry across tiles.  Sums associate differently from a
// sequential pass: integers are exact, floats differ by rounding only.
template <typename T, typename ACC>
__global__ void __launch_bounds__(1024)
cumsum_rows_kernel(const T* __restrict__ x, T* __restrict__ y, int64_t len) {
  __shared__ ACC wsum[16];
  __shared__ ACC carry_s;
  const T* xr = x + static_cast<int64_t>(blockIdx.x) * len;
  T* yr = y + static_cast<int64_t>(blockIdx.x) * len;
  const int lane = threadIdx.x % 64, wave = threadIdx.x / 64;
  if (threadIdx.x == 0) carry_s = 0;
  __syncthreads();
  for (int64_t base = 0; base < len; base += 8192) {
    const int64_t c0 = base + threadIdx.x * 8;
    ACC v[8];
    ACC run = 0;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      ACC a = 0;
      if (c0 + e < len) {
        if constexpr (std::is_same<T, half_t>::value || std::is_same<T, bf16_t>::value)
          a = Num<T>::to_f(xr[c0 + e]);
        else
          a = static_cast<ACC>(xr[c0 + e]);
      }
      run += a;
      v[e] = run;
    }
    // inclusive scan of the thread totals within the wave
    ACC t = run;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const ACC o = shfl_up_acc(t, d);
      if (lane >= d) t += o;
    }
    if (lane == 63) wsum[wave] = t;
    __syncthreads();
    ACC before = carry_s;
    for (int w = 0; w < wave; ++w) before += wsum[w];
    const ACC excl = before + t - run;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      if (c0 + e < len) {
        if constexpr (std::is_same<T, half_t>::value || std::is_same<T, bf16_t>::value)
          Put<T>::f(yr + c0 + e, excl + v[e]);
        else
          yr[c0 + e] = static_cast<T>(excl + v[e]);
      }
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      ACC tot = carry_s;
      for (int w = 0; w < 16; ++w) tot += wsum[w];
      carry_s = tot;
    }
    __syncthreads();
  }
}

template <typename T, typename ACC>
void launch_cumsum(const void* x, void* y, int64_t outer, int64_t len, int64_t inner,
                   hipStream_t st) {
  const T* xi = static_cast<const T*>(x);
  T* yo = static_cast<T*>(y);
  // columns, or rows short enough to walk one per thread: the sequential
  // kernel; long rows of the last dimension: a workgroup per row
  if (inner > 1 || len <= 8192 || outer > 0x7fffffffLL)
    cumsum_cols_kernel<T, ACC><<<fill_grid(outer * inner), kFillBlock, 0, st>>>(xi, yo, outer, len,
                                                                               inner);
  else
    cumsum_rows_kernel<T, ACC><<<static_cast<unsigned>(outer), 1024, 0, st>>>(xi, yo, len);
}

}  // namespace
}  // namespace sph

using namespace sph;

extern "C" int64_t sph_random_blocks(int kind, sph_dtype dtype, int64_t n, uint64_t irange) {
  if (n <= 0) return 0;
  const bool wide = (kind == SPH_RNG_INT) ? irange > 0xffffffffull : dtype == SPH_F64;
  return wide ? (n + 1) / 2 : (n + 3) / 4;
}

extern "C" int sph_random_fill(int kind, sph_dtype dtype, void* out, int64_t n, uint64_t seed,
                               uint64_t offset, double a, double b, int64_t ifrom,
                               uint64_t irange, sph_stream_t stream) {
  SPH_REQUIRE(n >= 0, SPH_ERR_INVALID_ARG, "random_fill: negative size");
  SPH_REQUIRE(kind == SPH_RNG_UNIFORM || kind == SPH_RNG_NORMAL || kind == SPH_RNG_INT,
              SPH_ERR_INVALID_ARG, "random_fill: unknown kind");
  if (n == 0) return SPH_OK;
  SPH_REQUIRE(out != nullptr, SPH_ERR_INVALID_ARG, "random_fill: null output");
  hipStream_t st = as_stream(stream);
  const uint32_t k0 = static_cast<uint32_t>(seed), k1 = static_cast<uint32_t>(seed >> 32);
  const int64_t blocks = sph_random_blocks(kind, dtype, n, irange);
  const unsigned g = fill_grid(blocks);
  if (kind == SPH_RNG_INT) {
    SPH_REQUIRE(irange > 0, SPH_ERR_INVALID_ARG, "random_fill: empty integer range");
    const bool wide = irange > 0xffffffffull;
#define SPH_RINT(T_)                                                                        \
  (wide ? (rng_int_kernel<T_, true><<<g, kFillBlock, 0, st>>>(static_cast<T_*>(out), n, k0, k1, \
                                                             offset, ifrom, irange), 0)       \
        : (rng_int_kernel<T_, false><<<g, kFillBlock, 0, st>>>(static_cast<T_*>(out), n, k0, k1, \
                                                              offset, ifrom, irange), 0))
    switch (dtype) {
      case SPH_F16: SPH_RINT(half_t); break;
      case SPH_BF16: SPH_RINT(bf16_t); break;
      case SPH_F32: SPH_RINT(float); break;
      case SPH_F64: SPH_RINT(double); break;
      case SPH_I8: SPH_RINT(int8_t); break;
      case SPH_U8: SPH_RINT(uint8_t); break;
      case SPH_I16: SPH_RINT(int16_t); break;
      case SPH_I32: SPH_RINT(int32_t); break;
      case SPH_I64: SPH_RINT(int64_t); break;
      case SPH_BOOL: SPH_RINT(uint8_t); break;
      default: return set_error(SPH_ERR_UNSUPPORTED, "random_fill: dtype");
    }
#undef SPH_RINT
    return check_launch("sph_random_fill");
  }
  SPH_REQUIRE(std::isfinite(a) && std::isfinite(b), SPH_ERR_INVALID_ARG,
              "random_fill: non-finite parameter");
  switch (dtype) {
    case SPH_F16:
      rng_f32_kernel<half_t><<<g, kFillBlock, 0, st>>>(static_cast<half_t*>(out), n, k0, k1, offset,
                                                        kind, static_cast<float>(a),
                                                        static_cast<float>(b));
      break;
    case SPH_BF16:
      rng_f32_kernel<bf16_t><<<g, kFillBlock, 0, st>>>(static_cast<bf16_t*>(out), n, k0, k1, offset,
                                                        kind, static_cast<float>(a),
                                                        static_cast<float>(b));
      break;
    case SPH_F32:
      rng_f32_kernel<float><<<g, kFillBlock, 0, st>>>(static_cast<float*>(out), n, k0, k1, offset,
                                                       kind, static_cast<float>(a),
                                                       static_cast<float>(b));
      break;
    case SPH_F64:
      rng_f64_kernel<<<g, kFillBlock, 0, st>>>(static_cast<double*>(out), n, k0, k1, offset, kind,
                                               a, b);
      break;
    default:
      return set_error(SPH_ERR_UNSUPPORTED, "random_fill: uniform / normal need a float dtype");
  }
  return check_launch("sph_random_fill");
}

extern "C" int sph_dropout(sph_dtype dtype, const void* x, void* y, uint8_t* mask, int64_t n,
                           float p, float scale, uint64_t seed, uint64_t offset,
                           sph_stream_t stream) {
  SPH_REQUIRE(n >= 0, SPH_ERR_INVALID_ARG, "dropout: negative size");
  SPH_REQUIRE(p >= 0.f && p <= 1.f, SPH_ERR_INVALID_ARG, "dropout: p outside [0, 1]");
  if (n == 0) return SPH_OK;
  hipStream_t st = as_stream(stream);
  const uint32_t k0 = static_cast<uint32_t>(seed), k1 = static_cast<uint32_t>(seed >> 32);
  const unsigned g = fill_grid((n + 3) / 4);
  switch (dtype) {
    case SPH_F16:
      dropout_kernel<half_t><<<g, kFillBlock, 0, st>>>(static_cast<const half_t*>(x),
                                                        static_cast<half_t*>(y), mask, n, p, scale,
                                                        k0, k1, offset);
      break;
    case SPH_BF16:
      dropout_kernel<bf16_t><<<g, kFillBlock, 0, st>>>(static_cast<const bf16_t*>(x),
                                                        static_cast<bf16_t*>(y), mask, n, p, scale,
                                                        k0, k1, offset);
      break;
    case SPH_F32:
      dropout_kernel<float><<<g, kFillBlock, 0, st>>>(static_cast<const float*>(x),
                                                       static_cast<float*>(y), mask, n, p, scale,
                                                       k0, k1, offset);
      break;
    default:
      return set_error(SPH_ERR_UNSUPPORTED, "dropout: dtype must be F16, BF16 or F32");
  }
  return check_launch("sph_dropout");
}

extern "C" int sph_arange(sph_dtype dtype, double start, double step, int64_t istart,
                          int64_t istep, int64_t n, void* out, sph_stream_t stream) {
  SPH_REQUIRE(n >= 0, SPH_ERR_INVALID_ARG, "arange: negative size");
  if (n == 0) return SPH_OK;
  hipStream_t st = as_stream(stream);
  const unsigned g = fill_grid(n);
  switch (dtype) {
    case SPH_F16:
      arange_kernel<half_t, float><<<g, kFillBlock, 0, st>>>(static_cast<half_t*>(out), n,
                                                               static_cast<float>(start),
                                                               static_cast<float>(step));
      break;
    case SPH_BF16:
      arange_kernel<bf16_t, float><<<g, kFillBlock, 0, st>>>(static_cast<bf16_t*>(out), n,
                                                               static_cast<float>(start),
                                                               static_cast<float>(step));
      break;
    case SPH_F32:
      arange_kernel<float, double><<<g, kFillBlock, 0, st>>>(static_cast<float*>(out), n, start,
                                                              step);
      break;
    case SPH_F64:
      arange_kernel<double, double><<<g, kFillBlock, 0, st>>>(static_cast<double*>(out), n, start,
                                                               step);
      break;
    case SPH_I8:
      arange_kernel<int8_t, int64_t><<<g, kFillBlock, 0, st>>>(static_cast<int8_t*>(out), n,
                                                                istart, istep);
      break;
    case SPH_U8:
      arange_kernel<uint8_t, int64_t><<<g, kFillBlock, 0, st>>>(static_cast<uint8_t*>(out), n,
                                                                 istart, istep);
      break;
    case SPH_I16:
      arange_kernel<int16_t, int64_t><<<g, kFillBlock, 0, st>>>(static_cast<int16_t*>(out), n,
                                                                 istart, istep);
      break;
    case SPH_I32:
      arange_kernel<int32_t, int64_t><<<g, kFillBlock, 0, st>>>(static_cast<int32_t*>(out), n,
                                                                 istart, istep);
      break;
    case SPH_I64:
      arange_kernel<int64_t, int64_t><<<g, kFillBlock, 0, st>>>(static_cast<int64_t*>(out), n,
                                                                 istart, istep);
      break;
    default:
      return set_error(SPH_ERR_UNSUPPORTED, "arange: dtype");
  }
  return check_launch("sph_arange");
}

extern "C" int sph_cumsum(sph_dtype dtype, const void* x, void* y, int64_t outer, int64_t len,
                          int64_t inner, sph_stream_t stream) {
  SPH_REQUIRE(outer >= 0 && len >= 0 && inner >= 0, SPH_ERR_INVALID_ARG, "cumsum: negative size");
  if (outer == 0 || len == 0 || inner == 0) return SPH_OK;
  hipStream_t st = as_stream(stream);
  switch (dtype) {
    case SPH_F16: launch_cumsum<half_t, float>(x, y, outer, len, inner, st); break;
    case SPH_BF16: launch_cumsum<bf16_t, float>(x, y, outer, len, inner, st); break;
    case SPH_F32: launch_cumsum<float, double>(x, y, outer, len, inner, st); break;
    case SPH_F64: launch_cumsum<double, double>(x, y, outer, len, inner, st); break;
    case SPH_I8: launch_cumsum<int8_t, int64_t>(x, y, outer, len, inner, st); break;
    case SPH_U8: launch_cumsum<uint8_t, int64_t>(x, y, outer, len, inner, st); break;
    case SPH_I16: launch_cumsum<int16_t, int64_t>(x, y, outer, len, inner, st); break;
    case SPH_I32: launch_cumsum<int32_t, int64_t>(x, y, outer, len, inner, st); break;
    case SPH_I64: launch_cumsum<int64_t, int64_t>(x, y, outer, len, inner, st); break;
    default: return set_error(SPH_ERR_UNSUPPORTED, "cumsum: dtype");
  }
  return check_launch("sph_cumsum");
}
