// Shared device/host helpers of the gfx950 kernel library.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cmath>
#include <string>

#include "spyre_hip.h"

namespace sph {

// ---------------------------------------------------------------------------
// Error handling (host)
// ---------------------------------------------------------------------------

// Records a message for sph_last_error() and returns `code`.
int set_error(int code, const std::string& msg);

// Returns 0 after a successful launch, else records the HIP error.
int check_launch(const char* what);

#define SPH_REQUIRE(cond, code, msg)                 \
  do {                                               \
    if (!(cond)) return ::sph::set_error((code), (msg)); \
  } while (0)

inline hipStream_t as_stream(sph_stream_t s) {
  return reinterpret_cast<hipStream_t>(s);
}

inline int dtype_size(int dt) {
  switch (dt) {
    case SPH_F16:
    case SPH_BF16:
    case SPH_I16:
      return 2;
    case SPH_F32:
    case SPH_I32:
      return 4;
    case SPH_F64:
    case SPH_I64:
      return 8;
    case SPH_I8:
    case SPH_U8:
    case SPH_BOOL:
      return 1;
    default:
      return 0;
  }
}

inline bool is_float_dtype(int dt) {
  return dt == SPH_F16 || dt == SPH_BF16 || dt == SPH_F32 || dt == SPH_F64;
}

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// ---------------------------------------------------------------------------
// Scalar types
// ---------------------------------------------------------------------------

typedef _Float16 half_t;

// bfloat16 stored as raw bits; conversions written out so the rounding is
// explicit (round to nearest even, NaN kept quiet).
struct bf16_t {
  uint16_t bits;
};

__device__ __host__ inline float bf16_to_float(bf16_t v) {
  uint32_t u = static_cast<uint32_t>(v.bits) << 16;
  float f;
  __builtin_memcpy(&f, &u, 4);
  return f;
}

__device__ __host__ inline bf16_t float_to_bf16(float f) {
  uint32_t u;
  __builtin_memcpy(&u, &f, 4);
  bf16_t r;
  if ((u & 0x7fffffffu) > 0x7f800000u) {  // NaN
    r.bits = static_cast<uint16_t>((u >> 16) | 0x0040u);
    return r;
  }
  uint32_t lsb = (u >> 16) & 1u;
  u += 0x7fffu + lsb;
  r.bits = static_cast<uint16_t>(u >> 16);
  return r;
}

template <typename T>
struct Num;

template <>
struct Num<half_t> {
  __device__ static inline float to_f(half_t v) { return static_cast<float>(v); }
  __device__ static inline half_t from_f(float v) { return static_cast<half_t>(v); }
};
template <>
struct Num<bf16_t> {
  __device__ static inline float to_f(bf16_t v) { return bf16_to_float(v); }
  __device__ static inline bf16_t from_f(float v) { return float_to_bf16(v); }
};
template <>
struct Num<float> {
  __device__ static inline float to_f(float v) { return v; }
  __device__ static inline float from_f(float v) { return v; }
};

// 16-byte vector of 8 two-byte values / 4 floats.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Loads 8 consecutive elements starting at p (p must be 16-byte aligned for
// 2-byte types, 32-byte-aligned pairs of 16-byte loads for float).
template <typename T>
__device__ inline void load8(const T* __restrict__ p, float (&v)[8]) {
  if constexpr (sizeof(T) == 2) {
    u32x4 raw = *reinterpret_cast<const u32x4*>(p);
    const T* e = reinterpret_cast<const T*>(&raw);
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = Num<T>::to_f(e[i]);
  } else {
    u32x4 r0 = *reinterpret_cast<const u32x4*>(p);
    u32x4 r1 = *reinterpret_cast<const u32x4*>(p + 4);
    const float* e0 = reinterpret_cast<const float*>(&r0);
    const float* e1 = reinterpret_cast<const float*>(&r1);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[i] = e0[i];
      v[i + 4] = e1[i];
    }
  }
}

// NT: a streaming (non-temporal) store, for outputs written once and not
// read back soon (the large row-kernel outputs: 3-5 % faster there).
template <typename T, bool NT = false>
__device__ inline void store8(T* __restrict__ p, const float (&v)[8]) {
  if constexpr (sizeof(T) == 2) {
    u32x4 raw;
    T* e = reinterpret_cast<T*>(&raw);
#pragma unroll
    for (int i = 0; i < 8; ++i) e[i] = Num<T>::from_f(v[i]);
    if constexpr (NT)
      __builtin_nontemporal_store(raw, reinterpret_cast<u32x4*>(p));
    else
      *reinterpret_cast<u32x4*>(p) = raw;
  } else {
    u32x4 r0, r1;
    float* e0 = reinterpret_cast<float*>(&r0);
    float* e1 = reinterpret_cast<float*>(&r1);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      e0[i] = v[i];
      e1[i] = v[i + 4];
    }
    *reinterpret_cast<u32x4*>(p) = r0;
    *reinterpret_cast<u32x4*>(p + 4) = r1;
  }
}

// Loads up to 8 elements [p, p+n) (n <= 8) element by element; the rest get
// `fill`.
template <typename T>
__device__ inline void load8_partial(const T* __restrict__ p, int n,
                                     float fill, float (&v)[8]) {
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = (i < n) ? Num<T>::to_f(p[i]) : fill;
}

template <typename T>
__device__ inline void store8_partial(T* __restrict__ p, int n,
                                      const float (&v)[8]) {
#pragma unroll
  for (int i = 0; i < 8; ++i)
    if (i < n) p[i] = Num<T>::from_f(v[i]);
}

// ---------------------------------------------------------------------------
// Wave64 / workgroup reductions
// ---------------------------------------------------------------------------

constexpr int kWave = 64;

struct SumOp {
  __device__ static inline float apply(float a, float b) { return a + b; }
};
struct MaxOp {
  __device__ static inline float apply(float a, float b) { return fmaxf(a, b); }
};

// Butterfly reduction over aligned groups of `Width` lanes (Width <= 64).
template <typename Op, int Width = kWave>
__device__ inline float wave_reduce(float v) {
#pragma unroll
  for (int off = Width / 2; off > 0; off >>= 1) v = Op::apply(v, __shfl_xor(v, off, Width));
  return v;
}

// Reduction over the `Threads` threads of a row group (Threads a multiple of
// 64, group = consecutive threads starting at a multiple of Threads).  `lds`
// must hold blockDim/64 floats; the call contains two barriers, so every
// thread of the workgroup must reach it.
template <typename Op, int Threads>
__device__ inline float group_reduce(float v, float* lds) {
  v = wave_reduce<Op>(v);
  if constexpr (Threads == kWave) {
    return v;
  } else {
    const int wave = threadIdx.x / kWave;
    const int lane = threadIdx.x % kWave;
    if (lane == 0) lds[wave] = v;
    __syncthreads();
    const int first = (wave / (Threads / kWave)) * (Threads / kWave);
    float r = lds[first];
#pragma unroll
    for (int i = 1; i < Threads / kWave; ++i) r = Op::apply(r, lds[first + i]);
    __syncthreads();
    return r;
  }
}

// Numerics shared by the kernels.
// erfc(a) for a >= 0 by Abramowitz & Stegun, Handbook of Mathematical
// Functions, 7.1.26: erfc(a) = t (a1 + t (a2 + t (a3 + t (a4 + t a5))))
// exp(-a^2) with t = 1 / (1 + p a); its error in erf is at most 1.5e-7.
// Two transcendental instructions (v_rcp_f32, v_exp_f32) and a few FMAs,
// against the dozens of instructions and branches of a full-precision erff.
constexpr float kAsP = 0.3275911f, kAsA1 = 0.254829592f, kAsA2 = -0.284496736f,
                kAsA3 = 1.421413741f, kAsA4 = -1.453152027f, kAsA5 = 1.061405429f;
__device__ inline float erfc_as(float a) {
  const float t = __builtin_amdgcn_rcpf(fmaf(kAsP, a, 1.0f));
  float q = fmaf(kAsA5, t, kAsA4);
  q = fmaf(q, t, kAsA3);
  q = fmaf(q, t, kAsA2);
  q = fmaf(q, t, kAsA1);
  return q * t * __builtin_amdgcn_exp2f(-a * a * 1.4426950408889634f);
}
// GELU in the exact (erf) form, gelu(x) = x Phi(x) = x (1 + erf(x / sqrt2)) / 2,
// rewritten as max(x, 0) - |x| h with h = erfc(|x| / sqrt2) / 2, the upper
// Gaussian tail Q(|x|) (the negative tail then needs no cancellation).
// log2 Q(a) is smooth, so h = 2^p(a) on [0, 9) with p the degree-6
// polynomial fit to log2 Q there by iteratively reweighted least squares
// (float64, 400001 points, Chebyshev basis, weights driving the absolute
// error of a Q toward equal ripple; converted to monomials, rounded to
// float32); from 9 on, Q < 1.2e-19 and h is taken as 0 (so +-inf and NaN
// give NaN, as torch's CPU gelu does).  One exp2, six FMAs, a min, a
// compare-select and a max per element.  Absolute error of gelu below 1e-6
// for every finite x (float32 evaluation against float64 erfc; the fit
// itself 7.4e-8).
__device__ inline float gelu_erf(float x) {
  const float ax = fabsf(x);
  const float a = fminf(ax, 9.0f);
  float p = fmaf(3.30928342e-05f, a, -0.000769219827f);
  p = fmaf(p, a, 0.00808071718f);
  p = fmaf(p, a, -0.0534121059f);
  p = fmaf(p, a, -0.458770961f);
  p = fmaf(p, a, -1.15120173f);
  p = fmaf(p, a, -0.999993086f);
  const float h = ax < 9.0f ? __builtin_amdgcn_exp2f(p) : 0.f;
  return fmaf(-ax, h, fmaxf(x, 0.f));
}
__device__ inline float gelu_tanh(float x) {
  const float k = 0.79788456080286535588f;  // sqrt(2/pi)
  return 0.5f * x * (1.0f + tanhf(k * (x + 0.044715f * x * x * x)));
}
__device__ inline float sigmoidf_(float x) { return 1.0f / (1.0f + expf(-x)); }
__device__ inline float silu(float x) { return x / (1.0f + expf(-x)); }

}  // namespace sph
