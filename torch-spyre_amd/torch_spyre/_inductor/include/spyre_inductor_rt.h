// Device runtime of the kernels the spyre Inductor backend generates
// (compiled with hiprtc for gfx950 at torch.compile time).
//
// Generated kernels are one of two hand-written templates, instantiated with
// the fused loop body Inductor produced:
//   * pointwise: one thread per output element, 1-D grid over xnumel;
//   * row reduction: one workgroup per output row; the threads stride over
//     the reduction index (coalesced), accumulate in fp32, and combine with
//     the wave64 / LDS block reductions below.  Several reductions of the
//     same row run in sequence inside one kernel (softmax, norms).
// All arithmetic is fp32 (fp16 / bf16 values are widened on load and
// rounded once on store), like torch's CPU kernels.
#pragma once

typedef long long int64_t;
typedef int int32_t;
typedef unsigned int uint32_t;
typedef unsigned short uint16_t;
typedef signed char int8_t;
typedef unsigned char uint8_t;

struct bfloat16 {
  uint16_t bits;
};

namespace spy {

constexpr int kWave = 64;

// ---- conversions ----------------------------------------------------------
__device__ inline float to_f(float v) { return v; }
__device__ inline float to_f(_Float16 v) { return static_cast<float>(v); }
__device__ inline float to_f(double v) { return static_cast<float>(v); }
__device__ inline float to_f(bfloat16 v) { return __uint_as_float(static_cast<uint32_t>(v.bits) << 16); }
__device__ inline float to_f(bool v) { return v ? 1.f : 0.f; }
__device__ inline float to_f(int8_t v) { return static_cast<float>(v); }
__device__ inline float to_f(uint8_t v) { return static_cast<float>(v); }
__device__ inline float to_f(int32_t v) { return static_cast<float>(v); }
__device__ inline float to_f(int64_t v) { return static_cast<float>(v); }

// Store-side conversion of a computed value (fp32, bool or integer) to the
// buffer's dtype: floats round to nearest even, integers truncate toward
// zero, bool tests != 0 -- torch's cast semantics.
template <typename T>
struct Cvt {
  template <typename V>
  __device__ static inline T from(V v) { return static_cast<T>(v); }
};
template <>
struct Cvt<_Float16> {
  template <typename V>
  __device__ static inline _Float16 from(V v) { return static_cast<_Float16>(static_cast<float>(v)); }
};
template <>
struct Cvt<bfloat16> {
  template <typename V>
  __device__ static inline bfloat16 from(V v) {
    uint32_t u = __float_as_uint(static_cast<float>(v));
    bfloat16 r;
    if ((u & 0x7fffffffu) > 0x7f800000u) {  // NaN stays quiet
      r.bits = static_cast<uint16_t>((u >> 16) | 0x40u);
      return r;
    }
    u += 0x7fffu + ((u >> 16) & 1u);
    r.bits = static_cast<uint16_t>(u >> 16);
    return r;
  }
};
template <>
struct Cvt<bool> {
  template <typename V>
  __device__ static inline bool from(V v) { return v != 0; }
};

template <typename T, typename V>
__device__ inline T cvt(V v) {
  return Cvt<T>::from(v);
}

// Streaming (non-temporal) store, for outputs too large to stay in the
// caches for their consumer.
template <typename T>
__device__ inline void store_nt(T* p, T v) { __builtin_nontemporal_store(v, p); }
template <>
__device__ inline void store_nt<bfloat16>(bfloat16* p, bfloat16 v) {
  __builtin_nontemporal_store(v.bits, &p->bits);
}

// ---- 8-element groups of the pointwise template ------------------------------
// A pointwise kernel whose direct accesses walk their buffers contiguously
// gives each thread 8 consecutive elements.  Such a load is one 16-byte load
// of the group (two for 4-byte elements) and such a store collects the 8
// values and writes them once; `al` (every such buffer 16-byte aligned, one
// uniform test per kernel) selects the wide form, element accesses otherwise.
typedef uint32_t spy_u32x4 __attribute__((ext_vector_type(4)));
template <typename T>
__device__ inline void load8f(const T* __restrict__ p, bool al, float (&v)[8]) {
  if (al && (sizeof(T) == 2 || sizeof(T) == 4)) {
    constexpr int W = 16 / sizeof(T);  // elements per 16-byte load
#pragma unroll
    for (int h = 0; h < 8 / W; ++h) {
      const spy_u32x4 w = *reinterpret_cast<const spy_u32x4*>(p + h * W);
      const T* e = reinterpret_cast<const T*>(&w);
#pragma unroll
      for (int i = 0; i < W; ++i) v[h * W + i] = to_f(e[i]);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = to_f(p[i]);
  }
}
// The group at p[i0 .. i0 + 7] of a buffer of n elements, for a masked load:
// whole where it lies inside the buffer, else element by element with the
// elements outside it read as 0 (the mask never selects them).
template <typename T>
__device__ inline void load8f_in(const T* __restrict__ p, int64_t i0, int64_t n, bool al,
                                 float (&v)[8]) {
  if (i0 >= 0 && i0 + 8 <= n) {
    load8f(p + i0, al, v);
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int64_t j = i0 + i;
      v[i] = (j >= 0 && j < n) ? to_f(p[j]) : 0.f;
    }
  }
}
template <typename T, bool NT>
__device__ inline void store8v(T* __restrict__ p, bool al, const T (&v)[8]) {
  if (al && (sizeof(T) == 2 || sizeof(T) == 4)) {
    constexpr int W = 16 / sizeof(T);
#pragma unroll
    for (int h = 0; h < 8 / W; ++h) {
      spy_u32x4 w;
      T* e = reinterpret_cast<T*>(&w);
#pragma unroll
      for (int i = 0; i < W; ++i) e[i] = v[h * W + i];
      if constexpr (NT)
        __builtin_nontemporal_store(w, reinterpret_cast<spy_u32x4*>(p + h * W));
      else
        *reinterpret_cast<spy_u32x4*>(p + h * W) = w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if constexpr (NT) store_nt(p + i, v[i]);
      else p[i] = v[i];
    }
  }
}

// Rounds an fp32 value to the precision of a narrower dtype (to_dtype).
__device__ inline float round_half(float v) { return static_cast<float>(static_cast<_Float16>(v)); }
__device__ inline float round_bf16(float v) { return to_f(Cvt<bfloat16>::from(v)); }

// ---- math -----------------------------------------------------------------
__device__ inline float inf() { return __builtin_inff(); }
__device__ inline float where(float c, float a, float b) { return c != 0.f ? a : b; }
__device__ inline float maximum(float a, float b) {
  return (a != a || b != b) ? __builtin_nanf("") : (a > b ? a : b);
}
__device__ inline float minimum(float a, float b) {
  return (a != a || b != b) ? __builtin_nanf("") : (a < b ? a : b);
}
__device__ inline float relu(float x) { return x > 0.f ? x : 0.f; }
__device__ inline float sigmoid(float x) { return 1.f / (1.f + expf(-x)); }
__device__ inline float rsqrt(float x) { return 1.f / sqrtf(x); }
__device__ inline float sign(float x) { return static_cast<float>((x > 0.f) - (x < 0.f)); }
__device__ inline float floordiv(float a, float b) { return floorf(a / b); }
__device__ inline float truncdiv(float a, float b) { return truncf(a / b); }
__device__ inline float remainder(float a, float b) {
  float r = fmodf(a, b);
  return (r != 0.f && ((r < 0.f) != (b < 0.f))) ? r + b : r;
}
__device__ inline float isnan_(float x) { return x != x ? 1.f : 0.f; }
__device__ inline float isinf_(float x) { return (x == inf() || x == -inf()) ? 1.f : 0.f; }
__device__ inline float round_even(float x) { return rintf(x); }

// erf without the branches of a full-precision erff (it sits on the GELU
// path of compiled graphs).  |x| < 0.5: the odd Maclaurin series
// 2/sqrt(pi) (x - x^3/3 + x^5/10 - x^7/42 + x^9/216 - x^11/1320), truncation
// error below 2e-8.  |x| >= 0.5: 1 - erfc(|x|) with erfc from Abramowitz &
// Stegun, Handbook of Mathematical Functions, 7.1.26 (error at most 1.5e-7):
// erfc(a) = t (a1 + t (a2 + t (a3 + t (a4 + t a5)))) exp(-a^2), t = 1/(1 + p a).
__device__ inline float erf_fast(float x) {
  const float y = x * x;
  float s = fmaf(y, -1.0f / 1320.0f, 1.0f / 216.0f);
  s = fmaf(s, y, -1.0f / 42.0f);
  s = fmaf(s, y, 1.0f / 10.0f);
  s = fmaf(s, y, -1.0f / 3.0f);
  s = fmaf(s, y, 1.0f);
  const float small = 1.1283791670955126f * x * s;  // 2 / sqrt(pi)
  const float a = fabsf(x);
  const float t = __builtin_amdgcn_rcpf(fmaf(0.3275911f, a, 1.0f));
  float q = fmaf(1.061405429f, t, -1.453152027f);
  q = fmaf(q, t, 1.421413741f);
  q = fmaf(q, t, -0.284496736f);
  q = fmaf(q, t, 0.254829592f);
  const float large = copysignf(1.0f - q * t * __expf(-y), x);
  return a < 0.5f ? small : large;
}

// GELU, erf form: x Phi(x) = max(x, 0) - |x| h(|x|) with h(a) = erfc(a/sqrt 2)/2
// the Gaussian tail.  h = 2^p(a) on [0, 9), p the degree-6 polynomial fit
// to log2 h there (iteratively reweighted least squares in float64 toward
// equal ripple of the absolute error of a h, converted to monomials); from
// 9 on h < 1.2e-19 and is taken as 0.  Absolute error below 1e-6 for every
// finite x (float32, against float64 erfc); +-inf and NaN give NaN.
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

// Integer index helpers used by printed index expressions.
__device__ inline int64_t floordiv_i(int64_t a, int64_t b) {
  int64_t q = a / b;
  return (a % b != 0 && ((a < 0) != (b < 0))) ? q - 1 : q;
}
__device__ inline int64_t mod_i(int64_t a, int64_t b) {
  int64_t r = a % b;
  return (r != 0 && ((r < 0) != (b < 0))) ? r + b : r;
}
__device__ inline int64_t min_i(int64_t a, int64_t b) { return a < b ? a : b; }
__device__ inline int64_t max_i(int64_t a, int64_t b) { return a > b ? a : b; }

// ---- block reductions (wave64 butterflies + one LDS exchange) -------------
struct SumF {
  __device__ static inline float id() { return 0.f; }
  __device__ static inline float op(float a, float b) { return a + b; }
};
struct ProdF {
  __device__ static inline float id() { return 1.f; }
  __device__ static inline float op(float a, float b) { return a * b; }
};
struct MaxF {
  __device__ static inline float id() { return -inf(); }
  __device__ static inline float op(float a, float b) { return maximum(a, b); }
};
struct MinF {
  __device__ static inline float id() { return inf(); }
  __device__ static inline float op(float a, float b) { return minimum(a, b); }
};
struct AnyF {
  __device__ static inline float id() { return 0.f; }
  __device__ static inline float op(float a, float b) { return (a != 0.f || b != 0.f) ? 1.f : 0.f; }
};

// Lane-to-lane move within a row of 16 lanes (DPP control CTRL: quad
// permutations, row mirrors), no LDS round trip.
template <int CTRL>
__device__ inline float dpp_f(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL,
                                                               0xf, 0xf, false));
}

// Reduction over the 64 lanes of a wave; every lane gets the result.  Within
// each row of 16 lanes: swap neighbours (quad_perm 1,0,3,2), pairs
// (2,3,0,1), then the mirrored half row and the mirrored row, so every lane
// holds its row's total; the four row totals are read as scalars (lanes 0,
// 16, 32, 48) and combined.
template <typename Op>
__device__ inline float wave_reduce(float v) {
  v = Op::op(v, dpp_f<0xb1>(v));
  v = Op::op(v, dpp_f<0x4e>(v));
  v = Op::op(v, dpp_f<0x141>(v));
  v = Op::op(v, dpp_f<0x140>(v));
  const int b = __builtin_bit_cast(int, v);
  const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 0));
  const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 16));
  const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 32));
  const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 48));
  return Op::op(Op::op(r0, r1), Op::op(r2, r3));
}

// Reduction over the BLOCK threads of the workgroup; every thread gets the
// result.  `lds` holds BLOCK/64 floats; two barriers, so every thread of the
// workgroup must call it.
template <typename Op, int BLOCK>
__device__ inline float block_reduce(float v, float* lds) {
  v = wave_reduce<Op>(v);
  if constexpr (BLOCK <= kWave) {
    return v;
  } else {
    const int w = threadIdx.x / kWave;
    if ((threadIdx.x % kWave) == 0) lds[w] = v;
    __syncthreads();
    float r = lds[0];
#pragma unroll
    for (int i = 1; i < BLOCK / kWave; ++i) r = Op::op(r, lds[i]);
    __syncthreads();
    return r;
  }
}

// (value, index) pairs for argmax / argmin; ties go to the lowest index and
// NaN wins, as in torch.
template <bool MAX>
__device__ inline void arg_combine(float& v, int64_t& i, float v2, int64_t i2) {
  const bool nan1 = v != v, nan2 = v2 != v2;
  bool take;
  if (nan1 || nan2) {
    take = nan2 && (!nan1 || i2 < i);
  } else {
    take = MAX ? (v2 > v || (v2 == v && i2 < i)) : (v2 < v || (v2 == v && i2 < i));
  }
  if (take) {
    v = v2;
    i = i2;
  }
}

template <bool MAX, int BLOCK>
__device__ inline int64_t block_arg(float v, int64_t i, float* lds_v, int64_t* lds_i) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    float v2 = __shfl_xor(v, off, kWave);
    int64_t i2 = __shfl_xor(i, off, kWave);
    arg_combine<MAX>(v, i, v2, i2);
  }
  if constexpr (BLOCK > kWave) {
    const int w = threadIdx.x / kWave;
    if ((threadIdx.x % kWave) == 0) {
      lds_v[w] = v;
      lds_i[w] = i;
    }
    __syncthreads();
    v = lds_v[0];
    i = lds_i[0];
#pragma unroll
    for (int k = 1; k < BLOCK / kWave; ++k) arg_combine<MAX>(v, i, lds_v[k], lds_i[k]);
    __syncthreads();
  }
  return i;
}

// Welford state (mean, m2, weight) and its combine (Chan et al. parallel
// variance update).
struct Welford {
  float mean, m2, weight;
};
__device__ inline Welford welford_combine(Welford a, Welford b) {
  if (b.weight == 0.f) return a;
  if (a.weight == 0.f) return b;
  const float w = a.weight + b.weight;
  const float delta = b.mean - a.mean;
  const float nb = b.weight / w;
  Welford r;
  r.mean = a.mean + delta * nb;
  r.m2 = a.m2 + b.m2 + delta * delta * a.weight * nb;
  r.weight = w;
  return r;
}
__device__ inline Welford welford_add(Welford a, float x) {
  Welford b;
  b.mean = x;
  b.m2 = 0.f;
  b.weight = 1.f;
  return welford_combine(a, b);
}

// One thread's share of a row, accumulated without a division per element:
// sums of x - c and (x - c)^2 around the thread's first element c (the
// shifted-data algorithm; Chan, Golub & LeVeque, "Algorithms for computing
// the sample variance", 1983, section 3).  c lies within the data, so the
// sums carry no cancellation beyond that of the data's own spread.
// welford_finish turns it into a Welford state for the cross-thread combine.
struct WelfordAcc {
  float shift, s1, s2, n;
};
__device__ inline WelfordAcc welford_acc_add(WelfordAcc a, float x) {
  const float c = a.n == 0.f ? x : a.shift;
  const float d = x - c;
  return WelfordAcc{c, a.s1 + d, fmaf(d, d, a.s2), a.n + 1.f};
}
__device__ inline Welford welford_finish(WelfordAcc a) {
  if (a.n == 0.f) return Welford{0.f, 0.f, 0.f};
  const float m = a.s1 / a.n;
  return Welford{a.shift + m, fmaxf(fmaf(-a.s1, m, a.s2), 0.f), a.n};
}

// Welford states summed around a shift k: (sum w, sum w (mean - k),
// sum m2 + w (mean - k)^2) add without divisions, and the state of the union
// is mean = k + S1/W, m2 = S2 - S1^2/W.  With k the mean of one member, the
// subtraction cancels only as much as that member's mean differs from the
// union's (the parallel form of the shifted-data algorithm; Chan, Golub &
// LeVeque 1983).  Empty members (w = 0) add nothing.
__device__ inline void welford_shifted(Welford s, float k, float& w, float& s1, float& s2) {
  const float d = s.weight > 0.f ? s.mean - k : 0.f;
  w = s.weight;
  s1 = s.weight * d;
  s2 = fmaf(s1, d, s.m2);
}
__device__ inline Welford welford_unshift(float k, float w, float s1, float s2) {
  if (!(w > 0.f)) return Welford{0.f, 0.f, 0.f};
  const float m = s1 / w;
  return Welford{k + m, fmaxf(fmaf(-s1, m, s2), 0.f), w};
}

// Welford state of the whole workgroup's row, on every thread: per wave,
// shifted sums around lane 0's mean (three butterflies, no divisions); across
// waves, the same around wave 0's mean.  Two barriers, so every thread of
// the workgroup must call it.
template <int BLOCK>
__device__ inline Welford block_welford(Welford s, float* lds) {
  const float k = __shfl(s.mean, 0, kWave);
  float w, s1, s2;
  welford_shifted(s, k, w, s1, s2);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    w += __shfl_xor(w, off, kWave);
    s1 += __shfl_xor(s1, off, kWave);
    s2 += __shfl_xor(s2, off, kWave);
  }
  s = welford_unshift(k, w, s1, s2);
  if constexpr (BLOCK > kWave) {
    constexpr int NW = BLOCK / kWave;
    const int wv = threadIdx.x / kWave;
    if ((threadIdx.x % kWave) == 0) {
      lds[wv] = s.mean;
      lds[NW + wv] = s.m2;
      lds[2 * NW + wv] = s.weight;
    }
    __syncthreads();
    const float k2 = lds[0];
    float tw = 0.f, t1 = 0.f, t2 = 0.f;
#pragma unroll
    for (int i = 0; i < NW; ++i) {
      float a, b, c;
      welford_shifted(Welford{lds[i], lds[NW + i], lds[2 * NW + i]}, k2, a, b, c);
      tw += a;
      t1 += b;
      t2 += c;
    }
    __syncthreads();
    s = welford_unshift(k2, tw, t1, t2);
  }
  return s;
}

}  // namespace spy
