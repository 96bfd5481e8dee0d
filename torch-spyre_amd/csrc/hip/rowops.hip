// Row-wise kernels: softmax / log-softmax, RMSNorm, LayerNorm (each with an
// optional fused residual add) and the GELU(x*s+b) + row-sum chain.
//
// Design (gfx950): these are HBM-bound (a few FLOP per byte), so each row is
// read once into registers with 16-byte vector loads (8 fp16 per load,
// consecutive lanes on consecutive 16-byte chunks => fully coalesced
// 1 KiB per wave instruction), reduced with wave64 butterflies (+ one LDS
// exchange when a row spans several waves) and written once.  A row of up to
// 64K elements stays in registers; longer rows use a two-pass looped kernel.
#include <type_traits>

#include "sph_common.h"

namespace sph {
namespace {

// Threads-per-row / 8-element-vectors-per-thread configurations.
struct RowCfg {
  int tpr;
  int vpt;
};
// ({1024, 4} before {1024, 8}: rows up to 32768 elements then run on the
// configuration whose registers hold them without spilling; with 8 chunks
// per thread a 1024-thread workgroup (128 registers per lane) spills.)
constexpr RowCfg kCfgs[] = {{64, 1}, {64, 4}, {256, 2}, {256, 4}, {1024, 4}, {1024, 8}};
constexpr int kNumCfgs = 6;

inline int pick_cfg(int64_t cols) {
  for (int i = 0; i < kNumCfgs; ++i)
    if (cols <= static_cast<int64_t>(kCfgs[i].tpr) * kCfgs[i].vpt * 8) return i;
  return -1;  // looped kernel
}

template <int TPR>
constexpr int block_of() {
  return TPR < 256 ? 256 : TPR;
}

// Loads one chunk of 8 elements starting at column c0 (out-of-row elements
// get `fill`).  VEC: the row base is 16-byte aligned, so a full chunk can be
// read with vector loads; a partial last chunk is read element-wise.
template <typename T, bool VEC>
__device__ inline void load_chunk(const T* __restrict__ row, int64_t cols,
                                  int64_t c0, float fill, float (&v)[8]) {
  if (VEC && c0 + 8 <= cols) {
    load8<T>(row + c0, v);
  } else {
    const int64_t n = cols - c0;
    load8_partial<T>(row + c0, n > 8 ? 8 : (n < 0 ? 0 : static_cast<int>(n)),
                     fill, v);
  }
}

// Column of element j of chunk i for thread t.
template <int TPR>
__device__ inline int64_t chunk_col(int i, int t) {
  return (static_cast<int64_t>(i) * TPR + t) * 8;
}

// Loads this thread's VPT chunks of a row.
template <typename T, int TPR, int VPT, bool VEC>
__device__ inline void load_row(const T* __restrict__ row, int64_t cols,
                                int t, float fill, float (&v)[VPT][8]) {
#pragma unroll
  for (int i = 0; i < VPT; ++i) load_chunk<T, VEC>(row, cols, chunk_col<TPR>(i, t), fill, v[i]);
}

template <typename T, int TPR, int VPT, bool VEC, bool NT = false>
__device__ inline void store_row(T* __restrict__ row, int64_t cols, int t,
                                 const float (&v)[VPT][8]) {
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int64_t c0 = chunk_col<TPR>(i, t);
    if (VEC && c0 + 8 <= cols) {
      store8<T, NT>(row + c0, v[i]);
    } else {
      const int64_t n = cols - c0;
      if (n > 0) store8_partial<T>(row + c0, n > 8 ? 8 : static_cast<int>(n), v[i]);
    }
  }
}

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// ----------------------------------------------------------------------------
// Softmax
// ----------------------------------------------------------------------------
template <typename TI, typename TO, int TPR, int VPT, bool VEC>
__global__ void __launch_bounds__(block_of<TPR>())
softmax_regs(const TI* __restrict__ x, int64_t ldx, TO* __restrict__ y,
             int64_t ldy, int64_t rows, int64_t cols, float scale, int flags,
             int64_t qlen, int64_t qoff) {
  constexpr int BLOCK = block_of<TPR>();
  constexpr int RPB = BLOCK / TPR;
  __shared__ float lds[BLOCK / kWave];
  const int t = threadIdx.x % TPR;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * RPB + threadIdx.x / TPR;
  const bool valid = row < rows;
  const float ninf = -INFINITY;

  float v[VPT][8];
  if (valid) {
    load_row<TI, TPR, VPT, VEC>(x + row * ldx, cols, t, ninf, v);
  } else {
#pragma unroll
    for (int i = 0; i < VPT; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j) v[i][j] = ninf;
  }
  // Row lengths here fit in 32 bits (at most TPR * VPT * 8 columns), so the
  // causal limit and the column index are 32-bit.  Values are kept in log2
  // units (x * scale * log2 e): the exponential is then the hardware exp2 of
  // a difference, whose results below 2^-126 flush to zero, which changes
  // nothing next to a row sum of at least 1.
  int limit = static_cast<int>(cols);
  if ((flags & SPH_SOFTMAX_CAUSAL) && valid) {
    const int64_t lim = (row % qlen) + qoff + 1;
    limit = lim < cols ? static_cast<int>(lim) : limit;
  }
  const float sl = scale * kLog2e;
  float m = ninf;
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int c = (i * TPR + t) * 8 + j;
      float a = v[i][j] * sl;
      a = (c < limit) ? a : ninf;
      v[i][j] = a;
      m = fmaxf(m, a);
    }
  }
  m = group_reduce<MaxOp, TPR>(m, lds);
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < VPT; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float e = __builtin_amdgcn_exp2f(v[i][j] - m);
      s += e;
      if (!(flags & SPH_SOFTMAX_LOG)) v[i][j] = e;
    }
  s = group_reduce<SumOp, TPR>(s, lds);
  if (!valid) return;
  if (flags & SPH_SOFTMAX_LOG) {
    const float ls = log2f(s);
#pragma unroll
    for (int i = 0; i < VPT; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j) v[i][j] = (v[i][j] - m - ls) * kLn2;
  } else {
    const float inv = 1.0f / s;
#pragma unroll
    for (int i = 0; i < VPT; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j) v[i][j] *= inv;
  }
  store_row<TO, TPR, VPT, VEC>(y + row * ldy, cols, t, v);
}

// (max, sum) state of an online softmax: `s` sums exp2(x - m) over the
// values seen, m their maximum.  Merging two states rescales both sums to the
// larger maximum.  A state that has seen only -inf is (-inf, 0); the base
// 0 in place of an infinite maximum keeps exp2 away from inf - inf.
__device__ inline void ms_merge(float& m, float& s, float mo, float so) {
  const float mn = fmaxf(m, mo);
  const float base = mn == -INFINITY ? 0.f : mn;
  s = s * __builtin_amdgcn_exp2f(m - base) + so * __builtin_amdgcn_exp2f(mo - base);
  m = mn;
}

template <int CTRL>
__device__ inline float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}

// (m, s) over the TPR threads of a row group (TPR a multiple of 64), every
// thread of the group receiving the result: DPP butterflies inside each
// 16-lane row (quad_perm [1,0,3,2], [2,3,0,1], row_half_mirror,
// row_mirror), the four rows of the wave through readlane, and for groups
// of several waves one LDS exchange with a single barrier.  `lds_m` and
// `lds_s` hold blockDim/64 floats each; every thread of the workgroup must
// reach the call.
template <int TPR>
__device__ inline void group_ms(float& m, float& s, float* lds_m, float* lds_s) {
  static_assert(TPR % kWave == 0, "row groups of whole waves");
  ms_merge(m, s, dpp_f<0xB1>(m), dpp_f<0xB1>(s));
  ms_merge(m, s, dpp_f<0x4E>(m), dpp_f<0x4E>(s));
  ms_merge(m, s, dpp_f<0x141>(m), dpp_f<0x141>(s));
  ms_merge(m, s, dpp_f<0x140>(m), dpp_f<0x140>(s));
  float rm[4], rs[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    rm[r] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(m), r * 16));
    rs[r] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(s), r * 16));
  }
  m = rm[0];
  s = rs[0];
#pragma unroll
  for (int r = 1; r < 4; ++r) ms_merge(m, s, rm[r], rs[r]);
  if constexpr (TPR > kWave) {
    constexpr int NW = TPR / kWave;
    const int wave = threadIdx.x / kWave;
    if (threadIdx.x % kWave == 0) {
      lds_m[wave] = m;
      lds_s[wave] = s;
    }
    __syncthreads();
    const int first = (wave / NW) * NW;
    m = lds_m[first];
    s = lds_s[first];
#pragma unroll
    for (int k = 1; k < NW; ++k) ms_merge(m, s, lds_m[first + k], lds_s[first + k]);
  }
}

// Rows of exactly TPR * VPT * 8 columns with 16-byte aligned rows (c1's
// [512, 4096] among them): whole chunks without per-chunk bounds tests, the
// causal mask and log form chosen once per thread rather than tested per
// element, and one combined (max, sum) reduction per row: each thread sums
// exp2 of its values against its own maximum, and the states merge in one
// pass (group_ms).  At this size the kernel is latency-bound: a kernel
// launched back to back costs 1.53 us empty and 2.69 us when one thread
// loads and stores one value, and this one 2.9-3.0 us at [512, 4096] (on
// 128 threads x 4 chunks per row, two rows per workgroup), against 3.3 us
// for two serial block reductions on 256 threads x 2 chunks.  A row past
// the end (several rows per workgroup) loads the last row and stores
// nothing.
template <typename TI, typename TO, int TPR, int VPT>
__global__ void __launch_bounds__(block_of<TPR>())
softmax_full(const TI* __restrict__ x, int64_t ldx, TO* __restrict__ y, int64_t ldy,
             int64_t rows, float scale, int flags, int64_t qlen, int64_t qoff) {
  constexpr int BLOCK = block_of<TPR>(), RPB = BLOCK / TPR, COLS = TPR * VPT * 8;
  __shared__ float lds_m[BLOCK / kWave], lds_s[BLOCK / kWave];
  const int t = threadIdx.x % TPR;
  int64_t row = static_cast<int64_t>(blockIdx.x) * RPB + threadIdx.x / TPR;
  const bool valid = row < rows;
  if (!valid) row = rows - 1;
  float v[VPT][8];
#pragma unroll
  for (int i = 0; i < VPT; ++i) load8<TI>(x + row * ldx + (i * TPR + t) * 8, v[i]);
  const float sl = scale * kLog2e;
  float m = -INFINITY;
  if (flags & SPH_SOFTMAX_CAUSAL) {
    const int64_t lim = (row % qlen) + qoff + 1;
    const int limit = lim < 0 ? 0 : (lim < COLS ? static_cast<int>(lim) : COLS);
#pragma unroll
    for (int i = 0; i < VPT; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float a = ((i * TPR + t) * 8 + j < limit) ? v[i][j] * sl : -INFINITY;
        v[i][j] = a;
        m = fmaxf(m, a);
      }
  } else {
#pragma unroll
    for (int i = 0; i < VPT; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        v[i][j] *= sl;
        m = fmaxf(m, v[i][j]);
      }
  }
  // this thread's state against its own maximum
  const float mt = m;
  const float bt = mt == -INFINITY ? 0.f : mt;
  float s = 0.f;
  const bool lg = flags & SPH_SOFTMAX_LOG;
  if (lg) {
#pragma unroll
    for (int i = 0; i < VPT; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j) s += __builtin_amdgcn_exp2f(v[i][j] - bt);
  } else {
#pragma unroll
    for (int i = 0; i < VPT; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        v[i][j] = __builtin_amdgcn_exp2f(v[i][j] - bt);
        s += v[i][j];
      }
  }
  group_ms<TPR>(m, s, lds_m, lds_s);
  if (!valid) return;
  if (lg) {
    const float ls = m + log2f(s);
#pragma unroll
    for (int i = 0; i < VPT; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j) v[i][j] = (v[i][j] - ls) * kLn2;
  } else {
    // e^(x - m) / s = exp2(v - bt) * exp2(bt - m) / s.  A thread whose
    // values are all masked holds zeros (its factor is 0, never exp2 of a
    // large difference); a row with no finite value is NaN, as softmax over
    // all -inf is.
    const float f = m == -INFINITY   ? NAN
                    : mt == -INFINITY ? 0.f
                                      : __builtin_amdgcn_exp2f(bt - m) / s;
#pragma unroll
    for (int i = 0; i < VPT; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j) v[i][j] *= f;
  }
#pragma unroll
  for (int i = 0; i < VPT; ++i) store8<TO>(y + row * ldy + (i * TPR + t) * 8, v[i]);
}

// Rows longer than the register-resident configs: online max/sum pass, then
// an output pass.  One 256-thread block per row.
template <typename TI, typename TO>
__global__ void __launch_bounds__(256)
softmax_looped(const TI* __restrict__ x, int64_t ldx, TO* __restrict__ y,
               int64_t ldy, int64_t rows, int64_t cols, float scale,
               int flags, int64_t qlen, int64_t qoff) {
  __shared__ float lds[4];
  const int64_t row = blockIdx.x;
  const TI* xr = x + row * ldx;
  int64_t limit = cols;
  if (flags & SPH_SOFTMAX_CAUSAL) {
    const int64_t lim = (row % qlen) + qoff + 1;
    limit = lim < cols ? lim : cols;
  }
  float m = -INFINITY, s = 0.f;
  for (int64_t c = threadIdx.x; c < cols; c += 256) {
    const float a = (c < limit) ? Num<TI>::to_f(xr[c]) * scale : -INFINITY;
    if (a > m) {
      s = s * exp2f((m - a) * kLog2e) + 1.0f;
      m = a;
    } else if (a != -INFINITY) {
      s += exp2f((a - m) * kLog2e);
    }
  }
  const float gm = group_reduce<MaxOp, 256>(m, lds);
  s = (m == -INFINITY) ? 0.f : s * exp2f((m - gm) * kLog2e);
  s = group_reduce<SumOp, 256>(s, lds);
  TO* yr = y + row * ldy;
  const float inv = 1.0f / s;
  const float ls = log2f(s) * kLn2;
  for (int64_t c = threadIdx.x; c < cols; c += 256) {
    const float a = (c < limit) ? Num<TI>::to_f(xr[c]) * scale : -INFINITY;
    const float o = (flags & SPH_SOFTMAX_LOG) ? (a - gm - ls)
                                              : exp2f((a - gm) * kLog2e) * inv;
    yr[c] = Num<TO>::from_f(o);
  }
}

// ----------------------------------------------------------------------------
// Residual add + RMSNorm / LayerNorm
// ----------------------------------------------------------------------------
template <typename T, typename W, int TPR, int VPT, bool VEC, bool LAYER>
__global__ void __launch_bounds__(block_of<TPR>())
norm_regs(const T* __restrict__ x, const T* __restrict__ res,
          const W* __restrict__ w, const W* __restrict__ b,
          T* __restrict__ y, T* __restrict__ h, float* __restrict__ mean_out,
          float* __restrict__ rstd_out, int64_t rows, int64_t cols,
          float eps) {
  constexpr int BLOCK = block_of<TPR>();
  constexpr int RPB = BLOCK / TPR;
  __shared__ float lds[BLOCK / kWave];
  const int t = threadIdx.x % TPR;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * RPB + threadIdx.x / TPR;
  const bool valid = row < rows;
  const int64_t rr = valid ? row : 0;

  float v[VPT][8];
  load_row<T, TPR, VPT, VEC>(x + rr * cols, cols, t, 0.f, v);
  if (res != nullptr) {
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      float r[8];
      load_chunk<T, VEC>(res + rr * cols, cols, chunk_col<TPR>(i, t), 0.f, r);
#pragma unroll
      for (int j = 0; j < 8; ++j)  // round the sum to T, as an eager add would
        v[i][j] = Num<T>::to_f(Num<T>::from_f(v[i][j] + r[j]));
    }
    if (valid && h != nullptr) store_row<T, TPR, VPT, VEC, true>(h + rr * cols, cols, t, v);
  }
  const float inv_n = 1.0f / static_cast<float>(cols);
  float mean = 0.f;
  if constexpr (LAYER) {
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < VPT; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j) s += v[i][j];
    mean = group_reduce<SumOp, TPR>(s, lds) * inv_n;
  }
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < VPT; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int64_t c = (static_cast<int64_t>(i) * TPR + t) * 8 + j;
      const float d = (c < cols) ? v[i][j] - mean : 0.f;
      ss += d * d;
    }
  ss = group_reduce<SumOp, TPR>(ss, lds);
  const float rstd = rsqrtf(ss * inv_n + eps);
  if (!valid) return;
  if (t == 0) {
    if (rstd_out) rstd_out[row] = rstd;
    if (LAYER && mean_out) mean_out[row] = mean;
  }
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int64_t c0 = chunk_col<TPR>(i, t);
    float wv[8], bv[8];
    if (w != nullptr) {
      load_chunk<W, VEC>(w, cols, c0, 1.f, wv);
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) wv[j] = 1.f;
    }
    if (LAYER && b != nullptr) {
      load_chunk<W, VEC>(b, cols, c0, 0.f, bv);
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) bv[j] = 0.f;
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) v[i][j] = fmaf((v[i][j] - mean) * rstd, wv[j], bv[j]);
  }
  store_row<T, TPR, VPT, VEC, true>(y + row * cols, cols, t, v);
}

template <typename T, typename W, bool LAYER>
__global__ void __launch_bounds__(256)
norm_looped(const T* __restrict__ x, const T* __restrict__ res,
            const W* __restrict__ w, const W* __restrict__ b,
            T* __restrict__ y, T* __restrict__ h, float* __restrict__ mean_out,
            float* __restrict__ rstd_out, int64_t rows, int64_t cols,
            float eps) {
  __shared__ float lds[4];
  const int64_t row = blockIdx.x;
  const T* xr = x + row * cols;
  const T* rr = res ? res + row * cols : nullptr;
  auto hval = [&](int64_t c) {
    float a = Num<T>::to_f(xr[c]);
    if (rr) a = Num<T>::to_f(Num<T>::from_f(a + Num<T>::to_f(rr[c])));
    return a;
  };
  float s = 0.f, ss = 0.f;
  for (int64_t c = threadIdx.x; c < cols; c += 256) {
    const float a = hval(c);
    s += a;
    ss += a * a;
  }
  const float inv_n = 1.0f / static_cast<float>(cols);
  float mean = 0.f;
  if (LAYER) mean = group_reduce<SumOp, 256>(s, lds) * inv_n;
  ss = group_reduce<SumOp, 256>(ss, lds) * inv_n;
  const float var = LAYER ? fmaxf(ss - mean * mean, 0.f) : ss;
  const float rstd = rsqrtf(var + eps);
  if (threadIdx.x == 0) {
    if (rstd_out) rstd_out[row] = rstd;
    if (LAYER && mean_out) mean_out[row] = mean;
  }
  for (int64_t c = threadIdx.x; c < cols; c += 256) {
    const float a = hval(c);
    if (rr && h) h[row * cols + c] = Num<T>::from_f(a);
    float o = (a - mean) * rstd * (w ? Num<W>::to_f(w[c]) : 1.f);
    if (LAYER && b) o += Num<W>::to_f(b[c]);
    y[row * cols + c] = Num<T>::from_f(o);
  }
}

// ----------------------------------------------------------------------------
// y = gelu_erf(x * s + b), rowsum = sum(y)
// ----------------------------------------------------------------------------
template <typename T, int TPR, int VPT, bool VEC>
__global__ void __launch_bounds__(block_of<TPR>())
gelu_rowsum_regs(const T* __restrict__ x, const T* __restrict__ sv,
                 const T* __restrict__ bv, float s0, float b0,
                 T* __restrict__ y, T* __restrict__ rowsum, int64_t rows,
                 int64_t cols) {
  constexpr int BLOCK = block_of<TPR>();
  constexpr int RPB = BLOCK / TPR;
  __shared__ float lds[BLOCK / kWave];
  const int t = threadIdx.x % TPR;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * RPB + threadIdx.x / TPR;
  const bool valid = row < rows;
  const int64_t rr = valid ? row : 0;
  float v[VPT][8];
  load_row<T, TPR, VPT, VEC>(x + rr * cols, cols, t, 0.f, v);
  float acc = 0.f;
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int64_t c0 = chunk_col<TPR>(i, t);
    float s[8], b[8];
    if (sv) {
      load_chunk<T, VEC>(sv, cols, c0, 0.f, s);
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) s[j] = s0;
    }
    if (bv) {
      load_chunk<T, VEC>(bv, cols, c0, 0.f, b);
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) b[j] = b0;
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float g = gelu_erf(fmaf(v[i][j], s[j], b[j]));
      v[i][j] = g;
      acc += (c0 + j < cols) ? g : 0.f;
    }
  }
  if (rowsum) acc = group_reduce<SumOp, TPR>(acc, lds);
  if (!valid) return;
  if (y) store_row<T, TPR, VPT, VEC, true>(y + row * cols, cols, t, v);
  if (rowsum && t == 0) rowsum[row] = Num<T>::from_f(acc);
}

// Whole-row path for rows of exactly NT * 8 * VPT 16-bit values (16-byte
// aligned): a workgroup of NT threads handles RPW consecutive rows.  The
// per-column scale and shift are loaded and widened once per thread and
// reused for every row, all RPW rows' loads are issued before any math
// (RPW * VPT 16-byte loads in flight per thread), and the RPW row sums share
// one block reduction.  Rows past the end are clamped for loading and not
// stored.  Plain (cached) loads: the non-temporal form measured 10-15 %
// slower here.
// SBV: s and b are both vectors; they then stay in the element type and,
// for fp16, the compiler forms x * s + b as one mixed-precision FMA from
// the three 16-bit values (no separate conversions).  Otherwise they are
// widened to fp32 once (scalars are used as given, in fp32).
template <typename T, int NT, int VPT, int RPW, bool SBV>
__global__ void __launch_bounds__(NT)
gelu_rowsum_rows(const T* __restrict__ x, const T* __restrict__ sv, const T* __restrict__ bv,
                 float s0, float b0, T* __restrict__ y, T* __restrict__ rowsum, int64_t rows) {
  constexpr int COLS = NT * 8 * VPT, NWAVE = NT / kWave;
  __shared__ float red[NWAVE][RPW];
  const int t = threadIdx.x;
  const int64_t r0 = static_cast<int64_t>(blockIdx.x) * RPW;
  using SB = typename std::conditional<SBV, T, float>::type;
  SB s[VPT][8], b[VPT][8];
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int c0 = (i * NT + t) * 8;
    if constexpr (SBV) {
      *reinterpret_cast<u32x4*>(s[i]) = *reinterpret_cast<const u32x4*>(sv + c0);
      *reinterpret_cast<u32x4*>(b[i]) = *reinterpret_cast<const u32x4*>(bv + c0);
    } else {
      if (sv) {
        load8<T>(sv + c0, s[i]);
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) s[i][j] = s0;
      }
      if (bv) {
        load8<T>(bv + c0, b[i]);
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) b[i][j] = b0;
      }
    }
  }
  u32x4 raw[RPW][VPT];
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    const int64_t row = r0 + r < rows ? r0 + r : rows - 1;
#pragma unroll
    for (int i = 0; i < VPT; ++i)
      raw[r][i] = *reinterpret_cast<const u32x4*>(x + row * COLS + (i * NT + t) * 8);
  }
  float acc[RPW];
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    acc[r] = 0.f;
    const int64_t row = r0 + r;
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const T* e = reinterpret_cast<const T*>(&raw[r][i]);
      float g[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        if constexpr (SBV)
          g[j] = gelu_erf(fmaf(Num<T>::to_f(e[j]), Num<T>::to_f(s[i][j]), Num<T>::to_f(b[i][j])));
        else
          g[j] = gelu_erf(fmaf(Num<T>::to_f(e[j]), s[i][j], b[i][j]));
        acc[r] += g[j];
      }
      if (y && row < rows) store8<T, true>(y + row * COLS + (i * NT + t) * 8, g);
    }
  }
  if (!rowsum) return;
  const int wave = t / kWave, lane = t % kWave;
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    const float v = wave_reduce<SumOp>(acc[r]);
    if (lane == 0) red[wave][r] = v;
  }
  __syncthreads();
  if (t < RPW && r0 + t < rows) {
    float v = 0.f;
#pragma unroll
    for (int w = 0; w < NWAVE; ++w) v += red[w][t];
    rowsum[r0 + t] = Num<T>::from_f(v);
  }
}

template <typename T>
__global__ void __launch_bounds__(256)
gelu_rowsum_looped(const T* __restrict__ x, const T* __restrict__ sv,
                   const T* __restrict__ bv, float s0, float b0,
                   T* __restrict__ y, T* __restrict__ rowsum, int64_t rows,
                   int64_t cols) {
  __shared__ float lds[4];
  const int64_t row = blockIdx.x;
  float acc = 0.f;
  for (int64_t c = threadIdx.x; c < cols; c += 256) {
    const float sc = sv ? Num<T>::to_f(sv[c]) : s0;
    const float bc = bv ? Num<T>::to_f(bv[c]) : b0;
    const float g = gelu_erf(fmaf(Num<T>::to_f(x[row * cols + c]), sc, bc));
    if (y) y[row * cols + c] = Num<T>::from_f(g);
    acc += g;
  }
  acc = group_reduce<SumOp, 256>(acc, lds);
  if (rowsum && threadIdx.x == 0) rowsum[row] = Num<T>::from_f(acc);
}

// ----------------------------------------------------------------------------
// Host dispatch
// ----------------------------------------------------------------------------
inline bool aligned16(const void* p) {
  return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}

template <typename T>
inline bool vec_ok(const void* p, int64_t ld) {
  const int64_t per16 = 16 / static_cast<int64_t>(sizeof(T));
  return p == nullptr || (aligned16(p) && (ld % per16) == 0);
}

template <int TPR>
inline unsigned grid_rows(int64_t rows) {
  constexpr int RPB = block_of<TPR>() / TPR;
  return static_cast<unsigned>((rows + RPB - 1) / RPB);
}

template <typename TI, typename TO>
int softmax_impl(const void* x, int64_t ldx, void* y, int64_t ldy, int64_t rows,
                 int64_t cols, float scale, int flags, int64_t qlen,
                 int64_t qoff, hipStream_t st) {
  const TI* xi = static_cast<const TI*>(x);
  TO* yo = static_cast<TO*>(y);
  const bool vec = vec_ok<TI>(x, ldx) && vec_ok<TO>(y, ldy);
  if (vec && cols == 4096 && rows <= 0xffffffffLL * 2) {
    // 128 threads x 4 chunks per row, two rows per workgroup (measured best
    // of the register layouts at [512, 4096])
    softmax_full<TI, TO, 128, 4><<<grid_rows<128>(rows), block_of<128>(), 0, st>>>(
        xi, ldx, yo, ldy, rows, scale, flags, qlen, qoff);
    return check_launch("sph_softmax_rows");
  }
  const int cfg = pick_cfg(cols);
#define SPH_SOFTMAX_CASE(I)                                                     \
  case I: {                                                                     \
    constexpr int TPR = kCfgs[I].tpr, VPT = kCfgs[I].vpt;                       \
    if (vec && cols == TPR * VPT * 8)                                           \
      softmax_full<TI, TO, TPR, VPT><<<grid_rows<TPR>(rows), block_of<TPR>(),   \
                                       0, st>>>(xi, ldx, yo, ldy, rows, scale,  \
                                                flags, qlen, qoff);             \
    else if (vec)                                                               \
      softmax_regs<TI, TO, TPR, VPT, true><<<grid_rows<TPR>(rows),              \
                                             block_of<TPR>(), 0, st>>>(         \
          xi, ldx, yo, ldy, rows, cols, scale, flags, qlen, qoff);              \
    else                                                                        \
      softmax_regs<TI, TO, TPR, VPT, false><<<grid_rows<TPR>(rows),             \
                                              block_of<TPR>(), 0, st>>>(        \
          xi, ldx, yo, ldy, rows, cols, scale, flags, qlen, qoff);              \
    break;                                                                      \
  }
  switch (cfg) {
    SPH_SOFTMAX_CASE(0)
    SPH_SOFTMAX_CASE(1)
    SPH_SOFTMAX_CASE(2)
    SPH_SOFTMAX_CASE(3)
    SPH_SOFTMAX_CASE(4)
    SPH_SOFTMAX_CASE(5)
    default:
      softmax_looped<TI, TO><<<static_cast<unsigned>(rows), 256, 0, st>>>(
          xi, ldx, yo, ldy, rows, cols, scale, flags, qlen, qoff);
  }
#undef SPH_SOFTMAX_CASE
  return check_launch("sph_softmax_rows");
}

template <typename T, typename W, bool LAYER>
int norm_impl(const void* x, const void* res, const void* w, const void* b,
              void* y, void* h, float* mean_out, float* rstd_out, int64_t rows,
              int64_t cols, float eps, hipStream_t st) {
  auto xi = static_cast<const T*>(x);
  auto ri = static_cast<const T*>(res);
  auto wi = static_cast<const W*>(w);
  auto bi = static_cast<const W*>(b);
  auto yo = static_cast<T*>(y);
  auto ho = static_cast<T*>(h);
  const bool vec = vec_ok<T>(x, cols) && vec_ok<T>(res, cols) &&
                   vec_ok<W>(w, cols) && vec_ok<W>(b, cols) &&
                   vec_ok<T>(y, cols) && vec_ok<T>(h, cols);
  const int cfg = pick_cfg(cols);
#define SPH_NORM_CASE(I)                                                           \
  case I: {                                                                        \
    constexpr int TPR = kCfgs[I].tpr, VPT = kCfgs[I].vpt;                          \
    if (vec)                                                                       \
      norm_regs<T, W, TPR, VPT, true, LAYER><<<grid_rows<TPR>(rows),               \
                                               block_of<TPR>(), 0, st>>>(          \
          xi, ri, wi, bi, yo, ho, mean_out, rstd_out, rows, cols, eps);            \
    else                                                                           \
      norm_regs<T, W, TPR, VPT, false, LAYER><<<grid_rows<TPR>(rows),              \
                                                block_of<TPR>(), 0, st>>>(         \
          xi, ri, wi, bi, yo, ho, mean_out, rstd_out, rows, cols, eps);            \
    break;                                                                         \
  }
  switch (cfg) {
    SPH_NORM_CASE(0)
    SPH_NORM_CASE(1)
    SPH_NORM_CASE(2)
    SPH_NORM_CASE(3)
    SPH_NORM_CASE(4)
    SPH_NORM_CASE(5)
    default:
      norm_looped<T, W, LAYER><<<static_cast<unsigned>(rows), 256, 0, st>>>(
          xi, ri, wi, bi, yo, ho, mean_out, rstd_out, rows, cols, eps);
  }
#undef SPH_NORM_CASE
  return check_launch(LAYER ? "sph_layernorm" : "sph_rmsnorm");
}

template <typename T>
int gelu_impl(const void* x, const void* s, const void* b, float s0, float b0,
              void* y, void* rowsum, int64_t rows, int64_t cols,
              hipStream_t st) {
  auto xi = static_cast<const T*>(x);
  auto si = static_cast<const T*>(s);
  auto bi = static_cast<const T*>(b);
  auto yo = static_cast<T*>(y);
  auto ro = static_cast<T*>(rowsum);
  const bool vec = vec_ok<T>(x, cols) && vec_ok<T>(s, cols) &&
                   vec_ok<T>(b, cols) && vec_ok<T>(y, cols);
  if constexpr (sizeof(T) == 2) {
    // two rows per workgroup, one 16-byte chunk per thread and row up to
    // 4096 columns (measured at [8192, 4096]: 21.8 us against 26.7 for four
    // rows of two chunks on 256 threads)
    constexpr int RPW = 2;
    const unsigned grid = static_cast<unsigned>(ceil_div(rows, RPW));
    if (vec && rows <= 0x7fffffffLL * RPW) {
      if (cols == 2048) {
        if (si && bi)
          gelu_rowsum_rows<T, 256, 1, RPW, true><<<grid, 256, 0, st>>>(xi, si, bi, s0, b0, yo, ro, rows);
        else
          gelu_rowsum_rows<T, 256, 1, RPW, false><<<grid, 256, 0, st>>>(xi, si, bi, s0, b0, yo, ro, rows);
        return check_launch("sph_gelu_affine_rowsum");
      }
      if (cols == 4096) {
        if (si && bi)
          gelu_rowsum_rows<T, 512, 1, RPW, true><<<grid, 512, 0, st>>>(xi, si, bi, s0, b0, yo, ro, rows);
        else
          gelu_rowsum_rows<T, 512, 1, RPW, false><<<grid, 512, 0, st>>>(xi, si, bi, s0, b0, yo, ro, rows);
        return check_launch("sph_gelu_affine_rowsum");
      }
      if (cols == 8192) {
        if (si && bi)
          gelu_rowsum_rows<T, 512, 2, RPW, true><<<grid, 512, 0, st>>>(xi, si, bi, s0, b0, yo, ro, rows);
        else
          gelu_rowsum_rows<T, 512, 2, RPW, false><<<grid, 512, 0, st>>>(xi, si, bi, s0, b0, yo, ro, rows);
        return check_launch("sph_gelu_affine_rowsum");
      }
    }
  }
  const int cfg = pick_cfg(cols);
#define SPH_GELU_CASE(I)                                                       \
  case I: {                                                                      \
    constexpr int TPR = kCfgs[I].tpr, VPT = kCfgs[I].vpt;                        \
    if (vec)                                                                     \
      gelu_rowsum_regs<T, TPR, VPT, true><<<grid_rows<TPR>(rows),                \
                                            block_of<TPR>(), 0, st>>>(           \
          xi, si, bi, s0, b0, yo, ro, rows, cols);                               \
    else                                                                         \
      gelu_rowsum_regs<T, TPR, VPT, false><<<grid_rows<TPR>(rows),               \
                                             block_of<TPR>(), 0, st>>>(          \
          xi, si, bi, s0, b0, yo, ro, rows, cols);                               \
    break;                                                                       \
  }
  switch (cfg) {
    SPH_GELU_CASE(0)
    SPH_GELU_CASE(1)
    SPH_GELU_CASE(2)
    SPH_GELU_CASE(3)
    SPH_GELU_CASE(4)
    SPH_GELU_CASE(5)
    default:
      gelu_rowsum_looped<T><<<static_cast<unsigned>(rows), 256, 0, st>>>(
          xi, si, bi, s0, b0, yo, ro, rows, cols);
  }
#undef SPH_GELU_CASE
  return check_launch("sph_gelu_affine_rowsum");
}

int check_rows(int64_t rows, int64_t cols) {
  SPH_REQUIRE(rows >= 0 && cols >= 0, SPH_ERR_INVALID_ARG, "negative size");
  SPH_REQUIRE(rows <= 0x7fffffffLL, SPH_ERR_TOO_LARGE, "too many rows");
  return SPH_OK;
}

}  // namespace
}  // namespace sph

using namespace sph;

extern "C" int sph_softmax_rows(sph_dtype in_dtype, sph_dtype out_dtype,
                                const void* x, int64_t ldx, void* y,
                                int64_t ldy, int64_t rows, int64_t cols,
                                float scale, int flags, int64_t causal_q_len,
                                int64_t causal_offset, sph_stream_t stream) {
  if (int e = check_rows(rows, cols)) return e;
  if (rows == 0 || cols == 0) return SPH_OK;
  SPH_REQUIRE(ldx >= cols && ldy >= cols, SPH_ERR_INVALID_ARG,
              "softmax: leading dimension smaller than cols");
  SPH_REQUIRE(!(flags & SPH_SOFTMAX_CAUSAL) || causal_q_len > 0,
              SPH_ERR_INVALID_ARG, "softmax: causal mask needs q_len > 0");
  hipStream_t st = as_stream(stream);
  if (in_dtype == SPH_F16 && out_dtype == SPH_F16)
    return softmax_impl<half_t, half_t>(x, ldx, y, ldy, rows, cols, scale, flags,
                                        causal_q_len, causal_offset, st);
  if (in_dtype == SPH_BF16 && out_dtype == SPH_BF16)
    return softmax_impl<bf16_t, bf16_t>(x, ldx, y, ldy, rows, cols, scale, flags,
                                        causal_q_len, causal_offset, st);
  if (in_dtype == SPH_F32 && out_dtype == SPH_F32)
    return softmax_impl<float, float>(x, ldx, y, ldy, rows, cols, scale, flags,
                                      causal_q_len, causal_offset, st);
  if (in_dtype == SPH_F16 && out_dtype == SPH_F32)
    return softmax_impl<half_t, float>(x, ldx, y, ldy, rows, cols, scale, flags,
                                       causal_q_len, causal_offset, st);
  if (in_dtype == SPH_BF16 && out_dtype == SPH_F32)
    return softmax_impl<bf16_t, float>(x, ldx, y, ldy, rows, cols, scale, flags,
                                       causal_q_len, causal_offset, st);
  return set_error(SPH_ERR_UNSUPPORTED, "softmax: unsupported dtype pair");
}

extern "C" int sph_softmax_rows_f16(const void* x, void* y, int64_t rows,
                                    int64_t cols, sph_stream_t stream) {
  return sph_softmax_rows(SPH_F16, SPH_F16, x, cols, y, cols, rows, cols, 1.0f,
                          0, 0, 0, stream);
}

namespace {
template <bool LAYER>
int norm_dispatch(sph_dtype dt, sph_dtype wdt, const void* x, const void* res,
                  const void* w, const void* b, void* y, void* h,
                  float* mean_out, float* rstd_out, int64_t rows, int64_t cols,
                  float eps, sph_stream_t stream) {
  if (int e = check_rows(rows, cols)) return e;
  if (rows == 0) return SPH_OK;
  SPH_REQUIRE(cols > 0, SPH_ERR_INVALID_ARG, "norm: cols must be > 0");
  hipStream_t st = as_stream(stream);
  if (dt == SPH_F16 && wdt == SPH_F16)
    return norm_impl<half_t, half_t, LAYER>(x, res, w, b, y, h, mean_out, rstd_out,
                                            rows, cols, eps, st);
  if (dt == SPH_F16 && wdt == SPH_F32)
    return norm_impl<half_t, float, LAYER>(x, res, w, b, y, h, mean_out, rstd_out,
                                           rows, cols, eps, st);
  if (dt == SPH_BF16 && wdt == SPH_BF16)
    return norm_impl<bf16_t, bf16_t, LAYER>(x, res, w, b, y, h, mean_out, rstd_out,
                                            rows, cols, eps, st);
  if (dt == SPH_BF16 && wdt == SPH_F32)
    return norm_impl<bf16_t, float, LAYER>(x, res, w, b, y, h, mean_out, rstd_out,
                                           rows, cols, eps, st);
  if (dt == SPH_F32 && wdt == SPH_F32)
    return norm_impl<float, float, LAYER>(x, res, w, b, y, h, mean_out, rstd_out,
                                          rows, cols, eps, st);
  return set_error(SPH_ERR_UNSUPPORTED, "norm: unsupported dtype pair");
}
}  // namespace

extern "C" int sph_rmsnorm(sph_dtype dtype, sph_dtype w_dtype, const void* x,
                           const void* residual, const void* weight, void* y,
                           void* h_out, float* rstd_out, int64_t rows,
                           int64_t cols, float eps, sph_stream_t stream) {
  return norm_dispatch<false>(dtype, w_dtype, x, residual, weight, nullptr, y,
                              h_out, nullptr, rstd_out, rows, cols, eps, stream);
}

extern "C" int sph_layernorm(sph_dtype dtype, sph_dtype w_dtype, const void* x,
                             const void* residual, const void* weight,
                             const void* bias, void* y, void* h_out,
                             float* mean_out, float* rstd_out, int64_t rows,
                             int64_t cols, float eps, sph_stream_t stream) {
  return norm_dispatch<true>(dtype, w_dtype, x, residual, weight, bias, y, h_out,
                             mean_out, rstd_out, rows, cols, eps, stream);
}

extern "C" int sph_rmsnorm_f16(const void* x, const void* residual,
                               const void* weight, void* y, void* h_out,
                               int64_t rows, int64_t cols, float eps,
                               sph_stream_t stream) {
  return sph_rmsnorm(SPH_F16, SPH_F16, x, residual, weight, y, h_out, nullptr,
                     rows, cols, eps, stream);
}

extern "C" int sph_layernorm_f16(const void* x, const void* residual,
                                 const void* weight, const void* bias, void* y,
                                 void* h_out, int64_t rows, int64_t cols,
                                 float eps, sph_stream_t stream) {
  return sph_layernorm(SPH_F16, SPH_F16, x, residual, weight, bias, y, h_out,
                       nullptr, nullptr, rows, cols, eps, stream);
}

extern "C" int sph_gelu_affine_rowsum(sph_dtype dtype, const void* x,
                                      const void* s, const void* b,
                                      float s_scalar, float b_scalar, void* y,
                                      void* rowsum, int64_t rows, int64_t cols,
                                      sph_stream_t stream) {
  if (int e = check_rows(rows, cols)) return e;
  if (rows == 0) return SPH_OK;
  hipStream_t st = as_stream(stream);
  switch (dtype) {
    case SPH_F16:
      return gelu_impl<half_t>(x, s, b, s_scalar, b_scalar, y, rowsum, rows, cols, st);
    case SPH_BF16:
      return gelu_impl<bf16_t>(x, s, b, s_scalar, b_scalar, y, rowsum, rows, cols, st);
    case SPH_F32:
      return gelu_impl<float>(x, s, b, s_scalar, b_scalar, y, rowsum, rows, cols, st);
    default:
      return set_error(SPH_ERR_UNSUPPORTED, "gelu_affine_rowsum: unsupported dtype");
  }
}

extern "C" int sph_gelu_affine_rowsum_f16(const void* x, const void* s,
                                          const void* b, void* y, void* rowsum,
                                          int64_t rows, int64_t cols,
                                          sph_stream_t stream) {
  return sph_gelu_affine_rowsum(SPH_F16, x, s, b, 1.0f, 0.0f, y, rowsum, rows,
                                cols, stream);
}
