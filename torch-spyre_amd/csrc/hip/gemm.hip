// fp16 / bf16 GEMM on gfx950 MFMA (v_mfma_f32_16x16x32 in the direct-load
// kernel, v_mfma_f32_32x32x16 elsewhere; {f16,bf16}), fp32 accumulate, with
// an alpha/beta/bias/activation epilogue.
//
// Structure
//   * Workgroup tile BM x BN, K step 64, WM x WN waves; each wave owns a
//     (BM/WM) x (BN/WN) block of 32x32 MFMA tiles whose fp32 accumulators
//     stay in registers for the whole K loop.  Whole 256x256 tiles use 8
//     waves (two per SIMD, so latency hides across waves).
//   * Both operands are staged in LDS "K-contiguous": tile row r (an M row of
//     A or an N column of B) holds its 64 K values as eight 16-byte chunks,
//     chunk c stored at slot c ^ ((r >> 1) & 7), which makes the 16-byte
//     fragment reads and the loaders' 16-byte writes free of bank conflicts
//     on gfx950's 64-bank LDS.
//   * An operand whose K is contiguous in memory (A row-major; B given as
//     B^T row-major, the nn.Linear weight layout) is copied chunk by chunk.
//     An operand whose K is strided (B row-major, A transposed) is loaded as
//     8x8 blocks (eight 16-byte rows) and transposed in registers with byte
//     permutes before the LDS write.
//   * Whole tiles (FULL) run a three-deep pipeline without bounds checks:
//     K tile k is multiplied from one LDS buffer while tile k+1 moves from
//     registers to the other buffer and tile k+2 is loaded from memory.
//     Partial tiles use bounds-checked loaders and a two-deep pipeline.
//   * The epilogue stages each 32-row slab of results in LDS and writes D
//     as whole rows with 16-byte stores; activation and the C term are
//     resolved once per slab, not per element.
//   * Workgroup ids are remapped so that the 8 XCDs (round-robin dispatch)
//     each get a compact group of C tiles, sharing A rows and B columns in
//     their own L2.
//   * Products with at most 16 rows of A whose operands are both
//     K-contiguous (decode steps and LM heads: x[M,K] times an nn.Linear
//     weight W[N,K]) are HBM-bound on reading W once; they run a separate
//     streaming kernel (gemm_skinny_kernel) with packed fp16 dot products
//     instead of MFMA tiles, which would leave most CUs idle at M <= 16.
#include <algorithm>
#include <type_traits>

#include "sph_common.h"

namespace sph {
namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int BK = 64;  // K per LDS stage (eight 16-byte chunks of fp16)

struct GemmArgs {
  int64_t m, n, k;
  const void* a;
  int64_t lda, stride_a;
  const void* b;
  int64_t ldb, stride_b;
  const void* c;
  int64_t ldc_row, ldc_col, stride_c;
  void* d;
  int64_t ldd, stride_d;
  float alpha, beta;
  int epilogue;
  int vec_a, vec_b, vec_d;
  int tiles_m, tiles_n;
  // Split-K tail (direct-load kernel): tiles ranked tail_start.. run as
  // `splits` workgroups each, over kslice K tiles apiece, writing fp32
  // partial tiles to part[(rank - tail_start) * splits + split] that
  // gemm_splitk_reduce sums.  tail_start = the tile count: no split.
  int tail_start, splits, kslice;
  float* part;
  int64_t part_bytes;
  // RMSNorm prologue of the small-M kernels (decode): with norm_w set, row m
  // of A enters the product as A[m] * norm_w * rsqrt(mean(A[m]^2) + norm_eps).
  // The weight multiplies each A chunk as it is loaded (rounded to the
  // element type, as a separate norm kernel's output would be); the row scale
  // multiplies the finished sums, its sum of squares accumulated alongside
  // them from the same loads.
  const void* norm_w;
  float norm_eps;
  // Batch entries (persistent kernels, whose grid does not carry them).
  int64_t batches;
};

template <typename T>
__device__ inline f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c) {
  if constexpr (sizeof(T) == 2 && __is_same(T, half_t)) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(
        __builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(
        __builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
}

// x * w elementwise on 8 packed 2-byte values, each product rounded to T;
// adds the squares of x's values to ss.
template <typename T>
__device__ inline u32x4 norm_chunk(u32x4 x, u32x4 w, float& ss) {
  const T* xe = reinterpret_cast<const T*>(&x);
  const T* we = reinterpret_cast<const T*>(&w);
  u32x4 r;
  T* re = reinterpret_cast<T*>(&r);
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float xf = Num<T>::to_f(xe[e]);
    ss = fmaf(xf, xf, ss);
    re[e] = Num<T>::from_f(xf * Num<T>::to_f(we[e]));
  }
  return r;
}

__device__ inline u32x4 zero4() {
  u32x4 z = {0u, 0u, 0u, 0u};
  return z;
}

// Reads `n` (< 8) two-byte elements with element stride `es` into a chunk,
// zero-filling the rest.
__device__ inline u32x4 load_partial(const uint16_t* p, int n, int64_t es) {
  uint16_t e[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) e[i] = (i < n) ? p[i * es] : static_cast<uint16_t>(0);
  u32x4 r;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    r[i] = static_cast<uint32_t>(e[2 * i]) | (static_cast<uint32_t>(e[2 * i + 1]) << 16);
  return r;
}

// LDS offset (in 2-byte elements) of chunk c of tile row r.  gfx950's LDS
// serves 16 lanes of a 16-byte access per cycle from 64 four-byte banks
// (a 256-byte window): a 128-byte tile row covers one half of the window
// (even rows the low half, odd rows the high half), so the eight rows of
// each parity among 16 consecutive rows must use eight different 16-byte
// slots, which c ^ ((r >> 1) & 7) guarantees for every fixed c.
__device__ inline int lds_off(int r, int c) { return r * BK + ((c ^ ((r >> 1) & 7)) << 3); }

// ---------------------------------------------------------------------------
// Tile loaders: global -> registers (issue) and registers -> LDS (commit).
// `rows` is the tile height (BM for A, BN for B); r0 the first global row
// (M index for A, N index for B); nrows the matrix extent in that dim.
// ---------------------------------------------------------------------------

// K-contiguous operand: element (r, k) at base[r * ld + k].
template <int ROWS, int NT>
struct KContLoader {
  static constexpr int PER_T = (ROWS * 8 + NT - 1) / NT;
  static constexpr int NLOADS = PER_T;  // global loads per issue
  u32x4 reg[PER_T];

  // FULL: the whole tile is in bounds and 16-byte aligned (no checks).
  template <bool FULL>
  __device__ inline void issue(const uint16_t* __restrict__ base, int64_t ld,
                               int64_t r0, int64_t nrows, int64_t k0,
                               int64_t kdim, bool vec) {
    const int t = threadIdx.x;
#pragma unroll
    for (int i = 0; i < PER_T; ++i) {
      const int idx = t + i * NT;
      const int r = idx >> 3, c = idx & 7;
      const int64_t gr = r0 + r, gk = k0 + c * 8;
      if ((ROWS * 8) % NT != 0 && idx >= ROWS * 8) continue;
      if (FULL || (gr < nrows && vec && gk + 8 <= kdim)) {
        reg[i] = *reinterpret_cast<const u32x4*>(base + gr * ld + gk);
      } else if (gr < nrows && gk < kdim) {
        const int64_t n = kdim - gk;
        reg[i] = load_partial(base + gr * ld + gk, n > 8 ? 8 : static_cast<int>(n), 1);
      } else {
        reg[i] = zero4();
      }
    }
  }

  __device__ inline void commit(uint16_t* __restrict__ lds) const {
    const int t = threadIdx.x;
#pragma unroll
    for (int i = 0; i < PER_T; ++i) {
      const int idx = t + i * NT;
      if ((ROWS * 8) % NT != 0 && idx >= ROWS * 8) continue;
      const int r = idx >> 3, c = idx & 7;
      *reinterpret_cast<u32x4*>(lds + lds_off(r, c)) = reg[i];
    }
  }
};

// K-strided operand: element (r, k) at base[k * ld + r].  Loaded as 8x8
// blocks: block (rb, kb) covers rows 8rb..8rb+7 and k 8kb..8kb+7; the 8
// global loads are along r (16 bytes each), the block is transposed in
// registers so each LDS write is one 16-byte K chunk of one row.
template <int ROWS, int NT>
struct KStridedLoader {
  static constexpr int NB = ROWS;  // (ROWS / 8) r-blocks x 8 k-blocks
  static constexpr int PER_T = (NB + NT - 1) / NT;
  static constexpr int NLOADS = PER_T * 8;
  u32x4 reg[PER_T][8];

  template <bool FULL>
  __device__ inline void issue(const uint16_t* __restrict__ base, int64_t ld,
                               int64_t r0, int64_t nrows, int64_t k0,
                               int64_t kdim, bool vec) {
    const int t = threadIdx.x;
#pragma unroll
    for (int i = 0; i < PER_T; ++i) {
      const int idx = t + i * NT;
      if (NB % NT != 0 && idx >= NB) continue;
      const int kb = idx & 7, rb = idx >> 3;
      const int64_t gr = r0 + rb * 8;
#pragma unroll
      for (int kr = 0; kr < 8; ++kr) {
        const int64_t gk = k0 + kb * 8 + kr;
        if (FULL || (gk < kdim && vec && gr + 8 <= nrows)) {
          reg[i][kr] = *reinterpret_cast<const u32x4*>(base + gk * ld + gr);
        } else if (gk < kdim && gr < nrows) {
          const int64_t n = nrows - gr;
          reg[i][kr] = load_partial(base + gk * ld + gr, n > 8 ? 8 : static_cast<int>(n), 1);
        } else {
          reg[i][kr] = zero4();
        }
      }
    }
  }

  __device__ inline void commit(uint16_t* __restrict__ lds) const {
    const int t = threadIdx.x;
#pragma unroll
    for (int i = 0; i < PER_T; ++i) {
      const int idx = t + i * NT;
      if (NB % NT != 0 && idx >= NB) continue;
      const int kb = idx & 7, rb = idx >> 3;
      // reg[i][kr] dword q holds rows (2q, 2q+1) of k row kr.  Output row j
      // (= r offset) dword p holds k values (2p, 2p+1).  Lanes of odd r
      // blocks write rows in the order 1,0,3,2,... so that the 16 lanes of
      // one LDS write cycle (two r blocks) cover rows of both parities.
      const int flip = rb & 1;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int jj = j ^ flip;
        const uint32_t sel = (jj & 1) ? 0x07060302u : 0x05040100u;
        u32x4 o;
#pragma unroll
        for (int p = 0; p < 4; ++p) {
          const uint32_t lo = reg[i][2 * p][j >> 1];
          const uint32_t hi = reg[i][2 * p + 1][j >> 1];
          o[p] = __builtin_amdgcn_perm(hi, lo, sel);
        }
        const int r = rb * 8 + jj;
        *reinterpret_cast<u32x4*>(lds + lds_off(r, kb)) = o;
      }
    }
  }
};

template <bool KCONT, int ROWS, int NT>
struct LoaderSel;
template <int ROWS, int NT>
struct LoaderSel<true, ROWS, NT> {
  using type = KContLoader<ROWS, NT>;
};
template <int ROWS, int NT>
struct LoaderSel<false, ROWS, NT> {
  using type = KStridedLoader<ROWS, NT>;
};


// Maps the linear workgroup id to a (tile_m, tile_n) pair: ids are first
// regrouped so that consecutive ids run on one XCD (dispatch is round-robin
// over 8 XCDs), then walked in GROUP_M-row bands for L2 reuse.
__device__ inline void tile_of(int bid, int tiles_m, int tiles_n, int& tm, int& tn) {
  const int nt = tiles_m * tiles_n;
  if ((nt & 7) == 0) bid = (bid & 7) * (nt >> 3) + (bid >> 3);
  constexpr int GROUP_M = 4;
  const int per_group = GROUP_M * tiles_n;
  const int g = bid / per_group;
  const int first_m = g * GROUP_M;
  const int gm = (tiles_m - first_m) < GROUP_M ? (tiles_m - first_m) : GROUP_M;
  const int in_g = bid - g * per_group;
  tm = first_m + in_g % gm;
  tn = in_g / gm;
}

// Writes one 32 x WTN slab of fp32 results (LDS, row pitch EPITCH floats)
// to D rows row0.., columns col0.. as D = epi(alpha * slab + beta * C).
// Lane l handles columns 8*(l % (WTN/8)) .. +7 of rows l / (WTN/8) + k*RPP.
// The activation and the C term are resolved outside the row loop.  A
// row-major C with 16-byte aligned rows (a residual, or a bias row with
// ldc_row 0) is read 16 bytes a lane, every row of the slab before the
// first store, so the slab waits for one C load latency instead of one per
// row (2048 x 4096 x 4096 + residual in 128-wide tiles: 76 -> 64 us).
template <typename T, int EPI, bool USE_C, int WTN, int EPITCH>
__device__ __attribute__((always_inline)) inline void store_slab_impl(const GemmArgs& p, const float* slab, T* D,
                                       const T* C, int64_t row0, int64_t col0,
                                       int lane) {
  constexpr int LPR = WTN / 8;   // lanes per row
  constexpr int RPP = 64 / LPR;  // rows per pass (48-wide slabs: 10, lanes 60-63 idle)
  const int er = lane / LPR, ec = (lane % LPR) * 8;
  const int64_t col = col0 + ec;
  if (er >= RPP || col >= p.n) return;
  const bool full_cols = p.vec_d && col + 8 <= p.n;
  const int ncols = p.n - col >= 8 ? 8 : static_cast<int>(p.n - col);
  // Lanes whose 8-column group has bit 3 set read the two 16-byte halves
  // in the opposite order, so each LDS read cycle touches 64 distinct banks.
  const int sw = (lane >> 3) & 1;
  // one row: cv holds the row's 8 C values as 16 bytes when vec_c (else C
  // is read element by element, when there is a C term)
  auto row_out = [&](int rr, int64_t row, u32x4 cv, bool vec_c) __attribute__((always_inline)) {
    const u32x4* sp = reinterpret_cast<const u32x4*>(slab + rr * EPITCH + ec);
    const u32x4 h0 = sp[sw], h1 = sp[sw ^ 1];
    float v[8];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[e] = __uint_as_float(sw ? h1[e] : h0[e]);
      v[e + 4] = __uint_as_float(sw ? h0[e] : h1[e]);
    }
    float cf[8];
    if constexpr (USE_C) {
      if (vec_c) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const uint32_t b16 = (cv[e >> 1] >> (16 * (e & 1))) & 0xffffu;
          if constexpr (__is_same(T, bf16_t))
            cf[e] = __uint_as_float(b16 << 16);
          else
            cf[e] = static_cast<float>(__builtin_bit_cast(half_t, static_cast<uint16_t>(b16)));
        }
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e)
          cf[e] = e < ncols ? Num<T>::to_f(C[row * p.ldc_row + (col + e) * p.ldc_col]) : 0.f;
      }
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float x = p.alpha * v[e];
      if constexpr (USE_C) x += p.beta * cf[e];
      if constexpr (EPI == SPH_EPI_RELU) x = fmaxf(x, 0.f);
      if constexpr (EPI == SPH_EPI_GELU) x = gelu_erf(x);
      if constexpr (EPI == SPH_EPI_SILU) x = silu(x);
      v[e] = x;
    }
    T* dp = D + row * p.ldd + col;
    // streaming stores: a launch's tiles tend to finish together, so the
    // output leaves in one burst (4096^3: 1305-1316 -> 1335-1337 TFLOP/s,
    // alternating builds on one box; the c4 / c5 decoder unchanged)
    if (full_cols)
      store8<T, true>(dp, v);
    else
      store8_partial<T>(dp, ncols, v);
  };
  if constexpr (USE_C && sizeof(T) == 2) {
    if (full_cols && p.ldc_col == 1 && (p.ldc_row & 7) == 0 &&
        (reinterpret_cast<uintptr_t>(C) & 15) == 0) {
      constexpr int NR = (32 + RPP - 1) / RPP;  // row passes per slab
      u32x4 cq[NR];
#pragma unroll
      for (int i = 0; i < NR; ++i) {
        const int rr = er + i * RPP;
        if (rr < 32 && row0 + rr < p.m)
          cq[i] = *reinterpret_cast<const u32x4*>(C + (row0 + rr) * p.ldc_row + col);
      }
#pragma unroll
      for (int i = 0; i < NR; ++i) {
        const int rr = er + i * RPP;
        if (rr < 32 && row0 + rr < p.m) row_out(rr, row0 + rr, cq[i], true);
      }
      return;
    }
  }
#pragma unroll 1
  for (int rr = er; rr < 32; rr += RPP) {
    const int64_t row = row0 + rr;
    if (row >= p.m) break;
    row_out(rr, row, u32x4{0, 0, 0, 0}, false);
  }
}

// Calls f(std::integral_constant<int, E>, std::bool_constant<USE_C>) for the
// call's activation E and C term, so that a kernel's epilogue loop (which
// calls store_slab_impl<T, E, USE_C, ..> per 32-row slab) is instantiated
// once per case.  With the choice made inside the loop instead, the bf16
// loop bodies grew past the unroller's limit and the accumulators, indexed
// by the slab number, were kept in scratch memory.
template <typename F>
__device__ inline void epi_dispatch(const GemmArgs& p, const void* c, F&& f) {
  const bool use_c = c != nullptr && p.beta != 0.f;
#define SPH_EPI_CASE(E)                                                            \
  if (use_c)                                                                       \
    f(std::integral_constant<int, E>{}, std::true_type{});                         \
  else                                                                             \
    f(std::integral_constant<int, E>{}, std::false_type{});
  switch (p.epilogue) {
    case SPH_EPI_RELU:
      SPH_EPI_CASE(SPH_EPI_RELU);
      break;
    case SPH_EPI_GELU:
      SPH_EPI_CASE(SPH_EPI_GELU);
      break;
    case SPH_EPI_SILU:
      SPH_EPI_CASE(SPH_EPI_SILU);
      break;
    default:
      SPH_EPI_CASE(SPH_EPI_NONE);
  }
#undef SPH_EPI_CASE
}

// Reads the MFMA fragments of K sub-step kk (16 K values) for this wave.
template <int TM, int TN, int WTM, int WTN>
__device__ inline void load_frags(const uint16_t* __restrict__ sa,
                                  const uint16_t* __restrict__ sb, int wm,
                                  int wn, int row_in, int khalf, int kk,
                                  u32x4 (&af)[TM], u32x4 (&bf)[TN]) {
  const int c = kk * 2 + khalf;
#pragma unroll
  for (int i = 0; i < TM; ++i)
    af[i] = *reinterpret_cast<const u32x4*>(sa + lds_off(wm * WTM + i * 32 + row_in, c));
#pragma unroll
  for (int j = 0; j < TN; ++j)
    bf[j] = *reinterpret_cast<const u32x4*>(sb + lds_off(wn * WTN + j * 32 + row_in, c));
}

template <typename T, int BM, int BN, int WM, int WN, bool A_KCONT, bool B_KCONT,
          bool FULL>
__global__ void __launch_bounds__(WM * WN * 64)
gemm_kernel(const GemmArgs p) {
  constexpr int NT = WM * WN * 64;
  constexpr int WTM = BM / WM, WTN = BN / WN;  // wave tile
  constexpr int TM = WTM / 32;                 // 32x32 MFMA tiles per wave along M
  constexpr int TN = WTN / 32;
  constexpr int STAGE = (BM + BN) * BK;        // LDS elements per pipeline stage
  // Epilogue staging: per wave one 32-row slab of fp32 accumulators, rows
  // padded by 8 floats so the two half-waves' rows land on different banks.
  constexpr int EPITCH = WTN + 8;
  static_assert(TM >= 1 && TN >= 1, "wave tile too small");
  static_assert(WM * WN * 32 * EPITCH * 4 <= 2 * STAGE * 2, "epilogue staging exceeds LDS");
  __shared__ __attribute__((aligned(16))) uint16_t lds[2 * STAGE];

  int tm, tn;
  tile_of(blockIdx.x, p.tiles_m, p.tiles_n, tm, tn);
  const int64_t batch = blockIdx.y;
  const uint16_t* A = static_cast<const uint16_t*>(p.a) + batch * p.stride_a;
  const uint16_t* B = static_cast<const uint16_t*>(p.b) + batch * p.stride_b;
  const int64_t m0 = static_cast<int64_t>(tm) * BM;
  const int64_t n0 = static_cast<int64_t>(tn) * BN;

  typename LoaderSel<A_KCONT, BM, NT>::type la;
  typename LoaderSel<B_KCONT, BN, NT>::type lb;

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int row_in = lane & 31;  // fragment row within a 32x32 tile
  const int khalf = lane >> 5;   // which 8-wide K half of a 16-K step

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  const int64_t ksteps = (p.k + BK - 1) / BK;
  if constexpr (FULL) {
    // Three-deep pipeline over K tiles: while the MFMAs consume tile ks
    // from LDS buffer ks&1, tile ks+1 (loaded into registers during the
    // previous step) is written to the other buffer, and tile ks+2 is
    // loaded from global memory into the freed registers.  Global loads
    // thus have a whole K step to land and the LDS writes never wait.
    // The body is branch-free (one scheduling region): indices past the
    // last tile are clamped, re-loading and re-writing the last tile into
    // the idle buffer, which nothing reads afterwards.
    const int64_t klast = (ksteps - 1) * BK;
    la.template issue<true>(A, p.lda, m0, p.m, 0, p.k, true);
    lb.template issue<true>(B, p.ldb, n0, p.n, 0, p.k, true);
    la.commit(lds);
    lb.commit(lds + BM * BK);
    const int64_t k1 = BK < klast ? BK : klast;
    la.template issue<true>(A, p.lda, m0, p.m, k1, p.k, true);
    lb.template issue<true>(B, p.ldb, n0, p.n, k1, p.k, true);
    __syncthreads();
    for (int64_t ks = 0; ks < ksteps; ++ks) {
      const int cur = static_cast<int>(ks & 1);
      const uint16_t* sa = lds + cur * STAGE;
      const uint16_t* sb = sa + BM * BK;
      u32x4 af[2][TM], bf[2][TN];
      load_frags<TM, TN, WTM, WTN>(sa, sb, wm, wn, row_in, khalf, 0, af[0], bf[0]);
#pragma unroll
      for (int kk = 0; kk < BK / 16; ++kk) {
        if (kk + 1 < BK / 16)
          load_frags<TM, TN, WTM, WTN>(sa, sb, wm, wn, row_in, khalf, kk + 1,
                                       af[(kk + 1) & 1], bf[(kk + 1) & 1]);
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j)
            acc[i][j] = mfma32<T>(af[kk & 1][i], bf[kk & 1][j], acc[i][j]);
      }
      la.commit(lds + (cur ^ 1) * STAGE);
      lb.commit(lds + (cur ^ 1) * STAGE + BM * BK);
      const int64_t k2 = (ks + 2) * BK < klast ? (ks + 2) * BK : klast;
      la.template issue<true>(A, p.lda, m0, p.m, k2, p.k, true);
      lb.template issue<true>(B, p.ldb, n0, p.n, k2, p.k, true);
      // Instruction order for the scheduler (one wave per SIMD, so latency
      // must be hidden inside the wave): fragment reads of sub-step 0;
      // sub-steps 0-2 alternate MFMAs with the next sub-step's fragment
      // reads; sub-step 3 interleaves each MFMA with the register
      // transposes, LDS writes and global loads of the pipeline.
      constexpr int NMF = TM * TN, NDS = TM + TN;
      constexpr int NVM = decltype(la)::NLOADS + decltype(lb)::NLOADS;
      constexpr int IO_PER = (NVM + NMF - 1) / NMF;  // one LDS write per global load
      // Sub-step kk's MFMAs run only after all fragment reads of sub-step
      // kk+1 were issued, so those reads overlap a whole sub-step of MFMAs.
      // (With two or more waves per SIMD the hardware interleaves waves and
      // the compiler's own order is kept.)
      if constexpr (WM * WN == 4) {
      __builtin_amdgcn_sched_group_barrier(0x100, 2 * NDS, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, NMF, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, NDS, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, NMF, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, NDS, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, NMF, 0);
#pragma unroll
      for (int x = 0; x < NMF; ++x) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);
        __builtin_amdgcn_sched_group_barrier(0x200, IO_PER, 0);
        __builtin_amdgcn_sched_group_barrier(0x020, IO_PER, 0);
      }
      }
      __syncthreads();
    }
  } else {
    if (ksteps > 0) {
      la.template issue<false>(A, p.lda, m0, p.m, 0, p.k, p.vec_a);
      lb.template issue<false>(B, p.ldb, n0, p.n, 0, p.k, p.vec_b);
      la.commit(lds);
      lb.commit(lds + BM * BK);
      __syncthreads();
    }
    for (int64_t ks = 0; ks < ksteps; ++ks) {
      const int cur = static_cast<int>(ks & 1);
      const bool more = ks + 1 < ksteps;
      if (more) {
        la.template issue<false>(A, p.lda, m0, p.m, (ks + 1) * BK, p.k, p.vec_a);
        lb.template issue<false>(B, p.ldb, n0, p.n, (ks + 1) * BK, p.k, p.vec_b);
      }
      const uint16_t* sa = lds + cur * STAGE;
      const uint16_t* sb = sa + BM * BK;
      u32x4 af[2][TM], bf[2][TN];
      load_frags<TM, TN, WTM, WTN>(sa, sb, wm, wn, row_in, khalf, 0, af[0], bf[0]);
#pragma unroll
      for (int kk = 0; kk < BK / 16; ++kk) {
        if (kk + 1 < BK / 16)
          load_frags<TM, TN, WTM, WTN>(sa, sb, wm, wn, row_in, khalf, kk + 1,
                                       af[(kk + 1) & 1], bf[(kk + 1) & 1]);
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j)
            acc[i][j] = mfma32<T>(af[kk & 1][i], bf[kk & 1][j], acc[i][j]);
      }
      if (more) {
        la.commit(lds + (cur ^ 1) * STAGE);
        lb.commit(lds + (cur ^ 1) * STAGE + BM * BK);
      }
      __syncthreads();
    }
  }

  // Epilogue.  Accumulator register r of tile (i, j) holds row
  // 8*(r/4) + 4*(lane/32) + r%4, column lane%32 of that 32x32 tile.  Each
  // 32-row slab of the wave tile goes through LDS so that the output is
  // written as whole rows with 16-byte stores.
  T* D = static_cast<T*>(p.d) + batch * p.stride_d;
  const T* C = p.c ? static_cast<const T*>(p.c) + batch * p.stride_c : nullptr;
  float* slab = reinterpret_cast<float*>(lds) + wave * (32 * EPITCH);
  const int64_t row0 = m0 + wm * WTM;
  const int64_t colw = n0 + wn * WTN;
  epi_dispatch(p, C, [&](auto epi_, auto use_c_) {
    constexpr int E = decltype(epi_)::value;
    constexpr bool UC = decltype(use_c_)::value;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          slab[((r >> 2) * 8 + (lane >> 5) * 4 + (r & 3)) * EPITCH + j * 32 + (lane & 31)] =
              acc[i][j][r];
      __syncthreads();
      store_slab_impl<T, E, UC, WTN, EPITCH>(p, slab, D, C, row0 + i * 32, colw, lane);
      __syncthreads();
    }
  });
}

// ---------------------------------------------------------------------------
// Whole 256-row tiles (256, 192 or 128 columns) with A K-contiguous: direct
// global -> LDS loads.
//
//   * Each 64-deep K tile moves from memory into LDS with
//     buffer_load_dwordx4 ... lds: no VGPR staging and no LDS write
//     instructions.  Lane l's 16 bytes land at line base + 16 l (one 1 KB
//     line per instruction), so the swizzled LDS layout is produced by
//     choosing which 16 global bytes each lane fetches.  The loads are
//     raw-buffer loads whose range ends where the tile's operand rows end:
//     an offset past it reads zeros instead of touching other memory.
//   * A (and a K-contiguous B) sits K-contiguous in LDS with the swizzle of
//     the register-staged kernel.  A row-major B ([K, N], N contiguous) sits
//     as 64 K rows of 256 N values; its MFMA fragments are read with
//     ds_read_b64_tr_b16, which works on groups of 16 lanes: lane 4e + q
//     points at 4 consecutive values of one row and lane i receives value
//     i % 4 of the rows addressed by lanes i / 4, 4 + i / 4, 8 + i / 4,
//     12 + i / 4.  Pointing lane 4e + q at (k0 + e, n0 + 4q) therefore gives
//     lane i the column n0 + i at k0 .. k0 + 3, half of a B fragment.  Row
//     k's 16-byte chunk c is stored at slot c ^ bswz(k) (4 (k & 3) + 2
//     (bit 3 of k)): the 8 rows x 2 chunks a half-wave reads then cover all
//     64 banks.  (With c ^ 4 (k & 3) alone, rows k and k + 8 share banks:
//     27 % of the LDS-active cycles were bank conflicts.)
//   * 16x16x32 MFMAs (v_mfma_f32_16x16x32_{f16,bf16}), not 32x32x16: the
//     same FLOPs per LDS byte for a given wave tile, but a quarter of the
//     accumulator registers per instruction.  This part runs the GEMM at
//     its power limit, and a loop of nothing but MFMAs sustains 2006
//     TFLOP/s with 16x16x32 against 1705 with 32x32x16 (8 waves per CU,
//     random operands); the kernel gained 5-10 % on every measured shape.
//   * Two LDS stages.  The K step is ordered by hand (sched_barrier): each of
//     the two 32-deep MFMA sub-steps issues its 32 MFMAs interleaved with
//     the LDS reads of the next sub-step's fragments (B first, each A tile
//     right after this sub-step's last use of the same A index).  Early in
//     sub-step 1 a wave waits for its own DMA of the next tile and its own
//     LDS reads, then joins the barrier; the rest of sub-step 1 issues the
//     DMA of the tile after next into the stage just vacated (one line
//     every two or three MFMAs: ~1 % faster than back to back) and reads
//     the next tile's first fragments.  Past the last tile the DMA re-loads the
//     last tile and the fragment reads fetch values nobody uses, so the
//     loop has no branches.
//   * The DMA is issued from inline asm: as an intrinsic, the compiler waits
//     for every outstanding LDS DMA before any later LDS read (it cannot tell
//     the stages apart), which would serialise load and compute.  Completion
//     is awaited explicitly (vmcnt) before the barrier.
//   * 8 waves (2 x 4, two per SIMD), each owning a 128 x 64 block of 16x16
//     MFMA tiles (128 x 48 on 192-wide tiles, 128 x 32 on 128-wide ones);
//     epilogue as in the register-staged kernel.
// ---------------------------------------------------------------------------
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
#define SPH_LDS __attribute__((address_space(3)))

// Raw buffer resource over [base, base + bytes) (stride 0; gfx9 dword 3).
__device__ inline i32x4 buffer_rsrc(const void* base, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  i32x4 r;
  r[0] = __builtin_amdgcn_readfirstlane(static_cast<int32_t>(static_cast<uint32_t>(a)));
  r[1] = __builtin_amdgcn_readfirstlane(static_cast<int32_t>(static_cast<uint32_t>(a >> 32) & 0xffffu));
  r[2] = __builtin_amdgcn_readfirstlane(static_cast<int32_t>(bytes));
  r[3] = 0x00020000;
  return r;
}

// 16 bytes per lane from rsrc[voff + soff] into LDS at lds_addr + 16 * lane.
__device__ inline void dma16(i32x4 rsrc, uint32_t lds_addr, uint32_t voff, uint32_t soff) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
               :
               : "s"(lds_addr), "v"(voff), "s"(rsrc), "s"(soff)
               : "memory", "m0");
}
template <int N>
__device__ inline void wait_vmcnt() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
__device__ inline void wait_lgkmcnt0() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

namespace dl {
// Shared by both tile widths: 256-row tiles, 64-deep K tiles, two waves
// along M, each wave owning a 128 x 64 block of 16x16 MFMA tiles
// (v_mfma_f32_16x16x32: two 32-deep sub-steps per K tile).
constexpr int BM = 256, BKD = 64, WM = 2, WTM = 128, WTN = 64, TM = WTM / 16;
constexpr int CPR = BKD / 8;                    // 16-byte chunks per K row
constexpr int A_BYTES = BM * BKD * 2;
constexpr int KK = BKD / 32;                     // MFMA sub-steps per K tile
// K-contiguous row r, chunk c -> 16-byte slot (c ^ ((r >> 1) & 7)).
__device__ inline int kslot(int r, int c) { return r * CPR + (c ^ ((r >> 1) & 7)); }
// Row-major B: K row k's 16-byte chunk c sits at slot c ^ bswz(k).  A
// transposing read's 32-lane half covers rows k0 .. k0 + 3 and k0 + 8 ..
// k0 + 11 (k0 a multiple of 4 with bit 3 clear) at the same two chunks:
// bits 2-3 of the XOR spread the four rows of a lane group over the 256
// bytes of banks, bit 1 moves the second group's rows to the other half.
__device__ inline int bswz(int k) { return 4 * (k & 3) + 2 * ((k >> 3) & 1); }

// BN = 256 with 128 x 64 wave tiles (8 waves, 2 x 4), 192 with WTN_ = 48
// (8 waves of 128 x 48, K-contiguous B only) or 128 with WTN_ = 32 (8 waves
// of 128 x 32).  (128-wide tiles on 4 waves of 128 x 64 measured 20-28 %
// slower than on 8 of 128 x 32, e.g. 869 against 1074 TFLOP/s at 2048 x
// 4096 x 4096: with one wave per SIMD the compiler keeps the accumulators in
// AGPRs and copies each through VGPRs on every K tile.)
// (WTN_ = 128, 128 x 128 wave tiles with 256 accumulator registers, one
// wave per SIMD on a 256-wide tile, reads a third less from LDS per MFMA
// but measured slower: 2-3 % with 32x32x16 MFMAs, 30 % with 16x16x32 ones,
// whose accumulators the compiler then moves between register files inside
// the loop; one wave per SIMD also hides less of the K-tile barrier and the
// LDS latency.)
template <int BN_, int WTN_ = WTN>
struct Cfg {
  static constexpr int WTN = WTN_, TN = WTN / 16, NMF = TM * TN, EPITCH = WTN + 8;
  static constexpr int BN = BN_, WN = BN / WTN, NW = WM * WN, NT = NW * 64;
  static constexpr int B_BYTES = BN * BKD * 2, STAGE = A_BYTES + B_BYTES;
  static constexpr int LPA = A_BYTES / 1024 / NW, LPB = B_BYTES / 1024 / NW;  // DMA lines per wave
  static constexpr int BCH = BN / 8;             // 16-byte chunks per row-major B row
  static_assert(LPA * NW * 1024 == A_BYTES && LPB * NW * 1024 == B_BYTES, "DMA lines");
  // the K-tile barrier comes before MFMA XB of the last sub-step
  static constexpr int XB = 8 < NMF - LPA - LPB ? 8 : NMF - LPA - LPB;
  static_assert(XB >= TN - 1, "barrier after the last reads of the stage");
  // the DMA lines after the barrier go out one every DSP MFMAs
  static constexpr int DSP = (NMF - XB) / (LPA + LPB) < 3 ? (NMF - XB) / (LPA + LPB) : 3;
  static_assert(DSP >= 1, "DMA fits in the post-barrier sub-step");
  static_assert(NW * 32 * EPITCH * 4 <= 2 * STAGE, "epilogue staging exceeds LDS");
};
}  // namespace dl

template <typename T>
__device__ inline f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
  if constexpr (__is_same(T, half_t)) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(
        __builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(
        __builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
}

// SWIGLU: B holds the gate rows [0, n) and the up rows [n, 2n) of one
// weight matrix (K-contiguous) and D[m, j] = silu(A B_gate[j]) * (A B_up[j]).
// A 256-wide tile then covers 128 output columns: in the 64 columns of wave
// wn, MFMA tiles 0 and 1 take gate rows j0 + 32 wn .. + 31 and tiles 2 and 3
// the up rows of the same columns, so a lane's accumulators j and j + 2
// hold the gate and up sums of the same output element and the epilogue
// combines them in registers.
template <typename T, bool B_KCONT, int BN_, bool SWIGLU = false, int WTN_ = dl::WTN>
__global__ void __launch_bounds__((dl::Cfg<BN_, WTN_>::NT)) gemm_dl_kernel(const GemmArgs p) {
  using namespace dl;
  using DC = Cfg<BN_, WTN_>;
  constexpr int WTN = DC::WTN, TN = DC::TN, NMF = DC::NMF, EPITCH = DC::EPITCH;
  static_assert(!SWIGLU || (B_KCONT && BN_ == 256), "SwiGLU tiles: K-contiguous B, 256 wide");
  static_assert(B_KCONT || (BN_ / 8) % 16 == 0, "row-major B: the swizzle needs 16-chunk row groups");
  constexpr int BN = DC::BN, WN = DC::WN, STAGE = DC::STAGE, LPA = DC::LPA, LPB = DC::LPB;
  constexpr int NBR = B_KCONT ? 1 : 2;           // LDS reads per B fragment
  constexpr int XB = DC::XB;                     // barrier before this MFMA of the last sub-step
  __shared__ __attribute__((aligned(1024))) char lds[2 * STAGE];

  // Tile rank and K slice: workgroups past tail_start are split-K slices of
  // the tail tiles.
  int rank = blockIdx.x, split = 0;
  const bool partial = rank >= p.tail_start;
  if (partial) {
    const int q = rank - p.tail_start;
    rank = p.tail_start + q / p.splits;
    split = q % p.splits;
  }
  int tm, tn;
  tile_of(rank, p.tiles_m, p.tiles_n, tm, tn);
  const int64_t batch = blockIdx.y;
  // first output column (SwiGLU: 128 output columns per tile)
  const int64_t m0 = static_cast<int64_t>(tm) * BM, n0 = static_cast<int64_t>(tn) * (SWIGLU ? BN / 2 : BN);
  const uint16_t* A = static_cast<const uint16_t*>(p.a) + batch * p.stride_a;
  const uint16_t* B = static_cast<const uint16_t*>(p.b) + batch * p.stride_b;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int lda = static_cast<int>(p.lda), ldb = static_cast<int>(p.ldb);
  const int ksteps_all = static_cast<int>(p.k / BKD);
  const int kt0 = partial ? split * p.kslice : 0;  // first K tile of this workgroup
  const int ksteps = partial ? min(p.kslice, ksteps_all - kt0) : ksteps_all;

  // Buffer ranges: exactly the bytes this tile's rows (columns) span.
  const i32x4 ra = buffer_rsrc(A + m0 * lda, static_cast<uint32_t>(((BM - 1) * static_cast<int64_t>(lda) + p.k) * 2));
  // (SwiGLU: from gate row n0 to up row n + n0 + 127)
  const i32x4 rb = SWIGLU
      ? buffer_rsrc(B + n0 * ldb, static_cast<uint32_t>(((p.n + BN / 2 - 1) * static_cast<int64_t>(ldb) + p.k) * 2))
      : B_KCONT
      ? buffer_rsrc(B + n0 * ldb, static_cast<uint32_t>(((BN - 1) * static_cast<int64_t>(ldb) + p.k) * 2))
      : buffer_rsrc(B + n0, static_cast<uint32_t>(((p.k - 1) * ldb + BN) * 2));
  // Per-lane global byte offsets of this wave's DMA lines (K tile 0).
  uint32_t va[LPA], vb[LPB];
#pragma unroll
  for (int i = 0; i < LPA; ++i) {
    const int s = (wave * LPA + i) * 64 + lane;  // LDS slot filled by this lane
    const int r = s / CPR, c = (s % CPR) ^ ((r >> 1) & 7);
    va[i] = static_cast<uint32_t>(r * lda * 2 + c * 16);
  }
#pragma unroll
  for (int i = 0; i < LPB; ++i) {
    const int s = (wave * LPB + i) * 64 + lane;
    if constexpr (SWIGLU) {
      // LDS row r (tile column) -> weight row: gate j0 + 32 (r / 64) + r % 32
      // for r % 64 < 32, else the matching up row (+ n)
      const int r = s / CPR, c = (s % CPR) ^ ((r >> 1) & 7);
      const int64_t wr = 32 * (r >> 6) + (r & 31) + ((r & 32) ? p.n : 0);
      vb[i] = static_cast<uint32_t>(wr * ldb * 2 + c * 16);
    } else if constexpr (B_KCONT) {
      const int r = s / CPR, c = (s % CPR) ^ ((r >> 1) & 7);
      vb[i] = static_cast<uint32_t>(r * ldb * 2 + c * 16);
    } else {
      const int k = s / DC::BCH, c = (s % DC::BCH) ^ bswz(k);
      vb[i] = static_cast<uint32_t>(k * ldb * 2 + c * 16);
    }
  }
  const uint32_t lds_base = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((SPH_LDS char*)(lds)));
  // Fragment reads.  16x16x32 operands: lane l holds row (column) l % 16 and
  // the 8 K values 8 (l / 16) .. + 7 of the sub-step, one 16-byte chunk of a
  // K-contiguous row: chunk 4 kk + l / 16, whose slot is swizzled by
  // (r >> 1) & 7 = (l % 16 >> 1) & 7 for every tile (tiles start at rows that
  // are multiples of 16), so offset(kk, tile t) = off[kk] + 2048 t.
  const int m16 = lane & 15, g4 = lane >> 4, sw = g4 ^ ((m16 >> 1) & 7);
  int aoff[KK], bkoff[KK];
#pragma unroll
  for (int kk = 0; kk < KK; ++kk) {
    aoff[kk] = (wm * WTM + m16) * (CPR * 16) + ((sw ^ (4 * kk)) << 4);
    bkoff[kk] = A_BYTES + (wn * WTN + m16) * (CPR * 16) + ((sw ^ (4 * kk)) << 4);
  }
  // Row-major B: two transposing reads per fragment.  ds_read_b64_tr_b16
  // has each 16-lane group read a 4 x 16 block (lane e * 4 + q: row e,
  // columns 4q .. 4q + 3) and hands lane m column m of it; group g4 reads K
  // rows 32 kk + 8 g4 + 4 h + e of the fragment's 16 columns.
  int boff[TN];
  {
    const int e = m16 >> 2, q = m16 & 3;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int n = wn * WTN + j * 16 + 4 * q;
      boff[j] = A_BYTES + (8 * g4 + e) * (BN * 2) + (((n >> 3) ^ bswz(8 * g4 + e)) << 4) + 8 * (q & 1);
    }
  }

  f32x4 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  u32x4 af[2][TM];
  u32x2 bl[2][TN], bh[2][TN];

// Fragment reads of sub-step KK_ from the stage at byte offset STB_ into
// buffer BUF_: A tile I_; B fragment read X_ (K-contiguous: fragment X_;
// row-major: fragment X_ / 2, half X_ % 2).
#define SPH_DL_READ_A(BUF_, I_, STB_, KK_)                                                  \
  af[BUF_][I_] = *reinterpret_cast<const u32x4*>(lds + (STB_) + aoff[KK_] + (I_) * 2048)
#define SPH_DL_READ_B(BUF_, X_, STB_, KK_)                                                  \
  do {                                                                                      \
    if constexpr (B_KCONT) {                                                                \
      const u32x4 v_ =                                                                      \
          *reinterpret_cast<const u32x4*>(lds + (STB_) + bkoff[KK_] + (X_) * 2048);         \
      bl[BUF_][X_] = u32x2{v_[0], v_[1]};                                                   \
      bh[BUF_][X_] = u32x2{v_[2], v_[3]};                                                   \
    } else {                                                                                \
      const int j_ = (X_) >> 1, h_ = (X_) & 1;                                              \
      const SPH_LDS char* p_ = (const SPH_LDS char*)(lds + (STB_)) + boff[j_] +             \
                               ((KK_) * 32 + 4 * h_) * (BN * 2);                            \
      const u32x2 v_ = __builtin_bit_cast(                                                  \
          u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((SPH_LDS s16x4*)(p_)));            \
      if (h_) bh[BUF_][j_] = v_;                                                            \
      else bl[BUF_][j_] = v_;                                                               \
    }                                                                                       \
  } while (0)
// DMA line LINE_ (A lines first, then B) of K tile T_ into stage SL_ & 1.
#define SPH_DL_DMA(T_, SL_, LINE_)                                                          \
  do {                                                                                      \
    const int t_ = (T_), l_ = (LINE_);                                                      \
    const uint32_t sb_ = lds_base + ((SL_) & 1) * STAGE;                                    \
    if (l_ < LPA)                                                                           \
      dma16(ra, __builtin_amdgcn_readfirstlane(sb_ + (wave * LPA + l_) * 1024), va[l_],     \
            __builtin_amdgcn_readfirstlane((kt0 + t_) * BKD * 2));                          \
    else                                                                                    \
      dma16(rb, __builtin_amdgcn_readfirstlane(sb_ + A_BYTES + (wave * LPB + l_ - LPA) * 1024), \
            vb[l_ - LPA],                                                                   \
            __builtin_amdgcn_readfirstlane(B_KCONT ? (kt0 + t_) * BKD * 2                   \
                                                   : (kt0 + t_) * BKD * ldb * 2));          \
  } while (0)

  // Prologue: K tiles 0 and 1 in flight; wait for tile 0; the fragments of
  // its first sub-step.
#pragma unroll
  for (int l = 0; l < LPA + LPB; ++l) SPH_DL_DMA(0, 0, l);
  if (ksteps > 1) {
#pragma unroll
    for (int l = 0; l < LPA + LPB; ++l) SPH_DL_DMA(1, 1, l);
    wait_vmcnt<LPA + LPB>();
  } else {
    wait_vmcnt<0>();
  }
  __syncthreads();
#pragma unroll
  for (int x = 0; x < TN * NBR; ++x) SPH_DL_READ_B(0, x, 0, 0);
#pragma unroll
  for (int i = 0; i < TM; ++i) SPH_DL_READ_A(0, i, 0, 0);

  // Sub-step kk: MFMA x = (A tile x / TN, B fragment x % TN, or TN - 1 -
  // x % TN for odd A tiles).  Its reads of
  // the next sub-step's fragments: the B reads first (the next sub-step's
  // first MFMAs need all of B), each A tile right after the last MFMA that
  // uses this sub-step's A tile of the same index (so the two can share
  // registers).  Before MFMA XB of the last sub-step a wave waits for its own
  // DMA of the next K tile and its own LDS reads, then joins the barrier;
  // after it the sub-step reads the next tile's fragments and issues the DMA
  // of the tile after next into the stage just vacated.  Past the last tile
  // the DMA re-loads the last tile and the fragment reads fetch values nobody
  // uses, so the loop has no branches.
  for (int ks = 0; ks < ksteps; ++ks) {
    const int cs = (ks & 1) * STAGE, ns = ((ks + 1) & 1) * STAGE;
    const int tnext = ks + 2 < ksteps ? ks + 2 : ksteps - 1;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      const bool lastk = kk == KK - 1;
      const int nst = lastk ? ns : cs;           // stage of the next sub-step
      const int nkk = lastk ? 0 : kk + 1;        // and its index
      const int x0 = lastk ? XB : 0;             // first slot of the B reads
#pragma unroll
      for (int x = 0; x < NMF; ++x) {
        // A tile i; B fragments in alternating directions, so consecutive
        // MFMAs across a tile boundary share their B operand (~1 % faster)
        const int i = x / TN, j = (x / TN) & 1 ? TN - 1 - x % TN : x % TN;
        if (lastk && x == XB) {
          wait_vmcnt<0>();
          wait_lgkmcnt0();
          __syncthreads();
        }
        {
          const u32x4 b_ = __builtin_shufflevector(bl[kk & 1][j], bh[kk & 1][j], 0, 1, 2, 3);
          acc[i][j] = mfma16<T>(af[kk & 1][i], b_, acc[i][j]);
        }
        if (x >= x0 && x - x0 < TN * NBR) SPH_DL_READ_B((kk + 1) & 1, x - x0, nst, nkk);
#pragma unroll
        for (int ii = 0; ii < TM; ++ii) {
          // after this sub-step's last use of A tile ii (the last sub-step
          // shifts the reads past the barrier)
          const int last_use = ii * TN + TN - 1;
          const int at = lastk ? min(NMF - 1, last_use + XB - (TN - 1)) : last_use;
          if (x == at) SPH_DL_READ_A((kk + 1) & 1, ii, nst, nkk);
        }
        if (lastk && x >= XB && (x - XB) % DC::DSP == 0 && (x - XB) / DC::DSP < LPA + LPB)
          SPH_DL_DMA(tnext, ks, (x - XB) / DC::DSP);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  }
#undef SPH_DL_READ_A
#undef SPH_DL_READ_B
#undef SPH_DL_DMA

  // Epilogue (LDS reused as fp32 slabs once every DMA has landed).  16x16
  // accumulator r of lane l: row 4 (l / 16) + r, column l % 16 of its tile.
  wait_vmcnt<0>();
  if (partial) {
    // split-K slice: the raw fp32 tile, element (r, c) at r * BN + c
    float* W = p.part + (static_cast<int64_t>(rank - p.tail_start) * p.splits + split) * (BM * BN);
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = wm * WTM + i * 16 + 4 * g4 + r;
          W[row * BN + wn * WTN + j * 16 + m16] = acc[i][j][r];
        }
    return;
  }
  __syncthreads();
  T* D = static_cast<T*>(p.d) + batch * p.stride_d;
  const T* C = p.c ? static_cast<const T*>(p.c) + batch * p.stride_c : nullptr;
  float* slab = reinterpret_cast<float*>(lds) + wave * (32 * EPITCH);
  const int64_t row0 = m0 + wm * WTM;
  auto chunks = [&](auto epi_, auto use_c_) {
    constexpr int E = decltype(epi_)::value;
    constexpr bool UC = decltype(use_c_)::value;
    if constexpr (SWIGLU) {
      // silu(gate) * up per element, 32 output columns per wave
      static_assert(TN == 4, "gate / up tile pairs");
      constexpr int SP = 32 + 8;
      const int64_t colw = n0 + wn * 32;
#pragma unroll
      for (int i2 = 0; i2 < TM / 2; ++i2) {
#pragma unroll
        for (int ii = 0; ii < 2; ++ii)
#pragma unroll
          for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r)
              slab[(ii * 16 + 4 * g4 + r) * SP + j * 16 + m16] =
                  silu(acc[2 * i2 + ii][j][r]) * acc[2 * i2 + ii][j + 2][r];
        __syncthreads();
        store_slab_impl<T, E, UC, 32, SP>(p, slab, D, C, row0 + i2 * 32, colw, lane);
        __syncthreads();
      }
    } else {
      const int64_t colw = n0 + wn * WTN;
#pragma unroll
      for (int i2 = 0; i2 < TM / 2; ++i2) {
#pragma unroll
        for (int ii = 0; ii < 2; ++ii)
#pragma unroll
          for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r)
              slab[(ii * 16 + 4 * g4 + r) * EPITCH + j * 16 + m16] = acc[2 * i2 + ii][j][r];
        __syncthreads();
        store_slab_impl<T, E, UC, WTN, EPITCH>(p, slab, D, C, row0 + i2 * 32, colw, lane);
        __syncthreads();
      }
    }
  };
  epi_dispatch(p, C, chunks);
}

// Sums the split-K slices of one tail tile and applies the epilogue: one
// workgroup per (tail tile, 1024 output elements); each thread takes 4
// consecutive output columns of one row (16-byte reads of every slice).
// SWIGLU: output column oc of the tile is silu(gate) * up with the gate sum
// at tile column 64 (oc / 32) + oc % 32 and the up sum 32 columns further.

template <typename T, int BN, bool SWIGLU>
__global__ void __launch_bounds__(256) gemm_splitk_reduce(const GemmArgs p) {
  constexpr int OUTN = SWIGLU ? BN / 2 : BN;   // output columns per tile
  constexpr int PER_WG = 1024;                  // outputs per workgroup
  const int t = blockIdx.x;                     // tail tile
  const int e = blockIdx.y * PER_WG + threadIdx.x * 4;
  const int r = e / OUTN, oc = e % OUTN;
  int tm, tn;
  tile_of(p.tail_start + t, p.tiles_m, p.tiles_n, tm, tn);
  const int64_t row = static_cast<int64_t>(tm) * dl::BM + r;
  const int64_t col = static_cast<int64_t>(tn) * OUTN + oc;
  const float* W = p.part + static_cast<int64_t>(t) * p.splits * (dl::BM * BN) + r * BN;
  float v[4] = {0.f, 0.f, 0.f, 0.f}, u[4] = {0.f, 0.f, 0.f, 0.f};
  const int cg = SWIGLU ? 64 * (oc / 32) + oc % 32 : oc;
  for (int sp = 0; sp < p.splits; ++sp) {
    const float* Ws = W + static_cast<int64_t>(sp) * (dl::BM * BN);
    const f32x4 a = *reinterpret_cast<const f32x4*>(Ws + cg);
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] += a[i];
    if constexpr (SWIGLU) {
      const f32x4 b = *reinterpret_cast<const f32x4*>(Ws + cg + 32);
#pragma unroll
      for (int i = 0; i < 4; ++i) u[i] += b[i];
    }
  }
  T* D = static_cast<T*>(p.d);
  float out[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float x;
    if constexpr (SWIGLU) {
      x = silu(v[i]) * u[i];
    } else {
      x = p.alpha * v[i];
      if (p.c != nullptr && p.beta != 0.f)
        x += p.beta * Num<T>::to_f(static_cast<const T*>(p.c)[row * p.ldc_row + (col + i) * p.ldc_col]);
      if (p.epilogue == SPH_EPI_RELU) x = fmaxf(x, 0.f);
      else if (p.epilogue == SPH_EPI_GELU) x = gelu_erf(x);
      else if (p.epilogue == SPH_EPI_SILU) x = silu(x);
    }
    out[i] = x;
  }
  u32x2 w;
  w[0] = static_cast<uint32_t>(__builtin_bit_cast(uint16_t, Num<T>::from_f(out[0]))) |
         (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, Num<T>::from_f(out[1]))) << 16);
  w[1] = static_cast<uint32_t>(__builtin_bit_cast(uint16_t, Num<T>::from_f(out[2]))) |
         (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, Num<T>::from_f(out[3]))) << 16);
  *reinterpret_cast<u32x2*>(D + row * p.ldd + col) = w;
}

// ---------------------------------------------------------------------------
// Short-K products (K = 64 or 128; e.g. attention scores Q K^T with head
// dim 128): at 2 M N K FLOP against 2 M N bytes of output they are bound by
// memory.  Design:
//   * 128x128 tiles on 4 waves (64x64 each); the whole K range is one LDS
//     stage (64 KB at K = 128), so two workgroups share a CU and one's
//     operand loads overlap the other's MFMAs and stores.  (A persistent
//     one-workgroup-per-CU variant with a two-stage operand ring, with and
//     without producer/consumer wave roles, measured slower: its DMA keeps
//     at most one tile in flight per CU, and under the output stream the
//     load latency, not bandwidth, then sets the pace.  A variant with A's
//     MFMA fragments loaded straight from memory into registers and only B
//     in LDS (32 KB: three workgroups per CU) measured 86 us against 77.5
//     on the c2 bmm shape.)
//   * Operands arrive by direct global->LDS DMA as in the whole-tile kernel
//     (one 64-deep K block after another, same layouts; row-major B rows
//     are 256 bytes here and use chunk slot c ^ 4 (k & 3)).
//   * The MFMAs take B as the first operand, so each lane's accumulators
//     hold 4 consecutive output columns of one row: converted to T they are
//     8-byte LDS writes into a per-wave 64 x 64 slab (16-byte chunk c of row
//     m at slot c ^ ((m >> 1) & 7)), read back as whole 128-byte rows and
//     stored with 16-byte stores.
//   * Plain products only (alpha = 1, no C, no activation): D rounds each
//     fp32 sum once.
// ---------------------------------------------------------------------------
namespace sk {
constexpr int BM = 128, BN = 128, WM = 2, WN = 2, NW = WM * WN, NT = NW * 64;
constexpr int WTM = BM / WM, WTN = BN / WN, TM = WTM / 32, TN = WTN / 32;
constexpr int KB = 64;                           // K block (one A and one B block per 64 K)
constexpr int A_BLK = BM * KB * 2, B_BLK = BN * KB * 2;  // 16 KB each
constexpr int LPW = A_BLK / 1024 / NW;           // DMA lines per wave per block
constexpr int SLAB = WTM * WTN * 2;              // per-wave output slab (bytes)
static_assert(LPW * NW * 1024 == A_BLK, "DMA lines");
__device__ inline int aslot(int r, int c) { return r * 8 + (c ^ ((r >> 1) & 7)); }
}  // namespace sk

template <typename T, bool B_KCONT, int KT>
__global__ void __launch_bounds__(sk::NT) gemm_shortk_kernel(const GemmArgs p) {
  using namespace sk;
  constexpr int OPS = KT * (A_BLK + B_BLK);
  static_assert(NW * SLAB <= OPS, "slab fits in the operand space");
  __shared__ __attribute__((aligned(1024))) char lds[OPS];
  int tm, tn;
  tile_of(blockIdx.x, p.tiles_m, p.tiles_n, tm, tn);
  const int64_t batch = blockIdx.y;
  const int64_t m0 = static_cast<int64_t>(tm) * BM, n0 = static_cast<int64_t>(tn) * BN;
  const uint16_t* A = static_cast<const uint16_t*>(p.a) + batch * p.stride_a;
  const uint16_t* B = static_cast<const uint16_t*>(p.b) + batch * p.stride_b;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int lda = static_cast<int>(p.lda), ldb = static_cast<int>(p.ldb);

  const i32x4 ra = buffer_rsrc(A + m0 * lda, static_cast<uint32_t>(((BM - 1) * static_cast<int64_t>(lda) + p.k) * 2));
  const i32x4 rb = B_KCONT
      ? buffer_rsrc(B + n0 * ldb, static_cast<uint32_t>(((BN - 1) * static_cast<int64_t>(ldb) + p.k) * 2))
      : buffer_rsrc(B + n0, static_cast<uint32_t>(((p.k - 1) * ldb + BN) * 2));
  const uint32_t lds_base = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((SPH_LDS char*)(lds)));
#pragma unroll
  for (int kb = 0; kb < KT; ++kb) {
#pragma unroll
    for (int i = 0; i < LPW; ++i) {
      const int line = wave * LPW + i;
      const int s = line * 64 + lane;
      const int r = s >> 3, c = (s & 7) ^ ((r >> 1) & 7);
      dma16(ra, __builtin_amdgcn_readfirstlane(lds_base + kb * A_BLK + line * 1024),
            static_cast<uint32_t>(r * lda * 2 + c * 16), __builtin_amdgcn_readfirstlane(kb * KB * 2));
      uint32_t vb;
      if constexpr (B_KCONT) {
        vb = static_cast<uint32_t>(r * ldb * 2 + c * 16);
      } else {
        const int k = s >> 4, cb = (s & 15) ^ (4 * (k & 3));
        vb = static_cast<uint32_t>(k * ldb * 2 + cb * 16);
      }
      dma16(rb, __builtin_amdgcn_readfirstlane(lds_base + KT * A_BLK + kb * B_BLK + line * 1024), vb,
            __builtin_amdgcn_readfirstlane(B_KCONT ? kb * KB * 2 : kb * KB * ldb * 2));
    }
  }
  wait_vmcnt<0>();
  __syncthreads();

  const int row_in = lane & 31, khalf = lane >> 5;
  const int g = lane >> 4, jj = lane & 15, e = jj >> 2, q = jj & 3;
  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
#pragma unroll
  for (int kb = 0; kb < KT; ++kb) {
    const char* sa = lds + kb * A_BLK;
    const char* sb = lds + KT * A_BLK + kb * B_BLK;
#pragma unroll
    for (int kk = 0; kk < KB / 16; ++kk) {
      u32x4 af[TM], bf[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i)
        af[i] = *reinterpret_cast<const u32x4*>(sa + aslot(wm * WTM + i * 32 + row_in, kk * 2 + khalf) * 16);
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        if constexpr (B_KCONT) {
          bf[j] = *reinterpret_cast<const u32x4*>(sb + aslot(wn * WTN + j * 32 + row_in, kk * 2 + khalf) * 16);
        } else {
          const int n = wn * WTN + j * 32 + 16 * (g & 1) + 4 * q;
          const int k = kk * 16 + 8 * (g >> 1) + e;
          const SPH_LDS char* p0 =
              (const SPH_LDS char*)(sb) + k * (BN * 2) + (((n >> 3) ^ (4 * e)) << 4) + 8 * (q & 1);
          const u32x2 lo = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((SPH_LDS s16x4*)(p0)));
          const u32x2 hi = __builtin_bit_cast(
              u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((SPH_LDS s16x4*)(p0 + 4 * BN * 2)));
          bf[j] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3);
        }
      }
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = mfma32<T>(bf[j], af[i], acc[i][j]);
    }
  }
  // acc[i][j][r]: row m = i*32 + lane%32, columns n = j*32 + 8*(r/4) + 4*(lane/32) + r%4
  __syncthreads();
  char* slab = lds + wave * SLAB;
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int m = i * 32 + row_in;
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int rg = 0; rg < 4; ++rg) {
        const int n = j * 32 + 8 * rg + 4 * khalf;
        uint32_t w[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const uint16_t lo = __builtin_bit_cast(uint16_t, Num<T>::from_f(acc[i][j][4 * rg + 2 * h]));
          const uint16_t hi = __builtin_bit_cast(uint16_t, Num<T>::from_f(acc[i][j][4 * rg + 2 * h + 1]));
          w[h] = static_cast<uint32_t>(lo) | (static_cast<uint32_t>(hi) << 16);
        }
        const int c = n >> 3;
        *reinterpret_cast<u32x2*>(slab + (m * 8 + (c ^ ((m >> 1) & 7))) * 16 + (n & 7) * 2) =
            u32x2{w[0], w[1]};
      }
  }
  // The slab belongs to this wave alone; a wave's LDS accesses run in order.
  // The output is written once and not read back by this kernel: streaming
  // (non-temporal) stores, 14 % faster than plain ones on the attention-
  // score shape (32 x 2048 x 2048 from K = 128).
  T* D = static_cast<T*>(p.d) + batch * p.stride_d;
#pragma unroll
  for (int it = 0; it < WTM / 8; ++it) {
    const int m = it * 8 + (lane >> 3), c = lane & 7;
    const u32x4 v = *reinterpret_cast<const u32x4*>(slab + (m * 8 + (c ^ ((m >> 1) & 7))) * 16);
    __builtin_nontemporal_store(
        v, reinterpret_cast<u32x4*>(D + (m0 + wm * WTM + m) * p.ldd + n0 + wn * WTN + c * 8));
  }
}

// ---------------------------------------------------------------------------
// Short-K products over many tiles (the attention scores of a whole batch):
// a persistent form of the kernel above, one workgroup of 4 waves (64x64
// each) per CU, walking a contiguous run of the (batch entry, tile row,
// tile column) sequence of 128x128 tiles.
//   * The A row panel of the current (batch entry, tile row) stays in LDS
//     while the workgroup walks that row's tile columns, so a tile streams
//     only its B block: half the operand bytes of the one-shot kernel.
//   * B blocks go through a three-stage LDS ring: while tile i computes,
//     tiles i+1 and i+2 are in flight (issued one and two tiles earlier).
//   * Results leave through a per-wave 32 x 64 slab (two halves per tile)
//     as streaming 16-byte stores of whole 128-byte rows that the loop never
//     waits for: vector memory counts return in issue order, so waiting for
//     an older block's DMA leaves the stores issued after it in flight.
//   * Consecutive workgroups of one XCD (dispatch is round-robin over the 8
//     XCDs) take consecutive runs, so one batch entry's B panel is fetched
//     into one XCD's L2 and re-read from there by its tile rows.
//   * The tile position advances by a cursor (no 64-bit divisions in the
//     loop) and each tile's first MFMAs take a zero accumulator operand.
// A new A panel (a run crossing into the next tile row) is loaded after
// every wave has finished the previous tile: one exposed load per switch,
// at most a few per workgroup.
// Measured on MI355X (attention-score shape 32 x 2048 x 2048 from K = 128,
// alternating on one box): 67.5-70 us against 79-81 for the one-shot
// kernel.  Not kept: 8 waves of 64x32 (64-byte row stores) 93-95 us; 8
// waves of 32x64, 69.6; 256-row tiles on 8 waves with a two-stage ring,
// 76.5 against 74.3 on a slower box; the same kernel with 64-bit tile
// divisions and zeroed accumulators, 75; tile i-1's slab epilogue and
// stores spread between tile i's MFMA sub-steps, 73-74 against 69-71.
// ---------------------------------------------------------------------------
namespace skr {
constexpr int NSTG = 3;                               // B stages
// Wave layout WM x WN over the 128x128 tile.
template <int WM_, int WN_>
struct L {
  static constexpr int WM = WM_, WN = WN_, NW = WM * WN, NT = NW * 64;
  static constexpr int WTM = sk::BM / WM, WTN = sk::BN / WN, TM = WTM / 32, TN = WTN / 32;
  static constexpr int CPR = WTN * 2 / 16;            // 16-byte chunks per slab row
  static constexpr int RPS = 1024 / (WTN * 2);        // slab rows per 16-byte store instruction
  static constexpr int SLAB = 32 * WTN * 2;           // per-wave slab: 32 rows of the wave tile
  static constexpr int STORES = TM * 32 / RPS;        // stores per wave per tile
  static constexpr int LPW = sk::A_BLK / 1024 / NW;   // DMA lines per wave per 64-deep block
  static_assert(LPW * NW * 1024 == sk::A_BLK && (CPR & (CPR - 1)) == 0, "wave layout");
  // slab row m, chunk c -> 16-byte slot
  __device__ static int sslot(int m, int c) { return m * CPR + (c ^ ((m >> 1) & (CPR - 1))); }
};
// Position (batch entry, tile row, tile column) in the tile sequence.
struct Cursor {
  int b, tm, tn;
  __device__ void next(int tiles_m, int tiles_n) {
    if (++tn == tiles_n) {
      tn = 0;
      if (++tm == tiles_m) tm = 0, ++b;
    }
  }
};
}  // namespace skr

template <typename T, bool B_KCONT, int KT, int WM_, int WN_>
__global__ void __launch_bounds__((skr::L<WM_, WN_>::NT)) gemm_shortk_ring_kernel(const GemmArgs p) {
  using sk::A_BLK;
  using sk::B_BLK;
  using sk::BM;
  using sk::BN;
  using sk::KB;
  using sk::aslot;
  using skr::Cursor;
  using skr::NSTG;
  using W = skr::L<WM_, WN_>;
  constexpr int WN = W::WN, WTM = W::WTM, WTN = W::WTN, TM = W::TM, TN = W::TN;
  constexpr int NW = W::NW, LPW = W::LPW, STORES = W::STORES, CPR = W::CPR, RPS = W::RPS;
  constexpr int A_PANEL = KT * A_BLK, B_TILE = KT * B_BLK;
  constexpr int LB = KT * LPW;                     // DMA lines per wave per B block (= per A panel)
  constexpr int SLAB_OFF = A_PANEL + NSTG * B_TILE;
  __shared__ __attribute__((aligned(1024))) char lds[SLAB_OFF + NW * W::SLAB];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int lda = static_cast<int>(p.lda), ldb = static_cast<int>(p.ldb);
  const int tiles_m = p.tiles_m, tiles_n = p.tiles_n;
  const uint32_t lds_base = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((SPH_LDS char*)(lds)));

  // This workgroup's run [t0, t0 + n) of the tile sequence.
  const int64_t total = p.batches * tiles_m * tiles_n;
  const int G = static_cast<int>(gridDim.x);
  int slot = static_cast<int>(blockIdx.x);
  if ((G & 7) == 0) slot = (slot & 7) * (G >> 3) + (slot >> 3);
  const int64_t t0 = total * slot / G;
  const int n = static_cast<int>(total * (slot + 1) / G - t0);
  if (n <= 0) return;
  Cursor cur;  // tile i
  {
    const int64_t u = t0 / tiles_n;
    cur.tn = static_cast<int>(t0 - u * tiles_n);
    cur.b = static_cast<int>(u / tiles_m);
    cur.tm = static_cast<int>(u - static_cast<int64_t>(cur.b) * tiles_m);
  }

  // Per-lane byte offsets of this wave's DMA lines within a 64-deep K block.
  uint32_t va[LPW], vb[LPW];
#pragma unroll
  for (int i = 0; i < LPW; ++i) {
    const int s = (wave * LPW + i) * 64 + lane;
    const int r = s >> 3, c = (s & 7) ^ ((r >> 1) & 7);
    va[i] = static_cast<uint32_t>(r * lda * 2 + c * 16);
    if constexpr (B_KCONT) {
      vb[i] = static_cast<uint32_t>(r * ldb * 2 + c * 16);
    } else {
      const int k = s >> 4, cb = (s & 15) ^ (4 * (k & 3));
      vb[i] = static_cast<uint32_t>(k * ldb * 2 + cb * 16);
    }
  }
  const uint16_t* const A0 = static_cast<const uint16_t*>(p.a);
  const uint16_t* const B0 = static_cast<const uint16_t*>(p.b);
  // A row panel of the cursor's (batch entry, tile row) into the panel slot.
  auto dma_a = [&](const Cursor& c) {
    const i32x4 ra = buffer_rsrc(A0 + c.b * p.stride_a + static_cast<int64_t>(c.tm) * BM * p.lda,
                                 static_cast<uint32_t>(((BM - 1) * static_cast<int64_t>(lda) + p.k) * 2));
#pragma unroll
    for (int kb = 0; kb < KT; ++kb)
#pragma unroll
      for (int i = 0; i < LPW; ++i)
        dma16(ra, __builtin_amdgcn_readfirstlane(lds_base + kb * A_BLK + (wave * LPW + i) * 1024), va[i],
              __builtin_amdgcn_readfirstlane(kb * KB * 2));
  };
  // B block of the cursor's tile into ring stage st.
  auto dma_b = [&](const Cursor& c, int st) {
    const uint16_t* B = B0 + c.b * p.stride_b;
    const i32x4 rb = B_KCONT
        ? buffer_rsrc(B + static_cast<int64_t>(c.tn) * BN * p.ldb,
                      static_cast<uint32_t>(((BN - 1) * static_cast<int64_t>(ldb) + p.k) * 2))
        : buffer_rsrc(B + static_cast<int64_t>(c.tn) * BN, static_cast<uint32_t>(((p.k - 1) * ldb + BN) * 2));
#pragma unroll
    for (int kb = 0; kb < KT; ++kb)
#pragma unroll
      for (int i = 0; i < LPW; ++i)
        dma16(rb,
              __builtin_amdgcn_readfirstlane(lds_base + A_PANEL + st * B_TILE + kb * B_BLK +
                                             (wave * LPW + i) * 1024),
              vb[i], __builtin_amdgcn_readfirstlane(B_KCONT ? kb * KB * 2 : kb * KB * ldb * 2));
  };

  Cursor ahead = cur;  // tile i + 2 once the loop runs
  dma_a(cur);
  dma_b(ahead, 0);
  ahead.next(tiles_m, tiles_n);
  if (n > 1) dma_b(ahead, 1);
  ahead.next(tiles_m, tiles_n);

  const int row_in = lane & 31, khalf = lane >> 5;
  const int g = lane >> 4, jj = lane & 15, e = jj >> 2, q = jj & 3;
  char* const slab = lds + SLAB_OFF + wave * W::SLAB;
  T* const D0 = static_cast<T*>(p.d);
  bool reloaded = false;  // the previous tile loaded a new A panel
  for (int i = 0; i < n; ++i) {
    const bool sw = i > 0 && cur.tn == 0;  // tile i starts a new tile row
    // B block i (and everything issued before it) has landed.  Issued
    // after it: the stores of tiles i-2 and i-1, B block i+1 unless i is
    // the last tile, and an A panel if tile i-1 switched rows; waiting for
    // fewer than that many waits longer, never shorter.
    if (i == 0) {
      wait_vmcnt<0>();
    } else if (i == 1) {
      wait_vmcnt<STORES>();
    } else if (!reloaded && i + 1 < n) {
      wait_vmcnt<2 * STORES + LB>();
    } else {
      wait_vmcnt<2 * STORES>();
    }
    // Past this barrier every wave is done with tile i-1: its ring stage
    // and, on a row switch, the A panel may be refilled.
    __syncthreads();
    if (sw) dma_a(cur);
    if (i + 2 < n) {
      dma_b(ahead, (i + 2) % NSTG);
      ahead.next(tiles_m, tiles_n);
    }
    if (sw) {
      if (i + 2 < n) wait_vmcnt<LB>();
      else wait_vmcnt<0>();
      __syncthreads();
    }
    reloaded = sw;

    const char* sb = lds + A_PANEL + (i % NSTG) * B_TILE;
    f32x16 acc[TM][TN];
#pragma unroll
    for (int kb = 0; kb < KT; ++kb) {
      const char* sa = lds + kb * A_BLK;
      const char* sbk = sb + kb * B_BLK;
#pragma unroll
      for (int kk = 0; kk < KB / 16; ++kk) {
        u32x4 af[TM], bf[TN];
#pragma unroll
        for (int a = 0; a < TM; ++a)
          af[a] = *reinterpret_cast<const u32x4*>(sa + aslot(wm * WTM + a * 32 + row_in, kk * 2 + khalf) * 16);
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          if constexpr (B_KCONT) {
            bf[j] = *reinterpret_cast<const u32x4*>(sbk + aslot(wn * WTN + j * 32 + row_in, kk * 2 + khalf) * 16);
          } else {
            const int nn = wn * WTN + j * 32 + 16 * (g & 1) + 4 * q;
            const int k = kk * 16 + 8 * (g >> 1) + e;
            const SPH_LDS char* p0 =
                (const SPH_LDS char*)(sbk) + k * (BN * 2) + (((nn >> 3) ^ (4 * e)) << 4) + 8 * (q & 1);
            const u32x2 lo = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((SPH_LDS s16x4*)(p0)));
            const u32x2 hi = __builtin_bit_cast(
                u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((SPH_LDS s16x4*)(p0 + 4 * BN * 2)));
            bf[j] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3);
          }
        }
        // (the first sub-step starts from a zero accumulator operand)
#pragma unroll
        for (int a = 0; a < TM; ++a)
#pragma unroll
          for (int j = 0; j < TN; ++j)
            acc[a][j] = mfma32<T>(bf[j], af[a], kb == 0 && kk == 0 ? f32x16{} : acc[a][j]);
      }
    }
    // acc[a][j][r]: row a*32 + lane%32, column j*32 + 8*(r/4) + 4*(lane/32) + r%4.
    // Each 32-row block goes through the wave's own slab: 8-byte writes,
    // 16-byte reads of whole slab rows, streaming stores.
    T* D = D0 + cur.b * p.stride_d + (static_cast<int64_t>(cur.tm) * BM + wm * WTM) * p.ldd +
           static_cast<int64_t>(cur.tn) * BN + wn * WTN;
#pragma unroll
    for (int a = 0; a < TM; ++a) {
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int rg = 0; rg < 4; ++rg) {
          uint32_t w[2];
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const uint16_t lo = __builtin_bit_cast(uint16_t, Num<T>::from_f(acc[a][j][4 * rg + 2 * h]));
            const uint16_t hi = __builtin_bit_cast(uint16_t, Num<T>::from_f(acc[a][j][4 * rg + 2 * h + 1]));
            w[h] = static_cast<uint32_t>(lo) | (static_cast<uint32_t>(hi) << 16);
          }
          *reinterpret_cast<u32x2*>(slab + W::sslot(row_in, j * 4 + rg) * 16 + khalf * 8) = u32x2{w[0], w[1]};
        }
#pragma unroll
      for (int it = 0; it < 32 / RPS; ++it) {
        const int m = it * RPS + lane / CPR, c = lane % CPR;
        const u32x4 v = *reinterpret_cast<const u32x4*>(slab + W::sslot(m, c) * 16);
        __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(D + (a * 32 + m) * p.ldd + c * 8));
      }
    }
    cur.next(tiles_m, tiles_n);
  }
}

// ---------------------------------------------------------------------------
// Small-M products: D[m, n] = epi(alpha * sum_k A[m, k] * B[n, k] + beta*C)
// for M <= MT rows, A and B K-contiguous and 16-byte aligned, K % 8 == 0.
// A group of TPR threads computes R output columns n for all M rows: thread t
// reads 16 bytes of each of the R weight rows at k = 8t + 8*TPR*j (whole row
// segments per group, coalesced) and keeps the R loads of two K steps in
// flight.  TPR follows K (256 threads for K >= 2048 down to 16 for K = 128,
// so short rows such as attention keys do not idle most of the workgroup)
// and a workgroup holds 256/TPR groups.  Workgroups loop over row blocks
// (grid capped near the number of resident workgroups), so long matrices do
// not end in a partial wave of workgroups.  A (at most 16 x K, read by every
// workgroup) comes through the caches.  fp16 uses v_dot2_f32_f16 (two
// products summed into an fp32 accumulator), bf16 widens with shifts and
// uses fp32 FMAs.  Partial sums are reduced within the group by butterflies
// and, for groups wider than a wave, through LDS.
// ---------------------------------------------------------------------------
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

template <typename T>
__device__ inline float dot8_acc(u32x4 a, u32x4 b, float acc) {
  if constexpr (__is_same(T, half_t)) {
    // (vector elements are copied to scalars first: this compiler lowers
    // __builtin_bit_cast of an indexed vector element to element 0)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t ai = a[i], bi = b[i];
      acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, ai), __builtin_bit_cast(f16x2, bi),
                                   acc, false);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      acc = fmaf(__uint_as_float(a[i] << 16), __uint_as_float(b[i] << 16), acc);
      acc = fmaf(__uint_as_float(a[i] & 0xffff0000u), __uint_as_float(b[i] & 0xffff0000u), acc);
    }
  }
  return acc;
}

constexpr int kSkinnyThreads = 256;

template <typename T>
__device__ inline float skinny_epilogue(const GemmArgs& p, float v, int64_t bz, int m, int64_t n) {
  v *= p.alpha;
  if (p.c != nullptr && p.beta != 0.f) {
    const T* C = static_cast<const T*>(p.c) + bz * p.stride_c;
    v += p.beta * Num<T>::to_f(C[m * p.ldc_row + n * p.ldc_col]);
  }
  if (p.epilogue == SPH_EPI_RELU) v = fmaxf(v, 0.f);
  else if (p.epilogue == SPH_EPI_GELU) v = gelu_erf(v);
  else if (p.epilogue == SPH_EPI_SILU) v = silu(v);
  return v;
}

// NORM: the RMSNorm prologue of GemmArgs (norm_w, norm_eps) on A's rows.
template <typename T, int MT, int R, int TPR, bool NORM = false>
__global__ void __launch_bounds__(kSkinnyThreads) gemm_skinny_kernel(const GemmArgs p,
                                                                     int64_t nblocks) {
  constexpr int G = kSkinnyThreads / TPR;   // row groups per workgroup
  constexpr int WPG = TPR > 64 ? TPR / 64 : 1;  // waves per group
  __shared__ float red[TPR > 64 ? G * WPG * MT * R : 1];
  __shared__ float red_ss[NORM && TPR > 64 ? G * WPG * MT : 1];
  const int g = threadIdx.x / TPR, t = threadIdx.x % TPR;
  const int64_t bz = blockIdx.y;
  const uint16_t* A = static_cast<const uint16_t*>(p.a) + bz * p.stride_a;
  const uint16_t* B = static_cast<const uint16_t*>(p.b) + bz * p.stride_b;
  const uint16_t* NW = static_cast<const uint16_t*>(p.norm_w);
  T* D = static_cast<T*>(p.d) + bz * p.stride_d;
  const int mrows = static_cast<int>(p.m);
  const float inv_k = 1.0f / static_cast<float>(p.k);
  // Every thread runs the same number of outer iterations (the bound does
  // not depend on the group), so the barriers below are uniform.
  for (int64_t base = static_cast<int64_t>(blockIdx.x) * G; base < nblocks;
       base += static_cast<int64_t>(gridDim.x) * G) {
    const int64_t blk = base + g;
    const int64_t n0 = blk * R;
    float acc[MT][R];
    float ss[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      ss[m] = 0.f;
#pragma unroll
      for (int r = 0; r < R; ++r) acc[m][r] = 0.f;
    }
    if (blk < nblocks) {
      // Loads are unconditional (rows past N and M read a valid row, whose
      // results are never stored) so no branch separates them: the R + MT
      // loads of the next K step are issued before the current step's dot
      // products and one wait covers them.
      const uint16_t* bp[R];
#pragma unroll
      for (int r = 0; r < R; ++r) bp[r] = B + (n0 + r < p.n ? n0 + r : p.n - 1) * p.ldb;
      const uint16_t* ap[MT];
#pragma unroll
      for (int m = 0; m < MT; ++m) ap[m] = A + (m < mrows ? m : mrows - 1) * p.lda;
      constexpr int64_t STEP = TPR * 8;
      int64_t k = static_cast<int64_t>(t) * 8;
      if (k < p.k) {
        u32x4 w[R], x[MT], nw = zero4();
#pragma unroll
        for (int r = 0; r < R; ++r)
          w[r] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(bp[r] + k));
#pragma unroll
        for (int m = 0; m < MT; ++m) x[m] = *reinterpret_cast<const u32x4*>(ap[m] + k);
        if constexpr (NORM) nw = *reinterpret_cast<const u32x4*>(NW + k);
        while (true) {
          const int64_t kn = k + STEP;
          const bool more = kn < p.k;
          const int64_t kl = more ? kn : k;  // reload the current step when done
          u32x4 w2[R], x2[MT], nw2 = zero4();
#pragma unroll
          for (int r = 0; r < R; ++r)
            w2[r] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(bp[r] + kl));
#pragma unroll
          for (int m = 0; m < MT; ++m) x2[m] = *reinterpret_cast<const u32x4*>(ap[m] + kl);
          if constexpr (NORM) nw2 = *reinterpret_cast<const u32x4*>(NW + kl);
#pragma unroll
          for (int m = 0; m < MT; ++m) {
            const u32x4 xm = NORM ? norm_chunk<T>(x[m], nw, ss[m]) : x[m];
#pragma unroll
            for (int r = 0; r < R; ++r) acc[m][r] = dot8_acc<T>(xm, w[r], acc[m][r]);
          }
          if (!more) break;
#pragma unroll
          for (int r = 0; r < R; ++r) w[r] = w2[r];
#pragma unroll
          for (int m = 0; m < MT; ++m) x[m] = x2[m];
          nw = nw2;
          k = kn;
        }
      }
    }
    // Butterflies within the group's wave segment (all lanes take part).
    constexpr int LANES = TPR > 64 ? 64 : TPR;
#pragma unroll
    for (int m = 0; m < MT; ++m) {
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int off = LANES / 2; off > 0; off >>= 1)
          acc[m][r] += __shfl_xor(acc[m][r], off, 64);
      if constexpr (NORM) {
#pragma unroll
        for (int off = LANES / 2; off > 0; off >>= 1) ss[m] += __shfl_xor(ss[m], off, 64);
      }
    }
    if constexpr (TPR > 64) {
      const int wig = t / 64;  // wave within the group
      if ((t & 63) == 0) {
#pragma unroll
        for (int m = 0; m < MT; ++m) {
#pragma unroll
          for (int r = 0; r < R; ++r) red[((g * WPG) + wig) * MT * R + m * R + r] = acc[m][r];
          if constexpr (NORM) red_ss[((g * WPG) + wig) * MT + m] = ss[m];
        }
      }
      __syncthreads();
      for (int q = t; q < MT * R; q += TPR) {
        const int m = q / R, r = q % R;
        const int64_t n = n0 + r;
        if (blk < nblocks && m < mrows && n < p.n) {
          float v = 0.f, sq = 0.f;
#pragma unroll
          for (int w = 0; w < WPG; ++w) {
            v += red[(g * WPG + w) * MT * R + q];
            if constexpr (NORM) sq += red_ss[(g * WPG + w) * MT + m];
          }
          if constexpr (NORM) v *= rsqrtf(sq * inv_k + p.norm_eps);
          D[m * p.ldd + n] = Num<T>::from_f(skinny_epilogue<T>(p, v, bz, m, n));
        }
      }
      __syncthreads();
    } else {
      if (blk < nblocks) {
#pragma unroll
        for (int m = 0; m < MT; ++m)
#pragma unroll
          for (int r = 0; r < R; ++r) {
            const int64_t n = n0 + r;
            if (t == (m * R + r) % TPR && m < mrows && n < p.n) {
              float v = acc[m][r];
              if constexpr (NORM) v *= rsqrtf(ss[m] * inv_k + p.norm_eps);
              D[m * p.ldd + n] = Num<T>::from_f(skinny_epilogue<T>(p, v, bz, m, n));
            }
          }
      }
    }
  }
}

template <typename T, int MT, int R, int TPR, bool NORM = false>
void launch_skinny_cfg(const GemmArgs& p, int64_t batch, hipStream_t st) {
  const int64_t nblocks = ceil_div(p.n, R);
  constexpr int G = kSkinnyThreads / TPR;
  int64_t gx = ceil_div(nblocks, G);
  const int64_t cap = batch >= 4096 ? 1 : 4096 / batch;
  if (gx > cap) gx = cap;
  dim3 grid(static_cast<unsigned>(gx), static_cast<unsigned>(batch));
  gemm_skinny_kernel<T, MT, R, TPR, NORM><<<grid, dim3(kSkinnyThreads), 0, st>>>(p, nblocks);
}

// Launch shape from a sweep on MI355X over the decode shapes (x[4, K] times
// W[N, K], 32 MB .. 400 MB of weights): two-wave groups (TPR 128) with two
// columns each for K ~ 4096, four columns for long rows, one-wave groups of
// four columns for very wide W (LM heads), whole-workgroup groups for narrow
// W; TPR never exceeds K / 8 (every thread owns at least one K chunk).
template <typename T, int MT, bool NORM = false>
void launch_skinny_m(const GemmArgs& p, int64_t batch, hipStream_t st) {
  int tmax = 256;
  while (tmax > 16 && static_cast<int64_t>(tmax) * 8 > p.k) tmax >>= 1;
  const int64_t cols = p.n * batch;
  int tpr = 128, r = p.k >= 8192 ? 4 : 2;
  if (cols >= 32768) tpr = 64, r = 4;
  else if (cols <= 2048) tpr = 256, r = 2;
  if (tpr > tmax) tpr = tmax, r = 2;
  if (r == 4 && tpr == 64) return launch_skinny_cfg<T, MT, 4, 64, NORM>(p, batch, st);
  if (r == 4) return launch_skinny_cfg<T, MT, 4, 128, NORM>(p, batch, st);
  switch (tpr) {
    case 256: return launch_skinny_cfg<T, MT, 2, 256, NORM>(p, batch, st);
    case 128: return launch_skinny_cfg<T, MT, 2, 128, NORM>(p, batch, st);
    case 64: return launch_skinny_cfg<T, MT, 2, 64, NORM>(p, batch, st);
    case 32: return launch_skinny_cfg<T, MT, 2, 32, NORM>(p, batch, st);
    default: return launch_skinny_cfg<T, MT, 2, 16, NORM>(p, batch, st);
  }
}

template <typename T, bool NORM = false>
int launch_skinny(const GemmArgs& p, int64_t batch, hipStream_t st) {
  if (p.m <= 1)
    launch_skinny_m<T, 1, NORM>(p, batch, st);
  else if (p.m <= 4)
    launch_skinny_m<T, 4, NORM>(p, batch, st);
  else if (p.m <= 8)
    launch_skinny_m<T, 8, NORM>(p, batch, st);
  else
    launch_skinny_m<T, 16, NORM>(p, batch, st);
  return check_launch("sph_gemm (small M)");
}

// ---------------------------------------------------------------------------
// Decode-shaped products (M <= 8 activation rows against a weight matrix
// W[N, K] read once; batch 1, K from 1024 to 16384): the weight stream is
// the whole cost, so the kernel is built to keep as many weight bytes in
// flight as the CU allows and to give every wave the same share of them.
//   * One workgroup of WV waves per CU (persistent over the rows; 16 waves,
//     or 12 / 10 where that makes the rows whole rounds of the grid): the
//     M x K activations are staged into LDS once and read from there
//     (16-byte chunks, a wave's 64 lanes on 1 KB of consecutive bytes).
//   * Each wave streams whole weight rows: lane l owns the 16-byte chunks
//     l, l + 64, ... of the row, in segments of SEG chunks.  The wave walks
//     a flat sequence of (row, segment) items and loads item i+1 into one
//     register buffer while it computes item i from the other, so loads of
//     the next row are in flight while a row's sums are reduced and stored.
//   * Rows go round-robin over all W waves of the grid for the N / W whole
//     rounds.  The N % W rows left over would leave most waves idle for a
//     whole row time (gate/up of a 4096-wide model: 12800 rows = 3.125
//     rounds of 4096), so each of them is split along K between Q waves of
//     one workgroup (Q = 16 / the workgroup's leftover rows, rounded to a
//     power of two): the slice is the last item of each of those waves, and
//     after one workgroup barrier the first wave of each group adds the Q
//     partial sums from LDS and writes the outputs.
//   * At the end of a row the 64 lane sums per activation row are reduced by
//     butterflies and one lane writes the M outputs (with the epilogue:
//     alpha, beta*C, activation).
// ---------------------------------------------------------------------------
namespace gv {
constexpr int WAVES = 16, SEG = 8;
}

// SWIGLU: W holds the gate rows [0, n) and the up rows [n, 2n); output j
// is silu(x W[j]) * (x W[n + j]).  A wave's item then loads SEG / 2 chunks
// of both rows (the same register footprint) and the end of the row
// combines the two sums.
// NORM: the RMSNorm prologue of GemmArgs (norm_w, norm_eps), applied while
// the activations are staged (sums of squares reduced through LDS at the
// staging barrier) and to the finished sums of each row.
template <typename T, int MT, int KMAX, bool SWIGLU = false, bool NORM = false,
          int WV = gv::WAVES>
__global__ void __launch_bounds__(WV * 64) gemm_stream_kernel(const GemmArgs p) {
  using gv::SEG;
  constexpr int WAVES = WV, THREADS = WV * 64;
  constexpr int NR = SWIGLU ? 2 : 1, SEGK = SEG / NR;  // rows per item, chunks per row
  __shared__ __attribute__((aligned(16))) uint16_t As[MT * KMAX];
  __shared__ float lds_ss[NORM ? WAVES * MT : 1];
  __shared__ float lds_part[WAVES * NR * MT];  // partial sums of split rows
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nc = static_cast<int>(p.k / 8);           // 16-byte chunks per row
  const int mrows = static_cast<int>(p.m);
  const uint16_t* A = static_cast<const uint16_t*>(p.a);
  const uint16_t* B = static_cast<const uint16_t*>(p.b);
  T* D = static_cast<T*>(p.d);
  const int64_t stride = static_cast<int64_t>(gridDim.x) * WAVES;  // W
  const int64_t rounds = p.n / stride;                 // whole rounds
  const int64_t main_end = rounds * stride;            // rows [0, main_end) whole
  const int64_t left = p.n - main_end;                 // rows split along K
  // This wave's slice of a split row: group `slot` of `qn` waves shares
  // leftover row main_end + slot * gridDim.x + blockIdx.x; this wave holds
  // chunks [tcb, tcb + tcn) of it.
  int qn = 1, q = 0, slot = 0, tcb = 0, tcn = 0;
  int64_t trow = -1;
  if (left > 0) {
    const int64_t G = gridDim.x;
    const int rpw = static_cast<int>((left + G - 1) / G);  // <= WAVES
    int p2 = 1;
    while (p2 < rpw) p2 <<= 1;
    qn = WAVES / p2;
    while (qn > 1 && nc / qn < 64) qn >>= 1;  // at least one chunk per lane
    slot = wave / qn;
    q = wave % qn;
    const int64_t t = static_cast<int64_t>(slot) * G + blockIdx.x;
    if (slot < rpw && t < left) {
      trow = main_end + t;
      const int cs = (nc + qn - 1) / qn;
      tcb = q * cs;
      tcn = nc - tcb < cs ? nc - tcb : cs;
    }
  }
  const int nseg = ((nc + 63) / 64 + SEGK - 1) / SEGK;            // segments of a row
  const int tseg = ((tcn + 63) / 64 + SEGK - 1) / SEGK;           // of this wave's slice
  u32x4 wa[SEG], wb[SEG];
  float acc[NR][MT];
#pragma unroll
  for (int r = 0; r < NR; ++r)
#pragma unroll
    for (int m = 0; m < MT; ++m) acc[r][m] = 0.f;

// Weight chunks of item (ROW_, chunks from CB_, segment SEG_) into register
// buffer W_ (row r of the item in entries r * SEGK ..; chunks past the
// range read a valid chunk that is not summed).
#define SPH_GV_LOAD(W_, ROW_, CB_, SEG_)                                                    \
  do {                                                                                      \
    _Pragma("unroll") for (int r_ = 0; r_ < NR; ++r_) {                                     \
      const uint16_t* rp_ = B + ((ROW_) + r_ * p.n) * p.ldb;                                \
      _Pragma("unroll") for (int j_ = 0; j_ < SEGK; ++j_) {                                 \
        int c_ = (CB_) + ((SEG_) * SEGK + j_) * 64 + lane;                                  \
        c_ = c_ < nc ? c_ : nc - 1;                                                         \
        W_[r_ * SEGK + j_] =                                                                \
            __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(rp_ + c_ * 8));       \
      }                                                                                     \
    }                                                                                       \
  } while (0)
#define SPH_GV_COMPUTE(W_, CB_, CE_, SEG_)                                                  \
  do {                                                                                      \
    _Pragma("unroll") for (int j_ = 0; j_ < SEGK; ++j_) {                                   \
      const int c_ = (CB_) + ((SEG_) * SEGK + j_) * 64 + lane;                              \
      if (c_ < (CE_)) {                                                                     \
        _Pragma("unroll") for (int m_ = 0; m_ < MT; ++m_) {                                 \
          const u32x4 a_ = *reinterpret_cast<const u32x4*>(As + (m_ * nc + c_) * 8);        \
          _Pragma("unroll") for (int r_ = 0; r_ < NR; ++r_)                                 \
              acc[r_][m_] = dot8_acc<T>(a_, W_[r_ * SEGK + j_], acc[r_][m_]);               \
        }                                                                                   \
      }                                                                                     \
    }                                                                                       \
  } while (0)
#define SPH_GV_REDUCE()                                                                     \
  _Pragma("unroll") for (int r_ = 0; r_ < NR; ++r_)                                         \
    _Pragma("unroll") for (int m_ = 0; m_ < MT; ++m_)                                       \
      _Pragma("unroll") for (int o_ = 32; o_ > 0; o_ >>= 1)                                 \
          acc[r_][m_] += __shfl_xor(acc[r_][m_], o_, 64)
// Output of row ROW_ from its two (SWIGLU) or one sums S0_(m), S1_(m):
// lane m < M writes element (m, ROW_).
#define SPH_GV_STORE(ROW_, S0_, S1_)                                                        \
  do {                                                                                      \
    float v_ = 0.f;                                                                         \
    _Pragma("unroll") for (int m_ = 0; m_ < MT; ++m_) {                                     \
      const float g_ = (S0_) * rs[m_];                                                      \
      const float x_ = SWIGLU ? silu(g_) * ((S1_) * rs[m_]) : g_;                           \
      v_ = lane == m_ ? x_ : v_;                                                            \
    }                                                                                       \
    if (lane < MT && lane < mrows)                                                          \
      D[lane * p.ldd + (ROW_)] = Num<T>::from_f(                                            \
          SWIGLU ? v_ : skinny_epilogue<T>(p, v_, 0, lane, (ROW_)));                        \
  } while (0)
// End of item (ROW_, SEG_) when it completes a row or a slice.
#define SPH_GV_FINISH(ROW_, TAIL_)                                                          \
  do {                                                                                      \
    SPH_GV_REDUCE();                                                                        \
    if (TAIL_) {                                                                            \
      if (lane == 0) {                                                                      \
        _Pragma("unroll") for (int r_ = 0; r_ < NR; ++r_)                                   \
          _Pragma("unroll") for (int m_ = 0; m_ < MT; ++m_)                                 \
            lds_part[(wave * NR + r_) * MT + m_] = acc[r_][m_];                             \
      }                                                                                     \
    } else {                                                                                \
      SPH_GV_STORE(ROW_, acc[0][m_], acc[NR - 1][m_]);                                      \
    }                                                                                       \
    _Pragma("unroll") for (int r_ = 0; r_ < NR; ++r_)                                       \
      _Pragma("unroll") for (int m_ = 0; m_ < MT; ++m_) acc[r_][m_] = 0.f;                  \
  } while (0)

  // This wave's item sequence: segments 0..nseg-1 of rows n0, n0 + W, ...
  // below main_end, then segments 0..tseg-1 of its split-row slice.
  int64_t n = static_cast<int64_t>(blockIdx.x) * WAVES + wave;
  int cb = 0, ce = nc, ns = nseg, s = 0;
  bool tail = false, have = n < main_end;
  if (!have && trow >= 0) {
    n = trow, cb = tcb, ce = tcb + tcn, ns = tseg, tail = true, have = true;
  }
  // The first weight loads go out before the activations are staged, so
  // the two latencies overlap.
  if (have) SPH_GV_LOAD(wa, n, cb, 0);
  // Stage the activations ([m][chunk], rows past M as zeros).
  float rs[MT];  // row scales of the RMSNorm prologue (1 without it)
#pragma unroll
  for (int m = 0; m < MT; ++m) rs[m] = 0.f;
  for (int i = threadIdx.x; i < MT * nc; i += THREADS) {
    const int m = i / nc, c = i - m * nc;
    u32x4 v = {0u, 0u, 0u, 0u};
    if (m < mrows) v = *reinterpret_cast<const u32x4*>(A + m * p.lda + c * 8);
    if constexpr (NORM) {
      float sq = 0.f;
      v = norm_chunk<T>(v, *reinterpret_cast<const u32x4*>(
                               static_cast<const uint16_t*>(p.norm_w) + c * 8), sq);
#pragma unroll
      for (int mm = 0; mm < MT; ++mm) rs[mm] += mm == m ? sq : 0.f;
    }
    *reinterpret_cast<u32x4*>(As + (m * nc + c) * 8) = v;
  }
  if constexpr (NORM) {
#pragma unroll
    for (int mm = 0; mm < MT; ++mm) {
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) rs[mm] += __shfl_xor(rs[mm], o, 64);
      if (lane == 0) lds_ss[wave * MT + mm] = rs[mm];
    }
  }
  __syncthreads();
  if constexpr (NORM) {
    const float inv_k = 1.0f / static_cast<float>(p.k);
#pragma unroll
    for (int mm = 0; mm < MT; ++mm) {
      float sq = 0.f;
      for (int w = 0; w < WAVES; ++w) sq += lds_ss[w * MT + mm];
      rs[mm] = rsqrtf(sq * inv_k + p.norm_eps);
    }
  } else {
#pragma unroll
    for (int m = 0; m < MT; ++m) rs[m] = 1.f;
  }
  // Items in order; item i+1 loads while item i computes.  (The next item
  // of the last segment of a row: the next whole row, else the slice.)
#define SPH_GV_NEXT(N2_, CB2_, CE2_, NS2_, S2_, T2_, MORE_)                                  \
  do {                                                                                      \
    N2_ = n, CB2_ = cb, CE2_ = ce, NS2_ = ns, S2_ = s + 1, T2_ = tail, MORE_ = true;        \
    if (S2_ == ns) {                                                                        \
      S2_ = 0;                                                                              \
      if (!tail && n + stride < main_end) {                                                 \
        N2_ = n + stride;                                                                   \
      } else if (!tail && trow >= 0) {                                                      \
        N2_ = trow, CB2_ = tcb, CE2_ = tcb + tcn, NS2_ = tseg, T2_ = true;                  \
      } else {                                                                              \
        MORE_ = false;                                                                      \
      }                                                                                     \
    }                                                                                       \
  } while (0)
  if (have) {
    while (true) {
      int64_t n2;
      int cb2, ce2, ns2, s2;
      bool t2, more;
      SPH_GV_NEXT(n2, cb2, ce2, ns2, s2, t2, more);
      if (more) SPH_GV_LOAD(wb, n2, cb2, s2);
      SPH_GV_COMPUTE(wa, cb, ce, s);
      if (s == ns - 1) SPH_GV_FINISH(n, tail);
      if (!more) break;
      n = n2, cb = cb2, ce = ce2, ns = ns2, s = s2, tail = t2;
      SPH_GV_NEXT(n2, cb2, ce2, ns2, s2, t2, more);
      if (more) SPH_GV_LOAD(wa, n2, cb2, s2);
      SPH_GV_COMPUTE(wb, cb, ce, s);
      if (s == ns - 1) SPH_GV_FINISH(n, tail);
      if (!more) break;
      n = n2, cb = cb2, ce = ce2, ns = ns2, s = s2, tail = t2;
    }
  }
  if (left > 0) {
    // uniform: `left` is the same for every wave of the grid
    __syncthreads();
    if (trow >= 0 && q == 0) {
      float s0[MT], s1[MT];
#pragma unroll
      for (int m = 0; m < MT; ++m) s0[m] = s1[m] = 0.f;
      for (int qq = 0; qq < qn; ++qq) {
        const int w = slot * qn + qq;
#pragma unroll
        for (int m = 0; m < MT; ++m) {
          s0[m] += lds_part[(w * NR) * MT + m];
          s1[m] += lds_part[(w * NR + NR - 1) * MT + m];
        }
      }
      SPH_GV_STORE(trow, s0[m_], s1[m_]);
    }
  }
#undef SPH_GV_NEXT
#undef SPH_GV_LOAD
#undef SPH_GV_COMPUTE
#undef SPH_GV_REDUCE
#undef SPH_GV_STORE
#undef SPH_GV_FINISH
}

// Streaming kernel fit: batch 1, M <= 8, K-contiguous 16-byte aligned rows,
// K % 8 == 0 within the LDS staging size (16384 for M <= 4, else 8192),
// and at least 8 M weights (16 MB of fp16): with the leftover rows split
// along K every wave streams the same share, which beats the small-M
// kernel's many short workgroups from the decode step's 32 MB O projection
// up (measured on MI355X, x[4, 4096] and x[4, 12800]).
constexpr int64_t kStreamMinWeights = 8LL << 20;

inline bool stream_fits(const GemmArgs& p, int64_t batch, bool a_kcont, bool b_kcont) {
  return batch == 1 && p.m >= 1 && p.m <= 8 && a_kcont && b_kcont && p.vec_a && p.vec_b &&
         p.k >= 1024 && p.k % 8 == 0 && p.k <= (p.m <= 4 ? 16384 : 8192) && p.n >= 1024 &&
         p.n < (1LL << 40) && p.n * p.k >= kStreamMinWeights;
}

// Waves per workgroup: 16, or 12 / 10 where that makes the N rows whole
// rounds of the 256-workgroup grid, so that no row is left to split along K
// (decode QKV: 6144 rows = 2 rounds of 12 waves, 15.7 -> 14.0 us; gate/up:
// 12800 rows = 5 rounds of 10 waves, 41.5 -> 39.0 us; measured on MI355X).
constexpr int64_t kStreamCUs = 256;  // one workgroup per MI355X compute unit
inline int stream_waves(int64_t n) {
  if (n % (kStreamCUs * gv::WAVES) == 0) return gv::WAVES;
  for (int w : {12, 10})
    if (n % (kStreamCUs * w) == 0) return w;
  return gv::WAVES;
}

template <typename T, int MT, int KMAX, bool SWIGLU, bool NORM>
void launch_stream_k(const GemmArgs& p, hipStream_t st) {
  const int w = stream_waves(p.n);
  const int64_t wgs = ceil_div(p.n, static_cast<int64_t>(w));
  const unsigned grid = static_cast<unsigned>(wgs < kStreamCUs ? wgs : kStreamCUs);
  if (w == 12)
    gemm_stream_kernel<T, MT, KMAX, SWIGLU, NORM, 12><<<grid, dim3(12 * 64), 0, st>>>(p);
  else if (w == 10)
    gemm_stream_kernel<T, MT, KMAX, SWIGLU, NORM, 10><<<grid, dim3(10 * 64), 0, st>>>(p);
  else
    gemm_stream_kernel<T, MT, KMAX, SWIGLU, NORM, 16><<<grid, dim3(16 * 64), 0, st>>>(p);
}

template <typename T, bool SWIGLU = false, bool NORM = false>
void launch_stream_t(const GemmArgs& p, hipStream_t st) {
  if (p.m <= 4 && p.k > 8192)
    launch_stream_k<T, 4, 16384, SWIGLU, NORM>(p, st);
  else if (p.m <= 4)
    launch_stream_k<T, 4, 8192, SWIGLU, NORM>(p, st);
  else
    launch_stream_k<T, 8, 8192, SWIGLU, NORM>(p, st);
}

template <typename T>
int launch_stream(const GemmArgs& p, hipStream_t st) {
  launch_stream_t<T>(p, st);
  return check_launch("sph_gemm (stream)");
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
template <typename T, int BM, int BN, int WM, int WN, bool FULL>
void launch_full(const GemmArgs& p, dim3 grid, dim3 block, bool a_kcont, bool b_kcont,
                 hipStream_t st) {
  if (a_kcont && b_kcont)
    gemm_kernel<T, BM, BN, WM, WN, true, true, FULL><<<grid, block, 0, st>>>(p);
  else if (a_kcont && !b_kcont)
    gemm_kernel<T, BM, BN, WM, WN, true, false, FULL><<<grid, block, 0, st>>>(p);
  else if (!a_kcont && b_kcont)
    gemm_kernel<T, BM, BN, WM, WN, false, true, FULL><<<grid, block, 0, st>>>(p);
  else
    gemm_kernel<T, BM, BN, WM, WN, false, false, FULL><<<grid, block, 0, st>>>(p);
}

// The direct-load kernel addresses a tile's operand rows with 32-bit buffer
// offsets: every byte it may touch must lie within 2^31 of the tile origin.
inline bool dl_fits(const GemmArgs& p, bool b_kcont, int bn) {
  constexpr int64_t kLim = (1LL << 31) - 1;
  if (p.lda > kLim / 2 || p.ldb > kLim / 2) return false;
  const int64_t a_bytes = ((dl::BM - 1) * p.lda + p.k) * 2;
  const int64_t b_bytes = b_kcont ? ((bn - 1) * p.ldb + p.k) * 2 : ((p.k - 1) * p.ldb + bn) * 2;
  return a_bytes < kLim && b_bytes < kLim;
}

constexpr int64_t kNumCUs = 256;  // MI355X compute units

// Split-K for the last, partial round of 256-wide tiles (batch 1): when
// `tiles` is not a multiple of the CU count, the tail tiles would run as a
// round of their own on a few CUs.  Each tail tile is split into up to 8
// K slices (enough to fill the CUs; K >= 2048, so a slice keeps >= 4 K
// tiles) whose fp32 partial tiles a reduce kernel sums.  A tail of 0 (e.g.
// 4096^3) takes no split.  Measured on one MI355X: the c4 decoder layer
// (M = 2048: gate/up 800 tiles, O and down 128 tiles) 1.143 -> 1.037 ms.
struct SplitPlan {
  int splits = 1, kslice = 0;
  int64_t tail_start = 0, bytes = 0;
};
inline SplitPlan splitk_plan(int64_t tiles, int64_t ksteps, int bn) {
  SplitPlan pl;
  pl.tail_start = tiles;
  if (tiles <= 0 || tiles >= (1LL << 30) || ksteps < 32) return pl;
  const int64_t full = tiles / kNumCUs * kNumCUs, tail = tiles - full;
  if (tail == 0) return pl;
  int64_t sp = kNumCUs / tail;
  sp = sp < 8 ? sp : 8;
  if (sp < 2) return pl;
  const int64_t kslice = ceil_div(ksteps, sp);
  sp = ceil_div(ksteps, kslice);  // every slice non-empty
  if (sp < 2) return pl;
  pl.splits = static_cast<int>(sp);
  pl.kslice = static_cast<int>(kslice);
  pl.tail_start = full;
  pl.bytes = tail * sp * dl::BM * bn * 4;
  return pl;
}

// Time model of the direct-load kernel, fitted to fp16 runs on one MI355X
// (us): a round of 256 x 256 tiles (one per CU) takes ~12 us + 22.4 ns per
// K column (104 us at K = 4096, 299 us at K = 12800); a split-K tail round
// the time of its K slice plus ~4 us and the fp32 partials' write and
// reduce at ~4.2 TB/s (~20 us for the 128 tiles x 2 slices of the c4 O and
// down shapes); a round of 128-wide tiles (8 waves of 128 x 32, half the
// MFMAs per K tile, so less time to cover each tile's loads) 0.62 of a
// 256-wide round with its operands in the caches but 0.78 with operands
// from HBM, as a model layer's weights are (2048 x 4096 x 4096 + residual:
// 65 us hot, 86 us cold, against 76 / 80 us split along K; a cold 256-wide
// round at K = 4096: 109 us).  The model takes the cold figure.
inline double dl_round_us(int64_t k) { return 12.0 + 0.0224 * static_cast<double>(k); }
inline double dl_est128(int64_t tiles128, int64_t k) {
  return static_cast<double>(ceil_div(tiles128, kNumCUs)) * 0.78 * dl_round_us(k);
}
inline double dl_est256(int64_t tiles256, int64_t k) {
  return static_cast<double>(ceil_div(tiles256, kNumCUs)) * dl_round_us(k);
}

// The split plan for `tiles` 256-wide tiles (batch 1, N % 256 == 0) where
// the model puts it ahead of whole rounds of 256- and of 128-wide tiles;
// else a plan of one split (no workspace).
inline SplitPlan splitk_choice(int64_t tiles, int64_t k) {
  const SplitPlan pl = splitk_plan(tiles, k / dl::BKD, 256);
  if (pl.splits <= 1) return pl;
  const double est = static_cast<double>(pl.tail_start / kNumCUs) * dl_round_us(k) +
                     dl_round_us(static_cast<int64_t>(pl.kslice) * dl::BKD) + 4.0 +
                     static_cast<double>(pl.bytes) / 4.2e6;
  if (est < dl_est256(tiles, k) && est < dl_est128(2 * tiles, k)) return pl;
  SplitPlan none;
  none.tail_start = tiles;
  return none;
}

// Launches the direct-load kernel (and, with a split plan, the reduce).
template <typename T, int BN, bool SWIGLU = false, int WTN_ = dl::WTN>
int launch_dl(GemmArgs& p, int64_t batch, bool b_kcont, hipStream_t st,
              const SplitPlan* plan = nullptr) {
  p.tiles_m = static_cast<int>(p.m / dl::BM);
  p.tiles_n = static_cast<int>(p.n / (SWIGLU ? BN / 2 : BN));
  const int64_t tiles = static_cast<int64_t>(p.tiles_m) * p.tiles_n;
  const bool split = plan != nullptr && plan->splits > 1 && batch == 1;
  p.tail_start = static_cast<int>(split ? plan->tail_start : tiles);
  p.splits = split ? plan->splits : 1;
  p.kslice = split ? plan->kslice : 0;
  const int64_t wgs = split ? plan->tail_start + (tiles - plan->tail_start) * plan->splits : tiles;
  dim3 grid(static_cast<unsigned>(wgs), static_cast<unsigned>(batch));
  constexpr int NTH = dl::Cfg<BN, WTN_>::NT;
  if (b_kcont)
    gemm_dl_kernel<T, true, BN, SWIGLU, WTN_><<<grid, dim3(NTH), 0, st>>>(p);
  else if constexpr (!SWIGLU && (BN / 8) % 16 == 0)
    gemm_dl_kernel<T, false, BN, false, WTN_><<<grid, dim3(NTH), 0, st>>>(p);
  if (split) {
    constexpr int OUTN = SWIGLU ? BN / 2 : BN;
    dim3 rg(static_cast<unsigned>(tiles - plan->tail_start), (dl::BM * OUTN) / 1024);
    gemm_splitk_reduce<T, BN, SWIGLU><<<rg, 256, 0, st>>>(p);
  }
  return check_launch("sph_gemm");
}

// Short-K problems of at least this many 128x128 tiles run the persistent
// ring kernel (two or more tiles per workgroup on 256 CUs).
constexpr int64_t kShortkRingTiles = 2 * kStreamCUs;

// Short-K kernel: K of 64 or 128, whole 128x128 tiles, K-contiguous A,
// 16-byte aligned rows everywhere, plain product, 32-bit buffer offsets.
inline bool shortk_fits(const GemmArgs& p, bool a_kcont, bool b_kcont) {
  if (!(p.k == 64 || p.k == 128) || p.m % sk::BM != 0 || p.n % sk::BN != 0 || !a_kcont ||
      !p.vec_a || !p.vec_b || !p.vec_d || p.alpha != 1.f || p.c != nullptr ||
      p.epilogue != SPH_EPI_NONE)
    return false;
  if (p.m / sk::BM * (p.n / sk::BN) >= (1LL << 31)) return false;
  constexpr int64_t kLim = (1LL << 31) - 1;
  if (p.lda > kLim / 2 || p.ldb > kLim / 2) return false;
  const int64_t a_bytes = ((sk::BM - 1) * p.lda + p.k) * 2;
  const int64_t b_bytes = b_kcont ? ((sk::BN - 1) * p.ldb + p.k) * 2 : ((p.k - 1) * p.ldb + sk::BN) * 2;
  return a_bytes < kLim && b_bytes < kLim;
}

// Launches BM x BN tiles on the register-staged kernel: whole tiles with the
// FULL variant on WMF x WNF waves, otherwise the checked one on WMP x WNP.
template <typename T, int BM, int BN, int WMF, int WNF, int WMP, int WNP>
int launch_cfg(GemmArgs& p, int64_t batch, bool a_kcont, bool b_kcont,
               hipStream_t st) {
  p.tiles_m = static_cast<int>(ceil_div(p.m, BM));
  p.tiles_n = static_cast<int>(ceil_div(p.n, BN));
  dim3 grid(static_cast<unsigned>(p.tiles_m) * p.tiles_n, static_cast<unsigned>(batch));
  // Every tile whole and every operand row 16-byte aligned: no bounds or
  // alignment checks in the K loop.
  const bool full = p.m % BM == 0 && p.n % BN == 0 && p.k % BK == 0 && p.k > 0 &&
                    p.vec_a && p.vec_b;
  if (full)
    launch_full<T, BM, BN, WMF, WNF, true>(p, grid, dim3(WMF * WNF * 64), a_kcont, b_kcont, st);
  else
    launch_full<T, BM, BN, WMP, WNP, false>(p, grid, dim3(WMP * WNP * 64), a_kcont, b_kcont, st);
  return check_launch("sph_gemm");
}

inline bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Chooses a tile configuration from the problem shape: 256x256 tiles when
// they give at least one tile per CU, else 128x128 (more workgroups for the
// 256 CUs), else 64x64 for small problems.
template <typename T>
int gemm_dispatch(GemmArgs& p, int64_t batch, bool a_kcont, bool b_kcont,
                  hipStream_t st) {
  if (stream_fits(p, batch, a_kcont, b_kcont))
    return launch_stream<T>(p, st);
  if (p.m <= 16 && a_kcont && b_kcont && p.vec_a && p.vec_b && p.k > 0 && p.k % 8 == 0 &&
      ceil_div(p.n, 2) < (1LL << 40))
    return launch_skinny<T>(p, batch, st);
  if (shortk_fits(p, a_kcont, b_kcont)) {
    p.tiles_m = static_cast<int>(p.m / sk::BM);
    p.tiles_n = static_cast<int>(p.n / sk::BN);
    const int64_t tiles = static_cast<int64_t>(p.tiles_m) * p.tiles_n * batch;
    if (tiles >= kShortkRingTiles && p.tiles_n >= 2) {
      // persistent: one workgroup per CU over runs of at least two tiles
      p.batches = batch;
      const dim3 grid(static_cast<unsigned>(kStreamCUs));
      constexpr int RWM = 2, RWN = 2, RNT = skr::L<RWM, RWN>::NT;
      if (p.k == 64) {
        if (b_kcont) gemm_shortk_ring_kernel<T, true, 1, RWM, RWN><<<grid, dim3(RNT), 0, st>>>(p);
        else gemm_shortk_ring_kernel<T, false, 1, RWM, RWN><<<grid, dim3(RNT), 0, st>>>(p);
      } else {
        if (b_kcont) gemm_shortk_ring_kernel<T, true, 2, RWM, RWN><<<grid, dim3(RNT), 0, st>>>(p);
        else gemm_shortk_ring_kernel<T, false, 2, RWM, RWN><<<grid, dim3(RNT), 0, st>>>(p);
      }
      return check_launch("sph_gemm (short K)");
    }
    dim3 grid(static_cast<unsigned>(p.tiles_m) * p.tiles_n, static_cast<unsigned>(batch));
    if (p.k == 64) {
      if (b_kcont) gemm_shortk_kernel<T, true, 1><<<grid, dim3(sk::NT), 0, st>>>(p);
      else gemm_shortk_kernel<T, false, 1><<<grid, dim3(sk::NT), 0, st>>>(p);
    } else {
      if (b_kcont) gemm_shortk_kernel<T, true, 2><<<grid, dim3(sk::NT), 0, st>>>(p);
      else gemm_shortk_kernel<T, false, 2><<<grid, dim3(sk::NT), 0, st>>>(p);
    }
    return check_launch("sph_gemm (short K)");
  }
  // Whole 256-row tiles with K-contiguous A run the direct-load kernel, 256
  // or 128 columns wide, or 256 wide with the last round split along K:
  // whichever the time model above puts first.
  if (a_kcont && p.m % dl::BM == 0 && p.k % dl::BKD == 0 && p.k > 0 && p.vec_a && p.vec_b &&
      p.n % 128 == 0) {
    auto fill = [](int64_t tiles) {
      return static_cast<double>(tiles) / (static_cast<double>(ceil_div(tiles, kNumCUs)) * kNumCUs);
    };
    const int64_t tw = (p.m / dl::BM) * (p.n / 256) * batch;
    const int64_t tn = (p.m / dl::BM) * (p.n / 128) * batch;
    const bool w256 = p.n % 256 == 0 && dl_fits(p, b_kcont, 256) && tw < (1LL << 31);
    const bool w128 = dl_fits(p, b_kcont, 128) && tn < (1LL << 31);
    // 256 x 192 tiles (8 waves of 128 x 48; K-contiguous B) where they fill
    // whole rounds of the CUs and 256-wide ones do not (QKV at N = 6144:
    // 256 tiles in one round instead of 192, or 512 in two instead of 384)
    const int64_t t192 = p.n % 192 == 0 ? (p.m / dl::BM) * (p.n / 192) * batch : 0;
    if (b_kcont && t192 > 0 && t192 % kNumCUs == 0 && fill(tw) < 1.0 && dl_fits(p, b_kcont, 192) &&
        t192 < (1LL << 31))
      return launch_dl<T, 192, false, 48>(p, batch, b_kcont, st);
    // with a workspace, 256-wide tiles whose last round is split along K
    if (w256 && batch == 1 && p.part != nullptr) {
      const SplitPlan pl = splitk_choice(tw, p.k);
      if (pl.splits > 1 && pl.bytes <= p.part_bytes) return launch_dl<T, 256>(p, batch, b_kcont, st, &pl);
    }
    if (w256 && (!w128 || dl_est256(tw, p.k) <= dl_est128(tn, p.k)))
      return launch_dl<T, 256>(p, batch, b_kcont, st);
    if (w128) return launch_dl<T, 128, false, 32>(p, batch, b_kcont, st);
  }
  const int64_t t256 = ceil_div(p.m, 256) * ceil_div(p.n, 256) * batch;
  const int64_t t128 = ceil_div(p.m, 128) * ceil_div(p.n, 128) * batch;
  // 256x256 whole tiles run 8 waves (128x64 each, two per SIMD, so one
  // wave's LDS and global-load latency hides under the other's MFMAs);
  // partial tiles keep 4 waves, whose bounds-checked loaders need the
  // larger per-wave register budget.
  if (t256 >= 256) return launch_cfg<T, 256, 256, 2, 4, 2, 2>(p, batch, a_kcont, b_kcont, st);
  if (t128 >= 128) return launch_cfg<T, 128, 128, 2, 2, 2, 2>(p, batch, a_kcont, b_kcont, st);
  return launch_cfg<T, 64, 64, 2, 2, 2, 2>(p, batch, a_kcont, b_kcont, st);
}

}  // namespace
}  // namespace sph

using namespace sph;

namespace {
int gemm_entry(sph_dtype dtype, int trans_a, int trans_b, int64_t batch, int64_t m, int64_t n,
               int64_t k, float alpha, const void* a, int64_t lda, int64_t stride_a,
               const void* b, int64_t ldb, int64_t stride_b, float beta, const void* c,
               int64_t ldc_row, int64_t ldc_col, int64_t stride_c, void* d, int64_t ldd,
               int64_t stride_d, int epilogue, void* workspace, int64_t workspace_bytes,
               sph_stream_t stream) {
  SPH_REQUIRE(m >= 0 && n >= 0 && k >= 0 && batch >= 0, SPH_ERR_INVALID_ARG,
              "gemm: negative size");
  SPH_REQUIRE(dtype == SPH_F16 || dtype == SPH_BF16, SPH_ERR_UNSUPPORTED,
              "gemm: dtype must be F16 or BF16");
  SPH_REQUIRE(epilogue >= SPH_EPI_NONE && epilogue <= SPH_EPI_SILU,
              SPH_ERR_INVALID_ARG, "gemm: bad epilogue");
  if (m == 0 || n == 0 || batch == 0) return SPH_OK;
  SPH_REQUIRE(batch <= 65535, SPH_ERR_TOO_LARGE, "gemm: batch > 65535");
  SPH_REQUIRE(ldd >= n, SPH_ERR_INVALID_ARG, "gemm: ldd < n");
  SPH_REQUIRE(k == 0 || (trans_a ? lda >= m : lda >= k), SPH_ERR_INVALID_ARG,
              "gemm: lda too small");
  SPH_REQUIRE(k == 0 || (trans_b ? ldb >= k : ldb >= n), SPH_ERR_INVALID_ARG,
              "gemm: ldb too small");
  SPH_REQUIRE(ceil_div(m, 64) * ceil_div(n, 64) < (1LL << 31), SPH_ERR_TOO_LARGE,
              "gemm: too many tiles");
  GemmArgs p{};
  p.m = m;
  p.n = n;
  p.k = k;
  p.a = a;
  p.lda = lda;
  p.stride_a = stride_a;
  p.b = b;
  p.ldb = ldb;
  p.stride_b = stride_b;
  p.c = (beta != 0.f) ? c : nullptr;
  p.ldc_row = ldc_row;
  p.ldc_col = ldc_col;
  p.stride_c = stride_c;
  p.d = d;
  p.ldd = ldd;
  p.stride_d = stride_d;
  p.alpha = alpha;
  p.beta = beta;
  p.epilogue = epilogue;
  // A is K-contiguous unless transposed; B is K-contiguous when transposed.
  const bool a_kcont = !trans_a, b_kcont = trans_b != 0;
  // 16-byte vector loads need aligned bases and leading dims (and batch
  // strides) that keep every row aligned.
  p.vec_a = al16(a) && (lda % 8 == 0) && (batch == 1 || stride_a % 8 == 0);
  p.vec_b = al16(b) && (ldb % 8 == 0) && (batch == 1 || stride_b % 8 == 0);
  p.vec_d = al16(d) && (ldd % 8 == 0) && (batch == 1 || stride_d % 8 == 0);
  p.part = workspace != nullptr && workspace_bytes > 0 && p.vec_d ? static_cast<float*>(workspace)
                                                                  : nullptr;
  p.part_bytes = p.part != nullptr ? workspace_bytes : 0;
  hipStream_t st = as_stream(stream);
  if (dtype == SPH_F16) return gemm_dispatch<half_t>(p, batch, a_kcont, b_kcont, st);
  return gemm_dispatch<bf16_t>(p, batch, a_kcont, b_kcont, st);
}
}  // namespace

extern "C" int sph_gemm_strided_batched(
    sph_dtype dtype, int trans_a, int trans_b, int64_t batch, int64_t m,
    int64_t n, int64_t k, float alpha, const void* a, int64_t lda,
    int64_t stride_a, const void* b, int64_t ldb, int64_t stride_b, float beta,
    const void* c, int64_t ldc_row, int64_t ldc_col, int64_t stride_c, void* d,
    int64_t ldd, int64_t stride_d, int epilogue, sph_stream_t stream) {
  return gemm_entry(dtype, trans_a, trans_b, batch, m, n, k, alpha, a, lda, stride_a, b, ldb,
                    stride_b, beta, c, ldc_row, ldc_col, stride_c, d, ldd, stride_d, epilogue,
                    nullptr, 0, stream);
}

extern "C" int64_t sph_gemm_workspace_bytes(int64_t batch, int64_t m, int64_t n, int64_t k) {
  if (batch != 1 || m % dl::BM != 0 || n % 256 != 0 || k % dl::BKD != 0 || k <= 0) return 0;
  return splitk_choice((m / dl::BM) * (n / 256), k).bytes;
}

extern "C" int sph_gemm_ex(sph_dtype dtype, int trans_a, int trans_b, int64_t batch, int64_t m,
                           int64_t n, int64_t k, float alpha, const void* a, int64_t lda,
                           int64_t stride_a, const void* b, int64_t ldb, int64_t stride_b,
                           float beta, const void* c, int64_t ldc_row, int64_t ldc_col,
                           int64_t stride_c, void* d, int64_t ldd, int64_t stride_d, int epilogue,
                           void* workspace, int64_t workspace_bytes, sph_stream_t stream) {
  SPH_REQUIRE(workspace_bytes >= 0, SPH_ERR_INVALID_ARG, "gemm: negative workspace size");
  return gemm_entry(dtype, trans_a, trans_b, batch, m, n, k, alpha, a, lda, stride_a, b, ldb,
                    stride_b, beta, c, ldc_row, ldc_col, stride_c, d, ldd, stride_d, epilogue,
                    workspace, workspace_bytes, stream);
}

extern "C" int sph_gemm(sph_dtype dtype, int trans_a, int trans_b, int64_t m,
                        int64_t n, int64_t k, float alpha, const void* a,
                        int64_t lda, const void* b, int64_t ldb, float beta,
                        const void* c, int64_t ldc_row, int64_t ldc_col,
                        void* d, int64_t ldd, int epilogue,
                        sph_stream_t stream) {
  return sph_gemm_strided_batched(dtype, trans_a, trans_b, 1, m, n, k, alpha, a,
                                  lda, 0, b, ldb, 0, beta, c, ldc_row, ldc_col,
                                  0, d, ldd, 0, epilogue, stream);
}

extern "C" int64_t sph_gemm_swiglu_workspace_bytes(int64_t m, int64_t n, int64_t k) {
  if (m <= 8 || m % dl::BM != 0 || n % 128 != 0 || k % dl::BKD != 0 || k <= 0) return 0;
  return splitk_plan((m / dl::BM) * (n / 128), k / dl::BKD, 256).bytes;
}

extern "C" int sph_gemm_swiglu(sph_dtype dtype, int64_t m, int64_t n, int64_t k, const void* a,
                               int64_t lda, const void* w, int64_t ldw, void* d, int64_t ldd,
                               void* workspace, int64_t workspace_bytes, sph_stream_t stream) {
  SPH_REQUIRE(m >= 0 && n >= 0 && k >= 0, SPH_ERR_INVALID_ARG, "gemm_swiglu: negative size");
  SPH_REQUIRE(dtype == SPH_F16 || dtype == SPH_BF16, SPH_ERR_UNSUPPORTED,
              "gemm_swiglu: dtype must be F16 or BF16");
  if (m == 0 || n == 0) return SPH_OK;
  SPH_REQUIRE(lda >= k && ldw >= k && ldd >= n, SPH_ERR_INVALID_ARG,
              "gemm_swiglu: leading dimension too small");
  SPH_REQUIRE(al16(a) && al16(w) && lda % 8 == 0 && ldw % 8 == 0, SPH_ERR_UNSUPPORTED,
              "gemm_swiglu: rows of x and w must be 16-byte aligned");
  if (m <= 8) {
    // decode shapes: the weight-stream kernel, gate and up rows per wave
    SPH_REQUIRE(k >= 64 && k % 8 == 0 && k <= 8192 && n < (1LL << 40), SPH_ERR_UNSUPPORTED,
                "gemm_swiglu: small m needs 64 <= k <= 8192, k % 8 == 0");
    GemmArgs q{};
    q.m = m;
    q.n = n;
    q.k = k;
    q.a = a;
    q.lda = lda;
    q.b = w;
    q.ldb = ldw;
    q.d = d;
    q.ldd = ldd;
    q.alpha = 1.f;
    hipStream_t st = as_stream(stream);
#define SPH_SW_STREAM(T_)                                                                       \
  do {                                                                                          \
    if (m <= 4)                                                                                 \
      launch_stream_k<T_, 4, 8192, true, false>(q, st);                                         \
    else                                                                                        \
      launch_stream_k<T_, 8, 8192, true, false>(q, st);                                         \
  } while (0)
    if (dtype == SPH_F16)
      SPH_SW_STREAM(half_t);
    else
      SPH_SW_STREAM(bf16_t);
#undef SPH_SW_STREAM
    return check_launch("sph_gemm_swiglu (stream)");
  }
  SPH_REQUIRE(m % dl::BM == 0 && n % 128 == 0 && k > 0 && k % dl::BKD == 0, SPH_ERR_UNSUPPORTED,
              "gemm_swiglu: needs m <= 8, or m % 256 == 0, n % 128 == 0, k % 64 == 0");
  SPH_REQUIRE(al16(d) && ldd % 8 == 0, SPH_ERR_UNSUPPORTED,
              "gemm_swiglu: rows of d must be 16-byte aligned");
  constexpr int64_t kLim = 1LL << 31;
  SPH_REQUIRE(((dl::BM - 1) * lda + k) * 2 < kLim && ((n + 127) * ldw + k) * 2 < kLim &&
                  (m / dl::BM) * (n / 128) < kLim,
              SPH_ERR_TOO_LARGE, "gemm_swiglu: operands too large for 32-bit tile offsets");
  GemmArgs p{};
  p.m = m;
  p.n = n;
  p.k = k;
  p.a = a;
  p.lda = lda;
  p.b = w;
  p.ldb = ldw;
  p.d = d;
  p.ldd = ldd;
  p.alpha = 1.f;
  p.epilogue = SPH_EPI_NONE;
  p.vec_a = p.vec_b = p.vec_d = 1;
  hipStream_t st = as_stream(stream);
  const SplitPlan pl = splitk_plan((m / dl::BM) * (n / 128), k / dl::BKD, 256);
  const bool split = pl.splits > 1 && workspace != nullptr && workspace_bytes >= pl.bytes;
  p.part = split ? static_cast<float*>(workspace) : nullptr;
  if (dtype == SPH_F16)
    return launch_dl<half_t, 256, true>(p, 1, true, st, split ? &pl : nullptr);
  return launch_dl<bf16_t, 256, true>(p, 1, true, st, split ? &pl : nullptr);
}

extern "C" int sph_gemm_rmsnorm(sph_dtype dtype, int64_t m, int64_t n, int64_t k, const void* a,
                                int64_t lda, const void* norm_w, float eps, const void* w,
                                int64_t ldw, void* d, int64_t ldd, int swiglu,
                                sph_stream_t stream) {
  SPH_REQUIRE(dtype == SPH_F16 || dtype == SPH_BF16, SPH_ERR_UNSUPPORTED,
              "gemm_rmsnorm: dtype must be F16 or BF16");
  SPH_REQUIRE(m >= 0 && n >= 0 && k >= 0, SPH_ERR_INVALID_ARG, "gemm_rmsnorm: negative size");
  if (m == 0 || n == 0) return SPH_OK;
  SPH_REQUIRE(m <= 8, SPH_ERR_UNSUPPORTED, "gemm_rmsnorm: at most 8 rows (decode shapes)");
  SPH_REQUIRE(k >= 64 && k % 8 == 0 && k <= 8192, SPH_ERR_UNSUPPORTED,
              "gemm_rmsnorm: needs 64 <= k <= 8192, k % 8 == 0");
  SPH_REQUIRE(std::isfinite(eps) && eps >= 0.f, SPH_ERR_INVALID_ARG,
              "gemm_rmsnorm: eps must be finite and >= 0");
  SPH_REQUIRE(lda >= k && ldw >= k && ldd >= n && n < (1LL << 40), SPH_ERR_INVALID_ARG,
              "gemm_rmsnorm: leading dimension too small");
  SPH_REQUIRE(al16(a) && al16(w) && al16(norm_w) && lda % 8 == 0 && ldw % 8 == 0,
              SPH_ERR_UNSUPPORTED, "gemm_rmsnorm: x, norm_w and w rows must be 16-byte aligned");
  GemmArgs q{};
  q.m = m;
  q.n = n;
  q.k = k;
  q.a = a;
  q.lda = lda;
  q.b = w;
  q.ldb = ldw;
  q.d = d;
  q.ldd = ldd;
  q.alpha = 1.f;
  q.epilogue = SPH_EPI_NONE;
  q.vec_a = q.vec_b = 1;
  q.vec_d = al16(d) && ldd % 8 == 0;
  q.norm_w = norm_w;
  q.norm_eps = eps;
  hipStream_t st = as_stream(stream);
#define SPH_RN_STREAM(T_, SW_)                                                              \
  do {                                                                                      \
    if (m <= 4)                                                                             \
      launch_stream_k<T_, 4, 8192, SW_, true>(q, st);                                       \
    else                                                                                    \
      launch_stream_k<T_, 8, 8192, SW_, true>(q, st);                                       \
  } while (0)
  if (swiglu) {
    // w holds the gate rows [0, n) and the up rows [n, 2n)
    if (dtype == SPH_F16) SPH_RN_STREAM(half_t, true);
    else SPH_RN_STREAM(bf16_t, true);
    return check_launch("sph_gemm_rmsnorm (swiglu stream)");
  }
  if (stream_fits(q, 1, true, true)) {
    if (dtype == SPH_F16) SPH_RN_STREAM(half_t, false);
    else SPH_RN_STREAM(bf16_t, false);
    return check_launch("sph_gemm_rmsnorm (stream)");
  }
#undef SPH_RN_STREAM
  if (dtype == SPH_F16) return launch_skinny<half_t, true>(q, 1, st);
  return launch_skinny<bf16_t, true>(q, 1, st);
}

extern "C" int sph_gemm_f16(int64_t m, int64_t n, int64_t k, const void* a,
                            const void* b, void* d, sph_stream_t stream) {
  return sph_gemm(SPH_F16, 0, 0, m, n, k, 1.0f, a, k, b, n, 0.0f, nullptr, 0, 0,
                  d, n, SPH_EPI_NONE, stream);
}

extern "C" int sph_bmm_f16(int64_t batch, int64_t m, int64_t n, int64_t k,
                           const void* a, const void* b, void* d,
                           sph_stream_t stream) {
  return sph_gemm_strided_batched(SPH_F16, 0, 0, batch, m, n, k, 1.0f, a, k,
                                  m * k, b, n, k * n, 0.0f, nullptr, 0, 0, 0, d,
                                  n, m * n, SPH_EPI_NONE, stream);
}
