// Fused attention forward: O = softmax(scale * Q K^T + mask) V for fp16 /
// bf16, head dim 128, without materialising the score matrix.
//
// Shapes: per batch b (one KV head with its stacked query heads), Q is
// [mq, 128], K and V are [sk, 128], O is [mq, 128]; rows of every operand
// are 16-byte aligned with arbitrary leading dims.  Masking: an additive
// [mq, sk] mask (natural-log units, -inf to drop a key) and/or causal
// positions (row r sits at position r % causal_q + causal_off and sees keys
// <= that position).
//
// Design (gfx950, MFMA 32x32x16):
//   * A workgroup of 4 waves takes 128 query rows (32 per wave) and walks
//     the keys in blocks of 64.  K and V blocks move into LDS by direct
//     global->LDS DMA (buffer_load_dwordx4 ... lds), two stages deep.
//   * Scores are computed transposed, S^T = K Q^T (K fragments from LDS as
//     the MFMA's first operand, the wave's Q fragments held in registers as
//     the second): each lane then owns one query column and 32 of the
//     block's scores for it, so the row max and sum are in-lane reductions
//     plus one exchange with the lane 32 away.
//   * The output is accumulated transposed too, O^T += V^T P^T: P^T is the
//     score accumulator itself (converted to fp16), V^T fragments come from
//     the N-contiguous V block through ds_read_b64_tr_b16.  The MFMA's 16 K
//     slots are mapped to keys so that a lane's 8 P values are 8
//     consecutive accumulator registers and its V values two 4-key
//     transpose reads.  The online-softmax rescale of O is per lane (each
//     lane's O^T registers belong to its query) - no shuffles.
//   * exp is computed as exp2 with scale * log2(e) folded into the scores.
//   * Causal: key blocks past the last position of the workgroup's rows are
//     skipped (about half the work for a square causal problem).
//   * LDS layouts chosen so every fragment read is a per-lane base plus a
//     compile-time offset (fewer live address registers) and bank-conflict
//     free: K rows are padded to 272 bytes (16 consecutive rows at one
//     16-byte chunk start 68 banks apart); V is split by 32-wide head-dim
//     slab, [dt][key][32 values], 64-byte rows, so a transpose read's 4 rows
//     x 4 chunks are one contiguous 256-byte run.
//   * Masks: a pre-pass classes every (128-row, 64-key) block of the mask as
//     all zero, mixed or all -inf (one byte each).  A workgroup walks only
//     the key range between its first and last block that is not all -inf,
//     skips all -inf blocks inside it and loads mask values only for mixed
//     blocks - a causal mask then costs what the causal-position mode costs.
//   * A workgroup is 8 waves in two groups of 4 on the same 128 query rows:
//     group g takes the key blocks kb with kb % 2 == g, each group with its
//     own two-stage LDS ring, and the two partial softmax states merge
//     through LDS at the end.  (Without a mask or causal positions, where
//     every job is equally long, one group per workgroup: the two groups of
//     one workgroup meet at every block's barrier, so their MFMA and
//     softmax phases coincide, while two workgroups on a CU drift apart.)
//     One 8-wave workgroup fills a CU (two waves per SIMD), so the grid is
//     longer than the CU count and its order matters:
//     jobs run longest first (causal positions: by position block; masks:
//     by the number of key blocks the mask leaves, counted and sorted on the
//     device from the block classes), so short jobs fill in behind long
//     ones.
#include <mutex>

#include "sph_common.h"

namespace sph {
namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
#define SPH_LDS __attribute__((address_space(3)))

constexpr int AQ = 128;   // query rows per workgroup (32 per wave)
constexpr int AK = 64;    // keys per block
constexpr int AD = 128;   // head dim
constexpr int KPITCH = AD * 2 + 16;       // padded K row (bytes)
constexpr int KBLK = AK * KPITCH;         // 17408 bytes: 17 DMA lines of 1 KB
constexpr int VBLK = AK * AD * 2;         // 16384 bytes: 16 lines
constexpr int KLINES = KBLK / 1024, VLINES = VBLK / 1024;
constexpr int STAGE = KBLK + VBLK;
constexpr int kMaxOrderBins = 4097;  // key blocks + 1 the job sort handles
static_assert(KBLK % 1024 == 0 && VBLK % 1024 == 0, "whole DMA lines");

struct AttnArgs {
  int64_t mq, sk;
  const void* q;
  int64_t ldq, sq;
  const void* k;
  int64_t ldk, skb;
  const void* v;
  int64_t ldv, svb;
  const void* mask;
  int64_t ldm, smb;
  int64_t causal_q, causal_off;
  int64_t batch, nbq;   // batch, query blocks per batch element (mq / 128)
  int64_t heads;        // > 0: causal rows are `heads` stacked runs of causal_q
  const int32_t* order; // job order (b * nbq + rb), longest first, or null
  const uint8_t* mblk;  // mask block classes [mask batch][nbq][nkb] or null
  int64_t mblk_b;       // row blocks per mask batch in mblk (0: one mask for all)
  int64_t nkb;          // key blocks (ceil(sk / 64))
  float scale_log2;  // scale * log2(e) (scale > 0)
  float inv_scale;   // 1 / scale: masks join the raw scores as mask / scale
  void* o;
  int64_t ldo, so;
};

template <typename T>
__device__ inline f32x16 mfma(u32x4 a, u32x4 b, f32x16 c) {
  if constexpr (__is_same(T, half_t)) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
}

// Two floats rounded to the nearest even element value and packed, lo in the
// low half: one v_cvt_pk_f16_f32 / v_cvt_pk_bf16_f32 (gfx950) instead of two
// conversions and an OR (the score-to-probability step packs 32 values per
// lane and key block; measured 2-3 % of the kernel, same bits).
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
template <typename T>
__device__ inline uint32_t pack2(float lo, float hi) {
  const f32x2_t v = {lo, hi};
  if constexpr (__is_same(T, half_t))
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2_t));
  else
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

__device__ inline i32x4 buffer_rsrc(const void* base, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  i32x4 r;
  r[0] = __builtin_amdgcn_readfirstlane(static_cast<int32_t>(static_cast<uint32_t>(a)));
  r[1] = __builtin_amdgcn_readfirstlane(static_cast<int32_t>(static_cast<uint32_t>(a >> 32) & 0xffffu));
  r[2] = __builtin_amdgcn_readfirstlane(static_cast<int32_t>(bytes));
  r[3] = 0x00020000;
  return r;
}
// 16 bytes per lane from rsrc[voff + soff] into LDS at lds_addr + 16 * lane
// (inline asm: the compiler would otherwise wait for it before every LDS
// read; completion is awaited explicitly).
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
// s_waitcnt immediate for vmcnt(0) alone (gfx9 fields: vmcnt [3:0] and
// [15:14], expcnt [6:4], lgkmcnt [11:8]; the others at their maximum).
constexpr int kWaitVmcnt0 = 0x0F70;

// Mask block classes (values of the pre-pass's bytes).
constexpr uint8_t MB_ZERO = 0, MB_MIXED = 1, MB_NEGINF = 2;

// One workgroup per (mask batch, row block, key block): class the block's
// 128 x 64 mask values (keys past sk ignored).  The classes are read off the
// 16-bit patterns (fp16 and bf16 alike: zero is +-0, -inf is one pattern), two
// values per 32-bit word, and the workgroup's verdicts meet in one LDS word
// per wave behind a single barrier.
template <typename T>
__global__ void __launch_bounds__(256) mask_blocks_kernel(const uint16_t* __restrict__ mask,
                                                          int64_t ldm, int64_t smb, int64_t sk,
                                                          int64_t nbq, int64_t nkb,
                                                          uint8_t* __restrict__ out) {
  constexpr uint16_t kNegInf = __is_same(T, half_t) ? 0xFC00u : 0xFF80u;
  constexpr uint32_t kNegInf2 = (static_cast<uint32_t>(kNegInf) << 16) | kNegInf;
  __shared__ uint32_t votes[4];
  const int64_t kb = blockIdx.x, rb = blockIdx.y, mb = blockIdx.z;
  const int t = threadIdx.x;
  const uint16_t* M = mask + mb * smb + (rb * AQ) * ldm + kb * AK;
  const int64_t kn = sk - kb * AK;  // keys of this block (<= 64 counts)
  bool nonzero = false, finite = false;
  // 128 rows x 8 chunks of 8 keys: 4 chunks per thread, all loads first
  u32x4 w[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c = t + 256 * i, r = c >> 3, k8 = (c & 7) * 8;
    if (k8 + 8 <= kn) w[i] = *reinterpret_cast<const u32x4*>(M + r * ldm + k8);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c = t + 256 * i, r = c >> 3, k8 = (c & 7) * 8;
    if (k8 + 8 <= kn) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        nonzero |= (w[i][e] & 0x7fff7fffu) != 0u;
        finite |= w[i][e] != kNegInf2;
      }
    } else {
      for (int e = 0; e < 8 && k8 + e < kn; ++e) {
        const uint16_t bits = M[r * ldm + k8 + e];
        nonzero |= (bits & 0x7fffu) != 0u;
        finite |= bits != kNegInf;
      }
    }
  }
  const uint64_t bnz = __ballot(nonzero), bfin = __ballot(finite);
  if (t % kWave == 0) votes[t / kWave] = (bnz != 0 ? 1u : 0u) | (bfin != 0 ? 2u : 0u);
  __syncthreads();
  if (t == 0) {
    const uint32_t v = votes[0] | votes[1] | votes[2] | votes[3];
    out[(mb * nbq + rb) * nkb + kb] = !(v & 2u) ? MB_NEGINF : ((v & 1u) ? MB_MIXED : MB_ZERO);
  }
}

// One workgroup: the jobs (b * nbq + rb) counting-sorted by the number of
// key blocks their mask leaves (first to last block not all -inf), longest
// first, into order[].  The classes of every job (jobs * nkb bytes, at most
// kMaxOrderBytes) are staged in LDS with 16-byte loads first.  Ties keep no
// particular order.
constexpr int kMaxOrderBytes = 48 * 1024;
__global__ void __launch_bounds__(1024) attn_order_kernel(const uint8_t* __restrict__ mblk,
                                                          int64_t mblk_b, int nkb, int nbq,
                                                          int jobs, int32_t* __restrict__ order) {
  __shared__ __attribute__((aligned(16))) uint8_t cls[kMaxOrderBytes];
  __shared__ int cnt[kMaxOrderBins];
  // the class rows are contiguous per mask batch: [mask batch][rb][kb]
  const int per_mb = nbq * nkb, nmb = mblk_b == 0 ? 1 : jobs / nbq;
  const int total = nmb * per_mb;
  for (int i = threadIdx.x * 16; i < total; i += 1024 * 16) {
    if (i + 16 <= total && ((reinterpret_cast<uintptr_t>(mblk) + i) & 15) == 0)
      *reinterpret_cast<u32x4*>(cls + i) = *reinterpret_cast<const u32x4*>(mblk + i);
    else
      for (int e = i; e < i + 16 && e < total; ++e) cls[e] = mblk[e];
  }
  for (int i = threadIdx.x; i <= nkb; i += 1024) cnt[i] = 0;
  __syncthreads();
  auto work = [&](int job) {
    const uint8_t* c = cls + ((mblk_b == 0 ? 0 : job / nbq) * nbq + job % nbq) * nkb;
    int lo = -1, hi = -1;
    for (int kb = 0; kb < nkb; ++kb)
      if (c[kb] != MB_NEGINF) {
        lo = lo < 0 ? kb : lo;
        hi = kb;
      }
    return hi < 0 ? 0 : hi - lo + 1;
  };
  for (int jb = threadIdx.x; jb < jobs; jb += 1024) atomicAdd(&cnt[work(jb)], 1);
  __syncthreads();
  if (threadIdx.x == 0) {
    int off = 0;
    for (int w = nkb; w >= 0; --w) {
      const int c = cnt[w];
      cnt[w] = off;
      off += c;
    }
  }
  __syncthreads();
  for (int jb = threadIdx.x; jb < jobs; jb += 1024) order[atomicAdd(&cnt[work(jb)], 1)] = jb;
}

template <typename T, bool MASK, bool CAUSAL, int GR>
__global__ void __launch_bounds__(GR * 256) __attribute__((amdgpu_waves_per_eu(2)))
attn_fwd_kernel(const AttnArgs p) {
  static_assert(GR == 1 || GR == 2, "key-block groups");
  __shared__ __attribute__((aligned(1024))) char lds[2 * GR * STAGE];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int grp = GR == 2 ? wave >> 2 : 0, wq = wave & 3;  // key-block group, wave within it (its rows)
  // The job: batch element b, row block rb.
  int64_t b, rb;
  const int64_t wg = blockIdx.x;
  if (p.order != nullptr) {
    const int64_t job = p.order[wg];
    b = job / p.nbq;
    rb = job % p.nbq;
  } else if (CAUSAL && p.heads > 0) {
    // longest first: position block descending, then batch and head
    const int64_t per = p.batch * p.heads, nbh = p.nbq / p.heads;
    const int64_t pb = nbh - 1 - wg / per, rem = wg % per;
    b = rem / p.heads;
    rb = (rem % p.heads) * nbh + pb;
  } else {
    b = wg / p.nbq;
    rb = wg % p.nbq;
  }
  const int64_t r0 = rb * AQ;                                 // first row of the workgroup
  const int64_t qrow = r0 + wq * 32 + (lane & 31);           // this lane's query row
  const int h = lane >> 5;

  // Key blocks this workgroup walks: [kb0, kb1).
  int64_t kend = p.sk;
  if constexpr (CAUSAL) {
    const int64_t last = r0 + AQ - 1;
    const int64_t pmax = (r0 / p.causal_q == last / p.causal_q) ? last % p.causal_q + p.causal_off
                                                                : p.causal_q - 1 + p.causal_off;
    kend = pmax + 1 < kend ? pmax + 1 : kend;
  }
  int kb0 = 0, kb1 = kend <= 0 ? 0 : static_cast<int>((kend + AK - 1) / AK);
  const uint8_t* mcls = nullptr;
  if (MASK && p.mblk != nullptr) {
    // first and last key block not entirely -inf
    mcls = p.mblk + (b * p.mblk_b + rb) * p.nkb;  // [mask batch][rb][kb]
    int lo = 0x7fffffff, hi = -1;
    for (int kb = lane; kb < kb1; kb += 64)
      if (mcls[kb] != MB_NEGINF) {
        lo = lo < kb ? lo : kb;
        hi = kb;
      }
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) {
      const int ol = __shfl_xor(lo, d, 64), oh = __shfl_xor(hi, d, 64);
      lo = lo < ol ? lo : ol;
      hi = hi > oh ? hi : oh;
    }
    kb0 = __builtin_amdgcn_readfirstlane(hi < 0 ? 0 : lo);
    kb1 = __builtin_amdgcn_readfirstlane(hi + 1);
  }
  // causal position of this lane's row and the smallest over the wave's 32
  // rows (blocks wholly at or below it need no per-key position check)
  const int qpos = CAUSAL ? static_cast<int>(qrow % p.causal_q + p.causal_off) : 0;
  int qpos_min = qpos;
  if constexpr (CAUSAL) {
#pragma unroll
    for (int d = 16; d >= 1; d >>= 1) qpos_min = min(qpos_min, __shfl_xor(qpos_min, d, 64));
    qpos_min = __builtin_amdgcn_readfirstlane(qpos_min);
  }
  const int sk32 = static_cast<int>(p.sk);

  // Q fragments: query qrow, head dims 16 kk + 8 h .. + 7.
  const uint16_t* Q = static_cast<const uint16_t*>(p.q) + b * p.sq + qrow * p.ldq;
  u32x4 qf[AD / 16];
#pragma unroll
  for (int kk = 0; kk < AD / 16; ++kk) qf[kk] = *reinterpret_cast<const u32x4*>(Q + 16 * kk + 8 * h);

  // DMA set-up.  K line L: 16-byte slot s = L*64 + lane of the padded
  // block, row s / 17, chunk s % 17 (chunk 16 is the pad: it fetches
  // nothing - its offset lies past the buffer range, which reads zeros).
  // V line L: slab dt = L / 4, keys 16 (L % 4) .., lanes in runs of 4
  // chunks per key.
  // Each block gets buffer resources based at its first key and bounded by
  // its last valid key, so rows past sk read zeros.
  const uint16_t* Kb = static_cast<const uint16_t*>(p.k) + b * p.skb;
  const uint16_t* Vb = static_cast<const uint16_t*>(p.v) + b * p.svb;
  // lines handled by this wave of its group: K lines wq, wq+4, ... (< 17),
  // V lines 4 per wave
  constexpr int KLW = (KLINES + 3) / 4, VLW = VLINES / 4;
  uint32_t vk[KLW], vv[VLW];
#pragma unroll
  for (int i = 0; i < KLW; ++i) {
    const int s = (wq + 4 * i) * 64 + lane;
    const int r = s / 17, c = s % 17;
    vk[i] = c < 16 ? static_cast<uint32_t>(r * p.ldk * 2 + c * 16) : 0xffffffffu;
  }
#pragma unroll
  for (int i = 0; i < VLW; ++i) {
    const int L = wq * VLW + i;
    const int dt = L >> 2, key = (L & 3) * 16 + (lane >> 2), c = 4 * dt + (lane & 3);
    vv[i] = static_cast<uint32_t>(key * p.ldv * 2 + c * 16);
  }
  const uint32_t lds_base = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((SPH_LDS char*)(lds)));
  auto issue = [&](int blk, int slot) {  // this group's ring slot
    const uint32_t sbase = lds_base + (grp * 2 + slot) * STAGE;
    const int64_t key0 = static_cast<int64_t>(blk) * AK;
    const int64_t nk = p.sk - key0 < AK ? p.sk - key0 : AK;
    const i32x4 rk = buffer_rsrc(Kb + key0 * p.ldk, static_cast<uint32_t>(((nk - 1) * p.ldk + AD) * 2));
    const i32x4 rv = buffer_rsrc(Vb + key0 * p.ldv, static_cast<uint32_t>(((nk - 1) * p.ldv + AD) * 2));
#pragma unroll
    for (int i = 0; i < KLW; ++i)
      if (wq + 4 * i < KLINES)
        dma16(rk, __builtin_amdgcn_readfirstlane(sbase + (wq + 4 * i) * 1024), vk[i], 0u);
#pragma unroll
    for (int i = 0; i < VLW; ++i)
      dma16(rv, __builtin_amdgcn_readfirstlane(sbase + KBLK + (wq * VLW + i) * 1024), vv[i], 0u);
  };

  // Fragment read bases of this lane (block-relative bytes): K row
  // lane % 32, chunk h; V^T transpose pointer at key 4 (g >> 1) + e, column
  // 16 (g & 1) + 4 q4 of slab 0.
  const int g = lane >> 4, jj = lane & 15, e = jj >> 2, q4 = jj & 3;
  const int kbase_lane = (lane & 31) * KPITCH + h * 16;
  const int vbase_lane = (4 * (g >> 1) + e) * 64 + (16 * (g & 1) + 4 * q4) * 2;
  f32x16 o[AD / 32];
#pragma unroll
  for (int t = 0; t < AD / 32; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[t][r] = 0.f;
  // Online softmax state per row, in log2 units: O and l are relative to
  // 2^m_ref; m_ref follows the running max lazily (moved only when a row's
  // max passes it by more than 8, so exp2 arguments stay <= 8 and most
  // blocks skip the rescale of O).
  float m_ref = -INFINITY, l_run = 0.f;
  const uint16_t* Mrow =
      MASK ? static_cast<const uint16_t*>(p.mask) + b * p.smb + qrow * p.ldm : nullptr;

  // Group g takes key blocks base + 2 it + g, it = 0 .. nit-1 (those in
  // [kb0, kb1)); base is kb0 rounded down to even, so which group a block
  // goes to does not depend on kb0.
  const int base = GR == 2 ? kb0 & ~1 : kb0;
  const int nit = kb1 > base ? (kb1 - base + GR - 1) / GR : 0;
  auto blk_of = [&](int it) { return base + GR * it + grp; };
  auto valid = [&](int kb) { return kb >= kb0 && kb < kb1; };
  auto cls_of = [&](int kb) -> uint8_t {  // (all mixed without the pre-pass)
    return !valid(kb) ? MB_NEGINF : MASK ? (mcls != nullptr ? mcls[kb] : MB_MIXED) : MB_ZERO;
  };

  {
    const bool v0 = nit > 0 && valid(blk_of(0)), v1 = nit > 1 && valid(blk_of(1));
    if (v0) issue(blk_of(0), 0);
    if (v1) issue(blk_of(1), 1);
    // Q fragments and both blocks landed.  The wait is the builtin (which
    // the compiler's wait-count pass sees), not inline asm: the pass does
    // not count the DMA and would otherwise place waits for the Q loads at
    // their uses inside the loop, where the hardware counter also holds the
    // DMA of a later block - every block would then wait for that DMA.
    __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
  }
  __syncthreads();
  for (int it = 0; it < nit; ++it) {
    const int kb = blk_of(it), slot = it & 1;
    const char* sK = lds + (grp * 2 + slot) * STAGE;
    const char* sV = sK + KBLK;
    const uint8_t cls = cls_of(kb);
    if (cls != MB_NEGINF) {
    // S^T for this block: two 32-key tiles.
    f32x16 s[2];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) s[t][r] = 0.f;
#pragma unroll
    for (int kk = 0; kk < AD / 16; ++kk) {
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const u32x4 kf = *reinterpret_cast<const u32x4*>(sK + kbase_lane + t * 32 * KPITCH + kk * 32);
        s[t] = mfma<T>(kf, qf[kk], s[t]);
      }
    }
    // Raw scores (the scale joins in the exponent); keys past sk and past a
    // row's position dropped, checked only in blocks that reach them.
    const int k0 = kb * AK;
    if (k0 + AK > sk32 || (CAUSAL && k0 + AK - 1 > qpos_min)) {
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int rg = 0; rg < 4; ++rg)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int key = k0 + t * 32 + 8 * rg + 4 * h + i;
            bool keep = key < sk32;
            if constexpr (CAUSAL) keep = keep && key <= qpos;
            s[t][4 * rg + i] = keep ? s[t][4 * rg + i] : -INFINITY;
          }
    }
    // Mixed mask blocks: add mask / scale.  Lane's keys for (t, rg):
    // k0 + 32 t + 8 rg + 4 h .. + 3, one 8-byte load each.
    if (MASK && cls == MB_MIXED) {
      const uint16_t* mp = Mrow + k0 + 4 * h;
      if (k0 + AK <= p.sk) {
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int rg = 0; rg < 4; ++rg) {
            const u32x2 mv = *reinterpret_cast<const u32x2*>(mp + 32 * t + 8 * rg);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const uint16_t bits = static_cast<uint16_t>(mv[i >> 1] >> (16 * (i & 1)));
              s[t][4 * rg + i] = fmaf(Num<T>::to_f(__builtin_bit_cast(T, bits)), p.inv_scale,
                                      s[t][4 * rg + i]);
            }
          }
      } else {
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int rg = 0; rg < 4; ++rg)
#pragma unroll
            for (int i = 0; i < 4; ++i)
              if (k0 + 32 * t + 8 * rg + 4 * h + i < sk32)
                s[t][4 * rg + i] = fmaf(Num<T>::to_f(reinterpret_cast<const T*>(mp)[32 * t + 8 * rg + i]),
                                        p.inv_scale, s[t][4 * rg + i]);
      }
    }
    float mb = -INFINITY;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) mb = fmaxf(mb, s[t][r]);
    mb = fmaxf(mb, __shfl_xor(mb, 32, 64));
    const float c = p.scale_log2;
    const float mbc = mb * c;  // block max, log2 units (-inf: nothing visible)
    const bool grow = mbc > m_ref + 8.f;
    if (__ballot(grow) != 0) {  // wave-uniform: some row moves its reference
      const float m_new = grow ? mbc : m_ref;
      const float alpha = grow ? __builtin_amdgcn_exp2f(m_ref - m_new) : 1.f;
      l_run *= alpha;
#pragma unroll
      for (int dt = 0; dt < AD / 32; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[dt][r] *= alpha;
      m_ref = m_new;
    }
    const float neg = m_ref == -INFINITY ? 0.f : -m_ref;
    float lb = 0.f;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float pr = __builtin_amdgcn_exp2f(fmaf(s[t][r], c, neg));
        s[t][r] = pr;
        lb += pr;
      }
    lb += __shfl_xor(lb, 32, 64);
    l_run += lb;
    // O^T += V^T P^T over the block's 4 sixteen-key steps.
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int t = c >> 1, rb = 8 * (c & 1);
      u32x4 pf;
#pragma unroll
      for (int i = 0; i < 4; ++i) pf[i] = pack2<T>(s[t][rb + 2 * i], s[t][rb + 2 * i + 1]);
#pragma unroll
      for (int dt = 0; dt < AD / 32; ++dt) {
        // slab dt, key rows 16 c + 4 (g >> 1) + e (+ 8 for the second read)
        const SPH_LDS char* p0 =
            (const SPH_LDS char*)(sV) + vbase_lane + dt * (AK * 64) + 16 * c * 64;
        const u32x2 lo = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((SPH_LDS s16x4*)(p0)));
        const u32x2 hi = __builtin_bit_cast(
            u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((SPH_LDS s16x4*)(p0 + 8 * 64)));
        const u32x4 vf = __builtin_shufflevector(lo, hi, 0, 1, 2, 3);
        o[dt] = mfma<T>(vf, pf, o[dt]);
      }
    }
    }  // cls != MB_NEGINF
    // The group's next block landed (own DMA) and every wave is done with
    // this slot.
    wait_vmcnt<0>();
    __syncthreads();
    if (it + 2 < nit && valid(blk_of(it + 2))) issue(blk_of(it + 2), slot);
  }
  if constexpr (GR == 2) {
  // Merge: group 1 hands (m_ref, l, O) to the group-0 lane of the same row
  // through LDS (all DMA has landed: the loop ends with a wait + barrier).
  float* mg = reinterpret_cast<float*>(lds) + wq * (66 * 64) + lane;
  if (grp == 1) {
    mg[0] = m_ref;
    mg[64] = l_run;
#pragma unroll
    for (int dt = 0; dt < AD / 32; ++dt)
#pragma unroll
      for (int r = 0; r < 16; ++r) mg[(2 + dt * 16 + r) * 64] = o[dt][r];
  }
  __syncthreads();
  if (grp == 1) return;
  {
    const float m1 = mg[0], l1 = mg[64];
    const float m = fmaxf(m_ref, m1);
    const float a0 = m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m_ref - m);
    const float a1 = m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m1 - m);
    l_run = l_run * a0 + l1 * a1;
#pragma unroll
    for (int dt = 0; dt < AD / 32; ++dt)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[dt][r] = o[dt][r] * a0 + mg[(2 + dt * 16 + r) * 64] * a1;
  }
  }
  // O[qrow][d], d = 32 dt + 8 rg + 4 h + i, normalised by the row sum.
  const float inv = 1.0f / l_run;
  uint16_t* O = static_cast<uint16_t*>(p.o) + b * p.so + qrow * p.ldo;
#pragma unroll
  for (int dt = 0; dt < AD / 32; ++dt)
#pragma unroll
    for (int rg = 0; rg < 4; ++rg) {
      u32x2 w;
      w[0] = pack2<T>(o[dt][4 * rg] * inv, o[dt][4 * rg + 1] * inv);
      w[1] = pack2<T>(o[dt][4 * rg + 2] * inv, o[dt][4 * rg + 3] * inv);
      *reinterpret_cast<u32x2*>(O + dt * 32 + 8 * rg + 4 * h) = w;
    }
}

inline bool al16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; }

}  // namespace
}  // namespace sph

using namespace sph;

namespace {
int64_t mask_batches(int64_t batch, int64_t stride_m) { return (batch == 1 || stride_m == 0) ? 1 : batch; }
}  // namespace

extern "C" int64_t sph_attention_workspace_bytes(int64_t batch, int64_t mq, int64_t sk,
                                                 int64_t stride_m) {
  if (batch <= 0 || mq <= 0 || sk <= 0) return 0;
  if (mq <= 16 && mq % AQ != 0) return sph_attention_decode_workspace_bytes(batch, mq, sk);
  // mask block classes, then (256-byte aligned) the job order
  const int64_t cls = mask_batches(batch, stride_m) * ((mq + AQ - 1) / AQ) * ((sk + AK - 1) / AK);
  return (cls + 255) / 256 * 256 + 4 * batch * ((mq + AQ - 1) / AQ);
}

extern "C" int sph_attention_fwd(sph_dtype dtype, int64_t batch, int64_t mq, int64_t sk,
                                 int64_t head_dim, const void* q, int64_t ldq, int64_t stride_q,
                                 const void* k, int64_t ldk, int64_t stride_k, const void* v,
                                 int64_t ldv, int64_t stride_v, const void* mask, int64_t ldm,
                                 int64_t stride_m, int64_t causal_q, int64_t causal_off,
                                 float scale, void* o, int64_t ldo, int64_t stride_o,
                                 void* workspace, int64_t workspace_bytes, sph_stream_t stream) {
  SPH_REQUIRE(dtype == SPH_F16 || dtype == SPH_BF16, SPH_ERR_UNSUPPORTED,
              "attention: dtype must be F16 or BF16");
  SPH_REQUIRE(head_dim == AD, SPH_ERR_UNSUPPORTED, "attention: head_dim must be 128");
  SPH_REQUIRE(batch >= 0 && mq >= 0 && sk >= 0, SPH_ERR_INVALID_ARG, "attention: negative size");
  if (batch == 0 || mq == 0) return SPH_OK;
  SPH_REQUIRE(sk > 0, SPH_ERR_INVALID_ARG, "attention: no keys");
  if (mq <= 16 && mq % AQ != 0)  // a decode step's rows
    return sph_attention_decode(dtype, batch, mq, sk, head_dim, q, ldq, stride_q, k, ldk, stride_k,
                                v, ldv, 1, stride_v, mask, ldm, stride_m, causal_q, causal_off,
                                scale, o, ldo, stride_o, workspace, workspace_bytes, stream);
  SPH_REQUIRE(mq % AQ == 0, SPH_ERR_UNSUPPORTED,
              "attention: query rows must be a multiple of 128 (or at most 16)");
  SPH_REQUIRE(batch * (mq / AQ) < (1LL << 31), SPH_ERR_TOO_LARGE, "attention: grid too large");
  SPH_REQUIRE(causal_q >= 0, SPH_ERR_INVALID_ARG, "attention: causal_q < 0");
  SPH_REQUIRE(scale > 0.f && scale < INFINITY, SPH_ERR_INVALID_ARG,
              "attention: scale must be positive and finite");
  SPH_REQUIRE(sk < (1LL << 30) && causal_q < (1LL << 30) && causal_off > -(1LL << 30) &&
                  causal_off < (1LL << 30),
              SPH_ERR_TOO_LARGE, "attention: positions must fit 30 bits");
  SPH_REQUIRE(ldq >= AD && ldk >= AD && ldv >= AD && ldo >= AD, SPH_ERR_INVALID_ARG,
              "attention: leading dimension below head_dim");
  SPH_REQUIRE(al16(q) && al16(k) && al16(v) && al16(o) && ldq % 8 == 0 && ldk % 8 == 0 &&
                  ldv % 8 == 0 && ldo % 8 == 0 && (batch == 1 || (stride_q % 8 == 0 &&
                  stride_k % 8 == 0 && stride_v % 8 == 0 && stride_o % 8 == 0)),
              SPH_ERR_INVALID_ARG, "attention: rows must be 16-byte aligned");
  SPH_REQUIRE(mask == nullptr || ((ldm == 0 || ldm >= sk) && ldm % 4 == 0 && (reinterpret_cast<uintptr_t>(mask) & 7u) == 0 &&
                                  (batch == 1 || stride_m % 4 == 0)),
              SPH_ERR_INVALID_ARG, "attention: mask rows must be 8-byte aligned, ldm 0 or >= sk");
  // DMA offsets within one key block are 32-bit.
  SPH_REQUIRE(AK * ldk * 2 < (1LL << 31) && AK * ldv * 2 < (1LL << 31), SPH_ERR_TOO_LARGE,
              "attention: K/V rows too long for 32-bit block offsets");
  SPH_REQUIRE(workspace_bytes >= 0, SPH_ERR_INVALID_ARG, "attention: negative workspace size");
  AttnArgs p{};
  p.mq = mq;
  p.sk = sk;
  p.q = q;
  p.ldq = ldq;
  p.sq = stride_q;
  p.k = k;
  p.ldk = ldk;
  p.skb = stride_k;
  p.v = v;
  p.ldv = ldv;
  p.svb = stride_v;
  p.mask = mask;
  p.ldm = ldm;
  p.smb = stride_m;
  p.causal_q = causal_q;
  p.causal_off = causal_off;
  p.batch = batch;
  p.nbq = mq / AQ;
  p.heads = (causal_q > 0 && causal_q % AQ == 0 && mq % causal_q == 0) ? mq / causal_q : 0;
  p.nkb = (sk + AK - 1) / AK;
  p.scale_log2 = scale * 1.4426950408889634f;
  p.inv_scale = 1.0f / scale;
  p.o = o;
  p.ldo = ldo;
  p.so = stride_o;
  hipStream_t st = as_stream(stream);
  // Mask block classes, when the caller gave room for them and the mask rows
  // allow 16-byte reads.
  const int64_t mbat = mask_batches(batch, stride_m);
  if (mask != nullptr && workspace != nullptr &&
      workspace_bytes >= sph_attention_workspace_bytes(batch, mq, sk, stride_m) &&
      al16(mask) && ldm % 8 == 0 && (mbat == 1 || stride_m % 8 == 0)) {
    SPH_REQUIRE(p.nkb < (1LL << 31) && mbat <= 65535 && p.nbq <= 65535, SPH_ERR_TOO_LARGE,
                "attention: mask too large for the block pre-pass");
    uint8_t* cls = static_cast<uint8_t*>(workspace);
    dim3 g(static_cast<unsigned>(p.nkb), static_cast<unsigned>(p.nbq), static_cast<unsigned>(mbat));
    if (dtype == SPH_F16)
      mask_blocks_kernel<half_t><<<g, 256, 0, st>>>(static_cast<const uint16_t*>(mask), ldm,
                                                    mbat == 1 ? 0 : stride_m, sk, p.nbq, p.nkb, cls);
    else
      mask_blocks_kernel<bf16_t><<<g, 256, 0, st>>>(static_cast<const uint16_t*>(mask), ldm,
                                                    mbat == 1 ? 0 : stride_m, sk, p.nbq, p.nkb, cls);
    p.mblk = cls;
    p.mblk_b = mbat == 1 ? 0 : p.nbq;
    // Longest-first job order from the classes (masks without causal
    // positions, small enough for one sorting workgroup).
    const int64_t jobs = batch * p.nbq;
    const int64_t cls_bytes = mbat * p.nbq * p.nkb;
    if (causal_q == 0 && p.nkb < kMaxOrderBins && cls_bytes <= kMaxOrderBytes) {
      int32_t* ord = reinterpret_cast<int32_t*>(cls + (cls_bytes + 255) / 256 * 256);
      attn_order_kernel<<<1, 1024, 0, st>>>(cls, p.mblk_b, static_cast<int>(p.nkb),
                                            static_cast<int>(p.nbq), static_cast<int>(jobs), ord);
      p.order = ord;
    }
  }
  dim3 grid(static_cast<unsigned>(batch * (mq / AQ)));
  const bool m = mask != nullptr, c = causal_q > 0;
  // Without a mask or causal positions every job has the same length and
  // needs no key split: one group of 4 waves per workgroup, two workgroups
  // per CU (c4's dense shape 79-81 us against 86.5-87 with two groups).
  constexpr int kDenseGroups = 1;
#define SPH_ATTN(T_)                                                                     \
  do {                                                                                   \
    if (m && c) attn_fwd_kernel<T_, true, true, 2><<<grid, 512, 0, st>>>(p);             \
    else if (m) attn_fwd_kernel<T_, true, false, 2><<<grid, 512, 0, st>>>(p);            \
    else if (c) attn_fwd_kernel<T_, false, true, 2><<<grid, 512, 0, st>>>(p);            \
    else attn_fwd_kernel<T_, false, false, kDenseGroups><<<grid, kDenseGroups * 256, 0, st>>>(p); \
  } while (0)
  if (dtype == SPH_F16)
    SPH_ATTN(half_t);
  else
    SPH_ATTN(bf16_t);
#undef SPH_ATTN
  return check_launch("sph_attention_fwd");
}

// ---------------------------------------------------------------------------
// sph_attention_fwd without a caller workspace, for callers that cannot
// allocate device memory (code under HIP graph capture, serving loops,
// harnesses that forbid hipMalloc).  The workspace of sph_attention_fwd (the
// mask-block classes and job order of a masked prefill call, the key-split
// partials of a decode call) lives in one file-scope device array of
// kScratchBytes per GPU, held until the process ends.  In host code the
// array's name is only a stand-in: its device address is looked up once per
// device with hipGetSymbolAddress (that device current) and that address is
// what the kernels get.  Nothing in the workspace needs to start at zero
// (every byte a call reads it has written before, on the same stream).
// Every call on a GPU shares that GPU's array and leaves its contents
// behind: calls that overlap on one GPU (different streams, or host threads
// without an order between their streams) race.
// ---------------------------------------------------------------------------
namespace {
constexpr int64_t kScratchBytes = int64_t(4) << 20;
constexpr int kScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kScratchDevices] = {};
}  // namespace

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {
// The device address of `scratch` on `dev` (looked up on first use).
int scratch_address(int dev, void** out) {
  SPH_REQUIRE(dev >= 0 && dev < kScratchDevices, SPH_ERR_INVALID_ARG,
              "attention (no-alloc): device index out of range");
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    int cur = -1;
    hipError_t e = hipGetDevice(&cur);
    if (e == hipSuccess && cur != dev) e = hipSetDevice(dev);
    void* p = nullptr;
    if (e == hipSuccess) e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (cur >= 0 && cur != dev) {
      const hipError_t e2 = hipSetDevice(cur);
      if (e == hipSuccess) e = e2;
    }
    if (e != hipSuccess || p == nullptr)
      return set_error(e != hipSuccess ? static_cast<int>(e) : SPH_ERR_INVALID_ARG,
                       std::string("attention (no-alloc): hipGetSymbolAddress(scratch) failed: ") +
                           hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return SPH_OK;
}
}  // namespace

extern "C" int64_t sph_attention_fwd_noalloc_max_bytes(void) { return kScratchBytes; }

extern "C" int sph_attention_fwd_noalloc(sph_dtype dtype, int64_t batch, int64_t mq, int64_t sk,
                                         int64_t head_dim, const void* q, int64_t ldq,
                                         int64_t stride_q, const void* k, int64_t ldk,
                                         int64_t stride_k, const void* v, int64_t ldv,
                                         int64_t stride_v, const void* mask, int64_t ldm,
                                         int64_t stride_m, int64_t causal_q, int64_t causal_off,
                                         float scale, void* o, int64_t ldo, int64_t stride_o,
                                         sph_stream_t stream) {
  SPH_REQUIRE(batch >= 0 && mq >= 0 && sk >= 0, SPH_ERR_INVALID_ARG,
              "attention (no-alloc): negative size");
  if (batch == 0 || mq == 0) return SPH_OK;
  // the workspace this call would use: decode partials, or the classes and
  // order of a masked prefill call (an unmasked prefill call uses none)
  const bool decode = mq <= 16 && mq % AQ != 0;
  const int64_t need = (decode || mask != nullptr)
                           ? sph_attention_workspace_bytes(batch, mq, sk, stride_m) : 0;
  SPH_REQUIRE(need <= kScratchBytes, SPH_ERR_TOO_LARGE,
              "attention (no-alloc): this shape needs " + std::to_string(need) +
                  " bytes of workspace, above the " + std::to_string(kScratchBytes) +
                  "-byte static scratch; call sph_attention_fwd with a workspace");
  void* ws = nullptr;
  if (need > 0) {
    hipDevice_t dev = 0;
    const hipError_t e = hipStreamGetDevice(as_stream(stream), &dev);
    if (e != hipSuccess)
      return set_error(static_cast<int>(e),
                       std::string("attention (no-alloc): hipStreamGetDevice failed: ") +
                           hipGetErrorString(e));
    const int rc = scratch_address(static_cast<int>(dev), &ws);
    if (rc != SPH_OK) return rc;
  }
  return sph_attention_fwd(dtype, batch, mq, sk, head_dim, q, ldq, stride_q, k, ldk, stride_k, v,
                           ldv, stride_v, mask, ldm, stride_m, causal_q, causal_off, scale, o, ldo,
                           stride_o, ws, need > 0 ? kScratchBytes : 0, stream);
}
