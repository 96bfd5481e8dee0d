// Attention for a few query rows per KV head (decode steps): O = softmax(
// scale * Q K^T + mask) V for fp16 / bf16, head dim 128, mq <= 16 rows per
// batch entry (one KV head and its group of query heads, one query position
// each), over the whole KV cache.
//
// Why a second kernel: the prefill kernel (attention.hip) takes 128 query
// rows per workgroup; a decode step has 4-16 rows per KV head and 32-64 KV
// heads in all, so its work is the K/V bytes, not MFMA time.  Here:
//   * the keys are split into chunks of 64 and each workgroup takes a range
//     of chunks of one batch entry (flash-decoding; one chunk each when the
//     grid allows), so 32 KV heads x 1152 keys give 576 workgroups;
//   * a workgroup stages its chunk's K rows and V (either layout: key-major
//     [sk, 128], or dim-major [128, sk] as a decode cache that feeds the P V
//     product keeps it) in LDS with 16-byte loads, computes the scores on
//     the vector ALUs (one key per lane, four query rows per wave), keeps an
//     online softmax state (max, sum) per row in log2 units, and
//     accumulates P V with one head-dim column per thread;
//   * a split workgroup writes its (max, sum, unnormalised O) in fp32 to the
//     workspace and a combine kernel merges the splits per row; without a
//     workspace one workgroup per batch entry walks every chunk and writes O.
// Rows whose keys are all masked yield NaN, as softmax over all -inf does.
#include "sph_common.h"

#include <type_traits>

namespace sph {
namespace {

constexpr int DD = 128;          // head dim
constexpr int DKC = 64;          // keys per chunk
constexpr int DMQ = 16;          // max query rows per batch entry
constexpr int KPITCH = DD + 8;   // K rows in LDS: 272 bytes
constexpr int VPITCH_T = DKC + 8;  // dim-major V rows in LDS: 144 bytes
constexpr float kLog2eD = 1.4426950408889634f;

struct DecArgs {
  const void* q;
  int64_t ldq, sq;
  const void* k;
  int64_t ldk, skb;
  const void* v;
  int64_t vks, vds, svb;  // V element (key, dim) strides, batch stride
  const void* mask;
  int64_t ldm, smb;
  int64_t causal_q, causal_off;
  int mq, sk, nchunks, cps, nsplit;
  float scale_log2;
  void* o;
  int64_t ldo, so;
  float* part;  // [batch][nsplit][mq][2 + 128] fp32, or null
};

constexpr int kPartRow = 2 + DD;

// One workgroup: batch entry blockIdx.y, chunks [split * cps, ...) of it.
template <typename T, bool VT>
__global__ void __launch_bounds__(256) attn_decode_kernel(const DecArgs p) {
  __shared__ __attribute__((aligned(16))) float qs[DMQ][DD];
  __shared__ __attribute__((aligned(16))) T ks[DKC][KPITCH];
  __shared__ __attribute__((aligned(16))) T vs[VT ? DD : DKC][VT ? VPITCH_T : KPITCH];
  __shared__ __attribute__((aligned(16))) float ps[DMQ][DKC];
  __shared__ float alpha[DMQ], lsum[DMQ], mrow[DMQ];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int64_t b = blockIdx.y;
  const int split = blockIdx.x;
  const int mq = p.mq, sk = p.sk;
  const T* Q = static_cast<const T*>(p.q) + b * p.sq;
  const T* K = static_cast<const T*>(p.k) + b * p.skb;
  const T* V = static_cast<const T*>(p.v) + b * p.svb;
  const T* M = p.mask ? static_cast<const T*>(p.mask) + b * p.smb : nullptr;

  // Q rows, pre-multiplied by scale * log2(e)
  for (int x = t; x < mq * (DD / 8); x += 256) {
    const int i = x / (DD / 8), c = (x % (DD / 8)) * 8;
    float f[8];
    load8<T>(Q + i * p.ldq + c, f);
#pragma unroll
    for (int e = 0; e < 8; ++e) qs[i][c + e] = f[e] * p.scale_log2;
  }
  // per-row softmax state, replicated across the lanes of the row's wave
  float m_run[4], l_run[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    m_run[r] = -INFINITY;
    l_run[r] = 0.f;
  }
  // P V accumulators: head-dim column d, rows rg + 2 * r
  const int d = t & (DD - 1), rg = t >> 7;
  float acc[DMQ / 2];
#pragma unroll
  for (int r = 0; r < DMQ / 2; ++r) acc[r] = 0.f;

  const int c0 = split * p.cps, c1 = min(p.nchunks, c0 + p.cps);
  for (int c = c0; c < c1; ++c) {
    const int kbase = c * DKC;
    const int kn = min(DKC, sk - kbase);  // keys in this chunk
    __syncthreads();  // previous chunk's LDS reads are done (and qs written)
    // K chunk: 64 rows x 16 chunks of 8 values
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int x = t + 256 * i, key = x >> 4, cc = (x & 15) * 8;
      u32x4 w = {0u, 0u, 0u, 0u};
      if (key < kn) w = *reinterpret_cast<const u32x4*>(K + (kbase + key) * p.ldk + cc);
      *reinterpret_cast<u32x4*>(&ks[key][cc]) = w;
    }
    if constexpr (VT) {
      // V dim-major: 128 rows (dims) x 8 chunks of 8 keys
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int x = t + 256 * i, dm = x >> 3, kc = (x & 7) * 8;
        const T* src = V + dm * p.vds + kbase + kc;
        u32x4 w = {0u, 0u, 0u, 0u};
        if (kc + 8 <= kn) {
          w = *reinterpret_cast<const u32x4*>(src);
        } else {
          T* e = reinterpret_cast<T*>(&w);
          for (int j = 0; j < 8 && kc + j < kn; ++j) e[j] = src[j];
        }
        *reinterpret_cast<u32x4*>(&vs[dm][kc]) = w;
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int x = t + 256 * i, key = x >> 4, cc = (x & 15) * 8;
        u32x4 w = {0u, 0u, 0u, 0u};
        if (key < kn) w = *reinterpret_cast<const u32x4*>(V + (kbase + key) * p.vks + cc);
        *reinterpret_cast<u32x4*>(&vs[key][cc]) = w;
      }
    }
    __syncthreads();

    // scores: key `lane`, rows wave + 4 r
    float s[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) s[r] = 0.f;
#pragma unroll
    for (int cc = 0; cc < DD; cc += 8) {
      float kf[8];
      const u32x4 kw = *reinterpret_cast<const u32x4*>(&ks[lane][cc]);
      const T* ke = reinterpret_cast<const T*>(&kw);
#pragma unroll
      for (int e = 0; e < 8; ++e) kf[e] = Num<T>::to_f(ke[e]);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = wave + 4 * r;
        if (i < mq) {
#pragma unroll
          for (int e = 0; e < 8; ++e) s[r] = fmaf(qs[i][cc + e], kf[e], s[r]);
        }
      }
    }
    const int key = kbase + lane;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = wave + 4 * r;
      if (i >= mq) continue;  // uniform per wave
      float x = s[r];
      bool vis = lane < kn;
      if (vis && M) x = fmaf(Num<T>::to_f(M[i * p.ldm + key]), kLog2eD, x);
      if (p.causal_q > 0) vis = vis && key <= (i % p.causal_q) + p.causal_off;
      x = vis ? x : -INFINITY;
      float mx = x;
#pragma unroll
      for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
      const float m_new = fmaxf(m_run[r], mx);
      // a row with nothing visible so far keeps a zero state (no -inf - -inf)
      const float a = m_new == -INFINITY ? 1.f : __builtin_amdgcn_exp2f(m_run[r] - m_new);
      const float pj = m_new == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(x - m_new);
      float sum = pj;
#pragma unroll
      for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off, 64);
      l_run[r] = l_run[r] * a + sum;
      m_run[r] = m_new;
      ps[i][lane] = pj;
      if (lane == 0) alpha[i] = a;
    }
    __syncthreads();

    // O[i][d] = O[i][d] * alpha[i] + sum_j P[i][j] V[j][d]
#pragma unroll
    for (int r = 0; r < DMQ / 2; ++r) {
      const int i = rg + 2 * r;
      if (i < mq) acc[r] *= alpha[i];
    }
#pragma unroll
    for (int j = 0; j < DKC; j += 8) {
      float vf[8];
      if constexpr (VT) {
        const u32x4 vw = *reinterpret_cast<const u32x4*>(&vs[d][j]);
        const T* ve = reinterpret_cast<const T*>(&vw);
#pragma unroll
        for (int e = 0; e < 8; ++e) vf[e] = Num<T>::to_f(ve[e]);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) vf[e] = Num<T>::to_f(vs[j + e][d]);
      }
#pragma unroll
      for (int r = 0; r < DMQ / 2; ++r) {
        const int i = rg + 2 * r;
        if (i < mq) {
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[r] = fmaf(ps[i][j + e], vf[e], acc[r]);
        }
      }
    }
  }

  // row states to LDS (lane 0 of the row's wave)
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int i = wave + 4 * r;
    if (i < mq && lane == 0) {
      lsum[i] = l_run[r];
      mrow[i] = m_run[r];
    }
  }
  __syncthreads();
  if (p.part == nullptr) {
    T* O = static_cast<T*>(p.o) + b * p.so;
#pragma unroll
    for (int r = 0; r < DMQ / 2; ++r) {
      const int i = rg + 2 * r;
      if (i < mq) O[i * p.ldo + d] = Num<T>::from_f(acc[r] / lsum[i]);
    }
  } else {
    float* P = p.part + (b * p.nsplit + split) * static_cast<int64_t>(mq) * kPartRow;
#pragma unroll
    for (int r = 0; r < DMQ / 2; ++r) {
      const int i = rg + 2 * r;
      if (i < mq) {
        P[i * kPartRow + 2 + d] = acc[r];
        if (d == 0) {
          P[i * kPartRow] = mrow[i];
          P[i * kPartRow + 1] = lsum[i];
        }
      }
    }
  }
}

// Merges the splits of batch entry blockIdx.y, row blockIdx.x: O = sum_s
// 2^(m_s - M) o_s / sum_s 2^(m_s - M) l_s with M the largest m_s.  One
// thread per head-dim column; every split's values are loaded before use
// (at most kMaxSplit splits).
constexpr int kMaxSplit = 32;
template <typename T>
__global__ void __launch_bounds__(DD) attn_decode_combine(const DecArgs p) {
  const int d = threadIdx.x, i = blockIdx.x;
  const int64_t b = blockIdx.y;
  const float* P = p.part + b * p.nsplit * static_cast<int64_t>(p.mq) * kPartRow + i * kPartRow;
  const int64_t step = static_cast<int64_t>(p.mq) * kPartRow;
  float m[kMaxSplit], l[kMaxSplit], o[kMaxSplit];
#pragma unroll
  for (int s = 0; s < kMaxSplit; ++s) {
    const bool in = s < p.nsplit;
    m[s] = in ? P[s * step] : -INFINITY;
    l[s] = in ? P[s * step + 1] : 0.f;
    o[s] = in ? P[s * step + 2 + d] : 0.f;
  }
  float mx = -INFINITY;
#pragma unroll
  for (int s = 0; s < kMaxSplit; ++s) mx = fmaxf(mx, m[s]);
  float lsum = 0.f, acc = 0.f;
#pragma unroll
  for (int s = 0; s < kMaxSplit; ++s) {
    const float w = (mx == -INFINITY || m[s] == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(m[s] - mx);
    lsum = fmaf(l[s], w, lsum);
    acc = fmaf(o[s], w, acc);
  }
  T* O = static_cast<T*>(p.o) + b * p.so;
  O[i * p.ldo + d] = Num<T>::from_f(acc / lsum);
}

// Chunks per split and split count for a launch of `batch` entries: enough
// workgroups for ~2 per CU, each at least one chunk.
void decode_plan(int64_t batch, int64_t sk, int& nchunks, int& cps, int& nsplit) {
  // A chunk's steps are a chain of dependent LDS and exp latencies, so
  // workgroups take one chunk each where the grid allows (several
  // workgroups per CU hide each other's latencies), up to kMaxSplit splits.
  nchunks = static_cast<int>((sk + DKC - 1) / DKC);
  const int64_t want = std::max<int64_t>(1, (2048 + batch - 1) / batch);
  const int64_t ns = std::min<int64_t>({static_cast<int64_t>(nchunks), want, kMaxSplit});
  cps = static_cast<int>((nchunks + ns - 1) / ns);
  nsplit = (nchunks + cps - 1) / cps;
}

bool al16d(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace
}  // namespace sph

using namespace sph;

extern "C" int64_t sph_attention_decode_workspace_bytes(int64_t batch, int64_t mq, int64_t sk) {
  if (batch <= 0 || mq <= 0 || sk <= 0 || mq > DMQ) return 0;
  int nchunks, cps, nsplit;
  decode_plan(batch, sk, nchunks, cps, nsplit);
  if (nsplit <= 1) return 0;
  return batch * nsplit * mq * kPartRow * 4;
}

extern "C" int sph_attention_decode(sph_dtype dtype, int64_t batch, int64_t mq, int64_t sk,
                                    int64_t head_dim, const void* q, int64_t ldq, int64_t stride_q,
                                    const void* k, int64_t ldk, int64_t stride_k, const void* v,
                                    int64_t v_key_stride, int64_t v_dim_stride, int64_t stride_v,
                                    const void* mask, int64_t ldm, int64_t stride_m,
                                    int64_t causal_q, int64_t causal_off, float scale, void* o,
                                    int64_t ldo, int64_t stride_o, void* workspace,
                                    int64_t workspace_bytes, sph_stream_t stream) {
  SPH_REQUIRE(dtype == SPH_F16 || dtype == SPH_BF16, SPH_ERR_UNSUPPORTED,
              "decode attention: dtype must be F16 or BF16");
  SPH_REQUIRE(head_dim == DD, SPH_ERR_UNSUPPORTED, "decode attention: head_dim must be 128");
  SPH_REQUIRE(batch >= 0 && mq >= 0 && sk >= 0, SPH_ERR_INVALID_ARG,
              "decode attention: negative size");
  if (batch == 0 || mq == 0) return SPH_OK;
  SPH_REQUIRE(sk > 0, SPH_ERR_INVALID_ARG, "decode attention: no keys");
  SPH_REQUIRE(mq <= DMQ, SPH_ERR_UNSUPPORTED, "decode attention: at most 16 query rows");
  SPH_REQUIRE(batch < 65536 && sk < (1LL << 30), SPH_ERR_TOO_LARGE, "decode attention: too large");
  SPH_REQUIRE(causal_q >= 0 && causal_q < (1LL << 30) && causal_off > -(1LL << 30) &&
                  causal_off < (1LL << 30),
              SPH_ERR_INVALID_ARG, "decode attention: causal positions must fit 30 bits");
  SPH_REQUIRE(scale > 0.f && scale < INFINITY, SPH_ERR_INVALID_ARG,
              "decode attention: scale must be positive and finite");
  SPH_REQUIRE((v_dim_stride == 1 && v_key_stride >= DD) || (v_key_stride == 1 && v_dim_stride >= sk),
              SPH_ERR_INVALID_ARG,
              "decode attention: V must be key-major (dim stride 1) or dim-major (key stride 1)");
  const bool vt = v_key_stride == 1 && v_dim_stride != 1;
  const int64_t vrow = vt ? v_dim_stride : v_key_stride;
  SPH_REQUIRE(ldq >= DD && ldk >= DD && ldo >= DD, SPH_ERR_INVALID_ARG,
              "decode attention: leading dimension below head_dim");
  SPH_REQUIRE(al16d(q) && al16d(k) && al16d(v) && ldq % 8 == 0 && ldk % 8 == 0 && vrow % 8 == 0 &&
                  (batch == 1 || (stride_q % 8 == 0 && stride_k % 8 == 0 && stride_v % 8 == 0)),
              SPH_ERR_INVALID_ARG, "decode attention: q, k, v rows must be 16-byte aligned");
  SPH_REQUIRE(mask == nullptr || ldm == 0 || ldm >= sk, SPH_ERR_INVALID_ARG,
              "decode attention: mask row stride must be 0 (one row for all) or >= sk");
  SPH_REQUIRE(workspace_bytes >= 0, SPH_ERR_INVALID_ARG, "decode attention: negative workspace size");
  DecArgs p{};
  p.q = q;
  p.ldq = ldq;
  p.sq = stride_q;
  p.k = k;
  p.ldk = ldk;
  p.skb = stride_k;
  p.v = v;
  p.vks = v_key_stride;
  p.vds = v_dim_stride;
  p.svb = stride_v;
  p.mask = mask;
  p.ldm = ldm;
  p.smb = stride_m;
  p.causal_q = causal_q;
  p.causal_off = causal_off;
  p.mq = static_cast<int>(mq);
  p.sk = static_cast<int>(sk);
  p.scale_log2 = scale * kLog2eD;
  p.o = o;
  p.ldo = ldo;
  p.so = stride_o;
  decode_plan(batch, sk, p.nchunks, p.cps, p.nsplit);
  const int64_t need = sph_attention_decode_workspace_bytes(batch, mq, sk);
  if (need == 0 || workspace == nullptr || workspace_bytes < need) {
    // one workgroup per batch entry over every chunk, O written directly
    p.cps = p.nchunks;
    p.nsplit = 1;
    p.part = nullptr;
  } else {
    p.part = static_cast<float*>(workspace);
  }
  hipStream_t st = as_stream(stream);
  dim3 grid(static_cast<unsigned>(p.nsplit), static_cast<unsigned>(batch));
  if (dtype == SPH_F16) {
    if (vt) attn_decode_kernel<half_t, true><<<grid, 256, 0, st>>>(p);
    else attn_decode_kernel<half_t, false><<<grid, 256, 0, st>>>(p);
    if (p.part) attn_decode_combine<half_t><<<dim3(static_cast<unsigned>(mq), static_cast<unsigned>(batch)), DD, 0, st>>>(p);
  } else {
    if (vt) attn_decode_kernel<bf16_t, true><<<grid, 256, 0, st>>>(p);
    else attn_decode_kernel<bf16_t, false><<<grid, 256, 0, st>>>(p);
    if (p.part) attn_decode_combine<bf16_t><<<dim3(static_cast<unsigned>(mq), static_cast<unsigned>(batch)), DD, 0, st>>>(p);
  }
  return check_launch("sph_attention_decode");
}

// ---------------------------------------------------------------------------
// One decode step of attention with its KV-cache append, for a model's
// whole batch in one launch: for every (batch entry b, KV head h) "unit",
// the unit's G query heads and its new key / value are read from the
// projection row qkv[b] (query heads first, then the KV heads' keys, then
// their values, 128 each), the queries and the new key are rotated by RoPE
// at position P = *pos (rotate-half: x cos + rot(x) sin, rot(x) = (-x2, x1),
// tables cos / sin [max_len, 128]), the key and value are written into the
// caches at P, and O = softmax(scale q K[0..P]^T) V[0..P] is written to
// out[b] (query head j at columns j * 128).
//
// Layout: K cache [.., max_len, 128] key-major (dim stride 1); V cache
// key-major or dim-major ([.., 128, max_len], key stride 1, the layout the
// decoders' caches keep).  Each workgroup (256 threads) takes one unit and
// one 64-key chunk (grid = chunks of max_len x units; P is only known on
// the device, so chunks past P do nothing but report), stages the chunk's
// K and V in LDS while the queries are rotated, computes the G x 64 scores
// (one key per lane, one query head per wave, v_dot2_f32_f16 on the
// rounded query), their softmax state (max, sum) and the unnormalised
// G x 128 output, and writes that partial to the workspace (a chunk past P
// writes a neutral one); a second kernel merges each unit's partials and
// writes O.  Measured alternatives (c5: 4 x 8 KV heads, 1152 slots,
// 18.9 MB of K / V): larger chunks on more threads (128 to 256 keys on 256
// to 1024 threads) run 8.0-11.3 us against 7.4, since fewer workgroups per
// CU overlap one's loads with another's arithmetic; one workgroup per
// unit with no merge reads the bytes alone in 11.5 us (one CU pulls ~50
// GB/s); merging in the last workgroup of a unit to arrive, behind an
// atomic count, needs a device-scope release per workgroup, which on this
// 8-XCD part writes back the XCD's L2 (576 of them took 87 us); with the
// partials stored and loaded with sc1 (written through to the coherence
// point, so no release) it ran 19.7 us per call against 14.6 for the pair
// and the c5 decode step 4.46 ms against 4.28: the wait for the stores to
// complete, the atomic and the coherent loads on the last workgroup's path
// cost more than the second launch.  The chunk
// holding P takes the new key and value from the rotated registers, not
// from the cache it writes in the same launch.
//
// Rounding: rotated q and k round once to the element type (k as it is
// stored); scores, softmax and the output sums are fp32; O rounds once.
// ---------------------------------------------------------------------------
namespace sph {
namespace {

constexpr int SG = 8;              // max query heads per KV head
constexpr int SKB = 64;            // keys per score block (one key per lane)
constexpr int kMaxUnits = 4096;    // batch x KV heads per launch
constexpr int kStepPart = 2 + DD;  // m, l, o[128] per query head
constexpr int32_t kStepBadPos = 2;  // error code: position outside [0, max_len)
constexpr int kMinChunk = 64;      // the smallest chunk any launch shape uses

struct StepArgs {
  const void* qkv;
  int64_t ld_qkv;
  const void* cos;
  const void* sin;
  int64_t ld_rope;
  const int64_t* pos;
  int32_t* err;  // device error word: set to kStepBadPos for P outside the cache
  void* kc;
  int64_t k_sb, k_sh, k_ss;
  void* vc;
  int64_t v_sb, v_sh, v_ks, v_ds;
  int v_al;  // dim-major V rows 16-byte aligned (else read element by element)
  int64_t max_len;
  int n_heads, n_kv, g, nchunks;
  float scale_log2;
  void* out;
  int64_t ld_out;
  float* part;  // [units][nchunks][g][kStepPart]
};

__device__ inline u32x4 zero_chunk() {
  u32x4 z = {0u, 0u, 0u, 0u};
  return z;
}

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

// acc + the dot product of 8 two-byte values a and b (16 bytes each):
// fp16 as four v_dot2_f32_f16 (exact products, fp32 sums), bf16 widened by
// shifts into fp32 FMAs.
template <typename T>
__device__ inline float dot8(u32x4 a, u32x4 b, float acc) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t ai = a[i], bi = b[i];
    if constexpr (__is_same(T, half_t)) {
      acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, ai), __builtin_bit_cast(f16x2, bi),
                                   acc, false);
    } else {
      acc = fmaf(__uint_as_float(ai << 16), __uint_as_float(bi << 16), acc);
      acc = fmaf(__uint_as_float(ai & 0xffff0000u), __uint_as_float(bi & 0xffff0000u), acc);
    }
  }
  return acc;
}

// One workgroup of NT threads: one unit (blockIdx.y) and one chunk of SKC
// keys (blockIdx.x).  The chunk's K and V (SKC * 16 / NT 16-byte loads of
// each per thread, all in flight at once) are loaded before P is known.
// Scores: work item (query head i, 64-key block kb) on a wave, one key per
// lane; each block keeps its own max and sum, so no barrier joins the
// blocks before P V.  P V: item (query head i, key split r) on a slot of
// 128 threads, one head-dim column per thread; the R splits of a head meet
// in LDS, each block's sum scaled by 2^(m_block - m_chunk).
template <typename T, bool VT, int SKC, int NT>
__global__ void __launch_bounds__(NT) attn_decode_step_kernel(const StepArgs p) {
  constexpr int NB = SKC / SKB;       // score blocks per chunk
  constexpr int NW = NT / 64;         // waves
  constexpr int SLOTS = NT / DD;      // P V thread slots
  constexpr int LOADS = SKC * DD / 8 / NT;  // 16-byte K (and V) loads per thread
  constexpr int SVPITCH = SKC + 8;    // dim-major V rows in LDS
  constexpr int VCH = SKC / 8;        // 16-byte chunks per dim-major V row
  static_assert(LOADS * NT * 8 == SKC * DD && NB * SKB == SKC && SLOTS >= 1, "launch shape");
  // ps holds the probabilities, then (after the P V sums) the split sums
  constexpr int PS = SKC > DD ? SG * SKC : SG * DD;
  constexpr int MAXW = (SG + SLOTS - 1) / SLOTS;  // P V items per slot, at most
  __shared__ __attribute__((aligned(16))) T ks[SKC][KPITCH];
  __shared__ __attribute__((aligned(16))) T vs[VT ? DD : SKC][VT ? SVPITCH : KPITCH];
  __shared__ __attribute__((aligned(16))) T qs[SG][DD];
  __shared__ __attribute__((aligned(16))) float ps[PS];
  __shared__ float mblk[SG][NB], lblk[SG][NB];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int unit = blockIdx.y, chunk = blockIdx.x;
  const int b = unit / p.n_kv, h = unit % p.n_kv, G = p.g;
  const int64_t kbase = static_cast<int64_t>(chunk) * SKC;
  T* Kc = static_cast<T*>(p.kc) + b * p.k_sb + h * p.k_sh;
  T* Vc = static_cast<T*>(p.vc) + b * p.v_sb + h * p.v_sh;
  const T* row = static_cast<const T*>(p.qkv) + b * p.ld_qkv;
  // The chunk's K / V (speculatively: the whole chunk, before P is known;
  // every address is inside the cache) and P itself are loaded together.
  const int64_t P = *p.pos;
  const int kmax = static_cast<int>(min<int64_t>(SKC, p.max_len - kbase));
  u32x4 kr[LOADS], vr[LOADS];
#pragma unroll
  for (int i = 0; i < LOADS; ++i) {
    const int x = t + NT * i, key = x >> 4, cc = (x & 15) * 8;
    kr[i] = key < kmax ? *reinterpret_cast<const u32x4*>(Kc + (kbase + key) * p.k_ss + cc)
                       : zero_chunk();
    if constexpr (VT) {
      const int dm = x / VCH, kc = (x % VCH) * 8;
      const T* src = Vc + dm * p.v_ds + kbase + kc;
      if (p.v_al && kc + 8 <= kmax) {
        vr[i] = *reinterpret_cast<const u32x4*>(src);
      } else {
        // the cache's last, partial chunk, or rows that are not 16-byte
        // aligned: element loads, zeros past the cache
        const uint16_t* s16 = reinterpret_cast<const uint16_t*>(src);
        uint32_t e[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) e[j] = kc + j < kmax ? s16[j] : 0u;
        vr[i] = u32x4{e[0] | (e[1] << 16), e[2] | (e[3] << 16), e[4] | (e[5] << 16),
                      e[6] | (e[7] << 16)};
      }
    } else {
      vr[i] = key < kmax ? *reinterpret_cast<const u32x4*>(Vc + (kbase + key) * p.v_ks + cc)
                         : zero_chunk();
    }
  }
  // The step's queries (element d and its rotate-half partner) and the new
  // key / value do not depend on P either.
  constexpr int QR = SG * DD / NT;  // query elements per thread
  static_assert(QR >= 1 && QR * NT == SG * DD, "whole query rows per thread");
  const int dq = t & (DD - 1), dpart = dq < DD / 2 ? dq + DD / 2 : dq - DD / 2;
  float qa[QR], qb[QR];
#pragma unroll
  for (int r = 0; r < QR; ++r) {
    const int i = (t + NT * r) / DD;
    const T* q = row + static_cast<int64_t>(h * G + (i < G ? i : 0)) * DD;
    qa[r] = Num<T>::to_f(q[dq]);
    qb[r] = Num<T>::to_f(q[dpart]);
  }
  const T* knew = row + static_cast<int64_t>(p.n_heads + h) * DD;
  const T* vnew = row + static_cast<int64_t>(p.n_heads + p.n_kv + h) * DD;
  const float ka = Num<T>::to_f(knew[dq]), kb_ = Num<T>::to_f(knew[dpart]);
  const T vv = vnew[dq];
  if (P < 0 || P >= p.max_len) {
    // nothing is written (every workgroup sees the same P); the caller's
    // error word reports it
    if (t == 0 && chunk == 0 && unit == 0 && p.err != nullptr) *p.err = kStepBadPos;
    return;
  }
  const bool active = kbase <= P;
  float* part = p.part + (static_cast<int64_t>(unit) * p.nchunks + chunk) * G * kStepPart;
  if (!active) {
    // a chunk past P: a neutral partial (m = -inf; the merge skips it)
    if (t < G) {
      part[t * kStepPart] = -INFINITY;
      part[t * kStepPart + 1] = 0.f;
    }
    return;
  }
  const int nkeys = static_cast<int>(min<int64_t>(SKC, P + 1 - kbase));
  const T* cs = static_cast<const T*>(p.cos) + P * p.ld_rope;
  const T* sn = static_cast<const T*>(p.sin) + P * p.ld_rope;
  const float cd = Num<T>::to_f(cs[dq]), sd = Num<T>::to_f(sn[dq]);
  const float sgn = dq < DD / 2 ? -1.f : 1.f;  // rot(x)[d] = -x[d + 64] | x[d - 64]
  // rotated queries, rounded as a stored tensor would be (the scores are
  // scaled into log2 units after the dot products)
#pragma unroll
  for (int r = 0; r < QR; ++r) {
    const int i = (t + NT * r) / DD;
    if (i < G) qs[i][dq] = Num<T>::from_f(qa[r] * cd + sgn * qb[r] * sd);
  }
  // Slots past P (the chunk holding P) may hold anything, NaN or Inf
  // included: their scores are replaced by -inf below, and their values
  // are staged as zeros so that a zero probability times a stale value
  // adds nothing to the output sums.
#pragma unroll
  for (int i = 0; i < LOADS; ++i) {
    const int x = t + NT * i, key = x >> 4, cc = (x & 15) * 8;
    *reinterpret_cast<u32x4*>(&ks[key][cc]) = kr[i];
    if constexpr (VT) {
      const int dm = x / VCH, kc = (x % VCH) * 8;
      u32x4 w = vr[i];
      if (kc + 8 > nkeys) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const uint32_t keep = (kc + 2 * q < nkeys ? 0x0000FFFFu : 0u) |
                                (kc + 2 * q + 1 < nkeys ? 0xFFFF0000u : 0u);
          w[q] &= keep;
        }
      }
      *reinterpret_cast<u32x4*>(&vs[dm][kc]) = w;
    } else {
      *reinterpret_cast<u32x4*>(&vs[key][cc]) = key < nkeys ? vr[i] : zero_chunk();
    }
  }
  const int own = static_cast<int>(P - kbase);  // the new key's slot, if here
  __syncthreads();  // chunk staged: the new key / value replace slot `own`
  if (own < SKC && t < DD) {
    const T kr_ = Num<T>::from_f(ka * cd + sgn * kb_ * sd);
    const T vr_ = vv;
    ks[own][t] = kr_;
    if constexpr (VT) vs[t][own] = vr_;
    else vs[own][t] = vr_;
    Kc[P * p.k_ss + t] = kr_;
    if constexpr (VT) Vc[t * p.v_ds + P] = vr_;
    else Vc[P * p.v_ks + t] = vr_;
  }
  __syncthreads();
  // scores: item (head i, block kb), key kb * 64 + lane; each block's
  // probabilities relative to its own max (a block with no visible key has
  // max -inf and contributes nothing)
  for (int it = wave; it < G * NB; it += NW) {
    const int i = it / NB, kb = it % NB, key = kb * SKB + lane;
    float s = 0.f;
#pragma unroll
    for (int cc = 0; cc < DD; cc += 8)
      s = dot8<T>(*reinterpret_cast<const u32x4*>(&qs[i][cc]),
                  *reinterpret_cast<const u32x4*>(&ks[key][cc]), s);
    s = key < nkeys ? s * p.scale_log2 : -INFINITY;
    float mx = s;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
    const float pj = mx == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(s - mx);
    float sum = pj;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off, 64);
    ps[i * SKC + key] = pj;
    if (lane == 0) {
      mblk[i][kb] = mx;
      lblk[i][kb] = sum;
    }
  }
  __syncthreads();
  // unnormalised P V: R key splits per head, the largest power of two
  // dividing NB with G * R <= SLOTS (at least 1: a slot then takes several
  // heads)
  int R = 1;
  while (2 * R <= NB && G * 2 * R <= SLOTS) R *= 2;
  const int slot = t >> 7, d = t & (DD - 1);
  const int bps = NB / R;  // blocks per split
  float acc_w[MAXW];
#pragma unroll
  for (int n = 0; n < MAXW; ++n) {
    const int w = slot + n * SLOTS;
    acc_w[n] = 0.f;
    if (w >= G * R) continue;
    const int i = w / R, split = w % R;
    float mi = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < NB; ++kb) mi = fmaxf(mi, mblk[i][kb]);
    float acc = 0.f;
    for (int kb = split * bps; kb < (split + 1) * bps; ++kb) {
      const float m = mblk[i][kb];
      if (m == -INFINITY) continue;
      float a = 0.f;
#pragma unroll
      for (int j = kb * SKB; j < (kb + 1) * SKB; j += 8) {
        float vf[8];
        if constexpr (VT) {
          const u32x4 vw = *reinterpret_cast<const u32x4*>(&vs[d][j]);
          const T* ve = reinterpret_cast<const T*>(&vw);
#pragma unroll
          for (int e = 0; e < 8; ++e) vf[e] = Num<T>::to_f(ve[e]);
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e) vf[e] = Num<T>::to_f(vs[j + e][d]);
        }
        const float4 p0 = *reinterpret_cast<const float4*>(&ps[i * SKC + j]);
        const float4 p1 = *reinterpret_cast<const float4*>(&ps[i * SKC + j + 4]);
        const float pv[8] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) a = fmaf(pv[e], vf[e], a);
      }
      acc = fmaf(a, __builtin_amdgcn_exp2f(m - mi), acc);
    }
    acc_w[n] = acc;
  }
  __syncthreads();  // every P V read of ps is done: it now takes the split sums
#pragma unroll
  for (int n = 0; n < MAXW; ++n) {
    const int w = slot + n * SLOTS;
    if (w < G * R) ps[w * DD + d] = acc_w[n];
  }
  __syncthreads();
  for (int i = slot; i < G; i += SLOTS) {
    float acc = 0.f;
    for (int r = 0; r < R; ++r) acc += ps[(i * R + r) * DD + d];
    part[i * kStepPart + 2 + d] = acc;
    if (d == 0) {
      float mi = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < NB; ++kb) mi = fmaxf(mi, mblk[i][kb]);
      float l = 0.f;
#pragma unroll
      for (int kb = 0; kb < NB; ++kb) {
        const float m = mblk[i][kb];
        l += m == -INFINITY ? 0.f : lblk[i][kb] * __builtin_amdgcn_exp2f(m - mi);
      }
      part[i * kStepPart] = mi;
      part[i * kStepPart + 1] = l;
    }
  }
}

// Merge of one query head of one unit (blockIdx.x = unit * g + head), one
// thread per output column: the partials of the chunks holding keys 0..P,
// O = sum_c 2^(m_c - M) o_c / sum_c 2^(m_c - M) l_c, M = max m_c.  Up to 32
// chunks' partials are loaded in one round (a 1152-slot cache has 18), so
// the kernel waits for memory once.
constexpr int kMergeThreads = DD;
template <typename T>
__global__ void __launch_bounds__(kMergeThreads) attn_decode_step_merge(const StepArgs p) {
  const int d = threadIdx.x, G = p.g;
  const int unit = blockIdx.x / G, i = blockIdx.x % G;
  const int b = unit / p.n_kv, h = unit % p.n_kv;
  // every chunk has a partial (those past P with m = -inf); P is read
  // alongside them, only to write nothing when the step kernel refused it
  const int nvis = p.nchunks;
  const int64_t P = *p.pos;
  const float* up = p.part + (static_cast<int64_t>(unit) * p.nchunks * G + i) * kStepPart;
  const int64_t cs = static_cast<int64_t>(G) * kStepPart;  // between chunks
  T* O = static_cast<T*>(p.out) + b * p.ld_out + static_cast<int64_t>(h * G + i) * DD;
  constexpr int NB = 32;  // partials loaded together (all loads in flight)
  float M = -INFINITY, l = 0.f, acc = 0.f;
  for (int c0 = 0; c0 < nvis; c0 += NB) {
    float mm[NB], ll[NB], oo[NB];
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const bool in = c0 + j < nvis;
      const float* pc = up + (in ? c0 + j : nvis - 1) * cs;  // a valid partial
      mm[j] = in ? pc[0] : -INFINITY;
      ll[j] = in ? pc[1] : 0.f;
      oo[j] = in ? pc[2 + d] : 0.f;
    }
    float bm = M;
#pragma unroll
    for (int j = 0; j < NB; ++j) bm = fmaxf(bm, mm[j]);
    // chunk 0 holds key 0, so bm is finite from the first batch on
    const float sc = __builtin_amdgcn_exp2f(M - bm);
    l *= sc;
    acc *= sc;
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      // a neutral partial (m = -inf) carries no output sums
      const bool live = mm[j] != -INFINITY;
      const float w = __builtin_amdgcn_exp2f(mm[j] - bm);
      l = live ? fmaf(ll[j], w, l) : l;
      acc = live ? fmaf(oo[j], w, acc) : acc;
    }
    M = bm;
  }
  if (P >= 0 && P < p.max_len) O[d] = Num<T>::from_f(acc / l);
}

}  // namespace
}  // namespace sph

extern "C" int64_t sph_decode_attention_step_workspace_bytes(int64_t batch, int64_t n_heads,
                                                              int64_t n_kv_heads,
                                                              int64_t max_len) {
  if (batch <= 0 || n_kv_heads <= 0 || n_heads <= 0 || max_len <= 0) return 0;
  const int64_t g = n_heads / n_kv_heads;
  return batch * n_kv_heads * ((max_len + kMinChunk - 1) / kMinChunk) * g * kStepPart * 4;
}

extern "C" int sph_decode_attention_step(
    sph_dtype dtype, int64_t batch, int64_t n_heads, int64_t n_kv_heads, int64_t head_dim,
    const void* qkv, int64_t ld_qkv, const void* cos, const void* sin, int64_t ld_rope,
    const int64_t* pos, int32_t* error_word, void* k_cache, int64_t k_stride_b, int64_t k_stride_h,
    int64_t k_stride_s, void* v_cache, int64_t v_stride_b, int64_t v_stride_h,
    int64_t v_key_stride, int64_t v_dim_stride, int64_t max_len, float scale, void* out,
    int64_t ld_out, void* workspace, int64_t workspace_bytes, sph_stream_t stream) {
  SPH_REQUIRE(dtype == SPH_F16 || dtype == SPH_BF16, SPH_ERR_UNSUPPORTED,
              "decode attention step: dtype must be F16 or BF16");
  SPH_REQUIRE(head_dim == DD, SPH_ERR_UNSUPPORTED, "decode attention step: head_dim must be 128");
  SPH_REQUIRE(batch >= 0 && n_heads > 0 && n_kv_heads > 0 && max_len > 0, SPH_ERR_INVALID_ARG,
              "decode attention step: bad sizes");
  if (batch == 0) return SPH_OK;
  SPH_REQUIRE(n_heads % n_kv_heads == 0 && n_heads / n_kv_heads <= SG, SPH_ERR_UNSUPPORTED,
              "decode attention step: query heads per KV head must divide and be <= 8");
  SPH_REQUIRE(batch * n_kv_heads <= kMaxUnits && max_len < (1LL << 30), SPH_ERR_TOO_LARGE,
              "decode attention step: at most 4096 (batch x KV heads) and 2^30 positions");
  SPH_REQUIRE(scale > 0.f && scale < INFINITY, SPH_ERR_INVALID_ARG,
              "decode attention step: scale must be positive and finite");
  SPH_REQUIRE(pos != nullptr && qkv != nullptr && k_cache != nullptr && v_cache != nullptr &&
                  out != nullptr,
              SPH_ERR_INVALID_ARG, "decode attention step: null pointer");
  SPH_REQUIRE((v_dim_stride == 1 && v_key_stride >= DD) ||
                  (v_key_stride == 1 && v_dim_stride >= max_len),
              SPH_ERR_INVALID_ARG,
              "decode attention step: V cache must be key-major or dim-major");
  const bool vt = v_key_stride == 1 && v_dim_stride != 1;
  SPH_REQUIRE(ld_qkv >= (n_heads + 2 * n_kv_heads) * DD && ld_rope >= DD && k_stride_s >= DD &&
                  ld_out >= n_heads * DD,
              SPH_ERR_INVALID_ARG, "decode attention step: leading dimension too small");
  SPH_REQUIRE(al16d(k_cache) && k_stride_s % 8 == 0 && k_stride_h % 8 == 0 &&
                  k_stride_b % 8 == 0,
              SPH_ERR_INVALID_ARG, "decode attention step: K cache rows must be 16-byte aligned");
  // V rows: key-major ones are read as 16-byte chunks and must be aligned;
  // dim-major ones (max_len keys each) may have any length
  const bool v_al = al16d(v_cache) && v_stride_b % 8 == 0 && v_stride_h % 8 == 0 &&
                    (vt ? v_dim_stride : v_key_stride) % 8 == 0;
  SPH_REQUIRE(vt || v_al, SPH_ERR_INVALID_ARG,
              "decode attention step: key-major V cache rows must be 16-byte aligned");
  SPH_REQUIRE((reinterpret_cast<uintptr_t>(v_cache) & 1u) == 0, SPH_ERR_INVALID_ARG,
              "decode attention step: V cache must be 2-byte aligned");
  const int64_t need =
      sph_decode_attention_step_workspace_bytes(batch, n_heads, n_kv_heads, max_len);
  SPH_REQUIRE(workspace != nullptr && workspace_bytes >= need, SPH_ERR_INVALID_ARG,
              "decode attention step: workspace too small");
  StepArgs p{};
  p.qkv = qkv;
  p.ld_qkv = ld_qkv;
  p.cos = cos;
  p.sin = sin;
  p.ld_rope = ld_rope;
  p.pos = pos;
  p.err = error_word;
  p.kc = k_cache;
  p.k_sb = k_stride_b;
  p.k_sh = k_stride_h;
  p.k_ss = k_stride_s;
  p.vc = v_cache;
  p.v_sb = v_stride_b;
  p.v_sh = v_stride_h;
  p.v_ks = v_key_stride;
  p.v_ds = v_dim_stride;
  p.v_al = v_al ? 1 : 0;
  p.max_len = max_len;
  p.n_heads = static_cast<int>(n_heads);
  p.n_kv = static_cast<int>(n_kv_heads);
  p.g = static_cast<int>(n_heads / n_kv_heads);
  // Launch shape: 64-key chunks on 256 threads (44 KB of LDS, three
  // workgroups per CU).  Measured on the c5 decode step (4 x 8 KV heads,
  // 1152 slots, position 1087): 7.4 us against 8.0 us for 128 keys x 512
  // threads; before the score dot products became v_dot2, 8.0 us against
  // 10.1 / 8.6 / 11.3 / 9.5 us for 128 x 256 / 128 x 512 / 256 x 512 /
  // 256 x 1024 (larger chunks leave fewer workgroups per CU to overlap one's
  // loads with another's arithmetic).
  constexpr int kChunk = 64, kThreads = 256;
  p.nchunks = static_cast<int>((max_len + kChunk - 1) / kChunk);
  p.scale_log2 = scale * kLog2eD;
  p.out = out;
  p.ld_out = ld_out;
  p.part = static_cast<float*>(workspace);
  hipStream_t st = as_stream(stream);
  dim3 grid(static_cast<unsigned>(p.nchunks), static_cast<unsigned>(batch * n_kv_heads));
  const dim3 mgrid(static_cast<unsigned>(batch * n_kv_heads * p.g));
  auto go = [&](auto tag, auto vt_tag) {
    using T = decltype(tag);
    constexpr bool VT = decltype(vt_tag)::value;
    attn_decode_step_kernel<T, VT, kChunk, kThreads><<<grid, kThreads, 0, st>>>(p);
    attn_decode_step_merge<T><<<mgrid, kMergeThreads, 0, st>>>(p);
  };
  if (dtype == SPH_F16) {
    if (vt) go(half_t{}, std::true_type{});
    else go(half_t{}, std::false_type{});
  } else {
    if (vt) go(bf16_t{}, std::true_type{});
    else go(bf16_t{}, std::false_type{});
  }
  return check_launch("sph_decode_attention_step");
}
