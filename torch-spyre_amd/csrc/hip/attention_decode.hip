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
