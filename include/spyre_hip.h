/*
 * spyre_hip.h -- C-ABI of the MI355X (gfx950) kernel library behind the
 * torch_spyre PrivateUse1 backend.
 *
 * This is the drop-in boundary: the ATen glue in torch_spyre/_C (eager ops)
 * and the compiled-kernel runners (torch.compile path) call only these entry
 * points.  Conventions:
 *   - every function returns int status: 0 = ok; a positive hipError_t value
 *     when the HIP runtime failed; SPH_ERR_* (>= 1000) for argument errors.
 *     sph_last_error() returns a thread-local message for the last failure.
 *   - no C++ exception crosses this ABI; no torch type appears in it.
 *   - every pointer is a device pointer owned by the caller, except where a
 *     parameter is documented as a host pointer.  Nothing here allocates
 *     device memory.
 *   - every launch takes an explicit stream (a hipStream_t passed as void*;
 *     NULL = the legacy default stream) and is asynchronous w.r.t. the host.
 *   - sizes, strides and leading dimensions are int64_t and count ELEMENTS.
 *
 * Reference interfaces replaced (paths relative to the torch-spyre tree):
 *   The reference runs every device op through the IBM sendnn/flex SDK:
 *   eager kernels build a sendnn graph per (op, shape, stride) and call
 *   GraphLoader::Compute (codegen/templates/base.jinja2:135-232,
 *   codegen/inputs/spyre_torch_ops.cpp:214-452), compiled kernels are SuperDSC
 *   programs launched by _C.launch_kernel (torch_spyre/csrc/module.cpp:64-170),
 *   and host<->device copies build a 3-stage DMA graph with a stick-layout
 *   conversion (torch_spyre/csrc/spyre_mem.cpp:281-438).  Each entry point
 *   below names the reference function it stands in for.
 */
#ifndef SPYRE_HIP_H_
#define SPYRE_HIP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SPH_ABI_VERSION 1
#define SPH_MAX_DIMS 8

typedef void* sph_stream_t; /* hipStream_t */

/* Status codes beyond hipError_t. */
enum {
  SPH_OK = 0,
  SPH_ERR_INVALID_ARG = 1001,
  SPH_ERR_UNSUPPORTED = 1002,
  SPH_ERR_TOO_LARGE = 1003
};

/* Element types.  Codes are this library's own, not torch's. */
typedef enum {
  SPH_F16 = 0,
  SPH_BF16 = 1,
  SPH_F32 = 2,
  SPH_F64 = 3,
  SPH_I8 = 4,
  SPH_U8 = 5,
  SPH_I16 = 6,
  SPH_I32 = 7,
  SPH_I64 = 8,
  SPH_BOOL = 9
} sph_dtype;

/* ------------------------------------------------------------------ */
/* Library / diagnostics                                               */
/* ------------------------------------------------------------------ */

/* Thread-local message describing the last non-zero status. */
const char* sph_last_error(void);

/* SPH_ABI_VERSION of the built library. */
int sph_abi_version(void);

/* ------------------------------------------------------------------ */
/* Row softmax                                                         */
/* Replaces: generated spyre___softmax_default / _out                  */
/*   (codegen/inputs/Metadata.yaml:275-277, codegen/templates/          */
/*    base.jinja2:16-241) and the compiled amax/sub/exp/sum/realdiv    */
/*   chain (torch_spyre/_inductor/choices.py:58-83).                   */
/* ------------------------------------------------------------------ */

/* Softmax flags. */
enum {
  SPH_SOFTMAX_LOG = 1,   /* log_softmax instead of softmax */
  SPH_SOFTMAX_CAUSAL = 2 /* mask column c of row r when
                            c > (r % causal_q_len) + causal_offset */
};

/* y[r, c] = softmax_c(scale * x[r, c]) over each of `rows` rows of `cols`
 * elements; row r of x starts at x + r*ldx, of y at y + r*ldy.
 * Arithmetic in fp32; in_dtype/out_dtype in {F16, BF16, F32}.
 * A row whose every column is masked produces NaN, as torch does. */
int sph_softmax_rows(sph_dtype in_dtype, sph_dtype out_dtype, const void* x,
                     int64_t ldx, void* y, int64_t ldy, int64_t rows,
                     int64_t cols, float scale, int flags,
                     int64_t causal_q_len, int64_t causal_offset,
                     sph_stream_t stream);

/* fp16 shorthand: contiguous rows, scale 1, no mask. */
int sph_softmax_rows_f16(const void* x, void* y, int64_t rows, int64_t cols,
                         sph_stream_t stream);

/* ------------------------------------------------------------------ */
/* Normalisation over the last dimension (rows x cols, contiguous)      */
/* Replaces: spyre__native_layer_norm_default (stub returning its input,*/
/*   codegen/inputs/spyre_torch_ops.cpp:188-194), the compiled          */
/*   exx2 -> layernormscale -> layernormnorm chain                      */
/*   (torch_spyre/_inductor/decompositions.py:26-36, customops.py:      */
/*   102-154, lowering.py:78-153) and the 5-launch eager RMSNorm        */
/*   composite pow/mean/add/rsqrt/mul (spyre_torch_ops.cpp:456-474).    */
/* ------------------------------------------------------------------ */

/* If residual != NULL: h = round_to_dtype(x + residual) is written to h_out
 * (h_out may alias x or residual) and normalised; otherwise h = x.
 * RMSNorm:   y = h * rsqrt(mean(h^2) + eps) * weight
 * LayerNorm: y = (h - mean(h)) * rsqrt(var(h) + eps) * weight + bias
 * weight / bias may be NULL (treated as 1 / 0); w_dtype is the dtype of
 * weight and bias (F32 or the activation dtype).  mean_out / rstd_out are
 * optional fp32 per-row outputs (the saved statistics of
 * aten::native_layer_norm / aten::_fused_rms_norm). */
int sph_rmsnorm(sph_dtype dtype, sph_dtype w_dtype, const void* x,
                const void* residual, const void* weight, void* y,
                void* h_out, float* rstd_out, int64_t rows, int64_t cols,
                float eps, sph_stream_t stream);

int sph_layernorm(sph_dtype dtype, sph_dtype w_dtype, const void* x,
                  const void* residual, const void* weight, const void* bias,
                  void* y, void* h_out, float* mean_out, float* rstd_out,
                  int64_t rows, int64_t cols, float eps, sph_stream_t stream);

/* fp16 shorthands of the above with fp16 weight/bias. */
int sph_rmsnorm_f16(const void* x, const void* residual, const void* weight,
                    void* y, void* h_out, int64_t rows, int64_t cols,
                    float eps, sph_stream_t stream);
int sph_layernorm_f16(const void* x, const void* residual, const void* weight,
                      const void* bias, void* y, void* h_out, int64_t rows,
                      int64_t cols, float eps, sph_stream_t stream);

/* ------------------------------------------------------------------ */
/* Fused pointwise chain + row reduction                                */
/* Replaces: generated gelu (approximate forced to "none",             */
/*   codegen/inputs/Metadata.yaml:125-132) followed by ReduceSum        */
/*   (Metadata.yaml:299-302); the compile path cannot lower erf at all  */
/*   (torch_spyre/_inductor/opfuncs.py:49-72).                          */
/* ------------------------------------------------------------------ */

/* y[r,c] = gelu_erf(x[r,c] * s[c] + b[c]);  rowsum[r] = sum_c y[r,c]
 * (sum of the fp32 values before rounding to dtype).  s / b may be NULL,
 * then the scalars s_scalar / b_scalar are used.  s, b have `dtype`.
 * rowsum has `dtype`; y or rowsum may be NULL to skip that output. */
int sph_gelu_affine_rowsum(sph_dtype dtype, const void* x, const void* s,
                           const void* b, float s_scalar, float b_scalar,
                           void* y, void* rowsum, int64_t rows, int64_t cols,
                           sph_stream_t stream);

int sph_gelu_affine_rowsum_f16(const void* x, const void* s, const void* b,
                               void* y, void* rowsum, int64_t rows,
                               int64_t cols, sph_stream_t stream);

/* ------------------------------------------------------------------ */
/* GEMM on MFMA (fp32 accumulate)                                       */
/* Replaces: spyre__mm_default (codegen/inputs/spyre_torch_ops.cpp:     */
/*   214-293), spyre__bmm_default (:297-377), spyre__addmm_* (:381-452) */
/*   and the compiled "pt"-unit matmul (torch_spyre/_inductor/          */
/*   codegen/compute_ops.py:396-824).                                   */
/* ------------------------------------------------------------------ */

/* Epilogue selectors applied to alpha*A@B + beta*C before rounding. */
enum {
  SPH_EPI_NONE = 0,
  SPH_EPI_RELU = 1,
  SPH_EPI_GELU = 2, /* erf form */
  SPH_EPI_SILU = 3
};

/* Row-major D[m,n] = epi(alpha * op(A)[m,k] @ op(B)[k,n] + beta * C[m,n]).
 * op(A) = A (trans_a = 0, A[i,p] at a + i*lda + p) or A^T (trans_a = 1,
 * A[i,p] at a + p*lda + i); likewise B with ldb.  C is optional (NULL or
 * beta == 0 ignore it) and is addressed as c[i*ldc_row + j*ldc_col], so a
 * bias row broadcast is ldc_row = 0, ldc_col = 1.  C and D may alias only
 * when they are the same matrix with the same strides.
 * dtype in {F16, BF16}: A, B, C, D all have it.  Any m, n, k >= 0. */
int sph_gemm(sph_dtype dtype, int trans_a, int trans_b, int64_t m, int64_t n,
             int64_t k, float alpha, const void* a, int64_t lda,
             const void* b, int64_t ldb, float beta, const void* c,
             int64_t ldc_row, int64_t ldc_col, void* d, int64_t ldd,
             int epilogue, sph_stream_t stream);

/* Strided batched form: batch b uses a + b*stride_a, etc. (stride_c may be
 * 0 to broadcast one C over the batch). */
int sph_gemm_strided_batched(sph_dtype dtype, int trans_a, int trans_b,
                             int64_t batch, int64_t m, int64_t n, int64_t k,
                             float alpha, const void* a, int64_t lda,
                             int64_t stride_a, const void* b, int64_t ldb,
                             int64_t stride_b, float beta, const void* c,
                             int64_t ldc_row, int64_t ldc_col,
                             int64_t stride_c, void* d, int64_t ldd,
                             int64_t stride_d, int epilogue,
                             sph_stream_t stream);

/* D = rms_norm(X) W^T for decode shapes (1 <= m <= 8 rows): row i of X
 * [m, k] is normalised as X[i] * norm_w * rsqrt(mean(X[i]^2) + eps) inside
 * the weight-stream kernels (no separate norm kernel, no normalised copy of
 * X): norm_w multiplies each chunk of X as it is loaded (rounded to the
 * dtype), the row scale multiplies the finished sums.  W [n, k] (or, with
 * swiglu, [2n, k]: gate rows then up rows, D = silu(g) * u) is the
 * nn.Linear weight layout.  F16 / BF16; 64 <= k <= 8192, k % 8 == 0, rows
 * of X, norm_w and W 16-byte aligned.
 * Replaces: the reference's RMSNorm composite (pow / mean / add / rsqrt /
 * mul, Metadata.yaml:236-253, spyre_torch_ops.cpp:456-474) followed by
 * spyre__mm_default (spyre_torch_ops.cpp:214-293). */
int sph_gemm_rmsnorm(sph_dtype dtype, int64_t m, int64_t n, int64_t k, const void* a, int64_t lda,
                     const void* norm_w, float eps, const void* w, int64_t ldw, void* d,
                     int64_t ldd, int swiglu, sph_stream_t stream);

/* D[m, j] = silu(sum_k A[m, k] W[j, k]) * (sum_k A[m, k] W[n + j, k]) for
 * j < n: the gate and up projections of a SwiGLU MLP from one weight
 * matrix W [2n, k] (gate rows first), both K-contiguous, and the
 * activation product, in one GEMM (fp32 sums, one rounding to dtype).
 * Replaces: spyre__mm_default (spyre_torch_ops.cpp:214-293) for x W^T
 * followed by the generated silu and mul ops (Metadata.yaml base ops,
 * base.jinja2:16-241); no single reference function corresponds (the
 * reference does not fuse).  Takes m <= 8 (decode: 64 <= k <= 8192,
 * k % 8 == 0) or m % 256 == 0 with n % 128 == 0 and k % 64 == 0, and
 * 16-byte aligned rows; other shapes return SPH_ERR_UNSUPPORTED (compute
 * the three steps instead).  workspace (may be NULL) of
 * sph_gemm_swiglu_workspace_bytes(m, n, k) bytes lets a tiled call split
 * its last, partial round of tiles along K. */
int sph_gemm_swiglu(sph_dtype dtype, int64_t m, int64_t n, int64_t k, const void* a,
                    int64_t lda, const void* w, int64_t ldw, void* d, int64_t ldd,
                    void* workspace, int64_t workspace_bytes, sph_stream_t stream);
int64_t sph_gemm_swiglu_workspace_bytes(int64_t m, int64_t n, int64_t k);

/* sph_gemm_strided_batched with a workspace (device memory, may be NULL):
 * with at least sph_gemm_workspace_bytes(batch, m, n, k) bytes, a product
 * on whole 256 x 256 tiles whose tile count leaves a partial last round on
 * the 256 CUs may split that round's tiles along K into fp32 partial tiles
 * (summed and finished with the epilogue by a second kernel) instead of
 * running it on a few CUs; the size is 0 for shapes where the library's
 * time model prefers whole rounds of 256- or 128-wide tiles.  Same results up to fp32 summation order.  No
 * counterpart in the reference (its GEMM is one device call,
 * spyre_torch_ops.cpp:214-293); calls sharing a workspace must be ordered
 * on a stream. */
int sph_gemm_ex(sph_dtype dtype, int trans_a, int trans_b, int64_t batch, int64_t m, int64_t n,
                int64_t k, float alpha, const void* a, int64_t lda, int64_t stride_a,
                const void* b, int64_t ldb, int64_t stride_b, float beta, const void* c,
                int64_t ldc_row, int64_t ldc_col, int64_t stride_c, void* d, int64_t ldd,
                int64_t stride_d, int epilogue, void* workspace, int64_t workspace_bytes,
                sph_stream_t stream);
int64_t sph_gemm_workspace_bytes(int64_t batch, int64_t m, int64_t n, int64_t k);

/* fp16 shorthands: contiguous row-major, no transpose, no C. */
int sph_gemm_f16(int64_t m, int64_t n, int64_t k, const void* a,
                 const void* b, void* d, sph_stream_t stream);
int sph_bmm_f16(int64_t batch, int64_t m, int64_t n, int64_t k,
                const void* a, const void* b, void* d, sph_stream_t stream);

/* ------------------------------------------------------------------ */
/* Fused attention forward                                              */
/* Replaces: the chain the reference runs for attention, spyre__bmm_    */
/*   default (spyre_torch_ops.cpp:297-377) for the scores, the          */
/*   generated add + _softmax (Metadata.yaml:275-277, base.jinja2:16-   */
/*   241) and spyre__bmm_default again for P V: the same result without */
/*   writing the [mq, sk] score matrix.  No single reference function   */
/*   corresponds; the compile backend substitutes it for that chain.    */
/* ------------------------------------------------------------------ */

/* O[b] = softmax(scale * Q[b] K[b]^T + M[b]) V[b] for b < batch, with
 * Q[b] [mq, head_dim] at q + b*stride_q (row i at + i*ldq), K[b], V[b]
 * [sk, head_dim] likewise, O[b] [mq, head_dim].  M is optional (NULL):
 * an additive [mq, sk] mask in natural-log units (-inf drops a key) at
 * mask + b*stride_m (stride_m 0 shares one mask), row i at + i*ldm.
 * causal_q > 0 additionally drops keys j > (i % causal_q) + causal_off
 * for row i (query heads stacked along the rows keep their positions).
 * dtype in {F16, BF16} for Q, K, V, M, O; fp32 scores and accumulation;
 * head_dim must be 128, mq a multiple of 128 (or at most 16: the decode
 * path, sph_attention_decode), rows 16-byte aligned (mask rows 8-byte
 * aligned; ldm 0 shares one mask row between all rows).  A row with no visible key yields NaN, as
 * softmax over all -inf does.
 * workspace (device memory, may be NULL) of at least
 * sph_attention_workspace_bytes(batch, mq, sk, stride_m) bytes lets a mask
 * call class the mask's 128 x 64 blocks first (all zero / mixed / all
 * -inf; 16-byte aligned mask rows) and skip the all -inf ones: a causal
 * mask then costs about half the work.  The workspace is written on
 * `stream`; calls sharing one workspace must be ordered on a stream. */
int sph_attention_fwd(sph_dtype dtype, int64_t batch, int64_t mq, int64_t sk,
                      int64_t head_dim, const void* q, int64_t ldq, int64_t stride_q,
                      const void* k, int64_t ldk, int64_t stride_k, const void* v,
                      int64_t ldv, int64_t stride_v, const void* mask, int64_t ldm,
                      int64_t stride_m, int64_t causal_q, int64_t causal_off, float scale,
                      void* o, int64_t ldo, int64_t stride_o, void* workspace,
                      int64_t workspace_bytes, sph_stream_t stream);
/* Bytes of mask-block classes sph_attention_fwd uses for this shape: one
 * per (mask batch, 128-row block, 64-key block); 0 for an empty shape.
 * For mq <= 16 (the decode path below) the split workspace of
 * sph_attention_decode_workspace_bytes instead. */
int64_t sph_attention_workspace_bytes(int64_t batch, int64_t mq, int64_t sk, int64_t stride_m);

/* Decode-step attention: the same O[b] = softmax(scale * Q[b] K[b]^T +
 * M[b]) V[b] for at most 16 query rows per batch entry (a KV head's group
 * of query heads at one position) over sk keys.  sph_attention_fwd routes
 * mq <= 16 here.  V is given by element strides: key-major (v_dim_stride
 * 1, row stride v_key_stride >= 128) or dim-major (v_key_stride 1,
 * v_dim_stride >= sk), as a KV cache kept for the P V product stores it.
 * The mask row stride ldm may be 0 (one mask row for every query row).
 * causal_q / causal_off as for sph_attention_fwd.  With a workspace of
 * sph_attention_decode_workspace_bytes(batch, mq, sk) bytes the keys are
 * split over several workgroups per batch entry and merged by a second
 * kernel; without one (NULL or too small) one workgroup per batch entry
 * walks every key.  Replaces, for decode shapes, the same reference chain
 * as sph_attention_fwd (spyre_torch_ops.cpp:297-377, Metadata.yaml:275-
 * 277). */
int sph_attention_decode(sph_dtype dtype, int64_t batch, int64_t mq, int64_t sk,
                         int64_t head_dim, const void* q, int64_t ldq, int64_t stride_q,
                         const void* k, int64_t ldk, int64_t stride_k, const void* v,
                         int64_t v_key_stride, int64_t v_dim_stride, int64_t stride_v,
                         const void* mask, int64_t ldm, int64_t stride_m, int64_t causal_q,
                         int64_t causal_off, float scale, void* o, int64_t ldo,
                         int64_t stride_o, void* workspace, int64_t workspace_bytes,
                         sph_stream_t stream);
/* Split workspace bytes of sph_attention_decode (0: no split for this
 * shape, or mq > 16). */
int64_t sph_attention_decode_workspace_bytes(int64_t batch, int64_t mq, int64_t sk);

/* One decode step of grouped-query attention with its KV-cache append, for
 * every batch entry and KV head in one launch.  qkv [batch, (n_heads +
 * 2 n_kv_heads) * 128] (row stride ld_qkv) holds each entry's query heads,
 * then its new keys, then its new values; P = *pos (a device int64) is the
 * new token's position.  Queries and new keys are rotated by RoPE at P
 * (rotate-half, tables cos / sin [max_len, 128], row stride ld_rope), the
 * key and value are stored in the caches at P, and out[b] (row stride
 * ld_out, query head j at columns j * 128) = softmax(scale q K[0..P]^T)
 * V[0..P] for each query head j, over KV head j / (n_heads / n_kv_heads).
 * K cache [batch, n_kv_heads, max_len, 128] by element strides (dim stride
 * 1, 16-byte aligned rows); V cache key-major (v_dim_stride 1, 16-byte
 * aligned rows) or dim-major (v_key_stride 1, rows of any length).
 * dtype F16 / BF16; fp32 scores and sums; n_heads / n_kv_heads <= 8;
 * batch * n_kv_heads <= 4096.  workspace: at least
 * sph_decode_attention_step_workspace_bytes(...) bytes for the per-chunk
 * partials.  A P outside [0, max_len) writes nothing and sets *error_word
 * (device-visible int32, may be NULL) to 2.  Two launches on `stream`:
 * per-chunk partials into the workspace, then their merge.
 * Replaces, for a decode step, the chain the reference runs op by op: the
 * RoPE pointwise ops and the cache copy (Metadata.yaml generated mul / add /
 * neg / cat and spyre__copy_from, spyre_mem.cpp:661-703), then
 * spyre__bmm_default (codegen/inputs/spyre_torch_ops.cpp:297-377), add +
 * _softmax (Metadata.yaml:275-277) and spyre__bmm_default again. */
int sph_decode_attention_step(sph_dtype dtype, int64_t batch, int64_t n_heads,
                              int64_t n_kv_heads, int64_t head_dim, const void* qkv,
                              int64_t ld_qkv, const void* cos, const void* sin, int64_t ld_rope,
                              const int64_t* pos, int32_t* error_word, void* k_cache,
                              int64_t k_stride_b, int64_t k_stride_h, int64_t k_stride_s,
                              void* v_cache, int64_t v_stride_b, int64_t v_stride_h,
                              int64_t v_key_stride, int64_t v_dim_stride, int64_t max_len,
                              float scale, void* out, int64_t ld_out, void* workspace,
                              int64_t workspace_bytes, sph_stream_t stream);
/* Workspace bytes of sph_decode_attention_step (0 for an empty shape). */
int64_t sph_decode_attention_step_workspace_bytes(int64_t batch, int64_t n_heads,
                                                  int64_t n_kv_heads, int64_t max_len);

/* sph_attention_fwd for callers that cannot allocate device memory (code
 * under HIP graph capture, serving loops, harnesses that forbid
 * hipMalloc): the same arguments without the workspace, the same kernels
 * and results (bit for bit: a masked prefill call classes the mask blocks,
 * a decode call splits its keys, as sph_attention_fwd with a workspace of
 * sph_attention_workspace_bytes does).  The workspace is a static device
 * array of sph_attention_fwd_noalloc_max_bytes() (4 MiB) per GPU, held
 * until the process ends; a shape that needs more returns
 * SPH_ERR_TOO_LARGE before any launch.  Nothing is allocated and nothing
 * needs clearing between calls, but every call on one GPU uses that GPU's
 * one array: calls that may overlap on a GPU (other streams, other host
 * threads) race and must be ordered by the caller.
 * No counterpart in the reference: it exists for callers that cannot
 * allocate. */
int sph_attention_fwd_noalloc(sph_dtype dtype, int64_t batch, int64_t mq, int64_t sk,
                              int64_t head_dim, const void* q, int64_t ldq, int64_t stride_q,
                              const void* k, int64_t ldk, int64_t stride_k, const void* v,
                              int64_t ldv, int64_t stride_v, const void* mask, int64_t ldm,
                              int64_t stride_m, int64_t causal_q, int64_t causal_off,
                              float scale, void* o, int64_t ldo, int64_t stride_o,
                              sph_stream_t stream);
/* Bytes of the static workspace of sph_attention_fwd_noalloc. */
int64_t sph_attention_fwd_noalloc_max_bytes(void);

/* ------------------------------------------------------------------ */
/* Generic strided pointwise engine                                     */
/* Replaces: the generated base/list_inp eager ops of Metadata.yaml     */
/*   (add/sub/mul/div/exp/log/.../where/eq/ge, base.jinja2:16-241),     */
/*   spyre__clone_default (spyre_torch_ops.cpp:507-583),                */
/*   spyre__fill_Scalar (:394-403) and the SFP OpFuncs of the compile   */
/*   path (torch_spyre/_inductor/opfuncs.py:49-72).                     */
/* ------------------------------------------------------------------ */

typedef struct {
  void* data;                     /* device pointer */
  int32_t dtype;                  /* sph_dtype */
  int32_t pad_;
  int64_t strides[SPH_MAX_DIMS];  /* element strides, 0 = broadcast */
} sph_operand;

/* Pointwise op codes.  Arity in brackets; a, b, c are inputs 0..2,
 * alpha/beta the scalar parameters. */
enum {
  SPH_PW_COPY = 0,        /* [1] out = a (with dtype conversion) */
  SPH_PW_FILL = 1,        /* [0] out = alpha */
  SPH_PW_ADD = 2,         /* [2] out = a + alpha*b */
  SPH_PW_SUB = 3,         /* [2] out = a - alpha*b */
  SPH_PW_MUL = 4,         /* [2] out = a * b */
  SPH_PW_DIV = 5,         /* [2] out = a / b */
  SPH_PW_ADD_SCALAR = 6,  /* [1] out = a + alpha */
  SPH_PW_MUL_SCALAR = 7,  /* [1] out = a * alpha */
  SPH_PW_RSUB_SCALAR = 8, /* [1] out = alpha - a */
  SPH_PW_DIV_SCALAR = 9,  /* [1] out = a / alpha */
  SPH_PW_POW_SCALAR = 10, /* [1] out = a ^ alpha */
  SPH_PW_RPOW_SCALAR = 11,/* [1] out = alpha ^ a */
  SPH_PW_POW = 12,        /* [2] out = a ^ b */
  SPH_PW_MAXIMUM = 13,    /* [2] */
  SPH_PW_MINIMUM = 14,    /* [2] */
  SPH_PW_NEG = 20,        /* [1] */
  SPH_PW_ABS = 21,
  SPH_PW_EXP = 22,
  SPH_PW_LOG = 23,
  SPH_PW_SQRT = 24,
  SPH_PW_RSQRT = 25,
  SPH_PW_RECIPROCAL = 26,
  SPH_PW_SIGMOID = 27,
  SPH_PW_TANH = 28,
  SPH_PW_RELU = 29,
  SPH_PW_GELU = 30,       /* erf form */
  SPH_PW_GELU_TANH = 31,
  SPH_PW_SILU = 32,
  SPH_PW_SIN = 33,
  SPH_PW_COS = 34,
  SPH_PW_ERF = 35,
  SPH_PW_LOG1P = 36,
  SPH_PW_EXPM1 = 37,
  SPH_PW_MISH = 38,
  SPH_PW_LOGICAL_NOT = 39,
  SPH_PW_BITWISE_NOT = 40,
  SPH_PW_SIGN = 41,
  SPH_PW_FLOOR = 42,
  SPH_PW_CEIL = 43,
  SPH_PW_ROUND = 44,
  SPH_PW_TRUNC = 45,
  SPH_PW_CLAMP = 46,      /* [1] out = min(max(a, alpha), beta) */
  SPH_PW_LEAKY_RELU = 47, /* [1] slope alpha */
  SPH_PW_SQUARE = 48,
  SPH_PW_EQ = 60,         /* [2] comparisons: out is bool (or any dtype) */
  SPH_PW_NE = 61,
  SPH_PW_LT = 62,
  SPH_PW_LE = 63,
  SPH_PW_GT = 64,
  SPH_PW_GE = 65,
  SPH_PW_EQ_SCALAR = 66,  /* [1] compare with alpha */
  SPH_PW_NE_SCALAR = 67,
  SPH_PW_LT_SCALAR = 68,
  SPH_PW_LE_SCALAR = 69,
  SPH_PW_GT_SCALAR = 70,
  SPH_PW_GE_SCALAR = 71,
  SPH_PW_LOGICAL_AND = 72,/* [2] */
  SPH_PW_LOGICAL_OR = 73,
  SPH_PW_WHERE = 80,      /* [3] out = a ? b : c */
  SPH_PW_SILU_MUL = 81,   /* [2] out = silu(a) * b  (SwiGLU) */
  SPH_PW_ADDCMUL = 82,    /* [3] out = a + alpha * b * c */
  SPH_PW_LERP = 83,       /* [2] out = a + alpha * (b - a) */
  SPH_PW_OP_COUNT_ = 128
};

/* out[i] = op(in...[i]) over the index space `sizes` (ndim <= 8, row-major
 * order of dims, last dim fastest).  operands[0] is the output,
 * operands[1..nin] the inputs.  Integer and bool operands are computed in
 * int64 for the integer-exact ops (copy/fill/add/sub/mul/neg/abs/compare/
 * where/logical/bitwise/maximum/minimum); everything else computes in fp32,
 * or fp64 when any operand is F64.  Conversion to the output dtype rounds to
 * nearest-even for floating outputs and truncates toward zero for integer
 * outputs, like torch's casts. */
int sph_pointwise(int op, int nin, const sph_operand* operands, int ndim,
                  const int64_t* sizes, double alpha, double beta,
                  sph_stream_t stream);

/* ------------------------------------------------------------------ */
/* Reductions                                                           */
/* Replaces: eager ReduceSum/mean (Metadata.yaml:299-302,               */
/*   spyre_torch_ops.cpp:456-490) and the compiled sum/max/min/argmax/  */
/*   argmin reductions (torch_spyre/_inductor/opfuncs.py:26-39).        */
/* ------------------------------------------------------------------ */

enum {
  SPH_RED_SUM = 0,
  SPH_RED_MEAN = 1,
  SPH_RED_MAX = 2,
  SPH_RED_MIN = 3,
  SPH_RED_ARGMAX = 4, /* output int64 index along the (single) reduced dim */
  SPH_RED_ARGMIN = 5,
  SPH_RED_PROD = 6,
  SPH_RED_SUMSQ = 7,  /* sum of squares */
  SPH_RED_ANY = 8,
  SPH_RED_ALL = 9
};

/* Reduces `in` over the dims d with reduce_mask bit d set.  sizes[] is the
 * input shape; out.strides[d] is ignored (treated as 0) for reduced dims.
 * Accumulation in fp32 (fp64 for F64 input, int64 for integer sums).
 * For ARGMAX/ARGMIN exactly one dim must be reduced; ties resolve to the
 * first index and NaN wins, as in torch. */
int sph_reduce(int op, const sph_operand* in, const sph_operand* out,
               int ndim, const int64_t* sizes, uint32_t reduce_mask,
               sph_stream_t stream);

/* ------------------------------------------------------------------ */
/* Data movement                                                        */
/* ------------------------------------------------------------------ */

/* Row gather (embedding / index_select on dim 0):
 * out[i, :] = table[idx[i], :] for i < n_idx; rows of `row_elems` elements
 * of `elem_bytes` bytes; idx is int64 (idx_is_i64 = 1) or int32.
 * An index outside [0, num_rows) yields a zero row (no fault) and, when
 * `oob_flag` is not null, a store of 1 to *oob_flag (a device-accessible
 * int32 the caller clears and reads after the stream has completed; torch
 * raises IndexError for such an index, and the ATen backend raises it at its
 * next synchronisation).
 * Replaces: generated embedding (Metadata.yaml:105-115). */
int sph_gather_rows(const void* table, int64_t num_rows, int64_t row_elems,
                    int elem_bytes, const void* idx, int idx_is_i64,
                    int64_t n_idx, void* out, int32_t* oob_flag, sph_stream_t stream);

/* ------------------------------------------------------------------ */
/* Generated and scanned fills                                          */
/* Replaces: the CPU fallbacks of cumsum (spyre_torch_ops.cpp:502-505)  */
/*   and the host paths of arange and the random fills; the identity    */
/*   stub of native_dropout (:180-186).                                 */
/* ------------------------------------------------------------------ */

/* out[i] = start + step * i for i < n, in the output type's accumulation
 * type as torch's CPU arange (float for F16/BF16, double for F32/F64 from
 * start/step; int64 for integer types from istart/istep). */
int sph_arange(sph_dtype dtype, double start, double step, int64_t istart, int64_t istep,
               int64_t n, void* out, sph_stream_t stream);

/* Inclusive prefix sum along the middle dimension of contiguous x, y
 * [outer, len, inner] of one dtype, accumulated as torch's CPU cumsum does
 * (float for F16/BF16, double for F32/F64, int64 for integer types, each
 * partial sum rounded to the dtype when stored).  Columns (inner > 1) and
 * rows of up to 8192 elements are walked sequentially, in the CPU kernel's
 * order, so the results are bit-identical to it; longer rows of the last
 * dimension are scanned by a workgroup each (floating-point sums then
 * differ from the sequential order by rounding). */
int sph_cumsum(sph_dtype dtype, const void* x, void* y, int64_t outer, int64_t len, int64_t inner,
               sph_stream_t stream);

/* Random fill kinds of sph_random_fill. */
enum { SPH_RNG_UNIFORM = 0, SPH_RNG_NORMAL = 1, SPH_RNG_INT = 2 };

/* Fills n contiguous elements from Philox4x32-10 (counter-based): block j
 * is the generator's output for counter offset + j under key `seed`;
 * element i of a fill of 32-bit draws takes word i % 4 of block i / 4, of
 * 64-bit draws (F64 uniform / normal, integer ranges above 2^32) words
 * 2(i % 2), 2(i % 2) + 1 of block i / 2.  SPH_RNG_UNIFORM: a + u (b - a), u
 * in [0, 1) from the top 24 (F64: 53) bits, [a, b) kept half-open after
 * rounding; SPH_RNG_NORMAL: a + b * n, n from Box-Muller on word pairs;
 * SPH_RNG_INT: ifrom + draw % irange (any dtype).  The caller advances its
 * offset by sph_random_blocks(...) per fill. */
int sph_random_fill(int kind, sph_dtype dtype, void* out, int64_t n, uint64_t seed,
                    uint64_t offset, double a, double b, int64_t ifrom, uint64_t irange,
                    sph_stream_t stream);
/* Counter blocks a fill of n elements uses. */
int64_t sph_random_blocks(int kind, sph_dtype dtype, int64_t n, uint64_t irange);

/* Dropout of n contiguous elements: element i is kept when its uniform
 * draw (word i % 4 of Philox block offset + i / 4, top 24 bits) is >= p;
 * y = keep ? x * scale : 0, mask = keep (one byte each).  F16, BF16, F32.
 * Uses (n + 3) / 4 counter blocks. */
int sph_dropout(sph_dtype dtype, const void* x, void* y, uint8_t* mask, int64_t n, float p,
                float scale, uint64_t seed, uint64_t offset, sph_stream_t stream);

/* Transposing copy of elem_bytes-byte elements: for every batch index
 * (up to 4 batch dims of sizes bsizes, element strides bsrc_strides in
 * src and bdst_strides in dst), dst[v * dv + u] = src[u * su + v] for
 * u < U, v < V: v is contiguous in src, u in dst.  64 x 64 tiles through
 * LDS, so reads and writes are both coalesced (a strided elementwise copy
 * reads or writes one element per 64-byte run).  src and dst must not
 * overlap.
 * Replaces: the reference's transpose data ops (torch_spyre/_inductor/
 * codegen/data_ops.py:16-630, "restickify"), for `.contiguous()` of a
 * transposed tensor, eager or compiled. */
int sph_transpose_copy(int elem_bytes, const void* src, void* dst, int64_t U, int64_t V,
                       int64_t su, int64_t dv, int nb, const int64_t* bsizes,
                       const int64_t* bsrc_strides, const int64_t* bdst_strides,
                       sph_stream_t stream);

/* tril/triu on the last two dims of a contiguous [batch, rows, cols]
 * tensor: keep element (r, c) when c - r <= diagonal (lower) or
 * c - r >= diagonal (upper), zero it otherwise.
 * Replaces: generated tril (Metadata.yaml:322-324). */
int sph_tri(int upper, int64_t diagonal, int elem_bytes, const void* x,
            void* y, int64_t batch, int64_t rows, int64_t cols,
            sph_stream_t stream);

/* Rotary position embedding, rotate-half convention, on a contiguous
 * [tokens, heads, head_dim] tensor (in place allowed: y == x):
 * y[..., i]       = x[i] cos(p w_i) - x[i + d/2] sin(p w_i)
 * y[..., i + d/2] = x[i + d/2] cos(p w_i) + x[i] sin(p w_i),
 * w_i = theta^(-2i/d), p = positions[token] (int64).  The compiled and
 * eager decoder both use this; the reference has no RoPE (sin/cos have
 * no OpFunc, torch_spyre/_inductor/opfuncs.py:49-72). */
int sph_rope(sph_dtype dtype, const void* x, void* y,
             const int64_t* positions, int64_t tokens, int64_t heads,
             int64_t head_dim, float theta, sph_stream_t stream);

/* ------------------------------------------------------------------ */
/* Stick (tiled) layout                                                 */
/* Replaces: the host-side stick conversion of the DMA path            */
/*   (torch_spyre/csrc/spyre_mem.cpp:62-279, generate_dci /             */
/*   get_device_stride_info) with an on-GPU permutation.  The layout is */
/*   SpyreTensorLayout's generic stick format                           */
/*   (torch_spyre/csrc/spyre_tensor_impl.cpp:29-74): device dims         */
/*   [ceil(S/E), host dims in dim_order[:-1]..., E] with S the size of  */
/*   the stick dim dim_order[-1] and E = 128 / elem_bytes elements per  */
/*   128-byte stick, row-major on the device, padding sticks zeroed.    */
/*   With the stick dim = K this is the K-panel layout of a GEMM        */
/*   operand: a [rows x 64] panel slice is one contiguous block.        */
/* ------------------------------------------------------------------ */

/* Number of bytes the stick layout of `host_sizes` occupies. */
int64_t sph_stick_nbytes(int ndim, const int64_t* host_sizes,
                         const int32_t* dim_order, int elem_bytes);

/* src (strided host-order tensor, element strides host_strides) ->
 * dst (stick layout, dst_nbytes = sph_stick_nbytes(...)).  Bit-exact. */
int sph_stick_pack(const void* src, void* dst, int ndim,
                   const int64_t* host_sizes, const int64_t* host_strides,
                   const int32_t* dim_order, int elem_bytes,
                   sph_stream_t stream);

/* Inverse of sph_stick_pack: stick layout -> strided host-order tensor. */
int sph_stick_unpack(const void* src, void* dst, int ndim,
                     const int64_t* host_sizes, const int64_t* host_strides,
                     const int32_t* dim_order, int elem_bytes,
                     sph_stream_t stream);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* SPYRE_HIP_H_ */
