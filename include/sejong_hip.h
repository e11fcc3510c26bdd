/*
 * sejong_hip.h -- C ABI of the MI355X (gfx950) kernels for Sejong's byte /
 * NativeValue Transformer training step.
 *
 * This library replaces the Triton launcher behind crates/sejong-gpu's
 * `Engine` (crates/sejong-gpu/src/lib.rs:366-487): each `Engine` op method
 * that today calls `self.launch("<triton op>", ...)` calls the function
 * declared here instead.  The citation above each declaration names the
 * reference method (and Triton kernel) it replaces.
 *
 * Conventions
 *  - Every function returns an int status: SJ_OK (0) or one of SJ_ERR_*.
 *    sj_last_error() returns the message of the last failure on the calling
 *    thread (the reference's Error::Message / Error::Capacity text).
 *  - `stream` is a hipStream_t passed as void*; NULL is the null stream.
 *    All launches are asynchronous on it; nothing here synchronises unless
 *    its comment says so (the model calls that read results back).
 *  - All pointers are caller-owned device pointers, row-major 2-D with an
 *    explicit leading dimension (`ld*`, in elements).  No call allocates
 *    device memory except sj_alloc and sj_model_create.  Calls that need
 *    scratch take a `workspace` pointer sized by the matching
 *    *_workspace_bytes query.
 *  - dtypes use the reference's DType order (crates/sejong-core/src/lib.rs:
 *    34-41) plus bf16: SJ_F32=0, SJ_F64=1, SJ_F16=2, SJ_I32=3, SJ_BF16=4.
 *    The kernels compute in fp32 (FP64 for norms and loss sums, as the
 *    reference does) and accept SJ_F32 or SJ_BF16 storage.
 *  - Calls on one stream are not re-entrant (the reference Engine is a
 *    single-thread, single-stream object: hip.rs:114-124).
 */
#ifndef SEJONG_HIP_H
#define SEJONG_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SJ_OK 0
#define SJ_ERR_INVALID 1     /* shape / argument error (Error::Message)     */
#define SJ_ERR_CAPACITY 2    /* memory or shared-memory budget (Error::Capacity) */
#define SJ_ERR_HIP 3         /* HIP runtime error (hip.rs:47-57)             */
#define SJ_ERR_UNSUPPORTED 4 /* dtype / layout combination not implemented  */
#define SJ_ERR_NONFINITE 5   /* non-finite clipping gradient (train lib.rs:210) */
#define SJ_ERR_IO 6          /* file read / write (Error::Io)               */

#define SJ_F32 0
#define SJ_F64 1
#define SJ_F16 2
#define SJ_I32 3
#define SJ_BF16 4

const char *sj_status_string(int status);
const char *sj_last_error(void);
/* Library / device identification: writes the gfx arch name (e.g. "gfx950")
 * and CU count of the current device. */
int sj_device_info(char *arch, size_t arch_len, int *compute_units);

/* Device memory, transfers and timing for callers without their own HIP
 * allocator (the reference Engine's empty / from_f32 / to_f32, crates/
 * sejong-gpu/src/lib.rs:234-365, and EventPair timing, hip.rs:59-112).
 * Transfers are synchronous; sj_event_elapsed waits for `end`. */
int sj_alloc(size_t bytes, void **ptr);
int sj_free(void *ptr);
/* Engine::available_memory_bytes (crates/sejong-gpu/src/lib.rs:243-245,
 * hip.rs:154): free and total device memory of the current device. */
int sj_memory_info(size_t *free_bytes, size_t *total_bytes);
int sj_upload(void *dst, const void *src, size_t bytes);
int sj_download(void *dst, const void *src, size_t bytes);
int sj_synchronize(void *stream);
int sj_event_create(void **ev);
int sj_event_destroy(void *ev);
int sj_event_record(void *ev, void *stream);
int sj_event_elapsed(void *start, void *end, float *ms);

/* ---------------------------------------------------------- elementwise */

/* Engine::full, crates/sejong-gpu/src/lib.rs:544-553 (kernel `fill`,
 * python/sejong_kernels/ops/kernels.py:6-9). */
int sj_fill(void *stream, void *y, int dtype, long n, float value);
/* Engine::cast / copy_into, lib.rs:554-571 (kernel `copy`, kernels.py:11-14).
 * Same dtype: a bit copy (16-byte vectors when both pointers are aligned);
 * fp32 -> bf16 rounds to nearest even. */
int sj_cast(void *stream, const void *x, int x_dtype, void *y, int y_dtype, long n);
/* Engine::add / add_into, lib.rs:572-593 (kernel `add`, kernels.py:16-21):
 * y = x + alpha*z computed in fp32, stored in y_dtype. */
int sj_add(void *stream, const void *x, int x_dtype, const void *z, int z_dtype,
           void *y, int y_dtype, long n, float alpha);

/* Engine::embedding, lib.rs:650-666 (kernels.py:41-45): Y[i] = W[ids[i]]. */
int sj_embedding_fwd(void *stream, const void *w, int w_dtype, const int32_t *ids,
                     void *y, int y_dtype, long n, long d);
/* Engine::embedding_backward, lib.rs:667-687 (kernels.py:47-52):
 * dW[v] = sum_{i: ids[i]=v} dY[i], written (not accumulated) over all V rows.
 * Deterministic: rows are summed in token order (the reference uses fp32
 * atomics).  Needs sj_embedding_bwd_workspace_bytes of scratch. */
size_t sj_embedding_bwd_workspace_bytes(long n, long vocab);
int sj_embedding_bwd(void *stream, const float *dy, const int32_t *ids, float *dw,
                     long n, long d, long vocab, void *workspace, size_t workspace_bytes);

/* Engine::rope, lib.rs:734-758 (kernels.py:103-113): interleaved pairs,
 * pos = (row / heads) mod t + offset (rows of width heads*head_dim, so row =
 * token index), inverse != 0 negates the sine (backward, graph.rs:879-882). */
int sj_rope(void *stream, const void *x, void *y, int dtype, long rows, long ld,
            long t, long heads, long head_dim, long offset, float theta, int inverse);
/* cos/sin table [t][head_dim/2] (interleaved cos, sin; angles formed in
 * double) consumed by the fused RoPE epilogues of sj_qkv_fwd and
 * sj_attention_bwd. */
int sj_rope_table(void *stream, float *table, long t, long head_dim, float theta);

/* Engine::swiglu / swiglu_backward, lib.rs:700-733 (kernels.py:90-101). */
int sj_swiglu_fwd(void *stream, const void *g, const void *u, void *h, int dtype, long n);
int sj_swiglu_bwd(void *stream, const void *g, const void *u, int gu_dtype,
                  const float *dy, float *dg, float *du, long n);

/* -------------------------------------------------------------- RMSNorm */

/* Engine::norm, lib.rs:688-699 (kernel `rmsnorm`, kernels.py:54-61):
 * y = x * (1/sqrt(mean x^2 + eps)) * w, stored in x's dtype. */
int sj_rmsnorm_fwd(void *stream, const void *x, int x_dtype, const void *w, int w_dtype,
                   void *y, long rows, long d, float eps);
/* Engine::norm_backward, crates/sejong-gpu/src/norm_ops.rs:14-71 (kernels
 * rmsnorm_backward_partial / _reduce, kernels.py:63-87):
 * dx = s*(dy*w - x*mean(dy*w*x)*s^2) [+ dx_acc], dw = sum_rows dy*x*s with
 * s = rsqrt(mean x^2 + eps).  dx_acc (nullable) fuses the tape's fp32
 * gradient accumulation (graph.rs:503-513).  dw is written, reduced
 * deterministically through `workspace` (sj_rmsnorm_bwd_workspace_bytes). */
size_t sj_rmsnorm_bwd_workspace_bytes(long rows, long d);
int sj_rmsnorm_bwd(void *stream, const void *x, int x_dtype, const void *w, int w_dtype,
                   const float *dy, const float *dx_acc, float *dx, float *dw,
                   long rows, long d, float eps, void *workspace, size_t workspace_bytes);
/* MFMA-layout forms used by the bf16 step (same formulas as above, bf16 x
 * and w): the forward also writes y transposed, y_t [d][ldt] (the A operand
 * of the dW GEMMs); the backward (d <= 1024) also writes dx as hi/lo bf16
 * planes, normal [rows][d] and transposed [d][ldt] (dX / dW GEMM operands
 * of the layer below; each pair optional: both pointers or neither).
 * Workspace: sj_rmsnorm_bwd_p_workspace_bytes. */
int sj_rmsnorm_fwd_t(void *stream, const uint16_t *x, const uint16_t *w, uint16_t *y, uint16_t *y_t,
                     long ldt, long rows, long d, float eps);
size_t sj_rmsnorm_bwd_p_workspace_bytes(long rows, long d);
int sj_rmsnorm_bwd_p(void *stream, const uint16_t *x, const uint16_t *w, const float *dy,
                     const float *dx_acc, float *dx, float *dw, uint16_t *dx_hi, uint16_t *dx_lo,
                     uint16_t *dx_t_hi, uint16_t *dx_t_lo, long ldt, long rows, long d, float eps,
                     void *workspace, size_t workspace_bytes);
/* No counterpart in the reference.  sj_rmsnorm_bwd_p without a workspace,
 * for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc): the dw
 * partials live in a file-scope device array of
 * SJ_RMSNORM_BWD_NOALLOC_MAX_BYTES per GPU, held until the process ends.
 * Shapes whose partials (ceil(rows / 16) * d * 4 bytes) exceed it return
 * SJ_ERR_CAPACITY.  The call allocates nothing (no hipMalloc / hipFree);
 * results are bit-identical to sj_rmsnorm_bwd_p.  All calls on one GPU
 * share that GPU's array: calls that overlap on one GPU (two streams, two
 * threads) race. */
#define SJ_RMSNORM_BWD_NOALLOC_MAX_BYTES (4u << 20)
int sj_rmsnorm_bwd_p_noalloc(void *stream, const uint16_t *x, const uint16_t *w, const float *dy,
                             const float *dx_acc, float *dx, float *dw, uint16_t *dx_hi, uint16_t *dx_lo,
                             uint16_t *dx_t_hi, uint16_t *dx_t_lo, long ldt, long rows, long d, float eps);

/* ----------------------------------------------------------------- GEMM */

/* Engine::matmul, lib.rs:594-649 (kernel `matmul`, kernels.py:23-39):
 * C[M,N] (+)= op(A)[M,K] * op(B)[K,N].  ta: A stored [K,M]; tb: B stored
 * [N,K].  A/B in SJ_F32 or SJ_BF16, C in SJ_F32 or SJ_BF16, fp32
 * accumulation on bf16 MFMA.  fp32 operands are fed as hi+lo bf16 pairs
 * (error ~2^-16 relative, the reference's fp32 "ieee" dot for dY operands).
 * accumulate != 0 adds into C (fp32 C only).  workspace: split-K partials,
 * sized by sj_gemm_workspace_bytes (0 is valid: no split-K). */
size_t sj_gemm_workspace_bytes(long M, long N, long K);
int sj_gemm(void *stream, int ta, int tb, long M, long N, long K,
            const void *a, int a_dtype, long lda, const void *b, int b_dtype, long ldb,
            void *c, int c_dtype, long ldc, int accumulate,
            void *workspace, size_t workspace_bytes);

/* Engine::project_qkv, crates/sejong-gpu/src/projection_ops.rs:6-43 (kernel
 * projection_qkv, python/sejong_kernels/ops/projection.py:6-44): one launch
 * computes Q = X Wq [M,N], K = X Wk and V = X Wv [M,KV], stored in x dtype.
 * With rope_table non-null (sj_rope_table of rope_t positions) the RoPE of
 * Engine::rope (rounded value in, fp32 math, stored again) is applied to the
 * head_dim-wide heads of Q and K in the epilogue, replacing the two rope
 * launches of Block::apply (crates/sejong-model/src/architecture.rs:215-216).
 * N and KV must be multiples of 64. */
int sj_qkv_fwd(void *stream, const void *x, long ldx, long M, long D,
               const void *wq, long ldwq, const void *wk, long ldwk, const void *wv, long ldwv,
               long N, long KV, void *q, long ldq, void *k, long ldk, void *v, long ldv,
               int dtype, const float *rope_table, long rope_t, long head_dim);

/* Engine::gate_up, projection_ops.rs:45-79 (kernel projection_gate_up,
 * projection.py:47-73): G = X Wg, U = X Wu rounded to the storage dtype,
 * H = g*sigmoid(g)*u from the rounded values. */
int sj_gate_up_fwd(void *stream, const void *x, long ldx, long M, long D,
                   const void *wg, long ldwg, const void *wu, long ldwu, long F,
                   void *g, void *u, void *h, long ldo, int dtype);

/* Residual projection: Y = R + round(X W), the `matmul` + `add` pair of
 * Block::apply (architecture.rs:226-227 and :245) fused in one epilogue
 * with the reference's two roundings (matmul output, then the sum). */
int sj_linear_residual_fwd(void *stream, const void *x, long ldx, long M, long K,
                           const void *w, long ldw, long N, const void *r, long ldr,
                           void *y, long ldy, int dtype);

/* dX of the gate/up pair fused with Engine::swiglu_backward (lib.rs:711-733):
 * dH = dY W_down^T (fp32) is never stored; the epilogue writes
 * dG = dH*u*s*(1+g(1-s)), dU = dH*g*s (s = sigmoid(g)) into dgu[:, 0:F] and
 * dgu[:, F:2F]. */
int sj_down_bwd_swiglu(void *stream, const float *dy, long lddy, long M, long D,
                       const void *w_down, long ldw, long F, const void *g, const void *u,
                       long ldgu_in, int gu_dtype, float *dgu, long lddgu);

/* ---------------------------------------------- MFMA-layout GEMM family
 * The same ops with every operand in the layout the MFMA streams: bf16
 * planes stored k-contiguous ([rows][K], leading dimension a multiple of 8,
 * 16-byte aligned).  An fp32 operand is passed as two planes hi = RNE(x),
 * lo = RNE(x - hi) (products hi*hi + hi*lo + lo*hi); a weight used as B in
 * the forward is passed transposed ([N][K]).  Tiles are streamed
 * global -> LDS with global_load_lds_dwordx4, three stages deep.  These are
 * what the step driver calls; the entries above keep the reference layouts.
 *
 * C[M,N] (+)= A B with A planes [M][K] (a_lo nullable) and B planes [N][K]
 * (b_lo nullable; with both split the products are hi*hi + hi*lo + lo*hi).
 * Split-K through `workspace`
 * (sj_gemm_planes_workspace_bytes) with a fixed-order reduction. */
size_t sj_gemm_planes_workspace_bytes(long M, long N, long K);
int sj_gemm_planes(void *stream, long M, long N, long K, const uint16_t *a_hi, const uint16_t *a_lo,
                   long lda, const uint16_t *b_hi, const uint16_t *b_lo, long ldb, void *c, int c_dtype,
                   long ldc, int accumulate, void *workspace, size_t workspace_bytes);
/* dW = X^T dY of a projection (graph.rs:829-851) from row-layout operands:
 * c [M][ldc] (+)= x^T y with x [K][ldx] (M columns, e.g. the layer input
 * [tokens][d]) and y [K][ldy] (N columns, e.g. dY as hi/lo planes
 * [tokens][n]); the tiles are staged in that orientation and the MFMA reads
 * their transposed fragments from LDS.  M, N, ldx, ldy multiples of 8;
 * workspace sj_gemm_planes_workspace_bytes(M, N, K). */
int sj_gemm_planes_tn(void *stream, long M, long N, long K, const uint16_t *x_hi, const uint16_t *x_lo, long ldx,
                      const uint16_t *y_hi, const uint16_t *y_lo, long ldy, void *c, int c_dtype, long ldc,
                      int accumulate, void *workspace, size_t workspace_bytes);
/* dX = dY W^T of a projection (graph.rs:829-851) with dY as hi/lo planes
 * [M][K] and W^T [N][K] bf16, its fp32 result written as hi/lo planes
 * c [M][ldc] (the dO operands of the attention backward) and, when c_t_hi
 * and c_t_lo are non-null, also transposed c_t [N][ldct] (ldct >= M,
 * multiple of 8).  With delta_t non-null (the attention output's dX), also
 * the attention backward's Delta (hierarchy.py:42-70): delta_t [N/64][ld]
 * = per row and 64-column head, the sum of the stored planes times
 * o [M][ldo]. */
int sj_gemm_planes_split_out(void *stream, long M, long N, long K, const uint16_t *a_hi, const uint16_t *a_lo,
                             long lda, const uint16_t *b, long ldb, uint16_t *c_hi, uint16_t *c_lo, long ldc,
                             uint16_t *c_t_hi, uint16_t *c_t_lo, long ldct, const uint16_t *o, long ldo,
                             float *delta_t, long ld_delta);
/* Engine::project_qkv (projection_ops.rs:6-43) + fused RoPE with the weights
 * transposed in one [N+2KV][D] buffer (query rows, then key, then value);
 * output one [M][N+2KV] bf16 buffer (q | k | v columns) and, when qkv_t is
 * not NULL, the same values transposed [N+2KV][ldqt] (ldqt >= M, multiple
 * of 8). */
int sj_qkv_fwd_t(void *stream, const uint16_t *x, long ldx, long M, long D, const uint16_t *wqkv_t,
                 long ldw, long N, long KV, uint16_t *qkv, long ldo, const float *rope_table, long rope_t,
                 long head_dim, uint16_t *qkv_t, long ldqt);
/* Engine::gate_up (projection_ops.rs:45-79) with transposed weights
 * ([F][D] each); h_t (nullable) receives h transposed [F][M] (the A operand
 * of the down projection's dW). */
int sj_gate_up_fwd_t(void *stream, const uint16_t *x, long ldx, long M, long D, const uint16_t *wg_t,
                     const uint16_t *wu_t, long ldw, long F, uint16_t *g, uint16_t *u, uint16_t *h, long ldo,
                     uint16_t *h_t, long ldht);
/* matmul + residual add (architecture.rs:226-227, :245) with W^T [N][K]. */
int sj_linear_residual_fwd_t(void *stream, const uint16_t *x, long ldx, long M, long K, const uint16_t *w_t,
                             long ldw, long N, const uint16_t *r, long ldr, uint16_t *y, long ldy);
/* Down-projection dX fused with Engine::swiglu_backward (lib.rs:711-733):
 * dY as planes [M][D], W_down [F][D] (its natural layout is k-contiguous
 * here); writes dG|dU as hi/lo planes [M][2F] and transposed [2F][M]. */
int sj_down_bwd_swiglu_p(void *stream, const uint16_t *dy_hi, const uint16_t *dy_lo, long lddy, long M,
                         long D, const uint16_t *w_down, long ldw, long F, const uint16_t *g,
                         const uint16_t *u, long ldgu, uint16_t *dgu_hi, uint16_t *dgu_lo, long lddgu,
                         uint16_t *dgu_t_hi, uint16_t *dgu_t_lo, long lddgu_t);

/* ------------------------------------------------------------ Attention */

/* Engine::attention_grouped, crates/sejong-gpu/src/hierarchy_ops.rs:10-72
 * (kernel hierarchy_attention, python/sejong_kernels/ops/hierarchy.py:7-39):
 * causal GQA attention (kv head = h / (HQ/HK)), scale head_dim^-1/2,
 * window 0 = full causal.  O stored in the q dtype, LSE fp32 [B*T*HQ].
 * Training shape (tq = tk = t, offset 0). */
int sj_attention_fwd(void *stream, const void *q, long ldq, const void *k, long ldk,
                     const void *v, long ldv, void *o, long ldo, float *lse, int dtype,
                     long batch, long t, long hq, long hk, long head_dim, long window);
/* Engine::attention_grouped_backward, hierarchy_ops.rs:74-147 (kernels
 * hierarchy_attention_dq, which writes Delta = sum dO*O, and
 * hierarchy_attention_dkv, which reads it and loops the group's query
 * heads: hierarchy.py:42-104).  dQ/dK/dV fp32.  With rope_table non-null
 * (sj_rope_table) the inverse RoPE (rope backward, graph.rs:879-882) is
 * applied to dQ and dK before they are stored.  delta: fp32 [B*T*HQ]
 * scratch/output (Delta of each query row). */
/* Engine::attention_grouped with an offset (hierarchy_ops.rs:10-70, kernel
 * hierarchy_attention hierarchy.py:7-39 with OFFSET) as the KV-cache path
 * calls it (architecture.rs:483-497): tq query rows q [tq][ldq] of one
 * sequence at positions offset .. offset+tq-1 against the keys and values of
 * positions 0 .. offset+tq-1, k / v [capacity][ldkv]; causal, optional
 * window.  A row is computed with the operations of the full forward
 * (sj_attention_fwd_tt for bf16 head_dim 64, the row kernel otherwise), so
 * cached and full outputs agree bit for bit.  No LSE (inference). */
int sj_attention_fwd_cached(void *stream, const void *q, long ldq, const void *k, const void *v, long ldkv,
                            long capacity, int dtype, long tq, long offset, long hq, long hk, long head_dim,
                            long window, void *o, long ldo);
int sj_attention_bwd(void *stream, const void *q, long ldq, const void *k, long ldk,
                     const void *v, long ldv, const void *o, long ldo, const float *lse,
                     const float *dout, long lddo, float *dq, long lddq, float *dk, long lddk,
                     float *dv, long lddv, float *delta, int dtype, long batch, long t,
                     long hq, long hk, long head_dim, long window, const float *rope_table);
/* MFMA-layout forms (bf16, head_dim 64, full causal).  sj_attention_fwd_t
 * also writes O transposed, o_t [hq*64][ldot].  sj_attention_bwd_p writes
 * dQ|dK|dV (inverse RoPE applied to dQ, dK) as hi/lo bf16 planes: normal
 * g [B*T][ldg] with dQ in columns [0, hq*64), dK then dV after it, and
 * transposed g_t [(hq+2hk)*64][ldgt] -- the operands of the QKV
 * projection's dX and dW GEMMs.  Both need t % 4 == 0 when batch > 1;
 * ldot a multiple of 4, ldgt of 8.  The backward sums dK / dV over the
 * group's query heads through `workspace`
 * (sj_attention_bwd_p_workspace_bytes) in a fixed order. */
int sj_attention_fwd_t(void *stream, const uint16_t *q, long ldq, const uint16_t *k, long ldk,
                       const uint16_t *v, long ldv, uint16_t *o, long ldo, float *lse, uint16_t *o_t,
                       long ldot, long batch, long t, long hq, long hk, long head_dim);
int sj_attention_bwd_p(void *stream, const uint16_t *q, long ldq, const uint16_t *k, long ldk,
                       const uint16_t *v, long ldv, const uint16_t *o, long ldo, const float *lse,
                       const float *dout, long lddo, float *delta, long batch, long t, long hq, long hk,
                       long head_dim, const float *rope_table, uint16_t *g_hi, uint16_t *g_lo, long ldg,
                       uint16_t *g_t_hi, uint16_t *g_t_lo, long ldgt, void *workspace, size_t workspace_bytes);
size_t sj_attention_bwd_p_workspace_bytes(long batch, long t, long hq, long hk, long head_dim);

/* ------------------------------------------- Hierarchical model patches
 * The byte <-> patch maps of the hierarchical (cfg3) model (hidden_from_
 * encoded, architecture.rs:368-393).  x, y, bos in the compute dtype (SJ_F32
 * or SJ_BF16), gradients fp32; sums are formed in the reference's order. */
/* Engine::patch_pool, hierarchy_ops.rs:149-169 (kernel hierarchy_patch_pool,
 * hierarchy.py:107-119): y [batch*ceil(t/patch)][d] = mean of each patch's
 * positions (the last patch of a sequence may be partial and divides by its
 * own count). */
int sj_patch_pool(void *stream, const void *x, int dtype, long batch, long t, long d, long patch, void *y);
/* Engine::patch_pool_backward, hierarchy_ops.rs:171-204
 * (hierarchy.py:122-131): dx [batch*t][d] = dy[patch of the position] /
 * count. */
int sj_patch_pool_bwd(void *stream, const float *dy, long batch, long t, long d, long patch, float *dx);
/* Engine::patch_broadcast, hierarchy_ops.rs:206-236 (hierarchy.py:134-143):
 * y [batch*t][d] = x row of the previous patch (positions of patch p see
 * patch p-1), bos [d] for the first patch. */
int sj_patch_broadcast(void *stream, const void *x, const void *bos, int dtype, long batch, long t, long d,
                       long patch, void *y);
/* Engine::patch_broadcast_backward, hierarchy_ops.rs:238-276
 * (hierarchy.py:146-172): dx [batch*ceil(t/patch)][d] = sum of dy over the
 * next patch's positions; dbos [d] = sum over batches of the first patch's
 * positions. */
int sj_patch_broadcast_bwd(void *stream, const float *dy, long batch, long t, long d, long patch, float *dx,
                           float *dbos);

/* The step's attention in MFMA layout (bf16, head_dim 64, t a multiple of
 * 64; window as sj_attention_fwd: a query sees the `window` last positions
 * up to itself, 0 = all): qkv [batch*t][ldqkv] (q | k | v columns, q and k
 * after RoPE; sj_qkv_fwd_t's output).  Forward = hierarchy_attention
 * (hierarchy.py:7-39): o [rows][ldo], lse [rows][hq] (nullable, the
 * reference layout) and lse_t [hq][ldt], o_t [hq*64][ldot] (nullable).
 * Backward = hierarchy_attention_dq + _dkv (hierarchy.py:42-104) from dO
 * as hi/lo planes [rows][lddo] (sj_gemm_planes_split_out), writing Delta
 * into delta_t [hq][ldt] and dQ | dK | dV (inverse RoPE on dQ, dK) as hi/lo
 * planes like sj_attention_bwd_p; workspace
 * sj_attention_bwd_tt_workspace_bytes.  ldt >= batch*t, a multiple of 8. */
int sj_attention_fwd_tt(void *stream, const uint16_t *qkv, long ldqkv, long ldt, long batch, long t, long hq,
                        long hk, long head_dim, long window, uint16_t *o, long ldo, float *lse, float *lse_t,
                        uint16_t *o_t, long ldot);
size_t sj_attention_bwd_tt_workspace_bytes(long batch, long t, long hq, long hk, long head_dim);
/* The workspace ends with the meeting counters of the grouped launch's cut
 * walks (the last sj_attention_bwd_tt_counter_bytes(batch, hk) bytes of the
 * size above; no counterpart in the reference, whose backward does not cut
 * walks): they must be zero before the first call on a workspace (clear them
 * when it is allocated) and nothing else may write them between calls;
 * every call leaves them zero.  Calls that share a workspace must not
 * overlap (as for any workspace); calls on different workspaces never share
 * counters. */
size_t sj_attention_bwd_tt_counter_bytes(long batch, long hk);
int sj_attention_bwd_tt(void *stream, const uint16_t *qkv, long ldqkv, long ldt, const uint16_t *o, long ldo,
                        const float *lse_t, const uint16_t *do_hi, const uint16_t *do_lo, long lddo, float *delta_t,
                        long batch, long t, long hq, long hk, long head_dim, long window, const float *rope_table,
                        uint16_t *g_hi, uint16_t *g_lo, long ldg, uint16_t *g_t_hi, uint16_t *g_t_lo, long ldgt,
                        void *workspace, size_t workspace_bytes);
/* Inspection of sj_attention_bwd_tt's work split for three query heads per
 * KV head (no counterpart in the reference: the split is this library's
 * scheduling, exposed for its tests).  The causal walks (dQ of query block
 * qb over key blocks ..qb, dK | dV of key block kb over query blocks kb..)
 * longer than a cap per role are cut into parts of at most the cap (up to
 * four); every piece (whole walk or part) is one workgroup per (KV head,
 * sequence) pair, dispatched costliest first; the caps are those whose
 * simulated dispatch of `pairs` pairs on `cus` CUs finishes first.  Writes
 * one word per piece into seg (cap words at least): bit 31 set, bits 0-5
 * block, 6-11 / 12-17 first / last block of the walk it covers, bit 18 role
 * (0 dQ, 1 dK | dV), 19-26 cut-walk index + 1 (0: whole walk), 27-28 part,
 * 29-30 the walk's parts - 1; *ncut = cut walks per pair.  Returns the
 * number of pieces, or a negative status. */
int sj_attention_bwd_plan(long t, long window, long pairs, int cus, uint32_t *seg, long cap, int *ncut);

/* ---------------------------------------------------- Mixture of experts
 * The MoE FFN of Block::apply (crates/sejong-model/src/architecture.rs:
 * 229-242) without host synchronisation: experts <= 32, top_k <= 8.  The
 * packed layout groups the routed slots by expert (ascending slot order
 * inside an expert, the reference's pack order) in segments starting at
 * multiples of 64 rows: segment e is rows [offsets[e], offsets[e+1]) of a
 * [capacity][*] matrix, of which the first counts[e] are real and the rest
 * zero padding.  pslot[row] = routed slot (token*top_k + k) or -1;
 * ppos[slot] = its packed row. */

/* Engine::route_topk, crates/sejong-gpu/src/hierarchy_ops.rs:280-295 (kernel
 * hierarchy_route_topk, hierarchy.py:175-191): softmax of each row's
 * logits (fp32 math), top_k rounds of argmax with the lowest index on ties,
 * weight = the full-softmax probability.  ids i32 and weights fp32 [rows][top_k]. */
int sj_route_topk(void *stream, const void *logits, int dtype, long rows, long experts, long top_k,
                  int32_t *ids, float *weights);
/* Router projection (Linear::apply, architecture.rs:230: logits = z W_router
 * stored in z's dtype, bf16) fused with sj_route_topk; w_router [d][experts]. */
int sj_router_topk(void *stream, const uint16_t *z, long ldz, const uint16_t *w_router, long d, long rows,
                   long experts, long top_k, uint16_t *logits, int32_t *ids, float *weights);
/* Engine::route_topk_backward, hierarchy_ops.rs:297-329 (hierarchy.py:194-209):
 * dx = p * (dy_selected - sum_k w_k dy_k), fp32 [rows][experts]. */
int sj_route_topk_bwd(void *stream, const void *logits, int dtype, const int32_t *ids, const float *weights,
                      const float *dy, float *dx, long rows, long experts, long top_k);
/* Engine::expert_routes, hierarchy_ops.rs:331-378 (hierarchy_route_pack,
 * hierarchy.py:212-225) with the counts kept on the device: tokens/slots
 * (nullable) in the reference's [experts][rows*top_k] layout, counts
 * [experts], offsets [experts+1], pslot [capacity], ppos [rows*top_k].
 * capacity >= sj_route_pack_capacity(rows*top_k, experts). */
long sj_route_pack_capacity(long slots, long experts);
int sj_route_pack(void *stream, const int32_t *ids, long rows, long top_k, long experts, int32_t *tokens,
                  int32_t *slots, int32_t *counts, int32_t *offsets, int32_t *pslot, int32_t *ppos,
                  long capacity);
/* Engine::gather (crates/sejong-gpu/src/lib.rs:1010-1028) of every
 * expert's input rows in one pass: y [capacity][d] (bf16, zero padding
 * rows) and y_t (nullable) = y transposed [d][ldt] (the expert dW operand).
 * d <= 1024. */
int sj_moe_gather(void *stream, const uint16_t *x, long ldx, long d, const int32_t *pslot, long top_k,
                  long capacity, uint16_t *y, uint16_t *y_t, long ldt);
/* Engine::expert_combine, hierarchy_ops.rs:380-414 (hierarchy.py:228-235):
 * u[t] = bf16(sum over the token's experts, ascending, of w*y) with each
 * product rounded to fp32 before its add, then out = bf16(residual + u)
 * (the residual add of architecture.rs:245; residual nullable). */
int sj_moe_combine(void *stream, const uint16_t *yp, long ldy, long d, const int32_t *ids, const int32_t *ppos,
                   const float *weights, long rows, long top_k, const uint16_t *residual, long ldr,
                   uint16_t *out, long ldo);
/* Engine::expert_combine_backward, hierarchy_ops.rs:416-454
 * (hierarchy.py:238-251): dx[row] = dy[token] * w[slot] as hi/lo planes,
 * normal [capacity][d] and transposed [d][ldt] (nullable, both or neither),
 * and dweights[slot] = sum_c y[row][c] dy[token][c].  d <= 1024. */
int sj_moe_combine_bwd(void *stream, const uint16_t *yp, long ldy, long d, const int32_t *pslot,
                       const float *weights, long top_k, long capacity, const float *dy, long lddy,
                       uint16_t *dx_hi, uint16_t *dx_lo, uint16_t *dx_t_hi, uint16_t *dx_t_lo, long ldt,
                       float *dweights);
/* Engine::gather_backward (lib.rs:1030-1050) summed per token without
 * atomics (expert order ascending), fused with Engine::route_topk_backward
 * (when logits is non-null: dlogits fp32 [rows][experts]) and the router's
 * dX (dlogits W_router^T, when w_router is non-null) and the tape's
 * accumulation into dz_acc (nullable): dz = dz_acc + sum + router dX. */
int sj_moe_gather_bwd(void *stream, const float *dxp, long lddx, long d, const int32_t *ids, const int32_t *ppos,
                      const float *weights, const uint16_t *logits, const float *dweights,
                      const uint16_t *w_router, long rows, long top_k, long experts, const float *dz_acc,
                      long ldacc, float *dz, long lddz, float *dlogits);
/* Grouped expert GEMMs: the per-expert loop of architecture.rs:233-239 and
 * its backward (graph.rs:829-851) in one launch each, expert e's weights at
 * base + e*w_stride.  gate/up with transposed weights [F][D] per expert
 * (SwiGLU epilogue, h_t [F][ldht] nullable); down with W_down^T [D][F]
 * (bf16 output); down dX fused with the SwiGLU derivative (dY planes, W_down
 * [F][D], dG|dU planes normal and transposed); a row-grouped dX GEMM
 * C[capacity][N] = A B_e with B_e [N][K]; and per-expert dW
 * C_e[M][N] = A^T B over the expert's rows (A [M][capacity] bf16, B planes
 * [N][capacity]), C_e at c + e*c_stride. */
int sj_moe_gate_up_fwd(void *stream, const int32_t *offsets, long experts, long capacity, const uint16_t *x,
                       long ldx, long D, const uint16_t *wg_t, const uint16_t *wu_t, long ldw, long w_stride,
                       long F, uint16_t *g, uint16_t *u, uint16_t *h, long ldo, uint16_t *h_t, long ldht);
int sj_moe_down_fwd(void *stream, const int32_t *offsets, long experts, long capacity, const uint16_t *h,
                    long ldh, long F, const uint16_t *wd_t, long ldw, long w_stride, long D, uint16_t *y,
                    long ldy);
int sj_moe_down_bwd_swiglu_p(void *stream, const int32_t *offsets, long experts, long capacity,
                             const uint16_t *dy_hi, const uint16_t *dy_lo, long lddy, long D,
                             const uint16_t *w_down, long ldw, long w_stride, long F, const uint16_t *g,
                             const uint16_t *u, long ldgu, uint16_t *dgu_hi, uint16_t *dgu_lo, long lddgu,
                             uint16_t *dgu_t_hi, uint16_t *dgu_t_lo, long ldt);
int sj_moe_gemm_rows(void *stream, const int32_t *offsets, long experts, long capacity, long N, long K,
                     const uint16_t *a_hi, const uint16_t *a_lo, long lda, const uint16_t *b, long ldb,
                     long b_stride, float *c, long ldc, int accumulate);
/* The per-expert dW from row-layout operands (no transposed copies): C_e
 * (+ e*c_stride) [M][N] = X_e^T Y_e over expert e's packed rows, X
 * [capacity][ldx] (M columns: packed h or expert inputs), Y [capacity][ldy]
 * (N columns, hi/lo gradient planes).  M, N, ldx, ldy multiples of 8. */
int sj_moe_gemm_dw_tn(void *stream, const int32_t *offsets, long experts, long capacity, long M, long N,
                      const uint16_t *x, long ldx, const uint16_t *y_hi, const uint16_t *y_lo, long ldy, float *c,
                      long ldc, long c_stride);
int sj_moe_gemm_dw(void *stream, const int32_t *offsets, long experts, long capacity, long M, long N,
                   const uint16_t *a, long lda, const uint16_t *b_hi, const uint16_t *b_lo, long ldb, float *c,
                   long ldc, long c_stride);

/* ------------------------------------------------------- Parameter VJP
 * Forward-basis parameter VJP and factored selected-row SGD
 * (crates/sejong-gpu/src/parameter_vjp.rs, python/sejong_kernels/ops/
 * parameter.py).  For Y = X W with X [n tokens][a features]: a rank-R token
 * basis Q [n][R] from R donor columns, S selected feature blocks of
 * block_rows rows, and the weight gradient as left [a][R] x right [R][b]
 * plus the selected rows (tail [k][b], k = S*block_rows) placed by
 * row_map [a] (-1 = not selected). */

/* budget, parameter_vjp.rs:85-97: rank = min(rank, n, a, donor), blocks =
 * ceil(a / block_rows), selected = clamp(ceil(blocks * fraction), 1, blocks). */
int sj_pvjp_budget(long rank, double residual_fraction, long block_rows, long n, long a, long donor,
                   long *out_rank, long *out_blocks, long *out_selected);
/* selects_compression, parameter_vjp.rs:100-130 (the tile-padded cost
 * model, exact integer arithmetic): 1 when the factored form is cheaper. */
int sj_pvjp_selects_compression(long rank, double residual_fraction, long block_rows, long n, long a, long b,
                                long donor, long uses);
/* The CGS2 drop threshold of prepare_parameter_vjp_reusing,
 * parameter_vjp.rs:214-220 (f32). */
float sj_pvjp_basis_tolerance(long rows, long rank);
/* kernel parameter_indices (parameter.py:25-62), launched by
 * prepare_parameter_vjp_reusing (parameter_vjp.rs:181-207) with seed = one
 * Rng::next_u64 of the caller's stream: partial Fisher-Yates of `rank`
 * donor columns then `selected` feature blocks on one SplitMix64 stream.
 * scratch i32 [donor_width + feature_blocks]; columns [rank]; rows
 * [selected*block_rows] (-1 past a); map [a]. */
int sj_pvjp_indices(void *stream, uint64_t seed, long a, long donor_width, long feature_blocks, long selected,
                    long rank, long block_rows, int32_t *scratch, int32_t *columns, int32_t *rows,
                    int32_t *map);
/* kernels parameter_basis / parameter_basis_register (parameter.py:65-128):
 * Q fp32 [n][rank], an orthonormal basis of the picked donor columns (y
 * [n][ldy], f32 or bf16) in column order, a column zeroed when its residual
 * after the earlier columns has |v|^2 <= eps^2 |orig|^2.  Computed as
 * CholeskyQR2 (FP64 Gram, the Cholesky pivot is that residual norm); Q
 * spans the same space as the reference's CGS2.  rank <= 64.  Workspace:
 * sj_pvjp_basis_workspace_bytes. */
size_t sj_pvjp_basis_workspace_bytes(long n, long rank);
int sj_pvjp_basis(void *stream, const void *y, int dtype, long ldy, long n, const int32_t *columns, long rank,
                  float eps, float *q, void *workspace, size_t workspace_bytes);
/* kernels parameter_prepare / parameter_residual (parameter.py:131-190)
 * with X given transposed (x_t [a][ldxt] bf16, columns n .. n rounded up
 * to 8 zero): left = X^T Q fp32 [a][rank];
 * e (nullable) = [Q^T ; (X[:, row] - Q left[row]^T) * inverse] fp32
 * [rank+k][lde], and as hi/lo planes (zero rows for row = -1).  Workspace:
 * sj_pvjp_prepare_workspace_bytes. */
size_t sj_pvjp_prepare_workspace_bytes(long a, long n, long rank);
int sj_pvjp_prepare(void *stream, const uint16_t *x_t, long ldxt, long a, long n, const float *q, long rank,
                    const int32_t *rows, long k, float inverse, float *left, float *e, uint16_t *e_hi,
                    uint16_t *e_lo, long lde, void *workspace, size_t workspace_bytes);
/* The same with X in row layout, x [n][ldx] (the stored activation itself,
 * no transposed copy): n, a and the leading dimensions multiples of 8.
 * Workspace: sj_pvjp_prepare_workspace_bytes. */
int sj_pvjp_prepare_rows(void *stream, const uint16_t *x, long ldx, long a, long n, const float *q, long rank,
                         const int32_t *rows, long k, float inverse, float *left, float *e, uint16_t *e_hi,
                         uint16_t *e_lo, long lde, void *workspace, size_t workspace_bytes);
/* Engine::parameter_vjp, parameter_vjp.rs:308-320: coefficients = E dY
 * [rows][b] (right = rows 0..rank-1, tail = the rest) from the E planes and
 * dY^T planes [b][lddy] (columns past n zero).  Workspace:
 * sj_pvjp_vjp_workspace_bytes. */
size_t sj_pvjp_vjp_workspace_bytes(long rows, long b, long n);
int sj_pvjp_vjp(void *stream, const uint16_t *e_hi, const uint16_t *e_lo, long lde, long rows, long n,
                const uint16_t *dy_t_hi, const uint16_t *dy_t_lo, long lddy, long b, float *coefficients,
                long ldc, void *workspace, size_t workspace_bytes);
/* The same with dY in row layout, hi/lo planes [n][lddy] (the gradient
 * planes the dX products read): n and b multiples of 8.  Workspace:
 * sj_pvjp_vjp_workspace_bytes. */
int sj_pvjp_vjp_rows(void *stream, const uint16_t *e_hi, const uint16_t *e_lo, long lde, long rows, long n,
                     const uint16_t *dy_hi, const uint16_t *dy_lo, long lddy, long b, float *coefficients,
                     long ldc, void *workspace, size_t workspace_bytes);
/* GradientPlan (parameter_vjp.rs:329-530; kernels parameter.py:193-291):
 * per parameter W [rows][cols] fp32, G = dense (nullable) + sum over its
 * terms of scale * (left right + tail rows placed by row_map).  Terms of a
 * parameter are terms[term_begin .. term_begin+term_count).  decay != 0
 * marks ndim > 1 (weight decay applies).  ld: row stride of w, dense and
 * mirror (0 = cols; a parameter may be a column block of a wider arena
 * matrix).  mirror (nullable): receives bf16(W) after an update (the next
 * step's Model::bind cast, model lib.rs:214-219, fused). */
typedef struct {
  float *w;
  const float *dense;
  long rows, cols;
  int decay;
  long term_begin, term_count;
  long ld;
  uint16_t *mirror;
} sj_factored_param;
typedef struct {
  const float *left;     /* [rows][rank] */
  const float *right;    /* [rank][ld] */
  const float *tail;     /* [k][ld] */
  const int32_t *row_map; /* [rows] */
  long rank;
  float scale;
  long ld;               /* row stride of right and tail; 0 = the parameter's cols */
} sj_factored_term;
/* GradientPlan::new + pack on the host: fills `host_meta`
 * (sj_factored_meta_bytes) with the device table the caller uploads
 * (parameters, terms and the owner of every 32x256 tile), and the number
 * of tiles. */
size_t sj_factored_meta_bytes(const sj_factored_param *params, long nparams, long nterms);
int sj_factored_pack(const sj_factored_param *params, long nparams, const sj_factored_term *terms, long nterms,
                     void *host_meta, size_t bytes, long *tiles);
/* GradientPlan::tiles: action 0 materialize (G written into w), 1 update
 * W = W*(1 - decay [ndim>1]) - lr*G with lr = learning_rate*clipping and
 * decay = learning_rate*weight_decay (parameter_vjp.rs:502-518), 2 FP64
 * sum of G^2 per tile into partials [tiles] (GradientPlan::norm). */
int sj_factored_apply(void *stream, const void *meta, long tiles, int action, float lr, float decay,
                      double *partials);
/* Fixed-order FP64 sum (the host sum of GradientPlan::norm, on device). */
int sj_sum_f64(void *stream, const double *x, long n, double *out);

/* -------------------------------------------------------- Cross entropy */

/* Engine::cross_entropy + cross_entropy_backward, lib.rs:881-913 (kernels
 * cross_entropy / cross_entropy_backward, kernels.py:176-191) in one pass:
 * loss[r] = logsumexp(x_r) - x_r[t_r]; dx = (softmax - onehot) * dy_r with
 * dy_r = dy ? dy[r] : dy_scalar (the mean-CE seed scale/count of
 * Graph::backward, graph.rs:539-549).  dx may be NULL (forward only). */
int sj_cross_entropy(void *stream, const float *x, long ldx, const int32_t *targets,
                     float *loss, float *dx, long lddx, long rows, long vocab,
                     const float *dy, float dy_scalar);
/* Engine::gather, lib.rs:1010-1028 (kernel gather, kernels.py:241-245):
 * y [rows][d] = x[idx[r]] (row stride ldx) in y's dtype (a gather followed
 * by Graph::cast to F32 when yd = SJ_F32). */
int sj_gather_rows(void *stream, const void *x, int xd, long ldx, const int32_t *idx, long rows, long d, void *y,
                   int yd);
/* Engine::gather_backward, lib.rs:1029-1050: dx [n][d] (row stride ldx) =
 * 0, then dx[idx[r]] += dy[r] for r in order (fp32). */
int sj_gather_rows_bwd(void *stream, const float *dy, const int32_t *idx, long rows, long d, float *dx, long ldx,
                       long n);
/* Engine::bias_add / bias_reduce, common_ops.rs:46-77 (common.py:28-36):
 * y = x + bias (row-broadcast); y[c] = sum over rows, in order, of x[r][c]. */
int sj_bias_add(void *stream, const float *x, long ldx, const float *bias, float *y, long ldy, long rows, long d);
int sj_bias_reduce(void *stream, const float *x, long ldx, long rows, long d, float *y);
/* Engine::loss_summary, lib.rs:524-543 (kernels.py:254-262): out[slot] =
 * (sum_i loss[i] in FP64) * weight / n. */
int sj_loss_summary(void *stream, const float *loss, long n, double *out, long slot, float weight);

/* ------------------------------------------------------------ Optimizer */

/* Engine::gradient_norm, lib.rs:494-523 (kernel gradient_norm, kernels.py:
 * 265-287): out_sumsq[0] = sum g^2 in FP64, deterministic two-stage
 * reduction, result left on the device (no host sync). */
size_t sj_sum_squares_workspace_bytes(long n);
int sj_sum_squares(void *stream, const float *g, long n, double *out_sumsq,
                   void *workspace, size_t workspace_bytes);
/* Engine::adamw, lib.rs:925-957 (kernel adamw, kernels.py:193-202), one
 * tensor, host-computed scalars exactly as the reference passes them. */
int sj_adamw(void *stream, float *w, const float *g, float *m, float *v, long n,
             float lr, float beta1, float beta2, float eps, float decay,
             float inv_b1, float inv_b2, float scale);

/* Device-resident step scalars for the multi-tensor AdamW (no host sync:
 * the clip factor of Adam::update, crates/sejong-train/src/lib.rs:199-238,
 * is formed on the device from the FP64 squared norm). */
typedef struct {
  float lr, beta1, beta2, eps, weight_decay, inv_b1, inv_b2, clip_norm, loss_scale;
  int32_t clip_enabled;
} sj_adam_step;
/* Adam::update over one flat parameter arena: elements [0, n_nodecay) are
 * 1-D tensors (no decay), the rest decay (`p.value.shape.len() > 1`,
 * train lib.rs:234).  scale = clip/loss_scale with clip = clip_norm/norm
 * when clip_enabled and norm > clip_norm, norm = sqrt(*sumsq)/loss_scale.
 * A non-finite norm sets *status_flag = 1 and leaves w, m, v untouched.
 * w_mirror (nullable, bf16) receives the compute-precision copy of the
 * updated w (the next step's Model::bind cast, model lib.rs:214-219). */
int sj_adamw_multi(void *stream, float *w, const float *g, float *m, float *v,
                   uint16_t *w_mirror, long n, long n_nodecay, const sj_adam_step *step,
                   const double *sumsq, int32_t *status_flag);

/* ---------------------------------------------------------------- Model
 *
 * Step driver for the dense byte Transformer (cfg1 / cfg2 family): the
 * per-step op sequence of train_configured (crates/sejong-train/src/lib.rs:
 * 387-453) -- Model::bind / logits (model lib.rs:206-340, Block::apply
 * architecture.rs:200-247), cross_entropy, Graph::backward (graph.rs:
 * 533-913), Adam::update -- issued on one stream over a preallocated
 * activation-retention arena, optionally replayed as a hipGraph.
 * Parameters are exchanged in the reference layout (architecture.rs:63-137,
 * names from sj_model_param_info); the device keeps fused internal copies.
 */
typedef struct sj_model sj_model;
typedef struct {
  long vocab;      /* 257 (core lib.rs:305)                 */
  long width;      /* d_model                                */
  long layers;
  long heads;      /* query heads                            */
  long kv_heads;
  long ffn_width;
  long sequence;   /* T                                      */
  long batch;      /* B                                      */
  float norm_epsilon;
  float rope_theta;
  int precision;   /* SJ_F32 or SJ_BF16 compute/storage dtype */
} sj_model_config;
typedef struct {
  float beta1, beta2, epsilon, weight_decay, clip_norm, loss_scale;
  int clip_enabled;
} sj_adam_config;

int sj_model_create(const sj_model_config *cfg, const sj_adam_config *adam, void *stream,
                    sj_model **out);
/* The hierarchical byte model (ModelConfig::hierarchy, core lib.rs:83-98;
 * architecture.rs:96-137 and 317-393): byte embedding [vocab][encoder
 * width] -> encoder blocks (local window) -> encoder_norm -> patch mean
 * pool (patch_size bytes) -> encoder_to_global -> cfg's blocks over
 * ceil(sequence / patch_size) patches -> global_norm -> global_to_decoder,
 * shifted by one patch behind global_bos's row (patch_broadcast) and added
 * to encoder_to_decoder of the encoded bytes -> decoder blocks (local
 * window) -> decoder_norm -> output_projection -> final_norm -> fp32 head.
 * cfg describes the global stage (width, layers, heads, kv_heads,
 * ffn_width) and the byte sequence; the local stages use heads = kv_heads.
 * Parameters in the reference layout order (sj_model_param_info);
 * input_projection (used only by injected inputs) keeps a zero gradient.
 * AdamW only.  sj_model_export_activations packs, per stage, the per-layer
 * activations, the stage's last residual and its closing-norm output, then
 * the pooled patches, global_to_decoder's output, the projected BOS row,
 * the broadcast rows, encoder_to_decoder's output, output_projection's
 * output and the final-norm output, then the logits. */
/* The MoE byte Transformer (ModelConfig::experts, core lib.rs:100-106;
 * Block::apply's MoE branch, architecture.rs:229-242): every block's FFN is
 * count SwiGLU experts of ffn_width behind a router [d][count] with top_k
 * routing (cfg's ffn_width is unused).  Parameters per layer in
 * stage_layout order: the norms and attention matrices, experts.<e>.gate /
 * up / down for every expert, then router.  bf16 with 64-wide heads (the
 * MFMA-layout step), experts <= 32, top_k <= 8, width <= 1024; AdamW.  The
 * activation pack replaces a layer's g, u, h by its router logits
 * [rows][count]. */
typedef struct {
  long count, top_k, ffn_width;
} sj_expert_config;
int sj_model_create_experts(const sj_model_config *cfg, const sj_expert_config *experts, const sj_adam_config *adam,
                            void *stream, sj_model **out);
typedef struct {
  long patch_size;
  long encoder_width, encoder_layers, encoder_heads, encoder_ffn_width;
  long decoder_width, decoder_layers, decoder_heads, decoder_ffn_width;
  long local_window; /* a byte sees the local_window last positions up to itself */
} sj_hierarchy_config;
int sj_model_create_hierarchy(const sj_model_config *cfg, const sj_hierarchy_config *hierarchy,
                              const sj_adam_config *adam, void *stream, sj_model **out);
/* SGD step driver (control_variate.rs:503-877 with accumulation 1 and no
 * control-variate blocks): forward, backward, FP64 norm of the compact
 * gradients and clip, GradientPlan::update W = W (1 - lr wd [ndim>1]) -
 * lr clip G.  vjp_rank > 0 turns on the parameter VJP
 * (ParameterVjpConfig, core lib.rs:447-466): Matmul nodes that share an
 * input with at least as many rows as columns form groups (graph.rs:
 * 551-566); a group's members that pass selects_compression get factored
 * gradients from one forward basis per (tokens, rank) and one feature
 * selection per width (graph.rs:915-1005), drawn with one next_u64 of the
 * parameter RNG (Rng::new(vjp_seed), carried across steps).  bf16 models
 * with 64-wide heads only.  loss_scale must be 1. */
typedef struct {
  float weight_decay, clip_norm, loss_scale;
  int clip_enabled;
  long vjp_rank;                /* 0: dense SGD */
  double vjp_residual_fraction;
  long vjp_block_rows;
  uint64_t vjp_seed;
} sj_sgd_config;
int sj_model_create_sgd(const sj_model_config *cfg, const sj_sgd_config *sgd, void *stream, sj_model **out);
/* NativeValue (crates/sejong-model/src/native/value.rs:111-160, trained
 * by train_value, crates/sejong-train/src/memory.rs:799-1065): the body
 * (cfg's blocks and final norm) under its own byte embedding [259][d]
 * (pad 256, BOS 257, SEP 258), the SEP row of each of the batch requests
 * gathered, cast to F32 and mapped by an affine head [d][values] + bias
 * [1][values]; loss = mean cross entropy of the value labels.  Parameters
 * in NativeValue::parameters order (the body without embedding and output,
 * then native_embedding, native_value, native_bias).  Exactly one of adam
 * / sgd.  cfg->sequence is the padded request length (>= the longest
 * prompt + 2: trailing pad bytes do not reach the causal SEP row). */
int sj_model_create_value(const sj_model_config *cfg, long values, const sj_adam_config *adam,
                          const sj_sgd_config *sgd, void *stream, sj_model **out);
/* One packed request batch: ids [batch*sequence] (row r = BOS, prompt,
 * SEP, pad), positions [batch] (the SEP index of row r, inside row r),
 * labels [batch].  Synchronous. */
int sj_model_set_value_batch(sj_model *m, const int32_t *ids, const int32_t *positions, const int32_t *labels);
/* GradientPlan::materialize for every parameter of an SGD model: the
 * gradient arena receives dense + factored G of the last backward (so
 * sj_model_get_grads returns it).  No-op for AdamW models. */
int sj_model_materialize_grads(sj_model *m);
/* VjpStatistics of one step (compressed / dense matrices, basis and
 * projection groups; control_variate.rs:577-578) and the parameter RNG
 * state (saved as sgd.parameter_rng, control_variate.rs:216-217). */
int sj_model_vjp_info(const sj_model *m, long *compressed, long *dense, long *basis_groups,
                      long *projection_groups, uint64_t *rng_state);
int sj_model_set_vjp_rng(sj_model *m, uint64_t rng_state);
/* Updates applied so far (Adam's step / the SGD state's step; the
 * checkpoint manifest's step). */
long sj_model_steps(const sj_model *m);
int sj_model_destroy(sj_model *m);
/* Number of parameter tensors / total elements in the reference layout. */
long sj_model_param_tensors(const sj_model *m);
long sj_model_param_count(const sj_model *m);
/* name, shape and element offset (reference layout order) of tensor i. */
int sj_model_param_info(const sj_model *m, long i, const char **name, long *rows, long *cols,
                        long *offset);
/* Host <-> device exchange in the reference layout (synchronous). */
int sj_model_set_params(sj_model *m, const float *host);
int sj_model_get_params(sj_model *m, float *host);
int sj_model_get_grads(sj_model *m, float *host);
int sj_model_get_adam_state(sj_model *m, float *m_host, float *v_host, long *step);
int sj_model_set_adam_state(sj_model *m, const float *m_host, const float *v_host, long step);
/* Batch input: host arrays (synchronous copy) or device arrays (async D2D
 * on the model stream).  ids/targets int32 [batch*sequence]. */
int sj_model_set_batch(sj_model *m, const int32_t *ids, const int32_t *targets, int on_device);
/* Gradient accumulation (TrainConfig::accumulation; train lib.rs:390-415
 * with Adam::accumulate, lib.rs:179-198): `observations` batches stacked
 * ([observations][batch*sequence], host arrays).  Each following
 * sj_model_train_step runs every observation's forward and backward on its
 * batch (objective seed loss_scale / observations, loss summary weighted
 * 1 / observations into its own slot), keeps the first observation's
 * gradients and adds the later ones in order, then takes one FP64 norm and
 * one AdamW update; sj_model_forward_backward leaves the summed gradients in
 * the gradient arena, and sj_model_read_loss returns the sum of the slots.
 * AdamW byte language models only; 1 <= observations <= 256.
 * sj_model_set_batch returns to one observation per update. */
int sj_model_set_batches(sj_model *m, const int32_t *ids, const int32_t *targets, long observations);
/* Forward + backward only (gradients left in the model's gradient arena). */
int sj_model_forward_backward(sj_model *m);
/* One full training step: forward, backward, FP64 grad norm, clip, AdamW
 * with learning rate lr (Adam::update increments the step first), or the
 * SGD update of an SGD model. */
int sj_model_train_step(sj_model *m, float lr);
/* Capture the step as a hipGraph on the next sj_model_train_step and replay
 * it afterwards (on != 0), or run eagerly (on == 0). */
int sj_model_use_graph(sj_model *m, int on);
/* Reads the last step's mean loss and gradient norm (synchronises the
 * model stream).  Returns SJ_ERR_NONFINITE if the last update saw a
 * non-finite norm. */
int sj_model_read_loss(sj_model *m, double *loss, double *grad_norm);
/* Forward only (Model::logits + Graph::cross_entropy, model lib.rs:336-340,
 * graph.rs:539-549): the loss of the staged batch without a backward or an
 * update -- the `evaluate` pass of the benchmark (benchmark.rs:71-99: BPB =
 * mean loss / ln 2).  Read the loss with sj_model_read_loss. */
int sj_model_forward(sj_model *m);

/* KV cache (Cache, model lib.rs:36-50; Model::new_cache / forward_cached /
 * hidden_cached, lib.rs:359-394; architecture.rs:428-533 and 758-799) for
 * the byte language models (dense and MoE; bf16 on the MFMA layout or
 * fp32): per layer the keys and values of one sequence, [capacity][HK *
 * head_dim] in the compute dtype.  sj_model_forward_cached runs n new tokens
 * (host array, bytes or EOS) at positions length .. length+n-1 through the
 * blocks with the training forward's kernels, writes the keys and values
 * into the cache, and leaves the fp32 logits of the last token in
 * `logits` (device, [vocab]; nullable).  Errors: "KV cache context limit
 * reached" past the capacity, "input tokens must be bytes or EOS". */
typedef struct sj_cache sj_cache;
int sj_cache_create(sj_model *m, long capacity, sj_cache **out);
int sj_cache_destroy(sj_cache *c);
int sj_cache_reset(sj_cache *c);
long sj_cache_length(const sj_cache *c);
int sj_model_forward_cached(sj_model *m, sj_cache *c, const int32_t *tokens, long n, float *logits);

/* Per-op timing (the reference's kernel-profile feature, crates/sejong-gpu/
 * src/lib.rs:451-482 and counters.rs:33-56): with profiling on, steps run
 * eagerly and every op is bracketed by a HIP event pair on the model stream.
 * sj_model_profile_collect synchronises, aggregates the ops recorded since
 * its last call by op name and returns the number of names (or -1);
 * sj_model_profile_entry reads one aggregate.  on = 2 times every op
 * cold: before its event pair the stream writes a 512 MiB buffer (twice the
 * 256 MB Infinity Cache), so the op's operands come from HBM.  on = 3 also
 * times each GEMM op's kernel alone, by events the launch records at the
 * kernel's own start and end (hipExtLaunchKernel: no launch gaps, no split-K
 * reduce), as an aggregate "<op>#kernel" (the extra packets lengthen the
 * op's own pair, so op times come from on = 1).  on = 4 records only those
 * kernel-own pairs (the "#kernel" aggregates) and keeps the step's second
 * stream: each kernel's time as it shares the chip in the step (no
 * counterpart in the reference).  sj_model_profile_kernel
 * names the GEMM kernel an aggregate's
 * op launched, as rocprofv3 lists it ("k_gemm_fast<BM, BN, PA, PB, EPI, NS,
 * TM>"; "" for ops without one); it has no counterpart in the reference. */
int sj_model_profile(sj_model *m, int on);
long sj_model_profile_collect(sj_model *m);
int sj_model_profile_entry(sj_model *m, long i, const char **name, double *total_ms, long *calls);
int sj_model_profile_kernel(sj_model *m, long i, const char **kernel);
/* The stored forward activations of the last step in a fixed pack order
 * (per layer x, z, q, k, v, o, lse, x1, z2, g, u, h; then the last residual
 * x_L, the final-norm output and the fp32 logits), converted to fp32 (exact
 * for bf16 storage).  Used to check the backward conditioned on the stored
 * operands.  Synchronous. */
long sj_model_activation_count(const sj_model *m);
int sj_model_export_activations(sj_model *m, float *host);
/* Device pointers of internal buffers for callers that time or inspect
 * kernels directly (what: "logits", "loss_rows", "ids", "targets",
 * "params", "grads", "mirror", "mirror_t", "workspace", "stream",
 * "grad_sq_slots" (fp64: the FP64 squared-norm partials the last backward's
 * gradient producers wrote; elements 0 when the update summed the arena
 * instead), and for
 * parameter-VJP models "vjp_columns", "vjp_rows", "vjp_map" (int32) and
 * "vjp_basis" (fp32 [tokens][rank]); for MoE models, per layer l,
 * "route_ids.<l>" (int32 [rows][top_k]), "route_weights.<l>" (fp32),
 * "route_counts.<l>", "route_offsets.<l>", "route_pslot.<l>" (the packed
 * slot per position, -1 for padding) and "route_ppos.<l>" (each slot's
 * packed position) (int32)). */
int sj_model_buffer(sj_model *m, const char *what, void **ptr, long *elements);

/* ----------------------------------------------------------- Checkpoints
 * Host code (no device work).  Files in the safetensors format of the
 * crate the reference pins (0.8.0): save_tensors / load_tensors, crates/
 * sejong-model/src/lib.rs:456-538.  Tensors are F32; tensor i has rank
 * ranks[i] and its dimensions next in dims (concatenated). */
/* save_tensors: written in byte-wise name order. */
int sj_safetensors_write(const char *path, long count, const char *const *names, const long *ranks,
                         const long *dims, const float *const *data);
/* The header JSON (validated: every tensor's byte range inside the file);
 * out (nullable) receives it NUL-terminated when capacity > *length. */
int sj_safetensors_header(const char *path, char *out, size_t capacity, size_t *length);
/* One F32 tensor of count elements by name; non-finite values are an error
 * (load_tensors, lib.rs:509-537). */
int sj_safetensors_read(const char *path, const char *name, float *out, long count);
/* Model::save (lib.rs:395-442): fails if directory exists; writes
 * weights.safetensors, optimizer.safetensors (n_optimizer > 0) and
 * manifest.json (the given text) into a staging directory
 * <parent>/.<name>.<pid>.tmp, renames it onto directory, and removes the
 * staging directory on failure. */
int sj_checkpoint_save(const char *directory, const char *manifest_json, long n_weights,
                       const char *const *weight_names, const long *weight_ranks, const long *weight_dims,
                       const float *const *weight_data, long n_optimizer, const char *const *optimizer_names,
                       const long *optimizer_ranks, const long *optimizer_dims, const float *const *optimizer_data);

/* Corpus::open's fingerprint hash (crates/sejong-train/src/lib.rs:32-56:
 * blake3::Hasher::new / update / finalize of the `blake3` crate 1.8.7):
 * BLAKE3 in its default hash mode, 32-byte output.  The caller owns the
 * state (sj_blake3_state_bytes bytes, 8-byte aligned); init, then any
 * number of updates, then finalize (which leaves the state usable for more
 * updates).  Host code: no device is touched. */
size_t sj_blake3_state_bytes(void);
int sj_blake3_init(void *state);
int sj_blake3_update(void *state, const void *data, size_t bytes);
int sj_blake3_finalize(const void *state, uint8_t *out32);

#ifdef __cplusplus
}
#endif
#endif /* SEJONG_HIP_H */
