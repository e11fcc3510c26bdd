// Shared device/host helpers for the gfx950 kernels of the Sejong training
// step.  Wave64 throughout; bf16 values are carried as raw 16-bit words in
// memory and converted with the hardware v_cvt_pk_bf16_f32 (round to nearest
// even) through the __bf16 type.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#include "../../include/sejong_hip.h"

namespace sj {

typedef uint16_t bf16_t;  // raw bf16 bits in memory
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int WAVE = 64;

__device__ __forceinline__ float bf2f(bf16_t b) { return __uint_as_float(((uint32_t)b) << 16); }

__device__ __forceinline__ bf16_t f2bf(float x) {
  __bf16 b = (__bf16)x;
  return __builtin_bit_cast(bf16_t, b);
}

// Round-to-nearest-even float -> bf16 value, returned as float.
__device__ __forceinline__ float round_bf(float x) { return bf2f(f2bf(x)); }

// Split an fp32 value into hi + lo bf16 words with x ~= hi + lo to ~2^-16
// relative: hi = RNE(x), lo = RNE(x - hi).  Used so fp32 gradient operands
// can feed bf16 MFMA without the ~1e-3 error of a single bf16 rounding.
__device__ __forceinline__ void split_bf(float x, bf16_t& hi, bf16_t& lo) {
  hi = f2bf(x);
  lo = f2bf(x - bf2f(hi));
}

// a * b rounded to fp32 and never fused into a following add (so a split
// of the product sees the stored fp32 value)
__device__ __forceinline__ float mul_rn(float a, float b) {
#pragma clang fp contract(off)
  return a * b;
}

__device__ __forceinline__ uint32_t pack2(bf16_t a, bf16_t b) { return (uint32_t)a | ((uint32_t)b << 16); }

// The scalars of one multi-tensor AdamW step (Adam::update, crates/sejong-
// train/src/lib.rs:199-238; kernel adamw, kernels.py:193-202): the clip
// factor formed on the device from the FP64 squared gradient norm.
struct AdamCoef {
  float scale, lr, b1, b2, eps, ib1, ib2, keep;
};
// false (and no update) when the norm is not finite
__device__ __forceinline__ bool adam_coef(const sj_adam_step* st, const double* sumsq, AdamCoef& c) {
  const double norm = sqrt(sumsq[0]) / (double)st->loss_scale;
  if (!isfinite(norm)) return false;
  const double clipping = (st->clip_enabled && norm > (double)st->clip_norm) ? (double)st->clip_norm / norm : 1.0;
  c.scale = (float)clipping / st->loss_scale;
  c.lr = st->lr; c.b1 = st->beta1; c.b2 = st->beta2; c.eps = st->eps; c.ib1 = st->inv_b1; c.ib2 = st->inv_b2;
  c.keep = 1.f - st->lr * st->weight_decay;
  return true;
}
// one parameter: m, v and w updated in place (decay: the parameter is a
// matrix, p.value.shape.len() > 1).  The fused multiply-adds are written
// out, so every kernel that updates parameters rounds them alike whatever
// the compiler would contract in its context.
__device__ __forceinline__ void adam_elem(float& w, float g, float& m, float& v, const AdamCoef& c, bool decay) {
  const float gi = g * c.scale;
  m = fmaf(c.b1, m, (1.f - c.b1) * gi);
  v = fmaf(c.b2, v, ((1.f - c.b2) * gi) * gi);
  const float den = sqrtf(v * c.ib2) + c.eps;
  const float stp = den > 0.f ? (m * c.ib1) / den : 0.f;
  w = fmaf(w, decay ? c.keep : 1.f, -(c.lr * stp));
}

// Load a value of dtype `dt` (SJ_F32 or SJ_BF16) at index i as float.
__device__ __forceinline__ float load_as_f32(const void* p, int dt, long i) {
  return dt == SJ_BF16 ? bf2f(((const bf16_t*)p)[i]) : ((const float*)p)[i];
}
__device__ __forceinline__ void store_from_f32(void* p, int dt, long i, float v) {
  if (dt == SJ_BF16)
    ((bf16_t*)p)[i] = f2bf(v);
  else
    ((float*)p)[i] = v;
}

template <typename T>
__device__ __forceinline__ T wave_sum(T v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, WAVE);
  return v;
}
template <typename T>
__device__ __forceinline__ T wave_max(T v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    T u = __shfl_xor(v, o, WAVE);
    v = u > v ? u : v;
  }
  return v;
}

// Block-wide sum for blockDim.x = NT (multiple of 64); `red` holds NT/64 T.
template <typename T, int NT>
__device__ __forceinline__ T block_sum(T v, T* red) {
  v = wave_sum(v);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  if (lane == 0) red[w] = v;
  __syncthreads();
  T s = 0;
#pragma unroll
  for (int i = 0; i < NT / 64; i++) s += red[i];
  __syncthreads();
  return s;
}

// one norm-weight gradient reduction: dw[c] = sum_g partial[g][c]
struct RmsReduceJob {
  const float* partial;
  float* dw;
  long groups, d;
};

}  // namespace sj

// ------------------------------------------------------------- host side
// Step record of the SGD step driver, staged on the device before each step
// so a captured step reads this step's values.
struct sj_sgd_step {
  float lr, weight_decay, clip_norm;
  int clip_enabled;
  uint64_t seed;  // parameter-VJP index seed (one Rng::next_u64 of the parameter RNG)
};

namespace sjh {
// parameter_indices with the seed read from device memory
int pvjp_indices_dev(hipStream_t stream, const uint64_t* seed, long a, long donor_width, long feature_blocks,
                     long selected, long rank, long block_rows, int32_t* scratch, int32_t* columns, int32_t* rows,
                     int32_t* map);
// GradientPlan::update with lr from a staged step record and the clipping
// factor formed on the device from the FP64 squared norm (nullable: no clip)
int factored_update_staged(hipStream_t stream, const void* meta, long tiles, const sj_sgd_step* step,
                           const double* sumsq);
// attention over transposed operands (attention_t.hip) and the group reduce
// of the per-head dK | dV partials it shares with attention.hip
int attention_t_prepare();
// whether attention_bwd_tt_parts runs the grouped launch for these sizes
// (dK | dV planes written by part 2, part 4 does nothing)
bool attention_bwd_grouped(long batch, long t, long hq, long hk, bool transposed);
// fp32 -> hi/lo bf16 planes of n contiguous values (hi = RNE(x), lo =
// RNE(x - hi)); n a multiple of 8, all three pointers 16-byte aligned
int split_planes(hipStream_t s, const float* x, long n, uint16_t* hi, uint16_t* lo);
// sj_rmsnorm_fwd_t with the embedding lookup fused in: row r of the input is
// row ids[r] of the bf16 table, also written to x0 [rows][d]
int rmsnorm_fwd_t_embed(void* stream, const uint16_t* table, const int32_t* ids, uint16_t* x0, const uint16_t* w,
                        uint16_t* y, uint16_t* y_t, long ldt, long rows, long d, float eps);
// router top-k (16 lanes per token, 16 tokens per workgroup) that also
// writes each workgroup's routed-slot count per expert into hist
// [router_hist_blocks(rows)][E], and the pack that reads those counts
// (the same counts, offsets, pslot and ppos as sj_route_pack); E == 8, K <= 4
bool router_pack_ok(long d, long ldz, long E, long K, const void* z, const void* wr, const void* logits);
long router_hist_blocks(long rows);
int router_topk_hist(hipStream_t s, const uint16_t* z, long ldz, const uint16_t* wr, long d, long rows, long E, long K,
                     uint16_t* logits, int32_t* ids, float* weights, int32_t* hist);
int route_pack_hist(hipStream_t s, const int32_t* ids, long rows, long K, long E, const int32_t* hist, int32_t* counts,
                    int32_t* offsets, int32_t* pslot, int32_t* ppos, long cap);
// cross entropy with dX as hi/lo bf16 planes [rows][ldp] (columns past vocab zero)
int cross_entropy_planes(void* stream, const float* x, long ldx, const int32_t* targets, float* loss, uint16_t* dx_hi,
                         uint16_t* dx_lo, long ldp, long rows, long vocab, float dy_scalar);
// project_qkv (MFMA layout) into separate q, k, v buffers
int qkv_fwd_t_out(void* stream, const uint16_t* x, long ldx, long M, long D, const uint16_t* wqkv_t, long ldw, long N,
                  long KV, uint16_t* q, long ldq, uint16_t* k, long ldk, uint16_t* v, long ldv, const float* rope_table,
                  long rope_t, long head_dim, uint16_t* qkv_t, long ldqt);
// cached grouped attention on the MFMA layout (bf16, head_dim 64), one sequence
int attention_fwd_cached_t(void* stream, const uint16_t* q, long ldq, const uint16_t* k, const uint16_t* v, long ldkv,
                           long capacity, long tq, long offset, long hq, long hk, long window, uint16_t* o, long ldo);
int attention_kv_reduce(hipStream_t s, const float* part, long group, long M, long T, long N, long KV,
                        const float* rope, uint16_t* g_hi, uint16_t* g_lo, long ldg, uint16_t* gt_hi, uint16_t* gt_lo,
                        long ldgt);
// parts: 1 Delta, 2 dQ | dK dV, 4 the group reduce; counters: the grouped
// launch's meeting counters (sj_attention_bwd_tt_counter_bytes, zero before
// the first call and left zero by each), null for the workspace's own tail
int attention_bwd_tt_parts(int parts, void* stream, const uint16_t* qkv, long ldqkv, long ldt, const uint16_t* o,
                           long ldo, const float* lse_t, const uint16_t* do_hi, const uint16_t* do_lo, long lddo,
                           float* delta_t, long batch, long t, long hq, long hk, long head_dim, long window,
                           const float* rope_table, uint16_t* g_hi, uint16_t* g_lo, long ldg, uint16_t* g_t_hi,
                           uint16_t* g_t_lo, long ldgt, void* workspace, size_t workspace_bytes,
                           uint32_t* counters);
// Profiling hook of the step driver: while one of its ops is timed
// (sj_model_profile), the op's GEMM launch notes the kernel's name and, in
// kernel timing mode (k0 set), launches it with hipExtLaunchKernel recording
// k0 / k1 at its own start and end (the kernel's duration, apart from launch
// gaps and any split-K reduce).
struct ProfHook {
  bool on = false;
  hipEvent_t k0 = nullptr, k1 = nullptr;
  bool used = false;
  char kernel[80] = {0};
};
ProfHook& prof_hook();
// Gradient-norm hook of the step driver.  While armed (base set) and `on`
// (around each call that writes a gradient), the gradient producer (the
// split-K reduce of a dW product, the norm-weight reduce, the embedding
// backward) also writes the FP64 sum of squares of the values it stores, one
// per workgroup, into the next slots of base[0 .. cap); a fixed-order sum
// over the slots then gives the squared gradient norm without a pass over
// the gradient arena.  A gradient written any other way (a dW product
// without split-K) sets `missed`, and the step sums the arena instead.
struct GradSq {
  double* base = nullptr;
  long next = 0, cap = 0;
  bool missed = false, on = false;
  double* take(long n) {
    if (!base || !on) return nullptr;
    if (next + n > cap) {
      missed = true;
      return nullptr;
    }
    double* p = base + next;
    next += n;
    return p;
  }
};
GradSq& grad_sq();
// Record a failure message for sj_last_error() and return the status.
int fail(int status, const char* fmt, ...);
int hip_check(hipError_t e, const char* what);
// sj_rmsnorm_bwd_p with the dw reduce left to rmsnorm_reduce_multi (partial:
// sj_rmsnorm_bwd_p_workspace_bytes of its own)
int rmsnorm_bwd_p_deferred(void* stream, const uint16_t* x, const uint16_t* w, const float* dy, const float* dx_acc,
                           float* dx, uint16_t* dx_hi, uint16_t* dx_lo, uint16_t* dx_t_hi, uint16_t* dx_t_lo,
                           long ldt, long rows, long d, float eps, float* partial);
int rmsnorm_reduce_multi(void* stream, const sj::RmsReduceJob* jobs, long njobs, long max_d);
// the parameter VJP's token-contracted products with one operand in row
// layout (gemm_fast.hip): C = X^T B^T (X [K][ldx] one plane, B [N][K] hi/lo)
// and C = A Y (A [M][K] hi/lo, Y [K][ldy] hi/lo); fp32 C, K % 8 == 0;
// workspace as sj_gemm_planes_workspace_bytes(M, N, K)
int gemm_planes_rows_a(void* stream, long M, long N, long K, const uint16_t* x, long ldx, const uint16_t* b_hi,
                       const uint16_t* b_lo, long ldb, float* c, long ldc, void* workspace, size_t workspace_bytes);
int gemm_planes_rows_b(void* stream, long M, long N, long K, const uint16_t* a_hi, const uint16_t* a_lo, long lda,
                       const uint16_t* y_hi, const uint16_t* y_lo, long ldy, float* c, long ldc, void* workspace,
                       size_t workspace_bytes);
// out[0] = FP64 sum of slots[0 .. count) in a fixed order (one workgroup)
int sum_slots(hipStream_t stream, const double* slots, long count, double* out);
// one-time kernel attribute setup (dynamic LDS limits), outside capture
int norm_prepare();
int gemm_fast_prepare();
int attention_prepare();
// sj_attention_bwd_p split so a caller can time its two kernels apart
int attention_bwd_p_parts(int parts, void* stream, const uint16_t* q, long ldq, const uint16_t* k, long ldk,
                          const uint16_t* v, long ldv, const uint16_t* o, long ldo, const float* lse,
                          const float* dout, long lddo, float* delta, long batch, long t, long hq, long hk,
                          long head_dim, const float* rope_table, uint16_t* g_hi, uint16_t* g_lo, long ldg,
                          uint16_t* gt_hi, uint16_t* gt_lo, long ldgt, void* workspace, size_t workspace_bytes);
}  // namespace sjh

#define SJ_REQUIRE(cond, ...)                                  \
  do {                                                         \
    if (!(cond)) return sjh::fail(SJ_ERR_INVALID, __VA_ARGS__); \
  } while (0)

#define SJ_HIP(call)                                          \
  do {                                                        \
    hipError_t _e = (call);                                   \
    if (_e != hipSuccess) return sjh::hip_check(_e, #call);   \
  } while (0)

#define SJ_LAUNCH_CHECK(what)                                 \
  do {                                                        \
    hipError_t _e = hipGetLastError();                        \
    if (_e != hipSuccess) return sjh::hip_check(_e, what);    \
  } while (0)
