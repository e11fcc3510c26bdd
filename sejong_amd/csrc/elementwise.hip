// Bandwidth-bound kernels of the training step: fill / cast / add,
// embedding forward and deterministic backward, RoPE (and its cos/sin
// table), SwiGLU, fused cross-entropy forward+backward, FP64 loss summary,
// FP64 sum of squares and AdamW (per tensor and multi-tensor with an
// on-device clip factor).
#include <math.h>

#include "common.h"

using namespace sj;

namespace {

constexpr int EW_THREADS = 256;

inline int ew_blocks(long n, int per_thread = 1) {
  long b = (n + (long)EW_THREADS * per_thread - 1) / ((long)EW_THREADS * per_thread);
  if (b > 65535L * 16) b = 65535L * 16;
  return (int)(b < 1 ? 1 : b);
}

inline bool dtype_ok(int dt) { return dt == SJ_F32 || dt == SJ_BF16; }

// kernels.py:6-9
__global__ void k_fill(void* y, int dt, long n, float value) {
  for (long i = blockIdx.x * (long)blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x)
    store_from_f32(y, dt, i, value);
}

// kernels.py:11-14 (copy with dtype conversion)
__global__ void k_cast(const void* x, int xd, void* y, int yd, long n) {
  for (long i = blockIdx.x * (long)blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x)
    store_from_f32(y, yd, i, load_as_f32(x, xd, i));
}

// the same copy without a dtype conversion: 16-byte vectors
__global__ __launch_bounds__(EW_THREADS) void k_copy16(const uint4* __restrict__ x, uint4* __restrict__ y, long n16) {
  for (long i = blockIdx.x * (long)blockDim.x + threadIdx.x; i < n16; i += (long)gridDim.x * blockDim.x) y[i] = x[i];
}

// fp32 values as hi/lo bf16 planes, 8 per thread (32-byte loads, 16-byte stores)
__global__ __launch_bounds__(EW_THREADS) void k_split_planes(const float* __restrict__ x, long n8,
                                                             uint16_t* __restrict__ hi, uint16_t* __restrict__ lo) {
  for (long i = blockIdx.x * (long)blockDim.x + threadIdx.x; i < n8; i += (long)gridDim.x * blockDim.x) {
    const float4 a = ((const float4*)x)[2 * i], b = ((const float4*)x)[2 * i + 1];
    const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    bf16_t h[8], l[8];
#pragma unroll
    for (int k = 0; k < 8; k++) split_bf(v[k], h[k], l[k]);
    ((u32x4*)hi)[i] = u32x4{pack2(h[0], h[1]), pack2(h[2], h[3]), pack2(h[4], h[5]), pack2(h[6], h[7])};
    ((u32x4*)lo)[i] = u32x4{pack2(l[0], l[1]), pack2(l[2], l[3]), pack2(l[4], l[5]), pack2(l[6], l[7])};
  }
}

// kernels.py:16-21: y = x + alpha*z in fp32
__global__ void k_add(const void* x, int xd, const void* z, int zd, void* y, int yd, long n, float alpha) {
  for (long i = blockIdx.x * (long)blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x)
    store_from_f32(y, yd, i, load_as_f32(x, xd, i) + alpha * load_as_f32(z, zd, i));
}

// kernels.py:41-45
__global__ void k_embedding_fwd(const void* w, int wd, const int32_t* ids, void* y, int yd, long n, long d) {
  long total = n * d;
  for (long i = blockIdx.x * (long)blockDim.x + threadIdx.x; i < total; i += (long)gridDim.x * blockDim.x) {
    long row = i / d, col = i - row * d;
    store_from_f32(y, yd, i, load_as_f32(w, wd, (long)ids[row] * d + col));
  }
}

// kernels.py:47-52 restated without atomics: workgroup v owns vocabulary
// row v, finds the tokens with id v in token order (block-wide ballot
// compaction) and sums their gradient rows in that order.
constexpr int EMB_THREADS = 256;
__global__ __launch_bounds__(EMB_THREADS) void k_embedding_bwd(const float* dy, const int32_t* ids, float* dw,
                                                               long n, long d) {
  __shared__ int matches[EMB_THREADS];
  __shared__ int wave_count[EMB_THREADS / 64];
  const int v = blockIdx.x;
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  // each thread owns columns t, t+256, ... (up to 8 per thread)
  constexpr int MAXC = 8;
  float acc[MAXC];
#pragma unroll
  for (int c = 0; c < MAXC; c++) acc[c] = 0.f;
  for (long base = 0; base < n; base += EMB_THREADS) {
    long i = base + t;
    bool hit = i < n && ids[i] == v;
    uint64_t mask = __ballot(hit);
    if (lane == 0) wave_count[w] = __popcll(mask);
    __syncthreads();
    int before = 0, total = 0;
    for (int j = 0; j < EMB_THREADS / 64; j++) {
      if (j < w) before += wave_count[j];
      total += wave_count[j];
    }
    if (hit) matches[before + __popcll(mask & ((1ull << lane) - 1))] = (int)i;
    __syncthreads();
    for (int m = 0; m < total; m++) {
      const float* row = dy + (long)matches[m] * d;
#pragma unroll
      for (int c = 0; c < MAXC; c++) {
        long col = t + (long)c * EMB_THREADS;
        if (col < d) acc[c] += row[col];
      }
    }
    __syncthreads();
  }
#pragma unroll
  for (int c = 0; c < MAXC; c++) {
    long col = t + (long)c * EMB_THREADS;
    if (col < d) dw[(long)v * d + col] = acc[c];
  }
}

// RoPE cos/sin table [t][head_dim/2] (cos, sin interleaved), angles in
// double: angle = pos * theta^(-2i/D) (kernels.py:108).
__global__ void k_rope_table(float* table, long t, long half, long head_dim, double theta) {
  long total = t * half;
  for (long i = blockIdx.x * (long)blockDim.x + threadIdx.x; i < total; i += (long)gridDim.x * blockDim.x) {
    long pos = i / half, pair = i - pos * half;
    double angle = (double)pos * exp((-2.0 * (double)pair / (double)head_dim) * log(theta));
    double s, c;
    sincos(angle, &s, &c);
    table[2 * i] = (float)c;
    table[2 * i + 1] = (float)s;
  }
}

// kernels.py:103-113 (one thread per pair)
__global__ void k_rope(const void* x, void* y, int dt, long rows, long ld, long t, long heads, long head_dim,
                       long offset, double theta, int inverse) {
  long half = head_dim / 2;
  long total = rows * heads * half;
  for (long i = blockIdx.x * (long)blockDim.x + threadIdx.x; i < total; i += (long)gridDim.x * blockDim.x) {
    long pair = i % half, hr = i / half;
    long h = hr % heads, row = hr / heads;
    long pos = row % t + offset;
    double angle = (double)pos * exp((-2.0 * (double)pair / (double)head_dim) * log(theta));
    double sd, cd;
    sincos(angle, &sd, &cd);
    float c = (float)cd, s = (float)sd;
    if (inverse) s = -s;
    long base = row * ld + h * head_dim + 2 * pair;
    float a = load_as_f32(x, dt, base), b = load_as_f32(x, dt, base + 1);
    store_from_f32(y, dt, base, a * c - b * s);
    store_from_f32(y, dt, base + 1, a * s + b * c);
  }
}

__device__ __forceinline__ float sigmoidf_(float g) { return 1.f / (1.f + __expf(-g)); }

// kernels.py:90-93
__global__ void k_swiglu_fwd(const void* g, const void* u, void* h, int dt, long n) {
  for (long i = blockIdx.x * (long)blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x) {
    float gv = load_as_f32(g, dt, i), uv = load_as_f32(u, dt, i);
    store_from_f32(h, dt, i, gv * (1.f / (1.f + expf(-gv))) * uv);
  }
}

// kernels.py:95-101
__global__ void k_swiglu_bwd(const void* g, const void* u, int dt, const float* dy, float* dg, float* du, long n) {
  for (long i = blockIdx.x * (long)blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x) {
    float gv = load_as_f32(g, dt, i), uv = load_as_f32(u, dt, i), d = dy[i];
    float s = 1.f / (1.f + expf(-gv));
    dg[i] = d * uv * s * (1.f + gv * (1.f - s));
    du[i] = d * gv * s;
  }
}

// kernels.py:176-191: one wavefront per row.
__global__ __launch_bounds__(256) void k_cross_entropy(const float* x, long ldx, const int32_t* targets, float* loss,
                                                       float* dx, long lddx, long rows, long vocab, const float* dy,
                                                       float dy_scalar) {
  const int lane = threadIdx.x & 63;
  long r = blockIdx.x * 4L + (threadIdx.x >> 6);
  if (r >= rows) return;
  const float* xr = x + r * ldx;
  float m = -INFINITY;
  for (long j = lane; j < vocab; j += 64) m = fmaxf(m, xr[j]);
  m = wave_max(m);
  float s = 0.f;
  for (long j = lane; j < vocab; j += 64) s += expf(xr[j] - m);
  s = wave_sum(s);
  int tg = targets[r];
  if (lane == 0) loss[r] = m + logf(s) - xr[tg];
  if (dx) {
    float d = dy ? dy[r] : dy_scalar;
    float inv = 1.f / s;
    for (long j = lane; j < vocab; j += 64)
      dx[r * lddx + j] = (expf(xr[j] - m) * inv - (j == tg ? 1.f : 0.f)) * d;
  }
}

// The same cross entropy with dX left as hi/lo bf16 planes [rows][width]
// (the output head's dX / dW GEMM operands); columns vocab .. width-1 of the
// planes are written as zero.
__global__ __launch_bounds__(256) void k_cross_entropy_planes(const float* x, long ldx, const int32_t* targets,
                                                              float* loss, bf16_t* dh, bf16_t* dl, long ldp, long rows,
                                                              long vocab, long width, float dy_scalar) {
  const int lane = threadIdx.x & 63;
  long r = blockIdx.x * 4L + (threadIdx.x >> 6);
  if (r >= rows) return;
  const float* xr = x + r * ldx;
  float m = -INFINITY;
  for (long j = lane; j < vocab; j += 64) m = fmaxf(m, xr[j]);
  m = wave_max(m);
  float s = 0.f;
  for (long j = lane; j < vocab; j += 64) s += expf(xr[j] - m);
  s = wave_sum(s);
  int tg = targets[r];
  if (lane == 0) loss[r] = m + logf(s) - xr[tg];
  const float inv = 1.f / s;
  for (long j = lane; j < width; j += 64) {
    bf16_t h = 0, l = 0;
    if (j < vocab) split_bf((expf(xr[j] - m) * inv - (j == tg ? 1.f : 0.f)) * dy_scalar, h, l);
    dh[r * ldp + j] = h;
    dl[r * ldp + j] = l;
  }
}

// kernels.py:254-262 (single workgroup, FP64, fixed order)
__global__ __launch_bounds__(256) void k_loss_summary(const float* loss, long n, double* out, long slot, float weight) {
  __shared__ double red[4];
  double s = 0.0;
  for (long i = threadIdx.x; i < n; i += 256) s += (double)loss[i];
  s = block_sum<double, 256>(s, red);
  if (threadIdx.x == 0) out[slot] = s * (double)weight / (double)n;
}

constexpr int SS_THREADS = 256;
constexpr int SS_BLOCKS_MAX = 1024;

inline int ss_blocks(long n) {
  long b = (n + SS_THREADS * 16L - 1) / (SS_THREADS * 16L);
  if (b > SS_BLOCKS_MAX) b = SS_BLOCKS_MAX;
  return (int)(b < 1 ? 1 : b);
}

// FP64 sum of squares, stage 1: block partials (kernels.py:265-287).  Each
// thread issues four 16-byte loads before it accumulates them, so a thread
// has 64 bytes in flight rather than one dependent 4-byte load per trip
// (the arena read runs near HBM rate instead of latency-bound).
__global__ __launch_bounds__(SS_THREADS) void k_sumsq_partial(const float* g, long n, double* partial) {
  __shared__ double red[SS_THREADS / 64];
  constexpr int U = 4;
  double s = 0.0, t = 0.0;
  const long n4 = ((uintptr_t)g & 15) == 0 ? n >> 2 : 0;
  const float4* g4 = (const float4*)g;
  const long stride = (long)gridDim.x * SS_THREADS;
  for (long i0 = blockIdx.x * (long)SS_THREADS + threadIdx.x; i0 < n4; i0 += U * stride) {
    float4 v[U];
#pragma unroll
    for (int u = 0; u < U; u++) v[u] = i0 + u * stride < n4 ? g4[i0 + u * stride] : float4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < U; u++) {
      s += (double)v[u].x * (double)v[u].x + (double)v[u].y * (double)v[u].y;
      t += (double)v[u].z * (double)v[u].z + (double)v[u].w * (double)v[u].w;
    }
  }
  for (long i = 4 * n4 + blockIdx.x * (long)SS_THREADS + threadIdx.x; i < n; i += stride) {
    const double v = (double)g[i];
    s += v * v;
  }
  s = block_sum<double, SS_THREADS>(s + t, red);
  if (threadIdx.x == 0) partial[blockIdx.x] = s;
}
__global__ __launch_bounds__(SS_THREADS) void k_sumsq_final(const double* partial, int count, double* out) {
  __shared__ double red[SS_THREADS / 64];
  double s = 0.0;
  for (int i = threadIdx.x; i < count; i += SS_THREADS) s += partial[i];
  s = block_sum<double, SS_THREADS>(s, red);
  if (threadIdx.x == 0) out[0] = s;
}

// kernels.py:193-202
__global__ void k_adamw(float* w, const float* g, float* m, float* v, long n, float lr, float b1, float b2, float eps,
                        float decay, float ib1, float ib2, float scale) {
  for (long i = blockIdx.x * (long)blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x) {
    float gi = g[i] * scale;
    float mi = b1 * m[i] + (1.f - b1) * gi;
    float vi = b2 * v[i] + (1.f - b2) * gi * gi;
    float den = sqrtf(vi * ib2) + eps;
    float st = den > 0.f ? (mi * ib1) / den : 0.f;
    w[i] = w[i] * (1.f - lr * decay) - lr * st;
    m[i] = mi;
    v[i] = vi;
  }
}

// Adam::update (train lib.rs:199-238) over the flat arena, 4 elements per
// thread, clip factor formed from the device FP64 squared norm.
__global__ __launch_bounds__(256) void k_adamw_multi(float* __restrict__ w, const float* __restrict__ g,
                                                      float* __restrict__ m, float* __restrict__ v,
                                                      bf16_t* __restrict__ mirror, long n, long n_nodecay,
                                                      const sj_adam_step* __restrict__ st,
                                                      const double* __restrict__ sumsq, int32_t* status) {
  AdamCoef c;
  if (!adam_coef(st, sumsq, c)) {
    if (blockIdx.x == 0 && threadIdx.x == 0) status[0] = 1;
    return;
  }
  for (long q = blockIdx.x * (long)blockDim.x + threadIdx.x; q * 4 < n; q += (long)gridDim.x * blockDim.x) {
    long i0 = q * 4;
    if (i0 + 4 <= n) {
      float4 wv = *(const float4*)(w + i0), gv = *(const float4*)(g + i0);
      float4 mv = *(const float4*)(m + i0), vv = *(const float4*)(v + i0);
      float ws[4] = {wv.x, wv.y, wv.z, wv.w}, gs[4] = {gv.x, gv.y, gv.z, gv.w};
      float ms[4] = {mv.x, mv.y, mv.z, mv.w}, vs[4] = {vv.x, vv.y, vv.z, vv.w};
#pragma unroll
      for (int j = 0; j < 4; j++) adam_elem(ws[j], gs[j], ms[j], vs[j], c, (i0 + j) >= n_nodecay);
      *(float4*)(w + i0) = make_float4(ws[0], ws[1], ws[2], ws[3]);
      *(float4*)(m + i0) = make_float4(ms[0], ms[1], ms[2], ms[3]);
      *(float4*)(v + i0) = make_float4(vs[0], vs[1], vs[2], vs[3]);
      if (mirror) {
        uint2 pk;
        pk.x = pack2(f2bf(ws[0]), f2bf(ws[1]));
        pk.y = pack2(f2bf(ws[2]), f2bf(ws[3]));
        *(uint2*)(mirror + i0) = pk;
      }
    } else {
      for (long i = i0; i < n; i++) {
        float wi = w[i], mi = m[i], vi = v[i];
        adam_elem(wi, g[i], mi, vi, c, i >= n_nodecay);
        w[i] = wi;
        m[i] = mi;
        v[i] = vi;
        if (mirror) mirror[i] = f2bf(wi);
      }
    }
  }
}


// Engine::gather (lib.rs:1010-1028): y[r] = x[idx[r]] converted to y's dtype
__global__ void k_gather_rows(const void* x, int xd, long ldx, const int32_t* idx, void* y, int yd, long rows, long d) {
  const long total = rows * d;
  for (long i = blockIdx.x * (long)blockDim.x + threadIdx.x; i < total; i += (long)gridDim.x * blockDim.x) {
    const long r = i / d, c = i - r * d;
    store_from_f32(y, yd, i, load_as_f32(x, xd, (long)idx[r] * ldx + c));
  }
}

__global__ void k_zero_rows(float* x, long ldx, long rows, long d) {
  const long total = rows * d;
  for (long i = blockIdx.x * (long)blockDim.x + threadIdx.x; i < total; i += (long)gridDim.x * blockDim.x) {
    const long r = i / d, c = i - r * d;
    x[r * ldx + c] = 0.f;
  }
}

// Engine::gather_backward (lib.rs:1029-1050): dx = 0, then dx[idx[r]] += dy[r]
// for r in order (one thread per column: fixed order, repeated rows add up)
__global__ void k_gather_rows_bwd(const float* dy, const int32_t* idx, float* dx, long ldx, long rows, long d) {
  const long c = blockIdx.x * (long)blockDim.x + threadIdx.x;
  if (c >= d) return;
  for (long r = 0; r < rows; r++) dx[(long)idx[r] * ldx + c] += dy[r * d + c];
}

// common.py:28-30 bias_add: y[r][c] = x[r][c] + b[c]
__global__ void k_bias_add(const float* x, long ldx, const float* b, float* y, long ldy, long rows, long d) {
  const long total = rows * d;
  for (long i = blockIdx.x * (long)blockDim.x + threadIdx.x; i < total; i += (long)gridDim.x * blockDim.x) {
    const long r = i / d, c = i - r * d;
    y[r * ldy + c] = x[r * ldx + c] + b[c];
  }
}

// common.py:33-36 bias_reduce: y[c] = sum over rows in order of x[r][c] (fp32)
__global__ void k_bias_reduce(const float* x, long ldx, float* y, long rows, long d) {
  const long c = blockIdx.x * (long)blockDim.x + threadIdx.x;
  if (c >= d) return;
  float acc = 0.f;
  for (long r = 0; r < rows; r++) acc += x[r * ldx + c];
  y[c] = acc;
}

}  // namespace

// ---------------------------------------------------------------- C ABI

int sjh::split_planes(hipStream_t s, const float* x, long n, uint16_t* hi, uint16_t* lo) {
  SJ_REQUIRE(n >= 0 && n % 8 == 0 && (((uintptr_t)x | (uintptr_t)hi | (uintptr_t)lo) & 15) == 0,
             "split planes: n %ld (multiple of 8, 16-byte aligned buffers)", n);
  if (n == 0) return SJ_OK;
  hipLaunchKernelGGL(k_split_planes, dim3(ew_blocks(n / 8)), dim3(EW_THREADS), 0, s, x, n / 8, hi, lo);
  SJ_LAUNCH_CHECK("split planes");
  return SJ_OK;
}

extern "C" int sj_fill(void* stream, void* y, int dtype, long n, float value) {
  SJ_REQUIRE(dtype_ok(dtype) && n >= 0, "fill: dtype %d / n %ld", dtype, n);
  if (n == 0) return SJ_OK;
  hipLaunchKernelGGL(k_fill, dim3(ew_blocks(n)), dim3(EW_THREADS), 0, (hipStream_t)stream, y, dtype, n, value);
  SJ_LAUNCH_CHECK("fill");
  return SJ_OK;
}

extern "C" int sj_cast(void* stream, const void* x, int xd, void* y, int yd, long n) {
  SJ_REQUIRE(dtype_ok(xd) && dtype_ok(yd) && n >= 0, "cast: dtypes %d->%d", xd, yd);
  if (n == 0) return SJ_OK;
  if (xd == yd && ((uintptr_t)x | (uintptr_t)y) % 16 == 0) {
    // same dtype: a bit copy in 16-byte vectors, the last < 16 bytes below
    const long es = xd == SJ_BF16 ? 2 : 4, n16 = n * es / 16, done = n16 * 16 / es;
    if (n16 > 0) {
      hipLaunchKernelGGL(k_copy16, dim3(ew_blocks(n16)), dim3(EW_THREADS), 0, (hipStream_t)stream, (const uint4*)x,
                         (uint4*)y, n16);
      SJ_LAUNCH_CHECK("copy");
    }
    if (done == n) return SJ_OK;
    x = (const char*)x + done * es;
    y = (char*)y + done * es;
    n -= done;
  }
  hipLaunchKernelGGL(k_cast, dim3(ew_blocks(n)), dim3(EW_THREADS), 0, (hipStream_t)stream, x, xd, y, yd, n);
  SJ_LAUNCH_CHECK("cast");
  return SJ_OK;
}

extern "C" int sj_add(void* stream, const void* x, int xd, const void* z, int zd, void* y, int yd, long n,
                      float alpha) {
  SJ_REQUIRE(dtype_ok(xd) && dtype_ok(zd) && dtype_ok(yd) && n >= 0, "add shape mismatch");
  if (n == 0) return SJ_OK;
  hipLaunchKernelGGL(k_add, dim3(ew_blocks(n)), dim3(EW_THREADS), 0, (hipStream_t)stream, x, xd, z, zd, y, yd, n,
                     alpha);
  SJ_LAUNCH_CHECK("add");
  return SJ_OK;
}

extern "C" int sj_embedding_fwd(void* stream, const void* w, int wd, const int32_t* ids, void* y, int yd, long n,
                                long d) {
  SJ_REQUIRE(dtype_ok(wd) && dtype_ok(yd) && n >= 0 && d > 0, "embedding: dtype/shape");
  if (n == 0) return SJ_OK;
  hipLaunchKernelGGL(k_embedding_fwd, dim3(ew_blocks(n * d)), dim3(EW_THREADS), 0, (hipStream_t)stream, w, wd, ids,
                     y, yd, n, d);
  SJ_LAUNCH_CHECK("embedding");
  return SJ_OK;
}

extern "C" size_t sj_embedding_bwd_workspace_bytes(long n, long vocab) { return 0; }

// Faster form for d % 4 == 0, d <= 2048: each round scans 16 ids per thread
// (4096 tokens), compacts the matches in token order with one block scan,
// then every thread adds up to two float4 columns of the matching rows in
// that order (the same order, hence the same bits, as k_embedding_bwd).
constexpr int EMB_IDS = 16;
// sq (nullable): FP64 sum of squares of the row this workgroup stores, at
// sq[blockIdx.x] (the gradient-norm hook)
__global__ __launch_bounds__(EMB_THREADS) void k_embedding_bwd4(const float* __restrict__ dy,
                                                                const int32_t* __restrict__ ids,
                                                                float* __restrict__ dw, long n, long d, double* sq) {
  __shared__ int matches[EMB_THREADS * EMB_IDS];
  __shared__ int wave_total[EMB_THREADS / 64];
  const int v = blockIdx.x;
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const long d4 = d >> 2;
  float4 acc[2] = {make_float4(0.f, 0.f, 0.f, 0.f), make_float4(0.f, 0.f, 0.f, 0.f)};
  for (long base = 0; base < n; base += (long)EMB_THREADS * EMB_IDS) {
    const long i0 = base + (long)t * EMB_IDS;
    uint32_t hit = 0;
#pragma unroll
    for (int k = 0; k < EMB_IDS; k++)
      if (i0 + k < n && ids[i0 + k] == v) hit |= 1u << k;
    const int cnt = __popc(hit);
    int incl = cnt;  // inclusive scan over the wave
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int y = __shfl_up(incl, o, 64);
      if (lane >= o) incl += y;
    }
    if (lane == 63) wave_total[w] = incl;
    __syncthreads();
    int before = 0, total = 0;
#pragma unroll
    for (int j = 0; j < EMB_THREADS / 64; j++) {
      if (j < w) before += wave_total[j];
      total += wave_total[j];
    }
    int pos = before + incl - cnt;
    while (hit) {
      const int k = __ffs(hit) - 1;
      hit &= hit - 1;
      matches[pos++] = (int)(i0 + k);
    }
    __syncthreads();
#pragma unroll
    for (int c = 0; c < 2; c++) {
      const long col = t + (long)c * EMB_THREADS;
      if (col < d4) {
        const float4* src = (const float4*)dy + col;
        for (int m = 0; m < total; m++) {
          const float4 r = src[(long)matches[m] * d4];
          acc[c].x += r.x; acc[c].y += r.y; acc[c].z += r.z; acc[c].w += r.w;
        }
      }
    }
    __syncthreads();
  }
  double q = 0.0;
#pragma unroll
  for (int c = 0; c < 2; c++) {
    const long col = t + (long)c * EMB_THREADS;
    if (col < d4) {
      ((float4*)(dw + (long)v * d))[col] = acc[c];
      q += (double)acc[c].x * acc[c].x + (double)acc[c].y * acc[c].y + (double)acc[c].z * acc[c].z +
           (double)acc[c].w * acc[c].w;
    }
  }
  if (sq) {
    __shared__ double qred[EMB_THREADS / 64];
    q = block_sum<double, EMB_THREADS>(q, qred);
    if (t == 0) sq[blockIdx.x] = q;
  }
}

extern "C" int sj_embedding_bwd(void* stream, const float* dy, const int32_t* ids, float* dw, long n, long d,
                                long vocab, void* workspace, size_t workspace_bytes) {
  SJ_REQUIRE(n >= 0 && d > 0 && d <= 8 * EMB_THREADS && vocab > 0, "embedding_backward: n %ld d %ld vocab %ld", n,
             d, vocab);
  if (d % 4 == 0 && d <= 8 * EMB_THREADS && ((uintptr_t)dy & 15) == 0 && ((uintptr_t)dw & 15) == 0) {
    hipLaunchKernelGGL(k_embedding_bwd4, dim3((unsigned)vocab), dim3(EMB_THREADS), 0, (hipStream_t)stream, dy, ids, dw,
                       n, d, sjh::grad_sq().take(vocab));
  } else {
    hipLaunchKernelGGL(k_embedding_bwd, dim3((unsigned)vocab), dim3(EMB_THREADS), 0, (hipStream_t)stream, dy, ids, dw,
                       n, d);
    if (sjh::grad_sq().base && sjh::grad_sq().on) sjh::grad_sq().missed = true;
  }
  SJ_LAUNCH_CHECK("embedding_backward");
  return SJ_OK;
}

namespace sjh {
int rope_table(hipStream_t stream, float* table, long t, long head_dim, double theta) {
  long half = head_dim / 2;
  hipLaunchKernelGGL(k_rope_table, dim3(ew_blocks(t * half)), dim3(EW_THREADS), 0, stream, table, t, half, head_dim,
                     theta);
  SJ_LAUNCH_CHECK("rope_table");
  return SJ_OK;
}
}  // namespace sjh

extern "C" int sj_rope_table(void* stream, float* table, long t, long head_dim, float theta) {
  SJ_REQUIRE(t > 0 && head_dim > 0 && head_dim % 2 == 0 && theta > 0, "rope_table: t %ld head_dim %ld", t, head_dim);
  return sjh::rope_table((hipStream_t)stream, table, t, head_dim, (double)theta);
}

extern "C" int sj_rope(void* stream, const void* x, void* y, int dtype, long rows, long ld, long t, long heads,
                       long head_dim, long offset, float theta, int inverse) {
  SJ_REQUIRE(dtype_ok(dtype) && rows >= 0 && t > 0 && heads > 0 && head_dim % 2 == 0 && ld >= heads * head_dim,
             "rope: shape");
  long total = rows * heads * (head_dim / 2);
  if (total == 0) return SJ_OK;
  hipLaunchKernelGGL(k_rope, dim3(ew_blocks(total)), dim3(EW_THREADS), 0, (hipStream_t)stream, x, y, dtype, rows, ld,
                     t, heads, head_dim, offset, (double)theta, inverse);
  SJ_LAUNCH_CHECK("rope");
  return SJ_OK;
}

extern "C" int sj_swiglu_fwd(void* stream, const void* g, const void* u, void* h, int dtype, long n) {
  SJ_REQUIRE(dtype_ok(dtype) && n >= 0, "SwiGLU shape mismatch");
  if (n == 0) return SJ_OK;
  hipLaunchKernelGGL(k_swiglu_fwd, dim3(ew_blocks(n)), dim3(EW_THREADS), 0, (hipStream_t)stream, g, u, h, dtype, n);
  SJ_LAUNCH_CHECK("swiglu");
  return SJ_OK;
}

extern "C" int sj_swiglu_bwd(void* stream, const void* g, const void* u, int dt, const float* dy, float* dg,
                             float* du, long n) {
  SJ_REQUIRE(dtype_ok(dt) && n >= 0, "swiglu_backward shape");
  if (n == 0) return SJ_OK;
  hipLaunchKernelGGL(k_swiglu_bwd, dim3(ew_blocks(n)), dim3(EW_THREADS), 0, (hipStream_t)stream, g, u, dt, dy, dg,
                     du, n);
  SJ_LAUNCH_CHECK("swiglu_backward");
  return SJ_OK;
}

extern "C" int sj_cross_entropy(void* stream, const float* x, long ldx, const int32_t* targets, float* loss,
                                float* dx, long lddx, long rows, long vocab, const float* dy, float dy_scalar) {
  SJ_REQUIRE(rows >= 0 && vocab > 0 && ldx >= vocab && (!dx || lddx >= vocab), "cross entropy row mismatch");
  if (rows == 0) return SJ_OK;
  hipLaunchKernelGGL(k_cross_entropy, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, (hipStream_t)stream, x, ldx,
                     targets, loss, dx, lddx, rows, vocab, dy, dy_scalar);
  SJ_LAUNCH_CHECK("cross_entropy");
  return SJ_OK;
}

int sjh::cross_entropy_planes(void* stream, const float* x, long ldx, const int32_t* targets, float* loss,
                              uint16_t* dx_hi, uint16_t* dx_lo, long ldp, long rows, long vocab, float dy_scalar) {
  SJ_REQUIRE(rows >= 0 && vocab > 0 && ldx >= vocab && ldp >= vocab && dx_hi && dx_lo,
             "cross entropy (planes) row mismatch");
  if (rows == 0) return SJ_OK;
  hipLaunchKernelGGL(k_cross_entropy_planes, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, (hipStream_t)stream, x,
                     ldx, targets, loss, (bf16_t*)dx_hi, (bf16_t*)dx_lo, ldp, rows, vocab, ldp, dy_scalar);
  SJ_LAUNCH_CHECK("cross_entropy");
  return SJ_OK;
}

extern "C" int sj_loss_summary(void* stream, const float* loss, long n, double* out, long slot, float weight) {
  SJ_REQUIRE(n > 0 && slot >= 0, "loss_summary: n %ld", n);
  hipLaunchKernelGGL(k_loss_summary, dim3(1), dim3(256), 0, (hipStream_t)stream, loss, n, out, slot, weight);
  SJ_LAUNCH_CHECK("loss_summary");
  return SJ_OK;
}

// one workgroup of 1024 threads, each summing eight neighbouring slots per
// trip with all eight loads in flight, then a fixed-order block sum
__global__ __launch_bounds__(1024) void k_sum_slots(const double* __restrict__ slots, long count, double* out) {
  __shared__ double red[16];
  double s = 0.0;
  for (long i0 = 8L * threadIdx.x; i0 < count; i0 += 8L * 1024) {
    double v[8];
#pragma unroll
    for (int u = 0; u < 8; u++) v[u] = i0 + u < count ? slots[i0 + u] : 0.0;
#pragma unroll
    for (int u = 0; u < 8; u++) s += v[u];
  }
  s = block_sum<double, 1024>(s, red);
  if (threadIdx.x == 0) out[0] = s;
}

int sjh::sum_slots(hipStream_t stream, const double* slots, long count, double* out) {
  SJ_REQUIRE(slots && out && count > 0 && count < (1L << 30), "sum_slots: %ld slots", count);
  hipLaunchKernelGGL(k_sum_slots, dim3(1), dim3(1024), 0, stream, slots, count, out);
  SJ_LAUNCH_CHECK("sum_slots");
  return SJ_OK;
}

extern "C" size_t sj_sum_squares_workspace_bytes(long n) { return sizeof(double) * (size_t)ss_blocks(n); }

extern "C" int sj_sum_squares(void* stream, const float* g, long n, double* out, void* workspace,
                              size_t workspace_bytes) {
  SJ_REQUIRE(n >= 0, "sum_squares: n %ld", n);
  int blocks = ss_blocks(n);
  if (workspace_bytes < sizeof(double) * (size_t)blocks || !workspace)
    return sjh::fail(SJ_ERR_CAPACITY, "sum_squares: required %zu bytes, available %zu bytes",
                     sizeof(double) * (size_t)blocks, workspace_bytes);
  hipLaunchKernelGGL(k_sumsq_partial, dim3(blocks), dim3(SS_THREADS), 0, (hipStream_t)stream, g, n,
                     (double*)workspace);
  hipLaunchKernelGGL(k_sumsq_final, dim3(1), dim3(SS_THREADS), 0, (hipStream_t)stream, (const double*)workspace,
                     blocks, out);
  SJ_LAUNCH_CHECK("sum_squares");
  return SJ_OK;
}

extern "C" int sj_adamw(void* stream, float* w, const float* g, float* m, float* v, long n, float lr, float b1,
                        float b2, float eps, float decay, float ib1, float ib2, float scale) {
  SJ_REQUIRE(n >= 0, "adamw: n %ld", n);
  if (n == 0) return SJ_OK;
  hipLaunchKernelGGL(k_adamw, dim3(ew_blocks(n)), dim3(EW_THREADS), 0, (hipStream_t)stream, w, g, m, v, n, lr, b1,
                     b2, eps, decay, ib1, ib2, scale);
  SJ_LAUNCH_CHECK("adamw");
  return SJ_OK;
}

extern "C" int sj_adamw_multi(void* stream, float* w, const float* g, float* m, float* v, uint16_t* mirror, long n,
                              long n_nodecay, const sj_adam_step* step, const double* sumsq, int32_t* status) {
  SJ_REQUIRE(n >= 0 && n_nodecay >= 0 && n_nodecay <= n && step && sumsq && status, "adamw_multi: arguments");
  if (n == 0) return SJ_OK;
  SJ_REQUIRE(((uintptr_t)w | (uintptr_t)g | (uintptr_t)m | (uintptr_t)v) % 16 == 0 && (!mirror || (uintptr_t)mirror % 8 == 0),
             "adamw_multi: arena pointers must be 16-byte aligned");
  long quads = (n + 3) / 4;
  hipLaunchKernelGGL(k_adamw_multi, dim3(ew_blocks(quads)), dim3(256), 0, (hipStream_t)stream, w, g, m, v,
                     (bf16_t*)mirror, n, n_nodecay, step, sumsq, status);
  SJ_LAUNCH_CHECK("adamw_multi");
  return SJ_OK;
}

extern "C" int sj_gather_rows(void* stream, const void* x, int xd, long ldx, const int32_t* idx, long rows, long d,
                              void* y, int yd) {
  SJ_REQUIRE(x && idx && y && rows >= 0 && d > 0 && ldx >= d && dtype_ok(xd) && dtype_ok(yd), "gather: arguments");
  if (rows == 0) return SJ_OK;
  hipLaunchKernelGGL(k_gather_rows, dim3(ew_blocks(rows * d)), dim3(EW_THREADS), 0, (hipStream_t)stream, x, xd, ldx,
                     idx, y, yd, rows, d);
  SJ_LAUNCH_CHECK("gather");
  return SJ_OK;
}

extern "C" int sj_gather_rows_bwd(void* stream, const float* dy, const int32_t* idx, long rows, long d, float* dx,
                                  long ldx, long n) {
  SJ_REQUIRE(dy && idx && dx && rows >= 0 && d > 0 && ldx >= d && n > 0, "gather_backward: arguments");
  hipStream_t s = (hipStream_t)stream;
  // zero dx with a kernel (not a memset: the call may sit in a captured graph)
  hipLaunchKernelGGL(k_zero_rows, dim3(ew_blocks(n * d)), dim3(EW_THREADS), 0, s, dx, ldx, n, d);
  SJ_LAUNCH_CHECK("gather_backward");
  if (rows == 0) return SJ_OK;
  hipLaunchKernelGGL(k_gather_rows_bwd, dim3((unsigned)((d + EW_THREADS - 1) / EW_THREADS)), dim3(EW_THREADS), 0, s, dy,
                     idx, dx, ldx, rows, d);
  SJ_LAUNCH_CHECK("gather_backward");
  return SJ_OK;
}

extern "C" int sj_bias_add(void* stream, const float* x, long ldx, const float* bias, float* y, long ldy, long rows,
                           long d) {
  SJ_REQUIRE(x && bias && y && rows >= 0 && d > 0 && ldx >= d && ldy >= d, "affine bias shape mismatch");
  if (rows == 0) return SJ_OK;
  hipLaunchKernelGGL(k_bias_add, dim3(ew_blocks(rows * d)), dim3(EW_THREADS), 0, (hipStream_t)stream, x, ldx, bias, y,
                     ldy, rows, d);
  SJ_LAUNCH_CHECK("bias_add");
  return SJ_OK;
}

extern "C" int sj_bias_reduce(void* stream, const float* x, long ldx, long rows, long d, float* y) {
  SJ_REQUIRE(x && y && rows >= 0 && d > 0 && ldx >= d, "bias gradient shape mismatch");
  hipLaunchKernelGGL(k_bias_reduce, dim3((unsigned)((d + EW_THREADS - 1) / EW_THREADS)), dim3(EW_THREADS), 0,
                     (hipStream_t)stream, x, ldx, y, rows, d);
  SJ_LAUNCH_CHECK("bias_reduce");
  return SJ_OK;
}
