// RMSNorm forward and backward (kernels.py:54-87, norm_ops.rs:14-71).
// One wavefront per row; each lane owns column pairs lane + 64*j, so loads
// are 4-byte (bf16x2) or 8-byte (f32x2) coalesced.  The backward writes dx
// per row and a per-workgroup dw partial, reduced in a second fixed-order
// pass (deterministic, no atomics -- the reference's partial/reduce split).
#include <math.h>

#include <mutex>

#include "common.h"

using namespace sj;

namespace {

constexpr int NT = 256;         // 4 waves
constexpr int MAXP = 16;        // column pairs per lane: d <= 2048
constexpr int BWD_ROWS = 16;    // rows per workgroup in the backward (4 per wave)

template <int XD>
__device__ __forceinline__ float2 ld2(const void* p, long i) {  // i even
  if constexpr (XD == SJ_BF16) {
    uint32_t u = *(const uint32_t*)((const bf16_t*)p + i);
    return make_float2(bf2f((bf16_t)(u & 0xffff)), bf2f((bf16_t)(u >> 16)));
  } else {
    return *(const float2*)((const float*)p + i);
  }
}
template <int XD>
__device__ __forceinline__ void st2(void* p, long i, float a, float b) {
  if constexpr (XD == SJ_BF16) {
    *(uint32_t*)((bf16_t*)p + i) = pack2(f2bf(a), f2bf(b));
  } else {
    *(float2*)((float*)p + i) = make_float2(a, b);
  }
}

template <int XD, int WD>
__global__ __launch_bounds__(NT) void k_rms_fwd(const void* __restrict__ x, const void* __restrict__ w,
                                                void* __restrict__ y, long rows, long d, float eps) {
  const int lane = threadIdx.x & 63;
  const long r = blockIdx.x * 4L + (threadIdx.x >> 6);
  if (r >= rows) return;
  const long pairs = d >> 1;
  float2 xv[MAXP];
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < MAXP; j++) {
    long p = lane + 64L * j;
    if (p < pairs) {
      xv[j] = ld2<XD>(x, r * d + 2 * p);
      s += xv[j].x * xv[j].x + xv[j].y * xv[j].y;
    }
  }
  s = wave_sum(s);
  const float inv = 1.f / sqrtf(s / (float)d + eps);
#pragma unroll
  for (int j = 0; j < MAXP; j++) {
    long p = lane + 64L * j;
    if (p < pairs) {
      float2 wv = ld2<WD>(w, 2 * p);
      st2<XD>(y, r * d + 2 * p, xv[j].x * inv * wv.x, xv[j].y * inv * wv.y);
    }
  }
}

template <int XD, int WD>
__global__ __launch_bounds__(NT) void k_rms_bwd(const void* __restrict__ x, const void* __restrict__ w,
                                                const float* __restrict__ dy, const float* __restrict__ dx_acc,
                                                float* __restrict__ dx, float* __restrict__ partial, long rows,
                                                long d, float eps) {
  __shared__ float red[4][2 * MAXP * 64];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const long pairs = d >> 1;
  float2 dwp[MAXP];
  float2 wreg[MAXP];
#pragma unroll
  for (int j = 0; j < MAXP; j++) {
    dwp[j] = make_float2(0.f, 0.f);
    long p = lane + 64L * j;
    if (p < pairs) wreg[j] = ld2<WD>(w, 2 * p);
  }
  const long r0 = blockIdx.x * (long)BWD_ROWS;
  for (int rr = wv; rr < BWD_ROWS; rr += 4) {
    const long r = r0 + rr;
    if (r >= rows) break;
    float2 xv[MAXP], gv[MAXP];
    float s = 0.f, sdx = 0.f;
#pragma unroll
    for (int j = 0; j < MAXP; j++) {
      long p = lane + 64L * j;
      if (p < pairs) {
        xv[j] = ld2<XD>(x, r * d + 2 * p);
        gv[j] = *(const float2*)(dy + r * d + 2 * p);
        s += xv[j].x * xv[j].x + xv[j].y * xv[j].y;
        sdx += gv[j].x * wreg[j].x * xv[j].x + gv[j].y * wreg[j].y * xv[j].y;
      }
    }
    s = wave_sum(s);
    sdx = wave_sum(sdx);
    const float inv = rsqrtf(s / (float)d + eps);
    const float c = (sdx / (float)d) * inv * inv;
#pragma unroll
    for (int j = 0; j < MAXP; j++) {
      long p = lane + 64L * j;
      if (p < pairs) {
        float a = inv * (gv[j].x * wreg[j].x - xv[j].x * c);
        float b = inv * (gv[j].y * wreg[j].y - xv[j].y * c);
        if (dx_acc) {
          float2 acc = *(const float2*)(dx_acc + r * d + 2 * p);
          a = acc.x + a;
          b = acc.y + b;
        }
        *(float2*)(dx + r * d + 2 * p) = make_float2(a, b);
        dwp[j].x += gv[j].x * xv[j].x * inv;
        dwp[j].y += gv[j].y * xv[j].y * inv;
      }
    }
  }
  // reduce the 4 waves' partials through LDS, fixed order
#pragma unroll
  for (int j = 0; j < MAXP; j++) {
    long p = lane + 64L * j;
    if (p < pairs) {
      red[wv][2 * p] = dwp[j].x;
      red[wv][2 * p + 1] = dwp[j].y;
    }
  }
  __syncthreads();
  for (long c = threadIdx.x; c < d; c += NT)
    partial[blockIdx.x * d + c] = ((red[0][c] + red[1][c]) + red[2][c]) + red[3][c];
}

// rmsnorm_backward_reduce (kernels.py:79-87): dw[c] = sum_g partial[g][c].
// 32 columns x 8 group-slices per workgroup; each thread keeps 4 independent
// accumulators so the loads overlap; slices are combined in fixed order.
__global__ __launch_bounds__(NT) void k_rms_reduce(const float* __restrict__ partial, float* __restrict__ dw,
                                                   long groups, long d) {
  __shared__ float red[8][32];
  const int col = threadIdx.x & 31, sl = threadIdx.x >> 5;
  const long c = blockIdx.x * 32L + col;
  float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
  if (c < d) {
    long g = sl;
    for (; g + 24 < groups; g += 32) {
      a0 += partial[g * d + c];
      a1 += partial[(g + 8) * d + c];
      a2 += partial[(g + 16) * d + c];
      a3 += partial[(g + 24) * d + c];
    }
    for (; g < groups; g += 8) a0 += partial[g * d + c];
  }
  red[sl][col] = (a0 + a1) + (a2 + a3);
  __syncthreads();
  if (sl == 0 && c < d) {
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 8; i++) s += red[i][col];
    dw[c] = s;
  }
}


// Many reductions in one launch (blockIdx.y = job): the norm-weight
// gradients of a whole backward, summed after the dX chain has passed.
// sq (nullable): FP64 sum of squares of the workgroup's dw values at
// sq[blockIdx.y * gridDim.x + blockIdx.x] (the gradient-norm hook)
__global__ __launch_bounds__(NT) void k_rms_reduce_multi(const sj::RmsReduceJob* __restrict__ jobs, double* sq) {
  const sj::RmsReduceJob jb = jobs[blockIdx.y];
  __shared__ float red[8][32];
  __shared__ double qred[NT / 64];
  const int col = threadIdx.x & 31, sl = threadIdx.x >> 5;
  const long c = blockIdx.x * 32L + col;
  if (blockIdx.x * 32L >= jb.d) {  // whole workgroup past this job's columns
    if (sq && threadIdx.x == 0) sq[blockIdx.y * gridDim.x + blockIdx.x] = 0.0;
    return;
  }
  float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
  const long groups = jb.groups, d = jb.d;
  const float* partial = jb.partial;
  if (c < d) {
    long g = sl;
    for (; g + 24 < groups; g += 32) {
      a0 += partial[g * d + c];
      a1 += partial[(g + 8) * d + c];
      a2 += partial[(g + 16) * d + c];
      a3 += partial[(g + 24) * d + c];
    }
    for (; g < groups; g += 8) a0 += partial[g * d + c];
  }
  red[sl][col] = (a0 + a1) + (a2 + a3);
  __syncthreads();
  double q = 0.0;
  if (sl == 0 && c < d) {
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 8; i++) s += red[i][col];
    jb.dw[c] = s;
    q = (double)s * (double)s;
  }
  if (sq) {
    q = block_sum<double, NT>(q, qred);
    if (threadIdx.x == 0) sq[blockIdx.y * gridDim.x + blockIdx.x] = q;
  }
}

// ----------------------------------------------------- MFMA-layout variants
// Row blocks of TR = 16 rows on 16 waves, one row per wave, so every row's
// loads are in flight at once; lanes own column pairs lane + 64 j, j < NP.
// The block stages its bf16 outputs in LDS and also writes them transposed
// ([d][rows], 32-byte column segments), the layout the dW GEMMs stream.
// Row blocks are ordered so each XCD (workgroup b runs on XCD b % 8) takes a
// contiguous run of them: neighbouring column segments then meet in one L2
// and leave it as whole lines.
constexpr int TR = 16;
constexpr int NTT = 1024;

__device__ __forceinline__ long xcd_block(long b, long nb) {
  const long xcd = b & 7, local = b >> 3, q = nb >> 3, r = nb & 7;
  return xcd * q + (xcd < r ? xcd : r) + local;
}

// 8 rows (row stride d in LDS) of column c -> one 16-byte store, or
// element stores at the ragged end
__device__ __forceinline__ void store_col8(bf16_t* dst, const bf16_t* src, long d, long c, long rbase, long rows) {
  bf16_t v[8];
#pragma unroll
  for (int i = 0; i < 8; i++) v[i] = src[i * d + c];
  if (rbase + 8 <= rows) {
    *(u32x4*)dst = u32x4{pack2(v[0], v[1]), pack2(v[2], v[3]), pack2(v[4], v[5]), pack2(v[6], v[7])};
  } else {
    for (int i = 0; i < 8; i++)
      if (rbase + i < rows) dst[i] = v[i];
  }
}

// y = rmsnorm(x) (bf16 x, w) -> y [rows][d] and y_t [d][ldt].  With ids,
// row r of x is row ids[r] of the table x (the embedding lookup), and xout
// receives the looked-up rows (the residual stream's input).
template <int NP>
__global__ __launch_bounds__(NTT) void k_rms_fwd_t(const bf16_t* __restrict__ x, const bf16_t* __restrict__ w,
                                                   bf16_t* __restrict__ y, bf16_t* __restrict__ yt, long rows,
                                                   long d, long ldt, float eps, const int32_t* __restrict__ ids,
                                                   bf16_t* __restrict__ xout) {
  extern __shared__ __attribute__((aligned(16))) bf16_t stage[];  // [TR][d]
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const long r0 = xcd_block(blockIdx.x, gridDim.x) * TR;
  const long pairs = d >> 1;
  const long r = r0 + wv;
  // the weight pairs are loaded with the row, so no second global-load
  // latency follows the row reduction
  float2 xv[NP], wt[NP];
  float s = 0.f;
  const long src = r < rows ? (ids ? (long)ids[r] : r) * d : 0;
#pragma unroll
  for (int j = 0; j < NP; j++) {
    const long p = lane + 64L * j;
    xv[j] = wt[j] = make_float2(0.f, 0.f);
    if (p < pairs) wt[j] = ld2<SJ_BF16>(w, 2 * p);
    if (p < pairs && r < rows) {
      xv[j] = ld2<SJ_BF16>(x, src + 2 * p);
      s += xv[j].x * xv[j].x + xv[j].y * xv[j].y;
    }
  }
  if (xout && r < rows) {
#pragma unroll
    for (int j = 0; j < NP; j++) {
      const long p = lane + 64L * j;
      if (p < pairs) *(uint32_t*)(xout + r * d + 2 * p) = pack2(f2bf(xv[j].x), f2bf(xv[j].y));
    }
  }
  s = wave_sum(s);
  const float inv = 1.f / sqrtf(s / (float)d + eps);
#pragma unroll
  for (int j = 0; j < NP; j++) {
    const long p = lane + 64L * j;
    if (p < pairs) {
      const float2 w2 = wt[j];
      const uint32_t pk = r < rows ? pack2(f2bf(xv[j].x * inv * w2.x), f2bf(xv[j].y * inv * w2.y)) : 0u;
      if (r < rows) *(uint32_t*)(y + r * d + 2 * p) = pk;
      *(uint32_t*)(stage + wv * d + 2 * p) = pk;
    }
  }
  if (!yt) return;  // no transposed output: the block is done (uniform)
  __syncthreads();
  for (long q = threadIdx.x; q < 2 * d; q += NTT) {
    const long c = q >> 1;
    const int ch = (int)(q & 1);
    const long rbase = r0 + ch * 8;
    store_col8(yt + c * ldt + rbase, stage + ch * 8 * d, d, c, rbase, rows);
  }
}

// backward with hi/lo plane outputs of dx (normal and transposed) next to the
// fp32 dx; dw partial per 16-row block (fixed-order sum of its rows)
template <int NP>
__global__ __launch_bounds__(NTT) void k_rms_bwd_p(const bf16_t* __restrict__ x, const bf16_t* __restrict__ w,
                                                   const float* __restrict__ dy, const float* __restrict__ dx_acc,
                                                   float* __restrict__ dx, bf16_t* __restrict__ hi,
                                                   bf16_t* __restrict__ lo, bf16_t* __restrict__ hit,
                                                   bf16_t* __restrict__ lot, float* __restrict__ partial, long rows,
                                                   long d, long ldt, float eps) {
  extern __shared__ __attribute__((aligned(16))) bf16_t stage[];  // hi [TR][d], lo [TR][d], red [TR][d] f32
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const long pairs = d >> 1;
  bf16_t* shi = stage;
  bf16_t* slo = stage + TR * d;
  float* red = (float*)(stage + 2 * TR * d);
  const long blk = xcd_block(blockIdx.x, gridDim.x);
  const long r0 = blk * TR;
  const long r = r0 + wv;
  const bool ok = r < rows;
  float2 xv[NP], gv[NP], wr[NP], av[NP];
  float s = 0.f, sdx = 0.f;
#pragma unroll
  for (int j = 0; j < NP; j++) {
    const long p = lane + 64L * j;
    xv[j] = gv[j] = wr[j] = av[j] = make_float2(0.f, 0.f);
    if (p < pairs) {
      wr[j] = ld2<SJ_BF16>(w, 2 * p);
      if (ok) {
        xv[j] = ld2<SJ_BF16>(x, r * d + 2 * p);
        gv[j] = *(const float2*)(dy + r * d + 2 * p);
        if (dx_acc) av[j] = *(const float2*)(dx_acc + r * d + 2 * p);
      }
    }
  }
#pragma unroll
  for (int j = 0; j < NP; j++) {
    s += xv[j].x * xv[j].x + xv[j].y * xv[j].y;
    sdx += gv[j].x * wr[j].x * xv[j].x + gv[j].y * wr[j].y * xv[j].y;
  }
  s = wave_sum(s);
  sdx = wave_sum(sdx);
  const float inv = rsqrtf(s / (float)d + eps);
  const float cc = (sdx / (float)d) * inv * inv;
#pragma unroll
  for (int j = 0; j < NP; j++) {
    const long p = lane + 64L * j;
    if (p < pairs) {
      uint32_t ph = 0u, pl = 0u;
      float2 dwv = make_float2(0.f, 0.f);
      if (ok) {
        float a = inv * (gv[j].x * wr[j].x - xv[j].x * cc);
        float b = inv * (gv[j].y * wr[j].y - xv[j].y * cc);
        if (dx_acc) {
          a = av[j].x + a;
          b = av[j].y + b;
        }
        *(float2*)(dx + r * d + 2 * p) = make_float2(a, b);
        dwv = make_float2(gv[j].x * xv[j].x * inv, gv[j].y * xv[j].y * inv);
        bf16_t ha, la, hb, lb;
        split_bf(a, ha, la);
        split_bf(b, hb, lb);
        ph = pack2(ha, hb);
        pl = pack2(la, lb);
        if (hi) {  // row-layout planes (optional)
          *(uint32_t*)(hi + r * d + 2 * p) = ph;
          *(uint32_t*)(lo + r * d + 2 * p) = pl;
        }
      }
      *(uint32_t*)(shi + wv * d + 2 * p) = ph;
      *(uint32_t*)(slo + wv * d + 2 * p) = pl;
      *(float2*)(red + wv * d + 2 * p) = dwv;
    }
  }
  __syncthreads();
  for (long c = threadIdx.x; c < d; c += NTT) {
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < TR; i++) acc += red[i * d + c];
    partial[blk * d + c] = acc;
  }
  for (long q = threadIdx.x; hit && q < 4 * d; q += NTT) {  // transposed planes (optional)
    const int plane = q >= 2 * d;
    const long qq = plane ? q - 2 * d : q;
    const long c = qq >> 1;
    const int ch = (int)(qq & 1);
    const long rbase = r0 + ch * 8;
    store_col8((plane ? lot : hit) + c * ldt + rbase, (plane ? slo : shi) + ch * 8 * d, d, c, rbase, rows);
  }
}

inline bool dt_ok(int dt) { return dt == SJ_F32 || dt == SJ_BF16; }

template <int XD, int WD>
void launch_fwd(hipStream_t s, const void* x, const void* w, void* y, long rows, long d, float eps) {
  hipLaunchKernelGGL((k_rms_fwd<XD, WD>), dim3((unsigned)((rows + 3) / 4)), dim3(NT), 0, s, x, w, y, rows, d, eps);
}
template <int XD, int WD>
void launch_bwd(hipStream_t s, const void* x, const void* w, const float* dy, const float* acc, float* dx,
                float* partial, long rows, long d, float eps) {
  long groups = (rows + BWD_ROWS - 1) / BWD_ROWS;
  hipLaunchKernelGGL((k_rms_bwd<XD, WD>), dim3((unsigned)groups), dim3(NT), 0, s, x, w, dy, acc, dx, partial, rows, d,
                     eps);
}

}  // namespace

extern "C" int sj_rmsnorm_fwd(void* stream, const void* x, int xd, const void* w, int wd, void* y, long rows, long d,
                              float eps) {
  SJ_REQUIRE(dt_ok(xd) && dt_ok(wd), "RMSNorm dtype %d/%d", xd, wd);
  SJ_REQUIRE(rows >= 0 && d > 0 && d % 2 == 0 && d <= 2 * 64 * MAXP, "RMSNorm weight mismatch (d %ld)", d);
  if (rows == 0) return SJ_OK;
  hipStream_t s = (hipStream_t)stream;
  if (xd == SJ_BF16 && wd == SJ_BF16) launch_fwd<SJ_BF16, SJ_BF16>(s, x, w, y, rows, d, eps);
  else if (xd == SJ_BF16) launch_fwd<SJ_BF16, SJ_F32>(s, x, w, y, rows, d, eps);
  else if (wd == SJ_BF16) launch_fwd<SJ_F32, SJ_BF16>(s, x, w, y, rows, d, eps);
  else launch_fwd<SJ_F32, SJ_F32>(s, x, w, y, rows, d, eps);
  SJ_LAUNCH_CHECK("rmsnorm");
  return SJ_OK;
}

extern "C" size_t sj_rmsnorm_bwd_workspace_bytes(long rows, long d) {
  return sizeof(float) * (size_t)((rows + BWD_ROWS - 1) / BWD_ROWS) * (size_t)d;
}

extern "C" int sj_rmsnorm_bwd(void* stream, const void* x, int xd, const void* w, int wd, const float* dy,
                              const float* dx_acc, float* dx, float* dw, long rows, long d, float eps, void* workspace,
                              size_t workspace_bytes) {
  SJ_REQUIRE(dt_ok(xd) && dt_ok(wd), "RMSNorm backward dtype %d/%d", xd, wd);
  SJ_REQUIRE(rows > 0 && d > 0 && d % 2 == 0 && d <= 2 * 64 * MAXP, "RMSNorm backward shape (rows %ld d %ld)", rows, d);
  size_t need = sj_rmsnorm_bwd_workspace_bytes(rows, d);
  if (!workspace || workspace_bytes < need)
    return sjh::fail(SJ_ERR_CAPACITY, "rmsnorm_backward: required %zu bytes, available %zu bytes", need,
                     workspace_bytes);
  hipStream_t s = (hipStream_t)stream;
  float* partial = (float*)workspace;
  if (xd == SJ_BF16 && wd == SJ_BF16) launch_bwd<SJ_BF16, SJ_BF16>(s, x, w, dy, dx_acc, dx, partial, rows, d, eps);
  else if (xd == SJ_BF16) launch_bwd<SJ_BF16, SJ_F32>(s, x, w, dy, dx_acc, dx, partial, rows, d, eps);
  else if (wd == SJ_BF16) launch_bwd<SJ_F32, SJ_BF16>(s, x, w, dy, dx_acc, dx, partial, rows, d, eps);
  else launch_bwd<SJ_F32, SJ_F32>(s, x, w, dy, dx_acc, dx, partial, rows, d, eps);
  long groups = (rows + BWD_ROWS - 1) / BWD_ROWS;
  hipLaunchKernelGGL(k_rms_reduce, dim3((unsigned)((d + 31) / 32)), dim3(NT), 0, s, partial, dw, groups, d);
  SJ_LAUNCH_CHECK("rmsnorm_backward");
  return SJ_OK;
}

// Allow the plane variants up to 160 KB of dynamic LDS (d <= 1024); run
// once, outside any stream capture (sj_model_create calls it).
namespace {
template <int NP>
hipError_t set_np_attrs() {
  hipError_t e = hipFuncSetAttribute((const void*)k_rms_bwd_p<NP>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                     160 * 1024);
  if (e == hipSuccess)
    e = hipFuncSetAttribute((const void*)k_rms_fwd_t<NP>, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
  return e;
}
}  // namespace

namespace sjh {
int norm_prepare() {
  static int done = 0, status = SJ_OK;
  if (done) return status;
  done = 1;
  hipError_t e = set_np_attrs<1>();
  if (e == hipSuccess) e = set_np_attrs<2>();
  if (e == hipSuccess) e = set_np_attrs<3>();
  if (e == hipSuccess) e = set_np_attrs<4>();
  if (e == hipSuccess) e = set_np_attrs<5>();
  if (e == hipSuccess) e = set_np_attrs<6>();
  if (e == hipSuccess) e = set_np_attrs<7>();
  if (e == hipSuccess) e = set_np_attrs<8>();
  status = e == hipSuccess ? SJ_OK : sjh::hip_check(e, "rmsnorm: LDS attribute");
  return status;
}
}  // namespace sjh

namespace {
template <int NP>
void launch_fwd_t(hipStream_t s, unsigned blocks, size_t lds, const uint16_t* x, const uint16_t* w, uint16_t* y,
                  uint16_t* y_t, long rows, long d, long ldt, float eps, const int32_t* ids = nullptr,
                  uint16_t* xout = nullptr) {
  hipLaunchKernelGGL(k_rms_fwd_t<NP>, dim3(blocks), dim3(NTT), lds, s, (const bf16_t*)x, (const bf16_t*)w, (bf16_t*)y,
                     (bf16_t*)y_t, rows, d, ldt, eps, ids, (bf16_t*)xout);
}
template <int NP>
void launch_bwd_p(hipStream_t s, unsigned blocks, size_t lds, const uint16_t* x, const uint16_t* w, const float* dy,
                  const float* dx_acc, float* dx, uint16_t* hi, uint16_t* lo, uint16_t* hit, uint16_t* lot,
                  float* partial, long rows, long d, long ldt, float eps) {
  hipLaunchKernelGGL(k_rms_bwd_p<NP>, dim3(blocks), dim3(NTT), lds, s, (const bf16_t*)x, (const bf16_t*)w, dy, dx_acc,
                     dx, (bf16_t*)hi, (bf16_t*)lo, (bf16_t*)hit, (bf16_t*)lot, partial, rows, d, ldt, eps);
}
}  // namespace

static int rmsnorm_fwd_t_any(void* stream, const uint16_t* x, const uint16_t* w, uint16_t* y, uint16_t* y_t, long ldt,
                             long rows, long d, float eps, const int32_t* ids, uint16_t* xout) {
  SJ_REQUIRE(rows >= 0 && d > 0 && d % 8 == 0 && d <= 1024 && (!y_t || (ldt >= rows && ldt % 8 == 0)) &&
                 ((uintptr_t)y_t & 15) == 0,
             "RMSNorm (transposed output): rows %ld d %ld ldt %ld (d <= 1024)", rows, d, ldt);
  if (rows == 0) return SJ_OK;
  if (int st0 = sjh::norm_prepare()) return st0;
  const size_t lds = sizeof(bf16_t) * TR * (size_t)d;
  const unsigned blocks = (unsigned)((rows + TR - 1) / TR);
  hipStream_t s = (hipStream_t)stream;
  switch ((d / 2 + 63) / 64) {
    case 1: launch_fwd_t<1>(s, blocks, lds, x, w, y, y_t, rows, d, ldt, eps, ids, xout); break;
    case 2: launch_fwd_t<2>(s, blocks, lds, x, w, y, y_t, rows, d, ldt, eps, ids, xout); break;
    case 3: launch_fwd_t<3>(s, blocks, lds, x, w, y, y_t, rows, d, ldt, eps, ids, xout); break;
    case 4: launch_fwd_t<4>(s, blocks, lds, x, w, y, y_t, rows, d, ldt, eps, ids, xout); break;
    case 5: launch_fwd_t<5>(s, blocks, lds, x, w, y, y_t, rows, d, ldt, eps, ids, xout); break;
    case 6: launch_fwd_t<6>(s, blocks, lds, x, w, y, y_t, rows, d, ldt, eps, ids, xout); break;
    case 7: launch_fwd_t<7>(s, blocks, lds, x, w, y, y_t, rows, d, ldt, eps, ids, xout); break;
    default: launch_fwd_t<8>(s, blocks, lds, x, w, y, y_t, rows, d, ldt, eps, ids, xout); break;
  }
  SJ_LAUNCH_CHECK("rmsnorm_t");
  return SJ_OK;
}

extern "C" int sj_rmsnorm_fwd_t(void* stream, const uint16_t* x, const uint16_t* w, uint16_t* y, uint16_t* y_t,
                                long ldt, long rows, long d, float eps) {
  return rmsnorm_fwd_t_any(stream, x, w, y, y_t, ldt, rows, d, eps, nullptr, nullptr);
}

// the embedding lookup (Engine::embedding) fused into the first block's
// norm: row r of the input is row ids[r] of the bf16 table, written to x0
int sjh::rmsnorm_fwd_t_embed(void* stream, const uint16_t* table, const int32_t* ids, uint16_t* x0,
                             const uint16_t* w, uint16_t* y, uint16_t* y_t, long ldt, long rows, long d, float eps) {
  SJ_REQUIRE(table && ids && x0, "RMSNorm with the embedding lookup: table, ids and x0 required");
  return rmsnorm_fwd_t_any(stream, table, w, y, y_t, ldt, rows, d, eps, ids, x0);
}

// sj_rmsnorm_bwd_p without its dw reduce: the partial sums [groups][d]
// stay in `partial` for sjh::rmsnorm_reduce_multi
int sjh::rmsnorm_bwd_p_deferred(void* stream, const uint16_t* x, const uint16_t* w, const float* dy,
                                const float* dx_acc, float* dx, uint16_t* dx_hi, uint16_t* dx_lo, uint16_t* dx_t_hi,
                                uint16_t* dx_t_lo, long ldt, long rows, long d, float eps, float* partial) {
  SJ_REQUIRE(rows > 0 && d > 0 && d % 8 == 0 && d <= 1024 && partial && !dx_t_hi == !dx_t_lo && !dx_hi == !dx_lo &&
                 (!dx_t_hi || (ldt >= rows && ldt % 8 == 0)) && ((uintptr_t)dx_t_hi & 15) == 0 &&
                 ((uintptr_t)dx_t_lo & 15) == 0,
             "RMSNorm backward (planes): rows %ld d %ld ldt %ld (d <= 1024; planes both or neither)", rows, d, ldt);
  if (int st0 = sjh::norm_prepare()) return st0;
  hipStream_t s = (hipStream_t)stream;
  const long groups = (rows + TR - 1) / TR;
  const size_t lds = 2 * sizeof(bf16_t) * TR * (size_t)d + sizeof(float) * TR * (size_t)d;
  const unsigned blocks = (unsigned)groups;
  switch ((d / 2 + 63) / 64) {
    case 1: launch_bwd_p<1>(s, blocks, lds, x, w, dy, dx_acc, dx, dx_hi, dx_lo, dx_t_hi, dx_t_lo, partial, rows, d, ldt, eps); break;
    case 2: launch_bwd_p<2>(s, blocks, lds, x, w, dy, dx_acc, dx, dx_hi, dx_lo, dx_t_hi, dx_t_lo, partial, rows, d, ldt, eps); break;
    case 3: launch_bwd_p<3>(s, blocks, lds, x, w, dy, dx_acc, dx, dx_hi, dx_lo, dx_t_hi, dx_t_lo, partial, rows, d, ldt, eps); break;
    case 4: launch_bwd_p<4>(s, blocks, lds, x, w, dy, dx_acc, dx, dx_hi, dx_lo, dx_t_hi, dx_t_lo, partial, rows, d, ldt, eps); break;
    case 5: launch_bwd_p<5>(s, blocks, lds, x, w, dy, dx_acc, dx, dx_hi, dx_lo, dx_t_hi, dx_t_lo, partial, rows, d, ldt, eps); break;
    case 6: launch_bwd_p<6>(s, blocks, lds, x, w, dy, dx_acc, dx, dx_hi, dx_lo, dx_t_hi, dx_t_lo, partial, rows, d, ldt, eps); break;
    case 7: launch_bwd_p<7>(s, blocks, lds, x, w, dy, dx_acc, dx, dx_hi, dx_lo, dx_t_hi, dx_t_lo, partial, rows, d, ldt, eps); break;
    default: launch_bwd_p<8>(s, blocks, lds, x, w, dy, dx_acc, dx, dx_hi, dx_lo, dx_t_hi, dx_t_lo, partial, rows, d, ldt, eps); break;
  }
  SJ_LAUNCH_CHECK("rmsnorm_backward_p");
  return SJ_OK;
}

int sjh::rmsnorm_reduce_multi(void* stream, const sj::RmsReduceJob* jobs, long njobs, long max_d) {
  SJ_REQUIRE(jobs && njobs > 0 && njobs < 65536 && max_d > 0, "rmsnorm reduce: %ld jobs", njobs);
  const unsigned bx = (unsigned)((max_d + 31) / 32);
  double* sq = sjh::grad_sq().take((long)bx * njobs);
  hipLaunchKernelGGL(k_rms_reduce_multi, dim3(bx, (unsigned)njobs), dim3(NT), 0, (hipStream_t)stream, jobs, sq);
  SJ_LAUNCH_CHECK("rmsnorm_backward_reduce");
  return SJ_OK;
}

extern "C" size_t sj_rmsnorm_bwd_p_workspace_bytes(long rows, long d) {
  return sizeof(float) * (size_t)((rows + TR - 1) / TR) * (size_t)d;
}

extern "C" int sj_rmsnorm_bwd_p(void* stream, const uint16_t* x, const uint16_t* w, const float* dy,
                                const float* dx_acc, float* dx, float* dw, uint16_t* dx_hi, uint16_t* dx_lo,
                                uint16_t* dx_t_hi, uint16_t* dx_t_lo, long ldt, long rows, long d, float eps,
                                void* workspace, size_t workspace_bytes) {
  SJ_REQUIRE(rows > 0 && d > 0 && d % 8 == 0 && d <= 1024 && !dx_t_hi == !dx_t_lo && !dx_hi == !dx_lo &&
                 (!dx_t_hi || (ldt >= rows && ldt % 8 == 0)) && ((uintptr_t)dx_t_hi & 15) == 0 &&
                 ((uintptr_t)dx_t_lo & 15) == 0,
             "RMSNorm backward (planes): rows %ld d %ld ldt %ld (d <= 1024; planes both or neither)", rows, d, ldt);
  if (int st0 = sjh::norm_prepare()) return st0;
  size_t need = sj_rmsnorm_bwd_p_workspace_bytes(rows, d);
  if (!workspace || workspace_bytes < need)
    return sjh::fail(SJ_ERR_CAPACITY, "rmsnorm_backward: required %zu bytes, available %zu bytes", need,
                     workspace_bytes);
  hipStream_t s = (hipStream_t)stream;
  const long groups = (rows + TR - 1) / TR;
  const size_t lds = 2 * sizeof(bf16_t) * TR * (size_t)d + sizeof(float) * TR * (size_t)d;
  float* partial = (float*)workspace;
  const unsigned blocks = (unsigned)groups;
  switch ((d / 2 + 63) / 64) {
    case 1: launch_bwd_p<1>(s, blocks, lds, x, w, dy, dx_acc, dx, dx_hi, dx_lo, dx_t_hi, dx_t_lo, partial, rows, d, ldt, eps); break;
    case 2: launch_bwd_p<2>(s, blocks, lds, x, w, dy, dx_acc, dx, dx_hi, dx_lo, dx_t_hi, dx_t_lo, partial, rows, d, ldt, eps); break;
    case 3: launch_bwd_p<3>(s, blocks, lds, x, w, dy, dx_acc, dx, dx_hi, dx_lo, dx_t_hi, dx_t_lo, partial, rows, d, ldt, eps); break;
    case 4: launch_bwd_p<4>(s, blocks, lds, x, w, dy, dx_acc, dx, dx_hi, dx_lo, dx_t_hi, dx_t_lo, partial, rows, d, ldt, eps); break;
    case 5: launch_bwd_p<5>(s, blocks, lds, x, w, dy, dx_acc, dx, dx_hi, dx_lo, dx_t_hi, dx_t_lo, partial, rows, d, ldt, eps); break;
    case 6: launch_bwd_p<6>(s, blocks, lds, x, w, dy, dx_acc, dx, dx_hi, dx_lo, dx_t_hi, dx_t_lo, partial, rows, d, ldt, eps); break;
    case 7: launch_bwd_p<7>(s, blocks, lds, x, w, dy, dx_acc, dx, dx_hi, dx_lo, dx_t_hi, dx_t_lo, partial, rows, d, ldt, eps); break;
    default: launch_bwd_p<8>(s, blocks, lds, x, w, dy, dx_acc, dx, dx_hi, dx_lo, dx_t_hi, dx_t_lo, partial, rows, d, ldt, eps); break;
  }
  hipLaunchKernelGGL(k_rms_reduce, dim3((unsigned)((d + 31) / 32)), dim3(NT), 0, s, (const float*)workspace, dw,
                     groups, d);
  SJ_LAUNCH_CHECK("rmsnorm_backward_p");
  return SJ_OK;
}

// ------------------------------------------------ allocation-free backward
// sj_rmsnorm_bwd_p_noalloc keeps the dw partials in this file-scope array
// instead of a caller workspace.  Host code never passes `scratch` itself to
// a kernel (in host code the name is a stand-in, not a device address): the
// first call on each device resolves the device's own copy with
// hipGetSymbolAddress, and every launch takes that pointer.
namespace {
constexpr size_t NOALLOC_FLOATS = SJ_RMSNORM_BWD_NOALLOC_MAX_BYTES / sizeof(float);
constexpr int NOALLOC_DEVICES = 64;
std::mutex g_noalloc_mu;
float* g_noalloc_ptr[NOALLOC_DEVICES] = {};
}  // namespace
static __device__ __align__(256) float scratch[NOALLOC_FLOATS];

extern "C" int sj_rmsnorm_bwd_p_noalloc(void* stream, const uint16_t* x, const uint16_t* w, const float* dy,
                                        const float* dx_acc, float* dx, float* dw, uint16_t* dx_hi, uint16_t* dx_lo,
                                        uint16_t* dx_t_hi, uint16_t* dx_t_lo, long ldt, long rows, long d,
                                        float eps) {
  SJ_REQUIRE(rows > 0 && d > 0, "RMSNorm backward (no allocation): rows %ld d %ld", rows, d);
  const size_t need = sj_rmsnorm_bwd_p_workspace_bytes(rows, d);
  if (need > SJ_RMSNORM_BWD_NOALLOC_MAX_BYTES)
    return sjh::fail(SJ_ERR_CAPACITY,
                     "rmsnorm_backward (no allocation): required %zu bytes of scratch, available %zu bytes "
                     "(ceil(rows / 16) * d * 4 must not exceed SJ_RMSNORM_BWD_NOALLOC_MAX_BYTES)",
                     need, (size_t)SJ_RMSNORM_BWD_NOALLOC_MAX_BYTES);
  int dev = 0;
  SJ_HIP(hipGetDevice(&dev));
  SJ_REQUIRE(dev >= 0 && dev < NOALLOC_DEVICES, "RMSNorm backward (no allocation): device %d", dev);
  float* part = nullptr;
  {
    std::lock_guard<std::mutex> lock(g_noalloc_mu);
    if (!g_noalloc_ptr[dev]) {
      void* p = nullptr;
      hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (e != hipSuccess) return sjh::hip_check(e, "rmsnorm_backward (no allocation): hipGetSymbolAddress");
      g_noalloc_ptr[dev] = (float*)p;
    }
    part = g_noalloc_ptr[dev];
  }
  // every partial entry [ceil(rows / 16)][d] is written by the row kernel
  // before the reduce reads it, so nothing needs clearing between calls
  return sj_rmsnorm_bwd_p(stream, x, w, dy, dx_acc, dx, dw, dx_hi, dx_lo, dx_t_hi, dx_t_lo, ldt, rows, d, eps, part,
                          need);
}
