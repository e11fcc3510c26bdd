// RMSNorm forward and backward (kernels.py:54-87, norm_ops.rs:14-71).
// One wavefront per row; each lane owns column pairs lane + 64*j, so loads
// are 4-byte (bf16x2) or 8-byte (f32x2) coalesced.  The backward writes dx
// per row and a per-workgroup dw partial, reduced in a second fixed-order
// pass (deterministic, no atomics -- the reference's partial/reduce split).
#include <math.h>

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


// ----------------------------------------------------- MFMA-layout variants
// Row blocks of TR = 32 rows: each wave normalises 8 rows, the block stages
// its bf16 outputs in LDS and also writes them transposed ([d][rows], 64 B
// per column segment), the layout the dW GEMMs stream.
constexpr int TR = 32;

// y = rmsnorm(x) (bf16 x, w) -> y [rows][d] and y_t [d][ldt]
__global__ __launch_bounds__(NT) void k_rms_fwd_t(const bf16_t* __restrict__ x, const bf16_t* __restrict__ w,
                                                  bf16_t* __restrict__ y, bf16_t* __restrict__ yt, long rows,
                                                  long d, long ldt, float eps) {
  extern __shared__ __attribute__((aligned(16))) bf16_t stage[];  // [TR][d]
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const long r0 = blockIdx.x * (long)TR;
  const long pairs = d >> 1;
  for (int rr = wv; rr < TR; rr += 4) {
    const long r = r0 + rr;
    float2 xv[MAXP];
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < MAXP; j++) {
      long p = lane + 64L * j;
      if (p < pairs && r < rows) {
        xv[j] = ld2<SJ_BF16>(x, r * d + 2 * p);
        s += xv[j].x * xv[j].x + xv[j].y * xv[j].y;
      }
    }
    s = wave_sum(s);
    const float inv = 1.f / sqrtf(s / (float)d + eps);
#pragma unroll
    for (int j = 0; j < MAXP; j++) {
      long p = lane + 64L * j;
      if (p < pairs) {
        float2 wv2 = ld2<SJ_BF16>(w, 2 * p);
        uint32_t pk = r < rows ? pack2(f2bf(xv[j].x * inv * wv2.x), f2bf(xv[j].y * inv * wv2.y)) : 0u;
        if (r < rows) *(uint32_t*)(y + r * d + 2 * p) = pk;
        *(uint32_t*)(stage + rr * d + 2 * p) = pk;
      }
    }
  }
  __syncthreads();
  // transposed: column c, rows r0..r0+31 -> 4 chunks of 8 bf16
  for (long q = threadIdx.x; q < d * (TR / 8); q += NT) {
    const long c = q / (TR / 8);
    const int ch = (int)(q % (TR / 8));
    bf16_t v[8];
#pragma unroll
    for (int i = 0; i < 8; i++) v[i] = stage[(ch * 8 + i) * d + c];
    const long rbase = r0 + ch * 8;
    bf16_t* dst = yt + c * ldt + rbase;
    if (rbase + 8 <= rows) {
      *(u32x4*)dst = u32x4{pack2(v[0], v[1]), pack2(v[2], v[3]), pack2(v[4], v[5]), pack2(v[6], v[7])};
    } else {
      for (int i = 0; i < 8; i++)
        if (rbase + i < rows) dst[i] = v[i];
    }
  }
}

// backward with hi/lo plane outputs of dx (normal and transposed) next to the
// fp32 dx; dw partial per 32-row block.
__global__ __launch_bounds__(NT) void k_rms_bwd_p(const bf16_t* __restrict__ x, const bf16_t* __restrict__ w,
                                                  const float* __restrict__ dy, const float* __restrict__ dx_acc,
                                                  float* __restrict__ dx, bf16_t* __restrict__ hi,
                                                  bf16_t* __restrict__ lo, bf16_t* __restrict__ hit,
                                                  bf16_t* __restrict__ lot, float* __restrict__ partial, long rows,
                                                  long d, long ldt, float eps) {
  extern __shared__ __attribute__((aligned(16))) bf16_t stage[];  // hi [TR][d], lo [TR][d], red [4][d] f32
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const long pairs = d >> 1;
  bf16_t* shi = stage;
  bf16_t* slo = stage + TR * d;
  float* red = (float*)(stage + 2 * TR * d);
  float2 dwp[MAXP], wreg[MAXP];
#pragma unroll
  for (int j = 0; j < MAXP; j++) {
    dwp[j] = make_float2(0.f, 0.f);
    long p = lane + 64L * j;
    if (p < pairs) wreg[j] = ld2<SJ_BF16>(w, 2 * p);
  }
  const long r0 = blockIdx.x * (long)TR;
  for (int rr = wv; rr < TR; rr += 4) {
    const long r = r0 + rr;
    const bool ok = r < rows;
    float2 xv[MAXP], gv[MAXP];
    float s = 0.f, sdx = 0.f;
#pragma unroll
    for (int j = 0; j < MAXP; j++) {
      long p = lane + 64L * j;
      if (p < pairs && ok) {
        xv[j] = ld2<SJ_BF16>(x, r * d + 2 * p);
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
        uint32_t ph = 0u, pl = 0u;
        if (ok) {
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
          bf16_t ha, la, hb, lb;
          split_bf(a, ha, la);
          split_bf(b, hb, lb);
          ph = pack2(ha, hb);
          pl = pack2(la, lb);
          *(uint32_t*)(hi + r * d + 2 * p) = ph;
          *(uint32_t*)(lo + r * d + 2 * p) = pl;
        }
        *(uint32_t*)(shi + rr * d + 2 * p) = ph;
        *(uint32_t*)(slo + rr * d + 2 * p) = pl;
      }
    }
  }
#pragma unroll
  for (int j = 0; j < MAXP; j++) {
    long p = lane + 64L * j;
    if (p < pairs) {
      red[wv * d + 2 * p] = dwp[j].x;
      red[wv * d + 2 * p + 1] = dwp[j].y;
    }
  }
  __syncthreads();
  for (long c = threadIdx.x; c < d; c += NT)
    partial[blockIdx.x * d + c] = ((red[c] + red[d + c]) + red[2 * d + c]) + red[3 * d + c];
  for (long q = threadIdx.x; q < 2 * d * (TR / 8); q += NT) {
    const int pl = q >= d * (TR / 8);
    const long qq = pl ? q - d * (TR / 8) : q;
    const long c = qq / (TR / 8);
    const int ch = (int)(qq % (TR / 8));
    const bf16_t* src = pl ? slo : shi;
    bf16_t v[8];
#pragma unroll
    for (int i = 0; i < 8; i++) v[i] = src[(ch * 8 + i) * d + c];
    const long rbase = r0 + ch * 8;
    bf16_t* dst = (pl ? lot : hit) + c * ldt + rbase;
    if (rbase + 8 <= rows) {
      *(u32x4*)dst = u32x4{pack2(v[0], v[1]), pack2(v[2], v[3]), pack2(v[4], v[5]), pack2(v[6], v[7])};
    } else {
      for (int i = 0; i < 8; i++)
        if (rbase + i < rows) dst[i] = v[i];
    }
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
namespace sjh {
int norm_prepare() {
  static int done = 0, status = SJ_OK;
  if (done) return status;
  done = 1;
  hipError_t e = hipFuncSetAttribute((const void*)k_rms_bwd_p, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
  if (e == hipSuccess)
    e = hipFuncSetAttribute((const void*)k_rms_fwd_t, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
  status = e == hipSuccess ? SJ_OK : sjh::hip_check(e, "rmsnorm: LDS attribute");
  return status;
}
}  // namespace sjh

extern "C" int sj_rmsnorm_fwd_t(void* stream, const uint16_t* x, const uint16_t* w, uint16_t* y, uint16_t* y_t,
                                long ldt, long rows, long d, float eps) {
  SJ_REQUIRE(rows >= 0 && d > 0 && d % 8 == 0 && d <= 2 * 64 * MAXP && ldt >= rows && ldt % 8 == 0 &&
                 ((uintptr_t)y_t & 15) == 0,
             "RMSNorm (transposed output): rows %ld d %ld ldt %ld", rows, d, ldt);
  if (rows == 0) return SJ_OK;
  if (int st0 = sjh::norm_prepare()) return st0;
  const size_t lds = sizeof(bf16_t) * TR * (size_t)d;
  hipLaunchKernelGGL(k_rms_fwd_t, dim3((unsigned)((rows + TR - 1) / TR)), dim3(NT), lds, (hipStream_t)stream,
                     (const bf16_t*)x, (const bf16_t*)w, (bf16_t*)y, (bf16_t*)y_t, rows, d, ldt, eps);
  SJ_LAUNCH_CHECK("rmsnorm_t");
  return SJ_OK;
}

extern "C" size_t sj_rmsnorm_bwd_p_workspace_bytes(long rows, long d) {
  return sizeof(float) * (size_t)((rows + TR - 1) / TR) * (size_t)d;
}

extern "C" int sj_rmsnorm_bwd_p(void* stream, const uint16_t* x, const uint16_t* w, const float* dy,
                                const float* dx_acc, float* dx, float* dw, uint16_t* dx_hi, uint16_t* dx_lo,
                                uint16_t* dx_t_hi, uint16_t* dx_t_lo, long ldt, long rows, long d, float eps,
                                void* workspace, size_t workspace_bytes) {
  SJ_REQUIRE(rows > 0 && d > 0 && d % 8 == 0 && d <= 1024 && ldt >= rows && ldt % 8 == 0 &&
                 ((uintptr_t)dx_t_hi & 15) == 0 && ((uintptr_t)dx_t_lo & 15) == 0,
             "RMSNorm backward (planes): rows %ld d %ld ldt %ld (d <= 1024)", rows, d, ldt);
  if (int st0 = sjh::norm_prepare()) return st0;
  size_t need = sj_rmsnorm_bwd_p_workspace_bytes(rows, d);
  if (!workspace || workspace_bytes < need)
    return sjh::fail(SJ_ERR_CAPACITY, "rmsnorm_backward: required %zu bytes, available %zu bytes", need,
                     workspace_bytes);
  hipStream_t s = (hipStream_t)stream;
  const long groups = (rows + TR - 1) / TR;
  const size_t lds = 2 * sizeof(bf16_t) * TR * (size_t)d + 4 * sizeof(float) * (size_t)d;
  hipLaunchKernelGGL(k_rms_bwd_p, dim3((unsigned)groups), dim3(NT), lds, s, (const bf16_t*)x, (const bf16_t*)w, dy,
                     dx_acc, dx, (bf16_t*)dx_hi, (bf16_t*)dx_lo, (bf16_t*)dx_t_hi, (bf16_t*)dx_t_lo,
                     (float*)workspace, rows, d, ldt, eps);
  hipLaunchKernelGGL(k_rms_reduce, dim3((unsigned)((d + 31) / 32)), dim3(NT), 0, s, (const float*)workspace, dw,
                     groups, d);
  SJ_LAUNCH_CHECK("rmsnorm_backward_p");
  return SJ_OK;
}
