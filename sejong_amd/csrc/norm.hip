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
constexpr int BWD_ROWS = 8;     // rows per workgroup in the backward

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

// rmsnorm_backward_reduce (kernels.py:79-87): dw[c] = sum_g partial[g][c]
__global__ __launch_bounds__(NT) void k_rms_reduce(const float* __restrict__ partial, float* __restrict__ dw,
                                                   long groups, long d) {
  // 4 row-slices x 64 columns per workgroup, combined in fixed order
  __shared__ float red[4][64];
  const int lane = threadIdx.x & 63, sl = threadIdx.x >> 6;
  const long c = blockIdx.x * 64L + lane;
  float s = 0.f;
  if (c < d)
    for (long g = sl; g < groups; g += 4) s += partial[g * d + c];
  red[sl][lane] = s;
  __syncthreads();
  if (sl == 0 && c < d) dw[c] = ((red[0][lane] + red[1][lane]) + red[2][lane]) + red[3][lane];
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
  hipLaunchKernelGGL(k_rms_reduce, dim3((unsigned)((d + 63) / 64)), dim3(NT), 0, s, partial, dw, groups, d);
  SJ_LAUNCH_CHECK("rmsnorm_backward");
  return SJ_OK;
}
