// Patch pooling and patch broadcast of the hierarchical (cfg3) byte model
// (Engine::patch_pool / patch_broadcast and their backwards,
// crates/sejong-gpu/src/hierarchy_ops.rs:149-278; kernels
// python/sejong_kernels/ops/hierarchy.py:107-172): the byte stream
// [batch*t][d] is pooled into ceil(t/patch) patch rows per sequence, and the
// global model's patch rows are broadcast back to the bytes shifted by one
// patch (the first patch of each sequence sees the learned BOS row).
//
// HBM-bound row streaming: one thread owns VEC consecutive columns of one
// output row (16-byte accesses when d and the pointers allow) and walks the
// positions it sums in the reference's order, so every fp32 sum is formed
// in the same sequence of roundings as the reference kernels.
#include <initializer_list>

#include "common.h"

using namespace sj;

namespace {

constexpr int PT = 256;

template <int VEC>
__device__ __forceinline__ void load_vec(const void* p, int dt, long i, float* v) {
  if constexpr (VEC == 8) {
    // bf16: one 16-byte load
    const u32x4 w = *(const u32x4*)((const bf16_t*)p + i);
#pragma unroll
    for (int j = 0; j < 4; j++) {
      v[2 * j] = bf2f((bf16_t)(w[j] & 0xffffu));
      v[2 * j + 1] = bf2f((bf16_t)(w[j] >> 16));
    }
  } else if constexpr (VEC == 4) {
    const float4 w = *(const float4*)((const float*)p + i);
    v[0] = w.x; v[1] = w.y; v[2] = w.z; v[3] = w.w;
  } else {
    v[0] = load_as_f32(p, dt, i);
  }
}

template <int VEC>
__device__ __forceinline__ void store_vec(void* p, int dt, long i, const float* v) {
  if constexpr (VEC == 8) {
    *(u32x4*)((bf16_t*)p + i) = u32x4{pack2(f2bf(v[0]), f2bf(v[1])), pack2(f2bf(v[2]), f2bf(v[3])),
                                      pack2(f2bf(v[4]), f2bf(v[5])), pack2(f2bf(v[6]), f2bf(v[7]))};
  } else if constexpr (VEC == 4) {
    *(float4*)((float*)p + i) = make_float4(v[0], v[1], v[2], v[3]);
  } else {
    store_from_f32(p, dt, i, v[0]);
  }
}

// hierarchy_patch_pool: y[row] = (sum over the patch's positions, in order) / count
template <int VEC>
__global__ __launch_bounds__(PT) void k_patch_pool(const void* __restrict__ x, int dt, void* __restrict__ y, long t,
                                                   long d, long patch, long rows) {
  const long chunks = d / VEC;
  const long i = blockIdx.x * (long)PT + threadIdx.x;
  if (i >= rows * chunks) return;
  const long row = i / chunks, c0 = (i - row * chunks) * VEC;
  const long patches = (t + patch - 1) / patch;
  const long batch = row / patches, start = (row % patches) * patch;
  const long count = patch < t - start ? patch : t - start;
  float total[VEC];
#pragma unroll
  for (int j = 0; j < VEC; j++) total[j] = 0.f;
  for (long p = 0; p < count; p++) {
    float v[VEC];
    load_vec<VEC>(x, dt, (batch * t + start + p) * d + c0, v);
#pragma unroll
    for (int j = 0; j < VEC; j++) total[j] += v[j];
  }
  const float cf = (float)count;
#pragma unroll
  for (int j = 0; j < VEC; j++) total[j] = total[j] / cf;
  store_vec<VEC>(y, dt, row * d + c0, total);
}

// hierarchy_patch_pool_backward: dx[b, pos] = dy[b, pos / patch] / count (fp32)
template <int VEC>
__global__ __launch_bounds__(PT) void k_patch_pool_bwd(const float* __restrict__ dy, float* __restrict__ dx, long t,
                                                       long d, long patch, long rows) {
  const long chunks = d / VEC;
  const long i = blockIdx.x * (long)PT + threadIdx.x;
  if (i >= rows * chunks) return;
  const long row = i / chunks, c0 = (i - row * chunks) * VEC;
  const long pos = row % t, batch = row / t, p = pos / patch;
  const long count = patch < t - p * patch ? patch : t - p * patch;
  const long patches = (t + patch - 1) / patch;
  float v[VEC];
  load_vec<VEC>(dy, SJ_F32, (batch * patches + p) * d + c0, v);
  const float cf = (float)count;
#pragma unroll
  for (int j = 0; j < VEC; j++) v[j] = v[j] / cf;
  store_vec<VEC>(dx, SJ_F32, row * d + c0, v);
}

// hierarchy_patch_broadcast: y[b, pos] = x[b, pos / patch - 1], or bos for
// the first patch
template <int VEC>
__global__ __launch_bounds__(PT) void k_patch_broadcast(const void* __restrict__ x, const void* __restrict__ bos,
                                                        int dt, void* __restrict__ y, long t, long d, long patch,
                                                        long rows) {
  const long chunks = d / VEC;
  const long i = blockIdx.x * (long)PT + threadIdx.x;
  if (i >= rows * chunks) return;
  const long row = i / chunks, c0 = (i - row * chunks) * VEC;
  const long pos = row % t, batch = row / t, p = pos / patch - 1;
  const long patches = (t + patch - 1) / patch;
  float v[VEC];
  if (p >= 0)
    load_vec<VEC>(x, dt, (batch * patches + p) * d + c0, v);
  else
    load_vec<VEC>(bos, dt, c0, v);
  store_vec<VEC>(y, dt, row * d + c0, v);
}

// hierarchy_patch_broadcast_backward: dx[b, p] = sum over the next patch's
// positions of dy (in position order); dbos = sum over batches, then over
// the first patch's positions.  Threads past the body rows form dbos.
template <int VEC>
__global__ __launch_bounds__(PT) void k_patch_broadcast_bwd(const float* __restrict__ dy, float* __restrict__ dx,
                                                            float* __restrict__ dbos, long batches, long t, long d,
                                                            long patch) {
  const long chunks = d / VEC;
  const long patches = (t + patch - 1) / patch;
  const long body = batches * patches * chunks;
  const long body_blocks = (body + PT - 1) / PT;
  float total[VEC];
#pragma unroll
  for (int j = 0; j < VEC; j++) total[j] = 0.f;
  if ((long)blockIdx.x < body_blocks) {
    const long i = blockIdx.x * (long)PT + threadIdx.x;
    if (i >= body) return;
    const long row = i / chunks, c0 = (i - row * chunks) * VEC;
    const long batch = row / patches, start = (row % patches + 1) * patch;
    for (long off = 0; off < patch; off++) {
      const long pos = start + off;
      float v[VEC];
      if (pos < t) {
        load_vec<VEC>(dy, SJ_F32, (batch * t + pos) * d + c0, v);
      } else {  // the reference adds the masked load's 0 (keeps the sign of a -0 sum identical)
#pragma unroll
        for (int j = 0; j < VEC; j++) v[j] = 0.f;
      }
#pragma unroll
      for (int j = 0; j < VEC; j++) total[j] += v[j];
    }
    store_vec<VEC>(dx, SJ_F32, row * d + c0, total);
    return;
  }
  const long c = ((long)blockIdx.x - body_blocks) * PT + threadIdx.x;
  if (c >= chunks) return;
  const long c0 = c * VEC, first = patch < t ? patch : t;
  for (long b = 0; b < batches; b++)
    for (long pos = 0; pos < first; pos++) {
      float v[VEC];
      load_vec<VEC>(dy, SJ_F32, (b * t + pos) * d + c0, v);
#pragma unroll
      for (int j = 0; j < VEC; j++) total[j] += v[j];
    }
  store_vec<VEC>(dbos, SJ_F32, c0, total);
}

bool al16(const void* p) { return ((uintptr_t)p & 15) == 0; }

// 16-byte vectors when the row width and every pointer allow it
int vec_for(int dt, long d, std::initializer_list<const void*> ptrs) {
  const int v = dt == SJ_BF16 ? 8 : 4;
  if (d % v) return 1;
  for (const void* p : ptrs)
    if (p && !al16(p)) return 1;
  return v;
}

unsigned blocks_for(long work) { return (unsigned)((work + PT - 1) / PT); }

}  // namespace

extern "C" int sj_patch_pool(void* stream, const void* x, int dtype, long batch, long t, long d, long patch,
                             void* y) {
  SJ_REQUIRE(x && y && batch > 0 && t > 0 && d > 0 && patch > 0 && patch <= 0x7fffffffL &&
                 (dtype == SJ_F32 || dtype == SJ_BF16),
             "patch pool sequence dimensions");
  hipStream_t s = (hipStream_t)stream;
  const long rows = batch * ((t + patch - 1) / patch);
  const int v = vec_for(dtype, d, {x, y});
  if (v == 8)
    hipLaunchKernelGGL(k_patch_pool<8>, dim3(blocks_for(rows * d / 8)), dim3(PT), 0, s, x, dtype, y, t, d, patch, rows);
  else if (v == 4)
    hipLaunchKernelGGL(k_patch_pool<4>, dim3(blocks_for(rows * d / 4)), dim3(PT), 0, s, x, dtype, y, t, d, patch, rows);
  else
    hipLaunchKernelGGL(k_patch_pool<1>, dim3(blocks_for(rows * d)), dim3(PT), 0, s, x, dtype, y, t, d, patch, rows);
  SJ_LAUNCH_CHECK("hierarchy_patch_pool");
  return SJ_OK;
}

extern "C" int sj_patch_pool_bwd(void* stream, const float* dy, long batch, long t, long d, long patch, float* dx) {
  SJ_REQUIRE(dy && dx && batch > 0 && t > 0 && d > 0 && patch > 0 && patch <= 0x7fffffffL,
             "patch pool backward sequence dimensions");
  hipStream_t s = (hipStream_t)stream;
  const long rows = batch * t;
  if (vec_for(SJ_F32, d, {dy, dx}) == 4)
    hipLaunchKernelGGL(k_patch_pool_bwd<4>, dim3(blocks_for(rows * d / 4)), dim3(PT), 0, s, dy, dx, t, d, patch, rows);
  else
    hipLaunchKernelGGL(k_patch_pool_bwd<1>, dim3(blocks_for(rows * d)), dim3(PT), 0, s, dy, dx, t, d, patch, rows);
  SJ_LAUNCH_CHECK("hierarchy_patch_pool_backward");
  return SJ_OK;
}

extern "C" int sj_patch_broadcast(void* stream, const void* x, const void* bos, int dtype, long batch, long t, long d,
                                  long patch, void* y) {
  SJ_REQUIRE(x && bos && y && batch > 0 && t > 0 && d > 0 && patch > 0 && patch <= 0x7fffffffL &&
                 (dtype == SJ_F32 || dtype == SJ_BF16),
             "patch broadcast sequence/BOS dimensions");
  hipStream_t s = (hipStream_t)stream;
  const long rows = batch * t;
  const int v = vec_for(dtype, d, {x, bos, y});
  if (v == 8)
    hipLaunchKernelGGL(k_patch_broadcast<8>, dim3(blocks_for(rows * d / 8)), dim3(PT), 0, s, x, bos, dtype, y, t, d,
                       patch, rows);
  else if (v == 4)
    hipLaunchKernelGGL(k_patch_broadcast<4>, dim3(blocks_for(rows * d / 4)), dim3(PT), 0, s, x, bos, dtype, y, t, d,
                       patch, rows);
  else
    hipLaunchKernelGGL(k_patch_broadcast<1>, dim3(blocks_for(rows * d)), dim3(PT), 0, s, x, bos, dtype, y, t, d,
                       patch, rows);
  SJ_LAUNCH_CHECK("hierarchy_patch_broadcast");
  return SJ_OK;
}

extern "C" int sj_patch_broadcast_bwd(void* stream, const float* dy, long batch, long t, long d, long patch,
                                      float* dx, float* dbos) {
  SJ_REQUIRE(dy && dx && dbos && batch > 0 && t > 0 && d > 0 && patch > 0 && patch <= 0x7fffffffL,
             "patch broadcast backward sequence dimensions");
  hipStream_t s = (hipStream_t)stream;
  const long patches = (t + patch - 1) / patch;
  const int v = vec_for(SJ_F32, d, {dy, dx, dbos});
  const long chunks = d / v;
  const unsigned grid = blocks_for(batch * patches * chunks) + blocks_for(chunks);
  if (v == 4)
    hipLaunchKernelGGL(k_patch_broadcast_bwd<4>, dim3(grid), dim3(PT), 0, s, dy, dx, dbos, batch, t, d, patch);
  else
    hipLaunchKernelGGL(k_patch_broadcast_bwd<1>, dim3(grid), dim3(PT), 0, s, dy, dx, dbos, batch, t, d, patch);
  SJ_LAUNCH_CHECK("hierarchy_patch_broadcast_backward");
  return SJ_OK;
}
