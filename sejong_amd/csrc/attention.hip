// GQA causal attention, forward and backward, for gfx950.
//
// Forward  (hierarchy.py:7-39):  one workgroup per (64-query block, query
//   head, batch); 4 waves x 16 queries.  S^T = K Q^T on MFMA so that each
//   lane holds 16 scores of ONE query -- the softmax statistics need only
//   xor-16/32 shuffles and the P fragment for O += P V is already in the
//   lane's registers (the key order inside the MFMA k-slots is permuted,
//   and V^T is read from LDS in the same permuted order).
// Backward (hierarchy.py:42-104), deterministic and atomic-free like the
//   reference: k_attn_dq (per query block; writes Delta = sum dO*O) then
//   k_attn_dkv (per key block of one KV head, looping the HQ/HK query heads
//   of its group).  Optional inverse RoPE on dQ/dK in the epilogue.
// P, dS and dO are fp32 values multiplied on bf16 MFMA as hi+lo pairs
// (error ~2^-16 relative); a single bf16 rounding of them costs ~1.6e-3
// normwise, more than the 1e-3 gradient tolerance.
//
// The MFMA kernels handle bf16 storage, head_dim 64 and full causal masks;
// fp32 storage, other head widths and sliding windows use the wavefront-
// per-row kernels at the end of this file (same formulas, fp32 FMA).
#include <math.h>

#include "common.h"

using namespace sj;

namespace {

constexpr int DH = 64;
constexpr int QB = 64;   // queries / keys per block
constexpr int LS = DH + 8;  // LDS row stride (bf16)
constexpr float LOG2E = 1.4426950408889634f;
constexpr float LN2 = 0.6931471805599453f;

__device__ __forceinline__ bf16x8 as_bf8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }
__device__ __forceinline__ f32x4 mfma(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// 8 bf16 from two 4-element LDS runs (permuted key order of the k-slots)
__device__ __forceinline__ bf16x8 ld_perm(const bf16_t* row, int a, int b) {
  u32x2 x = *(const u32x2*)(row + a);
  u32x2 y = *(const u32x2*)(row + b);
  return as_bf8(u32x4{x.x, x.y, y.x, y.y});
}

__device__ __forceinline__ bf16x8 pack8(const float* v) {
  return as_bf8(u32x4{pack2(f2bf(v[0]), f2bf(v[1])), pack2(f2bf(v[2]), f2bf(v[3])), pack2(f2bf(v[4]), f2bf(v[5])),
                      pack2(f2bf(v[6]), f2bf(v[7]))});
}
// hi/lo split of 8 floats
__device__ __forceinline__ void split8(const float* v, bf16x8& hi, bf16x8& lo) {
  bf16_t h[8], l[8];
#pragma unroll
  for (int i = 0; i < 8; i++) split_bf(v[i], h[i], l[i]);
  hi = as_bf8(u32x4{pack2(h[0], h[1]), pack2(h[2], h[3]), pack2(h[4], h[5]), pack2(h[6], h[7])});
  lo = as_bf8(u32x4{pack2(l[0], l[1]), pack2(l[2], l[3]), pack2(l[4], l[5]), pack2(l[6], l[7])});
}

// Stage rows [row0, row0+64) x cols [col0, col0+64) of a bf16 matrix.
// normal: dst[r][c]; transposed: dst[c][r].  Rows >= nrows read as zero.
__device__ __forceinline__ void stage_bf16(bf16_t* dst, const bf16_t* src, long ld, long row0, long nrows, long col0) {
  const int t = threadIdx.x;
#pragma unroll
  for (int p = 0; p < 2; p++) {
    int ch = t + p * 256;
    int r = ch >> 3, cc = ch & 7;
    long row = row0 + r;
    u32x4 v = u32x4{0, 0, 0, 0};
    if (row < nrows) v = *(const u32x4*)(src + row * ld + col0 + cc * 8);
    *(u32x4*)(dst + r * LS + cc * 8) = v;
  }
}
__device__ __forceinline__ void stage_bf16_t(bf16_t* dst, const bf16_t* src, long ld, long row0, long nrows,
                                             long col0) {
  const int t = threadIdx.x;
  const int rg = t >> 5, cp = t & 31;  // 8 row groups x 32 column pairs
  uint32_t w[8];
#pragma unroll
  for (int i = 0; i < 8; i++) {
    long row = row0 + rg * 8 + i;
    w[i] = row < nrows ? *(const uint32_t*)(src + row * ld + col0 + 2 * cp) : 0u;
  }
  bf16_t* d0 = dst + (2 * cp) * LS + rg * 8;
  *(u32x4*)d0 = u32x4{(w[0] & 0xffffu) | (w[1] << 16), (w[2] & 0xffffu) | (w[3] << 16),
                      (w[4] & 0xffffu) | (w[5] << 16), (w[6] & 0xffffu) | (w[7] << 16)};
  *(u32x4*)(d0 + LS) = u32x4{(w[0] >> 16) | (w[1] & 0xffff0000u), (w[2] >> 16) | (w[3] & 0xffff0000u),
                             (w[4] >> 16) | (w[5] & 0xffff0000u), (w[6] >> 16) | (w[7] & 0xffff0000u)};
}
// fp32 source -> hi/lo planes, normal and transposed
__device__ __forceinline__ void stage_f32_split(bf16_t* hi, bf16_t* lo, bf16_t* hit, bf16_t* lot, const float* src,
                                                long ld, long row0, long nrows, long col0) {
  const int t = threadIdx.x;
#pragma unroll
  for (int p = 0; p < 2; p++) {
    int ch = t + p * 256;
    int r = ch >> 3, cc = ch & 7;
    long row = row0 + r;
    float v[8];
    if (row < nrows) {
      float4 a = *(const float4*)(src + row * ld + col0 + cc * 8);
      float4 b = *(const float4*)(src + row * ld + col0 + cc * 8 + 4);
      v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else {
#pragma unroll
      for (int i = 0; i < 8; i++) v[i] = 0.f;
    }
    bf16x8 h, l;
    split8(v, h, l);
    *(bf16x8*)(hi + r * LS + cc * 8) = h;
    *(bf16x8*)(lo + r * LS + cc * 8) = l;
  }
  const int rg = t >> 5, cp = t & 31;
  bf16_t h0[8], l0[8], h1[8], l1[8];
#pragma unroll
  for (int i = 0; i < 8; i++) {
    long row = row0 + rg * 8 + i;
    float2 v = row < nrows ? *(const float2*)(src + row * ld + col0 + 2 * cp) : make_float2(0.f, 0.f);
    split_bf(v.x, h0[i], l0[i]);
    split_bf(v.y, h1[i], l1[i]);
  }
  bf16_t* d = hit + (2 * cp) * LS + rg * 8;
  *(u32x4*)d = u32x4{pack2(h0[0], h0[1]), pack2(h0[2], h0[3]), pack2(h0[4], h0[5]), pack2(h0[6], h0[7])};
  *(u32x4*)(d + LS) = u32x4{pack2(h1[0], h1[1]), pack2(h1[2], h1[3]), pack2(h1[4], h1[5]), pack2(h1[6], h1[7])};
  d = lot + (2 * cp) * LS + rg * 8;
  *(u32x4*)d = u32x4{pack2(l0[0], l0[1]), pack2(l0[2], l0[3]), pack2(l0[4], l0[5]), pack2(l0[6], l0[7])};
  *(u32x4*)(d + LS) = u32x4{pack2(l1[0], l1[1]), pack2(l1[2], l1[3]), pack2(l1[4], l1[5]), pack2(l1[6], l1[7])};
}

struct AttnArgs {
  const bf16_t *q, *k, *v, *o;
  long ldq, ldk, ldv, ldo;
  bf16_t* out;
  float* lse;
  const float* dout;
  long lddo;
  float *dq, *dk, *dv, *delta;
  long lddq, lddk, lddv;
  long T, HQ, HK;
  const float* rope;  // inverse-rope table (cos, sin) [T][DH/2] or null
  // MFMA-layout outputs (null: not written)
  bf16_t* ot;  // O^T [HQ*DH][ldot] (forward)
  long ldot;
  // backward as hi/lo planes instead of fp32: normal [rows][ldp] at the
  // q / k / v column offsets, transposed [cols][ldtp] at the row offsets
  bf16_t *pq[2], *pk[2], *pv[2], *tq[2], *tk[2], *tv[2];
  long ldp, ldtp;
};

// store one lane's 4 consecutive rows of column `col` of a gradient as
// hi/lo planes: normal rows (row0+r)*ldp + col, transposed col*ldtp + row0..+3
__device__ __forceinline__ void store_planes(bf16_t* const* pn, bf16_t* const* pt, long ldp, long ldtp, long row0,
                                             long col, const float* v, int nvalid) {
  bf16_t h[4], l[4];
#pragma unroll
  for (int r = 0; r < 4; r++) split_bf(v[r], h[r], l[r]);
  for (int r = 0; r < nvalid; r++) {
    pn[0][(row0 + r) * ldp + col] = h[r];
    pn[1][(row0 + r) * ldp + col] = l[r];
  }
  if (nvalid == 4) {
    *(u32x2*)(pt[0] + col * ldtp + row0) = u32x2{pack2(h[0], h[1]), pack2(h[2], h[3])};
    *(u32x2*)(pt[1] + col * ldtp + row0) = u32x2{pack2(l[0], l[1]), pack2(l[2], l[3])};
  } else {
    for (int r = 0; r < nvalid; r++) {
      pt[0][col * ldtp + row0 + r] = h[r];
      pt[1][col * ldtp + row0 + r] = l[r];
    }
  }
}

// two floats -> packed bf16 pair (RNE, one v_cvt_pk_bf16_f32)
typedef float f32x2v __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t cvt2(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2v){a, b}, bf16x2v));
}
// hi/lo split of 8 floats with packed conversions: hi = RNE(x), lo = RNE(x - hi)
__device__ __forceinline__ void split8p(const float* v, bf16x8& hi, bf16x8& lo) {
  u32x4 h, l;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const uint32_t hp = cvt2(v[2 * i], v[2 * i + 1]);
    h[i] = hp;
    l[i] = cvt2(v[2 * i] - __uint_as_float(hp << 16), v[2 * i + 1] - __uint_as_float(hp & 0xffff0000u));
  }
  hi = as_bf8(h);
  lo = as_bf8(l);
}
__device__ __forceinline__ float fexp2(float x) { return __builtin_amdgcn_exp2f(x); }

// ------------------------------------------------------------------ forward
// Lane (j, g) of wave w owns query q = 64*qb + 16w + j.  S^T = K Q^T puts
// the scores of keys 16sb + 4g + r of that query in the lane (raw dot
// products; the scale folds into the exp2 argument), so the online-softmax
// statistics are per lane after two cross-row shuffles, and O^T = V^T P^T
// (A = V^T rows in the permuted key order of the lane's k-slots, B = the
// lane's own P as hi/lo) leaves O^T[dims 16d + 4g + r][q] in the same lane:
// the rescale and the final normalisation need no shuffles.  Masks are
// applied on the diagonal block only (and past T when T is ragged).
template <bool FULLT>
__global__ __launch_bounds__(256) void k_attn_fwd(AttnArgs a) {
  __shared__ __attribute__((aligned(16))) bf16_t sK[QB * LS];
  __shared__ __attribute__((aligned(16))) bf16_t sVt[DH * LS];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g = lane >> 4, j = lane & 15;
  const int qb = (int)gridDim.x - 1 - (int)blockIdx.x;  // longest blocks first
  const int h = blockIdx.y, b = blockIdx.z;
  const int kvh = h / (int)(a.HQ / a.HK);
  const int T = (int)a.T;
  const int qloc = wave * 16 + j;
  const int myq = qb * QB + qloc;
  const float sc = 0.125f * LOG2E;  // DH^-1/2 * log2(e)
  const int ldk = (int)a.ldk, ldv = (int)a.ldv;

  bf16x8 qf[2];
  {
    const bf16_t* qrow = a.q + ((size_t)b * T + myq) * a.ldq + h * DH;
#pragma unroll
    for (int c = 0; c < 2; c++)
      qf[c] = as_bf8((FULLT || myq < T) ? *(const u32x4*)(qrow + 32 * c + 8 * g) : u32x4{0, 0, 0, 0});
  }
  f32x4 o[4];
#pragma unroll
  for (int d = 0; d < 4; d++) o[d] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, l = 0.f;  // running max (scaled, log2 units) and sum of this lane's query

  const bf16_t* kbase = a.k + (size_t)b * T * a.ldk + kvh * DH;
  const bf16_t* vbase = a.v + (size_t)b * T * a.ldv + kvh * DH;
  // the next key block is fetched into registers while this one computes:
  // K as 16-byte row chunks, V as the 8-row x 2-column pieces of its
  // transposed LDS tile (two 16-byte LDS runs per piece)
  u32x4 pk[2];
  uint32_t pv[8];
  const int vrg = threadIdx.x >> 5, vcp = threadIdx.x & 31;
  auto fetch = [&](int kb) {
#pragma unroll
    for (int p = 0; p < 2; p++) {
      const int ch = threadIdx.x + p * 256, r = ch >> 3, c8 = (ch & 7) * 8;
      const int row = kb * QB + r;
      pk[p] = (FULLT || row < T) ? *(const u32x4*)(kbase + row * ldk + c8) : u32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const int row = kb * QB + vrg * 8 + i;
      pv[i] = (FULLT || row < T) ? *(const uint32_t*)(vbase + row * ldv + 2 * vcp) : 0u;
    }
  };
  auto commit = [&]() {
#pragma unroll
    for (int p = 0; p < 2; p++) {
      const int ch = threadIdx.x + p * 256, r = ch >> 3, c8 = (ch & 7) * 8;
      *(u32x4*)(sK + r * LS + c8) = pk[p];
    }
    bf16_t* d0 = sVt + (2 * vcp) * LS + vrg * 8;
    *(u32x4*)d0 = u32x4{(pv[0] & 0xffffu) | (pv[1] << 16), (pv[2] & 0xffffu) | (pv[3] << 16),
                        (pv[4] & 0xffffu) | (pv[5] << 16), (pv[6] & 0xffffu) | (pv[7] << 16)};
    *(u32x4*)(d0 + LS) = u32x4{(pv[0] >> 16) | (pv[1] & 0xffff0000u), (pv[2] >> 16) | (pv[3] & 0xffff0000u),
                               (pv[4] >> 16) | (pv[5] & 0xffff0000u), (pv[6] >> 16) | (pv[7] & 0xffff0000u)};
  };
  fetch(0);
  for (int kb = 0; kb <= qb; kb++) {
    __syncthreads();
    commit();
    __syncthreads();
    if (kb < qb) fetch(kb + 1);
    f32x4 st[4];
#pragma unroll
    for (int sb = 0; sb < 4; sb++) {
      st[sb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < 2; c++)
        st[sb] = mfma(as_bf8(*(const u32x4*)(sK + (sb * 16 + j) * LS + 32 * c + 8 * g)), qf[c], st[sb]);
    }
    if (kb == qb) {  // causal mask inside the diagonal block
#pragma unroll
      for (int sb = 0; sb < 4; sb++)
#pragma unroll
        for (int r = 0; r < 4; r++)
          if (sb * 16 + 4 * g + r > qloc) st[sb][r] = -INFINITY;
    }
    if (!FULLT && (kb + 1) * QB > T) {
#pragma unroll
      for (int sb = 0; sb < 4; sb++)
#pragma unroll
        for (int r = 0; r < 4; r++)
          if (kb * QB + sb * 16 + 4 * g + r >= T) st[sb][r] = -INFINITY;
    }
    float bm = fmaxf(fmaxf(fmaxf(st[0][0], st[0][1]), fmaxf(st[0][2], st[0][3])),
                     fmaxf(fmaxf(st[1][0], st[1][1]), fmaxf(st[1][2], st[1][3])));
    bm = fmaxf(bm, fmaxf(fmaxf(fmaxf(st[2][0], st[2][1]), fmaxf(st[2][2], st[2][3])),
                         fmaxf(fmaxf(st[3][0], st[3][1]), fmaxf(st[3][2], st[3][3]))));
    bm = fmaxf(bm, __shfl_xor(bm, 16, 64));
    bm = fmaxf(bm, __shfl_xor(bm, 32, 64));
    const float mnew = fmaxf(m, bm * sc);  // finite: key 0 is visible to every query
    const float alpha = fexp2(m - mnew);   // 0 on the first block
    float ps = 0.f;
    float pr[4][4];
#pragma unroll
    for (int sb = 0; sb < 4; sb++)
#pragma unroll
      for (int r = 0; r < 4; r++) {
        pr[sb][r] = fexp2(fmaf(st[sb][r], sc, -mnew));
        ps += pr[sb][r];
      }
    ps += __shfl_xor(ps, 16, 64);
    ps += __shfl_xor(ps, 32, 64);
    l = fmaf(l, alpha, ps);
    m = mnew;
#pragma unroll
    for (int d = 0; d < 4; d++) o[d] *= alpha;
#pragma unroll
    for (int c = 0; c < 2; c++) {
      const float p8[8] = {pr[2 * c][0], pr[2 * c][1], pr[2 * c][2], pr[2 * c][3],
                           pr[2 * c + 1][0], pr[2 * c + 1][1], pr[2 * c + 1][2], pr[2 * c + 1][3]};
      bf16x8 ph, pl;
      split8p(p8, ph, pl);
#pragma unroll
      for (int d = 0; d < 4; d++) {
        const bf16x8 vf = ld_perm(sVt + (16 * d + j) * LS, 32 * c + 4 * g, 32 * c + 16 + 4 * g);
        o[d] = mfma(vf, ph, o[d]);
        o[d] = mfma(vf, pl, o[d]);
      }
    }
  }
  // O[q][16d + 4g + r] = o[d][r] / l: 4 consecutive dims per store; O^T rows
  if (FULLT || myq < T) {
    const float il = 1.f / l;
    bf16_t* orow = a.out + ((size_t)b * T + myq) * a.ldo + h * DH;
#pragma unroll
    for (int d = 0; d < 4; d++) {
      const float v0 = o[d][0] * il, v1 = o[d][1] * il, v2 = o[d][2] * il, v3 = o[d][3] * il;
      *(u32x2*)(orow + 16 * d + 4 * g) = u32x2{cvt2(v0, v1), cvt2(v2, v3)};
      if (a.ot) {
        bf16_t* dst = a.ot + (size_t)(h * DH + 16 * d + 4 * g) * a.ldot + (size_t)b * T + myq;
        dst[0] = f2bf(v0);
        dst[a.ldot] = f2bf(v1);
        dst[2 * a.ldot] = f2bf(v2);
        dst[3 * a.ldot] = f2bf(v3);
      }
    }
    if (g == 0) a.lse[((size_t)b * T + myq) * a.HQ + h] = (m + log2f(l)) * LN2;
  }
}

template <typename K>
void launch_attn(K kernel_full, K kernel_ragged, hipStream_t s, const AttnArgs& a, dim3 grid) {
  hipLaunchKernelGGL((a.T % QB == 0) ? kernel_full : kernel_ragged, grid, dim3(256), 0, s, a);
}

// ------------------------------------------------------------- backward dQ
__global__ __launch_bounds__(256) void k_attn_dq(AttnArgs a) {
  __shared__ __attribute__((aligned(16))) bf16_t sK[QB * LS];
  __shared__ __attribute__((aligned(16))) bf16_t sV[QB * LS];
  __shared__ __attribute__((aligned(16))) bf16_t sKt[DH * LS];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g = lane >> 4, j = lane & 15;
  const long qb = (long)gridDim.x - 1 - blockIdx.x;
  const long h = blockIdx.y, b = blockIdx.z;
  const long kvh = h / (a.HQ / a.HK);
  const long T = a.T;
  const long qrow0 = qb * QB + wave * 16;
  const long myq = qrow0 + j;
  const float sc = 0.125f * LOG2E;

  bf16x8 qf[2], dh[2], dl[2];
  float delta_part = 0.f;
#pragma unroll
  for (int c = 0; c < 2; c++) {
    u32x4 qv = u32x4{0, 0, 0, 0};
    float dov[8], ov[8];
    if (myq < T) {
      qv = *(const u32x4*)(a.q + (b * T + myq) * a.ldq + h * DH + 32 * c + 8 * g);
      const float* dp = a.dout + (b * T + myq) * a.lddo + h * DH + 32 * c + 8 * g;
      float4 x0 = *(const float4*)dp, x1 = *(const float4*)(dp + 4);
      dov[0] = x0.x; dov[1] = x0.y; dov[2] = x0.z; dov[3] = x0.w; dov[4] = x1.x; dov[5] = x1.y; dov[6] = x1.z; dov[7] = x1.w;
      u32x4 ow = *(const u32x4*)(a.o + (b * T + myq) * a.ldo + h * DH + 32 * c + 8 * g);
      uint32_t w4[4] = {ow.x, ow.y, ow.z, ow.w};
#pragma unroll
      for (int i = 0; i < 4; i++) {
        ov[2 * i] = bf2f((bf16_t)(w4[i] & 0xffff));
        ov[2 * i + 1] = bf2f((bf16_t)(w4[i] >> 16));
      }
    } else {
#pragma unroll
      for (int i = 0; i < 8; i++) dov[i] = ov[i] = 0.f;
    }
    qf[c] = as_bf8(qv);
    split8(dov, dh[c], dl[c]);
#pragma unroll
    for (int i = 0; i < 8; i++) delta_part += dov[i] * ov[i];
  }
  delta_part += __shfl_xor(delta_part, 16, 64);
  delta_part += __shfl_xor(delta_part, 32, 64);
  const float delta = delta_part;
  float lse2 = 0.f;
  if (myq < T) {
    lse2 = a.lse[(b * T + myq) * a.HQ + h] * LOG2E;
    if (g == 0) a.delta[(b * T + myq) * a.HQ + h] = delta;
  }

  f32x4 dq[4];
#pragma unroll
  for (int d = 0; d < 4; d++) dq[d] = f32x4{0.f, 0.f, 0.f, 0.f};
  const bf16_t* kbase = a.k + b * T * a.ldk + kvh * DH;
  const bf16_t* vbase = a.v + b * T * a.ldv + kvh * DH;
  // the next key block is fetched into registers while this one computes
  // (K, V as 16-byte row chunks; K again as the 8-row x 2-column pieces of
  // the transposed tile, written to LDS as two 16-byte runs)
  u32x4 pk[2], pv[2];
  uint32_t pkt[8];
  const int trg = threadIdx.x >> 5, tcp = threadIdx.x & 31;
  auto fetch = [&](long kb) {
#pragma unroll
    for (int p = 0; p < 2; p++) {
      const int ch = threadIdx.x + p * 256, r = ch >> 3, c8 = (ch & 7) * 8;
      const long row = kb * QB + r;
      pk[p] = pv[p] = u32x4{0, 0, 0, 0};
      if (row < T) {
        pk[p] = *(const u32x4*)(kbase + row * a.ldk + c8);
        pv[p] = *(const u32x4*)(vbase + row * a.ldv + c8);
      }
    }
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const long row = kb * QB + trg * 8 + i;
      pkt[i] = row < T ? *(const uint32_t*)(kbase + row * a.ldk + 2 * tcp) : 0u;
    }
  };
  auto commit = [&]() {
#pragma unroll
    for (int p = 0; p < 2; p++) {
      const int ch = threadIdx.x + p * 256, r = ch >> 3, c8 = (ch & 7) * 8;
      *(u32x4*)(sK + r * LS + c8) = pk[p];
      *(u32x4*)(sV + r * LS + c8) = pv[p];
    }
    bf16_t* d0 = sKt + (2 * tcp) * LS + trg * 8;
    *(u32x4*)d0 = u32x4{(pkt[0] & 0xffffu) | (pkt[1] << 16), (pkt[2] & 0xffffu) | (pkt[3] << 16),
                        (pkt[4] & 0xffffu) | (pkt[5] << 16), (pkt[6] & 0xffffu) | (pkt[7] << 16)};
    *(u32x4*)(d0 + LS) = u32x4{(pkt[0] >> 16) | (pkt[1] & 0xffff0000u), (pkt[2] >> 16) | (pkt[3] & 0xffff0000u),
                               (pkt[4] >> 16) | (pkt[5] & 0xffff0000u), (pkt[6] >> 16) | (pkt[7] & 0xffff0000u)};
  };
  fetch(0);
  for (long kb = 0; kb <= qb; kb++) {
    __syncthreads();
    commit();
    __syncthreads();
    if (kb < qb) fetch(kb + 1);
    float ds[4][4];
#pragma unroll
    for (int sb = 0; sb < 4; sb++) {
      f32x4 st = f32x4{0.f, 0.f, 0.f, 0.f}, dp = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < 2; c++) {
        st = mfma(as_bf8(*(const u32x4*)(sK + (sb * 16 + j) * LS + 32 * c + 8 * g)), qf[c], st);
        bf16x8 vf = as_bf8(*(const u32x4*)(sV + (sb * 16 + j) * LS + 32 * c + 8 * g));
        dp = mfma(vf, dh[c], dp);
        dp = mfma(vf, dl[c], dp);
      }
#pragma unroll
      for (int r = 0; r < 4; r++) {
        long key = kb * QB + sb * 16 + 4 * g + r;
        float p = (key <= myq && key < T) ? exp2f(st[r] * sc - lse2) : 0.f;
        ds[sb][r] = p * (dp[r] - delta) * 0.125f;
      }
    }
#pragma unroll
    for (int c = 0; c < 2; c++) {
      float dv8[8] = {ds[2 * c][0], ds[2 * c][1], ds[2 * c][2], ds[2 * c][3],
                      ds[2 * c + 1][0], ds[2 * c + 1][1], ds[2 * c + 1][2], ds[2 * c + 1][3]};
      bf16x8 sh, sl;
      split8(dv8, sh, sl);
#pragma unroll
      for (int d = 0; d < 4; d++) {
        bf16x8 kf = ld_perm(sKt + (16 * d + j) * LS, 32 * c + 4 * g, 32 * c + 16 + 4 * g);
        dq[d] = mfma(sh, kf, dq[d]);
        dq[d] = mfma(sl, kf, dq[d]);
      }
    }
  }
  // epilogue: optional inverse RoPE, pair (2i, 2i+1) in lanes (l, l^1)
  float outv[4][4];
#pragma unroll
  for (int r = 0; r < 4; r++) {
    long qpos = qrow0 + 4 * g + r;
#pragma unroll
    for (int d = 0; d < 4; d++) {
      float x = dq[d][r];
      float y = __shfl_xor(x, 1, 64);
      long col = 16 * d + j;
      if (a.rope && qpos < T) {
        float2 cs = *(const float2*)(a.rope + 2 * (qpos * (DH / 2) + (col >> 1)));
        x = (j & 1) ? (x * cs.x - y * cs.y) : (x * cs.x + y * cs.y);
      }
      outv[d][r] = x;
      if (!a.pq[0] && qpos < T) a.dq[(b * T + qpos) * a.lddq + h * DH + col] = x;
    }
  }
  if (a.pq[0]) {
    const long q0 = qrow0 + 4 * g;
    const int nv = (int)(T - q0 < 4 ? (T - q0 > 0 ? T - q0 : 0) : 4);
#pragma unroll
    for (int d = 0; d < 4; d++)
      store_planes(a.pq, a.tq, a.ldp, a.ldtp, b * T + q0, h * DH + 16 * d + j, outv[d], nv);
  }
}

// ------------------------------------------------------------ backward dKV
__global__ __launch_bounds__(256) void k_attn_dkv(AttnArgs a) {
  __shared__ __attribute__((aligned(16))) bf16_t sQ[QB * LS];
  __shared__ __attribute__((aligned(16))) bf16_t sQt[DH * LS];
  __shared__ __attribute__((aligned(16))) bf16_t sDh[QB * LS];
  __shared__ __attribute__((aligned(16))) bf16_t sDl[QB * LS];
  __shared__ __attribute__((aligned(16))) bf16_t sDth[DH * LS];
  __shared__ __attribute__((aligned(16))) bf16_t sDtl[DH * LS];
  __shared__ float sL[QB], sD[QB];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g = lane >> 4, j = lane & 15;
  const long kb = blockIdx.x;
  const long kvh = blockIdx.y, b = blockIdx.z;
  const long T = a.T;
  const long group = a.HQ / a.HK;
  const long krow0 = kb * QB + wave * 16;
  const long myk = krow0 + j;  // key whose fragments this lane supplies
  const float sc = 0.125f * LOG2E;

  bf16x8 kf[2], vf[2];
#pragma unroll
  for (int c = 0; c < 2; c++) {
    u32x4 kv = u32x4{0, 0, 0, 0}, vv = u32x4{0, 0, 0, 0};
    if (myk < T) {
      kv = *(const u32x4*)(a.k + (b * T + myk) * a.ldk + kvh * DH + 32 * c + 8 * g);
      vv = *(const u32x4*)(a.v + (b * T + myk) * a.ldv + kvh * DH + 32 * c + 8 * g);
    }
    kf[c] = as_bf8(kv);
    vf[c] = as_bf8(vv);
  }
  f32x4 dk[4], dv[4];
#pragma unroll
  for (int d = 0; d < 4; d++) dk[d] = dv[d] = f32x4{0.f, 0.f, 0.f, 0.f};
  const long nqb = (T + QB - 1) / QB;
  for (long gi = 0; gi < group; gi++) {
    const long h = kvh * group + gi;
    for (long qb = kb; qb < nqb; qb++) {
      __syncthreads();
      const bf16_t* qbase = a.q + b * T * a.ldq + h * DH;
      stage_bf16(sQ, qbase, a.ldq, qb * QB, T, 0);
      stage_bf16_t(sQt, qbase, a.ldq, qb * QB, T, 0);
      stage_f32_split(sDh, sDl, sDth, sDtl, a.dout + b * T * a.lddo + h * DH, a.lddo, qb * QB, T, 0);
      if (threadIdx.x < QB) {
        long q = qb * QB + threadIdx.x;
        sL[threadIdx.x] = q < T ? a.lse[(b * T + q) * a.HQ + h] * LOG2E : 0.f;
        sD[threadIdx.x] = q < T ? a.delta[(b * T + q) * a.HQ + h] : 0.f;
      }
      __syncthreads();
      float pp[4][4], ds[4][4];
#pragma unroll
      for (int sb = 0; sb < 4; sb++) {
        f32x4 st = f32x4{0.f, 0.f, 0.f, 0.f}, dp = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < 2; c++) {
          st = mfma(as_bf8(*(const u32x4*)(sQ + (sb * 16 + j) * LS + 32 * c + 8 * g)), kf[c], st);
          dp = mfma(as_bf8(*(const u32x4*)(sDh + (sb * 16 + j) * LS + 32 * c + 8 * g)), vf[c], dp);
          dp = mfma(as_bf8(*(const u32x4*)(sDl + (sb * 16 + j) * LS + 32 * c + 8 * g)), vf[c], dp);
        }
#pragma unroll
        for (int r = 0; r < 4; r++) {
          int ql = sb * 16 + 4 * g + r;
          long q = qb * QB + ql;
          float p = (q >= myk && q < T && myk < T) ? exp2f(st[r] * sc - sL[ql]) : 0.f;
          pp[sb][r] = p;
          ds[sb][r] = p * (dp[r] - sD[ql]) * 0.125f;
        }
      }
#pragma unroll
      for (int c = 0; c < 2; c++) {
        float p8[8] = {pp[2 * c][0], pp[2 * c][1], pp[2 * c][2], pp[2 * c][3],
                       pp[2 * c + 1][0], pp[2 * c + 1][1], pp[2 * c + 1][2], pp[2 * c + 1][3]};
        float s8[8] = {ds[2 * c][0], ds[2 * c][1], ds[2 * c][2], ds[2 * c][3],
                       ds[2 * c + 1][0], ds[2 * c + 1][1], ds[2 * c + 1][2], ds[2 * c + 1][3]};
        bf16x8 ph, pl, sh, sl;
        split8(p8, ph, pl);
        split8(s8, sh, sl);
#pragma unroll
        for (int d = 0; d < 4; d++) {
          const int ra = 32 * c + 4 * g, rb = 32 * c + 16 + 4 * g;
          bf16x8 doh = ld_perm(sDth + (16 * d + j) * LS, ra, rb);
          bf16x8 dol = ld_perm(sDtl + (16 * d + j) * LS, ra, rb);
          bf16x8 qt = ld_perm(sQt + (16 * d + j) * LS, ra, rb);
          dv[d] = mfma(ph, doh, dv[d]);
          dv[d] = mfma(ph, dol, dv[d]);
          dv[d] = mfma(pl, doh, dv[d]);
          dk[d] = mfma(sh, qt, dk[d]);
          dk[d] = mfma(sl, qt, dk[d]);
        }
      }
    }
  }
  float kout[4][4], vout[4][4];
#pragma unroll
  for (int r = 0; r < 4; r++) {
    long kpos = krow0 + 4 * g + r;
#pragma unroll
    for (int d = 0; d < 4; d++) {
      float x = dk[d][r];
      float y = __shfl_xor(x, 1, 64);
      long col = 16 * d + j;
      if (a.rope && kpos < T) {
        float2 cs = *(const float2*)(a.rope + 2 * (kpos * (DH / 2) + (col >> 1)));
        x = (j & 1) ? (x * cs.x - y * cs.y) : (x * cs.x + y * cs.y);
      }
      kout[d][r] = x;
      vout[d][r] = dv[d][r];
      if (!a.pk[0] && kpos < T) {
        a.dk[(b * T + kpos) * a.lddk + kvh * DH + col] = x;
        a.dv[(b * T + kpos) * a.lddv + kvh * DH + col] = dv[d][r];
      }
    }
  }
  if (a.pk[0]) {
    const long k0 = krow0 + 4 * g;
    const int nv = (int)(T - k0 < 4 ? (T - k0 > 0 ? T - k0 : 0) : 4);
#pragma unroll
    for (int d = 0; d < 4; d++) {
      store_planes(a.pk, a.tk, a.ldp, a.ldtp, b * T + k0, kvh * DH + 16 * d + j, kout[d], nv);
      store_planes(a.pv, a.tv, a.ldp, a.ldtp, b * T + k0, kvh * DH + 16 * d + j, vout[d], nv);
    }
  }
}

// --------------------------------------- backward dKV, one query head each
// MFMA-layout path.  Workgroup (key block, query head, batch): the dK / dV
// contribution of ONE query head of the group, fp32, into
// part[gi][row][dK | dV] (gi = head index inside its group); the next query
// block is fetched into registers while the current one computes, and the
// transposed LDS tiles (Q^T, dO^T) are written from those registers.  The
// group sum (fixed order), the inverse RoPE of dK and the plane split happen
// in k_attn_kv_reduce.  3x the workgroups of k_attn_dkv and a third of the
// serial loop, for one extra pass over 3 * B*T * 2*KV floats.
__global__ __launch_bounds__(256) void k_attn_dkv_h(AttnArgs a, float* __restrict__ part) {
  __shared__ __attribute__((aligned(16))) bf16_t smem[6 * QB * LS];
  bf16_t* sQ = smem;
  bf16_t* sQt = smem + QB * LS;
  bf16_t* sDh = smem + 2 * QB * LS;
  bf16_t* sDl = smem + 3 * QB * LS;
  bf16_t* sDth = smem + 4 * QB * LS;
  bf16_t* sDtl = smem + 5 * QB * LS;
  __shared__ float sL[QB], sD[QB];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g = lane >> 4, j = lane & 15;
  const long kb = blockIdx.x;
  const long h = blockIdx.y, b = blockIdx.z;
  const long T = a.T;
  const long group = a.HQ / a.HK;
  const long kvh = h / group, gi = h % group;
  const long krow0 = kb * QB + wave * 16;
  const long myk = krow0 + j;
  const float sc = 0.125f * LOG2E;

  bf16x8 kf[2], vf[2];
#pragma unroll
  for (int c = 0; c < 2; c++) {
    u32x4 kv = u32x4{0, 0, 0, 0}, vv = u32x4{0, 0, 0, 0};
    if (myk < T) {
      kv = *(const u32x4*)(a.k + (b * T + myk) * a.ldk + kvh * DH + 32 * c + 8 * g);
      vv = *(const u32x4*)(a.v + (b * T + myk) * a.ldv + kvh * DH + 32 * c + 8 * g);
    }
    kf[c] = as_bf8(kv);
    vf[c] = as_bf8(vv);
  }
  f32x4 dk[4], dv[4];
#pragma unroll
  for (int d = 0; d < 4; d++) dk[d] = dv[d] = f32x4{0.f, 0.f, 0.f, 0.f};

  const bf16_t* qbase = a.q + b * T * a.ldq + h * DH;
  const float* dbase = a.dout + b * T * a.lddo + h * DH;
  // next query block in registers: Q and dO as row chunks, and again as the
  // 8-row x 2-column pieces of their transposed LDS tiles (two 16-byte runs
  // per piece instead of scattered 2-byte stores)
  u32x4 pq[2];
  float4 pd[2][2];
  uint32_t pqt[8];
  float2 pdt[8];
  float pl = 0.f, pdl = 0.f;
  const int trg = threadIdx.x >> 5, tcp = threadIdx.x & 31;
  auto fetch = [&](long qb) {
#pragma unroll
    for (int p = 0; p < 2; p++) {
      const int ch = threadIdx.x + p * 256, r = ch >> 3, c8 = (ch & 7) * 8;
      const long row = qb * QB + r;
      pq[p] = u32x4{0, 0, 0, 0};
      pd[p][0] = pd[p][1] = make_float4(0.f, 0.f, 0.f, 0.f);
      if (row < T) {
        pq[p] = *(const u32x4*)(qbase + row * a.ldq + c8);
        pd[p][0] = *(const float4*)(dbase + row * a.lddo + c8);
        pd[p][1] = *(const float4*)(dbase + row * a.lddo + c8 + 4);
      }
    }
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const long row = qb * QB + trg * 8 + i;
      pqt[i] = 0u;
      pdt[i] = make_float2(0.f, 0.f);
      if (row < T) {
        pqt[i] = *(const uint32_t*)(qbase + row * a.ldq + 2 * tcp);
        pdt[i] = *(const float2*)(dbase + row * a.lddo + 2 * tcp);
      }
    }
    if (threadIdx.x < QB) {
      const long q = qb * QB + threadIdx.x;
      pl = q < T ? a.lse[(b * T + q) * a.HQ + h] * LOG2E : 0.f;
      pdl = q < T ? a.delta[(b * T + q) * a.HQ + h] : 0.f;
    }
  };
  auto commit = [&]() {
#pragma unroll
    for (int p = 0; p < 2; p++) {
      const int ch = threadIdx.x + p * 256, r = ch >> 3, c8 = (ch & 7) * 8;
      *(u32x4*)(sQ + r * LS + c8) = pq[p];
      float v8[8] = {pd[p][0].x, pd[p][0].y, pd[p][0].z, pd[p][0].w, pd[p][1].x, pd[p][1].y, pd[p][1].z, pd[p][1].w};
      bf16_t hh[8], ll[8];
#pragma unroll
      for (int i = 0; i < 8; i++) split_bf(v8[i], hh[i], ll[i]);
      *(u32x4*)(sDh + r * LS + c8) = u32x4{pack2(hh[0], hh[1]), pack2(hh[2], hh[3]), pack2(hh[4], hh[5]), pack2(hh[6], hh[7])};
      *(u32x4*)(sDl + r * LS + c8) = u32x4{pack2(ll[0], ll[1]), pack2(ll[2], ll[3]), pack2(ll[4], ll[5]), pack2(ll[6], ll[7])};
    }
    bf16_t* d0 = sQt + (2 * tcp) * LS + trg * 8;
    *(u32x4*)d0 = u32x4{(pqt[0] & 0xffffu) | (pqt[1] << 16), (pqt[2] & 0xffffu) | (pqt[3] << 16),
                        (pqt[4] & 0xffffu) | (pqt[5] << 16), (pqt[6] & 0xffffu) | (pqt[7] << 16)};
    *(u32x4*)(d0 + LS) = u32x4{(pqt[0] >> 16) | (pqt[1] & 0xffff0000u), (pqt[2] >> 16) | (pqt[3] & 0xffff0000u),
                               (pqt[4] >> 16) | (pqt[5] & 0xffff0000u), (pqt[6] >> 16) | (pqt[7] & 0xffff0000u)};
    bf16_t h0[8], l0[8], h1[8], l1[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
      split_bf(pdt[i].x, h0[i], l0[i]);
      split_bf(pdt[i].y, h1[i], l1[i]);
    }
    bf16_t* e = sDth + (2 * tcp) * LS + trg * 8;
    *(u32x4*)e = u32x4{pack2(h0[0], h0[1]), pack2(h0[2], h0[3]), pack2(h0[4], h0[5]), pack2(h0[6], h0[7])};
    *(u32x4*)(e + LS) = u32x4{pack2(h1[0], h1[1]), pack2(h1[2], h1[3]), pack2(h1[4], h1[5]), pack2(h1[6], h1[7])};
    e = sDtl + (2 * tcp) * LS + trg * 8;
    *(u32x4*)e = u32x4{pack2(l0[0], l0[1]), pack2(l0[2], l0[3]), pack2(l0[4], l0[5]), pack2(l0[6], l0[7])};
    *(u32x4*)(e + LS) = u32x4{pack2(l1[0], l1[1]), pack2(l1[2], l1[3]), pack2(l1[4], l1[5]), pack2(l1[6], l1[7])};
    if (threadIdx.x < QB) {
      sL[threadIdx.x] = pl;
      sD[threadIdx.x] = pdl;
    }
  };

  const long nqb = (T + QB - 1) / QB;
  fetch(kb);
  for (long qb = kb; qb < nqb; qb++) {
    __syncthreads();
    commit();
    __syncthreads();
    if (qb + 1 < nqb) fetch(qb + 1);
    float pp[4][4], ds[4][4];
#pragma unroll
    for (int sb = 0; sb < 4; sb++) {
      f32x4 st = f32x4{0.f, 0.f, 0.f, 0.f}, dp = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < 2; c++) {
        st = mfma(as_bf8(*(const u32x4*)(sQ + (sb * 16 + j) * LS + 32 * c + 8 * g)), kf[c], st);
        dp = mfma(as_bf8(*(const u32x4*)(sDh + (sb * 16 + j) * LS + 32 * c + 8 * g)), vf[c], dp);
        dp = mfma(as_bf8(*(const u32x4*)(sDl + (sb * 16 + j) * LS + 32 * c + 8 * g)), vf[c], dp);
      }
#pragma unroll
      for (int r = 0; r < 4; r++) {
        int ql = sb * 16 + 4 * g + r;
        long q = qb * QB + ql;
        float p = (q >= myk && q < T && myk < T) ? exp2f(st[r] * sc - sL[ql]) : 0.f;
        pp[sb][r] = p;
        ds[sb][r] = p * (dp[r] - sD[ql]) * 0.125f;
      }
    }
#pragma unroll
    for (int c = 0; c < 2; c++) {
      float p8[8] = {pp[2 * c][0], pp[2 * c][1], pp[2 * c][2], pp[2 * c][3],
                     pp[2 * c + 1][0], pp[2 * c + 1][1], pp[2 * c + 1][2], pp[2 * c + 1][3]};
      float s8[8] = {ds[2 * c][0], ds[2 * c][1], ds[2 * c][2], ds[2 * c][3],
                     ds[2 * c + 1][0], ds[2 * c + 1][1], ds[2 * c + 1][2], ds[2 * c + 1][3]};
      bf16x8 ph, plo, sh, sl;
      split8(p8, ph, plo);
      split8(s8, sh, sl);
#pragma unroll
      for (int d = 0; d < 4; d++) {
        const int ra = 32 * c + 4 * g, rb = 32 * c + 16 + 4 * g;
        bf16x8 doh = ld_perm(sDth + (16 * d + j) * LS, ra, rb);
        bf16x8 dol = ld_perm(sDtl + (16 * d + j) * LS, ra, rb);
        bf16x8 qt = ld_perm(sQt + (16 * d + j) * LS, ra, rb);
        dv[d] = mfma(ph, doh, dv[d]);
        dv[d] = mfma(ph, dol, dv[d]);
        dv[d] = mfma(plo, doh, dv[d]);
        dk[d] = mfma(sh, qt, dk[d]);
        dk[d] = mfma(sl, qt, dk[d]);
      }
    }
  }
  // stage the block's dK | dV (64 keys x 128 fp32) in LDS, then row stores
  __syncthreads();
  constexpr int OLD = 2 * DH + 4;
  float* so = (float*)smem;
#pragma unroll
  for (int r = 0; r < 4; r++) {
    const int kr = wave * 16 + 4 * g + r;
#pragma unroll
    for (int d = 0; d < 4; d++) {
      so[kr * OLD + 16 * d + j] = dk[d][r];
      so[kr * OLD + DH + 16 * d + j] = dv[d][r];
    }
  }
  __syncthreads();
  const long KV = a.HK * DH, M = a.T * (long)gridDim.z;
  for (int q = threadIdx.x; q < QB * (2 * DH / 4); q += 256) {
    const int kr = q / (2 * DH / 4), c4 = (q % (2 * DH / 4)) * 4;
    const long key = kb * QB + kr;
    if (key >= T) continue;
    const long col = c4 < DH ? kvh * DH + c4 : KV + kvh * DH + (c4 - DH);
    *(float4*)(part + (gi * M + b * T + key) * 2 * KV + col) = *(const float4*)(so + kr * OLD + c4);
  }
}

// dK = sum over the group's query heads (fixed order) with the inverse RoPE,
// dV = sum; both as hi/lo planes, normal (columns N.. of the [rows][ldg]
// gradient) and transposed (rows N.. of [.][ldgt]).  Thread: one column pair
// of dK or dV over 8 rows of a 16-row block (XCD-contiguous block order, so
// the 16-byte transposed pieces of neighbouring blocks meet in one L2).
constexpr int KVR_ROWS = 8;
__global__ __launch_bounds__(256) void k_attn_kv_reduce(const float* __restrict__ part, int group, long M, long T,
                                                        long N, long KV, const float* __restrict__ rope,
                                                        bf16_t* __restrict__ gh, bf16_t* __restrict__ gl, long ldg,
                                                        bf16_t* __restrict__ th, bf16_t* __restrict__ tl, long ldgt) {
  const long nb = gridDim.x, bx = blockIdx.x;
  const long xcd = bx & 7, local = bx >> 3, q8 = nb >> 3, r8 = nb & 7;
  const long row0 = (xcd * q8 + (xcd < r8 ? xcd : r8) + local) * (2 * KVR_ROWS) + (threadIdx.x >> 7) * KVR_ROWS;
  const int sel = (threadIdx.x >> 6) & 1;  // 0: dK, 1: dV
  for (long pc = threadIdx.x & 63; pc < KV / 2; pc += 64) {
    const long col = 2 * pc;
    const long gcol = N + sel * KV + col;
    uint32_t h0[KVR_ROWS / 2], h1[KVR_ROWS / 2], l0[KVR_ROWS / 2], l1[KVR_ROWS / 2];
#pragma unroll
    for (int i = 0; i < KVR_ROWS; i++) {
      const long row = row0 + i;
      float x = 0.f, y = 0.f;
      if (row < M) {
        for (int gi = 0; gi < group; gi++) {
          const float2 v = *(const float2*)(part + ((long)gi * M + row) * 2 * KV + sel * KV + col);
          x += v.x;
          y += v.y;
        }
        if (sel == 0 && rope) {
          const long pos = row % T;
          const float2 cs = *(const float2*)(rope + 2 * (pos * (DH / 2) + ((col % DH) >> 1)));
          const float xe = x * cs.x + y * cs.y, yo = y * cs.x - x * cs.y;
          x = xe;
          y = yo;
        }
      }
      bf16_t hx, lx, hy, ly;
      split_bf(x, hx, lx);
      split_bf(y, hy, ly);
      if (row < M) {
        *(uint32_t*)(gh + row * ldg + gcol) = pack2(hx, hy);
        *(uint32_t*)(gl + row * ldg + gcol) = pack2(lx, ly);
      }
      if (i & 1) {
        h0[i >> 1] |= (uint32_t)hx << 16; h1[i >> 1] |= (uint32_t)hy << 16;
        l0[i >> 1] |= (uint32_t)lx << 16; l1[i >> 1] |= (uint32_t)ly << 16;
      } else {
        h0[i >> 1] = hx; h1[i >> 1] = hy; l0[i >> 1] = lx; l1[i >> 1] = ly;
      }
    }
    if (!th) continue;  // transposed planes are optional
    if (row0 + KVR_ROWS <= M) {
      *(u32x4*)(th + gcol * ldgt + row0) = u32x4{h0[0], h0[1], h0[2], h0[3]};
      *(u32x4*)(th + (gcol + 1) * ldgt + row0) = u32x4{h1[0], h1[1], h1[2], h1[3]};
      *(u32x4*)(tl + gcol * ldgt + row0) = u32x4{l0[0], l0[1], l0[2], l0[3]};
      *(u32x4*)(tl + (gcol + 1) * ldgt + row0) = u32x4{l1[0], l1[1], l1[2], l1[3]};
    } else {
#pragma unroll
      for (int i = 0; i < KVR_ROWS; i++) {
        if (row0 + i >= M) break;
        const int sh = (i & 1) * 16;
        th[gcol * ldgt + row0 + i] = (bf16_t)(h0[i >> 1] >> sh);
        th[(gcol + 1) * ldgt + row0 + i] = (bf16_t)(h1[i >> 1] >> sh);
        tl[gcol * ldgt + row0 + i] = (bf16_t)(l0[i >> 1] >> sh);
        tl[(gcol + 1) * ldgt + row0 + i] = (bf16_t)(l1[i >> 1] >> sh);
      }
    }
  }
}

// The same group reduce without transposed planes: one thread per (row, 8
// consecutive columns of dK | dV), 16-byte loads of each head's partial
// (summed in head order, as above) and 16-byte plane stores.
__global__ __launch_bounds__(256) void k_attn_kv_reduce_rows(const float* __restrict__ part, int group, long M,
                                                             long T, long N, long KV, const float* __restrict__ rope,
                                                             bf16_t* __restrict__ gh, bf16_t* __restrict__ gl,
                                                             long ldg) {
  const long per_row = (2 * KV) >> 3;
  const long item = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (item >= M * per_row) return;
  const long row = item / per_row, c8 = (item - row * per_row) << 3;  // column in [0, 2 KV)
  float v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int gi = 0; gi < group; gi++) {
    const float4* src = (const float4*)(part + ((long)gi * M + row) * 2 * KV + c8);
    const float4 a = src[0], b = src[1];
    v[0] += a.x; v[1] += a.y; v[2] += a.z; v[3] += a.w;
    v[4] += b.x; v[5] += b.y; v[6] += b.z; v[7] += b.w;
  }
  if (c8 < KV && rope) {  // inverse RoPE on dK's pairs
    const long pos = row % T;
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const long col = c8 + 2 * k;
      const float2 cs = *(const float2*)(rope + 2 * (pos * (DH / 2) + ((col % DH) >> 1)));
      const float x = v[2 * k], y = v[2 * k + 1];
      v[2 * k] = x * cs.x + y * cs.y;
      v[2 * k + 1] = y * cs.x - x * cs.y;
    }
  }
  uint32_t h[4], l[4];
#pragma unroll
  for (int k = 0; k < 4; k++) {
    bf16_t ha, la, hb, lb;
    split_bf(v[2 * k], ha, la);
    split_bf(v[2 * k + 1], hb, lb);
    h[k] = pack2(ha, hb);
    l[k] = pack2(la, lb);
  }
  *(u32x4*)(gh + row * ldg + N + c8) = u32x4{h[0], h[1], h[2], h[3]};
  *(u32x4*)(gl + row * ldg + N + c8) = u32x4{l[0], l[1], l[2], l[3]};
}

// ----------------------------------------------- wavefront-per-row kernels
// Any storage dtype, head width <= 128, optional window (hierarchy.py:24,
// 60, 87).  Lanes span the head dimension; keys are walked in order.
struct RowArgs {
  const void *q, *k, *v, *o;
  long ldq, ldk, ldv, ldo;
  void* out;
  float* lse;
  const float* dout;
  long lddo;
  float *dq, *dk, *dv, *delta;
  long lddq, lddk, lddv;
  int dt;
  long B, T, HQ, HK, D, window;
  const float* rope;
  long offset;  // cached forward: T query rows at positions offset .. offset+T-1, keys 0 .. offset+T-1
};

// CACHED: the query rows of one sequence continue a KV cache (hierarchy.py:
// 7-39 with OFFSET): row r sits at position offset + r and reads key rows
// 0 .. offset + r; each row takes the same operations in the same order as
// in the full forward, so the two agree bit for bit.
template <bool CACHED>
__global__ __launch_bounds__(256) void k_attn_fwd_rows(RowArgs a) {
  const int lane = threadIdx.x & 63;
  const long row = blockIdx.x * 4L + (threadIdx.x >> 6);  // (b*T + pos)*HQ + h
  if (row >= a.B * a.T * a.HQ) return;
  const long h = row % a.HQ, bt = row / a.HQ, pos = CACHED ? a.offset + bt : bt % a.T, b = CACHED ? 0 : bt / a.T;
  const long kvh = h / (a.HQ / a.HK);
  const float scale = 1.f / sqrtf((float)a.D);
  float q[2], acc[2] = {0.f, 0.f};
  for (int i = 0; i < 2; i++) {
    long d = lane + 64 * i;
    q[i] = d < a.D ? load_as_f32(a.q, a.dt, bt * a.ldq + h * a.D + d) : 0.f;
  }
  float m = -INFINITY, l = 0.f;
  long first = a.window > 0 ? (pos + 1 - a.window > 0 ? pos + 1 - a.window : 0) : 0;
  for (long p = first; p <= pos; p++) {
    long kr = (b * a.T + p);
    float s = 0.f;
    for (int i = 0; i < 2; i++) {
      long d = lane + 64 * i;
      if (d < a.D) s += q[i] * load_as_f32(a.k, a.dt, kr * a.ldk + kvh * a.D + d);
    }
    s = wave_sum(s) * scale;
    float mn = fmaxf(m, s);
    float al = expf(m - mn), pr = expf(s - mn);
    for (int i = 0; i < 2; i++) {
      long d = lane + 64 * i;
      float vv = d < a.D ? load_as_f32(a.v, a.dt, kr * a.ldv + kvh * a.D + d) : 0.f;
      acc[i] = acc[i] * al + pr * vv;
    }
    l = l * al + pr;
    m = mn;
  }
  for (int i = 0; i < 2; i++) {
    long d = lane + 64 * i;
    if (d < a.D) store_from_f32(a.out, a.dt, bt * a.ldo + h * a.D + d, acc[i] / l);
  }
  if (!CACHED && lane == 0) a.lse[row] = m + logf(l);
}

__device__ __forceinline__ void inv_rope_store(float* dst, const float* rope, long pos, long D, int lane, float x0,
                                               float x1) {
  // lanes hold consecutive columns; pair partner is lane ^ 1 (D even)
  float y0 = __shfl_xor(x0, 1, 64), y1 = __shfl_xor(x1, 1, 64);
  float xs[2] = {x0, x1}, ys[2] = {y0, y1};
  for (int i = 0; i < 2; i++) {
    long d = lane + 64 * i;
    if (d < D) {
      float x = xs[i];
      if (rope) {
        float2 cs = *(const float2*)(rope + 2 * (pos * (D / 2) + (d >> 1)));
        x = (d & 1) ? (x * cs.x - ys[i] * cs.y) : (x * cs.x + ys[i] * cs.y);
      }
      dst[d] = x;
    }
  }
}

__global__ __launch_bounds__(256) void k_attn_dq_rows(RowArgs a) {
  const int lane = threadIdx.x & 63;
  const long row = blockIdx.x * 4L + (threadIdx.x >> 6);
  if (row >= a.B * a.T * a.HQ) return;
  const long h = row % a.HQ, bt = row / a.HQ, pos = bt % a.T, b = bt / a.T;
  const long kvh = h / (a.HQ / a.HK);
  const float scale = 1.f / sqrtf((float)a.D);
  float q[2], dy[2], acc[2] = {0.f, 0.f};
  float dl = 0.f;
  for (int i = 0; i < 2; i++) {
    long d = lane + 64 * i;
    q[i] = d < a.D ? load_as_f32(a.q, a.dt, bt * a.ldq + h * a.D + d) : 0.f;
    dy[i] = d < a.D ? a.dout[bt * a.lddo + h * a.D + d] : 0.f;
    float ov = d < a.D ? load_as_f32(a.o, a.dt, bt * a.ldo + h * a.D + d) : 0.f;
    dl += dy[i] * ov;
  }
  dl = wave_sum(dl);
  if (lane == 0) a.delta[row] = dl;
  const float lse = a.lse[row];
  long first = a.window > 0 ? (pos + 1 - a.window > 0 ? pos + 1 - a.window : 0) : 0;
  for (long p = first; p <= pos; p++) {
    long kr = b * a.T + p;
    float s = 0.f, dp = 0.f, kv[2];
    for (int i = 0; i < 2; i++) {
      long d = lane + 64 * i;
      kv[i] = d < a.D ? load_as_f32(a.k, a.dt, kr * a.ldk + kvh * a.D + d) : 0.f;
      float vv = d < a.D ? load_as_f32(a.v, a.dt, kr * a.ldv + kvh * a.D + d) : 0.f;
      s += q[i] * kv[i];
      dp += dy[i] * vv;
    }
    s = wave_sum(s);
    dp = wave_sum(dp);
    float pr = expf(s * scale - lse);
    float ds = pr * (dp - dl) * scale;
    for (int i = 0; i < 2; i++) acc[i] += ds * kv[i];
  }
  inv_rope_store(a.dq + bt * a.lddq + h * a.D, a.rope, pos, a.D, lane, acc[0], acc[1]);
}

__global__ __launch_bounds__(256) void k_attn_dkv_rows(RowArgs a) {
  const int lane = threadIdx.x & 63;
  const long row = blockIdx.x * 4L + (threadIdx.x >> 6);  // (b*T + pos)*HK + kvh
  if (row >= a.B * a.T * a.HK) return;
  const long kvh = row % a.HK, bt = row / a.HK, pos = bt % a.T, b = bt / a.T;
  const long group = a.HQ / a.HK;
  const float scale = 1.f / sqrtf((float)a.D);
  float k[2], v[2], ak[2] = {0.f, 0.f}, av[2] = {0.f, 0.f};
  for (int i = 0; i < 2; i++) {
    long d = lane + 64 * i;
    k[i] = d < a.D ? load_as_f32(a.k, a.dt, bt * a.ldk + kvh * a.D + d) : 0.f;
    v[i] = d < a.D ? load_as_f32(a.v, a.dt, bt * a.ldv + kvh * a.D + d) : 0.f;
  }
  long end = a.window > 0 ? (pos + a.window < a.T ? pos + a.window : a.T) : a.T;
  for (long gi = 0; gi < group; gi++) {
    long h = kvh * group + gi;
    for (long qp = pos; qp < end; qp++) {
      long qr = (b * a.T + qp);
      float s = 0.f, dp = 0.f, qv[2], dy[2];
      for (int i = 0; i < 2; i++) {
        long d = lane + 64 * i;
        qv[i] = d < a.D ? load_as_f32(a.q, a.dt, qr * a.ldq + h * a.D + d) : 0.f;
        dy[i] = d < a.D ? a.dout[qr * a.lddo + h * a.D + d] : 0.f;
        s += qv[i] * k[i];
        dp += dy[i] * v[i];
      }
      s = wave_sum(s);
      dp = wave_sum(dp);
      long qrow = qr * a.HQ + h;
      float pr = expf(s * scale - a.lse[qrow]);
      float ds = pr * (dp - a.delta[qrow]) * scale;
      for (int i = 0; i < 2; i++) {
        ak[i] += ds * qv[i];
        av[i] += pr * dy[i];
      }
    }
  }
  inv_rope_store(a.dk + bt * a.lddk + kvh * a.D, a.rope, pos, a.D, lane, ak[0], ak[1]);
  for (int i = 0; i < 2; i++) {
    long d = lane + 64 * i;
    if (d < a.D) a.dv[bt * a.lddv + kvh * a.D + d] = av[i];
  }
}

bool use_mfma(int dtype, long head_dim, long window, long t, long ldq, long ldk, long ldv, long ldo,
              const void* q, const void* k, const void* v, const void* o) {
  if (dtype != SJ_BF16 || head_dim != DH) return false;
  if (window > 0 && window < t) return false;
  if ((ldq | ldk | ldv | ldo) % 8) return false;
  // in-sequence offsets (row * leading dimension) are 32-bit in the kernels
  long ld = ldq > ldk ? ldq : ldk;
  ld = ld > ldv ? ld : ldv;
  ld = ld > ldo ? ld : ldo;
  if (t * ld >= (1L << 31)) return false;
  if (((uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)o) % 16) return false;
  return true;
}

}  // namespace

extern "C" int sj_attention_fwd(void* stream, const void* q, long ldq, const void* k, long ldk, const void* v, long ldv,
                                void* o, long ldo, float* lse, int dtype, long batch, long t, long hq, long hk,
                                long head_dim, long window) {
  SJ_REQUIRE(dtype == SJ_F32 || dtype == SJ_BF16, "grouped attention dtype %d", dtype);
  SJ_REQUIRE(batch > 0 && t > 0 && hq > 0 && hk > 0 && hq % hk == 0 && head_dim > 0 && head_dim <= 128 &&
                 head_dim % 2 == 0 && window >= 0,
             "grouped attention sequence/head dimensions");
  SJ_REQUIRE(ldq >= hq * head_dim && ldo >= hq * head_dim && ldk >= hk * head_dim && ldv >= hk * head_dim,
             "grouped attention head width/dtype mismatch");
  hipStream_t s = (hipStream_t)stream;
  if (use_mfma(dtype, head_dim, window, t, ldq, ldk, ldv, ldo, q, k, v, o)) {
    AttnArgs a = {};
    a.q = (const bf16_t*)q; a.k = (const bf16_t*)k; a.v = (const bf16_t*)v;
    a.ldq = ldq; a.ldk = ldk; a.ldv = ldv; a.ldo = ldo;
    a.out = (bf16_t*)o; a.lse = lse; a.T = t; a.HQ = hq; a.HK = hk;
    launch_attn(k_attn_fwd<true>, k_attn_fwd<false>, s, a,
                dim3((unsigned)((t + QB - 1) / QB), (unsigned)hq, (unsigned)batch));
  } else {
    RowArgs a = {};
    a.q = q; a.k = k; a.v = v; a.ldq = ldq; a.ldk = ldk; a.ldv = ldv; a.ldo = ldo;
    a.out = o; a.lse = lse; a.dt = dtype; a.B = batch; a.T = t; a.HQ = hq; a.HK = hk; a.D = head_dim;
    a.window = window;
    long rows = batch * t * hq;
    hipLaunchKernelGGL(k_attn_fwd_rows<false>, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, s, a);
  }
  SJ_LAUNCH_CHECK("hierarchy_attention");
  return SJ_OK;
}

extern "C" int sj_attention_fwd_cached(void* stream, const void* q, long ldq, const void* k, const void* v, long ldkv,
                                       long capacity, int dtype, long tq, long offset, long hq, long hk, long head_dim,
                                       long window, void* o, long ldo) {
  SJ_REQUIRE(dtype == SJ_F32 || dtype == SJ_BF16, "grouped attention dtype %d", dtype);
  SJ_REQUIRE(q && k && v && o && tq > 0 && offset >= 0 && offset + tq <= capacity && hq > 0 && hk > 0 &&
                 hq % hk == 0 && head_dim > 0 && head_dim <= 128 && head_dim % 2 == 0 && window >= 0 &&
                 ldq >= hq * head_dim && ldo >= hq * head_dim && ldkv >= hk * head_dim,
             "grouped attention sequence/head dimensions (cached: offset %ld + rows %ld <= capacity %ld)", offset, tq,
             capacity);
  hipStream_t s = (hipStream_t)stream;
  const bool mfma = dtype == SJ_BF16 && head_dim == 64 && ldq % 8 == 0 && ldkv % 8 == 0 && ldo % 8 == 0 &&
                    ((uintptr_t)q & 15) == 0 && ((uintptr_t)k & 15) == 0 && ((uintptr_t)v & 15) == 0 &&
                    ((uintptr_t)o & 15) == 0;
  if (mfma)
    return sjh::attention_fwd_cached_t(stream, (const uint16_t*)q, ldq, (const uint16_t*)k, (const uint16_t*)v, ldkv,
                                       capacity, tq, offset, hq, hk, window, (uint16_t*)o, ldo);
  RowArgs a = {};
  a.q = q; a.k = k; a.v = v; a.ldq = ldq; a.ldk = ldkv; a.ldv = ldkv; a.ldo = ldo;
  a.out = o; a.dt = dtype; a.B = 1; a.T = tq; a.HQ = hq; a.HK = hk; a.D = head_dim;
  a.window = window; a.offset = offset;
  long rows = tq * hq;
  hipLaunchKernelGGL(k_attn_fwd_rows<true>, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, s, a);
  SJ_LAUNCH_CHECK("hierarchy_attention (cached)");
  return SJ_OK;
}

extern "C" int sj_attention_bwd(void* stream, const void* q, long ldq, const void* k, long ldk, const void* v,
                                long ldv, const void* o, long ldo, const float* lse, const float* dout, long lddo,
                                float* dq, long lddq, float* dk, long lddk, float* dv, long lddv, float* delta,
                                int dtype, long batch, long t, long hq, long hk, long head_dim, long window,
                                const float* rope_table) {
  SJ_REQUIRE(dtype == SJ_F32 || dtype == SJ_BF16, "grouped attention backward dtype %d", dtype);
  SJ_REQUIRE(batch > 0 && t > 0 && hq > 0 && hk > 0 && hq % hk == 0 && head_dim > 0 && head_dim <= 128 &&
                 head_dim % 2 == 0 && window >= 0,
             "grouped attention backward dimensions");
  SJ_REQUIRE(ldq >= hq * head_dim && ldo >= hq * head_dim && lddo >= hq * head_dim && lddq >= hq * head_dim &&
                 ldk >= hk * head_dim && ldv >= hk * head_dim && lddk >= hk * head_dim && lddv >= hk * head_dim,
             "grouped attention backward head/LSE dimensions");
  hipStream_t s = (hipStream_t)stream;
  bool fast = use_mfma(dtype, head_dim, window, t, ldq, ldk, ldv, ldo, q, k, v, o) && lddo % 4 == 0 &&
              ((uintptr_t)dout % 16) == 0;
  if (fast) {
    AttnArgs a = {};
    a.q = (const bf16_t*)q; a.k = (const bf16_t*)k; a.v = (const bf16_t*)v; a.o = (const bf16_t*)o;
    a.ldq = ldq; a.ldk = ldk; a.ldv = ldv; a.ldo = ldo;
    a.lse = (float*)lse; a.dout = dout; a.lddo = lddo;
    a.dq = dq; a.dk = dk; a.dv = dv; a.delta = delta; a.lddq = lddq; a.lddk = lddk; a.lddv = lddv;
    a.T = t; a.HQ = hq; a.HK = hk; a.rope = rope_table;
    unsigned nb = (unsigned)((t + QB - 1) / QB);
    hipLaunchKernelGGL(k_attn_dq, dim3(nb, (unsigned)hq, (unsigned)batch), dim3(256), 0, s, a);
    hipLaunchKernelGGL(k_attn_dkv, dim3(nb, (unsigned)hk, (unsigned)batch), dim3(256), 0, s, a);
  } else {
    RowArgs a = {};
    a.q = q; a.k = k; a.v = v; a.o = o; a.ldq = ldq; a.ldk = ldk; a.ldv = ldv; a.ldo = ldo;
    a.lse = (float*)lse; a.dout = dout; a.lddo = lddo;
    a.dq = dq; a.dk = dk; a.dv = dv; a.delta = delta; a.lddq = lddq; a.lddk = lddk; a.lddv = lddv;
    a.dt = dtype; a.B = batch; a.T = t; a.HQ = hq; a.HK = hk; a.D = head_dim; a.window = window;
    a.rope = rope_table;
    long rows = batch * t * hq;
    hipLaunchKernelGGL(k_attn_dq_rows, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, s, a);
    long krows = batch * t * hk;
    hipLaunchKernelGGL(k_attn_dkv_rows, dim3((unsigned)((krows + 3) / 4)), dim3(256), 0, s, a);
  }
  SJ_LAUNCH_CHECK("hierarchy_attention_backward");
  return SJ_OK;
}

namespace sjh {
int attention_prepare() { return SJ_OK; }
}  // namespace sjh

extern "C" int sj_attention_fwd_t(void* stream, const uint16_t* q, long ldq, const uint16_t* k, long ldk,
                                  const uint16_t* v, long ldv, uint16_t* o, long ldo, float* lse, uint16_t* o_t,
                                  long ldot, long batch, long t, long hq, long hk, long head_dim) {
  SJ_REQUIRE(batch > 0 && t > 0 && hq > 0 && hk > 0 && hq % hk == 0 && head_dim == DH && ldot >= batch * t &&
                 ldot % 4 == 0 && ((uintptr_t)o_t & 7) == 0 && (batch == 1 || t % 4 == 0),
             "grouped attention (transposed output): head_dim must be %d", DH);
  SJ_REQUIRE(use_mfma(SJ_BF16, head_dim, 0, t, ldq, ldk, ldv, ldo, q, k, v, o), "grouped attention: alignment");
  AttnArgs a = {};
  a.q = (const bf16_t*)q; a.k = (const bf16_t*)k; a.v = (const bf16_t*)v;
  a.ldq = ldq; a.ldk = ldk; a.ldv = ldv; a.ldo = ldo;
  a.out = (bf16_t*)o; a.lse = lse; a.T = t; a.HQ = hq; a.HK = hk;
  a.ot = (bf16_t*)o_t; a.ldot = ldot;
  launch_attn(k_attn_fwd<true>, k_attn_fwd<false>, (hipStream_t)stream, a,
              dim3((unsigned)((t + QB - 1) / QB), (unsigned)hq, (unsigned)batch));
  SJ_LAUNCH_CHECK("hierarchy_attention_t");
  return SJ_OK;
}

extern "C" size_t sj_attention_bwd_p_workspace_bytes(long batch, long t, long hq, long hk, long head_dim) {
  if (batch <= 0 || t <= 0 || hq <= 0 || hk <= 0 || hq % hk) return 0;
  return sizeof(float) * (size_t)(hq / hk) * (size_t)(batch * t) * (size_t)(2 * hk * head_dim);
}

// parts: 1 = dQ kernel (also writes Delta), 2 = per-head dK/dV partials
// (reads Delta), 4 = group reduce into planes; 7 = all
int sjh::attention_bwd_p_parts(int parts, void* stream, const uint16_t* q, long ldq, const uint16_t* k, long ldk,
                               const uint16_t* v, long ldv, const uint16_t* o, long ldo, const float* lse,
                               const float* dout, long lddo, float* delta, long batch, long t, long hq, long hk,
                               long head_dim, const float* rope_table, uint16_t* g_hi, uint16_t* g_lo, long ldg,
                               uint16_t* gt_hi, uint16_t* gt_lo, long ldgt, void* workspace, size_t workspace_bytes) {
  SJ_REQUIRE(batch > 0 && t > 0 && hq > 0 && hk > 0 && hq % hk == 0 && head_dim == DH &&
                 ldg >= (hq + 2 * hk) * DH && ldgt >= batch * t && ldgt % 8 == 0 && lddo % 4 == 0 && (batch == 1 || t % 4 == 0) &&
                 ((uintptr_t)dout & 15) == 0 && ((uintptr_t)gt_hi & 15) == 0 && ((uintptr_t)gt_lo & 15) == 0,
             "grouped attention backward (planes): shape/alignment");
  SJ_REQUIRE(use_mfma(SJ_BF16, head_dim, 0, t, ldq, ldk, ldv, ldo, q, k, v, o), "grouped attention: alignment");
  const size_t need = sj_attention_bwd_p_workspace_bytes(batch, t, hq, hk, head_dim);
  if ((parts & 6) && (!workspace || workspace_bytes < need))
    return sjh::fail(SJ_ERR_CAPACITY, "attention_backward: required %zu bytes, available %zu bytes", need,
                     workspace_bytes);
  AttnArgs a = {};
  a.q = (const bf16_t*)q; a.k = (const bf16_t*)k; a.v = (const bf16_t*)v; a.o = (const bf16_t*)o;
  a.ldq = ldq; a.ldk = ldk; a.ldv = ldv; a.ldo = ldo;
  a.lse = (float*)lse; a.dout = dout; a.lddo = lddo; a.delta = delta;
  a.T = t; a.HQ = hq; a.HK = hk; a.rope = rope_table;
  const long N = hq * DH, KV = hk * DH;
  bf16_t* gh = (bf16_t*)g_hi; bf16_t* gl = (bf16_t*)g_lo;
  bf16_t* th = (bf16_t*)gt_hi; bf16_t* tl = (bf16_t*)gt_lo;
  a.pq[0] = gh; a.pq[1] = gl; a.pk[0] = gh + N; a.pk[1] = gl + N; a.pv[0] = gh + N + KV; a.pv[1] = gl + N + KV;
  a.tq[0] = th; a.tq[1] = tl; a.tk[0] = th; a.tk[1] = tl; a.tv[0] = th; a.tv[1] = tl;
  // transposed rows: dq rows [0, N), dk rows [N, N+KV), dv rows [N+KV, N+2KV):
  // the column index passed to store_planes already includes the head
  // offset, so shift the base by the block of rows instead
  a.tk[0] = th + N * ldgt; a.tk[1] = tl + N * ldgt; a.tv[0] = th + (N + KV) * ldgt; a.tv[1] = tl + (N + KV) * ldgt;
  a.ldp = ldg; a.ldtp = ldgt;
  hipStream_t s = (hipStream_t)stream;
  unsigned nb = (unsigned)((t + QB - 1) / QB);
  if (parts & 1) hipLaunchKernelGGL(k_attn_dq, dim3(nb, (unsigned)hq, (unsigned)batch), dim3(256), 0, s, a);
  if (parts & 2)
    hipLaunchKernelGGL(k_attn_dkv_h, dim3(nb, (unsigned)hq, (unsigned)batch), dim3(256), 0, s, a, (float*)workspace);
  if (parts & 4) {
    const long M = batch * t;
    hipLaunchKernelGGL(k_attn_kv_reduce, dim3((unsigned)((M + 2 * KVR_ROWS - 1) / (2 * KVR_ROWS))), dim3(256), 0, s,
                       (const float*)workspace,
                       (int)(hq / hk), M, t, N, KV, rope_table, gh, gl, ldg, th, tl, ldgt);
  }
  SJ_LAUNCH_CHECK("hierarchy_attention_backward_p");
  return SJ_OK;
}

extern "C" int sj_attention_bwd_p(void* stream, const uint16_t* q, long ldq, const uint16_t* k, long ldk,
                                  const uint16_t* v, long ldv, const uint16_t* o, long ldo, const float* lse,
                                  const float* dout, long lddo, float* delta, long batch, long t, long hq, long hk,
                                  long head_dim, const float* rope_table, uint16_t* g_hi, uint16_t* g_lo, long ldg,
                                  uint16_t* gt_hi, uint16_t* gt_lo, long ldgt, void* workspace,
                                  size_t workspace_bytes) {
  return sjh::attention_bwd_p_parts(7, stream, q, ldq, k, ldk, v, ldv, o, ldo, lse, dout, lddo, delta, batch, t, hq,
                                    hk, head_dim, rope_table, g_hi, g_lo, ldg, gt_hi, gt_lo, ldgt, workspace,
                                    workspace_bytes);
}

int sjh::attention_kv_reduce(hipStream_t s, const float* part, long group, long M, long T, long N, long KV,
                             const float* rope, uint16_t* g_hi, uint16_t* g_lo, long ldg, uint16_t* gt_hi,
                             uint16_t* gt_lo, long ldgt) {
  if (!gt_hi && ldg % 8 == 0 && N % 8 == 0 && KV % 4 == 0 && ((uintptr_t)g_hi & 15) == 0 &&
      ((uintptr_t)g_lo & 15) == 0 && ((uintptr_t)part & 15) == 0) {
    const long items = M * (2 * KV / 8);
    hipLaunchKernelGGL(k_attn_kv_reduce_rows, dim3((unsigned)((items + 255) / 256)), dim3(256), 0, s, part, (int)group,
                       M, T, N, KV, rope, (bf16_t*)g_hi, (bf16_t*)g_lo, ldg);
    SJ_LAUNCH_CHECK("hierarchy_attention_kv_reduce");
    return SJ_OK;
  }
  hipLaunchKernelGGL(k_attn_kv_reduce, dim3((unsigned)((M + 2 * KVR_ROWS - 1) / (2 * KVR_ROWS))), dim3(256), 0, s, part,
                     (int)group, M, T, N, KV, rope, (bf16_t*)g_hi, (bf16_t*)g_lo, ldg, (bf16_t*)gt_hi, (bf16_t*)gt_lo,
                     ldgt);
  SJ_LAUNCH_CHECK("hierarchy_attention_kv_reduce");
  return SJ_OK;
}
