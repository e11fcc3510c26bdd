// GQA causal attention for the MFMA-layout step (bf16 storage, head_dim 64,
// T a multiple of 64), forward and backward, fed by producers that already
// wrote every operand in the orientation the MFMA wants:
//   q|k|v [M][NQKV] (the QKV projection, RoPE applied), dO as hi/lo planes
//   [M][NQ] (the attention-output projection's dX), LSE and Delta
//   transposed [HQ][ldt].
// Every 64 x 64 tile streams global -> LDS in row orientation with
// global_load_lds_dwordx4, three stages deep, XOR-swizzled (chunk c of row
// r at c ^ sw(r)); a fragment of the tile itself is one 16-byte LDS read,
// a fragment of its transpose two ds_read_b64_tr_b16 (tr_frag).
//
// Layout trick: the rows of each 16-row block of S are read in a permuted
// key (or query) order, row i of block sb = 32(sb/2) + 8(i/4) + 4(sb%2) +
// i%4, so the 8 k-slots a lane contributes to the following P-product are 8
// consecutive keys -- one 16-byte chunk of the transposed tile.
//
// Forward (hierarchy.py:7-39): lane (j, g) of wave w owns query 64qb + 16w
// + j; S^T = K Q^T, online softmax per lane (two cross-row shuffles), O^T =
// V^T P^T with P as hi/lo.  Backward (hierarchy.py:42-104): dQ^T = K^T dS^T
// per query block (writes Delta), then per (key block, query head) dK^T =
// Q^T dS and dV^T = dO^T P into fp32 per-head partials that the group
// reduce of attention.hip sums in a fixed order (no atomics).
#include <math.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <functional>
#include <map>
#include <mutex>
#include <tuple>
#include <vector>

#include <hip/hip_ext.h>

#include "common.h"

using namespace sj;

namespace {

constexpr int DH = 64;
constexpr int QB = 64;
// DMA pipeline stages per kernel (stages issued ahead = stages - 1)
#ifndef SJ_ATTN_FWD_STAGES
#define SJ_ATTN_FWD_STAGES 3
#endif
#ifndef SJ_ATTN_DQ_STAGES
#define SJ_ATTN_DQ_STAGES 3
#endif
#ifndef SJ_ATTN_DKV_STAGES
#define SJ_ATTN_DKV_STAGES 2
#endif
// waves per SIMD the dK/dV kernels are compiled for (0: the compiler's
// choice, 2 at their register use); 3 fits their 50 KB of LDS three
// workgroups to a CU
#ifndef SJ_ATTN_BWD_WAVES
#define SJ_ATTN_BWD_WAVES 3
#endif
#if SJ_ATTN_BWD_WAVES
#define SJ_BWD_OCC __attribute__((amdgpu_waves_per_eu(SJ_ATTN_BWD_WAVES, SJ_ATTN_BWD_WAVES)))
#else
#define SJ_BWD_OCC
#endif
constexpr int NS_FWD = SJ_ATTN_FWD_STAGES;
constexpr int NS_DQ = SJ_ATTN_DQ_STAGES;
constexpr int NST = SJ_ATTN_DKV_STAGES;  // dK/dV stages
constexpr int TILE = 64 * 64;      // bf16 elements per tile
constexpr int TBYTES = TILE * 2;
constexpr float LOG2E = 1.4426950408889634f;
constexpr float LN2 = 0.6931471805599453f;

__device__ __attribute__((aligned(64))) uint8_t g_zero_t[64];  // zero source for masked DMA lanes

template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}
// LDS-DMA of one 16-byte chunk per lane to lds_addr + 16 * lane
__device__ __forceinline__ void dma16(const void* src, uint32_t lds_addr) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(lds_addr)
               : "memory", "m0");
}
// wait until at most n (0 <= n <= N) stages of PER loads each are in flight
template <int PER, int N>
__device__ __forceinline__ void wait_stages(int n) {
  if constexpr (N > 0) {
    if (n >= N) {
      wait_vm<PER * N>();
      return;
    }
    wait_stages<PER, N - 1>(n);
  } else {
    wait_vm<0>();
  }
}
__device__ __forceinline__ void block_barrier() {
  __builtin_amdgcn_s_waitcnt((15) | (3 << 14) | (7 << 4) | (0 << 8));  // lgkmcnt(0)
  asm volatile("s_barrier" ::: "memory");
}

__device__ __forceinline__ bf16x8 as_bf8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }
__device__ __forceinline__ f32x4 mfma(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
// 16-byte slot of chunk c in row r is c ^ sw(r): the row's low bits spread
// a column over the slots, and the 8-row block's index moves the rows that
// a transpose read takes from four consecutive blocks to different banks
__device__ __forceinline__ int sw(int row) { return (row & 7) ^ (((row >> 3) & 3) << 1); }
// chunk `ch` (8 bf16) of row `row` of a swizzled tile
__device__ __forceinline__ bf16x8 tf(const bf16_t* tile, int row, int ch) {
  return as_bf8(*(const u32x4*)(tile + row * 64 + ((ch ^ sw(row)) << 3)));
}
// permuted row of block sb read by A-operand lane j (see the file comment)
__device__ __forceinline__ int prow(int sb, int j) { return 32 * (sb >> 1) + 8 * (j >> 2) + 4 * (sb & 1) + (j & 3); }

// Transposed MFMA fragment from a swizzled row tile with ds_read_b64_tr_b16:
// lane (j, g) receives tile[row0 + 8g + 0..7][col0 + j] (eight consecutive
// rows of one column: the operand of the transposed tile).  Within a group
// of 16 lanes the instruction hands lane i element (i & 3) of the 8 bytes
// that source lane 4e + (i >> 2) read, as its e-th value; so source lane
// 4e + m of the group reads row row0 + 8g + 4h + e at columns col0 + 4m ..
// +3 (read h = 0, 1 gives rows +0..3 and +4..7).  row0 % 8 == 0, col0 % 16
// == 0.
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef short s16x8 __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
__device__ __forceinline__ bf16x8 tr_frag(const bf16_t* tile, int row0, int col0, int lane) {
  const int g = lane >> 4, e = (lane >> 2) & 3, m = lane & 3;
  const int col = col0 + 4 * m;
  s16x4 v[2];
#pragma unroll
  for (int h = 0; h < 2; h++) {
    const int row = row0 + 8 * g + 4 * h + e;
    const bf16_t* src = tile + row * 64 + (((col >> 3) ^ sw(row)) << 3) + (col & 7);
    v[h] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(src));
  }
  const s16x8 w = __builtin_shufflevector(v[0], v[1], 0, 1, 2, 3, 4, 5, 6, 7);
  return __builtin_bit_cast(bf16x8, w);
}

typedef float f32x2v __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t cvt2(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2v){a, b}, bf16x2v));
}
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
__device__ __forceinline__ float bflo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bfhi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

struct TArgs {
  const bf16_t* qkv;  // [M][ldqkv]: q (HQ*64) | k (HK*64) | v (HK*64), q and k after RoPE
  long ldqkv;
  long ldt;  // row stride of the transposed [.][rows] buffers
  int T, HQ, HK;
  int window;  // keys visible to a query: the `window` last positions up to it (0: every earlier one)
  // forward
  bf16_t* o;  // [M][ldo]
  long ldo;
  float* lse;    // [M][HQ] (reference layout, nullable)
  float* lse_t;  // [HQ][ldt]
  bf16_t* ot;    // O^T [HQ*64][ldot] (nullable)
  long ldot;
  // backward
  const bf16_t* ob;  // O (for Delta)
  const bf16_t *dh, *dl;  // dO planes [M][lddo]
  long lddo;
  const float* lse_in_t;  // [HQ][ldt]
  float* delta_t;         // [HQ][ldt]
  const float* rope;      // inverse-RoPE table (cos, sin) [T][32] or null
  bf16_t *gq[2], *gqt[2];  // dQ planes: normal [M][ldg] at columns h*64, transposed [.][ldgt] at rows h*64
  long ldg, ldgt;
  float* part;  // [group][M][2*HK*64] per-head dK | dV
  uint32_t* cnt;  // grouped backward: the cut walks' meeting counters, PLAN_CUTS per (KV head, sequence)
  int B;        // batch (rows M = B * T)
  // cached forward (one sequence): queries at positions pos0 .. pos0+nq-1
  // in qc [nq][ldqc]; keys and values of positions 0 .. pos0+nq-1 in kc / vc
  // [capacity][ldkc]; query blocks qb0 .. qb0 + gridDim.x - 1
  const bf16_t *qc, *kc, *vc;
  long ldqc, ldkc;
  int pos0, nq, qb0;
};

// DMA of one 64 x 64 bf16 tile (rows r of `src` with stride ld, 8 chunks of
// 16 bytes each): wave w moves rows 16w .. 16w+15 (two instructions).
// valid(r) false -> zeros.
// a pointer every lane holds alike, as a scalar value (the divergence
// analysis cannot always prove it)
__device__ __forceinline__ const uint8_t* uniform_ptr(const void* p) {
  const unsigned long long v = (unsigned long long)(uintptr_t)p;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v), hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return (const uint8_t*)(uintptr_t)(((unsigned long long)hi << 32) | lo);
}
// dma_tile with every row valid: a uniform base (the tile's first row) plus
// a fixed 32-bit byte offset per lane, no vector address arithmetic
__device__ __forceinline__ void dma_tile_all(const bf16_t* src, long ld, uint32_t lds_tile, int wave, int lane) {
  const uint8_t* bs = uniform_ptr(src);
  const int rl = lane >> 3;
#pragma unroll
  for (int k = 0; k < 2; k++) {
    const int r0 = wave * 16 + 8 * k;
    const int r = r0 + rl;
    const int ch = (lane & 7) ^ sw(r);  // LDS slot lane & 7 of row r holds source chunk ch
    const uint32_t off = (uint32_t)((r * ld + ch * 8) * 2);
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1 offset:0" ::"v"(off), "s"(bs),
                 "s"(lds_tile + (uint32_t)(r0 * 128))
                 : "memory", "m0");
  }
}

template <typename Valid>
__device__ __forceinline__ void dma_tile(const bf16_t* src, long ld, uint32_t lds_tile, int wave, int lane,
                                         Valid valid) {
  const int rl = lane >> 3;
#pragma unroll
  for (int k = 0; k < 2; k++) {
    const int r0 = wave * 16 + 8 * k;
    const int r = r0 + rl;
    const int ch = (lane & 7) ^ sw(r);  // LDS slot lane & 7 of row r holds source chunk ch
    const void* s = valid(r) ? (const void*)(src + r * ld + ch * 8) : (const void*)g_zero_t;
    dma16(s, lds_tile + (uint32_t)(r0 * 128));
  }
}

// Workgroup -> (rank, role, head, sequence).  Workgroups are dispatched
// round-robin over the 8 XCDs by linear id (id % 8).  The rank r (the causal
// walk length order: 0 is the longest) varies slowest and (head, sequence)
// fastest, so each XCD receives the same mix of walk lengths and the whole
// launch still starts with the longest walks; with the block index fastest,
// XCD k would receive only block k of every (head, sequence) and the XCD
// holding the longest walks would finish last.  grid = (roles * nb, H, B).
struct WgMap {
  int r, role, h, b;
};
__device__ __forceinline__ WgMap wg_map(int roles) {
  const long H = gridDim.y, HB = H * (long)gridDim.z;
  const long lin = (long)blockIdx.x + (long)gridDim.x * ((long)blockIdx.y + H * (long)blockIdx.z);
  const long rem = lin % (roles * HB), hb = rem % HB;
  WgMap m;
  m.r = (int)(lin / (roles * HB));
  m.role = (int)(rem / HB);
  m.h = (int)(hb % H);
  m.b = (int)(hb / H);
  return m;
}

// ------------------------------------------------------------------ forward
// CACHED: the same per-row arithmetic over a KV cache (Model::forward_cached,
// architecture.rs:474-533): query block qb holds the 64 positions qb*64 ..
// +63, of which pos0 .. pos0+nq-1 are real (read from qc, written to o at
// row position - pos0); key rows at or past pos0+nq load as zeros.  A real
// query sees the same key blocks, masks and operation order as in the full
// forward, so cached and full outputs agree bit for bit.
template <int NS, bool CACHED>
__device__ __forceinline__ void attn2_fwd_body(const TArgs& a, bf16_t* lds) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wave_s = __builtin_amdgcn_readfirstlane(wave);
  const int g = lane >> 4, j = lane & 15;
  const WgMap wm = wg_map(1);
  const int qb = (CACHED ? a.qb0 : 0) + (int)gridDim.x - 1 - wm.r;  // longest blocks first
  const int h = wm.h, b = wm.b;
  const int T = a.T, NQ = a.HQ * DH, NK = a.HK * DH;
  const int kvh = h / (a.HQ / a.HK);
  const int qloc = wave * 16 + j, myq = qb * QB + qloc;
  const long row0 = CACHED ? 0 : (long)b * T;
  const float sc = 0.125f * LOG2E;
  const bool qreal = !CACHED || (myq >= a.pos0 && myq < a.pos0 + a.nq);
  const int klen = CACHED ? a.pos0 + a.nq : 0;

  bf16x8 qf[2];
#pragma unroll
  for (int c = 0; c < 2; c++) {
    if constexpr (CACHED)
      qf[c] = qreal ? as_bf8(*(const u32x4*)(a.qc + (long)(myq - a.pos0) * a.ldqc + h * DH + 32 * c + 8 * g))
                    : as_bf8(u32x4{0u, 0u, 0u, 0u});
    else
      qf[c] = as_bf8(*(const u32x4*)(a.qkv + (row0 + myq) * a.ldqkv + h * DH + 32 * c + 8 * g));
  }

  const long ldk = CACHED ? a.ldkc : a.ldqkv;
  const bf16_t* ksrc = CACHED ? a.kc + kvh * DH : a.qkv + row0 * a.ldqkv + NQ + kvh * DH;
  const bf16_t* vsrc = CACHED ? a.vc + kvh * DH : ksrc + NK;
  const uint32_t base = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)lds);
  auto issue = [&](int kb, int buf) {
    const uint32_t st = base + (uint32_t)(buf * 2 * TBYTES);
    if constexpr (CACHED) {
      auto valid = [&](int r) { return kb * QB + r < klen; };
      dma_tile(ksrc + (long)kb * QB * ldk, ldk, st, wave_s, lane, valid);
      dma_tile(vsrc + (long)kb * QB * ldk, ldk, st + TBYTES, wave_s, lane, valid);
    } else {
      dma_tile_all(ksrc + (long)kb * QB * ldk, ldk, st, wave_s, lane);
      dma_tile_all(vsrc + (long)kb * QB * ldk, ldk, st + TBYTES, wave_s, lane);
    }
  };
  f32x4 o[4];
#pragma unroll
  for (int d = 0; d < 4; d++) o[d] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, l = 0.f;
  // first key block any query of this block sees (window: keys myq-window+1 .. myq)
  const int W = a.window;
  const int kb0 = W > 0 && qb * QB - W + 1 > 0 ? (qb * QB - W + 1) / QB : 0;
  wait_vm<0>();  // the fragments above are in registers before the DMA stream starts

#pragma unroll
  for (int s = 0; s < NS - 1; s++)
    if (kb0 + s <= qb) issue(kb0 + s, s);
  for (int kb = kb0; kb <= qb; kb++) {
    const int it = kb - kb0;
    wait_stages<4, NS - 2>(min(NS - 2, qb - kb));
    block_barrier();
    if (kb + NS - 1 <= qb) issue(kb + NS - 1, (it + NS - 1) % NS);
    const bf16_t* sK = lds + (it % NS) * 2 * TILE;
    const bf16_t* sV = sK + TILE;
    f32x4 st[4];
#pragma unroll
    for (int sb = 0; sb < 4; sb++) {
      st[sb] = f32x4{0.f, 0.f, 0.f, 0.f};
      const int kr = prow(sb, j);
#pragma unroll
      for (int c = 0; c < 2; c++) st[sb] = mfma(tf(sK, kr, 4 * c + g), qf[c], st[sb]);
    }
    if (kb == qb) {  // causal mask inside the diagonal block: key 32c + 8g + 4s + r
#pragma unroll
      for (int sb = 0; sb < 4; sb++)
#pragma unroll
        for (int r = 0; r < 4; r++)
          if (32 * (sb >> 1) + 8 * g + 4 * (sb & 1) + r > qloc) st[sb][r] = -INFINITY;
    }
    if (W > 0 && kb * QB < qb * QB + QB - W) {  // keys before some query's window
#pragma unroll
      for (int sb = 0; sb < 4; sb++)
#pragma unroll
        for (int r = 0; r < 4; r++)
          if (kb * QB + 32 * (sb >> 1) + 8 * g + 4 * (sb & 1) + r < myq - W + 1) st[sb][r] = -INFINITY;
    }
    float bm = fmaxf(fmaxf(fmaxf(st[0][0], st[0][1]), fmaxf(st[0][2], st[0][3])),
                     fmaxf(fmaxf(st[1][0], st[1][1]), fmaxf(st[1][2], st[1][3])));
    bm = fmaxf(bm, fmaxf(fmaxf(fmaxf(st[2][0], st[2][1]), fmaxf(st[2][2], st[2][3])),
                         fmaxf(fmaxf(st[3][0], st[3][1]), fmaxf(st[3][2], st[3][3]))));
    bm = fmaxf(bm, __shfl_xor(bm, 16, 64));
    bm = fmaxf(bm, __shfl_xor(bm, 32, 64));
    const float mnew = fmaxf(m, bm * sc);
    // a row whose keys so far are all outside its window keeps m = -inf: its
    // terms are exp2(-inf) = 0 against the reference point 0
    const float mref = mnew == -INFINITY ? 0.f : mnew;
    const float alpha = fexp2(m - mref);
    float pr[4][4], ps = 0.f;
#pragma unroll
    for (int sb = 0; sb < 4; sb++)
#pragma unroll
      for (int r = 0; r < 4; r++) {
        pr[sb][r] = fexp2(fmaf(st[sb][r], sc, -mref));
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
        const bf16x8 vf = tr_frag(sV, 32 * c, 16 * d, lane);  // V^T rows 16d.., keys 32c + 8g ..
        o[d] = mfma(vf, ph, o[d]);
        o[d] = mfma(vf, pl, o[d]);
      }
    }
  }
  const float il = 1.f / l;
  if constexpr (CACHED) {
    if (!qreal) return;
    bf16_t* orow = a.o + (long)(myq - a.pos0) * a.ldo + h * DH;
#pragma unroll
    for (int d = 0; d < 4; d++) {
      const float v0 = o[d][0] * il, v1 = o[d][1] * il, v2 = o[d][2] * il, v3 = o[d][3] * il;
      *(u32x2*)(orow + 16 * d + 4 * g) = u32x2{cvt2(v0, v1), cvt2(v2, v3)};
    }
    return;
  }
  bf16_t* orow = a.o + (row0 + myq) * a.ldo + h * DH;
#pragma unroll
  for (int d = 0; d < 4; d++) {
    const float v0 = o[d][0] * il, v1 = o[d][1] * il, v2 = o[d][2] * il, v3 = o[d][3] * il;
    *(u32x2*)(orow + 16 * d + 4 * g) = u32x2{cvt2(v0, v1), cvt2(v2, v3)};
    if (a.ot) {
      bf16_t* dst = a.ot + (long)(h * DH + 16 * d + 4 * g) * a.ldot + row0 + myq;
      const uint32_t w01 = cvt2(v0, v1), w23 = cvt2(v2, v3);
      dst[0] = (bf16_t)(w01 & 0xffffu);
      dst[a.ldot] = (bf16_t)(w01 >> 16);
      dst[2 * a.ldot] = (bf16_t)(w23 & 0xffffu);
      dst[3 * a.ldot] = (bf16_t)(w23 >> 16);
    }
  }
  if (g == 0) {
    const float lse = (m + log2f(l)) * LN2;
    if (a.lse) a.lse[(row0 + myq) * a.HQ + h] = lse;
    a.lse_t[(long)h * a.ldt + row0 + myq] = lse;
  }
}
template <int NS>
__global__ __launch_bounds__(256) void k_attn2_fwd(TArgs a) {
  extern __shared__ __attribute__((aligned(16))) bf16_t lds[];  // NS x [K | V]
  attn2_fwd_body<NS, false>(a, lds);
}
template <int NS>
__global__ __launch_bounds__(256) void k_attn2_fwd_cached(TArgs a) {
  extern __shared__ __attribute__((aligned(16))) bf16_t lds[];  // NS x [K | V]
  attn2_fwd_body<NS, true>(a, lds);
}

// ------------------------------------------------------------- backward dQ
// Workgroup (query block qb, query head h, batch b): dQ of its 64 queries,
// with Delta read from delta_t (k_attn_delta).  lds: NS x [K | V].
// wl: this wave's 16-query slice (0..3) of the block; dma: whether this wave
// takes part in staging K | V (the grouped launch shares one copy among the
// query heads of a KV head)
// first key block a query of block qb sees (window: keys pos - W + 1 .. pos)
__host__ __device__ inline int dq_first_kb(int qb, int W) {
  return W > 0 && qb * QB - W + 1 > 0 ? (qb * QB - W + 1) / QB : 0;
}
// one past the last query block that sees a key of block kb
__host__ __device__ inline int dkv_end_qb(int kb, int T, int W) {
  int nqb = T / QB;
  if (W > 0 && (kb * QB + QB - 1 + W - 1) / QB + 1 < nqb) nqb = (kb * QB + QB - 1 + W - 1) / QB + 1;
  return nqb;
}

// dQ^T of query head h, query block qb, over key blocks klo .. khi (a whole
// walk is dq_first_kb(qb) .. qb): lane (j, g) of slice wl leaves dQ^T[16d +
// 4g + r][query 16 wl + j] in dq (before dS's 1/8).  dma: this wave issues
// the K | V stages (one group of waves stages them for all groups).
template <int NS>
__device__ __forceinline__ void attn2_dq_walk(const TArgs& a, bf16_t* lds, int qb, int h, int b, int wl, bool dma,
                                              int klo, int khi, f32x4 (&dq)[4]) {
  const int lane = threadIdx.x & 63, wave = wl;
  const int wave_s = __builtin_amdgcn_readfirstlane(wl);
  const int g = lane >> 4, j = lane & 15;
  const int T = a.T, NQ = a.HQ * DH;
  const int kvh = h / (a.HQ / a.HK);
  const int qloc = wave * 16 + j, myq = qb * QB + qloc;
  const long row0 = (long)b * T, qrow = row0 + myq;
  const float sc = 0.125f * LOG2E;

  // this lane's query: Q, dO (hi, lo) fragments
  bf16x8 qf[2], dhf[2], dlf[2];
#pragma unroll
  for (int c = 0; c < 2; c++) {
    const int col = h * DH + 32 * c + 8 * g;
    qf[c] = as_bf8(*(const u32x4*)(a.qkv + qrow * a.ldqkv + col));
    dhf[c] = as_bf8(*(const u32x4*)(a.dh + qrow * a.lddo + col));
    dlf[c] = as_bf8(*(const u32x4*)(a.dl + qrow * a.lddo + col));
  }
  const float delta = a.delta_t[(long)h * a.ldt + qrow];
  const float lse2 = a.lse_in_t[(long)h * a.ldt + qrow] * LOG2E;

  const bf16_t* ksrc = a.qkv + row0 * a.ldqkv + NQ + kvh * DH;
  const bf16_t* vsrc = ksrc + a.HK * DH;
  const uint32_t base = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)lds);
  auto issue = [&](int kb, int buf) {
    if (!dma) return;
    const uint32_t st = base + (uint32_t)(buf * 2 * TBYTES);
    dma_tile_all(ksrc + (long)kb * QB * a.ldqkv, a.ldqkv, st, wave_s, lane);
    dma_tile_all(vsrc + (long)kb * QB * a.ldqkv, a.ldqkv, st + TBYTES, wave_s, lane);
  };
#pragma unroll
  for (int d = 0; d < 4; d++) dq[d] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int W = a.window;
  const bool low_edge_possible = W > 0;
  wait_vm<0>();
#pragma unroll
  for (int s = 0; s < NS - 1; s++)
    if (klo + s <= khi) issue(klo + s, s);
  for (int kb = klo; kb <= khi; kb++) {
    const int it = kb - klo;
    wait_stages<4, NS - 2>(min(NS - 2, khi - kb));
    block_barrier();
    if (kb + NS - 1 <= khi) issue(kb + NS - 1, (it + NS - 1) % NS);
    const bf16_t* sK = lds + (it % NS) * 2 * TILE;
    const bf16_t* sV = sK + TILE;
    float ds[4][4];
#pragma unroll
    for (int sb = 0; sb < 4; sb++) {
      f32x4 st = f32x4{0.f, 0.f, 0.f, 0.f}, dp = f32x4{0.f, 0.f, 0.f, 0.f};
      const int kr = prow(sb, j);
#pragma unroll
      for (int c = 0; c < 2; c++) {
        st = mfma(tf(sK, kr, 4 * c + g), qf[c], st);
        const bf16x8 vf = tf(sV, kr, 4 * c + g);
        dp = mfma(vf, dhf[c], dp);
        dp = mfma(vf, dlf[c], dp);
      }
#pragma unroll
      for (int r = 0; r < 4; r++) ds[sb][r] = fexp2(fmaf(st[r], sc, -lse2)) * (dp[r] - delta);
    }
    // causal and window masks only on the key blocks that can hold masked
    // pairs (uniform); a masked pair's dS is 0 * (dP - Delta), as ds * 0
    // gives it (the 1/8 of dS = P (dP - Delta) / 8 is applied to dQ after
    // the loop: a power of two, so the planes and sums scale exactly)
    if (kb == qb || (low_edge_possible && kb * QB < qb * QB + QB - 1 - W + 1)) {
      asm volatile("");  // keeps the branch (not if-converted into selects on every block)
#pragma unroll
      for (int sb = 0; sb < 4; sb++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const int kk = 32 * (sb >> 1) + 8 * g + 4 * (sb & 1) + r;
          if ((kb == qb && kk > qloc) || (low_edge_possible && kb * QB + kk < myq - W + 1)) ds[sb][r] *= 0.f;
        }
    }
#pragma unroll
    for (int c = 0; c < 2; c++) {
      const float s8[8] = {ds[2 * c][0], ds[2 * c][1], ds[2 * c][2], ds[2 * c][3],
                           ds[2 * c + 1][0], ds[2 * c + 1][1], ds[2 * c + 1][2], ds[2 * c + 1][3]};
      bf16x8 sh, sl;
      split8p(s8, sh, sl);
#pragma unroll
      for (int d = 0; d < 4; d++) {
        const bf16x8 kt = tr_frag(sK, 32 * c, 16 * d, lane);  // K^T rows 16d.., keys 32c + 8g ..
        dq[d] = mfma(kt, sh, dq[d]);
        dq[d] = mfma(kt, sl, dq[d]);
      }
    }
  }
}

// dQ of query head h, query block qb from the walk's dQ^T (slice wl): dS's
// 1/8 (1/sqrt(head_dim), a power of two: exact), the inverse RoPE on the
// pairs (r, r^1), then hi / lo planes, normal (4 consecutive columns) and
// transposed
__device__ __forceinline__ void attn2_dq_store(const TArgs& a, int qb, int h, int b, int wl, f32x4 (&dq)[4]) {
  const int lane = threadIdx.x & 63, g = lane >> 4, j = lane & 15;
  const int myq = qb * QB + wl * 16 + j;
  const long qrow = (long)b * a.T + myq;
#pragma unroll
  for (int d = 0; d < 4; d++) dq[d] *= 0.125f;
#pragma unroll
  for (int d = 0; d < 4; d++) {
    float v[4] = {dq[d][0], dq[d][1], dq[d][2], dq[d][3]};
    if (a.rope) {
#pragma unroll
      for (int pr = 0; pr < 2; pr++) {
        const int col = 16 * d + 4 * g + 2 * pr;
        const float2 c = *(const float2*)(a.rope + 2 * ((long)myq * (DH / 2) + (col >> 1)));
        const float x = v[2 * pr], y = v[2 * pr + 1];
        v[2 * pr] = x * c.x + y * c.y;
        v[2 * pr + 1] = y * c.x - x * c.y;
      }
    }
    const uint32_t h01 = cvt2(v[0], v[1]), h23 = cvt2(v[2], v[3]);
    const uint32_t l01 = cvt2(v[0] - bflo(h01), v[1] - bfhi(h01)), l23 = cvt2(v[2] - bflo(h23), v[3] - bfhi(h23));
    const long col = h * DH + 16 * d + 4 * g;
    *(u32x2*)(a.gq[0] + qrow * a.ldg + col) = u32x2{h01, h23};
    *(u32x2*)(a.gq[1] + qrow * a.ldg + col) = u32x2{l01, l23};
    const uint32_t hs[4] = {h01 & 0xffffu, h01 >> 16, h23 & 0xffffu, h23 >> 16};
    const uint32_t ls[4] = {l01 & 0xffffu, l01 >> 16, l23 & 0xffffu, l23 >> 16};
    if (a.gqt[0]) {  // transposed planes (optional)
#pragma unroll
      for (int r = 0; r < 4; r++) {
        a.gqt[0][(col + r) * a.ldgt + qrow] = (bf16_t)hs[r];
        a.gqt[1][(col + r) * a.ldgt + qrow] = (bf16_t)ls[r];
      }
    }
  }
}

// dQ of query head h, query block qb: the whole walk, then the planes
template <int NS>
__device__ __forceinline__ void attn2_dq(const TArgs& a, bf16_t* lds, int qb, int h, int b, int wl, bool dma) {
  f32x4 dq[4];
  attn2_dq_walk<NS>(a, lds, qb, h, b, wl, dma, dq_first_kb(qb, a.window), qb, dq);
  attn2_dq_store(a, qb, h, b, wl, dq);
}

// ------------------------------------------------------------ backward dKV
// A stage holds the query block's Q and dO planes in row orientation only:
// the products that need them transposed (dV^T = dO^T P, dK^T = Q^T dS) read
// their fragments with LDS transpose reads.
constexpr int SROW = 3 * TILE + 512;  // dK/dV stage size in bf16 elements (+1 KB of LSE / Delta)

// The dK / dV accumulation of head h over query blocks qlo .. qhi (a whole
// walk is kb .. dkv_end_qb(kb) - 1) for the 16 keys of slice wl (0..3) of
// key block kb; lds: NST x [Q | dOh | dOl | LSE,Delta] of this head.  Leaves
// dK^T / dV^T [16d + 4g + r][key] in dk / dv.
__device__ __forceinline__ void attn2_dkv_core(const TArgs& a, bf16_t* lds, int kb, int h, int b, int wl, int qlo,
                                               int qhi, f32x4 (&dk)[4], f32x4 (&dv)[4]) {
  const int lane = threadIdx.x & 63, wave = wl;
  const int wave_s = __builtin_amdgcn_readfirstlane(wl);
  const int g = lane >> 4, j = lane & 15;
  const int T = a.T, NQ = a.HQ * DH, NK = a.HK * DH;
  const int group = a.HQ / a.HK;
  const int kvh = h / group, gi = h % group;
  const int kloc = wave * 16 + j;
  const long row0 = (long)b * T, krow = row0 + kb * QB + kloc;
  const float sc = 0.125f * LOG2E;

  bf16x8 kf[2], vf[2];
#pragma unroll
  for (int c = 0; c < 2; c++) {
    kf[c] = as_bf8(*(const u32x4*)(a.qkv + krow * a.ldqkv + NQ + kvh * DH + 32 * c + 8 * g));
    vf[c] = as_bf8(*(const u32x4*)(a.qkv + krow * a.ldqkv + NQ + NK + kvh * DH + 32 * c + 8 * g));
  }
  const bf16_t* qsrc = a.qkv + row0 * a.ldqkv + h * DH;
  const bf16_t* dhsrc = a.dh + row0 * a.lddo + h * DH;
  const bf16_t* dlsrc = a.dl + row0 * a.lddo + h * DH;
  const float* lsesrc = a.lse_in_t + (long)h * a.ldt + row0;
  const float* dlsrc2 = a.delta_t + (long)h * a.ldt + row0;
  const uint32_t base = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)lds);
  auto issue = [&](int qb, int buf) {
    const uint32_t st = base + (uint32_t)(buf * SROW * 2);
    const long q0 = (long)qb * QB;
    dma_tile_all(qsrc + q0 * a.ldqkv, a.ldqkv, st, wave_s, lane);
    dma_tile_all(dhsrc + q0 * a.lddo, a.lddo, st + TBYTES, wave_s, lane);
    dma_tile_all(dlsrc + q0 * a.lddo, a.lddo, st + 2 * TBYTES, wave_s, lane);
    if (wave_s == 0) {  // LSE (lanes 0-15) and Delta (16-31) of the block's 64 queries
      const void* s = lane < 16 ? (const void*)(lsesrc + q0 + 4 * lane)
                                : lane < 32 ? (const void*)(dlsrc2 + q0 + 4 * (lane - 16)) : (const void*)g_zero_t;
      dma16(s, st + 3 * TBYTES);
    }
  };
#pragma unroll
  for (int d = 0; d < 4; d++) dk[d] = dv[d] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int W = a.window;
  const int nqb = qhi + 1;
  // no wait for the fragment loads above: vector memory operations count
  // down in issue order, so the first stage's wait covers them too
#pragma unroll
  for (int s = 0; s < NST - 1; s++)
    if (qlo + s < nqb) issue(qlo + s, s);
  for (int qb = qlo; qb < nqb; qb++) {
    const int it = qb - qlo;
    if (qb + 1 < nqb) {
      // a stage is 6 DMA instructions per wave (7 on wave 0): leave the
      // NST - 2 later stages in flight
      if (wave_s == 0) wait_vm<(NST - 2) * 7>(); else wait_vm<(NST - 2) * 6>();
    } else {
      wait_vm<0>();
    }
    block_barrier();
    if (qb + NST - 1 < nqb) issue(qb + NST - 1, (it + NST - 1) % NST);
    const bf16_t* sQ = lds + (it % NST) * SROW;
    const bf16_t* sDh = sQ + TILE;
    const bf16_t* sDl = sQ + 2 * TILE;
    const float* sL = (const float*)(sQ + 3 * TILE);
    const float* sD = sL + 64;
    float pp[4][4], ds[4][4];
#pragma unroll
    for (int sb = 0; sb < 4; sb++) {
      f32x4 st = f32x4{0.f, 0.f, 0.f, 0.f}, dp = f32x4{0.f, 0.f, 0.f, 0.f};
      const int qr = prow(sb, j);
#pragma unroll
      for (int c = 0; c < 2; c++) {
        st = mfma(tf(sQ, qr, 4 * c + g), kf[c], st);
        dp = mfma(tf(sDh, qr, 4 * c + g), vf[c], dp);
        dp = mfma(tf(sDl, qr, 4 * c + g), vf[c], dp);
      }
      const int q4 = 32 * (sb >> 1) + 8 * g + 4 * (sb & 1);  // this lane's 4 queries: q4 .. q4+3
      const float4 l4 = *(const float4*)(sL + q4);
      const float4 d4 = *(const float4*)(sD + q4);
      const float lv[4] = {l4.x, l4.y, l4.z, l4.w}, dv4[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const float p = fexp2(fmaf(st[r], sc, -lv[r] * LOG2E));
        pp[sb][r] = p;
        ds[sb][r] = p * (dp[r] - dv4[r]);  // the 1/8 is applied to dK after the loop
      }
    }
    // causal and window masks, only on the blocks that have masked pairs
    // (uniform): a masked pair gets p = 0 and dS = 0 * (dP - Delta) / 8 (the
    // sign of that zero follows dP - Delta, as ds * 0 keeps it)
    if (qb == kb || (W > 0 && qb * QB + QB - 1 > kb * QB + W - 1)) {
      asm volatile("");  // keeps the branch (not if-converted into selects on every block)
#pragma unroll
      for (int sb = 0; sb < 4; sb++) {
        const int q4 = 32 * (sb >> 1) + 8 * g + 4 * (sb & 1);
#pragma unroll
        for (int r = 0; r < 4; r++)
          if ((qb == kb && q4 + r < kloc) || (W > 0 && qb * QB + q4 + r > kb * QB + kloc + W - 1)) {
            pp[sb][r] = 0.f;
            ds[sb][r] *= 0.f;
          }
      }
    }
#pragma unroll
    for (int c = 0; c < 2; c++) {
      const float p8[8] = {pp[2 * c][0], pp[2 * c][1], pp[2 * c][2], pp[2 * c][3],
                           pp[2 * c + 1][0], pp[2 * c + 1][1], pp[2 * c + 1][2], pp[2 * c + 1][3]};
      const float s8[8] = {ds[2 * c][0], ds[2 * c][1], ds[2 * c][2], ds[2 * c][3],
                           ds[2 * c + 1][0], ds[2 * c + 1][1], ds[2 * c + 1][2], ds[2 * c + 1][3]};
      bf16x8 ph, pl, sh, sl;
      split8p(p8, ph, pl);
      split8p(s8, sh, sl);
#pragma unroll
      for (int d = 0; d < 4; d++) {
        const bf16x8 doh = tr_frag(sDh, 32 * c, 16 * d, lane), dol = tr_frag(sDl, 32 * c, 16 * d, lane);
        const bf16x8 qt = tr_frag(sQ, 32 * c, 16 * d, lane);
        dv[d] = mfma(doh, ph, dv[d]);
        dv[d] = mfma(dol, ph, dv[d]);
        dv[d] = mfma(doh, pl, dv[d]);
        dk[d] = mfma(qt, sh, dk[d]);
        dk[d] = mfma(qt, sl, dk[d]);
      }
    }
  }
#pragma unroll
  for (int d = 0; d < 4; d++) dk[d] *= 0.125f;  // dS's 1/8 (1/sqrt(head_dim)): a power of two, exact
}

// Workgroup (key block, query head, batch): this head's dK | dV share, fp32,
// into part[gi][row][dK | dV] (gi = head index inside its group).
__device__ __forceinline__ void attn2_dkv(const TArgs& a, bf16_t* lds, int kb, int h, int b) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, g = lane >> 4, j = lane & 15;
  f32x4 dk[4], dv[4];
  attn2_dkv_core(a, lds, kb, h, b, wave, kb, dkv_end_qb(kb, a.T, a.window) - 1, dk, dv);
  const int T = a.T, NK = a.HK * DH;
  const int group = a.HQ / a.HK;
  const int kvh = h / group, gi = h % group;
  const long krow = (long)b * T + kb * QB + wave * 16 + j;
  // lane holds dK^T / dV^T [16d + 4g + r][key]: 4 consecutive columns of the partial row
  if (group == 1 && !a.gqt[0]) {
    // one query head per KV head, row planes only: the head's share is the
    // whole gradient, so it goes straight to the dK | dV planes (dK rotated
    // back by the inverse RoPE, as the group reduce does) and no partials
    // or reduce pass follow
    const int pos = kb * QB + wave * 16 + j, NQ = a.HQ * DH;
#pragma unroll
    for (int d = 0; d < 4; d++) {
#pragma unroll
      for (int hf = 0; hf < 2; hf++) {
        float v[4] = {hf ? dv[d][0] : dk[d][0], hf ? dv[d][1] : dk[d][1], hf ? dv[d][2] : dk[d][2],
                      hf ? dv[d][3] : dk[d][3]};
        if (hf == 0 && a.rope) {
#pragma unroll
          for (int pr = 0; pr < 2; pr++) {
            const float2 c = *(const float2*)(a.rope + 2 * ((long)pos * (DH / 2) + ((16 * d + 4 * g + 2 * pr) >> 1)));
            const float x = v[2 * pr], y = v[2 * pr + 1];
            v[2 * pr] = x * c.x + y * c.y;
            v[2 * pr + 1] = y * c.x - x * c.y;
          }
        }
        bf16_t hv[4], lv[4];
#pragma unroll
        for (int r = 0; r < 4; r++) split_bf(v[r], hv[r], lv[r]);
        const long col = NQ + hf * NK + kvh * DH + 16 * d + 4 * g;
        *(u32x2*)(a.gq[0] + krow * a.ldg + col) = u32x2{pack2(hv[0], hv[1]), pack2(hv[2], hv[3])};
        *(u32x2*)(a.gq[1] + krow * a.ldg + col) = u32x2{pack2(lv[0], lv[1]), pack2(lv[2], lv[3])};
      }
    }
    return;
  }
  const long M = (long)T * a.B;
  float* prow_ = a.part + ((long)gi * M + krow) * 2 * NK + kvh * DH;
#pragma unroll
  for (int d = 0; d < 4; d++) {
    *(float4*)(prow_ + 16 * d + 4 * g) = make_float4(dk[d][0], dk[d][1], dk[d][2], dk[d][3]);
    *(float4*)(prow_ + NK + 16 * d + 4 * g) = make_float4(dv[d][0], dv[d][1], dv[d][2], dv[d][3]);
  }
}

// Delta = sum over the head's 64 columns of dO * O (dO = hi + lo), per
// (row, query head) into delta_t [HQ][ldt] (hierarchy.py:42-70 computes it
// in the dQ kernel; here it comes first so dQ and dK/dV are independent).
// Four lanes per (row, head), 16 columns each, summed (l0 + l1) + (l2 + l3).
__global__ __launch_bounds__(256) void k_attn_delta(TArgs a) {
  const long t = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const long M = (long)a.T * a.B;
  const int g = (int)(t & 3);
  const long rh = t >> 2;
  const bool ok = rh < M * a.HQ;
  const long row = ok ? rh / a.HQ : 0;
  const int h = ok ? (int)(rh % a.HQ) : 0;
  float dpart = 0.f;
  if (ok) {
#pragma unroll
    for (int c = 0; c < 2; c++) {
      const int col = h * DH + 32 * c + 8 * g;
      const u32x4 hv = *(const u32x4*)(a.dh + row * a.lddo + col);
      const u32x4 lv = *(const u32x4*)(a.dl + row * a.lddo + col);
      const u32x4 ov = *(const u32x4*)(a.ob + row * a.ldo + col);
#pragma unroll
      for (int i = 0; i < 4; i++) {
        dpart += (bflo(hv[i]) + bflo(lv[i])) * bflo(ov[i]);
        dpart += (bfhi(hv[i]) + bfhi(lv[i])) * bfhi(ov[i]);
      }
    }
  }
  dpart += __shfl_xor(dpart, 1, 64);
  dpart += __shfl_xor(dpart, 2, 64);
  if (ok && g == 0) a.delta_t[(long)h * a.ldt + row] = dpart;
}

// dQ and dK/dV in one launch (they share only Delta): grid.x = 2 T/64;
// rank r of role 0 is the dQ of query block T/64 - 1 - r, of role 1 the
// dK/dV of key block r (both longest first).  Both roles keep several
// latency-bound workgroups per CU busy.
__global__ __launch_bounds__(256) SJ_BWD_OCC void k_attn2_bwd(TArgs a) {
  extern __shared__ __attribute__((aligned(16))) bf16_t lds[];
  const int nb = (int)(gridDim.x >> 1);
  const WgMap wm = wg_map(2);
  if (wm.role == 0)
    attn2_dq<NS_DQ>(a, lds, nb - 1 - wm.r, wm.h, wm.b, threadIdx.x >> 6, true);
  else
    attn2_dkv(a, lds, wm.r, wm.h, wm.b);
}

// The same roles as separate launches: with thousands of workgroups per role
// (cfg5: 4096) each kernel fills the chip alone, and the dQ role keeps its
// smaller LDS and register footprint (more workgroups per CU).
__global__ __launch_bounds__(256) void k_attn2_bwd_dq(TArgs a) {
  extern __shared__ __attribute__((aligned(16))) bf16_t lds[];
  const WgMap wm = wg_map(1);
  attn2_dq<NS_DQ>(a, lds, (int)gridDim.x - 1 - wm.r, wm.h, wm.b, threadIdx.x >> 6, true);
}
__global__ __launch_bounds__(256) SJ_BWD_OCC void k_attn2_bwd_dkv(TArgs a) {
  extern __shared__ __attribute__((aligned(16))) bf16_t lds[];
  const WgMap wm = wg_map(1);
  attn2_dkv(a, lds, wm.r, wm.h, wm.b);
}

constexpr int GROUPED_G = 3;  // query heads per KV head of the grouped launch
constexpr size_t LDS_BWD_G = (size_t)GROUPED_G * NST * SROW * 2 > (size_t)NS_DQ * 2 * TBYTES
                                 ? (size_t)GROUPED_G * NST * SROW * 2
                                 : (size_t)NS_DQ * 2 * TBYTES;
static_assert(LDS_BWD_G + 16 <= 160 * 1024 && (size_t)(GROUPED_G - 1) * 8 * 256 * 16 <= LDS_BWD_G,
              "grouped LDS budget (+ the meeting's count)");


// ------------------------------------------ grouped backward (no partials)
// Both roles per KV head instead of per query head: a workgroup of G x 4
// waves holds the G query heads of KV head kvh (group gi of four waves:
// query head kvh * G + gi).  A dQ walk (query block qb): each group forms
// its head's dQ from K | V stages that group 0 alone stages for all G.  A
// dK | dV walk (key block kb): each group accumulates its head's share over
// its own Q / dO stages; the groups then add their shares through LDS in
// head order, ((0 + h0) + h1) + h2 as the group reduce sums the fp32
// partials (group 0 for dK, which it rotates back by the inverse RoPE,
// group 1 for dV, side by side), and each writes its hi / lo planes.  No
// per-head partials leave the workgroup and no reduce pass follows.  G x NST
// stages of dK/dV operands: G <= 3 fits the LDS.
//
// Balanced pieces.  The causal walks are 1 .. nb blocks long (dQ of query
// block qb: qb + 1 key blocks; dK | dV of key block kb: nb - kb query
// blocks), so with one workgroup per walk a launch that fills the chip once
// lasts as long as its longest walk, about twice the mean.  The host cuts
// each role's walks longer than a cap into parts of at most the cap (up to
// PLAN_PARTS; SplitPlan: a piece is a whole walk or a part, one workgroup
// each, dispatched costliest first as CUs free up) with the caps that finish
// a simulated dispatch first.  Each part of a cut walk writes its fp32 sum
// (the groups' dQ^T, or the dK | dV after the head sum) to its slot of the
// workspace and counts itself on the walk's counter; the part that counts
// last adds the parts' sums in part order (its own from registers: the same
// bits whichever part comes last), writes the planes and sets the counter
// back to zero for the next launch.  The counters are the caller's: a
// region of its workspace (PLAN_CUTS words per (KV head, sequence)) that is
// zero before the first launch and that every launch leaves zero, so
// launches on different workspaces (two models, a graph replay beside an
// eager call) never count on each other's counters.  (One piece per workgroup: a workgroup
// that ran several pieces in a loop held their addresses and arguments
// across the loop and ran every walk slower.)
constexpr int PLAN_PIECES = 128;  // pieces of both roles
constexpr int PLAN_CUTS = 64;     // cut walks per (KV head, sequence)
constexpr int PLAN_PARTS = 4;     // parts of a cut walk
// piece: bit 31 set, bits 0-5 block, 6-11 / 12-17 the first / last block of
// the walk it covers, bit 18 the role (0: dQ, 1: dK | dV), 19-26 cut-walk
// index + 1 (0: a whole walk), 27-28 the part, 29-30 the walk's parts - 1
struct SplitPlan {
  int ncut;    // cut walks per (KV head, sequence)
  int nslots;  // part sums per (KV head, sequence)
  uint16_t slot0[PLAN_CUTS];  // first part-sum slot of each cut walk
  uint32_t seg[PLAN_PIECES];
};

// A part's sum passes between workgroups (on different XCDs, each with its
// own L2) through device-scope accesses, relaxed atomics at agent scope:
// loads and stores coherent across the L2s by themselves, so the meeting
// needs no device-scope fence (whose L2 write-back and invalidate cover the
// whole L2 of the XCD: microseconds, and a cold L2 for the kernels beside).
// Element r of a thread's vector sits at p[r * stride]: with p the thread's
// index and stride the thread count, each store or load instruction of a
// wave covers 256 consecutive bytes (whole cache lines, one request each).
__device__ __forceinline__ void put4(float* p, long stride, f32x4 v) {
#pragma unroll
  for (int r = 0; r < 4; r++) __hip_atomic_store(p + r * stride, v[r], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ f32x4 get4(const float* p, long stride) {
  f32x4 v;
#pragma unroll
  for (int r = 0; r < 4; r++) v[r] = __hip_atomic_load(p + r * stride, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return v;
}

// The parts of a cut walk meet (every thread of the workgroup calls it,
// after put4 of its share of this part's sum): true in the workgroup that
// counts last, which may then get4 the other parts' sums, and which sets
// the counter back to zero.  The stores have completed (vmcnt 0) before the
// barrier that precedes the count, and the other parts' loads follow the
// barrier that hands the count out.
__device__ __forceinline__ bool meet_last(uint32_t* cnt, uint32_t* flag, int nparts) {
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  block_barrier();
  if (threadIdx.x == 0) *flag = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  block_barrier();
  const uint32_t n = __builtin_amdgcn_readfirstlane(*flag);  // the barrier's memory clobber: read after it
  if (n != (uint32_t)(nparts - 1)) return false;
  if (threadIdx.x == 0) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return true;
}

// where the sums of cut walk `cut` of (sequence b, KV head kvh) meet: the
// walk's first slot (part p at base + p * slot floats), this part, the
// walk's parts, its counter
struct Meet {
  float* base;
  int part, nparts;
  uint32_t* cnt;
};
__device__ __forceinline__ Meet meet_at(const TArgs& a, const SplitPlan& pl, int b, int kvh, uint32_t sg, long slot) {
  const int cut = (int)((sg >> 19) & 255) - 1, part = (int)((sg >> 27) & 3), nparts = (int)((sg >> 29) & 3) + 1;
  const long pair = (long)b * a.HK + kvh;
  float* base = a.part + (pair * pl.nslots + pl.slot0[cut]) * slot;
  return Meet{base, part, nparts, a.cnt + pair * PLAN_CUTS + cut};
}
// the walk's total of vector v (element r at off + r * stride of each
// part's slot), parts in order: ((s0 + s1) + s2) + s3, this part's own from
// registers
__device__ __forceinline__ f32x4 parts_total(const Meet& m, long slot, long off, long stride, f32x4 own) {
  f32x4 t = m.part == 0 ? own : get4(m.base + off, stride);
#pragma unroll
  for (int p = 1; p < PLAN_PARTS; p++)
    if (p < m.nparts) t = t + (p == m.part ? own : get4(m.base + p * slot + off, stride));
  return t;
}

// One piece: a whole walk, or a part of a cut walk, of one role.
template <int G, bool DQ>
__device__ __forceinline__ void grouped_piece(const TArgs& a, const SplitPlan& pl, bf16_t* lds, uint32_t sg, int kvh,
                                              int b) {
  constexpr int NT = 256 * G;  // threads
  constexpr long SLOT = 16 * NT;  // floats of one part's sum (dQ^T: 16 per thread; dK | dV: 32 per group-0 thread)
  static_assert(32 * 256 <= SLOT, "slot size");
  uint32_t* s_count = (uint32_t*)((char*)lds + LDS_BWD_G);  // the meeting's count, past the stages
  {
    const int tid = (int)threadIdx.x;
    const int w = tid >> 6, gi = __builtin_amdgcn_readfirstlane(w >> 2), wl = w & 3;
    const int lane = tid & 63, g = lane >> 4, j = lane & 15;
    const int h = kvh * G + gi;
    const int blk = (int)(sg & 63), lo = (int)((sg >> 6) & 63), hi = (int)((sg >> 12) & 63);
    const bool cut = ((sg >> 19) & 255) != 0;
    if constexpr (DQ) {
      f32x4 dq[4];
      attn2_dq_walk<NS_DQ>(a, lds, blk, h, b, wl, gi == 0, lo, hi, dq);
      if (cut) {
        const Meet m = meet_at(a, pl, b, kvh, sg, SLOT);
#pragma unroll
        for (int d = 0; d < 4; d++) put4(m.base + m.part * SLOT + 4 * d * NT + tid, NT, dq[d]);
        if (!meet_last(m.cnt, s_count, m.nparts)) return;
#pragma unroll
        for (int d = 0; d < 4; d++) dq[d] = parts_total(m, SLOT, 4 * d * NT + tid, NT, dq[d]);
      }
      attn2_dq_store(a, blk, h, b, wl, dq);
    } else {
      const int kb = blk;
      f32x4 dk[4], dv[4];
      attn2_dkv_core(a, lds + gi * NST * SROW, kb, h, b, wl, lo, hi, dk, dv);
      const int pos = kb * QB + wl * 16 + j;
      float2 cs[8];  // group 0: the inverse-RoPE (cos, sin) of dK columns 16d + 4g + 2pr, +1 (loaded before the exchange)
#pragma unroll
      for (int i = 0; i < 8; i++)
        cs[i] = gi == 0 && a.rope
                    ? *(const float2*)(a.rope + 2 * ((long)pos * (DH / 2) + ((16 * (i >> 1) + 4 * g + 2 * (i & 1)) >> 1)))
                    : float2{0.f, 0.f};
      block_barrier();  // every group is done reading its stages
      // dK is summed and stored by group 0, dV by group 1, side by side:
      // group q leaves vector d of half hf (0 dK, 1 dV) that it does not own
      // for lane L of slice wl at f32x4 index ((hf * G + q) * 4 + d) * 256 +
      // wl * 64 + L; the owner adds the heads in head order, ((0 + h0) + h1)
      // + h2 as the group reduce sums the fp32 partials
      static_assert(G >= 2 && (size_t)2 * G * 4 * 256 * 16 <= LDS_BWD_G, "grouped exchange");
      f32x4* sh = (f32x4*)lds;
      const int slot = wl * 64 + lane;
#pragma unroll
      for (int d = 0; d < 4; d++) {
        if (gi != 0) sh[((0 * G + gi) * 4 + d) * 256 + slot] = dk[d];
        if (gi != 1) sh[((1 * G + gi) * 4 + d) * 256 + slot] = dv[d];
      }
      block_barrier();
      const int hf = gi;  // the half this group owns (groups 0 and 1)
      f32x4 acc[4];
      if (hf < 2) {
#pragma unroll
        for (int d = 0; d < 4; d++) {
#pragma unroll
          for (int r = 0; r < 4; r++) {
            float s = 0.f;
#pragma unroll
            for (int q = 0; q < G; q++) s += q == gi ? (hf ? dv[d][r] : dk[d][r]) : sh[((hf * G + q) * 4 + d) * 256 + slot][r];
            acc[d][r] = s;
          }
        }
      }
      if (cut) {
        const Meet m = meet_at(a, pl, b, kvh, sg, SLOT);
        if (hf < 2) {
#pragma unroll
          for (int d = 0; d < 4; d++) put4(m.base + m.part * SLOT + 4 * (4 * hf + d) * 256 + slot, 256, acc[d]);
        }
        if (!meet_last(m.cnt, s_count, m.nparts)) return;
        if (hf < 2) {
#pragma unroll
          for (int d = 0; d < 4; d++) acc[d] = parts_total(m, SLOT, 4 * (4 * hf + d) * 256 + slot, 256, acc[d]);
        }
      }
      if (hf >= 2) return;
      const int T = a.T, NQ = a.HQ * DH, NK = a.HK * DH;
      const long krow = (long)b * T + pos;
#pragma unroll
      for (int d = 0; d < 4; d++) {
        float v[4] = {acc[d][0], acc[d][1], acc[d][2], acc[d][3]};
        if (hf == 0 && a.rope) {  // inverse RoPE on dK's pairs (columns 16d + 4g + 2pr, +1)
#pragma unroll
          for (int pr = 0; pr < 2; pr++) {
            const float2 c = cs[2 * d + pr];
            const float x = v[2 * pr], y = v[2 * pr + 1];
            v[2 * pr] = x * c.x + y * c.y;
            v[2 * pr + 1] = y * c.x - x * c.y;
          }
        }
        bf16_t hv[4], lv[4];
#pragma unroll
        for (int r = 0; r < 4; r++) split_bf(v[r], hv[r], lv[r]);
        const long col = NQ + hf * NK + kvh * DH + 16 * d + 4 * g;
        *(u32x2*)(a.gq[0] + krow * a.ldg + col) = u32x2{pack2(hv[0], hv[1]), pack2(hv[2], hv[3])};
        *(u32x2*)(a.gq[1] + krow * a.ldg + col) = u32x2{pack2(lv[0], lv[1]), pack2(lv[2], lv[3])};
      }
    }
  }
}

template <int G>
__global__ __launch_bounds__(256 * G) SJ_BWD_OCC void k_attn2_bwd_g(TArgs a, SplitPlan pl) {
  extern __shared__ __attribute__((aligned(16))) bf16_t lds[];
  const WgMap wm = wg_map(1);
  const uint32_t sg = pl.seg[wm.r];
  if (!((sg >> 18) & 1))
    grouped_piece<G, true>(a, pl, lds, sg, wm.h, wm.b);
  else
    grouped_piece<G, false>(a, pl, lds, sg, wm.h, wm.b);
}

constexpr long SEPARATE_ROLES = 2048;  // workgroups per role from which the roles launch separately

constexpr size_t LDS_FWD = (size_t)NS_FWD * 2 * TBYTES;
constexpr size_t LDS_DQ = (size_t)NS_DQ * 2 * TBYTES;
static_assert(NS_FWD >= 2 && NS_DQ >= 2 && LDS_FWD <= 160 * 1024 && LDS_DQ <= 160 * 1024, "LDS budget");
static_assert((NS_FWD - 2) * 4 < 64 && (NS_DQ - 2) * 4 < 64 && NST >= 2 && (NST - 2) * 7 < 64, "vmcnt range");
constexpr size_t LDS_DKV = (size_t)NST * (3 * TBYTES + 1024);
constexpr size_t LDS_BWD = LDS_DQ > LDS_DKV ? LDS_DQ : LDS_DKV;
static_assert(LDS_BWD <= 160 * 1024, "LDS budget");
static_assert(LDS_DKV <= 160 * 1024, "LDS budget");

}  // namespace

// SJ_ATTN_GROUPED=0 keeps the per-query-head launch with the group reduce
// (A/B comparisons)
static bool grouped_on() {
  static int on = -1;
  if (on < 0) {
    const char* e = getenv("SJ_ATTN_GROUPED");
    on = e ? atoi(e) != 0 : 1;
  }
  return on != 0;
}

bool sjh::attention_bwd_grouped(long batch, long t, long hq, long hk, bool transposed) {
  return hq == GROUPED_G * hk && !transposed && (t / QB) * hq * batch < SEPARATE_ROLES && 4 * (t / QB) <= PLAN_PIECES &&
         grouped_on();
}

// ----------------------------------------------- pieces of the grouped backward
namespace {
struct Walk {  // one role's walk for block `block`: blocks first .. last of the other operand
  int block, first, last;
  int len() const { return last - first + 1; }
};
struct Piece {
  int block, first, last, role, cut, part, nparts;  // cut -1: a whole walk
  double cost;
};

// cost of a piece, microseconds per workgroup at the cfg2 shape on MI355X
// (stamped workgroup start and end times): a dQ walk 5.0 + 1.85 per key
// block, a dK | dV walk 6.6 + 2.9 per query block, a cut part's meeting 5
// more (its sum written, counted and read at device scope)
constexpr double DQ_START = 5.0, DQ_STEP = 1.85, KV_START = 6.6, KV_STEP = 2.9, PIECE_MEET = 5.0;

// the walks of both roles for nb blocks and window W (0: causal), with the
// bounds the kernels' whole walks use
void role_walks(int nb, int W, std::vector<Walk>& wq, std::vector<Walk>& wk) {
  for (int i = 0; i < nb; i++) {
    wq.push_back(Walk{i, dq_first_kb(i, W), i});
    wk.push_back(Walk{i, i, dkv_end_qb(i, nb * QB, W) - 1});
  }
}

// a role's walks as pieces: one longer than cap is cut into parts of cap
// blocks and a last part of the rest (cut indices from *ncut on, part-sum
// slots counted in *nslots); false if a walk needs more than PLAN_PARTS
bool cut_walks(const std::vector<Walk>& ws, int role, int cap, std::vector<Piece>& out, int* ncut, int* nslots) {
  const double start = role == 0 ? DQ_START : KV_START, step = role == 0 ? DQ_STEP : KV_STEP;
  for (const Walk& w : ws) {
    if (w.len() > cap) {
      const int np = (w.len() + cap - 1) / cap;
      if (np > PLAN_PARTS) return false;
      const int c = (*ncut)++;
      *nslots += np;
      for (int q = 0; q < np; q++) {
        const int f = w.first + q * cap, l = std::min(w.last, f + cap - 1);
        out.push_back(Piece{w.block, f, l, role, c, q, np, start + (l - f + 1) * step + PIECE_MEET});
      }
    } else {
      out.push_back(Piece{w.block, w.first, w.last, role, -1, 0, 1, start + w.len() * step});
    }
  }
  return true;
}

// finish time of `pairs` copies of the pieces (costliest first, each copy
// of a piece before the next piece: the launch's dispatch order) taken in
// turn by the CU free first
double simulate(std::vector<Piece>& ps, long pairs, int cus) {
  std::stable_sort(ps.begin(), ps.end(), [](const Piece& x, const Piece& y) { return x.cost > y.cost; });
  std::vector<double> cu((size_t)cus, 0.0);  // min-heap of free times
  double end = 0;
  for (const Piece& p : ps)
    for (long i = 0; i < pairs; i++) {
      std::pop_heap(cu.begin(), cu.end(), std::greater<double>());
      cu.back() += p.cost;
      end = std::max(end, cu.back());
      std::push_heap(cu.begin(), cu.end(), std::greater<double>());
    }
  return end;
}

// The pieces of the launch: over every pair of caps (dQ, dK | dV), the one
// whose simulated dispatch finishes first (ties: the longer caps, fewer
// cuts), with at most 2 nb part sums per (KV head, sequence) -- they fit
// the workspace of the per-head partials --, PLAN_PIECES pieces,
// PLAN_CUTS cut walks per (KV head, sequence).
// cut = false: one piece per walk (the former launch).  caps_q / caps_k > 0
// fix the caps.
double plan_pieces(int nb, int W, long pairs, int cus, bool cut, int caps_q, int caps_k, std::vector<Piece>& best,
                   int& ncut, int& nslots) {
  std::vector<Walk> wq, wk;
  role_walks(nb, W, wq, wk);
  int maxq = 0, maxk = 0;
  for (const Walk& w : wq) maxq = std::max(maxq, w.len());
  for (const Walk& w : wk) maxk = std::max(maxk, w.len());
  double best_t = -1;
  for (int cq = maxq; cq >= 1; cq--)
    for (int ck = maxk; ck >= 1; ck--) {
      if (!cut && (cq != maxq || ck != maxk)) continue;
      if (caps_q > 0 && cq != std::min(caps_q, maxq)) continue;
      if (caps_k > 0 && ck != std::min(caps_k, maxk)) continue;
      std::vector<Piece> ps;
      int nc = 0, ns = 0;
      if (!cut_walks(wq, 0, cq, ps, &nc, &ns) || !cut_walks(wk, 1, ck, ps, &nc, &ns)) continue;
      if (ns > 2 * nb || nc > PLAN_CUTS || (int)ps.size() > PLAN_PIECES) continue;
      const double t = simulate(ps, pairs, cus);
      if (best_t < 0 || t < best_t - 1e-9) {
        best_t = t;
        best = ps;
        ncut = nc;
        nslots = ns;
      }
    }
  if (best_t < 0) return plan_pieces(nb, W, pairs, cus, false, 0, 0, best, ncut, nslots);
  return best_t;
}

int env_int(const char* name, int dflt) {
  const char* e = getenv(name);
  return e ? atoi(e) : dflt;
}

int device_cus() {
  static int n = 0;
  if (!n) {
    int dev = 0, cu = 0;
    n = hipGetDevice(&dev) == hipSuccess &&
                hipDeviceGetAttribute(&cu, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && cu > 0
            ? cu
            : 256;
  }
  return n;
}

// The launch's plan for `pairs` (KV head, sequence) pairs on `cus` CUs,
// searched once per shape (the search simulates every pair of caps) and
// kept.  SJ_ATTN_CUT=0: one piece
// per walk (A/B comparisons); SJ_ATTN_CAPS_Q / SJ_ATTN_CAPS_K fix the caps.
int make_plan(long t, long window, long pairs, int cus, SplitPlan& pl, int& npieces) {
  static const int cut_on = env_int("SJ_ATTN_CUT", 1), cq = env_int("SJ_ATTN_CAPS_Q", 0),
                   ck = env_int("SJ_ATTN_CAPS_K", 0);
  static std::mutex mu;
  static std::map<std::tuple<long, long, long, int>, std::pair<SplitPlan, int>> cache;
  const int nb = (int)(t / QB);
  if (4 * nb > PLAN_PIECES) return sjh::fail(SJ_ERR_INVALID, "grouped attention backward: t = %ld beyond the plan", t);
  {
    std::lock_guard<std::mutex> lock(mu);
    const auto key = std::make_tuple(t, window, pairs, cus);
    auto it = cache.find(key);
    if (it == cache.end()) {
      std::vector<Piece> ps;
      int ncut = 0, nslots = 0;
      plan_pieces(nb, (int)window, pairs, cus, cut_on != 0, cq, ck, ps, ncut, nslots);  // ps: costliest first
      SplitPlan p;
      memset(&p, 0, sizeof(p));
      for (size_t i = 0; i < ps.size(); i++) {
        const Piece& x = ps[i];
        p.seg[i] = (1u << 31) | (uint32_t)x.block | ((uint32_t)x.first << 6) | ((uint32_t)x.last << 12) |
                   ((uint32_t)x.role << 18) | ((uint32_t)(x.cut + 1) << 19) | ((uint32_t)x.part << 27) |
                   ((uint32_t)(x.nparts - 1) << 29);
      }
      {  // part-sum slots of each cut walk, in cut order
        std::vector<int> np((size_t)ncut, 0);
        for (const Piece& x : ps)
          if (x.cut >= 0) np[(size_t)x.cut] = x.nparts;
        int at = 0;
        for (int c = 0; c < ncut; c++) {
          p.slot0[c] = (uint16_t)at;
          at += np[(size_t)c];
        }
      }
      p.ncut = ncut;
      p.nslots = nslots;
      it = cache.emplace(key, std::make_pair(p, (int)ps.size())).first;
    }
    pl = it->second.first;
    npieces = it->second.second;
  }
  return SJ_OK;
}
}  // namespace

extern "C" int sj_attention_bwd_plan(long t, long window, long pairs, int cus, uint32_t* seg, long cap, int* ncut) {
  if (!(t > 0 && t % QB == 0 && window >= 0 && pairs > 0 && cus > 0 && seg && ncut))
    return -sjh::fail(SJ_ERR_INVALID, "attention backward plan: arguments");
  SplitPlan pl;
  int n = 0;
  if (int st = make_plan(t, window < t ? window : 0, pairs, cus, pl, n)) return -st;
  if (cap < n) return -sjh::fail(SJ_ERR_INVALID, "attention backward plan: capacity %ld < %d pieces", cap, n);
  for (int i = 0; i < n; i++) seg[i] = pl.seg[i];
  *ncut = pl.ncut;
  return n;
}

int sjh::attention_t_prepare() {
  static int done = 0, status = SJ_OK;
  if (done) return status;
  done = 1;
  hipError_t e = hipFuncSetAttribute((const void*)k_attn2_fwd<NS_FWD>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)LDS_FWD);
  if (e == hipSuccess)
    e = hipFuncSetAttribute((const void*)k_attn2_fwd_cached<NS_FWD>, hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)LDS_FWD);
  if (e == hipSuccess)
    e = hipFuncSetAttribute((const void*)k_attn2_bwd, hipFuncAttributeMaxDynamicSharedMemorySize, (int)LDS_BWD);
  if (e == hipSuccess)
    e = hipFuncSetAttribute((const void*)k_attn2_bwd_dq, hipFuncAttributeMaxDynamicSharedMemorySize, (int)LDS_DQ);
  if (e == hipSuccess)
    e = hipFuncSetAttribute((const void*)k_attn2_bwd_dkv, hipFuncAttributeMaxDynamicSharedMemorySize, (int)LDS_DKV);
  if (e == hipSuccess)
    e = hipFuncSetAttribute((const void*)k_attn2_bwd_g<GROUPED_G>, hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)(LDS_BWD_G + 16));
  status = e == hipSuccess ? SJ_OK : sjh::hip_check(e, "attention: LDS attribute");
  return status;
}

static int check_t(const void* qkv, long ldqkv, long ldt, long batch, long t, long hq, long hk, long head_dim,
                   long window) {
  SJ_REQUIRE(qkv && batch > 0 && t > 0 && t % QB == 0 && hq > 0 && hk > 0 && hq % hk == 0 && window >= 0 &&
                 head_dim == DH && ldqkv >= (hq + 2 * hk) * DH && ldqkv % 8 == 0 && ldt >= batch * t &&
                 ldt % 8 == 0 && ((uintptr_t)qkv & 15) == 0 && t * ldqkv < (1L << 31),
             "grouped attention (MFMA layout): bf16, head_dim 64, t %% 64 == 0, aligned q|k|v, ldt >= batch*t");
  return SJ_OK;
}


// One-kernel launch that, while an op is being profiled with kernel events
// (sjh::ProfHook), records events at the kernel's own start and end, so the
// kernel's time excludes any wait for CUs held by another stream's work
template <typename K, typename... A>
void launch_timed(K kern, const char* name, dim3 grid, dim3 block, size_t lds, hipStream_t s, const A&... args) {
  sjh::ProfHook& h = sjh::prof_hook();
  if (h.on && h.k0) {
    hipExtLaunchKernelGGL(kern, grid, block, (uint32_t)lds, s, h.k0, h.k1, 0u, args...);
    h.used = true;
  } else {
    hipLaunchKernelGGL(kern, grid, block, lds, s, args...);
  }
  if (h.on) snprintf(h.kernel, sizeof(h.kernel), "%s", name);
}

extern "C" int sj_attention_fwd_tt(void* stream, const uint16_t* qkv, long ldqkv, long ldt, long batch, long t,
                                   long hq, long hk, long head_dim, long window, uint16_t* o, long ldo, float* lse,
                                   float* lse_t, uint16_t* o_t, long ldot) {
  if (int st = check_t(qkv, ldqkv, ldt, batch, t, hq, hk, head_dim, window)) return st;
  SJ_REQUIRE(o && lse_t && ldo >= hq * DH && ldo % 8 == 0 && ((uintptr_t)o & 15) == 0 && (!o_t || ldot >= batch * t),
             "grouped attention: outputs");
  if (int st = sjh::attention_t_prepare()) return st;
  TArgs a = {};
  a.qkv = (const bf16_t*)qkv; a.ldqkv = ldqkv; a.ldt = ldt;
  a.T = (int)t; a.HQ = (int)hq; a.HK = (int)hk; a.window = window < t ? (int)window : 0;
  a.o = (bf16_t*)o; a.ldo = ldo; a.lse = lse; a.lse_t = lse_t; a.ot = (bf16_t*)o_t; a.ldot = ldot;
  launch_timed(k_attn2_fwd<NS_FWD>, "k_attn2_fwd<3>", dim3((unsigned)(t / QB), (unsigned)hq, (unsigned)batch),
               dim3(256), LDS_FWD, (hipStream_t)stream, a);
  SJ_LAUNCH_CHECK("hierarchy_attention");
  return SJ_OK;
}

// cached forward on the MFMA layout (one sequence; see attn2_fwd_body)
int sjh::attention_fwd_cached_t(void* stream, const uint16_t* q, long ldq, const uint16_t* k, const uint16_t* v,
                                long ldkv, long capacity, long tq, long offset, long hq, long hk, long window,
                                uint16_t* o, long ldo) {
  SJ_REQUIRE(tq > 0 && offset >= 0 && offset + tq <= capacity && capacity < (1L << 30) &&
                 (long)capacity * ldkv < (1L << 31) && hq % hk == 0 && ldq >= hq * DH && ldkv >= hk * DH &&
                 ldo >= hq * DH,
             "grouped attention (cached, MFMA layout): shapes");
  if (int st = sjh::attention_t_prepare()) return st;
  TArgs a = {};
  a.T = (int)(offset + tq); a.HQ = (int)hq; a.HK = (int)hk; a.window = (int)window; a.B = 1;
  a.qc = (const bf16_t*)q; a.ldqc = ldq; a.kc = (const bf16_t*)k; a.vc = (const bf16_t*)v; a.ldkc = ldkv;
  a.pos0 = (int)offset; a.nq = (int)tq; a.qb0 = (int)(offset / QB);
  a.o = (bf16_t*)o; a.ldo = ldo;
  const long nb = (offset + tq - 1) / QB - offset / QB + 1;
  hipLaunchKernelGGL(k_attn2_fwd_cached<NS_FWD>, dim3((unsigned)nb, (unsigned)hq, 1u), dim3(256), LDS_FWD,
                     (hipStream_t)stream, a);
  SJ_LAUNCH_CHECK("hierarchy_attention (cached)");
  return SJ_OK;
}

// the workspace: the per-head dK | dV partials (or the cut walks' part
// sums), then, 256-byte aligned, the grouped launch's meeting counters
static size_t attention_bwd_tt_partial_bytes(long batch, long t, long hq, long hk, long head_dim) {
  const size_t b = sizeof(float) * (size_t)(hq / (hk > 0 ? hk : 1)) * (size_t)(batch * t) * (size_t)(2 * hk * head_dim);
  return (b + 255) / 256 * 256;
}

extern "C" size_t sj_attention_bwd_tt_counter_bytes(long batch, long hk) {
  return sizeof(uint32_t) * (size_t)PLAN_CUTS * (size_t)(batch > 0 ? batch : 0) * (size_t)(hk > 0 ? hk : 0);
}

extern "C" size_t sj_attention_bwd_tt_workspace_bytes(long batch, long t, long hq, long hk, long head_dim) {
  return attention_bwd_tt_partial_bytes(batch, t, hq, hk, head_dim) + sj_attention_bwd_tt_counter_bytes(batch, hk);
}

int sjh::attention_bwd_tt_parts(int parts, void* stream, const uint16_t* qkv, long ldqkv, long ldt, const uint16_t* o,
                                long ldo, const float* lse_t, const uint16_t* do_hi, const uint16_t* do_lo, long lddo,
                                float* delta_t, long batch, long t, long hq, long hk, long head_dim, long window,
                                const float* rope_table, uint16_t* g_hi, uint16_t* g_lo, long ldg, uint16_t* g_t_hi,
                                uint16_t* g_t_lo, long ldgt, void* workspace, size_t workspace_bytes,
                                uint32_t* counters) {
  if (int st = check_t(qkv, ldqkv, ldt, batch, t, hq, hk, head_dim, window)) return st;
  SJ_REQUIRE(o && lse_t && do_hi && do_lo && delta_t && g_hi && g_lo && !g_t_hi == !g_t_lo && lddo >= hq * DH &&
                 lddo % 8 == 0 && ldo % 8 == 0 && ldg >= (hq + 2 * hk) * DH && (!g_t_hi || ldgt >= batch * t) &&
                 ((uintptr_t)do_hi & 15) == 0 && ((uintptr_t)do_lo & 15) == 0 && ((uintptr_t)o & 15) == 0 &&
                 ldg % 4 == 0,
             "grouped attention backward (transposed operands): buffers");
  const size_t need = counters ? attention_bwd_tt_partial_bytes(batch, t, hq, hk, head_dim)
                               : sj_attention_bwd_tt_workspace_bytes(batch, t, hq, hk, head_dim);
  if (!workspace || workspace_bytes < need)
    return sjh::fail(SJ_ERR_CAPACITY, "attention backward: required %zu bytes, available %zu bytes", need,
                     workspace_bytes);
  if (int st = sjh::attention_t_prepare()) return st;
  hipStream_t s = (hipStream_t)stream;
  TArgs a = {};
  a.qkv = (const bf16_t*)qkv; a.ldqkv = ldqkv; a.ldt = ldt;
  a.T = (int)t; a.HQ = (int)hq; a.HK = (int)hk; a.window = window < t ? (int)window : 0;
  a.ob = (const bf16_t*)o; a.ldo = ldo;
  a.dh = (const bf16_t*)do_hi; a.dl = (const bf16_t*)do_lo; a.lddo = lddo;
  a.lse_in_t = lse_t; a.delta_t = delta_t; a.rope = rope_table;
  a.gq[0] = (bf16_t*)g_hi; a.gq[1] = (bf16_t*)g_lo; a.gqt[0] = (bf16_t*)g_t_hi; a.gqt[1] = (bf16_t*)g_t_lo;
  a.ldg = ldg; a.ldgt = ldgt;
  a.part = (float*)workspace;
  a.cnt = counters ? counters
                   : (uint32_t*)((char*)workspace + attention_bwd_tt_partial_bytes(batch, t, hq, hk, head_dim));
  a.B = (int)batch;
  if (parts & 1) {  // Delta
    const long threads = 4 * batch * t * hq;
    hipLaunchKernelGGL(k_attn_delta, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s, a);
    SJ_LAUNCH_CHECK("hierarchy_attention_delta");
  }
  // the grouped launch (no dK | dV partials, no reduce): G = 3 query heads
  // per KV head, row planes only, sizes where the two roles share one launch
  const long nb = t / QB;
  const bool grouped = sjh::attention_bwd_grouped(batch, t, hq, hk, g_t_hi != nullptr);
  if ((parts & 2) && grouped) {
    SplitPlan pl;
    int npieces = 0;
    if (int st = make_plan(t, a.window, batch * hk, device_cus(), pl, npieces)) return st;
    launch_timed(k_attn2_bwd_g<GROUPED_G>, "k_attn2_bwd_g<3>", dim3((unsigned)npieces, (unsigned)hk, (unsigned)batch),
                 dim3(256 * GROUPED_G), LDS_BWD_G + 16, s, a, pl);
    SJ_LAUNCH_CHECK("hierarchy_attention_dq_dkv (grouped)");
    return SJ_OK;  // dK | dV planes written: nothing for the reduce part
  }
  if (grouped) return SJ_OK;
  if (parts & 2) {  // dQ | dK dV
    if (nb * hq * batch >= SEPARATE_ROLES) {
      const dim3 grid((unsigned)nb, (unsigned)hq, (unsigned)batch);
      hipLaunchKernelGGL(k_attn2_bwd_dq, grid, dim3(256), LDS_DQ, s, a);
      hipLaunchKernelGGL(k_attn2_bwd_dkv, grid, dim3(256), LDS_DKV, s, a);
    } else {
      hipLaunchKernelGGL(k_attn2_bwd, dim3((unsigned)(2 * nb), (unsigned)hq, (unsigned)batch), dim3(256), LDS_BWD, s,
                         a);
    }
    SJ_LAUNCH_CHECK("hierarchy_attention_dq_dkv");
  }
  if ((parts & 4) && !(hq == hk && !g_t_hi)) {  // one head per KV head: the dK | dV kernel wrote the planes
    const long M = batch * t;
    if (int st = sjh::attention_kv_reduce(s, a.part, hq / hk, M, t, hq * DH, hk * DH, rope_table, g_hi, g_lo, ldg,
                                          g_t_hi, g_t_lo, ldgt))
      return st;
  }
  return SJ_OK;
}

extern "C" int sj_attention_bwd_tt(void* stream, const uint16_t* qkv, long ldqkv, long ldt, const uint16_t* o, long ldo,
                                   const float* lse_t, const uint16_t* do_hi, const uint16_t* do_lo, long lddo,
                                   float* delta_t, long batch, long t, long hq, long hk, long head_dim, long window,
                                   const float* rope_table, uint16_t* g_hi, uint16_t* g_lo, long ldg, uint16_t* g_t_hi,
                                   uint16_t* g_t_lo, long ldgt, void* workspace, size_t workspace_bytes) {
  return sjh::attention_bwd_tt_parts(7, stream, qkv, ldqkv, ldt, o, ldo, lse_t, do_hi, do_lo, lddo, delta_t, batch, t,
                                     hq, hk, head_dim, window, rope_table, g_hi, g_lo, ldg, g_t_hi, g_t_lo, ldgt,
                                     workspace, workspace_bytes, nullptr);
}
