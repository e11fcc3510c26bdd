// bf16 MFMA GEMM family for gfx950 (v_mfma_f32_16x16x32_bf16).
//
// C[M,N] = op(A)[M,K] * op(B)[K,N] with fp32 accumulation.  One 256-thread
// workgroup (4 waves, 2x2) computes a BM x BN tile; each wave owns
// (BM/2) x (BN/2) as 16x16 MFMA blocks.  Operand tiles are staged through
// LDS in a k-contiguous layout ([row][BK] bf16, padded) so every MFMA
// fragment is one ds_read_b128, whatever the global layout:
//   kind 0  bf16, k contiguous in global  (A "N", B "T")
//   kind 1  bf16, row contiguous          (A "T", B "N")  -> 8x2 register transpose
//   kind 2  fp32, k contiguous                             -> hi/lo split
//   kind 3  fp32, row contiguous                           -> split + transpose
// fp32 operands are written to LDS as two bf16 planes (hi = RNE(x),
// lo = RNE(x - hi)) and multiplied as hi*hi + hi*lo + lo*hi, which keeps
// fp32 gradients (the reference's fp32 "ieee" dot, kernels.py:29) to ~2^-16
// relative on bf16 MFMA.  Global tiles are register double-buffered.
//
// Epilogues fuse the op that follows each projection in Block::apply
// (crates/sejong-model/src/architecture.rs:200-247): QKV + RoPE, gate/up +
// SwiGLU, projection + residual add, and on the backward the SwiGLU
// derivative into the dH GEMM.  dW GEMMs (K = tokens) use split-K with a
// fixed-order reduction (deterministic).
#include <math.h>

#include "common.h"

using namespace sj;

namespace {

constexpr int NT = 256;
constexpr int BK = 32;
constexpr int LDSK = BK + 8;  // padded row (bf16 elements)

enum Epi { EPI_STORE = 0, EPI_QKV = 1, EPI_RESID = 2, EPI_GATEUP = 3, EPI_SWIGLU_BWD = 4, EPI_PARTIAL = 5 };

struct GemmParams {
  const void* a;
  long lda;
  const void* b[3];  // B segments (QKV: Wq, Wk, Wv; gate/up: Wg, Wu)
  long ldb[3];
  long seg_n[3];  // first column of each B / output segment
  int nseg;
  void* c[3];  // outputs (QKV: Q,K,V; gate/up: G,U,H)
  long ldc[3];
  long M, N, K;
  int c_bf16;      // store dtype of outputs
  int accumulate;  // EPI_STORE fp32: C += result
  int a_vec, b_vec;
  // residual / swiglu-backward inputs
  const void* r;
  long ldr;
  const void* u;
  long ldu;
  int gu_bf16;
  long F;  // swiglu bwd: offset of dU columns
  // rope
  const float* rope;
  long rope_t, head_dim, rope_cols;  // columns [0, rope_cols) get RoPE
  // split-K
  int splits;
  long kchunk;
  float* partial;
};

__device__ __forceinline__ uint32_t lo_halves(uint32_t w0, uint32_t w1) { return (w0 & 0xffffu) | (w1 << 16); }
__device__ __forceinline__ uint32_t hi_halves(uint32_t w0, uint32_t w1) { return (w0 >> 16) | (w1 & 0xffff0000u); }

// ---------------------------------------------------------------- loaders
// A loader stages one ROWS x BK tile of an operand for rows [row0, row0+ROWS)
// and k in [k0, k0+BK).  It fetches into registers, then stores into LDS.
template <int KIND, int ROWS>
struct Loader {
  static constexpr bool F32 = (KIND >= 2);
  static constexpr bool KC = (KIND % 2 == 0);
  // k-contiguous: units of 8 k for one row
  static constexpr int KC_UNITS = ROWS * (BK / 8);
  // row-contiguous: units of 8 k x 2 rows
  static constexpr int RC_UNITS = (BK / 8) * (ROWS / 2);
  static constexpr int UNITS = KC ? KC_UNITS : RC_UNITS;
  static constexpr int PER = (UNITS + NT - 1) / NT;
  // registers: k-contig bf16: 4 words; k-contig f32: 8 floats;
  // row-contig bf16: 8 words; row-contig f32: 16 floats
  static constexpr int WORDS = KC ? (F32 ? 8 : 4) : (F32 ? 16 : 8);
  uint32_t reg[PER][WORDS];

  __device__ __forceinline__ void fetch(const void* base, long ld, long row0, long rows, long k0, long K, bool vec) {
    const int t = threadIdx.x;
#pragma unroll
    for (int p = 0; p < PER; p++) {
      const int u = t + p * NT;
      if (u >= UNITS) break;
      if constexpr (KC) {
        const int r = u / (BK / 8), kc = u % (BK / 8);
        const long row = row0 + r, k = k0 + kc * 8;
        const bool full = vec && row < rows && k + 8 <= K;
        if constexpr (!F32) {
          const bf16_t* src = (const bf16_t*)base + row * ld + k;
          if (full) {
            u32x4 v = *(const u32x4*)src;
            reg[p][0] = v.x; reg[p][1] = v.y; reg[p][2] = v.z; reg[p][3] = v.w;
          } else {
#pragma unroll
            for (int i = 0; i < 4; i++) {
              uint32_t lo = (row < rows && k + 2 * i < K) ? src[2 * i] : 0;
              uint32_t hi = (row < rows && k + 2 * i + 1 < K) ? src[2 * i + 1] : 0;
              reg[p][i] = lo | (hi << 16);
            }
          }
        } else {
          const float* src = (const float*)base + row * ld + k;
          if (full) {
            float4 v0 = *(const float4*)src, v1 = *(const float4*)(src + 4);
            reg[p][0] = __float_as_uint(v0.x); reg[p][1] = __float_as_uint(v0.y);
            reg[p][2] = __float_as_uint(v0.z); reg[p][3] = __float_as_uint(v0.w);
            reg[p][4] = __float_as_uint(v1.x); reg[p][5] = __float_as_uint(v1.y);
            reg[p][6] = __float_as_uint(v1.z); reg[p][7] = __float_as_uint(v1.w);
          } else {
#pragma unroll
            for (int i = 0; i < 8; i++)
              reg[p][i] = (row < rows && k + i < K) ? __float_as_uint(src[i]) : 0u;
          }
        }
      } else {
        const int kb = u / (ROWS / 2), rp = u % (ROWS / 2);
        const long row = row0 + 2 * rp, k = k0 + kb * 8;
        const bool full = vec && row + 2 <= rows && k + 8 <= K;
        if constexpr (!F32) {
          const bf16_t* src = (const bf16_t*)base + k * ld + row;
          if (full) {
#pragma unroll
            for (int i = 0; i < 8; i++) reg[p][i] = *(const uint32_t*)(src + (long)i * ld);
          } else {
#pragma unroll
            for (int i = 0; i < 8; i++) {
              bool kin = k + i < K;
              uint32_t lo = (kin && row < rows) ? src[(long)i * ld] : 0;
              uint32_t hi = (kin && row + 1 < rows) ? src[(long)i * ld + 1] : 0;
              reg[p][i] = lo | (hi << 16);
            }
          }
        } else {
          const float* src = (const float*)base + k * ld + row;
          if (full) {
#pragma unroll
            for (int i = 0; i < 8; i++) {
              float2 v = *(const float2*)(src + (long)i * ld);
              reg[p][2 * i] = __float_as_uint(v.x);
              reg[p][2 * i + 1] = __float_as_uint(v.y);
            }
          } else {
#pragma unroll
            for (int i = 0; i < 8; i++) {
              bool kin = k + i < K;
              reg[p][2 * i] = (kin && row < rows) ? __float_as_uint(src[(long)i * ld]) : 0u;
              reg[p][2 * i + 1] = (kin && row + 1 < rows) ? __float_as_uint(src[(long)i * ld + 1]) : 0u;
            }
          }
        }
      }
    }
  }

  // hi / lo planes, each ROWS x LDSK bf16
  __device__ __forceinline__ void store(bf16_t* hi, bf16_t* lo) const {
    const int t = threadIdx.x;
#pragma unroll
    for (int p = 0; p < PER; p++) {
      const int u = t + p * NT;
      if (u >= UNITS) break;
      if constexpr (KC) {
        const int r = u / (BK / 8), kc = u % (BK / 8);
        bf16_t* dh = hi + r * LDSK + kc * 8;
        if constexpr (!F32) {
          *(u32x4*)dh = u32x4{reg[p][0], reg[p][1], reg[p][2], reg[p][3]};
        } else {
          bf16_t h[8], l[8];
#pragma unroll
          for (int i = 0; i < 8; i++) split_bf(__uint_as_float(reg[p][i]), h[i], l[i]);
          *(u32x4*)dh = u32x4{pack2(h[0], h[1]), pack2(h[2], h[3]), pack2(h[4], h[5]), pack2(h[6], h[7])};
          *(u32x4*)(lo + r * LDSK + kc * 8) =
              u32x4{pack2(l[0], l[1]), pack2(l[2], l[3]), pack2(l[4], l[5]), pack2(l[6], l[7])};
        }
      } else {
        const int kb = u / (ROWS / 2), rp = u % (ROWS / 2);
        bf16_t* d0 = hi + (2 * rp) * LDSK + kb * 8;
        bf16_t* d1 = d0 + LDSK;
        if constexpr (!F32) {
          const uint32_t* w = reg[p];
          *(u32x4*)d0 = u32x4{lo_halves(w[0], w[1]), lo_halves(w[2], w[3]), lo_halves(w[4], w[5]),
                              lo_halves(w[6], w[7])};
          *(u32x4*)d1 = u32x4{hi_halves(w[0], w[1]), hi_halves(w[2], w[3]), hi_halves(w[4], w[5]),
                              hi_halves(w[6], w[7])};
        } else {
          // reg[2i] = (k=i, row0), reg[2i+1] = (k=i, row1)
          bf16_t h0[8], l0[8], h1[8], l1[8];
#pragma unroll
          for (int i = 0; i < 8; i++) {
            split_bf(__uint_as_float(reg[p][2 * i]), h0[i], l0[i]);
            split_bf(__uint_as_float(reg[p][2 * i + 1]), h1[i], l1[i]);
          }
          *(u32x4*)d0 = u32x4{pack2(h0[0], h0[1]), pack2(h0[2], h0[3]), pack2(h0[4], h0[5]), pack2(h0[6], h0[7])};
          *(u32x4*)d1 = u32x4{pack2(h1[0], h1[1]), pack2(h1[2], h1[3]), pack2(h1[4], h1[5]), pack2(h1[6], h1[7])};
          bf16_t* e0 = lo + (2 * rp) * LDSK + kb * 8;
          *(u32x4*)e0 = u32x4{pack2(l0[0], l0[1]), pack2(l0[2], l0[3]), pack2(l0[4], l0[5]), pack2(l0[6], l0[7])};
          *(u32x4*)(e0 + LDSK) =
              u32x4{pack2(l1[0], l1[1]), pack2(l1[2], l1[3]), pack2(l1[4], l1[5]), pack2(l1[6], l1[7])};
        }
      }
    }
  }
};

__device__ __forceinline__ float sigm(float g) { return 1.f / (1.f + expf(-g)); }

__device__ __forceinline__ float store_round(float v, int bf) { return bf ? round_bf(v) : v; }

__device__ __forceinline__ void put(void* c, long idx, float v, int bf) {
  if (bf)
    ((bf16_t*)c)[idx] = f2bf(v);
  else
    ((float*)c)[idx] = v;
}

// ------------------------------------------------------------------ kernel
template <int BM, int BN, int AK, int BKND, int EPI>
__global__ __launch_bounds__(NT) void k_gemm(GemmParams p) {
  constexpr bool DUAL = (EPI == EPI_GATEUP);
  constexpr bool AF = AK >= 2, BF = BKND >= 2;
  constexpr int NB_MAT = DUAL ? 2 : 1;
  constexpr int WM = BM / 2, WN = BN / 2;
  constexpr int MB = WM / 16, NB = WN / 16;
  constexpr int APL = AF ? 2 : 1, BPL = BF ? 2 : 1;
  constexpr int ASZ = BM * LDSK, BSZ = BN * LDSK;
  constexpr int STAGE = APL * ASZ + NB_MAT * BPL * BSZ;
  __shared__ __attribute__((aligned(16))) bf16_t lds[2 * STAGE];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const long m0 = (long)blockIdx.y * BM;
  const long n0 = (long)blockIdx.x * BN;
  // segment of the N axis this tile lies in
  int seg = 0;
#pragma unroll
  for (int s = 1; s < 3; s++)
    if (s < p.nseg && n0 >= p.seg_n[s]) seg = s;
  const long nl0 = n0 - p.seg_n[seg];  // tile start within the segment
  const long seg_end = (seg + 1 < p.nseg) ? p.seg_n[seg + 1] : p.N;
  const long nseg_cols = seg_end - p.seg_n[seg];
  const void* bptr0 = DUAL ? p.b[0] : p.b[seg];
  const long ldb0 = DUAL ? p.ldb[0] : p.ldb[seg];

  long kbeg = 0, kend = p.K;
  if (EPI == EPI_PARTIAL) {
    kbeg = (long)blockIdx.z * p.kchunk;
    kend = kbeg + p.kchunk < p.K ? kbeg + p.kchunk : p.K;
  }

  Loader<AK, BM> la;
  Loader<BKND, BN> lb0;
  Loader<BKND, BN> lb1;

  f32x4 acc[NB_MAT][MB][NB];
#pragma unroll
  for (int q = 0; q < NB_MAT; q++)
#pragma unroll
    for (int i = 0; i < MB; i++)
#pragma unroll
      for (int j = 0; j < NB; j++) acc[q][i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto fetch = [&](long k0) {
    la.fetch(p.a, p.lda, m0, p.M, k0, kend, p.a_vec);
    lb0.fetch(bptr0, ldb0, nl0, nseg_cols, k0, kend, p.b_vec);
    if constexpr (DUAL) lb1.fetch(p.b[1], p.ldb[1], nl0, nseg_cols, k0, kend, p.b_vec);
  };
  auto stage_ptr = [&](int s) { return lds + s * STAGE; };
  auto store = [&](int s) {
    bf16_t* base = stage_ptr(s);
    la.store(base, AF ? base + ASZ : nullptr);
    bf16_t* bb = base + APL * ASZ;
    lb0.store(bb, BF ? bb + BSZ : nullptr);
    if constexpr (DUAL) lb1.store(bb + BPL * BSZ, BF ? bb + BPL * BSZ + BSZ : nullptr);
  };

  const int fr = lane & 15, fk = (lane >> 4) * 8;
  if (kbeg < kend) {
    fetch(kbeg);
    store(0);
    __syncthreads();
    int cur = 0;
    for (long k0 = kbeg; k0 < kend; k0 += BK) {
      const bool more = k0 + BK < kend;
      if (more) fetch(k0 + BK);
      const bf16_t* base = stage_ptr(cur);
      bf16x8 ah[MB], al[MB];
#pragma unroll
      for (int i = 0; i < MB; i++) {
        const bf16_t* src = base + (wm * WM + i * 16 + fr) * LDSK + fk;
        ah[i] = __builtin_bit_cast(bf16x8, *(const u32x4*)src);
        if constexpr (AF) al[i] = __builtin_bit_cast(bf16x8, *(const u32x4*)(src + ASZ));
      }
#pragma unroll
      for (int q = 0; q < NB_MAT; q++) {
        const bf16_t* bb = base + APL * ASZ + q * BPL * BSZ;
#pragma unroll
        for (int j = 0; j < NB; j++) {
          const bf16_t* src = bb + (wn * WN + j * 16 + fr) * LDSK + fk;
          bf16x8 bh = __builtin_bit_cast(bf16x8, *(const u32x4*)src);
          bf16x8 bl;
          if constexpr (BF) bl = __builtin_bit_cast(bf16x8, *(const u32x4*)(src + BSZ));
#pragma unroll
          for (int i = 0; i < MB; i++) {
            acc[q][i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah[i], bh, acc[q][i][j], 0, 0, 0);
            if constexpr (BF) acc[q][i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah[i], bl, acc[q][i][j], 0, 0, 0);
            if constexpr (AF) acc[q][i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al[i], bh, acc[q][i][j], 0, 0, 0);
          }
        }
      }
      if (more) {
        store(cur ^ 1);
        __syncthreads();
        cur ^= 1;
      }
    }
  }

  // ---------------------------------------------------------- epilogue
  // acc[q][i][j][r] = C[m0 + wm*WM + 16i + 4*(lane/16) + r][n0 + wn*WN + 16j + lane%16]
  const int cr = (lane >> 4) * 4, cc = lane & 15;
#pragma unroll
  for (int i = 0; i < MB; i++) {
#pragma unroll
    for (int j = 0; j < NB; j++) {
      const long ncol = n0 + wn * WN + j * 16 + cc;  // global column
      const long nloc = ncol - p.seg_n[seg];         // column within segment
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const long m = m0 + wm * WM + i * 16 + cr + r;
        float v = acc[0][i][j][r];
        if constexpr (EPI == EPI_QKV) {
          // round to storage, RoPE pair (2i, 2i+1) lives in lanes (l, l^1)
          float a = store_round(v, p.c_bf16);
          float b = __shfl_xor(a, 1, 64);
          float outv = a;
          if (ncol < p.rope_cols) {
            const long pos = m % p.rope_t;
            const long pair = (nloc % p.head_dim) >> 1;
            const float2 cs = *(const float2*)(p.rope + 2 * (pos * (p.head_dim >> 1) + pair));
            outv = (cc & 1) ? (b * cs.y + a * cs.x) : (a * cs.x - b * cs.y);
          }
          if (m < p.M && ncol < p.N) put(p.c[seg], m * p.ldc[seg] + nloc, outv, p.c_bf16);
        } else if constexpr (EPI == EPI_RESID) {
          if (m < p.M && ncol < p.N) {
            float a = store_round(v, p.c_bf16);
            float rr = p.c_bf16 ? bf2f(((const bf16_t*)p.r)[m * p.ldr + ncol]) : ((const float*)p.r)[m * p.ldr + ncol];
            put(p.c[0], m * p.ldc[0] + ncol, rr + a, p.c_bf16);
          }
        } else if constexpr (EPI == EPI_GATEUP) {
          if (m < p.M && ncol < p.N) {
            float g = store_round(v, p.c_bf16);
            float uu = store_round(acc[1][i][j][r], p.c_bf16);
            put(p.c[0], m * p.ldc[0] + ncol, g, p.c_bf16);
            put(p.c[1], m * p.ldc[0] + ncol, uu, p.c_bf16);
            put(p.c[2], m * p.ldc[0] + ncol, g * sigm(g) * uu, p.c_bf16);
          }
        } else if constexpr (EPI == EPI_SWIGLU_BWD) {
          if (m < p.M && ncol < p.N) {
            float g = p.gu_bf16 ? bf2f(((const bf16_t*)p.r)[m * p.ldr + ncol]) : ((const float*)p.r)[m * p.ldr + ncol];
            float uu = p.gu_bf16 ? bf2f(((const bf16_t*)p.u)[m * p.ldu + ncol]) : ((const float*)p.u)[m * p.ldu + ncol];
            float s = sigm(g);
            float* out = (float*)p.c[0];
            out[m * p.ldc[0] + ncol] = v * uu * s * (1.f + g * (1.f - s));
            out[m * p.ldc[0] + p.F + ncol] = v * g * s;
          }
        } else if constexpr (EPI == EPI_PARTIAL) {
          if (m < p.M && ncol < p.N) p.partial[((long)blockIdx.z * p.M + m) * p.N + ncol] = v;
        } else {  // EPI_STORE
          if (m < p.M && ncol < p.N) {
            long idx = m * p.ldc[0] + ncol;
            if (p.c_bf16)
              ((bf16_t*)p.c[0])[idx] = f2bf(v);
            else if (p.accumulate)
              ((float*)p.c[0])[idx] += v;
            else
              ((float*)p.c[0])[idx] = v;
          }
        }
      }
    }
  }
}

// split-K reduction in fixed order, then the EPI_STORE semantics
__global__ __launch_bounds__(256) void k_splitk_reduce(const float* __restrict__ partial, int splits, long M, long N,
                                                       void* c, long ldc, int c_bf16, int accumulate) {
  const long total = M * N;
  for (long i = blockIdx.x * 256L + threadIdx.x; i < total; i += (long)gridDim.x * 256L) {
    float s = 0.f;
    for (int z = 0; z < splits; z++) s += partial[(long)z * total + i];
    const long m = i / N, n = i - m * N;
    const long idx = m * ldc + n;
    if (c_bf16)
      ((bf16_t*)c)[idx] = f2bf(s);
    else if (accumulate)
      ((float*)c)[idx] += s;
    else
      ((float*)c)[idx] = s;
  }
}

// ----------------------------------------------------------------- launch
template <int BM, int BN, int AK, int BKND, int EPI>
void launch_cfg(hipStream_t s, const GemmParams& p, int splits) {
  dim3 grid((unsigned)((p.N + BN - 1) / BN), (unsigned)((p.M + BM - 1) / BM), (unsigned)splits);
  hipLaunchKernelGGL((k_gemm<BM, BN, AK, BKND, EPI>), grid, dim3(NT), 0, s, p);
}

template <int AK, int BKND, int EPI>
int launch_tiles(hipStream_t s, const GemmParams& p, int bm, int bn, int splits) {
  if (bm == 128 && bn == 128) launch_cfg<128, 128, AK, BKND, EPI>(s, p, splits);
  else if (bm == 128 && bn == 64) launch_cfg<128, 64, AK, BKND, EPI>(s, p, splits);
  else if (bm == 64 && bn == 128) launch_cfg<64, 128, AK, BKND, EPI>(s, p, splits);
  else launch_cfg<64, 64, AK, BKND, EPI>(s, p, splits);
  return SJ_OK;
}

template <int EPI>
int launch_kinds(hipStream_t s, const GemmParams& p, int ak, int bk, int bm, int bn, int splits) {
#define SJ_CASE(A, B) \
  if (ak == A && bk == B) return launch_tiles<A, B, EPI>(s, p, bm, bn, splits);
  SJ_CASE(0, 0) SJ_CASE(0, 1) SJ_CASE(0, 2) SJ_CASE(0, 3)
  SJ_CASE(1, 0) SJ_CASE(1, 1) SJ_CASE(1, 2) SJ_CASE(1, 3)
  SJ_CASE(2, 0) SJ_CASE(2, 1) SJ_CASE(2, 2) SJ_CASE(2, 3)
  SJ_CASE(3, 0) SJ_CASE(3, 1) SJ_CASE(3, 2) SJ_CASE(3, 3)
#undef SJ_CASE
  return sjh::fail(SJ_ERR_UNSUPPORTED, "gemm: operand kinds %d/%d", ak, bk);
}

// fused epilogues only need the kinds the training step uses
template <int EPI>
int launch_fused(hipStream_t s, const GemmParams& p, int ak, int bk, int bm, int bn) {
  if (ak == 0 && bk == 1) return launch_tiles<0, 1, EPI>(s, p, bm, bn, 1);  // bf16 fwd
  if (ak == 2 && bk == 3) return launch_tiles<2, 3, EPI>(s, p, bm, bn, 1);  // fp32 fwd
  if (ak == 2 && bk == 0) return launch_tiles<2, 0, EPI>(s, p, bm, bn, 1);  // dY(f32) W^T(bf16)
  if (ak == 2 && bk == 2) return launch_tiles<2, 2, EPI>(s, p, bm, bn, 1);  // dY(f32) W^T(f32)
  return sjh::fail(SJ_ERR_UNSUPPORTED, "fused gemm: operand kinds %d/%d", ak, bk);
}

inline int kind_of(int dtype, bool kcontig) { return (dtype == SJ_F32 ? 2 : 0) + (kcontig ? 0 : 1); }

inline bool aligned(const void* ptr, long ld, int dtype, bool kcontig) {
  uintptr_t a = (uintptr_t)ptr;
  if (dtype == SJ_BF16) return kcontig ? (a % 16 == 0 && ld % 8 == 0) : (a % 4 == 0 && ld % 2 == 0);
  return kcontig ? (a % 16 == 0 && ld % 4 == 0) : (a % 8 == 0 && ld % 2 == 0);
}

int g_num_cu = 0;
int num_cu() {
  if (!g_num_cu) {
    int dev = 0, cu = 256;
    if (hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&cu, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess)
      g_num_cu = cu;
    else
      g_num_cu = 256;
  }
  return g_num_cu;
}

// Tile choice: the largest tile that still gives >= one workgroup per CU,
// else the smallest.
void choose_tiles(long M, long N, int& bm, int& bn) {
  const long cu = num_cu();
  const int cand[4][2] = {{128, 128}, {128, 64}, {64, 128}, {64, 64}};
  for (auto& c : cand) {
    long tiles = ((M + c[0] - 1) / c[0]) * ((N + c[1] - 1) / c[1]);
    if (tiles >= cu) {
      bm = c[0];
      bn = c[1];
      return;
    }
  }
  bm = 64;
  bn = 64;
}

int splitk_count(long M, long N, long K, int bm, int bn) {
  long tiles = ((M + bm - 1) / bm) * ((N + bn - 1) / bn);
  const long cu = num_cu();
  if (tiles >= cu || K < 1024) return 1;
  long s = (2 * cu + tiles - 1) / tiles;
  long maxs = K / 256;
  if (s > maxs) s = maxs;
  if (s > 32) s = 32;
  return s < 1 ? 1 : (int)s;
}

}  // namespace

// ============================================================== C ABI

extern "C" size_t sj_gemm_workspace_bytes(long M, long N, long K) {
  int bm, bn;
  choose_tiles(M, N, bm, bn);
  int s = splitk_count(M, N, K, bm, bn);
  return s > 1 ? sizeof(float) * (size_t)s * (size_t)M * (size_t)N : 0;
}

extern "C" int sj_gemm(void* stream, int ta, int tb, long M, long N, long K, const void* a, int ad, long lda,
                       const void* b, int bd, long ldb, void* c, int cd, long ldc, int accumulate, void* workspace,
                       size_t workspace_bytes) {
  SJ_REQUIRE((ad == SJ_F32 || ad == SJ_BF16) && (bd == SJ_F32 || bd == SJ_BF16) && (cd == SJ_F32 || cd == SJ_BF16),
             "matmul dtype %d/%d/%d", ad, bd, cd);
  SJ_REQUIRE(M >= 0 && N >= 0 && K >= 0, "matmul requires matrices");
  SJ_REQUIRE(lda >= (ta ? M : K) && ldb >= (tb ? K : N) && ldc >= N, "matmul inner dimension mismatch");
  SJ_REQUIRE(!(accumulate && cd == SJ_BF16), "matmul: accumulate needs an fp32 output");
  if (M == 0 || N == 0) return SJ_OK;
  hipStream_t s = (hipStream_t)stream;
  if (K == 0) {
    if (!accumulate) {
      for (long m = 0; m < M; m++) SJ_HIP(hipMemsetAsync((char*)c + m * ldc * (cd == SJ_F32 ? 4 : 2), 0, N * (cd == SJ_F32 ? 4 : 2), s));
    }
    return SJ_OK;
  }
  const bool akc = !ta, bkc = tb;  // A "N" is k-contiguous; B "T" is k-contiguous
  GemmParams p = {};
  p.a = a; p.lda = lda;
  p.b[0] = b; p.ldb[0] = ldb; p.seg_n[0] = 0; p.nseg = 1;
  p.c[0] = c; p.ldc[0] = ldc;
  p.M = M; p.N = N; p.K = K;
  p.c_bf16 = cd == SJ_BF16; p.accumulate = accumulate;
  p.a_vec = aligned(a, lda, ad, akc);
  p.b_vec = aligned(b, ldb, bd, bkc);
  int bm, bn;
  choose_tiles(M, N, bm, bn);
  int splits = splitk_count(M, N, K, bm, bn);
  const int ak = kind_of(ad, akc), bk = kind_of(bd, bkc);
  if (splits > 1 && workspace_bytes >= sizeof(float) * (size_t)splits * M * N && workspace) {
    long kchunk = (K + splits - 1) / splits;
    kchunk = (kchunk + BK - 1) / BK * BK;
    splits = (int)((K + kchunk - 1) / kchunk);
    p.splits = splits; p.kchunk = kchunk; p.partial = (float*)workspace;
    int st = launch_kinds<EPI_PARTIAL>(s, p, ak, bk, bm, bn, splits);
    if (st) return st;
    long total = M * N;
    long blocks = (total + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    hipLaunchKernelGGL(k_splitk_reduce, dim3((unsigned)blocks), dim3(256), 0, s, (const float*)workspace, splits, M, N,
                       c, ldc, (int)p.c_bf16, accumulate);
  } else {
    int st = launch_kinds<EPI_STORE>(s, p, ak, bk, bm, bn, 1);
    if (st) return st;
  }
  SJ_LAUNCH_CHECK("matmul");
  return SJ_OK;
}

extern "C" int sj_qkv_fwd(void* stream, const void* x, long ldx, long M, long D, const void* wq, long ldwq,
                          const void* wk, long ldwk, const void* wv, long ldwv, long N, long KV, void* q, long ldq,
                          void* k, long ldk, void* v, long ldv, int dtype, const float* rope_table, long rope_t,
                          long head_dim) {
  SJ_REQUIRE(dtype == SJ_F32 || dtype == SJ_BF16, "project_qkv dtype %d", dtype);
  SJ_REQUIRE(M >= 0 && D > 0 && N > 0 && KV > 0 && ldx >= D && ldwq >= N && ldwk >= KV && ldwv >= KV && ldq >= N &&
                 ldk >= KV && ldv >= KV,
             "project_qkv shape mismatch");
  if (rope_table) SJ_REQUIRE(rope_t > 0 && head_dim > 0 && head_dim % 2 == 0 && N % head_dim == 0 && KV % head_dim == 0,
                             "project_qkv rope: t %ld head_dim %ld", rope_t, head_dim);
  if (M == 0) return SJ_OK;
  int bm, bn;
  choose_tiles(M, N + 2 * KV, bm, bn);
  if (N % bn || KV % bn) bn = 64;
  SJ_REQUIRE(N % bn == 0 && KV % bn == 0, "project_qkv: widths %ld/%ld must be multiples of 64", N, KV);
  GemmParams p = {};
  p.a = x; p.lda = ldx;
  p.b[0] = wq; p.b[1] = wk; p.b[2] = wv;
  p.ldb[0] = ldwq; p.ldb[1] = ldwk; p.ldb[2] = ldwv;
  p.seg_n[0] = 0; p.seg_n[1] = N; p.seg_n[2] = N + KV; p.nseg = 3;
  p.c[0] = q; p.c[1] = k; p.c[2] = v;
  p.ldc[0] = ldq; p.ldc[1] = ldk; p.ldc[2] = ldv;
  p.M = M; p.N = N + 2 * KV; p.K = D;
  p.c_bf16 = dtype == SJ_BF16;
  p.a_vec = aligned(x, ldx, dtype, true);
  p.b_vec = aligned(wq, ldwq, dtype, false) && aligned(wk, ldwk, dtype, false) && aligned(wv, ldwv, dtype, false);
  p.rope = rope_table;
  p.rope_t = rope_t > 0 ? rope_t : 1;
  p.head_dim = head_dim > 0 ? head_dim : 2;
  p.rope_cols = rope_table ? N + KV : 0;
  int kd = dtype == SJ_F32 ? 2 : 0;
  int st = launch_fused<EPI_QKV>((hipStream_t)stream, p, kd, kd + 1, bm, bn);
  if (st) return st;
  SJ_LAUNCH_CHECK("project_qkv");
  return SJ_OK;
}

extern "C" int sj_gate_up_fwd(void* stream, const void* x, long ldx, long M, long D, const void* wg, long ldwg,
                              const void* wu, long ldwu, long F, void* g, void* u, void* h, long ldo, int dtype) {
  SJ_REQUIRE(dtype == SJ_F32 || dtype == SJ_BF16, "gate_up dtype %d", dtype);
  SJ_REQUIRE(M >= 0 && D > 0 && F > 0 && ldx >= D && ldwg >= F && ldwu >= F && ldo >= F, "gate_up shape mismatch");
  if (M == 0) return SJ_OK;
  int bm, bn;
  choose_tiles(M, F, bm, bn);
  GemmParams p = {};
  p.a = x; p.lda = ldx;
  p.b[0] = wg; p.b[1] = wu; p.ldb[0] = ldwg; p.ldb[1] = ldwu;
  p.seg_n[0] = 0; p.nseg = 1;
  p.c[0] = g; p.c[1] = u; p.c[2] = h; p.ldc[0] = ldo;
  p.M = M; p.N = F; p.K = D;
  p.c_bf16 = dtype == SJ_BF16;
  p.a_vec = aligned(x, ldx, dtype, true);
  p.b_vec = aligned(wg, ldwg, dtype, false) && aligned(wu, ldwu, dtype, false);
  int kd = dtype == SJ_F32 ? 2 : 0;
  int st = launch_fused<EPI_GATEUP>((hipStream_t)stream, p, kd, kd + 1, bm, bn);
  if (st) return st;
  SJ_LAUNCH_CHECK("gate_up");
  return SJ_OK;
}

extern "C" int sj_linear_residual_fwd(void* stream, const void* x, long ldx, long M, long K, const void* w, long ldw,
                                      long N, const void* r, long ldr, void* y, long ldy, int dtype) {
  SJ_REQUIRE(dtype == SJ_F32 || dtype == SJ_BF16, "linear_residual dtype %d", dtype);
  SJ_REQUIRE(M >= 0 && K > 0 && N > 0 && ldx >= K && ldw >= N && ldr >= N && ldy >= N, "add shape mismatch");
  if (M == 0) return SJ_OK;
  int bm, bn;
  choose_tiles(M, N, bm, bn);
  GemmParams p = {};
  p.a = x; p.lda = ldx;
  p.b[0] = w; p.ldb[0] = ldw; p.seg_n[0] = 0; p.nseg = 1;
  p.c[0] = y; p.ldc[0] = ldy;
  p.r = r; p.ldr = ldr;
  p.M = M; p.N = N; p.K = K;
  p.c_bf16 = dtype == SJ_BF16;
  p.a_vec = aligned(x, ldx, dtype, true);
  p.b_vec = aligned(w, ldw, dtype, false);
  int kd = dtype == SJ_F32 ? 2 : 0;
  int st = launch_fused<EPI_RESID>((hipStream_t)stream, p, kd, kd + 1, bm, bn);
  if (st) return st;
  SJ_LAUNCH_CHECK("linear_residual");
  return SJ_OK;
}

extern "C" int sj_down_bwd_swiglu(void* stream, const float* dy, long lddy, long M, long D, const void* w_down,
                                  long ldw, long F, const void* g, const void* u, long ldgu, int gu_dtype, float* dgu,
                                  long lddgu) {
  SJ_REQUIRE(gu_dtype == SJ_F32 || gu_dtype == SJ_BF16, "swiglu_backward dtype %d", gu_dtype);
  SJ_REQUIRE(M >= 0 && D > 0 && F > 0 && lddy >= D && ldw >= D && ldgu >= F && lddgu >= 2 * F,
             "swiglu_backward shape mismatch");
  if (M == 0) return SJ_OK;
  int bm, bn;
  choose_tiles(M, F, bm, bn);
  GemmParams p = {};
  p.a = dy; p.lda = lddy;
  p.b[0] = w_down; p.ldb[0] = ldw; p.seg_n[0] = 0; p.nseg = 1;  // B = W_down^T: B[k][n] = W[n][k], k-contiguous
  p.c[0] = dgu; p.ldc[0] = lddgu;
  p.r = g; p.ldr = ldgu; p.u = u; p.ldu = ldgu; p.gu_bf16 = gu_dtype == SJ_BF16; p.F = F;
  p.M = M; p.N = F; p.K = D;
  p.a_vec = aligned(dy, lddy, SJ_F32, true);
  p.b_vec = aligned(w_down, ldw, gu_dtype, true);
  int bk = gu_dtype == SJ_F32 ? 2 : 0;
  int st = launch_fused<EPI_SWIGLU_BWD>((hipStream_t)stream, p, 2, bk, bm, bn);
  if (st) return st;
  SJ_LAUNCH_CHECK("swiglu_backward");
  return SJ_OK;
}
