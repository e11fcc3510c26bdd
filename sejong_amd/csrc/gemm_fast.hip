// Streaming bf16 MFMA GEMM for operands laid out for the MFMA (gfx950).
//
// Every operand is one or two bf16 planes stored k-contiguous ([rows][K],
// row stride ld): an fp32 operand arrives pre-split as hi = RNE(x),
// lo = RNE(x - hi) by its producer, and an operand whose natural layout is
// row-contiguous (weights in the forward, activations / gradients in dW)
// arrives as the transposed copy its producer wrote.  The k-loop therefore
// only moves bytes: tiles go global -> LDS with global_load_lds_dwordx4 (no
// registers), three stages deep, BK = 64.  Each 16-byte chunk c of LDS row r
// is stored at position c ^ (r & 7) (the XOR is applied to the global
// address each lane fetches, since a DMA lane always writes base + 16*lane),
// so MFMA fragment reads (16 rows x one chunk) hit distinct banks without
// padding.  Products: hi*hi + hi*lo + lo*hi on v_mfma_f32_16x16x32_bf16.
//
// Epilogues fuse the op after each projection of Block::apply (crates/
// sejong-model/src/architecture.rs:200-247) and write the layouts the next
// GEMMs read:
//   QKV + RoPE (bf16), residual add (bf16), gate/up + SwiGLU (g, u, h and
//   h^T), SwiGLU derivative of the down dX (dG|dU as hi/lo planes, normal
//   and transposed), plain fp32 / bf16 stores and split-K partials.
#include <math.h>
#include <stdio.h>
#include <stdlib.h>

#include <hip/hip_ext.h>

#include "common.h"

using namespace sj;

namespace sjh {
int gemm_fast_prepare();
}

namespace {

constexpr int NT = 256;
constexpr int BK = 64;

typedef __attribute__((address_space(3))) void lds_void;

__device__ __attribute__((aligned(64))) uint8_t g_zero16[64];  // zero source for masked DMA lanes

// E_SWIGLU_ROWS: the SwiGLU derivative of E_SWIGLU_BWD with row planes only
// (no transposed outputs): G/U are prefetched as 16-byte vectors before the
// main loop, dH is staged in LDS as fp32 and each thread writes whole 16-byte
// chunks of the four planes
enum Epi { E_STORE = 0, E_PARTIAL = 1, E_QKV = 2, E_RESID = 3, E_GATEUP = 4, E_SWIGLU_BWD = 5, E_PLANES = 6,
           E_SWIGLU_ROWS = 7 };

struct FParams {
  const bf16_t* a[2];  // A planes (hi, lo), [M][K] k-contiguous
  long lda;
  const bf16_t* b[2][3];  // B planes x segments (QKV: Wq^T,Wk^T,Wv^T; gate/up: Wg^T,Wu^T), [N][K]
  long ldb[3];
  long seg_n[3];
  int nseg;
  long M, N, K;
  // outputs
  void* c[4];
  long ldc[4];
  int c_bf16, accumulate;
  // residual / swiglu inputs
  const bf16_t* r;
  long ldr;
  const bf16_t* gin;
  const bf16_t* uin;
  long ldgu;
  long F;
  // E_PLANES: Delta of the attention backward (nullable): delta[h][m] =
  // sum over head h's 64 columns of the stored dO planes times o
  const bf16_t* o;
  long ldo;
  float* delta;
  long lddelta;
  // rope
  const float* rope;
  long rope_t, head_dim, rope_cols;
  // split-K
  long kchunk;
  float* partial;
  int xcd_remap;
  // grouped (MoE) launches over expert segments given by device offsets
  // goff[0..gE] (multiples of 64):
  //   gmode 1: rows of the packed matrix; a tile's expert is the segment
  //            holding its first row (BM = 64), B is read at b + e*gstride_b;
  //   gmode 2: blockIdx.z = expert; K range [goff[e], goff[e+1]), C is
  //            written at c + e*gstride_c (per-expert dW).
  const int* goff;
  int gE, gmode;
  long gstride_b, gstride_c;
  // n / d as (n * m) >> 40 with m = 2^40 / d + 1 (exact for n, d < 2^20):
  // the grid's smaller tile count and the tiles of one K slice
  unsigned long long mdiv_lo, mdiv_xy;
  // k_gemm_kw E_STORE (nullable): FP64 sum of squares of the values each
  // workgroup stores, at sq[linear workgroup id] (the gradient-norm hook)
  double* sq;
  // tile order: row panels per group (0: the smaller tile dimension fastest)
  int group;
};

// Grouped tile order (row panels per group) when the B panels of one row of
// tiles exceed 4 MiB, the L2 of one XCD; SJ_GEMM_GROUP=<n> overrides it
// (0: off; sweeps).
int tile_group(long n_cols, long K, int planes, unsigned row_tiles) {
  static int ov = -2;
  if (ov == -2) {
    const char* e = getenv("SJ_GEMM_GROUP");
    ov = e ? atoi(e) : -1;
  }
  if (ov >= 0) return ov;
  const double bbytes = 2.0 * (double)n_cols * (double)K * planes;
  return bbytes > 4.0 * 1024 * 1024 && row_tiles >= 8 ? 4 : 0;
}

int g_remap = -1;
int xcd_remap() {
  if (g_remap < 0) {
    const char* e = getenv("SJ_GEMM_XCD_REMAP");
    g_remap = e ? atoi(e) != 0 : 1;
  }
  return g_remap;
}

// s_waitcnt vmcnt(N) with the other counters unconstrained (gfx9 encoding:
// vmcnt[3:0] in bits 3:0, vmcnt[5:4] in bits 15:14)
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// One LDS-DMA: each lane's 16 bytes at `src` land in LDS at lds_addr +
// 16 * lane.  Issued through inline asm so the compiler does not treat later
// LDS reads as dependent on it (it would otherwise wait for vmcnt(0) before
// every ds_read and drain the pipeline); completion is tracked explicitly
// with wait_vm before the barrier that publishes a stage.  M0 written by
// S_MOV needs one wait state before the LDS-DMA.
// a pointer every lane holds alike, as a scalar value (the divergence
// analysis cannot always prove it)
__device__ __forceinline__ const uint8_t* uniform_ptr(const void* p) {
  const unsigned long long v = (unsigned long long)(uintptr_t)p;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v), hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return (const uint8_t*)(uintptr_t)(((unsigned long long)hi << 32) | lo);
}

__device__ __forceinline__ void dma16(const void* src, uint32_t lds_addr) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(lds_addr)
               : "memory", "m0");
}

// wait until at most `after` stages (PW DMAs each) of this wave are in
// flight; after <= S
template <int PW, int S>
__device__ __forceinline__ void wait_stages(int after) {
  if constexpr (S <= 0) {
    wait_vm<0>();
  } else {
    if (after >= S)
      wait_vm<PW * S>();
    else
      wait_stages<PW, S - 1>(after);
  }
}

__device__ __forceinline__ void block_barrier() {
  // LDS reads of the previous stage are complete, then a plain s_barrier
  // (no release fence: it would wait for the DMA still in flight)
  __builtin_amdgcn_s_waitcnt((15) | (3 << 14) | (7 << 4) | (0 << 8));  // lgkmcnt(0)
  asm volatile("s_barrier" ::: "memory");
}

__device__ __forceinline__ bf16x8 frag(const bf16_t* tile, int row, int chunk) {
  return __builtin_bit_cast(bf16x8, *(const u32x4*)(tile + row * BK + ((chunk ^ (row & 7)) << 3)));
}

// Row-layout operands (X [K][M]: each k-row holds the M index contiguous)
// are staged as 64 k-rows x 64 columns sub-tiles; chunk c of k-row r sits at
// slot c ^ swt(r).
__device__ __forceinline__ int swt(int row) {
  // rows 4q .. 4q+3 (one transpose read's 16-lane group) take slot pairs
  // 0..3, and the 8-row block index XOR moves rows r and r + 8 (the groups
  // the LDS serves together) to complementary banks
  return (((row & 3) << 1) | ((row >> 2) & 1)) ^ (((row >> 3) & 3) << 1);
}
// MFMA fragment of the transposed sub-tile with ds_read_b64_tr_b16: lane
// (j, g) receives tile[row0 + 8g + 0..7][col0 + j].  Within a group of 16
// lanes the instruction hands lane i element (i & 3) of the 8 bytes that
// source lane 4e + (i >> 2) read as its e-th value, so source lane 4e + m
// reads k-row row0 + 8g + 4h + e at columns col0 + 4m .. +3 (h = 0, 1).
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
    const bf16_t* src = tile + row * BK + (((col >> 3) ^ swt(row)) << 3) + (col & 7);
    v[h] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(src));
  }
  const s16x8 w = __builtin_shufflevector(v[0], v[1], 0, 1, 2, 3, 4, 5, 6, 7);
  return __builtin_bit_cast(bf16x8, w);
}

__device__ __forceinline__ float sigm(float g) { return 1.f / (1.f + expf(-g)); }
// dG = dH*u*s*(1+g(1-s)), dU = dH*g*s with s = sigmoid(g)  (kernels.py:95-101)
__device__ __forceinline__ void swiglu_bwd1(float dh, float g, float u, float& dg, float& du) {
  const float sg = sigm(g);
  dg = dh * u * sg * (1.f + g * (1.f - sg));
  du = dh * g * sg;
}
__device__ __forceinline__ float bf_word(const u32x4& w, int e) {
  const uint32_t x = w[e >> 1];
  return __uint_as_float((e & 1) ? (x & 0xffff0000u) : (x << 16));
}
__device__ __forceinline__ float rnd(float v, int bf) { return bf ? round_bf(v) : v; }
__device__ __forceinline__ void put(void* c, long i, float v, int bf) {
  if (bf)
    ((bf16_t*)c)[i] = f2bf(v);
  else
    ((float*)c)[i] = v;
}
// 4 consecutive bf16 (transposed store of one lane's 4 rows)
__device__ __forceinline__ void put4(bf16_t* p, const float* v) {
  *(u32x2*)p = u32x2{pack2(f2bf(v[0]), f2bf(v[1])), pack2(f2bf(v[2]), f2bf(v[3]))};
}
__device__ __forceinline__ void put4_split(bf16_t* hi, bf16_t* lo, const float* v) {
  bf16_t h[4], l[4];
#pragma unroll
  for (int i = 0; i < 4; i++) split_bf(v[i], h[i], l[i]);
  *(u32x2*)hi = u32x2{pack2(h[0], h[1]), pack2(h[2], h[3])};
  *(u32x2*)lo = u32x2{pack2(l[0], l[1]), pack2(l[2], l[3])};
}

// Pipeline depth: two stages (double buffering).  Measured on gfx950: a
// workgroup's LDS footprint decides how many share a CU, and for the step's
// K (384..4096) a second resident workgroup hides more latency than deeper
// prefetch (64x128 tiles at K = 384: 28.3 -> 19.9 us; at K = 3072: 112 ->
// 84 us).  The LDS block is the larger of the two stages and the epilogue's
// staging tiles.
template <int BM, int BN, int PA, int PB, int EPI, int NS>
constexpr size_t lds_bytes() {
  constexpr int NBM = EPI == E_GATEUP ? 2 : 1;
  constexpr int NTILE = EPI == E_SWIGLU_BWD ? 4 : EPI == E_GATEUP ? 3 : EPI == E_PLANES ? 2 : 1;
  constexpr size_t pipe = (size_t)NS * (BM * PA + BN * PB * NBM) * BK * 2;
  constexpr size_t ep1 = (size_t)NTILE * BM * (BN + 8) * 2;
  constexpr size_t ep2 = (EPI == E_STORE || EPI == E_PARTIAL || EPI == E_SWIGLU_ROWS) ? (size_t)BM * (BN + 4) * 4 : 0;
  constexpr size_t e = ep1 > ep2 ? ep1 : ep2;
  return pipe > e ? pipe : e;
}

// TM: operand layouts.  Bit 0: A is given as X [K][M] (lda = its k-row
// stride), bit 1: B as Y [K][N]; C = X^T Y then (the dW form over rows of
// activations and gradients).  Otherwise operands are [rows][K] k-contiguous.
template <int BM, int BN, int PA, int PB, int EPI, int NS, int TM = 0>
__global__ __launch_bounds__(NT) void k_gemm_fast(FParams p) {
  constexpr bool TA = (TM & 1) != 0, TB = (TM & 2) != 0;
  static_assert(!(TA || TB) || ((EPI == E_STORE || EPI == E_PARTIAL) && BM % 64 == 0 && BN % 64 == 0),
                "row-layout operands: plain products with 64-multiple tiles");
  constexpr bool DUAL = EPI == E_GATEUP;
  constexpr int NBM = DUAL ? 2 : 1;
  constexpr int WM = BM / 2, WN = BN / 2, MB = WM / 16, NB = WN / 16;
  constexpr int AROWS = BM * PA, BROWS = BN * PB * NBM;
  constexpr int STAGE_ROWS = AROWS + BROWS;
  constexpr int BLOCKS8 = STAGE_ROWS / 8;       // DMA instructions per stage
  constexpr int PER_WAVE = BLOCKS8 / 4;
  static_assert(BLOCKS8 % 4 == 0, "tile rows must split evenly over the 4 waves");
  static_assert(PER_WAVE * (NS - 2) < 64, "outstanding DMA beyond vmcnt range");
  extern __shared__ __attribute__((aligned(16))) bf16_t lds[];  // NS * STAGE_ROWS * BK

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  // The kernel arguments the prologue reads, fetched together at entry and
  // held in SGPRs: loaded at their first uses, behind branches and address
  // arithmetic, they cost one dependent kernarg round trip each (about 6000
  // cycles before the first DMA).
  long pM = p.M, pN = p.N, pK = p.K, plda = p.lda, pkch = p.kchunk, sn1 = p.seg_n[1], sn2 = p.seg_n[2];
  int pxr = p.xcd_remap, pgm = p.gmode, pns = p.nseg, pgE = p.gE;
  const bf16_t *a0 = p.a[0], *a1 = p.a[1];
  const bf16_t *b00 = p.b[0][0], *b01 = p.b[0][1], *b02 = p.b[0][2], *b10 = p.b[1][0], *b11 = p.b[1][1],
               *b12 = p.b[1][2];
  long ldb0 = p.ldb[0], ldb1 = p.ldb[1], ldb2 = p.ldb[2], gsb = p.gstride_b, gsc = p.gstride_c;
  const int* goff = p.goff;
  unsigned nx = gridDim.x, ny = gridDim.y, nz = gridDim.z;
  asm volatile("" : "+s"(pM), "+s"(pN), "+s"(pK), "+s"(plda), "+s"(pkch), "+s"(sn1), "+s"(sn2), "+s"(pxr),
                    "+s"(pgm), "+s"(pns), "+s"(pgE));
  asm volatile("" : "+s"(a0), "+s"(a1), "+s"(b00), "+s"(b01), "+s"(b02), "+s"(b10), "+s"(b11), "+s"(b12));
  asm volatile("" : "+s"(ldb0), "+s"(ldb1), "+s"(ldb2), "+s"(gsb), "+s"(gsc), "+s"(goff), "+s"(nx), "+s"(ny),
                    "+s"(nz));
  unsigned long long mlo = p.mdiv_lo, mxy = p.mdiv_xy;
  asm volatile("" : "+s"(mlo), "+s"(mxy));
  auto fdiv = [](unsigned n, unsigned long long mg) { return (unsigned)(((unsigned long long)n * mg) >> 40); };
  // XCD-aware tile order: workgroups are dispatched round-robin over the 8
  // XCDs (linear id b -> XCD b % 8), each with its own L2.  Give XCD k a
  // contiguous run of the row-major tile order so the tiles that share A rows
  // (and split-K slices) meet in one L2.
  const unsigned nb = nx * ny * nz;
  const unsigned b = blockIdx.x + nx * (blockIdx.y + ny * blockIdx.z);
  unsigned logical = b;
  if (pxr) {
    const unsigned xcd = b & 7, local = b >> 3, q8 = nb >> 3, r8x = nb & 7;
    logical = xcd * q8 + (xcd < r8x ? xcd : r8x) + local;
  }
  // the smaller tile dimension varies fastest, so consecutive workgroups
  // (one XCD's run) share the operand of the larger one.  When B's column
  // panels together exceed an XCD's L2 (cfg5 gate/up: 43 panels, 11 MB),
  // that order streams every B panel from beyond the L2 once per row panel;
  // grouped order instead walks `group` row panels down one column before
  // the next column, so each B panel is read once per group and reused from
  // L2 (cfg5 gate/up forward 272 -> 236 us, step 34.9 -> 34.0 ms).
  unsigned tx, ty;
  const unsigned tz = fdiv(logical, mxy), in = logical - tz * nx * ny;  // index inside one K slice
  const unsigned pgrp = (unsigned)p.group;
  if (pgrp > 0) {
    const unsigned ning = pgrp * nx, gid = in / ning, first = gid * pgrp;
    const unsigned gs = ny - first < pgrp ? ny - first : pgrp;
    const unsigned loc = in - gid * ning;
    ty = first + loc % gs;
    tx = loc / gs;
  } else if (ny < nx) {
    ty = in - fdiv(in, mlo) * ny;
    tx = fdiv(in, mlo);
  } else {
    tx = in - fdiv(in, mlo) * nx;
    ty = fdiv(in, mlo);
  }
  const long m0 = (long)ty * BM, n0 = (long)tx * BN;
  int ge = 0;
  if (pgm == 1) {
    if (m0 >= goff[pgE]) return;  // beyond the last expert segment: the whole workgroup leaves
    while (ge + 1 < pgE && m0 >= goff[ge + 1]) ge++;
  } else if (pgm == 2) {
    ge = (int)tz;
  }
  const long boff = pgm == 1 ? (long)ge * gsb : 0;
  const long coff = pgm == 2 ? (long)ge * gsc : 0;
  int seg = 0;
#pragma unroll
  for (int s = 1; s < 3; s++)
    if (s < pns && n0 >= (s == 1 ? sn1 : sn2)) seg = s;
  const long seg0 = seg == 0 ? 0 : seg == 1 ? sn1 : sn2;
  const long nl0 = n0 - seg0;
  const long seg_end = (seg + 1 < pns) ? (seg == 0 ? sn1 : sn2) : pN;
  const long nrows_b = seg_end - seg0;

  long kbeg = 0, kend = pK;
  if (pgm == 2) {
    kbeg = goff[ge];
    kend = goff[ge + 1];
  } else if (EPI == E_PARTIAL) {
    kbeg = (long)tz * pkch;
    kend = kbeg + pkch < pK ? kbeg + pkch : pK;
  }
  const int nk = (int)((kend - kbeg + BK - 1) / BK);

  // Per-lane DMA sources of this wave's PER_WAVE 8-row blocks (fixed over
  // k): block j covers stage rows 8*(wave + 4j).  Row r of a block holds
  // 16-byte chunk c = (s & 7) ^ (r & 7) at slot s; since every block starts
  // at a multiple of 8, r & 7 = s >> 3 and c depends on the lane only.
  const int wave_s = __builtin_amdgcn_readfirstlane(wave);
  const int sl = lane;
  const int c8 = (((sl & 7) ^ (sl >> 3)) << 3);
  // Row-layout blocks (TM): stage rows r8 .. r8 + 7 of a plane are k-rows
  // (r8 % 64) + 0..7 of its sub-tile (r8 % BM) / 64, i.e. columns
  // 64 * subtile .. + 63 of X; the lane loads source chunk
  // (sl & 7) ^ swt(k-row) of k-row (r8 % 64) + (sl >> 3).
  // kpos[j]: the lane's largest k offset in the block (valid iff
  // kbeg + k0 + kpos < kend); kmul[j]: source elements per k step.
  // Lanes outside the operand read `zero` (kmul 0 keeps them there).  Its
  // address is held in registers: the DMA asm's memory clobber would
  // otherwise make the compiler reload it from the GOT, with an lgkmcnt(0)
  // wait, before every issue.
  const bf16_t* zero = (const bf16_t*)g_zero16;
  asm volatile("" : "+s"(zero));
  // Every block's DMA takes a uniform base (its operand at the tile's first
  // row or column and the K slice's first k, advanced a stage at a time by
  // scalar arithmetic) plus a fixed 32-bit byte offset per lane.  A row or
  // column past the operand reads its last one (rows) or last chunk
  // (columns) instead: it feeds only outputs that are never stored.  Tokens
  // past the K range (the last stage of a ragged K) read `zero`.
  const uint8_t* bj[PER_WAVE];
  uint32_t voff[PER_WAVE];
  long kstr[PER_WAVE];  // bytes per stage
  int kpos[PER_WAVE];
  // Block j of every wave starts at stage row 32 j + 8 wave: with AROWS,
  // BM and BN multiples of 32, whether it holds A or B, and which plane and
  // (gate/up) half, follow from j alone, so the unrolled setup has no
  // per-wave branches.
  static_assert(AROWS % 32 == 0 && BM % 32 == 0 && BN % 32 == 0, "block-to-operand map");
#pragma unroll
  for (int j = 0; j < PER_WAVE; j++) {
    // stage row 8 wave + 32 j: its offset inside a plane is 8 wave + c32
    // with c32 = (32 j) % plane rows (8 wave < 32 never carries), so every
    // per-block term below but 8 wave is a compile-time constant
    const bf16_t* base;
    long ld, row0, rows;
    bool tr;
    int c32;
    if (32 * j < AROWS) {
      const int pl = (32 * j) / BM;
      c32 = (32 * j) % BM;
      base = pl ? a1 : a0;
      ld = plda;
      tr = TA;
      row0 = m0;
      rows = pM;
    } else {
      const int rb32 = 32 * j - AROWS;
      const int q = rb32 / (BN * PB), pl = (rb32 % (BN * PB)) / BN;
      c32 = rb32 % BN;
      const int sg = DUAL ? q : seg;
      base = (pl ? (sg == 0 ? b10 : sg == 1 ? b11 : b12) : (sg == 0 ? b00 : sg == 1 ? b01 : b02)) + boff;
      ld = sg == 0 ? ldb0 : sg == 1 ? ldb1 : ldb2;
      tr = TB;
      row0 = nl0;
      rows = nrows_b;
    }
    if (tr) {
      const int kr = wave_s * 8 + c32 % 64 + (sl >> 3);
      long col = row0 + (c32 / 64) * 64 + 8 * ((sl & 7) ^ swt(kr));
      col = col < rows ? col : rows - 8;
      bj[j] = uniform_ptr(base + kbeg * ld + row0);
      voff[j] = (uint32_t)((kr * ld + (col - row0)) * 2);
      kstr[j] = (long)BK * ld * 2;
      kpos[j] = kr;
    } else {
      long row = row0 + wave_s * 8 + c32 + (sl >> 3);
      row = row < rows ? row : rows - 1;
      bj[j] = uniform_ptr(base + row0 * ld + kbeg);
      voff[j] = (uint32_t)(((row - row0) * ld + c8) * 2);
      kstr[j] = (long)BK * 2;
      kpos[j] = c8 + 7;
    }
  }
  const uint32_t lds_base = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_void*)lds);
  const long klen = kend - kbeg;
  // this wave's share of stage `it` into buffer `buf`
  auto issue = [&](int it, int buf) {
    const long k0 = (long)it * BK;  // relative to kbeg
    const uint32_t sbase = lds_base + (uint32_t)(buf * STAGE_ROWS * BK * 2) + (uint32_t)(wave_s * 8 * BK * 2);
    if (k0 + BK <= klen) {  // uniform: every lane's k offset is in range
#pragma unroll
      for (int j = 0; j < PER_WAVE; j++)
        asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1 offset:0" ::"v"(voff[j]),
                     "s"(bj[j] + it * kstr[j]), "s"(sbase + (uint32_t)(j * 32 * BK * 2))
                     : "memory", "m0");
    } else {
#pragma unroll
      for (int j = 0; j < PER_WAVE; j++) {
        const bool kin = k0 + kpos[j] < klen;
        dma16(kin ? (const void*)(bj[j] + it * kstr[j] + voff[j]) : (const void*)zero,
              sbase + (uint32_t)(j * 32 * BK * 2));
      }
    }
  };

  f32x4 acc[NBM][MB][NB];
#pragma unroll
  for (int q = 0; q < NBM; q++)
#pragma unroll
    for (int i = 0; i < MB; i++)
#pragma unroll
      for (int j = 0; j < NB; j++) acc[q][i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  // E_SWIGLU_ROWS: this thread's phase-2 chunks of G and U (8 columns of one
  // tile row each), loaded now so their latency hides under the main loop
  constexpr bool SROWS = EPI == E_SWIGLU_ROWS;
  constexpr int CPR8 = BN / 8, NCH = SROWS ? (BM * CPR8 + NT - 1) / NT : 1;
  u32x4 gpre[NCH], upre[NCH];
  if constexpr (SROWS) {
#pragma unroll
    for (int i = 0; i < NCH; i++) {
      const int q = threadIdx.x + i * NT;
      const long m = m0 + q / CPR8, n = n0 + (q % CPR8) * 8;
      gpre[i] = upre[i] = u32x4{0u, 0u, 0u, 0u};
      if (q < BM * CPR8 && m < pM && n + 8 <= pN) {
        gpre[i] = *(const u32x4*)(p.gin + m * p.ldgu + n);
        upre[i] = *(const u32x4*)(p.uin + m * p.ldgu + n);
      }
    }
  }

  const int fr = lane & 15, fg = lane >> 4;
#pragma unroll
  for (int s = 0; s < NS - 1; s++)
    if (s < nk) issue(s, s);
  for (int it = 0; it < nk; it++) {
    // wait for this wave's DMA of stage `it`; the stages issued after it
    // (up to NS - 2) may stay in flight
    const int after = (nk - 1 - it) < (NS - 2) ? (nk - 1 - it) : (NS - 2);
    wait_stages<PER_WAVE, NS - 2>(after);
    block_barrier();
    if (it + NS - 1 < nk) issue(it + NS - 1, (it + NS - 1) % NS);
    const bf16_t* st = lds + (it % NS) * STAGE_ROWS * BK;
#pragma unroll
    for (int h = 0; h < 2; h++) {
      const int ch = 4 * h + fg;
      bf16x8 ah[MB], al[MB];
#pragma unroll
      for (int i = 0; i < MB; i++) {
        const int row = wm * WM + i * 16 + fr;
        if constexpr (TA) {
          const int r16 = wm * WM + i * 16;
          const bf16_t* sub = st + (r16 / 64) * 64 * BK;
          ah[i] = tr_frag(sub, 32 * h, r16 % 64, lane);
          if constexpr (PA == 2) al[i] = tr_frag(sub + BM * BK, 32 * h, r16 % 64, lane);
        } else {
          ah[i] = frag(st, row, ch);
          if constexpr (PA == 2) al[i] = frag(st + BM * BK, row, ch);
        }
      }
#pragma unroll
      for (int q = 0; q < NBM; q++) {
        const bf16_t* bt = st + (AROWS + q * BN * PB) * BK;
#pragma unroll
        for (int j = 0; j < NB; j++) {
          const int row = wn * WN + j * 16 + fr;
          bf16x8 bh, bl;
          if constexpr (TB) {
            const int r16 = wn * WN + j * 16;
            const bf16_t* sub = bt + (r16 / 64) * 64 * BK;
            bh = tr_frag(sub, 32 * h, r16 % 64, lane);
            if constexpr (PB == 2) bl = tr_frag(sub + BN * BK, 32 * h, r16 % 64, lane);
          } else {
            bh = frag(bt, row, ch);
            if constexpr (PB == 2) bl = frag(bt + BN * BK, row, ch);
          }
#pragma unroll
          for (int i = 0; i < MB; i++) {
            acc[q][i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah[i], bh, acc[q][i][j], 0, 0, 0);
            if constexpr (PB == 2) acc[q][i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah[i], bl, acc[q][i][j], 0, 0, 0);
            if constexpr (PA == 2) acc[q][i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al[i], bh, acc[q][i][j], 0, 0, 0);
          }
        }
      }
    }
  }

  // ------------------------------------------------------------ epilogue
  // acc[q][i][j][r] = C[m0 + wm*WM + 16i + 4*(lane/16) + r][n0 + wn*WN + 16j + lane%16].
  // Phase 1: every lane applies the epilogue math to its values and leaves
  // the results in LDS tiles (the pipeline buffers are free now).  Phase 2:
  // the block writes each tile out in 16-byte chunks along rows (normal
  // outputs) or along columns (transposed outputs), so every global store
  // is a full vector and neighbouring lanes fill whole lines.
  block_barrier();  // every wave has finished reading the last stage
  constexpr int TLD = BN + 8;          // bf16 tile row stride (elements)
  constexpr int TP = BM * TLD;         // bf16 tile size (elements)
  constexpr int TLDF = BN + 4;         // fp32 tile row stride
  constexpr int NTILE = EPI == E_SWIGLU_BWD ? 4 : EPI == E_GATEUP ? 3 : EPI == E_PLANES ? 2 : 1;
  constexpr bool F32T = EPI == E_PARTIAL || EPI == E_STORE || SROWS;  // fp32 tile unless c_bf16
  static_assert((size_t)NTILE * TP * 2 <= lds_bytes<BM, BN, PA, PB, EPI, NS>(), "epilogue tiles exceed LDS");
  static_assert(!F32T || (size_t)BM * TLDF * 4 <= lds_bytes<BM, BN, PA, PB, EPI, NS>(), "epilogue tile exceeds LDS");
  bf16_t* T = lds;
  float* TF = (float*)lds;
  const bool f32out = F32T && (SROWS || !p.c_bf16);
  const int cc = lane & 15;
#pragma unroll
  for (int i = 0; i < MB; i++) {
    const int rl = wm * WM + i * 16 + fg * 4;  // tile row of this lane's first value
    const long mb = m0 + rl;
#pragma unroll
    for (int j = 0; j < NB; j++) {
      const int cl = wn * WN + j * 16 + cc;
      const long ncol = n0 + cl;
      const long nloc = ncol - seg0;
      const bool colok = ncol < pN;
      float v[4] = {acc[0][i][j][0], acc[0][i][j][1], acc[0][i][j][2], acc[0][i][j][3]};
      if constexpr (EPI == E_SWIGLU_BWD) {
        // v = dH; dG = dH*u*s*(1+g(1-s)), dU = dH*g*s  (kernels.py:95-101)
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const long m = mb + r;
          float g = 0.f, u = 0.f;
          if (m < pM && colok) {
            g = bf2f(p.gin[m * p.ldgu + ncol]);
            u = bf2f(p.uin[m * p.ldgu + ncol]);
          }
          float dg, du;
          swiglu_bwd1(v[r], g, u, dg, du);
          bf16_t h, l;
          split_bf(dg, h, l);
          T[(rl + r) * TLD + cl] = h;
          T[TP + (rl + r) * TLD + cl] = l;
          split_bf(du, h, l);
          T[2 * TP + (rl + r) * TLD + cl] = h;
          T[3 * TP + (rl + r) * TLD + cl] = l;
        }
      } else if constexpr (EPI == E_GATEUP) {
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const float g = round_bf(v[r]);
          const float u = round_bf(acc[1][i][j][r]);
          T[(rl + r) * TLD + cl] = f2bf(g);
          T[TP + (rl + r) * TLD + cl] = f2bf(u);
          T[2 * TP + (rl + r) * TLD + cl] = f2bf(g * sigm(g) * u);
        }
      } else if constexpr (EPI == E_PLANES) {
#pragma unroll
        for (int r = 0; r < 4; r++) {
          bf16_t h, l;
          split_bf(v[r], h, l);
          T[(rl + r) * TLD + cl] = h;
          T[TP + (rl + r) * TLD + cl] = l;
        }
      } else if constexpr (EPI == E_QKV) {
#pragma unroll
        for (int r = 0; r < 4; r++) T[(rl + r) * TLD + cl] = f2bf(v[r]);  // RoPE is applied in phase 2
      } else if constexpr (EPI == E_RESID) {
#pragma unroll
        for (int r = 0; r < 4; r++) T[(rl + r) * TLD + cl] = f2bf(v[r]);  // round_bf(v), added in phase 2
      } else {  // E_STORE / E_PARTIAL
        if (f32out) {
#pragma unroll
          for (int r = 0; r < 4; r++) TF[(rl + r) * TLDF + cl] = v[r];
        } else {
#pragma unroll
          for (int r = 0; r < 4; r++) T[(rl + r) * TLD + cl] = f2bf(v[r]);
        }
      }
    }
  }
  __syncthreads();

  // ---- phase 2
  const int tid = threadIdx.x;
  // rows: 8 bf16 of tile row r, cols c8..c8+7 -> dst row m, col n
  auto rows_bf16 = [&](const bf16_t* t, auto dst_of) {
    constexpr int CPR = BN / 8;
    for (int q = tid; q < BM * CPR; q += NT) {
      const int r = q / CPR, c8 = (q % CPR) * 8;
      const long m = m0 + r, n = n0 + c8;
      if (m >= pM || n >= pN) continue;
      const u32x4 val = *(const u32x4*)(t + r * TLD + c8);
      dst_of(m, n, val, t + r * TLD + c8);
    }
  };
  // columns: 8 rows of tile column c -> transposed dst[n][m..m+7]
  auto cols_bf16 = [&](const bf16_t* t, bf16_t* dst, long ldt) {
    constexpr int RPC = BM / 8;
    for (int q = tid; q < BN * RPC; q += NT) {
      const int c = q / RPC, r8 = (q % RPC) * 8;
      const long n = n0 + c, m = m0 + r8;
      if (n >= pN || m >= pM) continue;
      bf16_t v8[8];
#pragma unroll
      for (int i = 0; i < 8; i++) v8[i] = t[(r8 + i) * TLD + c];
      bf16_t* d = dst + n * ldt + m;
      if (m + 8 <= pM && (((uintptr_t)d & 15) == 0)) {
        *(u32x4*)d = u32x4{pack2(v8[0], v8[1]), pack2(v8[2], v8[3]), pack2(v8[4], v8[5]), pack2(v8[6], v8[7])};
      } else {
        for (int i = 0; i < 8; i++)
          if (m + i < pM) d[i] = v8[i];
      }
    }
  };
  // plain bf16 store of a chunk at d (8 values, n..n+7 of a row)
  auto put8 = [&](bf16_t* d, long n, const u32x4& val, const bf16_t* src) {
    if (n + 8 <= pN && (((uintptr_t)d & 15) == 0)) {
      *(u32x4*)d = val;
    } else {
      for (int i = 0; i < 8; i++)
        if (n + i < pN) d[i] = src[i];
    }
  };

  if constexpr (EPI == E_SWIGLU_BWD) {
    bf16_t* c0 = (bf16_t*)p.c[0];
    bf16_t* c1 = (bf16_t*)p.c[1];
#pragma unroll
    for (int t4 = 0; t4 < 4; t4++) {
      bf16_t* base = (t4 & 1) ? c1 : c0;
      const long coloff = (t4 >> 1) ? p.F : 0;
      rows_bf16(T + t4 * TP, [&](long m, long n, const u32x4& val, const bf16_t* src) {
        put8(base + m * p.ldc[0] + coloff + n, n, val, src);
      });
      bf16_t* tb = (t4 & 1) ? (bf16_t*)p.c[3] : (bf16_t*)p.c[2];
      if (tb) cols_bf16(T + t4 * TP, tb + coloff * p.ldc[2], p.ldc[2]);
    }
  } else if constexpr (SROWS) {
    bf16_t* c0 = (bf16_t*)p.c[0];
    bf16_t* c1 = (bf16_t*)p.c[1];
#pragma unroll
    for (int i = 0; i < NCH; i++) {
      const int q = tid + i * NT;
      const int r = q / CPR8, c8 = (q % CPR8) * 8;
      const long m = m0 + r, n = n0 + c8;
      if (q >= BM * CPR8 || m >= pM || n + 8 > pN) continue;
      const float4 d0 = *(const float4*)(TF + r * TLDF + c8);
      const float4 d1 = *(const float4*)(TF + r * TLDF + c8 + 4);
      const float dh[8] = {d0.x, d0.y, d0.z, d0.w, d1.x, d1.y, d1.z, d1.w};
      bf16_t gh[8], gl[8], uh[8], ul[8];
#pragma unroll
      for (int e = 0; e < 8; e++) {
        float dg, du;
        swiglu_bwd1(dh[e], bf_word(gpre[i], e), bf_word(upre[i], e), dg, du);
        split_bf(dg, gh[e], gl[e]);
        split_bf(du, uh[e], ul[e]);
      }
      const long o = m * p.ldc[0] + n;
      *(u32x4*)(c0 + o) = u32x4{pack2(gh[0], gh[1]), pack2(gh[2], gh[3]), pack2(gh[4], gh[5]), pack2(gh[6], gh[7])};
      *(u32x4*)(c1 + o) = u32x4{pack2(gl[0], gl[1]), pack2(gl[2], gl[3]), pack2(gl[4], gl[5]), pack2(gl[6], gl[7])};
      *(u32x4*)(c0 + o + p.F) =
          u32x4{pack2(uh[0], uh[1]), pack2(uh[2], uh[3]), pack2(uh[4], uh[5]), pack2(uh[6], uh[7])};
      *(u32x4*)(c1 + o + p.F) =
          u32x4{pack2(ul[0], ul[1]), pack2(ul[2], ul[3]), pack2(ul[4], ul[5]), pack2(ul[6], ul[7])};
    }
  } else if constexpr (EPI == E_PLANES) {
#pragma unroll
    for (int t2 = 0; t2 < 2; t2++) {
      bf16_t* base = (bf16_t*)p.c[t2];
      rows_bf16(T + t2 * TP, [&](long m, long n, const u32x4& val, const bf16_t* src) {
        put8(base + m * p.ldc[0] + n, n, val, src);
      });
      if (p.c[2 + t2]) cols_bf16(T + t2 * TP, (bf16_t*)p.c[2 + t2], p.ldc[2]);
    }
    if (p.delta) {
      // Delta[h][m] = sum (hi + lo) * o over head h's columns (n0 and BN are
      // multiples of 64): four lanes per (row, head), 16 columns each, then
      // (l0 + l1) + (l2 + l3) -- the order of the standalone Delta pass
      constexpr int NH = BN / 64;
      for (int q = threadIdx.x; q < BM * NH * 4; q += NT) {
        const int g = q & 3, rh = q >> 2, r = rh / NH, hc = rh % NH;
        const long m = m0 + r, col0 = n0 + 64 * hc;
        const bool ok = m < pM && col0 < pN;
        float dpart = 0.f;
        if (ok) {
#pragma unroll
          for (int c = 0; c < 2; c++) {
            const int cl = 64 * hc + 32 * c + 8 * g;
            const u32x4 hv = *(const u32x4*)(T + r * TLD + cl);
            const u32x4 lv = *(const u32x4*)(T + TP + r * TLD + cl);
            const u32x4 ov = *(const u32x4*)(p.o + m * p.ldo + col0 + 32 * c + 8 * g);
#pragma unroll
            for (int i = 0; i < 4; i++) {
              dpart += (__uint_as_float(hv[i] << 16) + __uint_as_float(lv[i] << 16)) * __uint_as_float(ov[i] << 16);
              dpart += (__uint_as_float(hv[i] & 0xffff0000u) + __uint_as_float(lv[i] & 0xffff0000u)) *
                       __uint_as_float(ov[i] & 0xffff0000u);
            }
          }
        }
        dpart += __shfl_xor(dpart, 1, 64);
        dpart += __shfl_xor(dpart, 2, 64);
        if (ok && g == 0) p.delta[(col0 / 64) * p.lddelta + m] = dpart;
      }
    }
  } else if constexpr (EPI == E_GATEUP) {
#pragma unroll
    for (int t3 = 0; t3 < 3; t3++) {
      bf16_t* base = (bf16_t*)p.c[t3];
      rows_bf16(T + t3 * TP, [&](long m, long n, const u32x4& val, const bf16_t* src) {
        put8(base + m * p.ldc[0] + n, n, val, src);
      });
    }
    if (p.c[3]) cols_bf16(T + 2 * TP, (bf16_t*)p.c[3], p.ldc[3]);
  } else if constexpr (EPI == E_QKV) {
    // RoPE on the stored (bf16-rounded) q and k values: pairs (2i, 2i+1) of
    // a chunk rotate by the angle of (token position, pair index), cos/sin
    // read from the table as one run per chunk (kernels.py:103-113)
    const int T32 = (int)p.rope_t, hd = (int)p.head_dim;
    rows_bf16(T, [&](long m, long n, const u32x4& val, const bf16_t* src) {
      int sg = 0;
      for (int s2 = 1; s2 < 3; s2++)
        if (s2 < pns && n >= (s2 == 1 ? sn1 : sn2)) sg = s2;
      const long nl = n - (sg == 0 ? 0 : sg == 1 ? sn1 : sn2);
      u32x4 o = val;
      bf16_t rot[8];
      if (n < p.rope_cols) {
        const int pos = (int)((unsigned)m % (unsigned)T32);
#pragma unroll
        for (int k = 0; k < 4; k++) {
          const int pair = ((int)(nl + 2 * k) % hd) >> 1;
          const float2 cs = *(const float2*)(p.rope + 2 * (pos * (hd >> 1) + pair));
          const float a = bf2f((bf16_t)(val[k] & 0xffffu)), b = bf2f((bf16_t)(val[k] >> 16));
          rot[2 * k] = f2bf(a * cs.x - b * cs.y);
          rot[2 * k + 1] = f2bf(b * cs.x + a * cs.y);
          o[k] = pack2(rot[2 * k], rot[2 * k + 1]);
        }
        if (p.c[3]) *(u32x4*)const_cast<bf16_t*>(src) = o;  // the rotated chunk feeds the transposed copy
      } else {
#pragma unroll
        for (int k = 0; k < 8; k++) rot[k] = src[k];
      }
      put8((bf16_t*)p.c[sg] + m * p.ldc[sg] + nl, n, o, rot);
    });
    if (p.c[3]) {  // q|k|v transposed [N][ldc[3]] (the attention kernels' Q^T, K^T, V^T tiles)
      __syncthreads();
      cols_bf16(T, (bf16_t*)p.c[3], p.ldc[3]);
    }
  } else if constexpr (EPI == E_RESID) {
    rows_bf16(T, [&](long m, long n, const u32x4& val, const bf16_t* src) {
      const bf16_t* rr = p.r + m * p.ldr + n;
      bf16_t* d = (bf16_t*)p.c[0] + m * p.ldc[0] + n;
      if (n + 8 <= pN && (((uintptr_t)d & 15) == 0) && (((uintptr_t)rr & 15) == 0)) {
        const u32x4 rv = *(const u32x4*)rr;
        u32x4 o;
#pragma unroll
        for (int k = 0; k < 4; k++) {
          const float a0 = bf2f((bf16_t)(rv[k] & 0xffffu)) + bf2f((bf16_t)(val[k] & 0xffffu));
          const float a1 = bf2f((bf16_t)(rv[k] >> 16)) + bf2f((bf16_t)(val[k] >> 16));
          o[k] = pack2(f2bf(a0), f2bf(a1));
        }
        *(u32x4*)d = o;
      } else {
        for (int i = 0; i < 8; i++)
          if (n + i < pN) d[i] = f2bf(bf2f(rr[i]) + bf2f(src[i]));
      }
    });
  } else {  // E_STORE / E_PARTIAL
    if (!f32out) {
      rows_bf16(T, [&](long m, long n, const u32x4& val, const bf16_t* src) {
        put8((bf16_t*)p.c[0] + coff + m * p.ldc[0] + n, n, val, src);
      });
    } else {
      constexpr int CPR = BN / 4;
      float* dst0 = EPI == E_PARTIAL ? p.partial + (long)tz * pM * pN : (float*)p.c[0] + coff;
      const long ldd = EPI == E_PARTIAL ? pN : p.ldc[0];
      const bool acc_out = EPI == E_STORE && p.accumulate;
      for (int q = tid; q < BM * CPR; q += NT) {
        const int r = q / CPR, c4 = (q % CPR) * 4;
        const long m = m0 + r, n = n0 + c4;
        if (m >= pM || n >= pN) continue;
        const float4 val = *(const float4*)(TF + r * TLDF + c4);
        float* d = dst0 + m * ldd + n;
        if (n + 4 <= pN && (((uintptr_t)d & 15) == 0)) {
          if (acc_out) {
            const float4 o = *(const float4*)d;
            *(float4*)d = make_float4(o.x + val.x, o.y + val.y, o.z + val.z, o.w + val.w);
          } else {
            *(float4*)d = val;
          }
        } else {
          const float vv[4] = {val.x, val.y, val.z, val.w};
          for (int k = 0; k < 4; k++)
            if (n + k < pN) d[k] = acc_out ? d[k] + vv[k] : vv[k];
        }
      }
    }
  }
}

// ------------------------------------------------------- token-split dW
// C = X^T Y for row-layout operands (X [K][M] one bf16 plane, Y [K][N] as PB
// planes): the weight gradient contracted over token rows.  In the k_gemm_fast
// form both operands reach the MFMA through LDS transpose reads, which the
// LDS serves at half the rate of ordinary reads, and with a 32x32 tile per
// wave the LDS port (DMA writes plus fragment reads) bounds a k-step at about
// four times its MFMA time.  Here every wave owns the whole 64x64 tile: the
// four waves take interleaved 32-token slices of the workgroup's K range
// (wave w: tokens 128 s + 32 w .. + 31 at step s), so each fragment read
// feeds twice the MFMAs.  A wave stages only its own slices, in its own LDS
// region, and waits only for its own DMA: the main loop has no workgroup
// barrier.  The four partial tiles are added in LDS in wave order,
// ((w0 + w1) + w2) + w3, so the result does not depend on timing.
constexpr int KW_ROWS = 32;                  // tokens per wave step
constexpr int KW_SUB = KW_ROWS * 64;         // elements of one 32 x 64 sub-tile
constexpr int KW_TLD = 64 + 4;               // fp32 reduction tile row stride

template <int PB, int NS>
constexpr size_t kw_lds_bytes() {
  constexpr size_t pipe = (size_t)4 * NS * (1 + PB) * KW_SUB * 2;
  constexpr size_t red = (size_t)4 * 64 * KW_TLD * 4;
  return pipe > red ? pipe : red;
}

template <int PB, int EPI, int NS>
__global__ __launch_bounds__(NT) void k_gemm_kw(FParams p) {
  static_assert(EPI == E_STORE || EPI == E_PARTIAL, "plain products only");
  constexpr int NSUB = 1 + PB;              // sub-tiles per stage: X, then the Y planes
  constexpr int STAGE = NSUB * KW_SUB;      // elements of one wave stage
  constexpr int PER = NSUB * 4;             // DMAs per wave stage (8 token rows each)
  static_assert(PER * NS < 64, "outstanding DMA beyond vmcnt range");
  static_assert(NS == 2, "two buffers");
  extern __shared__ __attribute__((aligned(16))) bf16_t lds[];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // kernel arguments fetched together at entry and held in SGPRs
  long pM = p.M, pN = p.N, pK = p.K, ldx = p.lda, ldy = p.ldb[0], pkch = p.kchunk;
  const bf16_t *x0 = p.a[0], *y0 = p.b[0][0], *y1 = p.b[1][0];
  int pxr = p.xcd_remap;
  unsigned nx = gridDim.x, ny = gridDim.y, nz = gridDim.z;
  unsigned long long mlo = p.mdiv_lo, mxy = p.mdiv_xy;
  asm volatile("" : "+s"(pM), "+s"(pN), "+s"(pK), "+s"(ldx), "+s"(ldy), "+s"(pkch), "+s"(pxr));
  asm volatile("" : "+s"(x0), "+s"(y0), "+s"(y1), "+s"(nx), "+s"(ny), "+s"(nz), "+s"(mlo), "+s"(mxy));
  auto fdiv = [](unsigned n, unsigned long long mg) { return (unsigned)(((unsigned long long)n * mg) >> 40); };
  // tile order as in k_gemm_fast: a contiguous run of the tile order per XCD,
  // the smaller tile dimension fastest
  const unsigned nb = nx * ny * nz;
  const unsigned b = blockIdx.x + nx * (blockIdx.y + ny * blockIdx.z);
  unsigned logical = b;
  if (pxr) {
    const unsigned xcd = b & 7, local = b >> 3, q8 = nb >> 3, r8x = nb & 7;
    logical = xcd * q8 + (xcd < r8x ? xcd : r8x) + local;
  }
  unsigned tx, ty;
  const unsigned tz = fdiv(logical, mxy), in = logical - tz * nx * ny;
  if (ny < nx) {
    ty = in - fdiv(in, mlo) * ny;
    tx = fdiv(in, mlo);
  } else {
    tx = in - fdiv(in, mlo) * nx;
    ty = fdiv(in, mlo);
  }
  const long m0 = (long)ty * 64, n0 = (long)tx * 64;
  long kbeg = 0, kend = pK;
  if constexpr (EPI == E_PARTIAL) {
    kbeg = (long)tz * pkch;
    kend = kbeg + pkch < pK ? kbeg + pkch : pK;
  }
  const long klen = kend - kbeg;
  const int nsw = (int)(klen / (4 * KW_ROWS));  // steps of every wave (klen is a multiple of 256)

  // DMA sources.  Block j (8 token rows) is rows 8 (j % 4) .. + 7 of
  // sub-tile j / 4 (0: X, 1: Y hi, 2: Y lo).  Chunk c of k-row r of a
  // sub-tile sits at slot c ^ swt(r) (the transpose-read swizzle), so the
  // lane writing slot lane % 8 of k-row kr fetches chunk (lane % 8) ^ swt(kr).
  // A column past the operand's last (M or N a multiple of 8, not of 64)
  // reads the last chunk instead: it feeds only outputs of rows or columns
  // that are never stored.  Every slice is an even number of steps (K and
  // the slice length are multiples of 256), so no token check is needed.
  // The DMA takes a uniform base (the step's first token row of the
  // operand, advanced by scalar arithmetic) plus a fixed 32-bit byte offset
  // per lane and block: no vector address arithmetic in the loop.
  uint32_t voff[PER];
#pragma unroll
  for (int j = 0; j < PER; j++) {
    const int sub = j / 4;
    const int kr = KW_ROWS * wave + 8 * (j % 4) + (lane >> 3);
    const long ld = sub == 0 ? ldx : ldy;
    const long cols = sub == 0 ? pM : pN;
    long col = (sub == 0 ? m0 : n0) + 8 * ((lane & 7) ^ swt(kr & 31));
    col = col < cols ? col : cols - 8;
    voff[j] = (uint32_t)((kr * ld + col) * 2);
  }
  const uint32_t lds_wave =
      __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_void*)lds) + (uint32_t)(wave * NS * STAGE * 2);
  // step `it` (a step past the wave's last reloads the last one into a
  // buffer no step reads) into buffer `buf`, blocks [j0, j1)
  auto issue = [&](int it, int buf, int j0, int j1) {
    const long st = (long)(it < nsw ? it : nsw - 1) * 4 * KW_ROWS + kbeg;  // first token row of the step
    const uint8_t* bx = (const uint8_t*)(x0 + st * ldx);
    const uint8_t* by0 = (const uint8_t*)(y0 + st * ldy);
    const uint8_t* by1 = (const uint8_t*)(y1 + st * ldy);
    const uint32_t sb = lds_wave + (uint32_t)(buf * STAGE * 2);
#pragma unroll
    for (int j = j0; j < j1; j++) {
      const uint8_t* bs = j < 4 ? bx : j < 8 ? by0 : by1;
      asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1 offset:0" ::"v"(voff[j]), "s"(bs),
                   "s"(sb + (uint32_t)(j * 1024))
                   : "memory", "m0");
    }
  };

  f32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 4; j++) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  // fragment f of a step: 0..3 the X columns 16f.., 4..7 the Y hi columns
  // 16 (f - 4).., 8..11 the Y lo columns
  constexpr int NF = 4 + 4 * PB;
  auto load_frag = [&](int buf, int f, bf16x8* fr) {
    const bf16_t* st = lds + (wave * NS + buf) * STAGE;
    fr[f] = tr_frag(st + (f / 4) * KW_SUB, 0, 16 * (f % 4), lane);
  };
  // MFMA q of a step: half q / (NQ / 2) covers column blocks 2 half, + 1;
  // an accumulator's hi- and lo-plane products are adjacent
  constexpr int NQ = 16 * PB;
  auto mfma_q = [&](int q, const bf16x8* fr) {
    const int r = q % (NQ / 2), pl = r % PB, j = 2 * (q / (NQ / 2)) + (r / (4 * PB)) % 2, i = (r / PB) % 4;
    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fr[i], fr[4 + 4 * pl + j], acc[i][j], 0, 0, 0);
  };

  // Software pipeline, two buffers, two steps in flight.  A step's
  // fragments are read into registers during the previous step, so its
  // buffer is free when the step starts and step it + 2 is loaded into it,
  // its DMA blocks between the first half of step it's MFMAs; step it + 1's
  // transpose reads go between the second half.  The loop is unrolled by
  // two, so buffers and fragment register sets alternate at compile time.
  static_assert(NS == 2, "two buffers");
  bf16x8 fa[NF], fb[NF];
  auto body = [&](int it, bf16x8* cur, bf16x8* nxt, int bcur, int bnxt) {
    __builtin_amdgcn_s_waitcnt((15) | (3 << 14) | (7 << 4) | (0 << 8));  // lgkmcnt(0): step it's reads done
#pragma unroll
    for (int q = 0; q < NQ / 2; q++) {
      mfma_q(q, cur);
      issue(it + 2, bcur, q * PER / (NQ / 2), (q + 1) * PER / (NQ / 2));
    }
    wait_vm<PER>();  // step it + 1 has landed
#pragma unroll
    for (int q = NQ / 2; q < NQ; q++) {
      mfma_q(q, cur);
      const int q2 = q - NQ / 2;
#pragma unroll
      for (int f = q2 * NF / (NQ / 2); f < (q2 + 1) * NF / (NQ / 2); f++) load_frag(bnxt, f, nxt);
    }
  };
  issue(0, 0, 0, PER);
  issue(1, 1, 0, PER);
  wait_vm<PER>();  // step 0 has landed
#pragma unroll
  for (int f = 0; f < NF; f++) load_frag(0, f, fa);
  for (int it = 0; it < nsw; it += 2) {  // nsw is even: slices are multiples of 256 tokens
    body(it, fa, fb, 0, 1);
    body(it + 1, fb, fa, 1, 0);
  }
  wait_vm<0>();  // the trailing reloads land before the LDS is reused

  // ---- the four partial tiles, added in wave order
  // acc[i][j][r] = C[m0 + 16i + 4 (lane / 16) + r][n0 + 16j + lane % 16]
  __syncthreads();  // every wave has finished reading its stages
  float* TF = (float*)lds;
  const int fg = lane >> 4, cc = lane & 15;
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
      for (int r = 0; r < 4; r++) TF[(wave * 64 + 16 * i + 4 * fg + r) * KW_TLD + 16 * j + cc] = acc[i][j][r];
  __syncthreads();
  float* dst0 = EPI == E_PARTIAL ? p.partial + (long)tz * pM * pN : (float*)p.c[0];
  const long ldd = EPI == E_PARTIAL ? pN : p.ldc[0];
  const bool acc_out = EPI == E_STORE && p.accumulate;
  const bool bfout = EPI == E_STORE && p.c_bf16;
  // every 4-column chunk is a whole vector when the base and the row stride are
  const bool vec = (ldd & 3) == 0 && ((uintptr_t)(bfout ? p.c[0] : (void*)dst0) & (bfout ? 7 : 15)) == 0;
  double q = 0.0;
  for (int c = threadIdx.x; c < 64 * 16; c += NT) {
    const int r = c >> 4, c4 = (c & 15) * 4;
    const long m = m0 + r, n = n0 + c4;
    if (m >= pM || n >= pN) continue;  // N % 8 == 0: a chunk is in or out whole
    float4 v = *(const float4*)(TF + r * KW_TLD + c4);
#pragma unroll
    for (int w = 1; w < 4; w++) {
      const float4 u = *(const float4*)(TF + (w * 64 + r) * KW_TLD + c4);
      v = make_float4(v.x + u.x, v.y + u.y, v.z + u.z, v.w + u.w);
    }
    if (bfout) {
      bf16_t* d = (bf16_t*)p.c[0] + m * ldd + n;
      if (vec) {
        *(u32x2*)d = u32x2{pack2(f2bf(v.x), f2bf(v.y)), pack2(f2bf(v.z), f2bf(v.w))};
      } else {
        d[0] = f2bf(v.x); d[1] = f2bf(v.y); d[2] = f2bf(v.z); d[3] = f2bf(v.w);
      }
    } else {
      float* d = dst0 + m * ldd + n;
      if (vec) {
        if (acc_out) {
          const float4 o = *(const float4*)d;
          v = make_float4(o.x + v.x, o.y + v.y, o.z + v.z, o.w + v.w);
        }
        *(float4*)d = v;
      } else {
        if (acc_out) {
          v.x += d[0]; v.y += d[1]; v.z += d[2]; v.w += d[3];
        }
        d[0] = v.x; d[1] = v.y; d[2] = v.z; d[3] = v.w;
      }
    }
    if constexpr (EPI == E_STORE)
      q += (double)v.x * v.x + (double)v.y * v.y + (double)v.z * v.z + (double)v.w * v.w;
  }
  if (EPI == E_STORE && p.sq) {
    __shared__ double red[NT / 64];
    q = block_sum<double, NT>(q, red);
    if (threadIdx.x == 0) p.sq[b] = q;
  }
}

// sq (nullable): FP64 sum of squares of the values this workgroup stores,
// at sq[blockIdx.x] (the gradient-norm hook)
__global__ __launch_bounds__(256) void k_reduce_partials(const float* __restrict__ partial, int splits, long M, long N,
                                                         void* c, long ldc, int c_bf16, int accumulate, double* sq) {
  const long total = M * N;
  double q = 0.0;
  // contiguous C (ldc == N) with 16-byte partials and 16- (fp32) or 8-byte
  // (bf16) aligned C: four elements per step at the partials' own index
  // (uniform; the same additions, in slice order from +0, as below)
  const bool vec = ldc == N && total % 4 == 0 && ((uintptr_t)partial & 15) == 0 &&
                   ((uintptr_t)c & (c_bf16 ? 7 : 15)) == 0;
  if (vec) {
    const long total4 = total / 4;
    const float4* p4 = (const float4*)partial;
    for (long t = blockIdx.x * 256L + threadIdx.x; t < total4; t += (long)gridDim.x * 256L) {
      f32x4 s = f32x4{0.f, 0.f, 0.f, 0.f};
      for (int z = 0; z < splits; z++) {
        const float4 v = p4[(long)z * total4 + t];
        s += f32x4{v.x, v.y, v.z, v.w};
      }
      if (c_bf16) {
        ((u32x2*)c)[t] = u32x2{pack2(f2bf(s[0]), f2bf(s[1])), pack2(f2bf(s[2]), f2bf(s[3]))};
      } else {
        if (accumulate) {
          const float4 o = ((const float4*)c)[t];
          s += f32x4{o.x, o.y, o.z, o.w};
        }
        ((float4*)c)[t] = make_float4(s[0], s[1], s[2], s[3]);
      }
      if (sq) q += (double)s[0] * s[0] + (double)s[1] * s[1] + (double)s[2] * s[2] + (double)s[3] * s[3];
    }
  }
  for (long i = vec ? total : blockIdx.x * 256L + threadIdx.x; i < total; i += (long)gridDim.x * 256L) {
    float s = 0.f;
    for (int z = 0; z < splits; z++) s += partial[(long)z * total + i];
    const long m = i / N, n = i - m * N;
    const long idx = m * ldc + n;
    if (c_bf16) {
      ((bf16_t*)c)[idx] = f2bf(s);
    } else if (accumulate) {
      s += ((float*)c)[idx];
      ((float*)c)[idx] = s;
    } else {
      ((float*)c)[idx] = s;
    }
    q += (double)s * (double)s;
  }
  if (sq) {
    __shared__ double red[4];
    q = block_sum<double, 256>(q, red);
    if (threadIdx.x == 0) sq[blockIdx.x] = q;
  }
}

template <int BM, int BN, int PA, int PB, int EPI, int NS, int TM = 0>
int launch_ns(hipStream_t s, const FParams& p, int splits) {
  constexpr int NBM = EPI == E_GATEUP ? 2 : 1;
  constexpr size_t lds = lds_bytes<BM, BN, PA, PB, EPI, NS>();
  static_assert(lds <= 160 * 1024, "LDS budget");
  auto kern = k_gemm_fast<BM, BN, PA, PB, EPI, NS, TM>;
  const_cast<FParams&>(p).xcd_remap = xcd_remap();
  // grid z: split-K slices, or the experts of a per-expert dW launch
  dim3 grid((unsigned)((p.N + BN - 1) / BN), (unsigned)((p.M + BM - 1) / BM), (unsigned)splits);
  const_cast<FParams&>(p).group = tile_group(p.N * (EPI == E_GATEUP ? 2 : 1), p.K, PB, grid.y);
  if ((unsigned long long)grid.x * grid.y * grid.z >= (1ull << 20))
    return sjh::fail(SJ_ERR_INVALID, "gemm: %u x %u x %u workgroups (at most 2^20)", grid.x, grid.y, grid.z);
  auto magic = [](unsigned long long d) { return (1ull << 40) / d + 1; };
  const unsigned small = grid.y < grid.x ? grid.y : grid.x;
  const_cast<FParams&>(p).mdiv_lo = magic(small);
  const_cast<FParams&>(p).mdiv_xy = magic((unsigned long long)grid.x * grid.y);
  sjh::ProfHook& h = sjh::prof_hook();
  if (h.on && h.k0) {  // kernel timing: events at the kernel's own start and end
    hipExtLaunchKernelGGL(kern, grid, dim3(NT), (uint32_t)lds, s, h.k0, h.k1, 0u, p);
    h.used = true;
  } else {
    hipLaunchKernelGGL(kern, grid, dim3(NT), lds, s, p);
  }
  if (h.on)
    snprintf(h.kernel, sizeof(h.kernel), "k_gemm_fast<%d, %d, %d, %d, %d, %d, %d>", BM, BN, PA, PB, EPI, NS, TM);
  return SJ_OK;
}

template <int PB, int EPI, int NS>
int launch_kw_ns(hipStream_t s, const FParams& p, int splits) {
  constexpr size_t lds = kw_lds_bytes<PB, NS>();
  static_assert(lds + 64 <= 160 * 1024, "LDS budget");
  auto kern = k_gemm_kw<PB, EPI, NS>;
  const_cast<FParams&>(p).xcd_remap = xcd_remap();
  dim3 grid((unsigned)((p.N + 63) / 64), (unsigned)((p.M + 63) / 64), (unsigned)splits);
  if ((unsigned long long)grid.x * grid.y * grid.z >= (1ull << 20))
    return sjh::fail(SJ_ERR_INVALID, "gemm: %u x %u x %u workgroups (at most 2^20)", grid.x, grid.y, grid.z);
  auto magic = [](unsigned long long d) { return (1ull << 40) / d + 1; };
  const unsigned small = grid.y < grid.x ? grid.y : grid.x;
  const_cast<FParams&>(p).mdiv_lo = magic(small);
  const_cast<FParams&>(p).mdiv_xy = magic((unsigned long long)grid.x * grid.y);
  sjh::ProfHook& h = sjh::prof_hook();
  if (h.on && h.k0) {
    hipExtLaunchKernelGGL(kern, grid, dim3(NT), (uint32_t)lds, s, h.k0, h.k1, 0u, p);
    h.used = true;
  } else {
    hipLaunchKernelGGL(kern, grid, dim3(NT), lds, s, p);
  }
  if (h.on) snprintf(h.kernel, sizeof(h.kernel), "k_gemm_kw<%d, %d, %d>", PB, EPI, NS);
  return SJ_OK;
}
template <int EPI>
int launch_kw(hipStream_t s, const FParams& p, int pb, int splits) {
  return pb == 2 ? launch_kw_ns<2, EPI, 2>(s, p, splits) : launch_kw_ns<1, EPI, 2>(s, p, splits);
}

// Pipeline depth (measured on gfx950 over the cfg2 and cfg5 step GEMMs):
// three stages when every workgroup of the launch is resident at three
// (deeper prefetch, nothing gained by more residency); otherwise two when
// two stages let more workgroups share a CU (64x128 tiles at K = 384:
// 28.3 -> 19.9 us), else three.  Residency comes from the runtime's
// occupancy query (LDS and registers of that instantiation).
// SJ_GEMM_STAGES=2|3 overrides it (sweeps).
int g_stages = -1;
int cus();
template <int BM, int BN, int PA, int PB, int EPI, int NS, int TM = 0>
int resident() {
  static int occ = -1;
  if (occ < 0) {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, k_gemm_fast<BM, BN, PA, PB, EPI, NS, TM>, NT,
                                                     lds_bytes<BM, BN, PA, PB, EPI, NS>()) != hipSuccess)
      n = 1;
    occ = n > 0 ? n : 1;
  }
  return occ;
}
template <int BM, int BN, int PA, int PB, int EPI, int TM = 0>
int launch(hipStream_t s, const FParams& p, int splits) {
  if (g_stages < 0) {
    const char* e = getenv("SJ_GEMM_STAGES");
    g_stages = e ? atoi(e) : 0;
  }
  constexpr bool three = lds_bytes<BM, BN, PA, PB, EPI, 3>() <= 160 * 1024;
  int ns = 2;
  if constexpr (three) {
    if (g_stages == 2 || g_stages == 3) {
      ns = g_stages;
    } else {
      const long wgs = ((p.N + BN - 1) / BN) * ((p.M + BM - 1) / BM) * (long)splits;
      const int o3 = resident<BM, BN, PA, PB, EPI, 3, TM>(), o2 = resident<BM, BN, PA, PB, EPI, 2, TM>();
      ns = (wgs <= (long)o3 * cus() || o2 <= o3) ? 3 : 2;
    }
    if (ns == 3) return launch_ns<BM, BN, PA, PB, EPI, 3, TM>(s, p, splits);
  }
  return launch_ns<BM, BN, PA, PB, EPI, 2, TM>(s, p, splits);
}

int g_cu = 0;
int cus() {
  if (!g_cu) {
    int dev = 0, cu = 256;
    if (hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&cu, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess)
      g_cu = cu;
    else
      g_cu = 256;
  }
  return g_cu;
}

inline long tiles(long M, long N, int bm, int bn) { return ((M + bm - 1) / bm) * ((N + bn - 1) / bn); }

// Tile heuristic: largest tile with >= 1 workgroup per CU, else 64x64.
// SJ_GEMM_TILE=<bm>x<bn> (64 or 128 each) overrides it, for tuning sweeps.
void pick(long M, long N, int& bm, int& bn) {
  static int obm = -1, obn = -1;
  if (obm < 0) {
    obm = obn = 0;
    if (const char* e = getenv("SJ_GEMM_TILE")) {
      int a = 0, b = 0;
      if (sscanf(e, "%dx%d", &a, &b) == 2 && (a == 64 || a == 128) && (b == 64 || b == 128)) {
        obm = a;
        obn = b;
      }
    }
  }
  if (obm) {
    bm = obm;
    bn = obn;
    return;
  }
  const long cu = cus();
  if (tiles(M, N, 128, 128) >= cu) { bm = 128; bn = 128; return; }
  if (tiles(M, N, 128, 64) >= cu) { bm = 128; bn = 64; return; }
  if (tiles(M, N, 64, 128) >= cu) { bm = 64; bn = 128; return; }
  bm = 64; bn = 64;
}

// Split-K count: enough slices for ~2 workgroups per CU when the tiles
// alone do not fill the chip.  SJ_GEMM_SPLITS=<n> overrides it (sweeps).
int splits_for(long M, long N, long K, int bm, int bn);

// Tile and split-K plan of sj_gemm_planes (measured on the cfg2 and cfg5
// step shapes with the occupancy-chosen pipeline depth):
//   very long K (>= 8192) with a short output (M <= 512 or N <= 64: the
//   token-contracted products of the parameter VJP): 64x64 tiles and
//   floor(4 x CUs / tiles) K slices, clamped to 8..16 and to slices of
//   >= 512 (cfg5 coefficients 144 x 1536 x 16384: 14 slices, 66 -> 51 us;
//   144 x 5504 x 16384: 8 slices, 175 -> 158 us; 64x128 tiles lose at every
//   slice count);
//   dW-shaped products (K >= 2048, at most one 64x64 tile per CU): one K
//   slice up to K = 4096, else 4, and the largest tile giving min(2 per CU,
//   slices x the 64x64 tiles) workgroups (cfg5 attention-output dW: 128x64
//   x 4 slices, 115 -> 90 us); SJ_GEMM_DW_SPLITS overrides the slices;
//   split-A products (dX): 64x128 tiles when they give two per CU, else
//   64x64 (cfg5 down dX: 662 -> 499 us; cfg2 dX: 64x64);
//   the rest pick().
void plan(long M, long N, long K, int pa, int& bm, int& bn, int& splits, bool row_layout = false) {
  const long cu = cus();
  const char* et = getenv("SJ_GEMM_TILE");
  const char* es = getenv("SJ_GEMM_SPLITS");
  if (!et && !es) {
    if (K >= 8192 && (M <= 512 || N <= 64)) {
      static int lkn = -1, lks = 0;
      if (lkn < 0) {  // sweeps: SJ_GEMM_LK_TILE=64x<bn>, SJ_GEMM_LK_SPLITS=<n>
        lkn = 0;
        const char* e = getenv("SJ_GEMM_LK_TILE");
        int a = 0, b = 0;
        if (e && sscanf(e, "%dx%d", &a, &b) == 2 && a == 64 && (b == 64 || b == 128)) lkn = b;
        if (const char* s = getenv("SJ_GEMM_LK_SPLITS")) lks = atoi(s);
      }
      bm = 64;
      bn = lkn && N >= 128 ? lkn : 64;
      const long t = tiles(M, N, bm, bn);
      long sp = 4 * cu / t;
      sp = sp < 8 ? 8 : sp;
      sp = sp > 16 ? 16 : sp;
      if (lks > 0) sp = lks;
      sp = sp > K / 512 ? K / 512 : sp;
      splits = (int)sp;
      return;
    }
    if (tiles(M, N, 64, 64) <= cu && K >= 2048) {
      static int dws = -1;
      if (dws < 0) {
        const char* e = getenv("SJ_GEMM_DW_SPLITS");  // sweeps
        dws = e ? atoi(e) : 0;
      }
      // the step runs dW beside the dX chain on its own stream: one slice up to
      // K = 4096 (cfg2: no partials pass, 2.24 -> 2.20 ms), four beyond (cfg5);
      // the row-layout form (LDS transpose reads, more LDS traffic per MFMA)
      // takes four from K = 4096 (cfg2 step 2.004 -> 1.981 ms; at K = 2048,
      // cfg3's global stage, slices of 512 lose: 4.07 -> 4.15 ms)
      const int want_s = dws > 0 ? dws : row_layout ? (K >= 4096 ? 4 : 1) : (K <= 4096 ? 1 : 4);
      splits = K / 256 < want_s ? (int)(K / 256) : want_s;
      static int dwt_m = -1, dwt_n = 0;
      if (dwt_m < 0) {
        dwt_m = 0;
        if (const char* e = getenv("SJ_GEMM_DW_TILE"))  // sweeps
          if (sscanf(e, "%dx%d", &dwt_m, &dwt_n) != 2 || (dwt_m != 64 && dwt_m != 128) || (dwt_n != 64 && dwt_n != 128))
            dwt_m = 0;
      }
      if (dwt_m) {
        bm = dwt_m;
        bn = dwt_n;
        return;
      }
      long want = tiles(M, N, 64, 64) * splits;
      want = want < 2 * cu ? want : 2 * cu;
      const int cand[4][2] = {{128, 128}, {128, 64}, {64, 128}, {64, 64}};
      for (const auto& c : cand)
        if (tiles(M, N, c[0], c[1]) * splits >= want || (c[0] == 64 && c[1] == 64)) {
          bm = c[0];
          bn = c[1];
          return;
        }
    }
    if (pa == 2) {
      bm = 64;
      bn = tiles(M, N, 64, 128) >= 2 * cu ? 128 : 64;
      splits = splits_for(M, N, K, bm, bn);
      return;
    }
  }
  pick(M, N, bm, bn);
  splits = splits_for(M, N, K, bm, bn);
}

int splits_for(long M, long N, long K, int bm, int bn) {
  static int ov = -1;
  if (ov < 0) {
    const char* e = getenv("SJ_GEMM_SPLITS");
    ov = e ? atoi(e) : 0;
  }
  if (ov > 0) {
    long s = ov < K / 64 ? ov : K / 64;
    return s < 1 ? 1 : (int)s;
  }
  const long t = tiles(M, N, bm, bn), cu = cus();
  if (t >= cu || K < 1024) return 1;
  long s = (2 * cu + t - 1) / t;
  if (s > K / 256) s = K / 256;
  if (s > 32) s = 32;
  return s < 1 ? 1 : (int)s;
}

// Token-split dW plan (row-layout X with one plane, dW-shaped: K >= 1024, a
// multiple of 256): 64x64 tiles, one workgroup per CU (96 KB of LDS for
// split Y), so as many K slices as fill the CUs once, each at least 512
// tokens.  SJ_GEMM_KW=0
// selects the k_gemm_fast form; SJ_GEMM_KW_SPLITS=<n> overrides the slices
// (sweeps).
bool plan_kw(long M, long N, long K, int pa, int& splits) {
  static int on = -1, ov = 0;
  if (on < 0) {
    const char* e = getenv("SJ_GEMM_KW");
    on = e ? atoi(e) != 0 : 1;
    const char* o = getenv("SJ_GEMM_KW_SPLITS");
    ov = o ? atoi(o) : 0;
  }
  if (!on || pa != 1 || K < 1024 || K % 256) return false;
  const long t = tiles(M, N, 64, 64), cu = cus();
  if (t > cu) return false;
  long sp = ov > 0 ? ov : cu / t;
  if (sp > K / 512) sp = K / 512;
  if (sp > 16) sp = 16;
  splits = sp < 1 ? 1 : (int)sp;
  return true;
}

template <int EPI, int PA, int PB, int TM = 0>
int launch_tile(hipStream_t s, const FParams& p, int bm, int bn, int splits) {
  // both operands split: a 128x128 stage does not fit three deep in LDS
  if constexpr (PA == 2 && PB == 2) {
    if (bm == 128 && bn == 128) bn = 64;
  } else {
    if (bm == 128 && bn == 128) return launch<128, 128, PA, PB, EPI, TM>(s, p, splits);
  }
  if (bm == 128 && bn == 64) return launch<128, 64, PA, PB, EPI, TM>(s, p, splits);
  if (bm == 64 && bn == 128) return launch<64, 128, PA, PB, EPI, TM>(s, p, splits);
  return launch<64, 64, PA, PB, EPI, TM>(s, p, splits);
}

// plane combinations each epilogue is used with: forward epilogues read
// one-plane operands, the SwiGLU derivative a split dY, plain GEMMs any
template <int EPI, int PA, int PB>
constexpr bool plane_combo() {
  if (EPI == E_STORE || EPI == E_PARTIAL) return true;
  if (EPI == E_SWIGLU_BWD || EPI == E_SWIGLU_ROWS || EPI == E_PLANES) return PA == 2 && PB == 1;
  return PA == 1 && PB == 1;
}

template <int EPI, int TM = 0>
int launch_planes(hipStream_t s, const FParams& p, int pa, int pb, int bm, int bn, int splits) {
  if constexpr (plane_combo<EPI, 1, 1>())
    if (pa == 1 && pb == 1) return launch_tile<EPI, 1, 1, TM>(s, p, bm, bn, splits);
  if constexpr (plane_combo<EPI, 2, 1>())
    if (pa == 2 && pb == 1) return launch_tile<EPI, 2, 1, TM>(s, p, bm, bn, splits);
  if constexpr (plane_combo<EPI, 1, 2>())
    if (pa == 1 && pb == 2) return launch_tile<EPI, 1, 2, TM>(s, p, bm, bn, splits);
  if constexpr (plane_combo<EPI, 2, 2>())
    if (pa == 2 && pb == 2) return launch_tile<EPI, 2, 2, TM>(s, p, bm, bn, splits);
  return sjh::fail(SJ_ERR_UNSUPPORTED, "gemm: planes %d/%d for this epilogue", pa, pb);
}

// One operand in row layout, the other k-contiguous (the parameter VJP's
// token-contracted products): TM 1, A = X [K][M] as one plane and B as two;
// TM 2, A as two planes and B = Y [K][N] as two.
template <int EPI, int TM>
int launch_planes_one(hipStream_t s, const FParams& p, int pa, int pb, int bm, int bn, int splits) {
  static_assert(TM == 1 || TM == 2, "one row-layout operand");
  constexpr int PA = TM == 1 ? 1 : 2, PB = 2;
  if (pa != PA || pb != PB) return sjh::fail(SJ_ERR_UNSUPPORTED, "gemm: planes %d/%d with row-layout operand %d", pa, pb, TM);
  return launch_tile<EPI, PA, PB, TM>(s, p, bm, bn, splits);
}

bool ok16(const void* q) { return ((uintptr_t)q & 15) == 0; }

// The row-plane SwiGLU epilogue moves G, U and the four planes in whole
// 16-byte chunks: no transposed outputs, 8-aligned widths and strides.
bool swiglu_rows_ok(const FParams& p) {
  return !p.c[2] && !p.c[3] && p.F % 8 == 0 && p.ldgu % 8 == 0 && p.ldc[0] % 8 == 0 && ok16(p.gin) && ok16(p.uin) &&
         ok16(p.c[0]) && ok16(p.c[1]);
}

template <int BM, int BN, int PA, int PB, int EPI, int NS, int TM = 0>
int set_attr_ns() {
  constexpr size_t lds = lds_bytes<BM, BN, PA, PB, EPI, NS>();
  hipError_t e = hipFuncSetAttribute((const void*)k_gemm_fast<BM, BN, PA, PB, EPI, NS, TM>,
                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  return e == hipSuccess ? SJ_OK : sjh::hip_check(e, "gemm: LDS attribute");
}
template <int BM, int BN, int PA, int PB, int EPI, int TM = 0>
int set_attr() {
  int st = set_attr_ns<BM, BN, PA, PB, EPI, 2, TM>();
  if constexpr (lds_bytes<BM, BN, PA, PB, EPI, 3>() <= 160 * 1024)
    if (!st) st = set_attr_ns<BM, BN, PA, PB, EPI, 3, TM>();
  return st;
}
template <int EPI, int PA, int PB, int TM = 0>
int set_attrs_tiles() {
  int s = SJ_OK;
  if constexpr (!(PA == 2 && PB == 2)) s = set_attr<128, 128, PA, PB, EPI, TM>();
  if (!s) s = set_attr<128, 64, PA, PB, EPI, TM>();
  if (!s) s = set_attr<64, 128, PA, PB, EPI, TM>();
  if (!s) s = set_attr<64, 64, PA, PB, EPI, TM>();
  return s;
}
template <int EPI, int TM = 0>
int set_attrs_planes() {
  int s = SJ_OK;
  if constexpr (plane_combo<EPI, 1, 1>()) s = set_attrs_tiles<EPI, 1, 1, TM>();
  if constexpr (plane_combo<EPI, 2, 1>()) if (!s) s = set_attrs_tiles<EPI, 2, 1, TM>();
  if constexpr (plane_combo<EPI, 1, 2>()) if (!s) s = set_attrs_tiles<EPI, 1, 2, TM>();
  if constexpr (plane_combo<EPI, 2, 2>()) if (!s) s = set_attrs_tiles<EPI, 2, 2, TM>();
  return s;
}

template <int PB, int EPI, int NS>
int set_attr_kw() {
  hipError_t e = hipFuncSetAttribute((const void*)k_gemm_kw<PB, EPI, NS>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                     (int)kw_lds_bytes<PB, NS>());
  return e == hipSuccess ? SJ_OK : sjh::hip_check(e, "gemm: LDS attribute");
}
template <int EPI>
int set_attrs_kw() {
  int s = set_attr_kw<2, EPI, 2>();
  if (!s) s = set_attr_kw<1, EPI, 2>();
  return s;
}

}  // namespace

// Raise the dynamic-LDS limit of every instantiation once (outside any
// stream capture); called by sj_model_create and lazily by the entry points.
namespace sjh {
int gemm_fast_prepare() {
  static int done = 0, status = SJ_OK;
  if (done) return status;
  done = 1;
  status = set_attrs_planes<E_STORE>();
  if (!status) status = set_attrs_planes<E_PARTIAL>();
  if (!status) status = set_attrs_planes<E_QKV>();
  if (!status) status = set_attrs_planes<E_RESID>();
  if (!status) status = set_attrs_planes<E_GATEUP>();
  if (!status) status = set_attrs_planes<E_SWIGLU_BWD>();
  if (!status) status = set_attrs_planes<E_SWIGLU_ROWS>();
  if (!status) status = set_attrs_planes<E_PLANES>();
  if (!status) status = set_attrs_planes<E_STORE, 3>();
  if (!status) status = set_attrs_planes<E_PARTIAL, 3>();
  if (!status) status = set_attrs_tiles<E_STORE, 1, 2, 1>();
  if (!status) status = set_attrs_tiles<E_PARTIAL, 1, 2, 1>();
  if (!status) status = set_attrs_tiles<E_STORE, 2, 2, 2>();
  if (!status) status = set_attrs_tiles<E_PARTIAL, 2, 2, 2>();
  if (!status) status = set_attrs_kw<E_STORE>();
  if (!status) status = set_attrs_kw<E_PARTIAL>();
  return status;
}
}  // namespace sjh

// ================================================================ C ABI

extern "C" size_t sj_gemm_planes_workspace_bytes(long M, long N, long K) {
  // the largest of the plans for a split and an unsplit A operand, with
  // k-contiguous and row-layout operands
  size_t need = 0;
  for (int pa = 1; pa <= 2; pa++)
    for (int rl = 0; rl < 2; rl++) {
      int bm, bn, s;
      plan(M, N, K, pa, bm, bn, s, rl != 0);
      int skw = 1;
      if (rl && plan_kw(M, N, K, pa, skw) && skw > s) s = skw;  // the token-split dW plan
      const size_t b = s > 1 ? sizeof(float) * (size_t)s * (size_t)M * (size_t)N : 0;
      need = b > need ? b : need;
    }
  return need;
}

namespace {
// split-K partials and their fixed-order reduce (with the gradient-norm
// slots when the hook is armed)
int reduce_partials(hipStream_t s, const FParams& p, int splits, void* workspace) {
  const long M = p.M, N = p.N;
  // the kernel's 16-byte path (same condition) takes four elements a thread
  const bool vec = p.ldc[0] == N && (M * N) % 4 == 0 && ((uintptr_t)workspace & 15) == 0 &&
                   ((uintptr_t)p.c[0] & (p.c_bf16 ? 7 : 15)) == 0;
  long total = M * N, blocks = (total + (vec ? 1023 : 255)) / (vec ? 1024 : 256);
  double* sq = nullptr;
  sjh::GradSq& gs = sjh::grad_sq();
  if (gs.base && gs.on) {  // gradient-norm slots: fewer, longer workgroups
    if (blocks > 1024) blocks = 1024;
    sq = gs.take(blocks);
  } else if (blocks > 4096) {
    blocks = 4096;
  }
  hipLaunchKernelGGL(k_reduce_partials, dim3((unsigned)blocks), dim3(256), 0, s, (const float*)workspace, splits, M, N,
                     p.c[0], p.ldc[0], (int)p.c_bf16, p.accumulate, sq);
  return SJ_OK;
}

int gemm_kw(hipStream_t s, FParams& p, int pb, int splits, void* workspace, size_t workspace_bytes) {
  const long M = p.M, N = p.N, K = p.K;
  if (splits > 1 && workspace && workspace_bytes >= sizeof(float) * (size_t)splits * M * N) {
    long kchunk = (K + splits - 1) / splits;
    kchunk = (kchunk + 255) / 256 * 256;  // an even number of 128-token steps
    splits = (int)((K + kchunk - 1) / kchunk);
    p.kchunk = kchunk;
    p.partial = (float*)workspace;
    if (int st = launch_kw<E_PARTIAL>(s, p, pb, splits)) return st;
    reduce_partials(s, p, splits, workspace);
  } else {
    sjh::GradSq& gs = sjh::grad_sq();
    if (gs.base && gs.on) p.sq = gs.take(tiles(M, N, 64, 64));  // slot per workgroup, linear id
    if (int st = launch_kw<E_STORE>(s, p, pb, 1)) return st;
  }
  SJ_LAUNCH_CHECK("matmul planes (token-split dW)");
  return SJ_OK;
}

template <int TM>
int gemm_planes(void* stream, long M, long N, long K, const uint16_t* a_hi, const uint16_t* a_lo, long lda,
                const uint16_t* b_hi, const uint16_t* b_lo, long ldb, void* c, int c_dtype, long ldc, int accumulate,
                void* workspace, size_t workspace_bytes) {
  if (M == 0 || N == 0 || K == 0) return SJ_OK;
  hipStream_t s = (hipStream_t)stream;
  FParams p = {};
  p.a[0] = (const bf16_t*)a_hi; p.a[1] = (const bf16_t*)a_lo; p.lda = lda;
  p.b[0][0] = (const bf16_t*)b_hi; p.b[1][0] = (const bf16_t*)b_lo; p.ldb[0] = ldb; p.seg_n[0] = 0; p.nseg = 1;
  p.M = M; p.N = N; p.K = K;
  p.c[0] = c; p.ldc[0] = ldc; p.c_bf16 = c_dtype == SJ_BF16; p.accumulate = accumulate;
  const int pa = a_lo ? 2 : 1, pb = b_lo ? 2 : 1;
  int bm, bn, splits;
  if constexpr (TM == 3)
    if (plan_kw(M, N, K, pa, splits)) return gemm_kw(s, p, pb, splits, workspace, workspace_bytes);
  plan(M, N, K, pa, bm, bn, splits, TM != 0);
  if (splits > 1 && workspace && workspace_bytes >= sizeof(float) * (size_t)splits * M * N) {
    long kchunk = (K + splits - 1) / splits;
    kchunk = (kchunk + BK - 1) / BK * BK;
    splits = (int)((K + kchunk - 1) / kchunk);
    p.kchunk = kchunk;
    p.partial = (float*)workspace;
    int st;
    if constexpr (TM == 1 || TM == 2)
      st = launch_planes_one<E_PARTIAL, TM>(s, p, pa, pb, bm, bn, splits);
    else
      st = launch_planes<E_PARTIAL, TM>(s, p, pa, pb, bm, bn, splits);
    if (st) return st;
    reduce_partials(s, p, splits, workspace);
  } else {
    int st;
    if constexpr (TM == 1 || TM == 2)
      st = launch_planes_one<E_STORE, TM>(s, p, pa, pb, bm, bn, 1);
    else
      st = launch_planes<E_STORE, TM>(s, p, pa, pb, bm, bn, 1);
    if (st) return st;
    if (sjh::grad_sq().base && sjh::grad_sq().on) sjh::grad_sq().missed = true;
  }
  SJ_LAUNCH_CHECK("matmul planes");
  return SJ_OK;
}
}  // namespace

// The parameter VJP's two token-contracted products with one operand in row
// layout (K = tokens, a multiple of 8; fp32 C):
//   rows_a: C [M][N] = X^T B^T, X [K][ldx] one bf16 plane (row layout), B
//           [N][K] hi/lo planes (k-contiguous);
//   rows_b: C [M][N] = A Y, A [M][K] hi/lo planes (k-contiguous), Y [K][ldy]
//           hi/lo planes (row layout).
int sjh::gemm_planes_rows_a(void* stream, long M, long N, long K, const uint16_t* x, long ldx, const uint16_t* b_hi,
                            const uint16_t* b_lo, long ldb, float* c, long ldc, void* workspace,
                            size_t workspace_bytes) {
  if (int st0 = sjh::gemm_fast_prepare()) return st0;
  SJ_REQUIRE(M > 0 && N > 0 && K > 0 && M % 8 == 0 && K % 8 == 0 && ldx % 8 == 0 && ldb % 8 == 0 && ldx >= M &&
                 ldb >= K && ldc >= N && x && b_hi && b_lo && ok16(x) && ok16(b_hi) && ok16(b_lo),
             "matmul planes (row-layout A): M %ld N %ld K %ld ldx %ld ldb %ld (M, K and ld multiples of 8)", M, N, K,
             ldx, ldb);
  return gemm_planes<1>(stream, M, N, K, x, nullptr, ldx, b_hi, b_lo, ldb, c, SJ_F32, ldc, 0, workspace,
                        workspace_bytes);
}
int sjh::gemm_planes_rows_b(void* stream, long M, long N, long K, const uint16_t* a_hi, const uint16_t* a_lo,
                            long lda, const uint16_t* y_hi, const uint16_t* y_lo, long ldy, float* c, long ldc,
                            void* workspace, size_t workspace_bytes) {
  if (int st0 = sjh::gemm_fast_prepare()) return st0;
  SJ_REQUIRE(M > 0 && N > 0 && K > 0 && N % 8 == 0 && K % 8 == 0 && lda % 8 == 0 && ldy % 8 == 0 && lda >= K &&
                 ldy >= N && ldc >= N && a_hi && a_lo && y_hi && y_lo && ok16(a_hi) && ok16(a_lo) && ok16(y_hi) &&
                 ok16(y_lo),
             "matmul planes (row-layout B): M %ld N %ld K %ld lda %ld ldy %ld (N, K and ld multiples of 8)", M, N, K,
             lda, ldy);
  return gemm_planes<2>(stream, M, N, K, a_hi, a_lo, lda, y_hi, y_lo, ldy, c, SJ_F32, ldc, 0, workspace,
                        workspace_bytes);
}

extern "C" int sj_gemm_planes(void* stream, long M, long N, long K, const uint16_t* a_hi, const uint16_t* a_lo,
                              long lda, const uint16_t* b_hi, const uint16_t* b_lo, long ldb, void* c, int c_dtype,
                              long ldc, int accumulate, void* workspace, size_t workspace_bytes) {
  if (int st0 = sjh::gemm_fast_prepare()) return st0;
  SJ_REQUIRE(M >= 0 && N >= 0 && K >= 0 && K % 8 == 0 && lda % 8 == 0 && ldb % 8 == 0 && lda >= K && ldb >= K &&
                 ldc >= N,
             "matmul planes: M %ld N %ld K %ld lda %ld ldb %ld (K and ld must be multiples of 8)", M, N, K, lda, ldb);
  SJ_REQUIRE(a_hi && b_hi && ok16(a_hi) && ok16(b_hi) && (!a_lo || ok16(a_lo)) && (!b_lo || ok16(b_lo)),
             "matmul planes: 16-byte aligned planes required");
  SJ_REQUIRE(c_dtype == SJ_F32 || c_dtype == SJ_BF16, "matmul planes: output dtype %d", c_dtype);
  SJ_REQUIRE(!(accumulate && c_dtype == SJ_BF16), "matmul: accumulate needs an fp32 output");
  return gemm_planes<0>(stream, M, N, K, a_hi, a_lo, lda, b_hi, b_lo, ldb, c, c_dtype, ldc, accumulate, workspace,
                        workspace_bytes);
}

extern "C" int sj_gemm_planes_tn(void* stream, long M, long N, long K, const uint16_t* x_hi, const uint16_t* x_lo,
                                 long ldx, const uint16_t* y_hi, const uint16_t* y_lo, long ldy, void* c, int c_dtype,
                                 long ldc, int accumulate, void* workspace, size_t workspace_bytes) {
  if (int st0 = sjh::gemm_fast_prepare()) return st0;
  SJ_REQUIRE(M >= 0 && N >= 0 && K >= 0 && M % 8 == 0 && N % 8 == 0 && ldx % 8 == 0 && ldy % 8 == 0 && ldx >= M &&
                 ldy >= N && ldc >= N,
             "matmul planes (row-layout operands): M %ld N %ld K %ld ldx %ld ldy %ld (M, N and ld multiples of 8)",
             M, N, K, ldx, ldy);
  SJ_REQUIRE(x_hi && y_hi && ok16(x_hi) && ok16(y_hi) && (!x_lo || ok16(x_lo)) && (!y_lo || ok16(y_lo)),
             "matmul planes (row-layout operands): 16-byte aligned planes required");
  SJ_REQUIRE(c_dtype == SJ_F32 || c_dtype == SJ_BF16, "matmul planes: output dtype %d", c_dtype);
  SJ_REQUIRE(!(accumulate && c_dtype == SJ_BF16), "matmul: accumulate needs an fp32 output");
  return gemm_planes<3>(stream, M, N, K, x_hi, x_lo, ldx, y_hi, y_lo, ldy, c, c_dtype, ldc, accumulate, workspace,
                        workspace_bytes);
}

extern "C" int sj_gemm_planes_split_out(void* stream, long M, long N, long K, const uint16_t* a_hi,
                                         const uint16_t* a_lo, long lda, const uint16_t* b, long ldb, uint16_t* c_hi,
                                         uint16_t* c_lo, long ldc, uint16_t* c_t_hi, uint16_t* c_t_lo, long ldct,
                                         const uint16_t* o, long ldo, float* delta_t, long ld_delta) {
  if (int st0 = sjh::gemm_fast_prepare()) return st0;
  SJ_REQUIRE(M > 0 && N > 0 && K > 0 && K % 8 == 0 && lda % 8 == 0 && ldb % 8 == 0 && lda >= K && ldb >= K &&
                 ldc >= N && (!c_t_hi || (ldct >= M && ldct % 8 == 0)),
             "matmul planes out: M %ld N %ld K %ld (K, ld multiples of 8)", M, N, K);
  SJ_REQUIRE(a_hi && a_lo && b && c_hi && c_lo && !c_t_hi == !c_t_lo && ok16(a_hi) && ok16(a_lo) && ok16(b) &&
                 (!c_t_hi || (ok16(c_t_hi) && ok16(c_t_lo))),
             "matmul planes out: 16-byte aligned operands required (transposed outputs both or neither)");
  SJ_REQUIRE(!delta_t || (o && N % 64 == 0 && ldo % 8 == 0 && ldo >= N && ok16(o) && ld_delta >= M),
             "matmul planes out: Delta needs o [M][ldo] (ldo % 8 == 0) and 64-column heads");
  FParams p = {};
  p.a[0] = (const bf16_t*)a_hi; p.a[1] = (const bf16_t*)a_lo; p.lda = lda;
  p.b[0][0] = (const bf16_t*)b; p.ldb[0] = ldb; p.seg_n[0] = 0; p.nseg = 1;
  p.M = M; p.N = N; p.K = K;
  p.c[0] = c_hi; p.c[1] = c_lo; p.c[2] = c_t_hi; p.c[3] = c_t_lo;
  p.ldc[0] = ldc; p.ldc[2] = ldct;
  p.o = (const bf16_t*)o; p.ldo = ldo; p.delta = delta_t; p.lddelta = ld_delta;
  int bm, bn, splits;
  plan(M, N, K, 2, bm, bn, splits);
  int st = launch_planes<E_PLANES>((hipStream_t)stream, p, 2, 1, bm, bn, 1);
  if (st) return st;
  SJ_LAUNCH_CHECK("matmul planes out");
  return SJ_OK;
}

// project_qkv with q, k, v written to separate buffers (the KV-cache path
// puts k and v straight into the cache rows)
int sjh::qkv_fwd_t_out(void* stream, const uint16_t* x, long ldx, long M, long D, const uint16_t* wqkv_t, long ldw,
                       long N, long KV, uint16_t* q, long ldq, uint16_t* k, long ldk, uint16_t* v, long ldv,
                       const float* rope_table, long rope_t, long head_dim, uint16_t* qkv_t, long ldqt) {
  if (int st0 = sjh::gemm_fast_prepare()) return st0;
  SJ_REQUIRE(M >= 0 && D > 0 && D % 8 == 0 && ldx % 8 == 0 && ldw % 8 == 0 && ldx >= D && ldw >= D && ldq >= N &&
                 ldk >= KV && ldv >= KV && ldq % 8 == 0 && ldk % 8 == 0 && ldv % 8 == 0 && N % 64 == 0 &&
                 KV % 64 == 0 && ok16(x) && ok16(wqkv_t) && ok16(q) && ok16(k) && ok16(v),
             "project_qkv (transposed weights): shape/alignment");
  if (rope_table) SJ_REQUIRE(rope_t > 0 && head_dim > 0 && head_dim % 2 == 0 && N % head_dim == 0 && KV % head_dim == 0 &&
                                 M < (1L << 31),
                             "project_qkv rope: t %ld head_dim %ld", rope_t, head_dim);
  if (M == 0) return SJ_OK;
  FParams p = {};
  p.a[0] = (const bf16_t*)x; p.lda = ldx;
  const bf16_t* w = (const bf16_t*)wqkv_t;
  p.b[0][0] = w; p.b[0][1] = w + N * ldw; p.b[0][2] = w + (N + KV) * ldw;
  p.ldb[0] = p.ldb[1] = p.ldb[2] = ldw;
  p.seg_n[0] = 0; p.seg_n[1] = N; p.seg_n[2] = N + KV; p.nseg = 3;
  p.c[0] = q; p.c[1] = k; p.c[2] = v;
  p.ldc[0] = ldq; p.ldc[1] = ldk; p.ldc[2] = ldv;
  p.M = M; p.N = N + 2 * KV; p.K = D; p.c_bf16 = 1;
  p.rope = rope_table; p.rope_t = rope_t > 0 ? rope_t : 1; p.head_dim = head_dim > 0 ? head_dim : 2;
  p.rope_cols = rope_table ? N + KV : 0;
  if (qkv_t) {
    SJ_REQUIRE(ldq == ldk && ldq == ldv && k == q + N && v == q + N + KV && ldqt >= M && ldqt % 8 == 0 && ok16(qkv_t),
               "project_qkv transposed output: ld %ld (one q|k|v buffer)", ldqt);
    p.c[3] = qkv_t;
    p.ldc[3] = ldqt;
  }
  // 64x128 tiles once they give two per CU (cfg5: 105 -> 96 us), else 64x64
  int bm = 64, bn = tiles(M, N + 2 * KV, 64, 128) >= 2 * cus() && N % 128 == 0 && KV % 128 == 0 ? 128 : 64;
  if (getenv("SJ_GEMM_TILE")) {
    pick(M, N + 2 * KV, bm, bn);
    if (N % bn || KV % bn) bn = 64;
  }
  int st = launch_planes<E_QKV>((hipStream_t)stream, p, 1, 1, bm, bn, 1);
  if (st) return st;
  SJ_LAUNCH_CHECK("project_qkv");
  return SJ_OK;
}

extern "C" int sj_qkv_fwd_t(void* stream, const uint16_t* x, long ldx, long M, long D, const uint16_t* wqkv_t,
                            long ldw, long N, long KV, uint16_t* qkv, long ldo, const float* rope_table, long rope_t,
                            long head_dim, uint16_t* qkv_t, long ldqt) {
  SJ_REQUIRE(ldo >= N + 2 * KV && ldo % 8 == 0 && ok16(qkv), "project_qkv (transposed weights): shape/alignment");
  return sjh::qkv_fwd_t_out(stream, x, ldx, M, D, wqkv_t, ldw, N, KV, qkv, ldo, qkv + N, ldo, qkv + N + KV, ldo,
                            rope_table, rope_t, head_dim, qkv_t, ldqt);
}

extern "C" int sj_gate_up_fwd_t(void* stream, const uint16_t* x, long ldx, long M, long D, const uint16_t* wg_t,
                                const uint16_t* wu_t, long ldw, long F, uint16_t* g, uint16_t* u, uint16_t* h, long ldo,
                                uint16_t* h_t, long ldht) {
  if (int st0 = sjh::gemm_fast_prepare()) return st0;
  SJ_REQUIRE(M >= 0 && D > 0 && D % 8 == 0 && ldx % 8 == 0 && ldw % 8 == 0 && ldx >= D && ldw >= D && ldo >= F &&
                 ok16(x) && ok16(wg_t) && ok16(wu_t) && (!h_t || (ldht >= M && ldht % 4 == 0)),
             "gate_up (transposed weights): shape/alignment");
  if (M == 0) return SJ_OK;
  FParams p = {};
  p.a[0] = (const bf16_t*)x; p.lda = ldx;
  p.b[0][0] = (const bf16_t*)wg_t; p.b[0][1] = (const bf16_t*)wu_t; p.ldb[0] = p.ldb[1] = ldw;
  p.seg_n[0] = 0; p.nseg = 1;
  p.c[0] = g; p.c[1] = u; p.c[2] = h; p.c[3] = h_t; p.ldc[0] = ldo; p.ldc[3] = ldht;
  p.M = M; p.N = F; p.K = D; p.c_bf16 = 1;
  int bm, bn;
  pick(M, F, bm, bn);
  if (bm == 128 && bn == 128) bn = 64;  // dual accumulators: keep the wave tile at 64x32
  int st = launch_planes<E_GATEUP>((hipStream_t)stream, p, 1, 1, bm, bn, 1);
  if (st) return st;
  SJ_LAUNCH_CHECK("gate_up");
  return SJ_OK;
}

extern "C" int sj_linear_residual_fwd_t(void* stream, const uint16_t* x, long ldx, long M, long K,
                                        const uint16_t* w_t, long ldw, long N, const uint16_t* r, long ldr,
                                        uint16_t* y, long ldy) {
  if (int st0 = sjh::gemm_fast_prepare()) return st0;
  SJ_REQUIRE(M >= 0 && K > 0 && K % 8 == 0 && ldx % 8 == 0 && ldw % 8 == 0 && ldx >= K && ldw >= K && ldr >= N &&
                 ldy >= N && ok16(x) && ok16(w_t),
             "linear_residual (transposed weights): shape/alignment");
  if (M == 0) return SJ_OK;
  FParams p = {};
  p.a[0] = (const bf16_t*)x; p.lda = ldx;
  p.b[0][0] = (const bf16_t*)w_t; p.ldb[0] = ldw; p.seg_n[0] = 0; p.nseg = 1;
  p.c[0] = y; p.ldc[0] = ldy; p.r = (const bf16_t*)r; p.ldr = ldr;
  p.M = M; p.N = N; p.K = K; p.c_bf16 = 1;
  int bm, bn;
  pick(M, N, bm, bn);
  int st = launch_planes<E_RESID>((hipStream_t)stream, p, 1, 1, bm, bn, 1);
  if (st) return st;
  SJ_LAUNCH_CHECK("linear_residual");
  return SJ_OK;
}

extern "C" int sj_down_bwd_swiglu_p(void* stream, const uint16_t* dy_hi, const uint16_t* dy_lo, long lddy, long M,
                                    long D, const uint16_t* w_down, long ldw, long F, const uint16_t* g,
                                    const uint16_t* u, long ldgu, uint16_t* dgu_hi, uint16_t* dgu_lo, long lddgu,
                                    uint16_t* dgu_t_hi, uint16_t* dgu_t_lo, long lddgu_t) {
  if (int st0 = sjh::gemm_fast_prepare()) return st0;
  SJ_REQUIRE(M >= 0 && D > 0 && D % 8 == 0 && lddy % 8 == 0 && ldw % 8 == 0 && lddy >= D && ldw >= D && ldgu >= F &&
                 lddgu >= 2 * F && !dgu_t_hi == !dgu_t_lo && (!dgu_t_hi || (lddgu_t >= M && lddgu_t % 4 == 0)) &&
                 ok16(dy_hi) && ok16(dy_lo) && ok16(w_down),
             "swiglu_backward (planes): shape/alignment (transposed outputs both or neither)");
  if (M == 0) return SJ_OK;
  FParams p = {};
  p.a[0] = (const bf16_t*)dy_hi; p.a[1] = (const bf16_t*)dy_lo; p.lda = lddy;
  p.b[0][0] = (const bf16_t*)w_down; p.ldb[0] = ldw; p.seg_n[0] = 0; p.nseg = 1;
  p.c[0] = dgu_hi; p.c[1] = dgu_lo; p.c[2] = dgu_t_hi; p.c[3] = dgu_t_lo; p.ldc[0] = lddgu; p.ldc[2] = lddgu_t;
  p.gin = (const bf16_t*)g; p.uin = (const bf16_t*)u; p.ldgu = ldgu; p.F = F;
  p.M = M; p.N = F; p.K = D;
  int bm, bn, splits;
  plan(M, F, D, 2, bm, bn, splits);
  int st = swiglu_rows_ok(p) ? launch_planes<E_SWIGLU_ROWS>((hipStream_t)stream, p, 2, 1, bm, bn, 1)
                             : launch_planes<E_SWIGLU_BWD>((hipStream_t)stream, p, 2, 1, bm, bn, 1);
  if (st) return st;
  SJ_LAUNCH_CHECK("swiglu_backward");
  return SJ_OK;
}

// ====================================================== grouped (MoE) GEMMs
// Expert segments come from sj_route_pack's device offsets (64-row aligned),
// so no count ever travels to the host: row-mode grids cover the packed
// capacity and workgroups past the last segment leave at once.

namespace {
// Column tile of the grouped expert products (rows: 64, the segment
// alignment).  `narrow`: the dual gate/up forward and the products with a
// split A (gate/up dX, down dX + SwiGLU) take 64 (cfg4: 52.5 -> 47.4,
// 67.1 -> 63.4, 57.5 -> 52.9 us against 128); the expert down forward keeps
// 128 once it gives a tile per CU (25.4 against 31.7 us at 64).
int grouped_bn(long cap, long N, bool narrow = false) {
  static int ov = -1;
  if (ov < 0) {
    const char* e = getenv("SJ_MOE_BN");  // sweeps: 64 or 128
    ov = e ? atoi(e) : 0;
  }
  if (ov == 64 || ov == 128) return ov;
  if (narrow) return 64;
  return tiles(cap, N, 64, 128) >= cus() ? 128 : 64;
}
bool grouped_ok(const int32_t* off, long experts, long cap) {
  return off && experts > 0 && experts <= 1024 && cap > 0 && cap % 64 == 0;
}
}  // namespace

extern "C" int sj_moe_gate_up_fwd(void* stream, const int32_t* offsets, long experts, long capacity,
                                  const uint16_t* x, long ldx, long D, const uint16_t* wg_t, const uint16_t* wu_t,
                                  long ldw, long w_stride, long F, uint16_t* g, uint16_t* u, uint16_t* h, long ldo,
                                  uint16_t* h_t, long ldht) {
  if (int st0 = sjh::gemm_fast_prepare()) return st0;
  SJ_REQUIRE(grouped_ok(offsets, experts, capacity) && D > 0 && D % 8 == 0 && ldx % 8 == 0 && ldw % 8 == 0 &&
                 ldx >= D && ldw >= D && ldo >= F && w_stride % 8 == 0 && ok16(x) && ok16(wg_t) && ok16(wu_t) &&
                 (!h_t || (ldht >= capacity && ldht % 4 == 0)),
             "expert gate_up: shape/alignment (capacity %ld must be a multiple of 64)", capacity);
  FParams p = {};
  p.a[0] = (const bf16_t*)x; p.lda = ldx;
  p.b[0][0] = (const bf16_t*)wg_t; p.b[0][1] = (const bf16_t*)wu_t; p.ldb[0] = p.ldb[1] = ldw;
  p.seg_n[0] = 0; p.nseg = 1;
  p.c[0] = g; p.c[1] = u; p.c[2] = h; p.c[3] = h_t; p.ldc[0] = ldo; p.ldc[3] = ldht;
  p.M = capacity; p.N = F; p.K = D; p.c_bf16 = 1;
  p.goff = offsets; p.gE = (int)experts; p.gmode = 1; p.gstride_b = w_stride;
  int st = launch_planes<E_GATEUP>((hipStream_t)stream, p, 1, 1, 64, grouped_bn(capacity, F, true), 1);
  if (st) return st;
  SJ_LAUNCH_CHECK("expert gate_up");
  return SJ_OK;
}

extern "C" int sj_moe_down_fwd(void* stream, const int32_t* offsets, long experts, long capacity, const uint16_t* h,
                               long ldh, long F, const uint16_t* wd_t, long ldw, long w_stride, long D, uint16_t* y,
                               long ldy) {
  if (int st0 = sjh::gemm_fast_prepare()) return st0;
  SJ_REQUIRE(grouped_ok(offsets, experts, capacity) && F > 0 && F % 8 == 0 && ldh % 8 == 0 && ldw % 8 == 0 &&
                 ldh >= F && ldw >= F && ldy >= D && w_stride % 8 == 0 && ok16(h) && ok16(wd_t),
             "expert down: shape/alignment");
  FParams p = {};
  p.a[0] = (const bf16_t*)h; p.lda = ldh;
  p.b[0][0] = (const bf16_t*)wd_t; p.ldb[0] = ldw; p.seg_n[0] = 0; p.nseg = 1;
  p.c[0] = y; p.ldc[0] = ldy; p.c_bf16 = 1;
  p.M = capacity; p.N = D; p.K = F;
  p.goff = offsets; p.gE = (int)experts; p.gmode = 1; p.gstride_b = w_stride;
  int st = launch_planes<E_STORE>((hipStream_t)stream, p, 1, 1, 64, grouped_bn(capacity, D), 1);
  if (st) return st;
  SJ_LAUNCH_CHECK("expert down");
  return SJ_OK;
}

extern "C" int sj_moe_down_bwd_swiglu_p(void* stream, const int32_t* offsets, long experts, long capacity,
                                        const uint16_t* dy_hi, const uint16_t* dy_lo, long lddy, long D,
                                        const uint16_t* w_down, long ldw, long w_stride, long F, const uint16_t* g,
                                        const uint16_t* u, long ldgu, uint16_t* dgu_hi, uint16_t* dgu_lo, long lddgu,
                                        uint16_t* dgu_t_hi, uint16_t* dgu_t_lo, long ldt) {
  if (int st0 = sjh::gemm_fast_prepare()) return st0;
  SJ_REQUIRE(grouped_ok(offsets, experts, capacity) && D > 0 && D % 8 == 0 && lddy % 8 == 0 && ldw % 8 == 0 &&
                 lddy >= D && ldw >= D && ldgu >= F && lddgu >= 2 * F && !dgu_t_hi == !dgu_t_lo &&
                 (!dgu_t_hi || (ldt >= capacity && ldt % 4 == 0)) && w_stride % 8 == 0 && ok16(dy_hi) &&
                 ok16(dy_lo) && ok16(w_down),
             "expert swiglu_backward: shape/alignment (transposed outputs both or neither)");
  FParams p = {};
  p.a[0] = (const bf16_t*)dy_hi; p.a[1] = (const bf16_t*)dy_lo; p.lda = lddy;
  p.b[0][0] = (const bf16_t*)w_down; p.ldb[0] = ldw; p.seg_n[0] = 0; p.nseg = 1;
  p.c[0] = dgu_hi; p.c[1] = dgu_lo; p.c[2] = dgu_t_hi; p.c[3] = dgu_t_lo; p.ldc[0] = lddgu; p.ldc[2] = ldt;
  p.gin = (const bf16_t*)g; p.uin = (const bf16_t*)u; p.ldgu = ldgu; p.F = F;
  p.M = capacity; p.N = F; p.K = D;
  p.goff = offsets; p.gE = (int)experts; p.gmode = 1; p.gstride_b = w_stride;
  const int bn = grouped_bn(capacity, F, true);
  int st = swiglu_rows_ok(p) ? launch_planes<E_SWIGLU_ROWS>((hipStream_t)stream, p, 2, 1, 64, bn, 1)
                             : launch_planes<E_SWIGLU_BWD>((hipStream_t)stream, p, 2, 1, 64, bn, 1);
  if (st) return st;
  SJ_LAUNCH_CHECK("expert swiglu_backward");
  return SJ_OK;
}

extern "C" int sj_moe_gemm_rows(void* stream, const int32_t* offsets, long experts, long capacity, long N, long K,
                                const uint16_t* a_hi, const uint16_t* a_lo, long lda, const uint16_t* b, long ldb,
                                long b_stride, float* c, long ldc, int accumulate) {
  if (int st0 = sjh::gemm_fast_prepare()) return st0;
  SJ_REQUIRE(grouped_ok(offsets, experts, capacity) && N > 0 && K > 0 && K % 8 == 0 && lda % 8 == 0 && ldb % 8 == 0 &&
                 lda >= K && ldb >= K && ldc >= N && b_stride % 8 == 0 && ok16(a_hi) && (!a_lo || ok16(a_lo)) &&
                 ok16(b),
             "expert matmul (rows): shape/alignment");
  FParams p = {};
  p.a[0] = (const bf16_t*)a_hi; p.a[1] = (const bf16_t*)a_lo; p.lda = lda;
  p.b[0][0] = (const bf16_t*)b; p.ldb[0] = ldb; p.seg_n[0] = 0; p.nseg = 1;
  p.c[0] = c; p.ldc[0] = ldc; p.accumulate = accumulate;
  p.M = capacity; p.N = N; p.K = K;
  p.goff = offsets; p.gE = (int)experts; p.gmode = 1; p.gstride_b = b_stride;
  int st = launch_planes<E_STORE>((hipStream_t)stream, p, a_lo ? 2 : 1, 1, 64, grouped_bn(capacity, N, a_lo != nullptr), 1);
  if (st) return st;
  SJ_LAUNCH_CHECK("expert matmul (rows)");
  return SJ_OK;
}

// Per-expert dW from row-layout operands: C_e (+ e * c_stride) [M][N] =
// X_e^T Y_e over expert e's packed rows [offsets[e], offsets[e+1]) with
// X [capacity][ldx] (M columns) and Y [capacity][ldy] (N columns, hi/lo).
extern "C" int sj_moe_gemm_dw_tn(void* stream, const int32_t* offsets, long experts, long capacity, long M, long N,
                                 const uint16_t* x, long ldx, const uint16_t* y_hi, const uint16_t* y_lo, long ldy,
                                 float* c, long ldc, long c_stride) {
  if (int st0 = sjh::gemm_fast_prepare()) return st0;
  SJ_REQUIRE(grouped_ok(offsets, experts, capacity) && experts <= 65535 && M > 0 && N > 0 && M % 8 == 0 &&
                 N % 8 == 0 && ldx % 8 == 0 && ldy % 8 == 0 && ldx >= M && ldy >= N && ldc >= N && ok16(x) &&
                 ok16(y_hi) && (!y_lo || ok16(y_lo)),
             "expert matmul (dW, row-layout operands): shape/alignment");
  FParams p = {};
  p.a[0] = (const bf16_t*)x; p.lda = ldx;
  p.b[0][0] = (const bf16_t*)y_hi; p.b[1][0] = (const bf16_t*)y_lo; p.ldb[0] = ldy; p.seg_n[0] = 0; p.nseg = 1;
  p.c[0] = c; p.ldc[0] = ldc;
  p.M = M; p.N = N; p.K = capacity;
  p.goff = offsets; p.gE = (int)experts; p.gmode = 2; p.gstride_c = c_stride;
  // split dY: 128 x 64 tiles, so a stage holds as many A rows (128) as
  // B rows (2 planes x 64), with two stages (two workgroups per CU).  cfg4
  // (8 experts of about 1024 tokens): gate/up dW 95 -> 71 us, down dW 54 ->
  // 44 us against 128 x 128 (one workgroup per CU); 64 x 64 and 64 x 128
  // land between.  One plane: the general tile heuristic.
  int bm = 128, bn = 64;
  if (!y_lo) pick(M * experts, N, bm, bn);
  if (const char* e = getenv("SJ_MOE_DW_TILE")) {  // sweeps
    int a = 0, b = 0;
    if (sscanf(e, "%dx%d", &a, &b) == 2 && (a == 64 || a == 128) && (b == 64 || b == 128)) { bm = a; bn = b; }
  }
  int st = launch_planes<E_STORE, 3>((hipStream_t)stream, p, 1, y_lo ? 2 : 1, bm, bn, (int)experts);
  if (st) return st;
  SJ_LAUNCH_CHECK("expert matmul (dW, row layout)");
  return SJ_OK;
}

extern "C" int sj_moe_gemm_dw(void* stream, const int32_t* offsets, long experts, long capacity, long M, long N,
                              const uint16_t* a, long lda, const uint16_t* b_hi, const uint16_t* b_lo, long ldb,
                              float* c, long ldc, long c_stride) {
  if (int st0 = sjh::gemm_fast_prepare()) return st0;
  SJ_REQUIRE(grouped_ok(offsets, experts, capacity) && experts <= 65535 && M > 0 && N > 0 && lda % 8 == 0 &&
                 ldb % 8 == 0 && lda >= capacity && ldb >= capacity && ldc >= N && ok16(a) && ok16(b_hi) &&
                 (!b_lo || ok16(b_lo)),
             "expert matmul (dW): shape/alignment");
  FParams p = {};
  p.a[0] = (const bf16_t*)a; p.lda = lda;
  p.b[0][0] = (const bf16_t*)b_hi; p.b[1][0] = (const bf16_t*)b_lo; p.ldb[0] = ldb; p.seg_n[0] = 0; p.nseg = 1;
  p.c[0] = c; p.ldc[0] = ldc;
  p.M = M; p.N = N; p.K = capacity;
  p.goff = offsets; p.gE = (int)experts; p.gmode = 2; p.gstride_c = c_stride;
  int bm, bn;
  pick(M * experts, N, bm, bn);
  int st = launch_planes<E_STORE>((hipStream_t)stream, p, 1, b_lo ? 2 : 1, bm, bn, (int)experts);
  if (st) return st;
  SJ_LAUNCH_CHECK("expert matmul (dW)");
  return SJ_OK;
}
