// Mixture-of-experts FFN around the grouped GEMMs (gfx950).
//
// The reference runs the MoE FFN of Block::apply (crates/sejong-model/src/
// architecture.rs:229-242) as: router matmul -> route_topk -> expert_routes
// (pack + a D2H read of the counts, hierarchy_ops.rs:331-378) -> per expert
// gather + gate_up + down -> expert_combine (fp32 atomics).  Here:
//   k_router_topk   router logits (bf16, as the reference stores them) and
//                   top-k routing in one pass, one wavefront per token;
//   k_route_pack    one workgroup: per-expert counts, 64-row aligned segment
//                   offsets and a stable slot-ordered packing, all on device;
//   k_moe_gather    packed expert inputs (zero padding rows) and their
//                   transpose (the dW operand);
//   grouped GEMMs   (gemm_fast.hip) run every expert in one launch;
//   k_moe_combine   weighted sum of a token's expert outputs in ascending
//                   expert order (the order the reference's per-expert
//                   launches add in) + the residual add;
// and the backward: k_moe_combine_bwd (dX of each expert output as hi/lo
// planes, normal and transposed, and the routing-weight gradient) and
// k_moe_gather_bwd (route_topk backward + router dX + the gather's
// scatter-add, summed per token without atomics).
#include <math.h>
#include <stdlib.h>

#include "common.h"

using namespace sj;

namespace {

constexpr int NT = 256;
constexpr int EMAX = 32;  // experts per layer supported by these kernels
constexpr int KMAX = 8;   // top-k
constexpr int SEG = 64;   // expert segment alignment in the packed layout

long pack_capacity(long S, long E) { return (S + (SEG - 1) * E + SEG - 1) / SEG * SEG; }

// top-k of E scores (registers, unrolled over EMAX): softmax over all E,
// K rounds of argmax with the lowest index on ties, weight = full-softmax
// probability (hierarchy.py:175-191)
template <int EM = EMAX>  // the score arrays' bound (E <= EM)
__device__ __forceinline__ void topk_rows(const float* sc_in, int E, int K, int32_t* ids, float* wout) {
  float sc[EM];
  float mx = -INFINITY;
#pragma unroll
  for (int e = 0; e < EM; e++) {
    sc[e] = e < E ? sc_in[e] : -INFINITY;
    mx = fmaxf(mx, sc[e]);
  }
  float den = 0.f;
#pragma unroll
  for (int e = 0; e < EM; e++)
    if (e < E) den += expf(sc[e] - mx);
#pragma unroll
  for (int k = 0; k < KMAX; k++) {
    if (k >= K) break;
    float best = -INFINITY;
    int idx = E;
#pragma unroll
    for (int e = 0; e < EM; e++)
      if (e < E && (sc[e] > best || (idx == E && sc[e] == best))) {
        best = sc[e];
        idx = e;
      }
    ids[k] = idx;
    wout[k] = expf(best - mx) / den;
#pragma unroll
    for (int e = 0; e < EM; e++)
      if (e == idx) sc[e] = -INFINITY;
  }
}

// logits = round_bf16(z W_r) (W_r [d][E] bf16), then routing.  One wave
// per token; lane l accumulates columns l, l+64, ... for every expert.
__global__ __launch_bounds__(NT) void k_router_topk(const bf16_t* __restrict__ z, long ldz, const bf16_t* __restrict__ wr,
                                                    long d, long R, int E, int K, bf16_t* __restrict__ logits,
                                                    int32_t* __restrict__ ids, float* __restrict__ weights) {
  const int lane = threadIdx.x & 63;
  const long r = blockIdx.x * 4L + (threadIdx.x >> 6);
  if (r >= R) return;
  float acc[EMAX];
#pragma unroll
  for (int e = 0; e < EMAX; e++) acc[e] = 0.f;
  for (long c = lane; c < d; c += 64) {
    const float zv = bf2f(z[r * ldz + c]);
#pragma unroll
    for (int e = 0; e < EMAX; e++)
      if (e < E) acc[e] += zv * bf2f(wr[c * E + e]);
  }
  float sc[EMAX];
#pragma unroll
  for (int e = 0; e < EMAX; e++) {
    sc[e] = 0.f;
    if (e < E) sc[e] = round_bf(wave_sum(acc[e]));
  }
  if (lane == 0) {
#pragma unroll
    for (int e = 0; e < EMAX; e++)
      if (e < E) logits[r * E + e] = f2bf(sc[e]);
    int32_t id[KMAX];
    float w[KMAX];
    topk_rows(sc, E, K, id, w);
#pragma unroll
    for (int k = 0; k < KMAX; k++)
      if (k < K) {
        ids[r * K + k] = id[k];
        weights[r * K + k] = w[k];
      }
  }
}

// The same with LPT lanes per token (64 / LPT tokens per wave; d a multiple
// of 8 LPT, E of 8, aligned rows): lane j of a token accumulates columns
// 8j .. 8j+7 (+ 8 LPT i) for every expert from 16-byte chunks of z and
// W_r, an xor tree over the token's lanes adds the sums (the same bits on
// every lane: each add is commutative), and the token's first lane rounds
// the logits, stores them and runs the top-k.  Against one wave per token,
// the reduction takes log2(LPT) steps instead of 6 and the serial top-k
// runs for 64 / LPT tokens per wave at once.
template <int EW, int LPT>
__global__ __launch_bounds__(NT) void k_router_topk_lanes(const bf16_t* __restrict__ z, long ldz,
                                                          const bf16_t* __restrict__ wr, long d, long R, int E, int K,
                                                          bf16_t* __restrict__ logits, int32_t* __restrict__ ids,
                                                          float* __restrict__ weights, int32_t* __restrict__ hist) {
  constexpr int EE = 8 * EW;
  const int j = threadIdx.x % LPT;
  const long r = (blockIdx.x * (long)NT + threadIdx.x) / LPT;
  const bool live = r < R;
  float acc[EE];
#pragma unroll
  for (int e = 0; e < EE; e++) acc[e] = 0.f;
  if (live) {
    for (long c8 = 8L * j; c8 < d; c8 += 8 * LPT) {
      const u32x4 zv = *(const u32x4*)(z + r * ldz + c8);
      float zf[8];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        zf[2 * i] = __uint_as_float(zv[i] << 16);
        zf[2 * i + 1] = __uint_as_float(zv[i] & 0xffff0000u);
      }
#pragma unroll
      for (int i = 0; i < 8; i++) {
        const bf16_t* wrow = wr + (c8 + i) * E;
#pragma unroll
        for (int e8 = 0; e8 < EE; e8 += 8) {
          if (e8 >= E) break;
          const u32x4 wv = *(const u32x4*)(wrow + e8);
#pragma unroll
          for (int q = 0; q < 4; q++) {
            acc[e8 + 2 * q] += zf[i] * __uint_as_float(wv[q] << 16);
            acc[e8 + 2 * q + 1] += zf[i] * __uint_as_float(wv[q] & 0xffff0000u);
          }
        }
      }
    }
  }
#pragma unroll
  for (int o = 1; o < LPT; o <<= 1)
#pragma unroll
    for (int e = 0; e < EE; e++) acc[e] += __shfl_xor(acc[e], o, WAVE);
  // hist (uniform): this workgroup's routed-slot count per expert, for the
  // pack that follows (integer adds, so their order does not matter)
  __shared__ int hcnt[EMAX];
  if (hist) {
    if (threadIdx.x < EMAX) hcnt[threadIdx.x] = 0;
    __syncthreads();
  }
  if (live && j == 0) {
  float sc[EMAX];
#pragma unroll
  for (int e = 0; e < EMAX; e++) sc[e] = e < EE && e < E ? round_bf(acc[e < EE ? e : 0]) : 0.f;
#pragma unroll
  for (int e8 = 0; e8 < EE; e8 += 8)
    if (e8 < E)
      *(u32x4*)(logits + r * E + e8) = u32x4{pack2(f2bf(sc[e8]), f2bf(sc[e8 + 1])), pack2(f2bf(sc[e8 + 2]), f2bf(sc[e8 + 3])),
                                             pack2(f2bf(sc[e8 + 4]), f2bf(sc[e8 + 5])), pack2(f2bf(sc[e8 + 6]), f2bf(sc[e8 + 7]))};
  int32_t id[KMAX];
  float w[KMAX];
  topk_rows<EE>(sc, E, K, id, w);
#pragma unroll
  for (int k = 0; k < KMAX; k++)
    if (k < K) {
      ids[r * K + k] = id[k];
      weights[r * K + k] = w[k];
      if (hist) atomicAdd(&hcnt[id[k]], 1);
    }
  }
  if (hist) {
    __syncthreads();
    if (threadIdx.x < E) hist[blockIdx.x * (long)E + threadIdx.x] = hcnt[threadIdx.x];
  }
}

// The pack (k_route_pack_wide's result) from the top-k workgroups' counts:
// workgroup b places the K-slots of top-k workgroup b's tokens (slots
// b * per .. b * per + per - 1, per <= 64, one per lane).  Its base in
// expert e's segment is the count of e in workgroups 0 .. b - 1, and the
// rank among its own slots of expert e is that of the lanes below with the
// same expert (a ballot per expert): every segment lists its slots in slot
// order, as the single-workgroup scan does.  Workgroup 0 also writes the
// counts and offsets and marks the segments' padding and the tail empty.
__global__ __launch_bounds__(64) void k_route_pack_hist(const int32_t* __restrict__ ids, long S, int E, long cap,
                                                        const int32_t* __restrict__ hist, int nblk, int per,
                                                        int32_t* __restrict__ counts, int32_t* __restrict__ offsets,
                                                        int32_t* __restrict__ pslot, int32_t* __restrict__ ppos) {
  constexpr int EP = 8;  // experts covered (E <= 8)
  const int lane = threadIdx.x, b = blockIdx.x;
  int tot[EP], base[EP];
#pragma unroll
  for (int e = 0; e < EP; e++) tot[e] = base[e] = 0;
  for (int r = lane; r < nblk; r += 64)
#pragma unroll
    for (int e = 0; e < EP; e++)
      if (e < E) {
        const int v = hist[(long)r * E + e];
        tot[e] += v;
        if (r < b) base[e] += v;
      }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1)
#pragma unroll
    for (int e = 0; e < EP; e++) {
      tot[e] += __shfl_xor(tot[e], o, WAVE);
      base[e] += __shfl_xor(base[e], o, WAVE);
    }
  int off[EP + 1];
  int o = 0;
#pragma unroll
  for (int e = 0; e < EP; e++) {
    off[e] = o;
    if (e < E) o += (tot[e] + SEG - 1) / SEG * SEG;
  }
  off[EP] = o;  // == off[E]
  const long s = (long)b * per + lane;
  const bool has = lane < per && s < S;
  const int ex = has ? ids[s] : -1;
  int pos = 0;
  const uint64_t below = (1ull << lane) - 1ull;
#pragma unroll
  for (int e = 0; e < EP; e++) {
    if (e >= E) break;
    const uint64_t m = __ballot(ex == e);
    if (ex == e) pos = off[e] + base[e] + __popcll(m & below);
  }
  if (has) {
    pslot[pos] = (int32_t)s;
    ppos[s] = pos;
  }
  if (b != 0) return;
#pragma unroll
  for (int e = 0; e < EP; e++) {
    if (e >= E) break;
    if (lane == 0) {
      offsets[e] = off[e];
      if (counts) counts[e] = tot[e];
    }
    for (long i = off[e] + tot[e] + lane; i < off[e + 1 < EP ? e + 1 : EP]; i += 64) pslot[i] = -1;
  }
  if (lane == 0) offsets[E] = off[EP];
  for (long i = off[EP] + lane; i < cap; i += 64) pslot[i] = -1;
}

// The same with 16-byte loads (d % 8 == 0, E % 8 == 0, aligned rows): lane
// l accumulates columns 8l .. 8l+7 (+ 512 i) for every expert from one z
// chunk and the matching E-wide rows of W_r, then the wave sums.
__global__ __launch_bounds__(NT) void k_router_topk8(const bf16_t* __restrict__ z, long ldz,
                                                     const bf16_t* __restrict__ wr, long d, long R, int E, int K,
                                                     bf16_t* __restrict__ logits, int32_t* __restrict__ ids,
                                                     float* __restrict__ weights) {
  const int lane = threadIdx.x & 63;
  const long r = blockIdx.x * 4L + (threadIdx.x >> 6);
  if (r >= R) return;
  float acc[EMAX];
#pragma unroll
  for (int e = 0; e < EMAX; e++) acc[e] = 0.f;
  for (long c8 = 8L * lane; c8 < d; c8 += 512) {
    const u32x4 zv = *(const u32x4*)(z + r * ldz + c8);
    float zf[8];
#pragma unroll
    for (int i = 0; i < 4; i++) {
      zf[2 * i] = __uint_as_float(zv[i] << 16);
      zf[2 * i + 1] = __uint_as_float(zv[i] & 0xffff0000u);
    }
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const bf16_t* wrow = wr + (c8 + i) * E;
#pragma unroll
      for (int e8 = 0; e8 < EMAX; e8 += 8) {
        if (e8 >= E) break;
        const u32x4 wv = *(const u32x4*)(wrow + e8);
#pragma unroll
        for (int q = 0; q < 4; q++) {
          acc[e8 + 2 * q] += zf[i] * __uint_as_float(wv[q] << 16);
          acc[e8 + 2 * q + 1] += zf[i] * __uint_as_float(wv[q] & 0xffff0000u);
        }
      }
    }
  }
  float sc[EMAX];
#pragma unroll
  for (int e = 0; e < EMAX; e++) {
    sc[e] = 0.f;
    if (e < E) sc[e] = round_bf(wave_sum(acc[e]));
  }
  if (lane == 0) {
#pragma unroll
    for (int e = 0; e < EMAX; e++)
      if (e < E) logits[r * E + e] = f2bf(sc[e]);
    int32_t id[KMAX];
    float w[KMAX];
    topk_rows(sc, E, K, id, w);
#pragma unroll
    for (int k = 0; k < KMAX; k++)
      if (k < K) {
        ids[r * K + k] = id[k];
        weights[r * K + k] = w[k];
      }
  }
}

// routing from stored logits (Engine::route_topk), one thread per row
__global__ __launch_bounds__(NT) void k_route_topk(const void* __restrict__ x, int xd, long R, int E, int K,
                                                   int32_t* __restrict__ ids, float* __restrict__ weights) {
  const long r = blockIdx.x * (long)NT + threadIdx.x;
  if (r >= R) return;
  float sc[EMAX];
#pragma unroll
  for (int e = 0; e < EMAX; e++) sc[e] = e < E ? load_as_f32(x, xd, r * E + e) : 0.f;
  int32_t id[KMAX];
  float w[KMAX];
  topk_rows(sc, E, K, id, w);
#pragma unroll
  for (int k = 0; k < KMAX; k++)
    if (k < K) {
      ids[r * K + k] = id[k];
      weights[r * K + k] = w[k];
    }
}

// Engine::route_topk_backward (hierarchy.py:194-209): dx = p (dy_sel - sum_k w_k dy_k)
template <int EM = EMAX>  // EM: the arrays' bound (E <= EM)
__device__ __forceinline__ void route_bwd_row(const float* lg, int E, int K, const int32_t* id, const float* w,
                                              const float* dy, float* dx) {
  float mx = -INFINITY;
#pragma unroll
  for (int e = 0; e < EM; e++)
    if (e < E) mx = fmaxf(mx, lg[e]);
  float den = 0.f, ex[EM];
#pragma unroll
  for (int e = 0; e < EM; e++) {
    ex[e] = e < E ? expf(lg[e] - mx) : 0.f;
    den += ex[e];
  }
  float total = 0.f, sel[EM];
#pragma unroll
  for (int e = 0; e < EM; e++) sel[e] = 0.f;
#pragma unroll
  for (int k = 0; k < KMAX; k++) {
    if (k >= K) break;
    total += w[k] * dy[k];
#pragma unroll
    for (int e = 0; e < EM; e++)
      if (e == id[k]) sel[e] += dy[k];
  }
#pragma unroll
  for (int e = 0; e < EM; e++)
    if (e < E) dx[e] = ex[e] / den * (sel[e] - total);
}

__global__ __launch_bounds__(NT) void k_route_topk_bwd(const void* __restrict__ x, int xd, const int32_t* __restrict__ ids,
                                                       const float* __restrict__ weights, const float* __restrict__ dy,
                                                       float* __restrict__ dx, long R, int E, int K) {
  const long r = blockIdx.x * (long)NT + threadIdx.x;
  if (r >= R) return;
  float lg[EMAX], d[EMAX], w[KMAX], g[KMAX];
  int32_t id[KMAX];
#pragma unroll
  for (int e = 0; e < EMAX; e++) lg[e] = e < E ? load_as_f32(x, xd, r * E + e) : 0.f;
#pragma unroll
  for (int k = 0; k < KMAX; k++) {
    id[k] = k < K ? ids[r * K + k] : -1;
    w[k] = k < K ? weights[r * K + k] : 0.f;
    g[k] = k < K ? dy[r * K + k] : 0.f;
  }
  route_bwd_row(lg, E, K, id, w, g, d);
#pragma unroll
  for (int e = 0; e < EMAX; e++)
    if (e < E) dx[r * E + e] = d[e];
}

// Engine::expert_routes (hierarchy_route_pack, hierarchy.py:212-225) without
// the host read: one workgroup.  Thread t owns slots [t*chunk, (t+1)*chunk);
// per-expert counts of each thread are scanned (one wavefront per expert) to
// give every slot its stable rank, the segments are laid out at 64-row
// aligned offsets, and padding rows get slot -1.
__global__ __launch_bounds__(NT) void k_route_pack(const int32_t* __restrict__ ids, long S, int K, int E, long cap,
                                                   int32_t* __restrict__ tokens, int32_t* __restrict__ slots,
                                                   int32_t* __restrict__ counts, int32_t* __restrict__ offsets,
                                                   int32_t* __restrict__ pslot, int32_t* __restrict__ ppos) {
  __shared__ int cnt[EMAX][NT];
  __shared__ int tot[EMAX];
  __shared__ int off[EMAX + 1];
  const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
  const long chunk = (S + NT - 1) / NT;
  const long s0 = t * chunk, s1 = s0 + chunk < S ? s0 + chunk : S;
  for (int e = 0; e < E; e++) cnt[e][t] = 0;
  for (long s = s0; s < s1; s++) {
    const int e = ids[s];
    if (e >= 0 && e < E) cnt[e][t]++;
  }
  __syncthreads();
  // exclusive scan of cnt[e][0..NT) per expert: 4 per lane + wave scan
  for (int e = wv; e < E; e += NT / 64) {
    int v[4], sum = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      v[i] = cnt[e][4 * lane + i];
      sum += v[i];
    }
    int incl = sum;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int y = __shfl_up(incl, o, 64);
      if (lane >= o) incl += y;
    }
    int run = incl - sum;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      cnt[e][4 * lane + i] = run;
      run += v[i];
    }
    if (lane == 63) tot[e] = incl;
  }
  __syncthreads();
  if (t == 0) {
    int o = 0;
    for (int e = 0; e < E; e++) {
      off[e] = o;
      o += (tot[e] + SEG - 1) / SEG * SEG;
    }
    off[E] = o;
  }
  __syncthreads();
  if (t <= E) offsets[t] = off[t];
  if (t < E && counts) counts[t] = tot[t];
  for (long s = s0; s < s1; s++) {
    const int e = ids[s];
    if (e < 0 || e >= E) {
      ppos[s] = -1;
      continue;
    }
    const int rank = cnt[e][t]++;
    const int pos = off[e] + rank;
    pslot[pos] = (int32_t)s;
    ppos[s] = pos;
    if (tokens) tokens[(long)e * S + rank] = (int32_t)(s / K);
    if (slots) slots[(long)e * S + rank] = (int32_t)s;
  }
  for (int e = 0; e < E; e++) {
    const long i = off[e] + tot[e] + t;
    if (t < SEG && i < off[e + 1]) pslot[i] = -1;
  }
  for (long i = off[E] + t; i < cap; i += NT) pslot[i] = -1;
}

// The same packing with 1024 threads: each owns a run of ceil(S/1024)
// slots, counts its experts in registers, and one block scan of the counts
// (two experts per 64-bit word) gives every slot its stable rank.
constexpr int PNT = 1024;
__device__ __forceinline__ uint64_t shfl_up64(uint64_t v, int o) {
  const uint32_t lo = __shfl_up((uint32_t)v, o, 64), hi = __shfl_up((uint32_t)(v >> 32), o, 64);
  return ((uint64_t)hi << 32) | lo;
}
template <int EP>  // 64-bit count words (two experts each), E <= 2 EP
__global__ __launch_bounds__(PNT) void k_route_pack_wide(const int32_t* __restrict__ ids, long S, int K, int E, long cap,
                                                         int32_t* __restrict__ tokens, int32_t* __restrict__ slots,
                                                         int32_t* __restrict__ counts, int32_t* __restrict__ offsets,
                                                         int32_t* __restrict__ pslot, int32_t* __restrict__ ppos) {
  constexpr int NW = PNT / 64, EM = 2 * EP;
  __shared__ uint64_t wsum[NW][EP];
  __shared__ int tot[EMAX], off[EMAX + 1];
  const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
  const long per = (S + PNT - 1) / PNT;
  const long s0 = t * per, s1 = s0 + per < S ? s0 + per : S;
  const int EH = (E + 1) / 2;
  // up to 8 of the thread's ids are loaded together and kept for the
  // placement pass (S <= 8192 at one load round)
  constexpr int IB = 8;
  int eid[IB];
  const bool held = per <= IB;
#pragma unroll
  for (int i = 0; i < IB; i++) eid[i] = held && s0 + i < s1 ? ids[s0 + i] : -1;
  uint64_t pc[EP];
#pragma unroll
  for (int j = 0; j < EP; j++) pc[j] = 0;
  for (long s = s0; s < s1; s++) {
    int e = 0;
    if (held) {
#pragma unroll
      for (int i = 0; i < IB; i++)
        if (s - s0 == i) e = eid[i];
    } else {
      e = ids[s];
    }
#pragma unroll
    for (int j = 0; j < EP; j++)
      if (j < EH) pc[j] += (uint64_t)(e == 2 * j) | ((uint64_t)(e == 2 * j + 1) << 32);
  }
  // inclusive scan over the wave, then the waves' totals
  uint64_t incl[EP];
#pragma unroll
  for (int j = 0; j < EP; j++) {
    incl[j] = pc[j];
    if (j >= EH) continue;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const uint64_t y = shfl_up64(incl[j], o);
      if (lane >= o) incl[j] += y;
    }
    if (lane == 63) wsum[wv][j] = incl[j];
  }
  __syncthreads();
  uint64_t before[EP];
#pragma unroll
  for (int j = 0; j < EP; j++) {
    before[j] = 0;
    if (j >= EH) continue;
    uint64_t all = 0;
    for (int w = 0; w < NW; w++) {
      const uint64_t v = wsum[w][j];
      if (w < wv) before[j] += v;
      all += v;
    }
    if (t == 0) {
      tot[2 * j] = (int)(uint32_t)all;
      if (2 * j + 1 < E) tot[2 * j + 1] = (int)(all >> 32);
    }
  }
  __syncthreads();
  if (t == 0) {
    int o = 0;
    for (int e = 0; e < E; e++) {
      off[e] = o;
      o += (tot[e] + SEG - 1) / SEG * SEG;
    }
    off[E] = o;
  }
  __syncthreads();
  if (t <= E) offsets[t] = off[t];
  if (t < E && counts) counts[t] = tot[t];
  int rank[EM];  // this thread's next rank per expert
#pragma unroll
  for (int j = 0; j < EP; j++) {
    const uint64_t ex = before[j] + incl[j] - pc[j];
    rank[2 * j] = (int)(uint32_t)ex;
    rank[2 * j + 1] = (int)(ex >> 32);
  }
  for (long s = s0; s < s1; s++) {
    int e = 0;
    if (held) {
#pragma unroll
      for (int i = 0; i < IB; i++)
        if (s - s0 == i) e = eid[i];
    } else {
      e = ids[s];
    }
    if (e < 0 || e >= E) {
      ppos[s] = -1;
      continue;
    }
    int rk = 0;
#pragma unroll
    for (int q = 0; q < EM; q++)
      if (q == e) rk = rank[q]++;
    const int pos = off[e] + rk;
    pslot[pos] = (int32_t)s;
    ppos[s] = pos;
    if (tokens) tokens[(long)e * S + rk] = (int32_t)(s / K);
    if (slots) slots[(long)e * S + rk] = (int32_t)s;
  }
  for (int e = 0; e < E; e++) {
    const long i = off[e] + tot[e] + t;
    if (t < SEG && i < off[e + 1]) pslot[i] = -1;
  }
  for (long i = off[E] + t; i < cap; i += PNT) pslot[i] = -1;
}

// packed rows: y[p] = x[token of pslot[p]] (zero for padding), plus y^T
// [d][ldt] staged through LDS in blocks of TR rows (d <= 1024)
constexpr int TR = 32;
__global__ __launch_bounds__(NT) void k_moe_gather(const bf16_t* __restrict__ x, long ldx, long d,
                                                   const int32_t* __restrict__ pslot, int K, long cap,
                                                   bf16_t* __restrict__ y, bf16_t* __restrict__ yt, long ldt) {
  extern __shared__ __attribute__((aligned(16))) bf16_t stage[];  // [TR][d]
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const long p0 = blockIdx.x * (long)TR;
  for (int rr = wv; rr < TR; rr += 4) {
    const long p = p0 + rr;
    const int s = p < cap ? pslot[p] : -1;
    const long tok = s >= 0 ? s / K : -1;
    for (long c = 2 * lane; c < d; c += 128) {
      const uint32_t v = tok >= 0 ? *(const uint32_t*)(x + tok * ldx + c) : 0u;
      if (p < cap) *(uint32_t*)(y + p * d + c) = v;
      *(uint32_t*)(stage + rr * d + c) = v;
    }
  }
  if (!yt) return;
  __syncthreads();
  for (long q = threadIdx.x; q < d * (TR / 8); q += NT) {
    const long c = q / (TR / 8);
    const int ch = (int)(q % (TR / 8));
    bf16_t v[8];
#pragma unroll
    for (int i = 0; i < 8; i++) v[i] = stage[(ch * 8 + i) * d + c];
    const long rbase = p0 + ch * 8;
    bf16_t* dst = yt + c * ldt + rbase;
    if (rbase + 8 <= cap)
      *(u32x4*)dst = u32x4{pack2(v[0], v[1]), pack2(v[2], v[3]), pack2(v[4], v[5]), pack2(v[6], v[7])};
  }
}

// the gather without the transposed copy (row-layout dW): one thread per
// 16-byte chunk of a packed row
__global__ __launch_bounds__(NT) void k_moe_gather16(const bf16_t* __restrict__ x, long ldx, long d,
                                                     const int32_t* __restrict__ pslot, int K, long cap,
                                                     bf16_t* __restrict__ y) {
  const long cpr = d / 8, total = cap * cpr;
  for (long q = blockIdx.x * (long)NT + threadIdx.x; q < total; q += (long)gridDim.x * NT) {
    const long p = q / cpr, c = (q - p * cpr) * 8;
    const int s = pslot[p];
    u32x4 v = u32x4{0u, 0u, 0u, 0u};
    if (s >= 0) v = *(const u32x4*)(x + (long)(s / K) * ldx + c);
    *(u32x4*)(y + p * d + c) = v;
  }
}

// a token's K (expert, packed position, weight) in ascending expert order
// (unrolled compare-exchange over KMAX entries; unused entries sort last)
template <int KM = KMAX>  // the route arrays' bound (K <= KM)
__device__ __forceinline__ int token_routes(long t, int K, const int32_t* ids, const int32_t* ppos, const float* w,
                                            int* pos, float* wk) {
  int e[KM], n = 0;
#pragma unroll
  for (int k = 0; k < KM; k++) {
    const int pk = k < K ? ppos[t * K + k] : -1;
    e[k] = pk >= 0 ? ids[t * K + k] : 0x7fffffff;
    pos[k] = pk;
    wk[k] = (pk >= 0 && w) ? w[t * K + k] : 0.f;
    n += pk >= 0;
  }
#pragma unroll
  for (int i = 0; i < KM; i++)
#pragma unroll
    for (int j = 0; j + 1 < KM - i; j++)
      if (e[j] > e[j + 1]) {
        const int te = e[j], tp = pos[j];
        const float tw = wk[j];
        e[j] = e[j + 1]; pos[j] = pos[j + 1]; wk[j] = wk[j + 1];
        e[j + 1] = te; pos[j + 1] = tp; wk[j + 1] = tw;
      }
  return n;
}

// Engine::expert_combine (hierarchy.py:228-235) + the residual add of
// Block::apply (architecture.rs:245): u = bf16(sum_e w*y_e) with each
// product rounded before its add (the reference's atomic_add of weight*value,
// launches in expert order), out = bf16(residual + u).  One wave per token.
template <bool V8, int KM = KMAX>
__global__ __launch_bounds__(NT) void k_moe_combine(const bf16_t* __restrict__ yp, long ldy, long d,
                                                    const int32_t* __restrict__ ids, const int32_t* __restrict__ ppos,
                                                    const float* __restrict__ weights, long R, int K,
                                                    const bf16_t* __restrict__ residual, long ldr,
                                                    bf16_t* __restrict__ out, long ldo) {
  const int lane = threadIdx.x & 63;
  const long t = blockIdx.x * 4L + (threadIdx.x >> 6);
  if (t >= R) return;
  int pos[KM];
  float wk[KM];
  const int n = token_routes<KM>(t, K, ids, ppos, weights, pos, wk);
  if constexpr (V8) {  // 8 columns per lane, 16-byte accesses; the same arithmetic per column
    for (long c = 8 * lane; c < d; c += 512) {
      float a[8];
#pragma unroll
      for (int i = 0; i < 8; i++) a[i] = 0.f;
#pragma unroll
      for (int j = 0; j < KM; j++) {
        if (j >= n) break;
        const u32x4 v = *(const u32x4*)(yp + pos[j] * ldy + c);
        const uint32_t vv[4] = {v[0], v[1], v[2], v[3]};
#pragma unroll
        for (int i = 0; i < 4; i++) {
          a[2 * i] = a[2 * i] + mul_rn(wk[j], bf2f((bf16_t)(vv[i] & 0xffffu)));
          a[2 * i + 1] = a[2 * i + 1] + mul_rn(wk[j], bf2f((bf16_t)(vv[i] >> 16)));
        }
      }
#pragma unroll
      for (int i = 0; i < 8; i++) a[i] = round_bf(a[i]);
      if (residual) {
        const u32x4 r = *(const u32x4*)(residual + t * ldr + c);
        const uint32_t rr[4] = {r[0], r[1], r[2], r[3]};
#pragma unroll
        for (int i = 0; i < 4; i++) {
          a[2 * i] = bf2f((bf16_t)(rr[i] & 0xffffu)) + a[2 * i];
          a[2 * i + 1] = bf2f((bf16_t)(rr[i] >> 16)) + a[2 * i + 1];
        }
      }
      *(u32x4*)(out + t * ldo + c) = u32x4{pack2(f2bf(a[0]), f2bf(a[1])), pack2(f2bf(a[2]), f2bf(a[3])),
                                           pack2(f2bf(a[4]), f2bf(a[5])), pack2(f2bf(a[6]), f2bf(a[7]))};
    }
    return;
  }
  for (long c = 2 * lane; c < d; c += 128) {
    float a = 0.f, b = 0.f;
#pragma unroll
    for (int j = 0; j < KM; j++) {
      if (j >= n) break;
      const uint32_t v = *(const uint32_t*)(yp + pos[j] * ldy + c);
      a = a + mul_rn(wk[j], bf2f((bf16_t)(v & 0xffffu)));
      b = b + mul_rn(wk[j], bf2f((bf16_t)(v >> 16)));
    }
    a = round_bf(a);
    b = round_bf(b);
    if (residual) {
      const uint32_t rv = *(const uint32_t*)(residual + t * ldr + c);
      a = bf2f((bf16_t)(rv & 0xffffu)) + a;
      b = bf2f((bf16_t)(rv >> 16)) + b;
    }
    *(uint32_t*)(out + t * ldo + c) = pack2(f2bf(a), f2bf(b));
  }
}

// Engine::expert_combine_backward (hierarchy.py:238-251) for all experts:
// dx[p] = dy[token] * w[slot] (as hi/lo planes, normal [cap][d] and
// transposed [d][ldt]) and dw[slot] = sum_c y[p][c] dy[token][c].
constexpr int TRB = 16;
__global__ __launch_bounds__(NT) void k_moe_combine_bwd(const bf16_t* __restrict__ yp, long ldy, long d,
                                                        const int32_t* __restrict__ pslot, const float* __restrict__ weights,
                                                        int K, long cap, const float* __restrict__ dy, long lddy,
                                                        bf16_t* __restrict__ hi, bf16_t* __restrict__ lo,
                                                        bf16_t* __restrict__ hit, bf16_t* __restrict__ lot, long ldt,
                                                        float* __restrict__ dw) {
  extern __shared__ __attribute__((aligned(16))) bf16_t stage[];  // hi [TRB][d], lo [TRB][d]
  bf16_t* shi = stage;
  bf16_t* slo = stage + TRB * d;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const long p0 = blockIdx.x * (long)TRB;
  for (int rr = wv; rr < TRB; rr += 4) {
    const long p = p0 + rr;
    const int s = p < cap ? pslot[p] : -1;
    const long tok = s >= 0 ? s / K : -1;
    const float w = s >= 0 ? weights[s] : 0.f;
    float dot = 0.f;
    for (long c = 2 * lane; c < d; c += 128) {
      uint32_t ph = 0u, pl = 0u;
      if (tok >= 0) {
        const float2 g = *(const float2*)(dy + tok * lddy + c);
        const uint32_t yv = *(const uint32_t*)(yp + p * ldy + c);
        dot += bf2f((bf16_t)(yv & 0xffffu)) * g.x + bf2f((bf16_t)(yv >> 16)) * g.y;
        bf16_t ha, la, hb, lb;
        // dx is the fp32 product (the reference stores it in fp32): round it
        // before the split so the lo plane is not formed from a fused product
        split_bf(mul_rn(g.x, w), ha, la);
        split_bf(mul_rn(g.y, w), hb, lb);
        ph = pack2(ha, hb);
        pl = pack2(la, lb);
      }
      if (p < cap) {
        *(uint32_t*)(hi + p * d + c) = ph;
        *(uint32_t*)(lo + p * d + c) = pl;
      }
      *(uint32_t*)(shi + rr * d + c) = ph;
      *(uint32_t*)(slo + rr * d + c) = pl;
    }
    dot = wave_sum(dot);
    if (lane == 0 && s >= 0) dw[s] = dot;
  }
  if (!hit) return;  // no transposed planes (uniform over the block)
  __syncthreads();
  for (long q = threadIdx.x; q < 2 * d * (TRB / 8); q += NT) {
    const int plane = q >= d * (TRB / 8);
    const long qq = plane ? q - d * (TRB / 8) : q;
    const long c = qq / (TRB / 8);
    const int ch = (int)(qq % (TRB / 8));
    const bf16_t* src = plane ? slo : shi;
    bf16_t v[8];
#pragma unroll
    for (int i = 0; i < 8; i++) v[i] = src[(ch * 8 + i) * d + c];
    const long rbase = p0 + ch * 8;
    if (rbase + 8 <= cap)
      *(u32x4*)((plane ? lot : hit) + c * ldt + rbase) =
          u32x4{pack2(v[0], v[1]), pack2(v[2], v[3]), pack2(v[4], v[5]), pack2(v[6], v[7])};
  }
}

// The combine backward without transposed planes (row-layout dW): one wave
// per packed row, 8 columns per lane in 16- and 32-byte accesses; dx and its
// planes as above, dw summed per lane over its columns in order, then across
// the wave.
__global__ __launch_bounds__(NT) void k_moe_combine_bwd8(const bf16_t* __restrict__ yp, long ldy, long d,
                                                         const int32_t* __restrict__ pslot,
                                                         const float* __restrict__ weights, int K, long cap,
                                                         const float* __restrict__ dy, long lddy,
                                                         bf16_t* __restrict__ hi, bf16_t* __restrict__ lo,
                                                         float* __restrict__ dw) {
  const int lane = threadIdx.x & 63;
  const long p = blockIdx.x * 4L + (threadIdx.x >> 6);
  if (p >= cap) return;
  const int s = pslot[p];
  const long tok = s >= 0 ? s / K : -1;
  const float w = s >= 0 ? weights[s] : 0.f;
  float dot = 0.f;
  for (long c = 8 * lane; c < d; c += 512) {
    u32x4 ph = u32x4{0u, 0u, 0u, 0u}, pl = u32x4{0u, 0u, 0u, 0u};
    if (tok >= 0) {
      const float4 g0 = *(const float4*)(dy + tok * lddy + c), g1 = *(const float4*)(dy + tok * lddy + c + 4);
      const u32x4 yv = *(const u32x4*)(yp + p * ldy + c);
      const float g[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
      bf16_t h[8], l[8];
#pragma unroll
      for (int i = 0; i < 8; i++) {
        const uint32_t word = yv[i >> 1];
        dot += bf2f((bf16_t)((i & 1) ? word >> 16 : word & 0xffffu)) * g[i];
        split_bf(mul_rn(g[i], w), h[i], l[i]);
      }
      ph = u32x4{pack2(h[0], h[1]), pack2(h[2], h[3]), pack2(h[4], h[5]), pack2(h[6], h[7])};
      pl = u32x4{pack2(l[0], l[1]), pack2(l[2], l[3]), pack2(l[4], l[5]), pack2(l[6], l[7])};
    }
    *(u32x4*)(hi + p * d + c) = ph;
    *(u32x4*)(lo + p * d + c) = pl;
  }
  dot = wave_sum(dot);
  if (lane == 0 && s >= 0) dw[s] = dot;
}

// Per token: route_topk backward (dlogits), router dX (dlogits W_r^T,
// W_r [d][E] bf16), the gather's scatter-add (sum of the token's expert
// input gradients in ascending expert order) and the tape's accumulation
// into dz_acc.  One wave per token; no atomics.
__global__ __launch_bounds__(NT) void k_moe_gather_bwd(const float* __restrict__ dxp, long lddx, long d,
                                                       const int32_t* __restrict__ ids, const int32_t* __restrict__ ppos,
                                                       const float* __restrict__ weights, const bf16_t* __restrict__ logits,
                                                       const float* __restrict__ dweights, const bf16_t* __restrict__ wr,
                                                       long R, int K, int E, const float* __restrict__ acc, long ldacc,
                                                       float* __restrict__ dz, long lddz, float* __restrict__ dlogits) {
  const int lane = threadIdx.x & 63;
  const long t = blockIdx.x * 4L + (threadIdx.x >> 6);
  if (t >= R) return;
  float dl[EMAX];
#pragma unroll
  for (int e = 0; e < EMAX; e++) dl[e] = 0.f;
  if (logits) {
    float lg[EMAX], w[KMAX], g[KMAX];
    int32_t id[KMAX];
#pragma unroll
    for (int e = 0; e < EMAX; e++) lg[e] = e < E ? bf2f(logits[t * E + e]) : 0.f;
#pragma unroll
    for (int k = 0; k < KMAX; k++) {
      id[k] = k < K ? ids[t * K + k] : -1;
      w[k] = k < K ? weights[t * K + k] : 0.f;
      g[k] = k < K ? dweights[t * K + k] : 0.f;
    }
    route_bwd_row(lg, E, K, id, w, g, dl);
    if (lane < E) {
      float v = 0.f;
#pragma unroll
      for (int e = 0; e < EMAX; e++)
        if (e == lane) v = dl[e];
      dlogits[t * E + lane] = v;
    }
  }
  int pos[KMAX];
  float unused[KMAX];
  const int n = token_routes(t, K, ids, ppos, nullptr, pos, unused);
  for (long c = lane; c < d; c += 64) {
    float s = acc ? acc[t * ldacc + c] : 0.f;
    float ex = 0.f;
#pragma unroll
    for (int j = 0; j < KMAX; j++)
      if (j < n) ex += dxp[pos[j] * lddx + c];
    s += ex;
    if (logits && wr) {
      float r = 0.f;
#pragma unroll
      for (int e = 0; e < EMAX; e++)
        if (e < E) r += dl[e] * bf2f(wr[c * E + e]);
      s += r;
    }
    dz[t * lddz + c] = s;
  }
}

// k_moe_gather_bwd with 8 consecutive columns per lane per step (16-byte
// loads and stores; d % 8 == 0, E % 8 == 0, row strides multiples of 4):
// every column's arithmetic is the same as above, in the same order.
template <int EM, int KM = KMAX>  // the expert and route arrays' bounds (E <= EM, K <= KM)
__global__ __launch_bounds__(NT) void k_moe_gather_bwd8(const float* __restrict__ dxp, long lddx, long d,
                                                        const int32_t* __restrict__ ids, const int32_t* __restrict__ ppos,
                                                        const float* __restrict__ weights,
                                                        const bf16_t* __restrict__ logits,
                                                        const float* __restrict__ dweights,
                                                        const bf16_t* __restrict__ wr, long R, int K, int E,
                                                        const float* __restrict__ acc, long ldacc,
                                                        float* __restrict__ dz, long lddz,
                                                        float* __restrict__ dlogits) {
  const int lane = threadIdx.x & 63;
  const long t = blockIdx.x * 4L + (threadIdx.x >> 6);
  if (t >= R) return;
  float dl[EM];
#pragma unroll
  for (int e = 0; e < EM; e++) dl[e] = 0.f;
  if (logits) {
    float lg[EM], w[KMAX], g[KMAX];
    int32_t id[KMAX];
#pragma unroll
    for (int e = 0; e < EM; e++) lg[e] = e < E ? bf2f(logits[t * E + e]) : 0.f;
#pragma unroll
    for (int k = 0; k < KMAX; k++) {
      id[k] = k < K ? ids[t * K + k] : -1;
      w[k] = k < K ? weights[t * K + k] : 0.f;
      g[k] = k < K ? dweights[t * K + k] : 0.f;
    }
    route_bwd_row<EM>(lg, E, K, id, w, g, dl);
    if (lane < E) {
      float v = 0.f;
#pragma unroll
      for (int e = 0; e < EM; e++)
        if (e == lane) v = dl[e];
      dlogits[t * E + lane] = v;
    }
  }
  int pos[KM];
  float unused[KM];
  const int n = token_routes<KM>(t, K, ids, ppos, nullptr, pos, unused);
  for (long c8 = 8L * lane; c8 < d; c8 += 512) {
    float s[8], ex[8];
#pragma unroll
    for (int i = 0; i < 8; i++) s[i] = ex[i] = 0.f;
    if (acc) {
      const float4 a0 = *(const float4*)(acc + t * ldacc + c8), a1 = *(const float4*)(acc + t * ldacc + c8 + 4);
      s[0] = a0.x; s[1] = a0.y; s[2] = a0.z; s[3] = a0.w; s[4] = a1.x; s[5] = a1.y; s[6] = a1.z; s[7] = a1.w;
    }
#pragma unroll
    for (int j = 0; j < KM; j++)
      if (j < n) {
        const float4 x0 = *(const float4*)(dxp + pos[j] * lddx + c8), x1 = *(const float4*)(dxp + pos[j] * lddx + c8 + 4);
        ex[0] += x0.x; ex[1] += x0.y; ex[2] += x0.z; ex[3] += x0.w;
        ex[4] += x1.x; ex[5] += x1.y; ex[6] += x1.z; ex[7] += x1.w;
      }
#pragma unroll
    for (int i = 0; i < 8; i++) s[i] += ex[i];
    if (logits && wr) {
#pragma unroll
      for (int i = 0; i < 8; i++) {
        const bf16_t* wrow = wr + (c8 + i) * E;
        float r = 0.f;
#pragma unroll
        for (int e8 = 0; e8 < EM; e8 += 8) {
          if (e8 >= E) break;
          const u32x4 wv = *(const u32x4*)(wrow + e8);
#pragma unroll
          for (int q = 0; q < 4; q++) {
            r += dl[e8 + 2 * q] * __uint_as_float(wv[q] << 16);
            r += dl[e8 + 2 * q + 1] * __uint_as_float(wv[q] & 0xffff0000u);
          }
        }
        s[i] += r;
      }
    }
    *(float4*)(dz + t * lddz + c8) = make_float4(s[0], s[1], s[2], s[3]);
    *(float4*)(dz + t * lddz + c8 + 4) = make_float4(s[4], s[5], s[6], s[7]);
  }
}

}  // namespace

// ================================================================ C ABI

extern "C" long sj_route_pack_capacity(long slots, long experts) {
  if (slots < 0 || experts <= 0) return -1;
  return pack_capacity(slots, experts);
}

bool sjh::router_pack_ok(long d, long ldz, long E, long K, const void* z, const void* wr, const void* logits) {
  return E == 8 && K > 0 && K <= 4 && d % 128 == 0 && ldz >= d && ldz % 8 == 0 &&
         (((uintptr_t)z | (uintptr_t)wr | (uintptr_t)logits) & 15) == 0;
}

long sjh::router_hist_blocks(long rows) { return (rows * 16 + NT - 1) / NT; }

int sjh::router_topk_hist(hipStream_t s, const uint16_t* z, long ldz, const uint16_t* wr, long d, long rows, long E,
                          long K, uint16_t* logits, int32_t* ids, float* weights, int32_t* hist) {
  SJ_REQUIRE(router_pack_ok(d, ldz, E, K, z, wr, logits) && rows > 0 && hist, "router top-k with counts: shapes");
  hipLaunchKernelGGL((k_router_topk_lanes<1, 16>), dim3((unsigned)router_hist_blocks(rows)), dim3(NT), 0, s,
                     (const bf16_t*)z, ldz, (const bf16_t*)wr, d, rows, (int)E, (int)K, (bf16_t*)logits, ids, weights,
                     hist);
  SJ_LAUNCH_CHECK("router_topk");
  return SJ_OK;
}

int sjh::route_pack_hist(hipStream_t s, const int32_t* ids, long rows, long K, long E, const int32_t* hist,
                         int32_t* counts, int32_t* offsets, int32_t* pslot, int32_t* ppos, long cap) {
  SJ_REQUIRE(E == 8 && K > 0 && K <= 4 && rows > 0 && hist && offsets && pslot && ppos &&
                 cap >= pack_capacity(rows * K, E),
             "route pack from counts: shapes (capacity %ld)", cap);
  const long nblk = router_hist_blocks(rows);
  hipLaunchKernelGGL(k_route_pack_hist, dim3((unsigned)nblk), dim3(64), 0, s, ids, rows * K, (int)E, cap, hist,
                     (int)nblk, (int)(NT / 16 * K), counts, offsets, pslot, ppos);
  SJ_LAUNCH_CHECK("hierarchy_route_pack");
  return SJ_OK;
}

extern "C" int sj_router_topk(void* stream, const uint16_t* z, long ldz, const uint16_t* w_router, long d, long rows,
                              long experts, long top_k, uint16_t* logits, int32_t* ids, float* weights) {
  SJ_REQUIRE(rows >= 0 && d > 0 && ldz >= d && experts > 0 && experts <= EMAX && top_k > 0 && top_k <= KMAX &&
                 top_k <= experts && logits && ids && weights,
             "router top-k dimensions (experts <= %d, top_k <= %d)", EMAX, KMAX);
  if (rows == 0) return SJ_OK;
  const bool vec = d % 8 == 0 && ldz % 8 == 0 && experts % 8 == 0 && ((uintptr_t)z & 15) == 0 &&
                   ((uintptr_t)w_router & 15) == 0 && ((uintptr_t)logits & 15) == 0;
  static int lpt = -1;
  if (lpt < 0) {
    const char* e = getenv("SJ_ROUTER_LANES");  // sweeps: 8, 16, or 64 (one wave per token)
    lpt = e ? atoi(e) : 16;
  }
  if (vec && (lpt == 8 || lpt == 16) && d % (8 * lpt) == 0) {
    const long threads = rows * lpt;
    const dim3 grid((unsigned)((threads + NT - 1) / NT));
    auto kern = lpt == 8 ? (experts <= 8 ? k_router_topk_lanes<1, 8> : experts <= 16 ? k_router_topk_lanes<2, 8>
                                                                                     : k_router_topk_lanes<4, 8>)
                         : (experts <= 8 ? k_router_topk_lanes<1, 16> : experts <= 16 ? k_router_topk_lanes<2, 16>
                                                                                      : k_router_topk_lanes<4, 16>);
    hipLaunchKernelGGL(kern, grid, dim3(NT), 0, (hipStream_t)stream, (const bf16_t*)z, ldz,
                       (const bf16_t*)w_router, d, rows, (int)experts, (int)top_k, (bf16_t*)logits, ids, weights,
                       (int32_t*)nullptr);
    SJ_LAUNCH_CHECK("router_topk");
    return SJ_OK;
  }
  hipLaunchKernelGGL(vec ? k_router_topk8 : k_router_topk, dim3((unsigned)((rows + 3) / 4)), dim3(NT), 0,
                     (hipStream_t)stream, (const bf16_t*)z, ldz, (const bf16_t*)w_router, d, rows, (int)experts,
                     (int)top_k, (bf16_t*)logits, ids, weights);
  SJ_LAUNCH_CHECK("router_topk");
  return SJ_OK;
}

extern "C" int sj_route_topk(void* stream, const void* logits, int dtype, long rows, long experts, long top_k,
                             int32_t* ids, float* weights) {
  SJ_REQUIRE(rows >= 0 && experts > 0 && experts <= EMAX && top_k > 0 && top_k <= KMAX && top_k <= experts &&
                 (dtype == SJ_F32 || dtype == SJ_BF16),
             "router top-k dimensions");
  if (rows == 0) return SJ_OK;
  hipLaunchKernelGGL(k_route_topk, dim3((unsigned)((rows + NT - 1) / NT)), dim3(NT), 0, (hipStream_t)stream, logits,
                     dtype, rows, (int)experts, (int)top_k, ids, weights);
  SJ_LAUNCH_CHECK("hierarchy_route_topk");
  return SJ_OK;
}

extern "C" int sj_route_topk_bwd(void* stream, const void* logits, int dtype, const int32_t* ids, const float* weights,
                                 const float* dy, float* dx, long rows, long experts, long top_k) {
  SJ_REQUIRE(rows >= 0 && experts > 0 && experts <= EMAX && top_k > 0 && top_k <= KMAX && top_k <= experts &&
                 (dtype == SJ_F32 || dtype == SJ_BF16),
             "router backward dimensions");
  if (rows == 0) return SJ_OK;
  hipLaunchKernelGGL(k_route_topk_bwd, dim3((unsigned)((rows + NT - 1) / NT)), dim3(NT), 0, (hipStream_t)stream,
                     logits, dtype, ids, weights, dy, dx, rows, (int)experts, (int)top_k);
  SJ_LAUNCH_CHECK("hierarchy_route_backward");
  return SJ_OK;
}

extern "C" int sj_route_pack(void* stream, const int32_t* ids, long rows, long top_k, long experts, int32_t* tokens,
                             int32_t* slots, int32_t* counts, int32_t* offsets, int32_t* pslot, int32_t* ppos,
                             long capacity) {
  const long S = rows * top_k;
  SJ_REQUIRE(rows >= 0 && top_k > 0 && experts > 0 && experts <= EMAX && S < (1L << 31) && offsets && pslot && ppos &&
                 capacity >= pack_capacity(S, experts),
             "expert route dimensions (capacity %ld, need %ld)", capacity, pack_capacity(S, experts));
  hipStream_t s = (hipStream_t)stream;
  const int E = (int)experts, Kk = (int)top_k;
  if (E <= 2)
    hipLaunchKernelGGL(k_route_pack_wide<1>, dim3(1), dim3(PNT), 0, s, ids, S, Kk, E, capacity, tokens, slots, counts,
                       offsets, pslot, ppos);
  else if (E <= 4)
    hipLaunchKernelGGL(k_route_pack_wide<2>, dim3(1), dim3(PNT), 0, s, ids, S, Kk, E, capacity, tokens, slots, counts,
                       offsets, pslot, ppos);
  else if (E <= 8)
    hipLaunchKernelGGL(k_route_pack_wide<4>, dim3(1), dim3(PNT), 0, s, ids, S, Kk, E, capacity, tokens, slots, counts,
                       offsets, pslot, ppos);
  else if (E <= 16)
    hipLaunchKernelGGL(k_route_pack_wide<8>, dim3(1), dim3(PNT), 0, s, ids, S, Kk, E, capacity, tokens, slots, counts,
                       offsets, pslot, ppos);
  else
    hipLaunchKernelGGL(k_route_pack, dim3(1), dim3(NT), 0, s, ids, S, Kk, E, capacity, tokens, slots, counts, offsets,
                       pslot, ppos);
  SJ_LAUNCH_CHECK("hierarchy_route_pack");
  return SJ_OK;
}

extern "C" int sj_moe_gather(void* stream, const uint16_t* x, long ldx, long d, const int32_t* pslot, long top_k,
                             long capacity, uint16_t* y, uint16_t* y_t, long ldt) {
  SJ_REQUIRE(d > 0 && d % 8 == 0 && d <= 1024 && ldx % 2 == 0 && ldx >= d && top_k > 0 && capacity % 64 == 0 &&
                 (!y_t || (ldt >= capacity && ldt % 8 == 0 && ((uintptr_t)y_t & 15) == 0)),
             "gather (experts): d %ld (<= 1024, multiple of 8), capacity %ld", d, capacity);
  if (capacity == 0) return SJ_OK;
  if (!y_t && ldx % 8 == 0 && ((uintptr_t)x & 15) == 0 && ((uintptr_t)y & 15) == 0) {
    const long chunks = capacity * (d / 8), blocks = (chunks + NT - 1) / NT;
    hipLaunchKernelGGL(k_moe_gather16, dim3((unsigned)(blocks < 65536 ? blocks : 65536)), dim3(NT), 0,
                       (hipStream_t)stream, (const bf16_t*)x, ldx, d, pslot, (int)top_k, capacity, (bf16_t*)y);
    SJ_LAUNCH_CHECK("gather");
    return SJ_OK;
  }
  const size_t lds = sizeof(bf16_t) * TR * (size_t)d;
  hipLaunchKernelGGL(k_moe_gather, dim3((unsigned)(capacity / TR)), dim3(NT), lds, (hipStream_t)stream,
                     (const bf16_t*)x, ldx, d, pslot, (int)top_k, capacity, (bf16_t*)y, (bf16_t*)y_t, ldt);
  SJ_LAUNCH_CHECK("gather");
  return SJ_OK;
}

extern "C" int sj_moe_combine(void* stream, const uint16_t* yp, long ldy, long d, const int32_t* ids,
                              const int32_t* ppos, const float* weights, long rows, long top_k, const uint16_t* residual,
                              long ldr, uint16_t* out, long ldo) {
  SJ_REQUIRE(rows >= 0 && d > 0 && d % 2 == 0 && ldy % 2 == 0 && ldo % 2 == 0 && (!residual || ldr % 2 == 0) &&
                 top_k > 0 && top_k <= KMAX,
             "expert combine dimensions");
  if (rows == 0) return SJ_OK;
  const bool v8 = d % 8 == 0 && ldy % 8 == 0 && ldo % 8 == 0 && (!residual || (ldr % 8 == 0 && ((uintptr_t)residual & 15) == 0)) &&
                  ((uintptr_t)yp & 15) == 0 && ((uintptr_t)out & 15) == 0;
  auto kern = v8 ? (top_k <= 2 ? k_moe_combine<true, 2> : k_moe_combine<true>) : k_moe_combine<false>;
  hipLaunchKernelGGL(kern, dim3((unsigned)((rows + 3) / 4)), dim3(NT), 0, (hipStream_t)stream, (const bf16_t*)yp, ldy, d, ids, ppos, weights, rows, (int)top_k,
                     (const bf16_t*)residual, ldr, (bf16_t*)out, ldo);
  SJ_LAUNCH_CHECK("hierarchy_expert_combine");
  return SJ_OK;
}

extern "C" int sj_moe_combine_bwd(void* stream, const uint16_t* yp, long ldy, long d, const int32_t* pslot,
                                  const float* weights, long top_k, long capacity, const float* dy, long lddy,
                                  uint16_t* dx_hi, uint16_t* dx_lo, uint16_t* dx_t_hi, uint16_t* dx_t_lo, long ldt,
                                  float* dweights) {
  SJ_REQUIRE(d > 0 && d % 8 == 0 && d <= 1024 && ldy % 2 == 0 && lddy % 2 == 0 && top_k > 0 && capacity % 64 == 0 &&
                 !dx_t_hi == !dx_t_lo && (!dx_t_hi || (ldt >= capacity && ldt % 8 == 0)) &&
                 ((uintptr_t)dx_t_hi & 15) == 0 && ((uintptr_t)dx_t_lo & 15) == 0,
             "expert combine backward dimensions (transposed planes both or neither)");
  if (capacity == 0) return SJ_OK;
  if (!dx_t_hi && ldy % 8 == 0 && lddy % 8 == 0 && ((uintptr_t)yp & 15) == 0 && ((uintptr_t)dy & 15) == 0 &&
      ((uintptr_t)dx_hi & 15) == 0 && ((uintptr_t)dx_lo & 15) == 0) {
    hipLaunchKernelGGL(k_moe_combine_bwd8, dim3((unsigned)(capacity / 4)), dim3(NT), 0, (hipStream_t)stream,
                       (const bf16_t*)yp, ldy, d, pslot, weights, (int)top_k, capacity, dy, lddy, (bf16_t*)dx_hi,
                       (bf16_t*)dx_lo, dweights);
    SJ_LAUNCH_CHECK("hierarchy_expert_backward");
    return SJ_OK;
  }
  const size_t lds = 2 * sizeof(bf16_t) * TRB * (size_t)d;
  hipLaunchKernelGGL(k_moe_combine_bwd, dim3((unsigned)(capacity / TRB)), dim3(NT), lds, (hipStream_t)stream,
                     (const bf16_t*)yp, ldy, d, pslot, weights, (int)top_k, capacity, dy, lddy, (bf16_t*)dx_hi,
                     (bf16_t*)dx_lo, (bf16_t*)dx_t_hi, (bf16_t*)dx_t_lo, ldt, dweights);
  SJ_LAUNCH_CHECK("hierarchy_expert_backward");
  return SJ_OK;
}

extern "C" int sj_moe_gather_bwd(void* stream, const float* dxp, long lddx, long d, const int32_t* ids,
                                 const int32_t* ppos, const float* weights, const uint16_t* logits,
                                 const float* dweights, const uint16_t* w_router, long rows, long top_k, long experts,
                                 const float* dz_acc, long ldacc, float* dz, long lddz, float* dlogits) {
  SJ_REQUIRE(rows >= 0 && d > 0 && top_k > 0 && top_k <= KMAX && experts > 0 && experts <= EMAX &&
                 (!logits || (dweights && dlogits)),
             "gather backward (experts) dimensions");
  if (rows == 0) return SJ_OK;
  const bool vec = d % 8 == 0 && experts % 8 == 0 && lddx % 4 == 0 && lddz % 4 == 0 && (!dz_acc || ldacc % 4 == 0) &&
                   ((uintptr_t)dxp & 15) == 0 && ((uintptr_t)dz & 15) == 0 && ((uintptr_t)dz_acc & 15) == 0 &&
                   ((uintptr_t)w_router & 15) == 0;
  auto kern = vec ? (experts <= 8 ? (top_k <= 2 ? k_moe_gather_bwd8<8, 2> : k_moe_gather_bwd8<8>)
                                   : k_moe_gather_bwd8<EMAX>)
                   : k_moe_gather_bwd;
  hipLaunchKernelGGL(kern, dim3((unsigned)((rows + 3) / 4)), dim3(NT), 0,
                     (hipStream_t)stream, dxp, lddx, d, ids, ppos, weights, (const bf16_t*)logits, dweights,
                     (const bf16_t*)w_router, rows, (int)top_k, (int)experts, dz_acc, ldacc, dz, lddz, dlogits);
  SJ_LAUNCH_CHECK("gather_backward");
  return SJ_OK;
}
