// Step driver for the dense byte Transformer: the per-step call sequence of
// train_configured (crates/sejong-train/src/lib.rs:387-453) restated for one
// stream and a preallocated arena:
//   Model::bind cast        -> fused into AdamW (bf16 mirror of the masters)
//   Model::logits           -> Block::apply per layer (architecture.rs:200-247)
//                              + final norm + fp32 head (model lib.rs:336-340)
//   cross_entropy + seed    -> one fused CE kernel (graph.rs:539-549)
//   Graph::backward         -> the reverse rules of graph.rs:567-911 in the
//                              fixed order of one block, gradients written
//                              straight into a gradient arena
//   Adam::update            -> FP64 norm on device + one multi-tensor AdamW
//                              with the clip factor formed on device
// so the whole step has no host synchronisation and can be captured once
// as a hipGraph and replayed.
//
// Internal parameter layout (all fp32 masters, 256-byte aligned tensors):
//   [no decay]  per layer attention_norm, ffn_norm; final_norm
//   [decay]     embedding [V][d]; per layer W_qkv [d][d+2J] (query|key|value
//               column blocks), attention_output [d][d], W_gu [d][2F]
//               (gate|up), down [F][d]; output [d][Vp] (Vp = V rounded up
//               to 8, padding columns stay zero)
// Exchange with the host uses the reference layout (architecture.rs:63-137).
//
// The hierarchical byte model (cfg3: ModelConfig::hierarchy, architecture.rs:
// 368-393) runs three stages through the same per-layer code: the byte
// encoder (local window), the global stack over patches and the byte decoder
// (local window), each a run of blocks with its own widths and sequence and
// its closing norm, joined by patch pooling / broadcast and the projections
// between the widths.
//
// bf16 steps run the MFMA-layout kernels: every GEMM operand is streamed
// k-contiguous, so the step keeps, next to the bf16 mirror, a transposed
// mirror of the four projection matrices per layer (forward B operands,
// rebuilt by one batched transpose after each AdamW update), writes the
// normalised activations, O and h also transposed ([cols][rows], the A
// operands of the dW GEMMs), and carries the fp32 gradients dY that feed
// GEMMs as hi/lo bf16 planes in both orientations (dX and dW operands).
#include <algorithm>
#include <math.h>
#include <stddef.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <string>
#include <vector>

#include "common.h"

extern "C" int sj_rope_table(void* stream, float* table, long t, long head_dim, float theta);

namespace {

long align64(long x) { return (x + 63) / 64 * 64; }

struct RefTensor {
  std::string name;
  long rows, cols;  // reference shape ([n] 1-D tensors have rows = 1)
  long ref_offset;  // offset in the reference-layout flat vector
  long int_offset;  // offset of element (0,0) in the internal arena
  long int_ld;      // internal row stride
  // projection-group membership (parameter VJP): kind 0 = q|k|v, 1 = gate|up,
  // -1 none; member index and first column in the group's concatenated width
  int layer = -1, kind = -1, member = -1;
  long col0 = 0;
  int ndim = 2;  // the reference tensor's rank (weight decay applies when > 1)
};

struct Layer {
  long an, fn, qkv, wo, gu, down;  // internal offsets
  long router = 0;                 // MoE: router [d][E] (gu = [E][d][2F], down = [E][F][d])
  int stage = 0;
};

// One run of blocks and its closing norm: the dense model has one (closed by
// the final norm); the hierarchical model has the encoder (closed by
// encoder_norm), the global stack (global_norm) and the decoder
// (decoder_norm).  Layer l of stage s reads x[l + s] and writes x[l + s + 1].
struct Stage {
  std::string prefix;         // parameter names: "<prefix>.<i>.<tensor>"
  int index = 0;
  long first = 0, count = 0;  // layers [first, first + count)
  long d = 0, HQ = 0, HK = 0, Dh = 0, J = 0, F = 0, NQKV = 0, T = 0, M = 0, ldt = 0;
  long window = 0;            // local causal window (0: every earlier position)
  long depth = 0;             // layers of the stage (initialisation scale)
  long norm = 0;              // internal offset of the closing norm's weight
  bool attn_tt = false;
  float* rope = nullptr;      // RoPE table [T][Dh/2] (cos, sin)
  void* out = nullptr;        // closing norm output [M][d], compute dtype
};

// one matrix of the batched bf16 transpose: src [rows][cols] -> dst [cols][rows]
struct TJob {
  long off;    // element offset in both the mirror and the transposed mirror
  long rows, cols;
  long tile0;  // first 64x64 tile of this job in the flat tile index
  long tiles_c;
  int kind;    // 0: bf16 mirror -> transposed mirror; 1: fp32 master -> hi/lo planes, normal and transposed
};

// outputs of a kind-1 job: hi, lo [rows][cols] and hi^T, lo^T [cols][rows]
struct TPlanes {
  uint16_t *hi, *lo, *hit, *lot;
};

// Keeps the profiled stream busy for `n` sleeps of ~8k clocks each while the
// host enqueues a whole eager step behind it, so the event pairs around each
// op time the GPU's work rather than the host's launch gaps.  Bounded: every
// wave leaves after n iterations.
__global__ __launch_bounds__(64) void k_profile_hold(int n) {
  for (int i = 0; i < n; i++) __builtin_amdgcn_s_sleep(127);
}

// jobs[0 .. njobs) with tiles tile_base .. tile_base + gridDim.x - 1 of the
// flat tile index (a subset of the table: one layer's matrices)
__global__ __launch_bounds__(256) void k_transpose_jobs(const uint16_t* __restrict__ src, uint16_t* __restrict__ dst,
                                                        const TJob* __restrict__ jobs, int njobs,
                                                        const float* __restrict__ master, TPlanes hp, long tile_base) {
  __shared__ __attribute__((aligned(16))) uint16_t tile[64 * 72];
  __shared__ __attribute__((aligned(16))) uint16_t tile_lo[64 * 72];
  const long b = tile_base + blockIdx.x;
  int ji = 0;
  while (ji + 1 < njobs && b >= jobs[ji + 1].tile0) ji++;
  const long off = jobs[ji].off, rows = jobs[ji].rows, cols = jobs[ji].cols;
  const long lt = b - jobs[ji].tile0;
  const long r0 = (lt / jobs[ji].tiles_c) * 64, c0 = (lt % jobs[ji].tiles_c) * 64;
  const int t = threadIdx.x;
  if (jobs[ji].kind == 1) {
    // fp32 master tile -> hi = RNE(w), lo = RNE(w - hi), stored [rows][cols]
    // and transposed [cols][rows] (the output head's GEMM operands)
    const float* S = master + off;
#pragma unroll
    for (int p = 0; p < 2; p++) {
      const int r = (t >> 3) + 32 * p, c = (t & 7) * 8;
      const long gr = r0 + r, gc = c0 + c;
      uint16_t h[8], l[8];
#pragma unroll
      for (int i = 0; i < 8; i++) {
        const float v = (gr < rows && gc + i < cols) ? S[gr * cols + gc + i] : 0.f;
        sj::split_bf(v, h[i], l[i]);
        tile[r * 72 + c + i] = h[i];
        tile_lo[r * 72 + c + i] = l[i];
      }
      if (gr < rows)
        for (int i = 0; i < 8; i++)
          if (gc + i < cols) {
            hp.hi[gr * cols + gc + i] = h[i];
            hp.lo[gr * cols + gc + i] = l[i];
          }
    }
    __syncthreads();
#pragma unroll
    for (int p = 0; p < 2; p++) {
      const int oc = (t >> 3) + 32 * p, orr = (t & 7) * 8;
      if (c0 + oc < cols)
        for (int i = 0; i < 8; i++)
          if (r0 + orr + i < rows) {
            hp.hit[(c0 + oc) * rows + r0 + orr + i] = tile[(orr + i) * 72 + oc];
            hp.lot[(c0 + oc) * rows + r0 + orr + i] = tile_lo[(orr + i) * 72 + oc];
          }
    }
    return;
  }
  const uint16_t* S = src + off;
  uint16_t* D = dst + off;
  const bool vec = (rows & 7) == 0 && (cols & 7) == 0 && r0 + 64 <= rows && c0 + 64 <= cols;
#pragma unroll
  for (int p = 0; p < 2; p++) {
    const int r = (t >> 3) + 32 * p, c = (t & 7) * 8;
    uint16_t v[8];
    if (vec) {
      sj::u32x4 w = *(const sj::u32x4*)(S + (r0 + r) * cols + c0 + c);
      for (int i = 0; i < 4; i++) {
        v[2 * i] = (uint16_t)(w[i] & 0xffffu);
        v[2 * i + 1] = (uint16_t)(w[i] >> 16);
      }
    } else {
      for (int i = 0; i < 8; i++)
        v[i] = (r0 + r < rows && c0 + c + i < cols) ? S[(r0 + r) * cols + c0 + c + i] : (uint16_t)0;
    }
    for (int i = 0; i < 8; i++) tile[r * 72 + c + i] = v[i];
  }
  __syncthreads();
#pragma unroll
  for (int p = 0; p < 2; p++) {
    const int oc = (t >> 3) + 32 * p, orr = (t & 7) * 8;  // source column oc, source rows orr..+7
    uint16_t v[8];
    for (int i = 0; i < 8; i++) v[i] = tile[(orr + i) * 72 + oc];
    if (vec) {
      *(sj::u32x4*)(D + (c0 + oc) * rows + r0 + orr) =
          sj::u32x4{sj::pack2(v[0], v[1]), sj::pack2(v[2], v[3]), sj::pack2(v[4], v[5]), sj::pack2(v[6], v[7])};
    } else if (c0 + oc < cols) {
      for (int i = 0; i < 8; i++)
        if (r0 + orr + i < rows) D[(c0 + oc) * rows + r0 + orr + i] = v[i];
    }
  }
}

// A run of parameters outside the transpose table, updated elementwise
struct FlatChunk {
  long begin, end;
};

// The AdamW update of the bf16 planes models with the mirrors it feeds
// written in the same pass (Adam::update, crates/sejong-train/src/lib.rs:
// 199-238, with Model::bind's cast, model lib.rs:206-250, fused).  Workgroup
// b < tiles takes tile b of the transpose table: it updates the tile's
// masters and moments row by row, writes the bf16 mirror, and from an LDS
// copy of the new values the transposed mirror the forward GEMMs read
// (kind 1, the output head: its hi/lo planes, normal and transposed).  The
// workgroups past the tiles update the flat chunks (everything else, 1024
// parameters each).  The per-parameter arithmetic is adam_elem, as in
// k_adamw_multi: the same bits, and the forward no longer waits for a
// transpose pass.
__global__ __launch_bounds__(256) void k_adamw_tiles(float* __restrict__ w, const float* __restrict__ g,
                                                     float* __restrict__ m, float* __restrict__ v,
                                                     uint16_t* __restrict__ mirror, uint16_t* __restrict__ mirror_t,
                                                     long n_nodecay, const sj_adam_step* __restrict__ st,
                                                     const double* __restrict__ sumsq, int32_t* status,
                                                     const TJob* __restrict__ jobs, int njobs, long tiles,
                                                     const FlatChunk* __restrict__ chunks, TPlanes hp) {
  sj::AdamCoef c;
  if (!sj::adam_coef(st, sumsq, c)) {
    if (blockIdx.x == 0 && threadIdx.x == 0) status[0] = 1;
    return;
  }
  const int t = threadIdx.x;
  const long b = blockIdx.x;
  // four parameters from i0 (vector path when they are whole and aligned)
  auto quad = [&](long i0, long end, float* out) {
    if (i0 + 4 <= end && (i0 & 3) == 0) {
      const float4 wv = *(const float4*)(w + i0), gv = *(const float4*)(g + i0);
      const float4 mv = *(const float4*)(m + i0), vv = *(const float4*)(v + i0);
      float ws[4] = {wv.x, wv.y, wv.z, wv.w}, gs[4] = {gv.x, gv.y, gv.z, gv.w};
      float ms[4] = {mv.x, mv.y, mv.z, mv.w}, vs[4] = {vv.x, vv.y, vv.z, vv.w};
#pragma unroll
      for (int j = 0; j < 4; j++) sj::adam_elem(ws[j], gs[j], ms[j], vs[j], c, (i0 + j) >= n_nodecay);
      *(float4*)(w + i0) = make_float4(ws[0], ws[1], ws[2], ws[3]);
      *(float4*)(m + i0) = make_float4(ms[0], ms[1], ms[2], ms[3]);
      *(float4*)(v + i0) = make_float4(vs[0], vs[1], vs[2], vs[3]);
      *(uint2*)(mirror + i0) = uint2{sj::pack2(sj::f2bf(ws[0]), sj::f2bf(ws[1])), sj::pack2(sj::f2bf(ws[2]), sj::f2bf(ws[3]))};
#pragma unroll
      for (int j = 0; j < 4; j++) out[j] = ws[j];
    } else {
      for (int j = 0; j < 4; j++) {
        const long i = i0 + j;
        if (i >= end) break;
        float wi = w[i], mi = m[i], vi = v[i];
        sj::adam_elem(wi, g[i], mi, vi, c, i >= n_nodecay);
        w[i] = wi;
        m[i] = mi;
        v[i] = vi;
        mirror[i] = sj::f2bf(wi);
        out[j] = wi;
      }
    }
  };
  if (b >= tiles) {  // a flat chunk: one quad per thread
    const FlatChunk ch = chunks[b - tiles];
    float tmp[4];
    const long i0 = ch.begin + 4L * t;
    if (i0 < ch.end) quad(i0, ch.end, tmp);
    return;
  }
  __shared__ __attribute__((aligned(16))) uint16_t tile[64 * 72];
  __shared__ __attribute__((aligned(16))) uint16_t tile_lo[64 * 72];
  int ji = 0;
  while (ji + 1 < njobs && b >= jobs[ji + 1].tile0) ji++;
  const long off = jobs[ji].off, rows = jobs[ji].rows, cols = jobs[ji].cols;
  const bool k1 = jobs[ji].kind == 1;
  const long lt = b - jobs[ji].tile0;
  const long r0 = (lt / jobs[ji].tiles_c) * 64, c0 = (lt % jobs[ji].tiles_c) * 64;
  // 16 rows per pass, 16 threads per 64-column row: 256-byte row segments
#pragma unroll
  for (int p = 0; p < 4; p++) {
    const int r = (t >> 4) + 16 * p, cc = 4 * (t & 15);
    const long gr = r0 + r, gc = c0 + cc;
    float nw[4] = {0.f, 0.f, 0.f, 0.f};
    if (gr < rows && gc < cols) {
      const long i0 = off + gr * cols + gc;
      quad(i0, i0 + (cols - gc < 4 ? cols - gc : 4), nw);
    }
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const bool in = gr < rows && gc + j < cols;
      if (k1) {
        sj::bf16_t h = 0, l = 0;
        if (in) sj::split_bf(nw[j], h, l);
        tile[r * 72 + cc + j] = h;
        tile_lo[r * 72 + cc + j] = l;
        if (in) {
          hp.hi[gr * cols + gc + j] = h;
          hp.lo[gr * cols + gc + j] = l;
        }
      } else {
        tile[r * 72 + cc + j] = in ? sj::f2bf(nw[j]) : (uint16_t)0;
      }
    }
  }
  __syncthreads();
  const bool vec = !k1 && (rows & 7) == 0 && r0 + 64 <= rows && c0 + 64 <= cols;
  uint16_t* D = mirror_t + off;
#pragma unroll
  for (int p = 0; p < 2; p++) {
    const int oc = (t >> 3) + 32 * p, orr = (t & 7) * 8;  // source column oc, source rows orr..+7
    uint16_t u[8];
    for (int i = 0; i < 8; i++) u[i] = tile[(orr + i) * 72 + oc];
    if (k1) {
      if (c0 + oc < cols)
        for (int i = 0; i < 8; i++)
          if (r0 + orr + i < rows) {
            hp.hit[(c0 + oc) * rows + r0 + orr + i] = u[i];
            hp.lot[(c0 + oc) * rows + r0 + orr + i] = tile_lo[(orr + i) * 72 + oc];
          }
    } else if (vec) {
      *(sj::u32x4*)(D + (c0 + oc) * rows + r0 + orr) =
          sj::u32x4{sj::pack2(u[0], u[1]), sj::pack2(u[2], u[3]), sj::pack2(u[4], u[5]), sj::pack2(u[6], u[7])};
    } else if (c0 + oc < cols) {
      for (int i = 0; i < 8; i++)
        if (r0 + orr + i < rows) D[(c0 + oc) * rows + r0 + orr + i] = u[i];
    }
  }
}

}  // namespace

struct sj_model {
  sj_model_config c;
  sj_adam_config adam;
  hipStream_t stream;
  long V, Vp, d, L, HQ, HK, Dh, J, F, T, B, M, NQKV;
  // stages (one for the dense model); d and M above are the head's width
  // and rows (the final norm's), the dense model's block shape otherwise
  std::vector<Stage> stages;
  bool hier = false;
  long P = 0;                                   // bytes per patch
  long h_inproj = 0, h_e2g = 0, h_e2d = 0, h_g2d = 0, h_bos = 0, h_op = 0;  // glue parameters
  void *pooled = nullptr, *gd = nullptr, *bosd = nullptr, *zb = nullptr, *bytes = nullptr, *opo = nullptr;
  float* hg[8] = {};                            // glue backward scratch
  // bf16 models: hi/lo planes of the glue products' dY (the final norm's
  // dX, d(decoder input), the broadcast's patch gradient, d(global input)),
  // each read by that glue pair's dX and row-layout dW products
  uint16_t* glue_p[4][2] = {};
  int32_t* mhist = nullptr;  // mixture of experts: the router top-k's per-workgroup counts (E == 8)
  // mixture of experts (every block; F is the expert width): routing, the
  // packed expert rows and, per layer, the backward planes the dW stream reads
  long E = 0, K = 0, cap = 0;
  std::vector<uint16_t*> mlog, mzp, mzpt, myp;
  std::vector<int32_t*> mids, mcnt, moff, mps, mpp;
  std::vector<float*> mwts, mdwts, mdlog;
  std::vector<uint16_t*> mdx[4], mdg[4];        // [layer]: hi, lo [cap][*]; hi^T, lo^T [*][cap]
  float* mdzp = nullptr;
  std::vector<hipEvent_t> ev_moe[2];
  // head: HV classes over HR rows (the LM head: V over all M tokens; the
  // NativeValue head: value_n classes over the B selected SEP rows); Vp =
  // HV rounded up to 8 (the head's row stride)
  long HV = 0, HR = 0;
  long value_n = 0;  // NativeValue head (native/value.rs:111-160) when > 0
  long bias = 0;     // internal offset of native_bias
  int32_t *sel = nullptr, *labels = nullptr;  // SEP row of each request, its value label
  float *hsel = nullptr, *dhsel = nullptr;    // selected hidden rows (fp32) and their gradient
  int dt;
  size_t esz;  // bytes per activation element
  // parameter arenas
  long n_params;   // internal arena elements
  long n_nodecay;  // [0, n_nodecay) not decayed
  long ref_count;  // reference layout elements
  std::vector<RefTensor> tensors;
  std::vector<Layer> layers;
  long emb, final_norm, out;
  float *w = nullptr, *g = nullptr, *m = nullptr, *v = nullptr;
  uint16_t* mirror = nullptr;  // bf16 compute copy (dt == bf16)
  // MFMA-layout path (bf16, head_dim 64)
  bool planes = false;
  // row-layout dW (planes path without the parameter VJP, every stage on the
  // MFMA-layout attention): the dW products read activations and gradient
  // planes in row orientation (sj_gemm_planes_tn), so no producer writes a
  // transposed copy; the gradient planes live in the parity buffers pt
  bool rowdw = false;
  long ldt = 0;                   // leading dimension of [cols][rows] activations (M rounded to 8)
  uint16_t* mirror_t = nullptr;   // transposed projection matrices, same offsets as the mirror
  // LM head on the planes kernels: W_out as hi/lo planes [d][Vp] and
  // transposed [Vp][d] (refreshed with the transposed mirror), dlogits as
  // hi/lo planes [M][Vp] written by the cross entropy
  bool lm_planes = false;
  bool defer_loss = false;  // set inside a training step: loss_summary runs after the backward's fork
  // gradient accumulation (train lib.rs:390-415): observations per update,
  // the observation being run, its batches stacked on the device, and the
  // accumulator arena (Adam::accumulate)
  static constexpr long OBS_MAX = 256;  // loss summary slots
  long obs = 1, obs_slot = 0;
  int32_t *obs_ids = nullptr, *obs_targets = nullptr;
  long obs_cap = 0;
  float* g_acc = nullptr;
  uint16_t* hp[4] = {};
  uint16_t* dlp[2] = {};
  TJob* tjobs = nullptr;
  int tjob_n = 0;
  long tjob_tiles = 0;
  // the AdamW update writes the mirrors itself (k_adamw_tiles): the
  // parameters outside the transpose table as flat chunks
  bool fused_update = false;
  FlatChunk* fchunks = nullptr;
  long nfchunks = 0;
  // the table in groups for the overlapped refresh: group 0 the output head
  // (absent without head planes), group 1 + l layer l; job start, job count,
  // first tile, tile count
  struct TGroup {
    int j0, nj;
    long t0, nt;
  };
  std::vector<TGroup> tgroups;
  std::vector<hipEvent_t> ev_tr;   // group g's transposes done (second stream)
  size_t tr_glue = (size_t)-1;     // the hierarchical glue matrices' transpose group (bf16)
  hipEvent_t ev_tr_fork = nullptr;
  bool mt_stale = false;           // the transposed mirror lags the last update
  bool tr_overlap = false;         // this forward refreshes it on the second stream
  std::vector<uint16_t*> zt, ot, z2t, ht;  // transposed activations per layer
  // attention over producer-transposed operands (T a multiple of 64): q|k|v^T
  // and LSE^T per layer, dO planes in both orientations and Delta^T scratch
  bool attn_tt = false;
  std::vector<float*> lset;
  uint16_t* dop[2] = {};  // dO hi, lo [M][d]
  float* deltat = nullptr;
  uint16_t *rp[4] = {}, *xp[4] = {}, *qp[4] = {}, *gp[4] = {};  // gradient planes: hi, lo, hi^T, lo^T
  // The dW products (and the parameter-VJP groups) run on a second stream
  // beside the dX chain; their transposed operand planes alternate by layer
  // parity ([kind][parity][hi, lo]; kind r, g, x, q) so the dX chain can
  // write layer l-1's while layer l's are still read.  Events: written
  // (second stream waits) and read (dX chain waits before overwriting).
  hipStream_t stream2 = nullptr;
  uint16_t* pt[4][2][2] = {};
  hipEvent_t ev_w[4][2] = {}, ev_r[4][2] = {}, ev_fork = nullptr, ev_join = nullptr, ev_norm = nullptr;
  // the hierarchy's glue on the second stream: [0, 1] backward written
  // events (the dX chain produced a glue product's dY), [2, 3] the forward's
  // fork and join around the decoder-side products of the encoder output
  hipEvent_t ev_glue[4] = {};
  // norm-weight gradients of the planes path: every RMSNorm backward leaves
  // its per-row-block partial sums in a slot of its own, and one batched
  // reduce at the end of the backward (second stream) forms all dw
  float* norm_part = nullptr;
  sj::RmsReduceJob* norm_jobs = nullptr;
  long norm_njobs = 0, norm_maxd = 0;
  std::vector<long> slot_close, slot_fn, slot_an;  // per stage / per layer (-1: row kernel)
  std::vector<float*> slot_ptr;
  void* ws2 = nullptr;
  // the grouped attention backward's meeting counters (zeroed at creation;
  // every launch leaves them zero): this model's own, not the workspace's,
  // which the other ops of the stream overwrite between launches
  uint32_t* attn_cnt = nullptr;
  // activations
  std::vector<void*> x;  // L+1 residual stream tensors
  std::vector<void*> z, qkv, o, x1, z2, gg, uu, hh;
  std::vector<float*> lse;
  void* hn = nullptr;
  float *logits = nullptr, *dlogits = nullptr, *loss_rows = nullptr;
  // backward scratch
  float *dres[2] = {nullptr, nullptr}, *dx1 = nullptr, *dO = nullptr, *dqkv = nullptr, *dgu = nullptr, *dz = nullptr,
        *delta = nullptr;
  void* ws = nullptr;
  size_t ws_bytes = 0;
  float* rope = nullptr;
  int32_t *ids = nullptr, *targets = nullptr;
  double *loss = nullptr, *sumsq = nullptr;
  // FP64 squared-norm partials written by the gradient producers of the
  // backward (sjh::GradSq): slots used by the last backward, and whether a
  // gradient escaped them (then the update sums the arena)
  static constexpr long GSQ_CAP = 32768;
  double* gsq = nullptr;
  long gsq_count = 0;
  bool gsq_ok = false;
  int32_t* status = nullptr;
  sj_adam_step* step_dev = nullptr;
  // pinned ring of host step records: slot k is reused only after the copy
  // issued from it RING steps earlier has completed (its event)
  static constexpr int RING = 64;
  sj_adam_step* step_host = nullptr;
  hipEvent_t step_done[RING] = {};
  long step = 0;
  long staged = 0;  // SGD step records staged (ring position)
  bool own_stream = false;
  // per-op HIP-event profile (eager steps only)
  bool profiling = false;
  // cold-cache profiling: before every op's event pair the stream writes a
  // buffer twice the Infinity Cache (512 MiB), so the op reads from HBM
  bool cold = false;
  // kernel timing: each GEMM op's kernel records events at its own start and
  // end (hipExtLaunchKernel; its extra packets lengthen the op's own pair)
  bool kernel_events = false;
  bool instep = false;  // profile mode 4: kernel events only, both streams as in the step
  float* flush = nullptr;
  std::vector<hipEvent_t> prof_events;  // start, end, GEMM kernel start, end per recorded op
  std::vector<const char*> prof_names;  // one per recorded op
  std::vector<char> prof_kused;         // the op's GEMM kernel recorded its own events
  std::vector<std::string> prof_kernel; // GEMM kernel the op launched ("" if none)
  std::vector<std::string> agg_names;
  std::vector<double> agg_ms;
  std::vector<long> agg_calls;
  std::vector<std::string> agg_kernel;
  // SGD step driver (optimizer 1) and its parameter VJP
  int optimizer = 0;  // 0 AdamW, 1 SGD
  sj_sgd_config sgd = {};
  sj_sgd_step* sgd_dev = nullptr;
  sj_sgd_step* sgd_host = nullptr;  // pinned ring, as step_host
  uint64_t vjp_rng = 0;             // parameter RNG state (SplitMix64)
  bool vjp = false;                 // some group is compressed
  bool comp[2][3] = {};             // compressed members: [0] q, k, v; [1] gate, up
  bool group_on[2] = {};            // the group has a compressed member
  bool group_all[2] = {};           // every member is compressed (no dense dW GEMM)
  long vjp_R = 0, vjp_blocks = 0, vjp_S = 0, vjp_k = 0;
  float vjp_inverse = 1.f, vjp_eps = 0.f;
  long st_compressed = 0, st_dense = 0, st_basis = 0, st_projection = 0;
  int32_t *vjp_scratch = nullptr, *vjp_cols = nullptr, *vjp_rows = nullptr, *vjp_map = nullptr;
  float* vjp_q = nullptr;
  float* vjp_e = nullptr;
  uint16_t *vjp_eh = nullptr, *vjp_el = nullptr;
  std::vector<float*> vjp_left[2], vjp_coeff[2];  // per layer: A = X^T Q [d][R]; E dY [R+k][width]
  uint8_t *fmeta = nullptr, *fmeta_mat = nullptr;  // GradientPlan tables: update, materialize
  long ftiles = 0;
  double* fpart = nullptr;
  // graph
  bool use_graph = false;
  hipGraphExec_t exec = nullptr;
  hipGraph_t graph = nullptr;
  std::vector<void*> allocations;
};

namespace {

int dalloc(sj_model* m, void** p, size_t bytes) {
  if (bytes == 0) bytes = 256;
  hipError_t e = hipMalloc(p, bytes);
  if (e != hipSuccess) {
    size_t fr = 0, tot = 0;
    hipMemGetInfo(&fr, &tot);
    return sjh::fail(SJ_ERR_CAPACITY, "model allocation: required %zu bytes, available %zu bytes", bytes, fr);
  }
  m->allocations.push_back(*p);
  return SJ_OK;
}

#define TRY(x)              \
  do {                      \
    int _s = (x);           \
    if (_s) return _s;      \
  } while (0)

constexpr long FLUSH_FLOATS = 128L << 20;  // 512 MiB

// Run one op; when profiling, bracket it with a pair of events on the model
// stream (the kernel-profile feature of the reference, lib.rs:451-482).  A
// GEMM op's kernel also records a second pair at its own start and end
// (through the GEMM's profiling hook), which notes the kernel's name.
int prof_mark(sj_model* m, const char* name) {
  size_t k = m->prof_names.size();
  if (4 * k + 4 > m->prof_events.size()) {
    for (int i = 0; i < 128; i++) {
      hipEvent_t e;
      SJ_HIP(hipEventCreate(&e));
      m->prof_events.push_back(e);
    }
  }
  m->prof_names.push_back(name);
  if (m->cold && m->flush) TRY(sj_fill(m->stream, m->flush, SJ_F32, FLUSH_FLOATS, 0.f));
  if (!m->instep) SJ_HIP(hipEventRecord(m->prof_events[4 * k], m->stream));
  sjh::ProfHook& h = sjh::prof_hook();
  h.on = true;
  h.k0 = m->kernel_events ? m->prof_events[4 * k + 2] : nullptr;
  h.k1 = m->kernel_events ? m->prof_events[4 * k + 3] : nullptr;
  h.used = false;
  h.kernel[0] = 0;
  return SJ_OK;
}
int prof_end(sj_model* m) {
  size_t k = m->prof_names.size() - 1;
  sjh::ProfHook& h = sjh::prof_hook();
  m->prof_kused.push_back(h.used ? 1 : 0);
  m->prof_kernel.emplace_back(h.kernel);
  h.on = false;
  h.k0 = h.k1 = nullptr;
  if (!m->instep) SJ_HIP(hipEventRecord(m->prof_events[4 * k + 1], m->stream));
  return SJ_OK;
}
#define OP(name, call)                         \
  do {                                         \
    if (m->profiling) TRY(prof_mark(m, name)); \
    TRY(call);                                 \
    if (m->profiling) TRY(prof_end(m));        \
  } while (0)
// an op that writes gradients: its producer adds FP64 squared-norm partials
// (sjh::GradSq) when the backward armed the hook
#define GOP(name, call)              \
  do {                               \
    sjh::grad_sq().on = true;        \
    OP(name, call);                  \
    sjh::grad_sq().on = false;       \
  } while (0)

// Build reference-layout tensor list and the internal arena layout.
void build_layout(sj_model* m) {
  const long V = m->V;
  long off = 0, ro = 0;
  m->layers.resize(m->L);
  auto add = [&](const std::string& name, long rows, long cols, long ioff, long ild, int layer = -1, int kind = -1,
                 int member = -1, long col0 = 0, int ndim = 2) {
    m->tensors.push_back(RefTensor{name, rows, cols, ro, ioff, ild, layer, kind, member, col0, ndim});
    ro += rows * cols;
  };
  // [no decay] the 1-D tensors: per layer attention_norm, ffn_norm; the
  // closing norms; final_norm
  for (Stage& S : m->stages)
    for (long l = S.first; l < S.first + S.count; l++) {
      m->layers[l].stage = S.index;
      m->layers[l].an = off; off = align64(off + S.d);
      m->layers[l].fn = off; off = align64(off + S.d);
    }
  for (Stage& S : m->stages)
    if (m->hier) { S.norm = off; off = align64(off + S.d); }
  m->final_norm = off; off = align64(off + m->d);
  if (!m->hier) m->stages[0].norm = m->final_norm;
  m->n_nodecay = off;
  // [decay] embedding, the block matrices, the hierarchy's projections and
  // BOS row, the head
  m->emb = off; off = align64(off + V * m->stages[0].d);
  const long NE = m->E > 0 ? m->E : 1;  // expert copies of gate|up and down
  for (Stage& S : m->stages)
    for (long l = S.first; l < S.first + S.count; l++) {
      m->layers[l].qkv = off; off = align64(off + S.d * S.NQKV);
      m->layers[l].wo = off; off = align64(off + S.d * S.d);
      m->layers[l].gu = off; off = align64(off + NE * S.d * 2 * S.F);
      m->layers[l].down = off; off = align64(off + NE * S.F * S.d);
      if (m->E) { m->layers[l].router = off; off = align64(off + S.d * m->E); }
    }
  if (m->hier) {
    const long de = m->stages[0].d, dg = m->stages[1].d, dd = m->stages[2].d;
    m->h_inproj = off; off = align64(off + dg * de);
    m->h_e2g = off; off = align64(off + de * dg);
    m->h_e2d = off; off = align64(off + de * dd);
    m->h_g2d = off; off = align64(off + dg * dd);
    m->h_bos = off; off = align64(off + dg);
    m->h_op = off; off = align64(off + dd * dg);
  }
  m->out = off; off = align64(off + m->d * m->Vp);
  if (m->value_n) { m->bias = off; off = align64(off + m->Vp); }  // [1][n]: 2-D, so it decays
  m->n_params = off;

  // stage_layout (architecture.rs:63-95): per layer the two norms, the four
  // attention matrices, gate, up, down
  auto blocks = [&](const Stage& S) {
    const long d = S.d, J = S.J, F = S.F;
    for (long l = S.first; l < S.first + S.count; l++) {
      std::string p = S.prefix + "." + std::to_string(l - S.first) + ".";
      const Layer& y = m->layers[l];
      add(p + "attention_norm", 1, d, y.an, d, -1, -1, -1, 0, 1);
      add(p + "ffn_norm", 1, d, y.fn, d, -1, -1, -1, 0, 1);
      const int li = (int)l;
      add(p + "query", d, d, y.qkv, S.NQKV, li, 0, 0, 0);
      add(p + "key", d, J, y.qkv + d, S.NQKV, li, 0, 1, d);
      add(p + "value", d, J, y.qkv + d + J, S.NQKV, li, 0, 2, d + J);
      add(p + "attention_output", d, d, y.wo, d);
      if (m->E) {  // experts.<e>.gate / up / down, then router
        for (long e = 0; e < m->E; e++) {
          const std::string q = p + "experts." + std::to_string(e) + ".";
          add(q + "gate", d, F, y.gu + e * d * 2 * F, 2 * F);
          add(q + "up", d, F, y.gu + e * d * 2 * F + F, 2 * F);
          add(q + "down", F, d, y.down + e * F * d, d);
        }
        add(p + "router", d, m->E, y.router, m->E);
        continue;
      }
      add(p + "gate", d, F, y.gu, 2 * F, li, 1, 0, 0);
      add(p + "up", d, F, y.gu + F, 2 * F, li, 1, 1, F);
      add(p + "down", F, d, y.down, d);
    }
  };
  const long d = m->d;
  if (m->hier) {
    // layout (architecture.rs:96-137): embedding, encoder blocks,
    // encoder_norm, input_projection, encoder_to_global, encoder_to_decoder,
    // global_to_decoder, global_bos, global_norm, global blocks, decoder
    // blocks, decoder_norm, output_projection, final_norm, output
    const Stage &E = m->stages[0], &G = m->stages[1], &D = m->stages[2];
    add("embedding", V, E.d, m->emb, E.d);
    blocks(E);
    add("encoder_norm", 1, E.d, E.norm, E.d, -1, -1, -1, 0, 1);
    add("input_projection", G.d, E.d, m->h_inproj, E.d);
    add("encoder_to_global", E.d, G.d, m->h_e2g, G.d);
    add("encoder_to_decoder", E.d, D.d, m->h_e2d, D.d);
    add("global_to_decoder", G.d, D.d, m->h_g2d, D.d);
    add("global_bos", 1, G.d, m->h_bos, G.d);
    add("global_norm", 1, G.d, G.norm, G.d, -1, -1, -1, 0, 1);
    blocks(G);
    blocks(D);
    add("decoder_norm", 1, D.d, D.norm, D.d, -1, -1, -1, 0, 1);
    add("output_projection", D.d, G.d, m->h_op, G.d);
    add("final_norm", 1, d, m->final_norm, d, -1, -1, -1, 0, 1);
    add("output", d, m->HV, m->out, m->Vp);
    m->ref_count = ro;
    return;
  }
  // NativeValue::parameters (native/value.rs:89-115): the body without its
  // embedding and output, then native_embedding [259][d], native_value
  // [d][n] and native_bias [1][n]
  if (!m->value_n) add("embedding", V, d, m->emb, d);
  blocks(m->stages[0]);
  add("final_norm", 1, d, m->final_norm, d, -1, -1, -1, 0, 1);
  if (m->value_n) {
    add("native_embedding", V, d, m->emb, d);
    add("native_value", d, m->HV, m->out, m->Vp);
    add("native_bias", 1, m->HV, m->bias, m->Vp);
  } else {
    add("output", d, m->HV, m->out, m->Vp);
  }
  m->ref_count = ro;
}

// reference <-> internal host conversion
void ref_to_internal(const sj_model* m, const float* ref, float* in) {
  for (const auto& t : m->tensors)
    for (long r = 0; r < t.rows; r++)
      memcpy(in + t.int_offset + r * t.int_ld, ref + t.ref_offset + r * t.cols, sizeof(float) * t.cols);
}
void internal_to_ref(const sj_model* m, const float* in, float* ref) {
  for (const auto& t : m->tensors)
    for (long r = 0; r < t.rows; r++)
      memcpy(ref + t.ref_offset + r * t.cols, in + t.int_offset + r * t.int_ld, sizeof(float) * t.cols);
}

// compute-precision view of a parameter (bf16 mirror or the fp32 master)
const void* wc(const sj_model* m, long off) {
  return m->dt == SJ_BF16 ? (const void*)(m->mirror + off) : (const void*)(m->w + off);
}

int transpose_mirror(sj_model* m) {
  if (!m->planes) return SJ_OK;
  hipLaunchKernelGGL(k_transpose_jobs, dim3((unsigned)m->tjob_tiles), dim3(256), 0, m->stream, m->mirror, m->mirror_t,
                     m->tjobs, m->tjob_n, (const float*)m->w, TPlanes{m->hp[0], m->hp[1], m->hp[2], m->hp[3]}, 0L);
  SJ_LAUNCH_CHECK("mirror transpose");
  m->mt_stale = false;
  return SJ_OK;
}

// The transposed mirror rebuilt on the second stream one group at a time
// (layer 0 first, the head last), each group's event marking it done: the
// forward's layer l waits only for its own matrices, so the rest of the
// refresh runs beside the forward instead of ahead of it.
int transpose_mirror_overlapped(sj_model* m) {
  hipStream_t s2 = m->stream2;
  SJ_HIP(hipEventRecord(m->ev_tr_fork, m->stream));  // after the last update wrote the mirror
  SJ_HIP(hipStreamWaitEvent(s2, m->ev_tr_fork, 0));
  const TPlanes hp{m->hp[0], m->hp[1], m->hp[2], m->hp[3]};
  const size_t n = m->tgroups.size();
  for (size_t k = 0; k < n; k++) {
    const size_t gidx = (k + 1) % n;  // layers first, the head (group 0) last
    const sj_model::TGroup& g = m->tgroups[gidx];
    if (g.nt > 0)
      hipLaunchKernelGGL(k_transpose_jobs, dim3((unsigned)g.nt), dim3(256), 0, s2, m->mirror, m->mirror_t,
                         m->tjobs + g.j0, g.nj, (const float*)m->w, hp, g.t0);
    SJ_HIP(hipEventRecord(m->ev_tr[gidx], s2));
  }
  SJ_LAUNCH_CHECK("mirror transpose (overlapped)");
  m->mt_stale = false;
  return SJ_OK;
}

// the forward's layer l (group 1 + l) or head (group 0) may read its
// transposed matrices from here on
int await_transposed(sj_model* m, hipStream_t s, size_t group) {
  if (!m->tr_overlap || group >= m->ev_tr.size()) return SJ_OK;
  SJ_HIP(hipStreamWaitEvent(s, m->ev_tr[group], 0));
  return SJ_OK;
}

int refresh_mirror(sj_model* m) {
  if (m->dt != SJ_BF16) return SJ_OK;
  TRY(sj_cast(m->stream, m->w, SJ_F32, m->mirror, SJ_BF16, m->n_params));
  return transpose_mirror(m);
}

// ---------------------------------------------------------------- forward
// stored activations of layer l: its input and output on the residual stream
void* xin(const sj_model* m, long l) { return m->x[l + m->layers[l].stage]; }
void* xout(const sj_model* m, long l) { return m->x[l + m->layers[l].stage + 1]; }
// the stage's last residual (the closing norm's input)
void* xtop(const sj_model* m, const Stage& S) { return m->x[S.first + S.count + S.index]; }

// Block::apply for every layer of stage si (architecture.rs:200-247), then
// its closing norm into S.out
int stage_forward(sj_model* m, int si) {
  const Stage& S = m->stages[si];
  hipStream_t s = m->stream;
  const long M = S.M, d = S.d, J = S.J, F = S.F, NQ = S.NQKV, ldt = S.ldt;
  const int dt = m->dt;
  const float eps = m->c.norm_epsilon;
  for (long l = S.first; l < S.first + S.count && m->planes; l++) {
    const Layer& y = m->layers[l];
    TRY(await_transposed(m, s, (size_t)(1 + l)));
    uint16_t* qkv = (uint16_t*)m->qkv[l];
    const uint16_t *W = m->mirror, *WT = m->mirror_t;
    const uint16_t *x = (const uint16_t*)xin(m, l), *x1 = (const uint16_t*)m->x1[l];
    uint16_t *z = (uint16_t*)m->z[l], *z2 = (uint16_t*)m->z2[l], *o = (uint16_t*)m->o[l];
    uint16_t *gg = (uint16_t*)m->gg[l], *uu = (uint16_t*)m->uu[l], *hh = (uint16_t*)m->hh[l];
    if (l == 0)  // the embedding lookup fused in (forward() leaves it to this norm)
      OP("rmsnorm", sjh::rmsnorm_fwd_t_embed(s, W + m->emb, m->ids, (uint16_t*)m->x[0], W + y.an, z,
                                             m->rowdw ? nullptr : m->zt[l], ldt, M, d, eps));
    else
      OP("rmsnorm", sj_rmsnorm_fwd_t(s, x, W + y.an, z, m->rowdw ? nullptr : m->zt[l], ldt, M, d, eps));
    OP("qkv_rope", sj_qkv_fwd_t(s, z, d, M, d, WT + y.qkv, d, d, J, qkv, NQ, S.rope, S.T, S.Dh, nullptr, ldt));
    if (S.attn_tt)
      OP("attention_fwd", sj_attention_fwd_tt(s, qkv, NQ, ldt, m->B, S.T, S.HQ, S.HK, S.Dh, S.window, o, d,
                                              m->lse[l], m->lset[l], m->rowdw ? nullptr : m->ot[l], ldt));
    else
      OP("attention_fwd", sj_attention_fwd_t(s, qkv, NQ, qkv + d, NQ, qkv + d + J, NQ, o, d, m->lse[l], m->ot[l],
                                             ldt, m->B, S.T, S.HQ, S.HK, S.Dh));
    OP("attn_out_residual", sj_linear_residual_fwd_t(s, o, d, M, d, WT + y.wo, d, d, x, d, (uint16_t*)m->x1[l], d));
    OP("rmsnorm", sj_rmsnorm_fwd_t(s, x1, W + y.fn, z2, m->rowdw ? nullptr : m->z2t[l], ldt, M, d, eps));
    if (m->E) {  // Block::apply's MoE branch (architecture.rs:229-242), packed by expert on the device
      const long E = m->E, K = m->K, cap = m->cap;
      if (m->mhist && sjh::router_pack_ok(d, d, E, K, z2, W + y.router, m->mlog[l])) {
        // the top-k also counts each workgroup's routed slots; the pack
        // places them from those counts in parallel
        OP("router_topk", sjh::router_topk_hist(s, z2, d, W + y.router, d, M, E, K, (uint16_t*)m->mlog[l],
                                                m->mids[l], m->mwts[l], m->mhist));
        OP("route_pack", sjh::route_pack_hist(s, m->mids[l], M, K, E, m->mhist, m->mcnt[l], m->moff[l], m->mps[l],
                                              m->mpp[l], cap));
      } else {
        OP("router_topk", sj_router_topk(s, z2, d, W + y.router, d, M, E, K, m->mlog[l], m->mids[l], m->mwts[l]));
        OP("route_pack", sj_route_pack(s, m->mids[l], M, K, E, nullptr, nullptr, m->mcnt[l], m->moff[l], m->mps[l],
                                       m->mpp[l], cap));
      }
      OP("moe_gather", sj_moe_gather(s, z2, d, d, m->mps[l], K, cap, m->mzp[l], m->rowdw ? nullptr : m->mzpt[l], cap));
      OP("expert_gate_up", sj_moe_gate_up_fwd(s, m->moff[l], E, cap, m->mzp[l], d, d, WT + y.gu, WT + y.gu + F * d, d,
                                              2 * F * d, F, gg, uu, hh, F, m->rowdw ? nullptr : m->ht[l], cap));
      OP("expert_down", sj_moe_down_fwd(s, m->moff[l], E, cap, hh, F, F, WT + y.down, F, d * F, d, m->myp[l], d));
      OP("combine_residual", sj_moe_combine(s, m->myp[l], d, d, m->mids[l], m->mpp[l], m->mwts[l], M, K, x1, d,
                                            (uint16_t*)xout(m, l), d));
      continue;
    }
    OP("gate_up_swiglu", sj_gate_up_fwd_t(s, z2, d, M, d, WT + y.gu, WT + y.gu + F * d, d, F, gg, uu, hh, F,
                                          m->rowdw ? nullptr : m->ht[l], ldt));
    OP("down_residual", sj_linear_residual_fwd_t(s, hh, F, M, F, WT + y.down, F, d, x1, d, (uint16_t*)xout(m, l), d));
  }
  for (long l = S.first; l < S.first + S.count && !m->planes; l++) {
    const Layer& y = m->layers[l];
    char* qkv = (char*)m->qkv[l];
    OP("rmsnorm", sj_rmsnorm_fwd(s, xin(m, l), dt, wc(m, y.an), dt, m->z[l], M, d, eps));
    const char* wq = (const char*)wc(m, y.qkv);
    OP("qkv_rope", sj_qkv_fwd(s, m->z[l], d, M, d, wq, NQ, wq + d * m->esz, NQ, wq + (d + J) * m->esz, NQ, d, J, qkv, NQ,
                   qkv + d * m->esz, NQ, qkv + (d + J) * m->esz, NQ, dt, S.rope, S.T, S.Dh));
    OP("attention_fwd", sj_attention_fwd(s, qkv, NQ, qkv + d * m->esz, NQ, qkv + (d + J) * m->esz, NQ, m->o[l], d,
                                         m->lse[l], dt, m->B, S.T, S.HQ, S.HK, S.Dh, S.window));
    OP("attn_out_residual", sj_linear_residual_fwd(s, m->o[l], d, M, d, wc(m, y.wo), d, d, xin(m, l), d, m->x1[l], d, dt));
    OP("rmsnorm", sj_rmsnorm_fwd(s, m->x1[l], dt, wc(m, y.fn), dt, m->z2[l], M, d, eps));
    const char* wg = (const char*)wc(m, y.gu);
    OP("gate_up_swiglu", sj_gate_up_fwd(s, m->z2[l], d, M, d, wg, 2 * F, wg + F * m->esz, 2 * F, F, m->gg[l], m->uu[l], m->hh[l], F, dt));
    OP("down_residual", sj_linear_residual_fwd(s, m->hh[l], F, M, F, wc(m, y.down), d, d, m->x1[l], d, xout(m, l), d, dt));
  }
  OP("rmsnorm", sj_rmsnorm_fwd(s, xtop(m, S), dt, wc(m, S.norm), dt, S.out, M, d, eps));
  return SJ_OK;
}

// hidden_from_encoded (architecture.rs:368-393) after the encoder stage:
// pool the encoded bytes into patches, encoder_to_global, the global stage,
// global_to_decoder of its output and of the BOS row, the shift-by-one-patch
// broadcast added to encoder_to_decoder of the encoded bytes, the decoder
// stage, output_projection and the final norm (into hn).  Every product
// stores in the compute dtype (Graph::matmul, graph.rs:212-221).
bool two_streams(const sj_model* m);
int hierarchy_forward(sj_model* m) {
  hipStream_t s = m->stream;
  const int dt = m->dt;
  const float eps = m->c.norm_epsilon;
  const Stage &E = m->stages[0], &G = m->stages[1], &D = m->stages[2];
  const long B = m->B, P = m->P, de = E.d, dg = G.d, dd = D.d, Ml = E.M, Mg = G.M;
  void* ws = m->ws;
  const size_t wsb = m->ws_bytes;
  // the BOS row's projection (parameters only) and encoder_to_decoder (the
  // encoder output only) run on the second stream beside the pool, the
  // global stage and global_to_decoder; the broadcast waits for both
  const bool two = two_streams(m);
  hipStream_t s2 = two ? m->stream2 : s;
  void* ws2 = two ? m->ws2 : ws;
  if (two) {
    SJ_HIP(hipEventRecord(m->ev_glue[2], s));
    SJ_HIP(hipStreamWaitEvent(s2, m->ev_glue[2], 0));
  }
  OP("bos_to_decoder", sj_gemm(s2, 0, 0, 1, dd, dg, wc(m, m->h_bos), dt, dg, wc(m, m->h_g2d), dt, dd, m->bosd, dt, dd, 0,
                               ws2, wsb));
  // bf16: the glue products on the MFMA layout, each weight's transposed
  // mirror the [N][K] operand (the second stream runs any transposes first)
  const bool pl = dt == SJ_BF16 && m->mirror_t && m->tr_glue != (size_t)-1 && (de | dg | dd) % 8 == 0;
  const uint16_t* WT = m->mirror_t;
  if (pl)
    OP("encoder_to_decoder", sj_gemm_planes(s2, Ml, dd, de, (const uint16_t*)E.out, nullptr, de, WT + m->h_e2d, nullptr,
                                            de, m->bytes, SJ_BF16, dd, 0, ws2, wsb));
  else
    OP("encoder_to_decoder", sj_gemm(s2, 0, 0, Ml, dd, de, E.out, dt, de, wc(m, m->h_e2d), dt, dd, m->bytes, dt, dd, 0,
                                     ws2, wsb));
  OP("patch_pool", sj_patch_pool(s, E.out, dt, B, E.T, de, P, m->pooled));
  if (pl) {
    TRY(await_transposed(m, s, m->tr_glue));
    OP("encoder_to_global", sj_gemm_planes(s, Mg, dg, de, (const uint16_t*)m->pooled, nullptr, de, WT + m->h_e2g,
                                           nullptr, de, xin(m, G.first), SJ_BF16, dg, 0, ws, wsb));
  } else {
    OP("encoder_to_global", sj_gemm(s, 0, 0, Mg, dg, de, m->pooled, dt, de, wc(m, m->h_e2g), dt, dg, xin(m, G.first),
                                    dt, dg, 0, ws, wsb));
  }
  TRY(stage_forward(m, 1));
  if (pl)
    OP("global_to_decoder", sj_gemm_planes(s, Mg, dd, dg, (const uint16_t*)G.out, nullptr, dg, WT + m->h_g2d, nullptr,
                                           dg, m->gd, SJ_BF16, dd, 0, ws, wsb));
  else
    OP("global_to_decoder", sj_gemm(s, 0, 0, Mg, dd, dg, G.out, dt, dg, wc(m, m->h_g2d), dt, dd, m->gd, dt, dd, 0, ws,
                                    wsb));
  if (two) {
    SJ_HIP(hipEventRecord(m->ev_glue[3], s2));
    SJ_HIP(hipStreamWaitEvent(s, m->ev_glue[3], 0));
  }
  OP("patch_broadcast", sj_patch_broadcast(s, m->gd, m->bosd, dt, B, E.T, dd, P, m->zb));
  OP("decoder_input", sj_add(s, m->bytes, dt, m->zb, dt, xin(m, D.first), dt, Ml * dd, 1.f));
  TRY(stage_forward(m, 2));
  if (pl)
    OP("output_projection", sj_gemm_planes(s, Ml, dg, dd, (const uint16_t*)D.out, nullptr, dd, WT + m->h_op, nullptr,
                                           dd, m->opo, SJ_BF16, dg, 0, ws, wsb));
  else
    OP("output_projection", sj_gemm(s, 0, 0, Ml, dg, dd, D.out, dt, dd, wc(m, m->h_op), dt, dg, m->opo, dt, dg, 0, ws,
                                    wsb));
  OP("rmsnorm", sj_rmsnorm_fwd(s, m->opo, dt, wc(m, m->final_norm), dt, m->hn, Ml, dg, eps));
  return SJ_OK;
}

int forward(sj_model* m);
bool two_streams(const sj_model* m);
// The gradient-norm partials cover every gradient of the bf16 byte LM step
// with AdamW (dW products through the split-K reduce, the norm weights, the
// embedding); the other models sum the arena.
bool gsq_eligible(const sj_model* m) {
  return m->planes && m->lm_planes && !m->E && !m->hier && !m->value_n && m->optimizer == 0 && !m->vjp;
}
// the step's forward: the loss sum waits for the backward's second stream,
// and the transposed mirror, unless the last update wrote it, is rebuilt
// beside the forward
int forward_deferred(sj_model* m) {
  m->defer_loss = !m->value_n && two_streams(m);
  m->tr_overlap = !m->fused_update && two_streams(m) && !m->tgroups.empty();
  const int st = forward(m);
  m->tr_overlap = false;
  if (st) m->defer_loss = false;
  return st;
}

int forward(sj_model* m) {
  hipStream_t s = m->stream;
  const long M = m->M, d = m->d;
  const int dt = m->dt;
  if (m->tr_overlap)
    OP("mirror_transpose", transpose_mirror_overlapped(m));
  else if (m->mt_stale)
    OP("mirror_transpose", transpose_mirror(m));
  // the MFMA-layout blocks fold the lookup into the first block's norm
  if (!(m->planes && m->L > 0 && m->stages[0].count > 0))
    OP("embedding", sj_embedding_fwd(s, wc(m, m->emb), dt, m->ids, m->x[0], dt, m->stages[0].M, m->stages[0].d));
  TRY(stage_forward(m, 0));
  if (m->hier) TRY(hierarchy_forward(m));
  if (m->value_n) {
    // NativeValue::forward_batch (native/value.rs:139-146): gather the SEP
    // rows, cast to F32, affine head (matmul + bias_add), then the mean CE
    // of the value labels (train_value, memory.rs:977-979)
    const long R = m->HR, n = m->HV;
    OP("value_gather", sj_gather_rows(s, m->hn, dt, d, m->sel, R, d, m->hsel, SJ_F32));
    OP("head_fwd", sj_gemm(s, 0, 0, R, n, d, m->hsel, SJ_F32, d, m->w + m->out, SJ_F32, m->Vp, m->logits, SJ_F32, m->Vp,
                           0, m->ws, m->ws_bytes));
    OP("value_bias", sj_bias_add(s, m->logits, m->Vp, m->w + m->bias, m->logits, m->Vp, R, n));
    OP("cross_entropy", sj_cross_entropy(s, m->logits, m->Vp, m->labels, m->loss_rows, m->dlogits, m->Vp, R, n,
                                         nullptr, 1.0f / (float)R));
    OP("loss_summary", sj_loss_summary(s, m->loss_rows, R, m->loss, m->obs_slot, 1.0f / (float)m->obs));
    return SJ_OK;
  }
  // fp32 head on the fp32 master (architecture.rs:160-167); hn's values are
  // exact in fp32 (Graph::cast to F32), so it is read in its storage dtype.
  // On the planes path the master enters as hi + lo bf16 planes (2^-17
  // relative) and the cross entropy leaves dlogits as hi/lo planes.
  // scale / count (graph.rs:546) with the objective's seed scale =
  // loss_scale / accumulation (train lib.rs:409) for AdamW; the SGD driver's
  // update takes its gradients unscaled (loss_scale 1 with the VJP)
  const float scale = m->optimizer == 1 ? 1.0f : m->adam.loss_scale / (float)m->obs;
  const float seed = scale / (float)M;
  if (m->lm_planes) {
    // no split-K (no workspace): a row's sum order does not depend on M,
    // so the cached forward's one-row product gives the same logits
    TRY(await_transposed(m, s, 0));
    OP("head_fwd", sj_gemm_planes(s, M, m->Vp, d, (const uint16_t*)m->hn, nullptr, d, m->hp[2], m->hp[3], d,
                                  m->logits, SJ_F32, m->Vp, 0, nullptr, 0));
    OP("cross_entropy", sjh::cross_entropy_planes(s, m->logits, m->Vp, m->targets, m->loss_rows, m->dlp[0], m->dlp[1],
                                                  m->Vp, M, m->HV, seed));
  } else {
    OP("head_fwd", sj_gemm(s, 0, 0, M, m->HV, d, m->hn, dt, d, m->w + m->out, SJ_F32, m->Vp, m->logits, SJ_F32, m->Vp, 0,
                           m->ws, m->ws_bytes));
    OP("cross_entropy", sj_cross_entropy(s, m->logits, m->Vp, m->targets, m->loss_rows, m->dlogits, m->Vp, M, m->HV,
                                         nullptr, seed));
  }
  // the loss sum is read only by read_loss: in a training step it runs on
  // the second stream after the backward's fork, off the dX chain
  if (!m->defer_loss)
    OP("loss_summary", sj_loss_summary(s, m->loss_rows, M, m->loss, m->obs_slot, 1.0f / (float)m->obs));
  return SJ_OK;
}

// ------------------------------------------------------- parameter VJP
// One projection group's factored gradient (compressed_parameter_vjp,
// graph.rs:915-1005): prepare (A = X^T Q and the E rows) from the group's
// stored input, then E dY over the concatenated member outputs (Engine::
// parameter_vjp, parameter_vjp.rs:308-320).  The first group of the
// backward (the last layer's gate/up group) draws the feature selection and
// the forward basis from the up projection's output (its widest member,
// the last one on ties: graph.rs:931-934); every later group reuses both
// (one basis per (tokens, rank), one selection per width, graph.rs:
// 957-982), so one seed is consumed per step.  Row-layout dW (rowdw): the
// group's stored input and the dX chain's gradient planes are read as they
// are; otherwise their transposed copies (x^T, dY^T).
int vjp_group(sj_model* m, long l, int kind, hipStream_t s, void* ws, size_t wsb, uint16_t* const* dy) {
  const long M = m->M, d = m->d, F = m->F, R = m->vjp_R, k = m->vjp_k, ldt = m->ldt;
  const long width = kind == 0 ? m->NQKV : 2 * F;
  if (l == m->L - 1 && kind == 1) {
    const uint64_t* seed = (const uint64_t*)((const char*)m->sgd_dev + offsetof(sj_sgd_step, seed));
    OP("pvjp_indices", sjh::pvjp_indices_dev(s, seed, d, F, m->vjp_blocks, m->vjp_S, R, m->sgd.vjp_block_rows,
                                             m->vjp_scratch, m->vjp_cols, m->vjp_rows, m->vjp_map));
    OP("pvjp_basis", sj_pvjp_basis(s, m->uu[m->L - 1], SJ_BF16, F, M, m->vjp_cols, R, m->vjp_eps, m->vjp_q, ws, wsb));
  }
  if (m->rowdw) {
    const uint16_t* x = (const uint16_t*)(kind == 0 ? m->z[l] : m->z2[l]);
    OP("pvjp_prepare", sj_pvjp_prepare_rows(s, x, d, d, M, m->vjp_q, R, m->vjp_rows, k, m->vjp_inverse,
                                            m->vjp_left[kind][l], nullptr, m->vjp_eh, m->vjp_el, ldt, ws, wsb));
    OP("pvjp_coefficients", sj_pvjp_vjp_rows(s, m->vjp_eh, m->vjp_el, ldt, R + k, M, dy[0], dy[1], width, width,
                                             m->vjp_coeff[kind][l], width, ws, wsb));
    return SJ_OK;
  }
  const uint16_t* xt = kind == 0 ? m->zt[l] : m->z2t[l];
  OP("pvjp_prepare", sj_pvjp_prepare(s, xt, ldt, d, M, m->vjp_q, R, m->vjp_rows, k, m->vjp_inverse,
                                     m->vjp_left[kind][l], nullptr, m->vjp_eh, m->vjp_el, ldt, ws, wsb));
  OP("pvjp_coefficients", sj_pvjp_vjp(s, m->vjp_eh, m->vjp_el, ldt, R + k, M, dy[0], dy[1], ldt, width,
                                      m->vjp_coeff[kind][l], width, ws, wsb));
  return SJ_OK;
}

// --------------------------------------------------------------- backward
// The dW products (and parameter-VJP groups) run on a second stream beside
// the dX chain (planes path, graph and plain eager steps; per-op profiling
// keeps one stream).
bool two_streams(const sj_model* m) { return m->planes && (!m->profiling || m->instep); }

// Backward of stage si from dzin = d(closing norm output) [M][d] (fp32):
// the closing norm, then per layer from the top down / SwiGLU / gate+up /
// ffn norm / attention output / attention (+ inverse RoPE) / QKV /
// attention norm (graph.rs:567-911 in one block's order).  Leaves
// d(stage input) in m->dres[cur].
int stage_backward(sj_model* m, int si, const float* dzin, int& cur) {
  const Stage& S = m->stages[si];
  hipStream_t s = m->stream;
  const long M = S.M, d = S.d, J = S.J, F = S.F, NQ = S.NQKV, ldt = S.ldt;
  const long top = S.first + S.count - 1;
  const int dt = m->dt;
  const float eps = m->c.norm_epsilon;
  float* G = m->g;
  if (m->planes) {
    const uint16_t* W = m->mirror;
    void* ws = m->ws;
    const size_t wsb = m->ws_bytes;
    uint16_t **rp = m->rp, **xp = m->xp, **qp = m->qp, **gp = m->gp;
    const bool two = two_streams(m);
    hipStream_t s2 = two ? m->stream2 : s;
    void* ws2 = two ? m->ws2 : ws;
    enum { KR = 0, KG = 1, KX = 2, KQ = 3 };
    auto written = [&](int k, int p) -> int {  // s2 may read planes (k, p) from here on
      if (!two) return SJ_OK;
      SJ_HIP(hipEventRecord(m->ev_w[k][p], s));
      SJ_HIP(hipStreamWaitEvent(s2, m->ev_w[k][p], 0));
      return SJ_OK;
    };
    auto read = [&](int k, int p) -> int {  // s2 is done with planes (k, p)
      if (!two) return SJ_OK;
      SJ_HIP(hipEventRecord(m->ev_r[k][p], s2));
      return SJ_OK;
    };
    auto reuse = [&](int k, int p) -> int {  // the dX chain may overwrite planes (k, p)
      if (!two) return SJ_OK;
      SJ_HIP(hipStreamWaitEvent(s, m->ev_r[k][p], 0));
      return SJ_OK;
    };
    auto T = [&](int k, int p) { return m->pt[k][p]; };
    // gradient planes of kind k for layer parity p: the row-orientation pair
    // [M][width] the dX products read (and, row-layout dW, the dW products),
    // and the transposed pair [width][ldt] (nullptr under row-layout dW)
    uint16_t* const nul[2] = {nullptr, nullptr};
    uint16_t* const* normal[4] = {rp, gp, xp, qp};
    const bool rdw = m->rowdw;
    auto NP = [&](int k, int p) -> uint16_t* const* { return rdw ? m->pt[k][p] : normal[k]; };
    auto TP = [&](int k, int p) -> uint16_t* const* { return rdw ? nul : m->pt[k][p]; };
    {
      const int p = (int)(top & 1);
      TRY(reuse(KR, p));
      OP("rmsnorm_bwd", sjh::rmsnorm_bwd_p_deferred(s, (const uint16_t*)xtop(m, S), W + S.norm, dzin, nullptr,
                                                    m->dres[cur], NP(KR, p)[0], NP(KR, p)[1], TP(KR, p)[0],
                                                    TP(KR, p)[1], ldt, M, d, eps, m->slot_ptr[m->slot_close[si]]));
      TRY(written(KR, p));
    }
    for (long l = top; l >= S.first; l--) {
      const Layer& y = m->layers[l];
      const uint16_t* qkv = (const uint16_t*)m->qkv[l];
      const int p = (int)(l & 1);
      if (m->E) {
        // x_{l+1} = x1 + combine(experts(z2)): combine backward (dY of every
        // packed row, routing-weight gradients), the experts' down dX with the
        // SwiGLU derivative, gate|up dX, the gather's sum with the routing and
        // router backward into dz; the experts' and router's dW on the second
        // stream from this layer's own planes
        const long E = m->E, K = m->K, cap = m->cap;
        uint16_t* mx[4] = {m->mdx[0][l], m->mdx[1][l], m->mdx[2][l], m->mdx[3][l]};
        uint16_t* mg[4] = {m->mdg[0][l], m->mdg[1][l], m->mdg[2][l], m->mdg[3][l]};
        TRY(read(KR, p));  // the rp transposed planes go unread here
        OP("combine_bwd", sj_moe_combine_bwd(s, m->myp[l], d, d, m->mps[l], m->mwts[l], K, cap, m->dres[cur], d, mx[0],
                                             mx[1], rdw ? nullptr : mx[2], rdw ? nullptr : mx[3], cap,
                                             m->mdwts[l]));
        OP("expert_down_dx_swiglu", sj_moe_down_bwd_swiglu_p(s, m->moff[l], E, cap, mx[0], mx[1], d, d, W + y.down, d,
                                                             F * d, F, (const uint16_t*)m->gg[l],
                                                             (const uint16_t*)m->uu[l], F, mg[0], mg[1], 2 * F,
                                                             rdw ? nullptr : mg[2], rdw ? nullptr : mg[3], cap));
        if (two) {
          SJ_HIP(hipEventRecord(m->ev_moe[0][l], s));
          SJ_HIP(hipStreamWaitEvent(s2, m->ev_moe[0][l], 0));
        }
        if (rdw)
          OP("expert_down_dw", sj_moe_gemm_dw_tn(s2, m->moff[l], E, cap, F, d, (const uint16_t*)m->hh[l], F, mx[0],
                                                 mx[1], d, G + y.down, d, F * d));
        else
          OP("expert_down_dw", sj_moe_gemm_dw(s2, m->moff[l], E, cap, F, d, m->ht[l], cap, mx[2], mx[3], cap,
                                              G + y.down, d, F * d));
        OP("expert_gate_up_dx", sj_moe_gemm_rows(s, m->moff[l], E, cap, d, 2 * F, mg[0], mg[1], 2 * F, W + y.gu, 2 * F,
                                                 d * 2 * F, m->mdzp, d, 0));
        if (rdw)
          OP("expert_gate_up_dw", sj_moe_gemm_dw_tn(s2, m->moff[l], E, cap, d, 2 * F, m->mzp[l], d, mg[0], mg[1],
                                                    2 * F, G + y.gu, 2 * F, d * 2 * F));
        else
          OP("expert_gate_up_dw", sj_moe_gemm_dw(s2, m->moff[l], E, cap, d, 2 * F, m->mzpt[l], cap, mg[2], mg[3],
                                                 cap, G + y.gu, 2 * F, d * 2 * F));
        OP("gather_route_bwd", sj_moe_gather_bwd(s, m->mdzp, d, d, m->mids[l], m->mpp[l], m->mwts[l], m->mlog[l],
                                                 m->mdwts[l], W + y.router, M, K, E, nullptr, d, m->dz, d,
                                                 m->mdlog[l]));
        if (two) {
          SJ_HIP(hipEventRecord(m->ev_moe[1][l], s));
          SJ_HIP(hipStreamWaitEvent(s2, m->ev_moe[1][l], 0));
        }
        OP("router_dw", sj_gemm(s2, 1, 0, d, E, M, m->z2[l], SJ_BF16, d, m->mdlog[l], SJ_F32, E, G + y.router, SJ_F32, E,
                                0, ws2, wsb));
      } else {
      // x_{l+1} = x1 + down(h): down's dW needs only the planes of dY (kind
      // KR, written above this layer).  While the layer's products leave
      // CUs idle (M F <= 8 Mi: cfg2, cfg3) it goes on the second stream
      // before that stream waits for the SwiGLU derivative's planes, beside
      // the dX product (cfg2 1.865 -> 1.821 ms/step); at cfg5's size it
      // would slow that product as much as it gains, so it follows it.
      auto down_dw = [&]() -> int {
        if (rdw)
          GOP("down_dw", sj_gemm_planes_tn(s2, F, d, M, (const uint16_t*)m->hh[l], nullptr, F, NP(KR, p)[0],
                                          NP(KR, p)[1], d, G + y.down, SJ_F32, d, 0, ws2, wsb));
        else
          GOP("down_dw", sj_gemm_planes(s2, F, d, M, m->ht[l], nullptr, ldt, T(KR, p)[0], T(KR, p)[1], ldt,
                                       G + y.down, SJ_F32, d, 0, ws2, wsb));
        return read(KR, p);
      };
      const bool early_dw = M * F <= (8L << 20);
      if (early_dw) TRY(down_dw());
      // down's dX fused with the SwiGLU derivative
      TRY(reuse(KG, p));
      OP("down_dx_swiglu", sj_down_bwd_swiglu_p(s, NP(KR, p)[0], NP(KR, p)[1], d, M, d, W + y.down, d, F,
                                                (const uint16_t*)m->gg[l], (const uint16_t*)m->uu[l], F,
                                                NP(KG, p)[0], NP(KG, p)[1], 2 * F, TP(KG, p)[0], TP(KG, p)[1], ldt));
      TRY(written(KG, p));
      if (!early_dw) TRY(down_dw());
      OP("gate_up_dx", sj_gemm_planes(s, M, d, 2 * F, NP(KG, p)[0], NP(KG, p)[1], 2 * F, W + y.gu, nullptr, 2 * F,
                                      m->dz, SJ_F32, d, 0, ws, wsb));
      if (m->group_on[1]) TRY(vjp_group(m, l, 1, s2, ws2, wsb, rdw ? NP(KG, p) : T(KG, p)));
      if (rdw && !m->group_all[1])
        GOP("gate_up_dw", sj_gemm_planes_tn(s2, d, 2 * F, M, (const uint16_t*)m->z2[l], nullptr, d, NP(KG, p)[0],
                                           NP(KG, p)[1], 2 * F, G + y.gu, SJ_F32, 2 * F, 0, ws2, wsb));
      else if (!m->group_all[1])
        GOP("gate_up_dw", sj_gemm_planes(s2, d, 2 * F, M, m->z2t[l], nullptr, ldt, T(KG, p)[0], T(KG, p)[1], ldt,
                                        G + y.gu, SJ_F32, 2 * F, 0, ws2, wsb));
      TRY(read(KG, p));
      }
      TRY(reuse(KX, p));
      OP("rmsnorm_bwd", sjh::rmsnorm_bwd_p_deferred(s, (const uint16_t*)m->x1[l], W + y.fn, m->dz, m->dres[cur], m->dx1,
                                                    NP(KX, p)[0], NP(KX, p)[1], TP(KX, p)[0], TP(KX, p)[1], ldt, M, d,
                                                    eps, m->slot_ptr[m->slot_fn[l]]));
      TRY(written(KX, p));
      // x1 = x + attention_output(o)
      if (S.attn_tt)  // dO as hi/lo planes: the attention backward's operands
        OP("attn_out_dx", sj_gemm_planes_split_out(s, M, d, d, NP(KX, p)[0], NP(KX, p)[1], d, W + y.wo, d, m->dop[0],
                                                   m->dop[1], d, nullptr, nullptr, 0, (const uint16_t*)m->o[l], d,
                                                   m->deltat, ldt));
      else
        OP("attn_out_dx", sj_gemm_planes(s, M, d, d, xp[0], xp[1], d, W + y.wo, nullptr, d, m->dO, SJ_F32, d, 0, ws,
                                         wsb));
      if (rdw)
        GOP("attn_out_dw", sj_gemm_planes_tn(s2, d, d, M, (const uint16_t*)m->o[l], nullptr, d, NP(KX, p)[0],
                                            NP(KX, p)[1], d, G + y.wo, SJ_F32, d, 0, ws2, wsb));
      else
        GOP("attn_out_dw", sj_gemm_planes(s2, d, d, M, m->ot[l], nullptr, ldt, T(KX, p)[0], T(KX, p)[1], ldt, G + y.wo,
                                         SJ_F32, d, 0, ws2, wsb));
      TRY(read(KX, p));
      TRY(reuse(KQ, p));
      // with dO as planes, attn_out_dx's epilogue has written Delta
      for (int part = S.attn_tt ? 2 : 1; part <= 4; part <<= 1) {
        if (part == 4 && S.attn_tt && sjh::attention_bwd_grouped(m->B, S.T, S.HQ, S.HK, TP(KQ, p)[0] != nullptr))
          continue;  // the grouped launch wrote the dK | dV planes
        const char* nm = part == 4   ? "attention_bwd_kv_reduce"
                         : S.attn_tt ? (part == 1 ? "attention_bwd_delta" : "attention_bwd_dq_dkv")
                                     : (part == 1 ? "attention_bwd_dq" : "attention_bwd_dkv");
        if (S.attn_tt)
          OP(nm, sjh::attention_bwd_tt_parts(part, s, qkv, NQ, ldt, (const uint16_t*)m->o[l], d, m->lset[l],
                                             m->dop[0], m->dop[1], d, m->deltat, m->B, S.T, S.HQ, S.HK, S.Dh,
                                             S.window, S.rope, NP(KQ, p)[0], NP(KQ, p)[1], NQ, TP(KQ, p)[0],
                                             TP(KQ, p)[1], ldt, ws, wsb, m->attn_cnt));
        else
          OP(nm, sjh::attention_bwd_p_parts(part, s, qkv, NQ, qkv + d, NQ, qkv + d + J, NQ, (const uint16_t*)m->o[l], d,
                                            m->lse[l], m->dO, d, m->delta, m->B, S.T, S.HQ, S.HK, S.Dh, S.rope,
                                            qp[0], qp[1], NQ, T(KQ, p)[0], T(KQ, p)[1], ldt, ws, wsb));
      }
      TRY(written(KQ, p));
      OP("qkv_dx", sj_gemm_planes(s, M, d, NQ, NP(KQ, p)[0], NP(KQ, p)[1], NQ, W + y.qkv, nullptr, NQ, m->dz, SJ_F32, d,
                                  0, ws, wsb));
      if (m->group_on[0]) TRY(vjp_group(m, l, 0, s2, ws2, wsb, rdw ? NP(KQ, p) : T(KQ, p)));
      if (rdw && !m->group_all[0])
        GOP("qkv_dw", sj_gemm_planes_tn(s2, d, NQ, M, (const uint16_t*)m->z[l], nullptr, d, NP(KQ, p)[0], NP(KQ, p)[1],
                                       NQ, G + y.qkv, SJ_F32, NQ, 0, ws2, wsb));
      else if (!m->group_all[0])
        GOP("qkv_dw", sj_gemm_planes(s2, d, NQ, M, m->zt[l], nullptr, ldt, T(KQ, p)[0], T(KQ, p)[1], ldt, G + y.qkv,
                                    SJ_F32, NQ, 0, ws2, wsb));
      TRY(read(KQ, p));
      if (l > S.first) {
        const int pn = (int)((l - 1) & 1);
        TRY(reuse(KR, pn));
        OP("rmsnorm_bwd", sjh::rmsnorm_bwd_p_deferred(s, (const uint16_t*)xin(m, l), W + y.an, m->dz, m->dx1,
                                                      m->dres[cur ^ 1], NP(KR, pn)[0], NP(KR, pn)[1], TP(KR, pn)[0],
                                                      TP(KR, pn)[1], ldt, M, d, eps, m->slot_ptr[m->slot_an[l]]));
        TRY(written(KR, pn));
      } else {  // the stage input's gradient feeds row-layout consumers only: fp32, no planes
        OP("rmsnorm_bwd", sjh::rmsnorm_bwd_p_deferred(s, (const uint16_t*)xin(m, l), W + y.an, m->dz, m->dx1,
                                                      m->dres[cur ^ 1], nullptr, nullptr, nullptr, nullptr, ldt, M, d,
                                                      eps, m->slot_ptr[m->slot_an[l]]));
      }
      cur ^= 1;
    }
    return SJ_OK;
  }
  OP("rmsnorm_bwd", sj_rmsnorm_bwd(s, xtop(m, S), dt, wc(m, S.norm), dt, dzin, nullptr, m->dres[cur], G + S.norm, M, d,
                                   eps, m->ws, m->ws_bytes));
  for (long l = top; l >= S.first; l--) {
    const Layer& y = m->layers[l];
    float* dres = m->dres[cur];
    // x_{l+1} = x1 + down(h): down's dX fused with the SwiGLU derivative
    OP("down_dx_swiglu", sj_down_bwd_swiglu(s, dres, d, M, d, wc(m, y.down), d, F, m->gg[l], m->uu[l], F, dt, m->dgu, 2 * F));
    OP("down_dw", sj_gemm(s, 1, 0, F, d, M, m->hh[l], dt, F, dres, SJ_F32, d, G + y.down, SJ_F32, d, 0, m->ws, m->ws_bytes));
    OP("gate_up_dx", sj_gemm(s, 0, 1, M, d, 2 * F, m->dgu, SJ_F32, 2 * F, wc(m, y.gu), dt, 2 * F, m->dz, SJ_F32, d, 0, m->ws,
                m->ws_bytes));
    OP("gate_up_dw", sj_gemm(s, 1, 0, d, 2 * F, M, m->z2[l], dt, d, m->dgu, SJ_F32, 2 * F, G + y.gu, SJ_F32, 2 * F, 0, m->ws,
                m->ws_bytes));
    OP("rmsnorm_bwd", sj_rmsnorm_bwd(s, m->x1[l], dt, wc(m, y.fn), dt, m->dz, dres, m->dx1, G + y.fn, M, d, eps, m->ws, m->ws_bytes));
    // x1 = x + attention_output(o)
    OP("attn_out_dx", sj_gemm(s, 0, 1, M, d, d, m->dx1, SJ_F32, d, wc(m, y.wo), dt, d, m->dO, SJ_F32, d, 0, m->ws, m->ws_bytes));
    OP("attn_out_dw", sj_gemm(s, 1, 0, d, d, M, m->o[l], dt, d, m->dx1, SJ_F32, d, G + y.wo, SJ_F32, d, 0, m->ws, m->ws_bytes));
    char* qkv = (char*)m->qkv[l];
    OP("attention_bwd", sj_attention_bwd(s, qkv, NQ, qkv + d * m->esz, NQ, qkv + (d + J) * m->esz, NQ, m->o[l], d, m->lse[l], m->dO, d,
                         m->dqkv, NQ, m->dqkv + d, NQ, m->dqkv + d + J, NQ, m->delta, dt, m->B, S.T, S.HQ, S.HK,
                         S.Dh, S.window, S.rope));
    OP("qkv_dx", sj_gemm(s, 0, 1, M, d, NQ, m->dqkv, SJ_F32, NQ, wc(m, y.qkv), dt, NQ, m->dz, SJ_F32, d, 0, m->ws, m->ws_bytes));
    OP("qkv_dw", sj_gemm(s, 1, 0, d, NQ, M, m->z[l], dt, d, m->dqkv, SJ_F32, NQ, G + y.qkv, SJ_F32, NQ, 0, m->ws, m->ws_bytes));
    OP("rmsnorm_bwd", sj_rmsnorm_bwd(s, xin(m, l), dt, wc(m, y.an), dt, m->dz, m->dx1, m->dres[cur ^ 1], G + y.an, M, d, eps, m->ws,
                       m->ws_bytes));
    cur ^= 1;
  }
  return SJ_OK;
}

// Reverse of hierarchy_forward (graph.rs rules for Norm, Matmul, Add,
// PatchBroadcast, PatchPool): m->dz holds d(hn) [Ml][width].  The encoded
// bytes feed both the pool and encoder_to_decoder, global_to_decoder both
// the patch rows and the BOS row: those gradients are summed in fp32
// (graph.rs:503-513).
int hierarchy_backward(sj_model* m, int& cur) {
  hipStream_t s = m->stream;
  const int dt = m->dt;
  const float eps = m->c.norm_epsilon;
  float* G = m->g;
  const Stage &E = m->stages[0], &Gs = m->stages[1], &D = m->stages[2];
  const long B = m->B, P = m->P, de = E.d, dg = Gs.d, dd = D.d, Ml = E.M, Mg = Gs.M;
  void* ws = m->ws;
  const size_t wsb = m->ws_bytes;
  float** hg = m->hg;
  // The glue products' weight gradients (and the BOS row's) whose dY the
  // dX chain never overwrites (hg[0], hg[3], hg[4]) go on the second stream
  // after a written event, beside the chain.  The two that read a stage's
  // d(input) (m->dres[cur], overwritten by the next stage's backward) stay
  // on the chain: a wait for the second stream, which queues the stages' dW
  // products too, cost more than they take (cfg3 3.51 against 3.45 ms).
  const bool two = two_streams(m);
  hipStream_t s2 = two ? m->stream2 : s;
  void* ws2 = two ? m->ws2 : ws;
  auto to_s2 = [&](int k) -> int {  // s2 may read what the chain wrote so far
    if (!two) return SJ_OK;
    SJ_HIP(hipEventRecord(m->ev_glue[k], s));
    SJ_HIP(hipStreamWaitEvent(s2, m->ev_glue[k], 0));
    return SJ_OK;
  };
  // bf16: each glue pair's dY as hi/lo planes (the final norm writes its
  // own; the other three take one split pass), read by the pair's dX
  // product (the weight's bf16 mirror is already the [N][K] operand) and
  // its row-layout dW product, as the stages' own products are
  const bool pl = dt == SJ_BF16 && m->glue_p[0][0] && (de | dg | dd) % 8 == 0 && dg <= 1024;
  auto& gp = m->glue_p;
  const uint16_t* W16 = (const uint16_t*)m->mirror;
  if (pl) {
    OP("rmsnorm_bwd", sj_rmsnorm_bwd_p(s, (const uint16_t*)m->opo, W16 + m->final_norm, m->dz, nullptr, hg[0],
                                       G + m->final_norm, gp[0][0], gp[0][1], nullptr, nullptr, 0, Ml, dg, eps, ws,
                                       wsb));
  } else {
    OP("rmsnorm_bwd", sj_rmsnorm_bwd(s, m->opo, dt, wc(m, m->final_norm), dt, m->dz, nullptr, hg[0],
                                     G + m->final_norm, Ml, dg, eps, ws, wsb));
  }
  TRY(to_s2(0));
  if (pl) {
    OP("output_projection_dw", sj_gemm_planes_tn(s2, dd, dg, Ml, (const uint16_t*)D.out, nullptr, dd, gp[0][0],
                                                 gp[0][1], dg, G + m->h_op, SJ_F32, dg, 0, ws2, wsb));
    OP("output_projection_dx", sj_gemm_planes(s, Ml, dd, dg, gp[0][0], gp[0][1], dg, W16 + m->h_op, nullptr, dg,
                                              hg[1], SJ_F32, dd, 0, ws, wsb));
  } else {
    OP("output_projection_dw", sj_gemm(s2, 1, 0, dd, dg, Ml, D.out, dt, dd, hg[0], SJ_F32, dg, G + m->h_op, SJ_F32,
                                       dg, 0, ws2, wsb));
    OP("output_projection_dx", sj_gemm(s, 0, 1, Ml, dd, dg, hg[0], SJ_F32, dg, wc(m, m->h_op), dt, dg, hg[1], SJ_F32,
                                       dd, 0, ws, wsb));
  }
  TRY(stage_backward(m, 2, hg[1], cur));
  const float* dxd = m->dres[cur];  // d(decoder input) = d(bytes) = d(broadcast output)
  if (pl) {
    OP("glue_split", sjh::split_planes(s, dxd, Ml * dd, gp[1][0], gp[1][1]));
    OP("encoder_to_decoder_dx", sj_gemm_planes(s, Ml, de, dd, gp[1][0], gp[1][1], dd, W16 + m->h_e2d, nullptr, dd,
                                               hg[2], SJ_F32, de, 0, ws, wsb));
  } else {
    OP("encoder_to_decoder_dx", sj_gemm(s, 0, 1, Ml, de, dd, dxd, SJ_F32, dd, wc(m, m->h_e2d), dt, dd, hg[2], SJ_F32,
                                        de, 0, ws, wsb));
  }
  OP("patch_broadcast_bwd", sj_patch_broadcast_bwd(s, dxd, B, E.T, dd, P, hg[3], hg[4]));
  if (pl) {
    OP("encoder_to_decoder_dw", sj_gemm_planes_tn(s, de, dd, Ml, (const uint16_t*)E.out, nullptr, de, gp[1][0],
                                                  gp[1][1], dd, G + m->h_e2d, SJ_F32, dd, 0, ws, wsb));
    OP("glue_split", sjh::split_planes(s, hg[3], Mg * dd, gp[2][0], gp[2][1]));
  } else {
    OP("encoder_to_decoder_dw", sj_gemm(s, 1, 0, de, dd, Ml, E.out, dt, de, dxd, SJ_F32, dd, G + m->h_e2d, SJ_F32, dd,
                                        0, ws, wsb));
  }
  TRY(to_s2(1));
  if (pl)
    OP("global_to_decoder_dw", sj_gemm_planes_tn(s2, dg, dd, Mg, (const uint16_t*)Gs.out, nullptr, dg, gp[2][0],
                                                 gp[2][1], dd, G + m->h_g2d, SJ_F32, dd, 0, ws2, wsb));
  else
    OP("global_to_decoder_dw", sj_gemm(s2, 1, 0, dg, dd, Mg, Gs.out, dt, dg, hg[3], SJ_F32, dd, G + m->h_g2d, SJ_F32,
                                       dd, 0, ws2, wsb));
  OP("bos_to_decoder_dw", sj_gemm(s2, 1, 0, dg, dd, 1, wc(m, m->h_bos), dt, dg, hg[4], SJ_F32, dd, G + m->h_g2d, SJ_F32,
                                  dd, 1, ws2, wsb));
  OP("bos_to_decoder_dx", sj_gemm(s2, 0, 1, 1, dg, dd, hg[4], SJ_F32, dd, wc(m, m->h_g2d), dt, dd, G + m->h_bos, SJ_F32,
                                  dg, 0, ws2, wsb));
  if (pl)
    OP("global_to_decoder_dx", sj_gemm_planes(s, Mg, dg, dd, gp[2][0], gp[2][1], dd, W16 + m->h_g2d, nullptr, dd,
                                              hg[5], SJ_F32, dg, 0, ws, wsb));
  else
    OP("global_to_decoder_dx", sj_gemm(s, 0, 1, Mg, dg, dd, hg[3], SJ_F32, dd, wc(m, m->h_g2d), dt, dd, hg[5], SJ_F32,
                                       dg, 0, ws, wsb));
  TRY(stage_backward(m, 1, hg[5], cur));
  const float* dxg = m->dres[cur];  // d(global input)
  if (pl) {
    OP("glue_split", sjh::split_planes(s, dxg, Mg * dg, gp[3][0], gp[3][1]));
    OP("encoder_to_global_dx", sj_gemm_planes(s, Mg, de, dg, gp[3][0], gp[3][1], dg, W16 + m->h_e2g, nullptr, dg,
                                              hg[6], SJ_F32, de, 0, ws, wsb));
    OP("encoder_to_global_dw", sj_gemm_planes_tn(s, de, dg, Mg, (const uint16_t*)m->pooled, nullptr, de, gp[3][0],
                                                 gp[3][1], dg, G + m->h_e2g, SJ_F32, dg, 0, ws, wsb));
  } else {
    OP("encoder_to_global_dx", sj_gemm(s, 0, 1, Mg, de, dg, dxg, SJ_F32, dg, wc(m, m->h_e2g), dt, dg, hg[6], SJ_F32,
                                       de, 0, ws, wsb));
    OP("encoder_to_global_dw", sj_gemm(s, 1, 0, de, dg, Mg, m->pooled, dt, de, dxg, SJ_F32, dg, G + m->h_e2g, SJ_F32,
                                       dg, 0, ws, wsb));
  }
  OP("patch_pool_bwd", sj_patch_pool_bwd(s, hg[6], B, E.T, de, P, hg[7]));
  OP("encoded_grad_sum", sj_add(s, hg[2], SJ_F32, hg[7], SJ_F32, hg[7], SJ_F32, Ml * de, 1.f));
  return stage_backward(m, 0, hg[7], cur);
}

// Arms the gradient-norm hook for one backward; on the way out records how
// many slots the producers used and whether every gradient went through one.
struct GsqArm {
  sj_model* m;
  explicit GsqArm(sj_model* mm) : m(mm) {
    sjh::GradSq& g = sjh::grad_sq();
    g = sjh::GradSq{};
    if (m->gsq) {
      g.base = m->gsq;
      g.cap = sj_model::GSQ_CAP;
    }
    m->gsq_ok = false;
  }
  ~GsqArm() {
    sjh::GradSq& g = sjh::grad_sq();
    m->gsq_count = g.next;
    m->gsq_ok = g.base && !g.missed && g.next > 0;
    g = sjh::GradSq{};
  }
};

int backward_body(sj_model* m);
int backward(sj_model* m) {
  GsqArm arm(m);
  const int st = backward_body(m);
  if (st) sjh::grad_sq().missed = true;
  return st;
}

int backward_body(sj_model* m) {
  hipStream_t s = m->stream;
  const long M = m->M, d = m->d;
  const int dt = m->dt;
  float* G = m->g;
  if (m->value_n) {
    // affine head backward (bias_reduce, the F32 matmul's dX / dW) and the
    // gather's backward into the full hidden gradient (zero off the SEP rows)
    const long R = m->HR, n = m->HV;
    OP("value_bias_bwd", sj_bias_reduce(s, m->dlogits, m->Vp, R, n, G + m->bias));
    OP("head_dx", sj_gemm(s, 0, 1, R, d, n, m->dlogits, SJ_F32, m->Vp, m->w + m->out, SJ_F32, m->Vp, m->dhsel, SJ_F32,
                          d, 0, m->ws, m->ws_bytes));
    OP("value_scatter", sj_gather_rows_bwd(s, m->dhsel, m->sel, R, d, m->dz, d, M));
  } else if (m->lm_planes) {
    // head: dh = dlogits W_out^T (hi/lo x hi/lo: three products)
    OP("head_dx", sj_gemm_planes(s, M, d, m->Vp, m->dlp[0], m->dlp[1], m->Vp, m->hp[0], m->hp[1], m->Vp, m->dz, SJ_F32,
                                 d, 0, m->ws, m->ws_bytes));
  } else {
    // head: dh = dlogits W_out^T ; dW_out = hn^T dlogits
    OP("head_dx", sj_gemm(s, 0, 1, M, d, m->HV, m->dlogits, SJ_F32, m->Vp, m->w + m->out, SJ_F32, m->Vp, m->dz, SJ_F32, d,
                          0, m->ws, m->ws_bytes));
  }
  const bool two = two_streams(m);
  if (two) {  // fork; every plane buffer starts out free for the dX chain
    SJ_HIP(hipEventRecord(m->ev_fork, s));
    SJ_HIP(hipStreamWaitEvent(m->stream2, m->ev_fork, 0));
    for (int k = 0; k < 4; k++)
      for (int p = 0; p < 2; p++) SJ_HIP(hipEventRecord(m->ev_r[k][p], m->stream2));
  }
  {  // the head's dW reads only the forward's rows and dlogits: second stream
    hipStream_t sw = two ? m->stream2 : s;
    void* wsw = two ? m->ws2 : m->ws;
    if (m->defer_loss) {
      m->defer_loss = false;
      OP("loss_summary", sj_loss_summary(sw, m->loss_rows, M, m->loss, m->obs_slot, 1.0f / (float)m->obs));
    }
    if (m->value_n)
      OP("head_dw", sj_gemm(sw, 1, 0, d, m->HV, m->HR, m->hsel, SJ_F32, d, m->dlogits, SJ_F32, m->Vp, G + m->out, SJ_F32,
                            m->Vp, 0, wsw, m->ws_bytes));
    else if (m->lm_planes)
      GOP("head_dw", sj_gemm_planes_tn(sw, d, m->Vp, M, (const uint16_t*)m->hn, nullptr, d, m->dlp[0], m->dlp[1], m->Vp,
                                      G + m->out, SJ_F32, m->Vp, 0, wsw, m->ws_bytes));
    else
      OP("head_dw", sj_gemm(sw, 1, 0, d, m->HV, M, m->hn, dt, d, m->dlogits, SJ_F32, m->Vp, G + m->out, SJ_F32, m->Vp, 0,
                            wsw, m->ws_bytes));
  }
  int cur = 0;
  if (m->hier)
    TRY(hierarchy_backward(m, cur));
  else
    TRY(stage_backward(m, 0, m->dz, cur));
  if (m->planes) {  // every norm-weight gradient, off the dX chain
    hipStream_t sr = s;
    if (two) {
      SJ_HIP(hipEventRecord(m->ev_norm, s));
      SJ_HIP(hipStreamWaitEvent(m->stream2, m->ev_norm, 0));
      sr = m->stream2;
    }
    GOP("rmsnorm_dw_reduce", sjh::rmsnorm_reduce_multi(sr, m->norm_jobs, m->norm_njobs, m->norm_maxd));
  }
  GOP("embedding_bwd", sj_embedding_bwd(s, m->dres[cur], m->ids, G + m->emb, m->stages[0].M, m->stages[0].d, m->V,
                                       nullptr, 0));
  if (two) {  // the update reads every gradient
    SJ_HIP(hipEventRecord(m->ev_join, m->stream2));
    SJ_HIP(hipStreamWaitEvent(s, m->ev_join, 0));
  }
  return SJ_OK;
}

int fused_adamw(sj_model* m) {
  const long blocks = m->tjob_tiles + m->nfchunks;
  if (blocks == 0) return SJ_OK;
  hipLaunchKernelGGL(k_adamw_tiles, dim3((unsigned)blocks), dim3(256), 0, m->stream, m->w, m->g, m->m, m->v,
                     m->mirror, m->mirror_t, m->n_nodecay, m->step_dev, m->sumsq, m->status, m->tjobs, m->tjob_n,
                     m->tjob_tiles, m->fchunks, TPlanes{m->hp[0], m->hp[1], m->hp[2], m->hp[3]});
  SJ_LAUNCH_CHECK("adamw (fused mirrors)");
  return SJ_OK;
}

int update(sj_model* m) {
  if (m->optimizer == 1) {
    // compact SGD (control_variate.rs:720-775): FP64 norm of the compact
    // gradients when clipping is on, then GradientPlan::update, whose kernel
    // also writes the bf16 mirror
    if (m->sgd.clip_enabled) {
      OP("factored_norm", sj_factored_apply(m->stream, m->fmeta, m->ftiles, 2, 0.f, 0.f, m->fpart));
      OP("norm_sum", sj_sum_f64(m->stream, m->fpart, m->ftiles, m->sumsq));
    }
    OP("sgd_update", sjh::factored_update_staged(m->stream, m->fmeta, m->ftiles, m->sgd_dev,
                                                 m->sgd.clip_enabled ? m->sumsq : nullptr));
    m->mt_stale = m->planes;  // the next forward rebuilds the transposed mirror
    return SJ_OK;
  }
  if (m->gsq_ok)  // the producers' partials, summed in slot order
    OP("grad_norm", sjh::sum_slots(m->stream, m->gsq, m->gsq_count, m->sumsq));
  else
    OP("grad_norm", sj_sum_squares(m->stream, m->g, m->n_params, m->sumsq, m->ws, m->ws_bytes));
  if (m->fused_update) {  // masters, moments and both mirrors in one pass
    OP("adamw", fused_adamw(m));
    m->mt_stale = false;
    return SJ_OK;
  }
  OP("adamw", sj_adamw_multi(m->stream, m->w, m->g, m->m, m->v, m->dt == SJ_BF16 ? m->mirror : nullptr, m->n_params,
                     m->n_nodecay, m->step_dev, m->sumsq, m->status));
  m->mt_stale = m->planes;  // the next forward rebuilds the transposed mirror
  return SJ_OK;
}

int accumulate_observations(sj_model* m, bool deferred);
int whole_step(sj_model* m) {
  if (m->obs <= 1) {
    TRY(forward_deferred(m));
    TRY(backward(m));
    TRY(update(m));
    return SJ_OK;
  }
  // gradient accumulation (train lib.rs:390-415): each observation runs on
  // its own batch, its loss summary lands in its slot with weight
  // 1/accumulation and its backward is seeded with loss_scale/accumulation;
  // Adam::accumulate keeps the first observation's gradients and adds the
  // later ones in order (current + incoming, lib.rs:179-198); the update
  // reads the accumulator.  The producers' FP64 norm slots hold only the last
  // observation's gradients, so the norm sums the accumulated arena.
  float* const g0 = m->g;
  int st = accumulate_observations(m, true);
  if (st) return st;
  m->gsq_ok = false;
  m->g = m->g_acc;
  st = update(m);
  m->g = g0;
  return st;
}

// the observations' forward and backward passes with their gradients summed
// into m->g_acc (deferred: the training step's two-stream form)
int accumulate_observations(sj_model* m, bool deferred) {
  float* const g0 = m->g;
  int32_t* const ids0 = m->ids;
  int32_t* const tg0 = m->targets;
  const size_t gbytes = sizeof(float) * (size_t)m->n_params;
  int st = SJ_OK;
  for (long o = 0; o < m->obs && !st; o++) {
    m->obs_slot = o;
    m->ids = m->obs_ids + o * m->M;
    m->targets = m->obs_targets + o * m->M;
    st = deferred ? forward_deferred(m) : forward(m);
    if (!st) st = backward(m);
    if (st) break;
    if (o == 0) {
      const hipError_t e = hipMemcpyAsync(m->g_acc, g0, gbytes, hipMemcpyDeviceToDevice, m->stream);
      if (e != hipSuccess) st = sjh::hip_check(e, "accumulate");
    } else {
      st = sj_add(m->stream, m->g_acc, SJ_F32, g0, SJ_F32, m->g_acc, SJ_F32, m->n_params, 1.0f);
    }
  }
  m->obs_slot = 0;
  m->ids = ids0;
  m->targets = tg0;
  return st;
}

// Rng::next_u64 (SplitMix64, crates/sejong-core/src/lib.rs:591-609) on the host
uint64_t splitmix64(uint64_t& s) {
  s += 0x9e3779b97f4a7c15ULL;
  uint64_t z = s;
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
  return z ^ (z >> 31);
}

// Compression decisions of the SGD driver, made once: every layer has the
// same groups, shapes and token count, so compressed_parameter_vjp
// (graph.rs:915-1005) decides the same way in every layer and step.  Groups
// by shared input with n >= a rows (graph.rs:551-566): q|k|v on z and
// gate|up on z2 (attention_output, down and the head are groups of one,
// never compressed: uses = 1).
int vjp_decide(sj_model* m) {
  const sj_sgd_config& c = m->sgd;
  const long n = m->M, a = m->d;
  const long total = 7 * m->L + 1;  // Matmul nodes with a parameter operand per step
  long ranks[2] = {0, 0}, blocks = 0, sel = 0;
  if (c.vjp_rank > 0) {
    SJ_REQUIRE(c.vjp_block_rows > 0 && c.vjp_residual_fraction > 0.0 && c.vjp_residual_fraction <= 1.0,
               "parameter VJP requires positive rank/block_rows and residual_fraction in (0,1]");
    SJ_REQUIRE(m->planes, "parameter VJP step driver: bf16 models with 64-wide heads (MFMA layout path)");
    SJ_REQUIRE(c.loss_scale == 1.0f, "parameter VJP step driver: loss_scale must be 1");
    if (n >= a) {
      const long widths[2][3] = {{m->d, m->J, m->J}, {m->F, m->F, 0}};
      const int members[2] = {3, 2};
      for (int kind = 0; kind < 2; kind++) {
        long donor = 0;  // widest member output (the last one on ties)
        for (int i = 0; i < members[kind]; i++)
          if (widths[kind][i] >= donor) donor = widths[kind][i];
        bool act[3] = {true, true, true};
        for (;;) {
          int count = 0, kept = 0;
          for (int i = 0; i < members[kind]; i++) count += act[i];
          if (count == 0) break;
          for (int i = 0; i < members[kind]; i++) {
            if (!act[i]) continue;
            act[i] = sj_pvjp_selects_compression(c.vjp_rank, c.vjp_residual_fraction, c.vjp_block_rows, n, a,
                                                 widths[kind][i], donor, count) == 1;
            kept += act[i];
          }
          if (kept == count) break;
        }
        bool all = true, any = false;
        for (int i = 0; i < members[kind]; i++) {
          m->comp[kind][i] = act[i];
          all = all && act[i];
          any = any || act[i];
        }
        m->group_on[kind] = any;
        m->group_all[kind] = any && all;
        if (any) TRY(sj_pvjp_budget(c.vjp_rank, c.vjp_residual_fraction, c.vjp_block_rows, n, a, donor, &ranks[kind],
                                    &blocks, &sel));
      }
    }
  }
  m->vjp = m->group_on[0] || m->group_on[1];
  long compressed = 0;
  for (int kind = 0; kind < 2; kind++)
    for (int i = 0; i < 3; i++) compressed += m->comp[kind][i];
  m->st_compressed = compressed * m->L;
  m->st_dense = total - m->st_compressed;
  m->st_basis = m->vjp ? 1 : 0;
  m->st_projection = m->L * ((long)m->group_on[0] + (long)m->group_on[1]);
  if (!m->vjp) return SJ_OK;
  if (!m->group_on[1])
    return sjh::fail(SJ_ERR_UNSUPPORTED,
                     "parameter VJP step driver: only q|k|v compresses, and its donor (the pre-RoPE query "
                     "projection) is not retained");
  if (m->group_on[0] && ranks[0] != ranks[1])
    return sjh::fail(SJ_ERR_UNSUPPORTED, "parameter VJP step driver: groups of different rank (%ld, %ld)", ranks[0],
                     ranks[1]);
  SJ_REQUIRE(ranks[1] <= 64, "parameter VJP step driver: rank %ld above 64", ranks[1]);
  m->vjp_R = ranks[1];
  m->vjp_blocks = blocks;
  m->vjp_S = sel;
  m->vjp_k = sel * c.vjp_block_rows;
  m->vjp_inverse = (float)blocks / (float)sel;  // INVERSE, parameter_vjp.rs:282
  m->vjp_eps = sj_pvjp_basis_tolerance(n, m->vjp_R);
  return SJ_OK;
}

// The GradientPlan tables of an SGD model (GradientPlan::new + pack,
// parameter_vjp.rs:329-470), built once: every pointer is fixed.  One table
// updates the masters (and the bf16 mirror); the other materialises G into
// the gradient arena.
int build_plan(sj_model* m) {
  std::vector<sj_factored_param> P, PM;
  std::vector<sj_factored_term> T;
  const long R = m->vjp_R;
  for (const RefTensor& t : m->tensors) {
    const bool c = m->vjp && t.kind >= 0 && m->comp[t.kind][t.member];
    sj_factored_param p = {};
    p.w = m->w + t.int_offset;
    p.dense = c ? nullptr : m->g + t.int_offset;
    p.rows = t.rows;
    p.cols = t.cols;
    p.decay = t.ndim > 1;
    p.ld = t.int_ld;
    p.mirror = m->mirror ? m->mirror + t.int_offset : nullptr;
    if (c) {
      const long width = t.kind == 0 ? m->NQKV : 2 * m->F;
      float* co = m->vjp_coeff[t.kind][t.layer];
      sj_factored_term term = {};
      term.left = m->vjp_left[t.kind][t.layer];
      term.right = co + t.col0;
      term.tail = co + R * width + t.col0;
      term.row_map = m->vjp_map;
      term.rank = R;
      term.scale = 1.f;  // weight 1/accumulation = 1, loss_scale 1 (control_variate.rs:305-309, 619-628)
      term.ld = width;
      p.term_begin = (long)T.size();
      p.term_count = 1;
      T.push_back(term);
    }
    P.push_back(p);
    sj_factored_param q = p;
    q.w = m->g + t.int_offset;
    q.mirror = nullptr;
    PM.push_back(q);
  }
  const size_t bytes = sj_factored_meta_bytes(P.data(), (long)P.size(), (long)T.size());
  std::vector<uint8_t> host(bytes), hostm(bytes);
  long tiles = 0, tiles_m = 0;
  TRY(sj_factored_pack(P.data(), (long)P.size(), T.data(), (long)T.size(), host.data(), bytes, &tiles));
  TRY(sj_factored_pack(PM.data(), (long)PM.size(), T.data(), (long)T.size(), hostm.data(), bytes, &tiles_m));
  TRY(dalloc(m, (void**)&m->fmeta, bytes));
  TRY(dalloc(m, (void**)&m->fmeta_mat, bytes));
  TRY(dalloc(m, (void**)&m->fpart, sizeof(double) * (size_t)tiles));
  SJ_HIP(hipMemcpy(m->fmeta, host.data(), bytes, hipMemcpyHostToDevice));
  SJ_HIP(hipMemcpy(m->fmeta_mat, hostm.data(), bytes, hipMemcpyHostToDevice));
  m->ftiles = tiles;
  return SJ_OK;
}

// Stage the SGD step record (learning rate, clip settings and, with the
// parameter VJP, this step's seed: one next_u64 of the carried parameter
// RNG, control_variate.rs:543,577) from the pinned ring.
int stage_sgd(sj_model* m, float lr) {
  const int slot = (int)(++m->staged % sj_model::RING);
  SJ_HIP(hipEventSynchronize(m->step_done[slot]));
  sj_sgd_step* h = m->sgd_host + slot;
  h->lr = lr;
  h->weight_decay = m->sgd.weight_decay;
  h->clip_norm = m->sgd.clip_norm;
  h->clip_enabled = m->sgd.clip_enabled;
  h->seed = m->vjp ? splitmix64(m->vjp_rng) : 0;
  SJ_HIP(hipMemcpyAsync(m->sgd_dev, h, sizeof(sj_sgd_step), hipMemcpyHostToDevice, m->stream));
  SJ_HIP(hipEventRecord(m->step_done[slot], m->stream));
  return SJ_OK;
}

int create_model(const sj_model_config* cfg, const sj_hierarchy_config* hc, const sj_expert_config* ec,
                 const sj_adam_config* adam, const sj_sgd_config* sgd, long value_n, void* stream, sj_model** out);

}  // namespace

// ================================================================ C ABI

extern "C" int sj_model_create(const sj_model_config* cfg, const sj_adam_config* adam, void* stream,
                               sj_model** out) {
  SJ_REQUIRE(cfg && adam && out, "model: null argument");
  return create_model(cfg, nullptr, nullptr, adam, nullptr, 0, stream, out);
}

extern "C" int sj_model_create_experts(const sj_model_config* cfg, const sj_expert_config* experts,
                                       const sj_adam_config* adam, void* stream, sj_model** out) {
  SJ_REQUIRE(cfg && experts && adam && out, "model: null argument");
  return create_model(cfg, nullptr, experts, adam, nullptr, 0, stream, out);
}

extern "C" int sj_model_create_hierarchy(const sj_model_config* cfg, const sj_hierarchy_config* hierarchy,
                                         const sj_adam_config* adam, void* stream, sj_model** out) {
  SJ_REQUIRE(cfg && hierarchy && adam && out, "model: null argument");
  return create_model(cfg, hierarchy, nullptr, adam, nullptr, 0, stream, out);
}

extern "C" int sj_model_create_sgd(const sj_model_config* cfg, const sj_sgd_config* sgd, void* stream,
                                   sj_model** out) {
  SJ_REQUIRE(cfg && sgd && out, "model: null argument");
  SJ_REQUIRE(sgd->loss_scale > 0.f && isfinite(sgd->loss_scale) && sgd->weight_decay >= 0.f &&
                 (!sgd->clip_enabled || (isfinite(sgd->clip_norm) && sgd->clip_norm > 0.f)),
             "optimizer requires nonnegative weight decay, positive loss scale and positive enabled clip norm");
  return create_model(cfg, nullptr, nullptr, nullptr, sgd, 0, stream, out);
}

extern "C" int sj_model_create_value(const sj_model_config* cfg, long values, const sj_adam_config* adam,
                                     const sj_sgd_config* sgd, void* stream, sj_model** out) {
  SJ_REQUIRE(cfg && out && values > 0 && ((adam != nullptr) != (sgd != nullptr)),
             "native value model: configuration, values > 0 and exactly one optimizer");
  SJ_REQUIRE(cfg->sequence >= 3, "native value model: the sequence holds BOS, the prompt and SEP");
  if (sgd)
    SJ_REQUIRE(sgd->loss_scale > 0.f && isfinite(sgd->loss_scale) && sgd->weight_decay >= 0.f &&
                   (!sgd->clip_enabled || (isfinite(sgd->clip_norm) && sgd->clip_norm > 0.f)),
               "optimizer requires nonnegative weight decay, positive loss scale and positive enabled clip norm");
  return create_model(cfg, nullptr, nullptr, adam, sgd, values, stream, out);
}

namespace {
int create_model(const sj_model_config* cfg, const sj_hierarchy_config* hc, const sj_expert_config* ec,
                 const sj_adam_config* adam, const sj_sgd_config* sgd, long value_n, void* stream, sj_model** out) {
  const sj_model_config& c = *cfg;
  SJ_REQUIRE(c.vocab > 0 && c.width > 0 && c.layers > 0 && c.heads > 0 && c.kv_heads > 0 && c.ffn_width > 0 &&
                 c.sequence > 0 && c.batch > 0,
             "layers, ffn_width and context must be positive");
  SJ_REQUIRE(c.width % c.heads == 0, "width must be divisible by heads");
  SJ_REQUIRE((c.width / c.heads) % 2 == 0, "RoPE requires an even head width");
  SJ_REQUIRE(c.heads % c.kv_heads == 0, "heads must be divisible by kv_heads");
  SJ_REQUIRE(c.precision == SJ_F32 || c.precision == SJ_BF16, "precision must be f32 or bf16");
  if (hc) {
    // HierarchyConfig checks (core lib.rs:81-98, ModelConfig::validate)
    SJ_REQUIRE(hc->patch_size > 0 && hc->encoder_width > 0 && hc->encoder_layers > 0 && hc->encoder_heads > 0 &&
                   hc->encoder_ffn_width > 0 && hc->decoder_width > 0 && hc->decoder_layers > 0 &&
                   hc->decoder_heads > 0 && hc->decoder_ffn_width > 0 && hc->local_window > 0,
               "hierarchy: patch size, widths, layers, heads, FFN widths and local window must be positive");
    SJ_REQUIRE(hc->encoder_width % hc->encoder_heads == 0 && hc->decoder_width % hc->decoder_heads == 0 &&
                   (hc->encoder_width / hc->encoder_heads) % 2 == 0 && (hc->decoder_width / hc->decoder_heads) % 2 == 0,
               "hierarchy: local widths must split into even heads");
    SJ_REQUIRE(!value_n && !sgd, "hierarchy: the hierarchical model trains with AdamW on the byte objective");
  }
  if (ec) {
    SJ_REQUIRE(ec->count > 0 && ec->count <= 32 && ec->top_k > 0 && ec->top_k <= 8 && ec->top_k <= ec->count &&
                   ec->ffn_width > 0 && ec->ffn_width % 8 == 0,
               "experts: 1..32 experts, top_k in 1..min(8, count), ffn_width a positive multiple of 8");
    SJ_REQUIRE(!hc && !value_n && !sgd, "experts: the MoE model trains with AdamW on the byte objective");
    SJ_REQUIRE(c.precision == SJ_BF16 && c.width / c.heads == 64 && c.width % 8 == 0 && c.width <= 1024,
               "experts: the MoE step runs the bf16 MFMA-layout path (64-wide heads, width <= 1024)");
  }
  sj_model* m = new sj_model();
  m->c = c;
  if (adam) m->adam = *adam;
  if (sgd) {
    m->optimizer = 1;
    m->sgd = *sgd;
    m->vjp_rng = sgd->vjp_seed;  // Rng::new(seed), control_variate.rs:73
  }
  m->stream = (hipStream_t)stream;
  if (!m->stream) {
    // graph capture needs a stream other than the null stream
    if (hipStreamCreate(&m->stream) != hipSuccess) {
      delete m;
      return sjh::fail(SJ_ERR_HIP, "model: stream creation");
    }
    m->own_stream = true;
  }
  m->value_n = value_n;
  m->V = value_n ? 259 : c.vocab;  // NativeValue: bytes, pad 256, BOS 257, SEP 258 (native/value.rs:15-16)
  m->HV = value_n ? value_n : m->V;
  m->HR = value_n ? c.batch : c.sequence * c.batch;
  m->Vp = (m->HV + 7) / 8 * 8;
  m->d = c.width;
  m->HQ = c.heads;
  m->HK = c.kv_heads;
  m->Dh = c.width / c.heads;
  m->J = m->Dh * c.kv_heads;
  m->F = ec ? ec->ffn_width : c.ffn_width;
  if (ec) {
    m->E = ec->count;
    m->K = ec->top_k;
    m->cap = sj_route_pack_capacity(c.sequence * c.batch * ec->top_k, ec->count);
  }
  m->T = c.sequence;
  m->B = c.batch;
  m->M = c.sequence * c.batch;
  m->NQKV = m->d + 2 * m->J;
  m->dt = c.precision;
  m->esz = m->dt == SJ_BF16 ? 2 : 4;
  m->ldt = (m->M + 7) / 8 * 8;
  // stages: (prefix, layers, width, heads, kv heads, FFN, sequence, window)
  auto stage = [&](const char* prefix, long layers, long d, long hq, long hk, long F, long T, long window) {
    Stage S;
    S.prefix = prefix;
    S.index = (int)m->stages.size();
    S.first = m->stages.empty() ? 0 : m->stages.back().first + m->stages.back().count;
    S.count = layers;
    S.depth = layers;
    S.d = d; S.HQ = hq; S.HK = hk; S.Dh = d / hq; S.J = S.Dh * hk; S.F = F; S.NQKV = d + 2 * S.J;
    S.T = T; S.M = T * c.batch; S.ldt = (S.M + 7) / 8 * 8;
    S.window = window < T ? window : 0;
    m->stages.push_back(S);
  };
  if (hc) {
    m->hier = true;
    m->P = hc->patch_size;
    const long Tg = (c.sequence + m->P - 1) / m->P;  // sequence.div_ceil(patch)
    stage("encoder", hc->encoder_layers, hc->encoder_width, hc->encoder_heads, hc->encoder_heads,
          hc->encoder_ffn_width, c.sequence, hc->local_window);
    stage("layers", c.layers, c.width, c.heads, c.kv_heads, c.ffn_width, Tg, 0);
    stage("decoder", hc->decoder_layers, hc->decoder_width, hc->decoder_heads, hc->decoder_heads,
          hc->decoder_ffn_width, c.sequence, hc->local_window);
  } else {
    stage("layers", c.layers, c.width, c.heads, c.kv_heads, m->F, c.sequence, 0);
  }
  m->L = 0;
  for (const Stage& S : m->stages) m->L += S.count;
  {
    // MFMA-layout path: bf16, 64-wide heads, 8-aligned widths, d <= 1024
    // (RMSNorm backward row staging), 4-row aligned sequences; windowed
    // stages need the transposed-operand attention (T a multiple of 64)
    const char* env = getenv("SJ_PLANES");
    const char* ev = getenv("SJ_ATTN_TT");
    const bool want = !(env && env[0] == '0'), want_tt = !(ev && ev[0] == '0');
    bool planes = want && m->dt == SJ_BF16;
    for (Stage& S : m->stages) {
      planes = planes && S.Dh == 64 && S.d % 8 == 0 && S.F % 8 == 0 && S.d <= 1024 && (m->B == 1 || S.T % 4 == 0);
      S.attn_tt = want_tt && S.T % 64 == 0;
      if (S.window > 0 && !S.attn_tt) planes = false;
    }
    if (m->hier) {  // the glue's row-layout products need 8-aligned widths; stages share
      planes = planes && m->d % 8 == 0;  // transposed plane buffers, so no padding columns either
      for (const Stage& S : m->stages) planes = planes && S.M % 8 == 0;
    }
    m->planes = planes;
    // the LM head (hn bf16 [M][d] times the fp32 master) on the planes GEMMs
    // with W_out split hi + lo; the hidden width and rows 8-aligned
    m->lm_planes = planes && !m->value_n && m->d % 8 == 0 && m->M % 8 == 0;
    if (m->E && !planes) {
      if (m->own_stream) hipStreamDestroy(m->stream);
      delete m;
      return sjh::fail(SJ_ERR_UNSUPPORTED, "experts: the MoE step needs the MFMA-layout path (SJ_PLANES unset)");
    }
    for (Stage& S : m->stages) S.attn_tt = S.attn_tt && planes;
    m->attn_tt = m->stages[0].attn_tt;
  }
  build_layout(m);
  int st = SJ_OK;
  auto fail_cleanup = [&](int s) {
    sj_model_destroy(m);
    return s;
  };
  if (m->optimizer == 1) {
    st = vjp_decide(m);
    if (st) return fail_cleanup(st);
  }
  // row-layout dW products (no transposed copies of activations or gradient
  // planes; the parameter VJP reads the row layout too): cfg5 34.5 -> 36.9
  // ms/step with the transposed copies written, dense SGD on one box
  m->rowdw = m->planes;
  for (const Stage& S : m->stages) m->rowdw = m->rowdw && S.attn_tt;
#define ALLOC(ptr, bytes)                                    \
  do {                                                       \
    void* _p = nullptr;                                      \
    st = dalloc(m, &_p, (size_t)(bytes));                    \
    if (st) return fail_cleanup(st);                         \
    ptr = (decltype(ptr))_p;                                 \
  } while (0)
  const size_t P = (size_t)m->n_params;
  ALLOC(m->w, P * 4);
  ALLOC(m->g, P * 4);
  if (m->optimizer == 0) {
    ALLOC(m->m, P * 4);
    ALLOC(m->v, P * 4);
  }
  if (m->dt == SJ_BF16) ALLOC(m->mirror, P * 2);
  if (m->planes) {
    ALLOC(m->mirror_t, P * 2);
    // transpose jobs: the four projection matrices of every layer
    std::vector<TJob> jobs;
    long tiles = 0;
    auto job = [&](long off, long rows, long cols, int kind = 0) {
      TJob j{off, rows, cols, tiles, (cols + 63) / 64, kind};
      tiles += ((rows + 63) / 64) * j.tiles_c;
      jobs.push_back(j);
    };
    auto group = [&](int j0, long t0) {
      m->tgroups.push_back(sj_model::TGroup{j0, (int)jobs.size() - j0, t0, tiles - t0});
    };
    if (m->lm_planes) {  // the output head's hi/lo planes from its fp32 master
      for (int k = 0; k < 4; k++) ALLOC(m->hp[k], (size_t)m->d * m->Vp * 2);
      for (int k = 0; k < 2; k++) ALLOC(m->dlp[k], (size_t)m->M * m->Vp * 2);
      job(m->out, m->d, m->Vp, 1);
    }
    group(0, 0);  // group 0: the head (empty without head planes)
    for (long l = 0; l < m->L; l++) {
      const Layer& y = m->layers[l];
      const Stage& S = m->stages[y.stage];
      const int j0 = (int)jobs.size();
      const long t0 = tiles;
      job(y.qkv, S.d, S.NQKV);
      job(y.wo, S.d, S.d);
      for (long e = 0; e < (m->E ? m->E : 1); e++) {
        job(y.gu + e * S.d * 2 * S.F, S.d, 2 * S.F);
        job(y.down + e * S.F * S.d, S.F, S.d);
      }
      group(j0, t0);  // group 1 + l: layer l
    }
    if (m->hier) {  // group 1 + L: the glue projections' [N][K] operands of the forward
      const long de = m->stages[0].d, dg = m->stages[1].d, dd = m->stages[2].d;
      const int j0 = (int)jobs.size();
      const long t0 = tiles;
      job(m->h_e2g, de, dg);
      job(m->h_e2d, de, dd);
      job(m->h_g2d, dg, dd);
      job(m->h_op, dd, dg);
      m->tr_glue = m->tgroups.size();
      group(j0, t0);
    }
    m->tjob_n = (int)jobs.size();
    m->tjob_tiles = tiles;
    ALLOC(m->tjobs, sizeof(TJob) * jobs.size());
    if (hipMemcpy(m->tjobs, jobs.data(), sizeof(TJob) * jobs.size(), hipMemcpyHostToDevice) != hipSuccess)
      return fail_cleanup(sjh::fail(SJ_ERR_HIP, "model: transpose job table"));
    // the fused update: the rest of the arena (norms, embedding, routers,
    // glue, padding) in chunks of at most 1024 parameters (a quad per thread)
    static const int fused_env = [] {
      const char* e = getenv("SJ_FUSED_ADAMW");  // 0: AdamW, then the transpose pass (A/B)
      return e ? atoi(e) : 1;
    }();
    if (m->optimizer == 0 && m->dt == SJ_BF16 && fused_env) {
      std::vector<std::pair<long, long>> spans;
      for (const TJob& j : jobs) spans.push_back({j.off, j.off + j.rows * j.cols});
      std::sort(spans.begin(), spans.end());
      std::vector<FlatChunk> ch;
      long at = 0;
      auto flat = [&](long a, long e) {
        for (long x = a; x < e; x += 1024) ch.push_back(FlatChunk{x, x + 1024 < e ? x + 1024 : e});
      };
      for (const auto& sp : spans) {
        if (sp.first < at) return fail_cleanup(sjh::fail(SJ_ERR_INVALID, "model: overlapping transpose jobs"));
        flat(at, sp.first);
        at = sp.second;
      }
      flat(at, (long)P);
      m->nfchunks = (long)ch.size();
      if (!ch.empty()) {
        ALLOC(m->fchunks, sizeof(FlatChunk) * ch.size());
        if (hipMemcpy(m->fchunks, ch.data(), sizeof(FlatChunk) * ch.size(), hipMemcpyHostToDevice) != hipSuccess)
          return fail_cleanup(sjh::fail(SJ_ERR_HIP, "model: flat update chunks"));
      }
      m->fused_update = true;
    }
  }
  const size_t es = m->esz;
  // largest per-stage extents (shared scratch) and the head's
  size_t mxMd = (size_t)m->M * (size_t)m->d, mxMF = 0, mxMNQ = 0, mxMHQ = 0, mxTd = 0, mxT = 0, mxLd = 0;
  size_t mxLF = 0, mxLNQ = 0, mxLHQ = 0;
  for (const Stage& S : m->stages) {
    auto mx = [](size_t& a, size_t b) { a = b > a ? b : a; };
    mx(mxMd, (size_t)(S.M * S.d)); mx(mxMF, (size_t)(S.M * S.F)); mx(mxMNQ, (size_t)(S.M * S.NQKV));
    mx(mxMHQ, (size_t)(S.M * S.HQ)); mx(mxTd, (size_t)(S.T * S.Dh)); mx(mxT, (size_t)S.T);
    mx(mxLd, (size_t)(S.ldt * S.d)); mx(mxLF, (size_t)(S.ldt * S.F)); mx(mxLNQ, (size_t)(S.ldt * S.NQKV));
    mx(mxLHQ, (size_t)(S.ldt * S.HQ));
  }
  m->x.resize(m->L + m->stages.size());
  for (const Stage& S : m->stages)
    for (long i = 0; i <= S.count; i++) ALLOC(m->x[S.first + S.index + i], (size_t)(S.M * S.d) * es);
  m->z.resize(m->L); m->qkv.resize(m->L); m->o.resize(m->L); m->x1.resize(m->L); m->z2.resize(m->L);
  m->gg.resize(m->L); m->uu.resize(m->L); m->hh.resize(m->L); m->lse.resize(m->L);
  for (long l = 0; l < m->L; l++) {
    const Stage& S = m->stages[m->layers[l].stage];
    const size_t M = (size_t)S.M, d = (size_t)S.d, F = (size_t)S.F;
    ALLOC(m->z[l], M * d * es);
    ALLOC(m->qkv[l], M * (size_t)S.NQKV * es);
    ALLOC(m->o[l], M * d * es);
    ALLOC(m->lse[l], M * (size_t)S.HQ * 4);
    ALLOC(m->x1[l], M * d * es);
    ALLOC(m->z2[l], M * d * es);
    const size_t FR = m->E ? (size_t)m->cap : M;  // rows of g, u, h: the packed expert rows under MoE
    ALLOC(m->gg[l], FR * F * es);
    ALLOC(m->uu[l], FR * F * es);
    ALLOC(m->hh[l], FR * F * es);
  }
  if (m->E) {
    const size_t M = (size_t)m->M, d = (size_t)m->d, F = (size_t)m->F, E = (size_t)m->E, S = M * (size_t)m->K;
    const size_t cap = (size_t)m->cap;
    for (auto* v : {&m->mlog, &m->mzp, &m->mzpt, &m->myp}) v->assign(m->L, nullptr);
    for (auto* v : {&m->mids, &m->mcnt, &m->moff, &m->mps, &m->mpp}) v->assign(m->L, nullptr);
    for (auto* v : {&m->mwts, &m->mdwts, &m->mdlog}) v->assign(m->L, nullptr);
    for (int i = 0; i < 4; i++) { m->mdx[i].assign(m->L, nullptr); m->mdg[i].assign(m->L, nullptr); }
    if (E == 8) ALLOC(m->mhist, (size_t)sjh::router_hist_blocks((long)M) * E * 4);
    for (long l = 0; l < m->L; l++) {
      ALLOC(m->mlog[l], M * E * 2);
      ALLOC(m->mids[l], S * 4);
      ALLOC(m->mwts[l], S * 4);
      ALLOC(m->mcnt[l], E * 4);
      ALLOC(m->moff[l], (E + 1) * 4);
      ALLOC(m->mps[l], cap * 4);
      ALLOC(m->mpp[l], S * 4);
      ALLOC(m->mzp[l], cap * d * 2);
      ALLOC(m->mzpt[l], d * cap * 2);
      ALLOC(m->myp[l], cap * d * 2);
      ALLOC(m->mdwts[l], S * 4);
      ALLOC(m->mdlog[l], M * E * 4);
      for (int i = 0; i < 4; i++) {
        ALLOC(m->mdx[i][l], cap * d * 2);
        ALLOC(m->mdg[i][l], cap * 2 * F * 2);
      }
    }
    ALLOC(m->mdzp, cap * d * 4);
  }
  if (m->planes) {
    // transposed copies of the retained activations: only the transposed-
    // operand dW products read them (row-layout dW reads the rows)
    m->zt.assign(m->L, nullptr); m->ot.assign(m->L, nullptr); m->z2t.assign(m->L, nullptr);
    m->ht.assign(m->L, nullptr);
    for (long l = 0; l < m->L && !m->rowdw; l++) {
      const Stage& S = m->stages[m->layers[l].stage];
      const size_t MT = (size_t)S.ldt, d = (size_t)S.d;
      ALLOC(m->zt[l], d * MT * 2);
      ALLOC(m->ot[l], d * MT * 2);
      ALLOC(m->z2t[l], d * MT * 2);
      ALLOC(m->ht[l], (size_t)S.F * (m->E ? (size_t)m->cap : MT) * 2);
    }
    bool any_tt = false;
    for (const Stage& S : m->stages) any_tt = any_tt || S.attn_tt;
    if (any_tt) {
      m->lset.assign(m->L, nullptr);
      for (long l = 0; l < m->L; l++) {
        const Stage& S = m->stages[m->layers[l].stage];
        if (!S.attn_tt) continue;
        ALLOC(m->lset[l], (size_t)S.HQ * (size_t)S.ldt * 4);
      }
      for (int i = 0; i < 2; i++) ALLOC(m->dop[i], mxMd * 2);
      ALLOC(m->deltat, mxLHQ * 4);
    }
    for (int i = 0; i < 4; i++) {
      ALLOC(m->rp[i], (i < 2 ? mxMd : mxLd) * 2);
      ALLOC(m->xp[i], (i < 2 ? mxMd : mxLd) * 2);
      ALLOC(m->qp[i], (i < 2 ? mxMNQ : mxLNQ) * 2);
      ALLOC(m->gp[i], (i < 2 ? mxMF : mxLF) * 2 * 2);
    }
    // transposed planes by layer parity: parity 0 is the set above
    uint16_t** base[4] = {m->rp, m->gp, m->xp, m->qp};
    const size_t sizes[4] = {mxLd, 2 * mxLF, mxLd, mxLNQ};
    for (int k = 0; k < 4; k++)
      for (int i = 0; i < 2; i++) {
        m->pt[k][0][i] = base[k][2 + i];
        ALLOC(m->pt[k][1][i], sizes[k] * 2);
      }
    // norm-weight partial slots: the closing norm of every stage, and per
    // layer the ffn norm and the attention norm
    std::vector<sj::RmsReduceJob> jobs;
    std::vector<size_t> offs;
    size_t total = 0;
    auto slot = [&](const Stage& S, long woff) -> long {
      const size_t n = sj_rmsnorm_bwd_p_workspace_bytes(S.M, S.d) / sizeof(float);
      jobs.push_back(sj::RmsReduceJob{nullptr, m->g + woff, (long)(n / (size_t)S.d), S.d});
      offs.push_back(total);
      total += (n + 63) / 64 * 64;
      m->norm_maxd = S.d > m->norm_maxd ? S.d : m->norm_maxd;
      return (long)jobs.size() - 1;
    };
    m->slot_fn.assign(m->L, -1);
    m->slot_an.assign(m->L, -1);
    for (const Stage& S : m->stages) {
      m->slot_close.push_back(slot(S, S.norm));
      for (long l = S.first; l < S.first + S.count; l++) {
        m->slot_fn[l] = slot(S, m->layers[l].fn);
        m->slot_an[l] = slot(S, m->layers[l].an);
      }
    }
    ALLOC(m->norm_part, total * sizeof(float));
    for (size_t i = 0; i < jobs.size(); i++) {
      jobs[i].partial = m->norm_part + offs[i];
      m->slot_ptr.push_back(m->norm_part + offs[i]);
    }
    m->norm_njobs = (long)jobs.size();
    ALLOC(m->norm_jobs, sizeof(sj::RmsReduceJob) * jobs.size());
    if (hipMemcpy(m->norm_jobs, jobs.data(), sizeof(sj::RmsReduceJob) * jobs.size(), hipMemcpyHostToDevice) !=
        hipSuccess)
      return fail_cleanup(sjh::fail(SJ_ERR_HIP, "model: norm reduce table"));
  }
  ALLOC(m->hn, (size_t)m->M * (size_t)m->d * es);
  if (m->hier) {
    Stage &E = m->stages[0], &Gs = m->stages[1], &D = m->stages[2];
    for (Stage* S : {&E, &Gs, &D}) ALLOC(S->out, (size_t)(S->M * S->d) * es);
    ALLOC(m->pooled, (size_t)(Gs.M * E.d) * es);
    ALLOC(m->gd, (size_t)(Gs.M * D.d) * es);
    ALLOC(m->bosd, (size_t)D.d * es + 256);
    ALLOC(m->zb, (size_t)(E.M * D.d) * es);
    ALLOC(m->bytes, (size_t)(E.M * D.d) * es);
    ALLOC(m->opo, (size_t)(E.M * Gs.d) * es);
    const size_t hsz[8] = {(size_t)(E.M * Gs.d), (size_t)(E.M * D.d), (size_t)(E.M * E.d), (size_t)(Gs.M * D.d),
                           (size_t)D.d, (size_t)(Gs.M * Gs.d), (size_t)(Gs.M * E.d), (size_t)(E.M * E.d)};
    for (int i = 0; i < 8; i++) ALLOC(m->hg[i], hsz[i] * 4);
    if (m->dt == SJ_BF16) {
      const size_t psz[4] = {(size_t)(E.M * Gs.d), (size_t)(E.M * D.d), (size_t)(Gs.M * D.d), (size_t)(Gs.M * Gs.d)};
      for (int i = 0; i < 4; i++)
        for (int h = 0; h < 2; h++) ALLOC(m->glue_p[i][h], psz[i] * 2);
    }
  } else {
    m->stages[0].out = m->hn;
  }
  ALLOC(m->logits, (size_t)m->HR * (size_t)m->Vp * 4);
  ALLOC(m->dlogits, (size_t)m->HR * (size_t)m->Vp * 4);
  if (m->value_n) {
    ALLOC(m->sel, sizeof(int32_t) * (size_t)m->HR);
    ALLOC(m->labels, sizeof(int32_t) * (size_t)m->HR);
    ALLOC(m->hsel, sizeof(float) * (size_t)m->HR * (size_t)m->d);
    ALLOC(m->dhsel, sizeof(float) * (size_t)m->HR * (size_t)m->d);
  }
  ALLOC(m->loss_rows, (size_t)m->M * 4);
  ALLOC(m->dres[0], mxMd * 4);
  ALLOC(m->dres[1], mxMd * 4);
  ALLOC(m->dx1, mxMd * 4);
  ALLOC(m->dO, mxMd * 4);
  ALLOC(m->dz, mxMd * 4);
  ALLOC(m->dqkv, mxMNQ * 4);
  ALLOC(m->dgu, mxMF * 2 * 4);
  ALLOC(m->delta, mxMHQ * 4);
  for (Stage& S : m->stages) ALLOC(S.rope, (size_t)(S.T * S.Dh) * 4);
  m->rope = m->stages[0].rope;
  ALLOC(m->ids, (size_t)m->M * 4);
  ALLOC(m->targets, (size_t)m->M * 4);
  ALLOC(m->loss, sizeof(double) * sj_model::OBS_MAX);
  ALLOC(m->sumsq, 64);
  if (gsq_eligible(m)) ALLOC(m->gsq, sizeof(double) * (size_t)sj_model::GSQ_CAP);
  ALLOC(m->status, 64);
  ALLOC(m->step_dev, sizeof(sj_adam_step));
  if (m->optimizer == 1) ALLOC(m->sgd_dev, sizeof(sj_sgd_step));
  const size_t M = (size_t)m->M, d = (size_t)m->d, F = (size_t)m->F;
  if (m->vjp) {
    const size_t R = (size_t)m->vjp_R, k = (size_t)m->vjp_k, rows = R + k, MT = (size_t)m->ldt;
    ALLOC(m->vjp_scratch, sizeof(int32_t) * (F + (size_t)m->vjp_blocks));
    ALLOC(m->vjp_cols, sizeof(int32_t) * R);
    ALLOC(m->vjp_rows, sizeof(int32_t) * (k > 0 ? k : 1));
    ALLOC(m->vjp_map, sizeof(int32_t) * d);
    ALLOC(m->vjp_q, sizeof(float) * M * R);
    ALLOC(m->vjp_eh, 2 * rows * MT);
    ALLOC(m->vjp_el, 2 * rows * MT);
    for (int kind = 0; kind < 2; kind++) {
      const size_t width = kind == 0 ? (size_t)m->NQKV : 2 * F;
      m->vjp_left[kind].assign(m->L, nullptr);
      m->vjp_coeff[kind].assign(m->L, nullptr);
      for (long l = 0; l < m->L && m->group_on[kind]; l++) {
        ALLOC(m->vjp_left[kind][l], sizeof(float) * d * R);
        ALLOC(m->vjp_coeff[kind][l], sizeof(float) * rows * width);
      }
    }
  }
  // workspace: max over the step's calls
  size_t ws = 0;
  auto upd = [&](size_t b) { ws = b > ws ? b : ws; };
  upd(sj_rmsnorm_bwd_workspace_bytes(m->M, m->d));
  upd(sj_sum_squares_workspace_bytes(m->n_params));
  upd(sj_gemm_workspace_bytes(m->HR, m->d, m->HV));
  upd(sj_gemm_workspace_bytes(m->d, m->HV, m->HR));
  upd(sj_gemm_workspace_bytes(m->HR, m->HV, m->d));
  if (m->lm_planes) upd(sj_gemm_planes_workspace_bytes(m->d, m->Vp, m->HR));  // head dW
  for (const Stage& S : m->stages) {
    const long Mi = S.M;
    upd(sj_rmsnorm_bwd_workspace_bytes(Mi, S.d));
    upd(sj_gemm_workspace_bytes(S.F, S.d, Mi));
    upd(sj_gemm_workspace_bytes(S.d, 2 * S.F, Mi));
    upd(sj_gemm_workspace_bytes(S.d, S.d, Mi));
    upd(sj_gemm_workspace_bytes(S.d, S.NQKV, Mi));
    upd(sj_gemm_workspace_bytes(Mi, S.d, 2 * S.F));
    upd(sj_gemm_workspace_bytes(Mi, S.d, S.NQKV));
    if (m->planes) {
      upd(sj_rmsnorm_bwd_p_workspace_bytes(Mi, S.d));
      upd(sj_attention_bwd_p_workspace_bytes(m->B, S.T, S.HQ, S.HK, S.Dh));
      upd(sj_attention_bwd_tt_workspace_bytes(m->B, S.T, S.HQ, S.HK, S.Dh));
      upd(sj_gemm_planes_workspace_bytes(S.F, S.d, Mi));
      upd(sj_gemm_planes_workspace_bytes(S.d, 2 * S.F, Mi));
      upd(sj_gemm_planes_workspace_bytes(S.d, S.d, Mi));
      upd(sj_gemm_planes_workspace_bytes(S.d, S.NQKV, Mi));
      upd(sj_gemm_planes_workspace_bytes(Mi, S.d, 2 * S.F));
      upd(sj_gemm_planes_workspace_bytes(Mi, S.d, S.d));
      upd(sj_gemm_planes_workspace_bytes(Mi, S.d, S.NQKV));
    }
  }
  if (m->E) upd(sj_gemm_workspace_bytes(m->d, m->E, m->M));
  if (m->hier) {
    const Stage &E = m->stages[0], &Gs = m->stages[1], &D = m->stages[2];
    const long de = E.d, dg = Gs.d, dd = D.d, Ml = E.M, Mg = Gs.M;
    const long shapes[][3] = {{Mg, dg, de}, {Mg, dd, dg}, {1, dd, dg}, {Ml, dd, de}, {Ml, dg, dd},
                              {Ml, dd, dg}, {dd, dg, Ml}, {Ml, de, dd}, {de, dd, Ml}, {dg, dd, Mg},
                              {dg, dd, 1},  {1, dg, dd},  {Mg, dg, dd}, {Mg, de, dg}, {de, dg, Mg}};
    for (const auto& sh : shapes) upd(sj_gemm_workspace_bytes(sh[0], sh[1], sh[2]));
    if (m->dt == SJ_BF16) {  // the glue products on planes and the final norm's planes
      const long pshapes[][3] = {{dd, dg, Ml}, {Ml, dd, dg}, {Ml, de, dd}, {de, dd, Ml}, {dg, dd, Mg},
                                 {Mg, dg, dd}, {Mg, de, dg}, {de, dg, Mg}, {Ml, dd, de}, {Mg, dg, de},
                                 {Mg, dd, dg}, {Ml, dg, dd}};
      for (const auto& sh : pshapes) upd(sj_gemm_planes_workspace_bytes(sh[0], sh[1], sh[2]));
      upd(sj_rmsnorm_bwd_p_workspace_bytes(Ml, dg));
    }
  }
  if (m->vjp) {
    const long rows = m->vjp_R + m->vjp_k;
    upd(sj_pvjp_basis_workspace_bytes(m->M, m->vjp_R));
    upd(sj_pvjp_prepare_workspace_bytes(m->d, m->M, m->vjp_R));
    upd(sj_pvjp_vjp_workspace_bytes(rows, m->NQKV, m->M));
    upd(sj_pvjp_vjp_workspace_bytes(rows, 2 * m->F, m->M));
  }
  m->ws_bytes = ws;
  ALLOC(m->ws, ws);
  if (m->planes) ALLOC(m->ws2, ws);
  size_t cnt_bytes = 0;
  for (const Stage& S : m->stages) {
    const size_t c = sj_attention_bwd_tt_counter_bytes(m->B, S.HK);
    cnt_bytes = c > cnt_bytes ? c : cnt_bytes;
  }
  if (m->planes) ALLOC(m->attn_cnt, cnt_bytes);
#undef ALLOC
  if (hipHostMalloc((void**)&m->step_host, sizeof(sj_adam_step) * sj_model::RING, 0) != hipSuccess)
    return fail_cleanup(sjh::fail(SJ_ERR_CAPACITY, "model: pinned step buffer"));
  if (m->optimizer == 1 &&
      hipHostMalloc((void**)&m->sgd_host, sizeof(sj_sgd_step) * sj_model::RING, 0) != hipSuccess)
    return fail_cleanup(sjh::fail(SJ_ERR_CAPACITY, "model: pinned step buffer"));
  for (int i = 0; i < sj_model::RING; i++)
    if (hipEventCreateWithFlags(&m->step_done[i], hipEventDisableTiming) != hipSuccess)
      return fail_cleanup(sjh::fail(SJ_ERR_HIP, "model: event creation"));
  // zero state, rope table
  hipStream_t s = m->stream;
  hipError_t e = hipSuccess;
  for (void* p : {(void*)m->w, (void*)m->g, (void*)m->m, (void*)m->v})
    if (e == hipSuccess && p) e = hipMemsetAsync(p, 0, P * 4, s);
  if (e == hipSuccess && m->mirror) e = hipMemsetAsync(m->mirror, 0, P * 2, s);
  if (e == hipSuccess && m->mirror_t) e = hipMemsetAsync(m->mirror_t, 0, P * 2, s);
  if (e == hipSuccess && m->attn_cnt) e = hipMemsetAsync(m->attn_cnt, 0, cnt_bytes, s);
  // padding columns [M, ldt) of the transposed activations stay zero
  for (long l = 0; l < m->L && m->planes && !m->rowdw; l++) {
    const Stage& S = m->stages[m->layers[l].stage];
    const size_t MT = (size_t)S.ldt;
    for (uint16_t* q : {m->zt[l], m->ot[l], m->z2t[l]})
      if (e == hipSuccess) e = hipMemsetAsync(q, 0, (size_t)S.d * MT * 2, s);
    if (e == hipSuccess) e = hipMemsetAsync(m->ht[l], 0, (size_t)S.F * (m->E ? (size_t)m->cap : MT) * 2, s);
  }
  {
    const size_t sizes[4] = {mxLd, 2 * mxLF, mxLd, mxLNQ};
    for (int k = 0; k < 4 && m->planes; k++)
      for (int i = 0; i < 2; i++)
        if (e == hipSuccess) e = hipMemsetAsync(m->pt[k][1][i], 0, sizes[k] * 2, s);
  }
  if (e == hipSuccess && m->planes) {
    e = hipStreamCreate(&m->stream2);
    for (int k = 0; k < 4 && e == hipSuccess; k++)
      for (int p = 0; p < 2 && e == hipSuccess; p++) {
        e = hipEventCreateWithFlags(&m->ev_w[k][p], hipEventDisableTiming);
        if (e == hipSuccess) e = hipEventCreateWithFlags(&m->ev_r[k][p], hipEventDisableTiming);
      }
    if (e == hipSuccess) e = hipEventCreateWithFlags(&m->ev_fork, hipEventDisableTiming);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&m->ev_join, hipEventDisableTiming);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&m->ev_norm, hipEventDisableTiming);
    for (int k = 0; k < 4 && e == hipSuccess && m->hier; k++) e = hipEventCreateWithFlags(&m->ev_glue[k], hipEventDisableTiming);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&m->ev_tr_fork, hipEventDisableTiming);
    m->ev_tr.assign(m->tgroups.size(), nullptr);
    for (size_t g = 0; g < m->ev_tr.size() && e == hipSuccess; g++)
      e = hipEventCreateWithFlags(&m->ev_tr[g], hipEventDisableTiming);
    for (int k = 0; k < 2 && m->E; k++) {
      m->ev_moe[k].assign(m->L, nullptr);
      for (long l = 0; l < m->L && e == hipSuccess; l++)
        e = hipEventCreateWithFlags(&m->ev_moe[k][l], hipEventDisableTiming);
    }
  }
  for (int i = 2; i < 4 && m->planes; i++) {
    if (e == hipSuccess) e = hipMemsetAsync(m->rp[i], 0, mxLd * 2, s);
    if (e == hipSuccess) e = hipMemsetAsync(m->xp[i], 0, mxLd * 2, s);
    if (e == hipSuccess) e = hipMemsetAsync(m->qp[i], 0, mxLNQ * 2, s);
    if (e == hipSuccess) e = hipMemsetAsync(m->gp[i], 0, mxLF * 2 * 2, s);
  }
  if (e == hipSuccess && m->planes) {
    int ps = sjh::norm_prepare();
    if (!ps) ps = sjh::gemm_fast_prepare();
    if (!ps) ps = sjh::attention_prepare();
    if (!ps) ps = sjh::attention_t_prepare();
    if (ps) return fail_cleanup(ps);
  }
  if (e == hipSuccess) e = hipMemsetAsync(m->status, 0, 64, s);
  if (e == hipSuccess) e = hipMemsetAsync(m->loss, 0, sizeof(double) * sj_model::OBS_MAX, s);
  if (e == hipSuccess) e = hipMemsetAsync(m->sumsq, 0, 64, s);
  if (e != hipSuccess) return fail_cleanup(sjh::hip_check(e, "model: clear arenas"));
  for (const Stage& S : m->stages) {
    st = sj_rope_table(s, S.rope, S.T, S.Dh, c.rope_theta);
    if (st) return fail_cleanup(st);
  }
  (void)mxTd;
  (void)mxT;
  if (m->optimizer == 1) {
    e = hipStreamSynchronize(s);
    if (e != hipSuccess) return fail_cleanup(sjh::hip_check(e, "model: init sync"));
    st = build_plan(m);
    if (st) return fail_cleanup(st);
  }
  e = hipStreamSynchronize(s);
  if (e != hipSuccess) return fail_cleanup(sjh::hip_check(e, "model: init sync"));
  *out = m;
  return SJ_OK;
}
}  // namespace

extern "C" int sj_model_destroy(sj_model* m) {
  if (!m) return SJ_OK;
  if (m->stream) hipStreamSynchronize(m->stream);
  if (m->exec) hipGraphExecDestroy(m->exec);
  if (m->graph) hipGraphDestroy(m->graph);
  for (void* p : m->allocations) hipFree(p);
  for (hipEvent_t e : m->prof_events) hipEventDestroy(e);
  if (m->step_host) hipHostFree(m->step_host);
  if (m->sgd_host) hipHostFree(m->sgd_host);
  for (int i = 0; i < sj_model::RING; i++)
    if (m->step_done[i]) hipEventDestroy(m->step_done[i]);
  for (int k = 0; k < 4; k++)
    for (int p = 0; p < 2; p++) {
      if (m->ev_w[k][p]) hipEventDestroy(m->ev_w[k][p]);
      if (m->ev_r[k][p]) hipEventDestroy(m->ev_r[k][p]);
    }
  if (m->ev_fork) hipEventDestroy(m->ev_fork);
  if (m->ev_join) hipEventDestroy(m->ev_join);
  if (m->ev_norm) hipEventDestroy(m->ev_norm);
  for (hipEvent_t ev : m->ev_glue)
    if (ev) hipEventDestroy(ev);
  if (m->ev_tr_fork) hipEventDestroy(m->ev_tr_fork);
  for (hipEvent_t ev : m->ev_tr)
    if (ev) hipEventDestroy(ev);
  for (int k = 0; k < 2; k++)
    for (hipEvent_t ev : m->ev_moe[k])
      if (ev) hipEventDestroy(ev);
  if (m->stream2) {
    hipStreamSynchronize(m->stream2);
    hipStreamDestroy(m->stream2);
  }
  if (m->own_stream) hipStreamDestroy(m->stream);
  delete m;
  return SJ_OK;
}

extern "C" long sj_model_param_tensors(const sj_model* m) { return m ? (long)m->tensors.size() : 0; }
extern "C" long sj_model_param_count(const sj_model* m) { return m ? m->ref_count : 0; }

extern "C" int sj_model_param_info(const sj_model* m, long i, const char** name, long* rows, long* cols,
                                   long* offset) {
  SJ_REQUIRE(m && i >= 0 && i < (long)m->tensors.size(), "param_info: index %ld", i);
  const RefTensor& t = m->tensors[i];
  if (name) *name = t.name.c_str();
  if (rows) *rows = t.rows;
  if (cols) *cols = t.cols;
  if (offset) *offset = t.ref_offset;
  return SJ_OK;
}

static int copy_arena_in(sj_model* m, const float* host, float* dev) {
  std::vector<float> in((size_t)m->n_params, 0.f);
  ref_to_internal(m, host, in.data());
  SJ_HIP(hipMemcpyAsync(dev, in.data(), sizeof(float) * in.size(), hipMemcpyHostToDevice, m->stream));
  SJ_HIP(hipStreamSynchronize(m->stream));
  return SJ_OK;
}
static int copy_arena_out(sj_model* m, const float* dev, float* host) {
  std::vector<float> in((size_t)m->n_params);
  SJ_HIP(hipStreamSynchronize(m->stream));
  SJ_HIP(hipMemcpy(in.data(), dev, sizeof(float) * in.size(), hipMemcpyDeviceToHost));
  internal_to_ref(m, in.data(), host);
  return SJ_OK;
}

extern "C" int sj_model_set_params(sj_model* m, const float* host) {
  SJ_REQUIRE(m && host, "set_params: null");
  TRY(copy_arena_in(m, host, m->w));
  TRY(refresh_mirror(m));
  SJ_HIP(hipStreamSynchronize(m->stream));
  return SJ_OK;
}
extern "C" int sj_model_get_params(sj_model* m, float* host) {
  SJ_REQUIRE(m && host, "get_params: null");
  return copy_arena_out(m, m->w, host);
}
extern "C" int sj_model_get_grads(sj_model* m, float* host) {
  SJ_REQUIRE(m && host, "get_grads: null");
  return copy_arena_out(m, m->g, host);
}
extern "C" int sj_model_get_adam_state(sj_model* m, float* mh, float* vh, long* step) {
  SJ_REQUIRE(m && m->optimizer == 0, "get_adam_state: AdamW model required");
  if (mh) TRY(copy_arena_out(m, m->m, mh));
  if (vh) TRY(copy_arena_out(m, m->v, vh));
  if (step) *step = m->step;
  return SJ_OK;
}
extern "C" int sj_model_set_adam_state(sj_model* m, const float* mh, const float* vh, long step) {
  SJ_REQUIRE(m && m->optimizer == 0 && mh && vh && step >= 0, "set_adam_state: arguments (AdamW model)");
  TRY(copy_arena_in(m, mh, m->m));
  TRY(copy_arena_in(m, vh, m->v));
  m->step = step;
  return SJ_OK;
}

// a change of the step's structure (the observation count) needs a new capture
static void drop_graph(sj_model* m) {
  if (m->exec) hipGraphExecDestroy(m->exec);
  if (m->graph) hipGraphDestroy(m->graph);
  m->exec = nullptr;
  m->graph = nullptr;
}

extern "C" int sj_model_set_batches(sj_model* m, const int32_t* ids, const int32_t* targets, long observations) {
  SJ_REQUIRE(m && ids && targets, "set_batches: null");
  SJ_REQUIRE(!m->value_n && m->optimizer == 0,
             "set_batches: gradient accumulation covers the byte language models trained with AdamW");
  SJ_REQUIRE(observations >= 1 && observations <= sj_model::OBS_MAX, "set_batches: observations %ld (1 .. %ld)",
             observations, sj_model::OBS_MAX);
  const long n = observations * m->M;
  for (long i = 0; i < n; i++)
    SJ_REQUIRE(ids[i] >= 0 && ids[i] < m->V && targets[i] >= 0 && targets[i] < m->V,
               "batch token %ld out of vocabulary", i);
  SJ_HIP(hipStreamSynchronize(m->stream));
  if (observations > m->obs_cap) {
    void *pi = nullptr, *pt = nullptr;
    TRY(dalloc(m, &pi, sizeof(int32_t) * (size_t)n));
    TRY(dalloc(m, &pt, sizeof(int32_t) * (size_t)n));
    m->obs_ids = (int32_t*)pi;
    m->obs_targets = (int32_t*)pt;
    m->obs_cap = observations;
  }
  if (observations > 1 && !m->g_acc) {
    void* pg = nullptr;
    TRY(dalloc(m, &pg, sizeof(float) * (size_t)m->n_params));
    m->g_acc = (float*)pg;
  }
  SJ_HIP(hipMemcpy(m->obs_ids, ids, sizeof(int32_t) * (size_t)n, hipMemcpyHostToDevice));
  SJ_HIP(hipMemcpy(m->obs_targets, targets, sizeof(int32_t) * (size_t)n, hipMemcpyHostToDevice));
  if (observations == 1) {  // one observation: the ordinary batch buffers
    SJ_HIP(hipMemcpy(m->ids, ids, sizeof(int32_t) * (size_t)m->M, hipMemcpyHostToDevice));
    SJ_HIP(hipMemcpy(m->targets, targets, sizeof(int32_t) * (size_t)m->M, hipMemcpyHostToDevice));
  }
  if (observations != m->obs) drop_graph(m);
  m->obs = observations;
  return SJ_OK;
}

extern "C" int sj_model_set_batch(sj_model* m, const int32_t* ids, const int32_t* targets, int on_device) {
  SJ_REQUIRE(m && ids && targets, "set_batch: null");
  SJ_REQUIRE(!m->value_n, "set_batch: a native value model takes sj_model_set_value_batch");
  if (m->obs != 1) {  // back to one observation per update
    SJ_HIP(hipStreamSynchronize(m->stream));
    drop_graph(m);
    m->obs = 1;
  }
  size_t bytes = sizeof(int32_t) * (size_t)m->M;
  if (on_device) {
    SJ_HIP(hipMemcpyAsync(m->ids, ids, bytes, hipMemcpyDeviceToDevice, m->stream));
    SJ_HIP(hipMemcpyAsync(m->targets, targets, bytes, hipMemcpyDeviceToDevice, m->stream));
  } else {
    for (long i = 0; i < m->M; i++)
      SJ_REQUIRE(ids[i] >= 0 && ids[i] < m->V && targets[i] >= 0 && targets[i] < m->V,
                 "batch token %ld out of vocabulary", i);
    SJ_HIP(hipMemcpyAsync(m->ids, ids, bytes, hipMemcpyHostToDevice, m->stream));
    SJ_HIP(hipMemcpyAsync(m->targets, targets, bytes, hipMemcpyHostToDevice, m->stream));
    SJ_HIP(hipStreamSynchronize(m->stream));
  }
  return SJ_OK;
}

extern "C" int sj_model_set_value_batch(sj_model* m, const int32_t* ids, const int32_t* positions,
                                        const int32_t* labels) {
  SJ_REQUIRE(m && m->value_n && ids && positions && labels, "set_value_batch: native value model and arrays");
  for (long i = 0; i < m->M; i++) SJ_REQUIRE(ids[i] >= 0 && ids[i] < m->V, "native token %ld out of vocabulary", i);
  for (long r = 0; r < m->HR; r++)
    SJ_REQUIRE(positions[r] >= r * m->T && positions[r] < (r + 1) * m->T && labels[r] >= 0 && labels[r] < m->value_n,
               "native request %ld: SEP position outside its row or label outside the values", r);
  SJ_HIP(hipMemcpyAsync(m->ids, ids, sizeof(int32_t) * (size_t)m->M, hipMemcpyHostToDevice, m->stream));
  SJ_HIP(hipMemcpyAsync(m->sel, positions, sizeof(int32_t) * (size_t)m->HR, hipMemcpyHostToDevice, m->stream));
  SJ_HIP(hipMemcpyAsync(m->labels, labels, sizeof(int32_t) * (size_t)m->HR, hipMemcpyHostToDevice, m->stream));
  SJ_HIP(hipStreamSynchronize(m->stream));
  return SJ_OK;
}

extern "C" int sj_model_forward_backward(sj_model* m) {
  SJ_REQUIRE(m, "forward_backward: null");
  if (m->optimizer == 1) TRY(stage_sgd(m, 0.f));  // the backward's parameter-VJP seed
  if (m->obs > 1) {  // the accumulated gradients of every observation, left in the gradient arena
    TRY(accumulate_observations(m, false));
    SJ_HIP(hipMemcpyAsync(m->g, m->g_acc, sizeof(float) * (size_t)m->n_params, hipMemcpyDeviceToDevice, m->stream));
    return SJ_OK;
  }
  TRY(forward(m));
  TRY(backward(m));
  return SJ_OK;
}

extern "C" int sj_model_use_graph(sj_model* m, int on) {
  SJ_REQUIRE(m, "use_graph: null");
  m->use_graph = on != 0;
  return SJ_OK;
}

static int run_step(sj_model* m);

extern "C" int sj_model_train_step(sj_model* m, float lr) {
  SJ_REQUIRE(m, "train_step: null");
  if (m->optimizer == 1) {
    TRY(stage_sgd(m, lr));
    m->step += 1;
    return run_step(m);
  }
  // Adam::update increments the step and forms 1/(1-beta^step) on the host
  // in f32 (crates/sejong-gpu/src/lib.rs:950-951).
  m->step += 1;
  const int slot = (int)(m->step % sj_model::RING);
  sj_adam_step* h = m->step_host + slot;
  SJ_HIP(hipEventSynchronize(m->step_done[slot]));  // copy from RING steps ago
  h->lr = lr;
  h->beta1 = m->adam.beta1;
  h->beta2 = m->adam.beta2;
  h->eps = m->adam.epsilon;
  h->weight_decay = m->adam.weight_decay;
  h->inv_b1 = 1.f / (1.f - powf(m->adam.beta1, (float)m->step));
  h->inv_b2 = 1.f / (1.f - powf(m->adam.beta2, (float)m->step));
  h->clip_norm = m->adam.clip_norm;
  h->loss_scale = m->adam.loss_scale;
  h->clip_enabled = m->adam.clip_enabled;
  SJ_HIP(hipMemcpyAsync(m->step_dev, h, sizeof(sj_adam_step), hipMemcpyHostToDevice, m->stream));
  SJ_HIP(hipEventRecord(m->step_done[slot], m->stream));
  return run_step(m);
}

// the step eagerly, or captured once as a hipGraph and replayed
static int run_step(sj_model* m) {
  if (m->profiling) {
    // ~5 ms at 2.4 GHz: longer than the host needs to enqueue one step
    k_profile_hold<<<1, 64, 0, m->stream>>>(1500);
    SJ_LAUNCH_CHECK("profile hold");
    return whole_step(m);
  }
  if (!m->use_graph) return whole_step(m);
  if (!m->exec) {
    SJ_HIP(hipStreamBeginCapture(m->stream, hipStreamCaptureModeThreadLocal));
    int st = whole_step(m);
    hipGraph_t g = nullptr;
    hipError_t e = hipStreamEndCapture(m->stream, &g);
    if (st) {
      if (g) hipGraphDestroy(g);
      return st;
    }
    SJ_HIP(e);
    m->graph = g;
    SJ_HIP(hipGraphInstantiate(&m->exec, g, nullptr, nullptr, 0));
  }
  SJ_HIP(hipGraphLaunch(m->exec, m->stream));
  m->mt_stale = m->planes && !m->fused_update;  // a replayed AdamW update rewrote the transposed mirror
  return SJ_OK;
}

extern "C" int sj_model_profile(sj_model* m, int on) {
  SJ_REQUIRE(m && on >= 0 && on <= 4, "profile: mode");
  if (on == 2 && !m->flush) TRY(dalloc(m, (void**)&m->flush, (size_t)FLUSH_FLOATS * 4));
  m->profiling = on != 0;
  m->cold = on == 2;
  m->kernel_events = on == 3 || on == 4;
  m->instep = on == 4;
  return SJ_OK;
}

// Aggregates the events of the ops recorded since the last call (syncs).
extern "C" long sj_model_profile_collect(sj_model* m) {
  if (!m) return -1;
  if (hipStreamSynchronize(m->stream) != hipSuccess) return -1;
  m->agg_names.clear();
  m->agg_ms.clear();
  m->agg_calls.clear();
  m->agg_kernel.clear();
  auto add = [&](const std::string& nm, float ms, const std::string& kernel) {
    size_t j = 0;
    while (j < m->agg_names.size() && m->agg_names[j] != nm) j++;
    if (j == m->agg_names.size()) {
      m->agg_names.push_back(nm);
      m->agg_ms.push_back(0.0);
      m->agg_calls.push_back(0);
      m->agg_kernel.push_back(kernel);
    }
    m->agg_ms[j] += ms;
    m->agg_calls[j] += 1;
  };
  if (m->prof_kused.size() != m->prof_names.size()) return -1;  // an op was left open
  for (size_t k = 0; k < m->prof_names.size(); k++) {
    float ms = 0.f;
    const std::string nm(m->prof_names[k]);
    if (!m->instep) {  // (in-step mode times the kernels only)
      if (hipEventElapsedTime(&ms, m->prof_events[4 * k], m->prof_events[4 * k + 1]) != hipSuccess) return -1;
      add(nm, ms, m->prof_kernel[k]);
    }
    if (m->prof_kused[k]) {  // the GEMM kernel alone, from its own start to its end
      if (hipEventElapsedTime(&ms, m->prof_events[4 * k + 2], m->prof_events[4 * k + 3]) != hipSuccess) return -1;
      add(nm + "#kernel", ms, m->prof_kernel[k]);
    }
  }
  m->prof_names.clear();
  m->prof_kused.clear();
  m->prof_kernel.clear();
  return (long)m->agg_names.size();
}

extern "C" int sj_model_profile_kernel(sj_model* m, long i, const char** kernel) {
  SJ_REQUIRE(m && i >= 0 && i < (long)m->agg_kernel.size(), "profile_kernel: index %ld", i);
  if (kernel) *kernel = m->agg_kernel[i].c_str();
  return SJ_OK;
}

extern "C" int sj_model_profile_entry(sj_model* m, long i, const char** name, double* total_ms, long* calls) {
  SJ_REQUIRE(m && i >= 0 && i < (long)m->agg_names.size(), "profile_entry: index %ld", i);
  if (name) *name = m->agg_names[i].c_str();
  if (total_ms) *total_ms = m->agg_ms[i];
  if (calls) *calls = m->agg_calls[i];
  return SJ_OK;
}

extern "C" int sj_model_read_loss(sj_model* m, double* loss, double* grad_norm) {
  SJ_REQUIRE(m, "read_loss: null");
  SJ_HIP(hipStreamSynchronize(m->stream));
  double l = 0, ss = 0;
  int32_t flag = 0;
  {  // the step's loss: the observations' summaries (each weighted 1/accumulation), in order
    double slots[sj_model::OBS_MAX];
    SJ_HIP(hipMemcpy(slots, m->loss, sizeof(double) * (size_t)m->obs, hipMemcpyDeviceToHost));
    for (long o = 0; o < m->obs; o++) l += slots[o];
  }
  SJ_HIP(hipMemcpy(&ss, m->sumsq, sizeof(double), hipMemcpyDeviceToHost));
  SJ_HIP(hipMemcpy(&flag, m->status, sizeof(int32_t), hipMemcpyDeviceToHost));
  if (loss) *loss = l;
  if (grad_norm) *grad_norm = sqrt(ss) / (m->optimizer == 1 ? 1.0 : (double)m->adam.loss_scale);
  if (flag) return sjh::fail(SJ_ERR_NONFINITE, "nonfinite clipping gradient");
  return SJ_OK;
}

// Activation pack in the oracle's order (per layer x, z, q, k, v, o, lse,
// x1, z2, g, u, h; then x_L, hn, logits), converted to fp32 (exact for bf16).
extern "C" long sj_model_activation_count(const sj_model* m) {
  if (!m) return -1;
  long n = 0;
  for (const Stage& S : m->stages)
    n += S.count * (6 * S.M * S.d + 2 * S.M * S.J + S.M * S.HQ + (m->E ? S.M * m->E : 3 * S.M * S.F)) +
         2 * S.M * S.d;
  if (m->hier) {
    const Stage &E = m->stages[0], &G = m->stages[1], &D = m->stages[2];
    n += G.M * E.d + G.M * D.d + D.d + 2 * E.M * D.d + 2 * E.M * G.d;
  }
  return n + m->HR * m->HV;
}

static int export_matrix(sj_model* m, const void* dev, int dt, long rows, long ld, long col0, long cols,
                         float* host) {
  size_t es = dt == SJ_BF16 ? 2 : 4;
  std::vector<uint8_t> raw((size_t)rows * ld * es);
  SJ_HIP(hipMemcpy(raw.data(), dev, raw.size(), hipMemcpyDeviceToHost));
  for (long r = 0; r < rows; r++)
    for (long c = 0; c < cols; c++) {
      size_t i = (size_t)r * ld + col0 + c;
      float v;
      if (dt == SJ_BF16) {
        uint32_t b = (uint32_t)((const uint16_t*)raw.data())[i] << 16;
        memcpy(&v, &b, 4);
      } else {
        v = ((const float*)raw.data())[i];
      }
      host[(size_t)r * cols + c] = v;
    }
  return SJ_OK;
}

extern "C" int sj_model_export_activations(sj_model* m, float* host) {
  SJ_REQUIRE(m && host, "export_activations: null");
  SJ_HIP(hipStreamSynchronize(m->stream));
  const int dt = m->dt;
  float* p = host;
  for (const Stage& S : m->stages) {
    const long M = S.M, d = S.d, J = S.J, F = S.F, NQ = S.NQKV;
    for (long l = S.first; l < S.first + S.count; l++) {
      TRY(export_matrix(m, xin(m, l), dt, M, d, 0, d, p)); p += M * d;
      TRY(export_matrix(m, m->z[l], dt, M, d, 0, d, p)); p += M * d;
      TRY(export_matrix(m, m->qkv[l], dt, M, NQ, 0, d, p)); p += M * d;
      TRY(export_matrix(m, m->qkv[l], dt, M, NQ, d, J, p)); p += M * J;
      TRY(export_matrix(m, m->qkv[l], dt, M, NQ, d + J, J, p)); p += M * J;
      TRY(export_matrix(m, m->o[l], dt, M, d, 0, d, p)); p += M * d;
      TRY(export_matrix(m, m->lse[l], SJ_F32, M, S.HQ, 0, S.HQ, p)); p += M * S.HQ;
      TRY(export_matrix(m, m->x1[l], dt, M, d, 0, d, p)); p += M * d;
      TRY(export_matrix(m, m->z2[l], dt, M, d, 0, d, p)); p += M * d;
      if (m->E) {  // the router's stored logits stand for g, u, h
        TRY(export_matrix(m, m->mlog[l], SJ_BF16, M, m->E, 0, m->E, p)); p += M * m->E;
        continue;
      }
      TRY(export_matrix(m, m->gg[l], dt, M, F, 0, F, p)); p += M * F;
      TRY(export_matrix(m, m->uu[l], dt, M, F, 0, F, p)); p += M * F;
      TRY(export_matrix(m, m->hh[l], dt, M, F, 0, F, p)); p += M * F;
    }
    TRY(export_matrix(m, xtop(m, S), dt, M, d, 0, d, p)); p += M * d;
    TRY(export_matrix(m, S.out, dt, M, d, 0, d, p)); p += M * d;
  }
  if (m->hier) {
    const Stage &E = m->stages[0], &G = m->stages[1], &D = m->stages[2];
    TRY(export_matrix(m, m->pooled, dt, G.M, E.d, 0, E.d, p)); p += G.M * E.d;
    TRY(export_matrix(m, m->gd, dt, G.M, D.d, 0, D.d, p)); p += G.M * D.d;
    TRY(export_matrix(m, m->bosd, dt, 1, D.d, 0, D.d, p)); p += D.d;
    TRY(export_matrix(m, m->zb, dt, E.M, D.d, 0, D.d, p)); p += E.M * D.d;
    TRY(export_matrix(m, m->bytes, dt, E.M, D.d, 0, D.d, p)); p += E.M * D.d;
    TRY(export_matrix(m, m->opo, dt, E.M, G.d, 0, G.d, p)); p += E.M * G.d;
    TRY(export_matrix(m, m->hn, dt, E.M, G.d, 0, G.d, p)); p += E.M * G.d;
  }
  TRY(export_matrix(m, m->logits, SJ_F32, m->HR, m->Vp, 0, m->HV, p));
  return SJ_OK;
}

extern "C" int sj_model_materialize_grads(sj_model* m) {
  SJ_REQUIRE(m, "materialize_grads: null");
  if (m->optimizer != 1) return SJ_OK;
  TRY(sj_factored_apply(m->stream, m->fmeta_mat, m->ftiles, 0, 0.f, 0.f, nullptr));
  SJ_HIP(hipStreamSynchronize(m->stream));
  return SJ_OK;
}

extern "C" int sj_model_vjp_info(const sj_model* m, long* compressed, long* dense, long* basis_groups,
                                 long* projection_groups, uint64_t* rng_state) {
  SJ_REQUIRE(m, "vjp_info: null");
  if (compressed) *compressed = m->st_compressed;
  if (dense) *dense = m->st_dense;
  if (basis_groups) *basis_groups = m->st_basis;
  if (projection_groups) *projection_groups = m->st_projection;
  if (rng_state) *rng_state = m->vjp_rng;
  return SJ_OK;
}

extern "C" long sj_model_steps(const sj_model* m) { return m ? m->step : -1; }

extern "C" int sj_model_set_vjp_rng(sj_model* m, uint64_t rng_state) {
  SJ_REQUIRE(m && m->optimizer == 1, "set_vjp_rng: SGD model required");
  m->vjp_rng = rng_state;
  return SJ_OK;
}

extern "C" int sj_model_buffer(sj_model* m, const char* what, void** ptr, long* elements) {
  SJ_REQUIRE(m && what && ptr, "buffer: null");
  std::string w(what);
  long n = 0;
  if (w == "logits") { *ptr = m->logits; n = m->HR * m->Vp; }
  else if (w == "dlogits") { *ptr = m->dlogits; n = m->HR * m->Vp; }
  else if (w == "loss_rows") { *ptr = m->loss_rows; n = m->M; }
  else if (w == "ids") { *ptr = m->ids; n = m->M; }
  else if (w == "targets") { *ptr = m->targets; n = m->M; }
  else if (w == "params") { *ptr = m->w; n = m->n_params; }
  else if (w == "grads") { *ptr = m->g; n = m->n_params; }
  else if (w == "mirror") { *ptr = m->mirror; n = m->mirror ? m->n_params : 0; }
  else if (w == "mirror_t") { *ptr = m->mirror_t; n = m->mirror_t ? m->n_params : 0; }
  else if (w == "workspace") { *ptr = m->ws; n = (long)m->ws_bytes; }
  else if (w == "stream") { *ptr = (void*)m->stream; n = 0; }
  else if (w == "grad_sq_slots") { *ptr = m->gsq; n = m->gsq_ok ? m->gsq_count : 0; }
  else if (w == "vjp_columns" && m->vjp) { *ptr = m->vjp_cols; n = m->vjp_R; }
  else if (w == "vjp_rows" && m->vjp) { *ptr = m->vjp_rows; n = m->vjp_k; }
  else if (w == "vjp_map" && m->vjp) { *ptr = m->vjp_map; n = m->d; }
  else if (w == "vjp_basis" && m->vjp) { *ptr = m->vjp_q; n = m->M * m->vjp_R; }
  else if (m->E && w.rfind("route_", 0) == 0 && w.find('.') != std::string::npos) {
    // route_ids.<l>, route_weights.<l> [rows][top_k], route_counts.<l>
    // [experts], route_offsets.<l> [experts + 1] of MoE layer l
    const std::string kind = w.substr(0, w.find('.'));
    char* end = nullptr;
    const long l = strtol(w.c_str() + w.find('.') + 1, &end, 10);
    SJ_REQUIRE(end && *end == 0 && l >= 0 && l < m->L, "buffer: bad layer in %s", what);
    if (kind == "route_ids") { *ptr = m->mids[l]; n = m->M * m->K; }
    else if (kind == "route_weights") { *ptr = m->mwts[l]; n = m->M * m->K; }
    else if (kind == "route_counts") { *ptr = m->mcnt[l]; n = m->E; }
    else if (kind == "route_offsets") { *ptr = m->moff[l]; n = m->E + 1; }
    else if (kind == "route_pslot") { *ptr = m->mps[l]; n = m->cap; }
    else if (kind == "route_ppos") { *ptr = m->mpp[l]; n = m->M * m->K; }
    else return sjh::fail(SJ_ERR_INVALID, "buffer: unknown name %s", what);
  }
  else return sjh::fail(SJ_ERR_INVALID, "buffer: unknown name %s", what);
  if (elements) *elements = n;
  return SJ_OK;
}

// ------------------------------------------------------------ KV cache
// Model::new_cache / forward_cached (model lib.rs:36-50, 359-394;
// architecture.rs:395-533, 651-799): per layer the keys and values of one
// sequence, [positions][HK * head_dim] in the compute dtype, and scratch for
// up to `capacity` new rows.  A call runs the blocks over the new tokens at
// their positions with the same kernels as the training forward (RoPE rows
// of a table over the stage's positions, the cached attention kernels
// reading the cache), so each row is computed exactly as in the full
// forward; then the final norm and the fp32 head on the last row.
//
// The hierarchical model (HierarchyCache, architecture.rs:399-412) keeps
// one cache per stage: the encoder's and decoder's over the bytes
// (`capacity` positions), the global stage's over the patches
// (ceil(capacity / patch) positions), plus the state of the patch being
// filled: its encoded rows (the reference keeps their fp32 sum, patch_sum,
// and their count; keeping the rows lets the completed patch be pooled by
// the full forward's own patch_pool, the same fp32 sum in the same order)
// and the decoder context of the last completed patch (global_context).
struct sj_cache {
  sj_model* m = nullptr;
  long capacity = 0, length = 0;
  std::vector<void*> keys, values;  // [layer] -> [positions of its stage][J]
  std::vector<long> scap;           // [stage] positions its cache holds
  std::vector<float*> rope;         // [stage] RoPE table [scap][Dh/2] (cos, sin)
  void *x[2] = {}, *z = nullptr, *q = nullptr, *o = nullptr, *x1 = nullptr, *z2 = nullptr;
  void *gg = nullptr, *uu = nullptr, *hh = nullptr, *hn = nullptr;
  int32_t* ids = nullptr;
  float* logits = nullptr;  // [Vp] fp32, the last row's
  // mixture of experts: routing and packed rows for up to `capacity` tokens
  long mcap = 0;
  uint16_t *mlog = nullptr, *mzp = nullptr, *myp = nullptr;
  int32_t *mids = nullptr, *mcnt = nullptr, *moff = nullptr, *mps = nullptr, *mpp = nullptr;
  float* mwts = nullptr;
  // hierarchical: encoded bytes (encoder_norm output), the filling patch's
  // encoded rows [patch][de], pooled patches, the global stage's normed
  // output, decoder contexts of the patches and of the BOS row, the
  // broadcast contexts, encoder_to_decoder, decoder_norm and
  // output_projection outputs
  void *enc = nullptr, *prow = nullptr, *pooled = nullptr, *gout = nullptr, *ctxs = nullptr, *bosd = nullptr;
  void *gctx = nullptr, *zb = nullptr, *bytes = nullptr, *dec = nullptr, *opo = nullptr;
  long pcount = 0;       // bytes of the filling patch (patch_count)
  bool has_ctx = false;  // gctx holds global_context
  std::vector<void*> allocations;
};

namespace {
int calloc_(sj_cache* c, void** p, size_t bytes) {
  if (bytes == 0) bytes = 256;
  hipError_t e = hipMalloc(p, bytes);
  if (e != hipSuccess) {
    size_t fr = 0, tot = 0;
    hipMemGetInfo(&fr, &tot);
    return sjh::fail(SJ_ERR_CAPACITY, "cache allocation: required %zu bytes, available %zu bytes", bytes, fr);
  }
  c->allocations.push_back(*p);
  return hipMemset(*p, 0, bytes) == hipSuccess ? SJ_OK : sjh::fail(SJ_ERR_HIP, "cache allocation: clear");
}

// cached_blocks (architecture.rs:474-533): the blocks of stage si over n
// new rows in c->x[0] at positions L .. L + n - 1 of the stage's cache;
// then the stage's closing norm into `out` (the encoder, global or decoder
// norm, or the final norm of a one-stage model)
int cached_blocks(sj_model* m, sj_cache* c, int si, long n, long L, void* out) {
  const Stage& S = m->stages[si];
  hipStream_t s = m->stream;
  const long d = S.d, J = S.J, F = S.F, cap = c->scap[si];
  const int dt = m->dt;
  const size_t es = m->esz;
  const float eps = m->c.norm_epsilon;
  const float* rope = c->rope[si] + L * S.Dh;  // row r of this view is position L + r
  const long rope_t = cap - L;
  int cur = 0;
  for (long l = S.first; l < S.first + S.count; l++) {
    const Layer& y = m->layers[l];
    void* x = c->x[cur];
    void* xo = c->x[cur ^ 1];
    char* kc = (char*)c->keys[l] + L * J * es;
    char* vc = (char*)c->values[l] + L * J * es;
    if (m->planes) {
      const uint16_t *W = m->mirror, *WT = m->mirror_t;
      TRY(sj_rmsnorm_fwd_t(s, (const uint16_t*)x, W + y.an, (uint16_t*)c->z, nullptr, 0, n, d, eps));
      TRY(sjh::qkv_fwd_t_out(s, (const uint16_t*)c->z, d, n, d, WT + y.qkv, d, d, J, (uint16_t*)c->q, d,
                             (uint16_t*)kc, J, (uint16_t*)vc, J, rope, rope_t, S.Dh, nullptr, 0));
      TRY(sj_attention_fwd_cached(s, c->q, d, c->keys[l], c->values[l], J, cap, dt, n, L, S.HQ, S.HK, S.Dh, S.window,
                                  c->o, d));
      TRY(sj_linear_residual_fwd_t(s, (const uint16_t*)c->o, d, n, d, WT + y.wo, d, d, (const uint16_t*)x, d,
                                   (uint16_t*)c->x1, d));
      TRY(sj_rmsnorm_fwd_t(s, (const uint16_t*)c->x1, W + y.fn, (uint16_t*)c->z2, nullptr, 0, n, d, eps));
      if (m->E) {  // routed experts over the new rows (architecture.rs:516-529)
        const long E = m->E, K = m->K, mc = sj_route_pack_capacity(n * K, E);
        TRY(sj_router_topk(s, (const uint16_t*)c->z2, d, W + y.router, d, n, E, K, c->mlog, c->mids, c->mwts));
        TRY(sj_route_pack(s, c->mids, n, K, E, nullptr, nullptr, c->mcnt, c->moff, c->mps, c->mpp, mc));
        TRY(sj_moe_gather(s, (const uint16_t*)c->z2, d, d, c->mps, K, mc, c->mzp, nullptr, mc));
        TRY(sj_moe_gate_up_fwd(s, c->moff, E, mc, c->mzp, d, d, WT + y.gu, WT + y.gu + F * d, d, 2 * F * d, F,
                               (uint16_t*)c->gg, (uint16_t*)c->uu, (uint16_t*)c->hh, F, nullptr, mc));
        TRY(sj_moe_down_fwd(s, c->moff, E, mc, (const uint16_t*)c->hh, F, F, WT + y.down, F, d * F, d, c->myp, d));
        TRY(sj_moe_combine(s, c->myp, d, d, c->mids, c->mpp, c->mwts, n, K, (const uint16_t*)c->x1, d,
                           (uint16_t*)xo, d));
      } else {
        TRY(sj_gate_up_fwd_t(s, (const uint16_t*)c->z2, d, n, d, WT + y.gu, WT + y.gu + F * d, d, F,
                             (uint16_t*)c->gg, (uint16_t*)c->uu, (uint16_t*)c->hh, F, nullptr, 0));
        TRY(sj_linear_residual_fwd_t(s, (const uint16_t*)c->hh, F, n, F, WT + y.down, F, d, (const uint16_t*)c->x1, d,
                                     (uint16_t*)xo, d));
      }
    } else {
      TRY(sj_rmsnorm_fwd(s, x, dt, wc(m, y.an), dt, c->z, n, d, eps));
      const char* wq = (const char*)wc(m, y.qkv);
      const long NQ = S.NQKV;
      TRY(sj_qkv_fwd(s, c->z, d, n, d, wq, NQ, wq + d * es, NQ, wq + (d + J) * es, NQ, d, J, c->q, d, kc, J, vc, J, dt,
                     rope, rope_t, S.Dh));
      TRY(sj_attention_fwd_cached(s, c->q, d, c->keys[l], c->values[l], J, cap, dt, n, L, S.HQ, S.HK, S.Dh, S.window,
                                  c->o, d));
      TRY(sj_linear_residual_fwd(s, c->o, d, n, d, wc(m, y.wo), d, d, x, d, c->x1, d, dt));
      TRY(sj_rmsnorm_fwd(s, c->x1, dt, wc(m, y.fn), dt, c->z2, n, d, eps));
      const char* wg = (const char*)wc(m, y.gu);
      TRY(sj_gate_up_fwd(s, c->z2, d, n, d, wg, 2 * F, wg + F * es, 2 * F, F, c->gg, c->uu, c->hh, F, dt));
      TRY(sj_linear_residual_fwd(s, c->hh, F, n, F, wc(m, y.down), d, d, c->x1, d, xo, d, dt));
    }
    cur ^= 1;
  }
  TRY(sj_rmsnorm_fwd(s, c->x[cur], dt, wc(m, S.norm), dt, out, n, d, eps));
  return SJ_OK;
}

// the embedding of n tokens (c->ids from row `at`) into c->x[0]
int cached_embed(sj_model* m, sj_cache* c, long at, long n) {
  return sj_embedding_fwd(m->stream, wc(m, m->emb), m->dt, c->ids + at, c->x[0], m->dt, n, m->stages[0].d);
}

// the decoder side of hidden_from_encoded for n bytes at position L whose
// encoded rows are in c->enc and whose broadcast contexts are in c->zb:
// encoder_to_decoder + contexts, the decoder stage, output_projection and
// the final norm into c->hn (architecture.rs:601-626, 690-725)
int cached_decoder(sj_model* m, sj_cache* c, long n, long L) {
  hipStream_t s = m->stream;
  const int dt = m->dt;
  const Stage &E = m->stages[0], &D = m->stages[2];
  const long de = E.d, dd = D.d, dg = m->stages[1].d;
  TRY(sj_gemm(s, 0, 0, n, dd, de, c->enc, dt, de, wc(m, m->h_e2d), dt, dd, c->bytes, dt, dd, 0, nullptr, 0));
  TRY(sj_add(s, c->bytes, dt, c->zb, dt, c->x[0], dt, n * dd, 1.f));
  TRY(cached_blocks(m, c, 2, n, L, c->dec));
  TRY(sj_gemm(s, 0, 0, n, dg, dd, c->dec, dt, dd, wc(m, m->h_op), dt, dg, c->opo, dt, dg, 0, nullptr, 0));
  return sj_rmsnorm_fwd(s, c->opo, dt, wc(m, m->final_norm), dt, c->hn, n, dg, m->c.norm_epsilon);
}

// hierarchical_prefill (architecture.rs:534-650): a fresh cache and at least
// one patch of bytes: the whole stack over the n bytes as the full forward
// runs it (the partial last patch pooled over its own bytes and run
// through the global stage at its slot, which its completion rewrites);
// then global_context = the last completed patch's context (or the BOS
// row's) and the filling patch's encoded rows
int hierarchical_prefill(sj_model* m, sj_cache* c, long n, long& last) {
  hipStream_t s = m->stream;
  const int dt = m->dt;
  const size_t es = m->esz;
  const long P = m->P, de = m->stages[0].d, dg = m->stages[1].d, dd = m->stages[2].d;
  const long np = (n + P - 1) / P, done = n / P;
  TRY(cached_embed(m, c, 0, n));
  TRY(cached_blocks(m, c, 0, n, 0, c->enc));
  TRY(sj_patch_pool(s, c->enc, dt, 1, n, de, P, c->pooled));
  TRY(sj_gemm(s, 0, 0, np, dg, de, c->pooled, dt, de, wc(m, m->h_e2g), dt, dg, c->x[0], dt, dg, 0, nullptr, 0));
  TRY(cached_blocks(m, c, 1, np, 0, c->gout));
  TRY(sj_gemm(s, 0, 0, np, dd, dg, c->gout, dt, dg, wc(m, m->h_g2d), dt, dd, c->ctxs, dt, dd, 0, nullptr, 0));
  TRY(sj_gemm(s, 0, 0, 1, dd, dg, wc(m, m->h_bos), dt, dg, wc(m, m->h_g2d), dt, dd, c->bosd, dt, dd, 0, nullptr, 0));
  TRY(sj_patch_broadcast(s, c->ctxs, c->bosd, dt, 1, n, dd, P, c->zb));
  TRY(cached_decoder(m, c, n, 0));
  last = n - 1;
  const void* ctx = done == 0 ? c->bosd : (const char*)c->ctxs + (done - 1) * dd * es;
  SJ_HIP(hipMemcpyAsync(c->gctx, ctx, (size_t)dd * es, hipMemcpyDeviceToDevice, s));
  c->has_ctx = true;
  c->pcount = n % P;
  if (c->pcount)
    SJ_HIP(hipMemcpyAsync(c->prow, (const char*)c->enc + done * P * de * es, (size_t)c->pcount * de * es,
                          hipMemcpyDeviceToDevice, s));
  return SJ_OK;
}

// hidden_cached's hierarchical loop (architecture.rs:667-783): the bytes in
// chunks that end at patch boundaries; each chunk through the encoder at
// its positions, the decoder with the filling patch's context (the last
// completed patch's, or the BOS row's), and its encoded rows appended to
// the filling patch; a completed patch is pooled, run through the global
// stage at its patch position and gives the next context.  `last`: the
// row of c->hn that holds the last byte's output (the last chunk's)
int hierarchical_cached(sj_model* m, sj_cache* c, long n, long& last) {
  hipStream_t s = m->stream;
  const int dt = m->dt;
  const size_t es = m->esz;
  const long P = m->P, de = m->stages[0].d, dg = m->stages[1].d, dd = m->stages[2].d;
  if (c->length == 0 && n >= P) return hierarchical_prefill(m, c, n, last);
  if (!c->has_ctx) {
    TRY(sj_gemm(s, 0, 0, 1, dd, dg, wc(m, m->h_bos), dt, dg, wc(m, m->h_g2d), dt, dd, c->gctx, dt, dd, 0, nullptr, 0));
    c->has_ctx = true;
  }
  long i = 0;
  while (i < n) {
    const long count = std::min(P - c->pcount, n - i), pos = c->length + i;
    TRY(cached_embed(m, c, i, count));
    TRY(cached_blocks(m, c, 0, count, pos, c->enc));
    // every row of the chunk lies in one patch: its broadcast row is the
    // context (the broadcast's first-patch rows take the BOS argument)
    TRY(sj_patch_broadcast(s, c->gctx, c->gctx, dt, 1, count, dd, P, c->zb));
    TRY(cached_decoder(m, c, count, pos));
    last = count - 1;
    SJ_HIP(hipMemcpyAsync((char*)c->prow + c->pcount * de * es, c->enc, (size_t)count * de * es,
                          hipMemcpyDeviceToDevice, s));
    c->pcount += count;
    if (c->pcount == P) {
      TRY(sj_patch_pool(s, c->prow, dt, 1, P, de, P, c->pooled));
      TRY(sj_gemm(s, 0, 0, 1, dg, de, c->pooled, dt, de, wc(m, m->h_e2g), dt, dg, c->x[0], dt, dg, 0, nullptr, 0));
      TRY(cached_blocks(m, c, 1, 1, pos / P, c->gout));
      TRY(sj_gemm(s, 0, 0, 1, dd, dg, c->gout, dt, dg, wc(m, m->h_g2d), dt, dd, c->gctx, dt, dd, 0, nullptr, 0));
      c->pcount = 0;
    }
    i += count;
  }
  return SJ_OK;
}
}  // namespace

extern "C" int sj_cache_create(sj_model* m, long capacity, sj_cache** out) {
  SJ_REQUIRE(m && out && capacity > 0, "new_cache: arguments");
  SJ_REQUIRE(!m->value_n, "new_cache: the cached forward covers the byte language models (dense, MoE, hierarchical)");
  for (const Stage& S : m->stages)
    SJ_REQUIRE(m->planes ? S.attn_tt : m->dt == SJ_F32,
               "new_cache: the cached forward needs the MFMA-layout attention (bf16) or fp32 storage");
  sj_cache* c = new sj_cache();
  c->m = m;
  c->capacity = capacity;
  const size_t es = m->esz;
  long dmax = m->d, fmax = 0;
  for (const Stage& S : m->stages) {
    dmax = std::max(dmax, S.d);
    fmax = std::max(fmax, S.F);
  }
  int st = SJ_OK;
  auto A = [&](void** p, size_t bytes) {
    if (!st) st = calloc_(c, p, bytes);
  };
  // positions per stage: the bytes, or the patches for the global stage
  c->scap.assign(m->stages.size(), capacity);
  if (m->hier) c->scap[1] = (capacity + m->P - 1) / m->P;
  c->rope.assign(m->stages.size(), nullptr);
  c->keys.assign(m->L, nullptr);
  c->values.assign(m->L, nullptr);
  for (size_t si = 0; si < m->stages.size(); si++) {
    const Stage& S = m->stages[si];
    for (long l = S.first; l < S.first + S.count; l++) {
      A(&c->keys[l], (size_t)c->scap[si] * S.J * es);
      A(&c->values[l], (size_t)c->scap[si] * S.J * es);
    }
    A((void**)&c->rope[si], (size_t)c->scap[si] * S.Dh * 4);
  }
  for (void** p : {&c->x[0], &c->x[1], &c->z, &c->q, &c->o, &c->x1, &c->z2, &c->hn})
    A(p, (size_t)capacity * dmax * es);
  if (m->E) {
    const Stage& S = m->stages[0];
    c->mcap = sj_route_pack_capacity(capacity * m->K, m->E);
    const long E = m->E, K = m->K, mc = c->mcap, d = S.d, F = S.F;
    A((void**)&c->mlog, (size_t)capacity * E * 2);
    A((void**)&c->mids, (size_t)capacity * K * 4);
    A((void**)&c->mwts, (size_t)capacity * K * 4);
    A((void**)&c->mcnt, (size_t)E * 4);
    A((void**)&c->moff, (size_t)(E + 1) * 4);
    A((void**)&c->mps, (size_t)mc * 4);
    A((void**)&c->mpp, (size_t)capacity * K * 4);
    A((void**)&c->mzp, (size_t)mc * d * 2);
    A((void**)&c->myp, (size_t)mc * d * 2);
    for (void** p : {&c->gg, &c->uu, &c->hh}) A(p, (size_t)mc * F * es);
  } else {
    for (void** p : {&c->gg, &c->uu, &c->hh}) A(p, (size_t)capacity * fmax * es);
  }
  if (m->hier) {
    const long de = m->stages[0].d, dg = m->stages[1].d, dd = m->stages[2].d, np = c->scap[1];
    A(&c->enc, (size_t)capacity * de * es);
    A(&c->prow, (size_t)m->P * de * es);
    A(&c->pooled, (size_t)np * de * es);
    A(&c->gout, (size_t)np * dg * es);
    A(&c->ctxs, (size_t)np * dd * es);
    A(&c->bosd, (size_t)dd * es);
    A(&c->gctx, (size_t)dd * es);
    A(&c->zb, (size_t)capacity * dd * es);
    A(&c->bytes, (size_t)capacity * dd * es);
    A(&c->dec, (size_t)capacity * dd * es);
    A(&c->opo, (size_t)capacity * dg * es);
  }
  A((void**)&c->ids, (size_t)capacity * 4);
  A((void**)&c->logits, (size_t)m->Vp * 4);
  for (size_t si = 0; si < m->stages.size() && !st; si++)
    st = sj_rope_table(m->stream, c->rope[si], c->scap[si], m->stages[si].Dh, m->c.rope_theta);
  if (!st && hipStreamSynchronize(m->stream) != hipSuccess) st = sjh::fail(SJ_ERR_HIP, "new_cache: sync");
  if (st) {
    sj_cache_destroy(c);
    return st;
  }
  *out = c;
  return SJ_OK;
}

extern "C" int sj_cache_destroy(sj_cache* c) {
  if (!c) return SJ_OK;
  if (c->m && c->m->stream) hipStreamSynchronize(c->m->stream);
  for (void* p : c->allocations) hipFree(p);
  delete c;
  return SJ_OK;
}

// HierarchyCache::reset (architecture.rs:406-412) with the length
extern "C" int sj_cache_reset(sj_cache* c) {
  SJ_REQUIRE(c, "cache reset: null");
  c->length = 0;
  c->pcount = 0;
  c->has_ctx = false;
  return SJ_OK;
}

extern "C" long sj_cache_length(const sj_cache* c) { return c ? c->length : -1; }

extern "C" int sj_model_forward_cached(sj_model* m, sj_cache* c, const int32_t* tokens, long n, float* logits) {
  SJ_REQUIRE(m && c && c->m == m && tokens && n > 0, "forward_cached: arguments");
  for (long i = 0; i < n; i++)
    SJ_REQUIRE(tokens[i] >= 0 && tokens[i] <= 256 && tokens[i] < m->V, "input tokens must be bytes or EOS");
  SJ_REQUIRE(c->length + n <= c->capacity, "KV cache context limit reached");
  hipStream_t s = m->stream;
  const long d = m->d;
  const int dt = m->dt;
  if (m->mt_stale) TRY(transpose_mirror(m));  // weights updated since the last forward
  SJ_HIP(hipMemcpyAsync(c->ids, tokens, (size_t)n * 4, hipMemcpyHostToDevice, s));
  long row = n - 1;  // the row of c->hn that holds the last token's output
  if (m->hier) {
    TRY(hierarchical_cached(m, c, n, row));
  } else {
    TRY(cached_embed(m, c, 0, n));
    TRY(cached_blocks(m, c, 0, n, c->length, c->hn));
  }
  // the last row, cast to F32, times the fp32 output matrix (model lib.rs:370-371)
  const char* last = (const char*)c->hn + row * d * m->esz;
  if (m->lm_planes)
    TRY(sj_gemm_planes(s, 1, m->Vp, d, (const uint16_t*)last, nullptr, d, m->hp[2], m->hp[3], d, c->logits, SJ_F32,
                       m->Vp, 0, nullptr, 0));
  else
    TRY(sj_gemm(s, 0, 0, 1, m->HV, d, last, dt, d, m->w + m->out, SJ_F32, m->Vp, c->logits, SJ_F32, m->Vp, 0, nullptr,
                0));
  if (logits) SJ_HIP(hipMemcpyAsync(logits, c->logits, (size_t)m->HV * 4, hipMemcpyDeviceToDevice, s));
  c->length += n;
  return SJ_OK;
}

extern "C" int sj_model_forward(sj_model* m) {
  SJ_REQUIRE(m, "forward: null");
  return forward(m);
}
