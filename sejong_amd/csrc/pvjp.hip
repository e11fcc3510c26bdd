// Forward-basis parameter VJP and the factored selected-row SGD (gfx950).
//
// Reference: crates/sejong-gpu/src/parameter_vjp.rs and
// python/sejong_kernels/ops/parameter.py.  For a projection Y = X W with a
// shared input X [n][a] (tokens x features):
//   indices   one SplitMix64 stream (seeded by one host draw) picks R donor
//             columns and S feature blocks by partial Fisher-Yates;
//   basis     Q [n][R] = classical Gram-Schmidt applied twice to the picked
//             donor columns, a column dropped when its residual norm falls
//             below the roundoff threshold;
//   prepare   A = X^T Q [a][R] and E = [Q^T ; (X[:, row] - Q A[row]^T) *
//             blocks/selected for the selected rows] [R+k][n];
//   vjp       coefficients = E dY [R+k][b]: right = the first R rows, tail
//             the rest;
//   apply     per parameter tile, G = dense + sum_terms scale (left right +
//             tail rows placed by row_map), then W update, or G written out,
//             or the FP64 sum of G^2.
// MI355X layout: X is read transposed (X^T [a][n], the layout the step
// already keeps for the dW GEMMs), so the feature rows of the residual are
// contiguous; E is kept as fp32 plus hi/lo bf16 planes, the operand form of
// the plane GEMMs that compute A and the coefficients.
#include <math.h>
#include <string.h>

#include "common.h"

using namespace sj;

namespace {

// ----------------------------------------------------------------- indices
__device__ __forceinline__ uint64_t splitmix_next(uint64_t& s) {
  s += 0x9e3779b97f4a7c15ULL;
  uint64_t z = s;
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
  return z ^ (z >> 31);
}
// Rng::index (crates/sejong-core/src/lib.rs:610-619, parameter.py:17-22)
__device__ __forceinline__ uint64_t splitmix_index(uint64_t& s, uint64_t n) {
  const uint64_t threshold = (0 - n) % n;
  for (;;) {
    const uint64_t x = splitmix_next(s);
    if (x >= threshold) return x % n;
  }
}

// parameter_indices (parameter.py:25-62).  One workgroup: the scratch
// permutations and the map are initialised in parallel, the draws are
// serial (each depends on the stream state) in lane 0, and the rows of a
// picked block are written by all lanes.
__global__ __launch_bounds__(256) void k_pvjp_indices(int32_t* __restrict__ scratch, int32_t* __restrict__ columns,
                                                      int32_t* __restrict__ rows, int32_t* __restrict__ map, long A,
                                                      long B, long NB, long S, long R, long group, uint64_t seed,
                                                      const uint64_t* __restrict__ seed_ptr) {
  __shared__ int32_t picked;
  const int t = threadIdx.x;
  for (long i = t; i < B; i += 256) scratch[i] = (int32_t)i;
  for (long i = t; i < NB; i += 256) scratch[B + i] = (int32_t)i;
  for (long i = t; i < A; i += 256) map[i] = -1;
  __syncthreads();
  uint64_t state = seed_ptr ? *seed_ptr : seed;  // a captured step reads the seed its host staged
  if (t == 0) {
    for (long i = 0; i < R; i++) {
      const long j = i + (long)splitmix_index(state, (uint64_t)(B - i));
      const int32_t old = scratch[i], value = scratch[j];
      scratch[i] = value;
      scratch[j] = old;
      columns[i] = value;
    }
  }
  for (long i = 0; i < S; i++) {
    if (t == 0) {
      const long j = i + (long)splitmix_index(state, (uint64_t)(NB - i));
      const int32_t old = scratch[B + i], value = scratch[B + j];
      scratch[B + i] = value;
      scratch[B + j] = old;
      picked = value;
    }
    __syncthreads();
    const long value = picked;
    for (long off = t; off < group; off += 256) {
      const long index = value * group + off, position = i * group + off;
      rows[position] = index < A ? (int32_t)index : -1;
      if (index < A) map[index] = (int32_t)position;
    }
    __syncthreads();
  }
}

// ------------------------------------------------------------------- basis
// The reference orthonormalises the picked donor columns with classical
// Gram-Schmidt applied twice in one workgroup (parameter.py:65-128).  Here:
// CholeskyQR2 -- G = V^T V in FP64 from partial sums over the whole chip, a
// one-wavefront Cholesky G = L L^T, Q = V L^-T applied row-parallel, and a
// second pass on Q.  The Cholesky pivot of column c is |v_c - its
// projection on the earlier columns|^2, the quantity CGS2 tests, so the same
// drop rule applies: a column whose pivot is <= eps^2 |v_c|^2 gets a zero
// column in L^-T (and so in Q) and is left out of the later projections.
// The factored gradient depends on Q only through the projector Q Q^T.
constexpr int RMAX = 64;
constexpr int GR = 64;      // rows staged per LDS chunk
constexpr int GBLK = 128;   // workgroups of the Gram pass

// partial Gram of rows: v[row][j] = source value; pass 1 gathers donor
// columns (dtype f32/bf16), pass 2 reads Q rows.  Pairs i <= j.
__global__ __launch_bounds__(256) void k_gram_partial(const void* __restrict__ y, int ydt, long ldy,
                                                      const int32_t* __restrict__ cols, const float* __restrict__ q,
                                                      long n, int R, double* __restrict__ partial) {
  __shared__ float sv[GR][RMAX + 1];
  const int t = threadIdx.x;
  const int P = R * (R + 1) / 2;
  double acc[9];
  int pi[9], pj[9];
#pragma unroll
  for (int u = 0; u < 9; u++) {
    acc[u] = 0.0;
    int p = t + 256 * u, i = 0;
    // pair p -> (i, j), i <= j, row-major over the upper triangle
    while (p >= R - i && i < R) {
      p -= R - i;
      i++;
    }
    pi[u] = i < R ? i : 0;
    pj[u] = i < R ? i + p : 0;
  }
  const long per = (n + gridDim.x - 1) / gridDim.x;
  const long r0 = blockIdx.x * per, r1 = r0 + per < n ? r0 + per : n;
  for (long c0 = r0; c0 < r1; c0 += GR) {
    __syncthreads();
    for (int q2 = t; q2 < GR * R; q2 += 256) {
      const int rr = q2 / R, j = q2 - rr * R;
      const long row = c0 + rr;
      float v = 0.f;
      if (row < r1) v = q ? q[row * R + j] : load_as_f32(y, ydt, row * ldy + cols[j]);
      sv[rr][j] = v;
    }
    __syncthreads();
#pragma unroll
    for (int u = 0; u < 9; u++) {
      if (t + 256 * u < P) {
        const float* ci = &sv[0][pi[u]];
        const float* cj = &sv[0][pj[u]];
        double a = 0.0;
        for (int rr = 0; rr < GR; rr++) a += (double)ci[rr * (RMAX + 1)] * (double)cj[rr * (RMAX + 1)];
        acc[u] += a;
      }
    }
  }
#pragma unroll
  for (int u = 0; u < 9; u++)
    if (t + 256 * u < P) partial[(long)blockIdx.x * P + t + 256 * u] = acc[u];
}

// one wavefront: G = sum of the partials (fixed order), Cholesky in place
// with the drop rule (pivot <= eps^2 * the column's |v|^2 -> dropped), and
// T = L^-T with zero columns for dropped ones: lane l owns row l of T
// (FP64 in t64, fp32 copy in tmat for the apply).
__global__ __launch_bounds__(256) void k_chol_inv(const double* __restrict__ partial, int nblk, int R, float eps,
                                                  double* __restrict__ part4, double* __restrict__ t64,
                                                  float* __restrict__ tmat) {
  __shared__ double G[RMAX][RMAX + 1];  // G; L in the lower triangle as it is formed
  __shared__ double dg[RMAX];
  __shared__ int keep[RMAX];
  const int l = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int P = R * (R + 1) / 2;
  // each wavefront sums a quarter of the blocks (part4 [4][P] in the
  // workspace), then the four are added in order
  for (int p = l; p < P; p += 64) {
    double sum = 0.0;
    for (int b = wv; b < nblk; b += 4) sum += partial[(long)b * P + p];
    part4[wv * P + p] = sum;
  }
  __syncthreads();
  for (int p = threadIdx.x; p < P; p += 256) {
    const double sum = ((part4[p] + part4[P + p]) + part4[2 * P + p]) + part4[3 * P + p];
    int i = 0, pp = p;
    while (pp >= R - i) {
      pp -= R - i;
      i++;
    }
    G[i][i + pp] = sum;
    G[i + pp][i] = sum;
  }
  __syncthreads();
  if (wv == 0 && l < R) dg[l] = G[l][l];
  __syncthreads();
  // the factorisation runs on wavefront 0; the others only keep the
  // barriers company
  const double e2 = (double)eps * (double)eps;
  for (int c = 0; c < R; c++) {
    double d = G[c][c];
    for (int k = 0; k < c; k++) d -= G[c][k] * G[c][k];
    const bool kp = d > e2 * dg[c] && d > 0.0;
    const double piv = kp ? sqrt(d) : 0.0;
    double v = 0.0;
    if (wv == 0 && l > c && l < R && kp) {
      v = G[l][c];
      for (int k = 0; k < c; k++) v -= G[l][k] * G[c][k];
      v /= piv;
    }
    __syncthreads();
    if (wv == 0 && l > c && l < R) G[l][c] = v;
    if (wv == 0 && l == c) {
      G[c][c] = piv;
      keep[c] = kp;
    }
    __syncthreads();
  }
  if (wv != 0) return;
  for (int j = 0; j < R; j++) {
    if (l < R) {
      double v = 0.0;
      if (keep[j]) {
        v = l == j ? 1.0 : 0.0;
        for (int k = 0; k < j; k++) v -= G[j][k] * t64[l * R + k];
        v /= G[j][j];
      }
      t64[l * R + j] = v;
      tmat[l * R + j] = (float)v;
    }
  }
}

// Q[row] = v[row] T (pass 1 from the donor columns, pass 2 in place)
__global__ __launch_bounds__(256) void k_basis_apply(const void* __restrict__ y, int ydt, long ldy,
                                                     const int32_t* __restrict__ cols, float* __restrict__ q, long n,
                                                     int R, const float* __restrict__ tmat, int from_q) {
  __shared__ float T[RMAX * RMAX];
  for (int p = threadIdx.x; p < R * R; p += 256) T[p] = tmat[p];
  __syncthreads();
  const long row = blockIdx.x * 256L + threadIdx.x;
  if (row >= n) return;
  float v[RMAX];
#pragma unroll
  for (int k = 0; k < RMAX; k++)
    if (k < R) v[k] = from_q ? q[row * R + k] : load_as_f32(y, ydt, row * ldy + cols[k]);
  for (int j = 0; j < R; j++) {
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < RMAX; k++)
      if (k < R) s += v[k] * T[k * R + j];
    q[row * R + j] = s;
  }
}

// ----------------------------------------------------------------- prepare
// E[0:R] = Q^T (fp32 and hi/lo planes; the planes double as the B operand
// of A = X^T Q).  Thread per (r, token).
__global__ __launch_bounds__(256) void k_pvjp_qt(const float* __restrict__ q, int R, long n, long n8,
                                                 float* __restrict__ e, bf16_t* __restrict__ eh, bf16_t* __restrict__ el,
                                                 long lde) {
  const long i = blockIdx.x * 256L + threadIdx.x;
  if (i >= (long)R * n8) return;
  const long r = i / n8, tok = i - r * n8;
  const float v = tok < n ? q[tok * R + r] : 0.f;  // columns [n, n8) are the GEMM's zero padding
  if (e) e[r * lde + tok] = v;
  bf16_t h, l;
  split_bf(v, h, l);
  eh[r * lde + tok] = h;
  el[r * lde + tok] = l;
}

// E[R+i][tok] = (X^T[row_i][tok] - sum_r Q[tok][r] A[row_i][r]) * inverse,
// zero for row_i = -1 (parameter.py:167-190); fp32 and planes.  Thread per
// token: its Q row is read once, the block's RROWS selected rows of A sit
// in LDS.  XROWS: X given in row layout, x [tok][ldxt] (else X^T [row][ldxt]).
// RB: a compile-time bound on the rank R (16, 32 or 64): the per-row sum
// runs over RB terms, the ones past R predicated off, in the same order
// whatever RB is.
constexpr int RROWS = 16;
template <bool XROWS, int RB>
__global__ __launch_bounds__(256) void k_pvjp_residual(const bf16_t* __restrict__ xt, long ldxt,
                                                       const float* __restrict__ q, int R, long n,
                                                       const float* __restrict__ left, const int32_t* __restrict__ rows,
                                                       long k, float inverse, float* __restrict__ e,
                                                       bf16_t* __restrict__ eh, bf16_t* __restrict__ el, long lde,
                                                       long n8) {
  __shared__ float sa[RROWS][RMAX];
  __shared__ long srow[RROWS];
  const long i0 = blockIdx.y * (long)RROWS;
  for (int p = threadIdx.x; p < RROWS * R; p += 256) {
    const int ii = p / R, r = p - ii * R;
    const long row = i0 + ii < k ? rows[i0 + ii] : -1;
    sa[ii][r] = row >= 0 ? left[row * R + r] : 0.f;
  }
  if (threadIdx.x < RROWS) srow[threadIdx.x] = i0 + threadIdx.x < k ? rows[i0 + threadIdx.x] : -1;
  __syncthreads();
  const long tok = blockIdx.x * 256L + threadIdx.x;
  if (tok >= n8) return;
  float qr[RB];
#pragma unroll
  for (int r = 0; r < RB; r++)
    if (r < R) qr[r] = tok < n ? q[tok * R + r] : 0.f;
  for (int ii = 0; ii < RROWS; ii++) {
    const long i = i0 + ii;
    if (i >= k) break;
    const long row = srow[ii];
    float v = 0.f;
    if (row >= 0 && tok < n) {
      float acc = 0.f;
#pragma unroll
      for (int r = 0; r < RB; r++)
        if (r < R) acc += qr[r] * sa[ii][r];
      v = (bf2f(xt[XROWS ? tok * ldxt + row : row * ldxt + tok]) - acc) * inverse;
    }
    const long o = (R + i) * lde + tok;
    if (e) e[o] = v;
    bf16_t h, l;
    split_bf(v, h, l);
    eh[o] = h;
    el[o] = l;
  }
}

template <bool XROWS>
void launch_residual(hipStream_t s, dim3 grid, const bf16_t* x, long ldx, const float* q, int R, long n,
                     const float* left, const int32_t* rows, long k, float inverse, float* e, bf16_t* eh,
                     bf16_t* el, long lde, long n8) {
  if (R <= 16)
    hipLaunchKernelGGL((k_pvjp_residual<XROWS, 16>), grid, dim3(256), 0, s, x, ldx, q, R, n, left, rows, k, inverse,
                       e, eh, el, lde, n8);
  else if (R <= 32)
    hipLaunchKernelGGL((k_pvjp_residual<XROWS, 32>), grid, dim3(256), 0, s, x, ldx, q, R, n, left, rows, k, inverse,
                       e, eh, el, lde, n8);
  else
    hipLaunchKernelGGL((k_pvjp_residual<XROWS, RMAX>), grid, dim3(256), 0, s, x, ldx, q, R, n, left, rows, k,
                       inverse, e, eh, el, lde, n8);
}

// ------------------------------------------------------------------- apply
// Device metadata of a factored update: parameters, then terms.
struct FParam {
  float* w;
  const float* dense;
  uint16_t* mirror;  // nullable bf16 copy of the updated w
  long rows, cols, ld, first_tile, col_tiles;
  int decay, term_begin, term_count, pad;
};
struct FTerm {
  const float* left;
  const float* right;
  const float* tail;
  const int32_t* row_map;
  long rank, ld;
  float scale;
  int pad;
};
struct FMetaHeader {
  long nparams, nterms, tiles, pad;
};
// metadata layout: header, params[nparams], terms[nterms], owners[tiles]
// (the parameter of each tile, as the reference's Owners table)

constexpr int FBM = 16;    // tile rows
constexpr int FBN = 1024;  // tile columns: 4 per thread
constexpr int FRMAX = 64;  // rank staged per LDS pass

// up to 4 floats at p[0..cnt), one 16-byte access when vec
__device__ __forceinline__ float4 ld4(const float* p, int cnt, bool vec) {
  if (vec && cnt == 4) return *(const float4*)p;
  float v[4] = {0.f, 0.f, 0.f, 0.f};
  for (int i = 0; i < cnt; i++) v[i] = p[i];
  return make_float4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ bool al16(const void* p) { return ((uintptr_t)p & 15) == 0; }

// parameter_gradient_update / _materialize / _norm (parameter.py:244-291):
// one workgroup per 16x1024 tile of one parameter (owner from the table).
// Action 0 materialize (G into w), 1 update, 2 FP64 sum of G^2 per tile.
__global__ __launch_bounds__(256) void k_factored_apply(const uint8_t* __restrict__ meta, int action, float lr,
                                                        float decay, double* __restrict__ partials,
                                                        const sj_sgd_step* __restrict__ step,
                                                        const double* __restrict__ sumsq) {
  const FMetaHeader* hd = (const FMetaHeader*)meta;
  const FParam* params = (const FParam*)(meta + sizeof(FMetaHeader));
  const FTerm* terms = (const FTerm*)(params + hd->nparams);
  const int32_t* owners = (const int32_t*)(terms + hd->nterms);
  __shared__ float sl[FBM][FRMAX + 1];  // (left * scale) rows of this tile
  const long tile = blockIdx.x;
  const FParam P = params[owners[tile]];
  const long local = tile - P.first_tile;
  const long m0 = (local / P.col_tiles) * FBM, n = (local % P.col_tiles) * FBN + 4 * threadIdx.x;
  const int cnt = n < P.cols ? (P.cols - n < 4 ? (int)(P.cols - n) : 4) : 0;
  const bool wvec = (P.cols & 3) == 0 && (P.ld & 3) == 0 && al16(P.w) && (!P.dense || al16(P.dense));
  float4 g[FBM];
#pragma unroll
  for (int i = 0; i < FBM; i++) g[i] = make_float4(0.f, 0.f, 0.f, 0.f);
  // head = sum over the terms' ranks of (left * scale) right
  for (int ti = 0; ti < P.term_count; ti++) {
    const FTerm tm = terms[P.term_begin + ti];
    const bool tvec = (tm.ld & 3) == 0 && al16(tm.right) && al16(tm.tail);
    for (long r0 = 0; r0 < tm.rank; r0 += FRMAX) {
      const long rn = tm.rank - r0 < FRMAX ? tm.rank - r0 : FRMAX;
      __syncthreads();
      for (long q = threadIdx.x; q < FBM * rn; q += 256) {
        const long i = q / rn, r = q - i * rn, m = m0 + i;
        sl[i][r] = m < P.rows ? tm.left[m * tm.rank + r0 + r] * tm.scale : 0.f;
      }
      __syncthreads();
      if (cnt > 0) {
        for (long r = 0; r < rn; r++) {
          const float4 rv = ld4(tm.right + (r0 + r) * tm.ld + n, cnt, tvec);
#pragma unroll
          for (int i = 0; i < FBM; i++) {
            const float a = sl[i][r];
            g[i].x += a * rv.x; g[i].y += a * rv.y; g[i].z += a * rv.z; g[i].w += a * rv.w;
          }
        }
      }
    }
  }
  // value = dense + head, then the tails
  if (cnt > 0) {
#pragma unroll
    for (int i = 0; i < FBM; i++) {
      const long m = m0 + i;
      if (P.dense && m < P.rows) {
        const float4 dv = ld4(P.dense + m * P.ld + n, cnt, wvec);
        g[i] = make_float4(dv.x + g[i].x, dv.y + g[i].y, dv.z + g[i].z, dv.w + g[i].w);
      }
    }
    for (int ti = 0; ti < P.term_count; ti++) {
      const FTerm tm = terms[P.term_begin + ti];
      const bool tvec = (tm.ld & 3) == 0 && al16(tm.right) && al16(tm.tail);
#pragma unroll
      for (int i = 0; i < FBM; i++) {
        const long m = m0 + i;
        if (m < P.rows) {
          const int sel = tm.row_map[m];
          if (sel >= 0) {
            const float4 tv = ld4(tm.tail + (long)sel * tm.ld + n, cnt, tvec);
            g[i].x += tv.x * tm.scale; g[i].y += tv.y * tm.scale;
            g[i].z += tv.z * tm.scale; g[i].w += tv.w * tm.scale;
          }
        }
      }
    }
  }
  if (action == 2) {
    double s = 0.0;
    if (cnt > 0) {
#pragma unroll
      for (int i = 0; i < FBM; i++) {
        if (m0 + i >= P.rows) continue;
        const float v[4] = {g[i].x, g[i].y, g[i].z, g[i].w};
        for (int c = 0; c < cnt; c++) s += (double)v[c] * (double)v[c];
      }
    }
    __shared__ double red[4];
    __syncthreads();
    s = wave_sum(s);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
    __syncthreads();
    if (threadIdx.x == 0) partials[tile] = ((red[0] + red[1]) + red[2]) + red[3];
    return;
  }
  if (cnt == 0) return;
  if (step) {
    // the step driver's update: learning rate from the staged step record,
    // clipping from the FP64 norm of this step (train lib.rs / control_
    // variate.rs: clipping = clip_norm / norm when enabled and norm >
    // clip_norm, formed in f64 and rounded to f32; LR = lr * clipping and
    // DECAY = lr * weight_decay in f32, parameter_vjp.rs:502-518)
    float clip = 1.f;
    if (step->clip_enabled && sumsq) {
      const double nrm = sqrt(fmax(*sumsq, 0.0));
      if (nrm > (double)step->clip_norm) clip = (float)((double)step->clip_norm / nrm);
    }
    lr = mul_rn(step->lr, clip);
    decay = mul_rn(step->lr, step->weight_decay);
  }
  const float keep = (P.decay && action == 1) ? 1.f - decay : 1.f;
#pragma unroll
  for (int i = 0; i < FBM; i++) {
    const long m = m0 + i;
    if (m >= P.rows) continue;
    float* wp = P.w + m * P.ld + n;
    float4 o = g[i];
    if (action == 1) {
      const float4 w4 = ld4(wp, cnt, wvec);
      o = make_float4(w4.x * keep - lr * g[i].x, w4.y * keep - lr * g[i].y, w4.z * keep - lr * g[i].z,
                      w4.w * keep - lr * g[i].w);
    }
    if (wvec && cnt == 4) {
      *(float4*)wp = o;
    } else {
      const float v[4] = {o.x, o.y, o.z, o.w};
      for (int c = 0; c < cnt; c++) wp[c] = v[c];
    }
    if (action == 1 && P.mirror) {
      bf16_t* mp = (bf16_t*)P.mirror + m * P.ld + n;
      if (wvec && cnt == 4) {
        *(u32x2*)mp = u32x2{pack2(f2bf(o.x), f2bf(o.y)), pack2(f2bf(o.z), f2bf(o.w))};
      } else {
        const float v[4] = {o.x, o.y, o.z, o.w};
        for (int c = 0; c < cnt; c++) mp[c] = f2bf(v[c]);
      }
    }
  }
}

// fixed-order FP64 sum of the per-tile partials (one workgroup)
__global__ __launch_bounds__(256) void k_sum_f64(const double* __restrict__ x, long n, double* __restrict__ out) {
  __shared__ double red[4];
  double s = 0.0;
  for (long i = threadIdx.x; i < n; i += 256) s += x[i];
  s = wave_sum(s);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) *out = ((red[0] + red[1]) + red[2]) + red[3];
}

}  // namespace

// ================================================================ C ABI

extern "C" int sj_pvjp_budget(long rank, double residual_fraction, long block_rows, long n, long a, long donor,
                              long* out_rank, long* out_blocks, long* out_selected) {
  SJ_REQUIRE(rank > 0 && block_rows > 0 && residual_fraction > 0.0 && residual_fraction <= 1.0 && n > 0 && a > 0 &&
                 donor > 0,
             "parameter VJP requires positive rank/block_rows and residual_fraction in (0,1]");
  long r = rank < n ? rank : n;
  r = r < a ? r : a;
  r = r < donor ? r : donor;
  const long blocks = (a + block_rows - 1) / block_rows;
  long sel = (long)ceil((double)blocks * residual_fraction);
  sel = sel < blocks ? sel : blocks;
  sel = sel > 1 ? sel : 1;
  if (out_rank) *out_rank = r;
  if (out_blocks) *out_blocks = blocks;
  if (out_selected) *out_selected = sel;
  return SJ_OK;
}

namespace {
typedef unsigned __int128 u128;
u128 issued(long m, long n, long k) {
  auto up = [](long v, long t) { return (u128)((v + t - 1) / t) * (u128)t; };
  return 2 * up(m, 16) * up(n, 32) * up(k, 32);
}
u128 pow2(long v) {
  u128 p = 1;
  while (p < (u128)v) p <<= 1;
  return p;
}
}  // namespace

extern "C" int sj_pvjp_selects_compression(long rank, double residual_fraction, long block_rows, long n, long a,
                                           long b, long donor, long uses) {
  if (n < a || uses <= 1) return 0;
  long r = 0, blocks = 0, sel = 0;
  if (sj_pvjp_budget(rank, residual_fraction, block_rows, n, a, donor, &r, &blocks, &sel)) return 0;
  if (sel == blocks) return 0;
  const long k = sel * block_rows;
  const u128 padded = (u128)((n + 15) / 16) * 16;
  const u128 last = r > 0 ? (u128)(r - 1) : 0;
  const u128 full = last / 32, tail = last % 32;
  const u128 tri = 32 * full * (full + 1) / 2 + tail * (full + 1);
  const u128 streaming = 2 * (4 * padded * 32 + padded) * tri + 5 * padded * (u128)r;
  const u128 resident = 8 * pow2(n) * pow2(r) * (u128)r + 5 * pow2(n) * (u128)r;
  const u128 qr = streaming > resident ? streaming : resident;
  const u128 shared = qr + issued(a, r, n) + issued(k, n, r);
  const u128 own = issued(r + k, b, n) + issued(a, b, r);
  return own * (u128)uses + shared < issued(a, b, n) * (u128)uses ? 1 : 0;
}

extern "C" float sj_pvjp_basis_tolerance(long rows, long rank) {
  const double ops = (double)rows * (4.0 * (double)rank + 1.0);
  const double roundoff = ops * (1.1920928955078125e-7 / 2.0);
  const double tol = roundoff < 1.0 ? roundoff / (1.0 - roundoff) : INFINITY;
  return (float)(tol < 3.4028234663852886e38 ? tol : 3.4028234663852886e38);
}

extern "C" int sj_pvjp_indices(void* stream, uint64_t seed, long a, long donor_width, long feature_blocks,
                               long selected, long rank, long block_rows, int32_t* scratch, int32_t* columns,
                               int32_t* rows, int32_t* map) {
  SJ_REQUIRE(a >= 0 && donor_width >= 0 && feature_blocks >= 0 && selected >= 0 && rank >= 0 && block_rows > 0 &&
                 rank <= donor_width && selected <= feature_blocks && donor_width + feature_blocks < (1L << 31) &&
                 scratch && (rank == 0 || columns) && (selected == 0 || (rows && map)),
             "parameter_indices: dimensions");
  hipLaunchKernelGGL(k_pvjp_indices, dim3(1), dim3(256), 0, (hipStream_t)stream, scratch, columns, rows, map, a,
                     donor_width, feature_blocks, selected, rank, block_rows, seed, (const uint64_t*)nullptr);
  SJ_LAUNCH_CHECK("parameter_indices");
  return SJ_OK;
}

int sjh::pvjp_indices_dev(hipStream_t stream, const uint64_t* seed, long a, long donor_width, long feature_blocks,
                          long selected, long rank, long block_rows, int32_t* scratch, int32_t* columns,
                          int32_t* rows, int32_t* map) {
  SJ_REQUIRE(seed && a >= 0 && donor_width >= 0 && feature_blocks >= 0 && selected >= 0 && rank >= 0 &&
                 block_rows > 0 && rank <= donor_width && selected <= feature_blocks &&
                 donor_width + feature_blocks < (1L << 31) && scratch && (rank == 0 || columns) &&
                 (selected == 0 || (rows && map)),
             "parameter_indices: dimensions");
  hipLaunchKernelGGL(k_pvjp_indices, dim3(1), dim3(256), 0, stream, scratch, columns, rows, map, a, donor_width,
                     feature_blocks, selected, rank, block_rows, (uint64_t)0, seed);
  SJ_LAUNCH_CHECK("parameter_indices");
  return SJ_OK;
}

extern "C" size_t sj_pvjp_basis_workspace_bytes(long n, long rank) {
  (void)n;
  return sizeof(double) * (size_t)(GBLK + 4) * (size_t)(rank * (rank + 1) / 2) +
         (sizeof(double) + sizeof(float)) * (size_t)(rank * rank);
}

extern "C" int sj_pvjp_basis(void* stream, const void* y, int dtype, long ldy, long n, const int32_t* columns,
                             long rank, float eps, float* q, void* workspace, size_t workspace_bytes) {
  SJ_REQUIRE(n > 0 && rank > 0 && rank <= RMAX && (dtype == SJ_F32 || dtype == SJ_BF16),
             "parameter_basis: rank %ld (<= %d)", rank, RMAX);
  const size_t need = sj_pvjp_basis_workspace_bytes(n, rank);
  if (!workspace || workspace_bytes < need)
    return sjh::fail(SJ_ERR_CAPACITY, "parameter_basis: required %zu bytes, available %zu bytes", need,
                     workspace_bytes);
  hipStream_t s = (hipStream_t)stream;
  double* partial = (double*)workspace;
  double* part4 = partial + (size_t)GBLK * (size_t)(rank * (rank + 1) / 2);
  double* t64 = part4 + 4 * (size_t)(rank * (rank + 1) / 2);
  float* tmat = (float*)(t64 + rank * rank);
  const int R = (int)rank;
  const unsigned rows_blocks = (unsigned)((n + 255) / 256);
  for (int pass = 0; pass < 2; pass++) {
    hipLaunchKernelGGL(k_gram_partial, dim3(GBLK), dim3(256), 0, s, y, dtype, ldy, columns, pass ? q : nullptr, n, R,
                       partial);
    hipLaunchKernelGGL(k_chol_inv, dim3(1), dim3(256), 0, s, (const double*)partial, GBLK, R, eps, part4, t64, tmat);
    hipLaunchKernelGGL(k_basis_apply, dim3(rows_blocks), dim3(256), 0, s, y, dtype, ldy, columns, q, n, R,
                       (const float*)tmat, pass);
  }
  SJ_LAUNCH_CHECK("parameter_basis");
  return SJ_OK;
}

extern "C" size_t sj_pvjp_prepare_workspace_bytes(long a, long n, long rank) {
  return sj_gemm_planes_workspace_bytes(a, rank, (n + 7) / 8 * 8);
}

extern "C" int sj_pvjp_prepare(void* stream, const uint16_t* x_t, long ldxt, long a, long n, const float* q, long rank,
                               const int32_t* rows, long k, float inverse, float* left, float* e, uint16_t* e_hi,
                               uint16_t* e_lo, long lde, void* workspace, size_t workspace_bytes) {
  const long n8 = (n + 7) / 8 * 8;
  SJ_REQUIRE(a > 0 && n > 0 && rank > 0 && rank <= RMAX && k >= 0 && ldxt >= n8 && ldxt % 8 == 0 && lde >= n8 &&
                 lde % 8 == 0 &&
                 ((uintptr_t)e_hi & 15) == 0 && ((uintptr_t)e_lo & 15) == 0 && ((uintptr_t)x_t & 15) == 0,
             "parameter_prepare: dimensions (rank <= 64, leading dimensions multiples of 8, >= n rounded up to 8)");
  hipStream_t s = (hipStream_t)stream;
  const long qn = rank * n8;
  hipLaunchKernelGGL(k_pvjp_qt, dim3((unsigned)((qn + 255) / 256)), dim3(256), 0, s, q, (int)rank, n, n8, e,
                     (bf16_t*)e_hi, (bf16_t*)e_lo, lde);
  SJ_LAUNCH_CHECK("parameter_prepare");
  // A = X^T Q: A operand X^T [a][n8] bf16 (zero columns past n), B operand
  // Q^T planes = E[0:R]
  if (int st = sj_gemm_planes(stream, a, rank, n8, x_t, nullptr, ldxt, e_hi, e_lo, lde, left, SJ_F32, rank, 0,
                              workspace, workspace_bytes))
    return st;
  if (k > 0) {
    launch_residual<false>(s, dim3((unsigned)((n8 + 255) / 256), (unsigned)((k + RROWS - 1) / RROWS)),
                           (const bf16_t*)x_t, ldxt, q, (int)rank, n, left, rows, k, inverse, e, (bf16_t*)e_hi,
                           (bf16_t*)e_lo, lde, n8);
    SJ_LAUNCH_CHECK("parameter_residual");
  }
  return SJ_OK;
}

// sj_pvjp_prepare with X in row layout (x [n][ldx], the stored activation
// itself): left = X^T Q on the row-layout product, the residual rows read
// X[tok][row].  n % 8 == 0 (the token rows are the products' K).
extern "C" int sj_pvjp_prepare_rows(void* stream, const uint16_t* x, long ldx, long a, long n, const float* q,
                                    long rank, const int32_t* rows, long k, float inverse, float* left, float* e,
                                    uint16_t* e_hi, uint16_t* e_lo, long lde, void* workspace,
                                    size_t workspace_bytes) {
  SJ_REQUIRE(a > 0 && n > 0 && n % 8 == 0 && a % 8 == 0 && rank > 0 && rank <= RMAX && k >= 0 && ldx >= a &&
                 ldx % 8 == 0 &&
                 lde >= n && lde % 8 == 0 && ((uintptr_t)e_hi & 15) == 0 && ((uintptr_t)e_lo & 15) == 0 &&
                 ((uintptr_t)x & 15) == 0,
             "parameter_prepare (row-layout X): a %ld n %ld ldx %ld lde %ld (rank <= 64; a, n and leading "
             "dimensions multiples of 8)", a, n, ldx, lde);
  hipStream_t s = (hipStream_t)stream;
  const long qn = rank * n;
  hipLaunchKernelGGL(k_pvjp_qt, dim3((unsigned)((qn + 255) / 256)), dim3(256), 0, s, q, (int)rank, n, n, e,
                     (bf16_t*)e_hi, (bf16_t*)e_lo, lde);
  SJ_LAUNCH_CHECK("parameter_prepare");
  if (int st = sjh::gemm_planes_rows_a(stream, a, rank, n, x, ldx, e_hi, e_lo, lde, left, rank, workspace,
                                       workspace_bytes))
    return st;
  if (k > 0) {
    launch_residual<true>(s, dim3((unsigned)((n + 255) / 256), (unsigned)((k + RROWS - 1) / RROWS)),
                          (const bf16_t*)x, ldx, q, (int)rank, n, left, rows, k, inverse, e, (bf16_t*)e_hi,
                          (bf16_t*)e_lo, lde, n);
    SJ_LAUNCH_CHECK("parameter_residual");
  }
  return SJ_OK;
}

extern "C" size_t sj_pvjp_vjp_workspace_bytes(long rows, long b, long n) {
  return sj_gemm_planes_workspace_bytes(rows, b, (n + 7) / 8 * 8);
}

extern "C" int sj_pvjp_vjp(void* stream, const uint16_t* e_hi, const uint16_t* e_lo, long lde, long rows, long n,
                           const uint16_t* dy_t_hi, const uint16_t* dy_t_lo, long lddy, long b, float* coefficients,
                           long ldc, void* workspace, size_t workspace_bytes) {
  const long n8 = (n + 7) / 8 * 8;
  SJ_REQUIRE(rows > 0 && n > 0 && b > 0 && ldc >= b && lde >= n8 && lddy >= n8,
             "parameter_vjp: dimensions (leading dimensions >= n rounded up to 8, zero padded)");
  return sj_gemm_planes(stream, rows, b, n8, e_hi, e_lo, lde, dy_t_hi, dy_t_lo, lddy, coefficients, SJ_F32, ldc, 0,
                        workspace, workspace_bytes);
}

// sj_pvjp_vjp with dY in row layout (planes [n][lddy], the dX chain's own
// gradient planes): coefficients = E dY on the row-layout product.
// n % 8 == 0.
extern "C" int sj_pvjp_vjp_rows(void* stream, const uint16_t* e_hi, const uint16_t* e_lo, long lde, long rows, long n,
                                const uint16_t* dy_hi, const uint16_t* dy_lo, long lddy, long b, float* coefficients,
                                long ldc, void* workspace, size_t workspace_bytes) {
  SJ_REQUIRE(rows > 0 && n > 0 && n % 8 == 0 && b > 0 && b % 8 == 0 && ldc >= b && lde >= n && lddy >= b,
             "parameter_vjp (row-layout dY): rows %ld n %ld b %ld (n and b multiples of 8)", rows, n, b);
  return sjh::gemm_planes_rows_b(stream, rows, b, n, e_hi, e_lo, lde, dy_hi, dy_lo, lddy, coefficients, ldc,
                                 workspace, workspace_bytes);
}

// tiles of a parameter list (the owners table's length)
static long factored_tiles(const sj_factored_param* params, long nparams) {
  long t = 0;
  for (long i = 0; i < nparams; i++)
    t += ((params[i].rows + FBM - 1) / FBM) * ((params[i].cols + FBN - 1) / FBN);
  return t;
}

extern "C" size_t sj_factored_meta_bytes(const sj_factored_param* params, long nparams, long nterms) {
  if (!params || nparams <= 0 || nterms < 0) return 0;
  return sizeof(FMetaHeader) + sizeof(FParam) * (size_t)nparams + sizeof(FTerm) * (size_t)nterms +
         sizeof(int32_t) * (size_t)factored_tiles(params, nparams);
}

extern "C" int sj_factored_pack(const sj_factored_param* params, long nparams, const sj_factored_term* terms,
                                long nterms, void* host_meta, size_t bytes, long* tiles) {
  SJ_REQUIRE(params && nparams > 0 && nterms >= 0 && (nterms == 0 || terms) && host_meta &&
                 bytes >= sj_factored_meta_bytes(params, nparams, nterms) &&
                 factored_tiles(params, nparams) < (1L << 31),
             "gradient plan requires parameters and a metadata buffer of %zu bytes",
             sj_factored_meta_bytes(params, nparams, nterms));
  uint8_t* out = (uint8_t*)host_meta;
  FMetaHeader hd = {nparams, nterms, 0, 0};
  FParam* fp = (FParam*)(out + sizeof(FMetaHeader));
  FTerm* ft = (FTerm*)(fp + nparams);
  long t = 0;
  for (long i = 0; i < nparams; i++) {
    const sj_factored_param& p = params[i];
    SJ_REQUIRE(p.w && p.rows > 0 && p.cols > 0 && p.term_begin >= 0 && p.term_count >= 0 &&
                   p.term_begin + p.term_count <= nterms,
               "compact SGD parameter %ld: shape or terms", i);
    FParam q = {};
    SJ_REQUIRE(p.ld == 0 || p.ld >= p.cols, "compact SGD parameter %ld: row stride %ld below %ld columns", i, p.ld,
               p.cols);
    q.w = p.w; q.dense = p.dense; q.mirror = p.mirror; q.rows = p.rows; q.cols = p.cols;
    q.ld = p.ld > 0 ? p.ld : p.cols;
    q.first_tile = t; q.col_tiles = (p.cols + FBN - 1) / FBN;
    q.decay = p.decay; q.term_begin = (int)p.term_begin; q.term_count = (int)p.term_count;
    t += ((p.rows + FBM - 1) / FBM) * q.col_tiles;
    memcpy(fp + i, &q, sizeof(q));
  }
  for (long i = 0; i < nterms; i++) {
    const sj_factored_term& s = terms[i];
    SJ_REQUIRE(s.left && s.right && s.tail && s.row_map && s.rank >= 0, "compact SGD term %ld", i);
    FTerm q = {};
    q.left = s.left; q.right = s.right; q.tail = s.tail; q.row_map = s.row_map; q.rank = s.rank; q.scale = s.scale;
    q.ld = s.ld;
    memcpy(ft + i, &q, sizeof(q));
  }
  // a term's ld defaults to the columns of the parameter that uses it
  for (long i = 0; i < nparams; i++)
    for (long j = params[i].term_begin; j < params[i].term_begin + params[i].term_count; j++) {
      FTerm* q = ft + j;
      if (q->ld <= 0) q->ld = params[i].cols;
      SJ_REQUIRE(q->ld >= params[i].cols, "compact SGD term %ld: row stride %ld below %ld columns", j, q->ld,
                 params[i].cols);
    }
  hd.tiles = t;
  memcpy(out, &hd, sizeof(hd));
  int32_t* own = (int32_t*)(ft + nterms);
  for (long i = 0; i < nparams; i++) {
    const long first = ((const FParam*)(fp + i))->first_tile;
    const long count = ((params[i].rows + FBM - 1) / FBM) * ((params[i].cols + FBN - 1) / FBN);
    for (long j = 0; j < count; j++) own[first + j] = (int32_t)i;
  }
  if (tiles) *tiles = t;
  return SJ_OK;
}

extern "C" int sj_factored_apply(void* stream, const void* meta, long tiles, int action, float lr, float decay,
                                 double* partials) {
  SJ_REQUIRE(meta && tiles > 0 && tiles < (1L << 31) && action >= 0 && action <= 2 && (action != 2 || partials),
             "compact SGD apply: action %d", action);
  hipLaunchKernelGGL(k_factored_apply, dim3((unsigned)tiles), dim3(256), 0, (hipStream_t)stream,
                     (const uint8_t*)meta, action, lr, decay, partials, (const sj_sgd_step*)nullptr,
                     (const double*)nullptr);
  SJ_LAUNCH_CHECK(action == 1 ? "parameter_gradient_update"
                              : action == 0 ? "parameter_gradient_materialize" : "parameter_gradient_norm");
  return SJ_OK;
}

int sjh::factored_update_staged(hipStream_t stream, const void* meta, long tiles, const sj_sgd_step* step,
                                const double* sumsq) {
  SJ_REQUIRE(meta && step && tiles > 0 && tiles < (1L << 31), "compact SGD update: arguments");
  hipLaunchKernelGGL(k_factored_apply, dim3((unsigned)tiles), dim3(256), 0, stream, (const uint8_t*)meta, 1, 0.f,
                     0.f, (double*)nullptr, step, sumsq);
  SJ_LAUNCH_CHECK("parameter_gradient_update");
  return SJ_OK;
}

extern "C" int sj_sum_f64(void* stream, const double* x, long n, double* out) {
  SJ_REQUIRE(x && out && n >= 0, "sum: arguments");
  hipLaunchKernelGGL(k_sum_f64, dim3(1), dim3(256), 0, (hipStream_t)stream, x, n, out);
  SJ_LAUNCH_CHECK("sum");
  return SJ_OK;
}
