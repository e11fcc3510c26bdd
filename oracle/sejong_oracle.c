/*
 * sejong_oracle.c -- FP64 CPU restatement of Sejong's byte-Transformer
 * training step.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker for the HIP product
 * path in sejong_amd/csrc.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it.  Nothing in the product links
 * against it or falls back to it.
 *
 * Every function restates one reference formula; the citation above each
 * function names the reference file:line it follows (paths relative to the
 * Miyamoto-Renya/Sejong checkout).  All arithmetic is double precision.
 * Storage rounding (the dtype a reference kernel stores its output in) is
 * applied explicitly by the model-level driver through or_round(), so the
 * oracle consumes the same rounded operands the device stores.
 *
 * Pinning (what checks each function; see tests/test_oracle.py):
 *   or_rng_*            SplitMix64 published constants + known first outputs
 *                       of seed 0 / seed 42, index() rejection threshold.
 *   or_round            exhaustive bf16 / f32 RNE properties vs numpy.
 *   or_matmul           numpy matmul on random input (all TA/TB combinations).
 *   or_rmsnorm_*        closed form; finite-difference VJP on tiny shapes.
 *   or_rope             norm preservation; forward∘inverse = identity; angle
 *                       closed form at pos 1 / pair 0.
 *   or_attention_*      reference FP64 check (gpu/examples/hierarchy_check.rs
 *                       :16-77) on its closed-form values(); GQA = MHA with
 *                       repeated K/V heads; window=0 vs window>=T; FD VJP.
 *   or_swiglu_*         closed form; FD derivative.
 *   or_cross_entropy    log-sum-exp closed form; gradient sums to zero; FD.
 *   or_adamw            two-step closed form (train/examples/system_check.rs
 *                       :135-163).
 *   or_route_*          closed-form router test (gpu/examples/
 *                       hierarchy_check.rs:164-252).
 *   or_model_*          FD directional derivative of the whole model loss
 *                       (train/examples/system_check.rs:53-107) in fp32
 *                       storage mode, batch separation, causal prefix
 *                       invariance.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define OR_VOCAB 257

/* ------------------------------------------------------------------ RNG */

/* Rng::next_u64, crates/sejong-core/src/lib.rs:600-606 (SplitMix64). */
uint64_t or_rng_next(uint64_t *state) {
    *state += 0x9e3779b97f4a7c15ULL;
    uint64_t z = *state;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
    return z ^ (z >> 31);
}

/* Rng::index, crates/sejong-core/src/lib.rs:610-619: rejection below
 * threshold = (2^64 - n) mod n. */
uint64_t or_rng_index(uint64_t *state, uint64_t n) {
    uint64_t threshold = (0 - n) % n;
    for (;;) {
        uint64_t x = or_rng_next(state);
        if (x >= threshold) return x % n;
    }
}

/* Rng::uniform, crates/sejong-core/src/lib.rs:607-609 (returned here in
 * double before the f32 cast the reference applies). */
double or_rng_uniform(uint64_t *state) {
    return ((double)(or_rng_next(state) >> 40) + 0.5) / 16777216.0;
}

/* Box-Muller normal in double (weights N(0, std) for the BASELINE configs;
 * the reference's f32 variant is lib.rs:620-622).  Fills n values. */
void or_rng_normal_fill(uint64_t *state, double *out, long n, double std) {
    for (long i = 0; i < n; i++) {
        double u1 = or_rng_uniform(state);
        double u2 = or_rng_uniform(state);
        out[i] = std * sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
    }
}

/* ------------------------------------------------------------ rounding */

static double round_bf16(double x) {
    if (x == 0.0 || !isfinite(x)) return x;
    int e;
    frexp(x, &e); /* |x| in [2^(e-1), 2^e) */
    int qe = (e > -125 ? e : -125) - 8;
    double q = ldexp(1.0, qe);
    double r = nearbyint(x / q) * q;
    if (fabs(r) > 3.3895313892515355e38) r = copysign(INFINITY, x);
    return r;
}

/* Storage rounding: dtype 0 = f32, 4 = bf16 (sj_dtype numbering), other =
 * none.  Models the store of a reference kernel into its output dtype. */
void or_round(double *x, long n, int dtype) {
    if (dtype == 0) {
        for (long i = 0; i < n; i++) x[i] = (double)(float)x[i];
    } else if (dtype == 4) {
        for (long i = 0; i < n; i++) x[i] = round_bf16(x[i]);
    }
}

/* -------------------------------------------------------------- matmul */

/* Engine::matmul / kernel `matmul`, python/sejong_kernels/ops/kernels.py:23-39:
 * C[M,N] = op(A)[M,K] op(B)[K,N]; TA: A stored [K,M]; TB: B stored [N,K]. */
void or_matmul(const double *A, const double *B, double *C, long M, long N,
               long K, int ta, int tb) {
    double *bt = (double *)malloc(sizeof(double) * (size_t)N * (size_t)K);
    /* bt[n*K + k] = B[k, n] */
    for (long k = 0; k < K; k++)
        for (long n = 0; n < N; n++)
            bt[n * K + k] = tb ? B[n * K + k] : B[k * N + n];
#pragma omp parallel
    {
        double *arow = (double *)malloc(sizeof(double) * (size_t)K);
#pragma omp for schedule(static)
        for (long m = 0; m < M; m++) {
            for (long k = 0; k < K; k++) arow[k] = ta ? A[k * M + m] : A[m * K + k];
            for (long n = 0; n < N; n++) {
                const double *b = bt + n * K;
                double s = 0.0;
                for (long k = 0; k < K; k++) s += arow[k] * b[k];
                C[m * N + n] = s;
            }
        }
        free(arow);
    }
    free(bt);
}

/* ------------------------------------------------------------- RMSNorm */

/* kernel `rmsnorm`, kernels.py:54-61: y = x * (1/sqrt(mean(x^2)+eps)) * w. */
void or_rmsnorm_fwd(const double *x, const double *w, double *y, long R, long D,
                    double eps) {
#pragma omp parallel for schedule(static)
    for (long r = 0; r < R; r++) {
        const double *xr = x + r * D;
        double s = 0.0;
        for (long j = 0; j < D; j++) s += xr[j] * xr[j];
        double inv = 1.0 / sqrt(s / (double)D + eps);
        for (long j = 0; j < D; j++) y[r * D + j] = xr[j] * inv * w[j];
    }
}

/* kernels `rmsnorm_backward_partial` + `rmsnorm_backward_reduce`,
 * kernels.py:63-87, driven by Engine::norm_backward norm_ops.rs:14-71:
 *   s = rsqrt(mean x^2 + eps), d = dy*w,
 *   dx = s*(d - x*(sum(d*x)/D)*s^2),  dw = sum_rows dy*x*s.
 * dx_acc (nullable) is added to dx: the tape's accumulate() of the residual
 * branch gradient, graph.rs:503-513. */
void or_rmsnorm_bwd(const double *x, const double *w, const double *dy,
                    const double *dx_acc, double *dx, double *dw, long R,
                    long D, double eps) {
    double *inv = (double *)malloc(sizeof(double) * (size_t)R);
#pragma omp parallel for schedule(static)
    for (long r = 0; r < R; r++) {
        const double *xr = x + r * D, *gr = dy + r * D;
        double s = 0.0, dxs = 0.0;
        for (long j = 0; j < D; j++) s += xr[j] * xr[j];
        double iv = 1.0 / sqrt(s / (double)D + eps);
        inv[r] = iv;
        for (long j = 0; j < D; j++) dxs += gr[j] * w[j] * xr[j];
        double c = dxs / (double)D * iv * iv;
        for (long j = 0; j < D; j++) {
            double v = iv * (gr[j] * w[j] - xr[j] * c);
            dx[r * D + j] = (dx_acc ? dx_acc[r * D + j] : 0.0) + v;
        }
    }
    for (long j = 0; j < D; j++) dw[j] = 0.0;
    for (long r = 0; r < R; r++)
        for (long j = 0; j < D; j++) dw[j] += dy[r * D + j] * x[r * D + j] * inv[r];
    free(inv);
}

/* ---------------------------------------------------------------- RoPE */

/* kernel `rope`, kernels.py:103-113: interleaved pairs (2i, 2i+1) of each
 * head, pos = (row / H) mod T + offset, angle = pos * theta^(-2i/D);
 * inverse negates the sine (graph.rs:879-882). x is [rows, H*D]. */
void or_rope(const double *x, double *y, long rows, long T, long H, long D,
             long offset, double theta, int inverse) {
#pragma omp parallel for schedule(static)
    for (long r = 0; r < rows; r++) {
        double pos = (double)(r % T + offset);
        for (long h = 0; h < H; h++) {
            for (long i = 0; i < D / 2; i++) {
                double angle = pos * exp((-2.0 * (double)i / (double)D) * log(theta));
                double c = cos(angle), s = sin(angle);
                if (inverse) s = -s;
                long base = (r * H + h) * D + 2 * i;
                double a = x[base], b = x[base + 1];
                y[base] = a * c - b * s;
                y[base + 1] = a * s + b * c;
            }
        }
    }
}

/* ----------------------------------------------------------- Attention */

/* GQA causal attention forward, python/sejong_kernels/ops/hierarchy.py:7-39
 * (the FP64 form of the reference check gpu/examples/hierarchy_check.rs:16-77).
 * q [B*T, HQ*D], k/v [B*T, HK*D]; kv head = h / (HQ/HK); scale D^-1/2;
 * window 0 = full causal, else keys in (pos-window, pos].  lse [B*T*HQ]. */
void or_attention_fwd(const double *q, const double *k, const double *v,
                      double *o, double *lse, long B, long T, long HQ, long HK,
                      long D, long window) {
    double scale = 1.0 / sqrt((double)D);
#pragma omp parallel
    {
        double *sc = (double *)malloc(sizeof(double) * (size_t)T);
#pragma omp for collapse(2) schedule(dynamic)
        for (long b = 0; b < B; b++) {
            for (long pos = 0; pos < T; pos++) {
                for (long h = 0; h < HQ; h++) {
                    long kvh = h / (HQ / HK);
                    const double *qr = q + ((b * T + pos) * HQ + h) * D;
                    long first = window > 0 ? (pos + 1 - window > 0 ? pos + 1 - window : 0) : 0;
                    double m = -INFINITY;
                    for (long p = first; p <= pos; p++) {
                        const double *kr = k + ((b * T + p) * HK + kvh) * D;
                        double s = 0.0;
                        for (long j = 0; j < D; j++) s += qr[j] * kr[j];
                        s *= scale;
                        sc[p] = s;
                        if (s > m) m = s;
                    }
                    double z = 0.0;
                    for (long p = first; p <= pos; p++) z += exp(sc[p] - m);
                    double *orow = o + ((b * T + pos) * HQ + h) * D;
                    for (long j = 0; j < D; j++) orow[j] = 0.0;
                    for (long p = first; p <= pos; p++) {
                        double pr = exp(sc[p] - m) / z;
                        const double *vr = v + ((b * T + p) * HK + kvh) * D;
                        for (long j = 0; j < D; j++) orow[j] += pr * vr[j];
                    }
                    lse[(b * T + pos) * HQ + h] = m + log(z);
                }
            }
        }
        free(sc);
    }
}

/* GQA attention backward: hierarchy_attention_dq (writes Delta = sum dO*O)
 * and hierarchy_attention_dkv (reads Delta), hierarchy.py:42-104.
 *   P = exp(s - lse), dS = P*(dO.V - Delta)*scale,
 *   dQ = sum dS K, dK = sum dS Q, dV = sum P dO.
 * o and lse are the stored forward outputs (the reference conditions on
 * them).  delta (nullable) receives Delta [B*T*HQ]. */
void or_attention_bwd(const double *q, const double *k, const double *v,
                      const double *o, const double *lse, const double *dout,
                      double *dq, double *dk, double *dv, double *delta, long B,
                      long T, long HQ, long HK, long D, long window) {
    double scale = 1.0 / sqrt((double)D);
    long nq = B * T * HQ * D, nk = B * T * HK * D;
    memset(dq, 0, sizeof(double) * (size_t)nq);
    memset(dk, 0, sizeof(double) * (size_t)nk);
    memset(dv, 0, sizeof(double) * (size_t)nk);
    /* parallel over (batch, kv head) so that dk/dv rows are owned by one
     * thread; query heads of the group are walked inside. */
#pragma omp parallel for collapse(2) schedule(dynamic)
    for (long b = 0; b < B; b++) {
        for (long kvh = 0; kvh < HK; kvh++) {
            long group = HQ / HK;
            for (long g = 0; g < group; g++) {
                long h = kvh * group + g;
                for (long pos = 0; pos < T; pos++) {
                    long row = (b * T + pos) * HQ + h;
                    const double *qr = q + row * D, *dor = dout + row * D, *orow = o + row * D;
                    double dl = 0.0;
                    for (long j = 0; j < D; j++) dl += dor[j] * orow[j];
                    if (delta) delta[row] = dl;
                    double l = lse[row];
                    long first = window > 0 ? (pos + 1 - window > 0 ? pos + 1 - window : 0) : 0;
                    double *dqr = dq + row * D;
                    for (long p = first; p <= pos; p++) {
                        long kr = ((b * T + p) * HK + kvh) * D;
                        double s = 0.0, dp = 0.0;
                        for (long j = 0; j < D; j++) {
                            s += qr[j] * k[kr + j];
                            dp += dor[j] * v[kr + j];
                        }
                        double pr = exp(s * scale - l);
                        double ds = pr * (dp - dl) * scale;
                        for (long j = 0; j < D; j++) {
                            dqr[j] += ds * k[kr + j];
                            dk[kr + j] += ds * qr[j];
                            dv[kr + j] += pr * dor[j];
                        }
                    }
                }
            }
        }
    }
}

/* -------------------------------------------------------------- SwiGLU */

/* kernel `swiglu`, kernels.py:90-93 and the fused epilogue of
 * projection_gate_up, projection.py:67-73: h = g*sigmoid(g)*u. */
void or_swiglu_fwd(const double *g, const double *u, double *h, long n) {
    for (long i = 0; i < n; i++) h[i] = g[i] / (1.0 + exp(-g[i])) * u[i];
}

/* kernel `swiglu_backward`, kernels.py:95-101:
 * s = sigmoid(g); dg = dy*u*s*(1+g*(1-s)); du = dy*g*s. */
void or_swiglu_bwd(const double *g, const double *u, const double *dy,
                   double *dg, double *du, long n) {
    for (long i = 0; i < n; i++) {
        double s = 1.0 / (1.0 + exp(-g[i]));
        dg[i] = dy[i] * u[i] * s * (1.0 + g[i] * (1.0 - s));
        du[i] = dy[i] * g[i] * s;
    }
}

/* ----------------------------------------------------------- Embedding */

/* kernel `embedding`, kernels.py:41-45: y[i] = W[ids[i]]. */
void or_embedding_fwd(const double *W, const int32_t *ids, double *y, long N,
                      long D) {
    for (long i = 0; i < N; i++) memcpy(y + i * D, W + (long)ids[i] * D, sizeof(double) * (size_t)D);
}

/* kernel `embedding_backward`, kernels.py:47-52: dW[ids[i]] += dy[i]
 * into a zero-filled [V, D] (lib.rs:667-687). */
void or_embedding_bwd(const double *dy, const int32_t *ids, double *dW, long N,
                      long D, long V) {
    memset(dW, 0, sizeof(double) * (size_t)(V * D));
    for (long i = 0; i < N; i++)
        for (long j = 0; j < D; j++) dW[(long)ids[i] * D + j] += dy[i * D + j];
}

/* ------------------------------------------------------- Cross-entropy */

/* kernels `cross_entropy` / `cross_entropy_backward`, kernels.py:176-191:
 * loss = logsumexp(x) - x[t]; dx = (softmax(x) - onehot(t)) * dy_scale,
 * with dy_scale = scale/count from Graph::backward, graph.rs:539-549. */
void or_cross_entropy(const double *x, const int32_t *targets, double *loss,
                      double *dx, long R, long V, double dy_scale) {
#pragma omp parallel for schedule(static)
    for (long r = 0; r < R; r++) {
        const double *xr = x + r * V;
        double m = -INFINITY;
        for (long j = 0; j < V; j++) if (xr[j] > m) m = xr[j];
        double z = 0.0;
        for (long j = 0; j < V; j++) z += exp(xr[j] - m);
        loss[r] = m + log(z) - xr[targets[r]];
        if (dx)
            for (long j = 0; j < V; j++)
                dx[r * V + j] = (exp(xr[j] - m) / z - (j == targets[r] ? 1.0 : 0.0)) * dy_scale;
    }
}

/* ------------------------------------------------------------ Optimizer */

/* Global gradient norm: kernel `gradient_norm` kernels.py:265-287 (FP64
 * sum of squares per tensor) summed and square-rooted on the host
 * (lib.rs:494-523). */
double or_sum_squares(const double *g, long n) {
    double s = 0.0;
    for (long i = 0; i < n; i++) s += g[i] * g[i];
    return s;
}

/* kernel `adamw`, kernels.py:193-202 (launched per tensor by Adam::update,
 * crates/sejong-train/src/lib.rs:199-238):
 *   g *= scale; m = b1 m + (1-b1) g; v = b2 v + (1-b2) g^2;
 *   den = sqrt(v*ib2) + eps; step = den > 0 ? m*ib1/den : 0;
 *   w = w*(1 - lr*decay) - lr*step. */
void or_adamw(double *w, const double *g, double *m, double *v, long n,
              double lr, double b1, double b2, double eps, double decay,
              double ib1, double ib2, double scale) {
    #pragma omp parallel for schedule(static)
    for (long i = 0; i < n; i++) {
        double gi = g[i] * scale;
        m[i] = b1 * m[i] + (1.0 - b1) * gi;
        v[i] = b2 * v[i] + (1.0 - b2) * gi * gi;
        double den = sqrt(v[i] * ib2) + eps;
        double st = den > 0.0 ? (m[i] * ib1) / den : 0.0;
        w[i] = w[i] * (1.0 - lr * decay) - lr * st;
    }
}

/* ------------------------------------------------------------- Routing */

/* kernel `hierarchy_route_topk`, hierarchy.py:175-191: softmax over E
 * logits; K rounds of argmax with lowest-index tie-break; weight = full
 * softmax probability of the chosen expert (not renormalised).
 * Logits are consumed as the float values the device reads. */
void or_route_topk(const float *x, int32_t *ids, double *weights, long R,
                   long E, long K) {
    for (long r = 0; r < R; r++) {
        float sc[256];
        double m = -INFINITY, z = 0.0;
        for (long e = 0; e < E; e++) {
            sc[e] = x[r * E + e];
            if (sc[e] > m) m = sc[e];
        }
        for (long e = 0; e < E; e++) z += exp((double)sc[e] - m);
        for (long s = 0; s < K; s++) {
            long best = -1;
            for (long e = 0; e < E; e++)
                if (best < 0 || sc[e] > sc[best]) best = e; /* strict: lowest index wins ties */
            ids[r * K + s] = (int32_t)best;
            weights[r * K + s] = exp((double)sc[best] - m) / z;
            sc[best] = -INFINITY;
        }
    }
}

/* kernel `hierarchy_route_backward`, hierarchy.py:194-209:
 * dx = p * (dy_sel - sum_k w_k dy_k). */
void or_route_topk_bwd(const float *x, const int32_t *ids, const double *weights,
                       const double *dy, double *dx, long R, long E, long K) {
    for (long r = 0; r < R; r++) {
        double m = -INFINITY, z = 0.0, total = 0.0;
        for (long e = 0; e < E; e++) if (x[r * E + e] > m) m = x[r * E + e];
        for (long e = 0; e < E; e++) z += exp((double)x[r * E + e] - m);
        for (long s = 0; s < K; s++) total += weights[r * K + s] * dy[r * K + s];
        for (long e = 0; e < E; e++) {
            double sel = 0.0;
            for (long s = 0; s < K; s++) if (ids[r * K + s] == e) sel += dy[r * K + s];
            dx[r * E + e] = exp((double)x[r * E + e] - m) / z * (sel - total);
        }
    }
}

/* kernel `hierarchy_route_pack`, hierarchy.py:212-225: per expert, stable
 * compaction of slots (ascending) whose id is that expert.  tokens/slots
 * are [E, R] (R = rows*K slots), counts [E]. */
void or_route_pack(const int32_t *ids, int32_t *tokens, int32_t *slots,
                   int32_t *counts, long S, long K, long E) {
    for (long e = 0; e < E; e++) {
        int32_t c = 0;
        for (long s = 0; s < S; s++)
            if (ids[s] == e) {
                tokens[e * S + c] = (int32_t)(s / K);
                slots[e * S + c] = (int32_t)s;
                c++;
            }
        counts[e] = c;
    }
}

/* ========================================================= Dense model
 *
 * Byte Transformer forward + backward, following Block::apply
 * (crates/sejong-model/src/architecture.rs:200-247), the head
 * (crates/sejong-model/src/lib.rs:336-340, architecture.rs:160-167) and the
 * tape's reverse rules (crates/sejong-gpu/src/graph.rs:567-911).
 *
 * Parameters are passed in the reference layout and order
 * (architecture.rs:63-137): embedding [V,d]; per layer attention_norm [d],
 * ffn_norm [d], query [d,d], key [d,J], value [d,J], attention_output [d,d],
 * gate [d,F], up [d,F], down [F,d]; final_norm [d]; output [d,V].
 *
 * Forward activations are rounded to `dtype` where the reference kernels
 * store them (compute precision; output head and CE stay fp32).  Backward
 * quantities are FP64 (the reference keeps them fp32: rounding them is
 * below the 1e-3 gate by four orders of magnitude).
 */
typedef struct {
    long d, layers, hq, hk, ffn, T, B;
    double eps, theta;
    int dtype; /* 0 f32, 4 bf16, negative = no rounding (exact FP64) */
    long window; /* local causal window of the hierarchical stages (0: none) */
} or_model_cfg;

static long or_param_count_internal(const or_model_cfg *c) {
    long d = c->d, J = c->d / c->hq * c->hk, F = c->ffn;
    long per = 2 * d + d * d + 2 * d * J + d * d + 2 * d * F + F * d;
    return OR_VOCAB * d + c->layers * per + d + d * OR_VOCAB;
}

long or_model_param_count(long d, long layers, long hq, long hk, long ffn) {
    or_model_cfg c = {d, layers, hq, hk, ffn, 1, 1, 0, 0, 0, 0};
    return or_param_count_internal(&c);
}

static double *dup_round(const double *x, long n, int dtype) {
    double *y = (double *)malloc(sizeof(double) * (size_t)n);
    memcpy(y, x, sizeof(double) * (size_t)n);
    or_round(y, n, dtype);
    return y;
}

/* Activation pack: the forward values every backward rule reads, in the
 * storage dtype of the step (already rounded), laid out per layer as
 *   x [M d], z [M d], qr [M d], kr [M J], v [M J], o [M d], lse [M HQ],
 *   x1 [M d], z2 [M d], g [M F], u [M F], h [M F]
 * followed by xL [M d], hn [M d], logits [M V].  The device step exports
 * the same pack, so the backward can be checked conditioned on the device's
 * stored operands (the reference checks condition the same way). */
long or_model_acts_count(long d, long layers, long hq, long hk, long ffn, long T, long B) {
    long M = T * B, J = d / hq * hk;
    long per = 6 * M * d + 2 * M * J + M * hq + 3 * M * ffn;
    return layers * per + 2 * M * d + M * OR_VOCAB;
}

typedef struct {
    const double *an, *fn, *wq, *wk, *wv, *wo, *wg, *wu, *wd;
    long o_an, o_fn, o_wq, o_wk, o_wv, o_wo, o_wg, o_wu, o_wd;
} lw;

typedef struct {
    long off_emb, off_final, off_out, total;
    lw *L;
    double *C; /* compute copies */
} plan_t;

static void make_plan(const or_model_cfg *c, const double *params, plan_t *pl) {
    const long d = c->d, V = OR_VOCAB, J = c->d / c->hq * c->hk, F = c->ffn;
    long off = 0;
    pl->off_emb = off; off += V * d;
    pl->L = (lw *)calloc((size_t)c->layers, sizeof(lw));
    for (long l = 0; l < c->layers; l++) {
        lw *y = &pl->L[l];
        y->o_an = off; off += d;
        y->o_fn = off; off += d;
        y->o_wq = off; off += d * d;
        y->o_wk = off; off += d * J;
        y->o_wv = off; off += d * J;
        y->o_wo = off; off += d * d;
        y->o_wg = off; off += d * F;
        y->o_wu = off; off += d * F;
        y->o_wd = off; off += F * d;
    }
    pl->off_final = off; off += d;
    pl->off_out = off; off += d * V;
    pl->total = off;
    /* compute copies: bind() casts every master to compute precision
     * (model lib.rs:214-219); the head keeps the fp32 master (lib.rs:336-340) */
    pl->C = dup_round(params, off, c->dtype);
    for (long l = 0; l < c->layers; l++) {
        lw *y = &pl->L[l];
        y->an = pl->C + y->o_an; y->fn = pl->C + y->o_fn; y->wq = pl->C + y->o_wq;
        y->wk = pl->C + y->o_wk; y->wv = pl->C + y->o_wv; y->wo = pl->C + y->o_wo;
        y->wg = pl->C + y->o_wg; y->wu = pl->C + y->o_wu; y->wd = pl->C + y->o_wd;
    }
}

typedef struct {
    double *x, *z, *qr, *kr, *v, *o, *lse, *x1, *z2, *g, *u, *h;
} layer_view;

static void view_acts(const or_model_cfg *c, double *acts, layer_view *lv, double **xl, double **hn,
                      double **logits) {
    const long M = c->T * c->B, d = c->d, J = c->d / c->hq * c->hk, F = c->ffn;
    double *p = acts;
    for (long l = 0; l < c->layers; l++) {
        layer_view *a = &lv[l];
        a->x = p; p += M * d;
        a->z = p; p += M * d;
        a->qr = p; p += M * d;
        a->kr = p; p += M * J;
        a->v = p; p += M * J;
        a->o = p; p += M * d;
        a->lse = p; p += M * c->hq;
        a->x1 = p; p += M * d;
        a->z2 = p; p += M * d;
        a->g = p; p += M * F;
        a->u = p; p += M * F;
        a->h = p; p += M * F;
    }
    *xl = p; p += M * d;
    *hn = p; p += M * d;
    *logits = p;
}

#define ALLOC(n) ((double *)malloc(sizeof(double) * (size_t)(n)))

/* Block::apply per layer from lv[0].x (architecture.rs:200-247, window as
 * hierarchy.py:24), then the closing norm into hn, rounded to the storage
 * dtype where the reference kernels store. */
static void body_forward(const or_model_cfg *c, const plan_t *pl, layer_view *lv, double *xl, double *hn) {
    const long d = c->d, layers = c->layers, hq = c->hq, hk = c->hk, T = c->T, B = c->B;
    const long M = T * B, Dh = d / hq, J = Dh * hk, F = c->ffn;
    const double eps = c->eps, theta = c->theta;
    const int dtype = c->dtype, rd = dtype < 0 ? -1 : 0; /* fp32 storage of LSE */
    double *q = ALLOC(M * d), *k = ALLOC(M * J), *tmp = ALLOC(M * (d > F ? d : F));
    for (long l = 0; l < layers; l++) {
        layer_view *a = &lv[l];
        const lw *y = &pl->L[l];
        double *xnext = (l + 1 < layers) ? lv[l + 1].x : xl;
        or_rmsnorm_fwd(a->x, y->an, a->z, M, d, eps); or_round(a->z, M * d, dtype);
        or_matmul(a->z, y->wq, q, M, d, d, 0, 0); or_round(q, M * d, dtype);
        or_matmul(a->z, y->wk, k, M, J, d, 0, 0); or_round(k, M * J, dtype);
        or_matmul(a->z, y->wv, a->v, M, J, d, 0, 0); or_round(a->v, M * J, dtype);
        or_rope(q, a->qr, M, T, hq, Dh, 0, theta, 0); or_round(a->qr, M * d, dtype);
        or_rope(k, a->kr, M, T, hk, Dh, 0, theta, 0); or_round(a->kr, M * J, dtype);
        or_attention_fwd(a->qr, a->kr, a->v, a->o, a->lse, B, T, hq, hk, Dh, c->window);
        or_round(a->o, M * d, dtype); or_round(a->lse, M * hq, rd);
        or_matmul(a->o, y->wo, tmp, M, d, d, 0, 0); or_round(tmp, M * d, dtype);
        for (long i = 0; i < M * d; i++) a->x1[i] = a->x[i] + tmp[i];
        or_round(a->x1, M * d, dtype);
        or_rmsnorm_fwd(a->x1, y->fn, a->z2, M, d, eps); or_round(a->z2, M * d, dtype);
        or_matmul(a->z2, y->wg, a->g, M, F, d, 0, 0); or_round(a->g, M * F, dtype);
        or_matmul(a->z2, y->wu, a->u, M, F, d, 0, 0); or_round(a->u, M * F, dtype);
        or_swiglu_fwd(a->g, a->u, a->h, M * F); or_round(a->h, M * F, dtype);
        or_matmul(a->h, y->wd, tmp, M, d, F, 0, 0); or_round(tmp, M * d, dtype);
        for (long i = 0; i < M * d; i++) xnext[i] = a->x1[i] + tmp[i];
        or_round(xnext, M * d, dtype);
    }
    or_rmsnorm_fwd(xl, pl->C + pl->off_final, hn, M, d, eps);
    or_round(hn, M * d, dtype); /* then cast to F32: exact */
    free(q); free(k); free(tmp);
}

/* Forward of Block::apply per layer + head, writing the activation pack
 * (rounded to the storage dtype where the reference kernels store). */
void or_model_forward(long d, long layers, long hq, long hk, long ffn, long T, long B, double eps,
                      double theta, int dtype, const double *params, const int32_t *ids, double *acts) {
    or_model_cfg cf = {d, layers, hq, hk, ffn, T, B, eps, theta, dtype, 0};
    const long M = T * B, V = OR_VOCAB;
    plan_t pl;
    make_plan(&cf, params, &pl);
    layer_view *lv = (layer_view *)calloc((size_t)layers, sizeof(layer_view));
    double *xl, *hn, *logits;
    view_acts(&cf, acts, lv, &xl, &hn, &logits);
    const int rd = dtype < 0 ? -1 : 0; /* fp32 storage of the logits */
    or_embedding_fwd(pl.C + pl.off_emb, ids, lv[0].x, M, d);
    body_forward(&cf, &pl, lv, xl, hn);
    or_matmul(hn, params + pl.off_out, logits, M, V, d, 0, 0);
    or_round(logits, M * V, rd);
    free(lv); free(pl.L); free(pl.C);
}

/* Backward (graph.rs:567-911 in one block's fixed order) from an
 * activation pack: CE on the stored logits with the mean seed, head, final
 * norm, then per layer down / SwiGLU / gate+up / ffn norm / attention
 * output / attention (+ inverse RoPE) / QKV / attention norm, embedding.
 * grads: reference layout (FP64).  Returns the mean loss of the logits. */
/* or_model_backward with the output gradients of the projection Matmul
 * nodes kept: dys (nullable) receives per layer, in this order, dY of the
 * query (pre-RoPE), key (pre-RoPE), value, gate and up projections
 * ([M][d], [M][J], [M][J], [M][F], [M][F]) -- the dY a parameter VJP
 * contracts with (graph.rs:829-851, parameter_vjp.rs:308-320). */
double or_model_backward_dys(long d, long layers, long hq, long hk, long ffn, long T, long B, double eps,
                             double theta, int dtype, const double *params, const double *acts_in,
                             const int32_t *ids, const int32_t *targets, double *grads, double *loss_rows,
                             double *dys);

double or_model_backward(long d, long layers, long hq, long hk, long ffn, long T, long B, double eps,
                         double theta, int dtype, const double *params, const double *acts_in,
                         const int32_t *ids, const int32_t *targets, double *grads, double *loss_rows) {
    return or_model_backward_dys(d, layers, hq, hk, ffn, T, B, eps, theta, dtype, params, acts_in, ids, targets,
                                 grads, loss_rows, NULL);
}

/* The body's backward from dx = d(final norm output) [M][d]: final norm,
 * then per layer down / SwiGLU / gate+up / ffn norm / attention output /
 * attention (+ inverse RoPE) / QKV / attention norm.  The gradient at the
 * embedding output is left in demb [M][d] (nullable: then the embedding
 * backward into grads runs here, ids < OR_VOCAB). */
static void body_backward(const or_model_cfg *c, const plan_t *pl, layer_view *lv, const double *xl, double *dx,
                          const int32_t *ids, double *grads, double *dys, double *demb) {
    const long d = c->d, layers = c->layers, hq = c->hq, hk = c->hk, T = c->T, B = c->B;
    const long M = T * B, V = OR_VOCAB, Dh = d / hq, J = Dh * hk, F = c->ffn;
    const double eps = c->eps, theta = c->theta;
    double *dres = ALLOC(M * d);
    or_rmsnorm_bwd(xl, pl->C + pl->off_final, dx, NULL, dres, grads + pl->off_final, M, d, eps);
    double *dbig = ALLOC(M * F), *dg = ALLOC(M * F), *du = ALLOC(M * F);
    double *dz = ALLOC(M * d), *dtmp = ALLOC(M * d), *dx1 = ALLOC(M * d), *dO = ALLOC(M * d);
    double *dq = ALLOC(M * d), *dk = ALLOC(M * J), *dv = ALLOC(M * J);
    double *dqr = ALLOC(M * d), *dkr = ALLOC(M * J), *dxn = ALLOC(M * d);
    for (long l = layers - 1; l >= 0; l--) {
        layer_view *a = &lv[l];
        const lw *y = &pl->L[l];
        /* x_{l+1} = x1 + down(h): dres flows to x1 and to down's output */
        or_matmul(dres, y->wd, dbig, M, F, d, 0, 1);              /* dh */
        or_matmul(a->h, dres, grads + y->o_wd, F, d, M, 1, 0);    /* dW_down */
        or_swiglu_bwd(a->g, a->u, dbig, dg, du, M * F);
        double *dyl = dys ? dys + l * M * (d + 2 * J + 2 * F) : NULL;
        if (dyl) {
            memcpy(dyl + M * (d + 2 * J), dg, sizeof(double) * (size_t)(M * F));
            memcpy(dyl + M * (d + 2 * J + F), du, sizeof(double) * (size_t)(M * F));
        }
        or_matmul(dg, y->wg, dz, M, d, F, 0, 1);
        or_matmul(du, y->wu, dtmp, M, d, F, 0, 1);
        for (long i = 0; i < M * d; i++) dz[i] += dtmp[i];
        or_matmul(a->z2, dg, grads + y->o_wg, d, F, M, 1, 0);
        or_matmul(a->z2, du, grads + y->o_wu, d, F, M, 1, 0);
        or_rmsnorm_bwd(a->x1, y->fn, dz, dres, dx1, grads + y->o_fn, M, d, eps);
        /* x1 = x + attention_output(o) */
        or_matmul(dx1, y->wo, dO, M, d, d, 0, 1);
        or_matmul(a->o, dx1, grads + y->o_wo, d, d, M, 1, 0);
        or_attention_bwd(a->qr, a->kr, a->v, a->o, a->lse, dO, dqr, dkr, dv, NULL, B, T, hq, hk, Dh, c->window);
        or_rope(dqr, dq, M, T, hq, Dh, 0, theta, 1);
        or_rope(dkr, dk, M, T, hk, Dh, 0, theta, 1);
        if (dyl) {
            memcpy(dyl, dq, sizeof(double) * (size_t)(M * d));
            memcpy(dyl + M * d, dk, sizeof(double) * (size_t)(M * J));
            memcpy(dyl + M * (d + J), dv, sizeof(double) * (size_t)(M * J));
        }
        or_matmul(dq, y->wq, dz, M, d, d, 0, 1);
        or_matmul(dk, y->wk, dtmp, M, d, J, 0, 1);
        for (long i = 0; i < M * d; i++) dz[i] += dtmp[i];
        or_matmul(dv, y->wv, dtmp, M, d, J, 0, 1);
        for (long i = 0; i < M * d; i++) dz[i] += dtmp[i];
        or_matmul(a->z, dq, grads + y->o_wq, d, d, M, 1, 0);
        or_matmul(a->z, dk, grads + y->o_wk, d, J, M, 1, 0);
        or_matmul(a->z, dv, grads + y->o_wv, d, J, M, 1, 0);
        or_rmsnorm_bwd(a->x, y->an, dz, dx1, dxn, grads + y->o_an, M, d, eps);
        double *t = dres; dres = dxn; dxn = t;
    }
    if (demb)
        memcpy(demb, dres, sizeof(double) * (size_t)(M * d));
    else
        or_embedding_bwd(dres, ids, grads + pl->off_emb, M, d, V);
    free(dres); free(dbig); free(dg); free(du); free(dz); free(dtmp);
    free(dx1); free(dO); free(dq); free(dk); free(dv); free(dqr); free(dkr); free(dxn);
}

double or_model_backward_dys(long d, long layers, long hq, long hk, long ffn, long T, long B, double eps,
                             double theta, int dtype, const double *params, const double *acts_in,
                             const int32_t *ids, const int32_t *targets, double *grads, double *loss_rows,
                             double *dys) {
    or_model_cfg cf = {d, layers, hq, hk, ffn, T, B, eps, theta, dtype, 0};
    const long M = T * B, V = OR_VOCAB;
    plan_t pl;
    make_plan(&cf, params, &pl);
    layer_view *lv = (layer_view *)calloc((size_t)layers, sizeof(layer_view));
    double *xl, *hn, *logits;
    view_acts(&cf, (double *)acts_in, lv, &xl, &hn, &logits);
    double *lrow = ALLOC(M), *dlog = ALLOC(M * V);
    /* seed scale/count, graph.rs:539-549 (f32 division in the reference) */
    double seed = (double)(1.0f / (float)M);
    or_cross_entropy(logits, targets, lrow, dlog, M, V, seed);
    double loss = 0.0;
    for (long i = 0; i < M; i++) loss += lrow[i];
    loss /= (double)M;
    if (loss_rows) memcpy(loss_rows, lrow, sizeof(double) * (size_t)M);
    memset(grads, 0, sizeof(double) * (size_t)pl.total);
    const double *wout = params + pl.off_out;
    double *dx = ALLOC(M * d);
    or_matmul(dlog, wout, dx, M, d, V, 0, 1);               /* dh = dlogits W^T */
    or_matmul(hn, dlog, grads + pl.off_out, d, V, M, 1, 0); /* dW_out = h^T dlogits */
    body_backward(&cf, &pl, lv, xl, dx, ids, grads, dys, NULL);
    free(lrow); free(dlog); free(dx);
    free(lv); free(pl.L); free(pl.C);
    return loss;
}

/* The body's backward from a given gradient of the final-norm output
 * dh [M][d] (another head on the body, e.g. NativeValue's affine value
 * head, native/value.rs:139-146): grads (reference layout; embedding and
 * output left zero) and the gradient at the embedding output demb [M][d]
 * for the caller's own embedding. */
void or_model_backward_hidden(long d, long layers, long hq, long hk, long ffn, long T, long B, double eps,
                              double theta, int dtype, const double *params, const double *acts_in,
                              const double *dh, double *grads, double *demb) {
    or_model_cfg cf = {d, layers, hq, hk, ffn, T, B, eps, theta, dtype, 0};
    const long M = T * B;
    plan_t pl;
    make_plan(&cf, params, &pl);
    layer_view *lv = (layer_view *)calloc((size_t)layers, sizeof(layer_view));
    double *xl, *hn, *logits;
    view_acts(&cf, (double *)acts_in, lv, &xl, &hn, &logits);
    memset(grads, 0, sizeof(double) * (size_t)pl.total);
    double *dx = ALLOC(M * d);
    memcpy(dx, dh, sizeof(double) * (size_t)(M * d));
    body_backward(&cf, &pl, lv, xl, dx, NULL, grads, NULL, demb);
    free(dx); free(lv); free(pl.L); free(pl.C);
}

/* One stage of the hierarchical model (architecture.rs:368-393): a run of
 * blocks with its own width, heads, FFN, sequence and local window, closed
 * by its norm.  sparams: per layer the nine tensors in stage_layout order
 * (architecture.rs:63-95), then the closing norm [d].  The activation pack
 * is the model's per-layer pack followed by the stage's last residual and
 * the closing norm's output. */
static double *stage_padded(const or_model_cfg *c, const double *sparams, long *total) {
    const long d = c->d, V = OR_VOCAB;
    long n = or_param_count_internal(c);
    long body = n - V * d - d - d * V; /* layer tensors */
    double *p = (double *)calloc((size_t)n, sizeof(double));
    memcpy(p + V * d, sparams, sizeof(double) * (size_t)(body + d));
    *total = n;
    return p;
}

long or_stage_acts_count(long d, long layers, long hq, long hk, long ffn, long T, long B) {
    long M = T * B, J = d / hq * hk;
    return layers * (6 * M * d + 2 * M * J + M * hq + 3 * M * ffn) + 2 * M * d;
}

void or_stage_forward(long d, long layers, long hq, long hk, long ffn, long T, long B, double eps, double theta,
                      int dtype, long window, const double *sparams, const double *x_in, double *acts) {
    or_model_cfg cf = {d, layers, hq, hk, ffn, T, B, eps, theta, dtype, window};
    long total;
    double *padded = stage_padded(&cf, sparams, &total);
    plan_t pl;
    make_plan(&cf, padded, &pl);
    layer_view *lv = (layer_view *)calloc((size_t)(layers > 0 ? layers : 1), sizeof(layer_view));
    double *xl, *hn, *logits;
    view_acts(&cf, acts, lv, &xl, &hn, &logits);
    const long M = T * B;
    if (layers > 0) memcpy(lv[0].x, x_in, sizeof(double) * (size_t)(M * d));
    else memcpy(xl, x_in, sizeof(double) * (size_t)(M * d));
    if (layers > 0) body_forward(&cf, &pl, lv, xl, hn);
    else {
        or_rmsnorm_fwd(xl, pl.C + pl.off_final, hn, M, d, eps);
        or_round(hn, M * d, dtype);
    }
    free(lv); free(pl.L); free(pl.C); free(padded);
}

/* dz = d(closing norm output) [M][d]; grads: the stage's tensors (sparams
 * layout); dx_in: d(stage input). */
void or_stage_backward(long d, long layers, long hq, long hk, long ffn, long T, long B, double eps, double theta,
                       int dtype, long window, const double *sparams, const double *acts_in, const double *dz,
                       double *grads, double *dx_in) {
    or_model_cfg cf = {d, layers, hq, hk, ffn, T, B, eps, theta, dtype, window};
    long total;
    double *padded = stage_padded(&cf, sparams, &total);
    plan_t pl;
    make_plan(&cf, padded, &pl);
    layer_view *lv = (layer_view *)calloc((size_t)layers, sizeof(layer_view));
    double *xl, *hn, *logits;
    view_acts(&cf, (double *)acts_in, lv, &xl, &hn, &logits);
    const long M = T * B, V = OR_VOCAB;
    double *g = (double *)calloc((size_t)total, sizeof(double));
    double *dx = ALLOC(M * d);
    memcpy(dx, dz, sizeof(double) * (size_t)(M * d));
    body_backward(&cf, &pl, lv, xl, dx, NULL, g, NULL, dx_in);
    memcpy(grads, g + V * d, sizeof(double) * (size_t)(total - V * d - d * V));
    free(dx); free(g); free(lv); free(pl.L); free(pl.C); free(padded);
}

/* One training forward+backward.  params: reference layout (above), fp32
 * master values.  grads: same layout, receives dL/dparam (FP64).  Returns
 * the mean cross-entropy.  loss_rows (nullable) receives per-row losses,
 * logits_out (nullable) the fp32 logits [M, V]. */
double or_model_fwd_bwd(long d, long layers, long hq, long hk, long ffn,
                        long T, long B, double eps, double theta, int dtype,
                        const double *params, const int32_t *ids,
                        const int32_t *targets, double *grads,
                        double *loss_rows, double *logits_out) {
    long na = or_model_acts_count(d, layers, hq, hk, ffn, T, B);
    double *acts = ALLOC(na);
    or_model_forward(d, layers, hq, hk, ffn, T, B, eps, theta, dtype, params, ids, acts);
    if (logits_out) {
        long M = T * B;
        memcpy(logits_out, acts + na - M * OR_VOCAB, sizeof(double) * (size_t)(M * OR_VOCAB));
    }
    double loss = or_model_backward(d, layers, hq, hk, ffn, T, B, eps, theta, dtype, params, acts, ids,
                                    targets, grads, loss_rows);
    free(acts);
    return loss;
}
#undef ALLOC

/* Loss only (forward), for finite-difference checks. */
double or_model_loss(long d, long layers, long hq, long hk, long ffn, long T,
                     long B, double eps, double theta, int dtype,
                     const double *params, const int32_t *ids,
                     const int32_t *targets) {
    or_model_cfg cf = {d, layers, hq, hk, ffn, T, B, eps, theta, dtype, 0};
    long n = or_param_count_internal(&cf);
    double *g = (double *)malloc(sizeof(double) * (size_t)n);
    double loss = or_model_fwd_bwd(d, layers, hq, hk, ffn, T, B, eps, theta, dtype,
                                   params, ids, targets, g, NULL, NULL);
    free(g);
    return loss;
}

int or_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
