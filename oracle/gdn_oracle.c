/*
 * gdn_oracle.c -- CPU restatement of the Qwen3.5 Gated DeltaNet layer, accumulating in fp64.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity checker for the HIP path: only the tests, the
 * smoke check and the CPU-baseline leg of the benchmark may load it.  The product never calls it.
 *
 * Every function restates the reference's algorithm from its source (paths relative to the
 * reference root; "HF:" = transformers/models/qwen3_5/modeling_qwen3_5.py, 5.15.0, the layer truth
 * the reference's tests compare against).  All arrays are row-major float32 at the boundary; every
 * sum, product and transcendental inside runs in double.
 *
 * Pins (see tests/test_oracle_*.py): golden vectors written by tests/golden/make_golden.py from the
 * HF torch path; closed forms and invariants; sequential == chunked identity.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define EXPORT __attribute__((visibility("default")))

EXPORT void orc_set_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}

EXPORT int orc_get_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* ------------------------------------------------------------------------------------------------ */
/* Integer rules (bit-exact contracts)                                                              */
/* ------------------------------------------------------------------------------------------------ */

/* v-head h reads k-head h / (nv / nk): repeat_interleave, not tile.
 * wormhole_n150/qwen3.5_9B/reference.py:21-23; HF:500-502; 9B/gdn_layer.py:51 (kh = h // 2). */
EXPORT int orc_khead_of_vhead(int h, int nv, int nk) { return h / (nv / nk); }

/* Source of the conv input x~[t - s] (s = 1..3) for token t of a T-token launch:
 * returns t - s (a row of this launch) when t >= s, else -(slot + 1) with slot = 3 + t - s of the
 * time-ordered history (slot 0 oldest).  9B/kernels/layer_reader.cpp:111-120. */
EXPORT int orc_conv_src(int t, int s, int T) {
    (void)T;
    return t >= s ? t - s : -((3 + t - s) + 1);
}

/* Source of the new history slot k (0..2) after a T-token launch: row T - 3 + k when T + k >= 3,
 * else old slot T + k encoded as -(slot + 1).  9B/kernels/layer_reader.cpp:184-197. */
EXPORT int orc_roll_src(int T, int k) { return T + k >= 3 ? T + k - 3 : -((T + k) + 1); }

/* Row m of a [B*T, ...] sequence-major launch is token t of sequence b.  9B/gdn_layer.py:291;
 * 9B/kernels/layer_reader.cpp:107-109; layer_compute.cpp:231 (state slot m / T). */
EXPORT void orc_row_to_bt(int m, int T, int* b, int* t) {
    *b = m / T;
    *t = m - (m / T) * T;
}

/* ------------------------------------------------------------------------------------------------ */
/* Scalar functions                                                                                  */
/* ------------------------------------------------------------------------------------------------ */

static double softplus_t20(double x) { return x > 20.0 ? x : log1p(exp(x)); } /* torch default threshold 20 */
static double sigmoid_d(double x) { return 1.0 / (1.0 + exp(-x)); }
static double silu_d(double x) { return x * sigmoid_d(x); }

/* ------------------------------------------------------------------------------------------------ */
/* Projections: y[M,N] = x[M,K] . w[N,K]^T  (nn.Linear, HF [out, in] weight layout)                   */
/* 9B/gdn_layer.py:255-259 (in_proj, a/b), 272-276 (out_proj); HF:459-466, 541.                       */
/* ------------------------------------------------------------------------------------------------ */
EXPORT void orc_linear(const float* x, const float* w, int M, int N, int K, float* y) {
#pragma omp parallel for schedule(static)
    for (int n = 0; n < N; ++n) {
        const float* wr = w + (size_t)n * K;
        for (int m = 0; m < M; ++m) {
            const float* xr = x + (size_t)m * K;
            double acc = 0.0;
            for (int k = 0; k < K; ++k) acc += (double)xr[k] * (double)wr[k];
            y[(size_t)m * N + n] = (float)acc;
        }
    }
}

/* The same in fp64 on fp64 activations.  Blocked so that a block of 32 activation rows stays in cache while
 * a block of weight rows streams past it; each dot product keeps four partial sums over k mod 4 (added at
 * the end) so the compiler can vectorise it.  The result is the fp64 dot product up to fp64 rounding. */
static double dot_d(const double* x, const float* w, int K) {
    double a0 = 0.0, a1 = 0.0, a2 = 0.0, a3 = 0.0;
    int k = 0;
    for (; k + 4 <= K; k += 4) {
        a0 += x[k] * (double)w[k];
        a1 += x[k + 1] * (double)w[k + 1];
        a2 += x[k + 2] * (double)w[k + 2];
        a3 += x[k + 3] * (double)w[k + 3];
    }
    double t = (a0 + a1) + (a2 + a3);
    for (; k < K; ++k) t += x[k] * (double)w[k];
    return t;
}

/* Four activation rows against two weight rows at once (eight dot products sharing their loads). */
static void dot_4x2(const double* x, size_t ldx, const float* w, size_t ldw, int K, double* y, size_t ldy) {
    double acc[4][2][4] = {{{0.0}}};
    int k = 0;
    for (; k + 4 <= K; k += 4) {
        double wv[2][4];
        for (int c = 0; c < 2; ++c)
            for (int j = 0; j < 4; ++j) wv[c][j] = (double)w[(size_t)c * ldw + k + j];
        for (int r = 0; r < 4; ++r)
            for (int c = 0; c < 2; ++c)
                for (int j = 0; j < 4; ++j) acc[r][c][j] += x[(size_t)r * ldx + k + j] * wv[c][j];
    }
    for (int r = 0; r < 4; ++r)
        for (int c = 0; c < 2; ++c) {
            double t = (acc[r][c][0] + acc[r][c][1]) + (acc[r][c][2] + acc[r][c][3]);
            for (int kk = k; kk < K; ++kk) t += x[(size_t)r * ldx + kk] * (double)w[(size_t)c * ldw + kk];
            y[(size_t)r * ldy + c] = t;
        }
}

static void linear_d(const double* x, const float* w, int M, int N, int K, double* y) {
    enum { MB = 32, NB = 128 };
    const int nmb = (M + MB - 1) / MB, nnb = (N + NB - 1) / NB;
#pragma omp parallel for schedule(dynamic)
    for (int blk = 0; blk < nmb * nnb; ++blk) {
        const int m0 = (blk / nnb) * MB, n0 = (blk % nnb) * NB;
        const int m1 = m0 + MB < M ? m0 + MB : M, n1 = n0 + NB < N ? n0 + NB : N;
        int n = n0;
        for (; n + 2 <= n1; n += 2) {
            int m = m0;
            for (; m + 4 <= m1; m += 4)
                dot_4x2(x + (size_t)m * K, (size_t)K, w + (size_t)n * K, (size_t)K, K, y + (size_t)m * N + n, (size_t)N);
            for (; m < m1; ++m)
                for (int c = 0; c < 2; ++c) y[(size_t)m * N + n + c] = dot_d(x + (size_t)m * K, w + (size_t)(n + c) * K, K);
        }
        for (; n < n1; ++n)
            for (int m = m0; m < m1; ++m) y[(size_t)m * N + n] = dot_d(x + (size_t)m * K, w + (size_t)n * K, K);
    }
}

/* ------------------------------------------------------------------------------------------------ */
/* Causal depthwise conv1d (4 taps) + SiLU with a 3-slot time-ordered history per sequence.           */
/*   c[t, ch] = sum_j w[ch, j] * x~[t - 3 + j, ch],   x~[t'] = x[t'] (t' >= 0) or hist[3 + t'] (t' < 0) */
/*   new hist[k] = x~[T - 3 + k]                                                                      */
/* 9B/gdn_layer.py:100-101 (out[t] = sum_shift w[:, 3 - shift] x[t - shift]);                          */
/* 9B/kernels/layer_reader.cpp:103-124 (shift sources), 184-197 (roll); HF:199-239.                    */
/* x rows have stride row_stride (the channel block of a wider projection row).                        */
/* ------------------------------------------------------------------------------------------------ */
static void conv_silu_d(const double* x, int B, int T, int C, size_t row_stride, const float* w, double* hist,
                        double* out, size_t out_stride) {
#pragma omp parallel for schedule(static)
    for (int b = 0; b < B; ++b) {
        for (int ch = 0; ch < C; ++ch) {
            double* hs = hist + ((size_t)b * C + ch) * 3;
            for (int t = 0; t < T; ++t) {
                double acc = 0.0;
                for (int j = 0; j < 4; ++j) {
                    const int src = orc_conv_src(t, 3 - j, T); /* shift s = 3 - j; j = 3 is x[t] itself */
                    double xv;
                    if (j == 3)
                        xv = x[((size_t)b * T + t) * row_stride + ch];
                    else if (src >= 0)
                        xv = x[((size_t)b * T + src) * row_stride + ch];
                    else
                        xv = hs[-src - 1];
                    acc += (double)w[(size_t)ch * 4 + j] * xv;
                }
                out[((size_t)b * T + t) * out_stride + ch] = silu_d(acc);
            }
            double nh[3];
            for (int k = 0; k < 3; ++k) {
                const int src = orc_roll_src(T, k);
                nh[k] = src >= 0 ? x[((size_t)b * T + src) * row_stride + ch] : hs[-src - 1];
            }
            hs[0] = nh[0], hs[1] = nh[1], hs[2] = nh[2];
        }
    }
}

/* float wrapper: x [B, T, C] (row stride C), hist [B, C, 3] in/out, out [B, T, C]. */
EXPORT void orc_conv1d_silu(const float* x, int B, int T, int C, const float* w, float* hist, float* out) {
    const size_t n = (size_t)B * T * C;
    double* xd = (double*)malloc(n * sizeof(double));
    double* od = (double*)malloc(n * sizeof(double));
    double* hd = (double*)malloc((size_t)B * C * 3 * sizeof(double));
    for (size_t i = 0; i < n; ++i) xd[i] = x[i];
    for (size_t i = 0; i < (size_t)B * C * 3; ++i) hd[i] = hist[i];
    conv_silu_d(xd, B, T, C, (size_t)C, w, hd, od, (size_t)C);
    for (size_t i = 0; i < n; ++i) out[i] = (float)od[i];
    for (size_t i = 0; i < (size_t)B * C * 3; ++i) hist[i] = (float)hd[i];
    free(xd), free(od), free(hd);
}

/* ------------------------------------------------------------------------------------------------ */
/* Gated delta rule, sequential form.  wormhole_n150/qwen3.5_9B/reference.py:11-35 (== HF:333-381).   */
/*   q, k: [B,T,Hk,dk]  v: [B,T,Hv,dv]  g, beta: [B,T,Hv]  state: [B,Hv,dk,dv] (S[k][v])               */
/*   per token:  S <- exp(g) S;  kv = S^T k;  delta = beta (v - kv);  S <- S + k delta^T;  o = S^T q   */
/* q, k are L2-normalised (eps 1e-6, reference.py:7-8) when use_qk_l2norm, q scaled by `scale`         */
/* (dk^-0.5 when scale <= 0, reference.py:24), v-head h reads k-head h / (Hv / Hk) (:21-23).           */
/* ------------------------------------------------------------------------------------------------ */
static void l2norm_d(double* x, int n) {
    double ss = 0.0;
    for (int i = 0; i < n; ++i) ss += x[i] * x[i];
    const double r = 1.0 / sqrt(ss + 1e-6);
    for (int i = 0; i < n; ++i) x[i] *= r;
}

/* one (b, h) stream over T tokens; qn/kn already normalised and scaled, row strides in elements */
static void recurrent_head_d(const double* qn, const double* kn, size_t qk_stride, const double* v, size_t v_stride,
                             const double* g, const double* beta, size_t gb_stride, int T, int dk, int dv, double* S,
                             double* o, size_t o_stride) {
    double* kv = (double*)malloc(sizeof(double) * dv);
    for (int t = 0; t < T; ++t) {
        const double* qt = qn + (size_t)t * qk_stride;
        const double* kt = kn + (size_t)t * qk_stride;
        const double* vt = v + (size_t)t * v_stride;
        const double d = exp(g[(size_t)t * gb_stride]);
        const double bt = beta[(size_t)t * gb_stride];
        for (size_t i = 0; i < (size_t)dk * dv; ++i) S[i] *= d;
        for (int j = 0; j < dv; ++j) kv[j] = 0.0;
        for (int i = 0; i < dk; ++i)
            for (int j = 0; j < dv; ++j) kv[j] += S[(size_t)i * dv + j] * kt[i];
        for (int j = 0; j < dv; ++j) kv[j] = (vt[j] - kv[j]) * bt; /* delta */
        for (int i = 0; i < dk; ++i)
            for (int j = 0; j < dv; ++j) S[(size_t)i * dv + j] += kt[i] * kv[j];
        double* ot = o + (size_t)t * o_stride;
        for (int j = 0; j < dv; ++j) ot[j] = 0.0;
        for (int i = 0; i < dk; ++i)
            for (int j = 0; j < dv; ++j) ot[j] += S[(size_t)i * dv + j] * qt[i];
    }
    free(kv);
}

/* prepare normalised, scaled q/k per (b, t, k-head) in double */
static void prep_qk_d(const float* q, const float* k, int n_rows, int dk, int use_l2, double scale, double* qn,
                      double* kn) {
#pragma omp parallel for schedule(static)
    for (int r = 0; r < n_rows; ++r) {
        double* qr = qn + (size_t)r * dk;
        double* kr = kn + (size_t)r * dk;
        for (int i = 0; i < dk; ++i) qr[i] = q[(size_t)r * dk + i], kr[i] = k[(size_t)r * dk + i];
        if (use_l2) l2norm_d(qr, dk), l2norm_d(kr, dk);
        for (int i = 0; i < dk; ++i) qr[i] *= scale;
    }
}

EXPORT void orc_recurrent_gated_delta_rule(const float* q, const float* k, const float* v, const float* g,
                                           const float* beta, int B, int T, int Hk, int Hv, int dk, int dv,
                                           const float* initial_state, int use_qk_l2norm, float scale, float* o,
                                           float* final_state) {
    const double sc = scale > 0.f ? (double)scale : 1.0 / sqrt((double)dk);
    const int rep = Hv / Hk;
    double* qn = (double*)malloc(sizeof(double) * (size_t)B * T * Hk * dk);
    double* kn = (double*)malloc(sizeof(double) * (size_t)B * T * Hk * dk);
    prep_qk_d(q, k, B * T * Hk, dk, use_qk_l2norm, sc, qn, kn);
#pragma omp parallel for collapse(2) schedule(static)
    for (int b = 0; b < B; ++b) {
        for (int h = 0; h < Hv; ++h) {
            const int kh = orc_khead_of_vhead(h, Hv, Hk);
            const size_t sz = (size_t)dk * dv;
            double* S = (double*)malloc(sizeof(double) * sz);
            double* vd = (double*)malloc(sizeof(double) * (size_t)T * dv);
            double* gd = (double*)malloc(sizeof(double) * T);
            double* bd = (double*)malloc(sizeof(double) * T);
            double* od = (double*)malloc(sizeof(double) * (size_t)T * dv);
            const size_t s_off = ((size_t)b * Hv + h) * sz;
            for (size_t i = 0; i < sz; ++i) S[i] = initial_state ? initial_state[s_off + i] : 0.0;
            for (int t = 0; t < T; ++t) {
                const size_t row = (size_t)b * T + t;
                for (int j = 0; j < dv; ++j) vd[(size_t)t * dv + j] = v[(row * Hv + h) * dv + j];
                gd[t] = g[row * Hv + h];
                bd[t] = beta[row * Hv + h];
            }
            (void)rep;
            recurrent_head_d(qn + ((size_t)b * T * Hk + kh) * dk, kn + ((size_t)b * T * Hk + kh) * dk,
                             (size_t)Hk * dk, vd, (size_t)dv, gd, bd, 1, T, dk, dv, S, od, (size_t)dv);
            for (int t = 0; t < T; ++t)
                for (int j = 0; j < dv; ++j) o[(((size_t)b * T + t) * Hv + h) * dv + j] = (float)od[(size_t)t * dv + j];
            if (final_state)
                for (size_t i = 0; i < sz; ++i) final_state[s_off + i] = (float)S[i];
            free(S), free(vd), free(gd), free(bd), free(od);
        }
    }
    free(qn), free(kn);
}

/* ------------------------------------------------------------------------------------------------ */
/* Gated delta rule, chunked (WY / UT) form, chunk C.  HF:248-328 (torch_chunk_gated_delta_rule).      */
/* Same arguments as the sequential form.  Per chunk, with G = in-chunk cumsum(g):                     */
/*   A_ij = -beta_i k_i.k_j exp(G_i - G_j) (i > j);  T = (I - A)^-1 by forward substitution (HF:294-298)*/
/*   U = T (beta v);  W = T (beta k exp(G));  Vn = U - W S;                                             */
/*   O = (q exp(G)) S + ((q k^T) o Gamma, lower incl. diag) Vn;                                         */
/*   S <- exp(G_last) S + (k exp(G_last - G))^T Vn                                                      */
/* The tail chunk is zero-padded as in HF:268-276 (padded rows have beta = 0, g = 0).                   */
/* ------------------------------------------------------------------------------------------------ */
EXPORT void orc_chunk_gated_delta_rule(const float* q, const float* k, const float* v, const float* g,
                                       const float* beta, int B, int T, int Hk, int Hv, int dk, int dv,
                                       const float* initial_state, int use_qk_l2norm, float scale, int chunk,
                                       float* o, float* final_state) {
    const double sc = scale > 0.f ? (double)scale : 1.0 / sqrt((double)dk);
    const int C = chunk;
    const int nchunks = (T + C - 1) / C;
    double* qn = (double*)malloc(sizeof(double) * (size_t)B * T * Hk * dk);
    double* kn = (double*)malloc(sizeof(double) * (size_t)B * T * Hk * dk);
    prep_qk_d(q, k, B * T * Hk, dk, use_qk_l2norm, sc, qn, kn);
#pragma omp parallel for collapse(2) schedule(static)
    for (int b = 0; b < B; ++b) {
        for (int h = 0; h < Hv; ++h) {
            const int kh = orc_khead_of_vhead(h, Hv, Hk);
            const size_t sz = (size_t)dk * dv;
            double* S = (double*)malloc(sizeof(double) * sz);
            double* Q = (double*)calloc((size_t)C * dk, sizeof(double));
            double* K = (double*)calloc((size_t)C * dk, sizeof(double));
            double* V = (double*)calloc((size_t)C * dv, sizeof(double));
            double* Bt = (double*)calloc(C, sizeof(double));
            double* G = (double*)calloc(C, sizeof(double));
            double* A = (double*)calloc((size_t)C * C, sizeof(double));
            double* U = (double*)calloc((size_t)C * dv, sizeof(double));
            double* W = (double*)calloc((size_t)C * dk, sizeof(double));
            double* Vn = (double*)calloc((size_t)C * dv, sizeof(double));
            double* Oc = (double*)calloc((size_t)C * dv, sizeof(double));
            const size_t s_off = ((size_t)b * Hv + h) * sz;
            for (size_t i = 0; i < sz; ++i) S[i] = initial_state ? initial_state[s_off + i] : 0.0;
            for (int c = 0; c < nchunks; ++c) {
                /* load the chunk, zero-padded */
                for (int i = 0; i < C; ++i) {
                    const int t = c * C + i;
                    const int valid = t < T;
                    const size_t row = (size_t)b * T + (valid ? t : 0);
                    for (int d = 0; d < dk; ++d) {
                        Q[(size_t)i * dk + d] = valid ? qn[(row * Hk + kh) * dk + d] : 0.0;
                        K[(size_t)i * dk + d] = valid ? kn[(row * Hk + kh) * dk + d] : 0.0;
                    }
                    for (int d = 0; d < dv; ++d) V[(size_t)i * dv + d] = valid ? v[(row * Hv + h) * dv + d] : 0.0;
                    Bt[i] = valid ? beta[row * Hv + h] : 0.0;
                    G[i] = (valid ? g[row * Hv + h] : 0.0) + (i ? G[i - 1] : 0.0); /* in-chunk cumsum */
                }
                /* A strictly lower: -(beta_i k_i . k_j) exp(G_i - G_j) */
                for (int i = 0; i < C; ++i)
                    for (int j = 0; j < C; ++j) {
                        double a = 0.0;
                        if (j < i) {
                            double dot = 0.0;
                            for (int d = 0; d < dk; ++d) dot += K[(size_t)i * dk + d] * K[(size_t)j * dk + d];
                            a = -(Bt[i] * dot) * exp(G[i] - G[j]);
                        }
                        A[(size_t)i * C + j] = a;
                    }
                /* forward substitution, row by row as in HF:294-298, then + I */
                for (int i = 1; i < C; ++i) {
                    double row[256];
                    for (int j = 0; j < i; ++j) {
                        double s = A[(size_t)i * C + j];
                        for (int m = 0; m < i; ++m) s += A[(size_t)i * C + m] * A[(size_t)m * C + j];
                        row[j] = s;
                    }
                    for (int j = 0; j < i; ++j) A[(size_t)i * C + j] = row[j];
                }
                for (int i = 0; i < C; ++i) A[(size_t)i * C + i] += 1.0;
                /* U = T (beta v), W = T (beta k exp(G)) */
                for (int i = 0; i < C; ++i) {
                    for (int d = 0; d < dv; ++d) {
                        double s = 0.0;
                        for (int j = 0; j <= i; ++j) s += A[(size_t)i * C + j] * Bt[j] * V[(size_t)j * dv + d];
                        U[(size_t)i * dv + d] = s;
                    }
                    for (int d = 0; d < dk; ++d) {
                        double s = 0.0;
                        for (int j = 0; j <= i; ++j)
                            s += A[(size_t)i * C + j] * Bt[j] * K[(size_t)j * dk + d] * exp(G[j]);
                        W[(size_t)i * dk + d] = s;
                    }
                }
                /* Vn = U - W S */
                for (int i = 0; i < C; ++i)
                    for (int d = 0; d < dv; ++d) {
                        double s = 0.0;
                        for (int e = 0; e < dk; ++e) s += W[(size_t)i * dk + e] * S[(size_t)e * dv + d];
                        Vn[(size_t)i * dv + d] = U[(size_t)i * dv + d] - s;
                    }
                /* O = (q exp(G)) S + (q k^T o Gamma, lower incl. diag) Vn */
                for (int i = 0; i < C; ++i) {
                    const double eg = exp(G[i]);
                    for (int d = 0; d < dv; ++d) {
                        double s = 0.0;
                        for (int e = 0; e < dk; ++e) s += Q[(size_t)i * dk + e] * eg * S[(size_t)e * dv + d];
                        Oc[(size_t)i * dv + d] = s;
                    }
                    for (int j = 0; j <= i; ++j) {
                        double dot = 0.0;
                        for (int e = 0; e < dk; ++e) dot += Q[(size_t)i * dk + e] * K[(size_t)j * dk + e];
                        const double a = dot * exp(G[i] - G[j]);
                        for (int d = 0; d < dv; ++d) Oc[(size_t)i * dv + d] += a * Vn[(size_t)j * dv + d];
                    }
                }
                /* S <- exp(G_last) S + (k exp(G_last - G))^T Vn */
                const double gl = G[C - 1];
                const double el = exp(gl);
                for (size_t i = 0; i < sz; ++i) S[i] *= el;
                for (int j = 0; j < C; ++j) {
                    const double f = exp(gl - G[j]);
                    for (int e = 0; e < dk; ++e) {
                        const double kf = K[(size_t)j * dk + e] * f;
                        for (int d = 0; d < dv; ++d) S[(size_t)e * dv + d] += kf * Vn[(size_t)j * dv + d];
                    }
                }
                for (int i = 0; i < C; ++i) {
                    const int t = c * C + i;
                    if (t >= T) break;
                    for (int d = 0; d < dv; ++d)
                        o[((((size_t)b * T + t) * Hv) + h) * dv + d] = (float)Oc[(size_t)i * dv + d];
                }
            }
            if (final_state)
                for (size_t i = 0; i < sz; ++i) final_state[s_off + i] = (float)S[i];
            free(S), free(Q), free(K), free(V), free(Bt), free(G), free(A), free(U), free(W), free(Vn), free(Oc);
        }
    }
    free(qn), free(kn);
}

/* ------------------------------------------------------------------------------------------------ */
/* Gated RMSNorm over each head: y = o * rsqrt(mean(o^2) + eps) * w * silu(z).                        */
/* HF:167-184 (Qwen3_5RMSNormGated); 9B/kernels/layer_compute.cpp:287-395 (C6).  rows x dv.           */
/* ------------------------------------------------------------------------------------------------ */
static void gated_rmsnorm_d(const double* o, const double* z, int rows, int dv, const float* w, double eps,
                            double* y) {
#pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; ++r) {
        const double* orow = o + (size_t)r * dv;
        const double* zrow = z + (size_t)r * dv;
        double ss = 0.0;
        for (int j = 0; j < dv; ++j) ss += orow[j] * orow[j];
        const double rstd = 1.0 / sqrt(ss / dv + eps);
        for (int j = 0; j < dv; ++j) y[(size_t)r * dv + j] = orow[j] * rstd * (double)w[j] * silu_d(zrow[j]);
    }
}

EXPORT void orc_gated_rmsnorm(const float* o, const float* z, int rows, int dv, const float* w, float eps, float* y) {
    const size_t n = (size_t)rows * dv;
    double* od = (double*)malloc(n * sizeof(double));
    double* zd = (double*)malloc(n * sizeof(double));
    double* yd = (double*)malloc(n * sizeof(double));
    for (size_t i = 0; i < n; ++i) od[i] = o[i], zd[i] = z[i];
    gated_rmsnorm_d(od, zd, rows, dv, w, (double)eps, yd);
    for (size_t i = 0; i < n; ++i) y[i] = (float)yd[i];
    free(od), free(zd), free(yd);
}

/* ------------------------------------------------------------------------------------------------ */
/* Front end after the conv: l2norm + scale of q/k, gating scalars.                                   */
/*   g = -exp(A_log[h]) softplus(a + dt_bias[h]) (threshold 20), beta = sigmoid(b)                     */
/* HF:497-499; 9B/kernels/layer_compute.cpp:148-199 (C3); reference.py:7-8,17-24.                      */
/* qkv: [M, conv_dim] post-conv (q | k | v); ab: a at column a_col, b at b_col of rows of ab_stride.    */
/* Outputs qn, kn [M, nk, dk] (qn scaled by dk^-0.5), v [M, nv, dv], g, beta [M, nv].                   */
/* ------------------------------------------------------------------------------------------------ */
typedef struct orc_dims {
    int hidden, nk, nv, dk, dv, kconv;
    float eps;
} orc_dims;

static void front_d(const orc_dims* dm, int M, const double* qkv, size_t qkv_stride, const double* ab,
                    size_t ab_stride, const float* A_log, const float* dt_bias, double* qn, double* kn, double* vv,
                    double* g, double* beta) {
    const int nk = dm->nk, nv = dm->nv, dk = dm->dk, dv = dm->dv;
    const int Kd = nk * dk;
    const double sc = 1.0 / sqrt((double)dk);
#pragma omp parallel for schedule(static)
    for (int m = 0; m < M; ++m) {
        const double* row = qkv + (size_t)m * qkv_stride;
        for (int h = 0; h < nk; ++h) {
            double* qr = qn + ((size_t)m * nk + h) * dk;
            double* kr = kn + ((size_t)m * nk + h) * dk;
            for (int i = 0; i < dk; ++i) qr[i] = row[h * dk + i], kr[i] = row[Kd + h * dk + i];
            l2norm_d(qr, dk), l2norm_d(kr, dk);
            for (int i = 0; i < dk; ++i) qr[i] *= sc;
        }
        for (int j = 0; j < nv * dv; ++j) vv[(size_t)m * nv * dv + j] = row[2 * Kd + j];
        const double* abr = ab + (size_t)m * ab_stride;
        for (int h = 0; h < nv; ++h) {
            const double a = abr[h], bb = abr[nv + h];
            g[(size_t)m * nv + h] = -exp((double)A_log[h]) * softplus_t20(a + (double)dt_bias[h]);
            beta[(size_t)m * nv + h] = sigmoid_d(bb);
        }
    }
}

/* ------------------------------------------------------------------------------------------------ */
/* Whole layer, one launch of B sequences x T tokens, continuing from (rec_state, conv_state).         */
/* 9B/gdn_layer.py:244-292 (_forward_rows / __call__), HF:432-543 (forward).                           */
/*   x [B,T,H] -> P = x [W_qkv; W_z; W_a; W_b]^T -> conv+SiLU(q|k|v) -> front -> sequential rule       */
/*   -> gated RMSNorm(o, z) -> out = y W_out^T                                                          */
/* rec_state [B,nv,dk,dv], conv_state [B,conv_dim,3] time order, both in/out.                           */
/* Optional taps (may be NULL): y_out [B*T, nv*dv] (norm output), o_out [B*T, nv*dv] (rule output).     */
/* ------------------------------------------------------------------------------------------------ */
EXPORT void orc_layer_forward(const orc_dims* dm, const float* w_qkv, const float* w_z, const float* w_a,
                              const float* w_b, const float* conv_w, const float* A_log, const float* dt_bias,
                              const float* norm_w, const float* w_out, const float* x, int B, int T,
                              float* rec_state, float* conv_state, float* out, float* y_out, float* o_out) {
    const int H = dm->hidden, nk = dm->nk, nv = dm->nv, dk = dm->dk, dv = dm->dv;
    const int Kd = nk * dk, Vd = nv * dv, CD = 2 * Kd + Vd;
    const int M = B * T;
    double* xd = (double*)malloc(sizeof(double) * (size_t)M * H);
    for (size_t i = 0; i < (size_t)M * H; ++i) xd[i] = x[i];
    double* qkv = (double*)malloc(sizeof(double) * (size_t)M * CD);
    double* z = (double*)malloc(sizeof(double) * (size_t)M * Vd);
    double* ab = (double*)malloc(sizeof(double) * (size_t)M * 2 * nv);
    double* a_tmp = (double*)malloc(sizeof(double) * (size_t)M * nv);
    linear_d(xd, w_qkv, M, CD, H, qkv);
    linear_d(xd, w_z, M, Vd, H, z);
    linear_d(xd, w_a, M, nv, H, a_tmp);
    for (int m = 0; m < M; ++m)
        for (int h = 0; h < nv; ++h) ab[(size_t)m * 2 * nv + h] = a_tmp[(size_t)m * nv + h];
    linear_d(xd, w_b, M, nv, H, a_tmp);
    for (int m = 0; m < M; ++m)
        for (int h = 0; h < nv; ++h) ab[(size_t)m * 2 * nv + nv + h] = a_tmp[(size_t)m * nv + h];
    free(a_tmp);

    /* conv + SiLU over all conv_dim channels, history in double */
    double* hist = (double*)malloc(sizeof(double) * (size_t)B * CD * 3);
    for (size_t i = 0; i < (size_t)B * CD * 3; ++i) hist[i] = conv_state[i];
    double* cv = (double*)malloc(sizeof(double) * (size_t)M * CD);
    conv_silu_d(qkv, B, T, CD, (size_t)CD, conv_w, hist, cv, (size_t)CD);
    for (size_t i = 0; i < (size_t)B * CD * 3; ++i) conv_state[i] = (float)hist[i];
    free(hist);

    double* qn = (double*)malloc(sizeof(double) * (size_t)M * Kd);
    double* kn = (double*)malloc(sizeof(double) * (size_t)M * Kd);
    double* vv = (double*)malloc(sizeof(double) * (size_t)M * Vd);
    double* g = (double*)malloc(sizeof(double) * (size_t)M * nv);
    double* beta = (double*)malloc(sizeof(double) * (size_t)M * nv);
    front_d(dm, M, cv, (size_t)CD, ab, (size_t)2 * nv, A_log, dt_bias, qn, kn, vv, g, beta);

    double* o = (double*)malloc(sizeof(double) * (size_t)M * Vd);
#pragma omp parallel for collapse(2) schedule(static)
    for (int b = 0; b < B; ++b) {
        for (int h = 0; h < nv; ++h) {
            const int kh = orc_khead_of_vhead(h, nv, nk);
            const size_t sz = (size_t)dk * dv;
            double* S = (double*)malloc(sizeof(double) * sz);
            const size_t s_off = ((size_t)b * nv + h) * sz;
            for (size_t i = 0; i < sz; ++i) S[i] = rec_state[s_off + i];
            const size_t r0 = (size_t)b * T;
            recurrent_head_d(qn + (r0 * nk + kh) * dk, kn + (r0 * nk + kh) * dk, (size_t)nk * dk,
                             vv + (r0 * nv + h) * dv, (size_t)Vd, g + r0 * nv + h, beta + r0 * nv + h, (size_t)nv,
                             T, dk, dv, S, o + r0 * Vd + (size_t)h * dv, (size_t)Vd);
            for (size_t i = 0; i < sz; ++i) rec_state[s_off + i] = (float)S[i];
            free(S);
        }
    }
    if (o_out)
        for (size_t i = 0; i < (size_t)M * Vd; ++i) o_out[i] = (float)o[i];

    double* y = (double*)malloc(sizeof(double) * (size_t)M * Vd);
    gated_rmsnorm_d(o, z, M * nv, dv, norm_w, (double)dm->eps, y);
    if (y_out)
        for (size_t i = 0; i < (size_t)M * Vd; ++i) y_out[i] = (float)y[i];
    double* od = (double*)malloc(sizeof(double) * (size_t)M * H);
    linear_d(y, w_out, M, H, Vd, od);
    for (size_t i = 0; i < (size_t)M * H; ++i) out[i] = (float)od[i];

    free(xd), free(qkv), free(z), free(ab), free(cv), free(qn), free(kn), free(vv), free(g), free(beta), free(o),
        free(y), free(od);
}

/* Front end of one launch as an op: conv + SiLU + l2norm + gating from a fused projection row
 * P [M, conv_dim + Vd + 2 nv] (q | k | v | z | a | b), with conv history [B, conv_dim, 3] in/out.
 * Outputs qn, kn [M,nk,dk], v [M,nv,dv], g, beta [M,nv].  Composition of 9B/kernels/layer_compute.cpp
 * C1-C3 (74-199) with layer_reader.cpp:103-124,184-197. */
EXPORT void orc_conv_front(const orc_dims* dm, const float* P, int B, int T, const float* conv_w, const float* A_log,
                           const float* dt_bias, float* conv_state, float* qn_out, float* kn_out, float* v_out,
                           float* g_out, float* beta_out) {
    const int nk = dm->nk, nv = dm->nv, dk = dm->dk, dv = dm->dv;
    const int Kd = nk * dk, Vd = nv * dv, CD = 2 * Kd + Vd, NP = CD + Vd + 2 * nv;
    const int M = B * T;
    double* pd = (double*)malloc(sizeof(double) * (size_t)M * NP);
    for (size_t i = 0; i < (size_t)M * NP; ++i) pd[i] = P[i];
    double* hist = (double*)malloc(sizeof(double) * (size_t)B * CD * 3);
    for (size_t i = 0; i < (size_t)B * CD * 3; ++i) hist[i] = conv_state[i];
    double* cv = (double*)malloc(sizeof(double) * (size_t)M * CD);
    conv_silu_d(pd, B, T, CD, (size_t)NP, conv_w, hist, cv, (size_t)CD);
    for (size_t i = 0; i < (size_t)B * CD * 3; ++i) conv_state[i] = (float)hist[i];
    double* qn = (double*)malloc(sizeof(double) * (size_t)M * Kd);
    double* kn = (double*)malloc(sizeof(double) * (size_t)M * Kd);
    double* vv = (double*)malloc(sizeof(double) * (size_t)M * Vd);
    double* g = (double*)malloc(sizeof(double) * (size_t)M * nv);
    double* beta = (double*)malloc(sizeof(double) * (size_t)M * nv);
    front_d(dm, M, cv, (size_t)CD, pd + CD + Vd, (size_t)NP, A_log, dt_bias, qn, kn, vv, g, beta);
    for (size_t i = 0; i < (size_t)M * Kd; ++i) qn_out[i] = (float)qn[i], kn_out[i] = (float)kn[i];
    for (size_t i = 0; i < (size_t)M * Vd; ++i) v_out[i] = (float)vv[i];
    for (size_t i = 0; i < (size_t)M * nv; ++i) g_out[i] = (float)g[i], beta_out[i] = (float)beta[i];
    free(pd), free(hist), free(cv), free(qn), free(kn), free(vv), free(g), free(beta);
}

/* ---- low-precision weights: E4M3 with one scale per output row -----------------------------------
 * The reference stores w_in and w_out in its weight_dtype (9B/gdn_layer.py:55, 115-120: ttnn.bfloat16 or
 * ttnn.bfloat8_b; w_ab stays bfloat16; 0.8B/gdn_l1.py:79-80).  bfloat8_b is a shared-exponent tile format
 * with no MI355X counterpart; the HIP path stores those matrices as OCP 8-bit floating point E4M3
 * (OCP 8-bit Floating Point Specification v1.0, 2023: 1 sign bit, 4 exponent bits with bias 7, 3
 * mantissa bits; no infinities; S.1111.111 is NaN; largest finite 448; subnormals m 2^-9) with
 * scale[n] = max_k |w[n, k]| / 448 (1 for an all-zero row) and code = nearest E4M3 value of w / scale,
 * ties to the even mantissa, saturating at +-448.  Dequantized weight = value(code) * scale.
 * Restated here from the specification: decode by the closed form, encode by exhaustive nearest search
 * over the 127 non-negative finite values (an independent route from the HIP path's bit arithmetic). */
EXPORT double orc_e4m3_value(int code) {
    const int s = (code >> 7) & 1, e = (code >> 3) & 15, m = code & 7;
    if (e == 15 && m == 7) return NAN;
    const double mag = e == 0 ? ldexp((double)m, -9) : ldexp(1.0 + m / 8.0, e - 7);
    return s ? -mag : mag;
}

EXPORT int orc_e4m3_encode(float v) {
    const double a = fmin(fabs((double)v), 448.0);
    int best = 0;
    double dbest = INFINITY;
    for (int c = 0; c <= 0x7e; ++c) {  /* codes 0..126 are the non-negative finite values, ascending */
        const double d = fabs(orc_e4m3_value(c) - a);
        if (d < dbest || (d == dbest && (c & 1) == 0)) best = c, dbest = d;
    }
    return (signbit(v) ? 0x80 : 0) | best;
}

EXPORT void orc_quantize_e4m3(const float* w, int N, int K, uint8_t* q, float* scale) {
#pragma omp parallel for schedule(static)
    for (int n = 0; n < N; ++n) {
        float m = 0.f;
        for (int k = 0; k < K; ++k) m = fmaxf(m, fabsf(w[(size_t)n * K + k]));
        const float s = m > 0.f ? m / 448.0f : 1.0f;
        scale[n] = s;
        for (int k = 0; k < K; ++k) q[(size_t)n * K + k] = (uint8_t)orc_e4m3_encode(w[(size_t)n * K + k] / s);
    }
}

/* ---- low-precision weights: MXFP4 (E2M1 elements, one E8M0 scale per 32 along K) ----------------------
 * The reference's other weight_dtype, ttnn.bfloat4_b (0.8B/gdn_l1.py:79-80; 0.8B/test_gdn_l1.py:88-92 runs
 * six resident layers in it), is a shared-exponent tile format with no MI355X counterpart; the HIP path
 * stores w_in (q|k|v|z rows) and w_out as OCP MXFP4 (OCP Microscaling Formats Specification v1.0, 2023):
 * blocks of 32 consecutive values of a row share the scale X = 2^(floor(log2(amax)) - 2) (emax of E2M1 is
 * 2; X stored as its E8M0 exponent byte, bias 127, the exponent clamped to [-127, 127]; an all-zero block
 * takes code 0), and each value is the FP4 E2M1 code nearest to w / X (1 sign bit, 2 exponent bits with
 * bias 1, 1 mantissa bit: 0, 0.5, 1, 1.5, 2, 3, 4, 6), ties to the even mantissa, saturating at +-6.
 * Dequantized weight = value(code) * X.  Restated from the specification: decode by the closed form,
 * encode by exhaustive nearest search over the eight magnitudes, the exponent by frexp. */
EXPORT double orc_e2m1_value(int code) {
    const int s = (code >> 3) & 1, e = (code >> 1) & 3, m = code & 1;
    const double mag = e == 0 ? 0.5 * m : ldexp(1.0 + 0.5 * m, e - 1);
    return s ? -mag : mag;
}

EXPORT int orc_e2m1_encode(float v) {
    const double a = fmin(fabs((double)v), 6.0);
    int best = 0;
    double dbest = INFINITY;
    for (int c = 0; c < 8; ++c) {  /* codes 0..7 are the non-negative values, ascending */
        const double d = fabs(orc_e2m1_value(c) - a);
        if (d < dbest || (d == dbest && (c & 1) == 0)) best = c, dbest = d;
    }
    return (signbit(v) ? 8 : 0) | best;
}

/* E8M0 exponent byte of the block scale for a block whose largest magnitude is amax */
EXPORT int orc_mx_scale_code(float amax) {
    if (!(amax > 0.f)) return 0;
    int e2;
    frexp((double)amax, &e2);   /* amax = f 2^e2, f in [0.5, 1): floor(log2 amax) = e2 - 1 */
    int x = e2 - 1 - 2;
    if (x < -127) x = -127;
    if (x > 127) x = 127;
    return x + 127;
}

/* w [N, K] (K % 32 == 0) -> codes [N, K] (one E2M1 code per byte, unpacked) and scale codes [N, K / 32] */
EXPORT void orc_quantize_mxfp4(const float* w, int N, int K, uint8_t* q, uint8_t* sc) {
#pragma omp parallel for schedule(static)
    for (int n = 0; n < N; ++n)
        for (int kb = 0; kb < K / 32; ++kb) {
            const float* b = w + (size_t)n * K + 32 * kb;
            float m = 0.f;
            for (int j = 0; j < 32; ++j) m = fmaxf(m, fabsf(b[j]));
            const int code = orc_mx_scale_code(m);
            sc[(size_t)n * (K / 32) + kb] = (uint8_t)code;
            const double X = ldexp(1.0, code - 127);
            for (int j = 0; j < 32; ++j) q[(size_t)n * K + 32 * kb + j] = (uint8_t)orc_e2m1_encode((float)(b[j] / X));
        }
}

/* ---- low-precision weights: MXINT8 (int8 elements worth code * 2^-6, one E8M0 scale per 32 along K) ------
 * The counterpart of the reference's ttnn.bfloat8_b (9B/gdn_layer.py:55,115-120; the default weight_dtype of
 * the 0.8B stack, 0.8B/gdn_l1.py:153), a shared-exponent tile format that keeps 7 significant bits per value.
 * The HIP path stores w_in (q|k|v|z rows) and w_out as OCP MXINT8 (OCP Microscaling Formats Specification
 * v1.0, 2023): blocks of 32 consecutive values of a row share the scale X = 2^(floor(log2(amax)) - emax) with
 * emax = 0 (the largest power of two of the element format, whose values are code * 2^-6 for two's-complement
 * codes in [-128, 127]); X is stored as its E8M0 exponent byte (bias 127, exponent clamped to [-127, 127], code
 * 0 for an all-zero block) and each value as the code nearest to w / X, ties to the even code, saturated to
 * [-128, 127].  Dequantized weight = code * 2^-6 * X.  Restated from the specification: the exponent by frexp,
 * the code by a nearest search over the candidate codes around 64 w / X with explicit tie-breaking. */
EXPORT int orc_mx_scale_code_emax(float amax, int emax) {
    if (!(amax > 0.f)) return 0;
    int e2;
    frexp((double)amax, &e2);   /* amax = f 2^e2, f in [0.5, 1): floor(log2 amax) = e2 - 1 */
    int x = e2 - 1 - emax;
    if (x < -127) x = -127;
    if (x > 127) x = 127;
    return x + 127;
}

EXPORT int orc_mxint8_encode(double v) {
    /* v is already divided by the block scale; the element value of code c is c / 64 */
    const double t = fmin(fmax(v * 64.0, -256.0), 256.0);  /* beyond the codes: saturates either way */
    int lo = (int)floor(t) - 1, best = 0;
    double dbest = INFINITY;
    for (int c = lo; c <= lo + 3; ++c) {
        const int cc = c < -128 ? -128 : (c > 127 ? 127 : c);
        const double d = fabs(cc / 64.0 - v);
        if (d < dbest || (d == dbest && (cc & 1) == 0 && (best & 1) != 0)) best = cc, dbest = d;
    }
    return best;
}

/* w [N, K] (K % 32 == 0) -> codes [N, K] (int8) and scale codes [N, K / 32] */
EXPORT void orc_quantize_mxint8(const float* w, int N, int K, int8_t* q, uint8_t* sc) {
#pragma omp parallel for schedule(static)
    for (int n = 0; n < N; ++n)
        for (int kb = 0; kb < K / 32; ++kb) {
            const float* b = w + (size_t)n * K + 32 * kb;
            float m = 0.f;
            for (int j = 0; j < 32; ++j) m = fmaxf(m, fabsf(b[j]));
            const int code = orc_mx_scale_code_emax(m, 0);
            sc[(size_t)n * (K / 32) + kb] = (uint8_t)code;
            const double X = ldexp(1.0, code - 127);
            for (int j = 0; j < 32; ++j) q[(size_t)n * K + 32 * kb + j] = (int8_t)orc_mxint8_encode(b[j] / X);
        }
}
