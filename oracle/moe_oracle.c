/*
 * moe_oracle.c -- CPU restatement of the reference C port's MoE layer.
 * TEST INFRASTRUCTURE ONLY (see moe_oracle.h for scope, citations and the
 * deliberate departures).  Built with -ffp-contract=off: every fused
 * multiply-add below is an explicit fmaf(), so the arithmetic is the same on
 * any x86-64 host.
 */
#define _POSIX_C_SOURCE 199309L
#include "moe_oracle.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------ bf16 */

/* c/src/util.h:56-61: widen by a 16-bit shift */
float orc_bf16_to_f32(uint16_t h) {
    uint32_t bits = (uint32_t)h << 16;
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* c/src/util.h:63-71: round to nearest even on the upper 16 bits, no NaN
 * special case */
uint16_t orc_f32_to_bf16(float f) {
    uint32_t bits;
    memcpy(&bits, &f, 4);
    uint32_t hi = bits >> 16;
    uint32_t lo = bits & 0xffffu;
    if (lo > 0x8000u || (lo == 0x8000u && (hi & 1u))) hi++;
    return (uint16_t)hi;
}

/* ----------------------------------------------------------- elementwise */

float orc_silu(float v) { return v / (1.0f + expf(-v)); }     /* kernel.c:38-43 */
float orc_sigmoid(float v) { return 1.0f / (1.0f + expf(-v)); } /* kernel.c:45-47 */

/* kernel.c:10-20 verbatim in arithmetic: sequential sum of squares,
 * r = 1/sqrt(ss/n + eps), y = x*r*w (two roundings, left to right) */
void orc_rmsnorm_seq(const float *x, const float *w, size_t n, float eps, float *y) {
    float ss = 0.0f;
    for (size_t i = 0; i < n; i++) ss = fmaf(x[i], x[i], ss);
    float r = 1.0f / sqrtf(ss / (float)n + eps);
    for (size_t i = 0; i < n; i++) y[i] = w ? (x[i] * r) * w[i] : x[i] * r;
}

/* ------------------------------------------------------------ R64 order
 * A length-K reduction is split into 8-element chunks; chunk c belongs to
 * leaf (c mod 64).  Each leaf is an fma chain over its chunks in ascending
 * order starting from +0.0f.  The 64 leaves are then combined by a
 * butterfly (p[l] += p[l^o] for o = 1,2,4,...,32), which is the pairwise
 * tree over the leaves in natural order.  A 64-lane wavefront that loads one
 * 16-byte bf16 chunk per lane and reduces across lanes in that order
 * computes exactly this value in every lane. */
static float r64_combine(float *p) {
    for (int o = 1; o <= 32; o <<= 1) {
        float q[64];
        for (int l = 0; l < 64; l++) q[l] = p[l] + p[l ^ o];
        memcpy(p, q, sizeof(q));
    }
    return p[0];
}

/* chunk c covers elements [8c, min(8c+8, K)) */
float orc_dot_r64_bf16w(const float *x, const uint16_t *w, int K) {
    float p[64];
    int chunks = (K + 7) / 8;
    for (int l = 0; l < 64; l++) {
        float acc = 0.0f;
        for (int c = l; c < chunks; c += 64)
            for (int j = 8 * c; j < 8 * c + 8 && j < K; j++)
                acc = fmaf(x[j], orc_bf16_to_f32(w[j]), acc);
        p[l] = acc;
    }
    return r64_combine(p);
}

float orc_sumsq_r64(const float *x, int K) {
    float p[64];
    int chunks = (K + 7) / 8;
    for (int l = 0; l < 64; l++) {
        float acc = 0.0f;
        for (int c = l; c < chunks; c += 64)
            for (int j = 8 * c; j < 8 * c + 8 && j < K; j++) acc = fmaf(x[j], x[j], acc);
        p[l] = acc;
    }
    return r64_combine(p);
}

/* kernel.c:10-20 with the sum of squares in R64 order */
void orc_rmsnorm_r64(const float *x, const float *w, size_t n, float eps, float *y) {
    float ss = orc_sumsq_r64(x, (int)n);
    float r = 1.0f / sqrtf(ss / (float)n + eps);
    for (size_t i = 0; i < n; i++) y[i] = w ? (x[i] * r) * w[i] : x[i] * r;
}

/* ----------------------------------------------------------------- top-k */

/* kernel.c:114-138: quickselect with the middle element as pivot, Lomuto
 * partition on strict '>' so the k largest end up in idx[0..k) */
static void quickselect_kth(const float *x, int *idx, int n, int k) {
    int lo = 0, hi = n;
    for (;;) {
        int mid = lo + (hi - lo) / 2;
        float pv = x[idx[mid]];
        int t = idx[mid];
        idx[mid] = idx[hi - 1];
        idx[hi - 1] = t;
        int store = lo;
        for (int i = lo; i < hi - 1; i++) {
            if (x[idx[i]] > pv) {
                t = idx[i];
                idx[i] = idx[store];
                idx[store] = t;
                store++;
            }
        }
        t = idx[store];
        idx[store] = idx[hi - 1];
        idx[hi - 1] = t;
        if (store == k - 1) return;
        if (store < k - 1)
            lo = store + 1;
        else
            hi = store;
    }
}

/* kernel.c:140-150 */
void orc_topk_quickselect(const float *x, int n, int k, int *out) {
    if (k >= n) {
        for (int i = 0; i < n; i++) out[i] = i;
        return;
    }
    int *idx = (int *)malloc((size_t)n * sizeof(int));
    for (int i = 0; i < n; i++) idx[i] = i;
    quickselect_kth(x, idx, n, k);
    memcpy(out, idx, (size_t)k * sizeof(int));
    free(idx);
}

/* a precedes b: larger value first, equal values (with -0 == +0) by lower id */
static int canon_before(float va, int ia, float vb, int ib) {
    if (va > vb) return 1;
    if (va < vb) return 0;
    return ia < ib;
}

/* canonical top-k: k passes of "best remaining" (value desc, id asc) */
void orc_topk_canonical(const float *x, int n, int k, int *out) {
    if (k > n) k = n;
    unsigned char *taken = (unsigned char *)calloc((size_t)n, 1);
    for (int s = 0; s < k; s++) {
        int best = -1;
        for (int i = 0; i < n; i++) {
            if (taken[i]) continue;
            if (best < 0 || canon_before(x[i] + 0.0f, i, x[best] + 0.0f, best)) best = i;
        }
        taken[best] = 1;
        out[s] = best;
    }
    free(taken);
}

/* -------------------------------------------------------------------- q4 */

/* kernel.c:152-173.  The reference writes q*s + b inside one expression;
 * Apple clang contracts it (-ffp-contract=on), so it is restated as fmaf. */
void orc_dequant_q4_f32sb(const uint32_t *q, const float *scales, const float *biases,
                          size_t rows, size_t cols, size_t group_size, float *out) {
    size_t words = cols / 8, groups = cols / group_size;
    for (size_t r = 0; r < rows; r++) {
        const uint32_t *qr = q + r * words;
        for (size_t c = 0; c < cols; c++) {
            size_t g = c / group_size;
            uint32_t v = qr[c / 8];
            float code = (float)((v >> (4 * (c % 8))) & 0xFu);
            out[r * cols + c] = fmaf(code, scales[r * groups + g], biases[r * groups + g]);
        }
    }
}

void orc_dequant_q4(const uint32_t *q, const uint16_t *scales, const uint16_t *biases,
                    size_t rows, size_t cols, size_t group_size, float *out) {
    size_t groups = cols / group_size;
    float *s = (float *)malloc(rows * groups * sizeof(float));
    float *b = (float *)malloc(rows * groups * sizeof(float));
    for (size_t i = 0; i < rows * groups; i++) {
        s[i] = orc_bf16_to_f32(scales[i]);
        b[i] = orc_bf16_to_f32(biases[i]);
    }
    orc_dequant_q4_f32sb(q, s, b, rows, cols, group_size, out);
    free(s);
    free(b);
}

/* kernel.c:181-186: C[M,N] = A[M,K] W[N,K]^T, sequential fma over k */
void orc_gemm_fp32(int M, int N, int K, const float *A, const float *W, float *C) {
    for (int m = 0; m < M; m++)
        for (int n = 0; n < N; n++) {
            float acc = 0.0f;
            for (int k = 0; k < K; k++) acc = fmaf(A[(size_t)m * K + k], W[(size_t)n * K + k], acc);
            C[(size_t)m * N + n] = acc;
        }
}

/* kernel.c:190-228 in naive form */
void orc_gemm_bf16(int M, int N, int K, const float *A, const uint16_t *W, float *C) {
    for (int m = 0; m < M; m++)
        for (int n = 0; n < N; n++) {
            float acc = 0.0f;
            for (int k = 0; k < K; k++)
                acc = fmaf(A[(size_t)m * K + k], orc_bf16_to_f32(W[(size_t)n * K + k]), acc);
            C[(size_t)m * N + n] = acc;
        }
}

/* One output of gemm_q4 (kernel.c:239-246, 289-305): per group
 * xq = sum x*q (fma chain), acc += s*xq + b*xsum.  Under Apple clang's
 * contraction the group update is acc + fma(s, xq, b*xsum). */
static float q4_row_dot(const float *a, const float *xsum, const uint32_t *w, const float *s,
                        const float *b, int K, int gs) {
    int groups = K / gs, wpg = gs / 8;
    float acc = 0.0f;
    for (int g = 0; g < groups; g++) {
        float xq = 0.0f;
        const float *ag = a + (size_t)g * gs;
        for (int wd = 0; wd < wpg; wd++) {
            uint32_t v = w[g * wpg + wd];
            for (int i = 0; i < 8; i++) xq = fmaf(ag[wd * 8 + i], (float)((v >> (4 * i)) & 0xFu), xq);
        }
        acc = acc + fmaf(s[g], xq, b[g] * xsum[g]);
    }
    return acc;
}

static void group_sums(const float *a, int K, int gs, float *xsum) {
    for (int g = 0; g < K / gs; g++) {
        float s = 0.0f;
        for (int i = 0; i < gs; i++) s += a[(size_t)g * gs + i];
        xsum[g] = s;
    }
}

void orc_gemm_q4_f32sb(int M, int N, int K, const float *A, const uint32_t *W,
                       const float *scales, const float *biases, int group_size, float *C) {
    if (M <= 0 || N <= 0) return;
    int groups = K / group_size;
    float *xsum = (float *)malloc((size_t)groups * sizeof(float));
    for (int m = 0; m < M; m++) {
        const float *a = A + (size_t)m * K;
        group_sums(a, K, group_size, xsum);
        for (int n = 0; n < N; n++)
            C[(size_t)m * N + n] = q4_row_dot(a, xsum, W + (size_t)n * (K / 8),
                                              scales + (size_t)n * groups,
                                              biases + (size_t)n * groups, K, group_size);
    }
    free(xsum);
}

void orc_gemm_q4(int M, int N, int K, const float *A, const uint32_t *W,
                 const uint16_t *scales, const uint16_t *biases, int group_size, float *C) {
    size_t ng = (size_t)N * (K / group_size);
    float *s = (float *)malloc(ng * sizeof(float));
    float *b = (float *)malloc(ng * sizeof(float));
    for (size_t i = 0; i < ng; i++) {
        s[i] = orc_bf16_to_f32(scales[i]);
        b[i] = orc_bf16_to_f32(biases[i]);
    }
    orc_gemm_q4_f32sb(M, N, K, A, W, s, b, group_size, C);
    free(s);
    free(b);
}

/* ------------------------------------------------------- hyper connection */

/* kernel.c:22-36 (groups of `group` with weight w[(g % per_row) * group..]);
 * the sum of squares contracts to an fma chain as kernel_rmsnorm's does */
static void rmsnorm_grouped(const float *x, const float *w, size_t total, size_t group, size_t rows,
                            float eps, float *y) {
    const size_t groups = total / group, per_row = rows ? groups / rows : groups;
    for (size_t g = 0; g < groups; g++) {
        const float *xg = x + g * group;
        float ss = 0.0f;
        for (size_t i = 0; i < group; i++) ss = fmaf(xg[i], xg[i], ss);
        const float r = 1.0f / sqrtf(ss / (float)group + eps);
        const float *wg = w ? w + (g % per_row) * group : NULL;
        for (size_t i = 0; i < group; i++) y[g * group + i] = xg[i] * r * (wg ? wg[i] : 1.0f);
    }
}

int orc_hc_mix(const orc_hc *H, const float *hyper, int n, float *mixed, float *inject,
               float *normed_out) {
    const int hc = H->hc, d = H->d, R = H->lowrank, hd = hc * d;
    if (n <= 0) return 0;
    float *normed = (float *)malloc((size_t)n * hd * sizeof(float));
    float *w = (float *)malloc((size_t)n * R * sizeof(float));
    float *tmp = (float *)malloc((size_t)n * hd * sizeof(float));
    if (!normed || !w || !tmp) {
        free(normed);
        free(w);
        free(tmp);
        return -1;
    }
    rmsnorm_grouped(hyper, H->hc_norm, (size_t)n * hd, (size_t)d, (size_t)n, 1e-6f, normed);
    /* w = silu(down(normed) / hc) (model.c:755-758) */
    orc_gemm_q4(n, R, hd, normed, H->down_q, H->down_s, H->down_b, H->group_size, w);
    for (size_t i = 0; i < (size_t)n * R; i++) w[i] = orc_silu(w[i] * (1.0f / hc));
    /* tmp = sigmoid(up(w)) (model.c:760-761) */
    orc_gemm_q4(n, hd, R, w, H->up_q, H->up_s, H->up_b, H->group_size, tmp);
    for (size_t i = 0; i < (size_t)n * hd; i++) tmp[i] = orc_sigmoid(tmp[i]);
    /* mixed = mean over hc of tmp * normed (model.c:776-785) */
    for (int t = 0; t < n; t++)
        for (int i = 0; i < d; i++) {
            float acc = 0.0f;
            for (int h = 0; h < hc; h++)
                acc = fmaf(tmp[(size_t)t * hd + (size_t)h * d + i], normed[(size_t)t * hd + (size_t)h * d + i],
                           acc);
            mixed[(size_t)t * d + i] = acc / (float)hc;
        }
    /* inject = 2 * sigmoid(block_inject(normed) / hc) (model.c:787-793) */
    if (inject) {
        orc_gemm_bf16(n, hc, hd, normed, H->inject_w, inject);
        for (size_t i = 0; i < (size_t)n * hc; i++)
            inject[i] = 2.0f * orc_sigmoid(inject[i] * (1.0f / hc));
    }
    if (normed_out) memcpy(normed_out, normed, (size_t)n * hd * sizeof(float));
    free(normed);
    free(w);
    free(tmp);
    return 0;
}

void orc_hc_inject(int hc, int d, int n, const float *inject, const float *out, float *hyper) {
    for (int t = 0; t < n; t++)
        for (int hh = 0; hh < hc; hh++) {
            const float inj = inject[(size_t)t * hc + hh];
            for (int j = 0; j < d; j++)
                hyper[((size_t)t * hc + hh) * d + j] =
                    fmaf(inj, out[(size_t)t * d + j], hyper[((size_t)t * hc + hh) * d + j]);
        }
}

/* -------------------------------------------------------------- dispatch */

/* Stable counting sort of flat slots f = t*k + s by expert id.  Because the
 * k experts of one token are distinct, "t ascending within an expert" and
 * "f ascending within an expert" are the same order. */
int orc_dispatch(const int *idx, int n, int k, int E, int *offsets, int *perm, int *pos,
                 int *active) {
    int *cnt = (int *)calloc((size_t)E + 1, sizeof(int));
    for (int f = 0; f < n * k; f++) cnt[idx[f]]++;
    offsets[0] = 0;
    for (int e = 0; e < E; e++) offsets[e + 1] = offsets[e] + cnt[e];
    int na = 0;
    for (int e = 0; e < E; e++)
        if (cnt[e]) active[na++] = e;
    memcpy(cnt, offsets, (size_t)E * sizeof(int));
    for (int f = 0; f < n * k; f++) {
        int p = cnt[idx[f]]++;
        perm[p] = f;
        if (pos) pos[f] = p;
    }
    free(cnt);
    return na;
}

/* ----------------------------------------------------------------- layer */

static int check_layer(const orc_layer *L, int n, char *err) {
    int H = L->hidden, E = L->n_experts, k = L->top_k, I = L->moe_inter, g = L->group_size;
    if (n < 0 || H <= 0 || E <= 0 || k <= 0 || k > E || I <= 0 || g <= 0 || g % 8 ||
        H % g || I % g || H % 8) {
        if (err) snprintf(err, 512, "bad layer shape H=%d E=%d k=%d I=%d g=%d n=%d", H, E, k, I, g, n);
        return -1;
    }
    return 0;
}

static void load_x(const void *x, int x_is_bf16, size_t count, float *dst) {
    if (x_is_bf16) {
        const uint16_t *xb = (const uint16_t *)x;
        for (size_t i = 0; i < count; i++) dst[i] = orc_bf16_to_f32(xb[i]);
    } else {
        memcpy(dst, x, count * sizeof(float));
    }
}

int orc_route(const orc_layer *L, const void *x, int x_is_bf16, int n, float *logits_out,
              float *gate_logit_out, int *idx_out, float *w_out, float *shared_gate_out,
              float *xn_out, int n_threads, char *err) {
    if (check_layer(L, n, err)) return -1;
    int H = L->hidden, E = L->n_experts, k = L->top_k;
#ifdef _OPENMP
    if (n_threads > 0) omp_set_num_threads(n_threads);
#else
    (void)n_threads;
#endif
    float *xn = (float *)malloc((size_t)n * H * sizeof(float));
    float *lg = (float *)malloc((size_t)n * (E + 1) * sizeof(float));
#pragma omp parallel for schedule(static)
    for (int t = 0; t < n; t++) {
        float *xr = xn + (size_t)t * H;
        load_x(x_is_bf16 ? (const void *)((const uint16_t *)x + (size_t)t * H)
                         : (const void *)((const float *)x + (size_t)t * H),
               x_is_bf16, (size_t)H, xr);
        if (L->norm_w) orc_rmsnorm_r64(xr, L->norm_w, (size_t)H, L->rms_eps, xr);
    }
    /* logits: every (token, row) dot is independent; row E is the shared gate */
#pragma omp parallel for schedule(static)
    for (long long q = 0; q < (long long)n * (E + 1); q++) {
        const int t = (int)(q / (E + 1)), e = (int)(q % (E + 1));
        const float *xr = xn + (size_t)t * H;
        float v = orc_dot_r64_bf16w(xr, e < E ? L->router_w + (size_t)e * H : L->sh_gate_w, H);
        if (e < E && L->router_bias) v = v + L->router_bias[e];
        lg[q] = v;
    }
#pragma omp parallel
    {
        int *id = (int *)malloc((size_t)k * sizeof(int));
        float *wt = (float *)malloc((size_t)k * sizeof(float));
#pragma omp for schedule(static)
        for (int t = 0; t < n; t++) {
            const float *row = lg + (size_t)t * (E + 1);
            orc_topk_canonical(row, E, k, id);
            /* model.c:1305-1318: softmax over the selected logits */
            float mx = -1e30f;
            for (int s = 0; s < k; s++)
                if (row[id[s]] > mx) mx = row[id[s]];
            float sum = 0.0f;
            for (int s = 0; s < k; s++) {
                wt[s] = expf(row[id[s]] - mx);
                sum += wt[s];
            }
            for (int s = 0; s < k; s++) wt[s] /= sum;
            if (logits_out) memcpy(logits_out + (size_t)t * E, row, (size_t)E * sizeof(float));
            if (gate_logit_out) gate_logit_out[t] = row[E];
            if (idx_out) memcpy(idx_out + (size_t)t * k, id, (size_t)k * sizeof(int));
            if (w_out) memcpy(w_out + (size_t)t * k, wt, (size_t)k * sizeof(float));
            if (shared_gate_out) shared_gate_out[t] = orc_sigmoid(row[E]);
        }
        free(id);
        free(wt);
    }
    if (xn_out) memcpy(xn_out, xn, (size_t)n * H * sizeof(float));
    free(xn);
    free(lg);
    return 0;
}

/* routed expert row dot, faithful mode: dequantise the row to fp32 with
 * fma(q,s,b) (model.c:603-662 + kernel.c:157-172) and take the fp32 dot
 * product (gemm_fp32, kernel.c:181-186) as one fma chain over k */
static float faithful_row_dot(const float *a, const uint32_t *q, const uint16_t *s,
                              const uint16_t *b, int K, int gs) {
    float acc = 0.0f;
    for (int c = 0; c < K; c++) {
        int g = c / gs;
        float code = (float)((q[c / 8] >> (4 * (c % 8))) & 0xFu);
        float w = fmaf(code, orc_bf16_to_f32(s[g]), orc_bf16_to_f32(b[g]));
        acc = fmaf(a[c], w, acc);
    }
    return acc;
}

static float q4_row_dot_bf16sb(const float *a, const float *xsum, const uint32_t *q,
                               const uint16_t *s, const uint16_t *b, int K, int gs) {
    float sf[1024], bf[1024];
    int groups = K / gs;
    float *sp = sf, *bp = bf;
    if (groups > 1024) {
        sp = (float *)malloc((size_t)groups * sizeof(float));
        bp = (float *)malloc((size_t)groups * sizeof(float));
    }
    for (int g = 0; g < groups; g++) {
        sp[g] = orc_bf16_to_f32(s[g]);
        bp[g] = orc_bf16_to_f32(b[g]);
    }
    float r = q4_row_dot(a, xsum, q, sp, bp, K, gs);
    if (sp != sf) {
        free(sp);
        free(bp);
    }
    return r;
}

/* The expert weights of one (token, expert) pair: routed expert e, or the
 * shared expert when e < 0. */
typedef struct {
    const uint32_t *gq, *uq, *dq;
    const uint16_t *gs, *gb, *us, *ub, *ds, *db;
} expert_ptrs;

static expert_ptrs expert_of(const orc_layer *L, int e) {
    expert_ptrs p;
    const int H = L->hidden, I = L->moe_inter, gs = L->group_size;
    if (e < 0) {
        p.gq = L->sh_gate_q; p.gs = L->sh_gate_s; p.gb = L->sh_gate_b;
        p.uq = L->sh_up_q; p.us = L->sh_up_s; p.ub = L->sh_up_b;
        p.dq = L->sh_down_q; p.ds = L->sh_down_s; p.db = L->sh_down_b;
        return p;
    }
    const size_t eq = (size_t)I * (H / 8), es = (size_t)I * (H / gs);
    const size_t dqs = (size_t)H * (I / 8), dss = (size_t)H * (I / gs);
    p.gq = L->gate_q + e * eq; p.gs = L->gate_s + e * es; p.gb = L->gate_b + e * es;
    p.uq = L->up_q + e * eq; p.us = L->up_s + e * es; p.ub = L->up_b + e * es;
    p.dq = L->down_q + e * dqs; p.ds = L->down_s + e * dss; p.db = L->down_b + e * dss;
    return p;
}

int orc_moe_forward(const orc_layer *L, const void *x, int n, float *out, const orc_opts *opt,
                    const int *token_sel, int n_sel, float *logits_out, float *gate_logit_out,
                    int *idx_out, float *w_out, float *shared_gate_out, float *xn_out, char *err) {
    if (check_layer(L, n, err)) return -1;
    orc_opts o = {0, 0, ORC_ROUTED_FAITHFUL, 0};
    if (opt) o = *opt;
    int H = L->hidden, E = L->n_experts, k = L->top_k, I = L->moe_inter, gs = L->group_size;
    if (n == 0) return 0;
    float *xn = (float *)malloc((size_t)n * H * sizeof(float));
    float *logits = (float *)malloc((size_t)n * E * sizeof(float));
    float *gl = (float *)malloc((size_t)n * sizeof(float));
    int *idx = (int *)malloc((size_t)n * k * sizeof(int));
    float *wts = (float *)malloc((size_t)n * k * sizeof(float));
    float *sg = (float *)malloc((size_t)n * sizeof(float));
    if (orc_route(L, x, o.x_is_bf16, n, logits, gl, idx, wts, sg, xn, o.n_threads, err)) return -1;
    if (logits_out) memcpy(logits_out, logits, (size_t)n * E * sizeof(float));
    if (gate_logit_out) memcpy(gate_logit_out, gl, (size_t)n * sizeof(float));
    if (idx_out) memcpy(idx_out, idx, (size_t)n * k * sizeof(int));
    if (w_out) memcpy(w_out, wts, (size_t)n * k * sizeof(float));
    if (shared_gate_out) memcpy(shared_gate_out, sg, (size_t)n * sizeof(float));
    if (xn_out) memcpy(xn_out, xn, (size_t)n * H * sizeof(float));

    if (out) {
        /* One (token, expert) "pair" per routed slot plus one for the shared
         * expert.  Pairs of output row j are ordered by ascending expert id
         * (the dispatch order, departure 3) with the shared expert last, which
         * is the combine order of model.c:1376-1403. */
        const int nout = token_sel ? n_sel : n;
        const int faithful = o.routed_mode == ORC_ROUTED_FAITHFUL;
        const int per = k + 1;
        const size_t npairs = (size_t)nout * per;
        const int G = H / gs, GI = I / gs;
        int *pe = (int *)malloc(npairs * sizeof(int));
        int *pt = (int *)malloc(npairs * sizeof(int));
        float *pw = (float *)malloc(npairs * sizeof(float));
        float *xs_h = (float *)malloc((size_t)nout * G * sizeof(float));
        float *xs_i = (float *)malloc(npairs * GI * sizeof(float));
        float *hb = (float *)malloc(npairs * I * sizeof(float));
        float *yb = (float *)malloc(npairs * H * sizeof(float));
        for (int j = 0; j < nout; j++) {
            const int t = token_sel ? token_sel[j] : j;
            int *ord = pe + (size_t)j * per; /* slots sorted by expert id */
            for (int s = 0; s < k; s++) ord[s] = s;
            for (int a2 = 1; a2 < k; a2++)
                for (int b2 = a2; b2 > 0 && idx[(size_t)t * k + ord[b2 - 1]] > idx[(size_t)t * k + ord[b2]]; b2--) {
                    int tmp = ord[b2];
                    ord[b2] = ord[b2 - 1];
                    ord[b2 - 1] = tmp;
                }
            for (int a2 = 0; a2 < k; a2++) {
                const int s = ord[a2];
                pw[(size_t)j * per + a2] = wts[(size_t)t * k + s];
                ord[a2] = idx[(size_t)t * k + s];
            }
            pe[(size_t)j * per + k] = -1;
            pw[(size_t)j * per + k] = sg[t];
            for (int a2 = 0; a2 < per; a2++) pt[(size_t)j * per + a2] = j;
            group_sums(xn + (size_t)t * H, H, gs, xs_h + (size_t)j * G);
        }
#ifdef _OPENMP
        if (o.n_threads > 0) omp_set_num_threads(o.n_threads);
#endif
        /* gate/up + SwiGLU: every (pair, row) independent.  Routed experts
         * follow model.c:1368-1375 (faithful: fp32-dequantised weights) or
         * gemm_q4 (q4 mode); the shared expert always uses gemm_q4
         * (linear_forward, model.c:193-202, 1388-1395). */
#pragma omp parallel for schedule(static)
        for (long long q = 0; q < (long long)(npairs * I); q++) {
            const size_t pr = (size_t)(q / I);
            const int r = (int)(q % I);
            const int e = pe[pr];
            const int t = token_sel ? token_sel[pt[pr]] : pt[pr];
            const float *xr = xn + (size_t)t * H;
            const float *xs = xs_h + (size_t)pt[pr] * G;
            const expert_ptrs P = expert_of(L, e);
            const size_t wq = (size_t)r * (H / 8), ws = (size_t)r * G;
            float g, u;
            if (faithful && e >= 0) {
                g = faithful_row_dot(xr, P.gq + wq, P.gs + ws, P.gb + ws, H, gs);
                u = faithful_row_dot(xr, P.uq + wq, P.us + ws, P.ub + ws, H, gs);
            } else {
                g = q4_row_dot_bf16sb(xr, xs, P.gq + wq, P.gs + ws, P.gb + ws, H, gs);
                u = q4_row_dot_bf16sb(xr, xs, P.uq + wq, P.us + ws, P.ub + ws, H, gs);
            }
            hb[pr * I + r] = orc_silu(g) * u; /* kernel_silu then kernel_mul */
        }
#pragma omp parallel for schedule(static)
        for (long long pr = 0; pr < (long long)npairs; pr++) group_sums(hb + pr * I, I, gs, xs_i + pr * GI);
#pragma omp parallel for schedule(static)
        for (long long q = 0; q < (long long)(npairs * H); q++) {
            const size_t pr = (size_t)(q / H);
            const int c = (int)(q % H);
            const int e = pe[pr];
            const expert_ptrs P = expert_of(L, e);
            const size_t wq = (size_t)c * (I / 8), ws = (size_t)c * GI;
            if (faithful && e >= 0)
                yb[pr * H + c] = faithful_row_dot(hb + pr * I, P.dq + wq, P.ds + ws, P.db + ws, I, gs);
            else
                yb[pr * H + c] = q4_row_dot_bf16sb(hb + pr * I, xs_i + pr * GI, P.dq + wq, P.ds + ws,
                                                   P.db + ws, I, gs);
        }
        /* combine: out = 0; out = fma(w, y, out) per pair in order (the
         * reference's out += w*r under Apple clang's contraction) */
#pragma omp parallel for schedule(static)
        for (int j = 0; j < nout; j++) {
            float *orow = out + (size_t)j * H;
            for (int c = 0; c < H; c++) orow[c] = 0.0f;
            for (int a2 = 0; a2 < per; a2++) {
                const size_t pr = (size_t)j * per + a2;
                const float wt = pw[pr];
                for (int c = 0; c < H; c++) orow[c] = fmaf(wt, yb[pr * H + c], orow[c]);
            }
            if (o.residual) { /* the un-normalised input row plus the layer output */
                const int t = token_sel ? token_sel[j] : j;
                if (o.x_is_bf16) {
                    const uint16_t *xb = (const uint16_t *)x + (size_t)t * H;
                    for (int c = 0; c < H; c++) orow[c] = orc_bf16_to_f32(xb[c]) + orow[c];
                } else {
                    const float *xf = (const float *)x + (size_t)t * H;
                    for (int c = 0; c < H; c++) orow[c] = xf[c] + orow[c];
                }
            }
        }
        free(pe);
        free(pt);
        free(pw);
        free(xs_h);
        free(xs_i);
        free(hb);
        free(yb);
    }
    free(xn);
    free(logits);
    free(gl);
    free(idx);
    free(wts);
    free(sg);
    return 0;
}

/* ------------------------------------------------------------ generators */

/* splitmix64 output function (Steele, Lea, Flood 2014; constants as
 * published by Vigna) */
uint64_t orc_mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

#define GOLDEN64 0x9E3779B97F4A7C15ull

uint64_t orc_tensor_key(uint64_t seed, uint32_t layer, uint32_t tag) {
    return orc_mix64(orc_mix64(seed + GOLDEN64) ^ (((uint64_t)layer << 32) | (uint64_t)tag));
}

/* element i of a stream: splitmix64 in counter mode */
static inline uint64_t stream_u64(uint64_t key, uint64_t i) { return orc_mix64(key + (i + 1) * GOLDEN64); }

/* Box-Muller in double from draws 2i and 2i+1; cosine branch only */
static inline double stream_normal(uint64_t key, uint64_t i) {
    uint64_t r1 = stream_u64(key, 2 * i), r2 = stream_u64(key, 2 * i + 1);
    double u1 = (double)((r1 >> 11) + 1) * 0x1.0p-53; /* (0,1] */
    double u2 = (double)(r2 >> 11) * 0x1.0p-53;       /* [0,1) */
    return sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
}

void orc_gen_normal_f32(float *out, size_t count, uint64_t key, uint64_t start, float stddev) {
#pragma omp parallel for schedule(static) if (count > 65536)
    for (size_t i = 0; i < count; i++) out[i] = (float)(stream_normal(key, start + i) * (double)stddev);
}

void orc_gen_normal_bf16(uint16_t *out, size_t count, uint64_t key, uint64_t start, float stddev) {
#pragma omp parallel for schedule(static) if (count > 65536)
    for (size_t i = 0; i < count; i++)
        out[i] = orc_f32_to_bf16((float)(stream_normal(key, start + i) * (double)stddev));
}

/* eight uniform 4-bit codes per word: the high half of the stream value */
void orc_gen_codes(uint32_t *out, size_t count, uint64_t key, uint64_t start) {
#pragma omp parallel for schedule(static) if (count > 65536)
    for (size_t i = 0; i < count; i++) out[i] = (uint32_t)(stream_u64(key, start + i) >> 32);
}

void orc_zipf_bias(float *bias, int E, double s, double scale, uint64_t seed) {
    int *perm = (int *)malloc((size_t)E * sizeof(int));
    for (int i = 0; i < E; i++) perm[i] = i;
    uint64_t key = orc_mix64(seed ^ 0x5A17F00Dull);
    for (int i = E - 1; i > 0; i--) {
        int j = (int)(stream_u64(key, (uint64_t)i) % (uint64_t)(i + 1));
        int t = perm[i];
        perm[i] = perm[j];
        perm[j] = t;
    }
    double z = 0.0;
    for (int r = 1; r <= E; r++) z += pow((double)r, -s);
    for (int e = 0; e < E; e++) {
        double p = pow((double)(perm[e] + 1), -s) / z;
        bias[e] = (float)(scale * log(p));
    }
    free(perm);
}

/* ------------------------------------------------------------ timing */

static double now_s(void) { /* util.h:73-77 */
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + (double)ts.tv_nsec * 1e-9;
}

static int cmp_dbl(const void *a, const void *b) {
    double x = *(const double *)a, y = *(const double *)b;
    return (x > y) - (x < y);
}

double orc_time_forward(const orc_layer *L, const void *x, int n, float *out, const orc_opts *opt,
                        int warmup, int iters) {
    char err[512];
    for (int i = 0; i < warmup; i++) orc_moe_forward(L, x, n, out, opt, NULL, 0, 0, 0, 0, 0, 0, 0, err);
    if (iters < 1) iters = 1;
    double *t = (double *)malloc((size_t)iters * sizeof(double));
    for (int i = 0; i < iters; i++) {
        double t0 = now_s();
        orc_moe_forward(L, x, n, out, opt, NULL, 0, 0, 0, 0, 0, 0, 0, err);
        t[i] = now_s() - t0;
    }
    qsort(t, (size_t)iters, sizeof(double), cmp_dbl);
    double med = t[iters / 2];
    free(t);
    return med;
}

/* ------------------------------------------------ warm fp32 experts (mode i) */

struct orc_warm {
    int E, H, I;
    int *slot;    /* [E]: index into w, or -1 */
    float *w;     /* [count][gate I*H | up I*H | down H*I] */
    size_t count;
};

orc_warm *orc_warm_create(const orc_layer *L, const int *experts, int count, int n_threads) {
    const int E = L->n_experts, H = L->hidden, I = L->moe_inter, gs = L->group_size;
    orc_warm *w = (orc_warm *)calloc(1, sizeof(orc_warm));
    if (!w) return NULL;
    w->E = E;
    w->H = H;
    w->I = I;
    w->slot = (int *)malloc((size_t)E * sizeof(int));
    int *list = (int *)malloc((size_t)(count > 0 ? count : 1) * sizeof(int));
    if (!w->slot || !list) {
        free(list);
        orc_warm_destroy(w);
        return NULL;
    }
    for (int e = 0; e < E; e++) w->slot[e] = -1;
    size_t m = 0;
    for (int i = 0; i < count; i++) {
        const int e = experts[i];
        if (e < 0 || e >= E || w->slot[e] >= 0) continue;
        w->slot[e] = (int)m;
        list[m++] = e;
    }
    const size_t per = (size_t)3 * I * H;
    w->w = (float *)malloc((m ? m : 1) * per * sizeof(float));
    if (!w->w) {
        free(list);
        orc_warm_destroy(w);
        return NULL;
    }
    w->count = m;
#ifdef _OPENMP
    if (n_threads > 0) omp_set_num_threads(n_threads);
#else
    (void)n_threads;
#endif
#pragma omp parallel for schedule(dynamic, 1)
    for (long long q = 0; q < (long long)(m * 3); q++) {
        const int e = list[q / 3], part = (int)(q % 3);
        const expert_ptrs P = expert_of(L, e);
        float *dst = w->w + (size_t)(q / 3) * per + (size_t)part * I * H;
        if (part == 0) orc_dequant_q4(P.gq, P.gs, P.gb, (size_t)I, (size_t)H, (size_t)gs, dst);
        else if (part == 1) orc_dequant_q4(P.uq, P.us, P.ub, (size_t)I, (size_t)H, (size_t)gs, dst);
        else orc_dequant_q4(P.dq, P.ds, P.db, (size_t)H, (size_t)I, (size_t)gs, dst);
    }
    free(list);
    return w;
}

void orc_warm_destroy(orc_warm *w) {
    if (!w) return;
    free(w->slot);
    free(w->w);
    free(w);
}

size_t orc_warm_bytes(const orc_warm *w) { return w ? w->count * (size_t)3 * w->I * w->H * sizeof(float) : 0; }

/* fp32 dot with 16 independent partial sums (vectorisable), tail in order */
static float dot16(const float *a, const float *b, int K) {
    float acc[16];
    for (int j = 0; j < 16; j++) acc[j] = 0.0f;
    int c = 0;
    for (; c + 16 <= K; c += 16)
        for (int j = 0; j < 16; j++) acc[j] = fmaf(a[c + j], b[c + j], acc[j]);
    for (int j = 8; j > 0; j >>= 1)
        for (int i = 0; i < j; i++) acc[i] = acc[i] + acc[i + j];
    float r = acc[0];
    for (; c < K; c++) r = fmaf(a[c], b[c], r);
    return r;
}

int orc_moe_forward_warm(const orc_layer *L, const orc_warm *W, const void *x, int n, float *out,
                         const orc_opts *opt, char *err) {
    if (check_layer(L, n, err)) return -1;
    if (!W || W->E != L->n_experts || W->H != L->hidden || W->I != L->moe_inter) {
        if (err) snprintf(err, 512, "warm expert set does not match the layer");
        return -1;
    }
    if (L->top_k > 64) {
        if (err) snprintf(err, 512, "top_k %d > 64", L->top_k);
        return -1;
    }
    orc_opts o = {0, 0, ORC_ROUTED_FAITHFUL, 0};
    if (opt) o = *opt;
    const int H = L->hidden, E = L->n_experts, k = L->top_k, I = L->moe_inter, gs = L->group_size;
    const int G = H / gs, GI = I / gs;
    if (n == 0) return 0;
    const size_t nk = (size_t)n * k, rows = nk + (size_t)n, per = (size_t)3 * I * H;
    float *xn = (float *)malloc((size_t)n * H * sizeof(float));
    int *idx = (int *)malloc(nk * sizeof(int));
    float *wts = (float *)malloc(nk * sizeof(float));
    float *sg = (float *)malloc((size_t)n * sizeof(float));
    int *offsets = (int *)malloc(((size_t)E + 1) * sizeof(int));
    int *perm = (int *)malloc(nk * sizeof(int));
    int *pos = (int *)malloc(nk * sizeof(int));
    int *active = (int *)malloc((size_t)E * sizeof(int));
    float *h = (float *)malloc(rows * I * sizeof(float));
    float *y = (float *)malloc(rows * H * sizeof(float));
    float *xs_h = (float *)malloc((size_t)n * G * sizeof(float));
    float *xs_i = (float *)malloc((size_t)n * GI * sizeof(float));
    int rc = -1;
    if (orc_route(L, x, o.x_is_bf16, n, NULL, NULL, idx, wts, sg, xn, o.n_threads, err)) goto done;
    const int na = orc_dispatch(idx, n, k, E, offsets, perm, pos, active);
    for (int a = 0; a < na; a++)
        if (W->slot[active[a]] < 0) {
            if (err) snprintf(err, 512, "expert %d is not in the warm set", active[a]);
            goto done;
        }
#ifdef _OPENMP
    if (o.n_threads > 0) omp_set_num_threads(o.n_threads);
#endif
    /* routed gate/up: one task per (active expert, row); the row's weights
     * stay in cache across the expert's tokens */
#pragma omp parallel for schedule(dynamic, 8)
    for (long long q = 0; q < (long long)na * I; q++) {
        const int e = active[q / I], r = (int)(q % I);
        const float *we = W->w + (size_t)W->slot[e] * per;
        const float *wg = we + (size_t)r * H, *wu = we + (size_t)I * H + (size_t)r * H;
        for (int p = offsets[e]; p < offsets[e + 1]; p++) {
            const float *xr = xn + (size_t)(perm[p] / k) * H;
            const float g = dot16(xr, wg, H), u = dot16(xr, wu, H);
            h[(size_t)p * I + r] = orc_silu(g) * u;
        }
    }
    /* shared expert gate/up: gemm_q4 */
    for (int t = 0; t < n; t++) group_sums(xn + (size_t)t * H, H, gs, xs_h + (size_t)t * G);
    {
        const expert_ptrs P = expert_of(L, -1);
#pragma omp parallel for schedule(static)
        for (long long q = 0; q < (long long)n * I; q++) {
            const int t = (int)(q / I), r = (int)(q % I);
            const float *xr = xn + (size_t)t * H;
            const size_t wq = (size_t)r * (H / 8), ws = (size_t)r * G;
            const float g = q4_row_dot_bf16sb(xr, xs_h + (size_t)t * G, P.gq + wq, P.gs + ws, P.gb + ws, H, gs);
            const float u = q4_row_dot_bf16sb(xr, xs_h + (size_t)t * G, P.uq + wq, P.us + ws, P.ub + ws, H, gs);
            h[(nk + (size_t)t) * I + r] = orc_silu(g) * u;
        }
    }
    /* routed down: one task per (active expert, output column) */
#pragma omp parallel for schedule(dynamic, 32)
    for (long long q = 0; q < (long long)na * H; q++) {
        const int e = active[q / H], c = (int)(q % H);
        const float *wd = W->w + (size_t)W->slot[e] * per + (size_t)2 * I * H + (size_t)c * I;
        for (int p = offsets[e]; p < offsets[e + 1]; p++) y[(size_t)p * H + c] = dot16(h + (size_t)p * I, wd, I);
    }
    for (int t = 0; t < n; t++) group_sums(h + (nk + (size_t)t) * I, I, gs, xs_i + (size_t)t * GI);
    {
        const expert_ptrs P = expert_of(L, -1);
#pragma omp parallel for schedule(static)
        for (long long q = 0; q < (long long)n * H; q++) {
            const int t = (int)(q / H), c = (int)(q % H);
            const size_t wq = (size_t)c * (I / 8), ws = (size_t)c * GI;
            y[(nk + (size_t)t) * H + c] = q4_row_dot_bf16sb(h + (nk + (size_t)t) * I, xs_i + (size_t)t * GI,
                                                           P.dq + wq, P.ds + ws, P.db + ws, I, gs);
        }
    }
    /* combine in ascending expert order, then the shared expert */
#pragma omp parallel for schedule(static)
    for (int t = 0; t < n; t++) {
        int ps[64], m = 0;
        for (int s2 = 0; s2 < k; s2++) ps[m++] = pos[(size_t)t * k + s2];
        for (int a2 = 1; a2 < m; a2++)
            for (int b2 = a2; b2 > 0 && ps[b2 - 1] > ps[b2]; b2--) {
                const int tmp = ps[b2];
                ps[b2] = ps[b2 - 1];
                ps[b2 - 1] = tmp;
            }
        float *orow = out + (size_t)t * H;
        for (int c = 0; c < H; c++) orow[c] = 0.0f;
        for (int a2 = 0; a2 < m; a2++) {
            const int p = ps[a2];
            const float wt = wts[perm[p]];
            for (int c = 0; c < H; c++) orow[c] = fmaf(wt, y[(size_t)p * H + c], orow[c]);
        }
        for (int c = 0; c < H; c++) orow[c] = fmaf(sg[t], y[(nk + (size_t)t) * H + c], orow[c]);
        if (o.residual) {
            if (o.x_is_bf16) {
                const uint16_t *xb = (const uint16_t *)x + (size_t)t * H;
                for (int c = 0; c < H; c++) orow[c] = orc_bf16_to_f32(xb[c]) + orow[c];
            } else {
                const float *xf = (const float *)x + (size_t)t * H;
                for (int c = 0; c < H; c++) orow[c] = xf[c] + orow[c];
            }
        }
    }
    rc = 0;
done:
    free(xn);
    free(idx);
    free(wts);
    free(sg);
    free(offsets);
    free(perm);
    free(pos);
    free(active);
    free(h);
    free(y);
    free(xs_h);
    free(xs_i);
    return rc;
}

double orc_time_forward_warm(const orc_layer *L, const orc_warm *W, const void *x, int n,
                             float *out, const orc_opts *opt, int warmup, int iters) {
    char err[512];
    for (int i = 0; i < warmup; i++)
        if (orc_moe_forward_warm(L, W, x, n, out, opt, err)) return -1.0;
    if (iters < 1) iters = 1;
    double *t = (double *)malloc((size_t)iters * sizeof(double));
    for (int i = 0; i < iters; i++) {
        double t0 = now_s();
        if (orc_moe_forward_warm(L, W, x, n, out, opt, err)) {
            free(t);
            return -1.0;
        }
        t[i] = now_s() - t0;
    }
    qsort(t, (size_t)iters, sizeof(double), cmp_dbl);
    double med = t[iters / 2];
    free(t);
    return med;
}
