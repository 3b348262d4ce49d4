/*
 * hyper.hip -- the MLP hyper connection around the MoE layer: the producer
 * of the layer's input, gated_residual (reference C port model.c:728-796;
 * MLX module src/colibri_runtime/model.py:463-481), for a hyper state of
 * hc copies of the hidden vector:
 *     normed = grouped RMSNorm of each copy (eps 1e-6) * hc_norm
 *     w      = silu(input_mix_weight_down(normed) / hc)          [n, R]
 *     gate   = sigmoid(input_mix_weight_up(w))                    [n, hc*d]
 *     mixed  = mean over the copies of gate * normed              [n, d]
 *     inject = 2 * sigmoid(block_inject_weight(normed) / hc)      [n, hc]
 * in two launches:
 *   k_hc_down         the copy norms, normed, the q4 GEMV normed -> w with
 *                     silu(./hc) and the hc inject dots (bf16 weights), each
 *                     wave on one copy so the norms need no second pass;
 *   k_hc_upmix        q4 GEMV w -> gates, with the mean over the
 *                     copies in its epilogue: a workgroup holds the rows
 *                     h*d + i of every copy h for its block of columns i,
 *                     so the [n, hc*d] gates never reach memory.
 * The consumer, hyper += inject (x) out (model.c:1724-1731), is the epilogue
 * of the layer's combine kernels (combine.hip, ffn_gemv.hip).
 *
 * Both linear layers are MLX affine q4 (linear_forward -> gemm_q4,
 * model.c:193-201), dequantised in registers with the per-group identity
 * of gemm_q4 (gemv_parts.h).
 */
#include "qk_device.h"
#include "gemv_parts.h"

#define HC_MAX 8

/* --------------------------------------------- norm + down + inject */

struct HcDownArgs {
    const float *hyper;        /* [n, hc*d] */
    const float *norm_w;       /* [hc*d] hc_norm */
    const uint32_t *q;         /* input_mix_weight_down [R, hc*d/8] */
    const uint16_t *s, *b;     /* [R, hc*d/64] */
    const uint16_t *inject_w;  /* block_inject_weight [hc, hc*d] bf16 */
    float *normed;             /* [n, hc*d], written by the first row block */
    float *w;                  /* [n, R]: silu(down(normed) / hc) */
    float *inject;             /* [n, hc] */
    int hc, d, R, n, tb;
    float eps;
};

#define HD_RW 2 /* down-matrix rows per workgroup */

/* one task of k_hc_down: INJ = one row of the inject matrix, else HD_RW
 * rows of the down matrix */
template <int P, bool INJ>
__device__ __forceinline__ void hc_down_body(const HcDownArgs &a, int tblk, int rb, int nrb) {
    constexpr int RW = INJ ? 1 : HD_RW; /* rows of this task */
    __shared__ float s_part[2][HC_MAX][HD_RW];
    const int lane = threadIdx.x & 63, h = threadIdx.x >> 6;
    const int D = a.hc * a.d, CPC = a.d >> 5, G = D >> 6;
    const size_t wrow = (size_t)D >> 3;
    const int r0 = INJ ? rb - nrb : rb * HD_RW;
    const int nrows = INJ ? a.hc : a.R;
    const int t0 = tblk * a.tb, m = min(a.tb, a.n - t0);
    if (m <= 0) return;
    const float inv_hc = 1.0f / (float)a.hc;

    /* this lane's chunks: copy-local chunk ps*64 + lane, global chunk gc[ps] */
    int gc[P];
    bool cok[P];
#pragma unroll
    for (int ps = 0; ps < P; ps++) {
        const int cc = ps * 64 + lane;
        cok[ps] = cc < CPC;
        gc[ps] = h * CPC + (cok[ps] ? cc : 0);
    }
    /* weights: q4 rows (codes, scale, bias) or one bf16 row (32 weights a chunk) */
    uint4 wq[RW][P];
    float ws[RW][P], wb[RW][P];
    uint4 wi[P][4];
    if (INJ) {
#pragma unroll
        for (int ps = 0; ps < P; ps++) {
            const uint4 *src = (const uint4 *)(a.inject_w + (size_t)r0 * D) + 4 * gc[ps];
#pragma unroll
            for (int v = 0; v < 4; v++) wi[ps][v] = cok[ps] ? qk_ld(src + v) : make_uint4(0u, 0u, 0u, 0u);
        }
    } else {
#pragma unroll
        for (int it = 0; it < RW; it++) {
            const int r = min(r0 + it, nrows - 1);
#pragma unroll
            for (int ps = 0; ps < P; ps++) {
                const bool ok = cok[ps] && r0 + it < nrows;
                wq[it][ps] = ok ? qk_ld((const uint4 *)(a.q + (size_t)r * wrow) + gc[ps])
                                : make_uint4(0u, 0u, 0u, 0u);
                ws[it][ps] = ok ? qk_bf16(qk_ld(a.s + (size_t)r * G + (gc[ps] >> 1))) : 0.0f;
                wb[it][ps] = ok ? qk_bf16(qk_ld(a.b + (size_t)r * G + (gc[ps] >> 1))) : 0.0f;
            }
        }
    }
    float4 wn[P][8];
#pragma unroll
    for (int ps = 0; ps < P; ps++)
#pragma unroll
        for (int v = 0; v < 8; v++)
            wn[ps][v] = qk_ld((const float4 *)(a.norm_w + (size_t)gc[ps] * 32) + v);
    const bool store_normed = !INJ && rb == 0;

    float4 xr[P][8];
    auto load_x = [&](int t) {
#pragma unroll
        for (int ps = 0; ps < P; ps++)
#pragma unroll
            for (int v = 0; v < 8; v++)
                xr[ps][v] = qk_ld((const float4 *)(a.hyper + (size_t)t * D + (size_t)gc[ps] * 32) + v);
    };
    load_x(t0);
    for (int j = 0; j < m; j++) {
        const int t = t0 + j;
        float xv[P][32];
        float ss = 0.0f;
#pragma unroll
        for (int ps = 0; ps < P; ps++)
#pragma unroll
            for (int v = 0; v < 8; v++) {
                const float4 f = xr[ps][v];
                xv[ps][4 * v] = cok[ps] ? f.x : 0.0f;
                xv[ps][4 * v + 1] = cok[ps] ? f.y : 0.0f;
                xv[ps][4 * v + 2] = cok[ps] ? f.z : 0.0f;
                xv[ps][4 * v + 3] = cok[ps] ? f.w : 0.0f;
            }
        if (j + 1 < m) load_x(t + 1);
#pragma unroll
        for (int ps = 0; ps < P; ps++)
#pragma unroll
            for (int i = 0; i < 32; i++) ss = fmaf(xv[ps][i], xv[ps][i], ss);
        ss = qk_group_sum<64>(ss);
        const float r = 1.0f / sqrtf(ss / (float)a.d + a.eps);
        XPairs<64, P, false> xp;
#pragma unroll
        for (int ps = 0; ps < P; ps++) {
            xp.xs[ps] = 0.0f;
#pragma unroll
            for (int v = 0; v < 8; v++) {
                const float4 wv = wn[ps][v];
                xv[ps][4 * v] = xv[ps][4 * v] * r * wv.x;
                xv[ps][4 * v + 1] = xv[ps][4 * v + 1] * r * wv.y;
                xv[ps][4 * v + 2] = xv[ps][4 * v + 2] * r * wv.z;
                xv[ps][4 * v + 3] = xv[ps][4 * v + 3] * r * wv.w;
            }
            if (store_normed && cok[ps]) {
                float4 *dst = (float4 *)(a.normed + (size_t)t * D + (size_t)gc[ps] * 32);
#pragma unroll
                for (int v = 0; v < 8; v++)
                    qk_st(dst + v, make_float4(xv[ps][4 * v], xv[ps][4 * v + 1], xv[ps][4 * v + 2],
                                               xv[ps][4 * v + 3]));
            }
#pragma unroll
            for (int w = 0; w < 4; w++)
                qk_f32x8_to_pairs(&xv[ps][8 * w], &xp.hi[ps][4 * w], &xp.lo[ps][4 * w], xp.xs[ps]);
        }
#pragma unroll
        for (int it = 0; it < RW; it++) {
            float part;
            if (INJ) {
                part = 0.0f;
#pragma unroll
                for (int ps = 0; ps < P; ps++)
#pragma unroll
                    for (int v = 0; v < 4; v++) {
                        uint32_t pr[4];
                        qk_bf16x8_to_pairs(wi[ps][v], pr);
#pragma unroll
                        for (int i = 0; i < 4; i++) {
                            part = qk_dot2(xp.hi[ps][4 * v + i], pr[i], part);
                            part = qk_dot2(xp.lo[ps][4 * v + i], pr[i], part);
                        }
                    }
            } else {
                part = row_part<64, P, false>(wq[it], ws[it], wb[it], xp);
            }
            const float v = qk_group_sum<64>(part);
            if (lane == 0) s_part[j & 1][h][it] = v;
        }
        __syncthreads();
        if ((int)threadIdx.x < RW && r0 + (int)threadIdx.x < nrows) {
            const int it = threadIdx.x;
            float acc = 0.0f;
            for (int hh = 0; hh < a.hc; hh++) acc += s_part[j & 1][hh][it];
            if (INJ) a.inject[(size_t)t * a.hc + r0 + it] = 2.0f * qk_sigmoid(acc * inv_hc);
            else a.w[(size_t)t * a.R + r0 + it] = qk_silu(acc * inv_hc);
        }
    }
}

/*
 * Workgroup = hc waves; wave h owns copy h (columns h*d .. h*d+d) of the
 * hyper state, P chunks of 32 columns per lane, so the copy's RMSNorm is a
 * wave sum and needs no other wave: normed = (x * r) * w with
 * r = 1/sqrt(ss/d + eps) (kernel_rmsnorm_grouped, kernel.c:22-36).  A task
 * is (block of tb tokens, block of HD_RW rows of the down matrix (q4) or
 * one row of the inject matrix (bf16; no inject tasks when inject_w is
 * NULL)); per token each wave leaves its copy's partial row sums in LDS
 * (double-buffered by token parity) and the first threads add the copies
 * in order and apply the activation: silu(v / hc) for down rows
 * (kernel_scale + kernel_silu, model.c:757-758), 2 * sigmoid(v / hc) for
 * inject rows (model.c:790-792).  The two task kinds are separate bodies,
 * so neither carries the other's weight registers.
 */
template <int P>
__global__ __launch_bounds__(64 * HC_MAX) void k_hc_down(HcDownArgs a) {
    const int nrb = (a.R + HD_RW - 1) / HD_RW;
    const int nblk = nrb + (a.inject_w ? a.hc : 0);
    const int tblk = blockIdx.x / nblk, rb = blockIdx.x - tblk * nblk;
    if (rb >= nrb) hc_down_body<P, true>(a, tblk, rb, nrb);
    else hc_down_body<P, false>(a, tblk, rb, nrb);
}

/* ------------------------------------------------------- up + mean mix */

struct HcUpArgs {
    const uint32_t *q;    /* input_mix_weight_up [hc*d, R/8] */
    const uint16_t *s;    /* [hc*d, R/64] */
    const uint16_t *b;
    const float *w;       /* [n, R] silu(down / hc) */
    const float *normed;  /* [n, hc*d] */
    float *mixed;         /* [n, d] */
    int hc, d, R, n, tb;
};

#define HU_RIT 2 /* row steps per wave: 2 * 64/LPR columns per workgroup */

/*
 * Workgroup = hc waves (wave h computes rows h*d + i of the up projection)
 * over a block of CB = HU_RIT * 64/LPR columns i and a block of tb tokens.
 * Per token the gates go through LDS (double-buffered by token parity, so
 * one barrier per token), and the first CB threads form
 * mixed[t, i] = (sum over h in order of fma(gate, normed, acc)) / hc as the
 * loop of model.c:776-785 does.
 */
template <int LPR, int P>
__global__ __launch_bounds__(64 * HC_MAX) void k_hc_upmix(HcUpArgs a) {
    constexpr int RPW = 64 / LPR;
    constexpr int CB = RPW * HU_RIT;
    __shared__ float s_g[2][HC_MAX][CB];
    const int lane = threadIdx.x & 63, h = threadIdx.x >> 6;
    const int sub = lane % LPR, rsub = lane / LPR;
    const int K = a.R, CH = K >> 5, G = K >> 6;
    const size_t wrow = (size_t)K >> 3;
    const int D = a.hc * a.d;
    const int ncb = (a.d + CB - 1) / CB;
    const int tblk = blockIdx.x / ncb, cb = blockIdx.x - tblk * ncb;
    const int c0 = cb * CB, t0 = tblk * a.tb;
    const int m = min(a.tb, a.n - t0);
    if (m <= 0) return;
    uint4 wq[HU_RIT][P];
    uint16_t rs[HU_RIT][P], rbi[HU_RIT][P];
    float ws[HU_RIT][P], wb[HU_RIT][P];
    XRaw<P, false> xr;
    load_xraw<LPR, P, false>(a.w, (size_t)t0, K, sub, xr);
#pragma unroll
    for (int it = 0; it < HU_RIT; it++) {
        const int i0 = c0 + it * RPW + rsub;
        const size_t r = (size_t)h * a.d + (i0 < a.d ? i0 : 0);
#pragma unroll
        for (int ps = 0; ps < P; ps++) {
            const int cc = ps * LPR + sub;
            const int c = cc < CH ? cc : 0;
            wq[it][ps] = qk_ld((const uint4 *)(a.q + r * wrow) + c);
            rs[it][ps] = qk_ld(a.s + r * G + (c >> 1));
            rbi[it][ps] = qk_ld(a.b + r * G + (c >> 1));
        }
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int it = 0; it < HU_RIT; it++) {
        const bool iok = c0 + it * RPW + rsub < a.d;
#pragma unroll
        for (int ps = 0; ps < P; ps++) {
            const bool ok = iok && ps * LPR + sub < CH;
            ws[it][ps] = ok ? qk_bf16(rs[it][ps]) : 0.0f;
            wb[it][ps] = ok ? qk_bf16(rbi[it][ps]) : 0.0f;
            if (!ok) wq[it][ps] = make_uint4(0u, 0u, 0u, 0u);
        }
    }
    const int mix_i = c0 + (int)threadIdx.x;
    const bool mixer = (int)threadIdx.x < CB && mix_i < a.d;
    for (int j = 0; j < m; j++) {
        const int t = t0 + j;
        /* the mixer threads' normed values, loaded before the barrier */
        float nv[HC_MAX];
#pragma unroll
        for (int hh = 0; hh < HC_MAX; hh++)
            nv[hh] = (mixer && hh < a.hc) ? qk_ld(a.normed + (size_t)t * D + (size_t)hh * a.d + mix_i)
                                          : 0.0f;
        XPairs<LPR, P, false> xp;
        convert_xraw<LPR, P, false>(xr, K, sub, xp);
        if (j + 1 < m) load_xraw<LPR, P, false>(a.w, (size_t)(t + 1), K, sub, xr);
#pragma unroll
        for (int it = 0; it < HU_RIT; it++) {
            const float v = qk_group_sum<LPR>(row_part<LPR, P, false>(wq[it], ws[it], wb[it], xp));
            if (sub == 0) s_g[j & 1][h][it * RPW + rsub] = qk_sigmoid(v);
        }
        __syncthreads();
        if (mixer) {
            float acc = 0.0f;
#pragma unroll
            for (int hh = 0; hh < HC_MAX; hh++)
                if (hh < a.hc) acc = fmaf(s_g[j & 1][hh][threadIdx.x], nv[hh], acc);
            qk_st(a.mixed + (size_t)t * a.d + mix_i, acc / (float)a.hc);
        }
    }
}

/* --------------------------------------------------------- inject update */

/* grid = (n, ceil(d/1024)), 256 threads x 4 columns (model.c:1724-1731) */
__global__ __launch_bounds__(256) void k_hc_inject(const float *inject, const float *out, int hc,
                                                   int d, float *hyper) {
    const int t = blockIdx.x;
    const int c = (blockIdx.y * 256 + threadIdx.x) * 4;
    if (c >= d) return;
    const float4 o = qk_ld((const float4 *)(out + (size_t)t * d + c));
    for (int j = 0; j < hc; j++) {
        const float inj = qk_ld(inject + (size_t)t * hc + j);
        float4 *hp = (float4 *)(hyper + ((size_t)t * hc + j) * d + c);
        float4 hv = *hp;
        hv.x = fmaf(inj, o.x, hv.x);
        hv.y = fmaf(inj, o.y, hv.y);
        hv.z = fmaf(inj, o.z, hv.z);
        hv.w = fmaf(inj, o.w, hv.w);
        *hp = hv;
    }
}

/* ---------------------------------------------------------------- launch */

static int hc_pick_lpr(int K) {
    const int ch = K / 32;
    int l = 2;
    while (l < ch && l < 64) l <<= 1;
    return l;
}

/* tokens per task: enough tasks to fill the chip about four times over */
static int hc_tokens_per_task(int n, int blocks) {
    const long long want = 1024;
    long long tb = ((long long)n * blocks + want - 1) / want;
    if (tb < 1) tb = 1;
    return (int)(tb < n ? tb : n);
}

extern "C" int qk_hc_shape_ok(int hc, int d, int R) {
    /* k_hc_down: one wave per copy, one 32-column chunk per lane (d <= 2048);
     * k_hc_upmix: one chunk of the low-rank vector per lane (R <= 2048) */
    return hc >= 1 && hc <= HC_MAX && d > 0 && d % 64 == 0 && d <= 2048 && R >= 64 &&
           R % 64 == 0 && R <= 2048;
}

extern "C" int qk_launch_hc_down(const float *hyper, const float *norm_w, const uint32_t *q,
                                 const uint16_t *s, const uint16_t *b, const uint16_t *inject_w,
                                 int hc, int d, int R, int n, float eps, float *normed, float *w,
                                 float *inject, void *stream) {
    if (n <= 0) return 0;
    if (!qk_hc_shape_ok(hc, d, R)) return (int)hipErrorInvalidValue;
    if (inject_w && !inject) return (int)hipErrorInvalidValue;
    /* no inject matrix (the final mixer): the down row blocks alone */
    const int nblk = (R + HD_RW - 1) / HD_RW + (inject_w ? hc : 0);
    const int tb = hc_tokens_per_task(n, nblk);
    HcDownArgs a{hyper, norm_w, q, s, b, inject_w, normed, w, inject, hc, d, R, n, tb, eps};
    const dim3 grid((unsigned)(((n + tb - 1) / tb) * nblk)), blk(64 * hc);
    hipStream_t st = (hipStream_t)stream;
    hipLaunchKernelGGL(k_hc_down<1>, grid, blk, 0, st, a);
    return QK_CHECK_LAUNCH();
}

extern "C" int qk_launch_hc_upmix(const uint32_t *q, const uint16_t *s, const uint16_t *b,
                                  const float *down, const float *normed, int hc, int d, int R,
                                  int n, float *mixed, void *stream) {
    if (n <= 0) return 0;
    if (hc < 1 || hc > HC_MAX) return (int)hipErrorInvalidValue;
    /* at least 4 lanes per row: a block then has at most 64 columns, one
     * per mixer thread of the smallest workgroup (hc = 1) */
    const int lpr = max(4, hc_pick_lpr(R)), ch = R / 32;
    const int P = (ch + lpr - 1) / lpr;
    const int cbw = HU_RIT * (64 / lpr);
    const int ncb = (d + cbw - 1) / cbw;
    const int tb = hc_tokens_per_task(n, ncb);
    HcUpArgs a{q, s, b, down, normed, mixed, hc, d, R, n, tb};
    const dim3 grid((unsigned)(((n + tb - 1) / tb) * ncb)), blk(64 * hc);
    hipStream_t st = (hipStream_t)stream;
#define HU(L, PP) hipLaunchKernelGGL((k_hc_upmix<L, PP>), grid, blk, 0, st, a)
    if (lpr == 64) {
        if (P == 1) HU(64, 1);
        else return (int)hipErrorInvalidValue;
    } else if (lpr == 32) HU(32, 1);
    else if (lpr == 16) HU(16, 1);
    else if (lpr == 8) HU(8, 1);
    else HU(4, 1);
#undef HU
    return QK_CHECK_LAUNCH();
}

extern "C" int qk_launch_hc_inject(const float *inject, const float *out, int hc, int d, int n,
                                   float *hyper, void *stream) {
    if (n <= 0) return 0;
    if (d % 4) return (int)hipErrorInvalidValue;
    const dim3 grid(n, (d + 1023) / 1024);
    hipLaunchKernelGGL(k_hc_inject, grid, dim3(256), 0, (hipStream_t)stream, inject, out, hc, d,
                       hyper);
    return QK_CHECK_LAUNCH();
}
