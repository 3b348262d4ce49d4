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
 * in three launches:
 *   k_hc_norm_inject  one token per workgroup: the copy norms, normed, and
 *                     the hc inject dots (bf16 weights, 64 KiB per token);
 *   k_hc_linear       q4 GEMV normed -> down outputs (before silu);
 *   k_hc_upmix        q4 GEMV silu(down/hc) -> gates, with the mean over the
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

__device__ __forceinline__ float hc_wave_sum(float v) { return qk_group_sum<64>(v); }

struct HcNormArgs {
    const float *hyper;        /* [n, hc*d] */
    const float *norm_w;       /* [hc*d] */
    const uint16_t *inject_w;  /* [hc, hc*d] bf16 */
    float *normed;             /* [n, hc*d] */
    float *inject;             /* [n, hc] */
    int hc, d;
    float eps;
};

/*
 * grid = n, 1024 threads, 4 columns per thread per step.  Copy h's norm is
 * kernel_rmsnorm_grouped's (kernel.c:22-36): r = 1/sqrt(ss/d + eps),
 * normed = (x * r) * w; the inject dots sum in a fixed order (per thread,
 * then the wave butterfly, then the 16 waves in order).
 */
__global__ __launch_bounds__(1024) void k_hc_norm_inject(HcNormArgs a) {
    __shared__ float s_ss[HC_MAX][16];
    __shared__ float s_ip[HC_MAX][16];
    const int t = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int D = a.hc * a.d;
    const float *x = a.hyper + (size_t)t * D;
    for (int h = 0; h < a.hc; h++) {
        float ss = 0.0f;
        for (int i = tid * 4; i < a.d; i += 4096) {
            const float4 v = qk_ld((const float4 *)(x + (size_t)h * a.d + i));
            ss = fmaf(v.x, v.x, ss);
            ss = fmaf(v.y, v.y, ss);
            ss = fmaf(v.z, v.z, ss);
            ss = fmaf(v.w, v.w, ss);
        }
        ss = hc_wave_sum(ss);
        if (lane == 0) s_ss[h][wave] = ss;
    }
    __syncthreads();
    float ip[HC_MAX];
#pragma unroll
    for (int j = 0; j < HC_MAX; j++) ip[j] = 0.0f;
    for (int h = 0; h < a.hc; h++) {
        float ss = 0.0f;
#pragma unroll
        for (int w = 0; w < 16; w++) ss += s_ss[h][w];
        const float r = 1.0f / sqrtf(ss / (float)a.d + a.eps);
        for (int i = tid * 4; i < a.d; i += 4096) {
            const size_t c = (size_t)h * a.d + i;
            const float4 v = qk_ld((const float4 *)(x + c));
            const float4 w = qk_ld((const float4 *)(a.norm_w + c));
            const float4 y = make_float4(v.x * r * w.x, v.y * r * w.y, v.z * r * w.z, v.w * r * w.w);
            qk_st((float4 *)(a.normed + (size_t)t * D + c), y);
#pragma unroll
            for (int j = 0; j < HC_MAX; j++) {
                if (j < a.hc) {
                    const uint2 wb = qk_ld((const uint2 *)(a.inject_w + (size_t)j * D + c));
                    ip[j] = fmaf(y.x, qk_bf16_lo(wb.x), ip[j]);
                    ip[j] = fmaf(y.y, qk_bf16_hi(wb.x), ip[j]);
                    ip[j] = fmaf(y.z, qk_bf16_lo(wb.y), ip[j]);
                    ip[j] = fmaf(y.w, qk_bf16_hi(wb.y), ip[j]);
                }
            }
        }
    }
#pragma unroll
    for (int j = 0; j < HC_MAX; j++) {
        if (j < a.hc) {
            const float v = hc_wave_sum(ip[j]);
            if (lane == 0) s_ip[j][wave] = v;
        }
    }
    __syncthreads();
    if (tid < a.hc) {
        float v = 0.0f;
#pragma unroll
        for (int w = 0; w < 16; w++) v += s_ip[tid][w];
        a.inject[(size_t)t * a.hc + tid] = 2.0f * qk_sigmoid(v * (1.0f / (float)a.hc));
    }
}

/* ---------------------------------------------------------------- q4 GEMV */

struct HcLinArgs {
    const uint32_t *q;  /* [N, K/8] */
    const uint16_t *s;  /* [N, K/64] bf16 */
    const uint16_t *b;
    const float *x;     /* [n, K] */
    float *out;         /* [n, N] */
    int K, N, n, tb;    /* tb: tokens per task */
};

#define HC_RITER 2

/*
 * out = x . W^T for a q4 W.  Task = (block of tb tokens, block of RB rows);
 * the workgroup keeps its rows' codes in registers and walks its tokens,
 * prefetching the next token's activations under the current token's math
 * (the lane mapping of the expert GEMV: LPR lanes per row, P chunks of 32
 * columns per lane).
 */
template <int LPR, int P>
__global__ __launch_bounds__(256) void k_hc_linear(HcLinArgs a) {
    constexpr int RPW = 64 / LPR;
    constexpr int RB = 4 * RPW * HC_RITER;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int sub = lane % LPR, rsub = lane / LPR;
    const int CH = a.K >> 5, G = a.K >> 6;
    const size_t wrow = (size_t)a.K >> 3;
    const int tps = (a.N + RB - 1) / RB;
    const int tblk = blockIdx.x / tps, rb = blockIdx.x - tblk * tps;
    const int t0 = tblk * a.tb;
    const int m = min(a.tb, a.n - t0);
    if (m <= 0) return;
    const int rbase = rb * RB + wave * RPW * HC_RITER;
    uint4 wq[HC_RITER][P];
    uint16_t rs[HC_RITER][P], rbi[HC_RITER][P];
    float ws[HC_RITER][P], wb[HC_RITER][P];
    XRaw<P, false> xr;
    load_xraw<LPR, P, false>(a.x, (size_t)t0, a.K, sub, xr);
#pragma unroll
    for (int it = 0; it < HC_RITER; it++) {
        const int r0 = rbase + it * RPW + rsub;
        const int r = r0 < a.N ? r0 : 0;
#pragma unroll
        for (int ps = 0; ps < P; ps++) {
            const int c0 = ps * LPR + sub;
            const int c = c0 < CH ? c0 : 0;
            wq[it][ps] = qk_ld((const uint4 *)(a.q + (size_t)r * wrow) + c);
            rs[it][ps] = qk_ld(a.s + (size_t)r * G + (c >> 1));
            rbi[it][ps] = qk_ld(a.b + (size_t)r * G + (c >> 1));
        }
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int it = 0; it < HC_RITER; it++) {
        const bool rok = rbase + it * RPW + rsub < a.N;
#pragma unroll
        for (int ps = 0; ps < P; ps++) {
            const bool ok = rok && ps * LPR + sub < CH;
            ws[it][ps] = ok ? qk_bf16(rs[it][ps]) : 0.0f;
            wb[it][ps] = ok ? qk_bf16(rbi[it][ps]) : 0.0f;
            if (!ok) wq[it][ps] = make_uint4(0u, 0u, 0u, 0u);
        }
    }
    for (int j = 0; j < m; j++) {
        XPairs<LPR, P, false> xp;
        convert_xraw<LPR, P, false>(xr, a.K, sub, xp);
        if (j + 1 < m) load_xraw<LPR, P, false>(a.x, (size_t)(t0 + j + 1), a.K, sub, xr);
#pragma unroll
        for (int it = 0; it < HC_RITER; it++) {
            const float v = qk_group_sum<LPR>(row_part<LPR, P, false>(wq[it], ws[it], wb[it], xp));
            const int r = rbase + it * RPW + rsub;
            if (sub == 0 && r < a.N) qk_st(a.out + (size_t)(t0 + j) * a.N + r, v);
        }
    }
}

/* ------------------------------------------------------- up + mean mix */

struct HcUpArgs {
    const uint32_t *q;    /* input_mix_weight_up [hc*d, R/8] */
    const uint16_t *s;    /* [hc*d, R/64] */
    const uint16_t *b;
    const float *down;    /* [n, R] down outputs before silu */
    const float *normed;  /* [n, hc*d] */
    float *mixed;         /* [n, d] */
    int hc, d, R, n, tb;
};

#define HU_RIT 4

/* this lane's chunks of w = silu(down / hc) as bf16 pairs (kernel_scale
 * then kernel_silu, model.c:757-758) */
template <int LPR, int P>
__device__ __forceinline__ void hc_convert_silu(const XRaw<P, false> &xr, int K, int sub, float inv_hc,
                                                XPairs<LPR, P, false> &xp) {
    const int CH = K >> 5;
#pragma unroll
    for (int ps = 0; ps < P; ps++) {
        const bool ok = ps * LPR + sub < CH;
        xp.xs[ps] = 0.0f;
#pragma unroll
        for (int w = 0; w < 4; w++) {
            const float4 a0 = xr.f[ps][2 * w], a1 = xr.f[ps][2 * w + 1];
            float v[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
#pragma unroll
            for (int j = 0; j < 8; j++) v[j] = ok ? qk_silu(v[j] * inv_hc) : 0.0f;
            qk_f32x8_to_pairs(v, &xp.hi[ps][4 * w], &xp.lo[ps][4 * w], xp.xs[ps]);
        }
    }
}

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
    const float inv_hc = 1.0f / (float)a.hc;
    uint4 wq[HU_RIT][P];
    uint16_t rs[HU_RIT][P], rbi[HU_RIT][P];
    float ws[HU_RIT][P], wb[HU_RIT][P];
    XRaw<P, false> xr;
    load_xraw<LPR, P, false>(a.down, (size_t)t0, K, sub, xr);
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
        hc_convert_silu<LPR, P>(xr, K, sub, inv_hc, xp);
        if (j + 1 < m) load_xraw<LPR, P, false>(a.down, (size_t)(t + 1), K, sub, xr);
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
    return hc >= 1 && hc <= HC_MAX && d > 0 && d % 64 == 0 && R >= 64 && R % 64 == 0 &&
           R <= 2048 && (long long)hc * d <= 8192;
}

extern "C" int qk_launch_hc_norm_inject(const float *hyper, const float *norm_w,
                                        const uint16_t *inject_w, int hc, int d, int n, float eps,
                                        float *normed, float *inject, void *stream) {
    if (n <= 0) return 0;
    HcNormArgs a{hyper, norm_w, inject_w, normed, inject, hc, d, eps};
    hipLaunchKernelGGL(k_hc_norm_inject, dim3(n), dim3(1024), 0, (hipStream_t)stream, a);
    return QK_CHECK_LAUNCH();
}

extern "C" int qk_launch_hc_linear(const uint32_t *q, const uint16_t *s, const uint16_t *b,
                                   const float *x, int n, int K, int N, float *out, void *stream) {
    if (n <= 0) return 0;
    const int lpr = hc_pick_lpr(K), ch = K / 32;
    const int P = (ch + lpr - 1) / lpr;
    const int rb = 4 * (64 / lpr) * HC_RITER;
    const int tps = (N + rb - 1) / rb;
    const int tb = hc_tokens_per_task(n, tps);
    HcLinArgs a{q, s, b, x, out, K, N, n, tb};
    const dim3 grid((unsigned)(((n + tb - 1) / tb) * tps));
    hipStream_t st = (hipStream_t)stream;
#define HL(L, PP) hipLaunchKernelGGL((k_hc_linear<L, PP>), grid, dim3(256), 0, st, a)
    if (lpr == 64) {
        if (P == 1) HL(64, 1);
        else if (P == 2) HL(64, 2);
        else if (P <= 4) HL(64, 4);
        else return (int)hipErrorInvalidValue;
    } else if (lpr == 32) HL(32, 1);
    else if (lpr == 16) HL(16, 1);
    else if (lpr == 8) HL(8, 1);
    else if (lpr == 4) HL(4, 1);
    else HL(2, 1);
#undef HL
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
