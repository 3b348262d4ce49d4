/*
 * ffn_gemv.hip -- grouped q4 GEMV for the expert FFN (decode shapes).
 *
 * Replaces the per-expert loop of the reference C port, model.c:1338-1387
 * (gather, gemm_fp32 x3 on fp32-dequantised weights, silu, mul) and the
 * shared expert model.c:1388-1395 (linear_forward -> gemm_q4).  The weights
 * stay in the checkpoint layout and are dequantised in registers with the
 * per-group identity of gemm_q4 (kernel.c:279-282):
 *     sum_k x_k (q_k s + b) = s * sum_k x_k q_k + b * sum_k x_k.
 *
 * Work item ("segment"): one expert with its contiguous run of dispatch
 * positions offsets[e]..offsets[e+1] (experts taken from the unique list),
 * plus one extra segment for the shared expert over all n tokens.  A task is
 * (segment, block of RB output rows); workgroups loop over tasks.
 *
 * Lane mapping: a weight row of K codes is cut into 32-code chunks (one
 * 16-byte load = four u32 words); LPR lanes share a row, so a wavefront
 * instruction reads 64 contiguous 16-byte pieces.  Codes become bf16 pairs
 * (128+q) and meet activation pairs in v_dot2c_f32_bf16; f32 activations
 * are split into hi+lo bf16 pairs (16 significant bits).
 */
#include "qk_device.h"

struct GemvArgs {
    const uint32_t *q[2];   /* routed [E, N, K/8] */
    const uint16_t *s[2];   /* routed [E, N, K/64] */
    const uint16_t *b[2];
    const uint32_t *sq[2];  /* shared [N, K/8] */
    const uint16_t *ss[2];
    const uint16_t *sb[2];
    const void *x;          /* input rows: tokens (gate/up) or dispatch positions (down) */
    float *out;             /* [n*k+n, N] */
    const int32_t *perm, *offsets, *unique;
    int K, N, n, k, E;
    int in_by_pos;          /* input row = dispatch position (down) instead of token */
};

#define GV_RITER 2

template <int LPR, int P, bool XBF16>
struct XPairs {
    uint32_t hi[P][16];
    uint32_t lo[XBF16 ? 1 : P][XBF16 ? 1 : 16];
    float xs[P];
};

template <int LPR, int P, bool XBF16>
__device__ __forceinline__ void load_xpairs(const void *x, size_t row, int K, int sub,
                                            XPairs<LPR, P, XBF16> &xp) {
    const int CH = K >> 5;
#pragma unroll
    for (int ps = 0; ps < P; ps++) {
        const int c = ps * LPR + sub;
        xp.xs[ps] = 0.0f;
        if (c < CH) {
            if (XBF16) {
                const uint4 *src = (const uint4 *)((const uint16_t *)x + row * K) + 4 * c;
#pragma unroll
                for (int w = 0; w < 4; w++) {
                    uint4 d = src[w];
                    qk_bf16x8_to_pairs(d, &xp.hi[ps][4 * w]);
                    float s = 0.0f;
                    s += qk_bf16_lo(d.x) + qk_bf16_hi(d.x);
                    s += qk_bf16_lo(d.y) + qk_bf16_hi(d.y);
                    s += qk_bf16_lo(d.z) + qk_bf16_hi(d.z);
                    s += qk_bf16_lo(d.w) + qk_bf16_hi(d.w);
                    xp.xs[ps] += s;
                }
            } else {
                const float4 *src = (const float4 *)((const float *)x + row * K) + 8 * c;
#pragma unroll
                for (int w = 0; w < 4; w++) {
                    float4 a0 = src[2 * w], a1 = src[2 * w + 1];
                    float v[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
                    qk_f32x8_to_pairs(v, &xp.hi[ps][4 * w], &xp.lo[XBF16 ? 0 : ps][XBF16 ? 0 : 4 * w],
                                      xp.xs[ps]);
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < 16; i++) xp.hi[ps][i] = 0u;
            if (!XBF16)
#pragma unroll
                for (int i = 0; i < 16; i++) xp.lo[XBF16 ? 0 : ps][i] = 0u;
        }
    }
}

/* sum over one 32-code chunk of x * (128 + q) */
template <int LPR, int P, bool XBF16>
__device__ __forceinline__ float chunk_dot(uint4 q4, const XPairs<LPR, P, XBF16> &xp, int ps) {
    float d = 0.0f;
    const uint32_t words[4] = {q4.x, q4.y, q4.z, q4.w};
#pragma unroll
    for (int w = 0; w < 4; w++) {
        uint32_t pr[4];
        qk_codes_to_pairs(words[w], pr);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            d = qk_dot2(xp.hi[ps][4 * w + i], pr[i], d);
            if (!XBF16) d = qk_dot2(xp.lo[XBF16 ? 0 : ps][XBF16 ? 0 : 4 * w + i], pr[i], d);
        }
    }
    return d;
}

template <int NMAT, int LPR, int P, bool XBF16>
__global__ __launch_bounds__(256) void k_q4gemv(GemvArgs a) {
    constexpr int RPW = 64 / LPR;
    constexpr int RPWAVE = RPW * GV_RITER;
    constexpr int RB = 4 * RPWAVE;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int sub = lane % LPR, rsub = lane / LPR;
    const int CH = a.K >> 5, G = a.K >> 6;
    const size_t wrow = (size_t)a.K >> 3; /* u32 words per weight row */
    const int U = a.unique[0];
    const int tps = (a.N + RB - 1) / RB;
    const int ntask = (U + 1) * tps;
    for (int task = blockIdx.x; task < ntask; task += gridDim.x) {
        const int seg = task / tps, rb = task - seg * tps;
        const bool shared = seg == U;
        int p0, m;
        const uint32_t *q[NMAT];
        const uint16_t *sc[NMAT], *bi[NMAT];
        if (!shared) {
            const int e = a.unique[1 + seg];
            if (e < 0 || e >= a.E) continue;
            p0 = a.offsets[e];
            m = a.offsets[e + 1] - p0;
            if (p0 < 0 || m < 0 || p0 + m > a.n * a.k) continue;
#pragma unroll
            for (int mt = 0; mt < NMAT; mt++) {
                q[mt] = a.q[mt] + (size_t)e * a.N * wrow;
                sc[mt] = a.s[mt] + (size_t)e * a.N * G;
                bi[mt] = a.b[mt] + (size_t)e * a.N * G;
            }
        } else {
            p0 = a.n * a.k;
            m = a.n;
#pragma unroll
            for (int mt = 0; mt < NMAT; mt++) {
                q[mt] = a.sq[mt];
                sc[mt] = a.ss[mt];
                bi[mt] = a.sb[mt];
            }
        }
        /* this lane's rows: rbase + it*RPW + rsub */
        const int rbase = rb * RB + wave * RPWAVE;
        uint4 wq[NMAT][GV_RITER][P];
        float ws[NMAT][GV_RITER][P], wb[NMAT][GV_RITER][P];
#pragma unroll
        for (int it = 0; it < GV_RITER; it++) {
            const int r = rbase + it * RPW + rsub;
#pragma unroll
            for (int ps = 0; ps < P; ps++) {
                const int c = ps * LPR + sub;
                const bool ok = r < a.N && c < CH;
#pragma unroll
                for (int mt = 0; mt < NMAT; mt++) {
                    if (ok) {
                        wq[mt][it][ps] = ((const uint4 *)(q[mt] + (size_t)r * wrow))[c];
                        ws[mt][it][ps] = qk_bf16(sc[mt][(size_t)r * G + (c >> 1)]);
                        wb[mt][it][ps] = qk_bf16(bi[mt][(size_t)r * G + (c >> 1)]);
                    } else {
                        wq[mt][it][ps] = make_uint4(0x0u, 0x0u, 0x0u, 0x0u);
                        ws[mt][it][ps] = 0.0f;
                        wb[mt][it][ps] = 0.0f;
                    }
                }
            }
        }
        for (int j = 0; j < m; j++) {
            const int p = p0 + j;
            size_t in_row;
            if (a.in_by_pos) {
                in_row = (size_t)p;
            } else if (shared) {
                in_row = (size_t)j;
            } else {
                const int f = a.perm[p];
                if (f < 0 || f >= a.n * a.k) continue;
                in_row = (size_t)(f / a.k);
            }
            XPairs<LPR, P, XBF16> xp;
            load_xpairs<LPR, P, XBF16>(a.x, in_row, a.K, sub, xp);
#pragma unroll
            for (int it = 0; it < GV_RITER; it++) {
                float acc[NMAT];
#pragma unroll
                for (int mt = 0; mt < NMAT; mt++) {
                    float part = 0.0f;
#pragma unroll
                    for (int ps = 0; ps < P; ps++) {
                        const float d = chunk_dot<LPR, P, XBF16>(wq[mt][it][ps], xp, ps);
                        const float dq = fmaf(-128.0f, xp.xs[ps], d);
                        part = fmaf(ws[mt][it][ps], dq, fmaf(wb[mt][it][ps], xp.xs[ps], part));
                    }
                    acc[mt] = qk_group_sum<LPR>(part);
                }
                const int r = rbase + it * RPW + rsub;
                if (sub == 0 && r < a.N) {
                    float v = NMAT == 2 ? qk_silu(acc[0]) * acc[NMAT - 1] : acc[0];
                    a.out[(size_t)p * a.N + r] = v;
                }
            }
        }
    }
}

static int pick_lpr(int K) {
    int ch = K / 32;
    int l = 2;
    while (l < ch && l < 64) l <<= 1;
    return l;
}

template <int NMAT, bool XBF16>
static int launch_gemv(const GemvArgs &a, int max_seg, hipStream_t st) {
    const int lpr = pick_lpr(a.K);
    const int ch = a.K / 32;
    const int P = (ch + lpr - 1) / lpr;
    const int rb = 4 * (64 / lpr) * GV_RITER;
    const int tps = (a.N + rb - 1) / rb;
    long long tasks = (long long)(max_seg + 1) * tps;
    const int grid = (int)(tasks < 4096 ? tasks : 4096);
#define GV_LAUNCH(L, PP) \
    hipLaunchKernelGGL((k_q4gemv<NMAT, L, PP, XBF16>), dim3(grid), dim3(256), 0, st, a)
    if (lpr == 64) {
        if (P == 1) GV_LAUNCH(64, 1);
        else if (P == 2) GV_LAUNCH(64, 2);
        else if (P <= 4) GV_LAUNCH(64, 4);
        else return (int)hipErrorInvalidValue;
    } else if (lpr == 32) GV_LAUNCH(32, 1);
    else if (lpr == 16) GV_LAUNCH(16, 1);
    else if (lpr == 8) GV_LAUNCH(8, 1);
    else if (lpr == 4) GV_LAUNCH(4, 1);
    else GV_LAUNCH(2, 1);
#undef GV_LAUNCH
    return QK_CHECK_LAUNCH();
}

extern "C" int qk_launch_gateup(const qmoe_layer_weights *W, qk_shape s, const void *x, int x_bf16,
                                int n, const int32_t *perm, const int32_t *offsets,
                                const int32_t *unique, float *h, void *stream) {
    if (n <= 0) return 0;
    GemvArgs a;
    a.q[0] = W->gate_q; a.s[0] = W->gate_s; a.b[0] = W->gate_b;
    a.q[1] = W->up_q;   a.s[1] = W->up_s;   a.b[1] = W->up_b;
    a.sq[0] = W->sh_gate_q; a.ss[0] = W->sh_gate_s; a.sb[0] = W->sh_gate_b;
    a.sq[1] = W->sh_up_q;   a.ss[1] = W->sh_up_s;   a.sb[1] = W->sh_up_b;
    a.x = x;
    a.out = h;
    a.perm = perm;
    a.offsets = offsets;
    a.unique = unique;
    a.K = s.H;
    a.N = s.I;
    a.n = n;
    a.k = s.k;
    a.E = s.E;
    a.in_by_pos = 0;
    const int max_seg = n * s.k < s.E ? n * s.k : s.E;
    hipStream_t st = (hipStream_t)stream;
    return x_bf16 ? launch_gemv<2, true>(a, max_seg, st) : launch_gemv<2, false>(a, max_seg, st);
}

extern "C" int qk_launch_down(const qmoe_layer_weights *W, qk_shape s, const float *h, int n,
                              const int32_t *perm, const int32_t *offsets, const int32_t *unique,
                              float *y, void *stream) {
    if (n <= 0) return 0;
    GemvArgs a;
    a.q[0] = a.q[1] = W->down_q;
    a.s[0] = a.s[1] = W->down_s;
    a.b[0] = a.b[1] = W->down_b;
    a.sq[0] = a.sq[1] = W->sh_down_q;
    a.ss[0] = a.ss[1] = W->sh_down_s;
    a.sb[0] = a.sb[1] = W->sh_down_b;
    a.x = h;
    a.out = y;
    a.perm = perm;
    a.offsets = offsets;
    a.unique = unique;
    a.K = s.I;
    a.N = s.H;
    a.n = n;
    a.k = s.k;
    a.E = s.E;
    a.in_by_pos = 1;
    const int max_seg = n * s.k < s.E ? n * s.k : s.E;
    return launch_gemv<1, false>(a, max_seg, (hipStream_t)stream);
}
