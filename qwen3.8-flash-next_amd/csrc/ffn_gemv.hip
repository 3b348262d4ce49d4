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
 * Work item ("segment"): segment 0 is the shared expert over all n tokens
 * (rows n*k .. n*k+n-1 of the output); segment i >= 1 is entry i-1 of the
 * segment table: one routed expert with its contiguous run of dispatch
 * positions.  A task is (segment, block of RB output rows); workgroups loop
 * over tasks.  Shared-expert tasks come first and need no routing data.
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
    const int32_t *perm, *segtab;
    int K, N, n, k, E;
    int max_m;              /* skip segments with >= max_m rows (0: none skipped) */
    int in_by_pos;          /* input row = dispatch position (down) instead of token */
};

#define GV_RITER 2

template <int LPR, int P, bool XBF16>
struct XPairs {
    uint32_t hi[P][16];
    uint32_t lo[XBF16 ? 1 : P][XBF16 ? 1 : 16];
    float xs[P];
};

/* raw activations of this lane's chunks of one input row (loaded from a
 * clamped chunk; chunks past the row are zeroed when converted) */
template <int P, bool XBF16>
struct XRaw {
    uint4 d[XBF16 ? P : 1][4];
    float4 f[XBF16 ? 1 : P][8];
};

template <int LPR, int P, bool XBF16>
__device__ __forceinline__ void load_xraw(const void *x, size_t row, int K, int sub,
                                          XRaw<P, XBF16> &xr) {
    const int CH = K >> 5;
#pragma unroll
    for (int ps = 0; ps < P; ps++) {
        const int c0 = ps * LPR + sub;
        const int c = c0 < CH ? c0 : 0;
        if (XBF16) {
            const uint4 *src = (const uint4 *)((const uint16_t *)x + row * K) + 4 * c;
#pragma unroll
            for (int w = 0; w < 4; w++) xr.d[XBF16 ? ps : 0][w] = qk_ld(src + w);
        } else {
            const float4 *src = (const float4 *)((const float *)x + row * K) + 8 * c;
#pragma unroll
            for (int w = 0; w < 8; w++) xr.f[XBF16 ? 0 : ps][w] = qk_ld(src + w);
        }
    }
}

/* raw activations -> bf16 pairs (hi, and lo for f32 input) + chunk sums */
template <int LPR, int P, bool XBF16>
__device__ __forceinline__ void convert_xraw(const XRaw<P, XBF16> &xr, int K, int sub,
                                             XPairs<LPR, P, XBF16> &xp) {
    const int CH = K >> 5;
#pragma unroll
    for (int ps = 0; ps < P; ps++) {
        const bool ok = ps * LPR + sub < CH;
        xp.xs[ps] = 0.0f;
        if (XBF16) {
#pragma unroll
            for (int w = 0; w < 4; w++) {
                uint4 d = xr.d[XBF16 ? ps : 0][w];
                if (!ok) d = make_uint4(0u, 0u, 0u, 0u);
                qk_bf16x8_to_pairs(d, &xp.hi[ps][4 * w]);
                float s = 0.0f;
                s += qk_bf16_lo(d.x) + qk_bf16_hi(d.x);
                s += qk_bf16_lo(d.y) + qk_bf16_hi(d.y);
                s += qk_bf16_lo(d.z) + qk_bf16_hi(d.z);
                s += qk_bf16_lo(d.w) + qk_bf16_hi(d.w);
                xp.xs[ps] += s;
            }
        } else {
#pragma unroll
            for (int w = 0; w < 4; w++) {
                const float4 a0 = xr.f[XBF16 ? 0 : ps][2 * w], a1 = xr.f[XBF16 ? 0 : ps][2 * w + 1];
                float v[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
                if (!ok)
#pragma unroll
                    for (int j = 0; j < 8; j++) v[j] = 0.0f;
                qk_f32x8_to_pairs(v, &xp.hi[ps][4 * w], &xp.lo[XBF16 ? 0 : ps][XBF16 ? 0 : 4 * w],
                                  xp.xs[ps]);
            }
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
    const int tps = (a.N + RB - 1) / RB;
    const int U = min(max(a.segtab[0], 0), a.E); /* first used by routed tasks */
    for (int task = blockIdx.x;; task += gridDim.x) {
        const int seg = task / tps, rb = task - seg * tps;
        const bool shared = seg == 0;
        if (!shared && seg > U) break;
        int p0, m;
        const uint32_t *q[NMAT];
        const uint16_t *sc[NMAT], *bi[NMAT];
        if (!shared) {
            const int e = a.segtab[3 * seg - 2];
            p0 = a.segtab[3 * seg - 1];
            m = a.segtab[3 * seg];
            if (e < 0 || e >= a.E || p0 < 0 || m < 0 || p0 + m > a.n * a.k) continue;
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
        if (a.max_m > 0 && m >= a.max_m) continue; /* taken by the MFMA kernel */
        /* this lane's rows: rbase + it*RPW + rsub */
        const int rbase = rb * RB + wave * RPWAVE;
        /* input row of the segment's first token: its (possible) perm load
         * goes first, so waiting for it does not wait for the weights */
        auto in_row_of = [&](int j) -> long {
            const int p = p0 + j;
            if (a.in_by_pos) return p;
            if (shared) return j;
            if (a.n == 1) return 0;
            const int f = qk_ld(a.perm + p);
            return (f < 0 || f >= a.n * a.k) ? -1 : f / a.k;
        };
        XRaw<P, XBF16> xr;
        long row_next = m > 0 ? in_row_of(0) : -1;
        if (row_next >= 0) load_xraw<LPR, P, XBF16>(a.x, (size_t)row_next, a.K, sub, xr);
        uint4 wq[NMAT][GV_RITER][P];
        uint16_t rs[NMAT][GV_RITER][P], rbi[NMAT][GV_RITER][P];
        float ws[NMAT][GV_RITER][P], wb[NMAT][GV_RITER][P];
        /* all weight loads of the task issue back to back from clamped
         * addresses (the scheduling barrier keeps the conversions below from
         * being interleaved with, and so waiting between, the loads);
         * out-of-range rows/chunks are zeroed by select afterwards */
#pragma unroll
        for (int it = 0; it < GV_RITER; it++) {
            const int r0 = rbase + it * RPW + rsub;
            const int r = r0 < a.N ? r0 : 0;
#pragma unroll
            for (int ps = 0; ps < P; ps++) {
                const int c0 = ps * LPR + sub;
                const int c = c0 < CH ? c0 : 0;
#pragma unroll
                for (int mt = 0; mt < NMAT; mt++) {
                    wq[mt][it][ps] = qk_ld((const uint4 *)(q[mt] + (size_t)r * wrow) + c);
                    rs[mt][it][ps] = qk_ld(sc[mt] + (size_t)r * G + (c >> 1));
                    rbi[mt][it][ps] = qk_ld(bi[mt] + (size_t)r * G + (c >> 1));
                }
            }
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int it = 0; it < GV_RITER; it++) {
            const bool rok = rbase + it * RPW + rsub < a.N;
#pragma unroll
            for (int ps = 0; ps < P; ps++) {
                const bool ok = rok && ps * LPR + sub < CH;
#pragma unroll
                for (int mt = 0; mt < NMAT; mt++) {
                    ws[mt][it][ps] = ok ? qk_bf16(rs[mt][it][ps]) : 0.0f;
                    wb[mt][it][ps] = ok ? qk_bf16(rbi[mt][it][ps]) : 0.0f;
                    if (!ok) wq[mt][it][ps] = make_uint4(0u, 0u, 0u, 0u);
                }
            }
        }
        for (int j = 0; j < m; j++) {
            const int p = p0 + j;
            const long row_cur = row_next;
            XPairs<LPR, P, XBF16> xp;
            convert_xraw<LPR, P, XBF16>(xr, a.K, sub, xp);
            /* prefetch the next token's activations under this token's math */
            if (j + 1 < m) {
                row_next = in_row_of(j + 1);
                if (row_next >= 0) load_xraw<LPR, P, XBF16>(a.x, (size_t)row_next, a.K, sub, xr);
            }
            if (row_cur < 0) continue;
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
                    qk_st(a.out + (size_t)p * a.N + r, v);
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
    /* workgroups loop over tasks until they pass the segment count, so the
     * grid only bounds the parallelism */
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
                                int n, const int32_t *perm, const int32_t *segtab, int max_m,
                                float *h, void *stream) {
    if (n <= 0) return 0;
    GemvArgs a;
    a.q[0] = W->gate_q; a.s[0] = W->gate_s; a.b[0] = W->gate_b;
    a.q[1] = W->up_q;   a.s[1] = W->up_s;   a.b[1] = W->up_b;
    a.sq[0] = W->sh_gate_q; a.ss[0] = W->sh_gate_s; a.sb[0] = W->sh_gate_b;
    a.sq[1] = W->sh_up_q;   a.ss[1] = W->sh_up_s;   a.sb[1] = W->sh_up_b;
    a.x = x;
    a.out = h;
    a.perm = perm;
    a.segtab = segtab;
    a.K = s.H;
    a.N = s.I;
    a.n = n;
    a.k = s.k;
    a.E = s.E;
    a.max_m = max_m;
    a.in_by_pos = 0;
    const int max_seg = n * s.k < s.E ? n * s.k : s.E;
    hipStream_t st = (hipStream_t)stream;
    return x_bf16 ? launch_gemv<2, true>(a, max_seg, st) : launch_gemv<2, false>(a, max_seg, st);
}

extern "C" int qk_launch_down(const qmoe_layer_weights *W, qk_shape s, const float *h, int n,
                              const int32_t *segtab, int max_m, float *y, void *stream) {
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
    a.perm = nullptr;
    a.segtab = segtab;
    a.K = s.I;
    a.N = s.H;
    a.n = n;
    a.k = s.k;
    a.E = s.E;
    a.max_m = max_m;
    a.in_by_pos = 1;
    const int max_seg = n * s.k < s.E ? n * s.k : s.E;
    return launch_gemv<1, false>(a, max_seg, (hipStream_t)stream);
}
