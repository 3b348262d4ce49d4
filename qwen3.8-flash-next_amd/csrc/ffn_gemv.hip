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
#include "gemv_decode.h"
#include "gemv_parts.h"

struct GemvArgs {
    const uint32_t *q[2];   /* routed [E, N, K/8] */
    const uint16_t *s[2];   /* routed [E, N, K/g] (g = 32 << (gsh == 1)) */
    const uint16_t *b[2];
    const uint32_t *sq[2];  /* shared [N, K/8] */
    const uint16_t *ss[2];
    const uint16_t *sb[2];
    const void *x;          /* input rows: tokens (gate/up) or dispatch positions (down) */
    float *out;             /* [n*k+n, N] */
    const int32_t *perm, *segtab;
    int K, N, n, k, E;
    int max_m;              /* skip segments with >= max_m rows (0: none skipped) */
    const int32_t *seglist; /* null, or [count, segment...]: only these segments */
    int in_by_pos;          /* input row = dispatch position (down) instead of token */
    int gsh;                /* log2(group size / 32): 32-column chunk c is in group c >> gsh */
};

#define GV_RITER 2

template <int NMAT, int LPR, int P, bool XBF16>
__global__ __launch_bounds__(256) void k_q4gemv(GemvArgs a) {
    constexpr int RPW = 64 / LPR;
    constexpr int RPWAVE = RPW * GV_RITER;
    constexpr int RB = 4 * RPWAVE;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int sub = lane % LPR, rsub = lane / LPR;
    const int CH = a.K >> 5, G = a.K >> (5 + a.gsh);
    const size_t wrow = (size_t)a.K >> 3; /* u32 words per weight row */
    const int tps = (a.N + RB - 1) / RB;
    const int u_raw = a.segtab[0];
    const int nlist = a.seglist ? qk_ld(a.seglist) : 0;
    for (int task = blockIdx.x;; task += gridDim.x) {
        int seg = task / tps;
        const int rb = task - seg * tps;
        if (a.seglist) {
            if (seg >= nlist) break;
            seg = qk_ld(a.seglist + 1 + seg);
        } else if (task >= (int)gridDim.x && seg > min(max(u_raw, 0), a.E)) {
            /* past the first task the segment count is known */
            break;
        }
        const bool shared = seg == 0;
        if (seg > a.E) break;
        int p0, m;
        const uint32_t *q[NMAT];
        const uint16_t *sc[NMAT], *bi[NMAT];
        if (!shared) {
            /* the entry is read before the segment count is known (the table
             * has room for E entries), so both loads are in flight at once */
            const int e = a.segtab[3 * seg - 2];
            p0 = a.segtab[3 * seg - 1];
            m = a.segtab[3 * seg];
            if (seg > min(max(u_raw, 0), a.E)) break;
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
        /* the first 64 slots of the segment, one per lane, read at once so
         * that each token's activation load does not wait for its slot */
        const bool gathered = !a.in_by_pos && !shared && a.n != 1;
        int pv = 0;
        if (gathered && lane < m) pv = qk_ld(a.perm + p0 + lane);
        auto in_row_of = [&](int j) -> long {
            const int p = p0 + j;
            if (a.in_by_pos) return p;
            if (shared) return j;
            if (a.n == 1) return 0;
            const int f = j < 64 ? __builtin_amdgcn_readlane(pv, j) : qk_ld(a.perm + p);
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
                    rs[mt][it][ps] = qk_ld(sc[mt] + (size_t)r * G + (c >> a.gsh));
                    rbi[mt][it][ps] = qk_ld(bi[mt] + (size_t)r * G + (c >> a.gsh));
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
                for (int mt = 0; mt < NMAT; mt++)
                    acc[mt] = qk_group_sum<LPR>(
                        row_part<LPR, P, XBF16>(wq[mt][it], ws[mt][it], wb[mt][it], xp));
                const int r = rbase + it * RPW + rsub;
                if (sub == 0 && r < a.N) {
                    float v = NMAT == 2 ? qk_silu(acc[0]) * acc[NMAT - 1] : acc[0];
                    qk_st(a.out + (size_t)p * a.N + r, v);
                }
            }
        }
    }
}

/*
 * Down projection fused with the combine, for a few tokens (decode).  A
 * workgroup owns RB = 2*(64/LPR) output rows of every token and computes
 * y for those rows for every segment (the waves take segments in turn),
 * keeping y in LDS; then each (token, row) is combined exactly as
 * k_combine does: out = 0, out = fma(w, y, out) over the token's slots in
 * ascending dispatch position (ascending expert id), out = fma(g, y_shared,
 * out), then the optional residual x + out.  The y values are computed with
 * the lane mapping and arithmetic of k_q4gemv<1, LPR, P, false>, so the
 * result is bit-identical to qk_launch_down followed by qk_launch_combine.
 */
struct DcArgs {
    const uint32_t *q, *sq;       /* routed [E, N, K/8], shared [N, K/8] */
    const uint16_t *s, *b, *ss, *sb;
    const float *h;               /* [n*k+n, K], rows in dispatch order */
    const int32_t *segtab, *pos;  /* pos [n*k]: dispatch position of slot t*k+s */
    const float *w, *sg;          /* [n, k], [n] */
    const void *xres;             /* [n, N] or null */
    float *out;                   /* [n, N] or null (with hyper) */
    float *hyper;                 /* [n, hc, N] or null: hyper[t, j] += inject[t, j] * out[t] */
    const float *inject;          /* [n, hc] */
    int K, N, n, k, E, xbf16, hc;
    int gsh;                      /* log2(group size / 32), as GemvArgs */
};

#define DC_WAVES 16

template <int LPR, int P>
__global__ __launch_bounds__(64 * DC_WAVES) void k_down_combine(DcArgs a,
                                                                const int32_t *__restrict__ segtab) {
    constexpr int RPW = 64 / LPR;
    constexpr int RB = RPW * GV_RITER;
    constexpr bool SHARE = P == 1 && (RPW == 2 || RPW == 4); /* convert_xshare */
    constexpr int NG = 4 / (RPW < 4 ? RPW : 4);
    extern __shared__ float dc_lds[];
    const int nk = a.n * a.k;
    float *s_y = dc_lds;                              /* [(nk + n) * RB] */
    float *s_w = s_y + (nk + a.n) * RB;               /* [nk] slot weights, position order */
    int *s_p = (int *)(s_w + nk);                     /* [nk] slot positions, ascending */
    /* per wave, when SHARE: [LPR][36] activation exchange (16-byte aligned) */
    uint32_t *s_x = (uint32_t *)dc_lds + ((((nk + a.n) * RB + 2 * nk) + 3) & ~3);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int sub = lane % LPR, rsub = lane / LPR;
    const int CH = a.K >> 5, G = a.K >> (5 + a.gsh);
    const size_t wrow = (size_t)a.K >> 3;
    const int r0 = blockIdx.x * RB;
    const int u_raw = segtab[0];

    /* each token's slots ranked by dispatch position (invalid last), by the
     * waves counted from the last: the first waves start their segments'
     * loads at once (wave 0 holds the shared expert, which needs no table),
     * and with k + 1 < DC_WAVES segments the last waves have none */
    for (int t = DC_WAVES - 1 - wave; t < a.n; t += DC_WAVES) {
        int p = 0x7FFFFFFF;
        float wt = 0.0f;
        if (lane < a.k) {
            p = a.pos[(size_t)t * a.k + lane];
            wt = a.w[(size_t)t * a.k + lane];
            if (p < 0 || p >= nk) {
                p = 0x7FFFFFFE;
                wt = 0.0f;
            }
        }
        /* rank by (position, slot): invalid slots share one position */
        int rank = 0;
        for (int s2 = 0; s2 < a.k; s2++) {
            const int q = __builtin_amdgcn_readlane(p, s2);
            rank += (q < p || (q == p && s2 < lane)) ? 1 : 0;
        }
        if (lane < a.k) {
            s_p[t * a.k + rank] = p;
            s_w[t * a.k + rank] = wt;
        }
    }

    /* y for this workgroup's rows, one segment per wave at a time */
    for (int seg = wave; seg <= a.E; seg += DC_WAVES) {
        const bool shared = seg == 0;
        /* past the first round the segment count is known: stop before
         * reading an entry that does not exist */
        if (seg >= DC_WAVES && seg > min(max(u_raw, 0), a.E)) break;
        int p0, m;
        const uint32_t *q;
        const uint16_t *sc, *bi;
        if (!shared) {
            /* entry and count are read together (the table has room for E) */
            const int e = segtab[3 * seg - 2];
            p0 = segtab[3 * seg - 1];
            m = segtab[3 * seg];
            if (seg > min(max(u_raw, 0), a.E)) break;
            if (e < 0 || e >= a.E || p0 < 0 || m < 0 || p0 + m > nk) continue;
            q = a.q + (size_t)e * a.N * wrow;
            sc = a.s + (size_t)e * a.N * G;
            bi = a.b + (size_t)e * a.N * G;
        } else {
            p0 = nk;
            m = a.n;
            q = a.sq;
            sc = a.ss;
            bi = a.sb;
        }
        XRaw<P, false> xr;
        XShare<NG> xq;
        if (m > 0) {
            if (SHARE) load_xshare<NG>(a.h, (size_t)p0, a.K, sub, rsub, xq);
            else load_xraw<LPR, P, false>(a.h, (size_t)p0, a.K, sub, xr);
        }
        uint4 wq[GV_RITER][P];
        uint16_t rs[GV_RITER][P], rbi[GV_RITER][P];
        float ws[GV_RITER][P], wb[GV_RITER][P];
#pragma unroll
        for (int it = 0; it < GV_RITER; it++) {
            const int rr = r0 + it * RPW + rsub;
            const int r = rr < a.N ? rr : 0;
#pragma unroll
            for (int ps = 0; ps < P; ps++) {
                const int c0 = ps * LPR + sub;
                const int c = c0 < CH ? c0 : 0;
                wq[it][ps] = qk_ld((const uint4 *)(q + (size_t)r * wrow) + c);
                rs[it][ps] = qk_ld(sc + (size_t)r * G + (c >> a.gsh));
                rbi[it][ps] = qk_ld(bi + (size_t)r * G + (c >> a.gsh));
            }
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int it = 0; it < GV_RITER; it++) {
            const bool rok = r0 + it * RPW + rsub < a.N;
#pragma unroll
            for (int ps = 0; ps < P; ps++) {
                const bool ok = rok && ps * LPR + sub < CH;
                ws[it][ps] = ok ? qk_bf16(rs[it][ps]) : 0.0f;
                wb[it][ps] = ok ? qk_bf16(rbi[it][ps]) : 0.0f;
                if (!ok) wq[it][ps] = make_uint4(0u, 0u, 0u, 0u);
            }
        }
        for (int j = 0; j < m; j++) {
            const int p = p0 + j;
            XPairs<LPR, P, false> xp;
            if (SHARE) {
                convert_xshare<LPR, NG>(xq, a.K, sub, rsub, s_x + wave * LPR * 36,
                                        (XPairs<LPR, 1, false> &)xp);
                if (j + 1 < m) load_xshare<NG>(a.h, (size_t)(p + 1), a.K, sub, rsub, xq);
            } else {
                convert_xraw<LPR, P, false>(xr, a.K, sub, xp);
                if (j + 1 < m) load_xraw<LPR, P, false>(a.h, (size_t)(p + 1), a.K, sub, xr);
            }
#pragma unroll
            for (int it = 0; it < GV_RITER; it++) {
                const float v = qk_group_sum<LPR>(row_part<LPR, P, false>(wq[it], ws[it], wb[it], xp));
                if (sub == 0) s_y[p * RB + it * RPW + rsub] = v;
            }
        }
    }
    __syncthreads();

    /* combine */
    for (int i = threadIdx.x; i < a.n * RB; i += 64 * DC_WAVES) {
        const int t = i / RB, rl = i - t * RB, r = r0 + rl;
        if (r >= a.N) continue;
        float acc = 0.0f;
        for (int s2 = 0; s2 < a.k; s2++) {
            const int p = s_p[t * a.k + s2];
            if (p < nk) acc = fmaf(s_w[t * a.k + s2], s_y[p * RB + rl], acc);
        }
        acc = fmaf(qk_ld(a.sg + t), s_y[(nk + t) * RB + rl], acc);
        if (a.xres) {
            const float xv = a.xbf16 ? qk_bf16(((const uint16_t *)a.xres)[(size_t)t * a.N + r])
                                     : ((const float *)a.xres)[(size_t)t * a.N + r];
            acc = xv + acc;
        }
        if (a.out) a.out[(size_t)t * a.N + r] = acc;
        if (a.hyper)
            for (int j = 0; j < a.hc; j++) {
                float *hp = a.hyper + ((size_t)t * a.hc + j) * a.N + r;
                *hp = fmaf(qk_ld(a.inject + (size_t)t * a.hc + j), acc, *hp);
            }
    }
}

static int pick_lpr(int K);

/* one token, layer path: gate/up with the top-k fused in (H/32 a power of
 * two >= 64, i.e. 64 lanes per weight row); returns -1 when the shape is
 * not covered */
template <bool XBF16, int PL>
static int launch_gateup_topk_pl(const DecArgs &a, int cpl, dim3 grid, const DecRouteOut &ro,
                                 hipStream_t st) {
    if (cpl == 1) hipLaunchKernelGGL((k_gateup_dec<64, 1, 2, XBF16, PL>), grid, dim3(256), 0, st, a, nullptr, ro);
    else if (cpl == 2) hipLaunchKernelGGL((k_gateup_dec<64, 2, 2, XBF16, PL>), grid, dim3(256), 0, st, a, nullptr, ro);
    else hipLaunchKernelGGL((k_gateup_dec<64, 4, 2, XBF16, PL>), grid, dim3(256), 0, st, a, nullptr, ro);
    return QK_CHECK_LAUNCH();
}

extern "C" int qk_gateup_topk_supported(qk_shape s) {
    const int ch = s.H / 32;
    return ch >= 64 && ch <= 256 && (ch & (ch - 1)) == 0 && s.E <= 64 * 16 && s.k <= QK_MAX_TOPK &&
           !s.g32;
}

extern "C" int qk_launch_gateup_topk(const qmoe_layer_weights *W, qk_shape s, const void *x,
                                     int x_bf16, const float *logits, int32_t *idx, float *w,
                                     float *sg, int32_t *perm, int32_t *pos, int32_t *segtab,
                                     float *h, void *stream) {
    if (!qk_gateup_topk_supported(s)) return (int)hipErrorInvalidValue;
    DecArgs a;
    a.q[0] = W->gate_q; a.s[0] = W->gate_s; a.b[0] = W->gate_b;
    a.q[1] = W->up_q;   a.s[1] = W->up_s;   a.b[1] = W->up_b;
    a.sq[0] = W->sh_gate_q; a.ss[0] = W->sh_gate_s; a.sb[0] = W->sh_gate_b;
    a.sq[1] = W->sh_up_q;   a.ss[1] = W->sh_up_s;   a.sb[1] = W->sh_up_b;
    a.x = x;
    a.out = h;
    a.K = s.H;
    a.N = s.I;
    a.k = s.k;
    a.E = s.E;
    const DecRouteOut ro{logits, idx, w, sg, perm, pos, segtab};
    const int cpl = s.H / 32 / 64;
    const int rb = 4 * 1 * 2;
    const dim3 grid((s.k + 1) * ((s.I + rb - 1) / rb));
    hipStream_t st = (hipStream_t)stream;
    int pl = 1;
    while (pl * 64 < s.E) pl <<= 1;
#define GT_PL(P) return x_bf16 ? launch_gateup_topk_pl<true, P>(a, cpl, grid, ro, st) \
                               : launch_gateup_topk_pl<false, P>(a, cpl, grid, ro, st)
    switch (pl) {
    case 1: GT_PL(1);
    case 2: GT_PL(2);
    case 4: GT_PL(4);
    case 8: GT_PL(8);
    default: GT_PL(16);
    }
#undef GT_PL
}

/* LDS bytes of k_down_combine for n tokens, or 0 when the fused path does
 * not apply (too many tokens for one workgroup's LDS) */
extern "C" size_t qk_down_combine_lds(qk_shape s, int n) {
    if (n <= 0 || n > QK_DC_MAX_N) return 0;
    const int lpr = pick_lpr(s.I);
    const int rb = (64 / lpr) * GV_RITER;
    const int P = (s.I / 32 + lpr - 1) / lpr;
    const bool share = P == 1 && (lpr == 32 || lpr == 16); /* the kernel's SHARE */
    const size_t nk = (size_t)n * s.k;
    const size_t words = (((nk + n) * rb + 2 * nk + 3) & ~(size_t)3) + (share ? DC_WAVES * lpr * 36 : 0);
    const size_t bytes = words * 4;
    return bytes <= QK_DC_MAX_LDS ? bytes : 0;
}

extern "C" int qk_launch_down_combine(const qmoe_layer_weights *W, qk_shape s, const float *h,
                                      int n, const int32_t *segtab, const int32_t *pos,
                                      const float *w, const float *sg, const void *x_res,
                                      int x_bf16, float *out, float *hyper, const float *inject,
                                      int hc, void *stream) {
    const size_t lds = qk_down_combine_lds(s, n);
    if (lds == 0) return (int)hipErrorInvalidValue;
    DcArgs a;
    a.q = W->down_q; a.s = W->down_s; a.b = W->down_b;
    a.sq = W->sh_down_q; a.ss = W->sh_down_s; a.sb = W->sh_down_b;
    a.h = h;
    a.segtab = segtab;
    a.pos = pos;
    a.w = w;
    a.sg = sg;
    a.xres = x_res;
    a.xbf16 = x_bf16;
    a.out = out;
    a.hyper = hyper;
    a.inject = inject;
    a.hc = hc;
    a.gsh = s.g32 ? 0 : 1;
    a.K = s.I;
    a.N = s.H;
    a.n = n;
    a.k = s.k;
    a.E = s.E;
    const int lpr = pick_lpr(s.I);
    const int ch = s.I / 32;
    const int P = (ch + lpr - 1) / lpr;
    const int rb = (64 / lpr) * GV_RITER;
    const dim3 grid((s.H + rb - 1) / rb);
    hipStream_t st = (hipStream_t)stream;
#define DC_LAUNCH(L, PP) \
    hipLaunchKernelGGL((k_down_combine<L, PP>), grid, dim3(64 * DC_WAVES), lds, st, a, a.segtab)
    if (lpr == 64) {
        if (P == 1) DC_LAUNCH(64, 1);
        else if (P == 2) DC_LAUNCH(64, 2);
        else if (P <= 4) DC_LAUNCH(64, 4);
        else return (int)hipErrorInvalidValue;
    } else if (lpr == 32) DC_LAUNCH(32, 1);
    else if (lpr == 16) DC_LAUNCH(16, 1);
    else if (lpr == 8) DC_LAUNCH(8, 1);
    else if (lpr == 4) DC_LAUNCH(4, 1);
    else DC_LAUNCH(2, 1);
#undef DC_LAUNCH
    return QK_CHECK_LAUNCH();
}

static int pick_lpr(int K) {
    int ch = K / 32;
    int l = 2;
    while (l < ch && l < 64) l <<= 1;
    return l;
}

/* one token: the straight-line decode kernel when K/32 is a power of two
 * (<= 256 chunks); returns -1 when it does not apply */
template <bool XBF16>
static int launch_gateup_dec(const GemvArgs &g, hipStream_t st) {
    const int ch = g.K / 32;
    if (ch < 2 || ch > 256 || (ch & (ch - 1)) != 0 || g.gsh != 1) return -1; /* groups of 64 only */
    DecArgs a;
    for (int mt = 0; mt < 2; mt++) {
        a.q[mt] = g.q[mt]; a.s[mt] = g.s[mt]; a.b[mt] = g.b[mt];
        a.sq[mt] = g.sq[mt]; a.ss[mt] = g.ss[mt]; a.sb[mt] = g.sb[mt];
    }
    a.x = g.x;
    a.out = g.out;
    a.K = g.K;
    a.N = g.N;
    a.k = g.k;
    a.E = g.E;
    const int lpr = ch < 64 ? ch : 64, cpl = ch / lpr;
    const int rb = 4 * (64 / lpr) * 2;
    const dim3 grid((g.k + 1) * ((g.N + rb - 1) / rb));
    const DecRouteOut none{};
#define GD_LAUNCH(L, C) \
    hipLaunchKernelGGL((k_gateup_dec<L, C, 2, XBF16>), grid, dim3(256), 0, st, a, g.segtab, none)
    if (lpr == 64) {
        if (cpl == 1) GD_LAUNCH(64, 1);
        else if (cpl == 2) GD_LAUNCH(64, 2);
        else GD_LAUNCH(64, 4);
    } else if (lpr == 32) GD_LAUNCH(32, 1);
    else if (lpr == 16) GD_LAUNCH(16, 1);
    else if (lpr == 8) GD_LAUNCH(8, 1);
    else if (lpr == 4) GD_LAUNCH(4, 1);
    else GD_LAUNCH(2, 1);
#undef GD_LAUNCH
    return QK_CHECK_LAUNCH();
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
                                const int32_t *seglist, float *h, void *stream) {
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
    a.seglist = seglist;
    a.in_by_pos = 0;
    a.gsh = s.g32 ? 0 : 1;
    const int max_seg = n * s.k < s.E ? n * s.k : s.E;
    hipStream_t st = (hipStream_t)stream;
    if (n == 1) {
        const int rc = x_bf16 ? launch_gateup_dec<true>(a, st) : launch_gateup_dec<false>(a, st);
        if (rc >= 0) return rc;
    }
    return x_bf16 ? launch_gemv<2, true>(a, max_seg, st) : launch_gemv<2, false>(a, max_seg, st);
}

extern "C" int qk_launch_down(const qmoe_layer_weights *W, qk_shape s, const float *h, int n,
                              const int32_t *segtab, int max_m, const int32_t *seglist, float *y,
                              void *stream) {
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
    a.seglist = seglist;
    a.in_by_pos = 1;
    a.gsh = s.g32 ? 0 : 1;
    const int max_seg = n * s.k < s.E ? n * s.k : s.E;
    return launch_gemv<1, false>(a, max_seg, (hipStream_t)stream);
}
