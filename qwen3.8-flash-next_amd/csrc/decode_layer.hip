/*
 * decode_layer.hip -- the MoE layer for one token in two launches (gfx950),
 * replacing model.c:1301-1403 of the reference C port for n = 1 (router,
 * top-k + renormalise, dispatch, routed and shared SwiGLU experts, weighted
 * combine).
 *
 * Launch 1, k_dec_front (256 threads per workgroup): workgroups [0, NR)
 * compute the router logits, one wave per row (the E experts, then the
 * shared-expert gate) in the R64 order of router_rows.h; workgroups
 * [NR, NR + NS) compute the shared expert's gate/up GEMV for 8 rows each
 * (h row k), RMS-normalising x themselves when the layer has a norm.
 * Nothing in this launch depends on the routing.
 *
 * Launch 2, k_dec_experts (1024 threads per workgroup):
 *   workgroups [0, ND): down + combine for RBD output rows each.  Wave 0
 *     selects the top k from the logits and ranks the experts (their
 *     dispatch positions); every wave then issues the loads of its
 *     down-projection rows of every segment, and only then waits for h:
 *     each thread takes its own 8 h values from this workgroup's replica,
 *     converts them to bf16 hi/lo pairs in LDS and puts the sentinel back.
 *   workgroups [ND, ND + k*NG): the routed slots' gate/up GEMV, 32 rows
 *     each, with k_gateup_dec's arithmetic and in-kernel top-k; each pair
 *     of h rows a wave computes is written into every down workgroup's
 *     replica.
 *
 * The h hand-off uses no fence and no read-modify-write atomic.  Each down
 * workgroup owns a replica [k, I] of the routed h rows (dispatch order)
 * whose words all hold QK_DEC_SENT between launches (set when the context
 * is created).  A gate/up wave writes each row pair with one 64-bit relaxed
 * agent-scope atomic store per replica; a down thread reads its words with
 * 64-bit relaxed agent-scope atomic loads until none holds the sentinel,
 * then stores the sentinel back.  Only per-location coherence is relied on:
 * a word read is either the sentinel or this launch's value, because the
 * previous launch's value was reset by its only reader and the kernel
 * boundary orders that reset before this launch's writes.  A value whose
 * bits equal the sentinel (one NaN pattern) is written as the canonical
 * quiet NaN.  The wait is bounded by time (QK_DEC_WAIT_TICKS of the 100 MHz
 * s_memrealtime clock): on expiry the thread sets QK_DEC_ERR_WAIT in the
 * status word and goes on; while the status word is non-zero the down
 * workgroups write NaN and wait for nothing, until the host clears it
 * (qmoe_decode_status).
 *
 * Deadlock freedom: only down workgroups wait, and only for gate/up
 * workgroups, which wait for nothing.  The down workgroups come first in
 * the grid and occupy at most ND (< the number of compute units) units, so
 * every gate/up workgroup can be placed whatever the order of placement.
 *
 * Arithmetic: every value is computed as in the three-launch path
 * (k_router, k_gateup_dec<.., TK>, k_down_combine), so outputs and routing
 * are bit-identical to it.
 */
#include "qk_device.h"
#include "gemv_decode.h"
#include "gemv_parts.h"
#include "router_rows.h"
#include "topk_wave.h"

#define DEC_WG 1024        /* threads per workgroup of the experts launch */
#define DEC_WAVES (DEC_WG / 64)
#define DEC_RB_G 32        /* gate/up rows per workgroup: 16 waves x 2 rows */
#define DEC_NPASS 8        /* down items per wave, at most */
#define DEC_FRONT_RB 8     /* shared gate/up rows per front workgroup */

__device__ __forceinline__ uint64_t dec_ald(const uint64_t *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void dec_ast(uint64_t *p, uint64_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t dec_ald32(const uint32_t *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
/* bits of a value for the replica: never the sentinel */
__device__ __forceinline__ uint32_t dec_bits(float v) {
    const uint32_t b = __float_as_uint(v);
    return b == QK_DEC_SENT ? 0x7FC00000u : b;
}

/* ------------------------------------------------------------ launch 1 */

struct DecFrontArgs {
    RouterArgs ra;             /* router rows (n = 1) */
    const uint32_t *sq[2];     /* shared gate, up [I, H/8] */
    const uint16_t *ss[2], *sb[2];
    float *h;                  /* [k+1, I]: row k = shared */
    int NR, k, I;
};

/*
 * r = 1/sqrt(mean(x^2) + eps) of the token row, in the R64 order of
 * router_rows (lane l owns the 8-element chunks l, l+64, ...; an fma chain
 * per lane, then the wave tree), so the value is the router's bit for bit.
 */
template <bool XBF16, int NCH>
__device__ __forceinline__ float dec_rms_r(const void *x, int H, float eps, int lane) {
    const int chunks = H >> 3;
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < NCH; i++) {
        const int c = lane + 64 * i;
        const bool cv = c < chunks;
        float v[8];
        load_x8<XBF16>(x, 0, cv ? c : 0, v);
        float s2 = ss;
#pragma unroll
        for (int j = 0; j < 8; j++) s2 = fmaf(v[j], v[j], s2);
        ss = cv ? s2 : ss;
    }
    ss = qk_group_sum<64>(ss);
    return 1.0f / sqrtf(ss / (float)H + eps);
}

/*
 * The activation pairs of one lane's CPL chunks (32 columns each, chunk
 * c0 + c) as k_gateup_dec forms them: bf16 x directly, or f32 values
 * (x itself, or x normalised here as (x*r)*w exactly as router_rows does)
 * split into hi and lo pairs with their chunk sums.
 */
template <int CPL, bool XBF16, bool NORM, int NCH>
__device__ __forceinline__ void dec_act_pairs(const void *x, const float *norm_w, int H, float eps,
                                              int lane, int c0, uint32_t (&hp)[CPL][16],
                                              uint32_t (&lp)[(XBF16 && !NORM) ? 1 : CPL][16],
                                              float (&xs)[CPL]) {
    constexpr bool PB = XBF16 && !NORM; /* bf16 pairs straight from x */
    float r = 1.0f;
    if (NORM) r = dec_rms_r<XBF16, NCH>(x, H, eps, lane);
#pragma unroll
    for (int c = 0; c < CPL; c++) {
        if (PB) {
            const uint4 *src = (const uint4 *)((const uint16_t *)x) + 4 * (c0 + c);
            float s = 0.0f;
#pragma unroll
            for (int w = 0; w < 4; w++) {
                qk_bf16x8_to_pairs(qk_ld(src + w), &hp[c][4 * w]);
            }
#pragma unroll
            for (int i = 0; i < 16; i++) s = qk_dot2(hp[c][i], QK_BF16_ONES, s);
            xs[c] = s;
        } else {
            xs[c] = 0.0f;
#pragma unroll
            for (int w = 0; w < 4; w++) {
                /* columns 32*(c0+c) + 8*w .. +7 */
                const int e0 = 32 * (c0 + c) + 8 * w;
                float v[8];
                load_x8<XBF16>(x, 0, e0 >> 3, v);
                if (NORM) {
                    const float4 *nw = (const float4 *)(norm_w + e0);
                    const float4 w0 = qk_ld(nw), w1 = qk_ld(nw + 1);
                    const float wn[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
                    for (int j = 0; j < 8; j++) v[j] = (v[j] * r) * wn[j];
                }
                qk_f32x8_to_pairs(v, &hp[c][4 * w], &lp[PB ? 0 : c][4 * w], xs[c]);
            }
        }
    }
}

/* one lane's share of a gate or up row: k_gateup_dec's inner loop */
template <int CPL, bool PB>
__device__ __forceinline__ float dec_row_part(const uint4 (&wq)[CPL], const float *ws, const float *wb,
                                              const uint32_t (&hp)[CPL][16],
                                              const uint32_t (&lp)[PB ? 1 : CPL][16],
                                              const float (&xs)[CPL]) {
    float part = 0.0f;
#pragma unroll
    for (int c = 0; c < CPL; c++) {
        const int gl = CPL >= 2 ? c >> 1 : 0;
        const float s = ws[gl];
        const float bp = fmaf(-128.0f, s, wb[gl]);
        const uint32_t words[4] = {wq[c].x, wq[c].y, wq[c].z, wq[c].w};
        float d = 0.0f;
#pragma unroll
        for (int w = 0; w < 4; w++) {
            uint32_t pr[4];
            qk_codes_to_pairs(words[w], pr);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                d = qk_dot2(hp[c][4 * w + i], pr[i], d);
                if (!PB) d = qk_dot2(lp[PB ? 0 : c][4 * w + i], pr[i], d);
            }
        }
        part = fmaf(s, d, fmaf(bp, xs[c], part));
    }
    return part;
}

template <bool XBF16, bool NORM, int NCH, int CPL>
__global__ __launch_bounds__(256) void k_dec_front(DecFrontArgs a) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if ((int)blockIdx.x < a.NR) {
        const int row = blockIdx.x * 4 + wave;
        if (row <= a.ra.E) router_rows<XBF16, NORM, NCH>(a.ra, row, 0, 1);
        return;
    }
    /* shared expert gate/up: rows j*8 + wave*2 + it (64 lanes per row,
     * lane `lane` owns chunks lane*CPL .. lane*CPL+CPL-1) */
    constexpr bool PB = XBF16 && !NORM;
    constexpr int GPL = CPL >= 2 ? CPL / 2 : 1;
    const int H = a.ra.H;
    const int G = H >> 6;
    const size_t wrow = (size_t)H >> 3;
    const int c0 = lane * CPL, g0 = c0 >> 1;
    const int rbase = (blockIdx.x - a.NR) * DEC_FRONT_RB + wave * 2;
    uint4 wq[2][2][CPL];
    float ws[2][2][GPL], wb[2][2][GPL];
#pragma unroll
    for (int it = 0; it < 2; it++) {
        const int r0 = rbase + it;
        const int r = r0 < a.I ? r0 : 0;
#pragma unroll
        for (int mt = 0; mt < 2; mt++) {
            const uint4 *src = (const uint4 *)(a.sq[mt] + (size_t)r * wrow) + c0;
#pragma unroll
            for (int c = 0; c < CPL; c++) wq[it][mt][c] = qk_ld(src + c);
            dec_ld_bf16<GPL>(a.ss[mt] + (size_t)r * G + g0, ws[it][mt]);
            dec_ld_bf16<GPL>(a.sb[mt] + (size_t)r * G + g0, wb[it][mt]);
        }
    }
    uint32_t hp[CPL][16], lp[PB ? 1 : CPL][16];
    float xs[CPL];
    dec_act_pairs<CPL, XBF16, NORM, NCH>(a.ra.x, a.ra.norm_w, H, a.ra.eps, lane, c0, hp, lp, xs);
#pragma unroll
    for (int it = 0; it < 2; it++) {
        float acc[2];
#pragma unroll
        for (int mt = 0; mt < 2; mt++)
            acc[mt] = qk_group_sum<64>(dec_row_part<CPL, PB>(wq[it][mt], ws[it][mt], wb[it][mt], hp, lp, xs));
        const int r = rbase + it;
        if (lane == 0 && r < a.I) qk_st(a.h + (size_t)a.k * a.I + r, qk_silu(acc[0]) * acc[1]);
    }
}

/* ------------------------------------------------------------ launch 2 */

struct DecExpertsArgs {
    const uint32_t *q[2];      /* routed gate, up [E, I, H/8] */
    const uint16_t *s[2], *b[2];
    const uint32_t *dq;        /* routed down [E, H, I/8] */
    const uint16_t *ds, *db;
    const uint32_t *sdq;       /* shared down [H, I/8] */
    const uint16_t *sds, *sdb;
    const void *act;           /* gate/up input: x (bf16 or f32) or the normalised row (f32) */
    const void *xres;          /* residual input (x) or NULL */
    int xres_bf16;
    const float *logits;       /* [E+1] */
    float *h;                  /* [k+1, I] */
    uint64_t *rep;             /* [ND, k, I/2] row pairs */
    uint32_t *status;
    int32_t *idx;              /* routing outputs (one workgroup writes them) */
    float *w, *sg;
    int32_t *perm, *pos, *segtab;
    float *out;                /* [H] or NULL */
    float *hyper;              /* [hc, H] or NULL */
    const float *inject;       /* [hc] */
    int hc;
    int H, E, k, I, ND, RBD, NG;
};

/* routed gate/up: 32 rows (16 waves x 2) of slot `slot`'s expert */
template <int CPL, bool PB, int PL>
__device__ __forceinline__ void dec_gateup_routed(const DecExpertsArgs &a, int slot, int rb, int *s_ep) {
    constexpr int GPL = CPL >= 2 ? CPL / 2 : 1;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int H = a.H, G = H >> 6;
    const size_t wrow = (size_t)H >> 3;
    const int c0 = lane * CPL, g0 = c0 >> 1;

    /* activations: no routing dependence, issued first */
    uint4 xd[PB ? CPL : 1][4];
    float4 xf[PB ? 1 : CPL][8];
#pragma unroll
    for (int c = 0; c < CPL; c++) {
        if (PB) {
            const uint4 *src = (const uint4 *)((const uint16_t *)a.act) + 4 * (c0 + c);
#pragma unroll
            for (int w = 0; w < 4; w++) xd[PB ? c : 0][w] = qk_ld(src + w);
        } else {
            const float4 *src = (const float4 *)((const float *)a.act) + 8 * (c0 + c);
#pragma unroll
            for (int w = 0; w < 8; w++) xf[PB ? 0 : c][w] = qk_ld(src + w);
        }
    }

    WaveTopk<PL> tks;
    uint32_t my_key = 0u;
    int my_id = 0x7FFFFFFF;
    if (wave == 0) {
        tks.init(a.logits, a.E, lane);
        int es = 0;
        for (int r = 0; r <= slot; r++) {
            uint32_t m;
            int ei;
            tks.next(lane, m, ei);
            if (lane == r) {
                my_key = m;
                my_id = ei;
            }
            es = ei;
        }
        if (lane == 0) s_ep[0] = es;
    }
    __syncthreads();
    const int e = s_ep[0];
    const int rbase = rb * DEC_RB_G + wave * 2;
    uint4 wq[2][2][CPL];
    float ws[2][2][GPL], wb[2][2][GPL];
#pragma unroll
    for (int it = 0; it < 2; it++) {
        const int r0 = rbase + it;
        const int r = r0 < a.I ? r0 : 0;
#pragma unroll
        for (int mt = 0; mt < 2; mt++) {
            const uint4 *src = (const uint4 *)(a.q[mt] + ((size_t)e * a.I + r) * wrow) + c0;
#pragma unroll
            for (int c = 0; c < CPL; c++) wq[it][mt][c] = qk_ld(src + c);
            dec_ld_bf16<GPL>(a.s[mt] + ((size_t)e * a.I + r) * G + g0, ws[it][mt]);
            dec_ld_bf16<GPL>(a.b[mt] + ((size_t)e * a.I + r) * G + g0, wb[it][mt]);
        }
    }
    __builtin_amdgcn_sched_barrier(0);

    /* under the loads: the remaining rounds, then this slot's rank */
    if (wave == 0) {
        for (int r = slot + 1; r < a.k; r++) {
            uint32_t m;
            int ei;
            tks.next(lane, m, ei);
            if (lane == r) {
                my_key = m;
                my_id = ei;
            }
        }
        const int rank = (int)__popcll(__ballot(my_id < e));
        if (lane == 0) s_ep[1] = rank;
        if (slot == 0 && rb == 0) {
            const float wt = topk_weight(my_key, a.k, lane);
            int rk = 0;
            for (int s2 = 0; s2 < a.k; s2++) rk += __builtin_amdgcn_readlane(my_id, s2) < my_id ? 1 : 0;
            if (lane < a.k) {
                a.idx[lane] = my_id;
                a.w[lane] = wt;
                a.perm[rk] = lane;
                a.pos[lane] = rk;
                a.segtab[1 + 3 * rk] = my_id;
                a.segtab[2 + 3 * rk] = rk;
                a.segtab[3 + 3 * rk] = 1;
            }
            if (lane == 0) {
                a.segtab[0] = a.k;
                a.sg[0] = qk_sigmoid(qk_ld(a.logits + a.E));
            }
        }
    }

    /* activation pairs (x_i, x_{i+4}) per 8 columns, and chunk sums */
    uint32_t hp[CPL][16], lp[PB ? 1 : CPL][16];
    float xs[CPL];
#pragma unroll
    for (int c = 0; c < CPL; c++) {
        if (PB) {
#pragma unroll
            for (int w = 0; w < 4; w++) qk_bf16x8_to_pairs(xd[PB ? c : 0][w], &hp[c][4 * w]);
            float s = 0.0f;
#pragma unroll
            for (int i = 0; i < 16; i++) s = qk_dot2(hp[c][i], QK_BF16_ONES, s);
            xs[c] = s;
        } else {
            xs[c] = 0.0f;
#pragma unroll
            for (int w = 0; w < 4; w++) {
                const float4 a0 = xf[PB ? 0 : c][2 * w], a1 = xf[PB ? 0 : c][2 * w + 1];
                const float v[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
                qk_f32x8_to_pairs(v, &hp[c][4 * w], &lp[PB ? 0 : c][4 * w], xs[c]);
            }
        }
    }
    float hv[2];
#pragma unroll
    for (int it = 0; it < 2; it++) {
        float acc[2];
#pragma unroll
        for (int mt = 0; mt < 2; mt++)
            acc[mt] = qk_group_sum<64>(dec_row_part<CPL, PB>(wq[it][mt], ws[it][mt], wb[it][mt], hp, lp, xs));
        hv[it] = qk_silu(acc[0]) * acc[1];
    }
    __syncthreads(); /* s_ep[1] */
    const int p0 = s_ep[1];
    if (rbase < a.I) {
        const uint64_t pair = (uint64_t)dec_bits(hv[0]) | ((uint64_t)dec_bits(hv[1]) << 32);
        const size_t col = (size_t)p0 * (a.I >> 1) + (rbase >> 1);
        for (int d = lane; d < a.ND; d += 64) dec_ast(a.rep + (size_t)d * a.k * (a.I >> 1) + col, pair);
        if (lane == 0) {
            qk_st(a.h + (size_t)p0 * a.I + rbase, hv[0]);
            qk_st(a.h + (size_t)p0 * a.I + rbase + 1, hv[1]);
        }
    }
}

/*
 * down + combine for output rows r0 .. r0+RBD-1.  Items are (segment,
 * group of RPW rows); segment p < k is dispatch position p (the routed
 * expert of rank p), segment k the shared expert.  The arithmetic per
 * (segment, row) and the combine are k_down_combine's.
 */
template <int LPRD, int PL>
__device__ __forceinline__ void dec_down_combine(const DecExpertsArgs &a, float *lds) {
    constexpr int RPW = 64 / LPRD;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int sub = lane % LPRD, rsub = lane / LPRD;
    const int k = a.k, I = a.I, H = a.H;
    const int CH = I >> 5, GI = I >> 6;
    const size_t wrow = (size_t)I >> 3;
    const int RBD = a.RBD;
    const int r0 = blockIdx.x * RBD;
    const int gps = RBD / RPW; /* row groups per segment */
    const int items = (k + 1) * gps;

    float *s_x = lds;                                  /* [(k+1) * CH * 36] pairs, sums */
    float *s_y = s_x + (size_t)(k + 1) * CH * 36;      /* [(k+1) * RBD] */
    float *s_pw = s_y + (size_t)(k + 1) * RBD;         /* [k] weight by position */
    int *s_pe = (int *)(s_pw + QK_MAX_TOPK);           /* [k] expert by position */
    int *s_misc = s_pe + QK_MAX_TOPK;                  /* [0] bad, [1] sigmoid bits */

    if (wave == 0) {
        const uint32_t st = dec_ald32(a.status);
        WaveTopk<PL> tks;
        tks.init(a.logits, a.E, lane);
        uint32_t my_key = 0u;
        int my_id = 0x7FFFFFFF;
        for (int r = 0; r < k; r++) {
            uint32_t m;
            int ei;
            tks.next(lane, m, ei);
            if (lane == r) {
                my_key = m;
                my_id = ei;
            }
        }
        const float wt = topk_weight(my_key, k, lane);
        int rk = 0;
        for (int s2 = 0; s2 < k; s2++) rk += __builtin_amdgcn_readlane(my_id, s2) < my_id ? 1 : 0;
        if (lane < k) {
            s_pe[rk] = my_id;
            s_pw[rk] = wt;
        }
        if (lane == 0) {
            s_misc[0] = st != 0u;
            s_misc[1] = __float_as_int(qk_sigmoid(qk_ld(a.logits + a.E)));
        }
    }
    __syncthreads();
    const bool bad = s_misc[0] != 0;

    /* the down rows of this wave's items (weights do not depend on h) */
    uint4 wq[DEC_NPASS][1];
    uint16_t rsv[DEC_NPASS], rbv[DEC_NPASS];
#pragma unroll
    for (int ps = 0; ps < DEC_NPASS; ps++) {
        const int item = ps * DEC_WAVES + wave;
        const int it = item < items ? item : 0;
        const int sgm = it / gps, g = it - sgm * gps;
        const int r = r0 + g * RPW + rsub;
        const uint32_t *q;
        const uint16_t *sc, *bi;
        if (sgm < k) {
            const int e = s_pe[sgm];
            q = a.dq + (size_t)e * H * wrow;
            sc = a.ds + (size_t)e * H * GI;
            bi = a.db + (size_t)e * H * GI;
        } else {
            q = a.sdq;
            sc = a.sds;
            bi = a.sdb;
        }
        wq[ps][0] = qk_ld((const uint4 *)(q + (size_t)r * wrow) + sub);
        rsv[ps] = qk_ld(sc + (size_t)r * GI + (sub >> 1));
        rbv[ps] = qk_ld(bi + (size_t)r * GI + (sub >> 1));
    }

    /* h: thread i takes 8 values (rows 8*q8 .. 8*q8+7 of segment sg8) */
    const int n8 = (k + 1) * (I >> 3);
    for (int i = threadIdx.x; i < n8; i += DEC_WG) {
        const int sg8 = i / (I >> 3), q8 = i - sg8 * (I >> 3);
        float v[8];
        if (sg8 < k) {
            uint64_t *src = a.rep + ((size_t)blockIdx.x * k + sg8) * (I >> 1) + 4 * q8;
            uint64_t u[4] = {0, 0, 0, 0};
            if (!bad) {
                uint64_t t0 = 0;
                while (true) {
#pragma unroll
                    for (int j = 0; j < 4; j++) u[j] = dec_ald(src + j);
                    bool ok = true;
#pragma unroll
                    for (int j = 0; j < 4; j++)
                        ok &= (uint32_t)u[j] != QK_DEC_SENT && (uint32_t)(u[j] >> 32) != QK_DEC_SENT;
                    if (ok) break;
                    const uint64_t now = __builtin_amdgcn_s_memrealtime();
                    if (t0 == 0) {
                        t0 = now;
                    } else if (now - t0 > QK_DEC_WAIT_TICKS) {
                        __hip_atomic_fetch_or(a.status, QK_DEC_ERR_WAIT, __ATOMIC_RELAXED,
                                              __HIP_MEMORY_SCOPE_AGENT);
                        break;
                    }
                    __builtin_amdgcn_s_sleep(1);
                }
#pragma unroll
                for (int j = 0; j < 4; j++) dec_ast(src + j, ((uint64_t)QK_DEC_SENT << 32) | QK_DEC_SENT);
            }
#pragma unroll
            for (int j = 0; j < 4; j++) {
                v[2 * j] = __uint_as_float((uint32_t)u[j]);
                v[2 * j + 1] = __uint_as_float((uint32_t)(u[j] >> 32));
            }
        } else {
            const float4 *src = (const float4 *)(a.h + (size_t)k * I + 8 * q8);
            const float4 f0 = qk_ld(src), f1 = qk_ld(src + 1);
            v[0] = f0.x; v[1] = f0.y; v[2] = f0.z; v[3] = f0.w;
            v[4] = f1.x; v[5] = f1.y; v[6] = f1.z; v[7] = f1.w;
        }
        uint32_t hi[4], lo[4];
        const float gs = qk_f32x8_pairs(v, hi, lo);
        uint32_t *cb = (uint32_t *)s_x + ((size_t)sg8 * CH + (q8 >> 2)) * 36;
        const int gi = q8 & 3;
        *(uint4 *)(cb + 4 * gi) = make_uint4(hi[0], hi[1], hi[2], hi[3]);
        *(uint4 *)(cb + 16 + 4 * gi) = make_uint4(lo[0], lo[1], lo[2], lo[3]);
        ((float *)cb)[32 + gi] = gs;
    }
    __syncthreads();

    /* y for every item */
#pragma unroll
    for (int ps = 0; ps < DEC_NPASS; ps++) {
        const int item = ps * DEC_WAVES + wave;
        if (item >= items) break;
        const int sgm = item / gps, g = item - sgm * gps;
        const uint32_t *cb = (const uint32_t *)s_x + ((size_t)sgm * CH + sub) * 36;
        XPairs<LPRD, 1, false> xp;
#pragma unroll
        for (int w = 0; w < 4; w++) {
            const uint4 hh = *(const uint4 *)(cb + 4 * w), ll = *(const uint4 *)(cb + 16 + 4 * w);
            xp.hi[0][4 * w] = hh.x;
            xp.hi[0][4 * w + 1] = hh.y;
            xp.hi[0][4 * w + 2] = hh.z;
            xp.hi[0][4 * w + 3] = hh.w;
            xp.lo[0][4 * w] = ll.x;
            xp.lo[0][4 * w + 1] = ll.y;
            xp.lo[0][4 * w + 2] = ll.z;
            xp.lo[0][4 * w + 3] = ll.w;
        }
        const float4 gsv = *(const float4 *)(cb + 32);
        xp.xs[0] = (((0.0f + gsv.x) + gsv.y) + gsv.z) + gsv.w;
        const float wsv[1] = {qk_bf16(rsv[ps])}, wbv[1] = {qk_bf16(rbv[ps])};
        const float v = qk_group_sum<LPRD>(row_part<LPRD, 1, false>(wq[ps], wsv, wbv, xp));
        if (sub == 0) s_y[sgm * RBD + g * RPW + rsub] = v;
    }
    __syncthreads();

    /* combine: out = sum over positions of w*y, then sigmoid * y_shared, + x */
    for (int t = threadIdx.x; t < RBD; t += DEC_WG) {
        const int r = r0 + t;
        float acc = 0.0f;
        for (int p = 0; p < k; p++) acc = fmaf(s_pw[p], s_y[p * RBD + t], acc);
        acc = fmaf(__int_as_float(s_misc[1]), s_y[k * RBD + t], acc);
        if (a.xres) {
            const float xv = a.xres_bf16 ? qk_bf16(((const uint16_t *)a.xres)[r])
                                         : ((const float *)a.xres)[r];
            acc = xv + acc;
        }
        if (bad) acc = __uint_as_float(0x7FC00000u);
        if (a.out) a.out[r] = acc;
        if (a.hyper)
            for (int j = 0; j < a.hc; j++) {
                float *hp = a.hyper + (size_t)j * H + r;
                *hp = fmaf(qk_ld(a.inject + j), acc, *hp);
            }
    }
}

template <int CPL, int LPRD, bool PB, int PL>
__global__ __launch_bounds__(DEC_WG) void k_dec_experts(DecExpertsArgs a) {
    extern __shared__ float dec_lds[];
    if ((int)blockIdx.x < a.ND) {
        dec_down_combine<LPRD, PL>(a, dec_lds);
        return;
    }
    const int gi = blockIdx.x - a.ND;
    const int slot = gi / a.NG, rb = gi - slot * a.NG;
    dec_gateup_routed<CPL, PB, PL>(a, slot, rb, (int *)dec_lds);
}

/* ------------------------------------------------------------ host side */

static int dec_pl(int E) {
    int pl = 2;
    while (pl * 64 < E) pl <<= 1;
    return pl;
}

/* rows per down workgroup: the largest power of two <= 32 dividing H with
 * every (segment, row group) item of a workgroup within DEC_NPASS passes;
 * 0 when none fits */
static int dec_rbd(qk_shape s) {
    const int rpw = 64 / (s.I / 32);
    for (int rbd = 32; rbd >= rpw; rbd >>= 1)
        if (s.H % rbd == 0 && (s.k + 1) * (rbd / rpw) <= DEC_NPASS * DEC_WAVES) return rbd;
    return 0;
}

extern "C" int qk_dec_supported(qk_shape s) {
    const int ch = s.H / 32;
    const int lprd = s.I / 32;
    if (!(ch == 64 || ch == 128)) return 0; /* gate/up: 64 lanes x 1 or 2 chunks */
    if (!(lprd == 16 || lprd == 32) || s.I % DEC_RB_G) return 0;
    if (s.E < s.k || s.E > 64 * 16 || s.k > 16) return 0;
    if ((size_t)(s.k + 1) * s.I / 8 > DEC_WG) return 0; /* one 8-group of h per thread */
    const int rbd = dec_rbd(s);
    if (!rbd || s.H / rbd > 256) return 0;
    return qk_dec_lds(s) <= 65536;
}

extern "C" size_t qk_dec_lds(qk_shape s) {
    const int rbd = dec_rbd(s);
    return ((size_t)(s.k + 1) * (s.I / 32) * 36 + (size_t)(s.k + 1) * rbd + 2 * QK_MAX_TOPK + 2) * 4;
}

extern "C" size_t qk_dec_replica_bytes(qk_shape s) {
    const int rbd = dec_rbd(s);
    return rbd ? (size_t)(s.H / rbd) * s.k * s.I * 4 : 0;
}

template <bool XBF16, bool NORM>
static void dec_front_launch(int cpl, dim3 grid, const DecFrontArgs &f, hipStream_t st) {
    if (cpl == 1) hipLaunchKernelGGL((k_dec_front<XBF16, NORM, 4, 1>), grid, dim3(256), 0, st, f);
    else hipLaunchKernelGGL((k_dec_front<XBF16, NORM, 8, 2>), grid, dim3(256), 0, st, f);
}

template <int CPL, int LPRD, bool PB>
static void dec_experts_launch(int pl, dim3 grid, size_t lds, const DecExpertsArgs &e, hipStream_t st) {
    switch (pl) {
    case 2: hipLaunchKernelGGL((k_dec_experts<CPL, LPRD, PB, 2>), grid, dim3(DEC_WG), lds, st, e); break;
    case 4: hipLaunchKernelGGL((k_dec_experts<CPL, LPRD, PB, 4>), grid, dim3(DEC_WG), lds, st, e); break;
    case 8: hipLaunchKernelGGL((k_dec_experts<CPL, LPRD, PB, 8>), grid, dim3(DEC_WG), lds, st, e); break;
    default: hipLaunchKernelGGL((k_dec_experts<CPL, LPRD, PB, 16>), grid, dim3(DEC_WG), lds, st, e); break;
    }
}

extern "C" int qk_launch_dec_layer(const qmoe_layer_weights *W, qk_shape s, const void *x, int x_bf16,
                                   float *logits, float *xn, float *h, uint32_t *rep, uint32_t *status,
                                   int32_t *idx, float *w, float *sg, int32_t *perm, int32_t *pos,
                                   int32_t *segtab, const void *x_res, float *out, float *hyper,
                                   const float *inject, int hc, void *stream) {
    if (!qk_dec_supported(s)) return (int)hipErrorInvalidValue;
    hipStream_t st = (hipStream_t)stream;
    const int cpl = s.H / 2048;
    const bool norm = W->norm_w != nullptr;

    DecFrontArgs f;
    f.ra.router_w = W->router_w;
    f.ra.router_bias = W->router_bias;
    f.ra.sh_gate_w = W->sh_gate_w;
    f.ra.norm_w = W->norm_w;
    f.ra.x = x;
    f.ra.logits = logits;
    f.ra.xn = norm ? xn : nullptr;
    f.ra.H = s.H;
    f.ra.E = s.E;
    f.ra.n = 1;
    f.ra.eps = s.eps;
    f.sq[0] = W->sh_gate_q; f.ss[0] = W->sh_gate_s; f.sb[0] = W->sh_gate_b;
    f.sq[1] = W->sh_up_q;   f.ss[1] = W->sh_up_s;   f.sb[1] = W->sh_up_b;
    f.h = h;
    f.NR = (s.E + 1 + 3) / 4;
    f.k = s.k;
    f.I = s.I;
    const dim3 fgrid(f.NR + s.I / DEC_FRONT_RB);
    if (x_bf16) {
        if (norm) dec_front_launch<true, true>(cpl, fgrid, f, st);
        else dec_front_launch<true, false>(cpl, fgrid, f, st);
    } else {
        if (norm) dec_front_launch<false, true>(cpl, fgrid, f, st);
        else dec_front_launch<false, false>(cpl, fgrid, f, st);
    }
    int rc = QK_CHECK_LAUNCH();
    if (rc) return rc;

    DecExpertsArgs e;
    e.q[0] = W->gate_q; e.s[0] = W->gate_s; e.b[0] = W->gate_b;
    e.q[1] = W->up_q;   e.s[1] = W->up_s;   e.b[1] = W->up_b;
    e.dq = W->down_q; e.ds = W->down_s; e.db = W->down_b;
    e.sdq = W->sh_down_q; e.sds = W->sh_down_s; e.sdb = W->sh_down_b;
    const bool pb = x_bf16 && !norm;
    e.act = norm ? (const void *)xn : x;
    e.xres = x_res;
    e.xres_bf16 = x_bf16;
    e.logits = logits;
    e.h = h;
    e.rep = (uint64_t *)rep;
    e.status = status;
    e.idx = idx; e.w = w; e.sg = sg; e.perm = perm; e.pos = pos; e.segtab = segtab;
    e.out = out;
    e.hyper = hyper;
    e.inject = inject;
    e.hc = hc;
    e.H = s.H; e.E = s.E; e.k = s.k; e.I = s.I;
    e.RBD = dec_rbd(s);
    e.ND = s.H / e.RBD;
    e.NG = s.I / DEC_RB_G;
    const dim3 egrid(e.ND + s.k * e.NG);
    const size_t lds = qk_dec_lds(s);
    const int pl = dec_pl(s.E);
    const int lprd = s.I / 32;
#define DEC_EX(C, L) \
    (pb ? dec_experts_launch<C, L, true>(pl, egrid, lds, e, st) : dec_experts_launch<C, L, false>(pl, egrid, lds, e, st))
    if (cpl == 1) {
        if (lprd == 16) DEC_EX(1, 16);
        else DEC_EX(1, 32);
    } else {
        if (lprd == 16) DEC_EX(2, 16);
        else DEC_EX(2, 32);
    }
#undef DEC_EX
    return QK_CHECK_LAUNCH();
}
