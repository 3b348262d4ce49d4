/*
 * decode_layer.hip -- the MoE layer for one token in one launch (gfx950),
 * replacing model.c:1301-1403 of the reference C port for n = 1 (router,
 * top-k + renormalise, dispatch, routed and shared SwiGLU experts, weighted
 * combine).
 *
 * k_dec_layer, 256 threads per workgroup, four roles by workgroup index:
 *   [0, NR)        router logits, DEC_RT_ROWS rows each (the E experts, then
 *                  the shared-expert gate), one wave per row in the R64
 *                  order of router_rows.h, the workgroup's logits going out
 *                  as one full 64-byte line;
 *   [NR, +NS)      the shared expert's gate/up GEMV, DEC_RB_G rows each;
 *   [.., +k*NG)    the routed slots' gate/up GEMV, DEC_RB_G rows of the
 *                  expert of slot s each: wave 0 waits for the logits and
 *                  runs the top-k rounds up to slot s, every wave loads its
 *                  rows, and the remaining rounds and the expert's dispatch
 *                  position run under the loads;
 *   [.., +ND)      down + combine for RBD output rows each: wave 0 waits
 *                  for the logits and ranks the k experts, every wave loads
 *                  its down rows of every segment, then the workgroup waits
 *                  for h.
 * Producers come first in the grid and wait for nothing placed after them.
 *
 * The hand-off uses no fence and no lock.  Every logit and h value goes out
 * as one 64-bit word (tag << 32 | f32 bits) by a relaxed agent-scope atomic
 * store, and a consumer reads the words with relaxed agent-scope atomic
 * loads until each carries this launch's tag; only per-location coherence
 * is relied on.  The tag is epoch + 1, with epoch = C / ND for a 64-bit
 * counter C that every down workgroup increments once, when it has taken
 * all of h, and that every workgroup reads as it starts.  C reaches the
 * next multiple of ND only when the last down workgroup has taken all of h,
 * and by then every workgroup has read C, since each has produced a word a
 * down workgroup consumed and that word's tag came from its read.  The next
 * launch reads C after the kernel boundary, so graph replays need nothing
 * from the host.
 *
 * Waits are bounded (QK_DEC_WAIT_TICKS of the 100 MHz s_memrealtime
 * clock): on expiry the thread sets QK_DEC_ERR_WAIT in the status word and
 * goes on; down workgroups that see the status set write NaN, and
 * qmoe_decode_status reports it, clears it and resets the hand-off state.
 *
 * Arithmetic: every value is computed as in the staged path (k_router,
 * k_gateup_dec, k_down_combine), so outputs and routing are bit-identical
 * to it.
 */
#include "qk_device.h"
#include "gemv_decode.h"
#include "gemv_parts.h"
#include "router_rows.h"
#include "topk_wave.h"

#define DEC_WG 256
#define DEC_WAVES (DEC_WG / 64)
#define DEC_GRW 4                       /* gate/up rows per wave */
#define DEC_RB_G (DEC_WAVES * DEC_GRW)  /* gate/up rows per workgroup */
#define DEC_NPASS 6                     /* down items per wave, at most */
#define DEC_CTL_BYTES 256               /* epoch, counter; then the tagged words */
#define DEC_RT_ROWS 8                   /* router rows per workgroup: a 64-byte line of words */

__device__ __forceinline__ uint64_t dec_ald(const uint64_t *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void dec_ast(uint64_t *p, uint64_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t dec_ald32(const uint32_t *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t dec_word(float v, uint32_t tag) {
    return ((uint64_t)tag << 32) | __float_as_uint(v);
}


/* a workgroup barrier that orders LDS only: loads and stores to global
 * memory stay in flight across it (__syncthreads would wait for them) */
__device__ __forceinline__ void dec_lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

__device__ __forceinline__ void dec_bump(uint64_t *c) {
    __hip_atomic_fetch_add(c, (uint64_t)1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

/* a bounded wait step: false once the bound has passed (status set) */
__device__ __forceinline__ bool dec_keep_waiting(uint64_t &t0, uint32_t *status) {
    const uint64_t now = __builtin_amdgcn_s_memrealtime();
    if (t0 == 0) {
        t0 = now;
    } else if (now - t0 > QK_DEC_WAIT_TICKS) {
        __hip_atomic_fetch_or(status, QK_DEC_ERR_WAIT, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return false;
    }
    __builtin_amdgcn_s_sleep(1);
    return true;
}

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

/* ------------------------------------------------------------ arguments */

struct DlArgs {
    RouterArgs ra;             /* router rows (n = 1) */
    uint64_t *lt;              /* [E+1] tagged logits */
    const uint32_t *q[2];      /* routed gate, up [E, I, H/8] */
    const uint16_t *s[2], *b[2];
    const uint32_t *sq[2];     /* shared gate, up [I, H/8] */
    const uint16_t *ss[2], *sb[2];
    const uint32_t *dq;        /* routed down [E, H, I/8] */
    const uint16_t *ds, *db;
    const uint32_t *sdq;       /* shared down [H, I/8] */
    const uint16_t *sds, *sdb;
    const void *xres;          /* residual input (x) or NULL */
    int xres_bf16;
    uint64_t *ctl;             /* [0] down workgroups past their wait for h, all launches */
    uint64_t *ht;              /* [(k+1)*I] tagged h: dispatch positions 0..k-1, then shared */
    uint32_t *status;
    float *h;                  /* [(k+1)*I] plain copy of h */
    int32_t *idx;              /* routing outputs (one workgroup writes them) */
    float *w, *sg;
    int32_t *perm, *pos, *segtab;
    float *out;                /* [H] or NULL */
    float *hyper;              /* [hc, H] or NULL */
    const float *inject;       /* [hc] */
    int hc;
    int H, E, k, I, NR, NS, NG, ND, RBD;
};

/*
 * Wave 0 of a consumer: this launch's logits, lane l getting row[l*PL + i]
 * in lv[i], and the shared-expert gate logit in lsh.  The tagged words are
 * read lane-contiguous (coalesced) and regrouped through s_lv.  False when
 * the wait expired (the values are then not this launch's).
 */
template <int PL>
__device__ __forceinline__ bool dec_take_logits(const DlArgs &a, uint32_t tag, float *s_lv,
                                                int lane, float (&lv)[PL], float &lsh) {
    const int n = a.E + 1; /* <= 64 * (PL + 1) */
    uint64_t t0 = 0;
    /* first one word per lane, spread over the router workgroups' lines
     * (every lane's line, and lane 0 the last line too): polling every word
     * slows the producers' own loads */
    {
        const int pw = min(lane * DEC_RT_ROWS, n - 1);
        while ((uint32_t)(dec_ald(a.lt + pw) >> 32) != tag ||
               (lane == 0 && (uint32_t)(dec_ald(a.lt + n - 1) >> 32) != tag))
            if (!dec_keep_waiting(t0, a.status)) break;
    }
    uint64_t u[PL + 1];
    bool all;
    do {
#pragma unroll
        for (int j = 0; j <= PL; j++) u[j] = dec_ald(a.lt + min(lane + 64 * j, n - 1));
        all = true;
#pragma unroll
        for (int j = 0; j <= PL; j++) all &= (uint32_t)(u[j] >> 32) == tag;
    } while (!all && dec_keep_waiting(t0, a.status));
#pragma unroll
    for (int j = 0; j <= PL; j++)
        if (lane + 64 * j < n) s_lv[lane + 64 * j] = __uint_as_float((uint32_t)u[j]);
    const bool ok = __all(all);
    qk_wave_lds_sync();
#pragma unroll
    for (int i = 0; i < PL; i++) lv[i] = s_lv[min(lane * PL + i, a.E - 1)];
    lsh = s_lv[a.E];
    return ok;
}

/* ------------------------------------------------------------ gate/up */

/* the workgroup's DEC_RB_G values of h (s_h) out as tagged words and as
 * plain floats, row r0 + t of segment p */
__device__ __forceinline__ void dec_put_h(const DlArgs &a, uint32_t tag, int p, int r0,
                                          const float *s_h) {
    const int t = threadIdx.x;
    if (t < DEC_RB_G && r0 + t < a.I) {
        const size_t i = (size_t)p * a.I + r0 + t;
        dec_ast(a.ht + i, dec_word(s_h[t], tag));
        a.h[i] = s_h[t];
    }
}

/* the shared expert's gate/up: rows j*DEC_RB_G + wave*DEC_GRW + it */
template <int CPL, bool XBF16, bool NORM, int NCH>
__device__ __forceinline__ void dec_gateup_shared(const DlArgs &a, uint32_t tag, int j, float *lds) {
    constexpr bool PB = XBF16 && !NORM;
    constexpr int GPL = CPL >= 2 ? CPL / 2 : 1;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int H = a.H, G = H >> 6;
    const size_t wrow = (size_t)H >> 3;
    const int c0 = lane * CPL, g0 = c0 >> 1;
    const int rbase = j * DEC_RB_G + wave * DEC_GRW;
    uint4 wq[DEC_GRW][2][CPL];
    float ws[DEC_GRW][2][GPL], wb[DEC_GRW][2][GPL];
#pragma unroll
    for (int it = 0; it < DEC_GRW; it++) {
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
    for (int it = 0; it < DEC_GRW; it++) {
        float acc[2];
#pragma unroll
        for (int mt = 0; mt < 2; mt++)
            acc[mt] = qk_group_sum<64>(dec_row_part<CPL, PB>(wq[it][mt], ws[it][mt], wb[it][mt], hp, lp, xs));
        if (lane == 0) lds[wave * DEC_GRW + it] = qk_silu(acc[0]) * acc[1];
    }
    dec_lds_barrier();
    dec_put_h(a, tag, a.k, j * DEC_RB_G, lds);
}

/* routed gate/up: DEC_RB_G rows (block rb) of the expert of slot `slot` */
template <int CPL, bool XBF16, bool NORM, int NCH, int PL>
__device__ __forceinline__ void dec_gateup_routed(const DlArgs &a, uint32_t tag, int slot, int rb,
                                                  float *lds) {
    constexpr bool PB = XBF16 && !NORM;
    constexpr int GPL = CPL >= 2 ? CPL / 2 : 1;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int H = a.H, G = H >> 6;
    const size_t wrow = (size_t)H >> 3;
    const int c0 = lane * CPL, g0 = c0 >> 1;
    float *s_h = lds;                               /* [DEC_RB_G] */
    int *s_i = (int *)(lds + DEC_RB_G);             /* [0] expert, [1] its dispatch position */
    float *s_lv = lds + DEC_RB_G + 4;               /* [64 * (PL + 1)] */

    /* the activation pairs do not depend on the routing: formed first */
    uint32_t hp[CPL][16], lp[PB ? 1 : CPL][16];
    float xs[CPL];
    dec_act_pairs<CPL, XBF16, NORM, NCH>(a.ra.x, a.ra.norm_w, H, a.ra.eps, lane, c0, hp, lp, xs);

    WaveTopk<PL> tks;
    uint32_t my_key = 0u;
    int my_id = 0x7FFFFFFF;
    float lsh = 0.0f;
    if (wave == 0) {
        float lv[PL];
        dec_take_logits<PL>(a, tag, s_lv, lane, lv, lsh);
        tks.init_vals(lv, a.E, lane);
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
        if (lane == 0) s_i[0] = min(max(es, 0), a.E - 1);
    }
    dec_lds_barrier();
    const int e = s_i[0];
    const int rbase = rb * DEC_RB_G + wave * DEC_GRW;
    uint4 wq[DEC_GRW][2][CPL];
    float ws[DEC_GRW][2][GPL], wb[DEC_GRW][2][GPL];
#pragma unroll
    for (int it = 0; it < DEC_GRW; it++) {
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

    /* under the loads: the remaining rounds, then this expert's position */
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
        if (lane == 0) s_i[1] = rank;
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
                a.sg[0] = qk_sigmoid(lsh);
            }
        }
    }
#pragma unroll
    for (int it = 0; it < DEC_GRW; it++) {
        float acc[2];
#pragma unroll
        for (int mt = 0; mt < 2; mt++)
            acc[mt] = qk_group_sum<64>(dec_row_part<CPL, PB>(wq[it][mt], ws[it][mt], wb[it][mt], hp, lp, xs));
        if (lane == 0) s_h[wave * DEC_GRW + it] = qk_silu(acc[0]) * acc[1];
    }
    dec_lds_barrier(); /* s_h, s_i[1] */
    dec_put_h(a, tag, s_i[1], rb * DEC_RB_G, s_h);
}

/* ------------------------------------------------------------ down */

#define DEC_HW 24 /* tagged h words per thread, at most: (k+1)*I <= DEC_WG * DEC_HW */
#define DEC_HPH 4 /* h is staged in this many parts */

/*
 * down + combine for output rows r0 .. r0+RBD-1.  Items are (segment,
 * group of RPW rows); segment p < k is dispatch position p (the routed
 * expert of rank p), segment k the shared expert.  The arithmetic per
 * (segment, row) and the combine are k_down_combine's.
 */
template <int LPRD, int PL>
__device__ __forceinline__ void dec_down_combine(const DlArgs &a, uint32_t tag, float *lds) {
    constexpr int RPW = 64 / LPRD;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int sub = lane % LPRD, rsub = lane / LPRD;
    const int k = a.k, I = a.I, H = a.H;
    const int CH = I >> 5, GI = I >> 6;
    const size_t wrow = (size_t)I >> 3;
    const int RBD = a.RBD;
    const int r0 = ((int)blockIdx.x - (a.NR + a.NS + a.k * a.NG)) * RBD;
    const int gps = RBD / RPW; /* row groups per segment */
    const int items = (k + 1) * gps;
    const int nw = (k + 1) * I, half = nw / DEC_HPH; /* words of one part */

    float *s_x = lds;                                  /* [(k+1) * CH * 36] pairs, sums */
    float *s_hv = s_x + (size_t)(k + 1) * CH * 36;     /* [half] h values of one part */
    float *s_y = s_hv + half;                          /* [(k+1) * RBD] */
    float *s_pw = s_y + (size_t)(k + 1) * RBD;         /* [k] weight by position */
    int *s_pe = (int *)(s_pw + QK_MAX_TOPK);           /* [k] expert by position */
    int *s_misc = s_pe + QK_MAX_TOPK;                  /* [0] bad, [1] sigmoid bits */
    float *s_lv = s_x;                                 /* logits, before s_x is used */

    if (wave == 0) {
        float lv[PL], lsh;
        const bool ok = dec_take_logits<PL>(a, tag, s_lv, lane, lv, lsh);
        /* outputs are NaN while the status is set or when a wait of this
         * workgroup expires */
        if (lane == 0) s_misc[0] = !ok || dec_ald32(a.status) != 0u;
        WaveTopk<PL> tks;
        tks.init_vals(lv, a.E, lane);
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
            s_pe[rk] = min(max(my_id, 0), a.E - 1);
            s_pw[rk] = wt;
        }
        if (lane == 0) s_misc[1] = __float_as_int(qk_sigmoid(lsh));
    }
    dec_lds_barrier();

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

    /* h in DEC_HPH parts: every thread reads words t + DEC_WG*j of a part
     * (coalesced; the next part's loads in flight under this part's work)
     * until each carries this launch's tag; the values go to s_hv and the
     * units of 8 become bf16 hi/lo pairs with group sums */
    const int u8 = I >> 3;
    constexpr int PW = DEC_HW / DEC_HPH;
    /* one word per thread first (spread over h: every producer's rows are
     * sampled), then every thread reads all of its words at once until each
     * carries this launch's tag */
    bool expired = false;
    {
        uint64_t t0 = 0;
        const int pw = min((int)threadIdx.x * (nw / DEC_WG), nw - 1);
        while ((uint32_t)(dec_ald(a.ht + pw) >> 32) != tag)
            if (!dec_keep_waiting(t0, a.status)) {
                expired = true;
                break;
            }
    }
    dec_lds_barrier();
    uint64_t u[DEC_HW];
    {
        uint64_t t0 = 0;
        while (true) {
#pragma unroll
            for (int hh = 0; hh < DEC_HPH; hh++)
#pragma unroll
                for (int j = 0; j < PW; j++)
                    u[hh * PW + j] = dec_ald(a.ht + (size_t)hh * half + min((int)threadIdx.x + DEC_WG * j, half - 1));
            bool all = true;
#pragma unroll
            for (int j = 0; j < DEC_HW; j++) all &= (uint32_t)(u[j] >> 32) == tag;
            if (all) break;
            if (!dec_keep_waiting(t0, a.status)) {
                expired = true;
                break;
            }
        }
    }
    if (threadIdx.x == 0) dec_bump(a.ctl); /* this workgroup has read all of h */
#pragma unroll
    for (int hh = 0; hh < DEC_HPH; hh++) {
#pragma unroll
        for (int j = 0; j < PW; j++) {
            const int i = (int)threadIdx.x + DEC_WG * j;
            if (i < half) s_hv[i] = __uint_as_float((uint32_t)u[hh * PW + j]);
        }
        dec_lds_barrier();
        {
            const int i = threadIdx.x; /* a part has at most DEC_WG units of 8 values */
            const int ui = hh * (half / 8) + min(i, half / 8 - 1);
            const int sg8 = ui / u8, q8 = ui - sg8 * u8;
            float v[8];
            const int li = 8 * min(i, half / 8 - 1);
            const float4 f0 = *(const float4 *)(s_hv + li), f1 = *(const float4 *)(s_hv + li + 4);
            v[0] = f0.x; v[1] = f0.y; v[2] = f0.z; v[3] = f0.w;
            v[4] = f1.x; v[5] = f1.y; v[6] = f1.z; v[7] = f1.w;
            uint32_t hi[4], lo[4];
            const float gs = qk_f32x8_pairs(v, hi, lo);
            uint32_t *cb = (uint32_t *)s_x + ((size_t)sg8 * CH + (q8 >> 2)) * 36;
            const int gi = q8 & 3;
            if (i < half / 8) {
                *(uint4 *)(cb + 4 * gi) = make_uint4(hi[0], hi[1], hi[2], hi[3]);
                *(uint4 *)(cb + 16 + 4 * gi) = make_uint4(lo[0], lo[1], lo[2], lo[3]);
                ((float *)cb)[32 + gi] = gs;
            }
        }
        dec_lds_barrier();
    }

    /* y for every item */
#pragma unroll
    for (int ps = 0; ps < DEC_NPASS; ps++) {
        const int item = ps * DEC_WAVES + wave;
        if (item >= items) continue;
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
    if (expired) s_misc[0] = 1;
    dec_lds_barrier();
    const bool bad = s_misc[0] != 0;

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

/* ------------------------------------------------------------ the launch */

template <int CPL, int LPRD, bool XBF16, bool NORM, int NCH, int PL>
__global__ __launch_bounds__(DEC_WG) void k_dec_layer(DlArgs a) {
    extern __shared__ float dec_lds[];
    const uint32_t tag = (uint32_t)(dec_ald(a.ctl) / (uint64_t)a.ND) + 1u;
    const int b = blockIdx.x;
    if (b < a.NR) {
        /* whole-line stores: partial-line stores under polling reach the
         * readers several times slower */
        const int wave = threadIdx.x >> 6;
#pragma unroll
        for (int i = 0; i < DEC_RT_ROWS / DEC_WAVES; i++) {
            const int row = b * DEC_RT_ROWS + i * DEC_WAVES + wave;
            if (row <= a.E) {
                const float v = router_rows<XBF16, NORM, NCH>(a.ra, row, 0, 1);
                if ((threadIdx.x & 63) == 0) dec_lds[i * DEC_WAVES + wave] = v;
            }
        }
        dec_lds_barrier();
        const int row = b * DEC_RT_ROWS + (int)threadIdx.x;
        if ((int)threadIdx.x < DEC_RT_ROWS && row <= a.E) dec_ast(a.lt + row, dec_word(dec_lds[threadIdx.x], tag));
        return;
    }
    if (b < a.NR + a.NS) {
        dec_gateup_shared<CPL, XBF16, NORM, NCH>(a, tag, b - a.NR, dec_lds);
        return;
    }
    const int g = b - a.NR - a.NS;
    if (g < a.k * a.NG) {
        const int slot = g / a.NG;
        dec_gateup_routed<CPL, XBF16, NORM, NCH, PL>(a, tag, slot, g - slot * a.NG, dec_lds);
        return;
    }
    dec_down_combine<LPRD, PL>(a, tag, dec_lds);
}

/* ------------------------------------------------------------ host side */

static int dec_pl(int E) {
    int pl = 2;
    while (pl * 64 < E) pl <<= 1;
    return pl;
}

/* rows per down workgroup: the largest power of two <= 32 dividing H with
 * every (segment, row group) item of a workgroup within DEC_NPASS passes;
 * 0 when none fits (16 lanes per down row, so 4 rows per wave item) */
static int dec_rbd(qk_shape s) {
    for (int rbd = 32; rbd >= 4; rbd >>= 1)
        if (s.H % rbd == 0 && (s.k + 1) * (rbd / 4) <= DEC_NPASS * DEC_WAVES) return rbd;
    return 0;
}

static size_t dec_up256(size_t b) { return (b + 255) & ~(size_t)255; }

extern "C" size_t qk_dec_lds(qk_shape s) {
    const int rbd = dec_rbd(s);
    const size_t down = ((size_t)(s.k + 1) * (s.I / 32) * 36 + (size_t)(s.k + 1) * s.I / DEC_HPH +
                         (size_t)(s.k + 1) * rbd + 2 * QK_MAX_TOPK + 4) * 4;
    const size_t gateup = (size_t)(DEC_RB_G + 4 + 64 * (dec_pl(s.E) + 1)) * 4;
    return down > gateup ? down : gateup;
}

extern "C" int qk_dec_supported(qk_shape s) {
    const int ch = s.H / 32;
    if (!(ch == 64 || ch == 128)) return 0;          /* gate/up: 64 lanes x 1 or 2 chunks */
    if (s.I != 512) return 0;                        /* down: 16 lanes per row of h */
    if (s.E < s.k || s.E > 64 * 16 || s.k > QK_MAX_TOPK) return 0;
    if ((s.k + 1) * s.I > DEC_WG * DEC_HW || (s.k + 1) * s.I % (8 * DEC_HPH)) return 0; /* h parts */
    if (!dec_rbd(s)) return 0;
    if ((size_t)(s.k + 1) * (s.I / 32) * 36 < (size_t)64 * (dec_pl(s.E) + 1)) return 0; /* logits in s_x */
    return qk_dec_lds(s) <= 65536;
}

extern "C" size_t qk_dec_handoff_bytes(qk_shape s) {
    return DEC_CTL_BYTES + dec_up256((size_t)(s.E + 1) * 8) + dec_up256((size_t)(s.k + 1) * s.I * 8);
}

template <int CPL, bool XBF16, bool NORM>
static void dec_launch(int pl, dim3 grid, size_t lds, const DlArgs &a, hipStream_t st) {
    constexpr int NCH = 4 * CPL; /* router: chunks of 8 per lane */
    switch (pl) {
    case 2: hipLaunchKernelGGL((k_dec_layer<CPL, 16, XBF16, NORM, NCH, 2>), grid, dim3(DEC_WG), lds, st, a); break;
    case 4: hipLaunchKernelGGL((k_dec_layer<CPL, 16, XBF16, NORM, NCH, 4>), grid, dim3(DEC_WG), lds, st, a); break;
    case 8: hipLaunchKernelGGL((k_dec_layer<CPL, 16, XBF16, NORM, NCH, 8>), grid, dim3(DEC_WG), lds, st, a); break;
    default: hipLaunchKernelGGL((k_dec_layer<CPL, 16, XBF16, NORM, NCH, 16>), grid, dim3(DEC_WG), lds, st, a); break;
    }
}

extern "C" int qk_launch_dec_layer(const qmoe_layer_weights *W, qk_shape s, const void *x, int x_bf16,
                                   float *logits, float *xn, float *h, void *handoff, uint32_t *status,
                                   int32_t *idx, float *w, float *sg, int32_t *perm, int32_t *pos,
                                   int32_t *segtab, const void *x_res, float *out, float *hyper,
                                   const float *inject, int hc, void *stream) {
    if (!qk_dec_supported(s) || !handoff) return (int)hipErrorInvalidValue;
    hipStream_t st = (hipStream_t)stream;
    const int cpl = s.H / 2048;
    const bool norm = W->norm_w != nullptr;
    char *hb = (char *)handoff;
    DlArgs a;
    a.ra.router_w = W->router_w;
    a.ra.router_bias = W->router_bias;
    a.ra.sh_gate_w = W->sh_gate_w;
    a.ra.norm_w = W->norm_w;
    a.ra.x = x;
    a.ra.logits = logits;
    a.ra.xn = norm ? xn : nullptr;
    a.ra.phi = a.ra.plo = nullptr;
    a.ra.pg = nullptr;
    a.ra.H = s.H;
    a.ra.E = s.E;
    a.ra.n = 1;
    a.ra.eps = s.eps;
    a.lt = (uint64_t *)(hb + DEC_CTL_BYTES);
    a.q[0] = W->gate_q; a.s[0] = W->gate_s; a.b[0] = W->gate_b;
    a.q[1] = W->up_q;   a.s[1] = W->up_s;   a.b[1] = W->up_b;
    a.sq[0] = W->sh_gate_q; a.ss[0] = W->sh_gate_s; a.sb[0] = W->sh_gate_b;
    a.sq[1] = W->sh_up_q;   a.ss[1] = W->sh_up_s;   a.sb[1] = W->sh_up_b;
    a.dq = W->down_q; a.ds = W->down_s; a.db = W->down_b;
    a.sdq = W->sh_down_q; a.sds = W->sh_down_s; a.sdb = W->sh_down_b;
    a.xres = x_res;
    a.xres_bf16 = x_bf16;
    a.ctl = (uint64_t *)hb;
    a.ht = (uint64_t *)(hb + DEC_CTL_BYTES + dec_up256((size_t)(s.E + 1) * 8));
    a.status = status;
    a.h = h;
    a.idx = idx; a.w = w; a.sg = sg; a.perm = perm; a.pos = pos; a.segtab = segtab;
    a.out = out;
    a.hyper = hyper;
    a.inject = inject;
    a.hc = hc;
    a.H = s.H; a.E = s.E; a.k = s.k; a.I = s.I;
    a.NR = (s.E + 1 + DEC_RT_ROWS - 1) / DEC_RT_ROWS;
    a.NS = s.I / DEC_RB_G;
    a.NG = s.I / DEC_RB_G;
    a.RBD = dec_rbd(s);
    a.ND = s.H / a.RBD;
    const dim3 grid(a.NR + a.NS + s.k * a.NG + a.ND);
    const size_t lds = qk_dec_lds(s);
    const int pl = dec_pl(s.E);
    if (cpl == 1) {
        if (x_bf16) norm ? dec_launch<1, true, true>(pl, grid, lds, a, st) : dec_launch<1, true, false>(pl, grid, lds, a, st);
        else norm ? dec_launch<1, false, true>(pl, grid, lds, a, st) : dec_launch<1, false, false>(pl, grid, lds, a, st);
    } else {
        if (x_bf16) norm ? dec_launch<2, true, true>(pl, grid, lds, a, st) : dec_launch<2, true, false>(pl, grid, lds, a, st);
        else norm ? dec_launch<2, false, true>(pl, grid, lds, a, st) : dec_launch<2, false, false>(pl, grid, lds, a, st);
    }
    return QK_CHECK_LAUNCH();
}
