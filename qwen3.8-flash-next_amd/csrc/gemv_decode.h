/*
 * gemv_decode.h -- grouped gate/up GEMV for one token (decode), gfx950.
 *
 * One workgroup per (segment, block of RB rows), no task loop: with one
 * token every segment has one row and there are at most k routed segments,
 * so the grid is (k+1) x blocks.  Segment 0 is the shared expert (output
 * row k); segment j >= 1 is entry j-1 of the segment table.
 *
 * Lane mapping: LPR lanes share a weight row and lane `sub` owns the CPL
 * consecutive 32-code chunks sub*CPL .. sub*CPL+CPL-1 (K = 32*LPR*CPL), so
 * its scales and biases are CPL/2 consecutive bf16 values and its
 * activations one contiguous run.  Per chunk the lane accumulates
 * D = sum x*(128+q) with v_dot2c_f32_bf16 on (code i, code i+4) pairs and
 * applies the gemm_q4 group identity (kernel.c:279-282) as
 *     acc = s*D + (b - 128*s)*xs,        xs = sum x over the chunk,
 * then the row is summed over its LPR lanes.  All loads are issued before
 * any test on the segment entry; an invalid entry reads expert 0 and
 * stores nothing.
 */
#ifndef GEMV_DECODE_H
#define GEMV_DECODE_H

#include "qk_device.h"
#include "topk_wave.h"

struct DecArgs {
    const uint32_t *q[2];  /* routed gate, up [E, N, K/8] */
    const uint16_t *s[2];  /* [E, N, K/64] */
    const uint16_t *b[2];
    const uint32_t *sq[2]; /* shared gate, up [N, K/8] */
    const uint16_t *ss[2];
    const uint16_t *sb[2];
    const void *x;         /* [1, K] bf16 or f32 */
    float *out;            /* [k+1, N]: h = silu(g) * u, rows in dispatch order */
    int K, N, k, E;
};

/* GPL consecutive bf16 values starting at p (GPL = 1, 2 or 4) */
template <int GPL>
__device__ __forceinline__ void dec_ld_bf16(const uint16_t *p, float v[GPL]) {
    if (GPL == 1) {
        v[0] = qk_bf16(qk_ld(p));
    } else if (GPL == 2) {
        const uint32_t w = qk_ld((const uint32_t *)p);
        v[0] = qk_bf16_lo(w);
        v[GPL > 1 ? 1 : 0] = qk_bf16_hi(w);
    } else {
        const uint2 w = qk_ld((const uint2 *)p);
        v[0] = qk_bf16_lo(w.x);
        v[GPL > 1 ? 1 : 0] = qk_bf16_hi(w.x);
        v[GPL > 2 ? 2 : 0] = qk_bf16_lo(w.y);
        v[GPL > 3 ? 3 : 0] = qk_bf16_hi(w.y);
    }
}

/* routing outputs written by the fused top-k variant (one workgroup) */
struct DecRouteOut {
    const float *logits; /* [E+1]: router logits, then the shared-gate logit */
    int32_t *idx;        /* [k] */
    float *w;            /* [k] */
    float *sg;           /* [1] */
    int32_t *perm, *pos; /* [k] */
    int32_t *segtab;     /* [1+3k] */
};

/*
 * TK = 0: segment j >= 1 is entry j-1 of `segtab` (any table made by the
 *         dispatch for one token).
 * TK = PL > 0: the workgroups of routed segments select the top k of the
 *         router logits themselves (wave 0, WaveTopk<PL>, broadcast through
 *         LDS) instead of waiting for a separate top-k launch.  Segment j
 *         computes the expert of slot j-1: wave 0 runs the selection rounds
 *         (two slots a round) up to that slot, every wave starts its weight
 *         loads, and wave 0
 *         runs the remaining rounds under the loads to find the expert's
 *         dispatch position (its rank among the selected ids), which only
 *         the stores need.  Workgroup (segment 1, block 0) writes the
 *         routing (idx, w, sigmoid gate, perm, pos, segment table) for the
 *         down projection and the combine, in the form the dispatch
 *         produces.
 */
template <int LPR, int CPL, int RIT, bool XBF16, int TK = 0>
__global__ __launch_bounds__(256) void k_gateup_dec(DecArgs a, const int32_t *__restrict__ segtab,
                                                    DecRouteOut ro) {
    constexpr int RPW = 64 / LPR;
    constexpr int RB = 4 * RPW * RIT;
    constexpr int GPL = CPL >= 2 ? CPL / 2 : 1; /* scale groups per lane */
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int sub = lane % LPR, rsub = lane / LPR;
    const int G = a.K >> 6;
    const size_t wrow = (size_t)a.K >> 3;
    const int tps = (a.N + RB - 1) / RB;
    const int seg = blockIdx.x / tps, rb = blockIdx.x - seg * tps;
    const int c0 = sub * CPL;     /* first chunk of this lane */
    const int g0 = (c0 >> 1);     /* first scale group of this lane */

    /* Activations, staged once per workgroup: the K/8 groups of 8 values
     * are loaded in address order (a wave's load covers one contiguous
     * run), converted to (x_i, x_{i+4}) bf16 pairs (f32: hi and lo pairs and
     * the group sum) and left in LDS for every lane's chunk.  In routed
     * workgroups of the fused top-k, wave 0 stages nothing, so its logit
     * loads are not queued behind activation loads. */
    constexpr int NG = 4 * LPR * CPL;            /* groups of 8 activations */
    constexpr int NSTG = (NG + 191) / 192;       /* groups per staging thread, at most */
    __shared__ uint4 s_xh[NG];
    __shared__ uint4 s_xl[XBF16 ? 1 : NG];
    __shared__ float s_xg[XBF16 ? 1 : NG];
    const bool shared = seg == 0;
    const int st0 = (TK > 0 && !shared) ? 64 : 0; /* first staging thread */
    const int sts = 256 - st0;
    uint4 xd[XBF16 ? NSTG : 1];
    float4 xf[XBF16 ? 1 : NSTG][2];
#pragma unroll
    for (int j = 0; j < NSTG; j++) {
        const int gi = min(max((int)threadIdx.x - st0, 0) + j * sts, NG - 1);
        if (XBF16) xd[XBF16 ? j : 0] = qk_ld((const uint4 *)a.x + gi);
        else {
            xf[XBF16 ? 0 : j][0] = qk_ld((const float4 *)a.x + 2 * gi);
            xf[XBF16 ? 0 : j][1] = qk_ld((const float4 *)a.x + 2 * gi + 1);
        }
    }
    /* groups -> LDS slots, XOR-swizzled within runs of four */
    auto xslot = [](int gi) { return gi ^ ((gi >> 2) & 3); };
    auto stage_x = [&]() {
#pragma unroll
        for (int j = 0; j < NSTG; j++) {
            const int gi = (int)threadIdx.x - st0 + j * sts;
            if ((int)threadIdx.x < st0 || gi >= NG) continue;
            uint32_t hp4[4];
            if (XBF16) {
                qk_bf16x8_to_pairs(xd[XBF16 ? j : 0], hp4);
            } else {
                const float4 a0 = xf[XBF16 ? 0 : j][0], a1 = xf[XBF16 ? 0 : j][1];
                const float v[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
                uint32_t lp4[4];
                s_xg[XBF16 ? 0 : gi] = qk_f32x8_pairs(v, hp4, lp4);
                s_xl[XBF16 ? 0 : xslot(gi)] = make_uint4(lp4[0], lp4[1], lp4[2], lp4[3]);
            }
            s_xh[xslot(gi)] = make_uint4(hp4[0], hp4[1], hp4[2], hp4[3]);
        }
    };

    const int slot = seg - 1;
    bool valid;
    int e, p0;
    __shared__ int s_ep[2]; /* the slot's expert, then its dispatch position */
    WaveTopk<(TK > 0 ? TK : 1)> tks;
    uint32_t my_key = 0u; /* lane r < k: slot r's key and expert, once known */
    int my_id = 0x7FFFFFFF;
    if (TK > 0) {
        if (!shared) {
            if (wave != 0) stage_x();
            if (wave == 0) {
                tks.init(ro.logits, a.E, lane);
                /* two slots a round, up to the round that yields this slot */
                int es = 0;
                for (int r = 0; 2 * r <= slot; r++) {
                    uint32_t m1, m2;
                    int ea, eb;
                    tks.next2(lane, m1, ea, m2, eb);
                    if (lane == 2 * r) {
                        my_key = m1;
                        my_id = ea;
                    }
                    if (lane == 2 * r + 1 && 2 * r + 1 < a.k) {
                        my_key = m2;
                        my_id = eb;
                    }
                    es = (2 * r == slot) ? ea : eb;
                }
                if (lane == 0) s_ep[0] = es;
            }
            __syncthreads();
        } else {
            stage_x(); /* read after the barrier below, under the weight loads */
        }
        valid = true;
        e = shared ? 0 : s_ep[0];
        p0 = a.k;
    } else {
        /* segment entry and count, read together; bitwise tests (no branches) */
        const int s1 = shared ? 1 : seg;
        const int u = segtab[0];
        const int e_raw = segtab[3 * s1 - 2], p_raw = segtab[3 * s1 - 1], m_raw = segtab[3 * s1];
        stage_x();
        valid = shared | ((seg <= u) & (e_raw >= 0) & (e_raw < a.E) & (p_raw >= 0) & (p_raw < a.k) &
                          (m_raw == 1));
        e = (valid && !shared) ? e_raw : 0;
        p0 = shared ? a.k : p_raw;
    }
    const uint32_t *q[2];
    const uint16_t *sc[2], *bi[2];
#pragma unroll
    for (int mt = 0; mt < 2; mt++) {
        q[mt] = shared ? a.sq[mt] : a.q[mt] + (size_t)e * a.N * wrow;
        sc[mt] = shared ? a.ss[mt] : a.s[mt] + (size_t)e * a.N * G;
        bi[mt] = shared ? a.sb[mt] : a.b[mt] + (size_t)e * a.N * G;
    }

    const int rbase = rb * RB + wave * (RPW * RIT);
    uint4 wq[RIT][2][CPL];
    float ws[RIT][2][GPL], wb[RIT][2][GPL];
#pragma unroll
    for (int it = 0; it < RIT; it++) {
        const int r0 = rbase + it * RPW + rsub;
        const int r = r0 < a.N ? r0 : 0;
#pragma unroll
        for (int mt = 0; mt < 2; mt++) {
            const uint4 *src = (const uint4 *)(q[mt] + (size_t)r * wrow) + c0;
#pragma unroll
            for (int c = 0; c < CPL; c++) wq[it][mt][c] = qk_ld(src + c);
            dec_ld_bf16<GPL>(sc[mt] + (size_t)r * G + g0, ws[it][mt]);
            dec_ld_bf16<GPL>(bi[mt] + (size_t)r * G + g0, wb[it][mt]);
        }
    }
    __builtin_amdgcn_sched_barrier(0);

    if (TK > 0 && !shared) {
        /* under the loads: the remaining rounds, then this slot's rank */
        if (wave == 0) {
            topk_rounds(tks, slot / 2 + 1, (a.k + 1) / 2, a.k, lane, my_key, my_id);
            const int rank = (int)__popcll(__ballot(my_id < e));
            if (lane == 0) s_ep[1] = rank;
            if (seg == 1 && rb == 0) {
                const float wt = topk_weight(my_key, a.k, lane);
                int rk = 0;
                for (int s2 = 0; s2 < a.k; s2++) rk += __builtin_amdgcn_readlane(my_id, s2) < my_id ? 1 : 0;
                if (lane < a.k) {
                    ro.idx[lane] = my_id;
                    ro.w[lane] = wt;
                    ro.perm[rk] = lane;
                    ro.pos[lane] = rk;
                    ro.segtab[1 + 3 * rk] = my_id;
                    ro.segtab[2 + 3 * rk] = rk;
                    ro.segtab[3 + 3 * rk] = 1;
                }
                if (lane == 0) {
                    ro.segtab[0] = a.k;
                    ro.sg[0] = qk_sigmoid(qk_ld(ro.logits + a.E));
                }
            }
        }
        qk_lds_barrier(); /* s_ep[1]; the weight loads stay in flight */
        p0 = s_ep[1];
    }

    if (!(TK > 0 && !shared)) qk_lds_barrier(); /* the staged groups; weight loads stay in flight */

    /* this lane's chunks from the staged groups: pairs (x_i, x_{i+4}) per 8
     * columns and the chunk sums (bf16: v_dot2 chain over the 16 pairs from
     * 0; f32: 0 + g0 + g1 + g2 + g3 over the four group sums, left to right) */
    uint32_t hp[CPL][16];
    uint32_t lp[XBF16 ? 1 : CPL][XBF16 ? 1 : 16];
    float xs[CPL];
#pragma unroll
    for (int c = 0; c < CPL; c++) {
#pragma unroll
        for (int w = 0; w < 4; w++) {
            const int gi = 4 * (c0 + c) + w;
            const uint4 h4 = s_xh[xslot(gi)];
            hp[c][4 * w] = h4.x; hp[c][4 * w + 1] = h4.y; hp[c][4 * w + 2] = h4.z; hp[c][4 * w + 3] = h4.w;
            if (!XBF16) {
                const uint4 l4 = s_xl[XBF16 ? 0 : xslot(gi)];
                uint32_t *l = lp[XBF16 ? 0 : c];
                l[XBF16 ? 0 : 4 * w] = l4.x; l[XBF16 ? 0 : 4 * w + 1] = l4.y;
                l[XBF16 ? 0 : 4 * w + 2] = l4.z; l[XBF16 ? 0 : 4 * w + 3] = l4.w;
            }
        }
        if (XBF16) {
            float s = 0.0f;
#pragma unroll
            for (int i = 0; i < 16; i++) s = qk_dot2(hp[c][i], QK_BF16_ONES, s);
            xs[c] = s;
        } else {
            const float4 g4 = *(const float4 *)&s_xg[XBF16 ? 0 : 4 * (c0 + c)];
            xs[c] = (((0.0f + g4.x) + g4.y) + g4.z) + g4.w;
        }
    }

#pragma unroll
    for (int it = 0; it < RIT; it++) {
        float acc[2];
#pragma unroll
        for (int mt = 0; mt < 2; mt++) {
            float part = 0.0f;
#pragma unroll
            for (int c = 0; c < CPL; c++) {
                const int gl = CPL >= 2 ? c >> 1 : 0;
                const float s = ws[it][mt][gl];
                const float bp = fmaf(-128.0f, s, wb[it][mt][gl]);
                const uint4 q4 = wq[it][mt][c];
                const uint32_t words[4] = {q4.x, q4.y, q4.z, q4.w};
                float d = 0.0f;
#pragma unroll
                for (int w = 0; w < 4; w++) {
                    uint32_t pr[4];
                    qk_codes_to_pairs(words[w], pr);
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        d = qk_dot2(hp[c][4 * w + i], pr[i], d);
                        if (!XBF16) d = qk_dot2(lp[XBF16 ? 0 : c][XBF16 ? 0 : 4 * w + i], pr[i], d);
                    }
                }
                part = fmaf(s, d, fmaf(bp, xs[c], part));
            }
            acc[mt] = qk_group_sum<LPR>(part);
        }
        const int r = rbase + it * RPW + rsub;
        if (valid && sub == 0 && r < a.N)
            qk_st(a.out + (size_t)p0 * a.N + r, qk_silu(acc[0]) * acc[1]);
    }
}

#endif
