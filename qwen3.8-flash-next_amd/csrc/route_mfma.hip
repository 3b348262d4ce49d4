/*
 * route_mfma.hip -- router logits + top-k for many tokens: logits from a
 * bf16 MFMA product, and the exact R64 logits (router_rows.h) recomputed
 * only for the experts that can enter a token's top k.  Replaces, for
 * batches of QK_ROUTE_MFMA_MIN_N tokens or more, the same steps as
 * router.hip: model.c:1301-1318 of the reference C port (gemm_bf16 router
 * product, kernel_topk_indices, softmax over the selected) with the
 * oracle's R64 order and canonical top-k (orc_dot_r64_bf16w,
 * orc_topk_canonical).
 *
 * Only the top k logits of a token, and its shared-expert gate logit, reach
 * the layer's outputs.  So:
 *
 *   k_rt_plane  (f32 input, or a pre-router norm) the token rows as bf16
 *               (RNE), and the normalised rows xn computed exactly as
 *               router_rows does (R64 sum of squares, r = 1/sqrt(ss/H +
 *               eps), (x*r)*w);
 *   k_rt_mm     a_e = (bf16 MFMA dot, f32 accumulation) + bias for every
 *               (token, expert), and the squared norms of the router rows;
 *   k_rt_exact  one wavefront per token: a bound eps_e >= |a_e - l_e|,
 *               l_e the exact R64 logit; T = the k-th largest a_e - eps_e;
 *               the exact logit of every e with a_e + eps_e >= T; then the
 *               canonical top-k and softmax of router.hip's k_topk on the
 *               row that holds those exact logits and -inf elsewhere.
 *
 * Two jobs of the following launches ride along when the caller asks: the
 * dispatch's token bitmask (k_rt_mm clears it, k_rt_exact sets the bits of
 * the token's k experts, as router.hip's k_fill_u32 + k_setbits), and the
 * grouped GEMM's operand planes of the rows k_rt_exact reads (pair-order
 * bf16 hi (+ lo for f32 rows) and P = -128 x group sums, k_pack_rows'
 * arithmetic term for term).
 *
 * Why the selection is the exact one: l_j >= a_j - eps_j for every j, so
 * the k-th largest exact logit is >= T, and every expert of the exact top
 * k has l_e >= T, hence a_e + eps_e >= T: it is recomputed.  An expert that
 * is not recomputed has l_j <= a_j + eps_j < T, below the k-th exact logit,
 * and lowering such values to -inf changes neither the selected set, nor
 * its order (value descending, ties to the lower id), nor the weights.
 *
 * The bound, per token x and router row w (K = H <= 2048 terms):
 *   - the R64 logit: each product passes through at most H/64 fma
 *     roundings of its lane's chain and 6 tree additions: within
 *     38 u sum|x w| of the real dot (u = 2^-24);
 *   - the MFMA dot: products of bf16 are exact; each passes through at
 *     most 32 additions inside one instruction, H/128 - 1 chained
 *     instructions and 2 additions joining the K quarters: within 2 * 81 u
 *     sum|x w| (2 u per addition also covers truncating hardware);
 *   - the bf16 rows of f32 input: |x - bf16(x)| <= 2^-9 |x|;
 *   - sum|x w| <= |x| |w| (Cauchy-Schwarz);
 *   - subnormal inputs, products or partial sums that the hardware may
 *     flush: below 2^-126 per term and per addition, within
 *     2^-110 (|x| + |w|) + 2^-100 for H <= 2048;
 *   - the bias addition and the rounding of a -+ eps: 2^-20 |a|.
 * eps = c |x| |w| + 2^-110 (|x| + |w|) + 2^-20 |a| + 2^-100 with
 * c = 2^-8 for rounded rows (2^-9 + 200 u needed) and 2^-12 for bf16 input
 * used as is (200 u = 1.2e-5 needed), so each leaves at least a factor 2.
 * A token for which any a_e or eps_e is not finite, or |x| |w| or |a_e|
 * reaches 2^126 (an exact partial sum could then overflow), has every
 * expert recomputed: its row is the full exact row.
 */
#include "qk_device.h"
#include "mfma_parts.h"
#include "gemv_parts.h"
#include "router_rows.h"
#include "topk_wave.h"

/* ------------------------------------------------------------ bf16 rows */

/* one wavefront per token; 4 per workgroup */
template <bool XBF16, bool NORM, int NCH>
__global__ __launch_bounds__(256) void k_rt_plane(RouterArgs a, uint16_t *plane) {
    constexpr int H = 512 * NCH;
    const int lane = threadIdx.x & 63;
    const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= a.n) return;
    const size_t roff = (size_t)t * H;
    float v[NCH][8];
#pragma unroll
    for (int i = 0; i < NCH; i++) load_x8<XBF16>(a.x, roff, lane + 64 * i, v[i]);
    if (NORM) {
        /* router_rows' arithmetic, term for term */
        float ss = 0.0f;
#pragma unroll
        for (int i = 0; i < NCH; i++)
#pragma unroll
            for (int j = 0; j < 8; j++) ss = fmaf(v[i][j], v[i][j], ss);
        ss = qk_group_sum<64>(ss);
        const float r = 1.0f / sqrtf(ss / (float)H + a.eps);
#pragma unroll
        for (int i = 0; i < NCH; i++) {
            const float4 *nw = (const float4 *)a.norm_w + 2 * (lane + 64 * i);
            const float4 w0 = qk_ld(nw), w1 = qk_ld(nw + 1);
            const float wn[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
            for (int j = 0; j < 8; j++) v[i][j] = (v[i][j] * r) * wn[j];
            float4 *o = (float4 *)(a.xn + roff) + 2 * (lane + 64 * i);
            o[0] = make_float4(v[i][0], v[i][1], v[i][2], v[i][3]);
            o[1] = make_float4(v[i][4], v[i][5], v[i][6], v[i][7]);
        }
    }
#pragma unroll
    for (int i = 0; i < NCH; i++)
        *((uint4 *)(plane + roff) + lane + 64 * i) =
            make_uint4(qk_cvt_pk_bf16(v[i][0], v[i][1]), qk_cvt_pk_bf16(v[i][2], v[i][3]),
                       qk_cvt_pk_bf16(v[i][4], v[i][5]), qk_cvt_pk_bf16(v[i][6], v[i][7]));
}

/* ------------------------------------------------------------ MFMA logits */

#define RTM_DEPTH 4 /* K-steps of operands in flight per wave */

struct RtMmArgs {
    const uint16_t *a;    /* [n, H] bf16 token rows */
    const uint16_t *w;    /* [E, H] router rows */
    const float *bias;    /* [E] or null */
    float *logits;        /* [n, E+1]: columns 0..E-1 written */
    float *wn2;           /* [E] squared norms of the router rows */
    uint4 *bits;          /* null, or the dispatch bitmask to clear */
    int nbits4;           /* its size in uint4 */
    int n, E, tiles, per; /* tiles of 64 tokens x 64 experts; per = ceil(tiles / 8) */
};

struct RtMmSmem {
    float p[4][64][65]; /* the four K quarters' partial tiles, [row][column] */
};

/* squared norm of router row e, one wave (lane sums, then the wave's tree) */
template <int NCH>
__device__ __forceinline__ float rt_row_norm2(const uint16_t *w, int e, int lane) {
    constexpr int H = 512 * NCH;
    uint4 d[NCH];
#pragma unroll
    for (int i = 0; i < NCH; i++) d[i] = qk_ld((const uint4 *)(w + (size_t)e * H) + lane + 64 * i);
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < NCH; i++) {
        const uint32_t u[4] = {d[i].x, d[i].y, d[i].z, d[i].w};
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const float lo = qk_bf16_lo(u[j]), hi = qk_bf16_hi(u[j]);
            ss = fmaf(lo, lo, ss);
            ss = fmaf(hi, hi, ss);
        }
    }
    return qk_group_sum<64>(ss);
}

/*
 * Grid: 8 * per tile workgroups.  Tile
 * workgroup L runs on XCD L % 8 and takes tile (L % 8) * per + L / 8, so an
 * XCD holds a contiguous range of tiles (tiles are token-major: a range is
 * a few token blocks against every expert, whose rows stay in its L2).
 * The 4 waves of a tile each take a quarter of K for all 64 x 64 outputs
 * (16 MFMA per K-step), and the quarters are summed through LDS in order.
 * 16x16x32 lane layout: A lane l holds token l%16, B lane l expert l%16,
 * both with K elements [8*(l/16), +8) of the step; D lane l holds expert
 * l%16 of tokens 4*(l/16) + i.  After its logits a tile workgroup also
 * writes the squared norms of ceil(64 / token blocks) of its 64 router rows
 * (rows its B operand just brought into L2): every row once, with no
 * workgroups of their own at the end of the grid.
 */
template <int NCH>
__global__ __launch_bounds__(256, 2) void k_rt_mm(RtMmArgs a) {
    constexpr int H = 512 * NCH;
    constexpr int S = H / 128; /* K-steps of 32 per wave */
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int L = blockIdx.x;
    if (a.bits)
        for (int i = L * 256 + tid; i < a.nbits4; i += (int)gridDim.x * 256) a.bits[i] = make_uint4(0u, 0u, 0u, 0u);
    const int tl = (L & 7) * a.per + (L >> 3);
    if (tl >= a.tiles) return;
    __shared__ __attribute__((aligned(16))) RtMmSmem sm;
    const int net = a.E >> 6;
    const int tt = tl / net, et = tl - tt * net;
    const int t0 = tt * 64, e0 = et * 64;
    const int r = lane & 15, kq = lane >> 4;
    const int kbase = wave * (H / 4) / 8 + kq; /* uint4 index of this lane's first K chunk */
    const uint4 *ap[4], *wp[4];
#pragma unroll
    for (int m = 0; m < 4; m++) {
        ap[m] = (const uint4 *)(a.a + (size_t)min(t0 + 16 * m + r, a.n - 1) * H) + kbase;
        wp[m] = (const uint4 *)(a.w + (size_t)(e0 + 16 * m + r) * H) + kbase;
    }
    uint4 A[RTM_DEPTH][4], B[RTM_DEPTH][4];
    auto load = [&](int s) {
#pragma unroll
        for (int m = 0; m < 4; m++) {
            A[s % RTM_DEPTH][m] = qk_ld(ap[m] + 4 * s);
            B[s % RTM_DEPTH][m] = qk_ld(wp[m] + 4 * s);
        }
    };
    qm_f32x4 acc[4][4];
#pragma unroll
    for (int m = 0; m < 4; m++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[m][j] = qm_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int s = 0; s < RTM_DEPTH - 1 && s < S; s++) load(s);
#pragma unroll
    for (int s = 0; s < S; s++) {
        if (s + RTM_DEPTH - 1 < S) load(s + RTM_DEPTH - 1);
        /* keep the prefetch here: left alone the scheduler sinks the loads
         * next to their MFMAs and the wave waits on every step */
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int m = 0; m < 4; m++)
#pragma unroll
            for (int j = 0; j < 4; j++)
                acc[m][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                    __builtin_bit_cast(qm_bf16x8, A[s % RTM_DEPTH][m]),
                    __builtin_bit_cast(qm_bf16x8, B[s % RTM_DEPTH][j]), acc[m][j], 0, 0, 0);
    }
#pragma unroll
    for (int m = 0; m < 4; m++)
#pragma unroll
        for (int j = 0; j < 4; j++)
#pragma unroll
            for (int i = 0; i < 4; i++) sm.p[wave][16 * m + 4 * kq + i][16 * j + r] = acc[m][j][i];
    __syncthreads();
    /* thread -> column tid % 64 of rows tid / 64 + 4 q: the quarters in
     * order, then the bias */
    const int c = tid & 63;
    const float b = a.bias ? qk_ld(a.bias + e0 + c) : 0.0f;
#pragma unroll
    for (int q = 0; q < 16; q++) {
        const int row = (tid >> 6) + 4 * q;
        const float v = ((sm.p[0][row][c] + sm.p[1][row][c]) + sm.p[2][row][c]) + sm.p[3][row][c];
        if (t0 + row < a.n) a.logits[(size_t)(t0 + row) * (a.E + 1) + e0 + c] = a.bias ? v + b : v;
    }
    /* rows e0 + tt * rpw .. of this expert block, one per wave in turn */
    const int ntt = a.tiles / net, rpw = (64 + ntt - 1) / ntt;
    for (int j = wave; j < rpw && tt * rpw + j < 64; j += 4) {
        const float ss = rt_row_norm2<NCH>(a.w, e0 + tt * rpw + j, lane);
        if (lane == 0) a.wn2[e0 + tt * rpw + j] = ss;
    }
}

/* ------------------------------------------------------------ exact top-k */

struct RtExactArgs {
    const void *x;          /* [n, H] rows of the exact dots (xn with a norm) */
    const uint16_t *w;      /* [E, H] */
    const uint16_t *sh_gate_w; /* [H] */
    const float *bias;      /* [E] or null */
    const float *logits;    /* [n, E+1] approximate, columns 0..E-1 */
    const float *wn2;       /* [E] */
    int32_t *idx;
    float *wt;
    float *sg;
    uint32_t *bits;         /* null, or the dispatch bitmask [E][NW] (cleared by k_rt_mm) */
    uint16_t *phi, *plo;    /* null, or the operand planes of x: hi; lo for f32 rows */
    float *pg;              /* with phi: P = -128 x the group sums, [n, H/64] */
    int n, E, k, NW;
    float coef;             /* 2^-8 for rounded MFMA rows, 2^-12 for bf16 input */
};

/* the exact R64 logit of row e (e == E: the shared gate), all lanes */
template <int NCH>
__device__ __forceinline__ const uint16_t *rt_row(const RtExactArgs &a, int e) {
    return e < a.E ? a.w + (size_t)e * (512 * NCH) : a.sh_gate_w;
}

/*
 * One wavefront per token, 4 per workgroup; PL = E / 64 experts per lane.
 * T is taken as the k-th largest of the 64 lane maxima of the lower
 * bounds: each of those maxima is some expert's bound, so at least k
 * bounds reach it and it is at most the k-th largest bound -- a valid
 * threshold that costs k rounds over one value per lane.  With at most 63
 * candidates (one lane each, the gate in the last list entry) the top k is
 * ranked among them directly: the rank of a candidate is the number of
 * candidates before it in k_topk's order (key descending, lower expert id
 * first, keys as WaveTopk makes them), so slot s holds what k_topk's round
 * s returns.  More candidates (ties, all-recomputed tokens) take k_topk's
 * selection on the whole row, non-candidates at -inf.
 */
template <bool XBF16, int NCH, int PL>
__global__ __launch_bounds__(256) void k_rt_exact(RtExactArgs a) {
    constexpr int H = 512 * NCH, E = 64 * PL;
    __shared__ int s_list[4][E + 1];
    __shared__ float s_res[4][E + 1];
    __shared__ float s_row[4][E];
    __shared__ int s_sid[4][64];
    __shared__ uint32_t s_skey[4][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int t = blockIdx.x * 4 + wave;
    if (t >= a.n) return; /* wave-level work only below: no workgroup barrier */
    int *list = s_list[wave];
    float *res = s_res[wave];

    float v[NCH][8];
#pragma unroll
    for (int i = 0; i < NCH; i++) load_x8<XBF16>(a.x, (size_t)t * H, lane + 64 * i, v[i]);
    if (a.phi) {
        /* the grouped GEMM's planes of this row: chunk lane + 64 i holds
         * columns 8 (lane + 64 i) .. +7, so the 8 lanes of a 64-column group
         * are adjacent, as the threads of k_pack_rows */
#pragma unroll
        for (int i = 0; i < NCH; i++) {
            uint32_t ph[4], pl[4];
            float gs = 0.0f;
            if (XBF16) {
                /* the rows' own bf16 (v holds them exactly) */
#pragma unroll
                for (int j = 0; j < 4; j++)
                    ph[j] = (__float_as_uint(v[i][j]) >> 16) | (__float_as_uint(v[i][j + 4]) & 0xFFFF0000u);
#pragma unroll
                for (int j = 0; j < 4; j++) gs = qk_dot2(ph[j], QK_BF16_ONES, gs);
            } else {
                qk_f32x8_to_pairs(v[i], ph, pl, gs);
                ((uint4 *)a.plo)[(size_t)t * (H / 8) + lane + 64 * i] = make_uint4(pl[0], pl[1], pl[2], pl[3]);
            }
            ((uint4 *)a.phi)[(size_t)t * (H / 8) + lane + 64 * i] = make_uint4(ph[0], ph[1], ph[2], ph[3]);
            gs += qk_dpp<QK_DPP_XOR1>(gs);
            gs += qk_dpp<QK_DPP_XOR2>(gs);
            gs += __shfl_xor(gs, 4, QK_WAVE);
            if ((lane & 7) == 0) a.pg[(size_t)t * (H / 64) + (lane >> 3) + 8 * i] = -128.0f * gs;
        }
    }
    float xs = 0.0f;
#pragma unroll
    for (int i = 0; i < NCH; i++)
#pragma unroll
        for (int j = 0; j < 8; j++) xs = fmaf(v[i][j], v[i][j], xs);
    const float xnorm = sqrtf(qk_group_sum<64>(xs));

    /* bounds of this lane's experts lane*PL + i */
    float up[PL];
    float lmax = -INFINITY;
    bool bad = false;
#pragma unroll
    for (int i = 0; i < PL; i++) {
        const int e = lane * PL + i;
        const float av = qk_ld(a.logits + (size_t)t * (E + 1) + e);
        const float wn = sqrtf(qk_ld(a.wn2 + e));
        const float xw = xnorm * wn;
        const float eps = a.coef * xw + 0x1p-110f * (xnorm + wn) + 0x1p-20f * fabsf(av) + 0x1p-100f;
        up[i] = av + eps;
        lmax = fmaxf(lmax, av - eps);
        /* false for NaN too */
        const bool ok = xw < 0x1p126f && fabsf(av) < 0x1p126f && eps < 0x1p126f;
        bad = bad || !ok;
    }
    const bool all = __ballot(bad) != 0ull;

    /* T = the k-th largest lane maximum */
    float T = -INFINITY;
    if (!all) {
        uint32_t key = qk_ordkey(lmax), m = 0u;
        for (int r = 0; r < a.k; r++) {
            m = qk_wave_max_u32(key);
            const int wl = (int)__builtin_ctzll(__ballot(key == m));
            if (lane == wl) key = 0u;
        }
        T = qk_ordkey_value(m);
    }

    /* candidates, listed in expert order; the shared gate last */
    int cnt = 0;
    bool cand[PL];
#pragma unroll
    for (int i = 0; i < PL; i++) {
        cand[i] = all || up[i] >= T;
        cnt += cand[i] ? 1 : 0;
    }
    int inc = cnt;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int u = __shfl_up(inc, o, QK_WAVE);
        if (lane >= o) inc += u;
    }
    const int C = __shfl(inc, 63, QK_WAVE);
    int p = inc - cnt;
#pragma unroll
    for (int i = 0; i < PL; i++)
        if (cand[i]) list[p++] = lane * PL + i;
    if (lane == 0) list[C] = E;
    qk_wave_lds_sync();

    /* exact logits, 4 rows in flight: router_rows' chains and tree */
    const int nl = C + 1;
    for (int j0 = 0; j0 < nl; j0 += 4) {
        int ee[4];
        uint4 wv[4][NCH];
#pragma unroll
        for (int u = 0; u < 4; u++) {
            ee[u] = list[min(j0 + u, nl - 1)];
            const uint16_t *row = rt_row<NCH>(a, ee[u]);
#pragma unroll
            for (int i = 0; i < NCH; i++) wv[u][i] = qk_ld((const uint4 *)row + lane + 64 * i);
        }
#pragma unroll
        for (int u = 0; u < 4; u++) {
            float acc = 0.0f;
#pragma unroll
            for (int i = 0; i < NCH; i++) {
                const uint4 d = wv[u][i];
                acc = fmaf(v[i][0], qk_bf16_lo(d.x), acc);
                acc = fmaf(v[i][1], qk_bf16_hi(d.x), acc);
                acc = fmaf(v[i][2], qk_bf16_lo(d.y), acc);
                acc = fmaf(v[i][3], qk_bf16_hi(d.y), acc);
                acc = fmaf(v[i][4], qk_bf16_lo(d.z), acc);
                acc = fmaf(v[i][5], qk_bf16_hi(d.z), acc);
                acc = fmaf(v[i][6], qk_bf16_lo(d.w), acc);
                acc = fmaf(v[i][7], qk_bf16_hi(d.w), acc);
            }
            acc = qk_group_sum<64>(acc);
            if (ee[u] < E && a.bias) acc = acc + qk_ld(a.bias + ee[u]);
            if (lane == 0 && j0 + u < nl) res[j0 + u] = acc;
        }
    }
    qk_wave_lds_sync();

    uint32_t my_key = 0u;
    int my_id = 0;
    if (C < 64) {
        const int id = lane < C ? list[lane] : 0;
        const uint32_t key = lane < C ? max(qk_ordkey(res[lane]), 1u) : 0u;
        int rank = 0;
        for (int j = 0; j < C; j++) {
            const uint32_t kj = (uint32_t)__builtin_amdgcn_readlane((int)key, j);
            const int ij = __builtin_amdgcn_readlane(id, j);
            rank += (kj > key || (kj == key && ij < id)) ? 1 : 0;
        }
        /* slot rank <- this candidate */
        int *slot_id = s_sid[wave];
        uint32_t *slot_key = s_skey[wave];
        if (lane < C && rank < a.k) {
            slot_id[rank] = id;
            slot_key[rank] = key;
        }
        qk_wave_lds_sync();
        if (lane < a.k) {
            my_id = slot_id[lane];
            my_key = slot_key[lane];
        }
    } else {
        /* k_topk's selection on the row */
        float *row = s_row[wave];
#pragma unroll
        for (int i = 0; i < PL; i++) row[lane * PL + i] = -INFINITY;
        qk_wave_lds_sync();
        for (int j = lane; j < C; j += 64) row[list[j]] = res[j];
        qk_wave_lds_sync();
        float lv[PL];
#pragma unroll
        for (int i = 0; i < PL; i++) lv[i] = row[lane * PL + i];
        WaveTopk<PL> st;
        st.init_vals(lv, E, lane);
        topk_rounds(st, 0, (a.k + 1) / 2, a.k, lane, my_key, my_id);
    }
    const float my_w = topk_weight(my_key, a.k, lane);
    if (lane < a.k) {
        a.idx[(size_t)t * a.k + lane] = my_id;
        a.wt[(size_t)t * a.k + lane] = my_w;
        /* ids outside [0, E) are not dispatched, as in k_setbits */
        if (a.bits && (unsigned)my_id < (unsigned)a.E) atomicOr(&a.bits[(size_t)my_id * a.NW + (t >> 5)], 1u << (t & 31));
    }
    if (lane == 0) a.sg[t] = qk_sigmoid(res[C]);
}

/* ------------------------------------------------------------ host */

static int rt_pl(int E) {
    for (int pl = 1; pl <= 16; pl <<= 1)
        if (64 * pl == E) return pl;
    return 0;
}

extern "C" int qk_route_mfma_ok(qk_shape s, int n) {
    /* instances for H = 512 * NCH, NCH = 1, 2, 4 */
    return n >= QK_ROUTE_MFMA_MIN_N && (s.H == 512 || s.H == 1024 || s.H == 2048) && rt_pl(s.E) > 0 &&
           s.k >= 1 && s.k <= 64 && s.k <= s.E;
}

extern "C" int qk_launch_route_mfma(const qmoe_layer_weights *W, qk_shape s, const void *x, int x_bf16,
                                    int n, float *logits, float *xn, uint16_t *plane, float *wn2,
                                    int32_t *idx, float *w, float *sg, uint32_t *bits, uint16_t *phi,
                                    uint16_t *plo, float *pg, void *stream) {
    if (n <= 0) return 0;
    if (!qk_route_mfma_ok(s, n)) return (int)hipErrorInvalidValue;
    hipStream_t st = (hipStream_t)stream;
    const int nch = s.H / 512, pl = rt_pl(s.E);
    const bool norm = W->norm_w != nullptr;
    const bool as_is = x_bf16 && !norm; /* the MFMA reads x itself */
    if (norm && !xn) return (int)hipErrorInvalidValue;
    /* the planes are of the rows k_rt_exact reads: f32 ones need lo too */
    if (phi && (!pg || (!as_is && !plo))) return (int)hipErrorInvalidValue;
    const int NW = (n + 31) / 32;

    RouterArgs ra;
    ra.router_w = W->router_w;
    ra.router_bias = W->router_bias;
    ra.sh_gate_w = W->sh_gate_w;
    ra.norm_w = W->norm_w;
    ra.x = x;
    ra.logits = logits;
    ra.xn = xn;
    ra.phi = ra.plo = nullptr;
    ra.pg = nullptr;
    ra.H = s.H;
    ra.E = s.E;
    ra.n = n;
    ra.eps = s.eps;
    if (!as_is) {
        const dim3 grid((n + 3) / 4);
#define RTP_L(XB, NR, NC) hipLaunchKernelGGL((k_rt_plane<XB, NR, NC>), grid, dim3(256), 0, st, ra, plane)
#define RTP_N(XB, NR) \
    do { if (nch == 1) RTP_L(XB, NR, 1); else if (nch == 2) RTP_L(XB, NR, 2); else RTP_L(XB, NR, 4); } while (0)
        if (x_bf16) RTP_N(true, true);
        else if (norm) RTP_N(false, true);
        else RTP_N(false, false);
#undef RTP_N
#undef RTP_L
        int rc = QK_CHECK_LAUNCH();
        if (rc) return rc;
    }

    RtMmArgs ma;
    ma.a = as_is ? (const uint16_t *)x : plane;
    ma.w = W->router_w;
    ma.bias = W->router_bias;
    ma.logits = logits;
    ma.wn2 = wn2;
    ma.bits = (uint4 *)bits;
    ma.nbits4 = bits ? s.E * NW / 4 : 0; /* E is a multiple of 64 */
    ma.n = n;
    ma.E = s.E;
    ma.tiles = (n + 63) / 64 * (s.E / 64);
    ma.per = (ma.tiles + 7) / 8;
    const dim3 mgrid(8 * ma.per);
    if (nch == 1) hipLaunchKernelGGL(k_rt_mm<1>, mgrid, dim3(256), 0, st, ma);
    else if (nch == 2) hipLaunchKernelGGL(k_rt_mm<2>, mgrid, dim3(256), 0, st, ma);
    else hipLaunchKernelGGL(k_rt_mm<4>, mgrid, dim3(256), 0, st, ma);
    int rc = QK_CHECK_LAUNCH();
    if (rc) return rc;

    RtExactArgs ea;
    ea.x = norm ? (const void *)xn : x;
    ea.w = W->router_w;
    ea.sh_gate_w = W->sh_gate_w;
    ea.bias = W->router_bias;
    ea.logits = logits;
    ea.wn2 = wn2;
    ea.idx = idx;
    ea.wt = w;
    ea.sg = sg;
    ea.bits = bits;
    ea.phi = phi;
    ea.plo = as_is ? nullptr : plo;
    ea.pg = pg;
    ea.n = n;
    ea.E = s.E;
    ea.k = s.k;
    ea.NW = NW;
    ea.coef = as_is ? 0x1p-12f : 0x1p-8f;
    const dim3 egrid((n + 3) / 4);
#define RTE_L(XB, NC, PL) hipLaunchKernelGGL((k_rt_exact<XB, NC, PL>), egrid, dim3(256), 0, st, ea)
#define RTE_P(XB, NC)                                                                          \
    do {                                                                                       \
        switch (pl) {                                                                          \
        case 1: RTE_L(XB, NC, 1); break;                                                       \
        case 2: RTE_L(XB, NC, 2); break;                                                       \
        case 4: RTE_L(XB, NC, 4); break;                                                       \
        case 8: RTE_L(XB, NC, 8); break;                                                       \
        default: RTE_L(XB, NC, 16); break;                                                     \
        }                                                                                      \
    } while (0)
#define RTE_N(XB) \
    do { if (nch == 1) RTE_P(XB, 1); else if (nch == 2) RTE_P(XB, 2); else RTE_P(XB, 4); } while (0)
    /* the exact dots read x as bf16 only when the MFMA read it as is */
    if (as_is) RTE_N(true);
    else RTE_N(false);
#undef RTE_N
#undef RTE_P
#undef RTE_L
    return QK_CHECK_LAUNCH();
}
