/*
 * router.hip -- router logits, top-k + renormalise, and token dispatch for
 * gfx950.  Replaces model.c:1301-1332 and 1354-1367 of the reference C port
 * (gemm_bf16 + kernel_topk_indices + softmax-over-selected + expert gather).
 *
 * Router reduction order ("R64", bit-exact with the oracle): for one
 * (token, expert) dot product the K axis is cut into 8-element chunks, chunk
 * c goes to lane c%64 of a wavefront, each lane runs an fma chain over its
 * chunks in ascending order starting at +0.0f, and the wave combines its
 * lanes with the pairwise tree of qk_group_sum<64> (partners l^1 ... l^32).
 */
#include "qk_device.h"
#include "mm_tasks.h"

#include "router_rows.h"

template <bool XBF16, bool NORM, int NCH>
__global__ __launch_bounds__(256) void k_router(RouterArgs a) {
    const int row = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (row > a.E) return;
    const int t0 = blockIdx.y * RT_TB;
    router_rows<XBF16, NORM, NCH>(a, row, t0, min(a.n, t0 + RT_TB));
}

/*
 * Many tokens: one workgroup per (block of RTT_TOK*4 tokens, slice of rows).
 * Each wave keeps RTT_TOK token rows in registers as f32 (lane l holds the
 * chunks l, l+64, ..; H = 512*NCH) and the workgroup streams its weight rows
 * through LDS, RTT_EB rows per stage, converted to f32 once and read by all
 * four waves, double buffered.  The arithmetic per (token, row) is the R64
 * order above (same chains, same tree), so logits are identical to k_router.
 */
#define RTT_TOK 4
#define RTT_MIN_N 16
#define RTT_EB 4
static_assert(RTT_TOK * RTT_EB == 16, "the tile router reduces 16 partials per lane");

template <bool XBF16, bool NORM, int NCH>
__global__ __launch_bounds__(256, 2) void k_router_tile(RouterArgs a, int rows_per_wg) {
    constexpr int H = 512 * NCH;
    __shared__ __attribute__((aligned(16))) float s_w[2][RTT_EB][H];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r0 = blockIdx.y * rows_per_wg;
    const int r1 = min(a.E + 1, r0 + rows_per_wg);
    if (r0 >= r1) return;
    const int tb = blockIdx.x * (4 * RTT_TOK) + wave * RTT_TOK;

    /* this wave's tokens (rows past n repeat token n-1; they are not stored) */
    float v[RTT_TOK][NCH][8];
#pragma unroll
    for (int t = 0; t < RTT_TOK; t++) {
        const size_t roff = (size_t)min(tb + t, a.n - 1) * H;
#pragma unroll
        for (int i = 0; i < NCH; i++) load_x8<XBF16>(a.x, roff, lane + 64 * i, v[t][i]);
        if (NORM) {
            float ss = 0.0f;
#pragma unroll
            for (int i = 0; i < NCH; i++)
#pragma unroll
                for (int j = 0; j < 8; j++) ss = fmaf(v[t][i][j], v[t][i][j], ss);
            ss = qk_group_sum<64>(ss);
            const float r = 1.0f / sqrtf(ss / (float)H + a.eps);
#pragma unroll
            for (int i = 0; i < NCH; i++) {
                const float4 *nw = (const float4 *)a.norm_w + 2 * (lane + 64 * i);
                const float4 w0 = qk_ld(nw), w1 = qk_ld(nw + 1);
                const float wn[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
                for (int j = 0; j < 8; j++) v[t][i][j] = (v[t][i][j] * r) * wn[j];
                if (blockIdx.y == 0 && a.xn && tb + t < a.n) {
                    float4 *o = (float4 *)(a.xn + (size_t)(tb + t) * H) + 2 * (lane + 64 * i);
                    o[0] = make_float4(v[t][i][0], v[t][i][1], v[t][i][2], v[t][i][3]);
                    o[1] = make_float4(v[t][i][4], v[t][i][5], v[t][i][6], v[t][i][7]);
                }
            }
        }
        if (a.phi) {
            /* the MFMA gate/up operand planes of the experts' input (x, or
             * the normed rows), k_pack_rows' arithmetic: the 8 chunks of a
             * 64-column group sit in lanes 8j..8j+7.  The token block's
             * chunk sets i = 0..NCH-1 go to row slices i % slices, so no
             * one workgroup carries them all */
            const bool two = !XBF16 || NORM;
#pragma unroll
            for (int i = 0; i < NCH; i++) {
                if ((int)blockIdx.y != i % (int)gridDim.y) continue;
                uint32_t ph[4], pl[4];
                float sg = 0.0f;
                if (two) {
                    qk_f32x8_to_pairs(v[t][i], ph, pl, sg);
                } else {
#pragma unroll
                    for (int j = 0; j < 4; j++) ph[j] = qk_cvt_pk_bf16(v[t][i][j], v[t][i][j + 4]);
#pragma unroll
                    for (int j = 0; j < 4; j++) sg = qk_dot2(ph[j], QK_BF16_ONES, sg);
                }
                sg += qk_dpp<QK_DPP_XOR1>(sg);
                sg += qk_dpp<QK_DPP_XOR2>(sg);
                sg += __shfl_xor(sg, 4, QK_WAVE);
                if (tb + t < a.n) {
                    const size_t ci = (size_t)(tb + t) * (H / 8) + lane + 64 * i;
                    ((uint4 *)a.phi)[ci] = make_uint4(ph[0], ph[1], ph[2], ph[3]);
                    if (two) ((uint4 *)a.plo)[ci] = make_uint4(pl[0], pl[1], pl[2], pl[3]);
                    if ((lane & 7) == 0) a.pg[ci >> 3] = -128.0f * sg;
                }
            }
        }
    }

    /* weight staging: stage row rr, 16-byte chunk q of the row, per thread
     * RTT_EB*H/8/256 chunks */
    constexpr int SCH = RTT_EB * H / 8 / 256;
    uint4 wst[SCH];
    auto load_rows = [&](int rb) {
#pragma unroll
        for (int i = 0; i < SCH; i++) {
            const int ci = tid + 256 * i;
            const int rr = ci / (H / 8), q = ci - rr * (H / 8);
            const int row = min(rb + rr, r1 - 1);
            const uint16_t *wrow = row < a.E ? a.router_w + (size_t)row * H : a.sh_gate_w;
            wst[i] = qk_ld((const uint4 *)wrow + q);
        }
    };
    auto store_rows = [&](int buf) {
#pragma unroll
        for (int i = 0; i < SCH; i++) {
            const int ci = tid + 256 * i;
            const int rr = ci / (H / 8), q = ci - rr * (H / 8);
            const uint4 d = wst[i];
            float4 *o = (float4 *)&s_w[buf][rr][8 * q];
            o[0] = make_float4(qk_bf16_lo(d.x), qk_bf16_hi(d.x), qk_bf16_lo(d.y), qk_bf16_hi(d.y));
            o[1] = make_float4(qk_bf16_lo(d.z), qk_bf16_hi(d.z), qk_bf16_lo(d.w), qk_bf16_hi(d.w));
        }
    };

    load_rows(r0);
    store_rows(0);
    if (r0 + RTT_EB < r1) load_rows(r0 + RTT_EB);
    __syncthreads();
    const int rs_d = qk_rs16_index(lane); /* this lane's (token, row) after the reduction */
    for (int rb = r0, it = 0; rb < r1; rb += RTT_EB, it++) {
        const int buf = it & 1;
        /* the bias of this lane's row, loaded before the sums: loaded at the
         * store, the barrier that ends the stage would wait for it */
        const float bv = a.router_bias ? qk_ld(a.router_bias + min(rb + rs_d % RTT_EB, a.E - 1)) : 0.0f;
        /* partial sums of this lane, d = t*RTT_EB + rr */
        float part[RTT_TOK * RTT_EB];
#pragma unroll
        for (int rr = 0; rr < RTT_EB; rr++) {
            float acc[RTT_TOK];
#pragma unroll
            for (int t = 0; t < RTT_TOK; t++) acc[t] = 0.0f;
#pragma unroll
            for (int i = 0; i < NCH; i++) {
                const float4 *wp = (const float4 *)&s_w[buf][rr][8 * (lane + 64 * i)];
                const float4 w0 = wp[0], w1 = wp[1];
                const float w[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
                for (int j = 0; j < 8; j++)
#pragma unroll
                    for (int t = 0; t < RTT_TOK; t++) acc[t] = fmaf(v[t][i][j], w[j], acc[t]);
            }
#pragma unroll
            for (int t = 0; t < RTT_TOK; t++) part[t * RTT_EB + rr] = acc[t];
            __builtin_amdgcn_sched_barrier(0); /* one row's LDS reads at a time */
        }
        /* the 16 wave sums, each in the R64 tree's pairing, spread over lanes */
        const float val = qk_reduce_scatter16(part, lane);
        {
            const int d = rs_d;
            const int t = d / RTT_EB, row = rb + d % RTT_EB;
            if (lane < 16 && row < r1 && tb + t < a.n) {
                float o = val;
                if (row < a.E && a.router_bias) o = o + bv;
                a.logits[(size_t)(tb + t) * (a.E + 1) + row] = o;
            }
        }
        /* the next stage goes into the other buffer, last read one stage ago */
        if (rb + RTT_EB < r1) {
            store_rows(buf ^ 1);
            if (rb + 2 * RTT_EB < r1) load_rows(rb + 2 * RTT_EB);
        }
        __syncthreads();
    }
}

/* chunks per lane rounded up to a power of two */
static int router_nch(int H) {
    const int per = (H / 8 + 63) / 64;
    int p = 1;
    while (p < per) p <<= 1;
    return p;
}

#ifndef RT_WPB
#define RT_WPB 2
#endif
#define RT_DISPATCH(KERNEL, XB, NORM, NCH, GRID, ARGS)                                         \
    do {                                                                                       \
        const dim3 blk(64 * RT_WPB);                                                           \
        if (NCH == 1) hipLaunchKernelGGL((KERNEL<XB, NORM, 1>), GRID, blk, 0, st, ARGS);        \
        else if (NCH == 2) hipLaunchKernelGGL((KERNEL<XB, NORM, 2>), GRID, blk, 0, st, ARGS);   \
        else if (NCH == 4) hipLaunchKernelGGL((KERNEL<XB, NORM, 4>), GRID, blk, 0, st, ARGS);   \
        else if (NCH == 8) hipLaunchKernelGGL((KERNEL<XB, NORM, 8>), GRID, blk, 0, st, ARGS);   \
        else hipLaunchKernelGGL((KERNEL<XB, NORM, 16>), GRID, blk, 0, st, ARGS);                \
    } while (0)

#define RT_DISPATCH4(KERNEL, XBF, NRM, NCH, GRID, ARGS)                                         \
    do {                                                                                       \
        if (XBF) {                                                                             \
            if (NRM) RT_DISPATCH(KERNEL, true, true, NCH, GRID, ARGS);                          \
            else RT_DISPATCH(KERNEL, true, false, NCH, GRID, ARGS);                             \
        } else {                                                                               \
            if (NRM) RT_DISPATCH(KERNEL, false, true, NCH, GRID, ARGS);                         \
            else RT_DISPATCH(KERNEL, false, false, NCH, GRID, ARGS);                            \
        }                                                                                      \
    } while (0)

/*
 * One token: one workgroup of 4 waves per row (E+1 workgroups, 4(E+1)
 * waves: two or more per SIMD where a wave per row would leave half the
 * SIMDs idle).  Wave w runs the R64 chains of lanes 16w..16w+15 (its lanes
 * 16..63 repeat lanes 0..15 and are ignored), sums them over l^1..l^8 as
 * qk_group_sum<64> does, and the l^16, l^32 levels of the tree are added
 * from LDS in the same order: (S0 + S1) + (S2 + S3).  With NORM the sum of
 * squares takes the same route, every wave forms r and the normalised row
 * itself (router_rows' arithmetic), and row 0's workgroup writes xn.  The
 * logits are the bits of k_router's.
 */
template <bool XBF16, bool NORM, int NCH>
__global__ __launch_bounds__(256) void k_router_one(RouterArgs a) {
    const int row = blockIdx.x;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int vl = 16 * wave + (lane & 15);
    const int chunks = a.H >> 3;
    const uint16_t *wrow = row < a.E ? a.router_w + (size_t)row * a.H : a.sh_gate_w;
    __shared__ float s_g[2][4];
    /* the bias, loaded now: after the last barrier it would cost a load
     * round trip of its own */
    const bool has_bias = row < a.E && a.router_bias;
    const float bias = (threadIdx.x == 0 && has_bias) ? qk_ld(a.router_bias + row) : 0.0f;
    uint4 wv[NCH];
    bool cv[NCH];
    int cc[NCH];
#pragma unroll
    for (int i = 0; i < NCH; i++) {
        const int c = vl + 64 * i;
        cv[i] = c < chunks;
        cc[i] = cv[i] ? c : 0;
        wv[i] = qk_ld((const uint4 *)wrow + cc[i]);
    }
    float v[NCH][8];
#pragma unroll
    for (int i = 0; i < NCH; i++) load_x8<XBF16>(a.x, 0, cc[i], v[i]);
    if (NORM) {
        float ss = 0.0f;
#pragma unroll
        for (int i = 0; i < NCH; i++) {
            float s2 = ss;
#pragma unroll
            for (int j = 0; j < 8; j++) s2 = fmaf(v[i][j], v[i][j], s2);
            ss = cv[i] ? s2 : ss;
        }
        ss = qk_group_sum<16>(ss);
        if (lane == 0) s_g[0][wave] = ss;
        __syncthreads();
        ss = (s_g[0][0] + s_g[0][1]) + (s_g[0][2] + s_g[0][3]);
        const float r = 1.0f / sqrtf(ss / (float)a.H + a.eps);
#pragma unroll
        for (int i = 0; i < NCH; i++) {
            const float4 *nw = (const float4 *)a.norm_w + 2 * cc[i];
            const float4 w0 = qk_ld(nw), w1 = qk_ld(nw + 1);
            const float wn[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
            for (int j = 0; j < 8; j++) v[i][j] = (v[i][j] * r) * wn[j];
            if (row == 0 && a.xn && cv[i] && lane < 16) {
                float4 *o = (float4 *)a.xn + 2 * cc[i];
                o[0] = make_float4(v[i][0], v[i][1], v[i][2], v[i][3]);
                o[1] = make_float4(v[i][4], v[i][5], v[i][6], v[i][7]);
            }
        }
    }
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < NCH; i++) {
        const uint4 d = wv[i];
        float a2 = acc;
        a2 = fmaf(v[i][0], qk_bf16_lo(d.x), a2);
        a2 = fmaf(v[i][1], qk_bf16_hi(d.x), a2);
        a2 = fmaf(v[i][2], qk_bf16_lo(d.y), a2);
        a2 = fmaf(v[i][3], qk_bf16_hi(d.y), a2);
        a2 = fmaf(v[i][4], qk_bf16_lo(d.z), a2);
        a2 = fmaf(v[i][5], qk_bf16_hi(d.z), a2);
        a2 = fmaf(v[i][6], qk_bf16_lo(d.w), a2);
        a2 = fmaf(v[i][7], qk_bf16_hi(d.w), a2);
        acc = cv[i] ? a2 : acc;
    }
    acc = qk_group_sum<16>(acc);
    if (lane == 0) s_g[1][wave] = acc;
    __syncthreads();
    if (threadIdx.x == 0) {
        float l = (s_g[1][0] + s_g[1][1]) + (s_g[1][2] + s_g[1][3]);
        if (has_bias) l = l + bias;
        a.logits[row] = l;
    }
}

/* the tiled router is instantiated for H = 512 * NCH with NCH = 1, 2, 4
 * (hidden 1536 is a multiple of 512 but has no instance: it takes k_router) */
extern "C" int qk_router_packs(qk_shape s, int n) {
    return n >= RTT_MIN_N && (s.H == 512 || s.H == 1024 || s.H == 2048);
}

extern "C" int qk_launch_router_pack(const qmoe_layer_weights *W, qk_shape s, const void *x, int x_bf16,
                                     int n, float *logits, float *xn, uint16_t *phi, uint16_t *plo,
                                     float *pg, void *stream);

extern "C" int qk_launch_router(const qmoe_layer_weights *W, qk_shape s, const void *x, int x_bf16,
                                int n, float *logits, float *xn, void *stream) {
    return qk_launch_router_pack(W, s, x, x_bf16, n, logits, xn, nullptr, nullptr, nullptr, stream);
}

extern "C" int qk_launch_router_pack(const qmoe_layer_weights *W, qk_shape s, const void *x, int x_bf16,
                                     int n, float *logits, float *xn, uint16_t *phi, uint16_t *plo,
                                     float *pg, void *stream) {
    if (n <= 0) return 0;
    /* the planes come from the tiled router only; lo is there for f32 or normed input */
    if (phi && (!qk_router_packs(s, n) || !pg || (!plo && (!x_bf16 || W->norm_w))))
        return (int)hipErrorInvalidValue;
    RouterArgs a;
    a.router_w = W->router_w;
    a.router_bias = W->router_bias;
    a.sh_gate_w = W->sh_gate_w;
    a.norm_w = W->norm_w;
    a.x = x;
    a.logits = logits;
    a.xn = xn;
    a.phi = phi;
    a.plo = plo;
    a.pg = pg;
    a.H = s.H;
    a.E = s.E;
    a.n = n;
    a.eps = s.eps;
    hipStream_t st = (hipStream_t)stream;
    if (qk_router_packs(s, n)) {
        /* tiled: about two workgroups per CU, rows split into slices of whole stages */
        const int tblocks = (n + 4 * RTT_TOK - 1) / (4 * RTT_TOK);
        const int stages = (s.E + 1 + RTT_EB - 1) / RTT_EB;
        int slices = 512 / tblocks;
        slices = slices < 1 ? 1 : (slices > stages ? stages : slices);
        const int rows = (stages + slices - 1) / slices * RTT_EB;
        slices = (s.E + 1 + rows - 1) / rows;
        dim3 grid(tblocks, slices);
        const int nch = s.H / 512;
        const bool nrm = W->norm_w != nullptr;
#define RTT_L(XB, NR, NC) hipLaunchKernelGGL((k_router_tile<XB, NR, NC>), grid, dim3(256), 0, st, a, rows)
#define RTT_N(XB, NR) \
    do { if (nch == 1) RTT_L(XB, NR, 1); else if (nch == 2) RTT_L(XB, NR, 2); else RTT_L(XB, NR, 4); } while (0)
        if (x_bf16) {
            if (nrm) RTT_N(true, true);
            else RTT_N(true, false);
        } else {
            if (nrm) RTT_N(false, true);
            else RTT_N(false, false);
        }
#undef RTT_N
#undef RTT_L
        return QK_CHECK_LAUNCH();
    }
    if (n == 1 && router_nch(s.H) <= 4) {
        const int nch = router_nch(s.H);
        const bool nrm = W->norm_w != nullptr;
#define R1_L(XB, NR)                                                                                      \
    do {                                                                                                  \
        if (nch == 1) hipLaunchKernelGGL((k_router_one<XB, NR, 1>), dim3(s.E + 1), dim3(256), 0, st, a); \
        else if (nch == 2) hipLaunchKernelGGL((k_router_one<XB, NR, 2>), dim3(s.E + 1), dim3(256), 0, st, a); \
        else hipLaunchKernelGGL((k_router_one<XB, NR, 4>), dim3(s.E + 1), dim3(256), 0, st, a);          \
    } while (0)
        if (x_bf16) {
            if (nrm) R1_L(true, true);
            else R1_L(true, false);
        } else {
            if (nrm) R1_L(false, true);
            else R1_L(false, false);
        }
#undef R1_L
        return QK_CHECK_LAUNCH();
    }
    /* one wave per (row, block of RT_TB tokens); RT_WPB waves per workgroup
     * (few, so that a one-token router spreads over every CU) */
    dim3 grid((s.E + 1 + RT_WPB - 1) / RT_WPB, (n + RT_TB - 1) / RT_TB);
    const int nch = router_nch(s.H);
    RT_DISPATCH4(k_router, x_bf16, W->norm_w != nullptr, nch, grid, a);
    return QK_CHECK_LAUNCH();
}

/* ------------------------------------------------------------- top-k */

#include "topk_wave.h"

/* experts per lane for E experts: the power of two >= ceil(E/64) */
static int topk_pl(int E) {
    int pl = 1;
    while (pl * 64 < E) pl <<= 1;
    return pl;
}

#define TK_DISPATCH(KERNEL, PL, GRID, BLOCK, ARGS)                                              \
    do {                                                                                       \
        switch (PL) {                                                                          \
        case 1: hipLaunchKernelGGL(KERNEL<1>, GRID, BLOCK, 0, st, ARGS); break;                \
        case 2: hipLaunchKernelGGL(KERNEL<2>, GRID, BLOCK, 0, st, ARGS); break;                \
        case 4: hipLaunchKernelGGL(KERNEL<4>, GRID, BLOCK, 0, st, ARGS); break;                \
        case 8: hipLaunchKernelGGL(KERNEL<8>, GRID, BLOCK, 0, st, ARGS); break;                \
        default: hipLaunchKernelGGL(KERNEL<16>, GRID, BLOCK, 0, st, ARGS); break;              \
        }                                                                                      \
    } while (0)

struct TopkArgs {
    const float *logits; /* [n, E+1] */
    float *logits_out;   /* [n, E] or null */
    int32_t *idx;
    float *w;
    float *sg;
    int E, k, n;
};

template <int PL>
__device__ __forceinline__ void topk_token(const TopkArgs &a, int t, int lane, int32_t *lds_idx) {
    const float *row = a.logits + (size_t)t * (a.E + 1);
    int id;
    float wt;
    wave_topk<PL>(row, a.E, a.k, lane, id, wt);
    if (lane < a.k) {
        a.idx[(size_t)t * a.k + lane] = id;
        a.w[(size_t)t * a.k + lane] = wt;
        if (lds_idx) lds_idx[t * a.k + lane] = id;
    }
    if (lane == 0) a.sg[t] = qk_sigmoid(qk_ld(row + a.E));
    if (a.logits_out)
        for (int e = lane; e < a.E; e += 64) a.logits_out[(size_t)t * a.E + e] = row[e];
}

template <int PL>
__global__ __launch_bounds__(256) void k_topk(TopkArgs a) {
    const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= a.n) return;
    topk_token<PL>(a, t, threadIdx.x & 63, nullptr);
}

extern "C" int qk_launch_topk(qk_shape s, int n, const float *logits, float *logits_out,
                              int32_t *idx, float *w, float *sg, void *stream) {
    if (n <= 0) return 0;
    TopkArgs a{logits, logits_out, idx, w, sg, s.E, s.k, n};
    hipStream_t st = (hipStream_t)stream;
    TK_DISPATCH(k_topk, topk_pl(s.E), dim3((n + 3) / 4), dim3(256), a);
    return QK_CHECK_LAUNCH();
}

/* ------------------------------------------------------------ dispatch
 *
 * Deterministic stable counting sort of flat slots f = t*k + s by expert.
 * Membership bitmask B[e][t/32] bit t%32 is set for every (t, e) pair
 * (atomicOr is order-independent); a slot's rank inside its expert is the
 * popcount of B[e] below bit t, which is exactly the number of earlier
 * tokens that chose e.  So the result equals the oracle's sequential
 * counting sort with no ordering dependence on the hardware.
 *
 * Outputs: offsets [E+1], perm [n*k], pos [n*k] (inverse) and the segment
 * table segtab [1+3E] (count U, then (expert, offsets[e], count[e]) for the
 * U experts with tokens, ascending).
 */

/* block-wide exclusive scan of NT/64 waves, one int per thread */
template <int NT>
__device__ int block_exscan(int v, int *lds /* >= NT/64 ints */, int &total) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int inc = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        int u = __shfl_up(inc, o, QK_WAVE);
        if (lane >= o) inc += u;
    }
    if (lane == 63) lds[wave] = inc;
    __syncthreads();
    int wbase = 0, tot = 0;
    for (int i = 0; i < NT / 64; i++) {
        int s = lds[i];
        if (i < wave) wbase += s;
        tot += s;
    }
    __syncthreads();
    total = tot;
    return wbase + inc - v;
}

/* per-expert counts (cnt[j] for experts e = threadIdx.x*PER + j) ->
 * offsets and segtab; lds_off gets offsets when non-null; returns the
 * total count (in every thread) */
/* the segment table goes to segtab and, when s_seg is given, to that LDS
 * mirror (for the task lists built next by the same workgroup) */
template <int NT>
__device__ int counts_to_offsets(const int *cnt, int E, int *lds_scan, int32_t *offsets,
                                  int32_t *segtab, int *lds_off, int32_t *s_seg) {
    constexpr int PER = QK_MAX_EXPERTS / NT;
    int csum = 0, asum = 0;
#pragma unroll
    for (int j = 0; j < PER; j++) {
        const int e = threadIdx.x * PER + j;
        if (e < E) {
            csum += cnt[j];
            asum += cnt[j] > 0 ? 1 : 0;
        }
    }
    int total, ntot;
    int off = block_exscan<NT>(csum, lds_scan, total);
    int uoff = block_exscan<NT>(asum, lds_scan, ntot);
#pragma unroll
    for (int j = 0; j < PER; j++) {
        const int e = threadIdx.x * PER + j;
        if (e < E) {
            offsets[e] = off;
            if (lds_off) lds_off[e] = off;
            if (cnt[j] > 0) {
                segtab[1 + 3 * uoff] = e;
                segtab[2 + 3 * uoff] = off;
                segtab[3 + 3 * uoff] = cnt[j];
                if (s_seg) {
                    s_seg[1 + 3 * uoff] = e;
                    s_seg[2 + 3 * uoff] = off;
                    s_seg[3 + 3 * uoff] = cnt[j];
                }
                uoff++;
            }
            off += cnt[j];
        }
    }
    if (threadIdx.x == 0) {
        offsets[E] = total;
        segtab[0] = ntot;
        if (s_seg) s_seg[0] = ntot;
    }
    return total;
}

/* dispatch of n <= QK_SMALL_N tokens whose expert ids are in LDS (s_idx),
 * run by one NT-thread workgroup */
template <int NT>
__device__ void dispatch_block(const int32_t *s_idx, int n, int k, int E, int32_t *offsets,
                               int32_t *perm, int32_t *pos, int32_t *segtab, int32_t *s_seg) {
    __shared__ uint32_t s_bits[QK_MAX_EXPERTS * (QK_SMALL_N / 32)];
    __shared__ int32_t s_wpre[QK_MAX_EXPERTS * (QK_SMALL_N / 32)];
    __shared__ int32_t s_off[QK_MAX_EXPERTS];
    __shared__ int s_scan[NT / 64];
    constexpr int PER = QK_MAX_EXPERTS / NT;
    const int tid = threadIdx.x;
    const int NW = (n + 31) >> 5;
    for (int i = tid; i < E * NW; i += NT) s_bits[i] = 0u;
    __syncthreads();
    for (int f = tid; f < n * k; f += NT) {
        const int t = f / k, e = s_idx[f];
        if (e >= 0 && e < E) atomicOr(&s_bits[e * NW + (t >> 5)], 1u << (t & 31));
    }
    __syncthreads();
    int cnt[PER];
#pragma unroll
    for (int j = 0; j < PER; j++) {
        const int e = tid * PER + j;
        cnt[j] = 0;
        if (e < E)
            for (int wd = 0; wd < NW; wd++) {
                s_wpre[e * NW + wd] = cnt[j];
                cnt[j] += __popc(s_bits[e * NW + wd]);
            }
    }
    counts_to_offsets<NT>(cnt, E, s_scan, offsets, segtab, s_off, s_seg);
    __syncthreads();
    for (int f = tid; f < n * k; f += NT) {
        const int t = f / k, e = s_idx[f], wd = t >> 5;
        if (e < 0 || e >= E) {
            if (pos) pos[f] = -1;
            continue;
        }
        const int rank = s_wpre[e * NW + wd] + __popc(s_bits[e * NW + wd] & ((1u << (t & 31)) - 1u));
        const int p = s_off[e] + rank;
        perm[p] = f;
        if (pos) pos[f] = p;
    }
}

struct SmallDispArgs {
    TopkArgs tk;
    int32_t *offsets, *perm, *pos, *segtab;
    int min_m;            /* MFMA task list from the table, when tasks is set */
    int32_t *tasks, *small;
};

/*
 * One token, one wavefront: top-k, then its k distinct experts sorted
 * ascending are the segments, one slot each (rank = number of selected
 * experts with a lower id).  Offsets are written only when asked for.
 */
template <int PL>
__global__ __launch_bounds__(64) void k_topk_dispatch_one(SmallDispArgs a) {
    const int lane = threadIdx.x;
    const int k = a.tk.k, E = a.tk.E;
    const float *row = a.tk.logits;
    int id;
    float wt;
    wave_topk<PL>(row, E, k, lane, id, wt);
    const int my_id = lane < k ? id : 0x7FFFFFFF;
    int rank = 0;
    for (int s2 = 0; s2 < k; s2++) rank += __builtin_amdgcn_readlane(my_id, s2) < my_id ? 1 : 0;
    if (lane < k) {
        a.tk.idx[lane] = id;
        a.tk.w[lane] = wt;
        a.perm[rank] = lane;
        a.pos[lane] = rank;
        a.segtab[1 + 3 * rank] = id;
        a.segtab[2 + 3 * rank] = rank;
        a.segtab[3 + 3 * rank] = 1;
    }
    if (lane == 0) {
        a.segtab[0] = k;
        a.tk.sg[0] = qk_sigmoid(qk_ld(row + E));
    }
    if (a.tk.logits_out)
        for (int e = lane; e < E; e += 64) a.tk.logits_out[e] = row[e];
    if (a.offsets)
        for (int e = lane; e <= E; e += 64) {
            int c = 0;
            for (int s2 = 0; s2 < k; s2++) c += __builtin_amdgcn_readlane(my_id, s2) < e ? 1 : 0;
            a.offsets[e] = c;
        }
}

/* 2 <= n <= QK_SMALL_N, n*k <= QK_SMALL_NK: top-k (one wave per token) and
 * the whole dispatch in one 1024-thread workgroup */
template <int PL>
__global__ __launch_bounds__(1024) void k_topk_dispatch_small(SmallDispArgs a) {
    __shared__ int32_t s_idx[QK_SMALL_NK];
    __shared__ int32_t s_seg[1 + 3 * QK_MAX_EXPERTS]; /* the segment table, mirrored */
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int t = wave; t < a.tk.n; t += 16) topk_token<PL>(a.tk, t, lane, s_idx);
    __syncthreads();
    dispatch_block<1024>(s_idx, a.tk.n, a.tk.k, a.tk.E, a.offsets, a.perm, a.pos, a.segtab, s_seg);
    if (a.tasks) {
        __syncthreads(); /* the segment table, written by this workgroup */
        mm_tasks_block<true>(s_seg, a.tk.n, a.tk.k, a.tk.E, a.min_m, a.tasks, a.small);
    }
}

/* the same dispatch with the expert ids read from global memory (after a
 * separate k_topk launch, one wave per token over many workgroups) */
__global__ __launch_bounds__(1024) void k_dispatch_small(const int32_t *idx, int n, int k, int E,
                                                         int32_t *offsets, int32_t *perm,
                                                         int32_t *pos, int32_t *segtab, int min_m,
                                                         int32_t *tasks, int32_t *small) {
    __shared__ int32_t s_idx[QK_SMALL_NK];
    __shared__ int32_t s_seg[1 + 3 * QK_MAX_EXPERTS]; /* the segment table, mirrored */
    for (int f = threadIdx.x; f < n * k; f += 1024) s_idx[f] = qk_ld(idx + f);
    __syncthreads();
    dispatch_block<1024>(s_idx, n, k, E, offsets, perm, pos, segtab, s_seg);
    if (tasks) {
        __syncthreads();
        mm_tasks_block<true>(s_seg, n, k, E, min_m, tasks, small);
    }
}

/* tokens above which the top-k runs as its own launch (one wave per token)
 * rather than 16 waves of one workgroup taking turns */
#define QK_TOPK_SPLIT_N 16

extern "C" int qk_launch_topk_dispatch_small(qk_shape s, int n, const float *logits,
                                             float *logits_out, int32_t *idx, float *w, float *sg,
                                             int32_t *offsets, int32_t *perm, int32_t *pos,
                                             int32_t *segtab, int min_m, int32_t *tasks,
                                             void *stream) {
    if (n <= 0) return 0;
    if (n > QK_SMALL_N || n * s.k > QK_SMALL_NK) return (int)hipErrorInvalidValue;
    if (n == 1 && tasks) return (int)hipErrorInvalidValue;
    SmallDispArgs a{{logits, logits_out, idx, w, sg, s.E, s.k, n}, offsets, perm, pos, segtab,
                    min_m, tasks, tasks ? qk_mfma_small_list(s, n, tasks) : nullptr};
    hipStream_t st = (hipStream_t)stream;
    if (n == 1) {
        TK_DISPATCH(k_topk_dispatch_one, topk_pl(s.E), dim3(1), dim3(64), a);
    } else if (n <= QK_TOPK_SPLIT_N) {
        if (!offsets) return (int)hipErrorInvalidValue;
        TK_DISPATCH(k_topk_dispatch_small, topk_pl(s.E), dim3(1), dim3(1024), a);
    } else {
        if (!offsets) return (int)hipErrorInvalidValue;
        TK_DISPATCH(k_topk, topk_pl(s.E), dim3((n + 3) / 4), dim3(256), a.tk);
        hipLaunchKernelGGL(k_dispatch_small, dim3(1), dim3(1024), 0, st, (const int32_t *)idx, n, s.k,
                           s.E, offsets, perm, pos, segtab, min_m, tasks,
                           tasks ? qk_mfma_small_list(s, n, tasks) : nullptr);
    }
    return QK_CHECK_LAUNCH();
}

/* ---- multi-kernel dispatch (any n) ---- */

__global__ void k_fill_u32(uint32_t *p, size_t count, uint32_t v) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < count) p[i] = v;
}

/* ids outside [0, E) are skipped (their slots are not dispatched) */
__global__ void k_setbits(const int32_t *idx, int n, int k, int E, int NW, uint32_t *bits) {
    int f = blockIdx.x * blockDim.x + threadIdx.x;
    if (f >= n * k) return;
    int t = f / k, e = idx[f];
    if (e < 0 || e >= E) return;
    atomicOr(&bits[(size_t)e * NW + (t >> 5)], 1u << (t & 31));
}

/* per-expert word prefixes, one wave per expert; the expert's token count
 * goes to cnt[e] */
__global__ __launch_bounds__(1024) void k_word_prefix(const uint32_t *bits, int32_t *wprefix, int E,
                                                      int NW, int32_t *cnt) {
    const int lane = threadIdx.x & 63;
    const int e = blockIdx.x * 16 + (threadIdx.x >> 6);
    if (e >= E) return;
    int base = 0;
    for (int w0 = 0; w0 < NW; w0 += 64) {
        const int wd = w0 + lane;
        const int c = wd < NW ? __popc(bits[(size_t)e * NW + wd]) : 0;
        int inc = c;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int u = __shfl_up(inc, o, QK_WAVE);
            if (lane >= o) inc += u;
        }
        if (wd < NW) wprefix[(size_t)e * NW + wd] = base + inc - c;
        base += __shfl(inc, 63, QK_WAVE);
    }
    if (lane == 0) cnt[e] = base;
}

/* one workgroup: counts (held in `offsets` on entry) -> offsets and the
 * segment table; perm entries past the dispatched total (slots with invalid
 * expert ids) are set to -1 */
__global__ __launch_bounds__(1024) void k_count_offsets(int E, int32_t *offsets, int32_t *segtab,
                                                        int32_t *perm, int nk, int n, int k,
                                                        int min_m, int32_t *tasks, int32_t *small) {
    __shared__ int s_scan[16];
    __shared__ int32_t s_seg[1 + 3 * QK_MAX_EXPERTS]; /* the segment table, mirrored */
    const int tid = threadIdx.x;
    int cnt[1] = {tid < E ? offsets[tid] : 0};
    __syncthreads();
    const int total = counts_to_offsets<1024>(cnt, E, s_scan, offsets, segtab, nullptr, s_seg);
    for (int i = total + tid; i < nk; i += 1024) perm[i] = -1;
    if (tasks) {
        __syncthreads(); /* the segment table, written by this workgroup */
        mm_tasks_block<true>(s_seg, n, k, E, min_m, tasks, small);
    }
}

__global__ void k_scatter(const int32_t *idx, int n, int k, int E, int NW, const uint32_t *bits,
                          const int32_t *wprefix, const int32_t *offsets, int32_t *perm,
                          int32_t *pos) {
    int f = blockIdx.x * blockDim.x + threadIdx.x;
    if (f >= n * k) return;
    int t = f / k, e = idx[f], wd = t >> 5;
    if (e < 0 || e >= E) {
        if (pos) pos[f] = -1;
        return;
    }
    size_t b = (size_t)e * NW + wd;
    int p = offsets[e] + wprefix[b] + __popc(bits[b] & ((1u << (t & 31)) - 1u));
    perm[p] = f;
    if (pos) pos[f] = p;
}

extern "C" int qk_launch_dispatch(qk_shape s, int n, const int32_t *idx, int32_t *offsets,
                                  int32_t *perm, int32_t *pos, int32_t *segtab,
                                  uint32_t *bits, int bits_set, int32_t *wprefix, int min_m,
                                  int32_t *tasks, void *stream) {
    hipStream_t st = (hipStream_t)stream;
    if (n <= 0) return 0;
    const int NW = (n + 31) / 32;
    const size_t nb = (size_t)s.E * NW;
    const int nk = n * s.k;
    if (!bits_set) {
        hipLaunchKernelGGL(k_fill_u32, dim3((unsigned)((nb + 255) / 256)), dim3(256), 0, st, bits, nb, 0u);
        hipLaunchKernelGGL(k_setbits, dim3((nk + 255) / 256), dim3(256), 0, st, idx, n, s.k, s.E, NW,
                           bits);
    }
    hipLaunchKernelGGL(k_word_prefix, dim3((s.E + 15) / 16), dim3(1024), 0, st, (const uint32_t *)bits,
                       wprefix, s.E, NW, offsets);
    hipLaunchKernelGGL(k_count_offsets, dim3(1), dim3(1024), 0, st, s.E, offsets, segtab, perm, nk, n,
                       s.k, min_m, tasks, tasks ? qk_mfma_small_list(s, n, tasks) : nullptr);
    hipLaunchKernelGGL(k_scatter, dim3((nk + 255) / 256), dim3(256), 0, st, idx, n, s.k, s.E, NW,
                       (const uint32_t *)bits, (const int32_t *)wprefix, (const int32_t *)offsets,
                       perm, pos);
    return QK_CHECK_LAUNCH();
}

/* pos[perm[p]] = p; entries outside [0, count) are skipped */
__global__ void k_invert_perm(int count, const int32_t *perm, int32_t *pos) {
    int p = blockIdx.x * blockDim.x + threadIdx.x;
    if (p >= count) return;
    int f = perm[p];
    if (f >= 0 && f < count) pos[f] = p;
}

__global__ void k_fill_i32(int32_t *p, int count, int32_t v) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < count) p[i] = v;
}

extern "C" int qk_launch_invert_perm(int count, const int32_t *perm, int32_t *pos, void *stream) {
    if (count <= 0) return 0;
    hipLaunchKernelGGL(k_fill_i32, dim3((count + 255) / 256), dim3(256), 0, (hipStream_t)stream,
                       pos, count, -1);
    hipLaunchKernelGGL(k_invert_perm, dim3((count + 255) / 256), dim3(256), 0, (hipStream_t)stream,
                       count, perm, pos);
    return QK_CHECK_LAUNCH();
}

/* offsets[e] (e = 0..E) from a segment table whose experts ascend: the
 * first dispatch position of the first segment with expert >= e, or the
 * total count when there is none */
__global__ void k_offsets_from_segtab(const int32_t *segtab, int E, int32_t *offsets) {
    const int e = blockIdx.x * blockDim.x + threadIdx.x;
    if (e > E) return;
    const int U = min(max(segtab[0], 0), E);
    int lo = 0, hi = U; /* first segment index with expert >= e */
    while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (segtab[1 + 3 * mid] < e) lo = mid + 1;
        else hi = mid;
    }
    int v;
    if (lo < U) v = segtab[2 + 3 * lo];
    else v = U > 0 ? segtab[2 + 3 * (U - 1)] + segtab[3 + 3 * (U - 1)] : 0;
    offsets[e] = v;
}

extern "C" int qk_launch_offsets_from_segtab(qk_shape s, const int32_t *segtab, int32_t *offsets,
                                             void *stream) {
    hipLaunchKernelGGL(k_offsets_from_segtab, dim3((s.E + 1 + 255) / 256), dim3(256), 0,
                       (hipStream_t)stream, segtab, s.E, offsets);
    return QK_CHECK_LAUNCH();
}
