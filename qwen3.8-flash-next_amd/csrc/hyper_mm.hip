/*
 * hyper_mm.hip -- the MLP hyper connection's producer (gated_residual,
 * reference C port model.c:728-796) for many tokens, on bf16 MFMA
 * (v_mfma_f32_16x16x32_bf16), in four launches:
 *
 *   k_hc_pack    per token: the copies' RMS scales r_h = 1/sqrt(ss/d + eps)
 *                and a = x * hc_norm as MFMA operand planes (bf16 hi + lo,
 *                x = hi + lo to 2^-17, in (x_i, x_{i+4}) pair order per 8
 *                columns) with P_g = -128 * (sum of the group's 64 a);
 *   k_hc_mm_down partial products of the down projection over one K range
 *                of one copy h, sum_k a_k W[r, k], and of the inject
 *                projection (bf16 weights; none for the final mixer) as
 *                one more column block;
 *   k_hc_finish  per token: w = silu(sum_h r_h * partial_h / hc) (the norm
 *                scale is constant over a copy, so it applies after the
 *                product), inject = 2 sigmoid(sum_h r_h * partial_h / hc),
 *                and the planes of w;
 *   k_hc_mm_up   the up projection of w for the columns h*d + i of every
 *                copy h of a block of columns i, so each lane ends with all
 *                copies of its (row, i): mixed = mean_h sigmoid(up) *
 *                normed with normed = (x * r_h) * hc_norm formed there.
 *
 * q4 arithmetic as the expert MFMA kernels (ffn_mfma.hip): codes enter as
 * the bf16 numbers 128 + q, the accumulator of a group starts at P_g, so
 * the two K-steps of the group leave sum_k a_k q_k; then acc += s_g * that
 * + b_g * X_g with X_g = P_g / -128 (exact).  Operands are read straight
 * from the planes (L2-resident), one 16-byte load per lane and K-step.
 *
 * 16x16x32 lane layout: A lane l holds row l%16, B lane l column l%16; in
 * K-step j of a group lane quarter kq = l/16 holds the 8 columns of chunk
 * 2*kq + j (one code word).  D lane l holds column l%16, rows 4*kq + i.
 */
#include "qk_device.h"
#include "mfma_parts.h"

#define HC_MAX 8
#define HM_BM 64 /* rows per workgroup (4 waves x 16) */

/* one group's four MFMAs of A (hi, lo) x B, starting from c */
__device__ __forceinline__ qm_f32x4 hm_group(const uint4 (&A)[2][2], qm_bf16x8 b0, qm_bf16x8 b1,
                                             qm_f32x4 c) {
    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(qm_bf16x8, A[0][0]), b0, c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(qm_bf16x8, A[0][1]), b1, c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(qm_bf16x8, A[1][0]), b0, c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(qm_bf16x8, A[1][1]), b1, c, 0, 0, 0);
    return c;
}

/* ------------------------------------------------------------ down GEMM */

struct HcMmDownArgs {
    const float *hyper;       /* [n, D] */
    const float *norm_w;      /* [D] */
    const uint32_t *q;        /* input_mix_weight_down [R, D/8] */
    const uint16_t *s, *b;    /* [R, D/64] */
    const uint16_t *inject_w; /* [hc, D] bf16 */
    float *pd;                /* [n, R, parts] */
    float *pi;                /* [n, 16, parts] */
    float *pss;               /* [n, parts]: sum of x^2 over the part's columns */
    int hc, d, R, n, kspl;
};

#define HM_CS 10 /* LDS words per weight column and group (8 used; stride 10
                  * puts the 16 columns of a tile on distinct banks) */

/* the workgroup's weights of one group, staged through registers into LDS:
 * NC columns x 8 code words, their scales and biases */
template <int NC>
struct HmStage {
    static constexpr int NQ = (NC * 2 + 255) / 256; /* uint4 loads per thread */
    static constexpr int NS = (NC + 255) / 256;     /* scale/bias pairs per thread */
    uint4 q[NQ];
    uint16_t sv[NS], bv[NS];
};

template <int NC, typename ColFn>
__device__ __forceinline__ void hm_stage_load(HmStage<NC> &st, const uint32_t *q, const uint16_t *s,
                                              const uint16_t *b, size_t wrow, int G, int g, ColFn colf) {
#pragma unroll
    for (int k = 0; k < HmStage<NC>::NQ; k++) {
        const int i = threadIdx.x + 256 * k; /* (column, half) */
        const int cl = min(i >> 1, NC - 1);
        st.q[k] = qk_ld((const uint4 *)(q + colf(cl) * wrow + 8 * g) + (i & 1));
    }
#pragma unroll
    for (int k = 0; k < HmStage<NC>::NS; k++) {
        const int cl = min((int)threadIdx.x + 256 * k, NC - 1);
        st.sv[k] = qk_ld(s + colf(cl) * G + g);
        st.bv[k] = qk_ld(b + colf(cl) * G + g);
    }
}

template <int NC>
__device__ __forceinline__ void hm_stage_store(const HmStage<NC> &st, uint32_t *sq, float *ss, float *sb) {
#pragma unroll
    for (int k = 0; k < HmStage<NC>::NQ; k++) {
        const int i = threadIdx.x + 256 * k;
        if (i < 2 * NC) {
            uint2 *dst = (uint2 *)(sq + (i >> 1) * HM_CS + 4 * (i & 1));
            dst[0] = make_uint2(st.q[k].x, st.q[k].y);
            dst[1] = make_uint2(st.q[k].z, st.q[k].w);
        }
    }
#pragma unroll
    for (int k = 0; k < HmStage<NC>::NS; k++) {
        const int cl = threadIdx.x + 256 * k;
        if (cl < NC) {
            ss[cl] = qk_bf16(st.sv[k]);
            sb[cl] = qk_bf16(st.bv[k]);
        }
    }
}

/* lane's x and hc_norm for one group: row l%16, chunks 2*kq and 2*kq+1 */
struct HmXRaw {
    float4 x[4], w[4];
};

__device__ __forceinline__ void hm_load_x(HmXRaw &r, const float *xr, const float *nw, int g, int kq) {
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int col = g * 64 + 8 * (2 * kq + j);
        r.x[2 * j] = qk_ld((const float4 *)(xr + col));
        r.x[2 * j + 1] = qk_ld((const float4 *)(xr + col) + 1);
        r.w[2 * j] = qk_ld((const float4 *)(nw + col));
        r.w[2 * j + 1] = qk_ld((const float4 *)(nw + col) + 1);
    }
}

/*
 * grid = (ceil(n/64), passes, hc * kspl); wave = 16 rows x NT column tiles
 * of 16 (pass p: tiles p*NT ..), pass 0 also the inject tile.  The z index
 * is (copy h, K range ks of kspl) over the copy's d/64 groups.  Per group
 * the workgroup's NT*16 weight columns go through LDS (double-buffered, the
 * next group's loads in flight under this group's MFMAs), and each lane
 * forms its A operands from x itself: its 16 columns of a = x * hc_norm as
 * bf16 hi + lo pairs, the group sum over the row's four lane quarters
 * (l^16, l^32) and P = -128 * sum moved to the D layout (rows 4*kq + i) by
 * lane permutes; the A operands then serve every column tile.
 */
template <int NT>
__global__ __launch_bounds__(256) void k_hc_mm_down(HcMmDownArgs a) {
    constexpr int NC = NT * 16;
    __shared__ uint32_t s_q[2][NC * HM_CS];
    __shared__ float s_s[2][NC], s_b[2][NC];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int c = lane & 15, kq = lane >> 4;
    const int D = a.hc * a.d, G = D >> 6;
    const size_t wrow = (size_t)D >> 3;
    const int parts = a.hc * a.kspl;
    const int part = blockIdx.z, h = part / a.kspl, ks = part - h * a.kspl;
    const int gpc = a.d >> 6, gper = gpc / a.kspl;
    const int g0 = h * gpc + ks * gper;
    const int t0 = (int)blockIdx.y * NT; /* first column tile of this pass */
    const bool with_ss = blockIdx.y == 0;                /* pass 0: the copy's sum of squares */
    const bool with_inj = with_ss && a.inject_w != nullptr; /* and the inject tile */
    const int r0 = blockIdx.x * HM_BM + 16 * wave;
    const size_t arow = (size_t)min(r0 + c, a.n - 1);
    const float *xr = a.hyper + arow * D;
    auto colf = [&](int cl) { return (size_t)(t0 * 16 + cl); };
    qm_f32x4 acc[NT], acci = qm_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int ct = 0; ct < NT; ct++) acc[ct] = qm_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    const bool iok = c < a.hc;
    const uint16_t *wi = with_inj ? a.inject_w + (size_t)(iok ? c : 0) * D : nullptr;
    float ssp = 0.0f;

    HmStage<NC> stg;
    HmXRaw xraw;
    uint4 iw[2];
    auto load_inj = [&](int g) {
        const uint4 *src = (const uint4 *)(wi + (size_t)g * 64) + 2 * kq;
        iw[0] = qk_ld(src);
        iw[1] = qk_ld(src + 1);
    };
    hm_stage_load<NC>(stg, a.q, a.s, a.b, wrow, G, g0, colf);
    hm_load_x(xraw, xr, a.norm_w, g0, kq);
    if (with_inj) load_inj(g0);
    for (int g = g0; g < g0 + gper; g++) {
        const int buf = (g - g0) & 1;
        hm_stage_store<NC>(stg, s_q[buf], s_s[buf], s_b[buf]);
        /* A operands of this group from the raw x */
        uint4 A[2][2];
        float gs = 0.0f;
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const float xv[8] = {xraw.x[2 * j].x, xraw.x[2 * j].y, xraw.x[2 * j].z, xraw.x[2 * j].w,
                                 xraw.x[2 * j + 1].x, xraw.x[2 * j + 1].y, xraw.x[2 * j + 1].z,
                                 xraw.x[2 * j + 1].w};
            const float wv[8] = {xraw.w[2 * j].x, xraw.w[2 * j].y, xraw.w[2 * j].z, xraw.w[2 * j].w,
                                 xraw.w[2 * j + 1].x, xraw.w[2 * j + 1].y, xraw.w[2 * j + 1].z,
                                 xraw.w[2 * j + 1].w};
            float av[8];
#pragma unroll
            for (int i = 0; i < 8; i++) {
                ssp = fmaf(xv[i], xv[i], ssp);
                av[i] = xv[i] * wv[i];
            }
            uint32_t hi[4], lo[4];
            gs += qk_f32x8_pairs(av, hi, lo);
            A[0][j] = make_uint4(hi[0], hi[1], hi[2], hi[3]);
            A[1][j] = make_uint4(lo[0], lo[1], lo[2], lo[3]);
        }
        qm_bf16x8 ib0, ib1;
        if (with_inj) {
            uint32_t p0[4], p1[4];
            qk_bf16x8_to_pairs(iok ? iw[0] : make_uint4(0u, 0u, 0u, 0u), p0);
            qk_bf16x8_to_pairs(iok ? iw[1] : make_uint4(0u, 0u, 0u, 0u), p1);
            ib0 = __builtin_bit_cast(qm_bf16x8, make_uint4(p0[0], p0[1], p0[2], p0[3]));
            ib1 = __builtin_bit_cast(qm_bf16x8, make_uint4(p1[0], p1[1], p1[2], p1[3]));
        }
        /* the next group's loads go out under this group's MFMAs */
        if (g + 1 < g0 + gper) {
            hm_stage_load<NC>(stg, a.q, a.s, a.b, wrow, G, g + 1, colf);
            hm_load_x(xraw, xr, a.norm_w, g + 1, kq);
            if (with_inj) load_inj(g + 1);
        }
        gs += __uint_as_float(qk_xor16_u(__float_as_uint(gs)));
        gs += __uint_as_float(qk_xor32_u(__float_as_uint(gs)));
        const float pa = -128.0f * gs; /* row c's P (every quarter holds it) */
        qm_f32x4 p;
#pragma unroll
        for (int i = 0; i < 4; i++) p[i] = __shfl(pa, 4 * kq + i, QK_WAVE);
        __syncthreads(); /* stage of group g visible; buf of group g-1 free next time */
        const uint32_t *sq = s_q[buf];
#pragma unroll
        for (int ct = 0; ct < NT; ct++) {
            const int cl = ct * 16 + c;
            const uint2 wv = *(const uint2 *)(sq + cl * HM_CS + 2 * kq);
            const float sc = s_s[buf][cl], bi = s_b[buf][cl];
            const qm_f32x4 tq = hm_group(A, qm_codes(wv.x), qm_codes(wv.y), p);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                acc[ct][i] = fmaf(sc, tq[i], acc[ct][i]);
                acc[ct][i] = fmaf(bi, p[i] * (-1.0f / 128.0f), acc[ct][i]);
            }
        }
        if (with_inj) acci = hm_group(A, ib0, ib1, acci);
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int row = r0 + 4 * kq + i;
        if (row < a.n) {
            float *o = a.pd + ((size_t)row * a.R + t0 * 16 + c) * parts + part;
#pragma unroll
            for (int ct = 0; ct < NT; ct++) qk_st(o + (size_t)16 * ct * parts, acc[ct][i]);
            if (with_inj) qk_st(a.pi + ((size_t)row * 16 + c) * parts + part, acci[i]);
        }
    }
    if (with_ss) {
        ssp += __uint_as_float(qk_xor16_u(__float_as_uint(ssp)));
        ssp += __uint_as_float(qk_xor32_u(__float_as_uint(ssp)));
        if (kq == 0 && r0 + c < a.n) qk_st(a.pss + (size_t)(r0 + c) * parts + part, ssp);
    }
}

/* ---------------------------------------------------------------- finish */

struct HcFinishArgs {
    const float *pd, *pi, *pss; /* [n, R, parts], [n, 16, parts], [n, parts] */
    float *rs;         /* [n, hc] */
    uint4 *whi, *wlo;  /* [n, R/8] planes of w */
    float *wp;         /* [n, R/64] */
    float *inject;     /* [n, hc] */
    int hc, d, R, n, kspl;
    float eps;
};

/* sum_h r[h] * (sum of copy h's kspl parts) over the parts at p (copy-major,
 * kspl = 1 << lk, parts <= PM), every load issued before the sums */
template <int PM>
__device__ __forceinline__ float hm_parts_dot(const float *p, int parts, int lk, const float *r) {
    float pv[PM];
    if ((parts & 3) == 0) {
#pragma unroll
        for (int q4 = 0; q4 < PM / 4; q4++) {
            const float4 v = 4 * q4 < parts ? qk_ld((const float4 *)p + q4) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            pv[4 * q4] = v.x;
            pv[4 * q4 + 1] = v.y;
            pv[4 * q4 + 2] = v.z;
            pv[4 * q4 + 3] = v.w;
        }
    } else {
#pragma unroll
        for (int q = 0; q < PM; q++) pv[q] = q < parts ? qk_ld(p + q) : 0.0f;
    }
    const int km = (1 << lk) - 1;
    float v = 0.0f, ph = 0.0f;
#pragma unroll
    for (int q = 0; q < PM; q++) {
        if (q < parts) {
            ph += pv[q];
            if (((q + 1) & km) == 0) {
                v = fmaf(r[q >> lk], ph, v);
                ph = 0.0f;
            }
        }
    }
    return v;
}

/* grid = n, 512 threads: r_h, w = silu(sum_h r_h * partial_h / hc),
 * inject, and the MFMA planes of w; PM bounds the parts */
template <int PM>
__global__ __launch_bounds__(512) void k_hc_finish(HcFinishArgs a) {
    __shared__ float s_w[2048];
    __shared__ float s_r[HC_MAX];
    const int t = blockIdx.x, tid = threadIdx.x;
    const int parts = a.hc * a.kspl;
    const float inv_hc = 1.0f / (float)a.hc;
    const int lk = 31 - __builtin_clz(a.kspl);
    if (tid < a.hc) {
        float ss = 0.0f;
        for (int k = 0; k < a.kspl; k++) ss += a.pss[(size_t)t * parts + tid * a.kspl + k];
        const float r = 1.0f / sqrtf(ss / (float)a.d + a.eps);
        s_r[tid] = r;
        a.rs[(size_t)t * a.hc + tid] = r;
    }
    __syncthreads();
    for (int r = tid; r < a.R + 16; r += 512) {
        const bool isw = r < a.R;
        if (!isw && (r - a.R >= a.hc || !a.inject)) continue;
        const float *p = isw ? a.pd + ((size_t)t * a.R + r) * parts
                             : a.pi + ((size_t)t * 16 + (r - a.R)) * parts;
        const float v = hm_parts_dot<PM>(p, parts, lk, s_r);
        if (isw) s_w[r] = qk_silu(v * inv_hc);
        else a.inject[(size_t)t * a.hc + (r - a.R)] = 2.0f * qk_sigmoid(v * inv_hc);
    }
    __syncthreads();
    const int NCH = a.R >> 3;
    for (int ch = tid; ch < NCH; ch += 512) {
        /* NCH is a multiple of 8: a group's 8 chunks stay in one pass */
        float v[8];
#pragma unroll
        for (int i = 0; i < 8; i++) v[i] = s_w[8 * ch + i];
        uint32_t hi[4], lo[4];
        float g = qk_f32x8_pairs(v, hi, lo);
        a.whi[(size_t)t * NCH + ch] = make_uint4(hi[0], hi[1], hi[2], hi[3]);
        a.wlo[(size_t)t * NCH + ch] = make_uint4(lo[0], lo[1], lo[2], lo[3]);
        g += qk_dpp<QK_DPP_XOR1>(g);
        g += qk_dpp<QK_DPP_XOR2>(g);
        g += __shfl_xor(g, 4, QK_WAVE);
        if ((ch & 7) == 0) a.wp[(size_t)t * (a.R >> 6) + (ch >> 3)] = -128.0f * g;
    }
}

/* -------------------------------------------------------------- up GEMM */

struct HcMmUpArgs {
    const uint4 *whi, *wlo; /* [n, R/8] */
    const float *wp;        /* [n, R/64] */
    const uint32_t *q;      /* input_mix_weight_up [hc*d, R/8] */
    const uint16_t *s, *b;  /* [hc*d, R/64] */
    const float *hyper;     /* [n, hc*d] */
    const float *norm_w;    /* [hc*d] */
    const float *rs;        /* [n, hc] */
    float *mixed;           /* [n, d] */
    int d, R, n;
};

/* grid = (ceil(n/64), d/(16*HU_NB)): wave = 16 rows x HU_NB blocks of 16
 * columns i, each for every copy (HC column tiles h*d + i); the
 * workgroup's HC*16*HU_NB weight columns of a group go through LDS as in
 * the down GEMM */
template <int HC, int HU_NB>
__global__ __launch_bounds__(256) void k_hc_mm_up(HcMmUpArgs a) {
    constexpr int NC = HC * 16 * HU_NB;
    __shared__ uint32_t s_q[2][NC * HM_CS];
    __shared__ float s_s[2][NC], s_b[2][NC];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int c = lane & 15, kq = lane >> 4;
    const int NCH = a.R >> 3, G = a.R >> 6;
    const int D = HC * a.d;
    const int r0 = blockIdx.x * HM_BM + 16 * wave;
    const int i0 = blockIdx.y * (16 * HU_NB);
    const size_t arow = (size_t)min(r0 + c, a.n - 1);
    int prow[4];
#pragma unroll
    for (int i = 0; i < 4; i++) prow[i] = min(r0 + 4 * kq + i, a.n - 1);
    /* staged column cl = (h, i-offset): h = cl / 64, column h*d + i0 + cl % 64 */
    auto colf = [&](int cl) { return (size_t)(cl / (16 * HU_NB)) * a.d + i0 + cl % (16 * HU_NB); };
    qm_f32x4 acc[HU_NB][HC];
#pragma unroll
    for (int nb = 0; nb < HU_NB; nb++)
#pragma unroll
        for (int h = 0; h < HC; h++) acc[nb][h] = qm_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    HmStage<NC> stg;
    uint4 A[2][2];
    qm_f32x4 p;
    auto load_a = [&](int g) {
        const size_t base = arow * NCH + (size_t)g * 8 + 2 * kq;
        A[0][0] = qk_ld(a.whi + base);
        A[0][1] = qk_ld(a.whi + base + 1);
        A[1][0] = qk_ld(a.wlo + base);
        A[1][1] = qk_ld(a.wlo + base + 1);
#pragma unroll
        for (int i = 0; i < 4; i++) p[i] = qk_ld(a.wp + (size_t)prow[i] * G + g);
    };
    hm_stage_load<NC>(stg, a.q, a.s, a.b, (size_t)NCH, G, 0, colf);
    load_a(0);
    for (int g = 0; g < G; g++) {
        const int buf = g & 1;
        hm_stage_store<NC>(stg, s_q[buf], s_s[buf], s_b[buf]);
        const uint4 Ac[2][2] = {{A[0][0], A[0][1]}, {A[1][0], A[1][1]}};
        const qm_f32x4 pc = p;
        if (g + 1 < G) {
            hm_stage_load<NC>(stg, a.q, a.s, a.b, (size_t)NCH, G, g + 1, colf);
            load_a(g + 1);
        }
        __syncthreads();
        const uint32_t *sq = s_q[buf];
#pragma unroll
        for (int nb = 0; nb < HU_NB; nb++)
#pragma unroll
            for (int h = 0; h < HC; h++) {
                const int cl = h * 16 * HU_NB + 16 * nb + c;
                const uint2 wv = *(const uint2 *)(sq + cl * HM_CS + 2 * kq);
                const float sc = s_s[buf][cl], bi = s_b[buf][cl];
                const qm_f32x4 tq = hm_group(Ac, qm_codes(wv.x), qm_codes(wv.y), pc);
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    acc[nb][h][i] = fmaf(sc, tq[i], acc[nb][h][i]);
                    acc[nb][h][i] = fmaf(bi, pc[i] * (-1.0f / 128.0f), acc[nb][h][i]);
                }
            }
    }
    /* mixed[row, i] = (sum over h in order of fma(gate, normed, m)) / hc */
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int row = r0 + 4 * kq + i;
        if (row >= a.n) continue;
        float rr[HC];
#pragma unroll
        for (int h = 0; h < HC; h++) rr[h] = qk_ld(a.rs + (size_t)row * HC + h);
#pragma unroll
        for (int nb = 0; nb < HU_NB; nb++) {
            const int ic = i0 + 16 * nb + c;
            float m = 0.0f;
#pragma unroll
            for (int h = 0; h < HC; h++) {
                const size_t col = (size_t)h * a.d + ic;
                const float nv = qk_ld(a.hyper + (size_t)row * D + col) * rr[h] * qk_ld(a.norm_w + col);
                m = fmaf(qk_sigmoid(acc[nb][h][i]), nv, m);
            }
            qk_st(a.mixed + (size_t)row * a.d + ic, m / (float)HC);
        }
    }
}

/* normed [n, hc*d] = (x * r_h) * hc_norm, for callers that ask for it */
__global__ __launch_bounds__(256) void k_hc_normed(const float *hyper, const float *norm_w,
                                                   const float *rs, int hc, int d, float *normed) {
    const int t = blockIdx.x;
    const int D = hc * d;
    for (int i = threadIdx.x; i < D; i += 256)
        normed[(size_t)t * D + i] = hyper[(size_t)t * D + i] * rs[(size_t)t * hc + i / d] * norm_w[i];
}

/* ---------------------------------------------------------------- launch */

/* column tiles per pass of the down GEMM: few tokens take narrow passes
 * (more workgroups), many take wide ones (x converted fewer times, at most
 * 10 tiles for two waves per SIMD) */
static int hc_down_nt(int R, int n) {
    const int tiles = R / 16;
    if (n > 256 && tiles % 10 == 0) return 10;
    return tiles % 8 == 0 && n > 256 ? 8 : 4;
}

extern "C" int qk_hc_mm_kspl(int hc, int d, int R, int n) {
    /* split each copy's K range until the down GEMM has ~256 workgroups
     * (k_hc_finish reduces the parts): at most 8, a divisor of the copy's
     * groups, and kspl * n <= 1024 once split (bounds the workspace) */
    const int gpc = d / 64;
    const long long base =
        (long long)((n + HM_BM - 1) / HM_BM) * hc * (R / 16 / hc_down_nt(R, n));
    int k = 1;
    while (k < 8 && base * k < 256 && gpc % (2 * k) == 0 && (long long)n * 2 * k <= 1024) k *= 2;
    return k;
}

template <int NB>
static void hc_launch_up(int hc, dim3 grid, hipStream_t st, const HcMmUpArgs &ua) {
    switch (hc) {
    case 1: hipLaunchKernelGGL((k_hc_mm_up<1, NB>), grid, dim3(256), 0, st, ua); break;
    case 2: hipLaunchKernelGGL((k_hc_mm_up<2, NB>), grid, dim3(256), 0, st, ua); break;
    case 3: hipLaunchKernelGGL((k_hc_mm_up<3, NB>), grid, dim3(256), 0, st, ua); break;
    case 4: hipLaunchKernelGGL((k_hc_mm_up<4, NB>), grid, dim3(256), 0, st, ua); break;
    case 5: hipLaunchKernelGGL((k_hc_mm_up<5, NB>), grid, dim3(256), 0, st, ua); break;
    case 6: hipLaunchKernelGGL((k_hc_mm_up<6, NB>), grid, dim3(256), 0, st, ua); break;
    case 7: hipLaunchKernelGGL((k_hc_mm_up<7, NB>), grid, dim3(256), 0, st, ua); break;
    default: hipLaunchKernelGGL((k_hc_mm_up<8, NB>), grid, dim3(256), 0, st, ua); break;
    }
}

extern "C" int qk_launch_hc_mm(const float *hyper, const float *norm_w, const uint32_t *dq,
                               const uint16_t *ds, const uint16_t *db, const uint32_t *uq,
                               const uint16_t *us, const uint16_t *ub, const uint16_t *inject_w,
                               int hc, int d, int R, int n, float eps, void *ws, float *mixed,
                               float *inject, float *normed, void *stream) {
    if (n <= 0) return 0;
    if (hc < 1 || hc > HC_MAX || d % 64 || R % 64 || R > 2048) return (int)hipErrorInvalidValue;
    if (inject_w && !inject) return (int)hipErrorInvalidValue;
    hipStream_t st = (hipStream_t)stream;
    const int kspl = qk_hc_mm_kspl(hc, d, R, n), parts = hc * kspl;
    /* workspace carve-up (qk_hc_mm_ws_bytes) */
    char *p = (char *)ws;
    auto take = [&](size_t bytes) {
        char *r = p;
        p += (bytes + 255) & ~(size_t)255;
        return (void *)r;
    };
    float *pd = (float *)take((size_t)parts * n * R * 4);
    float *pi = (float *)take((size_t)parts * n * 16 * 4);
    float *pss = (float *)take((size_t)parts * n * 4);
    float *rs = (float *)take((size_t)n * hc * 4);
    uint4 *whi = (uint4 *)take((size_t)n * R * 2), *wlo = (uint4 *)take((size_t)n * R * 2);
    float *wp = (float *)take((size_t)n * (R / 64) * 4);
    const unsigned nrb = (unsigned)((n + HM_BM - 1) / HM_BM);
    const int nt = hc_down_nt(R, n), passes = R / 16 / nt;
    HcMmDownArgs da{hyper, norm_w, dq, ds, db, inject_w, pd, pi, pss, hc, d, R, n, kspl};
    const dim3 gd(nrb, passes, parts);
    if (nt == 10) hipLaunchKernelGGL(k_hc_mm_down<10>, gd, dim3(256), 0, st, da);
    else if (nt == 8) hipLaunchKernelGGL(k_hc_mm_down<8>, gd, dim3(256), 0, st, da);
    else hipLaunchKernelGGL(k_hc_mm_down<4>, gd, dim3(256), 0, st, da);
    HcFinishArgs fa{pd, pi, pss, rs, whi, wlo, wp, inject_w ? inject : nullptr, hc, d, R, n, kspl, eps};
    if (parts <= 4) hipLaunchKernelGGL(k_hc_finish<4>, dim3(n), dim3(512), 0, st, fa);
    else if (parts <= 8) hipLaunchKernelGGL(k_hc_finish<8>, dim3(n), dim3(512), 0, st, fa);
    else if (parts <= 16) hipLaunchKernelGGL(k_hc_finish<16>, dim3(n), dim3(512), 0, st, fa);
    else if (parts <= 32) hipLaunchKernelGGL(k_hc_finish<32>, dim3(n), dim3(512), 0, st, fa);
    else hipLaunchKernelGGL(k_hc_finish<64>, dim3(n), dim3(512), 0, st, fa);
    HcMmUpArgs ua{whi, wlo, wp, uq, us, ub, hyper, norm_w, rs, mixed, d, R, n};
    /* few tokens: one block of 16 columns per workgroup (4x the workgroups) */
    if (n <= 256) hc_launch_up<1>(hc, dim3(nrb, d / 16), st, ua);
    else hc_launch_up<4>(hc, dim3(nrb, d / 64), st, ua);
    if (normed) hipLaunchKernelGGL(k_hc_normed, dim3(n), dim3(256), 0, st, hyper, norm_w, rs, hc, d, normed);
    return QK_CHECK_LAUNCH();
}

extern "C" size_t qk_hc_mm_ws_bytes(int hc, int d, int R, int max_n) {
    /* the largest carve-up over n <= max_n: every term grows with n except
     * the parts, whose count times n is at most hc * max(n, 1024) */
    const size_t n = (size_t)max_n;
    const size_t pn = (size_t)hc * (n > 1024 ? n : 1024);
    auto up = [](size_t b) { return (b + 255) & ~(size_t)255; };
    return up(pn * R * 4) + up(pn * 16 * 4) + up(pn * 4) + up(n * hc * 4) + 2 * up(n * R * 2) +
           up(n * (R / 64) * 4) + 256;
}
