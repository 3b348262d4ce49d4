/*
 * router_rows.h -- one router row (one wavefront) for a block of tokens,
 * shared by the router kernels (router.hip, route_mfma.hip).
 *
 * Router reduction order ("R64", bit-exact with the oracle): for one
 * (token, expert) dot product the K axis is cut into 8-element chunks, chunk
 * c goes to lane c%64 of a wavefront, each lane runs an fma chain over its
 * chunks in ascending order starting at +0.0f, and the wave combines its
 * lanes with the pairwise tree of qk_group_sum<64> (partners l^1 ... l^32).
 */
#ifndef ROUTER_ROWS_H
#define ROUTER_ROWS_H

#include "qk_device.h"

/* ------------------------------------------------------------ logits */

struct RouterArgs {
    const uint16_t *router_w;
    const float *router_bias;
    const uint16_t *sh_gate_w;
    const float *norm_w;
    const void *x;
    float *logits; /* [n, E+1] */
    float *xn;     /* [n, H] or null */
    uint16_t *phi, *plo; /* k_router_tile, or null: the MFMA gate/up operand planes of the */
    float *pg;           /* experts' input ([n, H] each, lo null for bf16) and P [n, H/64] */
    int H, E, n;
    float eps;
};

/* load the 8 activations of chunk c of a token row as f32 */
template <bool XBF16>
__device__ __forceinline__ void load_x8(const void *x, size_t row_off, int c, float v[8]) {
    if (XBF16) {
        uint4 d = qk_ld((const uint4 *)((const uint16_t *)x + row_off) + c);
        v[0] = qk_bf16_lo(d.x); v[1] = qk_bf16_hi(d.x);
        v[2] = qk_bf16_lo(d.y); v[3] = qk_bf16_hi(d.y);
        v[4] = qk_bf16_lo(d.z); v[5] = qk_bf16_hi(d.z);
        v[6] = qk_bf16_lo(d.w); v[7] = qk_bf16_hi(d.w);
    } else {
        const float4 *p = (const float4 *)((const float *)x + row_off) + 2 * c;
        float4 a = qk_ld(p), b = qk_ld(p + 1);
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
        v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    }
}

#define RT_TB 8 /* tokens per wave */

/*
 * One wavefront per (row, token block); NCH = chunks per lane (a power of
 * two >= ceil(H/512)).  Rows 0..E-1 are the router, row E is the
 * shared-expert gate.  Lanes whose chunk lies past the row load a valid
 * address and keep their partial unchanged (a select, not a branch), so
 * all loads issue back to back.  With NORM, every wave RMS-normalises its
 * tokens itself (R64 sum of squares, r = 1/sqrt(ss/H + eps), (x*r)*w as
 * kernel.c:10-20) and the wave of row 0 writes the normalised rows.
 * Returns the last token's logit (complete in lane 0).
 */
template <bool XBF16, bool NORM, int NCH>
__device__ __forceinline__ float router_rows(const RouterArgs &a, int row, int t0, int t1) {
    const int lane = threadIdx.x & 63;
    const int chunks = a.H >> 3;
    const uint16_t *wrow = row < a.E ? a.router_w + (size_t)row * a.H : a.sh_gate_w;
    uint4 wv[NCH];
    bool cv[NCH];
    int cc[NCH];
#pragma unroll
    for (int i = 0; i < NCH; i++) {
        const int c = lane + 64 * i;
        cv[i] = c < chunks;
        cc[i] = cv[i] ? c : 0;
        wv[i] = qk_ld((const uint4 *)wrow + cc[i]);
    }
    const float bias = (row < a.E && a.router_bias) ? a.router_bias[row] : 0.0f;
    float last = 0.0f;
    for (int t = t0; t < t1; t++) {
        const size_t roff = (size_t)t * a.H;
        float v[NCH][8];
#pragma unroll
        for (int i = 0; i < NCH; i++) load_x8<XBF16>(a.x, roff, cc[i], v[i]);
        if (NORM) {
            float ss = 0.0f;
#pragma unroll
            for (int i = 0; i < NCH; i++) {
                float s2 = ss;
#pragma unroll
                for (int j = 0; j < 8; j++) s2 = fmaf(v[i][j], v[i][j], s2);
                ss = cv[i] ? s2 : ss;
            }
            ss = qk_group_sum<64>(ss);
            const float r = 1.0f / sqrtf(ss / (float)a.H + a.eps);
#pragma unroll
            for (int i = 0; i < NCH; i++) {
                const float4 *nw = (const float4 *)a.norm_w + 2 * cc[i];
                const float4 w0 = qk_ld(nw), w1 = qk_ld(nw + 1);
                const float wn[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
                for (int j = 0; j < 8; j++) v[i][j] = (v[i][j] * r) * wn[j];
                if (row == 0 && a.xn && cv[i]) {
                    float4 *o = (float4 *)(a.xn + roff) + 2 * cc[i];
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
        acc = qk_group_sum<64>(acc);
        if (lane == 0) {
            if (row < a.E && a.router_bias) acc = acc + bias;
            a.logits[(size_t)t * (a.E + 1) + row] = acc;
        }
        last = acc;
    }
    return last; /* the logit of token t1-1 (lane 0 adds the bias) */
}

#endif
