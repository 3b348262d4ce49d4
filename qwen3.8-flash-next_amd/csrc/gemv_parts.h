/*
 * gemv_parts.h -- the pieces of the q4 GEMV kernels: activation chunks
 * (32 columns per lane) loaded raw, turned into bf16 pairs (hi, and lo for
 * f32 input: x = hi + lo to 16 significant bits) with chunk sums, and the
 * per-lane share of an output row
 *     s * (sum_k x_k (128 + q_k) - 128 * sum_k x_k) + b * sum_k x_k
 * summed over the lane's chunks (the per-group identity of gemm_q4,
 * c/src/kernel.c:279-282, with codes as the bf16 values 128 + q).
 */
#ifndef GEMV_PARTS_H
#define GEMV_PARTS_H

#include "qk_device.h"

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
#pragma unroll
                for (int i = 0; i < 4; i++) xp.xs[ps] = qk_dot2(xp.hi[ps][4 * w + i], QK_BF16_ONES, xp.xs[ps]);
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

/*
 * f32 activations shared by the RPW = 64/LPR lanes that use one chunk (one
 * chunk per lane, RPW = 2 or 4): lane (sub, rsub) loads and converts NG =
 * 4/RPW of the chunk's four 8-column groups, the wave exchanges pairs and
 * group sums through LDS (36 words per chunk: 16 hi, 16 lo, 4 sums), and
 * every lane ends with exactly what convert_xraw gives for its chunk.
 */
template <int NG>
struct XShare {
    float4 f[2 * NG];
};

template <int NG>
__device__ __forceinline__ void load_xshare(const float *x, size_t row, int K, int sub, int rsub,
                                            XShare<NG> &xq) {
    const int CH = K >> 5;
    const int c = sub < CH ? sub : 0;
    const float4 *src = (const float4 *)(x + row * K) + 8 * c + 2 * NG * rsub;
#pragma unroll
    for (int i = 0; i < 2 * NG; i++) xq.f[i] = qk_ld(src + i);
}

/* LDS written by other lanes of this wave: order the accesses (a wave's LDS
 * operations complete in issue order, so no hardware wait is needed) */
__device__ __forceinline__ void qk_wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

template <int LPR, int NG>
__device__ __forceinline__ void convert_xshare(const XShare<NG> &xq, int K, int sub, int rsub,
                                               uint32_t *wbuf, XPairs<LPR, 1, false> &xp) {
    const int CH = K >> 5;
    const bool ok = sub < CH;
    uint32_t *cb = wbuf + 36 * sub;
#pragma unroll
    for (int gi = 0; gi < NG; gi++) {
        const int g = NG * rsub + gi;
        const float4 a0 = xq.f[2 * gi], a1 = xq.f[2 * gi + 1];
        float v[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
        if (!ok)
#pragma unroll
            for (int j = 0; j < 8; j++) v[j] = 0.0f;
        uint32_t hi[4], lo[4];
        const float gs = qk_f32x8_pairs(v, hi, lo);
        *(uint4 *)(cb + 4 * g) = make_uint4(hi[0], hi[1], hi[2], hi[3]);
        *(uint4 *)(cb + 16 + 4 * g) = make_uint4(lo[0], lo[1], lo[2], lo[3]);
        ((float *)cb)[32 + g] = gs;
    }
    qk_wave_lds_sync();
#pragma unroll
    for (int w = 0; w < 4; w++) {
        const uint4 h = *(const uint4 *)(cb + 4 * w), l = *(const uint4 *)(cb + 16 + 4 * w);
        xp.hi[0][4 * w] = h.x;
        xp.hi[0][4 * w + 1] = h.y;
        xp.hi[0][4 * w + 2] = h.z;
        xp.hi[0][4 * w + 3] = h.w;
        xp.lo[0][4 * w] = l.x;
        xp.lo[0][4 * w + 1] = l.y;
        xp.lo[0][4 * w + 2] = l.z;
        xp.lo[0][4 * w + 3] = l.w;
    }
    const float4 gsv = *(const float4 *)(cb + 32);
    xp.xs[0] = (((0.0f + gsv.x) + gsv.y) + gsv.z) + gsv.w;
    qk_wave_lds_sync();
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

/* this lane's share of one output row: sum over its chunks of the group
 * update s*(D - 128*xs) + b*xs (a group is two chunks; the lanes of a row
 * are summed by qk_group_sum afterwards) */
template <int LPR, int P, bool XBF16>
__device__ __forceinline__ float row_part(const uint4 (&wq)[P], const float (&ws)[P],
                                          const float (&wb)[P], const XPairs<LPR, P, XBF16> &xp) {
    float part = 0.0f;
#pragma unroll
    for (int ps = 0; ps < P; ps++) {
        const float d = chunk_dot<LPR, P, XBF16>(wq[ps], xp, ps);
        const float dq = fmaf(-128.0f, xp.xs[ps], d);
        part = fmaf(ws[ps], dq, fmaf(wb[ps], xp.xs[ps], part));
    }
    return part;
}

#endif
