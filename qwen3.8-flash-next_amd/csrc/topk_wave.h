/*
 * topk_wave.h -- top-k of one logit row by one wavefront (gfx950), shared
 * by the router kernels and the one-token gate/up kernel.
 */
#ifndef TOPK_WAVE_H
#define TOPK_WAVE_H

#include "qk_device.h"

/* order-preserving map f32 -> u32; -0 is first made +0 so it ties with +0 */
__device__ __forceinline__ uint32_t qk_ordkey(float v) {
    uint32_t b = __float_as_uint(v + 0.0f);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float qk_ordkey_value(uint32_t o) {
    return __uint_as_float((o & 0x80000000u) ? (o & 0x7FFFFFFFu) : ~o);
}

/*
 * One wavefront selects the top k of row[0..E) in canonical order: value
 * descending, ties to the lower expert id, -0 equal to +0.  Lane l holds
 * the PL experts e = l*PL + i (E <= 64*PL) and sorts them descending with
 * an odd-even transposition network; it swaps neighbours only on strict
 * inequality, so equal keys keep ascending e.  Then one round per slot: the
 * wave maximum of the lane heads; the lowest lane holding it wins (lane
 * order is e order, so that is the lowest e among equal keys) and pops its
 * head.  Round s yields slot s.  Padding entries (e >= E) carry key 0 and
 * valid keys are at least 1, so padding is never chosen while E >= k.
 *
 * The state is resumable, so a caller may act on slot s (start loads for
 * its expert) before running the remaining rounds.
 */
template <int PL>
struct WaveTopk {
    static_assert(PL <= 16, "at most 16 experts per lane");
    uint32_t kk[PL];     /* this lane's remaining keys, descending */
    uint32_t pk0, pk1;   /* their local indices, 4 bits each (entries past 8 in pk1) */

    __device__ __forceinline__ void init(const float *row, int E, int lane) {
        float lv[PL];
        if (PL % 4 == 0 && E % PL == 0) {
            /* whole float4s; lanes past the row read its last PL values (unused) */
            const int e0 = min(lane * PL, E - PL);
#pragma unroll
            for (int i = 0; i < PL; i += 4) {
                const float4 q = qk_ld((const float4 *)(row + e0 + i));
                lv[i] = q.x;
                lv[(i + 1) % PL] = q.y;
                lv[(i + 2) % PL] = q.z;
                lv[(i + 3) % PL] = q.w;
            }
        } else {
#pragma unroll
            for (int i = 0; i < PL; i++) {
                const int e = lane * PL + i;
                lv[i] = qk_ld(row + (e < E ? e : E - 1));
            }
        }
        init_vals(lv, E, lane);
    }

    /* the same from values already loaded: lv[i] = row[lane*PL + i] (any
     * value where that index is past E) */
    __device__ __forceinline__ void init_vals(const float (&lv)[PL], int E, int lane) {
        int ii[PL]; /* local index i of each sorted entry */
#pragma unroll
        for (int i = 0; i < PL; i++) {
            const int e = lane * PL + i;
            kk[i] = e < E ? max(qk_ordkey(lv[i]), 1u) : 0u;
            ii[i] = i;
        }
#pragma unroll
        for (int pass = 0; pass < PL; pass++) {
#pragma unroll
            for (int i = pass & 1; i + 1 < PL; i += 2) {
                const bool sw = kk[i + 1] > kk[i];
                const uint32_t ka = kk[i], kb = kk[i + 1];
                const int ia = ii[i], ib = ii[i + 1];
                kk[i] = sw ? kb : ka;
                kk[i + 1] = sw ? ka : kb;
                ii[i] = sw ? ib : ia;
                ii[i + 1] = sw ? ia : ib;
            }
        }
        pk0 = 0u;
        pk1 = 0u;
#pragma unroll
        for (int i = 0; i < PL; i++) {
            if (i < 8) pk0 |= (uint32_t)ii[i] << (4 * i);
            else pk1 |= (uint32_t)ii[i] << (4 * (i - 8));
        }
    }

    /* one round: the next slot's key and expert (wave-uniform) */
    __device__ __forceinline__ void next(int lane, uint32_t &key, int &e) {
        const uint32_t m = qk_wave_max_u32(kk[0]);
        const uint64_t ball = __ballot(kk[0] == m);
        const int wl = (int)__builtin_ctzll(ball);
        e = wl * PL + (int)(__builtin_amdgcn_readlane((int)pk0, wl) & 15u);
        key = m;
        if (lane == wl) {
#pragma unroll
            for (int i = 0; i + 1 < PL; i++) kk[i] = kk[i + 1];
            kk[PL - 1] = 0u;
            if (PL > 8) {
                pk0 = (pk0 >> 4) | (pk1 << 28);
                pk1 >>= 4;
            } else {
                pk0 >>= 4;
            }
        }
    }
};

/*
 * Softmax over the selected: lane s < k holds slot s's key and gets
 * w_s = exp(v_s - v_0) / sum_j exp(v_j - v_0), summed in slot order
 * (model.c:1305-1318).
 */
__device__ __forceinline__ float topk_weight(uint32_t my_key, int k, int lane) {
    const float v = qk_ordkey_value(my_key);
    const float v0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float ev = lane < k ? expf(v - v0) : 0.0f;
    float sum = 0.0f;
    for (int j = 0; j < k; j++) sum += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ev), j));
    return ev / sum;
}

/* the whole selection: lane s < k gets slot s's expert and weight */
template <int PL>
__device__ __forceinline__ void wave_topk(const float *row, int E, int k, int lane, int &my_id,
                                          float &my_w) {
    WaveTopk<PL> st;
    st.init(row, E, lane);
    uint32_t my_key = 0u;
    my_id = 0;
    for (int r = 0; r < k; r++) {
        uint32_t m;
        int e;
        st.next(lane, m, e);
        if (lane == r) {
            my_key = m;
            my_id = e;
        }
    }
    my_w = topk_weight(my_key, k, lane);
}

#endif
