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
 * inequality, so equal keys keep ascending e.  Then one round per slot
 * (next) or per two slots (next2): the wave maximum of the lane heads; the
 * lowest lane holding it wins (lane order is e order, so that is the lowest
 * e among equal keys) and pops its head.  Padding entries (e >= E) carry
 * key 0 and valid keys are at least 1, so padding is never chosen while
 * E >= k.
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

    /* the two next slots at once (wave-uniform keys and experts).  Every
     * lane offers its two heads; a butterfly over the lanes (the in-row
     * DPP steps, then the row broadcasts, lanes outside the written rows
     * merging with empty key 0) keeps the two largest keys of the union of
     * two disjoint lane sets: first = max(a1, b1), second = max(a2, b2,
     * min(a1, b1)), so lane 63 ends with the wave's two largest keys m1 >=
     * m2 in about one reduction's depth.  Slot 1 is the lowest lane whose
     * head is m1 (lane order is e order); slot 2 is the lowest lane whose
     * offer is m2, where that lane offers its second entry and every other
     * lane its head -- the first lane's second entry precedes every higher
     * lane among equal keys, so ties keep the canonical order.  Slot 2 is
     * meaningful while two valid entries remain. */
    __device__ __forceinline__ static void top2_merge(uint32_t &a1, uint32_t &a2, uint32_t b1, uint32_t b2) {
        const uint32_t lo = min(a1, b1);
        a1 = max(a1, b1);
        a2 = max(max(a2, b2), lo);
    }
    template <int CTRL>
    __device__ __forceinline__ static void top2_dpp(uint32_t &a1, uint32_t &a2) {
        top2_merge(a1, a2, qk_dpp_u<CTRL>(a1), qk_dpp_u<CTRL>(a2));
    }
    template <int CTRL, int ROWS>
    __device__ __forceinline__ static void top2_bcast(uint32_t &a1, uint32_t &a2) {
        top2_merge(a1, a2, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)a1, CTRL, ROWS, 0xF, false),
                   (uint32_t)__builtin_amdgcn_update_dpp(0, (int)a2, CTRL, ROWS, 0xF, false));
    }
    __device__ __forceinline__ void next2(int lane, uint32_t &key1, int &e1, uint32_t &key2, int &e2) {
        uint32_t a1 = kk[0], a2 = PL > 1 ? kk[PL > 1 ? 1 : 0] : 0u;
        top2_dpp<QK_DPP_XOR1>(a1, a2);
        top2_dpp<QK_DPP_XOR2>(a1, a2);
        top2_dpp<QK_DPP_HALF_MIRROR>(a1, a2);
        top2_dpp<QK_DPP_MIRROR>(a1, a2);
        top2_bcast<QK_DPP_ROW_BCAST15, 0xA>(a1, a2);
        top2_bcast<QK_DPP_ROW_BCAST31, 0xC>(a1, a2);
        const uint32_t m1 = (uint32_t)__builtin_amdgcn_readlane((int)a1, 63);
        const uint32_t m2 = (uint32_t)__builtin_amdgcn_readlane((int)a2, 63);
        const int l1 = (int)__builtin_ctzll(__ballot(kk[0] == m1));
        const uint32_t offer = lane == l1 ? (PL > 1 ? kk[PL > 1 ? 1 : 0] : 0u) : kk[0];
        const int l2 = (int)__builtin_ctzll(__ballot(offer == m2));
        const uint32_t p1 = (uint32_t)__builtin_amdgcn_readlane((int)pk0, l1);
        const uint32_t p2 = (uint32_t)__builtin_amdgcn_readlane((int)pk0, l2);
        e1 = l1 * PL + (int)(p1 & 15u);
        e2 = l2 * PL + (int)((l2 == l1 ? p2 >> 4 : p2) & 15u);
        key1 = m1;
        key2 = m2;
        if (lane == l1 || lane == l2) {
            const bool two = l1 == l2;
#pragma unroll
            for (int i = 0; i < PL; i++) {
                const uint32_t n1 = i + 1 < PL ? kk[i + 1 < PL ? i + 1 : 0] : 0u;
                const uint32_t n2 = i + 2 < PL ? kk[i + 2 < PL ? i + 2 : 0] : 0u;
                kk[i] = two ? n2 : n1;
            }
            const int sh = two ? 8 : 4;
            if (PL > 8) {
                pk0 = (pk0 >> sh) | (pk1 << (32 - sh));
                pk1 >>= sh;
            } else {
                pk0 >>= sh;
            }
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

/* slots 2r and 2r+1 for rounds r in [r0, r1) of two-slot rounds: lane s
 * (s < k) takes slot s's key and expert.  Returns the expert of the last
 * slot the rounds produced below k. */
template <int PL>
__device__ __forceinline__ int topk_rounds(WaveTopk<PL> &st, int r0, int r1, int k, int lane,
                                           uint32_t &my_key, int &my_id) {
    int last = 0;
    for (int r = r0; r < r1; r++) {
        uint32_t m1, m2;
        int ea, eb;
        st.next2(lane, m1, ea, m2, eb);
        const int s0 = 2 * r;
        if (lane == s0) {
            my_key = m1;
            my_id = ea;
        }
        if (lane == s0 + 1 && s0 + 1 < k) {
            my_key = m2;
            my_id = eb;
        }
        last = s0 + 1 < k ? eb : ea;
    }
    return last;
}

/* the whole selection: lane s < k gets slot s's expert and weight */
template <int PL>
__device__ __forceinline__ void wave_topk(const float *row, int E, int k, int lane, int &my_id,
                                          float &my_w) {
    WaveTopk<PL> st;
    st.init(row, E, lane);
    uint32_t my_key = 0u;
    my_id = 0;
    topk_rounds(st, 0, (k + 1) / 2, k, lane, my_key, my_id);
    my_w = topk_weight(my_key, k, lane);
}

#endif
