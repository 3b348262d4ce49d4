/*
 * qk_device.h -- device helpers shared by the gfx950 kernels.
 */
#ifndef QK_DEVICE_H
#define QK_DEVICE_H

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "qmoe_internal.h"

typedef __bf16 qk_bf16x2 __attribute__((ext_vector_type(2)));

#define QK_WAVE 64

/* Loads through pointers known to be in global memory.  Pointers that
 * travel in argument structs are generic to the compiler, which then emits
 * flat loads; the cast gives global_load_* (vector memory counter only).
 * Hot loops issue these unconditionally from clamped addresses and select
 * the result afterwards, so independent loads are not serialised behind
 * per-load branches. */
#define QK_GLOBAL __attribute__((address_space(1)))
typedef unsigned int qk_u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int qk_u32x2 __attribute__((ext_vector_type(2)));
typedef float qk_f32x4 __attribute__((ext_vector_type(4)));

template <typename T>
__device__ __forceinline__ T qk_ld(const T *p) {
    return *(const QK_GLOBAL T *)p;
}
__device__ __forceinline__ uint4 qk_ld(const uint4 *p) {
    const qk_u32x4 v = *(const QK_GLOBAL qk_u32x4 *)p;
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint2 qk_ld(const uint2 *p) {
    const qk_u32x2 v = *(const QK_GLOBAL qk_u32x2 *)p;
    return make_uint2(v.x, v.y);
}
__device__ __forceinline__ int2 qk_ld(const int2 *p) {
    const qk_u32x2 v = *(const QK_GLOBAL qk_u32x2 *)p;
    return make_int2((int)v.x, (int)v.y);
}
__device__ __forceinline__ int4 qk_ld(const int4 *p) {
    const qk_u32x4 v = *(const QK_GLOBAL qk_u32x4 *)p;
    return make_int4((int)v.x, (int)v.y, (int)v.z, (int)v.w);
}
__device__ __forceinline__ float4 qk_ld(const float4 *p) {
    const qk_f32x4 v = *(const QK_GLOBAL qk_f32x4 *)p;
    return make_float4(v.x, v.y, v.z, v.w);
}
template <typename T>
__device__ __forceinline__ void qk_st(T *p, T v) {
    *(QK_GLOBAL T *)p = v;
}
__device__ __forceinline__ void qk_st(float4 *p, float4 v) {
    qk_f32x4 w = {v.x, v.y, v.z, v.w};
    *(QK_GLOBAL qk_f32x4 *)p = w;
}

/* bf16 bits -> f32 (exact widening, c/src/util.h:56-61) */
__device__ __forceinline__ float qk_bf16_lo(uint32_t v) { return __uint_as_float(v << 16); }
__device__ __forceinline__ float qk_bf16_hi(uint32_t v) { return __uint_as_float(v & 0xFFFF0000u); }
__device__ __forceinline__ float qk_bf16(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

/* f32 -> bf16 bits, round to nearest even, identical to c/src/util.h:63-71 */
__device__ __forceinline__ uint32_t qk_f2bf(float f) {
    uint32_t b = __float_as_uint(f);
    return (b + 0x7FFFu + ((b >> 16) & 1u)) >> 16;
}

/* fp32 dot of two bf16 pairs plus an fp32 accumulator (v_dot2c_f32_bf16) */
__device__ __forceinline__ float qk_dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(qk_bf16x2, a),
                                           __builtin_bit_cast(qk_bf16x2, b), c, false);
}

/*
 * q4 code word -> four bf16 pairs.  A u32 word holds the codes of 8
 * consecutive columns, low nibble first.  Pair i holds (code i, code i+4) as
 * the bf16 numbers 128+q (0x4300|q is exactly 128+q: the bf16 ulp in
 * [128,256) is 1), so a byte permute per pair builds an MFMA/dot2 operand.
 * The +128 is removed in the epilogue: sum x*(128+q) - 128*sum x.
 * The matching activation pairs are (x_i, x_{i+4}).
 */
__device__ __forceinline__ void qk_codes_to_pairs(uint32_t v, uint32_t p[4]) {
    /* the same four pairs in 7 instructions: the low nibbles of the four
     * bytes (q0, q2, q4, q6) and the high ones (q1, q3, q5, q7) each give two
     * pairs by one byte permute with the byte 0x43 (written as mask, shift
     * and or per pair, the compiler emits ~11) */
    const uint32_t lo = v & 0x0F0F0F0Fu, hi = (v >> 4) & 0x0F0F0F0Fu;
    const uint32_t k = 0x43434343u;
    p[0] = __builtin_amdgcn_perm(k, lo, 0x04020400u);
    p[1] = __builtin_amdgcn_perm(k, hi, 0x04020400u);
    p[2] = __builtin_amdgcn_perm(k, lo, 0x04030401u);
    p[3] = __builtin_amdgcn_perm(k, hi, 0x04030401u);
}

/* eight bf16 activations (dwords d0..d3 = (x0,x1),(x2,x3),(x4,x5),(x6,x7))
 * -> the pairs (x0,x4),(x1,x5),(x2,x6),(x3,x7) */
__device__ __forceinline__ void qk_bf16x8_to_pairs(uint4 d, uint32_t p[4]) {
    p[0] = (d.x & 0xFFFFu) | (d.z << 16);
    p[1] = (d.x >> 16) | (d.z & 0xFFFF0000u);
    p[2] = (d.y & 0xFFFFu) | (d.w << 16);
    p[3] = (d.y >> 16) | (d.w & 0xFFFF0000u);
}

__device__ __forceinline__ uint32_t qk_pack2(uint32_t lo, uint32_t hi) { return (lo & 0xFFFFu) | (hi << 16); }

/* two f32 -> a bf16 pair (a in the low half), round to nearest even:
 * v_cvt_pk_bf16_f32; same bits as qk_f2bf for finite values */
typedef __bf16 qk_bf16x2v __attribute__((ext_vector_type(2)));
typedef float qk_f32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t qk_cvt_pk_bf16(float a, float b) {
    const qk_f32x2 v = {a, b};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, qk_bf16x2v));
}

#define QK_BF16_ONES 0x3F803F80u /* the bf16 pair (1.0, 1.0) */

/* eight f32 activations -> hi and lo bf16 pair sets in (x_i, x_{i+4})
 * order with x ~= hi + lo (hi = RNE(x), lo = RNE(x - hi); x - hi is exact;
 * relative residual <= 2^-17); returns the group sum of (hi + lo): v_dot2
 * against (1, 1) from 0, hi pair then lo pair, i = 0..3.  A chunk sum is
 * 0 + g0 + g1 + g2 + g3 over its four groups, left to right, wherever the
 * groups were converted. */
__device__ __forceinline__ float qk_f32x8_pairs(const float x[8], uint32_t hi[4], uint32_t lo[4]) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
        hi[i] = qk_cvt_pk_bf16(x[i], x[i + 4]);
        lo[i] = qk_cvt_pk_bf16(x[i] - qk_bf16_lo(hi[i]), x[i + 4] - qk_bf16_hi(hi[i]));
    }
    float g = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        g = qk_dot2(hi[i], QK_BF16_ONES, g);
        g = qk_dot2(lo[i], QK_BF16_ONES, g);
    }
    return g;
}
__device__ __forceinline__ void qk_f32x8_to_pairs(const float x[8], uint32_t hi[4], uint32_t lo[4],
                                                  float &xsum) {
    xsum = xsum + qk_f32x8_pairs(x, hi, lo);
}

/* workgroup barrier that orders LDS only: the fences are limited to the
 * local address space, so global loads in flight are not waited for (a
 * plain __syncthreads waits for every outstanding load first) */
__device__ __forceinline__ void qk_lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

__device__ __forceinline__ float qk_silu(float v) { return v / (1.0f + expf(-v)); }
__device__ __forceinline__ float qk_sigmoid(float v) { return 1.0f / (1.0f + expf(-v)); }
/* silu with the hardware exp2 and reciprocal (a few ulp): for epilogues
 * where the correctly rounded division costs more than the output is worth */
__device__ __forceinline__ float qk_silu_fast(float v) {
    return v * __builtin_amdgcn_rcpf(1.0f + __expf(-v));
}

/* ------------------------------------------------ cross-lane reductions
 * DPP moves within a 16-lane row (no LDS round trip), ds_bpermute for the
 * two cross-row steps.  The sum is the pairwise tree over lanes in natural
 * order: partner l^1, then l^2, l^4, l^8, l^16, l^32.  After the two quad
 * steps every lane of a quad holds the same value, so the half-row mirror
 * (lane l <- 7-l) delivers exactly the l^4 partial, and the row mirror
 * (l <- 15-l) the l^8 partial.  Every lane of a group ends with the same
 * bits. */
template <int CTRL>
__device__ __forceinline__ float qk_dpp(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
__device__ __forceinline__ uint32_t qk_dpp_u(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, CTRL, 0xF, 0xF, false);
}
#define QK_DPP_XOR1 0xB1       /* quad_perm [1,0,3,2] */
#define QK_DPP_XOR2 0x4E       /* quad_perm [2,3,0,1] */
#define QK_DPP_HALF_MIRROR 0x141
#define QK_DPP_MIRROR 0x140

/* the value of lane l^16 (l^32): v_permlane16_swap (32_swap) with both
 * operands v leaves own and partner rows in its two results, so their xor
 * with v is the partner */
__device__ __forceinline__ uint32_t qk_xor16_u(uint32_t v) {
    const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    return r[0] ^ r[1] ^ v;
}
__device__ __forceinline__ uint32_t qk_xor32_u(uint32_t v) {
    const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return r[0] ^ r[1] ^ v;
}

/* sum over aligned groups of WIDTH lanes (WIDTH a power of 2, <= 64) */
template <int WIDTH>
__device__ __forceinline__ float qk_group_sum(float v) {
    if (WIDTH >= 2) v = v + qk_dpp<QK_DPP_XOR1>(v);
    if (WIDTH >= 4) v = v + qk_dpp<QK_DPP_XOR2>(v);
    if (WIDTH >= 8) v = v + qk_dpp<QK_DPP_HALF_MIRROR>(v);
    if (WIDTH >= 16) v = v + qk_dpp<QK_DPP_MIRROR>(v);
    if (WIDTH >= 32) v = v + __uint_as_float(qk_xor16_u(__float_as_uint(v)));
    if (WIDTH >= 64) v = v + __uint_as_float(qk_xor32_u(__float_as_uint(v)));
    return v;
}

/*
 * Wave sums of 16 per-lane partials v[0..15] at once, with the pairing of
 * qk_group_sum<64> (partners l^1, l^2, l^4, l^8, l^16, l^32 in that order),
 * so every sum has the same bits as qk_group_sum<64> of that partial.  At
 * the level of partner l^(2^b) a lane keeps the half of its values selected
 * by lane bit b and adds the partner's copy of that half (the partner keeps
 * the other half), so after four levels lane l holds partial
 * d = qk_rs16_index(l) summed over its 16-lane row, and the l^16 and l^32
 * levels add the other rows' sums of the same d.
 */
__device__ __forceinline__ int qk_rs16_index(int lane) {
    return ((lane & 1) << 3) | ((lane & 2) << 1) | ((lane & 4) >> 1) | ((lane & 8) >> 3);
}
template <int N, typename XCH>
__device__ __forceinline__ void qk_rs_level(const float *in, float *out, bool hi, XCH xch) {
#pragma unroll
    for (int i = 0; i < N / 2; i++) {
        const float keep = hi ? in[i + N / 2] : in[i];
        const float send = hi ? in[i] : in[i + N / 2];
        out[i] = keep + xch(send);
    }
}
__device__ __forceinline__ float qk_reduce_scatter16(const float v[16], int lane) {
    float a8[8], a4[4], a2[2], a1[1];
    qk_rs_level<16>(v, a8, lane & 1, [](float x) { return qk_dpp<QK_DPP_XOR1>(x); });
    qk_rs_level<8>(a8, a4, lane & 2, [](float x) { return qk_dpp<QK_DPP_XOR2>(x); });
    qk_rs_level<4>(a4, a2, lane & 4, [](float x) {
        /* ds_swizzle bit mode: and 0x1f, or 0, xor 4 (within 32 lanes) */
        return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(x), 0x101F));
    });
    qk_rs_level<2>(a2, a1, lane & 8, [](float x) { return qk_dpp<0x128>(x); /* row_ror:8 = l^8 in a row */ });
    float s = a1[0];
    s = s + __uint_as_float(qk_xor16_u(__float_as_uint(s)));
    s = s + __uint_as_float(qk_xor32_u(__float_as_uint(s)));
    return s;
}

/* wave-wide max / min of a u32, result uniform.  After the four in-row
 * DPP steps every lane of a row holds the row's extreme; row_bcast:15 then
 * carries row r's lane 15 into row r+1 (rows 1 and 3 written) and
 * row_bcast:31 carries lane 31 into rows 2 and 3, so lane 63 ends with the
 * extreme of the wave. */
#define QK_DPP_ROW_BCAST15 0x142
#define QK_DPP_ROW_BCAST31 0x143
__device__ __forceinline__ uint32_t qk_wave_max_u32(uint32_t v) {
    v = max(v, qk_dpp_u<QK_DPP_XOR1>(v));
    v = max(v, qk_dpp_u<QK_DPP_XOR2>(v));
    v = max(v, qk_dpp_u<QK_DPP_HALF_MIRROR>(v));
    v = max(v, qk_dpp_u<QK_DPP_MIRROR>(v));
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, QK_DPP_ROW_BCAST15, 0xA, 0xF, false));
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, QK_DPP_ROW_BCAST31, 0xC, 0xF, false));
    return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}
__device__ __forceinline__ uint32_t qk_wave_min_u32(uint32_t v) {
    v = min(v, qk_dpp_u<QK_DPP_XOR1>(v));
    v = min(v, qk_dpp_u<QK_DPP_XOR2>(v));
    v = min(v, qk_dpp_u<QK_DPP_HALF_MIRROR>(v));
    v = min(v, qk_dpp_u<QK_DPP_MIRROR>(v));
    v = min(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, QK_DPP_ROW_BCAST15, 0xA, 0xF, false));
    v = min(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, QK_DPP_ROW_BCAST31, 0xC, 0xF, false));
    return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

#define QK_CHECK_LAUNCH() ((int)hipGetLastError())

#endif
