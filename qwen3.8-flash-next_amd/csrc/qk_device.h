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
 * [128,256) is 1), so one v_and_or per pair builds an MFMA/dot2 operand.
 * The +128 is removed in the epilogue: sum x*(128+q) - 128*sum x.
 * The matching activation pairs are (x_i, x_{i+4}).
 */
__device__ __forceinline__ void qk_codes_to_pairs(uint32_t v, uint32_t p[4]) {
    p[0] = (v & 0x000F000Fu) | 0x43004300u;
    p[1] = ((v >> 4) & 0x000F000Fu) | 0x43004300u;
    p[2] = ((v >> 8) & 0x000F000Fu) | 0x43004300u;
    p[3] = ((v >> 12) & 0x000F000Fu) | 0x43004300u;
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

/* eight f32 activations -> hi and lo bf16 pair sets with x ~= hi + lo
 * (hi = RNE(x), lo = RNE(x - hi); relative residual <= 2^-17); xsum gets
 * the sum of (hi + lo) so that the +128 code offset cancels exactly. */
__device__ __forceinline__ void qk_f32x8_to_pairs(const float x[8], uint32_t hi[4], uint32_t lo[4],
                                                  float &xsum) {
    uint32_t h[8], l[8];
#pragma unroll
    for (int j = 0; j < 8; j++) {
        h[j] = qk_f2bf(x[j]);
        float hf = __uint_as_float(h[j] << 16);
        l[j] = qk_f2bf(x[j] - hf);
        xsum += hf + __uint_as_float(l[j] << 16);
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        hi[i] = qk_pack2(h[i], h[i + 4]);
        lo[i] = qk_pack2(l[i], l[i + 4]);
    }
}

__device__ __forceinline__ float qk_silu(float v) { return v / (1.0f + expf(-v)); }
__device__ __forceinline__ float qk_sigmoid(float v) { return 1.0f / (1.0f + expf(-v)); }

/* butterfly sum over aligned groups of `width` lanes (width a power of 2) */
template <int WIDTH>
__device__ __forceinline__ float qk_group_sum(float v) {
#pragma unroll
    for (int o = WIDTH / 2; o >= 1; o >>= 1) v += __shfl_xor(v, o, QK_WAVE);
    return v;
}

#define QK_CHECK_LAUNCH() ((int)hipGetLastError())

#endif
