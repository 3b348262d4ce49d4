/*
 * mfma_parts.h -- operand helpers for v_mfma_f32_16x16x32_bf16 on q4
 * weights: the vector types and the code word -> B operand conversion.
 */
#ifndef MFMA_PARTS_H
#define MFMA_PARTS_H

#include "qk_device.h"

typedef __bf16 qm_bf16x8 __attribute__((ext_vector_type(8)));
typedef float qm_f32x4 __attribute__((ext_vector_type(4)));

/* one code word -> the B operand: bf16 128+q in (q_i, q_{i+4}) pair order,
 * as qk_codes_to_pairs, built with byte permutes: the low nibbles of the
 * four bytes (q0, q2, q4, q6) and the high ones (q1, q3, q5, q7) each give
 * two pairs by interleaving with the byte 0x43 */
__device__ __forceinline__ qm_bf16x8 qm_codes(uint32_t w) {
    const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
    const uint32_t k = 0x43434343u;
    return __builtin_bit_cast(qm_bf16x8,
                              make_uint4(__builtin_amdgcn_perm(k, lo, 0x04020400u), __builtin_amdgcn_perm(k, hi, 0x04020400u),
                                         __builtin_amdgcn_perm(k, lo, 0x04030401u), __builtin_amdgcn_perm(k, hi, 0x04030401u)));
}

#endif
