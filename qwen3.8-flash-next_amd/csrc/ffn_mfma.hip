/*
 * ffn_mfma.hip -- grouped expert GEMM on bf16 MFMA (v_mfma_f32_16x16x32_bf16)
 * for segments with many rows (prefill, batched decode).  Same arithmetic
 * contract as the GEMV path (ffn_gemv.hip) and as gemm_q4 in the reference
 * (kernel.c:239-246, 279-282): per 64-column group g the exact integer-code
 * products are accumulated and the affine terms are applied in fp32,
 *     y = sum_g s_g * (sum_k x_k q_k) + sum_g b_g * X_g,   X_g = sum_k x_k.
 *
 * Operands.  Codes enter MFMA exactly as the bf16 numbers 128+q
 * (qk_codes_to_pairs); activations enter as bf16 planes in (x_i, x_{i+4})
 * pair order per 8 columns -- one plane for bf16 input, hi + lo planes for
 * f32 (x = hi + lo to 2^-17) -- written by k_pack_rows together with
 * P_g = -128 * X_g per row and group.  For one group the accumulator is
 * initialised with P_g (the MFMA C operand), so the two K-steps leave
 *     t = sum_k x_k (128 + q_k) - 128 X_g = sum_k x_k q_k
 * and one fp32 FMA per output adds s_g * t.  The bias term sum_g b_g X_g
 * is a K = G product done once per tile on MFMA: b is exact in bf16 and
 * X_g = P_g / -128 is split into bf16 hi + lo.  Weights are never rounded.
 *
 * Tiles.  A task is (segment, chunk of up to MM_BM rows); the grid is tasks
 * x column tiles.  The workgroup's 4 waves each own CT = 4 column tiles of
 * 16 (gate/up: 32 columns of Wg and the same 32 of Wu, so h = silu(g)*u is
 * formed in registers; down: 64 columns of Wd) and every 16-row tile of
 * the chunk.  Batches of at most 64 tokens use CT = 2 and 64-row chunks:
 * twice the workgroups, each with less LDS and fewer registers.  Per group the chunk's activation rows are staged in LDS
 * (double buffered, XOR-swizzled 16-byte chunks), the code words come from
 * a register ring MM_WD groups ahead, and the scales of the whole tile sit
 * in LDS.  The kernel body is specialised on the number of 16-row tiles.
 *
 * 16x16x32 lane layout: A lane l holds row l%16, B lane l column l%16, both
 * with K elements [8*(l/16), +8); D lane l holds column l%16, rows
 * 4*(l/16) + i.  Here the K-step j of a group gives lane quarter kq the code
 * word 2*kq + j of the group (8 columns), and the A chunk with the same
 * columns, so one 8-byte load per lane fetches both K-steps' codes.
 */
#include "qk_device.h"
#include "mm_tasks.h"
#include "mfma_parts.h"

#define MM_WD 2              /* code-word prefetch depth, groups */

struct MmArgs {
    const uint32_t *q[2]; /* routed [E, N, K/8]: gate, up (down: both Wd) */
    const uint16_t *s[2], *b[2];
    const uint32_t *sq[2]; /* shared expert [N, K/8] */
    const uint16_t *ss[2], *sb[2];
    const uint16_t *ap[2]; /* activation planes [rows, K] (hi, lo) */
    const float *ag;       /* [rows, G]: -128 * group sums */
    const float *af;       /* down: f32 activations [rows, K], split while staged */
    float *out;            /* gate/up: h [n*k+n, N]; down: y [n*k+n, N] */
    const int32_t *perm;   /* gate/up: dispatch permutation */
    const int32_t *tasks;
    int K, N, n, k, ntile;
};

#define MM_MAXG 32 /* K/64 groups held in LDS (scales, group sums) */

/* BMT = 16-row tiles a chunk can hold, CT = 16-column tiles per wave,
 * KS = 64-column groups staged per barrier */
template <int TERMS, int BMT, int CT, int KS>
struct MmSmem {
    uint4 a[2][TERMS][KS * BMT * 16 * 8]; /* activation chunks, double buffered */
    float p[MM_MAXG][BMT * 16];      /* P of the chunk's rows, [group][row] */
    uint16_t s[MM_MAXG][4][16][CT];  /* scales, [group][wave][column][tile] */
    int row[BMT * 16];
};

/* column of tile ct for this lane.  Down: a workgroup covers 64*CT
 * columns, 16*CT per wave.  Gate/up: tiles 0..CT/2-1 are gate and the rest
 * the same columns of up, so a workgroup covers 32*CT columns of h. */
template <bool DOWN, int CT>
__device__ __forceinline__ int mm_col(int nt, int wave, int ct, int c) {
    return DOWN ? nt * (64 * CT) + 16 * CT * wave + 16 * ct + c
                : nt * (32 * CT) + 8 * CT * wave + 16 * (ct % (CT / 2)) + c;
}
template <bool DOWN, int CT>
__device__ __forceinline__ int mm_mat(int ct) { return DOWN ? 0 : ct / (CT / 2); }

template <bool DOWN, int TERMS, int MS, int BMT, int CT, int KS>
__device__ __forceinline__ void mm_body(const MmArgs &a, MmSmem<TERMS, BMT, CT, KS> &sm, int e, int p0,
                                        int mstart, int mrows, int nt) {
    static_assert(MM_WD % KS == 0, "a stage of KS groups lies within one code-word ring pass");
    constexpr int BM = BMT * 16;
    constexpr int ACH = (MS * 16 * 8 + 255) / 256; /* staged 16-byte chunks per thread */
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int c = lane & 15, kq = lane >> 4;
    const int G = a.K >> 6;
    const size_t wrow = (size_t)a.K >> 3;
    const bool shared = e < 0;

    const uint32_t *wq[CT];
#pragma unroll
    for (int ct = 0; ct < CT; ct++) {
        const int mat = mm_mat<DOWN, CT>(ct);
        const uint32_t *base = shared ? a.sq[mat] : a.q[mat] + (size_t)e * a.N * wrow;
        wq[ct] = base + (size_t)mm_col<DOWN, CT>(nt, wave, ct, c) * wrow + 2 * kq;
    }
    uint2 wr[MM_WD][CT];
    auto load_w = [&](int slot, int g) {
#pragma unroll
        for (int ct = 0; ct < CT; ct++) wr[slot][ct] = qk_ld((const uint2 *)(wq[ct] + 8 * g));
    };
#pragma unroll
    for (int u = 0; u < MM_WD; u++)
        if (u < G) load_w(u, u);

    /* scales of the tile: thread -> (wave', tile', column') for the first
     * 64*CT threads, G/8 loads of 8 */
    const int w2 = tid / (16 * CT), ct2 = (tid >> 4) % CT, c2 = tid & 15;
    const bool sthr = tid < 64 * CT;
    uint4 sv[MM_MAXG / 8];
    if (sthr) {
        const int mat = mm_mat<DOWN, CT>(ct2);
        const uint16_t *sp = (shared ? a.ss[mat] : a.s[mat] + (size_t)e * a.N * G) +
                             (size_t)mm_col<DOWN, CT>(nt, w2, ct2, c2) * G;
#pragma unroll
        for (int i = 0; i < MM_MAXG / 8; i++)
            if (8 * i < G) sv[i] = qk_ld((const uint4 *)(sp + 8 * i));
    }
    __syncthreads(); /* sm.row, written by the caller */

    /* The down projection reads h in f32 and forms the hi/lo planes and the
     * group sums P while staging each group (as k_pack_rows would, in the
     * same order); the gate/up reads packed planes and their P. */
    constexpr bool F32IN = DOWN;
    static_assert(!F32IN || TERMS == 2, "f32 activations give two planes");

    /* P of the chunk's rows: 16-byte chunk ci -> row ci / (G/4), groups 4*(ci % (G/4)).. */
    constexpr int PCH = (BM * MM_MAXG / 4 + 255) / 256;
    float4 pv[PCH];
#pragma unroll
    for (int i = 0; i < PCH; i++) {
        const int ci = tid + 256 * i;
        if (!F32IN && ci < BM * (G >> 2)) {
            const int row = ci / (G >> 2), g4 = ci - row * (G >> 2);
            pv[i] = qk_ld((const float4 *)(a.ag + (size_t)sm.row[row] * G) + g4);
        }
    }

    /* element offsets of this thread's staged chunks in group 0 (rows are
     * fixed for the task; planes hold fewer than 2^31 elements) */
    uint32_t aoff[ACH];
#pragma unroll
    for (int i = 0; i < ACH; i++) {
        const int ci = tid + 256 * i;
        aoff[i] = ci < MS * 16 * 8 ? (uint32_t)sm.row[ci >> 3] * (uint32_t)a.K + (uint32_t)(ci & 7) * 8u : 0u;
    }
    /* stage st = groups st*KS .. st*KS+KS-1 (G is a multiple of 8, so of KS) */
    const int NST = G / KS;
    uint4 ar[F32IN ? 1 : KS][F32IN ? 1 : TERMS][F32IN ? 1 : ACH];
    float4 af[F32IN ? KS : 1][F32IN ? ACH : 1][2];
    auto load_a = [&](int st) {
#pragma unroll
        for (int kk = 0; kk < KS; kk++)
#pragma unroll
            for (int i = 0; i < ACH; i++) {
                const int ci = tid + 256 * i;
                if (ci < MS * 16 * 8) {
                    const uint32_t off = aoff[i] + (uint32_t)(st * KS + kk) * 64u;
                    if (F32IN) {
                        const float4 *src = (const float4 *)(a.af + off);
                        af[F32IN ? kk : 0][F32IN ? i : 0][0] = qk_ld(src);
                        af[F32IN ? kk : 0][F32IN ? i : 0][1] = qk_ld(src + 1);
                    } else {
#pragma unroll
                        for (int tm = 0; tm < TERMS; tm++)
                            ar[F32IN ? 0 : kk][F32IN ? 0 : tm][F32IN ? 0 : i] =
                                qk_ld((const uint4 *)(a.ap[tm] + off));
                    }
                }
            }
    };
    auto store_a = [&](int buf, int st) {
#pragma unroll
        for (int kk = 0; kk < KS; kk++)
#pragma unroll
            for (int i = 0; i < ACH; i++) {
                const int ci = tid + 256 * i;
                const bool ok = ci < MS * 16 * 8; /* uniform over each 8-lane row group */
                const int row = ci >> 3, kc = ci & 7;
                const int li = (kk * BM + row) * 8 + (kc ^ (row & 7));
                if (F32IN) {
                    /* k_pack_rows' arithmetic: pairs, then the group sum over
                     * the 8 chunk-lanes of the row (xor 1, 2, 4) */
                    const float4 a0 = af[F32IN ? kk : 0][F32IN ? i : 0][0], a1 = af[F32IN ? kk : 0][F32IN ? i : 0][1];
                    float v[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
                    if (!ok)
#pragma unroll
                        for (int j = 0; j < 8; j++) v[j] = 0.0f;
                    uint32_t hi[4], lo[4];
                    float sg = 0.0f;
                    sg = sg + qk_f32x8_pairs(v, hi, lo);
                    sg += qk_dpp<QK_DPP_XOR1>(sg);
                    sg += qk_dpp<QK_DPP_XOR2>(sg);
                    sg += __shfl_xor(sg, 4, QK_WAVE);
                    if (ok) {
                        sm.a[buf][0][li] = make_uint4(hi[0], hi[1], hi[2], hi[3]);
                        sm.a[buf][TERMS - 1][li] = make_uint4(lo[0], lo[1], lo[2], lo[3]);
                        if (kc == 0) sm.p[st * KS + kk][row] = -128.0f * sg;
                    }
                } else if (ok) {
#pragma unroll
                    for (int tm = 0; tm < TERMS; tm++)
                        sm.a[buf][tm][li] = ar[F32IN ? 0 : kk][F32IN ? 0 : tm][F32IN ? 0 : i];
                }
            }
    };
    load_a(0);

#pragma unroll
    for (int i = 0; i < MM_MAXG / 8; i++) {
        if (sthr && 8 * i < G) {
            const uint32_t wv[4] = {sv[i].x, sv[i].y, sv[i].z, sv[i].w};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                sm.s[8 * i + 2 * j][w2][c2][ct2] = (uint16_t)(wv[j] & 0xFFFFu);
                sm.s[8 * i + 2 * j + 1][w2][c2][ct2] = (uint16_t)(wv[j] >> 16);
            }
        }
    }
#pragma unroll
    for (int i = 0; i < PCH; i++) {
        const int ci = tid + 256 * i;
        if (!F32IN && ci < BM * (G >> 2)) {
            const int row = ci / (G >> 2), g4 = ci - row * (G >> 2);
            sm.p[4 * g4][row] = pv[i].x;
            sm.p[4 * g4 + 1][row] = pv[i].y;
            sm.p[4 * g4 + 2][row] = pv[i].z;
            sm.p[4 * g4 + 3][row] = pv[i].w;
        }
    }

    qm_f32x4 acc[MS][CT];
#pragma unroll
    for (int rt = 0; rt < MS; rt++)
#pragma unroll
        for (int ct = 0; ct < CT; ct++) acc[rt][ct] = qm_f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    store_a(0, 0);
    if (NST > 1) load_a(1);
    __syncthreads();

    /* G is a multiple of 8 (the host checks), so of MM_WD and KS.  For the
     * full-tile one-plane kernel the prefetches are unconditional, from
     * clamped groups past the end (their data is never used): a conditional
     * load makes the ring registers a merge of old and new values, and the
     * copies the compiler then places at the loop edge wait for every load
     * in flight (2 % at the prefill shape).  With two planes that costs
     * registers the kernel does not have (it spills); the narrow tiles
     * gained nothing. */
    constexpr bool UNCOND = TERMS == 1 && BMT == MM_MT;
    for (int g0 = 0; g0 < G; g0 += MM_WD) {
#pragma unroll
        for (int u = 0; u < MM_WD; u++) {
            const int g = g0 + u;
            if (UNCOND || g < G) {
                const int kk = u % KS; /* g0 is a multiple of MM_WD, so of KS */
                const int st = g / KS, buf = st & 1;
                /* buffer buf^1 was last read in stage st-1, before the barrier
                 * ending it (past the last stage it is not read again) */
                if (kk == 0 && (UNCOND || st + 1 < NST)) store_a(buf ^ 1, st + 1);
                if (kk == 0 && (UNCOND || st + 2 < NST)) load_a(min(st + 2, NST - 1));
                qm_bf16x8 bop[CT][2];
#pragma unroll
                for (int ct = 0; ct < CT; ct++) {
                    bop[ct][0] = qm_codes(wr[u][ct].x);
                    bop[ct][1] = qm_codes(wr[u][ct].y);
                }
                if (UNCOND || g + MM_WD < G) load_w(u, min(g + MM_WD, G - 1));
                float sc[CT];
                if (CT == 4) {
                    const uint2 sv = *(const uint2 *)&sm.s[g][wave][c][0];
                    sc[0] = qk_bf16_lo(sv.x);
                    sc[1 % CT] = qk_bf16_hi(sv.x);
                    sc[2 % CT] = qk_bf16_lo(sv.y);
                    sc[3 % CT] = qk_bf16_hi(sv.y);
                } else {
                    const uint32_t sv = *(const uint32_t *)&sm.s[g][wave][c][0];
                    sc[0] = qk_bf16_lo(sv);
                    sc[1 % CT] = qk_bf16_hi(sv);
                }
                /* LDS reads run one row tile ahead with one activation plane;
                 * with two the registers are not there */
                constexpr int PF = TERMS == 1 ? 2 : 1;
                qm_bf16x8 A[PF][TERMS][2];
                qm_f32x4 xi[PF];
                auto lds_a = [&](int rt, int sl) {
                    xi[sl] = *(const qm_f32x4 *)&sm.p[g][16 * rt + 4 * kq];
                    const int row = 16 * rt + c;
#pragma unroll
                    for (int tm = 0; tm < TERMS; tm++)
#pragma unroll
                        for (int j = 0; j < 2; j++)
                            A[sl][tm][j] = __builtin_bit_cast(
                                qm_bf16x8, sm.a[buf][tm][(kk * BM + row) * 8 + ((2 * kq + j) ^ (c & 7))]);
                };
                if (PF == 2) lds_a(0, 0);
#pragma unroll
                for (int rt = 0; rt < MS; rt++) {
                    const int sl = PF == 2 ? rt & 1 : 0;
                    if (PF == 1) lds_a(rt, 0);
                    else if (rt + 1 < MS) lds_a(rt + 1, (rt + 1) & (PF - 1));
                    qm_f32x4 t[CT];
#pragma unroll
                    for (int ct = 0; ct < CT; ct++)
                        t[ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[sl][0][0], bop[ct][0], xi[sl], 0, 0, 0);
#pragma unroll
                    for (int tm = 0; tm < TERMS; tm++)
#pragma unroll
                        for (int j = 0; j < 2; j++) {
                            if (tm == 0 && j == 0) continue;
#pragma unroll
                            for (int ct = 0; ct < CT; ct++)
                                t[ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[sl][tm][j], bop[ct][j], t[ct], 0, 0, 0);
                        }
#pragma unroll
                    for (int ct = 0; ct < CT; ct++)
#pragma unroll
                        for (int i = 0; i < 4; i++) acc[rt][ct][i] = fmaf(sc[ct], t[ct][i], acc[rt][ct][i]);
                }
                if (kk == KS - 1) __syncthreads();
            }
        }
    }

    /* bias term: acc += sum_g b[col][g] * X[row][g], X = P / -128 as bf16 hi + lo */
    for (int k0 = 0; k0 < G; k0 += 32) {
        const int gk = k0 + 8 * kq;
        qm_bf16x8 bb[CT];
#pragma unroll
        for (int ct = 0; ct < CT; ct++) {
            const int mat = mm_mat<DOWN, CT>(ct);
            const uint16_t *bp = (shared ? a.sb[mat] : a.b[mat] + (size_t)e * a.N * G) +
                                 (size_t)mm_col<DOWN, CT>(nt, wave, ct, c) * G;
            const uint4 v = gk < G ? qk_ld((const uint4 *)(bp + gk)) : make_uint4(0, 0, 0, 0);
            bb[ct] = __builtin_bit_cast(qm_bf16x8, v);
        }
#pragma unroll
        for (int rt = 0; rt < MS; rt++) {
            float xv[8];
#pragma unroll
            for (int j = 0; j < 8; j++) xv[j] = gk + j < G ? sm.p[gk + j][16 * rt + c] : 0.0f;
            uint32_t hi[4], lo[4];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const float x0 = xv[2 * j] * (-1.0f / 128.0f), x1 = xv[2 * j + 1] * (-1.0f / 128.0f);
                hi[j] = qk_cvt_pk_bf16(x0, x1);
                lo[j] = qk_cvt_pk_bf16(x0 - qk_bf16_lo(hi[j]), x1 - qk_bf16_hi(hi[j]));
            }
            const qm_bf16x8 AH = __builtin_bit_cast(qm_bf16x8, make_uint4(hi[0], hi[1], hi[2], hi[3]));
            const qm_bf16x8 AL = __builtin_bit_cast(qm_bf16x8, make_uint4(lo[0], lo[1], lo[2], lo[3]));
#pragma unroll
            for (int ct = 0; ct < CT; ct++) {
                acc[rt][ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(AH, bb[ct], acc[rt][ct], 0, 0, 0);
                acc[rt][ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(AL, bb[ct], acc[rt][ct], 0, 0, 0);
            }
        }
    }

    /* store rows of this chunk */
#pragma unroll
    for (int rt = 0; rt < MS; rt++) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int row = 16 * rt + 4 * kq + i;
            if (row < mrows) {
                float *o = a.out + (size_t)(p0 + mstart + row) * a.N;
                if (DOWN) {
#pragma unroll
                    for (int ct = 0; ct < CT; ct++) qk_st(o + mm_col<true, CT>(nt, wave, ct, c), acc[rt][ct][i]);
                } else {
#pragma unroll
                    for (int h2 = 0; h2 < CT / 2; h2++)
                        qk_st(o + mm_col<false, CT>(nt, wave, h2, c),
                              qk_silu_fast(acc[rt][h2][i]) * acc[rt][CT / 2 + h2][i]);
                }
            }
        }
    }
}

/* BMT * 16 must hold every chunk: BMT = MM_MT, or any BMT when the host
 * knows that no segment has more rows (a segment has at most n rows) */
/* bf16 gate/up at full tiles stages two groups per barrier (the LDS of two
 * workgroups per CU still fits) */
template <int TERMS, int BMT>
struct MmKs {
    static constexpr int value = (TERMS == 1 && BMT == MM_MT) ? 2 : 1;
};

template <bool DOWN, int TERMS, int BMT, int CT>
__global__ __launch_bounds__(256, 2) void k_mm(MmArgs a) {
    constexpr int KS = MmKs<TERMS, BMT>::value;
    __shared__ __attribute__((aligned(16))) MmSmem<TERMS, BMT, CT, KS> sm;
    /* workgroups are dealt round-robin over the 8 XCDs: workgroup L runs on
     * XCD L%8.  Tasks are interleaved over the XCDs (task 8j+x on XCD x) so
     * the real tasks, fewer than the grid allows for, spread over all of
     * them, and the column tiles of one task are consecutive workgroups of
     * one XCD, sharing its L2 */
    const int L = blockIdx.x;
    const int i8 = L >> 3;
    const int mt = (i8 / a.ntile) * 8 + (L & 7), nt = i8 - (i8 / a.ntile) * a.ntile;
    if (mt >= qk_ld(a.tasks)) return;
    const int4 tk = qk_ld((const int4 *)(a.tasks + MM_TASK_HDR) + mt);
    const int e = tk.x, p0 = tk.y, m = tk.z, mstart = tk.w * MM_BM;
    const int mrows = min(BMT * 16, m - mstart);
    if (mrows <= 0) return;
    const int tid = threadIdx.x;
    if (tid < BMT * 16) {
        /* activation row of chunk row tid (rows past the end repeat the last) */
        const int i = min(tid, mrows - 1);
        int r;
        if (DOWN) r = p0 + mstart + i;
        else if (e < 0) r = mstart + i;
        else r = qk_ld(a.perm + p0 + mstart + i) / a.k;
        sm.row[tid] = r;
    }
#define MM_CASE(T) mm_body<DOWN, TERMS, ((T) < BMT ? (T) : BMT), BMT, CT, KS>(a, sm, e, p0, mstart, mrows, nt)
    switch ((mrows + 15) >> 4) {
    case 1: MM_CASE(1); break;
    case 2: MM_CASE(2); break;
    case 3: MM_CASE(3); break;
    case 4: MM_CASE(4); break;
    case 5: MM_CASE(5); break;
    default: MM_CASE(BMT); break;
    }
#undef MM_CASE
}

/*
 * Activation rows -> MFMA planes.  One thread per 8 columns: the pair-order
 * bf16 plane (hi = RNE(x), and lo = RNE(x - hi) for f32 input) and, per row
 * and 64-column group, P = -128 * sum(hi + lo) summed in a fixed order
 * (8 columns with v_dot2 against ones, then the 8 threads of the group by a
 * butterfly).
 */
template <bool F32>
__global__ __launch_bounds__(256) void k_pack_rows(const void *x, size_t nchunks, uint16_t *hi,
                                                   uint16_t *lo, float *gsum) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= nchunks) return; /* nchunks is a multiple of 8: whole groups leave together */
    uint32_t ph[4], pl[4];
    float s = 0.0f;
    if (F32) {
        const float4 a0 = qk_ld((const float4 *)x + 2 * i), a1 = qk_ld((const float4 *)x + 2 * i + 1);
        const float v[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
        qk_f32x8_to_pairs(v, ph, pl, s);
        ((uint4 *)lo)[i] = make_uint4(pl[0], pl[1], pl[2], pl[3]);
    } else {
        qk_bf16x8_to_pairs(qk_ld((const uint4 *)x + i), ph);
#pragma unroll
        for (int j = 0; j < 4; j++) s = qk_dot2(ph[j], QK_BF16_ONES, s);
    }
    ((uint4 *)hi)[i] = make_uint4(ph[0], ph[1], ph[2], ph[3]);
    s += qk_dpp<QK_DPP_XOR1>(s);
    s += qk_dpp<QK_DPP_XOR2>(s);
    s += __shfl_xor(s, 4, QK_WAVE);
    if ((i & 7) == 0) gsum[i >> 3] = -128.0f * s;
}

/*
 * Down projection of batches of at most MM_NARROW_N tokens, K = 512, on the
 * dispatch's 16-row task list.  The 64-row kernel waits, every group, on
 * the chain activation load -> LDS store -> barrier -> LDS read (~1 us per
 * group at 1..16 rows).  Here the code words of the whole K slice of the
 * tile (8 groups, 16 bytes per lane and column tile) are loaded into
 * registers at the start, the chunk's f32 h is staged in LDS at once (hi +
 * lo planes and the group sums P, the arithmetic of k_pack_rows), and the
 * K loop reads LDS and registers only, with no barrier.  The products,
 * their order and the epilogue are those of mm_body: the outputs are
 * bit-identical.
 */
#define MMD_G 8 /* K / 64 of the shapes this kernel takes */

struct MmdSmem {
    uint4 a[2][MMD_G * 16 * 8]; /* hi, lo: [(g*16 + row)*8 + (kc ^ (row & 7))] */
    float p[MMD_G][16];         /* P = -128 X_g of the block's rows */
    uint16_t s[MMD_G][4][16][2]; /* scales, [group][wave][column][tile] */
};

__global__ __launch_bounds__(256, 2) void k_mm_down16(MmArgs a) {
    constexpr int G = MMD_G, CT = 2;
    __shared__ __attribute__((aligned(16))) MmdSmem sm;
    /* workgroups over the XCDs as for k_mm */
    const int L = blockIdx.x;
    const int i8 = L >> 3;
    const int mt = (i8 / a.ntile) * 8 + (L & 7), nt = i8 - (i8 / a.ntile) * a.ntile;
    if (mt >= qk_ld(a.tasks)) return;
    const int4 tk = qk_ld((const int4 *)(a.tasks + MM_TASK_HDR) + mt);
    const int e = tk.x, p0 = tk.y, m = tk.z, mstart = tk.w * MM_BM16;
    const int mrows = min(MM_BM16, m - mstart);
    if (mrows <= 0) return;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int c = lane & 15, kq = lane >> 4;
    const size_t wrow = (size_t)a.K >> 3;
    const bool shared = e < 0;

    /* every code word of the tile's K slice: words 2kq, 2kq+1 of each group */
    uint2 wr[G][CT];
#pragma unroll
    for (int ct = 0; ct < CT; ct++) {
        const uint32_t *base = shared ? a.sq[0] : a.q[0] + (size_t)e * a.N * wrow;
        const uint32_t *wq = base + (size_t)mm_col<true, CT>(nt, wave, ct, c) * wrow + 2 * kq;
#pragma unroll
        for (int g = 0; g < G; g++) wr[g][ct] = qk_ld((const uint2 *)(wq + 8 * g));
    }
    /* scales of the tile (as mm_body) */
    const int w2 = tid / (16 * CT), ct2 = (tid >> 4) % CT, c2 = tid & 15;
    uint4 sv = make_uint4(0, 0, 0, 0);
    if (tid < 64 * CT) {
        const uint16_t *sp = (shared ? a.ss[0] : a.s[0] + (size_t)e * a.N * G) +
                             (size_t)mm_col<true, CT>(nt, w2, ct2, c2) * G;
        sv = qk_ld((const uint4 *)sp);
    }
    /* bias words of the tile (one K step of 32 groups covers G = 8) */
    qm_bf16x8 bb[CT];
#pragma unroll
    for (int ct = 0; ct < CT; ct++) {
        const uint16_t *bp = (shared ? a.sb[0] : a.b[0] + (size_t)e * a.N * G) +
                             (size_t)mm_col<true, CT>(nt, wave, ct, c) * G;
        const uint4 v = kq == 0 ? qk_ld((const uint4 *)bp) : make_uint4(0, 0, 0, 0);
        bb[ct] = __builtin_bit_cast(qm_bf16x8, v);
    }

    /* thread -> row tid/16 of the chunk, 8-column chunks ci = tid%16 + 16 j
     * of that row (4 per thread) */
    const int arow = tid >> 4;
    {
        const int r0 = 0, brows = mrows;
        const float *src0 = a.af + (size_t)(p0 + mstart + r0 + min(arow, brows - 1)) * a.K + 8 * (tid & 15);
        float4 f[G / 2][2];
#pragma unroll
        for (int j = 0; j < G / 2; j++) {
            f[j][0] = qk_ld((const float4 *)(src0 + 128 * j));
            f[j][1] = qk_ld((const float4 *)(src0 + 128 * j) + 1);
        }
#pragma unroll
        for (int j = 0; j < G / 2; j++) {
            const int ci = (tid & 15) + 16 * j, g = ci >> 3, kc = ci & 7;
            /* k_pack_rows' arithmetic: pairs, then the group sum over the 8
             * chunk-lanes of the group (xor 1, 2, 4) */
            float v[8] = {f[j][0].x, f[j][0].y, f[j][0].z, f[j][0].w, f[j][1].x, f[j][1].y, f[j][1].z, f[j][1].w};
            uint32_t hi[4], lo[4];
            float sg = 0.0f;
            sg = sg + qk_f32x8_pairs(v, hi, lo);
            sg += qk_dpp<QK_DPP_XOR1>(sg);
            sg += qk_dpp<QK_DPP_XOR2>(sg);
            sg += __shfl_xor(sg, 4, QK_WAVE);
            const int li = (g * 16 + arow) * 8 + (kc ^ (arow & 7));
            sm.a[0][li] = make_uint4(hi[0], hi[1], hi[2], hi[3]);
            sm.a[1][li] = make_uint4(lo[0], lo[1], lo[2], lo[3]);
            if (kc == 0) sm.p[g][arow] = -128.0f * sg;
        }
        if (tid < 64 * CT) {
            const uint32_t wv[4] = {sv.x, sv.y, sv.z, sv.w};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                sm.s[2 * j][w2][c2][ct2] = (uint16_t)(wv[j] & 0xFFFFu);
                sm.s[2 * j + 1][w2][c2][ct2] = (uint16_t)(wv[j] >> 16);
            }
        }
        __syncthreads();

        qm_f32x4 acc[CT];
#pragma unroll
        for (int ct = 0; ct < CT; ct++) acc[ct] = qm_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int g = 0; g < G; g++) {
            qm_bf16x8 bop[CT][2];
#pragma unroll
            for (int ct = 0; ct < CT; ct++) {
                bop[ct][0] = qm_codes(wr[g][ct].x);
                bop[ct][1] = qm_codes(wr[g][ct].y);
            }
            qm_bf16x8 A[2][2];
#pragma unroll
            for (int tm = 0; tm < 2; tm++)
#pragma unroll
                for (int j = 0; j < 2; j++)
                    A[tm][j] = __builtin_bit_cast(qm_bf16x8, sm.a[tm][(g * 16 + c) * 8 + ((2 * kq + j) ^ (c & 7))]);
            const uint32_t sw = *(const uint32_t *)&sm.s[g][wave][c][0];
            const float sc[CT] = {qk_bf16_lo(sw), qk_bf16_hi(sw)};
            const qm_f32x4 xi = *(const qm_f32x4 *)&sm.p[g][4 * kq];
            qm_f32x4 t[CT];
#pragma unroll
            for (int ct = 0; ct < CT; ct++)
                t[ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[0][0], bop[ct][0], xi, 0, 0, 0);
#pragma unroll
            for (int tm = 0; tm < 2; tm++)
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    if (tm == 0 && j == 0) continue;
#pragma unroll
                    for (int ct = 0; ct < CT; ct++)
                        t[ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[tm][j], bop[ct][j], t[ct], 0, 0, 0);
                }
#pragma unroll
            for (int ct = 0; ct < CT; ct++)
#pragma unroll
                for (int i = 0; i < 4; i++) acc[ct][i] = fmaf(sc[ct], t[ct][i], acc[ct][i]);
        }
        /* bias term (as mm_body): acc += sum_g b[col][g] * X[row][g] */
        {
            float xv[8];
#pragma unroll
            for (int j = 0; j < 8; j++) xv[j] = 8 * kq + j < G ? sm.p[8 * kq + j][c] : 0.0f;
            uint32_t hi[4], lo[4];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const float x0 = xv[2 * j] * (-1.0f / 128.0f), x1 = xv[2 * j + 1] * (-1.0f / 128.0f);
                hi[j] = qk_cvt_pk_bf16(x0, x1);
                lo[j] = qk_cvt_pk_bf16(x0 - qk_bf16_lo(hi[j]), x1 - qk_bf16_hi(hi[j]));
            }
            const qm_bf16x8 AH = __builtin_bit_cast(qm_bf16x8, make_uint4(hi[0], hi[1], hi[2], hi[3]));
            const qm_bf16x8 AL = __builtin_bit_cast(qm_bf16x8, make_uint4(lo[0], lo[1], lo[2], lo[3]));
#pragma unroll
            for (int ct = 0; ct < CT; ct++) {
                acc[ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(AH, bb[ct], acc[ct], 0, 0, 0);
                acc[ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(AL, bb[ct], acc[ct], 0, 0, 0);
            }
        }
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int row = 4 * kq + i;
            if (row < brows) {
                float *o = a.out + (size_t)(p0 + mstart + r0 + row) * a.N;
#pragma unroll
                for (int ct = 0; ct < CT; ct++) qk_st(o + mm_col<true, CT>(nt, wave, ct, c), acc[ct][i]);
            }
        }
    }
}

/* the task list as its own launch (mm_tasks.h) */
__global__ __launch_bounds__(1024) void k_mm_tasks(const int32_t *segtab, int n, int k, int E,
                                                   int min_m, int32_t *tasks, int32_t *small) {
    mm_tasks_block(segtab, n, k, E, min_m, tasks, small);
}

/* Up to MM_NARROW_N tokens no segment exceeds 64 rows: the kernels then
 * hold 64-row chunks and give each wave 2 column tiles instead of 4, so a
 * batch of mostly small segments spreads over twice the workgroups (with
 * few rows per task the per-group latency, not the MFMA rate, bounds a
 * workgroup); the down projection at K = 512 runs on k_mm_down16 over the
 * 16-row list. */

static int mm_launch(MmArgs &a, bool down, int terms, int max_tasks, hipStream_t st,
                     const int32_t *list16 = nullptr, int max16 = 0) {
    const bool narrow = a.n <= MM_NARROW_N;
    const int ct = narrow ? 2 : 4;
    a.ntile = a.N / (down ? 64 * ct : 32 * ct);
    if (narrow && down && list16 && a.K == 64 * MMD_G) {
        a.tasks = list16;
        const long long wgs16 = (long long)(max16 + 7) / 8 * 8 * a.ntile;
        if (wgs16 <= 0) return 0;
        hipLaunchKernelGGL(k_mm_down16, dim3((unsigned)wgs16), dim3(256), 0, st, a);
        return QK_CHECK_LAUNCH();
    }
    /* every (task, column tile) once: 8 * ceil(max_tasks / 8) tasks */
    const long long wgs = (long long)(max_tasks + 7) / 8 * 8 * a.ntile;
    if (wgs <= 0) return 0;
    const dim3 grid((unsigned)wgs), blk(256);
#define MM_L(D, T, B, C) hipLaunchKernelGGL((k_mm<D, T, B, C>), grid, blk, 0, st, a)
    /* down: always the two planes formed from f32 h */
    if (narrow) {
        if (down) MM_L(true, 2, 4, 2);
        else { if (terms == 2) MM_L(false, 2, 4, 2); else MM_L(false, 1, 4, 2); }
    } else {
        if (down) MM_L(true, 2, MM_MT, 4);
        else { if (terms == 2) MM_L(false, 2, MM_MT, 4); else MM_L(false, 1, MM_MT, 4); }
    }
#undef MM_L
    return QK_CHECK_LAUNCH();
}

extern "C" int qk_mfma_max_tasks(qk_shape s, int n) {
    /* routed segments: at most min(E, n*k), plus their extra chunks; shared: ceil(n/BM) */
    const long long nk = (long long)n * s.k;
    const long long t = (nk < s.E ? nk : s.E) + nk / MM_BM + (n + MM_BM - 1) / MM_BM + 1;
    return (int)t;
}

/* entries of the 16-row list (0 above MM_NARROW_N tokens) */
static int mm_max_tasks16(qk_shape s, int n) {
    if (n > MM_NARROW_N) return 0;
    const long long nk = (long long)n * s.k;
    return (int)((nk < s.E ? nk : s.E) + nk / MM_BM16 + (n + MM_BM16 - 1) / MM_BM16 + 1);
}

extern "C" size_t qk_mfma_task_bytes(qk_shape s, int n) {
    const size_t t16 = n <= MM_NARROW_N ? (size_t)MM_TASK_HDR + 4 * (size_t)mm_max_tasks16(s, n) : 0;
    return ((size_t)MM_TASK_HDR + 4 * (size_t)qk_mfma_max_tasks(s, n) + (size_t)MM_SMALL16(s.E) + t16) * 4;
}

extern "C" int32_t *qk_mfma_small_list(qk_shape s, int n, int32_t *tasks) {
    return tasks + MM_TASK_HDR + 4 * (size_t)qk_mfma_max_tasks(s, n);
}

/* gate/up: K = H, N = I in tiles of 128 columns; down: K = I, N = H in
 * tiles of 256.  K/64 groups: a multiple of 8, at most MM_MAXG (the LDS
 * tables of scales and group sums). */
extern "C" int qk_mfma_gateup_ok(qk_shape s, int x_bf16) {
    const int G = s.H / 64;
    return s.H % 512 == 0 && s.I % 128 == 0 && G <= MM_MAXG && !s.g32;
}

extern "C" int qk_mfma_down_ok(qk_shape s) {
    const int G = s.I / 64;
    return s.I % 512 == 0 && s.H % 256 == 0 && G <= MM_MAXG && !s.g32;
}

extern "C" int qk_launch_mfma_tasks(qk_shape s, int n, const int32_t *segtab, int min_m,
                                    int32_t *tasks, void *stream) {
    hipLaunchKernelGGL(k_mm_tasks, dim3(1), dim3(1024), 0, (hipStream_t)stream, segtab, n, s.k, s.E,
                       min_m, tasks, qk_mfma_small_list(s, n, tasks));
    return QK_CHECK_LAUNCH();
}

extern "C" int qk_launch_pack_rows(const void *x, int x_bf16, size_t rows, int K, uint16_t *hi,
                                   uint16_t *lo, float *gsum, void *stream) {
    if (rows == 0) return 0;
    if (K % 64) return (int)hipErrorInvalidValue;
    const size_t nch = rows * (size_t)(K / 8);
    const unsigned grid = (unsigned)((nch + 255) / 256);
    if (x_bf16) hipLaunchKernelGGL(k_pack_rows<false>, dim3(grid), dim3(256), 0, (hipStream_t)stream, x, nch, hi, lo, gsum);
    else hipLaunchKernelGGL(k_pack_rows<true>, dim3(grid), dim3(256), 0, (hipStream_t)stream, x, nch, hi, lo, gsum);
    return QK_CHECK_LAUNCH();
}

extern "C" int qk_launch_gateup_mfma(const qmoe_layer_weights *W, qk_shape s, const uint16_t *xhi,
                                     const uint16_t *xlo, const float *xg, int n,
                                     const int32_t *perm, const int32_t *tasks, float *h,
                                     void *stream) {
    if (n <= 0) return 0;
    if (!qk_mfma_gateup_ok(s, xlo == NULL)) return (int)hipErrorInvalidValue;
    MmArgs a;
    a.q[0] = W->gate_q; a.s[0] = W->gate_s; a.b[0] = W->gate_b;
    a.q[1] = W->up_q;   a.s[1] = W->up_s;   a.b[1] = W->up_b;
    a.sq[0] = W->sh_gate_q; a.ss[0] = W->sh_gate_s; a.sb[0] = W->sh_gate_b;
    a.sq[1] = W->sh_up_q;   a.ss[1] = W->sh_up_s;   a.sb[1] = W->sh_up_b;
    a.ap[0] = xhi;
    a.ap[1] = xlo ? xlo : xhi;
    a.ag = xg;
    a.af = nullptr;
    a.out = h;
    a.perm = perm;
    a.tasks = tasks;
    a.K = s.H;
    a.N = s.I;
    a.n = n;
    a.k = s.k;
    return mm_launch(a, false, xlo ? 2 : 1, qk_mfma_max_tasks(s, n), (hipStream_t)stream);
}

extern "C" int qk_launch_down_mfma(const qmoe_layer_weights *W, qk_shape s, const float *h, int n,
                                   const int32_t *tasks, float *y, void *stream) {
    if (n <= 0) return 0;
    if (!qk_mfma_down_ok(s)) return (int)hipErrorInvalidValue;
    MmArgs a;
    a.q[0] = a.q[1] = W->down_q;
    a.s[0] = a.s[1] = W->down_s;
    a.b[0] = a.b[1] = W->down_b;
    a.sq[0] = a.sq[1] = W->sh_down_q;
    a.ss[0] = a.ss[1] = W->sh_down_s;
    a.sb[0] = a.sb[1] = W->sh_down_b;
    a.ap[0] = a.ap[1] = nullptr;
    a.ag = nullptr;
    a.af = h;
    a.out = y;
    a.perm = nullptr;
    a.tasks = tasks;
    a.K = s.I;
    a.N = s.H;
    a.n = n;
    a.k = s.k;
    return mm_launch(a, true, 2, qk_mfma_max_tasks(s, n), (hipStream_t)stream,
                     n <= MM_NARROW_N ? qk_mfma_small_list(s, n, (int32_t *)tasks) + MM_SMALL16(s.E) : nullptr,
                     mm_max_tasks16(s, n));
}
