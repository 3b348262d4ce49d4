/*
 * ffn_mfma.hip -- grouped expert GEMM on bf16 MFMA for prefill-shaped
 * segments (many tokens per expert).  Same arithmetic contract as the GEMV
 * path (ffn_gemv.hip) and as gemm_q4 in the reference (kernel.c:239-246,
 * 279-282): per 64-column group, MFMA accumulates x * (128 + q) exactly from
 * bf16 activations and integer codes, and an fp32 epilogue applies
 *     acc += s * (D - 128 * sum(x)) + b * sum(x).
 * Weights are never rounded: codes are exact in bf16, scales/biases enter
 * only the fp32 epilogue.
 *
 * Tiles.  A task is (segment, chunk of up to 128 rows of that segment, tile
 * of 128 output columns).  The workgroup's 4 waves split the columns (32
 * each); every wave runs all row subtiles (32 rows each) of the chunk.  The
 * activation rows (gathered through the dispatch permutation) are staged
 * per 64-column group in LDS, double buffered, already in the (x_i, x_{i+4})
 * pair order that matches the code-word pairs.
 *
 * v_mfma_f32_32x32x16_bf16 lane layout (probed on gfx950): A lane l holds
 * row l%32, B lane l column l%32, both with K elements [8*(l/32), +8); D
 * lane l holds column l%32, rows 8*(r/4) + 4*(l/32) + (r%4), r = 0..15.
 *
 * Gate/up: columns are rows of Wg and Wu; each wave holds both for the same
 * output column, so h = silu(g) * u is formed in registers.
 * Down:    the A operand is h (f32), split into bf16 hi + lo terms that
 *          accumulate into the same group result.
 */
#include "qk_device.h"

typedef __bf16 qk_bf16x8 __attribute__((ext_vector_type(8)));
typedef float qk_f32x16 __attribute__((ext_vector_type(16)));

#define MM_BM 128     /* rows per chunk */
#define MM_MSUB 4     /* 32-row subtiles per chunk */
#define MM_BN 128     /* output columns per tile (32 per wave) */
#define MM_ROWB 144   /* LDS bytes per staged row of one term (128 B data + pad) */

struct MfmaArgs {
    const uint32_t *q[2];  /* routed [E, N, K/8]: gate, up (or down, down) */
    const uint16_t *s[2], *b[2];
    const uint32_t *sq[2]; /* shared expert [N, K/8] */
    const uint16_t *ss[2], *sb[2];
    const void *x;         /* gate/up: bf16 [n, K] tokens; down: f32 [n*k+n, K] rows */
    float *out;            /* [n*k+n, N] */
    const int32_t *perm, *segtab, *tasks;
    int K, N, n, k, E;
    int ntile;             /* N / MM_BN */
};

__device__ __forceinline__ qk_bf16x8 qk_as_bf16x8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    const uint4 v = make_uint4(a, b, c, d);
    return __builtin_bit_cast(qk_bf16x8, v);
}

/* one code word -> the B operand (128+q as bf16, pair order) */
__device__ __forceinline__ qk_bf16x8 qk_codes_operand(uint32_t w) {
    uint32_t p[4];
    qk_codes_to_pairs(w, p);
    return qk_as_bf16x8(p[0], p[1], p[2], p[3]);
}

/* 8 bf16 activations in natural order -> pair order */
__device__ __forceinline__ uint4 qk_pair_order(uint4 d) {
    uint32_t p[4];
    qk_bf16x8_to_pairs(d, p);
    return make_uint4(p[0], p[1], p[2], p[3]);
}

/*
 * DOWN = false: gate/up (NMAT 2, activations bf16 tokens, output silu(g)*u)
 * DOWN = true : down    (NMAT 1, activations f32 rows by dispatch position,
 *                        hi/lo terms, output y)
 */
template <bool DOWN>
__global__ __launch_bounds__(256, 1) void k_mfma(MfmaArgs a) {
    constexpr int NMAT = DOWN ? 1 : 2;
    constexpr int TERMS = DOWN ? 2 : 1;
    __shared__ __attribute__((aligned(16))) uint8_t s_x[2][TERMS][MM_BM * MM_ROWB];
    __shared__ float s_xs[2][MM_BM];
    __shared__ int s_row[MM_BM];

    /* task decode: consecutive column tiles of one chunk go to one XCD
     * (workgroups are dealt round-robin over the 8 XCDs) */
    const int L = blockIdx.x;
    const int per_xcd = gridDim.x >> 3;
    const int lin = (L & 7) * per_xcd + (L >> 3);
    const int ntask = qk_ld(a.tasks);
    const int mt = lin / a.ntile, nt = lin - mt * a.ntile;
    if (mt >= ntask) return;
    const int2 tk = qk_ld((const int2 *)(a.tasks + 2) + mt);
    const int seg = tk.x, chunk = tk.y;
    int e = -1, p0, m;
    if (seg == 0) {
        p0 = a.n * a.k;
        m = a.n;
    } else {
        e = qk_ld(a.segtab + 3 * seg - 2);
        p0 = qk_ld(a.segtab + 3 * seg - 1);
        m = qk_ld(a.segtab + 3 * seg);
    }
    const int mstart = chunk * MM_BM;
    const int mrows = min(MM_BM, m - mstart);
    if (mrows <= 0) return;
    const int msub = (mrows + 31) >> 5;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int c = lane & 31, g = lane >> 5;
    const int G = a.K >> 6;

    /* staged row i -> source row of the activations */
    if (tid < MM_BM) {
        const int i = min(tid, mrows - 1);
        int r;
        if (DOWN) r = p0 + mstart + i;
        else if (seg == 0) r = mstart + i;
        else r = qk_ld(a.perm + p0 + mstart + i) / a.k;
        s_row[tid] = r;
    }

    /* weight rows of this lane: column n of the tile */
    const int n = nt * MM_BN + wave * 32 + c;
    const uint32_t *wq[NMAT];
    const uint16_t *ws[NMAT], *wb[NMAT];
    const size_t wrow = (size_t)a.K >> 3;
#pragma unroll
    for (int mt2 = 0; mt2 < NMAT; mt2++) {
        if (seg == 0) {
            wq[mt2] = a.sq[mt2] + (size_t)n * wrow;
            ws[mt2] = a.ss[mt2] + (size_t)n * G;
            wb[mt2] = a.sb[mt2] + (size_t)n * G;
        } else {
            wq[mt2] = a.q[mt2] + ((size_t)e * a.N + n) * wrow;
            ws[mt2] = a.s[mt2] + ((size_t)e * a.N + n) * G;
            wb[mt2] = a.b[mt2] + ((size_t)e * a.N + n) * G;
        }
    }
    __syncthreads();

    /* staging thread map: row si = tid/2, half sh = tid&1 (32 columns) */
    const int si = tid >> 1, sh = tid & 1;
    const int srow = s_row[si];

    /* raw activations of one group for this thread */
    uint4 xr_b[4];  /* bf16: 32 values */
    float4 xr_f[8]; /* f32: 32 values */
    auto load_x = [&](int gi) {
        if (DOWN) {
            const float4 *src = (const float4 *)((const float *)a.x + (size_t)srow * a.K + gi * 64 + sh * 32);
#pragma unroll
            for (int j = 0; j < 8; j++) xr_f[j] = qk_ld(src + j);
        } else {
            const uint4 *src = (const uint4 *)((const uint16_t *)a.x + (size_t)srow * a.K + gi * 64 + sh * 32);
#pragma unroll
            for (int j = 0; j < 4; j++) xr_b[j] = qk_ld(src + j);
        }
    };
    /* convert + store one group into LDS buffer `buf`, with the row sum */
    auto stage_x = [&](int buf) {
        float sum = 0.0f;
        uint8_t *dst0 = &s_x[buf][0][si * MM_ROWB + sh * 64];
        if (DOWN) {
            uint8_t *dst1 = &s_x[buf][TERMS - 1][si * MM_ROWB + sh * 64];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const float v[8] = {xr_f[2 * j].x, xr_f[2 * j].y, xr_f[2 * j].z, xr_f[2 * j].w,
                                    xr_f[2 * j + 1].x, xr_f[2 * j + 1].y, xr_f[2 * j + 1].z,
                                    xr_f[2 * j + 1].w};
                uint32_t hi[4], lo[4];
                qk_f32x8_to_pairs(v, hi, lo, sum);
                *(uint4 *)(dst0 + 16 * j) = make_uint4(hi[0], hi[1], hi[2], hi[3]);
                *(uint4 *)(dst1 + 16 * j) = make_uint4(lo[0], lo[1], lo[2], lo[3]);
            }
        } else {
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const uint4 d = xr_b[j];
                sum += (qk_bf16_lo(d.x) + qk_bf16_hi(d.x)) + (qk_bf16_lo(d.y) + qk_bf16_hi(d.y)) +
                       (qk_bf16_lo(d.z) + qk_bf16_hi(d.z)) + (qk_bf16_lo(d.w) + qk_bf16_hi(d.w));
                *(uint4 *)(dst0 + 16 * j) = qk_pair_order(d);
            }
        }
        sum += qk_dpp<QK_DPP_XOR1>(sum); /* the other half of the row */
        if (sh == 0) s_xs[buf][si] = sum;
    };

    /* weights of one group: this lane's 4 code words + scale/bias */
    uint4 bq[NMAT];
    uint16_t bs[NMAT], bb[NMAT];
    auto load_w = [&](int gi) {
#pragma unroll
        for (int mt2 = 0; mt2 < NMAT; mt2++) {
            bq[mt2] = qk_ld((const uint4 *)(wq[mt2] + gi * 8 + g * 4));
            bs[mt2] = qk_ld(ws[mt2] + gi);
            bb[mt2] = qk_ld(wb[mt2] + gi);
        }
    };

    qk_f32x16 acc[NMAT][MM_MSUB];
#pragma unroll
    for (int mt2 = 0; mt2 < NMAT; mt2++)
#pragma unroll
        for (int ms = 0; ms < MM_MSUB; ms++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[mt2][ms][r] = 0.0f;

    load_x(0);
    load_w(0);
    stage_x(0);
    __syncthreads();
    for (int gi = 0; gi < G; gi++) {
        const int buf = gi & 1;
        /* this group's weights into registers; prefetch the next group */
        uint4 cq[NMAT];
        float cs[NMAT], cb[NMAT];
#pragma unroll
        for (int mt2 = 0; mt2 < NMAT; mt2++) {
            cq[mt2] = bq[mt2];
            cs[mt2] = qk_bf16(bs[mt2]);
            cb[mt2] = qk_bf16(bb[mt2]);
        }
        if (gi + 1 < G) {
            load_x(gi + 1);
            load_w(gi + 1);
        }
        qk_bf16x8 bop[NMAT][4];
#pragma unroll
        for (int mt2 = 0; mt2 < NMAT; mt2++) {
            bop[mt2][0] = qk_codes_operand(cq[mt2].x);
            bop[mt2][1] = qk_codes_operand(cq[mt2].y);
            bop[mt2][2] = qk_codes_operand(cq[mt2].z);
            bop[mt2][3] = qk_codes_operand(cq[mt2].w);
        }
#pragma unroll
        for (int ms = 0; ms < MM_MSUB; ms++) {
            if (ms < msub) {
                qk_f32x16 t[NMAT];
#pragma unroll
                for (int mt2 = 0; mt2 < NMAT; mt2++)
#pragma unroll
                    for (int r = 0; r < 16; r++) t[mt2][r] = 0.0f;
#pragma unroll
                for (int tm = 0; tm < TERMS; tm++) {
                    const uint8_t *arow = &s_x[buf][tm][(32 * ms + c) * MM_ROWB];
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        const uint4 av = *(const uint4 *)(arow + (4 * g + j) * 16);
                        const qk_bf16x8 aop = __builtin_bit_cast(qk_bf16x8, av);
#pragma unroll
                        for (int mt2 = 0; mt2 < NMAT; mt2++)
                            t[mt2] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(aop, bop[mt2][j], t[mt2], 0, 0, 0);
                    }
                }
                /* group epilogue: acc += s*(D - 128*xs) + b*xs */
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int row = 32 * ms + 8 * (r >> 2) + 4 * g + (r & 3);
                    const float xs = s_xs[buf][row];
#pragma unroll
                    for (int mt2 = 0; mt2 < NMAT; mt2++) {
                        const float dq = fmaf(-128.0f, xs, t[mt2][r]);
                        acc[mt2][ms][r] = fmaf(cs[mt2], dq, fmaf(cb[mt2], xs, acc[mt2][ms][r]));
                    }
                }
            }
        }
        if (gi + 1 < G) {
            /* buffer buf^1 was last read in group gi-1, before the barrier
             * that ended it; one barrier per group suffices */
            stage_x(buf ^ 1);
            __syncthreads();
        }
    }

    /* store */
#pragma unroll
    for (int ms = 0; ms < MM_MSUB; ms++) {
        if (ms < msub) {
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int row = 32 * ms + 8 * (r >> 2) + 4 * g + (r & 3);
                if (row < mrows) {
                    const float v = DOWN ? acc[0][ms][r] : qk_silu(acc[0][ms][r]) * acc[NMAT - 1][ms][r];
                    qk_st(a.out + (size_t)(p0 + mstart + row) * a.N + n, v);
                }
            }
        }
    }
}

/* ---- task list: (segment, chunk) for every segment with at least
 * `min_m` rows; segment 0 is the shared expert over all n tokens.
 * tasks[0] = count, then int2 pairs from tasks[2]. */
__global__ __launch_bounds__(1024) void k_mfma_tasks(const int32_t *segtab, int n, int E, int min_m,
                                                     int32_t *tasks) {
    __shared__ int s_scan[16];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int U = min(max(qk_ld(segtab), 0), E);
    int base = 0;
    /* segments 0..U in blocks of 1024 */
    for (int s0 = 0; s0 <= U; s0 += 1024) {
        const int sg = s0 + tid;
        int m = 0;
        if (sg == 0) m = n;
        else if (sg <= U) m = qk_ld(segtab + 3 * sg);
        const int cnt = m >= min_m && m > 0 ? (m + MM_BM - 1) / MM_BM : 0;
        int inc = cnt;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            int u = __shfl_up(inc, o, QK_WAVE);
            if (lane >= o) inc += u;
        }
        if (lane == 63) s_scan[wave] = inc;
        __syncthreads();
        int wbase = 0, tot = 0;
        for (int i = 0; i < 16; i++) {
            if (i < wave) wbase += s_scan[i];
            tot += s_scan[i];
        }
        __syncthreads();
        const int off = base + wbase + inc - cnt;
        for (int ch = 0; ch < cnt; ch++) {
            tasks[2 + 2 * (off + ch)] = sg;
            tasks[3 + 2 * (off + ch)] = ch;
        }
        base += tot;
    }
    if (tid == 0) tasks[0] = base;
}

static int mfma_launch(const MfmaArgs &a, bool down, int max_tasks, hipStream_t st) {
    long long wgs = (long long)max_tasks * a.ntile;
    wgs = (wgs + 7) / 8 * 8;
    if (wgs <= 0) return 0;
    if (down) hipLaunchKernelGGL((k_mfma<true>), dim3((unsigned)wgs), dim3(256), 0, st, a);
    else hipLaunchKernelGGL((k_mfma<false>), dim3((unsigned)wgs), dim3(256), 0, st, a);
    return QK_CHECK_LAUNCH();
}

extern "C" int qk_mfma_max_tasks(qk_shape s, int n) {
    /* routed segments: at most min(E, n*k), plus their extra chunks; shared: ceil(n/BM) */
    const long long nk = (long long)n * s.k;
    long long t = (nk < s.E ? nk : s.E) + nk / MM_BM + (n + MM_BM - 1) / MM_BM + 1;
    return (int)t;
}

extern "C" int qk_launch_mfma_tasks(qk_shape s, int n, const int32_t *segtab, int min_m,
                                    int32_t *tasks, void *stream) {
    hipLaunchKernelGGL(k_mfma_tasks, dim3(1), dim3(1024), 0, (hipStream_t)stream, segtab, n, s.E,
                       min_m, tasks);
    return QK_CHECK_LAUNCH();
}

extern "C" int qk_launch_gateup_mfma(const qmoe_layer_weights *W, qk_shape s, const uint16_t *x,
                                     int n, const int32_t *perm, const int32_t *segtab,
                                     const int32_t *tasks, float *h, void *stream) {
    if (n <= 0) return 0;
    if (s.I % MM_BN || s.H % 64) return (int)hipErrorInvalidValue;
    MfmaArgs a;
    a.q[0] = W->gate_q; a.s[0] = W->gate_s; a.b[0] = W->gate_b;
    a.q[1] = W->up_q;   a.s[1] = W->up_s;   a.b[1] = W->up_b;
    a.sq[0] = W->sh_gate_q; a.ss[0] = W->sh_gate_s; a.sb[0] = W->sh_gate_b;
    a.sq[1] = W->sh_up_q;   a.ss[1] = W->sh_up_s;   a.sb[1] = W->sh_up_b;
    a.x = x;
    a.out = h;
    a.perm = perm;
    a.segtab = segtab;
    a.tasks = tasks;
    a.K = s.H;
    a.N = s.I;
    a.n = n;
    a.k = s.k;
    a.E = s.E;
    a.ntile = s.I / MM_BN;
    return mfma_launch(a, false, qk_mfma_max_tasks(s, n), (hipStream_t)stream);
}

extern "C" int qk_launch_down_mfma(const qmoe_layer_weights *W, qk_shape s, const float *h, int n,
                                   const int32_t *segtab, const int32_t *tasks, float *y,
                                   void *stream) {
    if (n <= 0) return 0;
    if (s.H % MM_BN || s.I % 64) return (int)hipErrorInvalidValue;
    MfmaArgs a;
    a.q[0] = a.q[1] = W->down_q;
    a.s[0] = a.s[1] = W->down_s;
    a.b[0] = a.b[1] = W->down_b;
    a.sq[0] = a.sq[1] = W->sh_down_q;
    a.ss[0] = a.ss[1] = W->sh_down_s;
    a.sb[0] = a.sb[1] = W->sh_down_b;
    a.x = h;
    a.out = y;
    a.perm = nullptr;
    a.segtab = segtab;
    a.tasks = tasks;
    a.K = s.I;
    a.N = s.H;
    a.n = n;
    a.k = s.k;
    a.E = s.E;
    a.ntile = s.H / MM_BN;
    return mfma_launch(a, true, qk_mfma_max_tasks(s, n), (hipStream_t)stream);
}
