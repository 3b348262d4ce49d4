/*
 * mm_tasks.h -- the task list of the grouped MFMA kernels, built by one
 * 1024-thread workgroup from a segment table: by its own launch
 * (ffn_mfma.hip) or at the end of the dispatch that wrote the table
 * (router.hip), which saves a launch per layer.
 */
#ifndef MM_TASKS_H
#define MM_TASKS_H

#include "qk_device.h"

#define MM_MT 6              /* 16-row tiles per chunk */
#define MM_BM (16 * MM_MT)   /* rows per chunk */
#define MM_TASK_HDR 4        /* int32 header before the int4 task entries */

#define MM_NARROW_N 64       /* batches up to this many tokens also get a 16-row list */
#define MM_BM16 16

/* a segment-table word: from LDS (the table this workgroup just built,
 * mirrored there) or from global memory */
template <bool LDS>
__device__ __forceinline__ int mm_seg_ld(const int32_t *p) {
    if (LDS) return *p;
    return qk_ld(p);
}

/* One task list: {expert (-1 = shared), first position, rows, chunk} for
 * every chunk of bm rows of the segments with at least min_m rows; the
 * shared expert covers all n tokens at positions n*k.. .  The first chunk
 * of every segment comes first (segment order), then the remaining chunks
 * (segment order): a segment's later chunks hold its remainder rows, so the
 * list runs roughly longest first and the short tasks end the launch.
 * list[0] = count; entries from list + MM_TASK_HDR.  With `small`, the
 * segments with 1..min_m-1 rows (0 = shared) are listed for the GEMV
 * kernels: small[0] = count, then ids.  LDS: segtab is the workgroup's LDS
 * mirror of the table (no global round trip). */
template <bool LDS>
static __device__ void mm_tasks_list(const int32_t *segtab, int n, int k, int E, int min_m, int bm,
                                     int32_t *list, int32_t *small) {
    __shared__ unsigned long long s_scan[16];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int U = min(max(mm_seg_ld<LDS>(segtab), 0), E);
    int4 *out = (int4 *)(list + MM_TASK_HDR);
    /* segment sg of the table: expert, first position, rows */
    auto seg = [&](int sg, int &e, int &p0, int &m) {
        e = -1; p0 = n * k; m = 0;
        if (sg == 0) {
            m = n;
        } else if (sg <= U) {
            e = mm_seg_ld<LDS>(segtab + 3 * sg - 2);
            p0 = mm_seg_ld<LDS>(segtab + 3 * sg - 1);
            m = mm_seg_ld<LDS>(segtab + 3 * sg);
        }
    };
    /* the first chunks' total (one per segment with chunks): counted ahead
     * only when the segments take more than one block; with one block the
     * scan below gives it before any entry is written */
    int nfirst = U < 1024 ? -1 : 0;
    if (U >= 1024)
        for (int s0 = 0; s0 <= U; s0 += 1024) {
            int e, p0, m;
            seg(s0 + tid, e, p0, m);
            nfirst += __syncthreads_count(m >= min_m && m > 0);
        }
    /* segments 0..U in blocks of 1024; segment 0 is the shared expert.  One
     * scan counts three things in 21-bit fields: first chunks, remaining
     * chunks, small segments */
    int bfirst = 0, brest = 0, sbase = 0;
    for (int s0 = 0; s0 <= U; s0 += 1024) {
        const int sg = s0 + tid;
        int e, p0, m;
        seg(sg, e, p0, m);
        const int cnt = m >= min_m && m > 0 ? (m + bm - 1) / bm : 0;
        const int sm = m > 0 && m < min_m ? 1 : 0;
        const unsigned long long own = (unsigned long long)(cnt > 0) | ((unsigned long long)(cnt > 0 ? cnt - 1 : 0) << 21) |
                                       ((unsigned long long)sm << 42);
        unsigned long long inc = own;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const unsigned long long u = __shfl_up(inc, o, QK_WAVE);
            if (lane >= o) inc += u;
        }
        if (lane == 63) s_scan[wave] = inc;
        __syncthreads();
        unsigned long long wbase = 0, tot = 0;
        for (int i = 0; i < 16; i++) {
            if (i < wave) wbase += s_scan[i];
            tot += s_scan[i];
        }
        __syncthreads();
        const unsigned long long ex = wbase + inc - own;
        const int F = 0x1FFFFF;
        if (nfirst < 0) nfirst = (int)(tot & F);
        const int offf = bfirst + (int)(ex & F), offr = nfirst + brest + (int)((ex >> 21) & F);
        const int soff = sbase + (int)(ex >> 42);
        for (int ch = 0; ch < cnt; ch++) {
            int *o = (int *)(out + (ch == 0 ? offf : offr + ch - 1));
            o[0] = e;
            o[1] = p0;
            o[2] = m;
            o[3] = ch;
        }
        if (sm && small) small[1 + soff] = sg;
        bfirst += (int)(tot & F);
        brest += (int)((tot >> 21) & F);
        sbase += (int)(tot >> 42);
    }
    if (tid == 0) {
        list[0] = bfirst + brest;
        if (small) small[0] = sbase;
    }
}

/* The task lists of a dispatch: chunks of MM_BM rows at `tasks` with the
 * small-segment list at `small`, and, up to MM_NARROW_N tokens, chunks of
 * MM_BM16 rows at small + MM_SMALL16(E) (the down projection's list there:
 * past the small list's 2 + E ints, rounded up to 16 bytes for its int4
 * entries). */
#define MM_SMALL16(E) ((2 + (E) + 3) & ~3)
template <bool LDS = false>
static __device__ void mm_tasks_block(const int32_t *segtab, int n, int k, int E, int min_m, int32_t *tasks,
                               int32_t *small) {
    mm_tasks_list<LDS>(segtab, n, k, E, min_m, MM_BM, tasks, small);
    if (n <= MM_NARROW_N) mm_tasks_list<LDS>(segtab, n, k, E, min_m, MM_BM16, small + MM_SMALL16(E), nullptr);
}

#endif
