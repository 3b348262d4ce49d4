/*
 * stream.hip -- kernels of the streamed-expert mode: experts copied from
 * the pinned host store into HBM slots, and (device-resolved mode) the
 * residency decision itself on the GPU, so a layer call needs no host
 * round trip and can be captured in a graph.
 */
#include "qk_device.h"

/* ------------------------------------------------------ expert copies
 * Routed experts of a streamed context move from the pinned host store
 * into HBM slots with one launch per batch of experts: every workgroup
 * reads a 16 KiB chunk of one tensor piece of one expert over PCIe
 * (16-byte loads from the host mapping) and writes it to the slot.  One
 * launch replaces nine DMA copies per expert, whose fixed cost dominated
 * the 32 KiB scale and bias pieces. */

#define XC_CHUNK 16384

__global__ __launch_bounds__(256) void k_expert_copy(QkExpertCopy a) {
    /* workgroup -> (pair, piece, chunk) */
    int rest = blockIdx.x;
    const int pair = rest / a.chunks_per_expert;
    rest -= pair * a.chunks_per_expert;
    int piece = 0;
    while (piece < QK_XC_PIECES - 1 && rest >= a.chunks[piece]) {
        rest -= a.chunks[piece];
        piece++;
    }
    const size_t tb = a.tb[piece];
    const uint4 *src = (const uint4 *)(a.src[piece] + (size_t)a.pair[pair][0] * tb);
    uint4 *dst = (uint4 *)(a.dst[piece] + (size_t)a.pair[pair][1] * tb);
    const size_t beg = (size_t)rest * (XC_CHUNK / 16), end = min(beg + XC_CHUNK / 16, tb / 16);
    for (size_t i = beg + threadIdx.x; i < end; i += 256) dst[i] = src[i];
}

extern "C" int qk_launch_expert_copy(const QkExpertCopy *a, void *stream) {
    if (a->n <= 0) return 0;
    QkExpertCopy k = *a;
    int per = 0;
    for (int p = 0; p < QK_XC_PIECES; p++) {
        if (k.tb[p] % 16) return (int)hipErrorInvalidValue;
        k.chunks[p] = (int)((k.tb[p] + XC_CHUNK - 1) / XC_CHUNK);
        per += k.chunks[p];
    }
    k.chunks_per_expert = per;
    hipLaunchKernelGGL(k_expert_copy, dim3((unsigned)(per * k.n)), dim3(256), 0, (hipStream_t)stream, k);
    return QK_CHECK_LAUNCH();
}

/* ------------------------------------------- device-resolved residency
 * The slot cache of one layer kept in device memory and updated by one
 * workgroup per layer call, with the decisions of the host cache
 * (qmoe_cache.c, the reference's cache.c:99-259): each routed expert in
 * segment order is a hit (freq + 1, newest) or a miss that takes the
 * lowest free slot or evicts.  The victim rule of pick_victim, visited
 * least recent first with its cold-before-hot switch, reduces to:
 *   no unpinned cold entry          -> min (score, touched) over the hot;
 *   the oldest unpinned one is cold -> min (score, touched) over the cold;
 *   else                            -> the oldest cold entry
 * (after a cold entry replaces a hot best the best score is 0, which no
 * later entry beats), with score 0 for LRU, freq for LFU and freq + 4*hot
 * for ADAPTIVE (the same order as (freq + 4*hot) / nbytes for one entry
 * size).  Two or three block-wide minima per eviction.  Slots are pinned for the
 * call, and after it each routed expert's frequency (routed slots so far)
 * marks it hot from 4 on, as the host path does. */

__device__ __forceinline__ uint64_t xr_block_min(uint64_t v, uint64_t *s_red) {
    for (int o = 32; o > 0; o >>= 1) {
        const uint64_t u = __shfl_xor(v, o, QK_WAVE);
        v = u < v ? u : v;
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) s_red[wave] = v;
    __syncthreads();
    uint64_t r = s_red[0];
    for (int w = 1; w < (int)(blockDim.x >> 6); w++) r = s_red[w] < r ? s_red[w] : r;
    return r;
}

/* threads of the resolve workgroup (one wave measured slower: the slot
 * scans grow and the serial walk stays) */
#define SR_T 256

__global__ __launch_bounds__(SR_T) void k_stream_resolve(QkStreamResolve a) {
    __shared__ uint64_t s_red[SR_T / 64];
    __shared__ int s_slot, s_nused;
    __shared__ uint32_t s_clock;
    /* the layer's cache state lives in LDS for the call (one writer, thread
     * 0, and block-wide readers between barriers) */
    extern __shared__ uint32_t s_dyn[];
    const int S = a.slots, E = a.E, UM = min(E, S);
    int32_t *where = (int32_t *)s_dyn;          /* [E] */
    uint32_t *efreq = (uint32_t *)(where + E);  /* [E] */
    int32_t *item = (int32_t *)(efreq + E);     /* [S] */
    uint32_t *freq = (uint32_t *)(item + S);    /* [S] */
    uint32_t *touched = freq + S;               /* [S] */
    uint32_t *hot = touched + S;                /* [S] */
    int32_t *seg = (int32_t *)(hot + S);        /* [3 * min(E, S)] the call's segments */
    uint32_t *pin = (uint32_t *)(seg + 3 * UM); /* [ceil(S/32)] */
    const int tid = threadIdx.x;
    /* everything the walk reads comes into LDS in one round of loads */
    const int U = min(max(a.segtab[0], 0), UM);
    for (int i = tid; i < 3 * U; i += SR_T) seg[i] = a.segtab[1 + i];
    for (int i = tid; i < E; i += SR_T) {
        where[i] = a.where[i];
        efreq[i] = a.efreq[i];
    }
    for (int i = tid; i < S; i += SR_T) {
        item[i] = a.item[i];
        freq[i] = a.freq[i];
        touched[i] = a.touched[i];
        hot[i] = a.hot[i];
    }
    for (int i = tid; i < (S + 31) / 32; i += SR_T) pin[i] = 0u;
    if (tid == 0) {
        s_nused = a.nused[0];
        s_clock = a.clock[0];
    }
    __syncthreads();
    int nmiss = 0;
    unsigned long long st[5] = {0, 0, 0, 0, 0};
    for (int start = 0;;) {
        /* the run of hits before the next miss, in parallel: distinct
         * experts hold distinct slots, and the run takes the next clock
         * ticks in segment order */
        uint64_t m = ~0ull;
        for (int j = start + tid; j < U; j += SR_T) {
            const int ej = seg[3 * j];
            if (ej < 0 || ej >= E || where[ej] < 0) {
                m = (uint64_t)j;
                break;
            }
        }
        m = xr_block_min(m, s_red);
        const int first = m == ~0ull ? U : (int)m;
        const uint32_t clk = s_clock;
        for (int j = start + tid; j < first; j += SR_T) {
            const int sj = where[seg[3 * j]];
            freq[sj] += 1u;
            touched[sj] = clk + 1u + (uint32_t)(j - start);
            atomicOr(&pin[sj >> 5], 1u << (sj & 31));
            a.out[1 + 3 * j] = sj;
            a.out[2 + 3 * j] = seg[3 * j + 1];
            a.out[3 + 3 * j] = seg[3 * j + 2];
        }
        if (tid == 0) st[0] += (unsigned long long)(first - start);
        __syncthreads();
        if (tid == 0) s_clock = clk + (uint32_t)(first - start);
        if (first >= U) break;
        /* entry `first` misses (or names no expert): decided alone */
        const int i = first;
        start = first + 1;
        const int e = seg[3 * i];
        const int ok = e >= 0 && e < E; /* the dispatch writes ids in [0, E) */
        const int nu = s_nused;
        int slot = ok ? where[e] : -1;
        /* every wave has read this entry's state before thread 0 changes it,
         * so all take the same branch (and the same barriers) */
        __syncthreads();
        if (ok && slot >= 0) {
            if (tid == 0) {
                freq[slot] += 1u;
                touched[slot] = ++s_clock;
                pin[slot >> 5] |= 1u << (slot & 31);
                st[0]++;
            }
        } else if (ok) {
            if (nu < S) {
                slot = nu;
            } else {
                /* the oldest unpinned entry and the oldest unpinned cold one */
                uint64_t oldest = ~0ull, oldest_cold = ~0ull;
                for (int s2 = tid; s2 < S; s2 += SR_T) {
                    if (pin[s2 >> 5] & (1u << (s2 & 31))) continue;
                    const uint64_t k = ((uint64_t)touched[s2] << 32) | (uint32_t)s2;
                    oldest = k < oldest ? k : oldest;
                    if (!hot[s2]) oldest_cold = k < oldest_cold ? k : oldest_cold;
                }
                oldest = xr_block_min(oldest, s_red);
                oldest_cold = xr_block_min(oldest_cold, s_red);
                int victim = -1;
                if (oldest != ~0ull) {
                    const int os = (int)(oldest & 0xFFFFFFFFu);
                    if (oldest_cold != ~0ull && hot[os]) {
                        victim = (int)(oldest_cold & 0xFFFFFFFFu);
                    } else {
                        /* min (score, touched) over the unpinned entries of the oldest's temperature */
                        const uint32_t want_hot = oldest_cold == ~0ull ? 1u : 0u;
                        uint64_t best = ~0ull;
                        for (int s2 = tid; s2 < S; s2 += SR_T) {
                            if (pin[s2 >> 5] & (1u << (s2 & 31))) continue;
                            if ((hot[s2] != 0u) != (want_hot != 0u)) continue;
                            uint64_t score = 0;
                            if (a.policy == 1) score = freq[s2];
                            else if (a.policy == 2) score = (uint64_t)freq[s2] + (hot[s2] ? 4u : 0u);
                            /* touched < 2^32 and unique: (score, touched) orders, and names the slot */
                            const uint64_t k = (score << 32) | touched[s2];
                            best = k < best ? k : best;
                        }
                        best = xr_block_min(best, s_red);
                        if (tid == 0) s_slot = -1;
                        __syncthreads();
                        for (int s2 = tid; s2 < S; s2 += SR_T)
                            if (!(pin[s2 >> 5] & (1u << (s2 & 31))) &&
                                touched[s2] == (uint32_t)(best & 0xFFFFFFFFu))
                                s_slot = s2;
                        __syncthreads();
                        victim = s_slot;
                    }
                }
                slot = victim;
            }
            if (tid == 0) {
                st[1]++;
                if (slot < 0) {
                    st[3]++; /* rejected: not reached, every call pins fewer than slots experts */
                } else {
                    if (nu < S) {
                        s_nused = nu + 1;
                    } else {
                        where[item[slot]] = -1;
                        st[2]++;
                    }
                    item[slot] = e;
                    where[e] = slot;
                    freq[slot] = 1u;
                    touched[slot] = ++s_clock;
                    hot[slot] = efreq[e] >= 4u ? 1u : 0u;
                    pin[slot >> 5] |= 1u << (slot & 31);
                    a.miss[1 + 2 * nmiss] = e;
                    a.miss[2 + 2 * nmiss] = slot;
                    st[4]++;
                }
            }
            if (slot >= 0) nmiss++;
        } else if (tid == 0) {
            st[3]++;
        }
        if (tid == 0) {
            /* an unresolved entry (not reached) still names a slot in the pool */
            a.out[1 + 3 * i] = slot >= 0 ? slot : 0;
            a.out[2 + 3 * i] = seg[3 * i + 1];
            a.out[3 + 3 * i] = seg[3 * i + 2];
        }
        __syncthreads();
    }
    if (tid == 0) {
        a.out[0] = U;
        a.miss[0] = nmiss;
        /* routed slots per expert, then hot marks (record_route's bookkeeping) */
        for (int i = 0; i < U; i++) {
            const int e = seg[3 * i];
            if (e < 0 || e >= E) continue;
            efreq[e] += (uint32_t)max(seg[3 * i + 2], 0);
            const int s2 = where[e];
            if (s2 >= 0) hot[s2] = efreq[e] >= 4u ? 1u : 0u;
        }
        a.nused[0] = s_nused;
        a.clock[0] = s_clock;
        for (int k = 0; k < 5; k++) a.stats[k] += st[k];
    }
    __syncthreads();
    for (int i = tid; i < E; i += SR_T) {
        a.where[i] = where[i];
        a.efreq[i] = efreq[i];
    }
    for (int i = tid; i < S; i += SR_T) {
        a.item[i] = item[i];
        a.freq[i] = freq[i];
        a.touched[i] = touched[i];
        a.hot[i] = (uint8_t)hot[i];
    }
}

extern "C" size_t qk_stream_resolve_lds(int E, int slots) {
    return (size_t)E * 8 + (size_t)slots * 16 + (size_t)(E < slots ? E : slots) * 12 +
           (size_t)((slots + 31) / 32) * 4;
}

extern "C" int qk_launch_stream_resolve(const QkStreamResolve *a, void *stream) {
    const size_t lds = qk_stream_resolve_lds(a->E, a->slots);
    if (a->E <= 0 || a->slots <= 0 || lds > 65536) return (int)hipErrorInvalidValue; /* E = S = 512: 18.5 KB */
    hipLaunchKernelGGL(k_stream_resolve, dim3(1), dim3(SR_T), lds, (hipStream_t)stream, *a);
    return QK_CHECK_LAUNCH();
}

/* copies of the experts the resolve kernel listed: miss = [count, (expert,
 * slot)...]; the grid covers max_pairs experts and workgroups past the
 * count exit */
__global__ __launch_bounds__(256) void k_expert_copy_list(QkExpertCopy a, const int32_t *miss) {
    int rest = blockIdx.x;
    const int pair = rest / a.chunks_per_expert;
    if (pair >= miss[0]) return;
    rest -= pair * a.chunks_per_expert;
    int piece = 0;
    while (piece < QK_XC_PIECES - 1 && rest >= a.chunks[piece]) {
        rest -= a.chunks[piece];
        piece++;
    }
    const size_t tb = a.tb[piece];
    const uint4 *src = (const uint4 *)(a.src[piece] + (size_t)miss[1 + 2 * pair] * tb);
    uint4 *dst = (uint4 *)(a.dst[piece] + (size_t)miss[2 + 2 * pair] * tb);
    const size_t beg = (size_t)rest * (XC_CHUNK / 16), end = min(beg + XC_CHUNK / 16, tb / 16);
    for (size_t i = beg + threadIdx.x; i < end; i += 256) dst[i] = src[i];
}

extern "C" int qk_launch_expert_copy_list(const QkExpertCopy *a, const int32_t *miss, int max_pairs,
                                          void *stream) {
    if (max_pairs <= 0) return 0;
    QkExpertCopy k = *a;
    int per = 0;
    for (int p = 0; p < QK_XC_PIECES; p++) {
        if (k.tb[p] % 16) return (int)hipErrorInvalidValue;
        k.chunks[p] = (int)((k.tb[p] + XC_CHUNK - 1) / XC_CHUNK);
        per += k.chunks[p];
    }
    k.chunks_per_expert = per;
    hipLaunchKernelGGL(k_expert_copy_list, dim3((unsigned)(per * max_pairs)), dim3(256), 0,
                       (hipStream_t)stream, k, miss);
    return QK_CHECK_LAUNCH();
}
