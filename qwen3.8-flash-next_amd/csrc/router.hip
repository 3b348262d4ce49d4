/*
 * router.hip -- router logits, top-k + renormalise, and token dispatch for
 * gfx950.  Replaces model.c:1301-1332 and 1354-1367 of the reference C port
 * (gemm_bf16 + kernel_topk_indices + softmax-over-selected + unique/gather).
 *
 * Router reduction order ("R64", bit-exact with the oracle): for one
 * (token, expert) dot product the K axis is cut into 8-element chunks, chunk
 * c goes to lane c%64 of a wavefront, each lane runs an fma chain over its
 * chunks in ascending order starting at +0.0f, and the wave combines lanes
 * with xor butterflies 32,16,...,1.  Every lane ends with the same value.
 */
#include "qk_device.h"

/* ------------------------------------------------------------ logits */

struct RouterArgs {
    const uint16_t *router_w;
    const float *router_bias;
    const uint16_t *sh_gate_w;
    const float *norm_w;
    const void *x;
    float *logits; /* [n, E+1] */
    float *xn;     /* [n, H] or null */
    int H, E, n;
    float eps;
};

/* load the 8 activations of chunk c of token row t as f32 */
template <bool XBF16>
__device__ __forceinline__ void load_x8(const void *x, size_t row_off, int c, float v[8]) {
    if (XBF16) {
        uint4 d = *((const uint4 *)((const uint16_t *)x + row_off) + c);
        v[0] = qk_bf16_lo(d.x); v[1] = qk_bf16_hi(d.x);
        v[2] = qk_bf16_lo(d.y); v[3] = qk_bf16_hi(d.y);
        v[4] = qk_bf16_lo(d.z); v[5] = qk_bf16_hi(d.z);
        v[6] = qk_bf16_lo(d.w); v[7] = qk_bf16_hi(d.w);
    } else {
        const float4 *p = (const float4 *)((const float *)x + row_off) + 2 * c;
        float4 a = p[0], b = p[1];
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
        v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    }
}

#define RT_MAXCH 16 /* chunks per lane: H <= 8192 */

/*
 * One wavefront per (row, token block).  Rows 0..E-1 are the router,
 * row E is the shared-expert gate.  grid.x = ceil((E+1)/4), grid.y = token
 * blocks of RT_TB tokens.  With NORM, every wave RMS-normalises its tokens
 * itself (R64 sum of squares, r = 1/sqrt(ss/H + eps), (x*r)*w as
 * kernel.c:10-20) and the wave of row 0 writes the normalised rows.
 */
#define RT_TB 8
template <bool XBF16, bool NORM>
__global__ __launch_bounds__(256) void k_router(RouterArgs a) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row > a.E) return;
    const int chunks = a.H >> 3;
    const uint16_t *wrow = row < a.E ? a.router_w + (size_t)row * a.H : a.sh_gate_w;
    uint4 wv[RT_MAXCH];
#pragma unroll
    for (int i = 0; i < RT_MAXCH; i++) {
        int c = lane + 64 * i;
        if (c < chunks) wv[i] = ((const uint4 *)wrow)[c];
    }
    const float bias = (row < a.E && a.router_bias) ? a.router_bias[row] : 0.0f;
    const int t0 = blockIdx.y * RT_TB;
    const int t1 = min(a.n, t0 + RT_TB);
    for (int t = t0; t < t1; t++) {
        const size_t roff = (size_t)t * a.H;
        float r = 1.0f;
        if (NORM) {
            float ss = 0.0f;
#pragma unroll
            for (int i = 0; i < RT_MAXCH; i++) {
                int c = lane + 64 * i;
                if (c < chunks) {
                    float v[8];
                    load_x8<XBF16>(a.x, roff, c, v);
#pragma unroll
                    for (int j = 0; j < 8; j++) ss = fmaf(v[j], v[j], ss);
                }
            }
            ss = qk_group_sum<64>(ss);
            r = 1.0f / sqrtf(ss / (float)a.H + a.eps);
        }
        float acc = 0.0f;
#pragma unroll
        for (int i = 0; i < RT_MAXCH; i++) {
            int c = lane + 64 * i;
            if (c < chunks) {
                float v[8];
                load_x8<XBF16>(a.x, roff, c, v);
                if (NORM) {
                    const float4 *nw = (const float4 *)a.norm_w + 2 * c;
                    float4 w0 = nw[0], w1 = nw[1];
                    float wn[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
                    for (int j = 0; j < 8; j++) v[j] = (v[j] * r) * wn[j];
                    if (row == 0 && a.xn) {
                        float4 *o = (float4 *)(a.xn + roff) + 2 * c;
                        o[0] = make_float4(v[0], v[1], v[2], v[3]);
                        o[1] = make_float4(v[4], v[5], v[6], v[7]);
                    }
                }
                const uint4 d = wv[i];
                acc = fmaf(v[0], qk_bf16_lo(d.x), acc);
                acc = fmaf(v[1], qk_bf16_hi(d.x), acc);
                acc = fmaf(v[2], qk_bf16_lo(d.y), acc);
                acc = fmaf(v[3], qk_bf16_hi(d.y), acc);
                acc = fmaf(v[4], qk_bf16_lo(d.z), acc);
                acc = fmaf(v[5], qk_bf16_hi(d.z), acc);
                acc = fmaf(v[6], qk_bf16_lo(d.w), acc);
                acc = fmaf(v[7], qk_bf16_hi(d.w), acc);
            }
        }
        acc = qk_group_sum<64>(acc);
        if (lane == 0) {
            if (row < a.E && a.router_bias) acc = acc + bias;
            a.logits[(size_t)t * (a.E + 1) + row] = acc;
        }
    }
}

extern "C" int qk_launch_router(const qmoe_layer_weights *W, qk_shape s, const void *x, int x_bf16,
                                int n, float *logits, float *xn, void *stream) {
    if (n <= 0) return 0;
    RouterArgs a;
    a.router_w = W->router_w;
    a.router_bias = W->router_bias;
    a.sh_gate_w = W->sh_gate_w;
    a.norm_w = W->norm_w;
    a.x = x;
    a.logits = logits;
    a.xn = xn;
    a.H = s.H;
    a.E = s.E;
    a.n = n;
    a.eps = s.eps;
    dim3 grid((s.E + 1 + 3) / 4, (n + RT_TB - 1) / RT_TB);
    hipStream_t st = (hipStream_t)stream;
    bool norm = W->norm_w != nullptr;
    if (x_bf16) {
        if (norm) hipLaunchKernelGGL((k_router<true, true>), grid, dim3(256), 0, st, a);
        else hipLaunchKernelGGL((k_router<true, false>), grid, dim3(256), 0, st, a);
    } else {
        if (norm) hipLaunchKernelGGL((k_router<false, true>), grid, dim3(256), 0, st, a);
        else hipLaunchKernelGGL((k_router<false, false>), grid, dim3(256), 0, st, a);
    }
    return QK_CHECK_LAUNCH();
}

/* ------------------------------------------------------------- top-k */

/* order-preserving map f32 -> u32; -0 is first made +0 so it ties with +0 */
__device__ __forceinline__ uint32_t qk_ordkey(float v) {
    uint32_t b = __float_as_uint(v + 0.0f);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int o) {
    uint32_t lo = __shfl_xor((uint32_t)v, o, QK_WAVE);
    uint32_t hi = __shfl_xor((uint32_t)(v >> 32), o, QK_WAVE);
    return ((uint64_t)hi << 32) | lo;
}

#define TK_MAXPL (QK_MAX_EXPERTS / 64)

/*
 * One wavefront selects the top k of row[0..E): k rounds of a wave-wide
 * max over keys (ordered value, ~id), so larger logits win and equal logits
 * go to the lower expert id.  Then w_s = exp(v_s - v_0) / sum (the selected
 * values are in descending order, so v_0 is their max; model.c:1305-1318).
 * Lane s < k returns slot s.
 */
__device__ __forceinline__ void wave_topk(const float *row, int E, int k, int lane, int &my_id,
                                          float &my_w) {
    uint64_t key[TK_MAXPL];
#pragma unroll
    for (int i = 0; i < TK_MAXPL; i++) {
        int e = lane + 64 * i;
        key[i] = e < E ? (((uint64_t)qk_ordkey(row[e]) << 32) | (uint32_t)(0xFFFFFFFFu - (uint32_t)e))
                       : 0ull;
    }
    float vmax = 0.0f, sum = 0.0f, my_e = 0.0f;
    my_id = 0;
    for (int s = 0; s < k; s++) {
        uint64_t best = key[0];
        int bi = 0;
#pragma unroll
        for (int i = 1; i < TK_MAXPL; i++)
            if (key[i] > best) {
                best = key[i];
                bi = i;
            }
        uint64_t m = best;
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) {
            uint64_t other = shfl_xor_u64(m, o);
            m = other > m ? other : m;
        }
        if (best == m) {
#pragma unroll
            for (int i = 0; i < TK_MAXPL; i++)
                if (i == bi) key[i] = 0ull;
        }
        const int id = (int)(0xFFFFFFFFu - (uint32_t)m);
        const float v = row[id];
        if (s == 0) vmax = v;
        const float ev = expf(v - vmax);
        sum += ev;
        if (lane == s) {
            my_id = id;
            my_e = ev;
        }
    }
    my_w = my_e / sum;
}

struct TopkArgs {
    const float *logits; /* [n, E+1] */
    float *logits_out;   /* [n, E] or null */
    int32_t *idx;
    float *w;
    float *sg;
    int E, k, n;
};

__device__ __forceinline__ void topk_token(const TopkArgs &a, int t, int lane, int32_t *lds_idx) {
    const float *row = a.logits + (size_t)t * (a.E + 1);
    int id;
    float wt;
    wave_topk(row, a.E, a.k, lane, id, wt);
    if (lane < a.k) {
        a.idx[(size_t)t * a.k + lane] = id;
        a.w[(size_t)t * a.k + lane] = wt;
        if (lds_idx) lds_idx[t * a.k + lane] = id;
    }
    if (lane == 0) a.sg[t] = qk_sigmoid(row[a.E]);
    if (a.logits_out)
        for (int e = lane; e < a.E; e += 64) a.logits_out[(size_t)t * a.E + e] = row[e];
}

__global__ __launch_bounds__(256) void k_topk(TopkArgs a) {
    const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= a.n) return;
    topk_token(a, t, threadIdx.x & 63, nullptr);
}

extern "C" int qk_launch_topk(qk_shape s, int n, const float *logits, float *logits_out,
                              int32_t *idx, float *w, float *sg, void *stream) {
    if (n <= 0) return 0;
    TopkArgs a{logits, logits_out, idx, w, sg, s.E, s.k, n};
    hipLaunchKernelGGL(k_topk, dim3((n + 3) / 4), dim3(256), 0, (hipStream_t)stream, a);
    return QK_CHECK_LAUNCH();
}

/* ------------------------------------------------------------ dispatch
 *
 * Deterministic stable counting sort of flat slots f = t*k + s by expert.
 * Membership bitmask B[e][t/32] bit t%32 is set for every (t, e) pair
 * (atomicOr is order-independent); a slot's rank inside its expert is the
 * popcount of B[e] below bit t, which is exactly the number of earlier
 * tokens that chose e.  So the result equals the oracle's sequential
 * counting sort with no ordering dependence on the hardware.
 */

/* block-wide exclusive scan of one int per thread (blockDim = 1024) */
__device__ int block_exscan_1024(int v, int *lds /* >= 16 ints */, int &total) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int inc = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        int u = __shfl_up(inc, o, QK_WAVE);
        if (lane >= o) inc += u;
    }
    if (lane == 63) lds[wave] = inc;
    __syncthreads();
    int wbase = 0, tot = 0;
    for (int i = 0; i < 16; i++) {
        int s = lds[i];
        if (i < wave) wbase += s;
        tot += s;
    }
    __syncthreads();
    total = tot;
    return wbase + inc - v;
}

/* offsets + unique list from per-expert counts held one per thread */
__device__ void counts_to_offsets(int e, int E, int cnt, int *lds_scan, int32_t *offsets,
                                  int32_t *unique, int *lds_off) {
    int total;
    int off = block_exscan_1024(e < E ? cnt : 0, lds_scan, total);
    int ntot;
    int uoff = block_exscan_1024((e < E && cnt > 0) ? 1 : 0, lds_scan, ntot);
    if (e < E) {
        offsets[e] = off;
        if (lds_off) lds_off[e] = off;
        if (cnt > 0) unique[1 + uoff] = e;
    }
    if (e == 0) {
        offsets[E] = total;
        unique[0] = ntot;
    }
}

struct SmallDispArgs {
    TopkArgs tk;
    int32_t *offsets, *perm, *pos, *unique;
};

/* n <= QK_SMALL_N, n*k <= QK_SMALL_NK, E <= 1024: top-k and the whole
 * dispatch in one 1024-thread workgroup */
__global__ __launch_bounds__(1024) void k_topk_dispatch_small(SmallDispArgs a) {
    __shared__ int32_t s_idx[QK_SMALL_NK];
    __shared__ uint32_t s_bits[QK_MAX_EXPERTS * (QK_SMALL_N / 32)];
    __shared__ int32_t s_wpre[QK_MAX_EXPERTS * (QK_SMALL_N / 32)];
    __shared__ int32_t s_off[QK_MAX_EXPERTS];
    __shared__ int s_scan[16];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int E = a.tk.E, k = a.tk.k, n = a.tk.n;
    const int NW = (n + 31) >> 5;
    for (int i = tid; i < E * NW; i += 1024) s_bits[i] = 0u;
    for (int t = wave; t < n; t += 16) topk_token(a.tk, t, lane, s_idx);
    __syncthreads();
    for (int f = tid; f < n * k; f += 1024) {
        int t = f / k;
        atomicOr(&s_bits[s_idx[f] * NW + (t >> 5)], 1u << (t & 31));
    }
    __syncthreads();
    int cnt = 0;
    if (tid < E)
        for (int wd = 0; wd < NW; wd++) {
            s_wpre[tid * NW + wd] = cnt;
            cnt += __popc(s_bits[tid * NW + wd]);
        }
    counts_to_offsets(tid, E, cnt, s_scan, a.offsets, a.unique, s_off);
    __syncthreads();
    for (int f = tid; f < n * k; f += 1024) {
        int t = f / k, e = s_idx[f], wd = t >> 5;
        int rank = s_wpre[e * NW + wd] + __popc(s_bits[e * NW + wd] & ((1u << (t & 31)) - 1u));
        int p = s_off[e] + rank;
        a.perm[p] = f;
        a.pos[f] = p;
    }
}

extern "C" int qk_launch_topk_dispatch_small(qk_shape s, int n, const float *logits,
                                             float *logits_out, int32_t *idx, float *w, float *sg,
                                             int32_t *offsets, int32_t *perm, int32_t *pos,
                                             int32_t *unique, void *stream) {
    if (n <= 0) return 0;
    SmallDispArgs a{{logits, logits_out, idx, w, sg, s.E, s.k, n}, offsets, perm, pos, unique};
    hipLaunchKernelGGL(k_topk_dispatch_small, dim3(1), dim3(1024), 0, (hipStream_t)stream, a);
    return QK_CHECK_LAUNCH();
}

/* ---- multi-kernel dispatch (any n) ---- */

__global__ void k_fill_u32(uint32_t *p, size_t count, uint32_t v) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < count) p[i] = v;
}

/* ids outside [0, E) are skipped (their slots are not dispatched) */
__global__ void k_setbits(const int32_t *idx, int n, int k, int E, int NW, uint32_t *bits) {
    int f = blockIdx.x * blockDim.x + threadIdx.x;
    if (f >= n * k) return;
    int t = f / k, e = idx[f];
    if (e < 0 || e >= E) return;
    atomicOr(&bits[(size_t)e * NW + (t >> 5)], 1u << (t & 31));
}

/* one workgroup: per-expert word prefixes (wave per expert) + offsets */
__global__ __launch_bounds__(1024) void k_count_offsets(const uint32_t *bits, int32_t *wprefix,
                                                        int E, int NW, int32_t *offsets,
                                                        int32_t *unique) {
    __shared__ int s_cnt[QK_MAX_EXPERTS];
    __shared__ int s_scan[16];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    for (int e = wave; e < E; e += 16) {
        int base = 0;
        for (int w0 = 0; w0 < NW; w0 += 64) {
            int wd = w0 + lane;
            int c = wd < NW ? __popc(bits[(size_t)e * NW + wd]) : 0;
            int inc = c;
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                int u = __shfl_up(inc, o, QK_WAVE);
                if (lane >= o) inc += u;
            }
            if (wd < NW) wprefix[(size_t)e * NW + wd] = base + inc - c;
            base += __shfl(inc, 63, QK_WAVE);
        }
        if (lane == 0) s_cnt[e] = base;
    }
    __syncthreads();
    counts_to_offsets(tid, E, tid < E ? s_cnt[tid] : 0, s_scan, offsets, unique, nullptr);
}

__global__ void k_scatter(const int32_t *idx, int n, int k, int E, int NW, const uint32_t *bits,
                          const int32_t *wprefix, const int32_t *offsets, int32_t *perm,
                          int32_t *pos) {
    int f = blockIdx.x * blockDim.x + threadIdx.x;
    if (f >= n * k) return;
    int t = f / k, e = idx[f], wd = t >> 5;
    if (e < 0 || e >= E) {
        if (pos) pos[f] = -1;
        return;
    }
    size_t b = (size_t)e * NW + wd;
    int p = offsets[e] + wprefix[b] + __popc(bits[b] & ((1u << (t & 31)) - 1u));
    perm[p] = f;
    if (pos) pos[f] = p;
}

extern "C" int qk_launch_dispatch(qk_shape s, int n, const int32_t *idx, int32_t *offsets,
                                  int32_t *perm, int32_t *pos, int32_t *unique, uint32_t *bits,
                                  int32_t *wprefix, void *stream) {
    hipStream_t st = (hipStream_t)stream;
    if (n <= 0) return 0;
    const int NW = (n + 31) / 32;
    const size_t nb = (size_t)s.E * NW;
    hipLaunchKernelGGL(k_fill_u32, dim3((unsigned)((nb + 255) / 256)), dim3(256), 0, st, bits, nb, 0u);
    const int nk = n * s.k;
    hipLaunchKernelGGL(k_setbits, dim3((nk + 255) / 256), dim3(256), 0, st, idx, n, s.k, s.E, NW,
                       bits);
    hipLaunchKernelGGL(k_count_offsets, dim3(1), dim3(1024), 0, st, (const uint32_t *)bits, wprefix,
                       s.E, NW, offsets, unique);
    hipLaunchKernelGGL(k_scatter, dim3((nk + 255) / 256), dim3(256), 0, st, idx, n, s.k, s.E, NW,
                       (const uint32_t *)bits, (const int32_t *)wprefix, (const int32_t *)offsets,
                       perm, pos);
    return QK_CHECK_LAUNCH();
}

/* pos[perm[p]] = p; entries outside [0, count) are skipped */
__global__ void k_invert_perm(int count, const int32_t *perm, int32_t *pos) {
    int p = blockIdx.x * blockDim.x + threadIdx.x;
    if (p >= count) return;
    int f = perm[p];
    if (f >= 0 && f < count) pos[f] = p;
}

__global__ void k_fill_i32(int32_t *p, int count, int32_t v) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < count) p[i] = v;
}

extern "C" int qk_launch_invert_perm(int count, const int32_t *perm, int32_t *pos, void *stream) {
    if (count <= 0) return 0;
    hipLaunchKernelGGL(k_fill_i32, dim3((count + 255) / 256), dim3(256), 0, (hipStream_t)stream,
                       pos, count, -1);
    hipLaunchKernelGGL(k_invert_perm, dim3((count + 255) / 256), dim3(256), 0, (hipStream_t)stream,
                       count, perm, pos);
    return QK_CHECK_LAUNCH();
}
