/*
 * combine.hip -- weighted combine of routed expert outputs plus the
 * sigmoid-gated shared expert (reference C port model.c:1376-1403), and the
 * synthetic-tensor generator used by the benchmarks.
 */
#include "qk_device.h"

/* y is read once: a streaming (nontemporal) load keeps it from displacing
 * other lines in the caches */
typedef float cb_f32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float4 qk_ld_stream(const float4 *p) {
    const cb_f32x4 v = __builtin_nontemporal_load((const cb_f32x4 *)p);
    return make_float4(v.x, v.y, v.z, v.w);
}

struct CombineArgs {
    const float *y;     /* [n*k+n, H] */
    const int32_t *pos; /* [n*k] dispatch position of slot t*k+s */
    const float *w;     /* [n, k] */
    const float *sg;    /* [n] */
    const void *xres;   /* [n, H] or null */
    float *out;         /* [n, H] or null (with hyper) */
    float *hyper;       /* [n, hc, H] or null: hyper[t, j] += inject[t, j] * out[t] */
    const float *inject; /* [n, hc] */
    int H, k, n, xbf16, hc;
};

/*
 * grid = (n, ceil(H/(1024*CB_HALVES))); 256 threads x 4 columns in each of
 * CB_HALVES blocks of 1024 (two from 256 tokens on, one for small batches
 * so that they still spread over the CUs).  For token t the k
 * slots are taken in ascending dispatch position, i.e. ascending expert id
 * (the MLX dispatch order, model.py:433-441; the C port's loop at
 * model.c:1338 takes the experts in first-seen order, which only reorders
 * these fp32 sums), each as out = fma(w, y, out)
 * from out = 0, then out = fma(g, y_shared, out), then the optional residual.
 * With a hyper state, every copy j of token t becomes
 * fma(inject[t, j], out, hyper[t, j]) (model.c:1724-1731).
 */
template <int CB_HALVES>
__global__ __launch_bounds__(256) void k_combine(CombineArgs a) {
    __shared__ int s_pos[QK_MAX_TOPK];
    __shared__ float s_w[QK_MAX_TOPK];
    const int t = blockIdx.x;
    if (threadIdx.x < 64) {
        const int s = threadIdx.x;
        int p = s < a.k ? a.pos[(size_t)t * a.k + s] : 0x7FFFFFFF;
        float wt = s < a.k ? a.w[(size_t)t * a.k + s] : 0.0f;
        if (s < a.k && (p < 0 || p >= a.n * a.k)) { /* undispatched slot: no contribution */
            p = 0x7FFFFFFE;
            wt = 0.0f;
        }
        /* rank by (position, slot): invalid slots share one position */
        int rank = 0;
        for (int s2 = 0; s2 < a.k; s2++) {
            const int q = __shfl(p, s2, QK_WAVE);
            rank += (q < p || (q == p && s2 < s)) ? 1 : 0;
        }
        if (s < a.k) {
            s_pos[rank] = p;
            s_w[rank] = wt;
        }
    }
    __syncthreads();
    /* a thread owns 4 columns in each of CB_HALVES blocks of 1024, so one
     * workgroup's prologue (positions, ranks, barrier) serves 2048 columns
     * and every thread has twice the row loads in flight */
    const int cb = blockIdx.y * (1024 * CB_HALVES) + threadIdx.x * 4;
    if (cb >= a.H) return;
    bool live[CB_HALVES];
#pragma unroll
    for (int hh = 0; hh < CB_HALVES; hh++) live[hh] = cb + 1024 * hh < a.H;
    const float g = qk_ld(a.sg + t);
    float4 acc[CB_HALVES], vs[CB_HALVES];
#pragma unroll
    for (int hh = 0; hh < CB_HALVES; hh++) {
        acc[hh] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        vs[hh] = live[hh] ? qk_ld_stream((const float4 *)(a.y + ((size_t)a.n * a.k + t) * a.H + cb + 1024 * hh))
                          : acc[hh];
    }
    /* issue the independent row loads (clamped rows, no branches on the
     * row) before the dependent fma chains */
    for (int j0 = 0; j0 < a.k; j0 += 8) {
        float4 v[CB_HALVES][8];
#pragma unroll
        for (int jj = 0; jj < 8; jj++) {
            const int j = min(j0 + jj, a.k - 1);
            const int p = s_pos[j] < a.n * a.k ? s_pos[j] : 0;
#pragma unroll
            for (int hh = 0; hh < CB_HALVES; hh++)
                if (live[hh]) v[hh][jj] = qk_ld_stream((const float4 *)(a.y + (size_t)p * a.H + cb + 1024 * hh));
        }
#pragma unroll
        for (int jj = 0; jj < 8; jj++) {
            const int j = j0 + jj;
            if (j < a.k && s_pos[j] < a.n * a.k) {
                const float wt = s_w[j];
#pragma unroll
                for (int hh = 0; hh < CB_HALVES; hh++) {
                    if (!live[hh]) continue;
                    acc[hh].x = fmaf(wt, v[hh][jj].x, acc[hh].x);
                    acc[hh].y = fmaf(wt, v[hh][jj].y, acc[hh].y);
                    acc[hh].z = fmaf(wt, v[hh][jj].z, acc[hh].z);
                    acc[hh].w = fmaf(wt, v[hh][jj].w, acc[hh].w);
                }
            }
        }
    }
#pragma unroll
    for (int hh = 0; hh < CB_HALVES; hh++) {
        if (!live[hh]) continue;
        const int c = cb + 1024 * hh;
        float4 r = acc[hh];
        r.x = fmaf(g, vs[hh].x, r.x);
        r.y = fmaf(g, vs[hh].y, r.y);
        r.z = fmaf(g, vs[hh].z, r.z);
        r.w = fmaf(g, vs[hh].w, r.w);
        if (a.xres) {
            float4 xv;
            if (a.xbf16) {
                const uint2 d = *(const uint2 *)((const uint16_t *)a.xres + (size_t)t * a.H + c);
                xv = make_float4(qk_bf16_lo(d.x), qk_bf16_hi(d.x), qk_bf16_lo(d.y), qk_bf16_hi(d.y));
            } else {
                xv = *(const float4 *)((const float *)a.xres + (size_t)t * a.H + c);
            }
            r.x = xv.x + r.x;
            r.y = xv.y + r.y;
            r.z = xv.z + r.z;
            r.w = xv.w + r.w;
        }
        if (a.out) *(float4 *)(a.out + (size_t)t * a.H + c) = r;
        if (a.hyper) {
            for (int j = 0; j < a.hc; j++) {
                const float inj = qk_ld(a.inject + (size_t)t * a.hc + j);
                float4 *hp = (float4 *)(a.hyper + ((size_t)t * a.hc + j) * a.H + c);
                float4 hv = *hp;
                hv.x = fmaf(inj, r.x, hv.x);
                hv.y = fmaf(inj, r.y, hv.y);
                hv.z = fmaf(inj, r.z, hv.z);
                hv.w = fmaf(inj, r.w, hv.w);
                *hp = hv;
            }
        }
    }
}

extern "C" int qk_launch_combine(qk_shape s, int n, const float *y, const int32_t *pos,
                                 const float *w, const float *sg, const void *x_res, int x_bf16,
                                 float *out, float *hyper, const float *inject, int hc,
                                 void *stream) {
    if (n <= 0) return 0;
    CombineArgs a{y, pos, w, sg, x_res, out, hyper, inject, s.H, s.k, n, x_bf16, hc};
    if (n >= 256) {
        dim3 grid(n, (s.H + 2047) / 2048);
        hipLaunchKernelGGL(k_combine<2>, grid, dim3(256), 0, (hipStream_t)stream, a);
    } else {
        dim3 grid(n, (s.H + 1023) / 1024);
        hipLaunchKernelGGL(k_combine<1>, grid, dim3(256), 0, (hipStream_t)stream, a);
    }
    return QK_CHECK_LAUNCH();
}

/* ------------------------------------------------------- synthetic data
 * Counter-based streams: element i of stream `key` is splitmix64's output
 * function applied to key + (i+1)*golden.  Normals use Box-Muller in double
 * on draws 2i, 2i+1 (cosine branch); codes are the high 32 bits.  The host
 * generator of the test oracle computes the same values. */

#define QK_GOLDEN 0x9E3779B97F4A7C15ull

__host__ __device__ __forceinline__ uint64_t qk_mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

extern "C" uint64_t qk_tensor_key(uint64_t seed, uint32_t layer, uint32_t tag) {
    return qk_mix64(qk_mix64(seed + QK_GOLDEN) ^ (((uint64_t)layer << 32) | (uint64_t)tag));
}

__device__ __forceinline__ double qk_stream_normal(uint64_t key, uint64_t i) {
    const uint64_t r1 = qk_mix64(key + (2 * i + 1) * QK_GOLDEN);
    const uint64_t r2 = qk_mix64(key + (2 * i + 2) * QK_GOLDEN);
    const double u1 = (double)((r1 >> 11) + 1) * 0x1.0p-53;
    const double u2 = (double)(r2 >> 11) * 0x1.0p-53;
    return sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
}

__global__ void k_synth(void *dst, size_t count, int kind, uint64_t key, uint64_t start,
                        float stddev) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < count;
         i += (size_t)gridDim.x * blockDim.x) {
        const uint64_t gi = start + i;
        if (kind == 0) {
            float v = (float)(qk_stream_normal(key, gi) * (double)stddev);
            ((uint16_t *)dst)[i] = (uint16_t)qk_f2bf(v);
        } else if (kind == 1) {
            ((float *)dst)[i] = (float)(qk_stream_normal(key, gi) * (double)stddev);
        } else if (kind == 2) {
            ((uint32_t *)dst)[i] = (uint32_t)(qk_mix64(key + (gi + 1) * QK_GOLDEN) >> 32);
        } else {
            ((float *)dst)[i] = stddev;
        }
    }
}

extern "C" int qk_launch_synth(void *dst, size_t count, int kind, uint64_t key, uint64_t start,
                               float stddev, void *stream) {
    if (count == 0) return 0;
    size_t blocks = (count + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(k_synth, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, dst,
                       count, kind, key, start, stddev);
    return QK_CHECK_LAUNCH();
}
