/*
 * attention.hip -- the full-attention mixer with the QSA indexer on gfx950,
 * replacing attention_forward of the reference C port (c/src/model.c:
 * 798-1144) for n tokens at positions offset.. in five or six launches:
 *
 *   k_rows    one wave per four rows of [q_proj | k_proj | v_proj] (q4) and
 *             index_qk_proj (bf16); x (f32) as bf16 hi + lo pairs, the q4
 *             rows with gemm_q4's per-group identity (gemv_parts.h).  Also
 *             o_proj at the end.
 *   k_at_qk   one wave per (token, head): rmsnorm with q_norm / k_norm /
 *             the indexer's q norm, then partial RoPE at position offset+t
 *             (kernel.c:80-93) from the host's cos / sin table; k, v and
 *             the indexer's raw key go into their caches at rows len0 + t.
 *   k_at_pool one wave per key block completed by the call: the block's
 *             mean-pooled indexer key, rmsnorm + RoPE at the block start,
 *             kept in HBM with the layer (a pooled key depends only on its
 *             block's cached keys, so the reference's per-call recomputation
 *             gives the same values).
 *   k_at_score (past the indexer budget) one workgroup per (token, 16
 *             blocks): score sum_heads sum_i relu(q_i p_i) / sqrt(ihd),
 *             invisible blocks -inf, as order keys.
 *   k_at_sel  one workgroup per token: the top budget/compress blocks (value
 *             descending, ties to the lower block) by an 8-bit radix select
 *             -> a bitmap of kept blocks.
 *   k_at_attn one workgroup per (token, kv head, 256 keys) for up to 8 of the
 *             query heads that read that kv head: each k and v row is loaded
 *             once for all of them; scores q.k/sqrt(hd), the causal mask
 *             kk > offset + t and the block mask, chunk max, sum of exp and
 *             exp-weighted v per head.
 *   k_at_comb one wave per (token, head): the chunks merged (max, rescaled
 *             sums), times sigmoid(gate).
 * The indexer path (index_qk_proj in the router's R64 order, rmsnorm sums
 * in index order, the table's cos / sin, the block scores in the
 * reference's order) has the oracle's bits, so the kept blocks are the
 * oracle's; the attention sums run in parallel orders and match the
 * reference to rounding.
 */
#include "qk_device.h"
#include "gemv_parts.h"
#include "topk_wave.h"

/* ------------------------------------------------------------ rows GEMV */

#define AT_SEGS 4
#define AT_RPW 4 /* rows per wave; every segment's row count is a multiple */

struct RowSeg {
    const uint32_t *q;          /* q4 codes [rows, K/8], or NULL for bf16 */
    const uint16_t *s, *b;      /* q4 scales, biases [rows, K/64] */
    const uint16_t *w;          /* bf16 weights [rows, K] */
    float *out;                 /* out[t * ostride + r] */
    int rows, ostride;
};

struct RowsArgs {
    RowSeg seg[AT_SEGS];
    int start[AT_SEGS + 1];     /* first global row of each segment, then the total */
    int nseg;
    const float *x;             /* [n, K] */
    int K, n;
    float *hyper;               /* INJ (one q4 segment): hyper[t, j] += inject[t, j] * out[t], */
    const float *inject;        /* [n, hc, ostride] and [n, hc] */
    int hc;
};

template <int P, bool INJ>
__global__ __launch_bounds__(256) void k_rows(RowsArgs a) {
    const int lane = threadIdx.x & 63;
    const int r0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * AT_RPW;
    if (r0 >= a.start[a.nseg]) return;
    /* the wave's segment (a segment's row count is a multiple of AT_RPW) */
    RowSeg S = a.seg[0];
    int rr = r0;
    if (a.nseg > 1 && r0 >= a.start[1]) { S = a.seg[1]; rr = r0 - a.start[1]; }
    if (a.nseg > 2 && r0 >= a.start[2]) { S = a.seg[2]; rr = r0 - a.start[2]; }
    if (a.nseg > 3 && r0 >= a.start[3]) { S = a.seg[3]; rr = r0 - a.start[3]; }
    const int CH = a.K >> 5, G = a.K >> 6;
    const size_t wrow = (size_t)a.K >> 3;
    if (S.q) {
        uint4 wq[AT_RPW][P];
        float ws[AT_RPW][P], wb[AT_RPW][P];
#pragma unroll
        for (int j = 0; j < AT_RPW; j++) {
            const int r = rr + j;
#pragma unroll
            for (int ps = 0; ps < P; ps++) {
                const int c0 = ps * 64 + lane;
                const bool ok = c0 < CH;
                const int c = ok ? c0 : 0;
                wq[j][ps] = qk_ld((const uint4 *)(S.q + (size_t)r * wrow + 4 * (size_t)c));
                ws[j][ps] = ok ? qk_bf16(qk_ld(S.s + (size_t)r * G + (c >> 1))) : 0.0f;
                wb[j][ps] = ok ? qk_bf16(qk_ld(S.b + (size_t)r * G + (c >> 1))) : 0.0f;
                if (!ok) wq[j][ps] = make_uint4(0u, 0u, 0u, 0u);
            }
        }
        for (int t = 0; t < a.n; t++) {
            /* INJ: the token's inject weights and the hyper values of this
             * wave's rows, loaded with x (clamped addresses) */
            float iv[INJ ? QK_INJECT_MAX_HC : 1], hv[INJ ? AT_RPW : 1][INJ ? QK_INJECT_MAX_HC : 1];
            if (INJ) {
#pragma unroll
                for (int q = 0; q < QK_INJECT_MAX_HC; q++) {
                    const int qc = min(q, a.hc - 1);
                    iv[INJ ? q : 0] = qk_ld(a.inject + (size_t)t * a.hc + qc);
#pragma unroll
                    for (int j = 0; j < AT_RPW; j++)
                        hv[INJ ? j : 0][INJ ? q : 0] =
                            qk_ld(a.hyper + ((size_t)t * a.hc + qc) * S.ostride + min(rr + j, S.rows - 1));
                }
            }
            XRaw<P, false> xr;
            load_xraw<64, P, false>(a.x, (size_t)t, a.K, lane, xr);
            XPairs<64, P, false> xp;
            convert_xraw<64, P, false>(xr, a.K, lane, xp);
#pragma unroll
            for (int j = 0; j < AT_RPW; j++) {
                const float v = qk_group_sum<64>(row_part<64, P, false>(wq[j], ws[j], wb[j], xp));
                if (lane == 0) {
                    if (S.out) qk_st(S.out + (size_t)t * S.ostride + rr + j, v);
                    if (INJ)
#pragma unroll
                        for (int q = 0; q < QK_INJECT_MAX_HC; q++)
                            if (q < a.hc)
                                qk_st(a.hyper + ((size_t)t * a.hc + q) * S.ostride + rr + j,
                                      fmaf(iv[INJ ? q : 0], v, hv[INJ ? j : 0][INJ ? q : 0]));
                }
            }
        }
        return;
    }
    /* bf16 rows (index_qk_proj): f32 x times the bf16 weights in the
     * router's R64 order -- 8-element chunk c on lane c % 64, an fma chain
     * per lane over its chunks in ascending order from +0, the lanes added
     * by qk_group_sum<64> -- so the indexer's keys and queries have the
     * oracle's bits (the block selection downstream compares them) */
    const int C8 = a.K >> 3;
    for (int t = 0; t < a.n; t++) {
        float acc[AT_RPW];
#pragma unroll
        for (int j = 0; j < AT_RPW; j++) acc[j] = 0.0f;
#pragma unroll
        for (int i = 0; i < 4 * P; i++) {
            const int c0 = lane + 64 * i;
            const bool ok = c0 < C8;
            const int c = ok ? c0 : 0;
            const float4 *xp = (const float4 *)(a.x + (size_t)t * a.K) + 2 * c;
            const float4 x0 = qk_ld(xp), x1 = qk_ld(xp + 1);
#pragma unroll
            for (int j = 0; j < AT_RPW; j++) {
                const uint4 d = qk_ld((const uint4 *)(S.w + (size_t)(rr + j) * a.K) + c);
                float a2 = acc[j];
                a2 = fmaf(x0.x, qk_bf16_lo(d.x), a2);
                a2 = fmaf(x0.y, qk_bf16_hi(d.x), a2);
                a2 = fmaf(x0.z, qk_bf16_lo(d.y), a2);
                a2 = fmaf(x0.w, qk_bf16_hi(d.y), a2);
                a2 = fmaf(x1.x, qk_bf16_lo(d.z), a2);
                a2 = fmaf(x1.y, qk_bf16_hi(d.z), a2);
                a2 = fmaf(x1.z, qk_bf16_lo(d.w), a2);
                a2 = fmaf(x1.w, qk_bf16_hi(d.w), a2);
                acc[j] = ok ? a2 : acc[j];
            }
        }
#pragma unroll
        for (int j = 0; j < AT_RPW; j++) {
            const float v = qk_group_sum<64>(acc[j]);
            if (lane == 0) qk_st(S.out + (size_t)t * S.ostride + rr + j, v);
        }
    }
}

/* ------------------------------------------------------------ norms, RoPE, caches */

struct AtQkArgs {
    const float *qg;        /* [n, 2h*hd]: q | gate per head */
    const float *kraw;      /* [n, kvh*hd] */
    const float *vraw;      /* [n, kvh*hd] */
    const float *qk;        /* [n, ih*ihd + ihd]: indexer q heads, raw key */
    const float *q_norm, *k_norm, *iq_norm;
    float *qn;              /* [n, h, hd] */
    float *k_cache, *v_cache; /* [cap, kvh*hd] */
    float *idx_keys;        /* [cap, ihd] */
    float *qi;              /* [n, ih, ihd], or NULL when the indexer is off */
    const float2 *rope;     /* [positions, rot/2] (cos, sin) */
    int n, h, kvh, hd, ih, ihd, len0, offset, rot;
};

/* rmsnorm (kernel.c:10-20: (x*r)*w) of the L values in s, then partial
 * RoPE of the first rot (kernel.c:80-93) at position pos; one wave.  The
 * sum of squares is one fma chain in index order (every lane runs it on
 * the LDS copy), and cos / sin come from the table the host fills with the
 * reference's formula (cosf / sinf of pos * theta^(-2i/rot)), so the
 * normed and rotated rows have the oracle's bits. */
__device__ __forceinline__ void at_norm_rope(float *s, const float *w, int L, int rot, const float2 *rope,
                                             int pos, float *dst, int lane) {
    /* the norm weights and this position's cos / sin are loaded first, so
     * they arrive while the sum of squares runs */
    const int half = rot / 2;
    const float2 *cs = rope + (size_t)pos * half;
    float wv[4];
#pragma unroll
    for (int e = 0; e < 4; e++) wv[e] = qk_ld(w + min(lane + 64 * e, L - 1));
    float2 c[4];
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const int i = lane + 64 * e;
        const int ci = i < half ? i : (i < rot ? i - half : 0);
        c[e] = half > 0 ? cs[ci] : make_float2(1.0f, 0.0f);
    }
    float ss = 0.0f;
    for (int i = 0; i < L; i += 4) {
        const float4 v = *(const float4 *)(s + i);
        ss = fmaf(v.x, v.x, ss);
        ss = fmaf(v.y, v.y, ss);
        ss = fmaf(v.z, v.z, ss);
        ss = fmaf(v.w, v.w, ss);
    }
    const float r = 1.0f / sqrtf(ss / (float)L + 1e-6f);
    qk_wave_lds_sync();
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const int i = lane + 64 * e;
        if (i < L) s[i] = (s[i] * r) * wv[e];
    }
    qk_wave_lds_sync();
    float v[4];
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const int i = lane + 64 * e;
        if (i >= L) break;
        if (i < half) v[e] = s[i] * c[e].x - s[i + half] * c[e].y;
        else if (i < rot) v[e] = s[i - half] * c[e].y + s[i] * c[e].x;
        else v[e] = s[i];
    }
    qk_wave_lds_sync(); /* dst may be s itself */
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const int i = lane + 64 * e;
        if (i >= L) break;
        dst[i] = v[e];
    }
}

/* the first L <= 256 floats of src for this lane (elements lane + 64 e),
 * all four loads issued together (a loop with a runtime trip count would
 * wait on each); past L the last element is read again and not used */
__device__ __forceinline__ void at_ld4(const float *src, int L, int lane, float v[4]) {
#pragma unroll
    for (int e = 0; e < 4; e++) v[e] = qk_ld(src + min(lane + 64 * e, L - 1));
}
__device__ __forceinline__ void at_st4(float *dst, int L, int lane, const float v[4]) {
#pragma unroll
    for (int e = 0; e < 4; e++)
        if (lane + 64 * e < L) dst[lane + 64 * e] = v[e];
}

__global__ __launch_bounds__(64) void k_at_qk(AtQkArgs a) {
    __shared__ __align__(16) float s[256];
    const int lane = threadIdx.x, t = blockIdx.x, role = blockIdx.y;
    const int pos = a.offset + t, row = a.len0 + t;
    if (role < a.h) {
        const float *src = a.qg + (size_t)t * 2 * a.h * a.hd + (size_t)role * 2 * a.hd;
        float v[4];
        at_ld4(src, a.hd, lane, v);
        at_st4(s, a.hd, lane, v);
        qk_wave_lds_sync();
        at_norm_rope(s, a.q_norm, a.hd, a.rot, a.rope, pos, a.qn + ((size_t)t * a.h + role) * a.hd, lane);
    } else if (role < a.h + a.kvh) {
        const int kh = role - a.h;
        const size_t off = (size_t)t * a.kvh * a.hd + (size_t)kh * a.hd;
        float kv[4], vv[4], iv[4];
        at_ld4(a.kraw + off, a.hd, lane, kv);
        at_ld4(a.vraw + off, a.hd, lane, vv);
        const float *rk = a.qk + (size_t)t * (a.ih + 1) * a.ihd + (size_t)a.ih * a.ihd;
        at_ld4(rk, a.ihd, lane, iv); /* every kv head loads it; head 0 stores it */
        at_st4(s, a.hd, lane, kv);
        at_st4(a.v_cache + (size_t)row * a.kvh * a.hd + (size_t)kh * a.hd, a.hd, lane, vv);
        if (kh == 0) at_st4(a.idx_keys + (size_t)row * a.ihd, a.ihd, lane, iv);
        qk_wave_lds_sync();
        at_norm_rope(s, a.k_norm, a.hd, a.rot, a.rope, pos,
                     a.k_cache + (size_t)row * a.kvh * a.hd + (size_t)kh * a.hd, lane);
    } else {
        const int ihh = role - a.h - a.kvh;
        const float *src = a.qk + (size_t)t * (a.ih + 1) * a.ihd + (size_t)ihh * a.ihd;
        float v[4];
        at_ld4(src, a.ihd, lane, v);
        at_st4(s, a.ihd, lane, v);
        qk_wave_lds_sync();
        at_norm_rope(s, a.iq_norm, a.ihd, a.rot, a.rope, pos, a.qi + ((size_t)t * a.ih + ihh) * a.ihd, lane);
    }
}

/* ------------------------------------------------------------ QSA block selection */

#define AT_SEL_T 256

struct AtPoolArgs {
    const float *idx_keys;  /* [cap, ihd] */
    const float *ik_norm;   /* [ihd] */
    float *pooled;          /* [cap/comp, ihd] */
    const float2 *rope;     /* [positions, rot/2] (cos, sin) */
    int ihd, comp, b0, b1, rot, pos0; /* pos0: position of cache row 0 */
};

/* one wave per block b in [b0, b1): mean of its comp keys, then rmsnorm +
 * RoPE at the block start (model.c:969-1000) */
__global__ __launch_bounds__(256) void k_at_pool(AtPoolArgs a) {
    __shared__ __align__(16) float s_p[4][256];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int b = a.b0 + (int)blockIdx.x * 4 + wave;
    if (b >= a.b1) return; /* the whole wave; nothing below synchronises the workgroup */
    float *pw = s_p[wave];
    /* the block's keys four at a time, every load of a round in flight;
     * each element summed over j in ascending order */
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int j0 = 0; j0 < a.comp; j0 += 4) {
        float v[4][4];
#pragma unroll
        for (int u = 0; u < 4; u++)
            at_ld4(a.idx_keys + ((size_t)b * a.comp + min(j0 + u, a.comp - 1)) * a.ihd, a.ihd, lane, v[u]);
#pragma unroll
        for (int u = 0; u < 4; u++)
            if (j0 + u < a.comp)
#pragma unroll
                for (int e = 0; e < 4; e++) acc[e] = acc[e] + v[u][e];
    }
#pragma unroll
    for (int e = 0; e < 4; e++) acc[e] = acc[e] / (float)a.comp;
    at_st4(pw, a.ihd, lane, acc);
    qk_wave_lds_sync();
    at_norm_rope(pw, a.ik_norm, a.ihd, a.rot, a.rope, a.pos0 + b * a.comp, a.pooled + (size_t)b * a.ihd, lane);
}

struct AtScoreArgs {
    const float *pooled;    /* [nb, ihd] */
    const float *qi;        /* [n, ih, ihd] */
    uint32_t *skey;         /* [n, ldk] order keys of the block scores */
    int ih, ihd, comp, nb, ldk, offset;
};

#define AT_SB 16 /* blocks per workgroup of k_at_score (16 beat 32 and 64 at one token) */

/* dynamic LDS of k_at_score: the token's queries, a tile of AT_SB pooled
 * keys (rows padded by 4 floats: 16-byte aligned, banks staggered), the
 * per-head dots; at most 53 KB (ih * ihd <= 8192, ihd <= 256) */
static size_t at_score_lds(int ih, int ihd) {
    return ((size_t)ih * ihd + (size_t)AT_SB * (ihd + 4) + (size_t)ih * AT_SB) * 4;
}

/* grid (n, ceil(nb / AT_SB)): workgroup = (token t, AT_SB blocks), thread
 * (block tid % AT_SB, head slot tid / AT_SB) runs the heads of its slot, reading
 * four query and key values per LDS access.  The arithmetic is the
 * reference's order (model.c:1030-1045): per head one chain dot = dot +
 * relu(q_i * p_i) over i ascending from 0, the heads added in order from
 * 0, then / sqrt(ihd); so the scores, and the blocks they keep, are the
 * oracle's bit for bit. */
__global__ __launch_bounds__(256) void k_at_score(AtScoreArgs a) {
    constexpr int SB = AT_SB;
    extern __shared__ float at_lds[];
    const int ih = a.ih, ihd = a.ihd, pl = ihd + 4;
    float *s_q = at_lds;                       /* [ih * ihd] */
    float *s_p = s_q + ih * ihd;               /* [SB][ihd + 4] */
    float *s_d = s_p + SB * pl;                /* [ih][SB] */
    const int tid = threadIdx.x, t = blockIdx.x, b0 = (int)blockIdx.y * SB;
    const int nbt = min(SB, a.nb - b0);
    /* staging in float4s, four loads in flight per thread and round (a
     * loop with a runtime trip count would wait on each load) */
    const int q4 = ih * ihd / 4, r4 = ihd / 4, p4 = nbt * r4;
    const float4 *qsrc = (const float4 *)(a.qi + (size_t)t * ih * ihd);
    const float4 *psrc = (const float4 *)(a.pooled + (size_t)b0 * ihd);
    for (int j0 = tid; j0 < q4 + p4; j0 += 4 * 256) {
        float4 v[4];
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int j = min(j0 + 256 * u, q4 + p4 - 1);
            v[u] = j < q4 ? qk_ld(qsrc + j) : qk_ld(psrc + (j - q4));
        }
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int j = j0 + 256 * u;
            if (j < q4) {
                *(float4 *)(s_q + 4 * j) = v[u];
            } else if (j < q4 + p4) {
                const int bb = (j - q4) / r4, c4 = (j - q4) - bb * r4;
                *(float4 *)(s_p + bb * pl + 4 * c4) = v[u];
            }
        }
    }
    __syncthreads();
    const int bl = tid % SB;
    if (bl < nbt)
        for (int hh = tid / SB; hh < ih; hh += 256 / SB) {
            const float4 *q = (const float4 *)(s_q + hh * ihd), *p = (const float4 *)(s_p + bl * pl);
            float dot = 0.0f;
#pragma unroll 4
            for (int i = 0; i < ihd / 4; i++) {
                const float4 qv = q[i], pv = p[i];
                const float v0 = qv.x * pv.x, v1 = qv.y * pv.y, v2 = qv.z * pv.z, v3 = qv.w * pv.w;
                dot = dot + (v0 > 0.0f ? v0 : 0.0f);
                dot = dot + (v1 > 0.0f ? v1 : 0.0f);
                dot = dot + (v2 > 0.0f ? v2 : 0.0f);
                dot = dot + (v3 > 0.0f ? v3 : 0.0f);
            }
            s_d[hh * SB + bl] = dot;
        }
    __syncthreads();
    if (tid < nbt) {
        float acc = 0.0f;
        for (int hh = 0; hh < ih; hh++) acc = acc + s_d[hh * SB + tid];
        const int b = b0 + tid;
        float score = acc / sqrtf((float)ihd);
        if ((long long)b * a.comp + a.comp - 1 > (long long)(a.offset + t)) score = -INFINITY;
        a.skey[(size_t)t * a.ldk + b] = qk_ordkey(score);
    }
}

struct AtSelArgs {
    const uint32_t *skey;   /* [n, ldk] */
    uint32_t *keep;         /* [n, kw] */
    int nb, btop, kw, ldk;
};

__global__ __launch_bounds__(AT_SEL_T) void k_at_sel(AtSelArgs a) {
    extern __shared__ float at_lds[];
    uint32_t *s_key = (uint32_t *)at_lds;              /* [nb] order keys of the scores */
    uint32_t *s_bits = s_key + a.nb;                   /* [kw] */
    int *s_hist = (int *)(s_bits + a.kw);              /* [256] */
    int *s_misc = s_hist + 256;                        /* [8] */
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, t = blockIdx.x;
    for (int i = tid; i < a.kw; i += AT_SEL_T) s_bits[i] = 0u;
    /* four key loads in flight per thread and round (a loop with a runtime
     * trip count would wait on each load) */
    const uint32_t *ksrc = a.skey + (size_t)t * a.ldk;
    for (int b0 = tid; b0 < a.nb; b0 += 4 * AT_SEL_T) {
        uint32_t v[4];
#pragma unroll
        for (int u = 0; u < 4; u++) v[u] = qk_ld(ksrc + min(b0 + AT_SEL_T * u, a.nb - 1));
#pragma unroll
        for (int u = 0; u < 4; u++)
            if (b0 + AT_SEL_T * u < a.nb) s_key[b0 + AT_SEL_T * u] = v[u];
    }
    __syncthreads();
    if (a.btop >= a.nb) {
        for (int b = tid; b < a.nb; b += AT_SEL_T) atomicOr(&s_bits[b >> 5], 1u << (b & 31));
    } else {
        /* radix select of the btop-th largest key, 8 bits a pass */
        uint32_t prefix = 0u, pmask = 0u;
        int need = a.btop;
        for (int shift = 24; shift >= 0; shift -= 8) {
            s_hist[tid] = 0;
            __syncthreads();
            for (int b = tid; b < a.nb; b += AT_SEL_T) {
                const uint32_t k = s_key[b];
                if ((k & pmask) == prefix) atomicAdd(&s_hist[(k >> shift) & 255], 1);
            }
            __syncthreads();
            if (wave == 0) {
                /* the digit where the count from the top first reaches
                 * need: lane l holds digits 255-4l .. 252-4l, an exclusive
                 * scan over the lanes, then the lane holding the crossing */
                int cnt[4], sum = 0;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    cnt[i] = s_hist[255 - 4 * lane - i];
                    sum += cnt[i];
                }
                int inc = sum;
                for (int o = 1; o < 64; o <<= 1) {
                    const int u = __shfl_up(inc, o, QK_WAVE);
                    if (lane >= o) inc += u;
                }
                const int before = inc - sum;
                if (before < need && inc >= need) {
                    int cum = before, i = 0;
                    while (i < 3 && cum + cnt[i] < need) cum += cnt[i++];
                    s_misc[0] = 255 - 4 * lane - i;
                    s_misc[1] = need - cum;
                } else if (lane == 63 && inc < need) { /* fewer keys than need: digit 0 */
                    s_misc[0] = 0;
                    s_misc[1] = need - (inc - cnt[3]);
                }
            }
            __syncthreads();
            prefix |= (uint32_t)s_misc[0] << shift;
            pmask |= 255u << shift;
            need = s_misc[1];
            __syncthreads();
        }
        /* keys above the threshold all, equal ones in block order up to need */
        const int per = (a.nb + AT_SEL_T - 1) / AT_SEL_T;
        const int b0 = tid * per;
        int eq = 0;
        for (int j = 0; j < per; j++) eq += (b0 + j < a.nb && s_key[b0 + j] == prefix) ? 1 : 0;
        /* exclusive scan of eq over the threads */
        int inc = eq;
        for (int o = 1; o < 64; o <<= 1) {
            const int u = __shfl_up(inc, o, QK_WAVE);
            if (lane >= o) inc += u;
        }
        if (lane == 63) s_hist[wave] = inc;
        __syncthreads();
        int base = 0;
        for (int w = 0; w < wave; w++) base += s_hist[w];
        int rank = base + inc - eq;
        for (int j = 0; j < per; j++) {
            const int b = b0 + j;
            if (b >= a.nb) break;
            const uint32_t k = s_key[b];
            bool kp = k > prefix;
            if (k == prefix) {
                kp = rank < need;
                rank++;
            }
            if (kp) atomicOr(&s_bits[b >> 5], 1u << (b & 31));
        }
    }
    __syncthreads();
    for (int i = tid; i < a.kw; i += AT_SEL_T) a.keep[(size_t)t * a.kw + i] = s_bits[i];
}

/* ------------------------------------------------------------ attention */

#define AT_CHUNK 256

struct AtAttnArgs {
    const float *qn;        /* [n, h, hd] */
    const float *k_cache, *v_cache;
    const uint32_t *keep;   /* [n, kw] or NULL */
    float *part;            /* [n, h, nchunks, hd + 2] */
    int h, kvh, hd, kv_total, offset, comp, nb, kw, nchunks;
};

#define AT_GMAX 8 /* query heads of one kv head per workgroup, at most */

/* grid (n * kvh * ngrp, nchunks): workgroup = (token t, kv head kh, group
 * of up to AT_GMAX of the heads kh, kh + kvh, ...) over 256 keys; thread
 * tid owns key c*256 + tid for the scores, wave w the keys w, w+4, .. for
 * the v sums; masked keys are not read.  Per head the arithmetic (fma chain
 * of q.k in dimension order, chunk max, exp, wave tree, the v sums per
 * wave, the waves added in order) is that of one head alone. */
__global__ __launch_bounds__(AT_CHUNK) void k_at_attn(AtAttnArgs a) {
    __shared__ float s_q[AT_GMAX][256];
    __shared__ float s_p[AT_GMAX][AT_CHUNK];
    __shared__ float s_red[4][AT_GMAX][256];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int G = a.h / a.kvh, ngrp = (G + AT_GMAX - 1) / AT_GMAX;
    const int t = blockIdx.x / (a.kvh * ngrp);
    const int r = blockIdx.x - t * a.kvh * ngrp, kh = r / ngrp, grp = r - kh * ngrp;
    const int j0 = grp * AT_GMAX, ng = min(AT_GMAX, G - j0);
    const int c = blockIdx.y, qpos = a.offset + t;
    const size_t kvw = (size_t)a.kvh * a.hd;
    for (int i = tid; i < AT_GMAX * a.hd; i += AT_CHUNK) {
        const int g = i / a.hd, d = i - g * a.hd;
        s_q[g][d] = g < ng ? qk_ld(a.qn + ((size_t)t * a.h + kh + (size_t)a.kvh * (j0 + g)) * a.hd + d) : 0.0f;
    }
    __syncthreads();
    const int ck = AT_CHUNK;
    const int kk = c * ck + tid;
    bool live = kk < a.kv_total && kk <= qpos;
    if (live && a.keep) {
        const int blk = kk / a.comp;
        bool kp = blk < a.nb && ((qk_ld(a.keep + (size_t)t * a.kw + (blk >> 5)) >> (blk & 31)) & 1u);
        const long long own = ((long long)(qpos + 1) / a.comp) * a.comp;
        if (kk >= own) kp = true;
        live = kp;
    }
    float sc[AT_GMAX];
    {
        float acc[AT_GMAX];
#pragma unroll
        for (int g = 0; g < AT_GMAX; g++) acc[g] = 0.0f;
        if (live) { /* masked keys are not read */
            const float4 *kr = (const float4 *)(a.k_cache + (size_t)kk * kvw + (size_t)kh * a.hd);
#pragma unroll 4
            for (int i = 0; i < a.hd / 4; i++) {
                const float4 k4 = qk_ld(kr + i);
#pragma unroll
                for (int g = 0; g < AT_GMAX; g++) {
                    acc[g] = fmaf(s_q[g][4 * i], k4.x, acc[g]);
                    acc[g] = fmaf(s_q[g][4 * i + 1], k4.y, acc[g]);
                    acc[g] = fmaf(s_q[g][4 * i + 2], k4.z, acc[g]);
                    acc[g] = fmaf(s_q[g][4 * i + 3], k4.w, acc[g]);
                }
            }
        }
#pragma unroll
        for (int g = 0; g < AT_GMAX; g++) sc[g] = live ? acc[g] * (1.0f / sqrtf((float)a.hd)) : -INFINITY;
    }
    /* per head: chunk max, exp, sum */
    float mg[AT_GMAX], lg[AT_GMAX];
#pragma unroll
    for (int g = 0; g < AT_GMAX; g++) {
        float m = sc[g];
        m = fmaxf(m, qk_dpp<QK_DPP_XOR1>(m));
        m = fmaxf(m, qk_dpp<QK_DPP_XOR2>(m));
        m = fmaxf(m, qk_dpp<QK_DPP_HALF_MIRROR>(m));
        m = fmaxf(m, qk_dpp<QK_DPP_MIRROR>(m));
        m = fmaxf(m, __uint_as_float(qk_xor16_u(__float_as_uint(m))));
        m = fmaxf(m, __uint_as_float(qk_xor32_u(__float_as_uint(m))));
        if (lane == 0) s_red[wave][g][0] = m;
    }
    __syncthreads();
#pragma unroll
    for (int g = 0; g < AT_GMAX; g++) {
        const float m = fmaxf(fmaxf(s_red[0][g][0], s_red[1][g][0]), fmaxf(s_red[2][g][0], s_red[3][g][0]));
        const float p = m == -INFINITY ? 0.0f : expf(sc[g] - m);
        s_p[g][tid] = p;
        mg[g] = m;
        lg[g] = qk_group_sum<64>(p);
    }
    __syncthreads(); /* s_red reused */
#pragma unroll
    for (int g = 0; g < AT_GMAX; g++)
        if (lane == 0) s_red[wave][g][1] = lg[g];
    __syncthreads();
#pragma unroll
    for (int g = 0; g < AT_GMAX; g++) lg[g] = ((s_red[0][g][1] + s_red[1][g][1]) + s_red[2][g][1]) + s_red[3][g][1];
    /* exp-weighted v: wave w takes the keys w, w+4, ...; lane the dims lane, lane+64, .. */
    float o[AT_GMAX][4];
#pragma unroll
    for (int g = 0; g < AT_GMAX; g++)
#pragma unroll
        for (int e = 0; e < 4; e++) o[g][e] = 0.0f;
    const int nk = min(ck, a.kv_total - c * ck);
#pragma unroll 8
    for (int j = wave; j < nk; j += 4) {
        /* a key with weight 0 for every head adds nothing: its row is not read */
        bool any = false;
#pragma unroll
        for (int g = 0; g < AT_GMAX; g++) any = any || s_p[g][j] != 0.0f;
        if (!any) continue;
        const float *vr = a.v_cache + (size_t)(c * ck + j) * kvw + (size_t)kh * a.hd;
        float vv[4];
#pragma unroll
        for (int e = 0; e < 4; e++) vv[e] = lane + 64 * e < a.hd ? qk_ld(vr + lane + 64 * e) : 0.0f;
#pragma unroll
        for (int g = 0; g < AT_GMAX; g++) {
            const float pj = s_p[g][j];
#pragma unroll
            for (int e = 0; e < 4; e++) o[g][e] = fmaf(pj, vv[e], o[g][e]);
        }
    }
    __syncthreads();
#pragma unroll
    for (int g = 0; g < AT_GMAX; g++)
#pragma unroll
        for (int e = 0; e < 4; e++)
            if (lane + 64 * e < a.hd) s_red[wave][g][lane + 64 * e] = o[g][e];
    __syncthreads();
    for (int g = 0; g < ng; g++) {
        const int hh = kh + a.kvh * (j0 + g);
        float *dst = a.part + (((size_t)t * a.h + hh) * a.nchunks + c) * (a.hd + 2);
        for (int i = tid; i < a.hd; i += AT_CHUNK)
            dst[2 + i] = ((s_red[0][g][i] + s_red[1][g][i]) + s_red[2][g][i]) + s_red[3][g][i];
        if (tid == 0) {
            dst[0] = mg[g];
            dst[1] = lg[g];
        }
    }
}

/* Calls of few tokens: chunks of 64 keys, so the cache spreads over many
 * workgroups (a token at 4096 cached keys: 65 chunks per kv head instead of
 * 17).  Four adjacent threads share a key, each an fma chain over a quarter
 * of its dims in order, added by a butterfly; each thread's k quarter and
 * its v rows (wave w: keys w, w+4, .., 16 of them) are loaded at the start,
 * with the query and the block mask, so the kernel waits on memory once.
 * A workgroup takes up to AT_G64 query heads, so a token's work spreads
 * over twice the workgroups of AT_GMAX.  Rows past the cache are loaded
 * clamped and never used. */
#define AT_C64 64
#define AT_HDMAX 256
#define AT_G64 4 /* query heads of one kv head per 64-key workgroup, at most */

__global__ __launch_bounds__(256) void k_at_attn64(AtAttnArgs a) {
    __shared__ float s_q[AT_G64][AT_HDMAX];
    __shared__ float s_p[AT_G64][AT_C64];
    __shared__ float s_red[4][AT_G64][AT_HDMAX];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int G = a.h / a.kvh, ngrp = (G + AT_G64 - 1) / AT_G64;
    const int t = blockIdx.x / (a.kvh * ngrp);
    const int r = blockIdx.x - t * a.kvh * ngrp, kh = r / ngrp, grp = r - kh * ngrp;
    const int j0 = grp * AT_G64, ng = min(AT_G64, G - j0);
    const int c = blockIdx.y, qpos = a.offset + t;
    const size_t kvw = (size_t)a.kvh * a.hd;
    const int kl = tid >> 2, part = tid & 3; /* key of the chunk, quarter of its dims */
    const int kk = c * AT_C64 + kl;
    const int nq = a.hd >> 4; /* float4 steps of a quarter */
    /* k quarter of the thread's key */
    float4 kr[AT_HDMAX / 16];
    {
        const float4 *src = (const float4 *)(a.k_cache + (size_t)min(kk, a.kv_total - 1) * kvw +
                                             (size_t)kh * a.hd) + part * nq;
#pragma unroll
        for (int i = 0; i < AT_HDMAX / 16; i++)
            if (i < nq) kr[i] = qk_ld(src + i);
    }
    /* v rows of the wave's keys, the lane's dims lane, lane + 64, .. */
    const int nk = min(AT_C64, a.kv_total - c * AT_C64);
    float vr[AT_C64 / 4][AT_HDMAX / 64];
#pragma unroll
    for (int i = 0; i < AT_C64 / 4; i++) {
        const float *src = a.v_cache + (size_t)(c * AT_C64 + min(wave + 4 * i, nk - 1)) * kvw + (size_t)kh * a.hd;
#pragma unroll
        for (int e = 0; e < AT_HDMAX / 64; e++)
            if (lane + 64 * e < a.hd) vr[i][e] = qk_ld(src + lane + 64 * e);
    }
    uint32_t kw_word = 0;
    if (a.keep && kk < a.kv_total && kk / a.comp < a.nb) kw_word = qk_ld(a.keep + (size_t)t * a.kw + ((kk / a.comp) >> 5));
    for (int i = tid; i < AT_G64 * a.hd; i += 256) {
        const int g = i / a.hd, d = i - g * a.hd;
        s_q[g][d] = g < ng ? qk_ld(a.qn + ((size_t)t * a.h + kh + (size_t)a.kvh * (j0 + g)) * a.hd + d) : 0.0f;
    }
    __syncthreads();
    bool live = kk < a.kv_total && kk <= qpos;
    if (live && a.keep) {
        const int blk = kk / a.comp;
        bool kp = blk < a.nb && ((kw_word >> (blk & 31)) & 1u);
        const long long own = ((long long)(qpos + 1) / a.comp) * a.comp;
        if (kk >= own) kp = true;
        live = kp;
    }
    float sc[AT_G64];
    {
        float acc[AT_G64];
#pragma unroll
        for (int g = 0; g < AT_G64; g++) acc[g] = 0.0f;
#pragma unroll
        for (int i = 0; i < AT_HDMAX / 16; i++)
            if (i < nq) {
                const int d = 4 * (part * nq + i);
#pragma unroll
                for (int g = 0; g < AT_G64; g++) {
                    acc[g] = fmaf(s_q[g][d], kr[i].x, acc[g]);
                    acc[g] = fmaf(s_q[g][d + 1], kr[i].y, acc[g]);
                    acc[g] = fmaf(s_q[g][d + 2], kr[i].z, acc[g]);
                    acc[g] = fmaf(s_q[g][d + 3], kr[i].w, acc[g]);
                }
            }
        /* the four quarters of a key (adjacent lanes), added by a butterfly */
#pragma unroll
        for (int g = 0; g < AT_G64; g++) {
            acc[g] += qk_dpp<QK_DPP_XOR1>(acc[g]);
            acc[g] += qk_dpp<QK_DPP_XOR2>(acc[g]);
            sc[g] = live ? acc[g] * (1.0f / sqrtf((float)a.hd)) : -INFINITY;
        }
    }
    float mg[AT_G64], lg[AT_G64];
#pragma unroll
    for (int g = 0; g < AT_G64; g++) {
        float m = sc[g];
        m = fmaxf(m, qk_dpp<QK_DPP_XOR1>(m));
        m = fmaxf(m, qk_dpp<QK_DPP_XOR2>(m));
        m = fmaxf(m, qk_dpp<QK_DPP_HALF_MIRROR>(m));
        m = fmaxf(m, qk_dpp<QK_DPP_MIRROR>(m));
        m = fmaxf(m, __uint_as_float(qk_xor16_u(__float_as_uint(m))));
        m = fmaxf(m, __uint_as_float(qk_xor32_u(__float_as_uint(m))));
        if (lane == 0) s_red[wave][g][0] = m;
    }
    __syncthreads();
#pragma unroll
    for (int g = 0; g < AT_G64; g++) {
        const float m = fmaxf(fmaxf(s_red[0][g][0], s_red[1][g][0]), fmaxf(s_red[2][g][0], s_red[3][g][0]));
        /* the first quarter of each key carries its weight */
        const float p = (m == -INFINITY || part != 0) ? 0.0f : expf(sc[g] - m);
        if (part == 0) s_p[g][kl] = p;
        mg[g] = m;
        lg[g] = qk_group_sum<64>(p);
    }
    __syncthreads(); /* s_red reused, s_p complete */
#pragma unroll
    for (int g = 0; g < AT_G64; g++)
        if (lane == 0) s_red[wave][g][1] = lg[g];
    float o[AT_G64][AT_HDMAX / 64];
#pragma unroll
    for (int g = 0; g < AT_G64; g++)
#pragma unroll
        for (int e = 0; e < AT_HDMAX / 64; e++) o[g][e] = 0.0f;
#pragma unroll
    for (int i = 0; i < AT_C64 / 4; i++) {
        const int j = wave + 4 * i;
        if (j < nk) {
#pragma unroll
            for (int g = 0; g < AT_G64; g++) {
                const float pj = s_p[g][j];
#pragma unroll
                for (int e = 0; e < AT_HDMAX / 64; e++) o[g][e] = fmaf(pj, vr[i][e], o[g][e]);
            }
        }
    }
    __syncthreads();
#pragma unroll
    for (int g = 0; g < AT_G64; g++) lg[g] = ((s_red[0][g][1] + s_red[1][g][1]) + s_red[2][g][1]) + s_red[3][g][1];
    __syncthreads(); /* s_red[.][.][1] read before the v sums overwrite it */
#pragma unroll
    for (int g = 0; g < AT_G64; g++)
#pragma unroll
        for (int e = 0; e < AT_HDMAX / 64; e++)
            if (lane + 64 * e < a.hd) s_red[wave][g][lane + 64 * e] = o[g][e];
    __syncthreads();
    for (int g = 0; g < ng; g++) {
        const int hh = kh + a.kvh * (j0 + g);
        float *dst = a.part + (((size_t)t * a.h + hh) * a.nchunks + c) * (a.hd + 2);
        for (int i = tid; i < a.hd; i += 256)
            dst[2 + i] = ((s_red[0][g][i] + s_red[1][g][i]) + s_red[2][g][i]) + s_red[3][g][i];
        if (tid == 0) {
            dst[0] = mg[g];
            dst[1] = lg[g];
        }
    }
}

struct AtCombArgs {
    const float *part;      /* [n, h, nchunks, hd + 2] */
    const float *qg;        /* [n, 2h*hd] */
    float *ao;              /* [n, h*hd] */
    int h, hd, nchunks;
};

#define AT_MAXCH 128 /* chunks of 64 keys: kv_cap <= 8192 */

/* one workgroup per (token, head): the chunks' maxima give M; wave w sums
 * the chunks w, w+4, .. in order, each with factor exp(max - M) (a chunk
 * with every key masked, max -inf and sums 0, enters with factor 0 and
 * leaves the sums unchanged), lane the dims lane, lane + 64, ..; the four
 * waves' sums are added in order */
template <int CPW> /* chunks per wave, at most: AT_MAXCH / 4 or 8 (256-key chunks) */
__global__ __launch_bounds__(256) void k_at_comb(AtCombArgs a) {
    __shared__ float s_m[AT_MAXCH];
    __shared__ float s_o[4][AT_HDMAX + 1];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, th = blockIdx.x;
    const int t = th / a.h, hh = th - t * a.h;
    const size_t cw = (size_t)a.hd + 2;
    const float *pp = a.part + (size_t)th * a.nchunks * cw;
    if (tid < AT_MAXCH) s_m[tid] = tid < a.nchunks ? qk_ld(pp + (size_t)tid * cw) : -INFINITY;
    __syncthreads();
    float M = fmaxf(s_m[lane], s_m[lane + 64]);
    M = fmaxf(M, qk_dpp<QK_DPP_XOR1>(M));
    M = fmaxf(M, qk_dpp<QK_DPP_XOR2>(M));
    M = fmaxf(M, qk_dpp<QK_DPP_HALF_MIRROR>(M));
    M = fmaxf(M, qk_dpp<QK_DPP_MIRROR>(M));
    M = fmaxf(M, __uint_as_float(qk_xor16_u(__float_as_uint(M))));
    M = fmaxf(M, __uint_as_float(qk_xor32_u(__float_as_uint(M))));
    /* every partial of the wave's chunks is loaded before the sums start
     * (a loop over a runtime count would wait for each chunk in turn) */
    float lv[CPW], vv[CPW][AT_HDMAX / 64];
#pragma unroll
    for (int i = 0; i < CPW; i++) {
        const int ci = wave + 4 * i;
        if (ci < a.nchunks) {
            const float *q = pp + (size_t)ci * cw;
            lv[i] = qk_ld(q + 1);
#pragma unroll
            for (int e = 0; e < AT_HDMAX / 64; e++)
                if (lane + 64 * e < a.hd) vv[i][e] = qk_ld(q + 2 + lane + 64 * e);
        }
    }
    float L = 0.0f;
    float o[AT_HDMAX / 64];
#pragma unroll
    for (int e = 0; e < AT_HDMAX / 64; e++) o[e] = 0.0f;
#pragma unroll
    for (int i = 0; i < CPW; i++) {
        const int ci = wave + 4 * i;
        if (ci < a.nchunks) {
            const float f = expf(s_m[ci] - M);
            L = fmaf(lv[i], f, L);
#pragma unroll
            for (int e = 0; e < AT_HDMAX / 64; e++)
                if (lane + 64 * e < a.hd) o[e] = fmaf(vv[i][e], f, o[e]);
        }
    }
#pragma unroll
    for (int e = 0; e < AT_HDMAX / 64; e++)
        if (lane + 64 * e < a.hd) s_o[wave][lane + 64 * e] = o[e];
    if (lane == 0) s_o[wave][AT_HDMAX] = L;
    __syncthreads();
    const float Ls = ((s_o[0][AT_HDMAX] + s_o[1][AT_HDMAX]) + s_o[2][AT_HDMAX]) + s_o[3][AT_HDMAX];
    const float inv = 1.0f / Ls;
    const float *g = a.qg + (size_t)t * 2 * a.h * a.hd + (size_t)hh * 2 * a.hd + a.hd;
    for (int i = tid; i < a.hd; i += 256) {
        const float v = ((s_o[0][i] + s_o[1][i]) + s_o[2][i]) + s_o[3][i];
        a.ao[(size_t)th * a.hd + i] = (v * inv) * (1.0f / (1.0f + expf(-qk_ld(g + i))));
    }
}

/* ------------------------------------------------------------ host side */

static int at_rows_launch(RowsArgs &r, hipStream_t st) {
    const int rows = r.start[r.nseg];
    const int waves = (rows + AT_RPW - 1) / AT_RPW;
    const dim3 grid((waves + 3) / 4);
    const bool inj = r.hyper != nullptr;
#define AT_ROWS_L(P)                                                                  \
    do {                                                                              \
        if (inj) hipLaunchKernelGGL((k_rows<P, true>), grid, dim3(256), 0, st, r);    \
        else hipLaunchKernelGGL((k_rows<P, false>), grid, dim3(256), 0, st, r);       \
    } while (0)
    switch ((r.K / 32 + 63) / 64) {
    case 1: AT_ROWS_L(1); break;
    case 2: AT_ROWS_L(2); break;
    case 3: AT_ROWS_L(3); break;
    default: AT_ROWS_L(4); break;
    }
#undef AT_ROWS_L
    return QK_CHECK_LAUNCH();
}

static void at_seg(RowsArgs &r, const uint32_t *q, const uint16_t *s, const uint16_t *b, const uint16_t *w,
                   int rows, float *out, int ostride) {
    RowSeg &g = r.seg[r.nseg];
    g.q = q; g.s = s; g.b = b; g.w = w; g.out = out; g.rows = rows; g.ostride = ostride;
    r.start[r.nseg + 1] = r.start[r.nseg] + rows;
    r.nseg++;
}

extern "C" int qk_at_shape_ok(const qk_at_shape *s) {
    if (s->d <= 0 || s->d % 64 || s->d > 8192) return 0;
    if (s->h <= 0 || s->kvh <= 0 || s->h % s->kvh) return 0;
    if (s->hd <= 0 || s->hd % 64 || s->hd > 256 || (s->h * s->hd) % 64 || s->h * s->hd > 8192) return 0;
    if (s->ih <= 0 || s->ih > 64 || s->ihd <= 0 || s->ihd % 4 || s->ihd > 256 || s->ih * s->ihd > 8192) return 0;
    if (s->rot < 0 || s->rot % 2 || s->rot > s->hd || s->rot > s->ihd) return 0;
    if (s->cap <= 0 || s->cap > 8192 || s->comp <= 0 || s->budget <= 0) return 0;
    return 1;
}

extern "C" size_t qk_at_sel_lds(const qk_at_shape *s, int nb) {
    const int kw = (nb + 31) / 32;
    (void)s;
    return ((size_t)nb + kw + 256 + 8) * 4;
}

extern "C" int qk_launch_at(const qk_at_shape *s, const qk_at_dev *W, const float *x, int n, int offset,
                            int pos0, int len0, float *out, float *k_cache, float *v_cache, float *idx_keys,
                            float *pooled, const qk_at_scratch *sc, const qk_inject *inj, void *stream) {
    if (n <= 0) return 0;
    if (inj && inj->hyper && (inj->hc < 1 || inj->hc > QK_INJECT_MAX_HC || !inj->inject))
        return (int)hipErrorInvalidValue;
    if (!qk_at_shape_ok(s)) return (int)hipErrorInvalidValue;
    hipStream_t st = (hipStream_t)stream;
    const int h = s->h, kvh = s->kvh, hd = s->hd, ih = s->ih, ihd = s->ihd;
    const int kv_total = len0 + n;
    const int use_idx = kv_total > s->budget;

    RowsArgs r;
    r.nseg = 0;
    r.start[0] = 0;
    r.x = x;
    r.K = s->d;
    r.n = n;
    r.hyper = nullptr;
    r.inject = nullptr;
    r.hc = 1;
    at_seg(r, W->q_q, W->q_s, W->q_b, nullptr, 2 * h * hd, sc->qg, 2 * h * hd);
    at_seg(r, W->k_q, W->k_s, W->k_b, nullptr, kvh * hd, sc->kraw, kvh * hd);
    at_seg(r, W->v_q, W->v_s, W->v_b, nullptr, kvh * hd, sc->vraw, kvh * hd);
    at_seg(r, nullptr, nullptr, nullptr, W->idx_w, (ih + 1) * ihd, sc->qk, (ih + 1) * ihd);
    int rc = at_rows_launch(r, st);
    if (rc) return rc;

    AtQkArgs q;
    q.qg = sc->qg; q.kraw = sc->kraw; q.vraw = sc->vraw; q.qk = sc->qk;
    q.q_norm = W->q_norm; q.k_norm = W->k_norm; q.iq_norm = W->idx_q_norm;
    q.qn = sc->qn; q.k_cache = k_cache; q.v_cache = v_cache; q.idx_keys = idx_keys;
    q.qi = use_idx ? sc->qi : nullptr;
    q.n = n; q.h = h; q.kvh = kvh; q.hd = hd; q.ih = ih; q.ihd = ihd; q.len0 = len0;
    q.offset = offset; q.rot = s->rot; q.rope = (const float2 *)W->rope;
    hipLaunchKernelGGL(k_at_qk, dim3(n, h + kvh + (use_idx ? ih : 0)), dim3(64), 0, st, q);
    rc = QK_CHECK_LAUNCH();
    if (rc) return rc;

    /* the pooled keys of the blocks this call completes, whether or not
     * the block mask runs yet */
    const int pb0 = len0 / s->comp, pb1 = kv_total / s->comp;
    if (pb1 > pb0) {
        AtPoolArgs pa;
        pa.idx_keys = idx_keys; pa.ik_norm = W->idx_k_norm; pa.pooled = pooled;
        pa.ihd = ihd; pa.comp = s->comp; pa.b0 = pb0; pa.b1 = pb1; pa.rot = s->rot; pa.rope = (const float2 *)W->rope;
        pa.pos0 = pos0;
        hipLaunchKernelGGL(k_at_pool, dim3((pb1 - pb0 + 3) / 4), dim3(256), 0, st, pa);
        rc = QK_CHECK_LAUNCH();
        if (rc) return rc;
    }
    const int nb = use_idx ? kv_total / s->comp : 0;
    const int kw = (nb + 31) / 32;
    const int ldk = s->cap / s->comp;
    if (use_idx && nb > 0) {
        AtScoreArgs ka;
        ka.pooled = pooled; ka.qi = sc->qi; ka.skey = sc->skey;
        ka.ih = ih; ka.ihd = ihd; ka.comp = s->comp; ka.nb = nb; ka.ldk = ldk; ka.offset = offset - pos0;
        hipLaunchKernelGGL(k_at_score, dim3(n, (nb + AT_SB - 1) / AT_SB), dim3(256), at_score_lds(ih, ihd), st, ka);
        rc = QK_CHECK_LAUNCH();
        if (rc) return rc;
        AtSelArgs e;
        e.skey = sc->skey; e.keep = sc->keep;
        e.nb = nb; e.btop = s->budget / s->comp; e.kw = kw; e.ldk = ldk;
        hipLaunchKernelGGL(k_at_sel, dim3(n), dim3(AT_SEL_T), qk_at_sel_lds(s, nb), st, e);
        rc = QK_CHECK_LAUNCH();
        if (rc) return rc;
    }

    AtAttnArgs at;
    at.qn = sc->qn; at.k_cache = k_cache; at.v_cache = v_cache;
    at.keep = use_idx ? sc->keep : nullptr;
    at.part = sc->part;
    at.h = h; at.kvh = kvh; at.hd = hd; at.kv_total = kv_total; at.offset = offset - pos0;
    at.comp = s->comp; at.nb = nb; at.kw = kw;
    const int ngrp = (h / kvh + AT_GMAX - 1) / AT_GMAX;
    /* 64-key chunks while 256-key ones leave the grid under 512 workgroups
     * and the partials of 64-key chunks fit the scratch */
    const long long n64 = (kv_total + AT_C64 - 1) / AT_C64;
    const bool c64 = (long long)n * kvh * ngrp * ((kv_total + AT_CHUNK - 1) / AT_CHUNK) < 512 &&
                     n * n64 <= sc->part_units && n64 <= AT_MAXCH;
    at.nchunks = c64 ? (int)n64 : (kv_total + AT_CHUNK - 1) / AT_CHUNK;
    if ((long long)n * at.nchunks > sc->part_units) return (int)hipErrorInvalidValue;
    const int ngrp64 = (h / kvh + AT_G64 - 1) / AT_G64;
    if (c64) hipLaunchKernelGGL(k_at_attn64, dim3(n * kvh * ngrp64, at.nchunks), dim3(256), 0, st, at);
    else hipLaunchKernelGGL(k_at_attn, dim3(n * kvh * ngrp, at.nchunks), dim3(AT_CHUNK), 0, st, at);
    rc = QK_CHECK_LAUNCH();
    if (rc) return rc;

    AtCombArgs cb;
    cb.part = sc->part; cb.qg = sc->qg; cb.ao = sc->ao; cb.h = h; cb.hd = hd; cb.nchunks = at.nchunks;
    if (at.nchunks <= 32) hipLaunchKernelGGL(k_at_comb<8>, dim3(n * h), dim3(256), 0, st, cb);
    else hipLaunchKernelGGL(k_at_comb<AT_MAXCH / 4>, dim3(n * h), dim3(256), 0, st, cb);
    rc = QK_CHECK_LAUNCH();
    if (rc) return rc;

    RowsArgs o;
    o.nseg = 0;
    o.start[0] = 0;
    o.x = sc->ao;
    o.K = h * hd;
    o.n = n;
    o.hyper = inj ? inj->hyper : nullptr;
    o.inject = inj ? inj->inject : nullptr;
    o.hc = inj && inj->hyper ? inj->hc : 1;
    at_seg(o, W->o_q, W->o_s, W->o_b, nullptr, s->d, out, s->d);
    return at_rows_launch(o, st);
}
