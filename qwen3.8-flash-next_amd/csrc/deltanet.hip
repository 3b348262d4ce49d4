/*
 * deltanet.hip -- the gated DeltaNet mixer (linear attention) on gfx950,
 * replacing deltanet_forward of the reference C port (c/src/model.c:
 * 1146-1278) for n tokens in three launches:
 *
 *   k_dn_in   one wave per four rows of [in_proj_qkv | in_proj_z | in_proj_a
 *             | in_proj_b]: the q4 rows with the per-group identity of
 *             gemm_q4 (kernel.c:279-282, gemv_parts.h), the bf16 rows as
 *             dot products of bf16 pairs; x (f32) enters as bf16 hi + lo
 *             pairs.  Writes mixed [n, conv_dim], z [n, value_dim], a, b
 *             [n, hv].
 *   k_dn_rec  one workgroup per (value head, block of 16 state rows), the
 *             state rows in registers across the tokens: per token the
 *             causal depthwise conv over [conv_state; mixed] (kernel.c:
 *             311-324) + silu for the head's q and k channels and its v
 *             rows, l2norm(q)*dk^-1/2 and l2norm(k) (kernel.c:73-78), the
 *             decay exp(-exp(A_log) softplus(a + dt_bias)) and beta =
 *             sigmoid(b), then per row S <- g S; kv = S.k; S += k (beta
 *             (v - kv)); o = S.q (model.c:1225-1248).  Writes o [n, value_dim]
 *             and the new recurrent state.
 *             The gated norm rmsnorm(o_h) * norm_w * sigmoid(z_h) (model.c:
 *             1263-1274) is split: k_dn_rec writes o * norm_w * sigmoid(z)
 *             per row and the sum of o^2 over its rows.
 *   k_dn_out  one wave per two rows of out_proj (q4); each lane scales its
 *             own columns by the head's 1/sqrt(sum(o^2)/dv + eps); also
 *             moves the conv state on by n tokens (its old rows are read by
 *             k_dn_rec, so it changes only here).
 *
 * Sums run in parallel orders (lane trees), so results match the reference
 * to rounding, not bit for bit.
 */
#include "qk_device.h"
#include "gemv_parts.h"

#define DN_RPW 4   /* rows per wave in the two GEMV kernels */
#define DN_RB 16   /* state rows per recurrence workgroup */

struct DnInArgs {
    const uint32_t *qkv_q, *z_q;
    const uint16_t *qkv_s, *qkv_b, *z_s, *z_b;
    const uint16_t *a_w, *b_w;
    const float *x;  /* [n, d] */
    float *mixed;    /* [n, conv_dim] */
    float *z;        /* [n, value_dim] */
    float *a, *b;    /* [n, hv] */
    int d, n, conv_dim, value_dim, hv;
};

/* x chunks of token t as bf16 pairs: lane owns chunks ps*64 + lane */
template <int P>
__device__ __forceinline__ void dn_x_pairs(const float *x, int t, int K, int lane, XPairs<64, P, false> &xp) {
    XRaw<P, false> xr;
    load_xraw<64, P, false>(x, (size_t)t, K, lane, xr);
    convert_xraw<64, P, false>(xr, K, lane, xp);
}

template <int P>
__global__ __launch_bounds__(256) void k_dn_in(DnInArgs a) {
    const int lane = threadIdx.x & 63;
    const int r0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * DN_RPW;
    const int R1 = a.conv_dim, R2 = R1 + a.value_dim, R3 = R2 + a.hv, R = R3 + a.hv;
    if (r0 >= R) return;
    const int CH = a.d >> 5, G = a.d >> 6;
    const size_t wrow = (size_t)a.d >> 3;
    if (r0 < R2) {
        /* q4 rows: codes, scales and biases of the wave's rows stay in registers */
        uint4 wq[DN_RPW][P];
        float ws[DN_RPW][P], wb[DN_RPW][P];
#pragma unroll
        for (int j = 0; j < DN_RPW; j++) {
            const int r = min(r0 + j, R2 - 1);
            const bool z = r >= R1;
            const int rr = z ? r - R1 : r;
            const uint32_t *q = (z ? a.z_q : a.qkv_q) + (size_t)rr * wrow;
            const uint16_t *s = (z ? a.z_s : a.qkv_s) + (size_t)rr * G;
            const uint16_t *bb = (z ? a.z_b : a.qkv_b) + (size_t)rr * G;
#pragma unroll
            for (int ps = 0; ps < P; ps++) {
                const int c0 = ps * 64 + lane;
                const bool ok = c0 < CH;
                const int c = ok ? c0 : 0;
                wq[j][ps] = qk_ld((const uint4 *)(q + 4 * (size_t)c));
                ws[j][ps] = ok ? qk_bf16(qk_ld(s + (c >> 1))) : 0.0f;
                wb[j][ps] = ok ? qk_bf16(qk_ld(bb + (c >> 1))) : 0.0f;
                if (!ok) wq[j][ps] = make_uint4(0u, 0u, 0u, 0u);
            }
        }
        for (int t = 0; t < a.n; t++) {
            XPairs<64, P, false> xp;
            dn_x_pairs<P>(a.x, t, a.d, lane, xp);
#pragma unroll
            for (int j = 0; j < DN_RPW; j++) {
                const float v = qk_group_sum<64>(row_part<64, P, false>(wq[j], ws[j], wb[j], xp));
                const int r = r0 + j;
                if (lane == 0 && r < R2) {
                    if (r < R1) qk_st(a.mixed + (size_t)t * a.conv_dim + r, v);
                    else qk_st(a.z + (size_t)t * a.value_dim + (r - R1), v);
                }
            }
        }
        return;
    }
    /* bf16 rows (in_proj_a, in_proj_b): w pairs against the x pairs */
    for (int t = 0; t < a.n; t++) {
        XPairs<64, P, false> xp;
        dn_x_pairs<P>(a.x, t, a.d, lane, xp);
#pragma unroll
        for (int j = 0; j < DN_RPW; j++) {
            const int r = r0 + j;
            const int rc = min(r, R - 1);
            const bool isb = rc >= R3;
            const uint16_t *w = (isb ? a.b_w : a.a_w) + (size_t)(isb ? rc - R3 : rc - R2) * a.d;
            float part = 0.0f;
#pragma unroll
            for (int ps = 0; ps < P; ps++) {
                const int c0 = ps * 64 + lane;
                const bool ok = c0 < CH;
                const uint4 *src = (const uint4 *)(w + 32 * (size_t)(ok ? c0 : 0));
#pragma unroll
                for (int g = 0; g < 4; g++) {
                    uint32_t wp[4];
                    qk_bf16x8_to_pairs(qk_ld(src + g), wp);
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const uint32_t w2 = ok ? wp[i] : 0u;
                        part = qk_dot2(xp.hi[ps][4 * g + i], w2, part);
                        part = qk_dot2(xp.lo[ps][4 * g + i], w2, part);
                    }
                }
            }
            const float v = qk_group_sum<64>(part);
            if (lane == 0 && r < R) {
                if (r < R3) qk_st(a.a + (size_t)t * a.hv + (r - R2), v);
                else qk_st(a.b + (size_t)t * a.hv + (r - R3), v);
            }
        }
    }
}

/* ------------------------------------------------------------ recurrence */

struct DnRecArgs {
    const float *mixed, *a, *b;  /* [n, conv_dim], [n, hv], [n, hv] */
    const float *conv_state;     /* [kc-1, conv_dim], the state before these tokens */
    const uint16_t *conv_w;      /* [conv_dim, kc] */
    const float *a_log, *dt_bias;
    const float *z;              /* [n, value_dim] */
    const float *norm_w;         /* [dv] */
    float *rec_state;            /* [hv, dv, dk] */
    float *core;                 /* [n, value_dim]: o * norm_w * sigmoid(z) */
    float *ssp;                  /* [n, hv, dv/16]: sums of o^2 over each block's rows */
    int n, hk, hv, dk, dv, kc, conv_dim;
};

/* silu(conv) of channels ch[0..NC) at token t: sum over taps i of
 * w[c, i] * seq[t+i, c] with seq = [conv_state rows; mixed rows], the fma
 * chain over i ascending.  The taps come four at a time with every load of
 * a round (all NC channels) in flight: a loop with a runtime trip count
 * would wait on each load.  Past kc the last tap is read again, unused. */
template <int NC>
__device__ __forceinline__ void dn_conv_silu(const DnRecArgs &a, int t, const int (&ch)[NC], float (&out)[NC]) {
    float acc[NC];
#pragma unroll
    for (int c = 0; c < NC; c++) acc[c] = 0.0f;
    for (int i0 = 0; i0 < a.kc; i0 += 4) {
        float sv[NC][4];
        uint16_t wv[NC][4];
#pragma unroll
        for (int c = 0; c < NC; c++)
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const int i = min(i0 + u, a.kc - 1), j = t + i;
                const float *src = j < a.kc - 1 ? a.conv_state + (size_t)j * a.conv_dim + ch[c]
                                                : a.mixed + (size_t)(j - (a.kc - 1)) * a.conv_dim + ch[c];
                sv[c][u] = qk_ld(src);
                wv[c][u] = qk_ld(a.conv_w + (size_t)ch[c] * a.kc + i);
            }
#pragma unroll
        for (int c = 0; c < NC; c++)
#pragma unroll
            for (int u = 0; u < 4; u++)
                if (i0 + u < a.kc) acc[c] = fmaf(sv[c][u], qk_bf16(wv[c][u]), acc[c]);
    }
#pragma unroll
    for (int c = 0; c < NC; c++) out[c] = qk_silu(acc[c]);
}

template <int EPL>
__global__ __launch_bounds__(256) void k_dn_rec(DnRecArgs a) {
    constexpr int DK = 16 * EPL;
    __shared__ float s_ch[2 * DK + DN_RB]; /* q, k, v of the block's rows */
    __shared__ float s_sc[4];              /* q and k norms, decay, beta */
    __shared__ float s_o[DN_RB];           /* the block's outputs of this token */
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int h = blockIdx.y, rb = blockIdx.x * DN_RB;
    const int kh = h / (a.hv / a.hk);
    const int key_dim = a.hk * DK, value_dim = a.hv * a.dv;
    const int row = rb + (tid >> 4), i0 = (tid & 15) * EPL;
    float *srow = a.rec_state + ((size_t)h * a.dv + row) * DK + i0;
    float s[EPL];
    if (EPL % 4 == 0) {
#pragma unroll
        for (int e = 0; e < EPL; e += 4) {
            const float4 v = qk_ld((const float4 *)(srow + e));
            s[e] = v.x; s[e + 1] = v.y; s[e + 2] = v.z; s[e + 3] = v.w;
        }
    } else {
#pragma unroll
        for (int e = 0; e < EPL; e++) s[e] = qk_ld(srow + e);
    }
    const float al = expf(qk_ld(a.a_log + h)), dtb = qk_ld(a.dt_bias + h);
    const float scale_q = 1.0f / sqrtf((float)DK);
    for (int t = 0; t < a.n; t++) {
        /* what the token's later steps read, loaded with the channels' taps
         * (every thread loads them; the addresses are shared) */
        const size_t zi = (size_t)t * value_dim + (size_t)h * a.dv + row;
        const float zv = qk_ld(a.z + zi), nwv = qk_ld(a.norm_w + row);
        const float av = qk_ld(a.a + (size_t)t * a.hv + h), bv = qk_ld(a.b + (size_t)t * a.hv + h);
        {
            /* the block's q, k, v channels, NCC per thread (all their loads
             * in flight); past the last one a thread repeats it */
            constexpr int NCC = (2 * DK + DN_RB + 255) / 256;
            int ch[NCC];
#pragma unroll
            for (int u = 0; u < NCC; u++) {
                const int c = min(tid + 256 * u, 2 * DK + DN_RB - 1);
                ch[u] = c < DK ? kh * DK + c
                      : c < 2 * DK ? key_dim + kh * DK + (c - DK)
                                   : 2 * key_dim + h * a.dv + rb + (c - 2 * DK);
            }
            float v[NCC];
            dn_conv_silu<NCC>(a, t, ch, v);
#pragma unroll
            for (int u = 0; u < NCC; u++)
                if (tid + 256 * u < 2 * DK + DN_RB) s_ch[tid + 256 * u] = v[u];
        }
        __syncthreads();
        if (wave < 2) {
            /* wave 0: |q|^2, wave 1: |k|^2 */
            float ss = 0.0f;
            for (int i = lane; i < DK; i += 64) {
                const float v = s_ch[wave * DK + i];
                ss = fmaf(v, v, ss);
            }
            ss = qk_group_sum<64>(ss);
            if (lane == 0) s_sc[wave] = 1.0f / sqrtf(ss + 1e-6f);
        } else if (tid == 128) {
            s_sc[2] = expf(-al * log1pf(expf(av + dtb)));
            s_sc[3] = 1.0f / (1.0f + expf(-bv));
        }
        __syncthreads();
        const float rq = s_sc[0], rk = s_sc[1], g = s_sc[2], beta = s_sc[3];
        float kk[EPL], qq[EPL];
#pragma unroll
        for (int e = 0; e < EPL; e++) {
            kk[e] = s_ch[DK + i0 + e] * rk;
            qq[e] = (s_ch[i0 + e] * rq) * scale_q;
        }
        float kv = 0.0f;
#pragma unroll
        for (int e = 0; e < EPL; e++) {
            s[e] = s[e] * g;
            kv = fmaf(s[e], kk[e], kv);
        }
        kv = qk_group_sum<16>(kv);
        const float delta = (s_ch[2 * DK + (tid >> 4)] - kv) * beta;
        float o = 0.0f;
#pragma unroll
        for (int e = 0; e < EPL; e++) {
            s[e] = fmaf(kk[e], delta, s[e]);
            o = fmaf(s[e], qq[e], o);
        }
        o = qk_group_sum<16>(o);
        if ((tid & 15) == 0) {
            /* the gated norm's row factors here, its head factor (from the
             * sums of squares) in k_dn_out */
            qk_st(a.core + zi, (o * nwv) * (1.0f / (1.0f + expf(-zv))));
            s_o[tid >> 4] = o;
        }
        __syncthreads();
        if (tid == 0) {
            float ss = 0.0f;
            for (int j = 0; j < DN_RB; j++) ss = fmaf(s_o[j], s_o[j], ss);
            qk_st(a.ssp + ((size_t)t * a.hv + h) * (a.dv / DN_RB) + blockIdx.x, ss);
        }
        __syncthreads(); /* s_ch, s_sc, s_o are rewritten for the next token */
    }
    if (EPL % 4 == 0) {
#pragma unroll
        for (int e = 0; e < EPL; e += 4)
            qk_st((float4 *)(srow + e), make_float4(s[e], s[e + 1], s[e + 2], s[e + 3]));
    } else {
#pragma unroll
        for (int e = 0; e < EPL; e++) qk_st(srow + e, s[e]);
    }
}

/* ------------------------------------------------------------ out_proj */

struct DnOutArgs {
    const uint32_t *out_q;
    const uint16_t *out_s, *out_b;
    const float *core;         /* [n, value_dim]: o * norm_w * sigmoid(z) */
    const float *ssp;          /* [n, hv, dv/16] */
    const float *mixed;        /* [n, conv_dim] */
    float *conv_state;         /* [kc-1, conv_dim], moved on by n tokens */
    float *out;                /* [n, d] */
    float *hyper;              /* INJ: [n, hc, d], hyper[t, j] += inject[t, j] * out[t] */
    const float *inject;       /* INJ: [n, hc] */
    int n, d, value_dim, dv, kc, conv_dim, ch_per_wg, hc;
};

#define DN_ORW 2 /* out_proj rows per wave */

#define DN_KCMAX 16 /* conv taps at most */
#define DN_NBU 16   /* sums-of-squares partials per head loaded at once */

/*
 * One wave per DN_ORW rows of out_proj.  The gated norm's head factor
 * r = 1/sqrt(sum(o^2)/dv + eps) comes from the per-block sums of squares
 * of k_dn_rec (dv/16 of them per head, loaded together and added in
 * order); each lane scales its own chunks (32 columns of one head) and
 * splits them into bf16 hi + lo pairs.  The code words are loaded first;
 * the conv state moves on at the end (its stores would otherwise hold the
 * loads back).  No LDS and no barrier.
 */
template <int P, bool INJ>
__global__ __launch_bounds__(256) void k_dn_out(DnOutArgs a) {
    const int tid = threadIdx.x, lane = tid & 63;
    const int K = a.value_dim, CH = K >> 5, G = K >> 6;
    const size_t wrow = (size_t)K >> 3;

    /* the conv state: channels [c0, c0 + ch_per_wg) move on by n tokens;
     * every new value is read now, written at the end */
    const int cc = blockIdx.x * a.ch_per_wg + tid;
    const bool cthr = tid < a.ch_per_wg && cc < a.conv_dim;
    float cv[DN_KCMAX - 1];
    if (cthr) {
#pragma unroll
        for (int j = 0; j < DN_KCMAX - 1; j++)
            if (j < a.kc - 1) {
                const int m = a.n + j;
                cv[j] = m < a.kc - 1 ? a.conv_state[(size_t)m * a.conv_dim + cc]
                                     : qk_ld(a.mixed + (size_t)(m - (a.kc - 1)) * a.conv_dim + cc);
            }
    }

    const int r0 = (blockIdx.x * 4 + (tid >> 6)) * DN_ORW;
    if (r0 < a.d) {
    uint4 wq[DN_ORW][P];
    float ws[DN_ORW][P], wb[DN_ORW][P];
#pragma unroll
    for (int j = 0; j < DN_ORW; j++) {
        const int r = min(r0 + j, a.d - 1);
#pragma unroll
        for (int ps = 0; ps < P; ps++) {
            const int c0 = ps * 64 + lane;
            const bool ok = c0 < CH;
            const int c = ok ? c0 : 0;
            wq[j][ps] = qk_ld((const uint4 *)(a.out_q + (size_t)r * wrow + 4 * (size_t)c));
            ws[j][ps] = ok ? qk_bf16(qk_ld(a.out_s + (size_t)r * G + (c >> 1))) : 0.0f;
            wb[j][ps] = ok ? qk_bf16(qk_ld(a.out_b + (size_t)r * G + (c >> 1))) : 0.0f;
            if (!ok) wq[j][ps] = make_uint4(0u, 0u, 0u, 0u);
        }
    }
    for (int t = 0; t < a.n; t++) {
        /* INJ: the token's inject weights and the hyper values of this
         * wave's rows, loaded before the row sums (clamped addresses) */
        float iv[INJ ? QK_INJECT_MAX_HC : 1], hv[INJ ? DN_ORW : 1][INJ ? QK_INJECT_MAX_HC : 1];
        if (INJ) {
#pragma unroll
            for (int j = 0; j < QK_INJECT_MAX_HC; j++) {
                const int jc = min(j, a.hc - 1);
                iv[INJ ? j : 0] = qk_ld(a.inject + (size_t)t * a.hc + jc);
#pragma unroll
                for (int q = 0; q < DN_ORW; q++)
                    hv[INJ ? q : 0][INJ ? j : 0] =
                        qk_ld(a.hyper + ((size_t)t * a.hc + jc) * a.d + min(r0 + q, a.d - 1));
            }
        }
        XRaw<P, false> xr;
#pragma unroll
        for (int ps = 0; ps < P; ps++) {
            const int c0 = ps * 64 + lane;
            const bool ok = c0 < CH;
            const int c = ok ? c0 : 0;
            const float4 *o = (const float4 *)(a.core + (size_t)t * K + 32 * c);
            const int head = (32 * c) / a.dv, nb = a.dv / DN_RB;
            const float *sp = a.ssp + ((size_t)t * (K / a.dv) + head) * nb;
            float ss = 0.0f;
            for (int j0 = 0; j0 < nb; j0 += DN_NBU) {
                float pv[DN_NBU];
#pragma unroll
                for (int j = 0; j < DN_NBU; j++) pv[j] = qk_ld(sp + min(j0 + j, nb - 1));
#pragma unroll
                for (int j = 0; j < DN_NBU; j++) ss = ss + (j0 + j < nb ? pv[j] : 0.0f);
            }
            const float r = 1.0f / sqrtf(ss / (float)a.dv + 1e-6f);
#pragma unroll
            for (int w = 0; w < 8; w++) {
                const float4 v = qk_ld(o + w);
                xr.f[ps][w] = make_float4(v.x * r, v.y * r, v.z * r, v.w * r);
            }
        }
        XPairs<64, P, false> xp;
        convert_xraw<64, P, false>(xr, K, lane, xp);
#pragma unroll
        for (int j = 0; j < DN_ORW; j++) {
            const float v = qk_group_sum<64>(row_part<64, P, false>(wq[j], ws[j], wb[j], xp));
            const int rr = r0 + j;
            if (lane == 0 && rr < a.d) {
                if (a.out) qk_st(a.out + (size_t)t * a.d + rr, v);
                if (INJ)
#pragma unroll
                    for (int q = 0; q < QK_INJECT_MAX_HC; q++)
                        if (q < a.hc)
                            qk_st(a.hyper + ((size_t)t * a.hc + q) * a.d + rr,
                                  fmaf(iv[INJ ? q : 0], v, hv[INJ ? j : 0][INJ ? q : 0]));
            }
        }
    }
    }
    if (cthr) {
#pragma unroll
        for (int j = 0; j < DN_KCMAX - 1; j++)
            if (j < a.kc - 1) a.conv_state[(size_t)j * a.conv_dim + cc] = cv[j];
    }
}

/* ------------------------------------------------------------ host side */

extern "C" int qk_dn_shape_ok(const qk_dn_shape *s) {
    const int key_dim = s->hk * s->dk, value_dim = s->hv * s->dv;
    const int conv_dim = 2 * key_dim + value_dim;
    if (s->d <= 0 || s->d % 64 || s->d > 8192) return 0;
    if (s->hk <= 0 || s->hv <= 0 || s->hv % s->hk) return 0;
    if (!(s->dk == 32 || s->dk == 64 || s->dk == 128 || s->dk == 256)) return 0;
    /* dv: a power-of-two count (<= 64) of 32-column chunks */
    if (!(s->dv == 32 || s->dv == 64 || s->dv == 128 || s->dv == 256 || s->dv == 512 ||
          s->dv == 1024 || s->dv == 2048))
        return 0;
    /* out_proj takes value_dim inputs in q4 groups of 64 */
    if (value_dim > 8192 || value_dim % 64) return 0;
    if (s->kc < 1 || s->kc > 16) return 0;
    if (conv_dim <= 0) return 0;
    return 1;
}

extern "C" int qk_launch_dn(const qk_dn_shape *s, const qk_dn_dev *W, const float *x, int n, float *out,
                            float *conv_state, float *rec_state, float *mixed, float *z, float *av,
                            float *bv, float *core, float *ssp, const qk_inject *inj_in, void *stream) {
    if (n <= 0) return 0;
    if (!qk_dn_shape_ok(s)) return (int)hipErrorInvalidValue;
    hipStream_t st = (hipStream_t)stream;
    const int key_dim = s->hk * s->dk, value_dim = s->hv * s->dv;
    const int conv_dim = 2 * key_dim + value_dim;

    DnInArgs ia;
    ia.qkv_q = W->qkv_q; ia.qkv_s = W->qkv_s; ia.qkv_b = W->qkv_b;
    ia.z_q = W->z_q; ia.z_s = W->z_s; ia.z_b = W->z_b;
    ia.a_w = W->a_w; ia.b_w = W->b_w;
    ia.x = x; ia.mixed = mixed; ia.z = z; ia.a = av; ia.b = bv;
    ia.d = s->d; ia.n = n; ia.conv_dim = conv_dim; ia.value_dim = value_dim; ia.hv = s->hv;
    const int rows = conv_dim + value_dim + 2 * s->hv;
    const int waves = (rows + DN_RPW - 1) / DN_RPW;
    const dim3 igrid((waves + 3) / 4);
    const int p_in = (s->d / 32 + 63) / 64;
    switch (p_in) {
    case 1: hipLaunchKernelGGL(k_dn_in<1>, igrid, dim3(256), 0, st, ia); break;
    case 2: hipLaunchKernelGGL(k_dn_in<2>, igrid, dim3(256), 0, st, ia); break;
    case 3: hipLaunchKernelGGL(k_dn_in<3>, igrid, dim3(256), 0, st, ia); break;
    default: hipLaunchKernelGGL(k_dn_in<4>, igrid, dim3(256), 0, st, ia); break;
    }
    int rc = QK_CHECK_LAUNCH();
    if (rc) return rc;

    DnRecArgs ra;
    ra.mixed = mixed; ra.a = av; ra.b = bv;
    ra.conv_state = conv_state; ra.conv_w = W->conv_w;
    ra.a_log = W->a_log; ra.dt_bias = W->dt_bias;
    ra.z = z; ra.norm_w = W->norm_w;
    ra.rec_state = rec_state; ra.core = core; ra.ssp = ssp;
    ra.n = n; ra.hk = s->hk; ra.hv = s->hv; ra.dk = s->dk; ra.dv = s->dv; ra.kc = s->kc;
    ra.conv_dim = conv_dim;
    const dim3 rgrid(s->dv / DN_RB, s->hv);
    switch (s->dk) {
    case 32: hipLaunchKernelGGL(k_dn_rec<2>, rgrid, dim3(256), 0, st, ra); break;
    case 64: hipLaunchKernelGGL(k_dn_rec<4>, rgrid, dim3(256), 0, st, ra); break;
    case 128: hipLaunchKernelGGL(k_dn_rec<8>, rgrid, dim3(256), 0, st, ra); break;
    default: hipLaunchKernelGGL(k_dn_rec<16>, rgrid, dim3(256), 0, st, ra); break;
    }
    rc = QK_CHECK_LAUNCH();
    if (rc) return rc;

    DnOutArgs oa;
    oa.out_q = W->out_q; oa.out_s = W->out_s; oa.out_b = W->out_b;
    oa.core = core; oa.ssp = ssp; oa.mixed = mixed;
    oa.conv_state = conv_state; oa.out = out;
    const bool inj = inj_in && inj_in->hyper;
    if (inj && (inj_in->hc < 1 || inj_in->hc > QK_INJECT_MAX_HC || !inj_in->inject)) return (int)hipErrorInvalidValue;
    oa.hyper = inj ? inj_in->hyper : nullptr;
    oa.inject = inj ? inj_in->inject : nullptr;
    oa.hc = inj ? inj_in->hc : 1;
    oa.n = n; oa.d = s->d; oa.value_dim = value_dim; oa.dv = s->dv; oa.kc = s->kc;
    oa.conv_dim = conv_dim;
    const int owgs = (s->d + 4 * DN_ORW - 1) / (4 * DN_ORW);
    oa.ch_per_wg = (conv_dim + owgs - 1) / owgs;
    if (oa.ch_per_wg > 256) return (int)hipErrorInvalidValue;
    const int p_out = (value_dim / 32 + 63) / 64;
    switch (p_out) {
#define DN_OUT_L(P)                                                                          \
    do {                                                                                     \
        if (inj) hipLaunchKernelGGL((k_dn_out<P, true>), dim3(owgs), dim3(256), 0, st, oa);  \
        else hipLaunchKernelGGL((k_dn_out<P, false>), dim3(owgs), dim3(256), 0, st, oa);     \
    } while (0)
    case 1: DN_OUT_L(1); break;
    case 2: DN_OUT_L(2); break;
    case 3: DN_OUT_L(3); break;
    default: DN_OUT_L(4); break;
#undef DN_OUT_L
    }
    return QK_CHECK_LAUNCH();
}

/* a fill kernel for the state (graph capture records no memset node) */
__global__ __launch_bounds__(256) void k_dn_zero(float *p, size_t count) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i < count) p[i] = 0.0f;
}

extern "C" int qk_launch_dn_zero(float *p, size_t count, void *stream) {
    if (count == 0) return 0;
    hipLaunchKernelGGL(k_dn_zero, dim3((unsigned)((count + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                       p, count);
    return QK_CHECK_LAUNCH();
}
