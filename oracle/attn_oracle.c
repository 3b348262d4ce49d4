/*
 * attn_oracle.c -- CPU restatement of the reference C port's full-attention
 * mixer with the QSA indexer (c/src/model.c:798-1144, attention_forward).
 * TEST INFRASTRUCTURE ONLY (the checker of the HIP attention kernels);
 * nothing in the product links it.
 *
 * Followed step by step, with the arithmetic of model.c and kernel.c:
 *   qk = x.idx_w^T (gemm_bf16, here in the router's R64 order); its raw key
 *   row appended to the indexer key cache                model.c:807-843
 *   q (+ gate, interleaved per head), k, v = q4 projections;
 *   v appended to its cache                              model.c:847-869
 *   per-head rmsnorm(q_norm / k_norm) then partial RoPE at positions
 *   offset + t; k appended to its cache                  model.c:871-937
 *   scores = q.k / sqrt(hd) (kv head = head % kv_heads), causal mask
 *   kk > offset + t                                       model.c:951-967
 *   past the indexer budget: mean-pooled key blocks (rmsnorm, RoPE at the
 *   block start), per-token indexer queries (rmsnorm, RoPE), block scores
 *   sum_heads sum_i relu(q_i p_i) / sqrt(idx_hd), invisible blocks -inf,
 *   top budget/compress blocks (kernel_topk_indices; exact ties at the
 *   k-th score to the lower block), keys outside the kept blocks and the
 *   own tail masked                                      model.c:969-1104
 *   softmax, weighted sum of v, * sigmoid(gate), o_proj   model.c:1107-1143
 * Multiply-adds of the form acc += a*b are fma chains (the convention of
 * moe_oracle.c); the ReLU products of the block scores are not contracted.
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "moe_oracle.h"

static void rmsnorm_w(const float *x, const float *w, int n, float *y) {
    float ss = 0.0f;
    for (int i = 0; i < n; i++) ss = fmaf(x[i], x[i], ss);
    const float r = 1.0f / sqrtf(ss / (float)n + 1e-6f);
    for (int i = 0; i < n; i++) y[i] = x[i] * r * w[i];
}

/* kernel_rope_partial (kernel.c:80-93) on one row of n values, the first d rotated */
static void rope_row(float *x, int n, int d, const float *cs, const float *sn) {
    const int half = d / 2;
    for (int i = 0; i < half; i++) {
        const float x0 = x[i], x1 = x[i + half];
        x[i] = x0 * cs[i] - x1 * sn[i];
        x[i + half] = x0 * sn[i] + x1 * cs[i];
    }
    (void)n;
}

int orc_attn_forward(const orc_attn *A, orc_attn_state *S, const float *x, int n, int offset,
                     float *out) {
    return orc_attn_forward_dbg(A, S, x, n, offset, out, NULL);
}

int orc_attn_forward_dbg(const orc_attn *A, orc_attn_state *S, const float *x, int n, int offset,
                         float *out, const orc_attn_dbg *dbg) {
    const int d = A->hidden, h = A->n_heads, kvh = A->n_kv_heads, hd = A->head_dim;
    const int ih = A->idx_heads, ihd = A->idx_head_dim, cap = A->kv_cap, gs = A->group_size;
    const int idx_out = ih * ihd, qkw = idx_out + ihd;
    if (n <= 0) return 0;
    /* past the capacity the reference drops the oldest rows of the v and
     * indexer caches but not of the k cache (model.c:815-821, 862-867,
     * 921), which misaligns k and v.  Without slide only calls that fit
     * are restated; with slide the oldest rows of all three caches go
     * together, idx_compress rows at a time, and positions are absolute
     * (base + row) */
    int pos0 = 0;
    if (A->slide) {
        if (offset != S->base + S->kv_len || S->kv_len != S->idx_len) return -3;
        if (S->kv_len + n > cap) {
            const int over = S->kv_len + n - cap;
            const int drop = (over + A->idx_compress - 1) / A->idx_compress * A->idx_compress;
            if (drop > S->kv_len) return -2;
            const size_t kr = (size_t)kvh * hd;
            memmove(S->k_cache, S->k_cache + (size_t)drop * kr, (size_t)(S->kv_len - drop) * kr * sizeof(float));
            memmove(S->v_cache, S->v_cache + (size_t)drop * kr, (size_t)(S->kv_len - drop) * kr * sizeof(float));
            memmove(S->idx_keys, S->idx_keys + (size_t)drop * ihd,
                    (size_t)(S->idx_len - drop) * ihd * sizeof(float));
            S->kv_len -= drop;
            S->idx_len -= drop;
            S->base += drop;
        }
        pos0 = S->base;
    }
    if (S->kv_len + n > cap || S->idx_len + n > cap) return -2;
    float *qk = (float *)malloc((size_t)n * qkw * sizeof(float));
    float *qbuf = (float *)malloc((size_t)n * h * hd * 2 * sizeof(float));
    float *kbuf = (float *)malloc((size_t)n * kvh * hd * sizeof(float));
    float *vbuf = (float *)malloc((size_t)n * kvh * hd * sizeof(float));
    float *qn = (float *)malloc((size_t)n * h * hd * sizeof(float));
    float *kn = (float *)malloc((size_t)n * kvh * hd * sizeof(float));
    float *ao = (float *)malloc((size_t)n * h * hd * sizeof(float));
    const int rot = (int)((float)hd * A->rotary_factor);
    float *rc = (float *)malloc((size_t)n * (rot / 2 + 1) * sizeof(float));
    float *rs = (float *)malloc((size_t)n * (rot / 2 + 1) * sizeof(float));
    float *inv = (float *)malloc((size_t)(rot / 2 + 1) * sizeof(float));
    if (!qk || !qbuf || !kbuf || !vbuf || !qn || !kn || !ao || !rc || !rs || !inv) return -1;

    /* index_qk_proj in the router's fixed R64 order (the reference's
     * gemm_bf16 leaves its order to BNNS) */
    for (int t = 0; t < n; t++)
        for (int r = 0; r < qkw; r++)
            qk[(size_t)t * qkw + r] = orc_dot_r64_bf16w(x + (size_t)t * d, A->idx_w + (size_t)r * d, d);
    for (int t = 0; t < n; t++)
        memcpy(S->idx_keys + (size_t)(S->idx_len + t) * ihd, qk + (size_t)t * qkw + idx_out,
               (size_t)ihd * sizeof(float));
    S->idx_len += n;

    orc_gemm_q4(n, h * hd * 2, d, x, A->q_q, A->q_s, A->q_b, gs, qbuf);
    orc_gemm_q4(n, kvh * hd, d, x, A->k_q, A->k_s, A->k_b, gs, kbuf);
    orc_gemm_q4(n, kvh * hd, d, x, A->v_q, A->v_s, A->v_b, gs, vbuf);
    memcpy(S->v_cache + (size_t)S->kv_len * kvh * hd, vbuf, (size_t)n * kvh * hd * sizeof(float));
    const int kv_total = S->kv_len + n;
    S->kv_len = kv_total;

    for (int i = 0; i < rot / 2; i++) inv[i] = powf(A->rope_theta, -(2.0f * (float)i) / (float)rot);
    for (int t = 0; t < n; t++)
        for (int i = 0; i < rot / 2; i++) {
            const float ang = (float)(offset + t) * inv[i];
            rc[(size_t)t * (rot / 2) + i] = cosf(ang);
            rs[(size_t)t * (rot / 2) + i] = sinf(ang);
        }
    for (int t = 0; t < n; t++) {
        const float *c = rc + (size_t)t * (rot / 2), *s = rs + (size_t)t * (rot / 2);
        for (int hh = 0; hh < h; hh++) {
            float *q = qn + ((size_t)t * h + hh) * hd;
            rmsnorm_w(qbuf + (size_t)t * h * hd * 2 + (size_t)hh * hd * 2, A->q_norm, hd, q);
            rope_row(q, hd, rot, c, s);
        }
        for (int hh = 0; hh < kvh; hh++) {
            float *k = kn + ((size_t)t * kvh + hh) * hd;
            rmsnorm_w(kbuf + ((size_t)t * kvh + hh) * hd, A->k_norm, hd, k);
            rope_row(k, hd, rot, c, s);
        }
    }
    memcpy(S->k_cache + (size_t)(kv_total - n) * kvh * hd, kn, (size_t)n * kvh * hd * sizeof(float));

    float *sc = (float *)malloc((size_t)kv_total * sizeof(float));
    unsigned char *keep_blk = NULL;
    const int use_idx = kv_total > A->idx_budget;
    const int comp = A->idx_compress;
    const int n_blocks = use_idx ? kv_total / comp : 0;
    const int btop = use_idx ? A->idx_budget / comp : 0;
    float *pooled = NULL, *bsc = NULL, *qs = NULL;
    int *top = NULL;
    if (use_idx) {
        pooled = (float *)malloc((size_t)n_blocks * ihd * sizeof(float));
        bsc = (float *)malloc((size_t)n_blocks * sizeof(float));
        qs = (float *)malloc((size_t)ih * ihd * sizeof(float));
        top = (int *)malloc((size_t)(btop > 0 ? btop : 1) * sizeof(int));
        keep_blk = (unsigned char *)malloc((size_t)n_blocks);
        float *tmp = (float *)malloc((size_t)ihd * sizeof(float));
        for (int b = 0; b < n_blocks; b++) {
            const float *blk = S->idx_keys + (size_t)b * comp * ihd;
            for (int i = 0; i < ihd; i++) {
                float acc = 0.0f;
                for (int j = 0; j < comp; j++) acc = acc + blk[(size_t)j * ihd + i];
                tmp[i] = acc / (float)comp;
            }
            rmsnorm_w(tmp, A->idx_k_norm, ihd, pooled + (size_t)b * ihd);
            float bc[512], bs[512];
            for (int i = 0; i < rot / 2; i++) {
                const float ang = (float)(pos0 + b * comp) * inv[i];
                bc[i] = cosf(ang);
                bs[i] = sinf(ang);
            }
            rope_row(pooled + (size_t)b * ihd, ihd, rot, bc, bs);
        }
        free(tmp);
        if (dbg && dbg->pooled) memcpy(dbg->pooled, pooled, (size_t)n_blocks * ihd * sizeof(float));
    }
    for (int t = 0; t < n; t++) {
        if (use_idx) {
            const float *c = rc + (size_t)t * (rot / 2), *s = rs + (size_t)t * (rot / 2);
            for (int hh = 0; hh < ih; hh++) {
                rmsnorm_w(qk + (size_t)t * qkw + (size_t)hh * ihd, A->idx_q_norm, ihd, qs + (size_t)hh * ihd);
                rope_row(qs + (size_t)hh * ihd, ihd, rot, c, s);
            }
            if (dbg && dbg->qs) memcpy(dbg->qs + (size_t)t * ih * ihd, qs, (size_t)ih * ihd * sizeof(float));
            for (int b = 0; b < n_blocks; b++) {
                float acc = 0.0f;
                const float *pb = pooled + (size_t)b * ihd;
                for (int hh = 0; hh < ih; hh++) {
                    float dot = 0.0f;
                    for (int i = 0; i < ihd; i++) {
                        const float v = qs[(size_t)hh * ihd + i] * pb[i];
                        dot = dot + (v > 0 ? v : 0);
                    }
                    acc = acc + dot;
                }
                bsc[b] = acc / sqrtf((float)ihd);
                if ((long long)pos0 + (long long)b * comp + comp - 1 > (long long)offset + t) bsc[b] = -INFINITY;
            }
            /* kernel_topk_indices (quickselect) fixes the k-th largest
             * score T; the blocks above T are kept whichever way it
             * partitions, and among the blocks equal to T (exact ties,
             * -inf ones included) the lowest ids are kept: the canonical
             * tie rule, where the reference's choice depends on its
             * partitioning order */
            orc_topk_quickselect(bsc, n_blocks, btop, top);
            memset(keep_blk, 0, (size_t)n_blocks);
            if (btop >= n_blocks) {
                memset(keep_blk, 1, (size_t)n_blocks);
            } else if (btop > 0) {
                float T = bsc[top[0]] + 0.0f;
                for (int j = 1; j < btop; j++)
                    if (bsc[top[j]] + 0.0f < T) T = bsc[top[j]] + 0.0f;
                int kept = 0;
                for (int b = 0; b < n_blocks; b++)
                    if (bsc[b] + 0.0f > T) keep_blk[b] = 1, kept++;
                for (int b = 0; b < n_blocks && kept < btop; b++)
                    if (bsc[b] + 0.0f == T) keep_blk[b] = 1, kept++;
            }
            if (dbg && dbg->scores) memcpy(dbg->scores + (size_t)t * n_blocks, bsc, (size_t)n_blocks * sizeof(float));
            if (dbg && dbg->keep) memcpy(dbg->keep + (size_t)t * n_blocks, keep_blk, (size_t)n_blocks);
        }
        for (int hh = 0; hh < h; hh++) {
            const int kh = hh % kvh;
            const float *q = qn + ((size_t)t * h + hh) * hd;
            for (int kk = 0; kk < kv_total; kk++) {
                const float *k = S->k_cache + (size_t)kk * kvh * hd + (size_t)kh * hd;
                float acc = 0.0f;
                for (int i = 0; i < hd; i++) acc = fmaf(q[i], k[i], acc);
                sc[kk] = acc * (1.0f / sqrtf((float)hd));
                if (pos0 + kk > offset + t) sc[kk] = -INFINITY;
            }
            if (use_idx) {
                const long long own_start = ((long long)(offset + t + 1) / comp) * comp;
                for (int kk = 0; kk < kv_total; kk++) {
                    const int blk = kk / comp;
                    int keep = blk < n_blocks && keep_blk[blk];
                    if (pos0 + kk >= own_start && pos0 + kk <= offset + t) keep = 1;
                    if (!keep && pos0 + kk <= offset + t) sc[kk] = -INFINITY;
                }
            }
            /* kernel_softmax (kernel.c:61-71) */
            float m = sc[0];
            for (int kk = 1; kk < kv_total; kk++)
                if (sc[kk] > m) m = sc[kk];
            float sum = 0.0f;
            for (int kk = 0; kk < kv_total; kk++) {
                sc[kk] = expf(sc[kk] - m);
                sum = sum + sc[kk];
            }
            const float is = 1.0f / sum;
            for (int kk = 0; kk < kv_total; kk++) sc[kk] = sc[kk] * is;
            float *o = ao + ((size_t)t * h + hh) * hd;
            for (int i = 0; i < hd; i++) {
                float acc = 0.0f;
                for (int kk = 0; kk < kv_total; kk++)
                    acc = fmaf(sc[kk], S->v_cache[(size_t)kk * kvh * hd + (size_t)kh * hd + i], acc);
                o[i] = acc;
            }
            const float *g = qbuf + (size_t)t * h * hd * 2 + (size_t)hh * hd * 2 + hd;
            for (int i = 0; i < hd; i++) o[i] = o[i] * (1.0f / (1.0f + expf(-g[i])));
        }
    }
    orc_gemm_q4(n, d, h * hd, ao, A->o_q, A->o_s, A->o_b, gs, out);
    free(sc), free(pooled), free(bsc), free(qs), free(top), free(keep_blk);
    free(qk), free(qbuf), free(kbuf), free(vbuf), free(qn), free(kn), free(ao), free(rc), free(rs), free(inv);
    return 0;
}
