/*
 * dn_oracle.c -- CPU restatement of the reference C port's gated DeltaNet
 * mixer (c/src/model.c:1146-1278, deltanet_forward), the linear-attention
 * layer of the decoder.  TEST INFRASTRUCTURE ONLY (the checker of the HIP
 * DeltaNet kernels); nothing in the product links it.
 *
 * Followed step by step, with the arithmetic of model.c and kernel.c:
 *   mixed = in_proj_qkv(x), z = in_proj_z(x)     model.c:1168-1170 (gemm_q4)
 *   a = x.Wa^T, b = x.Wb^T                       model.c:1172-1175 (gemm_bf16)
 *   conv over [conv_state; mixed], state <- last k-1 rows
 *                                                model.c:1177-1186, kernel.c:311-324
 *   silu                                         model.c:1187, kernel.c:38-43
 *   q, k, v split; l2norm(q), l2norm(k), q *= dk^-1/2
 *                                                model.c:1202-1222, kernel.c:73-78, 53-55
 *   recurrence per value head                    model.c:1225-1248
 *   rmsnorm(out) * norm_w * sigmoid(z)           model.c:1263-1274, kernel.c:10-20
 *   out = out_proj(.)                            model.c:1276 (gemm_q4)
 * Multiply-adds of the form acc += a*b are fma chains, as the reference's
 * compiler contracts them (the convention of moe_oracle.c).
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "moe_oracle.h"

/* kernel_conv1d_depthwise for the rows the layer keeps (kernel.c:311-324
 * with d = 1): y[t, c] = sum_i seq[t + i, c] * w[c, i], i ascending */
static void conv_rows(const float *seq, int n, int ch, const uint16_t *w, int k, float *y) {
    for (int t = 0; t < n; t++)
        for (int c = 0; c < ch; c++) {
            float acc = 0.0f;
            for (int i = 0; i < k; i++)
                acc = fmaf(seq[(size_t)(t + i) * ch + c], orc_bf16_to_f32(w[(size_t)c * k + i]), acc);
            y[(size_t)t * ch + c] = acc;
        }
}

/* kernel_l2norm (kernel.c:73-78) */
static void l2norm(float *x, int n, float eps) {
    float ss = 0.0f;
    for (int i = 0; i < n; i++) ss = fmaf(x[i], x[i], ss);
    const float r = 1.0f / sqrtf(ss + eps);
    for (int i = 0; i < n; i++) x[i] = x[i] * r;
}

float orc_dn_decay(float a_log, float a, float dt_bias) {
    return expf(-expf(a_log) * log1pf(expf(a + dt_bias)));
}

int orc_dn_forward(const orc_dn *D, const float *x, int n, float *out, float *conv_state,
                   float *rec_state, float *core_out) {
    const int d = D->hidden, hk = D->n_k_heads, hv = D->n_v_heads;
    const int dk = D->k_head_dim, dv = D->v_head_dim, kc = D->conv_kernel, gs = D->group_size;
    const int key_dim = hk * dk, value_dim = hv * dv, conv_dim = 2 * key_dim + value_dim;
    const int repeat = hv / hk;
    if (n <= 0) return 0;
    float *mixed = (float *)malloc((size_t)n * conv_dim * sizeof(float));
    float *z = (float *)malloc((size_t)n * value_dim * sizeof(float));
    float *a = (float *)malloc((size_t)n * hv * sizeof(float));
    float *b = (float *)malloc((size_t)n * hv * sizeof(float));
    float *seq = (float *)malloc((size_t)(kc - 1 + n) * conv_dim * sizeof(float));
    float *co = (float *)malloc((size_t)n * conv_dim * sizeof(float));
    float *o = (float *)malloc((size_t)n * value_dim * sizeof(float));
    if (!mixed || !z || !a || !b || !seq || !co || !o) {
        free(mixed), free(z), free(a), free(b), free(seq), free(co), free(o);
        return -1;
    }
    orc_gemm_q4(n, conv_dim, d, x, D->qkv_q, D->qkv_s, D->qkv_b, gs, mixed);
    orc_gemm_q4(n, value_dim, d, x, D->z_q, D->z_s, D->z_b, gs, z);
    orc_gemm_bf16(n, hv, d, x, D->a_w, a);
    orc_gemm_bf16(n, hv, d, x, D->b_w, b);

    memcpy(seq, conv_state, (size_t)(kc - 1) * conv_dim * sizeof(float));
    memcpy(seq + (size_t)(kc - 1) * conv_dim, mixed, (size_t)n * conv_dim * sizeof(float));
    memcpy(conv_state, seq + (size_t)n * conv_dim, (size_t)(kc - 1) * conv_dim * sizeof(float));
    conv_rows(seq, n, conv_dim, D->conv_w, kc, co);
    for (size_t i = 0; i < (size_t)n * conv_dim; i++) co[i] = orc_silu(co[i]);

    const float scale_q = 1.0f / sqrtf((float)dk);
    for (int t = 0; t < n; t++) {
        float *row = co + (size_t)t * conv_dim;
        for (int h = 0; h < hk; h++) {
            float *q = row + (size_t)h * dk, *k = row + key_dim + (size_t)h * dk;
            l2norm(q, dk, 1e-6f);
            l2norm(k, dk, 1e-6f);
            for (int i = 0; i < dk; i++) q[i] = q[i] * scale_q;
        }
    }

    for (int t = 0; t < n; t++) {
        const float *row = co + (size_t)t * conv_dim;
        for (int h = 0; h < hv; h++) {
            const int kh = h / repeat;
            const float gv = orc_dn_decay(D->a_log[h], a[(size_t)t * hv + h], D->dt_bias[h]);
            const float beta = 1.0f / (1.0f + expf(-b[(size_t)t * hv + h]));
            const float *q = row + (size_t)kh * dk, *k = row + key_dim + (size_t)kh * dk;
            const float *v = row + 2 * key_dim + (size_t)h * dv;
            float *S = rec_state + (size_t)h * dv * dk;
            for (int r = 0; r < dv; r++) {
                float *s = S + (size_t)r * dk;
                float kv = 0.0f;
                for (int i = 0; i < dk; i++) {
                    s[i] = s[i] * gv;
                    kv = fmaf(s[i], k[i], kv);
                }
                const float delta = (v[r] - kv) * beta;
                float acc = 0.0f;
                for (int i = 0; i < dk; i++) s[i] = fmaf(k[i], delta, s[i]);
                for (int i = 0; i < dk; i++) acc = fmaf(s[i], q[i], acc);
                o[(size_t)t * value_dim + (size_t)h * dv + r] = acc;
            }
        }
    }
    if (core_out) memcpy(core_out, o, (size_t)n * value_dim * sizeof(float));

    for (int t = 0; t < n; t++)
        for (int h = 0; h < hv; h++) {
            float *orow = o + (size_t)t * value_dim + (size_t)h * dv;
            const float *zrow = z + (size_t)t * value_dim + (size_t)h * dv;
            float ss = 0.0f;
            for (int i = 0; i < dv; i++) ss = fmaf(orow[i], orow[i], ss);
            const float r = 1.0f / sqrtf(ss / (float)dv + 1e-6f);
            for (int i = 0; i < dv; i++) orow[i] = orow[i] * r * D->norm_w[i];
            for (int i = 0; i < dv; i++) orow[i] = orow[i] * (1.0f / (1.0f + expf(-zrow[i])));
        }
    orc_gemm_q4(n, d, value_dim, o, D->out_q, D->out_s, D->out_b, gs, out);
    free(mixed), free(z), free(a), free(b), free(seq), free(co), free(o);
    return 0;
}
