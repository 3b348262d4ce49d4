/*
 * qmoe_dn.c -- C11 host side of the gated DeltaNet mixer: context, HBM
 * residency of each layer's weights and states, argument checks, and the
 * three launches of deltanet.hip.  Replaces deltanet_forward
 * (c/src/model.c:1146-1278) and the state handling around it
 * (model.c:341, 368-369, 402-403).
 */
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <hip/hip_runtime_api.h>

#include "qmoe_internal.h"

#define DN_ALIGN 256u

/* tensors of a layer allocation, in order */
enum { DT_QKV_Q, DT_QKV_S, DT_QKV_B, DT_Z_Q, DT_Z_S, DT_Z_B, DT_A_W, DT_B_W, DT_OUT_Q, DT_OUT_S,
       DT_OUT_B, DT_CONV_W, DT_NORM_W, DT_A_LOG, DT_DT_BIAS, DT_CONV_STATE, DT_REC_STATE, DT_COUNT };

typedef struct {
    void *mem;
    int ready;
} dn_layer;

struct qmoe_dn_ctx {
    qmoe_dn_config cfg;
    qk_dn_shape shape;
    int device;
    size_t off[DT_COUNT + 1], bytes[DT_COUNT];
    dn_layer *layers;
    void *scratch;
    float *mixed, *z, *a, *b, *core, *ssp;
};

static void dn_set_err(qmoe_err *err, const char *fmt, ...) {
    if (!err) return;
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(err->msg, sizeof(err->msg), fmt, ap);
    va_end(ap);
}

static int dn_hip_fail(qmoe_err *err, int rc, const char *what) {
    if (rc == 0) return 0;
    dn_set_err(err, "%s: HIP error %d (%s)", what, rc, hipGetErrorString((hipError_t)rc));
    return -1;
}

static size_t dn_align(size_t v) { return (v + DN_ALIGN - 1) / DN_ALIGN * DN_ALIGN; }

static void dn_dims(const qmoe_dn_config *c, size_t *key_dim, size_t *value_dim, size_t *conv_dim) {
    *key_dim = (size_t)c->n_k_heads * c->k_head_dim;
    *value_dim = (size_t)c->n_v_heads * c->v_head_dim;
    *conv_dim = 2 * *key_dim + *value_dim;
}

int qmoe_dn_create(qmoe_dn_ctx **out, const qmoe_dn_config *cfg, qmoe_err *err) {
    if (err) err->msg[0] = 0;
    if (!out || !cfg) {
        dn_set_err(err, "%s is NULL", out ? "cfg" : "ctx");
        return -1;
    }
    *out = NULL;
    const qk_dn_shape s = {cfg->hidden, cfg->n_k_heads, cfg->n_v_heads, cfg->k_head_dim,
                           cfg->v_head_dim, cfg->conv_kernel};
    if (cfg->group_size != 64 || !qk_dn_shape_ok(&s)) {
        dn_set_err(err, "DeltaNet shape unsupported: hidden %d (multiple of 64, <= 8192), heads %d/%d "
                        "(value heads a multiple of key heads), k_head_dim %d (32, 64, 128, 256), "
                        "v_head_dim %d (a power of two, 32..2048; heads*dim a multiple of 64, <= 8192), "
                        "conv_kernel %d (1..16), group_size %d (64)",
                   cfg->hidden, cfg->n_k_heads, cfg->n_v_heads, cfg->k_head_dim, cfg->v_head_dim,
                   cfg->conv_kernel, cfg->group_size);
        return -1;
    }
    if (cfg->n_layers < 1 || cfg->max_tokens < 1) {
        dn_set_err(err, "n_layers %d and max_tokens %d must be >= 1", cfg->n_layers, cfg->max_tokens);
        return -1;
    }
    qmoe_dn_ctx *c = (qmoe_dn_ctx *)calloc(1, sizeof(*c));
    if (!c) {
        dn_set_err(err, "out of host memory");
        return -1;
    }
    c->cfg = *cfg;
    c->shape = s;
    if (dn_hip_fail(err, (int)hipGetDevice(&c->device), "get device")) {
        free(c);
        return -1;
    }
    size_t key_dim, value_dim, conv_dim;
    dn_dims(cfg, &key_dim, &value_dim, &conv_dim);
    const size_t d = (size_t)cfg->hidden, hv = (size_t)cfg->n_v_heads, kc = (size_t)cfg->conv_kernel;
    const size_t sz[DT_COUNT] = {
        conv_dim * d / 2, conv_dim * (d / 64) * 2, conv_dim * (d / 64) * 2,
        value_dim * d / 2, value_dim * (d / 64) * 2, value_dim * (d / 64) * 2,
        hv * d * 2, hv * d * 2,
        d * value_dim / 2, d * (value_dim / 64) * 2, d * (value_dim / 64) * 2,
        conv_dim * kc * 2, (size_t)cfg->v_head_dim * 4, hv * 4, hv * 4,
        (kc - 1) * conv_dim * 4, hv * (size_t)cfg->v_head_dim * cfg->k_head_dim * 4};
    size_t total = 0;
    for (int i = 0; i < DT_COUNT; i++) {
        c->off[i] = total;
        c->bytes[i] = sz[i];
        total = dn_align(total + sz[i]);
    }
    c->off[DT_COUNT] = total;
    c->layers = (dn_layer *)calloc((size_t)cfg->n_layers, sizeof(dn_layer));
    const size_t n = (size_t)cfg->max_tokens;
    const size_t ssz[6] = {n * conv_dim * 4, n * value_dim * 4, n * hv * 4, n * hv * 4, n * value_dim * 4,
                           n * (value_dim / 16) * 4};
    size_t stot = 0, soff[6];
    for (int i = 0; i < 6; i++) {
        soff[i] = stot;
        stot = dn_align(stot + ssz[i]);
    }
    if (!c->layers || dn_hip_fail(err, (int)hipMalloc(&c->scratch, stot), "scratch")) {
        free(c->layers);
        free(c);
        return -1;
    }
    char *b = (char *)c->scratch;
    c->mixed = (float *)(b + soff[0]);
    c->z = (float *)(b + soff[1]);
    c->a = (float *)(b + soff[2]);
    c->b = (float *)(b + soff[3]);
    c->core = (float *)(b + soff[4]);
    c->ssp = (float *)(b + soff[5]);
    for (int l = 0; l < cfg->n_layers; l++) {
        if (dn_hip_fail(err, (int)hipMalloc(&c->layers[l].mem, total), "layer weights")) {
            qmoe_dn_destroy(c);
            return -1;
        }
    }
    *out = c;
    return 0;
}

void qmoe_dn_destroy(qmoe_dn_ctx *c) {
    if (!c) return;
    if (c->layers)
        for (int l = 0; l < c->cfg.n_layers; l++) hipFree(c->layers[l].mem);
    hipFree(c->scratch);
    free(c->layers);
    free(c);
}

static int dn_check_layer(qmoe_dn_ctx *c, int layer, qmoe_err *err) {
    if (err) err->msg[0] = 0;
    if (!c) {
        dn_set_err(err, "ctx is NULL");
        return -1;
    }
    if (layer < 0 || layer >= c->cfg.n_layers) {
        dn_set_err(err, "layer %d out of range [0, %d)", layer, c->cfg.n_layers);
        return -1;
    }
    return 0;
}

static void *dn_ptr(const qmoe_dn_ctx *c, int layer, int t) {
    return (char *)c->layers[layer].mem + c->off[t];
}

static int dn_zero_states(qmoe_dn_ctx *c, int layer, hipStream_t st, qmoe_err *err) {
    const int rc1 = qk_launch_dn_zero((float *)dn_ptr(c, layer, DT_CONV_STATE), c->bytes[DT_CONV_STATE] / 4, st);
    if (dn_hip_fail(err, rc1, "clear conv state")) return -1;
    const int rc2 = qk_launch_dn_zero((float *)dn_ptr(c, layer, DT_REC_STATE), c->bytes[DT_REC_STATE] / 4, st);
    return dn_hip_fail(err, rc2, "clear recurrent state");
}

int qmoe_dn_upload_layer(qmoe_dn_ctx *c, int layer, const qmoe_dn_weights *w, qmoe_err *err) {
    if (dn_check_layer(c, layer, err)) return -1;
    if (!w) {
        dn_set_err(err, "weights is NULL");
        return -1;
    }
    const void *src[DT_CONV_STATE] = {w->qkv_q, w->qkv_s, w->qkv_b, w->z_q, w->z_s, w->z_b, w->a_w,
                                      w->b_w, w->out_q, w->out_s, w->out_b, w->conv_w, w->norm_w,
                                      w->a_log, w->dt_bias};
    static const char *names[DT_CONV_STATE] = {"qkv_q", "qkv_s", "qkv_b", "z_q", "z_s", "z_b", "a_w",
                                               "b_w", "out_q", "out_s", "out_b", "conv_w", "norm_w",
                                               "a_log", "dt_bias"};
    for (int i = 0; i < DT_CONV_STATE; i++)
        if (!src[i]) {
            dn_set_err(err, "layer %d: %s is NULL", layer, names[i]);
            return -1;
        }
    c->layers[layer].ready = 0;
    for (int i = 0; i < DT_CONV_STATE; i++)
        if (dn_hip_fail(err, (int)hipMemcpy(dn_ptr(c, layer, i), src[i], c->bytes[i], hipMemcpyHostToDevice),
                        names[i]))
            return -1;
    if (dn_zero_states(c, layer, NULL, err) ||
        dn_hip_fail(err, (int)hipDeviceSynchronize(), "upload"))
        return -1;
    c->layers[layer].ready = 1;
    return 0;
}

int qmoe_dn_reset_state(qmoe_dn_ctx *c, int layer, void *stream, qmoe_err *err) {
    if (err) err->msg[0] = 0;
    if (!c) {
        dn_set_err(err, "ctx is NULL");
        return -1;
    }
    if (layer == -1) {
        for (int l = 0; l < c->cfg.n_layers; l++)
            if (dn_zero_states(c, l, (hipStream_t)stream, err)) return -1;
        return 0;
    }
    if (dn_check_layer(c, layer, err)) return -1;
    return dn_zero_states(c, layer, (hipStream_t)stream, err);
}

static int dn_forward(qmoe_dn_ctx *c, int layer, const float *x, int n, float *out,
                      const qk_inject *inj, void *stream, qmoe_err *err) {
    if (dn_check_layer(c, layer, err)) return -1;
    if (n < 0 || n > c->cfg.max_tokens) {
        dn_set_err(err, "n = %d out of range [0, max_tokens = %d]", n, c->cfg.max_tokens);
        return -1;
    }
    if (!c->layers[layer].ready) {
        dn_set_err(err, "layer %d has no weights", layer);
        return -1;
    }
    if (n == 0) return 0;
    if (!x || (!out && !inj)) {
        dn_set_err(err, "%s is NULL", x ? "out" : "x");
        return -1;
    }
    qk_dn_dev W;
    W.qkv_q = (const uint32_t *)dn_ptr(c, layer, DT_QKV_Q);
    W.qkv_s = (const uint16_t *)dn_ptr(c, layer, DT_QKV_S);
    W.qkv_b = (const uint16_t *)dn_ptr(c, layer, DT_QKV_B);
    W.z_q = (const uint32_t *)dn_ptr(c, layer, DT_Z_Q);
    W.z_s = (const uint16_t *)dn_ptr(c, layer, DT_Z_S);
    W.z_b = (const uint16_t *)dn_ptr(c, layer, DT_Z_B);
    W.a_w = (const uint16_t *)dn_ptr(c, layer, DT_A_W);
    W.b_w = (const uint16_t *)dn_ptr(c, layer, DT_B_W);
    W.out_q = (const uint32_t *)dn_ptr(c, layer, DT_OUT_Q);
    W.out_s = (const uint16_t *)dn_ptr(c, layer, DT_OUT_S);
    W.out_b = (const uint16_t *)dn_ptr(c, layer, DT_OUT_B);
    W.conv_w = (const uint16_t *)dn_ptr(c, layer, DT_CONV_W);
    W.norm_w = (const float *)dn_ptr(c, layer, DT_NORM_W);
    W.a_log = (const float *)dn_ptr(c, layer, DT_A_LOG);
    W.dt_bias = (const float *)dn_ptr(c, layer, DT_DT_BIAS);
    const int rc = qk_launch_dn(&c->shape, &W, x, n, out, (float *)dn_ptr(c, layer, DT_CONV_STATE),
                                (float *)dn_ptr(c, layer, DT_REC_STATE), c->mixed, c->z, c->a, c->b,
                                c->core, c->ssp, inj, stream);
    return dn_hip_fail(err, rc, "DeltaNet launch");
}

int qmoe_dn_forward(qmoe_dn_ctx *c, int layer, const float *x, int n, float *out, void *stream,
                    qmoe_err *err) {
    return dn_forward(c, layer, x, n, out, NULL, stream, err);
}

int qmoe_dn_forward_inject(qmoe_dn_ctx *c, int layer, const float *x, int n, float *out, float *hyper,
                           const float *inject, int hc, void *stream, qmoe_err *err) {
    if (!hyper || !inject) {
        dn_set_err(err, "%s is NULL", hyper ? "inject" : "hyper");
        return -1;
    }
    if (hc < 1 || hc > QK_INJECT_MAX_HC) {
        dn_set_err(err, "hc = %d out of range [1, %d]", hc, QK_INJECT_MAX_HC);
        return -1;
    }
    const qk_inject inj = {hyper, inject, hc};
    return dn_forward(c, layer, x, n, out, &inj, stream, err);
}

int qmoe_dn_state(qmoe_dn_ctx *c, int layer, float **conv_state, float **rec_state, qmoe_err *err) {
    if (dn_check_layer(c, layer, err)) return -1;
    if (conv_state) *conv_state = (float *)dn_ptr(c, layer, DT_CONV_STATE);
    if (rec_state) *rec_state = (float *)dn_ptr(c, layer, DT_REC_STATE);
    return 0;
}
