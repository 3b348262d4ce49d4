/*
 * qmoe_attn.c -- C11 host side of the full-attention mixer with the QSA
 * indexer: context, HBM residency of each layer's weights and caches, the
 * cache lengths, argument checks and the launches of attention.hip.
 * Replaces attention_forward (c/src/model.c:798-1144) and the cache state
 * around it (model.c:341-345, 402-406).
 */
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <hip/hip_runtime_api.h>

#include "qmoe_internal.h"

#define AT_ALIGN 256u

enum { AT_Q_Q, AT_Q_S, AT_Q_B, AT_K_Q, AT_K_S, AT_K_B, AT_V_Q, AT_V_S, AT_V_B, AT_O_Q, AT_O_S, AT_O_B,
       AT_IDX_W, AT_Q_NORM, AT_K_NORM, AT_IQ_NORM, AT_IK_NORM, AT_K_CACHE, AT_V_CACHE, AT_IDX_KEYS,
       AT_POOLED, AT_COUNT };

typedef struct {
    void *mem;
    int ready, len;
    int start; /* sliding window: first row of the window in the cache buffers */
    int base;  /* sliding window: position of the window's first row */
} at_layer;

struct qmoe_attn_ctx {
    qmoe_attn_config cfg;
    qk_at_shape shape;
    size_t off[AT_COUNT], bytes[AT_COUNT];
    at_layer *layers;
    void *scratch;
    qk_at_scratch sc;
    float *rope;    /* device [rope_rows, rot/2, 2] */
    int rope_rows;  /* positions the table covers */
    int last_kw;    /* kept-block bitmap words per token of the last masked call */
};

static void at_set_err(qmoe_err *err, const char *fmt, ...) {
    if (!err) return;
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(err->msg, sizeof(err->msg), fmt, ap);
    va_end(ap);
}

static int at_hip_fail(qmoe_err *err, int rc, const char *what) {
    if (rc == 0) return 0;
    at_set_err(err, "%s: HIP error %d (%s)", what, rc, hipGetErrorString((hipError_t)rc));
    return -1;
}

static size_t at_align(size_t v) { return (v + AT_ALIGN - 1) / AT_ALIGN * AT_ALIGN; }

/* cos / sin of pos * theta^(-2i/rot) for positions [0, rows) and i < rot/2,
 * with the reference's formula and float arithmetic (model.c: inv[i] =
 * powf(theta, -(2i)/rot), a = (float)pos * inv[i], cosf(a), sinf(a)) */
static int at_rope_table(qmoe_attn_ctx *c, qmoe_err *err) {
    const int half = c->shape.rot / 2;
    if (half == 0) return 0;
    const size_t cnt = (size_t)c->rope_rows * (size_t)half * 2;
    float *tab = (float *)malloc(cnt * sizeof(float));
    float *inv = (float *)malloc((size_t)half * sizeof(float));
    if (!tab || !inv) {
        free(tab);
        free(inv);
        at_set_err(err, "out of host memory");
        return -1;
    }
    for (int i = 0; i < half; i++)
        inv[i] = powf(c->shape.theta, -(2.0f * (float)i) / (float)c->shape.rot);
    for (int p = 0; p < c->rope_rows; p++)
        for (int i = 0; i < half; i++) {
            const float ang = (float)p * inv[i];
            tab[((size_t)p * half + i) * 2] = cosf(ang);
            tab[((size_t)p * half + i) * 2 + 1] = sinf(ang);
        }
    int rc = at_hip_fail(err, (int)hipMalloc((void **)&c->rope, cnt * sizeof(float)), "rope table");
    if (!rc)
        rc = at_hip_fail(err, (int)hipMemcpy(c->rope, tab, cnt * sizeof(float), hipMemcpyHostToDevice),
                         "rope table");
    free(tab);
    free(inv);
    return rc;
}

int qmoe_attn_create(qmoe_attn_ctx **out, const qmoe_attn_config *cfg, qmoe_err *err) {
    if (err) err->msg[0] = 0;
    if (!out || !cfg) {
        at_set_err(err, "%s is NULL", out ? "cfg" : "ctx");
        return -1;
    }
    *out = NULL;
    const qk_at_shape s = {cfg->hidden, cfg->n_heads, cfg->n_kv_heads, cfg->head_dim, cfg->idx_heads,
                           cfg->idx_head_dim, cfg->idx_budget, cfg->idx_compress, cfg->kv_cap,
                           (int)((float)cfg->head_dim * cfg->rotary_factor), cfg->rope_theta};
    if (cfg->group_size != 64 || !(cfg->rotary_factor > 0.0f && cfg->rotary_factor <= 1.0f) ||
        !qk_at_shape_ok(&s)) {
        at_set_err(err, "attention shape unsupported: hidden %d (multiple of 64, <= 8192), heads %d/%d "
                        "(kv heads divide heads), head_dim %d (multiple of 64, <= 256, heads*dim <= 8192), "
                        "indexer %d heads (<= 64) of %d (dim a multiple of 4, <= 256, >= the rotated dims %d, "
                        "even; heads*dim <= 8192), budget %d, compress %d, kv_cap %d (<= 8192), group_size %d (64)",
                   cfg->hidden, cfg->n_heads, cfg->n_kv_heads, cfg->head_dim, cfg->idx_heads,
                   cfg->idx_head_dim, s.rot, cfg->idx_budget, cfg->idx_compress, cfg->kv_cap,
                   cfg->group_size);
        return -1;
    }
    if (cfg->n_layers < 1 || cfg->max_tokens < 1 || cfg->max_tokens > cfg->kv_cap) {
        at_set_err(err, "n_layers %d and max_tokens %d must be >= 1 (max_tokens <= kv_cap %d)",
                   cfg->n_layers, cfg->max_tokens, cfg->kv_cap);
        return -1;
    }
    if (cfg->slide != 0 && (cfg->slide != 1 || cfg->kv_cap % cfg->idx_compress != 0)) {
        at_set_err(err, "slide %d: 0 or 1, and 1 needs kv_cap %d a multiple of idx_compress %d",
                   cfg->slide, cfg->kv_cap, cfg->idx_compress);
        return -1;
    }
    if (cfg->max_position < 0 || cfg->max_position > QMOE_ATTN_MAX_POSITION) {
        at_set_err(err, "max_position %d out of range [0, %d]", cfg->max_position, QMOE_ATTN_MAX_POSITION);
        return -1;
    }
    qmoe_attn_ctx *c = (qmoe_attn_ctx *)calloc(1, sizeof(*c));
    if (!c) {
        at_set_err(err, "out of host memory");
        return -1;
    }
    c->cfg = *cfg;
    c->shape = s;
    c->rope_rows = cfg->max_position > cfg->kv_cap ? cfg->max_position : cfg->kv_cap;
    const size_t d = (size_t)s.d, h = (size_t)s.h, kvh = (size_t)s.kvh, hd = (size_t)s.hd;
    const size_t ih = (size_t)s.ih, ihd = (size_t)s.ihd, cap = (size_t)s.cap;
    const size_t qr = 2 * h * hd, kr = kvh * hd, orow = d, ok = h * hd;
    /* a sliding window moves through buffers of twice the capacity and is
     * copied back to their start when it reaches their end */
    const size_t phys = cfg->slide ? 2 * cap : cap;
    const size_t sz[AT_COUNT] = {
        qr * d / 2, qr * (d / 64) * 2, qr * (d / 64) * 2,
        kr * d / 2, kr * (d / 64) * 2, kr * (d / 64) * 2,
        kr * d / 2, kr * (d / 64) * 2, kr * (d / 64) * 2,
        orow * ok / 2, orow * (ok / 64) * 2, orow * (ok / 64) * 2,
        (ih + 1) * ihd * d * 2, hd * 4, hd * 4, ihd * 4, ihd * 4,
        phys * kr * 4, phys * kr * 4, phys * ihd * 4, phys / (size_t)s.comp * ihd * 4};
    size_t total = 0;
    for (int i = 0; i < AT_COUNT; i++) {
        c->off[i] = total;
        c->bytes[i] = sz[i];
        total = at_align(total + sz[i]);
    }
    const size_t n = (size_t)cfg->max_tokens;
    /* the attention partials hold max_tokens calls' worth of 256-key chunks,
     * and at least one token's 64-key chunks (one-token calls split the
     * cache finer) */
    const size_t units = n * ((cap + 255) / 256) > (cap + 63) / 64 ? n * ((cap + 255) / 256) : (cap + 63) / 64;
    const size_t kw = (cap / (size_t)s.comp + 31) / 32 + 1;
    const size_t ssz[10] = {n * qr * 4, n * kr * 4, n * kr * 4, n * (ih + 1) * ihd * 4, n * h * hd * 4,
                            n * ih * ihd * 4, n * kw * 4, units * h * (hd + 2) * 4, n * h * hd * 4,
                            n * (cap / (size_t)s.comp) * 4};
    size_t stot = 0, soff[10];
    for (int i = 0; i < 10; i++) {
        soff[i] = stot;
        stot = at_align(stot + ssz[i]);
    }
    c->layers = (at_layer *)calloc((size_t)cfg->n_layers, sizeof(at_layer));
    if (!c->layers || at_hip_fail(err, (int)hipMalloc(&c->scratch, stot), "scratch")) {
        free(c->layers);
        free(c);
        return -1;
    }
    char *b = (char *)c->scratch;
    c->sc.qg = (float *)(b + soff[0]);
    c->sc.kraw = (float *)(b + soff[1]);
    c->sc.vraw = (float *)(b + soff[2]);
    c->sc.qk = (float *)(b + soff[3]);
    c->sc.qn = (float *)(b + soff[4]);
    c->sc.qi = (float *)(b + soff[5]);
    c->sc.keep = (uint32_t *)(b + soff[6]);
    c->sc.part_units = (long long)units;
    c->sc.part = (float *)(b + soff[7]);
    c->sc.ao = (float *)(b + soff[8]);
    c->sc.skey = (uint32_t *)(b + soff[9]);
    for (int l = 0; l < cfg->n_layers; l++)
        if (at_hip_fail(err, (int)hipMalloc(&c->layers[l].mem, total), "layer weights")) {
            qmoe_attn_destroy(c);
            return -1;
        }
    if (at_rope_table(c, err)) {
        qmoe_attn_destroy(c);
        return -1;
    }
    *out = c;
    return 0;
}

void qmoe_attn_destroy(qmoe_attn_ctx *c) {
    if (!c) return;
    if (c->layers)
        for (int l = 0; l < c->cfg.n_layers; l++) hipFree(c->layers[l].mem);
    hipFree(c->scratch);
    hipFree(c->rope);
    free(c->layers);
    free(c);
}

static int at_check_layer(qmoe_attn_ctx *c, int layer, qmoe_err *err) {
    if (err) err->msg[0] = 0;
    if (!c) {
        at_set_err(err, "ctx is NULL");
        return -1;
    }
    if (layer < 0 || layer >= c->cfg.n_layers) {
        at_set_err(err, "layer %d out of range [0, %d)", layer, c->cfg.n_layers);
        return -1;
    }
    return 0;
}

static void *at_ptr(const qmoe_attn_ctx *c, int layer, int t) {
    return (char *)c->layers[layer].mem + c->off[t];
}

int qmoe_attn_upload_layer(qmoe_attn_ctx *c, int layer, const qmoe_attn_weights *w, qmoe_err *err) {
    if (at_check_layer(c, layer, err)) return -1;
    if (!w) {
        at_set_err(err, "weights is NULL");
        return -1;
    }
    const void *src[AT_K_CACHE] = {w->q_q, w->q_s, w->q_b, w->k_q, w->k_s, w->k_b, w->v_q, w->v_s,
                                   w->v_b, w->o_q, w->o_s, w->o_b, w->idx_w, w->q_norm, w->k_norm,
                                   w->idx_q_norm, w->idx_k_norm};
    static const char *names[AT_K_CACHE] = {"q_q", "q_s", "q_b", "k_q", "k_s", "k_b", "v_q", "v_s",
                                            "v_b", "o_q", "o_s", "o_b", "idx_w", "q_norm", "k_norm",
                                            "idx_q_norm", "idx_k_norm"};
    for (int i = 0; i < AT_K_CACHE; i++)
        if (!src[i]) {
            at_set_err(err, "layer %d: %s is NULL", layer, names[i]);
            return -1;
        }
    c->layers[layer].ready = 0;
    for (int i = 0; i < AT_K_CACHE; i++)
        if (at_hip_fail(err, (int)hipMemcpy(at_ptr(c, layer, i), src[i], c->bytes[i], hipMemcpyHostToDevice),
                        names[i]))
            return -1;
    c->layers[layer].len = c->layers[layer].start = c->layers[layer].base = 0;
    c->layers[layer].ready = 1;
    return 0;
}

int qmoe_attn_reset(qmoe_attn_ctx *c, int layer, qmoe_err *err) {
    if (err) err->msg[0] = 0;
    if (!c) {
        at_set_err(err, "ctx is NULL");
        return -1;
    }
    if (layer == -1) {
        for (int l = 0; l < c->cfg.n_layers; l++) c->layers[l].len = c->layers[l].start = c->layers[l].base = 0;
        return 0;
    }
    if (at_check_layer(c, layer, err)) return -1;
    c->layers[layer].len = c->layers[layer].start = c->layers[layer].base = 0;
    return 0;
}

static int attn_forward(qmoe_attn_ctx *c, int layer, const float *x, int n, int offset, float *out,
                        const qk_inject *inj, void *stream, qmoe_err *err) {
    if (at_check_layer(c, layer, err)) return -1;
    if (n < 0 || n > c->cfg.max_tokens) {
        at_set_err(err, "n = %d out of range [0, max_tokens = %d]", n, c->cfg.max_tokens);
        return -1;
    }
    if (!c->layers[layer].ready) {
        at_set_err(err, "layer %d has no weights", layer);
        return -1;
    }
    if (offset < 0) {
        at_set_err(err, "offset %d is negative", offset);
        return -1;
    }
    if (n == 0) return 0;
    if (!x || (!out && !inj)) {
        at_set_err(err, "%s is NULL", x ? "out" : "x");
        return -1;
    }
    at_layer *L = &c->layers[layer];
    int len0 = L->len, drop = 0;
    const int comp = c->cfg.idx_compress, cap = c->cfg.kv_cap;
    if (c->cfg.slide) {
        if (offset != L->base + len0) {
            at_set_err(err, "layer %d: a sliding window continues at position %d (window from %d, "
                            "%d cached), not %d", layer, L->base + len0, L->base, len0, offset);
            return -1;
        }
        if (len0 + n > cap) {
            drop = (len0 + n - cap + comp - 1) / comp * comp;
            if (drop > len0) {
                at_set_err(err, "layer %d: %d new tokens would drop %d rows of the %d cached (calls of "
                                "at most kv_cap - idx_compress + 1 = %d tokens always fit)",
                           layer, n, drop, len0, cap - comp + 1);
                return -1;
            }
        }
    } else if (len0 + n > cap) {
        at_set_err(err, "layer %d: %d cached + %d new tokens pass kv_cap %d", layer, len0, n, cap);
        return -1;
    }
    if ((long long)offset + n > c->rope_rows) {
        at_set_err(err, "positions %d..%d pass max_position %d", offset, offset + n - 1, c->rope_rows);
        return -1;
    }
    if (drop) { /* the oldest rows leave the window */
        L->start += drop;
        L->base += drop;
        len0 -= drop;
        L->len = len0;
    }
    const size_t kr = (size_t)c->shape.kvh * c->shape.hd, ihd = (size_t)c->shape.ihd;
    float *kc = (float *)at_ptr(c, layer, AT_K_CACHE), *vc = (float *)at_ptr(c, layer, AT_V_CACHE);
    float *ic = (float *)at_ptr(c, layer, AT_IDX_KEYS), *pc = (float *)at_ptr(c, layer, AT_POOLED);
    if (c->cfg.slide && L->start + len0 + n > 2 * cap) {
        /* the window back to the buffers' start: rows [start, start + len0) to [0, len0),
         * disjoint because start > cap >= len0 + n; the pooled keys of its complete blocks too */
        hipStream_t st = (hipStream_t)stream;
        const size_t s0 = (size_t)L->start;
        int rc = (int)hipMemcpyAsync(kc, kc + s0 * kr, (size_t)len0 * kr * 4, hipMemcpyDeviceToDevice, st);
        if (!rc) rc = (int)hipMemcpyAsync(vc, vc + s0 * kr, (size_t)len0 * kr * 4, hipMemcpyDeviceToDevice, st);
        if (!rc) rc = (int)hipMemcpyAsync(ic, ic + s0 * ihd, (size_t)len0 * ihd * 4, hipMemcpyDeviceToDevice, st);
        if (!rc)
            rc = (int)hipMemcpyAsync(pc, pc + s0 / comp * ihd, (size_t)(len0 / comp) * ihd * 4,
                                     hipMemcpyDeviceToDevice, st);
        if (at_hip_fail(err, rc, "window copy")) return -1;
        L->start = 0;
    }
    const size_t w0 = (size_t)L->start;
    qk_at_dev W;
    W.q_q = (const uint32_t *)at_ptr(c, layer, AT_Q_Q);
    W.q_s = (const uint16_t *)at_ptr(c, layer, AT_Q_S);
    W.q_b = (const uint16_t *)at_ptr(c, layer, AT_Q_B);
    W.k_q = (const uint32_t *)at_ptr(c, layer, AT_K_Q);
    W.k_s = (const uint16_t *)at_ptr(c, layer, AT_K_S);
    W.k_b = (const uint16_t *)at_ptr(c, layer, AT_K_B);
    W.v_q = (const uint32_t *)at_ptr(c, layer, AT_V_Q);
    W.v_s = (const uint16_t *)at_ptr(c, layer, AT_V_S);
    W.v_b = (const uint16_t *)at_ptr(c, layer, AT_V_B);
    W.o_q = (const uint32_t *)at_ptr(c, layer, AT_O_Q);
    W.o_s = (const uint16_t *)at_ptr(c, layer, AT_O_S);
    W.o_b = (const uint16_t *)at_ptr(c, layer, AT_O_B);
    W.idx_w = (const uint16_t *)at_ptr(c, layer, AT_IDX_W);
    W.q_norm = (const float *)at_ptr(c, layer, AT_Q_NORM);
    W.k_norm = (const float *)at_ptr(c, layer, AT_K_NORM);
    W.idx_q_norm = (const float *)at_ptr(c, layer, AT_IQ_NORM);
    W.idx_k_norm = (const float *)at_ptr(c, layer, AT_IK_NORM);
    W.rope = c->rope;
    const int rc = qk_launch_at(&c->shape, &W, x, n, offset, c->cfg.slide ? L->base : 0, len0, out,
                                kc + w0 * kr, vc + w0 * kr, ic + w0 * ihd, pc + w0 / comp * ihd, &c->sc, inj,
                                stream);
    if (at_hip_fail(err, rc, "attention launch")) return -1;
    L->len = len0 + n;
    if (len0 + n > c->cfg.idx_budget) c->last_kw = ((len0 + n) / c->cfg.idx_compress + 31) / 32;
    return 0;
}

int qmoe_attn_forward(qmoe_attn_ctx *c, int layer, const float *x, int n, int offset, float *out,
                      void *stream, qmoe_err *err) {
    return attn_forward(c, layer, x, n, offset, out, NULL, stream, err);
}

int qmoe_attn_forward_inject(qmoe_attn_ctx *c, int layer, const float *x, int n, int offset, float *out,
                             float *hyper, const float *inject, int hc, void *stream, qmoe_err *err) {
    if (!hyper || !inject) {
        at_set_err(err, "%s is NULL", hyper ? "inject" : "hyper");
        return -1;
    }
    if (hc < 1 || hc > QK_INJECT_MAX_HC) {
        at_set_err(err, "hc = %d out of range [1, %d]", hc, QK_INJECT_MAX_HC);
        return -1;
    }
    const qk_inject inj = {hyper, inject, hc};
    return attn_forward(c, layer, x, n, offset, out, &inj, stream, err);
}

int qmoe_attn_cache(qmoe_attn_ctx *c, int layer, float **k_cache, float **v_cache, float **idx_keys,
                    int *len, qmoe_err *err) {
    if (at_check_layer(c, layer, err)) return -1;
    const size_t w0 = (size_t)c->layers[layer].start;
    const size_t kr = (size_t)c->shape.kvh * c->shape.hd;
    if (k_cache) *k_cache = (float *)at_ptr(c, layer, AT_K_CACHE) + w0 * kr;
    if (v_cache) *v_cache = (float *)at_ptr(c, layer, AT_V_CACHE) + w0 * kr;
    if (idx_keys) *idx_keys = (float *)at_ptr(c, layer, AT_IDX_KEYS) + w0 * (size_t)c->shape.ihd;
    if (len) *len = c->layers[layer].len;
    return 0;
}

int qmoe_attn_index_state(qmoe_attn_ctx *c, int layer, float **pooled, uint32_t **keep, int *keep_words,
                          uint32_t **score_keys, int *score_ld, qmoe_err *err) {
    if (at_check_layer(c, layer, err)) return -1;
    if (pooled)
        *pooled = (float *)at_ptr(c, layer, AT_POOLED) +
                  (size_t)(c->layers[layer].start / c->cfg.idx_compress) * c->shape.ihd;
    if (keep) *keep = c->sc.keep;
    if (keep_words) *keep_words = c->last_kw;
    if (score_keys) *score_keys = c->sc.skey;
    if (score_ld) *score_ld = c->cfg.kv_cap / c->cfg.idx_compress;
    return 0;
}
