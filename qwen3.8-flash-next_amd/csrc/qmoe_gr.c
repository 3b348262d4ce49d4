/*
 * qmoe_gr.c -- C11 host side of the stand-alone gated residual: weight
 * slots in HBM for the attention-block hyper connections and the final
 * mixer, argument checks, and the launches of hyper.hip / hyper_mm.hip.
 * Replaces the gated_residual calls of c/src/model.c:1671-1672 and
 * 1743-1745 and the inject update of model.c:1699-1707.
 */
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <hip/hip_runtime_api.h>

#include "qmoe_internal.h"

#define GR_ALIGN 256u

/* tensors of a slot allocation, in the order of qmoe_hc_weights */
enum { GT_NORM, GT_DOWN_Q, GT_DOWN_S, GT_DOWN_B, GT_UP_Q, GT_UP_S, GT_UP_B, GT_INJECT_W, GT_COUNT };

typedef struct {
    void *mem;
    int ready, has_inject;
} gr_slot;

struct qmoe_gr_ctx {
    qmoe_gr_config cfg;
    size_t off[GT_COUNT], bytes[GT_COUNT], slot_bytes;
    gr_slot *slots;
    void *scratch;       /* normed [n, hc*d], w [n, R], inject [n, hc] of the GEMV path */
    float *normed, *w, *inject;
    void *ws;            /* the MFMA path's workspace (n >= QK_HC_MM_MIN) */
};

static void gr_set_err(qmoe_err *err, const char *fmt, ...) {
    if (!err) return;
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(err->msg, sizeof(err->msg), fmt, ap);
    va_end(ap);
}

static int gr_hip_fail(qmoe_err *err, int rc, const char *what) {
    if (rc == 0) return 0;
    gr_set_err(err, "%s: HIP error %d (%s)", what, rc, hipGetErrorString((hipError_t)rc));
    return -1;
}

static size_t gr_align(size_t v) { return (v + GR_ALIGN - 1) / GR_ALIGN * GR_ALIGN; }

int qmoe_gr_create(qmoe_gr_ctx **out, const qmoe_gr_config *cfg, qmoe_err *err) {
    if (err) err->msg[0] = 0;
    if (!out || !cfg) {
        gr_set_err(err, "%s is NULL", out ? "cfg" : "ctx");
        return -1;
    }
    *out = NULL;
    if (!qk_hc_shape_ok(cfg->hc_count, cfg->hidden, cfg->hc_lowrank)) {
        gr_set_err(err, "gated residual shape unsupported: hidden %d (multiple of 64, <= 2048), "
                        "hc_count %d (1..8), hc_lowrank %d (multiple of 64, 64..2048)",
                   cfg->hidden, cfg->hc_count, cfg->hc_lowrank);
        return -1;
    }
    if (cfg->n_slots < 1 || cfg->max_tokens < 1) {
        gr_set_err(err, "n_slots %d and max_tokens %d must be >= 1", cfg->n_slots, cfg->max_tokens);
        return -1;
    }
    qmoe_gr_ctx *c = (qmoe_gr_ctx *)calloc(1, sizeof(*c));
    if (!c) {
        gr_set_err(err, "out of host memory");
        return -1;
    }
    c->cfg = *cfg;
    const size_t hc = (size_t)cfg->hc_count, D = hc * cfg->hidden, R = (size_t)cfg->hc_lowrank;
    const size_t sz[GT_COUNT] = {D * 4,          R * D / 2, R * (D / 64) * 2, R * (D / 64) * 2,
                                 D * R / 2,      D * (R / 64) * 2, D * (R / 64) * 2, hc * D * 2};
    size_t total = 0;
    for (int i = 0; i < GT_COUNT; i++) {
        c->off[i] = total;
        c->bytes[i] = sz[i];
        total = gr_align(total + sz[i]);
    }
    c->slot_bytes = total;
    const size_t n = (size_t)cfg->max_tokens;
    const size_t ssz[3] = {n * D * 4, n * R * 4, n * hc * 4};
    size_t stot = 0, soff[3];
    for (int i = 0; i < 3; i++) {
        soff[i] = stot;
        stot = gr_align(stot + ssz[i]);
    }
    c->slots = (gr_slot *)calloc((size_t)cfg->n_slots, sizeof(gr_slot));
    if (!c->slots || gr_hip_fail(err, (int)hipMalloc(&c->scratch, stot), "scratch")) {
        if (!c->slots) gr_set_err(err, "out of host memory");
        free(c->slots);
        free(c);
        return -1;
    }
    char *b = (char *)c->scratch;
    c->normed = (float *)(b + soff[0]);
    c->w = (float *)(b + soff[1]);
    c->inject = (float *)(b + soff[2]);
    if (cfg->max_tokens >= QK_HC_MM_MIN &&
        gr_hip_fail(err, (int)hipMalloc(&c->ws, qk_hc_mm_ws_bytes(cfg->hc_count, cfg->hidden,
                                                                 cfg->hc_lowrank, cfg->max_tokens)),
                    "workspace")) {
        qmoe_gr_destroy(c);
        return -1;
    }
    for (int s = 0; s < cfg->n_slots; s++)
        if (gr_hip_fail(err, (int)hipMalloc(&c->slots[s].mem, total), "slot weights")) {
            qmoe_gr_destroy(c);
            return -1;
        }
    *out = c;
    return 0;
}

void qmoe_gr_destroy(qmoe_gr_ctx *c) {
    if (!c) return;
    if (c->slots)
        for (int s = 0; s < c->cfg.n_slots; s++) hipFree(c->slots[s].mem);
    hipFree(c->scratch);
    hipFree(c->ws);
    free(c->slots);
    free(c);
}

static int gr_check_slot(qmoe_gr_ctx *c, int slot, qmoe_err *err) {
    if (err) err->msg[0] = 0;
    if (!c) {
        gr_set_err(err, "ctx is NULL");
        return -1;
    }
    if (slot < 0 || slot >= c->cfg.n_slots) {
        gr_set_err(err, "slot %d out of range [0, %d)", slot, c->cfg.n_slots);
        return -1;
    }
    return 0;
}

static void *gr_ptr(const qmoe_gr_ctx *c, int slot, int t) {
    return (char *)c->slots[slot].mem + c->off[t];
}

int qmoe_gr_upload_slot(qmoe_gr_ctx *c, int slot, const qmoe_hc_weights *w, qmoe_err *err) {
    if (gr_check_slot(c, slot, err)) return -1;
    if (!w) {
        gr_set_err(err, "weights is NULL");
        return -1;
    }
    const void *src[GT_COUNT] = {w->hc_norm, w->down_q, w->down_s, w->down_b,
                                 w->up_q,    w->up_s,   w->up_b,   w->inject_w};
    static const char *names[GT_COUNT] = {"hc_norm", "down_q", "down_s", "down_b",
                                          "up_q",    "up_s",   "up_b",   "inject_w"};
    for (int i = 0; i < GT_INJECT_W; i++)
        if (!src[i]) {
            gr_set_err(err, "slot %d: %s is NULL", slot, names[i]);
            return -1;
        }
    c->slots[slot].ready = 0;
    for (int i = 0; i < GT_COUNT; i++) {
        if (!src[i]) continue;
        if (gr_hip_fail(err, (int)hipMemcpy(gr_ptr(c, slot, i), src[i], c->bytes[i], hipMemcpyHostToDevice),
                        names[i]))
            return -1;
    }
    c->slots[slot].has_inject = w->inject_w != NULL;
    c->slots[slot].ready = 1;
    return 0;
}

static int gr_check_n(qmoe_gr_ctx *c, int n, qmoe_err *err) {
    if (n < 0 || n > c->cfg.max_tokens) {
        gr_set_err(err, "n = %d out of range [0, max_tokens = %d]", n, c->cfg.max_tokens);
        return -1;
    }
    return 0;
}

int qmoe_gr_mix(qmoe_gr_ctx *c, int slot, const float *hyper, int n, float *mixed_out,
                float *inject_out, void *stream, qmoe_err *err) {
    if (gr_check_slot(c, slot, err)) return -1;
    if (!c->slots[slot].ready) {
        gr_set_err(err, "slot %d has no weights", slot);
        return -1;
    }
    if (gr_check_n(c, n, err)) return -1;
    if (inject_out && !c->slots[slot].has_inject) {
        gr_set_err(err, "slot %d has no inject weights (inject_out must be NULL)", slot);
        return -1;
    }
    if (n == 0) return 0;
    if (!hyper || !mixed_out) {
        gr_set_err(err, "%s is NULL", hyper ? "mixed_out" : "hyper");
        return -1;
    }
    const int hc = c->cfg.hc_count, d = c->cfg.hidden, R = c->cfg.hc_lowrank;
    /* without inject_out the inject dots are skipped (the weights stay) */
    const uint16_t *iw = inject_out ? (const uint16_t *)gr_ptr(c, slot, GT_INJECT_W) : NULL;
    const float *nw = (const float *)gr_ptr(c, slot, GT_NORM);
    const uint32_t *dq = (const uint32_t *)gr_ptr(c, slot, GT_DOWN_Q);
    const uint16_t *ds = (const uint16_t *)gr_ptr(c, slot, GT_DOWN_S);
    const uint16_t *db = (const uint16_t *)gr_ptr(c, slot, GT_DOWN_B);
    const uint32_t *uq = (const uint32_t *)gr_ptr(c, slot, GT_UP_Q);
    const uint16_t *us = (const uint16_t *)gr_ptr(c, slot, GT_UP_S);
    const uint16_t *ub = (const uint16_t *)gr_ptr(c, slot, GT_UP_B);
    if (n >= QK_HC_MM_MIN && c->ws)
        return gr_hip_fail(err,
                           qk_launch_hc_mm(hyper, nw, dq, ds, db, uq, us, ub, iw, hc, d, R, n, 1e-6f,
                                           c->ws, mixed_out, inject_out, NULL, stream),
                           "gated residual (MFMA)");
    if (gr_hip_fail(err,
                    qk_launch_hc_down(hyper, nw, dq, ds, db, iw, hc, d, R, n, 1e-6f, c->normed, c->w,
                                      inject_out, stream),
                    "gated residual norm+down"))
        return -1;
    return gr_hip_fail(err,
                       qk_launch_hc_upmix(uq, us, ub, c->w, c->normed, hc, d, R, n, mixed_out, stream),
                       "gated residual up+mix");
}

int qmoe_gr_inject(qmoe_gr_ctx *c, const float *inject, const float *out, int n, float *hyper,
                   void *stream, qmoe_err *err) {
    if (err) err->msg[0] = 0;
    if (!c) {
        gr_set_err(err, "ctx is NULL");
        return -1;
    }
    if (gr_check_n(c, n, err)) return -1;
    if (n == 0) return 0;
    if (!inject || !out || !hyper) {
        gr_set_err(err, "%s is NULL", !inject ? "inject" : !out ? "out" : "hyper");
        return -1;
    }
    return gr_hip_fail(err,
                       qk_launch_hc_inject(inject, out, c->cfg.hc_count, c->cfg.hidden, n, hyper, stream),
                       "inject update");
}
