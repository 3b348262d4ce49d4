/*
 * qmoe_host.c -- C11 host side of libqmoe.so: context, HBM residency of the
 * layers, argument checking and the orchestration of the HIP kernels.
 *
 * Mirrors the reference C port's MoE-layer call contract
 * (c/src/model.c:1281-1405, c/src/kernel.h, c/src/util.h:11-27): plain C,
 * caller-owned outputs, 0 / -1 + message returns, no aborts.
 */
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <hip/hip_runtime_api.h>

#include "qmoe_internal.h"

#define QMOE_VERSION "qmoe 0.1 (gfx950)"
#define ALIGN 256u

typedef struct {
    void *mem;
    qmoe_layer_weights dev; /* pointers into mem; router_bias / norm_w NULL when absent */
    int ready;
} qmoe_layer_slot;

struct qmoe_ctx {
    qmoe_config cfg;
    qk_shape shape;
    int device;
    void *scratch_mem;
    size_t scratch_bytes;
    qk_scratch sc;
    float *host_x_dev, *host_out_dev; /* staging for qmoe_moe_forward_host */
    qmoe_layer_slot *layers;
    size_t layer_bytes;
    int last_n; /* token count of the last qmoe_layer_forward, -1 if none */
    /* second stream for the GEMV kernels of small segments, which run beside
     * the MFMA kernels of large ones (fork/join with two events) */
    hipStream_t aux;
    hipEvent_t ev_fork, ev_join;
    /* byte offsets of each tensor inside a layer allocation */
    size_t off[24];
    /* MLP hyper connection (qmoe_hc_enable): hc copies, low rank R, per-layer
     * weights in one allocation each, and the scratch of the mix */
    int hc, hc_R;
    size_t hc_off[QH_HC_COUNT], hc_layer_bytes;
    void **hc_mem;
    int *hc_ready;
    void *hc_scratch;
    float *hc_normed, *hc_down, *hc_inject, *hc_mixed;
    void *hc_ws; /* MFMA path workspace (max_tokens >= QK_HC_MM_MIN) */
    /* expert streaming (qmoe_stream_enable): routed experts in pinned host
     * memory, s_slots HBM slots per layer */
    int streamed, s_slots, s_prefetch, s_policy;
    qmoe_xcache *xc;
    void **s_host;               /* per layer: the routed tensors, checkpoint layout */
    void **s_hdev;               /* ... and its device mapping, looked up on first use */
    void *s_pool;                /* per layer, per routed tensor: s_slots experts */
    size_t s_tb[QH_T_COUNT];     /* per-expert bytes of a routed tensor (0: not routed) */
    size_t s_hoff[QH_T_COUNT];   /* offset of a routed tensor in a layer's host copy */
    size_t s_poff[QH_T_COUNT];   /* ... and in a layer's slot pool */
    size_t s_host_layer, s_pool_layer, s_expert_bytes;
    int32_t *s_seg;              /* pinned [1+3E]: the segment table, then its remap */
    int32_t *s_ids;              /* [E] the call's experts */
    int32_t *s_segtab;           /* device [1+3E]: segment table over slots */
    hipStream_t s_copy;          /* prefetch copies */
    hipEvent_t *s_ev_used, *s_ev_pf;
    int *s_pf_pending;
    uint32_t *s_freq;            /* [L, E] routed slots per expert */
    uint32_t *s_trans;           /* [L, E, E] experts of one call -> experts of the next */
    int32_t *s_prev;             /* [L, E+1]: count, then the previous call's experts */
    uint8_t *s_pf_flag;          /* [L, E] brought in by prefetch, not used yet */
    uint64_t s_bytes_in, s_prefetched, s_prefetch_hits;
    /* device-resolved mode (prefetch -1): the slot cache of every layer in
     * device memory, decided by k_stream_resolve inside the layer call */
    int s_dev;
    void *s_dstate;              /* per layer: where[E] item[S] | freq[S] touched[S] efreq[E] clock nused hot[S] */
    size_t s_dlayer;             /* bytes of one layer's state */
    int32_t *s_miss;             /* [1+2E] the call's misses */
    unsigned long long *s_dstats; /* [5] hits, misses, evictions, rejected, copies */
    uint8_t *s_dstale;           /* [L] 1: the layer's state could not be cleared at its last upload */
};

static int is_routed(int t) { return t >= QH_T_GATE_Q && t <= QH_T_DOWN_B; }

static void set_err(qmoe_err *err, const char *fmt, ...) {
    if (!err) return;
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(err->msg, sizeof(err->msg), fmt, ap);
    va_end(ap);
}

static void clear_err(qmoe_err *err) {
    if (err) err->msg[0] = 0;
}

static int hip_fail(qmoe_err *err, int rc, const char *what) {
    if (rc == 0) return 0;
    set_err(err, "%s: HIP error %d (%s)", what, rc, hipGetErrorString((hipError_t)rc));
    return -1;
}

static size_t align_up(size_t v) { return (v + ALIGN - 1) / ALIGN * ALIGN; }

/* element count and element size of each tensor */
static void tensor_shape(const qmoe_config *c, int t, size_t *count, size_t *esize) {
    const size_t H = (size_t)c->hidden, E = (size_t)c->n_experts, I = (size_t)c->moe_inter;
    const size_t g = (size_t)c->group_size;
    size_t n = 0, es = 2;
    switch (t) {
    case QH_T_ROUTER_W: n = E * H; break;
    case QH_T_ROUTER_BIAS: n = E; es = 4; break;
    case QH_T_GATE_Q: case QH_T_UP_Q: n = E * I * H / 8; es = 4; break;
    case QH_T_GATE_S: case QH_T_GATE_B: case QH_T_UP_S: case QH_T_UP_B: n = E * I * H / g; break;
    case QH_T_DOWN_Q: n = E * H * I / 8; es = 4; break;
    case QH_T_DOWN_S: case QH_T_DOWN_B: n = E * H * I / g; break;
    case QH_T_SH_GATE_Q: case QH_T_SH_UP_Q: n = I * H / 8; es = 4; break;
    case QH_T_SH_GATE_S: case QH_T_SH_GATE_B: case QH_T_SH_UP_S: case QH_T_SH_UP_B: n = I * H / g; break;
    case QH_T_SH_DOWN_Q: n = H * I / 8; es = 4; break;
    case QH_T_SH_DOWN_S: case QH_T_SH_DOWN_B: n = H * I / g; break;
    case QH_T_SHGATE_W: n = H; break;
    case QH_T_NORM_W: n = H; es = 4; break;
    }
    *count = n;
    *esize = es;
}

static int check_config(const qmoe_config *c, qmoe_err *err) {
    if (!c) {
        set_err(err, "config is NULL");
        return -1;
    }
    if (c->group_size != QK_GROUP && c->group_size != 32) {
        set_err(err, "group_size %d unsupported (this build takes %d, or 32 on the GEMV kernels)",
                c->group_size, QK_GROUP);
        return -1;
    }
    if (c->hidden <= 0 || c->hidden % QK_GROUP || c->hidden > 8192) {
        set_err(err, "hidden %d must be a positive multiple of %d and <= 8192", c->hidden, QK_GROUP);
        return -1;
    }
    if (c->moe_inter <= 0 || c->moe_inter % QK_GROUP || c->moe_inter > 8192) {
        set_err(err, "moe_inter %d must be a positive multiple of %d and <= 8192", c->moe_inter,
                QK_GROUP);
        return -1;
    }
    if (c->n_experts <= 0 || c->n_experts > QK_MAX_EXPERTS) {
        set_err(err, "n_experts %d must be in [1, %d]", c->n_experts, QK_MAX_EXPERTS);
        return -1;
    }
    if (c->top_k <= 0 || c->top_k > c->n_experts || c->top_k > QK_MAX_TOPK) {
        set_err(err, "top_k %d must be in [1, min(n_experts, %d)]", c->top_k, QK_MAX_TOPK);
        return -1;
    }
    if (c->n_layers <= 0) {
        set_err(err, "n_layers %d must be positive", c->n_layers);
        return -1;
    }
    if (c->max_tokens <= 0 || (long long)c->max_tokens * (c->top_k + 1) > (1LL << 30)) {
        set_err(err, "max_tokens %d out of range", c->max_tokens);
        return -1;
    }
    if (!(c->rms_eps >= 0.0f)) {
        set_err(err, "rms_eps must be >= 0");
        return -1;
    }
    return 0;
}

/* the layer scratch for n tokens, carved out of one block: region offsets
 * (QH_SC_COUNT of them) and the total */
enum { QH_SC_COUNT = 17 };
static size_t scratch_plan(qk_shape s, size_t n, size_t offs[QH_SC_COUNT]) {
    const size_t E = (size_t)s.E, k = (size_t)s.k, H = (size_t)s.H, I = (size_t)s.I;
    const size_t nw = (n + 31) / 32, rows = n * k + n;
    const size_t plane = n * H > rows * I ? n * H : rows * I;
    const size_t sz[QH_SC_COUNT] = {n * (E + 1) * 4, n * k * 4, n * k * 4, n * 4, (E + 1) * 4, n * k * 4,
                                    n * k * 4, E * nw * 4, E * nw * 4, n * H * 4, rows * I * 4,
                                    rows * H * 4, (3 * E + 1) * 4, qk_mfma_task_bytes(s, (int)n),
                                    plane * 2, plane * 2, plane / 64 * 4};
    size_t total = 0;
    for (int i = 0; i < QH_SC_COUNT; i++) {
        offs[i] = total;
        total = align_up(total + sz[i]);
    }
    return total;
}

static void scratch_bind(qk_scratch *sc, char *b, const size_t offs[QH_SC_COUNT]) {
    sc->logits = (float *)(b + offs[0]);
    sc->idx = (int32_t *)(b + offs[1]);
    sc->w = (float *)(b + offs[2]);
    sc->sg = (float *)(b + offs[3]);
    sc->offsets = (int32_t *)(b + offs[4]);
    sc->perm = (int32_t *)(b + offs[5]);
    sc->pos = (int32_t *)(b + offs[6]);
    sc->bits = (uint32_t *)(b + offs[7]);
    sc->wprefix = (int32_t *)(b + offs[8]);
    sc->xn = (float *)(b + offs[9]);
    sc->h = (float *)(b + offs[10]);
    sc->y = (float *)(b + offs[11]);
    sc->segtab = (int32_t *)(b + offs[12]);
    sc->tasks = (int32_t *)(b + offs[13]);
    sc->ahi = (uint16_t *)(b + offs[14]);
    sc->alo = (uint16_t *)(b + offs[15]);
    sc->ag = (float *)(b + offs[16]);
}

int qmoe_create(qmoe_ctx **out, const qmoe_config *cfg, qmoe_err *err) {
    clear_err(err);
    if (!out) {
        set_err(err, "ctx pointer is NULL");
        return -1;
    }
    *out = NULL;
    if (check_config(cfg, err)) return -1;
    qmoe_ctx *c = (qmoe_ctx *)calloc(1, sizeof(qmoe_ctx));
    if (!c) {
        set_err(err, "out of host memory");
        return -1;
    }
    c->cfg = *cfg;
    c->shape.H = cfg->hidden;
    c->shape.E = cfg->n_experts;
    c->shape.k = cfg->top_k;
    c->shape.I = cfg->moe_inter;
    c->shape.eps = cfg->rms_eps;
    c->shape.g32 = cfg->group_size == 32;
    if (hip_fail(err, (int)hipGetDevice(&c->device), "hipGetDevice")) {
        free(c);
        return -1;
    }
    /* layer layout */
    size_t o = 0;
    for (int t = 0; t < QH_T_COUNT; t++) {
        size_t n, es;
        tensor_shape(cfg, t, &n, &es);
        c->off[t] = o;
        o = align_up(o + n * es);
    }
    c->layer_bytes = o;
    c->last_n = -1;
    c->layers = (qmoe_layer_slot *)calloc((size_t)cfg->n_layers, sizeof(qmoe_layer_slot));
    if (!c->layers) {
        free(c);
        set_err(err, "out of host memory");
        return -1;
    }
    /* scratch */
    size_t offs[QH_SC_COUNT];
    const size_t total = scratch_plan(c->shape, (size_t)cfg->max_tokens, offs);
    c->scratch_bytes = total;
    if (hip_fail(err, (int)hipMalloc(&c->scratch_mem, total), "hipMalloc(scratch)")) {
        free(c->layers);
        free(c);
        return -1;
    }
    scratch_bind(&c->sc, (char *)c->scratch_mem, offs);
    if (hip_fail(err, (int)hipStreamCreateWithFlags(&c->aux, hipStreamNonBlocking), "stream") ||
        hip_fail(err, (int)hipEventCreateWithFlags(&c->ev_fork, hipEventDisableTiming), "event") ||
        hip_fail(err, (int)hipEventCreateWithFlags(&c->ev_join, hipEventDisableTiming), "event")) {
        qmoe_destroy(c);
        return -1;
    }
    *out = c;
    return 0;
}

static void stream_free(qmoe_ctx *c) {
    if (c->s_host) {
        for (int l = 0; l < c->cfg.n_layers; l++)
            if (c->s_host[l]) hipHostFree(c->s_host[l]);
        free(c->s_host);
    }
    if (c->s_pool) hipFree(c->s_pool);
    if (c->s_seg) hipHostFree(c->s_seg);
    if (c->s_segtab) hipFree(c->s_segtab);
    if (c->s_dstate) hipFree(c->s_dstate);
    if (c->s_copy) hipStreamDestroy(c->s_copy);
    for (int l = 0; l < c->cfg.n_layers; l++) {
        if (c->s_ev_used && c->s_ev_used[l]) hipEventDestroy(c->s_ev_used[l]);
        if (c->s_ev_pf && c->s_ev_pf[l]) hipEventDestroy(c->s_ev_pf[l]);
    }
    free(c->s_hdev);
    free(c->s_ev_used);
    free(c->s_ev_pf);
    free(c->s_pf_pending);
    free(c->s_freq);
    free(c->s_trans);
    free(c->s_prev);
    free(c->s_pf_flag);
    free(c->s_ids);
    free(c->s_dstale);
    qmoe_xcache_destroy(c->xc);
    c->s_host = c->s_hdev = NULL;
    c->s_pool = c->s_seg = NULL;
    c->s_segtab = NULL;
    c->s_dstate = NULL;
    c->s_miss = NULL;
    c->s_dstats = NULL;
    c->s_dev = 0;
    c->s_copy = NULL;
    c->s_ev_used = c->s_ev_pf = NULL;
    c->s_pf_pending = NULL;
    c->s_freq = c->s_trans = NULL;
    c->s_prev = c->s_ids = NULL;
    c->s_pf_flag = NULL;
    c->s_dstale = NULL;
    c->xc = NULL;
    c->streamed = 0;
}

void qmoe_destroy(qmoe_ctx *c) {
    if (!c) return;
    if (c->layers)
        for (int l = 0; l < c->cfg.n_layers; l++)
            if (c->layers[l].mem) hipFree(c->layers[l].mem);
    if (c->scratch_mem) hipFree(c->scratch_mem);
    if (c->ev_fork) hipEventDestroy(c->ev_fork);
    if (c->ev_join) hipEventDestroy(c->ev_join);
    if (c->aux) hipStreamDestroy(c->aux);
    if (c->host_x_dev) hipFree(c->host_x_dev);
    if (c->host_out_dev) hipFree(c->host_out_dev);
    if (c->hc_mem)
        for (int l = 0; l < c->cfg.n_layers; l++)
            if (c->hc_mem[l]) hipFree(c->hc_mem[l]);
    if (c->hc_scratch) hipFree(c->hc_scratch);
    if (c->hc_ws) hipFree(c->hc_ws);
    stream_free(c);
    free(c->hc_mem);
    free(c->hc_ready);
    free(c->layers);
    free(c);
}

size_t qmoe_scratch_bytes(const qmoe_ctx *c) { return c ? c->scratch_bytes : 0; }
size_t qmoe_layer_bytes(const qmoe_ctx *c) { return c ? c->layer_bytes : 0; }
const char *qmoe_version(void) { return QMOE_VERSION; }

static int check_layer_index(qmoe_ctx *c, int layer, qmoe_err *err) {
    if (!c) {
        set_err(err, "ctx is NULL");
        return -1;
    }
    if (layer < 0 || layer >= c->cfg.n_layers) {
        set_err(err, "layer %d out of range [0, %d)", layer, c->cfg.n_layers);
        return -1;
    }
    return 0;
}

/* device address of tensor t of a layer: its slot in the layer allocation,
 * or for a routed tensor of a streamed context the layer's slot pool */
static char *dev_tensor(qmoe_ctx *c, int layer, int t) {
    if (c->streamed && is_routed(t))
        return (char *)c->s_pool + (size_t)layer * c->s_pool_layer + c->s_poff[t];
    return (char *)c->layers[layer].mem + c->off[t];
}

static int ensure_layer_mem(qmoe_ctx *c, int layer, qmoe_err *err) {
    qmoe_layer_slot *L = &c->layers[layer];
    if (L->mem) return 0;
    if (hip_fail(err, (int)hipMalloc(&L->mem, c->layer_bytes), "hipMalloc(layer)")) return -1;
    qmoe_layer_weights *d = &L->dev;
    d->router_w = (const uint16_t *)dev_tensor(c, layer, QH_T_ROUTER_W);
    d->router_bias = NULL;
    d->gate_q = (const uint32_t *)dev_tensor(c, layer, QH_T_GATE_Q);
    d->gate_s = (const uint16_t *)dev_tensor(c, layer, QH_T_GATE_S);
    d->gate_b = (const uint16_t *)dev_tensor(c, layer, QH_T_GATE_B);
    d->up_q = (const uint32_t *)dev_tensor(c, layer, QH_T_UP_Q);
    d->up_s = (const uint16_t *)dev_tensor(c, layer, QH_T_UP_S);
    d->up_b = (const uint16_t *)dev_tensor(c, layer, QH_T_UP_B);
    d->down_q = (const uint32_t *)dev_tensor(c, layer, QH_T_DOWN_Q);
    d->down_s = (const uint16_t *)dev_tensor(c, layer, QH_T_DOWN_S);
    d->down_b = (const uint16_t *)dev_tensor(c, layer, QH_T_DOWN_B);
    d->sh_gate_q = (const uint32_t *)dev_tensor(c, layer, QH_T_SH_GATE_Q);
    d->sh_gate_s = (const uint16_t *)dev_tensor(c, layer, QH_T_SH_GATE_S);
    d->sh_gate_b = (const uint16_t *)dev_tensor(c, layer, QH_T_SH_GATE_B);
    d->sh_up_q = (const uint32_t *)dev_tensor(c, layer, QH_T_SH_UP_Q);
    d->sh_up_s = (const uint16_t *)dev_tensor(c, layer, QH_T_SH_UP_S);
    d->sh_up_b = (const uint16_t *)dev_tensor(c, layer, QH_T_SH_UP_B);
    d->sh_down_q = (const uint32_t *)dev_tensor(c, layer, QH_T_SH_DOWN_Q);
    d->sh_down_s = (const uint16_t *)dev_tensor(c, layer, QH_T_SH_DOWN_S);
    d->sh_down_b = (const uint16_t *)dev_tensor(c, layer, QH_T_SH_DOWN_B);
    d->sh_gate_w = (const uint16_t *)dev_tensor(c, layer, QH_T_SHGATE_W);
    d->norm_w = NULL;
    return 0;
}

static const void *host_tensor(const qmoe_layer_weights *h, int t) {
    switch (t) {
    case QH_T_ROUTER_W: return h->router_w;
    case QH_T_ROUTER_BIAS: return h->router_bias;
    case QH_T_GATE_Q: return h->gate_q;
    case QH_T_GATE_S: return h->gate_s;
    case QH_T_GATE_B: return h->gate_b;
    case QH_T_UP_Q: return h->up_q;
    case QH_T_UP_S: return h->up_s;
    case QH_T_UP_B: return h->up_b;
    case QH_T_DOWN_Q: return h->down_q;
    case QH_T_DOWN_S: return h->down_s;
    case QH_T_DOWN_B: return h->down_b;
    case QH_T_SH_GATE_Q: return h->sh_gate_q;
    case QH_T_SH_GATE_S: return h->sh_gate_s;
    case QH_T_SH_GATE_B: return h->sh_gate_b;
    case QH_T_SH_UP_Q: return h->sh_up_q;
    case QH_T_SH_UP_S: return h->sh_up_s;
    case QH_T_SH_UP_B: return h->sh_up_b;
    case QH_T_SH_DOWN_Q: return h->sh_down_q;
    case QH_T_SH_DOWN_S: return h->sh_down_s;
    case QH_T_SH_DOWN_B: return h->sh_down_b;
    case QH_T_SHGATE_W: return h->sh_gate_w;
    case QH_T_NORM_W: return h->norm_w;
    }
    return NULL;
}

static const char *tensor_name(int t) {
    static const char *names[QH_T_COUNT] = {
        "router_w", "router_bias", "gate_q", "gate_s", "gate_b", "up_q", "up_s", "up_b",
        "down_q", "down_s", "down_b", "sh_gate_q", "sh_gate_s", "sh_gate_b", "sh_up_q",
        "sh_up_s", "sh_up_b", "sh_down_q", "sh_down_s", "sh_down_b", "sh_gate_w", "norm_w"};
    return names[t];
}

/* host copy of routed tensor t of a streamed layer (allocated on first use) */
static char *host_tensor_store(qmoe_ctx *c, int layer, int t, qmoe_err *err) {
    if (!c->s_host[layer] &&
        hip_fail(err, (int)hipHostMalloc(&c->s_host[layer], c->s_host_layer, hipHostMallocDefault),
                 "hipHostMalloc(expert store)"))
        return NULL;
    return (char *)c->s_host[layer] + c->s_hoff[t];
}

/* Before a streamed layer's pinned host store or its slots are rewritten:
 * copies of expert pieces out of the store run asynchronously (prefetch on
 * the copy stream, demand misses on the caller's stream) and may still be
 * reading it or filling a slot, so every queued device operation is
 * finished first.  Uploads are not on the per-token path. */
static int stream_quiesce(qmoe_ctx *c, qmoe_err *err) {
    if (!c->streamed) return 0;
    return hip_fail(err, (int)hipDeviceSynchronize(), "wait for expert copies before an upload");
}

/* the device state of a layer back to empty: no resident expert, zero counts */
static int dstate_reset(qmoe_ctx *c, int layer) {
    const int E = c->cfg.n_experts, S = c->s_slots;
    char *p = (char *)c->s_dstate + (size_t)layer * c->s_dlayer;
    const size_t neg = (size_t)(E + S) * 4; /* where, item = -1 */
    if (hipMemset(p, 0xFF, neg) != hipSuccess) return -1;
    return hipMemset(p + neg, 0, c->s_dlayer - neg) == hipSuccess ? 0 : -1;
}

static void dstate_args(qmoe_ctx *c, int layer, QkStreamResolve *a) {
    const int E = c->cfg.n_experts, S = c->s_slots;
    char *p = (char *)c->s_dstate + (size_t)layer * c->s_dlayer;
    a->where = (int32_t *)p;
    a->item = a->where + E;
    a->freq = (uint32_t *)(a->item + S);
    a->touched = a->freq + S;
    a->efreq = a->touched + S;
    a->clock = a->efreq + E;
    a->nused = (int32_t *)(a->clock + 1);
    a->hot = (uint8_t *)(a->nused + 1);
    a->miss = c->s_miss;
    a->stats = c->s_dstats;
    a->E = E;
    a->slots = S;
    a->policy = c->s_policy;
}

/* a layer's weights were replaced: forget its resident experts (after
 * stream_quiesce, so no copy of the old weights is in flight) */
static void stream_layer_written(qmoe_ctx *c, int layer) {
    if (!c->streamed) return;
    if (c->s_dev) c->s_dstale[layer] = dstate_reset(c, layer) != 0; /* refused by the layer call */
    qmoe_xcache_clear(c->xc, layer);
    memset(c->s_pf_flag + (size_t)layer * c->cfg.n_experts, 0, (size_t)c->cfg.n_experts);
    c->s_pf_pending[layer] = 0;
}

int qmoe_upload_layer(qmoe_ctx *c, int layer, const qmoe_layer_weights *h, qmoe_err *err) {
    clear_err(err);
    if (check_layer_index(c, layer, err)) return -1;
    if (!h) {
        set_err(err, "weights pointer is NULL");
        return -1;
    }
    for (int t = 0; t < QH_T_COUNT; t++) {
        if (t == QH_T_ROUTER_BIAS || t == QH_T_NORM_W) continue;
        if (!host_tensor(h, t)) {
            set_err(err, "missing tensor %s for layer %d", tensor_name(t), layer);
            return -1;
        }
    }
    if (ensure_layer_mem(c, layer, err) || stream_quiesce(c, err)) return -1;
    qmoe_layer_slot *L = &c->layers[layer];
    L->ready = 0;
    char *b = (char *)L->mem;
    for (int t = 0; t < QH_T_COUNT; t++) {
        const void *src = host_tensor(h, t);
        if (!src) continue;
        size_t n, es;
        tensor_shape(&c->cfg, t, &n, &es);
        if (c->streamed && is_routed(t)) {
            char *dst = host_tensor_store(c, layer, t, err);
            if (!dst) return -1;
            memcpy(dst, src, n * es);
            continue;
        }
        if (hip_fail(err, (int)hipMemcpy(b + c->off[t], src, n * es, hipMemcpyHostToDevice),
                     "hipMemcpy(upload)"))
            return -1;
    }
    stream_layer_written(c, layer);
    L->dev.router_bias = h->router_bias ? (const float *)(b + c->off[QH_T_ROUTER_BIAS]) : NULL;
    L->dev.norm_w = h->norm_w ? (const float *)(b + c->off[QH_T_NORM_W]) : NULL;
    L->ready = 1;
    return 0;
}

/* ---------------------------------------------- slots for qmoe_st.c */

int qh_ctx_config(qmoe_ctx *c, int layer, qmoe_config *out, qmoe_err *err) {
    if (check_layer_index(c, layer, err)) return -1;
    *out = c->cfg;
    return 0;
}

int qh_host_alloc(void **p, size_t bytes, qmoe_err *err) {
    *p = NULL;
    return hip_fail(err, (int)hipHostMalloc(p, bytes, hipHostMallocDefault), "hipHostMalloc(staging)");
}

void qh_host_free(void *p) {
    if (p) (void)hipHostFree(p);
}

int qh_layer_begin(qmoe_ctx *c, int layer, qmoe_err *err) {
    if (c->layers[layer].mem) c->layers[layer].ready = 0;
    return stream_quiesce(c, err);
}

int qh_layer_slot(qmoe_ctx *c, int layer, int t, void **dst, size_t *bytes, int *on_host,
                  qmoe_err *err) {
    if (t < 0 || t >= QH_T_COUNT) {
        set_err(err, "tensor slot %d out of range", t);
        return -1;
    }
    if (ensure_layer_mem(c, layer, err)) return -1;
    c->layers[layer].ready = 0;
    size_t n, es;
    tensor_shape(&c->cfg, t, &n, &es);
    *bytes = n * es;
    *on_host = c->streamed && is_routed(t);
    if (*on_host) {
        *dst = host_tensor_store(c, layer, t, err);
        return *dst ? 0 : -1;
    }
    *dst = (char *)c->layers[layer].mem + c->off[t];
    return 0;
}

int qh_fill_zero(void *dst, size_t bytes, int on_host, qmoe_err *err) {
    if (on_host) {
        memset(dst, 0, bytes);
        return 0;
    }
    return hip_fail(err, (int)hipMemset(dst, 0, bytes), "hipMemset(zero biases)");
}

int qh_copy_to_slot(void *dst, const void *src, size_t bytes, int on_host, qmoe_err *err) {
    if (on_host) {
        memcpy(dst, src, bytes);
        return 0;
    }
    return hip_fail(err, (int)hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice), "hipMemcpy(checkpoint)");
}

void qh_layer_end(qmoe_ctx *c, int layer, int has_bias, int has_norm) {
    qmoe_layer_slot *L = &c->layers[layer];
    char *b = (char *)L->mem;
    stream_layer_written(c, layer);
    L->dev.router_bias = has_bias ? (const float *)(b + c->off[QH_T_ROUTER_BIAS]) : NULL;
    L->dev.norm_w = has_norm ? (const float *)(b + c->off[QH_T_NORM_W]) : NULL;
    L->ready = 1;
}

int qmoe_synth_layer(qmoe_ctx *c, int layer, uint64_t seed, int with_norm, const float *router_bias,
                     qmoe_err *err) {
    clear_err(err);
    if (check_layer_index(c, layer, err)) return -1;
    if (ensure_layer_mem(c, layer, err) || stream_quiesce(c, err)) return -1;
    qmoe_layer_slot *L = &c->layers[layer];
    L->ready = 0;
    char *b = (char *)L->mem;
    static const struct {
        int t, tag, kind;
        float sd;
    } spec[] = {
        {QH_T_ROUTER_W, QMOE_TAG_ROUTER_W, 0, 0.02f},   {QH_T_GATE_Q, QMOE_TAG_GATE_Q, 2, 0.0f},
        {QH_T_GATE_S, QMOE_TAG_GATE_S, 0, 0.02f},       {QH_T_GATE_B, QMOE_TAG_GATE_B, 0, 0.01f},
        {QH_T_UP_Q, QMOE_TAG_UP_Q, 2, 0.0f},            {QH_T_UP_S, QMOE_TAG_UP_S, 0, 0.02f},
        {QH_T_UP_B, QMOE_TAG_UP_B, 0, 0.01f},           {QH_T_DOWN_Q, QMOE_TAG_DOWN_Q, 2, 0.0f},
        {QH_T_DOWN_S, QMOE_TAG_DOWN_S, 0, 0.02f},       {QH_T_DOWN_B, QMOE_TAG_DOWN_B, 0, 0.01f},
        {QH_T_SH_GATE_Q, QMOE_TAG_SH_GATE_Q, 2, 0.0f},  {QH_T_SH_GATE_S, QMOE_TAG_SH_GATE_S, 0, 0.02f},
        {QH_T_SH_GATE_B, QMOE_TAG_SH_GATE_B, 0, 0.01f}, {QH_T_SH_UP_Q, QMOE_TAG_SH_UP_Q, 2, 0.0f},
        {QH_T_SH_UP_S, QMOE_TAG_SH_UP_S, 0, 0.02f},     {QH_T_SH_UP_B, QMOE_TAG_SH_UP_B, 0, 0.01f},
        {QH_T_SH_DOWN_Q, QMOE_TAG_SH_DOWN_Q, 2, 0.0f},  {QH_T_SH_DOWN_S, QMOE_TAG_SH_DOWN_S, 0, 0.02f},
        {QH_T_SH_DOWN_B, QMOE_TAG_SH_DOWN_B, 0, 0.01f}, {QH_T_SHGATE_W, QMOE_TAG_SHGATE_W, 0, 0.02f},
    };
    /* streamed: routed tensors are generated in a temporary buffer and
     * copied to the host store */
    void *tmp = NULL;
    if (c->streamed) {
        size_t big = 0;
        for (int t = 0; t < QH_T_COUNT; t++) {
            size_t n, es;
            tensor_shape(&c->cfg, t, &n, &es);
            if (is_routed(t) && n * es > big) big = n * es;
        }
        if (hip_fail(err, (int)hipMalloc(&tmp, big), "hipMalloc(synth staging)")) return -1;
    }
    for (size_t i = 0; i < sizeof(spec) / sizeof(spec[0]); i++) {
        size_t n, es;
        tensor_shape(&c->cfg, spec[i].t, &n, &es);
        uint64_t key = qk_tensor_key(seed, (uint32_t)layer, (uint32_t)spec[i].tag);
        const int host = c->streamed && is_routed(spec[i].t);
        char *dst = host ? (char *)tmp : b + c->off[spec[i].t];
        int rc = qk_launch_synth(dst, n, spec[i].kind, key, 0, spec[i].sd, NULL);
        if (!rc && host) {
            char *hd = host_tensor_store(c, layer, spec[i].t, err);
            rc = hd ? (int)hipMemcpy(hd, tmp, n * es, hipMemcpyDeviceToHost) : -1;
            if (!hd) {
                hipFree(tmp);
                return -1;
            }
        }
        if (hip_fail(err, rc, "synth")) {
            if (tmp) hipFree(tmp);
            return -1;
        }
    }
    if (tmp) hipFree(tmp);
    stream_layer_written(c, layer);
    if (with_norm) {
        if (hip_fail(err, qk_launch_synth(b + c->off[QH_T_NORM_W], (size_t)c->cfg.hidden, 3, 0, 0,
                                          1.0f, NULL),
                     "synth(norm)"))
            return -1;
    }
    if (router_bias) {
        if (hip_fail(err, (int)hipMemcpy(b + c->off[QH_T_ROUTER_BIAS], router_bias,
                                         (size_t)c->cfg.n_experts * 4, hipMemcpyHostToDevice),
                     "hipMemcpy(router_bias)"))
            return -1;
    }
    if (hip_fail(err, (int)hipDeviceSynchronize(), "synth sync")) return -1;
    L->dev.router_bias = router_bias ? (const float *)(b + c->off[QH_T_ROUTER_BIAS]) : NULL;
    L->dev.norm_w = with_norm ? (const float *)(b + c->off[QH_T_NORM_W]) : NULL;
    L->ready = 1;
    return 0;
}

int qmoe_synth_fill(void *dst, size_t count, int kind, uint64_t seed, uint32_t layer, uint32_t tag,
                    uint64_t start, float stddev, void *stream, qmoe_err *err) {
    clear_err(err);
    if (!dst && count) {
        set_err(err, "dst is NULL");
        return -1;
    }
    if (kind < 0 || kind > 2) {
        set_err(err, "kind %d must be 0 (bf16 normal), 1 (f32 normal) or 2 (u32 codes)", kind);
        return -1;
    }
    return hip_fail(err, qk_launch_synth(dst, count, kind, qk_tensor_key(seed, layer, tag), start,
                                         stddev, stream),
                    "synth_fill");
}

int qmoe_layer_device_weights(qmoe_ctx *c, int layer, qmoe_layer_weights *out, qmoe_err *err) {
    clear_err(err);
    if (check_layer_index(c, layer, err)) return -1;
    if (!c->layers[layer].ready) {
        set_err(err, "layer %d has no weights", layer);
        return -1;
    }
    if (!out) {
        set_err(err, "out is NULL");
        return -1;
    }
    *out = c->layers[layer].dev;
    return 0;
}

/* ------------------------------------------------------------ stages */

static int check_call(qmoe_ctx *c, int layer, int n, qmoe_err *err) {
    if (check_layer_index(c, layer, err)) return -1;
    if (!c->layers[layer].ready) {
        set_err(err, "layer %d has no weights", layer);
        return -1;
    }
    if (n < 0 || n > c->cfg.max_tokens) {
        set_err(err, "n = %d out of range [0, max_tokens = %d]", n, c->cfg.max_tokens);
        return -1;
    }
    return 0;
}

static int check_dtype(int dt, qmoe_err *err) {
    if (dt != QMOE_F32 && dt != QMOE_BF16) {
        set_err(err, "x_dtype %d must be QMOE_F32 (0) or QMOE_BF16 (1)", dt);
        return -1;
    }
    return 0;
}

#define NEED(p, name)                                                                          \
    do {                                                                                       \
        if (!(p)) {                                                                            \
            set_err(err, "%s is NULL", name);                                                  \
            return -1;                                                                         \
        }                                                                                      \
    } while (0)

int qmoe_router(qmoe_ctx *c, int layer, const void *x, int x_dtype, int n, float *logits_out,
                int32_t *idx_out, float *w_out, float *shared_gate_out, float *xn_out,
                void *stream, qmoe_err *err) {
    clear_err(err);
    if (check_call(c, layer, n, err) || check_dtype(x_dtype, err)) return -1;
    if (n == 0) return 0;
    NEED(x, "x");
    NEED(idx_out, "idx_out");
    NEED(w_out, "w_out");
    NEED(shared_gate_out, "shared_gate_out");
    const qmoe_layer_weights *W = &c->layers[layer].dev;
    if (!W->norm_w && xn_out) {
        set_err(err, "xn_out given but layer %d has no norm weight", layer);
        return -1;
    }
    float *xn = W->norm_w ? (xn_out ? xn_out : c->sc.xn) : NULL;
    if (!logits_out && qk_route_mfma_ok(c->shape, n))
        /* only the selection is asked for: MFMA logits, exact where they matter */
        return hip_fail(err,
                        qk_launch_route_mfma(W, c->shape, x, x_dtype == QMOE_BF16, n, c->sc.logits, xn,
                                             c->sc.ahi, c->sc.ag, idx_out, w_out, shared_gate_out,
                                             NULL, NULL, NULL, NULL, stream),
                        "router");
    if (hip_fail(err, qk_launch_router(W, c->shape, x, x_dtype == QMOE_BF16, n, c->sc.logits, xn,
                                       stream),
                 "router"))
        return -1;
    return hip_fail(err, qk_launch_topk(c->shape, n, c->sc.logits, logits_out, idx_out, w_out,
                                        shared_gate_out, stream),
                    "topk");
}

/* Grouped expert stages.  Segments with at least QK_MFMA_MIN_M rows (every
 * segment from QK_MFMA_ALL_N tokens on) run on the MFMA kernels, the others
 * on the GEMV kernels.  The MFMA kernels read
 * their activations as packed operand planes (qk_launch_pack_rows).  The
 * MFMA task list is built from the segment table unless the caller says it
 * is already current. */
/* what the layer's stages run on: the shape, a scratch carve-up, and the
 * second stream of the mixed MFMA + GEMV stages (NULL: both on `stream`,
 * in order) */
typedef struct {
    qk_shape s;
    qk_scratch *sc;
    hipStream_t aux;
    hipEvent_t ev_fork, ev_join;
} stage_env;

static stage_env ctx_env(qmoe_ctx *c) {
    stage_env e = {c->shape, &c->sc, c->aux, c->ev_fork, c->ev_join};
    return e;
}

/* the GEMV kernels of small segments go to the second stream, after
 * everything already on `stream` (fork), and `stream` waits for them before
 * its next launch (join); both work under stream capture */
static int fork(const stage_env *e, void *stream, qmoe_err *err) {
    if (!e->aux) return 0;
    if (hip_fail(err, (int)hipEventRecord(e->ev_fork, (hipStream_t)stream), "fork record")) return -1;
    return hip_fail(err, (int)hipStreamWaitEvent(e->aux, e->ev_fork, 0), "fork wait");
}
static int join(const stage_env *e, void *stream, qmoe_err *err) {
    if (!e->aux) return 0;
    if (hip_fail(err, (int)hipEventRecord(e->ev_join, e->aux), "join record")) return -1;
    return hip_fail(err, (int)hipStreamWaitEvent((hipStream_t)stream, e->ev_join, 0), "join wait");
}

static int mfma_usable(qk_shape s, int n, int stage) {
    const int ok = stage == 2 ? qk_mfma_down_ok(s) : qk_mfma_gateup_ok(s, stage == 0);
    /* the kernels address the operand planes with 32-bit element offsets */
    const size_t elems = stage == 2 ? (size_t)n * (s.k + 1) * s.I : (size_t)n * s.H;
    return ok && elems < ((size_t)1 << 31) && n * (s.k + 1) >= QK_MFMA_MIN_M;
}

/* segments with fewer rows than this go to the GEMV kernels (1 = none) */
static int mfma_min_m(int n) { return n >= QK_MFMA_ALL_N ? 1 : QK_MFMA_MIN_M; }

static int run_gateup(const stage_env *e, const qmoe_layer_weights *W, const void *x, int xbf, int n,
                      const int32_t *perm, const int32_t *segtab, int tasks_ready, int packed,
                      float *h, void *stream, qmoe_err *err) {
    const qk_shape s = e->s;
    const qk_scratch *sc = e->sc;
    const int mm = mfma_usable(s, n, xbf ? 0 : 1);
    const int min_m = mfma_min_m(n);
    const int gemv = !mm || min_m > 1; /* small segments left to the GEMV */
    void *gs = mm && e->aux ? (void *)e->aux : stream;
    int rc;
    if (mm) {
        if (!tasks_ready) {
            rc = qk_launch_mfma_tasks(s, n, segtab, min_m, sc->tasks, stream);
            if (hip_fail(err, rc, "mfma tasks")) return -1;
        }
        if (!packed) {
            rc = qk_launch_pack_rows(x, xbf, (size_t)n, s.H, sc->ahi, xbf ? NULL : sc->alo, sc->ag, stream);
            if (hip_fail(err, rc, "pack x")) return -1;
        }
    }
    if (mm && gemv && fork(e, stream, err)) return -1;
    if (gemv) {
        rc = qk_launch_gateup(W, s, x, xbf, n, perm, segtab, mm ? min_m : 0,
                              mm ? qk_mfma_small_list(s, n, sc->tasks) : NULL, h, gs);
        if (hip_fail(err, rc, "gateup")) return -1;
    }
    if (mm) {
        rc = qk_launch_gateup_mfma(W, s, sc->ahi, xbf ? NULL : sc->alo, sc->ag, n, perm, sc->tasks, h,
                                   stream);
        if (hip_fail(err, rc, "gateup mfma")) return -1;
        if (gemv && join(e, stream, err)) return -1;
    }
    return 0;
}

static int run_down(const stage_env *e, const qmoe_layer_weights *W, const float *h, int n,
                    const int32_t *segtab, int tasks_ready, float *y, void *stream, qmoe_err *err) {
    const qk_shape s = e->s;
    const qk_scratch *sc = e->sc;
    const int mm = mfma_usable(s, n, 2);
    const int min_m = mfma_min_m(n);
    const int gemv = !mm || min_m > 1;
    void *gs = mm && e->aux ? (void *)e->aux : stream;
    int rc;
    if (mm) {
        if (!tasks_ready) {
            rc = qk_launch_mfma_tasks(s, n, segtab, min_m, sc->tasks, stream);
            if (hip_fail(err, rc, "mfma tasks")) return -1;
        }
    }
    if (mm && gemv && fork(e, stream, err)) return -1;
    if (gemv) {
        rc = qk_launch_down(W, s, h, n, segtab, mm ? min_m : 0,
                            mm ? qk_mfma_small_list(s, n, sc->tasks) : NULL, y, gs);
        if (hip_fail(err, rc, "down")) return -1;
    }
    if (mm) {
        rc = qk_launch_down_mfma(W, s, h, n, sc->tasks, y, stream);
        if (hip_fail(err, rc, "down mfma")) return -1;
        if (gemv && join(e, stream, err)) return -1;
    }
    return 0;
}

int qmoe_dispatch(qmoe_ctx *c, const int32_t *idx, int n, int32_t *offsets_out, int32_t *perm_out,
                  int32_t *segments_out, void *stream, qmoe_err *err) {
    clear_err(err);
    if (!c) {
        set_err(err, "ctx is NULL");
        return -1;
    }
    if (n < 0 || n > c->cfg.max_tokens) {
        set_err(err, "n = %d out of range [0, max_tokens = %d]", n, c->cfg.max_tokens);
        return -1;
    }
    NEED(offsets_out, "offsets_out");
    NEED(segments_out, "segments_out");
    if (n == 0) {
        /* nothing routed: all offsets 0 and no segments */
        int32_t *z = (int32_t *)calloc((size_t)c->cfg.n_experts + 1, sizeof(int32_t));
        if (!z) {
            set_err(err, "out of host memory");
            return -1;
        }
        int rc = (int)hipMemcpyAsync(offsets_out, z, ((size_t)c->cfg.n_experts + 1) * 4,
                                     hipMemcpyHostToDevice, (hipStream_t)stream);
        if (!rc)
            rc = (int)hipMemcpyAsync(segments_out, z, 4, hipMemcpyHostToDevice, (hipStream_t)stream);
        if (!rc) rc = (int)hipStreamSynchronize((hipStream_t)stream);
        free(z);
        return hip_fail(err, rc, "dispatch(n=0)");
    }
    NEED(idx, "idx");
    NEED(perm_out, "perm_out");
    return hip_fail(err, qk_launch_dispatch(c->shape, n, idx, offsets_out, perm_out, c->sc.pos,
                                            segments_out, c->sc.bits, 0, c->sc.wprefix, 0,
                                            NULL, stream),
                    "dispatch");
}

int qmoe_expert_gateup(qmoe_ctx *c, int layer, const void *x, int x_dtype, int n,
                       const int32_t *perm, const int32_t *segments, float *h_out, void *stream,
                       qmoe_err *err) {
    clear_err(err);
    if (check_call(c, layer, n, err) || check_dtype(x_dtype, err)) return -1;
    if (c->streamed) {
        set_err(err, "expert stage calls are not available with streamed experts "
                     "(qmoe_layer_forward routes and stages them)");
        return -1;
    }
    if (n == 0) return 0;
    NEED(x, "x");
    NEED(perm, "perm");
    NEED(segments, "segments");
    NEED(h_out, "h_out");
    const stage_env e = ctx_env(c);
    return run_gateup(&e, &c->layers[layer].dev, x, x_dtype == QMOE_BF16, n, perm, segments, 0, 0, h_out,
                      stream, err);
}

int qmoe_expert_gateup_topk(qmoe_ctx *c, int layer, const void *x, int x_dtype,
                            const float *logits, int32_t *idx_out, float *w_out,
                            float *shared_gate_out, int32_t *perm_out, int32_t *segments_out,
                            float *h_out, void *stream, qmoe_err *err) {
    clear_err(err);
    if (check_call(c, layer, 1, err) || check_dtype(x_dtype, err)) return -1;
    if (c->streamed) {
        set_err(err, "expert stage calls are not available with streamed experts "
                     "(qmoe_layer_forward routes and stages them)");
        return -1;
    }
    if (!qk_gateup_topk_supported(c->shape)) {
        set_err(err, "one-token gate/up with top-k needs hidden/32 a power of two >= 64 (hidden = %d)",
                c->cfg.hidden);
        return -1;
    }
    NEED(x, "x");
    NEED(logits, "logits");
    NEED(idx_out, "idx_out");
    NEED(w_out, "w_out");
    NEED(shared_gate_out, "shared_gate_out");
    NEED(perm_out, "perm_out");
    NEED(segments_out, "segments_out");
    NEED(h_out, "h_out");
    return hip_fail(err, qk_launch_gateup_topk(&c->layers[layer].dev, c->shape, x,
                                               x_dtype == QMOE_BF16, logits, idx_out, w_out,
                                               shared_gate_out, perm_out, c->sc.pos, segments_out,
                                               h_out, stream),
                    "gate/up + top-k");
}

int qmoe_expert_down(qmoe_ctx *c, int layer, const float *h, int n, const int32_t *segments,
                     float *y_out, void *stream, qmoe_err *err) {
    clear_err(err);
    if (check_call(c, layer, n, err)) return -1;
    if (c->streamed) {
        set_err(err, "expert stage calls are not available with streamed experts "
                     "(qmoe_layer_forward routes and stages them)");
        return -1;
    }
    if (n == 0) return 0;
    NEED(h, "h");
    NEED(segments, "segments");
    NEED(y_out, "y_out");
    const stage_env e = ctx_env(c);
    return run_down(&e, &c->layers[layer].dev, h, n, segments, 0, y_out, stream, err);
}

int qmoe_expert_ffn(qmoe_ctx *c, int layer, const void *x, int x_dtype, int n, const int32_t *perm,
                    const int32_t *segments, float *y_out, void *stream, qmoe_err *err) {
    if (qmoe_expert_gateup(c, layer, x, x_dtype, n, perm, segments, c ? c->sc.h : NULL, stream, err))
        return -1;
    return qmoe_expert_down(c, layer, c->sc.h, n, segments, y_out, stream, err);
}

int qmoe_combine(qmoe_ctx *c, const float *y, const int32_t *perm, const float *w,
                 const float *shared_gate, int n, const void *x_residual, int x_dtype, float *out,
                 void *stream, qmoe_err *err) {
    clear_err(err);
    if (!c) {
        set_err(err, "ctx is NULL");
        return -1;
    }
    if (n < 0 || n > c->cfg.max_tokens) {
        set_err(err, "n = %d out of range [0, max_tokens = %d]", n, c->cfg.max_tokens);
        return -1;
    }
    if (x_residual && check_dtype(x_dtype, err)) return -1;
    if (n == 0) return 0;
    NEED(y, "y");
    NEED(perm, "perm");
    NEED(w, "w");
    NEED(shared_gate, "shared_gate");
    NEED(out, "out");
    if (hip_fail(err, qk_launch_invert_perm(n * c->cfg.top_k, perm, c->sc.pos, stream), "invert"))
        return -1;
    return hip_fail(err, qk_launch_combine(c->shape, n, y, c->sc.pos, w, shared_gate, x_residual,
                                           x_dtype == QMOE_BF16, out, NULL, NULL, 0, stream),
                    "combine");
}

/* the layer on checked arguments; with hyper set the combine also applies
 * the hyper connection's inject update (out may then be NULL) */
static int layer_forward_streamed(qmoe_ctx *c, int layer, const void *x, int xbf, int n,
                                  float *out, int residual, float *hyper, const float *inject,
                                  void *stream, qmoe_err *err);

/* the layer of resident weights W on the stages of e */
static int layer_core(const stage_env *e, const qmoe_layer_weights *W, int hc,
                      const void *x, int xbf, int n, float *out, int residual, float *hyper,
                      const float *inject, void *stream, qmoe_err *err) {
    const qk_shape s = e->s;
    qk_scratch *sc = e->sc;
    int rc;
    float *xn = W->norm_w ? sc->xn : NULL;
    const void *xf = W->norm_w ? (const void *)sc->xn : x;
    const int xf_bf = W->norm_w ? 0 : xbf;
    /* many tokens: router + top-k on MFMA with the exact logits of the
     * candidates (the top-k launch below is then skipped); else, when the
     * gate/up runs on MFMA and the tiled router takes n, the router also
     * writes the gate/up's operand planes (no packing launch) */
    const int rfast = qk_route_mfma_ok(s, n);
    const int rpack = !rfast && n >= 2 && mfma_usable(s, n, xf_bf ? 0 : 1) && qk_router_packs(s, n);
    /* the MFMA router's last launch also writes the gate/up's operand planes
     * when the gate/up runs on MFMA, and the dispatch's token bitmask (its
     * n >= QK_ROUTE_MFMA_MIN_N always takes qk_launch_dispatch below); its
     * wn2 scratch then goes to h, which the gate/up writes later */
    const int rmm = rfast && mfma_usable(s, n, xf_bf ? 0 : 1);
    if (rfast)
        rc = qk_launch_route_mfma(W, s, x, xbf, n, sc->logits, xn, sc->ahi, rmm ? sc->h : sc->ag, sc->idx,
                                  sc->w, sc->sg, sc->bits, rmm ? sc->ahi : NULL,
                                  rmm && !xf_bf ? sc->alo : NULL, rmm ? sc->ag : NULL, stream);
    else if (rpack)
        rc = qk_launch_router_pack(W, s, x, xbf, n, sc->logits, xn, sc->ahi, xf_bf ? NULL : sc->alo,
                                   sc->ag, stream);
    else
        rc = qk_launch_router(W, s, x, xbf, n, sc->logits, xn, stream);
    if (hip_fail(err, rc, "router")) return -1;
    if (n == 1 && qk_gateup_topk_supported(s) && qk_down_combine_lds(s, n) > 0) {
        /* one token: top-k inside the gate/up launch, then down + combine */
        rc = qk_launch_gateup_topk(W, s, xf, xf_bf, sc->logits, sc->idx, sc->w, sc->sg, sc->perm,
                                   sc->pos, sc->segtab, sc->h, stream);
        if (hip_fail(err, rc, "gate/up + top-k")) return -1;
        rc = qk_launch_down_combine(W, s, sc->h, n, sc->segtab, sc->pos, sc->w, sc->sg,
                                    residual ? x : NULL, xbf, out, hyper, inject, hc, stream);
        return hip_fail(err, rc, "down+combine");
    }
    /* the dispatch also builds the MFMA task list when the gate/up runs on
     * MFMA (one launch fewer) */
    const int gu_mm = n >= 2 && mfma_usable(s, n, xf_bf ? 0 : 1);
    int32_t *tasks = gu_mm ? sc->tasks : NULL;
    if (n <= QK_SMALL_N && n * s.k <= QK_SMALL_NK) {
        /* offsets are not used by the layer; qmoe_last_routing derives them */
        rc = qk_launch_topk_dispatch_small(s, n, sc->logits, NULL, sc->idx, sc->w, sc->sg,
                                           n == 1 ? NULL : sc->offsets, sc->perm, sc->pos,
                                           sc->segtab, mfma_min_m(n), tasks, stream);
        if (hip_fail(err, rc, "topk+dispatch")) return -1;
    } else {
        if (!rfast) {
            rc = qk_launch_topk(s, n, sc->logits, NULL, sc->idx, sc->w, sc->sg, stream);
            if (hip_fail(err, rc, "topk")) return -1;
        }
        rc = qk_launch_dispatch(s, n, sc->idx, sc->offsets, sc->perm, sc->pos, sc->segtab,
                                sc->bits, rfast, sc->wprefix, mfma_min_m(n), tasks, stream);
        if (hip_fail(err, rc, "dispatch")) return -1;
    }
    if (run_gateup(e, W, xf, xf_bf, n, sc->perm, sc->segtab, gu_mm, rpack || rmm, sc->h, stream, err))
        return -1;
    if (!mfma_usable(s, n, 2) && qk_down_combine_lds(s, n) > 0) {
        rc = qk_launch_down_combine(W, s, sc->h, n, sc->segtab, sc->pos, sc->w, sc->sg,
                                    residual ? x : NULL, xbf, out, hyper, inject, hc, stream);
        return hip_fail(err, rc, "down+combine");
    }
    if (run_down(e, W, sc->h, n, sc->segtab, mfma_usable(s, n, xf_bf ? 0 : 1), sc->y, stream, err))
        return -1;
    rc = qk_launch_combine(s, n, sc->y, sc->pos, sc->w, sc->sg, residual ? x : NULL, xbf, out,
                           hyper, inject, hc, stream);
    return hip_fail(err, rc, "combine");
}

static int layer_forward(qmoe_ctx *c, int layer, const void *x, int xbf, int n, float *out,
                         int residual, float *hyper, const float *inject, void *stream,
                         qmoe_err *err) {
    if (c->streamed)
        return layer_forward_streamed(c, layer, x, xbf, n, out, residual, hyper, inject, stream, err);
    c->last_n = n;
    const stage_env e = ctx_env(c);
    return layer_core(&e, &c->layers[layer].dev, hyper ? c->hc : 0, x, xbf, n, out,
                      residual, hyper, inject, stream, err);
}

int qmoe_layer_forward_noalloc(const qmoe_config *cfg, const qmoe_layer_weights *w, const void *x,
                               int x_dtype, int n, float *out, int flags, void *stream,
                               qmoe_err *err) {
    clear_err(err);
    if (!cfg || !w) {
        set_err(err, "%s is NULL", cfg ? "dev_weights" : "cfg");
        return -1;
    }
    if (check_config(cfg, err) || check_dtype(x_dtype, err)) return -1;
    if (flags & ~QMOE_RESIDUAL) {
        set_err(err, "unknown flags 0x%x", flags);
        return -1;
    }
    if (n < 0 || n > cfg->max_tokens) {
        set_err(err, "n = %d out of range [0, max_tokens = %d]", n, cfg->max_tokens);
        return -1;
    }
    const void *need[] = {w->router_w,  w->gate_q,    w->gate_s,    w->gate_b,    w->up_q,
                          w->up_s,      w->up_b,      w->down_q,    w->down_s,    w->down_b,
                          w->sh_gate_q, w->sh_gate_s, w->sh_gate_b, w->sh_up_q,   w->sh_up_s,
                          w->sh_up_b,   w->sh_down_q, w->sh_down_s, w->sh_down_b, w->sh_gate_w};
    for (size_t i = 0; i < sizeof(need) / sizeof(need[0]); i++)
        if (!need[i]) {
            set_err(err, "dev_weights: tensor %zu of the layout is NULL (only router_bias and norm_w "
                         "may be)", i);
            return -1;
        }
    if (n == 0) return 0;
    NEED(x, "x");
    NEED(out, "out");
    const qk_shape s = {cfg->hidden, cfg->n_experts, cfg->top_k, cfg->moe_inter, cfg->rms_eps,
                        cfg->group_size == 32};
    size_t offs[QH_SC_COUNT];
    const size_t bytes = scratch_plan(s, (size_t)n, offs);
    if (bytes > QK_NOALLOC_SCRATCH_BYTES) {
        set_err(err, "n = %d needs %zu bytes of scratch at this shape; the static scratch holds %zu "
                     "(call with fewer tokens)", n, bytes, (size_t)QK_NOALLOC_SCRATCH_BYTES);
        return -1;
    }
    void *base = NULL;
    if (hip_fail(err, qk_noalloc_scratch(&base), "static scratch address")) return -1;
    qk_scratch sc;
    scratch_bind(&sc, (char *)base, offs);
    const stage_env e = {s, &sc, NULL, NULL, NULL}; /* every stage on `stream` */
    return layer_core(&e, w, 0, x, x_dtype == QMOE_BF16, n, out, (flags & QMOE_RESIDUAL) != 0,
                      NULL, NULL, stream, err);
}

int qmoe_layer_forward(qmoe_ctx *c, int layer, const void *x, int x_dtype, int n, float *out,
                       int flags, void *stream, qmoe_err *err) {
    clear_err(err);
    if (check_call(c, layer, n, err) || check_dtype(x_dtype, err)) return -1;
    if (flags & ~QMOE_RESIDUAL) {
        set_err(err, "unknown flags 0x%x", flags);
        return -1;
    }
    if (n == 0) return 0;
    NEED(x, "x");
    NEED(out, "out");
    return layer_forward(c, layer, x, x_dtype == QMOE_BF16, n, out, (flags & QMOE_RESIDUAL) != 0,
                         NULL, NULL, stream, err);
}

/* ------------------------------------------------------ hyper connection */

static void hc_shape(const qmoe_ctx *c, int t, size_t *count, size_t *esize) {
    const size_t D = (size_t)c->hc * c->cfg.hidden, R = (size_t)c->hc_R, g = QK_GROUP;
    size_t n = 0, es = 2;
    switch (t) {
    case QH_HC_NORM: n = D; es = 4; break;
    case QH_HC_DOWN_Q: n = R * D / 8; es = 4; break;
    case QH_HC_DOWN_S: case QH_HC_DOWN_B: n = R * D / g; break;
    case QH_HC_UP_Q: n = D * R / 8; es = 4; break;
    case QH_HC_UP_S: case QH_HC_UP_B: n = D * R / g; break;
    case QH_HC_INJECT_W: n = (size_t)c->hc * D; break;
    }
    *count = n;
    *esize = es;
}

int qmoe_hc_enable(qmoe_ctx *c, int hc_count, int hc_lowrank, qmoe_err *err) {
    clear_err(err);
    if (!c) {
        set_err(err, "ctx is NULL");
        return -1;
    }
    if (c->hc) {
        if (c->hc == hc_count && c->hc_R == hc_lowrank) return 0;
        set_err(err, "hyper connection already enabled with hc_count %d, hc_lowrank %d", c->hc,
                c->hc_R);
        return -1;
    }
    if (!qk_hc_shape_ok(hc_count, c->cfg.hidden, hc_lowrank)) {
        set_err(err, "hc_count %d, hc_lowrank %d unsupported with hidden %d (needs 1 <= hc_count <= 8, "
                     "hc_lowrank a multiple of 64 in [64, 2048], hidden <= 2048)",
                hc_count, hc_lowrank, c->cfg.hidden);
        return -1;
    }
    c->hc = hc_count;
    c->hc_R = hc_lowrank;
    size_t o = 0;
    for (int t = 0; t < QH_HC_COUNT; t++) {
        size_t n, es;
        hc_shape(c, t, &n, &es);
        c->hc_off[t] = o;
        o = align_up(o + n * es);
    }
    c->hc_layer_bytes = o;
    c->hc_mem = (void **)calloc((size_t)c->cfg.n_layers, sizeof(void *));
    c->hc_ready = (int *)calloc((size_t)c->cfg.n_layers, sizeof(int));
    const size_t n = (size_t)c->cfg.max_tokens, H = (size_t)c->cfg.hidden;
    const size_t D = (size_t)hc_count * H, R = (size_t)hc_lowrank;
    const size_t sz[4] = {n * D * 4, n * R * 4, n * (size_t)hc_count * 4, n * H * 4};
    size_t total = 0, offs[4];
    for (int i = 0; i < 4; i++) {
        offs[i] = total;
        total = align_up(total + sz[i]);
    }
    if (!c->hc_mem || !c->hc_ready ||
        hip_fail(err, (int)hipMalloc(&c->hc_scratch, total), "hipMalloc(hc scratch)")) {
        if (!c->hc_mem || !c->hc_ready) set_err(err, "out of host memory");
        free(c->hc_mem);
        free(c->hc_ready);
        c->hc_mem = NULL;
        c->hc_ready = NULL;
        c->hc_scratch = NULL;
        c->hc = c->hc_R = 0;
        return -1;
    }
    if (c->cfg.max_tokens >= QK_HC_MM_MIN &&
        hip_fail(err, (int)hipMalloc(&c->hc_ws, qk_hc_mm_ws_bytes(hc_count, c->cfg.hidden, hc_lowrank,
                                                                 c->cfg.max_tokens)),
                 "hipMalloc(hc workspace)")) {
        hipFree(c->hc_scratch);
        free(c->hc_mem);
        free(c->hc_ready);
        c->hc_mem = NULL;
        c->hc_ready = NULL;
        c->hc_scratch = c->hc_ws = NULL;
        c->hc = c->hc_R = 0;
        return -1;
    }
    char *b = (char *)c->hc_scratch;
    c->hc_normed = (float *)(b + offs[0]);
    c->hc_down = (float *)(b + offs[1]);
    c->hc_inject = (float *)(b + offs[2]);
    c->hc_mixed = (float *)(b + offs[3]);
    return 0;
}

static int hc_check_layer(qmoe_ctx *c, int layer, qmoe_err *err) {
    if (check_layer_index(c, layer, err)) return -1;
    if (!c->hc) {
        set_err(err, "hyper connection not enabled (qmoe_hc_enable)");
        return -1;
    }
    return 0;
}

static int hc_ensure_mem(qmoe_ctx *c, int layer, qmoe_err *err) {
    if (c->hc_mem[layer]) return 0;
    return hip_fail(err, (int)hipMalloc(&c->hc_mem[layer], c->hc_layer_bytes), "hipMalloc(hc layer)");
}

static void hc_dev(const qmoe_ctx *c, int layer, qmoe_hc_weights *d) {
    char *b = (char *)c->hc_mem[layer];
    d->hc_norm = (const float *)(b + c->hc_off[QH_HC_NORM]);
    d->down_q = (const uint32_t *)(b + c->hc_off[QH_HC_DOWN_Q]);
    d->down_s = (const uint16_t *)(b + c->hc_off[QH_HC_DOWN_S]);
    d->down_b = (const uint16_t *)(b + c->hc_off[QH_HC_DOWN_B]);
    d->up_q = (const uint32_t *)(b + c->hc_off[QH_HC_UP_Q]);
    d->up_s = (const uint16_t *)(b + c->hc_off[QH_HC_UP_S]);
    d->up_b = (const uint16_t *)(b + c->hc_off[QH_HC_UP_B]);
    d->inject_w = (const uint16_t *)(b + c->hc_off[QH_HC_INJECT_W]);
}

int qh_hc_config(qmoe_ctx *c, int layer, int *hc, int *lowrank, int *d, qmoe_err *err) {
    if (hc_check_layer(c, layer, err)) return -1;
    *hc = c->hc;
    *lowrank = c->hc_R;
    *d = c->cfg.hidden;
    return 0;
}

int qh_hc_slot(qmoe_ctx *c, int layer, int t, void **dst, size_t *bytes, int *on_host,
               qmoe_err *err) {
    *on_host = 0;
    if (t < 0 || t >= QH_HC_COUNT) {
        set_err(err, "hc tensor slot %d out of range", t);
        return -1;
    }
    if (hc_ensure_mem(c, layer, err)) return -1;
    c->hc_ready[layer] = 0;
    size_t n, es;
    hc_shape(c, t, &n, &es);
    *dst = (char *)c->hc_mem[layer] + c->hc_off[t];
    *bytes = n * es;
    return 0;
}

int qh_hc_begin(qmoe_ctx *c, int layer, qmoe_err *err) {
    (void)err;
    c->hc_ready[layer] = 0;
    return 0;
}
void qh_hc_end(qmoe_ctx *c, int layer) { c->hc_ready[layer] = 1; }

int qmoe_hc_upload_layer(qmoe_ctx *c, int layer, const qmoe_hc_weights *h, qmoe_err *err) {
    clear_err(err);
    if (hc_check_layer(c, layer, err)) return -1;
    NEED(h, "weights");
    const void *src[QH_HC_COUNT] = {h->hc_norm, h->down_q, h->down_s, h->down_b,
                                    h->up_q,    h->up_s,   h->up_b,   h->inject_w};
    static const char *names[QH_HC_COUNT] = {"hc_norm", "down_q", "down_s", "down_b",
                                             "up_q",    "up_s",   "up_b",   "inject_w"};
    for (int t = 0; t < QH_HC_COUNT; t++)
        if (!src[t]) {
            set_err(err, "missing hyper-connection tensor %s for layer %d", names[t], layer);
            return -1;
        }
    if (hc_ensure_mem(c, layer, err)) return -1;
    c->hc_ready[layer] = 0;
    for (int t = 0; t < QH_HC_COUNT; t++) {
        size_t n, es;
        hc_shape(c, t, &n, &es);
        if (hip_fail(err, (int)hipMemcpy((char *)c->hc_mem[layer] + c->hc_off[t], src[t], n * es,
                                         hipMemcpyHostToDevice),
                     "hipMemcpy(hc upload)"))
            return -1;
    }
    c->hc_ready[layer] = 1;
    return 0;
}

int qmoe_hc_synth_layer(qmoe_ctx *c, int layer, uint64_t seed, qmoe_err *err) {
    clear_err(err);
    if (hc_check_layer(c, layer, err)) return -1;
    if (hc_ensure_mem(c, layer, err)) return -1;
    c->hc_ready[layer] = 0;
    static const struct {
        int t, tag, kind;
        float sd;
    } spec[] = {
        {QH_HC_NORM, 0, 3, 1.0f},
        {QH_HC_DOWN_Q, QMOE_TAG_HC_DOWN_Q, 2, 0.0f}, {QH_HC_DOWN_S, QMOE_TAG_HC_DOWN_S, 0, 0.02f},
        {QH_HC_DOWN_B, QMOE_TAG_HC_DOWN_B, 0, 0.01f}, {QH_HC_UP_Q, QMOE_TAG_HC_UP_Q, 2, 0.0f},
        {QH_HC_UP_S, QMOE_TAG_HC_UP_S, 0, 0.02f},     {QH_HC_UP_B, QMOE_TAG_HC_UP_B, 0, 0.01f},
        {QH_HC_INJECT_W, QMOE_TAG_HC_INJECT_W, 0, 0.02f},
    };
    for (size_t i = 0; i < sizeof(spec) / sizeof(spec[0]); i++) {
        size_t n, es;
        hc_shape(c, spec[i].t, &n, &es);
        const uint64_t key = qk_tensor_key(seed, (uint32_t)layer, (uint32_t)spec[i].tag);
        if (hip_fail(err, qk_launch_synth((char *)c->hc_mem[layer] + c->hc_off[spec[i].t], n,
                                          spec[i].kind, key, 0, spec[i].sd, NULL),
                     "synth(hc)"))
            return -1;
    }
    if (hip_fail(err, (int)hipDeviceSynchronize(), "synth sync")) return -1;
    c->hc_ready[layer] = 1;
    return 0;
}

int qmoe_hc_device_weights(qmoe_ctx *c, int layer, qmoe_hc_weights *out, qmoe_err *err) {
    clear_err(err);
    if (hc_check_layer(c, layer, err)) return -1;
    if (!c->hc_ready[layer]) {
        set_err(err, "layer %d has no hyper-connection weights", layer);
        return -1;
    }
    NEED(out, "out");
    hc_dev(c, layer, out);
    return 0;
}

static int hc_check_call(qmoe_ctx *c, int layer, int n, qmoe_err *err) {
    if (hc_check_layer(c, layer, err)) return -1;
    if (!c->hc_ready[layer]) {
        set_err(err, "layer %d has no hyper-connection weights", layer);
        return -1;
    }
    if (n < 0 || n > c->cfg.max_tokens) {
        set_err(err, "n = %d out of range [0, max_tokens = %d]", n, c->cfg.max_tokens);
        return -1;
    }
    return 0;
}

/* gated_residual (model.c:728-796): two GEMV launches for few tokens, the
 * MFMA path for many; normed_out (may be NULL) receives normed */
static int run_hc_mix(qmoe_ctx *c, int layer, const float *hyper, int n, float *mixed,
                      float *inject, float *normed_out, void *stream, qmoe_err *err) {
    qmoe_hc_weights W;
    hc_dev(c, layer, &W);
    const int d = c->cfg.hidden;
    int rc;
    if (n >= QK_HC_MM_MIN && c->hc_ws) {
        rc = qk_launch_hc_mm(hyper, W.hc_norm, W.down_q, W.down_s, W.down_b, W.up_q, W.up_s, W.up_b,
                             W.inject_w, c->hc, d, c->hc_R, n, 1e-6f, c->hc_ws, mixed, inject,
                             normed_out, stream);
        return hip_fail(err, rc, "hc mix (MFMA)");
    }
    rc = qk_launch_hc_down(hyper, W.hc_norm, W.down_q, W.down_s, W.down_b, W.inject_w, c->hc, d,
                               c->hc_R, n, 1e-6f, c->hc_normed, c->hc_down, inject, stream);
    if (hip_fail(err, rc, "hc norm+down+inject")) return -1;
    rc = qk_launch_hc_upmix(W.up_q, W.up_s, W.up_b, c->hc_down, c->hc_normed, c->hc, d, c->hc_R, n,
                            mixed, stream);
    if (hip_fail(err, rc, "hc up+mix")) return -1;
    if (normed_out &&
        hip_fail(err, (int)hipMemcpyAsync(normed_out, c->hc_normed,
                                          (size_t)n * c->hc * d * sizeof(float),
                                          hipMemcpyDeviceToDevice, (hipStream_t)stream),
                 "copy normed"))
        return -1;
    return 0;
}

int qmoe_hc_mix(qmoe_ctx *c, int layer, const float *hyper, int n, float *mixed_out,
                float *inject_out, float *normed_out, void *stream, qmoe_err *err) {
    clear_err(err);
    if (hc_check_call(c, layer, n, err)) return -1;
    if (n == 0) return 0;
    NEED(hyper, "hyper");
    NEED(mixed_out, "mixed_out");
    return run_hc_mix(c, layer, hyper, n, mixed_out, inject_out ? inject_out : c->hc_inject,
                      normed_out, stream, err);
}

int qmoe_hc_inject(qmoe_ctx *c, const float *inject, const float *moe_out, int n, float *hyper,
                   void *stream, qmoe_err *err) {
    clear_err(err);
    if (!c) {
        set_err(err, "ctx is NULL");
        return -1;
    }
    if (!c->hc) {
        set_err(err, "hyper connection not enabled (qmoe_hc_enable)");
        return -1;
    }
    if (n < 0 || n > c->cfg.max_tokens) {
        set_err(err, "n = %d out of range [0, max_tokens = %d]", n, c->cfg.max_tokens);
        return -1;
    }
    if (n == 0) return 0;
    NEED(inject, "inject");
    NEED(moe_out, "moe_out");
    NEED(hyper, "hyper");
    return hip_fail(err, qk_launch_hc_inject(inject, moe_out, c->hc, c->cfg.hidden, n, hyper, stream),
                    "hc inject");
}

int qmoe_hc_layer_forward(qmoe_ctx *c, int layer, float *hyper, int n, float *moe_out,
                          void *stream, qmoe_err *err) {
    clear_err(err);
    if (hc_check_call(c, layer, n, err) || check_call(c, layer, n, err)) return -1;
    if (n == 0) return 0;
    NEED(hyper, "hyper");
    if (run_hc_mix(c, layer, hyper, n, c->hc_mixed, c->hc_inject, NULL, stream, err)) return -1;
    return layer_forward(c, layer, c->hc_mixed, 0, n, moe_out, 0, hyper, c->hc_inject, stream, err);
}

/* ------------------------------------------------------ expert streaming */

int qmoe_stream_enable(qmoe_ctx *c, int slots, int policy, int prefetch, qmoe_err *err) {
    clear_err(err);
    if (!c) {
        set_err(err, "ctx is NULL");
        return -1;
    }
    const int E = c->cfg.n_experts, L = c->cfg.n_layers;
    if (c->streamed) {
        if (slots == c->s_slots && policy == c->s_policy &&
            (prefetch < 0 ? c->s_dev : !c->s_dev && prefetch == c->s_prefetch))
            return 0;
        set_err(err, "expert streaming already enabled with %d slots per layer, policy %d, prefetch %d",
                c->s_slots, c->s_policy, c->s_dev ? -1 : c->s_prefetch);
        return -1;
    }
    for (int l = 0; l < L; l++)
        if (c->layers[l].mem) {
            set_err(err, "qmoe_stream_enable must precede every layer upload (layer %d is allocated)", l);
            return -1;
        }
    const long long need = (long long)c->cfg.max_tokens * c->cfg.top_k < E
                               ? (long long)c->cfg.max_tokens * c->cfg.top_k : E;
    if (slots < need || slots > E) {
        set_err(err, "slots_per_layer %d must be in [%lld, %d] (one call routes up to "
                     "min(n_experts, max_tokens * top_k) experts)", slots, need, E);
        return -1;
    }
    if (policy < QMOE_CACHE_LRU || policy > QMOE_CACHE_ADAPTIVE || prefetch < -1 || prefetch > E) {
        set_err(err, "policy %d or prefetch %d out of range", policy, prefetch);
        return -1;
    }
    if (prefetch < 0 && qk_stream_resolve_lds(E, slots) > 65536) {
        set_err(err, "device-resolved streaming keeps a layer's slot cache in 64 KB of LDS: "
                     "%d experts and %d slots need %zu bytes", E, slots, qk_stream_resolve_lds(E, slots));
        return -1;
    }
    /* layouts: resident tensors in the layer allocation, routed ones in the
     * host copy (E experts) and the slot pool (slots experts) */
    size_t o = 0, ho = 0, po = 0, eb = 0;
    for (int t = 0; t < QH_T_COUNT; t++) {
        size_t n, es;
        tensor_shape(&c->cfg, t, &n, &es);
        if (is_routed(t)) {
            c->s_tb[t] = n * es / (size_t)E;
            eb += c->s_tb[t];
            c->s_hoff[t] = ho;
            ho = align_up(ho + n * es);
            c->s_poff[t] = po;
            po = align_up(po + c->s_tb[t] * (size_t)slots);
            c->off[t] = 0;
        } else {
            c->s_tb[t] = 0;
            c->off[t] = o;
            o = align_up(o + n * es);
        }
    }
    c->s_host_layer = ho;
    c->s_pool_layer = po;
    c->s_expert_bytes = eb;
    c->s_slots = slots;
    c->s_dev = prefetch < 0;
    c->s_prefetch = prefetch < 0 ? 0 : prefetch;
    c->s_policy = policy;
    c->streamed = 1; /* stream_free resets it on failure */
    int ok = hip_fail(err, (int)hipMalloc(&c->s_pool, po * (size_t)L), "hipMalloc(expert slots)") == 0 &&
             hip_fail(err, (int)hipHostMalloc((void **)&c->s_seg, (size_t)(3 * E + 1) * 4,
                                              hipHostMallocDefault), "hipHostMalloc(segments)") == 0 &&
             hip_fail(err, (int)hipMalloc((void **)&c->s_segtab, (size_t)(3 * E + 1) * 4),
                      "hipMalloc(segments)") == 0 &&
             hip_fail(err, (int)hipStreamCreateWithFlags(&c->s_copy, hipStreamNonBlocking),
                      "stream") == 0;
    if (ok) {
        c->s_host = (void **)calloc((size_t)L, sizeof(void *));
        c->s_hdev = (void **)calloc((size_t)L, sizeof(void *));
        c->s_ev_used = (hipEvent_t *)calloc((size_t)L, sizeof(hipEvent_t));
        c->s_ev_pf = (hipEvent_t *)calloc((size_t)L, sizeof(hipEvent_t));
        c->s_pf_pending = (int *)calloc((size_t)L, sizeof(int));
        c->s_freq = (uint32_t *)calloc((size_t)L * E, sizeof(uint32_t));
        c->s_trans = (uint32_t *)calloc((size_t)L * E * E, sizeof(uint32_t));
        c->s_prev = (int32_t *)calloc((size_t)L * (E + 1), sizeof(int32_t));
        c->s_pf_flag = (uint8_t *)calloc((size_t)L * E, 1);
        c->s_ids = (int32_t *)calloc((size_t)E, sizeof(int32_t));
        c->s_dstale = (uint8_t *)calloc((size_t)L, 1);
        ok = c->s_host && c->s_hdev && c->s_ev_used && c->s_ev_pf && c->s_pf_pending && c->s_freq && c->s_trans &&
             c->s_prev && c->s_pf_flag && c->s_ids && c->s_dstale;
        if (!ok) set_err(err, "out of host memory");
    }
    for (int l = 0; ok && l < L; l++)
        ok = hip_fail(err, (int)hipEventCreateWithFlags(&c->s_ev_used[l], hipEventDisableTiming), "event") == 0 &&
             hip_fail(err, (int)hipEventCreateWithFlags(&c->s_ev_pf[l], hipEventDisableTiming), "event") == 0;
    if (ok && qmoe_xcache_create(&c->xc, L, E, slots, policy, eb, err)) ok = 0;
    if (ok && c->s_dev) {
        /* where, item, freq, touched, efreq, clock, nused as 4-byte words, hot bytes */
        c->s_dlayer = align_up((size_t)(2 * E + 3 * slots + 2) * 4 + (size_t)slots);
        const size_t tail = (size_t)(1 + 2 * E) * 4;
        ok = hip_fail(err, (int)hipMalloc(&c->s_dstate, c->s_dlayer * (size_t)L + align_up(tail) + 64),
                      "hipMalloc(device cache state)") == 0;
        if (ok) {
            c->s_miss = (int32_t *)((char *)c->s_dstate + c->s_dlayer * (size_t)L);
            c->s_dstats = (unsigned long long *)((char *)c->s_miss + align_up(tail));
            ok = hip_fail(err, (int)hipMemset(c->s_miss, 0, align_up(tail) + 64), "clear state") == 0;
            for (int l = 0; ok && l < L; l++)
                if (dstate_reset(c, l)) ok = hip_fail(err, (int)hipErrorInvalidValue, "clear state") == 0;
        }
    }
    if (!ok) {
        stream_free(c);
        /* back to the resident layout */
        size_t r = 0;
        for (int t = 0; t < QH_T_COUNT; t++) {
            size_t n, es;
            tensor_shape(&c->cfg, t, &n, &es);
            c->off[t] = r;
            r = align_up(r + n * es);
        }
        c->layer_bytes = r;
        return -1;
    }
    c->layer_bytes = o;
    return 0;
}

int qmoe_stream_get_stats(qmoe_ctx *c, qmoe_stream_stats *out, qmoe_err *err) {
    clear_err(err);
    if (!c || !out) {
        set_err(err, "%s is NULL", c ? "out" : "ctx");
        return -1;
    }
    if (!c->streamed) {
        set_err(err, "expert streaming not enabled");
        return -1;
    }
    uint64_t k[5] = {0, 0, 0, 0, 0};
    if (c->s_dev) {
        unsigned long long d[5];
        if (hip_fail(err, (int)hipMemcpy(d, c->s_dstats, sizeof(d), hipMemcpyDeviceToHost), "stats to host"))
            return -1;
        for (int i = 0; i < 5; i++) k[i] = d[i];
        k[4] *= c->s_expert_bytes;
    } else {
        qmoe_xcache_counts(c->xc, k);
        k[4] = c->s_bytes_in;
    }
    out->hits = k[0];
    out->misses = k[1];
    out->evictions = k[2];
    out->rejected = k[3];
    out->bytes_in = k[4];
    out->prefetched = c->s_prefetched;
    out->prefetch_hits = c->s_prefetch_hits;
    return 0;
}

/* batches of whole-expert copies from a layer's host copy into its slots
 * (one k_expert_copy launch per batch) */
static int xc_begin(qmoe_ctx *c, int layer, QkExpertCopy *a, qmoe_err *err) {
    if (!c->s_hdev[layer] &&
        hip_fail(err, (int)hipHostGetDevicePointer(&c->s_hdev[layer], c->s_host[layer], 0), "host mapping"))
        return -1;
    const void *hd = c->s_hdev[layer];
    char *p = (char *)c->s_pool + (size_t)layer * c->s_pool_layer;
    for (int t = QH_T_GATE_Q, i = 0; t <= QH_T_DOWN_B; t++, i++) {
        a->src[i] = (const char *)hd + c->s_hoff[t];
        a->dst[i] = p + c->s_poff[t];
        a->tb[i] = c->s_tb[t];
    }
    a->n = 0;
    return 0;
}

static int xc_flush(QkExpertCopy *a, hipStream_t st, qmoe_err *err) {
    const int rc = qk_launch_expert_copy(a, st);
    a->n = 0;
    return hip_fail(err, rc, "expert copy");
}

static int xc_add(qmoe_ctx *c, QkExpertCopy *a, int e, int slot, hipStream_t st, qmoe_err *err) {
    a->pair[a->n][0] = e;
    a->pair[a->n][1] = slot;
    a->n++;
    c->s_bytes_in += c->s_expert_bytes;
    return a->n == QK_XC_MAX ? xc_flush(a, st, err) : 0;
}

/* prefetch requests of one layer (request(prefetch=True), streaming.py:360-398):
 * experts not resident go into slots on the copy stream, after the
 * compute stream's last use of that layer's slots */
static int stream_prefetch(qmoe_ctx *c, int layer, const int32_t *ids, int cnt, qmoe_err *err) {
    const int E = c->cfg.n_experts;
    int issued = 0;
    QkExpertCopy xc;
    if (xc_begin(c, layer, &xc, err)) return -1;
    for (int i = 0; i < cnt; i++) {
        const int e = ids[i];
        if (qmoe_xcache_peek(c->xc, layer, e) >= 0) continue;
        if (!issued &&
            hip_fail(err, (int)hipStreamWaitEvent(c->s_copy, c->s_ev_used[layer], 0), "prefetch wait"))
            return -1;
        int ev;
        const int slot = qmoe_xcache_put(c->xc, layer, e, 0, c->s_freq[(size_t)layer * E + e] >= 4, &ev);
        if (slot < 0) continue;
        if (ev >= 0) c->s_pf_flag[(size_t)layer * E + ev] = 0;
        if (xc_add(c, &xc, e, slot, c->s_copy, err)) return -1;
        c->s_pf_flag[(size_t)layer * E + e] = 1;
        c->s_prefetched++;
        issued = 1;
    }
    if (issued && xc_flush(&xc, c->s_copy, err)) return -1;
    if (issued) {
        if (hip_fail(err, (int)hipEventRecord(c->s_ev_pf[layer], c->s_copy), "prefetch record")) return -1;
        c->s_pf_pending[layer] = 1;
    }
    return 0;
}

/* the `cnt` largest of score[0..E) that are > 0, ties to the lower id */
static int top_scores(const uint64_t *score, int E, int cnt, int32_t *out) {
    int m = 0;
    for (int e = 0; e < E; e++) {
        if (!score[e]) continue;
        int pos = m < cnt ? m : cnt;
        while (pos > 0 && score[out[pos - 1]] < score[e]) pos--;
        if (pos >= cnt) continue;
        const int last = m < cnt ? m : cnt - 1;
        for (int j = last; j > pos; j--) out[j] = out[j - 1];
        out[pos] = e;
        if (m < cnt) m++;
    }
    return m;
}

/* record_route and prefetch_predictions (streaming.py:400-435): count the
 * experts after the previous call's experts of this layer and each
 * expert's routed slots, mark the frequent ones hot (>= 4), then request
 * the most likely experts of this layer (transitions from this call's
 * experts, else frequency, plus twice the next layer's frequency) and the
 * most frequent of the next layer.  Ties go to the lower expert id (the
 * MLX runtime keeps first-seen order). */
static int stream_after_route(qmoe_ctx *c, int layer, const int32_t *ids, const int32_t *counts,
                              int U, qmoe_err *err) {
    const int E = c->cfg.n_experts, L = c->cfg.n_layers;
    uint32_t *freq = c->s_freq + (size_t)layer * E;
    uint32_t *trans = c->s_trans + (size_t)layer * E * E;
    int32_t *prev = c->s_prev + (size_t)layer * (E + 1);
    for (int j = 0; j < prev[0]; j++)
        for (int i = 0; i < U; i++) trans[(size_t)prev[1 + j] * E + ids[i]]++;
    for (int i = 0; i < U; i++) freq[ids[i]] += (uint32_t)counts[i];
    prev[0] = U;
    for (int i = 0; i < U; i++) prev[1 + i] = ids[i];
    for (int i = 0; i < U; i++) qmoe_xcache_mark_hot(c->xc, layer, ids[i], freq[ids[i]] >= 4);
    if (!c->s_prefetch) return 0;
    uint64_t *cand = (uint64_t *)calloc((size_t)E, sizeof(uint64_t));
    int32_t *pick = (int32_t *)malloc((size_t)c->s_prefetch * sizeof(int32_t));
    if (!cand || !pick) {
        free(cand);
        free(pick);
        set_err(err, "out of host memory");
        return -1;
    }
    int any = 0;
    for (int i = 0; i < U; i++)
        for (int e = 0; e < E; e++) {
            cand[e] += trans[(size_t)ids[i] * E + e];
            any |= trans[(size_t)ids[i] * E + e] != 0;
        }
    if (!any)
        for (int e = 0; e < E; e++) cand[e] = freq[e];
    const uint32_t *nfreq = layer + 1 < L ? c->s_freq + (size_t)(layer + 1) * E : NULL;
    if (nfreq)
        for (int e = 0; e < E; e++) cand[e] += 2ull * nfreq[e];
    int m = top_scores(cand, E, c->s_prefetch, pick);
    int rc = stream_prefetch(c, layer, pick, m, err);
    if (!rc && nfreq) {
        for (int e = 0; e < E; e++) cand[e] = nfreq[e];
        m = top_scores(cand, E, c->s_prefetch, pick);
        rc = stream_prefetch(c, layer + 1, pick, m, err);
    }
    free(cand);
    free(pick);
    return rc;
}

/* the expert kernels on the slot pool, segments over slots (c->s_segtab) */
static int streamed_experts(qmoe_ctx *c, const qmoe_layer_weights *W, const void *x, int xbf,
                            const void *xf, int xf_bf, int n, float *out, int residual, float *hyper,
                            const float *inject, int hc, void *stream, qmoe_err *err) {
    const qk_shape s = c->shape;
    qk_scratch *sc = &c->sc;
    const stage_env e = ctx_env(c);
    const int gu_mm = n >= 2 && mfma_usable(s, n, xf_bf ? 0 : 1);
    int rc = run_gateup(&e, W, xf, xf_bf, n, sc->perm, c->s_segtab, 0, 0, sc->h, stream, err);
    if (rc) return rc;
    if (!mfma_usable(s, n, 2) && qk_down_combine_lds(s, n) > 0)
        return hip_fail(err, qk_launch_down_combine(W, s, sc->h, n, c->s_segtab, sc->pos, sc->w, sc->sg,
                                                    residual ? x : NULL, xbf, out, hyper, inject, hc,
                                                    stream),
                        "down+combine");
    rc = run_down(&e, W, sc->h, n, c->s_segtab, gu_mm, sc->y, stream, err);
    if (rc) return rc;
    return hip_fail(err, qk_launch_combine(s, n, sc->y, sc->pos, sc->w, sc->sg, residual ? x : NULL, xbf,
                                           out, hyper, inject, hc, stream),
                    "combine");
}

/* the layer with streamed experts: route and dispatch on the GPU, bring
 * the routed experts into the layer's slots (one host round trip for the
 * segment table), remap the segment table to slots, then the same expert
 * kernels on the slot pool */
static int layer_forward_streamed(qmoe_ctx *c, int layer, const void *x, int xbf, int n,
                                  float *out, int residual, float *hyper, const float *inject,
                                  void *stream, qmoe_err *err) {
    c->last_n = n;
    const qmoe_layer_weights *W = &c->layers[layer].dev;
    const qk_shape s = c->shape;
    qk_scratch *sc = &c->sc;
    const int hc = hyper ? c->hc : 0, E = s.E;
    hipStream_t st = (hipStream_t)stream;
    int rc;
    float *xn = W->norm_w ? sc->xn : NULL;
    const int rfast = qk_route_mfma_ok(s, n);
    if (rfast)
        rc = qk_launch_route_mfma(W, s, x, xbf, n, sc->logits, xn, sc->ahi, sc->ag, sc->idx, sc->w,
                                  sc->sg, sc->bits, NULL, NULL, NULL, stream);
    else
        rc = qk_launch_router(W, s, x, xbf, n, sc->logits, xn, stream);
    if (hip_fail(err, rc, "router")) return -1;
    const void *xf = W->norm_w ? (const void *)sc->xn : x;
    const int xf_bf = W->norm_w ? 0 : xbf;
    if (n <= QK_SMALL_N && n * s.k <= QK_SMALL_NK) {
        rc = qk_launch_topk_dispatch_small(s, n, sc->logits, NULL, sc->idx, sc->w, sc->sg,
                                           n == 1 ? NULL : sc->offsets, sc->perm, sc->pos,
                                           sc->segtab, 1, NULL, stream);
        if (hip_fail(err, rc, "topk+dispatch")) return -1;
    } else {
        if (!rfast) {
            rc = qk_launch_topk(s, n, sc->logits, NULL, sc->idx, sc->w, sc->sg, stream);
            if (hip_fail(err, rc, "topk")) return -1;
        }
        rc = qk_launch_dispatch(s, n, sc->idx, sc->offsets, sc->perm, sc->pos, sc->segtab, sc->bits,
                                rfast, sc->wprefix, 1, NULL, stream);
        if (hip_fail(err, rc, "dispatch")) return -1;
    }
    if (c->s_dev) {
        /* residency decided on the device: remap, then copy the misses, all
         * on the call's stream with no host round trip */
        if (c->s_dstale[layer]) {
            set_err(err, "the slot cache of layer %d could not be cleared after its upload", layer);
            return -1;
        }
        QkStreamResolve r;
        dstate_args(c, layer, &r);
        r.segtab = sc->segtab;
        r.out = c->s_segtab;
        QkExpertCopy xd;
        if (xc_begin(c, layer, &xd, err)) return -1;
        const int max_pairs = n * s.k < E ? n * s.k : E;
        if (hip_fail(err, qk_launch_stream_resolve(&r, stream), "stream resolve") ||
            hip_fail(err, qk_launch_expert_copy_list(&xd, c->s_miss, max_pairs, stream), "expert copy"))
            return -1;
        return streamed_experts(c, W, x, xbf, xf, xf_bf, n, out, residual, hyper, inject, hc, stream, err);
    }
    if (hip_fail(err, (int)hipMemcpyAsync(c->s_seg, sc->segtab, (size_t)(3 * E + 1) * 4,
                                          hipMemcpyDeviceToHost, st), "segments to host") ||
        hip_fail(err, (int)hipStreamSynchronize(st), "segments sync"))
        return -1;
    const int U = c->s_seg[0];
    if (U < 0 || U > c->s_slots || U > E) {
        set_err(err, "layer %d routed %d experts, more than its %d slots", layer, U, c->s_slots);
        return -1;
    }
    if (c->s_pf_pending[layer]) {
        if (hip_fail(err, (int)hipStreamWaitEvent(st, c->s_ev_pf[layer], 0), "prefetch join")) return -1;
        c->s_pf_pending[layer] = 0;
    }
    int32_t *cnt = (int32_t *)malloc((size_t)(U > 0 ? U : 1) * sizeof(int32_t));
    if (!cnt) {
        set_err(err, "out of host memory");
        return -1;
    }
    QkExpertCopy xc;
    if (xc_begin(c, layer, &xc, err)) {
        free(cnt);
        return -1;
    }
    for (int i = 0; i < U; i++) {
        const int e = c->s_seg[1 + 3 * i];
        c->s_ids[i] = e;
        cnt[i] = c->s_seg[3 + 3 * i];
        if (e < 0 || e >= E) {
            free(cnt);
            set_err(err, "segment %d names expert %d", i, e);
            return -1;
        }
        int slot = qmoe_xcache_get(c->xc, layer, e);
        if (slot >= 0) {
            uint8_t *f = &c->s_pf_flag[(size_t)layer * E + e];
            if (*f) {
                c->s_prefetch_hits++;
                *f = 0;
            }
            qmoe_xcache_pin(c->xc, layer, e, 1);
        } else {
            int ev;
            slot = qmoe_xcache_put(c->xc, layer, e, 1, c->s_freq[(size_t)layer * E + e] >= 4, &ev);
            if (slot < 0) {
                free(cnt);
                set_err(err, "no slot for expert %d of layer %d", e, layer);
                return -1;
            }
            if (ev >= 0) c->s_pf_flag[(size_t)layer * E + ev] = 0;
            if (xc_add(c, &xc, e, slot, st, err)) {
                free(cnt);
                return -1;
            }
        }
        c->s_seg[1 + 3 * i] = slot;
    }
    if (xc.n && xc_flush(&xc, st, err)) {
        free(cnt);
        return -1;
    }
    for (int i = 0; i < U; i++) qmoe_xcache_pin(c->xc, layer, c->s_ids[i], 0);
    if (hip_fail(err, (int)hipMemcpyAsync(c->s_segtab, c->s_seg, (size_t)(3 * U + 1) * 4,
                                          hipMemcpyHostToDevice, st), "segments to device")) {
        free(cnt);
        return -1;
    }
    rc = streamed_experts(c, W, x, xbf, xf, xf_bf, n, out, residual, hyper, inject, hc, stream, err);
    if (!rc) rc = hip_fail(err, (int)hipEventRecord(c->s_ev_used[layer], st), "layer record");
    if (!rc) rc = stream_after_route(c, layer, c->s_ids, cnt, U, err);
    free(cnt);
    return rc;
}

int qmoe_moe_forward_host(qmoe_ctx *c, int layer, const float *x, int n, float *out,
                          qmoe_err *err) {
    clear_err(err);
    if (check_call(c, layer, n, err)) return -1;
    if (n == 0) return 0;
    NEED(x, "x");
    NEED(out, "out");
    const size_t bytes = (size_t)c->cfg.max_tokens * c->cfg.hidden * sizeof(float);
    if (!c->host_x_dev) {
        if (hip_fail(err, (int)hipMalloc((void **)&c->host_x_dev, bytes), "hipMalloc(x)")) return -1;
        if (hip_fail(err, (int)hipMalloc((void **)&c->host_out_dev, bytes), "hipMalloc(out)")) {
            hipFree(c->host_x_dev);
            c->host_x_dev = NULL;
            return -1;
        }
    }
    const size_t nb = (size_t)n * c->cfg.hidden * sizeof(float);
    if (hip_fail(err, (int)hipMemcpy(c->host_x_dev, x, nb, hipMemcpyHostToDevice), "copy x"))
        return -1;
    if (qmoe_layer_forward(c, layer, c->host_x_dev, QMOE_F32, n, c->host_out_dev, 0, NULL, err))
        return -1;
    if (hip_fail(err, (int)hipMemcpy(out, c->host_out_dev, nb, hipMemcpyDeviceToHost), "copy out"))
        return -1;
    return 0;
}

int qmoe_last_routing(qmoe_ctx *c, int n, int32_t *idx_out, float *w_out, float *shared_gate_out,
                      int32_t *offsets_out, int32_t *perm_out, int32_t *segments_out, void *stream,
                      qmoe_err *err) {
    clear_err(err);
    if (!c) {
        set_err(err, "ctx is NULL");
        return -1;
    }
    if (n <= 0 || n != c->last_n) {
        set_err(err, "n = %d does not match the last layer_forward (n = %d)", n, c->last_n);
        return -1;
    }
    const size_t nk = (size_t)n * c->cfg.top_k, E1 = (size_t)c->cfg.n_experts + 1;
    if (offsets_out &&
        hip_fail(err, qk_launch_offsets_from_segtab(c->shape, c->sc.segtab, c->sc.offsets, stream),
                 "last_routing offsets"))
        return -1;
    struct {
        void *dst;
        const void *src;
        size_t bytes;
    } cp[6] = {{idx_out, c->sc.idx, nk * 4},         {w_out, c->sc.w, nk * 4},
               {shared_gate_out, c->sc.sg, (size_t)n * 4}, {offsets_out, c->sc.offsets, E1 * 4},
               {perm_out, c->sc.perm, nk * 4},
               {segments_out, c->sc.segtab, (3 * E1 - 2) * 4}};
    for (int i = 0; i < 6; i++) {
        if (!cp[i].dst) continue;
        if (hip_fail(err, (int)hipMemcpyAsync(cp[i].dst, cp[i].src, cp[i].bytes,
                                              hipMemcpyDeviceToDevice, (hipStream_t)stream),
                     "last_routing copy"))
            return -1;
    }
    return 0;
}
