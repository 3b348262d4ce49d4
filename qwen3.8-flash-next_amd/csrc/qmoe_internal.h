/*
 * qmoe_internal.h -- shared between the C host code (qmoe_host.c) and the
 * HIP kernels (*.hip).  Plain C declarations only: the launchers are
 * extern "C" functions defined in the .hip files and called from C.
 */
#ifndef QMOE_INTERNAL_H
#define QMOE_INTERNAL_H

#include <stddef.h>
#include <stdint.h>

#include "qmoe.h"

#ifdef __cplusplus
extern "C" {
#endif

/* limits of this implementation (checked by qmoe_create) */
#define QK_MAX_EXPERTS 1024
#define QK_MAX_TOPK 64
#define QK_GROUP 64
/* dispatch runs in one workgroup (LDS) when n <= QK_SMALL_N and
 * n*k <= QK_SMALL_NK, else in the multi-kernel global-memory path */
#define QK_SMALL_N 128
#define QK_SMALL_NK 1024

typedef struct {
    int H, E, k, I;
    float eps;
    int g32; /* 1: the experts' q4 groups are 32 columns (GEMV kernels only), 0: 64 */
} qk_shape;

/* device scratch carved out of one allocation by the host */
typedef struct {
    float *logits;     /* [n, E+1]: router logits, column E = shared-gate logit */
    int32_t *idx;      /* [n, k] */
    float *w;          /* [n, k] */
    float *sg;         /* [n] sigmoid(shared gate) */
    int32_t *offsets;  /* [E+1] */
    int32_t *perm;     /* [n*k] */
    int32_t *pos;      /* [n*k] inverse of perm */
    int32_t *segtab;   /* [1+3E]: U, then (expert, first position, count) per routed segment */
    int32_t *tasks;    /* MFMA task list (qk_mfma_task_bytes) */
    uint16_t *ahi;     /* MFMA activation planes: max(n*H, (n*k+n)*I) bf16 each */
    uint16_t *alo;
    float *ag;         /* their group sums: max(n*H, (n*k+n)*I) / 64 */
    uint32_t *bits;    /* [E, ceil(n/32)] token membership bitmask (large dispatch) */
    int32_t *wprefix;  /* [E, ceil(n/32)] per-word exclusive popcount prefix */
    float *xn;         /* [n, H] normalised router input */
    float *h;          /* [n*k+n, I] */
    float *y;          /* [n*k+n, H] */
} qk_scratch;

/* tensor slots inside a layer allocation, in allocation order */
enum {
    QH_T_ROUTER_W, QH_T_ROUTER_BIAS, QH_T_GATE_Q, QH_T_GATE_S, QH_T_GATE_B, QH_T_UP_Q, QH_T_UP_S,
    QH_T_UP_B, QH_T_DOWN_Q, QH_T_DOWN_S, QH_T_DOWN_B, QH_T_SH_GATE_Q, QH_T_SH_GATE_S,
    QH_T_SH_GATE_B, QH_T_SH_UP_Q, QH_T_SH_UP_S, QH_T_SH_UP_B, QH_T_SH_DOWN_Q, QH_T_SH_DOWN_S,
    QH_T_SH_DOWN_B, QH_T_SHGATE_W, QH_T_NORM_W, QH_T_COUNT
};

/* hyper-connection tensor slots inside a layer's hc allocation */
enum {
    QH_HC_NORM, QH_HC_DOWN_Q, QH_HC_DOWN_S, QH_HC_DOWN_B, QH_HC_UP_Q, QH_HC_UP_S, QH_HC_UP_B,
    QH_HC_INJECT_W, QH_HC_COUNT
};

/* host-side access to a context's layer slots (qmoe_host.c), for the
 * checkpoint reader (qmoe_st.c).  A layer being written is not ready until
 * qh_layer_end. */
int qh_ctx_config(qmoe_ctx *c, int layer, qmoe_config *out, qmoe_err *err);
int qh_host_alloc(void **p, size_t bytes, qmoe_err *err);
void qh_host_free(void *p);
int qh_layer_begin(qmoe_ctx *c, int layer, qmoe_err *err);
/* *on_host: the slot is host memory (a routed expert tensor of a context
 * with streamed experts) */
int qh_layer_slot(qmoe_ctx *c, int layer, int t, void **dst, size_t *bytes, int *on_host,
                  qmoe_err *err);
int qh_fill_zero(void *dst, size_t bytes, int on_host, qmoe_err *err);
int qh_copy_to_slot(void *dst, const void *src, size_t bytes, int on_host, qmoe_err *err);
void qh_layer_end(qmoe_ctx *c, int layer, int has_bias, int has_norm);
/* the same for the hyper-connection slots (after qmoe_hc_enable) */
int qh_hc_config(qmoe_ctx *c, int layer, int *hc, int *lowrank, int *d, qmoe_err *err);
int qh_hc_slot(qmoe_ctx *c, int layer, int t, void **dst, size_t *bytes, int *on_host,
               qmoe_err *err);
int qh_hc_begin(qmoe_ctx *c, int layer, qmoe_err *err);
void qh_hc_end(qmoe_ctx *c, int layer);

/* All launchers return a hipError_t value (0 = hipSuccess). */

/* logits[t, 0..E) = x_t . Wr^T (+bias), logits[t, E] = x_t . w_sg; with
 * norm_w set, x is RMS-normalised first and written to xn (if non-NULL) */
int qk_launch_router(const qmoe_layer_weights *W, qk_shape s, const void *x, int x_bf16, int n,
                     float *logits, float *xn, void *stream);
/* qk_router_packs: n tokens take the tiled router, which can also write
 * the MFMA gate/up operand planes of the experts' input (x, or the normed
 * rows) as qk_launch_pack_rows would: qk_launch_router_pack with phi, pg
 * (and plo for f32 or normed input) */
int qk_router_packs(qk_shape s, int n);
int qk_launch_router_pack(const qmoe_layer_weights *W, qk_shape s, const void *x, int x_bf16, int n,
                          float *logits, float *xn, uint16_t *phi, uint16_t *plo, float *pg,
                          void *stream);

/* router + top-k + renorm + sigmoid for n >= QK_ROUTE_MFMA_MIN_N tokens
 * (route_mfma.hip): logits on bf16 MFMA with an error bound per (token,
 * expert), the exact logits recomputed for the experts whose bound reaches
 * the token's top k; the same idx, w, sg (and xn) as qk_launch_router +
 * qk_launch_topk.  logits [n, E+1] is scratch here (no exact logits are
 * left in it); plane [n, H] bf16 and wn2 [E] are scratch.  qk_route_mfma_ok
 * says whether the shape and n are supported.  With bits set, the launch
 * also leaves the dispatch's token bitmask [E][(n+31)/32] as k_fill_u32 +
 * k_setbits would (qk_launch_dispatch with bits_set then skips both); with
 * phi set, the grouped GEMM's operand planes of the rows the gate/up reads
 * (x, or xn with a norm): phi, plo (f32 rows), pg as qk_launch_pack_rows
 * writes them.  wn2 must not overlap them. */
#define QK_ROUTE_MFMA_MIN_N 256
int qk_route_mfma_ok(qk_shape s, int n);
int qk_launch_route_mfma(const qmoe_layer_weights *W, qk_shape s, const void *x, int x_bf16, int n,
                         float *logits, float *xn, uint16_t *plane, float *wn2, int32_t *idx,
                         float *w, float *sg, uint32_t *bits, uint16_t *phi, uint16_t *plo, float *pg,
                         void *stream);

/* top-k + renorm + sigmoid; copies the first E logit columns to logits_out
 * when non-NULL. */
int qk_launch_topk(qk_shape s, int n, const float *logits, float *logits_out, int32_t *idx,
                   float *w, float *sg, void *stream);
/* top-k and the whole dispatch in one single-workgroup launch, for
 * n <= QK_SMALL_N and n*k <= QK_SMALL_NK; offsets may be NULL only for
 * n == 1.  With tasks set (n >= 2) the launch also builds the MFMA task
 * list for segments of at least min_m rows (as qk_launch_mfma_tasks). */
int qk_launch_topk_dispatch_small(qk_shape s, int n, const float *logits, float *logits_out,
                                  int32_t *idx, float *w, float *sg, int32_t *offsets,
                                  int32_t *perm, int32_t *pos, int32_t *segtab, int min_m,
                                  int32_t *tasks, void *stream);
/* dispatch from idx alone (any n); tasks as for qk_launch_topk_dispatch_small;
 * bits_set: the token bitmask in bits is already built (qk_launch_route_mfma) */
int qk_launch_dispatch(qk_shape s, int n, const int32_t *idx, int32_t *offsets, int32_t *perm,
                       int32_t *pos, int32_t *segtab, uint32_t *bits, int bits_set, int32_t *wprefix,
                       int min_m, int32_t *tasks, void *stream);
/* offsets [E+1] from a segment table */
int qk_launch_offsets_from_segtab(qk_shape s, const int32_t *segtab, int32_t *offsets,
                                  void *stream);
/* pos[perm[p]] = p */
int qk_launch_invert_perm(int count, const int32_t *perm, int32_t *pos, void *stream);

/* grouped expert kernels over the segment table (segment 0 = shared expert
 * on all n tokens at rows n*k.., segment i >= 1 = segtab entry i-1).
 * The GEMV kernels take segments with fewer than max_m rows (0 = all);
 * the MFMA kernels take the (segment, row chunk) tasks built by
 * qk_launch_mfma_tasks for segments with at least min_m rows. */
#define QK_MFMA_MIN_M 16
/* from this many tokens on every segment runs on the MFMA kernels: with
 * many small segments the GEMV kernels, which convert the codes again for
 * each row, cost more than MFMA tiles that are mostly padding */
#define QK_MFMA_ALL_N 64
int qk_launch_gateup(const qmoe_layer_weights *W, qk_shape s, const void *x, int x_bf16, int n,
                     const int32_t *perm, const int32_t *segtab, int max_m,
                     const int32_t *seglist, float *h, void *stream);
int qk_launch_down(const qmoe_layer_weights *W, qk_shape s, const float *h, int n,
                   const int32_t *segtab, int max_m, const int32_t *seglist, float *y,
                   void *stream);
int qk_mfma_max_tasks(qk_shape s, int n);
size_t qk_mfma_task_bytes(qk_shape s, int n);
/* the list of segments below min_m rows that the task kernel writes beside
 * the tasks (for the GEMV kernels): [count, segment...] */
int32_t *qk_mfma_small_list(qk_shape s, int n, int32_t *tasks);
/* shapes the MFMA kernels take (x_bf16: gate/up activations are bf16) */
int qk_mfma_gateup_ok(qk_shape s, int x_bf16);
int qk_mfma_down_ok(qk_shape s);
int qk_launch_mfma_tasks(qk_shape s, int n, const int32_t *segtab, int min_m, int32_t *tasks,
                         void *stream);
/* activation rows [rows, K] (bf16 or f32) -> MFMA operand planes: hi (and
 * lo for f32) bf16 in pair order, gsum [rows, K/64] = -128 * group sums */
int qk_launch_pack_rows(const void *x, int x_bf16, size_t rows, int K, uint16_t *hi, uint16_t *lo,
                        float *gsum, void *stream);
int qk_launch_gateup_mfma(const qmoe_layer_weights *W, qk_shape s, const uint16_t *xhi,
                          const uint16_t *xlo, const float *xg, int n, const int32_t *perm,
                          const int32_t *tasks, float *h, void *stream);
/* the down projection reads h [n*k+n, I] f32 itself (no packed planes) */
int qk_launch_down_mfma(const qmoe_layer_weights *W, qk_shape s, const float *h, int n,
                        const int32_t *tasks, float *y, void *stream);
/* one token, layer path: gate/up with the top-k of `logits` selected inside
 * the kernel, which also writes idx, w, sg, perm, pos and the segment
 * table (the form the dispatch produces for one token) */
int qk_gateup_topk_supported(qk_shape s);
int qk_launch_gateup_topk(const qmoe_layer_weights *W, qk_shape s, const void *x, int x_bf16,
                          const float *logits, int32_t *idx, float *w, float *sg, int32_t *perm,
                          int32_t *pos, int32_t *segtab, float *h, void *stream);
/* down projection fused with the combine for n <= QK_DC_MAX_N tokens;
 * bit-identical to qk_launch_down + qk_launch_combine.  qk_down_combine_lds
 * returns its LDS bytes, 0 when it does not apply. */
#define QK_DC_MAX_N 8
#define QK_DC_MAX_LDS 65536
size_t qk_down_combine_lds(qk_shape s, int n);
/* out may be NULL when hyper is set; with hyper [n, hc, H] every copy j
 * of token t becomes fma(inject[t, j], out[t], hyper[t, j]) */
int qk_launch_down_combine(const qmoe_layer_weights *W, qk_shape s, const float *h, int n,
                           const int32_t *segtab, const int32_t *pos, const float *w,
                           const float *sg, const void *x_res, int x_bf16, float *out,
                           float *hyper, const float *inject, int hc, void *stream);
int qk_launch_combine(qk_shape s, int n, const float *y, const int32_t *pos, const float *w,
                      const float *sg, const void *x_res, int x_bf16, float *out, float *hyper,
                      const float *inject, int hc, void *stream);

/* the gated DeltaNet mixer (deltanet.hip) */
typedef struct {
    int d, hk, hv, dk, dv, kc; /* hidden, key/value heads, head dims, conv taps */
} qk_dn_shape;
typedef struct {
    const uint32_t *qkv_q, *z_q, *out_q;
    const uint16_t *qkv_s, *qkv_b, *z_s, *z_b, *out_s, *out_b;
    const uint16_t *a_w, *b_w, *conv_w;
    const float *norm_w, *a_log, *dt_bias;
} qk_dn_dev;
int qk_dn_shape_ok(const qk_dn_shape *s);
/* x [n, d] f32 -> out [n, d]; conv_state and rec_state are updated;
 * mixed [n, conv_dim], z [n, value_dim], a, b [n, hv], core [n, value_dim]
 * and ssp [n, hv, dv/16] are scratch */
/* the gated residual's update after a mixer, fused into the mixer's last
 * launch: hyper[t, j] = fma(inject[t, j], out[t], hyper[t, j]) for j < hc,
 * the arithmetic of qk_launch_hc_inject (hyper NULL or no struct: none) */
#define QK_INJECT_MAX_HC 8
typedef struct {
    float *hyper;         /* [n, hc, d] */
    const float *inject;  /* [n, hc] */
    int hc;
} qk_inject;

int qk_launch_dn(const qk_dn_shape *s, const qk_dn_dev *W, const float *x, int n, float *out,
                 float *conv_state, float *rec_state, float *mixed, float *z, float *a, float *b,
                 float *core, float *ssp, const qk_inject *inj, void *stream);
int qk_launch_dn_zero(float *p, size_t count, void *stream);

/* the full-attention mixer with the QSA indexer (attention.hip) */
typedef struct {
    int d, h, kvh, hd, ih, ihd, budget, comp, cap, rot; /* rot: rotated dims per head */
    float theta;
} qk_at_shape;
typedef struct {
    const uint32_t *q_q, *k_q, *v_q, *o_q;
    const uint16_t *q_s, *q_b, *k_s, *k_b, *v_s, *v_b, *o_s, *o_b;
    const uint16_t *idx_w;
    const float *q_norm, *k_norm, *idx_q_norm, *idx_k_norm;
    const float *rope; /* [positions, rot/2, 2]: cos, sin of pos * theta^(-2i/rot) */
} qk_at_dev;
typedef struct {
    float *qg;    /* [n, 2h*hd] */
    float *kraw;  /* [n, kvh*hd] */
    float *vraw;  /* [n, kvh*hd] */
    float *qk;    /* [n, (ih+1)*ihd] */
    float *qn;    /* [n, h*hd] */
    float *qi;    /* [n, ih*ihd] */
    uint32_t *keep; /* [n, ceil(cap/comp/32)] */
    float *part;  /* [n, h, nchunks, hd+2]: part_units (token, chunk) pairs per head */
    float *ao;    /* [n, h*hd] */
    uint32_t *skey; /* [n, cap/comp] order keys of the block scores */
    long long part_units; /* capacity of part in (token, key chunk) pairs per head */
} qk_at_scratch;
int qk_at_shape_ok(const qk_at_shape *s);
size_t qk_at_sel_lds(const qk_at_shape *s, int nb);
/* x [n, d] f32 at positions offset.. -> out [n, d]; the caches hold len0
 * rows before the call and len0 + n after it (len0 + n <= cap); pooled
 * [cap/comp, ihd] holds the pooled, normed and rotated indexer key of every
 * complete block, len0/comp of them before the call.  pos0 (a multiple of
 * comp) is the position of cache row 0: the masks compare rows with
 * offset - pos0 and block b's pooled key is rotated to pos0 + b*comp. */
int qk_launch_at(const qk_at_shape *s, const qk_at_dev *W, const float *x, int n, int offset, int pos0,
                 int len0, float *out, float *k_cache, float *v_cache, float *idx_keys, float *pooled,
                 const qk_at_scratch *sc, const qk_inject *inj, void *stream);

/* the MLP hyper connection (hyper.hip): shapes it takes (hc <= 8, d and R
 * multiples of 64, d <= 2048, R <= 2048) */
int qk_hc_shape_ok(int hc, int d, int R);
/* from the hyper state [n, hc*d]: normed [n, hc*d], w [n, R] =
 * silu(normed . Wdown^T / hc) (Wdown q4 [R, hc*d/8]) and inject [n, hc] =
 * 2 sigmoid(normed . Winject^T / hc) (Winject bf16 [hc, hc*d]) */
int qk_launch_hc_down(const float *hyper, const float *norm_w, const uint32_t *q, const uint16_t *s,
                      const uint16_t *b, const uint16_t *inject_w, int hc, int d, int R, int n,
                      float eps, float *normed, float *w, float *inject, void *stream);
/* mixed [n, d] = mean_h sigmoid(w . Wup^T)[h*d + i] * normed[h*d + i] */
int qk_launch_hc_upmix(const uint32_t *q, const uint16_t *s, const uint16_t *b, const float *w,
                       const float *normed, int hc, int d, int R, int n, float *mixed,
                       void *stream);
/* the same on MFMA for many tokens (hyper_mm.hip), from this many on */
#define QK_HC_MM_MIN 16
size_t qk_hc_mm_ws_bytes(int hc, int d, int R, int max_n);
int qk_hc_mm_kspl(int hc, int d, int R, int n);
/* mixed [n, d], inject [n, hc] and (if non-NULL) normed [n, hc*d]; ws of
 * qk_hc_mm_ws_bytes(hc, d, R, >= n) bytes */
int qk_launch_hc_mm(const float *hyper, const float *norm_w, const uint32_t *dq, const uint16_t *ds,
                    const uint16_t *db, const uint32_t *uq, const uint16_t *us, const uint16_t *ub,
                    const uint16_t *inject_w, int hc, int d, int R, int n, float eps, void *ws,
                    float *mixed, float *inject, float *normed, void *stream);
/* hyper [n, hc, d]: every copy j of token t becomes fma(inject[t, j], out[t], hyper[t, j]) */
int qk_launch_hc_inject(const float *inject, const float *out, int hc, int d, int n, float *hyper,
                        void *stream);

/* copies of whole experts (the nine routed tensor pieces) from the
 * pinned host store into HBM slots: pair[i] = (expert, slot), src/dst =
 * each piece's base (host-mapped / device), tb = its bytes per expert (a
 * multiple of 16) */
#define QK_XC_PIECES 9
#define QK_XC_MAX 64
typedef struct {
    const char *src[QK_XC_PIECES];
    char *dst[QK_XC_PIECES];
    size_t tb[QK_XC_PIECES];
    int chunks[QK_XC_PIECES]; /* filled by the launcher */
    int chunks_per_expert;
    int n;
    int32_t pair[QK_XC_MAX][2];
} QkExpertCopy;
int qk_launch_expert_copy(const QkExpertCopy *a, void *stream);

/* device-resolved residency of one layer (stream.hip): per layer state in
 * device memory; out = the segment table over slots, miss = [count,
 * (expert, slot)...] for qk_launch_expert_copy_list; stats = hits, misses,
 * evictions, rejected, copies */
typedef struct {
    const int32_t *segtab;  /* [1+3E] expert segments */
    int32_t *out;           /* [1+3E] slot segments */
    int32_t *where;         /* [E] slot or -1 */
    int32_t *item;          /* [S] expert or -1 */
    uint32_t *freq, *touched; /* [S] */
    uint8_t *hot;           /* [S] */
    uint32_t *efreq;        /* [E] routed slots per expert */
    uint32_t *clock;        /* [1] */
    int32_t *nused;         /* [1] */
    int32_t *miss;          /* [1+2E] */
    unsigned long long *stats; /* [5] */
    int E, slots, policy;
} QkStreamResolve;
int qk_launch_stream_resolve(const QkStreamResolve *a, void *stream);
size_t qk_stream_resolve_lds(int E, int slots);
int qk_launch_expert_copy_list(const QkExpertCopy *a, const int32_t *miss, int max_pairs,
                               void *stream);

/* synthetic streams: kind 0 bf16 normal, 1 f32 normal, 2 u32 codes, 3 f32 constant (stddev) */
int qk_launch_synth(void *dst, size_t count, int kind, uint64_t key, uint64_t start, float stddev,
                    void *stream);
uint64_t qk_tensor_key(uint64_t seed, uint32_t layer, uint32_t tag);

/* the static scratch of qmoe_layer_forward_noalloc (noalloc.hip): its size
 * and its device address on the current device (looked up once per device) */
#define QK_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)
int qk_noalloc_scratch(void **ptr);

#ifdef __cplusplus
}
#endif
#endif
