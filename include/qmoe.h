/*
 * qmoe.h -- C ABI of the MI355X MoE-layer library (libqmoe.so).
 *
 * The entry points replace the MoE layer of the reference C port:
 *   c/src/model.c:1281-1405  moe_forward (the layer)
 *   c/src/model.c:1301-1318  router: gemm_bf16 + kernel_topk_indices + renorm
 *   c/src/model.c:1321-1367  unique experts + per-expert token gather
 *   c/src/model.c:1368-1375  routed SwiGLU FFN (gemm_fp32 x3, silu, mul)
 *   c/src/model.c:1376-1403  weighted combine + sigmoid-gated shared expert
 * and follow the conventions of c/src/kernel.h and c/src/util.h:
 *   - row-major tensors, y[M,N] = x[M,K] . W[N,K]^T (weight rows are
 *     output features), caller-owned outputs that are overwritten;
 *   - q4 weights are MLX affine 4-bit: uint32 words of 8 nibbles, low nibble
 *     first (kernel.h:46-50), one bf16 scale and one bf16 bias per group of
 *     `group_size` input columns, w = q*scale + bias;
 *   - every function returns 0 on success or -1 with a message in `err`
 *     (mirrors err_t, util.h:11-27); nothing aborts.
 *
 * Pointers passed to the stage and layer functions are DEVICE pointers
 * (hipMalloc'd or torch CUDA tensors).  Work is enqueued on `stream`
 * (a hipStream_t; NULL = the null stream) and is asynchronous: the caller
 * synchronises.  A context is not thread-safe: calls on one context must
 * not overlap (they share the context's scratch buffers).
 *
 * Weights stay resident in HBM in the checkpoint layout; there is no expert
 * cache and no streaming (the reference's SSD path, model.c:536-674).
 */
#ifndef QMOE_H
#define QMOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct qmoe_ctx qmoe_ctx;

/* error message buffer, as err_t (c/src/util.h:11-13) */
typedef struct {
    char msg[512];
} qmoe_err;

/* activation element types */
enum { QMOE_F32 = 0, QMOE_BF16 = 1 };

/* qmoe_layer_forward flags */
enum {
    QMOE_RESIDUAL = 1 /* out = x + moe(x) (x un-normalised) */
};

/* Layer shape, from the checkpoint's text_config (c/src/model.c:39-154).
 * The reference requires the shared expert's intermediate size to equal
 * moe_intermediate_size (model.c:1391-1395 passes moe_inter as N). */
typedef struct {
    int hidden;      /* H: hidden_size; multiple of 64 */
    int n_experts;   /* E: num_experts, <= 1024 */
    int top_k;       /* k: num_experts_per_tok, 1 <= k <= min(E, 64) */
    int moe_inter;   /* I: moe_intermediate_size; multiple of 64 */
    int group_size;  /* g: the experts' quantization group size (experts_load,
                        model.c:646-651): 64, or 32, which the GEMV kernels
                        take (a group-32 layer runs every segment on them; the
                        MFMA grouped GEMMs take groups of 64) */
    int n_layers;    /* number of resident layers */
    int max_tokens;  /* largest n accepted per call; sizes the scratch */
    float rms_eps;   /* pre-router RMSNorm epsilon (used only when norm_w is set) */
} qmoe_config;

/* One layer's tensors in the checkpoint layout (names: model.c:541-547 and
 * 1902-1923).  Shapes use the config letters above; G = H/g, GI = I/g. */
typedef struct {
    const uint16_t *router_w;   /* [E,H]     bf16  mlp.gate.weight */
    const float *router_bias;   /* [E]       f32   optional logit bias, or NULL */
    const uint32_t *gate_q;     /* [E,I,H/8] u32   mlp.switch_mlp.gate_proj.weight */
    const uint16_t *gate_s;     /* [E,I,G]   bf16  .scales */
    const uint16_t *gate_b;     /* [E,I,G]   bf16  .biases */
    const uint32_t *up_q;       /* [E,I,H/8]       mlp.switch_mlp.up_proj.* */
    const uint16_t *up_s;
    const uint16_t *up_b;
    const uint32_t *down_q;     /* [E,H,I/8]       mlp.switch_mlp.down_proj.* */
    const uint16_t *down_s;     /* [E,H,GI] */
    const uint16_t *down_b;
    const uint32_t *sh_gate_q;  /* [I,H/8]         mlp.shared_expert.gate_proj.* */
    const uint16_t *sh_gate_s;  /* [I,G] */
    const uint16_t *sh_gate_b;
    const uint32_t *sh_up_q;    /* [I,H/8]         mlp.shared_expert.up_proj.* */
    const uint16_t *sh_up_s;
    const uint16_t *sh_up_b;
    const uint32_t *sh_down_q;  /* [H,I/8]         mlp.shared_expert.down_proj.* */
    const uint16_t *sh_down_s;  /* [H,GI] */
    const uint16_t *sh_down_b;
    const uint16_t *sh_gate_w;  /* [H]       bf16  mlp.shared_expert_gate.weight */
    const float *norm_w;        /* [H]       f32   optional pre-router RMSNorm weight, or NULL */
} qmoe_layer_weights;

/* ------------------------------------------------------------ context */

/* Allocates the context, its scratch (sized by max_tokens) on the current
 * HIP device.  Layers are empty until uploaded, bound or synthesised. */
int qmoe_create(qmoe_ctx **ctx, const qmoe_config *cfg, qmoe_err *err);
void qmoe_destroy(qmoe_ctx *ctx);

/* Copies one layer from HOST memory (checkpoint layout) into HBM.
 * Replaces mw_load + experts_load (model.c:213-272, 536-674). */
int qmoe_upload_layer(qmoe_ctx *ctx, int layer, const qmoe_layer_weights *host, qmoe_err *err);

/* ------------------------------------------------------------ checkpoint
 * An index over the *.safetensors files of a checkpoint directory, as the
 * reference's st_index_open / st_find / st_read_tensor
 * (c/src/safetensors.h:51-63, safetensors.c:57-324): every header is parsed
 * and validated (dtype, shape, data range inside the file, no overlapping
 * ranges, no duplicate names); a leading "language_model." is dropped from
 * stored names, and a lookup of "model.X" also tries "language_model.model.X".
 * Host only: no HIP call is made by the index functions. */
typedef struct qmoe_st qmoe_st;

/* element types, in the order of the reference's st_dtype (safetensors.h:10-25) */
enum {
    QMOE_ST_BOOL, QMOE_ST_U8, QMOE_ST_I8, QMOE_ST_U16, QMOE_ST_I16, QMOE_ST_U32, QMOE_ST_I32,
    QMOE_ST_U64, QMOE_ST_I64, QMOE_ST_F16, QMOE_ST_BF16, QMOE_ST_F32, QMOE_ST_F64, QMOE_ST_COUNT
};

/* one indexed tensor (st_tensor, safetensors.h:27-35) */
typedef struct {
    int dtype;        /* QMOE_ST_* */
    int ndim;
    int64_t shape[8];
    int file;         /* index of the file, in sorted file-name order */
    uint64_t offset;  /* absolute byte offset of the data in that file */
    uint64_t nbytes;
} qmoe_st_tensor;

int qmoe_st_open(qmoe_st **ix, const char *dir, qmoe_err *err);
void qmoe_st_close(qmoe_st *ix);
size_t qmoe_st_count(const qmoe_st *ix);
/* the i-th indexed name in sorted order, or NULL past the end */
const char *qmoe_st_name(const qmoe_st *ix, size_t i);
/* 1 and *out filled when the tensor exists, else 0 */
int qmoe_st_find(const qmoe_st *ix, const char *name, qmoe_st_tensor *out);
/* reads a whole tensor into host memory dst of cap bytes */
int qmoe_st_read(const qmoe_st *ix, const char *name, void *dst, size_t cap, qmoe_err *err);
int qmoe_st_dtype_size(int dtype);
const char *qmoe_st_dtype_name(int dtype);

/* Uploads the MoE tensors of checkpoint layer `model_layer` into context
 * layer `layer`, replacing mw_load (model.c:213-272) for mlp.gate,
 * shared_expert.*, shared_expert_gate (model.c:1902-1912) and
 * experts_load (model.c:539-674) for switch_mlp.{gate,up,down}_proj.
 * Every tensor is found and checked against the context's config before
 * any is copied: expert and shared-expert projections must be q4 (U32
 * codes with BF16 .scales; a missing .biases reads as zero, as model.c:250-256),
 * group size = the config's; the router and the shared-expert gate must be
 * dense BF16.  Scales and biases stay bf16 in HBM (exact; the reference
 * widens them to f32 at load).  The layer has no logit bias and no
 * pre-router norm.  Copies go through a 64 MiB pinned staging buffer. */
int qmoe_upload_layer_st(qmoe_ctx *ctx, int layer, const qmoe_st *ix, int model_layer,
                         qmoe_err *err);

/* Fills one layer in HBM with the seeded synthetic distribution used by the
 * benchmarks: codes U{0..15}, scales N(0,0.02), biases N(0,0.01) (bf16),
 * router and shared-expert gate N(0,0.02) (bf16), norm weight ones when
 * with_norm.  router_bias (host, [E] f32) may be NULL.  No counterpart in
 * the reference (which loads checkpoints); used where no checkpoint exists. */
int qmoe_synth_layer(qmoe_ctx *ctx, int layer, uint64_t seed, int with_norm,
                     const float *router_bias, qmoe_err *err);

/* Device pointers of a resident layer (for callers that run the stage
 * functions themselves or inspect weights). */
int qmoe_layer_device_weights(qmoe_ctx *ctx, int layer, qmoe_layer_weights *out, qmoe_err *err);

/* Fills `count` elements of device memory with the synthetic stream
 * (seed, layer, tag) starting at element `start`: kind 0 = bf16 normal,
 * 1 = f32 normal, 2 = u32 codes.  Bench/test helper without a reference
 * counterpart. */
int qmoe_synth_fill(void *dst, size_t count, int kind, uint64_t seed, uint32_t layer,
                    uint32_t tag, uint64_t start, float stddev, void *stream, qmoe_err *err);

/* synthetic stream tags */
enum {
    QMOE_TAG_ROUTER_W = 1,
    QMOE_TAG_GATE_Q = 2, QMOE_TAG_GATE_S = 3, QMOE_TAG_GATE_B = 4,
    QMOE_TAG_UP_Q = 5, QMOE_TAG_UP_S = 6, QMOE_TAG_UP_B = 7,
    QMOE_TAG_DOWN_Q = 8, QMOE_TAG_DOWN_S = 9, QMOE_TAG_DOWN_B = 10,
    QMOE_TAG_SH_GATE_Q = 11, QMOE_TAG_SH_GATE_S = 12, QMOE_TAG_SH_GATE_B = 13,
    QMOE_TAG_SH_UP_Q = 14, QMOE_TAG_SH_UP_S = 15, QMOE_TAG_SH_UP_B = 16,
    QMOE_TAG_SH_DOWN_Q = 17, QMOE_TAG_SH_DOWN_S = 18, QMOE_TAG_SH_DOWN_B = 19,
    QMOE_TAG_SHGATE_W = 20,
    QMOE_TAG_X = 22,
    /* hyper connection (qmoe_hc_synth_layer) and hyper states */
    QMOE_TAG_HC_DOWN_Q = 24, QMOE_TAG_HC_DOWN_S = 25, QMOE_TAG_HC_DOWN_B = 26,
    QMOE_TAG_HC_UP_Q = 27, QMOE_TAG_HC_UP_S = 28, QMOE_TAG_HC_UP_B = 29,
    QMOE_TAG_HC_INJECT_W = 30, QMOE_TAG_HYPER = 31
};

/* ------------------------------------------------------------ stages */

/* (1) Router, model.c:1301-1318 (+ the shared-expert gate dot, model.c:1396).
 *   x [n,H] (x_dtype); when the layer has norm_w, x is RMS-normalised first
 *   (kernel.c:10-20) and the normalised rows are written to xn_out [n,H] f32
 *   (may be NULL).
 *   logits_out [n,E] f32 (may be NULL): x.Wr^T (+ router_bias), reduction in
 *   a fixed order, so selection is reproducible bit for bit.
 *   idx_out [n,k] i32: top-k experts, value descending, ties to the lower id.
 *   w_out [n,k] f32: softmax over the selected logits (renormalised top-k).
 *   shared_gate_out [n] f32: sigmoid(x . w_sg). */
int qmoe_router(qmoe_ctx *ctx, int layer, const void *x, int x_dtype, int n, float *logits_out,
                int32_t *idx_out, float *w_out, float *shared_gate_out, float *xn_out,
                void *stream, qmoe_err *err);

/* (2) Dispatch, model.c:1321-1367: stable counting sort of the flat slots
 *   f = t*k+s by expert.  offsets_out [E+1]: expert e's slots are
 *   perm_out[offsets[e] .. offsets[e+1]), tokens ascending.
 *   segments_out [1+3E]: segments_out[0] = U, the number of experts that
 *   received tokens, then one (expert, offsets[expert], count) triple per
 *   such expert, experts ascending.  This is the reference's `unique` list
 *   (model.c:1321-1332, first-seen order there) with each expert's run of
 *   dispatch positions attached. */
int qmoe_dispatch(qmoe_ctx *ctx, const int32_t *idx, int n, int32_t *offsets_out,
                  int32_t *perm_out, int32_t *segments_out, void *stream, qmoe_err *err);

/* (3) Expert SwiGLU FFN, model.c:1368-1375 and the shared expert
 *   model.c:1388-1395, as two grouped kernels over the segments of
 *   qmoe_dispatch:
 *   gate/up:  h[p] = silu(x[t].Wg_e^T) * (x[t].Wu_e^T)   -> h_out [n*k+n, I]
 *   down:     y[p] = h[p].Wd_e^T                         -> y_out [n*k+n, H]
 *   Row p < n*k belongs to slot perm[p] of the segment whose run contains p;
 *   rows n*k+t are the shared expert on token t.  x is the router input
 *   (xn_out of qmoe_router when the layer has a norm).  Segment entries
 *   that do not fit the layer are skipped. */
int qmoe_expert_gateup(qmoe_ctx *ctx, int layer, const void *x, int x_dtype, int n,
                       const int32_t *perm, const int32_t *segments, float *h_out, void *stream,
                       qmoe_err *err);
int qmoe_expert_down(qmoe_ctx *ctx, int layer, const float *h, int n, const int32_t *segments,
                     float *y_out, void *stream, qmoe_err *err);

/* (2+3) One token (decode): top-k, renormalisation, dispatch and gate/up in
 *   one launch; model.c:1303-1375 for n = 1.  This is the launch
 *   qmoe_layer_forward uses for one token when hidden/32 is a power of two
 *   >= 64.  logits [E+1] f32: the router output before top-k, i.e.
 *   x.Wr^T (+ router_bias) for the E experts followed by the shared-expert
 *   gate logit x.w_sg.  Outputs, as qmoe_router + qmoe_dispatch +
 *   qmoe_expert_gateup would give them for n = 1: idx_out [k], w_out [k],
 *   shared_gate_out [1], perm_out [k], segments_out [1+3k], h_out [k+1, I].
 *   Returns -1 for other shapes (use the separate stages). */
int qmoe_expert_gateup_topk(qmoe_ctx *ctx, int layer, const void *x, int x_dtype,
                            const float *logits, int32_t *idx_out, float *w_out,
                            float *shared_gate_out, int32_t *perm_out, int32_t *segments_out,
                            float *h_out, void *stream, qmoe_err *err);
/* both of the above */
int qmoe_expert_ffn(qmoe_ctx *ctx, int layer, const void *x, int x_dtype, int n,
                    const int32_t *perm, const int32_t *segments, float *y_out, void *stream,
                    qmoe_err *err);

/* (4) Combine, model.c:1376-1403:
 *   out[t] = sum over t's slots in ascending expert order of w[t,s]*y[pos]
 *            + shared_gate[t] * y[n*k+t]   (+ x[t] with QMOE_RESIDUAL)
 *   where pos is the position of slot t*k+s in perm. */
int qmoe_combine(qmoe_ctx *ctx, const float *y, const int32_t *perm, const float *w,
                 const float *shared_gate, int n, const void *x_residual, int x_dtype,
                 float *out, void *stream, qmoe_err *err);

/* The whole layer (stages 1-4) on device buffers; the drop-in for the call
 * at model.c:1712.  x [n,H] (x_dtype), out [n,H] f32.  flags: QMOE_RESIDUAL. */
int qmoe_layer_forward(qmoe_ctx *ctx, int layer, const void *x, int x_dtype, int n, float *out,
                       int flags, void *stream, qmoe_err *err);

/* qmoe_layer_forward that allocates nothing.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  No context: cfg gives the shape (n_layers unused; n <=
 * max_tokens) and dev_weights the layer as DEVICE pointers in the layout
 * of qmoe_layer_weights (qmoe_layer_device_weights of a resident layer, or
 * the caller's own copies); x, out, flags and stream as qmoe_layer_forward,
 * with the same kernels and the same results.  The scratch is one static
 * block of QMOE_NOALLOC_SCRATCH_BYTES per GPU, held from the first call on
 * that GPU until the process ends; a call whose scratch for n tokens does
 * not fit is refused with an error (hidden 2048, 512 experts, top-10,
 * moe_inter 512: n <= 459).  Every call on one GPU uses that one block:
 * calls that overlap on a GPU (two streams or two threads) race.  The
 * stages all run on `stream`; the call makes no hipMalloc, hipFree or
 * other allocating call. */
#define QMOE_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)
int qmoe_layer_forward_noalloc(const qmoe_config *cfg, const qmoe_layer_weights *dev_weights,
                               const void *x, int x_dtype, int n, float *out, int flags,
                               void *stream, qmoe_err *err);

/* Copies the routing of the last qmoe_layer_forward call on this context
 * (n must be that call's token count) into caller device buffers, any of
 * which may be NULL: idx [n,k], w [n,k], shared_gate [n], offsets [E+1],
 * perm [n*k], segments [1+3E].  An inspection hook for tests and tools; the
 * reference keeps these in moe_forward's scratch (model.c:1288-1300). */
int qmoe_last_routing(qmoe_ctx *ctx, int n, int32_t *idx_out, float *w_out, float *shared_gate_out,
                      int32_t *offsets_out, int32_t *perm_out, int32_t *segments_out, void *stream,
                      qmoe_err *err);

/* Host-memory shim with moe_forward's data contract (model.c:1281-1282):
 * x [n,H] f32 host in, out [n,H] f32 host out, synchronous.  The caller's
 * scratch is not needed (the context owns device scratch). */
int qmoe_moe_forward_host(qmoe_ctx *ctx, int layer, const float *x, int n, float *out,
                          qmoe_err *err);

/* ------------------------------------------------------ hyper connection
 * The MoE layer's input producer and output consumer in the reference
 * model: the MLP hyper connection of each decoder layer.  The residual
 * stream is a hyper state of hc copies of the hidden vector, [n, hc*H] f32
 * (c/src/model.c:1590-1606).  Before the MoE, gated_residual
 * (model.c:728-796, called at model.c:1710-1711) mixes it down to the MoE
 * input:
 *   normed = per-copy RMSNorm (eps 1e-6) * hc_norm            [n, hc*H]
 *   w      = silu(input_mix_weight_down(normed) / hc)         [n, R]
 *   mixed  = mean over copies of sigmoid(input_mix_weight_up(w)) * normed   [n, H]
 *   inject = 2 * sigmoid(block_inject_weight(normed) / hc)    [n, hc]
 * and after it every copy takes the MoE output (model.c:1724-1731):
 *   hyper[t, j, :] += inject[t, j] * out[t, :].
 * R = hc_lowrank.  The two mix weights are MLX q4 (group 64) as in the
 * checkpoint; block_inject_weight is dense bf16 (gemm_bf16, model.c:789). */
typedef struct {
    const float *hc_norm;     /* [hc*H]      f32   mlp_hyper_connection.hc_norm.weight */
    const uint32_t *down_q;   /* [R, hc*H/8] u32   .input_mix_weight_down.weight */
    const uint16_t *down_s;   /* [R, hc*H/g] bf16  .scales */
    const uint16_t *down_b;   /* [R, hc*H/g] bf16  .biases */
    const uint32_t *up_q;     /* [hc*H, R/8] u32   .input_mix_weight_up.weight */
    const uint16_t *up_s;     /* [hc*H, R/g] bf16  .scales */
    const uint16_t *up_b;     /* [hc*H, R/g] bf16  .biases */
    const uint16_t *inject_w; /* [hc, hc*H]  bf16  .block_inject_weight.weight */
} qmoe_hc_weights;

/* Gives the context hyper-connection slots for every layer and the mix
 * scratch (sized by max_tokens): hc_count (<= 8) copies, low rank
 * hc_lowrank (a multiple of 64, <= 2048), hidden <= 2048.  The
 * text_config's hc_count / hc_lowrank (model.c:86-87).  Calling it again
 * with the same values is a no-op. */
int qmoe_hc_enable(qmoe_ctx *ctx, int hc_count, int hc_lowrank, qmoe_err *err);
/* one layer's hyper-connection tensors from host memory (mw_load and
 * mw_load_f32 of model.c:1945-1952) */
int qmoe_hc_upload_layer(qmoe_ctx *ctx, int layer, const qmoe_hc_weights *host, qmoe_err *err);
/* the same from a checkpoint: model.layers.<model_layer>.mlp_hyper_connection.*
 * (model.c:1945-1952, 1959-1964).  hc_norm is BF16 in the file and widened
 * to f32 (mw_load_f32, model.c:275-294); the mix weights must be q4 (a
 * missing .biases reads as zero), block_inject_weight dense BF16. */
int qmoe_hc_upload_layer_st(qmoe_ctx *ctx, int layer, const qmoe_st *ix, int model_layer,
                            qmoe_err *err);
/* seeded synthetic hyper-connection weights: hc_norm ones, codes U{0..15},
 * scales N(0,0.02), biases N(0,0.01), block_inject_weight N(0,0.02).  No
 * counterpart in the reference (bench/test helper). */
int qmoe_hc_synth_layer(qmoe_ctx *ctx, int layer, uint64_t seed, qmoe_err *err);
int qmoe_hc_device_weights(qmoe_ctx *ctx, int layer, qmoe_hc_weights *out, qmoe_err *err);

/* gated_residual with inject (model.c:728-796): hyper [n, hc*H] f32 ->
 * mixed_out [n, H] f32, inject_out [n, hc] f32 (may be NULL), normed_out
 * [n, hc*H] f32 (may be NULL). */
int qmoe_hc_mix(qmoe_ctx *ctx, int layer, const float *hyper, int n, float *mixed_out,
                float *inject_out, float *normed_out, void *stream, qmoe_err *err);
/* the inject update alone (model.c:1724-1731), hyper updated in place */
int qmoe_hc_inject(qmoe_ctx *ctx, const float *inject, const float *moe_out, int n, float *hyper,
                   void *stream, qmoe_err *err);
/* model.c:1710-1731 on device buffers: gated_residual, the MoE layer on
 * the mixed input, and the inject update fused into the layer's combine;
 * hyper [n, hc*H] f32 is updated in place.  moe_out [n, H] f32 receives the
 * MoE output when non-NULL. */
int qmoe_hc_layer_forward(qmoe_ctx *ctx, int layer, float *hyper, int n, float *moe_out,
                          void *stream, qmoe_err *err);

/* ------------------------------------------------------ expert streaming
 * For family sizes whose experts do not fit in HBM: the routed experts of
 * every layer live in pinned host memory and each layer owns a pool of
 * HBM expert slots; qmoe_layer_forward then routes on the GPU, brings the
 * layer's missing experts into slots (evicting by the reference's policy,
 * c/src/cache.c:99-259), remaps the segment table from expert ids to slots
 * and runs the same expert kernels on the slot pool.  Replaces the SSD
 * stream + expert cache of experts_load (model.c:536-674) and the
 * route-transition prefetch of the MLX runtime (streaming.py:400-435).  The
 * router, shared expert and gates stay resident. */

/* cache policies, as CACHE_POLICY_* (c/src/cache.h:8-10) */
enum { QMOE_CACHE_LRU = 0, QMOE_CACHE_LFU = 1, QMOE_CACHE_ADAPTIVE = 2 };

/* Switches the context to streamed experts: slots_per_layer HBM expert
 * slots per layer (>= the distinct experts one call can route, i.e.
 * min(n_experts, max_tokens * top_k), and <= n_experts), the eviction
 * policy, and up to `prefetch` experts requested ahead per layer call (0 =
 * none).  Must precede every upload or synthesis.  In this mode the expert
 * stage functions (qmoe_expert_*) are refused: the layer call runs them.
 * prefetch = -1 selects the device-resolved mode: the same residency
 * decisions (hits, misses, victims) made by one GPU workgroup inside the
 * layer call, which then copies the misses and runs the experts with no
 * host round trip and no host synchronisation, so the call can be
 * captured in a graph; it requests nothing ahead.  Calls of one context
 * must then share one stream (the state of a layer is updated in stream
 * order). */
int qmoe_stream_enable(qmoe_ctx *ctx, int slots_per_layer, int policy, int prefetch,
                       qmoe_err *err);

typedef struct {
    uint64_t hits, misses, evictions, rejected; /* cache_snapshot's counters (cache.h:45-48) */
    uint64_t bytes_in;        /* host -> HBM expert bytes, demand and prefetch */
    uint64_t prefetched;      /* experts brought in ahead of use */
    uint64_t prefetch_hits;   /* ... of which a later call used */
} qmoe_stream_stats;

int qmoe_stream_get_stats(qmoe_ctx *ctx, qmoe_stream_stats *out, qmoe_err *err);

/* The slot cache itself, host only (the policy's test surface; mirrors
 * cache_init / cache_peek / cache_get / cache_put / cache_pin / cache_unpin /
 * cache_mark_hot / cache_snapshot of c/src/cache.h:36-58 for `parts`
 * partitions of `slots` entries of entry_bytes each over items 0..items-1).
 * qmoe_xcache_get and _put return the slot or -1; counts = hits, misses,
 * evictions, rejected. */
typedef struct qmoe_xcache qmoe_xcache;
int qmoe_xcache_create(qmoe_xcache **out, int parts, int items, int slots, int policy,
                       uint64_t entry_bytes, qmoe_err *err);
void qmoe_xcache_destroy(qmoe_xcache *c);
int qmoe_xcache_peek(qmoe_xcache *c, int part, int item);
int qmoe_xcache_get(qmoe_xcache *c, int part, int item);
int qmoe_xcache_put(qmoe_xcache *c, int part, int item, int pin, int hot, int *evicted);
int qmoe_xcache_pin(qmoe_xcache *c, int part, int item, int pinned);
int qmoe_xcache_mark_hot(qmoe_xcache *c, int part, int item, int hot);
void qmoe_xcache_clear(qmoe_xcache *c, int part);
void qmoe_xcache_counts(const qmoe_xcache *c, uint64_t out[4]);

/* Size in bytes of the context's device scratch and of one resident layer. */
size_t qmoe_scratch_bytes(const qmoe_ctx *ctx);
size_t qmoe_layer_bytes(const qmoe_ctx *ctx);

/* Library version string. */
const char *qmoe_version(void);

/* ------------------------------------------------------ gated DeltaNet
 * The linear-attention mixer of the decoder's DeltaNet layers, the step
 * before each MoE layer in the reference model: deltanet_forward
 * (c/src/model.c:1146-1278), per layer and per call of n tokens:
 *   mixed = in_proj_qkv(x), z = in_proj_z(x)        (q4, model.c:1168-1170)
 *   a = x.Wa^T, b = x.Wb^T                          (bf16, model.c:1172-1175)
 *   causal depthwise conv over [conv_state; mixed], the state keeps the last
 *   conv_kernel-1 rows, then silu                    (model.c:1177-1187)
 *   q, k, v = split; q = l2norm(q) / sqrt(dk), k = l2norm(k)  (model.c:1202-1222)
 *   per value head h (key head h / (hv/hk)), per token:
 *     g = exp(-exp(A_log[h]) * log1p(exp(a[h] + dt_bias[h]))), beta = sigmoid(b[h])
 *     S <- g S;  S += (beta (v - S k)) k^T;  o = S q  (S [dv, dk], model.c:1225-1248)
 *   o_h = rmsnorm(o_h) * norm_w * sigmoid(z_h)       (model.c:1263-1274)
 *   out = out_proj(o)                                (q4, model.c:1276)
 * The conv and recurrent states live in HBM with the layer and carry over
 * from call to call (tokens in order), as the reference's per-layer
 * conv_state / rec_state.  Sums run in parallel orders: results agree with
 * the reference to rounding, not bit for bit.  Weights, like the MoE
 * layer's, use the checkpoint layout (names model.c:1866-1883):
 * linear_attn.{in_proj_qkv,in_proj_z,out_proj} q4 (u32 codes, bf16
 * scales/biases per 64 columns), in_proj_{a,b} and conv1d bf16, norm,
 * A_log and dt_bias widened to f32 (the reference's mw_load_f32). */
typedef struct qmoe_dn_ctx qmoe_dn_ctx;

typedef struct {
    int hidden;      /* d: multiple of 64, <= 8192 */
    int n_k_heads;   /* hk: linear_num_key_heads */
    int n_v_heads;   /* hv: linear_num_value_heads, a multiple of hk */
    int k_head_dim;  /* dk: 32, 64, 128 or 256 */
    int v_head_dim;  /* dv: a power of two from 32 to 2048; hv*dv a multiple of 64, <= 8192 */
    int conv_kernel; /* linear_conv_kernel_dim, 1..16 */
    int group_size;  /* must be 64 */
    int n_layers;
    int max_tokens;
} qmoe_dn_config;

/* conv_dim = 2*hk*dk + hv*dv, value_dim = hv*dv */
typedef struct {
    const uint32_t *qkv_q;   /* [conv_dim, d/8]   in_proj_qkv.weight */
    const uint16_t *qkv_s;   /* [conv_dim, d/64]  .scales */
    const uint16_t *qkv_b;   /* [conv_dim, d/64]  .biases */
    const uint32_t *z_q;     /* [value_dim, d/8]  in_proj_z.* */
    const uint16_t *z_s, *z_b;
    const uint16_t *a_w;     /* [hv, d] bf16      in_proj_a.weight */
    const uint16_t *b_w;     /* [hv, d] bf16      in_proj_b.weight */
    const uint32_t *out_q;   /* [d, value_dim/8]  out_proj.* */
    const uint16_t *out_s, *out_b;
    const uint16_t *conv_w;  /* [conv_dim, conv_kernel] bf16  conv1d.weight */
    const float *norm_w;     /* [dv]  norm.weight */
    const float *a_log;      /* [hv]  A_log */
    const float *dt_bias;    /* [hv]  dt_bias */
} qmoe_dn_weights;

int qmoe_dn_create(qmoe_dn_ctx **ctx, const qmoe_dn_config *cfg, qmoe_err *err);
void qmoe_dn_destroy(qmoe_dn_ctx *ctx);
/* copies one layer from HOST memory and clears its states */
int qmoe_dn_upload_layer(qmoe_dn_ctx *ctx, int layer, const qmoe_dn_weights *host, qmoe_err *err);
/* zeroes the conv and recurrent states of one layer (-1: every layer), as
 * the reference's model reset (model.c:402-403), on `stream` */
int qmoe_dn_reset_state(qmoe_dn_ctx *ctx, int layer, void *stream, qmoe_err *err);
/* x [n, d] f32 device -> out [n, d] f32 device, n <= max_tokens; updates
 * the layer's states.  Asynchronous on `stream`. */
int qmoe_dn_forward(qmoe_dn_ctx *ctx, int layer, const float *x, int n, float *out, void *stream,
                    qmoe_err *err);
/* qmoe_dn_forward followed by the gated residual's update of the mixer's
 * output into the hyper state, hyper[t, j, :] += inject[t, j] * out[t, :]
 * for j < hc (qmoe_gr_inject, model.c:1699-1707), done in the mixer's last
 * launch with the same arithmetic: one launch fewer per layer.  hyper [n,
 * hc, d] and inject [n, hc] f32 device, 1 <= hc <= 8; out may be NULL (not
 * written).  No counterpart in the reference: its layer loop calls the
 * mixer and the update separately (model.c:1683-1688, 1699-1707). */
int qmoe_dn_forward_inject(qmoe_dn_ctx *ctx, int layer, const float *x, int n, float *out, float *hyper,
                           const float *inject, int hc, void *stream, qmoe_err *err);
/* device addresses of a layer's states: conv [conv_kernel-1, conv_dim] and
 * recurrent [hv, dv, dk] f32 (for inspection and for seeding a state) */
int qmoe_dn_state(qmoe_dn_ctx *ctx, int layer, float **conv_state, float **rec_state,
                  qmoe_err *err);

/* ------------------------------------------------------ full attention
 * The full-attention mixer of the decoder's attention layers with its QSA
 * indexer: attention_forward (c/src/model.c:798-1144), per layer and per
 * call of n tokens at positions offset..offset+n-1:
 *   qk = x.Wi^T (index_qk_proj, bf16): indexer query heads and a raw key,
 *   appended to the indexer key cache                    (model.c:807-843)
 *   q|gate (interleaved per head), k, v = q4 projections (model.c:847-862)
 *   q, k: per-head rmsnorm (q_norm, k_norm), then RoPE of the first
 *   rot = head_dim * rotary_factor dims at the token's position; k and v
 *   appended to the caches                                (model.c:871-937)
 *   scores q.k / sqrt(head_dim), head hh reading kv head hh % kv_heads,
 *   keys at cache rows > offset + t masked (causal)      (model.c:951-967)
 *   past idx_budget cached keys: the QSA block mask -- mean-pooled indexer
 *   keys per block of idx_compress rows, rmsnorm + RoPE at the block start,
 *   block score sum over indexer heads of sum relu(q_i p_i) / sqrt(idx_hd),
 *   blocks ending past the token invisible, the top idx_budget/idx_compress
 *   blocks and the token's own block tail kept            (model.c:969-1104)
 *   softmax, weighted sum of v, * sigmoid(gate), o_proj   (model.c:1107-1143)
 * The caches live in HBM with the layer, kv_cap rows; a call that would pass
 * kv_cap is refused, or with slide = 1 drops the oldest rows of all three
 * caches together (the reference drops the oldest rows of its v and
 * indexer caches there but not of its k cache, model.c:815-821, 862-867,
 * 921, which misaligns k and v; that is not reproduced).  Block selection ties go to the lower
 * block (the reference's quickselect leaves their order open).  The
 * indexer path runs in the reference's sequential orders (index_qk_proj in
 * the router's fixed R64 order), so block scores and kept blocks equal the
 * C restatement's bit for bit; attention sums run in parallel orders and
 * agree with the reference to rounding.
 * Weights use the checkpoint layout (names model.c:1833-1850). */
typedef struct qmoe_attn_ctx qmoe_attn_ctx;

typedef struct {
    int hidden;        /* d: multiple of 64, <= 8192 */
    int n_heads;       /* h: num_attention_heads */
    int n_kv_heads;    /* kvh: num_key_value_heads, divides h */
    int head_dim;      /* hd: multiple of 64, <= 256; h*hd <= 8192 */
    int idx_heads;     /* indexer_n_heads */
    int idx_head_dim;  /* indexer_head_dim: multiple of 4, <= 256, >= rot */
    int idx_budget;    /* indexer_budget */
    int idx_compress;  /* indexer_compress_ratio */
    int kv_cap;        /* cache rows, <= 8192 */
    int group_size;    /* must be 64 */
    float rotary_factor; /* partial_rotary_factor: rot = (int)(hd * factor), even */
    float rope_theta;
    int n_layers;
    int max_tokens;
    int max_position;  /* positions offset + t stay below max(max_position, kv_cap); 0: kv_cap.
                        * The RoPE table (cos, sin per position) is computed on the host at
                        * create with the reference's formula; at most QMOE_ATTN_MAX_POSITION */
    int slide;         /* 0: a call past kv_cap is refused.  1: sliding window -- a call that
                        * would pass kv_cap first drops the oldest rows of the k, v and
                        * indexer-key caches together (and the pooled keys of the blocks they
                        * made), a multiple of idx_compress of them so blocks stay aligned;
                        * positions are absolute, calls continue at position window start +
                        * cached rows, and kv_cap must be a multiple of idx_compress.  Unlike
                        * the reference's drop (model.c:815-821, 862-867), k stays aligned
                        * with v. */
} qmoe_attn_config;

#define QMOE_ATTN_MAX_POSITION (1 << 20)

typedef struct {
    const uint32_t *q_q;  /* [2*h*hd, d/8]   q_proj.weight (q | gate per head) */
    const uint16_t *q_s, *q_b;
    const uint32_t *k_q;  /* [kvh*hd, d/8]   k_proj.* */
    const uint16_t *k_s, *k_b;
    const uint32_t *v_q;  /* [kvh*hd, d/8]   v_proj.* */
    const uint16_t *v_s, *v_b;
    const uint32_t *o_q;  /* [d, h*hd/8]     o_proj.* */
    const uint16_t *o_s, *o_b;
    const uint16_t *idx_w;     /* [(idx_heads+1)*idx_hd, d] bf16  indexer.index_qk_proj.weight */
    const float *q_norm, *k_norm;          /* [hd] */
    const float *idx_q_norm, *idx_k_norm;  /* [idx_hd] */
} qmoe_attn_weights;

int qmoe_attn_create(qmoe_attn_ctx **ctx, const qmoe_attn_config *cfg, qmoe_err *err);
void qmoe_attn_destroy(qmoe_attn_ctx *ctx);
/* copies one layer from HOST memory and empties its caches */
int qmoe_attn_upload_layer(qmoe_attn_ctx *ctx, int layer, const qmoe_attn_weights *host,
                           qmoe_err *err);
/* empties the caches of one layer (-1: every layer) */
int qmoe_attn_reset(qmoe_attn_ctx *ctx, int layer, qmoe_err *err);
/* x [n, d] f32 device at positions offset.. -> out [n, d] f32 device;
 * appends n rows to the layer's caches.  Asynchronous on `stream`; the
 * cache length is host state, so calls on one layer run in call order. */
int qmoe_attn_forward(qmoe_attn_ctx *ctx, int layer, const float *x, int n, int offset, float *out,
                      void *stream, qmoe_err *err);
/* qmoe_attn_forward with the gated residual's update fused into o_proj's
 * launch, as qmoe_dn_forward_inject (hyper [n, hc, d], inject [n, hc],
 * 1 <= hc <= 8, out may be NULL).  No counterpart in the reference
 * (model.c:1683-1688 calls the mixer, 1699-1707 the update). */
int qmoe_attn_forward_inject(qmoe_attn_ctx *ctx, int layer, const float *x, int n, int offset, float *out,
                             float *hyper, const float *inject, int hc, void *stream, qmoe_err *err);
/* device addresses of a layer's caches (k and v [len, kvh*hd], indexer
 * keys [len, idx_hd]; with slide, the window's first row) and their current
 * length */
int qmoe_attn_cache(qmoe_attn_ctx *ctx, int layer, float **k_cache, float **v_cache, float **idx_keys,
                    int *len, qmoe_err *err);
/* device addresses of the QSA indexer's state, for inspection (the values
 * the reference computes inside attention_forward, model.c:955-1075): the
 * layer's pooled, normed and rotated block keys [kv_cap/idx_compress,
 * idx_hd] (block b valid once the cache holds (b+1)*idx_compress rows),
 * and, for the context's last forward call that ran the block mask, the
 * kept-block bitmap [n, keep_words] u32 (bit b%32 of word b/32; keep_words
 * = ceil(blocks of that call / 32)) and the
 * block scores as order keys [n, score_ld] u32 (bits of a float s >= 0:
 * bits | 0x80000000; s < 0: ~bits).  Read them after the call completes
 * on its stream and before the context's next call. */
int qmoe_attn_index_state(qmoe_attn_ctx *ctx, int layer, float **pooled, uint32_t **keep, int *keep_words,
                          uint32_t **score_keys, int *score_ld, qmoe_err *err);

/* ------------------------------------------------- gated residual slots
 * gated_residual (c/src/model.c:728-796) on its own, for the two hyper
 * connections that are not the MoE layer's: each decoder layer's
 * attention-block connection (attn_hyper_connection, model.c:1671-1672,
 * with inject, applied after the mixer as hyper += inject (x) out,
 * model.c:1699-1707) and the final mixer before the LM head
 * (hyper_connection_mixer, model.c:1743-1745, no inject).  The same
 * arithmetic and kernels as qmoe_hc_mix: normed = per-copy RMSNorm * hc_norm,
 * w = silu(down(normed)/hc), mixed = mean_h sigmoid(up(w)) * normed,
 * inject = 2 sigmoid(inject_w(normed)/hc).  A context holds n_slots weight
 * sets of one shape (a slot per layer plus one for the mixer, say), each
 * uploaded with or without its inject matrix. */
typedef struct qmoe_gr_ctx qmoe_gr_ctx;

typedef struct {
    int hidden;     /* d: multiple of 64, <= 2048 */
    int hc_count;   /* hc: 1..8 */
    int hc_lowrank; /* R: multiple of 64, 64..2048 */
    int n_slots;
    int max_tokens;
} qmoe_gr_config;

int qmoe_gr_create(qmoe_gr_ctx **ctx, const qmoe_gr_config *cfg, qmoe_err *err);
void qmoe_gr_destroy(qmoe_gr_ctx *ctx);
/* one slot's weights from HOST memory, the layout of qmoe_hc_weights
 * (model.layers.<i>.attn_hyper_connection.* or
 * model.hyper_connection_mixer.*, names model.c:1817-1824, 1925-1958);
 * inject_w NULL makes a slot without inject (the final mixer) */
int qmoe_gr_upload_slot(qmoe_gr_ctx *ctx, int slot, const qmoe_hc_weights *host, qmoe_err *err);
/* hyper [n, hc*d] f32 device -> mixed_out [n, d] f32 device and, for a
 * slot with inject, inject_out [n, hc] (may be NULL: not computed).  A slot
 * without inject refuses a non-NULL inject_out.  Asynchronous on `stream`;
 * calls on one context share its scratch, so they run on one stream. */
int qmoe_gr_mix(qmoe_gr_ctx *ctx, int slot, const float *hyper, int n, float *mixed_out,
                float *inject_out, void *stream, qmoe_err *err);
/* hyper[t, j, :] += inject[t, j] * out[t, :] (model.c:1699-1707) */
int qmoe_gr_inject(qmoe_gr_ctx *ctx, const float *inject, const float *out, int n, float *hyper,
                   void *stream, qmoe_err *err);

#ifdef __cplusplus
}
#endif
#endif
