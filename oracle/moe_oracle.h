/*
 * moe_oracle.h -- CPU restatement of the reference C port's MoE layer.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the HIP
 * path and the timed CPU baseline.  Only tests/, __graft_entry__.smoke() and
 * the cpu_baseline leg of bench.py may load it.  The product library
 * (libqmoe.so) never links, calls or falls back to it.
 *
 * What it restates (reference paths relative to the reference checkout):
 *   c/src/model.c:1281-1405   moe_forward (router, top-k, renorm, dispatch,
 *                             per-expert SwiGLU, combine, shared expert)
 *   c/src/kernel.c:10-20      kernel_rmsnorm
 *   c/src/kernel.c:38-59      kernel_silu / kernel_sigmoid / kernel_mul
 *   c/src/kernel.c:112-150    kth_largest + kernel_topk_indices (quickselect)
 *   c/src/kernel.c:152-179    kernel_dequant_q4(_row)
 *   c/src/kernel.c:181-186    gemm_fp32 (naive loops replace cblas_sgemm)
 *   c/src/kernel.c:190-228    gemm_bf16 (naive loops replace BNNSMatMul)
 *   c/src/kernel.c:230-309    gemm_q4 (per-group s*sum(xq) + b*sum(x) identity)
 *   c/src/util.h:56-71        bf16 <-> f32 (shift widen, RNE narrow)
 *   c/src/model.c:424-472,539-674  expert tensor layout [E,I,H/8] / [E,H,I/8]
 *   c/src/model.c:728-796,1703-1731  the MLP hyper connection around the layer
 *   c/src/kernel.c:22-36,45-55  kernel_rmsnorm_grouped, sigmoid, scale
 *
 * Deliberate departures (each is also a contract the GPU path keeps):
 *   1. Router dot products use the fixed "R64" order (orc_dot_r64): 64
 *      strided partial fma-chains over 8-element chunks, combined by a
 *      pairwise tree over the chunks' lanes in natural order.  The reference leaves the order to BNNS;
 *      fixing it makes expert selection bit-exact across CPU and GPU.
 *   2. Top-k order is canonical: value descending, ties to the lower expert
 *      id (-0.0 counts as +0.0).  The reference quickselect returns the same
 *      set whenever the k-th and (k+1)-th logits differ.
 *   3. Dispatch order: experts ascending, tokens ascending within an expert
 *      (the MLX order, src/colibri_runtime/model.py:433-441).  The C port's
 *      first-seen expert order only changes the fp32 summation order of the
 *      combine.
 *   4. Optional per-expert router bias (fp32, added after the dot product,
 *      before top-k and softmax).  NULL reproduces the reference.
 *   5. Optional pre-router RMSNorm (kernel.c:10-20) with its sum of squares in
 *      R64 order, and an optional residual add (out = x + moe(x)).
 *
 * Parity pins for every function are listed in tests/test_oracle.py.
 */
#ifndef MOE_ORACLE_H
#define MOE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- bf16 (c/src/util.h:56-71) ---- */
float orc_bf16_to_f32(uint16_t h);
uint16_t orc_f32_to_bf16(float f);

/* ---- elementwise (c/src/kernel.c:10-20, 38-59) ---- */
/* sequential sum of squares, exactly as kernel.c:12-14 */
void orc_rmsnorm_seq(const float *x, const float *w, size_t n, float eps, float *y);
/* R64-ordered sum of squares (departure 5); same formula otherwise */
void orc_rmsnorm_r64(const float *x, const float *w, size_t n, float eps, float *y);
float orc_silu(float v);
float orc_sigmoid(float v);

/* ---- fixed-order dot products (departure 1) ---- */
float orc_dot_r64_bf16w(const float *x, const uint16_t *w, int K);
float orc_sumsq_r64(const float *x, int K);

/* ---- top-k ---- */
/* faithful restatement of kth_largest / kernel_topk_indices (quickselect,
 * middle pivot, Lomuto with strict '>'), order unspecified */
void orc_topk_quickselect(const float *x, int n, int k, int *out);
/* canonical order: value desc, id asc (departure 2) */
void orc_topk_canonical(const float *x, int n, int k, int *out);

/* ---- q4 (c/src/kernel.c:152-179, 230-309) ---- */
/* scales/biases are given as bf16 (as stored on disk), widened exactly */
void orc_dequant_q4(const uint32_t *q, const uint16_t *scales, const uint16_t *biases,
                    size_t rows, size_t cols, size_t group_size, float *out);
void orc_dequant_q4_f32sb(const uint32_t *q, const float *scales, const float *biases,
                          size_t rows, size_t cols, size_t group_size, float *out);
void orc_gemm_fp32(int M, int N, int K, const float *A, const float *W, float *C);
void orc_gemm_bf16(int M, int N, int K, const float *A, const uint16_t *W, float *C);
void orc_gemm_q4_f32sb(int M, int N, int K, const float *A, const uint32_t *W,
                       const float *scales, const float *biases, int group_size, float *C);
void orc_gemm_q4(int M, int N, int K, const float *A, const uint32_t *W,
                 const uint16_t *scales, const uint16_t *biases, int group_size, float *C);

/* ---- dispatch (departure 3) ---- */
/* idx [n*k] -> offsets [E+1], perm [n*k] (flat t*k+s), pos [n*k] (inverse),
 * active [E] (experts with tokens, ascending); returns the active count */
int orc_dispatch(const int *idx, int n, int k, int E, int *offsets, int *perm, int *pos,
                 int *active);

/* ---- the layer ---- */
typedef struct {
    int hidden;       /* H */
    int n_experts;    /* E */
    int top_k;        /* k */
    int moe_inter;    /* I (routed and shared; the C port requires equality) */
    int group_size;   /* g */
    float rms_eps;
    const uint16_t *router_w;   /* [E,H] bf16   mlp.gate.weight */
    const float *router_bias;   /* [E] f32 or NULL */
    const uint32_t *gate_q;     /* [E,I,H/8]    switch_mlp.gate_proj.weight */
    const uint16_t *gate_s, *gate_b;   /* [E,I,H/g] bf16 */
    const uint32_t *up_q;
    const uint16_t *up_s, *up_b;
    const uint32_t *down_q;     /* [E,H,I/8]    switch_mlp.down_proj.weight */
    const uint16_t *down_s, *down_b;   /* [E,H,I/g] */
    const uint32_t *sh_gate_q;  /* [I,H/8]      shared_expert.gate_proj */
    const uint16_t *sh_gate_s, *sh_gate_b;
    const uint32_t *sh_up_q;
    const uint16_t *sh_up_s, *sh_up_b;
    const uint32_t *sh_down_q;  /* [H,I/8]      shared_expert.down_proj */
    const uint16_t *sh_down_s, *sh_down_b;
    const uint16_t *sh_gate_w;  /* [H] bf16     shared_expert_gate.weight */
    const float *norm_w;        /* [H] f32 or NULL: pre-router RMSNorm */
} orc_layer;

enum {
    ORC_ROUTED_FAITHFUL = 0, /* dequant to fp32 (fma(q,s,b)) + fp32 dot, as model.c:1368-1375 */
    ORC_ROUTED_Q4 = 1        /* gemm_q4 identity for routed experts too */
};

typedef struct {
    int x_is_bf16;   /* x element type: 0 = f32, 1 = bf16 */
    int residual;    /* out = x + moe(x) */
    int routed_mode; /* ORC_ROUTED_* */
    int n_threads;   /* OpenMP threads, <= 0: runtime default */
} orc_opts;

/* Full layer for n tokens.  Any of the *_out pointers may be NULL.
 *   logits_out [n,E] biased router logits, gate_logit_out [n],
 *   idx_out [n,k] canonical order, w_out [n,k], shared_gate_out [n] (sigmoid),
 *   xn_out [n,H] the router input (after RMSNorm when norm_w is set).
 * token_sel: if non-NULL, only tokens token_sel[0..n_sel) produce an `out`
 * row (out is then [n_sel,H]); routing outputs still cover all n tokens.
 * Returns 0, or -1 with a message in err (512 bytes) on a shape error. */
int orc_moe_forward(const orc_layer *L, const void *x, int n, float *out,
                    const orc_opts *opt, const int *token_sel, int n_sel,
                    float *logits_out, float *gate_logit_out, int *idx_out, float *w_out,
                    float *shared_gate_out, float *xn_out, char *err);

/* Router only (logits + top-k + renorm + shared gate), all n tokens. */
int orc_route(const orc_layer *L, const void *x, int x_is_bf16, int n, float *logits_out,
              float *gate_logit_out, int *idx_out, float *w_out, float *shared_gate_out,
              float *xn_out, int n_threads, char *err);

/* ---- the hyper connection around the MoE layer (c/src/model.c:728-796,
 * 1703-1731): the MLP's gated_residual produces the MoE input from the
 * hyper state, and the MoE output is injected back into every copy ---- */
typedef struct {
    int hc, d, lowrank, group_size;
    const float *hc_norm;          /* [hc*d] */
    const uint32_t *down_q;        /* [lowrank, hc*d/8] q4 (input_mix_weight_down) */
    const uint16_t *down_s, *down_b; /* [lowrank, hc*d/g] bf16 */
    const uint32_t *up_q;          /* [hc*d, lowrank/8] q4 (input_mix_weight_up) */
    const uint16_t *up_s, *up_b;   /* [hc*d, lowrank/g] bf16 */
    const uint16_t *inject_w;      /* [hc, hc*d] bf16 (block_inject_weight) */
} orc_hc;

/* gated_residual with inject (model.c:728-796): hyper [n, hc*d] ->
 * mixed [n, d] (the MoE input), inject [n, hc]; normed [n, hc*d] may be
 * NULL.  Grouped RMSNorm as kernel.c:22-36 (eps 1e-6), linear layers as
 * linear_forward (gemm_q4) and gemm_bf16 (naive order). */
int orc_hc_mix(const orc_hc *H, const float *hyper, int n, float *mixed, float *inject,
               float *normed_out);
/* model.c:1724-1731: hyper[t, hh, j] += inject[t, hh] * out[t, j] */
void orc_hc_inject(int hc, int d, int n, const float *inject, const float *out, float *hyper);

/* ---- seeded synthetic tensors (counter-based; the GPU generator in the
 * product library produces the same values) ---- */
uint64_t orc_mix64(uint64_t z);
uint64_t orc_tensor_key(uint64_t seed, uint32_t layer, uint32_t tag);
void orc_gen_normal_bf16(uint16_t *out, size_t count, uint64_t key, uint64_t start, float stddev);
void orc_gen_normal_f32(float *out, size_t count, uint64_t key, uint64_t start, float stddev);
void orc_gen_codes(uint32_t *out, size_t count, uint64_t key, uint64_t start);
/* Zipf(s) router bias: bias[e] = ln p_{pi(e)}, p_r = r^-s / sum, pi = seeded
 * Fisher-Yates permutation of 0..E-1, scaled by `scale` */
void orc_zipf_bias(float *bias, int E, double s, double scale, uint64_t seed);

/* ---- CPU baseline timing ---- */
/* times `iters` forward passes after `warmup` ones; returns median seconds */
double orc_time_forward(const orc_layer *L, const void *x, int n, float *out,
                        const orc_opts *opt, int warmup, int iters);

/* ---- CPU baseline, weight mode (i): warm fp32 experts ----
 * The steady state of the C port's expert cache: each listed routed expert
 * dequantised once to fp32 in the cache's gate | up | down layout
 * (model.c:603-662, dequant_raw + kernel_dequant_q4), then every layer call
 * runs gemm_fp32 on them (model.c:1368-1375, kernel.c:181-186).  The fp32
 * products here are blocked like a BLAS sgemm: each weight row is read once
 * per call and dotted with every token routed to its expert, 16 independent
 * partial sums per dot (the summation order is a BLAS's, not the oracle's
 * single fma chain).  The shared expert stays q4 (linear_forward ->
 * gemm_q4, model.c:193-202).  Timing only; the result is checked against
 * orc_moe_forward within fp32 tolerance. */
typedef struct orc_warm orc_warm;
orc_warm *orc_warm_create(const orc_layer *L, const int *experts, int count, int n_threads);
void orc_warm_destroy(orc_warm *w);
size_t orc_warm_bytes(const orc_warm *w);
/* -1 with a message when a routed expert is not in the warm set */
int orc_moe_forward_warm(const orc_layer *L, const orc_warm *W, const void *x, int n, float *out,
                         const orc_opts *opt, char *err);
/* median seconds of `iters` calls after `warmup`; < 0 on error */
double orc_time_forward_warm(const orc_layer *L, const orc_warm *W, const void *x, int n,
                             float *out, const orc_opts *opt, int warmup, int iters);

/* ---- gated DeltaNet mixer (dn_oracle.c; model.c:1146-1278) ---- */
typedef struct {
    int hidden;       /* d */
    int n_k_heads;    /* linear_num_key_heads */
    int n_v_heads;    /* linear_num_value_heads, a multiple of n_k_heads */
    int k_head_dim;   /* dk */
    int v_head_dim;   /* dv */
    int conv_kernel;  /* linear_conv_kernel_dim */
    int group_size;
    const uint32_t *qkv_q; const uint16_t *qkv_s, *qkv_b;  /* in_proj_qkv [2*hk*dk + hv*dv, d] q4 */
    const uint32_t *z_q; const uint16_t *z_s, *z_b;        /* in_proj_z [hv*dv, d] q4 */
    const uint16_t *a_w, *b_w;                              /* in_proj_a, in_proj_b [hv, d] bf16 */
    const uint32_t *out_q; const uint16_t *out_s, *out_b;  /* out_proj [d, hv*dv] q4 */
    const uint16_t *conv_w;                                 /* conv1d [conv_dim, conv_kernel] bf16 */
    const float *norm_w;                                    /* [dv] */
    const float *a_log, *dt_bias;                           /* [hv] */
} orc_dn;
/* the decay factor exp(-exp(a_log) * log1p(exp(a + dt_bias))) of model.c:1229 */
float orc_dn_decay(float a_log, float a, float dt_bias);
/* x [n, d] f32 -> out [n, d]; conv_state [conv_kernel-1, conv_dim] and
 * rec_state [hv, dv, dk] are read and updated in place; core_out (or NULL)
 * receives the recurrence output [n, hv*dv] before the gated norm */
int orc_dn_forward(const orc_dn *D, const float *x, int n, float *out, float *conv_state,
                   float *rec_state, float *core_out);

/* ---- full attention with the QSA indexer (attn_oracle.c; model.c:798-1144) ---- */
typedef struct {
    int hidden;         /* d */
    int n_heads;        /* h */
    int n_kv_heads;     /* kvh; head hh reads kv head hh % kvh */
    int head_dim;       /* hd */
    int idx_heads;      /* indexer_n_heads */
    int idx_head_dim;   /* indexer_head_dim */
    int idx_budget;     /* indexer_budget */
    int idx_compress;   /* indexer_compress_ratio */
    int kv_cap;         /* cache rows (QMODEL_KV_CAP) */
    int group_size;
    float rotary_factor, rope_theta;
    const uint32_t *q_q; const uint16_t *q_s, *q_b;   /* q_proj [2*h*hd, d] q4: q | gate per head */
    const uint32_t *k_q; const uint16_t *k_s, *k_b;   /* k_proj [kvh*hd, d] q4 */
    const uint32_t *v_q; const uint16_t *v_s, *v_b;   /* v_proj [kvh*hd, d] q4 */
    const uint32_t *o_q; const uint16_t *o_s, *o_b;   /* o_proj [d, h*hd] q4 */
    const uint16_t *idx_w;                              /* index_qk_proj [idx_heads*idx_hd + idx_hd, d] bf16 */
    const float *q_norm, *k_norm;                       /* [hd] */
    const float *idx_q_norm, *idx_k_norm;               /* [idx_hd] */
    int slide; /* 0: refuse calls past kv_cap; 1: sliding window (see orc_attn_forward) */
} orc_attn;
typedef struct {
    float *k_cache, *v_cache; /* [kv_cap, kvh*hd] */
    float *idx_keys;          /* [kv_cap, idx_hd] */
    int kv_len, idx_len;
    int base;                 /* sliding window: position of cache row 0 */
} orc_attn_state;
/* x [n, d] f32 at positions offset.. -> out [n, d]; appends to the caches;
 * -2 when the call would pass the cache capacity.  With slide, a call that
 * would pass it first drops the oldest rows of the k, v and indexer-key
 * caches together, a multiple of idx_compress of them (so blocks stay
 * aligned), and base advances by as many; every mask and block position
 * is then the absolute position base + row, and offset must equal base +
 * kv_len (-3 otherwise; -2 when the drop would exceed the cached rows) */
int orc_attn_forward(const orc_attn *A, orc_attn_state *S, const float *x, int n, int offset,
                     float *out);
/* optional copies of the indexer's intermediate values, written when the
 * call runs the block mask (n_blocks = cached keys / compress after the
 * call): the pooled keys [n_blocks, idx_hd], each token's normed and
 * rotated queries [n, idx_heads*idx_hd], block scores [n, n_blocks] and
 * kept-block flags [n, n_blocks] (1 = among the top budget/compress) */
typedef struct {
    float *pooled, *qs, *scores;
    unsigned char *keep;
} orc_attn_dbg;
int orc_attn_forward_dbg(const orc_attn *A, orc_attn_state *S, const float *x, int n, int offset,
                         float *out, const orc_attn_dbg *dbg);

#ifdef __cplusplus
}
#endif
#endif
