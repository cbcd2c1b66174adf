/*
 * styx_oracle.h -- CPU restatement of the reference MoE decode path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the HIP
 * product path (libstyx_hip.so).  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it, and only as the checker or as the
 * timed CPU baseline.  The product path never calls into it.
 *
 * Every function restates one piece of the reference (aDirtyScoundrel/styx,
 * "moe-stream") and cites the file:line it follows.  Quant blocks are read in
 * GGUF block layout (what the reference uploads byte-for-byte).  Evaluation
 * order follows the reference's CPU code; the library is compiled with
 * -ffp-contract=off so no multiply-add is fused behind the source's back.
 *
 * Pinning status of each function is recorded next to it ("pinned by ...").
 * Functions whose only check is a restatement would be marked
 * "parity unpinned"; none are at present.
 */
#ifndef STYX_ORACLE_H
#define STYX_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml type ids (crates/gguf-rs/src/lib.rs:242-332). */
enum {
    STYX_ORACLE_F32 = 0,
    STYX_ORACLE_F16 = 1,
    STYX_ORACLE_Q8_0 = 8,
    STYX_ORACLE_Q4_K = 12,
    STYX_ORACLE_Q5_K = 13,
    STYX_ORACLE_Q6_K = 14,
};

#define STYX_ORACLE_SKIP 0xFFFFFFFFu

/* Threads used by the row-parallel loops (1 = the faithful single-thread
 * path).  Results do not depend on the thread count: rows are independent
 * and each row's sum order is fixed. */
void styx_oracle_set_threads(int n);
int styx_oracle_get_threads(void);

/* IEEE binary16 -> binary32 (exact).  half 2.7.1 f16::to_f32
 * (Cargo.lock:49-50) as used by crates/model/src/moe.rs:508-509.
 * Pinned by: all 65536 inputs vs numpy float16. */
float styx_oracle_f16_to_f32(uint16_t h);

/* Elements and bytes per block; 0 on unknown type.
 * crates/gguf-rs/src/lib.rs:242-332. */
int styx_oracle_block_elems(int type);
int styx_oracle_block_bytes(int type);

/* Dequantize n_elems (a multiple of the block size) from GGUF blocks.
 *   q8_0: crates/model/src/lib.rs:103-113, crates/vk-backend/tests/ops2.rs:105-110
 *   q4_K: crates/model/src/moe.rs:506-533, crates/vk-backend/tests/kernels.rs:295-333
 *   q5_K, q6_K: public ggml block format (not in the reference tree).
 * Pinned by: exhaustive byte sweeps, q5_K(qh=0) == q4_K, hand-built q6_K
 * blocks, the gguf-rs block-size table (tests/test_oracle_quant.py). */
int styx_oracle_dequant(int type, const uint8_t *blocks, int64_t n_elems, float *out);

/* y[r] = sum_c deq(W)[r][c] * x[c]: dequantize the full row to f32, then a
 * sequential f32 sum of products (crates/vk-backend/tests/kernels.rs:183-198,
 * ops2.rs:242-250).  type 0 (f32) rows are supported too.
 * Pinned by: f64 closed form and the reference tests' LCG known-answer
 * setups (tests/test_oracle_ops.py). */
int styx_oracle_matvec(int type, const uint8_t *w, int nrows, int ncols,
                       const float *x, float *y);
/* Same dot in f64 (the checker for the above). */
int styx_oracle_matvec_f64(int type, const uint8_t *w, int nrows, int ncols,
                           const float *x, double *y);

/* Expert matvec, mul_mat_vec_id semantics (crates/vk-backend/tests/kernels.rs:124-131,
 * crates/model/src/moe.rs:1561-1606): for slot s < n_ids with e = ids[s] != SKIP,
 *   y[s*nrows + r] = dot(deq(W[e])[r], x[(s % ne11) * ncols ...])
 * W[e] starts at e * expert_stride_bytes.  SKIP slots are left untouched.
 * Pinned by: routing-permutation invariance (kernels.rs:256-279) and the
 * per-slot single-matrix matvec. */
int styx_oracle_matvec_id(int type, const uint8_t *w, int nrows, int ncols,
                          int64_t expert_stride_bytes, const uint32_t *ids, int n_ids,
                          const float *x, int ne11, float *y);

/* RMSNorm over nrows rows of ncols: mean = sum(v*v)/n (sequential f32),
 * scale = 1/sqrt(mean+eps), out = (v*scale)*w (w may be NULL).
 * crates/vk-backend/tests/kernels.rs:58-67; weight multiply per the
 * do_multiply spec constant used at crates/model/src/moe.rs:668,1746-1766.
 * Pinned by: f64 closed form, scale invariance. */
void styx_oracle_rms_norm(const float *x, const float *w, int ncols, int nrows,
                          float eps, float *out);

/* Router logits in the matvec_strided_f32 order: 32 lane-strided partial
 * sums then a fixed halving tree (shaders/matvec_strided_f32.comp:25-35).
 * Pinned by: f64 closed form. */
void styx_oracle_router_strided(const float *W, const float *x, int nrows, int ncols,
                                int stride, float *out);

/* Top-k softmax routing with the four id rows
 * (shaders/topk_softmax_f32.comp:29-67).  ids_row must hold 64 int32:
 * [0..k) original, [16+s) hot, [32+s) arena, [48+s) gtt.  remap/pmap may be
 * NULL (treated as all-SKIP).  Only the first k entries of each row are
 * written.  Ties keep the lowest index (strict '>').
 * Pinned by: brute-force stable sort, sum(w)=1 under renorm, row partition. */
void styx_oracle_topk_softmax(const float *logits, int n, int k, int renorm,
                              const uint32_t *remap, const uint32_t *pmap,
                              float *weights, int32_t *ids_row);

/* out = g/(1+exp(-g)) * u (crates/vk-backend/tests/ops2.rs:305-309).
 * Pinned by: f64 closed form. */
void styx_oracle_swiglu(const float *g, const float *u, int n, float *out);

/* x[i] += sum_{s<k} w[s]*d[s*ne+i], accumulated from 0 in ascending s
 * (shaders/moe_reduce_f32.comp:8-13).  Pinned by: f64 closed form. */
void styx_oracle_moe_reduce(const float *d, const float *w, int ne, int k, float *x);

/* d[i] += sigmoid(g0)*a[i] (shaders/axpy_sig_f32.comp:7-11). */
void styx_oracle_axpy_sig(const float *a, float g0, int n, float *d);

/* NEOX rope in place over nh heads of hd: pairs (i, i+hd/2),
 * theta = pos * base^(-2i/hd), rotation in f64 then rounded
 * (crates/vk-backend/tests/ops2.rs:426-442).
 * Pinned by: pos-0 identity, pair-norm preservation, angle addition. */
void styx_oracle_rope_neox(float *x, int hd, int nh, int pos, float base);

/* Decode attention, restating shaders/attn_decode_f32.comp:31-79: one head
 * at a time, online softmax over t < n_t, 128-lane tree dot products.
 * K and V are [t][kv_dim] row-major.  Requires hd <= 256.
 * Pinned by: two-pass f64 softmax attention (below), n_t=1 => out == V[0]. */
void styx_oracle_attn_decode(const float *q, const float *K, const float *V, int n_t,
                             int hd, int kv_dim, int gqa, int n_heads, float scale,
                             float *out);
void styx_oracle_attn_decode_f64(const float *q, const float *K, const float *V, int n_t,
                                 int hd, int kv_dim, int gqa, int n_heads, double scale,
                                 double *out);

/* gather_slabs semantics (shaders/gather_slabs_f32.comp:40-86): for slot
 * s<k with ids[s] != SKIP, copy slab ids[s] of each source tensor (src
 * slab bytes) to arena slot layer*k+s (dst slab bytes).  SKIP slots and
 * all other arena bytes are untouched.  Pinned by: memcmp. */
void styx_oracle_gather_slabs(const uint8_t *const src[3], const int64_t src_slab[3],
                              uint8_t *const dst[3], const int64_t dst_slab[3],
                              const uint32_t *ids, int k, int layer);

/* ------------------------------------------------------------------------
 * MoE block and full decode step.
 * ---------------------------------------------------------------------- */

typedef struct {
    int type;               /* ggml type id; 0 = f32 */
    int nrows;              /* rows per matrix (per expert for *_exps) */
    int ncols;
    const uint8_t *data;    /* GGUF layout; NULL = absent */
} styx_oracle_mat;

typedef struct {
    const float *attn_norm;     /* [H] */
    const float *q_norm;        /* [hd] */
    const float *k_norm;        /* [hd] */
    const float *ffn_norm;      /* [H] */
    styx_oracle_mat wq, wk, wv, wo;
    const float *router;        /* [E][H] f32 */
    const float *router_bias;   /* [E] additive logit bias, NULL = none */
    styx_oracle_mat gate_exps, up_exps, down_exps;
    /* shared expert (NULL data = absent) */
    styx_oracle_mat gate_sh, up_sh, down_sh;
    const float *gate_inp_sh;   /* [H] */
} styx_oracle_layer;

typedef struct {
    int n_layers, n_embd, n_heads, n_kv_heads, head_dim;
    int n_expert, n_expert_used, n_ff_exp, n_ff_sh, n_vocab, n_ctx;
    float rms_eps, rope_base;
    int norm_topk;
    const styx_oracle_layer *layers;
    const float *output_norm;   /* [H] */
    styx_oracle_mat output;     /* [V][H] */
    styx_oracle_mat token_embd; /* [V][H] */
    float *kcache;              /* [n_layers][n_ctx][kv_dim], caller-owned */
    float *vcache;
} styx_oracle_model;

/* One MoE FFN block in place on the residual x
 * (crates/model/src/moe.rs:1974-2062): ffn_norm -> router (+bias) ->
 * topk_softmax -> gate/up -> swiglu -> down -> moe_reduce, then the
 * shared-expert branch if present.  xn_out [H], logits_out [E], ids_out [k],
 * weights_out [k] may be NULL. */
int styx_oracle_moe_block(const styx_oracle_model *m, int layer, float *x,
                          float *xn_out, float *logits_out, int32_t *ids_out,
                          float *weights_out);

/* One decode step at position pos (crates/model/src/moe.rs:1780-2157):
 * embedding, the layer loop, final norm and LM head.  Writes K/V row pos.
 * logits [V] required; hidden [n_layers+1][H] (residual after each layer,
 * index 0 = embedding), ids [n_layers][k], margins [n_layers] (k-th minus
 * (k+1)-th routing logit) are optional. */
int styx_oracle_forward(styx_oracle_model *m, int pos, uint32_t token, float *logits,
                        float *hidden, int32_t *ids, float *margins);

/* Greedy argmax, ties -> highest index (Rust max_by + total_cmp,
 * crates/model/examples/generate_moe.rs:29). */
uint32_t styx_oracle_argmax(const float *v, int n);

#ifdef __cplusplus
}
#endif
#endif
