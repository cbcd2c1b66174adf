// kernels.h -- host-side launch interface of the HIP kernels in libstyx_hip.
#pragma once

#include "common.h"

namespace styx {

// Lane-group geometry for a matvec over rows of `ncols` values of type t.
struct Geo {
    int G;    // lanes per row
    int UPL;  // units per lane
    int units;
};
Geo pick_geo(int t, int ncols);

// Slab sources of one expert tensor for the three id rows written by the
// router (hot / arena / host), see topk_softmax_f32.comp:4-17.
struct ExpSrc {
    const uint8_t *hot;
    int64_t hot_slab;
    const uint8_t *arena;
    int64_t arena_slab;
    const uint8_t *gtt;
    int64_t gtt_slab;
};

struct DenseSeg {
    const uint8_t *w;  // split-layout matrix
    float *y;
    int rows;
};

// Limbs of x (u == null, norm_w == null), of rmsnorm(x) * norm_w, or of
// swiglu(x, u) (u != null), n <= XQ_MAX; xn_out (optional) gets the f32
// vector the limbs encode.  One workgroup.
hipError_t launch_xq(hipStream_t st, const float *x, const float *u, const float *norm_w,
                     float eps, int n, const Xq &q, float *xn_out);

// y_seg = W_seg . x for up to 3 matrices sharing type/ncols, x given by its
// limbs (times the RMSNorm scale of `ns` if given).  add != 0 accumulates
// into y.
struct NormScale;
hipError_t launch_dense(hipStream_t st, int t, int ncols, const DenseSeg *segs, int nseg,
                        const Xq &xq, int add, const NormScale *ns = nullptr,
                        unsigned long long *amax = nullptr);

// Router for one layer (fused ffn_norm): writes logits[E] and, from its first
// workgroup, xn (f32) and its limbs xq (if xq.A).  launch_router_topk also
// runs the top-k into weights[k] and the 64-int id row.
struct RouterArgs {
    const float *x, *norm_w, *W, *bias;
    float eps;
    float *xn, *logits, *wts;
    Xq xq;
    int32_t *ids;
    const uint32_t *remap, *pmap;
    int E, H, k, renorm, arena_mode, layer;
};
hipError_t launch_router(hipStream_t st, const RouterArgs &a);
hipError_t launch_router_topk(hipStream_t st, const RouterArgs &a);

// Top-k ids ranked inside a consumer kernel from the router logits
// (topk_softmax_f32 selection order); the first workgroup publishes the id
// row to ids_out.  The weights are formed by k_down_reduce.
struct Route {
    const float *logits;
    int E, k;
    const uint32_t *remap, *pmap;
    int arena_mode, layer;
    int32_t *ids_out;
};

// Standalone topk_softmax_f32 over given logits (one workgroup).
hipError_t launch_topk_softmax(hipStream_t st, const float *logits, int n, int k, int renorm,
                               const uint32_t *remap, const uint32_t *pmap, int arena_mode,
                               int layer, float *wts, int32_t *ids);

// gu[0][s] = Wg[e_s] xn, gu[1][s] = Wu[e_s] xn for the k routed slots, xn
// given by its limbs; routing from `route` (ranked in-kernel) or, if null,
// the id row `ids`.  With sh_gate/sh_up (split-layout matrices of the same
// types and width F) the shared expert is slot k: gu is [2][k+1][F].
// Slot filter of the expert kernels: every routed slot, only the slots whose
// expert is hot (in HBM; the shared expert counts as hot), or only the
// others (arena / host).  A filtered-out slot's outputs are left untouched,
// so a hot launch and a cold launch together write what one launch does.
enum SlotFilter { SLOTS_ALL = 0, SLOTS_HOT = 1, SLOTS_COLD = 2 };

hipError_t launch_moe_gate_up(hipStream_t st, int tg, int tu, const ExpSrc &g, const ExpSrc &u,
                              const int32_t *ids, const Route *route, const Xq &xq, float *gu,
                              int H, int F, int k, const uint8_t *sh_gate = nullptr,
                              const uint8_t *sh_up = nullptr, int filter = SLOTS_ALL);

// h[s] = swiglu(Wg[e_s] xn, Wu[e_s] xn) for the k slots, e_s = ids[s] (one
// id per slot; an id at or past n_slabs, SKIP among them, leaves h[s]
// untouched); wg / wu hold n_slabs split-layout slabs slab_g / slab_u bytes
// apart; xn given by its limbs; h is [k][F].
hipError_t launch_moe_gate_up_silu(hipStream_t st, int tg, int tu, const uint8_t *wg,
                                   int64_t slab_g, const uint8_t *wu, int64_t slab_u,
                                   const int32_t *ids, uint32_t n_slabs, const Xq &xq, float *h,
                                   int H, int F, int k);
// partial[s] = Wd[e_s] h[s] with e_s = ids[s] as above (a skipped slot's
// partial is zeros); partial is [k][H].
hipError_t launch_moe_down_h(hipStream_t st, int td, const uint8_t *wd, int64_t slab_d,
                             const int32_t *ids, uint32_t n_slabs, const float *h, float *partial,
                             int H, int F, int k);

// partial[s] = Wd[e_s] swiglu(gu[0][s], gu[1][s]) for the k routed slots
// (and the shared expert's down matrix as slot k if sh_down); gu is
// [2][nslots][F], partial [nslots][H].
hipError_t launch_moe_down(hipStream_t st, int td, const ExpSrc &d, const int32_t *ids,
                           const float *gu, float *partial, int H, int F, int k,
                           const uint8_t *sh_down = nullptr, int filter = SLOTS_ALL);

// The whole MoE block of one layer in one launch of nwg workgroups (all
// resident at once): ffn RMSNorm + router, top-k, gate/up, swiglu + down,
// the weighted combine into x and the next RMSNorm's limbs -- the results of
// launch_router + launch_moe_gate_up + launch_moe_down + launch_reduce_rows,
// bit for bit.  Workgroups exchange data through the tagged buffers t_lg
// [E], t_gu [k+1][F] (each slot's swiglu of its gate and up rows), t_part
// [k+1][H] (64-bit words, zeroed once at
// allocation) and draw a ticket at entry from one of 64 counters (ticket
// points at 64 x 16 zeroed u64; nwg a multiple of 64); a wait that exceeds
// max_polls rounds sets *abort.  trace (optional): [nwg][8] wall-clock
// stamps per workgroup at its phase boundaries.  hipErrorNotSupported: shapes outside the
// kernel's geometry (use the separate kernels).
struct MoeBlockArgs {
    int tg, tu, td;
    float *x;  // residual [H], updated in place
    const float *ffn_norm, *W, *bias;
    float eps;
    int H, F, E, k, renorm;
    ExpSrc src[3];
    Route route;  // remap, pmap, layer, ids_out; arena_mode must be 0
    const uint8_t *sh[3];
    const float *sh_ginp;
    const float *norm_next;  // null: no limbs for a next matvec
    Xq xq;
    float *ss;
    float *wts_out;
    uint64_t *t_lg, *t_gu, *t_part;
    unsigned long long *ticket;
    int *abort;
    int max_polls;
    uint64_t *trace;
    // optional: the next layer's q/k/v matvec folded into the tail (q8_0
    // split-layout matrices [rows][H]; the RMSNorm of norm_next applied as
    // by launch_dense with a NormScale); t_xq: tagged [xq_bytes(H)/4 +
    // H/256] words
    const uint8_t *wqkv[3];
    float *qkv_out[3];
    int qkv_rows[3];
    uint64_t *t_xq;
    int nwg;
};
hipError_t launch_moe_block(hipStream_t st, const MoeBlockArgs &a);
// Workgroups of the fused MoE kernel that fit on one CU at these shapes
// (0: shapes not handled by it).
int moe_block_occupancy(int tg, int tu, int td, int H, int F, int E, int k, int shexp);
// Whether a block of these shapes on nwg workgroups takes the next layer's
// q8_0 q/k/v (rows[3] rows of H columns) into its tail.
bool moe_block_fold_ok(int tg, int tu, int td, int H, int F, int E, int k, int shexp,
                       const int rows[3], int nwg);

// H / 256 workgroups: w_s from the router logits and the id row
// (topk_softmax_f32.comp:29-67) or given in wts;
//   x += sum_s w_s partial[s]  (s ascending, moe_reduce_f32.comp:11-13)
//   x += sigmoid(sh_ginp . xn) * sh_y  (axpy_sig_f32.comp)
// then, if norm_w, the limbs of x ⊙ norm_w and per-256-row partial sums of
// x^2 into ss ([ceil(H / 256)]) -- the next matvec applies the RMSNorm scale.
struct ReduceArgs {
    const float *partial;
    int k, H;
    const float *logits;   // null: weights from wts
    int E, renorm;
    const int32_t *ids;    // original expert per slot (id row)
    const float *wts;
    float *wts_out;        // optional: weights used
    float *x;
    const float *sh_y, *sh_ginp, *xn;
    const float *norm_w;
    Xq xq;
    float *ss;
};
hipError_t launch_reduce_rows(hipStream_t st, const ReduceArgs &a);

// The scale of an RMSNorm folded into a matvec whose limbs hold x ⊙ w:
// each dot is multiplied by 1/sqrt(sum(ss[0..n_ss)) / n + eps)
// (rms_norm_f32, crates/model/src/moe.rs:1746-1766).
struct NormScale {
    const float *ss;
    int n_ss, n;
    float eps;
};

// Decode attention over the paged f32 KV cache with fused per-head q/k
// RMSNorm, NEOX rope and the K/V append at the current position.
struct AttnArgs {
    const float *q, *k, *v;          // raw projections
    const float *q_norm, *k_norm;    // [hd] or null
    float eps;
    const double2 *rope;             // [n_pos][hd/2] (cos, sin) of pos * base^(-2i/hd)
    const double2 *rope_row;         // [hd/2]: the row of *pos, written before the launch
                                     // in stream order (the engine's embedding kernel),
                                     // loaded without waiting for the position; or null
    float *kpool, *vpool;            // [pages][page_tokens][kv_dim], or
                                     // [pages][nkv][page_tokens][hd] (kv_head_major)
    const int32_t *page_table;       // logical page -> physical page
    int page_tokens;
    int kv_head_major;
    int page_table_len;              // entries of page_table (0: not given)
    int solo_max;                    // contexts of up to this many tokens are one chunk
                                     // per kv head (no exchange between chunks; on the
                                     // matrix-core kernel when head_dim is 128 and 4 to 16
                                     // query heads share a kv head); 0: off.  Without
                                     // t_part it needs max_chunks == 1: every context is
                                     // then one chunk, written directly (no tickets drawn,
                                     // no combine kernel)
    const int32_t *pos;              // device scalar
    float *out;                      // [nh*hd]
    Xq xq;                           // optional limbs of out (o-proj input)
    float *part;                     // [nkv][max_chunks][gqa][hd+2]
    int nh, nkv, hd;
    int chunk;       // minimum tokens per workgroup (multiple of 16); a context of
                     // n_t uses max(chunk, ceil16(n_t / max_chunks))
    int max_chunks;  // workgroups per kv head (grid); partials are sized by it
    float scale;
    // In-kernel combine (optional): partials go out as tagged words to
    // t_part (same shape as part); for each query head one chunk's
    // workgroup merges them and writes out + xq, and no combine kernel runs.
    // tickets: 64 x 16 zeroed u64 (xchg.h); abort: the bounded-wait flag.
    uint64_t *t_part;
    unsigned long long *tickets;
    int *abort;
    int max_polls;
    // Optional phase stamps (measurement): AT_TRACE wall-clock ticks per
    // workgroup at trace[(kvh * gridDim.x + chunk) * AT_TRACE]; workgroups
    // past the context write nothing.
    uint64_t *trace;
};
// Stamps: 0 entry, 1 q heads rotated, 2 tiles done, 3 partials stored,
// 4 partials seen (in-kernel combine), 5 end, 6 active chunks, 7 the
// workgroup (kvh << 16 | chunk) + 1.
constexpr int AT_TRACE = 8;
hipError_t launch_attn_decode(hipStream_t st, const AttnArgs &a);
// Chunks per kv head up to which the partials are merged in-kernel (the
// caller's choice; with t_part the launch has no more chunk workgroups than
// this, which leaves the chunking of such contexts unchanged).
constexpr int ATTN_MERGE_MAX_CHUNKS = 32;

// x = dequant(token_embd[tok]) for the token held in device memory, and
// (if q.A) the limbs of x ⊙ norm_w (of x if norm_w is null) with ss[0] =
// sum x^2 for the consumer's RMSNorm scale.  With rope_row, also copies the
// rope table's row of *pos ([half] (cos, sin)) there, for the attention
// kernels of the token (AttnArgs::rope_row).
hipError_t launch_embed(hipStream_t st, int t, const uint8_t *w, int64_t nrows, int ncols,
                        const uint32_t *tok, float *x, const float *norm_w, const Xq &q,
                        float *ss, const double2 *rope = nullptr, const int32_t *pos = nullptr,
                        double2 *rope_row = nullptr, int half = 0);

// Greedy argmax over logits (ties -> highest index, generate_moe.rs:29),
// in two kernels through part_val/part_idx (64 entries each).  Writes
// out_tok; if advance != 0 also pos += 1 and hist[pos] = result.
hipError_t launch_argmax(hipStream_t st, const float *v, int n, uint32_t *out_tok,
                         float *part_val, uint32_t *part_idx, int32_t *pos, int advance,
                         uint32_t *hist);
// The token of a running argmax word that launch_dense(..., amax) filled
// (argmax_key order): written to out_tok (and hist[pos+1], pos advanced when
// advance != 0); the word is cleared for the next launch.
hipError_t launch_argmax_word(hipStream_t st, unsigned long long *amax, uint32_t *out_tok,
                              int32_t *pos, int advance, uint32_t *hist);

// gather_slabs_f32 semantics: for slot s<k with arena id != SKIP copy expert
// ids[s]'s slab of each tensor into arena slot ids[32+s].
hipError_t launch_gather(hipStream_t st, const uint8_t *const src[3], const int64_t src_slab[3],
                         uint8_t *const dst[3], const int64_t dst_slab[3],
                         const int32_t *ids, const Route *route, int k);
// Plain gather with explicit expert list (reference binding: ids = expert
// per slot, arena slot layer*k+s).  src_count (or null): slabs readable in
// each source; an id at or past it is skipped like SKIP.
hipError_t launch_gather_list(hipStream_t st, const uint8_t *const src[3],
                              const int64_t src_slab[3], uint8_t *const dst[3],
                              const int64_t dst_slab[3], const int32_t *ids, int k, int layer,
                              const int64_t *src_count = nullptr);

// GGUF block layout <-> split layout, for nmat matrices of nblocks blocks.
hipError_t launch_to_split(hipStream_t st, int t, const uint8_t *src, uint8_t *dst,
                           int64_t nblocks, int64_t nmat);
hipError_t launch_from_split(hipStream_t st, int t, const uint8_t *src, uint8_t *dst,
                             int64_t nblocks, int64_t nmat);

// Dequantize rows [r0, r0+nrows) of a split-layout matrix (nrows_total rows)
// to f32 with the reference evaluation order.
hipError_t launch_dequant_rows(hipStream_t st, int t, const uint8_t *w, int64_t nrows_total,
                               int ncols, int64_t r0, int64_t nrows, float *out);

// Seeded synthetic weights: N(0, sigma) quantized to GGUF blocks of type t
// (or f32), n values.  Deterministic in (seed, index).
hipError_t launch_gen_quant(hipStream_t st, int t, uint64_t seed, float sigma, uint8_t *dst,
                            int64_t n);
hipError_t launch_gen_f32(hipStream_t st, uint64_t seed, float mean, float sigma, float *dst,
                          int64_t n);

hipError_t launch_fill_u32(hipStream_t st, uint32_t *p, uint32_t v, int64_t n);
// dst[i] = min(src[i], maxv) (unsigned) for i < n.
hipError_t launch_clamp_copy_u32(hipStream_t st, const uint32_t *src, uint32_t *dst, uint32_t maxv,
                                 int64_t n);

// Streaming-read probe over bytes (multiple of 16); out gets 4*grid words.
hipError_t launch_read_probe(hipStream_t st, const void *p, int64_t bytes, uint32_t *out,
                             int grid);

}  // namespace styx
