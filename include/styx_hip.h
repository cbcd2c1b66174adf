/*
 * styx_hip.h -- C ABI of libstyx_hip.so, the MI355X (gfx950) backend of the
 * styx / moe-stream MoE decode hot path.
 *
 * It replaces the Rust crate crates/vk-backend (Vulkan) of aDirtyScoundrel/styx
 * as the engine's GPU boundary, and exports a C++ port of the engine API of
 * crates/model/src/moe.rs (MoeModel) on top of it.  Plain C types only: opaque
 * handles, pointers and sizes.  Every call returns 0 (STYX_OK) or a negative
 * status; styx_last_error() gives the thread's last message.  Nothing aborts
 * across the boundary.  Handles are owned by the caller and freed explicitly
 * (the reference's Buffer/Pipeline/Batch have no Drop either,
 * crates/vk-backend/src/lib.rs:18-52); a gpu must outlive its children.
 *
 * Threading: one batch / model per thread; all work of a gpu runs in order on
 * its compute stream.
 */
#ifndef STYX_HIP_H
#define STYX_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ----------------------------------------------------------- status ---- */
enum {
    STYX_OK = 0,
    STYX_E_INVALID = -1,      /* bad argument (reference: assert!/Err) */
    STYX_E_HIP = -2,          /* HIP runtime error */
    STYX_E_OOM = -3,
    STYX_E_IO = -4,
    STYX_E_FORMAT = -5,       /* GGUF / tensor layout rejected */
    STYX_E_STATE = -6,        /* call out of order (e.g. KV full) */
    STYX_E_UNSUPPORTED = -7,
    STYX_E_DEVICE = -8,       /* a device-side wait gave up (stage timing; tokens fall back) */
};
/* Thread-local message of the last failing call (never NULL). */
const char *styx_last_error(void);

/* ggml type ids (crates/gguf-rs/src/lib.rs:242-332) used on this path. */
enum { STYX_F32 = 0, STYX_F16 = 1, STYX_Q8_0 = 8, STYX_Q4_K = 12, STYX_Q5_K = 13, STYX_Q6_K = 14 };
#define STYX_SKIP 0xFFFFFFFFu

/* ----------------------------------------------------------- device ---- */
typedef struct styx_gpu styx_gpu;
/* Gpu::new (crates/vk-backend/src/lib.rs:356): opens HIP device `device`. */
int styx_gpu_new(int device, styx_gpu **out);
/* Drop for Gpu (lib.rs:1602-1611): waits for the device, frees the stream. */
void styx_gpu_free(styx_gpu *gpu);
/* Gpu::vram_bytes (lib.rs:534). */
uint64_t styx_gpu_hbm_bytes(const styx_gpu *gpu);
/* Gpu::device_name (lib.rs:336-353). */
const char *styx_gpu_name(const styx_gpu *gpu);
/* Gpu::wait_idle-equivalent: block until all queued work has finished. */
int styx_gpu_sync(styx_gpu *gpu);

/* ---------------------------------------------------------- buffers ---- */
typedef struct styx_buf styx_buf;
enum {
    STYX_BUF_DEVICE = 0,       /* HBM (create_buffer, lib.rs:568) */
    STYX_BUF_HOST_PINNED = 1,  /* pinned host memory mapped for the GPU
                                  (create_buffer_host / _host_shared,
                                  lib.rs:756, 802) */
};
int styx_buf_new(styx_gpu *gpu, uint64_t bytes, int kind, styx_buf **out);
/* destroy_buffer (lib.rs:1517). */
void styx_buf_free(styx_buf *buf);
uint64_t styx_buf_size(const styx_buf *buf);
/* Device address of the buffer (Gpu::device_address, lib.rs:1136). */
void *styx_buf_device_ptr(const styx_buf *buf);
/* Gpu::upload (lib.rs:1033) / download (lib.rs:1175): synchronous copies. */
int styx_upload(styx_gpu *gpu, styx_buf *dst, uint64_t off, const void *src, uint64_t n);
int styx_download(styx_gpu *gpu, const styx_buf *src, uint64_t off, void *dst, uint64_t n);
/* Gpu::copy_region (lib.rs:1192): device-side copy, synchronous. */
int styx_copy_region(styx_gpu *gpu, const styx_buf *src, uint64_t soff, styx_buf *dst,
                     uint64_t doff, uint64_t n);

/* ------------------------------------------------ kernels and batches ---- */
/* Gpu::create_pipeline (lib.rs:1222) and Batch (lib.rs:44-231).  A kernel is
 * named by the reference pipeline it replaces; bindings and push constants
 * keep the reference's order and byte layout (crates/vk-backend/src/ops.rs,
 * the shaders' push blocks), and (gx, gy, gz) is the reference's workgroup
 * grid, so engine code ports call for call.  Names:
 *   topk_softmax_f32, moe_reduce_f32, gather_slabs_f32, attn_decode_f32,
 *   matvec_strided_f32, add_flat_f32, axpy_sig_f32, swiglu_f32,
 *   rms_norm_f32, rope_neox_f32, cpy_f32_f32,
 *   mul_mat_vec_{q8_0,q4_k,q5_k,q6_k}_f32_f32 and the _id forms (weights in
 *   GGUF layout).
 * and the fused hot-path kernels (no reference pipeline of their own; each
 * replaces a run of the reference's dispatches, see the push blocks below):
 *   router_topk, moe_gate_up_silu_{q8_0,q4_k,q5_k,q6_k},
 *   moe_down_reduce_{q8_0,q4_k,q5_k,q6_k}, attn_decode_paged.
 * For the fused kernels the grid argument is ignored (the library sizes the
 * launch; it must still be non-zero), quant weights are in the split layout
 * of styx_op_to_split, and each dispatch may enqueue more than one kernel.
 * They use the gpu's op scratch (as the styx_op_* calls do): batches that
 * use them must not run on two streams at once.
 * styx_kernel_names() lists what this build provides. */
typedef struct styx_kernel styx_kernel;
int styx_kernel_get(styx_gpu *gpu, const char *name, const uint32_t *spec, int n_spec,
                    styx_kernel **out);
void styx_kernel_free(styx_kernel *k);
/* Comma-separated kernel names accepted by styx_kernel_get. */
const char *styx_kernel_names(void);

typedef struct {
    const styx_buf *buf;
    uint64_t offset;   /* bytes */
    uint64_t range;    /* bytes, or UINT64_MAX for the rest (vk::WHOLE_SIZE) */
} styx_binding;

typedef struct styx_batch styx_batch;
/* Gpu::create_batch (lib.rs:1530) / destroy_batch (lib.rs:1567). */
int styx_batch_new(styx_gpu *gpu, styx_batch **out);
void styx_batch_free(styx_batch *b);
/* Batch::begin (lib.rs:56). */
int styx_batch_begin(styx_batch *b);
/* Batch::dispatch_ranges_barrier (lib.rs:115-197).  Work runs in recording
 * order on one stream, so every dispatch is ordered after the previous one
 * whatever `barrier` says. */
int styx_batch_dispatch(styx_batch *b, const styx_kernel *k, const styx_binding *binds,
                        int n_binds, const void *push, uint32_t push_len, uint32_t gx,
                        uint32_t gy, uint32_t gz, int barrier);
/* Batch::submit (lib.rs:200-231): run the recorded work and wait for it
 * (an async batch runs it on its own stream). */
int styx_batch_submit(styx_batch *b);

/* Push blocks of the fused kernels (no reference counterpart; plain 32-bit
 * fields, sizes asserted below).
 *
 * router_topk replaces moe.rs:1975-2016 (rec_rms of ffn_norm, the
 * matvec_strided_f32 router, topk_softmax_f32).  10 bindings: 0 x [H] f32,
 * 1 ffn_norm [H], 2 router W [E][H] f32, 3 bias [E] (read if flags & 1),
 * 4 remap [E] u32 (flags & 2; else every expert resident at its own index),
 * 5 pmap [E] u32 (flags & 4), out: 6 xn [H], 7 logits [E], 8 weights [k],
 * 9 the 256-byte id row (topk_softmax_f32.comp:4-17 layout). */
typedef struct {
    uint32_t E, H, k, renorm, arena_mode, layer;
    float eps;
    uint32_t flags;
} styx_push_router_topk;
/* moe_gate_up_silu_{t}, t the gate type, replaces rec_matvec_id of gate and
 * of up plus swiglu_f32 (moe.rs:2023-2038): h[s] = silu(Wg[e_s] xn) *
 * (Wu[e_s] xn) for s < k with e_s = ids[s]; an id at or past n_slabs (SKIP
 * among them) leaves h[s] untouched, as SKIP does in mul_mat_vec_id.
 * 5 bindings: 0 gate weights (n_slabs slabs, slab_gate bytes apart), 1 up
 * weights (slab_up apart), 2 xn [H] f32, 3 ids: k i32 (one row of the id
 * table: +0 all experts, +64 hot, ...), 4 out h [k][F] f32.  A slab size of
 * 0 means F*H values of the type (the expert tensor's own stride). */
typedef struct {
    uint32_t H, F, k, type_up, n_slabs, slab_gate, slab_up;
} styx_push_moe_gate_up_silu;
/* moe_down_reduce_{t} replaces rec_matvec_id of down (ne11 = k) plus
 * moe_reduce_f32 (moe.rs:2039-2062): x += sum_s w_s Wd[e_s] h[s] in slot
 * order, skipped slots adding nothing (so hot and cold launches over
 * disjoint id rows together add every slot).  5 bindings: 0 down weights
 * (slab_down apart, 0 = H*F values), 1 h [k][F] f32, 2 ids [k] i32,
 * 3 weights [k] f32, 4 x [H] f32 updated in place. */
typedef struct {
    uint32_t H, F, k, n_slabs, slab_down;
} styx_push_moe_down_reduce;
/* attn_decode_paged replaces moe.rs:1875-1964 (per-head q/k rms_norm,
 * rope_neox_f32 of q and k, the two cpy_f32_f32 KV appends at pos and
 * attn_decode_f32) for one layer at position pos (context pos + 1).
 * 11 bindings: 0 q [nh*hd], 1 k [nkv*hd], 2 v [nkv*hd] (raw projections),
 * 3 q_norm [hd] (flags & 1), 4 k_norm [hd] (flags & 2), 5 rope table
 * [> pos][hd/2][2] f64 (styx_rope_table), 6 K pool, 7 V pool, 8 page table
 * [i32] (flags & 4: pools of whole pages of page_tokens rows [token][nkv*hd],
 * logical page i at physical page table[i]; otherwise the pools are the
 * reference's contiguous [cap][nkv*hd] caches), 9 out [nh*hd] f32, 10 part:
 * styx_op_attn_part_floats(nh, nkv, hd, max_chunks) floats.  The context
 * is split over max_chunks workgroups per kv head of at least `chunk`
 * tokens (a multiple of 16), as in styx_op_attn_decode.  Page-table entries
 * past the pool are clamped to its last page. */
typedef struct {
    float eps;
    uint32_t page_tokens, nh, nkv, hd, chunk, max_chunks;
    float scale;
    uint32_t flags, pos;
} styx_push_attn_decode_paged;
#ifdef __cplusplus
static_assert(sizeof(styx_push_router_topk) == 32, "push layout");
static_assert(sizeof(styx_push_moe_gate_up_silu) == 28, "push layout");
static_assert(sizeof(styx_push_moe_down_reduce) == 20, "push layout");
static_assert(sizeof(styx_push_attn_decode_paged) == 40, "push layout");
#endif

/* Gpu::dispatch_sync (lib.rs:1415-1515): one dispatch, run and waited for. */
int styx_dispatch_sync(styx_gpu *gpu, const styx_kernel *k, const styx_binding *binds,
                       int n_binds, const void *push, uint32_t push_len, uint32_t gx, uint32_t gy,
                       uint32_t gz);

/* Asynchronous submission (the reference's M7b-B prefetch path).
 * A timeline stands in for a Vulkan timeline semaphore: every
 * styx_batch_submit_async signals one value (values strictly increase), and
 * a batch submitted with styx_batch_submit_wait_sem starts once the
 * timeline has reached its value.  Deviation: a wait for a value that no
 * submit has signalled yet fails with STYX_E_STATE (Vulkan allows
 * wait-before-signal). */
typedef struct styx_timeline styx_timeline;
/* Gpu::create_timeline_semaphore (lib.rs:700-713), initial value 0. */
int styx_timeline_new(styx_gpu *gpu, styx_timeline **out);
void styx_timeline_free(styx_timeline *t);
/* The largest signalled value whose batch has completed
 * (vkGetSemaphoreCounterValue). */
int styx_timeline_value(styx_timeline *t, uint64_t *value);
/* Gpu::create_async_batch (lib.rs:716-754): a batch on a stream of its own
 * (default priority), beside the gpu's stream; styx_batch_free on it waits
 * for its in-flight work first (destroy_async_batch, lib.rs:1577-1589). */
int styx_batch_new_async(styx_gpu *gpu, styx_batch **out);
/* Batch::submit_async (lib.rs:233-271): run the recorded work on the async
 * batch's stream and return at once; the timeline reaches `value` when it
 * completes.  STYX_E_STATE for a batch not made by styx_batch_new_async. */
int styx_batch_submit_async(styx_batch *b, styx_timeline *t, uint64_t value);
/* Batch::wait_idle (lib.rs:273-287): wait for the last submit_async. */
int styx_batch_wait_idle(styx_batch *b);
/* Batch::submit_wait_sem (lib.rs:289-333): the recorded work starts once
 * the timeline reaches `value`; returns when it is done. */
int styx_batch_submit_wait_sem(styx_batch *b, styx_timeline *t, uint64_t value);

/* ------------------------------------------------------- hot-path ops ---- */
/* Direct entry points of the gfx950 kernels (device pointers, enqueued on
 * the gpu's stream; call styx_gpu_sync to wait).  Weights are in the split
 * layout produced by styx_op_to_split unless stated otherwise. */

/* GGUF block layout -> split layout (and back) for nmat matrices of
 * nblocks blocks each (an expert tensor is nmat = n_expert slabs). */
int styx_op_to_split(styx_gpu *gpu, int type, const void *src, void *dst, int64_t nblocks,
                     int64_t nmat);
int styx_op_from_split(styx_gpu *gpu, int type, const void *src, void *dst, int64_t nblocks,
                       int64_t nmat);
/* Dequantize rows [r0, r0+nrows) of a split matrix with nrows_total rows
 * to f32, in the reference's evaluation order (bit-exact dequant). */
int styx_op_dequant_rows(styx_gpu *gpu, int type, const void *w, int64_t nrows_total,
                         int ncols, int64_t r0, int64_t nrows, float *out);
/* y = W . xn (add: y += W . xn), xn = norm_w ? rmsnorm(x, eps) * norm_w : x.
 * mul_mat_vec_{t}_f32_f32 + rms_norm_f32 (crates/model/src/moe.rs:1523-1551,
 * 1746-1766). */
int styx_op_matvec(styx_gpu *gpu, int type, const void *w, int nrows, int ncols,
                   const float *x, const float *norm_w, float eps, float *y, int add);
/* Fused ffn_norm + router (matvec_strided_f32) + topk_softmax_f32
 * (crates/model/src/moe.rs:1974-2016).  W [E][H] f32, bias [E] or NULL,
 * remap/pmap [E] or NULL (NULL remap = every expert resident at its own
 * index), arena_mode: cold experts get arena slot layer*k+s.  Writes
 * xn [H], logits [E], weights [k], ids [64]. */
int styx_op_router_topk(styx_gpu *gpu, const float *x, const float *norm_w, float eps,
                        const float *W, const float *bias, int E, int H, int k, int renorm,
                        const uint32_t *remap, const uint32_t *pmap, int arena_mode, int layer,
                        float *xn, float *logits, float *weights, int32_t *ids);
/* topk_softmax_f32 alone (shaders/topk_softmax_f32.comp). */
int styx_op_topk_softmax(styx_gpu *gpu, const float *logits, int n, int k, int renorm,
                         const uint32_t *remap, const uint32_t *pmap, int arena_mode, int layer,
                         float *weights, int32_t *ids);
/* Expert slab sources selected per slot by the id row (moe.rs:1649-1700). */
typedef struct {
    const void *hot;    int64_t hot_slab;    /* HBM tensor / hot buffer */
    const void *arena;  int64_t arena_slab;  /* HBM arena slots */
    const void *host;   int64_t host_slab;   /* pinned host tensor */
} styx_expert_src;
/* gu[0][s] = Wg[e_s] . xn, gu[1][s] = Wu[e_s] . xn  (mul_mat_vec_id_*,
 * ne11 = 1, moe.rs:2023-2038).  gu is [2][k][F]. */
int styx_op_moe_gate_up(styx_gpu *gpu, int type_gate, int type_up, const styx_expert_src *gate,
                        const styx_expert_src *up, const int32_t *ids, const float *xn, float *gu,
                        int H, int F, int k);
/* x += sum_s w_s * Wd[e_s] . swiglu(gu[0][s], gu[1][s])  (swiglu_f32 +
 * mul_mat_vec_id ne11=k + moe_reduce_f32, moe.rs:2025-2062); gu is
 * [2][k][F] as written by styx_op_moe_gate_up, x [H] is updated in place. */
int styx_op_moe_down_reduce(styx_gpu *gpu, int type_down, const styx_expert_src *down,
                            const int32_t *ids, const float *weights, const float *gu, float *x,
                            int H, int F, int k);
/* Decode attention over the paged KV cache with fused per-head q/k RMSNorm,
 * NEOX rope and K/V append at *pos (attn_decode_f32.comp, moe.rs:1875-1964).
 * q [nh*hd], k/v [nkv*hd] raw projections; q_norm/k_norm [hd] or NULL;
 * rope [n_pos][hd/2][2] f64 (cos, sin) from styx_rope_table, n_pos > *pos;
 * kpool/vpool [pages][page_tokens][nkv*hd];
 * page_table [ceil(n_ctx/page_tokens)]; part: styx_op_attn_part_floats().
 * The context is split over max_chunks workgroups per kv head, each of at
 * least `chunk` tokens (a multiple of 16): a context of n_t tokens uses
 * max(chunk, ceil16(n_t / max_chunks)) tokens per workgroup. */
int styx_op_attn_decode(styx_gpu *gpu, const float *q, const float *k, const float *v,
                        const float *q_norm, const float *k_norm, float eps,
                        const double *rope, float *kpool, float *vpool,
                        const int32_t *page_table, int page_tokens, const int32_t *pos,
                        float *out, float *part, int nh, int nkv, int hd, int chunk,
                        int max_chunks, float scale);
int64_t styx_op_attn_part_floats(int nh, int nkv, int hd, int max_chunks);
/* No counterpart in the reference.  styx_op_attn_decode without the `part`
 * workspace, for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).  The
 * chunk partials live in a static device array of the library,
 * STYX_NOALLOC_ATTN_PART_FLOATS floats (8 MiB) per GPU, held until the
 * process ends; a call needing more (styx_op_attn_part_floats(nh, nkv, hd,
 * max_chunks) above it) is rejected with STYX_E_INVALID.  Allocates
 * nothing.  Every call on one GPU shares that array: calls that overlap on
 * one GPU (other streams or threads) race. */
#define STYX_NOALLOC_ATTN_PART_FLOATS (2u * 1024u * 1024u)
int styx_op_attn_decode_noalloc(styx_gpu *gpu, const float *q, const float *k, const float *v,
                                const float *q_norm, const float *k_norm, float eps,
                                const double *rope, float *kpool, float *vpool,
                                const int32_t *page_table, int page_tokens, const int32_t *pos,
                                float *out, int nh, int nkv, int hd, int chunk, int max_chunks,
                                float scale);
/* Host-side NEOX rope table: out[p][i] = (cos, sin)(p * base^(-2i/hd)) in
 * f64 for p < n_pos, i < hd/2 (crates/vk-backend/tests/ops2.rs:426-442).
 * out holds n_pos * hd doubles.  Needs no GPU. */
void styx_rope_table(float base, int hd, int n_pos, double *out);
/* gather_slabs_f32 (shaders/gather_slabs_f32.comp:40-86): for slot s < k
 * with expert ids[s] != SKIP copy that expert's slab of each of the three
 * tensors into arena slot layer*k+s.  Slab sizes multiples of 16. */
int styx_op_gather_slabs(styx_gpu *gpu, const void *const src[3], const int64_t src_slab[3],
                         void *const dst[3], const int64_t dst_slab[3], const int32_t *ids,
                         int k, int layer);
/* Greedy argmax, ties -> highest index (generate_moe.rs:29).  scratch:
 * 64 f32 + 64 u32. */
int styx_op_argmax(styx_gpu *gpu, const float *v, int n, uint32_t *out, float *scratch_val,
                   uint32_t *scratch_idx);
/* Measurement helper with no counterpart in the reference: reads every
 * 16-byte word of [p, p + bytes) once with grid x 256 threads (each
 * workgroup a contiguous chunk, 8 non-temporal 16-byte loads in flight per
 * lane) and writes 4*grid fold words to out, so its duration gives the
 * achievable HBM streaming-read bandwidth of the device. */
int styx_op_read_probe(styx_gpu *gpu, const void *p, int64_t bytes, uint32_t *out, int grid);
/* Seeded synthetic data: N(0, sigma) values quantized to GGUF blocks of
 * `type` (n values; STYX_F16: each value rounded to f16), or f32
 * N(mean, sigma). */
int styx_op_gen_quant(styx_gpu *gpu, int type, uint64_t seed, float sigma, void *dst, int64_t n);
int styx_op_gen_f32(styx_gpu *gpu, uint64_t seed, float mean, float sigma, float *dst, int64_t n);

/* ------------------------------------------------------------- GGUF ----- */
/* Gguf::open (crates/gguf-rs/src/lib.rs:41-120): parse the header of a GGUF
 * v2/v3 file and write a JSON summary {version, data_start, metadata: [keys],
 * tensors: [{name, dims, type, offset, size_bytes}]} into out.  Rejections
 * carry the reference's messages (lib.rs:46-332).  Needs no GPU. */
int styx_gguf_inspect(const char *path, char *out, uint64_t cap);

/* ------------------------------------------------------------ engine ---- */
/* C++ port of crates/model/src/moe.rs MoeModel (qwen3moe). */
typedef struct styx_moe styx_moe;

typedef struct {
    int n_ctx;               /* max context; 0 = 4096 (moe.rs:705) */
    int use_graph;           /* replay each token as one HIP graph */
    int64_t expert_budget_mb;/* <0: all experts in HBM; >=0: experts in
                                pinned host memory, this much HBM for hot
                                slabs (MOE_EXPERTS_VRAM_MB, moe.rs:692-767) */
    const char *expert_hist; /* popularity CSV "layer,expert,hits"
                                (MOE_EXPERT_HIST, moe.rs:774-813) or NULL */
    int arena;               /* cold experts: 1 gather into the HBM arena
                                in-stream, 0 read in place from host */
    int repin_interval;      /* MOE_REPIN_INTERVAL (moe.rs:1450-1508); 0 off */
    int repin_max;           /* MOE_REPIN_MAX; 0 = 2 */
    int record_hidden;       /* keep the residual after every layer */
    int time_kernels;        /* HIP events around the expert kernels */
    int no_fuse;             /* 1: run the MoE block as four kernels instead of
                                the fused persistent one (same results) */
    int no_fold_qkv;         /* 1: keep every layer's q/k/v matvec a kernel of
                                its own instead of the previous fused MoE
                                block's tail (same results) */
    int max_polls;           /* rounds a fused launch's workgroup waits for
                                another's data before it gives up; 0 =
                                200000.  A launch that gives up makes the
                                model fall back to the separate kernels,
                                which do not wait, and run the token(s)
                                again (tests lower it to force that) */
} styx_moe_opts;

typedef struct {
    int n_layers, n_embd, n_heads, n_kv_heads, head_dim;
    int n_expert, n_expert_used, n_ff_exp, n_ff_shexp, n_vocab, n_ctx;
    float rms_eps, rope_base;
    int norm_topk;
    uint64_t slab_bytes;     /* gate+up+down bytes of one (layer,expert) */
    uint64_t expert_bytes_hbm, expert_bytes_host;
    int unfused_fallbacks;   /* times a fused launch gave up and the model
                                went over to the separate kernels (0 or 1) */
} styx_moe_hparams;

typedef struct {
    int n_layers, n_embd, n_heads, n_kv_heads, head_dim;
    int n_expert, n_expert_used, n_ff_exp, n_ff_shexp, n_vocab;
    float rms_eps, rope_base;
    int attn_type, embd_type, head_type;
    int exp_type[3];         /* gate, up, down (used when exp_mix == 0) */
    int exp_mix;             /* 1: type(l, role) = [q4_K,q5_K,q6_K][(l+role)%3] */
    float sigma;             /* weight std, e.g. 0.02 */
    uint64_t seed;
    float router_zipf_s;     /* >0: Zipf(s) router bias by a seeded rank
                                permutation per layer, from
                                styx_zipf_bias_table(E, k, s,
                                0.9 * sigma * sqrt(H)) */
} styx_moe_synth_cfg;

/* Popularity pinning plan (crates/model/src/moe.rs:774-813), host only:
 * rank the "layer,expert,hits" rows of hist_csv by hits (descending; ties in
 * file order) and pin (layer, expert) slabs of slab_bytes[layer] bytes each
 * until the next does not fit in budget_mb MiB; without a CSV, whole layers
 * in order.  remap[l*n_expert + e] = hot slot (rank of e among layer l's
 * pinned experts) or 0xFFFFFFFF.  This is the placement styx_moe_load and
 * styx_moe_synth use when opts.expert_budget_mb >= 0.  Needs no GPU. */
int styx_residency_plan(const char *hist_csv, int n_layers, int n_expert,
                        const uint64_t *slab_bytes, int64_t budget_mb, uint32_t *remap,
                        uint64_t *pinned_slabs);

/* Repin choice of one layer (crates/model/src/moe.rs:1465-1497), host only:
 * the resident experts slot_experts[0..n_slots) ranked coldest first by
 * hits[], the other experts hottest first (both stable on ties); pair i
 * swaps while hits[outsider] >= 2 * max(hits[resident], 1), at most
 * repin_max pairs.  Writes the slot and incoming expert of each swap and
 * their count.  This is the selection styx_moe_* applies every
 * opts.repin_interval tokens.  Needs no GPU. */
int styx_repin_select(const uint64_t *hits, int n_expert, const uint32_t *slot_experts,
                      int n_slots, int repin_max, uint32_t *swap_slot, uint32_t *swap_expert,
                      int *n_swaps);

/* The checks MoeModel::load (moe.rs:536-1408) makes before it uploads
 * anything, without a device: GGUF header, qwen3moe hyperparameters, every
 * tensor's bytes inside the file, and every tensor the model reads against
 * the dims and type its hyperparameters imply.  Fills out (may be NULL;
 * n_ctx and the expert byte counts are 0).  styx_moe_load runs the same
 * checks first. */
int styx_moe_check_file(const char *path, styx_moe_hparams *out);

/* Router bias by popularity rank for the synthetic Zipf workload (no
 * counterpart in the reference, which has no router bias): out[r] is the
 * bias of the expert of rank r+1 such that, with router logit noise
 * N(0, sd^2) per expert and token, top-k routing picks it with probability
 * min(1, lambda * (r+1)^-s) per token (the pi summing to k): Zipf(s)
 * popularity wherever top-k selection can reach it.  Fitted on a seeded
 * sample of 4096 tokens; out[0] = 0.  Needs no GPU. */
int styx_zipf_bias_table(int n_expert, int k, float s, float sd, uint64_t seed, float *out);

/* MoeModel::load (moe.rs:536-1408) from a GGUF file. */
int styx_moe_load(styx_gpu *gpu, const char *path, const styx_moe_opts *opts, styx_moe **out);
/* Build a seeded synthetic model directly in HBM (no file). */
int styx_moe_synth(styx_gpu *gpu, const styx_moe_synth_cfg *cfg, const styx_moe_opts *opts,
                   styx_moe **out);
void styx_moe_free(styx_moe *m);
/* MoeModel.hp / slab_bytes (moe.rs:373-499). */
int styx_moe_get_hparams(const styx_moe *m, styx_moe_hparams *out);
/* MoeModel::forward_token (moe.rs:1780-2157): logits [n_vocab] (may be
 * NULL to skip the download). */
int styx_moe_forward_token(styx_moe *m, uint32_t token, float *logits);
/* generate_moe main loop (crates/model/examples/generate_moe.rs:44-67):
 * token-at-a-time prefill of the prompt, then n_predict greedy tokens
 * (the first from the prefill's logits), argmax on the device. */
int styx_moe_generate(styx_moe *m, const uint32_t *prompt, int n_prompt, int n_predict,
                      uint32_t *out_tokens, double *prefill_s, double *decode_s);
/* Continue greedy decoding from the current state: n_steps forward passes,
 * each on the previous argmax token (generate_moe.rs:58-67 loop body);
 * out[i] = the token produced by step i. */
int styx_moe_decode(styx_moe *m, int n_steps, uint32_t *out);
/* The fused launches' wait bound (styx_moe_opts.max_polls) for the tokens
 * that follow (test helper, no reference counterpart). */
int styx_moe_set_wait_limit(styx_moe *m, int max_polls);
/* Turn HIP-event timing of every kernel launch on or off (launches are then
 * enqueued one by one instead of replayed as a graph). */
int styx_moe_set_timing(styx_moe *m, int on);
/* Phase stamps of the fused MoE block kernel (measurement helper, no
 * counterpart in the reference) from the last token run with timing on:
 * [n_layers][*nwg][16] wall-clock ticks per workgroup -- 0 entry, 1 x
 * normalised, 2 limbs built, 3 logits seen, 4 ranked, 5 gate/up done, 6 g/u
 * seen, 7 swiglu limbs built, 8 down done, 9 partials seen, 10 end (in the
 * workgroups past the reduce ones that form the next layer's q/k/v: 9 its
 * limbs seen, 10 its rows stored), 11 gate/up loads issued, 12 gate/up
 * limbs loaded, 13 gate/up rows done, 14 gate/up block entered, 15 its slab
 * known (0: no such phase).  *nwg = 0 when the model runs the separate
 * kernels; out may be NULL to query *nwg. */
int styx_moe_moe_block_trace(styx_moe *m, uint64_t *out, int64_t max_count, int *nwg,
                             double *ticks_per_us);
/* Phase stamps of the attention launches from the last timed token
 * (measurement helper, no counterpart in the reference):
 * [n_layers][*nwg][8] wall-clock ticks per workgroup -- 0 entry, 1 q heads
 * normalised and rotated, 2 the chunk's tiles done, 3 partials stored, 4
 * partials of the first merged head seen (in-kernel combine), 5 end, 6 the
 * active chunks, 7 (kv head << 16 | chunk) + 1; all 0 for a workgroup past
 * the context.  out may be NULL to query *nwg. */
int styx_moe_attn_trace(styx_moe *m, uint64_t *out, int64_t max_count, int *nwg,
                        double *ticks_per_us);
/* Stage timing (measurement helper, no counterpart in the reference): the
 * launches of one stage ("embed", "qkv", "attn", "o_proj", "router",
 * "gather", "moe_gate_up", "shexp", "moe_down", "reduce", "lm_head") for
 * every layer of the last token, captured as one graph (repeated to at
 * least 32 launches for shallow models) and replayed `reps` times between
 * two HIP events; *us_per_replay = mean time of one pass over the layers,
 * *launches = kernels per pass.  Needs one token run first; overwrites
 * per-token scratch that the next token rewrites before reading. */
int styx_moe_time_stage(styx_moe *m, const char *stage, int reps, double *us_per_replay,
                        int *launches);
/* MoeModel::last_expert_ids (moe.rs:2387-2402): [n_layers][k]. */
int styx_moe_last_expert_ids(styx_moe *m, uint32_t *out);
/* MoeModel::last_hot_cold (moe.rs:1512-1521): [n_layers][2] (hot, cold). */
int styx_moe_last_hot_cold(styx_moe *m, uint32_t *out);
/* MoeModel::reset (moe.rs:1410-1412). */
int styx_moe_reset(styx_moe *m);
/* Synthetic context for long-context measurement (no counterpart in the
 * reference): fill the K and V rows of positions [0, n_t) of every layer
 * (the pages holding them whole) with N(0, sigma) values (seeded,
 * deterministic) and continue as if n_t tokens had been forwarded; the next
 * styx_moe_forward_token runs at position n_t. */
int styx_moe_fill_kv(styx_moe *m, int n_t, uint64_t seed, float sigma);
/* Copy K and V rows [t0, t0+n) of one layer to the host ([n][n_kv*hd]
 * each), through the page table. */
int styx_moe_read_kv(styx_moe *m, int layer, int t0, int n, float *k, float *v);
/* Total slab swaps done by repinning (MoeModel.repin_swaps). */
uint64_t styx_moe_repin_swaps(const styx_moe *m);
/* Residuals of the last token: [n_layers+1][n_embd] (needs record_hidden). */
int styx_moe_last_hidden(styx_moe *m, float *out);
/* Copy a tensor's bytes in GGUF layout (the model's own data). */
int styx_moe_export_tensor(styx_moe *m, const char *name, void *dst, uint64_t cap,
                           uint64_t *size, int *type, int64_t dims[4], int *n_dims);
/* Names of all tensors, '\n'-separated, into buf (size cap). */
int styx_moe_tensor_names(styx_moe *m, char *buf, uint64_t cap);
/* Per-kernel event timing when opts.time_kernels: name, launches, total
 * milliseconds, algorithmic bytes summed over launches. */
typedef struct {
    char name[32];
    uint64_t launches;
    double total_ms;
    double bytes;
} styx_kernel_stat;
int styx_moe_kernel_stats(styx_moe *m, styx_kernel_stat *out, int cap, int *n);
int styx_moe_kernel_stats_reset(styx_moe *m);

#ifdef __cplusplus
}
#endif
#endif
