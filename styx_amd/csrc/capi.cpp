// capi.cpp -- C ABI: device, buffers, transfers and the hot-path ops.
// (crates/vk-backend/src/lib.rs replacement; see include/styx_hip.h)
#include <cmath>
#include <cstring>
#include <mutex>
#include <vector>
#include <string>

#include "kernels.h"
#include "runtime.h"

namespace styx {

static thread_local std::string t_err = "";

int fail(int status, const std::string &msg)
{
    t_err = msg;
    return status;
}

int hip_fail(hipError_t e, const char *what)
{
    t_err = std::string(what) + ": " + hipGetErrorName(e) + " (" + hipGetErrorString(e) + ")";
    return e == hipErrorOutOfMemory ? STYX_E_OOM : STYX_E_HIP;
}

void clear_error() { t_err.clear(); }

// Chunk partials of styx_op_attn_decode_noalloc: a static device array, so
// that entry point allocates nothing.  Each GPU holds its own copy for the
// life of the process.  In host code `scratch` only names the symbol; its
// device address on each GPU comes from hipGetSymbolAddress (noalloc_scratch).
static __device__ __align__(256) float scratch[STYX_NOALLOC_ATTN_PART_FLOATS];

// Device address of this GPU's copy of `scratch`, looked up once per device
// with that device current (the caller has set it).
static int noalloc_scratch(int device, float **out)
{
    static std::mutex mu;
    static std::vector<float *> addr;
    std::lock_guard<std::mutex> lock(mu);
    if ((int)addr.size() <= device) addr.resize(device + 1, nullptr);
    if (!addr[device]) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) return hip_fail(e, "hipGetSymbolAddress(scratch)");
        addr[device] = (float *)p;
    }
    *out = addr[device];
    return STYX_OK;
}

static void gpu_destroy(styx_gpu *g)
{
    hipSetDevice(g->device);
    hipStreamSynchronize(g->stream);
    hipStreamDestroy(g->stream);
    if (g->xq_scratch) hipFree(g->xq_scratch);
    if (g->partial_scratch) hipFree(g->partial_scratch);
    if (g->fused_scalars) hipFree(g->fused_scalars);
    if (g->fused_pt) hipFree(g->fused_pt);
    delete g;
}

void gpu_release(styx_gpu *g)
{
    if (--g->live_children == 0 && g->closed) gpu_destroy(g);
}

}  // namespace styx

using namespace styx;

extern "C" {

const char *styx_last_error(void) { return t_err.c_str(); }

// ------------------------------------------------------------- device ----
int styx_gpu_new(int device, styx_gpu **out)
{
    if (!out) return fail(STYX_E_INVALID, "styx_gpu_new: out is NULL");
    int n = 0;
    STYX_HIP(hipGetDeviceCount(&n));
    if (device < 0 || device >= n)
        return fail(STYX_E_INVALID, "styx_gpu_new: no HIP device " + std::to_string(device));
    STYX_HIP(hipSetDevice(device));
    hipDeviceProp_t p;
    STYX_HIP(hipGetDeviceProperties(&p, device));
    if (std::strncmp(p.gcnArchName, "gfx950", 6) != 0)
        return fail(STYX_E_UNSUPPORTED,
                    std::string("styx_gpu_new: built for gfx950, device is ") + p.gcnArchName);
    styx_gpu *g = new styx_gpu();
    g->device = device;
    g->name = p.name;
    g->hbm = p.totalGlobalMem;
    hipError_t e = hipStreamCreateWithFlags(&g->stream, hipStreamNonBlocking);
    if (e != hipSuccess) {
        delete g;
        return hip_fail(e, "hipStreamCreateWithFlags");
    }
    if (int r = noalloc_scratch(device, &g->noalloc_part)) {
        hipStreamDestroy(g->stream);
        delete g;
        return r;
    }
    g->partial_bytes = sizeof(float) * MAX_TOPK * XQ_MAX;
    e = hipMalloc(&g->xq_scratch, xq_bytes(XQ_MAX));
    if (e == hipSuccess) e = hipMalloc(&g->partial_scratch, g->partial_bytes);
    if (e == hipSuccess) e = hipMalloc(&g->fused_scalars, 256);
    if (e == hipSuccess) e = hipMemset(g->fused_scalars, 0, 256);
    if (e == hipSuccess) e = hipMalloc(&g->fused_pt, sizeof(uint32_t) * styx_gpu::FUSED_PT_MAX);
    if (e != hipSuccess) {
        if (g->xq_scratch) hipFree(g->xq_scratch);
        if (g->partial_scratch) hipFree(g->partial_scratch);
        if (g->fused_scalars) hipFree(g->fused_scalars);
        if (g->fused_pt) hipFree(g->fused_pt);
        hipStreamDestroy(g->stream);
        delete g;
        return hip_fail(e, "hipMalloc(op scratch)");
    }
    *out = g;
    return STYX_OK;
}

void styx_gpu_free(styx_gpu *g)
{
    if (!g || g->closed) return;
    // children (buffers, kernels, batches, models) keep the device alive;
    // it is released with the last of them
    g->closed = true;
    if (g->live_children == 0) gpu_destroy(g);
}

uint64_t styx_gpu_hbm_bytes(const styx_gpu *g) { return g ? g->hbm : 0; }
const char *styx_gpu_name(const styx_gpu *g) { return g ? g->name.c_str() : ""; }

int styx_gpu_sync(styx_gpu *g)
{
    if (!g) return fail(STYX_E_INVALID, "styx_gpu_sync: NULL gpu");
    STYX_HIP(hipStreamSynchronize(g->stream));
    return STYX_OK;
}

// ------------------------------------------------------------ buffers ----
int styx_buf_new(styx_gpu *g, uint64_t bytes, int kind, styx_buf **out)
{
    if (!g || !out || bytes == 0) return fail(STYX_E_INVALID, "styx_buf_new: bad argument");
    STYX_HIP(hipSetDevice(g->device));
    void *p = nullptr;
    if (kind == STYX_BUF_DEVICE) {
        STYX_HIP(hipMalloc(&p, bytes));
    } else if (kind == STYX_BUF_HOST_PINNED) {
        STYX_HIP(hipHostMalloc(&p, bytes, hipHostMallocMapped | hipHostMallocPortable));
    } else {
        return fail(STYX_E_INVALID, "styx_buf_new: unknown kind");
    }
    styx_buf *b = new styx_buf();
    b->gpu = g;
    b->ptr = p;
    b->size = bytes;
    b->kind = kind;
    if (kind == STYX_BUF_HOST_PINNED) {
        b->host = p;
        void *dp = nullptr;
        if (hipHostGetDevicePointer(&dp, p, 0) == hipSuccess && dp) b->ptr = dp;
    }
    g->live_children++;
    *out = b;
    return STYX_OK;
}

void styx_buf_free(styx_buf *b)
{
    if (!b) return;
    hipSetDevice(b->gpu->device);
    hipStreamSynchronize(b->gpu->stream);
    if (b->kind == STYX_BUF_DEVICE)
        hipFree(b->ptr);
    else
        hipHostFree(b->host ? b->host : b->ptr);
    styx_gpu *g = b->gpu;
    delete b;
    gpu_release(g);
}

uint64_t styx_buf_size(const styx_buf *b) { return b ? b->size : 0; }
void *styx_buf_device_ptr(const styx_buf *b) { return b ? b->ptr : nullptr; }

static int range_ok(const styx_buf *b, uint64_t off, uint64_t n, const char *who)
{
    if (!b) return fail(STYX_E_INVALID, std::string(who) + ": NULL buffer");
    if (off > b->size || n > b->size - off)
        return fail(STYX_E_INVALID, std::string(who) + ": range [" + std::to_string(off) + ", +" +
                                        std::to_string(n) + ") outside buffer of " +
                                        std::to_string(b->size) + " bytes");
    return STYX_OK;
}

int styx_upload(styx_gpu *g, styx_buf *dst, uint64_t off, const void *src, uint64_t n)
{
    if (int r = range_ok(dst, off, n, "styx_upload")) return r;
    if (!g || (!src && n)) return fail(STYX_E_INVALID, "styx_upload: bad argument");
    STYX_HIP(hipMemcpyAsync((char *)dst->ptr + off, src, n, hipMemcpyHostToDevice, g->stream));
    STYX_HIP(hipStreamSynchronize(g->stream));
    return STYX_OK;
}

int styx_download(styx_gpu *g, const styx_buf *src, uint64_t off, void *dst, uint64_t n)
{
    if (int r = range_ok(src, off, n, "styx_download")) return r;
    if (!g || (!dst && n)) return fail(STYX_E_INVALID, "styx_download: bad argument");
    STYX_HIP(hipMemcpyAsync(dst, (const char *)src->ptr + off, n, hipMemcpyDeviceToHost, g->stream));
    STYX_HIP(hipStreamSynchronize(g->stream));
    return STYX_OK;
}

int styx_copy_region(styx_gpu *g, const styx_buf *src, uint64_t soff, styx_buf *dst,
                     uint64_t doff, uint64_t n)
{
    if (int r = range_ok(src, soff, n, "styx_copy_region(src)")) return r;
    if (int r = range_ok(dst, doff, n, "styx_copy_region(dst)")) return r;
    if (!g) return fail(STYX_E_INVALID, "styx_copy_region: NULL gpu");
    STYX_HIP(hipMemcpyAsync((char *)dst->ptr + doff, (const char *)src->ptr + soff, n,
                            hipMemcpyDefault, g->stream));
    STYX_HIP(hipStreamSynchronize(g->stream));
    return STYX_OK;
}

// ---------------------------------------------------------------- ops ----
#define OP_GPU(g)                                                         \
    do {                                                                  \
        if (!(g)) return fail(STYX_E_INVALID, "NULL gpu");                \
    } while (0)
#define OP_RUN(expr, what)                                                \
    do {                                                                  \
        hipError_t _e = (expr);                                           \
        if (_e == hipErrorInvalidValue)                                   \
            return fail(STYX_E_INVALID, std::string(what) + ": unsupported shape or type"); \
        if (_e != hipSuccess) return hip_fail(_e, what);                  \
    } while (0)

int styx_op_to_split(styx_gpu *g, int type, const void *src, void *dst, int64_t nblocks,
                     int64_t nmat)
{
    OP_GPU(g);
    OP_RUN(launch_to_split(g->stream, type, (const uint8_t *)src, (uint8_t *)dst, nblocks, nmat),
           "styx_op_to_split");
    return STYX_OK;
}

int styx_op_from_split(styx_gpu *g, int type, const void *src, void *dst, int64_t nblocks,
                       int64_t nmat)
{
    OP_GPU(g);
    OP_RUN(launch_from_split(g->stream, type, (const uint8_t *)src, (uint8_t *)dst, nblocks, nmat),
           "styx_op_from_split");
    return STYX_OK;
}

int styx_op_dequant_rows(styx_gpu *g, int type, const void *w, int64_t nrows_total, int ncols,
                         int64_t r0, int64_t nrows, float *out)
{
    OP_GPU(g);
    if (r0 < 0 || nrows < 0 || r0 + nrows > nrows_total)
        return fail(STYX_E_INVALID, "styx_op_dequant_rows: row range outside matrix");
    OP_RUN(launch_dequant_rows(g->stream, type, (const uint8_t *)w, nrows_total, ncols, r0, nrows,
                               out),
           "styx_op_dequant_rows");
    return STYX_OK;
}

int styx_op_matvec(styx_gpu *g, int type, const void *w, int nrows, int ncols, const float *x,
                   const float *norm_w, float eps, float *y, int add)
{
    OP_GPU(g);
    if (nrows < 1 || ncols < 32 || ncols % 32 || ncols > XQ_MAX)
        return fail(STYX_E_INVALID, "styx_op_matvec: bad shape");
    if (!w || !x || !y) return fail(STYX_E_INVALID, "styx_op_matvec: NULL pointer");
    const Xq q = xq_at(g->xq_scratch, ncols);
    OP_RUN(launch_xq(g->stream, x, nullptr, norm_w, eps, ncols, q, nullptr), "styx_op_matvec");
    DenseSeg s{(const uint8_t *)w, y, nrows};
    OP_RUN(launch_dense(g->stream, type, ncols, &s, 1, q, add), "styx_op_matvec");
    return STYX_OK;
}

int styx_op_router_topk(styx_gpu *g, const float *x, const float *norm_w, float eps,
                        const float *W, const float *bias, int E, int H, int k, int renorm,
                        const uint32_t *remap, const uint32_t *pmap, int arena_mode, int layer,
                        float *xn, float *logits, float *weights, int32_t *ids)
{
    OP_GPU(g);
    if (!x || !norm_w || !W || !xn || !logits || !weights || !ids)
        return fail(STYX_E_INVALID, "styx_op_router_topk: NULL pointer");
    RouterArgs a{};
    a.x = x;
    a.norm_w = norm_w;
    a.W = W;
    a.bias = bias;
    a.eps = eps;
    a.xn = xn;
    a.logits = logits;
    a.wts = weights;
    a.ids = ids;
    a.remap = remap;
    a.pmap = pmap;
    a.E = E;
    a.H = H;
    a.k = k;
    a.renorm = renorm;
    a.arena_mode = arena_mode;
    a.layer = layer;
    OP_RUN(launch_router_topk(g->stream, a), "styx_op_router_topk");
    return STYX_OK;
}

int styx_op_topk_softmax(styx_gpu *g, const float *logits, int n, int k, int renorm,
                         const uint32_t *remap, const uint32_t *pmap, int arena_mode, int layer,
                         float *weights, int32_t *ids)
{
    OP_GPU(g);
    OP_RUN(launch_topk_softmax(g->stream, logits, n, k, renorm, remap, pmap, arena_mode, layer,
                               weights, ids),
           "styx_op_topk_softmax");
    return STYX_OK;
}

static ExpSrc to_src(const styx_expert_src *s)
{
    ExpSrc e{};
    if (!s) return e;
    e.hot = (const uint8_t *)s->hot;
    e.hot_slab = s->hot_slab;
    e.arena = (const uint8_t *)s->arena;
    e.arena_slab = s->arena_slab;
    e.gtt = (const uint8_t *)s->host;
    e.gtt_slab = s->host_slab;
    return e;
}

int styx_op_moe_gate_up(styx_gpu *g, int tg, int tu, const styx_expert_src *gate,
                        const styx_expert_src *up, const int32_t *ids, const float *xn, float *gu,
                        int H, int F, int k)
{
    OP_GPU(g);
    if (!gate || !up || !ids || !xn || !gu || k < 1 || k > 16 || F < 1)
        return fail(STYX_E_INVALID, "styx_op_moe_gate_up: bad argument");
    if (H < 32 || H % 32 || H > XQ_MAX) return fail(STYX_E_INVALID, "styx_op_moe_gate_up: bad H");
    const Xq q = xq_at(g->xq_scratch, H);
    OP_RUN(launch_xq(g->stream, xn, nullptr, nullptr, 0.0f, H, q, nullptr), "styx_op_moe_gate_up");
    OP_RUN(launch_moe_gate_up(g->stream, tg, tu, to_src(gate), to_src(up), ids, nullptr, q, gu, H,
                              F, k),
           "styx_op_moe_gate_up");
    return STYX_OK;
}

int styx_op_moe_down_reduce(styx_gpu *g, int td, const styx_expert_src *down, const int32_t *ids,
                            const float *weights, const float *gu, float *x, int H, int F, int k)
{
    OP_GPU(g);
    if (!down || !ids || !weights || !gu || !x || k < 1 || k > 16)
        return fail(STYX_E_INVALID, "styx_op_moe_down_reduce: bad argument");
    if (F > XQ_MAX / 2) return fail(STYX_E_INVALID, "styx_op_moe_down_reduce: F > 8192");
    if (H < 32 || H % 32 || H > XQ_MAX)
        return fail(STYX_E_INVALID, "styx_op_moe_down_reduce: bad H");
    // gu [2][k][F] -> per-slot down rows into a scratch of k x H floats
    // held by the gpu (serialised with every other op on its stream)
    if ((size_t)k * H * 4 > g->partial_bytes)
        return fail(STYX_E_INVALID, "styx_op_moe_down_reduce: k * H too large");
    float *partial = (float *)g->partial_scratch;
    OP_RUN(launch_moe_down(g->stream, td, to_src(down), ids, gu, partial, H, F, k),
           "styx_op_moe_down_reduce");
    ReduceArgs a{};
    a.partial = partial;
    a.k = k;
    a.H = H;
    a.wts = weights;
    a.x = x;
    OP_RUN(launch_reduce_rows(g->stream, a), "styx_op_moe_down_reduce");
    return STYX_OK;
}

int styx_op_attn_decode(styx_gpu *g, const float *q, const float *k, const float *v,
                        const float *q_norm, const float *k_norm, float eps,
                        const double *rope, float *kpool, float *vpool,
                        const int32_t *page_table, int page_tokens, const int32_t *pos,
                        float *out, float *part, int nh, int nkv, int hd, int chunk,
                        int max_chunks, float scale)
{
    OP_GPU(g);
    AttnArgs a{};
    a.q = q;
    a.k = k;
    a.v = v;
    a.q_norm = q_norm;
    a.k_norm = k_norm;
    a.eps = eps;
    a.rope = (const double2 *)rope;
    a.kpool = kpool;
    a.vpool = vpool;
    a.page_table = page_table;
    a.page_tokens = page_tokens;
    a.pos = pos;
    a.out = out;
    a.part = part;
    a.nh = nh;
    a.nkv = nkv;
    a.hd = hd;
    a.chunk = chunk;
    a.max_chunks = max_chunks;
    a.scale = scale;
    OP_RUN(launch_attn_decode(g->stream, a), "styx_op_attn_decode");
    return STYX_OK;
}

int styx_op_attn_decode_noalloc(styx_gpu *g, const float *q, const float *k, const float *v,
                                const float *q_norm, const float *k_norm, float eps,
                                const double *rope, float *kpool, float *vpool,
                                const int32_t *page_table, int page_tokens, const int32_t *pos,
                                float *out, int nh, int nkv, int hd, int chunk, int max_chunks,
                                float scale)
{
    OP_GPU(g);
    const int64_t need = styx_op_attn_part_floats(nh, nkv, hd, max_chunks);
    if (need <= 0 || max_chunks < 1)
        return fail(STYX_E_INVALID, "styx_op_attn_decode_noalloc: bad head counts or max_chunks");
    if (need > (int64_t)STYX_NOALLOC_ATTN_PART_FLOATS)
        return fail(STYX_E_INVALID,
                    "styx_op_attn_decode_noalloc: partials of " + std::to_string(need) +
                        " floats (nh, nkv, hd, max_chunks) exceed the static scratch of " +
                        std::to_string((long long)STYX_NOALLOC_ATTN_PART_FLOATS) +
                        " floats; lower max_chunks or use styx_op_attn_decode");
    // the shared array needs no clearing between calls: the combine masks
    // every chunk past the context (its first batch of loads may read such
    // stale words before the position is known, and discards them), and
    // every chunk inside the context is written by the same launch first
    return styx_op_attn_decode(g, q, k, v, q_norm, k_norm, eps, rope, kpool, vpool, page_table,
                               page_tokens, pos, out, g->noalloc_part, nh, nkv, hd, chunk,
                               max_chunks, scale);
}

void styx_rope_table(float base, int hd, int n_pos, double *out)
{
    // theta_scale = base^(-2/hd), theta = pos * theta_scale^i, all in f64
    // (crates/vk-backend/tests/ops2.rs:426-442)
    if (!out || hd < 2 || n_pos < 1) return;
    const double ts = std::pow((double)base, -2.0 / (double)hd);
    std::vector<double> invf(hd / 2);
    for (int i = 0; i < hd / 2; i++) invf[i] = std::pow(ts, (double)i);
    for (int p = 0; p < n_pos; p++)
        for (int i = 0; i < hd / 2; i++) {
            const double th = (double)p * invf[i];
            out[((size_t)p * (hd / 2) + i) * 2] = std::cos(th);
            out[((size_t)p * (hd / 2) + i) * 2 + 1] = std::sin(th);
        }
}

int64_t styx_op_attn_part_floats(int nh, int nkv, int hd, int max_chunks)
{
    if (nkv < 1) return 0;
    return (int64_t)nkv * max_chunks * (nh / nkv) * (hd + 2);
}

int styx_op_gather_slabs(styx_gpu *g, const void *const src[3], const int64_t src_slab[3],
                         void *const dst[3], const int64_t dst_slab[3], const int32_t *ids, int k,
                         int layer)
{
    OP_GPU(g);
    const uint8_t *s[3] = {(const uint8_t *)src[0], (const uint8_t *)src[1],
                           (const uint8_t *)src[2]};
    uint8_t *d[3] = {(uint8_t *)dst[0], (uint8_t *)dst[1], (uint8_t *)dst[2]};
    OP_RUN(launch_gather_list(g->stream, s, src_slab, d, dst_slab, ids, k, layer),
           "styx_op_gather_slabs");
    return STYX_OK;
}

int styx_op_argmax(styx_gpu *g, const float *v, int n, uint32_t *out, float *sv, uint32_t *si)
{
    OP_GPU(g);
    OP_RUN(launch_argmax(g->stream, v, n, out, sv, si, nullptr, 0, nullptr), "styx_op_argmax");
    return STYX_OK;
}

int styx_op_read_probe(styx_gpu *g, const void *p, int64_t bytes, uint32_t *out, int grid)
{
    OP_GPU(g);
    if (!p || !out) return fail(STYX_E_INVALID, "styx_op_read_probe: NULL pointer");
    OP_RUN(launch_read_probe(g->stream, p, bytes, out, grid), "styx_op_read_probe");
    return STYX_OK;
}

int styx_op_gen_quant(styx_gpu *g, int type, uint64_t seed, float sigma, void *dst, int64_t n)
{
    OP_GPU(g);
    OP_RUN(launch_gen_quant(g->stream, type, seed, sigma, (uint8_t *)dst, n), "styx_op_gen_quant");
    return STYX_OK;
}

int styx_op_gen_f32(styx_gpu *g, uint64_t seed, float mean, float sigma, float *dst, int64_t n)
{
    OP_GPU(g);
    OP_RUN(launch_gen_f32(g->stream, seed, mean, sigma, dst, n), "styx_op_gen_f32");
    return STYX_OK;
}

}  // extern "C"
