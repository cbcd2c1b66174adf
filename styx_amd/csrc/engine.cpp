// engine.cpp -- C++ port of the qwen3moe MoeModel of crates/model/src/moe.rs
// on the gfx950 kernels: load (GGUF or seeded synthetic), placement and
// residency, per-token decode (one HIP graph per token), greedy generation,
// telemetry.
//
// Per layer the token runs 6 kernels (7 with an in-stream slab gather):
//   qkv matvec (+attn_norm) | attention (+q/k norm, rope, KV append) |
//   o-proj (+residual) | router+topk (+ffn_norm) | expert gate/up |
//   expert down (+swiglu, +weighted reduce into the residual)
// against 21 dispatches per layer in the reference (moe.rs:1845-2062).
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <functional>
#include <map>
#include <memory>
#include <numeric>
#include <sstream>
#include <string>
#include <vector>

#include "gguf.h"
#include "kernels.h"
#include "runtime.h"

namespace styx {
}  // namespace styx

using namespace styx;

namespace {

constexpr int KV_PAGE_TOKENS = 512;  // moe.rs:501-503

#define CK(call)                                                          \
    do {                                                                  \
        hipError_t _e = (call);                                           \
        if (_e == hipErrorInvalidValue)                                   \
            return fail(STYX_E_INVALID, std::string(#call) + ": unsupported shape or type"); \
        if (_e != hipSuccess) return hip_fail(_e, #call);                 \
    } while (0)

uint64_t fnv1a64(const std::string &s)
{
    uint64_t h = 0xcbf29ce484222325ull;
    for (unsigned char c : s) {
        h ^= c;
        h *= 0x100000001b3ull;
    }
    return h;
}

uint64_t splitmix(uint64_t &s)
{
    uint64_t z = (s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

struct Mat {
    std::string name;
    int type = 0;
    int rows = 0, cols = 0;   // per expert for expert tensors
    int nmat = 1;             // experts
    int64_t slab = 0;         // bytes per matrix
    uint8_t *dev = nullptr;   // HBM copy (split layout), or null
    uint8_t *host = nullptr;  // pinned host copy (split layout), or null
    uint8_t *host_dev = nullptr;
    uint8_t *hot = nullptr;   // hot slabs in HBM (host-resident experts)
    std::vector<int64_t> gguf_dims;
    int64_t bytes() const { return slab * nmat; }
};

struct Layer {
    float *attn_norm = nullptr, *q_norm = nullptr, *k_norm = nullptr, *ffn_norm = nullptr;
    float *router = nullptr, *router_bias = nullptr, *gate_inp_sh = nullptr;
    Mat wq, wk, wv, wo, gate, up, down, gsh, ush, dsh;
    bool host_experts = false;
    std::vector<uint32_t> remap;       // expert -> hot slot or SKIP
    uint32_t *remap_dev = nullptr;
    std::vector<uint32_t> slot_experts;
    std::vector<uint64_t> hits;
};

struct KStat {
    std::string name;
    uint64_t launches = 0;
    double ms = 0, bytes = 0;
};

}  // namespace

// Attention variants of a token (styx_moe::attn_mode).
enum AttnMode { AT_SOLO = 0, AT_MERGE = 1, AT_COMBINE = 2 };

struct styx_moe {
    styx_gpu *gpu = nullptr;
    styx_moe_opts opts{};
    // hparams
    int L = 0, H = 0, nh = 0, nkv = 0, hd = 0, E = 0, K = 0, F = 0, Fsh = 0, V = 0, n_ctx = 0;
    float eps = 1e-6f, rope_base = 10000.0f;
    int norm_topk = 1;
    uint64_t slab_bytes = 0, exp_hbm = 0, exp_host = 0;
    std::vector<Layer> layers;
    Mat embd, head;
    float *out_norm = nullptr;
    // f32 tensors for export: name -> (device ptr, count, dims)
    struct F32T {
        std::string name;
        float *p;
        int64_t n;
        std::vector<int64_t> dims;
    };
    std::vector<F32T> f32s;
    // activations / state
    float *x = nullptr, *q = nullptr, *kk = nullptr, *vv = nullptr, *attn = nullptr,
          *xn = nullptr, *rlog = nullptr, *wts = nullptr, *gu = nullptr, *partial = nullptr,
          *logits = nullptr, *hidden = nullptr, *sh_g = nullptr, *sh_u = nullptr, *sh_y = nullptr,
          *attn_part = nullptr;
    Xq xq_a{}, xq_o{}, xq_f{}, xq_sh{};  // limbs: layer input, attention out, ffn input, shexp hidden
    float *ss_a = nullptr;                // partial sums of x^2 behind xq_a (per 256 rows)
    int32_t *ids = nullptr, *d_pos = nullptr;
    uint32_t *d_tok = nullptr, *hist = nullptr;
    // running argmax of the LM head (argmax_key), cleared by its reader
    unsigned long long *am_word = nullptr;
    uint32_t *h_stage = nullptr;  // pinned: tok, pos
    // KV
    float *kpool = nullptr, *vpool = nullptr;
    // pages hold each kv head's rows together ([nkv][page_tokens][hd]): an
    // attention workgroup's rows are contiguous (about 1% faster at a 32K
    // context than the reference's [page_tokens][kv_dim] rows)
    int kv_head_major = 1;
    int32_t *d_pt = nullptr;
    std::vector<int32_t> h_pt;
    int pages_per_layer = 0, next_page = 0, chunk = 64, max_chunks = 1;
    // contexts of up to this many tokens run as one chunk per kv head on the
    // matrix-core attention kernel (AT_SOLO; head_dim 128, 4-16 query heads
    // per kv head): its four waves take one 16-token tile each at once and
    // the chunk's workgroup writes the output itself, with no exchange
    // between chunks.  Measured on configs[1] at up to 57 tokens: 497
    // against 474 tok/s with 16-token chunks merged in-kernel.  Past 64
    // tokens the waves would walk tiles one after another, slower than
    // splitting the context.
    int attn_solo_max = 64;
    double *rope = nullptr;  // [n_ctx][hd/2] (cos, sin)
    double *rope_cur = nullptr;  // [hd/2] (cos, sin) of the token's position (k_embed)
    // fused MoE block (moe_block.hip): tagged exchange buffers, ticket,
    // abort flag; mb_nwg = its grid (0: the separate kernels run), -1 until
    // first sized
    uint64_t *t_lg = nullptr, *t_gu = nullptr, *t_part = nullptr;
    // attention with the chunk partials merged inside its kernel: tagged
    // partials and the launch's ticket counters
    uint64_t *at_part = nullptr;
    unsigned long long *at_tickets = nullptr;
    unsigned long long *mb_ticket = nullptr;
    int *mb_abort = nullptr;
    // qkv_fold[l]: layer l's q/k/v matvec runs in the tail of layer l-1's
    // fused MoE block, from the tagged limbs in t_xq
    std::vector<char> qkv_fold;
    uint64_t *t_xq = nullptr;
    int mb_nwg = -1;
    uint64_t *mb_trace = nullptr;  // [L][mb_nwg][16] phase stamps of the last timed token
    uint64_t *at_trace = nullptr;  // [L][max_chunks * nkv][AT_TRACE] attention phase stamps
    // arena
    uint8_t *arena[3] = {nullptr, nullptr, nullptr};
    int64_t arena_slab[3] = {0, 0, 0};
    bool any_host = false;
    // graphs
    // [short context: attention partials merged in-kernel, long: combine kernel]
    // one graph per attention mode (AT_SOLO, AT_MERGE, AT_COMBINE), forward
    // and generate
    hipGraphExec_t g_fwd[3] = {nullptr, nullptr, nullptr}, g_gen[3] = {nullptr, nullptr, nullptr};
    // arena placement: the cold-slab gather runs on a second stream (same
    // priority), forked after the router and joined before the cold slots'
    // expert kernels, so that it overlaps the hot slots' gate/up and down
    hipStream_t st_copy = nullptr;
    hipEvent_t ev_fork = nullptr, ev_join = nullptr;
    int n_past = 0;
    uint64_t repin_swaps = 0;
    std::vector<void *> dev_allocs, host_allocs;
    // timing
    std::vector<KStat> stats;
    std::vector<std::pair<int, std::pair<hipEvent_t, hipEvent_t>>> pending;
    std::vector<hipEvent_t> ev_pool;
    size_t ev_next = 0;
    std::string stage_only;  // enqueue only this stage's launches (stage timing)

    ~styx_moe();
    int alloc(void **p, size_t n);
    int alloc_host(void **p, size_t n);
    template <typename T> int dalloc(T **p, size_t count)
    {
        return alloc((void **)p, sizeof(T) * count);
    }
    int setup_runtime();
    int size_moe_block();
    int check_abort();
    int fall_back_unfused();
    int fallbacks = 0;
    uint32_t *tok_save = nullptr;  // the pending token at a decode's start
    void queue_abort_read();
    int place_experts(const std::vector<std::vector<std::pair<uint32_t, uint64_t>>> *hist);
    int enqueue_token(bool gen, int attn_mode);
    int run_token(bool gen);
    bool attn_merge_in_kernel(int n_t) const;
    int attn_mode(int n_t) const;
    int ensure_pages(int upto_pos);
    int build_graphs();
    int maybe_repin();
    std::string broken;  // set when the model's device state can no longer be trusted
    int stat_id(const char *name);
    hipEvent_t ev();
    int collect_stats();
};

styx_moe::~styx_moe()
{
    if (gpu) {
        hipSetDevice(gpu->device);
        hipStreamSynchronize(gpu->stream);
    }
    for (int i = 0; i < 3; i++) {
        if (g_fwd[i]) hipGraphExecDestroy(g_fwd[i]);
        if (g_gen[i]) hipGraphExecDestroy(g_gen[i]);
    }
    for (auto e : ev_pool) hipEventDestroy(e);
    if (ev_fork) hipEventDestroy(ev_fork);
    if (ev_join) hipEventDestroy(ev_join);
    if (st_copy) {
        hipStreamSynchronize(st_copy);
        hipStreamDestroy(st_copy);
    }
    for (void *p : dev_allocs) hipFree(p);
    for (void *p : host_allocs) hipHostFree(p);
    if (gpu) gpu_release(gpu);
}

int styx_moe::alloc(void **p, size_t n)
{
    *p = nullptr;
    if (n == 0) n = 16;
    hipError_t e = hipMalloc(p, n);
    if (e != hipSuccess) return hip_fail(e, ("hipMalloc(" + std::to_string(n) + ")").c_str());
    dev_allocs.push_back(*p);
    return STYX_OK;
}

int styx_moe::alloc_host(void **p, size_t n)
{
    *p = nullptr;
    hipError_t e = hipHostMalloc(p, n, hipHostMallocMapped | hipHostMallocPortable);
    if (e != hipSuccess) return hip_fail(e, ("hipHostMalloc(" + std::to_string(n) + ")").c_str());
    host_allocs.push_back(*p);
    return STYX_OK;
}

hipEvent_t styx_moe::ev()
{
    if (ev_next == ev_pool.size()) {
        hipEvent_t e;
        hipEventCreate(&e);
        ev_pool.push_back(e);
    }
    return ev_pool[ev_next++];
}

int styx_moe::stat_id(const char *name)
{
    for (size_t i = 0; i < stats.size(); i++)
        if (stats[i].name == name) return (int)i;
    stats.push_back(KStat{name, 0, 0, 0});
    return (int)stats.size() - 1;
}

int styx_moe::collect_stats()
{
    if (pending.empty()) return STYX_OK;
    STYX_HIP(hipStreamSynchronize(gpu->stream));
    for (auto &p : pending) {
        float ms = 0;
        STYX_HIP(hipEventElapsedTime(&ms, p.second.first, p.second.second));
        stats[p.first].ms += ms;
        stats[p.first].launches++;
    }
    pending.clear();
    ev_next = 0;
    return STYX_OK;
}

// ------------------------------------------------------------ runtime ----
int styx_moe::setup_runtime()
{
    const int kv_dim = nkv * hd, q_dim = nh * hd;
    if (n_ctx <= 0) n_ctx = 4096;
    STYX_HIP(hipSetDevice(gpu->device));
    if (int r = dalloc(&x, H)) return r;
    if (int r = dalloc(&xn, H)) return r;
    if (int r = dalloc(&q, q_dim)) return r;
    if (int r = dalloc(&kk, kv_dim)) return r;
    if (int r = dalloc(&vv, kv_dim)) return r;
    if (int r = dalloc(&attn, q_dim)) return r;
    if (int r = dalloc(&rlog, E)) return r;
    if (int r = dalloc(&wts, (size_t)L * 16)) return r;
    if (int r = dalloc(&ids, (size_t)L * 64)) return r;
    // one more slot than k: the shared expert when it runs fused
    if (int r = dalloc(&gu, (size_t)2 * (K + 1) * F)) return r;
    if (int r = dalloc(&partial, (size_t)(K + 1) * H)) return r;
    if (int r = dalloc(&logits, V)) return r;
    if (int r = dalloc(&hidden, (size_t)(L + 1) * H)) return r;
    if (int r = dalloc(&am_word, 1)) return r;
    STYX_HIP(hipMemsetAsync(am_word, 0, sizeof(unsigned long long), gpu->stream));
    if (int r = dalloc(&d_pos, 1)) return r;
    if (int r = dalloc(&d_tok, 1)) return r;
    if (int r = dalloc(&hist, (size_t)n_ctx + 1)) return r;
    if (int r = dalloc(&ss_a, (size_t)H / 32)) return r;
    uint8_t *xqb = nullptr;
    const size_t xa = (xq_bytes(H) + 255) & ~(size_t)255, xo = (xq_bytes(q_dim) + 255) & ~(size_t)255;
    const size_t xs = (xq_bytes(std::max(Fsh, 32)) + 255) & ~(size_t)255;
    if (int r = dalloc(&xqb, 2 * xa + xo + xs)) return r;
    xq_a = xq_at(xqb, H);
    xq_f = xq_at(xqb + xa, H);
    xq_o = xq_at(xqb + 2 * xa, q_dim);
    if (Fsh > 0) xq_sh = xq_at(xqb + 2 * xa + xo, Fsh);
    if (Fsh > 0) {
        if (int r = dalloc(&sh_g, Fsh)) return r;
        if (int r = dalloc(&sh_u, Fsh)) return r;
        if (int r = dalloc(&sh_y, H)) return r;
    }
    STYX_HIP(hipMemsetAsync(ids, 0xFF, sizeof(int32_t) * L * 64, gpu->stream));
    STYX_HIP(hipMemsetAsync(d_pos, 0, 4, gpu->stream));
    STYX_HIP(hipMemsetAsync(d_tok, 0, 4, gpu->stream));
    void *hs;
    if (int r = alloc_host(&hs, 64)) return r;
    h_stage = (uint32_t *)hs;
    std::memset(h_stage, 0, 64);
    // paged KV: pool sized for n_ctx on every layer, pages handed out lazily
    pages_per_layer = (n_ctx + KV_PAGE_TOKENS - 1) / KV_PAGE_TOKENS;
    const size_t pool = (size_t)L * pages_per_layer * KV_PAGE_TOKENS * kv_dim;
    if (int r = dalloc(&kpool, pool)) return r;
    if (int r = dalloc(&vpool, pool)) return r;
    if (int r = dalloc(&d_pt, (size_t)L * pages_per_layer)) return r;
    h_pt.assign((size_t)L * pages_per_layer, -1);
    STYX_HIP(hipMemsetAsync(d_pt, 0, sizeof(int32_t) * L * pages_per_layer, gpu->stream));
    next_page = 0;
    // attention split: chunks of at least 16 tokens (one tile per wave when
    // the waves split heads); at most ~768 workgroups in all (one round of
    // 4-wave workgroups at 3 waves per SIMD on 256 CUs); the attention
    // kernels size the chunk from the live context
    chunk = 16;
    max_chunks = std::min((n_ctx + chunk - 1) / chunk, std::max(16, 768 / nkv));
    const int64_t pf = styx_op_attn_part_floats(nh, nkv, hd, max_chunks);
    if (int r = dalloc(&attn_part, (size_t)pf)) return r;
    if (int r = dalloc(&at_part, (size_t)pf)) return r;
    if (int r = dalloc(&at_tickets, 64 * 16)) return r;
    if (int r = dalloc(&at_trace, (size_t)L * max_chunks * nkv * AT_TRACE)) return r;
    STYX_HIP(hipMemsetAsync(at_trace, 0, sizeof(uint64_t) * L * max_chunks * nkv * AT_TRACE,
                            gpu->stream));
    STYX_HIP(hipMemsetAsync(at_part, 0, sizeof(uint64_t) * pf, gpu->stream));
    STYX_HIP(hipMemsetAsync(at_tickets, 0, sizeof(unsigned long long) * 64 * 16, gpu->stream));
    // tagged exchange of the fused MoE block: zero once (tag 0 is never a
    // launch's), never cleared again
    if (int r = dalloc(&t_lg, E)) return r;
    if (int r = dalloc(&t_gu, (size_t)(K + 1) * F)) return r;
    if (int r = dalloc(&t_part, (size_t)(K + 1) * H)) return r;
    if (int r = dalloc(&mb_ticket, 64 * 16)) return r;
    if (int r = dalloc(&mb_abort, 1)) return r;
    if (int r = dalloc(&tok_save, 1)) return r;
    STYX_HIP(hipMemsetAsync(t_lg, 0, sizeof(uint64_t) * E, gpu->stream));
    STYX_HIP(hipMemsetAsync(t_gu, 0, sizeof(uint64_t) * (K + 1) * F, gpu->stream));
    STYX_HIP(hipMemsetAsync(t_part, 0, sizeof(uint64_t) * (K + 1) * H, gpu->stream));
    STYX_HIP(hipMemsetAsync(mb_ticket, 0, sizeof(unsigned long long) * 64 * 16, gpu->stream));
    STYX_HIP(hipMemsetAsync(mb_abort, 0, sizeof(int), gpu->stream));
    // rope factors in f64 for every position of the context (ops2.rs:426-442)
    {
        std::vector<double> cs((size_t)n_ctx * hd);
        styx_rope_table(rope_base, hd, n_ctx, cs.data());
        if (int r = dalloc(&rope, cs.size())) return r;
        if (int r = dalloc(&rope_cur, (size_t)hd)) return r;
        STYX_HIP(hipMemcpyAsync(rope, cs.data(), sizeof(double) * cs.size(), hipMemcpyHostToDevice,
                                gpu->stream));
        STYX_HIP(hipStreamSynchronize(gpu->stream));
    }
    STYX_HIP(hipStreamSynchronize(gpu->stream));
    return STYX_OK;
}

int styx_moe::ensure_pages(int upto_pos)
{
    const int last = std::min(upto_pos, n_ctx - 1) / KV_PAGE_TOKENS;
    for (int l = 0; l < L; l++) {
        bool dirty = false;
        for (int p = 0; p <= last; p++) {
            int32_t &e = h_pt[(size_t)l * pages_per_layer + p];
            if (e < 0) {
                e = next_page++;
                dirty = true;
            }
        }
        if (dirty)
            STYX_HIP(hipMemcpyAsync(d_pt + (size_t)l * pages_per_layer,
                                    h_pt.data() + (size_t)l * pages_per_layer,
                                    sizeof(int32_t) * (last + 1), hipMemcpyHostToDevice,
                                    gpu->stream));
    }
    STYX_HIP(hipStreamSynchronize(gpu->stream));
    return STYX_OK;
}

// Which (layer, expert) slabs go to HBM under a byte budget
// (crates/model/src/moe.rs:774-813).  With a popularity histogram: rank all
// (layer, expert) entries by hits, descending (ties keep file order; the
// reference's sort_unstable leaves them unspecified), and take slabs until
// the next one does not fit.  Without one: whole layers in order.  Each
// layer's list comes back sorted, so a hot slot index is the rank of the
// expert id among that layer's hot experts.
static void plan_hot_experts(const std::vector<std::vector<std::pair<uint32_t, uint64_t>>> *hist,
                             int L, int E, const std::vector<uint64_t> &slab_cost,
                             const std::vector<uint64_t> &layer_cost, uint64_t budget,
                             std::vector<std::vector<uint32_t>> &hot)
{
    hot.assign(L, {});
    uint64_t left = budget;
    if (hist) {
        struct Ent { uint64_t hits; int layer; uint32_t e; };
        std::vector<Ent> ents;
        for (int l = 0; l < L && l < (int)hist->size(); l++)
            for (auto &p : (*hist)[l]) ents.push_back({p.second, l, p.first});
        std::stable_sort(ents.begin(), ents.end(),
                         [](const Ent &a, const Ent &b) { return a.hits > b.hits; });
        std::vector<std::vector<char>> seen(L, std::vector<char>(E, 0));
        for (auto &en : ents) {
            if (en.e >= (uint32_t)E || seen[en.layer][en.e]) continue;
            if (left < slab_cost[en.layer]) break;
            left -= slab_cost[en.layer];
            seen[en.layer][en.e] = 1;
            hot[en.layer].push_back(en.e);
        }
    } else {
        for (int l = 0; l < L; l++) {
            if (left < layer_cost[l]) break;
            left -= layer_cost[l];
            for (int e = 0; e < E; e++) hot[l].push_back((uint32_t)e);
        }
    }
    for (auto &v : hot) std::sort(v.begin(), v.end());
}

// Placement of expert tensors (moe.rs:692-880).  All experts stay in HBM
// unless opts.expert_budget_mb >= 0; then every expert tensor lives in
// pinned host memory and the budget buys HBM copies of the hottest
// (layer, expert) slabs from the popularity list, or -- without a list --
// whole layers in order.
int styx_moe::place_experts(const std::vector<std::vector<std::pair<uint32_t, uint64_t>>> *hist)
{
    for (auto &ly : layers) {
        ly.remap.assign(E, SKIP);
        ly.hits.assign(E, 0);
        ly.slot_experts.clear();
    }
    any_host = false;
    exp_hbm = exp_host = 0;
    if (opts.expert_budget_mb < 0) {
        for (auto &ly : layers) {
            for (int e = 0; e < E; e++) ly.remap[e] = (uint32_t)e;
            ly.slot_experts.resize(E);
            std::iota(ly.slot_experts.begin(), ly.slot_experts.end(), 0u);
            ly.host_experts = false;
            exp_hbm += ly.gate.bytes() + ly.up.bytes() + ly.down.bytes();
        }
        return STYX_OK;
    }
    any_host = true;
    std::vector<std::vector<uint32_t>> hot;
    std::vector<uint64_t> slab_cost(L), layer_cost(L);
    for (int l = 0; l < L; l++) {
        const auto &ly = layers[l];
        slab_cost[l] = ly.gate.slab + ly.up.slab + ly.down.slab;
        layer_cost[l] = ly.gate.bytes() + ly.up.bytes() + ly.down.bytes();
    }
    plan_hot_experts(hist, L, E, slab_cost, layer_cost, (uint64_t)opts.expert_budget_mb << 20, hot);
    for (int l = 0; l < L; l++) {
        auto &ly = layers[l];
        auto &ord = hot[l];
        std::sort(ord.begin(), ord.end());
        ly.host_experts = true;
        ly.slot_experts = ord;
        for (size_t i = 0; i < ord.size(); i++) ly.remap[ord[i]] = (uint32_t)i;
        for (Mat *m : {&ly.gate, &ly.up, &ly.down}) {
            exp_host += m->bytes();
            if (ord.empty()) continue;
            if (int r = alloc((void **)&m->hot, (size_t)ord.size() * m->slab)) return r;
            exp_hbm += (uint64_t)ord.size() * m->slab;
            for (size_t i = 0; i < ord.size(); i++)
                STYX_HIP(hipMemcpyAsync(m->hot + i * m->slab, m->host + (int64_t)ord[i] * m->slab,
                                        m->slab, hipMemcpyHostToDevice, gpu->stream));
        }
        if (int r = dalloc(&ly.remap_dev, E)) return r;
        STYX_HIP(hipMemcpyAsync(ly.remap_dev, ly.remap.data(), sizeof(uint32_t) * E,
                                hipMemcpyHostToDevice, gpu->stream));
    }
    // arena: k slots per tensor, each the largest slab of its kind, filled
    // by the gather on the copy stream
    if (opts.arena) {
        if (!st_copy) {
            STYX_HIP(hipStreamCreateWithFlags(&st_copy, hipStreamNonBlocking));
            STYX_HIP(hipEventCreateWithFlags(&ev_fork, hipEventDisableTiming));
            STYX_HIP(hipEventCreateWithFlags(&ev_join, hipEventDisableTiming));
        }
        for (int t = 0; t < 3; t++) {
            int64_t mx = 0;
            for (auto &ly : layers) mx = std::max(mx, (t == 0 ? ly.gate : t == 1 ? ly.up : ly.down).slab);
            arena_slab[t] = mx;
            if (int r = alloc((void **)&arena[t], (size_t)K * mx)) return r;
            exp_hbm += (uint64_t)K * mx;
        }
    }
    STYX_HIP(hipStreamSynchronize(gpu->stream));
    return STYX_OK;
}

// Grid of the fused MoE block: every workgroup resident at once, at most two
// per CU, the same for every layer (the launch tag is ticket / grid); 0 when
// a layer's shapes or placement need the separate kernels, or the model
// options ask for them.
int styx_moe::size_moe_block()
{
    mb_nwg = 0;
    qkv_fold.assign(L, 0);  // no fold without the fused block
    if (opts.no_fuse || L == 0) return STYX_OK;
    int per_cu = 2;
    for (const Layer &ly : layers) {
        const bool sh_fused = ly.gsh.dev && Fsh == F && ly.gsh.type == ly.gate.type &&
                              ly.ush.type == ly.up.type && ly.dsh.type == ly.down.type;
        if ((ly.gsh.dev && !sh_fused) || (ly.host_experts && opts.arena)) return STYX_OK;
        per_cu = std::min(per_cu, moe_block_occupancy(ly.gate.type, ly.up.type, ly.down.type, H, F,
                                                      E, K, sh_fused ? 1 : 0));
    }
    if (per_cu < 1) return STYX_OK;
    int ncu = 0;
    STYX_HIP(hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, gpu->device));
    mb_nwg = per_cu * ncu / 64 * 64;  // the kernel's ticket counters need a multiple of 64
    if (mb_nwg > 0 && !mb_trace)
        if (int r = dalloc(&mb_trace, (size_t)L * mb_nwg * 16)) return r;
    // the next layer's q/k/v folded into the block's tail: q8_0 matrices
    // whose rows fit the grid beside the reduce workgroups
    qkv_fold.assign(L, 0);
    if (mb_nwg > 0 && !opts.no_fold_qkv) {
        for (int l = 1; l < L; l++) {
            const Layer &p = layers[l - 1], &ly = layers[l];
            if (ly.wq.type != T_Q8_0 || ly.wk.type != T_Q8_0 || ly.wv.type != T_Q8_0) continue;
            const bool sh_fused = p.gsh.dev != nullptr;
            const int rows[3] = {ly.wq.rows, ly.wk.rows, ly.wv.rows};
            qkv_fold[l] = moe_block_fold_ok(p.gate.type, p.up.type, p.down.type, H, F, E, K,
                                            sh_fused ? 1 : 0, rows, mb_nwg)
                              ? 1
                              : 0;
        }
        bool any = false;
        for (char c : qkv_fold) any = any || c;
        if (any && !t_xq) {
            const size_t n = xq_bytes(H) / 4 + (size_t)(H + 255) / 256;
            if (int r = dalloc(&t_xq, n)) return r;
            STYX_HIP(hipMemsetAsync(t_xq, 0, sizeof(uint64_t) * n, gpu->stream));
        }
    }
    return STYX_OK;
}

// A fused MoE launch whose wait ran out sets the abort flag; the model's
// results are then invalid and it stays in error until reloaded.  The flag
// is copied into the pinned stage (h_stage[4]) ahead of the caller's stream
// synchronisation (queue_abort_read), then checked here.
void styx_moe::queue_abort_read()
{
    if (mb_abort && !opts.no_fuse)
        (void)hipMemcpyAsync(&h_stage[4], mb_abort, sizeof(int), hipMemcpyDeviceToHost, gpu->stream);
}

int styx_moe::check_abort()
{
    if (!mb_abort || opts.no_fuse) return STYX_OK;
    if (h_stage[4])
        return fail(STYX_E_DEVICE, "fused MoE block / attention: a workgroup's wait ran out (not "
                                   "all workgroups resident?); results of this model are invalid");
    return STYX_OK;
}

// After a fused launch gave up waiting: the model goes over to the separate
// kernels for good (they never wait on another workgroup), the graphs
// captured with the fused launches are replaced, and the flag is cleared.
// The caller then runs the failed token(s) again: a token rewrites every
// value it reads (the residual from the embedding, its KV row, the ids).
int styx_moe::fall_back_unfused()
{
    opts.no_fuse = 1;
    fallbacks++;
    STYX_HIP(hipStreamSynchronize(gpu->stream));
    for (int i = 0; i < 3; i++) {
        if (g_fwd[i]) hipGraphExecDestroy(g_fwd[i]);
        if (g_gen[i]) hipGraphExecDestroy(g_gen[i]);
        g_fwd[i] = g_gen[i] = nullptr;
    }
    if (int r = size_moe_block()) return r;
    STYX_HIP(hipMemsetAsync(mb_abort, 0, sizeof(int), gpu->stream));
    h_stage[4] = 0;
    return build_graphs();
}

// ------------------------------------------------------------ forward ----
// Whether the attention of a token at context length n_t merges its chunk
// partials inside the attention kernel: while a head has at most 32 chunks
// (chunking as the device computes it, attn.hip attn_chunk); beyond that the
// few merging workgroups are slower than the separate combine kernel.
bool styx_moe::attn_merge_in_kernel(int n_t) const
{
    if (opts.no_fuse) return false;
    const int gqa = nh / nkv;
    int ch_min = chunk, mc = max_chunks;
    if (hd == 128 && gqa == 16) {  // the matrix-core variant's chunking
        ch_min = std::max(chunk, 64);
        mc = std::max(1, std::min(max_chunks, 512 / nkv));
    }
    const int need = (n_t + mc - 1) / mc;
    const int ch = std::max(ch_min, (need + 15) / 16 * 16);
    return (n_t + ch - 1) / ch <= ATTN_MERGE_MAX_CHUNKS;
}

// Attention variant of a token at context n_t: one chunk on the matrix-core
// kernel (short contexts), chunks merged in the attention kernel, or merged
// by the combine kernel (the only variant with no_fuse, whose kernels never
// wait on another workgroup).
int styx_moe::attn_mode(int n_t) const
{
    if (!opts.no_fuse && hd == 128 && nh / nkv >= 4 && nh / nkv <= 16 && n_t <= attn_solo_max)
        return AT_SOLO;
    return attn_merge_in_kernel(n_t) ? AT_MERGE : AT_COMBINE;
}

int styx_moe::enqueue_token(bool gen, int mode)
{
    hipStream_t st = gpu->stream;
    const int q_dim = nh * hd;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    hipStreamIsCapturing(st, &cs);
    const bool timing = opts.time_kernels != 0 && cs == hipStreamCaptureStatusNone;
    auto tstart = [&](hipStream_t on = nullptr) -> hipEvent_t {
        if (!timing) return nullptr;
        hipEvent_t e = ev();
        hipEventRecord(e, on ? on : st);
        return e;
    };
    auto tend = [&](hipEvent_t a, const char *nm, double bytes, hipStream_t on = nullptr) {
        if (!timing) return;
        hipEvent_t e = ev();
        hipEventRecord(e, on ? on : st);
        const int id = stat_id(nm);
        stats[id].bytes += bytes;
        pending.push_back({id, {a, e}});
    };
    auto want = [&](const char *nm) { return stage_only.empty() || stage_only == nm; };
    if (mb_nwg < 0)
        if (int r = size_moe_block()) return r;
    // the first layer's q/k/v input: limbs of attn_norm_0(x) (or of the LM
    // head's output_norm(x) for a model without layers)
    const float *norm0 = L > 0 ? layers[0].attn_norm : out_norm;
    // (and the rope row of the token's position, which every layer's
    // attention then loads without waiting for the position)
    if (want("embed"))
        CK(launch_embed(st, embd.type, embd.dev, V, H, d_tok, x, norm0, xq_a, ss_a,
                        (const double2 *)rope, d_pos, (double2 *)rope_cur, hd / 2));
    // every consumer of xq_a applies the RMSNorm scale from the x^2 partials
    const NormScale ns_a{ss_a, (H + 255) / 256, H, eps};
    if (opts.record_hidden && stage_only.empty()) CK(hipMemcpyAsync(hidden, x, sizeof(float) * H, hipMemcpyDeviceToDevice, st));
    for (int l = 0; l < L; l++) {
        Layer &ly = layers[l];
        hipEvent_t e0 = tstart();
        const bool folded = !qkv_fold.empty() && qkv_fold[l];  // ran in the previous block
        if (folded) {
        } else if (ly.wq.type == ly.wk.type && ly.wq.type == ly.wv.type) {
            DenseSeg s[3] = {{ly.wq.dev, q, ly.wq.rows}, {ly.wk.dev, kk, ly.wk.rows},
                             {ly.wv.dev, vv, ly.wv.rows}};
            if (want("qkv")) CK(launch_dense(st, ly.wq.type, H, s, 3, xq_a, 0, &ns_a));
        } else {
            DenseSeg a{ly.wq.dev, q, ly.wq.rows}, b{ly.wk.dev, kk, ly.wk.rows},
                c{ly.wv.dev, vv, ly.wv.rows};
            if (want("qkv")) CK(launch_dense(st, ly.wq.type, H, &a, 1, xq_a, 0, &ns_a));
            if (want("qkv")) CK(launch_dense(st, ly.wk.type, H, &b, 1, xq_a, 0, &ns_a));
            if (want("qkv")) CK(launch_dense(st, ly.wv.type, H, &c, 1, xq_a, 0, &ns_a));
        }
        if (!folded)
            tend(e0, "qkv", (double)(ly.wq.bytes() + ly.wk.bytes() + ly.wv.bytes()) + xq_bytes(H));
        AttnArgs aa{};
        if (timing) {
            // phase stamps of every workgroup (eager timed tokens only)
            aa.trace = at_trace + (size_t)l * max_chunks * nkv * AT_TRACE;
            CK(hipMemsetAsync(aa.trace, 0, sizeof(uint64_t) * max_chunks * nkv * AT_TRACE, st));
        }
        e0 = tstart();
        aa.q = q;
        aa.k = kk;
        aa.v = vv;
        aa.q_norm = ly.q_norm;
        aa.k_norm = ly.k_norm;
        aa.eps = eps;
        aa.rope = (const double2 *)rope;
        aa.rope_row = (const double2 *)rope_cur;
        aa.kpool = kpool;
        aa.vpool = vpool;
        aa.page_table = d_pt + (size_t)l * pages_per_layer;
        aa.page_table_len = pages_per_layer;
        aa.page_tokens = KV_PAGE_TOKENS;
        aa.kv_head_major = kv_head_major;
        aa.pos = d_pos;
        aa.out = attn;
        aa.xq = xq_o;
        aa.part = attn_part;
        aa.nh = nh;
        aa.nkv = nkv;
        aa.hd = hd;
        aa.chunk = chunk;
        aa.max_chunks = mode == AT_SOLO ? 1 : max_chunks;
        aa.solo_max = mode == AT_SOLO ? attn_solo_max : 0;
        aa.scale = 1.0f / std::sqrt((float)hd);
        // the single-chunk mode exchanges nothing: no tagged words, and no
        // ticket draws (a launch of another grid drawing from the counters
        // would break the launch numbering the merged mode's tags rely on)
        if (mode == AT_MERGE) {
            aa.t_part = at_part;
            aa.tickets = at_tickets;
            aa.abort = mb_abort;
            aa.max_polls = opts.max_polls > 0 ? opts.max_polls : 200000;
        }
        if (want("attn")) CK(launch_attn_decode(st, aa));
        tend(e0, "attn", (double)(n_past + 1) * nkv * hd * 8.0);
        e0 = tstart();
        DenseSeg so{ly.wo.dev, x, H};
        if (want("o_proj")) CK(launch_dense(st, ly.wo.type, q_dim, &so, 1, xq_o, 1));
        tend(e0, "o_proj", (double)ly.wo.bytes() + xq_bytes(q_dim) + 8.0 * H);
        // the MoE block: one fused persistent launch, or router, gate/up,
        // down and reduce as separate kernels (identical results)
        const bool fused = mb_nwg > 0;
        e0 = tstart();
        RouterArgs ra{};
        ra.x = x;
        ra.norm_w = ly.ffn_norm;
        ra.W = ly.router;
        ra.bias = ly.router_bias;
        ra.eps = eps;
        ra.xn = xn;
        ra.xq = xq_f;
        ra.logits = rlog;
        ra.E = E;
        ra.H = H;
        ra.k = K;
        if (!fused && want("router")) CK(launch_router(st, ra));
        if (!fused) tend(e0, "router", (double)E * H * 4 + 8.0 * H + 4.0 * E);
        // top-k ids are ranked by every consumer workgroup from the logits;
        // gate_up's first workgroup publishes the id row, k_reduce_norm the
        // weights
        Route rt{};
        rt.logits = rlog;
        rt.E = E;
        rt.k = K;
        rt.remap = ly.host_experts ? ly.remap_dev : nullptr;
        rt.arena_mode = ly.host_experts && opts.arena ? 1 : 0;
        rt.layer = 0;
        rt.ids_out = ids + (size_t)l * 64;
        const int32_t *lid = ids + (size_t)l * 64;
        ExpSrc sg{}, su{}, sd{};
        Mat *ms[3] = {&ly.gate, &ly.up, &ly.down};
        ExpSrc *ss[3] = {&sg, &su, &sd};
        for (int t = 0; t < 3; t++) {
            Mat &m = *ms[t];
            ExpSrc &s = *ss[t];
            if (!ly.host_experts) {
                s.hot = m.dev;
                s.hot_slab = m.slab;
            } else {
                s.hot = m.hot;
                s.hot_slab = m.slab;
                s.arena = arena[t];
                s.arena_slab = arena_slab[t];
                s.gtt = m.host_dev;
                s.gtt_slab = m.slab;
            }
        }
        // the cold slabs are gathered on the copy stream while the hot
        // slots' expert kernels run on this one
        const bool overlap = ly.host_experts && opts.arena && st_copy;
        if (overlap) {
            CK(hipEventRecord(ev_fork, st));
            CK(hipStreamWaitEvent(st_copy, ev_fork, 0));
            e0 = tstart(st_copy);
            const uint8_t *src[3] = {ly.gate.host_dev, ly.up.host_dev, ly.down.host_dev};
            const int64_t sslab[3] = {ly.gate.slab, ly.up.slab, ly.down.slab};
            Route rg = rt;
            rg.ids_out = nullptr;
            if (want("gather"))
                CK(launch_gather(st_copy, src, sslab, arena, arena_slab, nullptr, &rg, K));
            tend(e0, "gather", 0.0, st_copy);
            CK(hipEventRecord(ev_join, st_copy));
        }
        // the shared expert runs as slot K of the expert kernels when it has
        // the routed experts' width and types; otherwise as dense matvecs
        const bool sh_fused = ly.gsh.dev && Fsh == F && ly.gsh.type == ly.gate.type &&
                              ly.ush.type == ly.up.type && ly.dsh.type == ly.down.type;
        const double sh_gu = sh_fused ? (double)(ly.gsh.bytes() + ly.ush.bytes()) : 0.0;
        const double slabs_gu = (double)K * (ly.gate.slab + ly.up.slab) + sh_gu;
        const int nsl = K + (sh_fused ? 1 : 0);
        if (fused) {
            e0 = tstart();
            MoeBlockArgs mb{};
            mb.tg = ly.gate.type;
            mb.tu = ly.up.type;
            mb.td = ly.down.type;
            mb.x = x;
            mb.ffn_norm = ly.ffn_norm;
            mb.W = ly.router;
            mb.bias = ly.router_bias;
            mb.eps = eps;
            mb.H = H;
            mb.F = F;
            mb.E = E;
            mb.k = K;
            mb.renorm = norm_topk;
            mb.src[0] = sg;
            mb.src[1] = su;
            mb.src[2] = sd;
            mb.route = rt;
            if (sh_fused) {
                mb.sh[0] = ly.gsh.dev;
                mb.sh[1] = ly.ush.dev;
                mb.sh[2] = ly.dsh.dev;
                mb.sh_ginp = ly.gate_inp_sh;
            }
            mb.norm_next = l + 1 < L ? layers[l + 1].attn_norm : out_norm;
            mb.xq = xq_a;
            mb.ss = ss_a;
            mb.wts_out = wts + (size_t)l * 16;
            mb.t_lg = t_lg;
            mb.t_gu = t_gu;
            mb.t_part = t_part;
            mb.ticket = mb_ticket;
            mb.abort = mb_abort;
            mb.max_polls = opts.max_polls;
            mb.nwg = mb_nwg;
            const bool fold_next = l + 1 < L && qkv_fold[l + 1];
            double qkv_bytes = 0.0;
            if (fold_next) {
                const Layer &nx = layers[l + 1];
                mb.wqkv[0] = nx.wq.dev;
                mb.wqkv[1] = nx.wk.dev;
                mb.wqkv[2] = nx.wv.dev;
                mb.qkv_out[0] = q;
                mb.qkv_out[1] = kk;
                mb.qkv_out[2] = vv;
                mb.qkv_rows[0] = nx.wq.rows;
                mb.qkv_rows[1] = nx.wk.rows;
                mb.qkv_rows[2] = nx.wv.rows;
                mb.t_xq = t_xq;
                qkv_bytes = (double)(nx.wq.bytes() + nx.wk.bytes() + nx.wv.bytes());
            }
            if (timing) {
                // phase stamps of every workgroup (eager timed tokens only)
                mb.trace = mb_trace + (size_t)l * mb_nwg * 16;
                CK(hipMemsetAsync(mb.trace, 0, sizeof(uint64_t) * mb_nwg * 16, st));
            }
            if (want("moe_block")) CK(launch_moe_block(st, mb));
            tend(e0, "moe_block", (double)E * H * 4 + slabs_gu + (double)K * ly.down.slab +
                                      (sh_fused ? (double)ly.dsh.bytes() : 0.0) + 16.0 * H +
                                      qkv_bytes);
        } else {
        // two passes with the copy stream (hot slots, then -- once the
        // gather has landed -- the arena slots), one without
        const int passes = overlap ? 2 : 1;
        for (int pass = 0; pass < passes; pass++) {
        const int filter = overlap ? (pass == 0 ? SLOTS_HOT : SLOTS_COLD) : SLOTS_ALL;
        if (pass == 1) CK(hipStreamWaitEvent(st, ev_join, 0));
        e0 = tstart();
        if (want("moe_gate_up")) CK(launch_moe_gate_up(st, ly.gate.type, ly.up.type, sg, su, nullptr, &rt, xq_f, gu, H, F,
                              K, sh_fused ? ly.gsh.dev : nullptr, sh_fused ? ly.ush.dev : nullptr, filter));
        tend(e0, "moe_gate_up", pass == 1 ? 0.0 : slabs_gu + xq_bytes(H) + 4.0 * E + 4.0 * 2 * nsl * F);
        if (pass == 0 && ly.gsh.dev && !sh_fused && want("shexp")) {
            e0 = tstart();
            DenseSeg s2[2] = {{ly.gsh.dev, sh_g, Fsh}, {ly.ush.dev, sh_u, Fsh}};
            if (ly.gsh.type == ly.ush.type) {
                CK(launch_dense(st, ly.gsh.type, H, s2, 2, xq_f, 0));
            } else {
                CK(launch_dense(st, ly.gsh.type, H, &s2[0], 1, xq_f, 0));
                CK(launch_dense(st, ly.ush.type, H, &s2[1], 1, xq_f, 0));
            }
            CK(launch_xq(st, sh_g, sh_u, nullptr, 0.0f, Fsh, xq_sh, nullptr));
            DenseSeg sd2{ly.dsh.dev, sh_y, H};
            CK(launch_dense(st, ly.dsh.type, Fsh, &sd2, 1, xq_sh, 0));
            tend(e0, "shexp", (double)(ly.gsh.bytes() + ly.ush.bytes() + ly.dsh.bytes()));
        }
        e0 = tstart();
        if (want("moe_down")) CK(launch_moe_down(st, ly.down.type, sd, lid, gu, partial, H, F, K,
                           sh_fused ? ly.dsh.dev : nullptr, filter));
        tend(e0, "moe_down", pass == 1 ? 0.0 : (double)K * ly.down.slab + (sh_fused ? (double)ly.dsh.bytes() : 0.0) +
                                 4.0 * 2 * nsl * F + 4.0 * nsl * H);
        }
        e0 = tstart();
        ReduceArgs rd{};
        rd.partial = partial;
        rd.k = K;
        rd.H = H;
        rd.logits = rlog;
        rd.E = E;
        rd.renorm = norm_topk;
        rd.ids = lid;
        rd.wts_out = wts + (size_t)l * 16;
        rd.x = x;
        if (ly.gsh.dev) {
            rd.sh_y = sh_fused ? partial + (size_t)K * H : sh_y;
            rd.sh_ginp = ly.gate_inp_sh;
            rd.xn = xn;
        }
        rd.norm_w = l + 1 < L ? layers[l + 1].attn_norm : out_norm;
        rd.xq = xq_a;
        rd.ss = ss_a;
        if (want("reduce")) CK(launch_reduce_rows(st, rd));
        tend(e0, "reduce", 4.0 * nsl * H + 12.0 * H + 4.0 * E + xq_bytes(H));
        }
        if (opts.record_hidden && stage_only.empty())
            CK(hipMemcpyAsync(hidden + (size_t)(l + 1) * H, x, sizeof(float) * H,
                              hipMemcpyDeviceToDevice, st));
    }
    hipEvent_t e0 = tstart();
    DenseSeg sh{head.dev, logits, V};
    // the greedy token is reduced inside the LM head (one atomic maximum per
    // workgroup); a one-thread kernel reads it out
    if (want("lm_head")) CK(launch_dense(st, head.type, H, &sh, 1, xq_a, 0, &ns_a, am_word));
    tend(e0, "lm_head", (double)head.bytes() + xq_bytes(H) + 4.0 * V);
    e0 = tstart();
    if (want("argmax")) CK(launch_argmax_word(st, am_word, d_tok, d_pos, gen ? 1 : 0, hist));
    tend(e0, "argmax", 8.0);
    return STYX_OK;
}

int styx_moe::build_graphs()
{
    if (!opts.use_graph) return STYX_OK;
    // forward / generate x the attention modes (attn_mode): one chunk
    // (short contexts), merged in the kernel, or by the combine kernel (long
    // ones; the only variant with no_fuse)
    for (int gm = 0; gm < 6; gm++) {
        const bool gen = gm / 3 == 1;
        const int mode = gm % 3;
        if (mode != AT_COMBINE && opts.no_fuse) continue;
        if (mode == AT_SOLO && attn_mode(1) != AT_SOLO) continue;  // shapes without it
        hipGraph_t g;
        STYX_HIP(hipStreamBeginCapture(gpu->stream, hipStreamCaptureModeThreadLocal));
        int r = enqueue_token(gen, mode);
        hipError_t e = hipStreamEndCapture(gpu->stream, &g);
        if (r) return r;
        if (e != hipSuccess) return hip_fail(e, "hipStreamEndCapture");
        hipGraphExec_t ex;
        e = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
        hipGraphDestroy(g);
        if (e != hipSuccess) return hip_fail(e, "hipGraphInstantiate");
        (gen ? g_gen : g_fwd)[mode] = ex;
    }
    return STYX_OK;
}

// The token at position n_past (context n_past + 1).
int styx_moe::run_token(bool gen)
{
    const int mode = attn_mode(n_past + 1);
    hipGraphExec_t g = (gen ? g_gen : g_fwd)[mode];
    if (g && !opts.time_kernels) {
        STYX_HIP(hipGraphLaunch(g, gpu->stream));
        return STYX_OK;
    }
    return enqueue_token(gen, mode);
}

// Repin choice for one layer (moe.rs:1465-1497): residents ranked coldest
// first, outsiders hottest first (both stable on ties, where the reference's
// sort_unstable leaves the order open); the i-th pair swaps while the
// outsider has at least twice the resident's hits (and at least 2), at most
// maxsw pairs.  resident[e] says whether expert e holds a hot slot.
static void repin_select(const uint64_t *hits, int E, const uint32_t *slot_experts, int n_slots,
                         const std::vector<char> &resident, int maxsw,
                         std::vector<std::pair<int, uint32_t>> &swaps)
{
    swaps.clear();
    std::vector<int> res(n_slots);
    std::iota(res.begin(), res.end(), 0);
    std::stable_sort(res.begin(), res.end(), [&](int a, int b) {
        return hits[slot_experts[a]] < hits[slot_experts[b]];
    });
    std::vector<uint32_t> out;
    for (int e = 0; e < E; e++)
        if (!resident[e]) out.push_back((uint32_t)e);
    std::stable_sort(out.begin(), out.end(),
                     [&](uint32_t a, uint32_t b) { return hits[a] > hits[b]; });
    for (int i = 0; i < maxsw && i < n_slots && i < (int)out.size(); i++) {
        const uint32_t old = slot_experts[res[i]], nw = out[i];
        if (hits[nw] < 2 * std::max<uint64_t>(hits[old], 1)) break;
        swaps.push_back({res[i], nw});
    }
}

// Online repinning (moe.rs:1450-1508): fold the last token's routing into
// per-layer hit counters; every repin_interval tokens swap up to repin_max
// cold slots per layer for outsiders with at least twice the hits.  The
// remap (host and device) changes only after the slab copies have landed;
// a copy that fails leaves a hot slot half-written, so the model is then
// marked broken and refuses further tokens.
int styx_moe::maybe_repin()
{
    if (opts.repin_interval <= 0 || !any_host) return STYX_OK;
    std::vector<int32_t> h((size_t)L * 64);
    STYX_HIP(hipMemcpy(h.data(), ids, sizeof(int32_t) * h.size(), hipMemcpyDeviceToHost));
    for (int l = 0; l < L; l++)
        for (int s = 0; s < K; s++) {
            const uint32_t e = (uint32_t)h[(size_t)l * 64 + s];
            if (e < (uint32_t)E) layers[l].hits[e]++;
        }
    if (n_past % opts.repin_interval != 0) return STYX_OK;
    const int maxsw = opts.repin_max > 0 ? opts.repin_max : 2;
    std::vector<std::pair<int, uint32_t>> swaps;
    auto broke = [&](hipError_t e, const char *what) {
        broken = std::string("repin: ") + what + " failed (" + hipGetErrorString(e) +
                 "); a hot slot may hold a partial slab, reload the model";
        return fail(STYX_E_HIP, broken);
    };
    for (auto &ly : layers) {
        const int n_slots = (int)ly.slot_experts.size();
        if (n_slots == 0 || !ly.host_experts) continue;
        std::vector<char> resident(E, 0);
        for (int e = 0; e < E; e++) resident[e] = ly.remap[e] != SKIP;
        repin_select(ly.hits.data(), E, ly.slot_experts.data(), n_slots, resident, maxsw, swaps);
        if (swaps.empty()) continue;
        for (auto &sw : swaps)
            for (Mat *m : {&ly.gate, &ly.up, &ly.down}) {
                const hipError_t e = hipMemcpyAsync(m->hot + (int64_t)sw.first * m->slab,
                                                    m->host + (int64_t)sw.second * m->slab,
                                                    m->slab, hipMemcpyHostToDevice, gpu->stream);
                if (e != hipSuccess) return broke(e, "slab copy");
            }
        if (hipError_t e = hipStreamSynchronize(gpu->stream); e != hipSuccess)
            return broke(e, "slab copy");
        for (auto &sw : swaps) {
            const uint32_t old = ly.slot_experts[sw.first];
            ly.remap[old] = SKIP;
            ly.remap[sw.second] = (uint32_t)sw.first;
            ly.slot_experts[sw.first] = sw.second;
            repin_swaps++;
        }
        if (hipError_t e = hipMemcpyAsync(ly.remap_dev, ly.remap.data(), sizeof(uint32_t) * E,
                                          hipMemcpyHostToDevice, gpu->stream);
            e != hipSuccess)
            return broke(e, "remap upload");
        if (hipError_t e = hipStreamSynchronize(gpu->stream); e != hipSuccess)
            return broke(e, "remap upload");
    }
    return STYX_OK;
}

// ---------------------------------------------------------- model build --
namespace {

struct TensorSpec {
    std::string name;
    int type;
    std::vector<int64_t> dims;  // GGUF order: dims[0] = columns
};

int64_t n_elems(const std::vector<int64_t> &d)
{
    int64_t n = 1;
    for (auto v : d) n *= v;
    return n;
}

// Source of a tensor's GGUF-layout bytes: either a host pointer (file) or
// the generator.
struct Source {
    const uint8_t *host = nullptr;
    uint64_t seed = 0;
    float sigma = 0, mean = 0;
    const std::vector<float> *values = nullptr;  // explicit f32 values
};

struct Builder {
    styx_moe *m;
    uint8_t *tmp = nullptr;  // staging for GGUF-layout bytes
    size_t tmp_size = 0;

    int stage(int type, int64_t n, const Source &src)
    {
        const int64_t bytes = n / blk_elems(type) * blk_bytes(type);
        if ((size_t)bytes > tmp_size) return fail(STYX_E_INVALID, "staging buffer too small");
        hipStream_t st = m->gpu->stream;
        if (src.host) {
            STYX_HIP(hipMemcpyAsync(tmp, src.host, bytes, hipMemcpyHostToDevice, st));
        } else if (src.values) {
            STYX_HIP(hipMemcpyAsync(tmp, src.values->data(), bytes, hipMemcpyHostToDevice, st));
        } else if (type == T_F32) {
            CK(launch_gen_f32(st, src.seed, src.mean, src.sigma, (float *)tmp, n));
        } else if (type == T_F16) {
            // f16 values of the same seeded N(0, sigma) draws
            CK(launch_gen_quant(st, T_F16, src.seed, src.sigma, tmp, n));
        } else {
            CK(launch_gen_quant(st, type, src.seed, src.sigma, tmp, n));
        }
        return STYX_OK;
    }

    int f32(const TensorSpec &t, const Source &src, float **out)
    {
        const int64_t n = n_elems(t.dims);
        if (t.type != T_F32) return fail(STYX_E_FORMAT, t.name + ": expected f32");
        if (int r = m->dalloc(out, n)) return r;
        if (int r = stage(T_F32, n, src)) return r;
        STYX_HIP(hipMemcpyAsync(*out, tmp, n * 4, hipMemcpyDeviceToDevice, m->gpu->stream));
        m->f32s.push_back({t.name, *out, n, t.dims});
        return STYX_OK;
    }

    // 2-D matrix or 3-D expert tensor into split layout; host_copy: keep the
    // split bytes in pinned host memory instead of HBM.
    int mat(const TensorSpec &t, const Source &src, Mat &o, bool host_copy, bool allow_float = false)
    {
        if (!is_quant(t.type) && !(allow_float && (t.type == T_F32 || t.type == T_F16)))
            return fail(STYX_E_FORMAT, t.name + ": matrix type must be q8_0/q4_K/q5_K/q6_K");
        if (t.dims.size() < 2) return fail(STYX_E_FORMAT, t.name + ": not a matrix");
        o.name = t.name;
        o.type = t.type;
        o.cols = (int)t.dims[0];
        o.rows = (int)t.dims[1];
        o.nmat = t.dims.size() > 2 ? (int)t.dims[2] : 1;
        o.gguf_dims = t.dims;
        if (o.cols % blk_elems(t.type))
            return fail(STYX_E_FORMAT, t.name + ": row length not a multiple of the block size");
        const int64_t nb = (int64_t)o.rows * (o.cols / blk_elems(t.type));
        o.slab = nb * blk_bytes(t.type);
        if (o.slab % 16) return fail(STYX_E_FORMAT, t.name + ": slab not a multiple of 16 bytes");
        const int64_t n = n_elems(t.dims);
        if (int r = stage(t.type, n, src)) return r;
        uint8_t *dst;
        if (int r = m->alloc((void **)&dst, o.bytes())) return r;
        CK(launch_to_split(m->gpu->stream, t.type, tmp, dst, nb, o.nmat));
        if (host_copy) {
            if (int r = m->alloc_host((void **)&o.host, o.bytes())) return r;
            STYX_HIP(hipMemcpyAsync(o.host, dst, o.bytes(), hipMemcpyDeviceToHost, m->gpu->stream));
            STYX_HIP(hipStreamSynchronize(m->gpu->stream));
            void *dp = nullptr;
            STYX_HIP(hipHostGetDevicePointer(&dp, o.host, 0));
            o.host_dev = (uint8_t *)dp;
            STYX_HIP(hipFree(dst));
            m->dev_allocs.erase(std::find(m->dev_allocs.begin(), m->dev_allocs.end(), (void *)dst));
        } else {
            o.dev = dst;
        }
        return STYX_OK;
    }
};

std::string blk(int l, const char *s) { return "blk." + std::to_string(l) + "." + s + ".weight"; }

// Tensor list of a qwen3moe model (names/dims the loader expects,
// moe.rs:550-599,1061-1108).
std::vector<TensorSpec> model_specs(const styx_moe_synth_cfg &c)
{
    std::vector<TensorSpec> v;
    const int64_t H = c.n_embd, qd = (int64_t)c.n_heads * c.head_dim,
                  kvd = (int64_t)c.n_kv_heads * c.head_dim;
    v.push_back({"token_embd.weight", c.embd_type, {H, c.n_vocab}});
    v.push_back({"output_norm.weight", T_F32, {H}});
    v.push_back({"output.weight", c.head_type, {H, c.n_vocab}});
    static const int mix[3] = {T_Q4_K, T_Q5_K, T_Q6_K};
    for (int l = 0; l < c.n_layers; l++) {
        auto et = [&](int role) { return c.exp_mix ? mix[(l + role) % 3] : c.exp_type[role]; };
        v.push_back({blk(l, "attn_norm"), T_F32, {H}});
        v.push_back({blk(l, "attn_q_norm"), T_F32, {c.head_dim}});
        v.push_back({blk(l, "attn_k_norm"), T_F32, {c.head_dim}});
        v.push_back({blk(l, "attn_q"), c.attn_type, {H, qd}});
        v.push_back({blk(l, "attn_k"), c.attn_type, {H, kvd}});
        v.push_back({blk(l, "attn_v"), c.attn_type, {H, kvd}});
        v.push_back({blk(l, "attn_output"), c.attn_type, {qd, H}});
        v.push_back({blk(l, "ffn_norm"), T_F32, {H}});
        v.push_back({blk(l, "ffn_gate_inp"), T_F32, {H, c.n_expert}});
        v.push_back({blk(l, "ffn_gate_exps"), et(0), {H, c.n_ff_exp, c.n_expert}});
        v.push_back({blk(l, "ffn_up_exps"), et(1), {H, c.n_ff_exp, c.n_expert}});
        v.push_back({blk(l, "ffn_down_exps"), et(2), {c.n_ff_exp, H, c.n_expert}});
        if (c.n_ff_shexp > 0) {
            v.push_back({blk(l, "ffn_gate_shexp"), et(0), {H, c.n_ff_shexp}});
            v.push_back({blk(l, "ffn_up_shexp"), et(1), {H, c.n_ff_shexp}});
            v.push_back({blk(l, "ffn_down_shexp"), et(2), {c.n_ff_shexp, H}});
            v.push_back({blk(l, "ffn_gate_inp_shexp"), T_F32, {H}});
        }
        if (c.router_zipf_s > 0)
            v.push_back({"blk." + std::to_string(l) + ".ffn_gate_inp.bias", T_F32, {c.n_expert}});
    }
    return v;
}

int64_t spec_bytes(const TensorSpec &t)
{
    return n_elems(t.dims) / blk_elems(t.type) * blk_bytes(t.type);
}

// Every tensor the model reads, with the GGUF dims (dims[0] = columns) and
// type class the hparams imply, checked before anything is allocated or
// uploaded: a short router, norm or LM-head tensor would otherwise make a
// kernel read past its allocation.  Names the model does not use are
// ignored, as the reference's loader ignores them.
int check_specs(const styx_moe_synth_cfg &c, std::vector<TensorSpec> &specs)
{
    const int64_t H = c.n_embd, qd = (int64_t)c.n_heads * c.head_dim,
                  kvd = (int64_t)c.n_kv_heads * c.head_dim, E = c.n_expert, F = c.n_ff_exp,
                  Fs = c.n_ff_shexp, V = c.n_vocab, hd = c.head_dim;
    struct Want { std::vector<int64_t> dims; bool quant; bool required; bool flt = false; };
    std::map<std::string, Want> want;
    // the embedding table: a quant type, or f32/f16, as MoeModel::load admits
    // (moe.rs:1107-1112, f32/f16/q8_0/q4_K; q5_K/q6_K decode here as well)
    want["token_embd.weight"] = {{H, V}, true, true, true};
    want["output.weight"] = {{H, V}, true, true};
    want["output_norm.weight"] = {{H}, false, true};
    for (int l = 0; l < c.n_layers; l++) {
        want[blk(l, "attn_norm")] = {{H}, false, true};
        want[blk(l, "attn_q_norm")] = {{hd}, false, false};
        want[blk(l, "attn_k_norm")] = {{hd}, false, false};
        want[blk(l, "ffn_norm")] = {{H}, false, true};
        want[blk(l, "attn_q")] = {{H, qd}, true, true};
        want[blk(l, "attn_k")] = {{H, kvd}, true, true};
        want[blk(l, "attn_v")] = {{H, kvd}, true, true};
        want[blk(l, "attn_output")] = {{qd, H}, true, true};
        want[blk(l, "ffn_gate_inp")] = {{H, E}, false, true};
        want["blk." + std::to_string(l) + ".ffn_gate_inp.bias"] = {{E}, false, false};
        want[blk(l, "ffn_gate_exps")] = {{H, F, E}, true, true};
        want[blk(l, "ffn_up_exps")] = {{H, F, E}, true, true};
        want[blk(l, "ffn_down_exps")] = {{F, H, E}, true, true};
        want[blk(l, "ffn_gate_shexp")] = {{H, Fs}, true, Fs > 0};
        want[blk(l, "ffn_up_shexp")] = {{H, Fs}, true, Fs > 0};
        want[blk(l, "ffn_down_shexp")] = {{Fs, H}, true, Fs > 0};
        want[blk(l, "ffn_gate_inp_shexp")] = {{H}, false, Fs > 0};
    }
    std::map<std::string, int> seen;
    std::vector<TensorSpec> used;
    for (const TensorSpec &t : specs) {
        auto it = want.find(t.name);
        if (it == want.end()) continue;
        used.push_back(t);
        if (seen[t.name]++) return fail(STYX_E_FORMAT, t.name + ": tensor listed twice");
        const Want &w = it->second;
        if (w.quant ? !(is_quant(t.type) || (w.flt && (t.type == T_F32 || t.type == T_F16)))
                    : t.type != T_F32)
            return fail(STYX_E_FORMAT,
                        t.name + (w.quant ? (w.flt ? ": type must be f32/f16/q8_0/q4_K/q5_K/q6_K"
                                                   : ": matrix type must be q8_0/q4_K/q5_K/q6_K")
                                          : ": expected f32"));
        if (t.dims != w.dims) {
            std::string d, e;
            for (auto v : t.dims) d += (d.empty() ? "" : ",") + std::to_string(v);
            for (auto v : w.dims) e += (e.empty() ? "" : ",") + std::to_string(v);
            return fail(STYX_E_FORMAT, t.name + ": dims [" + d + "] do not match the hparams [" + e + "]");
        }
    }
    for (auto &kv : want)
        if (kv.second.required && !seen.count(kv.first))
            return fail(STYX_E_FORMAT, "missing tensor " + kv.first);
    specs.swap(used);
    return STYX_OK;
}

// Hyperparameters the kernels support (the reference's own caps: k <= 16,
// moe.rs:587; E <= 512, moe.rs:3), checked before anything is allocated.
int check_cfg(const styx_moe_synth_cfg &c)
{
    if (c.n_layers < 1 || c.n_layers > 4096 || c.n_vocab < 1)
        return fail(STYX_E_INVALID, "n_layers must be in [1, 4096] and n_vocab positive");
    if (c.n_expert_used < 1 || c.n_expert_used > MAX_TOPK) return fail(STYX_E_INVALID, "n_expert_used must be in [1, 16] (moe.rs:587)");
    if (c.n_expert < c.n_expert_used || c.n_expert > MAX_EXPERTS || c.n_expert % 16) return fail(STYX_E_INVALID, "n_expert must be a multiple of 16 in [k, 512]");
    if (c.n_kv_heads < 1 || c.n_heads < 1 || c.n_heads > 1024 || c.n_heads % c.n_kv_heads || c.n_heads / c.n_kv_heads > 16) return fail(STYX_E_INVALID, "bad head counts");
    if (c.head_dim != 64 && c.head_dim != 128 && c.head_dim != 256) return fail(STYX_E_INVALID, "head_dim must be 64, 128 or 256");
    {
        const int gqa = c.n_heads / c.n_kv_heads, nhg = gqa % 4 == 0 ? 4 : gqa % 2 == 0 ? 2 : 1;
        if (gqa / nhg > 4) return fail(STYX_E_INVALID, "gqa must split into <= 4 heads per wave");
    }
    if (c.n_embd < 256 || c.n_embd % 256 || c.n_embd > XQ_MAX) return fail(STYX_E_INVALID, "n_embd must be a multiple of 256, <= 16384");
    if (c.n_heads * c.head_dim > XQ_MAX) return fail(STYX_E_INVALID, "n_head * head_dim must be <= 16384");
    if (c.n_ff_exp < 32 || c.n_ff_exp % 32 || c.n_ff_exp > 8192) return fail(STYX_E_INVALID, "expert FFN width must be a multiple of 32, <= 8192");
    if (c.n_ff_shexp < 0 || c.n_ff_shexp % 32 || c.n_ff_shexp > XQ_MAX) return fail(STYX_E_INVALID, "shared expert FFN width must be a multiple of 32, <= 16384");
    return STYX_OK;
}

// Common construction from a list of tensors with their sources.
int build_model(styx_moe *m, const styx_moe_synth_cfg &c, std::vector<TensorSpec> specs,
                const std::function<Source(const TensorSpec &)> &source,
                const std::vector<std::vector<std::pair<uint32_t, uint64_t>>> *hist)
{
    m->L = c.n_layers;
    m->H = c.n_embd;
    m->nh = c.n_heads;
    m->nkv = c.n_kv_heads;
    m->hd = c.head_dim;
    m->E = c.n_expert;
    m->K = c.n_expert_used;
    m->F = c.n_ff_exp;
    m->Fsh = c.n_ff_shexp;
    m->V = c.n_vocab;
    m->eps = c.rms_eps;
    m->rope_base = c.rope_base;
    m->norm_topk = 1;
    if (int r = check_cfg(c)) return r;
    if (int r = check_specs(c, specs)) return r;

    Builder b{m};
    int64_t mx = 0;
    for (auto &t : specs) mx = std::max(mx, spec_bytes(t));
    if (int r = m->alloc((void **)&b.tmp, (size_t)mx)) return r;
    b.tmp_size = (size_t)mx;
    const bool host_experts = m->opts.expert_budget_mb >= 0;
    m->layers.assign(m->L, Layer());
    for (auto &t : specs) {
        const Source src = source(t);
        const std::string &n = t.name;
        int l = -1;
        char role[64] = {0};
        if (sscanf(n.c_str(), "blk.%d.%63[^.]", &l, role) == 2 && l >= 0 && l < m->L) {
            Layer &ly = m->layers[l];
            const std::string r = role;
            int rc = 0;
            const bool is_bias = n.size() > 5 && n.compare(n.size() - 5, 5, ".bias") == 0;
            if (r == "attn_norm") rc = b.f32(t, src, &ly.attn_norm);
            else if (r == "attn_q_norm") rc = b.f32(t, src, &ly.q_norm);
            else if (r == "attn_k_norm") rc = b.f32(t, src, &ly.k_norm);
            else if (r == "ffn_norm") rc = b.f32(t, src, &ly.ffn_norm);
            else if (r == "ffn_gate_inp" && is_bias) rc = b.f32(t, src, &ly.router_bias);
            else if (r == "ffn_gate_inp") rc = b.f32(t, src, &ly.router);
            else if (r == "ffn_gate_inp_shexp") rc = b.f32(t, src, &ly.gate_inp_sh);
            else if (r == "attn_q") rc = b.mat(t, src, ly.wq, false);
            else if (r == "attn_k") rc = b.mat(t, src, ly.wk, false);
            else if (r == "attn_v") rc = b.mat(t, src, ly.wv, false);
            else if (r == "attn_output") rc = b.mat(t, src, ly.wo, false);
            else if (r == "ffn_gate_exps") rc = b.mat(t, src, ly.gate, host_experts);
            else if (r == "ffn_up_exps") rc = b.mat(t, src, ly.up, host_experts);
            else if (r == "ffn_down_exps") rc = b.mat(t, src, ly.down, host_experts);
            else if (r == "ffn_gate_shexp") rc = b.mat(t, src, ly.gsh, false);
            else if (r == "ffn_up_shexp") rc = b.mat(t, src, ly.ush, false);
            else if (r == "ffn_down_shexp") rc = b.mat(t, src, ly.dsh, false);
            if (rc) return rc;
        } else if (n == "token_embd.weight") {
            if (int r = b.mat(t, src, m->embd, false, true)) return r;
        } else if (n == "output.weight") {
            if (int r = b.mat(t, src, m->head, false)) return r;
        } else if (n == "output_norm.weight") {
            if (int r = b.f32(t, src, &m->out_norm)) return r;
        }
        STYX_HIP(hipStreamSynchronize(m->gpu->stream));
    }
    STYX_HIP(hipFree(b.tmp));
    m->dev_allocs.erase(std::find(m->dev_allocs.begin(), m->dev_allocs.end(), (void *)b.tmp));
    // completeness / shape checks
    if (!m->embd.dev || !m->head.dev || !m->out_norm) return fail(STYX_E_FORMAT, "missing token_embd/output/output_norm");
    for (int l = 0; l < m->L; l++) {
        Layer &ly = m->layers[l];
        const std::string p = "blk." + std::to_string(l) + ": ";
        if (!ly.attn_norm || !ly.ffn_norm || !ly.router || !ly.wq.slab || !ly.wk.slab ||
            !ly.wv.slab || !ly.wo.slab || !ly.gate.slab || !ly.up.slab || !ly.down.slab)
            return fail(STYX_E_FORMAT, p + "missing tensor");
        if (ly.wq.rows != m->nh * m->hd || ly.wk.rows != m->nkv * m->hd || ly.wv.rows != m->nkv * m->hd ||
            ly.wo.rows != m->H || ly.wo.cols != m->nh * m->hd || ly.wq.cols != m->H)
            return fail(STYX_E_FORMAT, p + "attention shapes do not match hparams");
        if (ly.gate.nmat != m->E || ly.gate.rows != m->F || ly.gate.cols != m->H ||
            ly.up.nmat != m->E || ly.up.rows != m->F || ly.down.nmat != m->E ||
            ly.down.rows != m->H || ly.down.cols != m->F)
            return fail(STYX_E_FORMAT, p + "expert shapes do not match hparams");
        if (blk_elems(ly.gate.type) != blk_elems(ly.up.type))
            return fail(STYX_E_UNSUPPORTED, p + "gate/up block sizes differ");
        if (m->Fsh > 0 && (!ly.gsh.dev || !ly.ush.dev || !ly.dsh.dev || !ly.gate_inp_sh))
            return fail(STYX_E_FORMAT, p + "missing shared-expert tensor");
        if (!pick_geo(ly.down.type, m->F).G || !pick_geo(ly.gate.type, m->H).G ||
            !pick_geo(ly.wo.type, m->nh * m->hd).G)
            return fail(STYX_E_UNSUPPORTED, p + "no kernel geometry for these shapes");
    }
    const Layer &l0 = m->layers[0];
    m->slab_bytes = l0.gate.slab + l0.up.slab + l0.down.slab;
    if (int r = m->place_experts(hist)) return r;
    if (int r = m->setup_runtime()) return r;
    if (int r = m->size_moe_block()) return r;
    if (int r = m->build_graphs()) return r;
    return STYX_OK;
}

// Router bias by popularity rank for a Zipf(s) skew under top-k routing.
// Zipf popularity cannot be met exactly by top-k selection (for s = 1.1,
// k = 8, E = 128 the top expert would need 1.8 picks per token), so the
// target is the closest feasible one: the expert of rank r is picked with
// probability pi_r = min(1, lambda * r^-s) per token, lambda such that the
// pi sum to k (the top expert is then picked on every token, the rest
// follow r^-s).  The biases are fitted on a seeded sample of 4096 tokens of
// router logit noise, N(0, sd^2) per expert and token (the synthetic
// router: weights N(0, sigma), unit-RMS normalised input, so
// sd = sigma * sqrt(H)): each round counts the top-k picks of bias + noise
// and moves log-popularity toward log pi.  Deterministic in the seed;
// entry 0 (rank 1) is 0.
std::vector<float> zipf_bias_table(int E, int k, double s, double sd, uint64_t seed)
{
    std::vector<double> z(E), pi(E), b(E);
    for (int r = 0; r < E; r++) z[r] = std::pow(r + 1.0, -s);
    double lo = 0.0, hi = 1e9;
    for (int it = 0; it < 200; it++) {
        const double mid = 0.5 * (lo + hi);
        double sum = 0.0;
        for (double v : z) sum += std::min(1.0, mid * v);
        (sum < k ? lo : hi) = mid;
    }
    for (int r = 0; r < E; r++) pi[r] = std::min(1.0, hi * z[r]);
    const int T = 4096;
    std::vector<float> noise((size_t)T * E);
    uint64_t st = seed;
    for (size_t i = 0; i < noise.size(); i += 2) {
        const double u1 = ((double)(splitmix(st) >> 11) + 1.0) * 0x1p-53;
        const double u2 = (double)(splitmix(st) >> 11) * 0x1p-53;
        const double rr = std::sqrt(-2.0 * std::log(u1));
        noise[i] = (float)(sd * rr * std::cos(6.283185307179586 * u2));
        if (i + 1 < noise.size()) noise[i + 1] = (float)(sd * rr * std::sin(6.283185307179586 * u2));
    }
    for (int r = 0; r < E; r++) b[r] = sd * std::log(pi[r]);
    std::vector<int> cnt(E);
    std::vector<std::pair<float, int>> row(E);
    for (int it = 0; it < 300; it++) {
        std::fill(cnt.begin(), cnt.end(), 0);
        for (int t = 0; t < T; t++) {
            for (int e = 0; e < E; e++) row[e] = {(float)b[e] + noise[(size_t)t * E + e], e};
            std::nth_element(row.begin(), row.begin() + (k - 1), row.end(),
                             [](const std::pair<float, int> &x, const std::pair<float, int> &y) {
                                 return x.first > y.first || (x.first == y.first && x.second < y.second);
                             });
            for (int i = 0; i < k; i++) cnt[row[i].second]++;
        }
        for (int r = 0; r < E; r++) {
            const double p = std::max((double)cnt[r], 0.5) / T;
            b[r] += 0.3 * sd * (std::log(pi[r]) - std::log(p));
        }
    }
    // popularity falls with rank: the tail's few picks per round leave
    // sampling noise, which a running minimum removes
    for (int r = 1; r < E; r++) b[r] = std::min(b[r], b[r - 1]);
    std::vector<float> out(E);
    for (int r = 0; r < E; r++) out[r] = (float)(b[r] - b[0]);
    return out;
}

int read_hist(const char *path, int L, std::vector<std::vector<std::pair<uint32_t, uint64_t>>> &h)
{
    std::ifstream f(path);
    if (!f) return fail(STYX_E_IO, std::string("cannot read expert histogram ") + path);
    h.assign(L, {});
    std::string line;
    std::getline(f, line);  // header
    while (std::getline(f, line)) {
        int l;
        unsigned e;
        unsigned long long hits;
        if (sscanf(line.c_str(), "%d,%u,%llu", &l, &e, &hits) == 3 && l >= 0 && l < L)
            h[l].push_back({e, hits});
    }
    return STYX_OK;
}

}  // namespace

// ------------------------------------------------------------------ C ABI --
extern "C" {

int styx_residency_plan(const char *hist_csv, int n_layers, int n_expert,
                        const uint64_t *slab_bytes, int64_t budget_mb, uint32_t *remap,
                        uint64_t *pinned_slabs)
{
    if (n_layers < 1 || n_expert < 1 || !slab_bytes || !remap || budget_mb < 0)
        return fail(STYX_E_INVALID, "styx_residency_plan: bad argument");
    std::vector<std::vector<std::pair<uint32_t, uint64_t>>> hist;
    if (hist_csv)
        if (int r = read_hist(hist_csv, n_layers, hist)) return r;
    std::vector<uint64_t> slab(slab_bytes, slab_bytes + n_layers), layer(n_layers);
    for (int l = 0; l < n_layers; l++) layer[l] = slab[l] * (uint64_t)n_expert;
    std::vector<std::vector<uint32_t>> hot;
    plan_hot_experts(hist_csv ? &hist : nullptr, n_layers, n_expert, slab, layer,
                     (uint64_t)budget_mb << 20, hot);
    uint64_t n = 0;
    for (int l = 0; l < n_layers; l++) {
        for (int e = 0; e < n_expert; e++) remap[(size_t)l * n_expert + e] = SKIP;
        for (size_t i = 0; i < hot[l].size(); i++) remap[(size_t)l * n_expert + hot[l][i]] = (uint32_t)i;
        n += hot[l].size();
    }
    if (pinned_slabs) *pinned_slabs = n;
    return STYX_OK;
}

int styx_zipf_bias_table(int n_expert, int k, float s, float sd, uint64_t seed, float *out)
{
    if (n_expert < 1 || k < 1 || k > n_expert || !(s > 0) || !(sd > 0) || !out)
        return fail(STYX_E_INVALID, "styx_zipf_bias_table: bad argument");
    const std::vector<float> t = zipf_bias_table(n_expert, k, s, sd, seed);
    std::copy(t.begin(), t.end(), out);
    return STYX_OK;
}

int styx_repin_select(const uint64_t *hits, int n_expert, const uint32_t *slot_experts,
                      int n_slots, int repin_max, uint32_t *swap_slot, uint32_t *swap_expert,
                      int *n_swaps)
{
    if (!hits || n_expert < 1 || n_slots < 0 || n_slots > n_expert || (n_slots && !slot_experts) ||
        !n_swaps || (repin_max > 0 && (!swap_slot || !swap_expert)))
        return fail(STYX_E_INVALID, "styx_repin_select: bad argument");
    std::vector<char> resident(n_expert, 0);
    for (int i = 0; i < n_slots; i++) {
        if (slot_experts[i] >= (uint32_t)n_expert || resident[slot_experts[i]])
            return fail(STYX_E_INVALID, "styx_repin_select: slot experts must be distinct ids < n_expert");
        resident[slot_experts[i]] = 1;
    }
    std::vector<std::pair<int, uint32_t>> swaps;
    repin_select(hits, n_expert, slot_experts, n_slots, resident, std::max(repin_max, 0), swaps);
    for (size_t i = 0; i < swaps.size(); i++) {
        swap_slot[i] = (uint32_t)swaps[i].first;
        swap_expert[i] = swaps[i].second;
    }
    *n_swaps = (int)swaps.size();
    return STYX_OK;
}

static styx_moe_opts default_opts()
{
    styx_moe_opts o{};
    o.n_ctx = 4096;
    o.use_graph = 1;
    o.expert_budget_mb = -1;
    o.arena = 1;
    o.repin_max = 2;
    return o;
}

int styx_moe_synth(styx_gpu *gpu, const styx_moe_synth_cfg *cfg, const styx_moe_opts *opts,
                   styx_moe **out)
{
    if (!gpu || !cfg || !out) return fail(STYX_E_INVALID, "styx_moe_synth: NULL argument");
    STYX_HIP(hipSetDevice(gpu->device));
    auto m = std::make_unique<styx_moe>();
    m->gpu = gpu;
    gpu->live_children++;
    m->opts = opts ? *opts : default_opts();
    m->n_ctx = m->opts.n_ctx > 0 ? m->opts.n_ctx : 4096;
    const styx_moe_synth_cfg c = *cfg;
    auto specs = model_specs(c);
    // router bias for Zipf-skewed routing: the bias of rank r from a table
    // calibrated to the synthetic router's logit spread, ranks a seeded
    // permutation per layer.  The spread is sigma * sqrt(H) (unit-RMS
    // input) times ZIPF_SPREAD, set on the 30B-A3B shape from the routing
    // of tokens drawn at random: the router logits there are not i.i.d.
    // across tokens (each expert has a persistent offset), and a table for
    // 0.9x the i.i.d. spread gives a fitted popularity exponent of 1.17
    // over the unsaturated ranks (1.0x: 1.45, 1.05x: 1.54)
    constexpr double ZIPF_SPREAD = 0.9;
    std::vector<std::vector<float>> biases(c.n_layers);
    if (c.router_zipf_s > 0) {
        const std::vector<float> tab =
            zipf_bias_table(c.n_expert, c.n_expert_used, c.router_zipf_s,
                            (double)c.sigma * std::sqrt((double)c.n_embd) * ZIPF_SPREAD,
                            c.seed ^ 0x5A1Full);
        for (int l = 0; l < c.n_layers; l++) {
            std::vector<int> rank(c.n_expert);
            std::iota(rank.begin(), rank.end(), 1);
            uint64_t s = c.seed ^ fnv1a64("zipf." + std::to_string(l));
            for (int i = c.n_expert - 1; i > 0; i--) std::swap(rank[i], rank[splitmix(s) % (i + 1)]);
            biases[l].resize(c.n_expert);
            for (int e = 0; e < c.n_expert; e++) biases[l][e] = tab[rank[e] - 1];
        }
    }
    auto source = [&](const TensorSpec &t) {
        Source s;
        s.seed = c.seed ^ fnv1a64(t.name);
        const bool norm = t.name.find("norm") != std::string::npos;
        if (t.type == T_F32 && norm) {
            s.mean = 1.0f;
            s.sigma = 0.0f;
        } else {
            s.sigma = c.sigma;
        }
        int l;
        if (t.name.find(".ffn_gate_inp.bias") != std::string::npos &&
            sscanf(t.name.c_str(), "blk.%d.", &l) == 1)
            s.values = &biases[l];
        return s;
    };
    std::vector<std::vector<std::pair<uint32_t, uint64_t>>> hist;
    if (m->opts.expert_hist) {
        if (int r = read_hist(m->opts.expert_hist, c.n_layers, hist)) return r;
    }
    if (int r = build_model(m.get(), c, specs, source, m->opts.expert_hist ? &hist : nullptr)) return r;
    *out = m.release();
    return STYX_OK;
}

}  // extern "C"

namespace {

// Everything MoeModel::load checks before it touches the device: the GGUF
// header (gguf-rs semantics), the qwen3moe hyperparameters, that every
// tensor's bytes lie inside the file, and every tensor the model reads
// against the dims its hyperparameters imply.  On success c holds the
// hyperparameters and specs the tensors to upload.
int parse_model_file(const char *path, Gguf &g, styx_moe_synth_cfg &c,
                     std::vector<TensorSpec> &specs)
{
    std::string err;
    if (!gguf_open(path, g, err)) return fail(STYX_E_FORMAT, std::string("gguf: ") + err);
    std::string arch;
    if (!g.get_str("general.architecture", arch))
        return fail(STYX_E_FORMAT, "missing general.architecture");
    if (arch != "qwen3moe")
        return fail(STYX_E_UNSUPPORTED, "unsupported architecture '" + arch + "' (qwen3moe only)");
    c = styx_moe_synth_cfg{};
    uint32_t u;
    auto need = [&](const std::string &k, int &dst) -> bool {
        if (!g.get_u32(arch + "." + k, u)) return false;
        dst = u > (uint32_t)INT32_MAX ? -1 : (int)u;
        return true;
    };
    if (!need("block_count", c.n_layers) || !need("embedding_length", c.n_embd) ||
        !need("attention.head_count", c.n_heads) || !need("attention.head_count_kv", c.n_kv_heads) ||
        !need("expert_count", c.n_expert) || !need("expert_used_count", c.n_expert_used))
        return fail(STYX_E_FORMAT, "missing qwen3moe hyperparameter metadata");
    if (!need("attention.key_length", c.head_dim)) c.head_dim = c.n_heads > 0 ? c.n_embd / c.n_heads : 0;
    auto dim_int = [](uint64_t d) { return d > (uint64_t)INT32_MAX ? -1 : (int)d; };
    if (!need("expert_feed_forward_length", c.n_ff_exp)) {
        const GgufTensor *t = g.find("blk.0.ffn_gate_exps.weight");
        if (!t || t->dims.size() < 2) return fail(STYX_E_FORMAT, "no expert_feed_forward_length and no ffn_gate_exps");
        c.n_ff_exp = dim_int(t->dims[1]);
    }
    if (!g.get_f32(arch + ".attention.layer_norm_rms_epsilon", c.rms_eps) ||
        !g.get_f32(arch + ".rope.freq_base", c.rope_base))
        return fail(STYX_E_FORMAT, "missing rms epsilon / rope base");
    const GgufTensor *te = g.find("token_embd.weight");
    if (!te || te->dims.size() != 2) return fail(STYX_E_FORMAT, "missing token_embd.weight");
    c.n_vocab = dim_int(te->dims[1]);
    if (const GgufTensor *ts = g.find("blk.0.ffn_gate_shexp.weight"))
        c.n_ff_shexp = ts->dims.size() == 2 ? dim_int(ts->dims[1]) : -1;
    if (check_cfg(c)) return fail(STYX_E_FORMAT, styx_last_error());
    struct stat stb;
    if (stat(path, &stb) != 0) return fail(STYX_E_IO, std::string("stat ") + path);
    const uint64_t len = (uint64_t)stb.st_size;
    specs.clear();
    for (auto &t : g.tensors) {
        // no sum of the three can wrap: each term is checked against what is left
        if (g.data_start > len || t.offset > len - g.data_start ||
            t.size_bytes > len - g.data_start - t.offset)
            return fail(STYX_E_FORMAT, t.name + ": tensor data past end of file");
        TensorSpec sp{t.name, (int)t.ggml_type, {}};
        for (auto d : t.dims) sp.dims.push_back(d > (uint64_t)INT64_MAX ? -1 : (int64_t)d);
        specs.push_back(sp);
    }
    return check_specs(c, specs);
}

}  // namespace

extern "C" {

int styx_moe_check_file(const char *path, styx_moe_hparams *out)
{
    if (!path) return fail(STYX_E_INVALID, "styx_moe_check_file: NULL path");
    Gguf g;
    styx_moe_synth_cfg c;
    std::vector<TensorSpec> specs;
    if (int r = parse_model_file(path, g, c, specs)) return r;
    if (out) {
        *out = styx_moe_hparams{};
        out->n_layers = c.n_layers;
        out->n_embd = c.n_embd;
        out->n_heads = c.n_heads;
        out->n_kv_heads = c.n_kv_heads;
        out->head_dim = c.head_dim;
        out->n_expert = c.n_expert;
        out->n_expert_used = c.n_expert_used;
        out->n_ff_exp = c.n_ff_exp;
        out->n_ff_shexp = c.n_ff_shexp;
        out->n_vocab = c.n_vocab;
        out->rms_eps = c.rms_eps;
        out->rope_base = c.rope_base;
        out->norm_topk = 1;
        for (const TensorSpec &t : specs)
            if (t.name == "blk.0.ffn_gate_exps.weight" || t.name == "blk.0.ffn_up_exps.weight" ||
                t.name == "blk.0.ffn_down_exps.weight")
                out->slab_bytes += (uint64_t)(spec_bytes(t) / c.n_expert);
    }
    return STYX_OK;
}

int styx_moe_load(styx_gpu *gpu, const char *path, const styx_moe_opts *opts, styx_moe **out)
{
    if (!gpu || !path || !out) return fail(STYX_E_INVALID, "styx_moe_load: NULL argument");
    Gguf g;
    styx_moe_synth_cfg c;
    std::vector<TensorSpec> specs;
    if (int r = parse_model_file(path, g, c, specs)) return r;
    STYX_HIP(hipSetDevice(gpu->device));
    // map the file
    int fd = open(path, O_RDONLY);
    if (fd < 0) return fail(STYX_E_IO, std::string("open ") + path);
    struct stat stb;
    if (fstat(fd, &stb) != 0) {
        close(fd);
        return fail(STYX_E_IO, std::string("fstat ") + path);
    }
    const size_t len = (size_t)stb.st_size;
    void *map = mmap(nullptr, len, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (map == MAP_FAILED) return fail(STYX_E_IO, std::string("mmap ") + path);
    struct Unmap { void *p; size_t n; ~Unmap() { munmap(p, n); } } unmap{map, len};
    // the file may have changed between the checks and the mapping
    for (const TensorSpec &t : specs) {
        const GgufTensor *gt = g.find(t.name);
        if (g.data_start > len || gt->offset > len - g.data_start ||
            gt->size_bytes > len - g.data_start - gt->offset)
            return fail(STYX_E_FORMAT, t.name + ": tensor data past end of file");
    }
    auto m = std::make_unique<styx_moe>();
    m->gpu = gpu;
    gpu->live_children++;
    m->opts = opts ? *opts : default_opts();
    m->n_ctx = m->opts.n_ctx > 0 ? m->opts.n_ctx : 4096;
    const uint8_t *data = (const uint8_t *)map + g.data_start;
    auto source = [&](const TensorSpec &t) {
        Source s;
        s.host = data + g.find(t.name)->offset;
        return s;
    };
    std::vector<std::vector<std::pair<uint32_t, uint64_t>>> hist;
    if (m->opts.expert_hist) {
        if (int r = read_hist(m->opts.expert_hist, c.n_layers, hist)) return r;
    }
    if (int r = build_model(m.get(), c, specs, source, m->opts.expert_hist ? &hist : nullptr)) return r;
    *out = m.release();
    return STYX_OK;
}

void styx_moe_free(styx_moe *m) { delete m; }

int styx_moe_get_hparams(const styx_moe *m, styx_moe_hparams *o)
{
    if (!m || !o) return fail(STYX_E_INVALID, "styx_moe_get_hparams: NULL argument");
    o->n_layers = m->L;
    o->n_embd = m->H;
    o->n_heads = m->nh;
    o->n_kv_heads = m->nkv;
    o->head_dim = m->hd;
    o->n_expert = m->E;
    o->n_expert_used = m->K;
    o->n_ff_exp = m->F;
    o->n_ff_shexp = m->Fsh;
    o->n_vocab = m->V;
    o->n_ctx = m->n_ctx;
    o->rms_eps = m->eps;
    o->rope_base = m->rope_base;
    o->norm_topk = m->norm_topk;
    o->slab_bytes = m->slab_bytes;
    o->expert_bytes_hbm = m->exp_hbm;
    o->expert_bytes_host = m->exp_host;
    o->unfused_fallbacks = m->fallbacks;
    return STYX_OK;
}

int styx_moe_forward_token(styx_moe *m, uint32_t token, float *logits_out)
{
    if (!m) return fail(STYX_E_INVALID, "styx_moe_forward_token: NULL model");
    if (m->n_past >= m->n_ctx)
        return fail(STYX_E_STATE, "KV arena full (" + std::to_string(m->n_ctx) + ")");
    if (token >= (uint32_t)m->V) return fail(STYX_E_INVALID, "token id out of range");
    if (!m->broken.empty()) return fail(STYX_E_STATE, m->broken);
    STYX_HIP(hipSetDevice(m->gpu->device));
    if (m->n_past > 0)
        if (int r = m->maybe_repin()) return r;
    if (int r = m->ensure_pages(m->n_past)) return r;
    m->h_stage[0] = token;
    m->h_stage[1] = (uint32_t)m->n_past;
    STYX_HIP(hipMemcpyAsync(m->d_tok, &m->h_stage[0], 4, hipMemcpyHostToDevice, m->gpu->stream));
    STYX_HIP(hipMemcpyAsync(m->d_pos, &m->h_stage[1], 4, hipMemcpyHostToDevice, m->gpu->stream));
    if (int r = m->run_token(false)) return r;
    m->n_past++;
    if (logits_out)
        STYX_HIP(hipMemcpyAsync(logits_out, m->logits, sizeof(float) * m->V, hipMemcpyDeviceToHost,
                                m->gpu->stream));
    m->queue_abort_read();
    STYX_HIP(hipStreamSynchronize(m->gpu->stream));
    if (m->check_abort()) {
        // the token again (same token and position, still in the stage), on
        // the separate kernels
        if (int r = m->fall_back_unfused()) return r;
        if (int r = m->collect_stats()) return r;
        m->n_past--;
        STYX_HIP(hipMemcpyAsync(m->d_tok, &m->h_stage[0], 4, hipMemcpyHostToDevice, m->gpu->stream));
        STYX_HIP(hipMemcpyAsync(m->d_pos, &m->h_stage[1], 4, hipMemcpyHostToDevice, m->gpu->stream));
        if (int r = m->run_token(false)) return r;
        m->n_past++;
        if (logits_out)
            STYX_HIP(hipMemcpyAsync(logits_out, m->logits, sizeof(float) * m->V,
                                    hipMemcpyDeviceToHost, m->gpu->stream));
        STYX_HIP(hipStreamSynchronize(m->gpu->stream));
    }
    return m->collect_stats();
}

int styx_moe_decode(styx_moe *m, int n_steps, uint32_t *out)
{
    if (!m || n_steps < 0 || (n_steps && !out)) return fail(STYX_E_INVALID, "styx_moe_decode: bad argument");
    if (m->n_past < 1) return fail(STYX_E_STATE, "styx_moe_decode: no token forwarded yet");
    if (m->n_past + n_steps > m->n_ctx) return fail(STYX_E_STATE, "styx_moe_decode: exceeds n_ctx");
    if (n_steps == 0) return STYX_OK;
    if (!m->broken.empty()) return fail(STYX_E_STATE, m->broken);
    STYX_HIP(hipSetDevice(m->gpu->device));
    const int start = m->n_past;  // position of the pending (argmax) token
    if (int r = m->ensure_pages(start + n_steps - 1)) return r;
    m->h_stage[1] = (uint32_t)start;
    STYX_HIP(hipMemcpyAsync(m->d_pos, &m->h_stage[1], 4, hipMemcpyHostToDevice, m->gpu->stream));
    // the pending token, for a run again after a fused launch gives up
    // (every step's argmax overwrites it)
    if (!m->opts.no_fuse)
        STYX_HIP(hipMemcpyAsync(m->tok_save, m->d_tok, 4, hipMemcpyDeviceToDevice, m->gpu->stream));
    const bool host_work = (m->opts.repin_interval > 0 && m->any_host) || m->opts.time_kernels;
    // With host work between tokens every step is waited for anyway, so a
    // fused launch that gives up is caught at its own step: the steps before
    // it stand (with the repins and hit counts they made), and that step
    // runs again on the separate kernels without repinning a second time --
    // host state then matches a run that never fell back.
    bool again = false;
    for (int i = 0; i < n_steps; i++) {
        if (host_work) {
            // host bookkeeping between tokens needs the previous token done
            // (as forward_token, the first step repins for the token before)
            STYX_HIP(hipStreamSynchronize(m->gpu->stream));
            if (!again)
                if (int r = m->maybe_repin()) return r;
            if (int r = m->collect_stats()) return r;
        }
        again = false;
        if (int r = m->run_token(true)) return r;
        m->n_past++;
        if (host_work && !m->opts.no_fuse) {
            m->queue_abort_read();
            STYX_HIP(hipStreamSynchronize(m->gpu->stream));
            if (m->check_abort()) {
                if (int r = m->fall_back_unfused()) return r;
                m->n_past--;
                m->h_stage[1] = (uint32_t)m->n_past;
                STYX_HIP(hipMemcpyAsync(m->d_pos, &m->h_stage[1], 4, hipMemcpyHostToDevice,
                                        m->gpu->stream));
                // the step's input token: the pending one, or the previous step's
                STYX_HIP(hipMemcpyAsync(m->d_tok, i == 0 ? m->tok_save : m->hist + start + i, 4,
                                        hipMemcpyDeviceToDevice, m->gpu->stream));
                again = true;
                i--;
            }
        }
    }
    STYX_HIP(hipMemcpyAsync(out, m->hist + start + 1, sizeof(uint32_t) * n_steps,
                            hipMemcpyDeviceToHost, m->gpu->stream));
    m->queue_abort_read();
    STYX_HIP(hipStreamSynchronize(m->gpu->stream));
    if (m->check_abort()) {
        // the steps again from the pending token, on the separate kernels
        // (no host work ran between them, so no host state to restore)
        if (int r = m->fall_back_unfused()) return r;
        if (int r = m->collect_stats()) return r;
        m->n_past = start;
        STYX_HIP(hipMemcpyAsync(m->d_tok, m->tok_save, 4, hipMemcpyDeviceToDevice, m->gpu->stream));
        return styx_moe_decode(m, n_steps, out);
    }
    return m->collect_stats();
}

int styx_moe_generate(styx_moe *m, const uint32_t *prompt, int n_prompt, int n_predict,
                      uint32_t *out, double *prefill_s, double *decode_s)
{
    if (!m || !prompt || n_prompt < 1 || n_predict < 1 || !out)
        return fail(STYX_E_INVALID, "styx_moe_generate: bad argument");
    if (m->n_past + n_prompt + n_predict - 1 > m->n_ctx)
        return fail(STYX_E_STATE, "prompt + generation exceeds n_ctx");
    using clk = std::chrono::steady_clock;
    const auto t0 = clk::now();
    for (int i = 0; i < n_prompt; i++)
        if (int r = styx_moe_forward_token(m, prompt[i], nullptr)) return r;
    const auto t1 = clk::now();
    // the first generated token is the prefill's argmax, already on device
    STYX_HIP(hipMemcpy(out, m->d_tok, 4, hipMemcpyDeviceToHost));
    if (int r = styx_moe_decode(m, n_predict - 1, out + 1)) return r;
    const auto t2 = clk::now();
    if (prefill_s) *prefill_s = std::chrono::duration<double>(t1 - t0).count();
    if (decode_s) *decode_s = std::chrono::duration<double>(t2 - t1).count();
    return STYX_OK;
}

// Stage timing (measurement, no reference counterpart): the launches of one
// stage for every layer of the last token, captured as one graph and replayed
// back to back between two HIP events.  Each layer's launch reads its own
// weights, so the replays stream as much memory as a token does for that
// stage.  The replays overwrite per-token scratch (ids rows, partials, the
// residual and the KV row at the pending position), all of which the next
// token rewrites before reading; argmax, which advances the decode state, is
// not a stage here.
int styx_moe_time_stage(styx_moe *m, const char *stage, int reps, double *us_per_replay,
                        int *launches)
{
    static const char *const ok[] = {"embed",    "qkv",    "attn",        "o_proj",
                                     "router",   "gather", "moe_gate_up", "shexp",
                                     "moe_down", "reduce", "moe_block",   "lm_head"};
    if (!m || !stage || reps < 1 || !us_per_replay)
        return fail(STYX_E_INVALID, "styx_moe_time_stage: bad argument");
    if (std::find_if(std::begin(ok), std::end(ok), [&](const char *s) { return !strcmp(s, stage); }) ==
        std::end(ok))
        return fail(STYX_E_INVALID, std::string("styx_moe_time_stage: unknown stage ") + stage);
    if (m->n_past < 1) return fail(STYX_E_STATE, "styx_moe_time_stage: run a token first");
    STYX_HIP(hipSetDevice(m->gpu->device));
    if (int r = m->collect_stats()) return r;
    hipStream_t st = m->gpu->stream;
    const int saved = m->opts.time_kernels;
    m->opts.time_kernels = 0;
    m->stage_only = stage;
    // at least 32 launches per graph: a shallow model's stage is repeated so
    // that the graph launch itself does not dominate
    const int nrep = std::max(1, 32 / std::max(1, m->L));
    hipGraph_t g = nullptr;
    hipError_t e = hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal);
    int r = STYX_OK;
    const int mode = m->attn_mode(m->n_past);  // the last token's context
    for (int i = 0; i < nrep && e == hipSuccess && !r; i++) r = m->enqueue_token(false, mode);
    hipError_t e2 = e == hipSuccess ? hipStreamEndCapture(st, &g) : e;
    m->stage_only.clear();
    m->opts.time_kernels = saved;
    if (r) {
        if (g) hipGraphDestroy(g);
        return r;
    }
    if (e2 != hipSuccess) return hip_fail(e2, "styx_moe_time_stage: capture");
    size_t n = 0;
    e = hipGraphGetNodes(g, nullptr, &n);
    hipGraphExec_t ex = nullptr;
    if (e == hipSuccess) e = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
    hipGraphDestroy(g);
    if (e != hipSuccess) return hip_fail(e, "styx_moe_time_stage: instantiate");
    hipEvent_t a = nullptr, b = nullptr;
    float ms = 0.0f;
    e = hipEventCreate(&a);
    if (e == hipSuccess) e = hipEventCreate(&b);
    for (int i = 0; i < 2 && e == hipSuccess; i++) e = hipGraphLaunch(ex, st);
    if (e == hipSuccess) e = hipEventRecord(a, st);
    for (int i = 0; i < reps && e == hipSuccess; i++) e = hipGraphLaunch(ex, st);
    if (e == hipSuccess) e = hipEventRecord(b, st);
    if (e == hipSuccess) m->queue_abort_read();
    if (e == hipSuccess) e = hipEventSynchronize(b);
    if (e == hipSuccess) e = hipEventElapsedTime(&ms, a, b);
    if (a) hipEventDestroy(a);
    if (b) hipEventDestroy(b);
    hipGraphExecDestroy(ex);
    if (e != hipSuccess) return hip_fail(e, "styx_moe_time_stage: replay");
    // LM-head replays leave their maximum in the argmax word: cleared before
    // the next token's head adds to it
    STYX_HIP(hipMemsetAsync(m->am_word, 0, sizeof(unsigned long long), st));
    STYX_HIP(hipStreamSynchronize(st));
    if (int rr = m->check_abort()) return rr;
    *us_per_replay = 1000.0 * ms / reps / nrep;
    if (launches) *launches = (int)(n / nrep);
    return STYX_OK;
}

// Phase stamps of the fused MoE block from the last timed token
// (measurement, no reference counterpart): [n_layers][nwg][16] wall-clock
// ticks (0 where a workgroup had no such phase).
int styx_moe_moe_block_trace(styx_moe *m, uint64_t *out, int64_t max_count, int *nwg,
                             double *ticks_per_us)
{
    if (!m || !nwg) return fail(STYX_E_INVALID, "styx_moe_moe_block_trace: bad argument");
    *nwg = m->mb_nwg > 0 ? m->mb_nwg : 0;
    if (*nwg == 0 || !out) return STYX_OK;
    const int64_t n = (int64_t)m->L * m->mb_nwg * 16;
    if (max_count < n) return fail(STYX_E_INVALID, "styx_moe_moe_block_trace: buffer too small");
    STYX_HIP(hipSetDevice(m->gpu->device));
    STYX_HIP(hipStreamSynchronize(m->gpu->stream));
    STYX_HIP(hipMemcpy(out, m->mb_trace, sizeof(uint64_t) * n, hipMemcpyDeviceToHost));
    if (ticks_per_us) {
        int khz = 0;
        STYX_HIP(hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, m->gpu->device));
        *ticks_per_us = khz / 1000.0;
    }
    return STYX_OK;
}

// Phase stamps of the attention launches from the last timed token
// (measurement, no reference counterpart): [n_layers][max_chunks * n_kv]
// [8] wall-clock ticks, 0 for workgroups past the context; slot 7 names the
// workgroup ((kv head << 16 | chunk) + 1), slot 6 holds the active chunks.
int styx_moe_attn_trace(styx_moe *m, uint64_t *out, int64_t max_count, int *nwg,
                        double *ticks_per_us)
{
    if (!m || !nwg) return fail(STYX_E_INVALID, "styx_moe_attn_trace: bad argument");
    *nwg = m->at_trace ? m->max_chunks * m->nkv : 0;
    if (*nwg == 0 || !out) return STYX_OK;
    const int64_t n = (int64_t)m->L * *nwg * AT_TRACE;
    if (max_count < n) return fail(STYX_E_INVALID, "styx_moe_attn_trace: buffer too small");
    STYX_HIP(hipSetDevice(m->gpu->device));
    STYX_HIP(hipStreamSynchronize(m->gpu->stream));
    STYX_HIP(hipMemcpy(out, m->at_trace, sizeof(uint64_t) * n, hipMemcpyDeviceToHost));
    if (ticks_per_us) {
        int khz = 0;
        STYX_HIP(hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, m->gpu->device));
        *ticks_per_us = khz / 1000.0;
    }
    return STYX_OK;
}

// The fused launches' wait bound (styx_moe_opts.max_polls) for the
// following tokens; the captured graphs are rebuilt with it (test helper, no
// reference counterpart: a tiny bound forces the fall back to the separate
// kernels from the host, with every kernel still ending normally).
int styx_moe_set_wait_limit(styx_moe *m, int max_polls)
{
    if (!m || max_polls < 0) return fail(STYX_E_INVALID, "styx_moe_set_wait_limit: bad argument");
    STYX_HIP(hipSetDevice(m->gpu->device));
    STYX_HIP(hipStreamSynchronize(m->gpu->stream));
    m->opts.max_polls = max_polls;
    for (int i = 0; i < 3; i++) {
        if (m->g_fwd[i]) hipGraphExecDestroy(m->g_fwd[i]);
        if (m->g_gen[i]) hipGraphExecDestroy(m->g_gen[i]);
        m->g_fwd[i] = m->g_gen[i] = nullptr;
    }
    return m->build_graphs();
}

int styx_moe_set_timing(styx_moe *m, int on)
{
    if (!m) return fail(STYX_E_INVALID, "styx_moe_set_timing: NULL model");
    if (int r = m->collect_stats()) return r;
    m->opts.time_kernels = on ? 1 : 0;
    return STYX_OK;
}

int styx_moe_last_expert_ids(styx_moe *m, uint32_t *out)
{
    if (!m || !out) return fail(STYX_E_INVALID, "styx_moe_last_expert_ids: NULL argument");
    std::vector<int32_t> h((size_t)m->L * 64);
    STYX_HIP(hipMemcpyAsync(h.data(), m->ids, sizeof(int32_t) * h.size(), hipMemcpyDeviceToHost,
                            m->gpu->stream));
    STYX_HIP(hipStreamSynchronize(m->gpu->stream));
    for (int l = 0; l < m->L; l++)
        for (int s = 0; s < m->K; s++) out[(size_t)l * m->K + s] = (uint32_t)h[(size_t)l * 64 + s];
    return STYX_OK;
}

int styx_moe_last_hot_cold(styx_moe *m, uint32_t *out)
{
    if (!m || !out) return fail(STYX_E_INVALID, "styx_moe_last_hot_cold: NULL argument");
    std::vector<uint32_t> ids((size_t)m->L * m->K);
    if (int r = styx_moe_last_expert_ids(m, ids.data())) return r;
    for (int l = 0; l < m->L; l++) {
        uint32_t hot = 0;
        for (int s = 0; s < m->K; s++) {
            const uint32_t e = ids[(size_t)l * m->K + s];
            if (e < (uint32_t)m->E && m->layers[l].remap[e] != SKIP) hot++;
        }
        out[2 * l] = hot;
        out[2 * l + 1] = (uint32_t)m->K - hot;
    }
    return STYX_OK;
}

int styx_moe_reset(styx_moe *m)
{
    if (!m) return fail(STYX_E_INVALID, "styx_moe_reset: NULL model");
    m->n_past = 0;
    return STYX_OK;
}

int styx_moe_fill_kv(styx_moe *m, int n_t, uint64_t seed, float sigma)
{
    if (!m || n_t < 1 || n_t >= m->n_ctx)
        return fail(STYX_E_INVALID, "styx_moe_fill_kv: need 1 <= n_t < n_ctx");
    STYX_HIP(hipSetDevice(m->gpu->device));
    if (int r = m->ensure_pages(n_t - 1)) return r;
    const int64_t kvd = (int64_t)m->nkv * m->hd;
    for (int l = 0; l < m->L; l++)
        for (int p = 0; p * KV_PAGE_TOKENS < n_t; p++) {
            const int32_t phys = m->h_pt[(size_t)l * m->pages_per_layer + p];
            // a head-major page holds each head's rows apart: fill it whole
            const int rows = m->kv_head_major ? KV_PAGE_TOKENS : std::min(KV_PAGE_TOKENS, n_t - p * KV_PAGE_TOKENS);
            const size_t off = (size_t)phys * KV_PAGE_TOKENS * kvd;
            const uint64_t s = seed ^ (((uint64_t)l << 32) | (uint64_t)p << 1);
            CK(launch_gen_f32(m->gpu->stream, s, 0.0f, sigma, m->kpool + off, rows * kvd));
            CK(launch_gen_f32(m->gpu->stream, s | 1u, 0.0f, sigma, m->vpool + off, rows * kvd));
        }
    STYX_HIP(hipStreamSynchronize(m->gpu->stream));
    m->n_past = n_t;
    return STYX_OK;
}

int styx_moe_read_kv(styx_moe *m, int layer, int t0, int n, float *k, float *v)
{
    if (!m || layer < 0 || layer >= m->L || t0 < 0 || n < 0 || t0 + n > m->n_past || !k || !v)
        return fail(STYX_E_INVALID, "styx_moe_read_kv: bad argument");
    STYX_HIP(hipSetDevice(m->gpu->device));
    const int64_t kvd = (int64_t)m->nkv * m->hd, page = (int64_t)KV_PAGE_TOKENS * kvd;
    // whole pages to the host, then each token's row [kv_dim] out of the
    // page's layout
    std::vector<float> pk((size_t)page), pv((size_t)page);
    for (int p = t0 / KV_PAGE_TOKENS; p * KV_PAGE_TOKENS < t0 + n; p++) {
        const int32_t phys = m->h_pt[(size_t)layer * m->pages_per_layer + p];
        STYX_HIP(hipMemcpyAsync(pk.data(), m->kpool + (size_t)phys * page, sizeof(float) * page,
                                hipMemcpyDeviceToHost, m->gpu->stream));
        STYX_HIP(hipMemcpyAsync(pv.data(), m->vpool + (size_t)phys * page, sizeof(float) * page,
                                hipMemcpyDeviceToHost, m->gpu->stream));
        STYX_HIP(hipStreamSynchronize(m->gpu->stream));
        const int a = std::max(t0, p * KV_PAGE_TOKENS), b = std::min(t0 + n, (p + 1) * KV_PAGE_TOKENS);
        for (int t = a; t < b; t++) {
            const int tp = t % KV_PAGE_TOKENS;
            for (int h = 0; h < m->nkv; h++) {
                const size_t src = m->kv_head_major ? ((size_t)h * KV_PAGE_TOKENS + tp) * m->hd
                                                    : (size_t)tp * kvd + (size_t)h * m->hd;
                const size_t dst = (size_t)(t - t0) * kvd + (size_t)h * m->hd;
                memcpy(k + dst, pk.data() + src, sizeof(float) * m->hd);
                memcpy(v + dst, pv.data() + src, sizeof(float) * m->hd);
            }
        }
    }
    return STYX_OK;
}

uint64_t styx_moe_repin_swaps(const styx_moe *m) { return m ? m->repin_swaps : 0; }

int styx_moe_last_hidden(styx_moe *m, float *out)
{
    if (!m || !out) return fail(STYX_E_INVALID, "styx_moe_last_hidden: NULL argument");
    if (!m->opts.record_hidden) return fail(STYX_E_STATE, "model was loaded without record_hidden");
    STYX_HIP(hipMemcpyAsync(out, m->hidden, sizeof(float) * (m->L + 1) * m->H,
                            hipMemcpyDeviceToHost, m->gpu->stream));
    STYX_HIP(hipStreamSynchronize(m->gpu->stream));
    return STYX_OK;
}

static const Mat *find_mat(const styx_moe *m, const std::string &name)
{
    if (name == m->embd.name) return &m->embd;
    if (name == m->head.name) return &m->head;
    for (auto &ly : m->layers)
        for (const Mat *x : {&ly.wq, &ly.wk, &ly.wv, &ly.wo, &ly.gate, &ly.up, &ly.down, &ly.gsh,
                             &ly.ush, &ly.dsh})
            if (x->name == name) return x;
    return nullptr;
}

int styx_moe_tensor_names(styx_moe *m, char *buf, uint64_t cap)
{
    if (!m || !buf) return fail(STYX_E_INVALID, "styx_moe_tensor_names: NULL argument");
    std::string s;
    auto add = [&](const std::string &n) {
        if (!n.empty()) s += n + "\n";
    };
    add(m->embd.name);
    add(m->head.name);
    for (auto &t : m->f32s) add(t.name);
    for (auto &ly : m->layers)
        for (const Mat *x : {&ly.wq, &ly.wk, &ly.wv, &ly.wo, &ly.gate, &ly.up, &ly.down, &ly.gsh,
                             &ly.ush, &ly.dsh})
            add(x->name);
    if (s.size() + 1 > cap) return fail(STYX_E_INVALID, "styx_moe_tensor_names: buffer too small");
    memcpy(buf, s.c_str(), s.size() + 1);
    return STYX_OK;
}

int styx_moe_export_tensor(styx_moe *m, const char *name, void *dst, uint64_t cap, uint64_t *size,
                           int *type, int64_t dims[4], int *n_dims)
{
    if (!m || !name) return fail(STYX_E_INVALID, "styx_moe_export_tensor: NULL argument");
    STYX_HIP(hipSetDevice(m->gpu->device));
    for (auto &t : m->f32s) {
        if (t.name != name) continue;
        if (size) *size = (uint64_t)t.n * 4;
        if (type) *type = T_F32;
        if (n_dims) *n_dims = (int)t.dims.size();
        if (dims)
            for (size_t i = 0; i < t.dims.size() && i < 4; i++) dims[i] = t.dims[i];
        if (!dst) return STYX_OK;
        if (cap < (uint64_t)t.n * 4) return fail(STYX_E_INVALID, "export: buffer too small");
        STYX_HIP(hipMemcpy(dst, t.p, (size_t)t.n * 4, hipMemcpyDeviceToHost));
        return STYX_OK;
    }
    const Mat *x = find_mat(m, name);
    if (!x) return fail(STYX_E_INVALID, std::string("export: no tensor ") + name);
    if (size) *size = (uint64_t)x->bytes();
    if (type) *type = x->type;
    if (n_dims) *n_dims = (int)x->gguf_dims.size();
    if (dims)
        for (size_t i = 0; i < x->gguf_dims.size() && i < 4; i++) dims[i] = x->gguf_dims[i];
    if (!dst) return STYX_OK;
    if (cap < (uint64_t)x->bytes()) return fail(STYX_E_INVALID, "export: buffer too small");
    void *tmp = nullptr;
    STYX_HIP(hipMalloc(&tmp, x->bytes()));
    const uint8_t *src = x->dev ? x->dev : x->host_dev;
    const int64_t nb = (int64_t)x->rows * (x->cols / blk_elems(x->type));
    hipError_t e = launch_from_split(m->gpu->stream, x->type, src, (uint8_t *)tmp, nb, x->nmat);
    if (e == hipSuccess)
        e = hipMemcpyAsync(dst, tmp, x->bytes(), hipMemcpyDeviceToHost, m->gpu->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(m->gpu->stream);
    hipFree(tmp);
    if (e != hipSuccess) return hip_fail(e, "export");
    return STYX_OK;
}

int styx_moe_kernel_stats(styx_moe *m, styx_kernel_stat *out, int cap, int *n)
{
    if (!m || !n) return fail(STYX_E_INVALID, "styx_moe_kernel_stats: NULL argument");
    if (int r = m->collect_stats()) return r;
    *n = (int)m->stats.size();
    for (int i = 0; i < cap && i < (int)m->stats.size(); i++) {
        memset(out[i].name, 0, sizeof(out[i].name));
        strncpy(out[i].name, m->stats[i].name.c_str(), sizeof(out[i].name) - 1);
        out[i].launches = m->stats[i].launches;
        out[i].total_ms = m->stats[i].ms;
        out[i].bytes = m->stats[i].bytes;
    }
    return STYX_OK;
}

int styx_moe_kernel_stats_reset(styx_moe *m)
{
    if (!m) return fail(STYX_E_INVALID, "styx_moe_kernel_stats_reset: NULL model");
    if (int r = m->collect_stats()) return r;
    m->stats.clear();
    return STYX_OK;
}

}  // extern "C"
