// dispatch_fused.cpp -- the fused hot-path kernels behind styx_kernel_get
// names: router_topk, moe_gate_up_silu_{t}, moe_down_reduce_{t} and
// attn_decode_paged (push blocks in include/styx_hip.h).  A dispatch checks
// its push block and every extent it implies against the bytes its bindings
// make visible, launching nothing when one does not fit, then enqueues the
// same launches as the styx_op_* entry points.  None of these names has a
// reference pipeline: each one replaces a run of crates/model/src/moe.rs
// dispatches (1975-2016, 2023-2038, 2039-2062, 1875-1964).
#include <algorithm>
#include <cstring>

#include "kernels.h"
#include "refk.h"
#include "runtime.h"

namespace styx {

namespace {

// n elements of elt bytes fit in size bytes (no overflow for any n).
bool fits(uint64_t size, uint64_t n, uint64_t elt) { return elt && n <= size / elt; }

int type_of(int i)
{
    static const int t[4] = {T_Q8_0, T_Q4_K, T_Q5_K, T_Q6_K};
    return i >= 0 && i < 4 ? t[i] : -1;
}

// Bytes of a rows x cols matrix of quant type t (0 if cols is not whole blocks).
uint64_t mat_bytes(int t, uint64_t rows, uint64_t cols)
{
    const int be = blk_elems(t);
    if (!is_quant(t) || cols % be) return 0;
    return rows * (cols / be) * (uint64_t)blk_bytes(t);
}

template <typename P> P push_as(const void *push)
{
    P p;
    std::memcpy(&p, push, sizeof(P));
    return p;
}

const hipError_t bad = hipErrorInvalidValue;

hipError_t router_topk(hipStream_t st, void *const *ptr, const uint64_t *size, const void *push)
{
    const auto p = push_as<styx_push_router_topk>(push);
    const uint64_t E = p.E, H = p.H, k = p.k;
    if (k < 1 || k > MAX_TOPK || E < k || E > MAX_EXPERTS || H < 32 || H % 32 || H > XQ_MAX)
        return bad;
    if (!fits(size[0], H, 4) || !fits(size[1], H, 4) || !fits(size[2], E * H, 4) ||
        ((p.flags & 1) && !fits(size[3], E, 4)) || ((p.flags & 2) && !fits(size[4], E, 4)) ||
        ((p.flags & 4) && !fits(size[5], E, 4)) || !fits(size[6], H, 4) ||
        !fits(size[7], E, 4) || !fits(size[8], k, 4) || !fits(size[9], IDS_ROW, 4))
        return bad;
    RouterArgs a{};
    a.x = (const float *)ptr[0];
    a.norm_w = (const float *)ptr[1];
    a.W = (const float *)ptr[2];
    a.bias = (p.flags & 1) ? (const float *)ptr[3] : nullptr;
    a.remap = (p.flags & 2) ? (const uint32_t *)ptr[4] : nullptr;
    a.pmap = (p.flags & 4) ? (const uint32_t *)ptr[5] : nullptr;
    a.eps = p.eps;
    a.xn = (float *)ptr[6];
    a.logits = (float *)ptr[7];
    a.wts = (float *)ptr[8];
    a.ids = (int32_t *)ptr[9];
    a.E = (int)E;
    a.H = (int)H;
    a.k = (int)k;
    a.renorm = p.renorm ? 1 : 0;
    a.arena_mode = p.arena_mode ? 1 : 0;
    a.layer = (int)p.layer;
    return launch_router_topk(st, a);
}

hipError_t gate_up_silu(styx_gpu *g, hipStream_t st, int tg, void *const *ptr,
                        const uint64_t *size, const void *push)
{
    const auto p = push_as<styx_push_moe_gate_up_silu>(push);
    const int tu = (int)p.type_up;
    const uint64_t H = p.H, F = p.F, k = p.k;
    if (k < 1 || k > MAX_TOPK || F < 1 || H < 32 || H % 32 || H > XQ_MAX || !is_quant(tu))
        return bad;
    const uint64_t ng = mat_bytes(tg, F, H), nu = mat_bytes(tu, F, H);
    const uint64_t sg = p.slab_gate ? p.slab_gate : ng, su = p.slab_up ? p.slab_up : nu;
    if (!ng || !nu || sg < ng || su < nu || sg % 16 || su % 16) return bad;
    if (!fits(size[0], p.n_slabs, sg) && p.n_slabs) return bad;
    if (!fits(size[1], p.n_slabs, su) && p.n_slabs) return bad;
    if (!fits(size[2], H, 4) || !fits(size[3], k, 4) || !fits(size[4], k * F, 4)) return bad;
    const Xq q = xq_at(g->xq_scratch, (int)H);
    hipError_t e = launch_xq(st, (const float *)ptr[2], nullptr, nullptr, 0.0f, (int)H, q, nullptr);
    if (e != hipSuccess) return e;
    return launch_moe_gate_up_silu(st, tg, tu, (const uint8_t *)ptr[0], (int64_t)sg,
                                   (const uint8_t *)ptr[1], (int64_t)su, (const int32_t *)ptr[3],
                                   p.n_slabs, q, (float *)ptr[4], (int)H, (int)F, (int)k);
}

hipError_t down_reduce(styx_gpu *g, hipStream_t st, int td, void *const *ptr,
                       const uint64_t *size, const void *push)
{
    const auto p = push_as<styx_push_moe_down_reduce>(push);
    const uint64_t H = p.H, F = p.F, k = p.k;
    if (k < 1 || k > MAX_TOPK || H < 32 || H % 32 || H > XQ_MAX || F < 1 || F > XQ_MAX / 2)
        return bad;
    const uint64_t nd = mat_bytes(td, H, F), sd = p.slab_down ? p.slab_down : nd;
    if (!nd || sd < nd || sd % 16) return bad;
    if (p.n_slabs && !fits(size[0], p.n_slabs, sd)) return bad;
    if (!fits(size[1], k * F, 4) || !fits(size[2], k, 4) || !fits(size[3], k, 4) ||
        !fits(size[4], H, 4) || k * H * 4 > g->partial_bytes)
        return bad;
    float *partial = (float *)g->partial_scratch;
    hipError_t e = launch_moe_down_h(st, td, (const uint8_t *)ptr[0], (int64_t)sd,
                                     (const int32_t *)ptr[2], p.n_slabs, (const float *)ptr[1],
                                     partial, (int)H, (int)F, (int)k);
    if (e != hipSuccess) return e;
    ReduceArgs a{};
    a.partial = partial;
    a.k = (int)k;
    a.H = (int)H;
    a.wts = (const float *)ptr[3];
    a.x = (float *)ptr[4];
    return launch_reduce_rows(st, a);
}

hipError_t attn_paged(styx_gpu *g, hipStream_t st, void *const *ptr, const uint64_t *size,
                      const void *push)
{
    const auto p = push_as<styx_push_attn_decode_paged>(push);
    const uint64_t nh = p.nh, nkv = p.nkv, hd = p.hd, pos = p.pos;
    if (nkv < 1 || nh < nkv || nh % nkv || nh / nkv > 16 || (hd != 64 && hd != 128 && hd != 256) ||
        p.chunk < 16 || p.chunk % 16 || p.max_chunks < 1 || p.max_chunks > 4096)
        return bad;
    const uint64_t kvd = nkv * hd, row = kvd * 4;
    if (!fits(size[0], nh * hd, 4) || !fits(size[1], kvd, 4) || !fits(size[2], kvd, 4) ||
        ((p.flags & 1) && !fits(size[3], hd, 4)) || ((p.flags & 2) && !fits(size[4], hd, 4)) ||
        !fits(size[5], (pos + 1) * (hd / 2) * 2, 8) || !fits(size[9], nh * hd, 4) ||
        !fits(size[10], (uint64_t)styx_op_attn_part_floats((int)nh, (int)nkv, (int)hd,
                                                          (int)p.max_chunks), 4))
        return bad;
    AttnArgs a{};
    const uint64_t pool = std::min(size[6], size[7]);
    hipError_t e = hipSuccess;
    if (p.flags & 4) {
        // whole pages of page_tokens rows; the table covers the context and
        // is read through a copy whose entries are clamped to the pool
        const uint64_t pt = p.page_tokens, need = pos / pt + 1;
        if (pt < 1 || !fits(size[8], need, 4) || need > (uint64_t)styx_gpu::FUSED_PT_MAX)
            return bad;
        const uint64_t pages = pool / (pt * row);
        if (pages < 1 || pages > 0x7FFFFFFF) return bad;
        e = launch_clamp_copy_u32(st, (const uint32_t *)ptr[8], g->fused_pt, (uint32_t)(pages - 1),
                                  (int64_t)need);
        if (e != hipSuccess) return e;
        a.page_table = (const int32_t *)g->fused_pt;
        a.page_tokens = (int)pt;
        a.page_table_len = (int)need;
    } else {
        // the reference's contiguous caches: one page of the whole capacity
        const uint64_t cap = pool / row;
        if (cap <= pos || cap > 0x7FFFFFFF) return bad;
        a.page_table = g->fused_scalars + 1;  // a single entry 0
        a.page_tokens = (int)cap;
        a.page_table_len = 1;
    }
    // the position: written to the gpu's scalar in stream order
    e = launch_fill_u32(st, (uint32_t *)g->fused_scalars, (uint32_t)pos, 1);
    if (e != hipSuccess) return e;
    a.q = (const float *)ptr[0];
    a.k = (const float *)ptr[1];
    a.v = (const float *)ptr[2];
    a.q_norm = (p.flags & 1) ? (const float *)ptr[3] : nullptr;
    a.k_norm = (p.flags & 2) ? (const float *)ptr[4] : nullptr;
    a.eps = p.eps;
    a.rope = (const double2 *)ptr[5];
    a.kpool = (float *)ptr[6];
    a.vpool = (float *)ptr[7];
    a.pos = g->fused_scalars;
    a.out = (float *)ptr[9];
    a.part = (float *)ptr[10];
    a.nh = (int)nh;
    a.nkv = (int)nkv;
    a.hd = (int)hd;
    a.chunk = (int)p.chunk;
    a.max_chunks = (int)p.max_chunks;
    a.scale = p.scale;
    return launch_attn_decode(st, a);
}

}  // namespace

hipError_t fused_launch(styx_gpu *g, hipStream_t st, int kid, void *const *ptr,
                        const uint64_t *size, const void *push)
{
    if (kid == RK_F_ROUTER_TOPK) return router_topk(st, ptr, size, push);
    if (kid >= RK_F_GATE_UP_SILU && kid < RK_F_GATE_UP_SILU + 4)
        return gate_up_silu(g, st, type_of(kid - RK_F_GATE_UP_SILU), ptr, size, push);
    if (kid >= RK_F_DOWN_REDUCE && kid < RK_F_DOWN_REDUCE + 4)
        return down_reduce(g, st, type_of(kid - RK_F_DOWN_REDUCE), ptr, size, push);
    if (kid == RK_F_ATTN_PAGED) return attn_paged(g, st, ptr, size, push);
    return bad;
}

}  // namespace styx
