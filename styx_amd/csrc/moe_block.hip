// moe_block.hip -- the MoE block of one layer as one persistent launch.
//
// One kernel runs what k_router, k_gate_up, k_down and k_reduce_rows do
// (ffn RMSNorm + router logits, top-k ranking, expert gate/up, swiglu +
// down, the weighted combine and the next RMSNorm's limbs) with the same
// arithmetic.  What changes is the schedule: no kernel boundary between the
// phases, the shared expert's gate/up rows before the routing is known, the
// top-k weights before the partials, and each phase's weights issued as
// soon as its rows are known.
//
// Cross-workgroup data (router logits, each slot's SwiGLU of its gate and
// up rows, per-slot down partials) travels as tagged 64-bit words (xchg.h):
// no fence and no counter is needed, and no buffer has to be cleared between
// launches.
//
// Every wait is bounded: after max_polls rounds, or once another workgroup
// has given up, a workgroup sets *abort and exits.  The grid is sized to be
// resident at once (two workgroups per CU), so in normal operation no wait
// ever approaches the bound; the host checks *abort after each token.
#include "kernels.h"
#include "qdot.h"
#include "router.h"
#include "topk.h"
#include "walk.h"
#include "xchg.h"

#include <algorithm>
#include <type_traits>

namespace styx {

constexpr int MB_RR = 256;         // reduce rows per workgroup, as k_reduce_rows
constexpr int MB_MAX_F = 2048;     // gate/up width handled here (g and u of a slot in LDS)
constexpr int MB_TICKETS = 64;     // ticket counters (workgroup w draws from counter w % 64)
constexpr int MB_GU_ROWS = 4;      // gate/up rows per lane group in flight at once
constexpr int MB_TRACE = 16;       // trace slots per workgroup
constexpr int MB_MAX_H = 4096;     // residual width when the next q/k/v is folded in
constexpr int MB_QJ = 7;           // tagged words per thread and poll round, q/k/v phase
constexpr int MB_SHJ = 8;          // shared-expert gate inputs per thread loaded before the partials' wait

struct MoeBlockK {
    const float *x;         // residual [H]: read at entry, updated by the reduce
    const float *ffn_norm;  // [H]
    const float *W;         // router [E][H] f32
    const float *bias;      // [E] or null
    const float *sh_ginp;   // shared-expert gate input [H] or null
    const uint8_t *sh[3];   // shared expert gate/up/down as slot k, or null
    ExpSrc src[3];          // gate, up, down
    Route route;            // E, k, remap, pmap, ids_out (logits unused)
    float eps;
    int H, F, E, k, renorm, nslots;
    int tg, tu;             // gate / up quant types (the down type is a template parameter)
    float *x_out;
    const float *norm_next;
    Xq xq;
    float *ss;
    float *wts_out;
    uint64_t *t_lg, *t_gu, *t_part;  // tagged [E], h [nslots][F], [nslots][H]
    unsigned long long *ticket;  // MB_TICKETS counters, 128 bytes apart
    int *abort;
    int max_polls;
    uint64_t *trace;  // optional: [gridDim][MB_TRACE] wall-clock stamps per workgroup
    // the next layer's q/k/v folded into the tail (wqkv[0] null: not folded)
    const uint8_t *wqkv[3];  // q8_0 split layout, [rows][H]
    float *qkv_out[3];
    int qkv_rows[3];
    uint64_t *t_xq;          // tagged limbs of x (.) w_next + the x^2 partials
    int G_q, UPL_q, nb_q, rpw_q, n_q;  // rows per workgroup, workgroups [nRed, nRed + n_q)
    int nR, rt_rows;                         // router workgroups, rows per router workgroup
    int G_gu, nb_gu, rpw_gu, bps_gu, n_gu;   // gate/up blocks: [2][nslots][bps_gu]
    int G_d, nb_d, rpw_d, bps_d, n_d;        // down blocks: [nslots][bps_d]
    int nRed;                                // reduce workgroups
    int off_xq, off_lg, off_gu, off_hs, off_xqh;  // dynamic LDS layout (bytes)
};

// Words i = tid + 256 j (i < n) of the workgroup: wait until the word at
// addr(i) carries `tag` and store its value to dst[i] (addr(i) == null: no
// word, dst[i] = 0).  Thread 0 decides for the whole workgroup whether to
// keep waiting.  Returns false when the wait is abandoned (*abort set).
template <int MAXJ, typename Addr>
__device__ __forceinline__ bool tpoll(int n, Addr addr, uint32_t tag, float *dst, const MoeBlockK &a)
{
    return tpoll_wg<MAXJ, WG>(n, addr, tag, dst, a.max_polls, a.abort);
}

// Routing for E <= 128 experts with a power-of-two quarter Q = E / 4:
// wave w polls the tagged logits of its quarter [w Q, (w + 1) Q) and ranks
// them among themselves as soon as they are in (rank_quarter, no workgroup
// barrier between the poll and that stage), then the 4k candidates are
// ranked (rank_candidates): the ids of rank_ids_lds with two workgroup
// barriers instead of six.  The logits land in s_lg for the reduce's
// weights.  Returns false when the wait was abandoned (*abort set).
__device__ __forceinline__ bool route_by_quarters(const MoeBlockK &a, uint32_t tag, float *s_lg,
                                                  int32_t *s_ids, bool publish, uint64_t *tr)
{
    __shared__ __align__(16) uint64_t q_key[128];
    __shared__ __align__(16) uint64_t c_key[4 * MAX_TOPK];
    __shared__ int q_fail[WAVES];
    const int Q = a.E / 4, k = a.k;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, e = wave * Q + lane;
    if (tid < IDS_ROW) s_ids[tid] = (int32_t)SKIP;  // read after the barrier below
    bool pend = lane < Q;
    int failed = 0;
    for (int polls = 0; __any(pend); polls++) {
        if (pend) {
            const uint64_t v = tget(a.t_lg + e);
            if (tvalid(v, tag)) {
                const float f = tval(v);
                s_lg[e] = f;
                q_key[e] = rank_key(f, e);
                pend = false;
            }
        }
        if (!__any(pend)) break;
        if (polls >= a.max_polls || ((polls & 31) == 31 && __any(abort_seen(a.abort)))) {
            failed = 1;
            break;
        }
        __builtin_amdgcn_s_sleep(1);
    }
    if (tr && tid == 0) tr[3] = wall_clock64();
    // this wave's candidate slots (a quarter of fewer than k keys leaves
    // some unwritten), then its ranking: all the wave's own LDS words
    if (lane < k) c_key[wave * k + lane] = 0;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (!failed) rank_quarter_any(q_key + wave * Q, Q, k, c_key + wave * k);
    if (lane == 0) q_fail[wave] = failed;
    __syncthreads();
    int any = 0;
    for (int i = 0; i < WAVES; i++) any |= q_fail[i];
    if (any) {
        if (tid == 0) abort_raise(a.abort);
        return false;
    }
    rank_candidates_any(c_key, k, s_ids);
    __syncthreads();
    if (publish) publish_id_row(a.route, s_ids);
    return true;
}

// Slab of expert e routed to `slot` (null when e is not a valid expert,
// which only non-finite logits can cause: the rows then publish zeros).
__device__ __forceinline__ const uint8_t *routed_slab(const MoeBlockK &a, const ExpSrc &src, int e,
                                                      int slot)
{
    if ((unsigned)e >= (unsigned)a.E) return nullptr;
    uint32_t r3[3];
    route_row(a.route, e, slot, r3);
    return slab_pick(src, r3[0], r3[1], r3[2]);
}

// Rows [r0, r1) of one expert matrix (gate or up) against the limbs of
// x (.) w in LDS, walked by the lane groups of waves [wave0, wave0 + 2); row
// r's dot times the RMSNorm scale xscale goes to dst[r - r0] (LDS).  A
// missing slab gives zeros.
// `between` runs once the rows' first weights are issued (the caller
// issues further loads there).
template <int T, typename Between>
__device__ __forceinline__ void gu_rows(const MoeBlockK &a, const uint8_t *slab, const Xq &xqx,
                               float xscale, int r0, int r1, int wave0, float *dst, Between between,
                               uint64_t *tr)
{
    if (!slab) {
        between();
        for (int r = r0 + (int)threadIdx.x - 64 * wave0; r < r1; r += 128) dst[r - r0] = 0.0f;
        return;
    }
    auto stamp = [&](int i) {
        if (tr && threadIdx.x == 0) tr[i] = wall_clock64();
    };
    walk_rows_pipelined<T, 1, MB_GU_ROWS / 2>(
        OneMat{mat_at(slab, T, (int64_t)a.F * a.nb_gu), a.nb_gu}, a.nb_gu, a.G_gu, r0, r1,
        [&](UX<T>(&x)[1], const LaneU<1> &lu) {
            stamp(11);
            between();
            XFrom<T, 1>{xqx}(x, lu);
            stamp(12);
            return true;
        },
        [&](int r, float v) { dst[r - r0] = v * xscale; }, 2, wave0);
    stamp(13);
}

// Gate/up block b: rows [r0, r1) of slot s, of both matrices.
struct GuPos {
    int s, r0, r1;
};
__device__ __forceinline__ GuPos gu_pos(const MoeBlockK &a, int b)
{
    const int s = b / a.bps_gu;
    const int r0 = (b - s * a.bps_gu) * a.rpw_gu;
    return {s, r0, min(a.F, r0 + a.rpw_gu)};
}

// Gate/up block bp: waves 0-1 walk its gate rows and waves 2-3 the same up
// rows, side by side (each matrix at its own type); then the block's
// h = swiglu_f32(g, u) (ops2.rs:305-309) is published, one tagged word per
// row, so a down workgroup waits for F words of its slot instead of 2F and
// every gate/up workgroup carries the same mix of the two matrices' bytes.
// gl holds 2 * rpw_gu floats of LDS.
// With every expert in HBM (no remap), the slab of expert e is hot +
// e * stride: the two are read from the arguments before the routing wait,
// so only the id read stands between the ranking and the first loads.
struct HotSlab {
    const uint8_t *hot;
    int64_t stride;
};
__device__ __forceinline__ HotSlab hot_slab(const MoeBlockK &a, int m)
{
    return a.route.remap ? HotSlab{nullptr, 0} : HotSlab{a.src[m].hot, a.src[m].hot_slab};
}
__device__ __forceinline__ const uint8_t *slot_slab(const MoeBlockK &a, const HotSlab &hs, int m,
                                                    const int32_t *s_ids, int s)
{
    if (s >= a.k) return a.sh[m];
    const int e = s_ids[s];
    if (hs.hot) return (unsigned)e < (unsigned)a.E ? hs.hot + (int64_t)e * hs.stride : nullptr;
    return routed_slab(a, a.src[m], e, s);
}

template <typename Between>
__device__ __forceinline__ void gu_block(const MoeBlockK &a, const GuPos &bp, bool routed_phase,
                                const int32_t *s_ids, const HotSlab &hs, const Xq &xqx, float xscale,
                                uint32_t tag, float *gl, Between between, uint64_t *tr)
{
    const int s = bp.s, r0 = bp.r0, r1 = bp.r1;
    if ((s < a.k) != routed_phase) return;
    const int m = (int)(threadIdx.x >> 7);  // 0: gate (waves 0, 1), 1: up (waves 2, 3)
    if (routed_phase && tr && threadIdx.x == 0) tr[14] = wall_clock64();
    const uint8_t *slab = slot_slab(a, hs, m, s_ids, s);
    if (routed_phase && tr && threadIdx.x == 0) tr[15] = wall_clock64();
    float *dst = gl + m * a.rpw_gu;
    switch (m == 0 ? a.tg : a.tu) {
    case T_Q8_0: gu_rows<T_Q8_0>(a, slab, xqx, xscale, r0, r1, 2 * m, dst, between, tr); break;
    case T_Q4_K: gu_rows<T_Q4_K>(a, slab, xqx, xscale, r0, r1, 2 * m, dst, between, tr); break;
    case T_Q5_K: gu_rows<T_Q5_K>(a, slab, xqx, xscale, r0, r1, 2 * m, dst, between, tr); break;
    default: gu_rows<T_Q6_K>(a, slab, xqx, xscale, r0, r1, 2 * m, dst, between, tr); break;
    }
    __syncthreads();
    uint64_t *y = a.t_gu + (size_t)s * a.F;
    for (int r = r0 + (int)threadIdx.x; r < r1; r += WG) {
        const float g = gl[r - r0];
        tput(y + r, tag, g / (1.0f + expf(-g)) * gl[a.rpw_gu + r - r0]);
    }
    __syncthreads();  // gl is rewritten by the next block
}

// The next layer's q/k/v rows [r0, r1) (of the three matrices stacked):
// their weights are issued first (two batches of NR rows per lane group),
// then the limbs of x (.) w_next and the x^2 partials are taken from the
// reduce workgroups' tagged words into LDS, then the rows are formed as
// k_mv_dense forms them (dot times the RMSNorm scale) and stored for the
// next kernel.  Returns false when the wait was abandoned.
// GC: the lane-group width when known at compile time (the rows' sums
// and lane map then fold to constants), 0: a.G_q.
template <int UPL, int NR, int GC>
__device__ __forceinline__ bool qkv_rows(const MoeBlockK &a, int r0, int r1, uint32_t tag, uint8_t *xq_lds,
                         uint64_t *tr)
{
    const int b1 = a.qkv_rows[0], b2 = b1 + a.qkv_rows[1];
    const Mat3 at(mat_at(a.wqkv[0], T_Q8_0, (int64_t)a.qkv_rows[0] * a.nb_q),
                  mat_at(a.wqkv[1], T_Q8_0, (int64_t)a.qkv_rows[1] * a.nb_q),
                  mat_at(a.wqkv[2], T_Q8_0, (int64_t)a.qkv_rows[2] * a.nb_q), b1, b2, a.nb_q);
    float scale = 0.0f;
    return walk_rows_pipelined<T_Q8_0, UPL, NR>(
        at, a.nb_q, GC ? GC : a.G_q, r0, r1,
        [&](UX<T_Q8_0>(&x)[UPL], const LaneU<UPL> &lu) {
            // the limbs (A | B | C | sx | s16, the layout of xq_at) and the
            // partials
            const int n_ss = (a.H + MB_RR - 1) / MB_RR;
            const int nw = (int)(xq_bytes(a.H) / 4) + n_ss;
            for (int c = 0; c < nw; c += MB_QJ * WG)
                if (!tpoll<MB_QJ>(min(MB_QJ * WG, nw - c), [&](int i) { return a.t_xq + c + i; }, tag,
                                  (float *)xq_lds + c, a))
                    return false;
            if (tr && threadIdx.x == 0) tr[9] = wall_clock64();
            const float *ss = (const float *)(xq_lds + xq_bytes(a.H));
            float t = 0.0f;
            for (int i = (int)threadIdx.x & 63; i < n_ss; i += 64) t += ss[i];
            t = wave_sum(t);
            scale = 1.0f / sqrtf(t / (float)a.H + a.eps);
            XFrom<T_Q8_0, UPL>{xq_at(xq_lds, a.H)}(x, lu);
            return true;
        },
        [&](int gr, float acc) {
            float *y = gr < b1 ? a.qkv_out[0] + gr : gr < b2 ? a.qkv_out[1] + (gr - b1)
                                                             : a.qkv_out[2] + (gr - b2);
            gst(y, acc * scale);
        });
}

// Gate/up types are switched at run time (one routed row block at a time,
// nothing held across); the down type and units per lane are template
// parameters because the down rows' weights stay in registers across the
// gate/up phase.
template <int TD, int UD>
__global__ void __launch_bounds__(WG, 2) k_moe_block(MoeBlockK args)
{
    // The arguments are copied to LDS once: this kernel is short of scalar
    // registers, and the compiler would otherwise re-read argument fields
    // from the kernarg segment wherever they are used -- chains of dependent
    // scalar loads on the critical path.
    static_assert(sizeof(MoeBlockK) % 4 == 0 && sizeof(MoeBlockK) / 4 <= WG, "args copy");
    __shared__ __align__(16) MoeBlockK s_args;
    if (threadIdx.x < sizeof(MoeBlockK) / 4)
        ((uint32_t *)&s_args)[threadIdx.x] = ((const uint32_t *)&args)[threadIdx.x];
    __syncthreads();
    const MoeBlockK &a = s_args;
    extern __shared__ __align__(16) uint8_t lds[];
    float *xs = (float *)lds;                         // x (.) w (the RMSNorm scale apart)
    const Xq xqx = xq_at(lds + a.off_xq, a.H);        // limbs of x (.) w
    float *s_lg = (float *)(lds + a.off_lg);          // router logits
    float *gus = (float *)(lds + a.off_gu);           // gate/up rows; then h[F]; reduce: partials
    float *hs = (float *)(lds + a.off_hs);            // the reduce's rows of x (.) w_next
    const Xq xqh = xq_at(lds + a.off_xqh, a.F);       // limbs of the slot's h
    __shared__ int32_t s_ids[IDS_ROW];
    __shared__ float red[16];
    __shared__ uint32_t s_tag;
    __shared__ float s_w[MAX_TOPK];
    __shared__ float s_wsum, s_sg;

    const int w = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nwg = gridDim.x;
    // every workgroup draws its ticket, also one without work: counter
    // w % 64 is drawn by nwg / 64 workgroups per launch, so
    // ticket / (nwg / 64) numbers the launch (spreading the draws over 64
    // counters keeps them from queueing on one address)
    // phase stamps go to LDS (a global store would hold up the next wait on
    // the vector memory counter) and are written out when the workgroup ends
    __shared__ uint64_t s_trace[MB_TRACE];
    uint64_t *tr = a.trace ? s_trace : nullptr;
    if (tr && tid < MB_TRACE) s_trace[tid] = 0;
    auto stamp = [&](int i) {
        if (tr && tid == 0) tr[i] = wall_clock64();
    };
    auto flush = [&] {  // at uniform exits only
        if (!tr) return;
        __syncthreads();
        if (tid < MB_TRACE) gst<uint64_t>(a.trace + (size_t)w * MB_TRACE + tid, tr[tid]);
    };
    __syncthreads();
    stamp(0);
    // this workgroup's first gate/up block and its down rows, decoded once
    // here: they do not depend on the routing, and the divisions would
    // otherwise sit between the ranking and the first weight loads
    const GuPos gp0 = gu_pos(a, w);
    const bool has_d = w < a.n_d;
    const int ds = has_d ? w / a.bps_d : 0;
    const int d0 = (w - ds * a.bps_d) * a.rpw_d, d1 = min(a.H, d0 + a.rpw_d);
    // the draw's result is first needed after the entry loads are issued
    unsigned long long ticket = 0;
    if (tid == 0) ticket = draw_ticket(a.ticket, MB_TICKETS, w);
    if (w >= a.n_gu && w >= a.n_d && w >= a.nRed && w >= a.nRed + a.n_q) {
        flush();
        return;
    }

    // ---- entry (workgroups with gate/up work; the router and reduce
    // workgroups are among them)
    const bool has_x = w < a.n_gu;
    const int nrt = w < a.nR ? a.rt_rows : 0;  // router rows of this workgroup
    uint32_t tag = 0;
    float xscale = 1.0f;  // the ffn RMSNorm scale (xs holds x (.) w unscaled)
    // x, the norm weight and (router workgroups) the workgroup's router rows
    // at columns 4 t + 1024 j of thread t, all issued before any reduction;
    // xs gets x (.) w, whose limbs need no sum of squares, and the router
    // dots and the x^2 sum are reduced together (router.h)
    __shared__ float s_rt[RT_RED];
    auto entry = [&](auto px) {
        constexpr int PX = decltype(px)::value;
        if (has_x) {
            float4 xv[PX], nv[PX], wv[PX][RT_ROWS];
#pragma unroll
            for (int j = 0; j < PX; j++) {
                const int i = tid * 4 + WG * 4 * j;
                const int ic = i < a.H ? i : 0;
                xv[j] = gld4(a.x + ic);
                nv[j] = gld4(a.ffn_norm + ic);
#pragma unroll
                for (int r = 0; r < RT_ROWS; r++)
                    if (r < nrt) wv[j][r] = gld4(a.W + (int64_t)min(w * a.rt_rows + r, a.E - 1) * a.H + ic);
            }
            float ss = 0.0f, p[RT_ROWS] = {};
#pragma unroll
            for (int j = 0; j < PX; j++) {
                const int i = tid * 4 + WG * 4 * j;
                if (i < a.H) *(float4 *)(xs + i) = router_acc(xv[j], nv[j], wv[j], nrt, ss, p);
            }
            for (int i = tid * 4 + WG * 4 * PX; i < a.H; i += WG * 4) {  // rows past MB_MAX_H
                float4 wt[RT_ROWS];
#pragma unroll
                for (int r = 0; r < RT_ROWS; r++)
                    wt[r] = r < nrt ? gld4(a.W + (int64_t)min(w * a.rt_rows + r, a.E - 1) * a.H + i)
                                    : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                *(float4 *)(xs + i) = router_acc(gld4(a.x + i), gld4(a.ffn_norm + i), wt, nrt, ss, p);
            }
            router_wave_part(ss, p, nrt, s_rt);
        }
        if (tid == 0) s_tag = ticket_tag(ticket, nwg, MB_TICKETS);
        __syncthreads();  // s_rt, s_tag, xs
        tag = s_tag;
        if (has_x) xscale = router_scale(s_rt, a.H, a.eps);
        stamp(1);
        // ---- router logits: thread r publishes row w * rt_rows + r
        const int rr = w * a.rt_rows + tid;
        if (tid < nrt && rr < a.E) {
            const float lg = xscale * router_dot(s_rt, tid);
            tput(a.t_lg + rr, tag, a.bias ? lg + gld(a.bias + rr) : lg);
        }
    };
    if (a.H <= 2048)
        entry(std::integral_constant<int, 2>{});
    else
        entry(std::integral_constant<int, MB_MAX_H / (4 * WG)>{});

    // the slab rules of this workgroup's gate/up matrix and down rows
    const HotSlab hs_gu = hot_slab(a, tid >> 7), hs_d = hot_slab(a, 2);

    // ---- limbs of x (.) w (before the routing wait: polling the logits
    // while the router workgroups still load their rows slows those loads);
    // the shared-expert gate/up rows need no routing
    auto nothing = [] {};
    if (has_x) {
        xq_build<WG>(xs, nullptr, 0.0f, false, a.H, xqx, red, nullptr);
        __syncthreads();
        stamp(2);
        for (int b = w; b < a.n_gu; b += nwg) gu_block(a, b == w ? gp0 : gu_pos(a, b), false, s_ids, hs_gu, xqx, xscale, tag, gus, nothing, tr);
    }

    // ---- routing: every workgroup ranks the logits (topk_softmax_f32 order)
    const int Qr = a.E / 4;
    if (a.E <= 128 && (Qr & (Qr - 1)) == 0) {
        if (!route_by_quarters(a, tag, s_lg, s_ids, w == 0, tr)) return;
    } else {
        if (!tpoll<MAX_EXPERTS / WG>(a.E, [&](int i) { return a.t_lg + i; }, tag, s_lg, a)) return;
        stamp(3);
        rank_ids_lds(a.route, s_ids, s_lg, w == 0);
    }
    stamp(4);

    // ---- this workgroup's down rows (their weights are issued after the
    // workgroup's own gate/up rows and before the wait for the slot's
    // outputs; issuing them during the gate/up phase delays that stream)
    const uint8_t *dslab = has_d ? slot_slab(a, hs_d, 2, s_ids, ds) : nullptr;

    // ---- routed gate/up rows
    if (has_x)
        for (int b = w; b < a.n_gu; b += nwg) gu_block(a, b == w ? gp0 : gu_pos(a, b), true, s_ids, hs_gu, xqx, xscale, tag, gus, nothing, tr);
    stamp(5);

    // ---- down: the slot's h (published by its gate/up workgroups) and its
    // limbs in LDS, then the rows whose weights are already in flight
    if (has_d) {
        const int F = a.F;
        const uint64_t *hw = a.t_gu + (size_t)ds * F;
        auto wait_gu = [&] {
            const bool ok = tpoll<MB_MAX_F / WG>(F, [&](int i) { return hw + i; }, tag, gus, a);
            stamp(6);
            return ok;
        };
        // the down weights go out first (two batches of rows per lane
        // group: of two rows each with one unit per lane, of one row with
        // more, as the registers allow), before the wait for the slot's h:
        // they stream while the slowest gate/up rows are finished, and the
        // limbs of h are built once it is in
        uint64_t *part = a.t_part + (size_t)ds * a.H;
        auto build = [&] {
            xq_build<WG>(gus, nullptr, 0.0f, false, F, xqh, red, nullptr);
            __syncthreads();
            stamp(7);
        };
        // the walk with the lane-group width a compile-time constant for the
        // widths of the configs' down rows (16: F 768 and 512 at one unit
        // per lane; 32: F 1536), so that its lane map and row sums fold
        auto down_walk = [&](auto gc) {
            constexpr int GC = decltype(gc)::value;
            return walk_rows_pipelined<TD, UD, UD == 1 ? 2 : 1>(
                OneMat{mat_at(dslab, TD, (int64_t)a.H * a.nb_d), a.nb_d}, a.nb_d, GC ? GC : a.G_d,
                d0, d1,
                [&](UX<TD>(&x)[UD], const LaneU<UD> &lu) {
                    if (!wait_gu()) return false;
                    build();
                    XFrom<TD, UD>{xqh}(x, lu);
                    return true;
                },
                [&](int r, float v) { tput(part + r, tag, v); });
        };
        if (dslab) {
            const bool ok = a.G_d == 16   ? down_walk(std::integral_constant<int, 16>{})
                            : a.G_d == 32 ? down_walk(std::integral_constant<int, 32>{})
                                          : down_walk(std::integral_constant<int, 0>{});
            if (!ok) return;
        } else {
            if (!wait_gu()) return;
            build();
            for (int r = d0 + tid; r < d1; r += WG) tput(part + r, tag, 0.0f);
        }
        stamp(8);
    }

    // ---- the next layer's q/k/v (folded in): workgroups past the reduce
    // ones, after their down rows
    if (a.wqkv[0] && w >= a.nRed && w < a.nRed + a.n_q) {
        const int q0 = (w - a.nRed) * a.rpw_q;
        const int q1 = min(a.qkv_rows[0] + a.qkv_rows[1] + a.qkv_rows[2], q0 + a.rpw_q);
        __syncthreads();  // the limbs of x (.) w are no longer read (their LDS is reused)
        // rows per lane group in flight: all of them at the shapes served
        // (a single memory round trip), as the registers allow
        const bool ok =
            a.G_q == 64 ? (a.UPL_q == 1 ? qkv_rows<1, 3, 64>(a, q0, q1, tag, lds + a.off_xq, tr)
                                        : qkv_rows<2, 3, 64>(a, q0, q1, tag, lds + a.off_xq, tr))
                        : (a.UPL_q == 1 ? qkv_rows<1, 3, 0>(a, q0, q1, tag, lds + a.off_xq, tr)
                                        : qkv_rows<2, 3, 0>(a, q0, q1, tag, lds + a.off_xq, tr));
        if (!ok) return;
        stamp(10);
        flush();
        return;  // a q/k/v workgroup is past the reduce ones
    }

    // ---- reduce (k_reduce_rows arithmetic): weights, x += sum_s w_s y_s,
    // the shared expert's axpy_sig, then the next RMSNorm's limbs.  The
    // weights and the shared-expert gate need no partials: formed while the
    // other workgroups' down rows are still being computed.
    if (w >= a.nRed) {
        flush();
        return;
    }
    const int r0 = w * MB_RR, nrow = min(MB_RR, a.H - r0);
    const int r = r0 + tid;
    const bool hr = tid < nrow;
    const bool shexp = a.nslots > a.k;
    const float x0 = hr ? gld(a.x + r) : 0.0f;
    const float nw = (a.norm_next && hr) ? gld(a.norm_next + r) : 1.0f;
    float lg_pick = 0.0f, mx = -INFINITY;
    for (int e = tid; e < a.E; e += WG) mx = fmaxf(mx, s_lg[e]);
    if (tid < a.k) {
        const int e = s_ids[tid];
        lg_pick = (e >= 0 && e < a.E) ? s_lg[e] : -INFINITY;
    }
    // the shared expert's gate input (columns tid + 256 j): loaded here,
    // reduced after the partials' wait, so that its memory round trip runs
    // during that wait instead of before it
    float shg[MB_SHJ];
    if (shexp) {
#pragma unroll
        for (int j = 0; j < MB_SHJ; j++) shg[j] = gld(a.sh_ginp + min(tid + WG * j, a.H - 1));
    }
    mx = wave_max(mx);
    if (lane == 0) red[wave] = mx;
    __syncthreads();
    mx = red[0];
    for (int i = 1; i < WAVES; i++) mx = fmaxf(mx, red[i]);
    float se = 0.0f;
    for (int e = tid; e < a.E; e += WG) se += expf(s_lg[e] - mx);
    se = block_sum<WG>(se, red);
    if (tid < a.k) s_w[tid] = expf(lg_pick - mx) / se;
    __syncthreads();
    if (tid == 0 && a.renorm) {
        float wsum = 0.0f;
        for (int s = 0; s < a.k; s++) wsum += s_w[s];
        s_wsum = wsum;
    }
    __syncthreads();
    if (tid < a.k) {
        const float wt = a.renorm ? s_w[tid] / s_wsum : s_w[tid];
        s_w[tid] = wt;
        if (a.wts_out && w == 0) gst(a.wts_out + tid, wt);
    }
    __syncthreads();  // gus is reused for the partials
    float *pl = gus;  // [nslots][MB_RR]
    if (!tpoll<MAX_TOPK + 1>(a.nslots * MB_RR,
                             [&](int i) -> const uint64_t * {
                                 const int s = i / MB_RR, t = i - s * MB_RR;
                                 return t < nrow ? a.t_part + (size_t)s * a.H + r0 + t : nullptr;
                             },
                             tag, pl, a))
        return;
    stamp(9);
    if (shexp) {
        float shd = 0.0f;
#pragma unroll
        for (int j = 0; j < MB_SHJ; j++)
            if (tid + WG * j < a.H) shd += shg[j] * xs[tid + WG * j];
        for (int i = tid + WG * MB_SHJ; i < a.H; i += WG) shd += gld(a.sh_ginp + i) * xs[i];
        const float d = block_sum<WG>(shd, red) * xscale;  // xs is x (.) w unscaled
        if (tid == 0) s_sg = 1.0f / (1.0f + expf(-d));
        __syncthreads();  // s_sg; red is read by every wave before it is rewritten below
    }
    float p[MAX_TOPK];
#pragma unroll
    for (int s = 0; s < MAX_TOPK; s++) p[s] = (s < a.k && hr) ? pl[s * MB_RR + tid] : 0.0f;
    const float y0 = (shexp && hr) ? pl[a.k * MB_RR + tid] : 0.0f;
    float acc = 0.0f;
#pragma unroll
    for (int s = 0; s < MAX_TOPK; s++)
        if (s < a.k) acc += s_w[s] * p[s];
    float xv = x0 + acc;
    if (shexp) xv = xv + s_sg * y0;
    if (hr) gst(a.x_out + r, xv);
    if (!a.norm_next) {
        stamp(10);
        flush();
        return;
    }
    // x (.) w_next for the limbs and the x^2 sums of the waves, behind one
    // barrier (red and hs are free: the partials' wait has passed barriers
    // since their last use); the four sums in block_sum's order
    float *xw = hs;  // MB_RR floats
    xw[tid] = xv * nw;
    const float sqw = wave_sum(hr ? xv * xv : 0.0f);
    if (lane == 0) red[wave] = sqw;
    __syncthreads();
    const float sq = ((red[0] + red[1]) + red[2]) + red[3];
    if (tid == 0) gst(a.ss + w, sq);
    if (!a.wqkv[0]) {
        if (tid < MB_RR / 4) {  // four rows per thread: 64 threads at work
            const bool act = 4 * tid < nrow;
            float h[4];
#pragma unroll
            for (int i = 0; i < 4; i++) h[i] = act ? xw[4 * tid + i] : 0.0f;
            xq_group4(h, act, tid, xq_shift(a.xq, r0));
        }
    } else {
        // the limbs of these rows, written to the limb buffer and published
        // as tagged words for the q/k/v workgroups by the threads that form
        // them
        if (tid < MB_RR / 4) {  // four rows per thread: 64 threads at work
            const bool act = 4 * tid < nrow;
            float h[4];
#pragma unroll
            for (int i = 0; i < 4; i++) h[i] = act ? xw[4 * tid + i] : 0.0f;
            xq_group4_put(h, act, tid, xq_shift(a.xq, r0), a.H, r0,
                          [&](int i, uint32_t v) { tput(a.t_xq + i, tag, __uint_as_float(v)); });
        }
        if (tid == 0) tput(a.t_xq + xq_bytes(a.H) / 4 + w, tag, sq);
    }
    stamp(10);
    flush();
}

// ------------------------------------------------------------------ host --
static int align16(size_t n) { return (int)((n + 15) / 16 * 16); }

using MoeKernel = void (*)(MoeBlockK);

static MoeKernel moe_kernel(int td, int ud)
{
    switch (td) {
    case T_Q8_0:
        switch (ud) {
        case 1: return k_moe_block<T_Q8_0, 1>;
        case 2: return k_moe_block<T_Q8_0, 2>;
        case 3: return k_moe_block<T_Q8_0, 3>;
        case 4: return k_moe_block<T_Q8_0, 4>;
        default: return nullptr;
        }
    case T_Q4_K: return ud == 1 ? k_moe_block<T_Q4_K, 1> : ud == 2 ? k_moe_block<T_Q4_K, 2> : nullptr;
    case T_Q5_K: return ud == 1 ? k_moe_block<T_Q5_K, 1> : ud == 2 ? k_moe_block<T_Q5_K, 2> : nullptr;
    case T_Q6_K: return ud == 1 ? k_moe_block<T_Q6_K, 1> : ud == 2 ? k_moe_block<T_Q6_K, 2> : nullptr;
    default: return nullptr;
    }
}

// Geometry and LDS of one launch; false if the shapes are outside what the
// kernel handles (the caller then runs the separate kernels).
static bool moe_geometry(const MoeBlockArgs &h, int nwg, MoeBlockK &a, size_t &lds)
{
    const Geo gg = pick_geo(h.tg, h.H), gd = pick_geo(h.td, h.F), gu = pick_geo(h.tu, h.H);
    if (!gg.G || !gd.G || gg.UPL != 1 || gu.G != gg.G || gu.UPL != 1 ||
        blk_elems(h.tg) != blk_elems(h.tu))
        return false;
    if (h.F > MB_MAX_F || h.F % 32 || h.H % 32 || h.H > XQ_MAX || h.E % 16 || h.E > MAX_EXPERTS ||
        h.k < 1 || h.k > MAX_TOPK || h.k > h.E || h.route.arena_mode)
        return false;
    a.nslots = h.k + (h.sh[0] ? 1 : 0);
    a.nRed = (h.H + MB_RR - 1) / MB_RR;
    // one gate/up block per workgroup, its rows of both matrices (half the
    // waves each): the walker keeps the next MB_GU_ROWS rows per lane group
    // in flight while a batch is consumed
    const int ngrp_gu = (WAVES / 2) * (64 / gg.G), ngrp_d = WAVES * (64 / gd.G);
    int rpw = (a.nslots * h.F + nwg - 1) / nwg;
    a.rpw_gu = (rpw + ngrp_gu - 1) / ngrp_gu * ngrp_gu;
    a.bps_gu = (h.F + a.rpw_gu - 1) / a.rpw_gu;
    a.n_gu = a.nslots * a.bps_gu;
    if (nwg % MB_TICKETS) return false;
    const int per_slot = nwg / a.nslots;
    if (per_slot < 1) return false;
    rpw = (h.H + per_slot - 1) / per_slot;
    a.rpw_d = std::max(ngrp_d, (rpw + ngrp_d - 1) / ngrp_d * ngrp_d);
    a.bps_d = (h.H + a.rpw_d - 1) / a.rpw_d;
    a.n_d = a.nslots * a.bps_d;
    // one router row per workgroup while there are enough gate/up
    // workgroups (each extra row lengthens its workgroup's entry loads),
    // else up to RT_ROWS
    a.rt_rows = (h.E + a.n_gu - 1) / a.n_gu;
    if (a.rt_rows > RT_ROWS) return false;
    a.nR = (h.E + a.rt_rows - 1) / a.rt_rows;
    // every workgroup that reads x at entry has gate/up work, whose outputs
    // the reduce (which rewrites x) waits on
    if (a.n_d > nwg || a.nR > a.n_gu || a.nRed > a.n_gu) return false;
    a.n_q = 0;
    if (h.wqkv[0]) {
        const Geo gq = pick_geo(T_Q8_0, h.H);
        if (!gq.G || gq.UPL > 2 || h.H > MB_MAX_H || !h.t_xq || !h.norm_next || !h.wqkv[1] ||
            !h.wqkv[2] || !h.qkv_out[0] || !h.qkv_out[1] || !h.qkv_out[2])
            return false;
        const int rows = h.qkv_rows[0] + h.qkv_rows[1] + h.qkv_rows[2];
        const int ngrp_q = WAVES * (64 / gq.G), avail = nwg - a.nRed;
        if (avail < 1) return false;
        const int r = (rows + avail - 1) / avail;
        a.G_q = gq.G;
        a.UPL_q = gq.UPL;
        a.nb_q = h.H / 32;
        a.rpw_q = std::max(ngrp_q, (r + ngrp_q - 1) / ngrp_q * ngrp_q);
        a.n_q = (rows + a.rpw_q - 1) / a.rpw_q;
        // the partial sums land after the limbs, in the logits' LDS
        if (a.nRed + a.n_q > nwg || a.nRed > h.E) return false;
    }
    a.G_gu = gg.G;
    a.nb_gu = h.H / blk_elems(h.tg);
    a.G_d = gd.G;
    a.nb_d = h.F / blk_elems(h.td);
    a.off_xq = align16((size_t)4 * h.H);
    a.off_lg = a.off_xq + align16(xq_bytes(h.H));
    a.off_gu = a.off_lg + align16((size_t)4 * h.E);
    // gate/up rows of a block (2 rpw) | h (F) | the reduce's partials
    a.off_hs = a.off_gu + align16(std::max({(size_t)8 * a.rpw_gu, (size_t)4 * h.F,
                                            (size_t)4 * a.nslots * MB_RR}));
    a.off_xqh = a.off_hs + align16((size_t)4 * MB_RR);
    lds = (size_t)a.off_xqh + align16(xq_bytes(h.F));
    return true;
}

bool moe_block_fold_ok(int tg, int tu, int td, int H, int F, int E, int k, int shexp,
                       const int rows[3], int nwg)
{
    static const uint8_t dummy = 0;
    static uint64_t dummy_t = 0;
    static float dummy_f = 0.0f;
    MoeBlockArgs h{};
    h.tg = tg;
    h.tu = tu;
    h.td = td;
    h.H = H;
    h.F = F;
    h.E = E;
    h.k = k;
    if (shexp) h.sh[0] = h.sh[1] = h.sh[2] = &dummy;
    h.norm_next = &dummy_f;
    h.t_xq = &dummy_t;
    for (int i = 0; i < 3; i++) {
        h.wqkv[i] = &dummy;
        h.qkv_out[i] = &dummy_f;
        h.qkv_rows[i] = rows[i];
    }
    MoeBlockK a{};
    size_t lds = 0;
    return moe_geometry(h, nwg, a, lds);
}

int moe_block_occupancy(int tg, int tu, int td, int H, int F, int E, int k, int shexp)
{
    MoeKernel kf = moe_kernel(td, pick_geo(td, F).UPL);
    if (!kf) return 0;
    MoeBlockArgs h{};
    h.tg = tg;
    h.tu = tu;
    h.td = td;
    h.H = H;
    h.F = F;
    h.E = E;
    h.k = k;
    static const uint8_t dummy = 0;
    if (shexp) h.sh[0] = h.sh[1] = h.sh[2] = &dummy;
    MoeBlockK a{};
    size_t lds = 0;
    if (!moe_geometry(h, 512, a, lds)) return 0;  // the LDS size does not depend on the grid
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, (const void *)kf, WG, lds) != hipSuccess)
        return 0;
    return n;
}

hipError_t launch_moe_block(hipStream_t st, const MoeBlockArgs &h)
{
    MoeKernel kf = moe_kernel(h.td, pick_geo(h.td, h.F).UPL);
    if (!kf || h.nwg < 1 || !h.x || !h.ffn_norm || !h.W || !h.t_lg || !h.t_gu || !h.t_part ||
        !h.ticket || !h.abort || (h.sh[0] && (!h.sh[1] || !h.sh[2] || !h.sh_ginp)) ||
        (h.norm_next && (!h.xq.A || !h.ss)))
        return hipErrorInvalidValue;
    MoeBlockK a{};
    size_t lds = 0;
    if (!moe_geometry(h, h.nwg, a, lds)) return hipErrorNotSupported;
    a.x = h.x;
    a.ffn_norm = h.ffn_norm;
    a.W = h.W;
    a.bias = h.bias;
    a.sh_ginp = h.sh_ginp;
    for (int i = 0; i < 3; i++) {
        a.sh[i] = h.sh[i];
        a.src[i] = h.src[i];
    }
    a.route = h.route;
    a.route.logits = nullptr;
    a.route.E = h.E;
    a.route.k = h.k;
    a.eps = h.eps;
    a.H = h.H;
    a.F = h.F;
    a.E = h.E;
    a.k = h.k;
    a.renorm = h.renorm;
    a.tg = h.tg;
    a.tu = h.tu;
    a.x_out = h.x;
    a.norm_next = h.norm_next;
    a.xq = h.xq;
    a.ss = h.ss;
    a.wts_out = h.wts_out;
    a.t_lg = h.t_lg;
    a.t_gu = h.t_gu;
    a.t_part = h.t_part;
    a.ticket = h.ticket;
    a.abort = h.abort;
    a.max_polls = h.max_polls > 0 ? h.max_polls : 200000;
    a.trace = h.trace;
    for (int i = 0; i < 3; i++) {
        a.wqkv[i] = h.wqkv[i];
        a.qkv_out[i] = h.qkv_out[i];
        a.qkv_rows[i] = h.qkv_rows[i];
    }
    a.t_xq = h.t_xq;
    hipLaunchKernelGGL(kf, dim3(h.nwg), dim3(WG), lds, st, a);
    return hipGetLastError();
}

}  // namespace styx
