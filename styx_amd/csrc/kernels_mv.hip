// kernels_mv.hip -- dequant-matvec kernels of the MoE decode hot path (gfx950).
//
//   k_xq            activation limbs (see qdot.h) of x, rmsnorm(x)*w or
//                   swiglu(g, u), one workgroup; used where no producer
//                   kernel writes them itself.
//   k_mv_dense      q/k/v, o-proj (+residual), LM head, shared expert: rows of
//                   one or up to three split-layout matrices against one limb
//                   vector.
//   k_router        ffn RMSNorm (rms_norm_f32 semantics, moe.rs:1746-1766) +
//                   f32 router matvec (shaders/matvec_strided_f32.comp); its
//                   first workgroup also writes the normalised vector and its
//                   limbs for the expert kernels.
//   k_gate_up       expert gate and up matvecs for the k routed slots
//                   (mul_mat_vec_id semantics, ne11 = 1), top-k ids ranked
//                   in-kernel from the router logits.
//   k_down          expert down matvec, swiglu + limbs of the slot's hidden
//                   vector built in LDS in front; per-slot rows to partial[s]
//                   (the shared expert as one more slot).
//   k_reduce_rows   topk_softmax weights of the selected ids, moe_reduce
//                   (x += sum_s w_s y_s, s ascending), the shared-expert
//                   axpy_sig, then the limbs of x ⊙ w for the next RMSNorm
//                   (whose scale the next matvec applies); 256 rows per
//                   workgroup.
//
// No kernel waits on another workgroup: every producer writes what its
// consumers read before the kernel boundary, so there is no device-scope
// fence or counter anywhere on the path.
#include "kernels.h"
#include "qdot.h"
#include "router.h"
#include "topk.h"
#include "walk.h"

#include <algorithm>
#include <type_traits>

namespace styx {

Geo pick_geo(int t, int ncols)
{
    Geo g{0, 0, 0};
    if (!is_quant(t) || ncols % blk_elems(t) != 0) return g;
    const int units = ncols / blk_elems(t) * units_per_blk(t);
    const int max_upl = t == T_Q8_0 ? 4 : 2;
    // lane groups of a power of two (a row's sum is then a butterfly of
    // lane permutes within a DPP row; a group of 12 needed dependent LDS
    // permutes), lanes past the row's units idle; the most lanes with units
    // per wave wins, then the fewest units per lane
    int best_used = -1;
    for (int upl = 1; upl <= max_upl; upl++) {
        if (units % upl) continue;
        const int Gu = units / upl;
        if (Gu > 64) continue;
        int G = 1;
        while (G < Gu) G *= 2;
        const int used = (64 / G) * Gu;
        if (used > best_used) {
            best_used = used;
            g.G = G;
            g.UPL = upl;
        }
    }
    g.units = units;
    return g;
}

// Units per lane are a compile-time parameter of every matvec kernel: one
// kernel per (type, UPL) keeps the register file to what that geometry
// needs (the activation limbs of UPL units live in registers), which sets
// the occupancy.
template <int N> using IC = std::integral_constant<int, N>;

template <int T, typename F> static void upl_dispatch(int upl, F f)
{
    if constexpr (T == T_Q8_0) {
        switch (upl) {
        case 1: f(IC<1>{}); break;
        case 2: f(IC<2>{}); break;
        case 3: f(IC<3>{}); break;
        default: f(IC<4>{}); break;
        }
    } else {
        if (upl == 1)
            f(IC<1>{});
        else
            f(IC<2>{});
    }
}

// Rows per workgroup: about `target` workgroups over `rows` rows, at least
// two rows per lane group, whole passes of the workgroup's groups.
static int rows_per_wg(int rows, int G, int target)
{
    const int ngrp = WAVES * (64 / G);
    int rpw = (rows + target - 1) / target;
    rpw = std::max(rpw, 2 * ngrp);
    return (rpw + ngrp - 1) / ngrp * ngrp;
}

// --------------------------------------------------------------- limbs ---
__global__ void __launch_bounds__(WG) k_xq(const float *x, const float *u, const float *nw,
                                           float eps, int n, Xq q, float *xn_out)
{
    extern __shared__ __align__(16) float hs[];
    __shared__ float red[16];
    if (u) {
        // swiglu_f32 (ops2.rs:305-309)
        for (int i = threadIdx.x; i < n; i += WG) hs[i] = x[i] / (1.0f + expf(-x[i])) * u[i];
        __syncthreads();
        xq_build(hs, nullptr, 0.0f, false, n, q, red, xn_out);
    } else {
        xq_build(x, nw, eps, nw != nullptr, n, q, red, xn_out);
    }
}

hipError_t launch_xq(hipStream_t st, const float *x, const float *u, const float *norm_w,
                     float eps, int n, const Xq &q, float *xn_out)
{
    if (n < 32 || n % 32 || n > XQ_MAX) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_xq, dim3(1), dim3(WG), u ? (size_t)n * 4 : 0, st, x, u, norm_w, eps, n,
                       q, xn_out);
    return hipGetLastError();
}

// ------------------------------------------------------------------ dense --
struct DenseK {
    const uint8_t *w[3];
    float *y[3];
    int rows[3];
    int nseg, total, nb, G, UPL, rpw, add;
    Xq xq;
    NormScale ns;  // ns.ss == null: no RMSNorm scale
    unsigned long long *amax;  // optional: running argmax word (argmax_key)
};

// Rows per lane group and batch of the dense walk: two batches are in
// flight, of more rows where a lane holds fewer units.
template <int UPL> constexpr int dense_nr() { return UPL <= 2 ? 2 : 1; }

// GC: the lane-group width when it is 64 (a whole wave per row: q/k/v,
// o-proj and LM head of the configs), known at compile time so that the
// walk's lane map and row sums fold; 0: a.G.
// STAGE (q8_0 rows of 64-lane groups whose limb buffer is one xq_at block
// of a multiple of 128 values): every wave reads the whole limb vector, so
// the workgroup loads it once, 2 UPL 16-byte pieces per thread issued before
// the weights, and the waves read it from LDS -- a quarter of the limb
// traffic through the CU's memory pipeline.  Taken for workgroups of many
// rows (the launcher's choice).
template <int T, int UPL, int GC, bool STAGE>
__global__ void __launch_bounds__(WG) k_mv_dense(DenseK a)
{
    const int r_begin = blockIdx.x * a.rpw, r_end = min(a.total, r_begin + a.rpw);
    constexpr int XC = STAGE ? 2 * UPL : 1;
    extern __shared__ __align__(16) uint8_t s_xq[];
    const int ncols = a.nb * blk_elems(T);
    const int nxc = STAGE ? (int)(xq_bytes(ncols) / 16) : 0;
    styx_u4 xc[XC];
    if constexpr (STAGE) {
        // unconditional loads (a piece past the end reads the last one), so
        // that the wait for them leaves the weights issued after in flight
        const styx_u4 STYX_GLOBAL *src = (const styx_u4 STYX_GLOBAL *)a.xq.A;
#pragma unroll
        for (int j = 0; j < XC; j++) xc[j] = src[min((int)threadIdx.x + WG * j, nxc - 1)];
    }
    unsigned long long best = 0;  // argmax_key of the best row this lane emitted
    // the segments are walked as one stack of rows, so that a workgroup's
    // rows that span two segments stream in one pass
    const int b1 = a.rows[0], b2 = b1 + (a.nseg > 1 ? a.rows[1] : 0);
    const Mat m0 = mat_at(a.w[0], T, (int64_t)a.rows[0] * a.nb);
    const Mat m1 = a.nseg > 1 ? mat_at(a.w[1], T, (int64_t)a.rows[1] * a.nb) : m0;
    const Mat m2 = a.nseg > 2 ? mat_at(a.w[2], T, (int64_t)a.rows[2] * a.nb) : m1;
    const int add = a.add;
    // the RMSNorm scale is summed while the first weights are in flight
    float scale = 1.0f;
    auto xload = [&](UX<T> (&x)[UPL], const LaneU<UPL> &lu) {
        if constexpr (STAGE) {
#pragma unroll
            for (int j = 0; j < XC; j++)
                if ((int)threadIdx.x + WG * j < nxc) ((styx_u4 *)s_xq)[threadIdx.x + WG * j] = xc[j];
            __syncthreads();
            XFrom<T, UPL>{xq_at(s_xq, ncols)}(x, lu);
        } else {
            XFrom<T, UPL>{a.xq}(x, lu);
        }
        if (a.ns.ss) {
            float t = 0.0f;
            for (int i = threadIdx.x & 63; i < a.ns.n_ss; i += 64) t += a.ns.ss[i];
            t = wave_sum(t);
            scale = 1.0f / sqrtf(t / (float)a.ns.n + a.ns.eps);
        }
        return true;
    };
    auto y_of = [&](int r) {
        const int s = (int)(r >= b1) + (int)(r >= b2);
        return s == 0 ? a.y[0] + r : s == 1 ? a.y[1] + (r - b1) : a.y[2] + (r - b2);
    };
    // a residual add with at most one row per thread reads the residual at
    // entry (it does not depend on the dot products) and adds it after the
    // walk, instead of a dependent load at the end of each row
    __shared__ float s_out[WG];
    const bool early = add && a.rpw <= WG;
    const int tr = r_begin + (int)threadIdx.x;
    float res = 0.0f;
    if (early && tr < r_end) res = *y_of(tr);
    auto emit = [&](int r, float v) {
        v *= scale;
        if (early) {
            s_out[r - r_begin] = v;
            return;
        }
        float *y = y_of(r);
        v = add ? *y + v : v;
        *y = v;
        if (a.amax) best = max(best, argmax_key(v, (uint32_t)r));
    };
    if (a.nseg == 1)
        walk_rows_pipelined<T, UPL, dense_nr<UPL>()>(OneMat{m0, a.nb}, a.nb, GC ? GC : a.G, r_begin, r_end,
                                                      xload, emit);
    else
        walk_rows_pipelined<T, UPL, dense_nr<UPL>()>(Mat3(m0, m1, m2, b1, b2, a.nb), a.nb, GC ? GC : a.G,
                                                      r_begin, r_end, xload, emit);
    if (early) {
        __syncthreads();
        if (tr < r_end) {
            const float v = res + s_out[threadIdx.x];
            *y_of(tr) = v;
            if (a.amax) best = max(best, argmax_key(v, (uint32_t)tr));
        }
    }
    if (a.amax) {
        // the workgroup's best row joins the launch's running maximum: one
        // relaxed device-scope atomic per workgroup (the reading kernel runs
        // after this one)
        __shared__ unsigned long long s_best[WAVES];
        for (int o = 32; o > 0; o >>= 1) best = max(best, (unsigned long long)__shfl_xor(best, o));
        if ((threadIdx.x & 63) == 0) s_best[threadIdx.x >> 6] = best;
        __syncthreads();
        if (threadIdx.x == 0) {
            for (int i = 1; i < WAVES; i++) best = max(best, s_best[i]);
            __hip_atomic_fetch_max(a.amax, best, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

hipError_t launch_dense(hipStream_t st, int t, int ncols, const DenseSeg *segs, int nseg,
                        const Xq &xq, int add, const NormScale *ns, unsigned long long *amax)
{
    const Geo g = pick_geo(t, ncols);
    if (g.G == 0 || nseg < 1 || nseg > 3 || !xq.A) return hipErrorInvalidValue;
    DenseK a{};
    a.total = 0;
    for (int i = 0; i < nseg; i++) {
        a.w[i] = segs[i].w;
        a.y[i] = segs[i].y;
        a.rows[i] = segs[i].rows;
        a.total += segs[i].rows;
    }
    a.nseg = nseg;
    a.nb = ncols / blk_elems(t);
    a.G = g.G;
    a.UPL = g.UPL;
    a.add = add;
    a.xq = xq;
    if (ns) a.ns = *ns;
    a.amax = amax;
    a.rpw = rows_per_wg(a.total, g.G, 1024);
    const dim3 grid((a.total + a.rpw - 1) / a.rpw);
    // the limb buffer as one xq_at block, staged in LDS by q8_0 64-lane walks
    // of one unit per lane and many rows per workgroup (the LM head of
    // 60.4 -> 58.0 us) and of four units per lane (the 8192
    // columns of configs[3]'s o-proj: 9.5 -> 8.3 us, its 27 KB of limbs
    // read by each of eight waves per CU otherwise).  With two units per
    // lane it measured slower: configs[1]'s o-proj (few rows: the barrier
    // costs more than the repeated reads, which hit the CU's cache; 4.3 ->
    // 4.5 us) and configs[3]'s LM head (the staging registers cost
    // occupancy; 108 -> 113 us)
    const Xq xc = xq_at(xq.A, ncols);
    const bool stage = ((g.UPL == 1 && a.rpw >= 32) || g.UPL == 4) && ncols % 128 == 0 && ((uintptr_t)xq.A & 15) == 0 && xq.B == xc.B &&
                       xq.C == xc.C && xq.sx == xc.sx && xq.s16 == xc.s16;
    const size_t lds_xq = stage ? xq_bytes(ncols) : 0;
    switch (t) {
    case T_Q8_0: upl_dispatch<T_Q8_0>(g.UPL, [&](auto u) {
        constexpr int U = decltype(u)::value;
        if (g.G == 64 && stage) hipLaunchKernelGGL((k_mv_dense<T_Q8_0, U, 64, true>), grid, dim3(WG), lds_xq, st, a);
        else if (g.G == 64) hipLaunchKernelGGL((k_mv_dense<T_Q8_0, U, 64, false>), grid, dim3(WG), 0, st, a);
        else hipLaunchKernelGGL((k_mv_dense<T_Q8_0, U, 0, false>), grid, dim3(WG), 0, st, a); }); break;
    case T_Q4_K: upl_dispatch<T_Q4_K>(g.UPL, [&](auto u) {
        if (g.G == 64) hipLaunchKernelGGL((k_mv_dense<T_Q4_K, decltype(u)::value, 64, false>), grid, dim3(WG), 0, st, a);
        else hipLaunchKernelGGL((k_mv_dense<T_Q4_K, decltype(u)::value, 0, false>), grid, dim3(WG), 0, st, a); }); break;
    case T_Q5_K: upl_dispatch<T_Q5_K>(g.UPL, [&](auto u) {
        if (g.G == 64) hipLaunchKernelGGL((k_mv_dense<T_Q5_K, decltype(u)::value, 64, false>), grid, dim3(WG), 0, st, a);
        else hipLaunchKernelGGL((k_mv_dense<T_Q5_K, decltype(u)::value, 0, false>), grid, dim3(WG), 0, st, a); }); break;
    case T_Q6_K: upl_dispatch<T_Q6_K>(g.UPL, [&](auto u) {
        if (g.G == 64) hipLaunchKernelGGL((k_mv_dense<T_Q6_K, decltype(u)::value, 64, false>), grid, dim3(WG), 0, st, a);
        else hipLaunchKernelGGL((k_mv_dense<T_Q6_K, decltype(u)::value, 0, false>), grid, dim3(WG), 0, st, a); }); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

__global__ void __launch_bounds__(64) k_topk(const float *logits, int n, int k, int renorm,
                                              const uint32_t *remap, const uint32_t *pmap,
                                              int arena_mode, int layer, float *wts,
                                              int32_t *ids)
{
    topk_wave(logits, n, k, renorm, remap, pmap, arena_mode, layer, wts, ids);
}

hipError_t launch_topk_softmax(hipStream_t st, const float *logits, int n, int k, int renorm,
                               const uint32_t *remap, const uint32_t *pmap, int arena_mode,
                               int layer, float *wts, int32_t *ids)
{
    if (n < 1 || n > MAX_EXPERTS || k < 1 || k > MAX_TOPK || k > n) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_topk, dim3(1), dim3(64), 0, st, logits, n, k, renorm, remap, pmap,
                       arena_mode, layer, wts, ids);
    return hipGetLastError();
}

// ------------------------------------------------------------- router ----
// ffn RMSNorm fused in front of the f32 router matvec
// (shaders/matvec_strided_f32.comp); one row per wave.  The top-k ids are
// ranked by each consumer workgroup from these logits (route_ids_wg) and the
// weights by k_reduce_norm, so no workgroup ever waits on another.

__global__ void __launch_bounds__(WG) k_router(RouterArgs a)
{
    extern __shared__ __align__(16) uint8_t lds[];
    float *xs = (float *)lds;          // x (.) w, H floats
    __shared__ float red[RT_RED];
    const int r0 = blockIdx.x * RT_ROWS;
    // x, the norm weight and the workgroup's RT_ROWS rows at columns
    // 4 t + 1024 j of thread t (router.h; the fused MoE block's order)
    const float *wr[RT_ROWS];
#pragma unroll
    for (int r = 0; r < RT_ROWS; r++) wr[r] = a.W + (int64_t)min(r0 + r, a.E - 1) * a.H;
    float ss = 0.0f, p[RT_ROWS] = {};
    for (int i = threadIdx.x * 4; i < a.H; i += WG * 4) {
        const float4 xv = *(const float4 *)(a.x + i);
        const float4 nv = *(const float4 *)(a.norm_w + i);
        float4 wv[RT_ROWS];
#pragma unroll
        for (int r = 0; r < RT_ROWS; r++) wv[r] = *(const float4 *)(wr[r] + i);
        *(float4 *)(xs + i) = router_acc(xv, nv, wv, RT_ROWS, ss, p);
    }
    router_wave_part(ss, p, RT_ROWS, red);
    __syncthreads();
    const float scale = router_scale(red, a.H, a.eps);
    if ((int)threadIdx.x < RT_ROWS && r0 + (int)threadIdx.x < a.E) {
        const int r = r0 + threadIdx.x;
        const float lg = scale * router_dot(red, threadIdx.x);
        a.logits[r] = a.bias ? lg + a.bias[r] : lg;
    }
    if (blockIdx.x != 0 || (!a.xq.A && !a.xn)) return;
    // the first workgroup: xn = rmsnorm(x) * w (the reference's (x s) w)
    // for the separate expert kernels, and its limbs
    for (int i = threadIdx.x * 4; i < a.H; i += WG * 4) {
        const float4 xv = *(const float4 *)(a.x + i);
        const float4 nv = *(const float4 *)(a.norm_w + i);
        *(float4 *)(xs + i) = make_float4((xv.x * scale) * nv.x, (xv.y * scale) * nv.y,
                                          (xv.z * scale) * nv.z, (xv.w * scale) * nv.w);
    }
    __syncthreads();
    if (a.xq.A)
        xq_build(xs, nullptr, 0.0f, false, a.H, a.xq, red, a.xn);
    else
        for (int i = threadIdx.x * 4; i < a.H; i += WG * 4)
            *(float4 *)(a.xn + i) = *(const float4 *)(xs + i);
}

hipError_t launch_router(hipStream_t st, const RouterArgs &a)
{
    if (a.E < 1 || a.E > MAX_EXPERTS || a.H % 32 || a.H > XQ_MAX) return hipErrorInvalidValue;
    const int nwg = (a.E + RT_ROWS - 1) / RT_ROWS;
    hipLaunchKernelGGL(k_router, dim3(nwg), dim3(WG), (size_t)a.H * 4, st, a);
    return hipGetLastError();
}

hipError_t launch_router_topk(hipStream_t st, const RouterArgs &a)
{
    if (a.k < 1 || a.k > MAX_TOPK || a.k > a.E) return hipErrorInvalidValue;
    hipError_t e = launch_router(st, a);
    if (e != hipSuccess) return e;
    return launch_topk_softmax(st, a.logits, a.E, a.k, a.renorm, a.remap, a.pmap, a.arena_mode,
                               a.layer, a.wts, a.ids);
}

// ------------------------------------------------------------ gate / up ---
// Whether a slot with hot id h (SKIP: not hot) passes the launch's filter
// (SlotFilter); the shared expert slot counts as hot.
__device__ __forceinline__ bool slot_passes(int filter, bool hot)
{
    return filter == SLOTS_ALL || (filter == SLOTS_HOT) == hot;
}

struct GateUpK {
    ExpSrc src[2];
    const uint8_t *sh[2];  // shared expert gate/up matrices (slot k) or null
    int G;
    const int32_t *ids;   // id row in memory, used when route.logits is null
    Route route;
    Xq xq;
    float *gu;  // [2][nslots][F]
    int F, k, nslots, nb, rpw, filter;
    // one expert id per slot (a single row of the id table), or null: slot
    // s reads slab id_one[s] of src[m].hot; an id at or past n_slabs (SKIP
    // among them) leaves the slot's outputs untouched
    const int32_t *id_one;
    uint32_t n_slabs;
    float *h;  // k_gate_up_silu: [nslots][F] = silu(gate rows) * up rows
};

// Slab of matrix m (0 gate, 1 up) for slot s < k from an id row in memory
// (the id_one row, or the hot / arena / host rows), or null when the slot
// is skipped (by its ids or the launch's filter).
__device__ __forceinline__ const uint8_t *gu_slab_of_ids(const GateUpK &a, int m, int s)
{
    if (a.id_one) {
        const uint32_t e = (uint32_t)a.id_one[s];
        return e < a.n_slabs ? a.src[m].hot + (int64_t)e * a.src[m].hot_slab : nullptr;
    }
    uint32_t r3[3];
    for (int j = 0; j < 3; j++) r3[j] = (uint32_t)a.ids[16 * (j + 1) + s];
    if (!slot_passes(a.filter, r3[0] != SKIP)) return nullptr;
    return slab_pick(a.src[m], r3[0], r3[1], r3[2]);
}

// Routing first (one trip for the logits, then LDS work), then the slot's
// weight loads, then the activation limbs.
template <int T, int UPL>
__device__ inline void gate_up_body(const GateUpK &a, int m, int s, int32_t *s_ids, float *s_lg)
{
    const uint8_t *slab;
    if (s < a.k) {
        if (a.route.logits) {
            uint32_t r3[3];
            const int32_t *ids = route_ids_wg(a.route, s_ids, s_lg);
            route_row(a.route, ids[s], s, r3);
            if (!slot_passes(a.filter, r3[0] != SKIP)) return;
            slab = slab_pick(a.src[m], r3[0], r3[1], r3[2]);
        } else {
            slab = gu_slab_of_ids(a, m, s);
        }
    } else {
        if (!slot_passes(a.filter, true)) return;
        slab = a.sh[m];  // the shared expert needs no routing
    }
    if (!slab) return;
    const Mat mat = mat_at(slab, T, (int64_t)a.F * a.nb);
    const int r_begin = blockIdx.x * a.rpw, r_end = min(a.F, r_begin + a.rpw);
    float *y = a.gu + ((int64_t)m * a.nslots + s) * a.F;
    // one row per batch: these launches give a lane group about two rows,
    // and a second register set of more would cost occupancy
    walk_rows_pipelined<T, UPL, 1>(
        OneMat{mat, a.nb}, a.nb, a.G, r_begin, r_end,
        [&](UX<T>(&x)[UPL], const LaneU<UPL> &lu) {
            XFrom<T, UPL>{a.xq}(x, lu);
            return true;
        },
        [=](int r, float v) { y[r] = v; });
}

template <int TG, int TU, int UPL>
__global__ void __launch_bounds__(WG) k_gate_up(GateUpK a)
{
    __shared__ int32_t s_ids[IDS_ROW];
    __shared__ __align__(16) float s_lg[MAX_EXPERTS];
    const int s = blockIdx.y, m = blockIdx.z;
    if (m == 0)
        gate_up_body<TG, UPL>(a, 0, s, s_ids, s_lg);
    else
        gate_up_body<TU, UPL>(a, 1, s, s_ids, s_lg);
}

// Gate and up rows [r0, r1) of one slot in one workgroup, then
// h = swiglu_f32(g, u) (ops2.rs:305-309) of those rows: the gate rows' first
// weights are issued, then the up rows are walked, then the gate rows; both
// land in LDS.  Ids from an id row in memory (no in-kernel routing).  A
// skipped slot writes nothing.
template <int TG, int TU, int UPL>
__global__ void __launch_bounds__(WG) k_gate_up_silu(GateUpK a)
{
    extern __shared__ __align__(16) float s_gu[];  // gate rows | up rows of the block
    const int s = blockIdx.y;
    const uint8_t *sg = s < a.k ? gu_slab_of_ids(a, 0, s) : a.sh[0];
    const uint8_t *su = s < a.k ? gu_slab_of_ids(a, 1, s) : a.sh[1];
    if (!sg || !su) return;
    const int r_begin = blockIdx.x * a.rpw, r_end = min(a.F, r_begin + a.rpw);
    float *gs = s_gu, *us = s_gu + a.rpw;
    walk_rows_pipelined<TG, UPL, 1>(
        OneMat{mat_at(sg, TG, (int64_t)a.F * a.nb), a.nb}, a.nb, a.G, r_begin, r_end,
        [&](UX<TG>(&x)[UPL], const LaneU<UPL> &lu) {
            walk_rows_pipelined<TU, UPL, 1>(
                OneMat{mat_at(su, TU, (int64_t)a.F * a.nb), a.nb}, a.nb, a.G, r_begin, r_end,
                [&](UX<TU>(&xu)[UPL], const LaneU<UPL> &luu) {
                    XFrom<TU, UPL>{a.xq}(xu, luu);
                    return true;
                },
                [&](int r, float v) { us[r - r_begin] = v; });
            XFrom<TG, UPL>{a.xq}(x, lu);
            return true;
        },
        [&](int r, float v) { gs[r - r_begin] = v; });
    __syncthreads();
    float *h = a.h + (int64_t)s * a.F;
    for (int i = threadIdx.x; i < r_end - r_begin; i += WG) {
        const float g = gs[i];
        h[r_begin + i] = g / (1.0f + expf(-g)) * us[i];
    }
}

// gate and up share the block size, so one geometry serves both
template <int TG>
static hipError_t launch_gu_tu(hipStream_t st, int tu, int upl, const GateUpK &a, dim3 grid)
{
    if constexpr (TG == T_Q8_0) {
        if (tu != T_Q8_0) return hipErrorInvalidValue;
        upl_dispatch<T_Q8_0>(upl, [&](auto u) { hipLaunchKernelGGL((k_gate_up<TG, T_Q8_0, decltype(u)::value>), grid, dim3(WG), 0, st, a); });
    } else {
        switch (tu) {
        case T_Q4_K: upl_dispatch<T_Q4_K>(upl, [&](auto u) { hipLaunchKernelGGL((k_gate_up<TG, T_Q4_K, decltype(u)::value>), grid, dim3(WG), 0, st, a); }); break;
        case T_Q5_K: upl_dispatch<T_Q5_K>(upl, [&](auto u) { hipLaunchKernelGGL((k_gate_up<TG, T_Q5_K, decltype(u)::value>), grid, dim3(WG), 0, st, a); }); break;
        case T_Q6_K: upl_dispatch<T_Q6_K>(upl, [&](auto u) { hipLaunchKernelGGL((k_gate_up<TG, T_Q6_K, decltype(u)::value>), grid, dim3(WG), 0, st, a); }); break;
        default: return hipErrorInvalidValue;
        }
    }
    return hipGetLastError();
}

hipError_t launch_moe_gate_up(hipStream_t st, int tg, int tu, const ExpSrc &g, const ExpSrc &u,
                              const int32_t *ids, const Route *route, const Xq &xq, float *gu,
                              int H, int F, int k, const uint8_t *sh_gate, const uint8_t *sh_up,
                              int filter)
{
    const Geo gg = pick_geo(tg, H);
    if (!gg.G || blk_elems(tg) != blk_elems(tu) || k < 1 || k > MAX_TOPK || !xq.A)
        return hipErrorInvalidValue;
    if (route && (route->E < k || route->E > MAX_EXPERTS || route->E % 16 || route->k != k))
        return hipErrorInvalidValue;
    if (!route && !ids) return hipErrorInvalidValue;
    GateUpK a{};
    a.src[0] = g;
    a.src[1] = u;
    a.sh[0] = sh_gate;
    a.sh[1] = sh_up;
    a.nslots = k + ((sh_gate && sh_up) ? 1 : 0);
    a.G = gg.G;
    a.ids = ids;
    if (route) a.route = *route;
    a.xq = xq;
    a.gu = gu;
    a.F = F;
    a.k = k;
    a.filter = filter;
    a.nb = H / blk_elems(tg);
    // ~1024 workgroups in total over the 2*k slot matrices
    a.rpw = rows_per_wg(2 * a.nslots * F, gg.G, 1024);
    const dim3 grid((F + a.rpw - 1) / a.rpw, a.nslots, 2);
    switch (tg) {
    case T_Q8_0: return launch_gu_tu<T_Q8_0>(st, tu, gg.UPL, a, grid);
    case T_Q4_K: return launch_gu_tu<T_Q4_K>(st, tu, gg.UPL, a, grid);
    case T_Q5_K: return launch_gu_tu<T_Q5_K>(st, tu, gg.UPL, a, grid);
    case T_Q6_K: return launch_gu_tu<T_Q6_K>(st, tu, gg.UPL, a, grid);
    default: return hipErrorInvalidValue;
    }
}

template <int TG, int TU>
static void launch_gus(hipStream_t st, int upl, const GateUpK &a, dim3 grid, size_t lds)
{
    upl_dispatch<TG>(upl, [&](auto u) {
        hipLaunchKernelGGL((k_gate_up_silu<TG, TU, decltype(u)::value>), grid, dim3(WG), lds, st, a);
    });
}

hipError_t launch_moe_gate_up_silu(hipStream_t st, int tg, int tu, const uint8_t *wg,
                                   int64_t slab_g, const uint8_t *wu, int64_t slab_u,
                                   const int32_t *ids, uint32_t n_slabs, const Xq &xq, float *h,
                                   int H, int F, int k)
{
    const Geo gg = pick_geo(tg, H), gu = pick_geo(tu, H);
    if (!gg.G || gu.G != gg.G || gu.UPL != gg.UPL || blk_elems(tg) != blk_elems(tu) || k < 1 ||
        k > MAX_TOPK || !xq.A || !wg || !wu || !ids || !h || F < 1)
        return hipErrorInvalidValue;
    GateUpK a{};
    a.src[0].hot = wg;
    a.src[0].hot_slab = slab_g;
    a.src[1].hot = wu;
    a.src[1].hot_slab = slab_u;
    a.nslots = k;
    a.G = gg.G;
    a.id_one = ids;
    a.n_slabs = n_slabs;
    a.xq = xq;
    a.h = h;
    a.F = F;
    a.k = k;
    a.nb = H / blk_elems(tg);
    // ~512 workgroups, each a row block of one slot's gate and up
    a.rpw = rows_per_wg(a.nslots * F, gg.G, 512);
    const dim3 grid((F + a.rpw - 1) / a.rpw, a.nslots, 1);
    const size_t lds = (size_t)8 * a.rpw;
    auto with_tu = [&](auto tgc) {
        constexpr int TG = decltype(tgc)::value;
        if constexpr (TG == T_Q8_0) {
            if (tu != T_Q8_0) return hipErrorInvalidValue;
            launch_gus<TG, T_Q8_0>(st, gg.UPL, a, grid, lds);
        } else {
            switch (tu) {
            case T_Q4_K: launch_gus<TG, T_Q4_K>(st, gg.UPL, a, grid, lds); break;
            case T_Q5_K: launch_gus<TG, T_Q5_K>(st, gg.UPL, a, grid, lds); break;
            case T_Q6_K: launch_gus<TG, T_Q6_K>(st, gg.UPL, a, grid, lds); break;
            default: return hipErrorInvalidValue;
            }
        }
        return hipGetLastError();
    };
    switch (tg) {
    case T_Q8_0: return with_tu(IC<T_Q8_0>{});
    case T_Q4_K: return with_tu(IC<T_Q4_K>{});
    case T_Q5_K: return with_tu(IC<T_Q5_K>{});
    case T_Q6_K: return with_tu(IC<T_Q6_K>{});
    default: return hipErrorInvalidValue;
    }
}

// ------------------------------------------------------------- down -------
// partial[s] = Wd[e_s] . swiglu(g_s, u_s) for every routed slot s; the
// weighted combine into the residual is k_reduce_rows.
struct DownK {
    ExpSrc src;
    const uint8_t *sh;  // shared expert down matrix (slot k) or null
    int G, UPL;
    const int32_t *ids;
    const float *gu;    // [2][nslots][F]
    float *partial;     // [nslots][H]
    int H, F, k, nslots, nb, rpw, filter;
    // one expert id per slot, or null (as GateUpK::id_one): slab id_one[s]
    // of src.hot; a skipped slot's partial is written as zeros
    const int32_t *id_one;
    uint32_t n_slabs;
    const float *h;     // [nslots][F] already silu(g) * u (gu unused), or null
};

template <int T, int UPL>
__global__ void __launch_bounds__(WG) k_down(DownK a)
{
    extern __shared__ __align__(16) uint8_t lds[];
    __shared__ float red[16];
    const int s = blockIdx.y;
    const int r_begin = blockIdx.x * a.rpw, r_end = min(a.H, r_begin + a.rpw);
    // the id row and this slot's gate/up rows are independent loads: issue
    // both; the weights go out as soon as the ids are in, and swiglu_f32
    // (ops2.rs:305-309) with the limbs of its output is built in LDS while
    // they are in flight
    int32_t idr[3] = {(int32_t)SKIP, (int32_t)SKIP, (int32_t)SKIP};
    if (s < a.k && !a.id_one) {
#pragma unroll
        for (int j = 0; j < 3; j++) idr[j] = a.ids[16 * (j + 1) + s];
    }
    if (!a.id_one && !slot_passes(a.filter, s >= a.k || (uint32_t)idr[0] != SKIP)) return;
    constexpr int PG = 4;  // gate/up values per thread held in registers
    const float *g = a.h ? a.h + (int64_t)s * a.F : a.gu + (int64_t)s * a.F;
    const float *u = a.h ? g : a.gu + ((int64_t)a.nslots + s) * a.F;
    float gv[PG], uv[PG];
#pragma unroll
    for (int j = 0; j < PG; j++) {
        const int i = threadIdx.x + WG * j;
        gv[j] = i < a.F ? g[i] : 0.0f;
        uv[j] = (i < a.F && !a.h) ? u[i] : 0.0f;
    }
    const uint8_t *slab = a.sh;
    if (s < a.k) {
        if (a.id_one) {
            const uint32_t e = (uint32_t)a.id_one[s];
            slab = e < a.n_slabs ? a.src.hot + (int64_t)e * a.src.hot_slab : nullptr;
        } else {
            slab = slab_pick(a.src, (uint32_t)idr[0], (uint32_t)idr[1], (uint32_t)idr[2]);
        }
    }
    float *part = a.partial + (int64_t)s * a.H;
    if (!slab) {
        for (int r = r_begin + threadIdx.x; r < r_end; r += WG) part[r] = 0.0f;
        return;
    }
    const Mat mat = mat_at(slab, T, (int64_t)a.H * a.nb);
    float *hs = (float *)lds;
    const Xq q = xq_at(lds + (size_t)a.F * 4, a.F);
    auto build = [&](UX<T> (&x)[UPL], const LaneU<UPL> &lu) {
        if (a.h) {
#pragma unroll
            for (int j = 0; j < PG; j++) {
                const int i = threadIdx.x + WG * j;
                if (i < a.F) hs[i] = gv[j];
            }
            for (int i = threadIdx.x + WG * PG; i < a.F; i += WG) hs[i] = g[i];
        } else {
#pragma unroll
            for (int j = 0; j < PG; j++) {
                const int i = threadIdx.x + WG * j;
                if (i < a.F) hs[i] = gv[j] / (1.0f + expf(-gv[j])) * uv[j];
            }
            for (int i = threadIdx.x + WG * PG; i < a.F; i += WG) hs[i] = g[i] / (1.0f + expf(-g[i])) * u[i];
        }
        __syncthreads();
        xq_build(hs, nullptr, 0.0f, false, a.F, q, red, nullptr);
        __syncthreads();
        XFrom<T, UPL>{q}(x, lu);
        return true;
    };
    walk_rows_pipelined<T, UPL, 1>(OneMat{mat, a.nb}, a.nb, a.G, r_begin, r_end, build,
                                   [=](int r, float v) { part[r] = v; });  // (as k_gate_up)
}

static hipError_t launch_down_k(hipStream_t st, int td, const DownK &a, const Geo &g);

hipError_t launch_moe_down_h(hipStream_t st, int td, const uint8_t *wd, int64_t slab_d,
                             const int32_t *ids, uint32_t n_slabs, const float *h, float *partial,
                             int H, int F, int k)
{
    const Geo g = pick_geo(td, F);
    if (!g.G || k < 1 || k > MAX_TOPK || F > XQ_MAX / 2 || !wd || !ids || !h || !partial)
        return hipErrorInvalidValue;
    DownK a{};
    a.src.hot = wd;
    a.src.hot_slab = slab_d;
    a.nslots = k;
    a.G = g.G;
    a.UPL = g.UPL;
    a.id_one = ids;
    a.n_slabs = n_slabs;
    a.h = h;
    a.partial = partial;
    a.H = H;
    a.F = F;
    a.k = k;
    a.nb = F / blk_elems(td);
    a.rpw = rows_per_wg(a.nslots * H, g.G, 1024);
    return launch_down_k(st, td, a, g);
}

hipError_t launch_moe_down(hipStream_t st, int td, const ExpSrc &d, const int32_t *ids,
                           const float *gu, float *partial, int H, int F, int k,
                           const uint8_t *sh_down, int filter)
{
    const Geo g = pick_geo(td, F);
    if (!g.G || k < 1 || k > MAX_TOPK || F > XQ_MAX / 2) return hipErrorInvalidValue;
    DownK a{};
    a.src = d;
    a.sh = sh_down;
    a.nslots = k + (sh_down ? 1 : 0);
    a.G = g.G;
    a.UPL = g.UPL;
    a.ids = ids;
    a.gu = gu;
    a.partial = partial;
    a.H = H;
    a.F = F;
    a.k = k;
    a.filter = filter;
    a.nb = F / blk_elems(td);
    a.rpw = rows_per_wg(a.nslots * H, g.G, 1024);
    return launch_down_k(st, td, a, g);
}

static hipError_t launch_down_k(hipStream_t st, int td, const DownK &a, const Geo &g)
{
    const int H = a.H, F = a.F;
    const dim3 grid((H + a.rpw - 1) / a.rpw, a.nslots, 1);
    const size_t lds = (size_t)F * 4 + xq_bytes(F);
    switch (td) {
    case T_Q8_0: upl_dispatch<T_Q8_0>(g.UPL, [&](auto u) { hipLaunchKernelGGL((k_down<T_Q8_0, decltype(u)::value>), grid, dim3(WG), lds, st, a); }); break;
    case T_Q4_K: upl_dispatch<T_Q4_K>(g.UPL, [&](auto u) { hipLaunchKernelGGL((k_down<T_Q4_K, decltype(u)::value>), grid, dim3(WG), lds, st, a); }); break;
    case T_Q5_K: upl_dispatch<T_Q5_K>(g.UPL, [&](auto u) { hipLaunchKernelGGL((k_down<T_Q5_K, decltype(u)::value>), grid, dim3(WG), lds, st, a); }); break;
    case T_Q6_K: upl_dispatch<T_Q6_K>(g.UPL, [&](auto u) { hipLaunchKernelGGL((k_down<T_Q6_K, decltype(u)::value>), grid, dim3(WG), lds, st, a); }); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// ------------------------------------------------------------ reduce ----
// The weighted combine and the next RMSNorm's limbs, over H / RR_ROWS
// workgroups of RR_ROWS rows each:
//   w_s = softmax(logits)[e_s], renormalised over the k picks
//         (topk_softmax_f32.comp:29-67; every workgroup forms them)
//   x[r] += sum_s w_s partial[s][r]        (moe_reduce_f32.comp:8-13)
//   x[r] += sigmoid(ginp . xn) * y_sh[r]   (axpy_sig_f32.comp)
// then the limbs of x ⊙ norm_w for these rows and the partial sum of x^2
// over them: the next matvec applies the RMSNorm scale 1/sqrt(sum/H + eps).
constexpr int RR_WG = 256;
constexpr int RR_ROWS = 256;

__global__ void __launch_bounds__(RR_WG) k_reduce_rows(ReduceArgs a)
{
    __shared__ float red[16];
    __shared__ float s_w[MAX_TOPK];
    __shared__ float s_wsum, s_sg;
    const int tid = threadIdx.x, r = blockIdx.x * RR_ROWS + tid;  // RR_ROWS == RR_WG
    const bool hr = r < a.H;
    // every load that does not depend on the weights first
    float p[MAX_TOPK];
#pragma unroll
    for (int s = 0; s < MAX_TOPK; s++) p[s] = (s < a.k && hr) ? a.partial[(int64_t)s * a.H + r] : 0.0f;
    const float x0 = hr ? a.x[r] : 0.0f;
    const float y0 = (a.sh_y && hr) ? a.sh_y[r] : 0.0f;
    const float nw = (a.norm_w && hr) ? a.norm_w[r] : 1.0f;
    float lg_pick = 0.0f, mx = -INFINITY;
    if (a.logits) {
        for (int e = tid; e < a.E; e += RR_WG) mx = fmaxf(mx, a.logits[e]);
        if (tid < a.k) {
            const int e = a.ids[tid];
            lg_pick = (e >= 0 && e < a.E) ? a.logits[e] : -INFINITY;
        }
    }
    float shd = 0.0f;
    if (a.sh_y)
        for (int i = tid; i < a.H; i += RR_WG) shd += a.sh_ginp[i] * a.xn[i];
    if (a.logits) {
        mx = wave_max(mx);
        if ((tid & 63) == 0) red[tid >> 6] = mx;
        __syncthreads();
        mx = red[0];
        for (int i = 1; i < RR_WG / 64; i++) mx = fmaxf(mx, red[i]);
        float se = 0.0f;
        for (int e = tid; e < a.E; e += RR_WG) se += expf(a.logits[e] - mx);
        se = block_sum(se, red);
        if (tid < a.k) s_w[tid] = expf(lg_pick - mx) / se;
        __syncthreads();
        if (tid == 0 && a.renorm) {
            float wsum = 0.0f;
            for (int s = 0; s < a.k; s++) wsum += s_w[s];
            s_wsum = wsum;
        }
        __syncthreads();
        if (tid < a.k) {
            const float w = a.renorm ? s_w[tid] / s_wsum : s_w[tid];
            s_w[tid] = w;  // only this thread touches slot tid here
            if (a.wts_out && blockIdx.x == 0) a.wts_out[tid] = w;
        }
    } else if (tid < a.k) {
        s_w[tid] = a.wts[tid];
    }
    if (a.sh_y) {
        const float d = block_sum(shd, red);
        if (tid == 0) s_sg = 1.0f / (1.0f + expf(-d));
    }
    __syncthreads();
    float acc = 0.0f;
#pragma unroll
    for (int s = 0; s < MAX_TOPK; s++)
        if (s < a.k) acc += s_w[s] * p[s];
    float xv = x0 + acc;
    if (a.sh_y) xv = xv + s_sg * y0;
    if (hr) a.x[r] = xv;
    if (!a.norm_w) return;
    // limbs of x ⊙ norm_w: 8 consecutive rows per thread of the first 32
    float sq = block_sum(hr ? xv * xv : 0.0f, red);
    if (tid == 0) a.ss[blockIdx.x] = sq;
    __shared__ __align__(16) float xw[RR_ROWS];
    xw[tid] = xv * nw;
    __syncthreads();
    const int nrow = min(RR_ROWS, a.H - blockIdx.x * RR_ROWS);
    if (tid < RR_ROWS / 4) {  // four rows per thread: 64 threads at work
        const bool act = 4 * tid < nrow;
        float h[4];
#pragma unroll
        for (int i = 0; i < 4; i++) h[i] = act ? xw[4 * tid + i] : 0.0f;
        xq_group4(h, act, tid, xq_shift(a.xq, blockIdx.x * RR_ROWS));
    }
}

hipError_t launch_reduce_rows(hipStream_t st, const ReduceArgs &a)
{
    if (a.k < 1 || a.k > MAX_TOPK || a.H < 32 || a.H % 32 ||
        (a.logits && (a.E < a.k || a.E > MAX_EXPERTS || !a.ids)) || (!a.logits && !a.wts) ||
        (a.sh_y && (!a.sh_ginp || !a.xn)) || (a.norm_w && (!a.xq.A || !a.ss)))
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_reduce_rows, dim3((a.H + RR_ROWS - 1) / RR_ROWS), dim3(RR_WG), 0, st, a);
    return hipGetLastError();
}

}  // namespace styx
