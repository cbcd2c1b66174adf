// kernels_mv.hip -- dequant-matvec kernels of the MoE decode hot path (gfx950).
//
//   k_mv_dense      q/k/v, o-proj (+residual), LM head: rows of one or up to
//                   three split-layout matrices against one activation vector,
//                   optional fused RMSNorm prologue (rms_norm_f32 semantics,
//                   crates/model/src/moe.rs:1746-1766) and residual add.
//   k_router_topk   f32 router matvec (shaders/matvec_strided_f32.comp) with the
//                   ffn RMSNorm fused in front and topk_softmax_f32 fused behind
//                   (last-workgroup-done).
//   k_gate_up       expert gate and up matvecs for the k routed slots
//                   (mul_mat_vec_id semantics, ne11 = 1).
//   k_down          expert down matvec with swiglu fused in its prologue and
//                   moe_reduce fused behind (last-workgroup-done per row tile):
//                   x[r] += sum_s w_s * y_s[r], s ascending.
//
// Every matvec workgroup (256 threads, 4 wave64) first issues nothing but
// builds the activation limbs in LDS, then each lane group walks rows with
// 16-byte loads of the split layout (see qdot.h).
#include "kernels.h"
#include "qdot.h"
#include "topk.h"

#include <algorithm>

namespace styx {

constexpr int WG = 256;
constexpr int WAVES = WG / 64;

Geo pick_geo(int t, int ncols)
{
    Geo g{0, 0, 0};
    if (!is_quant(t) || ncols % blk_elems(t) != 0) return g;
    const int units = ncols / blk_elems(t) * units_per_blk(t);
    const int max_upl = t == T_Q8_0 ? 4 : 2;
    int best_waste = 1 << 30;
    for (int upl = 1; upl <= max_upl; upl++) {
        if (units % upl) continue;
        const int G = units / upl;
        if (G > 64) continue;
        const int waste = 64 - (64 / G) * G;
        if (waste < best_waste) {
            best_waste = waste;
            g.G = G;
            g.UPL = upl;
        }
    }
    g.units = units;
    return g;
}

__device__ __forceinline__ const uint8_t *slab_for(const ExpSrc &s, const int32_t *ids, int slot)
{
    const uint32_t h = (uint32_t)ids[16 + slot];
    if (h != SKIP) return s.hot + (int64_t)h * s.hot_slab;
    const uint32_t a = (uint32_t)ids[32 + slot];
    if (a != SKIP) return s.arena + (int64_t)a * s.arena_slab;
    const uint32_t g = (uint32_t)ids[48 + slot];
    if (g != SKIP) return s.gtt + (int64_t)g * s.gtt_slab;
    return nullptr;
}

// ---------------------------------------------------------------------------
// Row walker: the calling workgroup's lane groups cover rows
// [r_begin, r_end) of a matrix; result of row r goes to emit(r, value) on the
// group leader.  Rows are taken two at a time so each lane has two rows of
// loads in flight.
// ---------------------------------------------------------------------------
struct LaneMap {
    int lane, wave, gpw, grp, gl, gid, ngrp;
    bool ok;
};

__device__ __forceinline__ LaneMap lane_map(int G)
{
    LaneMap m;
    m.lane = threadIdx.x & 63;
    m.wave = threadIdx.x >> 6;
    m.gpw = 64 / G;
    m.grp = m.lane / G;
    m.gl = m.lane - m.grp * G;
    m.ok = m.grp < m.gpw;
    m.gid = m.wave * m.gpw + m.grp;
    m.ngrp = WAVES * m.gpw;
    return m;
}

template <int T, int UPL, typename Emit>
__device__ inline void walk_rows(const XqLds &q, const Mat &mat, int nb, int G, int r_begin,
                                 int r_end, Emit emit)
{
    constexpr int UPB = T == T_Q8_0 ? 1 : 4;
    const LaneMap lm = lane_map(G);
    const int units = nb * UPB;
    UX<T> x[UPL];
    int ub[UPL], us[UPL];
    bool uv[UPL];
#pragma unroll
    for (int u = 0; u < UPL; u++) {
        const int un = lm.gl + u * G;
        uv[u] = lm.ok && un < units;
        ub[u] = un / UPB;
        us[u] = un % UPB;
        if (uv[u]) ux_load<T>(x[u], q, un);
    }
    for (int r = r_begin + lm.gid; r < r_end; r += 2 * lm.ngrp) {
        const int r2 = r + lm.ngrp;
        const bool has2 = r2 < r_end;
        UW<T> w0[UPL], w1[UPL];
#pragma unroll
        for (int u = 0; u < UPL; u++) {
            if (uv[u]) {
                uw_load<T>(w0[u], mat, (int64_t)r * nb + ub[u], us[u]);
                if (has2) uw_load<T>(w1[u], mat, (int64_t)r2 * nb + ub[u], us[u]);
            }
        }
        float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
        for (int u = 0; u < UPL; u++) {
            if (uv[u]) {
                a0 += udot(w0[u], x[u]);
                if (has2) a1 += udot(w1[u], x[u]);
            }
        }
        a0 = group_sum(a0, lm.gl, G);
        a1 = group_sum(a1, lm.gl, G);
        if (lm.ok && lm.gl == 0) {
            emit(r, a0);
            if (has2) emit(r2, a1);
        }
    }
}

template <int T, typename Emit>
__device__ inline void walk_rows_upl(int upl, const XqLds &q, const Mat &mat, int nb, int G,
                                     int r_begin, int r_end, Emit emit)
{
    if constexpr (T == T_Q8_0) {
        switch (upl) {
        case 1: walk_rows<T, 1>(q, mat, nb, G, r_begin, r_end, emit); break;
        case 2: walk_rows<T, 2>(q, mat, nb, G, r_begin, r_end, emit); break;
        case 3: walk_rows<T, 3>(q, mat, nb, G, r_begin, r_end, emit); break;
        default: walk_rows<T, 4>(q, mat, nb, G, r_begin, r_end, emit); break;
        }
    } else {
        if (upl == 1)
            walk_rows<T, 1>(q, mat, nb, G, r_begin, r_end, emit);
        else
            walk_rows<T, 2>(q, mat, nb, G, r_begin, r_end, emit);
    }
}

__host__ __device__ inline size_t red_off(int n) { return (xq_lds_bytes(n) + 15) & ~(size_t)15; }

// ------------------------------------------------------------------ dense --
struct DenseK {
    const uint8_t *w[3];
    float *y[3];
    int rows[3];
    int nseg, total, ncols, nb, G, UPL, rpw, add;
    const float *x, *nw;
    float eps;
};

template <int T>
__global__ void __launch_bounds__(WG) k_mv_dense(DenseK a)
{
    extern __shared__ __align__(16) uint8_t lds[];
    const XqLds q = xq_carve(lds, a.ncols);
    float *red = (float *)(lds + red_off(a.ncols));
    xq_build(a.x, a.nw, a.eps, a.nw != nullptr, a.ncols, q, red, nullptr);
    __syncthreads();
    const int r_begin = blockIdx.x * a.rpw, r_end = min(a.total, r_begin + a.rpw);
    // segments are walked one after another; each starts a fresh row walk
    int base = 0;
    for (int s = 0; s < a.nseg; s++) {
        const int lo = max(r_begin, base), hi = min(r_end, base + a.rows[s]);
        if (lo < hi) {
            const Mat mat = mat_at(a.w[s], T, (int64_t)a.rows[s] * a.nb);
            float *y = a.y[s];
            const int add = a.add;
            walk_rows_upl<T>(a.UPL, q, mat, a.nb, a.G, lo - base, hi - base,
                             [=](int r, float v) { y[r] = add ? y[r] + v : v; });
        }
        base += a.rows[s];
    }
}

hipError_t launch_dense(hipStream_t st, int t, int ncols, const DenseSeg *segs, int nseg,
                        const float *x, const float *norm_w, float eps, int add)
{
    const Geo g = pick_geo(t, ncols);
    if (g.G == 0 || nseg < 1 || nseg > 3) return hipErrorInvalidValue;
    DenseK a{};
    a.total = 0;
    for (int i = 0; i < nseg; i++) {
        a.w[i] = segs[i].w;
        a.y[i] = segs[i].y;
        a.rows[i] = segs[i].rows;
        a.total += segs[i].rows;
    }
    a.nseg = nseg;
    a.ncols = ncols;
    a.nb = ncols / blk_elems(t);
    a.G = g.G;
    a.UPL = g.UPL;
    a.add = add;
    a.x = x;
    a.nw = norm_w;
    a.eps = eps;
    const int ngrp = WAVES * (64 / g.G);
    // aim for ~1024 workgroups (4 per CU), at least 2 rows per group
    int rpw = (a.total + 1023) / 1024;
    rpw = std::max(rpw, 2 * ngrp);
    rpw = (rpw + ngrp - 1) / ngrp * ngrp;
    a.rpw = rpw;
    const int nwg = (a.total + rpw - 1) / rpw;
    const size_t lds = red_off(ncols) + 64;
    switch (t) {
    case T_Q8_0: hipLaunchKernelGGL(k_mv_dense<T_Q8_0>, dim3(nwg), dim3(WG), lds, st, a); break;
    case T_Q4_K: hipLaunchKernelGGL(k_mv_dense<T_Q4_K>, dim3(nwg), dim3(WG), lds, st, a); break;
    case T_Q5_K: hipLaunchKernelGGL(k_mv_dense<T_Q5_K>, dim3(nwg), dim3(WG), lds, st, a); break;
    case T_Q6_K: hipLaunchKernelGGL(k_mv_dense<T_Q6_K>, dim3(nwg), dim3(WG), lds, st, a); break;
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
// (shaders/matvec_strided_f32.comp); one row per wave.  The top-k is run by
// each consumer workgroup from these logits (see route_in_lds), so no
// workgroup ever waits on another inside a kernel.
constexpr int ROUTER_ROWS = 4;

__global__ void __launch_bounds__(WG) k_router(RouterArgs a)
{
    extern __shared__ __align__(16) uint8_t lds[];
    float *xs = (float *)lds;          // normalised x, H floats
    float *red = xs + a.H;             // 16 floats
    float ss = 0.0f;
    for (int i = threadIdx.x * 4; i < a.H; i += WG * 4) {
        const float4 v = *(const float4 *)(a.x + i);
        ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
    }
    ss = block_sum(ss, red);
    const float scale = 1.0f / sqrtf(ss / (float)a.H + a.eps);
    for (int i = threadIdx.x * 4; i < a.H; i += WG * 4) {
        const float4 v = *(const float4 *)(a.x + i);
        const float4 w = *(const float4 *)(a.norm_w + i);
        const float4 o = make_float4((v.x * scale) * w.x, (v.y * scale) * w.y,
                                     (v.z * scale) * w.z, (v.w * scale) * w.w);
        *(float4 *)(xs + i) = o;
        if (blockIdx.x == 0) *(float4 *)(a.xn + i) = o;
    }
    __syncthreads();
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r = blockIdx.x * ROUTER_ROWS + wave;
    if (r < a.E) {
        const float *w = a.W + (int64_t)r * a.H;
        float acc = 0.0f;
        for (int c = lane * 4; c < a.H; c += 256) {
            const float4 wv = *(const float4 *)(w + c);
            const float4 xv = *(const float4 *)(xs + c);
            acc += wv.x * xv.x + wv.y * xv.y + wv.z * xv.z + wv.w * xv.w;
        }
        acc = wave_sum(acc);
        if (lane == 0) a.logits[r] = a.bias ? acc + a.bias[r] : acc;
    }
}

hipError_t launch_router(hipStream_t st, const RouterArgs &a)
{
    if (a.E < 1 || a.E > MAX_EXPERTS || a.H % 4) return hipErrorInvalidValue;
    const int nwg = (a.E + ROUTER_ROWS - 1) / ROUTER_ROWS;
    hipLaunchKernelGGL(k_router, dim3(nwg), dim3(WG), (size_t)a.H * 4 + 64, st, a);
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
struct GateUpK {
    ExpSrc src[2];
    int type[2], G[2], UPL[2];
    const int32_t *ids;   // id row in memory, used when route.logits is null
    Route route;
    const float *xn;
    float *gu;  // [2][k][F]
    int H, F, k, nb, rpw;
};

template <int T>
__device__ inline void gate_up_body(const GateUpK &a, const XqLds &q, int m, int s,
                                    const uint8_t *slab)
{
    const Mat mat = mat_at(slab, T, (int64_t)a.F * a.nb);
    const int r_begin = blockIdx.x * a.rpw, r_end = min(a.F, r_begin + a.rpw);
    float *y = a.gu + ((int64_t)m * a.k + s) * a.F;
    walk_rows_upl<T>(a.UPL[m], q, mat, a.nb, a.G[m], r_begin, r_end,
                     [=](int r, float v) { y[r] = v; });
}

template <int TG, int TU>
__global__ void __launch_bounds__(WG) k_gate_up(GateUpK a)
{
    extern __shared__ __align__(16) uint8_t lds[];
    __shared__ int32_t s_ids[IDS_ROW];
    __shared__ float s_w[MAX_TOPK];
    const int s = blockIdx.y, m = blockIdx.z;
    const int32_t *ids = a.route.logits ? route_in_lds(a.route, s_ids, s_w) : a.ids;
    const uint8_t *slab = slab_for(a.src[m], ids, s);
    if (!slab) return;
    const XqLds q = xq_carve(lds, a.H);
    float *red = (float *)(lds + red_off(a.H));
    xq_build(a.xn, nullptr, 0.0f, false, a.H, q, red, nullptr);
    __syncthreads();
    if (m == 0)
        gate_up_body<TG>(a, q, 0, s, slab);
    else
        gate_up_body<TU>(a, q, 1, s, slab);
}

template <int TG>
static hipError_t launch_gu_tu(hipStream_t st, int tu, const GateUpK &a, dim3 grid, size_t lds)
{
    switch (tu) {
    case T_Q8_0: hipLaunchKernelGGL((k_gate_up<TG, T_Q8_0>), grid, dim3(WG), lds, st, a); break;
    case T_Q4_K: hipLaunchKernelGGL((k_gate_up<TG, T_Q4_K>), grid, dim3(WG), lds, st, a); break;
    case T_Q5_K: hipLaunchKernelGGL((k_gate_up<TG, T_Q5_K>), grid, dim3(WG), lds, st, a); break;
    case T_Q6_K: hipLaunchKernelGGL((k_gate_up<TG, T_Q6_K>), grid, dim3(WG), lds, st, a); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_moe_gate_up(hipStream_t st, int tg, int tu, const ExpSrc &g, const ExpSrc &u,
                              const int32_t *ids, const Route *route, const float *xn, float *gu,
                              int H, int F, int k)
{
    const Geo gg = pick_geo(tg, H), gv = pick_geo(tu, H);
    if (!gg.G || !gv.G || blk_elems(tg) != blk_elems(tu) || k < 1 || k > MAX_TOPK)
        return hipErrorInvalidValue;
    if (route && (route->E < k || route->E > MAX_EXPERTS || route->k != k))
        return hipErrorInvalidValue;
    if (!route && !ids) return hipErrorInvalidValue;
    GateUpK a{};
    a.src[0] = g;
    a.src[1] = u;
    a.type[0] = tg;
    a.type[1] = tu;
    a.G[0] = gg.G;
    a.G[1] = gv.G;
    a.UPL[0] = gg.UPL;
    a.UPL[1] = gv.UPL;
    a.ids = ids;
    if (route) a.route = *route;
    a.xn = xn;
    a.gu = gu;
    a.H = H;
    a.F = F;
    a.k = k;
    a.nb = H / blk_elems(tg);
    // rows per workgroup: ~1024 workgroups in total over 2*k slot-matrices
    const int ngrp = WAVES * (64 / std::max(gg.G, gv.G));
    int rpw = (2 * k * F + 1023) / 1024;
    rpw = std::max(rpw, 2 * ngrp);
    rpw = (rpw + ngrp - 1) / ngrp * ngrp;
    a.rpw = rpw;
    const dim3 grid((F + rpw - 1) / rpw, k, 2);
    const size_t lds = red_off(H) + 64;
    switch (tg) {
    case T_Q8_0: return launch_gu_tu<T_Q8_0>(st, tu, a, grid, lds);
    case T_Q4_K: return launch_gu_tu<T_Q4_K>(st, tu, a, grid, lds);
    case T_Q5_K: return launch_gu_tu<T_Q5_K>(st, tu, a, grid, lds);
    case T_Q6_K: return launch_gu_tu<T_Q6_K>(st, tu, a, grid, lds);
    default: return hipErrorInvalidValue;
    }
}

// ------------------------------------------------------------- down -------
// y_s = Wd[e_s] . swiglu(g_s, u_s) for every routed slot s into partial[s];
// the weighted combine into the residual is k_moe_reduce.
struct DownK {
    ExpSrc src;
    int G, UPL;
    const int32_t *ids;
    const float *gu;
    float *partial;
    int H, F, k, nb, rpw;
};

template <int T>
__global__ void __launch_bounds__(WG) k_down(DownK a)
{
    extern __shared__ __align__(16) uint8_t lds[];
    const int s = blockIdx.y;
    const int r_begin = blockIdx.x * a.rpw, r_end = min(a.H, r_begin + a.rpw);
    const uint8_t *slab = slab_for(a.src, a.ids, s);
    float *part = a.partial + (int64_t)s * a.H;
    if (!slab) {
        for (int r = r_begin + threadIdx.x; r < r_end; r += WG) part[r] = 0.0f;
        return;
    }
    // swiglu_f32 (ops2.rs:305-309) of this slot's gate/up rows into LDS
    float *hs = (float *)lds;
    const float *g = a.gu + (int64_t)s * a.F, *u = a.gu + ((int64_t)a.k + s) * a.F;
    for (int i = threadIdx.x; i < a.F; i += WG) hs[i] = g[i] / (1.0f + expf(-g[i])) * u[i];
    __syncthreads();
    uint8_t *qbase = lds + (((size_t)a.F * 4 + 15) & ~(size_t)15);
    const XqLds q = xq_carve(qbase, a.F);
    float *red = (float *)(qbase + red_off(a.F));
    xq_build(hs, nullptr, 0.0f, false, a.F, q, red, nullptr);
    __syncthreads();
    const Mat mat = mat_at(slab, T, (int64_t)a.H * a.nb);
    walk_rows_upl<T>(a.UPL, q, mat, a.nb, a.G, r_begin, r_end,
                     [=](int r, float v) { part[r] = v; });
}

// moe_reduce_f32 (shaders/moe_reduce_f32.comp:8-13): x[i] += sum_s w[s]*d[s][i],
// accumulated from 0 in ascending s.
__global__ void __launch_bounds__(WG) k_moe_reduce(const float *d, const float *w, float *x,
                                                   int ne, int k)
{
    const int i = blockIdx.x * WG + threadIdx.x;
    if (i >= ne) return;
    float acc = 0.0f;
    for (int s = 0; s < k; s++) acc += w[s] * d[(int64_t)s * ne + i];
    x[i] += acc;
}

hipError_t launch_moe_down(hipStream_t st, int td, const ExpSrc &d, const int32_t *ids,
                           const float *wts, const float *gu, float *x, float *partial, int H,
                           int F, int k)
{
    const Geo g = pick_geo(td, F);
    if (!g.G || k < 1 || k > MAX_TOPK) return hipErrorInvalidValue;
    DownK a{};
    a.src = d;
    a.G = g.G;
    a.UPL = g.UPL;
    a.ids = ids;
    a.gu = gu;
    a.partial = partial;
    a.H = H;
    a.F = F;
    a.k = k;
    a.nb = F / blk_elems(td);
    const int ngrp = WAVES * (64 / g.G);
    int rpw = (k * H + 1023) / 1024;
    rpw = std::max(rpw, 2 * ngrp);
    rpw = (rpw + ngrp - 1) / ngrp * ngrp;
    a.rpw = rpw;
    const dim3 grid((H + rpw - 1) / rpw, k, 1);
    const size_t lds = (((size_t)F * 4 + 15) & ~(size_t)15) + red_off(F) + 64;
    switch (td) {
    case T_Q8_0: hipLaunchKernelGGL(k_down<T_Q8_0>, grid, dim3(WG), lds, st, a); break;
    case T_Q4_K: hipLaunchKernelGGL(k_down<T_Q4_K>, grid, dim3(WG), lds, st, a); break;
    case T_Q5_K: hipLaunchKernelGGL(k_down<T_Q5_K>, grid, dim3(WG), lds, st, a); break;
    case T_Q6_K: hipLaunchKernelGGL(k_down<T_Q6_K>, grid, dim3(WG), lds, st, a); break;
    default: return hipErrorInvalidValue;
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_moe_reduce, dim3((H + WG - 1) / WG), dim3(WG), 0, st, partial, wts, x, H,
                       k);
    return hipGetLastError();
}

// ------------------------------------------------ shared-expert gating ----
__global__ void __launch_bounds__(WG) k_axpy_sig_dot(const float *ginp, const float *xn,
                                                     const float *y, float *x, int n)
{
    __shared__ float red[16];
    float acc = 0.0f;
    for (int i = threadIdx.x; i < n; i += WG) acc += ginp[i] * xn[i];
    acc = block_sum(acc, red);
    const float sg = 1.0f / (1.0f + expf(-acc));
    for (int i = blockIdx.x * WG + threadIdx.x; i < n; i += gridDim.x * WG) x[i] += sg * y[i];
}

hipError_t launch_axpy_sig_dot(hipStream_t st, const float *ginp, const float *xn,
                               const float *y, float *x, int n)
{
    hipLaunchKernelGGL(k_axpy_sig_dot, dim3(std::max(1, std::min(32, n / WG))), dim3(WG), 0, st,
                       ginp, xn, y, x, n);
    return hipGetLastError();
}

}  // namespace styx
