// walk.h -- the row walker shared by the matvec kernels: lane groups of G
// lanes own rows, each lane owns UPL units of a row, two rows are in flight
// per lane group, and the first rows' weights are issued before the
// activation limbs are loaded or built.
#pragma once

#include "kernels.h"
#include "qdot.h"

namespace styx {

constexpr int WG = 256;
constexpr int WAVES = WG / 64;

// Slab of one routed slot from its hot / arena / host ids (first non-SKIP).
__device__ __forceinline__ const uint8_t *slab_pick(const ExpSrc &s, uint32_t h, uint32_t a,
                                                    uint32_t g)
{
    if (h != SKIP) return s.hot + (int64_t)h * s.hot_slab;
    if (a != SKIP) return s.arena + (int64_t)a * s.arena_slab;
    if (g != SKIP) return s.gtt + (int64_t)g * s.gtt_slab;
    return nullptr;
}

__device__ __forceinline__ const uint8_t *slab_for(const ExpSrc &s, const int32_t *ids, int slot)
{
    return slab_pick(s, (uint32_t)ids[16 + slot], (uint32_t)ids[32 + slot],
                     (uint32_t)ids[48 + slot]);
}

struct LaneMap {
    int lane, wave, gpw, grp, gl, gid, ngrp;
    bool ok;
};

__device__ __forceinline__ LaneMap lane_map(int G, int nwaves = WAVES)
{
    LaneMap m;
    m.lane = threadIdx.x & 63;
    m.wave = threadIdx.x >> 6;
    m.gpw = 64 / G;
    m.grp = m.lane / G;
    m.gl = m.lane - m.grp * G;
    m.ok = m.grp < m.gpw;
    m.gid = m.wave * m.gpw + m.grp;
    m.ngrp = nwaves * m.gpw;
    return m;
}

// Units of one lane: unit gl + u*G of every row it visits.
template <int UPL> struct LaneU {
    int ub[UPL], us[UPL];  // block, sub-unit
    bool uv[UPL];
    int un[UPL];           // unit index in the row
};

template <int T, int UPL>
__device__ __forceinline__ LaneU<UPL> lane_units(const LaneMap &lm, int nb, int G)
{
    constexpr int UPB = T == T_Q8_0 ? 1 : 4;
    LaneU<UPL> lu;
#pragma unroll
    for (int u = 0; u < UPL; u++) {
        lu.un[u] = lm.gl + u * G;
        lu.uv[u] = lm.ok && lu.un[u] < nb * UPB;
        lu.ub[u] = lu.un[u] / UPB;
        lu.us[u] = lu.un[u] % UPB;
    }
    return lu;
}

template <int T, int UPL>
__device__ __forceinline__ void issue_rows(UW<T> (&w0)[UPL], UW<T> (&w1)[UPL], const LaneU<UPL> &lu,
                                           const Mat &mat, int nb, int r, int r2, bool has1,
                                           bool has2)
{
#pragma unroll
    for (int u = 0; u < UPL; u++) {
        if (lu.uv[u]) {
            if (has1) uw_load<T>(w0[u], mat, (int64_t)r * nb + lu.ub[u], lu.us[u]);
            if (has2) uw_load<T>(w1[u], mat, (int64_t)r2 * nb + lu.ub[u], lu.us[u]);
        }
    }
}

// Row walker: the calling workgroup's lane groups cover rows
// [r_begin, r_end) two at a time; the result of row r goes to emit(r, v) on
// the group leader.  The first rows' weight loads are issued before
// xload(x, lu) fetches (or builds) the lane's activation limbs, so the
// activation trip overlaps the HBM latency; each next pair of rows is
// issued as soon as the previous one is consumed.
template <int T, int UPL, typename XLoad, typename Emit>
__device__ inline void walk_rows_pf(const Mat &mat, int nb, int G, int r_begin, int r_end,
                                    XLoad xload, Emit emit)
{
    const LaneMap lm = lane_map(G);
    const LaneU<UPL> lu = lane_units<T, UPL>(lm, nb, G);
    int r = r_begin + lm.gid;
    UW<T> w0[UPL], w1[UPL];
    issue_rows<T, UPL>(w0, w1, lu, mat, nb, r, r + lm.ngrp, r < r_end, r + lm.ngrp < r_end);
    UX<T> x[UPL];
    xload(x, lu);
    for (; r < r_end; r += 2 * lm.ngrp) {
        const int r2 = r + lm.ngrp;
        const bool has2 = r2 < r_end;
        float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
        for (int u = 0; u < UPL; u++) {
            if (lu.uv[u]) {
                a0 += udot(w0[u], x[u]);
                if (has2) a1 += udot(w1[u], x[u]);
            }
        }
        const int rn = r + 2 * lm.ngrp;
        issue_rows<T, UPL>(w0, w1, lu, mat, nb, rn, rn + lm.ngrp, rn < r_end,
                           rn + lm.ngrp < r_end);
        a0 = group_sum(a0, lm.gl, G);
        a1 = group_sum(a1, lm.gl, G);
        if (lm.ok && lm.gl == 0) {
            emit(r, a0);
            if (has2) emit(r2, a1);
        }
    }
}

// Limbs of the lane's units from an Xq vector (global memory or LDS).
template <int T, int UPL> struct XFrom {
    Xq q;
    __device__ __forceinline__ void operator()(UX<T> (&x)[UPL], const LaneU<UPL> &lu) const
    {
#pragma unroll
        for (int u = 0; u < UPL; u++)
            if (lu.uv[u]) ux_load<T>(x[u], q, lu.un[u]);
    }
};

template <int T, int UPL, typename Emit>
__device__ inline void walk_rows(const Xq &q, const Mat &mat, int nb, int G, int r_begin,
                                 int r_end, Emit emit)
{
    walk_rows_pf<T, UPL>(mat, nb, G, r_begin, r_end, XFrom<T, UPL>{q}, emit);
}

// Rows [r_begin, r_end) in batches of NR per lane group, the next batch's
// loads issued before the current batch is consumed (two register sets,
// alternated in a loop unrolled by two), so that a block of several batches
// streams its weights in one pass instead of one memory round trip per
// batch; xload(x, lu) fetches or builds the limbs once the first batch is
// issued.  Same per-row arithmetic as walk_rows_pf.
template <int T, int UPL, int NR, typename XLoad, typename Emit>
__device__ __forceinline__ void walk_rows_pipelined(const Mat &mat, int nb, int G, int r_begin,
                                                    int r_end, XLoad xload, Emit emit)
{
    const LaneMap lm = lane_map(G);
    const LaneU<UPL> lu = lane_units<T, UPL>(lm, nb, G);
    const int step = NR * lm.ngrp;
    auto issue = [&](UW<T>(&w)[NR][UPL], int r) {
#pragma unroll
        for (int i = 0; i < NR; i++) {
#pragma unroll
            for (int u = 0; u < UPL; u++)
                if (lu.uv[u] && r + i * lm.ngrp < r_end)
                    uw_load<T>(w[i][u], mat, (int64_t)(r + i * lm.ngrp) * nb + lu.ub[u], lu.us[u]);
        }
    };
    UX<T> x[UPL];
    auto consume = [&](const UW<T>(&w)[NR][UPL], int r) {
#pragma unroll
        for (int i = 0; i < NR; i++) {
            float acc = 0.0f;
            const bool ok = r + i * lm.ngrp < r_end;
#pragma unroll
            for (int u = 0; u < UPL; u++)
                if (lu.uv[u] && ok) acc += udot(w[i][u], x[u]);
            acc = group_sum(acc, lm.gl, G);
            if (lm.ok && lm.gl == 0 && ok) emit(r + i * lm.ngrp, acc);
        }
    };
    UW<T> wa[NR][UPL], wb[NR][UPL];
    int r = r_begin + lm.gid;
    if (r < r_end) issue(wa, r);
    xload(x, lu);
    while (r < r_end) {
        if (r + step < r_end) issue(wb, r + step);
        consume(wa, r);
        r += step;
        if (r >= r_end) break;
        if (r + step < r_end) issue(wa, r + step);
        consume(wb, r);
        r += step;
    }
}

}  // namespace styx
