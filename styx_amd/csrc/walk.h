// walk.h -- the row walker shared by the matvec kernels: lane groups of G
// lanes own rows, each lane owns UPL units of a row, two batches of rows are
// in flight per lane group, and the first two batches' weights are issued
// before the activation limbs are loaded or built.
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

// Lane groups of G lanes over the waves [wave0, wave0 + nwaves) of the
// workgroup (the calling wave must be one of them).  G is a power of two
// (pick_geo): shifts and masks, no integer division.
__device__ __forceinline__ LaneMap lane_map(int G, int nwaves = WAVES, int wave0 = 0)
{
    LaneMap m;
    const int lg = __builtin_ctz((unsigned)G);
    m.lane = threadIdx.x & 63;
    m.wave = (int)(threadIdx.x >> 6) - wave0;
    m.gpw = 64 >> lg;
    m.grp = m.lane >> lg;
    m.gl = m.lane & (G - 1);
    m.ok = true;
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

// Where a walked row lives: at(row, mm, b0) gives the matrix and the block
// index of the row's first unit.  OneMat: rows of one matrix.
struct OneMat {
    Mat m;
    int nb;
    __device__ __forceinline__ void operator()(int row, Mat &mm, int64_t &b0) const
    {
        mm = m;
        b0 = (int64_t)row * nb;
    }
};

// Rows of up to three matrices stacked: rows [0, b1) of m0, [b1, b2) of
// m1, the rest of m2.  The regions of m1 and m2 are kept as byte offsets
// from the previous matrix's: a select among the matrices compiles to a
// table in scratch memory, this to adds.
struct Mat3 {
    uint64_t base[4], d1[4], d2[4];
    int b1, b2, nb;
    __device__ __forceinline__ Mat3(const Mat &m0, const Mat &m1, const Mat &m2, int b1_, int b2_,
                                    int nb_)
        : b1(b1_), b2(b2_), nb(nb_)
    {
        const Mat *m[3] = {&m0, &m1, &m2};
        uint64_t r[3][4];
#pragma unroll
        for (int i = 0; i < 3; i++) {
            r[i][0] = (uint64_t)(uintptr_t)m[i]->r0;
            r[i][1] = (uint64_t)(uintptr_t)m[i]->r1;
            r[i][2] = (uint64_t)(uintptr_t)m[i]->r2;
            r[i][3] = (uint64_t)(uintptr_t)m[i]->r3;
        }
#pragma unroll
        for (int j = 0; j < 4; j++) {
            base[j] = r[0][j];
            d1[j] = r[1][j] - r[0][j];
            d2[j] = r[2][j] - r[1][j];
        }
    }
    __device__ __forceinline__ void operator()(int row, Mat &mm, int64_t &b0) const
    {
        const uint64_t p1 = row >= b1, p2 = row >= b2;
        uint64_t r[4];
#pragma unroll
        for (int j = 0; j < 4; j++) r[j] = base[j] + p1 * d1[j] + p2 * d2[j];
        mm.r0 = (const uint8_t STYX_GLOBAL *)(uintptr_t)r[0];
        mm.r1 = (const uint8_t STYX_GLOBAL *)(uintptr_t)r[1];
        mm.r2 = (const uint8_t STYX_GLOBAL *)(uintptr_t)r[2];
        mm.r3 = (const uint8_t STYX_GLOBAL *)(uintptr_t)r[3];
        b0 = (int64_t)(row - (int)p1 * b1 - (int)p2 * (b2 - b1)) * nb;
    }
};

// Rows [r_begin, r_end) in batches of NR per lane group, with two batches
// in flight: the first two are issued before xload(x, lu) fetches or builds
// the limbs (and may wait for them: it returns false to abandon the walk,
// and the walker then returns false), and each later batch is issued as
// soon as the one two before it is consumed (two register sets, alternated
// in a loop unrolled by two).  A block of several batches thus streams its
// weights in one pass instead of one memory round trip per batch.  A row's
// result is the group sum of its lanes' unit dots.
//
// Every batch issues the same loads on every path: the batch count is the
// workgroup's (that of the lane group with the most rows), and a row past
// the block's end, or a lane without a unit, loads the first unit of the
// block's last row instead and discards it.  The compiler then knows at each consume that
// exactly the other batch's loads may still be in flight and waits for
// this batch's alone; with conditional issues it has to wait for all of
// them, and the walk degrades to one round trip per batch.
// The rows are spread over the lane groups of waves [wave0, wave0 + nwaves)
// (all four by default); only those waves call the walker.
template <int T, int UPL, int NR, typename RowAt, typename XLoad, typename Emit>
__device__ __forceinline__ bool walk_rows_pipelined(RowAt at, int nb, int G, int r_begin,
                                                    int r_end, XLoad xload, Emit emit,
                                                    int nwaves = WAVES, int wave0 = 0)
{
    const LaneMap lm = lane_map(G, nwaves, wave0);
    const LaneU<UPL> lu = lane_units<T, UPL>(lm, nb, G);
    const int step = NR * lm.ngrp;
    const int nbat = (r_end - r_begin + step - 1) / step;
    const int r0 = r_begin + lm.gid;
    auto issue = [&](UW<T>(&w)[NR][UPL], int b) {
#pragma unroll
        for (int i = 0; i < NR; i++) {
            const int row = r0 + b * step + i * lm.ngrp;
            Mat mm;
            int64_t b0;
            at(min(row, r_end - 1), mm, b0);
#pragma unroll
            for (int u = 0; u < UPL; u++) {
                const bool ok = lu.uv[u] && row < r_end;
                uw_load<T>(w[i][u], mm, ok ? b0 + lu.ub[u] : b0, ok ? lu.us[u] : 0);
            }
        }
    };
    UX<T> x[UPL];
    auto consume = [&](const UW<T>(&w)[NR][UPL], int b) {
#pragma unroll
        for (int i = 0; i < NR; i++) {
            const int row = r0 + b * step + i * lm.ngrp;
            const bool ok = row < r_end;
            float acc = 0.0f;
#pragma unroll
            for (int u = 0; u < UPL; u++)
                if (lu.uv[u] && ok) acc += udot(w[i][u], x[u]);
            acc = group_sum(acc, lm.gl, G);
            if (lm.ok && lm.gl == 0 && ok) emit(row, acc);
        }
    };
    UW<T> wa[NR][UPL], wb[NR][UPL];
    if (nbat <= 1) {
        if (nbat == 1) issue(wa, 0);
        if (!xload(x, lu)) return false;
        if (nbat == 1) consume(wa, 0);
        return true;
    }
    issue(wa, 0);
    issue(wb, 1);
    if (!xload(x, lu)) return false;
    int b = 0;
    for (; b + 3 < nbat; b += 2) {
        consume(wa, b);
        issue(wa, b + 2);
        consume(wb, b + 1);
        issue(wb, b + 3);
    }
    if (b + 2 < nbat) {
        consume(wa, b);
        issue(wa, b + 2);
        consume(wb, b + 1);
        consume(wa, b + 2);
    } else {
        consume(wa, b);
        consume(wb, b + 1);
    }
    return true;
}

}  // namespace styx
