// attn.hip -- split-context decode attention over the paged f32 KV cache.
//
// Semantics follow shaders/attn_decode_f32.comp:31-79 (softmax(scale*q.K)V
// per query head, GQA kvh = h / gqa, K/V rows [t][kv_dim]) with the per-head
// q/k RMSNorm (crates/model/src/moe.rs:1875-1913), NEOX rope
// (crates/vk-backend/tests/ops2.rs:426-442, angle in f64) and the KV append
// at the current position (moe.rs:1932-1943) fused in front.  The rope
// factors come from a table of (cos, sin) pairs in f64 per position, built
// on the host with the same formula (styx_rope_table), so the device does
// the rotation in f64 without evaluating a single trigonometric function.
//
// Layout: one workgroup per (context chunk, kv head) serves all gqa query
// heads of that kv head, so each K/V row comes from HBM once (the reference
// re-reads it per query head).  Its four waves split the query heads (and,
// for gqa < 4, the chunk's 16-token tiles); each wave runs its own online
// softmax over its tiles with no workgroup barrier until the end, where the
// waves sharing heads merge their (m, l, o) in LDS and one partial per
// (chunk, head) is written.  k_attn_combine merges the chunk partials of
// each query head, writes the output and the activation limbs of the o-proj
// input.  The current position is read from device memory, so a captured
// graph serves every step; chunks past the context exit at once.
#include "kernels.h"
#include "qdot.h"
#include "xchg.h"

#include <algorithm>
#include <type_traits>

namespace styx {

constexpr int AT_WG = 256;
constexpr int AT_WAVES = AT_WG / 64;
constexpr int TILE = 16;

// Tokens per chunk for a context of n_t tokens: at least a.chunk (a
// multiple of 16), and enough that n_t fits in a.max_chunks chunks.  Both
// kernels evaluate it from the device-side position, so the split follows
// the live context length inside one captured graph.
__device__ __forceinline__ int attn_chunk(const AttnArgs &a, int n_t)
{
    if (n_t <= a.solo_max) return max(a.chunk, (n_t + 15) / 16 * 16);  // one chunk
    const int need = (n_t + a.max_chunks - 1) / a.max_chunks;
    return max(a.chunk, (need + 15) / 16 * 16);
}

// Offset of the K/V row of kv head kvh at token tp of physical page pg.
// A page holds page_tokens tokens of every kv head, either token-major
// ([token][kv_dim], the reference's row layout) or head-major
// ([kv head][token][hd]: the rows a workgroup reads are contiguous).
__device__ __forceinline__ int64_t kv_row(const AttnArgs &a, int64_t pg, int tp, int kvh, int kv_dim)
{
    return a.kv_head_major ? ((pg * a.nkv + kvh) * a.page_tokens + tp) * (int64_t)a.hd
                           : (pg * a.page_tokens + tp) * (int64_t)kv_dim + (int64_t)kvh * a.hd;
}
__device__ __forceinline__ int64_t kv_off(const AttnArgs &a, int t, int kvh, int kv_dim)
{
    const int pt = a.page_tokens;
    if ((pt & (pt - 1)) == 0) {  // a power of two (the engine's pages): no division
        const int sh = __builtin_ctz((unsigned)pt);
        return kv_row(a, a.page_table[t >> sh], t & (pt - 1), kvh, kv_dim);
    }
    return kv_row(a, a.page_table[t / pt], t % pt, kvh, kv_dim);
}

// One head's RMSNorm(hd) * w and NEOX rope at pos, split into a load phase
// (every operand of the head issued at once) and a compute phase, so a wave
// can have all its heads' loads in flight together.  Lane l owns the rope
// pairs (i, i + hd/2) for i = l + 64 j, j < PPL; cs points at the (cos, sin)
// row of the position.
template <int PPL> struct HeadIn {
    float x0[PPL], x1[PPL], w0[PPL], w1[PPL];
};

template <int PPL>
__device__ __forceinline__ void head_load(HeadIn<PPL> &h, const float *src, const float *w, int hd)
{
    const int lane = threadIdx.x & 63, half = hd / 2;
#pragma unroll
    for (int j = 0; j < PPL; j++) {
        const int i = lane + 64 * j;
        const bool ok = i < half;
        h.x0[j] = ok ? src[i] : 0.0f;
        h.x1[j] = ok ? src[i + half] : 0.0f;
        h.w0[j] = (ok && w) ? w[i] : 1.0f;
        h.w1[j] = (ok && w) ? w[i + half] : 1.0f;
    }
}

// head_load for head_dim 128 with one pair per lane: every load issued
// unconditionally (without norm weights, the weights' loads read the head
// itself and are replaced by 1)
template <int PPL>
__device__ __forceinline__ void head_load_all(HeadIn<PPL> &h, const float *src, const float *w, int hd)
{
    static_assert(PPL == 1, "one rope pair per lane");
    const int lane = threadIdx.x & 63, half = hd / 2;
    const float *ws = w ? w : src;
    h.x0[0] = src[lane];
    h.x1[0] = src[lane + half];
    const float w0 = ws[lane], w1 = ws[lane + half];
    h.w0[0] = w ? w0 : 1.0f;
    h.w1[0] = w ? w1 : 1.0f;
}

template <int PPL>
__device__ __forceinline__ void cs_load(double2 *cs, const double2 *row, int hd)
{
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int j = 0; j < PPL; j++) {
        const int i = lane + 64 * j;
        cs[j] = i < hd / 2 ? row[i] : make_double2(1.0, 0.0);
    }
}

template <int PPL>
__device__ __forceinline__ void head_finish(const HeadIn<PPL> &h, const double2 *cs, bool norm,
                                            float eps, int hd, float *dst)
{
    const int lane = threadIdx.x & 63, half = hd / 2;
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < PPL; j++) ss += h.x0[j] * h.x0[j] + h.x1[j] * h.x1[j];
    ss = wave_sum(ss);
    const float scale = norm ? 1.0f / sqrtf(ss / (float)hd + eps) : 1.0f;
#pragma unroll
    for (int j = 0; j < PPL; j++) {
        const int i = lane + 64 * j;
        if (i >= half) continue;
        float x0 = h.x0[j], x1 = h.x1[j];
        if (norm) {
            x0 = (x0 * scale) * h.w0[j];
            x1 = (x1 * scale) * h.w1[j];
        }
        const double c = cs[j].x, sn = cs[j].y;
        dst[i] = (float)((double)x0 * c - (double)x1 * sn);
        dst[i + half] = (float)((double)x0 * sn + (double)x1 * c);
    }
}

// Reductions over the 16 lanes of a row (DPP butterflies, every lane of the
// row gets the result), and the sum over the four rows of a wave at the
// same row position (the two row swaps: v + (v of lane ^ 16), then + (the
// same of lane ^ 32), in the same order on both lanes of each pair).
__device__ __forceinline__ float max16(float v)
{
    return bfly<16>(v, [](float a, float b) { return fmaxf(a, b); });
}
__device__ __forceinline__ float sum16(float v) { return bfly_sum<16>(v); }
__device__ __forceinline__ float sum_rows(float v)
{
    const auto s = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(s[0]) + __uint_as_float(s[1]);
    const auto t = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(t[0]) + __uint_as_float(t[1]);
}

// Phase stamps of a workgroup (AttnArgs::trace): kept by thread 0 in LDS,
// written out when the workgroup ends.
struct AtStamps {
    uint64_t *s;  // LDS slots, or null when not tracing
    __device__ __forceinline__ void clear() const
    {
        if (s && threadIdx.x == 0)
            for (int i = 0; i < AT_TRACE; i++) s[i] = 0;
    }
    __device__ __forceinline__ void at(int i) const
    {
        if (s && threadIdx.x == 0) s[i] = wall_clock64();
    }
    __device__ __forceinline__ void flush(const AttnArgs &a, int c, int kvh, int n_active) const
    {
        if (!s || threadIdx.x != 0) return;
        s[6] = (uint64_t)n_active;
        s[7] = ((uint64_t)kvh << 16 | (uint64_t)c) + 1;
        uint64_t *d = a.trace + ((int64_t)kvh * gridDim.x + c) * AT_TRACE;
        for (int i = 0; i < AT_TRACE; i++) gst<uint64_t>(d + i, s[i]);
    }
};

// ------------------------------------------------------ in-kernel combine --
// With a.t_part the chunk workgroups publish their partials (m, l, o) as
// tagged words, and query head g of kv head kvh is merged by the workgroup
// of chunk g mod n_active: its four waves each take every fourth chunk in
// batches of 8 (all loads of a batch issued together, re-polled until every
// word carries the launch's tag), merge them online, then the waves merge in
// LDS and the head's output and its limbs are written.  Only workgroups of
// chunks below gqa ever wait, and they wait on chunks that never wait, so
// the launch drains even when not all its workgroups are resident.  A wait
// is bounded (a.max_polls rounds): a wave that gives up raises a.abort and
// treats the missing chunks as empty.
constexpr int CT_BATCH = 8;

__device__ __forceinline__ void part_put(const AttnArgs &a, int64_t idx, uint32_t tag, float v)
{
    if (a.t_part)
        tput(a.t_part + idx, tag, v);
    else
        a.part[idx] = v;
}

// Tag of this workgroup's launch (ticket drawn at entry by thread 0); every
// thread of the workgroup must call it.
__device__ __forceinline__ uint32_t attn_tag(const AttnArgs &a, unsigned long long ticket)
{
    __shared__ uint32_t s_tag;
    const int nwg = gridDim.x * gridDim.y;
    if (threadIdx.x == 0) s_tag = ticket_tag(ticket, nwg, ticket_counters(nwg));
    __syncthreads();
    return s_tag;
}

__device__ __forceinline__ unsigned long long attn_ticket(const AttnArgs &a)
{
    if (!a.t_part || threadIdx.x != 0) return 0;
    const int nwg = gridDim.x * gridDim.y;
    return draw_ticket(a.tickets, ticket_counters(nwg), blockIdx.x + blockIdx.y * gridDim.x);
}

template <int EPL>
__device__ void attn_combine_tail(const AttnArgs &a, int c, int kvh, int n_active, uint32_t tag,
                                  float *sm, AtStamps st)
{
    constexpr int HD = 64 * EPL;
    const int gqa = a.nh / a.nkv, ps = HD + 2;
    // this workgroup's heads: a contiguous run, so that each round of up to
    // four heads is one stretch of the output and of its limbs
    const int hpm = (gqa + n_active - 1) / n_active;
    const int g_begin = c * hpm, g_end = min(gqa, g_begin + hpm);
    if (g_begin >= gqa) return;
    __shared__ float red[16];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    float *go = sm, *gm = go + AT_WAVES * HD, *gl = gm + AT_WAVES, *xo = gl + AT_WAVES;
    const int64_t cs = (int64_t)gqa * ps;  // stride between chunks
    for (int r0 = g_begin; r0 < g_end; r0 += AT_WAVES) {
        // the round's heads are merged at once: wph waves per head, each
        // taking every wph-th chunk
        const int nr = min(AT_WAVES, g_end - r0), wph = AT_WAVES / nr;
        const int hs = wave / wph, sw = wave - hs * wph;
        float m = -INFINITY, l = 0.0f, o[EPL];
#pragma unroll
        for (int e = 0; e < EPL; e++) o[e] = 0.0f;
        if (hs < nr) {
            const uint64_t *pk = a.t_part + (int64_t)kvh * a.max_chunks * cs + (int64_t)(r0 + hs) * ps;
            for (int c0 = sw; c0 < n_active; c0 += wph * CT_BATCH) {
                float mc[CT_BATCH], lc[CT_BATCH], oc[CT_BATCH][EPL];
                uint32_t pend = 0;
#pragma unroll
                for (int b = 0; b < CT_BATCH; b++) {
                    mc[b] = -INFINITY;
                    lc[b] = 0.0f;
#pragma unroll
                    for (int e = 0; e < EPL; e++) oc[b][e] = 0.0f;
                    if (c0 + wph * b < n_active) pend |= 1u << b;
                }
                for (int polls = 0; __any(pend != 0); polls++) {
                    // every word of the batch is loaded each round, with no
                    // branch between the loads (a chunk past the context
                    // reads the batch's first): all of them are then in
                    // flight together, instead of one chunk per round trip
                    uint64_t wm[CT_BATCH], wl[CT_BATCH], wo[CT_BATCH][EPL];
#pragma unroll
                    for (int b = 0; b < CT_BATCH; b++) {
                        const int cc = c0 + wph * b;
                        const uint64_t *pp = pk + (int64_t)(cc < n_active ? cc : c0) * cs;
                        wm[b] = tget(pp + HD);
                        wl[b] = tget(pp + HD + 1);
#pragma unroll
                        for (int e = 0; e < EPL; e++) wo[b][e] = tget(pp + lane * EPL + e);
                    }
#pragma unroll
                    for (int b = 0; b < CT_BATCH; b++) {
                        bool ok = ((pend >> b) & 1u) && tvalid(wm[b], tag) && tvalid(wl[b], tag);
#pragma unroll
                        for (int e = 0; e < EPL; e++) ok = ok && tvalid(wo[b][e], tag);
                        if (ok) {
                            mc[b] = tval(wm[b]);
                            lc[b] = tval(wl[b]);
#pragma unroll
                            for (int e = 0; e < EPL; e++) oc[b][e] = tval(wo[b][e]);
                            pend &= ~(1u << b);
                        }
                    }
                    if (!__any(pend != 0)) break;
                    if (polls >= a.max_polls || ((polls & 31) == 31 && abort_seen(a.abort))) {
                        if (lane == 0) abort_raise(a.abort);
                        // missing chunks count as empty: the result is wrong
                        // and the launch reports it through the abort flag
#pragma unroll
                        for (int b = 0; b < CT_BATCH; b++)
                            if ((pend >> b) & 1u) mc[b] = -INFINITY;
                        break;
                    }
                    __builtin_amdgcn_s_sleep(1);
                }
                if (r0 == g_begin && c0 == sw) st.at(4);
                // the batch merged at once: its maximum first, then every
                // chunk's factor (independent exponentials, not a chain of
                // rescalings)
                float mn = m;
#pragma unroll
                for (int b = 0; b < CT_BATCH; b++) mn = fmaxf(mn, mc[b]);
                if (mn != -INFINITY) {
                    const float fa = expf(m - mn);  // 0 while nothing is merged (m = -inf)
                    l *= fa;
#pragma unroll
                    for (int e = 0; e < EPL; e++) o[e] *= fa;
#pragma unroll
                    for (int b = 0; b < CT_BATCH; b++) {
                        const float fb = mc[b] == -INFINITY ? 0.0f : expf(mc[b] - mn);
                        l += lc[b] * fb;
#pragma unroll
                        for (int e = 0; e < EPL; e++) o[e] += oc[b][e] * fb;
                    }
                    m = mn;
                }
            }
        }
        __syncthreads();  // sm is free (the attention phase is over, or the previous round)
#pragma unroll
        for (int e = 0; e < EPL; e++) go[wave * HD + lane * EPL + e] = o[e];
        if (lane == 0) {
            gm[wave] = m;
            gl[wave] = l;
        }
        __syncthreads();
        // the waves of each head merged, the outputs written, their limbs
        // built (the common one- and two-head rounds with constant bounds)
        auto finish = [&](auto wph_c, auto nr_c) {
            constexpr int WPH = decltype(wph_c)::value, NR = decltype(nr_c)::value;
            const int n = NR ? NR * HD : nr * HD;
            for (int t = threadIdx.x; t < n; t += AT_WG) {
                const int hl = t / HD, i = t - hl * HD, w0 = hl * WPH;
                float M = gm[w0];
#pragma unroll
                for (int q = 1; q < WPH; q++) M = fmaxf(M, gm[w0 + q]);
                float L = 0.0f, O = 0.0f;
#pragma unroll
                for (int q = 0; q < WPH; q++) {
                    const float f = gm[w0 + q] == -INFINITY ? 0.0f : expf(gm[w0 + q] - M);
                    L += gl[w0 + q] * f;
                    O += go[(w0 + q) * HD + i] * f;
                }
                const float v = O / L;
                gst(a.out + (int64_t)(kvh * gqa + r0 + hl) * HD + i, v);
                xo[t] = v;
            }
            if (a.xq.A) {
                __syncthreads();
                xq_build<AT_WG>(xo, nullptr, 0.0f, false, n, xq_shift(a.xq, (kvh * gqa + r0) * HD), red,
                         nullptr);
            }
        };
        if (wph == AT_WAVES)
            finish(std::integral_constant<int, AT_WAVES>{}, std::integral_constant<int, 1>{});
        else if (wph == AT_WAVES / 2)
            finish(std::integral_constant<int, AT_WAVES / 2>{}, std::integral_constant<int, 2>{});
        else
            finish(std::integral_constant<int, 1>{}, std::integral_constant<int, 0>{});
    }
}

// A context of one chunk per kv head (n_active == 1): the workgroup's merged
// (m, l, o) already is the output, O / L (the in-kernel merge of a single
// chunk computes the same quotient: its factor is exactly 1), so it is
// written directly with no exchange.  xo holds the kv head's gqa * HD output
// values in LDS; this builds their limbs (the o-proj input).
template <int HD>
__device__ __forceinline__ void attn_solo_limbs(const AttnArgs &a, int kvh, int gqa, const float *xo)
{
    __shared__ float red[16];
    if (!a.xq.A) return;
    __syncthreads();
    xq_build<AT_WG>(xo, nullptr, 0.0f, false, gqa * HD, xq_shift(a.xq, kvh * gqa * HD), red,
                    nullptr);
}

// Wave roles: the four waves of a workgroup split the gqa query heads into
// NHG head groups of HPW heads (HPW <= MAXH) and, when fewer than four
// groups exist, also split the chunk's 16-token tiles NTS = 4 / NHG ways.
// EPL = hd / 64 output values per lane.  Every global load of a tile (its
// K quarter-rows and all 16 V rows) is issued before any of it is used: the
// first tile's before the q heads are normalised and rotated, the next
// tile's K as soon as this tile's scores are formed and its V as soon as this
// tile's PV is done, with the page-table entries one tile further ahead.
// RR: the rope row of the position is given (AttnArgs::rope_row) and loaded
// at entry with the q heads.
template <int MAXH, int EPL, bool RR>
__global__ void __launch_bounds__(AT_WG) k_attn(AttnArgs a, int nhg, int hpw)
{
    constexpr int HD = 64 * EPL, PPL = (HD / 2 + 63) / 64, SEG = HD / 4;
    const int c = blockIdx.x, kvh = blockIdx.y;
    __shared__ uint64_t s_tr[AT_TRACE];
    const AtStamps st{a.trace ? s_tr : nullptr};
    st.clear();
    st.at(0);
    // the position through the scalar cache (the kernel never writes it):
    // its wait counts scalar loads only, not the vector loads below
    const int pos = *(const __attribute__((address_space(4))) int32_t *)a.pos;
    double2 cs[PPL];
    if constexpr (RR) cs_load<PPL>(cs, a.rope_row, HD);
    const int gqa = a.nh / a.nkv, kv_dim = a.nkv * HD;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int nts = AT_WAVES / nhg, hg = wave % nhg, ts = wave / nhg;
    const int g0 = hg * hpw;  // first head (within the kv head's group) of this wave
    const int tl = lane & (TILE - 1), qd = lane >> 4;  // token in tile, quarter of hd
    const int step = nts * TILE;  // this wave's tiles: tb, tb + step, ...
    // loads that do not depend on the position go out with it: this wave's
    // q heads and norm weights, the new k/v head, and the page-table entry
    // of this lane's first token for the minimum chunk size (the chunk size
    // of every short context)
    HeadIn<PPL> hq[MAXH], hk;
#pragma unroll
    for (int i = 0; i < MAXH; i++)
        if (i < hpw) head_load<PPL>(hq[i], a.q + (int64_t)(kvh * gqa + g0 + i) * HD, a.q_norm, HD);
    float vn[EPL];
    head_load<PPL>(hk, a.k + (int64_t)kvh * HD, a.k_norm, HD);
#pragma unroll
    for (int e = 0; e < EPL; e++) vn[e] = a.v[(int64_t)kvh * HD + lane * EPL + e];
    const int t_min = c * a.chunk + ts * TILE + tl, pg_min = t_min / a.page_tokens;
    const bool spec = pg_min < a.page_table_len;
    const int32_t pe_min = spec ? a.page_table[pg_min] : 0;
    const int n_t = pos + 1, chunk = attn_chunk(a, n_t);
    const int t0 = c * chunk;
    if (t0 >= n_t) {
        attn_ticket(a);  // every workgroup draws, also a chunk past the context
        return;
    }
    const int t1 = min(n_t, t0 + chunk);

    extern __shared__ __align__(16) float sm[];
    // per wave: q [MAXH][HD] | knew [HD] | vnew [HD] | p [MAXH][TILE]
    constexpr int PWF = MAXH * HD + 2 * HD + MAXH * TILE;
    float *qs = sm + wave * PWF;
    float *knew = qs + MAXH * HD;
    float *vnew = knew + HD;
    float *my_p = vnew + HD;

    // prologue loads, all independent: this wave's q heads, the rope row,
    // the new k/v head (in the chunk that holds pos), the first tile's
    // page-table entry
    const bool owns_pos = t1 == n_t;
    if constexpr (!RR) cs_load<PPL>(cs, a.rope + (int64_t)pos * (HD / 2), HD);
    int tb = t0 + ts * TILE;
    // K quarter-row of token tb+tl (this lane) and all 16 V rows of the tile
    // at [tb, tb+16): rows are pool offsets of each lane's token (lane i of
    // the first 16 holds token tb+i's)
    float4 kq[SEG / 4];
    float vv[TILE][EPL];
    auto load_k = [&](int64_t row, int tbase) {
        const bool ok = tbase + tl < t1;
#pragma unroll
        for (int j = 0; j < SEG / 4; j++)
            kq[j] = ok ? *(const float4 *)(a.kpool + row + qd * SEG + 4 * j)
                       : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    };
    // a lane's EPL values of a V row are contiguous: one load each
    auto load_v = [&](int64_t row, int tbase) {
        const int nt = min(TILE, t1 - tbase);
#pragma unroll
        for (int i = 0; i < TILE; i++) {
            const int64_t ri = __shfl(row, i);
            const float *src = a.vpool + ri + lane * EPL;
            if constexpr (EPL == 4) {
                const float4 v = i < nt ? *(const float4 *)src : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                vv[i][0] = v.x; vv[i][1] = v.y; vv[i][2] = v.z; vv[i][3] = v.w;
            } else if constexpr (EPL == 2) {
                const float2 v = i < nt ? *(const float2 *)src : make_float2(0.0f, 0.0f);
                vv[i][0] = v.x; vv[i][1] = v.y;
            } else {
                vv[i][0] = i < nt ? src[0] : 0.0f;
            }
        }
    };
    auto row_of = [&](int tbase) -> int64_t {
        return tbase + tl < t1 ? kv_off(a, tbase + tl, kvh, kv_dim) : 0;
    };
    if (tb < t1) {
        // the first tile's rows from the early page entry when the chunk
        // has its minimum size (then tb + tl == t_min)
        const int64_t row =
            spec && chunk == a.chunk
                ? (tb + tl < t1 ? kv_row(a, pe_min, t_min % a.page_tokens, kvh, kv_dim)
                                : 0)
                : row_of(tb);
        load_k(row, tb);
        load_v(row, tb);
    }
    int64_t row_n = row_of(tb + step);  // the next tile's rows, one tile ahead
    // the ticket (thread 0's atomic) after the q heads and the first tile:
    // vector loads and atomics are counted in order, so drawn before them
    // it would make the waits for the q heads wait for its round trip too
    const unsigned long long ticket = attn_ticket(a);

    // q heads (and the new k head) normalised and rotated into this wave's
    // LDS while the first tile's loads are in flight
#pragma unroll
    for (int i = 0; i < MAXH; i++)
        if (i < hpw) head_finish<PPL>(hq[i], cs, a.q_norm != nullptr, a.eps, HD, qs + i * HD);
    st.at(1);
    if (owns_pos) {
        head_finish<PPL>(hk, cs, a.k_norm != nullptr, a.eps, HD, knew);
#pragma unroll
        for (int e = 0; e < EPL; e++) vnew[lane * EPL + e] = vn[e];
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    float m_run[MAXH], l_run[MAXH], o[MAXH][EPL];
#pragma unroll
    for (int g = 0; g < MAXH; g++) {
        m_run[g] = -INFINITY;
        l_run[g] = 0.0f;
#pragma unroll
        for (int e = 0; e < EPL; e++) o[g][e] = 0.0f;
    }
    for (; tb < t1; tb += step) {
        const int t = tb + tl;
        const bool tv = t < t1;
        const int tn = tb + step;
        // the token at pos comes from LDS (its pool row is written at the end)
        if (t == pos) {
#pragma unroll
            for (int j = 0; j < SEG / 4; j++) kq[j] = *(const float4 *)(knew + qd * SEG + 4 * j);
        }
        if (pos >= tb && pos < tb + TILE) {
            const int ip = pos - tb;
#pragma unroll
            for (int i = 0; i < TILE; i++)
                if (i == ip) {
#pragma unroll
                    for (int e = 0; e < EPL; e++) vv[i][e] = vnew[lane * EPL + e];
                }
        }
        // scores: lane (tl, qd) dots quarter qd of K row tb+tl with each head
        float s[MAXH];
#pragma unroll
        for (int g = 0; g < MAXH; g++) {
            s[g] = 0.0f;
            if (g < hpw) {
#pragma unroll
                for (int j = 0; j < SEG / 4; j++) {
                    const float4 qv = *(const float4 *)(qs + g * HD + qd * SEG + 4 * j);
                    s[g] += qv.x * kq[j].x + qv.y * kq[j].y + qv.z * kq[j].z + qv.w * kq[j].w;
                }
            }
        }
        // kq is free: the next tile's K loads overlap this tile's softmax and PV
        if (tn < t1) load_k(row_n, tn);
#pragma unroll
        for (int g = 0; g < MAXH; g++) {
            if (g >= hpw) break;
            float v = sum_rows(s[g]);
            v = tv ? v * a.scale : -INFINITY;
            const float m_new = fmaxf(m_run[g], max16(v));
            const float p = tv ? expf(v - m_new) : 0.0f;
            const float corr = expf(m_run[g] - m_new);
            l_run[g] = l_run[g] * corr + sum16(p);
            m_run[g] = m_new;
#pragma unroll
            for (int e = 0; e < EPL; e++) o[g][e] *= corr;
            if (qd == 0) my_p[g * TILE + tl] = p;
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        // o[g][e] += sum_t p[g][t] * V[t][e] for this lane's EPL values
#pragma unroll
        for (int g = 0; g < MAXH; g++) {
            if (g < hpw) {
#pragma unroll
                for (int tt = 0; tt < TILE; tt += 4) {
                    const float4 p4 = *(const float4 *)(my_p + g * TILE + tt);
#pragma unroll
                    for (int e = 0; e < EPL; e++)
                        o[g][e] += p4.x * vv[tt][e] + p4.y * vv[tt + 1][e] + p4.z * vv[tt + 2][e] +
                                   p4.w * vv[tt + 3][e];
                }
            }
        }
        // vv is free: the next tile's V loads, then the page entries of the
        // tile after it
        if (tn < t1) load_v(row_n, tn);
        row_n = row_of(tn + step);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    st.at(2);
    if (owns_pos && wave == 0) {
        const int64_t po = kv_off(a, pos, kvh, kv_dim);
        for (int e = lane; e < HD; e += 64) {
            a.kpool[po + e] = knew[e];
            a.vpool[po + e] = vnew[e];
        }
    }

    const int ps = HD + 2;
    const int64_t part0 = ((int64_t)kvh * a.max_chunks + c) * gqa * ps;
    const uint32_t tag = a.t_part ? attn_tag(a, ticket) : 0u;
    const int n_active = (n_t + chunk - 1) / chunk;
    const bool solo = (a.t_part || a.solo_max > 0) && n_active == 1;
    if (nts == 1 && solo) {
        // every wave owns distinct heads: its running state is the output
        float *xo = sm + AT_WAVES * PWF;  // [gqa][HD] (the merge area, unused here)
#pragma unroll
        for (int g = 0; g < MAXH; g++) {
            if (g >= hpw) break;
#pragma unroll
            for (int e = 0; e < EPL; e++) {
                const int i = (g0 + g) * HD + lane * EPL + e;
                const float v = o[g][e] / l_run[g];
                gst(a.out + (int64_t)kvh * gqa * HD + i, v);
                xo[i] = v;
            }
        }
        st.at(3);
        attn_solo_limbs<HD>(a, kvh, gqa, xo);
        st.at(5);
        st.flush(a, c, kvh, n_active);
        return;
    }
    if (nts == 1) {
        // every wave owns distinct heads: its running state is the partial
#pragma unroll
        for (int g = 0; g < MAXH; g++) {
            if (g >= hpw) break;
            const int64_t pg = part0 + (g0 + g) * ps;
#pragma unroll
            for (int e = 0; e < EPL; e++) part_put(a, pg + lane * EPL + e, tag, o[g][e]);
            if (lane == 0) {
                part_put(a, pg + HD, tag, m_run[g]);
                part_put(a, pg + HD + 1, tag, l_run[g]);
            }
        }
        st.at(3);
        if (a.t_part) attn_combine_tail<EPL>(a, c, kvh, n_active, tag, sm, st);
        st.at(5);
        st.flush(a, c, kvh, n_active);
        return;
    }
    // merge the NTS waves of each head group: M = max m_w, L = sum l_w
    // e^(m_w-M), O likewise (LDS past the per-wave areas)
    float *mo = sm + AT_WAVES * PWF;          // [AT_WAVES][MAXH][HD]
    float *mm = mo + AT_WAVES * MAXH * HD;    // [AT_WAVES][MAXH]
    float *ml = mm + AT_WAVES * MAXH;         // [AT_WAVES][MAXH]
#pragma unroll
    for (int g = 0; g < MAXH; g++) {
        if (g >= hpw) break;
#pragma unroll
        for (int e = 0; e < EPL; e++) mo[(wave * MAXH + g) * HD + lane * EPL + e] = o[g][e];
        if (lane == 0) {
            mm[wave * MAXH + g] = m_run[g];
            ml[wave * MAXH + g] = l_run[g];
        }
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < gqa * HD; idx += AT_WG) {
        const int gg = idx / HD, e = idx - gg * HD;
        const int hgi = gg / hpw, gi = gg - hgi * hpw;  // head group, head within it
        float M = -INFINITY;
        for (int w = 0; w < nts; w++) M = fmaxf(M, mm[(w * nhg + hgi) * MAXH + gi]);
        float O = 0.0f, L = 0.0f;
        for (int w = 0; w < nts; w++) {
            const int wi = (w * nhg + hgi) * MAXH + gi;
            const float f = expf(mm[wi] - M);
            O += mo[wi * HD + e] * f;
            L += ml[wi] * f;
        }
        if (solo) {
            const float v = O / L;
            gst(a.out + (int64_t)kvh * gqa * HD + idx, v);
            sm[idx] = v;  // the per-wave areas are free after the barrier
            continue;
        }
        part_put(a, part0 + gg * ps + e, tag, O);
        if (e == 0) {
            part_put(a, part0 + gg * ps + HD, tag, M);
            part_put(a, part0 + gg * ps + HD + 1, tag, L);
        }
    }
    st.at(3);
    if (solo)
        attn_solo_limbs<HD>(a, kvh, gqa, sm);
    else if (a.t_part)
        attn_combine_tail<EPL>(a, c, kvh, n_active, tag, sm, st);
    st.at(5);
    st.flush(a, c, kvh, n_active);
}

// ---------------------------------------------------------------------------
// Matrix-core variant for head_dim 128 and 16 query heads per kv head (the
// 235B-A22B shape; fewer heads would be padded, which the head-split VALU
// kernel above does better).  Per 16-token tile a wave forms all heads' scores with
// v_mfma_f32_16x16x4_f32, S[h][t] = sum_d Q[h][d] K[t][d], 32 k-steps (lane
// l holds S[4(l/16)+r][l%16]); runs the online softmax with reductions over
// the 16 lanes of a row; moves P through LDS into the A-operand layout; and
// accumulates O[h][d] += sum_t P[h][t] V[t][d] with 32 more MFMAs.  The
// k dimension of Q.K is split as d = kcol(l/16, m) and the output columns
// as d = vcol(l%16, b) (below), so that each 16-byte load of a wave reads
// whole 64-byte runs of a K or V row (consecutive lanes, consecutive 16
// bytes).  Arithmetic stays f32 throughout.
// Lane layout of the builtin (checked on gfx950): lane l supplies
// A[l%16][l/16] and B[l/16][l%16], and receives D[4(l/16)+r][l%16], r < 4.
typedef float f4v __attribute__((ext_vector_type(4)));
constexpr int MH = 16;      // padded heads per kv head
constexpr int MHD = 128;    // head_dim of this variant
constexpr int MNB = MHD / 16;
constexpr int ATTN_PT_LDS = 256;  // page-table entries kept in LDS (128K tokens of 512)
// page-table entries copied to LDS by a FAST launch (1M tokens of 512)
constexpr int ATTN_PT_FAST = 2048;
static_assert(ATTN_PT_FAST % AT_WG == 0, "whole entries per thread");
// Column of Q and K that lane group g supplies at k-step m (m < 32), and
// the output column of lane r's accumulator block b (b < 8).
__device__ __forceinline__ constexpr int kcol(int g, int m) { return 16 * (m >> 2) + 4 * g + (m & 3); }
__device__ __forceinline__ constexpr int vcol(int r, int b) { return 64 * (b >> 2) + 4 * r + (b & 3); }

// FAST: the launch gives the rope row of the position (AttnArgs::rope_row),
// a page table of 1 to ATTN_PT_FAST entries (page_table_len) and pages of a
// power of two of tokens.  The
// table is then copied to LDS with the first loads and every K/V address
// comes from LDS; otherwise the position's rope row and the page entries
// past the minimum chunk size are read after the position.
// GQ: the query heads per kv head when known at compile time (8 or 16 on
// FAST launches: the merge and output loops then have constant bounds), 0:
// a.nh / a.nkv.
template <bool FAST, int GQ>
__global__ void __launch_bounds__(AT_WG) k_attn_mfma(AttnArgs a)
{
    const int c = blockIdx.x, kvh = blockIdx.y;
    __shared__ uint64_t s_tr[AT_TRACE];
    const AtStamps st{a.trace ? s_tr : nullptr};
    st.clear();
    st.at(0);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int lr = lane & 15, lg = lane >> 4;  // row-lane, k-group
    const int gqa = GQ ? GQ : a.nh / a.nkv, kv_dim = a.nkv * MHD;
    // The position goes through the scalar cache (the kernel never writes
    // it), so its wait counts scalar loads only.  The vector loads are
    // issued in the order they are needed, each of them on every path (a
    // head past gqa reads head gqa - 1, every wave reads the new k/v head,
    // a table entry past the end reads the last one): gfx950 counts vector
    // loads in order, and a wait for one then leaves the later ones in
    // flight.
    const int pos = *(const __attribute__((address_space(4))) int32_t *)a.pos;
    const int pt_n = a.page_table_len;
    constexpr int PT_CAP = FAST ? ATTN_PT_FAST : ATTN_PT_LDS;
    constexpr int PT_PER = FAST ? ATTN_PT_FAST / AT_WG : 1;
    __shared__ int32_t s_pt[PT_CAP];
    int32_t pte[PT_PER];
    int32_t pe_min = 0;
    const int t_min = c * a.chunk + wave * 16 + lr;
    const int pg_min = FAST ? 0 : t_min / a.page_tokens;  // (the early entry: generic launches)
    const bool spec = pg_min < pt_n;
    double2 cs[1];
    if constexpr (FAST) {
#pragma unroll
        for (int j = 0; j < PT_PER; j++)
            pte[j] = a.page_table[min((int)threadIdx.x + AT_WG * j, pt_n - 1)];
        cs_load<1>(cs, a.rope_row, MHD);
    } else {
        // the page entry of this lane's first token at the minimum chunk
        // size, the chunk size of every short context
        pe_min = a.page_table[spec ? pg_min : 0];
    }

    extern __shared__ __align__(16) float sm[];
    float *qs = sm;                      // [MH][MHD] normalised, rotated q (zero rows past gqa)
    float *knew = qs + MH * MHD;         // [MHD]
    float *vnew = knew + MHD;            // [MHD]
    float *pt = vnew + MHD;              // [AT_WAVES][MH][16] probabilities
    float *mo = pt + AT_WAVES * MH * 16; // [AT_WAVES][MH][MHD] merge area
    float *mm = mo + AT_WAVES * MH * MHD;
    float *ml = mm + AT_WAVES * MH;

    // this wave's q heads (heads wave + 4 j) and norm weights, and the new
    // k/v head
    constexpr int HPW = MH / AT_WAVES;
    HeadIn<1> hq[HPW], hk;
#pragma unroll
    for (int j = 0; j < HPW; j++) {
        const int i = min(wave + AT_WAVES * j, gqa - 1);
        head_load_all<1>(hq[j], a.q + (int64_t)(kvh * gqa + i) * MHD, a.q_norm, MHD);
    }
    float vn[MHD / 64];
    head_load_all<1>(hk, a.k + (int64_t)kvh * MHD, a.k_norm, MHD);
#pragma unroll
    for (int e = 0; e < MHD / 64; e++) vn[e] = a.v[(int64_t)kvh * MHD + lane + 64 * e];
    // the page table in LDS: the whole of it (FAST), or when it is short:
    // past the minimum chunk size (long contexts) the first tile's page
    // entry then needs no memory trip after the position, nor does any
    // later tile's
    const bool pt_lds = FAST || (pt_n > 0 && pt_n <= ATTN_PT_LDS);
    if constexpr (FAST) {
#pragma unroll
        for (int j = 0; j < PT_PER; j++) s_pt[threadIdx.x + AT_WG * j] = pte[j];
    } else if (pt_lds) {
        for (int i = threadIdx.x; i < pt_n; i += AT_WG) s_pt[i] = a.page_table[i];
    }

    const int n_t = pos + 1, chunk = attn_chunk(a, n_t);
    const int t0 = c * chunk;
    if (t0 >= n_t) {
        attn_ticket(a);  // every workgroup draws, also a chunk past the context
        return;
    }
    __syncthreads();  // s_pt
    const int t1 = min(n_t, t0 + chunk);
    const bool owns_pos = t1 == n_t;
    if constexpr (!FAST) cs_load<1>(cs, a.rope + (int64_t)pos * (MHD / 2), MHD);

    const int step = AT_WAVES * 16;
    int tb = t0 + wave * 16;
    float kv[MHD / 4];     // K[tb + lr][kcol(lg, m)]
    float vvr[4][MNB];     // V[tb + 4q + lg][vcol(lr, b)]
    // (FAST: page_tokens is a power of two, so the page and the row within
    // it are a shift and a mask)
    const int pshift = FAST ? __builtin_ctz((unsigned)a.page_tokens) : 0;
    auto kv_at = [&](int t) -> int64_t {
        if (FAST) return kv_row(a, s_pt[t >> pshift], t & (a.page_tokens - 1), kvh, kv_dim);
        if (!pt_lds) return kv_off(a, t, kvh, kv_dim);
        return kv_row(a, s_pt[t / a.page_tokens], t % a.page_tokens, kvh, kv_dim);
    };
    // Every tile issues the same loads on every lane, with nothing done to
    // their results before use, so that the waits for the q heads and for
    // each tile count only older loads: a token past the chunk reads the
    // new k and v heads of the launch (finite values: its score is masked
    // and its probability 0), and the token at pos reads V from the new v
    // head (its pool row is written at the end) and has its K replaced by
    // the rotated head from LDS
    const float *k_in = a.k + (int64_t)kvh * MHD, *v_in = a.v + (int64_t)kvh * MHD;
    // the early page entries apply to a table in memory at the minimum
    // chunk size
    const bool early = !FAST && chunk == a.chunk && !pt_lds && pt_n > 0;
    auto row_of = [&](int tbase) -> int64_t { return tbase + lr < t1 ? kv_at(tbase + lr) : 0; };
    auto load_k = [&](int64_t row, int tbase) {
        const float *src = tbase + lr < t1 ? a.kpool + row : k_in;
#pragma unroll
        for (int m = 0; m < MHD / 4; m += 4) {
            const float4 v = *(const float4 *)(src + kcol(lg, m));
            kv[m] = v.x; kv[m + 1] = v.y; kv[m + 2] = v.z; kv[m + 3] = v.w;
        }
    };
    auto load_v = [&](int64_t row, int tbase) {
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int t = tbase + 4 * q + lg;  // token of this k-step
            const int64_t rq = __shfl(row, 4 * q + lg);
            const float *src = t < t1 && t != pos ? a.vpool + rq : v_in;
#pragma unroll
            for (int b = 0; b < MNB; b += 4) {
                const float4 v = *(const float4 *)(src + vcol(lr, b));
                vvr[q][b] = v.x; vvr[q][b + 1] = v.y; vvr[q][b + 2] = v.z; vvr[q][b + 3] = v.w;
            }
        }
    };
    // the first tile's loads (every wave has one; t0 + 16 wave may be past
    // the chunk), from the early page entry when the table is in memory and
    // the chunk has its minimum size (then tb + lr == t_min)
    {
        const int64_t row = early && spec && tb + lr < t1
                                ? kv_row(a, pe_min, t_min % a.page_tokens, kvh, kv_dim)
                                : row_of(tb);
        load_k(row, tb);
        load_v(row, tb);
    }
    int64_t row_n = row_of(tb + step);
    // the ticket after the q heads and the first tile (as in k_attn)
    const unsigned long long ticket = attn_ticket(a);

    // the q heads and, in the chunk holding pos, the new k/v head,
    // normalised and rotated into LDS while the first tile is in flight
#pragma unroll
    for (int j = 0; j < HPW; j++) {
        const int i = wave + AT_WAVES * j;
        if (i < gqa)
            head_finish<1>(hq[j], cs, a.q_norm != nullptr, a.eps, MHD, qs + i * MHD);
        else
            for (int e = lane; e < MHD; e += 64) qs[i * MHD + e] = 0.0f;
    }
    st.at(1);
    if (owns_pos && wave == 0) {
        head_finish<1>(hk, cs, a.k_norm != nullptr, a.eps, MHD, knew);
#pragma unroll
        for (int e = 0; e < MHD / 64; e++) vnew[lane + 64 * e] = vn[e];
    }
    __syncthreads();
    // this lane's Q operand: Q[lr][kcol(lg, m)], m < 32
    float qv[MHD / 4];
#pragma unroll
    for (int m = 0; m < MHD / 4; m += 4) {
        const float4 v = *(const float4 *)(qs + lr * MHD + kcol(lg, m));
        qv[m] = v.x; qv[m + 1] = v.y; qv[m + 2] = v.z; qv[m + 3] = v.w;
    }

    float m_run[4], l_run[4];
    f4v o[MNB];
#pragma unroll
    for (int r = 0; r < 4; r++) {
        m_run[r] = -INFINITY;
        l_run[r] = 0.0f;
    }
#pragma unroll
    for (int b = 0; b < MNB; b++) o[b] = (f4v){0.0f, 0.0f, 0.0f, 0.0f};
    float *my_p = pt + wave * MH * 16;
    for (; tb < t1; tb += step) {
        const int tn = tb + step;
        const bool tv = tb + lr < t1;
        // the K of the token at pos comes from LDS (its pool row is written
        // at the end of the kernel)
        if (tb + lr == pos) {
#pragma unroll
            for (int m = 0; m < MHD / 4; m++) kv[m] = knew[kcol(lg, m)];
        }
        // four independent accumulation chains over the k-steps
        f4v sc4[4];
#pragma unroll
        for (int j = 0; j < 4; j++) sc4[j] = (f4v){0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int m = 0; m < MHD / 4; m++)
            sc4[m & 3] = __builtin_amdgcn_mfma_f32_16x16x4f32(qv[m], kv[m], sc4[m & 3], 0, 0, 0);
        const f4v sacc = (sc4[0] + sc4[1]) + (sc4[2] + sc4[3]);
        // kv is free: the next tile's K (issued also after the last tile, as
        // loads of the new k head, so that every trip issues the same loads
        // and the wait for this tile's V leaves them in flight)
        load_k(row_n, tn);
        // online softmax; lane holds heads 4 lg + r, token lr
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const float sv = tv ? sacc[r] * a.scale : -INFINITY;
            const float m_new = fmaxf(m_run[r], max16(sv));
            const float p = tv ? expf(sv - m_new) : 0.0f;
            const float corr = expf(m_run[r] - m_new);
            l_run[r] = l_run[r] * corr + sum16(p);
            m_run[r] = m_new;
#pragma unroll
            for (int b = 0; b < MNB; b++) o[b][r] *= corr;
            my_p[(4 * lg + r) * 16 + lr] = p;
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        // O += P V: A[h = lr][t = 4q + lg] = P, B[t][j = lr] = V[t][vcol(lr, b)]
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const float pa = my_p[lr * 16 + 4 * q + lg];
#pragma unroll
            for (int b = 0; b < MNB; b++)
                o[b] = __builtin_amdgcn_mfma_f32_16x16x4f32(pa, vvr[q][b], o[b], 0, 0, 0);
        }
        load_v(row_n, tn);  // vvr is free
        row_n = row_of(tn + step);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }

    st.at(2);
    // merge the four waves (each covered every head over its own tiles)
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const int h = 4 * lg + r;
#pragma unroll
        for (int b = 0; b < MNB; b++) mo[(wave * MH + h) * MHD + vcol(lr, b)] = o[b][r];
        if (lr == 0) {
            mm[wave * MH + h] = m_run[r];
            ml[wave * MH + h] = l_run[r];
        }
    }
    const uint32_t tag = a.t_part ? attn_tag(a, ticket) : 0u;  // (a barrier)
    __syncthreads();
    // per head: M = max_w m_w, the waves' factors f_w = e^(m_w - M) and
    // L = sum_w l_w f_w, once (in the probabilities' LDS, free now); then
    // O = sum_w o_w f_w per output value
    float *mf = pt;              // [AT_WAVES][MH]
    float *mM = pt + AT_WAVES * MH, *mL = mM + MH;
    if ((int)threadIdx.x < gqa) {
        const int h = threadIdx.x;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < AT_WAVES; w++) M = fmaxf(M, mm[w * MH + h]);
        float L = 0.0f;
#pragma unroll
        for (int w = 0; w < AT_WAVES; w++) {
            const float mw = mm[w * MH + h];
            const float f = mw == -INFINITY ? 0.0f : expf(mw - M);
            mf[w * MH + h] = f;
            L += ml[w * MH + h] * f;
        }
        mM[h] = M;
        mL[h] = L;
    }
    __syncthreads();
    const int ps = MHD + 2;
    const int64_t part0 = ((int64_t)kvh * a.max_chunks + c) * gqa * ps;
    const int n_active = (n_t + chunk - 1) / chunk;
    const bool solo = (a.t_part || a.solo_max > 0) && n_active == 1;
    for (int idx = threadIdx.x; idx < gqa * MHD; idx += AT_WG) {
        const int h = idx / MHD, e = idx - h * MHD;
        float O = 0.0f;
#pragma unroll
        for (int w = 0; w < AT_WAVES; w++) O += mo[(w * MH + h) * MHD + e] * mf[w * MH + h];
        if (solo) {
            const float v = O / mL[h];
            gst(a.out + (int64_t)kvh * gqa * MHD + idx, v);
            qs[idx] = v;  // q is no longer read
            continue;
        }
        part_put(a, part0 + h * ps + e, tag, O);
        if (e == 0) {
            part_put(a, part0 + h * ps + MHD, tag, mM[h]);
            part_put(a, part0 + h * ps + MHD + 1, tag, mL[h]);
        }
    }
    st.at(3);
    if (solo)
        attn_solo_limbs<MHD>(a, kvh, gqa, qs);
    else if (a.t_part)
        attn_combine_tail<MHD / 64>(a, c, kvh, n_active, tag, sm, st);
    // the new k/v rows go to the pool last (the tiles took them from LDS):
    // gfx950 counts stores with the loads, so a store issued earlier would
    // hold up every later wait for a load until it is acknowledged
    if (owns_pos && wave == 0) {
        const int64_t po = kv_at(pos);
        for (int e = lane; e < MHD; e += 64) {
            a.kpool[po + e] = knew[e];
            a.vpool[po + e] = vnew[e];
        }
    }
    st.at(5);
    st.flush(a, c, kvh, n_active);
}

// Merge the per-chunk partials (m, l, o) of one query head: M = max m_c,
// L = sum l_c e^(m_c-M), out = sum o_c e^(m_c-M) / L; then the limbs of the
// slice.  One workgroup per (head, 32 output values): at long contexts a
// head has up to a few hundred chunks, and spreading each head over hd / 32
// workgroups keeps the reads of one workgroup (and CU) small.  Each half
// wave takes every eighth chunk, lane l value l % 32, in batches of 8
// chunks whose loads are all issued before any is merged into the running
// (m, l, o), the first batch's together with the position's (16-chunk
// batches, one for the 128 chunks of a long context, measured no faster);
// the eight half waves are merged in LDS.
constexpr int CB_WG = 256, CB_DIMS = 32, CB_HALVES = CB_WG / 32, CB_BATCH = 8;

__global__ void __launch_bounds__(CB_WG) k_attn_combine(AttnArgs a)
{
    __shared__ float s_o[CB_HALVES][CB_DIMS], s_m[CB_HALVES], s_l[CB_HALVES], xs[CB_DIMS];
    __shared__ float red[16];
    const int h = blockIdx.x, d0 = blockIdx.y * CB_DIMS, gqa = a.nh / a.nkv, hd = a.hd, ps = hd + 2;
    const int kvh = h / gqa, g = h - kvh * gqa;
    const int64_t cs = (int64_t)gqa * ps;  // stride between chunks
    const float *pk = a.part + (int64_t)kvh * a.max_chunks * cs + (int64_t)g * ps;
    const int half = threadIdx.x >> 5, dl = threadIdx.x & 31;
    // the first batch's loads go out with the position's (every chunk of the
    // grid; those past the context are dropped once it is known)
    const int *posp = a.pos;
    int n_active = -1;
    float m = -INFINITY, l = 0.0f, o = 0.0f;
    // the batches past the first stop at the live context (known from then on)
    for (int c0 = half; c0 < (n_active < 0 ? a.max_chunks : n_active); c0 += CB_HALVES * CB_BATCH) {
        float mc[CB_BATCH], lc[CB_BATCH], oc[CB_BATCH];
#pragma unroll
        for (int b = 0; b < CB_BATCH; b++) {
            const int cc = c0 + CB_HALVES * b;
            const float *pp = pk + (cc < a.max_chunks ? cc : 0) * cs;
            mc[b] = pp[hd];
            lc[b] = pp[hd + 1];
            oc[b] = pp[d0 + dl];
        }
        if (n_active < 0) {
            const int n_t = *posp + 1, chunk = attn_chunk(a, n_t);
            n_active = (n_t + chunk - 1) / chunk;
        }
        // the batch merged at once (its maximum, then independent factors)
#pragma unroll
        for (int b = 0; b < CB_BATCH; b++)
            if (c0 + CB_HALVES * b >= n_active) {  // a chunk past the context: its words are stale
                mc[b] = -INFINITY;
                lc[b] = 0.0f;
                oc[b] = 0.0f;
            }
        float mn = m;
#pragma unroll
        for (int b = 0; b < CB_BATCH; b++) mn = fmaxf(mn, mc[b]);
        if (mn != -INFINITY) {
            const float fa = expf(m - mn);  // 0 while nothing is merged (m = -inf)
            l *= fa;
            o *= fa;
#pragma unroll
            for (int b = 0; b < CB_BATCH; b++) {
                const float fb = mc[b] == -INFINITY ? 0.0f : expf(mc[b] - mn);
                l += lc[b] * fb;
                o += oc[b] * fb;
            }
            m = mn;
        }
    }
    s_o[half][dl] = o;
    if (dl == 0) {
        s_m[half] = m;
        s_l[half] = l;
    }
    __syncthreads();
    if (threadIdx.x < CB_DIMS) {
        const int i = threadIdx.x;
        float M = s_m[0];
#pragma unroll
        for (int q = 1; q < CB_HALVES; q++) M = fmaxf(M, s_m[q]);
        float L = 0.0f, O = 0.0f;
#pragma unroll
        for (int q = 0; q < CB_HALVES; q++) {
            const float f = s_m[q] == -INFINITY ? 0.0f : expf(s_m[q] - M);
            L += s_l[q] * f;
            O += s_o[q][i] * f;
        }
        const float v = O / L;
        a.out[(int64_t)h * hd + d0 + i] = v;
        xs[i] = v;
    }
    if (!a.xq.A) return;
    __syncthreads();
    xq_build<CB_WG>(xs, nullptr, 0.0f, false, CB_DIMS, xq_shift(a.xq, h * hd + d0), red, nullptr);
}

template <int MAXH, bool RR>
static void launch_k_attn(hipStream_t st, const AttnArgs &a, int nhg, int hpw)
{
    const dim3 grid(a.max_chunks, a.nkv);
    const size_t lds = sizeof(float) * (AT_WAVES * ((size_t)MAXH * a.hd + 2 * a.hd + MAXH * TILE) +
                                        (size_t)AT_WAVES * MAXH * a.hd + 2 * AT_WAVES * MAXH);
    switch (a.hd) {
    case 64: hipLaunchKernelGGL((k_attn<MAXH, 1, RR>), grid, dim3(AT_WG), lds, st, a, nhg, hpw); break;
    case 128: hipLaunchKernelGGL((k_attn<MAXH, 2, RR>), grid, dim3(AT_WG), lds, st, a, nhg, hpw); break;
    default: hipLaunchKernelGGL((k_attn<MAXH, 4, RR>), grid, dim3(AT_WG), lds, st, a, nhg, hpw); break;
    }
}

hipError_t launch_attn_decode(hipStream_t st, const AttnArgs &a)
{
    const int gqa = a.nkv > 0 ? a.nh / a.nkv : 0;
    if (gqa < 1 || gqa > 16 || a.nh % a.nkv || (a.hd != 64 && a.hd != 128 && a.hd != 256) ||
        a.chunk < TILE || a.chunk % TILE || a.page_tokens < 1 || a.max_chunks < 1 ||
        (a.t_part && (!a.tickets || !a.abort || a.max_polls < 1)) ||
        (a.solo_max > 0 && !a.t_part && a.max_chunks != 1))
        return hipErrorInvalidValue;
    // the matrix-core variant serves 16 query heads per kv head, and a
    // single-chunk context (solo_max) of 4 to 16; its waves split tokens, so
    // its chunks hold at least one 16-token tile per wave
    const bool use_mfma = a.hd == MHD && (gqa == MH || (a.solo_max > 0 && gqa >= 4));
    AttnArgs am = a;
    if (use_mfma) {
        am.chunk = std::max(a.chunk, AT_WAVES * TILE);
        // two of its 4-wave workgroups fit a CU (about 220 registers per
        // lane): one round of workgroups on 256 CUs
        am.max_chunks = std::max(1, std::min(a.max_chunks, 512 / a.nkv));
    }
    // merged in-kernel: the context spans at most ATTN_MERGE_MAX_CHUNKS
    // chunks of the minimum size, so no chunk workgroup past that count has
    // work (and the chunk size is the same as with the full grid)
    if (a.t_part) am.max_chunks = std::min(am.max_chunks, ATTN_MERGE_MAX_CHUNKS);
    if (use_mfma) {
        const size_t lds = sizeof(float) * ((size_t)MH * MHD + 2 * MHD + AT_WAVES * MH * 16 +
                                            (size_t)AT_WAVES * MH * MHD + 2 * AT_WAVES * MH);
        const dim3 grid(am.max_chunks, am.nkv);
        if (a.rope_row && a.page_table_len >= 1 && a.page_table_len <= ATTN_PT_FAST &&
            (a.page_tokens & (a.page_tokens - 1)) == 0) {
            if (gqa == 8)
                hipLaunchKernelGGL((k_attn_mfma<true, 8>), grid, dim3(AT_WG), lds, st, am);
            else if (gqa == 16)
                hipLaunchKernelGGL((k_attn_mfma<true, 16>), grid, dim3(AT_WG), lds, st, am);
            else
                hipLaunchKernelGGL((k_attn_mfma<true, 0>), grid, dim3(AT_WG), lds, st, am);
        } else {
            hipLaunchKernelGGL((k_attn_mfma<false, 0>), grid, dim3(AT_WG), lds, st, am);
        }
    } else {
    // head groups: the largest of 4, 2, 1 dividing gqa
    const int nhg = gqa % 4 == 0 ? 4 : gqa % 2 == 0 ? 2 : 1;
    const int hpw = gqa / nhg;
    if (hpw <= 1)
        a.rope_row ? launch_k_attn<1, true>(st, am, nhg, hpw) : launch_k_attn<1, false>(st, am, nhg, hpw);
    else if (hpw <= 2)
        a.rope_row ? launch_k_attn<2, true>(st, am, nhg, hpw) : launch_k_attn<2, false>(st, am, nhg, hpw);
    else if (hpw <= 4)
        a.rope_row ? launch_k_attn<4, true>(st, am, nhg, hpw) : launch_k_attn<4, false>(st, am, nhg, hpw);
    else
        return hipErrorInvalidValue;  // gqa of 5, 7, 9.. above 4 heads per wave
    }
    hipError_t e = hipGetLastError();
    // combined inside the kernel, or a single chunk written directly
    if (e != hipSuccess || a.t_part || a.solo_max > 0) return e;
    hipLaunchKernelGGL(k_attn_combine, dim3(a.nh, a.hd / CB_DIMS), dim3(CB_WG), 0, st, am);
    return hipGetLastError();
}

}  // namespace styx
