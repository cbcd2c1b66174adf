// topk.h -- top-k softmax routing on one wave64 (topk_softmax_f32 semantics).
#pragma once

#include "kernels.h"
#include "qdot.h"

namespace styx {

// --------------------------------------------------------- top-k softmax --
// topk_softmax_f32.comp:29-67 on one wave64: softmax max/sum, then k rounds
// of argmax over untaken entries (ties -> lowest index), weights
// exp(best-mx)/sum, renormalised by their sum if renorm.  Id rows:
// [0,k) original, [16,..) hot, [32,..) arena, [48,..) host.
// remap == nullptr means every expert is resident at its own index.
__device__ __noinline__ void topk_wave(const float *logits, int n, int k, int renorm,
                                 const uint32_t *remap, const uint32_t *pmap, int arena_mode,
                                 int layer, float *wts, int32_t *ids)
{
    const int lane = threadIdx.x & 63;
    float v[MAX_EXPERTS / 64];
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < MAX_EXPERTS / 64; j++) {
        const int i = lane + 64 * j;
        v[j] = i < n ? logits[i] : -INFINITY;
        mx = fmaxf(mx, v[j]);
    }
    mx = wave_max(mx);
    float sum = 0.0f;
#pragma unroll
    for (int j = 0; j < MAX_EXPERTS / 64; j++)
        if (lane + 64 * j < n) sum += expf(v[j] - mx);
    sum = wave_sum(sum);

    uint32_t taken = 0;
    float my_w = 0.0f, wsum = 0.0f;
    int my_id = -1;
    for (int s = 0; s < k; s++) {
        float best = -INFINITY;
        int bi = 0x7FFFFFFF;
#pragma unroll
        for (int j = 0; j < MAX_EXPERTS / 64; j++) {
            const int i = lane + 64 * j;
            if (i < n && !((taken >> j) & 1u) && v[j] > best) {
                best = v[j];
                bi = i;
            }
        }
        for (int o = 32; o > 0; o >>= 1) {
            const float ob = __shfl_xor(best, o);
            const int oi = __shfl_xor(bi, o);
            if (ob > best || (ob == best && oi < bi)) {
                best = ob;
                bi = oi;
            }
        }
        if (bi != 0x7FFFFFFF && lane == (bi & 63)) taken |= 1u << (bi >> 6);
        const float w = expf(best - mx) / sum;
        wsum += w;
        if (lane == s) {
            my_w = w;
            my_id = bi;
        }
    }
    if (lane < k) {
        wts[lane] = renorm ? my_w / wsum : my_w;
        const uint32_t e = (uint32_t)my_id;
        ids[lane] = my_id;
        const uint32_t h = remap ? remap[e] : e;
        if (h != SKIP) {
            ids[16 + lane] = (int32_t)h;
            ids[32 + lane] = (int32_t)SKIP;
            ids[48 + lane] = (int32_t)SKIP;
        } else {
            uint32_t a = SKIP;
            if (arena_mode)
                a = (uint32_t)(layer * k + lane);
            else if (pmap)
                a = pmap[e];
            ids[16 + lane] = (int32_t)SKIP;
            ids[32 + lane] = (int32_t)a;
            ids[48 + lane] = a != SKIP ? (int32_t)SKIP : my_id;
        }
    }
}

// Hot / arena / host ids of expert e routed to `slot` (topk_softmax_f32.comp
// id rows 16/32/48): the hot slot from remap (every expert resident at its
// own index when remap is null), else an arena slot (arena_mode: layer*k +
// slot, or pmap), else the expert itself read from host memory.
__device__ __forceinline__ void route_row(const Route &r, int e, int slot, uint32_t ids3[3])
{
    const uint32_t h = r.remap ? *(const uint32_t STYX_GLOBAL *)(r.remap + e) : (uint32_t)e;
    ids3[0] = h;
    ids3[1] = ids3[2] = SKIP;
    if (h != SKIP) return;
    uint32_t a = SKIP;
    if (r.arena_mode)
        a = (uint32_t)(r.layer * r.k + slot);
    else if (r.pmap)
        a = *(const uint32_t STYX_GLOBAL *)(r.pmap + e);
    ids3[1] = a;
    if (a == SKIP) ids3[2] = (uint32_t)e;
}

// Rank key of logit v at index e: larger key = earlier in the reference's
// selection order (larger value first, equal values by lower index -- the
// strict '>' of topk_softmax_f32.comp:45).  High word: the f32 bits mapped
// to an order-preserving unsigned integer (-0 taken as +0, which compares
// equal to it); low word: ~e.  Every key of a real logit is non-zero.
__device__ __forceinline__ uint64_t rank_key(float v, int e)
{
    uint32_t u = __float_as_uint(v == 0.0f ? 0.0f : v);
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((uint64_t)u << 32) | (uint32_t)(0xFFFFFFFFu - (uint32_t)e);
}

template <int CTRL> __device__ __forceinline__ uint32_t dpp_u(uint32_t v)
{
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, true);
}
__device__ __forceinline__ uint64_t join64(uint32_t hi, uint32_t lo) { return ((uint64_t)hi << 32) | lo; }

// Maximum of a 32-bit value over the wave, every lane getting it: a
// butterfly of DPP moves within rows, then lane swaps across rows.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v)
{
    v = max(v, dpp_u<0xB1>(v));
    v = max(v, dpp_u<0x4E>(v));
    v = max(v, dpp_u<0x141>(v));
    v = max(v, dpp_u<0x140>(v));
    {
        const auto s = __builtin_amdgcn_permlane16_swap(v, v, false, false);
        v = max(s[0], s[1]);
    }
    {
        const auto s = __builtin_amdgcn_permlane32_swap(v, v, false, false);
        v = max(s[0], s[1]);
    }
    return v;
}

// Maximum of a 64-bit rank key over the wave, every lane getting it: the
// maximum of the high halves (the logit's order bits), then the low half
// (the expert) of the one lane holding it -- or, when several lanes hold
// that high half (equal logits), the maximum of their low halves.
__device__ __forceinline__ uint64_t wave_max_key(uint64_t v)
{
    const uint32_t hi = (uint32_t)(v >> 32);
    const uint32_t mh = wave_max_u32(hi);
    const uint64_t ball = __ballot(hi == mh);
    uint32_t ml;
    if ((ball & (ball - 1)) == 0)
        ml = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, (int)__builtin_ctzll(ball));
    else
        ml = wave_max_u32(hi == mh ? (uint32_t)v : 0u);
    return join64(mh, ml);
}

// Stage 1 of the two-stage ranking for one wave: the Q keys of its quarter
// (q[0..Q), in LDS, Q a power of two <= 32) ranked among themselves, P =
// min(64 / Q, Q / 2) lanes per key; a key of quarter rank below k goes to
// cand[rank] (cand: this wave's k candidate slots, zeroed by the caller).
__device__ __forceinline__ void rank_quarter(const uint64_t *q, int Q, int k, uint64_t *cand)
{
    const int lane = threadIdx.x & 63;
    const int P = min(64 / Q, Q / 2), span = Q / P;  // span >= 2, even
    const int e = lane / P, part = lane - e * P;
    int cnt = 0;
    uint64_t mk = 0;
    if (e < Q) {
        mk = q[e];
        const ulonglong2 *qq = (const ulonglong2 *)(q + part * span);
        for (int j2 = 0; j2 < span / 2; j2++) {
            const ulonglong2 u = qq[j2];
            cnt += (int)(u.x > mk) + (int)(u.y > mk);
        }
    }
    for (int sh = 1; sh < P; sh <<= 1) cnt += __shfl_xor(cnt, sh);
    if (e < Q && part == 0 && cnt < k) cand[cnt] = mk;
}

// Stage 2: the 4k candidate slots (unused ones hold key 0) ranked among
// themselves by the workgroup's first 4k threads; ranks below k give
// s_ids.  A key of the global top k has fewer than k larger keys in its
// quarter, so it is a candidate, and every key larger than it is a
// candidate too: its rank among the candidates is its rank.
__device__ __forceinline__ void rank_candidates(const uint64_t *c_key, int k, int32_t *s_ids)
{
    const int tid = threadIdx.x;
    if (tid < 4 * k) {
        const uint64_t ck = c_key[tid];
        int c2 = 0;
        const ulonglong2 *q = (const ulonglong2 *)c_key;
        for (int j2 = 0; j2 < 2 * k; j2++) {
            const ulonglong2 u = q[j2];
            c2 += (int)(u.x > ck) + (int)(u.y > ck);
        }
        if (ck != 0 && c2 < k) s_ids[c2] = (int32_t)(0xFFFFFFFFu - (uint32_t)ck);
    }
}

// The two stages with the quarter Q (a power of two <= 32) and k <= 8 known
// at compile time: every LDS read of a thread's compares is issued before
// the first compare (in the loops above each read waited in turn), and the
// P lanes of a key sum their counts with DPP quad permutes.  Same compares,
// same results.
template <int Q>
__device__ __forceinline__ void rank_quarter_q(const uint64_t *q, int k, uint64_t *cand)
{
    constexpr int P = (64 / Q < Q / 2) ? 64 / Q : Q / 2, SPAN = Q / P;
    static_assert(P >= 2 && P <= 4 && SPAN % 2 == 0, "quarter geometry");
    const int lane = threadIdx.x & 63;
    const int e = lane / P, part = lane - e * P;
    int cnt = 0;
    uint64_t mk = 0;
    if (e < Q) {
        mk = q[e];
        const ulonglong2 *qq = (const ulonglong2 *)(q + part * SPAN);
        ulonglong2 u[SPAN / 2];
#pragma unroll
        for (int j2 = 0; j2 < SPAN / 2; j2++) u[j2] = qq[j2];
#pragma unroll
        for (int j2 = 0; j2 < SPAN / 2; j2++) cnt += (int)(u[j2].x > mk) + (int)(u[j2].y > mk);
    }
    cnt += (int)dpp_u<0xB1>((uint32_t)cnt);  // lane ^ 1
    if constexpr (P == 4) cnt += (int)dpp_u<0x4E>((uint32_t)cnt);  // lane ^ 2
    if (e < Q && part == 0 && cnt < k) cand[cnt] = mk;
}
template <int K>
__device__ __forceinline__ void rank_candidates_k(const uint64_t *c_key, int32_t *s_ids)
{
    const int tid = threadIdx.x;
    if (tid < 4 * K) {
        const uint64_t ck = c_key[tid];
        ulonglong2 u[2 * K];
#pragma unroll
        for (int j2 = 0; j2 < 2 * K; j2++) u[j2] = ((const ulonglong2 *)c_key)[j2];
        int c2 = 0;
#pragma unroll
        for (int j2 = 0; j2 < 2 * K; j2++) c2 += (int)(u[j2].x > ck) + (int)(u[j2].y > ck);
        if (ck != 0 && c2 < K) s_ids[c2] = (int32_t)(0xFFFFFFFFu - (uint32_t)ck);
    }
}
__device__ __forceinline__ void rank_quarter_any(const uint64_t *q, int Q, int k, uint64_t *cand)
{
    switch (Q) {
    case 32: rank_quarter_q<32>(q, k, cand); break;
    case 16: rank_quarter_q<16>(q, k, cand); break;
    case 8: rank_quarter_q<8>(q, k, cand); break;
    case 4: rank_quarter_q<4>(q, k, cand); break;
    default: rank_quarter(q, Q, k, cand); break;
    }
}
__device__ __forceinline__ void rank_candidates_any(const uint64_t *c_key, int k, int32_t *s_ids)
{
    switch (k) {
    case 1: rank_candidates_k<1>(c_key, s_ids); break;
    case 2: rank_candidates_k<2>(c_key, s_ids); break;
    case 3: rank_candidates_k<3>(c_key, s_ids); break;
    case 4: rank_candidates_k<4>(c_key, s_ids); break;
    case 5: rank_candidates_k<5>(c_key, s_ids); break;
    case 6: rank_candidates_k<6>(c_key, s_ids); break;
    case 7: rank_candidates_k<7>(c_key, s_ids); break;
    case 8: rank_candidates_k<8>(c_key, s_ids); break;
    default: rank_candidates(c_key, k, s_ids); break;
    }
}

// The whole 64-int id row of the routed slots s_ids[0..k) to r.ids_out
// (orig | hot | arena | host, topk_softmax_f32.comp:4-17) by threads < 64.
__device__ __forceinline__ void publish_id_row(const Route &r, const int32_t *s_ids)
{
    const int tid = threadIdx.x;
    if (!r.ids_out || tid >= IDS_ROW) return;
    const int row = tid >> 4, slot = tid & 15;
    int32_t v = (int32_t)SKIP;
    if (slot < r.k) {
        const int e = s_ids[slot];
        if (row == 0) {
            v = e;
        } else {
            uint32_t ids3[3];
            route_row(r, e, slot, ids3);
            v = (int32_t)ids3[row - 1];
        }
    }
    *(int32_t STYX_GLOBAL *)(r.ids_out + tid) = v;
}

// Top-k ids of the router logits inside a workgroup, by ranking: the rank
// of a key is the number of larger keys, and ranks 0..k-1 are exactly the
// reference's selection order (keys of rank_key: larger value first, equal
// values by lower index).  Up to 128 experts (a power-of-two quarter) each
// wave ranks the keys of its quarter among themselves and keeps the top k as
// candidates, which are then ranked among themselves (16x fewer compares
// than ranking every key against all, the cost of which was VALU-bound);
// other counts up to 128 rank every key against all.  Above 128 each
// wave takes a quarter of the experts (at most two keys per lane) and draws
// its quarter's top min(k, E/4) keys one at a time -- the wave's largest key
// (wave_max_key), which its owner then drops -- and, every global top-k key
// being in its quarter's top k, the <= 4k candidates are ranked among
// themselves.  Integer compares only.
// Fills s_ids[0..k) with the routed experts (route_row gives a slot's other
// ids); weights are left to the caller.  The logits are in LDS (s_lg,
// filled by the caller; the ranking synchronises before reading them);
// the workgroup given `publish` writes the whole id row to r.ids_out.
// Needs blockDim.x == 256, E % 16 == 0, E <= 512, k <= 16.
__device__ inline const int32_t *rank_ids_lds(const Route &r, int32_t *s_ids, const float *s_lg,
                                              bool publish)
{
    __shared__ __align__(16) uint64_t s_key[128];
    __shared__ __align__(16) uint64_t c_key[4 * MAX_TOPK];
    const int E = r.E, k = r.k, Q = E / 4;  // quarter: Q % 4 == 0, Q <= 128
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, q0 = wave * Q;
    if (tid < IDS_ROW) s_ids[tid] = (int32_t)SKIP;
    if (tid < 4 * MAX_TOPK) c_key[tid] = 0;
    __syncthreads();  // also: the caller's logits are in s_lg
    if (E <= 128 && (Q & (Q - 1)) == 0) {
        // two stages: every wave ranks the keys of its quarter, then the
        // candidates are ranked among themselves
        for (int e = tid; e < E; e += 256) s_key[e] = rank_key(s_lg[e], e);
        __syncthreads();
        rank_quarter_any(s_key + q0, Q, k, c_key + wave * k);
        __syncthreads();
        rank_candidates_any(c_key, k, s_ids);
    } else if (E <= 128) {
        // direct: P = 256 / E threads rank each key against a slice of all
        for (int e = tid; e < E; e += 256) s_key[e] = rank_key(s_lg[e], e);
        __syncthreads();
        const int P = E <= 64 ? 4 : 2, span = E / P;
        const int e = tid / P, part = tid % P;
        int cnt = 0;
        if (e < E) {
            const uint64_t mk = s_key[e];
            const ulonglong2 *q = (const ulonglong2 *)(s_key + part * span);
#pragma unroll 8
            for (int j2 = 0; j2 < span / 2; j2++) {
                const ulonglong2 u = q[j2];
                cnt += (int)(u.x > mk) + (int)(u.y > mk);
            }
        }
        cnt += __shfl_xor(cnt, 1);
        if (P == 4) cnt += __shfl_xor(cnt, 2);
        if (e < E && part == 0 && cnt < k) s_ids[cnt] = e;
    } else {
        uint64_t k0 = lane < Q ? rank_key(s_lg[q0 + lane], q0 + lane) : 0;
        uint64_t k1 = lane + 64 < Q ? rank_key(s_lg[q0 + lane + 64], q0 + lane + 64) : 0;
        if (k1 > k0) {
            const uint64_t t = k0;
            k0 = k1;
            k1 = t;
        }
        const int kk = min(k, Q);
        for (int it = 0; it < kk; it++) {
            const uint64_t m = wave_max_key(k0);
            if (lane == 0) c_key[wave * k + it] = m;
            if (k0 == m) {  // keys are distinct: one lane
                k0 = k1;
                k1 = 0;
            }
        }
        __syncthreads();
        if (tid < 4 * MAX_TOPK) {
            // every candidate slot (unused ones hold key 0) against all 64
            const uint64_t mk = c_key[tid];
            int cnt = 0;
#pragma unroll
            for (int j2 = 0; j2 < 2 * MAX_TOPK; j2++) {
                const ulonglong2 u = ((const ulonglong2 *)c_key)[j2];
                cnt += (int)(u.x > mk) + (int)(u.y > mk);
            }
            if (mk != 0 && cnt < k) s_ids[cnt] = (int32_t)(0xFFFFFFFFu - (uint32_t)mk);
        }
    }
    __syncthreads();
    if (publish) publish_id_row(r, s_ids);
    return s_ids;
}

// Logits from global memory, then rank_ids_lds; the workgroup with all-zero
// block index publishes the 64-int id row.
__device__ inline const int32_t *route_ids_wg(const Route &r, int32_t *s_ids, float *s_lg)
{
    for (int e = threadIdx.x; e < r.E / 4; e += 256)  // blockDim.x == 256
        ((float4 *)s_lg)[e] = ((const float4 *)r.logits)[e];
    return rank_ids_lds(r, s_ids, s_lg, blockIdx.x == 0 && blockIdx.y == 0 && blockIdx.z == 0);
}

}  // namespace styx
