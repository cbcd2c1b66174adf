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

// Top-k ids of the router logits inside a workgroup, by ranking: the rank of
// logit e is the number of logits ordered before it (a larger value, or an
// equal value at a lower index -- the strict '>' of topk_softmax_f32.comp:45),
// so ranks 0..k-1 are exactly the reference's selection order.  Every thread
// ranks one logit against a slice of the others; no dependent shuffle chain.
// Fills the four id rows in s_ids (64 ints); weights are left to the caller.
// The workgroup with all-zero block index publishes the id row to r.ids_out.
__device__ inline const int32_t *route_ids_wg(const Route &r, int32_t *s_ids, float *s_lg)
{
    const int E = r.E, k = r.k;  // E % 16 == 0 (checked at launch)
    for (int e = threadIdx.x; e < E / 4; e += blockDim.x)
        ((float4 *)s_lg)[e] = ((const float4 *)r.logits)[e];
    if (threadIdx.x < IDS_ROW) s_ids[threadIdx.x] = (int32_t)SKIP;
    __syncthreads();
    const int P = E <= 64 ? 4 : E <= 128 ? 2 : 1;  // threads per logit
    const int per = (int)blockDim.x / P, span = E / P;  // span % 4 == 0
    for (int e0 = 0; e0 < E; e0 += per) {
        const int e = e0 + (int)threadIdx.x / P, part = (int)threadIdx.x % P;
        int cnt = 0;
        if (e < E) {
            const float v = s_lg[e];
            const int j0 = part * span;
            const float4 *q = (const float4 *)(s_lg + j0);
#pragma unroll 8
            for (int j4 = 0; j4 < span / 4; j4++) {
                const float4 u = q[j4];
                const int j = j0 + 4 * j4;
                cnt += (u.x > v) || (u.x == v && j < e);
                cnt += (u.y > v) || (u.y == v && j + 1 < e);
                cnt += (u.z > v) || (u.z == v && j + 2 < e);
                cnt += (u.w > v) || (u.w == v && j + 3 < e);
            }
        }
        if (P >= 2) cnt += __shfl_xor(cnt, 1);
        if (P >= 4) cnt += __shfl_xor(cnt, 2);
        if (e < E && part == 0 && cnt < k) s_ids[cnt] = e;
    }
    __syncthreads();
    if ((int)threadIdx.x < k) {
        const int s = threadIdx.x;
        const uint32_t e = (uint32_t)s_ids[s];
        const uint32_t h = r.remap ? r.remap[e] : e;
        if (h != SKIP) {
            s_ids[16 + s] = (int32_t)h;
        } else {
            uint32_t a = SKIP;
            if (r.arena_mode)
                a = (uint32_t)(r.layer * k + s);
            else if (r.pmap)
                a = r.pmap[e];
            s_ids[32 + s] = (int32_t)a;
            if (a == SKIP) s_ids[48 + s] = (int32_t)e;
        }
    }
    __syncthreads();
    if (r.ids_out && blockIdx.x == 0 && blockIdx.y == 0 && blockIdx.z == 0 &&
        threadIdx.x < IDS_ROW)
        r.ids_out[threadIdx.x] = s_ids[threadIdx.x];
    return s_ids;
}

}  // namespace styx
