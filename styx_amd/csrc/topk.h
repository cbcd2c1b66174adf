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

// Top-k of the router logits computed inside a workgroup (wave 0) into LDS;
// the workgroup with all-zero block index also publishes the weights and the
// id row to global memory for the kernels that follow.
__device__ inline const int32_t *route_in_lds(const Route &r, int32_t *s_ids, float *s_w)
{
    if (threadIdx.x < 64) {
        s_ids[threadIdx.x] = (int32_t)SKIP;
        topk_wave(r.logits, r.E, r.k, r.renorm, r.remap, r.pmap, r.arena_mode, r.layer, s_w,
                  s_ids);
    }
    __syncthreads();
    if (blockIdx.x == 0 && blockIdx.y == 0 && blockIdx.z == 0 && threadIdx.x < 64) {
        if (r.ids_out) r.ids_out[threadIdx.x] = s_ids[threadIdx.x];
        if (r.wts_out && threadIdx.x < r.k) r.wts_out[threadIdx.x] = s_w[threadIdx.x];
    }
    return s_ids;
}

}  // namespace styx
