// router.h -- the ffn RMSNorm's sum of squares and the router dots of one
// workgroup of 256 threads over its RT_ROWS router rows (rms_norm_f32 then
// matvec_strided_f32, crates/model/src/moe.rs:1974-1996), shared by the
// router kernel and the fused MoE block so that both form their logits
// with the same arithmetic.  Thread t holds columns 4 t + 1024 j of x, of the norm weight w
// and of each row.  The RMSNorm scale s is applied after the dot:
// logit_r = s * sum_c W_r[c] (x[c] w[c]), so that the dots need not wait for
// the sum of squares (the reference forms (x[c] s) w[c] first; the two
// differ by rounding only).  One workgroup barrier, the caller's, sits
// between router_wave_part and the reads of the totals.
#pragma once

#include "qdot.h"

namespace styx {

constexpr int RT_ROWS = 4;    // most router rows per workgroup
constexpr int RT_RED = 4 + 4 * RT_ROWS;  // floats of LDS for the wave parts

// One float4 of columns into the thread's parts: ss += x^2, p[r] += W_r .
// (x * w) for the workgroup's first nrows (<= RT_ROWS) rows.  Returns x * w.
__device__ __forceinline__ float4 router_acc(const float4 &x, const float4 &n,
                                             const float4 (&wr)[RT_ROWS], int nrows, float &ss,
                                             float (&p)[RT_ROWS])
{
    const float4 xw = make_float4(x.x * n.x, x.y * n.y, x.z * n.z, x.w * n.w);
    ss += x.x * x.x + x.y * x.y + x.z * x.z + x.w * x.w;
#pragma unroll
    for (int r = 0; r < RT_ROWS; r++)
        if (r < nrows) p[r] += wr[r].x * xw.x + wr[r].y * xw.y + wr[r].z * xw.z + wr[r].w * xw.w;
    return xw;
}

// Wave sums of the parts, written by lane 0 of each of the 4 waves to red
// (RT_RED floats); the caller's barrier follows.
__device__ __forceinline__ void router_wave_part(float ss, float (&p)[RT_ROWS], int nrows, float *red)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    ss = wave_sum(ss);
#pragma unroll
    for (int r = 0; r < RT_ROWS; r++)
        if (r < nrows) p[r] = wave_sum(p[r]);
    if (lane == 0) {
        red[wave] = ss;
#pragma unroll
        for (int r = 0; r < RT_ROWS; r++)
            if (r < nrows) red[4 + 4 * r + wave] = p[r];
    }
}

// After the barrier: the RMSNorm scale 1 / sqrt(sum x^2 / H + eps) (the
// four waves' sums in order) and the dot of row r (likewise).
__device__ __forceinline__ float router_scale(const float *red, int H, float eps)
{
    const float ss = ((red[0] + red[1]) + red[2]) + red[3];
    return 1.0f / sqrtf(ss / (float)H + eps);
}
__device__ __forceinline__ float router_dot(const float *red, int r)
{
    const float *q = red + 4 + 4 * r;
    return ((q[0] + q[1]) + q[2]) + q[3];
}

}  // namespace styx
