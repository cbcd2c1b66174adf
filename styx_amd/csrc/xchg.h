// xchg.h -- data exchange between the workgroups of one launch, without
// fences.  A value travels as a 64-bit word (launch tag << 32 | f32 bits),
// written and read with relaxed agent-scope atomics: on gfx950 these are
// plain global stores / loads with device scope (sc1), coherent across the
// XCDs' L2s, and a word is valid once it carries the reader's launch tag.
// The tag comes from a ticket every workgroup of the launch draws from one
// of ntk counters (128 bytes apart, so the draws do not queue on one
// address): counter i is drawn nwg / ntk times per launch, so
// ticket / (nwg / ntk) + 1 numbers the launch -- also when a captured graph
// replays the same launch.  Buffers start zeroed (tag 0 is never a
// launch's) and are never cleared again.
#pragma once

#include "common.h"

namespace styx {

// Global loads and stores through pointers that did not come from kernel
// arguments (a generic pointer would become a flat access, which also
// counts against the LDS wait counter).
__device__ __forceinline__ float gld(const float *p) { return *(const float STYX_GLOBAL *)p; }
__device__ __forceinline__ float4 gld4(const float *p)
{
    const styx_f4 v = *(const styx_f4 STYX_GLOBAL *)p;
    return make_float4(v.x, v.y, v.z, v.w);
}
template <typename T> __device__ __forceinline__ void gst(T *p, T v) { *(T STYX_GLOBAL *)p = v; }

__device__ __forceinline__ void tput(uint64_t *p, uint32_t tag, float v)
{
    __hip_atomic_store((uint64_t STYX_GLOBAL *)p, ((uint64_t)tag << 32) | __float_as_uint(v),
                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ uint64_t tget(const uint64_t *p)
{
    return __hip_atomic_load((uint64_t STYX_GLOBAL *)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ bool tvalid(uint64_t w, uint32_t tag) { return (uint32_t)(w >> 32) == tag; }
__device__ __forceinline__ float tval(uint64_t w) { return __uint_as_float((uint32_t)w); }

// Ticket of workgroup `wid` (ntk divides the launch's workgroup count).
__device__ __forceinline__ unsigned long long draw_ticket(unsigned long long *tickets, int ntk,
                                                          int wid)
{
    return __hip_atomic_fetch_add((unsigned long long STYX_GLOBAL *)(tickets + (wid % ntk) * 16),
                                  1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ uint32_t ticket_tag(unsigned long long t, int nwg, int ntk)
{
    return (uint32_t)(t / (unsigned long long)(nwg / ntk)) + 1u;
}

// The abort flag of bounded waits: set by a workgroup that gave up waiting,
// read by the others (and by the host after the launch).
__device__ __forceinline__ bool abort_seen(int *abort)
{
    return __hip_atomic_load((int STYX_GLOBAL *)abort, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0;
}
__device__ __forceinline__ void abort_raise(int *abort)
{
    __hip_atomic_store((int STYX_GLOBAL *)abort, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Wait until the n tagged words addr(0..n) carry `tag` and copy their values
// to dst[0..n) (LDS); addr(i) may return null for a word that is not needed
// (dst[i] = 0).  Thread t takes words t + blockDim.x j, j < MAXJ
// (n <= MAXJ * blockDim.x).  Each wave polls its own words until they are
// all in, with no workgroup barrier between rounds; one barrier at the end
// (workgroup-uniform call).  The wait is bounded: after max_polls rounds, or
// once another workgroup has raised the abort flag, the workgroup raises
// the flag and returns false.
// NT: the workgroup's thread count when known at compile time (0: read
// blockDim.x).
template <int MAXJ, int NT = 0, typename Addr>
__device__ __forceinline__ bool tpoll_wg(int n, Addr addr, uint32_t tag, float *dst, int max_polls,
                                         int *abort)
{
    const int nt = NT ? NT : (int)blockDim.x;
    uint32_t pend = 0;
#pragma unroll
    for (int j = 0; j < MAXJ; j++) {
        const int i = (int)threadIdx.x + nt * j;
        if (i < n) {
            if (addr(i))
                pend |= 1u << j;
            else
                dst[i] = 0.0f;
        }
    }
    int failed = 0;
    for (int polls = 0; __any(pend != 0); polls++) {
        uint64_t v[MAXJ];
#pragma unroll
        for (int j = 0; j < MAXJ; j++)
            v[j] = ((pend >> j) & 1u) ? tget(addr((int)threadIdx.x + nt * j)) : 0ull;
#pragma unroll
        for (int j = 0; j < MAXJ; j++) {
            if (((pend >> j) & 1u) && (uint32_t)(v[j] >> 32) == tag) {
                dst[threadIdx.x + nt * j] = __uint_as_float((uint32_t)v[j]);
                pend &= ~(1u << j);
            }
        }
        if (!__any(pend != 0)) break;
        // the bound every round, another workgroup's abort every 32nd (a
        // memory round trip of its own)
        if (polls >= max_polls || ((polls & 31) == 31 && __any(abort_seen(abort)))) {
            failed = 1;
            break;
        }
        __builtin_amdgcn_s_sleep(1);
    }
    // the workgroup's verdict from one flag per wave (failed is uniform in
    // a wave) in LDS; __syncthreads_or would read the wave count from the
    // dispatch packet, and that load's wait also waits for every store in
    // flight
    __shared__ int s_fail[16];
    if ((threadIdx.x & 63) == 0) s_fail[threadIdx.x >> 6] = failed;
    __syncthreads();
    int any = 0;
    for (int w = 0; w < nt / 64; w++) any |= s_fail[w];
    __syncthreads();  // read by every wave before a later call rewrites them
    if (any) {
        if (threadIdx.x == 0) abort_raise(abort);
        return false;
    }
    return true;
}

// Limbs of n values (a multiple of 32) built in LDS at ql, elements
// [e0, e0 + n) of an N-value vector (e0 a multiple of 32): copied into the
// plain limb buffer qg of the whole vector and published as tagged words in
// t, laid out as the 32-bit words of xq_at(., N): A | B | C | sx | s16.
// Threads [0, n / 4) take part.
__device__ __forceinline__ void xq_publish(const Xq &ql, int n, int e0, int N, const Xq &qg,
                                           uint64_t *t, uint32_t tag)
{
    const int tid = threadIdx.x, N4 = N / 4;
    const Xq g = xq_shift(qg, e0);
    if (tid < n / 4) {
        const uint32_t va = ((const uint32_t *)ql.A)[tid], vb = ((const uint32_t *)ql.B)[tid],
                       vc = ((const uint32_t *)ql.C)[tid];
        gst((uint32_t *)g.A + tid, va);
        gst((uint32_t *)g.B + tid, vb);
        gst((uint32_t *)g.C + tid, vc);
        const int o = e0 / 4 + tid;
        tput(t + o, tag, __uint_as_float(va));
        tput(t + N4 + o, tag, __uint_as_float(vb));
        tput(t + 2 * N4 + o, tag, __uint_as_float(vc));
    }
    if (tid < n / 32) {
        gst(g.sx + tid, ql.sx[tid]);
        tput(t + 3 * N4 + e0 / 32 + tid, tag, ql.sx[tid]);
    }
    if (tid < n / 16) {
        gst(g.s16 + tid, ql.s16[tid]);
        tput(t + 3 * N4 + N / 32 + e0 / 16 + tid, tag, ql.s16[tid]);
    }
}

// Number of ticket counters for a launch of nwg workgroups: the largest
// power of two dividing nwg, at most 64.
__host__ __device__ inline int ticket_counters(int nwg)
{
    int n = nwg & -nwg;
    return n > 64 ? 64 : n;
}

}  // namespace styx
