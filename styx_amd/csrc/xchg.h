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

// Number of ticket counters for a launch of nwg workgroups: the largest
// power of two dividing nwg, at most 64.
__host__ __device__ inline int ticket_counters(int nwg)
{
    int n = nwg & -nwg;
    return n > 64 ? 64 : n;
}

}  // namespace styx
