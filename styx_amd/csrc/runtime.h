// runtime.h -- host-side objects behind the C ABI handles.
#pragma once

#include <hip/hip_runtime.h>

#include <string>

#include "../../include/styx_hip.h"

struct styx_gpu {
    int device = 0;
    hipStream_t stream = nullptr;
    std::string name;
    uint64_t hbm = 0;
    int live_children = 0;
    bool closed = false;  // styx_gpu_free called while children were alive
    // Activation limbs of the op entry points that take an f32 vector
    // (matvec, gate/up): built into this buffer in stream order right before
    // the matvec that reads them.  Calls on one styx_gpu are serialised on
    // its stream, so one buffer serves them all.
    void *xq_scratch = nullptr;
    // Per-slot down rows of styx_op_moe_down_reduce (k x H floats, k <= 16,
    // H <= 16384), same stream-order rule.
    void *partial_scratch = nullptr;
    size_t partial_bytes = 0;
    // Device address of this device's copy of the static attention-partials
    // array of styx_op_attn_decode_noalloc (capi.cpp), looked up at
    // styx_gpu_new with the device current.
    float *noalloc_part = nullptr;
    // Device scalars of the fused dispatch kernels: [0] the position of an
    // attn_decode_paged dispatch (written in stream order by a fill kernel),
    // [1] = 0, the one-entry page table of a contiguous KV cache.
    int32_t *fused_scalars = nullptr;
    // attn_decode_paged's copy of a caller's page table, its entries clamped
    // to the pool (FUSED_PT_MAX entries): the kernel then reads nothing
    // outside the pools whatever the table holds.
    static constexpr int FUSED_PT_MAX = 65536;
    uint32_t *fused_pt = nullptr;
};

struct styx_buf {
    styx_gpu *gpu = nullptr;
    void *ptr = nullptr;  // device-visible address
    void *host = nullptr; // host address of a pinned buffer
    uint64_t size = 0;
    int kind = STYX_BUF_DEVICE;
};

namespace styx {

// Thread-local error message helpers.  fail() records the message and
// returns the status so callers can `return fail(...)`.
int fail(int status, const std::string &msg);
int hip_fail(hipError_t e, const char *what);
void clear_error();
// Drop one child of gpu; deletes the gpu if it was closed and this was the last.
void gpu_release(styx_gpu *gpu);

#define STYX_HIP(call)                                      \
    do {                                                    \
        hipError_t _e = (call);                             \
        if (_e != hipSuccess) return ::styx::hip_fail(_e, #call); \
    } while (0)

}  // namespace styx
