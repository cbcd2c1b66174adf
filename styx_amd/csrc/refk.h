// refk.h -- ids of the reference-interface kernels (kernels_ref.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

struct styx_gpu;

namespace styx {

enum RefKernel {
    RK_TOPK = 1,
    RK_MOE_REDUCE,
    RK_GATHER,
    RK_ATTN,
    RK_MATVEC_STRIDED,
    RK_ADD,
    RK_AXPY_SIG,
    RK_SWIGLU,
    RK_RMS_NORM,
    RK_ROPE_NEOX,
    RK_CPY,
    RK_MMV_BASE = 32,  // +0..3 mul_mat_vec_{q8_0,q4_k,q5_k,q6_k}, +4..7 the _id forms
    // fused hot-path kernels (dispatch_fused.cpp); +0..3: q8_0, q4_k, q5_k, q6_k
    RK_F_ROUTER_TOPK = 64,
    RK_F_GATE_UP_SILU = 68,
    RK_F_DOWN_REDUCE = 72,
    RK_F_ATTN_PAGED = 76,
};

// Launch reference kernel `kid` with resolved binding pointers and the bytes
// each binding makes visible, the raw push-constant block, the reference
// grid and spec constants (id, value pairs).  Returns hipErrorInvalidValue,
// launching nothing, when the push constants and grid would reach past a
// binding; ids read from device memory that name a matrix or slab past its
// binding are treated as SKIP by the kernels.
hipError_t refk_launch(hipStream_t st, int kid, void *const *ptr, const uint64_t *size,
                       const void *push, uint32_t gx, uint32_t gy, uint32_t gz,
                       const uint32_t *spec, int n_spec);

// Launch fused kernel `kid` (RK_F_*) of a batch on gpu g: the push block of
// include/styx_hip.h, bindings resolved as for refk_launch.  Returns
// hipErrorInvalidValue, launching nothing, when a shape or extent does not
// fit the bindings.
hipError_t fused_launch(styx_gpu *g, hipStream_t st, int kid, void *const *ptr,
                        const uint64_t *size, const void *push);

}  // namespace styx
