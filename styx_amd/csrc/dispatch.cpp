// dispatch.cpp -- pipelines by name and command batches: the
// Gpu::create_pipeline / Batch surface of crates/vk-backend/src/lib.rs
// (44-231, 1222-1312) over one HIP stream.  A batch records dispatches
// (kernel, resolved bindings, push bytes, grid) and runs them in order on
// submit, then waits -- the reference's submit + fence.
#include <algorithm>
#include <cstring>
#include <string>
#include <mutex>
#include <vector>

#include "refk.h"
#include "runtime.h"

using namespace styx;

struct styx_kernel {
    styx_gpu *gpu = nullptr;
    int kid = 0;
    int n_bindings = 0;
    uint32_t push_bytes = 0;
    std::vector<uint32_t> spec;  // (id, value) pairs
    std::string name;
};

struct styx_batch {
    styx_gpu *gpu = nullptr;
    bool recording = false;
    // An async batch (Gpu::create_async_batch) runs on a stream of its own
    // (the async queue); `done` marks the end of its last submit, which
    // wait_idle waits for.
    hipStream_t own = nullptr;
    hipEvent_t done = nullptr;
    bool pending = false;
    struct Cmd {
        const styx_kernel *k;
        std::vector<void *> ptr;
        std::vector<uint64_t> size;  // bytes each binding makes visible
        std::vector<uint8_t> push;
        uint32_t gx, gy, gz;
    };
    std::vector<Cmd> cmds;
};

namespace {

struct KDef {
    const char *name;
    int kid;
    int n_bindings;
    uint32_t push_bytes;
};

// binding counts and push sizes as created at crates/model/src/moe.rs:644-690
const KDef kdefs[] = {
    {"topk_softmax_f32", RK_TOPK, 5, 12},
    {"moe_reduce_f32", RK_MOE_REDUCE, 3, 8},
    {"gather_slabs_f32", RK_GATHER, 7, 36},
    {"attn_decode_f32", RK_ATTN, 4, 20},
    {"matvec_strided_f32", RK_MATVEC_STRIDED, 3, 8},
    {"add_flat_f32", RK_ADD, 3, 4},
    {"axpy_sig_f32", RK_AXPY_SIG, 3, 4},
    {"swiglu_f32", RK_SWIGLU, 3, 108},
    {"rms_norm_f32", RK_RMS_NORM, 3, 116},
    {"rope_neox_f32", RK_ROPE_NEOX, 5, 116},
    {"cpy_f32_f32", RK_CPY, 2, 120},
    {"mul_mat_vec_q8_0_f32_f32", RK_MMV_BASE + 0, 5, 52},
    {"mul_mat_vec_q4_k_f32_f32", RK_MMV_BASE + 1, 5, 52},
    {"mul_mat_vec_q5_k_f32_f32", RK_MMV_BASE + 2, 5, 52},
    {"mul_mat_vec_q6_k_f32_f32", RK_MMV_BASE + 3, 5, 52},
    {"mul_mat_vec_id_q8_0_f32_f32", RK_MMV_BASE + 4, 6, 48},
    {"mul_mat_vec_id_q4_k_f32_f32", RK_MMV_BASE + 5, 6, 48},
    {"mul_mat_vec_id_q5_k_f32_f32", RK_MMV_BASE + 6, 6, 48},
    {"mul_mat_vec_id_q6_k_f32_f32", RK_MMV_BASE + 7, 6, 48},
    // fused hot-path kernels: bindings and push blocks of include/styx_hip.h
    {"router_topk", RK_F_ROUTER_TOPK, 10, sizeof(styx_push_router_topk)},
    {"moe_gate_up_silu_q8_0", RK_F_GATE_UP_SILU + 0, 5, sizeof(styx_push_moe_gate_up_silu)},
    {"moe_gate_up_silu_q4_k", RK_F_GATE_UP_SILU + 1, 5, sizeof(styx_push_moe_gate_up_silu)},
    {"moe_gate_up_silu_q5_k", RK_F_GATE_UP_SILU + 2, 5, sizeof(styx_push_moe_gate_up_silu)},
    {"moe_gate_up_silu_q6_k", RK_F_GATE_UP_SILU + 3, 5, sizeof(styx_push_moe_gate_up_silu)},
    {"moe_down_reduce_q8_0", RK_F_DOWN_REDUCE + 0, 5, sizeof(styx_push_moe_down_reduce)},
    {"moe_down_reduce_q4_k", RK_F_DOWN_REDUCE + 1, 5, sizeof(styx_push_moe_down_reduce)},
    {"moe_down_reduce_q5_k", RK_F_DOWN_REDUCE + 2, 5, sizeof(styx_push_moe_down_reduce)},
    {"moe_down_reduce_q6_k", RK_F_DOWN_REDUCE + 3, 5, sizeof(styx_push_moe_down_reduce)},
    {"attn_decode_paged", RK_F_ATTN_PAGED, 11, sizeof(styx_push_attn_decode_paged)},
};

}  // namespace

// Timeline semaphore (Gpu::create_timeline_semaphore, lib.rs:700-713): each
// signal of value v is an event recorded on the signalling stream; a wait
// for v waits for the first recorded signal of a value >= v.
struct styx_timeline {
    styx_gpu *gpu = nullptr;
    std::mutex mu;
    std::vector<std::pair<uint64_t, hipEvent_t>> sig;  // values ascending
    uint64_t reached = 0;  // largest value whose signal has completed
};

namespace {

// The recorded work of b, launched in order on stream st.
int run_cmds(styx_batch *b, hipStream_t st)
{
    for (auto &c : b->cmds) {
        const uint32_t *spec = c.k->spec.empty() ? nullptr : c.k->spec.data();
        hipError_t e = c.k->kid >= RK_F_ROUTER_TOPK
                           ? fused_launch(b->gpu, st, c.k->kid, c.ptr.data(), c.size.data(),
                                          c.push.data())
                           : refk_launch(st, c.k->kid, c.ptr.data(), c.size.data(), c.push.data(),
                                         c.gx, c.gy, c.gz, spec, (int)c.k->spec.size() / 2);
        if (e == hipErrorInvalidValue)
            return fail(STYX_E_INVALID, c.k->name + ": unsupported parameters, or the push "
                                                    "constants and grid reach past a binding");
        if (e != hipSuccess) return hip_fail(e, c.k->name.c_str());
    }
    b->cmds.clear();
    return STYX_OK;
}

// Completed signals are dropped and `reached` raised to the largest
// completed value (caller holds mu).  Every pending signal is queried:
// signals of async batches on different streams may complete out of
// submission order, and a timeline's value is the largest one reached
// (vkGetSemaphoreCounterValue).
int timeline_poll(styx_timeline *t)
{
    std::vector<std::pair<uint64_t, hipEvent_t>> keep;
    keep.reserve(t->sig.size());
    int r = STYX_OK;
    for (auto &sg : t->sig) {
        const hipError_t e = r ? hipErrorNotReady : hipEventQuery(sg.second);
        if (e == hipErrorNotReady) {
            keep.push_back(sg);
            continue;
        }
        if (e != hipSuccess) {
            r = hip_fail(e, "hipEventQuery");
            keep.push_back(sg);
            continue;
        }
        t->reached = std::max(t->reached, sg.first);
        hipEventDestroy(sg.second);
    }
    t->sig.swap(keep);
    return r;
}

}  // namespace

extern "C" {

const char *styx_kernel_names(void)
{
    static std::string names;
    if (names.empty())
        for (const auto &d : kdefs) {
            if (!names.empty()) names += ",";
            names += d.name;
        }
    return names.c_str();
}

int styx_kernel_get(styx_gpu *gpu, const char *name, const uint32_t *spec, int n_spec,
                    styx_kernel **out)
{
    if (!gpu || !name || !out || n_spec < 0 || (n_spec && !spec))
        return fail(STYX_E_INVALID, "styx_kernel_get: bad argument");
    for (const auto &d : kdefs) {
        if (std::strcmp(d.name, name) != 0) continue;
        styx_kernel *k = new styx_kernel();
        k->gpu = gpu;
        k->kid = d.kid;
        k->n_bindings = d.n_bindings;
        k->push_bytes = d.push_bytes;
        k->spec.assign(spec, spec + 2 * n_spec);
        k->name = name;
        gpu->live_children++;
        *out = k;
        return STYX_OK;
    }
    return fail(STYX_E_UNSUPPORTED, std::string("styx_kernel_get: no kernel named ") + name);
}

void styx_kernel_free(styx_kernel *k)
{
    if (!k) return;
    styx_gpu *g = k->gpu;
    delete k;
    gpu_release(g);
}


int styx_batch_new(styx_gpu *gpu, styx_batch **out)
{
    if (!gpu || !out) return fail(STYX_E_INVALID, "styx_batch_new: bad argument");
    styx_batch *b = new styx_batch();
    b->gpu = gpu;
    gpu->live_children++;
    *out = b;
    return STYX_OK;
}

int styx_batch_new_async(styx_gpu *gpu, styx_batch **out)
{
    if (!gpu || !out) return fail(STYX_E_INVALID, "styx_batch_new_async: bad argument");
    STYX_HIP(hipSetDevice(gpu->device));
    hipStream_t st = nullptr;
    STYX_HIP(hipStreamCreateWithFlags(&st, hipStreamNonBlocking));  // default priority
    hipEvent_t ev = nullptr;
    const hipError_t e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
    if (e != hipSuccess) {
        hipStreamDestroy(st);
        return hip_fail(e, "hipEventCreateWithFlags");
    }
    styx_batch *b = new styx_batch();
    b->gpu = gpu;
    b->own = st;
    b->done = ev;
    gpu->live_children++;
    *out = b;
    return STYX_OK;
}

void styx_batch_free(styx_batch *b)
{
    if (!b) return;
    styx_gpu *g = b->gpu;
    if (b->own) {
        // destroy_async_batch waits on any in-flight submit first
        hipSetDevice(g->device);
        hipStreamSynchronize(b->own);
        hipEventDestroy(b->done);
        hipStreamDestroy(b->own);
    }
    delete b;
    gpu_release(g);
}

int styx_batch_begin(styx_batch *b)
{
    if (!b) return fail(STYX_E_INVALID, "styx_batch_begin: NULL batch");
    if (b->recording) return fail(STYX_E_STATE, "styx_batch_begin: batch already recording");
    b->cmds.clear();
    b->recording = true;
    return STYX_OK;
}

int styx_batch_dispatch(styx_batch *b, const styx_kernel *k, const styx_binding *binds,
                        int n_binds, const void *push, uint32_t push_len, uint32_t gx,
                        uint32_t gy, uint32_t gz, int barrier)
{
    (void)barrier;  // one in-order stream: every dispatch follows the previous one
    if (!b || !k) return fail(STYX_E_INVALID, "styx_batch_dispatch: NULL batch or kernel");
    if (!b->recording) return fail(STYX_E_STATE, "styx_batch_dispatch: batch not begun");
    if (n_binds != k->n_bindings)
        return fail(STYX_E_INVALID, k->name + ": expected " + std::to_string(k->n_bindings) +
                                        " bindings, got " + std::to_string(n_binds));
    if (push_len != k->push_bytes || (push_len && !push))
        return fail(STYX_E_INVALID, k->name + ": push constants must be " +
                                        std::to_string(k->push_bytes) + " bytes");
    if (gx == 0 || gy == 0 || gz == 0) return fail(STYX_E_INVALID, k->name + ": empty grid");
    styx_batch::Cmd c;
    c.k = k;
    for (int i = 0; i < n_binds; i++) {
        const styx_binding &bd = binds[i];
        if (!bd.buf) return fail(STYX_E_INVALID, k->name + ": NULL buffer in binding");
        if (bd.offset % 64 || bd.offset > bd.buf->size)
            return fail(STYX_E_INVALID, k->name + ": binding offset must be 64-byte aligned "
                                                  "and inside the buffer (lib.rs:98-100)");
        c.ptr.push_back((char *)bd.buf->ptr + bd.offset);
        const uint64_t rest = bd.buf->size - bd.offset;
        c.size.push_back(bd.range == UINT64_MAX ? rest : std::min(bd.range, rest));
    }
    c.push.assign((const uint8_t *)push, (const uint8_t *)push + push_len);
    c.gx = gx;
    c.gy = gy;
    c.gz = gz;
    b->cmds.push_back(std::move(c));
    return STYX_OK;
}

int styx_batch_submit(styx_batch *b)
{
    if (!b) return fail(STYX_E_INVALID, "styx_batch_submit: NULL batch");
    if (!b->recording) return fail(STYX_E_STATE, "styx_batch_submit: batch not begun");
    b->recording = false;
    STYX_HIP(hipSetDevice(b->gpu->device));
    hipStream_t st = b->own ? b->own : b->gpu->stream;
    if (int r = run_cmds(b, st)) return r;
    STYX_HIP(hipStreamSynchronize(st));
    return STYX_OK;
}

int styx_dispatch_sync(styx_gpu *gpu, const styx_kernel *k, const styx_binding *binds,
                       int n_binds, const void *push, uint32_t push_len, uint32_t gx, uint32_t gy,
                       uint32_t gz)
{
    if (!gpu || !k) return fail(STYX_E_INVALID, "styx_dispatch_sync: NULL gpu or kernel");
    if (k->gpu != gpu) return fail(STYX_E_INVALID, "styx_dispatch_sync: kernel of another styx_gpu");
    styx_batch b;
    b.gpu = gpu;
    b.recording = true;
    if (int r = styx_batch_dispatch(&b, k, binds, n_binds, push, push_len, gx, gy, gz, 1)) return r;
    return styx_batch_submit(&b);
}

int styx_timeline_new(styx_gpu *gpu, styx_timeline **out)
{
    if (!gpu || !out) return fail(STYX_E_INVALID, "styx_timeline_new: bad argument");
    styx_timeline *t = new styx_timeline();
    t->gpu = gpu;
    gpu->live_children++;
    *out = t;
    return STYX_OK;
}

void styx_timeline_free(styx_timeline *t)
{
    if (!t) return;
    styx_gpu *g = t->gpu;
    hipSetDevice(g->device);
    for (auto &p : t->sig) {
        hipEventSynchronize(p.second);
        hipEventDestroy(p.second);
    }
    delete t;
    gpu_release(g);
}

int styx_timeline_value(styx_timeline *t, uint64_t *value)
{
    if (!t || !value) return fail(STYX_E_INVALID, "styx_timeline_value: bad argument");
    std::lock_guard<std::mutex> lock(t->mu);
    STYX_HIP(hipSetDevice(t->gpu->device));
    if (int r = timeline_poll(t)) return r;
    *value = t->reached;
    return STYX_OK;
}

int styx_batch_submit_async(styx_batch *b, styx_timeline *t, uint64_t value)
{
    if (!b || !t) return fail(STYX_E_INVALID, "styx_batch_submit_async: NULL batch or timeline");
    if (!b->recording) return STYX_OK;  // nothing recorded: nothing to submit (lib.rs:243-245)
    if (!b->own)
        return fail(STYX_E_STATE, "styx_batch_submit_async: batch was not made by "
                                  "styx_batch_new_async");
    if (t->gpu != b->gpu)
        return fail(STYX_E_INVALID, "styx_batch_submit_async: timeline of another styx_gpu");
    std::lock_guard<std::mutex> lock(t->mu);
    const uint64_t last = t->sig.empty() ? t->reached : t->sig.back().first;
    if (value <= last)
        return fail(STYX_E_INVALID, "styx_batch_submit_async: a timeline's signal values must "
                                    "increase (last " + std::to_string(last) + ", got " +
                                        std::to_string(value) + ")");
    b->recording = false;
    STYX_HIP(hipSetDevice(b->gpu->device));
    if (int r = run_cmds(b, b->own)) return r;
    hipEvent_t ev = nullptr;
    STYX_HIP(hipEventCreateWithFlags(&ev, hipEventDisableTiming));
    hipError_t e = hipEventRecord(ev, b->own);
    if (e == hipSuccess) e = hipEventRecord(b->done, b->own);
    if (e != hipSuccess) {
        hipEventDestroy(ev);
        return hip_fail(e, "hipEventRecord");
    }
    t->sig.emplace_back(value, ev);
    b->pending = true;
    return STYX_OK;
}

int styx_batch_wait_idle(styx_batch *b)
{
    if (!b) return fail(STYX_E_INVALID, "styx_batch_wait_idle: NULL batch");
    if (!b->pending) return STYX_OK;
    STYX_HIP(hipSetDevice(b->gpu->device));
    STYX_HIP(hipEventSynchronize(b->done));
    b->pending = false;
    return STYX_OK;
}

int styx_batch_submit_wait_sem(styx_batch *b, styx_timeline *t, uint64_t value)
{
    if (!b || !t) return fail(STYX_E_INVALID, "styx_batch_submit_wait_sem: NULL batch or timeline");
    if (!b->recording) return STYX_OK;
    if (t->gpu != b->gpu)
        return fail(STYX_E_INVALID, "styx_batch_submit_wait_sem: timeline of another styx_gpu");
    STYX_HIP(hipSetDevice(b->gpu->device));
    hipStream_t st = b->own ? b->own : b->gpu->stream;
    {
        std::lock_guard<std::mutex> lock(t->mu);
        if (int r = timeline_poll(t)) return r;
        if (t->reached < value) {
            // the first pending signal that reaches the value; a wait for a
            // value nobody has submitted yet would never end on one stream
            size_t i = 0;
            while (i < t->sig.size() && t->sig[i].first < value) i++;
            if (i == t->sig.size())
                return fail(STYX_E_STATE, "styx_batch_submit_wait_sem: no signal of value >= " +
                                              std::to_string(value) + " has been submitted");
            STYX_HIP(hipStreamWaitEvent(st, t->sig[i].second, 0));
        }
    }
    b->recording = false;
    if (int r = run_cmds(b, st)) return r;
    STYX_HIP(hipStreamSynchronize(st));
    return STYX_OK;
}

}  // extern "C"
