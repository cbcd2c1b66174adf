// kernels_ref.hip -- kernels with the reference pipelines' exact interface,
// for the generic dispatch path (styx_batch_dispatch).  Each takes the
// bindings and push-constant block of the shader or vendored kernel it
// stands in for, with the same workgroup grid.  Quant weights are read in
// GGUF block layout, as the reference uploads them.
#include "deq.h"
#include "kernels.h"
#include "qdot.h"
#include "refk.h"
#include "topk.h"

#include <algorithm>
#include <cmath>
#include <cstring>

namespace styx {

#pragma clang fp contract(off)

// shaders/moe_reduce_f32.comp: x[i] += sum_s w[s]*d[s*ne+i]
__global__ void __launch_bounds__(256) kr_moe_reduce(const float *d, const float *w, float *x,
                                                     uint32_t ne, uint32_t k)
{
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i >= ne) return;
    float acc = 0.0f;
    for (uint32_t s = 0; s < k; s++) acc += w[s] * d[s * ne + i];
    x[i] += acc;
}

// shaders/add_flat_f32.comp
__global__ void __launch_bounds__(256) kr_add(const float *a, const float *b, float *d, uint32_t n)
{
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) d[i] = a[i] + b[i];
}

// shaders/axpy_sig_f32.comp
__global__ void __launch_bounds__(256) kr_axpy_sig(const float *a, const float *g, float *d,
                                                   uint32_t n)
{
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    const float s = 1.0f / (1.0f + expf(-g[0]));
    if (i < n) d[i] += s * a[i];
}

// shaders/matvec_strided_f32.comp: 32 strided partials, halving tree.
__global__ void __launch_bounds__(32) kr_matvec_strided(const float *A, const float *x, float *d,
                                                        uint32_t ncols, uint32_t stride)
{
    __shared__ float tmp[32];
    const uint32_t row = blockIdx.x, tid = threadIdx.x;
    const float *a = A + (int64_t)row * stride;
    float sum = 0.0f;
    for (uint32_t c = tid; c < ncols; c += 32) sum += a[c] * x[c];
    tmp[tid] = sum;
    __syncthreads();
    for (uint32_t s = 16; s > 0; s >>= 1) {
        if (tid < s) tmp[tid] += tmp[tid + s];
        __syncthreads();
    }
    if (tid == 0) d[row] = tmp[0];
}

// shaders/attn_decode_f32.comp:31-79 (one workgroup of 128 per query head).
__global__ void __launch_bounds__(128) kr_attn_decode(const float *Q, const float *K,
                                                      const float *V, float *O, uint32_t n_t,
                                                      uint32_t hd, uint32_t kv_dim, uint32_t gqa,
                                                      float scale)
{
    __shared__ float sh_q[256];
    __shared__ float sh_red[128];
    __shared__ float sh_prob, sh_m, sh_l, sh_corr;
    const uint32_t h = blockIdx.x, tid = threadIdx.x;
    const uint32_t kvoff = (h / gqa) * hd, qbase = h * hd;
    for (uint32_t i = tid; i < hd; i += 128) sh_q[i] = Q[qbase + i];
    __syncthreads();
    float acc0 = 0.0f, acc1 = 0.0f, m = -INFINITY, l = 0.0f;
    for (uint32_t t = 0; t < n_t; t++) {
        const int64_t krow = (int64_t)t * kv_dim + kvoff;
        float part = 0.0f;
        for (uint32_t i = tid; i < hd; i += 128) part += sh_q[i] * K[krow + i];
        sh_red[tid] = part;
        __syncthreads();
        for (uint32_t s = 64; s > 0; s >>= 1) {
            if (tid < s) sh_red[tid] += sh_red[tid + s];
            __syncthreads();
        }
        if (tid == 0) {
            const float sc = sh_red[0] * scale;
            const float m_new = fmaxf(m, sc);
            const float corr = expf(m - m_new);
            const float pr = expf(sc - m_new);
            sh_l = l * corr + pr;
            sh_m = m_new;
            sh_prob = pr;
            sh_corr = corr;
        }
        __syncthreads();
        const float pr = sh_prob, corr = sh_corr;
        m = sh_m;
        l = sh_l;
        if (tid < hd) acc0 = acc0 * corr + pr * V[krow + tid];
        if (tid + 128 < hd) acc1 = acc1 * corr + pr * V[krow + tid + 128];
        __syncthreads();
    }
    const float inv_l = 1.0f / l;
    if (tid < hd) O[qbase + tid] = acc0 * inv_l;
    if (tid + 128 < hd) O[qbase + tid + 128] = acc1 * inv_l;
}

// swiglu_f32 split mode over n values (GluPush.n).
__global__ void __launch_bounds__(256) kr_swiglu(const float *g, const float *u, float *d, uint32_t n)
{
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) d[i] = g[i] / (1.0f + expf(-g[i])) * u[i];
}

// rms_norm_f32 (generic_binary_head, do_multiply spec): one row per workgroup.
__global__ void __launch_bounds__(256) kr_rms_norm(const float *a, const float *w, float *d,
                                                   uint32_t ncols, uint32_t a_row, uint32_t d_row,
                                                   float eps, int mul)
{
    __shared__ float red[16];
    const float *x = a + (int64_t)blockIdx.x * a_row;
    float ss = 0.0f;
    for (uint32_t c = threadIdx.x; c < ncols; c += 256) ss += x[c] * x[c];
    ss = block_sum(ss, red);
    const float scale = 1.0f / sqrtf(ss / (float)ncols + eps);
    float *y = d + (int64_t)blockIdx.x * d_row;
    for (uint32_t c = threadIdx.x; c < ncols; c += 256) y[c] = mul ? (scale * x[c]) * w[c] : scale * x[c];
}

#pragma clang fp contract(on)

// mul_mat_vec_{t} / mul_mat_vec_id_{t} over GGUF-layout rows: one wave per
// (row, slot); lanes take blocks, dequantize in reference order and dot.
struct MmvRef {
    const uint8_t *A;
    const float *B;
    float *D;
    const int32_t *ids;  // null for the plain matvec
    int type;
    uint32_t ncols, stride_a, stride_b, stride_d, batch_stride_a, batch_stride_b, batch_stride_d;
    uint32_t ne11, expert_i1, nbi1, nrows, num_rows;
    int64_t n_mat;  // matrices readable from A (ids at or past it are skipped)
};

__global__ void __launch_bounds__(64) kr_mmv(MmvRef p)
{
    const int t = p.type, be = blk_elems(t), bb = blk_bytes(t);
    const uint32_t slot = blockIdx.y;
    int64_t a_blk = 0, b_off = 0, d_off = 0;
    if (p.ids) {
        // get_offsets() of mul_mat_vec_base (crates/vk-backend/tests/kernels.rs:124-131)
        const uint32_t e = (uint32_t)p.ids[slot + p.expert_i1 * p.nbi1];
        if (e == SKIP || (int64_t)e >= p.n_mat) return;
        a_blk = (int64_t)e * (p.batch_stride_a / be);
        b_off = (int64_t)(slot % p.ne11) * p.stride_b + (int64_t)p.expert_i1 * p.batch_stride_b;
        d_off = (int64_t)slot * p.stride_d + (int64_t)p.expert_i1 * p.batch_stride_d;
    }
    const uint32_t nb = p.ncols / be;
    for (uint32_t j = 0; j < p.num_rows; j++) {
        const uint32_t r = blockIdx.x * p.num_rows + j;
        if (r >= p.nrows) return;
        float acc = 0.0f;
        for (uint32_t b = threadIdx.x; b < nb; b += 64) {
            const uint8_t *blk = p.A + (a_blk + (int64_t)r * p.stride_a + b) * bb;
            float y[256];
            deq_block(t, gguf_blk(blk, t), 0, y, false);
            const float *x = p.B + b_off + (int64_t)b * be;
            for (int i = 0; i < be; i++) acc += y[i] * x[i];
        }
        acc = wave_sum(acc);
        if (threadIdx.x == 0) p.D[d_off + r] = acc;
    }
}

// topk_softmax_f32 with the shader's bindings (remap/pmap required).
__global__ void __launch_bounds__(64) kr_topk(const float *logits, float *w, int32_t *ids,
                                              const uint32_t *remap, const uint32_t *pmap,
                                              uint32_t n, uint32_t k, uint32_t renorm)
{
    topk_wave(logits, (int)n, (int)k, (int)renorm, remap, pmap, 0, 0, w, ids);
}

// rope_neox_f32 with the RopePush of crates/vk-backend/src/ops.rs:385-439
// for the mode the engine uses (NEOX, no frequency factors, no YaRN:
// ext_factor 0, freq_scale 1, attn_factor 1): row r = (i3, i2, i1) of
// (ne01, ne02) rows, pair i < ne00/2 of this thread; pairs (i, i + n/2) of
// the first n_dims values rotate by pos[i2] * base^(-2i/n_dims), the angle
// and its sine and cosine in f64 (the reference test's CPU formula,
// crates/vk-backend/tests/ops2.rs:426-442); values past n_dims are copied.
struct RopeArgs {
    const float *src;
    const int32_t *pos;
    float *dst;
    uint32_t nrows, n_dims, ne00, ne01, ne02;
    uint32_t nb01, nb02, nb03, nb11, nb12, nb13, a_off, d_off;
    double theta_scale;
};

__global__ void __launch_bounds__(256) kr_rope_neox(RopeArgs a)
{
    const uint32_t r = blockIdx.x, i = blockIdx.y * 256 + threadIdx.x;
    if (r >= a.nrows || 2 * i >= a.ne00) return;
    const uint32_t i1 = r % a.ne01, i2 = (r / a.ne01) % a.ne02, i3 = r / (a.ne01 * a.ne02);
    const int64_t s0 = a.a_off + (int64_t)i3 * a.nb03 + (int64_t)i2 * a.nb02 + (int64_t)i1 * a.nb01;
    const int64_t d0 = a.d_off + (int64_t)i3 * a.nb13 + (int64_t)i2 * a.nb12 + (int64_t)i1 * a.nb11;
    if (2 * i >= a.n_dims) {  // past the rotated dims: copied through
        a.dst[d0 + 2 * i] = a.src[s0 + 2 * i];
        a.dst[d0 + 2 * i + 1] = a.src[s0 + 2 * i + 1];
        return;
    }
    const uint32_t half = a.n_dims / 2;
    const double th = (double)a.pos[i2] * pow(a.theta_scale, (double)i);
    double sn, cs;
    sincos(th, &sn, &cs);
    const double x0 = a.src[s0 + i], x1 = a.src[s0 + i + half];
    a.dst[d0 + i] = (float)(x0 * cs - x1 * sn);
    a.dst[d0 + i + half] = (float)(x0 * sn + x1 * cs);
}

// cpy_f32_f32 with the UnaryPush of ops.rs:253-323: element j < ne of the
// source, at its 4-d index in src0's extents and strides (plus the
// misalignment offset's high half), goes to the same running index in dst's
// extents and strides (plus the low half).  512 elements per workgroup
// (the engine's grid, crates/model/src/moe.rs:1935-1943).
struct CpyArgs {
    const float *src;
    float *dst;
    uint32_t ne;
    uint32_t sne[4], snb[4], dne[4], dnb[4];
    uint32_t a_off, d_off;
};

__device__ __forceinline__ int64_t elem_at(uint32_t j, const uint32_t *ne, const uint32_t *nb)
{
    const uint32_t i0 = j % ne[0], i1 = (j / ne[0]) % ne[1], i2 = (j / (ne[0] * ne[1])) % ne[2],
                   i3 = j / (ne[0] * ne[1] * ne[2]);
    return (int64_t)i3 * nb[3] + (int64_t)i2 * nb[2] + (int64_t)i1 * nb[1] + (int64_t)i0 * nb[0];
}

__global__ void __launch_bounds__(256) kr_cpy(CpyArgs a)
{
    const uint64_t wg = ((uint64_t)blockIdx.z * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x;
    for (uint32_t t = threadIdx.x; t < 512; t += 256) {
        const uint64_t j = wg * 512 + t;
        if (j >= a.ne) return;
        a.dst[a.d_off + elem_at((uint32_t)j, a.dne, a.dnb)] = a.src[a.a_off + elem_at((uint32_t)j, a.sne, a.snb)];
    }
}

// Whether n elements of `bytes_each` bytes fit in a binding of `size` bytes
// (n may be 0).
static bool fits(uint64_t size, uint64_t n, uint64_t bytes_each)
{
    return n == 0 || (bytes_each != 0 && n <= size / bytes_each);
}

hipError_t refk_launch(hipStream_t st, int kid, void *const *ptr, const uint64_t *size,
                       const void *push, uint32_t gx, uint32_t gy, uint32_t gz,
                       const uint32_t *spec, int n_spec)
{
    const uint32_t *pc = (const uint32_t *)push;
    const hipError_t bad = hipErrorInvalidValue;
    switch (kid) {
    case RK_MOE_REDUCE: {
        // push: ne, k
        const uint64_t ne = pc[0], k = pc[1];
        if (!fits(size[0], k * ne, 4) || !fits(size[1], k, 4) || !fits(size[2], ne, 4)) return bad;
        hipLaunchKernelGGL(kr_moe_reduce, dim3(gx), dim3(256), 0, st, (const float *)ptr[0],
                           (const float *)ptr[1], (float *)ptr[2], pc[0], pc[1]);
        break;
    }
    case RK_ADD:
        if (!fits(size[0], pc[0], 4) || !fits(size[1], pc[0], 4) || !fits(size[2], pc[0], 4)) return bad;
        hipLaunchKernelGGL(kr_add, dim3(gx), dim3(256), 0, st, (const float *)ptr[0],
                           (const float *)ptr[1], (float *)ptr[2], pc[0]);
        break;
    case RK_AXPY_SIG:
        if (!fits(size[0], pc[0], 4) || !fits(size[1], 1, 4) || !fits(size[2], pc[0], 4)) return bad;
        hipLaunchKernelGGL(kr_axpy_sig, dim3(gx), dim3(256), 0, st, (const float *)ptr[0],
                           (const float *)ptr[1], (float *)ptr[2], pc[0]);
        break;
    case RK_MATVEC_STRIDED: {
        // push: ncols, stride; one row per workgroup
        const uint64_t nc = pc[0], stride = pc[1];
        if (!fits(size[0], (uint64_t)(gx - 1) * stride + nc, 4) || !fits(size[1], nc, 4) ||
            !fits(size[2], gx, 4))
            return bad;
        hipLaunchKernelGGL(kr_matvec_strided, dim3(gx), dim3(32), 0, st, (const float *)ptr[0],
                           (const float *)ptr[1], (float *)ptr[2], pc[0], pc[1]);
        break;
    }
    case RK_ATTN: {
        // push: n_t, hd, kv_dim, gqa, scale; one query head per workgroup
        float scale;
        std::memcpy(&scale, pc + 4, 4);
        const uint64_t n_t = pc[0], hd = pc[1], kvd = pc[2], gqa = pc[3];
        if (hd == 0 || hd > 256 || gqa == 0) return bad;
        const uint64_t kv_need = n_t ? (n_t - 1) * kvd + ((gx - 1) / gqa) * hd + hd : 0;
        if (!fits(size[0], (uint64_t)gx * hd, 4) || !fits(size[1], kv_need, 4) ||
            !fits(size[2], kv_need, 4) || !fits(size[3], (uint64_t)gx * hd, 4))
            return bad;
        hipLaunchKernelGGL(kr_attn_decode, dim3(gx), dim3(128), 0, st, (const float *)ptr[0],
                           (const float *)ptr[1], (const float *)ptr[2], (float *)ptr[3], pc[0],
                           pc[1], pc[2], pc[3], scale);
        break;
    }
    case RK_SWIGLU:
        // GluPush: n is the first field
        if (!fits(size[0], pc[0], 4) || !fits(size[1], pc[0], 4) || !fits(size[2], pc[0], 4)) return bad;
        hipLaunchKernelGGL(kr_swiglu, dim3((pc[0] + 255) / 256), dim3(256), 0, st,
                           (const float *)ptr[0], (const float *)ptr[1], (float *)ptr[2], pc[0]);
        break;
    case RK_RMS_NORM: {
        // BinaryPush: ne, src0[8] (ne00..ne03, nb00..nb03), src1[8], dst[8], misalign, param1
        float eps;
        std::memcpy(&eps, pc + 26, 4);
        int mul = 1;
        for (int i = 0; i + 1 < 2 * n_spec; i += 2)
            if (spec[i] == 1) mul = spec[i + 1] != 0;
        const uint64_t nc = pc[1], arow = pc[6], drow = pc[22];
        if (!fits(size[0], (uint64_t)(gx - 1) * arow + nc, 4) || (mul && !fits(size[1], nc, 4)) ||
            !fits(size[2], (uint64_t)(gx - 1) * drow + nc, 4))
            return bad;
        hipLaunchKernelGGL(kr_rms_norm, dim3(gx), dim3(256), 0, st, (const float *)ptr[0],
                           (const float *)ptr[1], (float *)ptr[2], pc[1], pc[6], pc[22], eps, mul);
        break;
    }
    case RK_ROPE_NEOX: {
        float f[29];
        std::memcpy(f, pc, sizeof(f));
        RopeArgs a{};
        a.nrows = pc[1];
        a.n_dims = pc[2];
        const float freq_scale = f[3], freq_base = f[4], ext_factor = f[5], attn_factor = f[6];
        a.ne00 = pc[18], a.ne01 = pc[19], a.ne02 = pc[20];
        a.nb01 = pc[21], a.nb02 = pc[22], a.nb03 = pc[23];
        a.nb11 = pc[24], a.nb12 = pc[25], a.nb13 = pc[26];
        a.a_off = pc[27], a.d_off = pc[28];
        // the supported mode: NEOX (2), no frequency factors, no YaRN, not
        // the backward pass, no set_rows, rotation within each row
        if (pc[0] != 2 || freq_scale != 1.0f || ext_factor != 0.0f || attn_factor != 1.0f ||
            pc[10] != 0 || pc[15] != 0 || pc[16] != 0 || pc[17] != 0 || a.n_dims == 0 ||
            a.n_dims % 2 || a.n_dims > a.ne00 || a.ne00 % 2 || a.ne01 == 0 || a.ne02 == 0 ||
            !(freq_base > 0.0f) || gx < a.nrows || (uint64_t)gy * 256 < a.ne00 / 2)
            return bad;
        const uint64_t n3 = ((uint64_t)a.nrows + a.ne01 * a.ne02 - 1) / ((uint64_t)a.ne01 * a.ne02);
        const uint64_t src_need = a.a_off + (n3 - 1) * a.nb03 + (uint64_t)(a.ne02 - 1) * a.nb02 +
                                  (uint64_t)(a.ne01 - 1) * a.nb01 + a.ne00;
        const uint64_t dst_need = a.d_off + (n3 - 1) * a.nb13 + (uint64_t)(a.ne02 - 1) * a.nb12 +
                                  (uint64_t)(a.ne01 - 1) * a.nb11 + a.ne00;
        if (!fits(size[0], src_need, 4) || !fits(size[1], a.ne02, 4) || !fits(size[3], dst_need, 4))
            return bad;
        a.src = (const float *)ptr[0];
        a.pos = (const int32_t *)ptr[1];
        a.dst = (float *)ptr[3];
        a.theta_scale = std::pow((double)freq_base, -2.0 / (double)a.n_dims);
        hipLaunchKernelGGL(kr_rope_neox, dim3(a.nrows, (a.ne00 / 2 + 255) / 256), dim3(256), 0, st,
                           a);
        break;
    }
    case RK_CPY: {
        CpyArgs a{};
        a.ne = pc[0];
        for (int i = 0; i < 4; i++) {
            a.sne[i] = pc[1 + i];
            a.snb[i] = pc[5 + i];
            a.dne[i] = pc[9 + i];
            a.dnb[i] = pc[13 + i];
        }
        a.a_off = pc[17] >> 16;
        a.d_off = pc[17] & 0xFFFF;
        uint64_t sn = 1, dn = 1, s_need = a.a_off + 1, d_need = a.d_off + 1;
        for (int i = 0; i < 4; i++) {
            if (a.sne[i] == 0 || a.dne[i] == 0) return bad;
            sn *= a.sne[i];
            dn *= a.dne[i];
            s_need += (uint64_t)(a.sne[i] - 1) * a.snb[i];
            d_need += (uint64_t)(a.dne[i] - 1) * a.dnb[i];
        }
        if (a.ne == 0 || sn < a.ne || dn < a.ne || sn > 0xFFFFFFFFull || dn > 0xFFFFFFFFull ||
            (uint64_t)gx * gy * gz * 512 < a.ne || !fits(size[0], s_need, 4) ||
            !fits(size[1], d_need, 4))
            return bad;
        a.src = (const float *)ptr[0];
        a.dst = (float *)ptr[1];
        hipLaunchKernelGGL(kr_cpy, dim3(gx, gy, gz), dim3(256), 0, st, a);
        break;
    }
    case RK_TOPK:
        // push: n, k, renorm; writes the 64-entry id row
        if (pc[0] < 1 || pc[0] > MAX_EXPERTS || pc[1] < 1 || pc[1] > MAX_TOPK)
            return bad;
        if (!fits(size[0], pc[0], 4) || !fits(size[1], pc[1], 4) || !fits(size[2], IDS_ROW, 4) ||
            !fits(size[3], pc[0], 4) || !fits(size[4], pc[0], 4))
            return bad;
        hipLaunchKernelGGL(kr_topk, dim3(1), dim3(64), 0, st, (const float *)ptr[0],
                           (float *)ptr[1], (int32_t *)ptr[2], (const uint32_t *)ptr[3],
                           (const uint32_t *)ptr[4], pc[0], pc[1], pc[2]);
        break;
    case RK_GATHER: {
        // push: dst_vg, dst_vu, dst_vd, src_vg, src_vu, src_vd, layer, k, canary
        if (pc[8] != 0) return bad;
        const uint8_t *src[3] = {(const uint8_t *)ptr[0], (const uint8_t *)ptr[1],
                                 (const uint8_t *)ptr[2]};
        uint8_t *dst[3] = {(uint8_t *)ptr[3], (uint8_t *)ptr[4], (uint8_t *)ptr[5]};
        const int64_t ss[3] = {16ll * pc[3], 16ll * pc[4], 16ll * pc[5]};
        const int64_t ds[3] = {16ll * pc[0], 16ll * pc[1], 16ll * pc[2]};
        const uint64_t k = pc[7], slots = ((uint64_t)pc[6] + 1) * k;
        if (k < 1 || k > MAX_TOPK || !fits(size[6], k, 4)) return bad;
        int64_t cnt[3];
        for (int t = 0; t < 3; t++) {
            if (ss[t] == 0 || !fits(size[3 + t], slots, (uint64_t)ds[t])) return bad;
            cnt[t] = (int64_t)(size[t] / (uint64_t)ss[t]);
        }
        return launch_gather_list(st, src, ss, dst, ds, (const int32_t *)ptr[6], (int)pc[7],
                                  (int)pc[6], cnt);
    }
    default: {
        if (kid < RK_MMV_BASE || kid >= RK_MMV_BASE + 8) return bad;
        const int ti = (kid - RK_MMV_BASE) % 4;
        const bool with_id = kid >= RK_MMV_BASE + 4;
        static const int types[4] = {T_Q8_0, T_Q4_K, T_Q5_K, T_Q6_K};
        MmvRef p{};
        p.type = types[ti];
        p.A = (const uint8_t *)ptr[0];
        p.B = (const float *)ptr[1];
        p.D = (float *)ptr[2];
        p.ncols = pc[0];
        p.stride_a = pc[1];
        p.stride_b = pc[2];
        p.stride_d = pc[3];
        p.batch_stride_a = pc[4];
        p.batch_stride_b = pc[5];
        p.batch_stride_d = pc[6];
        const uint64_t be = blk_elems(p.type), bb = blk_bytes(p.type), nb = p.ncols / be;
        if (p.ncols == 0 || p.ncols % be || p.stride_a < nb) return bad;
        if (with_id) {
            // MatVecIdPush: ..., fusion_flags, nei0, ne11, expert_i1, nbi1
            p.ids = (const int32_t *)ptr[5];
            p.ne11 = pc[9] ? pc[9] : 1;
            p.expert_i1 = pc[10];
            p.nbi1 = pc[11];
            p.nrows = gx;
            p.num_rows = 1;
            if (p.batch_stride_a % be) return bad;
            // one matrix: nrows rows of stride_a blocks, within the expert stride
            const uint64_t mat_blocks = (uint64_t)p.batch_stride_a / be;
            const uint64_t used_blocks = (uint64_t)(p.nrows - 1) * p.stride_a + nb;
            if (mat_blocks == 0 || used_blocks > mat_blocks) return bad;
            p.n_mat = (int64_t)(size[0] / (mat_blocks * bb));
            const uint64_t nsl = gy, ne11 = p.ne11;
            const uint64_t b_need = (std::min<uint64_t>(nsl, ne11) - 1) * p.stride_b +
                                    (uint64_t)p.expert_i1 * p.batch_stride_b + p.ncols;
            const uint64_t d_need = (nsl - 1) * p.stride_d +
                                    (uint64_t)p.expert_i1 * p.batch_stride_d + p.nrows;
            const uint64_t id_need = (nsl - 1) + (uint64_t)p.expert_i1 * p.nbi1 + 1;
            if (!fits(size[1], b_need, 4) || !fits(size[2], d_need, 4) || !fits(size[5], id_need, 4))
                return bad;
        } else {
            // MatVecPush: stride_d = nrows (MatVecPush::simple); NUM_ROWS spec id 1
            p.num_rows = 1;
            for (int i = 0; i + 1 < 2 * n_spec; i += 2)
                if (spec[i] == 1) p.num_rows = spec[i + 1] ? spec[i + 1] : 1;
            p.nrows = p.stride_d;
            p.n_mat = 1;
            if (p.nrows == 0 || !fits(size[0], (uint64_t)(p.nrows - 1) * p.stride_a + nb, bb) ||
                !fits(size[1], p.ncols, 4) || !fits(size[2], p.nrows, 4))
                return bad;
        }
        hipLaunchKernelGGL(kr_mmv, dim3(gx, with_id ? gy : 1, 1), dim3(64), 0, st, p);
        break;
    }
    }
    return hipGetLastError();
}

}  // namespace styx
