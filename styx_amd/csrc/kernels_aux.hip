// kernels_aux.hip -- layout conversion, dequant check, embedding, argmax,
// slab gather and the seeded synthetic-weight generator (gfx950).
#include "kernels.h"
#include "qdot.h"
#include "deq.h"
#include "topk.h"

#include <algorithm>

namespace styx {

// ------------------------------------------------- GGUF <-> split layout --
// One thread per block; each region's bytes are moved with byte loops (a
// load-time operation).
__global__ void k_to_split(int t, const uint8_t *src, uint8_t *dst, int64_t nblocks, int64_t nmat,
                           int dir)
{
    const Split s = split_of(t);
    const int bb = blk_bytes(t);
    const int64_t total = nblocks * nmat;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t m = i / nblocks, b = i - m * nblocks;
        const uint8_t *gs = (dir ? dst : src);
        (void)gs;
        const int64_t mbase = m * nblocks * bb;
        for (int r = 0; r < s.nreg; r++) {
            const int64_t so = mbase + b * bb + s.src[r];
            const int64_t po = mbase + region_off(s, r, nblocks);
            if (dir == 0)
                for (int j = 0; j < s.sz[r]; j++) dst[po + ilv_off(t, r, b, j)] = src[so + j];
            else
                for (int j = 0; j < s.sz[r]; j++) dst[so + j] = src[po + ilv_off(t, r, b, j)];
        }
    }
}

static hipError_t split_launch(hipStream_t st, int t, const uint8_t *src, uint8_t *dst,
                               int64_t nblocks, int64_t nmat, int dir)
{
    if (blk_bytes(t) == 0 || nblocks < 1 || nmat < 1 || nblocks % ilv_group(t))
        return hipErrorInvalidValue;
    const int64_t total = nblocks * nmat;
    const int64_t nwg = std::min<int64_t>((total + 255) / 256, 65536);
    hipLaunchKernelGGL(k_to_split, dim3((unsigned)std::max<int64_t>(nwg, 1)), dim3(256), 0, st, t,
                       src, dst, nblocks, nmat, dir);
    return hipGetLastError();
}

hipError_t launch_to_split(hipStream_t st, int t, const uint8_t *src, uint8_t *dst,
                           int64_t nblocks, int64_t nmat)
{
    return split_launch(st, t, src, dst, nblocks, nmat, 0);
}
hipError_t launch_from_split(hipStream_t st, int t, const uint8_t *src, uint8_t *dst,
                             int64_t nblocks, int64_t nmat)
{
    return split_launch(st, t, src, dst, nblocks, nmat, 1);
}

__global__ void k_dequant_rows(int t, const uint8_t *w, int64_t nrows_total, int ncols,
                               int64_t r0, int64_t nrows, float *out)
{
    const int be = blk_elems(t), nb = ncols / be;
    const Mat m = mat_at(w, t, nrows_total * nb);
    const int64_t total = nrows * nb;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = i / nb, b = i - r * nb;
        deq_block(t, m, (r0 + r) * nb + b, out + r * ncols + (int64_t)b * be);
    }
}

hipError_t launch_dequant_rows(hipStream_t st, int t, const uint8_t *w, int64_t nrows_total,
                               int ncols, int64_t r0, int64_t nrows, float *out)
{
    if (blk_bytes(t) == 0 || ncols % blk_elems(t)) return hipErrorInvalidValue;
    const int64_t total = nrows * (ncols / blk_elems(t));
    const int64_t nwg = std::min<int64_t>((total + 255) / 256, 65536);
    hipLaunchKernelGGL(k_dequant_rows, dim3((unsigned)std::max<int64_t>(nwg, 1)), dim3(256), 0,
                       st, t, w, nrows_total, ncols, r0, nrows, out);
    return hipGetLastError();
}

// ----------------------------------------------------------- embedding ----
// x = dequant(token_embd[tok]); the limbs of x ⊙ norm_w for the first
// layer's q/k/v matvec, which applies the RMSNorm scale from ss[0] = sum x^2
// (ss[1..nss) = 0); one workgroup.  With rope_row, the (cos, sin) row of
// *pos copied from the rope table.
__global__ void __launch_bounds__(256) k_embed(int t, const uint8_t *w, int64_t nrows, int ncols,
                                               const uint32_t *tok, float *x, const float *nw,
                                               Xq q, float *ss, int nss, const double2 *rope,
                                               const int32_t *pos, double2 *rope_row, int half)
{
    extern __shared__ __align__(16) float xs[];  // [ncols]
    __shared__ float red[16];
    // the rope row of the position by the last wave, whose threads have no
    // embedding blocks at the shapes served (nb <= 192): its two dependent
    // loads then run beside the token's, not before them
    if (rope_row && threadIdx.x >= blockDim.x - 64) {
        const int64_t p = *pos;
        for (int i = threadIdx.x - (blockDim.x - 64); i < half; i += 64) rope_row[i] = rope[p * half + i];
    }
    const int be = blk_elems(t), nb = ncols / be;
    const Mat m = mat_at(w, t, nrows * nb);
    const int64_t r = *tok;
    for (int b = threadIdx.x; b < nb; b += blockDim.x) deq_block(t, m, r * nb + b, xs + b * be);
    __syncthreads();
    float sq = 0.0f;
    for (int i = threadIdx.x; i < ncols; i += blockDim.x) {
        x[i] = xs[i];
        sq += xs[i] * xs[i];
    }
    sq = block_sum(sq, red);
    if (ss)
        for (int i = threadIdx.x; i < nss; i += blockDim.x) ss[i] = i == 0 ? sq : 0.0f;
    if (!q.A) return;
    for (int g0 = 0; g0 < ncols / 8; g0 += blockDim.x) {
        const int g = g0 + threadIdx.x;
        const bool act = g < ncols / 8;
        float v[8];
#pragma unroll
        for (int i = 0; i < 8; i++) v[i] = act ? xs[8 * g + i] * (nw ? nw[8 * g + i] : 1.0f) : 0.0f;
        xq_group(v, act, g, q);
    }
}

hipError_t launch_embed(hipStream_t st, int t, const uint8_t *w, int64_t nrows, int ncols,
                        const uint32_t *tok, float *x, const float *norm_w, const Xq &q,
                        float *ss, const double2 *rope, const int32_t *pos, double2 *rope_row,
                        int half)
{
    if (ncols % 32 || ncols > XQ_MAX || ncols % blk_elems(t)) return hipErrorInvalidValue;
    if (rope_row && (!rope || !pos || half < 1)) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_embed, dim3(1), dim3(256), (size_t)ncols * 4, st, t, w, nrows, ncols,
                       tok, x, norm_w, q, ss, ncols / 32, rope, pos, rope_row, half);
    return hipGetLastError();
}

// -------------------------------------------------------------- argmax ----
// Rust f32::total_cmp key; larger key wins, equal keys -> larger index
// (Iterator::max_by keeps the last maximum, generate_moe.rs:29).
__device__ __forceinline__ int32_t tkey(float v)
{
    int32_t b = __float_as_int(v);
    return b ^ (int32_t)(((uint32_t)(b >> 31)) >> 1);
}

constexpr int ARGMAX_WG = 64;

// Stage 1: each workgroup reduces a contiguous slice to (key, index).
__global__ void __launch_bounds__(256) k_argmax_part(const float *v, int n, float *part_key,
                                                     uint32_t *part_idx)
{
    __shared__ int32_t sk[4];
    __shared__ uint32_t si[4];
    const int per = (n + gridDim.x - 1) / gridDim.x;
    const int lo = blockIdx.x * per, hi = min(n, lo + per);
    int32_t bk = INT32_MIN;
    uint32_t bi = 0;
    for (int i = lo + threadIdx.x; i < hi; i += blockDim.x) {
        const int32_t k = tkey(v[i]);
        if (k > bk || (k == bk && (uint32_t)i > bi)) {
            bk = k;
            bi = i;
        }
    }
    for (int o = 32; o > 0; o >>= 1) {
        const int32_t ok = __shfl_xor(bk, o);
        const uint32_t oi = __shfl_xor(bi, o);
        if (ok > bk || (ok == bk && oi > bi)) {
            bk = ok;
            bi = oi;
        }
    }
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    if (lane == 0) {
        sk[w] = bk;
        si[w] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int j = 1; j < (int)(blockDim.x >> 6); j++)
            if (sk[j] > bk || (sk[j] == bk && si[j] > bi)) {
                bk = sk[j];
                bi = si[j];
            }
        part_key[blockIdx.x] = __int_as_float(bk);
        part_idx[blockIdx.x] = bi;
    }
}

// Stage 2: one wave reduces the stage-1 results in fixed order; optionally
// advances the device position and records the token (greedy decoding).
__global__ void __launch_bounds__(64) k_argmax_final(const float *part_key,
                                                     const uint32_t *part_idx, int nparts,
                                                     uint32_t *out_tok, int32_t *pos, int advance,
                                                     uint32_t *hist)
{
    if (threadIdx.x != 0) return;
    int32_t k = __float_as_int(part_key[0]);
    uint32_t idx = part_idx[0];
    for (int j = 1; j < nparts; j++) {
        const int32_t kj = __float_as_int(part_key[j]);
        if (kj > k || (kj == k && part_idx[j] > idx)) {
            k = kj;
            idx = part_idx[j];
        }
    }
    *out_tok = idx;
    if (advance) {
        const int32_t p = *pos + 1;
        *pos = p;
        if (hist) hist[p] = idx;
    }
}

__global__ void __launch_bounds__(64) k_argmax_word(unsigned long long *amax, uint32_t *out_tok,
                                                    int32_t *pos, int advance, uint32_t *hist)
{
    if (threadIdx.x != 0) return;
    // both loads before any store (one memory round trip, not two)
    const uint32_t idx = (uint32_t)*amax;
    const int32_t p = advance ? *pos + 1 : 0;
    *amax = 0ull;
    *out_tok = idx;
    if (advance) {
        *pos = p;
        if (hist) hist[p] = idx;
    }
}

hipError_t launch_argmax_word(hipStream_t st, unsigned long long *amax, uint32_t *out_tok,
                              int32_t *pos, int advance, uint32_t *hist)
{
    if (!amax || !out_tok || (advance && !pos)) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_argmax_word, dim3(1), dim3(64), 0, st, amax, out_tok, pos, advance, hist);
    return hipGetLastError();
}

hipError_t launch_argmax(hipStream_t st, const float *v, int n, uint32_t *out_tok,
                         float *part_val, uint32_t *part_idx, int32_t *pos, int advance,
                         uint32_t *hist)
{
    if (n < 1 || (advance && !pos)) return hipErrorInvalidValue;
    const int nwg = std::min(ARGMAX_WG, std::max(1, n / 1024));
    hipLaunchKernelGGL(k_argmax_part, dim3(nwg), dim3(256), 0, st, v, n, part_val, part_idx);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_argmax_final, dim3(1), dim3(64), 0, st, part_val, part_idx, nwg, out_tok,
                       pos, advance, hist);
    return hipGetLastError();
}

// -------------------------------------------------------------- gather ----
// shaders/gather_slabs_f32.comp:40-86: slot s with expert e != SKIP copies
// slab e of each tensor into its arena slot.  16-byte copies; grid
// (chunks, k, 3).
constexpr int64_t GATHER_CHUNK = 64 * 1024;

struct GatherK {
    const uint8_t *src[3];
    int64_t src_slab[3];
    uint8_t *dst[3];
    int64_t dst_slab[3];
    const int32_t *ids;
    Route route;  // mode 0 with route.logits: the id row is computed in-kernel
    int k, layer, mode;  // mode 0: arena row of an id row; 1: expert list
    int64_t src_count[3];  // mode 1: slabs readable per source (0: unbounded)
};

__global__ void __launch_bounds__(256) k_gather(GatherK a)
{
    __shared__ int32_t s_ids[IDS_ROW];
    __shared__ __align__(16) float s_lg[MAX_EXPERTS];
    const int s = blockIdx.y, t = blockIdx.z;
    uint32_t e, slot;
    if (a.mode == 0) {
        if (a.route.logits) {
            const int32_t *ids = route_ids_wg(a.route, s_ids, s_lg);
            uint32_t r3[3];
            route_row(a.route, ids[s], s, r3);
            slot = r3[1];
            e = (uint32_t)ids[s];
        } else {
            slot = (uint32_t)a.ids[32 + s];
            e = (uint32_t)a.ids[s];
        }
        if (slot == SKIP) return;
    } else {
        e = (uint32_t)a.ids[s];
        if (e == SKIP || (a.src_count[t] > 0 && (int64_t)e >= a.src_count[t])) return;
        slot = (uint32_t)(a.layer * a.k + s);
    }
    const int64_t n16 = a.src_slab[t] / 16;
    const int64_t c0 = blockIdx.x * (GATHER_CHUNK / 16);
    const int64_t c1 = min(n16, c0 + GATHER_CHUNK / 16);
    const uint4 *src = (const uint4 *)(a.src[t] + (int64_t)e * a.src_slab[t]);
    uint4 *dst = (uint4 *)(a.dst[t] + (int64_t)slot * a.dst_slab[t]);
    // four loads in flight per thread: the source is host memory across
    // PCIe, with a round trip of microseconds
    int64_t i = c0 + threadIdx.x;
    for (; i + 3 * 256 < c1; i += 4 * 256) {
        const uint4 v0 = src[i], v1 = src[i + 256], v2 = src[i + 512], v3 = src[i + 768];
        dst[i] = v0;
        dst[i + 256] = v1;
        dst[i + 512] = v2;
        dst[i + 768] = v3;
    }
    for (; i < c1; i += 256) dst[i] = src[i];
}

static hipError_t gather_launch(hipStream_t st, const uint8_t *const src[3],
                                const int64_t src_slab[3], uint8_t *const dst[3],
                                const int64_t dst_slab[3], const int32_t *ids, const Route *route,
                                int k, int layer, int mode, const int64_t *src_count = nullptr)
{
    if (route && (route->E < k || route->E > MAX_EXPERTS || route->E % 16 || route->k != k))
        return hipErrorInvalidValue;
    GatherK a{};
    if (route) a.route = *route;
    int64_t mx = 0;
    for (int t = 0; t < 3; t++) {
        if (src_slab[t] % 16 || dst_slab[t] % 16 || src_slab[t] > dst_slab[t])
            return hipErrorInvalidValue;
        a.src[t] = src[t];
        a.src_slab[t] = src_slab[t];
        a.dst[t] = dst[t];
        a.dst_slab[t] = dst_slab[t];
        a.src_count[t] = src_count ? src_count[t] : 0;
        mx = std::max(mx, src_slab[t]);
    }
    a.ids = ids;
    a.k = k;
    a.layer = layer;
    a.mode = mode;
    const int chunks = (int)((mx + GATHER_CHUNK - 1) / GATHER_CHUNK);
    hipLaunchKernelGGL(k_gather, dim3(std::max(chunks, 1), k, 3), dim3(256), 0, st, a);
    return hipGetLastError();
}

hipError_t launch_gather(hipStream_t st, const uint8_t *const src[3], const int64_t src_slab[3],
                         uint8_t *const dst[3], const int64_t dst_slab[3], const int32_t *ids,
                         const Route *route, int k)
{
    return gather_launch(st, src, src_slab, dst, dst_slab, ids, route, k, 0, 0);
}

hipError_t launch_gather_list(hipStream_t st, const uint8_t *const src[3],
                              const int64_t src_slab[3], uint8_t *const dst[3],
                              const int64_t dst_slab[3], const int32_t *ids, int k, int layer,
                              const int64_t *src_count)
{
    return gather_launch(st, src, src_slab, dst, dst_slab, ids, nullptr, k, layer, 1, src_count);
}

// ---------------------------------------------------------- generator ----
// Counter-based normal samples (splitmix64 + Box-Muller) quantized with
// simple min/max quantizers into GGUF blocks.  Deterministic in (seed, i).
__device__ __forceinline__ uint64_t mix64(uint64_t z)
{
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__device__ __forceinline__ float gauss(uint64_t seed, int64_t i)
{
    const uint64_t h1 = mix64(seed ^ mix64((uint64_t)i * 2 + 1));
    const uint64_t h2 = mix64(h1 ^ 0xD1B54A32D192ED03ull);
    const float u1 = ((float)(h1 >> 40) + 1.0f) * (1.0f / 16777216.0f);  // (0, 1]
    const float u2 = (float)(h2 >> 40) * (1.0f / 16777216.0f);
    return sqrtf(-2.0f * logf(u1)) * cosf(6.28318530717958648f * u2);
}

__device__ __forceinline__ uint16_t to_f16(float f)
{
    return __builtin_bit_cast(uint16_t, (_Float16)f);
}

__device__ void quant_block(int t, const float *x, uint8_t *o)
{
    if (t == T_F16) {  // one value, rounded to nearest even
        const uint16_t h = to_f16(x[0]);
        o[0] = h & 0xFF;
        o[1] = h >> 8;
        return;
    }
    if (t == T_Q8_0) {
        float am = 0.0f;
        for (int i = 0; i < 32; i++) am = fmaxf(am, fabsf(x[i]));
        const uint16_t dh = to_f16(am / 127.0f);
        const float d = f16f(dh), id = d > 0.0f ? 1.0f / d : 0.0f;
        o[0] = dh & 0xFF;
        o[1] = dh >> 8;
        for (int i = 0; i < 32; i++)
            o[2 + i] = (uint8_t)(int8_t)fminf(fmaxf(rintf(x[i] * id), -127.0f), 127.0f);
        return;
    }
    if (t == T_Q4_K || t == T_Q5_K) {
        const float lv = t == T_Q4_K ? 15.0f : 31.0f;
        float sc[8], mn[8], msc = 0.0f, mmn = 0.0f;
        for (int j = 0; j < 8; j++) {
            float lo = 0.0f, hi = -INFINITY;
            for (int i = 0; i < 32; i++) {
                lo = fminf(lo, x[32 * j + i]);
                hi = fmaxf(hi, x[32 * j + i]);
            }
            sc[j] = (hi - lo) / lv;
            mn[j] = -lo;
            msc = fmaxf(msc, sc[j]);
            mmn = fmaxf(mmn, mn[j]);
        }
        const uint16_t dh = to_f16(msc / 63.0f), mh = to_f16(mmn / 63.0f);
        const float d = f16f(dh), dmin = f16f(mh);
        int ls[8], lm[8];
        for (int j = 0; j < 8; j++) {
            ls[j] = d > 0.0f ? (int)fminf(rintf(sc[j] / d), 63.0f) : 0;
            lm[j] = dmin > 0.0f ? (int)fminf(rintf(mn[j] / dmin), 63.0f) : 0;
        }
        o[0] = dh & 0xFF; o[1] = dh >> 8; o[2] = mh & 0xFF; o[3] = mh >> 8;
        uint8_t *s = o + 4;
        for (int j = 0; j < 4; j++) {
            s[j] = (uint8_t)(ls[j] | ((ls[j + 4] >> 4) << 6));
            s[j + 4] = (uint8_t)(lm[j] | ((lm[j + 4] >> 4) << 6));
            s[j + 8] = (uint8_t)((ls[j + 4] & 0xF) | ((lm[j + 4] & 0xF) << 4));
        }
        int q[256];
        for (int j = 0; j < 8; j++) {
            const float ds = d * (float)ls[j], ms = dmin * (float)lm[j];
            for (int i = 0; i < 32; i++) {
                const float v = ds > 0.0f ? rintf((x[32 * j + i] + ms) / ds) : 0.0f;
                q[32 * j + i] = (int)fminf(fmaxf(v, 0.0f), lv);
            }
        }
        if (t == T_Q4_K) {
            uint8_t *qs = o + 16;
            for (int c = 0; c < 4; c++)
                for (int l = 0; l < 32; l++)
                    qs[32 * c + l] = (uint8_t)(q[64 * c + l] | (q[64 * c + 32 + l] << 4));
        } else {
            uint8_t *qh = o + 16, *qs = o + 48;
            for (int l = 0; l < 32; l++) qh[l] = 0;
            for (int c = 0; c < 4; c++)
                for (int l = 0; l < 32; l++) {
                    const int a = q[64 * c + l], b = q[64 * c + 32 + l];
                    qs[32 * c + l] = (uint8_t)((a & 15) | ((b & 15) << 4));
                    qh[l] |= (uint8_t)(((a >> 4) << (2 * c)) | ((b >> 4) << (2 * c + 1)));
                }
        }
        return;
    }
    if (t == T_Q6_K) {
        float sc[16], msc = 0.0f;
        for (int j = 0; j < 16; j++) {
            float am = 0.0f;
            for (int i = 0; i < 16; i++) am = fmaxf(am, fabsf(x[16 * j + i]));
            sc[j] = am / 31.0f;
            msc = fmaxf(msc, sc[j]);
        }
        const uint16_t dh = to_f16(msc / 127.0f);
        const float d = f16f(dh);
        int ls[16], q[256];
        for (int j = 0; j < 16; j++) {
            ls[j] = d > 0.0f ? (int)fminf(rintf(sc[j] / d), 127.0f) : 0;
            const float ds = d * (float)ls[j];
            for (int i = 0; i < 16; i++) {
                const float v = ds > 0.0f ? rintf(x[16 * j + i] / ds) : 0.0f;
                q[16 * j + i] = (int)fminf(fmaxf(v, -32.0f), 31.0f) + 32;
            }
        }
        uint8_t *ql = o, *qh = o + 128;
        int8_t *scs = (int8_t *)(o + 192);
        for (int n = 0; n < 2; n++)
            for (int l = 0; l < 32; l++) {
                const int q1 = q[128 * n + l], q2 = q[128 * n + 32 + l], q3 = q[128 * n + 64 + l],
                          q4 = q[128 * n + 96 + l];
                ql[64 * n + l] = (uint8_t)((q1 & 15) | ((q3 & 15) << 4));
                ql[64 * n + l + 32] = (uint8_t)((q2 & 15) | ((q4 & 15) << 4));
                qh[32 * n + l] =
                    (uint8_t)((q1 >> 4) | ((q2 >> 4) << 2) | ((q3 >> 4) << 4) | ((q4 >> 4) << 6));
            }
        for (int j = 0; j < 16; j++) scs[j] = (int8_t)ls[j];
        o[208] = dh & 0xFF;
        o[209] = dh >> 8;
        return;
    }
}

__global__ void __launch_bounds__(64) k_gen_quant(int t, uint64_t seed, float sigma, uint8_t *dst,
                                                  int64_t nblocks)
{
    const int be = blk_elems(t), bb = blk_bytes(t);
    for (int64_t b = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; b < nblocks;
         b += (int64_t)gridDim.x * blockDim.x) {
        float x[256];
        for (int i = 0; i < be; i++) x[i] = sigma * gauss(seed, b * be + i);
        quant_block(t, x, dst + b * bb);
    }
}

hipError_t launch_gen_quant(hipStream_t st, int t, uint64_t seed, float sigma, uint8_t *dst,
                            int64_t n)
{
    if ((!is_quant(t) && t != T_F16) || n % blk_elems(t)) return hipErrorInvalidValue;
    const int64_t nb = n / blk_elems(t);
    const int64_t nwg = std::min<int64_t>((nb + 63) / 64, 16384);
    hipLaunchKernelGGL(k_gen_quant, dim3((unsigned)std::max<int64_t>(nwg, 1)), dim3(64), 0, st, t,
                       seed, sigma, dst, nb);
    return hipGetLastError();
}

__global__ void k_gen_f32(uint64_t seed, float mean, float sigma, float *dst, int64_t n)
{
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x)
        dst[i] = sigma == 0.0f ? mean : mean + sigma * gauss(seed, i);
}

hipError_t launch_gen_f32(hipStream_t st, uint64_t seed, float mean, float sigma, float *dst,
                          int64_t n)
{
    const int64_t nwg = std::min<int64_t>((n + 255) / 256, 65536);
    hipLaunchKernelGGL(k_gen_f32, dim3((unsigned)std::max<int64_t>(nwg, 1)), dim3(256), 0, st, seed,
                       mean, sigma, dst, n);
    return hipGetLastError();
}

__global__ void k_fill_u32(uint32_t *p, uint32_t v, int64_t n)
{
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x)
        p[i] = v;
}

__global__ void k_clamp_copy_u32(const uint32_t *src, uint32_t *dst, uint32_t maxv, int64_t n)
{
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x)
        dst[i] = min(src[i], maxv);
}

// Streaming-read probe: every 16-byte word of [p, p + n16*16) is loaded
// once (4 loads in flight per lane) and folded into one word per workgroup,
// so the duration measures achievable HBM read bandwidth.
// Streaming-read probe: workgroup b reads the contiguous chunk
// [b * n16 / grid, (b + 1) * n16 / grid) of 16-byte words, each lane with
// 8 non-temporal dwordx4 loads in flight per trip (a wave covers 8 KB of
// consecutive lines per trip), and folds them into one word per wave so the
// loads cannot be dropped.
__global__ void __launch_bounds__(256) k_read_probe(const uint4 *p, int64_t n16, uint32_t *out)
{
    typedef unsigned int u4v __attribute__((ext_vector_type(4)));
    const u4v STYX_GLOBAL *q = (const u4v STYX_GLOBAL *)p;
    const int64_t c0 = n16 * blockIdx.x / gridDim.x, c1 = n16 * (blockIdx.x + 1) / gridDim.x;
    uint32_t acc = 0;
    int64_t i = c0 + threadIdx.x;
    for (; i + 7 * 256 < c1; i += 8 * 256) {
        u4v v[8];
#pragma unroll
        for (int j = 0; j < 8; j++) v[j] = __builtin_nontemporal_load(q + i + 256 * j);
#pragma unroll
        for (int j = 0; j < 8; j++) acc ^= v[j].x ^ v[j].y ^ v[j].z ^ v[j].w;
    }
    for (; i < c1; i += 256) {
        const u4v v = __builtin_nontemporal_load(q + i);
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    for (int o = 32; o > 0; o >>= 1) acc ^= __shfl_xor(acc, o);
    if ((threadIdx.x & 63) == 0) out[blockIdx.x * 4 + (threadIdx.x >> 6)] = acc;
}

hipError_t launch_read_probe(hipStream_t st, const void *p, int64_t bytes, uint32_t *out,
                             int grid)
{
    if (bytes < 16 || bytes % 16 || grid < 1 || grid > 65536) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_read_probe, dim3(grid), dim3(256), 0, st, (const uint4 *)p, bytes / 16,
                       out);
    return hipGetLastError();
}

hipError_t launch_fill_u32(hipStream_t st, uint32_t *p, uint32_t v, int64_t n)
{
    const int64_t nwg = std::min<int64_t>((n + 255) / 256, 4096);
    hipLaunchKernelGGL(k_fill_u32, dim3((unsigned)std::max<int64_t>(nwg, 1)), dim3(256), 0, st, p, v,
                       n);
    return hipGetLastError();
}

hipError_t launch_clamp_copy_u32(hipStream_t st, const uint32_t *src, uint32_t *dst, uint32_t maxv,
                                 int64_t n)
{
    const int64_t nwg = std::min<int64_t>((n + 255) / 256, 4096);
    hipLaunchKernelGGL(k_clamp_copy_u32, dim3((unsigned)std::max<int64_t>(nwg, 1)), dim3(256), 0, st,
                       src, dst, maxv, n);
    return hipGetLastError();
}

}  // namespace styx
