// attn.hip -- split-context decode attention over the paged f32 KV cache.
//
// Semantics follow shaders/attn_decode_f32.comp:31-79 (softmax(scale*q.K)V
// per query head, GQA kvh = h / gqa, K/V rows [t][kv_dim]) with the per-head
// q/k RMSNorm (crates/model/src/moe.rs:1875-1913), NEOX rope
// (crates/vk-backend/tests/ops2.rs:426-442, angle in f64) and the KV append
// at the current position (moe.rs:1932-1943) fused in front.
//
// Layout: one workgroup per (context chunk, kv head).  It loads its K/V rows
// once for all gqa query heads of that kv head (the reference re-reads them
// per query head), streams them through LDS in 32-token tiles with an online
// softmax, and writes a partial (m, l, o); k_attn_combine merges the
// partials in chunk order (a single active chunk writes the output itself).  The current position is read
// from device memory, so a captured graph serves every step; chunks past the
// context exit at once.
#include "kernels.h"
#include "qdot.h"

#include <algorithm>

namespace styx {

constexpr int AT_WG = 256;
constexpr int TT = 32;
constexpr int MAX_OWN = 8;  // outputs (g, i) per thread: gqa*hd <= 2048

__device__ __forceinline__ int64_t kv_off(const AttnArgs &a, int t, int kvh, int kv_dim)
{
    const int page = a.page_table[t / a.page_tokens];
    return ((int64_t)page * a.page_tokens + (t % a.page_tokens)) * kv_dim + (int64_t)kvh * a.hd;
}

// RMSNorm(hd) * w, then NEOX rope at pos, of one head held in src; one wave.
__device__ inline void norm_rope_head(const float *src, const float *w, float eps, int hd,
                                      const double *inv_freq, int pos, float *dst)
{
    const int lane = threadIdx.x & 63, half = hd / 2;
    float ss = 0.0f;
    for (int i = lane; i < hd; i += 64) ss += src[i] * src[i];
    ss = wave_sum(ss);
    const float scale = w ? 1.0f / sqrtf(ss / (float)hd + eps) : 1.0f;
    for (int i = lane; i < half; i += 64) {
        float x0 = src[i], x1 = src[i + half];
        if (w) {
            x0 = (x0 * scale) * w[i];
            x1 = (x1 * scale) * w[i + half];
        }
        const double th = (double)pos * inv_freq[i];
        const double sn = sin(th), cs = cos(th);
        dst[i] = (float)((double)x0 * cs - (double)x1 * sn);
        dst[i + half] = (float)((double)x0 * sn + (double)x1 * cs);
    }
}

__global__ void __launch_bounds__(AT_WG) k_attn(AttnArgs a)
{
    const int c = blockIdx.x, kvh = blockIdx.y;
    const int pos = *a.pos, n_t = pos + 1;
    const int t0 = c * a.chunk;
    if (t0 >= n_t) return;
    const int t1 = min(n_t, t0 + a.chunk);
    const int gqa = a.nh / a.nkv, hd = a.hd, kv_dim = a.nkv * hd, kp = hd + 4;
    const int n_active = (n_t + a.chunk - 1) / a.chunk;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;

    extern __shared__ __align__(16) float sm[];
    float *qs = sm;                   // [gqa][hd]
    float *kt = qs + gqa * hd;        // [TT][hd+4]
    float *vt = kt + TT * kp;         // [TT][hd]
    float *sc = vt + TT * hd;         // [gqa][TT]
    float *knew = sc + gqa * TT;      // [hd]
    float *vnew = knew + hd;          // [hd]
    float *mrun = vnew + hd;          // [gqa]
    float *lrun = mrun + 16;          // [gqa]
    float *corr = lrun + 16;          // [gqa]

    for (int g = wave; g < gqa; g += AT_WG / 64)
        norm_rope_head(a.q + (int64_t)(kvh * gqa + g) * hd, a.q_norm, a.eps, hd, a.inv_freq, pos,
                       qs + g * hd);
    const bool owns_pos = t1 == n_t;
    if (owns_pos && wave == 0) {
        norm_rope_head(a.k + (int64_t)kvh * hd, a.k_norm, a.eps, hd, a.inv_freq, pos, knew);
        for (int i = lane; i < hd; i += 64) vnew[i] = a.v[(int64_t)kvh * hd + i];
    }
    if (threadIdx.x < 16) {
        mrun[threadIdx.x] = -INFINITY;
        lrun[threadIdx.x] = 0.0f;
    }
    __syncthreads();
    if (owns_pos && wave == 0) {
        const int64_t o = kv_off(a, pos, kvh, kv_dim);
        for (int i = lane; i < hd; i += 64) {
            a.kpool[o + i] = knew[i];
            a.vpool[o + i] = vnew[i];
        }
    }

    const int nown = (gqa * hd + AT_WG - 1) / AT_WG;
    float acc[MAX_OWN];
#pragma unroll
    for (int j = 0; j < MAX_OWN; j++) acc[j] = 0.0f;

    const int hd4 = hd / 4;
    for (int ts = t0; ts < t1; ts += TT) {
        const int nt = min(TT, t1 - ts);
        for (int idx = threadIdx.x; idx < nt * hd4; idx += AT_WG) {
            const int row = idx / hd4, c4 = idx - row * hd4, t = ts + row;
            float4 kv, vv;
            if (t == pos) {
                kv = *(const float4 *)(knew + 4 * c4);
                vv = *(const float4 *)(vnew + 4 * c4);
            } else {
                const int64_t o = kv_off(a, t, kvh, kv_dim) + 4 * c4;
                kv = *(const float4 *)(a.kpool + o);
                vv = *(const float4 *)(a.vpool + o);
            }
            *(float4 *)(kt + row * kp + 4 * c4) = kv;
            *(float4 *)(vt + row * hd + 4 * c4) = vv;
        }
        __syncthreads();
        for (int p = threadIdx.x; p < gqa * nt; p += AT_WG) {
            const int g = p / nt, t = p - g * nt;
            const float4 *qv = (const float4 *)(qs + g * hd);
            const float4 *kr = (const float4 *)(kt + t * kp);
            float d = 0.0f;
            for (int i = 0; i < hd4; i++) {
                const float4 x = qv[i], y = kr[i];
                d += x.x * y.x + x.y * y.y + x.z * y.z + x.w * y.w;
            }
            sc[g * TT + t] = d * a.scale;
        }
        __syncthreads();
        for (int g = wave; g < gqa; g += AT_WG / 64) {
            const float s = lane < nt ? sc[g * TT + lane] : -INFINITY;
            const float mt = wave_max(s);
            const float m_old = mrun[g], m_new = fmaxf(m_old, mt);
            const float p = lane < nt ? expf(s - m_new) : 0.0f;
            const float ps = wave_sum(p);
            if (lane < nt) sc[g * TT + lane] = p;
            if (lane == 0) {
                const float cr = expf(m_old - m_new);
                corr[g] = cr;
                lrun[g] = lrun[g] * cr + ps;
                mrun[g] = m_new;
            }
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < MAX_OWN; j++) {
            if (j >= nown) break;
            const int o = threadIdx.x + j * AT_WG;
            if (o >= gqa * hd) break;
            const int g = o / hd, i = o - g * hd;
            float v = acc[j] * corr[g];
            for (int t = 0; t < nt; t++) v += sc[g * TT + t] * vt[t * hd + i];
            acc[j] = v;
        }
        __syncthreads();
    }

    if (n_active == 1) {
#pragma unroll
        for (int j = 0; j < MAX_OWN; j++) {
            const int o = threadIdx.x + j * AT_WG;
            if (j >= nown || o >= gqa * hd) break;
            const int g = o / hd;
            a.out[(int64_t)kvh * gqa * hd + o] = acc[j] * (1.0f / lrun[g]);
        }
        return;
    }
    const int ps = hd + 2;
    float *part = a.part + ((int64_t)kvh * a.max_chunks + c) * gqa * ps;
#pragma unroll
    for (int j = 0; j < MAX_OWN; j++) {
        const int o = threadIdx.x + j * AT_WG;
        if (j >= nown || o >= gqa * hd) break;
        const int g = o / hd, i = o - g * hd;
        part[g * ps + i] = acc[j];
    }
    if (threadIdx.x < gqa) {
        part[threadIdx.x * ps + hd] = mrun[threadIdx.x];
        part[threadIdx.x * ps + hd + 1] = lrun[threadIdx.x];
    }
}

// Merge the per-chunk partials (m, l, o) of one query head in chunk order:
// M = max m_c, L = sum l_c e^(m_c-M), out = sum o_c e^(m_c-M) / L.
__global__ void __launch_bounds__(256) k_attn_combine(AttnArgs a)
{
    const int h = blockIdx.x, gqa = a.nh / a.nkv, hd = a.hd, ps = hd + 2;
    const int n_t = *a.pos + 1;
    const int n_active = (n_t + a.chunk - 1) / a.chunk;
    if (n_active == 1) return;  // the single chunk wrote the output itself
    const int kvh = h / gqa, g = h - kvh * gqa;
    const float *pk = a.part + (int64_t)kvh * a.max_chunks * gqa * ps + (int64_t)g * ps;
    for (int i = threadIdx.x; i < hd; i += blockDim.x) {
        float M = -INFINITY;
        for (int cc = 0; cc < n_active; cc++) M = fmaxf(M, pk[(int64_t)cc * gqa * ps + hd]);
        float L = 0.0f, O = 0.0f;
        for (int cc = 0; cc < n_active; cc++) {
            const float *pp = pk + (int64_t)cc * gqa * ps;
            const float f = expf(pp[hd] - M);
            L += pp[hd + 1] * f;
            O += pp[i] * f;
        }
        a.out[(int64_t)h * hd + i] = O / L;
    }
}

hipError_t launch_attn_decode(hipStream_t st, const AttnArgs &a)
{
    const int gqa = a.nkv > 0 ? a.nh / a.nkv : 0;
    if (gqa < 1 || gqa > 16 || a.nh % a.nkv || a.hd % 4 || a.hd > 256 ||
        gqa * a.hd > MAX_OWN * AT_WG || a.chunk % TT || a.page_tokens % TT)
        return hipErrorInvalidValue;
    const size_t lds =
        sizeof(float) * ((size_t)gqa * a.hd + TT * (a.hd + 4) + TT * a.hd + gqa * TT + 2 * a.hd + 48);
    hipLaunchKernelGGL(k_attn, dim3(a.max_chunks, a.nkv), dim3(AT_WG), lds, st, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || a.max_chunks == 1) return e;
    hipLaunchKernelGGL(k_attn_combine, dim3(a.nh), dim3(std::min(256, a.hd)), 0, st, a);
    return hipGetLastError();
}

}  // namespace styx
