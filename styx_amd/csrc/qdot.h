// qdot.h -- device-side dequant dot products for the split quant layout.
//
// A matvec row is cut into "units": one q8_0 block (32 values) or a quarter of
// a K-quant block (64 values).  A lane group of G lanes owns a row; lane gl
// owns units gl, gl+G, ... and keeps the activation values for those units in
// registers for every row it visits (the activations are the same for all
// rows).  Activations are held as three int8 limbs per value,
//     x ~= sx * (a + (b + c/254)/254),   sx = max|x| / 127 per 32 values,
// which carries ~23 bits -- f32-class accuracy -- and lets the inner loop be
// one v_dot4c_i32_i8 per 4 quant values per limb, instead of a convert and an
// FMA per value.  Quant values of every format are small non-negative or
// signed integers that fit int8 unchanged.
#pragma once

#include "common.h"

namespace styx {

constexpr float R254 = 1.0f / 254.0f;

__device__ __forceinline__ float f16f(uint32_t h)
{
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(h & 0xFFFFu));
}

__device__ __forceinline__ int sdot4(uint32_t a, uint32_t b, int c)
{
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

__device__ __forceinline__ float limbs_to_f(int A, int B, int C)
{
    return (float)A + ((float)B + (float)C * R254) * R254;
}

// Butterfly reductions over aligned blocks of G = 2, 4, ..., 64 lanes in
// VALU operations only (DPP lane permutes, then the gfx950 row swaps), no
// LDS round trips.  Each step pairs every lane with one partner of the other
// half of its block and combines the two values; the partner combines the
// same two values, so after the last step every lane of the block holds the
// same bits.  Steps: quad_perm [1,0,3,2], quad_perm [2,3,0,1],
// row_half_mirror (lane i <-> 7-i of each 8), row_mirror (i <-> 15-i of each
// 16), v_permlane16_swap (rows 0<->1, 2<->3), v_permlane32_swap (halves).
template <int CTRL> __device__ __forceinline__ float dpp_f(float v)
{
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, true));
}
template <int G, typename Op> __device__ __forceinline__ float bfly(float v, Op op)
{
    static_assert(G >= 1 && G <= 64 && (G & (G - 1)) == 0, "power of two <= 64");
    if constexpr (G >= 2) v = op(v, dpp_f<0xB1>(v));
    if constexpr (G >= 4) v = op(v, dpp_f<0x4E>(v));
    if constexpr (G >= 8) v = op(v, dpp_f<0x141>(v));
    if constexpr (G >= 16) v = op(v, dpp_f<0x140>(v));
    if constexpr (G >= 32) {
        // one of the pair holds row 2j's value in both rows, the other row 2j+1's
        const auto s = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        v = op(__uint_as_float(s[0]), __uint_as_float(s[1]));
    }
    if constexpr (G >= 64) {
        const auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        v = op(__uint_as_float(s[0]), __uint_as_float(s[1]));
    }
    return v;
}
template <int G> __device__ __forceinline__ float bfly_sum(float v)
{
    return bfly<G>(v, [](float a, float b) { return a + b; });
}

__device__ __forceinline__ float wave_sum(float v) { return bfly_sum<64>(v); }
__device__ __forceinline__ float wave_max(float v)
{
    return bfly<64>(v, [](float a, float b) { return fmaxf(a, b); });
}

// Block-wide sum (blockDim.x multiple of 64, <= 1024).  All threads get it.
// NT: the workgroup's thread count when the caller knows it (0: read
// blockDim.x, which in some kernels becomes a vector load of the dispatch
// packet whose wait also waits for every store in flight).
template <int NT = 0> __device__ inline float block_sum(float v, float *red)
{
    v = wave_sum(v);
    const int w = threadIdx.x >> 6, nw = (NT ? NT : (int)blockDim.x) >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    float t = 0.0f;
    for (int i = 0; i < nw; i++) t += red[i];
    return t;
}

// The three int8 limbs of four values v scaled by inv, packed four to a
// dword (value i in byte i):
//   a = rint(v inv), d = v inv - a (one fused rounding),
//   b = rint(254 d), c = rint(254 (254 d - b)) (the inner one fused).
// Every rounding adds 1.5 * 2^23: the sum is the value rounded to the
// nearest integer, ties to even (as rintf), and its low byte is that
// integer as an int8; subtracting 1.5 * 2^23 again gives the rounded value
// exactly.  |v inv| <= 127 (inv = 127 / max |v|) and |d|, |254 d - b| are
// within 1/2 of a unit, so every limb lies in [-127, 127].  Contraction is
// off: only the two fmaf calls fuse.
__device__ __forceinline__ uint32_t pack_low_bytes(const uint32_t (&t)[4])
{
    const uint32_t lo = __builtin_amdgcn_perm(t[1], t[0], 0x0c0c0400u);
    const uint32_t hi = __builtin_amdgcn_perm(t[3], t[2], 0x0c0c0400u);
    return __builtin_amdgcn_perm(hi, lo, 0x05040100u);
}
__device__ __forceinline__ void limbs3x4(const float *v, float inv, uint32_t &pa, uint32_t &pb,
                                         uint32_t &pc)
{
#pragma clang fp contract(off)
    constexpr float M = 12582912.0f;
    uint32_t ta[4], tb[4], tc[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float t1 = v[i] * inv + M;
        const float d = fmaf(v[i], inv, -(t1 - M));
        const float t2 = d * 254.0f + M;
        const float t3 = fmaf(d, 254.0f, -(t2 - M)) * 254.0f + M;
        ta[i] = __float_as_uint(t1);
        tb[i] = __float_as_uint(t2);
        tc[i] = __float_as_uint(t3);
    }
    pa = pack_low_bytes(ta);
    pb = pack_low_bytes(tb);
    pc = pack_low_bytes(tc);
}

// Limbs of one group of 8 consecutive values (group g of the vector q).
// Four consecutive lanes hold the four groups of one 32-value block (groups
// are 4-aligned); all four must call this together.  Inactive groups pass
// zeros and write nothing.
__device__ __forceinline__ void xq_group(const float *v, bool act, int g, Xq q)
{
    float am = 0.0f, s8 = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        am = fmaxf(am, fabsf(v[i]));
        s8 += v[i];
    }
    // groups g^1, g^2 are the neighbouring lanes of a quad (callers run whole quads)
    am = fmaxf(am, dpp_f<0xB1>(am));
    am = fmaxf(am, dpp_f<0x4E>(am));
    const float s16 = s8 + dpp_f<0xB1>(s8);
    if (!act) return;
    const float inv = am > 0.0f ? 127.0f / am : 0.0f;
    uint32_t pa[2], pb[2], pc[2];
    limbs3x4(v, inv, pa[0], pb[0], pc[0]);
    limbs3x4(v + 4, inv, pa[1], pb[1], pc[1]);
    *(uint2 *)(q.A + 8 * g) = make_uint2(pa[0], pa[1]);
    *(uint2 *)(q.B + 8 * g) = make_uint2(pb[0], pb[1]);
    *(uint2 *)(q.C + 8 * g) = make_uint2(pc[0], pc[1]);
    if ((g & 3) == 0) q.sx[g >> 2] = am / 127.0f;
    if ((g & 1) == 0) q.s16[g >> 1] = s16;
}

// The same for a group of 4 values (group g of the vector q): eight
// consecutive lanes hold one 32-value block (groups 8-aligned), and all
// eight must call this together.  Twice the threads of xq_group for half
// the values each: for vectors of at most 4 values per thread.
__device__ __forceinline__ void xq_group4(const float *v, bool act, int g, Xq q)
{
    float am = 0.0f, s4 = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        am = fmaxf(am, fabsf(v[i]));
        s4 += v[i];
    }
    am = bfly<8>(am, [](float a, float b) { return fmaxf(a, b); });
    const float s16 = bfly_sum<4>(s4);
    if (!act) return;
    const float inv = am > 0.0f ? 127.0f / am : 0.0f;
    uint32_t pa, pb, pc;
    limbs3x4(v, inv, pa, pb, pc);
    *(uint32_t *)(q.A + 4 * g) = pa;
    *(uint32_t *)(q.B + 4 * g) = pb;
    *(uint32_t *)(q.C + 4 * g) = pc;
    if ((g & 7) == 0) q.sx[g >> 3] = am / 127.0f;
    if ((g & 3) == 0) q.s16[g >> 2] = s16;
}

// xq_group4 with the group's limbs written straight to the limb buffer q
// (shifted to the vector's element e0) and published as tagged words in t,
// laid out as the 32-bit words of xq_at(., N): A | B | C | sx | s16 (the
// layout of xq_publish), with no LDS pass.  tput is the caller's tagged
// store (xchg.h).
template <typename Put>
__device__ __forceinline__ void xq_group4_put(const float *v, bool act, int g, Xq q, int N, int e0,
                                              Put tput)
{
    float am = 0.0f, s4 = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        am = fmaxf(am, fabsf(v[i]));
        s4 += v[i];
    }
    am = bfly<8>(am, [](float a, float b) { return fmaxf(a, b); });
    const float s16 = bfly_sum<4>(s4);
    if (!act) return;
    const float inv = am > 0.0f ? 127.0f / am : 0.0f;
    uint32_t pa, pb, pc;
    limbs3x4(v, inv, pa, pb, pc);
    const int N4 = N / 4, o = e0 / 4 + g;
    *(uint32_t *)(q.A + 4 * g) = pa;
    *(uint32_t *)(q.B + 4 * g) = pb;
    *(uint32_t *)(q.C + 4 * g) = pc;
    tput(o, pa);
    tput(N4 + o, pb);
    tput(2 * N4 + o, pc);
    if ((g & 7) == 0) {
        const float sx = am / 127.0f;
        q.sx[g >> 3] = sx;
        tput(3 * N4 + e0 / 32 + (g >> 3), __float_as_uint(sx));
    }
    if ((g & 3) == 0) {
        q.s16[g >> 2] = s16;
        tput(3 * N4 + N / 32 + e0 / 16 + (g >> 2), __float_as_uint(s16));
    }
}

// Build the limb form of xn = norm ? x * rsqrt(mean(x^2)+eps) * w : x
// (n a multiple of 32).  If xn_out is non-null the normalised f32 vector is
// also written there.  Thread t owns 8 consecutive values per pass.
// NT: the workgroup's thread count if known at compile time (see block_sum).
template <int NT = 0>
__device__ inline void xq_build(const float *__restrict__ x, const float *__restrict__ nw,
                                float eps, bool norm, int n, Xq q, float *red, float *xn_out)
{
    const int nt = NT ? NT : (int)blockDim.x;
    float scale = 1.0f;
    if (norm) {
        float ss = 0.0f;
        for (int i = threadIdx.x * 4; i < n; i += nt * 4) {
            const float4 v = *(const float4 *)(x + i);
            ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
        }
        ss = block_sum<NT>(ss, red);
        scale = 1.0f / sqrtf(ss / (float)n + eps);
    }
    if (n <= 4 * nt) {
        // a short vector: four values per thread, more threads at work
        const int g = threadIdx.x;
        const bool act = g < n / 4;
        float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        if (act) {
            const float4 a = *(const float4 *)(x + 4 * g);
            v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
            if (norm) {
                const float4 wa = *(const float4 *)(nw + 4 * g);
                v[0] = (v[0] * scale) * wa.x;
                v[1] = (v[1] * scale) * wa.y;
                v[2] = (v[2] * scale) * wa.z;
                v[3] = (v[3] * scale) * wa.w;
            }
            if (xn_out) *(float4 *)(xn_out + 4 * g) = make_float4(v[0], v[1], v[2], v[3]);
        }
        xq_group4(v, act, g, q);
        return;
    }
    const int ngroups = n / 8;
    for (int g0 = 0; g0 < ngroups; g0 += nt) {
        const int g = g0 + threadIdx.x;
        const bool act = g < ngroups;
        float v[8];
        if (act) {
            const float4 a = *(const float4 *)(x + 8 * g), b = *(const float4 *)(x + 8 * g + 4);
            v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
            v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
            if (norm) {
                const float4 wa = *(const float4 *)(nw + 8 * g), wb = *(const float4 *)(nw + 8 * g + 4);
                const float w[8] = {wa.x, wa.y, wa.z, wa.w, wb.x, wb.y, wb.z, wb.w};
#pragma unroll
                for (int i = 0; i < 8; i++) v[i] = (v[i] * scale) * w[i];
            }
            if (xn_out) {
                *(float4 *)(xn_out + 8 * g) = make_float4(v[0], v[1], v[2], v[3]);
                *(float4 *)(xn_out + 8 * g + 4) = make_float4(v[4], v[5], v[6], v[7]);
            }
        } else {
#pragma unroll
            for (int i = 0; i < 8; i++) v[i] = 0.0f;
        }
        xq_group(v, act, g, q);
    }
}

// ----------------------------------------------------------------------------
// Per-format unit operands.
//   q8_0 unit  = block b (32 values at 32b).
//   q4_K/q5_K  = quarter c of block b: values 256b+64c .. +63
//                (low nibbles -> first 32, high nibbles -> next 32).
//   q6_K       = quarter u=(n=u>>1, h=u&1) of block b: four runs of 16 values
//                at 256b + 128n + 16h + 32r, r = 0..3.
// ----------------------------------------------------------------------------
template <int T> struct UX;
template <> struct UX<T_Q8_0> {
    uint32_t a[8], b[8], c[8];
    float sx;
};
template <> struct UX<T_Q4_K> {
    uint32_t a[16], b[16], c[16];
    float sx[2], s[2];
    int sh;     // byte shift of this quarter's scale pair (0 or 16)
    int high;   // quarters 2,3 use the 6-bit packed high scales
};
template <> struct UX<T_Q5_K> {
    uint32_t a[16], b[16], c[16];
    float sx[2], s[2];
    int sh, high, qsh;  // qsh = 2c: qh bit of the low nibbles
};
template <> struct UX<T_Q6_K> {
    uint32_t a[16], b[16], c[16];
    float sx[4], s[4];
    int h, n;
};

__device__ __forceinline__ void ld_limbs(const Xq &q, int e, int ndw, uint32_t *a,
                                         uint32_t *b, uint32_t *c)
{
    for (int i = 0; i < ndw; i += 4) {
        const uint4 va = *(const uint4 *)(q.A + e + 4 * i);
        const uint4 vb = *(const uint4 *)(q.B + e + 4 * i);
        const uint4 vc = *(const uint4 *)(q.C + e + 4 * i);
        a[i] = va.x; a[i + 1] = va.y; a[i + 2] = va.z; a[i + 3] = va.w;
        b[i] = vb.x; b[i + 1] = vb.y; b[i + 2] = vb.z; b[i + 3] = vb.w;
        c[i] = vc.x; c[i + 1] = vc.y; c[i + 2] = vc.z; c[i + 3] = vc.w;
    }
}

template <int T> __device__ inline void ux_load(UX<T> &u, const Xq &q, int unit);

template <> __device__ inline void ux_load<T_Q8_0>(UX<T_Q8_0> &u, const Xq &q, int unit)
{
    ld_limbs(q, 32 * unit, 8, u.a, u.b, u.c);
    u.sx = q.sx[unit];
}

template <> __device__ inline void ux_load<T_Q4_K>(UX<T_Q4_K> &u, const Xq &q, int unit)
{
    const int b = unit >> 2, c = unit & 3, e = 256 * b + 64 * c;
    ld_limbs(q, e, 16, u.a, u.b, u.c);
    u.sx[0] = q.sx[e / 32];
    u.sx[1] = q.sx[e / 32 + 1];
    u.s[0] = q.s16[e / 16] + q.s16[e / 16 + 1];
    u.s[1] = q.s16[e / 16 + 2] + q.s16[e / 16 + 3];
    u.sh = 16 * (c & 1);
    u.high = c >> 1;
}

template <> __device__ inline void ux_load<T_Q5_K>(UX<T_Q5_K> &u, const Xq &q, int unit)
{
    const int b = unit >> 2, c = unit & 3, e = 256 * b + 64 * c;
    ld_limbs(q, e, 16, u.a, u.b, u.c);
    u.sx[0] = q.sx[e / 32];
    u.sx[1] = q.sx[e / 32 + 1];
    u.s[0] = q.s16[e / 16] + q.s16[e / 16 + 1];
    u.s[1] = q.s16[e / 16 + 2] + q.s16[e / 16 + 3];
    u.sh = 16 * (c & 1);
    u.high = c >> 1;
    u.qsh = 2 * c;
}

template <> __device__ inline void ux_load<T_Q6_K>(UX<T_Q6_K> &u, const Xq &q, int unit)
{
    const int b = unit >> 2, n = (unit >> 1) & 1, h = unit & 1;
    const int e0 = 256 * b + 128 * n + 16 * h;
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const int e = e0 + 32 * r;
        ld_limbs(q, e, 4, u.a + 4 * r, u.b + 4 * r, u.c + 4 * r);
        u.sx[r] = q.sx[e / 32];
        u.s[r] = q.s16[e / 16];
    }
    u.h = h;
    u.n = n;
}

// ----------------------------------------------------------------------------
// Per-format weight operands of one unit, and their byte offsets inside a
// matrix in split layout.  `blk` = row * nb + block.
// ----------------------------------------------------------------------------
template <int T> struct UW;
template <> struct UW<T_Q8_0> { uint4 q0, q1; uint32_t d; };
template <> struct UW<T_Q4_K> { uint4 q0, q1, hd; };
template <> struct UW<T_Q5_K> { uint4 q0, q1, h0, h1, hd; };
template <> struct UW<T_Q6_K> { uint4 p0, p1, qh; uint2 sc; uint32_t d; };

// Region base pointers of one matrix (rows x nb blocks) in split layout.
struct Mat {
    const uint8_t STYX_GLOBAL *r0, *r1, *r2, *r3;
};

__device__ __forceinline__ Mat mat_at(const uint8_t *base, int t, int64_t nblocks)
{
    const Split s = split_of(t);
    Mat m;
    const uint8_t STYX_GLOBAL *g = (const uint8_t STYX_GLOBAL *)base;
    m.r0 = g;
    m.r1 = g + region_off(s, 1, nblocks);
    m.r2 = s.nreg > 2 ? g + region_off(s, 2, nblocks) : nullptr;
    m.r3 = s.nreg > 3 ? g + region_off(s, 3, nblocks) : nullptr;
    return m;
}

__device__ __forceinline__ uint4 ldg16(const uint8_t STYX_GLOBAL *p)
{
    const styx_u4 v = __builtin_nontemporal_load((const styx_u4 STYX_GLOBAL *)p);
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint32_t ldg2(const uint8_t STYX_GLOBAL *p)
{
    return __builtin_nontemporal_load((const uint16_t STYX_GLOBAL *)p);
}

template <int T> __device__ inline void uw_load(UW<T> &w, const Mat &m, int64_t blk, int sub);

// The quant regions are interleaved (ilv_off): the first 16 bytes of a
// 32-byte region sit at ilv8(blk), its last 16 bytes 128 bytes later; the
// two loads of unit v of a 128-byte region at ilv2(blk) + 16 v and 128
// bytes later.
__device__ __forceinline__ int64_t ilv8(int64_t blk) { return (blk >> 3) * 256 + (blk & 7) * 16; }
__device__ __forceinline__ int64_t ilv2(int64_t blk) { return (blk >> 1) * 256 + (blk & 1) * 64; }

template <> __device__ inline void uw_load<T_Q8_0>(UW<T_Q8_0> &w, const Mat &m, int64_t blk, int)
{
    const uint8_t STYX_GLOBAL *q = m.r0 + ilv8(blk);
    w.q0 = ldg16(q);
    w.q1 = ldg16(q + 128);
    w.d = ldg2(m.r1 + blk * 2);
}
template <> __device__ inline void uw_load<T_Q4_K>(UW<T_Q4_K> &w, const Mat &m, int64_t blk, int c)
{
    const uint8_t STYX_GLOBAL *q = m.r0 + ilv2(blk) + 16 * c;
    w.q0 = ldg16(q);
    w.q1 = ldg16(q + 128);
    w.hd = ldg16(m.r1 + blk * 16);
}
template <> __device__ inline void uw_load<T_Q5_K>(UW<T_Q5_K> &w, const Mat &m, int64_t blk, int c)
{
    const uint8_t STYX_GLOBAL *q = m.r0 + ilv2(blk) + 16 * c;
    w.q0 = ldg16(q);
    w.q1 = ldg16(q + 128);
    const uint8_t STYX_GLOBAL *h = m.r1 + ilv8(blk);
    w.h0 = ldg16(h);
    w.h1 = ldg16(h + 128);
    w.hd = ldg16(m.r2 + blk * 16);
}
template <> __device__ inline void uw_load<T_Q6_K>(UW<T_Q6_K> &w, const Mat &m, int64_t blk, int u)
{
    const int n = (u >> 1) & 1, h = u & 1;
    const uint8_t STYX_GLOBAL *ql = m.r0 + ilv2(blk) + 16 * u;
    w.p0 = ldg16(ql);
    w.p1 = ldg16(ql + 128);
    w.qh = ldg16(m.r1 + blk * 64 + 32 * n + 16 * h);
    const styx_u2 sc = *(const styx_u2 STYX_GLOBAL *)(m.r2 + blk * 16 + 8 * n);
    w.sc = make_uint2(sc.x, sc.y);
    w.d = ldg2(m.r3 + blk * 2);
}

__device__ __forceinline__ void u4_to(const uint4 v, uint32_t *o)
{
    o[0] = v.x; o[1] = v.y; o[2] = v.z; o[3] = v.w;
}

// q4_K / q5_K scale+min pair for quarter c (get_scale_min at 2c, 2c+1;
// crates/model/src/moe.rs:513-522), from the header dwords y,z,w.
__device__ __forceinline__ void k4_scales(const uint4 hd, int sh, int high, float &sc_lo,
                                          float &sc_hi, float &m_lo, float &m_hi)
{
    const uint32_t A = (hd.y >> sh) & 0xFFFFu, B = (hd.z >> sh) & 0xFFFFu,
                   C = (hd.w >> sh) & 0xFFFFu;
    uint32_t sc2, m2;
    if (high) {
        sc2 = (C & 0x0F0Fu) | ((A >> 2) & 0x3030u);
        m2 = ((C >> 4) & 0x0F0Fu) | ((B >> 2) & 0x3030u);
    } else {
        sc2 = A & 0x3F3Fu;
        m2 = B & 0x3F3Fu;
    }
    sc_lo = (float)(sc2 & 0xFFu);
    sc_hi = (float)(sc2 >> 8);
    m_lo = (float)(m2 & 0xFFu);
    m_hi = (float)(m2 >> 8);
}

// ---------------------------------------------------------------- dots ----
__device__ __forceinline__ float udot(const UW<T_Q8_0> &w, const UX<T_Q8_0> &x)
{
    uint32_t q[8];
    u4_to(w.q0, q);
    u4_to(w.q1, q + 4);
    int A = 0, B = 0, C = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        A = sdot4(q[i], x.a[i], A);
        B = sdot4(q[i], x.b[i], B);
        C = sdot4(q[i], x.c[i], C);
    }
    return (f16f(w.d) * x.sx) * limbs_to_f(A, B, C);
}

__device__ __forceinline__ float udot(const UW<T_Q4_K> &w, const UX<T_Q4_K> &x)
{
    uint32_t q[8];
    u4_to(w.q0, q);
    u4_to(w.q1, q + 4);
    int Al = 0, Bl = 0, Cl = 0, Ah = 0, Bh = 0, Ch = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const uint32_t lo = q[i] & 0x0F0F0F0Fu, hi = (q[i] >> 4) & 0x0F0F0F0Fu;
        Al = sdot4(lo, x.a[i], Al);
        Bl = sdot4(lo, x.b[i], Bl);
        Cl = sdot4(lo, x.c[i], Cl);
        Ah = sdot4(hi, x.a[8 + i], Ah);
        Bh = sdot4(hi, x.b[8 + i], Bh);
        Ch = sdot4(hi, x.c[8 + i], Ch);
    }
    float scl, sch, ml, mh;
    k4_scales(w.hd, x.sh, x.high, scl, sch, ml, mh);
    const float d = f16f(w.hd.x), dmin = f16f(w.hd.x >> 16);
    return (d * scl) * (x.sx[0] * limbs_to_f(Al, Bl, Cl)) - (dmin * ml) * x.s[0] +
           (d * sch) * (x.sx[1] * limbs_to_f(Ah, Bh, Ch)) - (dmin * mh) * x.s[1];
}

__device__ __forceinline__ float udot(const UW<T_Q5_K> &w, const UX<T_Q5_K> &x)
{
    uint32_t q[8], qh[8];
    u4_to(w.q0, q);
    u4_to(w.q1, q + 4);
    u4_to(w.h0, qh);
    u4_to(w.h1, qh + 4);
    int Al = 0, Bl = 0, Cl = 0, Ah = 0, Bh = 0, Ch = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const uint32_t hb = qh[i] >> x.qsh;
        const uint32_t lo = (q[i] & 0x0F0F0F0Fu) | ((hb & 0x01010101u) << 4);
        const uint32_t hi = ((q[i] >> 4) & 0x0F0F0F0Fu) | ((hb & 0x02020202u) << 3);
        Al = sdot4(lo, x.a[i], Al);
        Bl = sdot4(lo, x.b[i], Bl);
        Cl = sdot4(lo, x.c[i], Cl);
        Ah = sdot4(hi, x.a[8 + i], Ah);
        Bh = sdot4(hi, x.b[8 + i], Bh);
        Ch = sdot4(hi, x.c[8 + i], Ch);
    }
    float scl, sch, ml, mh;
    k4_scales(w.hd, x.sh, x.high, scl, sch, ml, mh);
    const float d = f16f(w.hd.x), dmin = f16f(w.hd.x >> 16);
    return (d * scl) * (x.sx[0] * limbs_to_f(Al, Bl, Cl)) - (dmin * ml) * x.s[0] +
           (d * sch) * (x.sx[1] * limbs_to_f(Ah, Bh, Ch)) - (dmin * mh) * x.s[1];
}

__device__ __forceinline__ float udot(const UW<T_Q6_K> &w, const UX<T_Q6_K> &x)
{
    uint32_t p0[4], p1[4], qh[4];
    u4_to(w.p0, p0);
    u4_to(w.p1, p1);
    u4_to(w.qh, qh);
    int A[4] = {0, 0, 0, 0}, B[4] = {0, 0, 0, 0}, C[4] = {0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t v[4] = {
            (p0[i] & 0x0F0F0F0Fu) | ((qh[i] << 4) & 0x30303030u),
            (p1[i] & 0x0F0F0F0Fu) | ((qh[i] << 2) & 0x30303030u),
            ((p0[i] >> 4) & 0x0F0F0F0Fu) | (qh[i] & 0x30303030u),
            ((p1[i] >> 4) & 0x0F0F0F0Fu) | ((qh[i] >> 2) & 0x30303030u),
        };
#pragma unroll
        for (int r = 0; r < 4; r++) {
            A[r] = sdot4(v[r], x.a[4 * r + i], A[r]);
            B[r] = sdot4(v[r], x.b[4 * r + i], B[r]);
            C[r] = sdot4(v[r], x.c[4 * r + i], C[r]);
        }
    }
    // scales[8n + h + {0,2,4,6}]: bytes h, h+2 of dwords sc.x (sc[8n..]) and sc.y
    const int b0 = 8 * x.h, b2 = 8 * x.h + 16;
    const float s0 = (float)(int8_t)(w.sc.x >> b0), s1 = (float)(int8_t)(w.sc.x >> b2);
    const float s2 = (float)(int8_t)(w.sc.y >> b0), s3 = (float)(int8_t)(w.sc.y >> b2);
    const float d = f16f(w.d);
    float acc = s0 * (x.sx[0] * limbs_to_f(A[0], B[0], C[0]) - 32.0f * x.s[0]);
    acc += s1 * (x.sx[1] * limbs_to_f(A[1], B[1], C[1]) - 32.0f * x.s[1]);
    acc += s2 * (x.sx[2] * limbs_to_f(A[2], B[2], C[2]) - 32.0f * x.s[2]);
    acc += s3 * (x.sx[3] * limbs_to_f(A[3], B[3], C[3]) - 32.0f * x.s[3]);
    return d * acc;
}

// Sum over the G lanes of a group; the group leader (gl == 0) gets the total.
// Groups are consecutive lanes [grp*G, grp*G+G); any 1 <= G <= 64.  A power
// of two (G is uniform) takes the butterfly, every lane getting the total.
__device__ __forceinline__ float group_sum(float v, int gl, int G)
{
    switch (G) {
    case 64: return bfly_sum<64>(v);
    case 32: return bfly_sum<32>(v);
    case 16: return bfly_sum<16>(v);
    case 8: return bfly_sum<8>(v);
    case 4: return bfly_sum<4>(v);
    case 2: return bfly_sum<2>(v);
    case 1: return v;
    default: break;
    }
    int off = 1;
    while (off * 2 < G) off *= 2;
    for (; off > 0; off >>= 1) {
        const float o = __shfl_down(v, off);
        if (gl + off < G) v += o;
    }
    return v;
}

}  // namespace styx
