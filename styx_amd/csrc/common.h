// common.h -- shared host/device definitions for libstyx_hip.
//
// Block formats are GGUF's (crates/gguf-rs/src/lib.rs:242-332).  In HBM the
// engine keeps every quant matrix in a "split" layout: the same bytes as the
// GGUF blocks, regrouped per matrix into aligned regions (quants, high bits,
// scales, f16 factors) so that every lane issues 16-byte loads, and inside
// the quant regions interleaved (ilv_off) so that the 16-byte loads of
// neighbouring lanes cover whole 128-byte lines.  The regrouping is a byte
// permutation: dequantized values are bit-identical.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

namespace styx {

// Global-memory pointers for device code: loads and stores through them are
// global_* instructions even when the pointer value comes from LDS or a
// computed struct (a generic pointer would give flat_* instructions, which
// also count against the LDS wait counter).  The vector types are clang's
// ext_vector_type so that both compilation passes accept the qualified
// loads.
#define STYX_GLOBAL __attribute__((address_space(1)))
typedef unsigned styx_u4 __attribute__((ext_vector_type(4)));
typedef unsigned styx_u2 __attribute__((ext_vector_type(2)));
typedef float styx_f4 __attribute__((ext_vector_type(4)));

enum QType : int { T_F32 = 0, T_F16 = 1, T_Q8_0 = 8, T_Q4_K = 12, T_Q5_K = 13, T_Q6_K = 14 };

constexpr uint32_t SKIP = 0xFFFFFFFFu;
constexpr int MAX_TOPK = 16;
constexpr int MAX_EXPERTS = 512;
constexpr int IDS_ROW = 64;  // int32 per layer id row (256 B), moe.rs:1114-1168

__host__ __device__ inline int blk_elems(int t)
{
    return t == T_Q8_0 ? 32 : (t == T_Q4_K || t == T_Q5_K || t == T_Q6_K) ? 256 : 1;
}
__host__ __device__ inline int blk_bytes(int t)
{
    switch (t) {
    case T_F32: return 4;
    case T_F16: return 2;
    case T_Q8_0: return 34;
    case T_Q4_K: return 144;
    case T_Q5_K: return 176;
    case T_Q6_K: return 210;
    default: return 0;
    }
}
__host__ __device__ inline bool is_quant(int t)
{
    return t == T_Q8_0 || t == T_Q4_K || t == T_Q5_K || t == T_Q6_K;
}
// Work units per block: one q8_0 block (32 values) or a quarter K-block (64 values).
__host__ __device__ inline int units_per_blk(int t) { return t == T_Q8_0 ? 1 : 4; }

// Split layout: up to 4 regions per matrix, each an array over (row, block)
// of a fixed per-block byte size, row-major.
struct Split {
    int nreg;
    int sz[4];    // bytes per block in region r
    int src[4];   // byte offset of region r's bytes inside a GGUF block
};

__host__ __device__ inline Split split_of(int t)
{
    Split s{};
    switch (t) {
    case T_Q8_0:  // qs[32] | d
        s.nreg = 2; s.sz[0] = 32; s.src[0] = 2; s.sz[1] = 2; s.src[1] = 0;
        break;
    case T_Q4_K:  // qs[128] | {d, dmin, scales[12]}
        s.nreg = 2; s.sz[0] = 128; s.src[0] = 16; s.sz[1] = 16; s.src[1] = 0;
        break;
    case T_Q5_K:  // qs[128] | qh[32] | {d, dmin, scales[12]}
        s.nreg = 3; s.sz[0] = 128; s.src[0] = 48; s.sz[1] = 32; s.src[1] = 16;
        s.sz[2] = 16; s.src[2] = 0;
        break;
    case T_Q6_K:  // ql[128] | qh[64] | scales[16] | d
        s.nreg = 4; s.sz[0] = 128; s.src[0] = 0; s.sz[1] = 64; s.src[1] = 128;
        s.sz[2] = 16; s.src[2] = 192; s.sz[3] = 2; s.src[3] = 208;
        break;
    default:  // f32 / f16: one region, identity
        s.nreg = 1; s.sz[0] = blk_bytes(t); s.src[0] = 0;
        break;
    }
    return s;
}

// Byte offset of region r inside a matrix of nblocks (rows*blocks-per-row) blocks.
__host__ __device__ inline int64_t region_off(const Split &s, int r, int64_t nblocks)
{
    int64_t o = 0;
    for (int i = 0; i < r; i++) o += (int64_t)s.sz[i] * nblocks;
    return o;
}

// Place of byte i (0 <= i < sz[r]) of block b inside region r.  A unit
// load reads 16 bytes of one block's quant region, and a wave's neighbouring
// lanes read the same 16-byte position of neighbouring units, so those
// halves are stored side by side:
//   - 32-byte regions (q8_0 quants, q5_K high bits), groups of 8 blocks: the
//     first 16 bytes of the 8 blocks, then their last 16 bytes;
//   - 128-byte regions (q4_K / q5_K quants, q6_K low bits), pairs of blocks:
//     each block is four units, unit v reading bytes [16 v', +16) and
//     [16 v' + 32, +16) of its 64-byte half (q6_K: v = 2n + h, runs
//     64n + 16h and +32) or [32 v, +16) and [32 v + 16, +16) (q4_K / q5_K
//     quarter v): per pair, the first load of all 8 units, then the second.
// Every other region keeps the blocks' bytes in order.  A matrix's block
// count must be a multiple of ilv_group(t).
__host__ __device__ inline int64_t ilv_off(int t, int r, int64_t b, int i)
{
    if (r == 0 && (t == T_Q4_K || t == T_Q5_K))
        return (b >> 1) * 256 + ((i >> 4) & 1) * 128 + (b & 1) * 64 + (i >> 5) * 16 + (i & 15);
    if (r == 0 && t == T_Q6_K)
        return (b >> 1) * 256 + ((i >> 5) & 1) * 128 + (b & 1) * 64 +
               (2 * (i >> 6) + ((i >> 4) & 1)) * 16 + (i & 15);
    if ((r == 0 && t == T_Q8_0) || (r == 1 && t == T_Q5_K))
        return (b >> 3) * 256 + (i >> 4) * 128 + (b & 7) * 16 + (i & 15);
    return b * split_of(t).sz[r] + i;
}

// Blocks per interleave group of type t (ilv_off): a matrix's block count
// must be a multiple of it.
__host__ __device__ inline int ilv_group(int t)
{
    return t == T_Q8_0 || t == T_Q5_K ? 8 : t == T_Q4_K || t == T_Q6_K ? 2 : 1;
}

// Map GGUF byte index (block b, byte i) of a matrix with nblocks blocks to its
// split-layout byte index.
__host__ __device__ inline int64_t split_index(int t, const Split &s, int64_t nblocks, int64_t b,
                                               int i)
{
    for (int r = 0; r < s.nreg; r++) {
        if (i >= s.src[r] && i < s.src[r] + s.sz[r]) {
            return region_off(s, r, nblocks) + ilv_off(t, r, b, i - s.src[r]);
        }
    }
    return -1;
}

// Greedy-sampling order as one unsigned 64-bit key: f32::total_cmp of the
// value in the high word (sign-magnitude bits made two's-complement order,
// then offset to unsigned), the row index in the low word, so the larger key
// is the larger value and, between equal values, the later row
// (Iterator::max_by keeps the last maximum, generate_moe.rs:29).  0 is below
// every key of a real row but the lowest NaN at row 0.
__device__ __forceinline__ unsigned long long argmax_key(float v, uint32_t idx)
{
    const int32_t b = __float_as_int(v);
    const uint32_t k = (uint32_t)(b ^ (int32_t)(((uint32_t)(b >> 31)) >> 1)) ^ 0x80000000u;
    return ((unsigned long long)k << 32) | idx;
}

// ----------------------------------------------------------------------------
// Activation limbs ("xq") of an n-value vector (n a multiple of 32): int8
// planes A, B, C with x ~= sx * (A + (B + C/254)/254), sx = max|x|/127 per 32
// values, plus s16 = plain f32 sums over runs of 16 values (for the
// per-sub-block offset terms of the K-quants).  One contiguous buffer:
//   A[n] | B[n] | C[n] | sx[n/32] f32 | s16[n/16] f32
// Written once by the kernel that produces the vector, read by every matvec
// lane that needs a slice of it.
// ----------------------------------------------------------------------------
constexpr int XQ_MAX = 16384;  // longest vector with limbs

struct Xq {
    int8_t *A, *B, *C;
    float *sx, *s16;
};

__host__ __device__ inline size_t xq_bytes(int n)
{
    return (size_t)3 * n + (size_t)(n / 32) * 4 + (size_t)(n / 16) * 4;
}

__host__ __device__ inline Xq xq_at(void *base, int n)
{
    Xq q;
    q.A = (int8_t *)base;
    q.B = q.A + n;
    q.C = q.B + n;
    q.sx = (float *)((uint8_t *)base + 3 * (size_t)n);
    q.s16 = q.sx + n / 32;
    return q;
}

// The same vector seen from element e0 (a multiple of 32) on.
__host__ __device__ inline Xq xq_shift(const Xq &q, int e0)
{
    Xq r;
    r.A = q.A + e0;
    r.B = q.B + e0;
    r.C = q.C + e0;
    r.sx = q.sx + e0 / 32;
    r.s16 = q.s16 + e0 / 16;
    return r;
}

}  // namespace styx
