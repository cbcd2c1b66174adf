// deq.h -- scalar dequantization of one block in the reference evaluation
// order, for the split layout (Mat) or a single GGUF block (gguf_blk).
#pragma once

#include "qdot.h"

namespace styx {

// Reference evaluation order of each format (crates/model/src/lib.rs:103-113,
// crates/model/src/moe.rs:506-533, ggml q5_K / q6_K): no contraction.
// Byte i of block blk's part of quant region r: interleaved in the split
// layout (ilv_off), in order in a single GGUF block.
__device__ __forceinline__ uint8_t qbyte(const uint8_t STYX_GLOBAL *reg, int t, int r, int64_t blk,
                                         int i, bool split)
{
    return split ? reg[ilv_off(t, r, blk, i)] : reg[blk * split_of(t).sz[r] + i];
}

#pragma clang fp contract(off)
__device__ __forceinline__ void deq_block(int t, const Mat &m, int64_t blk, float *y,
                                          bool split = true)
{
    if (t == T_Q8_0) {
        const float d = f16f(*(const uint16_t STYX_GLOBAL *)(m.r1 + blk * 2));
        for (int i = 0; i < 32; i++) y[i] = d * (float)(int8_t)qbyte(m.r0, t, 0, blk, i, split);
        return;
    }
    if (t == T_Q4_K || t == T_Q5_K) {
        const uint8_t STYX_GLOBAL *hd = (t == T_Q4_K ? m.r1 : m.r2) + blk * 16;
        const bool has_qh = t == T_Q5_K;
        const float d = f16f(hd[0] | (hd[1] << 8)), dmin = f16f(hd[2] | (hd[3] << 8));
        const uint8_t STYX_GLOBAL *sc = hd + 4;
        for (int j = 0; j < 4; j++) {
            float s1, m1, s2, m2;
            for (int h = 0; h < 2; h++) {
                const int jj = 2 * j + h;
                float a, b;
                if (jj < 4) {
                    a = (float)(sc[jj] & 63);
                    b = (float)(sc[jj + 4] & 63);
                } else {
                    a = (float)((sc[jj + 4] & 0x0F) | ((sc[jj - 4] >> 6) << 4));
                    b = (float)((sc[jj + 4] >> 4) | ((sc[jj] >> 6) << 4));
                }
                if (h == 0) { s1 = a; m1 = b; } else { s2 = a; m2 = b; }
            }
            const float d1 = d * s1, mm1 = dmin * m1, d2 = d * s2, mm2 = dmin * m2;
            for (int l = 0; l < 32; l++) {
                const uint8_t q = qbyte(m.r0, t, 0, blk, 32 * j + l, split);
                int lo = q & 0x0F, hi = q >> 4;
                if (has_qh) {
                    const uint8_t h = qbyte(m.r1, t, 1, blk, l, split);
                    lo += (h >> (2 * j)) & 1 ? 16 : 0;
                    hi += (h >> (2 * j + 1)) & 1 ? 16 : 0;
                }
                y[64 * j + l] = d1 * (float)lo - mm1;
                y[64 * j + 32 + l] = d2 * (float)hi - mm2;
            }
        }
        return;
    }
    if (t == T_Q6_K) {
        const float d = f16f(*(const uint16_t STYX_GLOBAL *)(m.r3 + blk * 2));
        for (int n = 0; n < 2; n++) {
            const uint8_t STYX_GLOBAL *qh = m.r1 + blk * 64 + 32 * n;
            const int8_t STYX_GLOBAL *sc = (const int8_t STYX_GLOBAL *)(m.r2 + blk * 16 + 8 * n);
            for (int l = 0; l < 32; l++) {
                const int is = l / 16;
                const uint8_t la = qbyte(m.r0, t, 0, blk, 64 * n + l, split),
                              lb = qbyte(m.r0, t, 0, blk, 64 * n + l + 32, split);
                const int q1 = (int)((la & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32;
                const int q2 = (int)((lb & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
                const int q3 = (int)((la >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                const int q4 = (int)((lb >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                y[128 * n + l] = d * (float)sc[is] * (float)q1;
                y[128 * n + l + 32] = d * (float)sc[is + 2] * (float)q2;
                y[128 * n + l + 64] = d * (float)sc[is + 4] * (float)q3;
                y[128 * n + l + 96] = d * (float)sc[is + 6] * (float)q4;
            }
        }
        return;
    }
    if (t == T_F32) {
        y[0] = *(const float STYX_GLOBAL *)(m.r0 + blk * 4);
        return;
    }
    if (t == T_F16) y[0] = f16f(*(const uint16_t STYX_GLOBAL *)(m.r0 + blk * 2));
}
#pragma clang fp contract(on)


// View of one GGUF-layout block as a one-block split matrix.
__device__ __forceinline__ Mat gguf_blk(const uint8_t *bp, int t)
{
    const uint8_t STYX_GLOBAL *b = (const uint8_t STYX_GLOBAL *)bp;
    Mat m{b, b, b, b};
    if (t == T_Q8_0) { m.r0 = b + 2; m.r1 = b; }
    else if (t == T_Q4_K) { m.r0 = b + 16; m.r1 = b; }
    else if (t == T_Q5_K) { m.r0 = b + 48; m.r1 = b + 16; m.r2 = b; }
    else if (t == T_Q6_K) { m.r0 = b; m.r1 = b + 128; m.r2 = b + 192; m.r3 = b + 208; }
    return m;
}

}  // namespace styx
