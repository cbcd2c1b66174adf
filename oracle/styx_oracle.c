/*
 * styx_oracle.c -- CPU restatement of the reference MoE decode path.
 * TEST INFRASTRUCTURE ONLY (see styx_oracle.h).  Build: oracle/Makefile
 * (-O2 -ffp-contract=off).  Each function cites the reference lines it
 * restates; the header records how each one is pinned.
 */
#include "styx_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static int g_threads = 1;

void styx_oracle_set_threads(int n) { g_threads = n < 1 ? 1 : n; }
int styx_oracle_get_threads(void) { return g_threads; }

/* ---------------------------------------------------------------- f16 -- */

float styx_oracle_f16_to_f32(uint16_t h)
{
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1Fu;
    uint32_t man = h & 0x3FFu;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else {
            /* subnormal: normalise into binary32 */
            int e = -1;
            do {
                man <<= 1;
                e++;
            } while ((man & 0x400u) == 0);
            man &= 0x3FFu;
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
        }
    } else if (exp == 0x1F) {
        bits = sign | 0x7F800000u | (man << 13);
    } else {
        bits = sign | ((exp + 127 - 15) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

static inline float rd_f16(const uint8_t *p)
{
    return styx_oracle_f16_to_f32((uint16_t)(p[0] | (p[1] << 8)));
}

/* --------------------------------------------------------- block table -- */

/* crates/gguf-rs/src/lib.rs:242-332 (subset on this path) */
int styx_oracle_block_elems(int type)
{
    switch (type) {
    case STYX_ORACLE_F32: return 1;
    case STYX_ORACLE_F16: return 1;
    case STYX_ORACLE_Q8_0: return 32;
    case STYX_ORACLE_Q4_K: return 256;
    case STYX_ORACLE_Q5_K: return 256;
    case STYX_ORACLE_Q6_K: return 256;
    default: return 0;
    }
}

int styx_oracle_block_bytes(int type)
{
    switch (type) {
    case STYX_ORACLE_F32: return 4;
    case STYX_ORACLE_F16: return 2;
    case STYX_ORACLE_Q8_0: return 34;
    case STYX_ORACLE_Q4_K: return 144;
    case STYX_ORACLE_Q5_K: return 176;
    case STYX_ORACLE_Q6_K: return 210;
    default: return 0;
    }
}

/* ------------------------------------------------------------- dequant -- */

/* crates/model/src/lib.rs:103-113: out[i] = d * (q as i8) as f32 */
static void deq_q8_0(const uint8_t *b, float *y)
{
    const float d = rd_f16(b);
    for (int i = 0; i < 32; i++) y[i] = d * (float)(int8_t)b[2 + i];
}

/* get_scale_min: crates/model/src/moe.rs:513-522 */
static void scale_min_k4(int j, const uint8_t *s, float *sc, float *m)
{
    if (j < 4) {
        *sc = (float)(s[j] & 63);
        *m = (float)(s[j + 4] & 63);
    } else {
        *sc = (float)((s[j + 4] & 0x0F) | ((s[j - 4] >> 6) << 4));
        *m = (float)((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
    }
}

/* crates/model/src/moe.rs:506-533 (== crates/vk-backend/tests/kernels.rs:295-333):
 * y = d*sc*q - dmin*m, evaluated ((d*sc)*q) - (dmin*m). */
static void deq_q4_k(const uint8_t *b, float *y)
{
    const float d = rd_f16(b), dmin = rd_f16(b + 2);
    const uint8_t *scales = b + 4, *qs = b + 16;
    for (int j = 0; j < 4; j++) {
        float sc1, m1, sc2, m2;
        scale_min_k4(2 * j, scales, &sc1, &m1);
        scale_min_k4(2 * j + 1, scales, &sc2, &m2);
        const float d1 = d * sc1, mm1 = dmin * m1;
        const float d2 = d * sc2, mm2 = dmin * m2;
        for (int l = 0; l < 32; l++) y[64 * j + l] = d1 * (float)(qs[32 * j + l] & 0x0F) - mm1;
        for (int l = 0; l < 32; l++) y[64 * j + 32 + l] = d2 * (float)(qs[32 * j + l] >> 4) - mm2;
    }
}

/* Public ggml q5_K block: {f16 d, f16 dmin, u8 scales[12], u8 qh[32], u8 qs[128]}.
 * Same scale/min packing and evaluation order as q4_K plus a fifth bit from
 * qh (bit 2c for the low nibbles of chunk c, bit 2c+1 for the high ones). */
static void deq_q5_k(const uint8_t *b, float *y)
{
    const float d = rd_f16(b), dmin = rd_f16(b + 2);
    const uint8_t *scales = b + 4, *qh = b + 16, *qs = b + 48;
    for (int j = 0; j < 4; j++) {
        float sc1, m1, sc2, m2;
        scale_min_k4(2 * j, scales, &sc1, &m1);
        scale_min_k4(2 * j + 1, scales, &sc2, &m2);
        const float d1 = d * sc1, mm1 = dmin * m1;
        const float d2 = d * sc2, mm2 = dmin * m2;
        const uint8_t u1 = (uint8_t)(1u << (2 * j)), u2 = (uint8_t)(2u << (2 * j));
        for (int l = 0; l < 32; l++)
            y[64 * j + l] = d1 * (float)((qs[32 * j + l] & 0x0F) + ((qh[l] & u1) ? 16 : 0)) - mm1;
        for (int l = 0; l < 32; l++)
            y[64 * j + 32 + l] = d2 * (float)((qs[32 * j + l] >> 4) + ((qh[l] & u2) ? 16 : 0)) - mm2;
    }
}

/* Public ggml q6_K block: {u8 ql[128], u8 qh[64], i8 scales[16], f16 d}
 * (d at byte 208).  y = (d*sc)*q with q = 6-bit value - 32. */
static void deq_q6_k(const uint8_t *b, float *y)
{
    const float d = rd_f16(b + 208);
    for (int n = 0; n < 2; n++) {
        const uint8_t *ql = b + 64 * n, *qh = b + 128 + 32 * n;
        const int8_t *sc = (const int8_t *)(b + 192 + 8 * n);
        float *yy = y + 128 * n;
        for (int l = 0; l < 32; l++) {
            const int is = l / 16;
            const int q1 = (int)((ql[l] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32;
            const int q2 = (int)((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
            const int q3 = (int)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
            const int q4 = (int)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
            yy[l] = d * (float)sc[is + 0] * (float)q1;
            yy[l + 32] = d * (float)sc[is + 2] * (float)q2;
            yy[l + 64] = d * (float)sc[is + 4] * (float)q3;
            yy[l + 96] = d * (float)sc[is + 6] * (float)q4;
        }
    }
}

int styx_oracle_dequant(int type, const uint8_t *blocks, int64_t n_elems, float *out)
{
    const int be = styx_oracle_block_elems(type), bb = styx_oracle_block_bytes(type);
    if (be == 0 || n_elems % be != 0) return -1;
    const int64_t nb = n_elems / be;
    for (int64_t i = 0; i < nb; i++) {
        const uint8_t *b = blocks + i * bb;
        float *y = out + i * be;
        switch (type) {
        case STYX_ORACLE_F32: memcpy(y, b, 4); break;
        case STYX_ORACLE_F16: y[0] = rd_f16(b); break;
        case STYX_ORACLE_Q8_0: deq_q8_0(b, y); break;
        case STYX_ORACLE_Q4_K: deq_q4_k(b, y); break;
        case STYX_ORACLE_Q5_K: deq_q5_k(b, y); break;
        case STYX_ORACLE_Q6_K: deq_q6_k(b, y); break;
        default: return -1;
        }
    }
    return 0;
}

static int64_t row_bytes(int type, int ncols)
{
    return (int64_t)(ncols / styx_oracle_block_elems(type)) * styx_oracle_block_bytes(type);
}

/* -------------------------------------------------------------- matvec -- */

/* crates/vk-backend/tests/kernels.rs:183-198, ops2.rs:242-250: dequantize
 * the row, then row_f.iter().zip(&x).map(|(w,v)| w*v).sum() (f32, in order). */
int styx_oracle_matvec(int type, const uint8_t *w, int nrows, int ncols, const float *x,
                       float *y)
{
    const int be = styx_oracle_block_elems(type);
    if (be == 0 || ncols % be != 0) return -1;
    const int64_t rb = row_bytes(type, ncols);
#pragma omp parallel num_threads(g_threads)
    {
        float *row = (float *)malloc(sizeof(float) * (size_t)ncols);
#pragma omp for schedule(static)
        for (int r = 0; r < nrows; r++) {
            styx_oracle_dequant(type, w + (int64_t)r * rb, ncols, row);
            float acc = 0.0f;
            for (int c = 0; c < ncols; c++) acc += row[c] * x[c];
            y[r] = acc;
        }
        free(row);
    }
    return 0;
}

int styx_oracle_matvec_f64(int type, const uint8_t *w, int nrows, int ncols, const float *x,
                           double *y)
{
    const int be = styx_oracle_block_elems(type);
    if (be == 0 || ncols % be != 0) return -1;
    const int64_t rb = row_bytes(type, ncols);
#pragma omp parallel num_threads(g_threads)
    {
        float *row = (float *)malloc(sizeof(float) * (size_t)ncols);
#pragma omp for schedule(static)
        for (int r = 0; r < nrows; r++) {
            styx_oracle_dequant(type, w + (int64_t)r * rb, ncols, row);
            double acc = 0.0;
            for (int c = 0; c < ncols; c++) acc += (double)row[c] * (double)x[c];
            y[r] = acc;
        }
        free(row);
    }
    return 0;
}

/* mul_mat_vec_id offsets (crates/vk-backend/tests/kernels.rs:124-131):
 * a = ids[s]*expert stride, b = (s % ne11)*ncols, d = s*nrows. */
int styx_oracle_matvec_id(int type, const uint8_t *w, int nrows, int ncols,
                          int64_t expert_stride_bytes, const uint32_t *ids, int n_ids,
                          const float *x, int ne11, float *y)
{
    if (ne11 < 1) return -1;
    for (int s = 0; s < n_ids; s++) {
        const uint32_t e = ids[s];
        if (e == STYX_ORACLE_SKIP) continue;
        int rc = styx_oracle_matvec(type, w + (int64_t)e * expert_stride_bytes, nrows, ncols,
                                    x + (int64_t)(s % ne11) * ncols, y + (int64_t)s * nrows);
        if (rc) return rc;
    }
    return 0;
}

/* ---------------------------------------------------------- elementwise -- */

/* crates/vk-backend/tests/kernels.rs:58-67 (+ weight multiply). */
void styx_oracle_rms_norm(const float *x, const float *w, int ncols, int nrows, float eps,
                          float *out)
{
    for (int r = 0; r < nrows; r++) {
        const float *row = x + (int64_t)r * ncols;
        float ss = 0.0f;
        for (int c = 0; c < ncols; c++) ss += row[c] * row[c];
        const float mean = ss / (float)ncols;
        const float scale = 1.0f / sqrtf(mean + eps);
        float *o = out + (int64_t)r * ncols;
        for (int c = 0; c < ncols; c++) {
            const float v = row[c] * scale;
            o[c] = w ? v * w[c] : v;
        }
    }
}

/* shaders/matvec_strided_f32.comp:25-35 */
void styx_oracle_router_strided(const float *W, const float *x, int nrows, int ncols,
                                int stride, float *out)
{
    for (int r = 0; r < nrows; r++) {
        float tmp[32];
        const float *a = W + (int64_t)r * stride;
        for (int t = 0; t < 32; t++) {
            float sum = 0.0f;
            for (int c = t; c < ncols; c += 32) sum += a[c] * x[c];
            tmp[t] = sum;
        }
        for (int s = 16; s > 0; s >>= 1)
            for (int t = 0; t < s; t++) tmp[t] += tmp[t + s];
        out[r] = tmp[0];
    }
}

/* shaders/topk_softmax_f32.comp:29-67 */
void styx_oracle_topk_softmax(const float *logits, int n, int k, int renorm,
                              const uint32_t *remap, const uint32_t *pmap, float *weights,
                              int32_t *ids)
{
    float mx = logits[0];
    for (int i = 1; i < n; i++) mx = fmaxf(mx, logits[i]);
    float sum = 0.0f;
    for (int i = 0; i < n; i++) sum += expf(logits[i] - mx);

    float picked[16];
    int pid[16];
    float wsum = 0.0f;
    for (int s = 0; s < k; s++) {
        float best = -INFINITY;
        int bi = -1;
        for (int i = 0; i < n; i++) {
            int taken = 0;
            for (int t = 0; t < s; t++)
                if (pid[t] == i) taken = 1;
            if (!taken && logits[i] > best) {
                best = logits[i];
                bi = i;
            }
        }
        const float w = expf(best - mx) / sum;
        picked[s] = w;
        pid[s] = bi;
        wsum += w;
    }
    for (int s = 0; s < k; s++) {
        weights[s] = renorm ? picked[s] / wsum : picked[s];
        const uint32_t e = (uint32_t)pid[s];
        ids[s] = pid[s];
        const uint32_t h = remap ? remap[e] : STYX_ORACLE_SKIP;
        if (h != STYX_ORACLE_SKIP) {
            ids[16 + s] = (int32_t)h;
            ids[32 + s] = (int32_t)STYX_ORACLE_SKIP;
            ids[48 + s] = (int32_t)STYX_ORACLE_SKIP;
        } else {
            const uint32_t a = pmap ? pmap[e] : STYX_ORACLE_SKIP;
            ids[16 + s] = (int32_t)STYX_ORACLE_SKIP;
            ids[32 + s] = (int32_t)a;
            ids[48 + s] = (a != STYX_ORACLE_SKIP) ? (int32_t)STYX_ORACLE_SKIP : pid[s];
        }
    }
}

/* crates/vk-backend/tests/ops2.rs:305-309 */
void styx_oracle_swiglu(const float *g, const float *u, int n, float *out)
{
    for (int i = 0; i < n; i++) out[i] = g[i] / (1.0f + expf(-g[i])) * u[i];
}

/* shaders/moe_reduce_f32.comp:8-13 */
void styx_oracle_moe_reduce(const float *d, const float *w, int ne, int k, float *x)
{
    for (int i = 0; i < ne; i++) {
        float acc = 0.0f;
        for (int s = 0; s < k; s++) acc += w[s] * d[(int64_t)s * ne + i];
        x[i] += acc;
    }
}

/* shaders/axpy_sig_f32.comp:7-11 */
void styx_oracle_axpy_sig(const float *a, float g0, int n, float *d)
{
    const float s = 1.0f / (1.0f + expf(-g0));
    for (int i = 0; i < n; i++) d[i] += s * a[i];
}

/* crates/vk-backend/tests/ops2.rs:426-442: theta_scale = base^(-2/hd) in
 * f64, theta = pos * theta_scale^i, rotate (x[i], x[i+hd/2]) in f64. */
void styx_oracle_rope_neox(float *x, int hd, int nh, int pos, float base)
{
    const int half = hd / 2;
    const double theta_scale = pow((double)base, -2.0 / (double)hd);
    for (int h = 0; h < nh; h++) {
        float *v = x + (int64_t)h * hd;
        for (int i = 0; i < half; i++) {
            const double theta = (double)pos * pow(theta_scale, (double)i);
            const double s = sin(theta), c = cos(theta);
            const double x0 = v[i], x1 = v[i + half];
            v[i] = (float)(x0 * c - x1 * s);
            v[i + half] = (float)(x0 * s + x1 * c);
        }
    }
}

/* ------------------------------------------------------------ attention -- */

/* shaders/attn_decode_f32.comp:31-79 (128 threads per workgroup). */
void styx_oracle_attn_decode(const float *q, const float *K, const float *V, int n_t, int hd,
                             int kv_dim, int gqa, int n_heads, float scale, float *out)
{
    for (int h = 0; h < n_heads; h++) {
        const int kvh = h / gqa;
        const float *qh = q + (int64_t)h * hd;
        const int kvoff = kvh * hd;
        float acc[256];
        for (int i = 0; i < hd; i++) acc[i] = 0.0f;
        float m = -INFINITY, l = 0.0f;
        for (int t = 0; t < n_t; t++) {
            const float *krow = K + (int64_t)t * kv_dim + kvoff;
            float red[128];
            for (int tid = 0; tid < 128; tid++) {
                float part = 0.0f;
                for (int i = tid; i < hd; i += 128) part += qh[i] * krow[i];
                red[tid] = part;
            }
            for (int s = 64; s > 0; s >>= 1)
                for (int tid = 0; tid < s; tid++) red[tid] += red[tid + s];
            const float sc = red[0] * scale;
            const float m_new = fmaxf(m, sc);
            const float corr = expf(m - m_new);
            const float pr = expf(sc - m_new);
            l = l * corr + pr;
            m = m_new;
            const float *vrow = V + (int64_t)t * kv_dim + kvoff;
            for (int i = 0; i < hd; i++) acc[i] = acc[i] * corr + pr * vrow[i];
        }
        const float inv_l = 1.0f / l;
        for (int i = 0; i < hd; i++) out[(int64_t)h * hd + i] = acc[i] * inv_l;
    }
}

/* Textbook two-pass softmax attention in f64 (the checker). */
void styx_oracle_attn_decode_f64(const float *q, const float *K, const float *V, int n_t,
                                 int hd, int kv_dim, int gqa, int n_heads, double scale,
                                 double *out)
{
    double *sc = (double *)malloc(sizeof(double) * (size_t)(n_t > 0 ? n_t : 1));
    for (int h = 0; h < n_heads; h++) {
        const int kvoff = (h / gqa) * hd;
        const float *qh = q + (int64_t)h * hd;
        double mx = -INFINITY;
        for (int t = 0; t < n_t; t++) {
            double d = 0.0;
            for (int i = 0; i < hd; i++) d += (double)qh[i] * (double)K[(int64_t)t * kv_dim + kvoff + i];
            sc[t] = d * scale;
            if (sc[t] > mx) mx = sc[t];
        }
        double den = 0.0;
        for (int t = 0; t < n_t; t++) {
            sc[t] = exp(sc[t] - mx);
            den += sc[t];
        }
        for (int i = 0; i < hd; i++) {
            double o = 0.0;
            for (int t = 0; t < n_t; t++) o += sc[t] * (double)V[(int64_t)t * kv_dim + kvoff + i];
            out[(int64_t)h * hd + i] = o / den;
        }
    }
    free(sc);
}

/* ---------------------------------------------------------------- gather -- */

/* shaders/gather_slabs_f32.comp:40-86 (non-canary branch). */
void styx_oracle_gather_slabs(const uint8_t *const src[3], const int64_t src_slab[3],
                              uint8_t *const dst[3], const int64_t dst_slab[3],
                              const uint32_t *ids, int k, int layer)
{
    for (int s = 0; s < k; s++) {
        const uint32_t e = ids[s];
        if (e == STYX_ORACLE_SKIP) continue;
        const int64_t slot = (int64_t)layer * k + s;
        for (int t = 0; t < 3; t++)
            memcpy(dst[t] + slot * dst_slab[t], src[t] + (int64_t)e * src_slab[t],
                   (size_t)src_slab[t]);
    }
}

/* -------------------------------------------------------------- model ---- */

static int64_t mat_bytes(const styx_oracle_mat *w)
{
    return (int64_t)w->nrows * row_bytes(w->type, w->ncols);
}

static int mv(const styx_oracle_mat *w, const float *x, float *y)
{
    return styx_oracle_matvec(w->type, w->data, w->nrows, w->ncols, x, y);
}

/* crates/model/src/moe.rs:1974-2062 (+ shared expert per
 * shaders/axpy_sig_f32.comp, + optional router bias). */
int styx_oracle_moe_block(const styx_oracle_model *m, int layer, float *x, float *xn_out,
                          float *logits_out, int32_t *ids_out, float *weights_out)
{
    const styx_oracle_layer *ly = &m->layers[layer];
    const int H = m->n_embd, E = m->n_expert, k = m->n_expert_used, F = m->n_ff_exp;
    if (k > 16 || E > 512) return -2;
    float *xn = (float *)malloc(sizeof(float) * H);
    float *logits = (float *)malloc(sizeof(float) * E);
    float *g = (float *)malloc(sizeof(float) * (size_t)k * F);
    float *u = (float *)malloc(sizeof(float) * (size_t)k * F);
    float *d = (float *)malloc(sizeof(float) * (size_t)k * H);
    int32_t ids[64];
    float w[16];
    int rc = 0;

    styx_oracle_rms_norm(x, ly->ffn_norm, H, 1, m->rms_eps, xn);
    styx_oracle_router_strided(ly->router, xn, E, H, H, logits);
    if (ly->router_bias)
        for (int e = 0; e < E; e++) logits[e] = logits[e] + ly->router_bias[e];
    styx_oracle_topk_softmax(logits, E, k, m->norm_topk, NULL, NULL, w, ids);

    uint32_t uid[16];
    for (int s = 0; s < k; s++) uid[s] = (uint32_t)ids[s];
    const int64_t gst = mat_bytes(&ly->gate_exps), ust = mat_bytes(&ly->up_exps),
                  dst = mat_bytes(&ly->down_exps);
    rc |= styx_oracle_matvec_id(ly->gate_exps.type, ly->gate_exps.data, F, H, gst, uid, k, xn, 1, g);
    rc |= styx_oracle_matvec_id(ly->up_exps.type, ly->up_exps.data, F, H, ust, uid, k, xn, 1, u);
    styx_oracle_swiglu(g, u, k * F, g);
    rc |= styx_oracle_matvec_id(ly->down_exps.type, ly->down_exps.data, H, F, dst, uid, k, g, k, d);
    styx_oracle_moe_reduce(d, w, H, k, x);

    if (ly->gate_sh.data) {
        const int Fs = ly->gate_sh.nrows;
        float *gs = (float *)malloc(sizeof(float) * Fs);
        float *us = (float *)malloc(sizeof(float) * Fs);
        float *ds = (float *)malloc(sizeof(float) * H);
        rc |= mv(&ly->gate_sh, xn, gs);
        rc |= mv(&ly->up_sh, xn, us);
        styx_oracle_swiglu(gs, us, Fs, gs);
        rc |= mv(&ly->down_sh, gs, ds);
        float g0 = 0.0f;
        for (int c = 0; c < H; c++) g0 += ly->gate_inp_sh[c] * xn[c];
        styx_oracle_axpy_sig(ds, g0, H, x);
        free(gs);
        free(us);
        free(ds);
    }

    if (xn_out) memcpy(xn_out, xn, sizeof(float) * H);
    if (logits_out) memcpy(logits_out, logits, sizeof(float) * E);
    if (ids_out) memcpy(ids_out, ids, sizeof(int32_t) * k);
    if (weights_out) memcpy(weights_out, w, sizeof(float) * k);
    free(xn);
    free(logits);
    free(g);
    free(u);
    free(d);
    return rc;
}

static int cmp_desc(const void *a, const void *b)
{
    const float x = *(const float *)a, y = *(const float *)b;
    return (x < y) - (x > y);
}

/* k-th largest minus (k+1)-th largest routing logit (0 on a tie). */
static float routing_margin(const float *logits, int n, int k)
{
    if (n <= k) return INFINITY;
    float *s = (float *)malloc(sizeof(float) * (size_t)n);
    memcpy(s, logits, sizeof(float) * (size_t)n);
    qsort(s, (size_t)n, sizeof(float), cmp_desc);
    const float r = s[k - 1] - s[k];
    free(s);
    return r;
}

/* crates/model/src/moe.rs:1780-2157 (all-resident path).  Deviation: the
 * embedding row is dequantized by its own type (the reference always
 * decodes q4_K, moe.rs:1824-1833). */
int styx_oracle_forward(styx_oracle_model *m, int pos, uint32_t token, float *logits,
                        float *hidden, int32_t *ids, float *margins)
{
    const int H = m->n_embd, nh = m->n_heads, nkv = m->n_kv_heads, hd = m->head_dim;
    const int kv_dim = nkv * hd, q_dim = nh * hd, k = m->n_expert_used, E = m->n_expert;
    if (pos >= m->n_ctx || token >= (uint32_t)m->n_vocab) return -3;
    const int n_t = pos + 1;
    const float scale = 1.0f / sqrtf((float)hd);
    int rc = 0;

    float *x = (float *)malloc(sizeof(float) * H);
    float *xn = (float *)malloc(sizeof(float) * H);
    float *q = (float *)malloc(sizeof(float) * q_dim);
    float *kk = (float *)malloc(sizeof(float) * kv_dim);
    float *vv = (float *)malloc(sizeof(float) * kv_dim);
    float *att = (float *)malloc(sizeof(float) * q_dim);
    float *proj = (float *)malloc(sizeof(float) * H);
    float *lg = (float *)malloc(sizeof(float) * E);

    const styx_oracle_mat *te = &m->token_embd;
    rc |= styx_oracle_dequant(te->type, te->data + (int64_t)token * row_bytes(te->type, H), H, x);
    if (hidden) memcpy(hidden, x, sizeof(float) * H);

    for (int l = 0; l < m->n_layers; l++) {
        const styx_oracle_layer *ly = &m->layers[l];
        float *kc = m->kcache + (int64_t)l * m->n_ctx * kv_dim;
        float *vc = m->vcache + (int64_t)l * m->n_ctx * kv_dim;
        styx_oracle_rms_norm(x, ly->attn_norm, H, 1, m->rms_eps, xn);
        rc |= mv(&ly->wq, xn, q);
        rc |= mv(&ly->wk, xn, kk);
        rc |= mv(&ly->wv, xn, vv);
        styx_oracle_rms_norm(q, ly->q_norm, hd, nh, m->rms_eps, q);
        styx_oracle_rms_norm(kk, ly->k_norm, hd, nkv, m->rms_eps, kk);
        styx_oracle_rope_neox(q, hd, nh, pos, m->rope_base);
        styx_oracle_rope_neox(kk, hd, nkv, pos, m->rope_base);
        memcpy(kc + (int64_t)pos * kv_dim, kk, sizeof(float) * kv_dim);
        memcpy(vc + (int64_t)pos * kv_dim, vv, sizeof(float) * kv_dim);
        styx_oracle_attn_decode(q, kc, vc, n_t, hd, kv_dim, nh / nkv, nh, scale, att);
        rc |= mv(&ly->wo, att, proj);
        for (int i = 0; i < H; i++) x[i] = x[i] + proj[i];
        rc |= styx_oracle_moe_block(m, l, x, NULL, lg, ids ? ids + (int64_t)l * k : NULL, NULL);
        if (margins) margins[l] = routing_margin(lg, E, k);
        if (hidden) memcpy(hidden + (int64_t)(l + 1) * H, x, sizeof(float) * H);
    }
    styx_oracle_rms_norm(x, m->output_norm, H, 1, m->rms_eps, xn);
    rc |= mv(&m->output, xn, logits);

    free(x);
    free(xn);
    free(q);
    free(kk);
    free(vv);
    free(att);
    free(proj);
    free(lg);
    return rc;
}

/* crates/model/examples/generate_moe.rs:29: max_by(total_cmp) keeps the
 * LAST maximal index. */
uint32_t styx_oracle_argmax(const float *v, int n)
{
    int best = 0;
    int32_t bk = 0;
    for (int i = 0; i < n; i++) {
        int32_t b;
        memcpy(&b, &v[i], 4);
        b ^= (int32_t)(((uint32_t)(b >> 31)) >> 1);
        if (i == 0 || b >= bk) {
            bk = b;
            best = i;
        }
    }
    return (uint32_t)best;
}
