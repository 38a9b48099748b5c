/* hymt2 oracle: TEST INFRASTRUCTURE ONLY (see hymt2_oracle.h).
 *
 * CPU restatement of the reference's scalar-ISA arithmetic. Compiled with -ffp-contract=off so
 * that every `a * b + c` is a separate IEEE multiply and add, as in the reference's x86-64
 * baseline build (no FMA instructions are available to it there). Row-parallel loops use
 * OpenMP; every output element is still computed by one thread in the reference's order, so
 * results do not depend on the thread count.
 */
#include "hymt2_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define QK OC_QK

/* ------------------------------------------------------------------ conversions */

/* IEEE binary16 -> binary32, exact for every input including subnormals, inf and NaN
 * payloads (same results as src/kernels.c:76-98). */
float oc_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h >> 15) << 31;
    const uint32_t e = (h >> 10) & 31u, m = h & 1023u;
    uint32_t bits;
    if (e == 31) {
        bits = sign | 0x7F800000u | (m << 13);
    } else if (e != 0) {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    } else {
        float v = (float)m * 0x1p-24f; /* m < 2^10: exact product, normal or zero result */
        memcpy(&bits, &v, 4);
        bits |= sign;
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* Round-to-nearest-even truncation to bfloat16 (src/kernels.c:107-111). */
uint16_t oc_f32_to_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

float oc_bf16_to_f32(uint16_t h) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

size_t oc_row_bytes(int type, int k) { /* src/kernels.c:113-124 */
    switch (type) {
    case OC_F32: return (size_t)k * 4;
    case OC_F16: return (size_t)k * 2;
    case OC_Q8_0: return (size_t)(k / 32) * 34;
    case OC_Q4_K: return (size_t)(k / QK) * 144;
    case OC_Q6_K: return (size_t)(k / QK) * 210;
    case OC_STQ1_0: return (size_t)(k / QK) * 42;
    case OC_Q2_0C: return (size_t)(k / 512) * 130;
    }
    return 0;
}

static inline uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* libm expf over an array: the exact function the reference calls in softmax and SiLU
 * (src/model.c:787, :875). */
void oc_expf_n(const float *x, float *y, int n) {
    for (int i = 0; i < n; i++) y[i] = expf(x[i]);
}

/* ------------------------------------------------------------------ Q8_K */

/* Q8_K activation quantization, src/kernels.c:128-165: the signed value of the first element
 * with the largest magnitude sets iscale = -127/max; q = clamp(rint(iscale*x), -127, 127);
 * d = 1/iscale; 16-element sums; reordered copy qp with piece order {0,2,1,3}
 * (src/internal.h:31-36). An all-zero block becomes an all-zero record. */
void oc_quantize_q8k(const float *x, int k, oc_q8k *y) {
    static const int piece[4] = {0, 2, 1, 3};
    for (int b = 0; b < k / QK; b++) {
        const float *src = x + (size_t)b * QK;
        oc_q8k *o = y + b;
        float amax = 0.f, vmax = 0.f;
        for (int j = 0; j < QK; j++) {
            float a = fabsf(src[j]);
            if (a > amax) {
                amax = a;
                vmax = src[j];
            }
        }
        memset(o, 0, sizeof(*o));
        if (amax == 0.f) continue;
        const float iscale = -127.f / vmax;
        o->d = 1.f / iscale;
        int total = 0;
        for (int g = 0; g < QK / 16; g++) {
            int part = 0;
            for (int j = 0; j < 16; j++) {
                long v = lrintf(iscale * src[g * 16 + j]);
                if (v > 127) v = 127;
                if (v < -127) v = -127;
                o->qs[g * 16 + j] = (int8_t)v;
                part += (int)v;
            }
            o->bsums[g] = (int16_t)part;
            total += part;
        }
        o->sum = total;
        for (int l = 0; l < 4; l++)
            for (int j = 0; j < 4; j++) memcpy(o->qp + l * 64 + j * 16, o->qs + piece[j] * 64 + l * 16, 16);
    }
}

/* ------------------------------------------------------------------ STQ1_0 / panel */

/* STQ1_0 4-weight group codebook (src/kernels.c:178-181). Each byte holds four 2-bit codes
 * (0 = -1, 1 = 0, 2 = +1), lane 0 in the low bits. Index = (sign << 4) | slot. The sign half
 * is the complement 0xAA - base, the identity the reference itself checks at init
 * (src/kernels.c:1417-1418). */
static const uint8_t STQ_BASE[16] = {0xA9, 0x89, 0x29, 0x09, 0xA6, 0x86, 0x26, 0x06,
                                     0x9A, 0x92, 0x1A, 0x12, 0x6A, 0x62, 0x4A, 0x42};

/* Packed codes of group g (0..63) of one 42-byte STQ1_0 block (src/kernels.c:184-188). */
uint8_t oc_stq_group_codes(const uint8_t *blk, int g) {
    const int slot = (blk[g >> 1] >> ((g & 1) * 4)) & 15;
    const int sign = (blk[32 + (g >> 3)] >> (g & 7)) & 1;
    return sign ? (uint8_t)(0xAA - STQ_BASE[slot]) : STQ_BASE[slot];
}

/* Panel repack, src/kernels.c:535-561. 64 bytes per 256-weight block: segment s holds chunk
 * {0,2,1,3}[s]; byte (s*16+o) holds in bits 2l..2l+1 the code of weight chunk*64 + o + 16*l.
 * Scale per block = f16 d of the source block (Q2_0C: both 256-halves share the 512 block's d). */
void oc_panel_repack(const oc_weight *w, uint8_t *pk, float *ps, int r0, int r1) {
    static const int seg_of_chunk[4] = {0, 2, 1, 3};
    const int nb = w->k / QK;
    const size_t rb = oc_row_bytes(w->type, w->k);
    for (int r = r0; r < r1; r++) {
        const uint8_t *row = w->data + (size_t)r * rb;
        for (int b = 0; b < nb; b++) {
            uint8_t *dst = pk + ((size_t)r * nb + b) * 64;
            if (w->type == OC_STQ1_0) {
                const uint8_t *blk = row + (size_t)b * 42;
                ps[(size_t)r * nb + b] = oc_f16_to_f32(rd16(blk + 40));
                for (int g = 0; g < 64; g++) dst[seg_of_chunk[g >> 4] * 16 + (g & 15)] = oc_stq_group_codes(blk, g);
            } else { /* OC_Q2_0C */
                const uint8_t *blk = row + (size_t)(b >> 1) * 130;
                const int half = b & 1;
                ps[(size_t)r * nb + b] = oc_f16_to_f32(rd16(blk));
                for (int g = 0; g < 64; g++) {
                    const int c = g >> 4, o = g & 15;
                    int byte = 0;
                    for (int l = 0; l < 4; l++) {
                        const int wi = half * 256 + c * 64 + o + 16 * l;
                        byte |= ((blk[2 + (wi >> 2)] >> ((wi & 3) * 2)) & 3) << (2 * l);
                    }
                    dst[seg_of_chunk[c] * 16 + o] = (uint8_t)byte;
                }
            }
        }
    }
}

static inline int32_t panel_enc(const uint8_t *pk, const oc_q8k *y) {
    int32_t enc = 0; /* src/kernels.c:574-575 */
    for (int l = 0; l < 4; l++)
        for (int i = 0; i < 64; i++) enc += ((pk[i] >> (2 * l)) & 3) * y->qp[l * 64 + i];
    return enc;
}

/* Panel row dot, src/kernels.c:565-581: acc += (ps*d) * float((enc << shift) - off*sum),
 * blocks in order. */
static float panel_dot(const oc_weight *w, int r, const oc_q8k *xq) {
    const int nb = w->k / QK;
    float acc = 0.f;
    for (int b = 0; b < nb; b++) {
        const uint8_t *pk = w->pk + ((size_t)r * nb + b) * 64;
        const oc_q8k *y = xq + b;
        const int32_t enc = panel_enc(pk, y);
        acc += w->ps[(size_t)r * nb + b] * y->d * (float)((enc << w->pshift) - w->poff * y->sum);
    }
    return acc;
}

/* Native STQ1_0 dot, src/kernels.c:202-215 (used when no panel is present). */
static float stq_dot(const uint8_t *row, const oc_q8k *y, int nb) {
    float sum = 0.f;
    for (int b = 0; b < nb; b++) {
        const uint8_t *blk = row + (size_t)b * 42;
        int si = 0;
        for (int g = 0; g < 64; g++) {
            const uint8_t cb = oc_stq_group_codes(blk, g);
            const int chunk = g >> 4, o = g & 15;
            for (int l = 0; l < 4; l++) si += (((cb >> (2 * l)) & 3) - 1) * y[b].qs[chunk * 64 + o + 16 * l];
        }
        sum += oc_f16_to_f32(rd16(blk + 40)) * y[b].d * (float)si;
    }
    return sum;
}

/* Native Q2_0C dot, src/kernels.c:1222-1237. */
static float q2c_dot(const uint8_t *row, const oc_q8k *y, int nb512) {
    float sum = 0.f;
    for (int b = 0; b < nb512; b++) {
        const uint8_t *blk = row + (size_t)b * 130;
        float acc = 0.f;
        for (int h = 0; h < 2; h++) {
            int s = 0;
            for (int j = 0; j < 256; j++) {
                const int wi = h * 256 + j;
                s += (2 * ((blk[2 + (wi >> 2)] >> ((wi & 3) * 2)) & 3) - 3) * y[2 * b + h].qs[j];
            }
            acc += (float)s * y[2 * b + h].d;
        }
        sum += oc_f16_to_f32(rd16(blk)) * acc;
    }
    return sum;
}

/* ------------------------------------------------------------------ Q6_K / Q4_K */

/* Q6_K signed 6-bit values of one 210-byte block in natural order, src/kernels.c:812-823.
 * Layout: ql[128] @0, qh[64] @128, scales[16] (int8) @192, f16 d @208. */
static void q6_values(const uint8_t *blk, int8_t *a) {
    const uint8_t *ql = blk, *qh = blk + 128;
    for (int half = 0; half < 2; half++) {
        for (int l = 0; l < 32; l++) {
            a[l] = (int8_t)(((ql[l] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32);
            a[l + 32] = (int8_t)(((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32);
            a[l + 64] = (int8_t)(((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32);
            a[l + 96] = (int8_t)(((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32);
        }
        a += 128;
        ql += 64;
        qh += 32;
    }
}

static int32_t q6_acc(const uint8_t *blk, const oc_q8k *y) { /* src/kernels.c:825-832 */
    int8_t a[QK];
    q6_values(blk, a);
    const int8_t *sc = (const int8_t *)(blk + 192);
    int32_t acc = 0;
    for (int j = 0; j < 16; j++) {
        int32_t t = 0;
        for (int l = 0; l < 16; l++) t += y->qs[j * 16 + l] * a[j * 16 + l];
        acc += sc[j] * t;
    }
    return acc;
}

static float q6_dot(const uint8_t *row, const oc_q8k *y, int nb) { /* src/kernels.c:808-835 */
    float sumf = 0.f;
    for (int b = 0; b < nb; b++) {
        const uint8_t *blk = row + (size_t)b * 210;
        sumf += oc_f16_to_f32(rd16(blk + 208)) * y[b].d * (float)q6_acc(blk, &y[b]);
    }
    return sumf;
}

/* 6-bit scale/min pair j of a Q4_K block, src/kernels.c:839-842. */
static void q4_scale_min(const uint8_t *s, int j, int *d, int *m) {
    if (j < 4) {
        *d = s[j] & 63;
        *m = s[j + 4] & 63;
    } else {
        *d = (s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4);
        *m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
}

/* Q4_K integer parts (sumi, summ), src/kernels.c:863-874. Layout: f16 d @0, f16 dmin @2,
 * scales[12] @4, qs[128] @16. */
static void q4_ints(const uint8_t *blk, const oc_q8k *y, int32_t *sumi_out, int32_t *summ_out) {
    int sc[8], mn[8];
    for (int j = 0; j < 8; j++) q4_scale_min(blk + 4, j, &sc[j], &mn[j]);
    int32_t sumi = 0, summ = 0;
    for (int g = 0; g < 4; g++) {
        const uint8_t *q = blk + 16 + 32 * g;
        int32_t s0 = 0, s1 = 0;
        for (int l = 0; l < 32; l++) {
            s0 += (q[l] & 0xF) * y->qs[64 * g + l];
            s1 += (q[l] >> 4) * y->qs[64 * g + 32 + l];
        }
        sumi += sc[2 * g] * s0 + sc[2 * g + 1] * s1;
    }
    for (int j = 0; j < 8; j++) summ += mn[j] * (y->bsums[2 * j] + y->bsums[2 * j + 1]);
    *sumi_out = sumi;
    *summ_out = summ;
}

static float q4_dot(const uint8_t *row, const oc_q8k *y, int nb) { /* src/kernels.c:861-877 */
    float sumf = 0.f;
    for (int b = 0; b < nb; b++) {
        const uint8_t *blk = row + (size_t)b * 144;
        int32_t sumi, summ;
        q4_ints(blk, &y[b], &sumi, &summ);
        sumf += y[b].d * (oc_f16_to_f32(rd16(blk)) * (float)sumi - oc_f16_to_f32(rd16(blk + 2)) * (float)summ);
    }
    return sumf;
}

/* ------------------------------------------------------------------ dequant */

/* Row dequantization, src/kernels.c:1304-1329 (with q6/q4/stq helpers at :786-806, :844-859,
 * :190-200). */
void oc_dequant_row(const oc_weight *w, int row, float *dst) {
    const size_t rb = oc_row_bytes(w->type, w->k);
    const uint8_t *p = w->data + (size_t)row * rb;
    switch (w->type) {
    case OC_F32: memcpy(dst, p, (size_t)w->k * 4); break;
    case OC_F16:
        for (int j = 0; j < w->k; j++) dst[j] = oc_f16_to_f32(rd16(p + 2 * j));
        break;
    case OC_Q8_0:
        for (int b = 0; b < w->k / 32; b++) {
            const float d = oc_f16_to_f32(rd16(p + b * 34));
            for (int j = 0; j < 32; j++) dst[b * 32 + j] = d * (float)(int8_t)p[b * 34 + 2 + j];
        }
        break;
    case OC_Q4_K:
        for (int b = 0; b < w->k / QK; b++) {
            const uint8_t *blk = p + (size_t)b * 144;
            const float d = oc_f16_to_f32(rd16(blk)), dm = oc_f16_to_f32(rd16(blk + 2));
            float *y = dst + b * QK;
            for (int g = 0; g < 4; g++) {
                int sc, mn;
                q4_scale_min(blk + 4, 2 * g, &sc, &mn);
                const float d1 = d * sc, m1 = dm * mn;
                q4_scale_min(blk + 4, 2 * g + 1, &sc, &mn);
                const float d2 = d * sc, m2 = dm * mn;
                const uint8_t *q = blk + 16 + 32 * g;
                for (int l = 0; l < 32; l++) y[64 * g + l] = d1 * (q[l] & 0xF) - m1;
                for (int l = 0; l < 32; l++) y[64 * g + 32 + l] = d2 * (q[l] >> 4) - m2;
            }
        }
        break;
    case OC_Q6_K:
        for (int b = 0; b < w->k / QK; b++) {
            const uint8_t *blk = p + (size_t)b * 210;
            const float d = oc_f16_to_f32(rd16(blk + 208));
            const int8_t *sc = (const int8_t *)(blk + 192);
            int8_t a[QK];
            q6_values(blk, a);
            /* the reference multiplies d * sc[is] * (q - 32) with is = l/16 + {0,2,4,6} per
             * 32-wide quarter, i.e. scale index = element / 16 */
            for (int j = 0; j < QK; j++) dst[b * QK + j] = d * sc[j / 16] * (float)a[j];
        }
        break;
    case OC_STQ1_0:
        for (int b = 0; b < w->k / QK; b++) {
            const uint8_t *blk = p + (size_t)b * 42;
            const float d = oc_f16_to_f32(rd16(blk + 40));
            for (int g = 0; g < 64; g++) {
                const uint8_t cb = oc_stq_group_codes(blk, g);
                const int chunk = g >> 4, o = g & 15;
                for (int l = 0; l < 4; l++) dst[b * QK + chunk * 64 + o + l * 16] = (float)(((cb >> (l * 2)) & 3) - 1) * d;
            }
        }
        break;
    case OC_Q2_0C:
        for (int b = 0; b < w->k / 512; b++) {
            const uint8_t *blk = p + (size_t)b * 130;
            const float d = oc_f16_to_f32(rd16(blk));
            for (int j = 0; j < 512; j++) dst[b * 512 + j] = (float)(2 * ((blk[2 + (j >> 2)] >> ((j & 3) * 2)) & 3) - 3) * d;
        }
        break;
    }
}

/* ------------------------------------------------------------------ matvec dispatch */

static float row_dot(const oc_weight *w, int r, const float *xf, const oc_q8k *xq) {
    const size_t rb = oc_row_bytes(w->type, w->k);
    const uint8_t *row = w->data ? w->data + (size_t)r * rb : NULL;
    if (w->pk) return panel_dot(w, r, xq);
    switch (w->type) {
    case OC_Q2_0C: return q2c_dot(row, xq, w->k / 512);
    case OC_STQ1_0: return stq_dot(row, xq, w->k / QK);
    case OC_Q4_K: return q4_dot(row, xq, w->k / QK);
    case OC_Q6_K: return q6_dot(row, xq, w->k / QK);
    case OC_Q8_0: { /* src/kernels.c:1099-1107 */
        float sum = 0.f;
        for (int b = 0; b < w->k / 32; b++) {
            float s = 0.f;
            for (int j = 0; j < 32; j++) s += (float)(int8_t)row[b * 34 + 2 + j] * xf[b * 32 + j];
            sum += oc_f16_to_f32(rd16(row + b * 34)) * s;
        }
        return sum;
    }
    case OC_F16: { /* src/kernels.c:1279-1289 */
        float s = 0.f;
        for (int j = 0; j < w->k; j++) s += oc_f16_to_f32(rd16(row + 2 * j)) * xf[j];
        return s;
    }
    case OC_F32: { /* src/kernels.c:1290-1300 */
        float s = 0.f;
        const float *wr = (const float *)row;
        for (int j = 0; j < w->k; j++) s += wr[j] * xf[j];
        return s;
    }
    }
    return 0.f;
}

/* matmul_rows, src/kernels.c:1241-1302, over all rows (row-parallel). */
void oc_matvec(const oc_weight *w, const float *xf, const oc_q8k *xq, int nt, float *out) {
    const int nbq = (w->type == OC_Q2_0C && !w->pk) ? (w->k / 512) * 2 : w->k / QK;
#pragma omp parallel for schedule(static)
    for (int r = 0; r < w->n; r++)
        for (int t = 0; t < nt; t++)
            out[(size_t)t * w->n + r] =
                row_dot(w, r, xf ? xf + (size_t)t * w->k : NULL, xq ? xq + (size_t)t * nbq : NULL);
}

void oc_block_ints(const oc_weight *w, const oc_q8k *xq, int nt, int kind, int32_t *enc) {
    const int nb = w->k / QK;
    const size_t rb = oc_row_bytes(w->type, w->k);
#pragma omp parallel for schedule(static)
    for (int r = 0; r < w->n; r++)
        for (int t = 0; t < nt; t++)
            for (int b = 0; b < nb; b++) {
                const oc_q8k *y = xq + (size_t)t * nb + b;
                int32_t v = 0;
                if (kind == 0) {
                    v = panel_enc(w->pk + ((size_t)r * nb + b) * 64, y);
                } else if (kind == 1 || kind == 2) {
                    int32_t si, sm;
                    q4_ints(w->data + (size_t)r * rb + (size_t)b * 144, y, &si, &sm);
                    v = kind == 1 ? si : sm;
                } else {
                    v = q6_acc(w->data + (size_t)r * rb + (size_t)b * 210, y);
                }
                enc[((size_t)t * w->n + r) * nb + b] = v;
            }
}

/* ------------------------------------------------------------------ attention helpers */

/* bf16 dot with four interleaved partial sums, src/kernels.c:1111-1121. */
float oc_dot_bf16(const float *q, const uint16_t *k, int n) {
    float a0 = 0, a1 = 0, a2 = 0, a3 = 0;
    int d = 0;
    for (; d + 4 <= n; d += 4) {
        a0 += q[d] * oc_bf16_to_f32(k[d]);
        a1 += q[d + 1] * oc_bf16_to_f32(k[d + 1]);
        a2 += q[d + 2] * oc_bf16_to_f32(k[d + 2]);
        a3 += q[d + 3] * oc_bf16_to_f32(k[d + 3]);
    }
    float s = (a0 + a1) + (a2 + a3);
    for (; d < n; d++) s += q[d] * oc_bf16_to_f32(k[d]);
    return s;
}

void oc_axpy_bf16(float *o, const uint16_t *v, float p, int n) { /* src/kernels.c:1122-1124 */
    for (int d = 0; d < n; d++) o[d] += p * oc_bf16_to_f32(v[d]);
}

/* ------------------------------------------------------------------ model */

/* RoPE tables, src/model.c:535-537 (alpha scaling of the base) and :576-586. */
void oc_rope_tables(int ctx, int rope_half, int hdim, float base, float alpha, float *cosv, float *sinv) {
    if (alpha > 0 && hdim > 2) base *= powf(alpha, (float)hdim / (float)(hdim - 2));
    for (int i = 0; i < rope_half; i++) {
        const float freq = 1.0f / powf(base, (float)i / (float)rope_half);
        for (int p = 0; p < ctx; p++) {
            const float a = (float)p * freq;
            cosv[(size_t)p * rope_half + i] = cosf(a);
            sinv[(size_t)p * rope_half + i] = sinf(a);
        }
    }
}

struct oc_state {
    oc_model m;
    int qdim, kvdim;
    uint16_t *kc, *vc; /* [n_layer][ctx][kvdim] */
    float *h, *xn, *q, *k, *v, *ao, *gate, *up, *tmp, *scores;
    oc_q8k *xq_h, *xq_q, *xq_f;
    int cap_nt;
    int *cache_tok; /* [ctx] ids whose K/V the cache holds (oc_gen_ids), n_cache of them */
    int n_cache;
};

static int g_threads = 0;
void oc_set_threads(int n) { g_threads = n; }

oc_state *oc_state_new(const oc_model *m) {
    oc_state *s = (oc_state *)calloc(1, sizeof(*s));
    s->m = *m;
    s->qdim = m->heads * m->hdim;
    s->kvdim = m->kv_heads * m->hdim;
    const size_t kvn = (size_t)m->n_layer * m->ctx * s->kvdim;
    s->kc = (uint16_t *)calloc(kvn, 2);
    s->vc = (uint16_t *)calloc(kvn, 2);
    s->cap_nt = 16;
    const size_t B = (size_t)s->cap_nt;
    int maxk = m->hidden > m->ffn ? m->hidden : m->ffn;
    if (s->qdim > maxk) maxk = s->qdim;
    s->h = (float *)calloc(B * m->hidden, 4);
    s->xn = (float *)calloc(B * maxk, 4);
    s->q = (float *)calloc(B * s->qdim, 4);
    s->k = (float *)calloc(B * s->kvdim, 4);
    s->v = (float *)calloc(B * s->kvdim, 4);
    s->ao = (float *)calloc(B * s->qdim, 4);
    s->gate = (float *)calloc(B * m->ffn, 4);
    s->up = (float *)calloc(B * m->ffn, 4);
    s->tmp = (float *)calloc(B * m->hidden, 4);
    s->scores = (float *)calloc(B * m->heads * (size_t)m->ctx, 4);
    s->xq_h = (oc_q8k *)aligned_alloc(64, sizeof(oc_q8k) * B * (m->hidden / QK + 1));
    s->xq_q = (oc_q8k *)aligned_alloc(64, sizeof(oc_q8k) * B * (s->qdim / QK + 1));
    s->xq_f = (oc_q8k *)aligned_alloc(64, sizeof(oc_q8k) * B * (m->ffn / QK + 1));
    if (g_threads > 0) {
#ifdef _OPENMP
        omp_set_num_threads(g_threads);
#endif
    }
    return s;
}

void oc_state_free(oc_state *s) {
    if (!s) return;
    free(s->kc); free(s->vc); free(s->h); free(s->xn); free(s->q); free(s->k); free(s->v);
    free(s->ao); free(s->gate); free(s->up); free(s->tmp); free(s->scores);
    free(s->xq_h); free(s->xq_q); free(s->xq_f); free(s->cache_tok);
    free(s);
}

const float *oc_state_hidden(const oc_state *s) { return s->h; }

/* RMSNorm, scalar branch of src/model.c:719-739. y may alias x. */
/* RMSNorm, src/model.c:719-739: sequential sum of squares, one reciprocal square root, then
 * x * scale * w per element. */
void oc_rmsnorm(const float *x, const float *w, float *y, int dim, float eps) {
    float sum = 0.f;
    for (int i = 0; i < dim; i++) sum += x[i] * x[i];
    const float scale = 1.0f / sqrtf(sum / (float)dim + eps);
    for (int i = 0; i < dim; i++) y[i] = x[i] * scale * w[i];
}

/* NeoX rotate-half RoPE with table rows at pos, src/model.c:754-765. */
static void rope(const oc_state *s, float *x, int heads, int pos) {
    const int half = s->m.rope_half, hd = s->m.hdim;
    const float *c = s->m.rope_cos + (size_t)pos * half, *sn = s->m.rope_sin + (size_t)pos * half;
    for (int h = 0; h < heads; h++) {
        float *row = x + (size_t)h * hd;
        for (int i = 0; i < half; i++) {
            const float x0 = row[i], x1 = row[i + half];
            row[i] = x0 * c[i] - x1 * sn[i];
            row[i + half] = x0 * sn[i] + x1 * c[i];
        }
    }
}

/* One (token, head) attention item, src/model.c:767-795. */
static void attn_item(oc_state *s, int layer, int pos0, int item) {
    const oc_model *m = &s->m;
    const int t = item / m->heads, h = item % m->heads;
    const int group = m->heads / m->kv_heads;
    const float scale = 1.0f / sqrtf((float)m->hdim);
    const int pos = pos0 + t, n = pos + 1, kvh = h / group;
    const float *qh = s->q + (size_t)t * s->qdim + (size_t)h * m->hdim;
    float *sc = s->scores + (size_t)item * m->ctx;
    const size_t lbase = (size_t)layer * m->ctx * s->kvdim;
    const uint16_t *K = s->kc + lbase + (size_t)kvh * m->hdim, *V = s->vc + lbase + (size_t)kvh * m->hdim;
    float mx = -INFINITY;
    for (int j = 0; j < n; j++) {
        const float v = oc_dot_bf16(qh, K + (size_t)j * s->kvdim, m->hdim) * scale;
        sc[j] = v;
        if (v > mx) mx = v;
    }
    float sum = 0.f;
    for (int j = 0; j < n; j++) {
        sc[j] = expf(sc[j] - mx);
        sum += sc[j];
    }
    const float inv = 1.0f / sum;
    float *o = s->ao + (size_t)t * s->qdim + (size_t)h * m->hdim;
    for (int d = 0; d < m->hdim; d++) o[d] = 0.f;
    for (int j = 0; j < n; j++) oc_axpy_bf16(o, V + (size_t)j * s->kvdim, sc[j] * inv, m->hdim);
}

static void quantize_rows(const float *x, int nt, int k, oc_q8k *y) {
    for (int t = 0; t < nt; t++) oc_quantize_q8k(x + (size_t)t * k, k, y + (size_t)t * (k / QK));
}

/* forward_batch, CPU branch of src/model.c:798-901 (the order of every operation is kept). */
int oc_forward(oc_state *s, const int *toks, int nt, int pos0, int want_logits, float *logits) {
    const oc_model *m = &s->m;
    const int H = m->hidden;
    if (nt < 1 || nt > s->cap_nt || pos0 < 0 || pos0 + nt > m->ctx) return -1;
    for (int t = 0; t < nt; t++)
        if (toks[t] < 0 || toks[t] >= m->embd.n) return -1;
    for (int t = 0; t < nt; t++) oc_dequant_row(&m->embd, toks[t], s->h + (size_t)t * H);
    for (int li = 0; li < m->n_layer; li++) {
        const oc_layer *L = &m->layers[li];
        for (int t = 0; t < nt; t++) oc_rmsnorm(s->h + (size_t)t * H, L->attn_norm, s->xn + (size_t)t * H, H, m->eps);
        quantize_rows(s->xn, nt, H, s->xq_h);
        oc_matvec(&L->wq, s->xn, s->xq_h, nt, s->q);
        oc_matvec(&L->wk, s->xn, s->xq_h, nt, s->k);
        oc_matvec(&L->wv, s->xn, s->xq_h, nt, s->v);
        for (int t = 0; t < nt; t++) {
            float *q = s->q + (size_t)t * s->qdim, *k = s->k + (size_t)t * s->kvdim, *v = s->v + (size_t)t * s->kvdim;
            rope(s, q, m->heads, pos0 + t);
            rope(s, k, m->kv_heads, pos0 + t);
            for (int h = 0; h < m->heads; h++) oc_rmsnorm(q + (size_t)h * m->hdim, L->q_norm, q + (size_t)h * m->hdim, m->hdim, m->eps);
            for (int h = 0; h < m->kv_heads; h++) oc_rmsnorm(k + (size_t)h * m->hdim, L->k_norm, k + (size_t)h * m->hdim, m->hdim, m->eps);
            const size_t off = ((size_t)li * m->ctx + (size_t)(pos0 + t)) * s->kvdim;
            for (int d = 0; d < s->kvdim; d++) {
                s->kc[off + d] = oc_f32_to_bf16(k[d]);
                s->vc[off + d] = oc_f32_to_bf16(v[d]);
            }
        }
#pragma omp parallel for schedule(dynamic, 1)
        for (int item = 0; item < nt * m->heads; item++) attn_item(s, li, pos0, item);
        quantize_rows(s->ao, nt, s->qdim, s->xq_q);
        oc_matvec(&L->wo, s->ao, s->xq_q, nt, s->tmp);
        for (size_t i = 0; i < (size_t)nt * H; i++) s->h[i] += s->tmp[i];

        for (int t = 0; t < nt; t++) oc_rmsnorm(s->h + (size_t)t * H, L->ffn_norm, s->xn + (size_t)t * H, H, m->eps);
        quantize_rows(s->xn, nt, H, s->xq_h);
        oc_matvec(&L->wg, s->xn, s->xq_h, nt, s->gate);
        oc_matvec(&L->wu, s->xn, s->xq_h, nt, s->up);
        for (size_t i = 0; i < (size_t)nt * m->ffn; i++) {
            const float g = s->gate[i];
            s->gate[i] = g / (1.0f + expf(-g)) * s->up[i];
        }
        quantize_rows(s->gate, nt, m->ffn, s->xq_f);
        oc_matvec(&L->wd, s->gate, s->xq_f, nt, s->tmp);
        for (size_t i = 0; i < (size_t)nt * H; i++) s->h[i] += s->tmp[i];
    }
    if (want_logits) {
        const float *last = s->h + (size_t)(nt - 1) * H;
        oc_rmsnorm(last, m->out_norm, s->xn, H, m->eps);
        quantize_rows(s->xn, 1, H, s->xq_h);
        oc_matvec(&m->outw, s->xn, s->xq_h, 1, logits);
    }
    return 0;
}

/* Greedy pick with first-index tie-break, src/model.c:945-948. */
int oc_argmax(const float *logits, int n) {
    int best = 0;
    float bv = logits[0];
    for (int j = 1; j < n; j++)
        if (logits[j] > bv) {
            bv = logits[j];
            best = j;
        }
    return best;
}

/* Greedy loop of src/model.c:914-958 on token ids (chunked prefill of `batch` tokens, then one
 * token per step; stop ids are not checked). */
int oc_generate(oc_state *s, const int *prompt, int n_prompt, int n_gen, int batch, int *out) {
    float *logits = (float *)malloc(sizeof(float) * (size_t)s->m.outw.n);
    if (batch < 1) batch = 1;
    if (batch > s->cap_nt) batch = s->cap_nt;
    for (int i = 0; i < n_prompt; i += batch) {
        const int nt = n_prompt - i < batch ? n_prompt - i : batch;
        if (oc_forward(s, prompt + i, nt, i, i + nt == n_prompt, logits)) {
            free(logits);
            return -1;
        }
    }
    int pos = n_prompt;
    for (int i = 0; i < n_gen; i++) {
        const int best = oc_argmax(logits, s->m.vocab_out);
        out[i] = best;
        if (i + 1 == n_gen) break;
        if (oc_forward(s, &best, 1, pos, 1, logits)) {
            free(logits);
            return -1;
        }
        pos++;
    }
    free(logits);
    return n_gen;
}


/* The reference's greedy loop gen_ids (src/model.c:914-958) from the prompt ids on (the chat
 * template and the tokenizer are outside the path): max_tokens capped at ctx - n (:925-926);
 * the K/V of the longest common prefix with the ids the cache holds is kept, at most n - 1
 * positions (:930-936); the rest of the prompt runs in chunks of `batch` (forward_tokens,
 * :904-909); then per step the first-index argmax (:945-948), a stop id ends the loop before it
 * is emitted (:949, tok_is_stop: src/tokenizer.c:179), and every emitted id but the last of a
 * full run is fed back (:950-953). Returns the number of ids written to out (-2: the prompt
 * leaves no room, -1: a bad id); *keep_out = the positions reused. */
int oc_gen_ids(oc_state *s, const int *prompt, int n, int max_tokens, int batch, const int *stop, int n_stop,
               int *out, int *keep_out) {
    const int ctx = s->m.ctx;
    if (n < 1) return -1;
    if (n + max_tokens > ctx) max_tokens = ctx - n;
    if (max_tokens <= 0) return -2;
    if (!s->cache_tok) s->cache_tok = (int *)calloc((size_t)ctx, sizeof(int));
    if (batch < 1) batch = 1;
    if (batch > s->cap_nt) batch = s->cap_nt;
    int keep = 0;
    while (keep < s->n_cache && keep < n - 1 && s->cache_tok[keep] == prompt[keep]) keep++;
    s->n_cache = keep;
    float *logits = (float *)malloc(sizeof(float) * (size_t)s->m.outw.n);
    for (int i = keep; i < n; i += batch) {
        const int nt = n - i < batch ? n - i : batch;
        if (oc_forward(s, prompt + i, nt, i, i + nt == n, logits)) {
            free(logits);
            return -1;
        }
    }
    memcpy(s->cache_tok + keep, prompt + keep, sizeof(int) * (size_t)(n - keep));
    s->n_cache = n;
    int ng = 0;
    for (int i = 0; i < max_tokens; i++) {
        const int best = oc_argmax(logits, s->m.vocab_out);
        int is_stop = 0;
        for (int j = 0; j < n_stop; j++) is_stop |= best == stop[j];
        if (is_stop) break;
        out[ng++] = best;
        if (i + 1 == max_tokens) break;
        if (oc_forward(s, &best, 1, s->n_cache, 1, logits)) {
            free(logits);
            return -1;
        }
        s->cache_tok[s->n_cache++] = best;
    }
    free(logits);
    if (keep_out) *keep_out = keep;
    return ng;
}
