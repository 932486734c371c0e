/*
 * kc_oracle.c -- CPU restatement of Kernelcore's K-quant LLM hot path (test infrastructure).
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP path, never part of the product.
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off: no fused multiply-add may change a
 * rounding, the reference's float order is reproduced operation by operation).
 * Citations are to files under the reference tree (arasheedu/Kernelcore).
 */
#include "kc_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ---- bytes and bits ---------------------------------------------------------------- */

static inline uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static inline int32_t rd32(const uint8_t* p) {
    int32_t v;
    memcpy(&v, p, 4);
    return v;
}
static inline int32_t sar(int32_t v, int s) { return v >> s; } /* arithmetic (gcc) */
static inline int32_t shl(int32_t v, int s) { return (int32_t)((uint32_t)v << s); }
/* signed byte i of w */
static inline int32_t byte_s(int32_t w, int i) { return sar(shl(w, 24 - 8 * i), 24); }

/* unsigned bytes of a times signed bytes of b, plus c (kc_dp4a, kernels/llm/matvec_q4k_q8.cu:14-27) */
static inline int32_t dp4a(int32_t a, int32_t b, int32_t c) {
    for (int i = 0; i < 4; ++i) c += ((a >> (8 * i)) & 255) * (int8_t)((uint32_t)b >> (8 * i));
    return c;
}

/* ---- fp16 ----------------------------------------------------------------------------- */

/* llm/llm_reference.cpp:284-309 */
float kco_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1Fu;
    uint32_t m = h & 0x3FFu, bits;
    if (e == 0) {
        if (m == 0) {
            bits = sign;
        } else { /* subnormal: shift the leading one up to bit 10 */
            int sh = 0;
            while ((m & 0x400u) == 0) {
                m <<= 1;
                ++sh;
            }
            bits = sign | (uint32_t)(127 - 15 - (sh - 1)) << 23 | (m & 0x3FFu) << 13;
        }
    } else if (e == 31) {
        bits = sign | 0x7F800000u | m << 13;
    } else {
        bits = sign | (e + 127 - 15) << 23 | m << 13;
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* llm/llm_reference.cpp:735-744 (set_rows_f16's conversion) */
uint16_t kco_f32_to_f16(float x) {
    const uint32_t sign = x < 0.0f ? 0x8000u : 0u;
    const float a = fabsf(x);
    if (!(a < 65520.0f)) return (uint16_t)(sign | 0x7bffu);
    if (a < 6.103515625e-05f) return (uint16_t)(sign | (uint32_t)nearbyintf(a * 16777216.0f));
    int e = 0;
    const float f = frexpf(a, &e); /* a = f * 2^e, f in [0.5, 1) */
    const uint32_t m = (uint32_t)nearbyintf((f * 2.0f - 1.0f) * 1024.0f);
    return (uint16_t)(sign | (((uint32_t)(e - 1 + 15) << 10) + m));
}

/* ---- K-quant dequantization ------------------------------------------------------------ */

/* ggml get_scale_min_k4 (llm/llm_reference.cpp:328-337) */
static void scale_min_k4(int j, const uint8_t* q, int* sc, int* m) {
    if (j < 4) {
        *sc = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *sc = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
        *m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

/* llm/llm_reference.cpp:342-359: y = d1 * q - m1, d1 = d * sc, m1 = dmin * m (two roundings) */
void kco_dequant_row_q4k(const uint8_t* src, int k, float* out) {
    for (int s = 0; s < k / 256; ++s) {
        const uint8_t* b = src + (size_t)s * 144;
        const float d = kco_f16_to_f32(rd16(b)), dmin = kco_f16_to_f32(rd16(b + 2));
        const uint8_t* q = b + 16;
        float* y = out + (size_t)s * 256;
        for (int j = 0; j < 4; ++j) {
            int sc, m;
            scale_min_k4(2 * j, b + 4, &sc, &m);
            const float d1 = d * (float)sc, m1 = dmin * (float)m;
            scale_min_k4(2 * j + 1, b + 4, &sc, &m);
            const float d2 = d * (float)sc, m2 = dmin * (float)m;
            for (int l = 0; l < 32; ++l) y[64 * j + l] = d1 * (float)(q[32 * j + l] & 0xF) - m1;
            for (int l = 0; l < 32; ++l) y[64 * j + 32 + l] = d2 * (float)(q[32 * j + l] >> 4) - m2;
        }
    }
}

/* llm/llm_reference.cpp:361-383: y = (d * sc) * (q - 32), q = ql nibble | qh bits << 4 */
void kco_dequant_row_q6k(const uint8_t* src, int k, float* out) {
    for (int s = 0; s < k / 256; ++s) {
        const uint8_t* b = src + (size_t)s * 210;
        const uint8_t* ql = b;
        const uint8_t* qh = b + 128;
        const int8_t* sc = (const int8_t*)(b + 192);
        const float d = kco_f16_to_f32(rd16(b + 208));
        float* y = out + (size_t)s * 256;
        for (int n = 0; n < 2; ++n) {
            for (int l = 0; l < 32; ++l) {
                const int is = l / 16;
                const int h = qh[32 * n + l];
                const int q1 = (int)((ql[64 * n + l] & 0xF) | ((h & 3) << 4)) - 32;
                const int q2 = (int)((ql[64 * n + l + 32] & 0xF) | (((h >> 2) & 3) << 4)) - 32;
                const int q3 = (int)((ql[64 * n + l] >> 4) | (((h >> 4) & 3) << 4)) - 32;
                const int q4 = (int)((ql[64 * n + l + 32] >> 4) | (((h >> 6) & 3) << 4)) - 32;
                y[128 * n + l] = d * (float)sc[8 * n + is + 0] * (float)q1;
                y[128 * n + l + 32] = d * (float)sc[8 * n + is + 2] * (float)q2;
                y[128 * n + l + 64] = d * (float)sc[8 * n + is + 4] * (float)q3;
                y[128 * n + l + 96] = d * (float)sc[8 * n + is + 6] * (float)q4;
            }
        }
    }
}

/* ---- activation quantizers ---------------------------------------------------------------- */

/* x*id rounded half away from zero, clamped to +-127 (kernels/llm/quantize_q8x4.cu:25-33) */
static inline int q8_round(float t) {
    int q = t >= 0.0f ? (int)(t + 0.5f) : (int)(t - 0.5f);
    return q > 127 ? 127 : q < -127 ? -127 : q;
}
/* max |x| as fmaxf(amax, fmaxf(v, -v)) (kernels/llm/quantize_q8x4.cu:15-19) */
static inline float amax_of(const float* x, int n) {
    float amax = 0.0f;
    for (int i = 0; i < n; ++i) {
        const float a = x[i] > 0.0f - x[i] ? x[i] : 0.0f - x[i];
        amax = amax > a ? amax : a;
    }
    return amax;
}

/* llm/llm_reference.cpp:79-104 */
void kco_quantize_q8x4(const float* x, int32_t* xq, float* xd, int count) {
    for (int b = 0; b < count; ++b) {
        const float* xb = x + (size_t)b * 32;
        const float d = amax_of(xb, 32) / 127.0f;
        const float id = d > 0.0f ? 1.0f / d : 0.0f;
        int sum = 0;
        for (int w = 0; w < 8; ++w) {
            uint32_t word = 0;
            for (int i = 0; i < 4; ++i) {
                const int q = q8_round(xb[w * 4 + i] * id);
                sum += q;
                word |= ((uint32_t)q & 255u) << (i * 8);
            }
            xq[(size_t)b * 8 + w] = (int32_t)word;
        }
        xd[(size_t)b * 2] = d;
        xd[(size_t)b * 2 + 1] = (float)sum;
    }
}

/* kernels/llm/quantize_cols.cu:27-52: slot = [nb*8 words | nb*2 floats | nb floats (untouched)] */
void kco_quantize_cols(const float* x, int32_t* q, int k, int ncols) {
    const int nb = k / 32;
    for (int c = 0; c < ncols; ++c) {
        int32_t* slot = q + (size_t)c * nb * 11;
        kco_quantize_q8x4(x + (size_t)c * k, slot, (float*)(slot + nb * 8), nb);
    }
}

/* llm/llm_reference.cpp:491-527: slot = [nsb*64 words | nsb floats d | nsb*16 sums of 16 |
 * nsb*4 words: sums of 32 B as bytes, B>>6 (sums 0-3, 4-7) then B&63] */
void kco_quantize_q8k(const float* x, int32_t* q, int nsb) {
    float* sc = (float*)(q + (size_t)nsb * 64);
    int32_t* bs = q + (size_t)nsb * 65;
    for (int s = 0; s < nsb; ++s) {
        const float* xs = x + (size_t)s * 256;
        const float d = amax_of(xs, 256) / 127.0f;
        const float id = d > 0.0f ? 1.0f / d : 0.0f;
        for (int g = 0; g < 16; ++g) {
            int sum = 0;
            for (int w = 0; w < 4; ++w) {
                uint32_t word = 0;
                for (int i = 0; i < 4; ++i) {
                    const int v = q8_round(xs[g * 16 + w * 4 + i] * id);
                    sum += v;
                    word |= ((uint32_t)v & 255u) << (i * 8);
                }
                q[(size_t)s * 64 + g * 4 + w] = (int32_t)word;
            }
            bs[(size_t)s * 16 + g] = sum;
        }
        sc[s] = d;
        uint32_t pw[4] = {0, 0, 0, 0};
        for (int i = 0; i < 8; ++i) {
            const int32_t b = bs[(size_t)s * 16 + 2 * i] + bs[(size_t)s * 16 + 2 * i + 1];
            pw[i / 4] |= ((uint32_t)sar(b, 6) & 255u) << (8 * (i % 4));
            pw[2 + i / 4] |= (uint32_t)(b & 63) << (8 * (i % 4));
        }
        for (int i = 0; i < 4; ++i) q[(size_t)nsb * 81 + (size_t)s * 4 + i] = (int32_t)pw[i];
    }
}

void kco_quantize_cols_k(const float* x, int32_t* q, int k, int ncols) {
    const int nsb = k / 256;
    for (int c = 0; c < ncols; ++c) kco_quantize_q8k(x + (size_t)c * k, q + (size_t)c * nsb * 85, nsb);
}

/* ---- matvecs ------------------------------------------------------------------------------ */

/* The 8 scales and mins of a Q4_K super-block, four per word (kernels/llm/matvec_q4k_q8.cu:52-56) */
typedef struct {
    int32_t sclo, mlo, schi, mhi;
} q4k_scales;
static inline q4k_scales q4k_unpack(const uint8_t* b) {
    const int32_t s0 = rd32(b + 4), s1 = rd32(b + 8), s2 = rd32(b + 12);
    q4k_scales r;
    r.sclo = s0 & 0x3F3F3F3F;
    r.mlo = s1 & 0x3F3F3F3F;
    r.schi = (s2 & 0x0F0F0F0F) | (sar(s0, 2) & 0x30303030);
    r.mhi = (sar(s2, 4) & 0x0F0F0F0F) | (sar(s1, 2) & 0x30303030);
    return r;
}

/* One row of llm/llm_reference.cpp:413-445 */
static float row_q4k_q8(const uint8_t* wr, const int32_t* xq, const float* xd, int nsb) {
    float acc = 0.0f;
    for (int s = 0; s < nsb; ++s) {
        const uint8_t* blk = wr + (size_t)s * 144;
        const float d = kco_f16_to_f32(rd16(blk)), dmin = kco_f16_to_f32(rd16(blk + 2));
        const q4k_scales u = q4k_unpack(blk);
        float fd = 0.0f, fm = 0.0f;
        for (int j = 0; j < 4; ++j) {
            const int b = s * 8 + j * 2;
            int32_t da = 0, db = 0;
            for (int w = 0; w < 8; ++w) {
                const int32_t q = rd32(blk + 16 + 4 * (j * 8 + w));
                da = dp4a(q & 0x0F0F0F0F, xq[b * 8 + w], da);
                db = dp4a(sar(q, 4) & 0x0F0F0F0F, xq[b * 8 + 8 + w], db);
            }
            const int sh = 16 * (j & 1);
            const int32_t scw = j < 2 ? u.sclo : u.schi, mw = j < 2 ? u.mlo : u.mhi;
            const int32_t sca = sar(scw, sh) & 255, scb = sar(scw, sh + 8) & 255;
            const int32_t ma = sar(mw, sh) & 255, mb = sar(mw, sh + 8) & 255;
            fd += (float)(sca * da) * xd[b * 2] + (float)(scb * db) * xd[b * 2 + 2];
            fm += (float)ma * (xd[b * 2] * xd[b * 2 + 1]) + (float)mb * (xd[b * 2 + 2] * xd[b * 2 + 3]);
        }
        acc += d * fd - dmin * fm;
    }
    return acc;
}

/* One row of llm/llm_reference.cpp:447-489 */
static float row_q6k_q8(const uint8_t* wr, const int32_t* xq, const float* xd, int nsb) {
    float acc = 0.0f;
    for (int s = 0; s < nsb; ++s) {
        const uint8_t* blk = wr + (size_t)s * 210;
        const float d = kco_f16_to_f32(rd16(blk + 208));
        for (int n = 0; n < 2; ++n) {
            const int b = s * 8 + n * 4;
            int32_t da[4] = {0, 0, 0, 0}, db[4] = {0, 0, 0, 0}, sa[4] = {0, 0, 0, 0};
            for (int w = 0; w < 8; ++w) {
                const int32_t qa = rd32(blk + 4 * (16 * n + w));     /* ql bytes 64n + 4w */
                const int32_t qc = rd32(blk + 4 * (16 * n + 8 + w)); /* ql bytes 64n + 32 + 4w */
                const int32_t h = rd32(blk + 128 + 4 * (8 * n + w)); /* qh bytes 32n + 4w */
                const int32_t q[4] = {(qa & 0x0F0F0F0F) | (shl(h, 4) & 0x30303030),
                                      (qc & 0x0F0F0F0F) | (shl(h, 2) & 0x30303030),
                                      (sar(qa, 4) & 0x0F0F0F0F) | (h & 0x30303030),
                                      (sar(qc, 4) & 0x0F0F0F0F) | (sar(h, 2) & 0x30303030)};
                for (int t = 0; t < 4; ++t) {
                    const int32_t x = xq[b * 8 + 8 * t + w];
                    if (w < 4) {
                        da[t] = dp4a(q[t], x, da[t]);
                        sa[t] = dp4a(0x01010101, x, sa[t]);
                    } else {
                        db[t] = dp4a(q[t], x, db[t]);
                    }
                }
            }
            const int32_t sw0 = rd32(blk + 192 + 8 * n), sw1 = rd32(blk + 192 + 8 * n + 4);
            int32_t is[4];
            for (int t = 0; t < 4; ++t) {
                const int32_t sw = t < 2 ? sw0 : sw1;
                const int lo = 2 * (t & 1);
                const int32_t sb = (int32_t)xd[(b + t) * 2 + 1] - sa[t];
                is[t] = byte_s(sw, lo) * (da[t] - 32 * sa[t]) + byte_s(sw, lo + 1) * (db[t] - 32 * sb);
            }
            acc += d * ((float)is[0] * xd[b * 2] + (float)is[1] * xd[b * 2 + 2] + (float)is[2] * xd[b * 2 + 4] +
                        (float)is[3] * xd[b * 2 + 6]);
        }
    }
    return acc;
}

/* One row of llm/llm_reference.cpp:529-562 */
static float row_q4k_q8k(const uint8_t* wr, const int32_t* xq, int nsb) {
    const float* xd = (const float*)(xq + (size_t)nsb * 64);
    const int32_t* bs = xq + (size_t)nsb * 65;
    float acc = 0.0f;
    for (int s = 0; s < nsb; ++s) {
        const uint8_t* blk = wr + (size_t)s * 144;
        const float d = kco_f16_to_f32(rd16(blk)), dmin = kco_f16_to_f32(rd16(blk + 2));
        const q4k_scales u = q4k_unpack(blk);
        int32_t is = 0, im = 0;
        for (int j = 0; j < 4; ++j) {
            const int32_t* xs = xq + (size_t)s * 64 + j * 16;
            int32_t da = 0, db = 0;
            for (int w = 0; w < 8; ++w) {
                const int32_t q = rd32(blk + 16 + 4 * (j * 8 + w));
                da = dp4a(q & 0x0F0F0F0F, xs[w], da);
                db = dp4a(sar(q, 4) & 0x0F0F0F0F, xs[8 + w], db);
            }
            const int sh = 16 * (j & 1);
            const int32_t scw = j < 2 ? u.sclo : u.schi, mw = j < 2 ? u.mlo : u.mhi;
            is += (sar(scw, sh) & 255) * da + (sar(scw, sh + 8) & 255) * db;
            const int32_t* b = bs + (size_t)s * 16 + j * 4;
            im += (sar(mw, sh) & 255) * (b[0] + b[1]) + (sar(mw, sh + 8) & 255) * (b[2] + b[3]);
        }
        acc += (d * xd[s]) * (float)is - (dmin * xd[s]) * (float)im;
    }
    return acc;
}

/* One row of llm/llm_reference.cpp:564-596 */
static float row_q6k_q8k(const uint8_t* wr, const int32_t* xq, int nsb) {
    const float* xd = (const float*)(xq + (size_t)nsb * 64);
    const int32_t* bs = xq + (size_t)nsb * 65;
    float acc = 0.0f;
    for (int s = 0; s < nsb; ++s) {
        const uint8_t* blk = wr + (size_t)s * 210;
        const float d = kco_f16_to_f32(rd16(blk + 208));
        int32_t is = 0;
        for (int n = 0; n < 2; ++n) {
            for (int t = 0; t < 4; ++t) {
                const int32_t* xs = xq + (size_t)s * 64 + (n * 4 + t) * 8;
                int32_t da = 0, db = 0;
                for (int w = 0; w < 8; ++w) {
                    const int32_t qa = rd32(blk + 4 * (16 * n + 8 * (t & 1) + w));
                    const int32_t h = rd32(blk + 128 + 4 * (8 * n + w));
                    const int32_t q = (sar(qa, 4 * (t >> 1)) & 0x0F0F0F0F) | (shl(sar(h, 2 * t), 4) & 0x30303030);
                    if (w < 4) da = dp4a(q, xs[w], da);
                    else db = dp4a(q, xs[w], db);
                }
                const int32_t sw = rd32(blk + 192 + 4 * (2 * n + (t >> 1)));
                const int lo = 2 * (t & 1);
                const int32_t* b = bs + (size_t)s * 16 + (n * 4 + t) * 2;
                is += byte_s(sw, lo) * (da - 32 * b[0]) + byte_s(sw, lo + 1) * (db - 32 * b[1]);
            }
        }
        acc += (d * xd[s]) * (float)is;
    }
    return acc;
}

void kco_matvec_q4k_q8(const uint8_t* w, const int32_t* xq, const float* xd, float* y, int rows, int k) {
    const int nsb = k / 256;
    for (int r = 0; r < rows; ++r) y[r] = row_q4k_q8(w + (size_t)r * nsb * 144, xq, xd, nsb);
}
void kco_matvec_q6k_q8(const uint8_t* w, const int32_t* xq, const float* xd, float* y, int rows, int k) {
    const int nsb = k / 256;
    for (int r = 0; r < rows; ++r) y[r] = row_q6k_q8(w + (size_t)r * nsb * 210, xq, xd, nsb);
}
void kco_matvec_q4k_q8k(const uint8_t* w, const int32_t* slot, float* y, int rows, int k) {
    const int nsb = k / 256;
    for (int r = 0; r < rows; ++r) y[r] = row_q4k_q8k(w + (size_t)r * nsb * 144, slot, nsb);
}
void kco_matvec_q6k_q8k(const uint8_t* w, const int32_t* slot, float* y, int rows, int k) {
    const int nsb = k / 256;
    for (int r = 0; r < rows; ++r) y[r] = row_q6k_q8k(w + (size_t)r * nsb * 210, slot, nsb);
}

/* matmul_*_q8x{4,8}: per column, bit-identical to the matvec (tests/test_llm_kernels.cpp:277-340) */
void kco_matmul_q4k_q8(const uint8_t* w, const int32_t* q, float* y, int rows, int k, int ncols) {
    const int nb = k / 32;
    for (int c = 0; c < ncols; ++c) {
        const int32_t* slot = q + (size_t)c * nb * 11;
        kco_matvec_q4k_q8(w, slot, (const float*)(slot + nb * 8), y + (size_t)c * rows, rows, k);
    }
}
void kco_matmul_q6k_q8(const uint8_t* w, const int32_t* q, float* y, int rows, int k, int ncols) {
    const int nb = k / 32;
    for (int c = 0; c < ncols; ++c) {
        const int32_t* slot = q + (size_t)c * nb * 11;
        kco_matvec_q6k_q8(w, slot, (const float*)(slot + nb * 8), y + (size_t)c * rows, rows, k);
    }
}
void kco_matmul_q4k_q8k(const uint8_t* w, const int32_t* q, float* y, int rows, int k, int ncols) {
    const int nsb = k / 256;
    for (int c = 0; c < ncols; ++c) kco_matvec_q4k_q8k(w, q + (size_t)c * nsb * 85, y + (size_t)c * rows, rows, k);
}
void kco_matmul_q6k_q8k(const uint8_t* w, const int32_t* q, float* y, int rows, int k, int ncols) {
    const int nsb = k / 256;
    for (int c = 0; c < ncols; ++c) kco_matvec_q6k_q8k(w, q + (size_t)c * nsb * 85, y + (size_t)c * rows, rows, k);
}

/* ---- layer ops -------------------------------------------------------------------------------- */

/* llm/llm_reference.cpp:141-151 (kernels/llm/rms_norm.cu) */
void kco_rms_norm(const float* x, const float* w, float* y, int n, int rows, float eps) {
    for (int row = 0; row < rows; ++row) {
        const float* xr = x + (size_t)row * n;
        float* yr = y + (size_t)row * n;
        float ss = 0.0f;
        for (int j = 0; j < n; ++j) ss += xr[j] * xr[j];
        const float r = 1.0f / sqrtf(ss / (float)n + eps);
        for (int j = 0; j < n; ++j) yr[j] = xr[j] * r * w[j];
    }
}

/* llm/llm_reference.cpp:600-602 */
void kco_mul_rows(const float* x, const float* w, float* y, int n, int count) {
    for (int i = 0; i < count; ++i) y[i] = x[i] * w[i % n];
}

/* llm/llm_reference.cpp:240-242: g / (1 + 2^(-g log2 e)) * u */
void kco_silu_mul(const float* g, const float* u, float* out, int count) {
    for (int i = 0; i < count; ++i) out[i] = g[i] / (1.0f + exp2f(-g[i] * 1.44269504f)) * u[i];
}

void kco_add(const float* a, const float* b, float* out, int count) {
    for (int i = 0; i < count; ++i) out[i] = a[i] + b[i];
}

static void rope_impl(const float* x, float* y, const int32_t* pos, const float* ff, int head_dim, int n_head,
                      int n_tokens, float log2_base, int neox, int turns) {
    const int pairs = head_dim / 2;
    for (int t = 0; t < n_tokens; ++t) {
        for (int i = 0; i < pairs; ++i) {
            const float theta = (float)pos[t] * exp2f(-(float)i / (float)pairs * log2_base) / ff[i];
            float c, s;
            if (turns) { /* llm/llm_reference.cpp:627-628 */
                const float tu = theta * 0.159154943f;
                c = cosf(tu * 6.28318548f);
                s = sinf(tu * 6.28318548f);
            } else { /* kernels/llm/rope_ggml.cu:30-31 */
                c = cosf(theta);
                s = sinf(theta);
            }
            for (int h = 0; h < n_head; ++h) {
                const size_t row = ((size_t)t * n_head + h) * head_dim;
                const size_t a = neox ? row + i : row + 2 * i, b = neox ? a + pairs : a + 1;
                const float x0 = x[a], x1 = x[b];
                y[a] = x0 * c - x1 * s;
                y[b] = x0 * s + x1 * c;
            }
        }
    }
}
void kco_rope_ggml(const float* x, float* y, const int32_t* pos, const float* ff, int head_dim, int n_head,
                   int n_tokens, float log2_base, int neox) {
    rope_impl(x, y, pos, ff, head_dim, n_head, n_tokens, log2_base, neox, 0);
}
void kco_rope_ggml_turns(const float* x, float* y, const int32_t* pos, const float* ff, int head_dim, int n_head,
                         int n_tokens, float log2_base, int neox) {
    rope_impl(x, y, pos, ff, head_dim, n_head, n_tokens, log2_base, neox, 1);
}

/* llm/llm_reference.cpp:651-667 */
void kco_add_sumsq_f(const float* a, const float* b, float* out, int32_t* q, int n, int rows) {
    const int nb = n / 32;
    for (int row = 0; row < rows; ++row) {
        float* ss = (float*)(q + (size_t)row * nb * 11 + nb * 10);
        for (int bl = 0; bl < nb; ++bl) {
            float s = 0.0f;
            for (int i = 0; i < 32; ++i) {
                const size_t o = (size_t)row * n + (size_t)bl * 32 + i;
                const float v = a[o] + b[o];
                out[o] = v;
                s += v * v;
            }
            ss[bl] = s;
        }
    }
}

/* llm/llm_reference.cpp:669-682 */
void kco_sumsq_part(const float* x, int32_t* q, int n, int rows) {
    const int nb = n / 32;
    for (int row = 0; row < rows; ++row) {
        float* ss = (float*)(q + (size_t)row * nb * 11 + nb * 10);
        for (int bl = 0; bl < nb; ++bl) {
            float s = 0.0f;
            for (int i = 0; i < 32; ++i) {
                const float v = x[(size_t)row * n + (size_t)bl * 32 + i];
                s += v * v;
            }
            ss[bl] = s;
        }
    }
}

static float rms_scale(const float* ss, int nb, int n, float eps) {
    float tot = 0.0f;
    for (int j = 0; j < nb; ++j) tot += ss[j];
    return 1.0f / sqrtf(tot / (float)n + eps);
}

/* llm/llm_reference.cpp:684-700 (kernels/llm/norm_mul_q8_f.cu) */
void kco_norm_mul_q8(const float* x, const float* w, float* y, int32_t* q, int n, int rows, float eps) {
    const int nb = n / 32;
    for (int row = 0; row < rows; ++row) {
        int32_t* qr = q + (size_t)row * nb * 11;
        const float r = rms_scale((const float*)(qr + nb * 10), nb, n, eps);
        for (int bl = 0; bl < nb; ++bl) {
            float* yb = y + (size_t)row * n + (size_t)bl * 32;
            const float* xb = x + (size_t)row * n + (size_t)bl * 32;
            for (int i = 0; i < 32; ++i) yb[i] = xb[i] * r * w[bl * 32 + i];
            float xd[2];
            kco_quantize_q8x4(yb, qr + bl * 8, xd, 1);
            ((float*)(qr + nb * 8))[bl * 2] = xd[0];
            ((float*)(qr + nb * 8))[bl * 2 + 1] = xd[1];
        }
    }
}

/* llm/llm_reference.cpp:702-713 (kernels/llm/norm_mul_q8k_f.cu) */
void kco_norm_mul_q8k(const float* x, const float* w, float* y, int32_t* q, const int32_t* sq, int n, int rows,
                      float eps) {
    const int nb = n / 32;
    for (int row = 0; row < rows; ++row) {
        const float r = rms_scale((const float*)(sq + (size_t)row * nb * 11 + nb * 10), nb, n, eps);
        for (int i = 0; i < n; ++i) y[(size_t)row * n + i] = x[(size_t)row * n + i] * r * w[i];
        kco_quantize_q8k(y + (size_t)row * n, q + (size_t)row * (n / 256 * 85), n / 256);
    }
}

/* llm/llm_reference.cpp:719-727 (kernels/llm/silu_mul_q8x4f.cu) */
void kco_silu_mul_q8f(const float* g, const float* u, float* y, int32_t* q, int n, int cols) {
    const int nb = n / 32;
    kco_silu_mul(g, u, y, n * cols);
    for (int c = 0; c < cols; ++c) {
        int32_t* qc = q + (size_t)c * nb * 11;
        kco_quantize_q8x4(y + (size_t)c * n, qc, (float*)(qc + nb * 8), nb);
    }
}

/* llm/llm_reference.cpp:714-717 (kernels/llm/silu_mul_q8kf.cu) */
void kco_silu_mul_q8k(const float* g, const float* u, float* y, int32_t* q, int n, int cols) {
    kco_silu_mul(g, u, y, n * cols);
    for (int c = 0; c < cols; ++c) kco_quantize_q8k(y + (size_t)c * n, q + (size_t)c * (n / 256 * 85), n / 256);
}

/* llm/llm_reference.cpp:766-772: rows outside [0, dst_rows) are skipped; the low 32-bit word of
 * the int64 index is the row (kernels/llm/set_rows_f16.cu:77) */
void kco_set_rows_f16(const float* src, const int64_t* idx, uint16_t* dst, int pairs, int rows, int src_row,
                      int dst_row, int dst_rows) {
    for (int r = 0; r < rows; ++r) {
        const int row = (int)(int32_t)(uint32_t)(uint64_t)idx[r];
        if (row < 0 || row >= dst_rows) continue;
        for (int j = 0; j < 2 * pairs; ++j)
            dst[(size_t)row * dst_row * 2 + j] = kco_f32_to_f16(src[(size_t)r * src_row + j]);
    }
}

/* llm/llm_reference.cpp:773-798 */
void kco_flash_attn_f16(const float* q, const uint16_t* k, const uint16_t* v, const uint16_t* mask, float* out,
                        const kco_fa_dims* d, float scale) {
    float* s = (float*)malloc(sizeof(float) * (size_t)(d->T > 0 ? d->T : 1));
    for (int i = 0; i < d->N; ++i) {
        for (int h = 0; h < d->H; ++h) {
            const int kvh = h / d->group;
            const float* qh = q + (size_t)i * d->q_tok + (size_t)h * d->q_head;
            float mx = -INFINITY;
            for (int t = 0; t < d->T; ++t) {
                const uint16_t* kr = k + ((size_t)t * d->k_row + (size_t)kvh * d->k_head) * 2;
                float a = 0.0f;
                for (int j = 0; j < d->D; ++j) a += qh[j] * kco_f16_to_f32(kr[j]);
                const float mv = d->has_mask ? kco_f16_to_f32(mask[(size_t)i * d->m_row * 2 + t]) : 0.0f;
                s[t] = a * scale + mv;
                mx = mx > s[t] ? mx : s[t];
            }
            float sum = 0.0f;
            for (int t = 0; t < d->T; ++t) sum += (s[t] = exp2f((s[t] - mx) * 1.44269504f));
            for (int dd = 0; dd < d->D; ++dd) {
                float a = 0.0f;
                for (int t = 0; t < d->T; ++t)
                    a += s[t] * kco_f16_to_f32(v[((size_t)t * d->v_row + (size_t)kvh * d->v_head) * 2 + dd]);
                out[((size_t)i * d->H + h) * d->D + dd] = a / sum;
            }
        }
    }
    free(s);
}

/* ---- f32 -> Q4_K / Q6_K weight quantizers ------------------------------------------------
 *
 * Third-party arithmetic: the reference has no quantizer (its tests fabricate random blocks,
 * tests/test_llm_kernels.cpp:209-219); its weights come from GGUF files written by ggml
 * (llama.cpp, not vendored, version unpinned; build ids c2eb060b2 / 8221f87ce in
 * bench_chart/results.json:48,56). These restate the published steps of ggml's reference
 * quantizers quantize_row_q4_K_ref and quantize_row_q6_K_ref with their scale searches
 * (make_qkx2_quants for Q4_K: weighted least-squares fit of a scale and a min per sub-block of 32
 * over 21 candidate inverse scales; make_qx_quants with rmse_type 1 for Q6_K: a scale per
 * sub-block of 16 chosen among 19 candidates by the x^2-weighted fit). Parity with a given ggml
 * build is unpinned; tests/test_quantizer.py pins the invariants the format and the method fix. */

/* round half to even (ggml's nearest_int for |f| < 2^22) */
static inline int nearest_even(float f) { return (int)rintf(f); }
static inline int clampi(int v, int lo, int hi) { return v < lo ? lo : v > hi ? hi : v; }

/* IEEE binary16, round to nearest even, overflow to infinity (ggml_fp32_to_fp16). */
uint16_t kco_f32_to_f16_rne(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    const uint32_t sign = (u >> 16) & 0x8000u;
    const uint32_t ax = u & 0x7fffffffu;
    if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);          /* NaN */
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);         /* rounds to >= 65536: inf */
    if (ax < 0x38800000u) {                                          /* below 2^-14: subnormal or 0 */
        if (ax < 0x33000000u) return (uint16_t)sign;                   /* below 2^-25: rounds to 0 */
        const uint32_t mant = (ax & 0x7fffffu) | 0x800000u;
        const int shift = 126 - (int)(ax >> 23);                       /* 14..24 */
        uint32_t h = mant >> shift;
        const uint32_t rem = mant & ((1u << shift) - 1), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (h & 1))) ++h;
        return (uint16_t)(sign | h);
    }
    uint32_t h = ((ax >> 13) - (112u << 10));
    const uint32_t rem = ax & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1))) ++h;
    return (uint16_t)(sign | h);
}

/* One sub-block of 32 for Q4_K: L[i] in 0..15 and (scale, -min) so that x ~ scale * L + min,
 * min <= 0; weights w. (make_qkx2_quants(32, 15, x, w, L, &the_min, Laux, -1, 0.1, 20, false).) */
static float fit_q4_subblock(const float* x, const float* w, uint8_t* L, float* neg_min) {
    float lo = x[0], hi = x[0], sw = w[0], sx = w[0] * x[0];
    for (int i = 1; i < 32; ++i) {
        if (x[i] < lo) lo = x[i];
        if (x[i] > hi) hi = x[i];
        sw += w[i];
        sx += w[i] * x[i];
    }
    if (lo > 0.0f) lo = 0.0f;
    if (hi == lo) {
        memset(L, 0, 32);
        *neg_min = -lo;
        return 0.0f;
    }
    float iscale = 15.0f / (hi - lo);
    float scale = 1.0f / iscale;
    float best = 0.0f;
    for (int i = 0; i < 32; ++i) {
        const int l = clampi(nearest_even(iscale * (x[i] - lo)), 0, 15);
        L[i] = (uint8_t)l;
        const float diff = scale * (float)l + lo - x[i];
        best += w[i] * (diff * diff);
    }
    uint8_t cand[32];
    for (int step = 0; step <= 20; ++step) {
        iscale = (-1.0f + 0.1f * (float)step + 15.0f) / (hi - lo);
        float sl = 0.0f, sl2 = 0.0f, sxl = 0.0f;
        for (int i = 0; i < 32; ++i) {
            const int l = clampi(nearest_even(iscale * (x[i] - lo)), 0, 15);
            cand[i] = (uint8_t)l;
            sl += w[i] * (float)l;
            sl2 += w[i] * (float)l * (float)l;
            sxl += w[i] * (float)l * x[i];
        }
        const float det = sw * sl2 - sl * sl;
        if (det > 0.0f) {
            float s = (sw * sxl - sx * sl) / det;
            float m = (sl2 * sx - sl * sxl) / det;
            if (m > 0.0f) {
                m = 0.0f;
                s = sxl / sl2;
            }
            float err = 0.0f;
            for (int i = 0; i < 32; ++i) {
                const float diff = s * (float)cand[i] + m - x[i];
                err += w[i] * (diff * diff);
            }
            if (err < best) {
                memcpy(L, cand, 32);
                best = err;
                scale = s;
                lo = m;
            }
        }
    }
    *neg_min = -lo;
    return scale;
}

void kco_quantize_row_q4k(const float* x, uint8_t* out, int k) {
    for (int sb = 0; sb < k / 256; ++sb) {
        const float* xs = x + (size_t)sb * 256;
        uint8_t* b = out + (size_t)sb * 144;
        uint8_t L[256];
        float scales[8], mins[8], w[32];
        float max_scale = 0.0f, max_min = 0.0f;
        for (int j = 0; j < 8; ++j) {
            float sum_x2 = 0.0f;
            for (int l = 0; l < 32; ++l) sum_x2 += xs[32 * j + l] * xs[32 * j + l];
            const float av = sqrtf(sum_x2 / 32.0f);
            for (int l = 0; l < 32; ++l) w[l] = av + fabsf(xs[32 * j + l]);
            scales[j] = fit_q4_subblock(xs + 32 * j, w, L + 32 * j, &mins[j]);
            if (scales[j] > max_scale) max_scale = scales[j];
            if (mins[j] > max_min) max_min = mins[j];
        }
        const float inv_scale = max_scale > 0.0f ? 63.0f / max_scale : 0.0f;
        const float inv_min = max_min > 0.0f ? 63.0f / max_min : 0.0f;
        memset(b, 0, 144);
        uint8_t* sc = b + 4;
        for (int j = 0; j < 8; ++j) {
            uint8_t ls = (uint8_t)nearest_even(inv_scale * scales[j]);
            uint8_t lm = (uint8_t)nearest_even(inv_min * mins[j]);
            if (ls > 63) ls = 63;
            if (lm > 63) lm = 63;
            if (j < 4) {
                sc[j] = ls;
                sc[j + 4] = lm;
            } else {
                sc[j + 4] = (uint8_t)((ls & 0xF) | ((lm & 0xF) << 4));
                sc[j - 4] |= (uint8_t)((ls >> 4) << 6);
                sc[j] |= (uint8_t)((lm >> 4) << 6);
            }
        }
        const uint16_t d16 = kco_f32_to_f16_rne(max_scale / 63.0f), m16 = kco_f32_to_f16_rne(max_min / 63.0f);
        b[0] = (uint8_t)d16, b[1] = (uint8_t)(d16 >> 8), b[2] = (uint8_t)m16, b[3] = (uint8_t)(m16 >> 8);
        for (int j = 0; j < 8; ++j) {
            int s6, m6;
            scale_min_k4(j, sc, &s6, &m6);
            const float d = kco_f16_to_f32(d16) * (float)s6;
            if (d == 0.0f) continue;  /* the sub-block keeps the fit's L */
            const float dm = kco_f16_to_f32(m16) * (float)m6;
            for (int i = 0; i < 32; ++i) L[32 * j + i] = (uint8_t)clampi(nearest_even((xs[32 * j + i] + dm) / d), 0, 15);
        }
        uint8_t* q = b + 16;
        for (int j = 0; j < 256; j += 64, q += 32)
            for (int l = 0; l < 32; ++l) q[l] = (uint8_t)(L[j + l] | (L[j + l + 32] << 4));
    }
}

/* One sub-block of 16 for Q6_K: L[i] = l + 32 with l in -32..31 and a scale so that x ~ scale * l,
 * x^2-weighted. (make_qx_quants(16, 32, x, L, 1, NULL).) */
static float fit_q6_subblock(const float* x, int8_t* L) {
    float mx = 0.0f, amax = 0.0f;
    for (int i = 0; i < 16; ++i) {
        const float ax = fabsf(x[i]);
        if (ax > amax) {
            amax = ax;
            mx = x[i];
        }
    }
    if (amax < 1e-15f) {
        memset(L, 0, 16);
        return 0.0f;
    }
    float iscale = -32.0f / mx;
    float sumlx = 0.0f, suml2 = 0.0f;
    for (int i = 0; i < 16; ++i) {
        const int l = clampi(nearest_even(iscale * x[i]), -32, 31);
        L[i] = (int8_t)(l + 32);
        const float w = x[i] * x[i];
        sumlx += w * x[i] * (float)l;
        suml2 += w * (float)l * (float)l;
    }
    float scale = suml2 != 0.0f ? sumlx / suml2 : 0.0f;
    float best = scale * sumlx;
    for (int step = -9; step <= 9; ++step) {
        if (step == 0) continue;
        iscale = -(32.0f + 0.1f * (float)step) / mx;
        sumlx = suml2 = 0.0f;
        for (int i = 0; i < 16; ++i) {
            const int l = clampi(nearest_even(iscale * x[i]), -32, 31);
            const float w = x[i] * x[i];
            sumlx += w * x[i] * (float)l;
            suml2 += w * (float)l * (float)l;
        }
        if (suml2 > 0.0f && sumlx * sumlx > best * suml2) {
            for (int i = 0; i < 16; ++i) L[i] = (int8_t)(32 + clampi(nearest_even(iscale * x[i]), -32, 31));
            scale = sumlx / suml2;
            best = scale * sumlx;
        }
    }
    return scale;
}

void kco_quantize_row_q6k(const float* x, uint8_t* out, int k) {
    for (int sb = 0; sb < k / 256; ++sb) {
        const float* xs = x + (size_t)sb * 256;
        uint8_t* b = out + (size_t)sb * 210;
        int8_t L[256];
        float scales[16];
        float max_scale = 0.0f, max_abs = 0.0f;
        for (int g = 0; g < 16; ++g) {
            scales[g] = fit_q6_subblock(xs + 16 * g, L + 16 * g);
            const float a = fabsf(scales[g]);
            if (a > max_abs) {
                max_abs = a;
                max_scale = scales[g];
            }
        }
        memset(b, 0, 210);
        if (max_abs < 1e-15f) continue;  /* all-zero block, d = 0 */
        const float iscale = -128.0f / max_scale;
        const uint16_t d16 = kco_f32_to_f16_rne(1.0f / iscale);
        b[208] = (uint8_t)d16, b[209] = (uint8_t)(d16 >> 8);
        int8_t* sc = (int8_t*)(b + 192);
        for (int g = 0; g < 16; ++g) {
            const int v = nearest_even(iscale * scales[g]);
            sc[g] = (int8_t)(v < 127 ? v : 127);
        }
        for (int g = 0; g < 16; ++g) {
            const float d = kco_f16_to_f32(d16) * (float)sc[g];
            if (d == 0.0f) continue;
            for (int i = 0; i < 16; ++i) L[16 * g + i] = (int8_t)(clampi(nearest_even(xs[16 * g + i] / d), -32, 31) + 32);
        }
        uint8_t* ql = b;
        uint8_t* qh = b + 128;
        for (int j = 0; j < 256; j += 128, ql += 64, qh += 32)
            for (int l = 0; l < 32; ++l) {
                const int q1 = L[j + l], q2 = L[j + l + 32], q3 = L[j + l + 64], q4 = L[j + l + 96];
                ql[l] = (uint8_t)((q1 & 0xF) | ((q3 & 0xF) << 4));
                ql[l + 32] = (uint8_t)((q2 & 0xF) | ((q4 & 0xF) << 4));
                qh[l] = (uint8_t)((q1 >> 4) | ((q2 >> 4) << 2) | ((q3 >> 4) << 4) | ((q4 >> 4) << 6));
            }
    }
}

/* rows x k floats -> rows of blocks, rows over OpenMP threads */
void kco_quantize_q4k_mt(const float* x, uint8_t* out, int rows, int k, int nthreads) {
#pragma omp parallel for num_threads(nthreads) schedule(static)
    for (int r = 0; r < rows; ++r) kco_quantize_row_q4k(x + (size_t)r * k, out + (size_t)r * (k / 256) * 144, k);
}
void kco_quantize_q6k_mt(const float* x, uint8_t* out, int rows, int k, int nthreads) {
#pragma omp parallel for num_threads(nthreads) schedule(static)
    for (int r = 0; r < rows; ++r) kco_quantize_row_q6k(x + (size_t)r * k, out + (size_t)r * (k / 256) * 210, k);
}

/* ---- CPU baseline (rows over OpenMP threads; per-row arithmetic as above) ---------------- */

int kco_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

void kco_matvec_q4k_q8_mt(const uint8_t* w, const int32_t* xq, const float* xd, float* y, int rows, int k,
                          int nthreads) {
    const int nsb = k / 256;
#pragma omp parallel for num_threads(nthreads) schedule(static)
    for (int r = 0; r < rows; ++r) y[r] = row_q4k_q8(w + (size_t)r * nsb * 144, xq, xd, nsb);
}
void kco_matvec_q6k_q8_mt(const uint8_t* w, const int32_t* xq, const float* xd, float* y, int rows, int k,
                          int nthreads) {
    const int nsb = k / 256;
#pragma omp parallel for num_threads(nthreads) schedule(static)
    for (int r = 0; r < rows; ++r) y[r] = row_q6k_q8(w + (size_t)r * nsb * 210, xq, xd, nsb);
}
void kco_matmul_q4k_q8k_mt(const uint8_t* w, const int32_t* q, float* y, int rows, int k, int ncols, int nthreads) {
    const int nsb = k / 256;
#pragma omp parallel for num_threads(nthreads) schedule(static) collapse(2)
    for (int c = 0; c < ncols; ++c)
        for (int r = 0; r < rows; ++r)
            y[(size_t)c * rows + r] = row_q4k_q8k(w + (size_t)r * nsb * 144, q + (size_t)c * nsb * 85, nsb);
}

/* llm/llm_reference.cpp:756-764: one pair of products per step, added to the running sum in order
 * (no fused multiply-add: the file is compiled with -ffp-contract=off). */
void kco_matmul_f16(const uint16_t* w, const float* x, float* y, int rows, int k, int ncols) {
    for (int c = 0; c < ncols; ++c)
        for (int r = 0; r < rows; ++r) {
            const uint16_t* wr = w + (size_t)r * k;
            const float* xc = x + (size_t)c * k;
            float a = 0.0f;
            for (int j = 0; j < k; j += 2) {
                const float p0 = kco_f16_to_f32(wr[j]) * xc[j];
                const float p1 = kco_f16_to_f32(wr[j + 1]) * xc[j + 1];
                a += p0 + p1;
            }
            y[(size_t)c * rows + r] = a;
        }
}
