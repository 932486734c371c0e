/*
 * kc_oracle_simd.c -- vectorised, multithreaded forms of the oracle's K-quant products and of its
 * flash attention (TEST INFRASTRUCTURE and the bench's CPU baseline only; never the product).
 *
 * Bit-identical to the scalar restatement in kc_oracle.c (tests/test_oracle_simd.py checks it):
 * the only vectorised part is integer arithmetic -- the dot products of the 4/6-bit weights with
 * the 8-bit activations per sub-block of 32 (Q4_K) or 16 (Q6_K), which are exact in any order --
 * and every float operation is the scalar code's, in its order, per (row, column, super-block).
 * The integer dots use AVX-512 VNNI (vpdpbusd: unsigned weight bytes x signed activation bytes,
 * four products per 32-bit lane) when the CPU has it, else AVX2 (vpmaddubsw + vpmaddwd: the pair
 * sums stay below 2 * 63 * 127 < 2^15, so the saturating step never saturates), else scalar.
 * Rows (and attention's (query, head) pairs) are split over OpenMP threads.
 *
 * This is also the "simd" CPU baseline the bench times beside the GPU: the reference's own
 * native/simd CPU paths need the Booth compiler, MSVC/Windows and closed prebuilt objects
 * (CMakeLists.txt:4-13, kernels/prebuilt/) and cannot run on Linux.
 */
#include "kc_oracle.h"

#include <immintrin.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static inline uint16_t rd16s(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* ---- the dot-product level ---------------------------------------------------------------- */

/* 2: AVX-512 VNNI, 1: AVX2, 0: scalar; KCO_SIMD=0/1/2 in the environment caps it. */
static int g_level = -1;
int kco_simd_level(void) {
    if (g_level < 0) {
        int lv = 0;
        __builtin_cpu_init();
        if (__builtin_cpu_supports("avx2")) lv = 1;
        if (__builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512bw") &&
            __builtin_cpu_supports("avx512vnni"))
            lv = 2;
        const char* cap = getenv("KCO_SIMD");
        if (cap && cap[0] >= '0' && cap[0] <= '2' && cap[0] - '0' < lv) lv = cap[0] - '0';
        g_level = lv;
    }
    return g_level;
}

/* s[j] = sum over the 32 values of sub-block j (j < 8) of w[i] * x[i]: w unsigned (< 64), x signed */
static void dots32_scalar(const uint8_t* w, const int8_t* x, int32_t* s) {
    for (int j = 0; j < 8; ++j) {
        int32_t a = 0;
        for (int i = 0; i < 32; ++i) a += (int32_t)w[32 * j + i] * x[32 * j + i];
        s[j] = a;
    }
}
/* s[g] = the same over the 16 values of group g (g < 16) */
static void dots16_scalar(const uint8_t* w, const int8_t* x, int32_t* s) {
    for (int g = 0; g < 16; ++g) {
        int32_t a = 0;
        for (int i = 0; i < 16; ++i) a += (int32_t)w[16 * g + i] * x[16 * g + i];
        s[g] = a;
    }
}

__attribute__((target("avx2"))) static inline __m256i dp8_avx2(__m256i w, __m256i x) {
    /* 8 lanes, each the sum of 4 consecutive products */
    return _mm256_madd_epi16(_mm256_maddubs_epi16(w, x), _mm256_set1_epi16(1));
}
/* the 8 lane sums of eight 8-lane vectors, as one vector (lane j = sum of v[j]) */
__attribute__((target("avx2"))) static inline __m256i hsum8x8(__m256i v0, __m256i v1, __m256i v2, __m256i v3,
                                                              __m256i v4, __m256i v5, __m256i v6, __m256i v7) {
    const __m256i a = _mm256_hadd_epi32(v0, v1), b = _mm256_hadd_epi32(v2, v3);
    const __m256i c = _mm256_hadd_epi32(v4, v5), d = _mm256_hadd_epi32(v6, v7);
    const __m256i ab = _mm256_hadd_epi32(a, b), cd = _mm256_hadd_epi32(c, d);
    /* ab = [s0 s1 s2 s3 | s0' s1' s2' s3'] (low / high 128-bit halves), likewise cd for s4..s7 */
    const __m256i lo = _mm256_permute2x128_si256(ab, cd, 0x20), hi = _mm256_permute2x128_si256(ab, cd, 0x31);
    return _mm256_add_epi32(lo, hi);
}
__attribute__((target("avx2"))) static void dots32_avx2(const uint8_t* w, const int8_t* x, int32_t* s) {
    __m256i v[8];
    for (int j = 0; j < 8; ++j)
        v[j] = dp8_avx2(_mm256_loadu_si256((const __m256i*)(w + 32 * j)), _mm256_loadu_si256((const __m256i*)(x + 32 * j)));
    _mm256_storeu_si256((__m256i*)s, hsum8x8(v[0], v[1], v[2], v[3], v[4], v[5], v[6], v[7]));
}
__attribute__((target("avx2"))) static void dots16_avx2(const uint8_t* w, const int8_t* x, int32_t* s) {
    /* group g = 4 lanes of one 128-bit half: pairwise horizontal adds of the 8 products vectors */
    __m256i v[8];
    for (int j = 0; j < 8; ++j)
        v[j] = dp8_avx2(_mm256_loadu_si256((const __m256i*)(w + 32 * j)), _mm256_loadu_si256((const __m256i*)(x + 32 * j)));
    for (int h = 0; h < 2; ++h) {
        const __m256i a = _mm256_hadd_epi32(v[4 * h + 0], v[4 * h + 1]);
        const __m256i b = _mm256_hadd_epi32(v[4 * h + 2], v[4 * h + 3]);
        const __m256i ab = _mm256_hadd_epi32(a, b);
        /* ab lane order: [g0 g2 g4 g6 | g1 g3 g5 g7] of this half's 8 groups (v[4h+i] holds groups
           8h + 2i and 8h + 2i + 1 in its low / high 128 bits) */
        int32_t t[8];
        _mm256_storeu_si256((__m256i*)t, ab);
        for (int i = 0; i < 4; ++i) {
            s[8 * h + 2 * i] = t[i];
            s[8 * h + 2 * i + 1] = t[4 + i];
        }
    }
}

__attribute__((target("avx512f,avx512bw,avx512vnni,avx2"))) static void dots32_vnni(const uint8_t* w, const int8_t* x,
                                                                                      int32_t* s) {
    __m256i v[8];
    for (int j = 0; j < 4; ++j) {
        const __m512i r = _mm512_dpbusd_epi32(_mm512_setzero_si512(), _mm512_loadu_si512(w + 64 * j),
                                              _mm512_loadu_si512(x + 64 * j));
        v[2 * j] = _mm512_castsi512_si256(r);
        v[2 * j + 1] = _mm512_extracti64x4_epi64(r, 1);
    }
    _mm256_storeu_si256((__m256i*)s, hsum8x8(v[0], v[1], v[2], v[3], v[4], v[5], v[6], v[7]));
}
__attribute__((target("avx512f,avx512bw,avx512vnni,avx2"))) static void dots16_vnni(const uint8_t* w, const int8_t* x,
                                                                                      int32_t* s) {
    for (int j = 0; j < 4; ++j) {
        __m512i r = _mm512_dpbusd_epi32(_mm512_setzero_si512(), _mm512_loadu_si512(w + 64 * j),
                                        _mm512_loadu_si512(x + 64 * j));
        /* each 128-bit lane is one group of 16: sum its 4 dwords */
        r = _mm512_add_epi32(r, _mm512_shuffle_epi32(r, _MM_PERM_CDAB));
        r = _mm512_add_epi32(r, _mm512_shuffle_epi32(r, _MM_PERM_BADC));
        int32_t t[16];
        _mm512_storeu_si512(t, r);
        for (int i = 0; i < 4; ++i) s[4 * j + i] = t[4 * i];
    }
}

/* Caps the level (tests run every path in one process): returns the level now in use. */
int kco_simd_cap(int cap) {
    g_level = -1;
    const int lv = kco_simd_level();
    g_level = cap < lv ? (cap < 0 ? 0 : cap) : lv;
    return g_level;
}

typedef void (*dots_fn)(const uint8_t*, const int8_t*, int32_t*);
static dots_fn dots32(void) { return kco_simd_level() == 2 ? dots32_vnni : kco_simd_level() == 1 ? dots32_avx2 : dots32_scalar; }
static dots_fn dots16(void) { return kco_simd_level() == 2 ? dots16_vnni : kco_simd_level() == 1 ? dots16_avx2 : dots16_scalar; }

/* ---- weight blocks as 256 unsigned bytes in activation order ---------------------------------- */

typedef struct {
    uint8_t q[256];
    float d, dmin;
    int32_t sc[16]; /* Q4_K: 8 six-bit scales then 8 mins; Q6_K: 16 signed scales */
} wblock;

static void unpack_q4k(const uint8_t* b, wblock* o) {
    o->d = kco_f16_to_f32(rd16s(b));
    o->dmin = kco_f16_to_f32(rd16s(b + 2));
    const uint8_t* s = b + 4;
    for (int j = 0; j < 8; ++j) {
        if (j < 4) {
            o->sc[j] = s[j] & 63;
            o->sc[8 + j] = s[j + 4] & 63;
        } else {
            o->sc[j] = (s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4);
            o->sc[8 + j] = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
        }
    }
    const uint8_t* qs = b + 16;
    for (int p = 0; p < 4; ++p)
        for (int l = 0; l < 32; ++l) {
            o->q[64 * p + l] = qs[32 * p + l] & 0xF;
            o->q[64 * p + 32 + l] = qs[32 * p + l] >> 4;
        }
}

static void unpack_q6k(const uint8_t* b, wblock* o) {
    o->d = kco_f16_to_f32(rd16s(b + 208));
    o->dmin = 0.0f;
    for (int g = 0; g < 16; ++g) o->sc[g] = (int8_t)b[192 + g];
    for (int n = 0; n < 2; ++n) {
        const uint8_t* ql = b + 64 * n;
        const uint8_t* qh = b + 128 + 32 * n;
        uint8_t* q = o->q + 128 * n;
        for (int l = 0; l < 32; ++l) {
            q[l] = (uint8_t)((ql[l] & 0xF) | ((qh[l] & 3) << 4));
            q[32 + l] = (uint8_t)((ql[32 + l] & 0xF) | (((qh[l] >> 2) & 3) << 4));
            q[64 + l] = (uint8_t)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4));
            q[96 + l] = (uint8_t)((ql[32 + l] >> 4) | (((qh[l] >> 6) & 3) << 4));
        }
    }
}

/* The same bytes as unpack_q4k / unpack_q6k, 32 at a time (AVX2: the level-1 and level-2 paths). */
__attribute__((target("avx2"))) static void unpack_q4k_avx2(const uint8_t* b, wblock* o) {
    o->d = kco_f16_to_f32(rd16s(b));
    o->dmin = kco_f16_to_f32(rd16s(b + 2));
    const uint8_t* s = b + 4;
    for (int j = 0; j < 8; ++j) {
        if (j < 4) {
            o->sc[j] = s[j] & 63;
            o->sc[8 + j] = s[j + 4] & 63;
        } else {
            o->sc[j] = (s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4);
            o->sc[8 + j] = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
        }
    }
    const __m256i m4 = _mm256_set1_epi8(0x0F);
    for (int p = 0; p < 4; ++p) {
        const __m256i v = _mm256_loadu_si256((const __m256i*)(b + 16 + 32 * p));
        _mm256_storeu_si256((__m256i*)(o->q + 64 * p), _mm256_and_si256(v, m4));
        _mm256_storeu_si256((__m256i*)(o->q + 64 * p + 32), _mm256_and_si256(_mm256_srli_epi16(v, 4), m4));
    }
}

__attribute__((target("avx2"))) static void unpack_q6k_avx2(const uint8_t* b, wblock* o) {
    o->d = kco_f16_to_f32(rd16s(b + 208));
    o->dmin = 0.0f;
    for (int g = 0; g < 16; ++g) o->sc[g] = (int8_t)b[192 + g];
    const __m256i m4 = _mm256_set1_epi8(0x0F), m2 = _mm256_set1_epi8(0x03);
    for (int n = 0; n < 2; ++n) {
        const __m256i l0 = _mm256_loadu_si256((const __m256i*)(b + 64 * n));
        const __m256i l1 = _mm256_loadu_si256((const __m256i*)(b + 64 * n + 32));
        const __m256i h = _mm256_loadu_si256((const __m256i*)(b + 128 + 32 * n));
        uint8_t* q = o->q + 128 * n;
        /* (qh >> 2t) & 3, moved up to bits 4-5: shifts on 16-bit lanes, then the byte mask */
        const __m256i h0 = _mm256_slli_epi16(_mm256_and_si256(h, m2), 4);
        const __m256i h1 = _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(h, 2), m2), 4);
        const __m256i h2 = _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(h, 4), m2), 4);
        const __m256i h3 = _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(h, 6), m2), 4);
        _mm256_storeu_si256((__m256i*)(q), _mm256_or_si256(_mm256_and_si256(l0, m4), h0));
        _mm256_storeu_si256((__m256i*)(q + 32), _mm256_or_si256(_mm256_and_si256(l1, m4), h1));
        _mm256_storeu_si256((__m256i*)(q + 64), _mm256_or_si256(_mm256_and_si256(_mm256_srli_epi16(l0, 4), m4), h2));
        _mm256_storeu_si256((__m256i*)(q + 96), _mm256_or_si256(_mm256_and_si256(_mm256_srli_epi16(l1, 4), m4), h3));
    }
}

typedef void (*unpack_fn)(const uint8_t*, wblock*);
static unpack_fn unpack4(void) { return kco_simd_level() >= 1 ? unpack_q4k_avx2 : unpack_q4k; }
static unpack_fn unpack6(void) { return kco_simd_level() >= 1 ? unpack_q6k_avx2 : unpack_q6k; }

static int threads_of(int n) {
#ifdef _OPENMP
    return n > 0 ? n : omp_get_max_threads();
#else
    (void)n;
    return 1;
#endif
}

/* ---- per-256 products (row_q4k_q8k / row_q6k_q8k of kc_oracle.c, columns of one row together) ---- */

enum { kRBMAX = 8 };

/* AVX-512 VNNI forms of one super-block of kRB rows x every column: the weight bytes times the
 * activation bytes per 32-bit lane (vpdpbusd), each lane times its sub-block's scale (vpmulld), one
 * reduction per (row, column): is and im are the same integers as the scalar code's. */
__attribute__((target("avx512f,avx512bw,avx512vnni,avx2"))) static void q4k_sb_vnni(const wblock* b, int nr,
                                                                                      const int32_t* q, size_t slot,
                                                                                      int nsb, int s, int ncols,
                                                                                      int acc_stride, float* acc) {
    __m512i scv[kRBMAX][4];
    __m256i mv[kRBMAX];
    for (int rr = 0; rr < nr; ++rr) {
        for (int j = 0; j < 4; ++j) {
            const __m256i lo = _mm256_set1_epi32(b[rr].sc[2 * j]), hi = _mm256_set1_epi32(b[rr].sc[2 * j + 1]);
            scv[rr][j] = _mm512_inserti64x4(_mm512_castsi256_si512(lo), hi, 1);
        }
        mv[rr] = _mm256_loadu_si256((const __m256i*)(b[rr].sc + 8));
    }
    for (int c = 0; c < ncols; ++c) {
        const int32_t* xq = q + (size_t)c * slot;
        const float xd = ((const float*)(xq + (size_t)nsb * 64))[s];
        const int32_t* bs = xq + (size_t)nsb * 65 + (size_t)s * 16;
        const int8_t* x = (const int8_t*)(xq + (size_t)s * 64);
        const __m512i x0 = _mm512_loadu_si512(x), x1 = _mm512_loadu_si512(x + 64);
        const __m512i x2 = _mm512_loadu_si512(x + 128), x3 = _mm512_loadu_si512(x + 192);
        /* B_j = bs[2j] + bs[2j + 1], as 8 lanes */
        const __m512i bsv = _mm512_loadu_si512(bs);
        const __m512i pair = _mm512_add_epi32(bsv, _mm512_shuffle_epi32(bsv, _MM_PERM_CDAB));  /* even lanes: B */
        const __m512i idx = _mm512_setr_epi32(0, 2, 4, 6, 8, 10, 12, 14, 0, 0, 0, 0, 0, 0, 0, 0);
        const __m256i B = _mm512_castsi512_si256(_mm512_permutexvar_epi32(idx, pair));
        for (int rr = 0; rr < nr; ++rr) {
            const uint8_t* w = b[rr].q;
            __m512i r = _mm512_mullo_epi32(_mm512_dpbusd_epi32(_mm512_setzero_si512(), _mm512_loadu_si512(w), x0), scv[rr][0]);
            r = _mm512_add_epi32(r, _mm512_mullo_epi32(_mm512_dpbusd_epi32(_mm512_setzero_si512(), _mm512_loadu_si512(w + 64), x1), scv[rr][1]));
            r = _mm512_add_epi32(r, _mm512_mullo_epi32(_mm512_dpbusd_epi32(_mm512_setzero_si512(), _mm512_loadu_si512(w + 128), x2), scv[rr][2]));
            r = _mm512_add_epi32(r, _mm512_mullo_epi32(_mm512_dpbusd_epi32(_mm512_setzero_si512(), _mm512_loadu_si512(w + 192), x3), scv[rr][3]));
            const int32_t is = _mm512_reduce_add_epi32(r);
            const __m256i mm = _mm256_mullo_epi32(B, mv[rr]);
            const __m128i m4 = _mm_add_epi32(_mm256_castsi256_si128(mm), _mm256_extracti128_si256(mm, 1));
            const __m128i m2 = _mm_add_epi32(m4, _mm_shuffle_epi32(m4, 0x4E));
            const int32_t im = _mm_cvtsi128_si32(_mm_add_epi32(m2, _mm_shuffle_epi32(m2, 0xB1)));
            acc[(size_t)rr * acc_stride + c] += (b[rr].d * xd) * (float)is - (b[rr].dmin * xd) * (float)im;
        }
    }
}

__attribute__((target("avx512f,avx512bw,avx512vnni,avx2"))) static void q6k_sb_vnni(const wblock* b, int nr,
                                                                                      const int32_t* q, size_t slot,
                                                                                      int nsb, int s, int ncols,
                                                                                      int acc_stride, float* acc) {
    __m512i scv[kRBMAX][4], sc16[kRBMAX];
    for (int rr = 0; rr < nr; ++rr) {
        for (int j = 0; j < 4; ++j)
            scv[rr][j] = _mm512_setr_epi32(b[rr].sc[4 * j], b[rr].sc[4 * j], b[rr].sc[4 * j], b[rr].sc[4 * j],
                                           b[rr].sc[4 * j + 1], b[rr].sc[4 * j + 1], b[rr].sc[4 * j + 1],
                                           b[rr].sc[4 * j + 1], b[rr].sc[4 * j + 2], b[rr].sc[4 * j + 2],
                                           b[rr].sc[4 * j + 2], b[rr].sc[4 * j + 2], b[rr].sc[4 * j + 3],
                                           b[rr].sc[4 * j + 3], b[rr].sc[4 * j + 3], b[rr].sc[4 * j + 3]);
        sc16[rr] = _mm512_loadu_si512(b[rr].sc);
    }
    for (int c = 0; c < ncols; ++c) {
        const int32_t* xq = q + (size_t)c * slot;
        const float xd = ((const float*)(xq + (size_t)nsb * 64))[s];
        const __m512i bsv = _mm512_loadu_si512(xq + (size_t)nsb * 65 + (size_t)s * 16);
        const int8_t* x = (const int8_t*)(xq + (size_t)s * 64);
        const __m512i x0 = _mm512_loadu_si512(x), x1 = _mm512_loadu_si512(x + 64);
        const __m512i x2 = _mm512_loadu_si512(x + 128), x3 = _mm512_loadu_si512(x + 192);
        for (int rr = 0; rr < nr; ++rr) {
            const uint8_t* w = b[rr].q;
            __m512i r = _mm512_mullo_epi32(_mm512_dpbusd_epi32(_mm512_setzero_si512(), _mm512_loadu_si512(w), x0), scv[rr][0]);
            r = _mm512_add_epi32(r, _mm512_mullo_epi32(_mm512_dpbusd_epi32(_mm512_setzero_si512(), _mm512_loadu_si512(w + 64), x1), scv[rr][1]));
            r = _mm512_add_epi32(r, _mm512_mullo_epi32(_mm512_dpbusd_epi32(_mm512_setzero_si512(), _mm512_loadu_si512(w + 128), x2), scv[rr][2]));
            r = _mm512_add_epi32(r, _mm512_mullo_epi32(_mm512_dpbusd_epi32(_mm512_setzero_si512(), _mm512_loadu_si512(w + 192), x3), scv[rr][3]));
            /* is = sum_g sc_g (S_g - 32 bs_g) = sum_g sc_g S_g - 32 sum_g sc_g bs_g */
            r = _mm512_sub_epi32(r, _mm512_slli_epi32(_mm512_mullo_epi32(sc16[rr], bsv), 5));
            const int32_t is = _mm512_reduce_add_epi32(r);
            acc[(size_t)rr * acc_stride + c] += (b[rr].d * xd) * (float)is;
        }
    }
}

/* Loop order: a thread takes blocks of kRB rows; per super-block it unpacks their kRB weight blocks
 * once, then streams every column's 256 activation bytes once for all kRB rows (they stay in L1).
 * Each (row, column) still adds its super-blocks in increasing order, as the scalar code does. */
enum { kRB = 8 };

void kco_matmul_q4k_q8k_simd(const uint8_t* w, const int32_t* q, float* y, int rows, int k, int ncols, int nthreads) {
    const int nsb = k / 256, nblk = (rows + kRB - 1) / kRB;
    const size_t slot = (size_t)nsb * 85;
    const dots_fn dot = dots32();
#pragma omp parallel num_threads(threads_of(nthreads))
    {
        float* acc = (float*)malloc(sizeof(float) * (size_t)ncols * kRB);
        wblock b[kRB];
#pragma omp for schedule(dynamic, 1)
        for (int rb = 0; rb < nblk; ++rb) {
            const int r0 = rb * kRB, nr = rows - r0 < kRB ? rows - r0 : kRB;
            for (size_t i = 0; i < (size_t)ncols * kRB; ++i) acc[i] = 0.0f;
            for (int s = 0; s < nsb; ++s) {
                for (int rr = 0; rr < nr; ++rr) unpack4()(w + ((size_t)(r0 + rr) * nsb + s) * 144, &b[rr]);
                if (kco_simd_level() == 2) {
                    q4k_sb_vnni(b, nr, q, slot, nsb, s, ncols, ncols, acc);
                    continue;
                }
                for (int c = 0; c < ncols; ++c) {
                    const int32_t* xq = q + (size_t)c * slot;
                    const float xd = ((const float*)(xq + (size_t)nsb * 64))[s];
                    const int32_t* bs = xq + (size_t)nsb * 65 + (size_t)s * 16;
                    const int8_t* x = (const int8_t*)(xq + (size_t)s * 64);
                    int32_t B[8];
                    for (int j = 0; j < 8; ++j) B[j] = bs[2 * j] + bs[2 * j + 1];
                    for (int rr = 0; rr < nr; ++rr) {
                        int32_t S[8];
                        dot(b[rr].q, x, S);
                        int32_t is = 0, im = 0;
                        for (int j = 0; j < 8; ++j) {
                            is += b[rr].sc[j] * S[j];
                            im += b[rr].sc[8 + j] * B[j];
                        }
                        acc[(size_t)rr * ncols + c] += (b[rr].d * xd) * (float)is - (b[rr].dmin * xd) * (float)im;
                    }
                }
            }
            for (int rr = 0; rr < nr; ++rr)
                for (int c = 0; c < ncols; ++c) y[(size_t)c * rows + r0 + rr] = acc[(size_t)rr * ncols + c];
        }
        free(acc);
    }
}

void kco_matmul_q6k_q8k_simd(const uint8_t* w, const int32_t* q, float* y, int rows, int k, int ncols, int nthreads) {
    const int nsb = k / 256, nblk = (rows + kRB - 1) / kRB;
    const size_t slot = (size_t)nsb * 85;
    const dots_fn dot = dots16();
#pragma omp parallel num_threads(threads_of(nthreads))
    {
        float* acc = (float*)malloc(sizeof(float) * (size_t)ncols * kRB);
        wblock b[kRB];
#pragma omp for schedule(dynamic, 1)
        for (int rb = 0; rb < nblk; ++rb) {
            const int r0 = rb * kRB, nr = rows - r0 < kRB ? rows - r0 : kRB;
            for (size_t i = 0; i < (size_t)ncols * kRB; ++i) acc[i] = 0.0f;
            for (int s = 0; s < nsb; ++s) {
                for (int rr = 0; rr < nr; ++rr) unpack6()(w + ((size_t)(r0 + rr) * nsb + s) * 210, &b[rr]);
                if (kco_simd_level() == 2) {
                    q6k_sb_vnni(b, nr, q, slot, nsb, s, ncols, ncols, acc);
                    continue;
                }
                for (int c = 0; c < ncols; ++c) {
                    const int32_t* xq = q + (size_t)c * slot;
                    const float xd = ((const float*)(xq + (size_t)nsb * 64))[s];
                    const int32_t* bs = xq + (size_t)nsb * 65 + (size_t)s * 16;
                    const int8_t* x = (const int8_t*)(xq + (size_t)s * 64);
                    for (int rr = 0; rr < nr; ++rr) {
                        int32_t S[16];
                        dot(b[rr].q, x, S);
                        int32_t is = 0;
                        for (int g = 0; g < 16; ++g) is += b[rr].sc[g] * (S[g] - 32 * bs[g]);
                        acc[(size_t)rr * ncols + c] += (b[rr].d * xd) * (float)is;
                    }
                }
            }
            for (int rr = 0; rr < nr; ++rr)
                for (int c = 0; c < ncols; ++c) y[(size_t)c * rows + r0 + rr] = acc[(size_t)rr * ncols + c];
        }
        free(acc);
    }
}

/* ---- per-32 matvecs (row_q4k_q8 / row_q6k_q8 of kc_oracle.c) ------------------------------------ */

void kco_matvec_q4k_q8_simd(const uint8_t* w, const int32_t* xq, const float* xd, float* y, int rows, int k,
                            int nthreads) {
    const int nsb = k / 256;
    const dots_fn dot = dots32();
    const unpack_fn unpack = unpack4();
#pragma omp parallel for num_threads(threads_of(nthreads)) schedule(static)
    for (int r = 0; r < rows; ++r) {
        float acc = 0.0f;
        for (int s = 0; s < nsb; ++s) {
            wblock b;
            unpack(w + ((size_t)r * nsb + s) * 144, &b);
            int32_t S[8];
            dot(b.q, (const int8_t*)(xq + (size_t)s * 64), S);
            float fd = 0.0f, fm = 0.0f;
            for (int j = 0; j < 4; ++j) {
                const int bb = s * 8 + j * 2;
                fd += (float)(b.sc[2 * j] * S[2 * j]) * xd[bb * 2] + (float)(b.sc[2 * j + 1] * S[2 * j + 1]) * xd[bb * 2 + 2];
                fm += (float)b.sc[8 + 2 * j] * (xd[bb * 2] * xd[bb * 2 + 1]) +
                      (float)b.sc[8 + 2 * j + 1] * (xd[bb * 2 + 2] * xd[bb * 2 + 3]);
            }
            acc += b.d * fd - b.dmin * fm;
        }
        y[r] = acc;
    }
}

void kco_matvec_q6k_q8_simd(const uint8_t* w, const int32_t* xq, const float* xd, float* y, int rows, int k,
                            int nthreads) {
    const int nsb = k / 256, nb = k / 32;
    const dots_fn dot = dots16();
    const unpack_fn unpack = unpack6();
    /* the sums of the first 16 values of every block of 32 (the activation side, once per call) */
    int32_t* sa = (int32_t*)malloc(sizeof(int32_t) * (size_t)nb);
    const int8_t* x8 = (const int8_t*)xq;
    for (int b = 0; b < nb; ++b) {
        int32_t a = 0;
        for (int i = 0; i < 16; ++i) a += x8[32 * b + i];
        sa[b] = a;
    }
#pragma omp parallel for num_threads(threads_of(nthreads)) schedule(static)
    for (int r = 0; r < rows; ++r) {
        float acc = 0.0f;
        for (int s = 0; s < nsb; ++s) {
            wblock b;
            unpack(w + ((size_t)r * nsb + s) * 210, &b);
            int32_t S[16];
            dot(b.q, (const int8_t*)(xq + (size_t)s * 64), S);
            for (int n = 0; n < 2; ++n) {
                const int bb = s * 8 + n * 4;
                int32_t is[4];
                for (int t = 0; t < 4; ++t) {
                    const int g = 2 * (4 * n + t);
                    const int32_t a = sa[bb + t], sb = (int32_t)xd[(bb + t) * 2 + 1] - a;
                    is[t] = b.sc[g] * (S[g] - 32 * a) + b.sc[g + 1] * (S[g + 1] - 32 * sb);
                }
                acc += b.d * ((float)is[0] * xd[bb * 2] + (float)is[1] * xd[bb * 2 + 2] + (float)is[2] * xd[bb * 2 + 4] +
                              (float)is[3] * xd[bb * 2 + 6]);
            }
        }
        y[r] = acc;
    }
    free(sa);
}

/* ---- flash attention over (query, head) pairs (kco_flash_attn_f16's arithmetic, per pair) ---- */

static float g_h2f[65536];
static int g_h2f_ready = 0;

static void h2f_init(void) {
#pragma omp critical(kco_h2f)
    if (!g_h2f_ready) {
        for (int i = 0; i < 65536; ++i) g_h2f[i] = kco_f16_to_f32((uint16_t)i);
        __atomic_store_n(&g_h2f_ready, 1, __ATOMIC_RELEASE);
    }
}

/* The scores of 8 consecutive positions, one per AVX2 lane (each lane the scalar dot, j in order),
 * from a per-call transposed copy of K; P.V over 8 consecutive head values per lane (t in order). Both
 * keep every float operation of the scalar code in its order: a multiply and an add, never fused. */
__attribute__((target("avx2,f16c"))) static void fa_pair_avx2(const float* qh, const float* kt, const float* vf,
                                                                const float* mrow, float* s, float* outp, int T,
                                                                int D, size_t vstride, float scale) {
    float mx = -INFINITY;
    int t = 0;
    for (; t + 8 <= T; t += 8) {
        __m256 a = _mm256_setzero_ps();
        for (int j = 0; j < D; ++j)
            a = _mm256_add_ps(a, _mm256_mul_ps(_mm256_set1_ps(qh[j]), _mm256_loadu_ps(kt + (size_t)j * T + t)));
        __m256 v = _mm256_mul_ps(a, _mm256_set1_ps(scale));
        if (mrow) v = _mm256_add_ps(v, _mm256_loadu_ps(mrow + t));
        _mm256_storeu_ps(s + t, v);
    }
    for (; t < T; ++t) {
        float a = 0.0f;
        for (int j = 0; j < D; ++j) a += qh[j] * kt[(size_t)j * T + t];
        s[t] = a * scale + (mrow ? mrow[t] : 0.0f);
    }
    for (t = 0; t < T; ++t) mx = mx > s[t] ? mx : s[t];
    float sum = 0.0f;
    for (t = 0; t < T; ++t) sum += (s[t] = exp2f((s[t] - mx) * 1.44269504f));
    int dd = 0;
    for (; dd + 8 <= D; dd += 8) {
        __m256 a = _mm256_setzero_ps();
        for (t = 0; t < T; ++t)
            a = _mm256_add_ps(a, _mm256_mul_ps(_mm256_set1_ps(s[t]), _mm256_loadu_ps(vf + (size_t)t * vstride + dd)));
        _mm256_storeu_ps(outp + dd, _mm256_div_ps(a, _mm256_set1_ps(sum)));
    }
    for (; dd < D; ++dd) {
        float a = 0.0f;
        for (t = 0; t < T; ++t) a += s[t] * vf[(size_t)t * vstride + dd];
        outp[dd] = a / sum;
    }
}

void kco_flash_attn_f16_mt(const float* q, const uint16_t* k, const uint16_t* v, const uint16_t* mask, float* out,
                           const kco_fa_dims* d, float scale, int nthreads) {
    if (!__atomic_load_n(&g_h2f_ready, __ATOMIC_ACQUIRE)) h2f_init();
    const int pairs = d->N * d->H, T = d->T, D = d->D;
    const int simd = kco_simd_level() >= 1 && T > 0;
    /* K of every KV head transposed to [head][j][t] and V to [t][head][j], as floats (exact) */
    float* kt = NULL;
    float* vf = NULL;
    float* mf = NULL;
    if (simd) {
        kt = (float*)malloc(sizeof(float) * (size_t)d->H_kv * D * T);
        vf = (float*)malloc(sizeof(float) * (size_t)T * d->H_kv * D);
        for (int h = 0; h < d->H_kv; ++h)
            for (int t = 0; t < T; ++t)
                for (int j = 0; j < D; ++j) {
                    kt[((size_t)h * D + j) * T + t] = g_h2f[k[((size_t)t * d->k_row + (size_t)h * d->k_head) * 2 + j]];
                    vf[((size_t)t * d->H_kv + h) * D + j] = g_h2f[v[((size_t)t * d->v_row + (size_t)h * d->v_head) * 2 + j]];
                }
        if (d->has_mask) {
            mf = (float*)malloc(sizeof(float) * (size_t)d->N * T);
            for (int i = 0; i < d->N; ++i)
                for (int t = 0; t < T; ++t) mf[(size_t)i * T + t] = g_h2f[mask[(size_t)i * d->m_row * 2 + t]];
        }
    }
#pragma omp parallel num_threads(threads_of(nthreads))
    {
        float* s = (float*)malloc(sizeof(float) * (size_t)(T > 0 ? T : 1));
#pragma omp for schedule(dynamic, 4)
        for (int p = 0; p < pairs; ++p) {
            const int i = p / d->H, h = p % d->H;
            const int kvh = h / d->group;
            const float* qh = q + (size_t)i * d->q_tok + (size_t)h * d->q_head;
            float* outp = out + ((size_t)i * d->H + h) * D;
            if (simd) {
                fa_pair_avx2(qh, kt + (size_t)kvh * D * T, vf + (size_t)kvh * D, mf ? mf + (size_t)i * T : NULL, s, outp,
                             T, D, (size_t)d->H_kv * D, scale);
                continue;
            }
            float mx = -INFINITY;
            for (int t = 0; t < T; ++t) {
                const uint16_t* kr = k + ((size_t)t * d->k_row + (size_t)kvh * d->k_head) * 2;
                float a = 0.0f;
                for (int j = 0; j < D; ++j) a += qh[j] * g_h2f[kr[j]];
                const float mv = d->has_mask ? g_h2f[mask[(size_t)i * d->m_row * 2 + t]] : 0.0f;
                s[t] = a * scale + mv;
                mx = mx > s[t] ? mx : s[t];
            }
            float sum = 0.0f;
            for (int t = 0; t < T; ++t) sum += (s[t] = exp2f((s[t] - mx) * 1.44269504f));
            for (int dd = 0; dd < D; ++dd) {
                float a = 0.0f;
                for (int t = 0; t < T; ++t) a += s[t] * g_h2f[v[((size_t)t * d->v_row + (size_t)kvh * d->v_head) * 2 + dd]];
                outp[dd] = a / sum;
            }
        }
        free(s);
    }
    free(kt);
    free(vf);
    free(mf);
}
