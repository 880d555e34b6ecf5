/*
 * CPU oracle, x86 SIMD variant: a restatement of the AVX2 + FMA vec_dot bodies
 * that candle-core compiles in when its build enables the `avx` target
 * feature (quantized/avx.rs at git rev 1e6aa85e, Cargo.toml:54; not in the
 * container).  TEST INFRASTRUCTURE ONLY: the product never links this file.
 *
 * Two uses:
 *  - the CPU baseline bench.py reports beside the generic build (a candle
 *    build with `-C target-feature=+avx2,+fma` or `target-cpu=native` runs
 *    these bodies; the workspace's default build sets no rustflags,
 *    .cargo/config.toml:1-36, and runs the generic ones);
 *  - a second, equally valid f32 accumulation order of the same integer
 *    block dots.  Its integer terms equal the generic ones exactly (the
 *    maddubs pair sums stay below 2^15 for every format here: Q4_K 2*15*128,
 *    Q6_K 2*63*128, Q8_0 2*127*128 on absolute values); only the f32 order
 *    differs (8 FMA lanes per block, then candle's hsum_float_8).
 *
 * Per super-block, following the published algorithm:
 *  Q4_K x Q8_K: d = dx*f16(d_w), dmin = -dx*f16(dmin_w); the mins term is
 *    (pairwise-added bsums) . (six-bit mins) in four i32 lanes, FMA'd by dmin
 *    into a 4-lane f32 accumulator; each 64-element chunk contributes
 *    madd(scale, maddubs(low nibbles, q8)) and the same for the high
 *    nibbles into eight i32 lanes; acc8 = fma(d, f32(sumi), acc8).
 *  Q6_K x Q8_K: per 128-half, four 32-element columns of q6 = low 4 bits |
 *    2 high bits << 4, maddubs(q6, q8) - maddubs(32, q8), madd with the
 *    sub-block scales (two per column), summed into eight i32 lanes;
 *    acc8 = fma(dx*f16(d_w), f32(sumi), acc8).
 *  Q8_0 x Q8_0: per block, 8 lanes of pairwise dot sums (sign trick:
 *    maddubs(|w|, sign(x, w)), madd with ones) converted to f32,
 *    acc8 = fma(f16(d_w)*f16(d_x), dots, acc8).
 */
#include "ggml_oracle.h"

#include <immintrin.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define QK 32
#define QK_K 256

#define AVX2_FN __attribute__((target("avx2,fma")))

static inline float rd_f16s(const uint8_t *p) { return orc_f16_to_f32((uint16_t)(p[0] | (p[1] << 8))); }
static inline float rd_f32s(const uint8_t *p) { float f; memcpy(&f, p, 4); return f; }

/* candle's hsum_float_8: high half + low half, then movehl, then movehdup. */
AVX2_FN static inline float hsum8(__m256 x) {
    __m128 r = _mm_add_ps(_mm256_extractf128_ps(x, 1), _mm256_castps256_ps128(x));
    r = _mm_add_ps(r, _mm_movehl_ps(r, r));
    r = _mm_add_ss(r, _mm_movehdup_ps(r));
    return _mm_cvtss_f32(r);
}

/* 6-bit scales and mins of a Q4_K block as 8 + 8 bytes (same values as
 * get_scale_min_k4 for j = 0..7). */
static inline void q4k_scales_mins(const uint8_t *s, uint8_t sc[8], uint8_t mn[8]) {
    for (int j = 0; j < 4; j++) {
        sc[j] = s[j] & 63;
        mn[j] = s[j + 4] & 63;
        sc[j + 4] = (uint8_t)((s[j + 8] & 0x0F) | ((s[j] >> 6) << 4));
        mn[j + 4] = (uint8_t)((s[j + 8] >> 4) | ((s[j + 4] >> 6) << 4));
    }
}

AVX2_FN static float vec_dot_q4k_avx2(int64_t k, const uint8_t *wall, const uint8_t *xall) {
    const __m256i m4 = _mm256_set1_epi8(0x0F);
    __m256 acc = _mm256_setzero_ps();
    __m128 acc_m = _mm_setzero_ps();
    for (int64_t b = 0; b < k / QK_K; b++) {
        const uint8_t *w = wall + 144 * b, *x = xall + 292 * b;
        const float dx = rd_f32s(x);
        const float d = dx * rd_f16s(w);
        const float dmin = -dx * rd_f16s(w + 2);
        uint8_t sc[8], mn[8];
        q4k_scales_mins(w + 4, sc, mn);
        /* mins term: bsums pairwise-added (16 -> 8 i16), madd with the mins */
        const __m256i bs = _mm256_loadu_si256((const __m256i *)(x + 4 + QK_K));
        const __m128i q8s = _mm_hadd_epi16(_mm256_castsi256_si128(bs), _mm256_extracti128_si256(bs, 1));
        const __m128i mins = _mm_cvtepu8_epi16(_mm_loadl_epi64((const __m128i *)mn));
        const __m128i prod = _mm_madd_epi16(mins, q8s);
        acc_m = _mm_fmadd_ps(_mm_set1_ps(dmin), _mm_cvtepi32_ps(prod), acc_m);
        const uint8_t *q4 = w + 16;
        const int8_t *q8 = (const int8_t *)(x + 4);
        __m256i sumi = _mm256_setzero_si256();
        for (int c = 0; c < QK_K / 64; c++) {
            const __m256i scale_l = _mm256_set1_epi16(sc[2 * c]);
            const __m256i scale_h = _mm256_set1_epi16(sc[2 * c + 1]);
            const __m256i bits = _mm256_loadu_si256((const __m256i *)(q4 + 32 * c));
            const __m256i q4l = _mm256_and_si256(bits, m4);
            const __m256i q4h = _mm256_and_si256(_mm256_srli_epi16(bits, 4), m4);
            const __m256i q8l = _mm256_loadu_si256((const __m256i *)(q8 + 64 * c));
            const __m256i q8h = _mm256_loadu_si256((const __m256i *)(q8 + 64 * c + 32));
            const __m256i pl = _mm256_madd_epi16(scale_l, _mm256_maddubs_epi16(q4l, q8l));
            const __m256i ph = _mm256_madd_epi16(scale_h, _mm256_maddubs_epi16(q4h, q8h));
            sumi = _mm256_add_epi32(sumi, pl);
            sumi = _mm256_add_epi32(sumi, ph);
        }
        acc = _mm256_fmadd_ps(_mm256_set1_ps(d), _mm256_cvtepi32_ps(sumi), acc);
    }
    acc_m = _mm_add_ps(acc_m, _mm_movehl_ps(acc_m, acc_m));
    acc_m = _mm_add_ss(acc_m, _mm_movehdup_ps(acc_m));
    return hsum8(acc) + _mm_cvtss_f32(acc_m);
}

AVX2_FN static float vec_dot_q6k_avx2(int64_t k, const uint8_t *wall, const uint8_t *xall) {
    const __m256i m4 = _mm256_set1_epi8(0x0F);
    const __m256i m2 = _mm256_set1_epi8(0x03);
    const __m256i m32 = _mm256_set1_epi8(32);
    __m256 acc = _mm256_setzero_ps();
    for (int64_t b = 0; b < k / QK_K; b++) {
        const uint8_t *w = wall + 210 * b, *x = xall + 292 * b;
        const float d = rd_f32s(x) * rd_f16s(w + 208);
        const int8_t *scales = (const int8_t *)(w + 192);
        const int8_t *q8 = (const int8_t *)(x + 4);
        __m256i sumi = _mm256_setzero_si256();
        for (int h = 0; h < 2; h++) {
            const uint8_t *ql = w + 64 * h, *qh = w + 128 + 32 * h;
            const __m256i l0 = _mm256_loadu_si256((const __m256i *)ql);
            const __m256i l1 = _mm256_loadu_si256((const __m256i *)(ql + 32));
            const __m256i hb = _mm256_loadu_si256((const __m256i *)qh);
            __m256i q6[4];
            q6[0] = _mm256_or_si256(_mm256_and_si256(l0, m4), _mm256_slli_epi16(_mm256_and_si256(hb, m2), 4));
            q6[1] = _mm256_or_si256(_mm256_and_si256(l1, m4),
                                    _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(hb, 2), m2), 4));
            q6[2] = _mm256_or_si256(_mm256_and_si256(_mm256_srli_epi16(l0, 4), m4),
                                    _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(hb, 4), m2), 4));
            q6[3] = _mm256_or_si256(_mm256_and_si256(_mm256_srli_epi16(l1, 4), m4),
                                    _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(hb, 6), m2), 4));
            for (int i = 0; i < 4; i++) {
                const __m256i q8v = _mm256_loadu_si256((const __m256i *)(q8 + 128 * h + 32 * i));
                const __m256i p16 = _mm256_sub_epi16(_mm256_maddubs_epi16(q6[i], q8v), _mm256_maddubs_epi16(m32, q8v));
                const int s0 = scales[8 * h + 2 * i], s1 = scales[8 * h + 2 * i + 1];
                /* i16 lanes 0..7 pair elements 0..15 (scale s0), lanes 8..15 elements 16..31 (s1) */
                const __m256i sc = _mm256_setr_epi16(s0, s0, s0, s0, s0, s0, s0, s0, s1, s1, s1, s1, s1, s1, s1, s1);
                sumi = _mm256_add_epi32(sumi, _mm256_madd_epi16(sc, p16));
            }
        }
        acc = _mm256_fmadd_ps(_mm256_set1_ps(d), _mm256_cvtepi32_ps(sumi), acc);
    }
    return hsum8(acc);
}

AVX2_FN static float vec_dot_q8_0_avx2(int64_t k, const uint8_t *w, const uint8_t *x) {
    const __m256i ones = _mm256_set1_epi16(1);
    __m256 acc = _mm256_setzero_ps();
    for (int64_t b = 0; b < k / QK; b++) {
        const uint8_t *wb = w + 34 * b, *xb = x + 34 * b;
        const __m256 d = _mm256_set1_ps(rd_f16s(wb) * rd_f16s(xb));
        const __m256i bw = _mm256_loadu_si256((const __m256i *)(wb + 2));
        const __m256i bx = _mm256_loadu_si256((const __m256i *)(xb + 2));
        const __m256i aw = _mm256_sign_epi8(bw, bw);
        const __m256i sx = _mm256_sign_epi8(bx, bw);
        const __m256i dots = _mm256_madd_epi16(_mm256_maddubs_epi16(aw, sx), ones);
        acc = _mm256_fmadd_ps(d, _mm256_cvtepi32_ps(dots), acc);
    }
    return hsum8(acc);
}

int orc_simd_supported(void) {
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma");
}

float orc_vec_dot_avx2(int dtype, int64_t k, const void *w_row, const void *x_row) {
    const uint8_t *w = (const uint8_t *)w_row, *x = (const uint8_t *)x_row;
    switch (dtype) {
    case ORC_Q8_0: return vec_dot_q8_0_avx2(k, w, x);
    case ORC_Q4K: return vec_dot_q4k_avx2(k, w, x);
    case ORC_Q6K: return vec_dot_q6k_avx2(k, w, x);
    default: return 0.0f / 0.0f;
    }
}

int orc_matmul_prequant_impl(int dtype, int64_t m, int64_t k, int64_t n, const void *xq, const void *rhs,
                             float *dst, int nthreads, int impl) {
    if (impl == ORC_IMPL_GENERIC) return orc_matmul_prequant(dtype, m, k, n, xq, rhs, dst, nthreads);
    if (impl != ORC_IMPL_AVX2 || !orc_simd_supported()) return -1;
    int vt = orc_vec_dot_type(dtype);
    if (vt < 0) return -1;
    int be = orc_block_elems(dtype), bb = orc_block_bytes(dtype);
    int vbe = orc_block_elems(vt), vbb = orc_block_bytes(vt);
    if (k % be || k % vbe) return -1;
    const uint8_t *w = (const uint8_t *)rhs, *x = (const uint8_t *)xq;
    int64_t wrow = (k / be) * bb, xrow = (k / vbe) * vbb;
#ifdef _OPENMP
    if (nthreads <= 0) nthreads = omp_get_max_threads();
#else
    (void)nthreads;
#endif
    for (int64_t r = 0; r < m; r++) {
        const uint8_t *xr = x + r * xrow;
        float *dr = dst + r * n;
#ifdef _OPENMP
#pragma omp parallel for schedule(static) num_threads(nthreads)
#endif
        for (int64_t c = 0; c < n; c++) dr[c] = orc_vec_dot_avx2(dtype, k, w + c * wrow, xr);
    }
    return 0;
}
