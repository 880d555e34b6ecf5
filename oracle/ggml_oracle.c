/*
 * CPU oracle: a plain-C restatement of Candle's CPU quantized matmul over the
 * GGML block formats Q8_0, Q4_K and Q6_K (with the Q8_0 / Q8_K activation
 * types).  TEST INFRASTRUCTURE ONLY: the product never links this file.
 *
 * Sources followed (paths relative to the reference checkout):
 *  - block layouts: crates/media/candle-gen/vendor/candle-kernels/src/quantized.cu:329-336
 *    (block_q8_0), :389-394 (block_q4_K), :419-425 (block_q6_K), :428-433 (block_q8_K);
 *    geometry crates/llm/mlx-llm/src/gguf/dequant.rs:115-141.
 *  - dequantization: crates/llm/mlx-llm/src/gguf/dequant.rs:284-290 (Q8_0),
 *    :379-416 (get_scale_min_k4, Q4_K), :452-474 (Q6_K).
 *  - quantizers (from_float), vec_dot and matmul: candle-core's
 *    quantized/k_quants.rs + quantized/utils.rs at git rev 1e6aa85e (Cargo.toml:54,
 *    Cargo.lock:360-362).  That crate is not in the container; the restatement
 *    follows its published algorithm (BlockQ8_0/BlockQ8K/BlockQ4K/BlockQ6K
 *    ::from_float, make_qkx1_quants, make_qx_quants, nearest_int = f32::round,
 *    the generic vec_dot bodies and k_quants::matmul).
 *
 * Floating point: compile with -ffp-contract=off and without -ffast-math so
 * every f32 operation is a single IEEE-rounded op in source order, as in Rust.
 */
#include "ggml_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define QK 32
#define QK_K 256

/* ------------------------------------------------------------------ */
/* geometry                                                            */
/* ------------------------------------------------------------------ */

int orc_block_elems(int dtype) {
    switch (dtype) {
    case ORC_F32: case ORC_F16: return 1;
    case ORC_Q8_0: return QK;
    case ORC_Q4K: case ORC_Q6K: case ORC_Q8K: return QK_K;
    default: return 0;
    }
}

int orc_block_bytes(int dtype) {
    switch (dtype) {
    case ORC_F32: return 4;
    case ORC_F16: return 2;
    case ORC_Q8_0: return 34;  /* dequant.rs:130  d + 32      */
    case ORC_Q4K: return 144;  /* dequant.rs:133  d+dmin+12+128 */
    case ORC_Q6K: return 210;  /* dequant.rs:135  128+64+16+2 */
    case ORC_Q8K: return 292;  /* quantized.cu:428-433       */
    default: return 0;
    }
}

int orc_vec_dot_type(int dtype) {
    switch (dtype) {
    case ORC_Q8_0: return ORC_Q8_0;
    case ORC_Q4K: case ORC_Q6K: return ORC_Q8K;
    default: return -1;
    }
}

/* ------------------------------------------------------------------ */
/* f16                                                                 */
/* ------------------------------------------------------------------ */

uint16_t orc_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t exp = (x >> 23) & 0xffu;
    uint32_t man = x & 0x7fffffu;
    if (exp == 0xffu) {
        if (man) return (uint16_t)(sign | 0x7e00u | (man >> 13));
        return (uint16_t)(sign | 0x7c00u);
    }
    int e = (int)exp - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        man |= 0x800000u;
        int shift = 14 - e;
        uint32_t hm = man >> shift;
        uint32_t rem = man & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (hm & 1u))) hm++;
        return (uint16_t)(sign | hm);
    }
    uint32_t hm = man >> 13;
    uint32_t rem = man & 0x1fffu;
    uint32_t h = sign | ((uint32_t)e << 10) | hm;
    if (rem > 0x1000u || (rem == 0x1000u && (hm & 1u))) h++;
    return (uint16_t)h;
}

float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t exp = ((uint32_t)h >> 10) & 0x1fu;
    uint32_t man = (uint32_t)h & 0x3ffu;
    uint32_t x;
    if (exp == 0) {
        if (man == 0) {
            x = sign;
        } else {
            int e = -1;
            do { man <<= 1; e++; } while (!(man & 0x400u));
            man &= 0x3ffu;
            x = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
        }
    } else if (exp == 0x1fu) {
        x = sign | 0x7f800000u | (man << 13);
    } else {
        x = sign | ((exp + 127 - 15) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &x, 4);
    return f;
}

static inline uint16_t rd_u16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static inline void wr_u16(uint8_t *p, uint16_t v) { p[0] = (uint8_t)v; p[1] = (uint8_t)(v >> 8); }
static inline float rd_f16(const uint8_t *p) { return orc_f16_to_f32(rd_u16(p)); }
static inline float rd_f32(const uint8_t *p) { float f; memcpy(&f, p, 4); return f; }
static inline void wr_f32(uint8_t *p, float f) { memcpy(p, &f, 4); }
static inline int16_t rd_i16(const uint8_t *p) { return (int16_t)rd_u16(p); }

/* Rust `f as i8` / `f as i32`: truncate toward zero, saturate, NaN -> 0. */
static inline int8_t sat_i8(float v) {
    if (v != v) return 0;
    if (v >= 127.0f) return 127;
    if (v <= -128.0f) return -128;
    return (int8_t)v;
}
static inline int32_t sat_i32(float v) {
    if (v != v) return 0;
    if (v >= 2147483647.0f) return 2147483647;
    if (v <= -2147483648.0f) return (int32_t)(-2147483647 - 1);
    return (int32_t)v;
}
/* candle quantized/utils.rs nearest_int: v.round() as i32 (ties away from zero). */
static inline int32_t nearest_int(float v) { return sat_i32(roundf(v)); }
static inline int32_t clampi(int32_t v, int32_t lo, int32_t hi) { return v < lo ? lo : (v > hi ? hi : v); }
/* f32::max / f32::min: NaN-ignoring. */
static inline float fmax_rs(float a, float b) { return fmaxf(a, b); }

/* ------------------------------------------------------------------ */
/* Q8_0 (weights and their activations)                                */
/* ------------------------------------------------------------------ */

/* BlockQ8_0::from_float [upstream k_quants.rs]: d = amax/127, q = round(x/d). */
static void quantize_q8_0(const float *x, int64_t n, uint8_t *out) {
    for (int64_t b = 0; b < n / QK; b++) {
        const float *xs = x + b * QK;
        uint8_t *blk = out + b * 34;
        float amax = 0.0f;
        for (int i = 0; i < QK; i++) amax = fmax_rs(amax, fabsf(xs[i]));
        float d = amax / 127.0f;
        float id = d != 0.0f ? 1.0f / d : 0.0f;
        wr_u16(blk, orc_f32_to_f16(d));
        for (int i = 0; i < QK; i++) blk[2 + i] = (uint8_t)sat_i8(roundf(xs[i] * id));
    }
}

/* dequant.rs:284-290 */
static void dequant_q8_0(const uint8_t *blk, float *y) {
    float d = rd_f16(blk);
    for (int j = 0; j < 32; j++) y[j] = (float)(int8_t)blk[2 + j] * d;
}

/* ------------------------------------------------------------------ */
/* Q8_K (activations of k-quant weights)                               */
/* ------------------------------------------------------------------ */

/* BlockQ8K::from_float [upstream k_quants.rs]: signed max-|x| element (first
 * wins), iscale = -128/max, q = min(127, round(iscale*x)), bsums per 16,
 * d = 1/iscale; an all-zero block gives d = 0. */
static void quantize_q8k(const float *x, int64_t n, uint8_t *out) {
    for (int64_t b = 0; b < n / QK_K; b++) {
        const float *xs = x + b * QK_K;
        uint8_t *blk = out + b * 292;
        int8_t *qs = (int8_t *)(blk + 4);
        uint8_t *bs = blk + 4 + QK_K;
        float max = 0.0f, amax = 0.0f;
        for (int j = 0; j < QK_K; j++) {
            float ax = fabsf(xs[j]);
            if (amax < ax) { amax = ax; max = xs[j]; }
        }
        if (amax == 0.0f) {
            memset(blk, 0, 292);
            continue;
        }
        float iscale = -128.0f / max;
        for (int j = 0; j < QK_K; j++) {
            float v = roundf(iscale * xs[j]);
            qs[j] = sat_i8(fminf(v, 127.0f));
        }
        for (int j = 0; j < QK_K / 16; j++) {
            int32_t s = 0;
            for (int i = 0; i < 16; i++) s += qs[16 * j + i];
            wr_u16(bs + 2 * j, (uint16_t)(int16_t)s);
        }
        wr_f32(blk, 1.0f / iscale);
    }
}

static void dequant_q8k(const uint8_t *blk, float *y) {
    float d = rd_f32(blk);
    for (int j = 0; j < QK_K; j++) y[j] = d * (float)(int8_t)blk[4 + j];
}

/* ------------------------------------------------------------------ */
/* Q4_K                                                                */
/* ------------------------------------------------------------------ */

/* dequant.rs:379-389 (= quantized.cu:925-932) */
static void get_scale_min_k4(int j, const uint8_t *q, uint8_t *d, uint8_t *m) {
    if (j < 4) {
        *d = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *d = (uint8_t)((q[j + 4] & 0x0F) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

/* make_qkx1_quants(nmax, ntry, x) [upstream quantized/utils.rs]: iterative
 * asymmetric fit of one sub-block; returns (scale, -min). */
static void make_qkx1_quants(int nmax, int ntry, const float *x, int n, float *out_scale,
                             float *out_min) {
    uint8_t l[QK_K];
    memset(l, 0, sizeof(l));
    float mn = x[0], mx = x[0];
    for (int i = 1; i < n; i++) {
        if (x[i] < mn) mn = x[i];
        if (x[i] > mx) mx = x[i];
    }
    if (mx == mn) {
        *out_scale = 0.0f;
        *out_min = 0.0f;
        return;
    }
    float min = fminf(mn, 0.0f);
    float iscale = (float)nmax / (mx - min);
    float scale = 1.0f / iscale;
    for (int it = 0; it < ntry; it++) {
        float sumlx = 0.0f;
        int32_t suml2 = 0;
        int did_change = 0;
        for (int i = 0; i < n; i++) {
            int32_t li = clampi(nearest_int(iscale * (x[i] - min)), 0, nmax);
            uint8_t cl = (uint8_t)li;
            if (cl != l[i]) {
                l[i] = cl;
                did_change = 1;
            }
            sumlx += (x[i] - min) * (float)li;
            suml2 += li * li;
        }
        scale = sumlx / (float)suml2;
        float sum = 0.0f;
        for (int i = 0; i < n; i++) sum += x[i] - scale * (float)l[i];
        min = sum / (float)n;
        if (min > 0.0f) min = 0.0f;
        iscale = 1.0f / scale;
        if (!did_change) break;
    }
    *out_scale = scale;
    *out_min = -min;
}

/* BlockQ4K::from_float [upstream k_quants.rs]. */
static void quantize_q4k(const float *xall, int64_t n, uint8_t *out) {
    for (int64_t b = 0; b < n / QK_K; b++) {
        const float *x = xall + b * QK_K;
        uint8_t *blk = out + b * 144;
        uint8_t *scales = blk + 4;
        uint8_t *qs = blk + 16;
        float mins[8], scl[8];
        memset(blk, 0, 144);
        for (int j = 0; j < 8; j++) make_qkx1_quants(15, 5, x + 32 * j, 32, &scl[j], &mins[j]);
        float max_scale = 0.0f, max_min = 0.0f;
        for (int j = 0; j < 8; j++) max_scale = fmax_rs(scl[j], max_scale);
        for (int j = 0; j < 8; j++) max_min = fmax_rs(mins[j], max_min);
        float inv_scale = max_scale > 0.0f ? 63.0f / max_scale : 0.0f;
        float inv_min = max_min > 0.0f ? 63.0f / max_min : 0.0f;
        for (int j = 0; j < 8; j++) {
            int32_t lsi = nearest_int(inv_scale * scl[j]);
            int32_t lmi = nearest_int(inv_min * mins[j]);
            uint8_t ls = (uint8_t)(lsi < 63 ? lsi : 63);
            uint8_t lm = (uint8_t)(lmi < 63 ? lmi : 63);
            if (j < 4) {
                scales[j] = ls;
                scales[j + 4] = lm;
            } else {
                scales[j + 4] = (uint8_t)((ls & 0xF) | ((lm & 0xF) << 4));
                scales[j - 4] |= (uint8_t)((ls >> 4) << 6);
                scales[j] |= (uint8_t)((lm >> 4) << 6);
            }
        }
        uint16_t dh = orc_f32_to_f16(max_scale / 63.0f);
        uint16_t mh = orc_f32_to_f16(max_min / 63.0f);
        wr_u16(blk, dh);
        wr_u16(blk + 2, mh);
        uint8_t L[QK_K];
        memset(L, 0, sizeof(L));
        for (int j = 0; j < 8; j++) {
            uint8_t sc, m;
            get_scale_min_k4(j, scales, &sc, &m);
            float d = orc_f16_to_f32(dh) * (float)sc;
            if (d != 0.0f) {
                float dm = orc_f16_to_f32(mh) * (float)m;
                for (int ii = 0; ii < 32; ii++) {
                    int32_t lv = nearest_int((x[32 * j + ii] + dm) / d);
                    L[32 * j + ii] = (uint8_t)clampi(lv, 0, 15);
                }
            }
        }
        for (int j = 0; j < QK_K; j += 64)
            for (int l = 0; l < 32; l++)
                qs[j / 2 + l] = (uint8_t)(L[j + l] | (L[j + l + 32] << 4));
    }
}

/* dequant.rs:391-416 */
static void dequant_q4k(const uint8_t *blk, float *y) {
    float d = rd_f16(blk), dmin = rd_f16(blk + 2);
    const uint8_t *scales = blk + 4, *qs = blk + 16;
    int is = 0, yi = 0;
    for (int j = 0; j < QK_K; j += 64) {
        const uint8_t *q = qs + j / 2;
        uint8_t sc, m;
        get_scale_min_k4(is, scales, &sc, &m);
        float d1 = d * (float)sc, m1 = dmin * (float)m;
        get_scale_min_k4(is + 1, scales, &sc, &m);
        float d2 = d * (float)sc, m2 = dmin * (float)m;
        for (int l = 0; l < 32; l++) y[yi++] = d1 * (float)(q[l] & 0xF) - m1;
        for (int l = 0; l < 32; l++) y[yi++] = d2 * (float)(q[l] >> 4) - m2;
        is += 2;
    }
}

/* ------------------------------------------------------------------ */
/* Q6_K                                                                */
/* ------------------------------------------------------------------ */

/* make_qx_quants(n, nmax, x, L, rmse_type) [upstream quantized/utils.rs]:
 * symmetric fit with least-squares refinement; L[i] holds l + nmax. Only the two forms this path
 * reaches are restated: rmse_type 0 (the bare rounding) and 1 (the x^2-weighted refinement that
 * BlockQ6K::from_float uses); any other rmse_type returns NaN. */
static float make_qx_quants_stages(int n, int nmax, const float *x, int8_t *L, int rmse_type,
                                   int *first_passes) {
    float max = 0.0f, amax = 0.0f;
    for (int i = 0; i < n; i++) {
        float ax = fabsf(x[i]);
        if (ax > amax) { amax = ax; max = x[i]; }
    }
    if (amax == 0.0f) {
        for (int i = 0; i < n; i++) L[i] = 0;
        return 0.0f;
    }
    float iscale = -(float)nmax / max;
    if (rmse_type == 0) {
        for (int i = 0; i < n; i++) {
            int32_t l = nearest_int(iscale * x[i]);
            L[i] = (int8_t)(nmax + clampi(l, -nmax, nmax - 1));
        }
        return 1.0f / iscale;
    }
    if (rmse_type != 1) return NAN;
#define QX_W(v) ((v) * (v))
    float sumlx = 0.0f, suml2 = 0.0f;
    for (int i = 0; i < n; i++) {
        int32_t l = clampi(nearest_int(iscale * x[i]), -nmax, nmax - 1);
        L[i] = (int8_t)(l + nmax);
        float w = QX_W(x[i]);
        float lf = (float)l;
        sumlx += w * x[i] * lf;
        suml2 += w * lf * lf;
    }
    float scale = sumlx / suml2;
    float best = scale * sumlx;
    for (int itry = 0; itry < 3; itry++) {
        float is = 1.0f / scale;
        float slx = 0.0f, sl2 = 0.0f;
        int changed = 0;
        for (int i = 0; i < n; i++) {
            int32_t l = clampi(nearest_int(is * x[i]), -nmax, nmax - 1);
            if (l + nmax != L[i]) changed = 1;
            float w = QX_W(x[i]);
            float lf = (float)l;
            slx += w * x[i] * lf;
            sl2 += w * lf * lf;
        }
        if (!changed || sl2 == 0.0f || slx * slx <= best * sl2) break;
        for (int i = 0; i < n; i++) {
            int32_t l = nearest_int(is * x[i]);
            L[i] = (int8_t)(nmax + clampi(l, -nmax, nmax - 1));
        }
        sumlx = slx;
        suml2 = sl2;
        scale = sumlx / suml2;
        best = scale * sumlx;
        if (first_passes) ++*first_passes;
    }
    /* test hook: stop after the first loop (the count of its accepted passes in *first_passes) */
    if (first_passes) return scale;
    for (int itry = 0; itry < 5; itry++) {
        int n_changed = 0;
        for (int i = 0; i < n; i++) {
            float w = QX_W(x[i]);
            int32_t l = L[i] - nmax;
            float slx = sumlx - w * x[i] * (float)l;
            if (slx > 0.0f) {
                float sl2 = suml2 - w * (float)l * (float)l;
                int32_t new_l = clampi(nearest_int(x[i] * sl2 / slx), -nmax, nmax - 1);
                if (new_l != l) {
                    slx += w * x[i] * (float)new_l;
                    sl2 += w * (float)new_l * (float)new_l;
                    if (sl2 > 0.0f && slx * slx * suml2 > sumlx * sumlx * sl2) {
                        L[i] = (int8_t)(nmax + new_l);
                        sumlx = slx;
                        suml2 = sl2;
                        scale = sumlx / suml2;
                        best = scale * sumlx;
                        n_changed++;
                    }
                }
            }
        }
        if (!n_changed) break;
    }
#undef QX_W
    return scale;
}

static float make_qx_quants(int n, int nmax, const float *x, int8_t *L, int rmse_type) {
    return make_qx_quants_stages(n, nmax, x, L, rmse_type, NULL);
}

void orc_make_qkx1_quants(int nmax, int ntry, const float *x, int n, float *scale, float *neg_min) {
    make_qkx1_quants(nmax, ntry, x, n, scale, neg_min);
}

float orc_make_qx_quants(int n, int nmax, const float *x, int8_t *L, int rmse_type) {
    return make_qx_quants(n, nmax, x, L, rmse_type);
}

float orc_make_qx_quants_first(int n, int nmax, const float *x, int8_t *L, int *passes) {
    *passes = 0;
    return make_qx_quants_stages(n, nmax, x, L, 1, passes);
}

/* BlockQ6K::from_float [upstream k_quants.rs]. */
static void quantize_q6k(const float *xall, int64_t n, uint8_t *out) {
    int8_t L[QK_K];
    float scales[QK_K / 16];
    memset(L, 0, sizeof(L));
    for (int64_t b = 0; b < n / QK_K; b++) {
        const float *x = xall + b * QK_K;
        uint8_t *blk = out + b * 210;
        uint8_t *ql = blk, *qh = blk + 128;
        int8_t *ysc = (int8_t *)(blk + 192);
        memset(blk, 0, 210);
        float max_scale = 0.0f, max_abs_scale = 0.0f;
        for (int ib = 0; ib < QK_K / 16; ib++) {
            float scale = make_qx_quants(16, 32, x + 16 * ib, L + 16 * ib, 1);
            scales[ib] = scale;
            float as = fabsf(scale);
            if (as > max_abs_scale) {
                max_abs_scale = as;
                max_scale = scale;
            }
        }
        float iscale = -128.0f / max_scale;
        uint16_t dh = orc_f32_to_f16(1.0f / iscale);
        wr_u16(blk + 208, dh);
        for (int j = 0; j < QK_K / 16; j++) {
            int32_t v = nearest_int(iscale * scales[j]);
            ysc[j] = (int8_t)(v < 127 ? v : 127);
        }
        for (int j = 0; j < QK_K / 16; j++) {
            float d = orc_f16_to_f32(dh) * (float)ysc[j];
            if (d == 0.0f) continue;
            for (int ii = 0; ii < 16; ii++) {
                int32_t ll = clampi(nearest_int(x[16 * j + ii] / d), -32, 31);
                L[16 * j + ii] = (int8_t)(ll + 32);
            }
        }
        for (int j = 0; j < QK_K; j += 128) {
            uint8_t *qlp = ql + j / 2, *qhp = qh + j / 4;
            for (int l = 0; l < 32; l++) {
                uint8_t q1 = L[j + l] & 0xF, q2 = L[j + l + 32] & 0xF;
                uint8_t q3 = L[j + l + 64] & 0xF, q4 = L[j + l + 96] & 0xF;
                qlp[l] = (uint8_t)(q1 | (q3 << 4));
                qlp[l + 32] = (uint8_t)(q2 | (q4 << 4));
                qhp[l] = (uint8_t)((L[j + l] >> 4) | ((L[j + l + 32] >> 4) << 2) |
                                   ((L[j + l + 64] >> 4) << 4) | ((L[j + l + 96] >> 4) << 6));
            }
        }
    }
}

/* Unpack the 256 signed q6-32 values of a Q6_K block (dequant.rs:452-474). */
static void unpack_q6k(const uint8_t *blk, int8_t *q) {
    const uint8_t *ql = blk, *qh = blk + 128;
    for (int n = 0; n < QK_K; n += 128) {
        const uint8_t *qlp = ql + n / 2, *qhp = qh + n / 4;
        for (int l = 0; l < 32; l++) {
            q[n + l] = (int8_t)(((qlp[l] & 0x0F) | ((qhp[l] & 3) << 4)) - 32);
            q[n + l + 32] = (int8_t)(((qlp[l + 32] & 0x0F) | (((qhp[l] >> 2) & 3) << 4)) - 32);
            q[n + l + 64] = (int8_t)(((qlp[l] >> 4) | (((qhp[l] >> 4) & 3) << 4)) - 32);
            q[n + l + 96] = (int8_t)(((qlp[l + 32] >> 4) | (((qhp[l] >> 6) & 3) << 4)) - 32);
        }
    }
}

/* dequant.rs:452-474 */
static void dequant_q6k(const uint8_t *blk, float *y) {
    const int8_t *scales = (const int8_t *)(blk + 192);
    float d = rd_f16(blk + 208);
    int8_t q[QK_K];
    unpack_q6k(blk, q);
    for (int n = 0; n < QK_K; n += 128) {
        int sco = 8 * (n / 128);
        for (int l = 0; l < 32; l++) {
            int is = l / 16;
            y[n + l] = d * (float)scales[sco + is] * (float)q[n + l];
            y[n + l + 32] = d * (float)scales[sco + is + 2] * (float)q[n + l + 32];
            y[n + l + 64] = d * (float)scales[sco + is + 4] * (float)q[n + l + 64];
            y[n + l + 96] = d * (float)scales[sco + is + 6] * (float)q[n + l + 96];
        }
    }
}

/* ------------------------------------------------------------------ */
/* public quantize / dequantize                                        */
/* ------------------------------------------------------------------ */

int orc_quantize(int dtype, const float *x, int64_t n, void *out) {
    int be = orc_block_elems(dtype);
    if (be <= 1 || n < 0 || n % be) return -1;
    switch (dtype) {
    case ORC_Q8_0: quantize_q8_0(x, n, (uint8_t *)out); return 0;
    case ORC_Q8K: quantize_q8k(x, n, (uint8_t *)out); return 0;
    case ORC_Q4K: quantize_q4k(x, n, (uint8_t *)out); return 0;
    case ORC_Q6K: quantize_q6k(x, n, (uint8_t *)out); return 0;
    default: return -1;
    }
}

int orc_dequantize(int dtype, const void *blocks, int64_t n, float *out) {
    int be = orc_block_elems(dtype), bb = orc_block_bytes(dtype);
    if (be <= 1 || n < 0 || n % be) return -1;
    const uint8_t *p = (const uint8_t *)blocks;
    for (int64_t b = 0; b < n / be; b++) {
        const uint8_t *blk = p + b * bb;
        float *y = out + b * be;
        switch (dtype) {
        case ORC_Q8_0: dequant_q8_0(blk, y); break;
        case ORC_Q8K: dequant_q8k(blk, y); break;
        case ORC_Q4K: dequant_q4k(blk, y); break;
        case ORC_Q6K: dequant_q6k(blk, y); break;
        default: return -1;
        }
    }
    return 0;
}

/* ------------------------------------------------------------------ */
/* exact integer block dots                                            */
/* ------------------------------------------------------------------ */

static int32_t bdot_q8_0(const uint8_t *w, const uint8_t *x) {
    int32_t s = 0;
    for (int i = 0; i < QK; i++) s += (int32_t)(int8_t)w[2 + i] * (int32_t)(int8_t)x[2 + i];
    return s;
}

/* Q4_K x Q8_K: isum_d = sum_j sc_j * sum_{l in j} q4*q8 ; isum_m = sum_j m_j * (bsum_2j + bsum_2j+1). */
static void bdot_q4k(const uint8_t *w, const uint8_t *x, int32_t *isd, int32_t *ism) {
    const uint8_t *scales = w + 4, *qs = w + 16;
    const int8_t *q8 = (const int8_t *)(x + 4);
    const uint8_t *bs = x + 4 + QK_K;
    int32_t sd = 0, sm = 0;
    for (int j = 0; j < 8; j++) {
        uint8_t sc, m;
        get_scale_min_k4(j, scales, &sc, &m);
        const uint8_t *q = qs + 32 * (j / 2);
        int shift = (j & 1) ? 4 : 0;
        int32_t s = 0;
        for (int l = 0; l < 32; l++) s += (int32_t)((q[l] >> shift) & 0xF) * (int32_t)q8[32 * j + l];
        sd += (int32_t)sc * s;
        sm += (int32_t)m * ((int32_t)rd_i16(bs + 4 * j) + (int32_t)rd_i16(bs + 4 * j + 2));
    }
    *isd = sd;
    *ism = sm;
}

/* Q6_K x Q8_K: isum = sum_j sc_j * sum_{l in j} (q6-32)*q8 (16 sub-blocks of 16). */
static int32_t bdot_q6k(const uint8_t *w, const uint8_t *x) {
    int8_t q[QK_K];
    unpack_q6k(w, q);
    const int8_t *sc = (const int8_t *)(w + 192);
    const int8_t *q8 = (const int8_t *)(x + 4);
    int32_t s = 0;
    for (int j = 0; j < 16; j++) {
        int32_t t = 0;
        for (int l = 0; l < 16; l++) t += (int32_t)q[16 * j + l] * (int32_t)q8[16 * j + l];
        s += (int32_t)sc[j] * t;
    }
    return s;
}

int orc_block_dots(int dtype, int64_t k, const void *w_row, const void *x_row, int32_t *isum) {
    const uint8_t *w = (const uint8_t *)w_row, *x = (const uint8_t *)x_row;
    switch (dtype) {
    case ORC_Q8_0:
        if (k % QK) return -1;
        for (int64_t b = 0; b < k / QK; b++) isum[b] = bdot_q8_0(w + 34 * b, x + 34 * b);
        return 0;
    case ORC_Q4K:
        if (k % QK_K) return -1;
        for (int64_t b = 0; b < k / QK_K; b++) bdot_q4k(w + 144 * b, x + 292 * b, &isum[2 * b], &isum[2 * b + 1]);
        return 0;
    case ORC_Q6K:
        if (k % QK_K) return -1;
        for (int64_t b = 0; b < k / QK_K; b++) isum[b] = bdot_q6k(w + 210 * b, x + 292 * b);
        return 0;
    default:
        return -1;
    }
}

/* ------------------------------------------------------------------ */
/* vec_dot (generic bodies, f32 accumulation in candle's order)        */
/* ------------------------------------------------------------------ */

/* BlockQ8_0::vec_dot generic [upstream]: sumf += isum * d_w * d_x per block. */
static float vec_dot_q8_0(int64_t k, const uint8_t *w, const uint8_t *x) {
    float sumf = 0.0f;
    for (int64_t b = 0; b < k / QK; b++) {
        int32_t s = bdot_q8_0(w + 34 * b, x + 34 * b);
        sumf += (float)s * rd_f16(w + 34 * b) * rd_f16(x + 34 * b);
    }
    return sumf;
}

/* BlockQ4K::vec_dot generic [upstream]: eight lane accumulators aux32[l]
 * (elements l mod 8 of every group of 8), sums[l] += d*aux32[l], and the
 * mins term subtracted from a separate sumf. */
static float vec_dot_q4k(int64_t k, const uint8_t *wall, const uint8_t *xall) {
    float sums[8] = {0};
    float sumf = 0.0f;
    for (int64_t b = 0; b < k / QK_K; b++) {
        const uint8_t *w = wall + 144 * b, *x = xall + 292 * b;
        const uint8_t *scales = w + 4, *qs = w + 16;
        const int8_t *q8 = (const int8_t *)(x + 4);
        const uint8_t *bs = x + 4 + QK_K;
        int8_t a[QK_K];
        for (int c = 0; c < 4; c++)
            for (int l = 0; l < 32; l++) {
                a[64 * c + l] = (int8_t)(qs[32 * c + l] & 0xF);
                a[64 * c + 32 + l] = (int8_t)(qs[32 * c + l] >> 4);
            }
        int32_t aux32[8] = {0};
        int32_t sumi = 0;
        for (int j = 0; j < QK_K / 16; j++) {
            uint8_t sc, m;
            get_scale_min_k4(j / 2, scales, &sc, &m);
            sumi += (int32_t)rd_i16(bs + 2 * j) * (int32_t)m;
        }
        for (int j = 0; j < 8; j++) {
            uint8_t sc, m;
            get_scale_min_k4(j, scales, &sc, &m);
            for (int g = 0; g < 4; g++)
                for (int l = 0; l < 8; l++) {
                    int idx = 32 * j + 8 * g + l;
                    int16_t p = (int16_t)((int16_t)q8[idx] * (int16_t)a[idx]);
                    aux32[l] += (int32_t)sc * (int32_t)p;
                }
        }
        float xd = rd_f32(x);
        float d = rd_f16(w) * xd;
        for (int l = 0; l < 8; l++) sums[l] += d * (float)aux32[l];
        float dmin = rd_f16(w + 2) * xd;
        sumf -= dmin * (float)sumi;
    }
    float t = 0.0f;
    for (int l = 0; l < 8; l++) t += sums[l];
    return sumf + t;
}

/* BlockQ6K::vec_dot generic [upstream]. */
static float vec_dot_q6k(int64_t k, const uint8_t *wall, const uint8_t *xall) {
    float sums[8] = {0};
    for (int64_t b = 0; b < k / QK_K; b++) {
        const uint8_t *w = wall + 210 * b, *x = xall + 292 * b;
        const int8_t *sc = (const int8_t *)(w + 192);
        const int8_t *q8 = (const int8_t *)(x + 4);
        int8_t a[QK_K];
        unpack_q6k(w, a);
        float aux32[8] = {0};
        for (int j = 0; j < 16; j++) {
            float scale = (float)sc[j];
            for (int g = 0; g < 2; g++)
                for (int l = 0; l < 8; l++) {
                    int idx = 16 * j + 8 * g + l;
                    int16_t p = (int16_t)((int16_t)q8[idx] * (int16_t)a[idx]);
                    aux32[l] += scale * (float)p;
                }
        }
        float d = rd_f16(w + 208) * rd_f32(x);
        for (int l = 0; l < 8; l++) sums[l] += aux32[l] * d;
    }
    float t = 0.0f;
    for (int l = 0; l < 8; l++) t += sums[l];
    return t;
}

float orc_vec_dot(int dtype, int64_t k, const void *w_row, const void *x_row) {
    const uint8_t *w = (const uint8_t *)w_row, *x = (const uint8_t *)x_row;
    switch (dtype) {
    case ORC_Q8_0: return vec_dot_q8_0(k, w, x);
    case ORC_Q4K: return vec_dot_q4k(k, w, x);
    case ORC_Q6K: return vec_dot_q6k(k, w, x);
    default: return NAN;
    }
}

/* ------------------------------------------------------------------ */
/* matmul (k_quants::matmul)                                           */
/* ------------------------------------------------------------------ */

int orc_matmul_prequant(int dtype, int64_t m, int64_t k, int64_t n, const void *xq,
                        const void *rhs, float *dst, int nthreads) {
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
        for (int64_t c = 0; c < n; c++) dr[c] = orc_vec_dot(dtype, k, w + c * wrow, xr);
    }
    return 0;
}

int orc_matmul(int dtype, int64_t m, int64_t k, int64_t n, const float *lhs, const void *rhs,
               float *dst, int nthreads) {
    return orc_matmul_impl(dtype, m, k, n, lhs, rhs, dst, nthreads, ORC_IMPL_GENERIC);
}

int orc_matmul_impl(int dtype, int64_t m, int64_t k, int64_t n, const float *lhs, const void *rhs,
                    float *dst, int nthreads, int impl) {
    int vt = orc_vec_dot_type(dtype);
    if (vt < 0) return -1;
    int vbe = orc_block_elems(vt), vbb = orc_block_bytes(vt);
    if (k % vbe) return -1;
    int64_t xrow = (k / vbe) * vbb;
    uint8_t *xq = (uint8_t *)calloc((size_t)(m * xrow), 1);
    if (!xq) return -1;
    for (int64_t r = 0; r < m; r++) orc_quantize(vt, lhs + r * k, k, xq + r * xrow);
    int rc = orc_matmul_prequant_impl(dtype, m, k, n, xq, rhs, dst, nthreads, impl);
    free(xq);
    return rc;
}
