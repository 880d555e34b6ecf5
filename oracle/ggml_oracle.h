/*
 * CPU oracle for the quantized-matmul path: a plain C restatement of the
 * GGML block formats and Candle's CPU quantized matmul (k_quants).
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (inference_amd/) may
 * include, link or call this code: it is the checker the tests, the smoke
 * entry point and the CPU-baseline leg of bench.py compare against.
 *
 * All byte layouts are the GGML on-disk/in-memory layouts (little endian),
 * i.e. exactly the bytes candle's QStorage::from_data receives:
 *   Q8_0 : 34 B / 32   { f16 d; i8 qs[32]; }
 *   Q4_K : 144 B / 256 { f16 d; f16 dmin; u8 scales[12]; u8 qs[128]; }
 *   Q6_K : 210 B / 256 { u8 ql[128]; u8 qh[64]; i8 scales[16]; f16 d; }
 *   Q8_K : 292 B / 256 { f32 d; i8 qs[256]; i16 bsums[16]; }
 */
#ifndef GGML_ORACLE_H
#define GGML_ORACLE_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGUF type tags (reference: crates/llm/mlx-llm/src/gguf/dequant.rs:87-113). */
enum { ORC_F32 = 0, ORC_F16 = 1, ORC_Q8_0 = 8, ORC_Q4K = 12, ORC_Q6K = 14, ORC_Q8K = 15 };

/* Geometry: elements per block and bytes per block; 0 for an unknown tag. */
int orc_block_elems(int dtype);
int orc_block_bytes(int dtype);
/* The activation ("vec-dot") type a weight type multiplies against. */
int orc_vec_dot_type(int dtype);

/* IEEE binary16 <-> binary32 (round-to-nearest-even, like half::f16::from_f32). */
uint16_t orc_f32_to_f16(float x);
float orc_f16_to_f32(uint16_t h);

/* from_float quantizers: n must be a multiple of the block size; return 0 or -1. */
int orc_quantize(int dtype, const float *x, int64_t n, void *out);
/* dequantize: blocks -> f32 (n elements). */
int orc_dequantize(int dtype, const void *blocks, int64_t n, float *out);

/* vec_dot of one weight row (k elements) against one activation row already
 * quantized to the vec-dot type; generic (non-SIMD) accumulation order. */
float orc_vec_dot(int dtype, int64_t k, const void *w_row, const void *x_row);

/* Exact integer block dots of one weight row against one activation row.
 *  Q8_0: isum[b]   = sum qw*qx over block b               (k/32 entries)
 *  Q4_K: isum[2b]  = sum_j sc_j * sum_{l in j} q4*q8      (isum_d)
 *        isum[2b+1]= sum_j m_j * (bsum_{2j} + bsum_{2j+1}) (isum_m)
 *  Q6_K: isum[b]   = sum_j sc_j * sum_{l in j} (q6-32)*q8 (k/256 entries) */
int orc_block_dots(int dtype, int64_t k, const void *w_row, const void *x_row, int32_t *isum);

/* Candle k_quants::matmul: dst[m, n] = vec_dot(W[n], quant(lhs[m])).
 * lhs is f32 [m, k]; rhs is n rows of k/QK blocks; dst f32 [m, n].
 * nthreads <= 0 uses the OpenMP default. */
int orc_matmul(int dtype, int64_t m, int64_t k, int64_t n, const float *lhs,
               const void *rhs, float *dst, int nthreads);
/* Same, with the activations already quantized (xq: m rows of k/QK vec-dot blocks). */
int orc_matmul_prequant(int dtype, int64_t m, int64_t k, int64_t n, const void *xq,
                        const void *rhs, float *dst, int nthreads);

/* vec_dot implementations: candle's generic bodies (the default build of the
 * reference) or its x86 AVX2 + FMA bodies (ggml_oracle_avx2.c).  Both give the
 * same integer block dots; they differ only in f32 accumulation order. */
enum { ORC_IMPL_GENERIC = 0, ORC_IMPL_AVX2 = 1 };
/* 1 when this CPU runs the AVX2 + FMA bodies. */
/* Test hooks: the sub-block fits of the weight quantizers (upstream
 * quantized/utils.rs make_qkx1_quants, make_qx_quants; the static functions
 * quantize_q4k / quantize_q6k call). make_qkx1_quants returns the scale and
 * -min of an asymmetric nmax-level fit; make_qx_quants returns the scale and
 * writes L[i] = l_i + nmax of a symmetric fit. */
void orc_make_qkx1_quants(int nmax, int ntry, const float *x, int n, float *scale, float *neg_min);
float orc_make_qx_quants(int n, int nmax, const float *x, int8_t *L, int rmse_type);
/* make_qx_quants (rmse_type 1) stopped after its first refinement loop; *passes = the loop's accepted
 * passes (0..3). Test hook for that loop's exit condition. */
float orc_make_qx_quants_first(int n, int nmax, const float *x, int8_t *L, int *passes);

int orc_simd_supported(void);
float orc_vec_dot_avx2(int dtype, int64_t k, const void *w_row, const void *x_row);
/* orc_matmul_prequant / orc_matmul with a chosen implementation; -1 for an
 * unknown one or AVX2 on a CPU without it. */
int orc_matmul_prequant_impl(int dtype, int64_t m, int64_t k, int64_t n, const void *xq,
                             const void *rhs, float *dst, int nthreads, int impl);
int orc_matmul_impl(int dtype, int64_t m, int64_t k, int64_t n, const float *lhs,
                    const void *rhs, float *dst, int nthreads, int impl);

#ifdef __cplusplus
}
#endif
#endif
