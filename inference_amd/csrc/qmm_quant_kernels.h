// Quantizers, layout conversion and dequantization kernels (gfx950).
//
// Activation quantizers follow the vec-dot types of Candle's CPU quantized
// matmul (candle-core quantized/k_quants.rs @1e6aa85e, Cargo.toml:54):
//   BlockQ8K::from_float  -- activations of Q4_K / Q6_K weights
//   BlockQ8_0::from_float -- activations (and weights) of Q8_0
// Weight quantizers restate BlockQ4K::from_float / BlockQ6K::from_float with
// their helpers make_qkx1_quants / make_qx_quants (quantized/utils.rs) step by
// step, because their output bytes depend on the exact f32 operation order.
// Every f32 operation in those functions is a single IEEE-rounded operation
// (contraction off, correctly rounded division), so the bytes match the CPU's.
// Byte layouts: crates/media/candle-gen/vendor/candle-kernels/src/quantized.cu:329-433.
#pragma once

#include "qmm_common.h"

namespace qmm {

// ---------------------------------------------------------------------------
// Q8_K activation quantizer: one wave per 256-element block.
//   max   = the element of largest |x| (the first one on ties)
//   iscale = -128 / max, q = min(127, round(iscale * x)) (ties away from zero)
//   bsums[j] = sum of q[16j .. 16j+16), d = 1 / iscale; an all-zero block is all zeros.
// ---------------------------------------------------------------------------
// Lane-local result of quantizing one 256-element block (lane owns elements
// 4*lane .. 4*lane+3).
// silu(g) * u as LlamaMlp::forward computes it (crates/llm/candle-llm/src/models/llama.rs:1386-1391):
// g / (1 + exp(-g)) * u, each operation rounded on its own.
__device__ __forceinline__ float silu_mul(float g, float u) {
#pragma clang fp contract(off)
  return g / (1.0f + expf(-g)) * u;
}

struct Q8KLane {
  uint32_t packed;  // its four int8 quants
  int sum16;        // sum of the 16-element group it belongs to
  float d;
};

__device__ __forceinline__ Q8KLane q8k_lane_vals(float e0, float e1, float e2, float e3, int lane) {
#pragma clang fp contract(off)
  const float amax = wave_max(fmaxf(fmaxf(fabsf(e0), fabsf(e1)), fmaxf(fabsf(e2), fabsf(e3))));
  Q8KLane r;
  if (amax == 0.0f) {
    r.packed = 0u;
    r.sum16 = 0;
    r.d = 0.0f;
    return r;
  }
  const int mine = fabsf(e0) == amax ? 0 : fabsf(e1) == amax ? 1 : fabsf(e2) == amax ? 2 : fabsf(e3) == amax ? 3 : 4;
  const int idx = wave_min(mine < 4 ? 4 * lane + mine : 256);
  const float cand = (idx & 3) == 0 ? e0 : (idx & 3) == 1 ? e1 : (idx & 3) == 2 ? e2 : e3;
  const float mx = readlane_f(cand, idx >> 2);
  const float iscale = -128.0f / mx;
  const float e[4] = {e0, e1, e2, e3};
  uint32_t packed = 0;
  int sum = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    float v = roundf(iscale * e[j]);
    v = fminf(v, 127.0f);
    int q = (int)v;
    q = q < -128 ? -128 : q;
    sum += q;
    packed |= (uint32_t)(q & 0xff) << (8 * j);
  }
  r.packed = packed;
  r.sum16 = quad_sum(sum);
  r.d = 1.0f / iscale;
  return r;
}

__device__ __forceinline__ Q8KLane q8k_lane(const float* __restrict__ xs, int lane) {
  return q8k_lane_vals(xs[4 * lane], xs[4 * lane + 1], xs[4 * lane + 2], xs[4 * lane + 3], lane);
}

// Standalone form: one wave writes one GGML Q8_K block.
__device__ __forceinline__ void q8k_block(const float* __restrict__ xs, uint8_t* __restrict__ blk, int lane) {
  const Q8KLane q = q8k_lane(xs, lane);
  reinterpret_cast<uint32_t*>(blk + 4)[lane] = q.packed;
  const int next = __shfl_down(q.sum16, 4);
  if ((lane & 7) == 0)
    reinterpret_cast<uint32_t*>(blk + 4 + 256)[lane >> 3] = ((uint32_t)q.sum16 & 0xffffu) | ((uint32_t)next << 16);
  if (lane == 0) *reinterpret_cast<float*>(blk) = q.d;
}

// ---------------------------------------------------------------------------
// Q8_0 quantizer (activations and weights): 8 lanes per 32-element block.
//   d = amax / 127, q = round(x * (1/d)) (0 when d == 0), d stored as f16.
// Writes GGML 34-byte blocks.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void q80_block(const float* __restrict__ xs, uint8_t* __restrict__ blk,
                                          int l, bool valid) {
#pragma clang fp contract(off)
  float e[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) e[j] = valid ? xs[4 * l + j] : 0.0f;
  float amax = 0.0f;
#pragma unroll
  for (int j = 0; j < 4; ++j) amax = fmaxf(amax, fabsf(e[j]));
  amax = fmaxf(amax, dpp_f<0xb1>(amax));   // max over the 8 lanes of the block
  amax = fmaxf(amax, dpp_f<0x4e>(amax));
  amax = fmaxf(amax, dpp_f<0x141>(amax));
  const float d = amax / 127.0f;
  const float id = d != 0.0f ? 1.0f / d : 0.0f;
  if (!valid) return;
  uint32_t q4 = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    float r = roundf(e[j] * id);
    r = fminf(fmaxf(r, -128.0f), 127.0f);
    q4 |= (uint32_t)((int)r & 0xff) << (8 * j);
  }
  uint16_t* p = reinterpret_cast<uint16_t*>(blk);
  if (l == 0) p[0] = f2h(d);
  p[1 + 2 * l] = (uint16_t)(q4 & 0xffff);
  p[2 + 2 * l] = (uint16_t)(q4 >> 16);
}

// ---------------------------------------------------------------------------
// Q4_K weight quantizer (one thread per 256-element super-block).
// ---------------------------------------------------------------------------
__device__ __forceinline__ int round_i(float v) {
  // f32::round (ties away from zero) then a saturating cast to i32.
  const float r = roundf(v);
  if (!(r == r)) return 0;
  if (r >= 2147483647.0f) return 2147483647;
  if (r <= -2147483648.0f) return (int)0x80000000;
  return (int)r;
}

__device__ __forceinline__ int clamp_i(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }

// Asymmetric fit of n values to [0, nmax] codes (make_qkx1_quants); returns
// the scale and writes the (positive) offset `-min`.
__device__ float fit_qkx1(int nmax, int ntry, const float* x, int n, float* neg_min) {
#pragma clang fp contract(off)
  uint8_t codes[32];
  for (int i = 0; i < n; ++i) codes[i] = 0;
  float lo = x[0], hi = x[0];
  for (int i = 1; i < n; ++i) {
    if (x[i] < lo) lo = x[i];
    if (x[i] > hi) hi = x[i];
  }
  if (hi == lo) {
    *neg_min = 0.0f;
    return 0.0f;
  }
  float mn = fminf(lo, 0.0f);
  float iscale = (float)nmax / (hi - mn);
  float scale = 1.0f / iscale;
  for (int it = 0; it < ntry; ++it) {
    float sumlx = 0.0f;
    int suml2 = 0;
    bool changed = false;
    for (int i = 0; i < n; ++i) {
      const int c = clamp_i(round_i(iscale * (x[i] - mn)), 0, nmax);
      if ((uint8_t)c != codes[i]) {
        codes[i] = (uint8_t)c;
        changed = true;
      }
      sumlx += (x[i] - mn) * (float)c;
      suml2 += c * c;
    }
    scale = sumlx / (float)suml2;
    float acc = 0.0f;
    for (int i = 0; i < n; ++i) acc += x[i] - scale * (float)codes[i];
    mn = acc / (float)n;
    if (mn > 0.0f) mn = 0.0f;
    iscale = 1.0f / scale;
    if (!changed) break;
  }
  *neg_min = -mn;
  return scale;
}

__device__ __forceinline__ void q4k_scale_min(int j, const uint8_t* s, int* sc, int* m) {
  if (j < 4) {
    *sc = s[j] & 63;
    *m = s[j + 4] & 63;
  } else {
    *sc = (s[j + 4] & 0x0f) | ((s[j - 4] >> 6) << 4);
    *m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
  }
}

__device__ void q4k_quantize_block(const float* __restrict__ x, uint8_t* __restrict__ out) {
#pragma clang fp contract(off)
  float sub_scale[8], sub_min[8];
  for (int j = 0; j < 8; ++j) sub_scale[j] = fit_qkx1(15, 5, x + 32 * j, 32, &sub_min[j]);
  float max_scale = 0.0f, max_min = 0.0f;
  for (int j = 0; j < 8; ++j) max_scale = fmaxf(sub_scale[j], max_scale);
  for (int j = 0; j < 8; ++j) max_min = fmaxf(sub_min[j], max_min);
  const float inv_scale = max_scale > 0.0f ? 63.0f / max_scale : 0.0f;
  const float inv_min = max_min > 0.0f ? 63.0f / max_min : 0.0f;
  uint8_t sc[12];
  for (int i = 0; i < 12; ++i) sc[i] = 0;
  for (int j = 0; j < 8; ++j) {
    int ls = round_i(inv_scale * sub_scale[j]);
    int lm = round_i(inv_min * sub_min[j]);
    ls = ls < 63 ? ls : 63;
    lm = lm < 63 ? lm : 63;
    if (j < 4) {
      sc[j] = (uint8_t)ls;
      sc[j + 4] = (uint8_t)lm;
    } else {
      sc[j + 4] = (uint8_t)((ls & 0x0f) | ((lm & 0x0f) << 4));
      sc[j - 4] |= (uint8_t)((ls >> 4) << 6);
      sc[j] |= (uint8_t)((lm >> 4) << 6);
    }
  }
  const uint16_t dh = f2h(max_scale / 63.0f);
  const uint16_t mh = f2h(max_min / 63.0f);
  const float df = h2f(dh), mf = h2f(mh);
  uint8_t codes[256];
  for (int i = 0; i < 256; ++i) codes[i] = 0;
  for (int j = 0; j < 8; ++j) {
    int s, m;
    q4k_scale_min(j, sc, &s, &m);
    const float d = df * (float)s;
    if (d == 0.0f) continue;
    const float dm = mf * (float)m;
    for (int i = 0; i < 32; ++i) codes[32 * j + i] = (uint8_t)clamp_i(round_i((x[32 * j + i] + dm) / d), 0, 15);
  }
  out[0] = (uint8_t)dh;
  out[1] = (uint8_t)(dh >> 8);
  out[2] = (uint8_t)mh;
  out[3] = (uint8_t)(mh >> 8);
  for (int i = 0; i < 12; ++i) out[4 + i] = sc[i];
  for (int c = 0; c < 4; ++c)
    for (int i = 0; i < 32; ++i)
      out[16 + 32 * c + i] = (uint8_t)(codes[64 * c + i] | (codes[64 * c + 32 + i] << 4));
}

// ---------------------------------------------------------------------------
// Q6_K weight quantizer (one thread per super-block).
// ---------------------------------------------------------------------------

// Symmetric fit of 16 values to [-nmax, nmax-1] with the squared-value
// weighting (make_qx_quants with rmse_type 1); codes are stored biased by nmax.
__device__ float fit_qx16(int nmax, const float* x, int8_t* codes) {
#pragma clang fp contract(off)
  const int n = 16;
  float amax = 0.0f, vmax = 0.0f;
  for (int i = 0; i < n; ++i) {
    const float a = fabsf(x[i]);
    if (a > amax) {
      amax = a;
      vmax = x[i];
    }
  }
  if (amax == 0.0f) {
    for (int i = 0; i < n; ++i) codes[i] = 0;
    return 0.0f;
  }
  float iscale = -(float)nmax / vmax;
  float sumlx = 0.0f, suml2 = 0.0f;
  for (int i = 0; i < n; ++i) {
    const int l = clamp_i(round_i(iscale * x[i]), -nmax, nmax - 1);
    codes[i] = (int8_t)(l + nmax);
    const float w = x[i] * x[i];
    const float lf = (float)l;
    sumlx += w * x[i] * lf;
    suml2 += w * lf * lf;
  }
  float scale = sumlx / suml2;
  float best = scale * sumlx;
  for (int t = 0; t < 3; ++t) {
    const float is = 1.0f / scale;
    float slx = 0.0f, sl2 = 0.0f;
    bool changed = false;
    for (int i = 0; i < n; ++i) {
      const int l = clamp_i(round_i(is * x[i]), -nmax, nmax - 1);
      if (l + nmax != codes[i]) changed = true;
      const float w = x[i] * x[i];
      const float lf = (float)l;
      slx += w * x[i] * lf;
      sl2 += w * lf * lf;
    }
    if (!changed || sl2 == 0.0f || slx * slx <= best * sl2) break;
    for (int i = 0; i < n; ++i) codes[i] = (int8_t)(nmax + clamp_i(round_i(is * x[i]), -nmax, nmax - 1));
    sumlx = slx;
    suml2 = sl2;
    scale = sumlx / suml2;
    best = scale * sumlx;
  }
  for (int t = 0; t < 5; ++t) {
    int n_changed = 0;
    for (int i = 0; i < n; ++i) {
      const float w = x[i] * x[i];
      const int l = codes[i] - nmax;
      float slx = sumlx - w * x[i] * (float)l;
      if (slx > 0.0f) {
        float sl2 = suml2 - w * (float)l * (float)l;
        const int nl = clamp_i(round_i(x[i] * sl2 / slx), -nmax, nmax - 1);
        if (nl != l) {
          slx += w * x[i] * (float)nl;
          sl2 += w * (float)nl * (float)nl;
          if (sl2 > 0.0f && slx * slx * suml2 > sumlx * sumlx * sl2) {
            codes[i] = (int8_t)(nmax + nl);
            sumlx = slx;
            suml2 = sl2;
            scale = sumlx / suml2;
            best = scale * sumlx;
            ++n_changed;
          }
        }
      }
    }
    if (n_changed == 0) break;
  }
  return scale;
}

__device__ void q6k_quantize_block(const float* __restrict__ x, uint8_t* __restrict__ out) {
#pragma clang fp contract(off)
  int8_t codes[256];
  float scales[16];
  float max_scale = 0.0f, max_abs = 0.0f;
  for (int ib = 0; ib < 16; ++ib) {
    const float s = fit_qx16(32, x + 16 * ib, codes + 16 * ib);
    scales[ib] = s;
    const float a = fabsf(s);
    if (a > max_abs) {
      max_abs = a;
      max_scale = s;
    }
  }
  const float iscale = -128.0f / max_scale;
  const uint16_t dh = f2h(1.0f / iscale);
  int8_t sc8[16];
  for (int j = 0; j < 16; ++j) {
    const int v = round_i(iscale * scales[j]);
    sc8[j] = (int8_t)(v < 127 ? v : 127);
  }
  const float df = h2f(dh);
  for (int j = 0; j < 16; ++j) {
    const float d = df * (float)sc8[j];
    if (d == 0.0f) continue;
    for (int i = 0; i < 16; ++i)
      codes[16 * j + i] = (int8_t)(clamp_i(round_i(x[16 * j + i] / d), -32, 31) + 32);
  }
  uint8_t* ql = out;
  uint8_t* qh = out + 128;
  for (int h = 0; h < 2; ++h) {
    const int8_t* c = codes + 128 * h;
    for (int l = 0; l < 32; ++l) {
      ql[64 * h + l] = (uint8_t)((c[l] & 0xf) | ((c[l + 64] & 0xf) << 4));
      ql[64 * h + 32 + l] = (uint8_t)((c[l + 32] & 0xf) | ((c[l + 96] & 0xf) << 4));
      qh[32 * h + l] = (uint8_t)(((c[l] >> 4) & 3) | (((c[l + 32] >> 4) & 3) << 2) |
                                 (((c[l + 64] >> 4) & 3) << 4) | (((c[l + 96] >> 4) & 3) << 6));
    }
  }
  for (int j = 0; j < 16; ++j) out[192 + j] = (uint8_t)sc8[j];
  out[208] = (uint8_t)dh;
  out[209] = (uint8_t)(dh >> 8);
}

}  // namespace qmm

// ===========================================================================
// kernels
// ===========================================================================

// x: f32 [m, k] row stride ldx; y: m*k/256 Q8_K blocks. One wave per block.
extern "C" __global__ void __launch_bounds__(256) qmm_quantize_q8k(const float* __restrict__ x,
                                                                   long long ldx, uint8_t* __restrict__ y,
                                                                   int k, int m) {
  const int nb = k / 256;
  const long long w = (long long)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (w >= (long long)m * nb) return;
  const int row = (int)(w / nb), b = (int)(w % nb);
  qmm::q8k_block(x + row * ldx + 256LL * b, y + w * qmm::kQ8KBytes, threadIdx.x & 63);
}

// x: f32 [m, k] row stride ldx; y: m*k/32 GGML Q8_0 blocks. 8 lanes per block.
extern "C" __global__ void __launch_bounds__(256) qmm_quantize_q8_0(const float* __restrict__ x,
                                                                    long long ldx, uint8_t* __restrict__ y,
                                                                    int k, int m) {
  const int nb = k / 32;
  const long long t = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  const long long blk = t >> 3;
  const bool valid = blk < (long long)m * nb;
  const long long bc = valid ? blk : 0;
  const int row = (int)(bc / nb), b = (int)(bc % nb);
  qmm::q80_block(x + row * ldx + 32LL * b, y + bc * qmm::kQ80Bytes, (int)(t & 7), valid);
}

// Weight quantizers to GGML bytes: one thread per super-block.
extern "C" __global__ void __launch_bounds__(64) qmm_quantize_q4k_w(const float* __restrict__ w,
                                                                   uint8_t* __restrict__ out,
                                                                   long long nblocks) {
  const long long b = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= nblocks) return;
  qmm::q4k_quantize_block(w + 256 * b, out + qmm::kQ4KBytes * b);
}

extern "C" __global__ void __launch_bounds__(64) qmm_quantize_q6k_w(const float* __restrict__ w,
                                                                   uint8_t* __restrict__ out,
                                                                   long long nblocks) {
  const long long b = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= nblocks) return;
  qmm::q6k_quantize_block(w + 256 * b, out + qmm::kQ6KBytes * b);
}

// GGML bytes <-> device layout for the formats whose blocks are not 16-byte
// multiples (Q6_K: body | d at the end; Q8_0: d | qs at the front).
// One thread per block, 16-bit copies (GGML blocks are 2-byte aligned).
extern "C" __global__ void qmm_ggml_to_dev(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst,
                                           long long nblocks, int fmt) {
  const long long b = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= nblocks) return;
  if (fmt == qmm::kFmtQ6K) {
    const uint16_t* s = reinterpret_cast<const uint16_t*>(src + qmm::kQ6KBytes * b);
    uint16_t* body = reinterpret_cast<uint16_t*>(dst + qmm::kQ6KBody * b);
    for (int i = 0; i < qmm::kQ6KBody / 2; ++i) body[i] = s[i];
    reinterpret_cast<uint16_t*>(dst + qmm::kQ6KBody * nblocks)[b] = s[qmm::kQ6KBody / 2];
  } else {
    const uint16_t* s = reinterpret_cast<const uint16_t*>(src + qmm::kQ80Bytes * b);
    uint16_t* body = reinterpret_cast<uint16_t*>(dst + qmm::kQ80Body * b);
    for (int i = 0; i < qmm::kQ80Body / 2; ++i) body[i] = s[1 + i];
    reinterpret_cast<uint16_t*>(dst + qmm::kQ80Body * nblocks)[b] = s[0];
  }
}

extern "C" __global__ void qmm_dev_to_ggml(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst,
                                           long long nblocks, int fmt) {
  const long long b = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= nblocks) return;
  if (fmt == qmm::kFmtQ6K) {
    const uint16_t* body = reinterpret_cast<const uint16_t*>(src + qmm::kQ6KBody * b);
    uint16_t* d = reinterpret_cast<uint16_t*>(dst + qmm::kQ6KBytes * b);
    for (int i = 0; i < qmm::kQ6KBody / 2; ++i) d[i] = body[i];
    d[qmm::kQ6KBody / 2] = reinterpret_cast<const uint16_t*>(src + qmm::kQ6KBody * nblocks)[b];
  } else {
    const uint16_t* body = reinterpret_cast<const uint16_t*>(src + qmm::kQ80Body * b);
    uint16_t* d = reinterpret_cast<uint16_t*>(dst + qmm::kQ80Bytes * b);
    d[0] = reinterpret_cast<const uint16_t*>(src + qmm::kQ80Body * nblocks)[b];
    for (int i = 0; i < qmm::kQ80Body / 2; ++i) d[1 + i] = body[i];
  }
}

// Dequantize a device-layout tensor (QTensor::dequantize). One thread per 32
// consecutive outputs; formulas of crates/llm/mlx-llm/src/gguf/dequant.rs
// :284-290 (Q8_0), :391-416 (Q4_K), :452-474 (Q6_K), one rounding per f32
// operation; the f16 / bf16 outputs round the f32 value once more, to
// nearest even (the f32 dequantize followed by to_dtype).
namespace qmm {
__device__ __forceinline__ void put_val(float* y, long long i, float v) { y[i] = v; }
__device__ __forceinline__ void put_val(_Float16* y, long long i, float v) { y[i] = (_Float16)v; }
__device__ __forceinline__ void put_val(uint16_t* y, long long i, float v) {  // bf16, round to nearest even
  const uint32_t b = __builtin_bit_cast(uint32_t, v);
  y[i] = (uint16_t)((b + 0x7fffu + ((b >> 16) & 1u)) >> 16);
}

template <class T>
__device__ __forceinline__ void dequantize_blocks(const uint8_t* __restrict__ src, T* __restrict__ y,
                                                  long long nblocks, int fmt) {
#pragma clang fp contract(off)
  const long long t = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (fmt == kFmtQ80) {
    if (t >= nblocks) return;
    const int8_t* q = reinterpret_cast<const int8_t*>(src + kQ80Body * t);
    const float d = h2f(reinterpret_cast<const uint16_t*>(src + kQ80Body * nblocks)[t]);
    for (int j = 0; j < 32; ++j) put_val(y, 32 * t + j, (float)q[j] * d);
    return;
  }
  const long long b = t >> 3;
  const int part = (int)(t & 7);
  if (b >= nblocks) return;
  const long long o = 256 * b + 32 * part;
  if (fmt == kFmtQ4K) {
    const uint8_t* blk = src + kQ4KBytes * b;
    const float d = h2f(blk[0] | (blk[1] << 8)), dmin = h2f(blk[2] | (blk[3] << 8));
    int sc, m;
    q4k_scale_min(part, blk + 4, &sc, &m);
    const float d1 = d * (float)sc, m1 = dmin * (float)m;
    const uint8_t* qs = blk + 16 + 32 * (part >> 1);
    const int sh = (part & 1) * 4;
    for (int l = 0; l < 32; ++l) put_val(y, o + l, d1 * (float)((qs[l] >> sh) & 0xf) - m1);
  } else {
    const uint8_t* body = src + kQ6KBody * b;
    const float d = h2f(reinterpret_cast<const uint16_t*>(src + kQ6KBody * nblocks)[b]);
    const int8_t* sc = reinterpret_cast<const int8_t*>(body + 192);
    // outputs 128h + 32s + [0, 32): ql low/high nibble and 2 bits of qh.
    const int h = part >> 2, s = part & 3;
    const uint8_t* ql = body + 64 * h + 32 * (s & 1);
    const uint8_t* qh = body + 128 + 32 * h;
    const int nsh = (s >> 1) * 4, hsh = 2 * s;
    for (int l = 0; l < 32; ++l) {
      const int q = (((ql[l] >> nsh) & 0xf) | (((qh[l] >> hsh) & 3) << 4)) - 32;
      put_val(y, o + l, d * (float)sc[8 * h + 2 * s + l / 16] * (float)q);
    }
  }
}
}  // namespace qmm

extern "C" __global__ void qmm_dequantize(const uint8_t* __restrict__ src, float* __restrict__ y, long long nblocks,
                                          int fmt) {
  qmm::dequantize_blocks(src, y, nblocks, fmt);
}
extern "C" __global__ void qmm_dequantize_f16(const uint8_t* __restrict__ src, _Float16* __restrict__ y,
                                              long long nblocks, int fmt) {
  qmm::dequantize_blocks(src, y, nblocks, fmt);
}
extern "C" __global__ void qmm_dequantize_bf16(const uint8_t* __restrict__ src, uint16_t* __restrict__ y,
                                               long long nblocks, int fmt) {
  qmm::dequantize_blocks(src, y, nblocks, fmt);
}
