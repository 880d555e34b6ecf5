// Decode GEMV (M = 1..8 activation rows) over Q8_0 / Q4_K / Q6_K weights.
//
// Work split (wave64, CDNA4):
//   * a k-quant super-block is decoded by 8 lanes, each owning one 16-byte
//     slice of its quants (one dwordx4 load); a wave-wide load therefore
//     covers 8 consecutive super-blocks of a row, i.e. ~1.1 KB (Q4_K) or
//     ~1.7 KB (Q6_K) of contiguous HBM. Q8_0 uses 2 lanes per 32-block.
//   * the activation rows (already quantized to Q8_K / Q8_0) are staged once
//     per workgroup in LDS, permuted so that each lane reads its two 16-byte
//     operand slices and its pair of 16-element sums with single LDS reads;
//   * each wave owns R weight rows and issues U iterations of loads for all of
//     them before using any, so every lane has R*U 16-byte loads in flight;
//   * integer block dots use v_dot4_i32_i8; the f32 row sums are reduced
//     across the wave with DPP row operations and two cross-row exchanges.
// Integer decomposition per super-block (the algebraic image of the GGML
// dequantizers, crates/llm/mlx-llm/src/gguf/dequant.rs:284-290, 391-416, 452-474):
//   Q4_K: y += d*dx*sum_j sc_j*(q4 . q8)_j - dmin*dx*sum_j m_j*(bsum_2j + bsum_2j+1)
//   Q6_K: y += d*dx*sum_j sc_j*((q6 . q8)_j - 32*bsum_j)
//   Q8_0: y += d*dx*(qw . qx)
// The CUDA kernel this replaces is mmvq_core_impl (candle-kernels/src/mmvq_gguf.cu:644-715).
#pragma once

#include "qmm_common.h"

namespace qmm {

template <int FMT>
struct FmtInfo;
template <>
struct FmtInfo<kFmtQ80> {
  static constexpr int kLanesPerBlock = 2;
  static constexpr int kBlockElems = 32;
  static constexpr int kBodyBytes = kQ80Body;
};
template <>
struct FmtInfo<kFmtQ4K> {
  static constexpr int kLanesPerBlock = 8;
  static constexpr int kBlockElems = 256;
  static constexpr int kBodyBytes = kQ4KBytes;
};
template <>
struct FmtInfo<kFmtQ6K> {
  static constexpr int kLanesPerBlock = 8;
  static constexpr int kBlockElems = 256;
  static constexpr int kBodyBytes = kQ6KBody;
};

// LDS bytes per staged activation block.
template <int FMT>
constexpr int lds_block_bytes() {
  return FMT == kFmtQ80 ? 32 + 4 : 256 + 32 + 4;
}

// Start of the two 16-element activation slices lane l (0..7) of a k-quant
// super-block multiplies.
//   Q4_K lane l: quants qs[16l, 16l+16): low nibbles are elements
//                64(l/2) + 16(l%2) + i, high nibbles 32 further.
//   Q6_K lane l: ql[16l, 16l+16) low nibbles are elements 128(l/4) + 16(l%4) + i,
//                high nibbles 64 further.
template <int FMT>
__device__ __forceinline__ int act_slice0(int l) {
  return FMT == kFmtQ4K ? 64 * (l >> 1) + 16 * (l & 1) : 128 * (l >> 2) + 16 * (l & 3);
}
template <int FMT>
constexpr int act_slice_gap() {
  return FMT == kFmtQ4K ? 32 : 64;
}

// Stage m_rows activation rows of nb blocks each into LDS.
//   k-quants: q8[blk][256] = [slice0 of lanes 0..7][slice1 of lanes 0..7],
//             bsum pairs u32[blk][8], d f32[blk]
//   Q8_0:     q8[blk][32], d f32[blk]
template <int FMT>
__device__ __forceinline__ void stage_act(const uint8_t* __restrict__ xq, int nblk, uint8_t* lds) {
  if constexpr (FMT == kFmtQ80) {
    float* ld = reinterpret_cast<float*>(lds + 32 * nblk);
    for (int t = threadIdx.x; t < 2 * nblk; t += blockDim.x) {
      const int blk = t >> 1, half = t & 1;
      const uint16_t* s = reinterpret_cast<const uint16_t*>(xq + (size_t)kQ80Bytes * blk);
      const uint16_t* q = s + 1 + 8 * half;
      uint4 v;
      v.x = q[0] | ((uint32_t)q[1] << 16);
      v.y = q[2] | ((uint32_t)q[3] << 16);
      v.z = q[4] | ((uint32_t)q[5] << 16);
      v.w = q[6] | ((uint32_t)q[7] << 16);
      *reinterpret_cast<uint4*>(lds + 32 * blk + 16 * half) = v;
      if (half == 0) ld[blk] = h2f(s[0]);
    }
  } else {
    uint32_t* lb = reinterpret_cast<uint32_t*>(lds + 256 * nblk);
    float* ld = reinterpret_cast<float*>(lb + 8 * nblk);
    for (int t = threadIdx.x; t < 8 * nblk; t += blockDim.x) {
      const int blk = t >> 3, l = t & 7;
      const uint8_t* s = xq + (size_t)kQ8KBytes * blk;
      const uint32_t* q = reinterpret_cast<const uint32_t*>(s + 4);
      const int s0 = act_slice0<FMT>(l), s1 = s0 + act_slice_gap<FMT>();
      uint4 a, b;
      a.x = q[s0 / 4 + 0];
      a.y = q[s0 / 4 + 1];
      a.z = q[s0 / 4 + 2];
      a.w = q[s0 / 4 + 3];
      b.x = q[s1 / 4 + 0];
      b.y = q[s1 / 4 + 1];
      b.z = q[s1 / 4 + 2];
      b.w = q[s1 / 4 + 3];
      *reinterpret_cast<uint4*>(lds + 256 * blk + 16 * l) = a;
      *reinterpret_cast<uint4*>(lds + 256 * blk + 128 + 16 * l) = b;
      const uint16_t* bs = reinterpret_cast<const uint16_t*>(s + 4 + 256);
      lb[8 * blk + l] = (uint32_t)bs[s0 / 16] | ((uint32_t)bs[s1 / 16] << 16);
      if (l == 0) ld[blk] = *reinterpret_cast<const float*>(s);
    }
  }
}

// One lane's share of one weight super-block.
struct WSlice {
  uint4 a;     // Q4_K: header (d, dmin, scales[12]); Q6_K: ql slice; Q8_0: qs slice
  uint4 b;     // Q4_K: qs slice; Q6_K: qh slice
  uint4 c;     // Q6_K: scales[16]
  uint32_t d;  // Q6_K / Q8_0: f16 scale
};

// Weight row pointers: `wq` = block bodies, `wd` = separated f16 scales.
template <int FMT>
__device__ __forceinline__ void load_slice(WSlice& s, const uint8_t* __restrict__ wq,
                                           const uint16_t* __restrict__ wd, size_t blk, int l) {
  if constexpr (FMT == kFmtQ4K) {
    const uint8_t* p = wq + blk * kQ4KBytes;
    s.a = *reinterpret_cast<const uint4*>(p);
    s.b = *reinterpret_cast<const uint4*>(p + 16 + 16 * l);
  } else if constexpr (FMT == kFmtQ6K) {
    const uint8_t* p = wq + blk * kQ6KBody;
    s.a = *reinterpret_cast<const uint4*>(p + 16 * l);
    s.b = *reinterpret_cast<const uint4*>(p + 128 + 32 * (l >> 2) + 16 * (l & 1));
    s.c = *reinterpret_cast<const uint4*>(p + 192);
    s.d = wd[blk];
  } else {
    s.a = *reinterpret_cast<const uint4*>(wq + blk * kQ80Body + 16 * l);
    s.d = wd[blk];
  }
}

// Multiply one lane's slice with the staged activation block `xb` of each of
// the M rows (row stride `nbx` blocks in LDS). Adds to acc (when ok) and
// returns the lane's integer partials in ia / ib.
template <int FMT, int M>
__device__ __forceinline__ void dot_slice(const WSlice& s, int l, const uint8_t* __restrict__ lds,
                                          int nblk, int xb, int nbx, bool ok, float (&acc)[M],
                                          int (&ia)[M], int (&ib)[M]) {
  if constexpr (FMT == kFmtQ4K) {
    const uint32_t* lb = reinterpret_cast<const uint32_t*>(lds + 256 * nblk);
    const float* ld = reinterpret_cast<const float*>(lb + 8 * nblk);
    const float dw = h2f(s.a.x), dm = h2f(s.a.x >> 16);
    // 6-bit scale/min pairs of sub-blocks 2c and 2c+1, c = l/2 (get_scale_min_k4).
    const int c = l >> 1;
    const int sh = (c & 1) * 16;
    const uint32_t A = s.a.y >> sh, B = s.a.z >> sh, C = s.a.w >> sh;
    const bool upper = c >= 2;
    const uint32_t scp = upper ? ((C & 0x0f0fu) | ((A >> 2) & 0x3030u)) : (A & 0x3f3fu);
    const uint32_t mnp = upper ? (((C >> 4) & 0x0f0fu) | ((B >> 2) & 0x3030u)) : (B & 0x3f3fu);
    const int sc0 = scp & 0xff, sc1 = (scp >> 8) & 0xff;
    const int m0 = mnp & 0xff, m1 = (mnp >> 8) & 0xff;
    const uint32_t lo0 = s.b.x & 0x0f0f0f0fu, hi0 = (s.b.x >> 4) & 0x0f0f0f0fu;
    const uint32_t lo1 = s.b.y & 0x0f0f0f0fu, hi1 = (s.b.y >> 4) & 0x0f0f0f0fu;
    const uint32_t lo2 = s.b.z & 0x0f0f0f0fu, hi2 = (s.b.z >> 4) & 0x0f0f0f0fu;
    const uint32_t lo3 = s.b.w & 0x0f0f0f0fu, hi3 = (s.b.w >> 4) & 0x0f0f0f0fu;
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const int bx = xb + m * nbx;
      const uint8_t* e = lds + 256 * bx + 16 * l;
      const uint4 x0 = *reinterpret_cast<const uint4*>(e);
      const uint4 x1 = *reinterpret_cast<const uint4*>(e + 128);
      int s0 = dot4(lo0, x0.x, 0);
      s0 = dot4(lo1, x0.y, s0);
      s0 = dot4(lo2, x0.z, s0);
      s0 = dot4(lo3, x0.w, s0);
      int s1 = dot4(hi0, x1.x, 0);
      s1 = dot4(hi1, x1.y, s1);
      s1 = dot4(hi2, x1.z, s1);
      s1 = dot4(hi3, x1.w, s1);
      const uint32_t bp = lb[8 * bx + l];
      const int bs0 = (int)(int16_t)(bp & 0xffffu), bs1 = (int)bp >> 16;
      const int isd = sc0 * s0 + sc1 * s1;
      const int ism = m0 * bs0 + m1 * bs1;
      const float t = dw * (float)isd - dm * (float)ism;
      acc[m] += ok ? ld[bx] * t : 0.0f;
      ia[m] = isd;
      ib[m] = ism;
    }
  } else if constexpr (FMT == kFmtQ6K) {
    const uint32_t* lb = reinterpret_cast<const uint32_t*>(lds + 256 * nblk);
    const float* ld = reinterpret_cast<const float*>(lb + 8 * nblk);
    const float dw = h2f(s.d);
    const int h = l >> 2, j = l & 3;
    const int sh0 = (j >> 1) * 2, sh1 = sh0 + 4;
    const uint32_t w0 = h ? s.c.z : s.c.x, w1 = h ? s.c.w : s.c.y;
    const int sc0 = (int)(int8_t)(w0 >> (8 * j)), sc1 = (int)(int8_t)(w1 >> (8 * j));
    uint32_t q0[4], q1[4];
    const uint32_t ql[4] = {s.a.x, s.a.y, s.a.z, s.a.w};
    const uint32_t qh[4] = {s.b.x, s.b.y, s.b.z, s.b.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      q0[k] = (ql[k] & 0x0f0f0f0fu) | (((qh[k] >> sh0) & 0x03030303u) << 4);
      q1[k] = ((ql[k] >> 4) & 0x0f0f0f0fu) | (((qh[k] >> sh1) & 0x03030303u) << 4);
    }
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const int bx = xb + m * nbx;
      const uint8_t* e = lds + 256 * bx + 16 * l;
      const uint4 x0 = *reinterpret_cast<const uint4*>(e);
      const uint4 x1 = *reinterpret_cast<const uint4*>(e + 128);
      int s0 = dot4(q0[0], x0.x, 0);
      s0 = dot4(q0[1], x0.y, s0);
      s0 = dot4(q0[2], x0.z, s0);
      s0 = dot4(q0[3], x0.w, s0);
      int s1 = dot4(q1[0], x1.x, 0);
      s1 = dot4(q1[1], x1.y, s1);
      s1 = dot4(q1[2], x1.z, s1);
      s1 = dot4(q1[3], x1.w, s1);
      const uint32_t bp = lb[8 * bx + l];
      const int bs0 = (int)(int16_t)(bp & 0xffffu), bs1 = (int)bp >> 16;
      const int is = sc0 * (s0 - 32 * bs0) + sc1 * (s1 - 32 * bs1);
      acc[m] += ok ? ld[bx] * (dw * (float)is) : 0.0f;
      ia[m] = is;
      ib[m] = 0;
    }
  } else {
    const float* ld = reinterpret_cast<const float*>(lds + 32 * nblk);
    const float dw = h2f(s.d);
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const int bx = xb + m * nbx;
      const uint4 x0 = *reinterpret_cast<const uint4*>(lds + 32 * bx + 16 * l);
      int s0 = dot4(s.a.x, x0.x, 0);
      s0 = dot4(s.a.y, x0.y, s0);
      s0 = dot4(s.a.z, x0.z, s0);
      s0 = dot4(s.a.w, x0.w, s0);
      acc[m] += ok ? (dw * ld[bx]) * (float)s0 : 0.0f;
      ia[m] = s0;
      ib[m] = 0;
    }
  }
}

// y[m, n] = sum_b dot(W[n, b], X[m, b]) for m < M, n < N.
//   wq: weight blocks (device layout), N rows of nb blocks; wd: separated f16
//   scales (Q6_K, Q8_0) right after the bodies; xq: M rows of nb activation
//   blocks (Q8_K or Q8_0, GGML bytes); dump (optional): int32 block dots.
template <int FMT, int M, int R, int U>
__device__ __forceinline__ void gemv(const uint8_t* __restrict__ wq, const uint8_t* __restrict__ xq,
                                     float* __restrict__ y, int N, int K, int ldy,
                                     int* __restrict__ dump) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  constexpr int LPB = FmtInfo<FMT>::kLanesPerBlock;
  constexpr int BPI = 64 / LPB;  // blocks per wave iteration
  const int nb = K / FmtInfo<FMT>::kBlockElems;
  stage_act<FMT>(xq, M * nb, lds);
  __syncthreads();

  const uint16_t* wd =
      FMT == kFmtQ4K ? nullptr
                     : reinterpret_cast<const uint16_t*>(wq + (size_t)N * nb * FmtInfo<FMT>::kBodyBytes);
  const int lane = threadIdx.x & 63;
  const int nw = blockDim.x >> 6;
  const int l = lane % LPB;
  const int g = lane / LPB;
  const int niter = (nb + BPI - 1) / BPI;
  const int row_step = gridDim.x * nw * R;

  for (int row0 = (blockIdx.x * nw + (threadIdx.x >> 6)) * R; row0 < N; row0 += row_step) {
    float acc[R][M];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int m = 0; m < M; ++m) acc[r][m] = 0.0f;

    for (int it0 = 0; it0 < niter; it0 += U) {
      WSlice ws[R][U];
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int b = (it0 + u) * BPI + g;
          ws[r][u] = WSlice{};
          if (row0 + r < N && b < nb) load_slice<FMT>(ws[r][u], wq, wd, (size_t)(row0 + r) * nb + b, l);
        }
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int b = (it0 + u) * BPI + g;
          const bool ok = row0 + r < N && b < nb;
          int ia[M], ib[M];
          dot_slice<FMT, M>(ws[r][u], l, lds, M * nb, ok ? b : 0, nb, ok, acc[r], ia, ib);
          if (dump != nullptr) {
#pragma unroll
            for (int m = 0; m < M; ++m) {
              int va = ia[m], vb = ib[m];
#pragma unroll
              for (int off = 1; off < LPB; off <<= 1) {
                va += __shfl_xor(va, off);
                vb += __shfl_xor(vb, off);
              }
              if (ok && l == 0) {
                const size_t o = ((size_t)m * N + row0 + r) * nb + b;
                if (FMT == kFmtQ4K) {
                  dump[2 * o] = va;
                  dump[2 * o + 1] = vb;
                } else {
                  dump[o] = va;
                }
              }
            }
          }
        }
    }
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int m = 0; m < M; ++m) {
        const float v = wave_sum(acc[r][m]);
        if (lane == 0 && row0 + r < N) y[(size_t)m * ldy + row0 + r] = v;
      }
  }
}

}  // namespace qmm

#define QMM_GEMV_KERNEL(FMT, NAME, M, R, U)                                                         \
  extern "C" __global__ void __launch_bounds__(256)                                                \
      qmm_gemv_##NAME##_m##M##_r##R##_u##U(const uint8_t* __restrict__ wq,                         \
                                           const uint8_t* __restrict__ xq, float* __restrict__ y,  \
                                           int N, int K, int ldy, int* __restrict__ dump) {        \
    qmm::gemv<FMT, M, R, U>(wq, xq, y, N, K, ldy, dump);                                           \
  }

#define QMM_GEMV_SHAPES(FMT, NAME, M) \
  QMM_GEMV_KERNEL(FMT, NAME, M, 4, 2) \
  QMM_GEMV_KERNEL(FMT, NAME, M, 2, 2) \
  QMM_GEMV_KERNEL(FMT, NAME, M, 1, 4) \
  QMM_GEMV_KERNEL(FMT, NAME, M, 1, 8)

#define QMM_GEMV_ALL_M(FMT, NAME) \
  QMM_GEMV_SHAPES(FMT, NAME, 1)   \
  QMM_GEMV_SHAPES(FMT, NAME, 2)   \
  QMM_GEMV_SHAPES(FMT, NAME, 3)   \
  QMM_GEMV_SHAPES(FMT, NAME, 4)   \
  QMM_GEMV_SHAPES(FMT, NAME, 5)   \
  QMM_GEMV_SHAPES(FMT, NAME, 6)   \
  QMM_GEMV_SHAPES(FMT, NAME, 7)   \
  QMM_GEMV_SHAPES(FMT, NAME, 8)

QMM_GEMV_ALL_M(qmm::kFmtQ4K, q4k)
QMM_GEMV_ALL_M(qmm::kFmtQ6K, q6k)
QMM_GEMV_ALL_M(qmm::kFmtQ80, q8_0)
