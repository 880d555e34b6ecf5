// Prefill GEMM (M > 8 activation rows) on int8 MFMA (v_mfma_i32_32x32x32_i8).
//
// The contraction is split the way the GGML formats scale it:
//   Q4_K: for each 32-element sub-block j, P_j = q8 . q4 is one MFMA (K = 32)
//         per 32x32 tile; isum_d += sc_j * P_j (v_mad_i32_i24); the mins term
//         isum_m = sum_j m_j * (bsum_2j + bsum_2j+1) is two zero-padded MFMAs
//         (activation sums split into 6-bit low / signed high bytes);
//         y += dx * (d * isum_d - dmin * isum_m) once per super-block.
//   Q6_K: each 32-element chunk is two 16-element groups with their own int8
//         scale; the activation operand is masked to one lane half (one group)
//         per MFMA; isum += sc_g * P_g; y += dx * d * isum per super-block.
//   Q8_0: one MFMA per 32-block, y += (dw * dx) * P.
// Activations come from a plane layout written by qmm_quantize_*_mmq (int8
// [M][K], f32 scales, int16 32-element sums), weights from the tensors'
// device layout; both are staged in LDS per 256-wide K step, the weights
// dequantized to int8 on the way.
// Workgroup: 256 threads, tile 64 (M) x 128 (N); wave w owns rows
// 32*(w&1) .. +32 and columns 64*(w>>1) .. +64 (two 32x32 MFMA tiles).
// The next K step's global loads are issued before the current step's MFMAs.
// The CUDA kernels this replaces are mul_mat_q (candle-kernels/src/mmq_gguf/mmq_gguf.cuh:3526-3778).
#pragma once

#include "qmm_common.h"
#include "qmm_quant_kernels.h"

namespace qmm {

typedef char i8x16 __attribute__((ext_vector_type(16)));
typedef int i32x16 __attribute__((ext_vector_type(16)));

constexpr int kMmqBM = 64;
constexpr int kMmqBN = 128;
constexpr int kMmqStride = 256 + 16;  // LDS row stride of the int8 tiles (16-byte skew per row)

struct MmqLds {
  int8_t a[kMmqBM * kMmqStride];   // activations, int8 [row][k]
  int8_t b[kMmqBN * kMmqStride];   // weights, int8 [col][k]
  float ad[kMmqBM * 8];            // activation scales: per row (k-quants) or per 32-block (Q8_0)
  int8_t as[kMmqBM * 16];          // Q4_K: 32-element sums, low 6 bits [0..8) and high part [8..16)
  int8_t bsc[kMmqBN * 16];         // Q4_K: sc[8] | m[8]; Q6_K: sc[16]
  float bd[kMmqBN * 8];            // Q4_K: d, dmin; Q6_K: d; Q8_0: d of the 8 blocks
};

// Per-thread registers of one K step (256 elements) before they go to LDS.
struct MmqRegs {
  uint4 a[4];   // 64 activation bytes of one row
  float ad[2];  // activation scale(s)
  uint4 as;     // Q4_K activation sums (8 x int16)
  uint4 w[8];   // weight bytes (format dependent)
  uint32_t wd[4];
};

template <int FMT>
__device__ __forceinline__ void mmq_load(MmqRegs& R, const int8_t* __restrict__ xq, const float* __restrict__ xd,
                                         const int16_t* __restrict__ xs, const uint8_t* __restrict__ wq,
                                         const uint16_t* __restrict__ wd, int M, int N, int K, int m0, int n0,
                                         int kb) {
  const int t = threadIdx.x;
  const int nbk = K / 256;
  // activations: thread t -> row t/4, bytes [64*(t%4), +64) of this K step
  {
    const int row = m0 + (t >> 2);
    const bool ok = row < M;
    const uint4* p = reinterpret_cast<const uint4*>(xq + (size_t)(ok ? row : 0) * K + 256 * kb + 64 * (t & 3));
#pragma unroll
    for (int i = 0; i < 4; ++i) R.a[i] = ok ? p[i] : make_uint4(0, 0, 0, 0);
  }
  if (FMT == kFmtQ80) {
    // 8 scales per row per K step: thread t < 256 -> row t/4, blocks 2*(t%4), +1
    const int row = m0 + (t >> 2);
    const bool ok = row < M;
    const float* p = xd + (size_t)(ok ? row : 0) * (K / 32) + 8 * kb + 2 * (t & 3);
    R.ad[0] = ok ? p[0] : 0.0f;
    R.ad[1] = ok ? p[1] : 0.0f;
  } else if (t < kMmqBM) {
    const int row = m0 + t;
    const bool ok = row < M;
    R.ad[0] = ok ? xd[(size_t)row * nbk + kb] : 0.0f;
    if (FMT == kFmtQ4K)
      R.as = ok ? *reinterpret_cast<const uint4*>(xs + ((size_t)row * nbk + kb) * 8) : make_uint4(0, 0, 0, 0);
  }
  // weights: thread t -> column t/2, half p = t%2 of the K step
  const int col = n0 + (t >> 1), p = t & 1;
  const bool okc = col < N;
  const size_t blk = (size_t)(okc ? col : 0) * (FMT == kFmtQ80 ? K / 32 : nbk) + (FMT == kFmtQ80 ? 8 * kb : kb);
  if (FMT == kFmtQ4K) {
    const uint4* b = reinterpret_cast<const uint4*>(wq + blk * kQ4KBytes);
    R.w[0] = b[0];  // d, dmin, scales
#pragma unroll
    for (int i = 0; i < 4; ++i) R.w[1 + i] = b[1 + 4 * p + i];  // qs[64p, 64p+64)
  } else if (FMT == kFmtQ6K) {
    const uint4* b = reinterpret_cast<const uint4*>(wq + blk * kQ6KBody);
#pragma unroll
    for (int i = 0; i < 4; ++i) R.w[i] = b[4 * p + i];         // ql[64p, 64p+64)
    R.w[4] = b[8 + 2 * p];                                      // qh[32p, 32p+32)
    R.w[5] = b[9 + 2 * p];
    R.w[6] = b[12];                                             // scales
    R.wd[0] = wd[blk];
  } else {
    const uint4* b = reinterpret_cast<const uint4*>(wq + (blk + 4 * p) * kQ80Body);
#pragma unroll
    for (int i = 0; i < 8; ++i) R.w[i] = b[i];  // blocks 4p .. 4p+3 of this K step
    R.wd[0] = wd[blk + 4 * p];
    R.wd[1] = wd[blk + 4 * p + 1];
    R.wd[2] = wd[blk + 4 * p + 2];
    R.wd[3] = wd[blk + 4 * p + 3];
  }
  if (!okc) {
#pragma unroll
    for (int i = 0; i < 8; ++i) R.w[i] = make_uint4(0, 0, 0, 0);
    R.wd[0] = R.wd[1] = R.wd[2] = R.wd[3] = 0;
  }
}

__device__ __forceinline__ uint32_t q6_sub32(uint32_t v) {
  // bytes in [0, 63] minus 32, as int8, without borrows between bytes
  return ((v | 0x80808080u) - 0x20202020u) ^ 0x80808080u;
}

template <int FMT>
__device__ __forceinline__ void mmq_store(const MmqRegs& R, MmqLds& L) {
  const int t = threadIdx.x;
  {
    uint4* dst = reinterpret_cast<uint4*>(L.a + (t >> 2) * kMmqStride + 64 * (t & 3));
#pragma unroll
    for (int i = 0; i < 4; ++i) dst[i] = R.a[i];
  }
  if (FMT == kFmtQ80) {  // [block][row] so a lane's four consecutive rows are one float4
    L.ad[(2 * (t & 3)) * kMmqBM + (t >> 2)] = R.ad[0];
    L.ad[(2 * (t & 3) + 1) * kMmqBM + (t >> 2)] = R.ad[1];
  } else if (t < kMmqBM) {
    L.ad[t] = R.ad[0];
    if (FMT == kFmtQ4K) {
      // 32-element sums s (|s| <= 4096): s = 64*hi + lo, lo in [0,63], hi in [-64, 64]
      const int16_t* s = reinterpret_cast<const int16_t*>(&R.as);
      int8_t* d = L.as + 16 * t;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int v = s[j];
        d[j] = (int8_t)(v & 63);
        d[8 + j] = (int8_t)(v >> 6);
      }
    }
  }
  const int c = t >> 1, p = t & 1;
  int8_t* brow = L.b + c * kMmqStride;
  if (FMT == kFmtQ4K) {
    // qs[64p + 16i ...] -> chunk cc = 2p + i/2: low nibbles at 64cc + 16(i%2), high at +32
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int cc = 2 * p + (i >> 1), off = 64 * cc + 16 * (i & 1);
      const uint4 v = R.w[1 + i];
      *reinterpret_cast<uint4*>(brow + off) =
          make_uint4(v.x & 0x0f0f0f0fu, v.y & 0x0f0f0f0fu, v.z & 0x0f0f0f0fu, v.w & 0x0f0f0f0fu);
      *reinterpret_cast<uint4*>(brow + off + 32) = make_uint4((v.x >> 4) & 0x0f0f0f0fu, (v.y >> 4) & 0x0f0f0f0fu,
                                                             (v.z >> 4) & 0x0f0f0f0fu, (v.w >> 4) & 0x0f0f0f0fu);
    }
    if (p == 0) {
      const uint8_t* hb = reinterpret_cast<const uint8_t*>(&R.w[0]);
      int8_t* sc = L.bsc + 16 * c;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        int s, m;
        q4k_scale_min(j, hb + 4, &s, &m);
        sc[j] = (int8_t)s;
        sc[8 + j] = (int8_t)m;
      }
      L.bd[8 * c] = h2f(R.w[0].x);
      L.bd[8 * c + 1] = h2f(R.w[0].x >> 16);
    }
  } else if (FMT == kFmtQ6K) {
    // half h = p: elements 128h + [0,128) from ql[64h, +64) and qh[32h, +32)
    const uint32_t* ql = reinterpret_cast<const uint32_t*>(&R.w[0]);  // 16 dwords
    const uint32_t* qh = reinterpret_cast<const uint32_t*>(&R.w[4]);  // 8 dwords
    int8_t* base = brow + 128 * p;
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const uint32_t l0 = ql[q], l1 = ql[8 + q], h = qh[q];
      const uint32_t e0 = (l0 & 0x0f0f0f0fu) | ((h & 0x03030303u) << 4);                // elements 4q .. (+0)
      const uint32_t e1 = (l1 & 0x0f0f0f0fu) | (((h >> 2) & 0x03030303u) << 4);         // +32
      const uint32_t e2 = ((l0 >> 4) & 0x0f0f0f0fu) | (((h >> 4) & 0x03030303u) << 4);  // +64
      const uint32_t e3 = ((l1 >> 4) & 0x0f0f0f0fu) | (((h >> 6) & 0x03030303u) << 4);  // +96
      *reinterpret_cast<uint32_t*>(base + 4 * q) = q6_sub32(e0);
      *reinterpret_cast<uint32_t*>(base + 32 + 4 * q) = q6_sub32(e1);
      *reinterpret_cast<uint32_t*>(base + 64 + 4 * q) = q6_sub32(e2);
      *reinterpret_cast<uint32_t*>(base + 96 + 4 * q) = q6_sub32(e3);
    }
    if (p == 0) {
      *reinterpret_cast<uint4*>(L.bsc + 16 * c) = R.w[6];
      L.bd[8 * c] = h2f(R.wd[0]);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) *reinterpret_cast<uint4*>(brow + 128 * p + 16 * i) = R.w[i];
#pragma unroll
    for (int i = 0; i < 4; ++i) L.bd[8 * c + 4 * p + i] = h2f(R.wd[i]);
  }
}

__device__ __forceinline__ i32x16 mfma_i8(i8x16 a, i8x16 b, i32x16 c) {
  return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ i8x16 as_i8x16(uint4 v) { return __builtin_bit_cast(i8x16, v); }

// Byte `i` (0..7) of an 8-byte word pair.
__device__ __forceinline__ uint32_t byte8(uint2 w, int i) { return ((i < 4 ? w.x : w.y) >> (8 * (i & 3))) & 0xffu; }

// This workgroup's (M tile, N tile). With remap, the grid's tiles are dealt
// so that the workgroups of one XCD take consecutive tiles in M-major order:
// the dispatcher hands workgroups to the eight XCDs round-robin by linear id
// and every XCD has its own L2, so an XCD's workgroups then share a few M
// tiles' activation rows in that L2 instead of each XCD streaming all of them.
// The map is a bijection of the grid; without remap, tile = (blockIdx.y, .x).
__device__ __forceinline__ void gemm_tile(int remap, int& mt, int& nt) {
  if (!remap) {
    mt = blockIdx.y;
    nt = blockIdx.x;
    return;
  }
  const int gx = gridDim.x, g = gx * gridDim.y;
  const int lin = blockIdx.y * gx + blockIdx.x;
  const int xcd = lin & 7, slot = lin >> 3, q = g >> 3, r = g & 7;
  const int t = (xcd < r ? xcd * (q + 1) : r * (q + 1) + (xcd - r) * q) + slot;
  mt = t / gx;
  nt = t - mt * gx;
}

// Split-K: the K steps [kb0, kb1) of split blockIdx.z (kc steps each); the
// split's f32 partial goes to y + blockIdx.z * ysplit (the host sums the
// splits in order). One split: kc = K / 256, ysplit = 0.
struct KRange {
  int kb0, kb1;
};
__device__ __forceinline__ KRange split_range(int K, int kc) {
  const int kb0 = (int)blockIdx.z * kc, nbk = K / 256;
  return {kb0, kb0 + kc < nbk ? kb0 + kc : nbk};
}

// f16 block scales of a scale-split Q6_K / Q8_0 weight of `rows` rows (they
// follow all block bodies); Q4_K keeps its scales inside the blocks.
template <int FMT>
__device__ __forceinline__ const uint16_t* split_scales(const uint8_t* wq, long long rows, int K) {
  const int nbw = FMT == kFmtQ80 ? K / 32 : K / 256;
  return FMT == kFmtQ4K ? nullptr
                        : reinterpret_cast<const uint16_t*>(wq + (size_t)rows * nbw * FmtInfo<FMT>::kBodyBytes);
}

// y[m, n] = sum over K of x[m, :] . W[n, :] with the formats' scaling; wd =
// the weight's block scales (split_scales). DUMP instantiations also write
// every integer block dot (debug entry point).
template <int FMT, bool DUMP>
__device__ __forceinline__ void mmq(const uint8_t* __restrict__ wq, const uint16_t* __restrict__ wd,
                                    const int8_t* __restrict__ xq, const float* __restrict__ xd,
                                    const int16_t* __restrict__ xs, float* __restrict__ y, int M, int N, int K,
                                    int ldy, int* __restrict__ dump, int accumulate, int remap, int kb0, int kb1) {
  __shared__ MmqLds L;
  int mt, nt;
  gemm_tile(remap, mt, nt);
  const int m0 = mt * kMmqBM, n0 = nt * kMmqBN;
  const int nbk = K / 256;
  const int nbw = FMT == kFmtQ80 ? K / 32 : nbk;  // weight blocks per row
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 31, h = lane >> 5;
  const int wm = wave & 1, wn = wave >> 1;
  const int col0 = 64 * wn + r, col1 = col0 + 32;  // this lane's output columns (tiles 0, 1)
  const int rowb = 32 * wm + 4 * h;                  // + 8g + i: this lane's output rows

  i32x16 zero;
#pragma unroll
  for (int j = 0; j < 16; ++j) zero[j] = 0;
  float acc0[16], acc1[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) acc0[j] = acc1[j] = 0.0f;

  MmqRegs R;
  mmq_load<FMT>(R, xq, xd, xs, wq, wd, M, N, K, m0, n0, kb0);
  for (int kb = kb0; kb < kb1; ++kb) {
    __syncthreads();
    mmq_store<FMT>(R, L);
    __syncthreads();
    if (kb + 1 < kb1) mmq_load<FMT>(R, xq, xd, xs, wq, wd, M, N, K, m0, n0, kb + 1);

    const int8_t* arow = L.a + (32 * wm + r) * kMmqStride + 16 * h;
    const int8_t* b0row = L.b + col0 * kMmqStride + 16 * h;
    const int8_t* b1row = L.b + col1 * kMmqStride + 16 * h;

    if constexpr (FMT == kFmtQ80) {
#pragma unroll 1
      for (int c = 0; c < 8; ++c) {
        const i8x16 a = *reinterpret_cast<const i8x16*>(arow + 32 * c);
        const i32x16 P0 = mfma_i8(a, *reinterpret_cast<const i8x16*>(b0row + 32 * c), zero);
        const i32x16 P1 = mfma_i8(a, *reinterpret_cast<const i8x16*>(b1row + 32 * c), zero);
        const float dw0 = L.bd[8 * col0 + c], dw1 = L.bd[8 * col1 + c];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const float4 dx = *reinterpret_cast<const float4*>(&L.ad[c * kMmqBM + rowb + 8 * g]);
          const float dxs[4] = {dx.x, dx.y, dx.z, dx.w};
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            acc0[4 * g + i] += (dw0 * dxs[i]) * (float)P0[4 * g + i];
            acc1[4 * g + i] += (dw1 * dxs[i]) * (float)P1[4 * g + i];
          }
        }
        if (DUMP) {
#pragma unroll
          for (int j = 0; j < 16; ++j) {
            const int row = m0 + rowb + 8 * (j >> 2) + (j & 3);
            if (row < M && n0 + col0 < N) dump[((size_t)row * N + n0 + col0) * nbw + 8 * kb + c] = P0[j];
            if (row < M && n0 + col1 < N) dump[((size_t)row * N + n0 + col1) * nbw + 8 * kb + c] = P1[j];
          }
        }
      }
      continue;
    }

    int is0[16], is1[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) is0[j] = is1[j] = 0;

    if constexpr (FMT == kFmtQ4K) {
      const uint2 sc0 = *reinterpret_cast<const uint2*>(L.bsc + 16 * col0);
      const uint2 sc1 = *reinterpret_cast<const uint2*>(L.bsc + 16 * col1);
#pragma unroll 1
      for (int c = 0; c < 8; ++c) {
        const i8x16 a = *reinterpret_cast<const i8x16*>(arow + 32 * c);
        const i32x16 P0 = mfma_i8(a, *reinterpret_cast<const i8x16*>(b0row + 32 * c), zero);
        const i32x16 P1 = mfma_i8(a, *reinterpret_cast<const i8x16*>(b1row + 32 * c), zero);
        const int s0 = (int)byte8(sc0, c), s1 = (int)byte8(sc1, c);
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          is0[j] += __mul24(s0, P0[j]);  // |P| < 2^23: full-rate 24-bit multiply
          is1[j] += __mul24(s1, P1[j]);
        }
      }
      // mins: sum_j m_j * (32-element sum)_j as two zero-padded MFMAs
      const uint4 sv = *reinterpret_cast<const uint4*>(L.as + 16 * (32 * wm + r));
      const uint4 zero4 = make_uint4(0, 0, 0, 0);
      const i8x16 alo = as_i8x16(h == 0 ? make_uint4(sv.x, sv.y, 0, 0) : zero4);
      const i8x16 ahi = as_i8x16(h == 0 ? make_uint4(sv.z, sv.w, 0, 0) : zero4);
      const uint2 mn0 = *reinterpret_cast<const uint2*>(L.bsc + 16 * col0 + 8);
      const uint2 mn1 = *reinterpret_cast<const uint2*>(L.bsc + 16 * col1 + 8);
      const i8x16 bm0 = as_i8x16(h == 0 ? make_uint4(mn0.x, mn0.y, 0, 0) : zero4);
      const i8x16 bm1 = as_i8x16(h == 0 ? make_uint4(mn1.x, mn1.y, 0, 0) : zero4);
      const i32x16 L0 = mfma_i8(alo, bm0, zero), H0 = mfma_i8(ahi, bm0, zero);
      const i32x16 L1 = mfma_i8(alo, bm1, zero), H1 = mfma_i8(ahi, bm1, zero);
      const float dw0 = L.bd[8 * col0], dm0 = L.bd[8 * col0 + 1];
      const float dw1 = L.bd[8 * col1], dm1 = L.bd[8 * col1 + 1];
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const float4 dx = *reinterpret_cast<const float4*>(&L.ad[rowb + 8 * g]);
        const float dxs[4] = {dx.x, dx.y, dx.z, dx.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int j = 4 * g + i;
          const int im0 = H0[j] * 64 + L0[j], im1 = H1[j] * 64 + L1[j];
          acc0[j] += dxs[i] * (dw0 * (float)is0[j] - dm0 * (float)im0);
          acc1[j] += dxs[i] * (dw1 * (float)is1[j] - dm1 * (float)im1);
          if (DUMP) {
            const int row = m0 + rowb + 8 * g + i;
            if (row < M && n0 + col0 < N) {
              const size_t o = ((size_t)row * N + n0 + col0) * nbk + kb;
              dump[2 * o] = is0[j];
              dump[2 * o + 1] = im0;
            }
            if (row < M && n0 + col1 < N) {
              const size_t o = ((size_t)row * N + n0 + col1) * nbk + kb;
              dump[2 * o] = is1[j];
              dump[2 * o + 1] = im1;
            }
          }
        }
      }
    } else {  // Q6_K: groups of 16 with their own scale; one MFMA per group (other half masked)
      const uint4 sc0 = *reinterpret_cast<const uint4*>(L.bsc + 16 * col0);
      const uint4 sc1 = *reinterpret_cast<const uint4*>(L.bsc + 16 * col1);
      const uint4 zero4 = make_uint4(0, 0, 0, 0);
#pragma unroll 1
      for (int c = 0; c < 8; ++c) {
        const uint4 av = *reinterpret_cast<const uint4*>(arow + 32 * c);
        const i8x16 alo = as_i8x16(h == 0 ? av : zero4), ahi = as_i8x16(h == 1 ? av : zero4);
        const i8x16 b0 = *reinterpret_cast<const i8x16*>(b0row + 32 * c);
        const i8x16 b1 = *reinterpret_cast<const i8x16*>(b1row + 32 * c);
        const i32x16 P00 = mfma_i8(alo, b0, zero), P01 = mfma_i8(ahi, b0, zero);
        const i32x16 P10 = mfma_i8(alo, b1, zero), P11 = mfma_i8(ahi, b1, zero);
        const uint32_t w0 = (c < 2 ? sc0.x : c < 4 ? sc0.y : c < 6 ? sc0.z : sc0.w) >> (16 * (c & 1));
        const uint32_t w1 = (c < 2 ? sc1.x : c < 4 ? sc1.y : c < 6 ? sc1.z : sc1.w) >> (16 * (c & 1));
        const int s00 = (int)(int8_t)(w0 & 0xff), s01 = (int)(int8_t)((w0 >> 8) & 0xff);
        const int s10 = (int)(int8_t)(w1 & 0xff), s11 = (int)(int8_t)((w1 >> 8) & 0xff);
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          is0[j] += __mul24(s00, P00[j]) + __mul24(s01, P01[j]);
          is1[j] += __mul24(s10, P10[j]) + __mul24(s11, P11[j]);
        }
      }
      const float dw0 = L.bd[8 * col0], dw1 = L.bd[8 * col1];
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const float4 dx = *reinterpret_cast<const float4*>(&L.ad[rowb + 8 * g]);
        const float dxs[4] = {dx.x, dx.y, dx.z, dx.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int j = 4 * g + i;
          acc0[j] += dxs[i] * (dw0 * (float)is0[j]);
          acc1[j] += dxs[i] * (dw1 * (float)is1[j]);
          if (DUMP) {
            const int row = m0 + rowb + 8 * g + i;
            if (row < M && n0 + col0 < N) dump[((size_t)row * N + n0 + col0) * nbk + kb] = is0[j];
            if (row < M && n0 + col1 < N) dump[((size_t)row * N + n0 + col1) * nbk + kb] = is1[j];
          }
        }
      }
    }
  }
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const int row = m0 + rowb + 8 * (j >> 2) + (j & 3);
    if (row < M && n0 + col0 < N) {
      float* yp = y + (size_t)row * ldy + n0 + col0;
      *yp = accumulate ? *yp + acc0[j] : acc0[j];
    }
    if (row < M && n0 + col1 < N) {
      float* yp = y + (size_t)row * ldy + n0 + col1;
      *yp = accumulate ? *yp + acc1[j] : acc1[j];
    }
  }
}

}  // namespace qmm

// Activation quantizers writing the GEMM's plane layout.
//   Q8_K: q8 int8 [m][k], d f32 [m][k/256], 32-element sums int16 [m][k/256][8]
namespace qmm {
// One wave's Q8_K block w (row w / nb, block w % nb) in the plane layout.
__device__ __forceinline__ void put_q8k_plane(const Q8KLane& q, long long w, int nb, int k, int8_t* __restrict__ q8,
                                              float* __restrict__ d, int16_t* __restrict__ s, int lane) {
  const int row = (int)(w / nb), b = (int)(w % nb);
  reinterpret_cast<uint32_t*>(q8 + (size_t)row * k + 256 * b)[lane] = q.packed;
  const int next = __shfl_down(q.sum16, 4);
  if ((lane & 7) == 0) s[w * 8 + (lane >> 3)] = (int16_t)(q.sum16 + next);
  if (lane == 0) d[w] = q.d;
}
}  // namespace qmm

extern "C" __global__ void __launch_bounds__(256) qmm_quantize_q8k_mmq(const float* __restrict__ x, long long ldx,
                                                                       int8_t* __restrict__ q8,
                                                                       float* __restrict__ d,
                                                                       int16_t* __restrict__ s, int k, int m) {
  const int nb = k / 256;
  const long long w = (long long)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (w >= (long long)m * nb) return;
  const int row = (int)(w / nb), b = (int)(w % nb), lane = threadIdx.x & 63;
  qmm::put_q8k_plane(qmm::q8k_lane(x + row * ldx + 256LL * b, lane), w, nb, k, q8, d, s, lane);
}

// The same planes for gathered rows: plane row i = x[rows[i]] (the grouped
// prefill's expert-ordered pairs, without a gathered f32 copy).
extern "C" __global__ void __launch_bounds__(256) qmm_quantize_q8k_mmq_rows(const float* __restrict__ x,
                                                                            long long ldx,
                                                                            const int* __restrict__ rows,
                                                                            int8_t* __restrict__ q8,
                                                                            float* __restrict__ d,
                                                                            int16_t* __restrict__ s, int k, int m) {
  const int nb = k / 256;
  const long long w = (long long)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (w >= (long long)m * nb) return;
  const int row = (int)(w / nb), b = (int)(w % nb), lane = threadIdx.x & 63;
  qmm::put_q8k_plane(qmm::q8k_lane(x + (long long)rows[row] * ldx + 256LL * b, lane), w, nb, k, q8, d, s, lane);
}

// The same planes for RMSNorm rows, x / sqrt(mean(x^2) + eps) * w, with
// qmm_rms_norm's values bit for bit: 1024 threads stage the row in LDS (k
// floats of dynamic LDS; at k = 4096 one load per thread, all in flight at
// once), then threads 0..255 form qmm_rms_norm's sum of squares in its order
// (thread t over t, t + 256, ... in turn, wave_sum, the four wave sums in
// order), every thread normalises its own elements, and each of the 16
// waves quantizes whole 256-element blocks (one at k = 4096): the planes of
// quantizing qmm_rms_norm's output, without its f32 copy or a launch.
extern "C" __global__ void __launch_bounds__(1024) qmm_rms_norm_q8k_mmq(const float* __restrict__ x, long long ldx,
                                                                        const float* __restrict__ w, float eps,
                                                                        int k, int8_t* __restrict__ q8,
                                                                        float* __restrict__ d,
                                                                        int16_t* __restrict__ s) {
#pragma clang fp contract(off)
  constexpr int NT = 1024, NS = 256;  // threads; the threads of qmm_rms_norm's sum
  extern __shared__ __attribute__((aligned(16))) float rowbuf[];
  __shared__ float red[NS / 64];
  const float* xr = x + blockIdx.x * ldx;
  const int t = threadIdx.x;
  for (int i0 = 4 * t; i0 < k; i0 += 4 * NT)  // k is a multiple of 256; rows need only 4-byte alignment
    *reinterpret_cast<float4*>(rowbuf + i0) = make_float4(xr[i0], xr[i0 + 1], xr[i0 + 2], xr[i0 + 3]);
  __syncthreads();
  if (t < NS) {
    float ss = 0.0f;
    for (int i = t; i < k; i += NS) ss += rowbuf[i] * rowbuf[i];
    ss = qmm::wave_sum(ss);
    if ((t & 63) == 0) red[t >> 6] = ss;
  }
  __syncthreads();
  float tot = 0.0f;
#pragma unroll
  for (int i = 0; i < NS / 64; ++i) tot += red[i];
  const float den = sqrtf(tot / (float)k + eps);
  for (int i0 = 4 * t; i0 < k; i0 += 4 * NT) {
    float4 v = *reinterpret_cast<const float4*>(rowbuf + i0);
    const float4 g = make_float4(w[i0], w[i0 + 1], w[i0 + 2], w[i0 + 3]);
    v.x = v.x / den * g.x;
    v.y = v.y / den * g.y;
    v.z = v.z / den * g.z;
    v.w = v.w / den * g.w;
    *reinterpret_cast<float4*>(rowbuf + i0) = v;
  }
  __syncthreads();
  const int nb = k / 256, lane = t & 63;
  for (int b = t >> 6; b < nb; b += NT / 64) {
    const float4 e = *reinterpret_cast<const float4*>(rowbuf + 256 * b + 4 * lane);
    qmm::put_q8k_plane(qmm::q8k_lane_vals(e.x, e.y, e.z, e.w, lane), (long long)blockIdx.x * nb + b, nb, k, q8, d, s,
                       lane);
  }
}

// The same planes for silu(g) * u (rows of k, row stride ld): the f32 values
// of qmm_silu_mul, quantized in registers.
extern "C" __global__ void __launch_bounds__(256) qmm_silu_mul_q8k_mmq(const float* __restrict__ g,
                                                                       const float* __restrict__ u, long long ld,
                                                                       int8_t* __restrict__ q8,
                                                                       float* __restrict__ d,
                                                                       int16_t* __restrict__ s, int k, int m) {
#pragma clang fp contract(off)
  const int nb = k / 256;
  const long long w = (long long)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (w >= (long long)m * nb) return;
  const int row = (int)(w / nb), b = (int)(w % nb), lane = threadIdx.x & 63;
  const long long o = row * ld + 256LL * b + 4 * lane;
  float e[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) e[j] = qmm::silu_mul(g[o + j], u[o + j]);
  qmm::put_q8k_plane(qmm::q8k_lane_vals(e[0], e[1], e[2], e[3], lane), w, nb, k, q8, d, s, lane);
}

// The same planes from the gate and up GEMMs' unsummed split-K partials
// (gp [gsplits][m][k], up [usplits][m][k]; one split is the plain output):
// each value is summed in split order as qmm_splitk_sum sums it, so the
// planes equal split sums, then qmm_silu_mul, then the quantizer, with three
// launches fewer.
extern "C" __global__ void __launch_bounds__(256) qmm_splitk_silu_mul_q8k_mmq(const float* __restrict__ gp, int gsplits,
                                                                              const float* __restrict__ up, int usplits,
                                                                              int8_t* __restrict__ q8,
                                                                              float* __restrict__ d,
                                                                              int16_t* __restrict__ s, int k, int m) {
#pragma clang fp contract(off)
  const int nb = k / 256;
  const long long w = (long long)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (w >= (long long)m * nb) return;
  const int row = (int)(w / nb), b = (int)(w % nb), lane = threadIdx.x & 63;
  const long long o = (long long)row * k + 256LL * b + 4 * lane;
  const size_t plane = (size_t)m * k;
  float4 g = *reinterpret_cast<const float4*>(gp + o);
  for (int j = 1; j < gsplits; ++j) {
    const float4 v = *reinterpret_cast<const float4*>(gp + o + j * plane);
    g.x += v.x;
    g.y += v.y;
    g.z += v.z;
    g.w += v.w;
  }
  float4 u = *reinterpret_cast<const float4*>(up + o);
  for (int j = 1; j < usplits; ++j) {
    const float4 v = *reinterpret_cast<const float4*>(up + o + j * plane);
    u.x += v.x;
    u.y += v.y;
    u.z += v.z;
    u.w += v.w;
  }
  qmm::put_q8k_plane(qmm::q8k_lane_vals(qmm::silu_mul(g.x, u.x), qmm::silu_mul(g.y, u.y), qmm::silu_mul(g.z, u.z),
                                        qmm::silu_mul(g.w, u.w), lane),
                     w, nb, k, q8, d, s, lane);
}

//   Q8_0: q8 int8 [m][k], d f32 [m][k/32] (the f16-rounded block scale)
extern "C" __global__ void __launch_bounds__(256) qmm_quantize_q8_0_mmq(const float* __restrict__ x, long long ldx,
                                                                        int8_t* __restrict__ q8,
                                                                        float* __restrict__ d, int k, int m) {
  const int nb = k / 32;
  const long long t = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  const long long blk = t >> 3;
  const bool valid = blk < (long long)m * nb;
  const long long bc = valid ? blk : 0;
  const int row = (int)(bc / nb), b = (int)(bc % nb), l = (int)(t & 7);
  uint8_t tmp[qmm::kQ80Bytes];
  qmm::q80_block(x + row * ldx + 32LL * b, tmp, l, valid);
  if (!valid) return;
  const uint16_t* p = reinterpret_cast<const uint16_t*>(tmp);
  reinterpret_cast<uint16_t*>(q8 + (size_t)row * k + 32 * b)[2 * l] = p[1 + 2 * l];
  reinterpret_cast<uint16_t*>(q8 + (size_t)row * k + 32 * b)[2 * l + 1] = p[2 + 2 * l];
  if (l == 0) d[bc] = qmm::h2f(p[0]);
}

#define QMM_MMQ_KERNEL(FMT, NAME)                                                                            \
  extern "C" __global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))               \
      qmm_mmq_##NAME(const uint8_t* __restrict__ wq, const int8_t* __restrict__ xq,                          \
                     const float* __restrict__ xd, const int16_t* __restrict__ xs, float* __restrict__ y,   \
                     int M, int N, int K, int ldy, int* __restrict__ dump, int accumulate, int remap,       \
                     int kc, long long ysplit) {                                                             \
    const qmm::KRange kr = qmm::split_range(K, kc);                                                          \
    qmm::mmq<FMT, false>(wq, qmm::split_scales<FMT>(wq, N, K), xq, xd, xs, y + blockIdx.z * ysplit, M, N, K,  \
                         ldy, dump, accumulate, remap, kr.kb0, kr.kb1);                                       \
  }                                                                                                          \
  extern "C" __global__ void __launch_bounds__(256)                                                          \
      qmm_mmq_##NAME##_dump(const uint8_t* __restrict__ wq, const int8_t* __restrict__ xq,                   \
                            const float* __restrict__ xd, const int16_t* __restrict__ xs,                    \
                            float* __restrict__ y, int M, int N, int K, int ldy, int* __restrict__ dump,     \
                            int accumulate, int remap, int kc, long long ysplit) {                           \
    const qmm::KRange kr = qmm::split_range(K, kc);                                                          \
    qmm::mmq<FMT, true>(wq, qmm::split_scales<FMT>(wq, N, K), xq, xd, xs, y + blockIdx.z * ysplit, M, N, K,   \
                        ldy, dump, accumulate, remap, kr.kb0, kr.kb1);                                        \
  }

QMM_MMQ_KERNEL(qmm::kFmtQ4K, q4k)
QMM_MMQ_KERNEL(qmm::kFmtQ6K, q6k)
QMM_MMQ_KERNEL(qmm::kFmtQ80, q8_0)

// GGML activation blocks (m rows of Q8_K / Q8_0) -> the GEMM plane layout.
// Q8_K: one wave per block; Q8_0: one thread per block.
extern "C" __global__ void __launch_bounds__(256) qmm_q8_blocks_to_planes(const uint8_t* __restrict__ xq,
                                                                          int8_t* __restrict__ q8,
                                                                          float* __restrict__ d,
                                                                          int16_t* __restrict__ s, int k, int m,
                                                                          int is_q8k) {
  if (is_q8k) {
    const int nb = k / 256;
    const long long w = (long long)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (w >= (long long)m * nb) return;
    const int row = (int)(w / nb), b = (int)(w % nb), lane = threadIdx.x & 63;
    const uint8_t* blk = xq + w * qmm::kQ8KBytes;
    reinterpret_cast<uint32_t*>(q8 + (size_t)row * k + 256 * b)[lane] = reinterpret_cast<const uint32_t*>(blk + 4)[lane];
    if (lane < 8) {
      const int16_t* bs = reinterpret_cast<const int16_t*>(blk + 4 + 256);
      s[w * 8 + lane] = (int16_t)(bs[2 * lane] + bs[2 * lane + 1]);
    }
    if (lane == 0) d[w] = *reinterpret_cast<const float*>(blk);
  } else {
    const int nb = k / 32;
    const long long b = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= (long long)m * nb) return;
    const int row = (int)(b / nb), bb = (int)(b % nb);
    const uint16_t* src = reinterpret_cast<const uint16_t*>(xq + b * qmm::kQ80Bytes);
    uint16_t* dst = reinterpret_cast<uint16_t*>(q8 + (size_t)row * k + 32 * bb);
    for (int i = 0; i < 16; ++i) dst[i] = src[1 + i];
    d[b] = qmm::h2f(src[0]);
  }
}

// ---------------------------------------------------------------------------
// Q4_K prefill GEMM, second generation: larger tiles, raw weight blocks in LDS.
//   * workgroup tile BM (64 or 128) rows x BN (64 or 128) columns; waves of
//     64 x 32 outputs (two v_mfma_i32_32x32x32_i8 tiles), BM/64 x BN/32 of
//     them; 64-row tiles keep a workgroup's LDS small enough for two per CU,
//     so one workgroup's MFMAs cover the other's loads;
//   * per 256-wide K step the activation rows (int8 planes) and the weight
//     columns' Q4_K blocks are copied to LDS unchanged (double-buffered, the
//     next step's global loads in flight during this step's MFMAs); a lane's
//     16-byte read of a block's quants yields the B operands of two
//     sub-blocks (low and high nibbles), and the scales/mins of all eight
//     sub-blocks are unpacked byte-parallel from the block header;
//   * per sub-block j: P = MFMA(x, q4) and isd += sc_j * P (24-bit); the mins
//     term ism = sum_j m_j * (32-sums)_j is two zero-padded MFMAs (sums split
//     into a 6-bit low byte and a signed high byte); then
//     y += dx * (d * isd - dmin * ism) once per step.
// The integer block dots are the same as mmq()'s (DUMP writes them).
// ---------------------------------------------------------------------------
namespace qmm {

constexpr int kM2AStride = 256 + 16;  // activation row in LDS (16-byte skew)
// Weight blocks in LDS at their own 144 B (9 x 16 B): an odd number of
// 16-byte units, so the 16 lanes of a ds_read_b128 pass (one block each) land
// on 16 distinct 4-bank groups, and the staging stores are contiguous.
constexpr int kM2BStride = 144;

// NT = threads of the workgroup (mmq2: one wave per 64 x 32 outputs).
template <int BM, int BN, int NT = 64 * (BM / 64) * (BN / 32)>
struct M2 {
  static constexpr int kWM = BM / 64, kWN = BN / 32;  // mmq2's waves along M and N
  static constexpr int kThreads = NT;
  static constexpr int kA = BM * kM2AStride;
  static constexpr int kB = BN * kM2BStride;
  static constexpr int kDx = BM * 4;
  static constexpr int kSum = BM * 16;
  static constexpr int kStage = kA + kB + kDx + kSum;  // bytes of one buffer
  static constexpr int kBytes = 2 * kStage;
  static constexpr int kAPer = BM * 16 / kThreads;                  // activation uint4 per thread
  static constexpr int kBPer = (BN * 9 + kThreads - 1) / kThreads;  // weight uint4 per thread
  static_assert(BM * 16 % kThreads == 0 && BM <= kThreads, "tile / thread count");
};

// Global loads of one K step into registers.
template <int BM, int BN, int NT = M2<BM, BN>::kThreads>
struct M2Regs {
  uint4 a[M2<BM, BN, NT>::kAPer];
  uint4 b[M2<BM, BN, NT>::kBPer];
  float dx;  // t < BM: activation scale of row t
  uint4 s;   // t < BM: eight int16 32-element sums of row t
};

template <int BM, int BN, int NT = M2<BM, BN>::kThreads>
__device__ __forceinline__ void m2_load(M2Regs<BM, BN, NT>& R, const int8_t* __restrict__ xq, const float* __restrict__ xd,
                                        const int16_t* __restrict__ xs, const uint8_t* __restrict__ wq, int M, int N,
                                        int K, int m0, int n0, int kb) {
  using C = M2<BM, BN, NT>;
  const int t = threadIdx.x, nbk = K / 256;
#pragma unroll
  for (int u = 0; u < C::kAPer; ++u) {
    const int idx = t + C::kThreads * u, row = m0 + (idx >> 4);
    const bool ok = row < M;
    R.a[u] = ok ? reinterpret_cast<const uint4*>(xq + (size_t)row * K + 256 * kb)[idx & 15] : make_uint4(0, 0, 0, 0);
  }
#pragma unroll
  for (int u = 0; u < C::kBPer; ++u) {
    const int idx = t + C::kThreads * u, col = idx / 9, piece = idx % 9;
    R.b[u] = make_uint4(0, 0, 0, 0);
    if (idx < BN * 9 && n0 + col < N)
      R.b[u] = reinterpret_cast<const uint4*>(wq + ((size_t)(n0 + col) * nbk + kb) * kQ4KBytes)[piece];
  }
  if (t < BM) {
    const int row = m0 + t;
    const bool ok = row < M;
    R.dx = ok ? xd[(size_t)row * nbk + kb] : 0.0f;
    R.s = ok ? *reinterpret_cast<const uint4*>(xs + ((size_t)row * nbk + kb) * 8) : make_uint4(0, 0, 0, 0);
  }
}

template <int BM, int BN, int NT = M2<BM, BN>::kThreads>
__device__ __forceinline__ void m2_store(const M2Regs<BM, BN, NT>& R, uint8_t* buf) {
  using C = M2<BM, BN, NT>;
  const int t = threadIdx.x;
#pragma unroll
  for (int u = 0; u < C::kAPer; ++u) {
    const int idx = t + C::kThreads * u;
    *reinterpret_cast<uint4*>(buf + (idx >> 4) * kM2AStride + 16 * (idx & 15)) = R.a[u];
  }
#pragma unroll
  for (int u = 0; u < C::kBPer; ++u) {
    const int idx = t + C::kThreads * u, col = idx / 9, piece = idx % 9;
    if (idx < BN * 9) *reinterpret_cast<uint4*>(buf + C::kA + col * kM2BStride + 16 * piece) = R.b[u];
  }
  if (t < BM) {
    reinterpret_cast<float*>(buf + C::kA + C::kB)[t] = R.dx;
    // 32-element sums s (|s| <= 4096) as s = 64 * hi + lo: lo in [0, 63], hi in [-64, 64]
    const int16_t* sv = reinterpret_cast<const int16_t*>(&R.s);
    uint32_t lo[2] = {0, 0}, hi[2] = {0, 0};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int v = sv[j];
      lo[j >> 2] |= (uint32_t)(v & 63) << (8 * (j & 3));
      hi[j >> 2] |= (uint32_t)((v >> 6) & 0xff) << (8 * (j & 3));
    }
    *reinterpret_cast<uint4*>(buf + C::kA + C::kB + C::kDx + 16 * t) = make_uint4(lo[0], lo[1], hi[0], hi[1]);
  }
}

template <int BM, int BN, bool DUMP>
__device__ __forceinline__ void mmq2_q4k(const uint8_t* __restrict__ wq, const int8_t* __restrict__ xq,
                                         const float* __restrict__ xd, const int16_t* __restrict__ xs,
                                         float* __restrict__ y, int M, int N, int K, int ldy, int* __restrict__ dump,
                                         int accumulate, int remap, int kb0, int kb1) {
  using C = M2<BM, BN>;
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  int mt, nt;
  gemm_tile(remap, mt, nt);
  const int m0 = mt * BM, n0 = nt * BN;
  const int nbk = K / 256;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 31, h = lane >> 5;
  const int wm = wave % C::kWM, wn = wave / C::kWM;
  const int arow0 = 64 * wm + r;  // + 32 i: A operand row of tile i
  const int bcol = 32 * wn + r;   // B operand column within the workgroup tile
  const int col = n0 + bcol;      // this lane's output column

  i32x16 zero;
#pragma unroll
  for (int j = 0; j < 16; ++j) zero[j] = 0;
  float acc[2][16];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 16; ++j) acc[i][j] = 0.0f;

  M2Regs<BM, BN> R;
  m2_load<BM, BN>(R, xq, xd, xs, wq, M, N, K, m0, n0, kb0);
  m2_store<BM, BN>(R, lds);
  __syncthreads();
  for (int kb = kb0; kb < kb1; ++kb) {
    uint8_t* buf = lds + ((kb - kb0) & 1) * C::kStage;
    if (kb + 1 < kb1) m2_load<BM, BN>(R, xq, xd, xs, wq, M, N, K, m0, n0, kb + 1);
    const int8_t* A = reinterpret_cast<const int8_t*>(buf);
    const uint8_t* Bc = buf + C::kA + bcol * kM2BStride;  // this lane's weight block
    const float* DX = reinterpret_cast<const float*>(buf + C::kA + C::kB);
    const uint8_t* SUM = buf + C::kA + C::kB + C::kDx;

    // scales / mins of the lane's column: byte j of (lo, hi) is sub-block j
    const uint4 hd = *reinterpret_cast<const uint4*>(Bc);
    const float dw = h2f(hd.x), dm = h2f(hd.x >> 16);
    const uint32_t sclo = hd.y & 0x3f3f3f3fu, schi = (hd.w & 0x0f0f0f0fu) | ((hd.y >> 2) & 0x30303030u);
    const uint32_t mnlo = hd.z & 0x3f3f3f3fu, mnhi = ((hd.w >> 4) & 0x0f0f0f0fu) | ((hd.z >> 2) & 0x30303030u);

    int isd[2][16];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 16; ++j) isd[i][j] = 0;
#pragma unroll 1
    for (int c2 = 0; c2 < 4; ++c2) {
      const uint4 qv = *reinterpret_cast<const uint4*>(Bc + 16 + 32 * c2 + 16 * h);
      const uint4 blo = make_uint4(qv.x & 0x0f0f0f0fu, qv.y & 0x0f0f0f0fu, qv.z & 0x0f0f0f0fu, qv.w & 0x0f0f0f0fu);
      const uint4 bhi = make_uint4((qv.x >> 4) & 0x0f0f0f0fu, (qv.y >> 4) & 0x0f0f0f0fu, (qv.z >> 4) & 0x0f0f0f0fu,
                                   (qv.w >> 4) & 0x0f0f0f0fu);
      const uint32_t scw = c2 < 2 ? sclo : schi;
      const int s0 = (int)((scw >> (16 * (c2 & 1))) & 0xffu), s1 = (int)((scw >> (16 * (c2 & 1) + 8)) & 0xffu);
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int8_t* ar = A + (arow0 + 32 * i) * kM2AStride + 64 * c2 + 16 * h;
        const i32x16 P0 = mfma_i8(*reinterpret_cast<const i8x16*>(ar), as_i8x16(blo), zero);
        const i32x16 P1 = mfma_i8(*reinterpret_cast<const i8x16*>(ar + 32), as_i8x16(bhi), zero);
#pragma unroll
        for (int e = 0; e < 16; ++e) isd[i][e] += __mul24(s0, P0[e]) + __mul24(s1, P1[e]);  // |P| < 2^23
      }
    }
    // mins term and the float update
    const uint4 zero4 = make_uint4(0, 0, 0, 0);
    const i8x16 bm = as_i8x16(h == 0 ? make_uint4(mnlo, mnhi, 0, 0) : zero4);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const uint4 sv = *reinterpret_cast<const uint4*>(SUM + 16 * (arow0 + 32 * i));
      const i8x16 alo = as_i8x16(h == 0 ? make_uint4(sv.x, sv.y, 0, 0) : zero4);
      const i8x16 ahi = as_i8x16(h == 0 ? make_uint4(sv.z, sv.w, 0, 0) : zero4);
      const i32x16 Lo = mfma_i8(alo, bm, zero), Hi = mfma_i8(ahi, bm, zero);
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const float4 dx = *reinterpret_cast<const float4*>(DX + 64 * wm + 32 * i + 8 * g + 4 * h);
        const float dxs[4] = {dx.x, dx.y, dx.z, dx.w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int e = 4 * g + q;
          const int ism = Hi[e] * 64 + Lo[e];
          acc[i][e] += dxs[q] * (dw * (float)isd[i][e] - dm * (float)ism);
          if (DUMP) {
            const int row = m0 + 64 * wm + 32 * i + 8 * g + 4 * h + q;
            if (row < M && col < N) {
              const size_t o = ((size_t)row * N + col) * nbk + kb;
              dump[2 * o] = isd[i][e];
              dump[2 * o + 1] = ism;
            }
          }
        }
      }
    }
    if (kb + 1 < kb1) m2_store<BM, BN>(R, lds + ((kb + 1 - kb0) & 1) * C::kStage);
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int row = m0 + 64 * wm + 32 * i + 8 * (e >> 2) + 4 * h + (e & 3);
      if (row < M && col < N) {
        float* yp = y + (size_t)row * ldy + col;
        *yp = accumulate ? *yp + acc[i][e] : acc[i][e];
      }
    }
}

// ---------------------------------------------------------------------------
// Q4_K prefill GEMM, split-scale form (mmq4): the sub-block scales move into
// the MFMA operands, so a super-block's contraction accumulates inside the
// matrix cores instead of one VALU scale-and-add per sub-block and output.
//   * each 6-bit scale is split as sc = 8 * sh + sl (sh, sl in [0, 7]); the
//     weight operand of sub-block j is taken twice, as sl_j * q4 and
//     sh_j * q4 (both <= 105: still int8), and
//       isd = sum_j sc_j (q8 . q4)_j = MFMA_acc(x, sl q4) + 8 MFMA_acc(x, sh q4)
//     exactly in int32 (|isd| <= 63 * 15 * 127 * 256 < 2^31); the per-byte
//     products are one packed 16-bit multiply per dword (q * s < 256, so no
//     carry crosses a byte);
//   * workgroup tile 128 x BN with four waves, one per SIMD, each owning
//     64 x BN/2 outputs (two M tiles x BN/64 N tiles of 32 x 32): a wave has
//     the whole register file, so the 2 x 2 x BN/64 accumulators, the f32
//     outputs and the next step's global loads fit without spilling, and
//     its MFMAs overlap its own VALU work;
//   * staging (double-buffered LDS, next step's loads in registers during
//     this step's MFMAs), the mins term (two zero-padded MFMAs) and the f32
//     update y += dx * (d * isd - dmin * ism) are mmq2's, so the integer
//     block dots are the same (DUMP writes them).
// ---------------------------------------------------------------------------
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

// Bytes of v times s (each product < 256): one packed 16-bit multiply.
__device__ __forceinline__ uint32_t bytes_times(uint32_t v, uint32_t s) {
  const u16x2 a = __builtin_bit_cast(u16x2, v);
  const u16x2 b = {(unsigned short)s, (unsigned short)s};
  return __builtin_bit_cast(uint32_t, a * b);
}
__device__ __forceinline__ i8x16 bytes_times4(uint4 v, uint32_t s) {
  return as_i8x16(make_uint4(bytes_times(v.x, s), bytes_times(v.y, s), bytes_times(v.z, s), bytes_times(v.w, s)));
}

template <int BN, bool DUMP>
__device__ __forceinline__ void mmq4_q4k(const uint8_t* __restrict__ wq, const int8_t* __restrict__ xq,
                                         const float* __restrict__ xd, const int16_t* __restrict__ xs,
                                         float* __restrict__ y, int M, int N, int K, int ldy, int* __restrict__ dump,
                                         int accumulate, int remap, int kb0, int kb1) {
  constexpr int BM = 128, NT = 256;
  constexpr int TN = BN / 64;  // N tiles per wave
  using C = M2<BM, BN, NT>;
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  int mt, nt;
  gemm_tile(remap, mt, nt);
  const int m0 = mt * BM, n0 = nt * BN;
  const int nbk = K / 256;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 31, h = lane >> 5;
  const int wm = wave & 1, wn = wave >> 1;
  const int arow0 = 64 * wm + r;  // + 32 i: A operand row of M tile i

  i32x16 zero;
#pragma unroll
  for (int j = 0; j < 16; ++j) zero[j] = 0;
  float acc[2][TN][16];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int t = 0; t < TN; ++t)
#pragma unroll
      for (int j = 0; j < 16; ++j) acc[i][t][j] = 0.0f;

  M2Regs<BM, BN, NT> R;
  m2_load<BM, BN, NT>(R, xq, xd, xs, wq, M, N, K, m0, n0, kb0);
  m2_store<BM, BN, NT>(R, lds);
  __syncthreads();
  // one K step from LDS buffer `buf` (the next step's loads are in flight)
  auto step = [&](const uint8_t* buf, int kb) {
    const int8_t* A = reinterpret_cast<const int8_t*>(buf);
    const float* DX = reinterpret_cast<const float*>(buf + C::kA + C::kB);
    const uint8_t* SUM = buf + C::kA + C::kB + C::kDx;

    // per N tile: this lane's column block, its scales (split) and mins
    const uint8_t* Bc[TN];
    float dw[TN], dm[TN];
    uint32_t sl[TN][2], sh[TN][2], mn[TN][2];
#pragma unroll
    for (int t = 0; t < TN; ++t) {
      Bc[t] = buf + C::kA + (BN / 2 * wn + 32 * t + r) * kM2BStride;
      const uint4 hd = *reinterpret_cast<const uint4*>(Bc[t]);
      dw[t] = h2f(hd.x);
      dm[t] = h2f(hd.x >> 16);
      const uint32_t sclo = hd.y & 0x3f3f3f3fu, schi = (hd.w & 0x0f0f0f0fu) | ((hd.y >> 2) & 0x30303030u);
      sl[t][0] = sclo & 0x07070707u;
      sl[t][1] = schi & 0x07070707u;
      sh[t][0] = (sclo >> 3) & 0x07070707u;
      sh[t][1] = (schi >> 3) & 0x07070707u;
      mn[t][0] = hd.z & 0x3f3f3f3fu;
      mn[t][1] = ((hd.w >> 4) & 0x0f0f0f0fu) | ((hd.z >> 2) & 0x30303030u);
    }
    i32x16 accl[2][TN], acch[2][TN];
#pragma unroll
    for (int c2 = 0; c2 < 4; ++c2) {
      const int sel = c2 >> 1, sb = 16 * (c2 & 1);
      i8x16 b0l[TN], b0h[TN], b1l[TN], b1h[TN];
#pragma unroll
      for (int t = 0; t < TN; ++t) {
        const uint4 qv = *reinterpret_cast<const uint4*>(Bc[t] + 16 + 32 * c2 + 16 * h);
        const uint4 blo = make_uint4(qv.x & 0x0f0f0f0fu, qv.y & 0x0f0f0f0fu, qv.z & 0x0f0f0f0fu, qv.w & 0x0f0f0f0fu);
        const uint4 bhi = make_uint4((qv.x >> 4) & 0x0f0f0f0fu, (qv.y >> 4) & 0x0f0f0f0fu,
                                     (qv.z >> 4) & 0x0f0f0f0fu, (qv.w >> 4) & 0x0f0f0f0fu);
        b0l[t] = bytes_times4(blo, (sl[t][sel] >> sb) & 0xffu);
        b0h[t] = bytes_times4(blo, (sh[t][sel] >> sb) & 0xffu);
        b1l[t] = bytes_times4(bhi, (sl[t][sel] >> (sb + 8)) & 0xffu);
        b1h[t] = bytes_times4(bhi, (sh[t][sel] >> (sb + 8)) & 0xffu);
      }
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int8_t* ar = A + (arow0 + 32 * i) * kM2AStride + 64 * c2 + 16 * h;
        const i8x16 a0 = *reinterpret_cast<const i8x16*>(ar);
        const i8x16 a1 = *reinterpret_cast<const i8x16*>(ar + 32);
#pragma unroll
        for (int t = 0; t < TN; ++t) {
          accl[i][t] = mfma_i8(a0, b0l[t], c2 == 0 ? zero : accl[i][t]);  // first: inline-zero accumulator
          acch[i][t] = mfma_i8(a0, b0h[t], c2 == 0 ? zero : acch[i][t]);
          accl[i][t] = mfma_i8(a1, b1l[t], accl[i][t]);
          acch[i][t] = mfma_i8(a1, b1h[t], acch[i][t]);
        }
      }
    }
    // mins term and the float update
    const uint4 zero4 = make_uint4(0, 0, 0, 0);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const uint4 sv = *reinterpret_cast<const uint4*>(SUM + 16 * (arow0 + 32 * i));
      const i8x16 alo = as_i8x16(h == 0 ? make_uint4(sv.x, sv.y, 0, 0) : zero4);
      const i8x16 ahi = as_i8x16(h == 0 ? make_uint4(sv.z, sv.w, 0, 0) : zero4);
#pragma unroll
      for (int t = 0; t < TN; ++t) {
        const i8x16 bm = as_i8x16(h == 0 ? make_uint4(mn[t][0], mn[t][1], 0, 0) : zero4);
        const i32x16 Lo = mfma_i8(alo, bm, zero), Hi = mfma_i8(ahi, bm, zero);
        const int col = n0 + BN / 2 * wn + 32 * t + r;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const float4 dx = *reinterpret_cast<const float4*>(DX + 64 * wm + 32 * i + 8 * g + 4 * h);
          const float dxs[4] = {dx.x, dx.y, dx.z, dx.w};
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int e = 4 * g + q;
            const int isd = accl[i][t][e] + 8 * acch[i][t][e];
            const int ism = Hi[e] * 64 + Lo[e];
            acc[i][t][e] += dxs[q] * (dw[t] * (float)isd - dm[t] * (float)ism);
            if (DUMP) {
              const int row = m0 + 64 * wm + 32 * i + 8 * g + 4 * h + q;
              if (row < M && col < N) {
                const size_t o = ((size_t)row * N + col) * nbk + kb;
                dump[2 * o] = isd;
                dump[2 * o + 1] = ism;
              }
            }
          }
        }
      }
    }
  };
  for (int kb = kb0; kb < kb1; ++kb) {
    if (kb + 1 < kb1) m2_load<BM, BN, NT>(R, xq, xd, xs, wq, M, N, K, m0, n0, kb + 1);
    step(lds + ((kb - kb0) & 1) * C::kStage, kb);
    if (kb + 1 < kb1) m2_store<BM, BN, NT>(R, lds + ((kb + 1 - kb0) & 1) * C::kStage);
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int t = 0; t < TN; ++t) {
      const int col = n0 + BN / 2 * wn + 32 * t + r;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int row = m0 + 64 * wm + 32 * i + 8 * (e >> 2) + 4 * h + (e & 3);
        if (row < M && col < N) {
          float* yp = y + (size_t)row * ldy + col;
          *yp = accumulate ? *yp + acc[i][t][e] : acc[i][t][e];
        }
      }
    }
}

// ---------------------------------------------------------------------------
// Q4_K prefill GEMM, split-scale with the mins term on bf16 matrix cores
// (mmqs). Per output and super-block the only VALU work left is one integer
// combine and one f32 multiply-add; everything else runs on MFMA:
//   * the d term exactly as mmq4: sc = 8 * sh + sl (both in [0, 7]), weight
//     operands sl * q4 and sh * q4 (int8, one packed 16-bit multiply per
//     dword), isd = MFMA_acc(x, sl q4) + 8 MFMA_acc(x, sh q4) in int32; then
//     acc += (dx * d) * isd once per super-block;
//   * the mins term sum_b dx * dmin * sum_j m_j S_j (S_j the 32-element sums of
//     the activation codes) is a dense product over (super-block, sub-block)
//     of A'[m][b, j] = dx * S_j and B'[b, j][n] = -dmin * m_j. Both factors
//     are formed in f32 while a K step is staged (B' exactly: an f16 times a
//     6-bit integer; A' rounded once) and split into three bf16 pieces each,
//     v = v1 + v2 + v3 exactly (8 + 8 + 8 significant bits). Three
//     v_mfma_f32_32x32x16_bf16 per tile and super-block, K-packed as
//     [a1 | a2] . [b1 | b1], [a1 | a2] . [b2 | b2] and [a1 | a3] . [b3 | b1],
//     accumulate every product of order <= 2 (a1b1, a2b1, a1b2, a2b2, a1b3,
//     a3b1) in f32 across all super-blocks, no per-step epilogue; the dropped
//     products are below 2^-24 of the term, so the mins term carries f32
//     rounding like the reference's own sum. (Two pieces, 16 of the 24 and 17
//     bits, left about 2^-16, which the near-cancellation of the d and mins
//     terms for zero-mean weights raised to ~1e-4 of an output's rms; f32
//     MFMAs, four per tile, cost 10% of the kernel time);
//   * workgroup tile 128 x 128, eight waves (two per SIMD, so one wave's
//     VALU epilogue and LDS waits overlap the other's MFMAs), two along M and
//     four along N; a wave owns 64 rows (two M tiles) x 32 columns, so a
//     column's operand products are formed once per K step for two tiles;
//     the mins MFMAs and the d-term multiply-adds share one f32 accumulator;
//   * staging: two LDS stages; the next step's activation rows and weight
//     quants go from global memory straight into the other stage
//     (global_load_lds, 16 bytes a lane, 1 KB a wave instruction: no
//     registers, no LDS store instructions) while this step computes. The
//     rows (256 bytes) and the quant runs (128 bytes) are unpadded; 16-byte
//     chunk c of row r sits at slot c ^ (r & 15), chunk k of column n at
//     slot k ^ ((n >> 1) & 7), so the MFMA operand reads of 32 rows or
//     columns at one chunk spread over all 64 banks (a 16-byte LDS read
//     serves 16 lanes at a time: columns n and n + 8 share a slot under
//     k ^ (n & 7) and their 128-byte runs the same bank half). Threads 0..127 load column t's block
//     header and form B' and the split-scale multipliers as packed 16-bit
//     pairs; threads 128..255 load row t - 128's scale and sums and form A'
//     (waves 0, 1 and 2, 3: the staging arithmetic lands on all four SIMDs,
//     wave w running on SIMD w % 4). A' / B' / multiplier rows sit at odd
//     multiples of 16 bytes (conflict-free 16-byte access).
// DUMP instantiations also compute ism exactly (two zero-padded int8 MFMAs)
// and write the integer block dots, which equal mmq2's.
// ---------------------------------------------------------------------------
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kSBM = 128, kSBN = 128;          // workgroup tile
constexpr int kSThreads = 512;                 // eight waves: two along M, four along N
constexpr int kSTM = 2;                        // M tiles (32 rows) per wave
constexpr int kSHalf = 48;                     // A' / B' row: bf16 v1[8] | v2[8] | v3[8] (odd 16-byte stride)
constexpr int kSOffBq = kSBM * 256;            // LDS: activation rows (swizzled chunks), then weight quants
constexpr int kSOffHd = kSOffBq + kSBN * 128;  // block headers, 16 bytes per column
constexpr int kSOffDx = kSOffHd + kSBN * 16;
constexpr int kSOffAm = kSOffDx + kSBM * 4;    // A' rows
constexpr int kSOffBm = kSOffAm + kSBM * kSHalf;  // B' columns
constexpr int kSOffSc = kSOffBm + kSBN * kSHalf;  // per column: sl_j | sl_j << 16 (j < 8), then sh_j | sh_j << 16
constexpr int kSScStride = 80;                 // 64 B of multipliers + 16 B pad (odd 16-byte stride)
constexpr int kSOffSum = kSOffSc + kSBN * kSScStride;  // DUMP: 32-sums as 6-bit low / high bytes
template <bool DUMP>
struct SLayout {
  static constexpr int kStage = kSOffSum + (DUMP ? kSBM * 16 : 0);
  static constexpr int kBytes = 2 * kStage;
};

struct SRegs {
  uint4 e;   // t < 128: block header of column t; 128 <= t < 256: sums of row t - 128
  float dx;  // 128 <= t < 256: scale of row t - 128
};

// 16 bytes per lane from `src` into LDS at dst + 16 * lane (dst wave-uniform).
__device__ __forceinline__ void lds_dma16(const void* src, uint8_t* dst) {
  __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)src,
                                   (__attribute__((address_space(3))) void*)dst, 16, 0, 0);
}

// Global loads of one K step. Wave w moves activation rows 16 w .. 16 w + 15
// (four instructions of four rows) and the quants of weight columns
// 16 w .. 16 w + 15 (two instructions of eight columns) straight into LDS
// stage `stg`, a lane's 16 bytes at its swizzled slot; rows and columns past
// M / N repeat the last one (their outputs are never stored). Threads 0..255
// load the block headers / the rows' scales and sums into registers (zero
// past the edges).
__device__ __forceinline__ void s_load(SRegs& R, uint8_t* stg, const int8_t* __restrict__ xq,
                                       const float* __restrict__ xd, const int16_t* __restrict__ xs,
                                       const uint8_t* __restrict__ wq, int M, int N, int K, int m0, int n0, int kb) {
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6, nbk = K / 256;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int row = 16 * wave + 4 * u + (lane >> 4);
    const int gr = min(m0 + row, M - 1);
    lds_dma16(xq + (size_t)gr * K + 256 * kb + 16 * ((lane & 15) ^ (row & 15)), stg + 256 * (16 * wave + 4 * u));
  }
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int col = 16 * wave + 8 * u + (lane >> 3);
    const int gc = min(n0 + col, N - 1);
    lds_dma16(wq + ((size_t)gc * nbk + kb) * kQ4KBytes + 16 + 16 * ((lane & 7) ^ ((col >> 1) & 7)),
              stg + kSOffBq + 128 * (16 * wave + 8 * u));
  }
  if (t < 128) {
    const int col = n0 + t;
    R.e = col < N ? *reinterpret_cast<const uint4*>(wq + ((size_t)col * nbk + kb) * kQ4KBytes) : make_uint4(0, 0, 0, 0);
  } else if (t < 256) {
    const int row = m0 + t - 128;
    const bool ok = row < M;
    R.dx = ok ? xd[(size_t)row * nbk + kb] : 0.0f;
    R.e = ok ? *reinterpret_cast<const uint4*>(xs + ((size_t)row * nbk + kb) * 8) : make_uint4(0, 0, 0, 0);
  }
}

// One A' / B' row: each of eight f32 values as three bf16 pieces
// v = p1 + p2 + p3 (each the round-to-nearest-even of what the previous ones
// leave; the remainders are exact in f32, so the three carry all 24 bits),
// stored as p1[8] | p2[8] | p3[8] (48 bytes).
__device__ __forceinline__ void s_store_row(uint8_t* dst, const float* v) {
  uint32_t w[3][4];
#pragma unroll
  for (int j = 0; j < 8; j += 2) {
    unsigned short p[3][2];
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      float r = v[j + e];
#pragma unroll
      for (int k = 0; k < 3; ++k) {
        const __bf16 b = (__bf16)r;
        p[k][e] = __builtin_bit_cast(unsigned short, b);
        r -= (float)b;
      }
    }
#pragma unroll
    for (int k = 0; k < 3; ++k) w[k][j >> 1] = p[k][0] | ((uint32_t)p[k][1] << 16);
  }
  uint4* o = reinterpret_cast<uint4*>(dst);
#pragma unroll
  for (int k = 0; k < 3; ++k) o[k] = make_uint4(w[k][0], w[k][1], w[k][2], w[k][3]);
}

// The register-staged parts of one K step into LDS stage `buf`.
template <bool DUMP>
__device__ __forceinline__ void s_store(const SRegs& R, uint8_t* buf) {
  const int t = threadIdx.x;
  float row8[8];
  if (t < 128) {
    // column t's header; B' = -dmin * m_j; the split scales sl_j = sc_j & 7, sh_j = sc_j >> 3 as packed
    // 16-bit pairs (the multipliers of the weight operands)
    const uint4 hd = R.e;
    *reinterpret_cast<uint4*>(buf + kSOffHd + 16 * t) = hd;
    const float dmin = h2f(hd.x >> 16);
    const uint32_t mn[2] = {hd.z & 0x3f3f3f3fu, ((hd.w >> 4) & 0x0f0f0f0fu) | ((hd.z >> 2) & 0x30303030u)};
#pragma unroll
    for (int j = 0; j < 8; ++j) row8[j] = -dmin * (float)((mn[j >> 2] >> (8 * (j & 3))) & 0xffu);
    s_store_row(buf + kSOffBm + kSHalf * t, row8);
    const uint32_t sc[2] = {hd.y & 0x3f3f3f3fu, (hd.w & 0x0f0f0f0fu) | ((hd.y >> 2) & 0x30303030u)};
    uint32_t v[16];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint32_t s8 = (sc[j >> 2] >> (8 * (j & 3))) & 0xffu;
      v[j] = (s8 & 7u) * 0x10001u;
      v[8 + j] = (s8 >> 3) * 0x10001u;
    }
    uint4* o = reinterpret_cast<uint4*>(buf + kSOffSc + kSScStride * t);
#pragma unroll
    for (int q = 0; q < 4; ++q) o[q] = make_uint4(v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]);
  } else if (t < 256) {
    // A' = dx * S_j of row c and the row's scale; (DUMP) the sums as 6-bit low and signed high bytes
    const int c = t - 128;
    reinterpret_cast<float*>(buf + kSOffDx)[c] = R.dx;
    const int16_t* sv = reinterpret_cast<const int16_t*>(&R.e);
#pragma unroll
    for (int j = 0; j < 8; ++j) row8[j] = R.dx * (float)sv[j];
    s_store_row(buf + kSOffAm + kSHalf * c, row8);
    if (DUMP) {
      uint32_t sl[2] = {0, 0}, sh[2] = {0, 0};
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int v = sv[j];
        sl[j >> 2] |= (uint32_t)(v & 63) << (8 * (j & 3));
        sh[j >> 2] |= (uint32_t)((v >> 6) & 0xff) << (8 * (j & 3));
      }
      *reinterpret_cast<uint4*>(buf + kSOffSum + 16 * c) = make_uint4(sl[0], sl[1], sh[0], sh[1]);
    }
  }
}

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ f32x16 mfma_bf16(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// Bytes of v times the packed pair s2 = s | s << 16 (each product < 256).
__device__ __forceinline__ i8x16 bytes_times4p(uint4 v, uint32_t s2) {
  const u16x2 b = __builtin_bit_cast(u16x2, s2);
  return as_i8x16(make_uint4(__builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, v.x) * b),
                             __builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, v.y) * b),
                             __builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, v.z) * b),
                             __builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, v.w) * b)));
}

// The integer part of one K step of mmqs from LDS stage `buf`: accl / acch =
// the split-scale MFMA sums (isd = accl + 8 acch).
__device__ __forceinline__ void mmqs_mfma(const uint8_t* __restrict__ buf, i32x16 (&accl)[kSTM],
                                          i32x16 (&acch)[kSTM], int wm, int r, int h, int bcol) {
  i32x16 zero;
#pragma unroll
  for (int j = 0; j < 16; ++j) zero[j] = 0;
  const int arow0 = 64 * wm + r;
  const int sa = r & 15, sb = (r >> 1) & 7;  // the swizzles of rows arow0 + 32 i and of column bcol
  const int8_t* A = reinterpret_cast<const int8_t*>(buf);
  const uint8_t* Bq = buf + kSOffBq + 128 * bcol;
  const uint4* SC = reinterpret_cast<const uint4*>(buf + kSOffSc + kSScStride * bcol);
  const uint4 sl4[2] = {SC[0], SC[1]}, sh4[2] = {SC[2], SC[3]};
  auto pick = [](const uint4* v, int j) {
    const uint4 q = v[j >> 2];
    return (j & 3) == 0 ? q.x : (j & 3) == 1 ? q.y : (j & 3) == 2 ? q.z : q.w;
  };
#pragma unroll
  for (int c2 = 0; c2 < 4; ++c2) {
    const uint4 qv = *reinterpret_cast<const uint4*>(Bq + 16 * ((2 * c2 + h) ^ sb));
    const uint4 blo = make_uint4(qv.x & 0x0f0f0f0fu, qv.y & 0x0f0f0f0fu, qv.z & 0x0f0f0f0fu, qv.w & 0x0f0f0f0fu);
    const uint4 bhi = make_uint4((qv.x >> 4) & 0x0f0f0f0fu, (qv.y >> 4) & 0x0f0f0f0fu, (qv.z >> 4) & 0x0f0f0f0fu,
                                 (qv.w >> 4) & 0x0f0f0f0fu);
    const i8x16 bl0 = bytes_times4p(blo, pick(sl4, 2 * c2));
    const i8x16 bh0 = bytes_times4p(blo, pick(sh4, 2 * c2));
    const i8x16 bl1 = bytes_times4p(bhi, pick(sl4, 2 * c2 + 1));
    const i8x16 bh1 = bytes_times4p(bhi, pick(sh4, 2 * c2 + 1));
    i8x16 a0[kSTM], a1[kSTM];
#pragma unroll
    for (int i = 0; i < kSTM; ++i) {
      const int8_t* ar = A + 256 * (arow0 + 32 * i);
      a0[i] = *reinterpret_cast<const i8x16*>(ar + 16 * ((4 * c2 + h) ^ sa));
      a1[i] = *reinterpret_cast<const i8x16*>(ar + 16 * ((4 * c2 + 2 + h) ^ sa));
    }
    // chains on one accumulator four MFMAs apart
#pragma unroll
    for (int i = 0; i < kSTM; ++i) accl[i] = mfma_i8(a0[i], bl0, c2 == 0 ? zero : accl[i]);
#pragma unroll
    for (int i = 0; i < kSTM; ++i) acch[i] = mfma_i8(a0[i], bh0, c2 == 0 ? zero : acch[i]);
#pragma unroll
    for (int i = 0; i < kSTM; ++i) accl[i] = mfma_i8(a1[i], bl1, accl[i]);
#pragma unroll
    for (int i = 0; i < kSTM; ++i) acch[i] = mfma_i8(a1[i], bh1, acch[i]);
  }
}

// The floating part of one K step from the same LDS stage: the mins term on
// the bf16 matrix cores (lane half h supplies K half h of each MFMA: pieces
// [a1 | a2] x [b1 | b1], [a1 | a2] x [b2 | b2], [a1 | a3] x [b3 | b1]) and
// acc += (dx * d) * isd.
__device__ __forceinline__ void mmqs_epi(const uint8_t* __restrict__ buf, const i32x16 (&accl)[kSTM],
                                         const i32x16 (&acch)[kSTM], f32x16 (&acc)[kSTM], int wm, int r, int h,
                                         int bcol) {
  const int arow0 = 64 * wm + r;
  const float* DX = reinterpret_cast<const float*>(buf + kSOffDx);
  const float dw = h2f(*reinterpret_cast<const uint32_t*>(buf + kSOffHd + 16 * bcol));
  const uint8_t* bmp = buf + kSOffBm + kSHalf * bcol;
  const bf16x8 b1 = *reinterpret_cast<const bf16x8*>(bmp);
  const bf16x8 b2 = *reinterpret_cast<const bf16x8*>(bmp + 16);
  const bf16x8 b31 = *reinterpret_cast<const bf16x8*>(bmp + (h == 0 ? 32 : 0));
#pragma unroll
  for (int i = 0; i < kSTM; ++i) {
    const uint8_t* amp = buf + kSOffAm + kSHalf * (arow0 + 32 * i);
    const bf16x8 a12 = *reinterpret_cast<const bf16x8*>(amp + 16 * h);
    const bf16x8 a13 = *reinterpret_cast<const bf16x8*>(amp + 32 * h);
    acc[i] = mfma_bf16(a12, b1, acc[i]);
    acc[i] = mfma_bf16(a12, b2, acc[i]);
    acc[i] = mfma_bf16(a13, b31, acc[i]);
  }
#pragma unroll
  for (int i = 0; i < kSTM; ++i) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const float4 dx = *reinterpret_cast<const float4*>(DX + 64 * wm + 32 * i + 8 * g + 4 * h);
      const float dxs[4] = {dx.x, dx.y, dx.z, dx.w};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int e = 4 * g + q;
        const int isd = accl[i][e] + (acch[i][e] << 3);
        acc[i][e] = __builtin_fmaf(dxs[q] * dw, (float)isd, acc[i][e]);
      }
    }
  }
}

// DUMP: one whole K step with exact integer mins, writing every block dot,
// acc += dx * (d * isd - dmin * ism).
__device__ __forceinline__ void mmqs_step_dump(const uint8_t* __restrict__ buf, f32x16 (&acc)[kSTM], int wm, int r,
                                               int h, int bcol, int m0, int col, int M, int N, int nbk, int kb,
                                               int* __restrict__ dump) {
  i32x16 zero;
#pragma unroll
  for (int j = 0; j < 16; ++j) zero[j] = 0;
  i32x16 accl[kSTM], acch[kSTM];
  mmqs_mfma(buf, accl, acch, wm, r, h, bcol);
  const int arow0 = 64 * wm + r;
  const float* DX = reinterpret_cast<const float*>(buf + kSOffDx);
  const uint4 hd = *reinterpret_cast<const uint4*>(buf + kSOffHd + 16 * bcol);
  const float dw = h2f(hd.x), dmw = h2f(hd.x >> 16);
  const uint32_t mnlo = hd.z & 0x3f3f3f3fu, mnhi = ((hd.w >> 4) & 0x0f0f0f0fu) | ((hd.z >> 2) & 0x30303030u);
  const uint4 zero4 = make_uint4(0, 0, 0, 0);
  const i8x16 bmi = as_i8x16(h == 0 ? make_uint4(mnlo, mnhi, 0, 0) : zero4);
#pragma unroll
  for (int i = 0; i < kSTM; ++i) {
    const uint4 sv = *reinterpret_cast<const uint4*>(buf + kSOffSum + 16 * (arow0 + 32 * i));
    const i8x16 alo = as_i8x16(h == 0 ? make_uint4(sv.x, sv.y, 0, 0) : zero4);
    const i8x16 ahi = as_i8x16(h == 0 ? make_uint4(sv.z, sv.w, 0, 0) : zero4);
    const i32x16 Lo = mfma_i8(alo, bmi, zero), Hi = mfma_i8(ahi, bmi, zero);
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int rt = 64 * wm + 32 * i + 8 * (e >> 2) + 4 * h + (e & 3);
      const int isd = accl[i][e] + (acch[i][e] << 3), ism = Hi[e] * 64 + Lo[e];
      acc[i][e] += DX[rt] * (dw * (float)isd - dmw * (float)ism);
      if (m0 + rt < M && col < N) {
        const size_t o = ((size_t)(m0 + rt) * N + col) * nbk + kb;
        dump[2 * o] = isd;
        dump[2 * o + 1] = ism;
      }
    }
  }
}

// K steps [kb0, kb1) of the 128 x 128 tile at (m0, n0) into acc (zeroed
// first): the staging / MFMA loop of one tile. Ends with a barrier after the
// last step, so the LDS stages are free for the next call.
template <bool DUMP>
__device__ __forceinline__ void mmqs_run(const uint8_t* __restrict__ wq, const int8_t* __restrict__ xq,
                                         const float* __restrict__ xd, const int16_t* __restrict__ xs, int M, int N,
                                         int K, int m0, int n0, int kb0, int kb1, int* __restrict__ dump,
                                         f32x16 (&acc)[kSTM]) {
  using Lay = SLayout<DUMP>;
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int nbk = K / 256;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 31, h = lane >> 5;
  const int wm = wave & 1, wn = wave >> 1;
  const int bcol = 32 * wn + r;  // this lane's column in the workgroup tile
  const int col = n0 + bcol;

  // one f32 accumulator per output: the bf16 MFMAs add the mins term to it, the VALU the d term
#pragma unroll
  for (int i = 0; i < kSTM; ++i)
#pragma unroll
    for (int j = 0; j < 16; ++j) acc[i][j] = 0.0f;

  // the next K step streams into the other LDS stage (and its headers / scales into registers) while this
  // step computes from stage (kb - kb0) & 1; each wave waits for its own LDS loads before the barrier
  SRegs R;
  s_load(R, lds, xq, xd, xs, wq, M, N, K, m0, n0, kb0);
  s_store<DUMP>(R, lds);
  __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0)
  __syncthreads();
  i32x16 accl[kSTM], acch[kSTM];
  for (int kb = kb0; kb < kb1; ++kb) {
    const uint8_t* cur = lds + ((kb - kb0) & 1) * Lay::kStage;
    uint8_t* nxt = lds + ((kb + 1 - kb0) & 1) * Lay::kStage;
    if (kb + 1 < kb1) s_load(R, nxt, xq, xd, xs, wq, M, N, K, m0, n0, kb + 1);
    if constexpr (DUMP) {
      mmqs_step_dump(cur, acc, wm, r, h, bcol, m0, col, M, N, nbk, kb, dump);
    } else {
      mmqs_mfma(cur, accl, acch, wm, r, h, bcol);
      mmqs_epi(cur, accl, acch, acc, wm, r, h, bcol);
    }
    if (kb + 1 < kb1) s_store<DUMP>(R, nxt);
    __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0)
    __syncthreads();
  }
}

// acc of the tile at (m0, n0) -> y (rows < M, columns < N; added to y when
// accumulate). Lane (r, h) of wave (wm, wn) holds column 32 wn + r and rows
// 64 wm + 32 i + 8 (e >> 2) + 4 h + (e & 3) (the 32x32 MFMA output layout).
__device__ __forceinline__ void mmqs_store(const f32x16 (&acc)[kSTM], float* __restrict__ y, int M, int N, int ldy,
                                           int m0, int n0, int accumulate) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 31, h = lane >> 5;
  const int wm = wave & 1, wn = wave >> 1;
  const int col = n0 + 32 * wn + r;
#pragma unroll
  for (int i = 0; i < kSTM; ++i)
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int row = m0 + 64 * wm + 32 * i + 8 * (e >> 2) + 4 * h + (e & 3);
      if (row < M && col < N) {
        float* yp = y + (size_t)row * ldy + col;
        *yp = accumulate ? *yp + acc[i][e] : acc[i][e];
      }
    }
}

template <bool DUMP>
__device__ __forceinline__ void mmqs_q4k(const uint8_t* __restrict__ wq, const int8_t* __restrict__ xq,
                                         const float* __restrict__ xd, const int16_t* __restrict__ xs,
                                         float* __restrict__ y, int M, int N, int K, int ldy, int* __restrict__ dump,
                                         int accumulate, int remap, int kb0, int kb1) {
  int mt, nt;
  gemm_tile(remap, mt, nt);
  const int m0 = mt * kSBM, n0 = nt * kSBN;
  f32x16 acc[kSTM];
  mmqs_run<DUMP>(wq, xq, xd, xs, M, N, K, m0, n0, kb0, kb1, dump, acc);
  mmqs_store(acc, y, M, N, ldy, m0, n0, accumulate);
}

// Stream-K schedule of mmqs over a grid of G workgroups (one per CU): the
// tiles split into sk_tiles stream-K tiles and T - sk_tiles data-parallel
// ones (a multiple of G). Tile v is (v % gy, v / gy) in (M tile, N tile), so
// consecutive tiles share their weight columns.
//   * Data-parallel: round q of workgroup w takes tile sk_tiles + u with
//     u = (w % 8) * (T_dp / 8) + w / 8 + q * G / 8: the workgroups of one XCD
//     (w % 8 is the XCD a workgroup runs on) take one contiguous run of
//     tiles, whose weight columns then come through that XCD's L2 once.
//   * Stream-K: the sk_tiles * nbk (tile, K step) iterations, tile-major,
//     are cut into G equal ranges, range w = [w I / G, (w + 1) I / G). A
//     workgroup walks its range as segments (one per tile it touches); a
//     segment that covers the whole tile stores it, any other one writes its
//     f32 partial to `part` (slot 2 w for the workgroup's first segment,
//     2 w + 1 for its last; element j of thread t at j * 512 + t, so a wave's
//     store covers whole lines) and bumps the tile's counter; the workgroup
//     that brings the counter to the tile's segment count adds the segments'
//     partials in K order (its own from registers), stores the tile and
//     resets the counter. The order of the sum depends only on the shapes,
//     never on arrival order.
// Ordering, as in the decode attention's merge: the partials are written and
// read with agent-scope atomics (relaxed), which on gfx950 carry sc1 (the
// stores write through the XCD's L2, the loads are served from the
// device-coherent level); every thread waits for its stores (vmcnt(0))
// before the barrier that precedes thread 0's counter atomic, and the
// partial loads issue after the counter's result is back. The
// acquire-release form (plain partials, release fences, acq_rel counter) is
// correct too but each agent-scope release and acquire writes back or
// invalidates the whole L2: at 14336 x 4096 x M 512 it ran 213 us against
// 106 us.
// Counters start at zero (the host clears them before the launch) and every
// one is back at zero when the grid ends.
__device__ __forceinline__ int sk_owner(long long i, long long I, int G) {
  return (int)(((i + 1) * G - 1) / I);
}

__device__ __forceinline__ void mmqs_q4k_sk(const uint8_t* __restrict__ wq, const int8_t* __restrict__ xq,
                                            const float* __restrict__ xd, const int16_t* __restrict__ xs,
                                            float* __restrict__ y, int M, int N, int K, int ldy, int accumulate,
                                            int gy, int T, int sk_tiles, float* __restrict__ part,
                                            unsigned* __restrict__ counters) {
  __shared__ int last_s;
  const int G = gridDim.x, w = blockIdx.x, t = threadIdx.x;
  const int nbk = K / 256;
  f32x16 acc[kSTM];
  // data-parallel tiles
  const int tdp = T - sk_tiles, rounds = tdp / G;
  for (int q = 0; q < rounds; ++q) {
    const int u = (w & 7) * (tdp >> 3) + (w >> 3) + q * (G >> 3);
    const int v = sk_tiles + u;
    const int m0 = (v % gy) * kSBM, n0 = (v / gy) * kSBN;
    mmqs_run<false>(wq, xq, xd, xs, M, N, K, m0, n0, 0, nbk, nullptr, acc);
    mmqs_store(acc, y, M, N, ldy, m0, n0, accumulate);
  }
  // stream-K range
  const long long I = (long long)sk_tiles * nbk;
  const long long it0 = (long long)w * I / G, it1 = (long long)(w + 1) * I / G;
  for (long long it = it0; it < it1;) {
    const int v = (int)(it / nbk);
    const int kb0 = (int)(it - (long long)v * nbk);
    const int kb1 = (int)min((long long)nbk, kb0 + (it1 - it));
    const int m0 = (v % gy) * kSBM, n0 = (v / gy) * kSBN;
    mmqs_run<false>(wq, xq, xd, xs, M, N, K, m0, n0, kb0, kb1, nullptr, acc);
    it += kb1 - kb0;
    if (kb0 == 0 && kb1 == nbk) {
      mmqs_store(acc, y, M, N, ldy, m0, n0, accumulate);
      continue;
    }
    const long long i0 = (long long)v * nbk;
    const int wf = sk_owner(i0, I, G), nseg = sk_owner(i0 + nbk - 1, I, G) - wf + 1;
    // this segment is the workgroup's first one when its range starts inside tile v
    float* mine = part + (size_t)(2 * w + (it0 >= i0 ? 0 : 1)) * kSBM * kSBN + t;
#pragma unroll
    for (int i = 0; i < kSTM; ++i)
#pragma unroll
      for (int e = 0; e < 16; ++e)
        __hip_atomic_store(mine + 512 * (16 * i + e), acc[i][e], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): this thread's partial is stored
    __syncthreads();
    if (t == 0)
      last_s = __hip_atomic_fetch_add(counters + v, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
               (unsigned)(nseg - 1);
    __syncthreads();
    if (!last_s) continue;
    f32x16 sum[kSTM];
#pragma unroll
    for (int i = 0; i < kSTM; ++i)
#pragma unroll
      for (int e = 0; e < 16; ++e) sum[i][e] = 0.0f;
    for (int sg = 0; sg < nseg; ++sg) {
      const int ws = wf + sg;
      if (ws == w) {
#pragma unroll
        for (int i = 0; i < kSTM; ++i) sum[i] += acc[i];
        continue;
      }
      const long long ws0 = (long long)ws * I / G;
      const float* src = part + (size_t)(2 * ws + (ws0 >= i0 ? 0 : 1)) * kSBM * kSBN + t;
#pragma unroll
      for (int i = 0; i < kSTM; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e)
          sum[i][e] += __hip_atomic_load(src + 512 * (16 * i + e), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    mmqs_store(sum, y, M, N, ldy, m0, n0, accumulate);
    if (t == 0) __hip_atomic_store(counters + v, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

}  // namespace qmm

#define QMM_MMQS_KERNEL(SUFFIX, DUMP)                                                                          \
  extern "C" __global__ void __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))                 \
      qmm_mmqs_q4k##SUFFIX(const uint8_t* __restrict__ wq, const int8_t* __restrict__ xq,                      \
                           const float* __restrict__ xd, const int16_t* __restrict__ xs, float* __restrict__ y, \
                           int M, int N, int K, int ldy, int* __restrict__ dump, int accumulate, int remap,     \
                           int kc, long long ysplit) {                                                          \
    const qmm::KRange kr = qmm::split_range(K, kc);                                                            \
    qmm::mmqs_q4k<DUMP>(wq, xq, xd, xs, y + blockIdx.z * ysplit, M, N, K, ldy, dump, accumulate, remap,        \
                        kr.kb0, kr.kb1);                                                                       \
  }
QMM_MMQS_KERNEL(, false)
QMM_MMQS_KERNEL(_dump, true)

// Two Q4_K weights of one shape over the same activation planes in one
// launch (the feed-forward block's gate and up: grid z = weight), unsplit: the
// tiles of both in one grid instead of two launches with split-K partials.
extern "C" __global__ void __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
qmm_mmqs2_q4k(const uint8_t* __restrict__ w0, const uint8_t* __restrict__ w1, const int8_t* __restrict__ xq,
              const float* __restrict__ xd, const int16_t* __restrict__ xs, float* __restrict__ y0,
              float* __restrict__ y1, int M, int N, int K, int ldy0, int ldy1, int accumulate) {
  const int j = (int)blockIdx.z;
  qmm::mmqs_q4k<false>(j ? w1 : w0, xq, xd, xs, j ? y1 : y0, M, N, K, j ? ldy1 : ldy0, nullptr, accumulate, 1, 0,
                       K / 256);
}

// ---------------------------------------------------------------------------
// mmqs6: the Q6_K prefill GEMM with the sub-block scales in the MFMA
// operands. A Q6_K code q - 32 lies in [-32, 31] and its 16-element sub-block
// scale sc is a signed byte; sc * q does not fit an int8 operand, but every
// sc in [-128, 127] is d0 + 8 d1 + 64 d2 with digits d in [-3, 4]
// (d0 = ((sc + 3) mod 8) - 3, then the same on (sc - d0) / 8; d2 stays in
// [-2, 2]), and d * q then lies in [-128, 124]. So per 32-element chunk the
// weight operand of digit i is d_i(sub-block) * q (a lane's 16 K elements
// belong to one sub-block) and
//   isum = MFMA-sum(x, d0 q) + 8 MFMA-sum(x, d1 q) + 64 MFMA-sum(x, d2 q)
// exactly in int32; y += dx * (d * isum) per super-block, the first-generation
// kernel's f32 sequence. Three int8 MFMA sets per chunk replace the two 24-bit
// multiply-adds per output and sub-block of the masked first-generation
// kernel (mmq<Q6_K>).
// Workgroup and waves as mmqs: a 128 x 128 tile, eight waves (two along M with
// 64 rows each, four along N with 32 columns), two LDS stages.
//   * Activation rows go straight to LDS (swizzled chunks), as in mmqs.
//   * Weights come through registers: thread t takes column t / 4's 64
//     elements of quarter t % 4 (ql of its half and qh), unpacks them to int8
//     q - 32 in LDS (16-byte chunk k of column n at slot k ^ (n & 15)) and
//     writes the digits of four of the column's sixteen scales.
//   * Per chunk a lane forms each digit's operand from its 16 codes: even and
//     odd bytes widened to 16-bit lanes, one packed 16-bit multiply each (the
//     low byte is the product modulo 256, i.e. the int8 product), one byte
//     permute back.
// DUMP instantiations write every block's isum, as mmq<Q6_K>'s dump does.
// ---------------------------------------------------------------------------
namespace qmm {

constexpr int kS6OffBq = kSBM * 256;             // int8 codes [col][256], swizzled 16-byte slots
constexpr int kS6OffDg = kS6OffBq + kSBN * 256;  // digit bytes [col][3][16]
constexpr int kS6OffDw = kS6OffDg + kSBN * 48;   // f32 d per column
constexpr int kS6OffDx = kS6OffDw + kSBN * 4;    // f32 scale per row
constexpr int kS6Stage = kS6OffDx + kSBM * 4;

struct SRegs6 {
  uint4 l0, l1, l2, l3;  // ql[64 n, +64) of the thread's column (n = its half)
  uint4 h0, h1;          // qh[32 n, +32)
  uint32_t sc4;          // the column's int8 scales 4 p .. 4 p + 3 (p = the thread's quarter)
  uint32_t dh;           // f16 d (quarter 0)
  float dx;              // t < 128: scale of row t
};

// Global loads of one K step: activation rows straight into stage `stg` (as
// s_load), the weight bytes and scales into registers (columns past N repeat
// the last one; their outputs are never stored).
__device__ __forceinline__ void s6_load(SRegs6& R, uint8_t* stg, const int8_t* __restrict__ xq,
                                        const float* __restrict__ xd, const uint8_t* __restrict__ wq,
                                        const uint16_t* __restrict__ wd, int M, int N, int K, int m0, int n0,
                                        int kb) {
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6, nbk = K / 256;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int row = 16 * wave + 4 * u + (lane >> 4);
    const int gr = min(m0 + row, M - 1);
    lds_dma16(xq + (size_t)gr * K + 256 * kb + 16 * ((lane & 15) ^ (row & 15)), stg + 256 * (16 * wave + 4 * u));
  }
  const int col = t >> 2, p = t & 3, n = p >> 1;
  const int gc = min(n0 + col, N - 1);
  const uint4* b = reinterpret_cast<const uint4*>(wq + ((size_t)gc * nbk + kb) * kQ6KBody);
  R.l0 = b[4 * n];
  R.l1 = b[4 * n + 1];
  R.l2 = b[4 * n + 2];
  R.l3 = b[4 * n + 3];
  R.h0 = b[8 + 2 * n];
  R.h1 = b[9 + 2 * n];
  R.sc4 = reinterpret_cast<const uint32_t*>(b + 12)[p];
  R.dh = p == 0 ? (uint32_t)wd[(size_t)gc * nbk + kb] : 0u;
  if (t < 128) {
    const int row = m0 + t;
    R.dx = row < M ? xd[(size_t)row * nbk + kb] : 0.0f;
  }
}

// The register-staged parts of one K step into stage `buf`: the int8 codes of
// elements 128 n + 32 j + l (j = 2 (p & 1) + {0, 1}, l < 32) of the thread's
// column, the digits of scales 4 p .. 4 p + 3, d and the row scales.
__device__ __forceinline__ void s6_store(const SRegs6& R, uint8_t* buf) {
  const int t = threadIdx.x, col = t >> 2, p = t & 3, n = p >> 1, hi = p & 1;
  uint8_t* bq = buf + kS6OffBq + 256 * col;
  const int sw = col & 15;
  // ql bytes [32 jj + 16 half, +16) of the half hold elements 32 j + 16 half + [0, 16) for j = 2 hi + jj
  // (low nibbles for hi = 0, high ones for hi = 1); qh bits 2 j of the same l
  const int ns = hi ? 4 : 0;
  auto put = [&](uint4 lq, uint4 hq, int j, int half) {
    const int qs = 2 * j;
    auto one = [&](uint32_t l, uint32_t h) {
      return q6_sub32(((l >> ns) & 0x0f0f0f0fu) | (((h >> qs) & 0x03030303u) << 4));
    };
    const int slot = 8 * n + 2 * j + half;
    *reinterpret_cast<uint4*>(bq + 16 * (slot ^ sw)) =
        make_uint4(one(lq.x, hq.x), one(lq.y, hq.y), one(lq.z, hq.z), one(lq.w, hq.w));
  };
  put(R.l0, R.h0, 2 * hi, 0);
  put(R.l1, R.h1, 2 * hi, 1);
  put(R.l2, R.h0, 2 * hi + 1, 0);
  put(R.l3, R.h1, 2 * hi + 1, 1);
  // digits of scales 4 p .. 4 p + 3
  const uint32_t sw4 = R.sc4;
  uint32_t dg[3] = {0u, 0u, 0u};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int s = (int)(int8_t)((sw4 >> (8 * i)) & 0xffu);
    const int d0 = ((s + 3) & 7) - 3;
    const int r = (s - d0) >> 3;
    const int d1 = ((r + 3) & 7) - 3;
    const int d2 = (r - d1) >> 3;
    dg[0] |= (uint32_t)(d0 & 0xff) << (8 * i);
    dg[1] |= (uint32_t)(d1 & 0xff) << (8 * i);
    dg[2] |= (uint32_t)(d2 & 0xff) << (8 * i);
  }
  uint32_t* dgp = reinterpret_cast<uint32_t*>(buf + kS6OffDg + 48 * col);
#pragma unroll
  for (int d = 0; d < 3; ++d) dgp[4 * d + p] = dg[d];
  if (p == 0) reinterpret_cast<float*>(buf + kS6OffDw)[col] = h2f(R.dh);
  if (t < 128) reinterpret_cast<float*>(buf + kS6OffDx)[t] = R.dx;
}

// One K step's digit sums from stage `buf`: acc[d][i] = MFMA-sum over the
// step of x (row tile i) and d_d * q (the lane's column).
__device__ __forceinline__ void mmqs6_mfma(const uint8_t* __restrict__ buf, i32x16 (&acc)[3][kSTM], int wm, int r,
                                           int h, int bcol) {
  i32x16 zero;
#pragma unroll
  for (int j = 0; j < 16; ++j) zero[j] = 0;
  const int arow0 = 64 * wm + r;
  const int sa = r & 15, sb = bcol & 15;
  const int8_t* A = reinterpret_cast<const int8_t*>(buf);
  const uint8_t* Bq = buf + kS6OffBq + 256 * bcol;
  const uint4* DG = reinterpret_cast<const uint4*>(buf + kS6OffDg + 48 * bcol);
  const uint4 dgv[3] = {DG[0], DG[1], DG[2]};
  auto dword = [](const uint4& v, int i) { return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w; };
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    const uint4 bv = *reinterpret_cast<const uint4*>(Bq + 16 * ((2 * c + h) ^ sb));
    const uint32_t bw[4] = {bv.x, bv.y, bv.z, bv.w};
    uint32_t ev[4], od[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      ev[k] = bw[k] & 0x00ff00ffu;
      od[k] = (bw[k] >> 8) & 0x00ff00ffu;
    }
    i8x16 a[kSTM];
#pragma unroll
    for (int i = 0; i < kSTM; ++i)
      a[i] = *reinterpret_cast<const i8x16*>(A + 256 * (arow0 + 32 * i) + 16 * ((2 * c + h) ^ sa));
    const int sh = 8 * (2 * (c & 1) + h);  // byte (2 c + h) of the digit rows: dword c / 2
#pragma unroll
    for (int d = 0; d < 3; ++d) {
      const int dv = (int)(int8_t)((dword(dgv[d], c >> 1) >> sh) & 0xffu);
      const u16x2 m2 = __builtin_bit_cast(u16x2, ((uint32_t)dv & 0xffffu) * 0x10001u);
      uint32_t w[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const uint32_t pe = __builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, ev[k]) * m2);
        const uint32_t po = __builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, od[k]) * m2);
        w[k] = __builtin_amdgcn_perm(po, pe, 0x06020400u);  // bytes pe.0, po.0, pe.2, po.2
      }
      const i8x16 bd = as_i8x16(make_uint4(w[0], w[1], w[2], w[3]));
#pragma unroll
      for (int i = 0; i < kSTM; ++i) acc[d][i] = mfma_i8(a[i], bd, c == 0 ? zero : acc[d][i]);
    }
  }
}

// acc = fma(dx, d * isum, acc) per output (isum = D0 + 8 D1 + 64 D2); DUMP:
// every block's isum.
template <bool DUMP>
__device__ __forceinline__ void mmqs6_epi(const uint8_t* __restrict__ buf, const i32x16 (&dsum)[3][kSTM],
                                          f32x16 (&acc)[kSTM], int wm, int r, int h, int bcol, int m0, int col,
                                          int M, int N, int nbk, int kb, int* __restrict__ dump) {
#pragma clang fp contract(off)
  const float* DX = reinterpret_cast<const float*>(buf + kS6OffDx);
  const float dw = reinterpret_cast<const float*>(buf + kS6OffDw)[bcol];
#pragma unroll
  for (int i = 0; i < kSTM; ++i) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const float4 dx = *reinterpret_cast<const float4*>(DX + 64 * wm + 32 * i + 8 * g + 4 * h);
      const float dxs[4] = {dx.x, dx.y, dx.z, dx.w};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int e = 4 * g + q;
        const int isum = dsum[0][i][e] + (dsum[1][i][e] << 3) + (dsum[2][i][e] << 6);
        // the first-generation tile's sequence (its += compiles to one fma): the same bits
        acc[i][e] = __builtin_fmaf(dxs[q], dw * (float)isum, acc[i][e]);
        if (DUMP) {
          const int rt = 64 * wm + 32 * i + 8 * g + 4 * h + q;
          if (m0 + rt < M && col < N) dump[((size_t)(m0 + rt) * N + col) * nbk + kb] = isum;
        }
      }
    }
  }
  (void)r;
}

// The 128 x 128 tile at (m0, n0), K steps [kb0, kb1), into y.
// wd: the weight's separated f16 d per block (row-major, K / 256 per row).
template <bool DUMP>
__device__ __forceinline__ void mmqs6_q6k_at(const uint8_t* __restrict__ wq, const uint16_t* __restrict__ wd,
                                             const int8_t* __restrict__ xq, const float* __restrict__ xd,
                                             float* __restrict__ y, int M, int N, int K, int ldy,
                                             int* __restrict__ dump, int accumulate, int m0, int n0, int kb0,
                                             int kb1) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int nbk = K / 256;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 31, h = lane >> 5;
  const int wm = wave & 1, wn = wave >> 1;
  const int bcol = 32 * wn + r;
  const int col = n0 + bcol;
  f32x16 acc[kSTM];
#pragma unroll
  for (int i = 0; i < kSTM; ++i)
#pragma unroll
    for (int j = 0; j < 16; ++j) acc[i][j] = 0.0f;
  SRegs6 R;
  s6_load(R, lds, xq, xd, wq, wd, M, N, K, m0, n0, kb0);
  s6_store(R, lds);
  __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0)
  __syncthreads();
  for (int kb = kb0; kb < kb1; ++kb) {
    const uint8_t* cur = lds + ((kb - kb0) & 1) * kS6Stage;
    uint8_t* nxt = lds + ((kb + 1 - kb0) & 1) * kS6Stage;
    if (kb + 1 < kb1) s6_load(R, nxt, xq, xd, wq, wd, M, N, K, m0, n0, kb + 1);
    i32x16 dsum[3][kSTM];
    mmqs6_mfma(cur, dsum, wm, r, h, bcol);
    mmqs6_epi<DUMP>(cur, dsum, acc, wm, r, h, bcol, m0, col, M, N, nbk, kb, dump);
    if (kb + 1 < kb1) s6_store(R, nxt);
    __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0)
    __syncthreads();
  }
  mmqs_store(acc, y, M, N, ldy, m0, n0, accumulate);
}

template <bool DUMP>
__device__ __forceinline__ void mmqs6_q6k(const uint8_t* __restrict__ wq, const uint16_t* __restrict__ wd,
                                          const int8_t* __restrict__ xq, const float* __restrict__ xd,
                                          float* __restrict__ y, int M, int N, int K, int ldy,
                                          int* __restrict__ dump, int accumulate, int remap, int kb0, int kb1) {
  int mt, nt;
  gemm_tile(remap, mt, nt);
  mmqs6_q6k_at<DUMP>(wq, wd, xq, xd, y, M, N, K, ldy, dump, accumulate, mt * kSBM, nt * kSBN, kb0, kb1);
}

// Q8_0 prefill GEMM on the mmqs scaffold (mmqs8_q8_0): 128 x 128 tiles of
// eight waves (four along M, two along N; each wave 32 rows x 64 columns), two
// LDS stages. Per 256-wide K step both operands are plain int8 rows of 256
// bytes (eight 32-blocks), so the activation rows and the weight codes both go
// from global memory straight into LDS (global_load_lds, 16-byte chunks
// swizzled by row / column as in mmqs); only the block scales pass through
// registers (the weight's f16 d as f32 [col][8], the activation's f32 d
// transposed to [block][row] so that four consecutive rows are one float4).
// Per 32-block one int8 MFMA per 32 x 32 tile gives the block dot P exactly;
// acc = fma(dw * dx, float(P), acc), the first-generation tile's sequence, so
// the outputs equal its bits.
constexpr int kS8OffBq = kSBM * 256;             // weight codes [col][256], swizzled 16-byte slots
constexpr int kS8OffDw = kS8OffBq + kSBN * 256;  // f32 d [col][8]
constexpr int kS8OffDx = kS8OffDw + kSBN * 32;   // f32 d [block][row]
constexpr int kS8Stage = kS8OffDx + 8 * kSBM * 4;

struct SRegs8 {
  uint4 dw;   // t < 128: column t's eight f16 block scales
  float4 dx;  // 128 <= t < 384: block scales 4 q .. 4 q + 3 of row (t - 128) / 2 (q = t & 1)
};

// Global loads of one K step: activation rows and weight codes straight into
// stage `stg` (wave w: rows / columns 16 w .. 16 w + 15, four instructions of
// four each); the scales into registers. Rows and columns past M / N repeat
// the last one (their outputs are never stored).
__device__ __forceinline__ void s8_load(SRegs8& R, uint8_t* stg, const int8_t* __restrict__ xq,
                                        const float* __restrict__ xd, const uint8_t* __restrict__ wq,
                                        const uint16_t* __restrict__ wd, int M, int N, int K, int m0, int n0,
                                        int kb) {
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6, nbw = K / 32;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int row = 16 * wave + 4 * u + (lane >> 4);
    const int gr = min(m0 + row, M - 1);
    lds_dma16(xq + (size_t)gr * K + 256 * kb + 16 * ((lane & 15) ^ (row & 15)), stg + 256 * (16 * wave + 4 * u));
  }
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int col = 16 * wave + 4 * u + (lane >> 4);
    const int gc = min(n0 + col, N - 1);
    lds_dma16(wq + ((size_t)gc * nbw + 8 * kb) * kQ80Body + 16 * ((lane & 15) ^ (col & 15)),
              stg + kS8OffBq + 256 * (16 * wave + 4 * u));
  }
  if (t < 128) {
    const int gc = min(n0 + t, N - 1);
    R.dw = *reinterpret_cast<const uint4*>(wd + (size_t)gc * nbw + 8 * kb);
  } else if (t < 384) {
    const int i = t - 128;
    const int gr = min(m0 + (i >> 1), M - 1);
    R.dx = *reinterpret_cast<const float4*>(xd + (size_t)gr * nbw + 8 * kb + 4 * (i & 1));
  }
}

__device__ __forceinline__ void s8_store(const SRegs8& R, uint8_t* buf) {
  const int t = threadIdx.x;
  if (t < 128) {
    float* dw = reinterpret_cast<float*>(buf + kS8OffDw) + 8 * t;
    const uint32_t v[4] = {R.dw.x, R.dw.y, R.dw.z, R.dw.w};
    *reinterpret_cast<float4*>(dw) = make_float4(h2f(v[0]), h2f(v[0] >> 16), h2f(v[1]), h2f(v[1] >> 16));
    *reinterpret_cast<float4*>(dw + 4) = make_float4(h2f(v[2]), h2f(v[2] >> 16), h2f(v[3]), h2f(v[3] >> 16));
  } else if (t < 384) {
    const int i = t - 128, row = i >> 1, q = i & 1;
    float* dx = reinterpret_cast<float*>(buf + kS8OffDx);
    dx[(4 * q) * kSBM + row] = R.dx.x;
    dx[(4 * q + 1) * kSBM + row] = R.dx.y;
    dx[(4 * q + 2) * kSBM + row] = R.dx.z;
    dx[(4 * q + 3) * kSBM + row] = R.dx.w;
  }
}

// One K step from stage `buf`. Wave w owns rows 32 (w & 3) .. + 32 and the
// two 32-column tiles of columns 64 (w >> 2) .. + 64, so a lane's 16 outputs
// per tile share their rows across both tiles: per 32-block c the lane reads
// its rows' 16 activation scales once (four float4 from the [block][row]
// layout) and one weight scale per tile. Per tile j, P = the MFMA block dot,
// acc += (dw * dx) * P. DUMP: every block dot.
template <bool DUMP>
__device__ __forceinline__ void mmqs8_step(const uint8_t* __restrict__ buf, f32x16 (&acc)[2], int wm, int wn, int r,
                                           int h, int m0, int n0, int M, int N, int nbw, int kb,
                                           int* __restrict__ dump) {
#pragma clang fp contract(off)
  i32x16 zero;
#pragma unroll
  for (int j = 0; j < 16; ++j) zero[j] = 0;
  const int arow = 32 * wm + r, sa = r & 15;
  const int8_t* A = reinterpret_cast<const int8_t*>(buf) + 256 * arow;
  const int8_t* B = reinterpret_cast<const int8_t*>(buf + kS8OffBq) + 256 * (64 * wn + r);
  const float* DW = reinterpret_cast<const float*>(buf + kS8OffDw) + 8 * (64 * wn + r);
  const float* DX = reinterpret_cast<const float*>(buf + kS8OffDx) + 32 * wm + 4 * h;
  // two blocks at a time (fully unrolled, the compiler hoists every MFMA of
  // the step ahead of the epilogues and spills)
#pragma unroll 2
  for (int c = 0; c < 8; ++c) {
    const int slot = 2 * c + h;  // 16-byte chunk of this lane half
    const i8x16 a = *reinterpret_cast<const i8x16*>(A + 16 * (slot ^ sa));
    float dxs[16];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const float4 dx = *reinterpret_cast<const float4*>(DX + c * kSBM + 8 * g);
      dxs[4 * g] = dx.x;
      dxs[4 * g + 1] = dx.y;
      dxs[4 * g + 2] = dx.z;
      dxs[4 * g + 3] = dx.w;
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      // columns 32 j + r: the swizzle of column 64 wn + 32 j + r is r & 15
      const i8x16 b = *reinterpret_cast<const i8x16*>(B + 256 * 32 * j + 16 * (slot ^ sa));
      const float dwc = DW[256 * j + c];
      const i32x16 P = mfma_i8(a, b, zero);
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        acc[j][e] = __builtin_fmaf(dwc * dxs[e], (float)P[e], acc[j][e]);
        if (DUMP) {
          const int row = m0 + 32 * wm + 8 * (e >> 2) + 4 * h + (e & 3), col = n0 + 64 * wn + 32 * j + r;
          if (row < M && col < N) dump[((size_t)row * N + col) * nbw + 8 * kb + c] = P[e];
        }
      }
    }
  }
}

// wd: the weight's separated f16 d per 32-block (row-major, K / 32 per row).
template <bool DUMP>
__device__ __forceinline__ void mmqs8_q8_0(const uint8_t* __restrict__ wq, const uint16_t* __restrict__ wd,
                                           const int8_t* __restrict__ xq, const float* __restrict__ xd,
                                           float* __restrict__ y, int M, int N, int K, int ldy,
                                           int* __restrict__ dump, int accumulate, int remap, int kb0, int kb1) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  int mt, nt;
  gemm_tile(remap, mt, nt);
  const int m0 = mt * kSBM, n0 = nt * kSBN;
  const int nbw = K / 32;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 31, h = lane >> 5;
  const int wm = wave & 3, wn = wave >> 2;
  f32x16 acc[2];
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[j][e] = 0.0f;
  SRegs8 R;
  s8_load(R, lds, xq, xd, wq, wd, M, N, K, m0, n0, kb0);
  s8_store(R, lds);
  __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0)
  __syncthreads();
  for (int kb = kb0; kb < kb1; ++kb) {
    const uint8_t* cur = lds + ((kb - kb0) & 1) * kS8Stage;
    uint8_t* nxt = lds + ((kb + 1 - kb0) & 1) * kS8Stage;
    if (kb + 1 < kb1) s8_load(R, nxt, xq, xd, wq, wd, M, N, K, m0, n0, kb + 1);
    mmqs8_step<DUMP>(cur, acc, wm, wn, r, h, m0, n0, M, N, nbw, kb, dump);
    if (kb + 1 < kb1) s8_store(R, nxt);
    __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0)
    __syncthreads();
  }
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int col = n0 + 64 * wn + 32 * j + r;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int row = m0 + 32 * wm + 8 * (e >> 2) + 4 * h + (e & 3);
      if (row < M && col < N) {
        float* yp = y + (size_t)row * ldy + col;
        *yp = accumulate ? *yp + acc[j][e] : acc[j][e];
      }
    }
  }
}

}  // namespace qmm

#define QMM_MMQS8_KERNEL(SUFFIX, DUMP)                                                                         \
  extern "C" __global__ void __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))                 \
      qmm_mmqs8_q8_0##SUFFIX(const uint8_t* __restrict__ wq, const int8_t* __restrict__ xq,                    \
                             const float* __restrict__ xd, const int16_t* __restrict__ xs,                     \
                             float* __restrict__ y, int M, int N, int K, int ldy, int* __restrict__ dump,       \
                             int accumulate, int remap, int kc, long long ysplit) {                            \
    (void)xs;                                                                                                  \
    const qmm::KRange kr = qmm::split_range(K, kc);                                                            \
    qmm::mmqs8_q8_0<DUMP>(wq, qmm::split_scales<qmm::kFmtQ80>(wq, N, K), xq, xd, y + blockIdx.z * ysplit, M, N, \
                          K, ldy, dump, accumulate, remap, kr.kb0, kr.kb1);                                    \
  }
QMM_MMQS8_KERNEL(, false)
QMM_MMQS8_KERNEL(_dump, true)

#define QMM_MMQS6_KERNEL(SUFFIX, DUMP)                                                                         \
  extern "C" __global__ void __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))                 \
      qmm_mmqs6_q6k##SUFFIX(const uint8_t* __restrict__ wq, const int8_t* __restrict__ xq,                     \
                            const float* __restrict__ xd, const int16_t* __restrict__ xs,                      \
                            float* __restrict__ y, int M, int N, int K, int ldy, int* __restrict__ dump,        \
                            int accumulate, int remap, int kc, long long ysplit) {                             \
    (void)xs;                                                                                                  \
    const qmm::KRange kr = qmm::split_range(K, kc);                                                            \
    qmm::mmqs6_q6k<DUMP>(wq, qmm::split_scales<qmm::kFmtQ6K>(wq, N, K), xq, xd, y + blockIdx.z * ysplit, M, N, \
                         K, ldy, dump, accumulate, remap, kr.kb0, kr.kb1);                                     \
  }
QMM_MMQS6_KERNEL(, false)
QMM_MMQS6_KERNEL(_dump, true)

// Up to three Q4_K / Q6_K weights of one K over the same activation planes in
// one launch (the prefill's q / k / v), each split over K into f32 partials:
// workgroup b of the 1-D grid belongs to job j with start[j] <= b <
// start[j + 1]; within the job, b - start[j] = split * tiles + tile, the tile
// row-major over gx column tiles, its K steps [split * kc, split * kc + kc),
// its partial at y + split * M * n (row stride n). The tiles and their
// arithmetic are the single-weight kernels' (mmqs_q4k, mmqs6_q6k); the
// dynamic LDS is the larger of their two layouts.
struct MmqsJobs {
  const uint8_t* w[3];
  float* y[3];
  int n[3], gx[3], kc[3], q6[3];  // q6: 1 for a Q6_K weight, 0 for Q4_K
  int start[4];
};

namespace qmm {
template <typename T>
__device__ __forceinline__ T job3(const T (&a)[3], int j) {  // constant indices only (no scratch)
  return j == 0 ? a[0] : j == 1 ? a[1] : a[2];
}
}  // namespace qmm

extern "C" __global__ void __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
qmm_mmqs_multi(MmqsJobs jobs, const int8_t* __restrict__ xq, const float* __restrict__ xd,
               const int16_t* __restrict__ xs, int M, int K) {
  const int b = (int)blockIdx.x;
  const int j = b < jobs.start[1] ? 0 : b < jobs.start[2] ? 1 : 2;
  const int local = b - (j == 0 ? jobs.start[0] : j == 1 ? jobs.start[1] : jobs.start[2]);
  const int n = qmm::job3(jobs.n, j), gx = qmm::job3(jobs.gx, j), kc = qmm::job3(jobs.kc, j);
  const int tiles = gx * ((M + qmm::kSBM - 1) / qmm::kSBM);
  const int split = local / tiles, tile = local - split * tiles;
  const int mt = tile / gx, nt = tile - mt * gx;
  const int nbk = K / 256, kb0 = split * kc, kb1 = min(kb0 + kc, nbk);
  const uint8_t* w = qmm::job3(jobs.w, j);
  float* y = qmm::job3(jobs.y, j) + (size_t)split * M * n;
  if (qmm::job3(jobs.q6, j))
    qmm::mmqs6_q6k_at<false>(w, qmm::split_scales<qmm::kFmtQ6K>(w, n, K), xq, xd, y, M, n, K, n, nullptr, 0,
                             mt * qmm::kSBM, nt * qmm::kSBN, kb0, kb1);
  else {
    qmm::f32x16 acc[qmm::kSTM];
    qmm::mmqs_run<false>(w, xq, xd, xs, M, n, K, mt * qmm::kSBM, nt * qmm::kSBN, kb0, kb1, nullptr, acc);
    qmm::mmqs_store(acc, y, M, n, n, mt * qmm::kSBM, nt * qmm::kSBN, 0);
  }
}

extern "C" __global__ void __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
qmm_mmqs_q4k_sk(const uint8_t* __restrict__ wq, const int8_t* __restrict__ xq, const float* __restrict__ xd,
                const int16_t* __restrict__ xs, float* __restrict__ y, int M, int N, int K, int ldy, int accumulate,
                int gy, int T, int sk_tiles, float* __restrict__ part, unsigned* __restrict__ counters) {
  qmm::mmqs_q4k_sk(wq, xq, xd, xs, y, M, N, K, ldy, accumulate, gy, T, sk_tiles, part, counters);
}

// counters[0..n) = 0 (the stream-K GEMM's tile counters, before its launch)
extern "C" __global__ void __launch_bounds__(256) qmm_zero_u32(unsigned* __restrict__ p, int n) {
  for (int i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256) p[i] = 0u;
}

#define QMM_MMQ4_KERNEL(BN)                                                                                    \
  extern "C" __global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))                 \
      qmm_mmq4_q4k_n##BN(const uint8_t* __restrict__ wq, const int8_t* __restrict__ xq,                        \
                         const float* __restrict__ xd, const int16_t* __restrict__ xs, float* __restrict__ y,   \
                         int M, int N, int K, int ldy, int* __restrict__ dump, int accumulate, int remap,       \
                         int kc, long long ysplit) {                                                            \
    const qmm::KRange kr = qmm::split_range(K, kc);                                                            \
    qmm::mmq4_q4k<BN, false>(wq, xq, xd, xs, y + blockIdx.z * ysplit, M, N, K, ldy, dump, accumulate, remap,   \
                             kr.kb0, kr.kb1);                                                                  \
  }                                                                                                            \
  extern "C" __global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))                 \
      qmm_mmq4_q4k_n##BN##_dump(const uint8_t* __restrict__ wq, const int8_t* __restrict__ xq,                 \
                                const float* __restrict__ xd, const int16_t* __restrict__ xs,                  \
                                float* __restrict__ y, int M, int N, int K, int ldy, int* __restrict__ dump,    \
                                int accumulate, int remap, int kc, long long ysplit) {                         \
    const qmm::KRange kr = qmm::split_range(K, kc);                                                            \
    qmm::mmq4_q4k<BN, true>(wq, xq, xd, xs, y + blockIdx.z * ysplit, M, N, K, ldy, dump, accumulate, remap,    \
                            kr.kb0, kr.kb1);                                                                   \
  }
QMM_MMQ4_KERNEL(128)
QMM_MMQ4_KERNEL(64)

#define QMM_MMQ2_KERNEL(BM, BN)                                                                                \
  extern "C" __global__ void __launch_bounds__(BM * BN / 32) __attribute__((amdgpu_waves_per_eu(2 * 64 / BM)))     \
      qmm_mmq2_q4k_m##BM##_n##BN(                                                                            \
      const uint8_t* __restrict__ wq, const int8_t* __restrict__ xq, const float* __restrict__ xd,           \
      const int16_t* __restrict__ xs, float* __restrict__ y, int M, int N, int K, int ldy,                   \
      int* __restrict__ dump, int accumulate, int remap, int kc, long long ysplit) {                         \
    const qmm::KRange kr = qmm::split_range(K, kc);                                                          \
    qmm::mmq2_q4k<BM, BN, false>(wq, xq, xd, xs, y + blockIdx.z * ysplit, M, N, K, ldy, dump, accumulate,    \
                                 remap, kr.kb0, kr.kb1);                                                      \
  }                                                                                                          \
  extern "C" __global__ void __launch_bounds__(BM * BN / 32) qmm_mmq2_q4k_m##BM##_n##BN##_dump(              \
      const uint8_t* __restrict__ wq, const int8_t* __restrict__ xq, const float* __restrict__ xd,           \
      const int16_t* __restrict__ xs, float* __restrict__ y, int M, int N, int K, int ldy,                   \
      int* __restrict__ dump, int accumulate, int remap, int kc, long long ysplit) {                         \
    const qmm::KRange kr = qmm::split_range(K, kc);                                                          \
    qmm::mmq2_q4k<BM, BN, true>(wq, xq, xd, xs, y + blockIdx.z * ysplit, M, N, K, ldy, dump, accumulate,     \
                                remap, kr.kb0, kr.kb1);                                                       \
  }

QMM_MMQ2_KERNEL(128, 128)
QMM_MMQ2_KERNEL(64, 128)
QMM_MMQ2_KERNEL(64, 64)

// Split-K sum: y[m, n] (+)= part[0][m, n] + ... + part[splits - 1][m, n], in
// split order (partials [splits][M][N], row stride N).
extern "C" __global__ void __launch_bounds__(256) qmm_splitk_sum(const float* __restrict__ part, int splits, int M,
                                                                 int N, float* __restrict__ y, int ldy,
                                                                 int accumulate) {
  const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
  if (i >= (long long)M * N) return;
  const int m = (int)(i / N), n = (int)(i - (long long)m * N);
  const size_t plane = (size_t)M * N;
  float s = part[i];
  for (int k = 1; k < splits; ++k) s += part[i + k * plane];
  float* yp = y + (size_t)m * ldy + n;
  *yp = accumulate ? *yp + s : s;
}
