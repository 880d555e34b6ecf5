// Multi-token GEMV on the int8 matrix cores: 2..16 activation rows against a
// k-quant weight, the expert GEMV of the MoE FFN and the dense small-batch
// GEMV (the reference's mmvq for batch 2..8, mmvq_gguf.cu:725-807, and the
// MoE expert GEMV, moe/moe_gguf.cu).
//
// The token-interleaved VALU kernels (moe_gemv1, gemv_rows) read every staged
// activation block from LDS once per token and weight slice, so at eight
// tokens each 2.3 KB of Q4_K weight pulls 32 KB through LDS, and their time
// grows with the tokens rather than with the bytes. Here one
// v_mfma_i32_16x16x64_i8 takes 16 token rows (A, M = 16) against 16 weight
// rows (B, N = 16) over 64 elements of K:
//   * lane l = 16 q + n holds weight row n's quarter q of a super-block (the
//     same 32 quant bytes and 16-element chunks as the one-row kernels:
//     chunk c of quarter q is elements 64 q + 16 c) and token n's activation
//     at those elements; D lane l holds tokens 4 q + i (i < 4) of weight row n;
//   * Q4_K: the sub-block scale of a lane's chunk is split as sc = 8 sh + sl
//     (both in [0, 7]) and multiplied into the weight bytes (sl * q, sh * q
//     fit int8), so isd = MFMA-sum(x, sl q) + 8 MFMA-sum(x, sh q) exactly; the
//     mins term ism = sum_j m_j S_j is two more MFMAs over the activation's
//     32-element sums split as S = 64 hi + lo (lo in [0, 63], |hi| <= 64);
//   * the block value dx * q4k_combine(d, dmin, isd, ism) is the one-row
//     kernels' (the same integers and f32 sequence per block), accumulated
//     over the blocks in order; the MFMA does the reduction over K, so no
//     cross-lane sum is left.
// The activation rows are staged once per workgroup (quants at a row stride
// of K + 16 bytes: the 16 token rows of one ds_read_b128 fall on distinct
// banks), with per-block f32 scales and the split sums.
#pragma once

#include "qmm_common.h"
#include "qmm_gemv_kernels.h"
#include "qmm_mmq_kernels.h"

namespace qmm {

typedef int i32x4m __attribute__((ext_vector_type(4)));

__device__ __forceinline__ i32x4m mfma_16x64(uint4 a, uint4 b, i32x4m c) {
  return __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(i32x4m, a), __builtin_bit_cast(i32x4m, b), c, 0, 0,
                                               0);
}

// LDS of the staged activation: quants [mt][K + 16], split 32-sums
// [nb][16][16 B] (lo[8] | hi[8]), scales [nb][16] f32.
__device__ __forceinline__ int gemvm_stride(int K) { return K + 16; }

// Stage mr (<= 16) Q8_K activation rows (nb blocks each, row stride xrow
// bytes) into LDS.
template <int NW>
__device__ __forceinline__ void gemvm_stage(const uint8_t* __restrict__ xs, long long xrow, int mr, int nb, int K,
                                            uint8_t* lds) {
  const int stride = gemvm_stride(K), nthr = 64 * NW;
  uint8_t* sums = lds + (size_t)mr * stride;
  float* dx = reinterpret_cast<float*>(sums + 256 * nb);
  // the first (row, block)'s sums and scale are loaded with the quants (one
  // memory round trip for both)
  const int nsb = mr * nb;
  uint32_t bs0[8];
  float d0 = 0.0f;
  if ((int)threadIdx.x < nsb) {
    const int t = threadIdx.x / nb, b = threadIdx.x - t * nb;
    const uint8_t* src = xs + t * xrow + (size_t)kQ8KBytes * b;
    const uint32_t* bs = reinterpret_cast<const uint32_t*>(src + 4 + 256);
#pragma unroll
    for (int j = 0; j < 8; ++j) bs0[j] = bs[j];
    d0 = *reinterpret_cast<const float*>(src);
  }
  auto put_sums = [&](int i, const uint32_t* bs, float d) {
    const int t = i / nb, b = i - t * nb;
    uint32_t lo[2] = {0u, 0u}, hi[2] = {0u, 0u};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint32_t pr = bs[j];
      const int S = (int)(int16_t)(pr & 0xffffu) + ((int)pr >> 16);  // 32-element sum, |S| <= 4096
      lo[j >> 2] |= (uint32_t)(S & 63) << (8 * (j & 3));
      hi[j >> 2] |= (uint32_t)((S >> 6) & 0xff) << (8 * (j & 3));
    }
    *reinterpret_cast<uint4*>(sums + 16 * (16 * b + t)) = make_uint4(lo[0], lo[1], hi[0], hi[1]);
    dx[16 * b + t] = d;
  };
  // quants: 16-byte pieces (4-byte aligned in the Q8_K blocks, so dword
  // loads), eight per thread in flight before their stores
  const int per = 16 * nb, tot = mr * per;
  for (int i0 = threadIdx.x; i0 < tot; i0 += 8 * nthr) {
    uint4 v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int i = i0 + u * nthr;
      if (i < tot) {
        const int t = i / per, r = i - t * per, b = r >> 4, p = r & 15;
        const uint32_t* src = reinterpret_cast<const uint32_t*>(xs + t * xrow + (size_t)kQ8KBytes * b + 4 + 16 * p);
        v[u] = make_uint4(src[0], src[1], src[2], src[3]);
      }
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int i = i0 + u * nthr;
      if (i < tot) {
        const int t = i / per, r = i - t * per;
        *reinterpret_cast<uint4*>(lds + (size_t)t * stride + r * 16) = v[u];
      }
    }
  }
  if ((int)threadIdx.x < nsb) put_sums(threadIdx.x, bs0, d0);
  for (int i = threadIdx.x + nthr; i < nsb; i += nthr) {  // more (row, block) pairs than threads
    const int t = i / nb, b = i - t * nb;
    const uint8_t* src = xs + t * xrow + (size_t)kQ8KBytes * b;
    const uint32_t* bs = reinterpret_cast<const uint32_t*>(src + 4 + 256);  // 16 int16 16-element sums
    uint32_t v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = bs[j];
    put_sums(i, v, *reinterpret_cast<const float*>(src));
  }
}

// One weight (or a gate | up pair: rows >= N are weight 1's) for the pass.
struct GvmJob {
  const uint8_t* wb0;  // first row body of weight 0 / 1
  const uint8_t* wb1;
  const uint16_t* db0;  // first separated f16 scale of weight 0 / 1 (Q6_K)
  const uint16_t* db1;
  float* y0;
  float* y1;
  int N, total, nb, ldy, accumulate;
  uint32_t rowb;   // row body bytes
  long long yrow;  // first output row of the pass's tokens
};

// Weight row groups (16 rows each) slot0, slot0 + sstep, ... of the job for
// wave slot0's workgroup: wave w takes slot slot0 + w. `stage` stages the
// activation (all threads) once the first weight loads are in flight. P
// slices (one super-block of the lane's row) in flight per wave.
template <int FMT, int NW, int P, typename Stage>
__device__ __forceinline__ void gemvm_rows(const GvmJob& a, int mr, int slot0, int sstep, uint8_t* lds,
                                           Stage stage) {
#pragma clang fp contract(off)
  static_assert(FMT == kFmtQ4K, "Q4_K weights");
  const int lane = threadIdx.x & 63, n = lane & 15, q = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int sl = slot0 + wave;
  const int nb = a.nb, total = a.total;
  const int ngrp = (total + 15) >> 4;
  const int ngw = sl < ngrp ? (ngrp - 1 - sl) / sstep + 1 : 0;  // this wave's groups
  const int nslices = ngw * nb;
  const int stride = gemvm_stride(256 * nb);

  // issue side: slice s = (group k, block b). Every step issues a load (past
  // the last slice it reloads that slice, and those compute steps store
  // nothing): a load issued under a condition leaves the compiler's wait
  // counts assuming no later load is in flight, which drains the ring at
  // every use.
  int is_s = 0, is_k = 0, is_b = 0;
  WSlice ring[P];
  auto issue = [&](WSlice& w) {
    const int row = min((sl + is_k * sstep) * 16 + n, total - 1);
    const int j = row >= a.N ? 1 : 0;
    const uint32_t r = (uint32_t)(row - j * a.N);
    const uint8_t* wrow = (j ? a.wb1 : a.wb0) + (size_t)r * a.rowb;
    const uint16_t* drow = (j ? a.db1 : a.db0) + (size_t)r * nb;
    load_slice<FMT>(w, wrow, drow, (uint32_t)is_b, q);
    if (is_s + 1 < nslices) {
      if (++is_b == nb) {
        is_b = 0;
        ++is_k;
      }
      ++is_s;
    }
  };
  if (nslices > 0) {
#pragma unroll
    for (int u = 0; u < P; ++u) issue(ring[u]);
  }
  stage();
  __syncthreads();
  if (nslices == 0) return;

  const uint8_t* sums = lds + (size_t)mr * stride;
  const float* dxs = reinterpret_cast<const float*>(sums + 256 * nb);
  const int tc = min(n, mr - 1);  // this lane's token row for the A operand (rows past mr are never stored)
  const uint8_t* arow = lds + (size_t)tc * stride + 64 * q;
  const i32x4m zero = {0, 0, 0, 0};
  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  int c_k = 0, c_b = 0;
  for (int s0 = 0; s0 < nslices; s0 += P) {
#pragma unroll
    for (int u = 0; u < P; ++u) {
      const bool live = s0 + u < nslices;
      const WSlice& s = ring[u];
      const int b = c_b;
      // weight side: nibbles of the lane's chunks, split scales, mins bytes
      const uint4 nib[4] = {lo_nib(s.b), lo_nib(s.c), hi_nib(s.b), hi_nib(s.c)};
      const float dw = h2f(s.a.x), dm = h2f(s.a.x >> 16);
      const int sh = (q & 1) * 16;
      const uint32_t A = s.a.y >> sh, B = s.a.z >> sh, C = s.a.w >> sh;
      const uint32_t scp = q >= 2 ? ((C & 0x0f0fu) | ((A >> 2) & 0x3030u)) : (A & 0x3f3fu);
      (void)B;
      const uint32_t sc0 = scp & 0xffu, sc1 = (scp >> 8) & 0xffu;  // sub-blocks 2q, 2q + 1
      const uint32_t spl[2] = {(sc0 & 7u) * 0x10001u, (sc1 & 7u) * 0x10001u};
      const uint32_t sph[2] = {(sc0 >> 3) * 0x10001u, (sc1 >> 3) * 0x10001u};
      const uint32_t mn0 = s.a.z & 0x3f3f3f3fu, mn1 = ((s.a.w >> 4) & 0x0f0f0f0fu) | ((s.a.z >> 2) & 0x30303030u);
      const uint4 z4 = make_uint4(0u, 0u, 0u, 0u);
      const uint4 bml = q == 0 ? make_uint4(mn0, mn1, 0u, 0u) : z4;
      const uint4 bmh = q == 0 ? make_uint4(0u, 0u, mn0, mn1) : z4;
      // activation side
      const uint8_t* ap = arow + 256 * b;
      const uint4 asum = q == 0 ? *reinterpret_cast<const uint4*>(sums + 16 * (16 * b + tc)) : z4;
      i32x4m accl = zero, acch = zero;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const uint4 av = *reinterpret_cast<const uint4*>(ap + 16 * c);
        const i8x16 wl = bytes_times4p(nib[c], spl[c >> 1]);
        const i8x16 wh = bytes_times4p(nib[c], sph[c >> 1]);
        accl = mfma_16x64(av, __builtin_bit_cast(uint4, wl), accl);
        acch = mfma_16x64(av, __builtin_bit_cast(uint4, wh), acch);
      }
      const i32x4m ml = mfma_16x64(asum, bml, zero), mh = mfma_16x64(asum, bmh, zero);
      const float4 dx = *reinterpret_cast<const float4*>(dxs + 16 * b + 4 * q);
      const float dxv[4] = {dx.x, dx.y, dx.z, dx.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int isd = accl[i] + (acch[i] << 3), ism = ml[i] + (mh[i] << 6);
        acc[i] += dxv[i] * q4k_combine(dw, dm, isd, ism);
      }
      if (++c_b == nb) {
        const int row = (sl + c_k * sstep) * 16 + n;
        if (live && row < total) {
          const int j = row >= a.N ? 1 : 0;
          float* yb = (j ? a.y1 : a.y0) + (row - j * a.N);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int t = 4 * q + i;
            if (t < mr) {
              float* yp = yb + (size_t)(a.yrow + t) * a.ldy;
              *yp = a.accumulate ? *yp + acc[i] : acc[i];
            }
          }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i] = 0.0f;
        c_b = 0;
        ++c_k;
      }
      issue(ring[u]);
    }
  }
}

// MoE expert GEMV on the matrix cores: grid (G, passes); pass y is tokens
// mt y .. mt y + mt - 1 of every expert holding more than mt y of them, and
// the pass's G workgroups are shared out over those experts as in moe_gemv1.
// Same arguments as qmm_moe_gemv1 plus mt.
template <int FMT, int NW, int P>
__device__ __forceinline__ void moe_gemvm(const uint8_t* __restrict__ w0, const uint8_t* __restrict__ w1, int njobs,
                                          int N, int E, float* __restrict__ y0, float* __restrict__ y1, int ldy,
                                          const uint8_t* __restrict__ xq, long long xrow,
                                          const int* __restrict__ counts, const int* __restrict__ offsets, int K,
                                          int mt) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  __shared__ int act[256];
  __shared__ int nact;
  const int lane = threadIdx.x & 63;
  const int mc = mt * (int)blockIdx.y;
  if (threadIdx.x < 64) {
    int base = 0;
    for (int e0 = 0; e0 < E; e0 += 64) {
      const bool a = e0 + lane < E && counts[e0 + lane] > mc;
      const unsigned long long msk = __ballot(a);
      if (a) act[base + __popcll(msk & ((1ull << lane) - 1ull))] = e0 + lane;
      base += __popcll(msk);
    }
    if (lane == 0) nact = base;
  }
  __syncthreads();
  const int na = __builtin_amdgcn_readfirstlane(nact);
  if (na == 0) return;
  const long long G = gridDim.x;
  const int slot = (int)((long long)blockIdx.x * na / G);
  const int first = (int)(((long long)slot * G + na - 1) / na);
  const int next = (int)(((long long)(slot + 1) * G + na - 1) / na);
  const int e = __builtin_amdgcn_readfirstlane(act[slot]), bx = (int)blockIdx.x - first, gx = next - first;
  const int me = __builtin_amdgcn_readfirstlane(counts[e]);
  const int off = __builtin_amdgcn_readfirstlane(offsets[e]);
  const int nb = K / 256;
  const int mr = min(mt, me - mc);
  GvmJob j;
  const size_t rowb = (size_t)nb * FmtInfo<FMT>::kBodyBytes, erow = (size_t)e * N, trows = (size_t)E * N;
  j.wb0 = w0 + erow * rowb;
  j.wb1 = w1 + erow * rowb;
  j.db0 = reinterpret_cast<const uint16_t*>(w0 + trows * rowb) + erow * nb;
  j.db1 = reinterpret_cast<const uint16_t*>(w1 + trows * rowb) + erow * nb;
  j.y0 = y0;
  j.y1 = y1;
  j.N = N;
  j.total = njobs * N;
  j.nb = nb;
  j.ldy = ldy;
  j.accumulate = 0;
  j.rowb = (uint32_t)rowb;
  j.yrow = off + mc;
  const uint8_t* xs = xq + (size_t)(off + mc) * xrow;
  gemvm_rows<FMT, NW, P>(j, mr, bx * NW, gx * NW, lds, [&] { gemvm_stage<NW>(xs, xrow, mr, nb, K, lds); });
}

// Dense GEMV of m (2..16) staged Q8_K activation rows against one weight.
template <int FMT, int NW, int P>
__device__ __forceinline__ void gemv_rowsm(const uint8_t* __restrict__ w, float* __restrict__ y, int ldy,
                                           const uint8_t* __restrict__ xq, int m, int K, int N, int accumulate) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int nb = K / 256;
  const size_t rowb = (size_t)nb * FmtInfo<FMT>::kBodyBytes;
  GvmJob j;
  j.wb0 = j.wb1 = w;
  j.db0 = j.db1 = reinterpret_cast<const uint16_t*>(w + (size_t)N * rowb);
  j.y0 = j.y1 = y;
  j.N = N;
  j.total = N;
  j.nb = nb;
  j.ldy = ldy;
  j.accumulate = accumulate;
  j.rowb = (uint32_t)rowb;
  j.yrow = 0;
  gemvm_rows<FMT, NW, P>(j, m, (int)blockIdx.x * NW, (int)gridDim.x * NW, lds,
                         [&] { gemvm_stage<NW>(xq, (long long)nb * kQ8KBytes, m, nb, K, lds); });
}

}  // namespace qmm

#define QMM_GEMVM_KERNELS(FMT, NAME, NW, P)                                                                     \
  extern "C" __global__ void __launch_bounds__(64 * NW)                                                         \
      qmm_moe_gemvm_##NAME##_w##NW##_p##P(const uint8_t* w0, const uint8_t* w1, int njobs, int N, int E, float* y0, float* y1, \
                           int ldy, const uint8_t* __restrict__ xq, long long xrow,                            \
                           const int* __restrict__ counts, const int* __restrict__ offsets, int K, int mt) {   \
    qmm::moe_gemvm<FMT, NW, P>(w0, w1, njobs, N, E, y0, y1, ldy, xq, xrow, counts, offsets, K, mt);            \
  }                                                                                                             \
  extern "C" __global__ void __launch_bounds__(64 * NW)                                                         \
      qmm_gemv_rowsm_##NAME##_w##NW##_p##P(const uint8_t* __restrict__ w, float* __restrict__ y, int ldy,                     \
                            const uint8_t* __restrict__ xq, int m, int K, int N, int accumulate) {             \
    qmm::gemv_rowsm<FMT, NW, P>(w, y, ldy, xq, m, K, N, accumulate);                                           \
  }
QMM_GEMVM_KERNELS(qmm::kFmtQ4K, q4k, 4, 4)
