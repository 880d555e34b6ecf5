// Mixture-of-experts FFN at decode batch sizes (config 5 of the benchmark):
// routing, per-expert gathered GEMVs over stacked expert weights, SiLU*mul
// and the weighted scatter back to tokens, all on the device.
//
// Host semantics followed: MoeMlp::forward (crates/llm/candle-llm/src/models/llama.rs:1416-1487):
// softmax over the router logits, top-k by probability, weights renormalised
// over the selected experts, each expert's LlamaMlp (gate, up, silu(gate)*up,
// down) on its tokens, outputs scaled by the weight and index_add-ed back in
// increasing expert order. The CUDA kernel the expert GEMV replaces is
// moe_gemm_gguf (candle-kernels/src/moe/moe_gguf.cu:56-216).
#pragma once

#include "qmm_common.h"
#include "qmm_gemv_kernels.h"
#include "qmm_gemv1p_kernels.h"
#include "qmm_quant_kernels.h"

// Routing: logits f32 [T][E] -> per-expert lists of (token, weight) pairs,
// experts in increasing order, tokens in increasing order within an expert.
//   counts[e], offsets[e] (exclusive prefix, offsets[E] = T*k),
//   pair_token[p], pair_weight[p] for p in [offsets[e], offsets[e] + counts[e]),
//   token_pairs[t*k + s] = the pairs of token t in increasing expert order.
// One workgroup of four waves; T <= 4096, T*k <= 8192, E <= 256, k <= 8.
// Pass 1: each thread routes tokens (softmax, top-k) into LDS and counts the
// selections per expert; the offsets are the exclusive prefix of the counts.
// Pass 2: each wave takes experts e = wave, wave + 4, ... and walks the tokens
// 64 at a time: a ballot of the lanes whose token selected e ranks them, so
// pair p = offsets[e] + (pairs of e so far) + (selecting lanes below).
extern "C" __global__ void __launch_bounds__(256) qmm_moe_route(const float* __restrict__ logits, int T, int E,
                                                                int k, int renorm, int* __restrict__ counts,
                                                                int* __restrict__ offsets,
                                                                int* __restrict__ pair_token,
                                                                float* __restrict__ pair_weight,
                                                                int* __restrict__ token_pairs) {
#pragma clang fp contract(off)
  constexpr int kThreads = 256, kWaves = kThreads / 64;
  __shared__ short sel_e[8192];
  __shared__ float sel_w[8192];
  __shared__ int ecount[256];
  __shared__ int eoff[257];
  for (int e = threadIdx.x; e < E; e += kThreads) ecount[e] = 0;
  __syncthreads();
  for (int t = threadIdx.x; t < T; t += kThreads) {
    const float* l = logits + (size_t)t * E;
    float mx = l[0];
    for (int e = 1; e < E; ++e) mx = fmaxf(mx, l[e]);
    float sum = 0.0f;
    for (int e = 0; e < E; ++e) sum += expf(l[e] - mx);
    // top-k by probability (highest first, lowest expert index on ties)
    unsigned long long taken[4] = {0, 0, 0, 0};
    float denom = 0.0f;
    float p[8];
    int ids[8];
    for (int s = 0; s < k; ++s) {
      int best = -1;
      float bp = 0.0f;
      for (int e = 0; e < E; ++e) {
        if ((taken[e >> 6] >> (e & 63)) & 1ull) continue;
        const float pe = expf(l[e] - mx) / sum;
        if (best < 0 || pe > bp) {
          best = e;
          bp = pe;
        }
      }
      taken[best >> 6] |= 1ull << (best & 63);
      ids[s] = best;
      p[s] = bp;
      denom += bp;
    }
    denom = fmaxf(denom, 1.17549435e-38f);
    for (int s = 0; s < k; ++s) {
      sel_e[t * k + s] = (short)ids[s];
      sel_w[t * k + s] = renorm ? p[s] / denom : p[s];
      atomicAdd(&ecount[ids[s]], 1);
    }
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    int pos = 0;
    for (int e = 0; e < E; ++e) {
      eoff[e] = pos;
      pos += ecount[e];
    }
    eoff[E] = pos;
  }
  __syncthreads();
  for (int e = threadIdx.x; e <= E; e += kThreads) {
    offsets[e] = eoff[e];
    if (e < E) counts[e] = ecount[e];
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  for (int e = wave; e < E; e += kWaves) {
    int base = eoff[e];
    for (int t0 = 0; t0 < T; t0 += 64) {
      const int t = t0 + lane;
      int slot = -1, before = 0;
      if (t < T)
        for (int s = 0; s < k; ++s) {
          const int es = sel_e[t * k + s];
          if (es == e) slot = s;
          before += es < e;
        }
      const unsigned long long m = __ballot(slot >= 0);
      if (slot >= 0) {
        const int pr = base + __popcll(m & ((1ull << lane) - 1ull));
        pair_token[pr] = t;
        pair_weight[pr] = sel_w[t * k + slot];
        token_pairs[t * k + before] = pr;  // the token's pairs in increasing expert order
      }
      base += __popcll(m);
    }
  }
}

// f32 row gather: out row i = x[rows[i]] (k columns).
extern "C" __global__ void qmm_gather_rows(const float* __restrict__ x, long long ldx, const int* __restrict__ rows,
                                           float* __restrict__ out, int k, int nrows) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long long)nrows * k) return;
  const int r = (int)(i / k), c = (int)(i % k);
  out[i] = x[(long long)rows[r] * ldx + c];
}

// Q8_K quantization of gathered rows: out row i = quantize(x[rows[i]]).
extern "C" __global__ void __launch_bounds__(256) qmm_quantize_q8k_gather(const float* __restrict__ x,
                                                                          long long ldx,
                                                                          const int* __restrict__ rows,
                                                                          uint8_t* __restrict__ y, int k,
                                                                          int nrows) {
  const int nb = k / 256;
  const long long w = (long long)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (w >= (long long)nrows * nb) return;
  const int i = (int)(w / nb), b = (int)(w % nb);
  qmm::q8k_block(x + (long long)rows[i] * ldx + 256LL * b, y + w * qmm::kQ8KBytes, threadIdx.x & 63);
}

// h = silu(g) * u, elementwise over [rows][k] (ld = row stride of g, u, h),
// with silu(v) = v / (1 + exp(-v)) as the reference's f32 op.
extern "C" __global__ void qmm_silu_mul(const float* __restrict__ g, const float* __restrict__ u,
                                        float* __restrict__ h, long long n) {
#pragma clang fp contract(off)
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  h[i] = qmm::silu_mul(g[i], u[i]);
}

// out[t][n] = sum over the pairs of token t (in increasing expert order) of
// weight * y_pair[n], accumulated from zero like index_add.
extern "C" __global__ void qmm_moe_combine(const float* __restrict__ yp, const float* __restrict__ pair_weight,
                                           const int* __restrict__ token_pairs, int T, int k, int N,
                                           float* __restrict__ out, int ldo) {
#pragma clang fp contract(off)
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long long)T * N) return;
  const int t = (int)(i / N), n = (int)(i % N);
  float acc = 0.0f;
  for (int s = 0; s < k; ++s) {
    const int p = token_pairs[t * k + s];
    const float v = yp[(size_t)p * N + n] * pair_weight[p];
    acc = acc + v;
  }
  out[(size_t)t * ldo + n] = acc;
}

// Expert-grouped GEMV: blockIdx.y = expert e; its counts[e] token rows (up to
// 8 per pass) of pre-quantized activations start at row offsets[e] of xq.
// Weights are stacked [E*N, K] tensors (njobs of them, e.g. gate and up);
// expert e uses rows [e*N, e*N + N). Outputs y_j[(offsets[e] + m) * ldy + n].
// Experts without tokens exit before reading any weight.
template <int FMT, int U>
__device__ __forceinline__ void moe_gemv(const uint8_t* w0, const uint8_t* w1, int njobs, int N, int E, float* y0,
                                         float* y1, int ldy, const uint8_t* __restrict__ xq, long long xrow,
                                         const int* __restrict__ counts, const int* __restrict__ offsets, int K) {
  const int e = blockIdx.y;
  const int me = counts[e];
  if (me == 0) return;
  const int off = offsets[e];
  for (int mc = 0; mc < me; mc += 8) {
    if (mc > 0) __syncthreads();
    qmm::GemvJobs jobs;
#pragma unroll
    for (int j = 0; j < qmm::kMaxJobs; ++j) {
      jobs.wq[j] = j == 0 ? w0 : j == 1 ? w1 : nullptr;
      jobs.y[j] = j == 0 ? y0 + (size_t)(off + mc) * ldy : j == 1 ? y1 + (size_t)(off + mc) * ldy : nullptr;
      jobs.rows[j] = j < 2 ? N : 0;
      jobs.ldy[j] = ldy;
      jobs.row0[j] = j < 2 ? e * N : 0;
      jobs.trows[j] = j < 2 ? E * N : 0;
    }
    jobs.njobs = njobs;
    jobs.total = njobs * N;
    const int mrows = me - mc < 8 ? me - mc : 8;
    qmm::gemv<FMT, 8, 1, U, false, qmm::kMaxJobs, false, 8>(jobs, xq + (size_t)(off + mc) * xrow, 0, K, nullptr, mrows);
  }
}

// Expert-grouped GEMV for k-quant weights, one row per wave at a time with a
// prefetch ring (the gemv1p structure): blockIdx.y = expert e, whose
// counts[e] token rows (8 per pass) are staged in LDS once per workgroup; a
// wave's weight slice is unpacked once (prep_w) and multiplied with each
// token row, and each row's outputs are stored by lanes 0..rows-1 together.
// The per-token accumulators are eight scalars, so register use stays at the
// one-row kernels' level (the generic M = 8 GEMV keeps eight activation
// slices live and spills at these shapes). Experts without tokens exit at once.
template <int FMT, int P, int NW>
__device__ __forceinline__ void moe_gemv1(const uint8_t* __restrict__ w0, const uint8_t* __restrict__ w1, int njobs,
                                          int N, int E, float* __restrict__ y0, float* __restrict__ y1, int ldy,
                                          const uint8_t* __restrict__ xq, long long xrow,
                                          const int* __restrict__ counts, const int* __restrict__ offsets, int K) {
  using namespace qmm;
  static_assert(FMT != kFmtQ80, "k-quant weights");
  constexpr int BPI = 16;
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  // The grid is shared out over the experts that have tokens: active
  // expert s (in expert order) gets workgroups [ceil(s G / na), ceil((s + 1) G / na))
  // of the G in the grid (G >= E), so every workgroup streams weights, however
  // many experts are idle.
  __shared__ int act[256];
  __shared__ int nact;
  const int lane = threadIdx.x & 63, l = lane & 3, g = lane >> 2;
  if (threadIdx.x < 64) {
    int base = 0;
    for (int e0 = 0; e0 < E; e0 += 64) {
      const bool a = e0 + lane < E && counts[e0 + lane] > 0;
      const unsigned long long msk = __ballot(a);
      if (a) act[base + __popcll(msk & ((1ull << lane) - 1ull))] = e0 + lane;
      base += __popcll(msk);
    }
    if (lane == 0) nact = base;
  }
  __syncthreads();
  const int na = nact;
  if (na == 0) return;
  const long long G = gridDim.x;
  const int slot = (int)((long long)blockIdx.x * na / G);
  const int first = (int)(((long long)slot * G + na - 1) / na);
  const int next = (int)(((long long)(slot + 1) * G + na - 1) / na);
  const int e = act[slot], bx = (int)blockIdx.x - first, gx = next - first;
  const int me = counts[e];
  const int off = offsets[e];
  const int nb = K / 256, niter = (nb + BPI - 1) / BPI;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int total = njobs * N;
  const int row_step = gx * NW;
  const int row0 = bx * NW + wave;
  const int nrows = row0 < total ? (total - 1 - row0) / row_step + 1 : 0;
  const int nslices = nrows * niter;
  const size_t rowb = (size_t)nb * FmtInfo<FMT>::kBodyBytes;
  const size_t trows = (size_t)E * N;
  for (int mc = 0; mc < me; mc += 8) {
    const int mr = min(8, me - mc);
    int is_s = 0, is_k = 0, is_it = 0;
    WSlice ring[P];
    auto issue = [&](WSlice& w) {
      const int gr = row0 + is_k * row_step;  // < total while is_s < nslices
      const int j = gr >= N ? 1 : 0;
      const uint8_t* wq = j ? w1 : w0;
      const size_t trow = (size_t)e * N + (gr - j * N);
      const uint8_t* wrow = wq + trow * rowb;
      const uint16_t* drow = reinterpret_cast<const uint16_t*>(wq + trows * rowb) + trow * nb;
      load_slice<FMT>(w, wrow, drow, (uint32_t)min(is_it * BPI + g, nb - 1), l);
      if (++is_it == niter) {
        is_it = 0;
        ++is_k;
      }
      ++is_s;
    };
#pragma unroll
    for (int u = 0; u < P; ++u)
      if (is_s < nslices) issue(ring[u]);
    if (mc > 0) __syncthreads();  // the previous pass's LDS reads are done
    stage_act<FMT, NW>(xq + (size_t)(off + mc) * xrow, mr * nb, lds);
    __syncthreads();
    float acc[8];
    int c_k = 0, c_it = 0;
    for (int s0 = 0; s0 < nslices; s0 += P) {
#pragma unroll
      for (int u = 0; u < P; ++u) {
        if (s0 + u < nslices) {
          const int b = c_it * BPI + g;
          const bool okb = b < nb;
          const int bx = okb ? b : 0;
          const WPrep wp = prep_w<FMT>(ring[u], l);
#pragma unroll
          for (int m = 0; m < 8; ++m) {
            if (m < mr) {  // wave-uniform
              XSlice x;
              load_x<FMT>(x, lds, mr * nb, m * nb + bx, l);
              int ia, ib;
              float p = dot_wx<FMT>(wp, x, ia, ib);
              p = okb ? p : 0.0f;
              acc[m] = c_it == 0 ? p : acc[m] + p;
            }
          }
          if (++c_it == niter) {
            const int gr = row0 + c_k * row_step;
            const int j = gr >= N ? 1 : 0;
            float out = 0.0f;
#pragma unroll
            for (int m = 0; m < 8; ++m) {
              if (m < mr) {
                const float v = wave_total(acc[m]);
                out = lane == m ? v : out;
              }
            }
            if (lane < mr) (j ? y1 : y0)[(size_t)(off + mc + lane) * ldy + (gr - j * N)] = out;
            c_it = 0;
            ++c_k;
          }
        }
        if (is_s < nslices) issue(ring[u]);
      }
    }
  }
}

#define QMM_MOE1_KERNEL(FMT, NAME, P)                                                                           \
  extern "C" __global__ void __launch_bounds__(1024)                                                            \
      qmm_moe_gemv1_##NAME##_p##P(const uint8_t* w0, const uint8_t* w1, int njobs, int N, int E, float* y0,   \
                                  float* y1, int ldy, const uint8_t* __restrict__ xq, long long xrow,           \
                                  const int* __restrict__ counts, const int* __restrict__ offsets, int K) {    \
    moe_gemv1<FMT, P, 16>(w0, w1, njobs, N, E, y0, y1, ldy, xq, xrow, counts, offsets, K);                     \
  }
QMM_MOE1_KERNEL(qmm::kFmtQ4K, q4k, 1)
QMM_MOE1_KERNEL(qmm::kFmtQ4K, q4k, 2)
QMM_MOE1_KERNEL(qmm::kFmtQ6K, q6k, 1)
QMM_MOE1_KERNEL(qmm::kFmtQ6K, q6k, 2)

#define QMM_MOE_KERNEL(FMT, NAME, U)                                                                          \
  extern "C" __global__ void __launch_bounds__(512)                                                           \
      qmm_moe_gemv_##NAME##_u##U(const uint8_t* w0, const uint8_t* w1, int njobs, int N, int E, float* y0,  \
                                 float* y1, int ldy, const uint8_t* __restrict__ xq, long long xrow,          \
                                 const int* __restrict__ counts, const int* __restrict__ offsets, int K) {   \
    moe_gemv<FMT, U>(w0, w1, njobs, N, E, y0, y1, ldy, xq, xrow, counts, offsets, K);                        \
  }

QMM_MOE_KERNEL(qmm::kFmtQ4K, q4k, 1)
QMM_MOE_KERNEL(qmm::kFmtQ4K, q4k, 2)
QMM_MOE_KERNEL(qmm::kFmtQ6K, q6k, 1)
QMM_MOE_KERNEL(qmm::kFmtQ6K, q6k, 2)
QMM_MOE_KERNEL(qmm::kFmtQ80, q8_0, 1)
QMM_MOE_KERNEL(qmm::kFmtQ80, q8_0, 2)

// ---------------------------------------------------------------------------
// MoE prefill: grouped GEMM over the expert-ordered pair rows (the grouped
// prefill of moe/moe_wmma_gguf.cu:124-354, here on the int8 MFMA GEMM tiles).
// blockIdx.z is the expert e; its rows are pairs offsets[e] ..
// offsets[e] + counts[e] - 1 of the activation planes and of y (row stride
// ldy), its weight rows e*N .. e*N + N - 1 of the stacked [E*N, K] tensor. An
// M tile past the expert's rows exits before any load, so every workgroup
// that runs computes exactly what the per-expert GEMM over that expert's
// gathered rows computes, in the same order.
// ---------------------------------------------------------------------------
namespace qmm {

// Planes of the expert's first row: int8 [row][K], scales [row][K/256] (Q8_K)
// or [row][K/32] (Q8_0), Q8_K 32-element sums [row][K/256][8].
struct GroupRows {
  const int8_t* xq;
  const float* xd;
  const int16_t* xs;
  float* y;
  int m;
};

template <int BM, bool Q80>
__device__ __forceinline__ bool group_rows(GroupRows& g, const int8_t* xq, const float* xd, const int16_t* xs,
                                           float* y, int K, int ldy, const int* __restrict__ counts,
                                           const int* __restrict__ offsets) {
  const int e = blockIdx.z;
  g.m = counts[e];
  if ((int)blockIdx.y * BM >= g.m) return false;
  const long long off = offsets[e];
  g.xq = xq + off * K;
  g.xd = xd + off * (Q80 ? K / 32 : K / 256);
  g.xs = xs + off * (K / 256) * 8;
  g.y = y + off * ldy;
  return true;
}

}  // namespace qmm

#define QMM_MOE_MMQ2_KERNEL(BM, SUFFIX)                                                                         \
  extern "C" __global__ void __launch_bounds__(BM * 4) __attribute__((amdgpu_waves_per_eu(2 * 64 / BM)))         \
      qmm_moe_mmq2_q4k##SUFFIX(const uint8_t* __restrict__ wq, const int8_t* __restrict__ xq,                   \
                               const float* __restrict__ xd, const int16_t* __restrict__ xs,                    \
                               float* __restrict__ y, int N, int K, int ldy, int E,                             \
                               const int* __restrict__ counts, const int* __restrict__ offsets) {               \
    qmm::GroupRows g;                                                                                           \
    if (!qmm::group_rows<BM, false>(g, xq, xd, xs, y, K, ldy, counts, offsets)) return;                         \
    const uint8_t* we = wq + (size_t)blockIdx.z * N * (K / 256) * qmm::kQ4KBytes;                               \
    qmm::mmq2_q4k<BM, 128, false>(we, g.xq, g.xd, g.xs, g.y, g.m, N, K, ldy, nullptr, 0, 0, 0, K / 256);        \
    (void)E;                                                                                                    \
  }
QMM_MOE_MMQ2_KERNEL(128, )
QMM_MOE_MMQ2_KERNEL(64, _m64)

#define QMM_MOE_MMQ_KERNEL(FMT, NAME)                                                                          \
  extern "C" __global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))                 \
      qmm_moe_mmq_##NAME(const uint8_t* __restrict__ wq, const int8_t* __restrict__ xq,                        \
                         const float* __restrict__ xd, const int16_t* __restrict__ xs, float* __restrict__ y,   \
                         int N, int K, int ldy, int E, const int* __restrict__ counts,                          \
                         const int* __restrict__ offsets) {                                                    \
    qmm::GroupRows g;                                                                                          \
    if (!qmm::group_rows<qmm::kMmqBM, FMT == qmm::kFmtQ80>(g, xq, xd, xs, y, K, ldy, counts, offsets)) return; \
    const int nbw = FMT == qmm::kFmtQ80 ? K / 32 : K / 256;                                                    \
    const size_t rows0 = (size_t)blockIdx.z * N;                                                               \
    const uint16_t* wd = qmm::split_scales<FMT>(wq, (long long)E * N, K) + rows0 * nbw;                        \
    const uint8_t* we = wq + rows0 * nbw * qmm::FmtInfo<FMT>::kBodyBytes;                                      \
    qmm::mmq<FMT, false>(we, wd, g.xq, g.xd, g.xs, g.y, g.m, N, K, ldy, nullptr, 0, 0, 0, K / 256);            \
  }
QMM_MOE_MMQ_KERNEL(qmm::kFmtQ6K, q6k)
QMM_MOE_MMQ_KERNEL(qmm::kFmtQ80, q8_0)
