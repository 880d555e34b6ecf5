// Decode GEMV for one activation row with a prefetch ring (gemv1p).
//
// A wave's work is a list of slices: its rows row0, row0 + row_step, ...,
// each cut into niter slices of 16 k-quant blocks (64 Q8_0 blocks), i.e. one
// wave-wide load of 2304 B (Q4_K) or 3360 B (Q6_K) of a row. The wave keeps
// P slices in flight: a ring of P register slices, each refilled with the
// slice P ahead as soon as it has been consumed. A launch that gives each
// wave at most P slices therefore has its whole weight stream in flight
// from the first instructions on, and the kernel time is one memory latency
// plus the transfer instead of one latency per row (gemv1 keeps one slice in
// flight, so a wave with four rows pays four round trips).
//
// The vector memory counter is in order, so the prologue issues the
// activation loads first (the f32 row and its RMSNorm weight, or the
// pre-quantized Q8_K items), then the ring, and only then waits for the
// activation: the quantization and LDS staging overlap the weight stream.
// Per-block arithmetic (prep_w / dot_wx), the LDS layouts, the summation
// order and the output path (outputs kept one per lane, written 64 at a time)
// are gemv1's, so results are bit-identical to it.
#pragma once

#include "qmm_gemv_kernels.h"

namespace qmm {

// One staged activation item per thread (the host guarantees 16 * nb <=
// threads): thread t stages chunk k = t & 3 of lane l = (t >> 2) & 3 of block
// t >> 4 of a GGML Q8_K row into stage_act's layout. Loads first
// (stage1_load), LDS writes later (stage1_store).
struct Stage1 {
  uint4 q;
  int s0, s1, s2, s3;
  float d;
};

template <int FMT>
__device__ __forceinline__ void stage1_load(Stage1& r, const uint8_t* __restrict__ xq, int nb) {
  static_assert(FMT != kFmtQ80, "k-quant activations");
  const int t = min((int)threadIdx.x, 16 * nb - 1);
  const int blk = t >> 4, l = (t >> 2) & 3, k = t & 3;
  const uint8_t* s = xq + (size_t)kQ8KBytes * blk;
  const uint32_t* q = reinterpret_cast<const uint32_t*>(s + 4 + act_chunk<FMT>(l, k));
  r.q = make_uint4(q[0], q[1], q[2], q[3]);
  const int16_t* bs = reinterpret_cast<const int16_t*>(s + 4 + 256);
  // the 16-element sums stage_act combines for this item
  const int k2 = 2 * (k & 1);
  r.s0 = bs[act_chunk<FMT>(l, k2) / 16];
  r.s1 = bs[act_chunk<FMT>(l, k2 + 1) / 16];
  r.s2 = bs[act_chunk<FMT>(l, 2) / 16];
  r.s3 = bs[act_chunk<FMT>(l, 3) / 16];
  r.d = *reinterpret_cast<const float*>(s);
}

template <int FMT>
__device__ __forceinline__ void stage1_store(const Stage1& r, int nb, uint8_t* lds) {
  const int t = threadIdx.x;
  if (t >= 16 * nb) return;
  const int blk = t >> 4, l = (t >> 2) & 3, k = t & 3;
  uint32_t* lsum = reinterpret_cast<uint32_t*>(lds + 256 * nb);
  float* ld = reinterpret_cast<float*>(lsum + 8 * nb);
  *reinterpret_cast<uint4*>(lds + 256 * blk + 16 * kq_slot(blk, l, k)) = r.q;
  if (FMT == kFmtQ4K) {
    if (k == 0) lsum[8 * blk + l] = ((uint32_t)(r.s0 + r.s1) & 0xffffu) | ((uint32_t)(r.s2 + r.s3) << 16);
  } else if (k < 2) {
    lsum[8 * blk + 2 * l + k] = ((uint32_t)(uint16_t)r.s0) | ((uint32_t)(uint16_t)r.s1 << 16);
  }
  if (l == 0 && k == 0) ld[blk] = r.d;
}

// P = prefetch depth (slices in flight per wave). A Q4_K slice is 12 VGPRs,
// a Q6_K slice 21; with 16 waves per CU a wave has 128.
// NW = waves per workgroup (the launch's block size, as a constant).
// ja_in / wg / ngrid: a group of a grouped launch, as for gemv1.
template <int FMT, int P, bool FUSED, int J, bool SILU = false, bool MIX = false, int NW = 16>
__device__ __forceinline__ void gemv1p(const GemvJobs& jobs, const void* __restrict__ act, int K,
                                       const float* __restrict__ norm_w, float eps, int accumulate,
                                       int mix_row = 0x7fffffff, const JobArg* ja_in = nullptr, int wg = -1,
                                       int ngrid = 0) {
  static_assert(FMT != kFmtQ80, "k-quant weights");
  static_assert(!MIX || FMT == kFmtQ4K, "mixed launches: Q4_K rows, then Q6_K rows");
  constexpr int F6 = kFmtQ6K;
  constexpr int BPI = 64 / FmtInfo<FMT>::kLanesPerBlock;
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int nb = K / FmtInfo<FMT>::kBlockElems;
  const int niter = (nb + BPI - 1) / BPI;
  const int lane = threadIdx.x & 63;
  constexpr int nw = NW;
  const int l = lane & 3;
  const int g = lane >> 2;
  const int row_step = (ngrid > 0 ? ngrid : (int)gridDim.x) * nw;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int row0 = (wg >= 0 ? wg : (int)blockIdx.x) * nw + wave;
  const int nrows = row0 < jobs.total ? (jobs.total - 1 - row0) / row_step + 1 : 0;
  const int nslices = nrows * niter;
  uint8_t* lds6 = lds + (MIX ? kQ8KBytes * nb : 0);  // Q6_K layout (MIX)
  const int end4 = MIX ? min(mix_row, jobs.total) : jobs.total;

  // 1. activation loads
  Act1Regs ar;
  Stage1 st, st6;
  if constexpr (FUSED)
    act1_load<SILU>(ar, reinterpret_cast<const float*>(act), nb, norm_w, nw);
  else {
    stage1_load<FMT>(st, reinterpret_cast<const uint8_t*>(act), nb);
    if constexpr (MIX) stage1_load<F6>(st6, reinterpret_cast<const uint8_t*>(act), nb);
  }

  // 2. the first P slices (issue side: slice is_s = row is_k, iteration is_it)
  const JobArg* ja = ja_in != nullptr ? ja_in : job_args();
  JobCursor jc;
  cursor_init(jc, ja);
  int is_s = 0, is_k = 0, is_it = 0;
  WSlice ring[P];
  auto issue = [&](WSlice& w) {
    const int row = row0 + is_k * row_step;
    const uint32_t b = (uint32_t)min(is_it * BPI + g, nb - 1);  // clamped: every lane loads
    if (MIX && row >= end4) {
      const RowRef rr = cursor_row<F6>(jc, ja, jobs.njobs, jobs.total, row, nb);
      load_slice<F6>(w, rr.wrow, rr.drow, b, l);
    } else {
      const RowRef rr = cursor_row<FMT>(jc, ja, jobs.njobs, jobs.total, row, nb);
      load_slice<FMT>(w, rr.wrow, rr.drow, b, l);
    }
    if (++is_it == niter) {
      is_it = 0;
      ++is_k;
    }
    ++is_s;
  };
#pragma unroll
  for (int u = 0; u < P; ++u)
    if (is_s < nslices) issue(ring[u]);

  // 3. quantization / staging into LDS while the ring streams
  if constexpr (FUSED)
    act1_finish<FMT, SILU, MIX>(ar, nb, lds, norm_w, eps, nw);
  else {
    stage1_store<FMT>(st, nb, lds);
    if constexpr (MIX) stage1_store<F6>(st6, nb, lds6);
  }
  __syncthreads();
  if (nslices == 0) return;

  // 4. consume the ring in slice order, refilling each entry P slices ahead
  // Q4_K-only launches keep iteration 0's activation in registers (Q6_K
  // slices leave no room for it)
  constexpr bool X0 = !MIX && FMT == kFmtQ4K;
  XSlice x0;
  if constexpr (X0) load_x<FMT>(x0, lds, nb, min(g, nb - 1), l);
  float acc = 0.0f;
  int c_k = 0, c_it = 0;
  float keep_v = 0.0f;  // this lane's kept output (global row keep_row)
  int keep_row = 0, slot = 0;
  for (int s0 = 0; s0 < nslices; s0 += P) {
#pragma unroll
    for (int u = 0; u < P; ++u) {
      if (s0 + u < nslices) {
        const int row = row0 + c_k * row_step;
        const int b = c_it * BPI + g;
        const bool okb = b < nb;
        const int bx = okb ? b : 0;
        int ia, ib;
        float p;
        if (MIX && row >= end4) {
          XSlice x;
          load_x<F6>(x, lds6, nb, bx, l);
          p = dot_wx<F6>(prep_w<F6>(ring[u], l), x, ia, ib);
        } else if (X0 && c_it == 0) {
          p = dot_wx<FMT>(prep_w<FMT>(ring[u], l), x0, ia, ib);
        } else {
          XSlice x;
          load_x<FMT>(x, lds, nb, bx, l);
          p = dot_wx<FMT>(prep_w<FMT>(ring[u], l), x, ia, ib);
        }
        p = okb ? p : 0.0f;
        acc = c_it == 0 ? p : acc + p;
        if (++c_it == niter) {
          const float v = wave_total(acc);
          if (lane == slot) {
            keep_v = v;
            keep_row = row;
          }
          if (++slot == 64) {
            flush_outputs<FMT, J>(jobs, nb, keep_v, keep_row, true, accumulate);
            slot = 0;
          }
          c_it = 0;
          ++c_k;
        }
      }
      if (is_s < nslices) issue(ring[u]);
    }
  }
  if (slot > 0) flush_outputs<FMT, J>(jobs, nb, keep_v, keep_row, lane < slot, accumulate);
}

}  // namespace qmm

// Kernels: the gemv1 argument list (four- or eight-job table), 16 waves,
// prefetch depth P in the name.
#define QMM_GEMV1P_KERNELS(FMT, NAME, P)                                                                      \
  extern "C" __global__ void __launch_bounds__(1024) qmm_gemv1p_##NAME##_w16_p##P(QMM_GEMV_PARAMS) {         \
    QMM_GEMV_JOBS                                                                                            \
    qmm::gemv1p<FMT, P, false, 4>(jobs, act, K, nullptr, 0.0f, accumulate);                                  \
  }                                                                                                          \
  extern "C" __global__ void __launch_bounds__(1024) qmm_gemv1pf_##NAME##_w16_p##P(QMM_GEMV_PARAMS) {        \
    QMM_GEMV_JOBS                                                                                            \
    qmm::gemv1p<FMT, P, true, 4>(jobs, act, K, norm_w, eps, accumulate);                                     \
  }                                                                                                          \
  extern "C" __global__ void __launch_bounds__(1024) qmm_gemv1p_##NAME##_w16_p##P##_j8(QMM_GEMV_PARAMS8) {   \
    QMM_GEMV_JOBS8                                                                                           \
    qmm::gemv1p<FMT, P, false, 8>(jobs, act, K, nullptr, 0.0f, accumulate);                                  \
  }                                                                                                          \
  extern "C" __global__ void __launch_bounds__(1024) qmm_gemv1pf_##NAME##_w16_p##P##_j8(QMM_GEMV_PARAMS8) {  \
    QMM_GEMV_JOBS8                                                                                           \
    qmm::gemv1p<FMT, P, true, 8>(jobs, act, K, norm_w, eps, accumulate);                                     \
  }
#define QMM_GEMV1P_MIX_KERNELS(P)                                                                              \
  extern "C" __global__ void __launch_bounds__(1024) qmm_gemv1p_q4k6k_w16_p##P(QMM_GEMV_PARAMS, int mix_row) { \
    QMM_GEMV_JOBS                                                                                             \
    qmm::gemv1p<qmm::kFmtQ4K, P, false, 4, false, true>(jobs, act, K, nullptr, 0.0f, accumulate, mix_row);    \
  }                                                                                                           \
  extern "C" __global__ void __launch_bounds__(1024) qmm_gemv1pf_q4k6k_w16_p##P(QMM_GEMV_PARAMS, int mix_row) { \
    QMM_GEMV_JOBS                                                                                             \
    qmm::gemv1p<qmm::kFmtQ4K, P, true, 4, false, true>(jobs, act, K, norm_w, eps, accumulate, mix_row);       \
  }                                                                                                           \
  extern "C" __global__ void __launch_bounds__(1024)                                                          \
      qmm_gemv1p_q4k6k_w16_p##P##_j8(QMM_GEMV_PARAMS8, int mix_row) {                                         \
    QMM_GEMV_JOBS8                                                                                            \
    qmm::gemv1p<qmm::kFmtQ4K, P, false, 8, false, true>(jobs, act, K, nullptr, 0.0f, accumulate, mix_row);    \
  }                                                                                                           \
  extern "C" __global__ void __launch_bounds__(1024)                                                          \
      qmm_gemv1pf_q4k6k_w16_p##P##_j8(QMM_GEMV_PARAMS8, int mix_row) {                                        \
    QMM_GEMV_JOBS8                                                                                            \
    qmm::gemv1p<qmm::kFmtQ4K, P, true, 8, false, true>(jobs, act, K, norm_w, eps, accumulate, mix_row);       \
  }

// Grouped launches (see QMM_GEMV1G_KERNEL): a group whose rows are several
// slices long (e.g. the down projection's K = 14336) runs the prefetch ring
// of depth PB, the other gemv1's one-row loop. PA / PB = 0: gemv1.
namespace qmm {
template <int FMT, int PP>
__device__ __forceinline__ void gemv1_group(const GemvJobs& jobs, const float* __restrict__ act, int K,
                                            int accumulate, const JobArg* ja, int wg, int ngrid) {
  if constexpr (PP == 0)
    gemv1<FMT, true, 8, false, false, 16>(jobs, act, 0, K, nullptr, 0.0f, accumulate, 0x7fffffff, ja, wg, ngrid);
  else
    gemv1p<FMT, PP, true, 8, false, false, 16>(jobs, act, K, nullptr, 0.0f, accumulate, 0x7fffffff, ja, wg, ngrid);
}
}  // namespace qmm
#define QMM_GEMV1G_RING_KERNEL(FMT, NAME, PA, PB)                                                                \
  extern "C" __global__ void __launch_bounds__(1024) qmm_gemv1g_##NAME##_w16_p##PA##_p##PB(                      \
      QMM_JOB_PARAMS(0), QMM_JOB_PARAMS(1), QMM_JOB_PARAMS(2), QMM_JOB_PARAMS(3), QMM_JOB_PARAMS(4),            \
      QMM_JOB_PARAMS(5), QMM_JOB_PARAMS(6), QMM_JOB_PARAMS(7), QMM_JOB_PARAMS(8), QMM_JOB_PARAMS(9),            \
      QMM_JOB_PARAMS(10), QMM_JOB_PARAMS(11), QMM_JOB_PARAMS(12), QMM_JOB_PARAMS(13), QMM_JOB_PARAMS(14),       \
      QMM_JOB_PARAMS(15), int njobs_a, int total_a, int njobs_b, int total_b, const float* __restrict__ act_a,   \
      const float* __restrict__ act_b, int k_a, int k_b, int ga, int accumulate) {                               \
    qmm::GemvJobs jobs;                                                                                          \
    if ((int)blockIdx.x < ga) {                                                                                  \
      QMM_JOB_SET_AS(jobs, 0, 0) QMM_JOB_SET_AS(jobs, 1, 1) QMM_JOB_SET_AS(jobs, 2, 2) QMM_JOB_SET_AS(jobs, 3, 3) \
      QMM_JOB_SET_AS(jobs, 4, 4) QMM_JOB_SET_AS(jobs, 5, 5) QMM_JOB_SET_AS(jobs, 6, 6) QMM_JOB_SET_AS(jobs, 7, 7) \
      jobs.njobs = njobs_a;                                                                                      \
      jobs.total = total_a;                                                                                      \
      qmm::gemv1_group<FMT, PA>(jobs, act_a, k_a, accumulate, qmm::job_args(), (int)blockIdx.x, ga);            \
    } else {                                                                                                     \
      QMM_JOB_SET_AS(jobs, 0, 8) QMM_JOB_SET_AS(jobs, 1, 9) QMM_JOB_SET_AS(jobs, 2, 10)                          \
      QMM_JOB_SET_AS(jobs, 3, 11) QMM_JOB_SET_AS(jobs, 4, 12) QMM_JOB_SET_AS(jobs, 5, 13)                        \
      QMM_JOB_SET_AS(jobs, 6, 14) QMM_JOB_SET_AS(jobs, 7, 15)                                                    \
      jobs.njobs = njobs_b;                                                                                      \
      jobs.total = total_b;                                                                                      \
      qmm::gemv1_group<FMT, PB>(jobs, act_b, k_b, accumulate, qmm::job_args() + 8, (int)blockIdx.x - ga,        \
                                (int)gridDim.x - ga);                                                            \
    }                                                                                                            \
  }
QMM_GEMV1G_RING_KERNEL(qmm::kFmtQ4K, q4k, 0, 2)
QMM_GEMV1G_RING_KERNEL(qmm::kFmtQ4K, q4k, 0, 4)
QMM_GEMV1G_RING_KERNEL(qmm::kFmtQ4K, q4k, 1, 4)
QMM_GEMV1G_RING_KERNEL(qmm::kFmtQ4K, q4k, 2, 4)
QMM_GEMV1G_RING_KERNEL(qmm::kFmtQ4K, q4k, 4, 4)
QMM_GEMV1G_RING_KERNEL(qmm::kFmtQ6K, q6k, 0, 2)
QMM_GEMV1G_RING_KERNEL(qmm::kFmtQ6K, q6k, 0, 3)

QMM_GEMV1P_KERNELS(qmm::kFmtQ4K, q4k, 1)
QMM_GEMV1P_KERNELS(qmm::kFmtQ4K, q4k, 2)
QMM_GEMV1P_KERNELS(qmm::kFmtQ4K, q4k, 4)
QMM_GEMV1P_KERNELS(qmm::kFmtQ6K, q6k, 1)
QMM_GEMV1P_KERNELS(qmm::kFmtQ6K, q6k, 2)
QMM_GEMV1P_KERNELS(qmm::kFmtQ6K, q6k, 3)
QMM_GEMV1P_MIX_KERNELS(1)
QMM_GEMV1P_MIX_KERNELS(2)
QMM_GEMV1P_MIX_KERNELS(3)
