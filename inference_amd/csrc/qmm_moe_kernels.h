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
namespace qmm {
// Routing of T tokens by one workgroup of NT threads (MoeMlp::forward's
// softmax, top-k with the lowest expert index on ties, renormalised or
// scaled weights), into per-expert pair lists in expert order: counts[e],
// offsets[e] (offsets[E] = T * k), pair_token / pair_weight per pair, and
// token_pairs (each token's pairs in increasing expert order). sel_e /
// sel_w (T * k), ecount (E) and eoff (E + 1) are LDS scratch; the outputs
// may be global or LDS. Ends after a barrier.
template <int NT>
__device__ __forceinline__ void moe_route_block(const float* __restrict__ logits, int T, int E, int k, int renorm,
                                                float post_scale, short* sel_e, float* sel_w, int* ecount,
                                                int* eoff, int* counts, int* offsets, int* pair_token,
                                                float* pair_weight, int* token_pairs) {
#pragma clang fp contract(off)
  constexpr int kWaves = NT / 64;
  for (int e = threadIdx.x; e < E; e += NT) ecount[e] = 0;
  __syncthreads();
  for (int t = threadIdx.x; t < T; t += NT) {
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
      // renormalised over the selection, or (norm_topk_prob false) times the
      // routed scaling factor: row[e] / denom * post_scale with denom = 1
      sel_w[t * k + s] = renorm ? p[s] / denom : p[s] * post_scale;
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
  for (int e = threadIdx.x; e <= E; e += NT) {
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
  __syncthreads();
}
}  // namespace qmm

extern "C" __global__ void __launch_bounds__(256) qmm_moe_route(const float* __restrict__ logits, int T, int E,
                                                                int k, int renorm, float post_scale,
                                                                int* __restrict__ counts,
                                                                int* __restrict__ offsets,
                                                                int* __restrict__ pair_token,
                                                                float* __restrict__ pair_weight,
                                                                int* __restrict__ token_pairs) {
  __shared__ short sel_e[8192];
  __shared__ float sel_w[8192];
  __shared__ int ecount[256];
  __shared__ int eoff[257];
  qmm::moe_route_block<256>(logits, T, E, k, renorm, post_scale, sel_e, sel_w, ecount, eoff, counts, offsets,
                            pair_token, pair_weight, token_pairs);
}

// Routing and the Q8_K gather of the routed rows in one launch, for decode-
// sized calls (T * k <= 256 pairs): every workgroup routes all T tokens in
// its own LDS (the same computation, so the same lists everywhere),
// workgroup 0 writes the routing arrays out, and wave w of the grid then
// quantizes block w % nb of pair w / nb's token row into xq (one Q8_K row
// per pair, as qmm_quantize_q8k_gather writes it).
extern "C" __global__ void __launch_bounds__(256) qmm_moe_route_gather_q8k(
    const float* __restrict__ logits, int T, int E, int k, int renorm, float post_scale, int* __restrict__ counts,
    int* __restrict__ offsets, int* __restrict__ pair_token, float* __restrict__ pair_weight,
    int* __restrict__ token_pairs, const float* __restrict__ x, long long ldx, uint8_t* __restrict__ xq, int hidden) {
  __shared__ short sel_e[256];
  __shared__ float sel_w[256];
  __shared__ int ecount[256];
  __shared__ int eoff[257];
  __shared__ int s_counts[256];
  __shared__ int s_offsets[257];
  __shared__ int s_ptok[256];
  __shared__ float s_pw[256];
  __shared__ int s_tp[256];
  qmm::moe_route_block<256>(logits, T, E, k, renorm, post_scale, sel_e, sel_w, ecount, eoff, s_counts, s_offsets,
                            s_ptok, s_pw, s_tp);
  const int P = T * k;
  if (blockIdx.x == 0) {
    for (int e = threadIdx.x; e <= E; e += 256) {
      offsets[e] = s_offsets[e];
      if (e < E) counts[e] = s_counts[e];
    }
    for (int i = threadIdx.x; i < P; i += 256) {
      pair_token[i] = s_ptok[i];
      pair_weight[i] = s_pw[i];
      token_pairs[i] = s_tp[i];
    }
  }
  const int nb = hidden / 256;
  const long long w = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (w >= (long long)P * nb) return;
  const int i = (int)(w / nb), b = (int)(w % nb);
  qmm::q8k_block(x + (long long)s_ptok[i] * ldx + 256LL * b, xq + w * qmm::kQ8KBytes, threadIdx.x & 63);
}

// Tails of the grouped prefill GEMM: an expert holding c >= tile rows whose
// last tile would hold r = c mod tile in [1, maxtail] rows leaves those r
// rows to the multi-token expert GEMV (cg = c - r rows for the GEMM, ct = r
// tail rows from row ot = offsets + cg); otherwise the GEMM takes all c rows
// (ct = 0).
extern "C" __global__ void __launch_bounds__(256) qmm_moe_split_tails(const int* __restrict__ counts,
                                                                      const int* __restrict__ offsets, int E,
                                                                      int tile, int maxtail, int* __restrict__ cg,
                                                                      int* __restrict__ ct, int* __restrict__ ot) {
  for (int e = blockIdx.x * 256 + threadIdx.x; e < E; e += gridDim.x * 256) {
    const int c = counts[e], r = c % tile;
    const bool split = c >= tile && r > 0 && r <= maxtail;
    const int g = split ? c - r : c;
    cg[e] = g;
    ct[e] = split ? r : 0;
    ot[e] = offsets[e] + g;
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
// weight * y_pair[n], accumulated from zero like index_add; then, with a
// shared expert, + shared[t][n] (times sg[t] when the shared expert is gated):
// MoeMlp::forward's `out + shared` (models/llama.rs:1476-1486).
extern "C" __global__ void qmm_moe_combine(const float* __restrict__ yp, const float* __restrict__ pair_weight,
                                           const int* __restrict__ token_pairs, int T, int k, int N,
                                           float* __restrict__ out, int ldo, const float* __restrict__ shared,
                                           const float* __restrict__ sg) {
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
  if (shared != nullptr) {
    const float sv = shared[(size_t)t * N + n];
    acc = acc + (sg != nullptr ? sv * sg[t] : sv);
  }
  out[(size_t)t * ldo + n] = acc;
}

// The shared expert's sigmoid gate: sg[t] = sigmoid(x[t] . g) (one wave per
// token; the f32 dot in lane order, then the wave sum), the reference's
// sigmoid(xf.matmul(shared_gate.t())) (models/llama.rs:1479-1482).
extern "C" __global__ void __launch_bounds__(256) qmm_moe_shared_gate(const float* __restrict__ x, long long ldx,
                                                                      const float* __restrict__ g, int H, int T,
                                                                      float* __restrict__ sg) {
#pragma clang fp contract(off)
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (t >= T) return;
  const float* xr = x + (long long)t * ldx;
  float acc = 0.0f;
  for (int h = lane; h < H; h += 64) acc += xr[h] * g[h];
  acc = qmm::wave_sum(acc);
  if (lane == 0) sg[t] = 1.0f / (1.0f + expf(-acc));
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
// prefetch ring (the gemv1p structure). blockIdx.y is the pass: tokens
// 8y .. 8y + 7 of every expert holding more than 8y of them; the pass's
// workgroups are shared out over those experts, and a workgroup stages its
// expert's pass rows in LDS once. A wave's weight slice is unpacked once and
// multiplied with each token row, and each row's outputs are stored by lanes
// 0..rows-1 together. The per-token accumulators are scalars, so register
// use stays near the one-row kernels' (the generic M = 8 GEMV keeps eight
// activation slices live and spills at these shapes).
//
// One pass over MR (compile-time) token rows, with the per-token work cut to
// the dot products and the block's integer and f32 combine:
//   * the activations are staged row-interleaved (block b of token m at LDS
//     block b * MR + m), so a token's reads are immediate offsets from the
//     first token's addresses, formed once per weight slice;
//   * the Q4_K high nibbles are unpacked once per slice (the one-row
//     kernels' 16q - 128 form needs a correction per token);
//   * a lane past the row's last block gets zero scales, so its products are
//     zero without a select per token, and the accumulators are cleared when
//     a row starts;
//   * no branch per token (the count is a template constant).
// The integer block dots and the f32 sequence per block are the one-row
// kernels', so the outputs are unchanged.
struct MoePass {
  const uint8_t* wb0;   // expert's first row body of weight 0 / 1
  const uint8_t* wb1;
  const uint16_t* db0;  // expert's first separated f16 scale of weight 0 / 1
  const uint16_t* db1;
  float* y0;
  float* y1;
  int N, ldy, nb, niter, row0, row_step, nslices;
  uint32_t rowb;   // row body bytes (an expert's rows span < 4 GiB: checked by the host)
  long long yrow;  // first output row of the pass (offsets[e] + mc)
  int accumulate;  // y += result (each output has one writer, so y + v exactly)
};

// A workgroup's rows of the `total` rows shared by gx workgroups (this one is
// bx). Rows longer than one slice (K > 4096): a contiguous block per
// workgroup, its waves taking every NW-th row of it, so the workgroups stream
// separate regions (config-5 down, 11.6 KB rows: 62.3 -> 58.8 us). One-slice
// rows stay grid-stride over the workgroups (gate/up, 2.3 KB rows: contiguous
// blocks measured 82.3 -> 84.1 us).
template <int NW>
__device__ __forceinline__ void pass_rows(MoePass& ps, int total, int bx, int gx, int wave) {
  int nrows;
  if (ps.niter > 1) {
    const int per = (total + gx - 1) / gx;
    const int rb0 = min(bx * per, total), rb1 = min(rb0 + per, total);
    ps.row_step = NW;
    ps.row0 = rb0 + wave;
    nrows = ps.row0 < rb1 ? (rb1 - 1 - ps.row0) / NW + 1 : 0;
  } else {
    ps.row_step = gx * NW;
    ps.row0 = bx * NW + wave;
    nrows = ps.row0 < total ? (total - 1 - ps.row0) / ps.row_step + 1 : 0;
  }
  ps.nslices = nrows * ps.niter;
}

// Weight-side values of a lane's slice for several tokens: the Q4_K high
// nibbles as plain 0..15 bytes, the scales that multiply the activation sums
// packed as int16 pairs for v_dot2 (Q4_K mins m0 | m1; Q6_K scales c0 | c1,
// c2 | c3), and all scales zero when the lane's block is past the row's end.
struct WTok {
  qmm::WPrep w;
  uint32_t p01, p23;
};

template <int FMT>
__device__ __forceinline__ WTok prep_w_tok(const qmm::WSlice& s, int l, bool ok) {
  using namespace qmm;
  WTok t;
  t.w = prep_w<FMT>(s, l);
  if constexpr (FMT == kFmtQ4K) {
    t.w.w2 = hi_nib(s.b);
    t.w.w3 = hi_nib(s.c);
    t.p01 = (uint32_t)t.w.c2 | ((uint32_t)t.w.c3 << 16);
    t.p23 = 0;
  } else {
    t.p01 = ((uint32_t)t.w.c0 & 0xffffu) | ((uint32_t)t.w.c1 << 16);
    t.p23 = ((uint32_t)t.w.c2 & 0xffffu) | ((uint32_t)t.w.c3 << 16);
  }
  if (!ok) {
    t.w.c0 = t.w.c1 = t.w.c2 = t.w.c3 = 0;
    t.p01 = t.p23 = 0;
    t.w.dw = t.w.dm = 0.0f;
  }
  return t;
}

typedef short moe_short2 __attribute__((ext_vector_type(2)));
// sum of the two int16 products of packed pairs a, b (v_dot2_i32_i16)
__device__ __forceinline__ int dot2_i16(uint32_t a, uint32_t b, int c) {
  return __builtin_amdgcn_sdot2(__builtin_bit_cast(moe_short2, a), __builtin_bit_cast(moe_short2, b), c, false);
}

// One lane's LDS addresses of block bx of the first token in the
// row-interleaved layout; token m's are fixed offsets from them.
struct XTok {
  const uint8_t* q[4];
  const uint32_t* s;
  const float* d;
};

template <int FMT, int MR>
__device__ __forceinline__ XTok xtok_base(const uint8_t* lds, int nb, int bx, int l) {
  using namespace qmm;
  XTok t;
  const int nblk = MR * nb;
  const uint8_t* e = lds + 256 * (bx * MR);
  const int sw = (bx & 3) ^ ((l >> 1) << 1);  // kq_slot's swizzle of block bx
#pragma unroll
  for (int i = 0; i < 4; ++i) t.q[i] = e + 16 * (4 * l + (i ^ sw));
  const uint32_t* lsum = reinterpret_cast<const uint32_t*>(lds + 256 * nblk);
  t.s = lsum + 8 * (bx * MR) + (FMT == kFmtQ4K ? l : 2 * l);
  t.d = reinterpret_cast<const float*>(lsum + 8 * nblk) + bx * MR;
  return t;
}

template <int FMT>
__device__ __forceinline__ qmm::XSlice load_xtok(const XTok& t, int m) {
  qmm::XSlice x;
  x.x0 = *reinterpret_cast<const uint4*>(t.q[0] + 256 * m);
  x.x1 = *reinterpret_cast<const uint4*>(t.q[1] + 256 * m);
  x.x2 = *reinterpret_cast<const uint4*>(t.q[2] + 256 * m);
  x.x3 = *reinterpret_cast<const uint4*>(t.q[3] + 256 * m);
  x.s0 = t.s[8 * m];
  x.s1 = FMT == qmm::kFmtQ4K ? 0u : t.s[8 * m + 1];
  x.d = t.d[m];
  return x;
}

// dot_wx's block value (the same integers, then the same f32 sequence) for
// prep_w_tok's weights:
//   Q4_K: isd = c0 s0 + c1 s1; ism = m0 bs0 + m1 bs1 in one v_dot2 over the
//         packed activation sums;
//   Q6_K: sum_i c_i (d_i - 32 S_i) = sum_i c_i d_i - 32 sum_i c_i S_i, the
//         second sum in two v_dot2.
// |s|, |d| < 2^23 and the sums of 32 int8 fit int16, so every step is exact.
template <int FMT>
__device__ __forceinline__ float dot_tok(const WTok& t, const qmm::XSlice& x) {
  using namespace qmm;
  const WPrep& w = t.w;
  if constexpr (FMT == kFmtQ4K) {
    const int s0 = dot16(w.w1, x.x1, dot16(w.w0, x.x0, 0));
    const int s1 = dot16(w.w3, x.x3, dot16(w.w2, x.x2, 0));
    const int isd = __mul24(w.c0, s0) + __mul24(w.c1, s1);
    const int ism = dot2_i16(t.p01, x.s0, 0);
    return x.d * q4k_combine(w.dw, w.dm, isd, ism);
  } else {
    static_assert(FMT == kFmtQ6K, "k-quant weights");
    const int d0 = dot16(w.w0, x.x0, 0), d1 = dot16(w.w1, x.x1, 0);
    const int d2 = dot16(w.w2, x.x2, 0), d3 = dot16(w.w3, x.x3, 0);
    const int cs = dot2_i16(t.p23, x.s1, dot2_i16(t.p01, x.s0, 0));
    const int cd = __mul24(w.c0, d0) + __mul24(w.c1, d1) + __mul24(w.c2, d2) + __mul24(w.c3, d3);
    const int is = cd - 32 * cs;
    return x.d * (w.dw * (float)is);
  }
}

// Per-token wave sums of acc[0..MR) with wave_total's summation tree, the
// tokens spread across lanes so that a level costs about three instructions
// per token pair instead of a wave_total per token:
//   * lanes carry the index v = lane, with bits 0 and 1 flipped in odd quads,
//     so that the half-row mirror (lane ^ 7) pairs v with v ^ 4;
//   * levels 1 (lane ^ 1), 2 (lane ^ 2) and 3 (half-row mirror): a lane keeps
//     the tokens whose index bit equals v's and adds the partner's copy of
//     them (halving its values while MR allows, else adding its one value);
//   * level 4 (row rotate by 8) joins the two 8-lane groups of a row;
//   * lane m < MR fetches token m's four row sums and adds
//     (R0 + R1) + (R2 + R3).
// Each add joins the same two partial sums as wave_total, so the totals are
// bit-identical. Returns token `lane`'s total on lanes < MR.
template <int MR>
__device__ __forceinline__ float wave_totals(const float (&acc)[MR], int lane) {
  using namespace qmm;
  if constexpr (MR == 1) {
    return wave_total(acc[0]);
  } else {
    constexpr int MRP = MR <= 2 ? 2 : MR <= 4 ? 4 : 8;  // padded with zero tokens
    const int v = lane ^ (((lane >> 2) & 1) ? 3 : 0);
    const bool b0 = v & 1, b1 = (v >> 1) & 1, b2 = (v >> 2) & 1;
    float t[MRP];
#pragma unroll
    for (int m = 0; m < MRP; ++m) t[m] = m < MR ? acc[m] : 0.0f;
    // level 1: u[j] = token 2j + b0
    float u[MRP / 2];
#pragma unroll
    for (int j = 0; j < MRP / 2; ++j) {
      const float keep = b0 ? t[2 * j + 1] : t[2 * j], send = b0 ? t[2 * j] : t[2 * j + 1];
      u[j] = keep + dpp_f<0xb1>(send);  // quad_perm [1,0,3,2]
    }
    // level 2: w[j] = token 4j + 2 b1 + b0 (MRP >= 4)
    float w[MRP >= 4 ? MRP / 4 : 1];
    if constexpr (MRP >= 4) {
#pragma unroll
      for (int j = 0; j < MRP / 4; ++j) {
        const float keep = b1 ? u[2 * j + 1] : u[2 * j], send = b1 ? u[2 * j] : u[2 * j + 1];
        w[j] = keep + dpp_f<0x4e>(send);  // quad_perm [2,3,0,1]
      }
    } else {
      w[0] = u[0] + dpp_f<0x4e>(u[0]);
    }
    // level 3: token v & (MRP - 1)
    float z;
    if constexpr (MRP == 8) {
      const float keep = b2 ? w[1] : w[0], send = b2 ? w[0] : w[1];
      z = keep + dpp_f<0x141>(send);  // row_half_mirror
    } else {
      z = w[0] + dpp_f<0x141>(w[0]);
    }
    z += dpp_f<0x128>(z);  // row_ror:8: the row's other 8-lane group
    // token m's row sums sit in lanes 16 r + j with j = v(m) (v is its own inverse)
    const int m = lane & 7, j = m ^ (((m >> 2) & 1) ? 3 : 0);
    auto row = [&](int r) {
      return __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(4 * (16 * r + j), __builtin_bit_cast(int, z)));
    };
    return (row(0) + row(1)) + (row(2) + row(3));
  }
}

template <int FMT, int P, int NW, int MR>
__device__ __forceinline__ void moe_gemv1_pass(const MoePass& a, const uint8_t* __restrict__ xs, uint8_t* lds) {
#pragma clang fp contract(off)
  using namespace qmm;
  constexpr int BPI = 16;
  const int lane = threadIdx.x & 63, l = lane & 3, g = lane >> 2;
  const int nb = a.nb, niter = a.niter, nslices = a.nslices;
  int is_s = 0, is_k = 0, is_it = 0;
  WSlice ring[P];
  auto issue = [&](WSlice& w) {
    const int gr = a.row0 + is_k * a.row_step;  // < total while is_s < nslices
    const int j = gr >= a.N ? 1 : 0;
    const uint32_t r = (uint32_t)(gr - j * a.N);  // row of the expert's weight j
    const uint8_t* wrow = (j ? a.wb1 : a.wb0) + r * a.rowb;
    const uint16_t* drow = (j ? a.db1 : a.db0) + r * (uint32_t)nb;
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
  stage_act<FMT, NW, MR>(xs, MR * nb, lds, nb);
  __syncthreads();
  float acc[MR];
#pragma unroll
  for (int m = 0; m < MR; ++m) acc[m] = 0.0f;
  int c_k = 0, c_it = 0;
  for (int s0 = 0; s0 < nslices; s0 += P) {
#pragma unroll
    for (int u = 0; u < P; ++u) {
      if (s0 + u < nslices) {
        const int b = c_it * BPI + g;
        const bool okb = b < nb;
        const WTok wp = prep_w_tok<FMT>(ring[u], l, okb);
        const XTok xt = xtok_base<FMT, MR>(lds, nb, okb ? b : 0, l);
#pragma unroll
        for (int m = 0; m < MR; ++m) acc[m] += dot_tok<FMT>(wp, load_xtok<FMT>(xt, m));
        if (++c_it == niter) {
          const int gr = a.row0 + c_k * a.row_step;
          const int j = gr >= a.N ? 1 : 0;
          const float out = wave_totals<MR>(acc, lane);
#pragma unroll
          for (int m = 0; m < MR; ++m) acc[m] = 0.0f;
          if (lane < MR) {
            float* yp = (j ? a.y1 : a.y0) + (size_t)(a.yrow + lane) * a.ldy + (gr - j * a.N);
            *yp = a.accumulate ? *yp + out : out;
          }
          c_it = 0;
          ++c_k;
        }
      }
      if (is_s < nslices) issue(ring[u]);
    }
  }
}

// The pass for mr (1..8, workgroup-uniform) token rows.
template <int FMT, int P, int NW>
__device__ __forceinline__ void moe_gemv1_rows(const MoePass& ps, int mr, const uint8_t* __restrict__ xs,
                                               uint8_t* lds) {
  switch (mr) {
    case 1: moe_gemv1_pass<FMT, P, NW, 1>(ps, xs, lds); break;
    case 2: moe_gemv1_pass<FMT, P, NW, 2>(ps, xs, lds); break;
    case 3: moe_gemv1_pass<FMT, P, NW, 3>(ps, xs, lds); break;
    case 4: moe_gemv1_pass<FMT, P, NW, 4>(ps, xs, lds); break;
    case 5: moe_gemv1_pass<FMT, P, NW, 5>(ps, xs, lds); break;
    case 6: moe_gemv1_pass<FMT, P, NW, 6>(ps, xs, lds); break;
    case 7: moe_gemv1_pass<FMT, P, NW, 7>(ps, xs, lds); break;
    default: moe_gemv1_pass<FMT, P, NW, 8>(ps, xs, lds); break;
  }
}

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
  const int lane = threadIdx.x & 63;
  const int mc = 8 * (int)blockIdx.y;  // this workgroup's pass: tokens mc .. mc + 7 of its expert
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
  // workgroup-uniform values read from LDS or memory go to scalar registers
  // (readfirstlane), which keeps the address arithmetic on the scalar unit
  // and the per-token passes within the vector register budget
  const int na = __builtin_amdgcn_readfirstlane(nact);
  if (na == 0) return;
  const long long G = gridDim.x;
  const int slot = (int)((long long)blockIdx.x * na / G);
  const int first = (int)(((long long)slot * G + na - 1) / na);
  const int next = (int)(((long long)(slot + 1) * G + na - 1) / na);
  const int e = __builtin_amdgcn_readfirstlane(act[slot]), bx = (int)blockIdx.x - first, gx = next - first;
  const int me = __builtin_amdgcn_readfirstlane(counts[e]);
  const int off = __builtin_amdgcn_readfirstlane(offsets[e]);
  const int nb = K / 256, niter = (nb + BPI - 1) / BPI;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int total = njobs * N;
  MoePass ps;
  const size_t rowb = (size_t)nb * FmtInfo<FMT>::kBodyBytes, erow = (size_t)e * N, trows = (size_t)E * N;
  ps.wb0 = w0 + erow * rowb;
  ps.wb1 = w1 + erow * rowb;
  ps.db0 = reinterpret_cast<const uint16_t*>(w0 + trows * rowb) + erow * nb;
  ps.db1 = reinterpret_cast<const uint16_t*>(w1 + trows * rowb) + erow * nb;
  ps.y0 = y0;
  ps.y1 = y1;
  ps.N = N;
  ps.ldy = ldy;
  ps.nb = nb;
  ps.niter = niter;
  ps.rowb = (uint32_t)rowb;
  ps.accumulate = 0;
  pass_rows<NW>(ps, total, bx, gx, wave);
  // a single pass per workgroup: with a loop over passes the state carried
  // across it pushes the eight inlined token counts past the scalar
  // registers (spilled into vector registers, then to memory)
  ps.yrow = off + mc;
  moe_gemv1_rows<FMT, P, NW>(ps, min(8, me - mc), xq + (size_t)(off + mc) * xrow, lds);
}

#define QMM_MOE1_KERNEL(FMT, NAME, P)                                                                           \
  extern "C" __global__ void __launch_bounds__(1024)                                                            \
      qmm_moe_gemv1_##NAME##_p##P(const uint8_t* w0, const uint8_t* w1, int njobs, int N, int E, float* y0,   \
                                  float* y1, int ldy, const uint8_t* __restrict__ xq, long long xrow,           \
                                  const int* __restrict__ counts, const int* __restrict__ offsets, int K) {    \
    moe_gemv1<FMT, P, 16>(w0, w1, njobs, N, E, y0, y1, ldy, xq, xrow, counts, offsets, K);                     \
  }
// Dense GEMV of m (1..8) staged activation rows against one k-quant weight
// [N, K] through the same pass (the expert GEMV with one expert holding every
// row): for m = 6..8 it beats the general multi-row GEMV, with the same bits.
template <int FMT, int P, int NW>
__device__ __forceinline__ void gemv_rows(const uint8_t* __restrict__ w, float* __restrict__ y, int ldy,
                                          const uint8_t* __restrict__ xq, int m, int K, int N, int accumulate) {
  using namespace qmm;
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int nb = K / 256;
  const size_t rowb = (size_t)nb * FmtInfo<FMT>::kBodyBytes;
  MoePass ps;
  ps.wb0 = ps.wb1 = w;
  ps.db0 = ps.db1 = reinterpret_cast<const uint16_t*>(w + (size_t)N * rowb);
  ps.y0 = ps.y1 = y;
  ps.N = N;
  ps.ldy = ldy;
  ps.nb = nb;
  ps.niter = (nb + 15) / 16;
  ps.rowb = (uint32_t)rowb;
  ps.yrow = 0;
  ps.accumulate = accumulate;
  pass_rows<NW>(ps, N, (int)blockIdx.x, (int)gridDim.x, __builtin_amdgcn_readfirstlane(threadIdx.x >> 6));
  moe_gemv1_rows<FMT, P, NW>(ps, m, xq, lds);
}

#define QMM_GEMV_ROWS_KERNEL(FMT, NAME)                                                                         \
  extern "C" __global__ void __launch_bounds__(1024) qmm_gemv_rows_##NAME(                                     \
      const uint8_t* __restrict__ w, float* __restrict__ y, int ldy, const uint8_t* __restrict__ xq, int m,     \
      int K, int N, int accumulate) {                                                                          \
    gemv_rows<FMT, 1, 16>(w, y, ldy, xq, m, K, N, accumulate);                                                  \
  }
QMM_GEMV_ROWS_KERNEL(qmm::kFmtQ4K, q4k)
QMM_GEMV_ROWS_KERNEL(qmm::kFmtQ6K, q6k)

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
                                           const int* __restrict__ offsets, int e) {
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
    if (!qmm::group_rows<BM, false>(g, xq, xd, xs, y, K, ldy, counts, offsets, blockIdx.z)) return;             \
    const uint8_t* we = wq + (size_t)blockIdx.z * N * (K / 256) * qmm::kQ4KBytes;                               \
    qmm::mmq2_q4k<BM, 128, false>(we, g.xq, g.xd, g.xs, g.y, g.m, N, K, ldy, nullptr, 0, 0, 0, K / 256);        \
    (void)E;                                                                                                    \
  }
QMM_MOE_MMQ2_KERNEL(128, )
QMM_MOE_MMQ2_KERNEL(64, _m64)

// Q4_K grouped GEMM on the split-scale tile (mmqs: the d term on int8 MFMA,
// the mins term on bf16 MFMA): an expert's rows give what the dense mmqs
// GEMM gives on them alone, unsplit.
extern "C" __global__ void __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
qmm_moe_mmqs_q4k(const uint8_t* __restrict__ wq, const int8_t* __restrict__ xq, const float* __restrict__ xd,
                 const int16_t* __restrict__ xs, float* __restrict__ y, int N, int K, int ldy, int E,
                 const int* __restrict__ counts, const int* __restrict__ offsets) {
  qmm::GroupRows g;
  if (!qmm::group_rows<qmm::kSBM, false>(g, xq, xd, xs, y, K, ldy, counts, offsets, blockIdx.z)) return;
  const uint8_t* we = wq + (size_t)blockIdx.z * N * (K / 256) * qmm::kQ4KBytes;
  qmm::mmqs_q4k<false>(we, g.xq, g.xd, g.xs, g.y, g.m, N, K, ldy, nullptr, 0, 0, 0, K / 256);
  (void)E;
}

// The same over two weights of one shape in one launch (gate and up: grid z =
// 2 E, weight z / E): the two launches' tiles in one grid, so that a partial
// last round of workgroups falls once instead of once per weight.
extern "C" __global__ void __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
qmm_moe_mmqs2_q4k(const uint8_t* __restrict__ w0, const uint8_t* __restrict__ w1, const int8_t* __restrict__ xq,
                  const float* __restrict__ xd, const int16_t* __restrict__ xs, float* __restrict__ y0,
                  float* __restrict__ y1, int N, int K, int ldy, int E, const int* __restrict__ counts,
                  const int* __restrict__ offsets) {
  const int j = (int)blockIdx.z >= E ? 1 : 0, e = (int)blockIdx.z - j * E;
  qmm::GroupRows g;
  if (!qmm::group_rows<qmm::kSBM, false>(g, xq, xd, xs, j ? y1 : y0, K, ldy, counts, offsets, e)) return;
  const uint8_t* we = (j ? w1 : w0) + (size_t)e * N * (K / 256) * qmm::kQ4KBytes;
  qmm::mmqs_q4k<false>(we, g.xq, g.xd, g.xs, g.y, g.m, N, K, ldy, nullptr, 0, 0, 0, K / 256);
}

// The first-generation tile (Q6_K, Q8_0) also splits K: blockIdx.z = expert
// + E * split, split s takes K steps [s kc, s kc + kc) and writes its f32
// partial to y + s * ysplit (the host sums them in split order).
#define QMM_MOE_MMQ_KERNEL(FMT, NAME)                                                                          \
  extern "C" __global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))                 \
      qmm_moe_mmq_##NAME(const uint8_t* __restrict__ wq, const int8_t* __restrict__ xq,                        \
                         const float* __restrict__ xd, const int16_t* __restrict__ xs, float* __restrict__ y,   \
                         int N, int K, int ldy, int E, const int* __restrict__ counts,                          \
                         const int* __restrict__ offsets, int kc, long long ysplit) {                          \
    const int e = (int)blockIdx.z % E, sp = (int)blockIdx.z / E;                                               \
    qmm::GroupRows g;                                                                                          \
    if (!qmm::group_rows<qmm::kMmqBM, FMT == qmm::kFmtQ80>(g, xq, xd, xs, y + sp * ysplit, K, ldy, counts,      \
                                                            offsets, e))                                       \
      return;                                                                                                  \
    const int nbw = FMT == qmm::kFmtQ80 ? K / 32 : K / 256;                                                    \
    const size_t rows0 = (size_t)e * N;                                                                        \
    const uint16_t* wd = qmm::split_scales<FMT>(wq, (long long)E * N, K) + rows0 * nbw;                        \
    const uint8_t* we = wq + rows0 * nbw * qmm::FmtInfo<FMT>::kBodyBytes;                                      \
    const int kb0 = sp * kc;                                                                                   \
    qmm::mmq<FMT, false>(we, wd, g.xq, g.xd, g.xs, g.y, g.m, N, K, ldy, nullptr, 0, 0, kb0,                    \
                         min(kb0 + kc, K / 256));                                                              \
  }
QMM_MOE_MMQ_KERNEL(qmm::kFmtQ6K, q6k)

// Q6_K grouped GEMM on the split-digit tile (128-row tiles; K split as above):
// for the grouped prefill with tails, whose experts' GEMM rows are whole tiles.
extern "C" __global__ void __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
qmm_moe_mmqs6_q6k(const uint8_t* __restrict__ wq, const int8_t* __restrict__ xq, const float* __restrict__ xd,
                  const int16_t* __restrict__ xs, float* __restrict__ y, int N, int K, int ldy, int E,
                  const int* __restrict__ counts, const int* __restrict__ offsets, int kc, long long ysplit) {
  const int e = (int)blockIdx.z % E, sp = (int)blockIdx.z / E;
  qmm::GroupRows g;
  if (!qmm::group_rows<qmm::kSBM, false>(g, xq, xd, xs, y + sp * ysplit, K, ldy, counts, offsets, e)) return;
  const int nbk = K / 256;
  const size_t rows0 = (size_t)e * N;
  const uint16_t* wd = qmm::split_scales<qmm::kFmtQ6K>(wq, (long long)E * N, K) + rows0 * nbk;
  const uint8_t* we = wq + rows0 * nbk * qmm::kQ6KBody;
  const int kb0 = sp * kc;
  qmm::mmqs6_q6k<false>(we, wd, g.xq, g.xd, g.y, g.m, N, K, ldy, nullptr, 0, 0, kb0, min(kb0 + kc, nbk));
}

QMM_MOE_MMQ_KERNEL(qmm::kFmtQ80, q8_0)
