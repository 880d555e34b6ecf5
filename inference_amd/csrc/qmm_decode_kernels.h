// Non-matmul kernels of one decode step of a Llama-style decoder (config 3 of
// the benchmark), all f32 as the reference's decode path:
//   embedding row gather           CausalLm embed (crates/llm/candle-llm/src/models/llama.rs:397-408)
//   RoPE (NeoX half-split) + KV append  apply_rope (primitives/rope.rs:289-323), kv_cache.rs:107-111
//   GQA attention for one query    repeat_kv + sdpa_eager (primitives/attention.rs:59-68, 154-186)
//   silu(gate) * up -> Q8_K        LlamaMlp::forward (models/llama.rs:1386-1391)
//   greedy argmax (lowest index on ties)  argmax_device (primitives/sampler.rs:216-219)
// The token position and token ids live in device memory (pos[0], tokens[]),
// so a captured step replays unchanged for every position.
#pragma once

#include "qmm_common.h"
#include "qmm_quant_kernels.h"

// x[0 : hidden) = table[tokens[pos[0]]][0 : hidden)
extern "C" __global__ void qmm_decode_embed(const float* __restrict__ table, long long ld,
                                            const int* __restrict__ tokens, const int* __restrict__ pos,
                                            float* __restrict__ x, int hidden) {
  const int tok = tokens[pos[0]];
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < hidden; i += gridDim.x * blockDim.x)
    x[i] = table[(long long)tok * ld + i];
}

// Rotates q (heads x dim) and k (kv_heads x dim) at position p = pos[0] with
// cos/sin rows [p][dim] (cat(freqs, freqs) layout: pairs (i, i + dim/2)), in
// place, and appends k, v to the layer's cache [kv_heads][max_seq][dim].
// One workgroup per head (q heads first, then kv heads). A position outside
// [0, max_seq) writes nothing.
extern "C" __global__ void qmm_decode_rope_kv(float* __restrict__ q, float* __restrict__ k,
                                              const float* __restrict__ v, const float* __restrict__ cos_t,
                                              const float* __restrict__ sin_t, const int* __restrict__ pos,
                                              float* __restrict__ kcache, float* __restrict__ vcache, int heads,
                                              int kv_heads, int dim, int max_seq) {
#pragma clang fp contract(off)
  const int p = pos[0];
  if (p < 0 || p >= max_seq) return;
  const int h = blockIdx.x;
  const int half = dim / 2;
  const float* c = cos_t + (size_t)p * dim;
  const float* s = sin_t + (size_t)p * dim;
  float* x = h < heads ? q + (size_t)h * dim : k + (size_t)(h - heads) * dim;
  const int i = threadIdx.x;
  float out = 0.0f;
  if (i < dim) {
    // x*cos + rotate_half(x)*sin, rotate_half = cat(-x2, x1)
    const float xi = x[i];
    const float rot = i < half ? -x[i + half] : x[i - half];
    out = xi * c[i] + rot * s[i];
  }
  __syncthreads();
  if (i < dim) {
    x[i] = out;
    if (h >= heads) {
      const int g = h - heads;
      kcache[((size_t)g * max_seq + p) * dim + i] = out;
      vcache[((size_t)g * max_seq + p) * dim + i] = v[(size_t)g * dim + i];
    }
  }
}

// One query token against positions 0..p of the cache (p = pos[0]),
// split over positions ("flash decoding") in two launches.
//
// qmm_decode_attention_split: workgroup (g, c) of a kv_heads x S grid takes
// the G = heads / kv_heads query heads of kv head g (repeat_kv maps query
// head h to kv head h / G) and the c-th of S contiguous chunks of the
// n = p + 1 positions, and writes per head the chunk's softmax state:
// m = max_j s_j, l = sum_j exp(s_j - m), o = sum_j exp(s_j - m) v_j, with
// s_j = (q . k_j) * scale (m = -inf, l = 0, o = 0 for an empty chunk).
// qmm_decode_attention_merge then forms, per head,
// out = sum_c exp(m_c - M) o_c / sum_c exp(m_c - M) l_c, M = max_c m_c,
// adding the chunks in chunk order. The launch boundary orders the two.
//
// With cos/sin (fused RoPE + KV append), q and k are the unrotated
// projections: q is rotated in LDS; the workgroup whose chunk holds p
// rotates k, appends k and v at position p of the cache and uses them for
// that position. Without cos/sin, q is already rotated and the cache already
// holds position p.
//
// The kernel is a chain of memory latencies, so its loads go out in two
// batches: pos, q and the new k/v rows (independent of each other), then
// the chunk's first K tile, its first v rows and the cos/sin rows (all
// functions of p only). K tiles sit in LDS rows padded to dim + 1 floats
// (conflict-free column reads); scores are one (position, head) per thread;
// v rows are read once per workgroup, each thread accumulating one float4
// column over a slot of rows. dim is 64, 128 or 256, G <= 8, chunk length
// <= 256 (max_seq <= 256 S).
namespace qmm {
constexpr int kAttnMaxG = 8;
constexpr int kAttnMaxChunk = 256;
constexpr int kAttnTileFloats = 8192;
constexpr int kAttnSplits = 16;  // S
}  // namespace qmm

extern "C" __global__ void __launch_bounds__(256) qmm_decode_attention_split(
    const float* __restrict__ q, const float* __restrict__ k_new, const float* __restrict__ v_new,
    const float* __restrict__ cos_t, const float* __restrict__ sin_t, const int* __restrict__ pos,
    float* __restrict__ kcache, float* __restrict__ vcache, float* __restrict__ part, int heads, int kv_heads,
    int dim, int max_seq, float scale) {
#pragma clang fp contract(off)
  using namespace qmm;
  constexpr int S = kAttnSplits;
  __shared__ float qs[kAttnMaxG * 256];
  __shared__ float sc[kAttnMaxG * kAttnMaxChunk];
  __shared__ __attribute__((aligned(16))) float kt[kAttnTileFloats + 128];  // padded K tile, then V partials
  __shared__ float knew[256];
  __shared__ float stat[2 * kAttnMaxG];
  const int g = blockIdx.x, c = blockIdx.y, t = threadIdx.x;
  const int lane = t & 63, wave = t >> 6;
  const int G = heads / kv_heads;
  const bool rope = cos_t != nullptr;
  const int half = dim >> 1, d4 = dim >> 2;
  const int gd = G * dim;

  // loads, batch 1: pos, q of the group's heads (contiguous rows), new k / v rows
  const int p = min(max(pos[0], 0), max_seq - 1);
  float qv[8];
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    const int i = t + 256 * u;
    if (i < gd) qv[u] = q[(size_t)g * gd + i];
  }
  float kn = 0.0f, vn = 0.0f;
  if (rope && t < dim) {
    kn = k_new[(size_t)g * dim + t];
    vn = v_new[(size_t)g * dim + t];
  }

  const int n = p + 1;
  const int L = (n + S - 1) / S;
  const int j0 = min(c * L, n), j1 = min(j0 + L, n);
  const int nc = j1 - j0;
  const bool own = j0 <= p && p < j1;
  const float* kc = kcache + (size_t)g * max_seq * dim;
  const float* vc = vcache + (size_t)g * max_seq * dim;
  const int TJ = kAttnTileFloats / dim;  // positions per K tile
  const int RS = 256 / d4;              // v row slots
  const int c4 = t % d4, rs = t / d4;

  // loads, batch 2: first K tile, first v rows, cos / sin rows
  float4 r[8];
  {
    const int nt = min(TJ, nc);
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int i = t + 256 * u, jj = i / d4;
      if (jj < nt) r[u] = reinterpret_cast<const float4*>(kc + (size_t)(j0 + jj) * dim)[i % d4];
    }
  }
  float4 vv[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int j = j0 + rs + u * RS;
    if (j < j1) {
      const float* row = (rope && j == p) ? v_new + (size_t)g * dim : vc + (size_t)j * dim;
      vv[u] = reinterpret_cast<const float4*>(row)[c4];
    }
  }
  float csv[8], snv[8], ck = 0.0f, sk = 0.0f;
  if (rope) {
    const float* cs = cos_t + (size_t)p * dim;
    const float* sn = sin_t + (size_t)p * dim;
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int i = t + 256 * u;
      if (i < gd) {
        csv[u] = cs[i % dim];
        snv[u] = sn[i % dim];
      }
    }
    if (t < dim) {
      ck = cs[t];
      sk = sn[t];
    }
  }

  // q (and k at p) into LDS, rotated when fused: x * cos + cat(-x2, x1) * sin
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    const int i = t + 256 * u;
    if (i < gd) qs[i] = qv[u];
  }
  if (rope && t < dim) knew[t] = kn;
  __syncthreads();
  if (rope) {
    float rq[8], rk = 0.0f;
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int i = t + 256 * u;
      if (i < gd) {
        const int d = i % dim;
        const float rot = d < half ? -qs[i + half] : qs[i - half];
        rq[u] = qv[u] * csv[u] + rot * snv[u];
      }
    }
    if (t < dim) {
      const float rot = t < half ? -knew[t + half] : knew[t - half];
      rk = kn * ck + rot * sk;
    }
    __syncthreads();
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int i = t + 256 * u;
      if (i < gd) qs[i] = rq[u];
    }
    if (t < dim) {
      knew[t] = rk;
      if (own) {
        kcache[((size_t)g * max_seq + p) * dim + t] = rk;
        vcache[((size_t)g * max_seq + p) * dim + t] = vn;
      }
    }
  }
  const int ld = dim + 1;

  // scores s_j = (q_h . k_j) * scale for the chunk, one K tile at a time
  for (int jt = j0; jt < j1; jt += TJ) {
    const int nt = min(TJ, j1 - jt);
    if (jt != j0) {
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int i = t + 256 * u, jj = i / d4;
        if (jj < nt) r[u] = reinterpret_cast<const float4*>(kc + (size_t)(jt + jj) * dim)[i % d4];
      }
    }
    __syncthreads();  // q / knew staged; the previous tile consumed
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int i = t + 256 * u, jj = i / d4;
      if (jj < nt) {
        float* dst = kt + jj * ld + 4 * (i % d4);
        dst[0] = r[u].x;
        dst[1] = r[u].y;
        dst[2] = r[u].z;
        dst[3] = r[u].w;
      }
    }
    __syncthreads();
    if (rope && own && p >= jt && p < jt + nt) {  // the appended position comes from LDS, not the cache
      for (int d = t; d < dim; d += 256) kt[(p - jt) * ld + d] = knew[d];
      __syncthreads();
    }
    const int jj = t % TJ;
    if (jj < nt) {
      const float* kr = kt + jj * ld;
      for (int hl = t / TJ; hl < G; hl += 256 / TJ) {
        const float* qh = qs + hl * dim;
        float acc = 0.0f;
        for (int d = 0; d < dim; ++d) acc += qh[d] * kr[d];
        sc[hl * kAttnMaxChunk + (jt - j0) + jj] = acc * scale;
      }
    }
  }
  __syncthreads();

  // chunk softmax state per head (one wave per head)
  for (int hl = wave; hl < G; hl += 4) {
    float* sh = sc + hl * kAttnMaxChunk;
    float mx = -INFINITY;
    for (int j = lane; j < nc; j += 64) mx = fmaxf(mx, sh[j]);
    mx = wave_max(mx);
    float sum = 0.0f;
    for (int j = lane; j < nc; j += 64) {
      const float e = expf(sh[j] - mx);
      sh[j] = e;
      sum += e;
    }
    sum = wave_sum(sum);
    if (lane == 0) {
      stat[2 * hl] = mx;
      stat[2 * hl + 1] = sum;
    }
  }
  __syncthreads();

  // o_h = sum_j e_hj v_j: thread (column c4, row slot rs) over rows j0 + rs + RS*k
  float4 acc[kAttnMaxG];
#pragma unroll
  for (int hl = 0; hl < kAttnMaxG; ++hl) acc[hl] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  for (int jb = j0 + rs; jb < j1; jb += 4 * RS) {
    if (jb != j0 + rs) {
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int j = jb + u * RS;
        if (j < j1) {
          const float* row = (rope && j == p) ? v_new + (size_t)g * dim : vc + (size_t)j * dim;
          vv[u] = reinterpret_cast<const float4*>(row)[c4];
        }
      }
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int j = jb + u * RS;
      if (j < j1) {
#pragma unroll
        for (int hl = 0; hl < kAttnMaxG; ++hl) {
          if (hl < G) {
            const float e = sc[hl * kAttnMaxChunk + (j - j0)];
            acc[hl].x += e * vv[u].x;
            acc[hl].y += e * vv[u].y;
            acc[hl].z += e * vv[u].z;
            acc[hl].w += e * vv[u].w;
          }
        }
      }
    }
  }
  float* red = kt;  // RS x G x dim partial sums (1024 * G floats)
#pragma unroll
  for (int hl = 0; hl < kAttnMaxG; ++hl)
    if (hl < G) reinterpret_cast<float4*>(red + (rs * G + hl) * dim)[c4] = acc[hl];
  __syncthreads();
  const size_t rec = (size_t)dim + 2;  // per (chunk, head): m, l, o[dim]
  for (int i = t; i < gd; i += 256) {
    const int hl = i / dim, dd = i % dim;
    float o = 0.0f;
    for (int q2 = 0; q2 < RS; ++q2) o += red[(q2 * G + hl) * dim + dd];
    part[((size_t)c * heads + g * G + hl) * rec + 2 + dd] = o;
  }
  if (t < G) {
    part[((size_t)c * heads + g * G + t) * rec] = nc > 0 ? stat[2 * t] : -INFINITY;
    part[((size_t)c * heads + g * G + t) * rec + 1] = nc > 0 ? stat[2 * t + 1] : 0.0f;
  }
}

// out[h] = sum_c exp(m_c - M) o_c / sum_c exp(m_c - M) l_c over the S chunk
// records of head h (chunk order). One workgroup of dim threads per head.
extern "C" __global__ void __launch_bounds__(256) qmm_decode_attention_merge(const float* __restrict__ part,
                                                                            float* __restrict__ out, int heads,
                                                                            int dim) {
#pragma clang fp contract(off)
  constexpr int S = qmm::kAttnSplits;
  const int h = blockIdx.x, d = threadIdx.x;
  const size_t rec = (size_t)dim + 2;
  float mc[S], lc[S], oc[S];
#pragma unroll
  for (int c = 0; c < S; ++c) {
    const float* r = part + ((size_t)c * heads + h) * rec;
    mc[c] = r[0];
    lc[c] = r[1];
    oc[c] = r[2 + d];
  }
  float M = -INFINITY;
#pragma unroll
  for (int c = 0; c < S; ++c) M = fmaxf(M, mc[c]);
  float lsum = 0.0f, o = 0.0f;
#pragma unroll
  for (int c = 0; c < S; ++c) {
    if (mc[c] != -INFINITY) {
      const float w = expf(mc[c] - M);
      lsum += lc[c] * w;
      o += oc[c] * w;
    }
  }
  out[(size_t)h * dim + d] = o / lsum;
}

// hq = Q8_K(silu(g) * u) for `rows` rows of k elements (one wave per block).
extern "C" __global__ void __launch_bounds__(256) qmm_silu_mul_q8k(const float* __restrict__ g,
                                                                   const float* __restrict__ u, long long ld,
                                                                   uint8_t* __restrict__ hq, int k, int rows) {
#pragma clang fp contract(off)
  const int nb = k / 256;
  const long long w = (long long)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (w >= (long long)rows * nb) return;
  const int row = (int)(w / nb), b = (int)(w % nb), lane = threadIdx.x & 63;
  const long long o = row * ld + 256LL * b + 4 * lane;
  float e[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) e[j] = qmm::silu_mul(g[o + j], u[o + j]);
  const qmm::Q8KLane q = qmm::q8k_lane_vals(e[0], e[1], e[2], e[3], lane);
  uint8_t* blk = hq + w * qmm::kQ8KBytes;
  reinterpret_cast<uint32_t*>(blk + 4)[lane] = q.packed;
  const int next = __shfl_down(q.sum16, 4);
  if ((lane & 7) == 0)
    reinterpret_cast<uint32_t*>(blk + 4 + 256)[lane >> 3] = ((uint32_t)q.sum16 & 0xffffu) | ((uint32_t)next << 16);
  if (lane == 0) *reinterpret_cast<float*>(blk) = q.d;
}

// Greedy step end: the argmax of logits (lowest index on ties) becomes
// tokens[p + 1] unless that slot is still inside the prompt (p + 1 < prompt);
// then pos[0] = p + 1. Nothing is written once p + 1 reaches `capacity`
// (the length of tokens and of the KV cache), so pos never leaves
// [0, capacity). Each workgroup reduces a contiguous slice to (value, index)
// in the workspace; the last one to finish (a counter it resets to zero)
// reduces the slices in order and advances the step.
namespace qmm {
__device__ __forceinline__ void argmax_merge(float& best, int& idx, float ov, int oi) {
  if (ov > best || (ov == best && oi < idx)) {
    best = ov;
    idx = oi;
  }
}

__device__ __forceinline__ void block_argmax(float& best, int& idx, float* bv, int* bi) {
  for (int off = 1; off < 64; off <<= 1) argmax_merge(best, idx, __shfl_xor(best, off), __shfl_xor(idx, off));
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) {
    bv[wave] = best;
    bi[wave] = idx;
  }
  __syncthreads();
  if (threadIdx.x == 0)
    for (int w = 1; w < (int)(blockDim.x >> 6); ++w) argmax_merge(best, idx, bv[w], bi[w]);
}
}  // namespace qmm

extern "C" __global__ void __launch_bounds__(256) qmm_decode_argmax(const float* __restrict__ logits, int n,
                                                                    int* __restrict__ tokens, int capacity,
                                                                    int* __restrict__ pos, int prompt,
                                                                    float* __restrict__ pval,
                                                                    int* __restrict__ pidx,
                                                                    unsigned* __restrict__ counter) {
  __shared__ float bv[4];
  __shared__ int bi[4];
  __shared__ int last;
  const int per = (n + gridDim.x - 1) / gridDim.x;
  const int i0 = blockIdx.x * per, i1 = min(n, i0 + per);
  float best = -INFINITY;
  int idx = 0x7fffffff;
  for (int i = i0 + threadIdx.x; i < i1; i += blockDim.x) qmm::argmax_merge(best, idx, logits[i], i);
  qmm::block_argmax(best, idx, bv, bi);
  if (threadIdx.x == 0) {
    pval[blockIdx.x] = best;
    pidx[blockIdx.x] = idx;
    __threadfence();
    last = atomicAdd(counter, 1u) == gridDim.x - 1;
  }
  __syncthreads();
  if (!last) return;
  __threadfence();  // acquire: the other workgroups' slices are visible to plain loads
  best = -INFINITY;
  idx = 0x7fffffff;
  for (int b = threadIdx.x; b < (int)gridDim.x; b += blockDim.x) qmm::argmax_merge(best, idx, pval[b], pidx[b]);
  __syncthreads();
  qmm::block_argmax(best, idx, bv, bi);
  if (threadIdx.x == 0) {
    const int p = pos[0];
    if (p + 1 < capacity) {
      if (p + 1 >= prompt) tokens[p + 1] = idx;
      pos[0] = p + 1;
    }
    __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// RMSNorm of m rows (row stride ldx) of k elements into out (row stride ldo):
// x / sqrt(mean(x^2) + eps) * w. One workgroup per row.
extern "C" __global__ void __launch_bounds__(256) qmm_rms_norm(const float* __restrict__ x, long long ldx,
                                                               const float* __restrict__ w, float eps, int k,
                                                               float* __restrict__ out, long long ldo) {
#pragma clang fp contract(off)
  __shared__ float red[4];
  const float* xr = x + blockIdx.x * ldx;
  float ss = 0.0f;
  for (int i = threadIdx.x; i < k; i += blockDim.x) ss += xr[i] * xr[i];
  ss = qmm::wave_sum(ss);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
  __syncthreads();
  float t = 0.0f;
  for (int i = 0; i < (int)(blockDim.x >> 6); ++i) t += red[i];
  const float den = sqrtf(t / (float)k + eps);
  for (int i = threadIdx.x; i < k; i += blockDim.x) out[blockIdx.x * ldo + i] = xr[i] / den * w[i];
}
