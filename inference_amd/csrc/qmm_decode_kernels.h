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

// One query token against positions 0..pos[0] of the cache: for head h (kv
// head h / (heads / kv_heads)), s_j = (q . k_j) * scale, p = softmax(s),
// out = sum_j p_j v_j. One workgroup (256 threads) per head; up to 4096
// positions.
extern "C" __global__ void __launch_bounds__(256) qmm_decode_attention(const float* __restrict__ q,
                                                                       const float* __restrict__ kcache,
                                                                       const float* __restrict__ vcache,
                                                                       const int* __restrict__ pos,
                                                                       float* __restrict__ out, int heads,
                                                                       int kv_heads, int dim, int max_seq,
                                                                       float scale) {
#pragma clang fp contract(off)
  __shared__ float qs[256];
  __shared__ float sc[4096];
  __shared__ float red[8];
  const int h = blockIdx.x, g = h / (heads / kv_heads);
  const int n = min(max(pos[0], 0), max_seq - 1) + 1;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6, nw = blockDim.x >> 6;
  for (int i = t; i < dim; i += blockDim.x) qs[i] = q[(size_t)h * dim + i];
  __syncthreads();
  const float* kc = kcache + (size_t)g * max_seq * dim;
  const float* vc = vcache + (size_t)g * max_seq * dim;
  // scores: one position per thread per pass, dot product in index order
  float mx = -INFINITY;
  for (int j = t; j < n; j += blockDim.x) {
    const float* kj = kc + (size_t)j * dim;
    float acc = 0.0f;
    for (int d = 0; d < dim; ++d) acc += qs[d] * kj[d];
    const float sj = acc * scale;
    sc[j] = sj;
    mx = fmaxf(mx, sj);
  }
  mx = qmm::wave_max(mx);
  if (lane == 0) red[wave] = mx;
  __syncthreads();
  mx = red[0];
  for (int w = 1; w < nw; ++w) mx = fmaxf(mx, red[w]);
  __syncthreads();
  float sum = 0.0f;
  for (int j = t; j < n; j += blockDim.x) {
    const float e = expf(sc[j] - mx);
    sc[j] = e;
    sum += e;
  }
  sum = qmm::wave_sum(sum);
  if (lane == 0) red[wave] = sum;
  __syncthreads();
  float tot = 0.0f;
  for (int w = 0; w < nw; ++w) tot += red[w];
  // weighted sum of values: one output dimension per thread
  for (int d = t; d < dim; d += blockDim.x) {
    float acc = 0.0f;
    for (int j = 0; j < n; ++j) acc += (sc[j] / tot) * vc[(size_t)j * dim + d];
    out[(size_t)h * dim + d] = acc;
  }
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
  for (int j = 0; j < 4; ++j) {
    const float v = g[o + j];
    e[j] = v / (1.0f + expf(-v)) * u[o + j];
  }
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
// [0, capacity). One workgroup of 1024 threads.
extern "C" __global__ void __launch_bounds__(1024) qmm_decode_argmax(const float* __restrict__ logits, int n,
                                                                     int* __restrict__ tokens, int capacity,
                                                                     int* __restrict__ pos, int prompt) {
  __shared__ float bv[16];
  __shared__ int bi[16];
  float best = -INFINITY;
  int idx = 0x7fffffff;
  for (int i = threadIdx.x; i < n; i += blockDim.x) {
    const float v = logits[i];
    if (v > best) {
      best = v;
      idx = i;
    }
  }
  for (int off = 1; off < 64; off <<= 1) {
    const float ov = __shfl_xor(best, off);
    const int oi = __shfl_xor(idx, off);
    if (ov > best || (ov == best && oi < idx)) {
      best = ov;
      idx = oi;
    }
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) {
    bv[wave] = best;
    bi[wave] = idx;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < (int)(blockDim.x >> 6); ++w)
      if (bv[w] > best || (bv[w] == best && bi[w] < idx)) {
        best = bv[w];
        idx = bi[w];
      }
    const int p = pos[0];
    if (p + 1 < capacity) {
      if (p + 1 >= prompt) tokens[p + 1] = idx;
      pos[0] = p + 1;
    }
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
