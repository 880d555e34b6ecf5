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

// Row `tok` of the embedding table into x[0 : hidden); a token id outside
// [0, vocab) reads nothing and writes a NaN row, so the step's logits show it.
namespace qmm {
__device__ __forceinline__ void embed_row(const float* __restrict__ table, long long ld, int tok, int vocab,
                                          float* __restrict__ x, int hidden) {
  const bool ok = tok >= 0 && tok < vocab;
  const float* row = table + (long long)(ok ? tok : 0) * ld;
  for (int c = blockIdx.x * blockDim.x + threadIdx.x; c < hidden; c += gridDim.x * blockDim.x)
    x[c] = ok ? row[c] : __builtin_nanf("");
}
}  // namespace qmm

// x[i][0 : hidden) = table[tokens[first + i]][0 : hidden) for i < gridDim.y
// (the prompt rows of a batched prefill).
extern "C" __global__ void qmm_prefill_embed(const float* __restrict__ table, long long ld, int vocab,
                                             const int* __restrict__ tokens, int first, float* __restrict__ x,
                                             int hidden) {
  const int i = blockIdx.y;
  qmm::embed_row(table, ld, tokens[first + i], vocab, x + (long long)i * hidden, hidden);
}

// x[0 : hidden) = table[tokens[pos[0]]][0 : hidden)
extern "C" __global__ void qmm_decode_embed(const float* __restrict__ table, long long ld, int vocab,
                                            const int* __restrict__ tokens, const int* __restrict__ pos,
                                            float* __restrict__ x, int hidden) {
  qmm::embed_row(table, ld, tokens[pos[0]], vocab, x, hidden);
}

// Rotates q (heads x dim) and k (kv_heads x dim) at position p = pos[0] with
// cos/sin rows [p][dim] (cat(freqs, freqs) layout: pairs (i, i + dim/2)), in
// place, and appends k, v to the layer's cache [kv_heads][max_seq][dim].
// One workgroup per head (q heads first, then kv heads). A position outside
// [0, max_seq) writes nothing.
namespace qmm {
__device__ __forceinline__ void rope_kv_row(float* __restrict__ q, float* __restrict__ k, const float* __restrict__ v,
                                            const float* __restrict__ cos_t, const float* __restrict__ sin_t, int p,
                                            float* __restrict__ kcache, float* __restrict__ vcache, int heads,
                                            int dim, int max_seq) {
#pragma clang fp contract(off)
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
}  // namespace qmm

extern "C" __global__ void qmm_decode_rope_kv(float* __restrict__ q, float* __restrict__ k,
                                              const float* __restrict__ v, const float* __restrict__ cos_t,
                                              const float* __restrict__ sin_t, const int* __restrict__ pos,
                                              float* __restrict__ kcache, float* __restrict__ vcache, int heads,
                                              int kv_heads, int dim, int max_seq) {
  (void)kv_heads;
  qmm::rope_kv_row(q, k, v, cos_t, sin_t, pos[0], kcache, vcache, heads, dim, max_seq);
}

// Prompt rows i < gridDim.y at positions first + i: row i of q / k / v starts
// at q + i * ldq (k, v likewise).
extern "C" __global__ void qmm_prefill_rope_kv(float* __restrict__ q, float* __restrict__ k,
                                               const float* __restrict__ v, long long ldq, long long ldk,
                                               long long ldv, const float* __restrict__ cos_t,
                                               const float* __restrict__ sin_t, int first,
                                               float* __restrict__ kcache, float* __restrict__ vcache, int heads,
                                               int dim, int max_seq) {
  const int i = blockIdx.y;
  qmm::rope_kv_row(q + i * ldq, k + i * ldk, v + i * ldv, cos_t, sin_t, first + i, kcache, vcache, heads, dim,
                   max_seq);
}

// The same from the q / k / v GEMMs' unsummed split-K partials (qp
// [qs][m][heads * dim], kp / vp [ks] / [vs][m][kv_heads * dim]; one split is
// the plain output): each element is summed in split order as qmm_splitk_sum
// sums it, then rotated exactly as qmm_prefill_rope_kv rotates it; the
// rotated q rows go to q (row stride ldq), k and v to the caches only.
extern "C" __global__ void qmm_prefill_splitk_rope_kv(const float* __restrict__ qp, int qs,
                                                      const float* __restrict__ kp, int ks,
                                                      const float* __restrict__ vp, int vs, int m,
                                                      float* __restrict__ q, long long ldq,
                                                      const float* __restrict__ cos_t,
                                                      const float* __restrict__ sin_t, int first,
                                                      float* __restrict__ kcache, float* __restrict__ vcache,
                                                      int heads, int kv_heads, int dim, int max_seq) {
#pragma clang fp contract(off)
  __shared__ float row[1024];
  const int r = blockIdx.y, h = blockIdx.x, i = threadIdx.x;
  const int p = first + r;
  if (p < 0 || p >= max_seq) return;
  const bool isq = h < heads;
  const int g = h - heads;
  const int width = isq ? heads * dim : kv_heads * dim;
  const float* src = isq ? qp : kp;
  const int splits = isq ? qs : ks;
  const size_t plane = (size_t)m * width;
  const size_t o = (size_t)r * width + (size_t)(isq ? h : g) * dim + i;
  float x = 0.0f;
  if (i < dim) {
    x = src[o];
    for (int j = 1; j < splits; ++j) x += src[o + j * plane];
    row[i] = x;
  }
  __syncthreads();
  if (i >= dim) return;
  const int half = dim / 2;
  const float rot = i < half ? -row[i + half] : row[i - half];
  const float out = x * cos_t[(size_t)p * dim + i] + rot * sin_t[(size_t)p * dim + i];
  if (isq) {
    q[(size_t)r * ldq + (size_t)h * dim + i] = out;
    return;
  }
  kcache[((size_t)g * max_seq + p) * dim + i] = out;
  float v = vp[o];
  for (int j = 1; j < vs; ++j) v += vp[o + j * (size_t)m * width];
  vcache[((size_t)g * max_seq + p) * dim + i] = v;
}

// One query token against positions 0..p of the cache (p = pos[0]) in one
// launch ("flash decoding" with the merge done by the last workgroup).
//
// Workgroup (g, c) of a kv_heads x S grid takes the G = heads / kv_heads
// query heads of kv head g (repeat_kv maps query head h to kv head h / G)
// and the c-th of S contiguous chunks of the n = p + 1 positions. Its lanes
// form 16-lane rows, 4 NW of them; row r scans positions c0 + r,
// c0 + r + 4 NW, ... of the chunk straight from the cache, lane i of a row
// holding dims [i * dim/16, (i+1) * dim/16) of q, k_j and v_j, so a score
// s_j = (q . k_j) * scale is a 16-lane sum (4 DPP steps) and the softmax runs
// online per row, a batch of positions at a time (m = running max,
// l = sum exp(s - m), o = sum exp(s - m) v). The next batch's k/v rows are
// loaded while the current batch is scored. The rows' states are combined
// through LDS.
//
// The chunk's record (m, l, o[dim]) per head goes to the workspace; one
// thread then bumps the kv head's counter with a device-scope (agent)
// atomic, and the workgroup that brings it to S is the last of its kv head:
// it reads the S records back, forms
// out = sum_c exp(m_c - M) o_c / sum_c exp(m_c - M) l_c (M = max_c m_c,
// chunks in order) and resets the counter to zero, so the workspace is ready
// for the next launch.
//
// Ordering. Every access to the records is an agent-scope atomic (relaxed),
// so the protocol is the memory model's release/acquire sequence without the
// cache maintenance that only non-atomic data needs. On gfx942/gfx950 an
// agent-scope release is "buffer_wbl2 sc1; s_waitcnt vmcnt(0)" and an
// acquire "s_waitcnt vmcnt(0); buffer_inv sc1" (LLVM AMDGPUUsage, memory
// model GFX942): the L2 writeback makes earlier plain stores visible across
// the XCDs' separate L2s, the invalidate keeps later plain loads from stale
// L2 lines. Agent-scope atomic stores and loads carry sc1 themselves (the
// store writes through the L2, the load is served from the device-coherent
// level), so neither is needed for them; what remains is the wait: each
// thread's s_waitcnt vmcnt(0) before the barrier completes its record
// stores before thread 0's counter atomic is issued, and the reader's loads
// are issued after the atomic's result is back. The full acquire-release
// form (plain records, acq_rel counter) was measured: its whole-L2 writeback
// and invalidate in every workgroup cost 1.4% of decode throughput (config 3:
// 488 vs 495 tok/s).
//
// With cos/sin (fused RoPE + KV append), q and k are the unrotated
// projections: q is rotated in registers (the partner of dim d is 8 lanes
// away in its row); the workgroup whose chunk holds p rotates k, appends k and v at
// position p of the cache and uses them for that position. Without cos/sin,
// q is already rotated and the cache already holds position p.
// dim = 64 * DPL (64, 128, 256); G <= GT (1, 2, 4, 8).
namespace qmm {
constexpr int kAttnSplits = 16;  // S

// One lane's share of a dim-wide row in the 16-lane-row layout: lane li
// (0..15) of every row holds dims [R * li, R * li + R) with R = dim / 16.
template <int R>
__device__ __forceinline__ void attn_part(float (&dst)[R], const float* __restrict__ row, int li) {
  const float4* p = reinterpret_cast<const float4*>(row + R * li);
#pragma unroll
  for (int c = 0; c < R / 4; ++c) {
    const float4 v = p[c];
    dst[4 * c] = v.x;
    dst[4 * c + 1] = v.y;
    dst[4 * c + 2] = v.z;
    dst[4 * c + 3] = v.w;
  }
}

// x * cos + rotate_half(x) * sin with rotate_half = cat(-x2, x1): lanes 0..7
// of a row hold the first half of the dims, their partners are 8 lanes on
// (a rotate by 8 within the row).
template <int R>
__device__ __forceinline__ void attn_rope(float (&x)[R], const float (&cs)[R], const float (&sn)[R], int li) {
#pragma clang fp contract(off)
#pragma unroll
  for (int e = 0; e < R; ++e) {
    const float other = dpp_f<0x128>(x[e]);  // row_ror:8
    const float rot = li < 8 ? -other : other;
    x[e] = x[e] * cs[e] + rot * sn[e];
  }
}

// Sum over a row of 16 lanes (every lane of the row receives it).
__device__ __forceinline__ float row16_total(float v) {
  v += dpp_f<0xb1>(v);   // quad_perm [1,0,3,2]
  v += dpp_f<0x4e>(v);   // quad_perm [2,3,0,1]
  v += dpp_f<0x141>(v);  // row_half_mirror
  v += dpp_f<0x140>(v);  // row_mirror
  return v;
}

// PREFILL: one query per workgroup row, all its positions in one chunk: query
// row i = blockIdx.y (position first + i, q row at q + i * ldq) attends to
// positions 0 ..= first + i of the cache (which already holds them, rotated;
// q is already rotated) and writes its normalised output to out + i * ldo.
// The arithmetic is the S = 1 case of the chunked form (the merge of one
// record multiplies by e^0 = 1).
// PLANES (PREFILL only): instead of f32 rows, the query row's G * dim
// outputs (whole 256-element blocks: G * dim % 256 == 0, starting at column
// g * G * dim) go to the Q8_K GEMM planes of row blockIdx.y (q8 / d / s over
// rows of kq values), quantized as qmm_quantize_q8k_mmq quantizes the f32 row.
template <int DPL, int GT, int NW, bool PREFILL = false, bool PLANES = false>
__device__ __forceinline__ void decode_attention(const float* __restrict__ q, const float* __restrict__ k_new,
                                                 const float* __restrict__ v_new, const float* __restrict__ cos_t,
                                                 const float* __restrict__ sin_t, const int* __restrict__ pos,
                                                 float* __restrict__ kcache, float* __restrict__ vcache,
                                                 float* __restrict__ part, unsigned* __restrict__ counters,
                                                 float* __restrict__ out, int heads, int kv_heads, int max_seq,
                                                 float scale, int first = 0, long long ldq = 0,
                                                 long long ldo = 0, int8_t* __restrict__ pq8 = nullptr,
                                                 float* __restrict__ pd = nullptr, int16_t* __restrict__ ps = nullptr,
                                                 int kq = 0) {
#pragma clang fp contract(off)
  constexpr int dim = 64 * DPL;
  constexpr int R = dim / 16;  // dims per lane: a 16-lane row holds one position's row
  constexpr int NR = 4 * NW;   // rows of 16 lanes in the workgroup, each scanning its own positions
  constexpr int B = 2;         // positions per row and batch
  constexpr int NT = 64 * NW;
  __shared__ float wst[NR][2 * GT];
  __shared__ __attribute__((aligned(16))) float wo[NR][GT * dim];
  __shared__ int last;
  __shared__ __attribute__((aligned(16))) float ob[PLANES ? GT * dim : 1];  // PLANES: the row's outputs
  const int g = blockIdx.x, c = PREFILL ? 0 : blockIdx.y, t = threadIdx.x;
  const int lane = t & 63, wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int li = lane & 15, row = 4 * wave + (lane >> 4);  // this lane's place in its row, the row's index
  const int G = heads / kv_heads;
  constexpr int S = PREFILL ? 1 : kAttnSplits;
  const bool rope = !PREFILL && cos_t != nullptr;
  if constexpr (PREFILL) {
    q += blockIdx.y * ldq;
    out += blockIdx.y * ldo;
  }

  // loads, batch 1: pos, q of the group's heads, new k / v rows
  const int p = PREFILL ? min(first + (int)blockIdx.y, max_seq - 1) : min(max(pos[0], 0), max_seq - 1);
  float qv[GT][R];
#pragma unroll
  for (int h = 0; h < GT; ++h) attn_part<R>(qv[h], q + (size_t)(g * G + min(h, G - 1)) * dim, li);
  float kn[R], vn[R];
  if (rope) {
    attn_part<R>(kn, k_new + (size_t)g * dim, li);
    attn_part<R>(vn, v_new + (size_t)g * dim, li);
  }

  const int n = p + 1;
  const int L = (n + S - 1) / S;
  const int j0 = min(c * L, n), j1 = min(j0 + L, n);
  const int nc = j1 - j0;
  const bool own = j0 <= p && p < j1;
  const float* kc = kcache + (size_t)g * max_seq * dim;
  const float* vc = vcache + (size_t)g * max_seq * dim;
  // row r scans positions j0 + r + NR i; the wave's first row has the most
  const int npos = nc > row ? (nc - row + NR - 1) / NR : 0;
  const int nwave = nc > 4 * wave ? (nc - 4 * wave + NR - 1) / NR : 0;  // wave-uniform loop bound

  // loads, batch 2: the row's first k / v rows (clamped into the chunk), cos / sin at p
  float kr[B][R], vr[B][R];
  const int jlast = max(j1 - 1, 0);
#pragma unroll
  for (int b = 0; b < B; ++b) {
    const int j = min(j0 + row + NR * b, jlast);
    attn_part<R>(kr[b], kc + (size_t)j * dim, li);
    attn_part<R>(vr[b], vc + (size_t)j * dim, li);
  }
  if (rope) {
    float cs[R], sn[R];
    attn_part<R>(cs, cos_t + (size_t)p * dim, li);
    attn_part<R>(sn, sin_t + (size_t)p * dim, li);
#pragma unroll
    for (int h = 0; h < GT; ++h) attn_rope<R>(qv[h], cs, sn, li);
    attn_rope<R>(kn, cs, sn, li);
    if (own && t < 16) {  // the first row appends position p
#pragma unroll
      for (int e = 0; e < R; ++e) {
        kcache[((size_t)g * max_seq + p) * dim + R * li + e] = kn[e];
        vcache[((size_t)g * max_seq + p) * dim + R * li + e] = vn[e];
      }
    }
  }

  float m[GT], l[GT], o[GT][R];
#pragma unroll
  for (int h = 0; h < GT; ++h) {
    m[h] = -INFINITY;
    l[h] = 0.0f;
#pragma unroll
    for (int e = 0; e < R; ++e) o[h][e] = 0.0f;
  }
  // One batch of B positions per row (i0 .. i0 + B - 1 of this row; those
  // past npos are clamped duplicates and are masked to score -inf, weight
  // 0): all B x GT scores first (16-lane row sums), then one online-softmax
  // update per head. A row with no position yet keeps m = -inf, and the
  // guards keep -inf - (-inf) out of exp.
  // A masked slot (a clamped duplicate past the row's positions) may hold a
  // cache row that is not written yet (the chunk owning p reads row p before
  // this launch appends it): its score is -inf and its value row is replaced
  // by zeros, so nothing stale (even a NaN) reaches the sums.
  auto scan = [&](const float (&kb)[B][R], const float (&vb)[B][R], int i0) {
    float sc[B][GT];
    float ks[B][R], vs[B][R];
#pragma unroll
    for (int b = 0; b < B; ++b) {
      const bool ok = i0 + b < npos;
      const bool at_p = rope && j0 + row + NR * (i0 + b) == p;
#pragma unroll
      for (int e = 0; e < R; ++e) {
        ks[b][e] = at_p ? kn[e] : kb[b][e];
        vs[b][e] = ok ? (at_p ? vn[e] : vb[b][e]) : 0.0f;
      }
#pragma unroll
      for (int h = 0; h < GT; ++h) {
        float d = 0.0f;
#pragma unroll
        for (int e = 0; e < R; ++e) d += qv[h][e] * ks[b][e];
        d = row16_total(d) * scale;
        sc[b][h] = ok ? d : -INFINITY;
      }
    }
#pragma unroll
    for (int h = 0; h < GT; ++h) {
      float mx = m[h];
#pragma unroll
      for (int b = 0; b < B; ++b) mx = fmaxf(mx, sc[b][h]);
      const float a = mx == -INFINITY ? 0.0f : expf(m[h] - mx);  // 0 while m = -inf
      float ls = l[h] * a;
      float acc[R];
#pragma unroll
      for (int e = 0; e < R; ++e) acc[e] = o[h][e] * a;
#pragma unroll
      for (int b = 0; b < B; ++b) {
        const float w = sc[b][h] == -INFINITY ? 0.0f : expf(sc[b][h] - mx);
        ls += w;
#pragma unroll
        for (int e = 0; e < R; ++e) acc[e] += w * vs[b][e];
      }
      m[h] = mx;
      l[h] = ls;
#pragma unroll
      for (int e = 0; e < R; ++e) o[h][e] = acc[e];
    }
  };
  if (nwave > 0) {
    int i0 = 0;
    for (; i0 + B < nwave; i0 += B) {
      // next batch in flight (clamped, unconditional) while this one is scored
      float kx[B][R], vx[B][R];
#pragma unroll
      for (int b = 0; b < B; ++b) {
        const int j = min(j0 + row + NR * (i0 + B + b), jlast);
        attn_part<R>(kx[b], kc + (size_t)j * dim, li);
        attn_part<R>(vx[b], vc + (size_t)j * dim, li);
      }
      scan(kr, vr, i0);
#pragma unroll
      for (int b = 0; b < B; ++b)
#pragma unroll
        for (int e = 0; e < R; ++e) {
          kr[b][e] = kx[b][e];
          vr[b][e] = vx[b][e];
        }
    }
    scan(kr, vr, i0);
  }

  // the rows' states -> the chunk's record per head
#pragma unroll
  for (int h = 0; h < GT; ++h)
#pragma unroll
    for (int e = 0; e < R; ++e) wo[row][h * dim + R * li + e] = o[h][e];
  if (li == 0) {
#pragma unroll
    for (int h = 0; h < GT; ++h) {
      wst[row][2 * h] = m[h];
      wst[row][2 * h + 1] = l[h];
    }
  }
  __syncthreads();
  const size_t rec = (size_t)dim + 2;  // per (chunk, head): m, l, o[dim]
  for (int i = t; i < G * dim; i += NT) {
    const int h = i / dim, d = i % dim;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < NR; ++w) M = fmaxf(M, wst[w][2 * h]);
    float lsum = 0.0f, osum = 0.0f;
#pragma unroll
    for (int w = 0; w < NR; ++w) {
      if (wst[w][2 * h] != -INFINITY) {
        const float a = expf(wst[w][2 * h] - M);
        lsum += wst[w][2 * h + 1] * a;
        osum += wo[w][i] * a;
      }
    }
    if constexpr (PLANES) {
      ob[i] = osum / lsum;
      continue;
    } else if constexpr (PREFILL) {
      out[(size_t)(g * G + h) * dim + d] = osum / lsum;
      continue;
    }
    float* r = part + ((size_t)c * heads + g * G + h) * rec;
    __hip_atomic_store(r + 2 + d, osum, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (d == 0) {
      __hip_atomic_store(r, M, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(r + 1, lsum, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  if constexpr (PLANES) {
    // one wave per 256-element block of the row's G * dim outputs
    __syncthreads();
    const int nb = kq / 256, nblk = G * dim / 256, b0 = g * G * dim / 256;
    for (int b = wave; b < nblk; b += NW)
      put_q8k_plane(q8k_lane(ob + 256 * b, lane), (long long)blockIdx.y * nb + b0 + b, nb, kq, pq8, pd, ps, lane);
    return;
  }
  if constexpr (PREFILL) return;
  // every thread's record stores have completed before the barrier, so they
  // precede thread 0's counter atomic
  __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0)
  __syncthreads();
  if (t == 0)
    last = __hip_atomic_fetch_add(counters + g, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (unsigned)(S - 1);
  __syncthreads();
  if (!last) return;

  // last workgroup of kv head g (its loads issue after the counter's result):
  // merge the S chunk records of its G heads
  for (int i = t; i < G * dim; i += NT) {
    const int h = g * G + i / dim, d = i % dim;
    float mc[S], lc[S], oc[S];
#pragma unroll
    for (int cc = 0; cc < S; ++cc) {
      const float* r = part + ((size_t)cc * heads + h) * rec;
      mc[cc] = __hip_atomic_load(r, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      lc[cc] = __hip_atomic_load(r + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      oc[cc] = __hip_atomic_load(r + 2 + d, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    float M = -INFINITY;
#pragma unroll
    for (int cc = 0; cc < S; ++cc) M = fmaxf(M, mc[cc]);
    float lsum = 0.0f, osum = 0.0f;
#pragma unroll
    for (int cc = 0; cc < S; ++cc) {
      if (mc[cc] != -INFINITY) {
        const float w = expf(mc[cc] - M);
        lsum += lc[cc] * w;
        osum += oc[cc] * w;
      }
    }
    out[(size_t)h * dim + d] = osum / lsum;
  }
  if (t == 0) __hip_atomic_store(counters + g, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
}  // namespace qmm

// L2 warming for the launches that follow the attention. The attention
// leaves most CUs idle and HBM nearly so for its whole duration, while the
// next launches (the o projection, then gate/up) each start by waiting on
// their first weight loads. Workgroups past the attention's own (grid rows
// y >= kAttnSplits) load those first rows instead: each L2 is private to one
// XCD and survives kernel boundaries, and a dispatch deals its workgroups to
// the eight XCDs round-robin by linear index, so warming workgroup j (the
// j-th past the attention's kv_heads * kAttnSplits, a multiple of 8) shares an
// XCD, and its L2, with workgroup j of the one-row GEMV launch whose rows it
// loads: rows j * nw + i + k * grid_waves (wave i, k-th row of the wave) of
// the launch's concatenated jobs. The loads change no memory; where the
// dispatch order differs, the rows are still warm in the memory-side cache.
namespace qmm {
constexpr int kPfJobs = 3;
struct PfJobs {
  const uint8_t* w[kPfJobs];   // device blocks of each job's rows (row-major)
  unsigned row_bytes[kPfJobs];  // bytes of one row's block bodies
  int rows[kPfJobs];            // rows of the job
  int first[kPfJobs];           // the job's first global row in its launch
  int grid_waves[kPfJobs];      // waves of the consuming launch
  int kmax[kPfJobs];            // rows per wave to warm
  int njobs;
  int nw;                       // waves per workgroup of the consuming launches
};

template <typename T>
__device__ __forceinline__ T pick3(const T (&a)[kPfJobs], int i) {  // constant indices only (no scratch)
  return i == 0 ? a[0] : i == 1 ? a[1] : a[2];
}

// Warming workgroup j (of nwarm, a multiple of 8) loads for the consuming
// launches' workgroups j, j + nwarm, ... (all on its XCD). The loads go
// straight to LDS (global_load_lds_dwordx4), into one 1 KB area per wave that
// nothing reads: they hold no registers, so a wave keeps all of its loads in
// flight at once instead of waiting a round trip per batch.
__device__ __forceinline__ void l2_warm(const PfJobs& pf, int j, int nwarm) {
  __shared__ __attribute__((aligned(16))) uint8_t dump[16 * 1024];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int nwv = blockDim.x >> 6;
  auto* dst = (__attribute__((address_space(3))) void*)(dump + 1024 * (wave & 15));
#pragma unroll 1
  for (int jb = 0; jb < pf.njobs; ++jb) {
    const uint8_t* w = pick3(pf.w, jb);
    const unsigned rb = pick3(pf.row_bytes, jb);
    const int rows = pick3(pf.rows, jb), first = pick3(pf.first, jb), gw = pick3(pf.grid_waves, jb);
    const int kmax = pick3(pf.kmax, jb), nc = gw / pf.nw;
#pragma unroll 1
    for (int k = 0; k < kmax; ++k)
#pragma unroll 1
      for (int c = j; c < nc; c += nwarm) {
        // the consuming workgroup c's rows c * nw + i (i < nw) of the k-th
        // round are consecutive rows of its launch: one contiguous range
        const int g0 = c * pf.nw + k * gw - first;
        const int r0 = max(g0, 0), r1 = min(g0 + pf.nw, rows);
        if (r0 >= r1) continue;
        const uint8_t* base = w + (size_t)r0 * rb;
        const unsigned len = (unsigned)(r1 - r0) * rb;  // a multiple of 16, inside the weight
#pragma unroll 1
        for (unsigned ch = (unsigned)wave; 1024u * ch < len; ch += (unsigned)nwv) {
          const unsigned o = min(1024u * ch + 16u * (unsigned)lane, len - 16u);
          __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(base + o), dst, 16, 0, 0);
        }
      }
  }
}
}  // namespace qmm

#define QMM_PF_PARAMS(i) const uint8_t *pfw##i, unsigned pfb##i, int pfr##i, int pff##i, int pfg##i, int pfk##i
#define QMM_PF_SET(i)  \
  pf.w[i] = pfw##i;    \
  pf.row_bytes[i] = pfb##i; \
  pf.rows[i] = pfr##i; \
  pf.first[i] = pff##i; \
  pf.grid_waves[i] = pfg##i; \
  pf.kmax[i] = pfk##i;

#define QMM_ATTN_KERNEL(DPL, GT, NW)                                                                             \
  extern "C" __global__ void __launch_bounds__(64 * NW) qmm_decode_attention_d##DPL##_g##GT##_w##NW(             \
      const float* __restrict__ q, const float* __restrict__ k_new, const float* __restrict__ v_new,            \
      const float* __restrict__ cos_t, const float* __restrict__ sin_t, const int* __restrict__ pos,            \
      float* __restrict__ kcache, float* __restrict__ vcache, float* __restrict__ part,                         \
      unsigned* __restrict__ counters, float* __restrict__ out, int heads, int kv_heads, int max_seq,           \
      float scale, QMM_PF_PARAMS(0), QMM_PF_PARAMS(1), QMM_PF_PARAMS(2), int pf_njobs, int pf_nw) {           \
    if (blockIdx.y >= (unsigned)qmm::kAttnSplits) {                                                              \
      qmm::PfJobs pf;                                                                                            \
      QMM_PF_SET(0) QMM_PF_SET(1) QMM_PF_SET(2)                                                                  \
      pf.njobs = pf_njobs;                                                                                       \
      pf.nw = pf_nw;                                                                                             \
      const int j = (int)(blockIdx.x + (blockIdx.y - qmm::kAttnSplits) * gridDim.x);                            \
      const int nwarm = (int)((gridDim.y - qmm::kAttnSplits) * gridDim.x);                                      \
      qmm::l2_warm(pf, j, nwarm);                                                                                \
      return;                                                                                                    \
    }                                                                                                            \
    qmm::decode_attention<DPL, GT, NW>(q, k_new, v_new, cos_t, sin_t, pos, kcache, vcache, part, counters, out, \
                                       heads, kv_heads, max_seq, scale);                                        \
  }
// Eight waves (32 rows) where their LDS staging of the rows' states fits
// (GT * dim <= 512: 64 KB), four otherwise; the host picks the same.
QMM_ATTN_KERNEL(1, 1, 8) QMM_ATTN_KERNEL(1, 2, 8) QMM_ATTN_KERNEL(1, 4, 8) QMM_ATTN_KERNEL(1, 8, 8)
QMM_ATTN_KERNEL(2, 1, 8) QMM_ATTN_KERNEL(2, 2, 8) QMM_ATTN_KERNEL(2, 4, 8) QMM_ATTN_KERNEL(2, 8, 4)
QMM_ATTN_KERNEL(4, 1, 8) QMM_ATTN_KERNEL(4, 2, 8) QMM_ATTN_KERNEL(4, 4, 4) QMM_ATTN_KERNEL(4, 8, 4)


// Causal attention of a prompt's rows (batched prefill): grid kv_heads x rows.
#define QMM_PREFILL_ATTN_KERNEL(DPL, GT)                                                                         \
  extern "C" __global__ void __launch_bounds__(256) qmm_prefill_attention_d##DPL##_g##GT(                        \
      const float* __restrict__ q, long long ldq, const float* __restrict__ kcache,                              \
      const float* __restrict__ vcache, int first, float* __restrict__ out, long long ldo, int heads,            \
      int kv_heads, int max_seq, float scale) {                                                                  \
    qmm::decode_attention<DPL, GT, 4, true>(q, nullptr, nullptr, nullptr, nullptr, nullptr,                      \
                                            const_cast<float*>(kcache), const_cast<float*>(vcache), nullptr,     \
                                            nullptr, out, heads, kv_heads, max_seq, scale, first, ldq, ldo);     \
  }
#define QMM_PREFILL_ATTN_KERNELS(DPL) \
  QMM_PREFILL_ATTN_KERNEL(DPL, 1) QMM_PREFILL_ATTN_KERNEL(DPL, 2) QMM_PREFILL_ATTN_KERNEL(DPL, 4) QMM_PREFILL_ATTN_KERNEL(DPL, 8)
QMM_PREFILL_ATTN_KERNELS(1)
QMM_PREFILL_ATTN_KERNELS(2)
QMM_PREFILL_ATTN_KERNELS(4)

// The same attention writing the o projection's Q8_K GEMM planes (rows of kq
// = heads * head_dim values) instead of f32 rows; G * head_dim a multiple of
// 256 (the host checks it).
#define QMM_PREFILL_ATTN_PLANES_KERNEL(DPL, GT)                                                                  \
  extern "C" __global__ void __launch_bounds__(256) qmm_prefill_attention_planes_d##DPL##_g##GT(                 \
      const float* __restrict__ q, long long ldq, const float* __restrict__ kcache,                              \
      const float* __restrict__ vcache, int first, int8_t* __restrict__ q8, float* __restrict__ d,               \
      int16_t* __restrict__ s, int kq, int heads, int kv_heads, int max_seq, float scale) {                      \
    qmm::decode_attention<DPL, GT, 4, true, true>(q, nullptr, nullptr, nullptr, nullptr, nullptr,                \
                                                  const_cast<float*>(kcache), const_cast<float*>(vcache),        \
                                                  nullptr, nullptr, nullptr, heads, kv_heads, max_seq, scale,    \
                                                  first, ldq, 0, q8, d, s, kq);                                  \
  }
QMM_PREFILL_ATTN_PLANES_KERNEL(1, 4) QMM_PREFILL_ATTN_PLANES_KERNEL(1, 8)
QMM_PREFILL_ATTN_PLANES_KERNEL(2, 2) QMM_PREFILL_ATTN_PLANES_KERNEL(2, 4) QMM_PREFILL_ATTN_PLANES_KERNEL(2, 8)
QMM_PREFILL_ATTN_PLANES_KERNEL(4, 1) QMM_PREFILL_ATTN_PLANES_KERNEL(4, 2) QMM_PREFILL_ATTN_PLANES_KERNEL(4, 4)
QMM_PREFILL_ATTN_PLANES_KERNEL(4, 8)

// One Q8_K block of silu(g) * u (one wave): the 256 elements at g / u
// into the 292-byte block at blk.
namespace qmm {
__device__ __forceinline__ void silu_mul_q8k_block(const float* __restrict__ g, const float* __restrict__ u,
                                                   uint8_t* __restrict__ blk, int lane) {
#pragma clang fp contract(off)
  float e[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) e[j] = silu_mul(g[4 * lane + j], u[4 * lane + j]);
  const Q8KLane q = q8k_lane_vals(e[0], e[1], e[2], e[3], lane);
  reinterpret_cast<uint32_t*>(blk + 4)[lane] = q.packed;
  const int next = __shfl_down(q.sum16, 4);
  if ((lane & 7) == 0)
    reinterpret_cast<uint32_t*>(blk + 4 + 256)[lane >> 3] = ((uint32_t)q.sum16 & 0xffffu) | ((uint32_t)next << 16);
  if (lane == 0) *reinterpret_cast<float*>(blk) = q.d;
}
}  // namespace qmm

// hq = Q8_K(silu(g) * u) for `rows` rows of k elements (one wave per block).
extern "C" __global__ void __launch_bounds__(256) qmm_silu_mul_q8k(const float* __restrict__ g,
                                                                   const float* __restrict__ u, long long ld,
                                                                   uint8_t* __restrict__ hq, int k, int rows) {
  const int nb = k / 256;
  const long long w = (long long)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (w >= (long long)rows * nb) return;
  const int row = (int)(w / nb), b = (int)(w % nb);
  const long long o = row * ld + 256LL * b;
  qmm::silu_mul_q8k_block(g + o, u + o, hq + w * qmm::kQ8KBytes, threadIdx.x & 63);
}

// The same for the rows of per-expert ranges only: rows ot[e] .. ot[e] +
// ct[e] - 1 (ct[e] <= maxrows) of every expert e (the grouped prefill GEMM's
// tails, see qmm_moe_split_tails); row r's blocks land at hq + r * nb * 292.
extern "C" __global__ void __launch_bounds__(256) qmm_silu_mul_q8k_ranges(const float* __restrict__ g,
                                                                          const float* __restrict__ u, long long ld,
                                                                          uint8_t* __restrict__ hq, int k, int E,
                                                                          int maxrows, const int* __restrict__ ct,
                                                                          const int* __restrict__ ot) {
  const int nb = k / 256;
  const long long w = (long long)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (w >= (long long)E * maxrows * nb) return;
  const int b = (int)(w % nb), i = (int)((w / nb) % maxrows), e = (int)(w / ((long long)nb * maxrows));
  if (i >= ct[e]) return;
  const long long row = ot[e] + i, o = row * ld + 256LL * b;
  qmm::silu_mul_q8k_block(g + o, u + o, hq + (row * nb + b) * qmm::kQ8KBytes, threadIdx.x & 63);
}

// Greedy step end: the argmax of logits (lowest index on ties) becomes
// tokens[p + 1] unless that slot is still inside the prompt (p + 1 < prompt);
// then pos[0] = p + 1. Nothing is written once p + 1 reaches `capacity`
// (the length of tokens and of the KV cache), so pos never leaves
// [0, capacity). Each workgroup reduces a contiguous slice to (value, index)
// in the workspace; the last one to finish (a counter it resets to zero)
// reduces the slices in order and advances the step.
namespace qmm {
// (value, index) order of the reduction: NaN above every number (torch.argmax's
// rule, so a NaN logit is reported rather than skipped), then the larger value,
// then the lower index. Every element therefore claims its slot and the
// result is always an index the reduction saw.
__device__ __forceinline__ void argmax_merge(float& best, int& idx, float ov, int oi) {
  const bool on = ov != ov, bn = best != best;
  const bool take = on ? (!bn || oi < idx) : (!bn && (ov > best || (ov == best && oi < idx)));
  if (take) {
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
      if (p + 1 >= prompt) tokens[p + 1] = idx < n ? idx : 0;  // n >= 1: some slice holds an element
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
  // 256 threads (the launch's); each thread walks i = t, t + 256, ... with
  // eight loads in flight per step (the order of its partial sum is the
  // same as one element at a time)
  constexpr int NT = 256, U = 8;
  __shared__ float red[NT / 64];
  const float* xr = x + blockIdx.x * ldx;
  float ss = 0.0f;
  for (int i0 = threadIdx.x; i0 < k; i0 += U * NT) {
    float v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) v[u] = i0 + u * NT < k ? xr[i0 + u * NT] : 0.0f;
#pragma unroll
    for (int u = 0; u < U; ++u) ss += v[u] * v[u];
  }
  ss = qmm::wave_sum(ss);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
  __syncthreads();
  float t = 0.0f;
#pragma unroll
  for (int i = 0; i < NT / 64; ++i) t += red[i];
  const float den = sqrtf(t / (float)k + eps);
  float* orow = out + blockIdx.x * ldo;
  for (int i0 = threadIdx.x; i0 < k; i0 += U * NT) {
    float v[U], g[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int i = i0 + u * NT;
      v[u] = i < k ? xr[i] : 0.0f;
      g[u] = i < k ? w[i] : 0.0f;
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (i0 + u * NT < k) orow[i0 + u * NT] = v[u] / den * g[u];
  }
}
