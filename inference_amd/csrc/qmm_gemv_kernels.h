// Decode GEMV (M = 1..8 activation rows) over Q8_0 / Q4_K / Q6_K weights.
//
// Work split (wave64, CDNA4):
//   * a k-quant super-block is decoded by 4 lanes, each owning 32 bytes of
//     its quants (two dwordx4 loads) plus the block header, so one wave-wide
//     iteration covers 16 consecutive super-blocks of a row: 2304 B (Q4_K) or
//     3360 B (Q6_K) of contiguous HBM. A Q8_0 block (32 quants) is one lane's,
//     64 blocks per iteration.
//   * the activation rows (already quantized to Q8_K / Q8_0) are staged once
//     per workgroup in LDS, in the order each lane consumes them, with the
//     16-byte chunks XOR-swizzled so that a wave's ds_read_b128 hits distinct
//     banks; each lane also gets its 32-element (Q4_K) or 16-element (Q6_K)
//     activation sums precombined.
//   * the first batch of weight loads is issued before the activation is
//     staged, so the HBM latency overlaps the LDS fill and the barrier.
//   * each wave owns R weight rows and issues U iterations of loads for all of
//     them before using any, so every lane has R*U*32 bytes in flight;
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
#include "qmm_quant_kernels.h"

namespace qmm {

template <int FMT>
struct FmtInfo;
template <>
struct FmtInfo<kFmtQ80> {
  static constexpr int kLanesPerBlock = 1;
  static constexpr int kBlockElems = 32;
  static constexpr int kBodyBytes = kQ80Body;
  static constexpr int kLdsBlock = 32 + 4;  // q8[32] | d (f32)
};
template <>
struct FmtInfo<kFmtQ4K> {
  static constexpr int kLanesPerBlock = 4;
  static constexpr int kBlockElems = 256;
  static constexpr int kBodyBytes = kQ4KBytes;
  static constexpr int kLdsBlock = 256 + 32 + 4;  // q8[256] | sums u32[8] | d (f32)
};
template <>
struct FmtInfo<kFmtQ6K> {
  static constexpr int kLanesPerBlock = 4;
  static constexpr int kBlockElems = 256;
  static constexpr int kBodyBytes = kQ6KBody;
  static constexpr int kLdsBlock = 256 + 32 + 4;
};

// First activation element of chunk k (16 elements, k = 0..3) of lane l of a
// k-quant super-block.
//   Q4_K lane l holds qs[32l, 32l+32): low nibbles are elements 64l + [0,32)
//        (chunks 0,1), high nibbles 64l + 32 + [0,32) (chunks 2,3).
//   Q6_K lane l holds ql[64h + 32p, +32) (h = l/2, p = l%2): low nibbles are
//        elements 128h + 32p + [0,32) (chunks 0,1), high nibbles 64 further (2,3).
// Waves per workgroup: the kernel's compile-time size when it has one (NW >
// 0), else blockDim (which costs a vector-memory load of the dispatch's
// implicit arguments before anything else can be issued).
template <int NW>
__device__ __forceinline__ int block_waves() {
  if constexpr (NW > 0)
    return NW;
  else
    return blockDim.x >> 6;
}

template <int FMT>
__device__ __forceinline__ int act_chunk(int l, int k) {
  return FMT == kFmtQ4K ? 64 * l + 16 * k : 128 * (l >> 1) + 32 * (l & 1) + 64 * (k >> 1) + 16 * (k & 1);
}

// LDS position (16-byte slot) of chunk k of lane l in block b. Blocks are
// 256 B apart, so without a swizzle the same (l, k) of every block falls on
// the same banks; XOR-ing k with the block's low two bits spreads four
// consecutive blocks (the 16 lanes of a ds_read_b128 pass over 64 banks), and
// the lane-pair bit keeps lanes l and l + 2 apart within 128 B.
__device__ __forceinline__ int kq_slot(int b, int l, int k) {
  return 4 * l + (k ^ ((b & 3) ^ ((l >> 1) << 1)));
}
__device__ __forceinline__ int q80_slot(int b, int k) { return k ^ ((b >> 2) & 1); }

// Stage nblk activation blocks (M rows of nb blocks, contiguous) into LDS.
//   k-quants: q8 [blk][256] (swizzled chunks), sums u32 [blk][8], d f32 [blk]
//     Q4_K sums: lane l -> (bsum_4l + bsum_4l+1) | (bsum_4l+2 + bsum_4l+3) << 16
//     Q6_K sums: lane l -> two u32: bsums of its chunks (0,1) and (2,3)
//   Q8_0: q8 [blk][32] (swizzled halves), d f32 [blk]
// MR > 0 (k-quants, nblk = MR * nb): block b of row m goes to LDS block
// b * MR + m with its chunks swizzled by b, so a lane's reads of one block
// for successive rows are fixed offsets apart (256 B of quants, 32 B of sums,
// 4 B of scale).
template <int FMT, int NW = 0, int MR = 0>
__device__ __forceinline__ void stage_act(const uint8_t* __restrict__ xq, int nblk, uint8_t* lds, int nb = 0) {
  static_assert(MR == 0 || FMT != kFmtQ80, "row-interleaved staging is for k-quant activations");
  const int nthr = 64 * block_waves<NW>();
  if constexpr (FMT == kFmtQ80) {
    float* ld = reinterpret_cast<float*>(lds + 32 * nblk);
    for (int t = threadIdx.x; t < 2 * nblk; t += nthr) {
      const int blk = t >> 1, half = t & 1;
      const uint16_t* s = reinterpret_cast<const uint16_t*>(xq + (size_t)kQ80Bytes * blk);
      const uint16_t* q = s + 1 + 8 * half;
      uint4 v;
      v.x = q[0] | ((uint32_t)q[1] << 16);
      v.y = q[2] | ((uint32_t)q[3] << 16);
      v.z = q[4] | ((uint32_t)q[5] << 16);
      v.w = q[6] | ((uint32_t)q[7] << 16);
      *reinterpret_cast<uint4*>(lds + 32 * blk + 16 * q80_slot(blk, half)) = v;
      if (half == 0) ld[blk] = h2f(s[0]);
    }
  } else {
    uint32_t* lsum = reinterpret_cast<uint32_t*>(lds + 256 * nblk);
    float* ld = reinterpret_cast<float*>(lsum + 8 * nblk);
    for (int t = threadIdx.x; t < 16 * nblk; t += nthr) {
      const int src = t >> 4, l = (t >> 2) & 3, k = t & 3;
      int blk = src, swb = src;  // LDS block, swizzle block
      if constexpr (MR > 0) {
        const int m = src / nb, b = src - m * nb;
        blk = b * MR + m;
        swb = b;
      }
      const uint8_t* s = xq + (size_t)kQ8KBytes * src;
      const uint32_t* q = reinterpret_cast<const uint32_t*>(s + 4 + act_chunk<FMT>(l, k));
      uint4 v;
      v.x = q[0];
      v.y = q[1];
      v.z = q[2];
      v.w = q[3];
      *reinterpret_cast<uint4*>(lds + 256 * blk + 16 * kq_slot(swb, l, k)) = v;
      const int16_t* bs = reinterpret_cast<const int16_t*>(s + 4 + 256);
      if (k < 2) {
        const int e0 = act_chunk<FMT>(l, 2 * k) / 16;  // chunks 2k and 2k+1
        const int e1 = act_chunk<FMT>(l, 2 * k + 1) / 16;
        if (FMT == kFmtQ4K) {
          if (k == 0) {
            const int a = bs[e0] + bs[e1];
            const int b2 = bs[act_chunk<FMT>(l, 2) / 16] + bs[act_chunk<FMT>(l, 3) / 16];
            lsum[8 * blk + l] = ((uint32_t)a & 0xffffu) | ((uint32_t)b2 << 16);
          }
        } else {
          lsum[8 * blk + 2 * l + k] = ((uint32_t)(uint16_t)bs[e0]) | ((uint32_t)(uint16_t)bs[e1] << 16);
        }
      }
      if (l == 0 && k == 0) ld[blk] = *reinterpret_cast<const float*>(s);
    }
  }
}

// One lane's share of one weight block.
struct WSlice {
  uint4 a;     // Q4_K: header (d, dmin, scales[12]); Q6_K: ql[0:16); Q8_0: qs[0:16)
  uint4 b;     // Q4_K: qs[0:16);  Q6_K: ql[16:32); Q8_0: qs[16:32)
  uint4 c;     // Q4_K: qs[16:32); Q6_K: qh[0:16)
  uint4 e;     // Q6_K: qh[16:32)
  uint4 f;     // Q6_K: scales[16]
  uint32_t d;  // Q6_K / Q8_0: f16 scale
};

// Block b of a row: `wrow` = the row's first block body, `drow` = its first
// separated f16 scale (both wave-uniform), so a lane's address is a scalar base
// plus a 32-bit offset.
template <int FMT>
__device__ __forceinline__ void load_slice(WSlice& s, const uint8_t* __restrict__ wrow,
                                           const uint16_t* __restrict__ drow, uint32_t b, int l) {
  // 32-bit offsets from the uniform row base (global_load with a scalar base).
  // Plain loads: a lane's two quant loads take alternating 16-byte pieces of
  // the same cache lines, so a streaming (nontemporal) hint that drops the
  // lines after the first use measured 25% slower.
  auto ld16 = [wrow](uint32_t o) { return *reinterpret_cast<const uint4*>(wrow + o); };
  // block offsets with the full-rate 24-bit multiply (b < 2^16); a 32-bit
  // product issues the quarter-rate v_mul_lo_u32
  if constexpr (FMT == kFmtQ4K) {
    const uint32_t o = __umul24(b, (uint32_t)kQ4KBytes), ol = o + 32u * (uint32_t)l;
    s.a = ld16(o);
    s.b = ld16(ol + 16u);
    s.c = ld16(ol + 32u);
  } else if constexpr (FMT == kFmtQ6K) {
    const uint32_t o = __umul24(b, (uint32_t)kQ6KBody), ol = o + 32u * (uint32_t)l, oh = o + 128u + 32u * (uint32_t)(l >> 1);
    s.a = ld16(ol);
    s.b = ld16(ol + 16u);
    s.c = ld16(oh);
    s.e = ld16(oh + 16u);
    s.f = ld16(o + 192u);
    s.d = *reinterpret_cast<const uint16_t*>(reinterpret_cast<const uint8_t*>(drow) + 2u * b);
  } else {
    const uint32_t o = b * (uint32_t)kQ80Body;
    s.a = ld16(o);
    s.b = ld16(o + 16u);
    s.d = *reinterpret_cast<const uint16_t*>(reinterpret_cast<const uint8_t*>(drow) + 2u * b);
  }
}

__device__ __forceinline__ int dot16(uint4 w, uint4 x, int acc) {
  acc = dot4(w.x, x.x, acc);
  acc = dot4(w.y, x.y, acc);
  acc = dot4(w.z, x.z, acc);
  return dot4(w.w, x.w, acc);
}

__device__ __forceinline__ uint4 lo_nib(uint4 v) {
  return make_uint4(v.x & 0x0f0f0f0fu, v.y & 0x0f0f0f0fu, v.z & 0x0f0f0f0fu, v.w & 0x0f0f0f0fu);
}
__device__ __forceinline__ uint4 hi_nib(uint4 v) {
  return make_uint4((v.x >> 4) & 0x0f0f0f0fu, (v.y >> 4) & 0x0f0f0f0fu, (v.z >> 4) & 0x0f0f0f0fu,
                    (v.w >> 4) & 0x0f0f0f0fu);
}
// High nibbles left in place with the sign bit flipped: byte = 16*q ^ 0x80,
// read as a signed byte 16*q - 128.
__device__ __forceinline__ uint4 hi_nib_x80(uint4 v) {
  return make_uint4((v.x & 0xf0f0f0f0u) ^ 0x80808080u, (v.y & 0xf0f0f0f0u) ^ 0x80808080u,
                    (v.z & 0xf0f0f0f0u) ^ 0x80808080u, (v.w & 0xf0f0f0f0u) ^ 0x80808080u);
}
// 6-bit Q6_K quants (0..63) of 16 elements: 4 low bits from `ql` (already
// shifted to the low nibble), 2 high bits at bit `sh` of `qh`.
__device__ __forceinline__ uint4 q6_bytes(uint4 ql, uint4 qh, int sh) {
  auto one = [sh](uint32_t l, uint32_t h) { return (l & 0x0f0f0f0fu) | (((h >> sh) & 0x03030303u) << 4); };
  return make_uint4(one(ql.x, qh.x), one(ql.y, qh.y), one(ql.z, qh.z), one(ql.w, qh.w));
}

// Weight-side values of one lane's slice of one block (unpacked quants, scales),
// shared by every activation row the slice meets.
struct WPrep {
  uint4 w0, w1, w2, w3;
  int c0, c1, c2, c3;  // Q4_K: sc0, sc1, m0, m1; Q6_K: the four group scales
  uint32_t scp, mn16;  // Q4_K: sc0 | sc1 << 8 (bytes); m0 | m1 << 16 (16-bit lanes)
  float dw, dm;
};

// v_dot2_i32_i16: c + the two products of the packed signed 16-bit pairs.
__device__ __forceinline__ int sdot2_pairs(uint32_t a, uint32_t b, int c) {
  typedef short s16x2 __attribute__((ext_vector_type(2)));
  return __builtin_amdgcn_sdot2(__builtin_bit_cast(s16x2, a), __builtin_bit_cast(s16x2, b), c, false);
}

template <int FMT>
__device__ __forceinline__ WPrep prep_w(const WSlice& s, int l) {
  WPrep w;
  if constexpr (FMT == kFmtQ4K) {
    w.dw = h2f(s.a.x);
    w.dm = h2f(s.a.x >> 16);
    // 6-bit scale/min of sub-blocks 2l and 2l+1 (get_scale_min_k4).
    const int sh = (l & 1) * 16;
    const uint32_t A = s.a.y >> sh, B = s.a.z >> sh, C = s.a.w >> sh;
    // lanes 2, 3 take the upper form: a bit-select on a lane mask (both forms
    // are a few instructions; a branch on the lane would run both and add
    // exec-mask bookkeeping)
    const uint32_t um = 0u - (uint32_t)(l >> 1);
    const uint32_t scu = (C & 0x0f0fu) | ((A >> 2) & 0x3030u), scl = A & 0x3f3fu;
    const uint32_t mnu = ((C >> 4) & 0x0f0fu) | ((B >> 2) & 0x3030u), mnl = B & 0x3f3fu;
    const uint32_t scp = (scu & um) | (scl & ~um);
    const uint32_t mnp = (mnu & um) | (mnl & ~um);
    w.c0 = scp & 0xff;
    w.c1 = (scp >> 8) & 0xff;
    w.c2 = mnp & 0xff;
    w.c3 = (mnp >> 8) & 0xff;
    w.scp = scp;
    w.mn16 = __builtin_amdgcn_perm(0u, mnp, 0x0c010c00u);  // m0 | m1 << 16
    // Low nibbles as bytes 0..15; high nibbles kept in place with the top bit
    // flipped, i.e. signed bytes 16*q - 128 (one mask-and-xor per dword instead
    // of shift-and-mask); their dot is corrected with the sub-block's
    // activation sum: sum(q*x) = (dot + 128*sum(x)) / 16, exactly.
    w.w0 = lo_nib(s.b);
    w.w1 = lo_nib(s.c);
    w.w2 = hi_nib_x80(s.b);
    w.w3 = hi_nib_x80(s.c);
  } else if constexpr (FMT == kFmtQ6K) {
    w.dw = h2f(s.d);
    w.dm = 0.0f;
    const int h = l >> 1, p = l & 1;
    // scales of the lane's four 16-element groups: 8h + 2p + {0, 1} and +4.
    const uint32_t wlo = h ? s.f.z : s.f.x, whi = h ? s.f.w : s.f.y;
    const uint32_t sl = wlo >> (16 * p), shh = whi >> (16 * p);
    w.c0 = (int)(int8_t)(sl & 0xff);
    w.c1 = (int)(int8_t)((sl >> 8) & 0xff);
    w.c2 = (int)(int8_t)(shh & 0xff);
    w.c3 = (int)(int8_t)((shh >> 8) & 0xff);
    const int sh0 = 2 * p, sh1 = 2 * p + 4;
    w.w0 = q6_bytes(s.a, s.c, sh0);          // elements 128h + 32p + [0,16)
    w.w1 = q6_bytes(s.b, s.e, sh0);          // +16
    w.w2 = q6_bytes(hi_nib(s.a), s.c, sh1);  // +64
    w.w3 = q6_bytes(hi_nib(s.b), s.e, sh1);  // +80
  } else {
    w.dw = h2f(s.d);
    w.dm = 0.0f;
    w.w0 = s.a;
    w.w1 = s.b;
    w.c0 = w.c1 = w.c2 = w.c3 = 0;
  }
  return w;
}

// Activation-side values of one lane for one staged block: its 16-element
// chunks, their precombined sums and the block scale.
struct XSlice {
  uint4 x0, x1, x2, x3;
  uint32_t s0, s1;  // Q4_K: sums of sub-blocks 2l | 2l+1; Q6_K: (chunks 0,1) and (2,3)
  float d;
};

// LDS layouts written by stage_act / quantize_act (nblk staged blocks).
template <int FMT>
__device__ __forceinline__ void load_x(XSlice& x, const uint8_t* __restrict__ lds, int nblk, int bx, int l) {
  if constexpr (FMT == kFmtQ80) {
    const float* ld = reinterpret_cast<const float*>(lds + 32 * nblk);
    const int sw = (bx >> 2) & 1;
    x.x0 = *reinterpret_cast<const uint4*>(lds + 32 * bx + 16 * (0 ^ sw));
    x.x1 = *reinterpret_cast<const uint4*>(lds + 32 * bx + 16 * (1 ^ sw));
    x.d = ld[bx];
  } else {
    const uint32_t* lsum = reinterpret_cast<const uint32_t*>(lds + 256 * nblk);
    const float* ld = reinterpret_cast<const float*>(lsum + 8 * nblk);
    const uint8_t* e = lds + 256 * bx;
    const int sw = (bx & 3) ^ ((l >> 1) << 1);  // kq_slot's swizzle
    x.x0 = *reinterpret_cast<const uint4*>(e + 16 * (4 * l + (0 ^ sw)));
    x.x1 = *reinterpret_cast<const uint4*>(e + 16 * (4 * l + (1 ^ sw)));
    x.x2 = *reinterpret_cast<const uint4*>(e + 16 * (4 * l + (2 ^ sw)));
    x.x3 = *reinterpret_cast<const uint4*>(e + 16 * (4 * l + (3 ^ sw)));
    if constexpr (FMT == kFmtQ4K) {
      x.s0 = lsum[8 * bx + l];
    } else {
      x.s0 = lsum[8 * bx + 2 * l];
      x.s1 = lsum[8 * bx + 2 * l + 1];
    }
    x.d = ld[bx];
  }
}

// A Q4_K block's d * isd - dmin * ism with one fixed rounding sequence (the
// d product fused), so every kernel that forms it (one-row, multi-row,
// expert GEMVs) gets the same bits.
__device__ __forceinline__ float q4k_combine(float dw, float dm, int isd, int ism) {
  return __builtin_fmaf(dw, (float)isd, -(dm * (float)ism));
}

// One lane's f32 contribution for one block; its integer partials go to ia / ib.
template <int FMT>
__device__ __forceinline__ float dot_wx(const WPrep& w, const XSlice& x, int& ia, int& ib) {
  if constexpr (FMT == kFmtQ4K) {
    const int bs1 = (int)x.s0 >> 16;
    const int s0 = dot16(w.w1, x.x1, dot16(w.w0, x.x0, 0));
    const int s1 = (dot16(w.w3, x.x3, dot16(w.w2, x.x2, 0)) + 128 * bs1) >> 4;
    // isd = sc0 s0 + sc1 s1 in f32, exactly: |s| <= 32*15*128 and sc < 64, so
    // each product and the sum are integers below 2^24 (as a 32-bit integer
    // product the compiler cannot prove s1 fits the 24-bit multiplier and
    // issues a quarter-rate v_mul_lo_u32)
    const float isd = __builtin_fmaf((float)(w.scp & 0xffu), (float)s0, (float)((w.scp >> 8) & 0xffu) * (float)s1);
    // ism = m0 bs0 + m1 bs1 as one dot of the packed 16-bit pairs
    const int ism = sdot2_pairs(w.mn16, x.s0, 0);
    ia = (int)isd;
    ib = ism;
    return x.d * __builtin_fmaf(w.dw, isd, -(w.dm * (float)ism));
  } else if constexpr (FMT == kFmtQ6K) {
    const int t0 = dot16(w.w0, x.x0, 0) - 32 * (int)(int16_t)(x.s0 & 0xffffu);
    const int t1 = dot16(w.w1, x.x1, 0) - 32 * ((int)x.s0 >> 16);
    const int t2 = dot16(w.w2, x.x2, 0) - 32 * (int)(int16_t)(x.s1 & 0xffffu);
    const int t3 = dot16(w.w3, x.x3, 0) - 32 * ((int)x.s1 >> 16);
    // |t| < 2^18 and int8 scales: exact 24-bit products
    const int is = __mul24(w.c0, t0) + __mul24(w.c1, t1) + __mul24(w.c2, t2) + __mul24(w.c3, t3);
    ia = is;
    ib = 0;
    return x.d * (w.dw * (float)is);
  } else {
    const int s0 = dot16(w.w1, x.x1, dot16(w.w0, x.x0, 0));
    ia = s0;
    ib = 0;
    return (w.dw * x.d) * (float)s0;
  }
}

// Multiply one lane's slice with the staged activation block `xb` of each of
// the M rows (row stride `nbx` blocks in LDS). Adds to acc (when ok; the
// product is computed on every lane, so there is no branch around the dot)
// and returns the lane's integer partials in ia / ib.
template <int FMT, int M>
__device__ __forceinline__ void dot_slice(const WSlice& s, int l, const uint8_t* __restrict__ lds,
                                          int nblk, int xb, int nbx, bool ok, float (&acc)[M],
                                          int (&ia)[M], int (&ib)[M], int mrows) {
  const WPrep w = prep_w<FMT>(s, l);
#pragma unroll
  for (int m = 0; m < M; ++m) {
    if (M > 1 && m >= mrows) break;  // wave-uniform
    XSlice x;
    load_x<FMT>(x, lds, nblk, xb + m * nbx, l);
    const float prod = dot_wx<FMT>(w, x, ia[m], ib[m]);
    acc[m] += ok ? prod : 0.0f;
  }
}

// Up to kMaxJobs weight matrices (same format and K) that share one activation;
// rows of job j are global rows [sum_{i<j} rows[i], sum_{i<=j} rows[i]).
constexpr int kMaxJobs = 8;

struct GemvJobs {
  const uint8_t* wq[kMaxJobs];  // device-layout blocks of each matrix
  float* y[kMaxJobs];           // outputs, y[j][m * ldy[j] + row]
  int rows[kMaxJobs];           // rows computed for job j
  int ldy[kMaxJobs];
  int row0[kMaxJobs];           // first row of job j within its tensor (stacked experts)
  int trows[kMaxJobs];          // rows of the whole tensor (its f16 scales follow all of them)
  int njobs;
  int total;
};

// Where one global row lives.
struct RowRef {
  const uint8_t* wq;
  const uint16_t* wd;
  const uint8_t* wrow;   // first block body of the row (wave-uniform)
  const uint16_t* drow;  // first separated f16 scale of the row (Q6_K / Q8_0)
  float* y;
  int ldy;
  int out;   // output row within its job
  int row;   // row within its tensor
  int rows;
  bool ok;
};

// Global row gr -> (job, row). Jobs are laid out back to back in job order.
// `gr` is wave-uniform and every job index below is a constant, so the lookup
// compiles to a chain of scalar selects (no indexed access into the table).
// J is the kernel's job capacity (its launch arguments carry J jobs).
template <int FMT, int J>
__device__ __forceinline__ RowRef locate(const GemvJobs& jobs, int gr, int nb) {
  RowRef r;
  int base = 0;
  const uint8_t* wq = jobs.wq[0];
  float* y = jobs.y[0];
  int rows = jobs.rows[0], ldy = jobs.ldy[0], row0 = jobs.row0[0], trows = jobs.trows[0];
#pragma unroll
  for (int j = 1; j < J; ++j) {
    if (j < jobs.njobs && gr >= base + rows) {
      base += rows;
      wq = jobs.wq[j];
      y = jobs.y[j];
      rows = jobs.rows[j];
      ldy = jobs.ldy[j];
      row0 = jobs.row0[j];
      trows = jobs.trows[j];
    }
  }
  r.wq = wq;
  r.wd = FMT == kFmtQ4K ? nullptr
                        : reinterpret_cast<const uint16_t*>(wq + (size_t)trows * nb * FmtInfo<FMT>::kBodyBytes);
  r.y = y;
  r.ldy = ldy;
  r.out = gr - base;   // output row
  r.row = r.out + row0;  // row within the tensor
  r.rows = rows;
  r.ok = gr < jobs.total;
  r.wrow = wq + (size_t)r.row * nb * FmtInfo<FMT>::kBodyBytes;
  r.drow = r.wd + (size_t)r.row * nb;
  return r;
}

// Job cursor: a wave visits its rows in increasing order, so instead of a
// lookup over the whole table per row it keeps the current job in scalar
// registers and steps forward when a row passes the job's end. The job fields
// are read from the kernel-argument segment, where each job's arguments
// (QMM_JOB_PARAMS) form one 32-byte record.
struct JobArg {
  const uint8_t* wq;
  float* y;
  int rows, ldy, row0, trows;
};
static_assert(sizeof(JobArg) == 32, "job argument record");

struct JobCursor {
  int j, base, end;  // current job, its first global row, one past its last
  const uint8_t* wq;
  float* y;
  int ldy, row0, trows;
};

__device__ __forceinline__ const JobArg* job_args() {
  return reinterpret_cast<const JobArg*>(__builtin_amdgcn_kernarg_segment_ptr());
}

__device__ __forceinline__ void cursor_load(JobCursor& c, const JobArg* ja) {
  const JobArg& a = ja[c.j];
  c.wq = a.wq;
  c.y = a.y;
  c.end = c.base + a.rows;
  c.ldy = a.ldy;
  c.row0 = a.row0;
  c.trows = a.trows;
}

__device__ __forceinline__ void cursor_init(JobCursor& c, const JobArg* ja) {
  c.j = 0;
  c.base = 0;
  cursor_load(c, ja);
}

// RowRef of global row gr (wave-uniform, not below the previous call's row).
template <int FMT>
__device__ __forceinline__ RowRef cursor_row(JobCursor& c, const JobArg* ja, int njobs, int total, int gr, int nb) {
  while (gr >= c.end && c.j + 1 < njobs) {
    c.base = c.end;
    ++c.j;
    cursor_load(c, ja);
  }
  RowRef r;
  r.wq = c.wq;
  r.wd = FMT == kFmtQ4K ? nullptr
                        : reinterpret_cast<const uint16_t*>(c.wq + (size_t)c.trows * nb * FmtInfo<FMT>::kBodyBytes);
  r.y = c.y;
  r.ldy = c.ldy;
  r.out = gr - c.base;
  r.row = r.out + c.row0;
  r.rows = c.end - c.base;
  r.ok = gr < total;
  r.wrow = c.wq + (size_t)r.row * nb * FmtInfo<FMT>::kBodyBytes;
  r.drow = r.wd + (size_t)r.row * nb;
  return r;
}

// Row lookup of gemv(): the job cursor when the job table is the kernel's own
// arguments (KARG), else the select chain over a table built in the kernel.
template <int FMT, int J, bool KARG>
__device__ __forceinline__ RowRef row_ref(JobCursor& c, const JobArg* ja, const GemvJobs& jobs, int gr, int nb) {
  if constexpr (KARG)
    return cursor_row<FMT>(c, ja, jobs.njobs, jobs.total, gr, nb);
  else
    return locate<FMT, J>(jobs, gr, nb);
}

// One batch of weight slices: U iterations of R rows. Every lane issues its
// loads (no zero-fill and branch around them): lanes past the row's last block
// read the last block again and rows past the end read the group's first row;
// the dot products mask those with RowRef::ok and b < nb. rr[0] must be valid.
template <int FMT, int R, int U>
__device__ __forceinline__ void load_batch_nc(WSlice (&ws)[R][U], const RowRef (&rr)[R], int it0, int nb, int g,
                                              int l) {
  constexpr int BPI = 64 / FmtInfo<FMT>::kLanesPerBlock;
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int b = min((it0 + u) * BPI + g, nb - 1);
      const RowRef& q = rr[r].ok ? rr[r] : rr[0];
      load_slice<FMT>(ws[r][u], q.wrow, q.drow, (uint32_t)b, l);
    }
}

// ---------------------------------------------------------------------------
// In-kernel activation quantization (the prologue of the fused GEMV): the
// same arithmetic as the standalone quantizers, written straight into the LDS
// layout stage_act produces from GGML bytes.
// ---------------------------------------------------------------------------

// (lane l, chunk k) of the weight-side lane group that consumes 16-element
// activation group c16 (inverse of act_chunk).
template <int FMT>
__device__ __forceinline__ void chunk_owner(int c16, int& l, int& k) {
  if (FMT == kFmtQ4K) {
    l = c16 >> 2;
    k = c16 & 3;
  } else {
    const int rem = c16 & 7;
    l = 2 * (c16 >> 3) + ((rem >> 1) & 1);
    k = 2 * ((rem >> 2) & 1) + (rem & 1);
  }
}

// RMSNorm denominators sqrt(mean(x^2) + eps) of mrows (<= 8) rows of k
// elements, written to den[m] (LDS); the whole workgroup reduces.
template <int NW = 0>
__device__ __forceinline__ void rms_denominators(const float* __restrict__ x, long long ldx, int mrows, int k,
                                                 float eps, float* den, float* red) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = block_waves<NW>();
  for (int m = 0; m < mrows; ++m) {
    float ss = 0.0f;
    for (int i = threadIdx.x; i < k; i += 64 * nw) {
      const float v = x[m * ldx + i];
      ss += v * v;
    }
    ss = wave_sum(ss);
    if (lane == 0) red[m * 16 + wave] = ss;
  }
  __syncthreads();
  if (threadIdx.x < mrows) {
    float t = 0.0f;
    for (int w = 0; w < nw; ++w) t += red[threadIdx.x * 16 + w];
    den[threadIdx.x] = sqrtf(t / (float)k + eps);
  }
  __syncthreads();
}

// Quantize mrows f32 rows (stride ldx) of nb blocks into the LDS layout. With
// norm_w, each row is first RMS-normalised: x / sqrt(mean(x^2) + eps) * w
// (rms_norm, crates/llm/candle-llm/src/primitives/nn.rs:22-31).
// With SILU, `x` is the gate row g and `norm_w` the up row u, and the
// quantized activation is silu(g) * u (silu_mul, the same arithmetic as the
// standalone qmm_silu_mul_q8k); no RMSNorm then.
template <int FMT, bool SILU = false, int NW = 0>
__device__ __forceinline__ void quantize_act(const float* __restrict__ x, long long ldx, int mrows, int nb,
                                             uint8_t* lds, const float* __restrict__ norm_w, float eps) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = block_waves<NW>();
  const int nblk = mrows * nb;
  __shared__ float den[8];
  __shared__ float red[8 * 16];
  if (!SILU && norm_w != nullptr)
    rms_denominators<NW>(x, ldx, mrows, nb * FmtInfo<FMT>::kBlockElems, eps, den, red);
  if constexpr (FMT == kFmtQ80) {
    float* ld = reinterpret_cast<float*>(lds + 32 * nblk);
    const int l8 = lane & 7;
    for (int base = 8 * wave; base < nblk; base += 8 * nw) {
      const int blk = base + (lane >> 3);
      const bool valid = blk < nblk;
      const int bc = valid ? blk : 0;
      const int row = bc / nb, col = 32 * (bc % nb) + 4 * l8;
      const float* xs = x + row * ldx + col;
      float e[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (SILU) {
          e[j] = valid ? silu_mul(xs[j], norm_w[row * ldx + col + j]) : 0.0f;
        } else {
          e[j] = valid ? xs[j] : 0.0f;
          if (norm_w != nullptr) e[j] = e[j] / den[row] * norm_w[col + j];
        }
      }
      float amax = fmaxf(fmaxf(fabsf(e[0]), fabsf(e[1])), fmaxf(fabsf(e[2]), fabsf(e[3])));
      amax = fmaxf(amax, dpp_f<0xb1>(amax));
      amax = fmaxf(amax, dpp_f<0x4e>(amax));
      amax = fmaxf(amax, dpp_f<0x141>(amax));
      const float d = amax / 127.0f;
      const float id = d != 0.0f ? 1.0f / d : 0.0f;
      uint32_t q4 = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float v = roundf(e[j] * id);
        v = fminf(fmaxf(v, -128.0f), 127.0f);
        q4 |= (uint32_t)((int)v & 0xff) << (8 * j);
      }
      if (valid) {
        *reinterpret_cast<uint32_t*>(lds + 32 * blk + 16 * q80_slot(blk, l8 >> 2) + 4 * (l8 & 3)) = q4;
        if (l8 == 0) ld[blk] = h2f(f2h(d));
      }
    }
  } else {
    uint32_t* lsum = reinterpret_cast<uint32_t*>(lds + 256 * nblk);
    float* ld = reinterpret_cast<float*>(lsum + 8 * nblk);
    const int c16 = lane >> 2;
    int lc, kc;
    chunk_owner<FMT>(c16, lc, kc);
    for (int blk = wave; blk < nblk; blk += nw) {
      const int row = blk / nb, col = 256 * (blk % nb) + 4 * lane;
      const float* xs = x + row * ldx + col;
      float e0 = xs[0], e1 = xs[1], e2 = xs[2], e3 = xs[3];
      if (SILU) {
        const float* us = norm_w + row * ldx + col;
        e0 = silu_mul(e0, us[0]);
        e1 = silu_mul(e1, us[1]);
        e2 = silu_mul(e2, us[2]);
        e3 = silu_mul(e3, us[3]);
      } else if (norm_w != nullptr) {
        const float dn = den[row];
        e0 = e0 / dn * norm_w[col];
        e1 = e1 / dn * norm_w[col + 1];
        e2 = e2 / dn * norm_w[col + 2];
        e3 = e3 / dn * norm_w[col + 3];
      }
      const Q8KLane q = q8k_lane_vals(e0, e1, e2, e3, lane);
      *reinterpret_cast<uint32_t*>(lds + 256 * blk + 16 * kq_slot(blk, lc, kc) + 4 * (lane & 3)) = q.packed;
      const int next = __shfl_down(q.sum16, 4);  // the following 16-group's sum
      if (FMT == kFmtQ4K) {
        const int s32 = q.sum16 + next;
        const int s32n = __shfl_down(s32, 8);
        if ((lane & 15) == 0) lsum[8 * blk + (lane >> 4)] = ((uint32_t)s32 & 0xffffu) | ((uint32_t)s32n << 16);
      } else {
        if ((lane & 7) == 0) lsum[8 * blk + 2 * lc + (kc >> 1)] = ((uint32_t)q.sum16 & 0xffffu) | ((uint32_t)next << 16);
      }
      if (lane == 0) ld[blk] = q.d;
    }
  }
}

// Writes the outputs kept by the lanes with `valid` (lane i holds one output of
// global row keep_row); `accumulate` adds them with a no-return atomic (one add
// per output, so the result is exactly y + v).
template <int FMT, int J>
__device__ __forceinline__ void flush_outputs(const GemvJobs& jobs, int nb, float keep_v, int keep_row, bool valid,
                                              int accumulate) {
  if (!valid) return;
  const RowRef q = locate<FMT, J>(jobs, keep_row, nb);
  float* yp = q.y + q.out;
  if (accumulate)
    __hip_atomic_fetch_add(yp, keep_v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  else
    *yp = keep_v;
}

// One-row prologue of the fused one-row GEMV (k-quant weights): every load
// of the activation row goes out before any block is quantized, so the
// prologue costs one memory round trip instead of one per block a wave owns.
// Wave w owns blocks w, w + nw, ... (up to kActPF of them; longer rows take
// quantize_act). RMSNorm (norm_w, not SILU) sums the squares from the same
// registers: lanes, then DPP rows and v_readlane, then waves in order.
// MIX (FMT = Q4_K) also writes the Q6_K layout of the same quantized row at
// lds + 292 * nb, for launches whose jobs mix the two formats.
constexpr int kActPF = 4;

template <int FMT>
__device__ __forceinline__ void put_q8k_lane(uint8_t* lds, int nb, int blk, const Q8KLane& q, int lane) {
  uint32_t* lsum = reinterpret_cast<uint32_t*>(lds + 256 * nb);
  float* ld = reinterpret_cast<float*>(lsum + 8 * nb);
  int lc, kc;
  chunk_owner<FMT>(lane >> 2, lc, kc);
  *reinterpret_cast<uint32_t*>(lds + 256 * blk + 16 * kq_slot(blk, lc, kc) + 4 * (lane & 3)) = q.packed;
  const int next = __shfl_down(q.sum16, 4);  // the following 16-group's sum
  if (FMT == kFmtQ4K) {
    const int s32 = q.sum16 + next;
    const int s32n = __shfl_down(s32, 8);
    if ((lane & 15) == 0) lsum[8 * blk + (lane >> 4)] = ((uint32_t)s32 & 0xffffu) | ((uint32_t)s32n << 16);
  } else {
    if ((lane & 7) == 0) lsum[8 * blk + 2 * lc + (kc >> 1)] = ((uint32_t)q.sum16 & 0xffffu) | ((uint32_t)next << 16);
  }
  if (lane == 0) ld[blk] = q.d;
}

// The prologue's registers: wave w's blocks w, w + nw, ... of the f32 row
// (e) and of the RMSNorm weight or the up row (a).
struct Act1Regs {
  float4 e[kActPF], a[kActPF];
};

// First half of the one-row prologue: the loads only, so that a caller can
// issue its weight loads behind them and still use the activation first.
// `nw` = waves per workgroup (a constant in kernels that know their size:
// blockDim costs a vector-memory load of the dispatch's implicit arguments).
template <bool SILU>
__device__ __forceinline__ void act1_load(Act1Regs& r, const float* __restrict__ x, int nb,
                                          const float* __restrict__ norm_w, int nw) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const bool aux = SILU || norm_w != nullptr;
#pragma unroll
  for (int i = 0; i < kActPF; ++i) {
    const int blk = wave + i * nw;
    r.e[i] = r.a[i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (blk < nb) {
      r.e[i] = *reinterpret_cast<const float4*>(x + 256 * blk + 4 * lane);
      if (aux) r.a[i] = *reinterpret_cast<const float4*>(norm_w + 256 * blk + 4 * lane);
    }
  }
}

// Second half: RMSNorm or silu(g) * u, Q8_K quantization, LDS layout(s).
template <int FMT, bool SILU, bool MIX = false>
__device__ __forceinline__ void act1_finish(Act1Regs& r, int nb, uint8_t* lds, const float* __restrict__ norm_w,
                                            float eps, int nw) {
#pragma clang fp contract(off)
  static_assert(FMT != kFmtQ80, "k-quant activations");
  static_assert(!MIX || FMT == kFmtQ4K, "mixed layouts: Q4_K then Q6_K");
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  __shared__ float red[16];
  float4* e = r.e;
  const float4* a = r.a;
  if (!SILU && norm_w != nullptr) {
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < kActPF; ++i) {
      ss += e[i].x * e[i].x;
      ss += e[i].y * e[i].y;
      ss += e[i].z * e[i].z;
      ss += e[i].w * e[i].w;
    }
    ss = wave_total(ss);
    if (lane == 0) red[wave] = ss;
    __syncthreads();
    // every wave adds the waves' partial sums itself, in wave order, so all
    // waves hold the same denominator without a second barrier (a single
    // thread summing them and broadcasting through LDS cost one more barrier
    // and a serial chain of LDS reads)
    float t = 0.0f;
    for (int w = 0; w < nw; ++w) t += red[w];
    const float dn = sqrtf(t / (float)(256 * nb) + eps);
    // only the wave's own blocks (IEEE divisions are long instruction
    // sequences; at K = 4096 a 16-wave workgroup holds one block per wave)
#pragma unroll
    for (int i = 0; i < kActPF; ++i) {
      if (wave + i * nw >= nb) break;  // wave-uniform
      e[i].x = e[i].x / dn * a[i].x;
      e[i].y = e[i].y / dn * a[i].y;
      e[i].z = e[i].z / dn * a[i].z;
      e[i].w = e[i].w / dn * a[i].w;
    }
  } else if (SILU) {
#pragma unroll
    for (int i = 0; i < kActPF; ++i) {
      if (wave + i * nw >= nb) break;  // wave-uniform
      e[i].x = silu_mul(e[i].x, a[i].x);
      e[i].y = silu_mul(e[i].y, a[i].y);
      e[i].z = silu_mul(e[i].z, a[i].z);
      e[i].w = silu_mul(e[i].w, a[i].w);
    }
  }
#pragma unroll
  for (int i = 0; i < kActPF; ++i) {
    const int blk = wave + i * nw;
    if (blk >= nb) break;  // wave-uniform
    const Q8KLane q = q8k_lane_vals(e[i].x, e[i].y, e[i].z, e[i].w, lane);
    put_q8k_lane<FMT>(lds, nb, blk, q, lane);
    if constexpr (MIX) put_q8k_lane<kFmtQ6K>(lds + kQ8KBytes * nb, nb, blk, q, lane);
  }
}

template <int FMT, bool SILU, bool MIX = false, int NW = 0>
__device__ __forceinline__ void quantize_act1(const float* __restrict__ x, int nb, uint8_t* lds,
                                              const float* __restrict__ norm_w, float eps) {
  const int nw = block_waves<NW>();
  if (nb > kActPF * nw) {
    quantize_act<FMT, SILU, NW>(x, 0, 1, nb, lds, norm_w, eps);
    if constexpr (MIX) {
      __syncthreads();  // quantize_act's LDS scratch is reused
      quantize_act<kFmtQ6K, SILU, NW>(x, 0, 1, nb, lds + kQ8KBytes * nb, norm_w, eps);
    }
    return;
  }
  Act1Regs r;
  act1_load<SILU>(r, x, nb, norm_w, nw);
  act1_finish<FMT, SILU, MIX>(r, nb, lds, norm_w, eps, nw);
}

// y_j[m, n] = sum_b dot(W_j[n, b], X[m, b]) for every job j, m < M, n < rows_j.
//   act: M rows of nb activation blocks (Q8_K or Q8_0, GGML bytes), or, when
//        FUSED, M rows of f32 (row stride ldx) quantized in the prologue;
//   dump (optional, single job): int32 block dots [M][rows][nb](x2 for Q4_K).
// With `accumulate`, outputs are added to y (y += result); norm_w (fused only)
// RMS-normalises the activation rows before quantization.
template <int FMT, int M, int R, int U, bool FUSED, int J = 4, bool KARG = true, int NW = 0>
__device__ __forceinline__ void gemv(const GemvJobs& jobs, const void* __restrict__ act, long long ldx, int K,
                                     int* __restrict__ dump, int mrows = M,
                                     const float* __restrict__ norm_w = nullptr, float eps = 0.0f,
                                     int accumulate = 0) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  constexpr int LPB = FmtInfo<FMT>::kLanesPerBlock;
  constexpr int BPI = 64 / LPB;  // blocks per wave iteration
  const int nb = K / FmtInfo<FMT>::kBlockElems;
  const int lane = threadIdx.x & 63;
  const int nw = block_waves<NW>();
  const int l = lane % LPB;
  const int g = lane / LPB;
  const int niter = (nb + BPI - 1) / BPI;
  const int row_step = gridDim.x * nw * R;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  int row0 = (blockIdx.x * nw + wave) * R;

  // First weight batch in flight before the activation is staged.
  const JobArg* ja = KARG ? job_args() : nullptr;
  JobCursor jc;
  if constexpr (KARG) cursor_init(jc, ja);
  RowRef rr[R];
  WSlice ws[R][U];
  {
    // a wave without rows still loads (row total-1) so that no load is conditional
    const int lr = min(row0, jobs.total - 1);
#pragma unroll
    for (int r = 0; r < R; ++r) rr[r] = row_ref<FMT, J, KARG>(jc, ja, jobs, lr + r, nb);
    load_batch_nc<FMT, R, U>(ws, rr, 0, nb, g, l);
  }
#pragma unroll
  for (int r = 0; r < R; ++r) rr[r] = row_ref<FMT, J, KARG>(jc, ja, jobs, row0 + r, nb);
  if constexpr (FUSED)
    quantize_act<FMT, false, NW>(reinterpret_cast<const float*>(act), ldx, mrows, nb, lds, norm_w, eps);
  else
    stage_act<FMT, NW>(reinterpret_cast<const uint8_t*>(act), mrows * nb, lds);
  __syncthreads();

  float keep_v = 0.0f;  // M = 1: this lane's kept output (global row keep_row)
  int keep_row = 0, slot = 0;
  for (; row0 < jobs.total; row0 += row_step) {
    float acc[R][M];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int m = 0; m < M; ++m) acc[r][m] = 0.0f;

    for (int it0 = 0; it0 < niter; it0 += U) {
      if (it0 > 0) load_batch_nc<FMT, R, U>(ws, rr, it0, nb, g, l);
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int b = (it0 + u) * BPI + g;
          const bool ok = rr[r].ok && b < nb;
          int ia[M], ib[M];
          dot_slice<FMT, M>(ws[r][u], l, lds, mrows * nb, ok ? b : 0, nb, ok, acc[r], ia, ib, mrows);
          if (dump != nullptr) {
#pragma unroll
            for (int m = 0; m < M; ++m) {
              int va = ia[m], vb = ib[m];
#pragma unroll
              for (int off = 1; off < LPB; off <<= 1) {
                va += __shfl_xor(va, off);
                vb += __shfl_xor(vb, off);
              }
              if (ok && l == 0 && m < mrows) {
                const size_t o = ((size_t)m * rr[r].rows + rr[r].out) * nb + b;
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
    // The next row group's first batch goes out before this group's reduction.
    RowRef cur[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      cur[r] = rr[r];
      rr[r] = row_ref<FMT, J, KARG>(jc, ja, jobs, row0 + row_step + r, nb);
    }
    if (row0 + row_step < jobs.total) load_batch_nc<FMT, R, U>(ws, rr, 0, nb, g, l);
    if constexpr (M == 1 && KARG) {
      // One output per row: lane `slot` keeps it and the wave writes 64 at a
      // time (a store per row would sit in the same in-order memory counter
      // that the next row's loads are waited on).
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const float v = wave_sum(acc[r][0]);
        if (cur[r].ok && lane == slot) {
          keep_v = v;
          keep_row = row0 + r;
        }
        slot += cur[r].ok ? 1 : 0;
      }
      if (slot > 64 - R) {
        flush_outputs<FMT, J>(jobs, nb, keep_v, keep_row, lane < slot, accumulate);
        slot = 0;
      }
    } else {
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < M; ++m) {
          if (M > 1 && m >= mrows) break;  // wave-uniform
          const float v = wave_sum(acc[r][m]);
          if (lane == 0 && cur[r].ok && m < mrows) {
            float* yp = cur[r].y + (size_t)m * cur[r].ldy + cur[r].out;
            *yp = accumulate ? *yp + v : v;
          }
        }
    }
  }
  if constexpr (M == 1 && KARG) {
    if (slot > 0) flush_outputs<FMT, J>(jobs, nb, keep_v, keep_row, lane < slot, accumulate);
  }
}

// Decode GEMV for one activation row (M = 1), one row per wave at a time:
// the leanest per-row instruction stream, because a wave's row time is its
// memory latency plus its own instruction issue. Against gemv():
//   * the activation slice of the first wave iteration (the whole row's when
//     K <= 64/LPB blocks, e.g. K = 4096 for k-quants) is read from LDS once
//     and kept in registers for every row;
//   * the row sum is reduced with DPP and v_readlane (no LDS round trip);
//   * outputs are kept one per lane and written 64 at a time.
// Rows row, row + row_step, ... below `end` of one format (gemv1's row loop):
// each row's dot, the next row's first slice loaded before this row's
// reduction, outputs kept one per lane (keep_v / keep_row, `slot` lanes
// filled) and flushed 64 at a time. ws holds row `row`'s first slice on entry.
// Q8_0 (one block per lane, so a K = 4096 row is two slices) keeps the next
// slice in flight while one is used: wn holds the row's second slice on
// entry (when it has one), and each iteration issues the one after.
template <int FMT>
constexpr bool kSlicePipe = FMT == kFmtQ80;
template <int FMT, int J>
__device__ __forceinline__ void gemv1_rows(const GemvJobs& jobs, JobCursor& jc, const JobArg* ja, RowRef& rr,
                                           WSlice& ws, WSlice& wn, const XSlice& x0,
                                           const uint8_t* __restrict__ lds, int nb, int& row, int end,
                                           int row_step, uint32_t b0, int g, int l, int lane, float& keep_v,
                                           int& keep_row, int& slot, int accumulate) {
  constexpr int BPI = 64 / FmtInfo<FMT>::kLanesPerBlock;
  const int niter = (nb + BPI - 1) / BPI;
  const bool ok0 = g < nb;
  for (;;) {
    int ia, ib;
    float acc;
    {
      const float p = dot_wx<FMT>(prep_w<FMT>(ws, l), x0, ia, ib);
      acc = ok0 ? p : 0.0f;
    }
    for (int it = 1; it < niter; ++it) {
      const int b = it * BPI + g;
      if constexpr (kSlicePipe<FMT>) {
        const WSlice cur = wn;
        if (it + 1 < niter) load_slice<FMT>(wn, rr.wrow, rr.drow, (uint32_t)min(b + BPI, nb - 1), l);
        XSlice x;
        load_x<FMT>(x, lds, nb, b < nb ? b : 0, l);
        const float p = dot_wx<FMT>(prep_w<FMT>(cur, l), x, ia, ib);
        acc += b < nb ? p : 0.0f;
      } else {
        load_slice<FMT>(ws, rr.wrow, rr.drow, (uint32_t)min(b, nb - 1), l);
        XSlice x;
        load_x<FMT>(x, lds, nb, b < nb ? b : 0, l);
        const float p = dot_wx<FMT>(prep_w<FMT>(ws, l), x, ia, ib);
        acc += b < nb ? p : 0.0f;
      }
    }
    const int nrow = row + row_step;
    if (nrow < end) {  // next row's first batch (and second slice) before this row's reduction
      rr = cursor_row<FMT>(jc, ja, jobs.njobs, jobs.total, nrow, nb);
      load_slice<FMT>(ws, rr.wrow, rr.drow, b0, l);
      if (kSlicePipe<FMT> && niter > 1) load_slice<FMT>(wn, rr.wrow, rr.drow, (uint32_t)min(BPI + g, nb - 1), l);
    }
    const float v = wave_total(acc);
    if (lane == slot) {
      keep_v = v;
      keep_row = row;
    }
    if (++slot == 64) {
      flush_outputs<FMT, J>(jobs, nb, keep_v, keep_row, true, accumulate);
      slot = 0;
    }
    row = nrow;
    if (row >= end) break;
  }
}

// Same per-block arithmetic (prep_w / dot_wx) as gemv(); no block-dot dump.
// MIX (FMT = Q4_K): global rows >= mix_row belong to Q6_K jobs (the host
// orders the jobs Q4_K first); the activation is staged in both layouts and
// a wave runs its Q4_K rows, then its Q6_K rows.
// A grouped launch (qmm_gemv1g_*) runs several of these in one grid: ja_in
// is then the group's job records, wg its workgroup's index within the group
// and ngrid the group's workgroup count (defaults: the whole launch).
template <int FMT, bool FUSED, int J, bool SILU = false, bool MIX = false, int NW = 0>
__device__ __forceinline__ void gemv1(const GemvJobs& jobs, const void* __restrict__ act, long long ldx, int K,
                                      const float* __restrict__ norm_w, float eps, int accumulate,
                                      int mix_row = 0x7fffffff, const JobArg* ja_in = nullptr, int wg = -1,
                                      int ngrid = 0) {
  static_assert(!MIX || FMT == kFmtQ4K, "mixed launches: Q4_K rows, then Q6_K rows");
  constexpr int F6 = kFmtQ6K;
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  constexpr int LPB = FmtInfo<FMT>::kLanesPerBlock;
  const int nb = K / FmtInfo<FMT>::kBlockElems;
  const int lane = threadIdx.x & 63;
  const int nw = block_waves<NW>();
  const int l = lane % LPB;
  const int g = lane / LPB;
  const int row_step = (ngrid > 0 ? ngrid : (int)gridDim.x) * nw;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  int row = (wg >= 0 ? wg : (int)blockIdx.x) * nw + wave;
  uint8_t* lds6 = lds + (MIX ? kQ8KBytes * nb : 0);  // Q6_K layout (MIX)
  const int end4 = MIX ? min(mix_row, jobs.total) : jobs.total;

  const JobArg* ja = ja_in != nullptr ? ja_in : job_args();
  JobCursor jc;
  cursor_init(jc, ja);
  WSlice ws, wn;
  const uint32_t b0 = (uint32_t)min(g, nb - 1);  // clamped: every lane loads
  RowRef rr;
  const bool first6 = MIX && min(row, jobs.total - 1) >= end4;  // the wave starts in the Q6_K rows
  {
    // first row in flight before staging
    const int r0 = min(row, jobs.total - 1);
    if (first6) {
      rr = cursor_row<F6>(jc, ja, jobs.njobs, jobs.total, r0, nb);
      load_slice<F6>(ws, rr.wrow, rr.drow, b0, l);
    } else {
      rr = cursor_row<FMT>(jc, ja, jobs.njobs, jobs.total, r0, nb);
      load_slice<FMT>(ws, rr.wrow, rr.drow, b0, l);
      if (kSlicePipe<FMT> && nb > 64 / LPB)
        load_slice<FMT>(wn, rr.wrow, rr.drow, (uint32_t)min(64 / LPB + g, nb - 1), l);
    }
  }
  if constexpr (FUSED) {
    if constexpr (FMT == kFmtQ80)
      quantize_act<FMT, SILU, NW>(reinterpret_cast<const float*>(act), ldx, 1, nb, lds, norm_w, eps);
    else
      quantize_act1<FMT, SILU, MIX, NW>(reinterpret_cast<const float*>(act), nb, lds, norm_w, eps);
  } else {
    stage_act<FMT, NW>(reinterpret_cast<const uint8_t*>(act), nb, lds);
    if constexpr (MIX) stage_act<F6, NW>(reinterpret_cast<const uint8_t*>(act), nb, lds6);
  }
  __syncthreads();
  if (row >= jobs.total) return;

  float keep_v = 0.0f;  // this lane's kept output (global row keep_row)
  int keep_row = 0, slot = 0;
  if (row < end4) {
    rr = cursor_row<FMT>(jc, ja, jobs.njobs, jobs.total, row, nb);
    XSlice x0;  // loop-invariant activation of the first iteration
    load_x<FMT>(x0, lds, nb, (int)b0, l);
    gemv1_rows<FMT, J>(jobs, jc, ja, rr, ws, wn, x0, lds, nb, row, end4, row_step, b0, g, l, lane, keep_v,
                       keep_row, slot, accumulate);
  }
  if constexpr (MIX) {
    if (row < jobs.total) {
      rr = cursor_row<F6>(jc, ja, jobs.njobs, jobs.total, row, nb);
      if (!first6) load_slice<F6>(ws, rr.wrow, rr.drow, b0, l);  // after Q4_K rows: not prefetched
      XSlice x06;
      load_x<F6>(x06, lds6, nb, (int)b0, l);
      gemv1_rows<F6, J>(jobs, jc, ja, rr, ws, wn, x06, lds6, nb, row, jobs.total, row_step, b0, g, l, lane,
                        keep_v, keep_row, slot, accumulate);
    }
  }
  if (slot > 0) flush_outputs<FMT, J>(jobs, nb, keep_v, keep_row, lane < slot, accumulate);
}

}  // namespace qmm

// Kernel arguments: the job table as plain scalars (a by-value struct would be
// copied to scratch), then the activation, its row stride, K and the dump.
#define QMM_JOB_PARAMS(i) \
  const uint8_t *wq##i, float *y##i, int rows##i, int ldy##i, int row0##i, int trows##i
#define QMM_GEMV_TAIL_PARAMS                                                                  \
  int njobs, int total, const void *__restrict__ act, long long ldx, int K, int *__restrict__ dump, \
      const float *__restrict__ norm_w, float eps, int accumulate
#define QMM_GEMV_PARAMS \
  QMM_JOB_PARAMS(0), QMM_JOB_PARAMS(1), QMM_JOB_PARAMS(2), QMM_JOB_PARAMS(3), QMM_GEMV_TAIL_PARAMS
#define QMM_GEMV_PARAMS8                                                                              \
  QMM_JOB_PARAMS(0), QMM_JOB_PARAMS(1), QMM_JOB_PARAMS(2), QMM_JOB_PARAMS(3), QMM_JOB_PARAMS(4),    \
      QMM_JOB_PARAMS(5), QMM_JOB_PARAMS(6), QMM_JOB_PARAMS(7), QMM_GEMV_TAIL_PARAMS
#define QMM_JOB_SET(i)   \
  jobs.wq[i] = wq##i;    \
  jobs.y[i] = y##i;      \
  jobs.rows[i] = rows##i; \
  jobs.ldy[i] = ldy##i;  \
  jobs.row0[i] = row0##i; \
  jobs.trows[i] = trows##i;
#define QMM_GEMV_JOBS \
  qmm::GemvJobs jobs; \
  QMM_JOB_SET(0)      \
  QMM_JOB_SET(1)      \
  QMM_JOB_SET(2)      \
  QMM_JOB_SET(3)      \
  jobs.njobs = njobs; \
  jobs.total = total;
#define QMM_GEMV_JOBS8 \
  QMM_GEMV_JOBS        \
  QMM_JOB_SET(4)       \
  QMM_JOB_SET(5)       \
  QMM_JOB_SET(6)       \
  QMM_JOB_SET(7)

#define QMM_GEMV_KERNEL(FMT, NAME, M, W, R, U)                                                            \
  extern "C" __global__ void __launch_bounds__(64 * W)                                                    \
      qmm_gemv_##NAME##_m##M##_w##W##_r##R##_u##U(QMM_GEMV_PARAMS) {                                      \
    QMM_GEMV_JOBS                                                                                         \
    qmm::gemv<FMT, M, R, U, false, 4, true, W>(jobs, act, ldx, K, dump, M, nullptr, 0.0f, accumulate);               \
  }

#define QMM_GEMVF_KERNEL(FMT, NAME, M, W, R, U)                                                           \
  extern "C" __global__ void __launch_bounds__(64 * W)                                                    \
      qmm_gemvf_##NAME##_m##M##_w##W##_r##R##_u##U(QMM_GEMV_PARAMS) {                                     \
    QMM_GEMV_JOBS                                                                                         \
    qmm::gemv<FMT, M, R, U, true, 4, true, W>(jobs, act, ldx, K, dump, M, norm_w, eps, accumulate);                  \
  }

// Eight-job variants (M = 1 only): one launch over up to eight weights that
// share the activation (e.g. a layer's q, k, v, gate and up). The longer
// argument list costs scalar registers, so four-job launches keep their own
// kernels.
#define QMM_GEMV_KERNEL8(FMT, NAME, W, R, U)                                                           \
  extern "C" __global__ void __launch_bounds__(64 * W)                                                 \
      qmm_gemv_##NAME##_m1_w##W##_r##R##_u##U##_j8(QMM_GEMV_PARAMS8) {                                 \
    QMM_GEMV_JOBS8                                                                                     \
    qmm::gemv<FMT, 1, R, U, false, 8, true, W>(jobs, act, ldx, K, dump, 1, nullptr, 0.0f, accumulate);          \
  }
#define QMM_GEMVF_KERNEL8(FMT, NAME, W, R, U)                                                          \
  extern "C" __global__ void __launch_bounds__(64 * W)                                                 \
      qmm_gemvf_##NAME##_m1_w##W##_r##R##_u##U##_j8(QMM_GEMV_PARAMS8) {                                \
    QMM_GEMV_JOBS8                                                                                     \
    qmm::gemv<FMT, 1, R, U, true, 8, true, W>(jobs, act, ldx, K, dump, 1, norm_w, eps, accumulate);             \
  }

// One-row decode kernels (gemv1): four-job and eight-job tables, staged
// (pre-quantized activation) and fused (quantized in the prologue).
#define QMM_GEMV1_KERNELS(FMT, NAME, W)                                                              \
  extern "C" __global__ void __launch_bounds__(64 * W) qmm_gemv1_##NAME##_w##W(QMM_GEMV_PARAMS) {    \
    QMM_GEMV_JOBS                                                                                    \
    qmm::gemv1<FMT, false, 4, false, false, W>(jobs, act, ldx, K, nullptr, 0.0f, accumulate);                         \
  }                                                                                                  \
  extern "C" __global__ void __launch_bounds__(64 * W) qmm_gemv1f_##NAME##_w##W(QMM_GEMV_PARAMS) {   \
    QMM_GEMV_JOBS                                                                                    \
    qmm::gemv1<FMT, true, 4, false, false, W>(jobs, act, ldx, K, norm_w, eps, accumulate);                            \
  }                                                                                                  \
  extern "C" __global__ void __launch_bounds__(64 * W) qmm_gemv1_##NAME##_w##W##_j8(QMM_GEMV_PARAMS8) { \
    QMM_GEMV_JOBS8                                                                                   \
    qmm::gemv1<FMT, false, 8, false, false, W>(jobs, act, ldx, K, nullptr, 0.0f, accumulate);                         \
  }                                                                                                  \
  extern "C" __global__ void __launch_bounds__(64 * W) qmm_gemv1f_##NAME##_w##W##_j8(QMM_GEMV_PARAMS8) { \
    QMM_GEMV_JOBS8                                                                                   \
    qmm::gemv1<FMT, true, 8, false, false, W>(jobs, act, ldx, K, norm_w, eps, accumulate);                            \
  }
// silu(g) * u quantized in the prologue (act = g, norm_w = u).
#define QMM_GEMV1S_KERNEL(FMT, NAME, W)                                                              \
  extern "C" __global__ void __launch_bounds__(64 * W) qmm_gemv1s_##NAME##_w##W(QMM_GEMV_PARAMS) {   \
    QMM_GEMV_JOBS                                                                                    \
    qmm::gemv1<FMT, true, 4, true, false, W>(jobs, act, ldx, K, norm_w, 0.0f, accumulate);                     \
  }
// Mixed Q4_K / Q6_K jobs (e.g. a layer's q, k and v projections in one
// launch); rows >= mix_row are the Q6_K jobs'.
#define QMM_GEMV1_MIX_KERNELS(W)                                                                               \
  extern "C" __global__ void __launch_bounds__(64 * W) qmm_gemv1_q4k6k_w##W(QMM_GEMV_PARAMS, int mix_row) {    \
    QMM_GEMV_JOBS                                                                                              \
    qmm::gemv1<qmm::kFmtQ4K, false, 4, false, true, W>(jobs, act, ldx, K, nullptr, 0.0f, accumulate, mix_row);     \
  }                                                                                                            \
  extern "C" __global__ void __launch_bounds__(64 * W) qmm_gemv1f_q4k6k_w##W(QMM_GEMV_PARAMS, int mix_row) {   \
    QMM_GEMV_JOBS                                                                                              \
    qmm::gemv1<qmm::kFmtQ4K, true, 4, false, true, W>(jobs, act, ldx, K, norm_w, eps, accumulate, mix_row);        \
  }                                                                                                            \
  extern "C" __global__ void __launch_bounds__(64 * W) qmm_gemv1_q4k6k_w##W##_j8(QMM_GEMV_PARAMS8, int mix_row) { \
    QMM_GEMV_JOBS8                                                                                             \
    qmm::gemv1<qmm::kFmtQ4K, false, 8, false, true, W>(jobs, act, ldx, K, nullptr, 0.0f, accumulate, mix_row);     \
  }                                                                                                            \
  extern "C" __global__ void __launch_bounds__(64 * W) qmm_gemv1f_q4k6k_w##W##_j8(QMM_GEMV_PARAMS8, int mix_row) { \
    QMM_GEMV_JOBS8                                                                                             \
    qmm::gemv1<qmm::kFmtQ4K, true, 8, false, true, W>(jobs, act, ldx, K, norm_w, eps, accumulate, mix_row);        \
  }
#define QMM_GEMV1_SHAPES(FMT, NAME) \
  QMM_GEMV1_KERNELS(FMT, NAME, 4)   \
  QMM_GEMV1_KERNELS(FMT, NAME, 8)   \
  QMM_GEMV1_KERNELS(FMT, NAME, 16)  \
  QMM_GEMV1S_KERNEL(FMT, NAME, 8)   \
  QMM_GEMV1S_KERNEL(FMT, NAME, 16)

// Launch shapes: W waves per workgroup, R rows per wave, U load iterations per batch.
#define QMM_GEMV_SHAPES_1(FMT, NAME)        \
  QMM_GEMV_KERNEL(FMT, NAME, 1, 4, 1, 1)    \
  QMM_GEMV_KERNEL(FMT, NAME, 1, 4, 2, 1)    \
  QMM_GEMV_KERNEL(FMT, NAME, 1, 4, 1, 2)    \
  QMM_GEMV_KERNEL(FMT, NAME, 1, 8, 1, 1)    \
  QMM_GEMV_KERNEL(FMT, NAME, 1, 8, 2, 1)    \
  QMM_GEMV_KERNEL(FMT, NAME, 1, 8, 1, 2)    \
  QMM_GEMV_KERNEL(FMT, NAME, 1, 16, 1, 1)   \
  QMM_GEMV_KERNEL(FMT, NAME, 1, 16, 1, 2)

#define QMM_GEMV_SHAPES(FMT, NAME, M)       \
  QMM_GEMV_KERNEL(FMT, NAME, M, 4, 1, 1)    \
  QMM_GEMV_KERNEL(FMT, NAME, M, 4, 2, 1)    \
  QMM_GEMV_KERNEL(FMT, NAME, M, 4, 1, 2)    \
  QMM_GEMV_KERNEL(FMT, NAME, M, 8, 1, 1)    \
  QMM_GEMV_KERNEL(FMT, NAME, M, 8, 1, 2)

#define QMM_GEMVF_SHAPES(FMT, NAME, M)      \
  QMM_GEMVF_KERNEL(FMT, NAME, M, 8, 1, 1)   \
  QMM_GEMVF_KERNEL(FMT, NAME, M, 8, 1, 2)   \
  QMM_GEMVF_KERNEL(FMT, NAME, M, 8, 2, 1)   \
  QMM_GEMVF_KERNEL(FMT, NAME, M, 16, 1, 1)  \
  QMM_GEMVF_KERNEL(FMT, NAME, M, 16, 1, 2)  \
  QMM_GEMVF_KERNEL(FMT, NAME, M, 16, 2, 1)

#define QMM_GEMV_ALL_M(FMT, NAME) \
  QMM_GEMV_SHAPES_1(FMT, NAME)    \
  QMM_GEMV_KERNEL8(FMT, NAME, 4, 1, 1)  \
  QMM_GEMV_KERNEL8(FMT, NAME, 4, 2, 1)  \
  QMM_GEMV_KERNEL8(FMT, NAME, 8, 1, 1)  \
  QMM_GEMV_KERNEL8(FMT, NAME, 8, 2, 1)  \
  QMM_GEMV_KERNEL8(FMT, NAME, 16, 1, 1) \
  QMM_GEMV_KERNEL8(FMT, NAME, 16, 2, 1) \
  QMM_GEMVF_KERNEL8(FMT, NAME, 8, 1, 1) \
  QMM_GEMVF_KERNEL8(FMT, NAME, 8, 2, 1) \
  QMM_GEMVF_KERNEL8(FMT, NAME, 16, 1, 1) \
  QMM_GEMVF_KERNEL8(FMT, NAME, 16, 2, 1) \
  QMM_GEMV_SHAPES(FMT, NAME, 2)   \
  QMM_GEMV_SHAPES(FMT, NAME, 3)   \
  QMM_GEMV_SHAPES(FMT, NAME, 4)   \
  QMM_GEMV_SHAPES(FMT, NAME, 5)   \
  QMM_GEMV_SHAPES(FMT, NAME, 6)   \
  QMM_GEMV_SHAPES(FMT, NAME, 7)   \
  QMM_GEMV_SHAPES(FMT, NAME, 8)   \
  QMM_GEMVF_SHAPES(FMT, NAME, 1)  \
  QMM_GEMVF_SHAPES(FMT, NAME, 2)  \
  QMM_GEMV1_SHAPES(FMT, NAME)

// Grouped one-row launch: two groups of up to eight jobs, each group with its
// own f32 activation row (length K of its jobs), quantized to Q8_K in the
// prologue of the group's workgroups. Workgroups [0, ga) serve group A, the
// rest group B; inside a group the rows are dealt as in gemv1. The job
// records of group A are the first eight of the argument segment, group B's
// the next eight. Independent GEMVs of one decoder layer's shapes (the q / k /
// v / gate / up projections of one row and the down projection of another)
// then stream as one launch, with one ramp-up and one drain.
#define QMM_JOB_SET_AS(dst, i, src) \
  dst.wq[i] = wq##src;              \
  dst.y[i] = y##src;                \
  dst.rows[i] = rows##src;          \
  dst.ldy[i] = ldy##src;            \
  dst.row0[i] = row0##src;          \
  dst.trows[i] = trows##src;
#define QMM_GEMV1G_KERNEL(FMT, NAME, W)                                                                          \
  extern "C" __global__ void __launch_bounds__(64 * W) qmm_gemv1g_##NAME##_w##W(                                \
      QMM_JOB_PARAMS(0), QMM_JOB_PARAMS(1), QMM_JOB_PARAMS(2), QMM_JOB_PARAMS(3), QMM_JOB_PARAMS(4),            \
      QMM_JOB_PARAMS(5), QMM_JOB_PARAMS(6), QMM_JOB_PARAMS(7), QMM_JOB_PARAMS(8), QMM_JOB_PARAMS(9),            \
      QMM_JOB_PARAMS(10), QMM_JOB_PARAMS(11), QMM_JOB_PARAMS(12), QMM_JOB_PARAMS(13), QMM_JOB_PARAMS(14),       \
      QMM_JOB_PARAMS(15), int njobs_a, int total_a, int njobs_b, int total_b, const float* __restrict__ act_a,   \
      const float* __restrict__ act_b, int k_a, int k_b, int ga, int accumulate) {                               \
    qmm::GemvJobs jobs;                                                                                          \
    const bool in_a = (int)blockIdx.x < ga;                                                                      \
    if (in_a) {                                                                                                  \
      QMM_JOB_SET_AS(jobs, 0, 0) QMM_JOB_SET_AS(jobs, 1, 1) QMM_JOB_SET_AS(jobs, 2, 2) QMM_JOB_SET_AS(jobs, 3, 3) \
      QMM_JOB_SET_AS(jobs, 4, 4) QMM_JOB_SET_AS(jobs, 5, 5) QMM_JOB_SET_AS(jobs, 6, 6) QMM_JOB_SET_AS(jobs, 7, 7) \
      jobs.njobs = njobs_a;                                                                                      \
      jobs.total = total_a;                                                                                      \
      qmm::gemv1<FMT, true, 8, false, false, W>(jobs, act_a, 0, k_a, nullptr, 0.0f, accumulate, 0x7fffffff,     \
                                                qmm::job_args(), (int)blockIdx.x, ga);                           \
    } else {                                                                                                     \
      QMM_JOB_SET_AS(jobs, 0, 8) QMM_JOB_SET_AS(jobs, 1, 9) QMM_JOB_SET_AS(jobs, 2, 10)                          \
      QMM_JOB_SET_AS(jobs, 3, 11) QMM_JOB_SET_AS(jobs, 4, 12) QMM_JOB_SET_AS(jobs, 5, 13)                        \
      QMM_JOB_SET_AS(jobs, 6, 14) QMM_JOB_SET_AS(jobs, 7, 15)                                                    \
      jobs.njobs = njobs_b;                                                                                      \
      jobs.total = total_b;                                                                                      \
      qmm::gemv1<FMT, true, 8, false, false, W>(jobs, act_b, 0, k_b, nullptr, 0.0f, accumulate, 0x7fffffff,     \
                                                qmm::job_args() + 8, (int)blockIdx.x - ga, (int)gridDim.x - ga); \
    }                                                                                                            \
  }

QMM_GEMV_ALL_M(qmm::kFmtQ4K, q4k)
QMM_GEMV1G_KERNEL(qmm::kFmtQ4K, q4k, 16)
QMM_GEMV1G_KERNEL(qmm::kFmtQ6K, q6k, 16)
QMM_GEMV_ALL_M(qmm::kFmtQ6K, q6k)
QMM_GEMV_ALL_M(qmm::kFmtQ80, q8_0)
QMM_GEMV1_MIX_KERNELS(4)
QMM_GEMV1_MIX_KERNELS(8)
QMM_GEMV1_MIX_KERNELS(16)
