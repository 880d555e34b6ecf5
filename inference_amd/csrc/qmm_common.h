// Shared device helpers for the gfx950 quantized-matmul kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qmm {

// GGML block geometry (bytes per block; the format tables of
// crates/llm/mlx-llm/src/gguf/dequant.rs:115-141).
constexpr int kQ80Bytes = 34;
constexpr int kQ4KBytes = 144;
constexpr int kQ6KBytes = 210;
constexpr int kQ8KBytes = 292;
// Device layouts that differ from GGML keep the same bytes per block but split
// the 2-byte f16 scale out of the block so every block body is 16-byte aligned:
//   Q6_K: body[208] = ql[128] | qh[64] | scales[16]; then one f16 d per block.
//   Q8_0: qs[32]; then one f16 d per block.
constexpr int kQ6KBody = 208;
constexpr int kQ80Body = 32;

enum Fmt { kFmtQ80 = 0, kFmtQ4K = 1, kFmtQ6K = 2 };

__device__ __forceinline__ float h2f(uint32_t h) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(h & 0xffffu));
}

// f32 -> IEEE binary16, round to nearest even (hardware conversion; the
// default MODE keeps f16 denormals).
__device__ __forceinline__ uint16_t f2h(float f) {
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}

// Signed 4x8-bit dot product with accumulate (v_dot4_i32_i8).
__device__ __forceinline__ int dot4(uint32_t a, uint32_t b, int c) {
  return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}

__device__ __forceinline__ float readlane_f(float v, int lane) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// Sum over the 64 lanes of a wave; every lane receives the total.
// Rows of 16 lanes are reduced with DPP (quad swaps, half-row and row
// mirrors), the four rows with two cross-row exchanges.
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_f<0xb1>(v);   // quad_perm [1,0,3,2]
  v += dpp_f<0x4e>(v);   // quad_perm [2,3,0,1]
  v += dpp_f<0x141>(v);  // row_half_mirror
  v += dpp_f<0x140>(v);  // row_mirror
  v += __shfl_xor(v, 16);
  v += __shfl_xor(v, 32);
  return v;
}

// Sum over the 64 lanes of a wave as a wave-uniform value: DPP inside rows of
// 16 lanes, then the four row sums are read with v_readlane (no LDS round
// trip). Summation order: rows, then (row 0 + row 1) + (row 2 + row 3).
__device__ __forceinline__ float wave_total(float v) {
  v += dpp_f<0xb1>(v);
  v += dpp_f<0x4e>(v);
  v += dpp_f<0x141>(v);
  v += dpp_f<0x140>(v);
  return (readlane_f(v, 0) + readlane_f(v, 16)) + (readlane_f(v, 32) + readlane_f(v, 48));
}

// Max over the 64 lanes of a wave (every lane receives it): DPP inside rows
// of 16 lanes, then the four row results are read with v_readlane.
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp_f<0xb1>(v));
  v = fmaxf(v, dpp_f<0x4e>(v));
  v = fmaxf(v, dpp_f<0x141>(v));
  v = fmaxf(v, dpp_f<0x140>(v));
  return fmaxf(fmaxf(readlane_f(v, 0), readlane_f(v, 16)), fmaxf(readlane_f(v, 32), readlane_f(v, 48)));
}

template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xf, 0xf, false);
}

// Min over the 64 lanes of a wave (every lane receives it).
__device__ __forceinline__ int wave_min(int v) {
  v = min(v, dpp_i<0xb1>(v));
  v = min(v, dpp_i<0x4e>(v));
  v = min(v, dpp_i<0x141>(v));
  v = min(v, dpp_i<0x140>(v));
  const int a = __builtin_amdgcn_readlane(v, 0), b = __builtin_amdgcn_readlane(v, 16);
  const int c = __builtin_amdgcn_readlane(v, 32), d = __builtin_amdgcn_readlane(v, 48);
  return min(min(a, b), min(c, d));
}

// Sum over aligned groups of 4 lanes (every lane of the group receives it).
__device__ __forceinline__ int quad_sum(int v) {
  v += dpp_i<0xb1>(v);
  return v + dpp_i<0x4e>(v);
}

}  // namespace qmm
