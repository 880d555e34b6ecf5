// Measurement aid: a plain streaming read of a device buffer, the ceiling a
// weight-streaming GEMV of the same size is compared with. Every thread reads
// 16-byte pieces in a grid-stride loop, four loads in flight per iteration,
// and folds them into one word; a word equal to an unlikely constant is
// stored, so the loads stay live without output traffic.
#pragma once

#include "qmm_common.h"

extern "C" __global__ void __launch_bounds__(256) qmm_stream_read(const uint4* __restrict__ p, long long n16,
                                                                  uint32_t* __restrict__ sink) {
  const long long stride = (long long)gridDim.x * 256;
  long long i = (long long)blockIdx.x * 256 + threadIdx.x;
  uint32_t x = 0;
  for (; i + 3 * stride < n16; i += 4 * stride) {
    const uint4 a = p[i], b = p[i + stride], c = p[i + 2 * stride], d = p[i + 3 * stride];
    x ^= a.x ^ a.y ^ a.z ^ a.w ^ b.x ^ b.y ^ b.z ^ b.w ^ c.x ^ c.y ^ c.z ^ c.w ^ d.x ^ d.y ^ d.z ^ d.w;
  }
  for (; i < n16; i += stride) {
    const uint4 a = p[i];
    x ^= a.x ^ a.y ^ a.z ^ a.w;
  }
  if (x == 0x9e3779b9u) sink[0] = x;
}
