// Measurement aid: plain streaming reads of a device buffer, the ceiling a
// weight-streaming GEMV of the same size is compared with. No single read
// pattern is fastest at every size, so three variants are kept and a
// calibration run takes the best per size:
//   gs4 / gs8  every thread reads 16-byte pieces in a grid-stride loop with
//              four / eight loads in flight per iteration;
//   ch8nt      workgroup b reads the b-th contiguous chunk of the buffer, the
//              workgroup's threads consecutive 16-byte pieces, eight
//              nontemporal loads in flight.
// Loads are folded into one word; a word equal to an unlikely constant is
// stored, so the loads stay live without output traffic.
#pragma once

#include "qmm_common.h"

namespace qmm {
typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));

template <int U, bool CHUNK, bool NT>
__device__ __forceinline__ void stream_read(const u32x4_t* __restrict__ p, long long n16, uint32_t* __restrict__ sink) {
  long long i, end, stride;
  if constexpr (CHUNK) {
    const long long per = (n16 + gridDim.x - 1) / gridDim.x;
    i = (long long)blockIdx.x * per + threadIdx.x;
    end = min((long long)(blockIdx.x + 1) * per, n16);
    stride = 256;
  } else {
    i = (long long)blockIdx.x * 256 + threadIdx.x;
    end = n16;
    stride = (long long)gridDim.x * 256;
  }
  uint32_t x = 0;
  for (; i + (U - 1) * stride < end; i += U * stride) {
    u32x4_t v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) v[u] = NT ? __builtin_nontemporal_load(p + i + u * stride) : p[i + u * stride];
#pragma unroll
    for (int u = 0; u < U; ++u) x ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  for (; i < end; i += stride) {
    const u32x4_t a = p[i];
    x ^= a.x ^ a.y ^ a.z ^ a.w;
  }
  if (x == 0x9e3779b9u) sink[0] = x;
}
}  // namespace qmm

#define QMM_STREAM_READ_KERNEL(NAME, U, CHUNK, NT)                                                       \
  extern "C" __global__ void __launch_bounds__(256) qmm_stream_read_##NAME(                              \
      const qmm::u32x4_t* __restrict__ p, long long n16, uint32_t* __restrict__ sink) {                  \
    qmm::stream_read<U, CHUNK, NT>(p, n16, sink);                                                        \
  }
QMM_STREAM_READ_KERNEL(gs4, 4, false, false)
QMM_STREAM_READ_KERNEL(gs8, 8, false, false)
QMM_STREAM_READ_KERNEL(ch8nt, 8, true, true)
