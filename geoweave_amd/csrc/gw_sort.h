// Wave-level sorting shared by the kernels that order a row's entries in registers.
#pragma once

#include "gw_common.h"

namespace gw {

// Ascending bitonic sort of 64 * R 64-bit keys held by one wave, element e = r * 64 + lane
// in register r: partners e ^ j < 64 apart are exchanged across lanes (shuffles), the
// others within the lane's registers.
template <int R>
__device__ __forceinline__ void wave_bitonic_sort(uint64_t (&key)[R]) {
  const int lane = threadIdx.x & 63;
  constexpr int P = 64 * R;
#pragma unroll
  for (int k = 2; k <= P; k <<= 1) {
#pragma unroll
    for (int j = k >> 1; j > 0; j >>= 1) {
      if (j >= 64) {
        const int jr = j / 64;
#pragma unroll
        for (int r = 0; r < R; ++r) {
          if ((r & jr) == 0) {
            const bool up = (((r * 64 + lane) & k) == 0);
            const uint64_t a = key[r], b = key[r ^ jr];
            const bool swap = (a > b) == up;
            key[r] = swap ? b : a;
            key[r ^ jr] = swap ? a : b;
          }
        }
      } else {
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const uint64_t a = key[r];
          const uint32_t lo = (uint32_t)__shfl_xor((int)(uint32_t)a, j);
          const uint32_t hi = (uint32_t)__shfl_xor((int)(uint32_t)(a >> 32), j);
          const uint64_t b = ((uint64_t)hi << 32) | lo;
          const bool up = (((r * 64 + lane) & k) == 0);
          const bool keep_min = ((lane & j) == 0) == up;
          key[r] = keep_min ? (a < b ? a : b) : (a < b ? b : a);
        }
      }
    }
  }
}

}  // namespace gw
