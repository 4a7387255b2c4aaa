// Block-wide exact radix selection and deterministic compaction used by the indexer
// top-k kernels. 256 threads per block (4 waves of 64).
#pragma once

#include "gw_common.h"

namespace gw {

constexpr int kSelThreads = 256;

// Order-preserving map fp32 -> uint32 (larger float <-> larger key; +NaN above +inf, which
// matches torch.topk's treatment of NaN as the largest value).
__device__ __forceinline__ uint32_t f2key(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float key2f(uint32_t k) {
  const uint32_t u = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
  return __uint_as_float(u);
}

__device__ __forceinline__ int wave_incl_scan(int x) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_up(x, off);
    if (lane >= off) x += y;
  }
  return x;
}

struct SelectShared {
  int hist[256];
  int bcast[4];
  int wave_tot[2][4];
};

// Finds the R-th largest (1-based, R <= n) of n keys read through key_at(i). Returns that
// key; take_eq receives how many elements equal to it belong to the top R (the rest of
// the top R are strictly greater). Must be called by all threads of the block.
template <typename KeyAt>
__device__ uint32_t block_radix_select(KeyAt key_at, int n, int R, SelectShared& sh, int& take_eq) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  uint32_t prefix = 0, pmask = 0;
  int rem = R;
#pragma unroll 1
  for (int shift = 24; shift >= 0; shift -= 8) {
    sh.hist[tid] = 0;
    __syncthreads();
    for (int i = tid; i < n; i += kSelThreads) {
      const uint32_t kk = key_at(i);
      if ((kk & pmask) == prefix) atomicAdd(&sh.hist[(kk >> shift) & 255u], 1);
    }
    __syncthreads();
    if (tid < 64) {
      int c[4];
      int local = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        c[j] = sh.hist[255 - 4 * lane - j];
        local += c[j];
      }
      const int incl = wave_incl_scan(local);
      const int excl = incl - local;
      if (excl < rem && rem <= incl) {
        int acc = excl;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if (acc + c[j] >= rem) {
            sh.bcast[0] = 255 - 4 * lane - j;
            sh.bcast[1] = acc;
            break;
          }
          acc += c[j];
        }
      }
    }
    __syncthreads();
    const uint32_t digit = (uint32_t)sh.bcast[0];
    rem -= sh.bcast[1];
    prefix |= digit << shift;
    pmask |= 0xFFu << shift;
    __syncthreads();
  }
  take_eq = rem;
  return prefix;
}

// Block exclusive scan of two counters; returns the prefixes for this thread.
__device__ __forceinline__ void block_excl_scan2(int a, int b, int& ea, int& eb, SelectShared& sh) {
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int ia = wave_incl_scan(a);
  const int ib = wave_incl_scan(b);
  if (lane == 63) {
    sh.wave_tot[0][wave] = ia;
    sh.wave_tot[1][wave] = ib;
  }
  __syncthreads();
  int oa = 0, ob = 0;
  for (int w = 0; w < wave; ++w) {
    oa += sh.wave_tot[0][w];
    ob += sh.wave_tot[1][w];
  }
  ea = oa + ia - a;
  eb = ob + ib - b;
  __syncthreads();
}

// Writes the top R elements (all keys > kth, then the first take_eq keys == kth in index
// order) through emit(out_slot, i). The result is independent of thread timing.
template <typename KeyAt, typename Emit>
__device__ void block_emit_topk(KeyAt key_at, int n, int R, uint32_t kth, int take_eq, Emit emit,
                                SelectShared& sh) {
  const int tid = threadIdx.x;
  const int chunk = (n + kSelThreads - 1) / kSelThreads;
  const int i0 = tid * chunk;
  const int i1 = min(n, i0 + chunk);
  int cg = 0, ce = 0;
  for (int i = i0; i < i1; ++i) {
    const uint32_t kk = key_at(i);
    cg += kk > kth;
    ce += kk == kth;
  }
  int og, oe;
  block_excl_scan2(cg, ce, og, oe, sh);
  const int n_gt = R - take_eq;
  for (int i = i0; i < i1; ++i) {
    const uint32_t kk = key_at(i);
    if (kk > kth) {
      emit(og++, i);
    } else if (kk == kth) {
      if (oe < take_eq) emit(n_gt + oe, i);
      ++oe;
    }
  }
}

}  // namespace gw
