// Pieces shared by the masked dense attention passes (forward: sparse_attn_dense.hip,
// backward: sparse_attn_dense_bwd.hip): the 32x32x16 matrix-core products, the XOR swizzle of
// 64-row LDS tiles, lane-pair exchanges, fp16/bf16 packing, and the selection-mask kernel.
#pragma once

#include <math.h>

#include "gw_common.h"
#include "gw_tile_rows.h"

namespace gw {
namespace {

constexpr float kDLog2e = 1.4426950408889634f;
constexpr float kDLn2 = 0.6931471805599453f;

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));

// D = A B + C for a 32x32 tile with a k-step of 16. Lane l supplies A[l % 32][8 (l / 32) + i]
// and B[8 (l / 32) + i][l % 32] (i < 8, one 16-byte register quad each); accumulator entry r
// of lane l is D[8 (r / 4) + 4 (l / 32) + r % 4][l % 32].
__device__ __forceinline__ f32x16 mma(BF16, uint4 a, uint4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}
__device__ __forceinline__ f32x16 mma(FP16, uint4 a, uint4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a),
                                                __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
}

// Keeps the compiler from moving LDS accesses across this point; within one wave the LDS
// performs them in issue order, so no barrier is needed between a wave's own write and read.
__device__ __forceinline__ void lds_fence() { asm volatile("" ::: "memory"); }

__device__ __forceinline__ uint16_t to_half_bits(BF16, float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }
__device__ __forceinline__ uint16_t to_half_bits(FP16, float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }

typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_v __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_v __attribute__((ext_vector_type(2)));
// Two floats to two 16-bit floats of the tag's type, round to nearest even, in one word
// (v_cvt_pk_f16_f32 / v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack_f16(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){a, b}, f16x2_v));
}
__device__ __forceinline__ uint32_t pack_pair(FP16, float a, float b) { return pack_f16(a, b); }
__device__ __forceinline__ uint32_t pack_pair(BF16, float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){a, b}, bf16x2_v));
}
// Eight consecutive floats as one 16-byte operand quad.
template <typename E>
__device__ __forceinline__ uint4 pack_quad(const float* v) {
  return make_uint4(pack_pair(E{}, v[0], v[1]), pack_pair(E{}, v[2], v[3]), pack_pair(E{}, v[4], v[5]),
                    pack_pair(E{}, v[6], v[7]));
}

// 0 where sel is all ones, neg where it is zero (v_bfi_b32: (sel & 0) | (~sel & neg)).
__device__ __forceinline__ float select_bias(int sel, float neg) {
  float r;
  asm("v_bfi_b32 %0, %1, 0, %2" : "=v"(r) : "v"(sel), "v"(neg));
  return r;
}
// Lanes l and l ^ 32 exchange (v_permlane32_swap); both get op(own, partner).
__device__ __forceinline__ float pair_max(float x) {
  const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
}
__device__ __forceinline__ float pair_sum(float x) {
  const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
}

// LDS tiles of 64 rows of 128 bytes: the 16-byte chunk c of row R sits at c ^ swz(R). Operand
// reads (consecutive rows, one chunk) and tile stores (8 lanes per row) then touch distinct
// banks in every group of 8 and of 16 lanes.
__device__ __forceinline__ int swz(int R) { return (R & 7) ^ ((R >> 3) & 1); }

__device__ __forceinline__ float in_to_float(int in_fp16, uint32_t u) {
  return in_fp16 ? (float)__builtin_bit_cast(_Float16, (uint16_t)u) : __uint_as_float(u << 16);
}

// Non-zero when either 16-bit half of w has its exponent field e all ones (inf or nan).
__device__ __forceinline__ uint32_t nonfinite2(uint32_t w, uint32_t e) {
  return (uint32_t)((w & e) == e) | (uint32_t)(((w >> 16) & e) == e);
}

// 32x32 bit-matrix transpose across the lanes of each half-wave: lane i holds row i (bit c =
// element (i, c)); afterwards lane c holds column c (bit i = element (i, c)). Five rounds of
// exchanging bit blocks with the lane 16, 8, 4, 2, 1 apart.
__device__ __forceinline__ uint32_t lane_bit_transpose32(uint32_t x, int lane) {
  const uint32_t masks[5] = {0x0000FFFFu, 0x00FF00FFu, 0x0F0F0F0Fu, 0x33333333u, 0x55555555u};
#pragma unroll
  for (int i = 0; i < 5; ++i) {
    const int j = 16 >> i;
    const uint32_t m = masks[i];
    const uint32_t y = (uint32_t)__shfl_xor((int)x, j);
    x = (lane & j) ? ((x & ~m) | ((y >> j) & m)) : ((x & m) | ((y << j) & ~m));
  }
  return x;
}

// ---------------------------------------------------------------------------------------
// Selection mask, query-major per 32-key sub-tile: word[b][j][t] has bit i set when query t
// selected key 32 j + i (t < T_pad = nqb_pad * 32, j < S_pad / 32; zero words past S and T).
// Built per (32-query block, chunk of chunk_keys keys) with LDS atomics. The atomic returns
// the word as it was: a bit already set means the query listed the key twice, and the block
// is flagged (flags[b][qb][chunk]; dup_b[b] = 1 too when dup_b is given). Positions are read
// 8 rows at a time (16 bytes per lane when the table allows), so the loads of a group are in
// flight together. With maskT, the same bits key-major as well: maskT[b][qb][s] has bit i set
// when query 32 qb + i selected key s (s < S_pad). With bias_order the words are stored for
// the kernels' selection bias instead: in a query-major word key 8 g + 4 h + j (g, j < 4,
// h < 2) sits at bit beta = 8 j + 7 - g - 4 h, in a key-major word query 8 g + 4 h + j does,
// and both are inverted (a set bit = not selected), so that shifting a word left by g + 4 h
// puts the entries of accumulator group g of lane half h at the sign bits of the four
// bytes. The first workgroup of each batch element clears vmax_words words of vmax and bad[b]
// (for the forward's dense_vmax_kernel), when given.
// ---------------------------------------------------------------------------------------
// Keys per workgroup: at most 606 sub-tiles of 33 words (two workgroups per CU), the key
// range split into equal chunks of whole sub-tiles, so that a key range just past a multiple
// of the largest chunk does not cost a chunk that rereads every position for a few keys.
constexpr int kMaskChunkMax = 606 * 32;
inline int mask_nchunk(int64_t spad) { return (int)((spad + kMaskChunkMax - 1) / kMaskChunkMax); }
inline int mask_chunk_keys(int64_t spad, int nchunk) { return (int)((spad / 32 + nchunk - 1) / nchunk * 32); }

__global__ __launch_bounds__(256) void dense_mask_kernel(const int32_t* __restrict__ pos, int64_t psb, int64_t pst,
                                                         int T, int S, int Spad, int K, int nqb, int tpad,
                                                         int nchunk, int vec, int vmax_words,
                                                         uint32_t* __restrict__ mask, int* __restrict__ flags,
                                                         uint32_t* __restrict__ vmax, int* __restrict__ bad,
                                                         uint32_t* __restrict__ maskT, int* __restrict__ dup_b,
                                                         int bias_order, int chunk_keys) {
  // [key / 32][query], rows padded to 33 words so that one query's atomics spread over banks
  __shared__ uint32_t words[(kMaskChunkMax / 32) * 33];
  __shared__ int dup_any;
  // The chunks of one block are consecutive workgroups: they run together and share the
  // block's positions through the caches.
  const int chunk = blockIdx.x, qb = blockIdx.y, b = blockIdx.z;
  const int c0 = chunk * chunk_keys;
  const int len = max(0, min(chunk_keys, S - c0));
  const int nkt = max(0, min(chunk_keys, Spad - c0)) >> 5;
  for (int i = threadIdx.x; i < nkt * 33; i += 256) words[i] = 0u;
  if (qb == 0 && chunk == 0 && vmax != nullptr) {
    for (int i = threadIdx.x; i < vmax_words; i += 256) vmax[(int64_t)b * vmax_words + i] = 0u;
    if (threadIdx.x == 0) bad[b] = 0;
  }
  if (threadIdx.x == 0) dup_any = 0;
  __syncthreads();
  bool dup = false;
  const int rows = min(32, T - qb * 32);  // <= 0 for the padding blocks
  const int32_t* pblk = pos + b * psb + (int64_t)min(qb * 32, T - 1) * pst;
  // Positions outside [c0, c0 + len) (other chunks, negative padding, >= S) wrap to large
  // unsigned offsets and are skipped.
  auto put = [&](int32_t sidx, int i) {
    const uint32_t sl = (uint32_t)sidx - (uint32_t)c0;
    if (sl < (uint32_t)len) {
      const uint32_t kk = sl & 31u;
      const uint32_t bit = 1u << (bias_order ? 8u * (kk & 3u) + 7u - (kk >> 3) - 4u * ((kk >> 2) & 1u) : kk);
      dup |= (atomicOr(&words[(sl >> 5) * 33 + i], bit) & bit) != 0u;
    }
  };
  if (vec) {
    // K % 4 == 0 and 16-byte aligned rows: one int4 per lane and row.
    const int n4 = K >> 2;
    for (int j4 = threadIdx.x; j4 < n4; j4 += 256) {
#pragma unroll 1
      for (int r0 = 0; r0 < rows; r0 += 8) {
        int4 v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u)
          v[u] = r0 + u < rows ? reinterpret_cast<const int4*>(pblk + (int64_t)(r0 + u) * pst)[j4] : make_int4(-1, -1, -1, -1);
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          put(v[u].x, r0 + u);
          put(v[u].y, r0 + u);
          put(v[u].z, r0 + u);
          put(v[u].w, r0 + u);
        }
      }
    }
  } else {
#pragma unroll 1
    for (int i = 0; i < rows; ++i) {
      const int32_t* prow = pblk + (int64_t)i * pst;
      for (int j = threadIdx.x; j < K; j += 256) put(prow[j], i);
    }
  }
  if (dup) dup_any = 1;
  __syncthreads();
  uint32_t* out = mask + ((int64_t)b * (Spad >> 5) + (c0 >> 5)) * tpad + qb * 32;
  for (int idx = threadIdx.x; idx < nkt * 32; idx += 256) {
    const int kt = idx >> 5, i = idx & 31;
    const uint32_t wv = words[kt * 33 + i];
    out[(int64_t)kt * tpad + i] = bias_order ? ~wv : wv;
  }
  if (maskT != nullptr) {
    // Two sub-tiles per wave at a time, one per half-wave: lane i reads query i's word and
    // after the transpose holds key 32 kt + i's word over the block's 32 queries. With
    // bias_order the LDS words hold key kk at bit beta(kk) (the permutation above): lane i
    // then reads query beta^-1(i)'s word, so that after the transpose lane i holds key
    // beta^-1(i)'s word with query q at bit beta(q), and stores it inverted at that key.
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int li = lane & 31;
    const int pi = bias_order ? 8 * ((7 - (li & 7)) & 3) + 4 * ((7 - (li & 7)) >> 2) + (li >> 3) : li;
    uint32_t* outT = maskT + ((int64_t)b * (tpad >> 5) + qb) * Spad + c0;
    for (int kt2 = wave * 2; kt2 < nkt; kt2 += 8) {
      const int kt = kt2 + (lane >> 5);
      uint32_t x = kt < nkt ? words[kt * 33 + pi] : 0u;
      x = lane_bit_transpose32(x, lane);
      if (kt < nkt) outT[kt * 32 + pi] = bias_order ? ~x : x;
    }
  }
  if (threadIdx.x == 0 && qb < nqb) {
    flags[((int64_t)b * nqb + qb) * nchunk + chunk] = dup_any;
    if (dup_any && dup_b != nullptr) dup_b[b] = 1;  // every writer stores the same value
  }
}

// ---------------------------------------------------------------------------------------
// The forward's selection words in one pass over the positions: a workgroup builds the words
// of 16 queries over every key (half hq of 32-query block qb) in LDS, [sub-tile][17 words],
// so each position is read once. Same words, bit order and repeat detection as
// dense_mask_kernel; the repeat flag of half hq goes to flags[b][qb][hq] (two entries per
// block). Holds S_pad / 32 <= kMaskRowsMaxSub sub-tiles (dynamic LDS: 68 bytes each).
// ---------------------------------------------------------------------------------------
constexpr int kMaskRowsQ = 16;              // queries per workgroup
constexpr int kMaskRowsMaxSub = 2048;       // sub-tiles held in LDS (139 KB)
constexpr int kMaskRowsThreads = 512;

__global__ __launch_bounds__(kMaskRowsThreads) void dense_mask_rows_kernel(
    const int32_t* __restrict__ pos, int64_t psb, int64_t pst, int T, int S, int Spad, int K, int nqb, int tpad,
    int vec, int vmax_words, uint32_t* __restrict__ mask, int* __restrict__ flags, uint32_t* __restrict__ vmax,
    int* __restrict__ bad, int bias_order) {
  extern __shared__ __align__(16) uint32_t words[];  // [sub-tile][kMaskRowsQ + 1]
  __shared__ int dup_any;
  constexpr int RW = kMaskRowsQ + 1;
  const int qb = blockIdx.x >> 1, hq = blockIdx.x & 1, b = blockIdx.y;
  const int q0 = qb * 32 + hq * kMaskRowsQ;
  const int nkt = Spad >> 5;
  {
    // Clear the words with 16-byte stores (the dynamic LDS array is 16-byte aligned).
    const int n = nkt * RW, n4 = n >> 2;
    for (int i = threadIdx.x; i < n4; i += kMaskRowsThreads) reinterpret_cast<uint4*>(words)[i] = make_uint4(0, 0, 0, 0);
    if (threadIdx.x < (n & 3)) words[4 * n4 + threadIdx.x] = 0u;
  }
  if (blockIdx.x == 0 && vmax != nullptr) {
    for (int i = threadIdx.x; i < vmax_words; i += kMaskRowsThreads) vmax[(int64_t)b * vmax_words + i] = 0u;
    if (threadIdx.x == 0) bad[b] = 0;
  }
  if (threadIdx.x == 0) dup_any = 0;
  __syncthreads();
  bool dup = false;
  const int rows = min(kMaskRowsQ, T - q0);  // <= 0 for the padding queries
  const int32_t* pblk = pos + b * psb + (int64_t)min(q0, T - 1) * pst;
  // Positions outside [0, S) (negative padding included) wrap to large unsigned values.
  auto put = [&](int32_t sidx, int i) {
    const uint32_t sl = (uint32_t)sidx;
    if (sl < (uint32_t)S) {
      const uint32_t kk = sl & 31u;
      const uint32_t bit = 1u << (bias_order ? 8u * (kk & 3u) + 7u - (kk >> 3) - 4u * ((kk >> 2) & 1u) : kk);
      dup |= (atomicOr(&words[(sl >> 5) * RW + i], bit) & bit) != 0u;
    }
  };
  if (vec) {
    const int n4 = K >> 2;
    for (int j4 = threadIdx.x; j4 < n4; j4 += kMaskRowsThreads) {
#pragma unroll 1
      for (int r0 = 0; r0 < rows; r0 += 8) {
        int4 v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u)
          v[u] = r0 + u < rows ? reinterpret_cast<const int4*>(pblk + (int64_t)(r0 + u) * pst)[j4] : make_int4(-1, -1, -1, -1);
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          put(v[u].x, r0 + u);
          put(v[u].y, r0 + u);
          put(v[u].z, r0 + u);
          put(v[u].w, r0 + u);
        }
      }
    }
  } else {
#pragma unroll 1
    for (int i = 0; i < rows; ++i) {
      const int32_t* prow = pblk + (int64_t)i * pst;
      for (int j = threadIdx.x; j < K; j += kMaskRowsThreads) put(prow[j], i);
    }
  }
  if (dup) dup_any = 1;
  __syncthreads();
  // Four consecutive words of a sub-tile row per thread, one 16-byte store (q0 and tpad are
  // multiples of 16 and 32).
  uint32_t* out = mask + (int64_t)b * nkt * tpad + q0;
  const uint32_t inv = bias_order ? 0xFFFFFFFFu : 0u;
  for (int idx = threadIdx.x; idx < nkt * (kMaskRowsQ / 4); idx += kMaskRowsThreads) {
    const int kt = idx / (kMaskRowsQ / 4), i = 4 * (idx % (kMaskRowsQ / 4));
    const uint32_t* wr = &words[kt * RW + i];
    *reinterpret_cast<uint4*>(out + (int64_t)kt * tpad + i) =
        make_uint4(wr[0] ^ inv, wr[1] ^ inv, wr[2] ^ inv, wr[3] ^ inv);
  }
  if (threadIdx.x == 0 && qb < nqb) flags[((int64_t)b * nqb + qb) * 2 + hq] = dup_any;
}

}  // namespace
}  // namespace gw
