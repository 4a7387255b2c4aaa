// Lightning-indexer score + exact per-query top-k for gfx950, without an N x N score
// matrix in memory.
//
//   score[b,t,s] = sum_h w[b,s,h] * relu(scale * <q[b,t,h], k[b,s,h]>)  (+ mask[b,t,s])
//                  (+ view_bias[b, q_view[b,t], s_view[b,s]])
//
// (reference easyvolcap/official_vggt/layers/indexer.py:430-466 and
// easyvolcap/utils/custom_indexer/sparse_topk_indexer.py:935-951). scale > 0 lets the
// scale move onto the gate: w*relu(scale*z) = (scale*w)*relu(z).
//
// Pipeline (all on the caller's stream, no host synchronisation):
//  K0 score_kernel<SAMPLE>: MFMA scores of every query against Ms strided sample keys
//                           (split over workgroups like K1).
//  K0b tau_kernel:          one wave per query: a threshold tau whose rank among the
//                           sample scores lies in [r, r + 8], r chosen so that at least
//                           topk keys of the whole row score >= tau with very high
//                           probability (about 1.7 x topk keys on average).
//  K1 score_kernel<FILTER>: MFMA scores against all keys; the epilogue appends
//                           (score, key) pairs with score > tau to the query's candidate
//                           list (one list per query and key split).
//  K2 select_kernel:        one wave per query: exact top-k of the candidates held in
//                           registers (bisection on the order-preserving score bits,
//                           ballot-ordered emit). A query whose lists overflowed or hold
//                           fewer than topk entries is queued for K3; one whose candidates
//                           exceed the register slots is queued for K2b.
//  K2b select_wide_kernel:  persistent workgroups: all candidates of a queued query in
//                           LDS, block radix select.
//  K3 score_kernel<SAMPLE> on the queued rows (up to kFullRows per batch element): MFMA
//                           scores of each queued row against every key, gathered rows,
//                           the key range split finely; full_select_kernel: exact top-k
//                           of those rows by range-relative histogram levels + block radix
//                           select; fallback_kernel: scores and selects any rows past
//                           kFullRows itself - correct for any input, used rarely.
// Exactness: if count(score > tau) >= topk, every member of the top-k scores > tau and is a
// candidate, so selecting among the candidates is exact (otherwise the query has fewer than
// topk candidates and goes to the brute force). Ties at the k-th value are broken
// deterministically (candidate order: split, then position in the list). No step bounds
// topk: one whose expected candidates exceed 3/4 of the candidate slots (kSubTotal) sends
// every row through K3's full scoring and row select, in rounds of up to 4 x kFullRows rows
// per batch element (no threshold, filter or list select), and one above the register slots (at most
// 96 per lane) sends most queries to K2b.
//
// MFMA layout (v_mfma_f32_32x32x16_{bf16,f16}), transposed: per tile of 32 keys a wave
// forms S^T[32 keys x 32 queries] = K Q^T with A = key rows staged through LDS (XOR-swizzled
// 16-byte chunks, conflict-free operand reads) and B = its 32 query rows, stationary in
// VGPRs for the whole key sweep. Lane l then holds query l%32 and keys 8*(r/4) + 4*(l/32) +
// r%4 of the tile in accumulator element r: all 16 elements of a lane belong to one query.
//
// Candidate appends: about 4 % of the elements pass the threshold, so a memory instruction
// per element would be mostly empty (and a wave issues one for most elements). Instead a
// lane only compares each element against its query's threshold (a bit in a mask) and puts
// its scores in an LDS staging row; once per stage of keys a short loop writes the marked
// entries, every lane its lowest marked one per round, to its query's list (one list per
// query and key split, shared by the query's two lanes). The lists come out in a fixed
// order, the same on every run.
//
// Key splits: to fill the chip, the key range is divided over nsplit workgroups per
// query tile. Split sp takes the key stages sp, sp + nsplit, sp + 2*nsplit, ...; the
// interleave spreads any locality of a query's favourite keys (e.g. its own view) evenly
// over the splits, so every list receives about candidates / (2 nsplit) entries.
#include <math.h>

#include <algorithm>
#include <mutex>

#include "gw_common.h"
#include "gw_select.h"

namespace gw {
namespace {

constexpr int kQW = 32;            // queries per wave
constexpr int kDI = 64;            // indexer head dim
constexpr int kSubTotal = 8192;    // candidate slots per query over all lists
constexpr int kMaxSplit = 8;
constexpr int kMaxLists = kMaxSplit;
constexpr int kFallbackBlocks = 256;
// Rows per batch element whose fallback scores come from the matrix cores (the rest, rare,
// are scored by the fallback kernel itself).
constexpr int kFullRows = 512;
// Candidate layout: int2 {score bits, key} lists, one per row and key split: list l = split
// of row r starts at cand[(r * nsplit + l) * cap], cap = kSubTotal / nsplit, and holds
// counts[r * nsplit + l] entries (more than cap: the list overflowed; entries past cap were
// not written).

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));

__device__ __forceinline__ f32x16 mfma32(BF16, uint4 a, uint4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}
__device__ __forceinline__ f32x16 mfma32(FP16, uint4 a, uint4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a),
                                                __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
}

// fp32 operands: v_mfma_f32_32x32x2_f32, one fp32 element of A and of B per lane (k index
// lane / 32), exact fp32 products accumulated in fp32.
__device__ __forceinline__ f32x16 mfma32_f32(uint32_t a, uint32_t b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a), __uint_as_float(b), c, 0, 0, 0);
}

// A gate value from its raw bits (the 16-bit pattern, or the fp32 bits).
__device__ __forceinline__ float to_f32(BF16, uint32_t x) { return __uint_as_float(x << 16); }
__device__ __forceinline__ float to_f32(FP16, uint32_t x) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)x);
}
__device__ __forceinline__ float to_f32(FP32, uint32_t x) { return __uint_as_float(x); }
__device__ __forceinline__ uint32_t raw_bits(BF16, const void* p, int64_t i) { return static_cast<const uint16_t*>(p)[i]; }
__device__ __forceinline__ uint32_t raw_bits(FP16, const void* p, int64_t i) { return static_cast<const uint16_t*>(p)[i]; }
__device__ __forceinline__ uint32_t raw_bits(FP32, const void* p, int64_t i) { return static_cast<const uint32_t*>(p)[i]; }

// relu on the bit pattern: every negative float (sign bit set) becomes +0, every
// non-negative one is kept bit for bit. One v_max_i32, where fmaxf(x, 0) costs a NaN
// canonicalisation plus the max.
__device__ __forceinline__ float relu_bits(float x) { return __int_as_float(max(__float_as_int(x), 0)); }

// Wave-wide reductions (all 64 lanes active): DPP within each 16-lane row, then the four
// row results through readlane; the result is wave-uniform.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u(uint32_t x) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, CTRL, 0xF, 0xF, true);
}
__device__ __forceinline__ uint32_t wave_sum_u(uint32_t x) {
  x += dpp_u<kDppXor1>(x);
  x += dpp_u<kDppXor2>(x);
  x += dpp_u<kDppHalfMirror>(x);
  x += dpp_u<kDppMirror>(x);
  return __builtin_amdgcn_readlane(x, 0) + __builtin_amdgcn_readlane(x, 16) +
         __builtin_amdgcn_readlane(x, 32) + __builtin_amdgcn_readlane(x, 48);
}
__device__ __forceinline__ uint32_t wave_min_u(uint32_t x) {
  x = min(x, dpp_u<kDppXor1>(x));
  x = min(x, dpp_u<kDppXor2>(x));
  x = min(x, dpp_u<kDppHalfMirror>(x));
  x = min(x, dpp_u<kDppMirror>(x));
  const uint32_t a = min((uint32_t)__builtin_amdgcn_readlane(x, 0), (uint32_t)__builtin_amdgcn_readlane(x, 16));
  const uint32_t b = min((uint32_t)__builtin_amdgcn_readlane(x, 32), (uint32_t)__builtin_amdgcn_readlane(x, 48));
  return min(a, b);
}
__device__ __forceinline__ uint32_t wave_max_u(uint32_t x) {
  x = max(x, dpp_u<kDppXor1>(x));
  x = max(x, dpp_u<kDppXor2>(x));
  x = max(x, dpp_u<kDppHalfMirror>(x));
  x = max(x, dpp_u<kDppMirror>(x));
  const uint32_t a = max((uint32_t)__builtin_amdgcn_readlane(x, 0), (uint32_t)__builtin_amdgcn_readlane(x, 16));
  const uint32_t b = max((uint32_t)__builtin_amdgcn_readlane(x, 32), (uint32_t)__builtin_amdgcn_readlane(x, 48));
  return max(a, b);
}

// Number of set bits of a wave mask below this lane.
__device__ __forceinline__ uint32_t lanes_below_u(uint64_t m) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

// Bisection for a threshold key over per-lane key slots, wave-wide. Invariant: cnt_lo =
// count(key >= lo) >= need > cnt_hi = count(key >= hi); each step counts the keys >= mid.
// Returns the final lo: hi = lo + 1, or the first lo whose count is <= need + slack.
// Only the keys in [lo, hi) can change a count, so once at most kCompactKeys of them are
// left they are copied (ballot-ordered) into the wave's LDS buffer and the remaining steps
// count those, one or a few per lane, plus cnt_hi, instead of every slot. The sequence of
// mid values and counts, and so the result, is the bisection's over all slots.
constexpr int kCompactKeys = 256;

template <int S>
__device__ __forceinline__ uint32_t wave_bisect_keys(const uint32_t (&kv)[S], int nslot, uint64_t lo, uint64_t hi,
                                                     int cnt_lo, int cnt_hi, int need, int slack, uint32_t* buf) {
  while (hi - lo > 1 && cnt_lo - cnt_hi > kCompactKeys) {
    const uint32_t mid = (uint32_t)(lo + ((hi - lo) >> 1));
    uint32_t cc = 0;
#pragma unroll
    for (int m0 = 0; m0 < S; m0 += 8) {
      if (m0 < nslot) {
#pragma unroll
        for (int m = m0; m < m0 + 8 && m < S; ++m) cc += kv[m] >= mid;
      }
    }
    const int c = (int)wave_sum_u(cc);
    if (c >= need) {
      lo = mid;
      cnt_lo = c;
      if (c <= need + slack) return (uint32_t)lo;
    } else {
      hi = mid;
      cnt_hi = c;
    }
  }
  if (hi - lo <= 1) return (uint32_t)lo;
  // Copy the keys in [lo, hi) (cnt_lo - cnt_hi of them) into buf, slot by slot.
  const uint32_t lo32 = (uint32_t)lo, span = (uint32_t)(hi - lo);
  int base = 0;
#pragma unroll
  for (int m0 = 0; m0 < S; m0 += 8) {
    if (m0 < nslot) {
#pragma unroll
      for (int m = m0; m < m0 + 8 && m < S; ++m) {
        const bool in = kv[m] - lo32 < span;
        const uint64_t bm = __ballot(in);
        const int at = base + (int)lanes_below_u(bm);
        if (in && at < kCompactKeys) buf[at] = kv[m];  // the bound holds by the invariant
        base += __popcll(bm);
      }
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const int lane = threadIdx.x & 63;
  constexpr int CS = kCompactKeys / 64;
  uint32_t cv[CS];
#pragma unroll
  for (int j = 0; j < CS; ++j) cv[j] = j * 64 + lane < base ? buf[j * 64 + lane] : 0u;  // 0 < every mid
  // Every copied key is below the hi of the copy, whose count cnt_hi stays the base.
  while (hi - lo > 1) {
    const uint32_t mid = (uint32_t)(lo + ((hi - lo) >> 1));
    uint32_t cc = 0;
#pragma unroll
    for (int j = 0; j < CS; ++j) cc += cv[j] >= mid;
    const int c = cnt_hi + (int)wave_sum_u(cc);
    if (c >= need) {
      lo = mid;
      if (c <= need + slack) break;
    } else {
      hi = mid;
    }
  }
  return (uint32_t)lo;
}

enum TauMode { kTauArray = 0, kTauPlusInf = 1, kTauMinusInf = 2 };

// Additive score terms (template flags): the dense mask [B, T, S] and the soft view bias, a
// [B, Vq, Vs] table indexed by the query's and the key's view ids (reference
// sparse_topk_indexer.py:935-951: (score + mask) + view_bias, in that order). View ids are
// clamped into the table, so bad ids cannot read outside it; the host checks their range.
constexpr int kBiasMask = 1;
constexpr int kBiasView = 2;

__device__ __forceinline__ int clamp_view(int v, int n) { return v < 0 ? 0 : (v >= n ? n - 1 : v); }

// Tensors are in the element type E of the launch (bf16, fp16 or fp32).
struct ScoreParams {
  const void* q;      // [B, T, HI, 64]
  const void* k;      // [B, S, HI, 64]
  const void* w;      // [B, S, HI]
  const void* mask;   // [B, T, S] or null
  const void* vbias;  // kBiasView: [B, Vq, Vs]
  const int* qview;       // kBiasView: [B, T]
  const int* sview;       // kBiasView: [B, S]
  int Vq, Vs;
  const float* tau;      // [B*T] or null (-inf)
  float* samp;           // SAMPLE: [B*T, Ms] (with rows: [B, rows_cap, Ms])
  // SAMPLE with rows != null: the queries are rows[b * T + j] (flat b * T + t indices) for j
  // below min(nrows[b], rows_cap), and row j's scores go to samp[(b * rows_cap + j) * Ms].
  const int* rows;
  const int* nrows;
  int rows_cap;
  int2* cand;            // FILTER: candidate lists (see kSubTotal)
  int* counts;           // FILTER: [B*T, nsplit] entries per list (more than cap: overflowed)
  int T, S;
  int nsplit, cap;       // FILTER: key splits; valid entries per list
  int nstages;           // key stages (ScoreShape::BN keys) of the sweep
  int Ms;
  int tau_mode;
  int force_wide;
  float scale;
};

// Key index of position i of the sweep (SAMPLE: i-th strided sample key).
template <bool SAMPLE>
__device__ __forceinline__ int sweep_key(int i, const ScoreParams& p) {
  if constexpr (SAMPLE) return (int)(((int64_t)i * p.S) / p.Ms);
  return i;
}

// Key tiles reach LDS through direct global->LDS loads (global_load_lds_dwordx4: lane l
// of a wave writes 16 bytes at the wave's LDS base + 16*l), so no staging registers are
// needed. Rows are stored unpadded with the 16-byte chunks of key row kl XOR-swizzled by
// (kl & SWZ), SWZ = 15 for rows of >= 16 chunks (HI >= 2), else 7: the MFMA operand reads
// (32 consecutive key rows at one logical chunk) then hit 16 distinct 16-byte bank groups
// per 16 lanes (8 for HI = 1), one LDS pass per 256 bytes.
//
// The loads are issued through inline asm, so the compiler does not see instructions that
// write LDS behind its back: otherwise it cannot tell that a prefetch into one stage buffer
// does not alias the operand reads of the other, and waits for the prefetch (vmcnt(0))
// before the first read. The kernel waits for the loads itself (vmcnt(0) before the stage
// barrier). M0 carries the wave's LDS destination and is restored after each load.
__device__ __forceinline__ void lds_dma16(const void* src, const void* lds_dst) {
  const uint32_t lds = (uint32_t)(uintptr_t)lds_dst;
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %2\n\t"
      "global_load_lds_dwordx4 %1, off\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(src), "s"(__builtin_amdgcn_readfirstlane(lds))
      : "memory");
}

// The same load from a wave-uniform base (an SGPR pair) plus a 32-bit per-lane offset: no
// 64-bit address arithmetic per load.
__device__ __forceinline__ void lds_dma16_s(const void* base, uint32_t off, const void* lds_dst) {
  const uint32_t lds = (uint32_t)(uintptr_t)lds_dst;
  const uint64_t b = reinterpret_cast<uintptr_t>(base);
  const uint64_t bu = ((uint64_t)__builtin_amdgcn_readfirstlane((uint32_t)(b >> 32)) << 32) |
                      (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)b);
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %3\n\t"
      "global_load_lds_dwordx4 %1, %2\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(off), "s"(bu), "s"(__builtin_amdgcn_readfirstlane(lds))
      : "memory");
}

// Workgroup shape of the score kernel, by the bytes of a key row (HI heads of 64 elements):
// NW waves of 32 queries share every key tile (a key tile read from L2 serves NW * 32
// queries). Rows of <= 512 bytes (16-bit HI <= 4, fp32 HI <= 2) keep the register file
// within 256 per lane, so 8 waves (two per SIMD) fit one workgroup; 1 KB rows (16-bit
// HI = 8, fp32 HI = 4: 128 registers of stationary query operands) need 4.
template <int ROW_BYTES>
struct ScoreShape {
  // keys per LDS stage (and split interleave granule): two 32-key tiles between barriers
  // (one for 1 KB rows), so that two stage buffers and the score staging below fit the LDS.
  static constexpr int BN = ROW_BYTES <= 512 ? 64 : 32;
  static constexpr int NW = ROW_BYTES <= 512 ? 8 : 4;
  static constexpr int BM = NW * kQW;        // queries per workgroup
  static constexpr int THREADS = NW * 64;
  static constexpr int MIN_WAVES_PER_EU = ROW_BYTES <= 512 ? 2 : 1;
};
template <typename E, int HI>
constexpr int row_bytes() {
  return HI * kDI * ElemBytes<E>::value;
}

// The products are transposed: per tile of 32 keys a wave forms S^T = K Q^T (A = key rows
// from LDS, B = its 32 query rows, stationary in VGPRs), so lane l holds query l % 32 and
// the 16 keys 8(r/4) + 4(l/32) + r%4 of the tile in accumulator element r: four groups of
// four consecutive keys. Every element of a lane belongs to one query: its threshold is
// one register, its gates are four broadcast LDS reads per head, and its candidates go to
// its own list with no exchange between lanes. The two lanes of a query (l and l ^ 32)
// hold disjoint keys and append to two lists of their own.
constexpr int kStageRow = 36;  // two tiles of 16 scores per lane, padded

template <typename E, int HI, bool SAMPLE, int BIAS>
__global__ __launch_bounds__((ScoreShape<row_bytes<E, HI>()>::THREADS),
                             (ScoreShape<row_bytes<E, HI>()>::MIN_WAVES_PER_EU)) void indexer_score_kernel(const ScoreParams p) {
  constexpr int ROW_BYTES = row_bytes<E, HI>();
  using Shape = ScoreShape<ROW_BYTES>;
  constexpr int NW = Shape::NW;
  constexpr int BM = Shape::BM;
  constexpr int THREADS = Shape::THREADS;
  constexpr bool F32 = ElemBytes<E>::value == 4;
  constexpr int HEAD_BYTES = kDI * ElemBytes<E>::value;
  constexpr int HC = HEAD_BYTES / 32;                 // 16-byte chunks per head and lane half
  constexpr int CHUNKS = ROW_BYTES / 16;              // 16-byte chunks per key row (>= 8)
  constexpr int BN = Shape::BN;
  constexpr int TILE_BYTES = BN * ROW_BYTES;
  constexpr int LOADS = TILE_BYTES / (THREADS * 16);  // direct loads per thread per stage
  constexpr int WVALS = BN * HI;
  constexpr int WLOADS = (WVALS + THREADS - 1) / THREADS;
  static_assert(LOADS * THREADS * 16 == TILE_BYTES, "key tile must split evenly over the threads");

  // Two stage buffers (the next stage is loaded into one while the other is read).
  __shared__ __attribute__((aligned(16))) uint8_t ktile0[TILE_BYTES];
  __shared__ __attribute__((aligned(16))) uint8_t ktile1[TILE_BYTES];
  __shared__ __attribute__((aligned(16))) float wtile0[HI * BN];  // [head][key], gate * scale
  __shared__ __attribute__((aligned(16))) float wtile1[HI * BN];
  // FILTER: each wave's scores of the current stage, [lane][kStageRow floats]: element r of
  // tile t at 16 t + r (rows padded by 4 floats against bank conflicts of the 16-byte stores).
  __shared__ __attribute__((aligned(16))) float sstage[SAMPLE ? 1 : NW][SAMPLE ? 1 : 64 * kStageRow];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int b = blockIdx.z;
  // Key splits: split sp sweeps stages sp, sp + nsplit, ... (SAMPLE: of the sample keys).
  const int split = (int)blockIdx.y;
  const int nsplit = p.nsplit;
  const int q0 = blockIdx.x * BM + wave * kQW;
  const int T = p.T, S = p.S;
  const int nkeys = SAMPLE ? p.Ms : S;
  const int col = lane & 31;
  const int half = lane >> 5;
  const int row = q0 + col;  // this lane's query (SAMPLE with rows: its position in the list)
  int nrow = T;
  if constexpr (SAMPLE) {
    if (p.rows != nullptr) {
      nrow = min(p.nrows[b], p.rows_cap);
      if ((int)blockIdx.x * BM >= nrow) return;  // the whole workgroup, before any barrier
    }
  }
  const bool row_ok = row < nrow;
  int64_t grow = (int64_t)b * T + (row_ok ? row : 0);
  int64_t out_row = grow;  // SAMPLE: row of samp
  if constexpr (SAMPLE) {
    if (p.rows != nullptr) {
      grow = row_ok ? (int64_t)p.rows[(int64_t)b * T + row] : (int64_t)b * T;
      out_row = (int64_t)b * p.rows_cap + row;
    }
  }
  // kBiasView: the view-bias table row of this lane's query (element offset).
  int64_t vrow = 0;
  if constexpr ((BIAS & kBiasView) != 0) vrow = ((int64_t)b * p.Vq + clamp_view(p.qview[grow], p.Vq)) * p.Vs;

  // B operands: this lane's query row; chunk 2 m + half (16 bytes) of each head for step m.
  // 16-bit: one k = 16 product per chunk (k-chunk lane / 32 of the step); fp32: four k = 2
  // products per chunk, its element i with element i of the partner lane's chunk (the
  // products' k indices pair dims 8m + i and 8m + 4 + i, every dim once).
  uint4 qop[HI][HC];
  {
    const char* qr = static_cast<const char*>(p.q) + grow * ROW_BYTES + half * 16;
#pragma unroll
    for (int h = 0; h < HI; ++h)
#pragma unroll
      for (int m = 0; m < HC; ++m)
        qop[h][m] = row_ok ? *reinterpret_cast<const uint4*>(qr + h * HEAD_BYTES + m * 32) : make_uint4(0, 0, 0, 0);
  }
  // Threshold of this lane's query (rows past T never pass).
  float tau_l = INFINITY;
  if (row_ok) {
    if (p.tau_mode == kTauPlusInf) tau_l = INFINITY;
    else if (p.tau_mode == kTauMinusInf || p.tau == nullptr) tau_l = -INFINITY;
    else tau_l = p.tau[grow];
  }
  // FILTER: the list of this lane's query for this split is list grow * nsplit + split,
  // kSubTotal / nsplit slots long; the two lanes of a query (l and l ^ 32) append to it
  // stage by stage, so both keep the same byte cursor woff. The wave's 32 rows have consecutive list
  // blocks, so a list is addressed as a byte offset (< 2 MB) from the wave's first list.
  const int stride = SAMPLE ? 0 : kSubTotal / nsplit;
  int2* const lbase = SAMPLE ? nullptr : p.cand + (((int64_t)b * T + q0) * nsplit + split) * stride;
  const uint32_t wstart = (uint32_t)(col * nsplit * stride) * 8u;
  const uint32_t wend = wstart + (uint32_t)p.cap * 8u;  // first byte past the list's slots
  uint32_t woff = wstart;

  // Loader geometry: load i of this thread fills LDS bytes [(i*NW + wave)*1024 + 16*lane, +16),
  // which hold physical chunk lane % CHUNKS of key row kl0 + i*RPI; its source is logical
  // chunk (lane % CHUNKS) ^ (row & SWZ). kl0 < RPI and RPI is a power of two, so
  // (row & SWZ) differs from (kl0 & SWZ) by the constant XOR (i*RPI) & SWZ.
  constexpr int SWZ = CHUNKS >= 16 ? 15 : 7;
  constexpr int RPW = 1024 / ROW_BYTES;  // key rows per 1 KB wave chunk
  constexpr int RPI = NW * RPW;          // key rows per load step
  const int kl0 = wave * RPW + (lane * 16) / ROW_BYTES;
  const int lc0 = (lane % CHUNKS) ^ (kl0 & SWZ);
  auto voff = [&](int i) { return (uint32_t)(kl0 * ROW_BYTES + (lc0 ^ ((i * RPI) & SWZ)) * 16); };
  uint32_t voffs[LOADS];  // byte offset of load i from the stage's first key row
#pragma unroll
  for (int i = 0; i < LOADS; ++i) voffs[i] = (uint32_t)(i * (NW * 1024)) + voff(i);
  // Operand read offsets. 16-bit: key row (nb*32 + col), logical chunk h*8 + 2*ks + half,
  // physical chunk (h*8 + 2*ks + half) ^ (col & SWZ) = 8*(h ^ c3) + ((2*ks + half) ^ (col & 7))
  // with c3 = bit 3 of col when SWZ = 15: head h sits at 128*h + 128*c3 (h even) or
  // 128*h - 128*c3 (h odd), so the head part stays an immediate offset. fp32: logical chunk
  // h*16 + 2*m + half, physical h*16 + ((2*m + half) ^ (col & 15)) (SWZ = 15): head h at 256*h.
  const int c3 = (!F32 && SWZ == 15) ? ((col >> 3) & 1) : 0;
  uint32_t rd_even[HC], rd_odd[HC];
#pragma unroll
  for (int ks = 0; ks < HC; ++ks) {
    if constexpr (F32) {
      static_assert(SWZ == 15, "fp32 rows hold >= 16 chunks");
      rd_even[ks] = rd_odd[ks] = col * ROW_BYTES + 16 * ((2 * ks + half) ^ (col & 15));
    } else {
      const uint32_t base = col * ROW_BYTES + 16 * ((2 * ks + half) ^ (col & 7));
      rd_even[ks] = base + 128 * c3;
      rd_odd[ks] = base - 128 * c3;
    }
  }

  // Gate values travel as raw 16-bit patterns until wstore converts them at the end of the
  // stage: converting at load time would make the wave wait (vmcnt) for the key tile
  // loads issued just before. Keys past the end: K rows are loaded from the last valid key
  // (harmless), and the gate is NaN (FILTER: the mark clears keys past the end)
  // or 0 (SAMPLE: not stored).
  constexpr uint32_t kNoGate = 0xFFFFFFFFu;
  uint32_t wraw[WLOADS];
  auto gload = [&](int kb, uint8_t* ktile) {
    const int live = min(BN, nkeys - kb);
    if (!SAMPLE && live == BN) {
      // Full stage of consecutive keys: uniform base + lane offset + i * NW KB.
      const char* kbase = static_cast<const char*>(p.k) + ((int64_t)b * S + kb) * ROW_BYTES;
#pragma unroll
      for (int i = 0; i < LOADS; ++i) lds_dma16_s(kbase, voffs[i], &ktile[(i * NW + wave) * 1024]);
    } else {
      // Sample keys or the last stage: rows past the end re-read the last valid key.
#pragma unroll
      for (int i = 0; i < LOADS; ++i) {
        const int kl = min(kl0 + i * RPI, live - 1);
        const int key = sweep_key<SAMPLE>(kb + kl, p);
        const int lc = lc0 ^ ((i * RPI) & SWZ);
        const char* src = static_cast<const char*>(p.k) + ((int64_t)b * S + key) * ROW_BYTES + lc * 16;
        lds_dma16(src, &ktile[(i * NW + wave) * 1024]);
      }
    }
#pragma unroll
    for (int i = 0; i < WLOADS; ++i) {
      const int c = tid + THREADS * i;
      const int kl = c / HI, h = c % HI;
      uint32_t wv = kNoGate;
      if (c < WVALS && kl < live) {
        const int key = sweep_key<SAMPLE>(kb + kl, p);
        wv = raw_bits(E{}, p.w, ((int64_t)b * S + key) * HI + h);
      }
      wraw[i] = wv;
    }
  };
  auto wstore = [&](float* wtile) {
#pragma unroll
    for (int i = 0; i < WLOADS; ++i) {
      const int c = tid + THREADS * i;
      if (c < WVALS) {
        const float wv = wraw[i] == kNoGate ? (SAMPLE ? 0.f : __builtin_nanf(""))
                                            : to_f32(E{}, wraw[i]) * p.scale;
        wtile[(c % HI) * BN + c / HI] = wv;
      }
    }
  };

  int st = split;
  if (st < p.nstages) {
    gload(st * BN, ktile0);
    wstore(wtile0);
  }
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the direct LDS loads have landed
  __syncthreads();

  // Scores of this lane's 16 keys of the tile at kb + nb*32 (+ mask); SAMPLE stores them.
  // Key of element r: k4 + 8(r/4) + r%4 with k4 = kb + nb*32 + 4*half.
  auto tile_scores = [&](float (&s)[16], int kb, int nb, const uint8_t* ktile, const float* wtile) {
    const uint8_t* tile = &ktile[nb * 32 * ROW_BYTES];
#pragma unroll
    for (int r = 0; r < 16; ++r) s[r] = 0.f;
    // Head h's products are issued before head h - 1's gate epilogue, and the scheduler may
    // not hoist them further: two accumulators live at a time, not HI.
    auto products = [&](int h) {
      f32x16 acc = f32x16{0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < HC; ++ks) {
        if constexpr (F32) {
          const uint4 kop = *reinterpret_cast<const uint4*>(tile + rd_even[ks] + h * HEAD_BYTES);
          acc = mfma32_f32(kop.x, qop[h][ks].x, acc);
          acc = mfma32_f32(kop.y, qop[h][ks].y, acc);
          acc = mfma32_f32(kop.z, qop[h][ks].z, acc);
          acc = mfma32_f32(kop.w, qop[h][ks].w, acc);
        } else {
          const uint4 kop = *reinterpret_cast<const uint4*>(tile + ((h & 1) ? rd_odd[ks] : rd_even[ks]) + h * 128);
          acc = mfma32(E{}, kop, qop[h][ks], acc);
        }
      }
      return acc;
    };
    auto gate = [&](int h, const f32x16& acc) {
      const float* wg = &wtile[h * BN + nb * 32 + 4 * half];
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const float4 w4 = *reinterpret_cast<const float4*>(wg + 8 * g);
        s[4 * g + 0] = fmaf(w4.x, relu_bits(acc[4 * g + 0]), s[4 * g + 0]);
        s[4 * g + 1] = fmaf(w4.y, relu_bits(acc[4 * g + 1]), s[4 * g + 1]);
        s[4 * g + 2] = fmaf(w4.z, relu_bits(acc[4 * g + 2]), s[4 * g + 2]);
        s[4 * g + 3] = fmaf(w4.w, relu_bits(acc[4 * g + 3]), s[4 * g + 3]);
      }
    };
    f32x16 acc_prev = products(0);
#pragma unroll
    for (int h = 1; h < HI; ++h) {
      const f32x16 acc = products(h);
      gate(h - 1, acc_prev);
      __builtin_amdgcn_sched_barrier(0);
      acc_prev = acc;
    }
    gate(HI - 1, acc_prev);
    const int k4 = kb + nb * 32 + 4 * half;
    if constexpr ((BIAS & kBiasMask) != 0) {
      if (row_ok) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int kidx = k4 + 8 * (r >> 2) + (r & 3);
          if (kidx < nkeys) s[r] += ld_f32(E{}, p.mask, grow * S + sweep_key<SAMPLE>(kidx, p));
        }
      }
    }
    if constexpr ((BIAS & kBiasView) != 0) {
      if (row_ok) {
        const int* sv = p.sview + (int64_t)b * S;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int kidx = k4 + 8 * (r >> 2) + (r & 3);
          if (kidx < nkeys) s[r] += ld_f32(E{}, p.vbias, vrow + clamp_view(sv[sweep_key<SAMPLE>(kidx, p)], p.Vs));
        }
      }
    }
    if constexpr (SAMPLE) {
      if (row_ok) {
        float* dst = p.samp + out_row * p.Ms;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int kidx = k4 + 8 * g;
          if (kidx + 3 < nkeys) {
            *reinterpret_cast<float4*>(dst + kidx) = make_float4(s[4 * g], s[4 * g + 1], s[4 * g + 2], s[4 * g + 3]);
          } else {
#pragma unroll
            for (int i = 0; i < 4; ++i)
              if (kidx + i < nkeys) dst[kidx + i] = s[4 * g + i];
          }
        }
      }
    }
  };
  // FILTER candidates. Per element the lane only compares: bit (16 t + r) of pmask marks
  // element r of tile t of the stage, whose score the lane has put in its staging row.
  // After the stage barrier one loop writes the stage's candidates: each round every lane
  // takes its lowest marked element (iterations: the most any lane holds, about 4 where a
  // lane holds 1.2 on average), so a stage issues a few mostly full stores instead of 16
  // mostly empty ones per tile. The two lanes of a query write adjacent slots in a round.
  constexpr int NT = BN / 32;  // tiles per stage
  static_assert(NT * 16 + 4 <= kStageRow, "staging row too short");
  float* const stg = &sstage[wave][lane * kStageRow];
  uint32_t pmask = 0;  // marked elements of the pending stage
  int kb_pend = 0;     // its first key + 4 half (this lane's key base)
  char* const lbytes = reinterpret_cast<char*>(lbase);
  // An element passes when score > tau: bit r = sign bit of tau - score, appended by
  // v_alignbit_b32 (two instructions per element). Keys past the end (NaN scores) are
  // cleared explicitly in the last stage.
  auto mark = [&](const float (&sv)[16], int t, int kb) {
#pragma unroll
    for (int g = 0; g < 4; ++g)
      *reinterpret_cast<float4*>(stg + 16 * t + 4 * g) = make_float4(sv[4 * g], sv[4 * g + 1], sv[4 * g + 2], sv[4 * g + 3]);
    uint32_t tb = 0;
#pragma unroll
    for (int r = 15; r >= 0; --r) tb = __builtin_amdgcn_alignbit(tb, __float_as_uint(tau_l - sv[r]), 31);
    if (kb + BN > S) {
      const int k4 = kb + 32 * t + 4 * half;
#pragma unroll
      for (int r = 0; r < 16; ++r)
        if (k4 + 8 * (r >> 2) + (r & 3) >= S) tb &= ~(1u << r);
    }
    pmask |= tb << (16 * t);
  };
  // Element idx = 16 t + r of the stage holds key 32 t + 8 (r / 4) + r % 4 + 4 half past the
  // stage's first key: idx + (idx & ~3) + 4 half. The stage's entries of a query follow its
  // list in one block: lane l (half 0) first, then lane l ^ 32, each in element order, so a
  // lane needs only its partner's count (one lane swap per stage) and writes its own entries
  // to consecutive slots; four per round, so that their LDS reads share one wait.
  auto flush = [&]() {
    uint32_t mm = pmask;
    pmask = 0;
    const uint32_t cnt = (uint32_t)__builtin_popcount(mm);
    const auto sw = __builtin_amdgcn_permlane32_swap(cnt, cnt, false, false);
    const uint32_t other = sw[0] ^ sw[1] ^ cnt;  // the partner lane's count
    uint32_t pos = woff + (half ? 8u * other : 0u);
    woff += 8u * (cnt + other);
    while (__ballot(mm != 0u) != 0ull) {
      uint32_t idx[4], has[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        has[u] = mm != 0u ? 1u : 0u;
        idx[u] = has[u] ? (uint32_t)__builtin_ctz(mm) : 0u;
        mm &= mm - 1u;
      }
      float sv[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) sv[u] = stg[idx[u]];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        if (has[u] && pos < wend)
          *reinterpret_cast<int2*>(lbytes + pos) =
              make_int2(__float_as_int(sv[u]), kb_pend + (int)(idx[u] + (idx[u] & ~3u)));
        pos += 8u * has[u];
      }
    }
  };

  // One stage on buffer (kt, wt), prefetching the next stage into (kn, wn).
  const bool OFFSET_GROUP = wave >= NW / 2;
  auto stage = [&](const uint8_t* kt, const float* wt, uint8_t* kn, float* wn) {
    const int kb = st * BN;
    const bool more = st + nsplit < p.nstages;
    if (more) gload((st + nsplit) * BN, kn);
    // The previous stage's candidates are written here, after its stage-end vmcnt(0) +
    // barrier: vmcnt counts stores as well as the direct LDS loads it waits for, so the
    // stores are followed by a stage of MFMA work before that wait.
    if constexpr (SAMPLE) {
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        float s0[16];
        tile_scores(s0, kb, t, kt, wt);
      }
    } else if (OFFSET_GROUP) {
      // The other wave of each SIMD starts with the first tile's products and writes the
      // previous stage's candidates after them, so the two waves of a SIMD leave the barrier
      // out of phase (one on the matrix cores while the other issues the writes).
      float s0[16];
      tile_scores(s0, kb, 0, kt, wt);
      flush();
      mark(s0, 0, kb);
#pragma unroll
      for (int t = 1; t < NT; ++t) {
        float s1[16];
        tile_scores(s1, kb, t, kt, wt);
        mark(s1, t, kb);
      }
    } else {
      flush();
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        float s0[16];
        tile_scores(s0, kb, t, kt, wt);
        mark(s0, t, kb);
      }
    }
    kb_pend = kb + 4 * half;

    // Keep the gate conversion (which waits for this stage's loads) after the tile work.
    __builtin_amdgcn_sched_barrier(0);
    if (more) wstore(wn);
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): next stage's direct LDS loads have landed
    __syncthreads();
    st += nsplit;
  };
  uint8_t* kt = ktile0;
  uint8_t* kn = ktile1;
  float* wt = wtile0;
  float* wn = wtile1;
  while (st < p.nstages) {
    stage(kt, wt, kn, wn);
    uint8_t* const kx = kt;
    kt = kn;
    kn = kx;
    float* const wx = wt;
    wt = wn;
    wn = wx;
  }
  if constexpr (!SAMPLE) {
    flush();
    // entries of the list (both lanes hold the same count); above cap: overflowed
    if (row_ok && half == 0) p.counts[grow * nsplit + split] = (int)((woff - wstart) >> 3);
  }
}

// ---------------------------------------------------------------------------------------
// Threshold from the sample scores: one wave per query row.
// ---------------------------------------------------------------------------------------
template <int MPL>
__global__ __launch_bounds__(256) void indexer_tau_kernel(const float* samp, int Ms, int rank, int slack,
                                                          float* tau, int64_t rows) {
  __shared__ uint32_t cbuf[4][kCompactKeys];
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;  // whole wave; no barriers below
  const float* src = samp + row * Ms;
  uint32_t kv[MPL];
  uint32_t lmin = 0xFFFFFFFFu, lmax = 0u;
#pragma unroll
  for (int m = 0; m < MPL; ++m) {
    kv[m] = f2key(src[lane + 64 * m]);
    lmin = min(lmin, kv[m]);
    lmax = max(lmax, kv[m]);
  }
  // Invariant: count(key >= lo) >= rank and count(key >= hi) < rank.
  const uint64_t lo = wave_min_u(lmin);
  const uint64_t hi = (uint64_t)wave_max_u(lmax) + 1;
  const uint32_t t = wave_bisect_keys<MPL>(kv, MPL, lo, hi, 64 * MPL, 0, rank, slack, cbuf[threadIdx.x >> 6]);
  if (lane == 0) tau[row] = key2f(t);
}

// ---------------------------------------------------------------------------------------
// Exact top-k among the candidates: one wave per query row, candidates in registers.
//
// The row's lists (one per key split) are read as one sequence: entry e of the sequence
// goes to register slot e / 64 of lane e % 64, for up to 64 * KS entries (about 1.7 x topk
// are expected; KS is the smallest of kSelRegsTiers whose slots hold 1.25 x the expected
// count plus five Poisson deviations, e.g. 48 for topk = 1024 and 64 for 2048 at S = 32). A row
// with an overflowed list or fewer than topk candidates goes to the exact fallback; one with
// more candidates than the registers hold goes to the LDS selection. No barriers:
// reductions are wave-wide.
// ---------------------------------------------------------------------------------------
constexpr int kSelRegsTiers[3] = {48, 64, 96};
static_assert(kSelRegsTiers[0] % 8 == 0 && kSelRegsTiers[1] % 8 == 0 && kSelRegsTiers[2] % 8 == 0,
              "the select kernel moves register slots in chunks of 8");

struct SelectParams {
  const int2* cand;
  const int* counts;
  int nlist, cap, stride;
  int32_t* out_idx;
  void* out_scores;  // [rows, Kk] in the element type of the launch
  int Kk;
  int T;
  int* fb_count;  // [B]: rows queued for the exact fallback, per batch element
  int* fb_list;   // [B * T]: batch element b's rows from fb_list[b * T]
  int* wide_count;
  int* wide_list;
  int64_t rows;
  int force_wide;  // test hook: every complete row takes the LDS selection
};

// Number of set bits of a wave mask below this lane.
__device__ __forceinline__ int lanes_below(uint64_t m) {
  return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

// Row lists as one sequence: off[l] = entries of the lists before list l (uniform);
// entry e sits at cand + (row * nlist + l) * stride + (e - off[l]) for the list l holding it.
struct RowLists {
  int64_t base;  // row * nlist * stride
  int off[kMaxLists + 1];
  int adj[kMaxLists];  // stride - (entries of list l - 1): the gap skipped past list l's start
  int nlist, stride;
  // The lists' entries lie within nlist * stride <= kSubTotal slots of the row: 32-bit
  // offsets, one compare and select per list start at or below e.
  __device__ __forceinline__ int64_t at(int e) const {
    int a = e;
#pragma unroll
    for (int s2 = 1; s2 < kMaxLists; ++s2)
      if (s2 < nlist) a += e >= off[s2] ? adj[s2] : 0;
    return base + a;
  }
};

__device__ __forceinline__ bool row_lists(const SelectParams& p, int64_t row, RowLists& rl) {
  rl.base = row * p.nlist * (int64_t)p.stride;
  rl.nlist = p.nlist;
  rl.stride = p.stride;
  bool bad = false;
  int acc = 0;
#pragma unroll
  for (int s2 = 0; s2 < kMaxLists; ++s2) {
    rl.off[s2] = acc;
    rl.adj[s2] = 0;
    if (s2 < p.nlist) {
      const int c = __builtin_amdgcn_readfirstlane(p.counts[row * p.nlist + s2]);  // row is wave-uniform
      bad |= c > p.cap;
      acc += min(c, p.cap);
    }
  }
  rl.off[kMaxLists] = acc;
#pragma unroll
  for (int s2 = 1; s2 < kMaxLists; ++s2) rl.adj[s2] = p.stride - (rl.off[s2] - rl.off[s2 - 1]);
  return bad;
}

template <typename E, int KS>
__global__ __launch_bounds__(256) void indexer_select_kernel(const SelectParams p) {
  __shared__ uint32_t cbuf[4][kCompactKeys];
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (row >= p.rows) return;
  RowLists rl;
  const bool bad = row_lists(p, row, rl);
  const int total = rl.off[kMaxLists];
  if (bad || total < p.Kk) {
    // The candidates may miss part of the top-k: exact brute force.
    if (lane == 0) {
      const int bb = (int)(row / p.T);
      p.fb_list[(int64_t)bb * p.T + atomicAdd(&p.fb_count[bb], 1)] = (int)row;
    }
    return;
  }
  if (p.force_wide || total > 64 * KS) {
    // Complete candidates, more than the registers hold: the LDS selection.
    if (lane == 0) p.wide_list[atomicAdd(p.wide_count, 1)] = (int)row;
    return;
  }
  const int nch = (total + 63) / 64;  // register slots in use, uniform

  // Slots past the end hold key 0, below the key of every finite score; chunks of 8 slots
  // past the last one in use are skipped with a uniform branch.
  // Each slot's key (order-preserving score bits) and key index stay in registers for the
  // output, so the list position of an entry is computed once.
  // All loads are issued before any is used (the score bits land in kv and become keys in a
  // second pass), so the chunks of 8 slots do not wait for each other.
  uint32_t kv[KS];
  int32_t ky[KS];
  uint32_t lmin = 0xFFFFFFFFu, lmax = 0u;
#pragma unroll
  for (int m0 = 0; m0 < KS; m0 += 8) {
#pragma unroll
    for (int m = m0; m < m0 + 8; ++m) {
      kv[m] = 0u;
      ky[m] = 0;
    }
    if (m0 < nch) {
#pragma unroll
      for (int m = m0; m < m0 + 8; ++m) {
        const int e = m * 64 + lane;
        if (e < total) {
          const int2 cdt = p.cand[rl.at(e)];
          kv[m] = (uint32_t)cdt.x;
          ky[m] = cdt.y;
        }
      }
    }
  }
#pragma unroll
  for (int m0 = 0; m0 < KS; m0 += 8) {
    if (m0 < nch) {
#pragma unroll
      for (int m = m0; m < m0 + 8; ++m)
        if (m * 64 + lane < total) kv[m] = f2key(__uint_as_float(kv[m]));
    }
  }
  // Key range of the live slots: empty slots hold 0, which kv - 1 wraps to the maximum (the
  // + 1 comes after the wave minimum, so a lane without live slots does not wrap back to 0).
  // Candidates passed a >= comparison and are never NaN, so no live key is 0.
#pragma unroll
  for (int m = 0; m < KS; ++m) {
    lmin = min(lmin, kv[m] - 1u);
    lmax = max(lmax, kv[m]);
  }
  // Bisection on the key value: count(key >= lo) = total >= Kk > count(key >= hi) = 0.
  const uint64_t lo = (uint64_t)wave_min_u(lmin) + 1, hi = (uint64_t)wave_max_u(lmax) + 1;
  const uint32_t thr = wave_bisect_keys<KS>(kv, nch, lo, hi, total, 0, p.Kk, 0, cbuf[threadIdx.x >> 6]);
  // Elements > thr are all selected; of those == thr, the first (Kk - count(> thr)) in
  // candidate order (split, position). Output positions come from wave ballots, so each
  // write goes to base + (selected lanes below this one).
  int n_gt = 0;
#pragma unroll
  for (int m0 = 0; m0 < KS; m0 += 8) {
    if (m0 < nch) {
#pragma unroll
      for (int m = m0; m < m0 + 8; ++m) n_gt += __popcll(__ballot(kv[m] > thr));
    }
  }
  const int need_eq = p.Kk - n_gt;
  int32_t* oi = p.out_idx + row * p.Kk;
  const int64_t os = row * p.Kk;
  int base = 0, eq_run = 0;
#pragma unroll
  for (int m0 = 0; m0 < KS; m0 += 8) {
    if (m0 < nch) {
#pragma unroll
      for (int m = m0; m < m0 + 8; ++m) {
        const bool eq = kv[m] == thr;
        const uint64_t eqm = __ballot(eq);
        const int eq_before = eq_run + lanes_below(eqm);
        eq_run += __popcll(eqm);
        const bool sel = kv[m] > thr || (eq && eq_before < need_eq);
        const uint64_t selm = __ballot(sel);
        const int slot_out = base + lanes_below(selm);
        base += __popcll(selm);
        if (sel) {
          oi[slot_out] = ky[m];
          st_f32(E{}, p.out_scores, os + slot_out, key2f(kv[m]));
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------------------
// Exact top-k of rows whose (complete) candidates exceed the register path: all of the
// row's candidates in LDS, block radix select. Persistent grid over the queue.
// ---------------------------------------------------------------------------------------
template <typename E>
__global__ __launch_bounds__(256) void indexer_select_wide_kernel(const SelectParams p) {
  __shared__ uint32_t keys[kSubTotal];
  __shared__ int vals[kSubTotal];
  __shared__ SelectShared sh;
  const int tid = threadIdx.x;
  const int nitems = *((volatile const int*)p.wide_count);
  for (int item = blockIdx.x; item < nitems; item += gridDim.x) {
    const int64_t row = p.wide_list[item];
    RowLists rl;
    row_lists(p, row, rl);
    const int total = rl.off[kMaxLists];
    for (int s2 = 0; s2 < p.nlist; ++s2) {
      const int2* src = p.cand + rl.base + (int64_t)s2 * p.stride;
      const int o = rl.off[s2], n = rl.off[s2 + 1] - o;
      for (int i = tid; i < n; i += kSelThreads) {
        const int2 e = src[i];
        keys[o + i] = f2key(__int_as_float(e.x));
        vals[o + i] = e.y;
      }
    }
    __syncthreads();
    int take_eq;
    auto key_at = [&](int i) { return keys[i]; };
    const uint32_t kth = block_radix_select(key_at, total, p.Kk, sh, take_eq);
    int32_t* oi = p.out_idx + row * p.Kk;
    const int64_t os = row * p.Kk;
    block_emit_topk(key_at, total, p.Kk, kth, take_eq,
                    [&](int slot, int i) {
                      if (slot < p.Kk) {
                        oi[slot] = vals[i];
                        st_f32(E{}, p.out_scores, os + slot, key2f(keys[i]));
                      }
                    },
                    sh);
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------------------
// Exact brute force for queued queries.
// ---------------------------------------------------------------------------------------
struct FallbackParams {
  const void* q;
  const void* k;
  const void* w;
  const void* mask;
  const void* vbias;
  const int* qview;
  const int* sview;
  int Vq, Vs;
  const int* fb_count;  // [B]
  const int* fb_list;   // [B * T], batch element b's rows from b * T
  // Scores of the first rows_cap queued rows of each batch element, computed on the matrix
  // cores by indexer_score_kernel<SAMPLE> over all keys: [B, rows_cap, S] (null: none).
  const float* full;
  int rows_cap;
  float* scratch;  // [gridDim.x, S]: rows beyond rows_cap are scored here
  int32_t* out_idx;
  void* out_scores;
  int B, T, S, Kk;
  float scale;
};

// Dot product of two 16-byte chunks accumulated onto z: 8 x 16-bit elements (dot2 pairs)
// or 4 x fp32.
__device__ __forceinline__ float dot_chunk(BF16, uint4 a, uint4 b, float z) {
  z = dot2(BF16{}, a.x, b.x, z);
  z = dot2(BF16{}, a.y, b.y, z);
  z = dot2(BF16{}, a.z, b.z, z);
  return dot2(BF16{}, a.w, b.w, z);
}
__device__ __forceinline__ float dot_chunk(FP16, uint4 a, uint4 b, float z) {
  z = dot2(FP16{}, a.x, b.x, z);
  z = dot2(FP16{}, a.y, b.y, z);
  z = dot2(FP16{}, a.z, b.z, z);
  return dot2(FP16{}, a.w, b.w, z);
}
__device__ __forceinline__ float dot_chunk(FP32, uint4 a, uint4 b, float z) {
  z = fmaf(__uint_as_float(a.x), __uint_as_float(b.x), z);
  z = fmaf(__uint_as_float(a.y), __uint_as_float(b.y), z);
  z = fmaf(__uint_as_float(a.z), __uint_as_float(b.z), z);
  return fmaf(__uint_as_float(a.w), __uint_as_float(b.w), z);
}

template <typename E, int HI, int BIAS>
__global__ __launch_bounds__(256) void indexer_fallback_kernel(const FallbackParams p) {
  constexpr int ROW_BYTES = row_bytes<E, HI>();
  constexpr int HEAD_CHUNKS = kDI * ElemBytes<E>::value / 16;
  __shared__ __attribute__((aligned(16))) uint4 qs[ROW_BYTES / 16];
  __shared__ SelectShared sh;
  const int tid = threadIdx.x;
  float* const own = p.scratch + (int64_t)blockIdx.x * p.S;
  // Exact top-k of one row's scores sc[0, S).
  auto select_row = [&](const float* sc, int row) {
    int take_eq;
    auto key_at = [&](int i) { return f2key(sc[i]); };
    const uint32_t kth = block_radix_select(key_at, p.S, p.Kk, sh, take_eq);
    int32_t* oi = p.out_idx + (int64_t)row * p.Kk;
    const int64_t os = (int64_t)row * p.Kk;
    block_emit_topk(key_at, p.S, p.Kk, kth, take_eq,
                    [&](int slot, int i) {
                      if (slot < p.Kk) {
                        oi[slot] = i;
                        st_f32(E{}, p.out_scores, os + slot, sc[i]);
                      }
                    },
                    sh);
    __syncthreads();
  };
  // Rows below rows_cap have their scores computed on the matrix cores and are selected by
  // indexer_full_select_kernel; this kernel scores and selects the rest.
  const int first = p.full != nullptr ? p.rows_cap : 0;
  for (int b = 0; b < p.B; ++b) {
    const int nitems = *((volatile const int*)(p.fb_count + b));
    for (int item = first + blockIdx.x; item < nitems; item += gridDim.x) {
      const int row = p.fb_list[(int64_t)b * p.T + item];
      const uint4* qrow = reinterpret_cast<const uint4*>(static_cast<const char*>(p.q) + (int64_t)row * ROW_BYTES);
      for (int i = tid; i < ROW_BYTES / 16; i += kSelThreads) qs[i] = qrow[i];
      __syncthreads();
      for (int j = tid; j < p.S; j += kSelThreads) {
        const uint4* kr =
            reinterpret_cast<const uint4*>(static_cast<const char*>(p.k) + ((int64_t)b * p.S + j) * ROW_BYTES);
        float s = 0.f;
#pragma unroll
        for (int h = 0; h < HI; ++h) {
          float z = 0.f;
#pragma unroll
          for (int c = 0; c < HEAD_CHUNKS; ++c) z = dot_chunk(E{}, qs[h * HEAD_CHUNKS + c], kr[h * HEAD_CHUNKS + c], z);
          const float wv = ld_f32(E{}, p.w, ((int64_t)b * p.S + j) * HI + h) * p.scale;
          s = fmaf(wv, relu_bits(z), s);
        }
        if constexpr ((BIAS & kBiasMask) != 0) s += ld_f32(E{}, p.mask, (int64_t)row * p.S + j);
        if constexpr ((BIAS & kBiasView) != 0)
          s += ld_f32(E{}, p.vbias,
                      ((int64_t)b * p.Vq + clamp_view(p.qview[row], p.Vq)) * p.Vs +
                          clamp_view(p.sview[(int64_t)b * p.S + j], p.Vs));
        own[j] = s;
      }
      __threadfence_block();
      __syncthreads();
      select_row(own, row);
    }
  }
}

// ---------------------------------------------------------------------------------------
// Exact top-k of queued rows whose scores the matrix cores computed (full[b, j, :] for the
// first rows_cap queued rows of batch element b). Per row, on the order-preserving keys:
//  1. the row's smallest and largest key;
//  2. a 2048-bin histogram over the key range [lo, hi] (bins of 2^sh keys from the top)
//     finds the bin of the k-th largest key; while that bin holds more keys than the LDS
//     buffer and is wider than one key, the range narrows to it and step 2 repeats (at most
//     three times: each level takes 11 bits);
//  3. keys above the range go straight out and the range's keys are gathered into LDS, both
//     in a fixed order (round, thread, key of the thread); a block radix select settles the
//     rest (a one-key range with more keys than the buffer: its first keys in that order).
// Ties at the k-th value are taken in that fixed order, the same on every run. Every pass
// reads the row in rounds of kFullPer keys per thread (key r0 + m * 256 + thread: coalesced
// loads, issued together).
// ---------------------------------------------------------------------------------------
constexpr int kFullBins = 2048;
constexpr int kFullEqCap = 4096;
constexpr int kFullPer = 64;  // contiguous keys per thread and round

template <typename E>
__global__ __launch_bounds__(256) void indexer_full_select_kernel(const FallbackParams p) {
  __shared__ int hist[kFullBins];
  __shared__ uint32_t ekeys[kFullEqCap];
  __shared__ int eidx[kFullEqCap];
  __shared__ SelectShared sh;
  __shared__ uint32_t bcast[4][2];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int Kk = p.Kk, S = p.S;
  constexpr int ROUND = kFullPer * kSelThreads;
  // Key m of this thread in round r0: r0 + m * 256 + tid (coalesced loads).
  auto load_round = [&](const float* sc, int r0, uint32_t (&kv)[kFullPer]) {
    const int i0 = r0 + tid;
    float v[kFullPer];
#pragma unroll
    for (int m = 0; m < kFullPer; ++m) v[m] = i0 + m * kSelThreads < S ? sc[i0 + m * kSelThreads] : 0.f;
#pragma unroll
    for (int m = 0; m < kFullPer; ++m) kv[m] = f2key(v[m]);
    return i0;
  };
  for (int b = 0; b < p.B; ++b) {
    const int nitems = min(*((volatile const int*)(p.fb_count + b)), p.rows_cap);
    for (int item = blockIdx.x; item < nitems; item += gridDim.x) {
      const int row = p.fb_list[(int64_t)b * p.T + item];
      const float* sc = p.full + ((int64_t)b * p.rows_cap + item) * S;
      int32_t* oi = p.out_idx + (int64_t)row * Kk;
      const int64_t os = (int64_t)row * Kk;
      // 1. key range of the row
      uint32_t kmin = 0xFFFFFFFFu, kmax = 0u;
      for (int r0 = 0; r0 < S; r0 += ROUND) {
        uint32_t kv[kFullPer];
        const int i0 = load_round(sc, r0, kv);
#pragma unroll
        for (int m = 0; m < kFullPer; ++m)
          if (i0 + m * kSelThreads < S) {
            kmin = min(kmin, kv[m]);
            kmax = max(kmax, kv[m]);
          }
      }
#pragma unroll
      for (int off = 32; off > 0; off >>= 1) {
        kmin = min(kmin, (uint32_t)__shfl_xor((int)kmin, off));
        kmax = max(kmax, (uint32_t)__shfl_xor((int)kmax, off));
      }
      if (lane == 0) {
        bcast[wave][0] = kmin;
        bcast[wave][1] = kmax;
      }
      __syncthreads();
      uint32_t lo = min(min(bcast[0][0], bcast[1][0]), min(bcast[2][0], bcast[3][0]));
      uint32_t hi = max(max(bcast[0][1], bcast[1][1]), max(bcast[2][1], bcast[3][1]));
      __syncthreads();
      // 2. narrow [lo, hi] to the k-th key's bin
      int above = 0, need = Kk, cnt = 0;
      for (int level = 0; level < 3; ++level) {
        const uint32_t span = hi - lo;
        const int shb = span < (uint32_t)kFullBins ? 0 : 32 - __builtin_clz(span) - 11;
        for (int i = tid; i < kFullBins; i += kSelThreads) hist[i] = 0;
        __syncthreads();
        for (int r0 = 0; r0 < S; r0 += ROUND) {
          uint32_t kv[kFullPer];
          const int i0 = load_round(sc, r0, kv);
#pragma unroll
          for (int m = 0; m < kFullPer; ++m)
            if (i0 + m * kSelThreads < S && kv[m] - lo <= span) atomicAdd(&hist[(hi - kv[m]) >> shb], 1);
        }
        __syncthreads();
        // bins 8 t .. 8 t + 7 per thread: thread order is descending key order
        int c[8], local = 0;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          c[j] = hist[8 * tid + j];
          local += c[j];
        }
        int ex, ex_unused;
        block_excl_scan2(local, 0, ex, ex_unused, sh);
        if (ex < need && need <= ex + local) {
          int acc = ex;
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            if (acc + c[j] >= need) {
              sh.bcast[0] = 8 * tid + j;
              sh.bcast[1] = acc;
              break;
            }
            acc += c[j];
          }
        }
        __syncthreads();
        const int d = sh.bcast[0];
        above += sh.bcast[1];
        need -= sh.bcast[1];
        cnt = hist[d];
        const uint32_t nhi = hi - ((uint32_t)d << shb);
        const uint32_t width = shb >= 32 ? 0xFFFFFFFFu : ((1u << shb) - 1u);
        lo = max(lo, nhi - min(width, nhi));
        hi = nhi;
        __syncthreads();
        if (cnt <= kFullEqCap || shb == 0) break;
      }
      // 3. keys above hi out, keys in [lo, hi] to LDS (or, for a one-key range too large for
      // the buffer, its first need keys out), in index order
      const bool gather = cnt <= kFullEqCap;
      int base_g = 0, base_e = 0;
      for (int r0 = 0; r0 < S; r0 += ROUND) {
        uint32_t kv[kFullPer];
        const int i0 = load_round(sc, r0, kv);
        int cg = 0, ce = 0;
#pragma unroll
        for (int m = 0; m < kFullPer; ++m) {
          const bool ok = i0 + m * kSelThreads < S;
          cg += ok && kv[m] > hi;
          ce += ok && kv[m] >= lo && kv[m] <= hi;
        }
        int og, oe;
        block_excl_scan2(cg, ce, og, oe, sh);
        og += base_g;
        oe += base_e;
#pragma unroll
        for (int m = 0; m < kFullPer; ++m) {
          if (i0 + m * kSelThreads >= S) continue;
          if (kv[m] > hi) {
            oi[og] = i0 + m * kSelThreads;
            st_f32(E{}, p.out_scores, os + og, key2f(kv[m]));
            ++og;
          } else if (kv[m] >= lo) {
            if (gather) {
              ekeys[oe] = kv[m];
              eidx[oe] = i0 + m * kSelThreads;
            } else if (oe < need) {
              oi[above + oe] = i0 + m * kSelThreads;
              st_f32(E{}, p.out_scores, os + above + oe, key2f(kv[m]));
            }
            ++oe;
          }
        }
        if (tid == kSelThreads - 1) {
          bcast[0][0] = (uint32_t)og;  // block totals so far (the last thread ends at them)
          bcast[0][1] = (uint32_t)oe;
        }
        __syncthreads();
        base_g = (int)bcast[0][0];
        base_e = (int)bcast[0][1];
        __syncthreads();
      }
      if (gather) {
        int take_eq;
        auto ekey_at = [&](int i) { return ekeys[i]; };
        const uint32_t kth = block_radix_select(ekey_at, cnt, need, sh, take_eq);
        block_emit_topk(ekey_at, cnt, need, kth, take_eq,
                        [&](int slot, int i) {
                          if (slot < need) {
                            oi[above + slot] = eidx[i];
                            st_f32(E{}, p.out_scores, os + above + slot, key2f(ekeys[i]));
                          }
                        },
                        sh);
      }
      __syncthreads();
    }
  }
}

__global__ void set_ints_kernel(int* ptr, int n, int value) {
  for (int i = threadIdx.x; i < n; i += blockDim.x) ptr[i] = value;
}

__global__ void iota_kernel(int* ptr, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    ptr[i] = (int)i;
}


// ---------------------------------------------------------------------------------------
// Host-side plan.
// ---------------------------------------------------------------------------------------
size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

struct Plan {
  int Kk = 0;
  bool sample = false;
  bool full_all = false;  // every row through the full scoring and the row select
  int full_rows = 0;      // rows per batch element scored per round on the full path
  int Ms = 0, rank = 0;
  int nsplit = 1, cap = 0;
  size_t off_tau = 0, off_samp = 0, off_counts = 0, off_cand = 0, off_fb = 0, off_fblist = 0,
         off_widelist = 0, off_scratch = 0, off_full = 0, total = 0;
};

// Workspace layout (independent of the split count, which depends on the device).
Plan make_layout(int64_t B, int64_t T, int64_t S, int64_t topk) {
  Plan pl;
  pl.Kk = (int)(topk < S ? topk : S);
  pl.sample = S > kSubTotal / 2;
  if (pl.sample) {
    pl.Ms = (int)(S >= 65536 ? 4096 : 2048);
    const double lam = (double)pl.Kk * pl.Ms / (double)S;
    int r = (int)ceil(lam + 4.5 * sqrt(lam) + 2.0);
    pl.rank = r > pl.Ms ? pl.Ms : r;
    // Expected candidates per query (rank of Ms samples, scaled to S keys) beyond 3/4 of
    // the candidate slots: the lists would overflow for many rows, so every row takes the
    // full path instead.
    pl.full_all = (double)pl.rank * (double)S / (double)pl.Ms > 0.75 * kSubTotal;
  }
  // Full-path rounds: kFullRows rows per batch element for the queued rows of the usual
  // path; when every row takes it, up to 4 x as many (fewer, fuller rounds) while their
  // scores stay within 512 MiB.
  pl.full_rows = kFullRows;
  if (pl.full_all) {
    const int64_t fit = ((int64_t)512 << 20) / ((int64_t)B * S * 4);
    pl.full_rows = (int)std::max<int64_t>(kFullRows, std::min<int64_t>(4 * kFullRows, fit / kFullRows * kFullRows));
  }
  const size_t rows = (size_t)B * (size_t)T;
  size_t off = 0;
  pl.off_tau = off;      off = align_up(off + rows * 4, 256);
  pl.off_samp = off;     off = align_up(off + (pl.sample ? rows * (size_t)pl.Ms * 4 : 0), 256);
  pl.off_counts = off;   off = align_up(off + rows * kMaxLists * 4, 256);
  pl.off_cand = off;     off = align_up(off + rows * (size_t)kSubTotal * 8, 256);
  pl.off_fb = off;       off = align_up(off + (size_t)(B + 1) * 4, 256);  // wide count, then B fallback counts
  pl.off_fblist = off;   off = align_up(off + rows * 4, 256);
  pl.off_widelist = off; off = align_up(off + rows * 4, 256);
  pl.off_scratch = off;  off = align_up(off + (size_t)kFallbackBlocks * (size_t)S * 4, 256);
  pl.off_full = off;     off = align_up(off + (size_t)B * pl.full_rows * (size_t)S * 4, 256);
  pl.total = off;
  return pl;
}

// Concurrent workgroups of a filter kernel instance on the current device (cached per
// device and kernel).
int filter_slots(const void* kernel, int threads) {
  struct Entry {
    const void* kernel;
    int dev, slots;
  };
  static Entry cache[64];
  static int n_cache = 0;
  static std::mutex mu;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 512;
  {
    std::lock_guard<std::mutex> lock(mu);
    for (int i = 0; i < n_cache; ++i)
      if (cache[i].kernel == kernel && cache[i].dev == dev) return cache[i].slots;
  }
  int cus = 0, per_cu = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, threads, 0) != hipSuccess || per_cu <= 0)
    per_cu = 1;
  const int slots = cus * per_cu;
  std::lock_guard<std::mutex> lock(mu);
  if (n_cache < 64) cache[n_cache++] = Entry{kernel, dev, slots};
  return slots;
}

// Picks the key split count: the fraction of the last wave of workgroups that is busy,
// highest first, fewer splits on ties; each split keeps >= 8 stages of 64 keys.
int choose_nsplit(int64_t tiles, int64_t S, int slots, bool sample, int bn) {
  if (!sample) return 1;
  int best = 1;
  double best_eff = -1.0;
  for (int ns = 1; ns <= kMaxSplit; ++ns) {
    if (ns > 1 && S / (ns * (int64_t)bn) < 8) break;
    const double waves = (double)(tiles * ns) / slots;
    const double eff = waves / ceil(waves);
    if (eff > best_eff + 1e-9) {
      best_eff = eff;
      best = ns;
    }
  }
  return best;
}

// Launch configuration of indexer_score_kernel<SAMPLE> over every key for up to rows_cap
// queued rows per batch element (rows and their count set by the caller).
template <typename E, int HI, int BIAS>
ScoreParams full_rows_params(const ScoreParams& base, float* full, int rows_cap) {
  using Shape = ScoreShape<row_bytes<E, HI>()>;
  ScoreParams fp2 = base;
  fp2.samp = full;
  fp2.Ms = base.S;
  fp2.rows_cap = rows_cap;
  fp2.tau = nullptr;
  fp2.tau_mode = kTauArray;
  fp2.nstages = (base.S + Shape::BN - 1) / Shape::BN;
  return fp2;
}

// A top-k whose expected candidates would overflow the lists (Plan::full_all): every row is
// scored over every key on the matrix cores and selected exactly by
// indexer_full_select_kernel, in rounds of Plan::full_rows rows per batch element (round r0
// takes rows r0 .. r0 + full_rows - 1 of each batch element through a queue that lists
// every row).
template <typename E, int HI, int BIAS>
int run_full_rows(const ScoreParams& base, const Plan& pl, int64_t B, int32_t* out_idx, void* out_scores,
                  uint8_t* ws, hipStream_t st) {
  using Shape = ScoreShape<row_bytes<E, HI>()>;
  constexpr int BM = Shape::BM;
  constexpr int THREADS = Shape::THREADS;
  const int64_t rows = B * (int64_t)base.T;
  int* counts = reinterpret_cast<int*>(ws + pl.off_fb) + 1;  // [B]: rows left from the round's first
  int* list = reinterpret_cast<int*>(ws + pl.off_fblist);    // [B * T]: row i = i
  float* full = reinterpret_cast<float*>(ws + pl.off_full);
  hipLaunchKernelGGL(iota_kernel, dim3((unsigned)std::min<int64_t>((rows + 255) / 256, 4096)), dim3(256), 0, st,
                     list, rows);
  GW_HIP_LAUNCH_CHECK("iota_kernel");
  const int nr = pl.full_rows;
  ScoreParams fp2 = full_rows_params<E, HI, BIAS>(base, full, nr);
  fp2.nrows = counts;
  const int ftiles = (nr + BM - 1) / BM;
  const int fslots = filter_slots((const void*)indexer_score_kernel<E, HI, true, BIAS>, THREADS);
  const int64_t want = (2 * (int64_t)fslots + (int64_t)ftiles * B - 1) / ((int64_t)ftiles * B);
  fp2.nsplit = (int)std::max<int64_t>(1, std::min<int64_t>(want, std::max(1, fp2.nstages / 2)));
  FallbackParams bp{};
  bp.fb_count = counts;
  bp.full = full;
  bp.rows_cap = nr;
  bp.B = (int)B;
  bp.out_idx = out_idx;
  bp.out_scores = out_scores;
  bp.T = base.T;
  bp.S = base.S;
  bp.Kk = pl.Kk;
  bp.scale = base.scale;
  for (int r0 = 0; r0 < base.T; r0 += nr) {
    hipLaunchKernelGGL(set_ints_kernel, dim3(1), dim3(256), 0, st, counts, (int)B, base.T - r0);
    GW_HIP_LAUNCH_CHECK("set_ints_kernel");
    fp2.rows = list + r0;
    hipLaunchKernelGGL((indexer_score_kernel<E, HI, true, BIAS>),
                       dim3((unsigned)ftiles, (unsigned)fp2.nsplit, (unsigned)B), dim3(THREADS), 0, st, fp2);
    GW_HIP_LAUNCH_CHECK("indexer_score_kernel<full rows>");
    bp.fb_list = list + r0;
    hipLaunchKernelGGL((indexer_full_select_kernel<E>), dim3(2 * kFallbackBlocks), dim3(256), 0, st, bp);
    GW_HIP_LAUNCH_CHECK("indexer_full_select_kernel");
  }
  return GW_OK;
}

template <typename E, int HI, int BIAS>
int run_typed(const ScoreParams& base, Plan pl, int64_t B, int32_t* out_idx, void* out_scores,
              uint8_t* ws, hipStream_t st) {
  if (pl.full_all) return run_full_rows<E, HI, BIAS>(base, pl, B, out_idx, out_scores, ws, st);
  int* counters = reinterpret_cast<int*>(ws + pl.off_fb);  // [0] wide select, [1 + b] fallback of b
  hipLaunchKernelGGL(set_ints_kernel, dim3(1), dim3(256), 0, st, counters, (int)B + 1, 0);
  GW_HIP_LAUNCH_CHECK("set_ints_kernel");
  using Shape = ScoreShape<row_bytes<E, HI>()>;
  constexpr int BM = Shape::BM;
  constexpr int THREADS = Shape::THREADS;
  constexpr int BN = Shape::BN;
  const int64_t tiles = (base.T + BM - 1) / BM;
  const int64_t rows = B * (int64_t)base.T;
  pl.nsplit = choose_nsplit(tiles * B, base.S, filter_slots((const void*)indexer_score_kernel<E, HI, false, BIAS>, THREADS),
                            pl.sample, BN);
  const int stride = kSubTotal / pl.nsplit;
  pl.cap = stride;
  float* tau = reinterpret_cast<float*>(ws + pl.off_tau);
  if (pl.sample) {
    ScoreParams sp = base;
    sp.samp = reinterpret_cast<float*>(ws + pl.off_samp);
    sp.Ms = pl.Ms;
    sp.tau = nullptr;
    sp.tau_mode = kTauArray;
    // The sample keys split over workgroups too: one workgroup per query tile would leave
    // most of the chip idle.
    sp.nsplit = choose_nsplit(tiles * B, pl.Ms, filter_slots((const void*)indexer_score_kernel<E, HI, true, BIAS>, THREADS),
                              true, BN);
    sp.nstages = (pl.Ms + BN - 1) / BN;
    hipLaunchKernelGGL((indexer_score_kernel<E, HI, true, BIAS>),
                       dim3((unsigned)tiles, (unsigned)sp.nsplit, (unsigned)B), dim3(THREADS), 0, st, sp);
    GW_HIP_LAUNCH_CHECK("indexer_score_kernel<sample>");
    const dim3 tgrid((unsigned)((rows + 3) / 4));
    if (pl.Ms == 4096)
      hipLaunchKernelGGL((indexer_tau_kernel<64>), tgrid, dim3(256), 0, st, sp.samp, pl.Ms, pl.rank, 8, tau, rows);
    else
      hipLaunchKernelGGL((indexer_tau_kernel<32>), tgrid, dim3(256), 0, st, sp.samp, pl.Ms, pl.rank, 8, tau, rows);
    GW_HIP_LAUNCH_CHECK("indexer_tau_kernel");
  }
  ScoreParams fp = base;
  fp.tau = pl.sample ? tau : nullptr;
  fp.cand = reinterpret_cast<int2*>(ws + pl.off_cand);
  fp.counts = reinterpret_cast<int*>(ws + pl.off_counts);
  fp.nsplit = pl.nsplit;
  fp.cap = pl.cap;
  fp.nstages = (base.S + BN - 1) / BN;
  hipLaunchKernelGGL((indexer_score_kernel<E, HI, false, BIAS>),
                     dim3((unsigned)tiles, (unsigned)pl.nsplit, (unsigned)B), dim3(THREADS), 0, st, fp);
  GW_HIP_LAUNCH_CHECK("indexer_score_kernel<filter>");
  SelectParams fs{};
  fs.cand = fp.cand;
  fs.counts = fp.counts;
  fs.nlist = pl.nsplit;
  fs.cap = pl.cap;
  fs.stride = stride;
  fs.out_idx = out_idx;
  fs.out_scores = out_scores;
  fs.Kk = pl.Kk;
  fs.T = base.T;
  fs.fb_count = counters + 1;
  fs.fb_list = reinterpret_cast<int*>(ws + pl.off_fblist);
  fs.wide_count = counters;
  fs.wide_list = reinterpret_cast<int*>(ws + pl.off_widelist);
  fs.rows = rows;
  fs.force_wide = base.force_wide;
  const dim3 sgrid2((unsigned)((rows + 3) / 4));
  // Register slots: the fewest that hold 1.25 x the expected candidates per query plus five
  // Poisson deviations (the largest tier when none does: rows beyond it take the LDS
  // selection). Real rows spread wider than Poisson: for topk = 1024 at S = 32 (1,880
  // candidates on average) 32 slots sent so many rows to the LDS selection that the call
  // took 2.87 instead of 2.12 ms.
  const double expect = pl.sample ? (double)pl.rank * (double)base.S / (double)pl.Ms : (double)base.S;
  const double need = 1.25 * expect + 5.0 * std::sqrt(expect);
  if (need <= 64.0 * kSelRegsTiers[0])
    hipLaunchKernelGGL((indexer_select_kernel<E, kSelRegsTiers[0]>), sgrid2, dim3(256), 0, st, fs);
  else if (need <= 64.0 * kSelRegsTiers[1])
    hipLaunchKernelGGL((indexer_select_kernel<E, kSelRegsTiers[1]>), sgrid2, dim3(256), 0, st, fs);
  else
    hipLaunchKernelGGL((indexer_select_kernel<E, kSelRegsTiers[2]>), sgrid2, dim3(256), 0, st, fs);
  GW_HIP_LAUNCH_CHECK("indexer_select_kernel");
  hipLaunchKernelGGL((indexer_select_wide_kernel<E>), dim3(kFallbackBlocks), dim3(256), 0, st, fs);
  GW_HIP_LAUNCH_CHECK("indexer_select_wide_kernel");
  // Rows queued for the exact fallback (sampled threshold too high or a list overflowed):
  // scores over all keys on the matrix cores, rows gathered from the queue, key range split
  // finely so that a few hundred rows still fill the chip (workgroups of batch elements with
  // fewer queued rows return at once).
  float* full = reinterpret_cast<float*>(ws + pl.off_full);
  {
    ScoreParams fp2 = full_rows_params<E, HI, BIAS>(base, full, kFullRows);
    fp2.rows = fs.fb_list;
    fp2.nrows = fs.fb_count;
    const int ftiles = (kFullRows + BM - 1) / BM;
    const int fslots = filter_slots((const void*)indexer_score_kernel<E, HI, true, BIAS>, THREADS);
    const int64_t want = (2 * (int64_t)fslots + (int64_t)ftiles * B - 1) / ((int64_t)ftiles * B);
    fp2.nsplit = (int)std::max<int64_t>(1, std::min<int64_t>(want, std::max(1, fp2.nstages / 2)));
    hipLaunchKernelGGL((indexer_score_kernel<E, HI, true, BIAS>),
                       dim3((unsigned)ftiles, (unsigned)fp2.nsplit, (unsigned)B), dim3(THREADS), 0, st, fp2);
    GW_HIP_LAUNCH_CHECK("indexer_score_kernel<fallback rows>");
  }
  FallbackParams bp{};
  bp.q = base.q;
  bp.k = base.k;
  bp.w = base.w;
  bp.mask = base.mask;
  bp.vbias = base.vbias;
  bp.qview = base.qview;
  bp.sview = base.sview;
  bp.Vq = base.Vq;
  bp.Vs = base.Vs;
  bp.fb_count = fs.fb_count;
  bp.fb_list = fs.fb_list;
  bp.full = full;
  bp.rows_cap = kFullRows;
  bp.B = (int)B;
  bp.scratch = reinterpret_cast<float*>(ws + pl.off_scratch);
  bp.out_idx = out_idx;
  bp.out_scores = fs.out_scores;
  bp.T = base.T;
  bp.S = base.S;
  bp.Kk = pl.Kk;
  bp.scale = base.scale;
  hipLaunchKernelGGL((indexer_full_select_kernel<E>), dim3(2 * kFallbackBlocks), dim3(256), 0, st, bp);
  GW_HIP_LAUNCH_CHECK("indexer_full_select_kernel");
  hipLaunchKernelGGL((indexer_fallback_kernel<E, HI, BIAS>), dim3(kFallbackBlocks), dim3(256), 0, st, bp);
  GW_HIP_LAUNCH_CHECK("indexer_fallback_kernel");
  return GW_OK;
}

template <typename E, int BIAS>
int dispatch_hi(int hi, const ScoreParams& base, const Plan& pl, int64_t B, int32_t* out_idx,
                void* out_scores, uint8_t* ws, hipStream_t st) {
  switch (hi) {
    case 1: return run_typed<E, 1, BIAS>(base, pl, B, out_idx, out_scores, ws, st);
    case 2: return run_typed<E, 2, BIAS>(base, pl, B, out_idx, out_scores, ws, st);
    case 4: return run_typed<E, 4, BIAS>(base, pl, B, out_idx, out_scores, ws, st);
    default:
      // fp32 rows of 8 heads would need 256 registers of stationary query operands.
      if constexpr (ElemBytes<E>::value == 4)
        return set_error(GW_ERR_UNSUPPORTED, "fp32 indexer inputs support 1, 2 or 4 heads, got %d", hi);
      else
        return run_typed<E, 8, BIAS>(base, pl, B, out_idx, out_scores, ws, st);
  }
}

}  // namespace
}  // namespace gw

extern "C" size_t gw_indexer_topk_workspace_size(int64_t B, int64_t T, int64_t S, int64_t topk) {
  if (B <= 0 || T <= 0 || S <= 0 || topk <= 0) return 0;
  return gw::make_layout(B, T, S, topk).total;
}

namespace gw {
namespace {

int indexer_topk_impl(int dtype, const void* q, const void* k, const void* w, const void* mask,
                      const void* view_bias, const int32_t* q_view_ids, const int32_t* s_view_ids, int64_t Vq,
                      int64_t Vs, int64_t B, int64_t T, int64_t S, int64_t Hi, int64_t Di, int64_t topk,
                      float softmax_scale, int flags, int32_t* out_indices, void* out_scores, void* workspace,
                      size_t workspace_bytes, void* stream) {
  GW_CHECK_ARG(dtype == GW_DTYPE_BF16 || dtype == GW_DTYPE_FP16 || dtype == GW_DTYPE_FP32, "unsupported dtype code %d",
               dtype);
  GW_CHECK_ARG(B >= 0 && T >= 0 && S >= 0 && topk >= 1, "invalid sizes B=%lld T=%lld S=%lld topk=%lld",
               (long long)B, (long long)T, (long long)S, (long long)topk);
  if (Di != kDI || !(Hi == 1 || Hi == 2 || Hi == 4 || Hi == 8))
    return set_error(GW_ERR_UNSUPPORTED, "indexer heads x dim %lld x %lld not supported (1/2/4/8 x 64)",
                     (long long)Hi, (long long)Di);
  if (dtype == GW_DTYPE_FP32 && Hi == 8)
    return set_error(GW_ERR_UNSUPPORTED, "fp32 indexer inputs support 1, 2 or 4 heads, got %lld", (long long)Hi);
  GW_CHECK_ARG(softmax_scale > 0.f, "softmax_scale must be positive, got %g", (double)softmax_scale);
  GW_CHECK_ARG((flags & ~7) == 0 && (flags & 3) != 3, "invalid flags %d", flags);
  const bool has_view = view_bias != nullptr;
  if (has_view)
    GW_CHECK_ARG(q_view_ids && s_view_ids && Vq >= 1 && Vs >= 1 && Vq * Vs < (1ll << 30),
                 "view bias needs q/s view ids and a [B, Vq, Vs] table (Vq=%lld Vs=%lld)", (long long)Vq,
                 (long long)Vs);
  if (B == 0 || T == 0) return GW_OK;
  GW_CHECK_ARG(S >= 1, "empty key set");
  const int64_t Kk = topk < S ? topk : S;
  GW_CHECK_ARG(q && k && w && out_indices && out_scores, "null tensor pointer");
  GW_CHECK_ARG(aligned16(q) && aligned16(k), "q and k must be 16-byte aligned");
  GW_CHECK_ARG(B <= 65535 && T < (1ll << 30) && B * T < (1ll << 30), "size exceeds grid or int32 range");
  // A sublist's byte cursor advances 8 KB per append and must stay below 2^32.
  if (S > (1ll << 24))
    return set_error(GW_ERR_UNSUPPORTED, "S=%lld exceeds the supported maximum %lld", (long long)S, 1ll << 24);
  const Plan pl = make_layout(B, T, S, topk);
  GW_CHECK_ARG(workspace != nullptr && workspace_bytes >= pl.total, "workspace needs %zu bytes, got %zu",
               pl.total, workspace_bytes);
  GW_CHECK_ARG(gw::aligned16(workspace), "workspace must be 16-byte aligned");

  ScoreParams base{};
  base.q = q;
  base.k = k;
  base.w = w;
  base.mask = mask;
  base.vbias = view_bias;
  base.qview = q_view_ids;
  base.sview = s_view_ids;
  base.Vq = (int)Vq;
  base.Vs = (int)Vs;
  base.T = (int)T;
  base.S = (int)S;
  base.scale = softmax_scale;
  base.tau_mode = (flags & GW_TOPK_FLAG_TAU_PLUS_INF) ? kTauPlusInf
                  : (flags & GW_TOPK_FLAG_TAU_MINUS_INF) ? kTauMinusInf
                                                         : kTauArray;
  base.force_wide = (flags & GW_TOPK_FLAG_FORCE_WIDE) ? 1 : 0;
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int bias = (mask != nullptr ? kBiasMask : 0) | (has_view ? kBiasView : 0);
  const int hi = (int)Hi;
  if (dtype == GW_DTYPE_BF16) {
    switch (bias) {
      case 0: return dispatch_hi<BF16, 0>(hi, base, pl, B, out_indices, out_scores, ws, st);
      case kBiasMask: return dispatch_hi<BF16, kBiasMask>(hi, base, pl, B, out_indices, out_scores, ws, st);
      case kBiasView: return dispatch_hi<BF16, kBiasView>(hi, base, pl, B, out_indices, out_scores, ws, st);
      default: return dispatch_hi<BF16, kBiasMask | kBiasView>(hi, base, pl, B, out_indices, out_scores, ws, st);
    }
  }
  if (dtype == GW_DTYPE_FP32) {
    switch (bias) {
      case 0: return dispatch_hi<FP32, 0>(hi, base, pl, B, out_indices, out_scores, ws, st);
      case kBiasMask: return dispatch_hi<FP32, kBiasMask>(hi, base, pl, B, out_indices, out_scores, ws, st);
      case kBiasView: return dispatch_hi<FP32, kBiasView>(hi, base, pl, B, out_indices, out_scores, ws, st);
      default: return dispatch_hi<FP32, kBiasMask | kBiasView>(hi, base, pl, B, out_indices, out_scores, ws, st);
    }
  }
  switch (bias) {
    case 0: return dispatch_hi<FP16, 0>(hi, base, pl, B, out_indices, out_scores, ws, st);
    case kBiasMask: return dispatch_hi<FP16, kBiasMask>(hi, base, pl, B, out_indices, out_scores, ws, st);
    case kBiasView: return dispatch_hi<FP16, kBiasView>(hi, base, pl, B, out_indices, out_scores, ws, st);
    default: return dispatch_hi<FP16, kBiasMask | kBiasView>(hi, base, pl, B, out_indices, out_scores, ws, st);
  }
}

}  // namespace
}  // namespace gw

extern "C" int gw_indexer_topk_fwd(int dtype, const void* q, const void* k, const void* w,
                                   const void* mask, int64_t B, int64_t T, int64_t S, int64_t Hi,
                                   int64_t Di, int64_t topk, float softmax_scale, int flags,
                                   int32_t* out_indices, void* out_scores, void* workspace,
                                   size_t workspace_bytes, void* stream) {
  gw::clear_error();
  return gw::indexer_topk_impl(dtype, q, k, w, mask, nullptr, nullptr, nullptr, 0, 0, B, T, S, Hi, Di, topk,
                               softmax_scale, flags, out_indices, out_scores, workspace, workspace_bytes, stream);
}

extern "C" int gw_indexer_topk_fwd_view_bias(int dtype, const void* q, const void* k, const void* w,
                                             const void* mask, const void* view_bias, const int32_t* q_view_ids,
                                             const int32_t* s_view_ids, int64_t Vq, int64_t Vs, int64_t B,
                                             int64_t T, int64_t S, int64_t Hi, int64_t Di, int64_t topk,
                                             float softmax_scale, int flags, int32_t* out_indices,
                                             void* out_scores, void* workspace, size_t workspace_bytes,
                                             void* stream) {
  gw::clear_error();
  GW_CHECK_ARG(view_bias != nullptr, "null view-bias table");
  return gw::indexer_topk_impl(dtype, q, k, w, mask, view_bias, q_view_ids, s_view_ids, Vq, Vs, B, T, S, Hi, Di,
                               topk, softmax_scale, flags, out_indices, out_scores, workspace, workspace_bytes,
                               stream);
}
