// Lightning-indexer score + exact per-query top-k for gfx950, without an N x N score
// matrix in memory.
//
//   score[b,t,s] = sum_h w[b,s,h] * relu(scale * <q[b,t,h], k[b,s,h]>)  (+ mask[b,t,s])
//
// (reference easyvolcap/official_vggt/layers/indexer.py:430-466 and
// easyvolcap/utils/custom_indexer/sparse_topk_indexer.py:935-951). scale > 0 lets the
// scale move onto the gate: w*relu(scale*z) = (scale*w)*relu(z).
//
// Pipeline (all on the caller's stream, no host synchronisation):
//  K0 score_kernel<SAMPLE>: MFMA scores of every query against Ms strided sample keys.
//  K0b tau_kernel:          one wave per query: a threshold tau whose rank among the
//                           sample scores lies in [r, r + 8], r chosen so that at least
//                           topk keys of the whole row score >= tau with very high
//                           probability (about 1.7 x topk keys on average).
//  K1 score_kernel<FILTER>: MFMA scores against all keys; the epilogue appends
//                           (score, key) pairs with score >= tau to the query's candidate
//                           list (one list per query and key split).
//  K2 select_kernel:        one wave per query: exact top-k of the candidates held in
//                           registers (bisection on the order-preserving score bits,
//                           ballot-ordered emit). A query whose lists overflowed or hold
//                           fewer than topk entries is queued for K3; one whose candidates
//                           exceed the register slots is queued for K2b.
//  K2b select_wide_kernel:  persistent workgroups: all candidates of a queued query in
//                           LDS, block radix select.
//  K3 fallback_kernel:      exact brute force for queued queries (scores to scratch, radix
//                           select) - correct for any input, used rarely.
// Exactness: if count(score >= tau) >= topk, every member of the top-k scores >= tau and
// is a candidate, so selecting among the candidates is exact. Ties at the k-th value are
// broken deterministically (candidate order: split, then position in the list).
//
// MFMA layout (v_mfma_f32_32x32x16_{bf16,f16}): C[32 queries x 32 keys]; A = q rows
// (stationary in VGPRs for the whole key sweep), B = key rows staged through LDS
// (XOR-swizzled 16-byte chunks, conflict-free operand reads). Lane l owns key column l%32
// and query rows 8*(r/4) + 4*(l/32) + r%4 of accumulator element r.
//
// Candidate appends: about 2 % of scores pass tau, so most accumulator elements have a
// passing lane somewhere in the wave and a store per element would issue a mostly empty
// memory instruction per element. Instead each wave compacts its passing entries into an
// LDS queue (a ballot and a lane count per element, one LDS write), and every 64 queued
// entries are written out by one full store: each lane takes one entry, ranks it among
// the lanes holding the same query row (ballots on the row bits) and writes it to that
// row's list after the entries already written. Everything is in a fixed order, so the
// lists are deterministic.
//
// Key splits: to fill the chip, the key range is divided over nsplit workgroups per
// query tile. Split sp takes the 64-key stages sp, sp + nsplit, sp + 2*nsplit, ...; the
// interleave spreads any locality of a query's favourite keys (e.g. its own view) evenly
// over the splits, so every list receives about (candidates / nsplit) entries.
#include <math.h>

#include <mutex>

#include "gw_common.h"
#include "gw_select.h"

namespace gw {
namespace {

constexpr int kQW = 32;            // queries per wave
constexpr int kBN = 64;            // keys per LDS stage (and split interleave granule)
constexpr int kDI = 64;            // indexer head dim
constexpr int kSubTotal = 8192;    // candidate slots per query over all key splits
constexpr int kMaxSplit = 8;
constexpr int kMaxTopk = 2048;
constexpr int kFallbackBlocks = 256;
// Candidate layout: int2 {score bits, key} lists cand[(row * nsplit + split) * cap + i],
// row = b * T + t, cap = kSubTotal / nsplit; counts[row * nsplit + split] = entries
// appended (more than cap means the list overflowed).

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

__device__ __forceinline__ float to_f32(BF16, uint16_t x) { return __uint_as_float((uint32_t)x << 16); }
__device__ __forceinline__ float to_f32(FP16, uint16_t x) {
  return (float)__builtin_bit_cast(_Float16, x);
}

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

enum TauMode { kTauArray = 0, kTauPlusInf = 1, kTauMinusInf = 2 };

struct ScoreParams {
  const uint16_t* q;     // [B, T, HI, 64]
  const uint16_t* k;     // [B, S, HI, 64]
  const uint16_t* w;     // [B, S, HI]
  const uint16_t* mask;  // [B, T, S] or null
  const float* tau;      // [B*T] or null (-inf)
  float* samp;           // SAMPLE: [B*T, Ms]
  int2* cand;            // FILTER: candidate lists, see kQueue
  int* counts;           // FILTER: [B*T, nsplit] appends per list (may exceed cap)
  int T, S;
  int nsplit, cap;
  int nstages;           // 64-key stages of the sweep
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
typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) void glb_void_t;

// Workgroup shape of the score kernel: NW waves of 32 queries share every key tile (a
// key tile read from L2 serves NW * 32 queries). HI <= 4 keeps its register file within
// 256 per lane, so 8 waves (two per SIMD) fit one workgroup; HI = 8 needs 4.
template <int HI>
struct ScoreShape {
  static constexpr int NW = HI <= 4 ? 8 : 4;
  static constexpr int BM = NW * kQW;        // queries per workgroup
  static constexpr int THREADS = NW * 64;
  static constexpr int MIN_WAVES_PER_EU = HI <= 4 ? 2 : 1;
  // Per-wave LDS candidate queue (entries): written out when it holds FLUSH entries at a
  // check after every 8 accumulator elements, so at most FLUSH - 1 + 8 * 64 < QUEUE are
  // ever queued.
  static constexpr int QUEUE = HI <= 4 ? 1024 : 640;
  static constexpr int FLUSH = HI <= 4 ? 256 : 128;
};

template <typename E, int HI, bool SAMPLE, bool HAS_MASK>
__global__ __launch_bounds__(ScoreShape<HI>::THREADS, ScoreShape<HI>::MIN_WAVES_PER_EU) void indexer_score_kernel(
    const ScoreParams p) {
  constexpr int NW = ScoreShape<HI>::NW;
  constexpr int BM = ScoreShape<HI>::BM;
  constexpr int THREADS = ScoreShape<HI>::THREADS;
  constexpr int ROW_BYTES = HI * kDI * 2;
  constexpr int CHUNKS = ROW_BYTES / 16;              // 16-byte chunks per key row (>= 8)
  constexpr int TILE_BYTES = kBN * ROW_BYTES;
  constexpr int LOADS = TILE_BYTES / (THREADS * 16);  // direct loads per thread per stage
  constexpr int WVALS = kBN * HI;
  constexpr int WLOADS = (WVALS + THREADS - 1) / THREADS;
  static_assert(LOADS * THREADS * 16 == TILE_BYTES, "key tile must split evenly over the threads");

  __shared__ __attribute__((aligned(16))) uint8_t ktile[2][TILE_BYTES];
  __shared__ float wtile[2][WVALS];
  __shared__ __attribute__((aligned(16))) float tau_s[BM];
  constexpr int QUEUE = ScoreShape<HI>::QUEUE;
  __shared__ int2 cq[SAMPLE ? 1 : NW][SAMPLE ? 1 : QUEUE];  // FILTER: per-wave candidate queue
  __shared__ int rcnt[SAMPLE ? 1 : NW][kQW];                 // FILTER: entries appended per row

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int b = blockIdx.z;
  const int split = SAMPLE ? 0 : (int)blockIdx.y;
  const int nsplit = SAMPLE ? 1 : p.nsplit;
  const int q0 = blockIdx.x * BM + wave * kQW;
  const int T = p.T, S = p.S;
  const int nkeys = SAMPLE ? p.Ms : S;
  const int col = lane & 31;
  const int half = lane >> 5;

  // A operands: this lane's query row (lane % 32), k-chunk (lane / 32) of each 16-wide step.
  uint4 a[HI][4];
  {
    const int row = q0 + col;
    const bool ok = row < T;
    const uint16_t* qr = p.q + ((int64_t)b * T + (ok ? row : 0)) * (HI * kDI) + half * 8;
#pragma unroll
    for (int h = 0; h < HI; ++h)
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
        a[h][ks] = ok ? *reinterpret_cast<const uint4*>(qr + h * kDI + ks * 16) : make_uint4(0, 0, 0, 0);
  }

  // Per-row thresholds of this wave's 32 rows (rows past T never pass).
  if (lane < kQW) {
    const int row = q0 + lane;
    float tv = INFINITY;
    if (row < T) {
      if (p.tau_mode == kTauPlusInf) tv = INFINITY;
      else if (p.tau_mode == kTauMinusInf || p.tau == nullptr) tv = -INFINITY;
      else tv = p.tau[(int64_t)b * T + row];
    }
    tau_s[wave * kQW + lane] = tv;
  }
  // FILTER: list of query row q0 + rr at cand + (((b * T + q0 + rr) * nsplit + split) * cap.
  const int64_t list0 = ((int64_t)b * T + q0) * nsplit + split;
  const uint32_t half_tag = (uint32_t)(4 * half) << 24;  // row bits of this lane's half
  uint32_t qn = 0;                                       // queued entries (wave-uniform)
  if constexpr (!SAMPLE) {
    if (lane < kQW) rcnt[wave][lane] = 0;
  }
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
  // Operand read offsets: key row (nb*32 + col), logical chunk h*8 + 2*ks + half, physical
  // chunk (h*8 + 2*ks + half) ^ (col & SWZ) = 8*(h ^ c3) + ((2*ks + half) ^ (col & 7)) with
  // c3 = bit 3 of col when SWZ = 15: head h sits at 128*h + 128*c3 (h even) or
  // 128*h - 128*c3 (h odd), so the head part stays an immediate offset.
  const int c3 = SWZ == 15 ? ((col >> 3) & 1) : 0;
  uint32_t rd_even[4], rd_odd[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    const uint32_t base = col * ROW_BYTES + 16 * ((2 * ks + half) ^ (col & 7));
    rd_even[ks] = base + 128 * c3;
    rd_odd[ks] = base - 128 * c3;
  }

  // Gate values travel as raw 16-bit patterns until wstore converts them at the end of the
  // stage: converting at load time would make the wave wait (vmcnt) for the key tile
  // loads issued just before. Keys past the end: K rows are loaded from the last valid key
  // (harmless), and the gate is NaN (FILTER: the score is NaN and fails every `>= tau`)
  // or 0 (SAMPLE: not stored).
  constexpr uint32_t kNoGate = 0xFFFFFFFFu;
  uint32_t wraw[WLOADS];
  auto gload = [&](int kb, int buf) {
    const int live = min(kBN, nkeys - kb);
    if (!SAMPLE && live == kBN) {
      // Full stage of consecutive keys: uniform base + lane offset + i * NW KB.
      const char* kbase = reinterpret_cast<const char*>(p.k + ((int64_t)b * S + kb) * (HI * kDI));
#pragma unroll
      for (int i = 0; i < LOADS; ++i) {
        const char* src = kbase + i * (NW * 1024) + voff(i);
        __builtin_amdgcn_global_load_lds((glb_void_t*)src, (lds_void_t*)(&ktile[buf][(i * NW + wave) * 1024]), 16, 0, 0);
      }
    } else {
      // Sample keys or the last stage: rows past the end re-read the last valid key.
#pragma unroll
      for (int i = 0; i < LOADS; ++i) {
        const int kl = min(kl0 + i * RPI, live - 1);
        const int key = sweep_key<SAMPLE>(kb + kl, p);
        const int lc = lc0 ^ ((i * RPI) & SWZ);
        const uint16_t* src = p.k + ((int64_t)b * S + key) * (HI * kDI) + lc * 8;
        __builtin_amdgcn_global_load_lds((glb_void_t*)src, (lds_void_t*)(&ktile[buf][(i * NW + wave) * 1024]), 16, 0, 0);
      }
    }
#pragma unroll
    for (int i = 0; i < WLOADS; ++i) {
      const int c = tid + THREADS * i;
      const int kl = c / HI, h = c % HI;
      uint32_t wv = kNoGate;
      if (c < WVALS && kl < live) {
        const int key = sweep_key<SAMPLE>(kb + kl, p);
        wv = p.w[((int64_t)b * S + key) * HI + h];
      }
      wraw[i] = wv;
    }
  };
  auto wstore = [&](int buf) {
#pragma unroll
    for (int i = 0; i < WLOADS; ++i) {
      if (tid + THREADS * i < WVALS) {
        const float wv = wraw[i] == kNoGate ? (SAMPLE ? 0.f : __builtin_nanf(""))
                                            : to_f32(E{}, (uint16_t)wraw[i]) * p.scale;
        wtile[buf][tid + THREADS * i] = wv;
      }
    }
  };

  int st = split;
  if (st < p.nstages) {
    gload(st * kBN, 0);
    wstore(0);
  }
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the direct LDS loads have landed
  __syncthreads();

  // Appends of one 32-key tile (FILTER). The second tile of a stage is appended one
  // iteration late, after the stage-end vmcnt(0) + barrier: vmcnt counts stores as well
  // as the direct LDS loads it waits for, so every store issued before that wait is
  // followed by at least one tile of MFMA work rather than waited on at once.
  float tau_r[16];  // thresholds of this lane's 16 rows (filled after the first barrier)
  // Writes the queued entries to their rows' lists: all of them (`all`) or every full
  // chunk of 64, moving the rest (< 64) to the front; qn is wave-uniform. Queue entries
  // are {score bits, key | row << 24}. A row's next slot comes from an LDS atomic on the
  // wave's own row counters: one instruction's lanes and successive instructions are
  // served in order, so the lists come out the same on every run. Up to four chunks go
  // per round, their LDS reads and atomics issued back to back.
  auto flush = [&](bool all) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const uint32_t full = all ? qn : (qn & ~63u);
    for (uint32_t h = 0; h < full; h += 256) {
      int2 e[4];
      int slot[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const uint32_t i = h + 64 * c + lane;
        e[c] = i < full ? cq[wave][i] : make_int2(0, -1);
      }
#pragma unroll
      for (int c = 0; c < 4; ++c)
        slot[c] = e[c].y != -1 ? atomicAdd(&rcnt[wave][((uint32_t)e[c].y >> 24) & 31u], 1) : p.cap;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        if (slot[c] < p.cap) {
          const uint32_t rr = ((uint32_t)e[c].y >> 24) & 31u;
          p.cand[(list0 + (int64_t)rr * nsplit) * p.cap + slot[c]] = make_int2(e[c].x, e[c].y & 0xFFFFFF);
        }
      }
    }
    const uint32_t rem = qn - full;
    if (rem > 0 && full > 0) {
      int2 mv = make_int2(0, 0);
      if ((uint32_t)lane < rem) mv = cq[wave][full + lane];
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      if ((uint32_t)lane < rem) cq[wave][lane] = mv;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    qn = rem;
  };
  // Queues the passing entries of a tile: a ballot, a count of the passing lanes below,
  // one LDS write; the queue is written out once it holds FLUSH entries (checked after
  // every 8 elements).
  auto append = [&](const float (&sv)[16], int key) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const bool pass = sv[r] >= tau_r[r];  // NaN (key past the end) never passes
      const uint64_t m = __ballot(pass);
      const uint32_t addr = (uint32_t)(uintptr_t)&cq[wave][0] + 8u * (qn + lanes_below_u(m));
      const uint32_t kt = (uint32_t)key | (half_tag + ((uint32_t)(8 * (r / 4) + (r % 4)) << 24));
      // The LDS write runs with exec = the passing lanes, set and restored inside one asm
      // statement, so there is no branch around it (a branch per accumulator element splits
      // the epilogue into small blocks). The compiler does not count this write in its
      // lgkmcnt waits; LDS operations of a wave complete in issue order, so an extra
      // operation can only make those waits stricter, never release one early.
      uint64_t saved;
      asm volatile(
          "s_and_saveexec_b64 %0, %1\n\t"
          "ds_write_b64 %2, %3\n\t"
          "s_or_b64 exec, exec, %0"
          : "=&s"(saved)
          : "s"(m), "v"(addr), "v"(make_uint2(__float_as_uint(sv[r]), kt))
          : "memory", "scc");
      qn += (uint32_t)__popcll(m);
      if ((r & 7) == 7 && qn >= (uint32_t)ScoreShape<HI>::FLUSH) flush(false);
    }
  };
  // Scores of the tile of 32 keys at kb + nb*32 (+ mask); SAMPLE stores them directly.
  auto tile_scores = [&](float (&s)[16], int kb, int nb, int buf) {
    const int kl = nb * 32 + col;
    const uint8_t* tile = &ktile[buf][nb * 32 * ROW_BYTES];
#pragma unroll
    for (int r = 0; r < 16; ++r) s[r] = 0.f;
#pragma unroll
    for (int h = 0; h < HI; ++h) {
      f32x16 acc = f32x16{0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const uint4 bop = *reinterpret_cast<const uint4*>(tile + ((h & 1) ? rd_odd[ks] : rd_even[ks]) + h * 128);
        acc = mfma32(E{}, a[h][ks], bop, acc);
      }
      const float wv = wtile[buf][kl * HI + h];
#pragma unroll
      for (int r = 0; r < 16; ++r) s[r] = fmaf(wv, relu_bits(acc[r]), s[r]);
    }
    const int kidx = kb + kl;
    const bool kvalid = kidx < nkeys;
    const int key = sweep_key<SAMPLE>(kidx, p);
    if constexpr (HAS_MASK) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = q0 + 8 * (r / 4) + 4 * half + (r % 4);
        if (kvalid && row < T) s[r] += to_f32(E{}, p.mask[((int64_t)b * T + row) * S + key]);
      }
    }
    if constexpr (SAMPLE) {
      if (kvalid) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int row = q0 + 8 * (r / 4) + 4 * half + (r % 4);
          if (row < T) p.samp[((int64_t)b * T + row) * p.Ms + kidx] = s[r];
        }
      }
    }
  };
  static_assert(kBN == 64, "two 32-key tiles per stage");

  if constexpr (!SAMPLE) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const float4 t4 = *reinterpret_cast<const float4*>(&tau_s[wave * kQW + 8 * g + 4 * half]);
      tau_r[4 * g + 0] = t4.x;
      tau_r[4 * g + 1] = t4.y;
      tau_r[4 * g + 2] = t4.z;
      tau_r[4 * g + 3] = t4.w;
    }
  }
  float sp[16];      // FILTER: scores of the pending tile
  int key_prev = -1; // uniform >= 0: key column base of the pending tile (+ col per lane)
  int buf = 0;
  for (; st < p.nstages; st += nsplit) {
    const int kb = st * kBN;
    const bool more = st + nsplit < p.nstages;
    if (more) gload((st + nsplit) * kBN, buf ^ 1);
    if constexpr (!SAMPLE) {
      if (key_prev >= 0) append(sp, key_prev + col);
    }
    float s0[16];
    tile_scores(s0, kb, 0, buf);
    if constexpr (!SAMPLE) append(s0, kb + col);
    tile_scores(sp, kb, 1, buf);
    key_prev = kb + 32;

    // Keep the gate conversion (which waits for this stage's loads) after the tile work.
    __builtin_amdgcn_sched_barrier(0);
    if (more) wstore(buf ^ 1);
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): next stage's direct LDS loads have landed
    __syncthreads();
    buf ^= 1;
  }
  if constexpr (!SAMPLE) {
    if (key_prev >= 0) append(sp, key_prev + col);
  }

  if constexpr (!SAMPLE) {
    flush(true);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (lane < kQW && q0 + lane < T) p.counts[list0 + (int64_t)lane * nsplit] = rcnt[wave][lane];
  }
}

// ---------------------------------------------------------------------------------------
// Threshold from the sample scores: one wave per query row.
// ---------------------------------------------------------------------------------------
template <int MPL>
__global__ __launch_bounds__(256) void indexer_tau_kernel(const float* samp, int Ms, int rank, int slack,
                                                          float* tau, int64_t rows) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
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
  uint64_t lo = wave_min_u(lmin);
  uint64_t hi = (uint64_t)wave_max_u(lmax) + 1;
  while (hi - lo > 1) {
    const uint32_t mid = (uint32_t)(lo + ((hi - lo) >> 1));
    uint32_t c = 0;
#pragma unroll
    for (int m = 0; m < MPL; ++m) c += kv[m] >= mid;
    c = wave_sum_u(c);
    if ((int)c < rank) {
      hi = mid;
    } else {
      lo = mid;
      if ((int)c <= rank + slack) break;
    }
  }
  if (lane == 0) tau[row] = key2f((uint32_t)lo);
}

// ---------------------------------------------------------------------------------------
// Exact top-k among the candidates: one wave per query row, candidates in registers.
//
// The row's lists (one per key split) are read as one sequence: entry e of the sequence
// goes to register slot e / 64 of lane e % 64, for up to 64 * kSelRegs entries (about
// 1.7 x topk are expected). A row with an overflowed list or fewer than topk candidates
// goes to the exact fallback; one with more candidates than the registers hold goes to
// the LDS selection. No barriers: reductions are wave-wide.
// ---------------------------------------------------------------------------------------
constexpr int kSelRegs = 48;

struct SelectParams {
  const int2* cand;
  const int* counts;
  int nsplit, cap;
  int32_t* out_idx;
  uint16_t* out_scores;
  int Kk;
  int* fb_count;
  int* fb_list;
  int* wide_count;
  int* wide_list;
  int64_t rows;
  int force_wide;  // test hook: every complete row takes the LDS selection
};

// Number of set bits of a wave mask below this lane.
__device__ __forceinline__ int lanes_below(uint64_t m) {
  return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

// Row lists as one sequence: off[s] = entries of the lists before split s (uniform);
// entry e sits at cand + (row * nsplit + s) * cap + (e - off[s]) for the split s holding it.
struct RowLists {
  int64_t base;  // (row * nsplit) * cap
  int off[kMaxSplit + 1];
  int nsplit, cap;
  __device__ __forceinline__ int64_t at(int e) const {
    int64_t a = base + e;
#pragma unroll
    for (int s2 = 1; s2 < kMaxSplit; ++s2)
      if (s2 < nsplit && e >= off[s2]) a += cap - (off[s2] - off[s2 - 1]);
    return a;
  }
};

__device__ __forceinline__ bool row_lists(const SelectParams& p, int64_t row, RowLists& rl) {
  rl.base = row * p.nsplit * (int64_t)p.cap;
  rl.nsplit = p.nsplit;
  rl.cap = p.cap;
  bool bad = false;
  int acc = 0;
#pragma unroll
  for (int s2 = 0; s2 < kMaxSplit; ++s2) {
    rl.off[s2] = acc;
    if (s2 < p.nsplit) {
      const int c = p.counts[row * p.nsplit + s2];
      bad |= c > p.cap;
      acc += min(c, p.cap);
    }
  }
  rl.off[kMaxSplit] = acc;
  return bad;
}

template <typename E>
__global__ __launch_bounds__(256) void indexer_select_kernel(const SelectParams p) {
  constexpr int KS = kSelRegs;
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (row >= p.rows) return;
  RowLists rl;
  const bool bad = row_lists(p, row, rl);
  const int total = rl.off[kMaxSplit];
  if (bad || total < p.Kk) {
    // The candidates may miss part of the top-k: exact brute force.
    if (lane == 0) p.fb_list[atomicAdd(p.fb_count, 1)] = (int)row;
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
  uint32_t kv[KS];
  uint32_t lmin = 0xFFFFFFFFu, lmax = 0u;
#pragma unroll
  for (int m0 = 0; m0 < KS; m0 += 8) {
#pragma unroll
    for (int m = m0; m < m0 + 8; ++m) kv[m] = 0u;
    if (m0 < nch) {
#pragma unroll
      for (int m = m0; m < m0 + 8; ++m) {
        const int e = m * 64 + lane;
        if (e < total) kv[m] = f2key(__int_as_float(p.cand[rl.at(e)].x));
      }
    }
  }
  // Key range of the live slots: empty slots hold 0, which kv - 1 wraps to the maximum.
#pragma unroll
  for (int m = 0; m < KS; ++m) {
    lmin = min(lmin, kv[m] - 1u);
    lmax = max(lmax, kv[m]);
  }
  lmin += 1u;
  // Bisection on the key value: count(key >= lo) >= Kk > count(key >= hi).
  uint64_t lo = wave_min_u(lmin), hi = (uint64_t)wave_max_u(lmax) + 1;
  while (hi - lo > 1) {
    const uint32_t mid = (uint32_t)(lo + ((hi - lo) >> 1));
    uint32_t cc = 0;
#pragma unroll
    for (int m0 = 0; m0 < KS; m0 += 8) {
      if (m0 < nch) {
#pragma unroll
        for (int m = m0; m < m0 + 8; ++m) cc += kv[m] >= mid;
      }
    }
    const int n = (int)wave_sum_u(cc);
    if (n >= p.Kk) {
      lo = mid;
      if (n == p.Kk) break;
    } else {
      hi = mid;
    }
  }
  const uint32_t thr = (uint32_t)lo;
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
  uint16_t* os = p.out_scores + row * p.Kk;
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
          const int2 cdt = p.cand[rl.at(m * 64 + lane)];
          oi[slot_out] = cdt.y;
          os[slot_out] = (uint16_t)pack1(E{}, __int_as_float(cdt.x));
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
    const int total = rl.off[kMaxSplit];
    for (int s2 = 0; s2 < p.nsplit; ++s2) {
      const int2* src = p.cand + rl.base + (int64_t)s2 * p.cap;
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
    uint16_t* os = p.out_scores + row * p.Kk;
    block_emit_topk(key_at, total, p.Kk, kth, take_eq,
                    [&](int slot, int i) {
                      if (slot < p.Kk) {
                        oi[slot] = vals[i];
                        os[slot] = (uint16_t)pack1(E{}, key2f(keys[i]));
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
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* w;
  const uint16_t* mask;
  const int* fb_count;
  const int* fb_list;
  float* scratch;  // [gridDim.x, S]
  int32_t* out_idx;
  uint16_t* out_scores;
  int T, S, Kk;
  float scale;
};

template <typename E, int HI, bool HAS_MASK>
__global__ __launch_bounds__(256) void indexer_fallback_kernel(const FallbackParams p) {
  __shared__ __attribute__((aligned(16))) uint32_t qs[HI * kDI / 2];
  __shared__ SelectShared sh;
  const int tid = threadIdx.x;
  const int nitems = *((volatile const int*)p.fb_count);
  float* sc = p.scratch + (int64_t)blockIdx.x * p.S;
  for (int item = blockIdx.x; item < nitems; item += gridDim.x) {
    const int row = p.fb_list[item];
    const int b = row / p.T;
    const uint32_t* qrow = reinterpret_cast<const uint32_t*>(p.q + (int64_t)row * HI * kDI);
    for (int i = tid; i < HI * kDI / 2; i += kSelThreads) qs[i] = qrow[i];
    __syncthreads();
    for (int j = tid; j < p.S; j += kSelThreads) {
      const uint4* kr = reinterpret_cast<const uint4*>(p.k + ((int64_t)b * p.S + j) * HI * kDI);
      float s = 0.f;
#pragma unroll
      for (int h = 0; h < HI; ++h) {
        float z = 0.f;
#pragma unroll
        for (int c = 0; c < kDI / 8; ++c) {
          const uint4 kv = kr[h * (kDI / 8) + c];
          const uint4 qv = *reinterpret_cast<const uint4*>(&qs[h * (kDI / 2) + c * 4]);
          z = dot2(E{}, qv.x, kv.x, z);
          z = dot2(E{}, qv.y, kv.y, z);
          z = dot2(E{}, qv.z, kv.z, z);
          z = dot2(E{}, qv.w, kv.w, z);
        }
        const float wv = to_f32(E{}, p.w[((int64_t)b * p.S + j) * HI + h]) * p.scale;
        s = fmaf(wv, relu_bits(z), s);
      }
      if constexpr (HAS_MASK) s += to_f32(E{}, p.mask[(int64_t)row * p.S + j]);
      sc[j] = s;
    }
    __threadfence_block();
    __syncthreads();
    int take_eq;
    auto key_at = [&](int i) { return f2key(sc[i]); };
    const uint32_t kth = block_radix_select(key_at, p.S, p.Kk, sh, take_eq);
    int32_t* oi = p.out_idx + (int64_t)row * p.Kk;
    uint16_t* os = p.out_scores + (int64_t)row * p.Kk;
    block_emit_topk(key_at, p.S, p.Kk, kth, take_eq,
                    [&](int slot, int i) {
                      if (slot < p.Kk) {
                        oi[slot] = i;
                        os[slot] = (uint16_t)pack1(E{}, sc[i]);
                      }
                    },
                    sh);
    __syncthreads();
  }
}

__global__ void set_int_kernel(int* ptr, int value) {
  if (threadIdx.x < 2 && blockIdx.x == 0) ptr[threadIdx.x] = value;
}

// ---------------------------------------------------------------------------------------
// Host-side plan.
// ---------------------------------------------------------------------------------------
size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

struct Plan {
  int Kk = 0;
  bool sample = false;
  int Ms = 0, rank = 0;
  int nsplit = 1, cap = 0;
  size_t off_tau = 0, off_samp = 0, off_counts = 0, off_cand = 0, off_fb = 0, off_fblist = 0,
         off_widelist = 0, off_scratch = 0, total = 0;
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
  }
  const size_t rows = (size_t)B * (size_t)T;
  size_t off = 0;
  pl.off_tau = off;      off = align_up(off + rows * 4, 256);
  pl.off_samp = off;     off = align_up(off + (pl.sample ? rows * (size_t)pl.Ms * 4 : 0), 256);
  pl.off_counts = off;   off = align_up(off + rows * kMaxSplit * 4, 256);
  pl.off_cand = off;     off = align_up(off + rows * (size_t)kSubTotal * 8, 256);
  pl.off_fb = off;       off = align_up(off + 64, 256);
  pl.off_fblist = off;   off = align_up(off + rows * 4, 256);
  pl.off_widelist = off; off = align_up(off + rows * 4, 256);
  pl.off_scratch = off;  off = align_up(off + (size_t)kFallbackBlocks * (size_t)S * 4, 256);
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
int choose_nsplit(int64_t tiles, int64_t S, int slots, bool sample) {
  if (!sample) return 1;
  int best = 1;
  double best_eff = -1.0;
  for (int ns = 1; ns <= kMaxSplit; ++ns) {
    if (ns > 1 && S / (ns * (int64_t)kBN) < 8) break;
    const double waves = (double)(tiles * ns) / slots;
    const double eff = waves / ceil(waves);
    if (eff > best_eff + 1e-9) {
      best_eff = eff;
      best = ns;
    }
  }
  return best;
}

template <typename E, int HI, bool HAS_MASK>
int run_typed(const ScoreParams& base, Plan pl, int64_t B, int32_t* out_idx, void* out_scores,
              uint8_t* ws, hipStream_t st) {
  int* fb_count = reinterpret_cast<int*>(ws + pl.off_fb);  // [0] brute force, [1] wide select
  hipLaunchKernelGGL(set_int_kernel, dim3(1), dim3(64), 0, st, fb_count, 0);
  GW_HIP_LAUNCH_CHECK("set_int_kernel");
  constexpr int BM = ScoreShape<HI>::BM;
  constexpr int THREADS = ScoreShape<HI>::THREADS;
  const int64_t tiles = (base.T + BM - 1) / BM;
  const int64_t rows = B * (int64_t)base.T;
  pl.nsplit = choose_nsplit(tiles * B, base.S, filter_slots((const void*)indexer_score_kernel<E, HI, false, HAS_MASK>, THREADS),
                            pl.sample);
  pl.cap = kSubTotal / pl.nsplit;
  float* tau = reinterpret_cast<float*>(ws + pl.off_tau);
  if (pl.sample) {
    ScoreParams sp = base;
    sp.samp = reinterpret_cast<float*>(ws + pl.off_samp);
    sp.Ms = pl.Ms;
    sp.tau = nullptr;
    sp.tau_mode = kTauArray;
    sp.nsplit = 1;
    sp.nstages = (pl.Ms + kBN - 1) / kBN;
    hipLaunchKernelGGL((indexer_score_kernel<E, HI, true, HAS_MASK>), dim3((unsigned)tiles, 1, (unsigned)B), dim3(THREADS),
                       0, st, sp);
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
  fp.nstages = (base.S + kBN - 1) / kBN;
  hipLaunchKernelGGL((indexer_score_kernel<E, HI, false, HAS_MASK>),
                     dim3((unsigned)tiles, (unsigned)pl.nsplit, (unsigned)B), dim3(THREADS), 0, st, fp);
  GW_HIP_LAUNCH_CHECK("indexer_score_kernel<filter>");
  SelectParams fs{};
  fs.cand = fp.cand;
  fs.counts = fp.counts;
  fs.nsplit = pl.nsplit;
  fs.cap = pl.cap;
  fs.out_idx = out_idx;
  fs.out_scores = static_cast<uint16_t*>(out_scores);
  fs.Kk = pl.Kk;
  fs.fb_count = fb_count;
  fs.fb_list = reinterpret_cast<int*>(ws + pl.off_fblist);
  fs.wide_count = fb_count + 1;
  fs.wide_list = reinterpret_cast<int*>(ws + pl.off_widelist);
  fs.rows = rows;
  fs.force_wide = base.force_wide;
  const dim3 sgrid2((unsigned)((rows + 3) / 4));
  hipLaunchKernelGGL((indexer_select_kernel<E>), sgrid2, dim3(256), 0, st, fs);
  GW_HIP_LAUNCH_CHECK("indexer_select_kernel");
  hipLaunchKernelGGL((indexer_select_wide_kernel<E>), dim3(kFallbackBlocks), dim3(256), 0, st, fs);
  GW_HIP_LAUNCH_CHECK("indexer_select_wide_kernel");
  FallbackParams bp{};
  bp.q = base.q;
  bp.k = base.k;
  bp.w = base.w;
  bp.mask = base.mask;
  bp.fb_count = fb_count;
  bp.fb_list = fs.fb_list;
  bp.scratch = reinterpret_cast<float*>(ws + pl.off_scratch);
  bp.out_idx = out_idx;
  bp.out_scores = fs.out_scores;
  bp.T = base.T;
  bp.S = base.S;
  bp.Kk = pl.Kk;
  bp.scale = base.scale;
  hipLaunchKernelGGL((indexer_fallback_kernel<E, HI, HAS_MASK>), dim3(kFallbackBlocks), dim3(256), 0, st, bp);
  GW_HIP_LAUNCH_CHECK("indexer_fallback_kernel");
  return GW_OK;
}

template <typename E, bool HAS_MASK>
int dispatch_hi(int hi, const ScoreParams& base, const Plan& pl, int64_t B, int32_t* out_idx,
                void* out_scores, uint8_t* ws, hipStream_t st) {
  switch (hi) {
    case 1: return run_typed<E, 1, HAS_MASK>(base, pl, B, out_idx, out_scores, ws, st);
    case 2: return run_typed<E, 2, HAS_MASK>(base, pl, B, out_idx, out_scores, ws, st);
    case 4: return run_typed<E, 4, HAS_MASK>(base, pl, B, out_idx, out_scores, ws, st);
    default: return run_typed<E, 8, HAS_MASK>(base, pl, B, out_idx, out_scores, ws, st);
  }
}

}  // namespace
}  // namespace gw

extern "C" size_t gw_indexer_topk_workspace_size(int64_t B, int64_t T, int64_t S, int64_t topk) {
  if (B <= 0 || T <= 0 || S <= 0 || topk <= 0) return 0;
  return gw::make_layout(B, T, S, topk).total;
}

extern "C" int gw_indexer_topk_fwd(int dtype, const void* q, const void* k, const void* w,
                                   const void* mask, int64_t B, int64_t T, int64_t S, int64_t Hi,
                                   int64_t Di, int64_t topk, float softmax_scale, int flags,
                                   int32_t* out_indices, void* out_scores, void* workspace,
                                   size_t workspace_bytes, void* stream) {
  using namespace gw;
  clear_error();
  GW_CHECK_ARG(dtype == GW_DTYPE_BF16 || dtype == GW_DTYPE_FP16, "unsupported dtype code %d", dtype);
  GW_CHECK_ARG(B >= 0 && T >= 0 && S >= 0 && topk >= 1, "invalid sizes B=%lld T=%lld S=%lld topk=%lld",
               (long long)B, (long long)T, (long long)S, (long long)topk);
  if (Di != kDI || !(Hi == 1 || Hi == 2 || Hi == 4 || Hi == 8))
    return set_error(GW_ERR_UNSUPPORTED, "indexer heads x dim %lld x %lld not supported (1/2/4/8 x 64)",
                     (long long)Hi, (long long)Di);
  GW_CHECK_ARG(softmax_scale > 0.f, "softmax_scale must be positive, got %g", (double)softmax_scale);
  GW_CHECK_ARG((flags & ~7) == 0 && (flags & 3) != 3, "invalid flags %d", flags);
  if (B == 0 || T == 0) return GW_OK;
  GW_CHECK_ARG(S >= 1, "empty key set");
  const int64_t Kk = topk < S ? topk : S;
  if (Kk > kMaxTopk)
    return set_error(GW_ERR_UNSUPPORTED, "topk %lld exceeds the supported maximum %d", (long long)Kk, kMaxTopk);
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
  base.q = static_cast<const uint16_t*>(q);
  base.k = static_cast<const uint16_t*>(k);
  base.w = static_cast<const uint16_t*>(w);
  base.mask = static_cast<const uint16_t*>(mask);
  base.T = (int)T;
  base.S = (int)S;
  base.scale = softmax_scale;
  base.tau_mode = (flags & GW_TOPK_FLAG_TAU_PLUS_INF) ? kTauPlusInf
                  : (flags & GW_TOPK_FLAG_TAU_MINUS_INF) ? kTauMinusInf
                                                         : kTauArray;
  base.force_wide = (flags & GW_TOPK_FLAG_FORCE_WIDE) ? 1 : 0;
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool has_mask = mask != nullptr;
  if (dtype == GW_DTYPE_BF16)
    return has_mask ? dispatch_hi<BF16, true>((int)Hi, base, pl, B, out_indices, out_scores, ws, st)
                    : dispatch_hi<BF16, false>((int)Hi, base, pl, B, out_indices, out_scores, ws, st);
  return has_mask ? dispatch_hi<FP16, true>((int)Hi, base, pl, B, out_indices, out_scores, ws, st)
                  : dispatch_hi<FP16, false>((int)Hi, base, pl, B, out_indices, out_scores, ws, st);
}
