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
//  K0b select_kernel<TAU>:  tau0[t] = the rank-r largest sample score, r chosen so that
//                           the number of keys scoring >= tau0 is >= topk with very high
//                           probability and about 1.2-2x topk on average.
//  K1 score_kernel<FILTER>: MFMA scores against all keys (split into nsplit key ranges for
//                           load balance); the epilogue keeps (score, key) pairs with
//                           score >= tau0 in per-(query, split) candidate lists.
//  K2 select_kernel<FINAL>: exact top-k of the candidates (radix select in LDS). A query
//                           whose lists overflowed or hold fewer than topk entries is
//                           queued for K3 instead.
//  K3 fallback_kernel:      exact brute force for queued queries (scores to scratch, radix
//                           select) - correct for any input, used rarely.
// Exactness: if count(score >= tau0) >= topk, every member of the top-k scores >= tau0 and
// is a candidate, so selecting among the candidates is exact. Ties at the k-th value are
// broken deterministically (lowest candidate position first).
//
// MFMA layout (v_mfma_f32_32x32x16_{bf16,f16}): C[32 queries x 32 keys]; A = q rows
// (stationary in VGPRs for the whole key sweep), B = key rows staged through LDS (padded
// rows, conflict-free 16-byte reads). Lane l owns key column l%32 and query rows
// 8*(r/4) + 4*(l/32) + r%4 of accumulator element r.
#include <math.h>

#include "gw_common.h"
#include "gw_select.h"

namespace gw {
namespace {

constexpr int kQW = 32;          // queries per wave
constexpr int kWaves = 4;
constexpr int kBM = kQW * kWaves; // queries per workgroup
constexpr int kBN = 64;          // keys per LDS stage
constexpr int kDI = 64;          // indexer head dim
constexpr int kCapTotal = 4096;  // candidate slots per query (split evenly over splits)
constexpr int kMaxSplit = 4;
constexpr int kMaxTopk = 2048;
constexpr int kFallbackBlocks = 256;

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

enum TauMode { kTauArray = 0, kTauPlusInf = 1, kTauMinusInf = 2 };

struct ScoreParams {
  const uint16_t* q;     // [B, T, HI, 64]
  const uint16_t* k;     // [B, S, HI, 64]
  const uint16_t* w;     // [B, S, HI]
  const uint16_t* mask;  // [B, T, S] or null
  const float* tau;      // [B*T] or null (-inf)
  float* samp;           // SAMPLE: [B*T, Ms]
  int2* cand;            // FILTER: [B*T, nsplit, cap]
  int* counts;           // FILTER: [B*T, nsplit]
  int T, S;
  int nsplit, split_len, cap;
  int Ms;
  int tau_mode;
  float scale;
};

// Key index of position i of the sweep (SAMPLE: i-th strided sample key).
template <bool SAMPLE>
__device__ __forceinline__ int sweep_key(int i, const ScoreParams& p) {
  if constexpr (SAMPLE) return (int)(((int64_t)i * p.S) / p.Ms);
  return i;
}

template <typename E, int HI, bool SAMPLE, bool HAS_MASK>
__global__ __launch_bounds__(256) void indexer_score_kernel(const ScoreParams p) {
  constexpr int ROW_BYTES = HI * kDI * 2;
  constexpr int ROW_STRIDE = ROW_BYTES + 16;
  constexpr int CHUNKS = ROW_BYTES / 16;
  constexpr int LOADS = (kBN * CHUNKS + 255) / 256;
  constexpr int WVALS = kBN * HI;
  constexpr int WLOADS = (WVALS + 255) / 256;

  __shared__ __attribute__((aligned(16))) uint8_t ktile[2][kBN * ROW_STRIDE];
  __shared__ float wtile[2][WVALS];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int b = blockIdx.z;
  const int split = blockIdx.y;
  const int q0 = blockIdx.x * kBM + wave * kQW;
  const int T = p.T, S = p.S;

  int kbeg, kend;  // sweep range
  if constexpr (SAMPLE) {
    kbeg = 0;
    kend = p.Ms;
  } else {
    kbeg = split * p.split_len;
    kend = min(S, kbeg + p.split_len);
  }

  // A operands: this lane's query row (lane % 32), k-chunk (lane / 32) of each 16-wide step.
  uint4 a[HI][4];
  {
    const int row = q0 + (lane & 31);
    const bool ok = row < T;
    const uint16_t* qr = p.q + ((int64_t)b * T + (ok ? row : 0)) * (HI * kDI) + (lane >> 5) * 8;
#pragma unroll
    for (int h = 0; h < HI; ++h)
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
        a[h][ks] = ok ? *reinterpret_cast<const uint4*>(qr + h * kDI + ks * 16) : make_uint4(0, 0, 0, 0);
  }

  float tau[16];
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int row = q0 + 8 * (r / 4) + 4 * (lane >> 5) + (r % 4);
    float tv = INFINITY;
    if (row < T) {
      if (p.tau_mode == kTauPlusInf) tv = INFINITY;
      else if (p.tau_mode == kTauMinusInf || p.tau == nullptr) tv = -INFINITY;
      else tv = p.tau[(int64_t)b * T + row];
    }
    tau[r] = tv;
  }

  int cnt[32];
#pragma unroll
  for (int i = 0; i < 32; ++i) cnt[i] = 0;

  uint4 kreg[LOADS];
  float wreg[WLOADS];

  auto gload = [&](int kb) {
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
      const int c = tid + 256 * i;
      const int kl = c / CHUNKS;
      const int ch = c % CHUNKS;
      uint4 v = make_uint4(0, 0, 0, 0);
      if (c < kBN * CHUNKS && kb + kl < kend) {
        const int key = sweep_key<SAMPLE>(kb + kl, p);
        v = *reinterpret_cast<const uint4*>(p.k + ((int64_t)b * S + key) * (HI * kDI) + ch * 8);
      }
      kreg[i] = v;
    }
#pragma unroll
    for (int i = 0; i < WLOADS; ++i) {
      const int c = tid + 256 * i;
      const int kl = c / HI, h = c % HI;
      float wv = 0.f;
      if (c < WVALS && kb + kl < kend) {
        const int key = sweep_key<SAMPLE>(kb + kl, p);
        wv = to_f32(E{}, p.w[((int64_t)b * S + key) * HI + h]) * p.scale;
      }
      wreg[i] = wv;
    }
  };
  auto lstore = [&](int buf) {
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
      const int c = tid + 256 * i;
      if (c < kBN * CHUNKS) {
        const int kl = c / CHUNKS;
        const int ch = c % CHUNKS;
        *reinterpret_cast<uint4*>(&ktile[buf][kl * ROW_STRIDE + ch * 16]) = kreg[i];
      }
    }
#pragma unroll
    for (int i = 0; i < WLOADS; ++i)
      if (tid + 256 * i < WVALS) wtile[buf][tid + 256 * i] = wreg[i];
  };

  const int64_t row_stride_c = (int64_t)p.nsplit * p.cap;
  int2* cand_base = nullptr;
  if constexpr (!SAMPLE) cand_base = p.cand + ((int64_t)b * T + q0) * row_stride_c + (int64_t)split * p.cap;

  if (kbeg < kend) {
    gload(kbeg);
    lstore(0);
  }
  __syncthreads();

  int buf = 0;
  for (int kb = kbeg; kb < kend; kb += kBN) {
    const bool more = kb + kBN < kend;
    if (more) gload(kb + kBN);

#pragma unroll
    for (int nb = 0; nb < kBN / 32; ++nb) {
      const int kl = nb * 32 + (lane & 31);
      const uint8_t* brow = &ktile[buf][kl * ROW_STRIDE + (lane >> 5) * 16];
      f32x16 acc[HI];
#pragma unroll
      for (int h = 0; h < HI; ++h) {
        acc[h] = f32x16{0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          const uint4 bop = *reinterpret_cast<const uint4*>(brow + h * (kDI * 2) + ks * 32);
          acc[h] = mfma32(E{}, a[h][ks], bop, acc[h]);
        }
      }
      float wv[HI];
#pragma unroll
      for (int h = 0; h < HI; ++h) wv[h] = wtile[buf][kl * HI + h];
      const int kidx = kb + kl;
      const bool kvalid = kidx < kend;
      const int key = sweep_key<SAMPLE>(kidx, p);

#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float s = 0.f;
#pragma unroll
        for (int h = 0; h < HI; ++h) s = fmaf(wv[h], fmaxf(acc[h][r], 0.f), s);
        const int rlo = 8 * (r / 4) + (r % 4);
        const int rrow = rlo + 4 * (lane >> 5);
        if constexpr (HAS_MASK) {
          const int row = q0 + rrow;
          if (kvalid && row < T) s += to_f32(E{}, p.mask[((int64_t)b * T + row) * S + key]);
        }
        if constexpr (SAMPLE) {
          const int row = q0 + rrow;
          if (kvalid && row < T) p.samp[((int64_t)b * T + row) * p.Ms + kidx] = s;
        } else {
          const bool pass = kvalid && (q0 + rrow < T) && (s >= tau[r]);
          const uint64_t m = __ballot(pass);
          if (m) {
            const uint32_t lo = (uint32_t)m, hi = (uint32_t)(m >> 32);
            const int plo = __popc(lo), phi = __popc(hi);
            const int pre = __builtin_amdgcn_mbcnt_hi(hi, __builtin_amdgcn_mbcnt_lo(lo, 0));
            const int slot = (lane < 32) ? (cnt[rlo] + pre) : (cnt[rlo + 4] + pre - plo);
            if (pass && slot < p.cap)
              cand_base[(int64_t)rrow * row_stride_c + slot] = make_int2(__float_as_int(s), key);
            cnt[rlo] += plo;
            cnt[rlo + 4] += phi;
          }
        }
      }
    }

    if (more) lstore(buf ^ 1);
    __syncthreads();
    buf ^= 1;
  }

  if constexpr (!SAMPLE) {
    int mine = 0;
#pragma unroll
    for (int i = 0; i < 32; ++i)
      if ((lane & 31) == i) mine = cnt[i];
    const int row = q0 + lane;
    if (lane < 32 && row < T) p.counts[((int64_t)b * T + row) * p.nsplit + split] = mine;
  }
}

// ---------------------------------------------------------------------------------------
// Selection over candidates (FINAL) or over the sample scores (TAU).
// ---------------------------------------------------------------------------------------
struct SelectParams {
  const float* samp;
  int Ms, rank;
  float* tau;
  const int2* cand;
  const int* counts;
  int nsplit, cap;
  int32_t* out_idx;
  uint16_t* out_scores;
  int Kk;
  int* fb_count;
  int* fb_list;
  int T;
};

template <typename E, bool FINAL>
__global__ __launch_bounds__(256) void indexer_select_kernel(const SelectParams p) {
  __shared__ uint32_t keys[kCapTotal];
  __shared__ int vals[FINAL ? kCapTotal : 1];
  __shared__ SelectShared sh;
  __shared__ int offs[kMaxSplit + 1];
  const int tid = threadIdx.x;
  const int t = blockIdx.x, b = blockIdx.y;
  const int64_t row = (int64_t)b * p.T + t;

  if constexpr (!FINAL) {
    const float* src = p.samp + row * p.Ms;
    for (int i = tid; i < p.Ms; i += kSelThreads) keys[i] = f2key(src[i]);
    __syncthreads();
    int take_eq;
    const uint32_t kth = block_radix_select([&](int i) { return keys[i]; }, p.Ms, p.rank, sh, take_eq);
    if (tid == 0) p.tau[row] = key2f(kth);
  } else {
    if (tid == 0) {
      int total = 0;
      bool bad = false;
      for (int sp = 0; sp < p.nsplit; ++sp) {
        const int c = p.counts[row * p.nsplit + sp];
        bad |= c > p.cap;
        offs[sp] = total;
        total += min(c, p.cap);
      }
      offs[p.nsplit] = total;
      if (bad || total < p.Kk) offs[p.nsplit] = -1;
    }
    __syncthreads();
    const int total = offs[p.nsplit];
    if (total < 0) {
      if (tid == 0) p.fb_list[atomicAdd(p.fb_count, 1)] = (int)row;
      return;
    }
    for (int sp = 0; sp < p.nsplit; ++sp) {
      const int o = offs[sp], n = offs[sp + 1] - o;
      const int2* src = p.cand + (row * p.nsplit + sp) * p.cap;
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
    const int b = row / p.T, t = row - b * p.T;
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
        s = fmaf(wv, fmaxf(z, 0.f), s);
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
  if (threadIdx.x == 0 && blockIdx.x == 0) *ptr = value;
}

// ---------------------------------------------------------------------------------------
// Host-side plan.
// ---------------------------------------------------------------------------------------
size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

struct Plan {
  int Kk = 0;
  bool sample = false;
  int Ms = 0, rank = 0;
  int nsplit = 1, split_len = 0, cap = kCapTotal;
  size_t off_tau = 0, off_samp = 0, off_counts = 0, off_cand = 0, off_fb = 0, off_fblist = 0,
         off_scratch = 0, total = 0;
};

Plan make_plan(int64_t B, int64_t T, int64_t S, int64_t topk) {
  Plan pl;
  pl.Kk = (int)(topk < S ? topk : S);
  pl.sample = S > kCapTotal;
  if (pl.sample) {
    pl.Ms = (int)(S >= 65536 ? 4096 : 2048);
    if (pl.Ms > S) pl.Ms = (int)S;
    const double lam = (double)pl.Kk * pl.Ms / (double)S;
    int r = (int)ceil(lam + 4.5 * sqrt(lam) + 2.0);
    pl.rank = r > pl.Ms ? pl.Ms : r;
    const int64_t qtiles = ((T + kBM - 1) / kBM) * B;
    int ns = (int)((1024 + qtiles - 1) / qtiles);
    ns = ns < 1 ? 1 : (ns > kMaxSplit ? kMaxSplit : ns);
    const int64_t max_by_len = (S + 1023) / 1024;  // keep >= ~1024 keys per split
    if (ns > max_by_len) ns = (int)max_by_len;
    int64_t len = (S + ns - 1) / ns;
    len = (len + kBN - 1) / kBN * kBN;
    pl.split_len = (int)len;
    pl.nsplit = (int)((S + len - 1) / len);
  } else {
    pl.nsplit = 1;
    pl.split_len = (int)((S + kBN - 1) / kBN * kBN);
  }
  pl.cap = kCapTotal / pl.nsplit;
  const size_t rows = (size_t)B * (size_t)T;
  size_t off = 0;
  pl.off_tau = off;      off = align_up(off + rows * 4, 256);
  pl.off_samp = off;     off = align_up(off + (pl.sample ? rows * (size_t)pl.Ms * 4 : 0), 256);
  pl.off_counts = off;   off = align_up(off + rows * pl.nsplit * 4, 256);
  pl.off_cand = off;     off = align_up(off + rows * (size_t)pl.nsplit * pl.cap * 8, 256);
  pl.off_fb = off;       off = align_up(off + 64, 256);
  pl.off_fblist = off;   off = align_up(off + rows * 4, 256);
  pl.off_scratch = off;  off = align_up(off + (size_t)kFallbackBlocks * (size_t)S * 4, 256);
  pl.total = off;
  return pl;
}

template <typename E, int HI, bool HAS_MASK>
int run_typed(const ScoreParams& base, const Plan& pl, int64_t B, int32_t* out_idx, void* out_scores,
              uint8_t* ws, hipStream_t st) {
  int* fb_count = reinterpret_cast<int*>(ws + pl.off_fb);
  hipLaunchKernelGGL(set_int_kernel, dim3(1), dim3(64), 0, st, fb_count, 0);
  GW_HIP_LAUNCH_CHECK("set_int_kernel");
  const dim3 sgrid((base.T + kBM - 1) / kBM, 1, (unsigned)B);
  float* tau = reinterpret_cast<float*>(ws + pl.off_tau);
  if (pl.sample) {
    ScoreParams sp = base;
    sp.samp = reinterpret_cast<float*>(ws + pl.off_samp);
    sp.Ms = pl.Ms;
    sp.tau = nullptr;
    sp.tau_mode = kTauArray;
    hipLaunchKernelGGL((indexer_score_kernel<E, HI, true, HAS_MASK>), sgrid, dim3(256), 0, st, sp);
    GW_HIP_LAUNCH_CHECK("indexer_score_kernel<sample>");
    SelectParams tp{};
    tp.samp = sp.samp;
    tp.Ms = pl.Ms;
    tp.rank = pl.rank;
    tp.tau = tau;
    tp.T = base.T;
    hipLaunchKernelGGL((indexer_select_kernel<E, false>), dim3(base.T, (unsigned)B), dim3(256), 0, st, tp);
    GW_HIP_LAUNCH_CHECK("indexer_select_kernel<tau>");
  }
  ScoreParams fp = base;
  fp.tau = pl.sample ? tau : nullptr;
  fp.cand = reinterpret_cast<int2*>(ws + pl.off_cand);
  fp.counts = reinterpret_cast<int*>(ws + pl.off_counts);
  fp.nsplit = pl.nsplit;
  fp.split_len = pl.split_len;
  fp.cap = pl.cap;
  const dim3 fgrid((base.T + kBM - 1) / kBM, pl.nsplit, (unsigned)B);
  hipLaunchKernelGGL((indexer_score_kernel<E, HI, false, HAS_MASK>), fgrid, dim3(256), 0, st, fp);
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
  fs.T = base.T;
  hipLaunchKernelGGL((indexer_select_kernel<E, true>), dim3(base.T, (unsigned)B), dim3(256), 0, st, fs);
  GW_HIP_LAUNCH_CHECK("indexer_select_kernel<final>");
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
  return gw::make_plan(B, T, S, topk).total;
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
  GW_CHECK_ARG((flags & ~3) == 0 && flags != 3, "invalid flags %d", flags);
  if (B == 0 || T == 0) return GW_OK;
  GW_CHECK_ARG(S >= 1, "empty key set");
  const int64_t Kk = topk < S ? topk : S;
  if (Kk > kMaxTopk)
    return set_error(GW_ERR_UNSUPPORTED, "topk %lld exceeds the supported maximum %d", (long long)Kk, kMaxTopk);
  GW_CHECK_ARG(q && k && w && out_indices && out_scores, "null tensor pointer");
  GW_CHECK_ARG(aligned16(q) && aligned16(k), "q and k must be 16-byte aligned");
  GW_CHECK_ARG(B <= 65535 && T < (1ll << 31) && S < (1ll << 30), "size exceeds grid or int32 range");
  const Plan pl = make_plan(B, T, S, topk);
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
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool has_mask = mask != nullptr;
  if (dtype == GW_DTYPE_BF16)
    return has_mask ? dispatch_hi<BF16, true>((int)Hi, base, pl, B, out_indices, out_scores, ws, st)
                    : dispatch_hi<BF16, false>((int)Hi, base, pl, B, out_indices, out_scores, ws, st);
  return has_mask ? dispatch_hi<FP16, true>((int)Hi, base, pl, B, out_indices, out_scores, ws, st)
                  : dispatch_hi<FP16, false>((int)Hi, base, pl, B, out_indices, out_scores, ws, st);
}
