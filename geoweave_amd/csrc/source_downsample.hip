// Source-downsample coarse selector for gfx950: the two device steps around the indexer
// top-k over pooled keys (reference: the "legacy" strategy of DSAAttention's
// source-downsample selector, easyvolcap/official_vggt/layers/dsa_attention.py:3386-3542
// and :4079-4128, :4187-4217).
//
// A source row r covers the fine tokens source_to_fine[r, 0..M) (-1 past its count): one
// token for a special or edge row, the tokens of a factor x factor cell (or its
// representative points) for a coarse row.
//
//  * gw_source_downsample_pool: the indexer key and gate of every source row are the mean
//    of its fine rows (F.avg_pool2d over a cell, or the mean of the representative points;
//    special and edge rows are copies): fp32 sum in listed order, divided by the count,
//    rounded once to the 16-bit input type. One thread per 8 elements of a row.
//  * gw_source_downsample_expand: the chosen source rows of a query, in their given order
//    or, with their scores, by score descending (row index ascending on ties), become fine
//    tokens: round robin (the m-th token of every chosen row for m = 0, 1, ...)
//    or row by row, invalid slots skipped, cut to the target; a query with fewer valid
//    tokens repeats its last min(count, pad_window) tokens cyclically (also when Kc * M is
//    below the target, where the reference fails on a shape mismatch). One wave per
//    query: ballots compact the tokens into LDS, then the row is written once.
#include "gw_common.h"
#include "gw_sort.h"

namespace gw {
namespace {

constexpr int kExpandMaxTarget = 4096;
constexpr int kExpandMaxKc = 4096;
constexpr int kSortRegsMax = 16;  // register bitonic sort up to 64 * 16 chosen rows

template <typename E>
__global__ __launch_bounds__(256) void sd_pool_kernel(const uint16_t* k, const uint16_t* w, int S, int E8, int Hi,
                                                      const int32_t* stf, int L, int M, uint16_t* sk,
                                                      uint16_t* sw) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;  // (row, chunk) within batch b
  const int b = blockIdx.y;
  if (i >= (int64_t)L * E8) return;
  const int r = (int)(i / E8), c = (int)(i - (int64_t)r * E8);
  const int32_t* toks = stf + (int64_t)r * M;
  float acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = 0.f;
  float wacc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) wacc[e] = 0.f;
  int cnt = 0;
  const int row_elems = E8 * 8;
  for (int m = 0; m < M; ++m) {
    const int tok = toks[m];
    if (tok < 0 || tok >= S) continue;
    ++cnt;
    const uint4 v = *reinterpret_cast<const uint4*>(k + ((int64_t)b * S + tok) * row_elems + c * 8);
    float f[8];
    unpack8<E>(v, f);
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] += f[e];
    if (c == 0) {
      for (int h = 0; h < Hi && h < 8; ++h) {
        const uint32_t u = w[((int64_t)b * S + tok) * Hi + h];
        float lo, hi;
        unpack2(E{}, u, lo, hi);
        wacc[h] += lo;
      }
    }
  }
  const float n = cnt > 0 ? (float)cnt : 1.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = acc[e] / n;
  *reinterpret_cast<uint4*>(sk + ((int64_t)b * L + r) * row_elems + c * 8) = pack8<E>(acc);
  if (c == 0) {
    for (int h = 0; h < Hi && h < 8; ++h) sw[((int64_t)b * L + r) * Hi + h] = (uint16_t)pack1(E{}, wacc[h] / n);
  }
}

struct ExpandParams {
  const int32_t* cidx;
  const uint16_t* cscore;  // nullable: order the chosen rows by (score desc, row asc)
  int64_t csb, cst;
  int T, Kc;
  const int32_t* stf;
  int L, M;
  int round_robin;
  int target, window;
  int P;  // Kc rounded up to a power of two
  int32_t* out;
  int64_t rows;
};

template <int R>
__device__ __forceinline__ void order_rows_regs(uint64_t (&key)[R], int Kc, int32_t* ordered) {
  const int lane = threadIdx.x & 63;
  wave_bitonic_sort<R>(key);
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int e = r * 64 + lane;
    if (e < Kc) ordered[e] = (int32_t)(uint32_t)key[r];
  }
}

template <typename E>
__global__ __launch_bounds__(64) void sd_expand_kernel(const ExpandParams p) {
  // Dynamic LDS: buf[target] (compacted tokens), then, when scores are given, the ordered
  // rows [Kc] and, for lists longer than the register sort takes, keys[P] (P = Kc rounded
  // up to a power of two) for an LDS sort.
  extern __shared__ int32_t lds[];
  int32_t* buf = lds;
  const int lane = threadIdx.x;
  const int64_t row = blockIdx.x;
  if (row >= p.rows) return;
  const int64_t b = row / p.T, t = row - b * p.T;
  const int32_t* ci = p.cidx + b * p.csb + t * p.cst;
  if (p.cscore != nullptr) {
    // Canonical order of the chosen rows: score descending, row index ascending on ties.
    // Bitonic sort of the keys (~orderable(score) << 32 | row), ascending, padded with
    // all-ones keys; the wave runs every stage (LDS ops of one wave complete in order).
    const uint16_t* cs = p.cscore + b * p.csb + t * p.cst;
    auto make_key = [&](int c) -> uint64_t {
      if (c >= p.Kc) return ~0ull;
      float sc, unused;
      unpack2(E{}, (uint32_t)cs[c], sc, unused);
      const uint32_t u = __float_as_uint(sc);
      const uint32_t ord = (u & 0x80000000u) ? ~u : (u | 0x80000000u);  // monotonic in sc
      return ((uint64_t)(~ord) << 32) | (uint32_t)ci[c];
    };
    int32_t* ordered = buf + ((p.target + 1) & ~1);  // [Kc], after the compaction buffer
    if (p.P <= 64 * kSortRegsMax) {
      switch (p.P / 64) {
        case 0:
        case 1: { uint64_t kr[1]; for (int r = 0; r < 1; ++r) kr[r] = make_key(r * 64 + lane); order_rows_regs<1>(kr, p.Kc, ordered); break; }
        case 2: { uint64_t kr[2]; for (int r = 0; r < 2; ++r) kr[r] = make_key(r * 64 + lane); order_rows_regs<2>(kr, p.Kc, ordered); break; }
        case 4: { uint64_t kr[4]; for (int r = 0; r < 4; ++r) kr[r] = make_key(r * 64 + lane); order_rows_regs<4>(kr, p.Kc, ordered); break; }
        case 8: { uint64_t kr[8]; for (int r = 0; r < 8; ++r) kr[r] = make_key(r * 64 + lane); order_rows_regs<8>(kr, p.Kc, ordered); break; }
        default: { uint64_t kr[16]; for (int r = 0; r < 16; ++r) kr[r] = make_key(r * 64 + lane); order_rows_regs<16>(kr, p.Kc, ordered); break; }
      }
    } else {
      // Longer lists: the same sort through LDS.
      uint64_t* keys = reinterpret_cast<uint64_t*>(ordered + ((p.Kc + 1) & ~1));
      for (int c = lane; c < p.P; c += 64) keys[c] = make_key(c);
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      for (int kk = 2; kk <= p.P; kk <<= 1) {
        for (int j = kk >> 1; j > 0; j >>= 1) {
          for (int i = lane; i < p.P; i += 64) {
            const int ixj = i ^ j;
            if (ixj > i) {
              const uint64_t a = keys[i], c2 = keys[ixj];
              if ((a > c2) == ((i & kk) == 0)) {
                keys[i] = c2;
                keys[ixj] = a;
              }
            }
          }
          __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
          __builtin_amdgcn_wave_barrier();
          __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        }
      }
      for (int c = lane; c < p.Kc; c += 64) ordered[c] = (int32_t)(uint32_t)keys[c];
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    ci = ordered;
  }
  const int n = p.Kc * p.M;
  int base = 0;  // valid tokens seen so far (uniform)
  for (int p0 = 0; p0 < n && base < p.target; p0 += 64) {
    const int q = p0 + lane;
    int tok = -1;
    if (q < n) {
      int c, m;
      if (p.round_robin) {
        m = q / p.Kc;
        c = q - m * p.Kc;
      } else {
        c = q / p.M;
        m = q - c * p.M;
      }
      const int s = ci[c];
      if (s >= 0 && s < p.L) tok = p.stf[(int64_t)s * p.M + m];
    }
    const bool valid = tok >= 0;
    const uint64_t vm = __ballot(valid);
    const int pos = base + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(vm >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)vm, 0u));
    if (valid && pos < p.target) buf[pos] = tok;
    base += __popcll(vm);
  }
  __syncthreads();
  const int cnt = min(base, p.target);
  const int window = min(max(cnt, 1), p.window);
  const int start = max(cnt, 1) - window;
  int32_t* o = p.out + row * p.target;
  for (int j = lane; j < p.target; j += 64) {
    int v;
    if (j < cnt) v = buf[j];
    else if (cnt == 0) v = -1;  // no valid token: the reference repeats an empty slot
    else v = buf[start + (j - cnt) % window];
    o[j] = v;
  }
}

}  // namespace
}  // namespace gw

extern "C" int gw_source_downsample_pool(int dtype, const void* k, const void* w, int64_t B, int64_t S,
                                         int64_t Hi, int64_t Di, const int32_t* source_to_fine, int64_t L,
                                         int64_t M, void* source_k, void* source_w, void* stream) {
  using namespace gw;
  clear_error();
  GW_CHECK_ARG(dtype == GW_DTYPE_BF16 || dtype == GW_DTYPE_FP16, "unsupported dtype code %d", dtype);
  GW_CHECK_ARG(B >= 0 && S >= 1 && L >= 0 && M >= 1, "invalid sizes B=%lld S=%lld L=%lld M=%lld", (long long)B,
               (long long)S, (long long)L, (long long)M);
  GW_CHECK_ARG(Hi >= 1 && Hi <= 8 && Di >= 8 && (Hi * Di) % 8 == 0,
               "indexer heads x dim %lld x %lld not supported (Hi <= 8, Hi*Di a multiple of 8)", (long long)Hi,
               (long long)Di);
  if (B == 0 || L == 0) return GW_OK;
  GW_CHECK_ARG(k && w && source_to_fine && source_k && source_w, "null tensor pointer");
  GW_CHECK_ARG(aligned16(k) && aligned16(source_k), "k and source_k must be 16-byte aligned");
  GW_CHECK_ARG(B <= 65535 && S < (1ll << 31) && L * Hi * Di / 8 < (1ll << 31), "size exceeds grid or int32 range");
  const int E8 = (int)(Hi * Di / 8);
  const dim3 grid((unsigned)((L * E8 + 255) / 256), (unsigned)B);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == GW_DTYPE_BF16)
    hipLaunchKernelGGL(sd_pool_kernel<BF16>, grid, dim3(256), 0, st, static_cast<const uint16_t*>(k),
                       static_cast<const uint16_t*>(w), (int)S, E8, (int)Hi, source_to_fine, (int)L, (int)M,
                       static_cast<uint16_t*>(source_k), static_cast<uint16_t*>(source_w));
  else
    hipLaunchKernelGGL(sd_pool_kernel<FP16>, grid, dim3(256), 0, st, static_cast<const uint16_t*>(k),
                       static_cast<const uint16_t*>(w), (int)S, E8, (int)Hi, source_to_fine, (int)L, (int)M,
                       static_cast<uint16_t*>(source_k), static_cast<uint16_t*>(source_w));
  GW_HIP_LAUNCH_CHECK("sd_pool_kernel");
  return GW_OK;
}

extern "C" int gw_source_downsample_expand(int dtype, const int32_t* coarse_idx, const void* coarse_scores,
                                           int64_t idx_stride_b, int64_t idx_stride_t,
                                           int64_t B, int64_t T, int64_t Kc, const int32_t* source_to_fine,
                                           int64_t L, int64_t M, int round_robin, int64_t target,
                                           int64_t pad_window, int32_t* out, void* stream) {
  using namespace gw;
  clear_error();
  GW_CHECK_ARG(B >= 0 && T >= 0 && Kc >= 1 && L >= 1 && M >= 1 && target >= 1,
               "invalid sizes B=%lld T=%lld Kc=%lld L=%lld M=%lld target=%lld", (long long)B, (long long)T,
               (long long)Kc, (long long)L, (long long)M, (long long)target);
  GW_CHECK_ARG(dtype == GW_DTYPE_BF16 || dtype == GW_DTYPE_FP16, "unsupported dtype code %d", dtype);
  if (coarse_scores != nullptr && Kc > kExpandMaxKc)
    return set_error(GW_ERR_UNSUPPORTED, "ordering %lld chosen rows exceeds the supported maximum %d",
                     (long long)Kc, kExpandMaxKc);
  if (target > kExpandMaxTarget)
    return set_error(GW_ERR_UNSUPPORTED, "target %lld exceeds the supported maximum %d", (long long)target,
                     kExpandMaxTarget);
  GW_CHECK_ARG(pad_window >= 1, "pad_window must be positive, got %lld", (long long)pad_window);
  if (B == 0 || T == 0) return GW_OK;
  GW_CHECK_ARG(coarse_idx && source_to_fine && out, "null tensor pointer");
  GW_CHECK_ARG(B * T < (1ll << 31) && Kc * M < (1ll << 30) && L * M < (1ll << 31), "size exceeds int32 range");
  ExpandParams p;
  p.cidx = coarse_idx;
  p.cscore = static_cast<const uint16_t*>(coarse_scores);
  p.csb = idx_stride_b;
  p.cst = idx_stride_t;
  p.T = (int)T;
  p.Kc = (int)Kc;
  p.stf = source_to_fine;
  p.L = (int)L;
  p.M = (int)M;
  p.round_robin = round_robin ? 1 : 0;
  p.target = (int)target;
  p.window = (int)(pad_window < target ? pad_window : target);
  p.out = out;
  p.rows = B * T;
  size_t pow2 = 1;
  while ((int64_t)pow2 < Kc) pow2 <<= 1;
  p.P = (int)pow2;
  const size_t words = (size_t)((target + 1) & ~1ll) + (coarse_scores ? (size_t)((Kc + 1) & ~1ll) : 0);
  const size_t lds = ((words + 1) & ~(size_t)1) * 4 + (coarse_scores && pow2 > 64 * kSortRegsMax ? pow2 * 8 : 0);
  if (dtype == GW_DTYPE_BF16)
    hipLaunchKernelGGL(sd_expand_kernel<BF16>, dim3((unsigned)(B * T)), dim3(64), lds,
                       static_cast<hipStream_t>(stream), p);
  else
    hipLaunchKernelGGL(sd_expand_kernel<FP16>, dim3((unsigned)(B * T)), dim3(64), lds,
                       static_cast<hipStream_t>(stream), p);
  GW_HIP_LAUNCH_CHECK("sd_expand_kernel");
  return GW_OK;
}
