// Key-major (CSR) transpose of a [B, T, K] position table for the atomic-free backward
// passes, built on the device without host synchronisation.
//
// The forward passes are query-major: query t reads the K rows pos[b,t,:]. The gradients
// of those rows (dK, dV of the attention; dK, dW of the indexer) are sums over every
// (t, j) with pos[b,t,j] == s. The reference scatters them with fp32 atomics
// (sparse_index_flash_attn.py:739-740, sparse_topk_indexer.py:1936-1941). Here the
// entries are grouped by key once per layer and shared by all heads and by both
// backward passes, so each key's gradient is reduced by one wave with no float atomics.
//
// Layout of the CSR buffer (offsets 256-byte aligned, see csr_layout()):
//   header   int32[4]    {n_items, n_parts, -, -}
//   count    int32[NK]   entries per key (NK = B*S; key = b*S + s); reused as fill cursor
//   off      int32[NK+1] exclusive prefix of count
//   item_off int32[NK+1] prefix of max(1, ceil(count/CH)): work items of <= CH entries
//   part_off int32[NK+1] prefix of (items of the key if it has > 1 item, else 0):
//                         slots for fp32 partial sums of keys split over several items
//   item_key int32[max_items] key of each work item
//   entries  int2[B*T*K] {t, j} of each valid entry, grouped by key
//   scratch  int2[B*T*K] ping-pong buffer of the sort of long key lists
// Entries with pos outside [0, S) are not recorded. Within a key, entries are sorted by
// (t, j) after the fill, so every reduction below runs in a fixed order and the
// backward is bitwise reproducible.
#include "gw_common.h"
#include "gw_csr.h"

namespace gw {
namespace {

constexpr int kScanThreads = 1024;
constexpr int kSortCap = 4096;  // entries sorted in LDS by one workgroup

__global__ __launch_bounds__(256) void csr_zero_kernel(int* count, int nk, int* header) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < nk) count[i] = 0;
  if (i < 4) header[i] = 0;
}

// One thread per (row, j); rows are (b, t).
__global__ __launch_bounds__(256) void csr_count_kernel(const int32_t* pos, int64_t psb, int64_t pst,
                                                        int T, int S, int K, int64_t n, int* count) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const int64_t row = i / K;
  const int j = (int)(i - row * K);
  const int b = (int)(row / T);
  const int t = (int)(row - (int64_t)b * T);
  const int s = pos[b * psb + t * pst + j];
  if (s >= 0 && s < S) atomicAdd(&count[b * S + s], 1);
}

__device__ __forceinline__ int items_of(int c) { return c <= kCsrChunk ? 1 : (c + kCsrChunk - 1) / kCsrChunk; }

// Single workgroup: exclusive scans of count, items and parts; resets count to 0 for
// use as the fill cursor.
__global__ __launch_bounds__(kScanThreads) void csr_scan_kernel(int* count, int* off, int* item_off,
                                                                int* part_off, int nk, int* header) {
  __shared__ int s_tot[3][kScanThreads / 64];
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int per = (nk + kScanThreads - 1) / kScanThreads;
  const int i0 = min(nk, tid * per), i1 = min(nk, i0 + per);
  int a = 0, bi = 0, cp = 0;
  for (int i = i0; i < i1; ++i) {
    const int c = count[i];
    const int it = items_of(c);
    a += c;
    bi += it;
    cp += it > 1 ? it : 0;
  }
  // block exclusive scan of (a, bi, cp)
  int xa = a, xb = bi, xc = cp;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int ya = __shfl_up(xa, o), yb = __shfl_up(xb, o), yc = __shfl_up(xc, o);
    if (lane >= o) {
      xa += ya;
      xb += yb;
      xc += yc;
    }
  }
  if (lane == 63) {
    s_tot[0][wave] = xa;
    s_tot[1][wave] = xb;
    s_tot[2][wave] = xc;
  }
  __syncthreads();
  int ba = 0, bb = 0, bc = 0;
  for (int w = 0; w < wave; ++w) {
    ba += s_tot[0][w];
    bb += s_tot[1][w];
    bc += s_tot[2][w];
  }
  int ea = ba + xa - a, eb = bb + xb - bi, ec = bc + xc - cp;
  for (int i = i0; i < i1; ++i) {
    const int c = count[i];
    const int it = items_of(c);
    off[i] = ea;
    item_off[i] = eb;
    part_off[i] = ec;
    ea += c;
    eb += it;
    ec += it > 1 ? it : 0;
    count[i] = 0;
  }
  if (tid == kScanThreads - 1) {
    off[nk] = ea;
    item_off[nk] = eb;
    part_off[nk] = ec;
    header[0] = eb;
    header[1] = ec;
  }
}

__global__ __launch_bounds__(256) void csr_fill_kernel(const int32_t* pos, int64_t psb, int64_t pst, int T,
                                                       int S, int K, int64_t n, int* cursor, const int* off,
                                                       int2* entries) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const int64_t row = i / K;
  const int j = (int)(i - row * K);
  const int b = (int)(row / T);
  const int t = (int)(row - (int64_t)b * T);
  const int s = pos[b * psb + t * pst + j];
  if (s >= 0 && s < S) {
    const int key = b * S + s;
    const int slot = off[key] + atomicAdd(&cursor[key], 1);
    entries[slot] = make_int2(t, j);
  }
}

// One thread per key: writes the key of each of its work items.
__global__ __launch_bounds__(256) void csr_items_kernel(const int* item_off, int nk, int* item_key) {
  const int key = blockIdx.x * 256 + threadIdx.x;
  if (key >= nk) return;
  for (int i = item_off[key]; i < item_off[key + 1]; ++i) item_key[i] = key;
}

__device__ __forceinline__ uint64_t pack_tj(int2 e) { return ((uint64_t)(uint32_t)e.x << 32) | (uint32_t)e.y; }
__device__ __forceinline__ int2 unpack_tj(uint64_t v) { return make_int2((int)(v >> 32), (int)(uint32_t)v); }

constexpr int kRadixBits = 6;
constexpr int kRadixBins = 1 << kRadixBits;
constexpr int kRadixPasses = 6;  // 36 bits cover any t*K + j < 2^31

// Sorts each key's entries by (t, j), in two kernels so that the common short lists do
// not pay for the long-list histogram's LDS. Lists of up to kSortCap entries are sorted in
// LDS with a bitonic network (csr_sort_short_kernel). Longer ones (keys chosen by very many
// queries) go through a stable LSD radix sort on t*K + j, one workgroup per key
// (csr_sort_long_kernel): every thread owns a contiguous sub-range, per-thread digit counts
// are scanned digit-major, and each thread scatters its sub-range in order, so every pass
// is stable. The passes alternate between the list and the same range of `scratch` and
// end in the list.
__global__ __launch_bounds__(256) void csr_sort_short_kernel(const int* off, int nk, int2* entries) {
  __shared__ uint64_t buf[kSortCap];
  const int key = blockIdx.x;
  if (key >= nk) return;
  const int beg = off[key], n = off[key + 1] - beg;
  if (n <= 1 || n > kSortCap) return;
  const int tid = threadIdx.x;
  int2* seg = entries + beg;
  int np = 1;
  while (np < n) np <<= 1;
  for (int i = tid; i < np; i += 256) buf[i] = i < n ? pack_tj(seg[i]) : ~0ull;
  __syncthreads();
  for (int size = 2; size <= np; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int i = tid; i < np / 2; i += 256) {
        const int lo = 2 * i - (i & (stride - 1));
        const int hi = lo + stride;
        const bool up = (lo & size) == 0;
        const uint64_t x = buf[lo], y = buf[hi];
        if ((x > y) == up) {
          buf[lo] = y;
          buf[hi] = x;
        }
      }
      __syncthreads();
    }
  }
  for (int i = tid; i < n; i += 256) seg[i] = unpack_tj(buf[i]);
}

__global__ __launch_bounds__(256) void csr_sort_long_kernel(const int* off, int nk, int K, int2* entries,
                                                            int2* scratch) {
  __shared__ int hist[kRadixBins * 256];  // hist[digit * 256 + thread]
  __shared__ int wave_tot[4];
  const int key = blockIdx.x;
  if (key >= nk) return;
  const int beg = off[key], n = off[key + 1] - beg;
  if (n <= kSortCap) return;
  const int tid = threadIdx.x;
  int2* seg = entries + beg;
  const int per = (n + 255) / 256;
  const int i0 = min(n, tid * per), i1 = min(n, i0 + per);
  int2* src = seg;
  int2* dst = scratch + beg;
  const int lane = tid & 63, wave = tid >> 6;
  for (int pass = 0; pass < kRadixPasses; ++pass) {
    const int shift = pass * kRadixBits;
    for (int d = 0; d < kRadixBins; ++d) hist[d * 256 + tid] = 0;
    for (int i = i0; i < i1; ++i) {
      const int2 e = src[i];
      const uint32_t kv = (uint32_t)e.x * (uint32_t)K + (uint32_t)e.y;
      hist[((kv >> shift) & (kRadixBins - 1)) * 256 + tid] += 1;
    }
    __syncthreads();
    // Exclusive scan of hist in flat (digit-major) order: thread x owns cells
    // [x * kRadixBins, (x + 1) * kRadixBins).
    int local = 0;
    for (int c = 0; c < kRadixBins; ++c) local += hist[tid * kRadixBins + c];
    int incl = local;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int y = __shfl_up(incl, o);
      if (lane >= o) incl += y;
    }
    if (lane == 63) wave_tot[wave] = incl;
    __syncthreads();
    int run = incl - local;
    for (int w = 0; w < wave; ++w) run += wave_tot[w];
    for (int c = 0; c < kRadixBins; ++c) {
      const int v = hist[tid * kRadixBins + c];
      hist[tid * kRadixBins + c] = run;
      run += v;
    }
    __syncthreads();
    for (int i = i0; i < i1; ++i) {
      const int2 e = src[i];
      const uint32_t kv = (uint32_t)e.x * (uint32_t)K + (uint32_t)e.y;
      int& slot = hist[((kv >> shift) & (kRadixBins - 1)) * 256 + tid];
      dst[slot] = e;
      ++slot;
    }
    __threadfence_block();
    __syncthreads();
    int2* tmp = src;
    src = dst;
    dst = tmp;
  }
}

}  // namespace

CsrLayout csr_layout(int64_t B, int64_t T, int64_t S, int64_t K) {
  CsrLayout L;
  const size_t nk = (size_t)B * (size_t)S;
  const size_t ne = (size_t)B * (size_t)T * (size_t)K;
  size_t o = 0;
  auto take = [&](size_t bytes) {
    const size_t at = o;
    o = (o + bytes + 255) / 256 * 256;
    return at;
  };
  L.nk = (int64_t)nk;
  L.header = take(16);
  L.count = take(nk * 4);
  L.off = take((nk + 1) * 4);
  L.item_off = take((nk + 1) * 4);
  L.part_off = take((nk + 1) * 4);
  L.max_items = (int64_t)nk + (int64_t)((ne + kCsrChunk - 1) / kCsrChunk);
  L.item_key = take((size_t)L.max_items * 4);
  L.entries = take(ne * 8);
  L.scratch = take(ne * 8);
  L.total = o;
  L.max_parts = 2 * (int64_t)((ne + kCsrChunk - 1) / kCsrChunk);
  return L;
}

CsrView csr_view(const void* csr, const CsrLayout& L) {
  const uint8_t* base = static_cast<const uint8_t*>(csr);
  CsrView v;
  v.header = reinterpret_cast<const int*>(base + L.header);
  v.off = reinterpret_cast<const int*>(base + L.off);
  v.item_off = reinterpret_cast<const int*>(base + L.item_off);
  v.part_off = reinterpret_cast<const int*>(base + L.part_off);
  v.item_key = reinterpret_cast<const int*>(base + L.item_key);
  v.entries = reinterpret_cast<const int2*>(base + L.entries);
  v.nk = (int)L.nk;
  return v;
}

}  // namespace gw

extern "C" size_t gw_kv_csr_size(int64_t B, int64_t T, int64_t S, int64_t K) {
  if (B <= 0 || T <= 0 || S <= 0 || K <= 0) return 256;
  return gw::csr_layout(B, T, S, K).total;
}

extern "C" int gw_kv_csr_build(const int32_t* pos, int64_t pos_stride_b, int64_t pos_stride_t, int64_t B,
                               int64_t T, int64_t S, int64_t K, void* csr, size_t csr_bytes, void* stream) {
  using namespace gw;
  clear_error();
  GW_CHECK_ARG(B >= 0 && T >= 0 && S >= 0 && K >= 0, "invalid sizes B=%lld T=%lld S=%lld K=%lld", (long long)B,
               (long long)T, (long long)S, (long long)K);
  GW_CHECK_ARG(csr != nullptr && aligned16(csr), "csr buffer must be non-null and 16-byte aligned");
  GW_CHECK_ARG(csr_bytes >= gw_kv_csr_size(B, T, S, K), "csr buffer needs %zu bytes, got %zu",
               gw_kv_csr_size(B, T, S, K), csr_bytes);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (B == 0 || T == 0 || S == 0 || K == 0) {
    // Empty table: zero header only.
    hipLaunchKernelGGL(csr_zero_kernel, dim3(1), dim3(256), 0, st, static_cast<int*>(csr), 0,
                       static_cast<int*>(csr));
    GW_HIP_LAUNCH_CHECK("csr_zero_kernel");
    return GW_OK;
  }
  GW_CHECK_ARG(pos != nullptr, "null position table");
  GW_CHECK_ARG(B * S < (1ll << 30) && B * T * K < (1ll << 31) && T < (1ll << 31),
               "table too large for int32 CSR offsets");
  const CsrLayout L = csr_layout(B, T, S, K);
  uint8_t* base = static_cast<uint8_t*>(csr);
  int* header = reinterpret_cast<int*>(base + L.header);
  int* count = reinterpret_cast<int*>(base + L.count);
  int* off = reinterpret_cast<int*>(base + L.off);
  int* item_off = reinterpret_cast<int*>(base + L.item_off);
  int* part_off = reinterpret_cast<int*>(base + L.part_off);
  int* item_key = reinterpret_cast<int*>(base + L.item_key);
  int2* entries = reinterpret_cast<int2*>(base + L.entries);
  int2* scratch = reinterpret_cast<int2*>(base + L.scratch);
  const int nk = (int)L.nk;
  const int64_t n = B * T * K;
  hipLaunchKernelGGL(csr_zero_kernel, dim3((nk + 255) / 256), dim3(256), 0, st, count, nk, header);
  GW_HIP_LAUNCH_CHECK("csr_zero_kernel");
  const dim3 egrid((unsigned)((n + 255) / 256));
  hipLaunchKernelGGL(csr_count_kernel, egrid, dim3(256), 0, st, pos, pos_stride_b, pos_stride_t, (int)T, (int)S,
                     (int)K, n, count);
  GW_HIP_LAUNCH_CHECK("csr_count_kernel");
  hipLaunchKernelGGL(csr_scan_kernel, dim3(1), dim3(kScanThreads), 0, st, count, off, item_off, part_off, nk,
                     header);
  GW_HIP_LAUNCH_CHECK("csr_scan_kernel");
  hipLaunchKernelGGL(csr_items_kernel, dim3((nk + 255) / 256), dim3(256), 0, st, item_off, nk, item_key);
  GW_HIP_LAUNCH_CHECK("csr_items_kernel");
  hipLaunchKernelGGL(csr_fill_kernel, egrid, dim3(256), 0, st, pos, pos_stride_b, pos_stride_t, (int)T, (int)S,
                     (int)K, n, count, off, entries);
  GW_HIP_LAUNCH_CHECK("csr_fill_kernel");
  hipLaunchKernelGGL(csr_sort_short_kernel, dim3(nk), dim3(256), 0, st, off, nk, entries);
  GW_HIP_LAUNCH_CHECK("csr_sort_short_kernel");
  hipLaunchKernelGGL(csr_sort_long_kernel, dim3(nk), dim3(256), 0, st, off, nk, (int)K, entries, scratch);
  GW_HIP_LAUNCH_CHECK("csr_sort_long_kernel");
  return GW_OK;
}
