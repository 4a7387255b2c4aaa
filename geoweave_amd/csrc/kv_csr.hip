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
// Construction: a stable LSD radix sort of the entries by key (6 bits per pass), keyed
// entries taken in row-major (b, t, j) order, so within a key the entries come out in
// (t, j) order with no further sort; entries with pos outside [0, S) get the key NK and
// sort past every valid key. Each pass is a per-tile digit histogram, one exclusive scan
// of the (digit, tile) counts and a stable scatter. A tile of 64 x kRounds entries belongs
// to one wave, which ranks equal digits with ballots (no atomics) and orders the tile by
// digit in LDS before writing it out, so every step is deterministic. Offsets come from the boundaries of the sorted keys.
//
// Layout of the CSR buffer (offsets 256-byte aligned, see csr_layout()):
//   header   int32[4]    {n_items, n_parts, -, -}
//   count    int32[NK]   entries per key (NK = B*S; key = b*S + s)
//   off      int32[NK+1] exclusive prefix of count (off[NK] = number of valid entries)
//   item_off int32[NK+1] prefix of max(1, ceil(count/CH)): work items of <= CH entries
//   part_off int32[NK+1] prefix of (items of the key if it has > 1 item, else 0):
//                         slots for fp32 partial sums of keys split over several items
//   item_key int32[max_items] key of each work item
//   entries  int2[B*T*K] {t, j} of each valid entry, grouped by key, (t, j)-ordered
//   keys/vals uint32[2][2][B*T*K] radix-sort ping-pong buffers (key, flat entry index)
//   hist     uint32[64 * (tiles + 1)] per-pass (digit, tile) counts, scanned in place per
//            digit, then the 64 digit totals (a tile is 2048 entries)
//   raw      uint32[64 * tiles] the same counts, unscanned
#include "gw_common.h"
#include "gw_csr.h"

namespace gw {
namespace {

constexpr int kScanThreads = 1024;
constexpr int kRadixBits = 6;
constexpr int kBins = 1 << kRadixBits;
constexpr int kRounds = 32;                  // 64-entry rounds per wave tile
constexpr int kTile = 64 * kRounds;          // entries per wave tile

__global__ __launch_bounds__(256) void csr_zero_kernel(int* count, int nk, int* header) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < nk) count[i] = 0;
  if (i < 4) header[i] = 0;
}

__device__ __forceinline__ int items_of(int c) { return c <= kCsrChunk ? 1 : (c + kCsrChunk - 1) / kCsrChunk; }

// Key of flat entry i = (b*T + t)*K + j read from the position table.
__device__ __forceinline__ uint32_t entry_key(const int32_t* pos, int64_t psb, int64_t pst, int T, int S, int K,
                                              int nk, uint32_t i) {
  const uint32_t row = i / (uint32_t)K;
  const int j = (int)(i - row * (uint32_t)K);
  const int b = (int)(row / (uint32_t)T);
  const int t = (int)(row - (uint32_t)b * (uint32_t)T);
  const int s = pos[b * psb + t * pst + j];
  return (s >= 0 && s < S) ? (uint32_t)(b * S + s) : (uint32_t)nk;
}

struct RadixPass {
  const int32_t* pos;  // first pass: the position table
  int64_t psb, pst;
  int T, S, K, nk;
  const uint32_t* keys_in;
  const uint32_t* vals_in;
  uint32_t* keys_out;
  uint32_t* vals_out;
  int2* entries;       // last pass: {t, j}
  uint32_t* hist;      // [kBins][tiles] counts, scanned per digit, then [kBins] digit totals
  uint32_t* raw;       // [kBins][tiles] counts
  uint32_t n, tiles;
  int shift;
};

// Digit counts of one wave tile (LDS atomics: counts do not depend on order).
template <bool FIRST>
__global__ __launch_bounds__(256) void csr_radix_hist_kernel(const RadixPass p) {
  __shared__ uint32_t wh[4][kBins];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t tile = blockIdx.x * 4 + wave;
  wh[wave][lane] = 0u;
  __syncthreads();
  if (tile < p.tiles) {
    for (int r = 0; r < kRounds; ++r) {
      const uint32_t i = tile * kTile + r * 64 + lane;
      if (i < p.n) {
        const uint32_t key = FIRST ? entry_key(p.pos, p.psb, p.pst, p.T, p.S, p.K, p.nk, i) : p.keys_in[i];
        atomicAdd(&wh[wave][(key >> p.shift) & (kBins - 1)], 1u);
      }
    }
  }
  __syncthreads();
  if (tile < p.tiles) {
    const uint32_t c = wh[wave][lane];
    p.hist[(uint32_t)lane * p.tiles + tile] = c;
    p.raw[(uint32_t)lane * p.tiles + tile] = c;
  }
}

// One workgroup per digit: in-place exclusive scan of that digit's tile counts (a row of
// hist), and the digit's total into totals[digit].
__global__ __launch_bounds__(kScanThreads) void csr_radix_scan_kernel(uint32_t* hist, uint32_t tiles,
                                                                      uint32_t* totals) {
  __shared__ uint32_t s_w[kScanThreads / 64];
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  uint32_t* row = hist + (size_t)blockIdx.x * tiles;
  uint32_t carry = 0;
  for (uint32_t base = 0; base < tiles; base += kScanThreads) {
    const uint32_t i = base + tid;
    const uint32_t v = i < tiles ? row[i] : 0u;
    uint32_t x = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const uint32_t y = __shfl_up(x, o);
      if (lane >= o) x += y;
    }
    if (lane == 63) s_w[wave] = x;
    __syncthreads();
    uint32_t before = carry, chunk = 0;
#pragma unroll
    for (int w = 0; w < kScanThreads / 64; ++w) {
      const uint32_t t = s_w[w];
      before += w < wave ? t : 0u;
      chunk += t;
    }
    if (i < tiles) row[i] = before + x - v;
    carry += chunk;
    __syncthreads();
  }
  if (tid == 0) totals[blockIdx.x] = carry;
}

// Stable scatter of one wave tile, staged through LDS so that the global writes come out
// as runs of consecutive slots per digit. Entries are taken in index order (round, lane);
// lanes with equal digits are ranked by ballots, lane d keeps the next tile-local slot of
// digit d, and the tile, ordered by digit in LDS, is then written out in order.
template <bool FIRST, bool LAST>
__global__ __launch_bounds__(256) void csr_radix_scatter_kernel(const RadixPass p) {
  __shared__ uint32_t wc[4][kBins];
  __shared__ int32_t wdelta[4][kBins];
  __shared__ uint32_t sk[4][kTile];
  __shared__ uint32_t sv[4][kTile];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t tile = blockIdx.x * 4 + wave;
  if (tile >= p.tiles) return;  // whole waves; only wave-local LDS below
  // Global first slot of digit `lane` in this tile: entries of smaller digits plus this
  // digit's entries in earlier tiles; tile-local first slot from this tile's counts.
  const uint32_t tot = p.hist[64u * p.tiles + lane];
  const uint32_t cnt = p.raw[(uint32_t)lane * p.tiles + tile];
  uint32_t below_d = tot, local = cnt;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t y = __shfl_up(below_d, o), z = __shfl_up(local, o);
    if (lane >= o) {
      below_d += y;
      local += z;
    }
  }
  local -= cnt;
  const uint32_t gstart = below_d - tot + p.hist[(uint32_t)lane * p.tiles + tile];
  wc[wave][lane] = 0u;
  wdelta[wave][lane] = (int32_t)(gstart - local);
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  uint32_t next = local;
  const uint64_t below = (1ull << lane) - 1ull;
  for (int r = 0; r < kRounds; ++r) {
    const uint32_t i = tile * kTile + r * 64 + lane;
    const bool live = i < p.n;
    uint32_t key = 0, val = i;
    if (live) {
      if constexpr (FIRST) {
        key = entry_key(p.pos, p.psb, p.pst, p.T, p.S, p.K, p.nk, i);
      } else {
        key = p.keys_in[i];
        val = p.vals_in[i];
      }
    }
    const int d = (int)((key >> p.shift) & (kBins - 1));
    uint64_t peers = __ballot(live);
#pragma unroll
    for (int bit = 0; bit < kRadixBits; ++bit) {
      const uint64_t bb = __ballot((d >> bit) & 1);
      peers &= ((d >> bit) & 1) ? bb : ~bb;
    }
    const uint32_t rank = (uint32_t)__popcll(peers & below);
    const uint32_t slot = (uint32_t)__shfl((int)next, d) + rank;  // < kTile
    if (live) {
      sk[wave][slot] = key;
      sv[wave][slot] = val;
      if (rank == 0) wc[wave][d] = (uint32_t)__popcll(peers);  // one writer per digit
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    next += wc[wave][lane];
    wc[wave][lane] = 0u;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
  // Write-out in tile-local slot order: slot i of digit d goes to i + (gstart_d - local_d).
  const uint32_t m = min((uint32_t)kTile, p.n - tile * kTile);
  for (uint32_t i = lane; i < m; i += 64) {
    const uint32_t key = sk[wave][i], val = sv[wave][i];
    const uint32_t g = (uint32_t)((int32_t)i + wdelta[wave][(key >> p.shift) & (kBins - 1)]);
    p.keys_out[g] = key;
    if constexpr (LAST) {
      const uint32_t row = val / (uint32_t)p.K;
      const int j = (int)(val - row * (uint32_t)p.K);
      const int t = (int)(row % (uint32_t)p.T);
      p.entries[g] = make_int2(t, j);
    } else {
      p.vals_out[g] = val;
    }
  }
}

// off[k] = first position of key k in the sorted keys (keys are <= nk, nk = invalid).
__global__ __launch_bounds__(256) void csr_bounds_kernel(const uint32_t* keys, uint32_t n, int nk, int* off) {
  const uint32_t i = blockIdx.x * 256 + threadIdx.x;
  if (i > n) return;
  const int lo = i == 0 ? -1 : (int)keys[i - 1];
  const int hi = i == n ? nk : (int)keys[i];
  for (int k = lo + 1; k <= hi; ++k) off[k] = (int)i;
}

__global__ __launch_bounds__(256) void csr_count_from_off_kernel(const int* off, int nk, int* count) {
  const int k = blockIdx.x * 256 + threadIdx.x;
  if (k < nk) count[k] = off[k + 1] - off[k];
}

// Single workgroup: exclusive scans of count, items and parts, 1024 keys per step.
__global__ __launch_bounds__(kScanThreads) void csr_scan_kernel(const int* count, int* off, int* item_off,
                                                                int* part_off, int nk, int* header) {
  __shared__ int s_w[3][kScanThreads / 64];
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  int ca = 0, cb = 0, cc = 0;  // carries
  for (int base = 0; base < nk; base += kScanThreads) {
    const int i = base + tid;
    const int c = i < nk ? count[i] : 0;
    const int it = i < nk ? items_of(c) : 0;
    const int pt = it > 1 ? it : 0;
    int xa = c, xb = it, xc = pt;
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
      s_w[0][wave] = xa;
      s_w[1][wave] = xb;
      s_w[2][wave] = xc;
    }
    __syncthreads();
    int ba = ca, bb = cb, bc = cc;
#pragma unroll
    for (int w = 0; w < kScanThreads / 64; ++w) {
      const int ta = s_w[0][w], tb = s_w[1][w], tc = s_w[2][w];
      if (w < wave) {
        ba += ta;
        bb += tb;
        bc += tc;
      }
      ca += ta;
      cb += tb;
      cc += tc;
    }
    if (i < nk) {
      off[i] = ba + xa - c;
      item_off[i] = bb + xb - it;
      part_off[i] = bc + xc - pt;
    }
    __syncthreads();
  }
  if (tid == 0) {
    off[nk] = ca;
    item_off[nk] = cb;
    part_off[nk] = cc;
    header[0] = cb;
    header[1] = cc;
  }
}

// One thread per key: writes the key of each of its work items.
__global__ __launch_bounds__(256) void csr_items_kernel(const int* item_off, int nk, int* item_key) {
  const int key = blockIdx.x * 256 + threadIdx.x;
  if (key >= nk) return;
  for (int i = item_off[key]; i < item_off[key + 1]; ++i) item_key[i] = key;
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
  L.total = o;
  o = 0;
  L.scratch = take(ne * 16);
  const size_t tiles = (ne + kTile - 1) / kTile;
  L.hist = take((tiles + 1) * 64 * 4);  // [64][tiles] counts + [64] digit totals
  L.raw = take(tiles * 64 * 4);         // [64][tiles] counts
  L.ws_total = o;
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

extern "C" size_t gw_kv_csr_build_workspace_size(int64_t B, int64_t T, int64_t S, int64_t K) {
  if (B <= 0 || T <= 0 || S <= 0 || K <= 0) return 256;
  return gw::csr_layout(B, T, S, K).ws_total;
}

extern "C" int gw_kv_csr_build(const int32_t* pos, int64_t pos_stride_b, int64_t pos_stride_t, int64_t B,
                               int64_t T, int64_t S, int64_t K, void* csr, size_t csr_bytes, void* workspace,
                               size_t workspace_bytes, void* stream) {
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
  GW_CHECK_ARG(workspace != nullptr && aligned16(workspace) && workspace_bytes >= L.ws_total,
               "the build needs a 16-byte aligned %zu-byte workspace, got %zu", L.ws_total, workspace_bytes);
  uint8_t* base = static_cast<uint8_t*>(csr);
  uint8_t* wbase = static_cast<uint8_t*>(workspace);
  int* header = reinterpret_cast<int*>(base + L.header);
  int* count = reinterpret_cast<int*>(base + L.count);
  int* off = reinterpret_cast<int*>(base + L.off);
  int* item_off = reinterpret_cast<int*>(base + L.item_off);
  int* part_off = reinterpret_cast<int*>(base + L.part_off);
  int* item_key = reinterpret_cast<int*>(base + L.item_key);
  int2* entries = reinterpret_cast<int2*>(base + L.entries);
  const int nk = (int)L.nk;
  const uint32_t n = (uint32_t)(B * T * K);
  uint32_t* keys_a = reinterpret_cast<uint32_t*>(wbase + L.scratch);
  uint32_t* vals_a = keys_a + n;
  uint32_t* keys_b = vals_a + n;
  uint32_t* vals_b = keys_b + n;
  // keys/vals pairs: pass p reads pair (p+1)%2 and writes pair p%2 (pass 0 reads pos).
  uint32_t* kp[2] = {keys_a, keys_b};
  uint32_t* vp[2] = {vals_a, vals_b};
  RadixPass rp{};
  rp.pos = pos;
  rp.psb = pos_stride_b;
  rp.pst = pos_stride_t;
  rp.T = (int)T;
  rp.S = (int)S;
  rp.K = (int)K;
  rp.nk = nk;
  rp.entries = entries;
  rp.hist = reinterpret_cast<uint32_t*>(wbase + L.hist);
  rp.raw = reinterpret_cast<uint32_t*>(wbase + L.raw);
  rp.n = n;
  rp.tiles = (n + kTile - 1) / kTile;
  int passes = 0;
  while ((1ll << (kRadixBits * passes)) <= (int64_t)nk) ++passes;  // keys 0..nk
  const dim3 tgrid((rp.tiles + 3) / 4);
  for (int ps = 0; ps < passes; ++ps) {
    rp.shift = kRadixBits * ps;
    rp.keys_in = kp[(ps + 1) & 1];
    rp.vals_in = vp[(ps + 1) & 1];
    rp.keys_out = kp[ps & 1];
    rp.vals_out = vp[ps & 1];
    const bool first = ps == 0, last = ps == passes - 1;
    if (first)
      hipLaunchKernelGGL((csr_radix_hist_kernel<true>), tgrid, dim3(256), 0, st, rp);
    else
      hipLaunchKernelGGL((csr_radix_hist_kernel<false>), tgrid, dim3(256), 0, st, rp);
    GW_HIP_LAUNCH_CHECK("csr_radix_hist_kernel");
    hipLaunchKernelGGL(csr_radix_scan_kernel, dim3(kBins), dim3(kScanThreads), 0, st, rp.hist, rp.tiles,
                       rp.hist + (size_t)kBins * rp.tiles);
    GW_HIP_LAUNCH_CHECK("csr_radix_scan_kernel");
    if (first && last)
      hipLaunchKernelGGL((csr_radix_scatter_kernel<true, true>), tgrid, dim3(256), 0, st, rp);
    else if (first)
      hipLaunchKernelGGL((csr_radix_scatter_kernel<true, false>), tgrid, dim3(256), 0, st, rp);
    else if (last)
      hipLaunchKernelGGL((csr_radix_scatter_kernel<false, true>), tgrid, dim3(256), 0, st, rp);
    else
      hipLaunchKernelGGL((csr_radix_scatter_kernel<false, false>), tgrid, dim3(256), 0, st, rp);
    GW_HIP_LAUNCH_CHECK("csr_radix_scatter_kernel");
  }
  const uint32_t* sorted_keys = kp[(passes - 1) & 1];
  hipLaunchKernelGGL(csr_bounds_kernel, dim3((n + 1 + 255) / 256), dim3(256), 0, st, sorted_keys, n, nk, off);
  GW_HIP_LAUNCH_CHECK("csr_bounds_kernel");
  hipLaunchKernelGGL(csr_count_from_off_kernel, dim3((nk + 255) / 256), dim3(256), 0, st, off, nk, count);
  GW_HIP_LAUNCH_CHECK("csr_count_from_off_kernel");
  hipLaunchKernelGGL(csr_scan_kernel, dim3(1), dim3(kScanThreads), 0, st, count, off, item_off, part_off, nk,
                     header);
  GW_HIP_LAUNCH_CHECK("csr_scan_kernel");
  hipLaunchKernelGGL(csr_items_kernel, dim3((nk + 255) / 256), dim3(256), 0, st, item_off, nk, item_key);
  GW_HIP_LAUNCH_CHECK("csr_items_kernel");
  return GW_OK;
}
