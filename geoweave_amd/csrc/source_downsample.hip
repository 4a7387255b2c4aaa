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
//    query: ballots compact the tokens into LDS, then the row is written once. The table
//    may differ per batch element (subcell_static_pack4), and an output row may read
//    another row's choice (qk_sym_x2_broadcast: every fine query reads its coarse query's).
//
// The other strategies of the reference (:3599-4078), each one workgroup per query row:
//  * gw_source_downsample_rerank (exact_rerank): the fine tokens of the chosen rows are
//    scored exactly with the indexer formula and the top target of them kept (block radix
//    select, ties in candidate order); a row with fewer valid candidates than the target
//    raises the fail flag, and the host grows the coarse budget as the reference does.
//  * gw_source_downsample_subcell_top1: the chosen special/edge rows give their token;
//    the remaining budget goes to the best-scoring 2 x 2 sub-cells of the chosen cells
//    (exact scores against the pooled sub-cell keys), four tokens each.
//  * gw_source_downsample_static_pack4: per batch element, the sub-cell each cell expands
//    to under subcell_static_pack4 (largest head-mean of the pooled sub-cell gates).
#include "gw_common.h"
#include "gw_select.h"
#include "gw_sort.h"

namespace gw {
namespace {

constexpr int kExpandMaxTarget = 4096;
constexpr int kExpandMaxKc = 4096;
constexpr int kSortRegsMax = 16;  // register bitonic sort up to 64 * 16 chosen rows

// Rounds to the 16-bit type and back.
template <typename E>
__device__ __forceinline__ float round16(float x) {
  float lo, hi;
  unpack2(E{}, pack1(E{}, x), lo, hi);
  return lo;
}

template <typename E>
__global__ __launch_bounds__(256) void sd_pool_kernel(const uint16_t* k, const uint16_t* w, int S, int E8, int Hi,
                                                      const int32_t* stf, int L, int M, uint16_t* sk,
                                                      uint16_t* sw, int round_sum) {
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
    if (c == 0 && w != nullptr) {
      for (int h = 0; h < Hi && h < 8; ++h) {
        const uint32_t u = w[((int64_t)b * S + tok) * Hi + h];
        float lo, hi;
        unpack2(E{}, u, lo, hi);
        wacc[h] += lo;
      }
    }
  }
  const float n = cnt > 0 ? (float)cnt : 1.f;
  // round_sum: the sum is a 16-bit tensor before the division (the reference's query mean).
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = (round_sum ? round16<E>(acc[e]) : acc[e]) / n;
  *reinterpret_cast<uint4*>(sk + ((int64_t)b * L + r) * row_elems + c * 8) = pack8<E>(acc);
  if (c == 0 && w != nullptr) {
    for (int h = 0; h < Hi && h < 8; ++h)
      sw[((int64_t)b * L + r) * Hi + h] = (uint16_t)pack1(E{}, (round_sum ? round16<E>(wacc[h]) : wacc[h]) / n);
  }
}

struct ExpandParams {
  const int32_t* cidx;
  const uint16_t* cscore;  // nullable: order the chosen rows by (score desc, row asc)
  int64_t csb, cst;
  int T, Kc;
  const int32_t* row_map;  // nullable: output row t of a batch element reads chosen row row_map[t]
  int Tout;                // output rows per batch element
  const int32_t* stf;
  int64_t tsb;             // table elements between batch elements (0: one shared table)
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
  const int64_t b = row / p.Tout, to = row - b * p.Tout;
  const int64_t t = p.row_map != nullptr ? (int64_t)p.row_map[to] : to;
  const int32_t* ci = p.cidx + b * p.csb + t * p.cst;
  const int32_t* stf = p.stf + b * p.tsb;
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
      if (s >= 0 && s < p.L) tok = stf[(int64_t)s * p.M + m];
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


// ---------------------------------------------------------------------------------------
// exact_rerank and subcell_top1: one 256-thread workgroup per query row.
// ---------------------------------------------------------------------------------------
constexpr int kRerankMaxCand = 8192;  // chosen rows x tokens per row
constexpr int kMaxQElems = 1024;      // Hi * Di of the indexer query
constexpr int kSubcellMaxKc = 2048;   // chosen rows (subcell_top1)
constexpr int kSubcellMaxUnits = 8192;  // chosen rows x sub-cells per cell

// Indexer score of the query staged in LDS (16-bit, [Hi][Di] as 16-byte chunks) against
// one key row: sum_h w_h * relu(scale * <q_h, k_h>), fp32 (products exact, dot2 sums).
template <typename E>
__device__ __forceinline__ float row_score(const uint4* qs, const uint16_t* krow, const uint16_t* wrow, int Hi,
                                           int D8, float scale) {
  const uint4* kp = reinterpret_cast<const uint4*>(krow);
  float s = 0.f;
  for (int h = 0; h < Hi; ++h) {
    float z = 0.f;
    for (int c = 0; c < D8; ++c) {
      const uint4 a = qs[h * D8 + c], b = kp[h * D8 + c];
      z = dot2(E{}, a.x, b.x, z);
      z = dot2(E{}, a.y, b.y, z);
      z = dot2(E{}, a.z, b.z, z);
      z = dot2(E{}, a.w, b.w, z);
    }
    float wv, unused;
    unpack2(E{}, (uint32_t)wrow[h], wv, unused);
    s += fmaxf(scale * z, 0.f) * wv;
  }
  return s;
}

// Order key of a chosen row for the canonical expansion order: score descending, row
// ascending (ascending sort of (~orderable(score) << 32 | row)).
template <typename E>
__device__ __forceinline__ uint64_t chosen_key(uint16_t score_bits, int32_t row) {
  float sc, unused;
  unpack2(E{}, (uint32_t)score_bits, sc, unused);
  return ((uint64_t)(~f2key(sc)) << 32) | (uint32_t)row;
}

// Ascending bitonic sort of P (a power of two) keys in LDS by the whole block.
__device__ void block_bitonic_sort(uint64_t* keys, int P) {
  for (int kk = 2; kk <= P; kk <<= 1) {
    for (int j = kk >> 1; j > 0; j >>= 1) {
      for (int i = threadIdx.x; i < P; i += blockDim.x) {
        const int ixj = i ^ j;
        if (ixj > i) {
          const uint64_t a = keys[i], c = keys[ixj];
          if ((a > c) == ((i & kk) == 0)) {
            keys[i] = c;
            keys[ixj] = a;
          }
        }
      }
      __syncthreads();
    }
  }
}

struct RerankParams {
  const uint16_t* q;  // [B, T, Hi * Di]
  const uint16_t* k;  // [B, S, Hi * Di]   (subcell_top1: pooled sub-cell keys [B, C * G, ...])
  const uint16_t* w;  // [B, S, Hi]        (subcell_top1: [B, C * G, Hi])
  int T, S, Hi, D8;
  const int32_t* cidx;
  const uint16_t* cscore;  // subcell_top1: chosen rows' scores (expansion order)
  int64_t csb, cst;
  int Kc, P;
  const int32_t* stf;
  int L, M;
  int off;             // subcell_top1: first coarse row
  const int32_t* sub;  // subcell_top1: [C * G, W] tokens per sub-cell
  int C, G, W;
  int target;
  float scale;
  int32_t* out;  // [B, T, target]
  int* fail;     // set to 1 when a row has fewer candidates than the target
};

template <typename E>
__global__ __launch_bounds__(256) void sd_rerank_kernel(const RerankParams p) {
  __shared__ uint4 qs[kMaxQElems / 8];
  __shared__ int32_t cand[kRerankMaxCand];
  __shared__ uint32_t keys[kRerankMaxCand];
  __shared__ SelectShared sh;
  __shared__ int nvalid;
  const int tid = threadIdx.x;
  const int64_t row = blockIdx.x;
  const int64_t b = row / p.T, t = row - b * p.T;
  const int HD8 = p.Hi * p.D8;
  const uint4* qrow = reinterpret_cast<const uint4*>(p.q) + row * HD8;
  for (int i = tid; i < HD8; i += 256) qs[i] = qrow[i];
  if (tid == 0) nvalid = 0;
  __syncthreads();
  // Candidates in (chosen row, slot) order.
  const int32_t* ci = p.cidx + b * p.csb + t * p.cst;
  const int n = p.Kc * p.M;
  int cnt = 0;
  for (int i = tid; i < n; i += 256) {
    const int c = i / p.M, m = i - c * p.M;
    const int r = ci[c];
    int tok = -1;
    if (r >= 0 && r < p.L) tok = p.stf[(int64_t)r * p.M + m];
    if (tok >= p.S) tok = -1;
    cand[i] = tok;
    cnt += tok >= 0;
  }
  if (cnt) atomicAdd(&nvalid, cnt);
  __syncthreads();
  if (nvalid < p.target) {  // uniform
    if (tid == 0) atomicOr(p.fail, 1);
    return;
  }
  const uint16_t* kb = p.k + (int64_t)b * p.S * (HD8 * 8);
  const uint16_t* wb = p.w + (int64_t)b * p.S * p.Hi;
  for (int i = tid; i < n; i += 256) {
    const int tok = cand[i];
    // Empty slots get key 0, below the key of every score that is not a NaN.
    keys[i] = tok >= 0 ? f2key(row_score<E>(qs, kb + (int64_t)tok * HD8 * 8, wb + (int64_t)tok * p.Hi, p.Hi, p.D8,
                                            p.scale))
                       : 0u;
  }
  __syncthreads();
  auto key_at = [&](int i) { return keys[i]; };
  int take_eq = 0;
  const uint32_t kth = block_radix_select(key_at, n, p.target, sh, take_eq);
  int32_t* o = p.out + row * p.target;
  block_emit_topk(key_at, n, p.target, kth, take_eq, [&](int slot, int i) { o[slot] = cand[i]; }, sh);
}

template <typename E>
__global__ __launch_bounds__(256) void sd_subcell_top1_kernel(const RerankParams p) {
  __shared__ uint4 qs[kMaxQElems / 8];
  __shared__ uint64_t ord[kSubcellMaxKc];      // chosen rows, sorted
  __shared__ int32_t blk[kSubcellMaxKc];       // cells of the chosen coarse rows, in order
  __shared__ uint32_t keys[kSubcellMaxUnits];  // sub-cell score keys (0: not selectable)
  __shared__ SelectShared sh;
  __shared__ int totals[3];
  const int tid = threadIdx.x;
  const int64_t row = blockIdx.x;
  const int64_t b = row / p.T, t = row - b * p.T;
  const int HD8 = p.Hi * p.D8;
  const uint4* qrow = reinterpret_cast<const uint4*>(p.q) + row * HD8;
  for (int i = tid; i < HD8; i += 256) qs[i] = qrow[i];
  // Expansion order of the chosen rows: score descending, row ascending.
  const int32_t* ci = p.cidx + b * p.csb + t * p.cst;
  const uint16_t* cs = p.cscore + b * p.csb + t * p.cst;
  for (int i = tid; i < p.P; i += 256) ord[i] = i < p.Kc ? chosen_key<E>(cs[i], ci[i]) : ~0ull;
  __syncthreads();
  block_bitonic_sort(ord, p.P);
  // Singles (chosen special/edge rows with a token) and cells, each counted over a
  // contiguous range of the order per thread.
  const int ch = (p.Kc + 255) / 256;
  const int c0 = min(p.Kc, tid * ch), c1 = min(p.Kc, c0 + ch);
  int ns = 0, nb = 0;
  for (int c = c0; c < c1; ++c) {
    const int r = (int)(uint32_t)ord[c];
    if (r < 0 || r >= p.L) continue;
    if (r < p.off) ns += p.stf[(int64_t)r * p.M] >= 0;
    else nb += 1;
  }
  int os, ob;
  block_excl_scan2(ns, nb, os, ob, sh);
  int32_t* o = p.out + row * p.target;
  for (int c = c0; c < c1; ++c) {
    const int r = (int)(uint32_t)ord[c];
    if (r < 0 || r >= p.L) continue;
    if (r < p.off) {
      const int tok = p.stf[(int64_t)r * p.M];
      if (tok >= 0) {
        if (os < p.target) o[os] = tok;
        ++os;
      }
    } else {
      blk[ob++] = r - p.off;
    }
  }
  if (c1 == p.Kc && c0 <= c1 && (c0 < c1 || tid == 0)) {
    // the thread holding the end of the order (or thread 0 when Kc = 0) has the totals
    totals[0] = os;
    totals[1] = ob;
  }
  __syncthreads();
  const int n_single = totals[0], n_cell = totals[1];
  const int n_units = n_cell * p.G;
  // Sub-cell scores of the chosen cells (units in order: cell, then sub-cell).
  const uint16_t* kb = p.k + (int64_t)b * p.C * p.G * (HD8 * 8);
  const uint16_t* wb = p.w + (int64_t)b * p.C * p.G * p.Hi;
  int nv = 0;
  for (int u = tid; u < n_units; u += 256) {
    const int cell = blk[u / p.G], g = u - (u / p.G) * p.G;
    const int64_t sc = (int64_t)cell * p.G + g;
    uint32_t key = 0u;
    if (p.sub[sc * p.W] >= 0) {
      ++nv;
      const float v = row_score<E>(qs, kb + sc * HD8 * 8, wb + sc * p.Hi, p.Hi, p.D8, p.scale);
      if (isfinite(v)) key = f2key(v);  // a non-finite score is never kept
    }
    keys[u] = key;
  }
  if (tid == 0) totals[2] = 0;
  __syncthreads();
  if (nv) atomicAdd(&totals[2], nv);
  __syncthreads();
  const int remain = max(p.target - n_single, 0);
  const int keep = min((remain + p.W - 1) / p.W, totals[2]);
  int n_tok = 0;
  if (keep > 0) {
    auto key_at = [&](int i) { return keys[i]; };
    int take_eq = 0;
    const uint32_t kth = block_radix_select(key_at, n_units, keep, sh, take_eq);
    // The kept sub-cells in unit order: keys above kth, and the first take_eq equal to it.
    const int uch = (n_units + 255) / 256;
    const int u0 = min(n_units, tid * uch), u1 = min(n_units, u0 + uch);
    int cg = 0, ce = 0;
    for (int u = u0; u < u1; ++u) {
      cg += keys[u] > kth;
      ce += keys[u] == kth;
    }
    int og, oe;
    block_excl_scan2(cg, ce, og, oe, sh);
    int ntok = 0;
    int e = oe;
    for (int u = u0; u < u1; ++u) {
      const uint32_t kk = keys[u];
      bool sel = kk > kth;
      if (kk == kth) sel = e++ < take_eq;
      if (sel && kk != 0u) {
        const int64_t sc = (int64_t)blk[u / p.G] * p.G + (u - (u / p.G) * p.G);
        for (int j = 0; j < p.W; ++j) ntok += p.sub[sc * p.W + j] >= 0;
      }
    }
    int ot, unused;
    block_excl_scan2(ntok, 0, ot, unused, sh);
    int slot = n_single + ot;
    e = oe;
    for (int u = u0; u < u1; ++u) {
      const uint32_t kk = keys[u];
      bool sel = kk > kth;
      if (kk == kth) sel = e++ < take_eq;
      if (sel && kk != 0u) {
        const int64_t sc = (int64_t)blk[u / p.G] * p.G + (u - (u / p.G) * p.G);
        for (int j = 0; j < p.W; ++j) {
          const int tok = p.sub[sc * p.W + j];
          if (tok >= 0) {
            if (slot < p.target) o[slot] = tok;
            ++slot;
          }
        }
      }
    }
    if (u1 == n_units && (u0 < u1 || tid == 0)) totals[0] = ot + ntok;  // the end of the unit order
    __syncthreads();
    n_tok = totals[0];
  }
  if (tid == 0 && n_single + n_tok < p.target) atomicOr(p.fail, 1);
}

// subcell_static_pack4 table: row r < off keeps its token; cell row off + c expands to
// the sub-cell g with the largest head-mean of its pooled gates (fp32 sum times 1 / Hi,
// rounded to the 16-bit type; the first on ties).
template <typename E>
__global__ __launch_bounds__(256) void sd_static_pack_kernel(const uint16_t* sw, int C, int G, int Hi,
                                                             const int32_t* stf, int L, int M, int off,
                                                             const int32_t* sub, int W, int32_t* table) {
  const int r = blockIdx.x * 256 + threadIdx.x;
  const int b = blockIdx.y;
  if (r >= L) return;
  int32_t* o = table + ((int64_t)b * L + r) * W;
  if (r < off) {
    o[0] = stf[(int64_t)r * M];
    for (int j = 1; j < W; ++j) o[j] = -1;
    return;
  }
  const int c = r - off;
  const float inv = 1.f / (float)Hi;
  int best = 0;
  float bestv = 0.f;
  for (int g = 0; g < G; ++g) {
    const uint16_t* wr = sw + (((int64_t)b * C + c) * G + g) * Hi;
    float acc = 0.f;
    for (int h = 0; h < Hi; ++h) {
      float v, unused;
      unpack2(E{}, (uint32_t)wr[h], v, unused);
      acc += v;
    }
    const float m = round16<E>(acc * inv);
    if (g == 0 || m > bestv) {
      best = g;
      bestv = m;
    }
  }
  for (int j = 0; j < W; ++j) o[j] = sub[((int64_t)c * G + best) * W + j];
}

}  // namespace
}  // namespace gw

extern "C" int gw_source_downsample_pool(int dtype, const void* k, const void* w, int64_t B, int64_t S,
                                         int64_t Hi, int64_t Di, const int32_t* source_to_fine, int64_t L,
                                         int64_t M, int round_sum, void* source_k, void* source_w,
                                         void* stream) {
  using namespace gw;
  clear_error();
  GW_CHECK_ARG(dtype == GW_DTYPE_BF16 || dtype == GW_DTYPE_FP16, "unsupported dtype code %d", dtype);
  GW_CHECK_ARG(B >= 0 && S >= 1 && L >= 0 && M >= 1, "invalid sizes B=%lld S=%lld L=%lld M=%lld", (long long)B,
               (long long)S, (long long)L, (long long)M);
  GW_CHECK_ARG(Hi >= 1 && Hi <= 8 && Di >= 8 && (Hi * Di) % 8 == 0,
               "indexer heads x dim %lld x %lld not supported (Hi <= 8, Hi*Di a multiple of 8)", (long long)Hi,
               (long long)Di);
  if (B == 0 || L == 0) return GW_OK;
  GW_CHECK_ARG(k && source_to_fine && source_k && (w == nullptr) == (source_w == nullptr), "null tensor pointer");
  GW_CHECK_ARG(aligned16(k) && aligned16(source_k), "k and source_k must be 16-byte aligned");
  GW_CHECK_ARG(B <= 65535 && S < (1ll << 31) && L * Hi * Di / 8 < (1ll << 31), "size exceeds grid or int32 range");
  const int E8 = (int)(Hi * Di / 8);
  const dim3 grid((unsigned)((L * E8 + 255) / 256), (unsigned)B);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == GW_DTYPE_BF16)
    hipLaunchKernelGGL(sd_pool_kernel<BF16>, grid, dim3(256), 0, st, static_cast<const uint16_t*>(k),
                       static_cast<const uint16_t*>(w), (int)S, E8, (int)Hi, source_to_fine, (int)L, (int)M,
                       static_cast<uint16_t*>(source_k), static_cast<uint16_t*>(source_w), round_sum ? 1 : 0);
  else
    hipLaunchKernelGGL(sd_pool_kernel<FP16>, grid, dim3(256), 0, st, static_cast<const uint16_t*>(k),
                       static_cast<const uint16_t*>(w), (int)S, E8, (int)Hi, source_to_fine, (int)L, (int)M,
                       static_cast<uint16_t*>(source_k), static_cast<uint16_t*>(source_w), round_sum ? 1 : 0);
  GW_HIP_LAUNCH_CHECK("sd_pool_kernel");
  return GW_OK;
}

extern "C" int gw_source_downsample_expand(int dtype, const int32_t* coarse_idx, const void* coarse_scores,
                                           int64_t idx_stride_b, int64_t idx_stride_t,
                                           int64_t B, int64_t T, int64_t Kc, const int32_t* source_to_fine,
                                           int64_t table_stride_b, int64_t L, int64_t M, int round_robin,
                                           int64_t target, int64_t pad_window, const int32_t* row_map,
                                           int64_t T_out, int32_t* out, void* stream) {
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
  GW_CHECK_ARG(table_stride_b >= 0, "table_stride_b must be >= 0");
  if (row_map == nullptr) T_out = T;
  GW_CHECK_ARG(T_out >= 0, "invalid T_out %lld", (long long)T_out);
  if (B == 0 || T_out == 0) return GW_OK;
  GW_CHECK_ARG(T >= 1, "row_map given with no chosen rows");
  GW_CHECK_ARG(coarse_idx && source_to_fine && out, "null tensor pointer");
  GW_CHECK_ARG(B * T_out < (1ll << 31) && Kc * M < (1ll << 30) && L * M < (1ll << 31), "size exceeds int32 range");
  ExpandParams p;
  p.cidx = coarse_idx;
  p.cscore = static_cast<const uint16_t*>(coarse_scores);
  p.csb = idx_stride_b;
  p.cst = idx_stride_t;
  p.T = (int)T;
  p.Kc = (int)Kc;
  p.row_map = row_map;
  p.Tout = (int)T_out;
  p.stf = source_to_fine;
  p.tsb = table_stride_b;
  p.L = (int)L;
  p.M = (int)M;
  p.round_robin = round_robin ? 1 : 0;
  p.target = (int)target;
  p.window = (int)(pad_window < target ? pad_window : target);
  p.out = out;
  p.rows = B * T_out;
  size_t pow2 = 1;
  while ((int64_t)pow2 < Kc) pow2 <<= 1;
  p.P = (int)pow2;
  const size_t words = (size_t)((target + 1) & ~1ll) + (coarse_scores ? (size_t)((Kc + 1) & ~1ll) : 0);
  const size_t lds = ((words + 1) & ~(size_t)1) * 4 + (coarse_scores && pow2 > 64 * kSortRegsMax ? pow2 * 8 : 0);
  if (dtype == GW_DTYPE_BF16)
    hipLaunchKernelGGL(sd_expand_kernel<BF16>, dim3((unsigned)(B * T_out)), dim3(64), lds,
                       static_cast<hipStream_t>(stream), p);
  else
    hipLaunchKernelGGL(sd_expand_kernel<FP16>, dim3((unsigned)(B * T_out)), dim3(64), lds,
                       static_cast<hipStream_t>(stream), p);
  GW_HIP_LAUNCH_CHECK("sd_expand_kernel");
  return GW_OK;
}

namespace {

int check_query_shape(int64_t Hi, int64_t Di) {
  using namespace gw;
  if (Hi < 1 || Hi > 8 || Di < 8 || Di % 8 != 0 || Hi * Di > kMaxQElems)
    return set_error(GW_ERR_UNSUPPORTED, "indexer heads x dim %lld x %lld not supported (Hi <= 8, Di a multiple "
                     "of 8, Hi * Di <= %d)", (long long)Hi, (long long)Di, kMaxQElems);
  return GW_OK;
}

}  // namespace

extern "C" int gw_source_downsample_rerank(int dtype, const void* q, const void* k, const void* w, int64_t B,
                                           int64_t T, int64_t S, int64_t Hi, int64_t Di, const int32_t* coarse_idx,
                                           int64_t idx_stride_b, int64_t idx_stride_t, int64_t Kc,
                                           const int32_t* source_to_fine, int64_t L, int64_t M, int64_t target,
                                           float scale, int32_t* out, int* fail, void* stream) {
  using namespace gw;
  clear_error();
  GW_CHECK_ARG(dtype == GW_DTYPE_BF16 || dtype == GW_DTYPE_FP16, "unsupported dtype code %d", dtype);
  GW_CHECK_ARG(B >= 0 && T >= 0 && S >= 1 && Kc >= 1 && L >= 1 && M >= 1 && target >= 1,
               "invalid sizes B=%lld T=%lld S=%lld Kc=%lld L=%lld M=%lld target=%lld", (long long)B, (long long)T,
               (long long)S, (long long)Kc, (long long)L, (long long)M, (long long)target);
  if (int rc = check_query_shape(Hi, Di)) return rc;
  if (Kc * M > kRerankMaxCand)
    return set_error(GW_ERR_UNSUPPORTED, "%lld candidates (chosen rows x %lld) exceed the supported maximum %d",
                     (long long)(Kc * M), (long long)M, kRerankMaxCand);
  if (B == 0 || T == 0) return GW_OK;
  GW_CHECK_ARG(q && k && w && coarse_idx && source_to_fine && out && fail, "null tensor pointer");
  GW_CHECK_ARG(aligned16(q) && aligned16(k), "q and k must be 16-byte aligned");
  GW_CHECK_ARG(B * T < (1ll << 31) && S < (1ll << 31) && L * M < (1ll << 31), "size exceeds int32 range");
  RerankParams p{};
  p.q = static_cast<const uint16_t*>(q);
  p.k = static_cast<const uint16_t*>(k);
  p.w = static_cast<const uint16_t*>(w);
  p.T = (int)T;
  p.S = (int)S;
  p.Hi = (int)Hi;
  p.D8 = (int)(Di / 8);
  p.cidx = coarse_idx;
  p.csb = idx_stride_b;
  p.cst = idx_stride_t;
  p.Kc = (int)Kc;
  p.stf = source_to_fine;
  p.L = (int)L;
  p.M = (int)M;
  p.target = (int)target;
  p.scale = scale;
  p.out = out;
  p.fail = fail;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == GW_DTYPE_BF16)
    hipLaunchKernelGGL(sd_rerank_kernel<BF16>, dim3((unsigned)(B * T)), dim3(256), 0, st, p);
  else
    hipLaunchKernelGGL(sd_rerank_kernel<FP16>, dim3((unsigned)(B * T)), dim3(256), 0, st, p);
  GW_HIP_LAUNCH_CHECK("sd_rerank_kernel");
  return GW_OK;
}

extern "C" int gw_source_downsample_subcell_top1(int dtype, const void* q, const void* sub_k, const void* sub_w,
                                                 int64_t B, int64_t T, int64_t C, int64_t G, int64_t Hi, int64_t Di,
                                                 const int32_t* coarse_idx, const void* coarse_scores,
                                                 int64_t idx_stride_b, int64_t idx_stride_t, int64_t Kc,
                                                 const int32_t* source_to_fine, int64_t L, int64_t M,
                                                 int64_t first_cell_row, const int32_t* subcell_to_fine, int64_t W,
                                                 int64_t target, float scale, int32_t* out, int* fail,
                                                 void* stream) {
  using namespace gw;
  clear_error();
  GW_CHECK_ARG(dtype == GW_DTYPE_BF16 || dtype == GW_DTYPE_FP16, "unsupported dtype code %d", dtype);
  GW_CHECK_ARG(B >= 0 && T >= 0 && C >= 0 && G >= 1 && Kc >= 1 && L >= 1 && M >= 1 && W >= 1 && target >= 1 &&
                   first_cell_row >= 0 && first_cell_row + C == L,
               "invalid sizes B=%lld T=%lld C=%lld G=%lld Kc=%lld L=%lld M=%lld W=%lld target=%lld first=%lld",
               (long long)B, (long long)T, (long long)C, (long long)G, (long long)Kc, (long long)L, (long long)M,
               (long long)W, (long long)target, (long long)first_cell_row);
  if (int rc = check_query_shape(Hi, Di)) return rc;
  if (Kc > kSubcellMaxKc || Kc * G > kSubcellMaxUnits)
    return set_error(GW_ERR_UNSUPPORTED, "%lld chosen rows (x %lld sub-cells) exceed the supported maximum %d (%d)",
                     (long long)Kc, (long long)G, kSubcellMaxKc, kSubcellMaxUnits);
  if (B == 0 || T == 0) return GW_OK;
  GW_CHECK_ARG(q && (C == 0 || (sub_k && sub_w && subcell_to_fine)) && coarse_idx && coarse_scores &&
                   source_to_fine && out && fail,
               "null tensor pointer");
  GW_CHECK_ARG(aligned16(q) && (C == 0 || aligned16(sub_k)), "q and sub_k must be 16-byte aligned");
  GW_CHECK_ARG(B * T < (1ll << 31) && C * G * W < (1ll << 31) && L * M < (1ll << 31), "size exceeds int32 range");
  RerankParams p{};
  p.q = static_cast<const uint16_t*>(q);
  p.k = static_cast<const uint16_t*>(sub_k);
  p.w = static_cast<const uint16_t*>(sub_w);
  p.T = (int)T;
  p.Hi = (int)Hi;
  p.D8 = (int)(Di / 8);
  p.cidx = coarse_idx;
  p.cscore = static_cast<const uint16_t*>(coarse_scores);
  p.csb = idx_stride_b;
  p.cst = idx_stride_t;
  p.Kc = (int)Kc;
  int P = 1;
  while (P < Kc) P <<= 1;
  p.P = P;
  p.stf = source_to_fine;
  p.L = (int)L;
  p.M = (int)M;
  p.off = (int)first_cell_row;
  p.sub = subcell_to_fine;
  p.C = (int)C;
  p.G = (int)G;
  p.W = (int)W;
  p.target = (int)target;
  p.scale = scale;
  p.out = out;
  p.fail = fail;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == GW_DTYPE_BF16)
    hipLaunchKernelGGL(sd_subcell_top1_kernel<BF16>, dim3((unsigned)(B * T)), dim3(256), 0, st, p);
  else
    hipLaunchKernelGGL(sd_subcell_top1_kernel<FP16>, dim3((unsigned)(B * T)), dim3(256), 0, st, p);
  GW_HIP_LAUNCH_CHECK("sd_subcell_top1_kernel");
  return GW_OK;
}

extern "C" int gw_source_downsample_static_pack4(int dtype, const void* sub_w, int64_t B, int64_t C, int64_t G,
                                                 int64_t Hi, const int32_t* source_to_fine, int64_t L, int64_t M,
                                                 int64_t first_cell_row, const int32_t* subcell_to_fine, int64_t W,
                                                 int32_t* table, void* stream) {
  using namespace gw;
  clear_error();
  GW_CHECK_ARG(dtype == GW_DTYPE_BF16 || dtype == GW_DTYPE_FP16, "unsupported dtype code %d", dtype);
  GW_CHECK_ARG(B >= 0 && C >= 0 && G >= 1 && Hi >= 1 && L >= 1 && M >= 1 && W >= 1 && first_cell_row >= 0 &&
                   first_cell_row + C == L,
               "invalid sizes B=%lld C=%lld G=%lld Hi=%lld L=%lld M=%lld W=%lld first=%lld", (long long)B,
               (long long)C, (long long)G, (long long)Hi, (long long)L, (long long)M, (long long)W,
               (long long)first_cell_row);
  if (B == 0) return GW_OK;
  GW_CHECK_ARG((C == 0 || (sub_w && subcell_to_fine)) && source_to_fine && table, "null tensor pointer");
  GW_CHECK_ARG(B <= 65535 && L * W < (1ll << 31) && C * G * Hi < (1ll << 31), "size exceeds grid or int32 range");
  const dim3 grid((unsigned)((L + 255) / 256), (unsigned)B);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == GW_DTYPE_BF16)
    hipLaunchKernelGGL(sd_static_pack_kernel<BF16>, grid, dim3(256), 0, st, static_cast<const uint16_t*>(sub_w),
                       (int)C, (int)G, (int)Hi, source_to_fine, (int)L, (int)M, (int)first_cell_row, subcell_to_fine,
                       (int)W, table);
  else
    hipLaunchKernelGGL(sd_static_pack_kernel<FP16>, grid, dim3(256), 0, st, static_cast<const uint16_t*>(sub_w),
                       (int)C, (int)G, (int)Hi, source_to_fine, (int)L, (int)M, (int)first_cell_row, subcell_to_fine,
                       (int)W, table);
  GW_HIP_LAUNCH_CHECK("sd_static_pack_kernel");
  return GW_OK;
}
