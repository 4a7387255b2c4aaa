// Lightning-indexer backward as masked dense passes on the matrix cores (gfx950, bf16, Di = 64).
//
// Math (reference _indexer_topk_bwd_kernel,
// easyvolcap/utils/custom_indexer/sparse_topk_indexer.py:1847-1944), per head h, query t and
// selected key s = idx[b,t,j] with upstream gradient g = grad[b,t,j]:
//   z = scale q_t.k_s,   f = g w_s [z > 0] scale
//   dq_t += f k_s,   dk_s += f q_t,   dw_s += g relu(z)
// With G[t,s] = g at the selected pairs (0 elsewhere), Z = Q K^T (unscaled) and
// F = G o [Z > 0]:
//   dQ = scale F (w o K)         dK = scale w o (F^T Q)        dw_s = scale k_s . (F^T Q)_s
// (the last because sum_t F[t,s] Z[t,s] = k_s . sum_t F[t,s] q_t). Every pair (t, s) is
// computed on the matrix cores, like the masked dense attention backward; G enters as a tile
// gathered from the key-ordered gradients, so unselected pairs contribute exactly zero.
//
//  idxd_prep_kernel   per 8 queries: selection words in natural bit order,
//                     the number of selected keys of the row before every 32-key block, and
//                     the row's gradients in key order (gs[b][t][rank]); a position listed
//                     twice in a row flags the batch element in route[b].
//  idxd_t_kernel      q^T and (w o k)^T in the operand order of the products (rows permuted
//                     within every 16); a non-finite q, k, w or w k flags route[b].
//  idxd_pass_kernel   <false>: query-major, dQ^T += (w o K)^T F^T per 32-key tile;
//                     <true>:  key-major,  dK^T += Q^T F per 32-query tile, dw from dK^T.
//                     Persistent workgroups split the (row group, tile) iterations evenly
//                     (stream-K); a row group cut between workgroups leaves fp32 partials.
//  idxd_fixup_kernel  sums the partials of cut row groups in workgroup order.
// No atomics on gradients: every sum has a fixed order and the backward is reproducible.
// A batch element flagged in route[b] is left untouched; the caller computes it with the CSR
// backward (gw_indexer_topk_bwd).
#include <math.h>

#include <algorithm>
#include <mutex>

#include "gw_common.h"
#include "gw_dense.h"

namespace gw {
namespace {

constexpr int kXD = 64;            // head dim
constexpr int kXRows = 256;        // stationary rows per row group (4 waves x 2 blocks of 32)
constexpr int kXMaxS = 65536;      // keys: the prep kernel holds a row's words in LDS
constexpr int kXMaxK = 2048;
constexpr int kPrepQ = 8;          // queries per prep workgroup

__global__ __launch_bounds__(256) void idxd_clear_kernel(int* __restrict__ route, int B) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < B) route[i] = 0;
}

// ---------------------------------------------------------------------------------------
// Prep: words[b][t / 8][kb][t % 8] bit i = query t selected key 32 kb + i; pre (same
// layout) = number of keys of row t selected below key 32 kb; gs[b][t][r] = the gradient of
// the row's r-th selected key in increasing key order (r < the row's count; the rest of the
// row is zero).
// Rows t in [T, tpad) get zero words. LDS: words [nsub][9], prefixes [nsub][8] (u16), the
// 8 rows of gs [8][K].
// ---------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void idxd_prep_kernel(const int32_t* __restrict__ idx,
                                                        const uint16_t* __restrict__ grad, int T, int S, int K,
                                                        int nsub, int tpad, int vec, uint32_t* __restrict__ words_g,
                                                        uint16_t* __restrict__ pre_g, uint16_t* __restrict__ gs,
                                                        int* __restrict__ route) {
  extern __shared__ __align__(16) uint32_t lds[];
  constexpr int RW = kPrepQ + 1;
  const int off_pre = (nsub * RW + 3) & ~3;              // in words
  const int off_g = off_pre + ((nsub * kPrepQ / 2 + 3) & ~3);
  uint32_t* words = lds;
  uint16_t* pre = reinterpret_cast<uint16_t*>(lds + off_pre);
  uint16_t* grow = reinterpret_cast<uint16_t*>(lds + off_g);
  __shared__ int dup_any;
  const int tid = threadIdx.x;
  const int q0 = blockIdx.x * kPrepQ, b = blockIdx.y;
  {
    const int n4 = (off_g + (kPrepQ * K + 1) / 2 + 3) >> 2;  // words, prefixes and gs rows
    for (int i = tid; i < n4; i += 256) reinterpret_cast<uint4*>(lds)[i] = make_uint4(0, 0, 0, 0);
  }
  if (tid == 0) dup_any = 0;
  __syncthreads();
  const int rows = min(kPrepQ, T - q0);  // <= 0 for padding rows
  const int32_t* pblk = idx + ((int64_t)b * T + min(q0, T - 1)) * K;
  bool dup = false;
  auto put = [&](int32_t s, int i) {
    if ((uint32_t)s < (uint32_t)S) {
      const uint32_t bit = 1u << (s & 31);
      dup |= (atomicOr(&words[(s >> 5) * RW + i], bit) & bit) != 0u;
    }
  };
  // 16-byte path (K % 4 == 0, aligned positions): a thread's positions and their gradients
  // (four of each per row and step) stay in registers from the words to the ranks.
  constexpr int kNJ = kXMaxK / 4 / 256;
  const uint16_t* gblk = grad + ((int64_t)b * T + min(q0, T - 1)) * K;
  int4 pv[kNJ][kPrepQ];
  uint2 gv[kNJ][kPrepQ];
  if (vec) {
    const int n4 = K >> 2;
#pragma unroll
    for (int jj = 0; jj < kNJ; ++jj) {
      const int j4 = tid + 256 * jj;
#pragma unroll
      for (int u = 0; u < kPrepQ; ++u) {
        const bool ok = j4 < n4 && u < rows;
        pv[jj][u] = ok ? reinterpret_cast<const int4*>(pblk + (int64_t)u * K)[j4] : make_int4(-1, -1, -1, -1);
        gv[jj][u] = ok ? reinterpret_cast<const uint2*>(gblk + (int64_t)u * K)[j4] : make_uint2(0, 0);
      }
#pragma unroll
      for (int u = 0; u < kPrepQ; ++u) {
        put(pv[jj][u].x, u);
        put(pv[jj][u].y, u);
        put(pv[jj][u].z, u);
        put(pv[jj][u].w, u);
      }
    }
  } else {
    for (int i = 0; i < rows; ++i)
      for (int j = tid; j < K; j += 256) put(pblk[(int64_t)i * K + j], i);
  }
  if (dup) dup_any = 1;
  __syncthreads();
  if (tid == 0 && dup_any) route[b] = 1;
  {
    // Row i's prefixes: 32 threads, each over a run of consecutive blocks, then a scan of
    // the 32 run totals.
    const int i = tid >> 5, l = tid & 31;
    const int per = (nsub + 31) >> 5;
    const int k0 = min(nsub, l * per), k1 = min(nsub, k0 + per);
    int sum = 0;
    for (int kb = k0; kb < k1; ++kb) sum += __popc(words[kb * RW + i]);
    int x = sum;
#pragma unroll
    for (int off = 1; off < 32; off <<= 1) {
      const int y = __shfl_up(x, off, 32);
      if (l >= off) x += y;
    }
    int run = x - sum;
    for (int kb = k0; kb < k1; ++kb) {
      pre[kb * kPrepQ + i] = (uint16_t)run;
      run += __popc(words[kb * RW + i]);
    }
  }
  __syncthreads();
  // [b][t / 8][kb][t % 8]: this workgroup's words are one contiguous run; a thread writes
  // one block's 8 words and 8 prefixes with 16-byte stores.
  {
    uint32_t* wo = words_g + ((int64_t)b * (tpad >> 3) + blockIdx.x) * nsub * kPrepQ;
    uint16_t* po = pre_g + ((int64_t)b * (tpad >> 3) + blockIdx.x) * nsub * kPrepQ;
    static_assert(kPrepQ == 8, "one block of words is two 16-byte stores");
    for (int kb = tid; kb < nsub; kb += 256) {
      const uint32_t* wr = words + kb * RW;
      reinterpret_cast<uint4*>(wo + kb * 8)[0] = make_uint4(wr[0], wr[1], wr[2], wr[3]);
      reinterpret_cast<uint4*>(wo + kb * 8)[1] = make_uint4(wr[4], wr[5], wr[6], wr[7]);
      reinterpret_cast<uint4*>(po + kb * 8)[0] = reinterpret_cast<const uint4*>(pre + kb * 8)[0];
    }
  }
  // Each selected key's rank in its row: the prefix of its block plus the bits below it.
  auto rank = [&](int32_t s, int i) {
    return pre[(s >> 5) * kPrepQ + i] + __popc(words[(s >> 5) * RW + i] & ((1u << (s & 31)) - 1u));
  };
  if (vec) {
#pragma unroll
    for (int jj = 0; jj < kNJ; ++jj)
#pragma unroll
      for (int u = 0; u < kPrepQ; ++u) {
        const int32_t sv[4] = {pv[jj][u].x, pv[jj][u].y, pv[jj][u].z, pv[jj][u].w};
        const uint32_t gw[2] = {gv[jj][u].x, gv[jj][u].y};
#pragma unroll
        for (int c = 0; c < 4; ++c)
          if ((uint32_t)sv[c] < (uint32_t)S) {
            const int r = rank(sv[c], u);
            if (r < K) grow[u * K + r] = (uint16_t)(gw[c >> 1] >> (16 * (c & 1)));
          }
      }
  } else {
    for (int i = 0; i < rows; ++i)
      for (int j = tid; j < K; j += 256) {
        const int32_t s = pblk[(int64_t)i * K + j];
        if ((uint32_t)s < (uint32_t)S) {
          const int r = rank(s, i);
          if (r < K) grow[i * K + r] = gblk[(int64_t)i * K + j];
        }
      }
  }
  __syncthreads();
  for (int i = 0; i < rows; ++i) {
    uint16_t* orow = gs + ((int64_t)b * T + q0 + i) * K;
    if ((K & 7) == 0) {
      for (int c = tid; c < (K >> 3); c += 256)
        reinterpret_cast<uint4*>(orow)[c] = reinterpret_cast<const uint4*>(grow + i * K)[c];
    } else {
      for (int c = tid; c < K; c += 256) orow[c] = grow[i * K + c];
    }
  }
}

// ---------------------------------------------------------------------------------------
// x [B][R][HI][64] bf16 (times w [B][R][HI] when given, rounded to nearest even) ->
// xt[b][h][d][r'] (r' < Rpad, zero past R), rows permuted within every 16 by exchanging bits
// 2 and 3 of the row index: the order in which a lane's accumulator entries enter a product
// as its B operand (entries r < 8 of lane l are rows 8 (r / 4) + 4 (l / 32) + r % 4, which
// the operand's k-chunk l / 32 lists as k = 8 (l / 32) + r). Flags route[b] on a non-finite
// x, w or product.
// ---------------------------------------------------------------------------------------
constexpr int kTTiles = 4;  // 64-row tiles per workgroup of idxd_t_kernel

__global__ __launch_bounds__(256) void idxd_t_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
                                                     int R, int Rpad, int HI, uint16_t* __restrict__ xt,
                                                     int* __restrict__ route) {
  __shared__ __align__(16) uint16_t tile[64][72];  // [d][row]
  const int h = blockIdx.y, b = blockIdx.z;
  uint32_t nf = 0u;
  // kTTiles tiles of 64 rows per workgroup (one tile alone is too little work for a workgroup).
  for (int rt = 0; rt < kTTiles; ++rt) {
    const int r0 = (blockIdx.x * kTTiles + rt) * 64;
    if (r0 >= Rpad) break;
    if (rt > 0) __syncthreads();  // the previous tile's reads of the LDS tile are done
#pragma unroll
    for (int it = 0; it < 2; ++it) {
      const int e = threadIdx.x + it * 256;
      const int row = e >> 3, c = e & 7;
      uint4 val = make_uint4(0, 0, 0, 0);
      float ws = 1.f;
      if (r0 + row < R) {
        const int64_t tok = ((int64_t)b * R + r0 + row) * HI + h;
        val = *reinterpret_cast<const uint4*>(x + tok * kXD + c * 8);
        if (w != nullptr) {
          const uint32_t wb = w[tok];
          nf |= (uint32_t)((wb & 0x7F80u) == 0x7F80u);
          ws = __uint_as_float(wb << 16);
        }
      }
      uint32_t u[4] = {val.x, val.y, val.z, val.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        nf |= nonfinite2(u[i], 0x7F80u);
        if (w != nullptr) {
          u[i] = pack_pair(BF16{}, __uint_as_float(u[i] << 16) * ws, __uint_as_float(u[i] & 0xFFFF0000u) * ws);
          nf |= nonfinite2(u[i], 0x7F80u);
        }
        tile[c * 8 + 2 * i][row] = (uint16_t)(u[i] & 0xFFFFu);
        tile[c * 8 + 2 * i + 1][row] = (uint16_t)(u[i] >> 16);
      }
    }
    __syncthreads();
#pragma unroll
    for (int it = 0; it < 2; ++it) {
      const int e = threadIdx.x + it * 256;
      const int d = e >> 3, kc = e & 7;
      if (r0 + kc * 8 >= Rpad) continue;
      // r' = 8 kc + 0..7 holds rows 16 (kc / 2) + 4 (kc % 2) + {0..3, 8..11}
      const int k0 = 16 * (kc >> 1) + 4 * (kc & 1);
      const uint2 lo = *reinterpret_cast<const uint2*>(&tile[d][k0]);
      const uint2 hi = *reinterpret_cast<const uint2*>(&tile[d][k0 + 8]);
      *reinterpret_cast<uint4*>(xt + (((int64_t)b * HI + h) * kXD + d) * Rpad + r0 + kc * 8) =
          make_uint4(lo.x, lo.y, hi.x, hi.y);
    }
  }
  if (nf != 0u) route[b] = 1;  // every writer stores the same value
}

struct IdxDenseParams {
  const uint16_t* q;       // [B][T][HI][64]
  const uint16_t* k;       // [B][S][HI][64]
  const uint16_t* w;       // [B][S][HI]
  const uint16_t* qt;      // [B][HI][64][tpad], rows permuted
  const uint16_t* kwt;     // [B][HI][64][spad], (w o k)^T, rows permuted
  const uint32_t* words;   // [B][tpad / 8][nsub][8]
  const uint16_t* pre;     // [B][tpad / 8][nsub][8]
  const uint16_t* gs;      // [B][T][K]
  const int* route;        // [B]
  float* part;             // [nwg][2][256][64]
  uint16_t* dq;
  uint16_t* dk;
  uint16_t* dw;
  int64_t iters;           // row groups x tiles of the pass
  int nwg;                 // persistent workgroups of the pass
  int T, S, HI, K, tpad, spad, nsub;
  float scale;
};

// One 16-bit half of g per z: kept where z > 0. z is rounded to bf16 first (a positive float
// stays positive, a negative one negative or -0); as signed 16-bit integers, min(., 1) then
// max(., 0) leaves 1 exactly where z > 0 (-0 is -32768), and the packed product keeps or
// clears g: four instructions per pair.
__device__ __forceinline__ uint32_t gate2(uint32_t g, float z0, float z1) {
  const uint32_t zb = pack_pair(BF16{}, z0, z1);
  uint32_t r;
  asm("v_pk_min_i16 %0, %1, %2\n\t"
      "v_pk_max_i16 %0, %0, 0\n\t"
      "v_pk_mul_lo_u16 %0, %3, %0"
      : "=&v"(r)
      : "v"(zb), "s"(0x00010001u), "v"(g));
  return r;
}

struct PassShape {
  int Rs, Ry, ypad, ntiles, nsg;
};
template <bool KEYS>
__host__ __device__ __forceinline__ PassShape pass_shape(const IdxDenseParams& p) {
  PassShape s;
  s.Rs = KEYS ? p.S : p.T;  // stationary rows (held in registers)
  s.Ry = KEYS ? p.T : p.S;  // streamed rows (tiles of 32)
  s.ypad = KEYS ? p.tpad : p.spad;
  s.ntiles = s.ypad >> 5;
  s.nsg = (s.Rs + kXRows - 1) / kXRows;
  return s;
}

// ---------------------------------------------------------------------------------------
// One pass. Workgroup: 4 waves on one head and a group of 256 stationary rows (queries for
// dQ, keys for dK), each wave on two 32-row blocks held as B operands. Per 32-row tile of the
// streamed side (keys for dQ, queries for dK): the streamed rows Y (4 KB) and their permuted
// transpose Y'^T (4 KB: (w o k)^T for dQ, q^T for dK) in one of four LDS sets, and the
// gradient tile G (16 KB, [streamed row / 4][stationary row][4] bf16, zero at unselected
// pairs) in one of three sets (read, built, cleared). Per block: Z^T = Y X^T,
// F^T = G^T o [Z^T > 0], acc^T += Y'^T F^T.
// G is built by the 256 threads, one per (stationary row or query, 32-key block) unit: its
// selection word and prefix (from the prep kernel) are loaded four tiles ahead, its first
// eight gradients (one 16-byte load from gs) two tiles ahead; more are read while the tile
// is built. Tile n + 3 is staged while tile n is computed: every load has at least two
// tiles of time to arrive. The loop body covers four tiles, so that the sets and the
// registers of the loads in flight rotate without copies (a copy would wait for its load).
// ---------------------------------------------------------------------------------------
template <bool KEYS>
__global__ __launch_bounds__(256, 2) void idxd_pass_kernel(const IdxDenseParams p) {
  // The staging sets are distinct arrays, so that the compiler sees that staging one set
  // does not touch the others (no wait for the staging before reading the current set).
  __shared__ __align__(16) uint8_t ys0[4096], ys1[4096], ys2[4096], ys3[4096];
  __shared__ __align__(16) uint8_t yts0[4096], yts1[4096], yts2[4096], yts3[4096];
  __shared__ __align__(16) uint16_t gtile[3][8 * kXRows * 4];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 31, half = lane >> 5;
  const PassShape sh = pass_shape<KEYS>(p);
  const int HI = p.HI;
  const int64_t it0 = (int64_t)blockIdx.x * p.iters / p.nwg;
  const int64_t it1 = (int64_t)(blockIdx.x + 1) * p.iters / p.nwg;
  const int g_first = (int)(it0 / sh.ntiles);
  const uint16_t* X = KEYS ? p.k : p.q;
  const uint16_t* Y = KEYS ? p.q : p.k;
  const uint16_t* YT = KEYS ? p.qt : p.kwt;
  const uint32_t yrow_b = (uint32_t)HI * 128u;  // bytes per streamed token (all heads)

  // Staging (one 16-byte chunk of Y and one of Y'^T per thread). Y: wave w fills rows
  // 8 w .. 8 w + 7 (128 bytes each, chunk c at c ^ swz(row)); Y'^T: wave w fills d-rows
  // 16 w .. 16 w + 15 (64 bytes each, chunk c at c ^ ((d / 2) % 4)).
  const int yrow = 8 * wave + (lane >> 3);
  const int ylc = (lane & 7) ^ swz(yrow);
  const int ytd = 16 * wave + (lane >> 2);
  const int ytlc = (lane & 3) ^ ((ytd >> 1) & 3);
  // Operand reads: Y row col, chunk 2 ks + half; Y'^T row 32 db + col, chunk 2 ks + half.
  const int fc = swz(col);
  auto yoff = [&](int ks) { return col * 128 + (((2 * ks + half) ^ fc) << 4); };
  auto ytoff = [&](int db, int ks) {
    const int d = 32 * db + col;
    return d * 64 + (((2 * ks + half) ^ ((d >> 1) & 3)) << 4);
  };

  int64_t it = it0;
  while (it < it1) {
    const int g = (int)(it / sh.ntiles);
    const int n0 = (int)(it - (int64_t)g * sh.ntiles);
    const int n1 = (int)min((int64_t)sh.ntiles, n0 + (it1 - it));
    it += n1 - n0;
    const int h = g % HI;
    const int sg = (g / HI) % sh.nsg;
    const int b = g / (HI * sh.nsg);
    if (p.route[b] != 0) continue;  // the whole workgroup, before any barrier
    const int sbase = sg * kXRows;

    // Stationary B operands: row sbase + 64 wave + 32 a + col, dims 16 ks + 8 half + 0..7.
    uint4 xa[2][4];
#pragma unroll
    for (int a = 0; a < 2; ++a) {
      const int si = sbase + 64 * wave + 32 * a + col;
      const bool ok = si < sh.Rs;
      const uint16_t* xr = X + (((int64_t)b * sh.Rs + (ok ? si : 0)) * HI + h) * kXD + half * 8;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
        xa[a][ks] = ok ? *reinterpret_cast<const uint4*>(xr + ks * 16) : make_uint4(0, 0, 0, 0);
    }
    f32x16 acc[2][2];
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
      for (int db = 0; db < 2; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[a][db][r] = 0.f;

    const char* ybase_h = reinterpret_cast<const char*>(Y + (int64_t)b * sh.Ry * HI * kXD + (int64_t)h * kXD);
    const char* ytbase_h = reinterpret_cast<const char*>(YT + ((int64_t)b * HI + h) * kXD * sh.ypad);
    const uint32_t ytl = ((uint32_t)ytd * (uint32_t)sh.ypad + (uint32_t)ytlc * 8u) * 2u;
    // Stages tile min(n, n1 - 1) (past the end: a repeat into a set no tile reads).
    auto dload = [&](int n, uint8_t* yd, uint8_t* ytd_) {
      const int r0 = 32 * min(n, n1 - 1);
      const int base = min(r0, sh.Ry - 1);
      const uint32_t rowoff = (uint32_t)(min(r0 + yrow, sh.Ry - 1) - base);
      buffer_load16_lds(ybase_h + (int64_t)base * yrow_b, rowoff * yrow_b + (uint32_t)ylc * 16u, yd + wave * 1024);
      buffer_load16_lds(ytbase_h + (int64_t)r0 * 2, ytl, ytd_ + wave * 1024);
    };

    // Builder unit of this thread.
    const int qq = tid & 31, wi = tid >> 5;              // dK: query of the tile, key block
    const int ukb = KEYS ? sg * (kXRows / 32) + wi : 0;  // dK: the unit's 32-key block
    const bool uok = KEYS ? ukb < p.nsub : sbase + tid < p.tpad;
    auto unit_t = [&](int n) { return KEYS ? 32 * n + qq : sbase + tid; };
    auto unit_kb = [&](int n) { return KEYS ? ukb : n; };
    // dQ: (bit / 4) * 4 kXRows + 4 tid + bit % 4 = bit + (bit / 4) (4 kXRows - 4) + 4 tid
    // (one shift and one 24-bit multiply-add per entry).
    auto gpos = [&](int bit) {
      return KEYS ? (((qq >> 2) * kXRows + 32 * wi + bit) << 2) + (qq & 3)
                  : (int)__umul24((uint32_t)bit >> 2, 4u * kXRows - 4u) + bit + 4 * tid;
    };
    // Words and prefixes: [b][t / 8][kb][t % 8]. Loads for tiles ahead are unconditional (an
    // invalid unit or a tile past n1 reads element 0) and are masked when used.
    struct WP {
      uint32_t w;
      uint16_t p;  // 16-bit until used: widening a loaded value right away would wait for it
    };
    auto wp_load = [&](int n) {
      const int t = unit_t(n);
      const int64_t o = n < n1 && uok ? (((int64_t)b * (p.tpad >> 3) + (t >> 3)) * p.nsub + unit_kb(n)) * 8 + (t & 7)
                                      : (int64_t)0;
      return WP{p.words[o], p.pre[o]};
    };
    auto wmask = [&](int n, uint32_t w) { return n < n1 && uok ? w : 0u; };
    auto grow = [&](int n, uint32_t P0) { return p.gs + ((int64_t)b * p.T + unit_t(n)) * p.K + P0; };
    // The unit's first eight gradients in one 16-byte load (no alignment needed; the gs
    // region has slack past its end).
    auto vload = [&](int n, WP x) {
      const uint16_t* gr = wmask(n, x.w) != 0u ? grow(n, x.p) : p.gs;
      uint4 v;
      __builtin_memcpy(&v, gr, 16);
      return v;
    };
    auto scatter = [&](uint16_t* gt, int n, WP x, uint4 v) {
      uint32_t bits = wmask(n, x.w);
      int m = 0;
      while (bits != 0u) {
        const int bit = __builtin_ctz(bits);
        bits &= bits - 1u;
        uint32_t val;
        if (m < 8) {
          const uint32_t d = m < 4 ? (m < 2 ? v.x : v.y) : (m < 6 ? v.z : v.w);
          val = (d >> (16 * (m & 1))) & 0xFFFFu;
        } else {
          val = grow(n, x.p)[m];
        }
        gt[gpos(bit)] = (uint16_t)val;
        ++m;
      }
    };
    auto zero_tile = [&](uint16_t* gt) {
#pragma unroll
      for (int i = 0; i < 8 * kXRows * 4 / 8 / 256; ++i) reinterpret_cast<uint4*>(gt)[tid + 256 * i] = make_uint4(0, 0, 0, 0);
    };

    // Segment prologue: zero the gradient tiles, stage tiles n0 .. n0 + 2, load the words of
    // n0 .. n0 + 3 and the gradients of n0 and n0 + 1, build the gradient tile of n0.
    // Tile n: Y and Y'^T in set (n - n0) % 4, G in set (n - n0) % 3.
    zero_tile(gtile[0]);
    zero_tile(gtile[1]);
    zero_tile(gtile[2]);
    dload(n0, ys0, yts0);
    dload(n0 + 1, ys1, yts1);
    dload(n0 + 2, ys2, yts2);
    WP wp0 = wp_load(n0), wp1 = wp_load(n0 + 1), wp2 = wp_load(n0 + 2), wp3 = wp_load(n0 + 3);
    uint4 va = vload(n0, wp0);  // gradients of the tile the next build is for
    uint4 vb = vload(n0 + 1, wp1);
    __syncthreads();  // the tiles are zero before any thread writes its entries
    scatter(gtile[0], n0, wp0, va);
    __builtin_amdgcn_s_waitcnt(0x0070);  // vmcnt(0) lgkmcnt(0): tiles n0 .. n0 + 2 are in LDS
    __syncthreads();

    int gc = 0;  // gradient-tile set of tile n
    // One tile. cur: Y / Y'^T of tile n; stg: the set of tile n - 1, which receives tile
    // n + 3. wn1, wn2: words of tiles n + 1, n + 2; wld: receives the words of tile n + 4
    // (it held tile n's). vcur: gradients of tile n + 1 (loaded a tile ago); vnext: receives
    // those of tile n + 2.
    auto step = [&](int n, const uint8_t* yt, const uint8_t* ytt, uint8_t* ys, uint8_t* yts, const WP& wn1,
                    const WP& wn2, WP& wld, const uint4& vcur, uint4& vnext) {
      const int gn = gc == 2 ? 0 : gc + 1;  // set of tile n + 1 (zeroed a tile ago)
      const int gz = gn == 2 ? 0 : gn + 1;  // set of tile n - 1: cleared for tile n + 2
      // Five vector-memory instructions per tile, in this order. The words of tile n + 2
      // are taken here (not earlier, where the compiler would wait for them before the
      // barrier).
      WP w2 = wn2;
      asm volatile("" : "+v"(w2.w), "+v"(w2.p));
      vnext = vload(n + 2, w2);
      wld = wp_load(n + 4);
      dload(n + 3, ys, yts);
      zero_tile(gtile[gz]);

      // Gradient tile entries of this lane: group gq = streamed rows 8 gq + 4 half + 0..3.
      const uint16_t* gt = gtile[gc];
      uint2 gv[2][4];
#pragma unroll
      for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int gq = 0; gq < 4; ++gq)
          gv[a][gq] = *reinterpret_cast<const uint2*>(gt + ((((2 * gq + half) * kXRows) + 64 * wave + 32 * a + col) << 2));
      // Products for every tile, also where the wave's gradient entries are all zero: the
      // gate clears F there (an integer product, whatever z is) and the staged tiles are
      // finite (non-finite inputs flag the batch element), so they add exact zeros. A skip
      // branch would split the step and cost more than the rare all-zero tile saves.
      {
        f32x16 z[2];
#pragma unroll
        for (int a = 0; a < 2; ++a)
#pragma unroll
          for (int r = 0; r < 16; ++r) z[a][r] = 0.f;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          const uint4 ya = *reinterpret_cast<const uint4*>(yt + yoff(ks));
#pragma unroll
          for (int a = 0; a < 2; ++a) z[a] = mma(BF16{}, ya, xa[a][ks], z[a]);
        }
        // Per block: its gate, then its products, so that the second block's gate overlaps
        // the first block's products (the Y'^T operands read once for both).
        uint4 ta[2][2];
#pragma unroll
        for (int db = 0; db < 2; ++db)
#pragma unroll
          for (int ks = 0; ks < 2; ++ks) ta[db][ks] = *reinterpret_cast<const uint4*>(ytt + ytoff(db, ks));
#pragma unroll
        for (int a = 0; a < 2; ++a) {
          uint4 fb[2];
#pragma unroll
          for (int ks = 0; ks < 2; ++ks) {
            const uint2 g0 = gv[a][2 * ks], g1 = gv[a][2 * ks + 1];
            const f32x16& zz = z[a];
            fb[ks] = make_uint4(gate2(g0.x, zz[8 * ks + 0], zz[8 * ks + 1]), gate2(g0.y, zz[8 * ks + 2], zz[8 * ks + 3]),
                                gate2(g1.x, zz[8 * ks + 4], zz[8 * ks + 5]), gate2(g1.y, zz[8 * ks + 6], zz[8 * ks + 7]));
          }
#pragma unroll
          for (int db = 0; db < 2; ++db)
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) acc[a][db] = mma(BF16{}, ta[db][ks], fb[ks], acc[a][db]);
        }
      }

      scatter(gtile[gn], n + 1, wn1, vcur);
      gc = gn;
      // vmcnt(10): the staging of tile n + 1 (two tiles back; ten vector-memory
      // instructions since) has landed. lgkmcnt(0): the gradient tile is written.
      __builtin_amdgcn_s_waitcnt(0x007A);
      asm volatile("" ::: "memory");
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
    };
    // Four tiles per trip, unconditionally: a tile past n1 has an all-zero gradient tile and
    // adds nothing.
#pragma unroll 1
    for (int n = n0; n < n1; n += 4) {
      step(n, ys0, yts0, ys3, yts3, wp1, wp2, wp0, vb, va);
      step(n + 1, ys1, yts1, ys0, yts0, wp2, wp3, wp1, va, vb);
      step(n + 2, ys2, yts2, ys1, yts1, wp3, wp0, wp2, vb, va);
      step(n + 3, ys3, yts3, ys2, yts2, wp0, wp1, wp3, va, vb);
    }
    // Staging issued for tiles past the end targets sets no tile reads; drain it before the
    // sets are reused.
    __builtin_amdgcn_s_waitcnt(0x0070);

    // Epilogue. acc[a][db] entry r: d = 32 db + 8 (r / 4) + 4 half + r % 4, row of block a.
    const bool whole = n0 == 0 && n1 == sh.ntiles;
    if (!whole) {
      float* pp = p.part + ((int64_t)blockIdx.x * 2 + (g == g_first ? 0 : 1)) * kXRows * kXD;
#pragma unroll
      for (int a = 0; a < 2; ++a) {
        const int sl = 64 * wave + 32 * a + col;
#pragma unroll
        for (int db = 0; db < 2; ++db)
#pragma unroll
          for (int gq = 0; gq < 4; ++gq)
            *reinterpret_cast<float4*>(pp + sl * kXD + 32 * db + 8 * gq + 4 * half) =
                make_float4(acc[a][db][4 * gq], acc[a][db][4 * gq + 1], acc[a][db][4 * gq + 2], acc[a][db][4 * gq + 3]);
      }
      continue;
    }
#pragma unroll
    for (int a = 0; a < 2; ++a) {
      const int si = sbase + 64 * wave + 32 * a + col;
      const bool ok = si < sh.Rs;
      const int64_t tok = ((int64_t)b * sh.Rs + (ok ? si : 0)) * HI + h;
      float osc = p.scale;
      float dwp = 0.f;
      if constexpr (KEYS) {
        osc *= __uint_as_float((uint32_t)p.w[tok] << 16);
        const uint16_t* kr = p.k + tok * kXD;
#pragma unroll
        for (int db = 0; db < 2; ++db)
#pragma unroll
          for (int gq = 0; gq < 4; ++gq) {
            const uint2 kv = *reinterpret_cast<const uint2*>(kr + 32 * db + 8 * gq + 4 * half);
            dwp = fmaf(__uint_as_float(kv.x << 16), acc[a][db][4 * gq], dwp);
            dwp = fmaf(__uint_as_float(kv.x & 0xFFFF0000u), acc[a][db][4 * gq + 1], dwp);
            dwp = fmaf(__uint_as_float(kv.y << 16), acc[a][db][4 * gq + 2], dwp);
            dwp = fmaf(__uint_as_float(kv.y & 0xFFFF0000u), acc[a][db][4 * gq + 3], dwp);
          }
        dwp = pair_sum(dwp);
      }
      if (!ok) continue;
      uint16_t* orow = (KEYS ? p.dk : p.dq) + tok * kXD;
#pragma unroll
      for (int db = 0; db < 2; ++db)
#pragma unroll
        for (int gq = 0; gq < 4; ++gq) {
          const uint32_t lo = pack_pair(BF16{}, acc[a][db][4 * gq] * osc, acc[a][db][4 * gq + 1] * osc);
          const uint32_t hi = pack_pair(BF16{}, acc[a][db][4 * gq + 2] * osc, acc[a][db][4 * gq + 3] * osc);
          *reinterpret_cast<uint2*>(orow + 32 * db + 8 * gq + 4 * half) = make_uint2(lo, hi);
        }
      if constexpr (KEYS) {
        if (half == 0) p.dw[tok] = to_half_bits(BF16{}, dwp * p.scale);
      }
    }
  }
}

// ---------------------------------------------------------------------------------------
// Row groups that the pass split between workgroups: the partials of the covering
// workgroups, summed in workgroup order, then the pass's epilogue. One thread per row.
// Workgroup w covers iterations [w iters / nwg, (w + 1) iters / nwg); its partial for a
// group is in slot 0 when the group holds its first iteration, else in slot 1.
// ---------------------------------------------------------------------------------------
template <bool KEYS>
__global__ __launch_bounds__(256) void idxd_fixup_kernel(const IdxDenseParams p) {
  const PassShape sh = pass_shape<KEYS>(p);
  const int g = blockIdx.x;
  const int h = g % p.HI;
  const int sg = (g / p.HI) % sh.nsg;
  const int b = g / (p.HI * sh.nsg);
  if (p.route[b] != 0) return;
  const int64_t lo = (int64_t)g * sh.ntiles, hi = lo + sh.ntiles;
  auto beg = [&](int64_t w) { return w * p.iters / p.nwg; };
  int64_t w0 = lo * p.nwg / p.iters;
  while (w0 > 0 && beg(w0) > lo) --w0;
  while (w0 + 1 < p.nwg && beg(w0 + 1) <= lo) ++w0;
  if (beg(w0) <= lo && beg(w0 + 1) >= hi) return;  // one workgroup ran the whole group
  const int r = threadIdx.x;
  const int si = sg * kXRows + r;
  if (si >= sh.Rs) return;
  float sum[kXD];
#pragma unroll
  for (int d = 0; d < kXD; ++d) sum[d] = 0.f;
  for (int64_t w = w0; w < p.nwg && beg(w) < hi; ++w) {
    const int slot = beg(w) / sh.ntiles == g ? 0 : 1;
    const float4* pp = reinterpret_cast<const float4*>(p.part + ((w * 2 + slot) * kXRows + r) * kXD);
#pragma unroll
    for (int c = 0; c < kXD / 4; ++c) {
      const float4 x = pp[c];
      sum[4 * c] += x.x;
      sum[4 * c + 1] += x.y;
      sum[4 * c + 2] += x.z;
      sum[4 * c + 3] += x.w;
    }
  }
  const int64_t tok = ((int64_t)b * sh.Rs + si) * p.HI + h;
  float osc = p.scale;
  if constexpr (KEYS) {
    osc *= __uint_as_float((uint32_t)p.w[tok] << 16);
    const uint16_t* kr = p.k + tok * kXD;
    float dwv = 0.f;
#pragma unroll
    for (int d = 0; d < kXD; ++d) dwv = fmaf(__uint_as_float((uint32_t)kr[d] << 16), sum[d], dwv);
    p.dw[tok] = to_half_bits(BF16{}, dwv * p.scale);
  }
  uint16_t* orow = (KEYS ? p.dk : p.dq) + tok * kXD;
#pragma unroll
  for (int c = 0; c < kXD / 8; ++c) {
    float f[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) f[i] = sum[8 * c + i] * osc;
    *reinterpret_cast<uint4*>(orow + 8 * c) = pack_quad<BF16>(f);
  }
}

struct IdxDenseLayout {
  size_t words, pre, gs, qt, kwt, part, total;
  int tpad, spad, nsub, slots;
};

// Resident workgroups of the pass kernel on the current device (cached).
int idxd_slots() {
  struct Entry {
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
      if (cache[i].dev == dev) return cache[i].slots;
  }
  int cus = 0, per_cu = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void*>(idxd_pass_kernel<false>),
                                                   256, 0) != hipSuccess ||
      per_cu <= 0)
    per_cu = 1;
  const int slots = cus * per_cu;
  std::lock_guard<std::mutex> lock(mu);
  if (n_cache < 64) cache[n_cache++] = Entry{dev, slots};
  return slots;
}

IdxDenseLayout idxd_layout(int64_t B, int64_t T, int64_t S, int64_t HI, int64_t K) {
  IdxDenseLayout L;
  L.tpad = (int)((T + 31) / 32 * 32);
  L.spad = (int)((S + 31) / 32 * 32);
  L.nsub = L.spad / 32;
  L.slots = idxd_slots();
  auto up = [](size_t x) { return (x + 255) / 256 * 256; };
  size_t o = 0;
  L.words = o;
  o = up(o + (size_t)B * L.nsub * L.tpad * 4);
  L.pre = o;
  o = up(o + (size_t)B * L.nsub * L.tpad * 2);
  L.gs = o;
  o = up(o + (size_t)B * T * K * 2 + 32);  // slack: a thread loads 8 gradients past any rank
  L.qt = o;
  o = up(o + (size_t)B * HI * kXD * L.tpad * 2);
  L.kwt = o;
  o = up(o + (size_t)B * HI * kXD * L.spad * 2);
  L.part = o;
  o = up(o + (size_t)L.slots * 2 * kXRows * kXD * 4);
  L.total = o;
  return L;
}

size_t idxd_prep_lds(int nsub, int K) {
  const size_t off_pre = (size_t)((nsub * (kPrepQ + 1) + 3) & ~3);
  const size_t off_g = off_pre + (size_t)((nsub * kPrepQ / 2 + 3) & ~3);
  return (off_g + (size_t)((kPrepQ * K + 1) / 2 + 3) / 4 * 4) * 4;
}

template <bool KEYS>
int launch_pass(IdxDenseParams p, int B, const IdxDenseLayout& L, hipStream_t st) {
  const PassShape sh = pass_shape<KEYS>(p);
  const int64_t groups = (int64_t)B * p.HI * sh.nsg;
  p.iters = groups * sh.ntiles;
  p.nwg = (int)std::min<int64_t>((int64_t)L.slots, p.iters);
  hipLaunchKernelGGL((idxd_pass_kernel<KEYS>), dim3((unsigned)p.nwg), dim3(256), 0, st, p);
  GW_HIP_LAUNCH_CHECK(KEYS ? "idxd_pass_kernel<dk> launch" : "idxd_pass_kernel<dq> launch");
  if (p.nwg > 1) {
    hipLaunchKernelGGL((idxd_fixup_kernel<KEYS>), dim3((unsigned)groups), dim3(256), 0, st, p);
    GW_HIP_LAUNCH_CHECK("idxd_fixup_kernel launch");
  }
  return GW_OK;
}

}  // namespace
}  // namespace gw

extern "C" size_t gw_indexer_topk_bwd_dense_workspace_size(int64_t B, int64_t T, int64_t S, int64_t Hi, int64_t Di,
                                                           int64_t K) {
  if (B <= 0 || T <= 0 || S <= 0 || Hi <= 0 || K <= 0 || Di != gw::kXD) return 256;
  return gw::idxd_layout(B, T, S, Hi, K).total;
}

extern "C" int gw_indexer_topk_bwd_dense(int dtype, const void* q, const void* k, const void* w,
                                         const int32_t* topk_indices, const void* grad_scores, void* dq, void* dk,
                                         void* dw, int64_t B, int64_t T, int64_t S, int64_t Hi, int64_t Di,
                                         int64_t K, float softmax_scale, int* route, void* workspace,
                                         size_t workspace_bytes, void* stream) {
  using namespace gw;
  clear_error();
  GW_CHECK_ARG(dtype == GW_DTYPE_BF16 || dtype == GW_DTYPE_FP16 || dtype == GW_DTYPE_FP32, "unsupported dtype code %d",
               dtype);
  GW_CHECK_ARG(B >= 0 && T >= 0 && S >= 0 && K >= 0, "invalid sizes B=%lld T=%lld S=%lld K=%lld", (long long)B,
               (long long)T, (long long)S, (long long)K);
  if (dtype != GW_DTYPE_BF16) return set_error(GW_ERR_UNSUPPORTED, "the dense indexer backward takes bf16 only");
  if (Di != kXD || !(Hi == 1 || Hi == 2 || Hi == 4 || Hi == 8))
    return set_error(GW_ERR_UNSUPPORTED, "indexer heads x dim %lld x %lld not supported (1/2/4/8 x 64)",
                     (long long)Hi, (long long)Di);
  if (S > kXMaxS || K > kXMaxK)
    return set_error(GW_ERR_UNSUPPORTED, "the dense indexer backward takes S <= %d and K <= %d", kXMaxS, kXMaxK);
  if (T > (1ll << 22) - 32)
    return set_error(GW_ERR_UNSUPPORTED, "the dense indexer backward takes T <= 2^22 - 32");
  if (B == 0 || T == 0 || S == 0) return GW_OK;
  GW_CHECK_ARG(K >= 1, "empty top-k table");
  GW_CHECK_ARG(B <= 65535, "batch exceeds the grid");
  GW_CHECK_ARG(q && k && w && topk_indices && grad_scores && dq && dk && dw && route, "null pointer");
  GW_CHECK_ARG(aligned16(q) && aligned16(k) && aligned16(dq) && aligned16(dk), "q/k/dq/dk must be 16-byte aligned");
  GW_CHECK_ARG(softmax_scale > 0.f, "softmax_scale must be positive");
  const IdxDenseLayout L = idxd_layout(B, T, S, Hi, K);
  GW_CHECK_ARG(workspace != nullptr && aligned16(workspace) && workspace_bytes >= L.total,
               "workspace needs %zu bytes (16-byte aligned), got %zu", L.total, workspace_bytes);
  char* ws = static_cast<char*>(workspace);
  IdxDenseParams p{};
  p.q = static_cast<const uint16_t*>(q);
  p.k = static_cast<const uint16_t*>(k);
  p.w = static_cast<const uint16_t*>(w);
  p.qt = reinterpret_cast<const uint16_t*>(ws + L.qt);
  p.kwt = reinterpret_cast<const uint16_t*>(ws + L.kwt);
  p.words = reinterpret_cast<const uint32_t*>(ws + L.words);
  p.pre = reinterpret_cast<const uint16_t*>(ws + L.pre);
  p.gs = reinterpret_cast<const uint16_t*>(ws + L.gs);
  p.route = route;
  p.part = reinterpret_cast<float*>(ws + L.part);
  p.dq = static_cast<uint16_t*>(dq);
  p.dk = static_cast<uint16_t*>(dk);
  p.dw = static_cast<uint16_t*>(dw);
  p.T = (int)T;
  p.S = (int)S;
  p.HI = (int)Hi;
  p.K = (int)K;
  p.tpad = L.tpad;
  p.spad = L.spad;
  p.nsub = L.nsub;
  p.scale = softmax_scale;
  hipStream_t st = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(idxd_clear_kernel, dim3((unsigned)((B + 255) / 256)), dim3(256), 0, st, route, (int)B);
  GW_HIP_LAUNCH_CHECK("idxd_clear_kernel launch");
  const int vec = (K % 4 == 0 && (reinterpret_cast<uintptr_t>(topk_indices) & 15u) == 0 &&
                   (reinterpret_cast<uintptr_t>(grad_scores) & 7u) == 0)
                      ? 1
                      : 0;
  hipLaunchKernelGGL(idxd_prep_kernel, dim3((unsigned)(L.tpad / kPrepQ), (unsigned)B), dim3(256),
                     idxd_prep_lds(L.nsub, (int)K), st, topk_indices, static_cast<const uint16_t*>(grad_scores),
                     (int)T, (int)S, (int)K, L.nsub, L.tpad, vec, reinterpret_cast<uint32_t*>(ws + L.words),
                     reinterpret_cast<uint16_t*>(ws + L.pre), reinterpret_cast<uint16_t*>(ws + L.gs), route);
  GW_HIP_LAUNCH_CHECK("idxd_prep_kernel launch");
  const unsigned tq = (unsigned)(((L.tpad + 63) / 64 + kTTiles - 1) / kTTiles);
  const unsigned tk = (unsigned)(((L.spad + 63) / 64 + kTTiles - 1) / kTTiles);
  hipLaunchKernelGGL(idxd_t_kernel, dim3(tq, (unsigned)Hi, (unsigned)B), dim3(256), 0, st,
                     p.q, nullptr, (int)T, L.tpad, (int)Hi, reinterpret_cast<uint16_t*>(ws + L.qt), route);
  GW_HIP_LAUNCH_CHECK("idxd_t_kernel<q> launch");
  hipLaunchKernelGGL(idxd_t_kernel, dim3(tk, (unsigned)Hi, (unsigned)B), dim3(256), 0, st,
                     p.k, p.w, (int)S, L.spad, (int)Hi, reinterpret_cast<uint16_t*>(ws + L.kwt), route);
  GW_HIP_LAUNCH_CHECK("idxd_t_kernel<wk> launch");
  const int rc = launch_pass<false>(p, (int)B, L, st);
  return rc != GW_OK ? rc : launch_pass<true>(p, (int)B, L, st);
}
