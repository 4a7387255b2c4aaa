// Sparse-index attention forward as a masked dense pass on the matrix cores (gfx950, D = 64).
//
// The reference forms softmax(q·k_s)·v_s over the keys s each query selected by gathering
// their K and V rows (_fwd_kernel, sparse_index_flash_attn.py:129-259). For 16 heads of 64 a gathered
// (query, key) pair moves 4 KiB; when a query selects a few per cent of all keys (1,024 of
// 43,968 at 32 views) computing every (query, key) product on the matrix cores costs less
// than gathering the selected ones. This file does that: per tile of 32 queries x 32 keys,
// S = Q·Kᵀ and O += P·V are v_mfma_f32_32x32x16 products, and the selection enters as a
// mask — P is zero at every pair the query did not select, so O, the row sums and the lse are
// those of the sparse attention, up to fp32 summation order.
//
// The softmax only runs on the selected pairs. Per tile the selected (row, key) entries are
// compacted into a list once, shared by the wave's two heads; for each head the S tile is
// staged in LDS, the listed scores are read back and exponentiated, and each p is written
// as hi + lo 16-bit parts (p - hi is exact in fp32) into zeroed P tiles that feed two P·V
// products, so the weights keep ~16 significant bits. Row sums are taken from the same P
// operands (v_dot2 with ones), in a fixed order.
//
// Online softmax with a lazy reference maximum: a row's reference m is raised only when an
// entry exceeds it by more than kLazy in the exp2 domain; O and the row sum are then rescaled.
// Every p = exp2(t - m) lies in [0, 2^kLazy], so P fits bf16/fp16 without overflow, and the
// final o = O / l and lse = m + log2(l) do not depend on which m was used.
//
// Pieces (all on the caller's stream):
//   dense_mask_kernel  — maskT[b][qb][key]: bit i set when query qb*32 + i selected the key
//                        (LDS atomic OR per listed position, per chunk of keys). A position
//                        listed twice for one query (the atomic returns the bit already set)
//                        flags the block: the gather kernel then computes that block, since
//                        the reference counts a repeated position twice.
//   dense_vt_kernel    — V as [B][H][64][S_pad] (S_pad = S rounded up to 64, zero padded):
//                        the P·V B operand is 8 consecutive keys of one column, one 16-byte load.
//   dense_attn_kernel  — 8 waves per workgroup, one per 32-query block, all on the same 2
//                        heads: each K and V^T tile is read from memory once per workgroup
//                        and shared through LDS.
#include <math.h>

#include "gw_attn.h"
#include "gw_common.h"
#include "gw_select.h"
#include "gw_sort.h"

namespace gw {
namespace {

constexpr float kDLog2e = 1.4426950408889634f;
constexpr float kDLn2 = 0.6931471805599453f;
constexpr int kDHpw = 2;           // heads per wave
constexpr float kLazy = 8.f;       // p <= 2^kLazy before a rescale

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));

__device__ __forceinline__ f32x16 mma(BF16, uint4 a, uint4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}
__device__ __forceinline__ f32x16 mma(FP16, uint4 a, uint4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a),
                                                __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
}

// ---------------------------------------------------------------------------------------
// Selection mask, key-major per 32-query block, built per (block, chunk of kMaskChunk keys)
// with LDS atomics. The atomic returns the word as it was: a bit already set means the query
// listed the key twice, and the block is flagged. Positions are read 8 rows at a time (16
// bytes per lane when the table allows), so the loads of a group are in flight together.
// ---------------------------------------------------------------------------------------
constexpr int kMaskChunk = 16384;  // keys per workgroup (64 KiB of LDS words)

__global__ __launch_bounds__(256) void dense_mask_kernel(const int32_t* __restrict__ pos, int64_t psb, int64_t pst,
                                                         int T, int S, int K, int nqb, int nchunk, int vec,
                                                         uint32_t* __restrict__ mask, int* __restrict__ flags) {
  __shared__ uint32_t words[kMaskChunk];
  __shared__ int dup_any;
  const int qb = blockIdx.x, chunk = blockIdx.y, b = blockIdx.z;
  const int c0 = chunk * kMaskChunk;
  const int len = min(kMaskChunk, S - c0);
  for (int i = threadIdx.x; i < len; i += 256) words[i] = 0u;
  if (threadIdx.x == 0) dup_any = 0;
  __syncthreads();
  bool dup = false;
  const int rows = min(32, T - qb * 32);
  const int32_t* pblk = pos + b * psb + (int64_t)(qb * 32) * pst;
  // Positions outside [c0, c0 + len) (other chunks, negative padding, >= S) wrap to large
  // unsigned offsets and are skipped.
  auto put = [&](int32_t sidx, uint32_t bit) {
    const uint32_t sl = (uint32_t)sidx - (uint32_t)c0;
    if (sl < (uint32_t)len) dup |= (atomicOr(&words[sl], bit) & bit) != 0u;
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
          const uint32_t bit = 1u << ((r0 + u) & 31);
          put(v[u].x, bit);
          put(v[u].y, bit);
          put(v[u].z, bit);
          put(v[u].w, bit);
        }
      }
    }
  } else {
#pragma unroll 1
    for (int i = 0; i < rows; ++i) {
      const int32_t* prow = pblk + (int64_t)i * pst;
      for (int j = threadIdx.x; j < K; j += 256) put(prow[j], 1u << i);
    }
  }
  if (dup) dup_any = 1;
  __syncthreads();
  uint32_t* out = mask + ((int64_t)b * nqb + qb) * S + c0;
  for (int i = threadIdx.x; i < len; i += 256) out[i] = words[i];
  if (threadIdx.x == 0) flags[((int64_t)b * nqb + qb) * nchunk + chunk] = dup_any;
}

// ---------------------------------------------------------------------------------------
// V transposed per head: vt[b][h][d][s], s < S_pad, zero past S.
// ---------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void dense_vt_kernel(const uint16_t* __restrict__ v, int64_t vsb, int64_t vss,
                                                       int64_t vsh, int S, int Spad, int H,
                                                       uint16_t* __restrict__ vt) {
  __shared__ __align__(16) uint16_t tile[64][72];  // [d][key], rows of 144 bytes
  const int s0 = blockIdx.x * 64, h = blockIdx.y, b = blockIdx.z;
#pragma unroll
  for (int it = 0; it < 2; ++it) {
    const int idx = threadIdx.x + it * 256;
    const int key = idx >> 3, c = idx & 7;
    uint4 val = make_uint4(0, 0, 0, 0);
    if (s0 + key < S)
      val = *reinterpret_cast<const uint4*>(v + b * vsb + (int64_t)(s0 + key) * vss + h * vsh + c * 8);
    const uint32_t w[4] = {val.x, val.y, val.z, val.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      tile[c * 8 + 2 * i][key] = (uint16_t)(w[i] & 0xFFFFu);
      tile[c * 8 + 2 * i + 1][key] = (uint16_t)(w[i] >> 16);
    }
  }
  __syncthreads();
#pragma unroll
  for (int it = 0; it < 2; ++it) {
    const int idx = threadIdx.x + it * 256;
    const int d = idx >> 3, kc = idx & 7;
    const uint4 val = *reinterpret_cast<const uint4*>(&tile[d][kc * 8]);
    *reinterpret_cast<uint4*>(vt + (((int64_t)b * H + h) * 64 + d) * Spad + s0 + kc * 8) = val;
  }
}

// ---------------------------------------------------------------------------------------
// The attention. Accumulator element r of lane l holds (row 8*(r/4) + 4*(l/32) + r%4,
// column l%32) of a 32x32 tile; A operands hold row l%32, B operands column l%32, each with
// the 8-element k-chunk (l/32) of a 16-wide step.
// ---------------------------------------------------------------------------------------
struct DenseParams {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* vt;
  const uint32_t* mask;
  const int* flags;
  uint16_t* o;
  float* lse;
  int64_t qsb, qst, qsh;
  int64_t ksb, kss, ksh;
  int64_t osb, ost, osh;
  int T, S, Spad, H, nqb, nchunk;
  float scale_log2;
  // attn_sum (ATTN kernels only): the scaled score of every selected (query, key) and head,
  // sws[((b * T + t) * K + slot) * H + h], slot = rank of the key among the query's
  // selected keys in ascending key order.
  float* sws;
  int K;
};

// The attention runs one wave per workgroup. LDS operations of a wave are performed in
// issue order, so another lane's LDS write is visible to a later LDS read of this wave once
// the compiler keeps them in program order; no s_barrier and, unlike __syncthreads, no wait
// for the global loads in flight.
__device__ __forceinline__ void lds_fence() { asm volatile("" ::: "memory"); }

// Inclusive prefix sum over the 64 lanes with DPP row shifts and row broadcasts.
__device__ __forceinline__ int wave_scan_dpp(int x) {
  x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xF, 0xF, true);  // row_shr:1
  x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xF, 0xF, true);  // row_shr:2
  x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xF, 0xF, true);  // row_shr:4
  x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xF, 0xF, true);  // row_shr:8
  x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xA, 0xF, false); // row_bcast:15 -> rows 1, 3
  x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xC, 0xF, false); // row_bcast:31 -> rows 2, 3
  return x;
}

__device__ __forceinline__ int tile_row(int r, int half) { return 8 * (r >> 2) + 4 * half + (r & 3); }

__device__ __forceinline__ uint16_t to_half_bits(BF16, float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }
__device__ __forceinline__ uint16_t to_half_bits(FP16, float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }
// Sum of the 8 16-bit values of v added to c, in a fixed order (exact products with 1.0).
__device__ __forceinline__ float sum8(BF16 e, uint4 v, float c) {
  constexpr uint32_t one2 = 0x3F803F80u;
  c = dot2(e, v.x, one2, c);
  c = dot2(e, v.y, one2, c);
  c = dot2(e, v.z, one2, c);
  return dot2(e, v.w, one2, c);
}
__device__ __forceinline__ float sum8(FP16 e, uint4 v, float c) {
  constexpr uint32_t one2 = 0x3C003C00u;
  c = dot2(e, v.x, one2, c);
  c = dot2(e, v.y, one2, c);
  c = dot2(e, v.z, one2, c);
  return dot2(e, v.w, one2, c);
}
__device__ __forceinline__ float from_half_bits(BF16, uint16_t x) { return __uint_as_float((uint32_t)x << 16); }
__device__ __forceinline__ float from_half_bits(FP16, uint16_t x) { return (float)__builtin_bit_cast(_Float16, x); }
__device__ __forceinline__ uint32_t pack_pair(BF16 e, float lo, float hi) {
  return (uint32_t)to_half_bits(e, lo) | ((uint32_t)to_half_bits(e, hi) << 16);
}
__device__ __forceinline__ uint32_t pack_pair(FP16 e, float lo, float hi) {
  return (uint32_t)to_half_bits(e, lo) | ((uint32_t)to_half_bits(e, hi) << 16);
}

constexpr int kDW = 8;      // waves (32-query blocks) per workgroup, sharing each K/V tile
constexpr int kPElems = 32 * 32 + 64;  // P tile (32 rows x 32 keys, 16-bit) + dummy slots

// K tile: 32 keys x (2 heads x 64) bf16 = 32 rows of 256 bytes; the 16-byte chunk c of key
// row kl sits at position c ^ (kl & 15). V^T tile: 128 rows (head, d) x 32 keys = 128 rows of
// 64 bytes; chunk c of row rr sits at c ^ ((rr >> 2) & 3). Both layouts make the MFMA operand
// reads (32 consecutive rows at one chunk) touch distinct bank groups within 16 lanes.
template <typename E, bool ATTN>
__global__ __launch_bounds__(kDW * 64) void dense_attn_kernel(const DenseParams p) {
  constexpr int HPW = kDHpw;
  // Ring of kRing K/V tiles (tile t in buffer t % kRing), one barrier per kDist tiles. With
  // attn_sum the per-wave slot arrays need the LDS of two ring buffers: two tiles, a barrier
  // per tile.
  constexpr int kRing = ATTN ? 2 : 4;
  constexpr int kDist = kRing / 2;
  __shared__ __align__(16) uint8_t ktile[kRing][8192];
  __shared__ __align__(16) uint8_t vtile[kRing][8192];
  // attn_sum: per wave, each listed entry's slot and the rows' running slot counts.
  __shared__ uint16_t eslot_all[ATTN ? kDW : 1][ATTN ? 32 * 32 + 64 : 1];
  __shared__ uint32_t rcnt_all[ATTN ? kDW : 1][ATTN ? 33 : 1];
  // Per wave: the S tile staged as float4 groups, lane-contiguous (element r of lane l at
  // ((r >> 2) * 64 + l) * 4 + (r & 3)); P as two 16-bit tiles hi and lo (p = hi + lo to
  // ~16 significant bits), rows of 64 bytes with XOR-swizzled 16-byte chunks; the compacted
  // entry list. Lanes without an entry use dummy slots, so no per-entry step needs a branch:
  // row 32 (m = +inf there, so p = 0), P slot 1024 + lane, list slot 1024 + lane.
  __shared__ __align__(16) float stage_all[kDW][16 * 64];
  __shared__ __align__(16) uint16_t phi_all[kDW][kPElems];
  __shared__ __align__(16) uint16_t plo_all[kDW][kPElems];
  __shared__ uint16_t elist_all[kDW][32 * 32 + 64];
  __shared__ __align__(16) float mrow_all[kDW][HPW][36];
  __shared__ __align__(16) float arow_all[kDW][32];
  __shared__ uint32_t mx_all[kDW][33];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  float* stage = stage_all[wave];
  uint16_t* phi = phi_all[wave];
  uint16_t* plo = plo_all[wave];
  uint16_t* elist = elist_all[wave];
  float (*mrow)[36] = mrow_all[wave];
  float* arow = arow_all[wave];
  uint32_t* mx = mx_all[wave];
  uint16_t* eslot = eslot_all[ATTN ? wave : 0];
  uint32_t* rcnt = rcnt_all[ATTN ? wave : 0];

  const int nhg = p.H / HPW;
  const int hg = blockIdx.x % nhg;  // consecutive workgroups (different XCDs) take different heads
  const int qb = (blockIdx.x / nhg) * kDW + wave;
  const int b = blockIdx.y;
  bool active = qb < p.nqb;
  if (active) {
    // A block holding a repeated position is computed by the gather kernel.
    const int* f = p.flags + ((int64_t)b * p.nqb + qb) * p.nchunk;
    for (int c = 0; c < p.nchunk; ++c) active &= f[c] == 0;
  }
  const int col = lane & 31, half = lane >> 5;
  const int q0 = qb * 32;
  const int h0 = hg * HPW;

  uint4 a[HPW][4];
  {
    const int t = q0 + col;
    const bool ok = active && t < p.T;
    const uint16_t* qr = p.q + b * p.qsb + (int64_t)(ok ? t : 0) * p.qst + half * 8;
#pragma unroll
    for (int hh = 0; hh < HPW; ++hh)
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
        a[hh][ks] = ok ? *reinterpret_cast<const uint4*>(qr + (h0 + hh) * p.qsh + ks * 16) : make_uint4(0, 0, 0, 0);
  }
  f32x16 acc[HPW][2];
#pragma unroll
  for (int hh = 0; hh < HPW; ++hh)
#pragma unroll
    for (int nb = 0; nb < 2; ++nb)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[hh][nb][r] = 0.f;
  if (lane < 33) {
#pragma unroll
    for (int hh = 0; hh < HPW; ++hh) {
      mrow[hh][lane] = lane < 32 ? -INFINITY : INFINITY;
    }
    if constexpr (ATTN) rcnt[lane] = 0u;
  }
  for (int i = lane; i < kPElems / 8; i += 64) {
    reinterpret_cast<uint4*>(phi)[i] = make_uint4(0, 0, 0, 0);
    reinterpret_cast<uint4*>(plo)[i] = make_uint4(0, 0, 0, 0);
  }
  // Row sums: this lane's share of row `col` (keys 8*half + 0..7 and 16 + 8*half + 0..7 of
  // each tile, the keys of its P·V operand), summed in a fixed order from hi and lo.
  float lpart[HPW];
#pragma unroll
  for (int hh = 0; hh < HPW; ++hh) lpart[hh] = 0.f;

  const uint32_t* mbase = p.mask + ((int64_t)b * p.nqb + (active ? qb : 0)) * p.S;
  const float sl2 = p.scale_log2;

  // Tile loads: per wave one 16-byte chunk per lane of K and one of V^T (1 KB each), loaded
  // into registers two tiles ahead and written to LDS one tile ahead.
  const int krow = 4 * wave + (lane >> 4);                 // key row of this lane's K chunk
  const int kchunk = (lane & 15) ^ (krow & 15);            // global chunk it loads
  const uint16_t* ksrc0 = p.k + b * p.ksb + (int64_t)(h0 + (kchunk >> 3)) * p.ksh + (kchunk & 7) * 8;
  const int vrow = 16 * wave + (lane >> 2);                // (head, d) row of this lane's V chunk
  const int vchunk = (lane & 3) ^ ((vrow >> 2) & 3);
  const uint16_t* vsrc0 = p.vt + (((int64_t)b * p.H + h0 + (vrow >> 6)) * 64 + (vrow & 63)) * p.Spad + vchunk * 8;
  auto gload = [&](int kb0, uint4& kr, uint4& vr) {
    const int key = min(kb0 + krow, p.S - 1);  // keys past S: any valid row (their P is 0)
    kr = *reinterpret_cast<const uint4*>(ksrc0 + (int64_t)key * p.kss);
    vr = *reinterpret_cast<const uint4*>(vsrc0 + kb0);
  };
  auto lstore = [&](int bf, const uint4& kr, const uint4& vr) {
    *reinterpret_cast<uint4*>(&ktile[bf][wave * 1024 + lane * 16]) = kr;
    *reinterpret_cast<uint4*>(&vtile[bf][wave * 1024 + lane * 16]) = vr;
  };
  // Loads in the tile loop are unconditional (clamped addresses): with no control flow around
  // them the compiler's memory waits count exactly the loads still needed.
  // The raw word is loaded a tile ahead; its validity select waits until the word is used.
  auto mask_raw = [&](int kb0) -> uint32_t { return mbase[min(kb0 + col, p.S - 1)]; };
  // Operand read offsets (bytes) within a tile.
  uint32_t koff[HPW][4], voff[HPW][2][2];
#pragma unroll
  for (int hh = 0; hh < HPW; ++hh) {
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) koff[hh][ks] = col * 256 + (((hh * 8 + 2 * ks + half) ^ (col & 15)) * 16);
#pragma unroll
    for (int nb = 0; nb < 2; ++nb)
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const int rr = hh * 64 + nb * 32 + col;
        voff[hh][nb][ks] = rr * 64 + (((2 * ks + half) ^ ((rr >> 2) & 3)) * 16);
      }
  }

  struct Ent {
    int sa, row, pa;
    bool ok;
  };
  auto decode = [&](int i, int nsel) {
    Ent en;
    en.ok = i < nsel;
    const int e = elist[en.ok ? i : 1024 + lane];
    const int r = e >> 6, ln = e & 63;
    const int row = tile_row(r, ln >> 5);
    en.sa = en.ok ? ((r >> 2) * 64 + ln) * 4 + (r & 3) : 0;
    en.row = en.ok ? row : 32;
    // P tile rows of 64 bytes, 16-byte chunk c of row rr at c ^ ((rr >> 2) & 3).
    en.pa = en.ok ? row * 32 + ((((ln & 31) >> 3) ^ ((row >> 2) & 3)) << 3) + (ln & 7) : 1024 + lane;
    return en;
  };

  // Tile t lives in LDS buffer t % kRing. While computing tile t a wave writes tile
  // t + kDist from registers into buffer (t + kDist) % kRing (last read before the last
  // barrier) and loads tile t + 2 kDist into the freed registers; the barrier after every
  // kDist tiles makes the next tiles visible. kDist register sets alternate by tile (no
  // register copies, which would wait for the loads). The wave's private LDS needs no
  // barrier (one wave).
  const int ntiles = (p.S + 31) / 32;
  const int last = (ntiles - 1) * 32;
  // Staging registers: named variables (an array of them indexed through the tile calls
  // would live in scratch memory).
  uint4 kra, vra, krb, vrb;
  {
    uint4 k0r, v0r;
    gload(0, k0r, v0r);
    lstore(0, k0r, v0r);
    if constexpr (kDist == 2) {
      gload(min(32, last), k0r, v0r);
      lstore(1, k0r, v0r);
    }
  }
  gload(min(32 * kDist, last), kra, vra);
  if constexpr (kDist == 2) gload(min(96, last), krb, vrb);
  uint32_t wraw = mask_raw(0);
  __syncthreads();
  auto tile = [&](int n, uint4& kr, uint4& vr, bool sync_after) {
    const int k0 = n * 32;
    const int buf = n & (kRing - 1);
    lstore((n + kDist) & (kRing - 1), kr, vr);  // past the last tile: never read
    gload(min(k0 + 64 * kDist, last), kr, vr);
    const uint32_t wnext = mask_raw(k0 + 32);  // past the last tile: unused
    const uint32_t w = (active && k0 + col < p.S) ? wraw : 0u;
    // This lane's rows 8g + 4*half + i (g, i < 4) are bits 8g + 4*half + i of w; bit r of
    // m16 is accumulator element r.
    const uint32_t xw = w >> (4 * half);
    const uint32_t m16 = (xw & 0xFu) | ((xw >> 4) & 0xF0u) | ((xw >> 8) & 0xF00u) | ((xw >> 12) & 0xF000u);
    if (__ballot(m16 != 0u) != 0ull) {
      const uint8_t* kt = ktile[buf];
      const uint8_t* vt = vtile[buf];
      // Compact the selected entries (lane order, then r): exclusive prefix of the counts.
      const int cnt = __popc(m16);
      const int incl = wave_scan_dpp(cnt);
      const int nsel = __builtin_amdgcn_readlane(incl, 63);
      {
        int at = incl - cnt;
        uint32_t mm = m16;
        while (__ballot(mm != 0u) != 0ull) {
          const bool has = mm != 0u;
          elist[has ? at : 1024 + lane] = (uint16_t)(((__ffs(mm) - 1) << 6) | lane);
          at += has ? 1 : 0;
          mm &= mm - 1u;
        }
      }
      lds_fence();
      const Ent e0 = decode(lane, nsel);  // entries 0..63; later chunks are decoded on the fly
      if constexpr (ATTN) {
        // Slots in ascending key order per row: the list is in key order and one atomic's
        // lanes are served in lane order.
        for (int c0 = 0; c0 < nsel; c0 += 64) {
          const Ent en = c0 == 0 ? e0 : decode(c0 + lane, nsel);
          if (en.ok) eslot[c0 + lane] = (uint16_t)atomicAdd(&rcnt[en.row], 1u);
        }
        lds_fence();
      }

      // Both heads' score products first: head 1's MFMAs run while head 0's softmax does.
      f32x16 sacc[HPW];
#pragma unroll
      for (int hh = 0; hh < HPW; ++hh) {
        sacc[hh] = f32x16{0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
          sacc[hh] = mma(E{}, a[hh][ks], *reinterpret_cast<const uint4*>(kt + koff[hh][ks]), sacc[hh]);
      }
#pragma unroll
      for (int hh = 0; hh < HPW; ++hh) {
        const f32x16 s = sacc[hh];
#pragma unroll
        for (int g = 0; g < 4; ++g)
          *reinterpret_cast<float4*>(&stage[(g * 64 + lane) * 4]) = make_float4(s[4 * g], s[4 * g + 1], s[4 * g + 2], s[4 * g + 3]);
        lds_fence();

        // A row's reference maximum moves only when one of its own entries of this tile
        // exceeds it by more than kLazy, and then to the largest such entry: every row's
        // arithmetic is independent of the other rows of the block (and of the chunking).
        // Entries 0..63 keep their score and maximum in registers.
        const float t0 = stage[e0.sa] * sl2;
        float mo0 = mrow[hh][e0.row];
        bool lift = __ballot(t0 > mo0 + kLazy) != 0ull;
        for (int c0 = 64; c0 < nsel; c0 += 64) {
          const Ent en = decode(c0 + lane, nsel);
          lift |= __ballot(stage[en.sa] * sl2 > mrow[hh][en.row] + kLazy) != 0ull;
        }
        if (lift) {
          if (lane < 32) mx[lane] = f2key(mrow[hh][lane]);
          lds_fence();
          for (int c0 = 0; c0 < nsel; c0 += 64) {
            const Ent en = c0 == 0 ? e0 : decode(c0 + lane, nsel);
            const float t = stage[en.sa] * sl2;
            if (t > mrow[hh][en.row] + kLazy) atomicMax(&mx[en.row], f2key(t));
          }
          lds_fence();
          if (lane < 32) {
            const float mold = mrow[hh][lane];
            const float mnew = key2f(mx[lane]);
            float alpha = 1.f;
            if (mnew > mold) {
              alpha = fexp2(mold - mnew);
              mrow[hh][lane] = mnew;
            }
            arow[lane] = alpha;
          }
          lds_fence();
          lpart[hh] *= arow[col];
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const float4 al = *reinterpret_cast<const float4*>(&arow[8 * g + 4 * half]);
            const float alv[4] = {al.x, al.y, al.z, al.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              acc[hh][0][4 * g + i] *= alv[i];
              acc[hh][1][4 * g + i] *= alv[i];
            }
          }
          mo0 = mrow[hh][e0.row];
        }
        auto emit = [&](int pa_, float t, float mo) {
          const float pv = fexp2(t - mo);
          const uint16_t hb = to_half_bits(E{}, pv);
          phi[pa_] = hb;
          plo[pa_] = to_half_bits(E{}, pv - from_half_bits(E{}, hb));  // exact difference
        };
        emit(e0.pa, t0, mo0);
        for (int c0 = 64; c0 < nsel; c0 += 64) {
          const Ent en = decode(c0 + lane, nsel);
          emit(en.pa, stage[en.sa] * sl2, mrow[hh][en.row]);
        }
        if constexpr (ATTN) {
          auto keep = [&](const Ent& en, int i, float t) {
            if (en.ok) p.sws[(((int64_t)b * p.T + q0 + en.row) * p.K + eslot[i]) * p.H + h0 + hh] = t;
          };
          keep(e0, lane, t0);
          for (int c0 = 64; c0 < nsel; c0 += 64) {
            const Ent en = decode(c0 + lane, nsel);
            keep(en, c0 + lane, stage[en.sa] * sl2);
          }
        }
        lds_fence();
        // P enters the P·V product as its hi and lo parts: two products, weights with ~16
        // significant bits, close to the fp32 p of the gather kernel.
        uint4 pa[2], pl[2];
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          const int pofs = col * 32 + (((2 * ks + half) ^ ((col >> 2) & 3)) << 3);
          pa[ks] = *reinterpret_cast<const uint4*>(&phi[pofs]);
          pl[ks] = *reinterpret_cast<const uint4*>(&plo[pofs]);
        }
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) lpart[hh] = sum8(E{}, pa[ks], lpart[hh]);
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) lpart[hh] = sum8(E{}, pl[ks], lpart[hh]);
#pragma unroll
        for (int nb = 0; nb < 2; ++nb)
#pragma unroll
          for (int ks = 0; ks < 2; ++ks) {
            const uint4 vb = *reinterpret_cast<const uint4*>(vt + voff[hh][nb][ks]);
            acc[hh][nb] = mma(E{}, pa[ks], vb, acc[hh][nb]);
            acc[hh][nb] = mma(E{}, pl[ks], vb, acc[hh][nb]);
          }
        // Clear the written P entries for the next use of the tile.
        phi[e0.pa] = 0;
        plo[e0.pa] = 0;
        for (int c0 = 64; c0 < nsel; c0 += 64) {
          const int pa_ = decode(c0 + lane, nsel).pa;
          phi[pa_] = 0;
          plo[pa_] = 0;
        }
        lds_fence();
      }
    }
    wraw = wnext;
    if (sync_after) {
      // This wave's LDS writes of the next pair's tiles are done; after the barrier every
      // wave's are, and every wave is done with this pair's buffers before they are refilled.
      // No wait for the global loads in flight (a raw barrier, unlike __syncthreads).
      __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
      asm volatile("" ::: "memory");
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
    }
  };
  if constexpr (kDist == 2) {
    for (int n = 0; n < ntiles; n += 2) {
      tile(n, kra, vra, false);
      if (n + 1 < ntiles) tile(n + 1, krb, vrb, true);
    }
  } else {
    for (int n = 0; n < ntiles; ++n) tile(n, kra, vra, true);
  }
  if (!active) return;

  // o = O / l, lse = (m + log2 l) ln 2; rows without any selected key give o = 0, lse = -inf.
  // l of row r = the shares of lanes r and r + 32.
  float (*lrow)[32] = reinterpret_cast<float (*)[32]>(stage);  // the staging area is free now
#pragma unroll
  for (int hh = 0; hh < HPW; ++hh) {
    if (half == 1) lrow[hh][col] = lpart[hh];
    lds_fence();
    if (half == 0) lrow[hh][col] = lpart[hh] + lrow[hh][col];
    lds_fence();
  }
#pragma unroll
  for (int hh = 0; hh < HPW; ++hh) {
    const int h = h0 + hh;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const float4 lv = *reinterpret_cast<const float4*>(&lrow[hh][8 * g + 4 * half]);
      const float lvv[4] = {lv.x, lv.y, lv.z, lv.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int t = q0 + 8 * g + 4 * half + i;
        if (t < p.T) {
          const float inv = lvv[i] > 0.f ? __frcp_rn(lvv[i]) : 0.f;
          uint16_t* orow = p.o + b * p.osb + (int64_t)t * p.ost + h * p.osh + col;
          orow[0] = to_half_bits(E{}, acc[hh][0][4 * g + i] * inv);
          orow[32] = to_half_bits(E{}, acc[hh][1][4 * g + i] * inv);
        }
      }
    }
    if (lane < 32 && q0 + lane < p.T && p.lse) {
      const float l = lrow[hh][lane];
      p.lse[((int64_t)b * p.T + q0 + lane) * p.H + h] = l > 0.f ? (mrow[hh][lane] + flog2(l)) * kDLn2 : -INFINITY;
    }
  }
}

// ---------------------------------------------------------------------------------------
// attn_sum from the slot-indexed scores: one wave per query row. The row's valid positions,
// sorted ascending, are in slot order: slot i holds the i-th smallest selected key. So
// attn_sum[t, j] = sum_h exp2(sws[t, i(j), h] - lse2[t, h]) with i(j) the rank of position j
// (a wave bitonic sort of (position, j)); invalid positions give 0. With KL, the row's
// indexer KL loss follows from the same registers (the per-row term of
// sparse_indexer_kl_loss, indexer_kl_fused.py:8-155, as in the gather kernel's epilogue).
// Rows of blocks flagged for a repeated position were computed by the gather kernel.
// ---------------------------------------------------------------------------------------
struct AttnSumParams {
  const int32_t* pos;
  int64_t psb, pst;
  const float* sws;
  const float* lse;  // natural log, [B, T, H]
  const int* flags;
  float* attn_sum;   // [B, T, K]
  const void* logits;
  int logits_dt;
  int64_t lsb, lst;
  float kl_eps;
  float* row_loss;
  int B, T, S, H, K, nqb, nchunk;
};

__device__ __forceinline__ float as_load(int dt, const void* base, int64_t i) {
  if (dt == GW_DTYPE_FP32) return static_cast<const float*>(base)[i];
  const uint32_t u = static_cast<const uint16_t*>(base)[i];
  if (dt == GW_DTYPE_BF16) return __uint_as_float(u << 16);
  return (float)__builtin_bit_cast(_Float16, (uint16_t)u);
}

__device__ __forceinline__ float as_wave_sum(float x) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) x += __shfl_xor(x, off);
  return x;
}
__device__ __forceinline__ float as_wave_max(float x) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) x = fmaxf(x, __shfl_xor(x, off));
  return x;
}

template <int R, bool KL>
__global__ __launch_bounds__(256) void dense_attn_sum_kernel(const AttnSumParams p) {
  __shared__ float lse2_s[4][64];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t row = (int64_t)blockIdx.x * 4 + wave;
  if (row >= (int64_t)p.B * p.T) return;  // whole wave; no barriers below
  const int b = (int)(row / p.T), t = (int)(row - (int64_t)b * p.T);
  {
    const int* f = p.flags + ((int64_t)b * p.nqb + (t >> 5)) * p.nchunk;
    bool flagged = false;
    for (int c = 0; c < p.nchunk; ++c) flagged |= f[c] != 0;
    if (flagged) return;
  }
  if (lane < p.H) lse2_s[wave][lane] = p.lse[row * p.H + lane] * kDLog2e;
  const int32_t* prow = p.pos + b * p.psb + (int64_t)t * p.pst;
  uint64_t key[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int j = r * 64 + lane;
    const int32_t ps = j < p.K ? prow[j] : -1;
    const bool ok = ps >= 0 && ps < p.S;
    // invalid positions (and padding past K) sort last, after every valid key
    key[r] = ((uint64_t)(ok ? (uint32_t)ps : 0xFFFFFFFFu) << 32) | (uint32_t)j;
  }
  wave_bitonic_sort<R>(key);
  lds_fence();
  const float* srow = p.sws + row * (int64_t)p.K * p.H;
  float av[R], zv[R];
  float sa = 0.f, mz = -INFINITY;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int i = r * 64 + lane;  // slot = sorted rank
    const int j = (int)(uint32_t)key[r];
    const bool ok = (key[r] >> 32) != 0xFFFFFFFFull;
    float sum = 0.f;
    if (ok) {
      const float* sp = srow + (int64_t)i * p.H;
      for (int h = 0; h < p.H; ++h) {
        const float l2 = lse2_s[wave][h];
        if (l2 != -INFINITY) sum += fexp2(sp[h] - l2);
      }
    }
    av[r] = sum;
    zv[r] = -INFINITY;
    if (j < p.K) {
      p.attn_sum[row * p.K + j] = sum;
      if constexpr (KL) {
        zv[r] = as_load(p.logits_dt, p.logits, b * p.lsb + (int64_t)t * p.lst + j);
        sa += sum;
        mz = fmaxf(mz, zv[r]);
      }
    }
  }
  if constexpr (KL) {
    sa = as_wave_sum(sa);
    mz = as_wave_max(mz);
    float se = 0.f;
#pragma unroll
    for (int r = 0; r < R; ++r)
      if ((int)(uint32_t)key[r] < p.K) se += expf(zv[r] - mz);
    se = as_wave_sum(se);
    const float lse = mz + logf(se);
    const float denom = sa + p.kl_eps;
    float acc = 0.f;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if ((int)(uint32_t)key[r] < p.K) {
        const float pj = av[r] / denom;
        acc += pj * (logf(pj + p.kl_eps) - (zv[r] - lse));
      }
    }
    acc = as_wave_sum(acc);
    if (lane == 0) p.row_loss[row] = acc;
  }
}

struct DenseLayout {
  size_t mask, flags, vt, sws, total;
  int nqb, nchunk, spad;
};

DenseLayout dense_layout(int64_t B, int64_t T, int64_t S, int64_t H, int64_t K, bool attn) {
  DenseLayout L;
  L.nqb = (int)((T + 31) / 32);
  L.nchunk = (int)((S + kMaskChunk - 1) / kMaskChunk);
  if (L.nchunk < 1) L.nchunk = 1;
  L.spad = (int)((S + 63) / 64 * 64);
  auto up = [](size_t x) { return (x + 255) / 256 * 256; };
  size_t o = 0;
  L.mask = o;
  o = up(o + (size_t)B * L.nqb * (size_t)S * 4);
  L.flags = o;
  o = up(o + (size_t)B * L.nqb * (size_t)L.nchunk * 4);
  L.vt = o;
  o = up(o + (size_t)B * (size_t)H * 64 * (size_t)L.spad * 2);
  L.sws = o;
  if (attn) o = up(o + (size_t)B * (size_t)T * (size_t)K * (size_t)H * 4);
  L.total = o;
  return L;
}

constexpr int kDenseAttnMaxK = 1024;  // attn_sum: a row's positions sorted in registers

int pow2_at_least(int64_t x) {
  int r = 1;
  while (r < x) r <<= 1;
  return r;
}

template <bool KL>
int launch_attn_sum(const AttnSumParams& p, int rows, hipStream_t st) {
  const dim3 grid((unsigned)((rows + 3) / 4));
  switch (pow2_at_least((p.K + 63) / 64)) {
    case 1: hipLaunchKernelGGL((dense_attn_sum_kernel<1, KL>), grid, dim3(256), 0, st, p); break;
    case 2: hipLaunchKernelGGL((dense_attn_sum_kernel<2, KL>), grid, dim3(256), 0, st, p); break;
    case 4: hipLaunchKernelGGL((dense_attn_sum_kernel<4, KL>), grid, dim3(256), 0, st, p); break;
    case 8: hipLaunchKernelGGL((dense_attn_sum_kernel<8, KL>), grid, dim3(256), 0, st, p); break;
    default: hipLaunchKernelGGL((dense_attn_sum_kernel<16, KL>), grid, dim3(256), 0, st, p); break;
  }
  GW_HIP_LAUNCH_CHECK("dense_attn_sum_kernel launch");
  return GW_OK;
}

}  // namespace
}  // namespace gw

extern "C" size_t gw_sparse_attn_fwd_dense_workspace_size(int64_t B, int64_t T, int64_t S, int64_t H, int64_t D,
                                                          int64_t K, int want_attn_sum) {
  if (B <= 0 || T <= 0 || S <= 0 || H <= 0 || K <= 0 || D != 64) return 0;
  return gw::dense_layout(B, T, S, H, K, want_attn_sum != 0).total;
}

extern "C" int gw_sparse_attn_fwd_dense(int dtype, const void* q, const int64_t* q_strides, const void* k,
                                        const int64_t* k_strides, const void* v, const int64_t* v_strides,
                                        const int32_t* kv_pos, int64_t pos_stride_b, int64_t pos_stride_t,
                                        void* o, const int64_t* o_strides, float* lse, float* attn_sum, int64_t B,
                                        int64_t T, int64_t S, int64_t H, int64_t D, int64_t K, float softmax_scale,
                                        const void* logits, int logits_dtype, int64_t logits_stride_b,
                                        int64_t logits_stride_t, float eps, float* row_loss, void* workspace,
                                        size_t workspace_bytes, void* stream) {
  using namespace gw;
  clear_error();
  GW_CHECK_ARG(dtype == GW_DTYPE_BF16 || dtype == GW_DTYPE_FP16, "unsupported dtype code %d", dtype);
  GW_CHECK_ARG(B >= 0 && T >= 0 && S >= 0 && H >= 1 && K >= 0, "invalid sizes B=%lld T=%lld S=%lld H=%lld K=%lld",
               (long long)B, (long long)T, (long long)S, (long long)H, (long long)K);
  if (D != 64) return set_error(GW_ERR_UNSUPPORTED, "the dense forward needs head dim 64, got %lld", (long long)D);
  if (H % kDHpw != 0)
    return set_error(GW_ERR_UNSUPPORTED, "the dense forward needs an even head count, got %lld", (long long)H);
  const bool want_attn = attn_sum != nullptr;
  const bool want_kl = logits != nullptr;
  if (want_attn && K > kDenseAttnMaxK)
    return set_error(GW_ERR_UNSUPPORTED, "the dense forward computes attn_sum for K <= %d, got %lld", kDenseAttnMaxK,
                     (long long)K);
  if (B == 0 || T == 0) return GW_OK;
  GW_CHECK_ARG(K >= 1 && S >= 1, "kv_positions must have at least one candidate and S >= 1");
  GW_CHECK_ARG(q && k && v && kv_pos && o, "null tensor pointer");
  GW_CHECK_ARG(q_strides && k_strides && v_strides && o_strides, "null stride array");
  GW_CHECK_ARG(aligned16(q) && aligned16(k) && aligned16(v) && aligned16(o), "q/k/v/o must be 16-byte aligned");
  for (int i = 0; i < 3; ++i)
    GW_CHECK_ARG(q_strides[i] % 8 == 0 && k_strides[i] % 8 == 0 && v_strides[i] % 8 == 0 && o_strides[i] % 8 == 0,
                 "b/t/h strides must be multiples of 8 elements");
  GW_CHECK_ARG(B <= 65535 && T < (1ll << 31) && S < (1ll << 30) && K < (1ll << 31), "size exceeds the grid range");
  GW_CHECK_ARG(!want_kl || want_attn, "the fused KL loss needs attn_sum");
  GW_CHECK_ARG(!want_attn || lse != nullptr, "attn_sum needs the lse output");
  if (want_kl) {
    GW_CHECK_ARG(row_loss != nullptr, "null row_loss pointer");
    GW_CHECK_ARG(logits_dtype == GW_DTYPE_BF16 || logits_dtype == GW_DTYPE_FP16 || logits_dtype == GW_DTYPE_FP32,
                 "unsupported logits dtype code %d", logits_dtype);
    GW_CHECK_ARG(eps >= 0.f, "eps must be non-negative, got %g", (double)eps);
  }
  const DenseLayout L = dense_layout(B, T, S, H, K, want_attn);
  GW_CHECK_ARG((int64_t)L.nqb * (H / kDHpw) < (1ll << 31), "too many query blocks");
  GW_CHECK_ARG(workspace != nullptr && workspace_bytes >= L.total && aligned16(workspace),
               "the dense forward needs a 16-byte aligned %zu-byte workspace, got %zu", L.total, workspace_bytes);
  hipStream_t st = static_cast<hipStream_t>(stream);
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  uint32_t* mask = reinterpret_cast<uint32_t*>(ws + L.mask);
  int* flags = reinterpret_cast<int*>(ws + L.flags);
  uint16_t* vt = reinterpret_cast<uint16_t*>(ws + L.vt);
  float* sws = want_attn ? reinterpret_cast<float*>(ws + L.sws) : nullptr;

  {
    const int vec = (K % 4 == 0 && pos_stride_t % 4 == 0 && pos_stride_b % 4 == 0 &&
                     (reinterpret_cast<uintptr_t>(kv_pos) & 15) == 0)
                        ? 1
                        : 0;
    hipLaunchKernelGGL(dense_mask_kernel, dim3(L.nqb, L.nchunk, (unsigned)B), dim3(256), 0, st, kv_pos, pos_stride_b,
                       pos_stride_t, (int)T, (int)S, (int)K, L.nqb, L.nchunk, vec, mask, flags);
    GW_HIP_LAUNCH_CHECK("dense_mask_kernel launch");
  }
  hipLaunchKernelGGL(dense_vt_kernel, dim3(L.spad / 64, (unsigned)H, (unsigned)B), dim3(256), 0, st,
                     static_cast<const uint16_t*>(v), v_strides[0], v_strides[1], v_strides[2], (int)S, L.spad,
                     (int)H, vt);
  GW_HIP_LAUNCH_CHECK("dense_vt_kernel launch");

  DenseParams p;
  p.q = static_cast<const uint16_t*>(q);
  p.k = static_cast<const uint16_t*>(k);
  p.vt = vt;
  p.mask = mask;
  p.flags = flags;
  p.o = static_cast<uint16_t*>(o);
  p.lse = lse;
  p.qsb = q_strides[0]; p.qst = q_strides[1]; p.qsh = q_strides[2];
  p.ksb = k_strides[0]; p.kss = k_strides[1]; p.ksh = k_strides[2];
  p.osb = o_strides[0]; p.ost = o_strides[1]; p.osh = o_strides[2];
  p.T = (int)T;
  p.S = (int)S;
  p.Spad = L.spad;
  p.H = (int)H;
  p.nqb = L.nqb;
  p.nchunk = L.nchunk;
  p.scale_log2 = softmax_scale * kDLog2e;
  p.sws = sws;
  p.K = (int)K;
  const dim3 grid((unsigned)((L.nqb + kDW - 1) / kDW * (H / kDHpw)), (unsigned)B);
  if (dtype == GW_DTYPE_BF16) {
    if (want_attn)
      hipLaunchKernelGGL((dense_attn_kernel<BF16, true>), grid, dim3(kDW * 64), 0, st, p);
    else
      hipLaunchKernelGGL((dense_attn_kernel<BF16, false>), grid, dim3(kDW * 64), 0, st, p);
  } else {
    if (want_attn)
      hipLaunchKernelGGL((dense_attn_kernel<FP16, true>), grid, dim3(kDW * 64), 0, st, p);
    else
      hipLaunchKernelGGL((dense_attn_kernel<FP16, false>), grid, dim3(kDW * 64), 0, st, p);
  }
  GW_HIP_LAUNCH_CHECK("dense_attn_kernel launch");
  if (want_attn) {
    AttnSumParams ap;
    ap.pos = kv_pos;
    ap.psb = pos_stride_b;
    ap.pst = pos_stride_t;
    ap.sws = sws;
    ap.lse = lse;
    ap.flags = flags;
    ap.attn_sum = attn_sum;
    ap.logits = logits;
    ap.logits_dt = logits_dtype;
    ap.lsb = logits_stride_b;
    ap.lst = logits_stride_t;
    ap.kl_eps = eps;
    ap.row_loss = row_loss;
    ap.B = (int)B;
    ap.T = (int)T;
    ap.S = (int)S;
    ap.H = (int)H;
    ap.K = (int)K;
    ap.nqb = L.nqb;
    ap.nchunk = L.nchunk;
    const int rows = (int)(B * T);
    const int rc = want_kl ? launch_attn_sum<true>(ap, rows, st) : launch_attn_sum<false>(ap, rows, st);
    if (rc != GW_OK) return rc;
  }
  // Blocks with a repeated position: the gather kernel (it returns at once for the others),
  // with attn_sum and the KL loss when asked (its score workspace is the same region).
  return attn_fwd_flagged_blocks(dtype, q, q_strides, k, k_strides, v, v_strides, kv_pos, pos_stride_b, pos_stride_t,
                                 o, o_strides, lse, attn_sum, B, T, S, H, D, K, softmax_scale, logits, logits_dtype,
                                 logits_stride_b, logits_stride_t, eps, row_loss, sws,
                                 want_attn ? (size_t)B * T * K * H * 4 : 0, flags, L.nqb, L.nchunk, stream);
}
