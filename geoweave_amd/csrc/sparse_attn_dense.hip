// Sparse-index attention forward as a masked dense pass on the matrix cores (gfx950, D = 64).
//
// The reference forms softmax(q·k_s)·v_s over the keys s each query selected by gathering
// their K and V rows (_fwd_kernel, sparse_index_flash_attn.py:129-259). For 16 heads of 64 a gathered
// (query, key) pair moves 4 KiB; when a query selects a few per cent of all keys (1,024 of
// 43,968 at 32 views) computing every (query, key) product on the matrix cores costs less
// than gathering the selected ones. This file does that: per 32 queries x 32 keys and head,
// S^T = K Q^T and O^T += V^T P^T are v_mfma_f32_32x32x16 products, and the selection enters
// as the initial accumulator of S^T (0 where the query selected the key, -inf elsewhere), so P
// is zero at every pair the query did not select and O, the row sums and the lse are those
// of the sparse attention, up to fp32 summation order and the fp16 rounding of P.
//
// Transposed products keep the softmax in registers: the S^T accumulator of a lane holds 16
// keys of one query (lanes l and l ^ 32 share the query), so the row maximum is a reduction
// within the lane and one v_permlane32_swap, and the exponentiated entries packed to fp16 are
// already the lane's B operand of the P·V product (V^T stored with the keys in that operand
// order). V enters in fp16 scaled per column by an exact power of two that fits its range.
// P holds 11 significant bits (the reference's fp32 weights, rounded to nearest); the row
// sums add the fp32 weights.
//
// Online softmax with a lazy reference maximum: the weights p = exp2(t - m) of a sub-tile are
// formed with the query's current m, and m is raised (O and the row sum rescaled, the weights
// formed again) only when a lane's weights sum to more than kSumCap — the sum bounds every
// weight, so P fits fp16 without overflow and no per-tile maximum is needed otherwise. The
// final o = O / l and lse = m + log2(l) do not depend on which m was used.
//
// Pieces (all on the caller's stream):
//   dense_mask_kernel  — selection words per (32-key sub-tile, query) (LDS atomic OR per listed
//                        position, per chunk of keys). A position listed twice for one query
//                        (the atomic returns the bit already set) flags the query's 32-query
//                        block: the gather kernel then computes that block, since the
//                        reference counts a repeated position twice.
//   dense_vmax_kernel  — largest |v| per (head, d) column, for the fp16 scaling of V; it also
//                        flags a batch element whose K or V holds an inf or nan anywhere:
//                        the dense products would carry it from rows a query did not select
//                        (0 * inf, -inf + inf), so such a batch element is computed by the
//                        gather kernel, which reads only the selected rows, as the reference
//                        does.
//   dense_vt_kernel    — V^T as [B][H][64][S_pad] fp16 (S_pad = S rounded up to 128, zero
//                        padded), keys in operand order: one 16-byte load per operand chunk.
//   dense_attn_kernel  — 4 waves per workgroup, each on two 32-query blocks, all on one
//                        head: each K and V^T tile is read from memory once per workgroup
//                        and shared through LDS, and each K and V^T operand read from LDS
//                        feeds the products of both blocks.
#include <math.h>

#include "gw_attn.h"
#include "gw_common.h"
#include "gw_dense.h"
#include "gw_select.h"
#include "gw_sort.h"

namespace gw {
namespace {

constexpr float kSumCap = 32768.f;  // a lane's weights of one sub-tile sum to at most this

// ---------------------------------------------------------------------------------------
// V enters the P·V product in fp16, scaled per (head, d) column by a power of two 2^e that
// puts the column's largest |v| in [2^14, 2^15): the scaling is exact, every scaled value
// fits fp16, and values down to 2^-28 of the column's largest stay normal. o is scaled back
// by 2^-e. dense_vmax_kernel takes the column maxima (as ordered bit patterns of
// non-negative floats, atomic max); columns that are all zero or hold inf/nan keep e = 0.
// It reads the K rows of the same keys and head too, and sets bad[b] when any K or V value
// of the batch element is an inf or a nan (exponent field all ones).
// ---------------------------------------------------------------------------------------
__device__ __forceinline__ int vscale_exp(uint32_t bits) {
  const float mx = __uint_as_float(bits);
  if (!(mx > 0.f) || !(mx <= 3.4028234663852886e38f)) return 0;
  int x;
  frexpf(mx, &x);  // mx = f 2^x, f in [0.5, 1)
  return min(15 - x, 126);
}

// LDS byte address of a pointer into a __shared__ array (the operand of a ds_* instruction).
__device__ __forceinline__ uint32_t lds_addr(const float* p) {
  return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const float*)p;
}

constexpr int kVmaxKeys = 256;  // keys per workgroup of dense_vmax_kernel (one head)

__global__ __launch_bounds__(256) void dense_vmax_kernel(const uint16_t* __restrict__ v, int64_t vsb, int64_t vss,
                                                         int64_t vsh, const uint16_t* __restrict__ k, int64_t ksb,
                                                         int64_t kss, int64_t ksh, int S, int H, int in_fp16,
                                                         uint32_t* __restrict__ vmax, int* __restrict__ bad) {
  __shared__ float part[4][64];
  const int h = blockIdx.y, b = blockIdx.z;
  const int dc = threadIdx.x & 7, kr = threadIdx.x >> 3;  // 16-byte chunk of the row, key
  const int s0 = blockIdx.x * kVmaxKeys;
  const uint16_t* src = v + b * vsb + h * vsh + dc * 8;
  const uint16_t* ksrc = k + b * ksb + h * ksh + dc * 8;
  const uint32_t e = in_fp16 ? 0x7C00u : 0x7F80u;
  float mx[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) mx[i] = 0.f;
  uint4 val[8], kval[8];
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    const int s = s0 + kr + 32 * u;
    val[u] = s < S ? *reinterpret_cast<const uint4*>(src + (int64_t)s * vss) : make_uint4(0, 0, 0, 0);
    kval[u] = s < S ? *reinterpret_cast<const uint4*>(ksrc + (int64_t)s * kss) : make_uint4(0, 0, 0, 0);
  }
  uint32_t nf = 0u;
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    const uint32_t w[4] = {val[u].x, val[u].y, val[u].z, val[u].w};
    const uint32_t kw[4] = {kval[u].x, kval[u].y, kval[u].z, kval[u].w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      mx[2 * i] = fmaxf(mx[2 * i], fabsf(in_to_float(in_fp16, w[i] & 0xFFFFu)));
      mx[2 * i + 1] = fmaxf(mx[2 * i + 1], fabsf(in_to_float(in_fp16, w[i] >> 16)));
      nf |= nonfinite2(w[i], e) | nonfinite2(kw[i], e);
    }
  }
  if (nf != 0u) bad[b] = 1;  // every writer stores the same value
  // lanes with the same chunk: xor 8, 16, 32; then the four waves
#pragma unroll
  for (int i = 0; i < 8; ++i) {
#pragma unroll
    for (int off = 8; off < 64; off <<= 1) mx[i] = fmaxf(mx[i], __shfl_xor(mx[i], off));
  }
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (lane < 8) {
#pragma unroll
    for (int i = 0; i < 8; ++i) part[wave][lane * 8 + i] = mx[i];
  }
  __syncthreads();
  if (threadIdx.x < 64) {
    const float m4 = fmaxf(fmaxf(part[0][threadIdx.x], part[1][threadIdx.x]), fmaxf(part[2][threadIdx.x], part[3][threadIdx.x]));
    atomicMax(vmax + ((int64_t)b * H + h) * 64 + threadIdx.x, __float_as_uint(m4));
  }
}

// ---------------------------------------------------------------------------------------
// V^T per head in fp16 (scaled as above): vt[b][h][d][s'], s' < S_pad, zero past S. Within
// every 16 keys, key s sits at s' = s with bits 2 and 3 exchanged: that is the order in which
// a lane's S^T accumulator entries enter the P·V product as its B operand (entries r < 8 of
// lane l are keys 8(r/4) + 4(l/32) + r%4, which the operand's k-chunk l/32 lists as k =
// 8(l/32) + r), so each V^T operand chunk is 8 consecutive s', one 16-byte load.
// ---------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void dense_vt_kernel(const uint16_t* __restrict__ v, int64_t vsb, int64_t vss,
                                                       int64_t vsh, int S, int Spad, int H, int in_fp16,
                                                       const uint32_t* __restrict__ vmax,
                                                       uint16_t* __restrict__ vt) {
  __shared__ __align__(16) uint16_t tile[64][72];  // [d][key], rows of 144 bytes
  __shared__ int es[64];
  const int s0 = blockIdx.x * 64, h = blockIdx.y, b = blockIdx.z;
  if (threadIdx.x < 64) es[threadIdx.x] = vscale_exp(vmax[((int64_t)b * H + h) * 64 + threadIdx.x]);
  __syncthreads();
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
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int d = c * 8 + 2 * i + u;
        const float f = ldexpf(in_to_float(in_fp16, u ? w[i] >> 16 : w[i] & 0xFFFFu), es[d]);
        tile[d][key] = __builtin_bit_cast(uint16_t, (_Float16)f);
      }
    }
  }
  __syncthreads();
#pragma unroll
  for (int it = 0; it < 2; ++it) {
    const int idx = threadIdx.x + it * 256;
    const int d = idx >> 3, kc = idx & 7;
    // s' = 8 kc + 0..7 holds keys 16 (kc/2) + 4 (kc%2) + {0..3, 8..11}
    const int k0 = 16 * (kc >> 1) + 4 * (kc & 1);
    const uint2 lo = *reinterpret_cast<const uint2*>(&tile[d][k0]);
    const uint2 hi = *reinterpret_cast<const uint2*>(&tile[d][k0 + 8]);
    *reinterpret_cast<uint4*>(vt + (((int64_t)b * H + h) * 64 + d) * Spad + s0 + kc * 8) =
        make_uint4(lo.x, lo.y, hi.x, hi.y);
  }
}

// ---------------------------------------------------------------------------------------
// The attention, transposed: per sub-tile of 32 keys a wave forms S^T = K Q^T (32 keys x 32
// queries), so accumulator entry r of lane l holds query l%32 and key 8(r/4) + 4(l/32) + r%4:
// every entry of a lane belongs to one query, and lanes l and l ^ 32 share it. The
// exponentiated entries, packed to fp16, are already the B operand of O^T += V^T P^T
// (32 keys x 32 queries, two k-steps of 16) — P never leaves the registers. The selection
// enters as the initial accumulator of S^T: 0 where the query selected the key, -inf
// elsewhere, so p = exp2(-inf) = 0 there.
// ---------------------------------------------------------------------------------------
struct DenseParams {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* vt;
  const uint32_t* mask;
  const uint32_t* vmax;
  const int* flags;
  const int* bad;  // [B]: K or V of the batch element holds an inf or nan
  uint16_t* o;
  float* lse;
  int64_t qsb, qst, qsh;
  int64_t ksb, kss, ksh;
  int64_t osb, ost, osh;
  int T, S, Spad, H, nqb, tpad, nchunk;
  float scale_log2;
  // attn_sum (ATTN kernels only): the score q.k (not yet scaled) of every selected (query,
  // key) and head, sws[((b * H + h) * T + t) * sws_row(K) + slot] (head-major: one
  // workgroup, which holds one head, fills whole cache lines of a row), slot = rank of the
  // key among the query's selected keys in ascending key order.
  float* sws;
  int K;
};

// attn_sum score rows are K rounded up to 8, plus kSwsPad floats long (32-byte aligned): the
// forward writes a query's selected scores 4 slots at a time, so the last 4 written may run
// past its last slot in use (those are never read).
constexpr int kSwsPad = 8;
__host__ __device__ __forceinline__ int64_t sws_row(int64_t K) { return (K + 7) / 8 * 8 + kSwsPad; }

// Waves per workgroup, sharing each K/V tile. Two workgroups share a CU (two waves per SIMD
// from different workgroups): one wave's barrier or memory wait is not the other's.
constexpr int kDW = 4;
// Limits of the 32-bit lane offsets of the tile loads: a K token stride below 2^23 elements
// (2^24 bytes, a 24-bit multiply), 64 rows of V^T (S padded to 128) below 2^32 bytes.
constexpr int64_t kDenseMaxKRowStride = 1ll << 23;
constexpr int64_t kDenseMaxS = (1ll << 25) - 128;
constexpr int kQPW = 2;  // 32-query blocks per wave (one head): each K and V^T operand feeds two products
constexpr int kQBW = kDW * kQPW;  // 32-query blocks per workgroup
static_assert(kDW == 4, "the tile staging moves two K and two V^T rows of 64 per thread");

template <typename E, bool ATTN>
__global__ __launch_bounds__(kDW * 64, 2) void dense_attn_kernel(const DenseParams p) {
  // Two buffers of each tile, as separate arrays indexed at compile time (the tile loop is
  // unrolled by two): the compiler then knows which LDS reads a pending direct-to-LDS load
  // can overlap, and waits for none of them in the loop.
  // Tiles of kHT 64-key halves: one with attn_sum (whose staging rows need the LDS), two
  // without.
  constexpr int kHT = ATTN ? 1 : 2;
  __shared__ __align__(16) uint8_t ktile0[kHT * 8192], ktile1[kHT * 8192];
  __shared__ __align__(16) uint8_t vtile0[kHT * 8192], vtile1[kHT * 8192];
  __shared__ float vsc_s[64];
  // attn_sum: per query of the wave (block a, column col) a row of 44 floats (176 bytes, an odd
  // multiple of 16, so the 16-byte stores of 16 consecutive lanes touch distinct banks): a ring
  // of 8 slots that gathers the query's selected scores until 4 consecutive slots of its row
  // are complete (bytes 0-31), then the sub-tile's 32 scores in key order (bytes 32-159).
  constexpr int kArow = 44;
  __shared__ __align__(16) float ascore[ATTN ? kDW * 32 * kQPW * kArow : 4];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: addresses built from it stay scalar
  const int h = blockIdx.x % p.H;  // consecutive workgroups (different XCDs) take different heads
  const int qb0 = (blockIdx.x / p.H) * kQBW + wave * kQPW;  // this wave's blocks qb0, qb0 + 1 (< nqb_pad)
  const int b = blockIdx.y;
  const int col = lane & 31, half = lane >> 5;
  const float sl2 = p.scale_log2;
  int tq[kQPW];  // this lane's query in each block
#pragma unroll
  for (int a = 0; a < kQPW; ++a) tq[a] = (qb0 + a) * 32 + col;

  if (tid < 64) vsc_s[tid] = ldexpf(1.f, -vscale_exp(p.vmax[((int64_t)b * p.H + h) * 64 + tid]));

  // Q^T operands (B of S^T = K Q^T): query tq[a], dims 16 ks + 8 half + 0..7.
  uint4 qa[kQPW][4];
#pragma unroll
  for (int a = 0; a < kQPW; ++a) {
    const bool ok = tq[a] < p.T;
    const uint16_t* qr = p.q + b * p.qsb + (int64_t)(ok ? tq[a] : 0) * p.qst + h * p.qsh + half * 8;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
      qa[a][ks] = ok ? *reinterpret_cast<const uint4*>(qr + ks * 16) : make_uint4(0, 0, 0, 0);
  }
  f32x16 acc[kQPW][2];
#pragma unroll
  for (int a = 0; a < kQPW; ++a)
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[a][db][r] = 0.f;
  // Lazy reference maximum per query (exp2 domain), the same in lanes l and l ^ 32; a finite
  // start keeps t - m = -inf at unselected entries. Row sums: this lane's keys only.
  float m[kQPW], l[kQPW];
#pragma unroll
  for (int a = 0; a < kQPW; ++a) {
    m[a] = -3.4028234663852886e38f;
    l[a] = 0.f;
  }

  // Tile staging: each thread moves two 16-byte chunks of K and two of V^T per 64-key half of
  // a tile (rows srow and srow + 32), loaded straight into LDS. Lane i of a wave writes the 16 bytes at the
  // wave's 1 KB segment + 16 i = row srow, physical chunk sc, so it reads the chunk
  // sc ^ swz(srow) that the swizzled layout keeps there (swz(srow + 32) = swz(srow)).
  const int srow = tid >> 3, sc = tid & 7;
  const int lc = sc ^ swz(srow);
  const int wseg = wave * 1024;
  // A tile's base addresses are uniform (scalar registers); a lane adds a 32-bit byte offset
  // (the host keeps a K row stride below 2^24 bytes and 64 rows of V^T below 2^32 bytes).
  const char* kbase = uniform_ptr(reinterpret_cast<const char*>(p.k + b * p.ksb + (int64_t)h * p.ksh));
  const char* vbase = uniform_ptr(reinterpret_cast<const char*>(p.vt + ((int64_t)b * p.H + h) * 64 * p.Spad));
  const uint32_t kss_b = (uint32_t)p.kss * 2u;
  const uint32_t kcol = (uint32_t)lc * 16u;
  const uint32_t vo0 = ((uint32_t)srow * (uint32_t)p.Spad + (uint32_t)lc * 8u) * 2u;
  const uint32_t vo1 = vo0 + (uint32_t)p.Spad * 64u;  // row srow + 32
  auto dload = [&](int k0, uint8_t* kdst, uint8_t* vdst) {
    // Rows past the end read row S - 1 (their keys are never selected), taken from a base row
    // at most S - 1 so that the lane offsets stay in [0, 63] rows wherever the tile starts.
    const TileRows tr = tile_rows(k0, srow, p.S);
    const char* kt = kbase + (int64_t)tr.base * kss_b;
    buffer_load16_lds(kt, __umul24(tr.r0, kss_b) + kcol, kdst + wseg);
    buffer_load16_lds(kt, __umul24(tr.r1, kss_b) + kcol, kdst + wseg + 4096);
    const char* vsrc = vbase + (int64_t)k0 * 2;
    buffer_load16_lds(vsrc, vo0, vdst + wseg);
    buffer_load16_lds(vsrc, vo1, vdst + wseg + 4096);
  };
  // Operand reads: K rows 32 st + col (chunk 2 ks + half), V^T rows 32 db + col (chunk
  // 4 st + 2 ks + half); swz of these rows is swz(col).
  const int fc = swz(col);
  auto koff = [&](int st, int ks) { return col * 128 + st * 4096 + (((2 * ks + half) ^ fc) << 4); };
  auto voff = [&](int db, int st, int ks) { return col * 128 + db * 4096 + (((4 * st + 2 * ks + half) ^ fc) << 4); };
  // Mask words of the lane's queries, one per 32-key sub-tile.
  const int nsub = p.Spad >> 5;
  const char* mblk = uniform_ptr(reinterpret_cast<const char*>(p.mask + (int64_t)b * nsub * p.tpad + qb0 * 32));
  const int64_t mrow_b = (int64_t)p.tpad * 4;  // bytes per sub-tile row of mask words
  auto mword = [&](int j, int a) {
    return buffer_load4(mblk + min(j, nsub - 1) * mrow_b, (uint32_t)(col + 32 * a) * 4u);
  };

  // attn_sum: lane (col, half) stores the scores of query tq[half] (block half), whose selected
  // keys before the current sub-tile number rank_base; slots [0, fl) of its row are written.
  uint32_t rank_base = 0u, fl = 0u;
  float* const srow_ws =
      ATTN ? p.sws + (((int64_t)b * p.H + h) * p.T + min(tq[half], p.T - 1)) * sws_row(p.K) : nullptr;
  // LDS byte addresses (see ascore): this lane's chunk of group 0 of block 0 in the staging
  // (group g at + 32 g, block 1 at + 32 rows), and its query's staging and ring.
  uint32_t st_w = 0u, st_r = 0u, st_f = 0u;
  if constexpr (ATTN) {
    const uint32_t rows = lds_addr(ascore + wave * (32 * kQPW * kArow));
    st_w = rows + (uint32_t)col * (kArow * 4) + 32u + 16u * (uint32_t)half;
    st_f = rows + (uint32_t)(32 * half + col) * (kArow * 4);
    st_r = st_f + 32u;
  }
  // Writes slots [fl, fl + 4) of the row (read from the ring by the caller) when `flush`,
  // then advances fl; lanes that do not flush are masked off inside the asm block (no branch).
  typedef float f32x4r __attribute__((ext_vector_type(4)));
  auto ring_store = [&](bool flush, const f32x4r& f) {
    float* dst = srow_ws + fl;
    uint64_t sv;
    asm volatile(
        "s_mov_b64 %0, exec\n\tv_cmp_ne_u32 vcc, 0, %3\n\ts_and_b64 exec, exec, vcc\n\t"
        "global_store_dwordx4 %1, %2, off\n\ts_mov_b64 exec, %0"
        : "=&s"(sv)
        : "v"(dst), "v"(f), "v"((uint32_t)flush)
        : "vcc", "memory");
    fl += flush ? 4u : 0u;
  };

  // One 32-key sub-tile in two parts. sub_qk: S^T for both blocks from the selection bias;
  // sub_pv: the softmax in registers and O^T += V^T P^T.
  auto sub_qk = [&](const uint8_t* kt, int st, const uint32_t (&w)[kQPW], f32x16 (&s)[kQPW])
                    __attribute__((always_inline)) {
    // The sub-tile's four K operands first: their LDS latency passes under the bias.
    uint4 ka[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) ka[ks] = *reinterpret_cast<const uint4*>(kt + koff(st, ks));
#pragma unroll
    for (int a = 0; a < kQPW; ++a) {
      if constexpr (ATTN) {
        // Natural-order words (bit i: key i selected): entry 4 g + j of this lane, key 8 g + 4
        // half + j, is the sign bit of byte g of ~w << (7 - 4 half - j), set when the key is not
        // selected; a sign-extended byte select masks -inf (one instruction per entry).
        const uint32_t nw = ~w[a];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t sh = nw << (7 - 4 * half - j);
#pragma unroll
          for (int g = 0; g < 4; ++g)
            s[a][4 * g + j] = __uint_as_float((uint32_t)(int32_t)(int8_t)(sh >> (8 * g)) & 0xFF800000u);
        }
      } else {
        // Bias-order words: entry 4 g + j of this lane is the sign bit of byte j of w << (g + 4
        // half), set when the key is not selected; a sign-extended byte select masks -inf
        // (one instruction per entry).
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const uint32_t sh = w[a] << (g + 4 * half);
#pragma unroll
          for (int j = 0; j < 4; ++j)
            s[a][4 * g + j] = __uint_as_float((uint32_t)(int32_t)(int8_t)(sh >> (8 * j)) & 0xFF800000u);
        }
      }
    }
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int a = 0; a < kQPW; ++a) s[a] = mma(E{}, ka[ks], qa[a][ks], s[a]);
  };
  auto sub_pv = [&](const uint8_t* vt, int st, const uint32_t (&w)[kQPW], f32x16 (&s)[kQPW])
                    __attribute__((always_inline)) {
    // attn_sum round state (see below): the selected-key word of this lane's query, its count,
    // and the entries and ring slots read by issue() for finish().
    uint32_t selw = 0u, cnt = 0u;
    bool flush0 = false;
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    float rv0 = 0.f, rv1 = 0.f, rv2 = 0.f, rv3 = 0.f;
    f32x4 rf = {0.f, 0.f, 0.f, 0.f};
    // One round of the attn_sum stores, in two parts. issue(): the ring's oldest 4 slots (rf)
    // and the next four selected entries (rv) read without waiting (selw = 0: v_ffbl gives -1,
    // the float before the staging, inside the row; not used). finish(): the wait, the flush
    // when `flush`, then the entries into the ring at slots rank_base + done + i (mod 8) when
    // `append`. Between the two the sub-tile's weights and products run, and no instruction
    // touches rv or rf.
    auto issue = [&]() {
      uint32_t ad[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        uint32_t e;
        asm("v_ffbl_b32 %0, %1" : "=v"(e) : "v"(selw));
        ad[i] = st_r + (e << 2);
        selw &= selw - 1u;
      }
      const uint32_t fa = st_f + ((fl << 2) & 16u);
      asm volatile(
          "ds_read_b32 %0, %5\n\tds_read_b32 %1, %6\n\tds_read_b32 %2, %7\n\tds_read_b32 %3, %8\n\t"
          "ds_read_b128 %4, %9"
          : "=&v"(rv0), "=&v"(rv1), "=&v"(rv2), "=&v"(rv3), "=&v"(rf)
          : "v"(ad[0]), "v"(ad[1]), "v"(ad[2]), "v"(ad[3]), "v"(fa)
          : "memory");
    };
    // The staging of block a's scores (see the attn_sum stores below), by the lanes that hold
    // a selected key of the sub-tile (only selected entries are read back): the other lanes are
    // masked off inside the asm block, so the code around it stays one basic block.
    auto stage = [&](const f32x16& sa, int a) {
      static_assert(kQPW == 2 && kArow * 32 * 4 == 5632, "block 1 rows at +5632 bytes");
      const uint32_t bits = w[a] & (0x0F0F0F0Fu << (4 * half));
      uint64_t sv;
      if (a == 0)
        asm volatile(
            "s_mov_b64 %0, exec\n\tv_cmp_ne_u32 vcc, 0, %6\n\ts_and_b64 exec, exec, vcc\n\t"
            "ds_write_b128 %1, %2\n\tds_write_b128 %1, %3 offset:32\n\t"
            "ds_write_b128 %1, %4 offset:64\n\tds_write_b128 %1, %5 offset:96\n\ts_mov_b64 exec, %0"
            : "=&s"(sv)
            : "v"(st_w), "v"(__builtin_shufflevector(sa, sa, 0, 1, 2, 3)),
              "v"(__builtin_shufflevector(sa, sa, 4, 5, 6, 7)), "v"(__builtin_shufflevector(sa, sa, 8, 9, 10, 11)),
              "v"(__builtin_shufflevector(sa, sa, 12, 13, 14, 15)), "v"(bits)
            : "vcc", "memory");
      else
        asm volatile(
            "s_mov_b64 %0, exec\n\tv_cmp_ne_u32 vcc, 0, %6\n\ts_and_b64 exec, exec, vcc\n\t"
            "ds_write_b128 %1, %2 offset:5632\n\tds_write_b128 %1, %3 offset:5664\n\t"
            "ds_write_b128 %1, %4 offset:5696\n\tds_write_b128 %1, %5 offset:5728\n\ts_mov_b64 exec, %0"
            : "=&s"(sv)
            : "v"(st_w), "v"(__builtin_shufflevector(sa, sa, 0, 1, 2, 3)),
              "v"(__builtin_shufflevector(sa, sa, 4, 5, 6, 7)), "v"(__builtin_shufflevector(sa, sa, 8, 9, 10, 11)),
              "v"(__builtin_shufflevector(sa, sa, 12, 13, 14, 15)), "v"(bits)
            : "vcc", "memory");
    };
    auto finish = [&](uint32_t done, bool flush, bool append) {
      asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(rv0), "+v"(rv1), "+v"(rv2), "+v"(rv3), "+v"(rf) : : "memory");
      ring_store(flush, rf);
      if (append) {
        const uint32_t r4 = (rank_base + done) << 2;
        asm volatile(
            "ds_write_b32 %0, %4\n\tds_write_b32 %1, %5\n\tds_write_b32 %2, %6\n\tds_write_b32 %3, %7"
            :
            : "v"(st_f + (r4 & 28u)), "v"(st_f + ((r4 + 4u) & 28u)), "v"(st_f + ((r4 + 8u) & 28u)),
              "v"(st_f + ((r4 + 12u) & 28u)), "v"(rv0), "v"(rv1), "v"(rv2), "v"(rv3)
            : "memory");
      }
    };
    // Per block: the weights, then its P·V products, so that the second block's exp2 (which
    // co-executes with matrix products on this GPU, unlike fp32 VALU) overlaps the first
    // block's products. The V^T operands are read once for both blocks.
    uint4 va[2][2];
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) va[db][ks] = *reinterpret_cast<const uint4*>(vt + voff(db, st, ks));
#pragma unroll
    for (int a = 0; a < kQPW; ++a) {
      if constexpr (ATTN) {
        // attn_sum: each selected entry's score (unscaled: dense_attn_sum_kernel applies the
        // scale) goes to the slot of its key's rank. The sub-tile's selected keys of a query take
        // consecutive slots from rank_base on, so no lane works per entry: the two lanes of each
        // query put its 32 scores in key order into the query's LDS row (block a's, as soon as
        // its products are done), then lane (col, half) reads the scores of query tq[half] at its
        // four lowest selected keys (issue(), here, while block 1's weights and products run)
        // and appends them to the query's ring (finish(), at the end); whenever 4 slots of the
        // row are complete they go to memory in one 16-byte store. The staging array is written
        // and read by inline asm only: for any access the compiler sees it would first wait for
        // the next tile's direct-to-LDS loads. A wave's LDS operations complete in issue order,
        // so the partner lane's half of a row written here is in place for the reads.
        stage(s[a], a);
        if (a == kQPW - 1) {
          selw = half ? w[1] : w[0];
          cnt = __popc(selw);
          flush0 = rank_base - fl >= 4u;
          issue();
        }
      }
      // Weights with the current reference maximum. Their sum bounds each weight: while no
      // lane's sum exceeds kSumCap every p fits fp16, and the maximum stays where it is.
      float pv[16];
      float ls = 0.f;
      uint4 pb[2];
      // The P operand in fp16 and the row sum of the fp32 weights (the sum of the fp16 operand
      // instead, by v_dot2_f32_f16 against ones, is half the instructions but moves o by up to
      // 4e-2 through the whole aggregator).
      auto weights = [&](float nm) {
#pragma unroll
        for (int r = 0; r < 16; ++r) pv[r] = fexp2(fmaf(s[a][r], sl2, nm));
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
          pb[ks] = make_uint4(pack_f16(pv[8 * ks], pv[8 * ks + 1]), pack_f16(pv[8 * ks + 2], pv[8 * ks + 3]),
                              pack_f16(pv[8 * ks + 4], pv[8 * ks + 5]), pack_f16(pv[8 * ks + 6], pv[8 * ks + 7]));
        // Two independent accumulation chains (a wave has few others to hide their latency).
        float t[2] = {pv[0], pv[8]};
#pragma unroll
        for (int r = 1; r < 8; ++r) {
          t[0] += pv[r];
          t[1] += pv[8 + r];
        }
        return t[0] + t[1];
      };
      ls = weights(-m[a]);
      if (__builtin_amdgcn_ballot_w64(!(ls <= kSumCap)) != 0ull) {
        // Some query of the block has an entry above its maximum by more than log2(kSumCap /
        // 16) (or its first selected entry): every query of the block moves its maximum to
        // its largest selected entry of this sub-tile if that is higher, rescales O and the
        // row sum, and the weights are formed again.
        float mx = s[a][0];
#pragma unroll
        for (int r = 1; r < 16; ++r) mx = fmaxf(mx, s[a][r]);
        const float mn = fmaxf(m[a], pair_max(mx) * sl2);
        const float alpha = fexp2(m[a] - mn);
        m[a] = mn;
        l[a] *= alpha;
#pragma unroll
        for (int db = 0; db < 2; ++db)
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[a][db][r] *= alpha;
        ls = weights(-mn);
      }
      l[a] += ls;
#pragma unroll
      for (int db = 0; db < 2; ++db)
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) acc[a][db] = mma(FP16{}, va[db][ks], pb[ks], acc[a][db]);
    }
    if constexpr (ATTN) {
      // The ring holds slots [fl, rank_base) (at most 7) and receives at most four more per
      // round: a block of 4 completed earlier is written out first. Rarely a query selects
      // more than four keys of a sub-tile: further rounds, each read and finished at once.
      finish(0u, flush0, true);
      for (uint32_t done = 4; __builtin_amdgcn_ballot_w64(cnt > done) != 0ull; done += 4) {
        const bool more = cnt > done;
        const bool fl_more = more && rank_base + done - fl >= 4u;
        issue();
        finish(done, fl_more, more);
      }
      rank_base += cnt;
      asm volatile("" ::: "memory");
    }
  };

  // Tile n (kHT halves of 64 keys, kSPT sub-tiles) lives in LDS buffer n % 2. While computing
  // tile n the workgroup loads tile n + 1 into the other buffer (last read before the previous
  // barrier); one barrier per tile. The mask words of tile n + 2 are loaded after tile n's
  // products, into the registers tile n used: they have a whole tile to arrive and are not
  // waited for at the barrier.
  constexpr int kSPT = 2 * kHT;
  const int ntiles = p.Spad / (64 * kHT);  // Spad is a whole number of 128-key tiles
  auto tload = [&](int n, uint8_t* kd, uint8_t* vd) __attribute__((always_inline)) {
#pragma unroll
    for (int hf = 0; hf < kHT; ++hf) dload((n * kHT + hf) * 64, kd + hf * 8192, vd + hf * 8192);
  };
  auto words = [&](int n, uint32_t (&wd)[kSPT][kQPW]) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < kSPT; ++j)
#pragma unroll
      for (int a = 0; a < kQPW; ++a) wd[j][a] = mword(kSPT * n + j, a);
  };
  uint32_t wA[kSPT][kQPW], wB[kSPT][kQPW];  // words of the even and the odd tiles
  tload(0, ktile0, vtile0);
  words(0, wA);
  words(1, wB);
  __builtin_amdgcn_s_waitcnt(0x0070);  // vmcnt(0) lgkmcnt(0): tile 0 is in LDS
  __syncthreads();
  auto tile = [&](int n, const uint8_t* kc, const uint8_t* vc, uint8_t* kn, uint8_t* vn,
                  uint32_t (&wd)[kSPT][kQPW]) __attribute__((always_inline)) {
    // Past the end the last tile again, into the buffer no tile reads any more: no branch
    // around the loads, so the compiler's count of those in flight stays exact.
    tload(min(n + 1, ntiles - 1), kn, vn);
    // The products run one sub-tile ahead of the softmax: sub-tile j's are issued before
    // sub-tile j - 1's weights, so they run on the matrix cores while those are formed.
    // (attn_sum takes the sub-tiles' scores in key order: sub_pv in order.)
    f32x16 ss[2][kQPW];
    sub_qk(kc, 0, wd[0], ss[0]);
#pragma unroll
    for (int j = 1; j < kSPT; ++j) {
      sub_qk(kc + (j >> 1) * 8192, j & 1, wd[j], ss[j & 1]);
      sub_pv(vc + ((j - 1) >> 1) * 8192, (j - 1) & 1, wd[j - 1], ss[(j - 1) & 1]);
    }
    sub_pv(vc + ((kSPT - 1) >> 1) * 8192, (kSPT - 1) & 1, wd[kSPT - 1], ss[(kSPT - 1) & 1]);
    words(n + 2, wd);
    // vmcnt(kSPT kQPW): all but the word loads just issued have landed, so this thread's
    // loads of the next tile are in LDS; after the barrier every thread's are, and every wave
    // is done with this tile's buffer before it is refilled.
    static_assert(kSPT * kQPW <= 15, "vmcnt immediate");
    __builtin_amdgcn_s_waitcnt(0x0070 | (kSPT * kQPW));  // vmcnt(kSPT kQPW) lgkmcnt(0)
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };
  // Pairs of tiles, then a last odd one: the loop returns to its top only after both tiles
  // of a pair, so the words it starts with are always two barriers old.
  int n = 0;
#pragma unroll 1
  for (; n + 1 < ntiles; n += 2) {
    tile(n, ktile0, vtile0, ktile1, vtile1, wA);
    tile(n + 1, ktile1, vtile1, ktile0, vtile0, wB);
  }
  if (n < ntiles) tile(n, ktile0, vtile0, ktile1, vtile1, wA);
  __builtin_amdgcn_s_waitcnt(0x0070);  // the loads issued past the end

  if constexpr (ATTN) {
    // The ring's last slots (at most 7: two blocks of 4, the second partly past the row's
    // count, inside its padding).
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const uint32_t fa = st_f + ((fl << 2) & 16u);
      float4 f;
      asm volatile("ds_read_b128 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=&v"(f) : "v"(fa) : "memory");
      ring_store(fl < rank_base, (f32x4r){f.x, f.y, f.z, f.w});
    }
  }
  // o = O / l scaled back by 2^-e per column, lse = (m + log2 l) ln 2; queries without any
  // selected key give o = 0, lse = -inf. Blocks holding a repeated position, and batch
  // elements with a non-finite K or V value, are written by the gather kernel.
  const bool finite = p.bad[b] == 0;

#pragma unroll
  for (int a = 0; a < kQPW; ++a) {
    const int qb = qb0 + a, t = tq[a];
    bool active = finite && qb < p.nqb && t < p.T;
    if (qb < p.nqb) {
      const int* f = p.flags + ((int64_t)b * p.nqb + qb) * p.nchunk;
      for (int c = 0; c < p.nchunk; ++c) active &= f[c] == 0;
    }
    const float lt = pair_sum(l[a]);
    if (active) {
      const float inv = lt > 0.f ? __frcp_rn(lt) : 0.f;
      uint16_t* orow = p.o + b * p.osb + (int64_t)t * p.ost + h * p.osh;
#pragma unroll
      for (int db = 0; db < 2; ++db)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int d0 = 32 * db + 8 * g + 4 * half;
          uint16_t hv[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) hv[i] = to_half_bits(E{}, acc[a][db][4 * g + i] * inv * vsc_s[d0 + i]);
          *reinterpret_cast<uint2*>(orow + d0) =
              make_uint2((uint32_t)hv[0] | ((uint32_t)hv[1] << 16), (uint32_t)hv[2] | ((uint32_t)hv[3] << 16));
        }
      if (half == 0 && p.lse)
        p.lse[((int64_t)b * p.T + t) * p.H + h] = lt > 0.f ? (m[a] + flog2(lt)) * kDLn2 : -INFINITY;
    }
  }
}

// ---------------------------------------------------------------------------------------
// attn_sum from the slot-indexed scores: one wave per query row. The row's valid positions,
// sorted ascending, are in slot order: slot i holds the i-th smallest selected key. So
// attn_sum[t, j] = sum_h exp2(sws[h][t][i(j)] * scale log2(e) - lse2[t, h]) with i(j) the rank of position j
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
  const int* bad;    // [B]
  float* attn_sum;   // [B, T, K]
  const void* logits;
  int logits_dt;
  int64_t lsb, lst;
  float kl_eps;
  float* row_loss;
  int B, T, S, H, K, nqb, nchunk;
  float scale_log2;  // sws holds unscaled scores
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
  __shared__ __align__(16) float slot_sum[4][R * 64 + 4];  // per wave: the row's per-slot head sums
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t row = (int64_t)blockIdx.x * 4 + wave;
  if (row >= (int64_t)p.B * p.T) return;  // whole wave; no barriers below
  const int b = (int)(row / p.T), t = (int)(row - (int64_t)b * p.T);
  {
    const int* f = p.flags + ((int64_t)b * p.nqb + (t >> 5)) * p.nchunk;
    bool flagged = p.bad[b] != 0;
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
  // Per-slot sums over the heads, in slot order: head h's scores of this row are the K floats
  // at srow + h * hstride (head-major workspace), four slots per lane and load, the loads of 16
  // heads in flight at once; the sums go through the wave's LDS row to the lanes that hold each
  // slot's position after the sort below (the sums do not depend on it).
  lds_fence();
  const float* srow = p.sws + ((int64_t)b * p.H * p.T + t) * sws_row(p.K);
  const int64_t hstride = (int64_t)p.T * sws_row(p.K);
  int nvalid = 0;  // valid positions sort first: slots [0, nvalid) are in use
#pragma unroll
  for (int r = 0; r < R; ++r) nvalid += __popcll(__builtin_amdgcn_ballot_w64((key[r] >> 32) != 0xFFFFFFFFull));
  float* ssum = &slot_sum[wave][0];
  for (int i0 = 4 * lane; i0 < nvalid; i0 += 256) {
    float a4[4] = {0.f, 0.f, 0.f, 0.f};
    for (int h0 = 0; h0 < p.H; h0 += 16) {
      // 16-byte loads: head rows are 32-byte aligned and padded past any slot in use by at
      // least 3 (slots at or past nvalid are never used); heads past H re-read head H - 1.
      float4 f[16];
#pragma unroll
      for (int u = 0; u < 16; ++u)
        f[u] = *reinterpret_cast<const float4*>(srow + min(h0 + u, p.H - 1) * hstride + i0);
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        if (h0 + u >= p.H) break;
        const float l2 = lse2_s[wave][h0 + u];
        if (l2 == -INFINITY) continue;  // a row without valid keys (the same for every head)
        a4[0] += fexp2(fmaf(f[u].x, p.scale_log2, -l2));
        a4[1] += fexp2(fmaf(f[u].y, p.scale_log2, -l2));
        a4[2] += fexp2(fmaf(f[u].z, p.scale_log2, -l2));
        a4[3] += fexp2(fmaf(f[u].w, p.scale_log2, -l2));
      }
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) ssum[i0 + u] = a4[u];
  }
  wave_bitonic_sort<R>(key);
  lds_fence();
  float av[R], zv[R];
  float sa = 0.f, mz = -INFINITY;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int i = r * 64 + lane;  // slot = sorted rank
    const int j = (int)(uint32_t)key[r];
    const bool ok = (key[r] >> 32) != 0xFFFFFFFFull;
    const float sum = ok ? ssum[i] : 0.f;
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
  size_t mask, flags, bad, vmax, vt, sws, total;
  int nqb, nqb_pad, nchunk, spad;
  bool rows_pass;  // selection words built by dense_mask_rows_kernel
};

DenseLayout dense_layout(int64_t B, int64_t T, int64_t S, int64_t H, int64_t K, bool attn) {
  DenseLayout L;
  L.nqb = (int)((T + 31) / 32);
  L.nqb_pad = (L.nqb + kQBW - 1) / kQBW * kQBW;
  L.spad = (int)((S + 127) / 128 * 128);  // whole 128-key tiles of the plain forward
  // One pass over the positions (two 16-query halves per block) when the sub-tile words of
  // 16 queries fit the LDS, else equal chunks of at most kMaskChunkMax keys.
  L.rows_pass = L.spad / 32 <= kMaskRowsMaxSub;
  L.nchunk = L.rows_pass ? 2 : mask_nchunk(L.spad);
  if (L.nchunk < 1) L.nchunk = 1;
  auto up = [](size_t x) { return (x + 255) / 256 * 256; };
  size_t o = 0;
  L.mask = o;
  o = up(o + (size_t)B * (size_t)(L.spad / 32) * (size_t)L.nqb_pad * 32 * 4);
  L.flags = o;
  o = up(o + (size_t)B * L.nqb * (size_t)L.nchunk * 4);
  L.bad = o;
  o = up(o + (size_t)B * 4);
  L.vmax = o;
  o = up(o + (size_t)B * (size_t)H * 64 * 4);
  L.vt = o;
  o = up(o + (size_t)B * (size_t)H * 64 * (size_t)L.spad * 2);
  L.sws = o;
  if (attn) o = up(o + (size_t)B * (size_t)T * (size_t)sws_row(K) * (size_t)H * 4);
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
  if (!(softmax_scale > 0.f) || !(softmax_scale < 3.4e38f))
    return set_error(GW_ERR_UNSUPPORTED, "the dense forward needs a positive finite softmax scale, got %g",
                     (double)softmax_scale);
  const bool want_attn = attn_sum != nullptr;
  const bool want_kl = logits != nullptr;
  if (want_attn && H > 64)
    return set_error(GW_ERR_UNSUPPORTED, "the dense forward computes attn_sum for H <= 64, got %lld", (long long)H);
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
  // Query blocks: at most 65535 (T <= 65528 * 32 once padded to whole workgroups).
  if ((int64_t)(L.nqb_pad / kQBW) * H >= (1ll << 31) || L.nqb_pad > 65535)
    return set_error(GW_ERR_UNSUPPORTED, "the dense forward takes at most %d queries, got %lld", 65528 * 32,
                     (long long)T);
  if (k_strides[1] >= kDenseMaxKRowStride || (int64_t)L.spad * 128 >= (1ll << 32))
    return set_error(GW_ERR_UNSUPPORTED,
                     "the dense forward needs a K token stride below %lld elements and S <= %lld, got %lld and %lld",
                     (long long)kDenseMaxKRowStride, (long long)kDenseMaxS, (long long)k_strides[1], (long long)S);
  GW_CHECK_ARG(workspace != nullptr && workspace_bytes >= L.total && aligned16(workspace),
               "the dense forward needs a 16-byte aligned %zu-byte workspace, got %zu", L.total, workspace_bytes);
  hipStream_t st = static_cast<hipStream_t>(stream);
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  uint32_t* mask = reinterpret_cast<uint32_t*>(ws + L.mask);
  int* flags = reinterpret_cast<int*>(ws + L.flags);
  int* bad = reinterpret_cast<int*>(ws + L.bad);
  uint32_t* vmax = reinterpret_cast<uint32_t*>(ws + L.vmax);
  uint16_t* vt = reinterpret_cast<uint16_t*>(ws + L.vt);
  const int in_fp16 = dtype == GW_DTYPE_FP16 ? 1 : 0;
  float* sws = want_attn ? reinterpret_cast<float*>(ws + L.sws) : nullptr;

  {
    const int vec = (K % 4 == 0 && pos_stride_t % 4 == 0 && pos_stride_b % 4 == 0 &&
                     (reinterpret_cast<uintptr_t>(kv_pos) & 15) == 0)
                        ? 1
                        : 0;
    if (L.rows_pass) {
      const size_t lds = (size_t)(L.spad / 32) * (kMaskRowsQ + 1) * 4;
      hipLaunchKernelGGL(dense_mask_rows_kernel, dim3((unsigned)(L.nqb_pad * 2), (unsigned)B), dim3(kMaskRowsThreads),
                         lds, st, kv_pos, pos_stride_b, pos_stride_t, (int)T, (int)S, L.spad, (int)K, L.nqb,
                         L.nqb_pad * 32, vec, (int)(H * 64), mask, flags, vmax, bad, want_attn ? 0 : 1);
      GW_HIP_LAUNCH_CHECK("dense_mask_rows_kernel launch");
    } else {
      hipLaunchKernelGGL(dense_mask_kernel, dim3(L.nchunk, L.nqb_pad, (unsigned)B), dim3(256), 0, st, kv_pos,
                         pos_stride_b, pos_stride_t, (int)T, (int)S, L.spad, (int)K, L.nqb, L.nqb_pad * 32, L.nchunk,
                         vec, (int)(H * 64), mask, flags, vmax, bad, nullptr, nullptr, want_attn ? 0 : 1,
                         mask_chunk_keys(L.spad, L.nchunk));
      GW_HIP_LAUNCH_CHECK("dense_mask_kernel launch");
    }
  }
  hipLaunchKernelGGL(dense_vmax_kernel, dim3((unsigned)((S + kVmaxKeys - 1) / kVmaxKeys), (unsigned)H, (unsigned)B),
                     dim3(256), 0, st, static_cast<const uint16_t*>(v), v_strides[0], v_strides[1], v_strides[2],
                     static_cast<const uint16_t*>(k), k_strides[0], k_strides[1], k_strides[2], (int)S, (int)H,
                     in_fp16, vmax, bad);
  GW_HIP_LAUNCH_CHECK("dense_vmax_kernel launch");
  hipLaunchKernelGGL(dense_vt_kernel, dim3(L.spad / 64, (unsigned)H, (unsigned)B), dim3(256), 0, st,
                     static_cast<const uint16_t*>(v), v_strides[0], v_strides[1], v_strides[2], (int)S, L.spad,
                     (int)H, in_fp16, vmax, vt);
  GW_HIP_LAUNCH_CHECK("dense_vt_kernel launch");

  DenseParams p;
  p.q = static_cast<const uint16_t*>(q);
  p.k = static_cast<const uint16_t*>(k);
  p.vt = vt;
  p.mask = mask;
  p.vmax = vmax;
  p.flags = flags;
  p.bad = bad;
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
  p.tpad = L.nqb_pad * 32;
  p.nchunk = L.nchunk;
  p.scale_log2 = softmax_scale * kDLog2e;
  p.sws = sws;
  p.K = (int)K;
  const dim3 grid((unsigned)(L.nqb_pad / kQBW * H), (unsigned)B);
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
    ap.bad = bad;
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
    ap.scale_log2 = p.scale_log2;
    const int rows = (int)(B * T);
    const int rc = want_kl ? launch_attn_sum<true>(ap, rows, st) : launch_attn_sum<false>(ap, rows, st);
    if (rc != GW_OK) return rc;
  }
  // Blocks with a repeated position, and every block of a batch element with a non-finite
  // K or V value: the gather kernel (it returns at once for the others), with attn_sum and
  // the KL loss when asked (its score workspace is the same region).
  return attn_fwd_flagged_blocks(dtype, q, q_strides, k, k_strides, v, v_strides, kv_pos, pos_stride_b, pos_stride_t,
                                 o, o_strides, lse, attn_sum, B, T, S, H, D, K, softmax_scale, logits, logits_dtype,
                                 logits_stride_b, logits_stride_t, eps, row_loss, sws,
                                 want_attn ? (size_t)B * T * K * H * 4 : 0, flags, bad, L.nqb, L.nchunk, stream);
}
