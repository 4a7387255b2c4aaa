// Sparse-index attention backward as masked dense passes on the matrix cores (gfx950, D = 64).
//
// Math (reference _bwd_preprocess_do_o_dot + _bwd_sparse_index_kernel,
// easyvolcap/utils/custom_flash_attn/sparse_index_flash_attn.py:534-576, :579-743), per
// (b, h), query t and selected key s:
//   p     = exp(scale q_t.k_s - lse_t)            (recomputed from the forward's lse)
//   dp    = dO_t . v_s
//   delta = sum_d o_t dO_t                        (from the saved o)
//   ds    = p (dp - delta)
//   dq_t  = scale sum_s ds k_s,   dk_s = scale sum_t ds q_t,   dv_s = sum_t p dO_t
// The reference gathers the selected K/V rows per query and scatters dk/dv with fp32 atomics.
// When a query selects a few per cent of all keys, computing every (query, key) pair on the
// matrix cores costs less, as in the dense forward: the selection enters as the initial
// accumulator of the score product (0 where the query selected the key, -inf elsewhere), so p
// and ds are exactly zero at every other pair. Two passes, neither with atomics, so every
// gradient is a fixed-order sum and the backward is bitwise reproducible:
//   dense_bwd_dq_kernel    query-major, the forward's transposed products: per 32-key
//                          sub-tile S^T = K Q^T, dP^T = V dO^T (a lane holds one query and
//                          16 keys: lse and delta are one register each), dS^T in registers
//                          is already the B operand of dQ^T += K^T dS^T.
//   dense_bwd_dkdv_kernel  key-major: per 32-query sub-tile S = Q K^T, dP = dO V^T (a lane
//                          holds one key and 16 queries), P and dS are the B operands of
//                          dV^T += dO^T P and dK^T += Q^T dS; dK and dV stay in registers
//                          over all queries.
// P and dS enter their products in the input type (bf16 or fp16; for fp16, dS is scaled by a
// power of two per (b, h) that keeps it clear of fp16 underflow and overflow); every product
// accumulates in fp32.
//
// This covers the backward without an attn_sum gradient (the reference presets detach the
// attention mass before the indexer loss: detach_input, dsa_attention.py:4694-4695), with
// finite inputs and no position listed twice in a row. A batch element that breaks the last
// two (a repeated position counts twice in the reference; a non-finite value in a row a query
// did not select would reach the dense products) is flagged in route[b] and left untouched;
// the caller computes it with the CSR backward (gw_sparse_attn_bwd).
#include <math.h>

#include "gw_common.h"
#include "gw_dense.h"

namespace gw {
namespace {

// ---------------------------------------------------------------------------------------
// Clears the route flags and the |dO|, |V| maxima before the other kernels set them.
// ---------------------------------------------------------------------------------------
constexpr int64_t kDenseBwdMaxRowStride = 1ll << 23;

__global__ __launch_bounds__(256) void dense_bwd_clear_kernel(int* __restrict__ route, int B,
                                                              uint32_t* __restrict__ amax, int n_amax) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < B) route[i] = 0;
  if (i < n_amax) amax[i] = 0u;
}

// ---------------------------------------------------------------------------------------
// Per (b, h, t): {lse * log2(e), delta = sum_d o dO} as ls[(b * H + h) * tpad + t] ({+inf, 0}
// past T; +inf too for a row without any selected key, lse = -inf, so that every weight of
// the row is exp2(-inf) = 0). Eight lanes per (t, h), 16-byte loads of o and dO. A nan lse
// or a non-finite delta routes the batch element to the CSR backward.
// ---------------------------------------------------------------------------------------
template <typename E>
__global__ __launch_bounds__(256) void dense_bwd_rowstats_kernel(const uint16_t* __restrict__ o, int64_t osb,
                                                                 int64_t ost, int64_t osh,
                                                                 const uint16_t* __restrict__ dout, int64_t dsb,
                                                                 int64_t dst, int64_t dsh, const float* __restrict__ lse,
                                                                 int T, int H, int tpad, float2* __restrict__ ls,
                                                                 int* __restrict__ route) {
  const int b = blockIdx.y;
  const int64_t g = (int64_t)blockIdx.x * 32 + (threadIdx.x >> 3);  // (t, h), h fastest
  const int c = threadIdx.x & 7;
  if (g >= (int64_t)tpad * H) return;  // whole groups of 8 lanes
  const int t = (int)(g / H), h = (int)(g - (int64_t)t * H);
  float acc = 0.f;
  float l2 = INFINITY;
  if (t < T) {
    const uint4 ov = *reinterpret_cast<const uint4*>(o + b * osb + (int64_t)t * ost + h * osh + c * 8);
    const uint4 dv = *reinterpret_cast<const uint4*>(dout + b * dsb + (int64_t)t * dst + h * dsh + c * 8);
    float of[8], df[8];
    unpack8<E>(ov, of);
    unpack8<E>(dv, df);
#pragma unroll
    for (int i = 0; i < 8; ++i) acc = fmaf(of[i], df[i], acc);
    const float lv = lse[((int64_t)b * T + t) * H + h];
    l2 = lv == -INFINITY ? INFINITY : lv * kDLog2e;
    if (c == 0 && (isnan(lv) || lv == INFINITY)) route[b] = 1;
  }
  acc = group_sum<8>(acc);
  if (c == 0) {
    if (!isfinite(acc)) route[b] = 1;  // every writer stores the same value
    ls[((int64_t)b * H + h) * tpad + t] = make_float2(l2, acc);
  }
}

// ---------------------------------------------------------------------------------------
// X [B][R][H][64] (strided) -> xt[b][h][d][r'] (r' < Rpad, zero past R) in the same 16-bit
// type, the rows permuted within every 16 by exchanging bits 2 and 3 of the row index: that is
// the order in which a lane's accumulator entries enter a product as its B operand (entries
// r < 8 of lane l are rows 8 (r / 4) + 4 (l / 32) + r % 4, which the operand's k-chunk l / 32
// lists as k = 8 (l / 32) + r), so each operand chunk of 8 is one 16-byte load. xt may be
// null (check only). Sets route[b] when a value is an inf or a nan, and with amax the largest
// |x| of the (b, h) slice (ordered float bits, atomic max).
// ---------------------------------------------------------------------------------------
constexpr int kTRows = 4;  // 64-row tiles per workgroup of dense_bwd_t_kernel

__global__ __launch_bounds__(256) void dense_bwd_t_kernel(const uint16_t* __restrict__ x, int64_t xsb, int64_t xsr,
                                                          int64_t xsh, int R, int Rpad, int H, int in_fp16,
                                                          uint16_t* __restrict__ xt, int* __restrict__ route,
                                                          uint32_t* __restrict__ amax) {
  __shared__ __align__(16) uint16_t tile[64][72];  // [d][row], rows of 144 bytes
  __shared__ float wmax[4];
  const int h = blockIdx.y, b = blockIdx.z;
  const uint32_t e = in_fp16 ? 0x7C00u : 0x7F80u;
  uint32_t nf = 0u;
  float mx = 0.f;
  // kTRows tiles of 64 rows per workgroup (one tile alone is too little work for a workgroup).
  for (int rt = 0; rt < kTRows; ++rt) {
    const int r0 = (blockIdx.x * kTRows + rt) * 64;
    if (r0 >= Rpad) break;
    if (rt > 0) __syncthreads();  // the previous tile's reads of the LDS tile are done
#pragma unroll
    for (int it = 0; it < 2; ++it) {
      const int idx = threadIdx.x + it * 256;
      const int row = idx >> 3, c = idx & 7;
      uint4 val = make_uint4(0, 0, 0, 0);
      if (r0 + row < R) val = *reinterpret_cast<const uint4*>(x + b * xsb + (int64_t)(r0 + row) * xsr + h * xsh + c * 8);
      const uint32_t w[4] = {val.x, val.y, val.z, val.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        nf |= nonfinite2(w[i], e);
        mx = fmaxf(mx, fmaxf(fabsf(in_to_float(in_fp16, w[i] & 0xFFFFu)), fabsf(in_to_float(in_fp16, w[i] >> 16))));
        if (xt != nullptr) {
          tile[c * 8 + 2 * i][row] = (uint16_t)(w[i] & 0xFFFFu);
          tile[c * 8 + 2 * i + 1][row] = (uint16_t)(w[i] >> 16);
        }
      }
    }
    if (xt == nullptr) continue;
    __syncthreads();
#pragma unroll
    for (int it = 0; it < 2; ++it) {
      const int idx = threadIdx.x + it * 256;
      const int d = idx >> 3, kc = idx & 7;
      // r' = 8 kc + 0..7 holds rows 16 (kc / 2) + 4 (kc % 2) + {0..3, 8..11}
      const int k0 = 16 * (kc >> 1) + 4 * (kc & 1);
      const uint2 lo = *reinterpret_cast<const uint2*>(&tile[d][k0]);
      const uint2 hi = *reinterpret_cast<const uint2*>(&tile[d][k0 + 8]);
      *reinterpret_cast<uint4*>(xt + (((int64_t)b * H + h) * 64 + d) * Rpad + r0 + kc * 8) =
          make_uint4(lo.x, lo.y, hi.x, hi.y);
    }
  }
  if (nf != 0u) route[b] = 1;  // every writer stores the same value
  if (amax != nullptr) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
    __syncthreads();
    if ((threadIdx.x & 63) == 0) wmax[threadIdx.x >> 6] = mx;
    __syncthreads();
    if (threadIdx.x == 0)
      atomicMax(amax + (int64_t)b * H + h, __float_as_uint(fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]))));
  }
}

struct DenseBwdParams {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const uint16_t* dout;
  const uint16_t* qt;   // [B][H][64][tpad], rows permuted
  const uint16_t* dot;  // [B][H][64][tpad], rows permuted
  const uint16_t* kt;   // [B][H][64][spad], rows permuted
  const uint32_t* mask;   // query-major selection words [B][spad / 32][tpad]
  const uint32_t* maskT;  // key-major selection words [B][tpad / 32][spad]
  const float2* ls;       // [B][H][tpad] {lse * log2(e), delta}
  const uint32_t* amax;   // [2][B][H] largest |dO|, |V| (float bits)
  const int* route;       // [B]: computed by the CSR backward instead
  uint16_t* dq;
  uint16_t* dk;
  uint16_t* dv;
  int64_t qsb, qst, qsh;
  int64_t ksb, kss, ksh;
  int64_t vsb, vss, vsh;
  int64_t dosb, dost, dosh;
  int64_t dqsb, dqst, dqsh;
  int64_t dksb, dkss, dksh;
  int64_t dvsb, dvss, dvsh;
  int B, T, S, H, tpad, spad;
  float scale, scale_log2;
};

// dS enters its products as fp16 scaled by 2^e per (b, h): |ds| <= |dp| + |delta| <=
// 2 * 64 * max|dO| * max|V|, so e puts that bound at or below 2^14 (no overflow) while
// keeping small values normal. bf16 has fp32's exponent range: no scaling.
__device__ __forceinline__ float ds_scale(BF16, const DenseBwdParams&, int, int) { return 1.f; }
__device__ __forceinline__ float ds_scale(FP16, const DenseBwdParams& p, int b, int h) {
  const float mdo = __uint_as_float(p.amax[(int64_t)b * p.H + h]);
  const float mv = __uint_as_float(p.amax[((int64_t)p.B + b) * p.H + h]);
  const float bound = 128.f * mdo * mv;
  if (!(bound > 0.f) || !(bound <= 3.4028234663852886e38f)) return 1.f;
  int x;
  frexpf(bound, &x);  // bound <= 2^x
  return ldexpf(1.f, max(-100, min(100, 14 - x)));
}

constexpr int kBW = 4;    // waves per workgroup (two workgroups per CU)
constexpr int kBQPW = 2;  // 32-query blocks per wave in the dq pass
constexpr int kBQPB = kBW * kBQPW;  // 32-query blocks per workgroup in the dq pass (256 queries)
constexpr int kBKPB = kBW;          // 32-key blocks per workgroup in the dk/dv pass (128 keys)

// ---------------------------------------------------------------------------------------
// dq pass: 4 waves per workgroup, each on two 32-query blocks of one head (the forward's
// decomposition). Per 64-key tile the K rows, V rows and K^T (8 KB each for 64 keys of one
// head) are loaded straight into LDS a tile ahead, one barrier per tile.
// Per 32-key sub-tile and block: S^T = K Q^T from the selection bias, dP^T = V dO^T,
// p = exp2(s log2(e) scale - lse2), ds = p (dp - delta), dQ^T += K^T dS^T.
// ---------------------------------------------------------------------------------------
template <typename E>
__global__ __launch_bounds__(kBW * 64, 2) void dense_bwd_dq_kernel(const DenseBwdParams p) {
  __shared__ __align__(16) uint8_t ktile[2][8192];
  __shared__ __align__(16) uint8_t vtile[2][8192];
  __shared__ __align__(16) uint8_t kttile[2][8192];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: addresses built from it stay scalar
  const int h = blockIdx.x % p.H;
  const int qb0 = (blockIdx.x / p.H) * kBQPB + wave * kBQPW;
  const int b = blockIdx.y;
  if (p.route[b] != 0) return;  // the whole workgroup: before any barrier
  const int col = lane & 31, half = lane >> 5;
  const float sl2 = p.scale_log2;
  const float sig = ds_scale(E{}, p, b, h);
  int tq[kBQPW];
#pragma unroll
  for (int a = 0; a < kBQPW; ++a) tq[a] = (qb0 + a) * 32 + col;

  // B operands of S^T = K Q^T and dP^T = V dO^T: the lane's query, dims 16 ks + 8 half + 0..7.
  uint4 qa[kBQPW][4], da[kBQPW][4];
  float lse2[kBQPW], dlt[kBQPW];
#pragma unroll
  for (int a = 0; a < kBQPW; ++a) {
    const bool ok = tq[a] < p.T;
    const int t = ok ? tq[a] : 0;
    const uint16_t* qr = p.q + b * p.qsb + (int64_t)t * p.qst + h * p.qsh + half * 8;
    const uint16_t* dr = p.dout + b * p.dosb + (int64_t)t * p.dost + h * p.dosh + half * 8;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      qa[a][ks] = ok ? *reinterpret_cast<const uint4*>(qr + ks * 16) : make_uint4(0, 0, 0, 0);
      da[a][ks] = ok ? *reinterpret_cast<const uint4*>(dr + ks * 16) : make_uint4(0, 0, 0, 0);
    }
    const float2 st = p.ls[((int64_t)b * p.H + h) * p.tpad + tq[a]];
    lse2[a] = st.x;
    dlt[a] = st.y;
  }
  f32x16 acc[kBQPW][2];
#pragma unroll
  for (int a = 0; a < kBQPW; ++a)
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[a][db][r] = 0.f;

  // Tile staging: each thread moves two 16-byte chunks of each of K, V and K^T per tile
  // (rows srow and srow + 32), loaded straight into LDS. Lane i of a wave writes the 16 bytes
  // at the wave's 1 KB segment + 16 i = row srow, physical chunk sc, so it reads the chunk
  // sc ^ swz(srow) that the swizzled layout keeps there (swz(srow + 32) = swz(srow)).
  const int srow = tid >> 3, sc = tid & 7;
  const int lc = sc ^ swz(srow);
  const int wseg = wave * 1024;
  // A tile's base addresses are uniform (scalar registers); a lane adds a 32-bit byte offset
  // (the host keeps the K and V token strides below 2^24 bytes and 64 rows of K^T below 2^32
  // bytes).
  const char* kbase = uniform_ptr(reinterpret_cast<const char*>(p.k + b * p.ksb + (int64_t)h * p.ksh));
  const char* vbase = uniform_ptr(reinterpret_cast<const char*>(p.v + b * p.vsb + (int64_t)h * p.vsh));
  const char* tbase = uniform_ptr(reinterpret_cast<const char*>(p.kt + ((int64_t)b * p.H + h) * 64 * p.spad));
  const uint32_t kss_b = (uint32_t)p.kss * 2u, vss_b = (uint32_t)p.vss * 2u;
  const uint32_t ccol = (uint32_t)lc * 16u;
  const uint32_t to0 = ((uint32_t)srow * (uint32_t)p.spad + (uint32_t)lc * 8u) * 2u;
  const uint32_t to1 = to0 + (uint32_t)p.spad * 64u;  // row srow + 32
  auto dload = [&](int k0, int bf) {
    // Rows past the end read row S - 1 (their keys are never selected). The tile may start
    // past it (S_pad is a whole number of key blocks): rows are taken from a base row at most
    // S - 1, so the lane offsets stay in [0, 63] rows.
    const TileRows tr = tile_rows(k0, srow, p.S);
    const uint32_t r0 = tr.r0, r1 = tr.r1;
    const char* kt = kbase + (int64_t)tr.base * kss_b;
    const char* vt = vbase + (int64_t)tr.base * vss_b;
    const char* tt = tbase + (int64_t)k0 * 2;
    buffer_load16_lds(kt, __umul24(r0, kss_b) + ccol, &ktile[bf][wseg]);
    buffer_load16_lds(kt, __umul24(r1, kss_b) + ccol, &ktile[bf][wseg + 4096]);
    buffer_load16_lds(vt, __umul24(r0, vss_b) + ccol, &vtile[bf][wseg]);
    buffer_load16_lds(vt, __umul24(r1, vss_b) + ccol, &vtile[bf][wseg + 4096]);
    buffer_load16_lds(tt, to0, &kttile[bf][wseg]);
    buffer_load16_lds(tt, to1, &kttile[bf][wseg + 4096]);
  };
  // Operand reads: K and V rows 32 st + col (chunk 2 ks + half); K^T rows 32 db + col (chunk
  // 4 st + 2 ks + half); swz of these rows is swz(col).
  const int fc = swz(col);
  auto koff = [&](int st, int ks) { return col * 128 + st * 4096 + (((2 * ks + half) ^ fc) << 4); };
  auto toff = [&](int db, int st, int ks) { return col * 128 + db * 4096 + (((4 * st + 2 * ks + half) ^ fc) << 4); };
  const int nsub = p.spad >> 5;
  const char* mblk = uniform_ptr(reinterpret_cast<const char*>(p.mask + (int64_t)b * nsub * p.tpad + qb0 * 32));
  const int64_t mrow_b = (int64_t)p.tpad * 4;  // bytes per sub-tile row of selection words
  auto mword = [&](int j, int a) {
    return buffer_load4(mblk + min(j, nsub - 1) * mrow_b, (uint32_t)(col + 32 * a) * 4u);
  };

  auto sub = [&](const uint8_t* kt, const uint8_t* vt, const uint8_t* ktt, int st, const uint32_t (&w)[kBQPW]) {
    f32x16 s[kBQPW], dp[kBQPW];
#pragma unroll
    for (int a = 0; a < kBQPW; ++a) {
      // Bias-order words: entry 4 g + j of this lane is the sign bit of byte j of w << (g + 4
      // half), set when the key is not selected; a sign-extended byte select masks -inf (one
      // instruction per entry).
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const uint32_t sh = w[a] << (g + 4 * half);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          s[a][4 * g + j] = __uint_as_float((uint32_t)(int32_t)(int8_t)(sh >> (8 * j)) & 0xFF800000u);
          dp[a][4 * g + j] = 0.f;
        }
      }
    }
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const uint4 ka = *reinterpret_cast<const uint4*>(kt + koff(st, ks));
#pragma unroll
      for (int a = 0; a < kBQPW; ++a) s[a] = mma(E{}, ka, qa[a][ks], s[a]);
    }
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const uint4 va = *reinterpret_cast<const uint4*>(vt + koff(st, ks));
#pragma unroll
      for (int a = 0; a < kBQPW; ++a) dp[a] = mma(E{}, va, da[a][ks], dp[a]);
    }
    // Per block: p and dS, then its dQ products, so that the second block's exp2 overlaps the
    // first block's products (the K^T operands read once for both).
    uint4 ta[2][2];
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) ta[db][ks] = *reinterpret_cast<const uint4*>(ktt + toff(db, st, ks));
#pragma unroll
    for (int a = 0; a < kBQPW; ++a) {
      float dsv[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float pv = fexp2(fmaf(s[a][r], sl2, -lse2[a]));
        dsv[r] = pv * ((dp[a][r] - dlt[a]) * sig);
      }
      const uint4 dsb[2] = {pack_quad<E>(dsv), pack_quad<E>(dsv + 8)};
#pragma unroll
      for (int db = 0; db < 2; ++db)
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) acc[a][db] = mma(E{}, ta[db][ks], dsb[ks], acc[a][db]);
    }
  };

  // Tile n (64 keys) lives in LDS buffer n % 2; while computing it the workgroup loads tile
  // n + 1 into the other buffer; one barrier per tile.
  const int ntiles = p.spad >> 6;
  dload(0, 0);
  uint32_t w0[kBQPW] = {mword(0, 0), mword(0, 1)}, w1[kBQPW] = {mword(1, 0), mword(1, 1)};
  __builtin_amdgcn_s_waitcnt(0x0070);  // vmcnt(0) lgkmcnt(0): tile 0 is in LDS
  __syncthreads();
#pragma unroll 1
  for (int n = 0; n < ntiles; ++n) {
    const int buf = n & 1;
    const uint32_t wn0[kBQPW] = {mword(2 * n + 2, 0), mword(2 * n + 2, 1)};
    const uint32_t wn1[kBQPW] = {mword(2 * n + 3, 0), mword(2 * n + 3, 1)};
    // the other buffer was last read before the previous barrier
    if (n + 1 < ntiles) dload((n + 1) * 64, buf ^ 1);
    sub(ktile[buf], vtile[buf], kttile[buf], 0, w0);
    sub(ktile[buf], vtile[buf], kttile[buf], 1, w1);
#pragma unroll
    for (int a = 0; a < kBQPW; ++a) {
      w0[a] = wn0[a];
      w1[a] = wn1[a];
    }
    __builtin_amdgcn_s_waitcnt(0x0070);  // vmcnt(0) lgkmcnt(0): the next tile is in LDS
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  }

  // dq = scale * dQ^T / sig; entry r of d-tile db is d = 32 db + 8 (r / 4) + 4 half + r % 4.
  const float osc = p.scale / sig;
#pragma unroll
  for (int a = 0; a < kBQPW; ++a) {
    const int t = tq[a];
    if (t >= p.T) continue;
    uint16_t* orow = p.dq + b * p.dqsb + (int64_t)t * p.dqst + h * p.dqsh;
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
      for (int gq = 0; gq < 4; ++gq) {
        const int d0 = 32 * db + 8 * gq + 4 * half;
        uint16_t hv[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) hv[i] = to_half_bits(E{}, acc[a][db][4 * gq + i] * osc);
        *reinterpret_cast<uint2*>(orow + d0) =
            make_uint2((uint32_t)hv[0] | ((uint32_t)hv[1] << 16), (uint32_t)hv[2] | ((uint32_t)hv[3] << 16));
      }
  }
}

// ---------------------------------------------------------------------------------------
// dk/dv pass: 4 waves per workgroup, each on one 32-key block of one head; the key block's K
// and V rows are the stationary B operands, dK^T and dV^T accumulate in registers over every
// query. Per 64-query tile the Q rows, dO rows, Q^T, dO^T (8 KB each) and the queries' {lse2,
// delta} are loaded straight into LDS a tile ahead, one barrier per tile. Per 32-query
// sub-tile: S = Q K^T from the selection bias (key-major words), dP = dO V^T, p and ds as in
// the dq pass, dV^T += dO^T P, dK^T += Q^T dS.
// ---------------------------------------------------------------------------------------
template <typename E>
__global__ __launch_bounds__(kBW * 64, 2) void dense_bwd_dkdv_kernel(const DenseBwdParams p) {
  __shared__ __align__(16) uint8_t qtile[2][8192];
  __shared__ __align__(16) uint8_t dotile[2][8192];
  __shared__ __align__(16) uint8_t qttile[2][8192];
  __shared__ __align__(16) uint8_t dottile[2][8192];
  __shared__ __align__(16) float2 lstile[2][64];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: addresses built from it stay scalar
  const int h = blockIdx.x % p.H;
  const int kb = (blockIdx.x / p.H) * kBKPB + wave;
  const int b = blockIdx.y;
  if (p.route[b] != 0) return;  // the whole workgroup: before any barrier
  const int col = lane & 31, half = lane >> 5;
  const float sl2 = p.scale_log2;
  const float sig = ds_scale(E{}, p, b, h);
  const int key = kb * 32 + col;
  const bool kok = key < p.S;

  // B operands of S = Q K^T and dP = dO V^T: the lane's key, dims 16 ks + 8 half + 0..7.
  uint4 kbo[4], vbo[4];
  {
    const int s = kok ? key : 0;
    const uint16_t* kr = p.k + b * p.ksb + (int64_t)s * p.kss + h * p.ksh + half * 8;
    const uint16_t* vr = p.v + b * p.vsb + (int64_t)s * p.vss + h * p.vsh + half * 8;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      kbo[ks] = kok ? *reinterpret_cast<const uint4*>(kr + ks * 16) : make_uint4(0, 0, 0, 0);
      vbo[ks] = kok ? *reinterpret_cast<const uint4*>(vr + ks * 16) : make_uint4(0, 0, 0, 0);
    }
  }
  f32x16 dka[2], dva[2];
#pragma unroll
  for (int db = 0; db < 2; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      dka[db][r] = 0.f;
      dva[db][r] = 0.f;
    }

  // Tile staging: two 16-byte chunks of each of Q, dO (rows = queries srow, srow + 32), Q^T
  // and dO^T (rows = d srow, srow + 32) per thread, loaded straight into LDS; threads 0..31
  // move the {lse2, delta} of two queries each. Lane i of a wave writes the 16 bytes at the
  // wave's 1 KB segment + 16 i = row srow, physical chunk sc, so it reads the chunk
  // sc ^ swz(srow) that the swizzled layout keeps there (swz(srow + 32) = swz(srow)).
  const int srow = tid >> 3, sc = tid & 7;
  const int lc = sc ^ swz(srow);
  const int wseg = wave * 1024;
  // A tile's base addresses are uniform (scalar registers); a lane adds a 32-bit byte offset
  // (the host keeps the q and dO token strides below 2^24 bytes and 64 rows of Q^T below
  // 2^32 bytes).
  const char* qbase = uniform_ptr(reinterpret_cast<const char*>(p.q + b * p.qsb + (int64_t)h * p.qsh));
  const char* dbase = uniform_ptr(reinterpret_cast<const char*>(p.dout + b * p.dosb + (int64_t)h * p.dosh));
  const int64_t thead = ((int64_t)b * p.H + h) * 64 * p.tpad;
  const char* qtbase = uniform_ptr(reinterpret_cast<const char*>(p.qt + thead));
  const char* dtbase = uniform_ptr(reinterpret_cast<const char*>(p.dot + thead));
  const char* lbase = uniform_ptr(reinterpret_cast<const char*>(p.ls + ((int64_t)b * p.H + h) * p.tpad));
  const uint32_t qst_b = (uint32_t)p.qst * 2u, dst_b = (uint32_t)p.dost * 2u;
  const uint32_t ccol = (uint32_t)lc * 16u;
  const uint32_t to0 = ((uint32_t)srow * (uint32_t)p.tpad + (uint32_t)lc * 8u) * 2u;
  const uint32_t to1 = to0 + (uint32_t)p.tpad * 64u;  // row srow + 32
  const uint32_t lo = (uint32_t)(tid & 31) * 16u;     // two {lse2, delta} per thread
  auto dload = [&](int t0, int bf) {
    // Rows past the end read row T - 1 (their queries never selected a key). The tile may
    // start past it (T_pad is a whole number of query blocks): rows are taken from a base row
    // at most T - 1, so the lane offsets stay in [0, 63] rows.
    const TileRows tr = tile_rows(t0, srow, p.T);
    const uint32_t r0 = tr.r0, r1 = tr.r1;
    const char* qt = qbase + (int64_t)tr.base * qst_b;
    const char* dt = dbase + (int64_t)tr.base * dst_b;
    const char* qtt = qtbase + (int64_t)t0 * 2;
    const char* dtt = dtbase + (int64_t)t0 * 2;
    buffer_load16_lds(qt, __umul24(r0, qst_b) + ccol, &qtile[bf][wseg]);
    buffer_load16_lds(qt, __umul24(r1, qst_b) + ccol, &qtile[bf][wseg + 4096]);
    buffer_load16_lds(dt, __umul24(r0, dst_b) + ccol, &dotile[bf][wseg]);
    buffer_load16_lds(dt, __umul24(r1, dst_b) + ccol, &dotile[bf][wseg + 4096]);
    buffer_load16_lds(qtt, to0, &qttile[bf][wseg]);
    buffer_load16_lds(qtt, to1, &qttile[bf][wseg + 4096]);
    buffer_load16_lds(dtt, to0, &dottile[bf][wseg]);
    buffer_load16_lds(dtt, to1, &dottile[bf][wseg + 4096]);
    if (tid < 32) buffer_load16_lds(lbase + (int64_t)t0 * 8, lo, &lstile[bf][0]);
  };
  const int fc = swz(col);
  auto koff = [&](int st, int ks) { return col * 128 + st * 4096 + (((2 * ks + half) ^ fc) << 4); };
  auto toff = [&](int db, int st, int ks) { return col * 128 + db * 4096 + (((4 * st + 2 * ks + half) ^ fc) << 4); };
  // Key-major selection words of the lane's key, one per 32-query block.
  const int nqbp = p.tpad >> 5;
  const char* mblk = uniform_ptr(reinterpret_cast<const char*>(p.maskT + (int64_t)b * nqbp * p.spad + kb * 32));
  const int64_t mrow_b = (int64_t)p.spad * 4;  // bytes per query-block row of selection words
  auto mword = [&](int j) { return buffer_load4(mblk + min(j, nqbp - 1) * mrow_b, (uint32_t)col * 4u); };

  auto sub = [&](const uint8_t* qtl, const uint8_t* dtl, const uint8_t* qttl, const uint8_t* dttl,
                 const float2* lsl, int st, uint32_t w) {
    // {lse2, delta} of queries 32 st + 8 gq + 4 half + 0..3, read before the products so that
    // their LDS latency hides behind them
    float4 u[8];
#pragma unroll
    for (int gq = 0; gq < 4; ++gq) {
      const float4* l4 = reinterpret_cast<const float4*>(lsl + 32 * st + 8 * gq + 4 * half);
      u[2 * gq] = l4[0];
      u[2 * gq + 1] = l4[1];
    }
    f32x16 s, dp;
    // Entry r = 4 g + j of this lane is query 8 g + 4 half + j of the sub-tile. Bias-order
    // words: it is the sign bit of byte j of w << (g + 4 half), set when the query did not
    // select the key; a sign-extended byte select masks -inf (one instruction per entry).
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const uint32_t sh = w << (g + 4 * half);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        s[4 * g + j] = __uint_as_float((uint32_t)(int32_t)(int8_t)(sh >> (8 * j)) & 0xFF800000u);
        dp[4 * g + j] = 0.f;
      }
    }
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) s = mma(E{}, *reinterpret_cast<const uint4*>(qtl + koff(st, ks)), kbo[ks], s);
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) dp = mma(E{}, *reinterpret_cast<const uint4*>(dtl + koff(st, ks)), vbo[ks], dp);
    float pv[16], dsv[16];
#pragma unroll
    for (int gq = 0; gq < 4; ++gq) {
      const float4 u0 = u[2 * gq], u1 = u[2 * gq + 1];
      const float l2[4] = {u0.x, u0.z, u1.x, u1.z};
      const float dl[4] = {u0.y, u0.w, u1.y, u1.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = 4 * gq + i;
        pv[r] = fexp2(fmaf(s[r], sl2, -l2[i]));
        dsv[r] = pv[r] * ((dp[r] - dl[i]) * sig);
      }
    }
    const uint4 pb[2] = {pack_quad<E>(pv), pack_quad<E>(pv + 8)};
    const uint4 sb[2] = {pack_quad<E>(dsv), pack_quad<E>(dsv + 8)};
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        dva[db] = mma(E{}, *reinterpret_cast<const uint4*>(dttl + toff(db, st, ks)), pb[ks], dva[db]);
        dka[db] = mma(E{}, *reinterpret_cast<const uint4*>(qttl + toff(db, st, ks)), sb[ks], dka[db]);
      }
  };

  const int ntiles = p.tpad >> 6;
  dload(0, 0);
  uint32_t w0 = mword(0), w1 = mword(1);
  __builtin_amdgcn_s_waitcnt(0x0070);  // vmcnt(0) lgkmcnt(0): tile 0 is in LDS
  __syncthreads();
#pragma unroll 1
  for (int n = 0; n < ntiles; ++n) {
    const int buf = n & 1;
    const uint32_t wn0 = mword(2 * n + 2), wn1 = mword(2 * n + 3);
    // the other buffer was last read before the previous barrier
    if (n + 1 < ntiles) dload((n + 1) * 64, buf ^ 1);
    sub(qtile[buf], dotile[buf], qttile[buf], dottile[buf], lstile[buf], 0, w0);
    sub(qtile[buf], dotile[buf], qttile[buf], dottile[buf], lstile[buf], 1, w1);
    w0 = wn0;
    w1 = wn1;
    __builtin_amdgcn_s_waitcnt(0x0070);  // vmcnt(0) lgkmcnt(0): the next tile is in LDS
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  }

  if (!kok) return;
  // entry r of d-tile db is d = 32 db + 8 (r / 4) + 4 half + r % 4
  const float ksc = p.scale / sig;
  uint16_t* krow = p.dk + b * p.dksb + (int64_t)key * p.dkss + h * p.dksh;
  uint16_t* vrow = p.dv + b * p.dvsb + (int64_t)key * p.dvss + h * p.dvsh;
#pragma unroll
  for (int db = 0; db < 2; ++db)
#pragma unroll
    for (int gq = 0; gq < 4; ++gq) {
      const int d0 = 32 * db + 8 * gq + 4 * half;
      uint16_t hk[4], hv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        hk[i] = to_half_bits(E{}, dka[db][4 * gq + i] * ksc);
        hv[i] = to_half_bits(E{}, dva[db][4 * gq + i]);
      }
      *reinterpret_cast<uint2*>(krow + d0) =
          make_uint2((uint32_t)hk[0] | ((uint32_t)hk[1] << 16), (uint32_t)hk[2] | ((uint32_t)hk[3] << 16));
      *reinterpret_cast<uint2*>(vrow + d0) =
          make_uint2((uint32_t)hv[0] | ((uint32_t)hv[1] << 16), (uint32_t)hv[2] | ((uint32_t)hv[3] << 16));
    }
}

struct DenseBwdLayout {
  size_t mask, maskT, flags, amax, ls, qt, dot, kt, total;
  int nqb, nqb_pad, tpad, spad, nchunk;
};

DenseBwdLayout dense_bwd_layout(int64_t B, int64_t T, int64_t S, int64_t H) {
  DenseBwdLayout L;
  L.nqb = (int)((T + 31) / 32);
  L.nqb_pad = (L.nqb + kBQPB - 1) / kBQPB * kBQPB;
  L.tpad = L.nqb_pad * 32;
  L.spad = (int)((S + 32 * kBKPB - 1) / (32 * kBKPB) * (32 * kBKPB));
  L.nchunk = mask_nchunk(L.spad);
  if (L.nchunk < 1) L.nchunk = 1;
  auto up = [](size_t x) { return (x + 255) / 256 * 256; };
  size_t o = 0;
  L.mask = o;
  o = up(o + (size_t)B * (size_t)(L.spad / 32) * (size_t)L.tpad * 4);
  L.maskT = o;
  o = up(o + (size_t)B * (size_t)L.nqb_pad * (size_t)L.spad * 4);
  L.flags = o;
  o = up(o + (size_t)B * L.nqb * (size_t)L.nchunk * 4);
  L.amax = o;
  o = up(o + (size_t)2 * B * (size_t)H * 4);
  L.ls = o;
  o = up(o + (size_t)B * (size_t)H * (size_t)L.tpad * 8);
  L.qt = o;
  o = up(o + (size_t)B * (size_t)H * 64 * (size_t)L.tpad * 2);
  L.dot = o;
  o = up(o + (size_t)B * (size_t)H * 64 * (size_t)L.tpad * 2);
  L.kt = o;
  o = up(o + (size_t)B * (size_t)H * 64 * (size_t)L.spad * 2);
  L.total = o;
  return L;
}

}  // namespace
}  // namespace gw

extern "C" size_t gw_sparse_attn_bwd_dense_workspace_size(int64_t B, int64_t T, int64_t S, int64_t H, int64_t D,
                                                          int64_t K) {
  if (B <= 0 || T <= 0 || S <= 0 || H <= 0 || K <= 0 || D != 64) return 256;
  return gw::dense_bwd_layout(B, T, S, H).total;
}

extern "C" int gw_sparse_attn_bwd_dense(int dtype, const void* q, const int64_t* q_strides, const void* k,
                                        const int64_t* k_strides, const void* v, const int64_t* v_strides,
                                        const int32_t* kv_pos, int64_t pos_stride_b, int64_t pos_stride_t,
                                        const void* o, const int64_t* o_strides, const void* dout,
                                        const int64_t* do_strides, const float* lse, void* dq,
                                        const int64_t* dq_strides, void* dk, const int64_t* dk_strides, void* dv,
                                        const int64_t* dv_strides, int64_t B, int64_t T, int64_t S, int64_t H,
                                        int64_t D, int64_t K, float softmax_scale, int* route, void* workspace,
                                        size_t workspace_bytes, void* stream) {
  using namespace gw;
  clear_error();
  GW_CHECK_ARG(dtype == GW_DTYPE_BF16 || dtype == GW_DTYPE_FP16, "unsupported dtype code %d", dtype);
  GW_CHECK_ARG(B >= 0 && T >= 0 && S >= 0 && H >= 1 && K >= 0, "invalid sizes B=%lld T=%lld S=%lld H=%lld K=%lld",
               (long long)B, (long long)T, (long long)S, (long long)H, (long long)K);
  if (D != 64) return set_error(GW_ERR_UNSUPPORTED, "the dense backward needs head dim 64, got %lld", (long long)D);
  if (!(softmax_scale > 0.f) || !(softmax_scale < 3.4e38f))
    return set_error(GW_ERR_UNSUPPORTED, "the dense backward needs a positive finite softmax scale, got %g",
                     (double)softmax_scale);
  if (B == 0 || T == 0 || S == 0) return GW_OK;
  GW_CHECK_ARG(K >= 1, "kv_positions must have at least one candidate");
  GW_CHECK_ARG(q && k && v && kv_pos && o && dout && lse && dq && dk && dv && route, "null pointer");
  GW_CHECK_ARG(q_strides && k_strides && v_strides && o_strides && do_strides && dq_strides && dk_strides &&
                   dv_strides,
               "null stride array");
  GW_CHECK_ARG(aligned16(q) && aligned16(k) && aligned16(v) && aligned16(o) && aligned16(dout) && aligned16(dq) &&
                   aligned16(dk) && aligned16(dv),
               "q/k/v/o/dO/dq/dk/dv must be 16-byte aligned");
  const int64_t* all[] = {q_strides, k_strides, v_strides, o_strides, do_strides, dq_strides, dk_strides, dv_strides};
  for (const int64_t* st : all)
    for (int i = 0; i < 3; ++i) GW_CHECK_ARG(st[i] % 8 == 0, "b/t/h strides must be multiples of 8 elements");
  GW_CHECK_ARG(B <= 65535 && T < (1ll << 30) && S < (1ll << 30) && K < (1ll << 31), "size exceeds the grid range");
  const DenseBwdLayout L = dense_bwd_layout(B, T, S, H);
  // Query blocks: at most 65535 (T <= 65528 * 32 once padded to whole workgroups).
  if ((int64_t)(L.nqb_pad / kBQPB) * H >= (1ll << 31) || (int64_t)(L.spad / (32 * kBKPB)) * H >= (1ll << 31) ||
      L.nqb_pad > 65535 || H > 65535)
    return set_error(GW_ERR_UNSUPPORTED, "the dense backward takes at most %d queries, got %lld", 65528 * 32,
                     (long long)T);
  // Limits of the kernels' 32-bit lane offsets: token strides of q, k, v, dO below 2^23
  // elements (a 24-bit multiply), 64 rows of the transposed operands below 2^32 bytes. T is
  // padded to a multiple of 256 and S to one of 128, so T, S <= 2^25 - 256 keeps both padded
  // lengths below 2^25.
  if (q_strides[1] >= kDenseBwdMaxRowStride || k_strides[1] >= kDenseBwdMaxRowStride ||
      v_strides[1] >= kDenseBwdMaxRowStride || do_strides[1] >= kDenseBwdMaxRowStride ||
      (int64_t)L.spad * 128 >= (1ll << 32) || (int64_t)L.tpad * 128 >= (1ll << 32))
    return set_error(GW_ERR_UNSUPPORTED,
                     "the dense backward needs token strides below %lld elements and T, S <= %lld",
                     (long long)kDenseBwdMaxRowStride, (long long)((1ll << 25) - 256));
  GW_CHECK_ARG(workspace != nullptr && workspace_bytes >= L.total && aligned16(workspace),
               "the dense backward needs a 16-byte aligned %zu-byte workspace, got %zu", L.total, workspace_bytes);
  hipStream_t st = static_cast<hipStream_t>(stream);
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  uint32_t* mask = reinterpret_cast<uint32_t*>(ws + L.mask);
  uint32_t* maskT = reinterpret_cast<uint32_t*>(ws + L.maskT);
  int* flags = reinterpret_cast<int*>(ws + L.flags);
  uint32_t* amax = reinterpret_cast<uint32_t*>(ws + L.amax);
  float2* ls = reinterpret_cast<float2*>(ws + L.ls);
  uint16_t* qt = reinterpret_cast<uint16_t*>(ws + L.qt);
  uint16_t* dot = reinterpret_cast<uint16_t*>(ws + L.dot);
  uint16_t* kt = reinterpret_cast<uint16_t*>(ws + L.kt);
  const int in_fp16 = dtype == GW_DTYPE_FP16 ? 1 : 0;

  {
    const int n = (int)(2 * B * H > B ? 2 * B * H : B);
    hipLaunchKernelGGL(dense_bwd_clear_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, route, (int)B,
                       amax, (int)(2 * B * H));
    GW_HIP_LAUNCH_CHECK("dense_bwd_clear_kernel launch");
  }
  {
    const int vec = (K % 4 == 0 && pos_stride_t % 4 == 0 && pos_stride_b % 4 == 0 &&
                     (reinterpret_cast<uintptr_t>(kv_pos) & 15) == 0)
                        ? 1
                        : 0;
    hipLaunchKernelGGL(dense_mask_kernel, dim3(L.nchunk, L.nqb_pad, (unsigned)B), dim3(256), 0, st, kv_pos,
                       pos_stride_b, pos_stride_t, (int)T, (int)S, L.spad, (int)K, L.nqb, L.tpad, L.nchunk, vec, 0,
                       mask, flags, nullptr, nullptr, maskT, route, 1, mask_chunk_keys(L.spad, L.nchunk));
    GW_HIP_LAUNCH_CHECK("dense_mask_kernel launch");
  }
  {
    const dim3 grid((unsigned)(((int64_t)L.tpad * H + 31) / 32), (unsigned)B);
    if (dtype == GW_DTYPE_BF16)
      hipLaunchKernelGGL((dense_bwd_rowstats_kernel<BF16>), grid, dim3(256), 0, st,
                         static_cast<const uint16_t*>(o), o_strides[0], o_strides[1], o_strides[2],
                         static_cast<const uint16_t*>(dout), do_strides[0], do_strides[1], do_strides[2], lse, (int)T,
                         (int)H, L.tpad, ls, route);
    else
      hipLaunchKernelGGL((dense_bwd_rowstats_kernel<FP16>), grid, dim3(256), 0, st,
                         static_cast<const uint16_t*>(o), o_strides[0], o_strides[1], o_strides[2],
                         static_cast<const uint16_t*>(dout), do_strides[0], do_strides[1], do_strides[2], lse, (int)T,
                         (int)H, L.tpad, ls, route);
    GW_HIP_LAUNCH_CHECK("dense_bwd_rowstats_kernel launch");
  }
  {
    const dim3 gq((unsigned)((L.tpad / 64 + kTRows - 1) / kTRows), (unsigned)H, (unsigned)B);
    hipLaunchKernelGGL(dense_bwd_t_kernel, gq, dim3(256), 0, st, static_cast<const uint16_t*>(q), q_strides[0],
                       q_strides[1], q_strides[2], (int)T, L.tpad, (int)H, in_fp16, qt, route, nullptr);
    GW_HIP_LAUNCH_CHECK("dense_bwd_t_kernel (q) launch");
    hipLaunchKernelGGL(dense_bwd_t_kernel, gq, dim3(256), 0, st, static_cast<const uint16_t*>(dout), do_strides[0],
                       do_strides[1], do_strides[2], (int)T, L.tpad, (int)H, in_fp16, dot, route, amax);
    GW_HIP_LAUNCH_CHECK("dense_bwd_t_kernel (dO) launch");
    const dim3 gk((unsigned)((L.spad / 64 + kTRows - 1) / kTRows), (unsigned)H, (unsigned)B);
    hipLaunchKernelGGL(dense_bwd_t_kernel, gk, dim3(256), 0, st, static_cast<const uint16_t*>(k), k_strides[0],
                       k_strides[1], k_strides[2], (int)S, L.spad, (int)H, in_fp16, kt, route, nullptr);
    GW_HIP_LAUNCH_CHECK("dense_bwd_t_kernel (k) launch");
    hipLaunchKernelGGL(dense_bwd_t_kernel, gk, dim3(256), 0, st, static_cast<const uint16_t*>(v), v_strides[0],
                       v_strides[1], v_strides[2], (int)S, L.spad, (int)H, in_fp16, nullptr, route, amax + B * H);
    GW_HIP_LAUNCH_CHECK("dense_bwd_t_kernel (v) launch");
  }

  DenseBwdParams p;
  p.q = static_cast<const uint16_t*>(q);
  p.k = static_cast<const uint16_t*>(k);
  p.v = static_cast<const uint16_t*>(v);
  p.dout = static_cast<const uint16_t*>(dout);
  p.qt = qt;
  p.dot = dot;
  p.kt = kt;
  p.mask = mask;
  p.maskT = maskT;
  p.ls = ls;
  p.amax = amax;
  p.route = route;
  p.dq = static_cast<uint16_t*>(dq);
  p.dk = static_cast<uint16_t*>(dk);
  p.dv = static_cast<uint16_t*>(dv);
  p.qsb = q_strides[0]; p.qst = q_strides[1]; p.qsh = q_strides[2];
  p.ksb = k_strides[0]; p.kss = k_strides[1]; p.ksh = k_strides[2];
  p.vsb = v_strides[0]; p.vss = v_strides[1]; p.vsh = v_strides[2];
  p.dosb = do_strides[0]; p.dost = do_strides[1]; p.dosh = do_strides[2];
  p.dqsb = dq_strides[0]; p.dqst = dq_strides[1]; p.dqsh = dq_strides[2];
  p.dksb = dk_strides[0]; p.dkss = dk_strides[1]; p.dksh = dk_strides[2];
  p.dvsb = dv_strides[0]; p.dvss = dv_strides[1]; p.dvsh = dv_strides[2];
  p.B = (int)B;
  p.T = (int)T;
  p.S = (int)S;
  p.H = (int)H;
  p.tpad = L.tpad;
  p.spad = L.spad;
  p.scale = softmax_scale;
  p.scale_log2 = softmax_scale * kDLog2e;
  const dim3 gq((unsigned)(L.nqb_pad / kBQPB * H), (unsigned)B);
  const dim3 gk((unsigned)(L.spad / (32 * kBKPB) * H), (unsigned)B);
  if (dtype == GW_DTYPE_BF16) {
    hipLaunchKernelGGL((dense_bwd_dq_kernel<BF16>), gq, dim3(kBW * 64), 0, st, p);
    GW_HIP_LAUNCH_CHECK("dense_bwd_dq_kernel launch");
    hipLaunchKernelGGL((dense_bwd_dkdv_kernel<BF16>), gk, dim3(kBW * 64), 0, st, p);
    GW_HIP_LAUNCH_CHECK("dense_bwd_dkdv_kernel launch");
  } else {
    hipLaunchKernelGGL((dense_bwd_dq_kernel<FP16>), gq, dim3(kBW * 64), 0, st, p);
    GW_HIP_LAUNCH_CHECK("dense_bwd_dq_kernel launch");
    hipLaunchKernelGGL((dense_bwd_dkdv_kernel<FP16>), gk, dim3(kBW * 64), 0, st, p);
    GW_HIP_LAUNCH_CHECK("dense_bwd_dkdv_kernel launch");
  }
  return GW_OK;
}
