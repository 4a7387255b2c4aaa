// DSA layer glue: per-head LayerNorm, 2D rotary embedding and the 16-bit cast of the
// attention q/k and the lightning-indexer q/k/w, in one pass over the fused projection.
//
// Reference: DSAAttention._project_qkv_and_indexer_fused
// (easyvolcap/official_vggt/layers/dsa_attention.py:583-625) and the per-layer glue
// around the kernels (:4928-4948: q_norm/k_norm, rope, score_dtype cast;
// easyvolcap/official_vggt/layers/indexer.py:302-328: indexer k_norm, rope, cast), with
// RotaryPositionEmbedding2D (easyvolcap/official_vggt/layers/rope.py:62-200).
//
// Input y: the output of one GEMM of the token features with the concatenated weights
// [qkv | indexer q | indexer k | indexer w], row r = (b, n), columns
//   q: [q_off, +H*64), k: [k_off, +H*64), v: (left in place: the attention kernels read it
//   through strides), indexer q: [iq_off, +Hi*64), indexer k: [ik_off, +Hi*64),
//   indexer w: [iw_off, +Hi).
// Per 64-wide head vector x (fp32 math on the 16-bit inputs, one rounding at the end):
//   LayerNorm (attention q, k; indexer k; optional): (x - mean) / sqrt(var + eps) * g + b
//   2D RoPE (optional): dims [0, 32) rotate with the row's position p.y, dims [32, 64) with
//   p.x; within each 32-dim half, for i < 16 with c = cos[p][i], s = sin[p][i]:
//     out[i] = x[i] c - x[i+16] s,   out[i+16] = x[i+16] c + x[i] s
//   (rope.py:120-152: x * cos + cat(-x2, x1) * sin with cos/sin = cat(t, t) tables).
#include <algorithm>

#include "gw_common.h"

namespace gw {
namespace {

constexpr int kGlueD = 64;

struct GlueParams {
  const uint16_t* y;
  int64_t ldy;
  int q_off, k_off, iq_off, ik_off, iw_off;
  int H, Hi;
  const float* qn_w;
  const float* qn_b;
  const float* kn_w;
  const float* kn_b;
  const float* ikn_w;
  const float* ikn_b;
  float ln_eps;
  const int32_t* pos;      // [rows, 2] (y, x) or null
  const float* rope_cos;   // [rope_len, 16]
  const float* rope_sin;
  int rope_len;
  uint16_t* q_out;         // [rows, H, 64]
  uint16_t* k_out;         // [rows, H, 64]
  uint16_t* iq_out;        // [rows, Hi, 64]
  uint16_t* ik_out;        // [rows, Hi, 64]
  uint16_t* iw_out;        // [rows, Hi]
  int64_t rows;
};

// Eight lanes per head vector: lane j of a group holds dims [8j, 8j + 8) as one 16-byte
// chunk, so a wave moves 1 KB of consecutive columns per load or store; each wave takes
// kGlueVecs * 8 consecutive vectors per step (all loads issued first) in a grid-stride
// loop, with the LayerNorm parameters and rotary tables staged in LDS once per block.
// LayerNorm sums over the 8 lanes with DPP; the rotary partner of dims [8j, 8j + 8)
// within each 32-dim half is lane j ^ 2 (dims i and i + 16), one DPP quad permute.
constexpr int kGlueVecs = 4;
constexpr int kGlueMaxRope = 256;  // rotary positions staged in LDS (else read from global)

struct GlueVec {
  uint32_t row;
  int head, out_heads, col;
  int norm;  // -1: none, 0: attention q, 1: attention k, 2: indexer k
  uint16_t* out;
  bool live, gate;
};

__device__ __forceinline__ GlueVec glue_vec(const GlueParams& p, uint32_t vid, uint32_t nvec, uint32_t slots) {
  GlueVec v{};
  v.live = vid < nvec;
  if (!v.live) vid = 0;
  v.row = vid / slots;
  const int slot = (int)(vid - v.row * slots);
  v.norm = -1;
  if (slot < p.H) {
    v.head = slot;
    v.col = p.q_off + v.head * kGlueD;
    v.norm = p.qn_w ? 0 : -1;
    v.out = p.q_out;
    v.out_heads = p.H;
  } else if (slot < 2 * p.H) {
    v.head = slot - p.H;
    v.col = p.k_off + v.head * kGlueD;
    v.norm = p.kn_w ? 1 : -1;
    v.out = p.k_out;
    v.out_heads = p.H;
  } else if (slot < 2 * p.H + p.Hi) {
    v.head = slot - 2 * p.H;
    v.col = p.iq_off + v.head * kGlueD;
    v.out = p.iq_out;
    v.out_heads = p.Hi;
    v.gate = true;  // the indexer gate of this head travels with its query vector
  } else {
    v.head = slot - 2 * p.H - p.Hi;
    v.col = p.ik_off + v.head * kGlueD;
    v.norm = p.ikn_w ? 2 : -1;
    v.out = p.ik_out;
    v.out_heads = p.Hi;
  }
  return v;
}

template <typename E>
__global__ __launch_bounds__(256) void dsa_glue_kernel(const GlueParams p) {
  __shared__ float ln_s[3][2][kGlueD];  // (q, k, indexer k) x (weight, bias)
  __shared__ float rope_s[2][kGlueMaxRope * 16];
  const float* lnw[3] = {p.qn_w, p.kn_w, p.ikn_w};
  const float* lnb[3] = {p.qn_b, p.kn_b, p.ikn_b};
  for (int i = threadIdx.x; i < 3 * kGlueD; i += blockDim.x) {
    const int t = i / kGlueD, d = i % kGlueD;
    ln_s[t][0][d] = lnw[t] ? lnw[t][d] : 1.f;
    ln_s[t][1][d] = lnb[t] ? lnb[t][d] : 0.f;
  }
  const bool rope_lds = p.pos != nullptr && p.rope_len <= kGlueMaxRope;
  if (rope_lds) {
    for (int i = threadIdx.x; i < p.rope_len * 16; i += blockDim.x) {
      rope_s[0][i] = p.rope_cos[i];
      rope_s[1][i] = p.rope_sin[i];
    }
  }
  __syncthreads();
  const float* cos_t = rope_lds ? rope_s[0] : p.rope_cos;
  const float* sin_t = rope_lds ? rope_s[1] : p.rope_sin;

  const uint32_t slots = 2 * p.H + 2 * p.Hi;
  const uint32_t nvec = (uint32_t)(p.rows * slots);
  const int lane = threadIdx.x & 63;
  const int j = lane & 7;  // 16-byte chunk of each vector
  const int grp = lane >> 3;
  const uint32_t nwaves = gridDim.x * (blockDim.x >> 6);
  constexpr uint32_t kStep = 8 * kGlueVecs;
  for (uint32_t w = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6); w * kStep < nvec; w += nwaves) {
    GlueVec v[kGlueVecs];
    uint4 raw[kGlueVecs];
#pragma unroll
    for (int u = 0; u < kGlueVecs; ++u) {
      v[u] = glue_vec(p, w * kStep + u * 8 + grp, nvec, slots);
      raw[u] = *reinterpret_cast<const uint4*>(p.y + (int64_t)v[u].row * p.ldy + v[u].col + 8 * j);
    }
#pragma unroll
    for (int u = 0; u < kGlueVecs; ++u) {
      if (!v[u].live) continue;  // uniform over the 8-lane group
      const int64_t row = v[u].row;
      float x[8];
      unpack8<E>(raw[u], x);
      if (v[u].gate && j == 0) p.iw_out[row * p.Hi + v[u].head] = p.y[row * p.ldy + p.iw_off + v[u].head];
      if (v[u].norm >= 0) {  // uniform over the 8-lane group
        const float* g = &ln_s[v[u].norm][0][8 * j];
        const float* bta = &ln_s[v[u].norm][1][8 * j];
        float s = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) s += x[e];
        const float mean = group_sum<8>(s) * (1.f / kGlueD);
        float var = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float d = x[e] - mean;
          var += d * d;
        }
        const float rstd = 1.f / sqrtf(group_sum<8>(var) * (1.f / kGlueD) + p.ln_eps);
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] = (x[e] - mean) * rstd * g[e] + bta[e];
      }
      if (p.pos != nullptr) {
        const int pp = min(max(p.pos[row * 2 + (j >> 2)], 0), p.rope_len - 1);  // y below dim 32, x above
        const float* c = cos_t + pp * 16 + 8 * (j & 1);
        const float* sn = sin_t + pp * 16 + 8 * (j & 1);
        const float sign = (j & 2) ? 1.f : -1.f;  // dims [0, 16) take -x[i + 16] sin, [16, 32) +x[i] sin
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float partner = dpp<kDppXor2>(x[e]);
          x[e] = x[e] * c[e] + sign * partner * sn[e];
        }
      }
      *reinterpret_cast<uint4*>(v[u].out + (row * v[u].out_heads + v[u].head) * kGlueD + 8 * j) = pack8<E>(x);
    }
  }
}

// Backward of the glue, one head vector per 8 lanes as in the forward. With
// u = LN(x) (x_hat * g + b, or x without a norm) and o = R(p) u the rotation:
//   du = R(p)^T do:  du[i] = do[i] c + do[i+16] s,  du[i+16] = do[i+16] c - do[i] s
//   dg += du * x_hat,  db += du,  dx_hat = du * g,
//   dx = rstd * (dx_hat - mean(dx_hat) - x_hat * mean(dx_hat * x_hat))
// dy receives dx in the q, k, indexer q/k blocks and the gate gradient in the w block
// (the v block is not written). dg/db are summed per workgroup into ws[block][3][2][64]
// in a fixed order, then over workgroups by dsa_glue_ln_reduce_kernel.
struct GlueBwdParams {
  GlueParams f;            // forward inputs (y, layout, norms, rope); outputs unused
  const uint16_t* dq;      // [rows, H, 64]
  const uint16_t* dk;
  const uint16_t* diq;     // [rows, Hi, 64]
  const uint16_t* dik;
  const uint16_t* diw;     // [rows, Hi]
  uint16_t* dy;            // [rows, ldy]
  float* ws;               // [gridDim.x][3][2][64]
};

template <typename E>
__global__ __launch_bounds__(256) void dsa_glue_bwd_kernel(const GlueBwdParams bp) {
  const GlueParams& p = bp.f;
  __shared__ float ln_s[3][2][kGlueD];
  __shared__ float rope_s[2][kGlueMaxRope * 16];
  __shared__ float red[4][3][2][kGlueD];  // per-wave partial dg/db
  const float* lnw[3] = {p.qn_w, p.kn_w, p.ikn_w};
  const float* lnb[3] = {p.qn_b, p.kn_b, p.ikn_b};
  for (int i = threadIdx.x; i < 3 * kGlueD; i += blockDim.x) {
    const int t = i / kGlueD, d = i % kGlueD;
    ln_s[t][0][d] = lnw[t] ? lnw[t][d] : 1.f;
    ln_s[t][1][d] = lnb[t] ? lnb[t][d] : 0.f;
  }
  const bool rope_lds = p.pos != nullptr && p.rope_len <= kGlueMaxRope;
  if (rope_lds) {
    for (int i = threadIdx.x; i < p.rope_len * 16; i += blockDim.x) {
      rope_s[0][i] = p.rope_cos[i];
      rope_s[1][i] = p.rope_sin[i];
    }
  }
  __syncthreads();
  const float* cos_t = rope_lds ? rope_s[0] : p.rope_cos;
  const float* sin_t = rope_lds ? rope_s[1] : p.rope_sin;

  float acc[3][2][8];
#pragma unroll
  for (int t = 0; t < 3; ++t)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[t][0][e] = acc[t][1][e] = 0.f;

  const uint32_t slots = 2 * p.H + 2 * p.Hi;
  const uint32_t nvec = (uint32_t)(p.rows * slots);
  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  const int j = lane & 7;
  const int grp = lane >> 3;
  const uint32_t nwaves = gridDim.x * (blockDim.x >> 6);
  for (uint32_t w = blockIdx.x * (blockDim.x >> 6) + wv; w * 8 < nvec; w += nwaves) {
    const GlueVec v = glue_vec(p, w * 8 + grp, nvec, slots);
    if (!v.live) continue;  // uniform over the 8-lane group
    const int64_t row = v.row;
    const int slot = (int)(w * 8 + grp - v.row * slots);
    const uint16_t* gsrc;
    if (slot < p.H) gsrc = bp.dq;
    else if (slot < 2 * p.H) gsrc = bp.dk;
    else if (slot < 2 * p.H + p.Hi) gsrc = bp.diq;
    else gsrc = bp.dik;
    float x[8], d[8];
    unpack8<E>(*reinterpret_cast<const uint4*>(p.y + row * p.ldy + v.col + 8 * j), x);
    unpack8<E>(*reinterpret_cast<const uint4*>(gsrc + (row * v.out_heads + v.head) * kGlueD + 8 * j), d);
    if (v.gate && j == 0) bp.dy[row * p.ldy + p.iw_off + v.head] = bp.diw[row * p.Hi + v.head];
    if (p.pos != nullptr) {  // du = R^T do
      const int pp = min(max(p.pos[row * 2 + (j >> 2)], 0), p.rope_len - 1);
      const float* c = cos_t + pp * 16 + 8 * (j & 1);
      const float* sn = sin_t + pp * 16 + 8 * (j & 1);
      const float sign = (j & 2) ? -1.f : 1.f;  // dims [0, 16) take +do[i+16] s, [16, 32) -do[i] s
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float partner = dpp<kDppXor2>(d[e]);
        d[e] = d[e] * c[e] + sign * partner * sn[e];
      }
    }
    if (v.norm >= 0) {
      const float* g = &ln_s[v.norm][0][8 * j];
      float s = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) s += x[e];
      const float mean = group_sum<8>(s) * (1.f / kGlueD);
      float var = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float t = x[e] - mean;
        var += t * t;
      }
      const float rstd = 1.f / sqrtf(group_sum<8>(var) * (1.f / kGlueD) + p.ln_eps);
      float xh[8], dxh[8], m1 = 0.f, m2 = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        xh[e] = (x[e] - mean) * rstd;
        dxh[e] = d[e] * g[e];
        m1 += dxh[e];
        m2 += dxh[e] * xh[e];
      }
      m1 = group_sum<8>(m1) * (1.f / kGlueD);
      m2 = group_sum<8>(m2) * (1.f / kGlueD);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        acc[v.norm][0][e] += d[e] * xh[e];
        acc[v.norm][1][e] += d[e];
        d[e] = rstd * (dxh[e] - m1 - xh[e] * m2);
      }
    }
    *reinterpret_cast<uint4*>(bp.dy + row * p.ldy + v.col + 8 * j) = pack8<E>(d);
  }
  // Block sums of dg/db: lanes with the same chunk j (8 groups of a wave) first, then the
  // four waves, in a fixed order.
#pragma unroll
  for (int t = 0; t < 3; ++t)
#pragma unroll
    for (int k = 0; k < 2; ++k)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float x = acc[t][k][e];
        x += __shfl_xor(x, 8);
        x += __shfl_xor(x, 16);
        x += __shfl_xor(x, 32);
        if (grp == 0) red[wv][t][k][8 * j + e] = x;
      }
  __syncthreads();
  for (int i = threadIdx.x; i < 3 * 2 * kGlueD; i += blockDim.x) {
    const float* r = &red[0][0][0][0] + i;
    const int stride = 3 * 2 * kGlueD;
    bp.ws[(int64_t)blockIdx.x * stride + i] = ((r[0] + r[stride]) + r[2 * stride]) + r[3 * stride];
  }
}

__global__ __launch_bounds__(256) void dsa_glue_ln_reduce_kernel(const float* ws, int nblocks, float* dln) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= 3 * 2 * kGlueD) return;
  float s = 0.f;
  for (int b = 0; b < nblocks; ++b) s += ws[(int64_t)b * 3 * 2 * kGlueD + i];
  dln[i] = s;
}

}  // namespace
}  // namespace gw

extern "C" int gw_dsa_glue_fwd(int dtype, const void* y, int64_t rows, int64_t ldy, int64_t q_off, int64_t k_off,
                               int64_t iq_off, int64_t ik_off, int64_t iw_off, int64_t H, int64_t Hi, int64_t D,
                               const float* q_norm_w, const float* q_norm_b, const float* k_norm_w,
                               const float* k_norm_b, const float* idx_k_norm_w, const float* idx_k_norm_b,
                               float ln_eps, const int32_t* pos, const float* rope_cos, const float* rope_sin,
                               int64_t rope_len, void* q_out, void* k_out, void* idx_q_out, void* idx_k_out,
                               void* idx_w_out, void* stream) {
  using namespace gw;
  clear_error();
  GW_CHECK_ARG(dtype == GW_DTYPE_BF16 || dtype == GW_DTYPE_FP16, "unsupported dtype code %d", dtype);
  if (D != kGlueD) return set_error(GW_ERR_UNSUPPORTED, "head dim %lld not supported (64)", (long long)D);
  GW_CHECK_ARG(rows >= 0 && H >= 1 && Hi >= 0 && H <= 64 && Hi <= 64, "invalid sizes rows=%lld H=%lld Hi=%lld",
               (long long)rows, (long long)H, (long long)Hi);
  if (rows == 0) return GW_OK;
  GW_CHECK_ARG(y && q_out && k_out && (Hi == 0 || (idx_q_out && idx_k_out && idx_w_out)), "null tensor pointer");
  GW_CHECK_ARG(ldy % 8 == 0 && aligned16(y), "projection rows must be 16-byte aligned (ldy %% 8 == 0)");
  const int64_t offs[4] = {q_off, k_off, iq_off, ik_off};
  const int64_t widths[4] = {H * D, H * D, Hi * D, Hi * D};
  for (int i = 0; i < 4; ++i)
    GW_CHECK_ARG(offs[i] >= 0 && offs[i] % 8 == 0 && offs[i] + widths[i] <= ldy,
                 "column block %d at %lld (+%lld) must be 8-aligned and inside ldy=%lld", i, (long long)offs[i],
                 (long long)widths[i], (long long)ldy);
  GW_CHECK_ARG(iw_off >= 0 && iw_off + Hi <= ldy, "indexer gate columns outside the row");
  GW_CHECK_ARG((q_norm_w == nullptr) == (q_norm_b == nullptr) && (k_norm_w == nullptr) == (k_norm_b == nullptr) &&
                   (idx_k_norm_w == nullptr) == (idx_k_norm_b == nullptr),
               "LayerNorm weight and bias must both be given or both be null");
  GW_CHECK_ARG(pos == nullptr || (rope_cos && rope_sin && rope_len >= 1), "rope tables missing");
  GW_CHECK_ARG(aligned16(q_out) && aligned16(k_out) && aligned16(idx_q_out) && aligned16(idx_k_out),
               "outputs must be 16-byte aligned");  // null (Hi = 0) counts as aligned
  GW_CHECK_ARG(rows * (2 * H + 2 * Hi) < (1ll << 31) - 64, "rows x head vectors exceeds the 32-bit index range");
  GlueParams p{};
  p.y = static_cast<const uint16_t*>(y);
  p.ldy = ldy;
  p.q_off = (int)q_off;
  p.k_off = (int)k_off;
  p.iq_off = (int)iq_off;
  p.ik_off = (int)ik_off;
  p.iw_off = (int)iw_off;
  p.H = (int)H;
  p.Hi = (int)Hi;
  p.qn_w = q_norm_w;
  p.qn_b = q_norm_b;
  p.kn_w = k_norm_w;
  p.kn_b = k_norm_b;
  p.ikn_w = idx_k_norm_w;
  p.ikn_b = idx_k_norm_b;
  p.ln_eps = ln_eps;
  p.pos = pos;
  p.rope_cos = rope_cos;
  p.rope_sin = rope_sin;
  p.rope_len = (int)rope_len;
  p.q_out = static_cast<uint16_t*>(q_out);
  p.k_out = static_cast<uint16_t*>(k_out);
  p.iq_out = static_cast<uint16_t*>(idx_q_out);
  p.ik_out = static_cast<uint16_t*>(idx_k_out);
  p.iw_out = static_cast<uint16_t*>(idx_w_out);
  p.rows = rows;
  const int64_t vectors = rows * (2 * H + 2 * Hi);
  const int64_t waves = (vectors + 8 * kGlueVecs - 1) / (8 * kGlueVecs);
  const dim3 grid((unsigned)std::min<int64_t>((waves + 3) / 4, 2048));
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == GW_DTYPE_BF16)
    hipLaunchKernelGGL((dsa_glue_kernel<BF16>), grid, dim3(256), 0, st, p);
  else
    hipLaunchKernelGGL((dsa_glue_kernel<FP16>), grid, dim3(256), 0, st, p);
  GW_HIP_LAUNCH_CHECK("dsa_glue_kernel");
  return GW_OK;
}

extern "C" size_t gw_dsa_glue_bwd_workspace_size(int64_t rows, int64_t H, int64_t Hi) {
  const int64_t vectors = rows * (2 * H + 2 * Hi);
  const int64_t blocks = std::max<int64_t>(1, std::min<int64_t>((vectors + 31) / 32, 2048));
  return (size_t)blocks * 3 * 2 * 64 * sizeof(float);
}

extern "C" int gw_dsa_glue_bwd(int dtype, const void* y, int64_t rows, int64_t ldy, int64_t q_off, int64_t k_off,
                               int64_t iq_off, int64_t ik_off, int64_t iw_off, int64_t H, int64_t Hi, int64_t D,
                               const float* q_norm_w, const float* q_norm_b, const float* k_norm_w,
                               const float* k_norm_b, const float* idx_k_norm_w, const float* idx_k_norm_b,
                               float ln_eps, const int32_t* pos, const float* rope_cos, const float* rope_sin,
                               int64_t rope_len, const void* dq, const void* dk, const void* d_idx_q,
                               const void* d_idx_k, const void* d_idx_w, void* dy, float* d_norm,
                               void* workspace, size_t workspace_bytes, void* stream) {
  using namespace gw;
  clear_error();
  GW_CHECK_ARG(dtype == GW_DTYPE_BF16 || dtype == GW_DTYPE_FP16, "unsupported dtype code %d", dtype);
  if (D != kGlueD) return set_error(GW_ERR_UNSUPPORTED, "head dim %lld not supported (64)", (long long)D);
  GW_CHECK_ARG(rows >= 0 && H >= 1 && Hi >= 0 && H <= 64 && Hi <= 64, "invalid sizes rows=%lld H=%lld Hi=%lld",
               (long long)rows, (long long)H, (long long)Hi);
  GW_CHECK_ARG(d_norm != nullptr, "null d_norm");
  GW_CHECK_ARG(y && dy && dq && dk && (Hi == 0 || (d_idx_q && d_idx_k && d_idx_w)), "null tensor pointer");
  GW_CHECK_ARG(ldy % 8 == 0 && aligned16(y) && aligned16(dy), "rows must be 16-byte aligned (ldy %% 8 == 0)");
  const int64_t offs[4] = {q_off, k_off, iq_off, ik_off};
  const int64_t widths[4] = {H * D, H * D, Hi * D, Hi * D};
  for (int i = 0; i < 4; ++i)
    GW_CHECK_ARG(offs[i] >= 0 && offs[i] % 8 == 0 && offs[i] + widths[i] <= ldy,
                 "column block %d at %lld (+%lld) must be 8-aligned and inside ldy=%lld", i, (long long)offs[i],
                 (long long)widths[i], (long long)ldy);
  GW_CHECK_ARG(iw_off >= 0 && iw_off + Hi <= ldy, "indexer gate columns outside the row");
  GW_CHECK_ARG((q_norm_w == nullptr) == (q_norm_b == nullptr) && (k_norm_w == nullptr) == (k_norm_b == nullptr) &&
                   (idx_k_norm_w == nullptr) == (idx_k_norm_b == nullptr),
               "LayerNorm weight and bias must both be given or both be null");
  GW_CHECK_ARG(pos == nullptr || (rope_cos && rope_sin && rope_len >= 1), "rope tables missing");
  GW_CHECK_ARG(aligned16(dq) && aligned16(dk) && aligned16(d_idx_q) && aligned16(d_idx_k),
               "gradients must be 16-byte aligned");
  GW_CHECK_ARG(rows * (2 * H + 2 * Hi) < (1ll << 31) - 64, "rows x head vectors exceeds the 32-bit index range");
  const size_t need = gw_dsa_glue_bwd_workspace_size(rows, H, Hi);
  GW_CHECK_ARG(workspace && workspace_bytes >= need && aligned16(workspace), "workspace needs %zu bytes", need);
  GlueBwdParams bp{};
  GlueParams& p = bp.f;
  p.y = static_cast<const uint16_t*>(y);
  p.ldy = ldy;
  p.q_off = (int)q_off;
  p.k_off = (int)k_off;
  p.iq_off = (int)iq_off;
  p.ik_off = (int)ik_off;
  p.iw_off = (int)iw_off;
  p.H = (int)H;
  p.Hi = (int)Hi;
  p.qn_w = q_norm_w;
  p.qn_b = q_norm_b;
  p.kn_w = k_norm_w;
  p.kn_b = k_norm_b;
  p.ikn_w = idx_k_norm_w;
  p.ikn_b = idx_k_norm_b;
  p.ln_eps = ln_eps;
  p.pos = pos;
  p.rope_cos = rope_cos;
  p.rope_sin = rope_sin;
  p.rope_len = (int)rope_len;
  p.rows = rows;
  bp.dq = static_cast<const uint16_t*>(dq);
  bp.dk = static_cast<const uint16_t*>(dk);
  bp.diq = static_cast<const uint16_t*>(d_idx_q);
  bp.dik = static_cast<const uint16_t*>(d_idx_k);
  bp.diw = static_cast<const uint16_t*>(d_idx_w);
  bp.dy = static_cast<uint16_t*>(dy);
  bp.ws = static_cast<float*>(workspace);
  const int64_t vectors = rows * (2 * H + 2 * Hi);
  const int nblocks = (int)std::max<int64_t>(1, std::min<int64_t>((vectors + 31) / 32, 2048));
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == GW_DTYPE_BF16)
    hipLaunchKernelGGL((dsa_glue_bwd_kernel<BF16>), dim3(nblocks), dim3(256), 0, st, bp);
  else
    hipLaunchKernelGGL((dsa_glue_bwd_kernel<FP16>), dim3(nblocks), dim3(256), 0, st, bp);
  GW_HIP_LAUNCH_CHECK("dsa_glue_bwd_kernel");
  hipLaunchKernelGGL(dsa_glue_ln_reduce_kernel, dim3(2), dim3(256), 0, st, static_cast<const float*>(workspace),
                     nblocks, d_norm);
  GW_HIP_LAUNCH_CHECK("dsa_glue_ln_reduce_kernel");
  return GW_OK;
}
