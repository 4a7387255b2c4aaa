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
