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
// One thread per (row, head vector); the whole vector lives in registers.
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

__device__ __forceinline__ void layer_norm64(float (&x)[kGlueD], const float* g, const float* bta, float eps) {
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < kGlueD; ++i) s += x[i];
  const float mean = s * (1.f / kGlueD);
  float v = 0.f;
#pragma unroll
  for (int i = 0; i < kGlueD; ++i) {
    const float d = x[i] - mean;
    v += d * d;
  }
  const float rstd = 1.f / sqrtf(v * (1.f / kGlueD) + eps);
#pragma unroll
  for (int i = 0; i < kGlueD; ++i) x[i] = (x[i] - mean) * rstd * g[i] + bta[i];
}

__device__ __forceinline__ void rope_half(float (&x)[kGlueD], int base, const float* c, const float* s) {
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const float a = x[base + i], bb = x[base + 16 + i];
    x[base + i] = a * c[i] - bb * s[i];
    x[base + 16 + i] = bb * c[i] + a * s[i];
  }
}

template <typename E>
__global__ __launch_bounds__(256) void dsa_glue_kernel(const GlueParams p) {
  const int slots = 2 * p.H + 2 * p.Hi;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= p.rows * slots) return;
  const int64_t row = gid / slots;
  const int slot = (int)(gid - row * slots);

  int col, head;
  const float* g = nullptr;
  const float* bta = nullptr;
  uint16_t* out;
  int out_heads;
  if (slot < p.H) {
    head = slot;
    col = p.q_off + head * kGlueD;
    g = p.qn_w;
    bta = p.qn_b;
    out = p.q_out;
    out_heads = p.H;
  } else if (slot < 2 * p.H) {
    head = slot - p.H;
    col = p.k_off + head * kGlueD;
    g = p.kn_w;
    bta = p.kn_b;
    out = p.k_out;
    out_heads = p.H;
  } else if (slot < 2 * p.H + p.Hi) {
    head = slot - 2 * p.H;
    col = p.iq_off + head * kGlueD;
    out = p.iq_out;
    out_heads = p.Hi;
    // The indexer gate of this head travels with its query vector.
    p.iw_out[row * p.Hi + head] = p.y[row * p.ldy + p.iw_off + head];
  } else {
    head = slot - 2 * p.H - p.Hi;
    col = p.ik_off + head * kGlueD;
    g = p.ikn_w;
    bta = p.ikn_b;
    out = p.ik_out;
    out_heads = p.Hi;
  }

  const uint4* src = reinterpret_cast<const uint4*>(p.y + row * p.ldy + col);
  float x[kGlueD];
#pragma unroll
  for (int c = 0; c < kGlueD / 8; ++c) unpack8<E>(src[c], x + 8 * c);
  if (g != nullptr) layer_norm64(x, g, bta, p.ln_eps);
  if (p.pos != nullptr) {
    const int py = min(max(p.pos[row * 2 + 0], 0), p.rope_len - 1);
    const int px = min(max(p.pos[row * 2 + 1], 0), p.rope_len - 1);
    rope_half(x, 0, p.rope_cos + py * 16, p.rope_sin + py * 16);
    rope_half(x, 32, p.rope_cos + px * 16, p.rope_sin + px * 16);
  }
  uint4* dst = reinterpret_cast<uint4*>(out + (row * out_heads + head) * kGlueD);
#pragma unroll
  for (int c = 0; c < kGlueD / 8; ++c) dst[c] = pack8<E>(x + 8 * c);
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
  GW_CHECK_ARG(rows >= 0 && H >= 1 && Hi >= 1 && H <= 64 && Hi <= 64, "invalid sizes rows=%lld H=%lld Hi=%lld",
               (long long)rows, (long long)H, (long long)Hi);
  if (rows == 0) return GW_OK;
  GW_CHECK_ARG(y && q_out && k_out && idx_q_out && idx_k_out && idx_w_out, "null tensor pointer");
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
               "outputs must be 16-byte aligned");
  GW_CHECK_ARG(rows * (2 * H + 2 * Hi) / 256 < (1ll << 31) - 1, "too many rows for one launch");
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
  const int64_t threads = rows * (2 * H + 2 * Hi);
  const dim3 grid((unsigned)((threads + 255) / 256));
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == GW_DTYPE_BF16)
    hipLaunchKernelGGL((dsa_glue_kernel<BF16>), grid, dim3(256), 0, st, p);
  else
    hipLaunchKernelGGL((dsa_glue_kernel<FP16>), grid, dim3(256), 0, st, p);
  GW_HIP_LAUNCH_CHECK("dsa_glue_kernel");
  return GW_OK;
}
