// KL(p || softmax(logits)) over the top-k support: the indexer's training loss.
//
// Reference: sparse_indexer_kl_loss / _SparseIndexerKLLossFunc
// (easyvolcap/utils/custom_indexer/indexer_kl_fused.py:158-298, row kernels :8-155) and the
// torch path it replaces (easyvolcap/official_vggt/layers/dsa_attention.py:4688-4715). For
// each of R = B*T rows of K entries (attn = attention mass per selected key, z = the
// indexer's top-k scores, both of one dtype, math in fp32):
//   p_j    = attn_j / (sum_j attn_j + eps)
//   lq_j   = z_j - (max z + log sum_j exp(z_j - max z))
//   loss_r = sum_j p_j * (log(p_j + eps) - lq_j)          (the caller takes the mean)
// Backward with grad_scale = dL/dloss / R:
//   g_j       = log(p_j + eps) - lq_j + p_j / (p_j + eps),   gbar = sum_j p_j g_j
//   dattn_j   = (g_j - gbar) * grad_scale / (sum_j attn_j + eps)
//   dlogits_j = (exp(lq_j) - p_j) * grad_scale
// One wave per row with the row held in registers (K <= 64 * PER), so each direction reads
// attn and z once; dL/dloss is read from device memory, so no host synchronisation.
#include <math.h>

#include "gw_common.h"

namespace gw {
namespace {

constexpr int kKlMaxK = 4096;

__device__ __forceinline__ float load_val(int dt, const void* p, int64_t i) {
  if (dt == GW_DTYPE_FP32) return static_cast<const float*>(p)[i];
  const uint32_t u = static_cast<const uint16_t*>(p)[i];
  if (dt == GW_DTYPE_BF16) return __uint_as_float(u << 16);
  return (float)__builtin_bit_cast(_Float16, (uint16_t)u);
}
__device__ __forceinline__ void store_val(int dt, void* p, int64_t i, float v) {
  if (dt == GW_DTYPE_FP32) {
    static_cast<float*>(p)[i] = v;
    return;
  }
  static_cast<uint16_t*>(p)[i] = (uint16_t)(dt == GW_DTYPE_BF16 ? pack1(BF16{}, v) : pack1(FP16{}, v));
}

// Wave-wide sum and max; every lane receives the result. The four 16-lane partial values
// are combined in a fixed order, so the result does not depend on scheduling.
__device__ __forceinline__ float lane_f(float x, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), l));
}
__device__ __forceinline__ float wave_sum_f(float x) {
  x = group_sum<16>(x);
  return (lane_f(x, 0) + lane_f(x, 16)) + (lane_f(x, 32) + lane_f(x, 48));
}
__device__ __forceinline__ float wave_max_f(float x) {
  x = fmaxf(x, dpp<kDppXor1>(x));
  x = fmaxf(x, dpp<kDppXor2>(x));
  x = fmaxf(x, dpp<kDppHalfMirror>(x));
  x = fmaxf(x, dpp<kDppMirror>(x));
  return fmaxf(fmaxf(lane_f(x, 0), lane_f(x, 16)), fmaxf(lane_f(x, 32), lane_f(x, 48)));
}

struct KlParams {
  const void* attn;
  const void* logits;
  const float* grad_out;  // backward: device scalar dL/dloss
  float* row_loss;        // forward: [R]
  void* d_attn;           // backward: [R, K], dtype dt
  void* d_logits;         // backward: [R, K], dtype dt
  int64_t rows;
  int K;
  int dt;
  float eps;
};

template <int PER, bool BWD>
__global__ __launch_bounds__(256) void indexer_kl_kernel(const KlParams p) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (row >= p.rows) return;
  const int64_t base = row * p.K;
  float a[PER], z[PER];
  float sa = 0.f, zm = -INFINITY;
#pragma unroll
  for (int m = 0; m < PER; ++m) {
    const int j = lane + 64 * m;
    const bool ok = j < p.K;
    a[m] = ok ? load_val(p.dt, p.attn, base + j) : 0.f;
    z[m] = ok ? load_val(p.dt, p.logits, base + j) : -INFINITY;
    sa += a[m];
    zm = fmaxf(zm, z[m]);
  }
  sa = wave_sum_f(sa);
  zm = wave_max_f(zm);
  float se = 0.f;
#pragma unroll
  for (int m = 0; m < PER; ++m) se += (lane + 64 * m < p.K) ? expf(z[m] - zm) : 0.f;
  se = wave_sum_f(se);
  const float lse = zm + logf(se);
  const float denom = sa + p.eps;
  if constexpr (!BWD) {
    float acc = 0.f;
#pragma unroll
    for (int m = 0; m < PER; ++m) {
      if (lane + 64 * m < p.K) {
        const float pj = a[m] / denom;
        acc += pj * (logf(pj + p.eps) - (z[m] - lse));
      }
    }
    acc = wave_sum_f(acc);
    if (lane == 0) p.row_loss[row] = acc;
  } else {
    const float gs = p.grad_out[0] / (float)p.rows;
    float g[PER];
    float gbar = 0.f;
#pragma unroll
    for (int m = 0; m < PER; ++m) {
      const float pj = a[m] / denom;
      g[m] = logf(pj + p.eps) - (z[m] - lse) + pj / (pj + p.eps);
      if (lane + 64 * m < p.K) gbar += pj * g[m];
    }
    gbar = wave_sum_f(gbar);
    const float da_scale = gs / denom;
#pragma unroll
    for (int m = 0; m < PER; ++m) {
      const int j = lane + 64 * m;
      if (j < p.K) {
        const float pj = a[m] / denom;
        store_val(p.dt, p.d_attn, base + j, (g[m] - gbar) * da_scale);
        store_val(p.dt, p.d_logits, base + j, (expf(z[m] - lse) - pj) * gs);
      }
    }
  }
}

template <bool BWD>
int launch_kl(const KlParams& p, hipStream_t st) {
  const dim3 grid((unsigned)((p.rows + 3) / 4));
  const int per = (p.K + 63) / 64;
  if (per <= 2) hipLaunchKernelGGL((indexer_kl_kernel<2, BWD>), grid, dim3(256), 0, st, p);
  else if (per <= 4) hipLaunchKernelGGL((indexer_kl_kernel<4, BWD>), grid, dim3(256), 0, st, p);
  else if (per <= 8) hipLaunchKernelGGL((indexer_kl_kernel<8, BWD>), grid, dim3(256), 0, st, p);
  else if (per <= 16) hipLaunchKernelGGL((indexer_kl_kernel<16, BWD>), grid, dim3(256), 0, st, p);
  else if (per <= 32) hipLaunchKernelGGL((indexer_kl_kernel<32, BWD>), grid, dim3(256), 0, st, p);
  else hipLaunchKernelGGL((indexer_kl_kernel<64, BWD>), grid, dim3(256), 0, st, p);
  GW_HIP_LAUNCH_CHECK("indexer_kl_kernel");
  return GW_OK;
}

int check_kl_args(int dt, const void* attn, const void* logits, int64_t rows, int64_t K) {
  GW_CHECK_ARG(dt == GW_DTYPE_BF16 || dt == GW_DTYPE_FP16 || dt == GW_DTYPE_FP32,
               "unsupported dtype code %d", dt);
  GW_CHECK_ARG(rows >= 0 && K >= 1, "invalid sizes rows=%lld K=%lld", (long long)rows, (long long)K);
  if (K > kKlMaxK)
    return set_error(GW_ERR_UNSUPPORTED, "K=%lld exceeds the supported maximum %d", (long long)K, kKlMaxK);
  GW_CHECK_ARG(rows <= 4ll * 0x7fffffffll, "rows=%lld exceeds the grid limit", (long long)rows);
  GW_CHECK_ARG(rows == 0 || (attn && logits), "null attn_sum or logits pointer");
  return GW_OK;
}

}  // namespace
}  // namespace gw

extern "C" int gw_indexer_kl_fwd(int dtype, const void* attn_sum, const void* logits, int64_t rows, int64_t K,
                                 float eps, float* row_loss, void* stream) {
  using namespace gw;
  clear_error();
  const int rc = check_kl_args(dtype, attn_sum, logits, rows, K);
  if (rc != GW_OK) return rc;
  if (rows == 0) return GW_OK;
  GW_CHECK_ARG(row_loss != nullptr, "null row_loss pointer");
  KlParams p{};
  p.attn = attn_sum;
  p.logits = logits;
  p.row_loss = row_loss;
  p.rows = rows;
  p.K = (int)K;
  p.dt = dtype;
  p.eps = eps;
  return launch_kl<false>(p, static_cast<hipStream_t>(stream));
}

extern "C" int gw_indexer_kl_bwd(int dtype, const void* attn_sum, const void* logits, const float* grad_out,
                                 int64_t rows, int64_t K, float eps, void* d_attn, void* d_logits,
                                 void* stream) {
  using namespace gw;
  clear_error();
  const int rc = check_kl_args(dtype, attn_sum, logits, rows, K);
  if (rc != GW_OK) return rc;
  if (rows == 0) return GW_OK;
  GW_CHECK_ARG(grad_out && d_attn && d_logits, "null gradient pointer");
  KlParams p{};
  p.attn = attn_sum;
  p.logits = logits;
  p.grad_out = grad_out;
  p.d_attn = d_attn;
  p.d_logits = d_logits;
  p.rows = rows;
  p.K = (int)K;
  p.dt = dtype;
  p.eps = eps;
  return launch_kl<true>(p, static_cast<hipStream_t>(stream));
}
