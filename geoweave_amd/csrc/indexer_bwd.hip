// Lightning-indexer backward for gfx950: gradients of the selected top-k scores with
// respect to q, k and w, without float atomics.
//
// Math (reference _indexer_topk_bwd_kernel,
// easyvolcap/utils/custom_indexer/sparse_topk_indexer.py:1847-1944), for each query t,
// head h and selected key s = idx[b,t,j] with upstream gradient g = grad[b,t,j]:
//   z  = scale * q[t,h] . k[s,h]
//   f  = g * w[s,h] * [z > 0] * scale
//   dq[t,h] += f * k[s,h]      dk[s,h] += f * q[t,h]      dw[s,h] += g * relu(z)
// The reference accumulates dk and dw with fp32 atomics (:1936-1941). Here:
//  dq pass  (query-major): one wave per query holds q[t, all heads] and gathers the
//           selected k rows (Hi * 64 elements each) and gates.
//  dkw pass (key-major over the CSR of kv_csr.hip, shared with the attention backward):
//           one wave per work item holds k[s, all heads] and w[s, :], gathers q rows and
//           gradients of the entries, and reduces dk and dw in fp32 in a fixed order.
#include <math.h>

#include "gw_common.h"
#include "gw_csr.h"

namespace gw {
namespace {

constexpr int kDI = 64;

// Tensors other than idx and part are in the element type E of the launch.
struct IdxBwdParams {
  const void* q;       // [B, T, HI, 64]
  const void* k;       // [B, S, HI, 64]
  const void* w;       // [B, S, HI]
  const int32_t* idx;  // [B, T, K]
  const void* grad;    // [B, T, K]
  void* dq;
  void* dk;
  void* dw;
  float* part;  // [parts, HI * 64 + HI]
  CsrView csr;
  int T, S, K;
  float scale;
};

// Lane layout (both passes): HL = HI * 8 lanes hold one token's HI heads (8 lanes x 8
// elements per head); G = 64 / HL entries are processed side by side.
template <typename E, int HI>
__global__ __launch_bounds__(256) void indexer_bwd_dq_kernel(const IdxBwdParams p) {
  constexpr int HL = HI * 8;
  constexpr int G = 64 / HL;
  constexpr int U = 2;  // small blocks: 5+ waves per SIMD for the latency-bound gathers
  constexpr int STEP = U * G;
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int b = blockIdx.y;
  if (t >= p.T) return;
  const int g = lane / HL;
  const int h = (lane % HL) / 8;
  const int c = lane % 8;
  const int64_t row = (int64_t)b * p.T + t;
  const Raw8<E> qv = ld8<E>(p.q, (row * HI + h) * kDI + c * 8);
  const int32_t* irow = p.idx + row * p.K;
  const int64_t grow = row * p.K;
  const int64_t kb = (int64_t)b * p.S * HI * kDI + h * kDI + c * 8;  // element offsets
  const int64_t wb = (int64_t)b * p.S * HI + h;

  float acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = 0.f;

  // Three-stage pipeline: indices (and gradients) two blocks ahead, key rows and gates
  // one block ahead, compute on the current block.
  struct Idx {
    int s;
    float g;
  };
  struct Row {
    Raw8<E> k;
    float gw;  // g * w * scale
  };
  auto load_idx = [&](Idx (&xi)[U], int j0) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int j = j0 + u * G + g;
      const int s = j < p.K ? irow[j] : -1;
      xi[u].s = (s >= 0 && s < p.S) ? s : -1;
      xi[u].g = j < p.K ? ld_f32(E{}, p.grad, grow + j) : 0.f;
    }
  };
  auto load_row = [&](Row (&xr)[U], const Idx (&xi)[U]) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int s = xi[u].s;
      if (s >= 0) {
        xr[u].k = ld8<E>(p.k, kb + (int64_t)s * HI * kDI);
        xr[u].gw = xi[u].g * ld_f32(E{}, p.w, wb + (int64_t)s * HI) * p.scale;
      } else {
        xr[u].k = zero8<E>();
        xr[u].gw = 0.f;
      }
    }
  };
  Idx in[U];
  Row cur[U];
  load_idx(in, 0);
  load_row(cur, in);
  load_idx(in, STEP);
  for (int j0 = 0; j0 < p.K; j0 += STEP) {
    Row nxt[U];
    load_row(nxt, in);
    load_idx(in, j0 + 2 * STEP);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const float z = group_sum<8>(dot8r<E>(qv, cur[u].k)) * p.scale;
      const float f = z > 0.f ? cur[u].gw : 0.f;
      float kf[8];
      up8<E>(cur[u].k, kf);
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[i] = fmaf(f, kf[i], acc[i]);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) cur[u] = nxt[u];
  }
#pragma unroll
  for (int off = HL; off < 64; off <<= 1)
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] += __shfl_xor(acc[i], off);
  if (g == 0) st8<E>(p.dq, (row * HI + h) * kDI + c * 8, acc);
}

template <typename E, int HI>
__global__ __launch_bounds__(256) void indexer_bwd_dkw_kernel(const IdxBwdParams p) {
  constexpr int HL = HI * 8;
  constexpr int G = 64 / HL;
  constexpr int U = 2;  // small blocks: 5+ waves per SIMD for the latency-bound gathers
  constexpr int STEP = U * G;
  const int lane = threadIdx.x & 63;
  const int item = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (item >= p.csr.header[0]) return;
  const CsrItem it = csr_item(p.csr, item);
  const int b = it.key / p.S;
  const int s = it.key - b * p.S;
  const int g = lane / HL;
  const int h = (lane % HL) / 8;
  const int c = lane % 8;
  const int64_t krow = (int64_t)b * p.S + s;
  const Raw8<E> kv = ld8<E>(p.k, (krow * HI + h) * kDI + c * 8);
  const float wsc = ld_f32(E{}, p.w, krow * HI + h) * p.scale;
  const int64_t qb = (int64_t)b * p.T * HI * kDI + h * kDI + c * 8;  // element offsets
  const int64_t gb = (int64_t)b * p.T * p.K;

  float ak[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) ak[i] = 0.f;
  float aw = 0.f;

  struct Slot {
    Raw8<E> q;
    float g;
  };
  auto load = [&](Slot (&sl)[U], int i0) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int i = i0 + u * G + g;
      Slot& x = sl[u];
      if (i < it.end) {
        const int2 e = p.csr.entries[i];
        x.q = ld8<E>(p.q, qb + (int64_t)e.x * HI * kDI);
        x.g = ld_f32(E{}, p.grad, gb + (int64_t)e.x * p.K + e.y);
      } else {
        x.q = zero8<E>();
        x.g = 0.f;
      }
    }
  };
  Slot cur[U];
  load(cur, it.beg);
  for (int i0 = it.beg; i0 < it.end; i0 += STEP) {
    Slot nxt[U];
    load(nxt, i0 + STEP);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const float z = group_sum<8>(dot8r<E>(cur[u].q, kv)) * p.scale;
      const bool on = z > 0.f;
      const float f = on ? cur[u].g * wsc : 0.f;
      aw = on ? fmaf(cur[u].g, z, aw) : aw;
      float qf[8];
      up8<E>(cur[u].q, qf);
#pragma unroll
      for (int i = 0; i < 8; ++i) ak[i] = fmaf(f, qf[i], ak[i]);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) cur[u] = nxt[u];
  }
#pragma unroll
  for (int off = HL; off < 64; off <<= 1) {
#pragma unroll
    for (int i = 0; i < 8; ++i) ak[i] += __shfl_xor(ak[i], off);
    aw += __shfl_xor(aw, off);
  }
  if (g == 0) {
    if (it.nchunk == 1) {
      st8<E>(p.dk, (krow * HI + h) * kDI + c * 8, ak);
      if (c == 0) st_f32(E{}, p.dw, krow * HI + h, aw);
    } else {
      float* pk = p.part + (int64_t)it.part * (HI * kDI + HI);
#pragma unroll
      for (int i = 0; i < 8; i += 4)
        *reinterpret_cast<float4*>(pk + h * kDI + c * 8 + i) = make_float4(ak[i], ak[i + 1], ak[i + 2], ak[i + 3]);
      if (c == 0) pk[HI * kDI + h] = aw;
    }
  }
}

template <typename E, int HI>
__global__ __launch_bounds__(256) void indexer_bwd_reduce_kernel(const IdxBwdParams p) {
  const int key = blockIdx.x;
  const int n = p.csr.item_off[key + 1] - p.csr.item_off[key];
  if (n <= 1) return;
  constexpr int ROW = HI * kDI + HI;
  const int base = p.csr.part_off[key];
  for (int i = threadIdx.x; i < ROW; i += 256) {
    float sum = 0.f;
    for (int c = 0; c < n; ++c) sum += p.part[(int64_t)(base + c) * ROW + i];
    if (i < HI * kDI) st_f32(E{}, p.dk, (int64_t)key * HI * kDI + i, sum);
    else st_f32(E{}, p.dw, (int64_t)key * HI + (i - HI * kDI), sum);
  }
}

template <typename E, int HI>
int launch_idx_bwd(const IdxBwdParams& p, int B, int64_t max_items, hipStream_t st) {
  hipLaunchKernelGGL((indexer_bwd_dq_kernel<E, HI>), dim3((p.T + 3) / 4, B), dim3(256), 0, st, p);
  GW_HIP_LAUNCH_CHECK("indexer_bwd_dq_kernel launch");
  hipLaunchKernelGGL((indexer_bwd_dkw_kernel<E, HI>), dim3((unsigned)((max_items + 3) / 4)), dim3(256), 0, st, p);
  GW_HIP_LAUNCH_CHECK("indexer_bwd_dkw_kernel launch");
  hipLaunchKernelGGL((indexer_bwd_reduce_kernel<E, HI>), dim3(p.csr.nk), dim3(256), 0, st, p);
  GW_HIP_LAUNCH_CHECK("indexer_bwd_reduce_kernel launch");
  return GW_OK;
}

template <typename E>
int dispatch_idx_bwd(int hi, const IdxBwdParams& p, int B, int64_t mi, hipStream_t st) {
  switch (hi) {
    case 1: return launch_idx_bwd<E, 1>(p, B, mi, st);
    case 2: return launch_idx_bwd<E, 2>(p, B, mi, st);
    case 4: return launch_idx_bwd<E, 4>(p, B, mi, st);
    default: return launch_idx_bwd<E, 8>(p, B, mi, st);
  }
}

}  // namespace
}  // namespace gw

extern "C" size_t gw_indexer_topk_bwd_workspace_size(int64_t B, int64_t T, int64_t S, int64_t Hi, int64_t Di,
                                                     int64_t K) {
  if (B <= 0 || T <= 0 || S <= 0 || Hi <= 0 || Di <= 0 || K <= 0) return 256;
  const gw::CsrLayout L = gw::csr_layout(B, T, S, K);
  return (size_t)L.max_parts * (size_t)(Hi * Di + Hi) * 4 + 256;
}

extern "C" int gw_indexer_topk_bwd(int dtype, const void* q, const void* k, const void* w,
                                   const int32_t* topk_indices, const void* grad_scores, void* dq, void* dk,
                                   void* dw, int64_t B, int64_t T, int64_t S, int64_t Hi, int64_t Di, int64_t K,
                                   float softmax_scale, const void* csr, size_t csr_bytes, void* workspace,
                                   size_t workspace_bytes, void* stream) {
  using namespace gw;
  clear_error();
  GW_CHECK_ARG(dtype == GW_DTYPE_BF16 || dtype == GW_DTYPE_FP16 || dtype == GW_DTYPE_FP32, "unsupported dtype code %d",
               dtype);
  GW_CHECK_ARG(B >= 0 && T >= 0 && S >= 0 && K >= 0, "invalid sizes B=%lld T=%lld S=%lld K=%lld", (long long)B,
               (long long)T, (long long)S, (long long)K);
  if (Di != kDI || !(Hi == 1 || Hi == 2 || Hi == 4 || Hi == 8))
    return set_error(GW_ERR_UNSUPPORTED, "indexer heads x dim %lld x %lld not supported (1/2/4/8 x 64)",
                     (long long)Hi, (long long)Di);
  if (B == 0 || T == 0 || S == 0) return GW_OK;
  GW_CHECK_ARG(K >= 1, "empty top-k table");
  GW_CHECK_ARG(q && k && w && topk_indices && grad_scores && dq && dk && dw, "null tensor pointer");
  GW_CHECK_ARG(aligned16(q) && aligned16(k) && aligned16(dq) && aligned16(dk), "q/k/dq/dk must be 16-byte aligned");
  GW_CHECK_ARG(B <= 65535 && T < (1ll << 31), "size exceeds grid or int32 range");
  GW_CHECK_ARG(csr != nullptr && csr_bytes >= gw_kv_csr_size(B, T, S, K),
               "csr buffer needs %zu bytes (built by gw_kv_csr_build), got %zu", gw_kv_csr_size(B, T, S, K),
               csr_bytes);
  const size_t need = gw_indexer_topk_bwd_workspace_size(B, T, S, Hi, Di, K);
  GW_CHECK_ARG(workspace != nullptr && aligned16(workspace) && workspace_bytes >= need,
               "workspace needs %zu bytes (16-byte aligned), got %zu", need, workspace_bytes);
  GW_CHECK_ARG(softmax_scale > 0.f, "softmax_scale must be positive");
  const CsrLayout L = csr_layout(B, T, S, K);
  IdxBwdParams p{};
  p.q = q;
  p.k = k;
  p.w = w;
  p.idx = topk_indices;
  p.grad = grad_scores;
  p.dq = dq;
  p.dk = dk;
  p.dw = dw;
  p.part = static_cast<float*>(workspace);
  p.csr = csr_view(csr, L);
  p.T = (int)T;
  p.S = (int)S;
  p.K = (int)K;
  p.scale = softmax_scale;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == GW_DTYPE_BF16) return dispatch_idx_bwd<BF16>((int)Hi, p, (int)B, L.max_items, st);
  if (dtype == GW_DTYPE_FP32) return dispatch_idx_bwd<FP32>((int)Hi, p, (int)B, L.max_items, st);
  return dispatch_idx_bwd<FP16>((int)Hi, p, (int)B, L.max_items, st);
}

// ---------------------------------------------------------------------------------------
// Soft view-bias gradient, per query row (reference _scatter_view_bias_grad,
// sparse_topk_indexer.py:898-932: grad_view_bias[b, q_view[t], s_view[idx[b,t,j]]] +=
// grad_scores[b,t,j] in fp32). This pass writes the row sums over key views,
// part[b, t, v] = sum_{j : s_view[idx[b,t,j]] == v} grad[b,t,j]; the host groups the rows
// by query view (a one-hot product). One wave per row: lane l adds entries l, l + 64, ...
// into its own LDS histogram, then bin v sums the 64 histograms in lane order — a fixed
// order, no atomics. Positions outside [0, S) contribute nothing.
namespace gw {
namespace {

constexpr int kViewChunk = 128;  // key-view bins per pass (a 32 KB LDS histogram set)

// View ids are clamped into the table (the host checks their range).
__device__ __forceinline__ int clamp_bin(int v, int n) { return v < 0 ? 0 : (v >= n ? n - 1 : v); }

template <typename E>
__global__ __launch_bounds__(64) void view_bias_rows_kernel(const int32_t* __restrict__ idx,
                                                            const void* __restrict__ grad,
                                                            const int32_t* __restrict__ sview, int T, int S,
                                                            int K, int Vs, float* __restrict__ part) {
  __shared__ float hist[64 * kViewChunk];  // [lane][bin of the current chunk]
  const int lane = threadIdx.x;
  const int64_t row = blockIdx.x;  // b * T + t
  const int b = (int)(row / T);
  float* mine = hist + lane * kViewChunk;
  const int32_t* ir = idx + row * K;
  const int64_t gr = row * K;
  const int32_t* sv = sview + (int64_t)b * S;
  for (int v0 = 0; v0 < Vs; v0 += kViewChunk) {
    const int nb = min(kViewChunk, Vs - v0);
    for (int v = 0; v < nb; ++v) mine[v] = 0.f;
    for (int j = lane; j < K; j += 64) {
      const int s = ir[j];
      if (s >= 0 && s < S) {
        const int v = clamp_bin(sv[s], Vs) - v0;
        if (v >= 0 && v < nb) mine[v] += ld_f32(E{}, grad, gr + j);
      }
    }
    __syncthreads();
    for (int v = lane; v < nb; v += 64) {
      float acc = 0.f;
      for (int l = 0; l < 64; ++l) acc += hist[l * kViewChunk + v];
      part[row * Vs + v0 + v] = acc;
    }
    __syncthreads();
  }
}

}  // namespace
}  // namespace gw

extern "C" int gw_indexer_view_bias_bwd_rows(int dtype, const int32_t* topk_indices, const void* grad_scores,
                                             const int32_t* s_view_ids, int64_t B, int64_t T, int64_t S,
                                             int64_t K, int64_t Vs, float* row_grad, void* stream) {
  using namespace gw;
  clear_error();
  GW_CHECK_ARG(dtype == GW_DTYPE_BF16 || dtype == GW_DTYPE_FP16 || dtype == GW_DTYPE_FP32, "unsupported dtype code %d",
               dtype);
  GW_CHECK_ARG(B >= 0 && T >= 0 && S >= 1 && K >= 0, "invalid sizes B=%lld T=%lld S=%lld K=%lld", (long long)B,
               (long long)T, (long long)S, (long long)K);
  GW_CHECK_ARG(Vs >= 1 && Vs < (1ll << 20), "invalid key view count %lld", (long long)Vs);
  if (B * T == 0) return GW_OK;
  GW_CHECK_ARG(topk_indices && grad_scores && s_view_ids && row_grad, "null tensor pointer");
  GW_CHECK_ARG(B * T < (1ll << 31) && S < (1ll << 31) && K < (1ll << 31), "size exceeds the int32 range");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == GW_DTYPE_BF16)
    hipLaunchKernelGGL(view_bias_rows_kernel<BF16>, dim3((unsigned)(B * T)), dim3(64), 0, st, topk_indices,
                       grad_scores, s_view_ids, (int)T, (int)S, (int)K, (int)Vs, row_grad);
  else if (dtype == GW_DTYPE_FP32)
    hipLaunchKernelGGL(view_bias_rows_kernel<FP32>, dim3((unsigned)(B * T)), dim3(64), 0, st, topk_indices,
                       grad_scores, s_view_ids, (int)T, (int)S, (int)K, (int)Vs, row_grad);
  else
    hipLaunchKernelGGL(view_bias_rows_kernel<FP16>, dim3((unsigned)(B * T)), dim3(64), 0, st, topk_indices,
                       grad_scores, s_view_ids, (int)T, (int)S, (int)K, (int)Vs, row_grad);
  GW_HIP_LAUNCH_CHECK("view_bias_rows_kernel");
  return GW_OK;
}
