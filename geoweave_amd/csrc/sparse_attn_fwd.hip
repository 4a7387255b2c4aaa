// Sparse-index attention forward for gfx950.
//
// Work decomposition: one wave per (query t, group of HPW heads). A lane owns one
// (key group g, head hh, 8-element slice c of the head dim); LPH = D/8 lanes cover one
// head row, HL = HPW*LPH lanes one head group, G = 64/HL key groups run in parallel when
// a head group is narrower than the wave. Because the reference shares kv_positions
// across heads (sparse_index_flash_attn.py:196-197), a wave reads, for every selected key,
// HPW contiguous head rows of K and of V: for D = 64 and HPW = 8 that is 1 KB of K and
// 1 KB of V per key in 16-byte, fully coalesced lane loads.
//
// Scores use v_dot2_f32_{bf16,f16} (exact products, fp32 accumulation) and a DPP
// reduction over the LPH lanes of a head. Softmax runs online in the log2 domain in fp32
// over blocks of U keys; loads of block i+1 are issued before block i is consumed.
//
// attn_sum (optional, training only in the reference): the scaled score of every
// (key, head) is written to a workspace during the pass; after the pass the workgroup,
// which holds every head of its queries, sums exp2(s - lse2) over heads for each key and
// writes attn_sum once. This replaces the reference's second K gather + per-head atomics
// (_attn_sum_kernel, sparse_index_flash_attn.py:375-458) with 2 * K * H * 4 bytes of
// workspace traffic per query.
//
// Indexer KL loss fused into that epilogue (optional, training): with the query's attn_sum
// row still in registers, the workgroup also reads the row's indexer logits z (the top-k
// scores) and writes row_loss = KL(p || softmax(z)), p = attn_sum / (sum attn_sum + eps),
// the per-row term of sparse_indexer_kl_loss (indexer_kl_fused.py:8-155): one pass for
// sum(attn_sum) and max(z), one for sum exp(z - max z), one for the terms, each reduced over
// the query's head-group waves in a fixed order.
#include <math.h>

#include "gw_attn.h"
#include "gw_common.h"

namespace gw {
namespace {

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

struct AttnFwdParams {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const int32_t* pos;
  uint16_t* o;
  float* lse;
  float* attn_sum;
  float* ws;
  int64_t qsb, qst, qsh;
  int64_t ksb, kss, ksh;
  int64_t vsb, vss, vsh;
  int64_t osb, ost, osh;
  int64_t psb, pst;
  // fused KL (KL kernels only)
  const void* logits;
  int logits_dt;  // GW_DTYPE_*
  int64_t lsb, lst;
  float kl_eps;
  float* row_loss;
  // Optional: run only the 32-query blocks flagged here ([B][nqb][nchunk]), and every block
  // of a batch element whose batch_flags[b] is non-zero (nullable).
  const int* blk_flags;
  const int* batch_flags;
  int nqb, nchunk;
  int T, S, H, K;
  int NG;   // head groups (waves) per query
  int QPB;  // queries per workgroup
  float scale_log2;
};

constexpr int kMaxHeadsLds = 64;
constexpr int kMaxQpb = 4;
constexpr int kKlRegs = 16;  // attn_sum entries per thread held for the fused KL

__device__ __forceinline__ float kl_lane(float x, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), l));
}
__device__ __forceinline__ float kl_wave_sum(float x) {
  x = group_sum<16>(x);
  return (kl_lane(x, 0) + kl_lane(x, 16)) + (kl_lane(x, 32) + kl_lane(x, 48));
}
__device__ __forceinline__ float kl_wave_max(float x) {
  x = fmaxf(x, dpp<kDppXor1>(x));
  x = fmaxf(x, dpp<kDppXor2>(x));
  x = fmaxf(x, dpp<kDppHalfMirror>(x));
  x = fmaxf(x, dpp<kDppMirror>(x));
  return fmaxf(fmaxf(kl_lane(x, 0), kl_lane(x, 16)), fmaxf(kl_lane(x, 32), kl_lane(x, 48)));
}
__device__ __forceinline__ float kl_load(int dt, const void* base, int64_t i) {
  if (dt == GW_DTYPE_FP32) return static_cast<const float*>(base)[i];
  const uint32_t u = static_cast<const uint16_t*>(base)[i];
  if (dt == GW_DTYPE_BF16) return __uint_as_float(u << 16);
  return (float)__builtin_bit_cast(_Float16, (uint16_t)u);
}

template <typename E, int D, int HPW, bool ATTN, bool KL>
__global__ __launch_bounds__(256) void sparse_attn_fwd_kernel(const AttnFwdParams p) {
  static_assert(ATTN || !KL, "the fused KL needs attn_sum");
  constexpr int LPH = D / 8;
  constexpr int HL = HPW * LPH;
  constexpr int G = 64 / HL;
  constexpr int U = 8;           // keys per lane per block
  constexpr int STEP = U * G;    // keys per wave per block
  static_assert(HL * G == 64, "lane decomposition must cover one wave");

  __shared__ float lse2_s[kMaxQpb][kMaxHeadsLds];

  if (p.blk_flags != nullptr) {
    // All QPB (1, 2 or 4) queries of a workgroup sit in one 32-query block: the test is
    // uniform over the workgroup.
    const int qb = (int)((blockIdx.x * p.QPB) >> 5);
    const int* f = p.blk_flags + ((int64_t)blockIdx.y * p.nqb + qb) * p.nchunk;
    bool run = p.batch_flags != nullptr && p.batch_flags[blockIdx.y] != 0;
    for (int c = 0; c < p.nchunk; ++c) run |= f[c] != 0;
    if (!run) return;
  }

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int ql = wave / p.NG;
  const int hg = wave - ql * p.NG;
  const int t = blockIdx.x * p.QPB + ql;
  const int b = blockIdx.y;
  const int g = lane / HL;
  const int hh = (lane % HL) / LPH;
  const int c = lane % LPH;
  const int h = hg * HPW + hh;
  const bool head_ok = h < p.H;
  const bool t_ok = t < p.T;

  float m = -INFINITY, l = 0.f;
  float acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = 0.f;

  if (t_ok) {
    const uint16_t* kb = p.k + b * p.ksb + h * p.ksh + c * 8;
    const uint16_t* vb = p.v + b * p.vsb + h * p.vsh + c * 8;
    const int32_t* prow = p.pos + b * p.psb + (int64_t)t * p.pst;
    uint4 qv = make_uint4(0, 0, 0, 0);
    if (head_ok) qv = *reinterpret_cast<const uint4*>(p.q + b * p.qsb + (int64_t)t * p.qst + h * p.qsh + c * 8);
    float* wsrow = nullptr;
    if constexpr (ATTN) wsrow = p.ws + ((int64_t)b * p.T + t) * (int64_t)p.K * p.H + h;

    auto load_pos = [&](int (&pp)[U], int j0) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int j = j0 + u * G + g;
        pp[u] = (j < p.K) ? prow[j] : -1;
      }
    };
    auto load_kv = [&](uint4 (&kk)[U], uint4 (&vv)[U], const int (&pp)[U]) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int s = pp[u];
        if (head_ok && s >= 0 && s < p.S) {
          kk[u] = *reinterpret_cast<const uint4*>(kb + (int64_t)s * p.kss);
          vv[u] = *reinterpret_cast<const uint4*>(vb + (int64_t)s * p.vss);
        } else {
          kk[u] = make_uint4(0, 0, 0, 0);
          vv[u] = make_uint4(0, 0, 0, 0);
        }
      }
    };

    int pc[U], pn[U];
    uint4 kc[U], vc[U];
    load_pos(pc, 0);
    load_kv(kc, vc, pc);
    load_pos(pn, STEP);

    for (int j0 = 0; j0 < p.K; j0 += STEP) {
      uint4 kn[U], vn[U];
      int pnn[U];
      load_kv(kn, vn, pn);       // block i+1 (all-invalid past the end: no traffic)
      load_pos(pnn, j0 + 2 * STEP);

      float s2[U];
      float mb = -INFINITY;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        float d = group_sum<LPH>(dot8<E>(qv, kc[u]));
        const bool valid = pc[u] >= 0 && pc[u] < p.S;
        s2[u] = valid ? d * p.scale_log2 : -INFINITY;
        mb = fmaxf(mb, s2[u]);
        if constexpr (ATTN) {
          const int j = j0 + u * G + g;
          if (c == 0 && head_ok && j < p.K) wsrow[(int64_t)j * p.H] = s2[u];
        }
      }
      const float mn = fmaxf(m, mb);
      const float mref = (mn == -INFINITY) ? 0.f : mn;
      const float alpha = fexp2(m - mref);
      l *= alpha;
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[i] *= alpha;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const float pj = fexp2(s2[u] - mref);
        l += pj;
        float vf[8];
        unpack8<E>(vc[u], vf);
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[i] = fmaf(pj, vf[i], acc[i]);
      }
      m = mn;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        kc[u] = kn[u];
        vc[u] = vn[u];
        pc[u] = pn[u];
        pn[u] = pnn[u];
      }
    }

    // Merge the G key groups (lanes HL apart hold the same head slice).
#pragma unroll
    for (int off = HL; off < 64; off <<= 1) {
      const float mo = __shfl_xor(m, off);
      const float lo = __shfl_xor(l, off);
      const float mn = fmaxf(m, mo);
      const float mref = (mn == -INFINITY) ? 0.f : mn;
      const float a = fexp2(m - mref), bo = fexp2(mo - mref);
      l = l * a + lo * bo;
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[i] = acc[i] * a + __shfl_xor(acc[i], off) * bo;
      m = mn;
    }

    const float inv = l > 0.f ? 1.f / l : 0.f;
    if (g == 0 && head_ok) {
      float of[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) of[i] = acc[i] * inv;
      *reinterpret_cast<uint4*>(p.o + b * p.osb + (int64_t)t * p.ost + h * p.osh + c * 8) = pack8<E>(of);
      // l = 0: no valid entry (lse = -inf); a nan l (an inf or nan score of a selected
      // key) gives a nan lse, as the reference's m + log(l) does
      const float lse2 = l != 0.f ? m + flog2(l) : -INFINITY;
      if (c == 0) {
        if (p.lse) p.lse[((int64_t)b * p.T + t) * p.H + h] = lse2 * kLn2;
        if constexpr (ATTN) lse2_s[ql][h] = lse2;
      }
    }
  }

  if constexpr (ATTN && !KL) {
    __threadfence_block();
    __syncthreads();
    if (t_ok) {
      const int nthr = p.NG * 64;
      const int lid = hg * 64 + lane;
      const float* wsq = p.ws + ((int64_t)b * p.T + t) * (int64_t)p.K * p.H;
      float* out = p.attn_sum + ((int64_t)b * p.T + t) * (int64_t)p.K;
      for (int j = lid; j < p.K; j += nthr) {
        const float* srow = wsq + (int64_t)j * p.H;
        float sum = 0.f;
        for (int hx = 0; hx < p.H; ++hx) {
          const float l2 = lse2_s[ql][hx];
          if (l2 != -INFINITY) sum += fexp2(srow[hx] - l2);
        }
        out[j] = sum;
      }
    }
  }
  if constexpr (KL) {
    // attn_sum as above, entry j = lid + r * nthr held in av[r] (the host checks
    // K <= kKlRegs * nthr), then the KL row loss. Barriers are reached by every thread.
    __shared__ float kl_red[kMaxQpb][4][2];
    __threadfence_block();
    __syncthreads();
    const int nthr = p.NG * 64;
    const int lid = hg * 64 + lane;
    float av[kKlRegs], zv[kKlRegs];
    float sa = 0.f, mz = -INFINITY;
#pragma unroll
    for (int r = 0; r < kKlRegs; ++r) {
      av[r] = 0.f;
      zv[r] = -INFINITY;
      const int j = lid + r * nthr;
      if (t_ok && j < p.K) {
        const float* srow = p.ws + (((int64_t)b * p.T + t) * (int64_t)p.K + j) * p.H;
        float sum = 0.f;
        for (int hx = 0; hx < p.H; ++hx) {
          const float l2 = lse2_s[ql][hx];
          if (l2 != -INFINITY) sum += fexp2(srow[hx] - l2);
        }
        p.attn_sum[((int64_t)b * p.T + t) * (int64_t)p.K + j] = sum;
        av[r] = sum;
        zv[r] = kl_load(p.logits_dt, p.logits, b * p.lsb + (int64_t)t * p.lst + j);
        sa += sum;
        mz = fmaxf(mz, zv[r]);
      }
    }
    sa = kl_wave_sum(sa);
    mz = kl_wave_max(mz);
    if (lane == 0) {
      kl_red[ql][hg][0] = sa;
      kl_red[ql][hg][1] = mz;
    }
    __syncthreads();
    float sa_t = 0.f, mz_t = -INFINITY;
    for (int g2 = 0; g2 < p.NG; ++g2) {
      sa_t += kl_red[ql][g2][0];
      mz_t = fmaxf(mz_t, kl_red[ql][g2][1]);
    }
    const float denom = sa_t + p.kl_eps;
    float se = 0.f;
#pragma unroll
    for (int r = 0; r < kKlRegs; ++r) {
      if (t_ok && lid + r * nthr < p.K) se += expf(zv[r] - mz_t);
    }
    se = kl_wave_sum(se);
    __syncthreads();  // every wave has read kl_red
    if (lane == 0) kl_red[ql][hg][0] = se;
    __syncthreads();
    float se_t = 0.f;
    for (int g2 = 0; g2 < p.NG; ++g2) se_t += kl_red[ql][g2][0];
    const float lse = mz_t + logf(se_t);
    float acc = 0.f;
#pragma unroll
    for (int r = 0; r < kKlRegs; ++r) {
      if (t_ok && lid + r * nthr < p.K) {
        const float pj = av[r] / denom;
        acc += pj * (logf(pj + p.kl_eps) - (zv[r] - lse));
      }
    }
    acc = kl_wave_sum(acc);
    __syncthreads();
    if (lane == 0) kl_red[ql][hg][0] = acc;
    __syncthreads();
    if (t_ok && lid == 0) {
      float loss = 0.f;
      for (int g2 = 0; g2 < p.NG; ++g2) loss += kl_red[ql][g2][0];
      p.row_loss[(int64_t)b * p.T + t] = loss;
    }
  }
}

template <typename E, int D, int HPW>
int launch_typed(const AttnFwdParams& p, int B, bool attn, hipStream_t stream) {
  dim3 grid((p.T + p.QPB - 1) / p.QPB, B);
  dim3 block(64 * p.NG * p.QPB);
  if (p.row_loss)
    hipLaunchKernelGGL((sparse_attn_fwd_kernel<E, D, HPW, true, true>), grid, block, 0, stream, p);
  else if (attn)
    hipLaunchKernelGGL((sparse_attn_fwd_kernel<E, D, HPW, true, false>), grid, block, 0, stream, p);
  else
    hipLaunchKernelGGL((sparse_attn_fwd_kernel<E, D, HPW, false, false>), grid, block, 0, stream, p);
  GW_HIP_LAUNCH_CHECK("sparse_attn_fwd_kernel launch");
  return GW_OK;
}

template <typename E>
int dispatch_d(const AttnFwdParams& p, int B, int D, int hpw, bool attn, hipStream_t stream) {
  if (D == 64) {
    switch (hpw) {
      case 1: return launch_typed<E, 64, 1>(p, B, attn, stream);
      case 2: return launch_typed<E, 64, 2>(p, B, attn, stream);
      case 4: return launch_typed<E, 64, 4>(p, B, attn, stream);
      default: return launch_typed<E, 64, 8>(p, B, attn, stream);
    }
  }
  switch (hpw) {
    case 1: return launch_typed<E, 128, 1>(p, B, attn, stream);
    case 2: return launch_typed<E, 128, 2>(p, B, attn, stream);
    default: return launch_typed<E, 128, 4>(p, B, attn, stream);
  }
}

int pow2_ceil(int x) {
  int r = 1;
  while (r < x) r <<= 1;
  return r;
}

}  // namespace
}  // namespace gw

extern "C" size_t gw_sparse_attn_fwd_workspace_size(int64_t B, int64_t T, int64_t H, int64_t K,
                                                    int want_attn_sum) {
  if (!want_attn_sum || B <= 0 || T <= 0 || H <= 0 || K <= 0) return 0;
  return (size_t)B * (size_t)T * (size_t)K * (size_t)H * sizeof(float);
}

namespace gw {
namespace {

struct KlArgs {
  const void* logits;
  int dtype;
  int64_t stride_b, stride_t;
  float eps;
  float* row_loss;
};

int attn_fwd_impl(int dtype, const void* q, const int64_t* q_strides, const void* k, const int64_t* k_strides,
                  const void* v, const int64_t* v_strides, const int32_t* kv_pos, int64_t pos_stride_b,
                  int64_t pos_stride_t, void* o, const int64_t* o_strides, float* lse, float* attn_sum, int64_t B,
                  int64_t T, int64_t S, int64_t H, int64_t D, int64_t K, float softmax_scale, void* workspace,
                  size_t workspace_bytes, const KlArgs* kl, void* stream, const int* blk_flags = nullptr,
                  const int* batch_flags = nullptr, int nqb = 0, int nchunk = 0) {
  GW_CHECK_ARG(dtype == GW_DTYPE_BF16 || dtype == GW_DTYPE_FP16, "unsupported dtype code %d", dtype);
  GW_CHECK_ARG(B >= 0 && T >= 0 && S >= 0 && H >= 1 && K >= 0,
               "invalid sizes B=%lld T=%lld S=%lld H=%lld K=%lld", (long long)B, (long long)T,
               (long long)S, (long long)H, (long long)K);
  if (D != 64 && D != 128)
    return set_error(GW_ERR_UNSUPPORTED, "head dim %lld not supported (64 or 128)", (long long)D);
  GW_CHECK_ARG(H <= kMaxHeadsLds, "at most %d heads supported, got %lld", kMaxHeadsLds, (long long)H);
  if (B == 0 || T == 0) return GW_OK;
  GW_CHECK_ARG(K >= 1, "kv_positions must have at least one candidate");
  GW_CHECK_ARG(q && k && v && kv_pos && o, "null tensor pointer");
  GW_CHECK_ARG(q_strides && k_strides && v_strides && o_strides, "null stride array");
  GW_CHECK_ARG(aligned16(q) && aligned16(k) && aligned16(v) && aligned16(o),
               "q/k/v/o must be 16-byte aligned");
  for (int i = 0; i < 3; ++i) {
    GW_CHECK_ARG(q_strides[i] % 8 == 0 && k_strides[i] % 8 == 0 && v_strides[i] % 8 == 0 &&
                     o_strides[i] % 8 == 0,
                 "b/t/h strides must be multiples of 8 elements");
  }
  GW_CHECK_ARG(B <= 65535, "batch %lld exceeds grid limit", (long long)B);
  GW_CHECK_ARG(T < (1ll << 31) && S < (1ll << 31) && K < (1ll << 31), "size exceeds int32 range");
  const bool want_attn = attn_sum != nullptr;
  if (want_attn) {
    const size_t need = gw_sparse_attn_fwd_workspace_size(B, T, H, K, 1);
    GW_CHECK_ARG(workspace != nullptr && workspace_bytes >= need,
                 "attn_sum needs a %zu-byte workspace, got %zu", need, workspace_bytes);
  }

  const int lph = (int)D / 8;
  const int hpw_max = 64 / lph;
  const int hpw = pow2_ceil((int)H) < hpw_max ? pow2_ceil((int)H) : hpw_max;
  AttnFwdParams p;
  p.q = static_cast<const uint16_t*>(q);
  p.k = static_cast<const uint16_t*>(k);
  p.v = static_cast<const uint16_t*>(v);
  p.pos = kv_pos;
  p.o = static_cast<uint16_t*>(o);
  p.lse = lse;
  p.attn_sum = attn_sum;
  p.ws = static_cast<float*>(workspace);
  p.qsb = q_strides[0]; p.qst = q_strides[1]; p.qsh = q_strides[2];
  p.ksb = k_strides[0]; p.kss = k_strides[1]; p.ksh = k_strides[2];
  p.vsb = v_strides[0]; p.vss = v_strides[1]; p.vsh = v_strides[2];
  p.osb = o_strides[0]; p.ost = o_strides[1]; p.osh = o_strides[2];
  p.psb = pos_stride_b;
  p.pst = pos_stride_t;
  p.logits = nullptr;
  p.logits_dt = GW_DTYPE_FP32;
  p.lsb = p.lst = 0;
  p.kl_eps = 0.f;
  p.row_loss = nullptr;
  p.blk_flags = blk_flags;
  p.batch_flags = batch_flags;
  p.nqb = nqb;
  p.nchunk = nchunk;
  p.T = (int)T;
  p.S = (int)S;
  p.H = (int)H;
  p.K = (int)K;
  p.NG = (int)((H + hpw - 1) / hpw);
  GW_CHECK_ARG(p.NG <= 4, "too many head groups (%d) for one workgroup", p.NG);
  p.QPB = 4 / p.NG;
  if (p.QPB < 1) p.QPB = 1;
  p.scale_log2 = softmax_scale * kLog2e;
  if (kl != nullptr) {
    GW_CHECK_ARG(want_attn, "the fused KL loss needs attn_sum");
    GW_CHECK_ARG(kl->logits != nullptr && kl->row_loss != nullptr, "null logits or row_loss pointer");
    GW_CHECK_ARG(kl->dtype == GW_DTYPE_BF16 || kl->dtype == GW_DTYPE_FP16 || kl->dtype == GW_DTYPE_FP32,
                 "unsupported logits dtype code %d", kl->dtype);
    GW_CHECK_ARG(kl->eps >= 0.f, "eps must be non-negative, got %g", (double)kl->eps);
    if (K > (int64_t)kKlRegs * p.NG * 64)
      return set_error(GW_ERR_UNSUPPORTED, "fused KL supports K <= %d for %lld heads, got %lld",
                       kKlRegs * p.NG * 64, (long long)H, (long long)K);
    p.logits = kl->logits;
    p.logits_dt = kl->dtype;
    p.lsb = kl->stride_b;
    p.lst = kl->stride_t;
    p.kl_eps = kl->eps;
    p.row_loss = kl->row_loss;
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == GW_DTYPE_BF16) return dispatch_d<BF16>(p, (int)B, (int)D, hpw, want_attn, st);
  return dispatch_d<FP16>(p, (int)B, (int)D, hpw, want_attn, st);
}

}  // namespace
}  // namespace gw

extern "C" int gw_sparse_attn_fwd(int dtype, const void* q, const int64_t* q_strides,
                                  const void* k, const int64_t* k_strides, const void* v,
                                  const int64_t* v_strides, const int32_t* kv_pos,
                                  int64_t pos_stride_b, int64_t pos_stride_t, void* o,
                                  const int64_t* o_strides, float* lse, float* attn_sum,
                                  int64_t B, int64_t T, int64_t S, int64_t H, int64_t D,
                                  int64_t K, float softmax_scale, void* workspace,
                                  size_t workspace_bytes, void* stream) {
  gw::clear_error();
  return gw::attn_fwd_impl(dtype, q, q_strides, k, k_strides, v, v_strides, kv_pos, pos_stride_b, pos_stride_t, o,
                           o_strides, lse, attn_sum, B, T, S, H, D, K, softmax_scale, workspace, workspace_bytes,
                           nullptr, stream);
}

extern "C" int gw_sparse_attn_fwd_kl(int dtype, const void* q, const int64_t* q_strides, const void* k,
                                     const int64_t* k_strides, const void* v, const int64_t* v_strides,
                                     const int32_t* kv_pos, int64_t pos_stride_b, int64_t pos_stride_t, void* o,
                                     const int64_t* o_strides, float* lse, float* attn_sum, int64_t B, int64_t T,
                                     int64_t S, int64_t H, int64_t D, int64_t K, float softmax_scale,
                                     const void* logits, int logits_dtype, int64_t logits_stride_b,
                                     int64_t logits_stride_t, float eps, float* row_loss, void* workspace,
                                     size_t workspace_bytes, void* stream) {
  gw::clear_error();
  const gw::KlArgs kl{logits, logits_dtype, logits_stride_b, logits_stride_t, eps, row_loss};
  return gw::attn_fwd_impl(dtype, q, q_strides, k, k_strides, v, v_strides, kv_pos, pos_stride_b, pos_stride_t, o,
                           o_strides, lse, attn_sum, B, T, S, H, D, K, softmax_scale, workspace, workspace_bytes,
                           &kl, stream);
}

int gw::attn_fwd_flagged_blocks(int dtype, const void* q, const int64_t* q_strides, const void* k,
                                const int64_t* k_strides, const void* v, const int64_t* v_strides,
                                const int32_t* kv_pos, int64_t pos_stride_b, int64_t pos_stride_t, void* o,
                                const int64_t* o_strides, float* lse, float* attn_sum, int64_t B, int64_t T,
                                int64_t S, int64_t H, int64_t D, int64_t K, float softmax_scale, const void* logits,
                                int logits_dtype, int64_t logits_stride_b, int64_t logits_stride_t, float eps,
                                float* row_loss, void* workspace, size_t workspace_bytes, const int* blk_flags,
                                const int* batch_flags, int nqb, int nchunk, void* stream) {
  const gw::KlArgs kl{logits, logits_dtype, logits_stride_b, logits_stride_t, eps, row_loss};
  return gw::attn_fwd_impl(dtype, q, q_strides, k, k_strides, v, v_strides, kv_pos, pos_stride_b, pos_stride_t, o,
                           o_strides, lse, attn_sum, B, T, S, H, D, K, softmax_scale, workspace, workspace_bytes,
                           logits != nullptr ? &kl : nullptr, stream, blk_flags, batch_flags, nqb, nchunk);
}
