// Sparse-index attention backward for gfx950, without float atomics.
//
// Math (reference _bwd_preprocess_do_o_dot + _bwd_sparse_index_kernel,
// easyvolcap/utils/custom_flash_attn/sparse_index_flash_attn.py:534-743), per (b, t, h)
// and candidate j with s = pos[b,t,j] valid:
//   p_j   = exp(scale * q.k_s - lse)          (recomputed from the forward's lse)
//   dp_j  = v_s . dO (+ dattn[b,t,j])
//   total = sum_d o*dO (+ sum_j dattn_j p_j)
//   ds_j  = (dp_j - total) * p_j
//   dq    = scale * sum_j ds_j k_s
//   dk_s += scale * ds_j * q,   dv_s += p_j * dO
//
// Two passes over the (t, j) pairs instead of one pass with fp32 atomics:
//  dq pass  (query-major, the forward's layout: one wave per query and group of heads,
//            gathering the selected K and V rows). It also writes {lse * log2(e), total}
//            per (b, t, h) for the key pass (one 8-byte load per entry there). With
//            dattn, total is only known after the sweep, so the wave accumulates
//            A1 = sum_j dp_j p_j k_s and A2 = sum_j p_j k_s and forms
//            dq = scale * (A1 - total * A2) at the end: one K/V gather instead of the
//            reference's two (:640-676 then :678-740).
//  dkv pass (key-major over the CSR of kv_csr.hip: one wave per work item = up to 2048
//            entries of one key, and group of heads). The key's K and V rows stay in
//            registers; the wave gathers q, dO and {lse, total} of each entry's query
//            (2 entries per block, the next block's gathers in flight while one is
//            consumed), recomputes p_j and ds_j, and accumulates dk and dv in fp32.
// Both passes are latency-bound random gathers; their block sizes (4 keys per lane group
// in the dq pass, 2 entries in the dkv pass) were chosen by measurement: smaller blocks
// leave fewer bytes in flight per wave but let more waves run per SIMD. A key whose
//            entries span several items writes fp32 partials that a reduce kernel sums
//            in item order.
// Every sum runs in a fixed order, so the backward is bitwise reproducible.
#include <math.h>

#include "gw_common.h"
#include "gw_csr.h"

namespace gw {
namespace {

constexpr float kLog2e = 1.4426950408889634f;

struct AttnBwdParams {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const uint16_t* o;
  const uint16_t* dout;
  const uint16_t* dattn;  // [B, T, K] contiguous or null
  const int32_t* pos;
  const float* lse;  // [B, T, H]
  float2* lse_tot;   // [B, T, H] {lse * log2(e), total}
  uint16_t* dq;
  uint16_t* dk;
  uint16_t* dv;
  float* part;  // [parts, 2, H, D]
  CsrView csr;
  int64_t qsb, qst, qsh;
  int64_t ksb, kss, ksh;
  int64_t vsb, vss, vsh;
  int64_t osb, ost, osh;
  int64_t dosb, dost, dosh;
  int64_t dqsb, dqst, dqsh;
  int64_t dksb, dkss, dksh;
  int64_t dvsb, dvss, dvsh;
  int64_t psb, pst;
  int T, S, H, D, K;
  int NG;   // head groups (waves) per query / item
  int QPB;  // queries (dq pass) or items (dkv pass) per workgroup
  float scale, scale_log2;
};

__device__ __forceinline__ float to_f32(BF16, uint16_t x) { return __uint_as_float((uint32_t)x << 16); }
__device__ __forceinline__ float to_f32(FP16, uint16_t x) { return (float)__builtin_bit_cast(_Float16, x); }

template <typename E, int D, int HPW, bool DATTN>
__global__ __launch_bounds__(256) void sparse_attn_bwd_dq_kernel(const AttnBwdParams p) {
  constexpr int LPH = D / 8;
  constexpr int HL = HPW * LPH;
  constexpr int G = 64 / HL;
  constexpr int U = 4;  // keys per block and lane group (136 VGPRs: 3 waves per SIMD)
  constexpr int STEP = U * G;
  static_assert(HL * G == 64, "lane decomposition must cover one wave");

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int ql = wave / p.NG;
  const int hg = wave - ql * p.NG;
  const int t = blockIdx.x * p.QPB + ql;
  const int b = blockIdx.y;
  if (t >= p.T) return;
  const int g = lane / HL;
  const int hh = (lane % HL) / LPH;
  const int c = lane % LPH;
  const int h = hg * HPW + hh;
  const bool head_ok = h < p.H;

  uint4 qv = make_uint4(0, 0, 0, 0), ov = qv, dov = qv;
  float lse2 = -INFINITY;
  if (head_ok) {
    qv = *reinterpret_cast<const uint4*>(p.q + b * p.qsb + (int64_t)t * p.qst + h * p.qsh + c * 8);
    ov = *reinterpret_cast<const uint4*>(p.o + b * p.osb + (int64_t)t * p.ost + h * p.osh + c * 8);
    dov = *reinterpret_cast<const uint4*>(p.dout + b * p.dosb + (int64_t)t * p.dost + h * p.dosh + c * 8);
    lse2 = p.lse[((int64_t)b * p.T + t) * p.H + h] * kLog2e;
  }
  const float delta = group_sum<LPH>(dot8<E>(ov, dov));
  const bool row_ok = lse2 != -INFINITY;

  const uint16_t* kb = p.k + b * p.ksb + h * p.ksh + c * 8;
  const uint16_t* vb = p.v + b * p.vsb + h * p.vsh + c * 8;
  const int32_t* prow = p.pos + b * p.psb + (int64_t)t * p.pst;
  const uint16_t* darow = DATTN ? p.dattn + ((int64_t)b * p.T + t) * p.K : nullptr;

  float acc[8], acc2[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = acc2[i] = 0.f;
  float sdp = 0.f;

  auto load_pos = [&](int (&pp)[U], float (&dd)[U], int j0) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int j = j0 + u * G + g;
      pp[u] = (j < p.K) ? prow[j] : -1;
      if constexpr (DATTN) dd[u] = (j < p.K) ? to_f32(E{}, darow[j]) : 0.f;
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
  float dc[U], dn[U];
  uint4 kc[U], vc[U];
  load_pos(pc, dc, 0);
  load_kv(kc, vc, pc);
  load_pos(pn, dn, STEP);

  for (int j0 = 0; j0 < p.K; j0 += STEP) {
    uint4 kn[U], vn[U];
    int pnn[U];
    float dnn[U];
    load_kv(kn, vn, pn);
    load_pos(pnn, dnn, j0 + 2 * STEP);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const float sd = group_sum<LPH>(dot8<E>(qv, kc[u]));
      const bool valid = row_ok && pc[u] >= 0 && pc[u] < p.S;
      const float pj = valid ? fexp2(sd * p.scale_log2 - lse2) : 0.f;
      float dp = group_sum<LPH>(dot8<E>(vc[u], dov));
      float coef;
      if constexpr (DATTN) {
        dp += dc[u];
        sdp = fmaf(dc[u], pj, sdp);
        coef = dp * pj;
      } else {
        coef = (dp - delta) * pj;
      }
      float kf[8];
      unpack8<E>(kc[u], kf);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        acc[i] = fmaf(coef, kf[i], acc[i]);
        if constexpr (DATTN) acc2[i] = fmaf(pj, kf[i], acc2[i]);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      kc[u] = kn[u];
      vc[u] = vn[u];
      pc[u] = pn[u];
      pn[u] = pnn[u];
      if constexpr (DATTN) {
        dc[u] = dn[u];
        dn[u] = dnn[u];
      }
    }
  }

#pragma unroll
  for (int off = HL; off < 64; off <<= 1) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      acc[i] += __shfl_xor(acc[i], off);
      if constexpr (DATTN) acc2[i] += __shfl_xor(acc2[i], off);
    }
    if constexpr (DATTN) sdp += __shfl_xor(sdp, off);
  }
  const float total = delta + sdp;
  if (g == 0 && head_ok) {
    float out[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float a = DATTN ? fmaf(-total, acc2[i], acc[i]) : acc[i];
      out[i] = a * p.scale;
    }
    *reinterpret_cast<uint4*>(p.dq + b * p.dqsb + (int64_t)t * p.dqst + h * p.dqsh + c * 8) = pack8<E>(out);
    if (c == 0) p.lse_tot[((int64_t)b * p.T + t) * p.H + h] = make_float2(lse2, total);
  }
}

template <typename E, int D, int HPW, bool DATTN>
__global__ __launch_bounds__(256) void sparse_attn_bwd_dkv_kernel(const AttnBwdParams p) {
  constexpr int LPH = D / 8;
  constexpr int HL = HPW * LPH;
  constexpr int G = 64 / HL;
  constexpr int U = 2;  // entries per block and lane group (small blocks: more waves in flight)
  constexpr int STEP = U * G;
  static_assert(HL * G == 64, "lane decomposition must cover one wave");

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int il = wave / p.NG;
  const int hg = wave - il * p.NG;
  const int item = blockIdx.x * p.QPB + il;
  if (item >= p.csr.header[0]) return;
  const CsrItem it = csr_item(p.csr, item);
  const int b = it.key / p.S;
  const int s = it.key - b * p.S;
  const int g = lane / HL;
  const int hh = (lane % HL) / LPH;
  const int c = lane % LPH;
  const int h = hg * HPW + hh;
  const bool head_ok = h < p.H;
  const int hs = head_ok ? h : 0;

  uint4 kv = make_uint4(0, 0, 0, 0), vv = kv;
  if (head_ok) {
    kv = *reinterpret_cast<const uint4*>(p.k + b * p.ksb + (int64_t)s * p.kss + h * p.ksh + c * 8);
    vv = *reinterpret_cast<const uint4*>(p.v + b * p.vsb + (int64_t)s * p.vss + h * p.vsh + c * 8);
  }
  const uint16_t* qb = p.q + b * p.qsb + hs * p.qsh + c * 8;
  const uint16_t* dob = p.dout + b * p.dosb + hs * p.dosh + c * 8;
  const float2* ltb = p.lse_tot + (int64_t)b * p.T * p.H + hs;
  const uint16_t* dab = DATTN ? p.dattn + (int64_t)b * p.T * p.K : nullptr;

  float ak[8], av[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) ak[i] = av[i] = 0.f;

  // Software-pipelined gathers: the q/dO/{lse,total} rows of block i+1 are issued before
  // block i is consumed, and the entries of block i+2 before that.
  auto load_entries = [&](int2 (&ee)[U], int i0) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int i = i0 + u * G + g;
      ee[u] = i < it.end ? p.csr.entries[i] : make_int2(-1, 0);
    }
  };
  auto gather = [&](uint4 (&qv)[U], uint4 (&dv)[U], float2 (&lt)[U], float (&da)[U], const int2 (&ee)[U]) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const bool ok = ee[u].x >= 0;
      const int64_t tt = ok ? ee[u].x : 0;
      qv[u] = make_uint4(0, 0, 0, 0);
      dv[u] = qv[u];
      lt[u] = make_float2(0.f, 0.f);
      da[u] = 0.f;
      if (ok) {
        qv[u] = *reinterpret_cast<const uint4*>(qb + tt * p.qst);
        dv[u] = *reinterpret_cast<const uint4*>(dob + tt * p.dost);
        lt[u] = ltb[tt * p.H];
        if constexpr (DATTN) da[u] = to_f32(E{}, dab[tt * p.K + ee[u].y]);
      }
    }
  };
  int2 ec[U], en[U];
  uint4 qc[U], dc[U];
  float2 lc[U];
  float dac[U];
  load_entries(ec, it.beg);
  gather(qc, dc, lc, dac, ec);
  load_entries(en, it.beg + STEP);
  for (int i0 = it.beg; i0 < it.end; i0 += STEP) {
    uint4 qn[U], dn[U];
    float2 ln[U];
    float dan[U];
    gather(qn, dn, ln, dan, en);  // block i+1 (past the end: no traffic)
    int2 enn[U];
    load_entries(enn, i0 + 2 * STEP);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const bool ok = ec[u].x >= 0 && head_ok;
      const float sd = group_sum<LPH>(dot8<E>(qc[u], kv));
      const float pj = ok ? fexp2(sd * p.scale_log2 - lc[u].x) : 0.f;
      const float dp = group_sum<LPH>(dot8<E>(vv, dc[u])) + dac[u];
      const float ds = (dp - lc[u].y) * pj;
      float qf[8], df[8];
      unpack8<E>(qc[u], qf);
      unpack8<E>(dc[u], df);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        ak[i] = fmaf(ds, qf[i], ak[i]);
        av[i] = fmaf(pj, df[i], av[i]);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      ec[u] = en[u];
      en[u] = enn[u];
      qc[u] = qn[u];
      dc[u] = dn[u];
      lc[u] = ln[u];
      dac[u] = dan[u];
    }
  }

#pragma unroll
  for (int off = HL; off < 64; off <<= 1) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      ak[i] += __shfl_xor(ak[i], off);
      av[i] += __shfl_xor(av[i], off);
    }
  }
  if (g == 0 && head_ok) {
#pragma unroll
    for (int i = 0; i < 8; ++i) ak[i] *= p.scale;
    if (it.nchunk == 1) {
      *reinterpret_cast<uint4*>(p.dk + b * p.dksb + (int64_t)s * p.dkss + h * p.dksh + c * 8) = pack8<E>(ak);
      *reinterpret_cast<uint4*>(p.dv + b * p.dvsb + (int64_t)s * p.dvss + h * p.dvsh + c * 8) = pack8<E>(av);
    } else {
      float* pk = p.part + ((int64_t)it.part * 2 * p.H + h) * p.D + c * 8;
      float* pv = pk + (int64_t)p.H * p.D;
#pragma unroll
      for (int i = 0; i < 8; i += 4) {
        *reinterpret_cast<float4*>(pk + i) = make_float4(ak[i], ak[i + 1], ak[i + 2], ak[i + 3]);
        *reinterpret_cast<float4*>(pv + i) = make_float4(av[i], av[i + 1], av[i + 2], av[i + 3]);
      }
    }
  }
}

// Sums the partials of keys split over several items, in item order.
template <typename E>
__global__ __launch_bounds__(256) void sparse_attn_bwd_reduce_kernel(const AttnBwdParams p) {
  const int key = blockIdx.x;
  const int n = p.csr.item_off[key + 1] - p.csr.item_off[key];
  if (n <= 1) return;
  const int b = key / p.S, s = key - b * p.S;
  const int base = p.csr.part_off[key];
  const int HD = p.H * p.D;
  for (int i = threadIdx.x; i < HD; i += 256) {
    float sk = 0.f, sv = 0.f;
    for (int c = 0; c < n; ++c) {
      const float* pk = p.part + (int64_t)(base + c) * 2 * HD;
      sk += pk[i];
      sv += pk[HD + i];
    }
    const int h = i / p.D, d = i - h * p.D;
    p.dk[b * p.dksb + (int64_t)s * p.dkss + h * p.dksh + d] = (uint16_t)pack1(E{}, sk);
    p.dv[b * p.dvsb + (int64_t)s * p.dvss + h * p.dvsh + d] = (uint16_t)pack1(E{}, sv);
  }
}

template <typename E, int D, int HPW, bool DATTN>
int launch_bwd(AttnBwdParams p, int B, int64_t max_items, hipStream_t st) {
  {
    dim3 grid((p.T + p.QPB - 1) / p.QPB, B);
    hipLaunchKernelGGL((sparse_attn_bwd_dq_kernel<E, D, HPW, DATTN>), grid, dim3(64 * p.NG * p.QPB), 0, st, p);
    GW_HIP_LAUNCH_CHECK("sparse_attn_bwd_dq_kernel launch");
  }
  {
    dim3 grid((unsigned)((max_items + p.QPB - 1) / p.QPB));
    hipLaunchKernelGGL((sparse_attn_bwd_dkv_kernel<E, D, HPW, DATTN>), grid, dim3(64 * p.NG * p.QPB), 0, st, p);
    GW_HIP_LAUNCH_CHECK("sparse_attn_bwd_dkv_kernel launch");
  }
  hipLaunchKernelGGL((sparse_attn_bwd_reduce_kernel<E>), dim3(p.csr.nk), dim3(256), 0, st, p);
  GW_HIP_LAUNCH_CHECK("sparse_attn_bwd_reduce_kernel launch");
  return GW_OK;
}

template <typename E, int D, int HPW>
int dispatch_dattn(const AttnBwdParams& p, int B, int64_t mi, bool dattn, hipStream_t st) {
  return dattn ? launch_bwd<E, D, HPW, true>(p, B, mi, st) : launch_bwd<E, D, HPW, false>(p, B, mi, st);
}

template <typename E>
int dispatch_bwd(const AttnBwdParams& p, int B, int64_t mi, int hpw, bool dattn, hipStream_t st) {
  if (p.D == 64) {
    switch (hpw) {
      case 1: return dispatch_dattn<E, 64, 1>(p, B, mi, dattn, st);
      case 2: return dispatch_dattn<E, 64, 2>(p, B, mi, dattn, st);
      case 4: return dispatch_dattn<E, 64, 4>(p, B, mi, dattn, st);
      default: return dispatch_dattn<E, 64, 8>(p, B, mi, dattn, st);
    }
  }
  switch (hpw) {
    case 1: return dispatch_dattn<E, 128, 1>(p, B, mi, dattn, st);
    case 2: return dispatch_dattn<E, 128, 2>(p, B, mi, dattn, st);
    default: return dispatch_dattn<E, 128, 4>(p, B, mi, dattn, st);
  }
}

int pow2_ceil(int x) {
  int r = 1;
  while (r < x) r <<= 1;
  return r;
}

struct BwdWs {
  size_t lt_off, part_off, bytes;
};

BwdWs bwd_ws(int64_t B, int64_t T, int64_t S, int64_t H, int64_t D, int64_t K) {
  BwdWs w;
  const CsrLayout L = csr_layout(B, T, S, K);
  w.lt_off = 0;
  w.part_off = ((size_t)B * T * H * 8 + 255) / 256 * 256;
  w.bytes = w.part_off + (size_t)L.max_parts * 2 * H * D * 4;
  return w;
}

}  // namespace
}  // namespace gw

extern "C" size_t gw_sparse_attn_bwd_workspace_size(int64_t B, int64_t T, int64_t S, int64_t H, int64_t D,
                                                    int64_t K) {
  if (B <= 0 || T <= 0 || S <= 0 || H <= 0 || D <= 0 || K <= 0) return 256;
  return gw::bwd_ws(B, T, S, H, D, K).bytes;
}

extern "C" int gw_sparse_attn_bwd(int dtype, const void* q, const int64_t* q_strides, const void* k,
                                  const int64_t* k_strides, const void* v, const int64_t* v_strides,
                                  const int32_t* kv_pos, int64_t pos_stride_b, int64_t pos_stride_t,
                                  const void* o, const int64_t* o_strides, const void* dout,
                                  const int64_t* do_strides, const float* lse, const void* dattn_sum, void* dq,
                                  const int64_t* dq_strides, void* dk, const int64_t* dk_strides, void* dv,
                                  const int64_t* dv_strides, int64_t B, int64_t T, int64_t S, int64_t H,
                                  int64_t D, int64_t K, float softmax_scale, const void* csr, size_t csr_bytes,
                                  void* workspace, size_t workspace_bytes, void* stream) {
  using namespace gw;
  clear_error();
  GW_CHECK_ARG(dtype == GW_DTYPE_BF16 || dtype == GW_DTYPE_FP16, "unsupported dtype code %d", dtype);
  GW_CHECK_ARG(B >= 0 && T >= 0 && S >= 0 && H >= 1 && K >= 0, "invalid sizes B=%lld T=%lld S=%lld H=%lld K=%lld",
               (long long)B, (long long)T, (long long)S, (long long)H, (long long)K);
  if (D != 64 && D != 128)
    return set_error(GW_ERR_UNSUPPORTED, "head dim %lld not supported (64 or 128)", (long long)D);
  if (B == 0 || T == 0 || S == 0) return GW_OK;
  GW_CHECK_ARG(K >= 1, "kv_positions must have at least one candidate");
  GW_CHECK_ARG(q && k && v && kv_pos && o && dout && lse && dq && dk && dv, "null tensor pointer");
  GW_CHECK_ARG(q_strides && k_strides && v_strides && o_strides && do_strides && dq_strides && dk_strides &&
                   dv_strides,
               "null stride array");
  GW_CHECK_ARG(aligned16(q) && aligned16(k) && aligned16(v) && aligned16(o) && aligned16(dout) &&
                   aligned16(dq) && aligned16(dk) && aligned16(dv),
               "q/k/v/o/dO/dq/dk/dv must be 16-byte aligned");
  const int64_t* all[] = {q_strides, k_strides, v_strides, o_strides, do_strides, dq_strides, dk_strides, dv_strides};
  for (const int64_t* st : all)
    for (int i = 0; i < 3; ++i) GW_CHECK_ARG(st[i] % 8 == 0, "b/t/h strides must be multiples of 8 elements");
  GW_CHECK_ARG(B <= 65535 && T < (1ll << 31), "size exceeds grid or int32 range");
  GW_CHECK_ARG(csr != nullptr && csr_bytes >= gw_kv_csr_size(B, T, S, K),
               "csr buffer needs %zu bytes (built by gw_kv_csr_build), got %zu", gw_kv_csr_size(B, T, S, K),
               csr_bytes);
  const BwdWs w = bwd_ws(B, T, S, H, D, K);
  GW_CHECK_ARG(workspace != nullptr && aligned16(workspace) && workspace_bytes >= w.bytes,
               "workspace needs %zu bytes (16-byte aligned), got %zu", w.bytes, workspace_bytes);

  const CsrLayout L = csr_layout(B, T, S, K);
  const int lph = (int)D / 8;
  const int hpw_max = 64 / lph;
  const int hpw = pow2_ceil((int)H) < hpw_max ? pow2_ceil((int)H) : hpw_max;
  AttnBwdParams p{};
  p.q = static_cast<const uint16_t*>(q);
  p.k = static_cast<const uint16_t*>(k);
  p.v = static_cast<const uint16_t*>(v);
  p.o = static_cast<const uint16_t*>(o);
  p.dout = static_cast<const uint16_t*>(dout);
  p.dattn = static_cast<const uint16_t*>(dattn_sum);
  p.pos = kv_pos;
  p.lse = lse;
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  p.lse_tot = reinterpret_cast<float2*>(ws + w.lt_off);
  p.part = reinterpret_cast<float*>(ws + w.part_off);
  p.dq = static_cast<uint16_t*>(dq);
  p.dk = static_cast<uint16_t*>(dk);
  p.dv = static_cast<uint16_t*>(dv);
  p.csr = csr_view(csr, L);
  p.qsb = q_strides[0]; p.qst = q_strides[1]; p.qsh = q_strides[2];
  p.ksb = k_strides[0]; p.kss = k_strides[1]; p.ksh = k_strides[2];
  p.vsb = v_strides[0]; p.vss = v_strides[1]; p.vsh = v_strides[2];
  p.osb = o_strides[0]; p.ost = o_strides[1]; p.osh = o_strides[2];
  p.dosb = do_strides[0]; p.dost = do_strides[1]; p.dosh = do_strides[2];
  p.dqsb = dq_strides[0]; p.dqst = dq_strides[1]; p.dqsh = dq_strides[2];
  p.dksb = dk_strides[0]; p.dkss = dk_strides[1]; p.dksh = dk_strides[2];
  p.dvsb = dv_strides[0]; p.dvss = dv_strides[1]; p.dvsh = dv_strides[2];
  p.psb = pos_stride_b;
  p.pst = pos_stride_t;
  p.T = (int)T;
  p.S = (int)S;
  p.H = (int)H;
  p.D = (int)D;
  p.K = (int)K;
  p.NG = (int)((H + hpw - 1) / hpw);
  GW_CHECK_ARG(p.NG <= 4, "too many head groups (%d) for one workgroup", p.NG);
  p.QPB = 4 / p.NG;
  if (p.QPB < 1) p.QPB = 1;
  p.scale = softmax_scale;
  p.scale_log2 = softmax_scale * kLog2e;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool has_dattn = dattn_sum != nullptr;
  if (dtype == GW_DTYPE_BF16) return dispatch_bwd<BF16>(p, (int)B, L.max_items, hpw, has_dattn, st);
  return dispatch_bwd<FP16>(p, (int)B, L.max_items, hpw, has_dattn, st);
}
