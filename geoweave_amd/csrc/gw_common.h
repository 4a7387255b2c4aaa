// Shared host and device helpers for the gfx950 sparse global-attention kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#include "geoweave_hip.h"

// ---------------------------------------------------------------------------------------
// Host side: per-thread error message behind gw_last_error().
// ---------------------------------------------------------------------------------------
namespace gw {

// Records a printf-style message for gw_last_error() and returns `code`.
int set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();

// Maps a failed HIP call to GW_ERR_HIP with the call site in the message.
int hip_error(hipError_t err, const char* what);

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace gw

#define GW_CHECK_ARG(cond, ...)                                  \
  do {                                                           \
    if (!(cond)) return ::gw::set_error(GW_ERR_INVALID, __VA_ARGS__); \
  } while (0)

#define GW_HIP_LAUNCH_CHECK(what)                                \
  do {                                                           \
    hipError_t e__ = hipGetLastError();                          \
    if (e__ != hipSuccess) return ::gw::hip_error(e__, what);    \
  } while (0)

// ---------------------------------------------------------------------------------------
// Device side.
// ---------------------------------------------------------------------------------------
namespace gw {

// Element-type tags. BF16/FP16 are stored as their 16-bit pattern, FP32 as the float.
struct BF16 {};
struct FP16 {};
struct FP32 {};

template <typename E>
struct ElemBytes {
  static constexpr int value = 2;
};
template <>
struct ElemBytes<FP32> {
  static constexpr int value = 4;
};

// Element i of a tensor of element type E, as fp32 / stored from fp32 (16-bit types: round
// to nearest even).
__device__ __forceinline__ float ld_f32(BF16, const void* p, int64_t i) {
  return __uint_as_float((uint32_t)static_cast<const uint16_t*>(p)[i] << 16);
}
__device__ __forceinline__ float ld_f32(FP16, const void* p, int64_t i) {
  return (float)__builtin_bit_cast(_Float16, static_cast<const uint16_t*>(p)[i]);
}
__device__ __forceinline__ float ld_f32(FP32, const void* p, int64_t i) { return static_cast<const float*>(p)[i]; }

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

// fp32 dot of two packed pairs accumulated onto c: v_dot2_f32_bf16 / v_dot2_f32_f16.
// The products of two 16-bit floats are exact in fp32; only the accumulation rounds.
__device__ __forceinline__ float dot2(BF16, uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                         __builtin_bit_cast(bf16x2_t, b), c, false);
}
__device__ __forceinline__ float dot2(FP16, uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, a), __builtin_bit_cast(f16x2_t, b),
                                c, false);
}

// 8-element dot product of two 16-byte vectors (8 x 16-bit each).
template <typename E>
__device__ __forceinline__ float dot8(uint4 a, uint4 b) {
  float s = dot2(E{}, a.x, b.x, 0.f);
  s = dot2(E{}, a.y, b.y, s);
  s = dot2(E{}, a.z, b.z, s);
  s = dot2(E{}, a.w, b.w, s);
  return s;
}

// Unpacks a 32-bit word holding two 16-bit floats (low half first) to fp32.
__device__ __forceinline__ void unpack2(BF16, uint32_t u, float& lo, float& hi) {
  lo = __uint_as_float(u << 16);
  hi = __uint_as_float(u & 0xffff0000u);
}
__device__ __forceinline__ void unpack2(FP16, uint32_t u, float& lo, float& hi) {
  f16x2_t h = __builtin_bit_cast(f16x2_t, u);
  lo = (float)h.x;
  hi = (float)h.y;
}

template <typename E>
__device__ __forceinline__ void unpack8(uint4 v, float* f) {
  unpack2(E{}, v.x, f[0], f[1]);
  unpack2(E{}, v.y, f[2], f[3]);
  unpack2(E{}, v.z, f[4], f[5]);
  unpack2(E{}, v.w, f[6], f[7]);
}

// fp32 -> 16-bit float, round to nearest even (NaN kept quiet).
__device__ __forceinline__ uint32_t pack1(BF16, float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}
__device__ __forceinline__ uint32_t pack1(FP16, float f) {
  _Float16 h = (_Float16)f;
  return (uint32_t)__builtin_bit_cast(uint16_t, h);
}
__device__ __forceinline__ void st_f32(BF16, void* p, int64_t i, float f) {
  static_cast<uint16_t*>(p)[i] = (uint16_t)pack1(BF16{}, f);
}
__device__ __forceinline__ void st_f32(FP16, void* p, int64_t i, float f) {
  static_cast<uint16_t*>(p)[i] = (uint16_t)pack1(FP16{}, f);
}
__device__ __forceinline__ void st_f32(FP32, void* p, int64_t i, float f) { static_cast<float*>(p)[i] = f; }

// Eight consecutive elements: one 16-byte word for the 16-bit types, two for fp32.
template <typename E>
struct Raw8 {
  uint4 v;
};
template <>
struct Raw8<FP32> {
  uint4 lo, hi;
};
// Loads elements [i, i + 8) (16-byte aligned for 16-bit types, 32-byte for fp32).
template <typename E>
__device__ __forceinline__ Raw8<E> ld8(const void* p, int64_t i) {
  Raw8<E> r;
  if constexpr (ElemBytes<E>::value == 4) {
    const uint4* s = reinterpret_cast<const uint4*>(static_cast<const float*>(p) + i);
    r.lo = s[0];
    r.hi = s[1];
  } else {
    r.v = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(p) + i);
  }
  return r;
}
template <typename E>
__device__ __forceinline__ Raw8<E> zero8() {
  Raw8<E> r;
  if constexpr (ElemBytes<E>::value == 4) {
    r.lo = make_uint4(0, 0, 0, 0);
    r.hi = make_uint4(0, 0, 0, 0);
  } else {
    r.v = make_uint4(0, 0, 0, 0);
  }
  return r;
}
template <typename E>
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  return pack1(E{}, lo) | (pack1(E{}, hi) << 16);
}
template <typename E>
__device__ __forceinline__ uint4 pack8(const float* f) {
  return make_uint4(pack2<E>(f[0], f[1]), pack2<E>(f[2], f[3]), pack2<E>(f[4], f[5]),
                    pack2<E>(f[6], f[7]));
}

// Raw8 <-> fp32, its 8-element dot product (fp32 accumulation in element order) and store.
template <typename E>
__device__ __forceinline__ void up8(const Raw8<E>& r, float* f) {
  if constexpr (ElemBytes<E>::value == 4) {
    f[0] = __uint_as_float(r.lo.x);
    f[1] = __uint_as_float(r.lo.y);
    f[2] = __uint_as_float(r.lo.z);
    f[3] = __uint_as_float(r.lo.w);
    f[4] = __uint_as_float(r.hi.x);
    f[5] = __uint_as_float(r.hi.y);
    f[6] = __uint_as_float(r.hi.z);
    f[7] = __uint_as_float(r.hi.w);
  } else {
    unpack8<E>(r.v, f);
  }
}
template <typename E>
__device__ __forceinline__ float dot8r(const Raw8<E>& a, const Raw8<E>& b) {
  if constexpr (ElemBytes<E>::value == 4) {
    float x[8], y[8];
    up8<E>(a, x);
    up8<E>(b, y);
    float s = x[0] * y[0];
#pragma unroll
    for (int i = 1; i < 8; ++i) s = fmaf(x[i], y[i], s);
    return s;
  } else {
    return dot8<E>(a.v, b.v);
  }
}
template <typename E>
__device__ __forceinline__ void st8(void* p, int64_t i, const float* f) {
  if constexpr (ElemBytes<E>::value == 4) {
    uint4* d = reinterpret_cast<uint4*>(static_cast<float*>(p) + i);
    d[0] = make_uint4(__float_as_uint(f[0]), __float_as_uint(f[1]), __float_as_uint(f[2]), __float_as_uint(f[3]));
    d[1] = make_uint4(__float_as_uint(f[4]), __float_as_uint(f[5]), __float_as_uint(f[6]), __float_as_uint(f[7]));
  } else {
    *reinterpret_cast<uint4*>(static_cast<uint16_t*>(p) + i) = pack8<E>(f);
  }
}

__device__ __forceinline__ float fexp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float flog2(float x) { return __builtin_amdgcn_logf(x); }

// DPP lane exchange within a 16-lane row (gfx9 encodings).
template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, true));
}
constexpr int kDppXor1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141; // lane i <- lane 7-i within 8 lanes
constexpr int kDppMirror = 0x140;     // lane i <- lane 15-i within 16 lanes

// Sum over aligned groups of N consecutive lanes (N in {1,2,4,8,16}); every lane of the
// group receives the total.
template <int N>
__device__ __forceinline__ float group_sum(float x) {
  if constexpr (N >= 2) x += dpp<kDppXor1>(x);
  if constexpr (N >= 4) x += dpp<kDppXor2>(x);
  if constexpr (N >= 8) x += dpp<kDppHalfMirror>(x);
  if constexpr (N >= 16) x += dpp<kDppMirror>(x);
  return x;
}

// A wave-uniform address pinned to scalar registers (both halves read from the first active
// lane).
__device__ __forceinline__ const char* uniform_ptr(const char* p) {
  const uint64_t u = reinterpret_cast<uint64_t>(p);
  const uint64_t r = ((uint64_t)__builtin_amdgcn_readfirstlane((uint32_t)(u >> 32)) << 32) |
                     (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)u);
  return reinterpret_cast<const char*>(r);
}

// Loads through a buffer descriptor built in scalar registers from a wave-uniform base (raw
// buffer, stride 0, the full 32-bit range: no clamping of in-range offsets) and a 32-bit lane
// offset in bytes. The descriptor's third word is the gfx9-family data format for raw loads.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t uniform_rsrc(const char* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(uniform_ptr(base)), (short)0, -1, 0x00020000);
}
__device__ __forceinline__ uint4 buffer_load16(const char* base, uint32_t off) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b128(uniform_rsrc(base), (int)off, 0, 0);
  return make_uint4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ uint32_t buffer_load4(const char* base, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b32(uniform_rsrc(base), (int)off, 0, 0);
}

// 16-byte buffer load straight into LDS (no registers): lane i of the wave writes the 16
// bytes it reads at lds + 16 i, whatever its offset; lds must be the same in every lane of
// the wave. The data is in LDS once vmcnt has drained (s_waitcnt vmcnt(0), then a barrier
// for the other waves).
__device__ __forceinline__ void buffer_load16_lds(const char* base, uint32_t off, void* lds) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(uniform_rsrc(base), (__attribute__((address_space(3))) void*)lds, 16,
                                           (int)off, 0, 0, 0);
}

}  // namespace gw
