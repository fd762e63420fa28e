// Shared device helpers for the gfx950 (CDNA4) kernels of libllmy.
//
// Storage conventions used by every kernel in this library:
//   * bf16 tensors are passed as raw 16-bit words (uint16_t); conversion to
//     fp32 is a 16-bit shift, conversion back is round-to-nearest-even (the
//     same rounding torch uses for .to(torch.bfloat16)).
//   * every buffer is a plain contiguous device allocation owned by the
//     caller; kernels never allocate.
//   * wavefronts are 64 lanes wide.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace llmy {

constexpr int kWave = 64;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ float bf2f(uint16_t v) {
  return __uint_as_float(static_cast<uint32_t>(v) << 16);
}

// fp32 -> bf16 with round-to-nearest-even (NaN stays NaN): one
// v_cvt_pk_bf16_f32 on gfx950, the rounding torch applies in .to(bfloat16).
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint16_t f2bf(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

__device__ __forceinline__ uint32_t pack_bf2(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a, b}, bf16x2_t));
}

// Unpack 8 bf16 held in a 16-byte vector into fp32.
__device__ __forceinline__ void unpack8(const uint4& v, float* out) {
  out[0] = __uint_as_float(v.x << 16);
  out[1] = __uint_as_float(v.x & 0xffff0000u);
  out[2] = __uint_as_float(v.y << 16);
  out[3] = __uint_as_float(v.y & 0xffff0000u);
  out[4] = __uint_as_float(v.z << 16);
  out[5] = __uint_as_float(v.z & 0xffff0000u);
  out[6] = __uint_as_float(v.w << 16);
  out[7] = __uint_as_float(v.w & 0xffff0000u);
}

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// 16-byte load of data that is streamed once per kernel (weights, the KV
// window): with LLMY_NT the load carries the non-temporal hint so it does not
// displace reusable lines in L2 / the Infinity Cache.
__device__ __forceinline__ uint4 ld_stream(const void* p) {
#if defined(LLMY_NT) && LLMY_NT
  const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  return uint4{v.x, v.y, v.z, v.w};
#else
  return *reinterpret_cast<const uint4*>(p);
#endif
}

__device__ __forceinline__ bf16x8 as_bf16x8(const uint4& v) {
  return __builtin_bit_cast(bf16x8, v);
}

// Reductions across one 64-lane wavefront with DPP row operations (quad
// xor-1, quad xor-2, half-row mirror, row mirror: every lane of a 16-lane row
// ends with the row's result) and four readlanes to combine the rows.  The
// combination order is fixed, so results are deterministic, and no LDS
// crossbar (ds_bpermute) round trips are needed.
constexpr int kDppXor1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141; // row_half_mirror
constexpr int kDppMirror = 0x140;     // row_mirror

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

template <int CTRL>
__device__ __forceinline__ uint64_t dpp_u64(uint64_t v) {
  const int lo = __builtin_amdgcn_update_dpp(0, static_cast<int>(v & 0xffffffffu), CTRL, 0xF, 0xF, false);
  const int hi = __builtin_amdgcn_update_dpp(0, static_cast<int>(v >> 32), CTRL, 0xF, 0xF, false);
  return (static_cast<uint64_t>(static_cast<uint32_t>(hi)) << 32) | static_cast<uint32_t>(lo);
}

__device__ __forceinline__ float readlane_f(float v, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_f<kDppXor1>(v);
  v += dpp_f<kDppXor2>(v);
  v += dpp_f<kDppHalfMirror>(v);
  v += dpp_f<kDppMirror>(v);
  return (readlane_f(v, 0) + readlane_f(v, 16)) + (readlane_f(v, 32) + readlane_f(v, 48));
}

__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp_f<kDppXor1>(v));
  v = fmaxf(v, dpp_f<kDppXor2>(v));
  v = fmaxf(v, dpp_f<kDppHalfMirror>(v));
  v = fmaxf(v, dpp_f<kDppMirror>(v));
  return fmaxf(fmaxf(readlane_f(v, 0), readlane_f(v, 16)),
               fmaxf(readlane_f(v, 32), readlane_f(v, 48)));
}

__device__ __forceinline__ uint64_t umax64(uint64_t a, uint64_t b) { return a > b ? a : b; }

__device__ __forceinline__ uint64_t readlane_u64(uint64_t v, int l) {
  const uint32_t lo = __builtin_amdgcn_readlane(static_cast<int>(v & 0xffffffffu), l);
  const uint32_t hi = __builtin_amdgcn_readlane(static_cast<int>(v >> 32), l);
  return (static_cast<uint64_t>(hi) << 32) | lo;
}

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
  v = umax64(v, dpp_u64<kDppXor1>(v));
  v = umax64(v, dpp_u64<kDppXor2>(v));
  v = umax64(v, dpp_u64<kDppHalfMirror>(v));
  v = umax64(v, dpp_u64<kDppMirror>(v));
  return umax64(umax64(readlane_u64(v, 0), readlane_u64(v, 16)),
                umax64(readlane_u64(v, 32), readlane_u64(v, 48)));
}

// Total-order key for an fp32 value: larger value -> larger key.  NaN (any
// sign) sorts above +inf, and -0.0 equals +0.0, matching torch's topk/argmax
// comparison rules.
__device__ __forceinline__ uint32_t order_key(float f) {
  if (f != f) return 0xffffffffu;
  if (f == 0.0f) f = 0.0f;
  uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// (value, index) packed so that an unsigned max picks the largest value and,
// among equal values, the lowest index.
__device__ __forceinline__ uint64_t value_index_key(float f, uint32_t idx) {
  return (static_cast<uint64_t>(order_key(f)) << 32) | static_cast<uint64_t>(~idx);
}

__device__ __forceinline__ uint32_t key_index(uint64_t key) {
  return ~static_cast<uint32_t>(key & 0xffffffffu);
}

// 2^x as the single v_exp_f32 instruction (exp2f adds a range rescale
// around it for results below 2^-126).  Used for softmax weights, whose
// exponents are <= 0: results under 2^-126 flush to zero, all others are
// within about 1 ulp.  exp2(-inf) = 0.
__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ float sigmoidf_(float x) { return 1.0f / (1.0f + expf(-x)); }

__device__ __forceinline__ float siluf_(float x) { return x / (1.0f + expf(-x)); }

// silu(x) = x * sigma(x) from single instructions: v_exp_f32 and v_rcp_f32
// (each within about 1 ulp), so within a few fp32 ulp of siluf_; at bf16
// output precision the two differ only where a value sits on a rounding
// boundary.  Saturates correctly: x * rcp(1 + inf) = -0 for very negative x.
__device__ __forceinline__ float silu_fast(float x) {
  return x * __builtin_amdgcn_rcpf(1.0f + exp2_fast(-1.4426950408889634f * x));
}

}  // namespace llmy
