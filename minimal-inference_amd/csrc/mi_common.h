// Shared device helpers and host error plumbing for the gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mi_amd.h"

namespace mi {

// ---------------------------------------------------------------- host side
// Records a printf-style message as the calling thread's last error and
// returns `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
// Clears the calling thread's last error.
void clear_error();
// Converts a pending HIP launch error into MI_ERR_LAUNCH.
int check_launch(const char* what);
// Number of compute units of the current device (cached per device).
int num_cus();

inline size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

// ---------------------------------------------------------------- bf16
// bf16 bits <-> fp32.  Rounding is to nearest even; NaN maps to a quiet NaN
// with the sign kept, which is what torch's float->bfloat16 cast produces.
__device__ __forceinline__ float bf16_lo(uint32_t packed) { return __uint_as_float(packed << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t packed) {
  return __uint_as_float(packed & 0xffff0000u);
}
__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __uint_as_float(uint32_t(b) << 16); }
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return uint16_t((u >> 16) | 0x0040u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return uint16_t(u >> 16);
}
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return uint32_t(f32_to_bf16(lo)) | (uint32_t(f32_to_bf16(hi)) << 16);
}
// The same rounding (to nearest even) in one gfx950 instruction
// (v_cvt_pk_bf16_f32) per pair, for kernel outputs: finite values convert
// bit-identically to f32_to_bf16; a NaN comes out as a quiet NaN.
typedef __attribute__((ext_vector_type(2))) float f32x2_hw;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_hw;
__device__ __forceinline__ uint32_t cvt_pk_bf16(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_hw){lo, hi}, bf16x2_hw));
}
__device__ __forceinline__ uint16_t cvt_bf16(float f) { return uint16_t(cvt_pk_bf16(f, 0.f)); }
// 1 / x by the hardware reciprocal (1 ulp), for normalising outputs that are
// rounded to bf16 anyway.
__device__ __forceinline__ float fast_rcp(float x) { return __builtin_amdgcn_rcpf(x); }

// ---------------------------------------------------------------- MFMA types
typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;

__device__ __forceinline__ bf16x8_t as_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8_t, v); }

// D(16x16 fp32) += A(16x32 bf16) * B(32x16 bf16).  Lane l supplies A row
// (l & 15), B column (l & 15), both at k = 8 * (l >> 4) + [0, 8); lane l
// receives D rows 4 * (l >> 4) + [0, 4) of column (l & 15).
__device__ __forceinline__ f32x4_t mfma_16x16x32_bf16(bf16x8_t a, bf16x8_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// ---------------------------------------------------------------- cross-lane
// DPP controls (gfx9 encoding).
constexpr int kDppQuadSwap1 = 0xB1;    // quad_perm [1,0,3,2]
constexpr int kDppQuadSwap2 = 0x4E;    // quad_perm [2,3,0,1]
constexpr int kDppRowHalfMirror = 0x141;
constexpr int kDppRowMirror = 0x140;

template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, false));
}

// Max / sum over each aligned group of 16 lanes; every lane gets the result.
__device__ __forceinline__ float group16_max(float x) {
  x = fmaxf(x, dpp<kDppQuadSwap1>(x));
  x = fmaxf(x, dpp<kDppQuadSwap2>(x));
  x = fmaxf(x, dpp<kDppRowHalfMirror>(x));
  x = fmaxf(x, dpp<kDppRowMirror>(x));
  return x;
}
__device__ __forceinline__ float group16_sum(float x) {
  x += dpp<kDppQuadSwap1>(x);
  x += dpp<kDppQuadSwap2>(x);
  x += dpp<kDppRowHalfMirror>(x);
  x += dpp<kDppRowMirror>(x);
  return x;
}

// Value of `x` held by lane `src` (0..63), for every lane.
__device__ __forceinline__ float lane_shuffle(float x, int src) {
  return __int_as_float(__builtin_amdgcn_ds_bpermute(src << 2, __float_as_int(x)));
}
__device__ __forceinline__ int lane_shuffle_i(int x, int src) {
  return __builtin_amdgcn_ds_bpermute(src << 2, x);
}
// Wave-uniform value of `x` in lane `src` (src must be uniform).
__device__ __forceinline__ float read_lane(float x, int src) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), src));
}
__device__ __forceinline__ int read_lane_i(int x, int src) { return __builtin_amdgcn_readlane(x, src); }

__device__ __forceinline__ float wave_max(float x) {
  x = group16_max(x);
  x = fmaxf(x, lane_shuffle(x, (threadIdx.x & 63) ^ 16));
  x = fmaxf(x, lane_shuffle(x, (threadIdx.x & 63) ^ 32));
  return x;
}
__device__ __forceinline__ float wave_sum(float x) {
  x = group16_sum(x);
  x += lane_shuffle(x, (threadIdx.x & 63) ^ 16);
  x += lane_shuffle(x, (threadIdx.x & 63) ^ 32);
  return x;
}

__device__ __forceinline__ uint4 load16(const void* p) { return *reinterpret_cast<const uint4*>(p); }
// A 16-byte load marked non-temporal (nt): for rows read once, so they do not
// push reused data out of L2.
typedef __attribute__((ext_vector_type(4))) unsigned int u32x4_nt_t;
__device__ __forceinline__ uint4 load16_nt(const void* p) {
  const u32x4_nt_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_nt_t*>(p));
  return make_uint4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ void store16(void* p, uint4 v) { *reinterpret_cast<uint4*>(p) = v; }

constexpr float kLog2e = 1.4426950408889634f;

// ---------------------------------------------------------------- RoPE
// Rotate-half RoPE of 8 element pairs (d, d + D/2) with bf16 cos / sin, the
// reference's bf16 composition x * cos + rotate_half(x) * sin (model.py:
// 92-107): out_lo = x1 * c1 + (-x2) * s1, out_hi = x2 * c2 + x1 * s2, where
// each product is exact in fp32 (8-bit x 8-bit mantissas) and rounded to
// bf16 and the sum is taken in fp32 and rounded to bf16 -- what the three
// bf16 torch ops do -- so results are bit-identical to the unfused ops.
__device__ __forceinline__ void rope8(uint4 x1, uint4 x2, uint4 c1, uint4 s1, uint4 c2, uint4 s2, uint4& o1,
                                      uint4& o2) {
  const uint32_t* a = &x1.x;
  const uint32_t* b = &x2.x;
  const uint32_t* ca = &c1.x;
  const uint32_t* sa = &s1.x;
  const uint32_t* cb = &c2.x;
  const uint32_t* sb = &s2.x;
  uint32_t* oa = &o1.x;
  uint32_t* ob = &o2.x;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const uint32_t ac = cvt_pk_bf16(bf16_lo(a[w]) * bf16_lo(ca[w]), bf16_hi(a[w]) * bf16_hi(ca[w]));
    const uint32_t bs = cvt_pk_bf16(-bf16_lo(b[w]) * bf16_lo(sa[w]), -bf16_hi(b[w]) * bf16_hi(sa[w]));
    oa[w] = cvt_pk_bf16(bf16_lo(ac) + bf16_lo(bs), bf16_hi(ac) + bf16_hi(bs));
    const uint32_t bc = cvt_pk_bf16(bf16_lo(b[w]) * bf16_lo(cb[w]), bf16_hi(b[w]) * bf16_hi(cb[w]));
    const uint32_t as = cvt_pk_bf16(bf16_lo(a[w]) * bf16_lo(sb[w]), bf16_hi(a[w]) * bf16_hi(sb[w]));
    ob[w] = cvt_pk_bf16(bf16_lo(bc) + bf16_lo(as), bf16_hi(bc) + bf16_hi(as));
  }
}

}  // namespace mi
