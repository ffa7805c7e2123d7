// Shared device helpers and the C-ABI error plumbing for the gfx950 kernels.
//
// Every exported entry point returns int: 0 on success, a negative LFS_E*
// code for an argument error detected on the host (nothing was launched), or
// a positive hipError_t from the launch.  The message for the last failure on
// the calling thread is available from lfs_last_error().
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdarg.h>
#include <stdio.h>

#include "../../include/lfs_kernels.h"

namespace lfs {

// ---------------------------------------------------------------- errors --
void set_error(const char* fmt, ...);
int check_launch(const char* what);  // hipGetLastError -> code + message

#define LFS_REQUIRE(cond, ...)            \
  do {                                    \
    if (!(cond)) {                        \
      ::lfs::set_error(__VA_ARGS__);      \
      return LFS_EINVAL;                  \
    }                                     \
  } while (0)

// ------------------------------------------------------------ conversions --
__device__ __forceinline__ float bf16_to_f32(uint32_t h16) {
  return __uint_as_float(h16 << 16);
}
// two bf16 packed in one dword -> floats
__device__ __forceinline__ float bf16lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }

// fp32 -> bf16 bits: round to nearest even, a NaN keeps its sign and upper
// payload bits with the quiet bit set ((u >> 16) | 0x40).  gfx950's
// v_cvt_pk_bf16_f32 computes exactly this for every one of the 2^32 fp32
// inputs (compared exhaustively against the integer formula on the GPU), in
// one instruction per pair.
typedef float lfs_f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 lfs_bf16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(lfs_f32x2{lo, hi}, lfs_bf16x2));
}
__device__ __forceinline__ uint32_t f32_to_bf16(float f) {
  return (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)f);
}

// eight bf16 (one 16-byte chunk) -> floats
__device__ __forceinline__ void unpack8(const uint4& v, float* f) {
  f[0] = bf16lo(v.x); f[1] = bf16hi(v.x);
  f[2] = bf16lo(v.y); f[3] = bf16hi(v.y);
  f[4] = bf16lo(v.z); f[5] = bf16hi(v.z);
  f[6] = bf16lo(v.w); f[7] = bf16hi(v.w);
}

// Four floats -> four OCP e4m3fn codes in one dword (byte i = value i).
// v_cvt_pk_fp8_f32 rounds to nearest even; callers clamp to +-448 first.
__device__ __forceinline__ uint32_t f32x4_to_e4m3(float a, float b, float c, float d) {
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  w = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true);
  return (uint32_t)w;
}

// e4m3fn code pairs -> floats (exact); word_sel picks bytes 0-1 or 2-3
__device__ __forceinline__ void e4m3x4_to_f32(uint32_t w, float* o) {
  auto lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, false);
  auto hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, true);
  o[0] = lo[0]; o[1] = lo[1]; o[2] = hi[0]; o[3] = hi[1];
}

// ------------------------------------------------ e4m3 block quantisation --
// fp32(1/448): the reference multiplies the fp32 amax by fp8_max_inv
// (utils.py:101, :135); 1.0f/448.0f is the same correctly rounded constant.
constexpr float kFp8Max = 448.0f;
constexpr float kFp8MaxInv = 1.0f / 448.0f;
constexpr float kAmaxFloor = 1e-4f;  // utils.py:131

__device__ __forceinline__ float scale_from_amax(float amax, bool round_scale) {
  float s = fmaxf(amax, kAmaxFloor) * kFp8MaxInv;
  if (round_scale) {
    // ue8m0: smallest power of two >= s (utils.py:81-94)
    uint32_t b = __float_as_uint(s);
    int e = (int)((b >> 23) & 0xFFu) - 127 + ((b & 0x7FFFFFu) != 0u ? 1 : 0);
    s = __uint_as_float((uint32_t)(e + 127) << 23);
  }
  return s;
}

// clamp(x / s, -448, 448) with an IEEE divide; NaN passes through
__device__ __forceinline__ float qdiv(float x, float s) {
  float q = x / s;
  q = q > kFp8Max ? kFp8Max : q;
  q = q < -kFp8Max ? -kFp8Max : q;
  return q;
}

__device__ __forceinline__ uint2 quant8_ieee(const float* f, float s) {
  uint2 o;
  o.x = f32x4_to_e4m3(qdiv(f[0], s), qdiv(f[1], s), qdiv(f[2], s), qdiv(f[3], s));
  o.y = f32x4_to_e4m3(qdiv(f[4], s), qdiv(f[5], s), qdiv(f[6], s), qdiv(f[7], s));
  return o;
}

// Quotients x / s by a group's scale s = scale_from_amax(amax) for |x| <= amax.
// This is the compiler's correctly rounded fp32 divide (v_div_scale, rcp,
// one Newton step on the reciprocal, two residual corrections of the
// quotient, v_div_fmas, v_div_fixup) with the divisor's half -- y = rcp(s)
// refined by y += y * (1 - s*y) -- done once per group instead of once per
// element.  v_div_scale changes neither operand here: s lies in
// [1e-4/448, 2^120] (normal, 1/s normal), and it only scales a numerator
// below 2^-104 or 2^96 times smaller than s, whose quotient is below 2^-96
// and encodes as a signed zero whatever its low bits; with no scaling
// v_div_fmas is a plain fma and v_div_fixup passes a finite quotient
// through.  So an element costs a multiply and four FMAs and gets the
// divide's bits, except that a zero quotient may lose x's sign (callers put
// it back).  |x / s| <= 448 * (1 + 2^-23), which e4m3's round-to-nearest
// sends to 448, so the clamp is a no-op.  An infinite s (an infinite input)
// must take quant8_ieee instead.
__device__ __forceinline__ float recip_for_div(float s) {
  const float y = __builtin_amdgcn_rcpf(s);
  return fmaf(fmaf(-s, y, 1.0f), y, y);
}

__device__ __forceinline__ float div_by_group(float x, float s, float y) {
  float q = x * y;
  float e = fmaf(-s, q, x);
  q = fmaf(e, y, q);
  e = fmaf(-s, q, x);
  return fmaf(e, y, q);
}

// e4m3 codes of clamp(f[i] / s, -448, 448) (IEEE divide) for a group scale
// s = scale_from_amax(amax) with every |f[i]| <= amax
__device__ __forceinline__ uint2 quant8(const float* f, float s) {
  if (!(s < INFINITY)) return quant8_ieee(f, s);
  const float y = recip_for_div(s);
  float q[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) q[i] = copysignf(div_by_group(f[i], s, y), f[i]);
  uint2 o;
  o.x = f32x4_to_e4m3(q[0], q[1], q[2], q[3]);
  o.y = f32x4_to_e4m3(q[4], q[5], q[6], q[7]);
  return o;
}

// ------------------------------------------------------- wave reductions --
// The value of lane (lane ^ O), O = 1 .. 32 -- the partner __shfl_xor(v, O,
// 64) reads -- moved without the LDS permute unit: DPP quad permutations
// for O = 1, 2; for O = 4 a row shift left into banks 0 and 2 (lanes 0-3,
// 8-11 of each 16) and right into banks 1 and 3; a row rotation by 8 for
// O = 8; the permlane swaps for 16 and 32, which return the values of lanes
// l & ~O and l | O.  One or two VALU instructions instead of an LDS round
// trip in a dependent chain.  The lanes read must be active: every group of
// 2*O lanes all in or all out.
template <int O>
__device__ __forceinline__ int xor_partner(int v) {
  static_assert(O == 1 || O == 2 || O == 4 || O == 8 || O == 16 || O == 32, "xor distance");
  if constexpr (O == 1) {
    return __builtin_amdgcn_update_dpp(v, v, 0xB1, 0xF, 0xF, false);  // quad_perm [1, 0, 3, 2]
  } else if constexpr (O == 2) {
    return __builtin_amdgcn_update_dpp(v, v, 0x4E, 0xF, 0xF, false);  // quad_perm [2, 3, 0, 1]
  } else if constexpr (O == 4) {
    const int t = __builtin_amdgcn_update_dpp(v, v, 0x104, 0xF, 0x5, false);  // row_shl:4
    return __builtin_amdgcn_update_dpp(t, v, 0x114, 0xF, 0xA, false);         // row_shr:4
  } else if constexpr (O == 8) {
    return __builtin_amdgcn_update_dpp(v, v, 0x128, 0xF, 0xF, false);  // row_ror:8
  } else if constexpr (O == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    return (int)((__lane_id() & 16) ? r[0] : r[1]);
  } else {
    const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return (int)((__lane_id() & 32) ? r[0] : r[1]);
  }
}
__device__ __forceinline__ float as_float(int v) { return __int_as_float(v); }
// v op v(lane ^ O), the same operands as v op __shfl_xor(v, O, 64): IEEE add
// and max are commutative, so the results are bit-identical.  For 16 and 32
// the swap's two results are the two operands.
template <int O>
__device__ __forceinline__ float xor_sum(float v) {
  if constexpr (O == 16 || O == 32) {
    const auto r = O == 16 ? __builtin_amdgcn_permlane16_swap(__float_as_int(v), __float_as_int(v), false, false)
                           : __builtin_amdgcn_permlane32_swap(__float_as_int(v), __float_as_int(v), false, false);
    return as_float((int)r[0]) + as_float((int)r[1]);
  } else {
    return v + as_float(xor_partner<O>(__float_as_int(v)));
  }
}
template <int O>
__device__ __forceinline__ float xor_max(float v) {
  if constexpr (O == 16 || O == 32) {
    const auto r = O == 16 ? __builtin_amdgcn_permlane16_swap(__float_as_int(v), __float_as_int(v), false, false)
                           : __builtin_amdgcn_permlane32_swap(__float_as_int(v), __float_as_int(v), false, false);
    return fmaxf(as_float((int)r[0]), as_float((int)r[1]));
  } else {
    return fmaxf(v, as_float(xor_partner<O>(__float_as_int(v))));
  }
}

// xor-butterfly over groups of W consecutive lanes (W a power of two <= 64),
// distances W/2 down to 1 (the order of the sums)
template <int W>
__device__ __forceinline__ float group_max(float v) {
  if constexpr (W > 32) v = xor_max<32>(v);
  if constexpr (W > 16) v = xor_max<16>(v);
  if constexpr (W > 8) v = xor_max<8>(v);
  if constexpr (W > 4) v = xor_max<4>(v);
  if constexpr (W > 2) v = xor_max<2>(v);
  if constexpr (W > 1) v = xor_max<1>(v);
  return v;
}
template <int W>
__device__ __forceinline__ float group_sum(float v) {
  if constexpr (W > 32) v = xor_sum<32>(v);
  if constexpr (W > 16) v = xor_sum<16>(v);
  if constexpr (W > 8) v = xor_sum<8>(v);
  if constexpr (W > 4) v = xor_sum<4>(v);
  if constexpr (W > 2) v = xor_sum<2>(v);
  if constexpr (W > 1) v = xor_sum<1>(v);
  return v;
}

}  // namespace lfs
