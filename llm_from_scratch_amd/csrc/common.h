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
// xor-butterfly over groups of W consecutive lanes (W a power of two <= 64)
template <int W>
__device__ __forceinline__ float group_max(float v) {
#pragma unroll
  for (int o = W / 2; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
template <int W>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int o = W / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

}  // namespace lfs
