// q/k RMSNorm + half-split RoPE of one token's fused qkv row
// (model/attention/GQA.py:39-40, 80-82; model/attention/utils.py:34-45): the
// device code shared by qk_norm_rope_store (fused.hip) and the decode
// attention that runs it as its prologue (paged_kv.hip), so that both give
// the same bits.
#pragma once

#include "common.h"

namespace lfs {

// torch's elementwise ops round every product and sum on its own: no
// contraction into FMAs where the reference computes two ops
__device__ __forceinline__ float mul_rn(float a, float b) { return __fmul_rn(a, b); }
__device__ __forceinline__ float add_rn(float a, float b) { return __fadd_rn(a, b); }
__device__ __forceinline__ float sub_rn(float a, float b) { return __fsub_rn(a, b); }

// Units per thread of qk_norm_rope_store.  A "unit" is one head's pair of
// 8-element chunks (d0..d0+7 and D/2+d0..D/2+d0+7) that RoPE combines; q has
// Hq*D/16 units, k Hkv*D/16.  Thread tid < 256 owns units tid, tid + 256,
// ... (at most UPT); the sums run in that order whatever UPT is, so UPT = 1
// gives the same bits as UPT = 4 whenever there are at most 256 units.
constexpr int kRopeUPT = 4;

// One token row, in phases so that a caller can issue every load early and
// do the arithmetic later:
//   init(...)       the shape and the thread (load(row, ...) = init + load(row));
//   load(row, ...)  issues the loads of the thread's units of q and k;
//   load_weights(q_weight, k_weight), load_rope(cs)  those of the units'
//                   norm weights and of the token's RoPE row
//                   cs = [cos(0..D/2) | sin(0..D/2)];
//   finish(...)     q' = bf16(q_weight * q * rsqrt(mean(q^2) + eps)) over
//                   all Hq*D values, k' likewise over Hkv*D; then per head
//                   y1 = x1*c - x2*s, y2 = x2*c + x1*s in fp32, with
//                   c, s = cs[d], cs[D/2 + d], and
//                   emit(isq, h, d0, lo, hi) for unit (h, d0) of q (isq) or
//                   k: lo = bf16 y1[d0..d0+7], hi = bf16 y2[d0..d0+7]
//                   (elements D/2+d0..).
// Threads tid >= 256 load and emit nothing, but every thread of the
// workgroup must call finish (it holds one barrier); red: 8 floats of LDS.
template <int UPT>
struct RopeRow {
  uint4 ra[UPT], rb[UPT];
  float w1[UPT][8], w2[UPT][8], c1[UPT][8], s1[UPT][8];  // the units' weights and cos / sin
  int Hq, Hkv, D, tid;

  __device__ __forceinline__ static void load8(const float* p, float* f) {
    const float4 x = *reinterpret_cast<const float4*>(p), y = *reinterpret_cast<const float4*>(p + 4);
    f[0] = x.x; f[1] = x.y; f[2] = x.z; f[3] = x.w;
    f[4] = y.x; f[5] = y.y; f[6] = y.z; f[7] = y.w;
  }

  __device__ __forceinline__ bool valid(int i) const {
    return tid < 256 && tid + 256 * i < (Hq + Hkv) * (D / 16);
  }
  __device__ __forceinline__ void unit(int i, bool& isq, int& h, int& d0) const {
    const int upr = D / 16, uq = Hq * upr;
    const int u = tid + 256 * i;
    isq = u < uq;
    const int uu = isq ? u : u - uq;
    h = uu / upr;
    d0 = (uu % upr) * 8;
  }

  __device__ __forceinline__ void init(int Hq_, int Hkv_, int D_, int tid_) {
    Hq = Hq_;
    Hkv = Hkv_;
    D = D_;
    tid = tid_;
  }
  __device__ __forceinline__ void load(const uint16_t* __restrict__ row, int Hq_, int Hkv_, int D_, int tid_) {
    init(Hq_, Hkv_, D_, tid_);
    load(row);
  }
  // after init()
  __device__ __forceinline__ void load(const uint16_t* __restrict__ row) {
#pragma unroll
    for (int i = 0; i < UPT; ++i) {
      ra[i] = rb[i] = make_uint4(0, 0, 0, 0);
      if (valid(i)) {
        bool isq;
        int h, d0;
        unit(i, isq, h, d0);
        const uint16_t* src = row + (isq ? 0 : Hq * D) + h * D;
        ra[i] = *reinterpret_cast<const uint4*>(src + d0);
        rb[i] = *reinterpret_cast<const uint4*>(src + D / 2 + d0);
      }
    }
  }

  __device__ __forceinline__ void load_weights(const float* __restrict__ qw, const float* __restrict__ kw) {
#pragma unroll
    for (int i = 0; i < UPT; ++i) {
      if (valid(i)) {
        bool isq;
        int h, d0;
        unit(i, isq, h, d0);
        const float* wt = (isq ? qw : kw) + h * D;
        load8(wt + d0, w1[i]);
        load8(wt + D / 2 + d0, w2[i]);
      }
    }
  }
  __device__ __forceinline__ void load_rope(const float* __restrict__ cs) {
#pragma unroll
    for (int i = 0; i < UPT; ++i) {
      if (valid(i)) {
        bool isq;
        int h, d0;
        unit(i, isq, h, d0);
        load8(cs + d0, c1[i]);
        load8(cs + D / 2 + d0, s1[i]);
      }
    }
  }

  template <class Emit>
  __device__ __forceinline__ void finish(float eps, float* red, Emit&& emit) const {
    float a[UPT][8], b[UPT][8];
    float ssq = 0.f, ssk = 0.f;
#pragma unroll
    for (int i = 0; i < UPT; ++i) {
      if (valid(i)) {
        bool isq;
        int h, d0;
        unit(i, isq, h, d0);
        unpack8(ra[i], a[i]);
        unpack8(rb[i], b[i]);
        float s = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) s = add_rn(s, add_rn(mul_rn(a[i][e], a[i][e]), mul_rn(b[i][e], b[i][e])));
        if (isq) ssq = add_rn(ssq, s); else ssk = add_rn(ssk, s);
      }
    }
    // the two sums over the first four waves
    ssq = group_sum<64>(ssq);
    ssk = group_sum<64>(ssk);
    const int wave = tid >> 6;
    if (tid < 256 && (tid & 63) == 0) {
      red[wave] = ssq;
      red[4 + wave] = ssk;
    }
    __syncthreads();
    const float tq = add_rn(add_rn(red[0], red[1]), add_rn(red[2], red[3]));
    const float tk = add_rn(add_rn(red[4], red[5]), add_rn(red[6], red[7]));
    const float invq = rsqrtf(add_rn(mul_rn(tq, 1.0f / (float)(Hq * D)), eps));
    const float invk = rsqrtf(add_rn(mul_rn(tk, 1.0f / (float)(Hkv * D)), eps));
#pragma unroll
    for (int i = 0; i < UPT; ++i) {
      if (valid(i)) {
        bool isq;
        int h, d0;
        unit(i, isq, h, d0);
        const float inv = isq ? invq : invk;
        float y1[8], y2[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          // norm output rounded to bf16 (the norm returns the input dtype)
          const float x1 = bf16_to_f32(f32_to_bf16(mul_rn(mul_rn(w1[i][e], a[i][e]), inv)));
          const float x2 = bf16_to_f32(f32_to_bf16(mul_rn(mul_rn(w2[i][e], b[i][e]), inv)));
          const float c = c1[i][e], s = s1[i][e];
          y1[e] = sub_rn(mul_rn(x1, c), mul_rn(x2, s));
          y2[e] = add_rn(mul_rn(x2, c), mul_rn(x1, s));
        }
        uint4 o1, o2;
        o1.x = pack_bf16x2(y1[0], y1[1]); o1.y = pack_bf16x2(y1[2], y1[3]);
        o1.z = pack_bf16x2(y1[4], y1[5]); o1.w = pack_bf16x2(y1[6], y1[7]);
        o2.x = pack_bf16x2(y2[0], y2[1]); o2.y = pack_bf16x2(y2[2], y2[3]);
        o2.z = pack_bf16x2(y2[4], y2[5]); o2.w = pack_bf16x2(y2[6], y2[7]);
        emit(isq, h, d0, o1, o2);
      }
    }
  }
};

}  // namespace lfs
