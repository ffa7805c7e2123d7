// Row-wise fused kernels of the paged GQA + MoE decode step (gfx950).
//
// Each replaces a chain of small elementwise / reduction launches around the
// FP8 GEMMs with one launch that reads its rows once:
//
//  add_rmsnorm        fused residual add + RMSNorm (model/utils.py:53-67),
//                     optionally also act_quant of the normalised row
//                     (model/attention/utils.py:129-139) for the next FP8
//                     linear.
//  qk_norm_rope_store q_norm over d_model and k_norm over Hkv*D (fp32, as
//                     torch.nn.RMSNorm, model/attention/GQA.py:39-40, 80-81),
//                     half-split RoPE (model/attention/utils.py:34-45) of q
//                     and k, q to its own buffer, k and v to the paged cache
//                     slot (engine/model_runner.py:226-230, :261).
//  moe_route          sigmoid gate, top-k of the biased logits, weights
//                     renormalised over the chosen experts
//                     (model/architecture/moe.py:45-90) as a dense [T, E+S]
//                     matrix (shared experts weight 1), and the routed bias
//                     sum_e w[t,e] * b2[e,:] of the experts' down projections.
//  swiglu_quant       silu(w1 x) * (w3 x) with the reference's bf16 roundings
//                     (model/architecture/mlp.py:60-67), act_quant of the
//                     result per 128 group, each group's scale multiplied by
//                     the token's routing weight for that expert.
//
// Rounding follows the torch ops they replace: fp32 math, products and sums
// as separate correctly rounded operations (no contraction into FMAs where
// torch computes two ops), bf16 round-to-nearest-even where torch stores
// bf16.  Row reductions (the RMS mean, the gate dot products) are summed in a
// different order than torch's reduction kernels, so their results can differ
// in the last fp32 bit.
#include "common.h"
#include "rope.h"

namespace lfs {
namespace {

// (best, bi) of the whole wave in every lane: the largest value, ties to
// the lowest index -- a total order, so the butterfly's pairing does not
// change the result.
template <int O>
__device__ __forceinline__ void argmax_step(float& best, int& bi) {
  const float ob = as_float(xor_partner<O>(__float_as_int(best)));
  const int oi = xor_partner<O>(bi);
  if (ob > best || (ob == best && oi < bi)) {
    best = ob;
    bi = oi;
  }
}
__device__ __forceinline__ void wave_argmax(float& best, int& bi) {
  argmax_step<32>(best, bi);
  argmax_step<16>(best, bi);
  argmax_step<8>(best, bi);
  argmax_step<4>(best, bi);
  argmax_step<2>(best, bi);
  argmax_step<1>(best, bi);
}
// v of lane `src` (wave-uniform)
__device__ __forceinline__ float lane_value(float v, int src) {
  return as_float(__builtin_amdgcn_readlane(__float_as_int(v), __builtin_amdgcn_readfirstlane(src)));
}

// Sum over a workgroup of NW waves; every thread gets the total.
template <int NW>
__device__ __forceinline__ float block_sum(float v, float* red) {
  v = group_sum<64>(v);
  if (NW == 1) return v;
  const int wave = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[wave] = v;
  __syncthreads();
  float t = 0.f;
#pragma unroll
  for (int w = 0; w < NW; ++w) t += red[w];
  return t;
}

// ------------------------------------------------------------ add_rmsnorm --
// One workgroup of 128 threads per row; thread c handles 16-byte chunks
// c, c + 128, ... (CPT of them).  With quantisation, a 128-element group is
// 16 consecutive chunks, which sit in 16 consecutive lanes of one wave.
// (h_lds: optionally also the bf16 output row, for a consumer in the same
// workgroup)
// x from split-K partials: the row is bf16(sum of nparts fp32 partial rows
// in order from 0.f, plus the bias), the value and rounding splitk_reduce8
// writes for the same partials (parts[s][row][col], s < nparts, rows MN
// floats apart; bias null, a vector (bias_ld 0) or a per-row matrix).
struct RowParts {
  const float* parts;
  int nparts;
  int64_t MN;
  const float* bias;
  int64_t bias_ld;
};

__device__ __forceinline__ void parts_chunk(const RowParts& rp, int64_t row, int d, int c, float (&f)[8]) {
  const float* src = rp.parts + row * d + c * 8;
  float v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int s0 = 0; s0 < rp.nparts; s0 += 8) {
    float4 lo[8], hi[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if (s0 + j < rp.nparts) {
        lo[j] = *reinterpret_cast<const float4*>(src + (s0 + j) * rp.MN);
        hi[j] = *reinterpret_cast<const float4*>(src + (s0 + j) * rp.MN + 4);
      }
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if (s0 + j < rp.nparts) {
        v[0] += lo[j].x; v[1] += lo[j].y; v[2] += lo[j].z; v[3] += lo[j].w;
        v[4] += hi[j].x; v[5] += hi[j].y; v[6] += hi[j].z; v[7] += hi[j].w;
      }
    }
  }
  if (rp.bias != nullptr) {
    const float* b = rp.bias + (rp.bias_ld ? row * rp.bias_ld : 0) + c * 8;
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] += b[e];
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) f[e] = bf16_to_f32(f32_to_bf16(v[e]));
}

template <int CPT, bool QUANT, int NW = 2, bool PARTS = false>
__device__ __forceinline__ void add_rmsnorm_row(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ residual,
    const float* __restrict__ w, uint16_t* __restrict__ out, uint16_t* __restrict__ res_out,
    uint8_t* __restrict__ q, float* __restrict__ qs, int d, float eps, int64_t row, float* red,
    uint16_t* h_lds, const RowParts& rp = RowParts{}) {
  const int cpr = d / 8;
  float f[CPT][8];
  float4 wq[CPT][2];  // weights, loaded before the reduction
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int c = threadIdx.x + 128 * i;
    if (c < cpr && threadIdx.x < 128) {  // chunks on the first 128 threads only
      wq[i][0] = *reinterpret_cast<const float4*>(w + c * 8);
      wq[i][1] = *reinterpret_cast<const float4*>(w + c * 8 + 4);
      if constexpr (PARTS) parts_chunk(rp, row, d, c, f[i]);
      else unpack8(*reinterpret_cast<const uint4*>(x + row * d + c * 8), f[i]);
      if (residual != nullptr) {
        float r[8];
        unpack8(*reinterpret_cast<const uint4*>(residual + row * d + c * 8), r);
#pragma unroll
        for (int e = 0; e < 8; ++e) f[i][e] = add_rn(f[i][e], r[e]);
        uint4 o;
        o.x = pack_bf16x2(f[i][0], f[i][1]);
        o.y = pack_bf16x2(f[i][2], f[i][3]);
        o.z = pack_bf16x2(f[i][4], f[i][5]);
        o.w = pack_bf16x2(f[i][6], f[i][7]);
        *reinterpret_cast<uint4*>(res_out + row * d + c * 8) = o;
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) ss = add_rn(ss, mul_rn(f[i][e], f[i][e]));
    }
  }
  const float total = block_sum<NW>(ss, red);  // NW waves (threads past 128 hold no chunk)
  const float inv = rsqrtf(add_rn(mul_rn(total, 1.0f / (float)d), eps));
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int c = threadIdx.x + 128 * i;
    const bool ok = c < cpr && threadIdx.x < 128;
    float y[8];
    if (ok) {
      const float4 w0 = wq[i][0], w1 = wq[i][1];
      const float wv[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
      for (int e = 0; e < 8; ++e) y[e] = bf16_to_f32(f32_to_bf16(mul_rn(mul_rn(wv[e], f[i][e]), inv)));
      uint4 o;
      o.x = pack_bf16x2(y[0], y[1]);
      o.y = pack_bf16x2(y[2], y[3]);
      o.z = pack_bf16x2(y[4], y[5]);
      o.w = pack_bf16x2(y[6], y[7]);
      if (out != nullptr) *reinterpret_cast<uint4*>(out + row * d + c * 8) = o;
      if (h_lds != nullptr) *reinterpret_cast<uint4*>(h_lds + c * 8) = o;
    }
    if (QUANT) {
      float amax = 0.f;
      if (ok) {
#pragma unroll
        for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(y[e]));
      }
      amax = group_max<16>(amax);
      if (ok) {
        const float sc = scale_from_amax(amax, false);
        *reinterpret_cast<uint2*>(q + row * d + c * 8) = quant8(y, sc);
        if ((c & 15) == 0) qs[row * (d / 128) + c / 16] = sc;
      }
    }
  }
}

template <int CPT, bool QUANT>
__global__ __launch_bounds__(128) void add_rmsnorm_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ residual,
    const float* __restrict__ w, uint16_t* __restrict__ out, uint16_t* __restrict__ res_out,
    uint8_t* __restrict__ q, float* __restrict__ qs, int d, float eps) {
  __shared__ float red[2];
  add_rmsnorm_row<CPT, QUANT>(x, residual, w, out, res_out, q, qs, d, eps, blockIdx.x, red, nullptr);
}

// add_rmsnorm whose x is the split-K reduction of a GEMM (its partials and
// bias), so that the reduction needs no launch of its own
template <int CPT, bool QUANT>
__global__ __launch_bounds__(128) void add_rmsnorm_parts_kernel(
    RowParts rp, const uint16_t* __restrict__ residual, const float* __restrict__ w, uint16_t* __restrict__ out,
    uint16_t* __restrict__ res_out, uint8_t* __restrict__ q, float* __restrict__ qs, int d, float eps) {
  __shared__ float red[2];
  add_rmsnorm_row<CPT, QUANT, 2, true>(nullptr, residual, w, out, res_out, q, qs, d, eps, blockIdx.x, red,
                                       nullptr, rp);
}

// ----------------------------------------------------- qk_norm_rope_store --
// One workgroup of 256 threads per token (RopeRow: thread t owns the units
// t, t + 256, ... of q then k).
__global__ __launch_bounds__(256) void qk_norm_rope_store_kernel(
    const uint16_t* __restrict__ qkv, int64_t ld, const float* __restrict__ qw,
    const float* __restrict__ kw, const float* __restrict__ cos_sin, const int64_t* __restrict__ pos,
    const int64_t* __restrict__ slots, uint16_t* __restrict__ q_out, uint16_t* __restrict__ kc,
    uint16_t* __restrict__ vc, int Hq, int Hkv, int D, int64_t num_slots, int64_t max_pos,
    float eps) {
  __shared__ float red[8];
  const int64_t t = blockIdx.x;
  const uint16_t* row = qkv + t * ld;
  const int half = D / 2;
  int64_t p = pos[t];
  p = p < 0 ? 0 : (p >= max_pos ? max_pos - 1 : p);
  const float* cs = cos_sin + p * D;  // [cos(0..D/2) | sin(0..D/2)]
  const int64_t slot = slots != nullptr ? slots[t] : -1;
  const bool store = slot >= 0 && slot < num_slots;
  // v: straight copy into the cache slot (Hkv*D/8 chunks)
  if (store) {
    const int64_t dst = slot * (int64_t)Hkv * D;
    for (int c = threadIdx.x; c < Hkv * D / 8; c += 256)
      *reinterpret_cast<uint4*>(vc + dst + c * 8) =
          *reinterpret_cast<const uint4*>(row + (Hq + Hkv) * D + c * 8);
  }
  RopeRow<kRopeUPT> rr;
  rr.load(row, Hq, Hkv, D, threadIdx.x);
  rr.load_weights(qw, kw);
  rr.load_rope(cs);
  rr.finish(eps, red, [&](bool isq, int h, int d0, const uint4& o1, const uint4& o2) {
    uint16_t* dst;
    if (isq) {
      dst = q_out + (t * Hq + h) * D;
    } else {
      if (!store) return;
      dst = kc + (slot * Hkv + h) * D;
    }
    *reinterpret_cast<uint4*>(dst + d0) = o1;
    *reinterpret_cast<uint4*>(dst + half + d0) = o2;
  });
}

// --------------------------------------------------------------- moe_route --
// Large batches: four tokens per workgroup.  Phase 1, one wave per token: lane l sums the
// products of 16-byte chunks l, l+64, ... of the token row with the same
// chunks of up to 8 experts' gate rows at a time, then a butterfly per
// expert leaves expert e's logit in lane e; the top k is a repeated wave
// argmax.  Phase 2, the whole workgroup: the routed bias of the four tokens,
// one column per thread and pass (each b2 value loaded once for the four).
constexpr int kMaxExperts = 64;
constexpr int kRouteTokens = 4;  // tokens (waves) per workgroup
constexpr int kRouteSmallT = 1024;  // up to this many tokens: one workgroup per token

__global__ __launch_bounds__(64 * kRouteTokens) void moe_route_kernel(
    const uint16_t* __restrict__ h, const uint16_t* __restrict__ gw, const float* __restrict__ ebias,
    const float* __restrict__ b2, float* __restrict__ dense, float* __restrict__ bias_out, int64_t T, int d,
    int E, int S, int top_k, int64_t* __restrict__ topk_idx, float* __restrict__ topk_w) {
  __shared__ float wsel[kRouteTokens][kMaxExperts];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t t0 = (int64_t)blockIdx.x * kRouteTokens;
  const int64_t t = t0 + wave;
  if (t < T) {
    const int cpr = d / 8;
    const uint16_t* hrow = h + t * d;
    float logit = 0.f;  // lane e: expert e's logit
    for (int e0 = 0; e0 < E; e0 += 8) {
      float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
      for (int c = lane; c < cpr; c += 64) {
        float hv[8];
        unpack8(*reinterpret_cast<const uint4*>(hrow + c * 8), hv);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          if (e0 + j >= E) break;
          float gv[8];
          unpack8(*reinterpret_cast<const uint4*>(gw + (int64_t)(e0 + j) * d + c * 8), gv);
#pragma unroll
          for (int i = 0; i < 8; ++i) acc[j] = add_rn(acc[j], mul_rn(hv[i], gv[i]));
        }
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        if (e0 + j >= E) break;
        const float tot = group_sum<64>(acc[j]);
        if (lane == e0 + j) logit = tot;
      }
    }
    const bool valid = lane < E;
    // sigmoid score and biased logit of expert `lane`
    const float score = valid ? 1.0f / (1.0f + expf(-logit)) : 0.f;
    const float key = valid ? add_rn(logit, ebias[lane]) : -INFINITY;
    // top-k by repeated wave argmax (ties: lowest expert index)
    bool chosen = false;
    int myk = -1;  // pick order of this lane's expert
    float wsum = 0.f;
    for (int k = 0; k < top_k; ++k) {
      float best = chosen ? -INFINITY : key;
      int bi = valid && !chosen ? lane : kMaxExperts;
      wave_argmax(best, bi);
      if (lane == bi) { chosen = true; myk = k; }
      wsum = add_rn(wsum, lane_value(score, bi < 64 ? bi : 0) * (bi < 64 ? 1.f : 0.f));
    }
    float wgt = chosen ? score : 0.f;
    if (top_k > 1) wgt = chosen ? wgt / add_rn(wsum, 1e-10f) : 0.f;
    const float v = lane < E ? wgt : (lane < E + S ? 1.0f : 0.f);  // lane e: weight of expert e
    wsel[wave][lane] = v;
    if (dense != nullptr && lane < E + S) dense[t * (E + S) + lane] = v;
    // the picks in index form (the reference gate's topk_idx / topk_weight)
    if (topk_idx != nullptr && chosen) {
      topk_idx[t * top_k + myk] = lane;
      topk_w[t * top_k + myk] = wgt;
    }
  } else {
    wsel[wave][lane] = 0.f;
  }
  if (bias_out == nullptr) return;  // uniform: no barrier below is skipped by part of the workgroup
  __syncthreads();
  // routed bias: sum_e w[e] * b2[e, n], experts in index order
  const int EE = E + S;
  if (EE <= 16) {
    // every b2 load of a pass issued before the first use: one memory latency
    for (int n0 = 0; n0 < d; n0 += 64 * kRouteTokens * 4) {
      float bv[16][4];
#pragma unroll
      for (int e = 0; e < 16; ++e)
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const int n = n0 + threadIdx.x + 64 * kRouteTokens * c;
          bv[e][c] = (e < EE && n < d) ? b2[(int64_t)e * d + n] : 0.f;
        }
#pragma unroll
      for (int w = 0; w < kRouteTokens; ++w) {
        float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          if (e < EE) {
            const float we = wsel[w][e];
#pragma unroll
            for (int c = 0; c < 4; ++c) acc[c] = add_rn(acc[c], mul_rn(we, bv[e][c]));
          }
        }
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const int n = n0 + threadIdx.x + 64 * kRouteTokens * c;
          if (n < d && t0 + w < T) bias_out[(t0 + w) * d + n] = acc[c];
        }
      }
    }
    return;
  }
  for (int n0 = 0; n0 < d; n0 += 64 * kRouteTokens * 4) {
    float acc[kRouteTokens][4] = {};
    for (int e0 = 0; e0 < EE; e0 += 2) {
      float bv[2][4];
#pragma unroll
      for (int x = 0; x < 2; ++x)
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const int n = n0 + threadIdx.x + 64 * kRouteTokens * c;
          bv[x][c] = (e0 + x < EE && n < d) ? b2[(int64_t)(e0 + x) * d + n] : 0.f;
        }
#pragma unroll
      for (int x = 0; x < 2; ++x) {
        if (e0 + x < EE) {
#pragma unroll
          for (int w = 0; w < kRouteTokens; ++w) {
            const float we = wsel[w][e0 + x];
#pragma unroll
            for (int c = 0; c < 4; ++c) acc[w][c] = add_rn(acc[w][c], mul_rn(we, bv[x][c]));
          }
        }
      }
    }
#pragma unroll
    for (int w = 0; w < kRouteTokens; ++w) {
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int n = n0 + threadIdx.x + 64 * kRouteTokens * c;
        if (n < d && t0 + w < T) bias_out[(t0 + w) * d + n] = acc[w][c];
      }
    }
  }
}

// Small batches (decode): one workgroup of 4 waves per token, so that the
// tokens spread over as many CUs as possible.
// One token's gate: h_row (global or LDS) of d bf16 values; nthr threads
// (whole waves).  Wave w of the workgroup computes the logits of experts w,
// w + nwaves, ... (lane l sums chunks l, l+64, ... then a butterfly: the same
// arithmetic whatever the wave count); wave 0 picks the top k; all threads
// form the routed bias.
__device__ __forceinline__ void route_token(
    const uint16_t* h_row, const uint16_t* __restrict__ gw, const float* __restrict__ ebias,
    const float* __restrict__ b2, float* __restrict__ dense, float* __restrict__ bias_out, int d,
    int E, int S, int top_k, int64_t* __restrict__ topk_idx, float* __restrict__ topk_w, int64_t t,
    float* logits, float* wsel, int* sel) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nwaves = blockDim.x >> 6;
  const int cpr = d / 8;
  for (int e = wave; e < E; e += nwaves) {
    float acc = 0.f;
    for (int c = lane; c < cpr; c += 64) {
      float hv[8], gv[8];
      unpack8(*reinterpret_cast<const uint4*>(h_row + c * 8), hv);
      unpack8(*reinterpret_cast<const uint4*>(gw + (int64_t)e * d + c * 8), gv);
#pragma unroll
      for (int i = 0; i < 8; ++i) acc = add_rn(acc, mul_rn(hv[i], gv[i]));
    }
    acc = group_sum<64>(acc);
    if (lane == 0) logits[e] = acc;
  }
  __syncthreads();
  if (wave == 0) {
    const bool valid = lane < E;
    const float logit = valid ? logits[lane] : 0.f;
    // sigmoid score and biased logit of expert `lane`
    const float score = valid ? 1.0f / (1.0f + expf(-logit)) : 0.f;
    const float key = valid ? add_rn(logit, ebias[lane]) : -INFINITY;
    // top-k by repeated wave argmax (ties: lowest expert index)
    bool chosen = false;
    float wsum = 0.f;
    for (int k = 0; k < top_k; ++k) {
      float best = chosen ? -INFINITY : key;
      int bi = valid && !chosen ? lane : kMaxExperts;
      wave_argmax(best, bi);
      if (lane == bi) chosen = true;
      if (lane == 0) sel[k] = bi;
      wsum = add_rn(wsum, lane_value(score, bi < 64 ? bi : 0) * (bi < 64 ? 1.f : 0.f));
    }
    float wgt = chosen ? score : 0.f;
    if (top_k > 1) wgt = chosen ? wgt / add_rn(wsum, 1e-10f) : 0.f;
    if (lane < E + S) {
      const float v = lane < E ? wgt : 1.0f;
      if (dense != nullptr) dense[t * (E + S) + lane] = v;
      wsel[lane] = v;
    }
  }
  __syncthreads();
  // the picks in index form (the reference gate's topk_idx / topk_weight)
  if (topk_idx != nullptr && (int)threadIdx.x < top_k) {
    topk_idx[t * top_k + threadIdx.x] = sel[threadIdx.x];
    topk_w[t * top_k + threadIdx.x] = wsel[sel[threadIdx.x]];
  }
  // routed bias: sum_e w[e] * b2[e, n], experts in index order
  if (bias_out == nullptr) return;
  for (int n = threadIdx.x; n < d; n += blockDim.x) {
    float acc = 0.f;
    for (int e = 0; e < E + S; ++e) acc = add_rn(acc, mul_rn(wsel[e], b2[(int64_t)e * d + n]));
    bias_out[t * d + n] = acc;
  }
}

__global__ __launch_bounds__(256) void moe_route_token_kernel(
    const uint16_t* __restrict__ h, const uint16_t* __restrict__ gw, const float* __restrict__ ebias,
    const float* __restrict__ b2, float* __restrict__ dense, float* __restrict__ bias_out, int d,
    int E, int S, int top_k, int64_t* __restrict__ topk_idx, float* __restrict__ topk_w) {
  __shared__ float logits[kMaxExperts];
  __shared__ float wsel[kMaxExperts];
  __shared__ int sel[kMaxExperts];
  const int64_t t = blockIdx.x;
  route_token(h + t * d, gw, ebias, b2, dense, bias_out, d, E, S, top_k, topk_idx, topk_w, t, logits, wsel, sel);
}

// The decode step's ffn_norm and MoE gate in one launch: add_rmsnorm of the
// row (with its act_quant, the expert GEMMs' input), the bf16 row kept in
// LDS, then the gate over it -- bit-identical to add_rmsnorm followed by
// moe_route (the same arithmetic in the same order).  One workgroup of 256
// threads per token: the norm's chunks on the first 128 (as add_rmsnorm),
// the gate on all four waves (as moe_route; with two waves it took 14.5 us
// against 4.8 + 8.2 us for the separate launches).
constexpr int kNormRouteMaxD = 8192;
// Gate rows and down biases staged in LDS by the waves the norm leaves idle
// (threads 128..255), when both fit: their loads then overlap the norm's
// instead of following it (two dependent round trips fewer).
constexpr int kRouteStageBytes = 48 * 1024;
constexpr int kRouteStagePerThread = kRouteStageBytes / 16 / 128;  // 16-byte chunks per staging thread

template <int CPT>
__global__ __launch_bounds__(256) void add_rmsnorm_route_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ residual, const float* __restrict__ w,
    uint16_t* __restrict__ out, uint16_t* __restrict__ res_out, uint8_t* __restrict__ q, float* __restrict__ qs,
    int d, float eps, const uint16_t* __restrict__ gw, const float* __restrict__ ebias,
    const float* __restrict__ b2, float* __restrict__ dense, float* __restrict__ bias_out, int E, int S,
    int top_k) {
  __shared__ float red[4];
  __shared__ __attribute__((aligned(16))) uint16_t h_lds[kNormRouteMaxD];
  __shared__ __attribute__((aligned(16))) uint4 stage[kRouteStageBytes / 16];
  __shared__ float logits[kMaxExperts];
  __shared__ float wsel[kMaxExperts];
  __shared__ int sel[kMaxExperts];
  const int64_t t = blockIdx.x;
  // gw: E x d bf16 (16-byte aligned, d % 8 == 0: checked on the host); b2:
  // (E+S) x d fp32 when given and 16-byte aligned
  const int gw16 = E * d / 8;
  const bool b2_ok = b2 != nullptr && ((uintptr_t)b2 & 15u) == 0;
  const int b216 = b2_ok ? (E + S) * d / 4 : 0;
  const bool staged = gw16 + b216 <= kRouteStageBytes / 16;
  if (staged && threadIdx.x >= 128) {
    const uint4* gsrc = reinterpret_cast<const uint4*>(gw);
    const uint4* bsrc = reinterpret_cast<const uint4*>(b2);
    const int tot = gw16 + b216;
    uint4 v[kRouteStagePerThread];
#pragma unroll
    for (int k = 0; k < kRouteStagePerThread; ++k) {
      const int i = (int)threadIdx.x - 128 + 128 * k;
      const uint4* src = i < gw16 ? gsrc + i : bsrc + (i - gw16);
      v[k] = i < tot ? *src : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int k = 0; k < kRouteStagePerThread; ++k) {
      const int i = (int)threadIdx.x - 128 + 128 * k;
      if (i < tot) stage[i] = v[k];
    }
  }
  add_rmsnorm_row<CPT, true, 4>(x, residual, w, out, res_out, q, qs, d, eps, t, red, h_lds);
  __syncthreads();  // (also: the staged rows are visible)
  const uint16_t* gws = staged ? reinterpret_cast<const uint16_t*>(stage) : gw;
  const float* b2s = staged && b2_ok ? reinterpret_cast<const float*>(stage + gw16) : b2;
  route_token(h_lds, gws, ebias, b2s, dense, bias_out, d, E, S, top_k, nullptr, nullptr, t, logits, wsel, sel);
}

// ------------------------------------------------------------ swiglu_quant --
// One wave per (token, expert), workgroup index t * E + e; lane l handles
// chunks l, l+64, ... of the expert's F outputs (a 128 group = 16
// consecutive lanes).
__global__ __launch_bounds__(64) void swiglu_quant_kernel(
    const uint16_t* __restrict__ h13, const float* __restrict__ route, uint8_t* __restrict__ q,
    float* __restrict__ qs, int E, int F) {
  const int64_t t = blockIdx.x / E;
  const int e = (int)(blockIdx.x - t * E);
  const int lane = threadIdx.x;
  const uint16_t* a = h13 + (t * E + e) * 2 * (int64_t)F;
  const uint16_t* b = a + F;
  const float r = route[t * E + e];
  const int64_t orow = t * (int64_t)E * F + (int64_t)e * F;
  for (int c = lane; c < F / 8; c += 64) {
    float av[8], bv[8], g[8];
    unpack8(*reinterpret_cast<const uint4*>(a + c * 8), av);
    unpack8(*reinterpret_cast<const uint4*>(b + c * 8), bv);
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float sl = bf16_to_f32(f32_to_bf16(av[i] / add_rn(1.0f, expf(-av[i]))));
      g[i] = bf16_to_f32(f32_to_bf16(mul_rn(sl, bv[i])));
      amax = fmaxf(amax, fabsf(g[i]));
    }
    amax = group_max<16>(amax);
    const float sc = scale_from_amax(amax, false);
    *reinterpret_cast<uint2*>(q + orow + c * 8) = quant8(g, sc);
    if ((c & 15) == 0) qs[(orow + c * 8) / 128] = mul_rn(sc, r);
  }
}

template <int CPT>
int launch_add_rmsnorm(bool quant, const void* x, const void* residual, const float* w, void* out,
                       void* res_out, void* q, float* qs, int64_t T, int d, float eps,
                       hipStream_t st) {
  if (quant)
    hipLaunchKernelGGL((add_rmsnorm_kernel<CPT, true>), dim3((unsigned)T), dim3(128), 0, st,
                       (const uint16_t*)x, (const uint16_t*)residual, w, (uint16_t*)out,
                       (uint16_t*)res_out, (uint8_t*)q, qs, d, eps);
  else
    hipLaunchKernelGGL((add_rmsnorm_kernel<CPT, false>), dim3((unsigned)T), dim3(128), 0, st,
                       (const uint16_t*)x, (const uint16_t*)residual, w, (uint16_t*)out,
                       (uint16_t*)res_out, (uint8_t*)q, qs, d, eps);
  return check_launch("add_rmsnorm");
}

template <int CPT>
int launch_add_rmsnorm_parts(const RowParts& rp, const void* residual, const float* w, void* out, void* res_out,
                             void* q, float* qs, int64_t T, int d, float eps, hipStream_t st) {
  if (q != nullptr)
    hipLaunchKernelGGL((add_rmsnorm_parts_kernel<CPT, true>), dim3((unsigned)T), dim3(128), 0, st, rp,
                       (const uint16_t*)residual, w, (uint16_t*)out, (uint16_t*)res_out, (uint8_t*)q, qs, d, eps);
  else
    hipLaunchKernelGGL((add_rmsnorm_parts_kernel<CPT, false>), dim3((unsigned)T), dim3(128), 0, st, rp,
                       (const uint16_t*)residual, w, (uint16_t*)out, (uint16_t*)res_out, (uint8_t*)q, qs, d, eps);
  return check_launch("add_rmsnorm_partials");
}

}  // namespace
}  // namespace lfs

using namespace lfs;

extern "C" int lfs_add_rmsnorm(const void* x, const void* residual, const float* weight, void* out,
                               void* residual_out, void* q, float* q_scale, int64_t T, int32_t d,
                               float eps, void* stream) {
  LFS_REQUIRE(T >= 0 && d > 0, "add_rmsnorm: bad shape");
  LFS_REQUIRE(d % 8 == 0 && d <= 128 * 8 * 8, "add_rmsnorm: d=%d must be a multiple of 8 and <= 8192", d);
  LFS_REQUIRE((residual == nullptr) == (residual_out == nullptr),
              "add_rmsnorm: residual and residual_out go together");
  LFS_REQUIRE((q == nullptr) == (q_scale == nullptr), "add_rmsnorm: q and q_scale go together");
  LFS_REQUIRE(q == nullptr || d % 128 == 0, "add_rmsnorm: quantised output needs d %% 128 == 0");
  LFS_REQUIRE(out != nullptr || q != nullptr, "add_rmsnorm: no output");
  if (T == 0) return 0;
  LFS_REQUIRE(x && weight, "add_rmsnorm: null pointer");
  LFS_REQUIRE(((uintptr_t)x | (uintptr_t)residual | (uintptr_t)out | (uintptr_t)residual_out |
               (uintptr_t)weight | (uintptr_t)q) % 16 == 0,
              "add_rmsnorm: buffers must be 16-byte aligned");
  LFS_REQUIRE(T < (1ll << 31), "add_rmsnorm: too many rows");
  hipStream_t st = (hipStream_t)stream;
  const int cpr = d / 8;
  const bool quant = q != nullptr;
  if (cpr <= 128) return launch_add_rmsnorm<1>(quant, x, residual, weight, out, residual_out, q, q_scale, T, d, eps, st);
  if (cpr <= 256) return launch_add_rmsnorm<2>(quant, x, residual, weight, out, residual_out, q, q_scale, T, d, eps, st);
  if (cpr <= 512) return launch_add_rmsnorm<4>(quant, x, residual, weight, out, residual_out, q, q_scale, T, d, eps, st);
  return launch_add_rmsnorm<8>(quant, x, residual, weight, out, residual_out, q, q_scale, T, d, eps, st);
}

extern "C" int lfs_add_rmsnorm_partials(const float* parts, int32_t nparts, const float* bias, int64_t bias_ld,
                                        const void* residual, const float* weight, void* out, void* residual_out,
                                        void* q, float* q_scale, int64_t T, int32_t d, float eps, void* stream) {
  LFS_REQUIRE(T >= 0 && d > 0 && nparts >= 1, "add_rmsnorm_partials: bad shape");
  LFS_REQUIRE(d % 8 == 0 && d <= 128 * 8 * 8, "add_rmsnorm_partials: d=%d must be a multiple of 8 and <= 8192",
              d);
  LFS_REQUIRE((residual == nullptr) == (residual_out == nullptr),
              "add_rmsnorm_partials: residual and residual_out go together");
  LFS_REQUIRE((q == nullptr) == (q_scale == nullptr), "add_rmsnorm_partials: q and q_scale go together");
  LFS_REQUIRE(q == nullptr || d % 128 == 0, "add_rmsnorm_partials: quantised output needs d %% 128 == 0");
  LFS_REQUIRE(out != nullptr || q != nullptr, "add_rmsnorm_partials: no output");
  LFS_REQUIRE(bias_ld == 0 || (bias != nullptr && bias_ld >= d), "add_rmsnorm_partials: bias_ld must be 0 or >= d");
  if (T == 0) return 0;
  LFS_REQUIRE(parts && weight, "add_rmsnorm_partials: null pointer");
  LFS_REQUIRE(((uintptr_t)parts | (uintptr_t)residual | (uintptr_t)out | (uintptr_t)residual_out |
               (uintptr_t)weight | (uintptr_t)q) % 16 == 0,
              "add_rmsnorm_partials: buffers must be 16-byte aligned");
  LFS_REQUIRE(T < (1ll << 31), "add_rmsnorm_partials: too many rows");
  const RowParts rp{parts, nparts, T * d, bias, bias_ld};
  hipStream_t st = (hipStream_t)stream;
  const int cpr = d / 8;
  if (cpr <= 128) return launch_add_rmsnorm_parts<1>(rp, residual, weight, out, residual_out, q, q_scale, T, d, eps, st);
  if (cpr <= 256) return launch_add_rmsnorm_parts<2>(rp, residual, weight, out, residual_out, q, q_scale, T, d, eps, st);
  if (cpr <= 512) return launch_add_rmsnorm_parts<4>(rp, residual, weight, out, residual_out, q, q_scale, T, d, eps, st);
  return launch_add_rmsnorm_parts<8>(rp, residual, weight, out, residual_out, q, q_scale, T, d, eps, st);
}

extern "C" int lfs_qk_norm_rope_store(const void* qkv, int64_t ld, const float* q_weight,
                                      const float* k_weight, const float* cos_sin,
                                      const int64_t* positions, const int64_t* slot_mapping,
                                      void* q_out, void* k_cache, void* v_cache, int64_t T,
                                      int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                                      int64_t num_slots, int64_t max_positions, float eps,
                                      void* stream) {
  const int Hq = num_q_heads, Hkv = num_kv_heads, D = head_dim;
  LFS_REQUIRE(T >= 0 && Hq > 0 && Hkv > 0, "qk_norm_rope_store: bad shape");
  LFS_REQUIRE(D % 16 == 0 && D > 0 && D <= 512, "qk_norm_rope_store: head_dim=%d must be a multiple of 16", D);
  LFS_REQUIRE((int64_t)(Hq + Hkv) * D / 16 <= 256 * kRopeUPT,
              "qk_norm_rope_store: (Hq+Hkv)*D/16 must be <= %d", 256 * kRopeUPT);
  LFS_REQUIRE(ld >= (int64_t)(Hq + 2 * Hkv) * D && ld % 8 == 0, "qk_norm_rope_store: bad row stride");
  LFS_REQUIRE(max_positions > 0, "qk_norm_rope_store: empty RoPE table");
  if (T == 0) return 0;
  LFS_REQUIRE(qkv && q_weight && k_weight && cos_sin && positions && q_out,
              "qk_norm_rope_store: null pointer");
  LFS_REQUIRE(slot_mapping == nullptr || (k_cache && v_cache), "qk_norm_rope_store: null cache");
  LFS_REQUIRE(((uintptr_t)qkv | (uintptr_t)q_out | (uintptr_t)k_cache | (uintptr_t)v_cache) % 16 == 0,
              "qk_norm_rope_store: buffers must be 16-byte aligned");
  hipLaunchKernelGGL(qk_norm_rope_store_kernel, dim3((unsigned)T), dim3(256), 0, (hipStream_t)stream,
                     (const uint16_t*)qkv, ld, q_weight, k_weight, cos_sin, positions, slot_mapping,
                     (uint16_t*)q_out, (uint16_t*)k_cache, (uint16_t*)v_cache, Hq, Hkv, D, num_slots,
                     max_positions, eps);
  return check_launch("qk_norm_rope_store");
}

extern "C" int lfs_moe_route(const void* h, const void* gate_weight, const float* expert_bias,
                             const float* down_bias, float* dense_weights, float* bias_out, int64_t T,
                             int32_t d, int32_t num_experts, int32_t num_shared, int32_t top_k,
                             int64_t* topk_idx, float* topk_weight, void* stream) {
  LFS_REQUIRE(T >= 0 && d > 0 && d % 8 == 0, "moe_route: d=%d must be a positive multiple of 8", d);
  LFS_REQUIRE(num_experts > 0 && num_shared >= 0 && num_experts + num_shared <= kMaxExperts,
              "moe_route: at most %d experts", kMaxExperts);
  LFS_REQUIRE(top_k >= 1 && top_k <= num_experts, "moe_route: bad top_k");
  if (T == 0) return 0;
  LFS_REQUIRE(h && gate_weight && expert_bias, "moe_route: null pointer");
  LFS_REQUIRE(bias_out == nullptr || down_bias != nullptr, "moe_route: bias_out needs down_bias");
  LFS_REQUIRE(dense_weights != nullptr || topk_idx != nullptr, "moe_route: no output");
  LFS_REQUIRE(((uintptr_t)h | (uintptr_t)gate_weight) % 16 == 0, "moe_route: h and gate_weight must be 16-byte aligned");
  LFS_REQUIRE((topk_idx == nullptr) == (topk_weight == nullptr), "moe_route: topk_idx and topk_weight go together");
  LFS_REQUIRE(T < (1ll << 31), "moe_route: too many tokens");
  if (T <= kRouteSmallT)
    hipLaunchKernelGGL(moe_route_token_kernel, dim3((unsigned)T), dim3(256), 0, (hipStream_t)stream,
                       (const uint16_t*)h, (const uint16_t*)gate_weight, expert_bias, down_bias, dense_weights,
                       bias_out, d, num_experts, num_shared, top_k, topk_idx, topk_weight);
  else
    hipLaunchKernelGGL(moe_route_kernel, dim3((unsigned)((T + kRouteTokens - 1) / kRouteTokens)),
                       dim3(64 * kRouteTokens), 0, (hipStream_t)stream, (const uint16_t*)h,
                       (const uint16_t*)gate_weight, expert_bias, down_bias, dense_weights, bias_out, T, d,
                       num_experts, num_shared, top_k, topk_idx, topk_weight);
  return check_launch("moe_route");
}

extern "C" int lfs_add_rmsnorm_route(const void* x, const void* residual, const float* weight, void* out,
                                     void* residual_out, void* q, float* q_scale, int64_t T, int32_t d,
                                     float eps, const void* gate_weight, const float* expert_bias,
                                     const float* down_bias, float* dense_weights, float* bias_out,
                                     int32_t num_experts, int32_t num_shared, int32_t top_k, void* stream) {
  LFS_REQUIRE(T >= 0 && d > 0, "add_rmsnorm_route: bad shape");
  LFS_REQUIRE(d % 128 == 0 && d <= kNormRouteMaxD, "add_rmsnorm_route: d=%d must be a multiple of 128 and <= %d",
              d, kNormRouteMaxD);
  LFS_REQUIRE((residual == nullptr) == (residual_out == nullptr),
              "add_rmsnorm_route: residual and residual_out go together");
  LFS_REQUIRE(num_experts > 0 && num_shared >= 0 && num_experts + num_shared <= kMaxExperts,
              "add_rmsnorm_route: at most %d experts", kMaxExperts);
  LFS_REQUIRE(top_k >= 1 && top_k <= num_experts, "add_rmsnorm_route: bad top_k");
  if (T == 0) return 0;
  LFS_REQUIRE(x && weight && q && q_scale && gate_weight && expert_bias && dense_weights,
              "add_rmsnorm_route: null pointer");
  LFS_REQUIRE(bias_out == nullptr || down_bias != nullptr, "add_rmsnorm_route: bias_out needs down_bias");
  LFS_REQUIRE(((uintptr_t)x | (uintptr_t)residual | (uintptr_t)out | (uintptr_t)residual_out |
               (uintptr_t)weight | (uintptr_t)q | (uintptr_t)gate_weight) % 16 == 0,
              "add_rmsnorm_route: buffers must be 16-byte aligned");
  LFS_REQUIRE(T < (1ll << 31), "add_rmsnorm_route: too many rows");
  hipStream_t st = (hipStream_t)stream;
  const int cpr = d / 8;
#define LFS_NR(C)                                                                                              \
  hipLaunchKernelGGL((add_rmsnorm_route_kernel<C>), dim3((unsigned)T), dim3(256), 0, st, (const uint16_t*)x,      \
                     (const uint16_t*)residual, weight, (uint16_t*)out, (uint16_t*)residual_out, (uint8_t*)q,    \
                     q_scale, d, eps, (const uint16_t*)gate_weight, expert_bias, down_bias, dense_weights,      \
                     bias_out, num_experts, num_shared, top_k)
  if (cpr <= 128) LFS_NR(1);
  else if (cpr <= 256) LFS_NR(2);
  else if (cpr <= 512) LFS_NR(4);
  else LFS_NR(8);
#undef LFS_NR
  return check_launch("add_rmsnorm_route");
}

extern "C" int lfs_swiglu_quant(const void* h13, const float* route_weights, void* q, float* q_scale,
                                int64_t T, int32_t num_experts, int32_t d_ff, void* stream) {
  LFS_REQUIRE(T >= 0 && num_experts > 0, "swiglu_quant: bad shape");
  LFS_REQUIRE(d_ff > 0 && d_ff % 128 == 0, "swiglu_quant: d_ff=%d must be a multiple of 128", d_ff);
  if (T == 0) return 0;
  LFS_REQUIRE(h13 && route_weights && q && q_scale, "swiglu_quant: null pointer");
  LFS_REQUIRE(((uintptr_t)h13 | (uintptr_t)q) % 16 == 0, "swiglu_quant: buffers must be 16-byte aligned");
  LFS_REQUIRE(T * num_experts < (1ll << 31), "swiglu_quant: too many rows");
  hipLaunchKernelGGL(swiglu_quant_kernel, dim3((unsigned)(T * num_experts)), dim3(64), 0,
                     (hipStream_t)stream, (const uint16_t*)h13, route_weights, (uint8_t*)q, q_scale,
                     num_experts, d_ff);
  return check_launch("swiglu_quant");
}
