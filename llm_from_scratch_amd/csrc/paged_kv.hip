// Paged-KV kernels for gfx950: KV slot writes and split-K paged decode.
//
// KV pool layout per layer: [num_blocks, block_size, num_kv_heads, head_dim]
// bf16, as allocated by engine/model_runner.py:184-190 of the reference; one
// token's K (or V) row for all kv heads is Hkv*D*2 contiguous bytes.
//
// paged decode, phase 1 (paged_decode_split): one wave per (sequence, kv
//   head, chunk of blocks_per_split KV blocks), four kv heads of one
//   sequence and chunk per workgroup, grid (sequence, chunk, head group).
//   The wave walks its chunk in tiles of up to 64 tokens that never cross a
//   KV block (one block-table lookup per tile): S = K q^T on MFMA for the G
//   query heads of its kv head, online softmax in the log2 domain, P through
//   a wave-private LDS slice, P.V in fp32 registers.  Loads run two tiles
//   ahead.  The partial (unnormalised o, m, l) of the chunk goes to the
//   workspace, or, when the chunk is the whole context, the normalised bf16
//   output is written directly.
// phase 2 (paged_decode_merge, one workgroup per (head, sequence)):
//   log-sum-exp merge of the chunks, normalise, bf16.  Padding rows
//   (context_len 0) get zeros.  paged_decode_merge_quant (one workgroup per
//   sequence) does the same and also writes the act_quant codes and scales
//   of the bf16 output row (the output projection's FP8 input).
#include "common.h"

namespace lfs {
namespace {

// ---------------------------------------------------------- store_kvcache --
template <int VEC>
__global__ __launch_bounds__(128) void store_kvcache_kernel(
    const uint16_t* __restrict__ key, int64_t ks, const uint16_t* __restrict__ value, int64_t vs,
    uint16_t* __restrict__ kc, uint16_t* __restrict__ vc, const int64_t* __restrict__ slots,
    int HD, int64_t num_slots) {
  const int64_t t = blockIdx.x;
  const int64_t slot = slots[t];
  if (slot < 0 || slot >= num_slots) return;  // -1 = padding / skipped token
  const uint16_t* ksrc = key + t * ks;
  const uint16_t* vsrc = value + t * vs;
  uint16_t* kdst = kc + slot * HD;
  uint16_t* vdst = vc + slot * HD;
  if constexpr (VEC == 8) {
    for (int i = threadIdx.x; i < HD / 8; i += blockDim.x) {
      reinterpret_cast<uint4*>(kdst)[i] = reinterpret_cast<const uint4*>(ksrc)[i];
      reinterpret_cast<uint4*>(vdst)[i] = reinterpret_cast<const uint4*>(vsrc)[i];
    }
  } else {
    for (int i = threadIdx.x; i < HD; i += blockDim.x) {
      kdst[i] = ksrc[i];
      vdst[i] = vsrc[i];
    }
  }
}

// ------------------------------------------------------------ decode split --
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));

// One wave per (sequence, kv head, chunk of the context).  Per tile of T
// tokens (one KV block never straddled):
//   K  : MFMA A operand straight from HBM -- lane l loads token (l % 16) of a
//        16-token group, dims c*32 + (l / 16)*8 .. +7 (16 B);
//   q^T: MFMA B operand, column j = l % 16 is query head kh*G + j (zero for
//        j >= G), preloaded once;
//   S  = K q^T with v_mfma_f32_16x16x32_bf16: lane l ends with the scores of
//        head (l % 16) for tokens 4*(l / 16) .. +3 of each group, so the
//        online-softmax max/sum per head is a 2-step xor over lanes 16, 32;
//   P  goes through a wave-private LDS slice [T][G] to the P.V mapping;
//   V  : lane l owns token (l / (D/8)) + (64/(D/8))*i and dims
//        (l % (D/8))*8 .. +7 (coalesced 16-byte loads), fp32 FMAs into
//        acc[G][8], rescaled by exp2(m_old - m_new) read from lane g.
// Loads are software-pipelined two tiles ahead (two K and two V buffers,
// each refilled as soon as its tile is consumed) with nontemporal 16-byte
// loads, since every KV row is read exactly once.  There is no workgroup
// barrier: waves exit independently.  A chunk that covers
// the whole context writes the normalised bf16 output directly; otherwise
// the unnormalised partial (o, m, l) goes to the workspace for the merge.
template <int D>
struct DecodeGeom {
  static constexpr int LPR = D / 8;               // lanes per token row in the P.V mapping
  static constexpr int TPI = 64 / LPR;            // tokens per V load instruction
  static constexpr int T = (D == 64) ? 64 : 32;   // tokens per tile
  static constexpr int NG = T / 16;               // 16-token MFMA groups per tile
  static constexpr int NDC = D / 32;              // 32-wide head-dim chunks
  static constexpr int UV = T / TPI;              // V loads per lane per tile
};

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
// 16-byte streaming load (nontemporal: the KV rows are read exactly once)
__device__ __forceinline__ uint4 nt_load16(const uint16_t* p) {
  const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  return make_uint4(v[0], v[1], v[2], v[3]);
}

__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

template <int D, int G>
__global__ __launch_bounds__(256) void paged_decode_split(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ kc,
    const uint16_t* __restrict__ vc, const int64_t* __restrict__ ctx_lens,
    const int32_t* __restrict__ bt, int64_t bt_stride, float* __restrict__ ws_o,
    float* __restrict__ ws_ml, uint16_t* __restrict__ out, int Hkv, int BS, int64_t NB,
    int max_blocks, int bps, int tile, float scale_log2, int max_splits) {
  using Geo = DecodeGeom<D>;
  constexpr int GP = G <= 4 ? 4 : 8;  // padded heads per token in the P slice
  __shared__ __attribute__((aligned(16))) float p_lds[4][Geo::T * GP];

  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int kh = blockIdx.z * (blockDim.x >> 6) + wave;
  if (kh >= Hkv) return;
  // sequence index fastest: workgroups are dealt round-robin to the 8 XCDs,
  // so consecutive ids must not be the splits of one sequence (split s would
  // always land on XCD s mod 8, and short contexts leave the high splits
  // empty, i.e. whole XCDs idle)
  const int b = blockIdx.x, split = blockIdx.y;
  const int64_t Lc = min(ctx_lens[b], (int64_t)max_blocks * BS);
  const int64_t chunk = (int64_t)bps * BS;
  const int64_t t_begin = (int64_t)split * chunk;
  const int64_t t_end = min(Lc, t_begin + chunk);
  if (t_begin >= t_end) return;
  const int Hq = Hkv * G;
  const int64_t row = (int64_t)Hkv * D;

  const int j = lane & 15, kq = lane >> 4;
  v8bf qb[Geo::NDC];
#pragma unroll
  for (int c = 0; c < Geo::NDC; ++c) {
    uint4 w = make_uint4(0, 0, 0, 0);
    if (j < G) w = *reinterpret_cast<const uint4*>(q + ((int64_t)b * Hq + kh * G + j) * D + c * 32 + kq * 8);
    qb[c] = __builtin_bit_cast(v8bf, w);
  }
  const int ts = lane / Geo::LPR, dc = lane % Geo::LPR;
  float acc[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[g][e] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;
  float* pw = p_lds[wave];
  const int32_t* btrow = bt + (int64_t)b * bt_stride;

  const int ntiles = (int)((t_end - t_begin + tile - 1) / tile);
  // tile i of the chunk: valid row count (0 for a skipped block) and the
  // element offset of its first row.  Tiles at or past `last` are
  // look-ahead fillers: n = 0 and row 0 of block 0, so their loads all hit
  // one line (they only keep the per-step load count constant).
  int last = 0;
  auto tile_at = [&](int i, int& n, int64_t& off) {
    if (i >= last) {
      n = 0;
      off = (int64_t)kh * D;
      return;
    }
    const int64_t t0 = t_begin + (int64_t)i * tile;
    n = (int)min((int64_t)tile, t_end - t0);
    const int32_t blk = btrow[t0 / BS];
    const bool ok = blk >= 0 && (int64_t)blk < NB;
    if (!ok) n = 0;  // invalid block: contributes nothing
    off = ((int64_t)(ok ? blk : 0) * BS + (t0 % BS)) * row + (int64_t)kh * D;
  };
  // Every load is issued unconditionally: rows past the valid count n read
  // row n-1 (row 0 of block 0 for a skipped block), whose scores are masked
  // and whose P is 0 (a skipped block's P.V is not run).  Offsets inside a
  // tile are 32-bit from a wave-uniform base.
  auto load_k = [&](uint4 (&ka)[Geo::NG][Geo::NDC], int n, int64_t off) {
    const uint16_t* kb = kc + off;
    const int nn = max(n, 1);
#pragma unroll
    for (int g16 = 0; g16 < Geo::NG; ++g16) {
      const int tr = min(g16 * 16 + j, nn - 1);
#pragma unroll
      for (int c = 0; c < Geo::NDC; ++c)
        ka[g16][c] = nt_load16(kb + (uint32_t)(tr * (int)row + c * 32 + kq * 8));
    }
  };
  auto load_v = [&](uint4 (&va)[Geo::UV], int n, int64_t off) {
    const uint16_t* vb = vc + off;
    const int nn = max(n, 1);
#pragma unroll
    for (int i = 0; i < Geo::UV; ++i)
      va[i] = nt_load16(vb + (uint32_t)(min(ts + Geo::TPI * i, nn - 1) * (int)row + dc * 8));
  };

  // Software pipeline two tiles deep, two K and two V buffers.  Issue order:
  //   prologue K0 V0 K1 V1;  tile i: [QK_i] K_{i+2} [softmax, P.V_i] V_{i+2}
  // Each buffer is refilled with tile i+2 as soon as tile i has consumed it,
  // so up to two tiles of K and V are in flight while a tile is computed.
  // The tiles of a chunk are processed in straight-line code (MAXT steps
  // unrolled, with early exits), every step issuing the same loads, so the
  // compiler's in-order wait counts are exact: QK_i waits only for K_i and
  // P.V_i only for V_i.  (In a loop, its conservative merge at the loop
  // header drains every load in flight once per iteration.)  Chunks longer
  // than MAXT tiles are walked MAXT tiles at a time.
  constexpr int MAXT = 8;
  uint4 ka0[Geo::NG][Geo::NDC], ka1[Geo::NG][Geo::NDC];
  uint4 va0[Geo::UV], va1[Geo::UV];
  int nb0 = 0, nb1 = 0;
  auto step = [&](int i, uint4 (&ka)[Geo::NG][Geo::NDC], uint4 (&va)[Geo::UV], int& nb) {
    const int n = nb;
    int n2;
    int64_t o2;
    tile_at(i + 2, n2, o2);

    // ---- scores (log2 domain) and online-softmax update for head j
    float s[Geo::NG][4];
    float tmax = -INFINITY;
#pragma unroll
    for (int g16 = 0; g16 < Geo::NG; ++g16) {
      v4f sc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < Geo::NDC; ++c)
        sc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, ka[g16][c]), qb[c], sc, 0, 0, 0);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int tok = g16 * 16 + kq * 4 + r;
        s[g16][r] = tok < n ? sc[r] * scale_log2 : -INFINITY;
        tmax = fmaxf(tmax, s[g16][r]);
      }
    }
    __builtin_amdgcn_sched_barrier(0);  // keep the issue order the wait counts assume
    load_k(ka, n2, o2);
    __builtin_amdgcn_sched_barrier(0);
    tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
    const float m_new = fmaxf(m_run, tmax);
    const bool live = m_new != -INFINITY;
    const float alpha = live ? exp2f(m_run - m_new) : 1.f;
    float psum = 0.f;
#pragma unroll
    for (int g16 = 0; g16 < Geo::NG; ++g16)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float p = live ? exp2f(s[g16][r] - m_new) : 0.f;
        psum += p;
        if (j < G) pw[(g16 * 16 + kq * 4 + r) * GP + j] = p;
      }
    psum += __shfl_xor(psum, 16, 64);
    psum += __shfl_xor(psum, 32, 64);
    l_run = l_run * alpha + psum;
    m_run = m_new;
    wave_lds_sync();

    // ---- P.V (rows past n have P = 0; a skipped block adds nothing)
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(alpha), g));
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[g][e] *= a;
    }
    if (n > 0) {
#pragma unroll
      for (int iv = 0; iv < Geo::UV; ++iv) {
        const int tok = ts + Geo::TPI * iv;
        float pg[GP];
#pragma unroll
        for (int g4 = 0; g4 < GP; g4 += 4) {
          const float4 p4 = *reinterpret_cast<const float4*>(&pw[tok * GP + g4]);
          pg[g4] = p4.x; pg[g4 + 1] = p4.y; pg[g4 + 2] = p4.z; pg[g4 + 3] = p4.w;
        }
        float vf[8];
        unpack8(va[iv], vf);
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[g][e] = fmaf(pg[g], vf[e], acc[g][e]);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    load_v(va, n2, o2);
    __builtin_amdgcn_sched_barrier(0);
    wave_lds_sync();
    nb = n2;
  };
  for (int base = 0; base < ntiles; base += MAXT) {
    last = min(ntiles, base + MAXT);
    {
      int64_t o0, o1;
      tile_at(base, nb0, o0);
      tile_at(base + 1, nb1, o1);
      load_k(ka0, nb0, o0);
      load_v(va0, nb0, o0);
      load_k(ka1, nb1, o1);
      load_v(va1, nb1, o1);
    }
#pragma unroll
    for (int u = 0; u < MAXT; u += 2) {
      if (base + u >= last) break;
      step(base + u, ka0, va0, nb0);
      if (base + u + 1 >= last) break;
      step(base + u + 1, ka1, va1, nb1);
    }
    __builtin_amdgcn_s_waitcnt(0x0F70);  // drain the look-ahead loads
  }

  // ---- reduce the token subgroups (lanes with the same dc)
#pragma unroll
  for (int o = Geo::LPR; o < 64; o <<= 1)
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[g][e] += __shfl_xor(acc[g][e], o, 64);

  if (t_begin == 0 && t_end >= Lc) {
    // the whole context is in this chunk: normalise and write bf16
    if (ts == 0) {
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float lg = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(l_run), g));
        const float inv = lg > 0.f ? 1.f / lg : 0.f;
        uint4 o;
        o.x = pack_bf16x2(acc[g][0] * inv, acc[g][1] * inv);
        o.y = pack_bf16x2(acc[g][2] * inv, acc[g][3] * inv);
        o.z = pack_bf16x2(acc[g][4] * inv, acc[g][5] * inv);
        o.w = pack_bf16x2(acc[g][6] * inv, acc[g][7] * inv);
        *reinterpret_cast<uint4*>(out + ((int64_t)b * Hq + kh * G + g) * D + dc * 8) = o;
      }
    }
  } else {
    const int64_t pbase = (int64_t)b * max_splits + split;
    if (ts == 0) {
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float* dst = ws_o + (pbase * Hq + kh * G + g) * D + dc * 8;
        *reinterpret_cast<float4*>(dst) = make_float4(acc[g][0], acc[g][1], acc[g][2], acc[g][3]);
        *reinterpret_cast<float4*>(dst + 4) = make_float4(acc[g][4], acc[g][5], acc[g][6], acc[g][7]);
      }
    }
    if (lane < G) {
      ws_ml[(pbase * Hq + kh * G + lane) * 2 + 0] = m_run;
      ws_ml[(pbase * Hq + kh * G + lane) * 2 + 1] = l_run;
    }
  }
}

// ------------------------------------------------------------ decode merge --
// One workgroup per (head, sequence), one lane per head dim.  Sequences whose
// context fits one chunk were finished by the split kernel; padding rows
// (context 0) get zeros.
__global__ __launch_bounds__(128) void paged_decode_merge(
    const float* __restrict__ ws_o, const float* __restrict__ ws_ml,
    const int64_t* __restrict__ ctx_lens, uint16_t* __restrict__ out, int Hq, int D, int BS,
    int max_blocks, int bps, int max_splits) {
  const int h = blockIdx.x, b = blockIdx.y, d = threadIdx.x;
  const int64_t Lc = min(ctx_lens[b], (int64_t)max_blocks * BS);
  const int64_t chunk = (int64_t)bps * BS;
  const int ns = (int)((Lc + chunk - 1) / chunk);
  if (ns == 1 || d >= D) return;
  float res = 0.f;
  if (ns > 1) {
    const int64_t pbase = (int64_t)b * max_splits;
    float M = -INFINITY;
    for (int s = 0; s < ns; ++s) M = fmaxf(M, ws_ml[((pbase + s) * Hq + h) * 2]);
    float num = 0.f, den = 0.f;
    if (M != -INFINITY) {
      for (int s = 0; s < ns; ++s) {
        const float w = exp2f(ws_ml[((pbase + s) * Hq + h) * 2] - M);
        den = fmaf(w, ws_ml[((pbase + s) * Hq + h) * 2 + 1], den);
        num = fmaf(w, ws_o[((pbase + s) * Hq + h) * D + d], num);
      }
    }
    res = den > 0.f ? num / den : 0.f;
  }
  out[((int64_t)b * Hq + h) * D + d] = (uint16_t)f32_to_bf16(res);
}

// Phase 2 fused with the output projection's act_quant: one workgroup per
// sequence merges every head (or re-reads the rows the split kernel wrote
// for a single-chunk context; zeros for context 0), writes the bf16 output,
// and quantises the row per 128-value group with act_quant's formula and
// rounding (the codes equal act_quant of the bf16 output bit for bit).
constexpr int MQ_MAXE = 8192;  // Hq * D per sequence
constexpr int MQ_MAXH = 128;
constexpr int MQ_MAXW = 4096;  // (split, head) weights staged in LDS

__global__ __launch_bounds__(256) void paged_decode_merge_quant(
    const float* __restrict__ ws_o, const float* __restrict__ ws_ml, const int64_t* __restrict__ ctx_lens,
    uint16_t* __restrict__ out, uint8_t* __restrict__ qo, float* __restrict__ qs, int Hq, int D, int BS,
    int max_blocks, int bps, int max_splits) {
  __shared__ float hDen[MQ_MAXH];
  __shared__ float wts[MQ_MAXW];  // [split][head]: exp2(m - M_head), then the per-head sums
  __shared__ __attribute__((aligned(16))) uint16_t vals[MQ_MAXE];
  const int b = blockIdx.x, tid = threadIdx.x;
  const int64_t Lc = min(ctx_lens[b], (int64_t)max_blocks * BS);
  const int64_t chunk = (int64_t)bps * BS;
  const int ns = (int)((Lc + chunk - 1) / chunk);
  const int E = Hq * D;
  uint16_t* orow = out + (int64_t)b * E;
  if (ns > 1) {
    const int64_t pbase = (int64_t)b * max_splits;
    // (m, l) of every (split, head) in one parallel step; the per-head max,
    // weights and denominators from LDS (the unfused merge's arithmetic)
    const bool staged = ns * Hq <= MQ_MAXW;
    if (staged) {
      for (int x = tid; x < ns * Hq; x += 256) wts[x] = ws_ml[(pbase * Hq + x) * 2];
      __syncthreads();
    }
    auto mval = [&](int sp, int h) -> float { return staged ? wts[sp * Hq + h] : ws_ml[((pbase + sp) * Hq + h) * 2]; };
    for (int h = tid; h < Hq; h += 256) {
      float M = -INFINITY;
      for (int sp = 0; sp < ns; ++sp) M = fmaxf(M, mval(sp, h));
      float den = 0.f;
      if (M != -INFINITY)
        for (int sp = 0; sp < ns; ++sp) {
          const float w = exp2f(mval(sp, h) - M);
          den = fmaf(w, ws_ml[((pbase + sp) * Hq + h) * 2 + 1], den);
          if (staged) wts[sp * Hq + h] = w;  // this thread alone reads / writes head h's entries
        }
      else if (staged)
        for (int sp = 0; sp < ns; ++sp) wts[sp * Hq + h] = 0.f;
      hDen[h] = M != -INFINITY ? den : 0.f;
    }
    __syncthreads();
    for (int e = tid; e < E; e += 256) {
      const int h = e / D, d = e - h * D;
      const float den = hDen[h];
      float num = 0.f;
      if (staged) {
        for (int sp = 0; sp < ns; ++sp) num = fmaf(wts[sp * Hq + h], ws_o[((pbase + sp) * Hq + h) * D + d], num);
      } else {
        float M = -INFINITY;
        for (int sp = 0; sp < ns; ++sp) M = fmaxf(M, mval(sp, h));
        if (M != -INFINITY)
          for (int sp = 0; sp < ns; ++sp)
            num = fmaf(exp2f(mval(sp, h) - M), ws_o[((pbase + sp) * Hq + h) * D + d], num);
      }
      const uint16_t v = (uint16_t)f32_to_bf16(den > 0.f ? num / den : 0.f);
      orow[e] = v;
      vals[e] = v;
    }
  } else if (ns == 1) {
    for (int e = tid; e < E; e += 256) vals[e] = orow[e];  // written by the split kernel
  } else {
    for (int e = tid; e < E; e += 256) {
      orow[e] = 0;
      vals[e] = 0;
    }
  }
  __syncthreads();
  // act_quant of the row: 16 lanes per 128-value group, 8 values per lane
  // (E / 8 is a multiple of 16, so a group's lanes are all in or all out)
  for (int c8 = tid; c8 < E / 8; c8 += 256) {
    float f[8];
    unpack8(*reinterpret_cast<const uint4*>(&vals[c8 * 8]), f);
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(f[i]));
    amax = group_max<16>(amax);
    const float sc = scale_from_amax(amax, false);
    *reinterpret_cast<uint2*>(qo + (int64_t)b * E + c8 * 8) = quant8(f, sc);
    if ((c8 & 15) == 0) qs[(int64_t)b * (E / 128) + c8 / 16] = sc;
  }
}

template <int D, int G>
void launch_split(dim3 grid, dim3 block, hipStream_t st, const uint16_t* q, const uint16_t* kc,
                  const uint16_t* vc, const int64_t* cl, const int32_t* bt, int64_t bts, float* wo,
                  float* wml, uint16_t* out, int Hkv, int BS, int64_t NB, int max_blocks, int bps,
                  int tile, float sl2, int max_splits) {
  hipLaunchKernelGGL((paged_decode_split<D, G>), grid, block, 0, st, q, kc, vc, cl, bt, bts, wo, wml,
                     out, Hkv, BS, NB, max_blocks, bps, tile, sl2, max_splits);
}

template <int D>
bool dispatch_g(int G, dim3 grid, dim3 block, hipStream_t st, const uint16_t* q,
                const uint16_t* kc, const uint16_t* vc, const int64_t* cl, const int32_t* bt,
                int64_t bts, float* wo, float* wml, uint16_t* out, int Hkv, int BS, int64_t NB,
                int max_blocks, int bps, int tile, float sl2, int max_splits) {
#define LFS_G(GG) \
  case GG: launch_split<D, GG>(grid, block, st, q, kc, vc, cl, bt, bts, wo, wml, out, Hkv, BS, NB, max_blocks, bps, tile, sl2, max_splits); return true;
  switch (G) {
    LFS_G(1) LFS_G(2) LFS_G(3) LFS_G(4) LFS_G(5) LFS_G(6) LFS_G(7) LFS_G(8)
    default: return false;
  }
#undef LFS_G
}

}  // namespace
}  // namespace lfs

using namespace lfs;

extern "C" int lfs_store_kvcache(const void* key, int64_t k_stride_t, const void* value,
                                 int64_t v_stride_t, void* k_cache, void* v_cache,
                                 const int64_t* slot_mapping, int64_t T, int32_t num_kv_heads,
                                 int32_t head_dim, int64_t num_slots, void* stream) {
  LFS_REQUIRE(T >= 0 && num_kv_heads > 0 && head_dim > 0 && num_slots >= 0,
              "store_kvcache: bad shape T=%lld Hkv=%d D=%d", (long long)T, num_kv_heads, head_dim);
  if (T == 0) return 0;
  LFS_REQUIRE(key && value && k_cache && v_cache && slot_mapping, "store_kvcache: null pointer");
  LFS_REQUIRE(T < (1ll << 31), "store_kvcache: too many tokens");
  const int HD = num_kv_heads * head_dim;
  const bool vec = HD % 8 == 0 && k_stride_t % 8 == 0 && v_stride_t % 8 == 0 &&
                   ((((uintptr_t)key) | ((uintptr_t)value) | ((uintptr_t)k_cache) |
                     ((uintptr_t)v_cache)) & 15u) == 0;
  hipStream_t st = (hipStream_t)stream;
  if (vec)
    hipLaunchKernelGGL(store_kvcache_kernel<8>, dim3((unsigned)T), dim3(128), 0, st,
                       (const uint16_t*)key, k_stride_t, (const uint16_t*)value, v_stride_t,
                       (uint16_t*)k_cache, (uint16_t*)v_cache, slot_mapping, HD, num_slots);
  else
    hipLaunchKernelGGL(store_kvcache_kernel<1>, dim3((unsigned)T), dim3(128), 0, st,
                       (const uint16_t*)key, k_stride_t, (const uint16_t*)value, v_stride_t,
                       (uint16_t*)k_cache, (uint16_t*)v_cache, slot_mapping, HD, num_slots);
  return check_launch("store_kvcache");
}

extern "C" int64_t lfs_paged_decode_workspace_bytes(int64_t B, int32_t num_q_heads,
                                                    int32_t head_dim, int32_t max_blocks,
                                                    int32_t blocks_per_split) {
  if (B < 0 || num_q_heads <= 0 || head_dim <= 0 || max_blocks < 0 || blocks_per_split <= 0)
    return -1;
  const int64_t splits = ((int64_t)max_blocks + blocks_per_split - 1) / blocks_per_split;
  return 4 * B * splits * (int64_t)num_q_heads * ((int64_t)head_dim + 2);
}

extern "C" int lfs_paged_decode(const void* q, const void* k_cache, const void* v_cache,
                                const int64_t* context_lens, const int32_t* block_tables,
                                int64_t bt_stride, void* out, void* workspace,
                                int64_t workspace_bytes, int64_t B, int32_t num_q_heads,
                                int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                                int64_t num_blocks, int32_t max_blocks, float scale,
                                int32_t blocks_per_split, void* q_out, float* q_scale, void* stream) {
  const int Hq = num_q_heads, Hkv = num_kv_heads, D = head_dim, BS = block_size;
  LFS_REQUIRE(B >= 0 && Hq > 0 && Hkv > 0 && BS > 0 && num_blocks >= 0 && max_blocks >= 0,
              "paged_decode: bad shape");
  LFS_REQUIRE(D == 64 || D == 128, "paged_decode: head_dim must be 64 or 128 (got %d)", D);
  LFS_REQUIRE(Hq % Hkv == 0 && Hq / Hkv <= 8,
              "paged_decode: num_q_heads (%d) must be a multiple of num_kv_heads (%d), ratio <= 8", Hq, Hkv);
  LFS_REQUIRE(BS % 16 == 0, "paged_decode: block_size must be a multiple of 16 (got %d)", BS);
  LFS_REQUIRE(blocks_per_split > 0, "paged_decode: blocks_per_split must be positive");
  LFS_REQUIRE(bt_stride >= max_blocks, "paged_decode: block table stride < max_blocks");
  LFS_REQUIRE(num_blocks >= 1 || max_blocks == 0, "paged_decode: empty KV pool");
  if (B == 0) return 0;
  LFS_REQUIRE(q && k_cache && v_cache && context_lens && out, "paged_decode: null pointer");
  LFS_REQUIRE(max_blocks == 0 || block_tables, "paged_decode: null block table");
  LFS_REQUIRE(((((uintptr_t)q) | ((uintptr_t)k_cache) | ((uintptr_t)v_cache)) & 15u) == 0,
              "paged_decode: q and caches must be 16-byte aligned");
  LFS_REQUIRE(B < 65536, "paged_decode: batch too large");
  LFS_REQUIRE((q_out == nullptr) == (q_scale == nullptr), "paged_decode: q_out and q_scale go together");
  LFS_REQUIRE(q_out == nullptr || (Hq * D % 128 == 0 && Hq * D <= MQ_MAXE && Hq <= MQ_MAXH),
              "paged_decode: the quantised output needs Hq*D %% 128 == 0, Hq*D <= %d", MQ_MAXE);
  const int64_t need = lfs_paged_decode_workspace_bytes(B, Hq, D, max_blocks, blocks_per_split);
  LFS_REQUIRE(workspace_bytes >= need && (need == 0 || workspace),
              "paged_decode: workspace of %lld bytes < required %lld", (long long)workspace_bytes,
              (long long)need);
  const int max_splits = (max_blocks + blocks_per_split - 1) / blocks_per_split;
  float* ws_o = (float*)workspace;
  float* ws_ml = ws_o + (size_t)B * max_splits * Hq * D;
  hipStream_t st = (hipStream_t)stream;
  const int Tmax = D == 64 ? 64 : 32;
  int tile = 16;
  for (int t = Tmax; t >= 16; t >>= 1)
    if (BS % t == 0) { tile = t; break; }
  const float sl2 = scale * 1.4426950408889634f;
  if (max_splits > 0) {
    const int wpg = Hkv < 4 ? Hkv : 4;  // waves (kv heads) per workgroup
    const dim3 grid((unsigned)B, (unsigned)max_splits, (unsigned)((Hkv + wpg - 1) / wpg));
    LFS_REQUIRE(grid.z < 65536u && grid.y < 65536u, "paged_decode: too many kv heads or splits");
    const dim3 block((unsigned)(64 * wpg));
    const int G = Hq / Hkv;
    const bool ok = D == 64
        ? dispatch_g<64>(G, grid, block, st, (const uint16_t*)q, (const uint16_t*)k_cache,
                         (const uint16_t*)v_cache, context_lens, block_tables, bt_stride, ws_o,
                         ws_ml, (uint16_t*)out, Hkv, BS, num_blocks, max_blocks, blocks_per_split,
                         tile, sl2, max_splits)
        : dispatch_g<128>(G, grid, block, st, (const uint16_t*)q, (const uint16_t*)k_cache,
                          (const uint16_t*)v_cache, context_lens, block_tables, bt_stride, ws_o,
                          ws_ml, (uint16_t*)out, Hkv, BS, num_blocks, max_blocks, blocks_per_split,
                          tile, sl2, max_splits);
    LFS_REQUIRE(ok, "paged_decode: unsupported group size %d", G);
    const int rc = check_launch("paged_decode(split)");
    if (rc) return rc;
  }
  if (q_out != nullptr) {
    hipLaunchKernelGGL(paged_decode_merge_quant, dim3((unsigned)B), dim3(256), 0, st, ws_o, ws_ml, context_lens,
                       (uint16_t*)out, (uint8_t*)q_out, q_scale, Hq, D, BS, max_blocks, blocks_per_split,
                       max_splits);
    return check_launch("paged_decode(merge + quant)");
  }
  hipLaunchKernelGGL(paged_decode_merge, dim3((unsigned)Hq, (unsigned)B), dim3((unsigned)D), 0, st,
                     ws_o, ws_ml, context_lens, (uint16_t*)out, Hq, D, BS, max_blocks,
                     blocks_per_split, max_splits);
  return check_launch("paged_decode(merge)");
}
