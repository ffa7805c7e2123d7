// Paged-KV kernels for gfx950: KV slot writes and split-K paged decode.
//
// KV pool layout per layer: [num_blocks, block_size, num_kv_heads, head_dim]
// bf16, as allocated by engine/model_runner.py:184-190 of the reference; one
// token's K (or V) row for all kv heads is Hkv*D*2 contiguous bytes.
//
// paged decode, phase 1 (one workgroup per (split, sequence)):
//   The workgroup walks its chunk of the context in tiles of up to 128 tokens
//   (a tile never crosses a KV block, so one block-table lookup per tile).
//   Lane mapping inside a tile: lane j of a token row (j < Hkv*D/8) owns kv
//   head j/(D/8) and dims (j%(D/8))*8 .. +7, so a token row is read with
//   fully coalesced 16-byte loads; 256/(Hkv*D/8) tokens are in flight per
//   pass.  Scores for the G query heads sharing a kv head are reduced over
//   the D/8 lanes with an xor butterfly and staged in LDS; each wave then
//   does the online-softmax update for a subset of heads (running max and
//   sum in LDS, exp2 with log2(e) folded into q); V is streamed with the same
//   lane mapping and accumulated in fp32 registers, rescaled per tile.
//   The partial (unnormalised o, m, l) of the chunk goes to the workspace.
// phase 2 (one workgroup per sequence): log-sum-exp merge of the chunks,
//   normalise, bf16.  Padding rows (context_len 0) get zeros.
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
constexpr int kThreads = 256;
constexpr int kMaxTile = 128;
constexpr int kUnroll = 8;  // 16-byte loads kept in flight per lane

__device__ __forceinline__ void unpack8(const uint4& v, float* f) {
  f[0] = bf16lo(v.x); f[1] = bf16hi(v.x);
  f[2] = bf16lo(v.y); f[3] = bf16hi(v.y);
  f[4] = bf16lo(v.z); f[5] = bf16hi(v.z);
  f[6] = bf16lo(v.w); f[7] = bf16hi(v.w);
}

template <int D, int G>
__global__ __launch_bounds__(kThreads) void paged_decode_split(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ kc,
    const uint16_t* __restrict__ vc, const int64_t* __restrict__ ctx_lens,
    const int32_t* __restrict__ bt, int64_t bt_stride, float* __restrict__ ws_o,
    float* __restrict__ ws_ml, int Hkv, int BS, int64_t NB, int max_blocks, int bps, int tile,
    float scale_log2, int max_splits) {
  constexpr int DV = D / 8;  // lanes per (token, kv head)
  extern __shared__ __attribute__((aligned(16))) float smem[];
  const int Hq = Hkv * G;
  float* sS = smem;                  // [Hq][kMaxTile] scores / probabilities
  float* sO = sS + Hq * kMaxTile;    // [Hq][D] cross-subgroup reduction
  float* sM = sO + Hq * D;           // [Hq] running max (log2 domain)
  float* sL = sM + Hq;               // [Hq] running sum
  float* sA = sL + Hq;               // [Hq] per-tile rescale factor

  const int b = blockIdx.y, split = blockIdx.x;
  const int64_t L = ctx_lens[b];
  const int64_t cap = (int64_t)max_blocks * BS;
  const int64_t t_begin = (int64_t)split * bps * BS;
  const int64_t t_end = min(min(L, cap), t_begin + (int64_t)bps * BS);
  if (t_begin >= t_end) return;  // whole workgroup leaves together

  const int tid = threadIdx.x;
  const int LPT = Hkv * DV;  // lanes per token row (divides 256, host-checked)
  const int TPP = kThreads / LPT;
  const int jl = tid & (LPT - 1);
  const int kh = jl / DV, ds = jl % DV;
  const int sub = tid / LPT;
  const int lane = tid & 63, wave = tid >> 6;
  const int row_elems = Hkv * D;

  float qf[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const uint4 v = *reinterpret_cast<const uint4*>(q + ((int64_t)b * Hq + kh * G + g) * D + ds * 8);
    unpack8(v, qf[g]);
#pragma unroll
    for (int e = 0; e < 8; ++e) qf[g][e] *= scale_log2;
  }
  float acc[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[g][e] = 0.f;

  for (int i = tid; i < Hq * D; i += kThreads) sO[i] = 0.f;
  for (int i = tid; i < Hq; i += kThreads) {
    sM[i] = -INFINITY;
    sL[i] = 0.f;
  }
  __syncthreads();

  const int32_t* btrow = bt + (int64_t)b * bt_stride;
  for (int64_t t0 = t_begin; t0 < t_end; t0 += tile) {
    const int n = (int)min((int64_t)tile, t_end - t0);
    const int32_t blk = btrow[t0 / BS];
    const bool valid = blk >= 0 && (int64_t)blk < NB;
    const int64_t base = ((int64_t)(valid ? blk : 0) * BS + (t0 % BS)) * row_elems + kh * D + ds * 8;

    // ---- phase A: scores for this tile
    for (int p0 = sub; p0 < tile; p0 += TPP * kUnroll) {
      uint4 kv[kUnroll];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const int p = p0 + u * TPP;
        kv[u] = (valid && p < n) ? *reinterpret_cast<const uint4*>(kc + base + (int64_t)p * row_elems)
                                 : make_uint4(0, 0, 0, 0);
      }
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const int p = p0 + u * TPP;
        float kf[8];
        unpack8(kv[u], kf);
        float sc[G];
#pragma unroll
        for (int g = 0; g < G; ++g) {
          float d = 0.f;
#pragma unroll
          for (int e = 0; e < 8; ++e) d = fmaf(qf[g][e], kf[e], d);
          sc[g] = group_sum<DV>(d);
        }
        if (ds == 0 && p < tile) {
          const bool live = valid && p < n;
#pragma unroll
          for (int g = 0; g < G; ++g) sS[(kh * G + g) * kMaxTile + p] = live ? sc[g] : -INFINITY;
        }
      }
    }
    __syncthreads();

    // ---- phase B: online softmax update, one wave per head
    for (int h = wave; h < Hq; h += kThreads / 64) {
      float* srow = sS + h * kMaxTile;
      const float v0 = lane < tile ? srow[lane] : -INFINITY;
      const float v1 = lane + 64 < tile ? srow[lane + 64] : -INFINITY;
      const float tmax = group_max<64>(fmaxf(v0, v1));
      const float m_old = sM[h];
      const float m_new = fmaxf(m_old, tmax);
      float p0 = 0.f, p1 = 0.f, alpha = 1.f;
      if (m_new != -INFINITY) {
        p0 = exp2f(v0 - m_new);
        p1 = exp2f(v1 - m_new);
        alpha = exp2f(m_old - m_new);
      }
      if (lane < tile) srow[lane] = p0;
      if (lane + 64 < tile) srow[lane + 64] = p1;
      const float psum = group_sum<64>(p0 + p1);
      if (lane == 0) {
        sM[h] = m_new;
        sL[h] = sL[h] * alpha + psum;
        sA[h] = alpha;
      }
    }
    __syncthreads();

    // ---- phase C: P.V
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float a = sA[kh * G + g];
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[g][e] *= a;
    }
    if (valid) {
      for (int p0 = sub; p0 < n; p0 += TPP * kUnroll) {
        uint4 vv[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
          const int p = p0 + u * TPP;
          vv[u] = p < n ? *reinterpret_cast<const uint4*>(vc + base + (int64_t)p * row_elems)
                        : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
          const int p = p0 + u * TPP;
          if (p < n) {
            float vf[8];
            unpack8(vv[u], vf);
#pragma unroll
            for (int g = 0; g < G; ++g) {
              const float w = sS[(kh * G + g) * kMaxTile + p];
#pragma unroll
              for (int e = 0; e < 8; ++e) acc[g][e] = fmaf(w, vf[e], acc[g][e]);
            }
          }
        }
      }
    }
    __syncthreads();
  }

  // ---- reduce the token subgroups, write the chunk partial
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int e = 0; e < 8; ++e) atomicAdd(&sO[(kh * G + g) * D + ds * 8 + e], acc[g][e]);
  __syncthreads();
  const int64_t pbase = (int64_t)b * max_splits + split;
  float* wo = ws_o + pbase * Hq * D;
  for (int i = tid; i < Hq * D; i += kThreads) wo[i] = sO[i];
  for (int h = tid; h < Hq; h += kThreads) {
    ws_ml[(pbase * Hq + h) * 2 + 0] = sM[h];
    ws_ml[(pbase * Hq + h) * 2 + 1] = sL[h];
  }
}

// ------------------------------------------------------------ decode merge --
__global__ __launch_bounds__(256) void paged_decode_merge(
    const float* __restrict__ ws_o, const float* __restrict__ ws_ml,
    const int64_t* __restrict__ ctx_lens, uint16_t* __restrict__ out, int Hq, int D, int BS,
    int max_blocks, int bps, int max_splits) {
  const int b = blockIdx.x;
  const int64_t L = min(ctx_lens[b], (int64_t)max_blocks * BS);
  const int64_t chunk = (int64_t)bps * BS;
  const int ns = L > 0 ? (int)min((L + chunk - 1) / chunk, (int64_t)max_splits) : 0;
  const int64_t pbase = (int64_t)b * max_splits;
  for (int i = threadIdx.x; i < Hq * D; i += blockDim.x) {
    const int h = i / D;
    float res = 0.f;
    if (ns > 0) {
      float M = -INFINITY;
      for (int s = 0; s < ns; ++s) M = fmaxf(M, ws_ml[((pbase + s) * Hq + h) * 2]);
      float num = 0.f, den = 0.f;
      if (M != -INFINITY) {
        for (int s = 0; s < ns; ++s) {
          const float m = ws_ml[((pbase + s) * Hq + h) * 2];
          const float w = exp2f(m - M);
          den = fmaf(w, ws_ml[((pbase + s) * Hq + h) * 2 + 1], den);
          num = fmaf(w, ws_o[(pbase + s) * Hq * D + i], num);
        }
      }
      res = den > 0.f ? num / den : 0.f;
    }
    out[(int64_t)b * Hq * D + i] = (uint16_t)f32_to_bf16(res);
  }
}

template <int D, int G>
void launch_split(dim3 grid, size_t shmem, hipStream_t st, const uint16_t* q, const uint16_t* kc,
                  const uint16_t* vc, const int64_t* cl, const int32_t* bt, int64_t bts, float* wo,
                  float* wml, int Hkv, int BS, int64_t NB, int max_blocks, int bps, int tile,
                  float sl2, int max_splits) {
  hipLaunchKernelGGL((paged_decode_split<D, G>), grid, dim3(kThreads), shmem, st, q, kc, vc, cl, bt,
                     bts, wo, wml, Hkv, BS, NB, max_blocks, bps, tile, sl2, max_splits);
}

template <int D>
bool dispatch_g(int G, dim3 grid, size_t shmem, hipStream_t st, const uint16_t* q,
                const uint16_t* kc, const uint16_t* vc, const int64_t* cl, const int32_t* bt,
                int64_t bts, float* wo, float* wml, int Hkv, int BS, int64_t NB, int max_blocks,
                int bps, int tile, float sl2, int max_splits) {
#define LFS_G(GG) \
  case GG: launch_split<D, GG>(grid, shmem, st, q, kc, vc, cl, bt, bts, wo, wml, Hkv, BS, NB, max_blocks, bps, tile, sl2, max_splits); return true;
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
                                int32_t blocks_per_split, void* stream) {
  const int Hq = num_q_heads, Hkv = num_kv_heads, D = head_dim, BS = block_size;
  LFS_REQUIRE(B >= 0 && Hq > 0 && Hkv > 0 && BS > 0 && num_blocks >= 0 && max_blocks >= 0,
              "paged_decode: bad shape");
  LFS_REQUIRE(D == 64 || D == 128, "paged_decode: head_dim must be 64 or 128 (got %d)", D);
  LFS_REQUIRE(Hq % Hkv == 0 && Hq / Hkv <= 8,
              "paged_decode: num_q_heads (%d) must be a multiple of num_kv_heads (%d), ratio <= 8", Hq, Hkv);
  const int LPT = Hkv * (D / 8);
  LFS_REQUIRE(LPT <= 256 && (256 % LPT) == 0,
              "paged_decode: num_kv_heads*head_dim/8 (%d) must divide 256", LPT);
  LFS_REQUIRE(BS % 16 == 0, "paged_decode: block_size must be a multiple of 16 (got %d)", BS);
  LFS_REQUIRE(blocks_per_split > 0, "paged_decode: blocks_per_split must be positive");
  LFS_REQUIRE(bt_stride >= max_blocks, "paged_decode: block table stride < max_blocks");
  if (B == 0) return 0;
  LFS_REQUIRE(q && k_cache && v_cache && context_lens && out, "paged_decode: null pointer");
  LFS_REQUIRE(max_blocks == 0 || block_tables, "paged_decode: null block table");
  LFS_REQUIRE(((((uintptr_t)q) | ((uintptr_t)k_cache) | ((uintptr_t)v_cache)) & 15u) == 0,
              "paged_decode: q and caches must be 16-byte aligned");
  LFS_REQUIRE(B < 65536, "paged_decode: batch too large");
  const int64_t need = lfs_paged_decode_workspace_bytes(B, Hq, D, max_blocks, blocks_per_split);
  LFS_REQUIRE(workspace_bytes >= need && (need == 0 || workspace),
              "paged_decode: workspace of %lld bytes < required %lld", (long long)workspace_bytes,
              (long long)need);
  const int max_splits = (max_blocks + blocks_per_split - 1) / blocks_per_split;
  float* ws_o = (float*)workspace;
  float* ws_ml = ws_o + (size_t)B * max_splits * Hq * D;
  hipStream_t st = (hipStream_t)stream;
  int tile = 16;
  for (int t = kMaxTile; t >= 16; t >>= 1)
    if (BS % t == 0) { tile = t; break; }
  const float sl2 = scale * 1.4426950408889634f;
  if (max_splits > 0) {
    const dim3 grid((unsigned)max_splits, (unsigned)B);
    const size_t shmem = sizeof(float) * ((size_t)Hq * kMaxTile + (size_t)Hq * D + 3 * (size_t)Hq);
    LFS_REQUIRE(shmem <= 64 * 1024, "paged_decode: too many heads for LDS (%d)", Hq);
    const int G = Hq / Hkv;
    const bool ok = D == 64
        ? dispatch_g<64>(G, grid, shmem, st, (const uint16_t*)q, (const uint16_t*)k_cache,
                         (const uint16_t*)v_cache, context_lens, block_tables, bt_stride, ws_o,
                         ws_ml, Hkv, BS, num_blocks, max_blocks, blocks_per_split, tile, sl2, max_splits)
        : dispatch_g<128>(G, grid, shmem, st, (const uint16_t*)q, (const uint16_t*)k_cache,
                          (const uint16_t*)v_cache, context_lens, block_tables, bt_stride, ws_o,
                          ws_ml, Hkv, BS, num_blocks, max_blocks, blocks_per_split, tile, sl2, max_splits);
    LFS_REQUIRE(ok, "paged_decode: unsupported group size %d", G);
    const int rc = check_launch("paged_decode(split)");
    if (rc) return rc;
  }
  hipLaunchKernelGGL(paged_decode_merge, dim3((unsigned)B), dim3(256), 0, st, ws_o, ws_ml,
                     context_lens, (uint16_t*)out, Hq, D, BS, max_blocks, blocks_per_split,
                     max_splits);
  return check_launch("paged_decode(merge)");
}
