// Fused temperature + Gumbel-max sampler for gfx950 (the decode step's
// last op, utils/sampler.py:35-53 of the reference):
//
//   token[b] = argmax_i softmax(logits[b] / T[b])_i / max(e[b,i], 1e-10)
//
// e[b,i] ~ Exp(1) from a counter-based generator, Philox4x32-10 (Salmon,
// Moraes, Dror, Shaw, SC'11): counter (i/4 + offset_lo, offset_hi (+carry),
// b, 0x53414D50), key (seed_lo, seed_hi), word i % 4 as w, then
// e = -log((w + 1) * 2^-32) to float rounding.  One workgroup per row and
// one pass: the pick maximises x_i / T - log(max(e_i, 1e-10)), which orders
// the elements as softmax(x / T)_i / max(e_i, 1e-10) does (the softmax's
// normaliser is common to the row); ties go to the lowest index.  Four
// consecutive elements per lane per step (one 8-byte load, one Philox call).
// With a workspace (lfs_sample_gumbel_split) each row is cut into S slices
// of consecutive elements, one workgroup per (row, slice) writing its
// slice's best (score, index), and a second launch picks each row's best
// slice by the same rule -- the same picks, with S times the workgroups
// when the batch alone would leave CUs idle.
#include "common.h"

#include <algorithm>

namespace lfs {
namespace {

constexpr int SNT = 1024;  // threads per row

__device__ __forceinline__ void philox4x32_10(uint32_t (&c)[4], uint32_t k0, uint32_t k1) {
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    if (r) {
      k0 += 0x9E3779B9u;
      k1 += 0xBB67AE85u;
    }
    const uint64_t p0 = (uint64_t)c[0] * 0xD2511F53u;
    const uint64_t p1 = (uint64_t)c[2] * 0xCD9E8D57u;
    const uint32_t n0 = (uint32_t)(p1 >> 32) ^ c[1] ^ k0;
    const uint32_t n2 = (uint32_t)(p0 >> 32) ^ c[3] ^ k1;
    c[1] = (uint32_t)p1;
    c[3] = (uint32_t)p0;
    c[0] = n0;
    c[2] = n2;
  }
}

// e = -log(u), u = (w + 1) * 2^-32 in (0, 1], to float rounding: for
// u >= 1/2 through log1p of the (exact) complement v = (2^32 - 1 - w) * 2^-32,
// so that u close to 1 keeps its small e; otherwise the log of u itself
// (float(w + 1) is within 2^-24 relative, the power-of-two scale exact).
__device__ __forceinline__ float exp1_from_word(uint32_t w) {
  if (w >= 0x80000000u) return -log1pf(-(float)(0xFFFFFFFFu - w) * 0x1p-32f);
  return -logf(((float)w + 1.0f) * 0x1p-32f);
}

__device__ __forceinline__ void load4(const uint16_t* row, int64_t i, int V, float (&x)[4], bool vec) {
  if (vec && i + 3 < V) {
    const uint2 w = *reinterpret_cast<const uint2*>(row + i);
    x[0] = bf16lo(w.x); x[1] = bf16hi(w.x); x[2] = bf16lo(w.y); x[3] = bf16hi(w.y);
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) x[e] = i + e < V ? bf16_to_f32(row[i + e]) : -INFINITY;
  }
}

// One workgroup per (row b, slice blockIdx.y of gridDim.y): the element
// groups of the slice; the slice's best goes to part[b * S + slice] (score
// bits, index) when part is given, else (one slice) straight to out[b].
__global__ __launch_bounds__(1024) void sample_gumbel_kernel(const uint16_t* __restrict__ logits, int64_t ld,
                                                            const float* __restrict__ temps, int V, uint64_t seed,
                                                            uint64_t offset, int64_t* __restrict__ out,
                                                            float* __restrict__ noise_out, uint2* __restrict__ part) {
  __shared__ float red_v[SNT / 64];
  __shared__ int red_i[SNT / 64];
  const int b = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int S = gridDim.y, slice = blockIdx.y;
  const uint16_t* row = logits + (int64_t)b * ld;
  const float T = temps[b];
  const bool vec = ((ld & 3) == 0) && ((((uintptr_t)logits) & 7u) == 0);
  const int n4 = (V + 3) / 4;
  const int chunk = (n4 + S - 1) / S;
  const int g_end = min(n4, (slice + 1) * chunk);

  // ---- one pass: softmax(x / T)_i / e_i = exp(x_i / T - log e_i) / Z, so
  // its argmax is the argmax of x_i / T - log(max(e_i, 1e-10)) (ties: lowest
  // index); no max / sum over the row is needed for the pick
  const uint32_t k0 = (uint32_t)seed, k1 = (uint32_t)(seed >> 32);
  const float invT = 1.0f / T;
  float best = -INFINITY;
  int besti = 0x7FFFFFFF;
  for (int g = slice * chunk + tid; g < g_end; g += SNT) {
    float x[4];
    load4(row, 4ll * g, V, x, vec);
    const uint64_t lo = (uint64_t)(uint32_t)offset + (uint64_t)g;
    uint32_t c[4] = {(uint32_t)lo, (uint32_t)(offset >> 32) + (uint32_t)(lo >> 32), (uint32_t)b, 0x53414D50u};
    philox4x32_10(c, k0, k1);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int i = 4 * g + e;
      if (i >= V) continue;
      const float ev = exp1_from_word(c[e]);
      if (noise_out != nullptr) noise_out[(int64_t)b * V + i] = ev;
      // ranking only: x * (1/T) and the hardware log2 are within a few ulp
      // of x / T and log, which can only reorder near-ties
      const float score = x[e] * invT - __log2f(fmaxf(ev, 1e-10f)) * 0.6931471805599453f;
      if (score > best || (score == best && i < besti)) {
        best = score;
        besti = i;
      }
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float v2 = __shfl_xor(best, o, 64);
    const int i2 = __shfl_xor(besti, o, 64);
    if (v2 > best || (v2 == best && i2 < besti)) { best = v2; besti = i2; }
  }
  if (lane == 0) { red_v[wave] = best; red_i[wave] = besti; }
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < SNT / 64; ++w)
      if (red_v[w] > best || (red_v[w] == best && red_i[w] < besti)) { best = red_v[w]; besti = red_i[w]; }
    if (part != nullptr) part[(int64_t)b * S + slice] = make_uint2(__float_as_uint(best), (uint32_t)besti);
    else out[b] = besti == 0x7FFFFFFF ? 0 : besti;
  }
}

// Each row's best over its S slices (slices in index order, so the rule
// "larger score, or equal score and smaller index" picks what one pass
// over the row picks).
__global__ __launch_bounds__(256) void sample_gumbel_reduce_kernel(const uint2* __restrict__ part, int64_t B, int S,
                                                                   int64_t* __restrict__ out) {
  const int64_t b = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (b >= B) return;
  float best = -INFINITY;
  int besti = 0x7FFFFFFF;
  for (int s = 0; s < S; ++s) {
    const uint2 p = part[b * S + s];
    const float v = __uint_as_float(p.x);
    const int i = (int)p.y;
    if (v > best || (v == best && i < besti)) { best = v; besti = i; }
  }
  out[b] = besti == 0x7FFFFFFF ? 0 : besti;
}

// Slices per row: enough workgroups for two per CU, each slice at least
// one element group per thread.
int sampler_slices(int64_t B, int V) {
  static int cu_cache[64] = {0};
  int cus = 256, dev = 0;
  if (hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < 64) {
    if (cu_cache[dev] == 0) {
      int n = 0;
      cu_cache[dev] = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0
                          ? n : 256;
    }
    cus = cu_cache[dev];
  }
  if (B <= 0) return 1;
  const int64_t by_cus = (2 * (int64_t)cus + B - 1) / B;
  const int64_t by_len = std::max<int64_t>(1, ((int64_t)V + 4 * SNT - 1) / (4 * SNT));
  return (int)std::max<int64_t>(1, std::min<int64_t>({by_cus, by_len, 16}));
}

}  // namespace
}  // namespace lfs

using namespace lfs;

extern "C" int lfs_sample_gumbel(const void* logits, int64_t ld, const float* temperatures, int64_t B,
                                 int32_t vocab, uint64_t seed, uint64_t offset, int64_t* out, float* noise_out,
                                 void* stream) {
  LFS_REQUIRE(B >= 0 && vocab > 0 && ld >= vocab, "sample_gumbel: bad shape B=%lld V=%d ld=%lld", (long long)B,
              vocab, (long long)ld);
  if (B == 0) return 0;
  LFS_REQUIRE(logits && temperatures && out, "sample_gumbel: null pointer");
  LFS_REQUIRE(B < (1ll << 31), "sample_gumbel: too many rows");
  hipLaunchKernelGGL(sample_gumbel_kernel, dim3((unsigned)B, 1), dim3(SNT), 0, (hipStream_t)stream,
                     (const uint16_t*)logits, ld, temperatures, vocab, seed, offset, out, noise_out, nullptr);
  return check_launch("sample_gumbel");
}

extern "C" int64_t lfs_sample_gumbel_workspace_bytes(int64_t B, int32_t vocab) {
  if (B < 0 || vocab <= 0) return -1;
  const int S = sampler_slices(B, vocab);
  return S > 1 ? 8 * B * S : 0;
}

extern "C" int lfs_sample_gumbel_split(const void* logits, int64_t ld, const float* temperatures, int64_t B,
                                       int32_t vocab, uint64_t seed, uint64_t offset, int64_t* out,
                                       float* noise_out, void* workspace, int64_t workspace_bytes, void* stream) {
  LFS_REQUIRE(B >= 0 && vocab > 0 && ld >= vocab, "sample_gumbel: bad shape B=%lld V=%d ld=%lld", (long long)B,
              vocab, (long long)ld);
  if (B == 0) return 0;
  LFS_REQUIRE(logits && temperatures && out, "sample_gumbel: null pointer");
  LFS_REQUIRE(B < (1ll << 31), "sample_gumbel: too many rows");
  const int S = sampler_slices(B, vocab);
  if (S == 1)
    return lfs_sample_gumbel(logits, ld, temperatures, B, vocab, seed, offset, out, noise_out, stream);
  LFS_REQUIRE(workspace != nullptr && workspace_bytes >= 8 * B * S && ((uintptr_t)workspace & 7u) == 0,
              "sample_gumbel: workspace of %lld bytes < required %lld (8-byte aligned)", (long long)workspace_bytes,
              (long long)(8 * B * S));
  hipStream_t st = (hipStream_t)stream;
  hipLaunchKernelGGL(sample_gumbel_kernel, dim3((unsigned)B, (unsigned)S), dim3(SNT), 0, st, (const uint16_t*)logits,
                     ld, temperatures, vocab, seed, offset, out, noise_out, (uint2*)workspace);
  const int rc = check_launch("sample_gumbel(slices)");
  if (rc) return rc;
  hipLaunchKernelGGL(sample_gumbel_reduce_kernel, dim3((unsigned)((B + 255) / 256)), dim3(256), 0, st,
                     (const uint2*)workspace, B, S, out);
  return check_launch("sample_gumbel(reduce)");
}
