// FP8 lightning-indexer scores for gfx950 (the DSA indexer's fp8_index,
// model/attention/utils.py:175-250 of the reference):
//
//   o[b, m, n] = k_s[b, n] * sum_h relu(q[b, m, h, :] . k[b, n, :]) * q_s[b, m, h]
//
// q, k e4m3fn; the dot products on v_mfma_f32_16x16x128_f8f6f4 (head dim
// d <= 128, zero-padded to 128), fp32 everywhere after.  A 16-head block of
// q[b, m] is the first operand and a 16-key block of k[b] the second, so
// lane l ends with key (l % 16) and heads 4(l / 16) .. +3 of the block: the
// ReLU, the head weights and three of the head sums stay in the lane, the
// rest is two xor shuffles (16, 32).
//
// One workgroup per (b, 8 queries, chunk of IDX_NCHUNK keys), one wave per
// query; the wave keeps its query's H/16 operand fragments in registers.
// The chunk's keys pass through LDS in tiles of 64, loaded once for the
// eight waves (double-buffered, the next tile's global loads in flight
// during the current tile's MFMAs).  Operand K bytes: lane l supplies
// 16-byte chunks g and g + 4 (g = l / 16) of the 128-byte row for both q
// and k -- the same permutation of the head dim on both sides -- so the
// sixteen rows of one LDS read hit every bank once with the swizzle below.
#include "common.h"

namespace lfs {
namespace {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int IDX_NCHUNK = 512;  // keys per workgroup
constexpr int IDX_QPW = 8;       // queries (waves) per workgroup
constexpr int IDX_KT = 64;       // keys per LDS tile

// byte offset of 16-byte chunk c of key row r in an LDS tile of D-byte rows
template <int D>
__device__ __forceinline__ int kswz(int r, int c) {
  if constexpr (D == 128) return r * 128 + ((c ^ (((r >> 1) & 7) ^ ((r & 1) << 2))) << 4);
  else if constexpr (D == 64) return r * 64 + ((c ^ ((r >> 2) & 3)) << 4);
  else return r * D + (c << 4);
}

template <int HB, int D>  // HB: 16-head blocks
__global__ __launch_bounds__(64 * IDX_QPW) void fp8_index_kernel(
    const uint8_t* __restrict__ q, const float* __restrict__ q_s, const uint8_t* __restrict__ k,
    const float* __restrict__ k_s, float* __restrict__ o, int M, int N, int H, int64_t k_stride_b,
    int64_t ks_stride_b) {
  constexpr int CPR = D / 16;                 // 16-byte chunks per key row
  constexpr int TCH = IDX_KT * CPR;           // chunks per LDS tile
  constexpr int NT = 64 * IDX_QPW;
  constexpr int CPT = (TCH + NT - 1) / NT;    // chunks per thread per tile
  __shared__ __attribute__((aligned(16))) uint8_t kt[2][IDX_KT * D];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int b = blockIdx.z, m = blockIdx.y * IDX_QPW + wave;
  const bool active = m < M;  // inactive waves still take part in the barriers
  const int n_begin = blockIdx.x * IDX_NCHUNK;
  const int n_end = min(N, n_begin + IDX_NCHUNK);
  const int c16 = lane & 15, g = lane >> 4;
  const bool lo_ok = 16 * g < D, hi_ok = 16 * (g + 4) < D;  // this lane's chunks g, g + 4 exist

  // q fragments (head hb*16 + c16, chunks g and g + 4) and the weights of
  // the heads this lane's results belong to
  v8i qf[HB];
  float qw[HB][4];
  const int64_t qrow = ((int64_t)b * M + min(m, M - 1)) * H;
#pragma unroll
  for (int hb = 0; hb < HB; ++hb) {
    const int h = hb * 16 + c16;
    uint4 lo = make_uint4(0, 0, 0, 0), hi = make_uint4(0, 0, 0, 0);
    if (h < H) {
      const uint8_t* p = q + (qrow + h) * D;
      if (lo_ok) lo = *reinterpret_cast<const uint4*>(p + 16 * g);
      if (hi_ok) hi = *reinterpret_cast<const uint4*>(p + 16 * (g + 4));
    }
    qf[hb] = v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int hr = hb * 16 + 4 * g + r;
      qw[hb][r] = hr < H ? q_s[qrow + hr] : 0.f;
    }
  }

  const uint8_t* kb = k + (int64_t)b * k_stride_b;
  const float* ksb = k_s + (int64_t)b * ks_stride_b;
  float* orow = o + ((int64_t)b * M + m) * N;
  // chunk u of tile starting at key t0: key t0 + u / CPR (clamped to the
  // last key; those rows are never stored), chunk u % CPR
  auto load_tile = [&](uint4 (&kr)[CPT], int t0) {
#pragma unroll
    for (int e = 0; e < CPT; ++e) {
      const int u = threadIdx.x + NT * e;
      kr[e] = make_uint4(0, 0, 0, 0);
      if (u < TCH) kr[e] = *reinterpret_cast<const uint4*>(kb + (int64_t)min(t0 + u / CPR, N - 1) * D + (u % CPR) * 16);
    }
  };
  auto store_tile = [&](const uint4 (&kr)[CPT], int buf) {
#pragma unroll
    for (int e = 0; e < CPT; ++e) {
      const int u = threadIdx.x + NT * e;
      if (u < TCH) *reinterpret_cast<uint4*>(&kt[buf][kswz<D>(u / CPR, u % CPR)]) = kr[e];
    }
  };

  const int ntiles = (n_end - n_begin + IDX_KT - 1) / IDX_KT;
  uint4 kr[CPT];
  load_tile(kr, n_begin);
  store_tile(kr, 0);
  __syncthreads();
  for (int ti = 0; ti < ntiles; ++ti) {
    const int t0 = n_begin + ti * IDX_KT;
    const int buf = ti & 1;
    if (ti + 1 < ntiles) load_tile(kr, t0 + IDX_KT);
    if (active) {
      const uint8_t* tile = kt[buf];
#pragma unroll
      for (int st = 0; st < IDX_KT / 16; ++st) {
        const int r = 16 * st + c16;
        uint4 lo = make_uint4(0, 0, 0, 0), hi = make_uint4(0, 0, 0, 0);
        if (lo_ok) lo = *reinterpret_cast<const uint4*>(tile + kswz<D>(r, g));
        if (hi_ok) hi = *reinterpret_cast<const uint4*>(tile + kswz<D>(r, g + 4));
        const v8i kf = v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
        float acc = 0.f;
#pragma unroll
        for (int hb = 0; hb < HB; ++hb) {
          const v4f z = {0.f, 0.f, 0.f, 0.f};
          // D[head][key]: lane holds key c16, heads hb*16 + 4g .. +3
          const v4f s = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(qf[hb], kf, z, 0, 0, 0, 0, 0, 0);
#pragma unroll
          for (int x = 0; x < 4; ++x) acc = fmaf(fmaxf(s[x], 0.f), qw[hb][x], acc);
        }
        acc += __shfl_xor(acc, 16, 64);
        acc += __shfl_xor(acc, 32, 64);
        const int n = t0 + 16 * st + c16;
        if (g == 0 && n < n_end) orow[n] = acc * ksb[n];
      }
    }
    if (ti + 1 < ntiles) store_tile(kr, buf ^ 1);  // buffer buf ^ 1 was last read in tile ti - 1
    __syncthreads();
  }
}

}  // namespace
}  // namespace lfs

using namespace lfs;

extern "C" int lfs_fp8_index(const void* q, const float* q_s, const void* k, const float* k_s, float* o,
                             int64_t B, int32_t M, int32_t N, int32_t H, int32_t D, int64_t k_stride_b,
                             int64_t ks_stride_b, void* stream) {
  LFS_REQUIRE(B >= 0 && M >= 0 && N >= 0 && H > 0, "fp8_index: bad shape");
  LFS_REQUIRE(D == 32 || D == 64 || D == 128, "fp8_index: head_dim must be 32, 64 or 128 (got %d)", D);
  LFS_REQUIRE(H <= 128, "fp8_index: at most 128 heads (got %d)", H);
  if (B == 0 || M == 0 || N == 0) return 0;
  LFS_REQUIRE(q && q_s && k && k_s && o, "fp8_index: null pointer");
  LFS_REQUIRE(k_stride_b >= (int64_t)N * D && ks_stride_b >= N, "fp8_index: k batch stride too small");
  LFS_REQUIRE(((((uintptr_t)q) | ((uintptr_t)k)) & 15u) == 0 && (k_stride_b % 16) == 0,
              "fp8_index: q and k rows must be 16-byte aligned");
  LFS_REQUIRE(B < 65536 && (M + IDX_QPW - 1) / IDX_QPW < 65536, "fp8_index: grid too large");
  const dim3 grid((unsigned)((N + IDX_NCHUNK - 1) / IDX_NCHUNK), (unsigned)((M + IDX_QPW - 1) / IDX_QPW),
                  (unsigned)B);
  hipStream_t st = (hipStream_t)stream;
  const int hb = (H + 15) / 16;
  const uint8_t *qq = (const uint8_t*)q, *kk = (const uint8_t*)k;
#define LFS_IX(HB, DD)                                                                                       \
  hipLaunchKernelGGL((fp8_index_kernel<HB, DD>), grid, dim3(64 * IDX_QPW), 0, st, qq, q_s, kk, k_s, o, M, N, H, \
                     k_stride_b, ks_stride_b)
#define LFS_IXD(HB)                    \
  case HB:                             \
    if (D == 128) LFS_IX(HB, 128);     \
    else if (D == 64) LFS_IX(HB, 64);  \
    else LFS_IX(HB, 32);               \
    break;
  switch (hb) {
    LFS_IXD(1) LFS_IXD(2) LFS_IXD(3) LFS_IXD(4) LFS_IXD(5) LFS_IXD(6) LFS_IXD(7) LFS_IXD(8)
    default: LFS_REQUIRE(false, "fp8_index: unsupported head count %d", H);
  }
#undef LFS_IXD
#undef LFS_IX
  return check_launch("fp8_index");
}
