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
// rest is two xor shuffles (16, 32).  One wave per (b, query m, chunk of
// 256 keys), four queries of one batch row per workgroup; the wave keeps
// its q rows (h / 16 operand fragments) in registers and streams k.
#include "common.h"

namespace lfs {
namespace {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int IDX_NCHUNK = 256;  // keys per wave

template <int HB>  // 16-head blocks
__global__ __launch_bounds__(256) void fp8_index_kernel(const uint8_t* __restrict__ q, const float* __restrict__ q_s,
                                                        const uint8_t* __restrict__ k, const float* __restrict__ k_s,
                                                        float* __restrict__ o, int M, int N, int H, int D,
                                                        int64_t k_stride_b, int64_t ks_stride_b) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int b = blockIdx.z, m = blockIdx.y * 4 + wave;
  if (m >= M) return;
  const int n_begin = blockIdx.x * IDX_NCHUNK;
  const int c16 = lane & 15, g = lane >> 4;
  // this lane's 32 bytes of a row: [32g, 32g + 32) of the (zero-padded) 128
  const bool have = 32 * g < D;

  // q fragments: head hb*16 + c16, and its weight for the fold below
  v8i qf[HB];
  float qw[HB][4];
  const int64_t qrow = ((int64_t)b * M + m) * H;
#pragma unroll
  for (int hb = 0; hb < HB; ++hb) {
    const int h = hb * 16 + c16;
    uint4 lo = make_uint4(0, 0, 0, 0), hi = make_uint4(0, 0, 0, 0);
    if (have && h < H) {
      const uint8_t* p = q + (qrow + h) * D + 32 * g;
      lo = *reinterpret_cast<const uint4*>(p);
      hi = *reinterpret_cast<const uint4*>(p + 16);
    }
    qf[hb] = v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int hr = hb * 16 + 4 * g + r;  // the heads this lane's results belong to
      qw[hb][r] = hr < H ? q_s[qrow + hr] : 0.f;
    }
  }

  const uint8_t* kb = k + (int64_t)b * k_stride_b;
  const float* ksb = k_s + (int64_t)b * ks_stride_b;
  float* orow = o + ((int64_t)b * M + m) * N;
  const int n_end = min(N, n_begin + IDX_NCHUNK);
  for (int n0 = n_begin; n0 < n_end; n0 += 16) {
    const int n = min(n0 + c16, N - 1);  // rows past N are clamped, not stored
    uint4 lo = make_uint4(0, 0, 0, 0), hi = make_uint4(0, 0, 0, 0);
    if (have) {
      const uint8_t* p = kb + (int64_t)n * D + 32 * g;
      lo = *reinterpret_cast<const uint4*>(p);
      hi = *reinterpret_cast<const uint4*>(p + 16);
    }
    const v8i kf = v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
    float acc = 0.f;
#pragma unroll
    for (int hb = 0; hb < HB; ++hb) {
      const v4f z = {0.f, 0.f, 0.f, 0.f};
      // D[head][key]: lane holds key c16, heads hb*16 + 4g .. +3
      const v4f s = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(qf[hb], kf, z, 0, 0, 0, 0, 0, 0);
#pragma unroll
      for (int r = 0; r < 4; ++r) acc = fmaf(fmaxf(s[r], 0.f), qw[hb][r], acc);
    }
    acc += __shfl_xor(acc, 16, 64);
    acc += __shfl_xor(acc, 32, 64);
    if (g == 0 && n0 + c16 < n_end) orow[n0 + c16] = acc * ksb[n0 + c16];
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
  LFS_REQUIRE(B < 65536 && (M + 3) / 4 < 65536, "fp8_index: grid too large");
  const dim3 grid((unsigned)((N + IDX_NCHUNK - 1) / IDX_NCHUNK), (unsigned)((M + 3) / 4), (unsigned)B);
  hipStream_t st = (hipStream_t)stream;
  const int hb = (H + 15) / 16;
#define LFS_IX(HB)                                                                                             \
  case HB:                                                                                                     \
    hipLaunchKernelGGL(fp8_index_kernel<HB>, grid, dim3(256), 0, st, (const uint8_t*)q, q_s, (const uint8_t*)k, \
                       k_s, o, M, N, H, D, k_stride_b, ks_stride_b);                                           \
    break;
  switch (hb) {
    LFS_IX(1) LFS_IX(2) LFS_IX(3) LFS_IX(4) LFS_IX(5) LFS_IX(6) LFS_IX(7) LFS_IX(8)
    default: LFS_REQUIRE(false, "fp8_index: unsupported head count %d", H);
  }
#undef LFS_IX
  return check_launch("fp8_index");
}
