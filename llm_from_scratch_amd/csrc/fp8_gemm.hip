// Block-scaled FP8 GEMM on gfx950 MFMA.
//
//   C[m,n] = bf16( sum_kb a_s[m,kb] * b_s[n/128,kb] * (A[m,kb*128:+128] . B[n,kb*128:+128]) + bias[n] )
//
// One 128-wide K block is exactly one v_mfma_f32_16x16x128_f8f6f4 per 16x16
// output tile, so every MFMA starts from a zero accumulator and its result is
// folded into the fp32 running sum with the per-row x per-block scale product
// (4 FMAs per tile per K block).  The scales are arbitrary fp32 values, so the
// hardware's power-of-two (E8M0) operand scaling cannot carry them.
//
// Workgroup tile 128x128, four waves in a 2x2 grid, 64x64 per wave (4x4 MFMA
// tiles).  A and B K-tiles (16 KB each) are staged through LDS with a double
// buffer: the next K block's global loads are issued before the current
// block's MFMAs and written to the other LDS buffer afterwards, so one
// barrier per K block suffices.  16-byte chunks are XOR-swizzled within each
// 128-byte LDS row to spread the MFMA operand reads over the banks.
//
// MFMA operand convention: lane l supplies row (l % 16) of A and row (l % 16)
// of B (= column of C) and the 32 bytes [32*(l/16), 32*(l/16)+32) of the
// 128-byte K block; A and B use the same K assignment, so the dot products
// pair the same K indices whatever order the instruction sums them in.  The
// 16x16 fp32 result in lane l is column (l % 16), rows 4*(l/16) .. +3.
#include "common.h"

namespace lfs {
namespace {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int BM = 128, BN = 128, BK = 128;

__device__ __forceinline__ int swz(int row, int chunk) {
  return row * BK + ((chunk ^ (row & 7)) << 4);
}

__device__ __forceinline__ v4f mfma_fp8(const v8i& a, const v8i& b) {
  const v4f z = {0.f, 0.f, 0.f, 0.f};
  // format codes 0/0 = e4m3 x e4m3; zero scale operands select the unscaled op
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, z, 0, 0, 0, 0, 0, 0);
}

__global__ __launch_bounds__(256, 2) void fp8_gemm_128x128(
    const uint8_t* __restrict__ A, const float* __restrict__ As, const uint8_t* __restrict__ B,
    const float* __restrict__ Bs, const float* __restrict__ bias, uint16_t* __restrict__ C, int M,
    int N, int K) {
  __shared__ __attribute__((aligned(16))) uint8_t sA[2][BM * BK];
  __shared__ __attribute__((aligned(16))) uint8_t sB[2][BN * BK];
  __shared__ __attribute__((aligned(16))) float sAs[2][BM];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
  const int KT = K / BK;

  uint4 ra[4], rb[4];
  float ras = 0.f;
  auto gload = [&](int kt) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = tid + 256 * i;
      const int row = c >> 3, ch = c & 7;
      const int gm = m0 + row, gn = n0 + row;
      ra[i] = gm < M ? *reinterpret_cast<const uint4*>(A + (size_t)gm * K + kt * BK + ch * 16)
                     : make_uint4(0, 0, 0, 0);
      rb[i] = gn < N ? *reinterpret_cast<const uint4*>(B + (size_t)gn * K + kt * BK + ch * 16)
                     : make_uint4(0, 0, 0, 0);
    }
    if (tid < BM) {
      const int gm = m0 + tid;
      ras = gm < M ? As[(size_t)gm * KT + kt] : 0.f;
    }
  };
  auto sstore = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = tid + 256 * i;
      const int row = c >> 3, ch = c & 7;
      *reinterpret_cast<uint4*>(&sA[buf][swz(row, ch)]) = ra[i];
      *reinterpret_cast<uint4*>(&sB[buf][swz(row, ch)]) = rb[i];
    }
    if (tid < BM) sAs[buf][tid] = ras;
  };

  v4f acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};

  const int r16 = lane & 15, g = lane >> 4;
  const float* bs_row = Bs + (size_t)(n0 / 128) * KT;

  gload(0);
  sstore(0);
  __syncthreads();
  for (int kt = 0; kt < KT; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < KT) gload(kt + 1);
    const float bsv = bs_row[kt];

    v8i fa[4], fb[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = wm * 64 + i * 16 + r16;
      const uint4 lo = *reinterpret_cast<const uint4*>(&sA[buf][swz(row, 2 * g)]);
      const uint4 hi = *reinterpret_cast<const uint4*>(&sA[buf][swz(row, 2 * g + 1)]);
      fa[i] = v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int row = wn * 64 + j * 16 + r16;
      const uint4 lo = *reinterpret_cast<const uint4*>(&sB[buf][swz(row, 2 * g)]);
      const uint4 hi = *reinterpret_cast<const uint4*>(&sB[buf][swz(row, 2 * g + 1)]);
      fb[j] = v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
    }
    float sc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float4 a4 = *reinterpret_cast<const float4*>(&sAs[buf][wm * 64 + i * 16 + g * 4]);
      sc[i][0] = a4.x * bsv; sc[i][1] = a4.y * bsv; sc[i][2] = a4.z * bsv; sc[i][3] = a4.w * bsv;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const v4f t = mfma_fp8(fa[i], fb[j]);
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[i][j][r] = fmaf(t[r], sc[i][r], acc[i][j][r]);
      }
    if (kt + 1 < KT) sstore(buf ^ 1);
    __syncthreads();
  }

#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int col = n0 + wn * 64 + j * 16 + r16;
    const float bv = (bias != nullptr && col < N) ? bias[col] : 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = m0 + wm * 64 + i * 16 + g * 4 + r;
        if (row < M && col < N) C[(size_t)row * N + col] = (uint16_t)f32_to_bf16(acc[i][j][r] + bv);
      }
  }
}

}  // namespace
}  // namespace lfs

using namespace lfs;

extern "C" int lfs_fp8_gemm(const void* a, const float* a_s, const void* b, const float* b_s,
                            const float* bias, void* c, int64_t M, int64_t N, int64_t K,
                            void* stream) {
  LFS_REQUIRE(M >= 0 && N >= 0 && K >= 0, "fp8_gemm: negative shape");
  LFS_REQUIRE(K % 128 == 0, "fp8_gemm: K=%lld must be a multiple of 128", (long long)K);
  LFS_REQUIRE(M < (1ll << 31) && N < (1ll << 31) && K < (1ll << 31) && M * K < (1ll << 40),
              "fp8_gemm: shape too large");
  if (M == 0 || N == 0) return 0;
  LFS_REQUIRE(a && a_s && b && b_s && c, "fp8_gemm: null pointer");
  LFS_REQUIRE(K > 0, "fp8_gemm: K must be positive");
  LFS_REQUIRE((((uintptr_t)a | (uintptr_t)b) & 15u) == 0, "fp8_gemm: a and b must be 16-byte aligned");
  const dim3 grid((unsigned)((N + BN - 1) / BN), (unsigned)((M + BM - 1) / BM));
  LFS_REQUIRE(grid.y < 65536u, "fp8_gemm: M too large");
  hipLaunchKernelGGL(fp8_gemm_128x128, grid, dim3(256), 0, (hipStream_t)stream, (const uint8_t*)a,
                     a_s, (const uint8_t*)b, b_s, bias, (uint16_t*)c, (int)M, (int)N, (int)K);
  return check_launch("fp8_gemm");
}
