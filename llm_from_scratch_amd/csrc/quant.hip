// Block-wise FP8 (OCP e4m3fn) quantisation kernels for gfx950.
//
//  act_quant       1 x GS groups along rows (GS = 32/64/128), one 16-byte
//                  chunk (8 bf16) per lane, group amax by an xor butterfly
//                  over GS/8 lanes.  Restates model/attention/utils.py:97-172.
//  weight_quant    GS x GS blocks, one workgroup per block, block amax via
//                  a wave butterfly plus LDS across the four waves.
//  weight_dequant  bf16_RNE(e4m3 * block scale), 8 elements per lane.
//
// All three are HBM-bound streaming kernels (2 B read + 1 B written per
// element for the quantisers, 1 B read + 2 B written for dequant).
#include "common.h"

namespace lfs {

// ------------------------------------------------------------ act_quant --
// One lane per 8 consecutive elements (one 16-byte load); a group of GS
// elements is GS/8 consecutive lanes of one wave, reduced with shuffles.
// A workgroup takes AQ_U blocks of 256 consecutive chunks and issues all
// their loads before any arithmetic; input and codes are streamed once, so
// loads and stores are nontemporal.  A chunk's row is floor(idx * m >> sh)
// with m = ceil(2^sh / cpr), sh = 31 + ceil(log2 cpr) (Granlund and
// Montgomery, "Division by invariant integers using multiplication", 1994:
// exact for every idx below 2^31), not a 64-bit division.
//
// The quotients are div_by_group's (the IEEE divide with the divisor's
// half done once per group); the sign of a zero quotient comes back from
// the input's bf16 sign bits by one byte permute per four codes.
constexpr int AQ_U = 2;

// e4m3 codes of 4 quotients, with the sign bits of their inputs (two bf16
// pairs lo, hi) or-ed in: bytes 1 and 3 of each pair hold the signs at bit 7
__device__ __forceinline__ uint32_t e4m3_signed(float a, float b, float c, float d, uint32_t lo, uint32_t hi) {
  const uint32_t sg = __builtin_amdgcn_perm(hi, lo, 0x07050301u) & 0x80808080u;
  return f32x4_to_e4m3(a, b, c, d) | sg;
}

template <int GS, bool ROUND>
__global__ __launch_bounds__(256) void act_quant_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                        uint8_t* __restrict__ y,
                                                        float* __restrict__ s, uint32_t total,
                                                        uint32_t cpr, uint64_t magic, uint32_t shift) {
  constexpr int LPG = GS / 8;  // lanes per group; groups never straddle waves
  typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
  typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));
  const uint32_t base = blockIdx.x * (256u * AQ_U) + threadIdx.x;
  u32x4_t v[AQ_U];
  uint32_t rows[AQ_U], cols[AQ_U];
#pragma unroll
  for (int j = 0; j < AQ_U; ++j) {
    const uint32_t idx = base + 256u * j;
    rows[j] = (uint32_t)(((uint64_t)idx * magic) >> shift);
    cols[j] = idx - rows[j] * cpr;
    if (idx < total)
      v[j] = __builtin_nontemporal_load(
          reinterpret_cast<const u32x4_t*>(x + (int64_t)rows[j] * ldx + (int64_t)cols[j] * 8));
  }
#pragma unroll
  for (int j = 0; j < AQ_U; ++j) {
    // cpr % LPG == 0 and 256 % LPG == 0, so a group's lanes are all in or all out
    if (base + 256u * j >= total) break;
    const int64_t row = rows[j], c8 = cols[j];
    const uint4 w = make_uint4(v[j][0], v[j][1], v[j][2], v[j][3]);
    float f[8];
    unpack8(w, f);
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(f[i]));
    amax = group_max<LPG>(amax);
    const float sc = scale_from_amax(amax, ROUND);
    uint2 o;
    if (sc < INFINITY) {
      const float r = recip_for_div(sc);
      float q[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) q[i] = div_by_group(f[i], sc, r);
      o.x = e4m3_signed(q[0], q[1], q[2], q[3], w.x, w.y);
      o.y = e4m3_signed(q[4], q[5], q[6], q[7], w.z, w.w);
    } else {
      o = quant8_ieee(f, sc);
    }
    __builtin_nontemporal_store(u32x2_t{o.x, o.y}, reinterpret_cast<u32x2_t*>(y + row * (int64_t)cpr * 8 + c8 * 8));
    if ((c8 & (LPG - 1)) == 0) s[row * ((int64_t)cpr * 8 / GS) + c8 / LPG] = sc;
  }
}

// --------------------------------------------------------- weight_quant --
template <int BS>
__global__ __launch_bounds__(256) void weight_quant_kernel(const uint16_t* __restrict__ w,
                                                           uint8_t* __restrict__ y,
                                                           float* __restrict__ s, int64_t N,
                                                           int64_t K, int64_t kblocks) {
  constexpr int CPR = BS / 8;                     // 16-byte chunks per block row
  constexpr int CHUNKS = BS * CPR;
  constexpr int PER = (CHUNKS + 255) / 256;       // chunks per thread
  __shared__ float red[4];
  const int64_t r0 = (int64_t)blockIdx.y * BS;
  const int64_t c0 = (int64_t)blockIdx.x * BS;
  float f[PER][8];
  bool ok[PER];
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int c = threadIdx.x + 256 * i;
    const int64_t row = r0 + c / CPR;
    const int64_t col = c0 + (c % CPR) * 8;
    ok[i] = (c < CHUNKS) && row < N && col < K;
    if (ok[i]) {
      const uint4 v = *reinterpret_cast<const uint4*>(w + row * K + col);
      unpack8(v, f[i]);
#pragma unroll
      for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(f[i][e]));
    }
  }
  amax = group_max<64>(amax);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float sc = scale_from_amax(amax, false);
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    if (ok[i]) {
      const int c = threadIdx.x + 256 * i;
      const int64_t row = r0 + c / CPR;
      const int64_t col = c0 + (c % CPR) * 8;
      *reinterpret_cast<uint2*>(y + row * K + col) = quant8(f[i], sc);
    }
  }
  if (threadIdx.x == 0) s[(int64_t)blockIdx.y * kblocks + blockIdx.x] = sc;
}

// ------------------------------------------------------- weight_dequant --
__global__ __launch_bounds__(256) void weight_dequant_kernel(const uint8_t* __restrict__ w,
                                                             const float* __restrict__ s,
                                                             uint16_t* __restrict__ y, int64_t N,
                                                             int64_t K, int bs, int64_t kblocks) {
  const int64_t cpr = K / 8;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= N * cpr) return;
  const int64_t row = idx / cpr;
  const int64_t col = (idx - row * cpr) * 8;
  const float sc = s[(row / bs) * kblocks + col / bs];  // a chunk never straddles a block
  const uint2 v = *reinterpret_cast<const uint2*>(w + row * K + col);
  float f[8];
  e4m3x4_to_f32(v.x, f);
  e4m3x4_to_f32(v.y, f + 4);
  uint4 o;
  o.x = pack_bf16x2(f[0] * sc, f[1] * sc);
  o.y = pack_bf16x2(f[2] * sc, f[3] * sc);
  o.z = pack_bf16x2(f[4] * sc, f[5] * sc);
  o.w = pack_bf16x2(f[6] * sc, f[7] * sc);
  *reinterpret_cast<uint4*>(y + row * K + col) = o;
}

static bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

}  // namespace lfs

using namespace lfs;

extern "C" int lfs_act_quant(const void* x, int64_t ldx, void* y, float* s, int64_t M, int64_t K,
                             int32_t block_size, int32_t round_scale, void* stream) {
  LFS_REQUIRE(M >= 0 && K >= 0, "act_quant: negative shape M=%lld K=%lld", (long long)M,
              (long long)K);
  LFS_REQUIRE(block_size == 32 || block_size == 64 || block_size == 128,
              "act_quant: block_size must be 32, 64 or 128 (got %d)", block_size);
  LFS_REQUIRE(K % block_size == 0,
              "Last dimension size must be divisible by block_size (block_size=%d)", block_size);
  LFS_REQUIRE(ldx >= K && ldx % 8 == 0, "act_quant: row stride %lld must be >= K and a multiple of 8",
              (long long)ldx);
  if (M == 0 || K == 0) return 0;
  LFS_REQUIRE(x && y && s, "act_quant: null pointer");
  LFS_REQUIRE(aligned16(x) && ((uintptr_t)y & 7u) == 0 && ((uintptr_t)s & 3u) == 0,
              "act_quant: misaligned buffer");
  const int64_t chunks = M * (K / 8);
  LFS_REQUIRE(chunks + 256 * AQ_U < (1ll << 31), "act_quant: M*K=%lld elements is too large", (long long)(M * K));
  // m * cpr - 2^sh lies in [0, cpr) and cpr <= 2^(sh - 31), so idx * m >> sh
  // is floor(idx / cpr) for idx < 2^31; m < 2^33 keeps idx * m below 2^64
  const uint32_t cpr = (uint32_t)(K / 8);
  uint32_t lg = 0;
  while ((1ull << lg) < cpr) ++lg;
  const uint32_t shift = 31 + lg;
  const uint64_t magic = ((1ull << shift) + cpr - 1) / cpr;
  const dim3 grid((unsigned)((chunks + 256 * AQ_U - 1) / (256 * AQ_U)));
  hipStream_t st = (hipStream_t)stream;
  const uint16_t* xp = (const uint16_t*)x;
  uint8_t* yp = (uint8_t*)y;
#define LFS_AQ(GS, R) \
  hipLaunchKernelGGL((act_quant_kernel<GS, R>), grid, dim3(256), 0, st, xp, ldx, yp, s, (uint32_t)chunks, cpr, magic, shift)
  if (round_scale) {
    if (block_size == 32) LFS_AQ(32, true);
    else if (block_size == 64) LFS_AQ(64, true);
    else LFS_AQ(128, true);
  } else {
    if (block_size == 32) LFS_AQ(32, false);
    else if (block_size == 64) LFS_AQ(64, false);
    else LFS_AQ(128, false);
  }
#undef LFS_AQ
  return check_launch("act_quant");
}

extern "C" int lfs_weight_quant(const void* w, void* y, float* s, int64_t N, int64_t K,
                                int32_t block_size, void* stream) {
  LFS_REQUIRE(N >= 0 && K >= 0, "weight_quant: negative shape");
  LFS_REQUIRE(block_size == 32 || block_size == 64 || block_size == 128,
              "weight_quant: block_size must be 32, 64 or 128 (got %d)", block_size);
  LFS_REQUIRE(K % 8 == 0, "weight_quant: K=%lld must be a multiple of 8", (long long)K);
  if (N == 0 || K == 0) return 0;
  LFS_REQUIRE(w && y && s, "weight_quant: null pointer");
  LFS_REQUIRE(aligned16(w) && ((uintptr_t)y & 7u) == 0, "weight_quant: misaligned buffer");
  const int64_t nb = (N + block_size - 1) / block_size, kb = (K + block_size - 1) / block_size;
  LFS_REQUIRE(nb < 65536, "weight_quant: N too large");
  const dim3 grid((unsigned)kb, (unsigned)nb);
  hipStream_t st = (hipStream_t)stream;
  if (block_size == 128)
    hipLaunchKernelGGL(weight_quant_kernel<128>, grid, dim3(256), 0, st, (const uint16_t*)w, (uint8_t*)y, s, N, K, kb);
  else if (block_size == 64)
    hipLaunchKernelGGL(weight_quant_kernel<64>, grid, dim3(256), 0, st, (const uint16_t*)w, (uint8_t*)y, s, N, K, kb);
  else
    hipLaunchKernelGGL(weight_quant_kernel<32>, grid, dim3(256), 0, st, (const uint16_t*)w, (uint8_t*)y, s, N, K, kb);
  return check_launch("weight_quant");
}

extern "C" int lfs_weight_dequant(const void* w, const float* s, void* y, int64_t N, int64_t K,
                                  int32_t block_size, void* stream) {
  LFS_REQUIRE(N >= 0 && K >= 0, "weight_dequant: negative shape");
  LFS_REQUIRE(block_size >= 8 && block_size % 8 == 0, "weight_dequant: block_size must be a multiple of 8");
  LFS_REQUIRE(K % 8 == 0, "weight_dequant: K=%lld must be a multiple of 8", (long long)K);
  if (N == 0 || K == 0) return 0;
  LFS_REQUIRE(w && s && y, "weight_dequant: null pointer");
  LFS_REQUIRE(((uintptr_t)w & 7u) == 0 && aligned16(y), "weight_dequant: misaligned buffer");
  const int64_t kb = (K + block_size - 1) / block_size;
  const int64_t chunks = N * (K / 8);
  hipLaunchKernelGGL(weight_dequant_kernel, dim3((unsigned)((chunks + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, (const uint8_t*)w, s, (uint16_t*)y, N, K, block_size, kb);
  return check_launch("weight_dequant");
}
