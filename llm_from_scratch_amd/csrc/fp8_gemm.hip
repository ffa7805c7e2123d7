// Block-scaled FP8 GEMM on gfx950 MFMA.
//
//   C[m,n] = bf16( sum_kb a_s[m,kb] * b_s[n/128,kb] * (A[m,kb*128:+128] . B[n,kb*128:+128]) + bias )
//   with bias = bias[n] (bias_ld == 0) or bias[m*bias_ld + n] (a per-row bias matrix)
//
// One 128-wide K block is exactly one v_mfma_f32_16x16x128_f8f6f4 per 16x16
// output tile, so every MFMA starts from a zero accumulator and its result is
// folded into the fp32 running sum with the per-row x per-block scale product
// (4 FMAs per tile per K block).  The scales are arbitrary fp32 values, so the
// hardware's power-of-two (E8M0) operand scaling cannot carry them.
//
// Kernels: fp8_gemm_persist, 256 x 256 tiles (128x64 per wave, one 8-wave
// workgroup per CU walking its tiles) for shapes with at least half a round
// of such tiles; fp8_gemm_big, the same tile with one workgroup per tile,
// for the other large shapes; fp8_gemm_tile, a 128 x 128 tile (64x64 per
// wave, two workgroups per CU, optional split-K or two K slices per
// workgroup; also the grouped MoE GEMM); fp8_gemm_skinny for M <= 128.
// A and B K-tiles are copied global -> LDS by DMA (no register staging);
// the activation scales follow in chunks of whole rows.
//
// MFMA operand convention: lane l supplies row (l % 16) of each operand and
// 32 bytes of the 128-byte K block: 16-byte chunks (l/16) and (l/16)+4.
// Both operands use the same K assignment, so the dot products pair the
// same K indices whatever order the instruction sums them in.  (Chunks g and
// g+4 rather than 2g and 2g+1 make the sixteen rows of one read touch every
// LDS bank once with the swizzle below: full LDS read bandwidth on gfx950,
// against half of it for the adjacent pair.)  The 16x16 fp32 result
// D = X Y^T in lane l is column (l % 16), rows 4*(l/16) .. +3.
//
// Tile order: workgroup ids are dealt round-robin to the 8 XCDs, so the id
// is remapped to give each XCD a contiguous range of tiles, walked in groups
// of row-tiles so that concurrently running tiles share A rows and B
// columns in that XCD's L2.
#include <algorithm>

#include "common.h"

namespace lfs {
namespace {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

constexpr int BN = 128, BK = 128;
constexpr int GROUP_M = 8;

__device__ __forceinline__ v8i frag(const uint8_t* tile, int off_lo, int off_hi) {
  const u32x4 lo = *reinterpret_cast<const u32x4*>(tile + off_lo);
  const u32x4 hi = *reinterpret_cast<const u32x4*>(tile + off_hi);
  return __builtin_bit_cast(v8i, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
}

__device__ __forceinline__ v4f mfma_fp8(const v8i& a, const v8i& b) {
  const v4f z = {0.f, 0.f, 0.f, 0.f};
  // format codes 0/0 = e4m3 x e4m3; zero scale operands select the unscaled op
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, z, 0, 0, 0, 0, 0, 0);
}

typedef __attribute__((address_space(3))) uint8_t lds_u8;
__device__ __forceinline__ unsigned lds_addr(const void* p) {
  return (unsigned)(uintptr_t)(const lds_u8*)p;
}

// Direct global -> LDS loads (no VGPR staging).  Lane i's 16 (or 4) bytes
// land at LDS address m0 + 16*i (or 4*i).  Issued through inline asm so that
// the compiler does not pessimise every later LDS read with vmcnt(0); the
// kernel waits for them explicitly (wait_vm) before its barrier.  m0 is saved
// and restored around the load.
__device__ __forceinline__ void dma16(const void* g, unsigned lds) {
  unsigned tmp;
  asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %2, off\n\ts_mov_b32 m0, %0"
               : "=&s"(tmp) : "s"(lds), "v"(g) : "memory");
}
__device__ __forceinline__ void dma4(const void* g, unsigned lds) {
  unsigned tmp;
  asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\tglobal_load_lds_dword %2, off\n\ts_mov_b32 m0, %0"
               : "=&s"(tmp) : "s"(lds), "v"(g) : "memory");
}
// Same copy with a wave-uniform base address (SGPR pair) and a 32-bit
// per-lane byte offset, so that per-lane addresses cost one VGPR.
__device__ __forceinline__ void dma16s(const void* base_any, unsigned off, unsigned lds) {
  // uniform by construction; make it an SGPR pair (readfirstlane returns
  // int: each half goes through uint32_t so that the low word is not
  // sign-extended into the high one)
  const uint64_t b = (uint64_t)(uintptr_t)base_any;
  const uint64_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(b >> 32));
  const uint64_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)b);
  const void* base = (const void*)(uintptr_t)((hi << 32) | lo);
  unsigned tmp;
  asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %2, %3\n\ts_mov_b32 m0, %0"
               : "=&s"(tmp) : "s"(lds), "v"(off), "s"(base) : "memory");
}
// C is written once and never read again by the GEMM, while the A and B
// panels are re-read by the tiles of other XCDs (each XCD's 4 MB L2 holds
// only its own concurrent tiles' panels): C goes out with the streaming
// cache policy (nt sc1) so that it does not displace those panels from the
// 256 MB last-level cache.  Measured on the cfg2 sweep (six GEMMs back to
// back, as the benchmark runs them): 1.62 -> 1.97 PFLOP/s, bit-identical;
// nt alone gives 1.82.  kStreamStore is the buffer-store cache-policy
// operand (sc1 = 16, nt = 2); store_stream16 is the same store through a
// 64-bit address.
constexpr int kStreamStore = 16 | 2;
__device__ __forceinline__ void store_stream16(void* p, const u32x4& v) {
  asm volatile("global_store_dwordx4 %0, %1, off nt sc1" : : "v"(p), "v"(v) : "memory");
}

// LDS writes of this wave visible to its other lanes (no workgroup barrier)
__device__ __forceinline__ void wave_lds_fence() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// s_waitcnt lgkmcnt(0) (LDS reads of this wave complete), vmcnt unconstrained
__device__ __forceinline__ void wait_lgkm0() { __builtin_amdgcn_s_waitcnt(0xC07F); }

// s_waitcnt vmcnt(N), other counters unconstrained
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// LDS tile layout: 128-byte rows; 16-byte chunk c of row r is stored in
// chunk slot c ^ f(r), f(r) = ((r >> 1) & 7) ^ ((r & 1) << 2), which spreads
// the MFMA operand reads (16 rows x chunk g or g+4 per 16 lanes) over the
// banks.
// Each DMA instruction fills 8 whole rows: lane l writes slot (l & 7) of row
// 8s + (l >> 3), so it fetches logical chunk (l & 7) ^ f(row) -- 8 complete
// 128-byte lines per instruction, the access pattern the load path streams
// at full L2 bandwidth (a permutation inside a line costs nothing, a 16-byte
// gather over 16 rows costs 3x).
__device__ __forceinline__ int swz(int r, int c) {
  return r * BK + ((c ^ (((r >> 1) & 7) ^ ((r & 1) << 2))) << 4);
}

// Tile BM x 128 (BM = 128: 4 waves, BM = 256: 8 waves), 64x64 per wave,
// waves (wave >> 1, wave & 1) over the tile; 2 waves per SIMD either way.
// NST LDS stages, NST K blocks in flight during the MFMAs (see the
// read-then-refill loop below).
//   BM = 128, NST = 2: 72 KB of LDS, two workgroups per CU, so one
//     workgroup's barriers and LDS waits are covered by the other's MFMAs;
//   BM = 256, NST = 3: 152 KB, one workgroup per CU, every B tile shared by
//     four waves (not dispatched: slower on every benchmark shape).
// Scale products a_s * b_s are staged per chunk of SCK K blocks in a
// k-major table ([SCK][BM+1] floats) instead of one strided 4-byte gather
// per K block.
//
// GROUPED: one GEMM per expert over row segments (the MoE expert GEMMs).  C
// rows are grouped in 128-row tiles, tile tm belonging to expert
// tile_expert[tm] (< 0: the tile is unused and exits).  Row m of C takes A
// row row_index[m] (a gather of the tokens routed to the expert; < 0 reads
// row 0, whose result is padding) or, with row_index null, A row m.  The
// expert's weights are B + e * b_es (rows ldb bytes apart), its scales
// Bs + e * bs_es (rows ldbs floats apart), its bias bias + e * bias_es.
struct Grouped {
  const int32_t* tile_expert;
  const int32_t* row_index;
  int64_t b_es, bs_es, bias_es;
  int a_rows;
};

template <int BM, int NST, int SCK, bool GROUPED = false, int KS = 1>
__global__ __launch_bounds__(BM * 2 * KS, KS == 1 ? 256 / BM : 1) void fp8_gemm_tile(
    const uint8_t* __restrict__ A, const float* __restrict__ As, const uint8_t* __restrict__ B,
    const float* __restrict__ Bs, const float* __restrict__ bias, int64_t bias_ld, uint16_t* __restrict__ C, int M,
    int N, int K, int tiles_m, int tiles_n, float* __restrict__ ws, int kps, int64_t ldb, int ldbs, Grouped grp) {
  constexpr int NW = BM / 32;       // waves per K slice
  constexpr int NT = 64 * NW * KS;  // threads
  constexpr int SCP = BM + 1;       // padded row of the k-major scale table
  constexpr int A_BYTES = BM * BK, B_BYTES = BN * BK;
  constexpr int SLOT = A_BYTES + B_BYTES;  // one K block
  constexpr int STAGE = KS * SLOT;         // one K block per slice
  constexpr int A_PER_WAVE = A_BYTES / 1024 / NW;  // 1 KB (8-row) segments per wave
  constexpr int B_PER_WAVE = B_BYTES / 1024 / NW;
  constexpr int LOADS = A_PER_WAVE + B_PER_WAVE;  // DMA instructions per wave per stage
  static_assert(NW * 8192 <= NST * STAGE, "epilogue staging must fit the stage buffers");
  static_assert(KS == 1 || (KS - 1) * NW * 16384 <= NST * STAGE, "slice partials must fit the stage buffers");
  static_assert(SCK % KS == 0, "a scale chunk holds whole iterations");
  __shared__ __attribute__((aligned(1024))) uint8_t smem[NST * STAGE];
  __shared__ __attribute__((aligned(16))) float ssc[SCK * SCP];

  // ---- tile order (XCD-contiguous ranges, grouped rows)
  int pid = blockIdx.x;
  const int ntiles = tiles_m * tiles_n;
  if ((ntiles & 7) == 0) pid = (pid & 7) * (ntiles >> 3) + (pid >> 3);
  const int group = pid / (GROUP_M * tiles_n);
  const int first_m = group * GROUP_M;
  const int gsize = min(tiles_m - first_m, GROUP_M);
  const int tm = first_m + (pid % gsize);
  const int tn = (pid % (GROUP_M * tiles_n)) / gsize;
  const int m0 = tm * BM, n0 = tn * BN;
  __shared__ int s_arow[GROUPED ? BM : 1];  // A row of each tile row (gathered)
  if constexpr (GROUPED) {
    const int e = grp.tile_expert[tm];
    if (e < 0) return;  // whole workgroup, before any barrier
    B += e * grp.b_es;
    Bs += e * grp.bs_es;
    if (bias != nullptr) bias += e * grp.bias_es;
    for (int r = threadIdx.x; r < BM; r += BM * 2) {
      const int m = min(m0 + r, M - 1);
      const int ar = grp.row_index != nullptr ? grp.row_index[m] : m;
      s_arow[r] = min(max(ar, 0), grp.a_rows - 1);
    }
    __syncthreads();
  }
  // A row of tile row r (rows past M are clamped; their results are never stored)
  auto arow = [&](int r) -> int {
    if constexpr (GROUPED) return s_arow[r];
    else return min(m0 + r, M - 1);
  };

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  // KS > 1: KS slices of NW waves; slice ks multiplies K blocks ks, ks + KS,
  // ... of the range (two waves per SIMD on a workgroup that has its CU to
  // itself), and the slices' sums are added through LDS at the end
  const int ks = __builtin_amdgcn_readfirstlane((tid >> 6) / NW);  // wave-uniform (SGPR)
  const int wave = __builtin_amdgcn_readfirstlane((tid >> 6) % NW);
  const int wm = wave >> 1, wn = wave & 1;
  const int KTA = K / BK;                  // K blocks of a row (scale row stride)
  // split-K: this workgroup sums K blocks kb0 .. kb0+KT-1 (blockIdx.y-th
  // split of kps blocks) and, with more than one split, writes its fp32
  // partial tile to ws[split] instead of C
  const int kb0 = blockIdx.y * kps;
  const int KT = min(kps, KTA - kb0);
  const int r16 = lane & 15, g = lane >> 4;

  // ---- DMA sources: segment q = wave + NW*u covers tile rows 8q .. 8q+7
  // (rows past M / N are clamped; their results are never stored)
  const uint8_t* srcA[A_PER_WAVE];
  const uint8_t* srcB[B_PER_WAVE];
#pragma unroll
  for (int u = 0; u < A_PER_WAVE; ++u) {
    const int r = 8 * (wave + NW * u) + (lane >> 3);
    const int c = (lane & 7) ^ (((r >> 1) & 7) ^ ((r & 1) << 2));
    srcA[u] = A + (size_t)arow(r) * K + (size_t)kb0 * BK + c * 16;
  }
#pragma unroll
  for (int u = 0; u < B_PER_WAVE; ++u) {
    const int r = 8 * (wave + NW * u) + (lane >> 3);
    const int c = (lane & 7) ^ (((r >> 1) & 7) ^ ((r & 1) << 2));
    srcB[u] = B + (size_t)min(n0 + r, N - 1) * ldb + (size_t)kb0 * BK + c * 16;
  }
  const unsigned lds0 = __builtin_amdgcn_readfirstlane(lds_addr(smem));
  const float* bs_row = Bs + (size_t)(n0 / 128) * ldbs + kb0;
  const float* as_base = As + kb0;

  auto issue = [&](int kt, int buf) {  // K block kt into slot ks of stage buf
    const unsigned base = lds0 + buf * STAGE + ks * SLOT;
#pragma unroll
    for (int u = 0; u < A_PER_WAVE; ++u) dma16(srcA[u] + kt * BK, base + (wave + NW * u) * 1024);
#pragma unroll
    for (int u = 0; u < B_PER_WAVE; ++u) dma16(srcB[u] + kt * BK, base + A_BYTES + (wave + NW * u) * 1024);
  };
  // scale products a_s[m, kb] * b_s[n0/128, kb] for K blocks kt0 .. +SCK-1,
  // stored k-major ([SCK][BM+1], conflict-free both ways); ordinary
  // bounds-checked loads, 16 consecutive K blocks of a row per 16 lanes
  auto load_scales = [&](int kt0) {
    const int nk = min(SCK, KT - kt0);
#pragma unroll
    for (int v = 0; v < BM * SCK / NT; ++v) {
      const int idx = tid + NT * v;
      const int row = idx / SCK, k = idx % SCK;
      ssc[k * SCP + row] =
          k < nk ? as_base[(size_t)arow(row) * KTA + kt0 + k] * bs_row[kt0 + k] : 0.f;
    }
  };

  // operand read offsets (loop invariant)
  int offA[4][2], offB[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    offA[i][0] = swz(wm * 64 + i * 16 + r16, g);
    offA[i][1] = swz(wm * 64 + i * 16 + r16, g + 4);
    offB[i][0] = A_BYTES + swz(wn * 64 + i * 16 + r16, g);
    offB[i][1] = A_BYTES + swz(wn * 64 + i * 16 + r16, g + 4);
  }
  // C = A B^T is formed as (B A^T)^T: the MFMA's first operand is the B
  // fragment, so lane l holds output row 16i + (l % 16), columns
  // 16j + 4(l / 16) .. +3 -- one activation scale per lane per m-tile, and
  // 8 contiguous bytes of C per lane in the epilogue
  const float* scrow = ssc + wm * 64 + r16;

  v4f acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};

  // Read-then-refill ring: an iteration copies its whole stage into
  // registers (fragments + scales), passes a second barrier, and only then
  // refills that same buffer with K block kt + NST, so NST blocks are in
  // flight while the MFMAs run (the LDS holds only NST stages).
  // Every stage refill is issued, also past the last K block (it then
  // re-copies block KT-1 into the stage just read, which is never read
  // again), so that exactly NST-1 copy groups follow block kt's and the wait
  // below is one constant count.
  // the stage copies go out first: the scale table's loads (whose values
  // must be in registers before they are staged) then share their round trip
  // (KS > 1: iteration it holds blocks it*KS .. it*KS + KS-1, slot ks
  // holding block it*KS + ks; a slot past the last block re-copies it)
  const int IT = (KT + KS - 1) / KS;
#pragma unroll
  for (int s = 0; s < NST; ++s) issue(min(s * KS + ks, KT - 1), s);
  load_scales(0);
  // A bias vector is loaded now, inside the first copies' round trip: read
  // in the epilogue it would cost short-K calls one more round trip there.
  float bvec[4][4];
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int col = n0 + wn * 64 + j * 16 + 4 * g + r;
      bvec[j][r] = (bias != nullptr && bias_ld == 0 && ws == nullptr && col < N) ? bias[col] : 0.f;
    }

  for (int it = 0; it < IT; ++it) {
    const int kt = it * KS + ks;  // this slice's K block (past the range: nothing to multiply)
    if (it > 0 && (it * KS) % SCK == 0) load_scales(it * KS);  // old chunk last read before the previous B2
    wait_vm<(NST - 1) * LOADS>();  // this wave's copies of iteration it landed
    __syncthreads();  // B1: iteration it (and the scale chunk) visible to every wave
    const uint8_t* st = smem + (it % NST) * STAGE + ks * SLOT;
    const int kc = kt % SCK;
    v8i fa[4], fb[4];
    float sc[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      fa[i] = frag(st, offA[i][0], offA[i][1]);
      fb[i] = frag(st, offB[i][0], offB[i][1]);
      sc[i] = scrow[kc * SCP + i * 16];
    }
    wait_lgkm0();     // this wave's reads of the buffer have completed
    __syncthreads();  // B2: every wave is done with buffer it % NST
    // refill buffer it % NST with iteration it + NST; its copies are spread
    // over the MFMA sequence (one per two MFMAs) so that no wave waits
    // behind a full load queue before its MFMAs.
    const int kn = min((it + NST) * KS + ks, KT - 1);
    const unsigned rbase = lds0 + (it % NST) * STAGE + ks * SLOT;
    const bool live = KS == 1 || kt < KT;
    // MFMA k is issued, then the FMAs fold the product of MFMA k-2, which
    // has retired by then; scheduling fences keep the compiler from pulling
    // a fold up behind its own MFMA (which would idle the matrix core)
    v4f t[16];
#pragma unroll
    for (int k = 0; k < 18; ++k) {
      if (k < 16) t[k] = mfma_fp8(fb[k & 3], fa[k >> 2]);
      if ((k & 1) == 1 && (k >> 1) < LOADS) {
        const int d = k >> 1;
        if (d < A_PER_WAVE) dma16(srcA[d] + kn * BK, rbase + (wave + NW * d) * 1024);
        else dma16(srcB[d - A_PER_WAVE] + kn * BK, rbase + A_BYTES + (wave + NW * (d - A_PER_WAVE)) * 1024);
      }
      if (k >= 2) {
        const int p = k - 2;
        const float f = live ? sc[p >> 2] : 0.f;  // a slice past the range adds zeros
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[p >> 2][p & 3][r] = fmaf(t[p][r], f, acc[p >> 2][p & 3][r]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  wait_vm<0>();  // the trailing re-copies have landed before the stages are reused or the workgroup ends
  if constexpr (KS > 1) {
    // slice sums into slice 0, in slice order, through the idle stage buffers
    __syncthreads();  // every wave is done with the stage buffers
    v4f* part = reinterpret_cast<v4f*>(smem);  // [KS-1][NW][16 tiles][64 lanes]
    if (ks > 0) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) part[(((ks - 1) * NW + wave) * 16 + i * 4 + j) * 64 + lane] = acc[i][j];
    }
    __syncthreads();
    if (ks == 0) {
#pragma unroll
      for (int s2 = 1; s2 < KS; ++s2)
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const v4f x = part[(((s2 - 1) * NW + wave) * 16 + i * 4 + j) * 64 + lane];
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[i][j][r] += x[r];
          }
    }
    if (ws != nullptr && ks > 0) return;  // (the split-K store below has no barrier)
  }
  if (ws != nullptr) {
    // split-K partial: fp32, no bias; lane holds rows 16i + r16, columns
    // 16j + 4g .. +3 of its wave's 64x64 tile
    float* wsp = ws + (size_t)blockIdx.y * M * N;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = m0 + wm * 64 + i * 16 + r16;
      if (row >= M) continue;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int col = n0 + wn * 64 + j * 16 + 4 * g;
        float* dst = wsp + (size_t)row * N + col;
        if (col + 3 < N && (N & 3) == 0) {
          *reinterpret_cast<float4*>(dst) = make_float4(acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]);
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (col + r < N) dst[r] = acc[i][j][r];
        }
      }
    }
    return;
  }

  // ---- epilogue: bias, bf16 (RNE), then each wave's 64x64 tile goes
  // through LDS (the idle stage buffers) so that global stores are whole
  // 128-byte rows: 16-byte chunk c of row r sits at chunk slot c ^ (r & 7)
  __syncthreads();  // every wave is done with the stage buffers (and with the slice sums)
  if (KS > 1 && ks > 0) return;
  uint8_t* ot = smem + wave * 8192;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int cl = j * 16 + 4 * g;  // first of this lane's 4 columns in the wave tile
    float bv[4] = {bvec[j][0], bvec[j][1], bvec[j][2], bvec[j][3]};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int rl = i * 16 + r16;
      if (bias != nullptr && bias_ld != 0) {
        const int row = m0 + wm * 64 + rl;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int col = n0 + wn * 64 + cl + r;
          bv[r] = (row < M && col < N) ? bias[(int64_t)row * bias_ld + col] : 0.f;
        }
      }
      uint2 o;
      o.x = pack_bf16x2(acc[i][j][0] + bv[0], acc[i][j][1] + bv[1]);
      o.y = pack_bf16x2(acc[i][j][2] + bv[2], acc[i][j][3] + bv[3]);
      *reinterpret_cast<uint2*>(ot + rl * 128 + (((cl >> 3) ^ (rl & 7)) << 4) + (cl & 7) * 2) = o;
    }
  }
  wave_lds_fence();
  const int colw = n0 + wn * 64;
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    const int rl = u * 8 + (lane >> 3), c = lane & 7;
    const int row = m0 + wm * 64 + rl;
    const u32x4 v = *reinterpret_cast<const u32x4*>(ot + rl * 128 + ((c ^ (rl & 7)) << 4));
    if (row >= M) continue;
    uint16_t* dst = C + (size_t)row * N + colw + c * 8;
    if (colw + c * 8 + 7 < N && (N & 7) == 0) {
      store_stream16(dst, v);
    } else {
      const uint16_t* h = reinterpret_cast<const uint16_t*>(&v);
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (colw + c * 8 + e < N) dst[e] = h[e];
    }
  }
}

// ---------------------------------------------------------------------------
// Skinny GEMM for decode-sized M (<= 128): one workgroup per 16 * NT
// (NT = 2, or 1 for narrow N) output columns and all M rows, in WGM groups of four waves; group gm owns row
// tiles gm*MTW .. gm*MTW + MTW - 1, and its wave kw takes K blocks kw,
// kw+4, ... (each block: MTW x 2 MFMAs, the B fragments as the first operand
// so a lane ends with one activation row and four weight columns, i.e. one
// a_s * b_s product per lane and row tile; the next block's fragments are
// loaded before the current block's MFMAs).  The four partial sums of a
// group are added through LDS in wave order, wave kw finishing row tiles
// kw, kw + 4, ... of its group (bias, bf16 rounding).  At M = 128 and
// N = 1280 that is 40 workgroups where the 128 x 128 tile kernel has 10,
// with no split-K workspace or second kernel.

// KW waves of a group split the K blocks (4, or 8 / 16 for one 16-row tile
// and long K: more K blocks in flight at once, still one launch).
template <int MTW, int WGM, int KW = 4, int NT = 2>
__global__ __launch_bounds__(64 * KW * WGM) void fp8_gemm_skinny(
    const uint8_t* __restrict__ A, const float* __restrict__ As, const uint8_t* __restrict__ B,
    const float* __restrict__ Bs, const float* __restrict__ bias, int64_t bias_ld, uint16_t* __restrict__ C,
    int M, int N, int K) {
  __shared__ __attribute__((aligned(16))) v4f red[WGM][KW][MTW][NT][64];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int gm = wave / KW, kw = wave % KW;
  const int r16 = lane & 15, g = lane >> 4;
  const int n0 = blockIdx.x * 16 * NT;
  const int KT = K / BK;
  const uint8_t* brow[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) brow[nt] = B + (size_t)min(n0 + 16 * nt + r16, N - 1) * K + g * 16;
  // activation rows as 32-bit offsets (M * K < 2^31 is checked on the host)
  uint32_t aoff[MTW], soff[MTW];
#pragma unroll
  for (int mt = 0; mt < MTW; ++mt) {
    const uint32_t m = (uint32_t)min(16 * (gm * MTW + mt) + r16, M - 1);
    aoff[mt] = m * (uint32_t)K + g * 16;
    soff[mt] = m * (uint32_t)KT;
  }
  const float* bsrow = Bs + (size_t)(n0 / 128) * KT;  // the 16 NT columns share one 128-row scale block

  v4f acc[MTW][NT];
#pragma unroll
  for (int mt = 0; mt < MTW; ++mt)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) acc[mt][nt] = v4f{0.f, 0.f, 0.f, 0.f};

  // operand chunks g and g + 4 of the 128-byte K block (both operands)
  auto ld = [](const uint8_t* p) -> v8i {
    const u32x4 lo = *reinterpret_cast<const u32x4*>(p);
    const u32x4 hi = *reinterpret_cast<const u32x4*>(p + 64);
    return __builtin_bit_cast(v8i, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
  };
  // two register buffers, filled alternately (no copies between them)
  v8i bf0[NT], af0[MTW], bf1[NT], af1[MTW];
  float sa0[MTW], sa1[MTW], sb0 = 0.f, sb1 = 0.f;
  auto load_block = [&](v8i (&bf)[NT], v8i (&af)[MTW], float (&sa)[MTW], float& sb, int kb) {
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) bf[nt] = ld(brow[nt] + (size_t)kb * BK);
#pragma unroll
    for (int mt = 0; mt < MTW; ++mt) {
      af[mt] = ld(A + aoff[mt] + (uint32_t)kb * BK);
      sa[mt] = As[soff[mt] + kb];
    }
    sb = bsrow[kb];
  };
  auto compute = [&](const v8i (&bf)[NT], const v8i (&af)[MTW], const float (&sa)[MTW], float sb) {
#pragma unroll
    for (int mt = 0; mt < MTW; ++mt) {
      const float sc = sa[mt] * sb;
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        const v4f t = mfma_fp8(bf[nt], af[mt]);
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[mt][nt][r] = fmaf(t[r], sc, acc[mt][nt][r]);
      }
    }
  };
  if (kw < KT) load_block(bf0, af0, sa0, sb0, kw);
  // a bias vector rides the first round trip (read after the reduction it
  // would add one at the end)
  float bvec[NT][4];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int col = n0 + 16 * nt + 4 * g + r;
      bvec[nt][r] = (bias != nullptr && bias_ld == 0 && kw < MTW && col < N) ? bias[col] : 0.f;
    }
  for (int kb = kw; kb < KT; kb += 2 * KW) {
    if (kb + KW < KT) load_block(bf1, af1, sa1, sb1, kb + KW);
    compute(bf0, af0, sa0, sb0);
    if (kb + KW >= KT) break;
    if (kb + 2 * KW < KT) load_block(bf0, af0, sa0, sb0, kb + 2 * KW);
    compute(bf1, af1, sa1, sb1);
  }

  // ---- the KW partials of the group, summed in wave order
#pragma unroll
  for (int mt = 0; mt < MTW; ++mt)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) red[gm][kw][mt][nt][lane] = acc[mt][nt];
  __syncthreads();
  for (int mt = kw; mt < MTW; mt += KW) {
    const int m = 16 * (gm * MTW + mt) + r16;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      v4f s = red[gm][0][mt][nt][lane];
#pragma unroll
      for (int w = 1; w < KW; ++w) {
        const v4f x = red[gm][w][mt][nt][lane];
#pragma unroll
        for (int r = 0; r < 4; ++r) s[r] += x[r];
      }
      const int col = n0 + 16 * nt + 4 * g;
      if (m >= M) continue;
      float bv[4] = {bvec[nt][0], bvec[nt][1], bvec[nt][2], bvec[nt][3]};
      if (bias != nullptr && bias_ld != 0) {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (col + r < N) bv[r] = bias[(int64_t)m * bias_ld + col + r];
      }
      uint16_t* dst = C + (size_t)m * N + col;
      if (col + 3 < N && (N & 3) == 0) {
        uint2 o;
        o.x = pack_bf16x2(s[0] + bv[0], s[1] + bv[1]);
        o.y = pack_bf16x2(s[2] + bv[2], s[3] + bv[3]);
        *reinterpret_cast<uint2*>(dst) = o;
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (col + r < N) dst[r] = (uint16_t)f32_to_bf16(s[r] + bv[r]);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// One-shot GEMM for decode-sized M (<= 16 * MT <= 128).  A workgroup owns all
// M rows, NC 16-column tiles (n0 = 16 * NC * blockIdx.x) and a range of at
// most KBM K blocks (blockIdx.y-th split of kps blocks), and copies every
// operand byte it needs -- the A rows and B rows of its K range -- global ->
// LDS in one burst before its first MFMA: a call is one memory round trip,
// its MFMAs and its store, instead of a pipeline that pays a round trip per
// stage refill.  Waves are WR row groups x WK K groups: wave (rg, kg)
// multiplies row tiles rg*MT/WR .. +MT/WR-1 by all NC column tiles over the
// K blocks kg, kg + WK, ... of the range; the WK partial sums of a row group
// are added through LDS in K-group order.  With one split the result is
// bf16(sum + bias); with several, the fp32 partial tile goes to
// ws[split][M][N] (no bias) for a reduction or a consumer that sums them.
// LDS: K block j of the range holds A (16 * MT rows) then, after all A
// blocks, B (16 * NC rows), 128-byte rows in the swizzled chunk order of the
// tile kernels.
// AQ: A is bf16 (row stride lda elements) and the workgroup quantises its
// rows itself as act_quant(A, 128) does -- each 128-value group's amax over
// 16 lanes, the same scale and codes -- writing the codes to LDS where the
// copies would have put act_quant's, and the scales to a small LDS table:
// the result equals act_quant followed by the same kernel on its output,
// bit for bit (one split only).
template <int MT, int NC, int KBM, int WR, int WK, bool AQ = false>
__global__ __launch_bounds__(64 * WR * WK) void fp8_gemm_flat(
    const uint8_t* __restrict__ A, const float* __restrict__ As, const uint8_t* __restrict__ B,
    const float* __restrict__ Bs, const float* __restrict__ bias, int64_t bias_ld, uint16_t* __restrict__ C,
    float* __restrict__ ws, int M, int N, int K, int kps, int64_t lda = 0) {
  constexpr int NW = WR * WK;
  constexpr int RT = MT / WR;                  // row tiles per wave
  constexpr int KW = (KBM + WK - 1) / WK;      // K blocks per wave (at most)
  constexpr int A_BLK = MT * 16 * BK, B_BLK = NC * 16 * BK;
  constexpr int SEGS = 2 * (MT + NC);          // 1 KB copies per K block
  static_assert(MT % WR == 0 && NC <= 8, "flat GEMM geometry");
  // 128-column weight-scale blocks the workgroup's columns touch: one when
  // 16*NC divides 128 (n0 is then a multiple of 16*NC inside one block)
  constexpr bool ONE_SB = 128 % (16 * NC) == 0;
  static_assert((WK - 1) * WR * RT * NC * 1024 <= KBM * (A_BLK + B_BLK), "K-group sums must fit the LDS");
  __shared__ __attribute__((aligned(1024))) uint8_t smem[KBM * (A_BLK + B_BLK)];
  __shared__ float sa_lds[AQ ? MT * 16 * KBM : 1];  // AQ: scale of (row, K block)

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int rg = wave / WK, kg = wave % WK;
  const int r16 = lane & 15, g = lane >> 4;
  const int n0 = blockIdx.x * 16 * NC;
  const int m0 = blockIdx.z * 16 * MT;  // first row of this workgroup's row tiles
  const int KT = K / BK;
  const int kb0 = blockIdx.y * kps;
  const int nkb = min(kps, KT - kb0);  // K blocks of this workgroup (1 .. KBM)
  const unsigned lds0 = __builtin_amdgcn_readfirstlane(lds_addr(smem));

  // ---- every copy of the workgroup, spread over its waves
  const int lrow = lane >> 3;
  for (int i = wave; i < nkb * SEGS; i += NW) {
    const int j = i / SEGS, seg = i - j * SEGS;
    const bool isA = seg < 2 * MT;
    if (AQ && isA) continue;  // quantised into LDS below
    const int r = 8 * (isA ? seg : seg - 2 * MT) + lrow;  // tile row of this lane
    const int c = (lane & 7) ^ (((r >> 1) & 7) ^ ((r & 1) << 2));
    const uint8_t* src = isA ? A + (size_t)min(m0 + r, M - 1) * K : B + (size_t)min(n0 + r, N - 1) * K;
    const unsigned dst = lds0 + (isA ? j * A_BLK + (r - lrow) * BK : KBM * A_BLK + j * B_BLK + (r - lrow) * BK);
    dma16(src + (size_t)(kb0 + j) * BK + c * 16, dst);
  }
  if constexpr (AQ) {
    // the workgroup's 16*MT rows x nkb K blocks of bf16 A as 8-value chunks,
    // chunk c = (row, K block, 16-byte-of-codes half): the 16 chunks of a
    // 128-value group are 16 consecutive lanes
    constexpr int NT = 64 * NW;
    constexpr int CPT = (MT * 16 * KBM * 16 + NT - 1) / NT;
    const int total = MT * 16 * nkb * 16;
    const uint16_t* Ab = reinterpret_cast<const uint16_t*>(A);
    uint4 raw[CPT];
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int c = threadIdx.x + NT * k;
      raw[k] = make_uint4(0, 0, 0, 0);
      if (c < total) {
        const int r = c / (nkb * 16), kc = c - r * (nkb * 16);
        raw[k] = *reinterpret_cast<const uint4*>(Ab + (int64_t)min(m0 + r, M - 1) * lda +
                                                 (int64_t)(kb0 * 16 + kc) * 8);
      }
    }
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int c = threadIdx.x + NT * k;
      if (c >= total) break;  // whole 16-lane groups are in or out (total % 16 == 0)
      const int r = c / (nkb * 16), kc = c - r * (nkb * 16);
      const int j = kc >> 4, cc = kc & 15;  // K block, chunk of the block
      float f[8];
      unpack8(raw[k], f);
      float amax = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(f[e]));
      amax = group_max<16>(amax);
      const float sc = scale_from_amax(amax, false);
      // logical 16-byte unit cc/2 of row r sits at unit (cc/2) ^ swz(r)
      const int unit = (cc >> 1) ^ (((r >> 1) & 7) ^ ((r & 1) << 2));
      *reinterpret_cast<uint2*>(smem + j * A_BLK + r * BK + unit * 16 + (cc & 1) * 8) = quant8(f, sc);
      if (cc == 0) sa_lds[r * KBM + j] = sc;
    }
  }
  // scales of this wave's rows and K blocks, and the bias vector, in the same round trip
  constexpr int NSB = ONE_SB ? 1 : NC;  // weight scales per K block: per column tile unless one block
  float sa[RT][KW], sb[NSB][KW];
#pragma unroll
  for (int jj = 0; jj < KW; ++jj) {
    const int j = kg + WK * jj;
    const int kb = kb0 + min(j, nkb - 1);
#pragma unroll
    for (int c = 0; c < NSB; ++c) sb[c][jj] = Bs[(size_t)(min(n0 + 16 * c, N - 1) / 128) * KT + kb];
    if constexpr (!AQ) {
#pragma unroll
      for (int t = 0; t < RT; ++t) sa[t][jj] = As[(size_t)min(m0 + 16 * (rg * RT + t) + r16, M - 1) * KT + kb];
    }
  }
  float bvec[NC][4];
#pragma unroll
  for (int c = 0; c < NC; ++c)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int col = n0 + 16 * c + 4 * g + r;
      bvec[c][r] = (bias != nullptr && bias_ld == 0 && ws == nullptr && col < N) ? bias[col] : 0.f;
    }
  wait_vm<0>();
  __syncthreads();
  if constexpr (AQ) {
#pragma unroll
    for (int jj = 0; jj < KW; ++jj) {
      const int j = min(kg + WK * jj, nkb - 1);
#pragma unroll
      for (int t = 0; t < RT; ++t) sa[t][jj] = sa_lds[(16 * (rg * RT + t) + r16) * KBM + j];
    }
  }

  v4f acc[RT][NC];
#pragma unroll
  for (int t = 0; t < RT; ++t)
#pragma unroll
    for (int c = 0; c < NC; ++c) acc[t][c] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int jj = 0; jj < KW; ++jj) {
    const int j = kg + WK * jj;
    if (j >= nkb) break;
    const uint8_t* at = smem + j * A_BLK;
    const uint8_t* bt = smem + KBM * A_BLK + j * B_BLK;
    v8i fb[NC], fa[RT];
#pragma unroll
    for (int c = 0; c < NC; ++c) fb[c] = frag(bt, swz(16 * c + r16, g), swz(16 * c + r16, g + 4));
#pragma unroll
    for (int t = 0; t < RT; ++t) {
      const int rt = rg * RT + t;
      fa[t] = frag(at, swz(16 * rt + r16, g), swz(16 * rt + r16, g + 4));
    }
#pragma unroll
    for (int t = 0; t < RT; ++t) {
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const float sc = sa[t][jj] * sb[ONE_SB ? 0 : c][jj];
        const v4f p = mfma_fp8(fb[c], fa[t]);  // lane: row 16 rt + r16, columns 16 c + 4 g .. +3
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[t][c][r] = fmaf(p[r], sc, acc[t][c][r]);
      }
    }
  }

  if constexpr (WK > 1) {  // K groups 1 .. WK-1 into group 0, in order, through the operand LDS
    __syncthreads();
    v4f* part = reinterpret_cast<v4f*>(smem);  // [WK-1][WR][RT][NC][64]
    if (kg > 0) {
#pragma unroll
      for (int t = 0; t < RT; ++t)
#pragma unroll
        for (int c = 0; c < NC; ++c) part[((((kg - 1) * WR + rg) * RT + t) * NC + c) * 64 + lane] = acc[t][c];
    }
    __syncthreads();
    if (kg > 0) return;
#pragma unroll
    for (int k2 = 1; k2 < WK; ++k2)
#pragma unroll
      for (int t = 0; t < RT; ++t)
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          const v4f x = part[((((k2 - 1) * WR + rg) * RT + t) * NC + c) * 64 + lane];
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[t][c][r] += x[r];
        }
  }

#pragma unroll
  for (int t = 0; t < RT; ++t) {
    const int row = m0 + 16 * (rg * RT + t) + r16;
    if (row >= M) continue;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int col = n0 + 16 * c + 4 * g;
      if (ws != nullptr) {
        float* dst = ws + (size_t)blockIdx.y * M * N + (size_t)row * N + col;
        if (col + 3 < N && (N & 3) == 0) {
          *reinterpret_cast<float4*>(dst) = make_float4(acc[t][c][0], acc[t][c][1], acc[t][c][2], acc[t][c][3]);
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (col + r < N) dst[r] = acc[t][c][r];
        }
        continue;
      }
      float bv[4] = {bvec[c][0], bvec[c][1], bvec[c][2], bvec[c][3]};
      if (bias != nullptr && bias_ld != 0) {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (col + r < N) bv[r] = bias[(int64_t)row * bias_ld + col + r];
      }
      uint16_t* dst = C + (size_t)row * N + col;
      if (col + 3 < N && (N & 3) == 0) {
        uint2 o;
        o.x = pack_bf16x2(acc[t][c][0] + bv[0], acc[t][c][1] + bv[1]);
        o.y = pack_bf16x2(acc[t][c][2] + bv[2], acc[t][c][3] + bv[3]);
        *reinterpret_cast<uint2*>(dst) = o;
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (col + r < N) dst[r] = (uint16_t)f32_to_bf16(acc[t][c][r] + bv[r]);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// 256x256 tile, 8 waves (2 x 4), 128 x 64 per wave (8 x 4 MFMA tiles).
//
// Half the global->LDS bytes per flop of the 128x128 tile and 3/4 of its LDS
// reads per MFMA.  Two 64 KB stages and one barrier per K block: after the
// barrier of block kt every wave has finished block kt-1, so block kt+1 is
// copied into that stage while block kt is multiplied.  The activation
// scales (k-major [SCKB][256] floats per chunk of SCKB K blocks, double
// buffered) and the tile's two weight-scale columns ([SCKB][2]) come through
// the same DMA path, so everything an iteration copies is one group that the
// wave waits for with vmcnt(0) before the barrier.  The eight 1 KB copies of
// a wave are spread over the first half of its MFMA sequence (one per two
// MFMAs): early enough that they land before the next barrier, spaced so
// that no wave waits behind a full load queue before its MFMAs (one per
// four MFMAs over the whole sequence measured 6-11% slower on the cfg2
// shapes).
//
// Per K block a wave reads its four B fragments, then streams its eight A
// fragments one 16-row m-tile ahead of the MFMAs; the fold of MFMA k into
// the fp32 accumulator runs two MFMAs behind it.
constexpr int BIG = 256, SCKB = 8, GROUP_M_BIG = 4;

__global__ __launch_bounds__(512, 1) void fp8_gemm_big(
    const uint8_t* __restrict__ A, const float* __restrict__ As, const uint8_t* __restrict__ B,
    const float* __restrict__ Bs, const float* __restrict__ bias, int64_t bias_ld, uint16_t* __restrict__ C, int M,
    int N, int K, int tiles_m, int tiles_n) {
  constexpr int A_BYTES = BIG * BK;    // 32 KB (B tile the same)
  constexpr int STAGE = 2 * A_BYTES;   // 64 KB
  __shared__ __attribute__((aligned(1024))) uint8_t smem[2 * STAGE];
  __shared__ __attribute__((aligned(1024))) float sas[2][SCKB][BIG];
  __shared__ __attribute__((aligned(64))) float sbs[2][SCKB][2];

  // ---- tile order (XCD-contiguous ranges, groups of GROUP_M_BIG row-tiles)
  int pid = blockIdx.x;
  const int ntiles = tiles_m * tiles_n;
  if ((ntiles & 7) == 0) pid = (pid & 7) * (ntiles >> 3) + (pid >> 3);
  const int group = pid / (GROUP_M_BIG * tiles_n);
  const int first_m = group * GROUP_M_BIG;
  const int gsize = min(tiles_m - first_m, GROUP_M_BIG);
  const int tm = first_m + (pid % gsize);
  const int tn = (pid % (GROUP_M_BIG * tiles_n)) / gsize;
  const int m0 = tm * BIG, n0 = tn * BIG;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 2, wn = wave & 3;
  const int KT = K / BK;
  const int nbs = (N + 127) / 128;  // weight-scale rows
  const int r16 = lane & 15, g = lane >> 4;

  // ---- DMA sources: segment q = wave + 8u (u = 0..3) is tile rows 8q .. 8q+7,
  // addressed as a uniform tile base plus a per-lane offset (rows past M / N
  // are clamped; their results are never stored).  The host guarantees
  // 256 * K < 2^31.
  unsigned offA[4], offB[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int r = 8 * (wave + 8 * u) + (lane >> 3);
    const int c = (lane & 7) ^ (((r >> 1) & 7) ^ ((r & 1) << 2));
    offA[u] = (unsigned)(min(m0 + r, M - 1) - m0) * (unsigned)K + c * 16;
    offB[u] = (unsigned)(min(n0 + r, N - 1) - n0) * (unsigned)K + c * 16;
  }
  const uint8_t* tileA = A + (size_t)m0 * K;
  const uint8_t* tileB = B + (size_t)n0 * K;
  const unsigned lds0 = __builtin_amdgcn_readfirstlane(lds_addr(smem));
  const unsigned lsas = __builtin_amdgcn_readfirstlane(lds_addr(&sas[0][0][0]));
  const unsigned lsbs = __builtin_amdgcn_readfirstlane(lds_addr(&sbs[0][0][0]));

  auto issue = [&](int kt, int buf) {
    const unsigned base = lds0 + buf * STAGE;
#pragma unroll
    for (int u = 0; u < 4; ++u) dma16s(tileA + (size_t)kt * BK, offA[u], base + (wave + 8 * u) * 1024);
#pragma unroll
    for (int u = 0; u < 4; ++u) dma16s(tileB + (size_t)kt * BK, offB[u], base + A_BYTES + (wave + 8 * u) * 1024);
  };
  // scale chunk for K blocks kb0 .. kb0+SCKB-1: wave w copies K block
  // kb0 + w for 256 rows (four 64-row dword copies); lanes 0-15 of wave 0
  // copy b_s[n0/128 + h][kb0 + k] to sbs[buf][k][h] (k = lane/2, h = lane%2).
  // Rows, weight-scale rows and K blocks past the end are clamped (unused).
  auto issue_scales = [&](int kb0, int buf) {
    const int kb = min(kb0 + wave, KT - 1);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const float* src = As + (size_t)min(m0 + 64 * u + lane, M - 1) * KT + kb;
      dma4(src, lsas + ((buf * SCKB + wave) * BIG + 64 * u) * 4);
    }
    if (wave == 0 && lane < 16) {
      const float* src = Bs + (size_t)min(n0 / 128 + (lane & 1), nbs - 1) * KT + min(kb0 + (lane >> 1), KT - 1);
      dma4(src, lsbs + buf * SCKB * 2 * 4);
    }
  };

  // operand read offsets: rows base + 16 i + r16 sit at i * 2048 plus a
  // per-lane offset (the swizzle depends only on r16)
  const int fsw = ((r16 >> 1) & 7) ^ ((r16 & 1) << 2);
  const int la0 = (wm * 128 + r16) * BK + ((g ^ fsw) << 4);
  const int la1 = (wm * 128 + r16) * BK + (((g + 4) ^ fsw) << 4);
  const int lb0 = A_BYTES + (wn * 64 + r16) * BK + ((g ^ fsw) << 4);
  const int lb1 = A_BYTES + (wn * 64 + r16) * BK + (((g + 4) ^ fsw) << 4);

  v4f acc[8][4];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};

  issue_scales(0, 0);
  issue(0, 0);
  for (int kt = 0; kt < KT; ++kt) {
    wait_vm<0>();     // this wave's copies of block kt (and its scale chunk) landed
    __syncthreads();  // everyone's copies landed; everyone is done with block kt-1
    if (kt + 1 < KT && (kt + 1) % SCKB == 0) issue_scales(kt + 1, ((kt + 1) / SCKB) & 1);
    const unsigned nbase = lds0 + ((kt + 1) & 1) * STAGE;
    const int kn = min(kt + 1, KT - 1);  // the last block re-copies itself into the free stage
    const uint8_t* st = smem + (kt & 1) * STAGE;
    const int sbuf = (kt / SCKB) & 1, kc = kt % SCKB;
    const float* sa = &sas[sbuf][kc][wm * 128 + r16];
    const float bsv = sbs[sbuf][kc][wn >> 1];
    v8i fb[4], fa[8];
    float sc[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) fb[j] = frag(st + j * 2048, lb0, lb1);
    fa[0] = frag(st, la0, la1);
    sc[0] = sa[0] * bsv;
    v4f t[32];
#pragma unroll
    for (int k = 0; k < 34; ++k) {
      if (k < 32) t[k] = mfma_fp8(fb[k & 3], fa[k >> 2]);
      if ((k & 1) == 0 && k < 16) {
        const int u = (k >> 1) & 3;
        if (k < 8) dma16s(tileA + (size_t)kn * BK, offA[u], nbase + (wave + 8 * u) * 1024);
        else dma16s(tileB + (size_t)kn * BK, offB[u], nbase + A_BYTES + (wave + 8 * u) * 1024);
      }
      if ((k & 3) == 0 && (k >> 2) + 1 < 8) {
        const int i1 = (k >> 2) + 1;
        fa[i1] = frag(st + i1 * 2048, la0, la1);
        sc[i1] = sa[16 * i1] * bsv;
      }
      if (k >= 2) {
        const int p = k - 2;
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[p >> 2][p & 3][r] = fmaf(t[p][r], sc[p >> 2], acc[p >> 2][p & 3][r]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  // ---- epilogue: bias, bf16 (RNE), each wave's 128x64 tile staged in LDS
  // (16 KB per wave, chunk c of row r at slot c ^ (r & 7)) so that global
  // stores are whole 128-byte rows
  wait_vm<0>();  // the last iteration's copy must land before the stages are reused
  __syncthreads();
  uint8_t* ot = smem + wave * 16384;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int cl = j * 16 + 4 * g;
    float bv[4] = {0.f, 0.f, 0.f, 0.f};
    if (bias != nullptr && bias_ld == 0) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int col = n0 + wn * 64 + cl + r;
        bv[r] = col < N ? bias[col] : 0.f;
      }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int rl = i * 16 + r16;
      if (bias != nullptr && bias_ld != 0) {
        const int row = m0 + wm * 128 + rl;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int col = n0 + wn * 64 + cl + r;
          bv[r] = (row < M && col < N) ? bias[(int64_t)row * bias_ld + col] : 0.f;
        }
      }
      uint2 o;
      o.x = pack_bf16x2(acc[i][j][0] + bv[0], acc[i][j][1] + bv[1]);
      o.y = pack_bf16x2(acc[i][j][2] + bv[2], acc[i][j][3] + bv[3]);
      *reinterpret_cast<uint2*>(ot + rl * 128 + (((cl >> 3) ^ (rl & 7)) << 4) + (cl & 7) * 2) = o;
    }
  }
  wave_lds_fence();
  const int colw = n0 + wn * 64;
#pragma unroll
  for (int u = 0; u < 16; ++u) {
    const int rl = u * 8 + (lane >> 3), c = lane & 7;
    const int row = m0 + wm * 128 + rl;
    const u32x4 v = *reinterpret_cast<const u32x4*>(ot + rl * 128 + ((c ^ (rl & 7)) << 4));
    if (row >= M) continue;
    uint16_t* dst = C + (size_t)row * N + colw + c * 8;
    if (colw + c * 8 + 7 < N && (N & 7) == 0) {
      store_stream16(dst, v);
    } else {
      const uint16_t* h = reinterpret_cast<const uint16_t*>(&v);
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (colw + c * 8 + e < N) dst[e] = h[e];
    }
  }
}


// ---------------------------------------------------------------------------
// Persistent 256x256 kernel: the K loop of fp8_gemm_big, one workgroup per CU
// walking the tile sequence t = slot, slot + nwg, ... so that a tile's
// prologue and epilogue overlap work instead of idling the CU:
//   * the last K block of a tile copies the next tile's first block (and its
//     scale chunk) into the free stage, so the next tile starts on data that
//     is already in LDS;
//   * C is written straight from the accumulators: per 16-row m-tile and pair
//     of 16-column n-tiles a lane holds 2 x 4 adjacent columns of one row;
//     one v_permlane16_swap per packed bf16 pair moves them so that every
//     lane holds 8 adjacent columns, stored as one 16-byte write (a store
//     instruction covers 16 rows x 64 contiguous bytes).  The stores are
//     bounds-checked buffer stores (rows past M fall outside the buffer's
//     M*N*2 bytes and are dropped by the hardware), so every wave issues
//     exactly 16 of them per tile; they stay in flight over the next tile's
//     first 28 MFMAs;
//   * one barrier per K block, placed after its MFMA 28 instead of before
//     its first MFMA: by then every wave has consumed its last operand
//     fragment of block k (so block k's stage is free for the copies of
//     block k + 2) and has waited for its copies of block k + 1, so the B
//     fragments, first A fragment and scales of block k + 1 are read while
//     MFMAs 29-31 of block k run.  (With the barrier at the block start,
//     every SIMD's two waves waited out the same ~500-cycle LDS round trip
//     with the MFMA pipe empty; a timeline of s_memtime stamps per wave
//     showed it on every block.)  The scales of the block are read as two
//     16-byte loads: the scale table is stored with a lane's eight rows
//     (16 i + r16) adjacent.
// Tile order: round r of the sequence is tiles r*nwg .. r*nwg + nwg - 1 of
// the grouped order (GROUP_M_BIG row-tiles per group); workgroup w runs on
// XCD w % 8 and takes position (w % 8) * (nwg / 8) + w / 8 of each round, so
// the tiles an XCD runs concurrently are consecutive in the grouped order
// and share A and B panels in that XCD's L2.
// Requires N % 256 == 0, M * N * 2 < 2^31, ceil(M / 256) * 256 * N * 2 < 2^32
// (the 32-bit store offsets of padded rows stay past C), 256 * K < 2^31,
// nwg % 8 == 0;
// bias: null or an fp32 vector of N (16-byte aligned).
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ unsigned cvt_pk_bf16(float lo, float hi) {
  // v_cvt_pk_bf16_f32: round to nearest even, as f32_to_bf16
  return __builtin_bit_cast(unsigned, __builtin_convertvector(f32x2_t{lo, hi}, bf16x2_t));
}

// x, with the compiler unable to see its value: per-lane addresses derived
// from it are recomputed where they are used instead of being hoisted out of
// the K loop and kept live (the K loop has no registers to spare)
__device__ __forceinline__ int opaque(int x) {
  asm volatile("" : "+v"(x));
  return x;
}

// HALF: the tail launch for a last round of at most half the CUs' worth of
// tiles -- tiles ntiles .. tiles_m * tiles_n - 1 of the grouped order, each
// as two 256 x 128 halves (half 2i + p: tile ntiles + i, columns 128 p ..;
// a grid of a multiple of 8 workgroups), so that twice as many CUs share the
// round.  A half is
// computed by waves 0-3 (one per SIMD, as 2 x 2 waves of 128 x 64); waves
// 4-7 only copy and take the barriers.  Otherwise workgroups walk tiles
// 0 .. ntiles - 1.
template <bool HAS_BIAS, bool HALF>
__global__ __launch_bounds__(512, 1) void fp8_gemm_persist(
    const uint8_t* __restrict__ A, const float* __restrict__ As, const uint8_t* __restrict__ B,
    const float* __restrict__ Bs, const float* __restrict__ bias, uint16_t* __restrict__ C, int M, int N, int K,
    int tiles_m, int tiles_n, int ntiles) {
  constexpr int A_BYTES = BIG * BK;
  constexpr int STAGE = 2 * A_BYTES;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[2 * STAGE];
  __shared__ __attribute__((aligned(1024))) float sas[2][SCKB][BIG];
  __shared__ __attribute__((aligned(64))) float sbs[2][SCKB][2];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = HALF ? (wave >> 1) & 1 : wave >> 2, wn = HALF ? wave & 1 : wave & 3;
  const bool active = !HALF || wave < 4;
  const int KT = K / BK;
  const int nch = (KT + SCKB - 1) / SCKB;  // scale chunks per tile
  const int nbs = N / 128;
  const int r16 = lane & 15, g = lane >> 4;
  const int nwg = gridDim.x;
  auto tile_of = [&](int t, int& m0, int& n0) {
    const int group = t / (GROUP_M_BIG * tiles_n);
    const int first_m = group * GROUP_M_BIG;
    const int gsize = min(tiles_m - first_m, GROUP_M_BIG);
    m0 = (first_m + (t % gsize)) * BIG;
    n0 = ((t % (GROUP_M_BIG * tiles_n)) / gsize) * BIG;
  };
  int t = HALF ? 0 : (blockIdx.x & 7) * (nwg >> 3) + (blockIdx.x >> 3);
  if (!HALF && t >= ntiles) return;  // whole workgroup, before any barrier
  int m0, n0;
  if constexpr (HALF) {
    // halves h = 2 i + p in XCD order (workgroup w runs on XCD w mod 8): the
    // two halves of a tile, and consecutive tiles, share one XCD's L2
    const int h = (blockIdx.x & 7) * (nwg >> 3) + (blockIdx.x >> 3);
    if (h >= 2 * (tiles_m * tiles_n - ntiles)) return;  // whole workgroup, before any barrier
    tile_of(ntiles + (h >> 1), m0, n0);
    n0 += (h & 1) * 128;
  } else {
    tile_of(t, m0, n0);
  }

  const unsigned lds0 = __builtin_amdgcn_readfirstlane(lds_addr(smem));
  const unsigned lsas = __builtin_amdgcn_readfirstlane(lds_addr(&sas[0][0][0]));
  const unsigned lsbs = __builtin_amdgcn_readfirstlane(lds_addr(&sbs[0][0][0]));
  // per-lane copy offsets of tile rows 8 (wave + 8u) + lane / 8 from the
  // tile's first row; rows past M are clamped to M - 1 (their results are
  // dropped).  The swizzled chunk does not depend on u.
  auto offs = [&](int lim, unsigned (&o)[4]) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int r = 8 * wave + 64 * u + (lane >> 3);
      const int c = (lane & 7) ^ ((((8 * wave + (lane >> 3)) >> 1) & 7) ^ ((lane >> 3) & 1) << 2);
      o[u] = (unsigned)min(r, lim) * (unsigned)K + c * 16;
    }
  };
  unsigned offA[4], offB[4];
  offs(M - 1 - m0, offA);
  offs(255, offB);
  const uint8_t* tileA = A + (size_t)m0 * K;
  const uint8_t* tileB = B + (size_t)n0 * K;
  // scale chunk for K blocks kb0 .. kb0 + SCKB - 1 of tile (mm0, nn0), as in
  // fp8_gemm_big but with the rows permuted: table position p = 64 u + lane
  // holds row (p / 128) * 128 + 16 (p % 8) + (p / 8) % 16, so lane l of a
  // wave finds its rows 16 i + l % 16 (i = 0..7) at 8 (l % 16) .. + 7
  auto issue_scales = [&](int mm0, int nn0, int kb0, int buf) {
    const int kb = min(kb0 + wave, KT - 1);
    const int ln = opaque(lane);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int p = 64 * u + ln;
      const int r = (p >> 7) * 128 + 16 * (p & 7) + ((p >> 3) & 15);
      const float* src = As + (size_t)min(mm0 + r, M - 1) * KT + kb;
      dma4(src, lsas + ((buf * SCKB + wave) * BIG + 64 * u) * 4);
    }
    if (wave == 0 && ln < 16) {
      const float* src = Bs + (size_t)min(nn0 / 128 + (ln & 1), nbs - 1) * KT + min(kb0 + (ln >> 1), KT - 1);
      dma4(src, lsbs + buf * SCKB * 2 * 4);
    }
  };
  const int fsw = ((r16 >> 1) & 7) ^ ((r16 & 1) << 2);
  const int la0 = (wm * 128 + r16) * BK + ((g ^ fsw) << 4);
  const int la1 = (wm * 128 + r16) * BK + (((g + 4) ^ fsw) << 4);
  const int lb0 = A_BYTES + (wn * 64 + r16) * BK + ((g ^ fsw) << 4);
  const int lb1 = A_BYTES + (wn * 64 + r16) * BK + (((g + 4) ^ fsw) << 4);
  const __amdgpu_buffer_rsrc_t crs = __builtin_amdgcn_make_buffer_rsrc(C, (short)0, M * N * 2, 0x00020000);

  v4f acc[8][4];
  issue_scales(m0, n0, 0, 0);
#pragma unroll
  for (int u = 0; u < 4; ++u) dma16s(tileA, offA[u], lds0 + (wave + 8 * u) * 1024);
#pragma unroll
  for (int u = 0; u < (HALF ? 2 : 4); ++u) dma16s(tileB, offB[u], lds0 + A_BYTES + (wave + 8 * u) * 1024);

  // block 0's operands
  wait_vm<0>();
  __syncthreads();
  v8i fb[4], fa[8];
  float4 s0, s1;
  float bsv;
  {
    const float4* sa4 = reinterpret_cast<const float4*>(&sas[0][0][wm * 128 + 8 * r16]);
    s0 = sa4[0];
    s1 = sa4[1];
    bsv = sbs[0][0][wn >> 1];
    fb[0] = frag(smem, lb0, lb1);
    fa[0] = frag(smem, la0, la1);
#pragma unroll
    for (int j = 1; j < 4; ++j) fb[j] = frag(smem + j * 2048, lb0, lb1);
  }

  int gk = 0;     // K blocks done by this workgroup (stage parity)
  int cbase = 0;  // scale chunks done (scale buffer parity)
  for (;;) {
    const int t_next = t + nwg;
    const bool has_next = !HALF && t_next < ntiles;
    int m0n = m0, n0n = n0;
    if (has_next) tile_of(t_next, m0n, n0n);
    for (int kt = 0; kt < KT; ++kt, ++gk) {
      const bool last = kt + 1 == KT;
      const uint8_t* dA = tileA;
      const uint8_t* dB = tileB;
      int kn = min(kt + 1, KT - 1);  // the last tile's last block re-copies itself
      if (!last && (kt + 1) % SCKB == 0) issue_scales(m0, n0, kt + 1, (cbase + (kt + 1) / SCKB) & 1);
      if (last && has_next) {  // the next tile's first block and scale chunk
        issue_scales(m0n, n0n, 0, (cbase + nch) & 1);
        offs(M - 1 - m0n, offA);
        dA = A + (size_t)m0n * K;
        dB = B + (size_t)n0n * K;
        kn = 0;
      }
      const unsigned nbase = lds0 + ((gk + 1) & 1) * STAGE;
      const uint8_t* st = smem + (gk & 1) * STAGE;
      const uint8_t* nst = smem + ((gk + 1) & 1) * STAGE;
      // scale location of block kt + 1 (the next tile's first block after the last)
      const int sbufn = last ? (cbase + nch) & 1 : (cbase + (kt + 1) / SCKB) & 1;
      const int kcn = last ? 0 : (kt + 1) % SCKB;
      float sc[8];
      float4 s0n, s1n;
      float bsvn;
      if (HALF && !active) {  // an idle wave's copies of block kt + 1, then the block's barrier
#pragma unroll
        for (int u = 0; u < 4; ++u) dma16s(dA + (size_t)kn * BK, offA[u], nbase + (wave + 8 * u) * 1024);
#pragma unroll
        for (int u = 0; u < 2; ++u) dma16s(dB + (size_t)kn * BK, offB[u], nbase + A_BYTES + (wave + 8 * u) * 1024);
        wait_vm<0>();
        __syncthreads();
        continue;
      }
      v4f tp[32];
#pragma unroll
      for (int k = 0; k < 34; ++k) {
        if (k < 32) tp[k] = mfma_fp8(fb[k & 3], fa[k >> 2]);
        if (k == 0) {
          sc[0] = s0.x * bsv; sc[1] = s0.y * bsv; sc[2] = s0.z * bsv; sc[3] = s0.w * bsv;
          sc[4] = s1.x * bsv; sc[5] = s1.y * bsv; sc[6] = s1.z * bsv; sc[7] = s1.w * bsv;
        }
        if ((k & 1) == 0 && k < 16) {
          const int u = (k >> 1) & 3;
          if (k < 8) dma16s(dA + (size_t)kn * BK, offA[u], nbase + (wave + 8 * u) * 1024);
          else if (!HALF || u < 2) dma16s(dB + (size_t)kn * BK, offB[u], nbase + A_BYTES + (wave + 8 * u) * 1024);
        }
        if ((k & 3) == 0 && (k >> 2) + 1 < 8) {
          const int i1 = (k >> 2) + 1;
          fa[i1] = frag(st + i1 * 2048, la0, la1);
        }
        if (k == 28) {
          // MFMA 28 consumed this wave's last fragment of block kt: once every
          // wave is here, block kt's stage is free and block kt + 1 (copied
          // during this block) has landed, so its first operands are read
          // while MFMAs 29-31 run
          wait_vm<0>();
          __syncthreads();
          const float4* sa4 = reinterpret_cast<const float4*>(&sas[sbufn][kcn][wm * 128 + 8 * r16]);
          s0n = sa4[0];
          s1n = sa4[1];
          bsvn = sbs[sbufn][kcn][wn >> 1];
          fa[0] = frag(nst, la0, la1);
          fb[0] = frag(nst, lb0, lb1);
        }
        if (k >= 29 && k < 32) fb[k - 28] = frag(nst + (k - 28) * 2048, lb0, lb1);
        if (k >= 2) {
          const int p = k - 2;
          if (kt == 0) {  // the tile's first K block starts the sums
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[p >> 2][p & 3][r] = tp[p][r] * sc[p >> 2];
          } else {
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[p >> 2][p & 3][r] = fmaf(tp[p][r], sc[p >> 2], acc[p >> 2][p & 3][r]);
          }
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      s0 = s0n;
      s1 = s1n;
      bsv = bsvn;
    }
    // ---- epilogue: bias, bf16 pairs, permlane16 swap, 16 stores per wave
    if (!active) break;  // (a half's idle waves; a half is its workgroup's only item)
    float bv[4][4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if constexpr (HAS_BIAS) {
        const float4 b4 = *reinterpret_cast<const float4*>(bias + n0 + wn * 64 + 16 * j + 4 * g);
        bv[j][0] = b4.x; bv[j][1] = b4.y; bv[j][2] = b4.z; bv[j][3] = b4.w;
      } else {
        bv[j][0] = bv[j][1] = bv[j][2] = bv[j][3] = 0.f;
      }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const unsigned row = (unsigned)(m0 + wm * 128 + 16 * i + r16);
#pragma unroll
      for (int jp = 0; jp < 2; ++jp) {
        const v4f& x = acc[i][2 * jp];
        const v4f& y = acc[i][2 * jp + 1];
        const float* bx = bv[2 * jp];
        const float* by = bv[2 * jp + 1];
        const unsigned a0 = cvt_pk_bf16(x[0] + bx[0], x[1] + bx[1]), a1 = cvt_pk_bf16(x[2] + bx[2], x[3] + bx[3]);
        const unsigned b0 = cvt_pk_bf16(y[0] + by[0], y[1] + by[1]), b1 = cvt_pk_bf16(y[2] + by[2], y[3] + by[3]);
        // lanes of row group g: (a of g, a of g+1) for even g, (b of g-1, b of g) for odd g
        const auto s0 = __builtin_amdgcn_permlane16_swap(a0, b0, false, false);
        const auto s1 = __builtin_amdgcn_permlane16_swap(a1, b1, false, false);
        const u32x4 d = {s0[0], s1[0], s0[1], s1[1]};
        const unsigned col = (unsigned)(n0 + wn * 64 + 32 * jp + (g & 1) * 16 + (g >> 1) * 8);
        __builtin_amdgcn_raw_buffer_store_b128(d, crs, (row * (unsigned)N + col) * 2u, 0, kStreamStore);
      }
    }
    if (!has_next) break;
    t = t_next;
    m0 = m0n;
    n0 = n0n;
    tileA = A + (size_t)m0 * K;
    tileB = B + (size_t)n0 * K;
    cbase += nch;
  }
  wait_vm<0>();  // the final re-copy lands before the workgroup's LDS is released
}

// out[m, n] = bf16(sum_s ws[s, m, n] + bias), four columns per thread
__global__ __launch_bounds__(256) void splitk_reduce(const float* __restrict__ ws, int splits,
                                                     const float* __restrict__ bias, int64_t bias_ld,
                                                     uint16_t* __restrict__ C, int64_t M, int64_t N) {
  const int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x;  // float4 index
  const int64_t nq = (N + 3) / 4;
  if (q >= M * nq) return;
  const int64_t m = q / nq, n = (q - m * nq) * 4;
  const int64_t MN = M * N;
  float v[4] = {0.f, 0.f, 0.f, 0.f};
  for (int s = 0; s < splits; ++s) {
#pragma unroll
    for (int r = 0; r < 4; ++r)
      if (n + r < N) v[r] += ws[s * MN + m * N + n + r];
  }
  if (bias != nullptr) {
#pragma unroll
    for (int r = 0; r < 4; ++r)
      if (n + r < N) v[r] += bias[(bias_ld ? m * bias_ld : 0) + n + r];
  }
#pragma unroll
  for (int r = 0; r < 4; ++r)
    if (n + r < N) C[m * N + n + r] = (uint16_t)f32_to_bf16(v[r]);
}

// The same sums, eight columns per thread (N % 8 == 0, C 16-byte aligned,
// M * N / 8 < 2^31): every split's two float4 loads are issued before any
// sum, up to 8 splits at a time, and the eight bf16 results go out as one
// 16-byte store.  Per element the additions run in split order from 0.f,
// then the bias, as in splitk_reduce, so the results are bit-identical.
__global__ __launch_bounds__(256) void splitk_reduce8(const float* __restrict__ ws, int splits,
                                                      const float* __restrict__ bias, int64_t bias_ld,
                                                      uint16_t* __restrict__ C, int M, int N) {
  const int nq = N / 8;
  const int q = blockIdx.x * 256 + threadIdx.x;
  if (q >= M * nq) return;
  const int m = q / nq, n = (q - m * nq) * 8;
  const int64_t MN = (int64_t)M * N;
  const float* src = ws + (int64_t)m * N + n;
  float v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int s0 = 0; s0 < splits; s0 += 8) {
    float4 lo[8], hi[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if (s0 + j < splits) {
        lo[j] = *reinterpret_cast<const float4*>(src + (s0 + j) * MN);
        hi[j] = *reinterpret_cast<const float4*>(src + (s0 + j) * MN + 4);
      }
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if (s0 + j < splits) {
        v[0] += lo[j].x; v[1] += lo[j].y; v[2] += lo[j].z; v[3] += lo[j].w;
        v[4] += hi[j].x; v[5] += hi[j].y; v[6] += hi[j].z; v[7] += hi[j].w;
      }
    }
  }
  if (bias != nullptr) {
    const float* b = bias + (bias_ld ? (int64_t)m * bias_ld : 0) + n;
#pragma unroll
    for (int r = 0; r < 8; ++r) v[r] += b[r];
  }
  uint4 o;
  o.x = pack_bf16x2(v[0], v[1]);
  o.y = pack_bf16x2(v[2], v[3]);
  o.z = pack_bf16x2(v[4], v[5]);
  o.w = pack_bf16x2(v[6], v[7]);
  *reinterpret_cast<uint4*>(C + (int64_t)m * N + n) = o;
}

}  // namespace
}  // namespace lfs

using namespace lfs;

extern "C" int64_t lfs_fp8_gemm_workspace_bytes(int64_t M, int64_t N, int64_t K, int32_t splits) {
  if (M <= 0 || N <= 0 || K <= 0 || splits <= 1) return 0;
  const int64_t KT = K / 128;
  const int64_t kps = (KT + splits - 1) / splits;
  const int64_t used = (KT + kps - 1) / kps;
  return used > 1 ? used * M * N * 4 : 0;
}

namespace {
// compute units of the current device (the persistent kernel's grid)
int cu_count() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

// 256x256 tiles (one workgroup per CU) when they fill the chip with at most
// 15% of the last round idle, K is long enough to amortise the 64 KB
// prologue copy, and the per-lane 32-bit copy offsets fit (256 rows of K bytes)
bool use_big_tiles(int64_t M, int64_t N, int64_t K) {
  const int64_t t = ((M + BIG - 1) / BIG) * ((N + BIG - 1) / BIG);
  const int64_t cus = cu_count();
  const int64_t rounds = (t + cus - 1) / cus;
  return t >= cus && t * 100 >= rounds * cus * 85 && K >= 512 && 256 * K < (1ll << 31);
}

// The persistent 256x256 kernel: N a multiple of 256 (its stores write 16-byte
// row segments and rely on the buffer range for rows only), a vector bias or
// none, byte offsets of C and of a 256-row panel within 32 bits -- including
// the padded rows of the last row of tiles, whose 32-bit store offsets must
// not wrap back into C -- and at least half a round of 256x256 tiles (fewer
// leave most CUs idle; the 128x128 kernel fills them).
bool use_persistent(int64_t M, int64_t N, int64_t K, const float* bias, int64_t bias_ld) {
  const int64_t tm = (M + BIG - 1) / BIG;
  const int64_t t = tm * (N / BIG);
  return N % BIG == 0 && bias_ld == 0 && ((uintptr_t)bias & 15u) == 0 && M * N * 2 < (1ll << 31) &&
         tm * BIG * N * 2 < (1ll << 32) && 256 * K < (1ll << 31) && K >= 256 && 2 * t >= cu_count();
}

// One-shot configurations for 16 < M <= 128 (fp8_gemm_flat<MT, NC, KBM, WR,
// WK>), picked from the shape alone.  Measured on MI355X, calls back to back
// in a graph over rotating weight copies, against the 128x128 tile kernel:
//   FLAT_R32_C16  (2, 1, 8, 2, 4): K <= 1024, ceil(M/32) * ceil(N/16) <= 512
//                  workgroups -- M = 128, K = 768: N = 1280 4.3 us (6.8),
//                  N = 768 3.9 us (6.6) (4.4 / 4.1 us with two K groups);
//   FLAT_R32_C32  (2, 2, 8, 2, 2): K <= 1024 with <= 512 such workgroups --
//                  M = 128, K = 1024, N = 4096 6.8 us (9.6);
//   FLAT_S32_C32  (2, 2, 8, 2, 4): the split partials of at most 8 K blocks
//                  each -- M = 128, K = 4608, N = 768 in 5 splits 5.7 us
//                  (6.4 us with two K groups, 6 tile splits 11.5 us);
//   FLAT_R128_C48 (8, 3, 6, 8, 1): K <= 768, ceil(N/48) <= 256 workgroups --
//                  M = 128, K = 768, N = 9216 8.1 us (r128c64 9.5, r64c96
//                  8.9, r64c64 11.7; tile kernel 11.0);
//   FLAT_R128_C64 (8, 4, 6, 4, 2): K <= 768, ceil(N/64) <= 256 workgroups;
//   FLAT_R16_C16  (1, 1, 32, 1, 8): K <= 4096, ceil(M/16) * ceil(N/16) <= 512
//                  -- M = 128, K = 4096, N = 1024 10.2 us (15.5).
// A workgroup streams its operands at roughly 30 GB/s (a per-CU limit seen
// in every kernel here), so the smaller the workgroup's operand footprint
// ((rows + columns) x K bytes) at a grid of one or two rounds, the shorter
// the call; wider N (lm_head, N = 32000: 18 us against 13 us) stays on the
// tile kernel.
enum FlatVariant { FLAT_NONE = -1, FLAT_R32_C16, FLAT_R32_C32, FLAT_S32_C32, FLAT_R128_C48, FLAT_R128_C64, FLAT_R16_C16 };

FlatVariant flat_variant(int64_t M, int64_t N, int64_t K, int64_t kps, bool split) {
  if (M <= 16 || M > 128) return FLAT_NONE;
  const int64_t kb = K / 128;
  const int64_t r32 = (M + 31) / 32, c16 = (N + 15) / 16, c32 = (N + 31) / 32;
  if (split) return kps <= 8 && r32 * c32 * ((kb + kps - 1) / kps) <= 1024 ? FLAT_S32_C32 : FLAT_NONE;
  if (kb <= 8 && r32 * c16 <= 512) return FLAT_R32_C16;
  if (kb <= 8 && r32 * c32 <= 512) return FLAT_R32_C32;
  if (kb <= 6 && (N + 47) / 48 <= 256) return FLAT_R128_C48;
  if (kb <= 6 && (N + 63) / 64 <= 256) return FLAT_R128_C64;
  if (kb <= 32 && ((M + 15) / 16) * c16 <= 512) return FLAT_R16_C16;
  return FLAT_NONE;
}

// aq: a is bf16 with row stride lda, quantised inside the kernel (one split)
void launch_flat(FlatVariant v, const void* a, const float* a_s, const void* b, const float* b_s, const float* bias,
                 int64_t bias_ld, void* c, float* ws, int64_t M, int64_t N, int64_t K, int kps, hipStream_t st,
                 bool aq = false, int64_t lda = 0) {
  const int nsplit = (int)((K / 128 + kps - 1) / kps);
#define LFS_FLAT(MT, NC, KBM, WR, WK)                                                                               \
  if (aq)                                                                                                            \
    hipLaunchKernelGGL((fp8_gemm_flat<MT, NC, KBM, WR, WK, true>),                                                   \
                       dim3((unsigned)((N + 16 * NC - 1) / (16 * NC)), (unsigned)nsplit,                             \
                            (unsigned)((M + 16 * MT - 1) / (16 * MT))),                                              \
                       dim3(64 * WR * WK), 0, st, (const uint8_t*)a, a_s, (const uint8_t*)b, b_s, bias, bias_ld,     \
                       (uint16_t*)c, ws, (int)M, (int)N, (int)K, kps, lda);                                          \
  else                                                                                                               \
    hipLaunchKernelGGL((fp8_gemm_flat<MT, NC, KBM, WR, WK>),                                                         \
                       dim3((unsigned)((N + 16 * NC - 1) / (16 * NC)), (unsigned)nsplit,                             \
                            (unsigned)((M + 16 * MT - 1) / (16 * MT))),                                              \
                       dim3(64 * WR * WK), 0, st, (const uint8_t*)a, a_s, (const uint8_t*)b, b_s, bias, bias_ld,     \
                       (uint16_t*)c, ws, (int)M, (int)N, (int)K, kps)
  switch (v) {
    case FLAT_R32_C16: LFS_FLAT(2, 1, 8, 2, 4); break;
    case FLAT_R32_C32: LFS_FLAT(2, 2, 8, 2, 2); break;
    case FLAT_S32_C32: LFS_FLAT(2, 2, 8, 2, 4); break;
    case FLAT_R128_C48: LFS_FLAT(8, 3, 6, 8, 1); break;
    case FLAT_R128_C64: LFS_FLAT(8, 4, 6, 4, 2); break;
    case FLAT_R16_C16: LFS_FLAT(1, 1, 32, 1, 8); break;
    default: break;
  }
#undef LFS_FLAT
}

// reduce == false: split-K partials only (ws[s][M][N] fp32, no bias, C not
// written); at least two K splits must result.
int fp8_gemm_impl(const void* a, const float* a_s, const void* b, const float* b_s, const float* bias,
                  int64_t bias_ld, void* c, int64_t M, int64_t N, int64_t K, int32_t splits,
                  void* workspace, int64_t workspace_bytes, void* stream, bool reduce = true) {
  LFS_REQUIRE(M >= 0 && N >= 0 && K >= 0, "fp8_gemm: negative shape");
  LFS_REQUIRE(K % 128 == 0, "fp8_gemm: K=%lld must be a multiple of 128", (long long)K);
  LFS_REQUIRE(M < (1ll << 31) && N < (1ll << 31) && K < (1ll << 31) && M * K < (1ll << 40),
              "fp8_gemm: shape too large");
  LFS_REQUIRE(splits >= 1, "fp8_gemm: splits must be >= 1");
  if (M == 0 || N == 0) return 0;
  LFS_REQUIRE(a && a_s && b && b_s && (c || !reduce), "fp8_gemm: null pointer");
  LFS_REQUIRE(K > 0, "fp8_gemm: K must be positive");
  LFS_REQUIRE((((uintptr_t)a | (uintptr_t)b) & 15u) == 0, "fp8_gemm: a and b must be 16-byte aligned");
  LFS_REQUIRE(((uintptr_t)c & 15u) == 0, "fp8_gemm: c must be 16-byte aligned");
  LFS_REQUIRE(reduce || bias == nullptr, "fp8_gemm_splitk_partials: the bias is added by the consumer");
  LFS_REQUIRE(bias_ld == 0 || (bias != nullptr && bias_ld >= N), "fp8_gemm: bias_ld must be 0 or >= N");
  const int64_t tiles_n = (N + BN - 1) / BN;
  const int64_t tiles_m128 = (M + 127) / 128;
  LFS_REQUIRE(tiles_m128 * tiles_n < (1ll << 31), "fp8_gemm: too many tiles");
  const int KT = (int)(K / 128);
  int kps = (KT + splits - 1) / splits;
  const int used = (KT + kps - 1) / kps;
  float* ws = nullptr;
  if (used > 1) {
    const int64_t need = (int64_t)used * M * N * 4;
    LFS_REQUIRE(workspace != nullptr && workspace_bytes >= need,
                "fp8_gemm: split-K needs a workspace of %lld bytes", (long long)need);
    LFS_REQUIRE(((uintptr_t)workspace & 15u) == 0, "fp8_gemm: workspace must be 16-byte aligned");
    ws = (float*)workspace;
  } else {
    kps = KT;
  }
  LFS_REQUIRE(reduce || ws != nullptr, "fp8_gemm_splitk_partials: K=%lld in %d splits gives one split",
              (long long)K, splits);
  hipStream_t st = (hipStream_t)stream;
  const FlatVariant fv = flat_variant(M, N, K, kps, ws != nullptr);
  if (fv != FLAT_NONE) {
    launch_flat(fv, a, a_s, b, b_s, ws != nullptr ? nullptr : bias, bias_ld, c, ws, M, N, K, kps, st);
    int rc = check_launch("fp8_gemm(flat)");
    if (rc != 0 || ws == nullptr || !reduce) return rc;
    if (N % 8 == 0 && ((uintptr_t)c & 15u) == 0 && M * (N / 8) < (1ll << 31) - 256) {
      const int64_t octs = M * (N / 8);
      hipLaunchKernelGGL(splitk_reduce8, dim3((unsigned)((octs + 255) / 256)), dim3(256), 0, st, ws, used, bias,
                         bias_ld, (uint16_t*)c, (int)M, (int)N);
      return check_launch("fp8_gemm split-K reduce");
    }
    const int64_t quads = M * ((N + 3) / 4);
    hipLaunchKernelGGL(splitk_reduce, dim3((unsigned)((quads + 255) / 256)), dim3(256), 0, st, ws, used, bias,
                       bias_ld, (uint16_t*)c, M, N);
    return check_launch("fp8_gemm split-K reduce");
  }
  if (ws == nullptr && use_persistent(M, N, K, bias, bias_ld)) {
    const int64_t bm = (M + BIG - 1) / BIG, bn = N / BIG;
    const int64_t ntiles = bm * bn;
    const int nwg = (int)std::min<int64_t>(std::max(8, cu_count() / 8 * 8), (ntiles + 7) / 8 * 8);
    // a last round of at most half the workgroups' worth of tiles runs as a
    // second launch of 256 x 128 halves
    const int64_t rem = ntiles % nwg;
    const int64_t nmain = rem > 0 && 2 * rem <= nwg && ntiles > nwg ? ntiles - rem : ntiles;
    if (bias != nullptr)
      hipLaunchKernelGGL((fp8_gemm_persist<true, false>), dim3((unsigned)nwg), dim3(512), 0, st, (const uint8_t*)a,
                         a_s, (const uint8_t*)b, b_s, bias, (uint16_t*)c, (int)M, (int)N, (int)K, (int)bm, (int)bn,
                         (int)nmain);
    else
      hipLaunchKernelGGL((fp8_gemm_persist<false, false>), dim3((unsigned)nwg), dim3(512), 0, st, (const uint8_t*)a,
                         a_s, (const uint8_t*)b, b_s, bias, (uint16_t*)c, (int)M, (int)N, (int)K, (int)bm, (int)bn,
                         (int)nmain);
    if (nmain < ntiles) {
      const unsigned nh = (unsigned)((2 * (ntiles - nmain) + 7) / 8 * 8);
      if (bias != nullptr)
        hipLaunchKernelGGL((fp8_gemm_persist<true, true>), dim3(nh), dim3(512), 0, st, (const uint8_t*)a, a_s,
                           (const uint8_t*)b, b_s, bias, (uint16_t*)c, (int)M, (int)N, (int)K, (int)bm, (int)bn,
                           (int)nmain);
      else
        hipLaunchKernelGGL((fp8_gemm_persist<false, true>), dim3(nh), dim3(512), 0, st, (const uint8_t*)a, a_s,
                           (const uint8_t*)b, b_s, bias, (uint16_t*)c, (int)M, (int)N, (int)K, (int)bm, (int)bn,
                           (int)nmain);
    }
    return check_launch("fp8_gemm");
  }
  if (ws == nullptr && use_big_tiles(M, N, K)) {
    const int64_t bm = (M + BIG - 1) / BIG, bn = (N + BIG - 1) / BIG;
    hipLaunchKernelGGL(fp8_gemm_big, dim3((unsigned)(bm * bn)), dim3(512), 0, st, (const uint8_t*)a, a_s,
                       (const uint8_t*)b, b_s, bias, bias_ld, (uint16_t*)c, (int)M, (int)N, (int)K, (int)bm,
                       (int)bn);
    return check_launch("fp8_gemm");
  }
  // 128x128 tiles, two workgroups per CU.  (256x128 tiles with one
  // 8-wave workgroup per CU measured 10-15% slower on every benchmark shape.)
  // A grid of at most one workgroup per CU gets two K slices per workgroup
  // instead (8 waves, two per SIMD, as two 4-wave workgroups would give):
  // M = 4096, K = 4096, N = 1024 (256 tiles) 30.1 -> 26.1 us, the cfg5
  // decode step's w13 and down projections 0.3-0.5 us each.
  const dim3 tgrid((unsigned)(tiles_m128 * tiles_n), (unsigned)(used > 1 ? used : 1));
  if ((int64_t)tgrid.x * tgrid.y <= cu_count())
    hipLaunchKernelGGL((fp8_gemm_tile<128, 2, 16, false, 2>), tgrid, dim3(512), 0, st, (const uint8_t*)a, a_s,
                       (const uint8_t*)b, b_s, bias, bias_ld, (uint16_t*)c, (int)M, (int)N, (int)K, (int)tiles_m128,
                       (int)tiles_n, ws, kps, (int64_t)K, (int)KT, Grouped{});
  else
    hipLaunchKernelGGL((fp8_gemm_tile<128, 2, 16>), tgrid, dim3(256), 0, st, (const uint8_t*)a, a_s,
                       (const uint8_t*)b, b_s, bias, bias_ld, (uint16_t*)c, (int)M, (int)N, (int)K, (int)tiles_m128,
                       (int)tiles_n, ws, kps, (int64_t)K, (int)KT, Grouped{});
  int rc = check_launch("fp8_gemm");
  if (rc != 0 || ws == nullptr || !reduce) return rc;
  if (N % 8 == 0 && ((uintptr_t)c & 15u) == 0 && M * (N / 8) < (1ll << 31) - 256) {
    const int64_t octs = M * (N / 8);
    hipLaunchKernelGGL(splitk_reduce8, dim3((unsigned)((octs + 255) / 256)), dim3(256), 0, st, ws, used, bias,
                       bias_ld, (uint16_t*)c, (int)M, (int)N);
    return check_launch("fp8_gemm split-K reduce");
  }
  const int64_t quads = M * ((N + 3) / 4);
  hipLaunchKernelGGL(splitk_reduce, dim3((unsigned)((quads + 255) / 256)), dim3(256), 0, st, ws, used, bias,
                     bias_ld, (uint16_t*)c, M, N);
  return check_launch("fp8_gemm split-K reduce");
}
}  // namespace

extern "C" int lfs_fp8_gemm(const void* a, const float* a_s, const void* b, const float* b_s,
                            const float* bias, int64_t bias_ld, void* c, int64_t M, int64_t N,
                            int64_t K, void* stream) {
  return fp8_gemm_impl(a, a_s, b, b_s, bias, bias_ld, c, M, N, K, 1, nullptr, 0, stream);
}

extern "C" int lfs_fp8_gemm_act_supported(int64_t M, int64_t N, int64_t K) {
  if (M <= 0 || N <= 0 || K <= 0 || K % 128 != 0 || M >= (1ll << 31) || N >= (1ll << 31) || K >= (1ll << 31))
    return 0;
  return flat_variant(M, N, K, K / 128, false) != FLAT_NONE ? 1 : 0;
}

extern "C" int lfs_fp8_gemm_act(const void* a, int64_t lda, const void* b, const float* b_s, const float* bias,
                                int64_t bias_ld, void* c, int64_t M, int64_t N, int64_t K, void* stream) {
  LFS_REQUIRE(M >= 0 && N >= 0 && K >= 0, "fp8_gemm_act: negative shape");
  LFS_REQUIRE(K % 128 == 0 && K > 0, "fp8_gemm_act: K=%lld must be a positive multiple of 128", (long long)K);
  if (M == 0 || N == 0) return 0;
  LFS_REQUIRE(lfs_fp8_gemm_act_supported(M, N, K),
              "fp8_gemm_act: no one-shot tiling for M=%lld N=%lld K=%lld (16 < M <= 128, small K and N)",
              (long long)M, (long long)N, (long long)K);
  LFS_REQUIRE(a && b && b_s && c, "fp8_gemm_act: null pointer");
  LFS_REQUIRE(lda >= K && lda % 8 == 0, "fp8_gemm_act: the row stride lda=%lld must be >= K and a multiple of 8",
              (long long)lda);
  LFS_REQUIRE((((uintptr_t)a | (uintptr_t)b | (uintptr_t)c) & 15u) == 0,
              "fp8_gemm_act: a, b and c must be 16-byte aligned");
  LFS_REQUIRE(bias_ld == 0 || (bias != nullptr && bias_ld >= N), "fp8_gemm_act: bias_ld must be 0 or >= N");
  const FlatVariant fv = flat_variant(M, N, K, K / 128, false);
  launch_flat(fv, a, nullptr, b, b_s, bias, bias_ld, c, nullptr, M, N, K, (int)(K / 128), (hipStream_t)stream, true,
              lda);
  return check_launch("fp8_gemm_act");
}

extern "C" int lfs_fp8_gemm_splitk(const void* a, const float* a_s, const void* b, const float* b_s,
                                   const float* bias, int64_t bias_ld, void* c, int64_t M, int64_t N,
                                   int64_t K, int32_t splits, void* workspace, int64_t workspace_bytes,
                                   void* stream) {
  return fp8_gemm_impl(a, a_s, b, b_s, bias, bias_ld, c, M, N, K, splits, workspace, workspace_bytes,
                       stream);
}

extern "C" int lfs_fp8_gemm_splitk_partials(const void* a, const float* a_s, const void* b, const float* b_s,
                                            int64_t M, int64_t N, int64_t K, int32_t splits, void* workspace,
                                            int64_t workspace_bytes, void* stream) {
  return fp8_gemm_impl(a, a_s, b, b_s, nullptr, 0, nullptr, M, N, K, splits, workspace, workspace_bytes, stream,
                       false);
}

extern "C" int lfs_fp8_grouped_gemm(const void* a, const float* a_s, int64_t a_rows, const int32_t* row_index,
                                    const int32_t* tile_expert, int64_t num_tiles, const void* b, const float* b_s,
                                    int64_t b_expert_stride, int64_t ldb, int64_t bs_expert_stride, int64_t ldbs,
                                    const float* bias, int64_t bias_expert_stride, void* c, float* c_f32, int64_t N,
                                    int64_t K, void* stream) {
  LFS_REQUIRE(a_rows >= 0 && num_tiles >= 0 && N >= 0 && K >= 0, "fp8_grouped_gemm: negative shape");
  LFS_REQUIRE(K % 128 == 0 && K > 0, "fp8_grouped_gemm: K=%lld must be a positive multiple of 128", (long long)K);
  LFS_REQUIRE(ldb >= K && ldb % 16 == 0 && b_expert_stride >= 0 && b_expert_stride % 16 == 0,
              "fp8_grouped_gemm: weight rows must be 16-byte aligned, ldb >= K");
  LFS_REQUIRE(ldbs >= K / 128 && bs_expert_stride >= 0 && bias_expert_stride >= 0,
              "fp8_grouped_gemm: bad scale / bias strides");
  LFS_REQUIRE((c == nullptr) != (c_f32 == nullptr), "fp8_grouped_gemm: exactly one of c (bf16) and c_f32");
  LFS_REQUIRE(c_f32 == nullptr || bias == nullptr, "fp8_grouped_gemm: the fp32 output takes no bias");
  const int64_t M = num_tiles * 128;
  LFS_REQUIRE(M < (1ll << 31) && N < (1ll << 31) && K < (1ll << 31) && a_rows < (1ll << 31) && ldb < (1ll << 31),
              "fp8_grouped_gemm: shape too large");
  if (num_tiles == 0 || N == 0) return 0;
  LFS_REQUIRE(a_rows > 0 && a && a_s && b && b_s && tile_expert, "fp8_grouped_gemm: null pointer");
  LFS_REQUIRE(row_index != nullptr || a_rows >= M, "fp8_grouped_gemm: without row_index A needs num_tiles*128 rows");
  LFS_REQUIRE((((uintptr_t)a | (uintptr_t)b) & 15u) == 0, "fp8_grouped_gemm: a and b must be 16-byte aligned");
  LFS_REQUIRE((((uintptr_t)c | (uintptr_t)c_f32) & 15u) == 0, "fp8_grouped_gemm: output must be 16-byte aligned");
  const int64_t tiles_n = (N + BN - 1) / BN;
  LFS_REQUIRE(num_tiles * tiles_n < (1ll << 31), "fp8_grouped_gemm: too many tiles");
  const Grouped grp{tile_expert, row_index, b_expert_stride, bs_expert_stride, bias_expert_stride, (int)a_rows};
  // the dense kernel's rule: two K slices per workgroup for at most one
  // workgroup per CU (so a tile's sums match fp8_gemm's on a grid as small)
  const dim3 grid((unsigned)(num_tiles * tiles_n));
  if ((int64_t)grid.x <= cu_count())
    hipLaunchKernelGGL((fp8_gemm_tile<128, 2, 16, true, 2>), grid, dim3(512), 0, (hipStream_t)stream,
                       (const uint8_t*)a, a_s, (const uint8_t*)b, b_s, bias, (int64_t)0, (uint16_t*)c, (int)M, (int)N,
                       (int)K, (int)num_tiles, (int)tiles_n, c_f32, (int)(K / 128), ldb, (int)ldbs, grp);
  else
    hipLaunchKernelGGL((fp8_gemm_tile<128, 2, 16, true>), grid, dim3(256), 0, (hipStream_t)stream,
                       (const uint8_t*)a, a_s, (const uint8_t*)b, b_s, bias, (int64_t)0, (uint16_t*)c, (int)M, (int)N,
                       (int)K, (int)num_tiles, (int)tiles_n, c_f32, (int)(K / 128), ldb, (int)ldbs, grp);
  return check_launch("fp8_grouped_gemm");
}

extern "C" int lfs_fp8_gemm_skinny(const void* a, const float* a_s, const void* b, const float* b_s,
                                   const float* bias, int64_t bias_ld, void* c, int64_t M, int64_t N, int64_t K,
                                   void* stream) {
  LFS_REQUIRE(M >= 0 && N >= 0 && K >= 0, "fp8_gemm_skinny: negative shape");
  LFS_REQUIRE(M <= 128, "fp8_gemm_skinny: M=%lld must be <= 128", (long long)M);
  LFS_REQUIRE(K % 128 == 0, "fp8_gemm_skinny: K=%lld must be a multiple of 128", (long long)K);
  LFS_REQUIRE(N < (1ll << 31) && K < (1ll << 24), "fp8_gemm_skinny: shape too large");
  if (M == 0 || N == 0) return 0;
  LFS_REQUIRE(K > 0 && a && a_s && b && b_s && c, "fp8_gemm_skinny: null pointer");
  LFS_REQUIRE((((uintptr_t)a | (uintptr_t)b) & 15u) == 0, "fp8_gemm_skinny: a and b must be 16-byte aligned");
  LFS_REQUIRE(bias_ld == 0 || (bias != nullptr && bias_ld >= N), "fp8_gemm_skinny: bias_ld must be 0 or >= N");
  hipStream_t st = (hipStream_t)stream;
  const int mt = (int)((M + 15) / 16);
  const int KT = (int)(K / 128);
  // N <= 4096 (<= 128 groups of 32 columns): groups of 16 columns, twice
  // the workgroups, each re-reading all M activation rows.  Measured back to
  // back: M = 16, K 1024 / N 4096 4.8 -> 3.9 us, K 4096 / N 1024 9.5 -> 7.3
  // us; M = 128, K 768 / N 1280 7.9 -> 6.7 us, K 1024 / N 4096 10.8 -> 9.6
  // us; but M = 16, N = 5632 (176 groups of 32) 6.6 -> 7.4 us
  const bool narrow = N <= 4096;
  const dim3 grid((unsigned)((N + (narrow ? 15 : 31)) / (narrow ? 16 : 32)));
#define LFS_SK(MTW, WGM, KW, NT)                                                                                \
  hipLaunchKernelGGL((fp8_gemm_skinny<MTW, WGM, KW, NT>), grid, dim3(64 * KW * WGM), 0, st, (const uint8_t*)a,   \
                     a_s, (const uint8_t*)b, b_s, bias, bias_ld, (uint16_t*)c, (int)M, (int)N, (int)K)
  // one 16-row tile: the K blocks over 16 / 8 / 4 waves (>= 1.5 blocks per wave)
  if (narrow && mt <= 1 && KT >= 24) LFS_SK(1, 1, 16, 1);
  else if (narrow && mt <= 1 && KT >= 12) LFS_SK(1, 1, 8, 1);
  else if (narrow && mt <= 1) LFS_SK(1, 1, 4, 1);
  else if (mt <= 1 && KT >= 24) LFS_SK(1, 1, 16, 2);
  else if (mt <= 1 && KT >= 12) LFS_SK(1, 1, 8, 2);
  else if (mt <= 1) LFS_SK(1, 1, 4, 2);
  else if (narrow && mt <= 2) LFS_SK(2, 1, 4, 1);
  else if (narrow && mt <= 4) LFS_SK(4, 1, 4, 1);
  else if (narrow) LFS_SK(4, 2, 4, 1);
  else if (mt <= 2) LFS_SK(2, 1, 4, 2);
  else if (mt <= 4) LFS_SK(4, 1, 4, 2);
  else LFS_SK(4, 2, 4, 2);
#undef LFS_SK
  return check_launch("fp8_gemm_skinny");
}

