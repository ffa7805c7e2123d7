// MoE dispatch and combine for gfx950: the pieces around the grouped FP8
// expert GEMMs (the GEMM itself is fp8_gemm_tile's grouped mode).
//
//   moe_align        (token, pick) entries -> rows grouped by expert, each
//                    expert's segment padded to 128-row tiles, plus the
//                    tile -> expert map and each entry's row; three
//                    launches over 1024-entry chunks, stable (entries of an
//                    expert keep their flat order), no host synchronisation (model/architecture/moe.py:288-341
//                    does argsort + bincount + .tolist()).
//   moe_combine      y[t] = bf16( sum_j out[row(t, j)] + sum_j w_tj * b2[e_tj] )
//                    over the token's picks and shared experts, fp32, in pick
//                    order (the weights are already inside out: they scale
//                    the down GEMM's activation scales); out bf16 or fp32.
//   segment_reduce_weighted / scatter_add_weighted
//                    y[t] = sum_{i : idx[i] = t} w_i * x_i in fp32, rounded to
//                    x's dtype: the Triton kernels of
//                    model/architecture/moe_kernels.py:6-171.  The sorted form
//                    finds each token's segment by binary search (the
//                    reference's searchsorted); the unsorted form counts,
//                    scans and places the entries per token, then sums each
//                    segment in increasing entry order.
#include <algorithm>

#include "common.h"

namespace lfs {
namespace {

constexpr int kAlignThreads = 1024;
constexpr int kAlignMaxExperts = 64;
constexpr int kTile = 128;  // rows per grouped-GEMM tile

// Entry i = t * kk + j of the (token, pick) list, kk = top_k + S: picks
// j < top_k are routed expert topk_idx[t, j] with weight topk_w[t, j]; the
// rest are the shared experts E + (j - top_k) with weight 1.
__device__ __forceinline__ void entry(const int64_t* idx, const float* w, int64_t i, int kk, int top_k, int E,
                                      int& t, int& e, float& wt) {
  t = (int)(i / kk);
  const int j = (int)(i - (int64_t)t * kk);
  if (j < top_k) {
    const int64_t v = idx[(int64_t)t * top_k + j];
    e = (v >= 0 && v < E) ? (int)v : -1;  // out-of-range picks are dropped
    wt = w[(int64_t)t * top_k + j];
  } else {
    e = E + (j - top_k);
    wt = 1.0f;
  }
}

// moe_align in three launches over chunks of 1024 entries (workspace:
// hist[chunks][E'] counts then bases, cnt[E'], off[E' + 1]):
//   rank     per chunk: each entry's rank among the chunk's entries of its
//            expert (wave ballots + a prefix over the waves) -> entry_row
//            (temporarily), the chunk's count per expert -> hist
//   offsets  one workgroup: per expert an exclusive scan of hist over the
//            chunks, the padded segment offsets, tile_expert, padding rows
//   place    per chunk: row = off[e] + hist[chunk][e] + rank -> row_token,
//            row_weight, entry_row
// The order is stable: entry i precedes entry i' > i of the same expert.
__global__ __launch_bounds__(kAlignThreads) void moe_align_rank_kernel(
    const int64_t* __restrict__ topk_idx, const float* __restrict__ topk_w, int T, int top_k, int E, int S,
    int32_t* __restrict__ entry_row, int32_t* __restrict__ hist) {
  constexpr int NW = kAlignThreads / 64;
  __shared__ int wcnt[NW][kAlignMaxExperts];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int kk = top_k + S, EE = E + S;
  const int64_t n = (int64_t)T * kk;
  for (int x = tid; x < NW * kAlignMaxExperts; x += kAlignThreads) (&wcnt[0][0])[x] = 0;
  __syncthreads();
  const int64_t i = (int64_t)blockIdx.x * kAlignThreads + tid;
  int t = 0, e = -1;
  float wt = 0.f;
  if (i < n) entry(topk_idx, topk_w, i, kk, top_k, E, t, e, wt);
  // rank inside the wave: one ballot per distinct expert present
  int rank = 0;
  uint64_t todo = __ballot(e >= 0);
  while (todo != 0) {
    const int leader = __builtin_ctzll(todo);
    const int el = __shfl(e, leader, 64);
    const uint64_t same = __ballot(e == el);
    if (e == el) rank = __builtin_popcountll(same & ((1ull << lane) - 1ull));
    if (lane == leader) wcnt[wave][el] = __builtin_popcountll(same);
    todo &= ~same;
  }
  __syncthreads();
  if (tid < EE) {  // exclusive prefix over the waves; the chunk's total
    int acc = 0;
    for (int w = 0; w < NW; ++w) {
      const int c = wcnt[w][tid];
      wcnt[w][tid] = acc;
      acc += c;
    }
    hist[(int64_t)blockIdx.x * EE + tid] = acc;
  }
  __syncthreads();
  if (i < n) entry_row[i] = e >= 0 ? wcnt[wave][e] + rank : -1;
}

__global__ __launch_bounds__(kAlignThreads) void moe_align_offsets_kernel(
    int chunks, int E, int S, int32_t* __restrict__ hist, int32_t* __restrict__ cnt_out,
    int32_t* __restrict__ off_out, int32_t* __restrict__ row_token, float* __restrict__ row_weight,
    int32_t* __restrict__ tile_expert, int num_tiles) {
  __shared__ int cnt[kAlignMaxExperts];
  __shared__ int off[kAlignMaxExperts + 1];
  const int tid = threadIdx.x, EE = E + S;
  if (tid < EE) {
    int run = 0;
    for (int c = 0; c < chunks; ++c) {
      const int v = hist[(int64_t)c * EE + tid];
      hist[(int64_t)c * EE + tid] = run;
      run += v;
    }
    cnt[tid] = run;
    cnt_out[tid] = run;
  }
  __syncthreads();
  if (tid == 0) {
    int o = 0;
    for (int e = 0; e < EE; ++e) {
      off[e] = o;
      o += (cnt[e] + kTile - 1) / kTile * kTile;
    }
    off[EE] = o;
  }
  __syncthreads();
  if (tid <= EE) off_out[tid] = off[tid];
  for (int tile = tid; tile < num_tiles; tile += kAlignThreads) {
    const int r = tile * kTile;
    int ex = -1;
    if (r < off[EE]) {  // off[lo] <= r < off[hi]
      int lo = 0, hi = EE;
      while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (off[mid] <= r) lo = mid;
        else hi = mid;
      }
      ex = lo;
    }
    tile_expert[tile] = ex;
  }
  // padding: each segment's tail, then the rows past the last segment
  for (int e = 0; e <= EE; ++e) {
    const int b = e < EE ? off[e] + cnt[e] : off[EE];
    const int end = e < EE ? off[e + 1] : num_tiles * kTile;
    for (int r = b + tid; r < end; r += kAlignThreads) {
      row_token[r] = -1;
      row_weight[r] = 0.f;
    }
  }
}

__global__ __launch_bounds__(kAlignThreads) void moe_align_place_kernel(
    const int64_t* __restrict__ topk_idx, const float* __restrict__ topk_w, int T, int top_k, int E, int S,
    const int32_t* __restrict__ hist, const int32_t* __restrict__ off, int32_t* __restrict__ row_token,
    float* __restrict__ row_weight, int32_t* __restrict__ entry_row) {
  const int kk = top_k + S, EE = E + S;
  const int64_t n = (int64_t)T * kk;
  const int64_t i = (int64_t)blockIdx.x * kAlignThreads + threadIdx.x;
  if (i >= n) return;
  int t, e;
  float wt;
  entry(topk_idx, topk_w, i, kk, top_k, E, t, e, wt);
  if (e < 0) return;  // entry_row already -1
  const int row = off[e] + hist[(int64_t)blockIdx.x * EE + e] + entry_row[i];
  row_token[row] = t;
  row_weight[row] = wt;
  entry_row[i] = row;
}

// One workgroup per token, 8 consecutive columns per thread and pass.
template <typename OutT>
__global__ __launch_bounds__(256) void moe_combine_kernel(const OutT* __restrict__ out, int64_t ld,
                                                          const int32_t* __restrict__ entry_row,
                                                          const int64_t* __restrict__ topk_idx,
                                                          const float* __restrict__ topk_w, int top_k, int E,
                                                          int S, const float* __restrict__ b2, int d,
                                                          uint16_t* __restrict__ y) {
  const int t = blockIdx.x, kk = top_k + S;
  __shared__ int rows[kAlignMaxExperts];
  __shared__ int exs[kAlignMaxExperts];
  __shared__ float wts[kAlignMaxExperts];
  if ((int)threadIdx.x < kk) {
    int tt, e;
    float wt;
    entry(topk_idx, topk_w, (int64_t)t * kk + threadIdx.x, kk, top_k, E, tt, e, wt);
    rows[threadIdx.x] = entry_row[(int64_t)t * kk + threadIdx.x];
    exs[threadIdx.x] = e;
    wts[threadIdx.x] = wt;
  }
  __syncthreads();
  for (int c = threadIdx.x * 8; c < d; c += 256 * 8) {
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int j = 0; j < kk; ++j) {
      if (rows[j] < 0) continue;
      float v[8];
      if constexpr (sizeof(OutT) == 4) {
        const float4* p = reinterpret_cast<const float4*>(out + (int64_t)rows[j] * ld + c);
        const float4 a = p[0], b = p[1];
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
      } else {
        unpack8(*reinterpret_cast<const uint4*>(out + (int64_t)rows[j] * ld + c), v);
      }
#pragma unroll
      for (int x = 0; x < 8; ++x) acc[x] += v[x];
    }
    if (b2 != nullptr) {
      for (int j = 0; j < kk; ++j) {
        if (rows[j] < 0) continue;
        const float* bb = b2 + (int64_t)exs[j] * d + c;
#pragma unroll
        for (int x = 0; x < 8; ++x) acc[x] = fmaf(wts[j], bb[x], acc[x]);
      }
    }
    uint4 o;
    o.x = pack_bf16x2(acc[0], acc[1]);
    o.y = pack_bf16x2(acc[2], acc[3]);
    o.z = pack_bf16x2(acc[4], acc[5]);
    o.w = pack_bf16x2(acc[6], acc[7]);
    *reinterpret_cast<uint4*>(y + (int64_t)t * d + c) = o;
  }
}

// ------------------------------------------------ segment reduce (Triton) --
__device__ __forceinline__ float load_val(const void* p, int64_t i, bool f32) {
  return f32 ? reinterpret_cast<const float*>(p)[i] : bf16_to_f32(reinterpret_cast<const uint16_t*>(p)[i]);
}
__device__ __forceinline__ void store_val(void* p, int64_t i, float v, bool f32) {
  if (f32) reinterpret_cast<float*>(p)[i] = v;
  else reinterpret_cast<uint16_t*>(p)[i] = (uint16_t)f32_to_bf16(v);
}

// first position p in [0, n) with idx[p] >= key (n if none)
__device__ __forceinline__ int64_t lower_bound(const int64_t* idx, int64_t n, int64_t key) {
  int64_t lo = 0, hi = n;
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    if (idx[mid] < key) lo = mid + 1;
    else hi = mid;
  }
  return lo;
}

// One workgroup per output token; entries p of its segment in increasing
// order (perm == nullptr: p itself, sorted input; else perm[p], the entry
// placed at p by the unsorted form).
constexpr int kSegSort = 256;  // segments up to this length are summed in entry order

__global__ __launch_bounds__(256) void segment_reduce_kernel(const void* __restrict__ x, bool x_f32, int64_t ldx,
                                                             const void* __restrict__ w, bool w_f32,
                                                             const int64_t* __restrict__ sorted_idx, int64_t n,
                                                             const int32_t* __restrict__ seg_off,
                                                             const int32_t* __restrict__ perm, int d,
                                                             void* __restrict__ y) {
  __shared__ int64_t bounds[2];
  __shared__ int order[kSegSort];
  const int t = blockIdx.x;
  if (threadIdx.x == 0) {
    if (seg_off != nullptr) {
      bounds[0] = seg_off[t];
      bounds[1] = seg_off[t + 1];
    } else {
      bounds[0] = lower_bound(sorted_idx, n, t);
      bounds[1] = lower_bound(sorted_idx, n, (int64_t)t + 1);
    }
  }
  __syncthreads();
  const int64_t s0 = bounds[0], len = bounds[1] - bounds[0];
  // the unsorted form places a token's entries in arbitrary order: sort the
  // (unique) entry indices of short segments so that the sum runs in entry order
  const bool sorted_here = perm != nullptr && len <= kSegSort;
  if (sorted_here) {
    const int j = threadIdx.x;
    int v = 0, rank = 0;
    if (j < len) {
      v = perm[s0 + j];
      for (int q = 0; q < len; ++q) rank += perm[s0 + q] < v;
      order[rank] = v;
    }
    __syncthreads();
  }
  for (int c = threadIdx.x; c < d; c += 256) {
    float acc = 0.f;
    for (int64_t q = 0; q < len; ++q) {
      const int64_t p = sorted_here ? order[q] : (perm != nullptr ? perm[s0 + q] : s0 + q);
      acc = fmaf(load_val(x, p * ldx + c, x_f32), load_val(w, p, w_f32), acc);
    }
    store_val(y, (int64_t)t * d + c, acc, x_f32);
  }
}

__global__ __launch_bounds__(256) void fill_i32_kernel(int32_t* __restrict__ p, int64_t n, int32_t v) {
  for (int64_t i = blockIdx.x * 256ll + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) p[i] = v;
}

__global__ __launch_bounds__(256) void count_tokens_kernel(const int64_t* __restrict__ idx, int64_t n,
                                                           int num_tokens, int32_t* __restrict__ cnt) {
  for (int64_t i = blockIdx.x * 256ll + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const int64_t t = idx[i];
    if (t >= 0 && t < num_tokens) atomicAdd(&cnt[t], 1);
  }
}

// exclusive scan of cnt[0 .. m) into off[0 .. m] by one workgroup
__global__ __launch_bounds__(1024) void scan_counts_kernel(const int32_t* __restrict__ cnt, int m,
                                                           int32_t* __restrict__ off) {
  __shared__ int part[1024];
  const int tid = threadIdx.x;
  const int per = (m + 1023) / 1024;
  const int b = tid * per, e = min(m, b + per);
  int s = 0;
  for (int i = b; i < e; ++i) s += cnt[i];
  part[tid] = s;
  __syncthreads();
  for (int o = 1; o < 1024; o <<= 1) {  // Hillis-Steele inclusive scan
    const int v = tid >= o ? part[tid - o] : 0;
    __syncthreads();
    part[tid] += v;
    __syncthreads();
  }
  int run = tid > 0 ? part[tid - 1] : 0;
  for (int i = b; i < e; ++i) {
    off[i] = run;
    run += cnt[i];
  }
  if (tid == 1023) off[m] = part[1023];
}

__global__ __launch_bounds__(256) void place_tokens_kernel(const int64_t* __restrict__ idx, int64_t n,
                                                           int num_tokens, const int32_t* __restrict__ off,
                                                           int32_t* __restrict__ cursor,
                                                           int32_t* __restrict__ perm) {
  for (int64_t i = blockIdx.x * 256ll + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const int64_t t = idx[i];
    if (t >= 0 && t < num_tokens) perm[off[t] + atomicAdd(&cursor[t], 1)] = (int32_t)i;
  }
}

unsigned grid_for(int64_t n) { return (unsigned)std::min<int64_t>((n + 255) / 256, 4096); }

}  // namespace
}  // namespace lfs

using namespace lfs;

extern "C" int64_t lfs_moe_align_tiles(int64_t T, int32_t top_k, int32_t num_experts, int32_t num_shared) {
  if (T <= 0 || top_k <= 0 || num_experts <= 0 || num_shared < 0) return 0;
  const int64_t n = T * (top_k + num_shared);
  // sum_e ceil(c_e / 128) <= (n + E' * 127) / 128 over E' non-empty segments
  return (n + (int64_t)(num_experts + num_shared) * (kTile - 1) + kTile - 1) / kTile;
}

extern "C" int64_t lfs_moe_align_workspace_bytes(int64_t T, int32_t top_k, int32_t num_experts,
                                                 int32_t num_shared) {
  if (T < 0 || top_k <= 0 || num_experts <= 0 || num_shared < 0) return 0;
  const int64_t EE = num_experts + num_shared;
  const int64_t chunks = (T * (top_k + num_shared) + kAlignThreads - 1) / kAlignThreads;
  return 4 * (chunks * EE + 2 * EE + 1);
}

extern "C" int lfs_moe_align(const int64_t* topk_idx, const float* topk_weight, int64_t T, int32_t top_k,
                             int32_t num_experts, int32_t num_shared, int32_t* row_token, float* row_weight,
                             int32_t* tile_expert, int64_t num_tiles, int32_t* entry_row, void* workspace,
                             int64_t workspace_bytes, void* stream) {
  LFS_REQUIRE(T >= 0 && top_k >= 1 && num_experts >= 1 && num_shared >= 0, "moe_align: bad shape");
  LFS_REQUIRE(num_experts + num_shared <= kAlignMaxExperts && top_k <= num_experts,
              "moe_align: at most %d experts, top_k <= num_experts", kAlignMaxExperts);
  const int64_t need = lfs_moe_align_tiles(T, top_k, num_experts, num_shared);
  LFS_REQUIRE(num_tiles >= need, "moe_align: %lld tiles needed, %lld given", (long long)need,
              (long long)num_tiles);
  LFS_REQUIRE(num_tiles * kTile < (1ll << 31) && T * (top_k + num_shared) < (1ll << 31),
              "moe_align: too many rows");
  if (num_tiles == 0) return 0;
  LFS_REQUIRE(row_token && row_weight && tile_expert, "moe_align: null pointer");
  hipStream_t st = (hipStream_t)stream;
  const int EE = num_experts + num_shared;
  // (T == 0: no chunks; every tile unused, every row padding)
  const int64_t wneed = lfs_moe_align_workspace_bytes(T, top_k, num_experts, num_shared);
  LFS_REQUIRE(workspace != nullptr && workspace_bytes >= wneed,
              "moe_align: needs a workspace of %lld bytes", (long long)wneed);
  LFS_REQUIRE(T == 0 || (topk_idx && topk_weight && entry_row), "moe_align: null pointer");
  const int chunks = (int)((T * (top_k + num_shared) + kAlignThreads - 1) / kAlignThreads);
  int32_t* hist = (int32_t*)workspace;
  int32_t* cnt = hist + (int64_t)chunks * EE;
  int32_t* off = cnt + EE;
  if (chunks > 0)
    hipLaunchKernelGGL(moe_align_rank_kernel, dim3((unsigned)chunks), dim3(kAlignThreads), 0, st, topk_idx,
                       topk_weight, (int)T, top_k, num_experts, num_shared, entry_row, hist);
  hipLaunchKernelGGL(moe_align_offsets_kernel, dim3(1), dim3(kAlignThreads), 0, st, chunks, num_experts,
                     num_shared, hist, cnt, off, row_token, row_weight, tile_expert, (int)num_tiles);
  if (chunks > 0)
    hipLaunchKernelGGL(moe_align_place_kernel, dim3((unsigned)chunks), dim3(kAlignThreads), 0, st, topk_idx,
                       topk_weight, (int)T, top_k, num_experts, num_shared, (const int32_t*)hist,
                       (const int32_t*)off, row_token, row_weight, entry_row);
  return check_launch("moe_align");
}

extern "C" int lfs_moe_combine(const void* out, int32_t out_is_f32, int64_t ld, const int32_t* entry_row,
                               const int64_t* topk_idx, const float* topk_weight, int64_t T, int32_t top_k,
                               int32_t num_experts, int32_t num_shared, const float* down_bias, int32_t d, void* y,
                               void* stream) {
  LFS_REQUIRE(T >= 0 && top_k >= 1 && num_experts >= 1 && num_shared >= 0 &&
                  top_k + num_shared <= kAlignMaxExperts,
              "moe_combine: bad shape");
  LFS_REQUIRE(d > 0 && d % 8 == 0 && ld >= d && ld % 8 == 0, "moe_combine: d=%d must be a multiple of 8", d);
  if (T == 0) return 0;
  LFS_REQUIRE(out && entry_row && topk_idx && topk_weight && y, "moe_combine: null pointer");
  LFS_REQUIRE((((uintptr_t)out) | ((uintptr_t)y)) % 16 == 0, "moe_combine: buffers must be 16-byte aligned");
  LFS_REQUIRE(T < (1ll << 31), "moe_combine: too many tokens");
  if (out_is_f32)
    hipLaunchKernelGGL(moe_combine_kernel<float>, dim3((unsigned)T), dim3(256), 0, (hipStream_t)stream,
                       (const float*)out, ld, entry_row, topk_idx, topk_weight, top_k, num_experts, num_shared,
                       down_bias, d, (uint16_t*)y);
  else
    hipLaunchKernelGGL(moe_combine_kernel<uint16_t>, dim3((unsigned)T), dim3(256), 0, (hipStream_t)stream,
                       (const uint16_t*)out, ld, entry_row, topk_idx, topk_weight, top_k, num_experts, num_shared,
                       down_bias, d, (uint16_t*)y);
  return check_launch("moe_combine");
}

extern "C" int lfs_segment_reduce_weighted(const void* x, int32_t x_is_f32, int64_t ldx, const void* weights,
                                           int32_t w_is_f32, const int64_t* sorted_token_idx, int64_t n,
                                           int64_t num_tokens, int32_t d, void* y, void* stream) {
  LFS_REQUIRE(n >= 0 && num_tokens >= 0 && d > 0 && ldx >= d, "segment_reduce_weighted: bad shape");
  LFS_REQUIRE(num_tokens < (1ll << 31), "segment_reduce_weighted: too many tokens");
  if (num_tokens == 0) return 0;
  LFS_REQUIRE(y && (n == 0 || (x && weights && sorted_token_idx)), "segment_reduce_weighted: null pointer");
  hipLaunchKernelGGL(segment_reduce_kernel, dim3((unsigned)num_tokens), dim3(256), 0, (hipStream_t)stream, x,
                     x_is_f32 != 0, ldx, weights, w_is_f32 != 0, sorted_token_idx, n, (const int32_t*)nullptr,
                     (const int32_t*)nullptr, d, y);
  return check_launch("segment_reduce_weighted");
}

extern "C" int64_t lfs_scatter_add_weighted_workspace_bytes(int64_t n, int64_t num_tokens) {
  if (n < 0 || num_tokens < 0) return 0;
  return 4 * (3 * num_tokens + 1 + n);  // counts, offsets (+1), cursors, placement
}

extern "C" int lfs_scatter_add_weighted(const void* x, int32_t x_is_f32, int64_t ldx, const void* weights,
                                        int32_t w_is_f32, const int64_t* token_idx, int64_t n, int64_t num_tokens,
                                        int32_t d, void* y, void* workspace, int64_t workspace_bytes,
                                        void* stream) {
  LFS_REQUIRE(n >= 0 && num_tokens >= 0 && d > 0 && ldx >= d, "scatter_add_weighted: bad shape");
  LFS_REQUIRE(num_tokens < (1ll << 30) && n < (1ll << 31), "scatter_add_weighted: too large");
  if (num_tokens == 0) return 0;
  const int64_t need = lfs_scatter_add_weighted_workspace_bytes(n, num_tokens);
  LFS_REQUIRE(workspace != nullptr && workspace_bytes >= need,
              "scatter_add_weighted: needs a workspace of %lld bytes", (long long)need);
  LFS_REQUIRE(y && (n == 0 || (x && weights && token_idx)), "scatter_add_weighted: null pointer");
  hipStream_t st = (hipStream_t)stream;
  int32_t* cnt = (int32_t*)workspace;
  int32_t* off = cnt + num_tokens;
  int32_t* cur = off + num_tokens + 1;
  int32_t* perm = cur + num_tokens;
  // zero the counts and cursors with a kernel (capturable, unlike a memset node)
  hipLaunchKernelGGL(fill_i32_kernel, dim3(grid_for(num_tokens)), dim3(256), 0, st, cnt, num_tokens, 0);
  hipLaunchKernelGGL(fill_i32_kernel, dim3(grid_for(num_tokens)), dim3(256), 0, st, cur, num_tokens, 0);
  if (n > 0)
    hipLaunchKernelGGL(count_tokens_kernel, dim3(grid_for(n)), dim3(256), 0, st, token_idx, n, (int)num_tokens,
                       cnt);
  hipLaunchKernelGGL(scan_counts_kernel, dim3(1), dim3(1024), 0, st, (const int32_t*)cnt, (int)num_tokens, off);
  if (n > 0)
    hipLaunchKernelGGL(place_tokens_kernel, dim3(grid_for(n)), dim3(256), 0, st, token_idx, n, (int)num_tokens,
                       (const int32_t*)off, cur, perm);
  hipLaunchKernelGGL(segment_reduce_kernel, dim3((unsigned)num_tokens), dim3(256), 0, st, x, x_is_f32 != 0, ldx,
                     weights, w_is_f32 != 0, (const int64_t*)nullptr, n, (const int32_t*)off,
                     (const int32_t*)perm, d, y);
  return check_launch("scatter_add_weighted");
}
