// Read ceiling for the paged decode (benchmark instrument, not part of the
// kernel library).  lfs_probe_read_chunks reads a list of byte ranges -- on
// the decode benchmark, exactly the K and V token rows the decode reads:
// each (sequence, block) contributes the block's valid rows, which are
// contiguous in the [num_blocks, block_size, Hkv, D] pool -- with nothing
// computed on the data, so its time is what a read of those bytes costs at
// that size, cold (the benchmark flushes the 256 MB last-level cache
// before every call).
//
// The ranges arrive as 4 KB chunks (absolute device address, byte count
// <= 4096, a multiple of 16).  Workgroup w owns chunks [w*C, (w+1)*C),
// C = ceil(n / gridDim.x): it copies their descriptors to LDS in one round
// trip, then its 256 threads stream U chunks at a time, one 16-byte
// nontemporal load per thread per chunk, all U loads in flight together.
// The loaded words are folded into one float per thread that is stored
// only if it equals a value no read produces, so every load is kept and
// nothing is written.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/lfs_kernels.h"

namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int kMaxChunksPerGroup = 1024;

template <int U>
__global__ __launch_bounds__(256) void read_chunks_kernel(const uint64_t* __restrict__ addr,
                                                          const uint32_t* __restrict__ nbytes, int64_t n,
                                                          int64_t per_group, float* __restrict__ sink) {
  __shared__ uint64_t s_addr[kMaxChunksPerGroup];
  __shared__ uint32_t s_bytes[kMaxChunksPerGroup];
  const int64_t c0 = (int64_t)blockIdx.x * per_group;
  const int cnt = (int)max((int64_t)0, min(per_group, n - c0));
  for (int i = threadIdx.x; i < cnt; i += blockDim.x) {
    s_addr[i] = addr[c0 + i];
    s_bytes[i] = nbytes[c0 + i];
  }
  __syncthreads();
  const uint32_t off = threadIdx.x * 16u;
  uint32_t fold = 0;
  for (int i0 = 0; i0 < cnt; i0 += U) {
    u32x4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      v[u] = u32x4{0u, 0u, 0u, 0u};
      const int i = i0 + u;
      if (i < cnt && off < s_bytes[i])
        v[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(s_addr[i] + off));
    }
#pragma unroll
    for (int u = 0; u < U; ++u) fold ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
  }
  if (fold == 0x7FC01234u) sink[blockIdx.x * blockDim.x + threadIdx.x] = __uint_as_float(fold);
}

}  // namespace

// Read every byte range of the chunk list once (see above).  Returns 0, or
// -1 for bad arguments (per-group chunk count above 1024), or the launch
// error.  sink: at least ngroups * 256 floats (never written in practice).
extern "C" int lfs_probe_read_chunks(const uint64_t* chunk_addr, const uint32_t* chunk_bytes, int64_t nchunks,
                                     int32_t ngroups, int32_t unroll, float* sink, void* stream) {
  if (nchunks <= 0) return 0;
  if (ngroups <= 0 || chunk_addr == nullptr || chunk_bytes == nullptr || sink == nullptr) return -1;
  const int64_t per = (nchunks + ngroups - 1) / ngroups;
  if (per > kMaxChunksPerGroup) return -1;
  hipStream_t st = (hipStream_t)stream;
  if (unroll == 16)
    hipLaunchKernelGGL(read_chunks_kernel<16>, dim3((unsigned)ngroups), dim3(256), 0, st, chunk_addr, chunk_bytes,
                       nchunks, per, sink);
  else if (unroll == 8)
    hipLaunchKernelGGL(read_chunks_kernel<8>, dim3((unsigned)ngroups), dim3(256), 0, st, chunk_addr, chunk_bytes,
                       nchunks, per, sink);
  else
    return -1;
  return (int)hipGetLastError();
}
