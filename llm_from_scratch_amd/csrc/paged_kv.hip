// Paged-KV kernels for gfx950: KV slot writes and split-K paged decode.
//
// KV pool layout per layer: [num_blocks, block_size, num_kv_heads, head_dim]
// bf16, as allocated by engine/model_runner.py:184-190 of the reference; one
// token's K (or V) row for all kv heads is Hkv*D*2 contiguous bytes.
//
// paged decode, phase 1: a wave streams a range of one (sequence, kv head)'s
//   context (decode_chunk) in tiles of up to 64 tokens that never cross a
//   KV block (one block-table lookup per tile): S = K q^T on MFMA for the G
//   query heads of its kv head, online softmax in the log2 domain, P through
//   a wave-private LDS slice, P.V in fp32 registers.  Loads run one tile
//   ahead.  The partial (unnormalised o, m, l) of the range goes to the
//   workspace, or, when the range is the whole context, the normalised bf16
//   output is written directly.  The ranges come from either
//   paged_decode_balanced (default: one 4-wave workgroup per CU, each an
//   equal share of the (sequence, kv-head group, tile) work) or
//   paged_decode_split (one wave per (sequence, kv head, chunk of
//   blocks_per_split blocks)).
// phase 2 (paged_decode_merge, one workgroup per (head, sequence)):
//   log-sum-exp merge of the chunks, normalise, bf16.  Padding rows
//   (context_len 0) get zeros.  paged_decode_merge_quant_group (one
//   workgroup per 128-value group of an output row) does the same and also
//   writes the group's act_quant codes and scale (the output projection's
//   FP8 input).
#include "common.h"
#include "rope.h"

#include <mutex>

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

// One wave per (sequence, kv head, range of the context).  Per tile of T
// tokens (one KV block never straddled):
//   K  : MFMA A operand straight from HBM -- lane l loads token (l % 16) of a
//        16-token group, dims c*32 + (l / 16)*8 .. +7 (16 B);
//   q^T: MFMA B operand, column j = l % 16 is query head kh*G + j (zero for
//        j >= G);
//   S  = K q^T with v_mfma_f32_16x16x32_bf16: lane l ends with the scores of
//        head (l % 16) for tokens 4*(l / 16) .. +3 of each group, so the
//        online-softmax max/sum per head is a 2-step xor over lanes 16, 32;
//   P  goes through a wave-private LDS slice [T][G] to the P.V mapping;
//   V  : lane l owns token (l / (D/8)) + (64/(D/8))*i and dims
//        (l % (D/8))*8 .. +7 (coalesced 16-byte loads), fp32 FMAs into
//        acc[G][8], rescaled by exp2(m_old - m_new) read from lane g.
// Loads are software-pipelined one tile ahead (two K and two V buffers: a
// step issues the next tile's loads, then computes on the tile loaded by
// the step before) with nontemporal 16-byte loads, since every KV row is
// read exactly once.  One tile in flight per wave is 16 KiB, 16 MiB over
// the chip: enough to keep HBM busy, and a new request does not queue
// behind twice that (two tiles ahead measured 4 % slower on every decode
// shape).  There is no workgroup barrier: waves exit independently.  A
// range that covers the whole context writes the normalised bf16 output
// directly; otherwise the unnormalised partial (o, m, l) goes to the
// workspace for the merge.
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

// Reductions over lanes l, l^16 (and l^32) without LDS: v_permlane16_swap
// (v_permlane32_swap) of a value with itself leaves the value of lane l in
// one result and that of lane l^16 (l^32) in the other, in both lanes of the
// pair.  Same operands in the same order as x op __shfl_xor(x, 16 / 32), so
// the results are bit-identical (IEEE add and max are commutative).
__device__ __forceinline__ float max_xor16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float max_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_xor16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float sum_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// The per-wave pieces of a decode range.  A tile is (n, off): n valid rows
// (0 for a skipped block or a look-ahead filler) starting at element offset
// off of the cache.
template <int D, int G>
struct DecodeWave {
  using Geo = DecodeGeom<D>;
  static constexpr int GP = G <= 4 ? 4 : 8;  // padded heads per token in the P slice
  typedef uint4 KBuf[Geo::NG][Geo::NDC];
  typedef uint4 VBuf[Geo::UV];
  typedef uint4 QBuf[Geo::NDC];

  int lane, j, kq, ts, dc;
  int64_t row;  // elements per token row of the cache (Hkv * D)
  float acc[G][8];
  float m_run, l_run;

  __device__ __forceinline__ DecodeWave(int lane_, int Hkv) : lane(lane_) {
    j = lane & 15;
    kq = lane >> 4;
    ts = lane / Geo::LPR;
    dc = lane % Geo::LPR;
    row = (int64_t)Hkv * D;
    reset();
  }
  __device__ __forceinline__ void reset() {
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[g][e] = 0.f;
    m_run = -INFINITY;
    l_run = 0.f;
  }
  // q^T columns of kv head kh of sequence b (lanes j >= G load nothing)
  __device__ __forceinline__ void load_q(QBuf& qa, const uint16_t* __restrict__ q, int64_t b, int kh, int Hq) const {
#pragma unroll
    for (int c = 0; c < Geo::NDC; ++c) {
      uint4 w = make_uint4(0, 0, 0, 0);
      if (j < G) w = *reinterpret_cast<const uint4*>(q + ((int64_t)b * Hq + kh * G + j) * D + c * 32 + kq * 8);
      qa[c] = w;
    }
  }
  // the same from a [G][D] bf16 block in LDS (this kv head's query rows)
  __device__ __forceinline__ void load_q_lds(QBuf& qa, const uint16_t* ql) const {
#pragma unroll
    for (int c = 0; c < Geo::NDC; ++c) {
      uint4 w = make_uint4(0, 0, 0, 0);
      if (j < G) w = *reinterpret_cast<const uint4*>(ql + j * D + c * 32 + kq * 8);
      qa[c] = w;
    }
  }
  // a tile whose rows are all the one token row k / v (bf16 [D] each, in
  // LDS): with n = 1 in tile() it adds that single token
  __device__ __forceinline__ void row_tile(KBuf& ka, VBuf& va, const uint16_t* kl, const uint16_t* vl) const {
#pragma unroll
    for (int g16 = 0; g16 < Geo::NG; ++g16)
#pragma unroll
      for (int c = 0; c < Geo::NDC; ++c) ka[g16][c] = *reinterpret_cast<const uint4*>(kl + c * 32 + kq * 8);
#pragma unroll
    for (int i = 0; i < Geo::UV; ++i) va[i] = *reinterpret_cast<const uint4*>(vl + dc * 8);
  }
  // Every load is issued unconditionally: rows past the valid count n read
  // row n-1 (row 0 of block 0 for a skipped block), whose scores are masked
  // and whose P is 0 (a skipped block's P.V is not run).  Offsets inside a
  // tile are 32-bit from a wave-uniform base.
  __device__ __forceinline__ void load_k(KBuf& ka, const uint16_t* __restrict__ kc, int n, int64_t off) const {
    const uint16_t* kb = kc + off;
    const int nn = max(n, 1);
#pragma unroll
    for (int g16 = 0; g16 < Geo::NG; ++g16) {
      const int tr = min(g16 * 16 + j, nn - 1);
#pragma unroll
      for (int c = 0; c < Geo::NDC; ++c)
        ka[g16][c] = nt_load16(kb + (uint32_t)(tr * (int)row + c * 32 + kq * 8));
    }
  }
  __device__ __forceinline__ void load_v(VBuf& va, const uint16_t* __restrict__ vc, int n, int64_t off) const {
    const uint16_t* vb = vc + off;
    const int nn = max(n, 1);
#pragma unroll
    for (int i = 0; i < Geo::UV; ++i)
      va[i] = nt_load16(vb + (uint32_t)(min(ts + Geo::TPI * i, nn - 1) * (int)row + dc * 8));
  }

  // One tile of n valid rows: scores (log2 domain), online-softmax update
  // for head j, P through the LDS slice pw, P.V into acc.
  __device__ __forceinline__ void tile(const KBuf& ka, const VBuf& va, const QBuf& qa, int n, float scale_log2,
                                       float* __restrict__ pw) {
    float s[Geo::NG][4];
    float tmax = -INFINITY;
#pragma unroll
    for (int g16 = 0; g16 < Geo::NG; ++g16) {
      v4f sc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < Geo::NDC; ++c)
        sc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, ka[g16][c]),
                                                     __builtin_bit_cast(v8bf, qa[c]), sc, 0, 0, 0);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int tok = g16 * 16 + kq * 4 + r;
        s[g16][r] = tok < n ? sc[r] * scale_log2 : -INFINITY;
        tmax = fmaxf(tmax, s[g16][r]);
      }
    }
    tmax = max_xor16(tmax);
    tmax = max_xor32(tmax);
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
    psum = sum_xor16(psum);
    psum = sum_xor32(psum);
    l_run = l_run * alpha + psum;
    m_run = m_new;
    wave_lds_sync();

    // P.V (rows past n have P = 0; a skipped block adds nothing)
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
    wave_lds_sync();
  }

  // End of a range: sum the token subgroups (lanes with the same dc), then
  // the normalised bf16 output of query heads kh*G + g (whole context) or
  // the unnormalised partial to workspace rows prow + g.
  // Sum acc over the token subgroups: afterwards lanes with ts == 0 hold the
  // wave's totals for dims dc*8 .. +7 of every head.
  // (distances LPR, 2 LPR, ..., 32: the same sums as acc += __shfl_xor(acc, o))
  template <int O = Geo::LPR>
  __device__ __forceinline__ void reduce_lanes() {
    if constexpr (O < 64) {
#pragma unroll
      for (int g = 0; g < G; ++g)
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[g][e] = xor_sum<O>(acc[g][e]);
      reduce_lanes<2 * O>();
    }
  }
  __device__ __forceinline__ void finish(bool whole, uint16_t* __restrict__ out, float* __restrict__ ws_o,
                                         float* __restrict__ ws_ml, int64_t b, int kh, int Hq, int64_t prow) {
    reduce_lanes();
    if (whole) {
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
          *reinterpret_cast<uint4*>(out + (b * Hq + kh * G + g) * D + dc * 8) = o;
        }
      }
    } else {
      if (ts == 0) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
          float* dst = ws_o + (prow + g) * D + dc * 8;
          *reinterpret_cast<float4*>(dst) = make_float4(acc[g][0], acc[g][1], acc[g][2], acc[g][3]);
          *reinterpret_cast<float4*>(dst + 4) = make_float4(acc[g][4], acc[g][5], acc[g][6], acc[g][7]);
        }
      }
      if (lane < G) {
        ws_ml[(prow + lane) * 2 + 0] = m_run;
        ws_ml[(prow + lane) * 2 + 1] = l_run;
      }
    }
  }
};

// One wave streams tiles of kv head kh of one sequence into w: tile i of the
// walk covers context rows [t_begin + i*tstride*tile, +tile) clipped to
// t_end (t_begin a multiple of `tile`, t_end <= the context length), so a
// range of consecutive tiles is tstride 1 and every S-th tile from s*tile
// is t_begin = s*tile, tstride S.  btrow: the sequence's block-table row;
// block ids at or past id_end are never loaded.  pw: the wave's private
// LDS slice (T * GP floats).  pro() runs once, after the first tile's loads
// are issued and before anything reads qa (a caller may fill qa there); an
// empty walk does not run it.
struct NoPrologue {
  __device__ __forceinline__ void operator()() const {}
};
template <int D, int G, class Pro = NoPrologue>
__device__ __forceinline__ void decode_walk(
    DecodeWave<D, G>& w, const typename DecodeWave<D, G>::QBuf& qa, const uint16_t* __restrict__ kc,
    const uint16_t* __restrict__ vc, const int32_t* __restrict__ btrow, int BS, int64_t NB, int tile,
    float scale_log2, int kh, int64_t t_begin, int64_t t_end, int tstride, int64_t id_end,
    float* __restrict__ pw, Pro&& pro = Pro()) {
  using W = DecodeWave<D, G>;
  const int lane = w.lane;
  const int64_t step_rows = (int64_t)tile * tstride;
  const int ntiles = (int)((t_end - t_begin + step_rows - 1) / step_rows);
  // The walk's block ids, 256 at a time (window w0 .. w0 + 255 of the table
  // row): lane l holds ids 4l .. 4l+3 of the window, read back with
  // readlane, so no tile waits on a scalar load of its block id.  Ids at or
  // past id_end are never read (loaded as 0 to stay in bounds).  The window
  // is (re)loaded only where a group of MAXT tiles starts, and waited for
  // there: the group's tiles then read ids with no load pending on them, so
  // the compiler puts no vmcnt(0) between a tile's loads and the next
  // tile's (which would drain the tile in flight).  A group spans
  // (MAXT-1)*tstride*tile + tile <= 256*BS rows for tstride <= 36.
  int64_t w0 = -1;
  uint4 ids = make_uint4(0, 0, 0, 0);
  auto load_window = [&](int64_t wb) {
    w0 = wb;
    const int64_t e = wb + 4 * lane;
    uint32_t v[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) v[c] = e + c < id_end ? (uint32_t)btrow[e + c] : 0u;
    ids = make_uint4(v[0], v[1], v[2], v[3]);
    __builtin_amdgcn_s_waitcnt(0x0F70);
  };
  auto block_id = [&](int64_t bi) -> int32_t {
    const int e = __builtin_amdgcn_readfirstlane((int)(bi - w0));
    const int src = e >> 2, c = e & 3;
    const uint32_t x = c == 0 ? ids.x : c == 1 ? ids.y : c == 2 ? ids.z : ids.w;
    return (int32_t)__builtin_amdgcn_readlane((int)x, src);
  };
  // tile i of the walk: valid row count (0 for a skipped block) and the
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
    const int64_t t0 = t_begin + (int64_t)i * step_rows;
    n = (int)min((int64_t)tile, t_end - t0);
    const int32_t blk = block_id(t0 / BS);
    const bool ok = blk >= 0 && (int64_t)blk < NB;
    if (!ok) n = 0;  // invalid block: contributes nothing
    off = ((int64_t)(ok ? blk : 0) * BS + (t0 % BS)) * w.row + (int64_t)kh * D;
  };

  // Pipeline one tile deep over two K and two V buffers: step i issues the
  // loads of tile i+1 into the other buffers, then computes tile i.  The
  // tiles of a walk are processed in straight-line code (MAXT steps
  // unrolled, with early exits), every step issuing the same loads, so the
  // compiler's in-order wait counts are exact: tile i waits only for its own
  // loads.  Walks longer than MAXT tiles go MAXT tiles at a time.
  constexpr int MAXT = 8;
  typename W::KBuf ka0, ka1;
  typename W::VBuf va0, va1;
  int nb0 = 0, nb1 = 0;
  auto step = [&](int i, typename W::KBuf& ka, typename W::VBuf& va, int nb, typename W::KBuf& kx,
                  typename W::VBuf& vx, int& nbx) {
    int n1;
    int64_t o1;
    tile_at(i + 1, n1, o1);
    __builtin_amdgcn_sched_barrier(0);  // keep the issue order the wait counts assume
    w.load_k(kx, kc, n1, o1);
    w.load_v(vx, vc, n1, o1);
    __builtin_amdgcn_sched_barrier(0);
    nbx = n1;
    w.tile(ka, va, qa, nb, scale_log2, pw);
  };
  for (int base = 0; base < ntiles; base += MAXT) {
    last = min(ntiles, base + MAXT);
    {
      const int64_t bf = (t_begin + (int64_t)base * step_rows) / BS;
      const int64_t bl = (t_begin + (int64_t)(last - 1) * step_rows) / BS;
      if (base == 0 || __builtin_amdgcn_readfirstlane((int)(bf < w0 || bl >= w0 + 256))) load_window(bf);
    }
    {
      int64_t o0;
      tile_at(base, nb0, o0);
      w.load_k(ka0, kc, nb0, o0);
      w.load_v(va0, vc, nb0, o0);
    }
    if (base == 0) pro();
#pragma unroll
    for (int u = 0; u < MAXT; u += 2) {
      if (base + u >= last) break;
      step(base + u, ka0, va0, nb0, ka1, va1, nb1);
      if (base + u + 1 >= last) break;
      step(base + u + 1, ka1, va1, nb1, ka0, va0, nb0);
    }
    __builtin_amdgcn_s_waitcnt(0x0F70);  // drain the look-ahead loads
  }
  (void)lane;
}

// One wave: kv head kh of sequence b over context rows [t_begin, t_end)
// (t_begin a multiple of `tile`, t_end <= Lc).  A range that is the whole
// context (t_begin == 0, t_end >= Lc) writes the normalised bf16 output;
// otherwise the unnormalised partial of query head kh*G + g goes to row
// prow + g of the workspace (o: ws_o[row*D ..], (m, l): ws_ml[row*2 ..]).
// pw: the wave's private LDS slice (T * GP floats).
template <int D, int G>
__device__ __forceinline__ void decode_chunk(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ kc,
    const uint16_t* __restrict__ vc, const int32_t* __restrict__ btrow, float* __restrict__ ws_o,
    float* __restrict__ ws_ml, uint16_t* __restrict__ out, int Hkv, int BS, int64_t NB, int tile,
    float scale_log2, int b, int kh, int64_t t_begin, int64_t t_end, int64_t Lc, int64_t prow,
    float* __restrict__ pw, int lane) {
  using W = DecodeWave<D, G>;
  W w(lane, Hkv);
  const int Hq = Hkv * G;
  typename W::QBuf qa;
  w.load_q(qa, q, b, kh, Hq);
  decode_walk<D, G>(w, qa, kc, vc, btrow, BS, NB, tile, scale_log2, kh, t_begin, t_end, 1,
                    (t_end - 1) / BS + 1, pw);
  w.finish(t_begin == 0 && t_end >= Lc, out, ws_o, ws_ml, b, kh, Hq, prow);
}

// Fixed chunks: one wave per (sequence, kv head, chunk of bps blocks), four
// kv heads of one sequence and chunk per workgroup.  Grid x = (sequence,
// kv-head group), group fastest; y = split.
// Sequence before split: workgroups are dealt round-robin to the 8 XCDs,
// so consecutive ids must not be the splits of one sequence (split s would
// always land on XCD s mod 8, and short contexts leave the high splits
// empty, i.e. whole XCDs idle).  Group fastest: the groups of one token
// row (Hkv*D*2 bytes) are read at about the same time, not one half of
// every row in the first half of the launch and the rest in the second
// (cfg4, 2 groups: 1626 -> 1523 us).
template <int D, int G>
__global__ __launch_bounds__(256) void paged_decode_split(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ kc,
    const uint16_t* __restrict__ vc, const int64_t* __restrict__ ctx_lens,
    const int32_t* __restrict__ bt, int64_t bt_stride, float* __restrict__ ws_o,
    float* __restrict__ ws_ml, uint16_t* __restrict__ out, int Hkv, int BS, int64_t NB,
    int max_blocks, int bps, int tile, float scale_log2, int max_splits, int nz) {
  using Geo = DecodeGeom<D>;
  constexpr int GP = G <= 4 ? 4 : 8;
  __shared__ __attribute__((aligned(16))) float p_lds[4][Geo::T * GP];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int kh = (int)(blockIdx.x % nz) * (blockDim.x >> 6) + wave;
  if (kh >= Hkv) return;
  const int b = (int)(blockIdx.x / nz), split = blockIdx.y;
  const int64_t Lc = min(ctx_lens[b], (int64_t)max_blocks * BS);
  const int64_t chunk = (int64_t)bps * BS;
  const int64_t t_begin = (int64_t)split * chunk;
  const int64_t t_end = min(Lc, t_begin + chunk);
  if (t_begin >= t_end) return;
  const int64_t prow = ((int64_t)b * max_splits + split) * (Hkv * G) + kh * G;
  decode_chunk<D, G>(q, kc, vc, bt + (int64_t)b * bt_stride, ws_o, ws_ml, out, Hkv, BS, NB, tile,
                     scale_log2, b, kh, t_begin, t_end, Lc, prow, p_lds[wave], lane);
}

// Balanced split: a fixed grid of nwg workgroups (wpg waves each, one kv
// head per wave; one workgroup per CU) shares the work evenly, whatever the
// context lengths.
// Work units are (sequence b, kv-head group, tile) triples in that order,
// n_b = ceil(L_b / tile) tiles per (sequence, group), where L_b is the
// clamped context length; workgroup w takes the units [w*Ct, (w+1)*Ct),
// Ct = ceil(total / nwg), and its waves walk the same tiles for the heads of
// the group (so a workgroup reads wpg adjacent head slices of each row
// together).  A (sequence, group) range that one workgroup covers entirely
// is written out directly; otherwise workgroup w's partial of pair group
// pg = b*ngroups + group is slot (w + pg)*wpg + wave -- unique, since along
// the units both w and pg are non-decreasing and one of them grows at every
// step from one (pg, w) overlap to the next.  Every workgroup scans the
// per-sequence tile counts into LDS (B <= BAL_MAXB); workgroup 0 also
// writes the scan (B+1 ints) to tp_out for the merge.
constexpr int BAL_MAXB = 8192;

__device__ __forceinline__ int decode_tiles(const int64_t* ctx_lens, int b, int64_t cap, int tile) {
  const int64_t L = min(ctx_lens[b], cap);
  return L > 0 ? (int)((L + tile - 1) / tile) : 0;
}

template <int D, int G>
__global__ __launch_bounds__(256) void paged_decode_balanced(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ kc,
    const uint16_t* __restrict__ vc, const int64_t* __restrict__ ctx_lens,
    const int32_t* __restrict__ bt, int64_t bt_stride, float* __restrict__ ws_o,
    float* __restrict__ ws_ml, int* __restrict__ tp_out, uint16_t* __restrict__ out, int Hkv, int BS,
    int64_t NB, int max_blocks, int B, int tile, float scale_log2, int ngroups) {
  using Geo = DecodeGeom<D>;
  constexpr int GP = G <= 4 ? 4 : 8;
  __shared__ __attribute__((aligned(16))) float p_lds[4][Geo::T * GP];
  __shared__ int tp[BAL_MAXB + 1];
  __shared__ int wsum[4];
  const int tid = threadIdx.x, nthr = blockDim.x;
  const int wave = tid >> 6, lane = tid & 63, wpg = nthr >> 6;
  const int64_t cap = (int64_t)max_blocks * BS;

  // ---- tp[b] = sum of n_b' for b' < b (each thread a run of sequences)
  const int per = (B + nthr - 1) / nthr;
  const int lo = min(B, tid * per), hi = min(B, lo + per);
  int run = 0;
  for (int i = lo; i < hi; ++i) {
    run += decode_tiles(ctx_lens, i, cap, tile);
    tp[i + 1] = run;
  }
  int incl = run;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int v = __shfl_up(incl, o, 64);
    if (lane >= o) incl += v;
  }
  if (lane == 63) wsum[wave] = incl;
  __syncthreads();
  int excl = incl - run;
  for (int w = 0; w < wave; ++w) excl += wsum[w];
  for (int i = lo; i < hi; ++i) tp[i + 1] += excl;
  if (tid == 0) tp[0] = 0;
  __syncthreads();
  if (blockIdx.x == 0)
    for (int i = tid; i <= B; i += nthr) tp_out[i] = tp[i];

  const int64_t total = (int64_t)ngroups * tp[B];
  const int nwg = gridDim.x;
  const int64_t Ct = max((int64_t)1, (total + nwg - 1) / nwg);
  int64_t u = (int64_t)blockIdx.x * Ct;
  const int64_t u_end = min(total, u + Ct);
  if (u >= u_end) return;
  // first sequence: the largest b with ngroups * tp[b] <= u (it has n_b > 0)
  int b_lo = 0, b_hi = B - 1;
  while (b_lo < b_hi) {
    const int mid = (b_lo + b_hi + 1) >> 1;
    if ((int64_t)ngroups * tp[mid] <= u) b_lo = mid;
    else b_hi = mid - 1;
  }
  int b = b_lo;
  float* pw = p_lds[wave];
  while (u < u_end) {
    const int nb = tp[b + 1] - tp[b];
    const int64_t base = (int64_t)ngroups * tp[b];
    const int grp = (int)((u - base) / nb);
    const int64_t i0 = (u - base) - (int64_t)grp * nb;
    const int64_t seg_end = min(u_end, base + (int64_t)(grp + 1) * nb);
    const int kh = grp * wpg + wave;
    if (kh < Hkv) {
      const int64_t Lc = min(ctx_lens[b], cap);
      const int64_t t_begin = i0 * tile;
      const int64_t t_end = min(Lc, (i0 + (seg_end - u)) * tile);
      const int64_t slot = ((int64_t)blockIdx.x + (int64_t)b * ngroups + grp) * wpg + wave;
      decode_chunk<D, G>(q, kc, vc, bt + (int64_t)b * bt_stride, ws_o, ws_ml, out, Hkv, BS, NB, tile,
                         scale_log2, b, kh, t_begin, t_end, Lc, slot * G, pw, lane);
    }
    u = seg_end;
    if (u >= base + (int64_t)ngroups * nb) {
      ++b;
      while (b < B && tp[b + 1] == tp[b]) ++b;  // sequences with no context
    }
  }
}

// Single launch (blocks_per_split -1), one workgroup per (sequence, group of
// HG kv heads): the workgroup's NW waves are HG heads x S = NW/HG
// interleaved walks, wave s of a head taking the tiles s, s + S, s + 2S, ...
// of the context, so the walks start at fixed block-table columns (their
// first block ids load alongside the context length, not after it) and all
// finish within a tile of each other.  The waves' partials (o, m, l) meet
// in LDS and the log-sum-exp merge writes the bf16 output: no tile-count
// scan, no second launch, no partial round trip through HBM.  With qo / qs
// the workgroup also writes the act_quant codes and scales of its HG*G*D
// output values, which must be whole 128-value groups (HG*G*D % 128 == 0).
// Grid: B * ngrp workgroups, the head group fastest, so a sequence's groups
// (adjacent pieces of the same token rows) are read at about the same time.
// A workgroup's throughput is bounded by its CU (about 30 GB/s measured), so
// this pays only when the grid covers every CU and no context is much
// longer than the rest can hide: the host's default takes it for B * ngrp >=
// CUs and tables of at most 8192 tokens.
//
// ROPE: the decode step's qk_norm_rope_store runs inside the same launch.
// The workgroup reads the new token's fused qkv row (q | k | v), normalises
// and rotates q and k with RopeRow (the code qk_norm_rope_store runs, so
// the same bits), writes the k and v rows of its own kv heads to the cache
// slot, and keeps its q rows and the new k and v rows in LDS.  The walks
// stop before the new token (context position L-1); the first walk of each
// head adds it from LDS before its own tiles, so nothing this launch writes
// is read back from memory.  The row's loads are issued at the start and
// the arithmetic runs after the first tile's loads (the walk's prologue
// hook), so it overlaps the first round trip.
struct RopeIn {
  const uint16_t* qkv;
  int64_t ld;
  const float* qw;
  const float* kw;
  const float* cos_sin;
  const int64_t* pos;
  const int64_t* slots;
  uint16_t* kc;
  uint16_t* vc;
  uint16_t* q_out;  // optional copy of the rotated q rows
  int64_t num_slots, max_pos;
  float eps;
};

template <int D, int G, int HG, int NW, bool ROPE, bool PAIR>
__global__ __launch_bounds__(64 * NW, PAIR ? 2 : 1) void paged_decode_pairs(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ kc, const uint16_t* __restrict__ vc,
    const int64_t* __restrict__ ctx_lens, const int32_t* __restrict__ bt, int64_t bt_stride,
    uint16_t* __restrict__ out, uint8_t* __restrict__ qo, float* __restrict__ qs, int Hkv, int BS, int64_t NB,
    int max_blocks, int tile, float scale_log2, int ngrp, int ncu, RopeIn ri) {
  using Geo = DecodeGeom<D>;
  using W = DecodeWave<D, G>;
  constexpr int S = NW / HG;
  static_assert(!PAIR || (HG == 1 && NW == 4), "the paired order runs one kv head per 4-wave workgroup");
  constexpr int E = HG * G * D;  // output values of the workgroup
  __shared__ __attribute__((aligned(16))) float p_lds[NW][Geo::T * W::GP];
  __shared__ __attribute__((aligned(16))) float part_o[NW][G * D];
  __shared__ float part_m[NW][G], part_l[NW][G];
  __shared__ __attribute__((aligned(16))) uint16_t vals[E];
  __shared__ __attribute__((aligned(16))) uint16_t new_q[ROPE ? E : 8];           // rotated q rows of the group
  __shared__ __attribute__((aligned(16))) uint16_t new_kv[ROPE ? 2 * HG * D : 8];  // new token: k rows | v rows
  __shared__ float red[8];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int hl = wave / S, s = wave - hl * S;
  const int Hq = Hkv * G;
  constexpr int CPH = D / 8;  // 16-byte chunks per head row
  RopeRow<1> rr;
  if constexpr (ROPE) {
    rr.init(Hq, Hkv, D, threadIdx.x);
    rr.load_weights(ri.qw, ri.kw);  // the same for every sequence: before the order is known
  }
  int b, grp;
  int64_t L;
  if constexpr (PAIR) {
    // Sequences ranked by context length, longest first (ties: lower index),
    // and workgroup w given unit rank r(w) so that the two workgroups a CU
    // holds at once -- w and w + ncu, the first round dealt one per CU --
    // pair a long (sequence, kv head) with a short one: ranks 0 .. ncu-P-1
    // (the longest) run alone, rank ncu-P+c shares CU c < P with rank
    // W-1-c, P = W - ncu.  A permutation of the units for any W.
    // key = (length clamped to 2^40) << 8 | (255 - index): distinct keys,
    // larger for a longer context or, at equal length, a lower index; the
    // rank of sequence i is the number of larger keys, counted by threads i
    // (keys 0..127) and i + 128 (keys 128..255) from 16-byte LDS reads
    __shared__ __attribute__((aligned(16))) uint64_t pkey[256];
    __shared__ int64_t plen[256];
    __shared__ int prank[256];
    __shared__ int porder[256];
    const int B = gridDim.x / ngrp;  // <= 256: checked on the host
    const int t = threadIdx.x;
    const int64_t lt = t < B ? ctx_lens[t] : 0;
    pkey[t] = t < B ? ((uint64_t)min(max(lt, (int64_t)0), (int64_t)1 << 40) << 8) | (uint64_t)(255 - t) : 0;
    plen[t] = lt;
    auto count = [&](int i, int half) {  // keys of half `half` larger than sequence i's
      int r = 0;
      if (i < B && 128 * half < B) {
        const uint64_t ki = pkey[i];
        const uint4* kk = reinterpret_cast<const uint4*>(pkey + 128 * half);
#pragma unroll 4
        for (int j2 = 0; j2 < 64; ++j2) {  // padding keys are 0: never larger
          const uint4 two = kk[j2];
          r += (((uint64_t)two.y << 32 | two.x) > ki) + (((uint64_t)two.w << 32 | two.z) > ki);
        }
      }
      return r;
    };
    for (int base = 0; base < B; base += 128) {  // sequences base .. base + 127
      __syncthreads();
      prank[t] = count(base + (t & 127), t >> 7);
      __syncthreads();
      if (t < 128 && base + t < B) porder[prank[t] + prank[t + 128]] = base + t;
    }
    __syncthreads();
    const int Wg = gridDim.x, w = blockIdx.x;
    const int P = max(0, min(Wg - ncu, ncu));
    const int r = w >= ncu ? Wg - 1 - (w - ncu) : (w < P ? ncu - P + w : w - P);
    b = porder[r / ngrp];
    grp = r - (r / ngrp) * ngrp;
    L = plen[b];
  } else {
    b = blockIdx.x / ngrp;
    grp = blockIdx.x - b * ngrp;
    L = ctx_lens[b];
  }
  const int kh = grp * HG + hl;
  // with ROPE the walks cover [0, L-1): the new token comes from the qkv row
  const int64_t Lc = min(ROPE ? L - 1 : L, (int64_t)max_blocks * BS);

  // the RoPE prologue's loads, all issued before the walk (the position's
  // scalar load returns with the context length's, which the walk waits for
  // anyway), so that its arithmetic in pro() waits for none of the walk's
  // loads: issued after the first tile's, they would have to return first
  const int h0 = grp * HG;  // first kv head of the workgroup
  int64_t slot = -1, p = 0;
  uint4 vnew = make_uint4(0, 0, 0, 0);
  const uint16_t* row = nullptr;
  if constexpr (ROPE) {
    row = ri.qkv + (int64_t)b * ri.ld;
    p = ri.pos[b];
    p = p < 0 ? 0 : (p >= ri.max_pos ? ri.max_pos - 1 : p);
    slot = ri.slots != nullptr ? ri.slots[b] : -1;
    rr.load(row);
    if (threadIdx.x < HG * CPH && h0 + (int)threadIdx.x / CPH < Hkv)
      vnew = *reinterpret_cast<const uint4*>(row + (int64_t)(Hq + Hkv + h0) * D + threadIdx.x * 8);
    rr.load_rope(ri.cos_sin + p * D);
  }
  bool pro_done = false;
  auto prologue = [&]() {
    if constexpr (ROPE) {
      const bool store = slot >= 0 && slot < ri.num_slots;
      if (threadIdx.x < HG * CPH && h0 + (int)threadIdx.x / CPH < Hkv) {
        *reinterpret_cast<uint4*>(&new_kv[HG * D + threadIdx.x * 8]) = vnew;
        if (store) *reinterpret_cast<uint4*>(ri.vc + (slot * Hkv + h0) * D + threadIdx.x * 8) = vnew;
      }
      rr.finish(ri.eps, red,
                [&](bool isq, int h, int d0, const uint4& o1, const uint4& o2) {
                  const int hk = isq ? h / G : h;
                  if (hk < h0 || hk >= h0 + HG) return;  // another workgroup's head
                  uint16_t* l = isq ? &new_q[(h - h0 * G) * D] : &new_kv[(hk - h0) * D];
                  *reinterpret_cast<uint4*>(l + d0) = o1;
                  *reinterpret_cast<uint4*>(l + D / 2 + d0) = o2;
                  uint16_t* g = nullptr;
                  if (isq) {
                    if (ri.q_out != nullptr) g = ri.q_out + ((int64_t)b * Hq + h) * D;
                  } else if (store) {
                    g = ri.kc + (slot * Hkv + h) * D;
                  }
                  if (g != nullptr) {
                    *reinterpret_cast<uint4*>(g + d0) = o1;
                    *reinterpret_cast<uint4*>(g + D / 2 + d0) = o2;
                  }
                });
      __syncthreads();
    }
    pro_done = true;
  };
  if (kh < Hkv) {
    W w(lane, Hkv);
    typename W::QBuf qa;
    // the new token as a tile of one row, on the first walk of its head
    auto new_token = [&]() {
      typename W::KBuf ka;
      typename W::VBuf va;
      w.row_tile(ka, va, &new_kv[hl * D], &new_kv[(HG + hl) * D]);
      w.tile(ka, va, qa, 1, scale_log2, p_lds[wave]);
    };
    auto pro = [&]() {
      prologue();
      if constexpr (ROPE) {
        w.load_q_lds(qa, &new_q[hl * G * D]);
        // while the walk's first tile is still in flight; the paired form
        // adds it after the walk, where the walk's buffers are free
        if (!PAIR && s == 0 && L >= 1) new_token();
      }
    };
    if (!ROPE) w.load_q(qa, q, b, kh, Hq);
    // the paired form (two workgroups per CU, 256 registers a wave) runs the
    // prologue before its walk: run inside the walk, its registers would be
    // live across the walk's loop and spill
    if constexpr (PAIR) pro();
    if (Lc > (int64_t)s * tile) {
      if constexpr (PAIR)
        decode_walk<D, G>(w, qa, kc, vc, bt + (int64_t)b * bt_stride, BS, NB, tile, scale_log2, kh,
                          (int64_t)s * tile, Lc, S, max_blocks, p_lds[wave]);
      else
        decode_walk<D, G>(w, qa, kc, vc, bt + (int64_t)b * bt_stride, BS, NB, tile, scale_log2, kh,
                          (int64_t)s * tile, Lc, S, max_blocks, p_lds[wave], pro);
    }
    if (!pro_done) pro();
    if constexpr (ROPE && PAIR) {
      if (s == 0 && L >= 1) new_token();
    }
    w.reduce_lanes();
    if (w.ts == 0) {
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float* dst = &part_o[wave][g * D + w.dc * 8];
        *reinterpret_cast<float4*>(dst) = make_float4(w.acc[g][0], w.acc[g][1], w.acc[g][2], w.acc[g][3]);
        *reinterpret_cast<float4*>(dst + 4) = make_float4(w.acc[g][4], w.acc[g][5], w.acc[g][6], w.acc[g][7]);
      }
    }
    if (lane < G) {
      part_m[wave][lane] = w.m_run;
      part_l[wave][lane] = w.l_run;
    }
  } else {
    prologue();  // a wave without a head still takes the prologue's barriers
  }
  __syncthreads();
  // log-sum-exp merge of the S walks of each head (L = 0: zeros)
  for (int e = threadIdx.x; e < E; e += blockDim.x) {
    const int h2 = e / (G * D), r = e - h2 * (G * D), g = r / D;
    if (grp * HG + h2 >= Hkv) continue;
    const int w0 = h2 * S;
    float M = -INFINITY;
#pragma unroll
    for (int t = 0; t < S; ++t) M = fmaxf(M, part_m[w0 + t][g]);
    float num = 0.f, den = 0.f;
    if (M != -INFINITY) {
#pragma unroll
      for (int t = 0; t < S; ++t) {
        const float wt = exp2f(part_m[w0 + t][g] - M);
        den = fmaf(wt, part_l[w0 + t][g], den);
        num = fmaf(wt, part_o[w0 + t][r], num);
      }
    }
    const uint16_t v = (uint16_t)f32_to_bf16(den > 0.f ? num / den : 0.f);
    out[((int64_t)b * Hq + (int64_t)(grp * HG + h2) * G) * D + r] = v;
    vals[e] = v;
  }
  if (qo == nullptr) return;
  __syncthreads();
  // act_quant of the workgroup's E / 128 groups, 16 lanes x 8 values each
  const int t = threadIdx.x;
  if (t < E / 8) {
    float f[8];
    unpack8(*reinterpret_cast<const uint4*>(&vals[t * 8]), f);
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(f[i]));
    amax = group_max<16>(amax);
    const float sc = scale_from_amax(amax, false);
    const int64_t e0 = (int64_t)b * Hq * D + (int64_t)grp * E;  // first output value of the workgroup
    *reinterpret_cast<uint2*>(qo + e0 + t * 8) = quant8(f, sc);
    if ((t & 15) == 0) qs[e0 / 128 + t / 16] = sc;
  }
}

// ------------------------------------------------------------ decode merge --
// Where the partials of (sequence b, query head h) live: ns of them, the
// s-th at workspace row r0 + s * rstep (o at ws_o[row * D], (m, l) at
// ws_ml[row * 2]).  ns == 1: the split kernel wrote the output itself;
// ns == 0: no context.
struct PartMap {
  int bps, max_splits;  // fixed chunks of bps blocks (bps > 0)
  const int* tp;        // balanced split (bps == 0): tile-count scan, B + 1 ints
  int tile, ngroups, wpg, G, nwg, B;
};

__device__ __forceinline__ int part_span(const PartMap& pm, int b, int h, int Hq, int64_t Lc, int BS,
                                         int64_t& r0, int64_t& rstep) {
  if (pm.bps > 0) {
    const int64_t chunk = (int64_t)pm.bps * BS;
    r0 = (int64_t)b * pm.max_splits * Hq + h;
    rstep = Hq;
    return Lc > 0 ? (int)((Lc + chunk - 1) / chunk) : 0;
  }
  r0 = 0;
  rstep = (int64_t)pm.wpg * pm.G;
  const int nb = pm.tp[b + 1] - pm.tp[b];
  if (nb == 0) return 0;
  const int kh = h / pm.G, g = h - kh * pm.G;
  const int grp = kh / pm.wpg, wv = kh - grp * pm.wpg;
  const int64_t total = (int64_t)pm.ngroups * pm.tp[pm.B];
  const int64_t Ct = max((int64_t)1, (total + pm.nwg - 1) / pm.nwg);
  const int64_t start = (int64_t)pm.ngroups * pm.tp[b] + (int64_t)grp * nb;
  const int64_t wf = start / Ct, wl = (start + nb - 1) / Ct;
  r0 = ((wf + (int64_t)b * pm.ngroups + grp) * pm.wpg + wv) * pm.G + g;
  return (int)(wl - wf + 1);
}

// Log-sum-exp merge of one output element: partials s = 0 .. ns-1 of a
// (sequence, head) at workspace rows r0 + s*rs, element d.  Up to MERGE_NS
// partials are loaded together (one memory round trip), more in a loop with
// the same arithmetic in the same order.  ns == 0 (no context) gives 0.
constexpr int MERGE_NS = 16;
__device__ __forceinline__ float merge_element(const float* __restrict__ ws_o, const float* __restrict__ ws_ml,
                                               int64_t r0, int64_t rs, int ns, int D, int d) {
  float res = 0.f;
  if (ns > 1 && ns <= MERGE_NS) {
    float mv[MERGE_NS], lv[MERGE_NS], ov[MERGE_NS];
#pragma unroll
    for (int s = 0; s < MERGE_NS; ++s) {
      const int64_t r = r0 + (s < ns ? s : 0) * rs;
      mv[s] = ws_ml[r * 2];
      lv[s] = ws_ml[r * 2 + 1];
      ov[s] = ws_o[r * D + d];
    }
    float M = -INFINITY;
#pragma unroll
    for (int s = 0; s < MERGE_NS; ++s)
      if (s < ns) M = fmaxf(M, mv[s]);
    float num = 0.f, den = 0.f;
    if (M != -INFINITY) {
#pragma unroll
      for (int s = 0; s < MERGE_NS; ++s)
        if (s < ns) {
          const float w = exp2f(mv[s] - M);
          den = fmaf(w, lv[s], den);
          num = fmaf(w, ov[s], num);
        }
    }
    res = den > 0.f ? num / den : 0.f;
  } else if (ns > 1) {
    float M = -INFINITY;
    for (int s = 0; s < ns; ++s) M = fmaxf(M, ws_ml[(r0 + s * rs) * 2]);
    float num = 0.f, den = 0.f;
    if (M != -INFINITY) {
      for (int s = 0; s < ns; ++s) {
        const int64_t r = r0 + s * rs;
        const float w = exp2f(ws_ml[r * 2] - M);
        den = fmaf(w, ws_ml[r * 2 + 1], den);
        num = fmaf(w, ws_o[r * D + d], num);
      }
    }
    res = den > 0.f ? num / den : 0.f;
  }
  return res;
}

// One thread per output element: workgroup (x, b) merges elements
// x*256 .. x*256+255 of sequence b's Hq*D outputs (whole heads for D = 64 /
// 128).  256-thread workgroups, one per CU at the cfg3 shapes: the same
// arithmetic as one 64 / 128-thread workgroup per (head, sequence), bit for
// bit, and 0.1-0.2 us (cfg3) to 2 us (cfg4) less kernel time -- fewer
// workgroups to dispatch; the two dependent round trips (lengths and scan,
// then the partials) remain.
constexpr int MERGE_THREADS = 256;
__global__ __launch_bounds__(MERGE_THREADS) void paged_decode_merge(
    const float* __restrict__ ws_o, const float* __restrict__ ws_ml,
    const int64_t* __restrict__ ctx_lens, uint16_t* __restrict__ out, int Hq, int D, int BS,
    int max_blocks, PartMap pm) {
  const int b = blockIdx.y;
  const int e = blockIdx.x * MERGE_THREADS + threadIdx.x;
  if (e >= Hq * D) return;
  const int h = e / D, d = e - h * D;
  const int64_t Lc = min(ctx_lens[b], (int64_t)max_blocks * BS);
  int64_t r0, rs;
  const int ns = part_span(pm, b, h, Hq, Lc, BS, r0, rs);
  if (ns == 1) return;
  out[(int64_t)b * Hq * D + e] = (uint16_t)f32_to_bf16(merge_element(ws_o, ws_ml, r0, rs, ns, D, d));
}

// The merge fused with the act_quant of its output row (the output
// projection's FP8 input): one 128-thread workgroup per (128-value act_quant
// group, sequence), every group independent.  Each thread merges one element
// of the group (the arithmetic of paged_decode_merge; ns == 1: the split
// kernel wrote the value), then 16 lanes quantise the group's 128 bf16
// values 8 each, as act_quant does: codes and scale bit-identical to
// act_quant(out row, 128).  Needs Hq * D % 128 == 0.
__global__ __launch_bounds__(128) void paged_decode_merge_quant_group(
    const float* __restrict__ ws_o, const float* __restrict__ ws_ml, const int64_t* __restrict__ ctx_lens,
    uint16_t* __restrict__ out, uint8_t* __restrict__ qo, float* __restrict__ qs, int Hq, int D, int BS,
    int max_blocks, PartMap pm) {
  __shared__ __attribute__((aligned(16))) uint16_t vals[128];
  const int g = blockIdx.x, b = blockIdx.y, t = threadIdx.x;
  const int E = Hq * D;
  const int e = g * 128 + t;
  const int h = e / D, d = e - h * D;
  const int64_t Lc = min(ctx_lens[b], (int64_t)max_blocks * BS);
  int64_t r0, rs;
  const int ns = part_span(pm, b, h, Hq, Lc, BS, r0, rs);
  uint16_t* orow = out + (int64_t)b * E;
  uint16_t v;
  if (ns == 1) {
    v = orow[e];  // written by the split kernel
  } else {
    v = (uint16_t)f32_to_bf16(merge_element(ws_o, ws_ml, r0, rs, ns, D, d));
    orow[e] = v;
  }
  vals[t] = v;
  __syncthreads();
  if (t < 16) {
    float f[8];
    unpack8(*reinterpret_cast<const uint4*>(&vals[t * 8]), f);
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(f[i]));
    amax = group_max<16>(amax);
    const float sc = scale_from_amax(amax, false);
    *reinterpret_cast<uint2*>(qo + (int64_t)b * E + g * 128 + t * 8) = quant8(f, sc);
    if (t == 0) qs[(int64_t)b * (E / 128) + g] = sc;
  }
}

template <int D, int G>
void launch_split(dim3 grid, dim3 block, hipStream_t st, const uint16_t* q, const uint16_t* kc,
                  const uint16_t* vc, const int64_t* cl, const int32_t* bt, int64_t bts, float* wo,
                  float* wml, uint16_t* out, int Hkv, int BS, int64_t NB, int max_blocks, int bps,
                  int tile, float sl2, int max_splits) {
  // grid = (sequence, split, kv-head group) on input; launched with the
  // group folded into x, fastest
  const int nz = (int)grid.z;
  hipLaunchKernelGGL((paged_decode_split<D, G>), dim3(grid.x * grid.z, grid.y, 1), block, 0, st, q, kc, vc, cl,
                     bt, bts, wo, wml, out, Hkv, BS, NB, max_blocks, bps, tile, sl2, max_splits, nz);
}

template <int D, int G>
void launch_balanced(unsigned nwg, dim3 block, hipStream_t st, const uint16_t* q, const uint16_t* kc,
                     const uint16_t* vc, const int64_t* cl, const int32_t* bt, int64_t bts, float* wo,
                     float* wml, int* tp, uint16_t* out, int Hkv, int BS, int64_t NB, int max_blocks, int B,
                     int tile, float sl2, int ngroups) {
  hipLaunchKernelGGL((paged_decode_balanced<D, G>), dim3(nwg), block, 0, st, q, kc, vc, cl, bt, bts, wo, wml,
                     tp, out, Hkv, BS, NB, max_blocks, B, tile, sl2, ngroups);
}

template <int D>
bool dispatch_balanced(int G, unsigned nwg, dim3 block, hipStream_t st, const uint16_t* q,
                       const uint16_t* kc, const uint16_t* vc, const int64_t* cl, const int32_t* bt,
                       int64_t bts, float* wo, float* wml, int* tp, uint16_t* out, int Hkv, int BS,
                       int64_t NB, int max_blocks, int B, int tile, float sl2, int ngroups) {
#define LFS_G(GG) \
  case GG: launch_balanced<D, GG>(nwg, block, st, q, kc, vc, cl, bt, bts, wo, wml, tp, out, Hkv, BS, NB, max_blocks, B, tile, sl2, ngroups); return true;
  switch (G) {
    LFS_G(1) LFS_G(2) LFS_G(3) LFS_G(4) LFS_G(5) LFS_G(6) LFS_G(7) LFS_G(8)
    default: return false;
  }
#undef LFS_G
}

int decode_cu_count();
// the paired order ranks the sequences with one context length per thread
constexpr int kPairMaxB = 256;
// longest table (tokens) lfs_paged_decode_rope takes the paired order for:
// a workgroup walks a whole (sequence, kv head), so the longest context
// bounds the call
constexpr int64_t kPairMaxContext = 8192;

template <int D, int HG, int NW, bool ROPE, bool PAIR = false>
bool dispatch_pairs_hg(int G, unsigned nwg, hipStream_t st, const uint16_t* q, const uint16_t* kc,
                       const uint16_t* vc, const int64_t* cl, const int32_t* bt, int64_t bts, uint16_t* out,
                       uint8_t* qo, float* qs, int Hkv, int BS, int64_t NB, int max_blocks, int tile, float sl2,
                       int ngrp, const RopeIn& ri) {
  const int ncu = decode_cu_count();
#define LFS_G(GG)                                                                                               \
  case GG:                                                                                                      \
    hipLaunchKernelGGL((paged_decode_pairs<D, GG, HG, NW, ROPE, PAIR>), dim3(nwg), dim3(64 * NW), 0, st, q, kc, \
                       vc, cl, bt, bts, out, qo, qs, Hkv, BS, NB, max_blocks, tile, sl2, ngrp, ncu, ri);        \
    return true;
  switch (G) {
    LFS_G(1) LFS_G(2) LFS_G(3) LFS_G(4) LFS_G(5) LFS_G(6) LFS_G(7) LFS_G(8)
    default: return false;
  }
#undef LFS_G
}

template <int D, bool ROPE>
bool dispatch_pairs(int HG, int G, unsigned nwg, hipStream_t st, const uint16_t* q, const uint16_t* kc,
                    const uint16_t* vc, const int64_t* cl, const int32_t* bt, int64_t bts, uint16_t* out,
                    uint8_t* qo, float* qs, int Hkv, int BS, int64_t NB, int max_blocks, int tile, float sl2,
                    int ngrp, const RopeIn& ri, bool pair = false) {
  // paired order: one kv head per 4-wave workgroup, two workgroups per CU
  if (pair)
    return dispatch_pairs_hg<D, 1, 4, ROPE, true>(G, nwg, st, q, kc, vc, cl, bt, bts, out, qo, qs, Hkv, BS, NB,
                                                  max_blocks, tile, sl2, ngrp, ri);
  // the RoPE prologue runs on 4 waves per workgroup (one per SIMD, so up to
  // 512 registers a wave): with 8 its registers and the walk's do not fit in
  // 256 and spill inside the tile loop
  constexpr int NW = ROPE ? 4 : 8;
  return HG == 1 ? dispatch_pairs_hg<D, 1, NW, ROPE>(G, nwg, st, q, kc, vc, cl, bt, bts, out, qo, qs, Hkv, BS,
                                                      NB, max_blocks, tile, sl2, ngrp, ri)
                 : dispatch_pairs_hg<D, 2, NW, ROPE>(G, nwg, st, q, kc, vc, cl, bt, bts, out, qo, qs, Hkv, BS,
                                                      NB, max_blocks, tile, sl2, ngrp, ri);
}

// kv heads per workgroup of the single-launch decode: two when Hkv is even
// (a workgroup then reads 2*D*2 of each token row's Hkv*D*2 bytes: at the
// cfg5 attention shape 46.1 us against 48.9 us with one head per
// workgroup), else one.  The fused act_quant needs HG*G*D % 128 == 0.
int pairs_heads_per_group(int Hkv) { return Hkv % 2 == 0 ? 2 : 1; }

// compute units of the current device (the balanced split's grid)
int decode_cu_count() {
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

// balanced split geometry: wpg waves (kv heads) per workgroup, ngroups
// groups, nwg workgroups -- one 4-wave workgroup per CU, one round.  Fewer,
// longer streams beat filling the kernel's occupancy (two waves per SIMD):
// measured at 1 / 2 / 3 / 4 / 8 workgroups per CU, cfg3 44.3 / 49.4 / 56.6 /
// 56.0 / 66.2 us, cfg4 1169 / 1190 / 1202 / 1212 / 1257 us (fewer tile
// pipelines to ramp up, fewer partials, fewer concurrent DRAM streams).
struct BalancedGeom {
  int wpg, ngroups, nwg;
};
BalancedGeom balanced_geom(int Hkv) {
  BalancedGeom g;
  g.wpg = Hkv < 4 ? Hkv : 4;
  g.ngroups = (Hkv + g.wpg - 1) / g.wpg;
  g.nwg = decode_cu_count() * (4 / g.wpg);
  return g;
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

namespace {
int paged_decode_merge_launch(float* ws_o, float* ws_ml, const int64_t* context_lens, void* out, void* q_out,
                              float* q_scale, int64_t B, int Hq, int D, int BS, int max_blocks, const PartMap& pm,
                              hipStream_t st);
}

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
  if (B < 0 || num_q_heads <= 0 || head_dim <= 0 || max_blocks < 0 || blocks_per_split < -2) return -1;
  if (blocks_per_split < 0) return 0;  // single launch: the partials stay in LDS
  if (blocks_per_split == 0) {
    // balanced split: partial rows (nwg + B*ngroups)*wpg*G <= (8*CUs + 2*B)*Hq
    // (wpg*G <= Hq, nwg*wpg <= 4*CUs, ngroups*wpg < 2*Hkv), then B+1 ints
    const int64_t rows = (8 * (int64_t)decode_cu_count() + 2 * B) * num_q_heads;
    return 4 * rows * ((int64_t)head_dim + 2) + 4 * (B + 1);
  }
  const int64_t splits = ((int64_t)max_blocks + blocks_per_split - 1) / blocks_per_split;
  return 4 * B * splits * (int64_t)num_q_heads * ((int64_t)head_dim + 2);
}

namespace {
// Argument checks, then the split (balanced or fixed chunks) and the merge.
// `noalloc` only changes the wording of the workspace error.
int paged_decode_impl(const void* q, const void* k_cache, const void* v_cache, const int64_t* context_lens,
                      const int32_t* block_tables, int64_t bt_stride, void* out, void* workspace,
                      int64_t workspace_bytes, int64_t B, int32_t num_q_heads, int32_t num_kv_heads,
                      int32_t head_dim, int32_t block_size, int64_t num_blocks, int32_t max_blocks, float scale,
                      int32_t blocks_per_split, void* q_out, float* q_scale, void* stream, bool noalloc) {
  const int Hq = num_q_heads, Hkv = num_kv_heads, D = head_dim, BS = block_size;
  LFS_REQUIRE(B >= 0 && Hq > 0 && Hkv > 0 && BS > 0 && num_blocks >= 0 && max_blocks >= 0,
              "paged_decode: bad shape");
  LFS_REQUIRE(D == 64 || D == 128, "paged_decode: head_dim must be 64 or 128 (got %d)", D);
  LFS_REQUIRE(Hq % Hkv == 0 && Hq / Hkv <= 8,
              "paged_decode: num_q_heads (%d) must be a multiple of num_kv_heads (%d), ratio <= 8", Hq, Hkv);
  LFS_REQUIRE(BS % 16 == 0, "paged_decode: block_size must be a multiple of 16 (got %d)", BS);
  LFS_REQUIRE(blocks_per_split >= -2,
              "paged_decode: blocks_per_split must be >= -2 (-1: single launch, -2: single launch in the "
              "paired order, 0: balanced split)");
  LFS_REQUIRE(blocks_per_split > 0 || B <= BAL_MAXB, "paged_decode: the balanced split (blocks_per_split 0) needs B <= %d",
              BAL_MAXB);
  LFS_REQUIRE(bt_stride >= max_blocks, "paged_decode: block table stride < max_blocks");
  LFS_REQUIRE(num_blocks >= 1 || max_blocks == 0, "paged_decode: empty KV pool");
  if (B == 0) return 0;
  LFS_REQUIRE(q && k_cache && v_cache && context_lens && out, "paged_decode: null pointer");
  LFS_REQUIRE(max_blocks == 0 || block_tables, "paged_decode: null block table");
  LFS_REQUIRE(((((uintptr_t)q) | ((uintptr_t)k_cache) | ((uintptr_t)v_cache) | ((uintptr_t)out)) & 15u) == 0,
              "paged_decode: q, caches and out must be 16-byte aligned");
  LFS_REQUIRE(B < 65536, "paged_decode: batch too large");
  LFS_REQUIRE((q_out == nullptr) == (q_scale == nullptr), "paged_decode: q_out and q_scale go together");
  LFS_REQUIRE(q_out == nullptr || Hq * D % 128 == 0, "paged_decode: the quantised output needs Hq*D %% 128 == 0");
  const int64_t need = lfs_paged_decode_workspace_bytes(B, Hq, D, max_blocks, blocks_per_split);
  LFS_REQUIRE(!noalloc || need <= workspace_bytes,
              "paged_decode_noalloc: this shape needs %lld bytes of workspace, more than the library's "
              "static scratch of %lld bytes (call lfs_paged_decode with a caller-owned workspace)",
              (long long)need, (long long)workspace_bytes);
  LFS_REQUIRE(workspace_bytes >= need && (need == 0 || workspace),
              "paged_decode: workspace of %lld bytes < required %lld", (long long)workspace_bytes,
              (long long)need);
  hipStream_t st = (hipStream_t)stream;
  const int Tmax = D == 64 ? 64 : 32;
  int tile = 16;
  for (int t = Tmax; t >= 16; t >>= 1)
    if (BS % t == 0) { tile = t; break; }
  const float sl2 = scale * 1.4426950408889634f;
  const int G = Hq / Hkv;
  if (blocks_per_split < 0) {
    const bool pair = blocks_per_split == -2;
    const int HG = pair ? 1 : pairs_heads_per_group(Hkv);
    LFS_REQUIRE(q_out == nullptr || (HG * G * D) % 128 == 0,
                "paged_decode: the single launch (blocks_per_split %d) cannot quantise this output "
                "(Hkv = %d, G*D = %d: needs %s)", blocks_per_split, Hkv, G * D,
                pair ? "G*D a multiple of 128" : "an even Hkv or G*D a multiple of 128");
    LFS_REQUIRE(!pair || B <= kPairMaxB, "paged_decode: the paired order (blocks_per_split -2) needs B <= %d",
                kPairMaxB);
    const int ngrp = (Hkv + HG - 1) / HG;
    LFS_REQUIRE(B * ngrp < (1ll << 31), "paged_decode: too many (sequence, kv head) workgroups");
    const RopeIn none{};
    const bool ok = D == 64
        ? dispatch_pairs<64, false>(HG, G, (unsigned)(B * ngrp), st, (const uint16_t*)q, (const uint16_t*)k_cache,
                                    (const uint16_t*)v_cache, context_lens, block_tables, bt_stride,
                                    (uint16_t*)out, (uint8_t*)q_out, q_scale, Hkv, BS, num_blocks, max_blocks,
                                    tile, sl2, ngrp, none, pair)
        : dispatch_pairs<128, false>(HG, G, (unsigned)(B * ngrp), st, (const uint16_t*)q,
                                     (const uint16_t*)k_cache, (const uint16_t*)v_cache, context_lens,
                                     block_tables, bt_stride, (uint16_t*)out, (uint8_t*)q_out, q_scale, Hkv, BS,
                                     num_blocks, max_blocks, tile, sl2, ngrp, none, pair);
    LFS_REQUIRE(ok, "paged_decode: unsupported group size %d", G);
    return check_launch("paged_decode(single launch)");
  }
  PartMap pm{};
  if (blocks_per_split == 0) {
    const BalancedGeom bg = balanced_geom(Hkv);
    const int64_t rows = ((int64_t)bg.nwg + B * bg.ngroups) * bg.wpg * G;
    LFS_REQUIRE((int64_t)bg.ngroups * B * (((int64_t)max_blocks * BS + tile - 1) / tile) < (1ll << 31),
                "paged_decode: too many context tiles for the balanced split");
    float* ws_o = (float*)workspace;
    float* ws_ml = ws_o + rows * D;
    int* tp = (int*)(ws_ml + rows * 2);
    pm = PartMap{0, 0, tp, tile, bg.ngroups, bg.wpg, G, bg.nwg, (int)B};
    {  // launched also when max_blocks == 0: it then writes the all-zero scan the merge reads
      const bool ok = D == 64
          ? dispatch_balanced<64>(G, (unsigned)bg.nwg, dim3(64 * bg.wpg), st, (const uint16_t*)q,
                                  (const uint16_t*)k_cache, (const uint16_t*)v_cache, context_lens, block_tables,
                                  bt_stride, ws_o, ws_ml, tp, (uint16_t*)out, Hkv, BS, num_blocks, max_blocks,
                                  (int)B, tile, sl2, bg.ngroups)
          : dispatch_balanced<128>(G, (unsigned)bg.nwg, dim3(64 * bg.wpg), st, (const uint16_t*)q,
                                   (const uint16_t*)k_cache, (const uint16_t*)v_cache, context_lens,
                                   block_tables, bt_stride, ws_o, ws_ml, tp, (uint16_t*)out, Hkv, BS,
                                   num_blocks, max_blocks, (int)B, tile, sl2, bg.ngroups);
      LFS_REQUIRE(ok, "paged_decode: unsupported group size %d", G);
      const int rc = check_launch("paged_decode(balanced split)");
      if (rc) return rc;
    }
    return paged_decode_merge_launch(ws_o, ws_ml, context_lens, out, q_out, q_scale, B, Hq, D, BS, max_blocks, pm, st);
  }
  const int max_splits = (max_blocks + blocks_per_split - 1) / blocks_per_split;
  float* ws_o = (float*)workspace;
  float* ws_ml = ws_o + (size_t)B * max_splits * Hq * D;
  pm = PartMap{blocks_per_split, max_splits, nullptr, tile, 0, 0, G, 0, (int)B};
  if (max_splits > 0) {
    const int wpg = Hkv < 4 ? Hkv : 4;  // waves (kv heads) per workgroup
    const dim3 grid((unsigned)B, (unsigned)max_splits, (unsigned)((Hkv + wpg - 1) / wpg));
    LFS_REQUIRE(grid.z < 65536u && grid.y < 65536u && (int64_t)grid.x * grid.z < (1ll << 31),
                "paged_decode: too many kv heads or splits");
    const dim3 block((unsigned)(64 * wpg));
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
  return paged_decode_merge_launch(ws_o, ws_ml, context_lens, out, q_out, q_scale, B, Hq, D, BS, max_blocks, pm, st);
}

// Workspace of lfs_paged_decode_noalloc: one array per GPU, allocated when the
// code object is loaded on that GPU and held until the process ends.  Host
// code never passes `scratch` itself to a kernel (in host code the name is a
// stand-in, not a device address); it passes the address hipGetSymbolAddress
// returns for the current device, looked up once per device.
constexpr int64_t kDecodeScratchBytes = LFS_DECODE_SCRATCH_BYTES;
static __device__ __align__(256) uint8_t scratch[kDecodeScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// device address of the current device's scratch array (nullptr + message on failure)
void* device_scratch() {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    set_error("paged_decode_noalloc: no current device (%s)", hipGetErrorString(e));
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      set_error("paged_decode_noalloc: hipGetSymbolAddress(scratch) on device %d failed: %s", dev,
                hipGetErrorString(e));
      return nullptr;
    }
    g_scratch_ptr[dev] = p;
  }
  return g_scratch_ptr[dev];
}
}  // namespace

extern "C" int lfs_paged_decode(const void* q, const void* k_cache, const void* v_cache,
                                const int64_t* context_lens, const int32_t* block_tables,
                                int64_t bt_stride, void* out, void* workspace,
                                int64_t workspace_bytes, int64_t B, int32_t num_q_heads,
                                int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                                int64_t num_blocks, int32_t max_blocks, float scale,
                                int32_t blocks_per_split, void* q_out, float* q_scale, void* stream) {
  return paged_decode_impl(q, k_cache, v_cache, context_lens, block_tables, bt_stride, out, workspace,
                           workspace_bytes, B, num_q_heads, num_kv_heads, head_dim, block_size, num_blocks,
                           max_blocks, scale, blocks_per_split, q_out, q_scale, stream, false);
}

extern "C" int lfs_paged_decode_noalloc(const void* q, const void* k_cache, const void* v_cache,
                                        const int64_t* context_lens, const int32_t* block_tables,
                                        int64_t bt_stride, void* out, int64_t B, int32_t num_q_heads,
                                        int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                                        int64_t num_blocks, int32_t max_blocks, float scale,
                                        int32_t blocks_per_split, void* q_out, float* q_scale, void* stream) {
  // the kernels fully rewrite the part of the workspace they read (tile scan,
  // partial rows): nothing in it has to start at zero
  void* ws = device_scratch();
  if (ws == nullptr) return LFS_EINVAL;
  return paged_decode_impl(q, k_cache, v_cache, context_lens, block_tables, bt_stride, out, ws,
                           kDecodeScratchBytes, B, num_q_heads, num_kv_heads, head_dim, block_size, num_blocks,
                           max_blocks, scale, blocks_per_split, q_out, q_scale, stream, true);
}

extern "C" int lfs_paged_decode_rope(const void* qkv, int64_t ld, const float* q_weight, const float* k_weight,
                                     const float* cos_sin, int64_t max_positions, const int64_t* positions,
                                     const int64_t* slot_mapping, float eps, void* q_rot, void* k_cache,
                                     void* v_cache, const int64_t* context_lens, const int32_t* block_tables,
                                     int64_t bt_stride, void* out, int64_t B, int32_t num_q_heads,
                                     int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                                     int64_t num_blocks, int32_t max_blocks, float scale, void* q_out,
                                     float* q_scale, void* stream) {
  const int Hq = num_q_heads, Hkv = num_kv_heads, D = head_dim, BS = block_size;
  LFS_REQUIRE(B >= 0 && Hq > 0 && Hkv > 0 && BS > 0 && num_blocks >= 0 && max_blocks >= 0,
              "paged_decode_rope: bad shape");
  LFS_REQUIRE(D == 64 || D == 128, "paged_decode_rope: head_dim must be 64 or 128 (got %d)", D);
  LFS_REQUIRE(Hq % Hkv == 0 && Hq / Hkv <= 8,
              "paged_decode_rope: num_q_heads (%d) must be a multiple of num_kv_heads (%d), ratio <= 8", Hq, Hkv);
  LFS_REQUIRE(BS % 16 == 0, "paged_decode_rope: block_size must be a multiple of 16 (got %d)", BS);
  LFS_REQUIRE((Hq + Hkv) * D / 16 <= 256, "paged_decode_rope: (Hq+Hkv)*D/16 must be <= 256 (got %d)",
              (Hq + Hkv) * D / 16);
  LFS_REQUIRE(ld >= (int64_t)(Hq + 2 * Hkv) * D && ld % 8 == 0, "paged_decode_rope: bad qkv row stride");
  LFS_REQUIRE(max_positions > 0, "paged_decode_rope: empty RoPE table");
  LFS_REQUIRE(bt_stride >= max_blocks, "paged_decode_rope: block table stride < max_blocks");
  LFS_REQUIRE(num_blocks >= 1 || max_blocks == 0, "paged_decode_rope: empty KV pool");
  LFS_REQUIRE(B < 65536, "paged_decode_rope: batch too large");
  if (B == 0) return 0;
  LFS_REQUIRE(qkv && q_weight && k_weight && cos_sin && positions && k_cache && v_cache && context_lens && out,
              "paged_decode_rope: null pointer");
  LFS_REQUIRE(max_blocks == 0 || block_tables, "paged_decode_rope: null block table");
  LFS_REQUIRE(((((uintptr_t)qkv) | ((uintptr_t)q_weight) | ((uintptr_t)k_weight) | ((uintptr_t)cos_sin) |
                ((uintptr_t)q_rot) | ((uintptr_t)k_cache) | ((uintptr_t)v_cache) | ((uintptr_t)out)) & 15u) == 0,
              "paged_decode_rope: qkv, weights, cos_sin, q_rot, caches and out must be 16-byte aligned");
  LFS_REQUIRE((q_out == nullptr) == (q_scale == nullptr), "paged_decode_rope: q_out and q_scale go together");
  const int G = Hq / Hkv;
  // Without the quantised output, the paired order (one kv head per 4-wave
  // workgroup, a long and a short one per CU) when the B*Hkv workgroups fill
  // between one and two per CU
  const int64_t units = B * (int64_t)Hkv, ncu = decode_cu_count();
  const bool pair = q_out == nullptr && B <= kPairMaxB && units > ncu && units <= 2 * ncu &&
                    (int64_t)max_blocks * BS <= kPairMaxContext;
  const int HG = pair ? 1 : pairs_heads_per_group(Hkv);
  LFS_REQUIRE(q_out == nullptr || (HG * G * D) % 128 == 0,
              "paged_decode_rope: cannot quantise this output (Hkv = %d, G*D = %d: needs an even Hkv or G*D "
              "a multiple of 128)", Hkv, G * D);
  const int ngrp = (Hkv + HG - 1) / HG;
  const int Tmax = D == 64 ? 64 : 32;
  int tile = 16;
  for (int t = Tmax; t >= 16; t >>= 1)
    if (BS % t == 0) { tile = t; break; }
  const RopeIn ri{(const uint16_t*)qkv, ld, q_weight, k_weight, cos_sin, positions, slot_mapping,
                  (uint16_t*)k_cache, (uint16_t*)v_cache, (uint16_t*)q_rot, num_blocks * BS, max_positions, eps};
  const float sl2 = scale * 1.4426950408889634f;
  hipStream_t st = (hipStream_t)stream;
  const bool ok = D == 64
      ? dispatch_pairs<64, true>(HG, G, (unsigned)(B * ngrp), st, nullptr, (const uint16_t*)k_cache,
                                 (const uint16_t*)v_cache, context_lens, block_tables, bt_stride, (uint16_t*)out,
                                 (uint8_t*)q_out, q_scale, Hkv, BS, num_blocks, max_blocks, tile, sl2, ngrp, ri,
                                 pair)
      : dispatch_pairs<128, true>(HG, G, (unsigned)(B * ngrp), st, nullptr, (const uint16_t*)k_cache,
                                  (const uint16_t*)v_cache, context_lens, block_tables, bt_stride, (uint16_t*)out,
                                  (uint8_t*)q_out, q_scale, Hkv, BS, num_blocks, max_blocks, tile, sl2, ngrp, ri,
                                  pair);
  LFS_REQUIRE(ok, "paged_decode_rope: unsupported group size %d", G);
  return check_launch("paged_decode_rope");
}

namespace {
int paged_decode_merge_launch(float* ws_o, float* ws_ml, const int64_t* context_lens, void* out, void* q_out,
                              float* q_scale, int64_t B, int Hq, int D, int BS, int max_blocks, const PartMap& pm,
                              hipStream_t st) {
  if (q_out != nullptr) {
    hipLaunchKernelGGL(paged_decode_merge_quant_group, dim3((unsigned)(Hq * D / 128), (unsigned)B), dim3(128), 0, st,
                       ws_o, ws_ml, context_lens, (uint16_t*)out, (uint8_t*)q_out, q_scale, Hq, D, BS, max_blocks, pm);
    return check_launch("paged_decode(merge + quant)");
  }
  hipLaunchKernelGGL(paged_decode_merge, dim3((unsigned)((Hq * D + MERGE_THREADS - 1) / MERGE_THREADS), (unsigned)B),
                     dim3(MERGE_THREADS), 0, st, ws_o, ws_ml, context_lens, (uint16_t*)out, Hq, D, BS, max_blocks, pm);
  return check_launch("paged_decode(merge)");
}
}  // namespace
