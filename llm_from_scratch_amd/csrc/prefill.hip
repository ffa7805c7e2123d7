// Varlen causal prefill attention for gfx950 (the prefill half of the
// engine step).
//
// Sequence i of the batch has lq = cu_q[i+1] - cu_q[i] new query tokens
// (rows cu_q[i] .. of q) at positions lk - lq .. lk - 1 of its context of
// lk = cu_k[i+1] - cu_k[i] keys; query token p attends to keys 0 .. p
// (causal, aligned to the end of the context, as with a cached prefix).
// Key t of sequence i is row cu_k[i] + t of k / v (contiguous mode) or slot
// block_table[i][t / BS] * BS + t % BS of the KV pool (paged mode, a
// prefix-cache hit: the cached blocks and the just-stored new tokens).
//
// One workgroup per (sequence, tile of 16, 32 or 64 query tokens, kv head), one
// wave per (query head of the kv head's group, 16-query sub-tile).  Per tile of 32 keys:
//   S^T = K Q^T   v_mfma_f32_16x16x32_bf16, K as the A operand loaded from
//                 HBM in operand layout (lane l: key l % 16, dims
//                 32c + 8(l / 16) .. +7), Q^T as the B operand (preloaded);
//                 lane l ends with the scores of query (l % 16) for keys
//                 4(l / 16) .. +3 of each 16-key half;
//   softmax       online, log2 domain, max / sum over the four lanes of a
//                 query with xor 16 / 32;
//   O^T += V^T P^T  P^T is the B operand straight from the softmax registers:
//                 MFMA k-index 8g + j (g = l / 16) stands for key 4g + j
//                 (j < 4) or 16 + 4g + j - 4 -- the same permutation of the
//                 32 keys on both operands leaves the sum unchanged; V^T is
//                 the A operand, read from a transposed LDS copy of the V tile
//                 ([dim][key]) that the G waves share, two 8-byte reads per
//                 fragment.
// The V tile is double-buffered in LDS with one barrier per key tile; K and
// V of the next tile are loaded while the current one is computed.
#include "common.h"

namespace lfs {
namespace {

typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int KT = 64;               // keys per tile
constexpr int NH = KT / 16;          // 16-key halves (S MFMA row blocks) per tile
constexpr int NKS = KT / 32;         // 32-key MFMA k steps of P.V per tile
constexpr int QT = 16;               // query tokens per wave (one MFMA column block)
constexpr int VT_PITCH = 2 * KT + 8; // bytes per dim row of the transposed V tile (+ pad)

// QW: 16-query sub-tiles per workgroup (G * QW waves share each K / V tile)
template <int D, int G, bool PAGED, int QW>
__global__ __launch_bounds__(64 * G * QW) void prefill_attention_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
    const int32_t* __restrict__ cu_q, const int32_t* __restrict__ cu_k, const int32_t* __restrict__ bt,
    int64_t bt_stride, int BS, int64_t num_slots, uint16_t* __restrict__ out, int Hkv, int qtiles,
    float scale_log2) {
  constexpr int NDC = D / 32;                        // 32-dim chunks (MFMA k steps of S)
  constexpr int NDB = D / 16;                        // 16-dim blocks of O^T
  constexpr int CPK = D / 8;                         // 16-byte chunks of a key row
  constexpr int VUN = KT / 2 * CPK;                  // (key pair, chunk) units of a V tile
  constexpr int NT = 64 * G * QW;                    // threads
  constexpr int VPT = (VUN + NT - 1) / NT;           // units per thread
  constexpr int KUN = KT * CPK;                      // 16-byte chunks of a K tile
  constexpr int KPT = (KUN + NT - 1) / NT;           // chunks per thread
  __shared__ __attribute__((aligned(16))) uint8_t vt[2][D * VT_PITCH];
  __shared__ __attribute__((aligned(16))) uint8_t kt[2][KT * 2 * D];

  // Workgroup ids are dealt round-robin to the 8 XCDs (id % 8): remap so
  // that each XCD takes a contiguous range of (sequence, kv head) pairs --
  // all query tiles of a pair read the same K / V, which then stays in that
  // XCD's L2 -- and walk a pair's query tiles from the last (longest
  // causal range) to the first.
  const int nwg = gridDim.x * gridDim.y;
  int wid = blockIdx.y * gridDim.x + blockIdx.x;
  if ((nwg & 7) == 0) wid = (wid & 7) * (nwg >> 3) + (wid >> 3);
  const int pair = wid / qtiles;
  const int i = pair / Hkv, kh = pair - i * Hkv;
  const int wq0 = (qtiles - 1 - (wid - pair * qtiles)) * QT * QW;  // the workgroup's first query
  const int q0 = cu_q[i], lq = cu_q[i + 1] - q0;
  if (wq0 >= lq) return;  // the whole workgroup
  const int k0 = cu_k[i], lk = cu_k[i + 1] - k0;
  const int off = lk - lq;  // position of query token 0
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  // wave -> (query head of the group, 16-query sub-tile); a sub-tile past lq
  // still runs the loop (the barriers) and stores nothing
  const int sub = wave / G;
  const int tq0 = wq0 + QT * sub;
  const int h = kh * G + (wave - sub * G), Hq = Hkv * G;
  const int c16 = lane & 15, g = lane >> 4;
  const int64_t row = (int64_t)Hkv * D;  // elements per token row of k / v
  const int64_t hoff = (int64_t)kh * D;

  // Key addresses per 16-key half of a tile.  Keys past the context read
  // the row of key lk - 1 (their scores are masked, but their V rows still
  // enter the P.V product with weight 0, so they must hold finite data:
  // pool slots past a sequence's keys may hold anything).  Paged: BS % 16
  // == 0, so a half (16-aligned) lies in one block and key x of it is the
  // half's slot base + x; an invalid table entry reads slot 0.
  // Contiguous: key t is row k0 + min(t, lk - 1) of k / v.
  auto half_slot = [&](int tstart) -> int64_t {  // paged only
    const int tc = min(tstart, lk - 1);
    const int32_t blk = bt[(int64_t)i * bt_stride + min((int64_t)(tc / BS), bt_stride - 1)];
    if (blk < 0 || (int64_t)blk * BS >= num_slots) return 0;
    return (int64_t)blk * BS + tc % BS;
  };
  auto key_elem = [&](const int64_t (&hs)[NH], int t0, int kx) -> int64_t {  // key t0 + kx, kx < KT
    const int hf = kx >> 4;
    if constexpr (PAGED) {
      // half base = slot of key min(t0 + 16 hf, lk - 1)
      return (hs[hf] + max(0, min(kx & 15, lk - 1 - (t0 + 16 * hf)))) * row + hoff;
    } else {
      return ((int64_t)k0 + min(t0 + kx, lk - 1)) * row + hoff;
    }
  };

  // Q^T (B operand): lane l supplies query tq0 + l % 16, dims 32c + 8g .. +7
  v8bf qb[NDC];
  {
    const int tq = tq0 + c16;
#pragma unroll
    for (int c = 0; c < NDC; ++c) {
      uint4 w = make_uint4(0, 0, 0, 0);
      if (tq < lq) w = *reinterpret_cast<const uint4*>(q + ((int64_t)(q0 + tq) * Hq + h) * D + c * 32 + g * 8);
      qb[c] = __builtin_bit_cast(v8bf, w);
    }
  }
  // this lane's query position; rows past lq are computed (finite) and not stored
  const int qp = min(off + tq0 + c16, lk - 1);
  // keys up to the last query of the tile
  const int nkt = (min(lk, off + wq0 + QT * QW) + KT - 1) / KT;

  auto halves = [&](int64_t (&hs)[NH], int t0) {
#pragma unroll
    for (int hf = 0; hf < NH; ++hf) {
      if constexpr (PAGED) hs[hf] = half_slot(t0 + 16 * hf);
      else hs[hf] = 0;
    }
  };
  // K tile in LDS: key rows of 2D bytes, 16-byte chunk c of row r at chunk
  // slot c ^ f(r) -- f(r) = ((r >> 1) & 7) ^ ((r & 1) << 2) for D = 64 (the
  // sixteen rows of one operand read, chunks g or g + 4, then touch every
  // bank once), r & 15 for D = 128
  auto kswz = [](int r, int c) -> int {
    const int f = D == 64 ? (((r >> 1) & 7) ^ ((r & 1) << 2)) : (r & 15);
    return r * 2 * D + ((c ^ f) << 4);
  };
  // chunk u of the tile: key u / CPK, chunk u % CPK (a row per CPK lanes)
  auto load_k = [&](uint4 (&kr)[KPT], const int64_t (&hs)[NH], int t0) {
#pragma unroll
    for (int e = 0; e < KPT; ++e) {
      const int u = threadIdx.x + NT * e;
      kr[e] = make_uint4(0, 0, 0, 0);
      if (u < KUN) kr[e] = *reinterpret_cast<const uint4*>(k + key_elem(hs, t0, u / CPK) + (u % CPK) * 8);
    }
  };
  auto store_kt = [&](const uint4 (&kr)[KPT], int buf) {
#pragma unroll
    for (int e = 0; e < KPT; ++e) {
      const int u = threadIdx.x + NT * e;
      if (u < KUN) *reinterpret_cast<uint4*>(&kt[buf][kswz(u / CPK, u % CPK)]) = kr[e];
    }
  };
  // V unit u of a tile: key pair kp (keys 2kp, 2kp + 1), 16-byte chunk cc of
  // both rows; eight consecutive units cover the chunks of one pair (whole
  // rows per eight lanes), the pair index is swizzled by the chunk's high
  // half so that a wave's 32-bit LDS writes below hit distinct banks
  auto vunit = [&](int u, int& kp, int& cc) {
    cc = (u & 7) + 8 * ((u >> 3) / (KT / 2) % (CPK / 8));
    const int kpl = (u >> 3) % (KT / 2);
    kp = (kpl + 8 * ((u & 7) >> 2)) % (KT / 2);
  };
  auto load_v = [&](uint4 (&vr)[VPT][2], const int64_t (&hs)[NH], int t0) {
#pragma unroll
    for (int e = 0; e < VPT; ++e) {
      const int u = threadIdx.x + NT * e;
      vr[e][0] = vr[e][1] = make_uint4(0, 0, 0, 0);
      if (u < VUN) {
        int kp, cc;
        vunit(u, kp, cc);
        vr[e][0] = *reinterpret_cast<const uint4*>(v + key_elem(hs, t0, 2 * kp) + cc * 8);
        vr[e][1] = *reinterpret_cast<const uint4*>(v + key_elem(hs, t0, 2 * kp + 1) + cc * 8);
      }
    }
  };
  // transposed store: dim d of keys (2kp, 2kp + 1) as one 32-bit word at
  // vt[d][2kp]
  auto store_vt = [&](const uint4 (&vr)[VPT][2], int buf) {
#pragma unroll
    for (int e = 0; e < VPT; ++e) {
      const int u = threadIdx.x + NT * e;
      if (u < VUN) {
        int kp, cc;
        vunit(u, kp, cc);
        const uint32_t* a = reinterpret_cast<const uint32_t*>(&vr[e][0]);
        const uint32_t* b = reinterpret_cast<const uint32_t*>(&vr[e][1]);
#pragma unroll
        for (int x = 0; x < 4; ++x) {
          // dims 8cc + 2x (low halves) and 8cc + 2x + 1 (high halves)
          const uint32_t lo = (a[x] & 0xFFFFu) | (b[x] << 16);
          const uint32_t hi = (a[x] >> 16) | (b[x] & 0xFFFF0000u);
          *reinterpret_cast<uint32_t*>(&vt[buf][(8 * cc + 2 * x) * VT_PITCH + kp * 4]) = lo;
          *reinterpret_cast<uint32_t*>(&vt[buf][(8 * cc + 2 * x + 1) * VT_PITCH + kp * 4]) = hi;
        }
      }
    }
  };

  v4f o[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) o[db] = v4f{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.f;

  uint4 kr[KPT], vr[VPT][2];
  int64_t hs[NH];
  halves(hs, 0);
  load_k(kr, hs, 0);
  load_v(vr, hs, 0);
  for (int j = 0; j < nkt; ++j) {
    const int t0 = j * KT;
    const int buf = j & 1;
    store_kt(kr, buf);
    store_vt(vr, buf);
    // K and V^T of tile j visible to every wave.  The buffers written next
    // (tile j+1) were last read in tile j-1, which every wave finished
    // before this barrier.
    __syncthreads();
    if (j + 1 < nkt) {
      halves(hs, t0 + KT);
      load_k(kr, hs, t0 + KT);
      load_v(vr, hs, t0 + KT);
    }
    const uint8_t* kb8 = kt[buf];

    // ---- S^T for the 16-key halves; the causal mask only where the tile
    // reaches past the tile's first query position
    const bool need_mask = t0 + KT - 1 > off + tq0;
    float s[NH][4];
    float tmax = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < NH; ++kb) {
      v4f sc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < NDC; ++c) {
        const uint4 kf = *reinterpret_cast<const uint4*>(kb8 + kswz(16 * kb + c16, 4 * c + g));
        sc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, kf), qb[c], sc, 0, 0, 0);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        s[kb][r] = sc[r] * scale_log2;
        if (need_mask && t0 + 16 * kb + 4 * g + r > qp) s[kb][r] = -INFINITY;
        tmax = fmaxf(tmax, s[kb][r]);
      }
    }
    tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
    const float m_new = fmaxf(m_run, tmax);  // finite: key 0 is never masked
    // exp2 on the hardware instruction (arguments <= 0; results below 2^-126 flush to 0)
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
    float psum = 0.f;
    float p[NH][4];
#pragma unroll
    for (int kb = 0; kb < NH; ++kb)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        p[kb][r] = __builtin_amdgcn_exp2f(s[kb][r] - m_new);
        psum += p[kb][r];
      }
    psum += __shfl_xor(psum, 16, 64);
    psum += __shfl_xor(psum, 32, 64);
    l_run = l_run * alpha + psum;
    m_run = m_new;

    // ---- O^T = O^T * alpha + V^T P^T, one MFMA k step per 32 keys
    v8bf pb[NKS];
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        pb[ks][r] = (__bf16)p[2 * ks][r];
        pb[ks][4 + r] = (__bf16)p[2 * ks + 1][r];
      }
    const uint8_t* vb = vt[buf];
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      const int dim = db * 16 + c16;
#pragma unroll
      for (int r = 0; r < 4; ++r) o[db][r] *= alpha;
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) {
        const uint2 lo = *reinterpret_cast<const uint2*>(vb + dim * VT_PITCH + (32 * ks + 4 * g) * 2);
        const uint2 hi = *reinterpret_cast<const uint2*>(vb + dim * VT_PITCH + (32 * ks + 16 + 4 * g) * 2);
        const uint4 w = make_uint4(lo.x, lo.y, hi.x, hi.y);
        o[db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, w), pb[ks], o[db], 0, 0, 0);
      }
    }
  }

  // ---- normalise and store: lane l holds query tq0 + l % 16, dims 16db + 4g .. +3
  const int tq = tq0 + c16;
  if (tq < lq) {
    const float inv = l_run > 0.f ? 1.f / l_run : 0.f;
    uint16_t* dst = out + ((int64_t)(q0 + tq) * Hq + h) * D;
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      uint2 w;
      w.x = pack_bf16x2(o[db][0] * inv, o[db][1] * inv);
      w.y = pack_bf16x2(o[db][2] * inv, o[db][3] * inv);
      *reinterpret_cast<uint2*>(dst + db * 16 + 4 * g) = w;
    }
  }
}

template <int D, bool PAGED, int QW>
bool launch_prefill(int G, dim3 grid, hipStream_t st, const uint16_t* q, const uint16_t* k, const uint16_t* v,
                    const int32_t* cu_q, const int32_t* cu_k, const int32_t* bt, int64_t bts, int BS,
                    int64_t num_slots, uint16_t* out, int Hkv, int qtiles, float sl2) {
#define LFS_PG(GG)                                                                                          \
  case GG:                                                                                                  \
    hipLaunchKernelGGL((prefill_attention_kernel<D, GG, PAGED, QW>), grid, dim3(64 * GG * QW), 0, st, q, k, \
                       v, cu_q, cu_k, bt, bts, BS, num_slots, out, Hkv, qtiles, sl2);                       \
    return true;
  switch (G) {
    LFS_PG(1) LFS_PG(2) LFS_PG(3) LFS_PG(4) LFS_PG(5) LFS_PG(6) LFS_PG(7) LFS_PG(8)
    default: return false;
  }
#undef LFS_PG
}

}  // namespace
}  // namespace lfs

using namespace lfs;

extern "C" int lfs_prefill_attention(const void* q, const void* k, const void* v, const int32_t* cu_seqlens_q,
                                     const int32_t* cu_seqlens_k, const int32_t* block_tables,
                                     int64_t bt_stride, int32_t block_size, int64_t num_slots, void* out,
                                     int64_t B, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                                     int32_t max_seqlen_q, float scale, void* stream) {
  const int Hq = num_q_heads, Hkv = num_kv_heads, D = head_dim;
  LFS_REQUIRE(B >= 0 && Hq > 0 && Hkv > 0 && max_seqlen_q >= 0, "prefill_attention: bad shape");
  LFS_REQUIRE(D == 64 || D == 128, "prefill_attention: head_dim must be 64 or 128 (got %d)", D);
  LFS_REQUIRE(Hq % Hkv == 0 && Hq / Hkv <= 8,
              "prefill_attention: num_q_heads (%d) must be a multiple of num_kv_heads (%d), ratio <= 8", Hq, Hkv);
  if (B == 0 || max_seqlen_q == 0) return 0;
  LFS_REQUIRE(q && k && v && cu_seqlens_q && cu_seqlens_k && out, "prefill_attention: null pointer");
  LFS_REQUIRE(((((uintptr_t)q) | ((uintptr_t)k) | ((uintptr_t)v) | ((uintptr_t)out)) & 15u) == 0,
              "prefill_attention: q, k, v and out must be 16-byte aligned");
  if (block_tables != nullptr) {
    LFS_REQUIRE(block_size > 0 && block_size % 16 == 0 && num_slots >= block_size && bt_stride > 0,
                "prefill_attention: bad paged KV geometry (block_size must be a multiple of 16)");
  }
  // Four (G <= 4) or two 16-query sub-tiles per workgroup (each K / V tile
  // feeds four or two times the queries) when that grid still fills every
  // CU several times over; otherwise one, for finer load balance.  Measured
  // on 16 x 2048-token prompts: four 254 us against two 266 us (10 launches
  // back to back); two 301 us against one 322 us (one launch).  16 x 512
  // queries over 2048 paged keys: two 220 us, one 194 us (one launch).
  // Results are bit-identical: a sub-tile's extra key tiles are all masked.
  const int G = Hq / Hkv;
  const int64_t qtiles2 = ((int64_t)max_seqlen_q + 2 * QT - 1) / (2 * QT);
  static int cu_cache[64] = {0};  // compute units per device, read once
  int cus = 256, dev = 0;
  if (hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < 64) {
    if (cu_cache[dev] == 0) {
      int n = 0;
      cu_cache[dev] = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0
                          ? n : 256;
    }
    cus = cu_cache[dev];
  }
  const int64_t qtiles4 = ((int64_t)max_seqlen_q + 4 * QT - 1) / (4 * QT);
  const int QWs = (G <= 4 && B * qtiles4 * Hkv >= 8ll * cus) ? 4 : (B * qtiles2 * Hkv >= 8ll * cus ? 2 : 1);
  const int64_t qtiles = ((int64_t)max_seqlen_q + QT * QWs - 1) / (QT * QWs);
  LFS_REQUIRE(B * qtiles < (1ll << 31) && Hkv < 65536, "prefill_attention: grid too large");
  const dim3 grid((unsigned)(B * qtiles), (unsigned)Hkv);
  const float sl2 = scale * 1.4426950408889634f;
  hipStream_t st = (hipStream_t)stream;
  const uint16_t *qq = (const uint16_t*)q, *kk = (const uint16_t*)k, *vv = (const uint16_t*)v;
  uint16_t* oo = (uint16_t*)out;
  const int32_t* bt = block_tables;
  const int64_t bts = bt != nullptr ? bt_stride : 0;
  const int BS = bt != nullptr ? block_size : 0;
  const int qt = (int)qtiles;
#define LFS_PF(DD, PG, QQ) \
  launch_prefill<DD, PG, QQ>(G, grid, st, qq, kk, vv, cu_seqlens_q, cu_seqlens_k, bt, bts, BS, num_slots, oo, Hkv, qt, sl2)
  bool ok;
  if (bt != nullptr)
    ok = D == 64 ? (QWs == 4 ? LFS_PF(64, true, 4) : QWs == 2 ? LFS_PF(64, true, 2) : LFS_PF(64, true, 1))
                 : (QWs == 4 ? LFS_PF(128, true, 4) : QWs == 2 ? LFS_PF(128, true, 2) : LFS_PF(128, true, 1));
  else
    ok = D == 64 ? (QWs == 4 ? LFS_PF(64, false, 4) : QWs == 2 ? LFS_PF(64, false, 2) : LFS_PF(64, false, 1))
                 : (QWs == 4 ? LFS_PF(128, false, 4) : QWs == 2 ? LFS_PF(128, false, 2) : LFS_PF(128, false, 1));
#undef LFS_PF
  LFS_REQUIRE(ok, "prefill_attention: unsupported group size %d", G);
  return check_launch("prefill_attention");
}
