/*
 * lfs_kernels.h -- C ABI of the MI355X (gfx950) block-wise FP8 and paged-KV
 * kernels.  Plain pointers and sizes only; no torch types.
 *
 * Conventions (all entry points):
 *   - Return 0 on success; a negative LFS_E* code for an argument error found
 *     on the host before anything was launched; a positive hipError_t value
 *     when the launch failed.  lfs_last_error() gives the message of the last
 *     failure on the calling thread.
 *   - `stream` is a hipStream_t (NULL = the default stream).  Work is only
 *     enqueued: nothing synchronises, allocates or frees.  The caller owns
 *     every buffer, including the paged-decode workspace (except
 *     lfs_paged_decode_noalloc, whose workspace is a library-owned static
 *     device array).
 *   - Device pointers must be 16-byte aligned unless stated otherwise.
 *   - bf16 buffers hold uint16 bit patterns; fp8 buffers hold OCP
 *     float8_e4m3fn bytes (torch.float8_e4m3fn).
 *
 * Reference interfaces replaced (paths relative to the reference repository):
 *   lfs_act_quant           act_quant(x, block_size, scale_fmt)
 *                           model/attention/utils.py:148-172 (kernel :97-145)
 *   lfs_weight_quant        128x128 weight-block quantisation; no reference
 *                           counterpart (defined by the benchmark configs);
 *                           same scale formula as utils.py:129-139
 *   lfs_weight_dequant      weight_dequant(x, s, block_size); named by the
 *                           benchmark, no reference counterpart
 *   lfs_fp8_gemm            fp8_gemm(a, a_s, b, b_s) (+bias for the
 *                           nn.Linear sites model/attention/GQA.py:34-37,
 *                           model/architecture/mlp.py:56-58); no reference
 *                           counterpart
 *   lfs_fp8_gemm_splitk     the same GEMM split over K for small M (the
 *                           decode-step linears)
 *   lfs_fp8_gemm_splitk_partials  its partial sums without the reduction,
 *                           for a consumer that sums them itself
 *                           (lfs_add_rmsnorm_partials); no reference
 *                           counterpart
 *   lfs_fp8_gemm_skinny     the same GEMM for M <= 128 (decode batches):
 *                           K split across the waves of a workgroup
 *   lfs_store_kvcache       the KV slot write of the attention layer that
 *                           engine/model_runner.py:8 imports (absent from the
 *                           reference); slot contract model_runner.py:226-230,
 *                           :261, :303
 *   lfs_paged_decode        paged-attention decode over block tables, the
 *                           decode call of the same absent layer; math of
 *                           model/attention/GQA.py:118-130, metadata contract
 *                           engine/model_runner.py:253-278 and :288-312
 *   lfs_paged_decode_rope   qk_norm_rope_store + the slot write + the
 *                           single-launch decode of one new token per
 *                           sequence, fused (GQA.py:80-95 and :118-130,
 *                           model_runner.py:226-230)
 *   lfs_paged_decode_noalloc  the same decode with a library-owned static
 *                           workspace; no reference counterpart (for callers
 *                           that cannot allocate)
 *   lfs_prefill_attention   varlen causal prefill attention, the
 *                           flash_attn_varlen_func(..., causal=True) call the
 *                           reference names at engine/model_runner.py:291-292
 *                           (metadata :202-249; paged keys on a prefix-cache
 *                           hit, :231-237); math of model/attention/GQA.py:118-130
 *   lfs_fp8_index           fp8_index(q, q_s, k, k_s), the DSA indexer score,
 *                           model/attention/utils.py:175-250 (caller
 *                           model/attention/DSA.py:105)
 *   lfs_sample_gumbel       temperature + Gumbel-max sampling,
 *                           utils/sampler.py:35-53 (Sampler.forward), with
 *                           its Exp(1) noise from Philox4x32-10
 *   lfs_sample_gumbel_split  the same sampler with each row cut into slices
 *                           (a caller workspace; same picks)
 * Fused row kernels of the decode step around those calls (each replaces a
 * chain of torch ops of the reference model):
 *   lfs_add_rmsnorm         RMSNorm with fused residual add, model/utils.py:53-67
 *                           (+ act_quant of the output for the next FP8 linear)
 *   lfs_add_rmsnorm_partials  the same with x the split-K reduction of the
 *                           previous FP8 linear (the MoE down projection
 *                           feeding the next layer's fused add & norm,
 *                           model/transformer.py:90-118)
 *   lfs_qk_norm_rope_store  q_norm/k_norm + RoPE + KV slot write,
 *                           model/attention/GQA.py:80-95,
 *                           model/attention/utils.py:34-45
 *   lfs_moe_route           MoE gate, model/architecture/moe.py:45-90
 *   lfs_add_rmsnorm_route   ffn_norm + MoE gate in one launch (decode step)
 *   lfs_swiglu_quant        silu(w1 x) * w3 x, model/architecture/mlp.py:60-67,
 *                           quantised for the experts' down projection
 * MoE expert dispatch (MoE.moe_infer, model/architecture/moe.py:288-341,
 * without its argsort / bincount / .tolist() host sync and scatter_add_):
 *   lfs_moe_align_tiles     capacity (128-row tiles) lfs_moe_align needs
 *   lfs_moe_align_workspace_bytes
 *   lfs_moe_align           (token, pick) entries grouped by expert into
 *                           128-row tiles (moe.py:298-307)
 *   lfs_fp8_grouped_gemm    one FP8 block-scaled GEMM per expert segment (the
 *                           per-expert MLP calls, moe.py:318-330)
 *   lfs_moe_combine         weighted sum of a token's expert rows (the
 *                           scatter_add_ of moe.py:332-339 and the shared
 *                           expert add of moe.py:272-273)
 * Weighted segment reduction (the Triton kernels of
 * model/architecture/moe_kernels.py):
 *   lfs_segment_reduce_weighted   segment_reduce_weighted, :70-125
 *   lfs_scatter_add_weighted      fused_scatter_add_weighted, :128-171
 *   lfs_scatter_add_weighted_workspace_bytes
 */
#ifndef LFS_KERNELS_H
#define LFS_KERNELS_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LFS_ABI_VERSION 15

/* argument errors (negative); launch errors are positive hipError_t values */
#define LFS_EINVAL (-1)

int lfs_abi_version(void);
const char* lfs_last_error(void);

/*
 * act_quant: per row, per group of `block_size` consecutive elements of the
 * last dimension:
 *   amax = max(max|x|, 1e-4); s = amax * fp32(1/448)
 *   (round_scale != 0: s = 2^ceil(log2(amax * fp32(1/448))), the ue8m0 form)
 *   y = e4m3fn(clamp(x / s, -448, 448))   (IEEE fp32 divide, RNE)
 * x: bf16 [M, K] with row stride ldx elements (ldx >= K, ldx % 8 == 0);
 * y: e4m3fn [M, K] contiguous; s: fp32 [M, K / block_size] contiguous.
 * block_size in {32, 64, 128}; K % block_size == 0; M * K < 2^34.
 */
int lfs_act_quant(const void* x, int64_t ldx, void* y, float* s, int64_t M, int64_t K,
                  int32_t block_size, int32_t round_scale, void* stream);

/*
 * weight_quant: same formula over 2-D blocks of block_size x block_size of
 * w: bf16 [N, K] contiguous -> y: e4m3fn [N, K], s: fp32
 * [ceil(N/bs), ceil(K/bs)].  Ragged tail blocks use their valid elements.
 * block_size in {32, 64, 128}; K % 8 == 0.
 */
int lfs_weight_quant(const void* w, void* y, float* s, int64_t N, int64_t K, int32_t block_size,
                     void* stream);

/*
 * weight_dequant: y[n,k] = bf16_RNE(fp32(w[n,k]) * s[n/bs, k/bs]).
 * w: e4m3fn [N, K]; s: fp32 [ceil(N/bs), ceil(K/bs)]; y: bf16 [N, K].
 * K % 8 == 0.
 */
int lfs_weight_dequant(const void* w, const float* s, void* y, int64_t N, int64_t K,
                       int32_t block_size, void* stream);

/*
 * fp8_gemm: c[m,n] = bf16_RNE( sum_kb a_s[m,kb] * b_s[n/128,kb] *
 *                              sum_{k in kb} a[m,k] * b[n,k]  (+ bias) )
 * with fp32 accumulation, the per-block scales applied to each 128-wide
 * K-block partial in the fp32 accumulator, and the bias added in fp32 before
 * the single rounding: bias[n] when bias_ld == 0, bias[m * bias_ld + n]
 * (a per-row bias matrix, bias_ld >= N) otherwise; bias may be NULL.
 * a: e4m3fn [M, K]; a_s: fp32 [M, K/128]; b: e4m3fn [N, K] (nn.Linear
 * weight layout); b_s: fp32 [ceil(N/128), K/128]; c: bf16 [M, N].
 * All contiguous; K % 128 == 0.  The kernel follows from the shape: for
 * 16 < M <= 128 and short K a one-shot kernel (each workgroup copies all
 * its operands to LDS at once), for large M persistent 256x256 tiles, else
 * 128x128 tiles; the results differ only in fp32 summation order.
 */
int lfs_fp8_gemm(const void* a, const float* a_s, const void* b, const float* b_s,
                 const float* bias, int64_t bias_ld, void* c, int64_t M, int64_t N, int64_t K,
                 void* stream);

/*
 * FP8Linear's forward (model/architecture/mlp.py:56-58, GQA.py:34-37 with
 * the linears in FP8) in one launch: c = lfs_fp8_gemm(act_quant(a, 128),
 * b, b_s, bias) for bf16 a [M, K] with row stride lda (>= K, a multiple of
 * 8), bit for bit -- the act_quant codes and scales are computed inside the
 * one-shot kernel's workgroups, where lfs_fp8_gemm would copy them.  No
 * counterpart in the reference as one call.  Only the shapes that
 * lfs_fp8_gemm runs on its one-shot kernel (16 < M <= 128, K and N small
 * enough): lfs_fp8_gemm_act_supported(M, N, K) returns 1 for them; other
 * shapes are refused with LFS_EINVAL.
 */
int lfs_fp8_gemm_act_supported(int64_t M, int64_t N, int64_t K);
int lfs_fp8_gemm_act(const void* a, int64_t lda, const void* b, const float* b_s, const float* bias,
                     int64_t bias_ld, void* c, int64_t M, int64_t N, int64_t K, void* stream);

/*
 * fp8_gemm with the K blocks split over `splits` workgroups per output tile
 * (for small M, where the tiles alone cannot fill the GPU): each split sums
 * ceil((K/128) / splits) consecutive K blocks into an fp32 partial tile in
 * `workspace`; a second kernel adds the partials in split order, adds the
 * bias and rounds to bf16.  Same result contract as lfs_fp8_gemm (fp32
 * accumulation; the order of the K-block sums differs).  workspace: at least
 * lfs_fp8_gemm_workspace_bytes(M, N, K, splits) bytes (0 when the split
 * count reduces to one), 16-byte aligned.
 */
int64_t lfs_fp8_gemm_workspace_bytes(int64_t M, int64_t N, int64_t K, int32_t splits);
int lfs_fp8_gemm_splitk(const void* a, const float* a_s, const void* b, const float* b_s,
                        const float* bias, int64_t bias_ld, void* c, int64_t M, int64_t N, int64_t K,
                        int32_t splits, void* workspace, int64_t workspace_bytes, void* stream);

/*
 * The first kernel of lfs_fp8_gemm_splitk alone: the fp32 partial sums
 * workspace[s][M][N] for s < n, n = ceil(KT / ceil(KT / splits)), KT = K/128
 * (no bias, no C).  The split must leave n >= 2 (an argument error
 * otherwise).  Summing them in order s = 0 .. n-1 from 0.f, adding the bias
 * and rounding to bf16 gives lfs_fp8_gemm_splitk's C bit for bit.
 */
int lfs_fp8_gemm_splitk_partials(const void* a, const float* a_s, const void* b, const float* b_s, int64_t M,
                                 int64_t N, int64_t K, int32_t splits, void* workspace, int64_t workspace_bytes,
                                 void* stream);

/*
 * fp8_gemm for decode-sized batches, M <= 128: the same result as
 * lfs_fp8_gemm up to fp32 summation order (the K blocks are split over 4, 8
 * or 16 waves of a workgroup and the partials added through LDS, in wave
 * order).  One workgroup per 16 or 32 output columns; no workspace.
 */
int lfs_fp8_gemm_skinny(const void* a, const float* a_s, const void* b, const float* b_s, const float* bias,
                        int64_t bias_ld, void* c, int64_t M, int64_t N, int64_t K, void* stream);

/*
 * store_kvcache: for t < T with slot = slot_mapping[t] != -1,
 *   k_cache[slot / BS][slot % BS][:][:] = key[t][:][:]   (same for value)
 * key/value: bf16 [T, Hkv, D] with token stride k_stride_t / v_stride_t
 * elements (heads and head_dim contiguous); caches: bf16 [NB, BS, Hkv, D]
 * contiguous; num_slots = NB * BS.  Slots outside [0, num_slots) are
 * skipped.  16-byte vector copies when every row is 16-byte aligned, 2-byte
 * copies otherwise.
 */
int lfs_store_kvcache(const void* key, int64_t k_stride_t, const void* value, int64_t v_stride_t,
                      void* k_cache, void* v_cache, const int64_t* slot_mapping, int64_t T,
                      int32_t num_kv_heads, int32_t head_dim, int64_t num_slots, void* stream);

/*
 * Paged-attention decode (one query token per sequence), GQA:
 *   o[b,h,:] = sum_{t < L_b} softmax_t(scale * q[b,h,:] . K[b,t,h/G,:]) V[b,t,h/G,:]
 *   K[b,t,kh,:] = k_cache[block_tables[b][t / BS]][t % BS][kh][:], G = Hq/Hkv
 * q: bf16 [B, Hq, D] contiguous; caches: bf16 [NB, BS, Hkv, D] contiguous;
 * context_lens: int64 [B] (0 = padding row -> o = 0); block_tables: int32
 * [B, bt_stride], entries t/BS < ceil(L_b/BS) valid, the rest ignored (-1
 * padding); out: bf16 [B, Hq, D].  Block ids outside [0, NB) contribute
 * nothing.
 * blocks_per_split = n > 0: every context is split into chunks of n blocks
 * processed in parallel (one wave per sequence, kv head and chunk) and
 * merged by log-sum-exp.  blocks_per_split = 0 (B <= 8192): balanced split,
 * a fixed grid of one 4-wave workgroup per CU, each taking an equal share of
 * the (sequence, kv-head group, tile) work whatever the lengths, then the
 * same merge.  blocks_per_split = -1: single launch, one 8-wave workgroup
 * per (sequence, pair of kv heads) (one kv head when Hkv is odd) whose waves
 * walk interleaved tiles and merge through LDS; no workspace, no second
 * launch.  blocks_per_split = -2 (B <= 256): the single launch in the
 * paired order, one 4-wave workgroup per (sequence, kv head); every
 * workgroup ranks the sequences by context length (longest first, ties to
 * the lower index) and takes its (sequence, kv head) from that order so
 * that the two workgroups a CU holds at once -- w and w + CUs -- are a long
 * and a short one (the longest run alone when fewer than two rounds).
 * Whatever the mode, the grid depends only on the shapes (not on the
 * lengths), so the call is graph-capturable.
 * workspace: at least lfs_paged_decode_workspace_bytes(...) bytes (for 0 a
 * bound from the current device's CU count: size it on that device; for -1
 * and -2 zero, and workspace may be NULL).
 * Optionally (q_out and q_scale both non-NULL) also the act_quant of each
 * output row, the output projection's FP8 input: q_out e4m3fn [B, Hq*D],
 * q_scale fp32 [B, Hq*D/128], bit-identical to lfs_act_quant(out, 128)
 * (needs Hq*D % 128 == 0, for -1 also an even Hkv or G*D % 128 == 0, for
 * -2 G*D % 128 == 0);
 * the merge then runs one workgroup per (128-value group, sequence) instead
 * of one per (head, sequence).
 * D in {64, 128}; Hq % Hkv == 0, Hq/Hkv <= 8; block_size a multiple of 16.
 */
int64_t lfs_paged_decode_workspace_bytes(int64_t B, int32_t num_q_heads, int32_t head_dim,
                                         int32_t max_blocks, int32_t blocks_per_split);

int lfs_paged_decode(const void* q, const void* k_cache, const void* v_cache,
                     const int64_t* context_lens, const int32_t* block_tables, int64_t bt_stride,
                     void* out, void* workspace, int64_t workspace_bytes, int64_t B,
                     int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                     int32_t block_size, int64_t num_blocks, int32_t max_blocks, float scale,
                     int32_t blocks_per_split, void* q_out, float* q_scale, void* stream);

/*
 * The decode step's qk_norm_rope_store followed by lfs_paged_decode with
 * blocks_per_split -1, in one launch (no counterpart in the reference as one
 * call: it replaces model/attention/GQA.py:80-95's q/k norms and RoPE, the
 * KV slot write of engine/model_runner.py:226-230, and the decode attention
 * of GQA.py:118-130 for one new token per sequence).  For sequence b:
 * qkv[b] (bf16, row stride ld) is normalised and rotated as
 * lfs_qk_norm_rope_store does (same bits); its k and v rows are written to
 * the cache slot slot_mapping[b] (skipped outside [0, num_blocks *
 * block_size), or when slot_mapping is NULL); the attention then runs over
 * the context_lens[b] tokens of the sequence, the first L-1 read from the
 * pool and the newest (position L-1) taken from the row itself, so nothing
 * written by the call is read back.  out, q_out / q_scale as for
 * lfs_paged_decode (q_out needs an even num_kv_heads or G*D % 128 == 0);
 * q_rot (optional, bf16 [B, Hq, D]) receives the rotated q.  Needs
 * (Hq + Hkv) * D / 16 <= 256 besides lfs_paged_decode's shape limits.  The
 * results equal the two calls' up to fp32 summation order (the newest token
 * enters the softmax first).  Without q_out, the launch takes the paired
 * order of blocks_per_split -2 when B <= 256, CUs < B * Hkv <= 2 * CUs and
 * the table holds at most 8192 tokens; its workgroups then run the q/k
 * prologue before their walks, and the newest token enters the softmax
 * last.
 */
int lfs_paged_decode_rope(const void* qkv, int64_t ld, const float* q_weight, const float* k_weight,
                          const float* cos_sin, int64_t max_positions, const int64_t* positions,
                          const int64_t* slot_mapping, float eps, void* q_rot, void* k_cache, void* v_cache,
                          const int64_t* context_lens, const int32_t* block_tables, int64_t bt_stride,
                          void* out, int64_t B, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                          int32_t block_size, int64_t num_blocks, int32_t max_blocks, float scale,
                          void* q_out, float* q_scale, void* stream);

/*
 * lfs_paged_decode without a caller workspace: the split partials live in a
 * library-owned device array of LFS_DECODE_SCRATCH_BYTES per GPU (allocated
 * when the library's code object loads on that GPU, held until the process
 * ends); the call allocates and frees nothing.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops).  Same arguments, result and
 * kernels as lfs_paged_decode; a shape whose
 * lfs_paged_decode_workspace_bytes(...) exceeds LFS_DECODE_SCRATCH_BYTES is
 * rejected with LFS_EINVAL (cfg4's B 256, Hq 32, D 128 needs 42.6 MB on 256
 * CUs).  Every call on one GPU shares that GPU's array: calls that overlap
 * on one GPU (two streams, two threads) race and must be serialised by the
 * caller.
 */
#define LFS_DECODE_SCRATCH_BYTES (64ll << 20)

int lfs_paged_decode_noalloc(const void* q, const void* k_cache, const void* v_cache,
                             const int64_t* context_lens, const int32_t* block_tables, int64_t bt_stride,
                             void* out, int64_t B, int32_t num_q_heads, int32_t num_kv_heads,
                             int32_t head_dim, int32_t block_size, int64_t num_blocks, int32_t max_blocks,
                             float scale, int32_t blocks_per_split, void* q_out, float* q_scale,
                             void* stream);

/*
 * Varlen causal prefill attention, GQA (G = Hq / Hkv):
 *   sequence i: queries q[cu_q[i] .. cu_q[i+1]) at positions lk-lq .. lk-1 of
 *   its context of lk = cu_k[i+1] - cu_k[i] keys; query position p:
 *   o[:, h] = sum_{t <= p} softmax_t(scale * q[:, h] . K_i[t, h/G]) V_i[t, h/G]
 *   K_i[t] = k[cu_k[i] + t]                          (block_tables == NULL;
 *            k, v bf16 [cu_k[B], Hkv, D])
 *   K_i[t] = k[block_tables[i][t / BS] * BS + t % BS] (paged; k, v the pool
 *            bf16 [num_slots / BS, BS, Hkv, D], block_tables int32
 *            [B, bt_stride]; entries outside [0, num_slots / BS) read slot 0)
 * q, out: bf16 [cu_q[B], Hq, D] contiguous; cu_seqlens int32 [B + 1];
 * max_seqlen_q >= every lq (sets the grid, so a fixed value keeps the call
 * capturable).  D in {64, 128}; Hq % Hkv == 0, Hq / Hkv <= 8.
 */
int lfs_prefill_attention(const void* q, const void* k, const void* v, const int32_t* cu_seqlens_q,
                          const int32_t* cu_seqlens_k, const int32_t* block_tables, int64_t bt_stride,
                          int32_t block_size, int64_t num_slots, void* out, int64_t B,
                          int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                          int32_t max_seqlen_q, float scale, void* stream);

/*
 * FP8 indexer score (DSA lightning indexer):
 *   o[b,m,n] = k_s[b][n] * sum_h relu(q[b,m,h,:] . k[b,n,:]) * q_s[b,m,h]
 * q: e4m3fn [B, M, H, D] contiguous; q_s fp32 [B, M, H]; k: e4m3fn rows of
 * D bytes, batch b at k + b * k_stride_b (bytes, multiple of 16, >= N*D);
 * k_s fp32 [B, ks_stride_b]; o fp32 [B, M, N].  D in {32, 64, 128}; H <= 128.
 */
int lfs_fp8_index(const void* q, const float* q_s, const void* k, const float* k_s, float* o, int64_t B,
                  int32_t M, int32_t N, int32_t H, int32_t D, int64_t k_stride_b, int64_t ks_stride_b,
                  void* stream);

/*
 * Temperature + Gumbel-max sampling, per row b of logits (bf16 [B, ld]):
 *   out[b] = argmax_i softmax(logits[b, :vocab] / T[b])_i / max(e[b,i], 1e-10)
 * (ties: lowest index); e[b,i] = -log((w + 1) * 2^-32), w = word i % 4 of
 * Philox4x32-10 with counter (i/4 + offset_lo, offset_hi + carry, b,
 * 0x53414D50) and key (seed_lo, seed_hi).  temperatures fp32 [B] (> 0);
 * out int64 [B]; noise_out (fp32 [B, vocab]) receives e when not NULL.
 * A caller advances offset by ceil(vocab / 4) per call for fresh noise.
 */
int lfs_sample_gumbel(const void* logits, int64_t ld, const float* temperatures, int64_t B, int32_t vocab,
                      uint64_t seed, uint64_t offset, int64_t* out, float* noise_out, void* stream);

/*
 * The same sampling with each row cut into slices of consecutive elements,
 * one workgroup per (row, slice), then a per-row pick of the best slice:
 * the same picks (and noise) as lfs_sample_gumbel, with more workgroups
 * when the batch alone would leave compute units idle.  workspace: at least
 * lfs_sample_gumbel_workspace_bytes(B, vocab) bytes, 8-byte aligned (0
 * bytes: the call is one pass and needs none; size it on the device that
 * runs the call).
 */
int64_t lfs_sample_gumbel_workspace_bytes(int64_t B, int32_t vocab);
int lfs_sample_gumbel_split(const void* logits, int64_t ld, const float* temperatures, int64_t B,
                            int32_t vocab, uint64_t seed, uint64_t offset, int64_t* out, float* noise_out,
                            void* workspace, int64_t workspace_bytes, void* stream);

/*
 * add_rmsnorm, per row t of x: bf16 [T, d]:
 *   r = x[t] (+ residual[t])                    fp32 sum of the bf16 inputs
 *   residual_out[t] = bf16(r)                    (only with a residual)
 *   out[t] = bf16(weight * r * rsqrt(mean(r^2) + eps))       weight fp32 [d]
 *   q[t], q_scale[t] = act_quant(out[t], 128)    (optional)
 * residual and residual_out are both given or both NULL; q and q_scale
 * likewise (needs d % 128 == 0); out may be NULL when q is given.
 * d % 8 == 0, d <= 8192; all rows contiguous.
 */
int lfs_add_rmsnorm(const void* x, const void* residual, const float* weight, void* out,
                    void* residual_out, void* q, float* q_scale, int64_t T, int32_t d, float eps,
                    void* stream);

/*
 * lfs_add_rmsnorm with x[t] = bf16(sum over s < nparts of parts[s][t] (fp32
 * [nparts][T][d], summed in order from 0.f) + bias[t]): the output of
 * lfs_fp8_gemm_splitk_partials followed by the reduction lfs_fp8_gemm_splitk
 * performs, bit for bit, without its launch.  bias: NULL, fp32 [d]
 * (bias_ld 0) or rows bias_ld >= d floats apart.  d % 8 == 0, d <= 8192.
 */
int lfs_add_rmsnorm_partials(const float* parts, int32_t nparts, const float* bias, int64_t bias_ld,
                             const void* residual, const float* weight, void* out, void* residual_out, void* q,
                             float* q_scale, int64_t T, int32_t d, float eps, void* stream);

/*
 * qk_norm_rope_store, per token t of qkv: bf16 [T, ld], row = [q (Hq*D) |
 * k (Hkv*D) | v (Hkv*D)]:
 *   q' = bf16(q_weight * q * rsqrt(mean(q^2) + eps)) over all Hq*D values,
 *   k' likewise over Hkv*D with k_weight; then per head the half-split
 *   rotation with c, s = cos_sin[positions[t]][0..D/2), [D/2..D):
 *   y1 = x1*c - x2*s, y2 = x2*c + x1*s (fp32), rounded to bf16;
 *   q_out[t] (bf16 [T, Hq, D]) = rotated q'; rotated k' and v are written to
 *   k_cache / v_cache (bf16 [NB, BS, Hkv, D]) at slot slot_mapping[t] when
 *   0 <= slot < num_slots (slot_mapping may be NULL: no cache write).
 * cos_sin: fp32 [max_positions, D]; positions int64 [T] (clamped to the
 * table).  D % 16 == 0; (Hq + Hkv) * D <= 16384.
 */
int lfs_qk_norm_rope_store(const void* qkv, int64_t ld, const float* q_weight, const float* k_weight,
                           const float* cos_sin, const int64_t* positions,
                           const int64_t* slot_mapping, void* q_out, void* k_cache, void* v_cache,
                           int64_t T, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                           int64_t num_slots, int64_t max_positions, float eps, void* stream);

/*
 * moe_route, per token t of h: bf16 [T, d]:
 *   logit[e] = h[t] . gate_weight[e] (fp32), gate_weight bf16 [E, d];
 *   the top_k experts by logit + expert_bias[e] (ties: lower index) get
 *   weight sigmoid(logit[e]) / (sum over the chosen + 1e-10) (top_k > 1) or
 *   sigmoid(logit[e]) (top_k == 1), the others 0;
 *   dense_weights[t] (fp32 [T, E + S]) = those weights, then S ones for the
 *   shared experts; bias_out[t] (fp32 [T, d]) = sum_e dense_weights[t][e] *
 *   down_bias[e] (fp32 [E + S, d]).
 *   Optionally (both or neither) the picks in the gate's index form:
 *   topk_idx (int64 [T, top_k], in pick order) and topk_weight (fp32
 *   [T, top_k], their weights) -- the (topk_idx, topk_weight) the reference
 *   gate returns (moe.py:90).  dense_weights may be NULL when topk_idx is
 *   given; bias_out may be NULL (then down_bias may be too).
 * E + S <= 64; d % 8 == 0.
 */
int lfs_moe_route(const void* h, const void* gate_weight, const float* expert_bias,
                  const float* down_bias, float* dense_weights, float* bias_out, int64_t T,
                  int32_t d, int32_t num_experts, int32_t num_shared, int32_t top_k,
                  int64_t* topk_idx, float* topk_weight, void* stream);

/*
 * add_rmsnorm_route: lfs_add_rmsnorm (quantised output required) and
 * lfs_moe_route (dense weights, optional routed bias) of the same rows in one
 * launch -- the decode step's ffn_norm (model/transformer.py:90-118) followed
 * by the MoE gate (model/architecture/moe.py:45-90), replacing the pair
 * add_rmsnorm + moe_route.  Outputs bit-identical to that pair; out (the bf16
 * normalised rows) may be NULL.  d % 128 == 0, d <= 8192; E + S <= 64.
 */
int lfs_add_rmsnorm_route(const void* x, const void* residual, const float* weight, void* out,
                          void* residual_out, void* q, float* q_scale, int64_t T, int32_t d, float eps,
                          const void* gate_weight, const float* expert_bias, const float* down_bias,
                          float* dense_weights, float* bias_out, int32_t num_experts, int32_t num_shared,
                          int32_t top_k, void* stream);

/*
 * swiglu_quant, for h13: bf16 [T, E, 2, F] (per expert the w1 then the w3
 * output rows):
 *   g = bf16(bf16(silu(a)) * b), silu(a) = a / (1 + exp(-a)) in fp32;
 *   q (e4m3fn [T, E*F]), s = act_quant(g, 128) per row;
 *   q_scale[t][e*F/128 + i] = s * route_weights[t][e] (fp32 [T, E]).
 * F % 128 == 0.
 */
int lfs_swiglu_quant(const void* h13, const float* route_weights, void* q, float* q_scale, int64_t T,
                     int32_t num_experts, int32_t d_ff, void* stream);

/* ------------------------------------------------------------ MoE dispatch */

/*
 * Number of 128-row tiles lfs_moe_align may fill for T tokens with top_k
 * picks and S shared experts over E routed ones:
 * ceil((T * (top_k + S) + (E + S) * 127) / 128).
 */
int64_t lfs_moe_align_tiles(int64_t T, int32_t top_k, int32_t num_experts, int32_t num_shared);

/*
 * moe_align.  Entry i = t * (top_k + S) + j: for j < top_k the routed expert
 * topk_idx[t][j] (int64 [T, top_k]; values outside [0, E) are dropped) with
 * weight topk_weight[t][j] (fp32), for j >= top_k the shared expert
 * E + j - top_k with weight 1.  Rows are grouped by expert, experts in index
 * order, each expert's entries in entry order, each expert's segment padded
 * to a multiple of 128 rows:
 *   row_token[r] (int32 [num_tiles*128])  token of row r, -1 for padding
 *   row_weight[r] (fp32 [num_tiles*128])  weight of row r, 0 for padding
 *   tile_expert[i] (int32 [num_tiles])    expert of rows 128i .. 128i+127,
 *                                         -1 for tiles past the last segment
 *   entry_row[i] (int32 [T*(top_k+S)])    row of entry i (-1 if dropped)
 * num_tiles >= lfs_moe_align_tiles(...); E + S <= 64.  Three launches
 * (per-chunk ranks, one-workgroup offsets, per-chunk placement) whose shapes
 * depend only on T and num_tiles (graph-capturable); the caller-owned int32
 * workspace holds the per-chunk counts.
 */
int lfs_moe_align(const int64_t* topk_idx, const float* topk_weight, int64_t T, int32_t top_k,
                  int32_t num_experts, int32_t num_shared, int32_t* row_token, float* row_weight,
                  int32_t* tile_expert, int64_t num_tiles, int32_t* entry_row, void* workspace,
                  int64_t workspace_bytes, void* stream);

/* workspace bytes of lfs_moe_align: 4 * (chunks * (E + S) + 2 * (E + S) + 1),
 * chunks = ceil(T * (top_k + S) / 1024) */
int64_t lfs_moe_align_workspace_bytes(int64_t T, int32_t top_k, int32_t num_experts, int32_t num_shared);

/*
 * fp8_grouped_gemm: for every tile i < num_tiles with e = tile_expert[i] >= 0
 * and every row m of it (m = 128i .. 128i+127):
 *   C[m, n] = sum_kb a_s[r, kb] * Bs_e[n/128, kb] * (A[r, kb] . B_e[n, kb]) (+ bias_e[n])
 * with r = row_index[m] (row_index NULL: r = m; r < 0 reads row 0 -- a
 * padding row, whose result is written but means nothing), A e4m3fn
 * [a_rows, K], a_s fp32 [a_rows, K/128], B_e = b + e*b_expert_stride (row n
 * at + n*ldb bytes), Bs_e = b_s + e*bs_expert_stride (row n/128 at
 * + (n/128)*ldbs floats), bias_e = bias + e*bias_expert_stride (fp32, NULL
 * for none).  Exactly one output: c bf16 [num_tiles*128, N] (with the
 * bias), or c_f32 fp32 [num_tiles*128, N] (no bias).  Rows of tiles with
 * e < 0 are not written.  K % 128 == 0; ldb, b_expert_stride % 16 == 0.
 */
int lfs_fp8_grouped_gemm(const void* a, const float* a_s, int64_t a_rows, const int32_t* row_index,
                         const int32_t* tile_expert, int64_t num_tiles, const void* b, const float* b_s,
                         int64_t b_expert_stride, int64_t ldb, int64_t bs_expert_stride, int64_t ldbs,
                         const float* bias, int64_t bias_expert_stride, void* c, float* c_f32, int64_t N,
                         int64_t K, void* stream);

/*
 * moe_combine, per token t (entries i = t*(top_k+S) + j as in moe_align):
 *   y[t] = bf16( sum_j out[entry_row[i]] + sum_j w_j * down_bias[e_j] )
 * summed in fp32 in j order, entries with entry_row < 0 skipped; out
 * [rows, ld] bf16 (out_is_f32 = 0) or fp32 (the down projection's rows,
 * routing weights already applied), down_bias fp32 [E + S, d] or NULL;
 * y bf16 [T, d].  d % 8 == 0, ld % 8 == 0.
 */
int lfs_moe_combine(const void* out, int32_t out_is_f32, int64_t ld, const int32_t* entry_row,
                    const int64_t* topk_idx, const float* topk_weight, int64_t T, int32_t top_k,
                    int32_t num_experts, int32_t num_shared, const float* down_bias, int32_t d, void* y,
                    void* stream);

/*
 * segment_reduce_weighted: y[t] = sum_{p : idx[p] == t} w[p] * x[p] for
 * t < num_tokens, p in increasing order, fp32 accumulation, stored in x's
 * dtype.  x: bf16 (x_is_f32 = 0) or fp32 [n, ldx]; w: bf16 or fp32 [n];
 * sorted_token_idx: int64 [n], non-decreasing (each token's segment is
 * found by binary search, like torch.searchsorted).  y contiguous
 * [num_tokens, d].  Every entry of a segment is summed (the reference's
 * kernel stops after next_pow2(max(top_k, 2)) of them).  2-byte alignment
 * suffices.
 */
int lfs_segment_reduce_weighted(const void* x, int32_t x_is_f32, int64_t ldx, const void* weights,
                                int32_t w_is_f32, const int64_t* sorted_token_idx, int64_t n,
                                int64_t num_tokens, int32_t d, void* y, void* stream);

/* workspace bytes of lfs_scatter_add_weighted: 4 * (3 * num_tokens + 1 + n) */
int64_t lfs_scatter_add_weighted_workspace_bytes(int64_t n, int64_t num_tokens);

/*
 * scatter_add_weighted: the same sum for any order of token_idx (int64 [n];
 * entries outside [0, num_tokens) are skipped): the entries are counted,
 * scanned and placed per token in a caller-owned int32 workspace, then
 * each token's segment is summed in increasing entry order (segments of
 * more than 256 entries in placement order).  Six launches, no
 * synchronisation, no memset (the counters are cleared by a kernel).
 */
int lfs_scatter_add_weighted(const void* x, int32_t x_is_f32, int64_t ldx, const void* weights,
                             int32_t w_is_f32, const int64_t* token_idx, int64_t n, int64_t num_tokens,
                             int32_t d, void* y, void* workspace, int64_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* LFS_KERNELS_H */
