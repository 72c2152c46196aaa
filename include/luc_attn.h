/*
 * luc_attn.h -- C ABI of the MI355X (gfx950) paged-attention path for the
 * lucciola-rs Qwen2 engine.
 *
 * The library (liblucattn.so) loads gfx950 code objects with hipModuleLoad and
 * launches hand-written HIP kernels on the caller's stream.  It replaces the
 * engine's NVRTC/PTX loader (build.rs:14-42, src/ptx.rs:1-22,
 * src/utils.rs:10-18) and three CUDA kernels: rope (src/kernels/rope.cu:3-54),
 * update_kv_cache_kernel (src/kernels/kv_cache.cu:3-59) and
 * flash_decoding_kernel_{64,128} (src/kernels/attention.cu:4-240).
 *
 * Conventions (all entry points):
 *  - Plain pointers and sizes.  Device pointers are hipMalloc'd memory owned by
 *    the caller; the library never allocates or frees caller memory, and the
 *    split-K workspace is caller-provided.
 *  - `stream` is a hipStream_t passed as void*; NULL means the null stream.
 *    Launches are asynchronous; no entry point synchronises.
 *  - Return 0 (LUC_OK) or a negative luc_status.  luc_last_error() returns a
 *    thread-local message for the last failure on the calling thread.
 *  - 16-bit storage (bf16 or fp16, luc_dtype), f32 arithmetic.
 *  - KV pools use the engine's layout [phys_block][num_layers][Hkv][16][head_dim]
 *    (src/layers/kv_cache.rs:50-68); block tables are int32 [rows][table_stride].
 *  - Positions are device int32 arrays: the position of the current token, so a
 *    sequence attends to positions 0..pos (ctx = pos + 1), as the reference's
 *    device-resident pos_ptr (src/models.rs:489-493, :715).
 *  - Entry points that address pages through block tables take num_blocks,
 *    the number of pages in each pool (the reference's num_physical_blocks,
 *    kv_cache.rs:57-59; its kernels read table entries unchecked,
 *    kv_cache.cu:28, attention.cu:82).  A table entry outside [0, num_blocks)
 *    is never used as an address: the cache write that would go through it is
 *    skipped (the row's q and k are still roped in place, by every entry point
 *    alike) and every attention output whose context reaches that page is NaN.
 *    A position outside its table row (or negative) leaves the row untouched.
 *    num_blocks < 1 is LUC_E_INVALID.
 *  - Only block_size 16 (kv_cache.rs:35) and head_dim 64/128
 *    (kernels.rs:37-46) are supported; Hq must be a multiple of Hkv with
 *    Hq/Hkv <= 8.
 */
#ifndef LUC_ATTN_H
#define LUC_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LUC_ABI_VERSION 4
#define LUC_BLOCK_SIZE 16

typedef struct luc_ctx luc_ctx;

typedef enum luc_dtype { LUC_BF16 = 0, LUC_F16 = 1 } luc_dtype;

typedef enum luc_status {
    LUC_OK = 0,
    LUC_E_INVALID = -1,     /* bad argument (null pointer, bad size, misalignment) */
    LUC_E_UNSUPPORTED = -2, /* head_dim / block_size / group size outside what is built */
    LUC_E_LOAD = -3,        /* code object or kernel symbol could not be loaded */
    LUC_E_HIP = -4,         /* a HIP runtime call failed */
    LUC_E_WORKSPACE = -5,   /* workspace missing or smaller than required */
    LUC_E_NOMEM = -6        /* the page allocator's free list is short */
} luc_status;

/* ABI version compiled into the library (LUC_ABI_VERSION). */
int luc_abi_version(void);

/* Thread-local description of the last error on this thread ("" if none). */
const char* luc_last_error(void);

/* Load the gfx950 code objects for `device` and resolve every kernel.
 * `code_object_dir` is the directory holding the .hsaco files; NULL means the
 * directory of the loaded library.  Replaces CudaFunctions::load
 * (src/kernels.rs:32-107) and load_cuda_funtion (src/utils.rs:10-18). */
int luc_init(int device, const char* code_object_dir, luc_ctx** out_ctx);
void luc_destroy(luc_ctx* ctx);

/* Host-side RoPE table, f32 [max_pos][head_dim/2] each, from the same f32
 * formula as RopeCache::new (src/layers/rope.rs:11-40).  scale_factor <= 0
 * means no rope_scaling (factor 1).  The caller copies it to the device. */
int luc_rope_table(float* cos_out, float* sin_out, int max_pos, int head_dim, float base,
                   float scale_factor);

/* RoPE with q/k bias, in place, for num_tokens rows -- rope
 * (src/kernels/rope.cu:3-54) as launched by CudaFunctions::apply_rope
 * (src/kernels.rs:203-246).  Row r of q is q + r*row_stride, likewise k; the
 * engine passes views into qkv_states, so row_stride = (Hq + 2*Hkv)*head_dim.
 * positions[r] selects the cos/sin row.  Biases may be NULL (read as zero). */
int luc_rope(luc_ctx* ctx, void* stream, int dtype, void* q, const void* q_bias, void* k,
             const void* k_bias, int64_t row_stride, const float* cos_table,
             const float* sin_table, const int32_t* positions, int num_tokens, int num_q_heads,
             int num_kv_heads, int head_dim);

/* Paged cache write of one token per row -- update_kv_cache_kernel
 * (src/kernels/kv_cache.cu:3-59) as launched by KVCache::update
 * (src/layers/kv_cache.rs:124-173).  Row r writes k (bit copy) and v + v_bias
 * at slot positions[r] of table row r.  v_bias may be NULL. */
int luc_kv_cache_update(luc_ctx* ctx, void* stream, int dtype, void* k_pool, void* v_pool,
                        const void* k, const void* v, const void* v_bias, int64_t row_stride,
                        const int32_t* block_tables, int table_stride, int num_blocks,
                        const int32_t* positions, int num_tokens, int layer, int num_layers,
                        int num_kv_heads, int head_dim, int block_size);

/* Fused RoPE + cache write: the two calls above in one launch, with the same
 * results (q and k roped in place, roped k and v + v_bias written to the
 * pools).  This is what the engine's per-layer step src/models.rs:505-534
 * becomes. */
int luc_rope_append(luc_ctx* ctx, void* stream, int dtype, void* q, const void* q_bias,
                    void* k, const void* k_bias, const void* v, const void* v_bias,
                    int64_t row_stride, const float* cos_table, const float* sin_table,
                    const int32_t* positions, const int32_t* block_tables, int table_stride,
                    int num_blocks, void* k_pool, void* v_pool, int num_tokens, int layer, int num_layers,
                    int num_q_heads, int num_kv_heads, int head_dim, int block_size);

/* Bytes of split-K workspace luc_paged_decode / luc_decode_step need for these
 * sizes (0 when every sequence fits one split; the workspace may then be
 * NULL).  split_tokens: tokens per split-K chunk, rounded up to a multiple of
 * 256 (head_dim 64) or 128 (head_dim 128), i.e. of 4 tiles of 8 KB of K;
 * 0 = the library's choice.
 * The workspace must be 256-byte aligned and zero-filled once before its
 * first use; every launch leaves it ready for the next (its split arrival
 * counters, the first 256 KiB, return to zero), whatever the batch and
 * max_ctx of the next call, as long as the workspace is large enough for it.
 * Split-K calls handle batch x num_kv_heads <= 65536.  Launches that may run
 * concurrently (different streams) need separate workspaces. */
size_t luc_paged_decode_workspace_size(int batch, int num_q_heads, int num_kv_heads,
                                       int head_dim, int max_ctx, int split_tokens);

/* Batched paged decode attention: flash_decoding_kernel_{64,128}
 * (src/kernels/attention.cu:4-240) as launched by
 * CudaFunctions::apply_flash_decoding (src/kernels.rs:248-320), for `batch`
 * sequences at once.  Sequence b attends with q row b (q + b*q_row_stride,
 * [Hq][head_dim]) to positions 0..positions[b] through table row b, and writes
 * out row b (out + b*out_row_stride).  max_ctx is a host-side upper bound of
 * positions[b]+1 (the reference's host `pos`, kernels.rs:266); a sequence
 * whose context exceeds it, or is empty, gets NaN outputs, as the reference
 * yields NaN for an empty context.  sm_scale is 1/sqrt(head_dim) in the
 * engine (kernels.rs:264).  Work is split into split-K chunks whose partials
 * go to `workspace` (see luc_paged_decode_workspace_size); the last chunk of a
 * sequence to finish merges them with the log-sum-exp rule, in the same
 * launch. */
int luc_paged_decode(luc_ctx* ctx, void* stream, int dtype, void* out, int64_t out_row_stride,
                     const void* q, int64_t q_row_stride, const void* k_pool, const void* v_pool,
                     const int32_t* block_tables, int table_stride, int num_blocks,
                     const int32_t* positions,
                     int batch, int max_ctx, int layer, int num_layers, int num_q_heads,
                     int num_kv_heads, int head_dim, int block_size, float sm_scale,
                     int split_tokens, void* workspace, size_t workspace_bytes);

/* One whole decode step of the attention path for a batch, in one launch:
 * per sequence b, bias + RoPE of q and k at positions[b] (in place in the qkv
 * row), the cache write of the roped k and v + v_bias at that position, and
 * paged attention over positions 0..positions[b] into out row b.  This is the
 * engine's per-layer sequence apply_rope -> KVCache::update ->
 * apply_flash_decoding (src/models.rs:505-549, src/kernels.rs:203-320,
 * src/layers/kv_cache.rs:124-173) for a batch, with the same results as
 * luc_rope_append followed by luc_paged_decode.
 * qkv rows are the engine's qkv_states rows [q (Hq*d) | k (Hkv*d) | v (Hkv*d)]
 * at qkv + b*qkv_row_stride.  Biases may be NULL.  A sequence whose context is
 * empty or exceeds max_ctx gets NaN outputs and no cache write. */
int luc_decode_step(luc_ctx* ctx, void* stream, int dtype, void* qkv, int64_t qkv_row_stride,
                    const void* q_bias, const void* k_bias, const void* v_bias,
                    const float* cos_table, const float* sin_table, void* k_pool, void* v_pool,
                    const int32_t* block_tables, int table_stride, int num_blocks,
                     const int32_t* positions,
                    int batch, int max_ctx, int layer, int num_layers, int num_q_heads,
                    int num_kv_heads, int head_dim, int block_size, float sm_scale,
                    int split_tokens, void* out, int64_t out_row_stride, void* workspace,
                    size_t workspace_bytes);

/* luc_decode_step for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * It has no counterpart in the reference (whose attention needs no
 * workspace).  The same launch and results as luc_decode_step with the same
 * arguments, except that the split-K workspace is the library's own fixed
 * scratch: a device array of LUC_SCRATCH_BYTES per GPU, held until the
 * process ends.  Every luc_init resolves its address on its device; the first
 * luc_init for a device zero-fills it, and so does any later luc_init that
 * finds the address changed (the device was reset).  Every launch leaves its
 * arrival counters at zero again, so later contexts on the device reuse it
 * as it is.  Calls whose
 * workspace (luc_paged_decode_workspace_size of the same sizes) exceeds
 * LUC_SCRATCH_BYTES fail with LUC_E_WORKSPACE before any launch.  The entry
 * point itself calls no allocator.  Every call on one GPU shares that GPU's
 * scratch: calls that overlap on one GPU (other streams, other threads, other
 * contexts on the same device) race and give undefined results; the caller
 * serialises them (one stream, in order). */
#define LUC_SCRATCH_BYTES (16u << 20)
int luc_decode_step_noalloc(luc_ctx* ctx, void* stream, int dtype, void* qkv,
                            int64_t qkv_row_stride, const void* q_bias, const void* k_bias,
                            const void* v_bias, const float* cos_table, const float* sin_table,
                            void* k_pool, void* v_pool, const int32_t* block_tables,
                            int table_stride, int num_blocks, const int32_t* positions, int batch, int max_ctx,
                            int layer, int num_layers, int num_q_heads, int num_kv_heads,
                            int head_dim, int block_size, float sm_scale, int split_tokens,
                            void* out, int64_t out_row_stride);

/* Measurement entry points; they have no counterpart in the reference and
 * compute nothing the engine uses.  luc_gather_floor reads exactly the K and V
 * page slabs a decode step over the same arguments reads (pages 0 ..
 * positions[b] / 16 of table row b, layer `layer`, every kv head), with
 * luc_paged_decode's work split and no arithmetic: its duration is the floor
 * of the decode kernel's KV stream with this cache layout.  luc_stream_read
 * reads `bytes` (a multiple of 16) contiguously from `src`.  Both write
 * `sink` (one device uint32) only if the XOR of what they read equals a fixed
 * pattern, so no load is dead. */
int luc_gather_floor(luc_ctx* ctx, void* stream, const void* k_pool, const void* v_pool,
                     const int32_t* block_tables, int table_stride, int num_blocks,
                     const int32_t* positions,
                     int batch, int max_ctx, int layer, int num_layers, int num_kv_heads,
                     int head_dim, uint32_t* sink);
int luc_stream_read(luc_ctx* ctx, void* stream, const void* src, size_t bytes, uint32_t* sink);

/* Causal prefill of packed prompts: the engine's per-token prefill loop
 * (Qwen2Model::forward_layer, src/models.rs:485-550 -- rope
 * (src/kernels/rope.cu), the cache write (src/kernels/kv_cache.cu) and
 * flash_decoding (src/kernels/attention.cu:4-176) for each prompt token in
 * turn) for whole prompts at once.  Rows cu_seqlens[b] .. cu_seqlens[b+1]-1 of
 * qkv ([q (Hq*d) | k (Hkv*d) | v (Hkv*d)] at qkv + r*qkv_row_stride) are the
 * prompt of sequence b, at positions start_pos[b] + (r - cu_seqlens[b]) of
 * table row b (cu_seqlens and start_pos are device int32 arrays of batch+1
 * and batch entries; total_rows = cu_seqlens[batch]).  Every row's q and k
 * get bias + RoPE in place, its roped k and v + v_bias go to the cache, and
 * every row attends to positions 0..its own of its sequence (the cached
 * prefix and the prompt rows up to itself); out row r = out + r*out_row_stride,
 * [Hq][head_dim].  max_ctx is a host-side upper bound of start_pos[b] plus the
 * rows of b; a sequence beyond it gets NaN outputs.  qkv must be 16-byte
 * aligned with a row stride that is a multiple of 8 elements; out 8-byte
 * aligned with a row stride that is a multiple of 4.  Biases may be NULL.  Rows whose position lies outside
 * the table row (or is negative) are left untouched, as in luc_rope_append.
 * Attention runs on bf16/fp16 MFMA (v_mfma_f32_32x32x16). */
int luc_paged_prefill(luc_ctx* ctx, void* stream, int dtype, void* qkv, int64_t qkv_row_stride,
                      const void* q_bias, const void* k_bias, const void* v_bias,
                      const float* cos_table, const float* sin_table, void* k_pool, void* v_pool,
                      const int32_t* block_tables, int table_stride, int num_blocks,
                      const int32_t* cu_seqlens,
                      const int32_t* start_pos, int batch, int total_rows, int max_ctx, int layer,
                      int num_layers, int num_q_heads, int num_kv_heads, int head_dim,
                      int block_size, float sm_scale, void* out, int64_t out_row_stride);

/* ---- The model loop's small kernels (bf16 only) ---- */

/* RMSNorm of `rows` rows of `cols` elements: out = round((x * inv) * w) with
 * inv = 1/sqrt(mean(x^2) + eps), f32 arithmetic -- rmsnorm_nvidia
 * (src/kernels/rmsnorm.cu:4-70) as called by CudaFunctions::apply_rmsnorm.
 * cols a multiple of 8, every operand 16-byte aligned; out may equal in.
 * The sum of squares has a fixed order (per thread over 16-byte chunks
 * t, t+256, ..., then a halving tree over 256 partials), so results are
 * reproducible bit for bit. */
int luc_rmsnorm(luc_ctx* ctx, void* stream, int dtype, void* out, const void* in,
                const void* weight, float eps, int rows, int cols);

/* y = x W^T (+ residual) for one row x of k elements and W row-major
 * [n][k] (bf16): y[i] = round(sum_j x[j] W[i][j] (+ residual[i])), f32
 * accumulation in a fixed order -- the m = 1 case of Qwen2Model::matmul_bf16
 * (src/models.rs:252-295, cublasGemmEx with compute type 32F), with residual
 * as its beta = 1 output (the residual adds, one rounding).  residual may
 * equal y; x may not overlap y.  k a multiple of 8 in [8, 8192]; x and W
 * 16-byte aligned.  The decode step's o and down projections and lm_head:
 * HBM-bound, every weight byte read once. */
int luc_gemv(luc_ctx* ctx, void* stream, int dtype, void* y, const void* x, const void* w,
             const void* residual, int n, int k);

/* luc_gemv of x' = luc_rmsnorm(x, norm_weight, eps) (x: one row of k), with
 * x' formed in registers and never stored: the same bits as luc_rmsnorm then
 * luc_gemv.  Replaces apply_rmsnorm + matmul_bf16 of one row
 * (src/models.rs:455-482 for q/k/v, :568-590 for gate/up).  norm_weight
 * 16-byte aligned. */
int luc_rmsnorm_gemv(luc_ctx* ctx, void* stream, int dtype, void* y, const void* x,
                     const void* norm_weight, float eps, const void* w, const void* residual, int n,
                     int k);

/* act = round(silu(g) * u) (intermediate values) with [g | u] the bf16 rows
 * x' W^T of W = [gate rows; up rows] ([2 * intermediate][k], the reference's
 * gate_up_proj) and x' = luc_rmsnorm(x, norm_weight, eps), or x' = x when
 * norm_weight is NULL: the same bits as luc_rmsnorm, luc_gemv into [g | u]
 * and luc_silu_mul, without the [g | u] row.  Replaces apply_rmsnorm +
 * matmul_bf16 + apply_activation_fused of one row (src/models.rs:568-590,
 * :671).  x and W 16-byte aligned; act may not overlap x. */
int luc_gate_up_silu(luc_ctx* ctx, void* stream, int dtype, void* act, const void* x,
                     const void* norm_weight, float eps, const void* w, int intermediate, int k);

/* In place on rows [gate (intermediate) | up (intermediate)]:
 * gate = round(silu(gate) * up), silu(g) = g / (1 + exp(-g)) in f32 --
 * silu_and_mul_fused_kernel (src/kernels/activation.cu:6-29).
 * intermediate a multiple of 8, gate_up 16-byte aligned. */
int luc_silu_mul(luc_ctx* ctx, void* stream, int dtype, void* gate_up, int rows,
                 int intermediate);

/* out[t] = table[ids[t]] for num_tokens device ids -- batched_embedding_kernel
 * (src/kernels/embedding.cu:3-39).  An id at or past `vocab` gives a NaN row
 * (the reference reads past its table).  hidden a multiple of 8, out and
 * table 16-byte aligned. */
int luc_embedding(luc_ctx* ctx, void* stream, int dtype, void* out, const void* table,
                  const uint32_t* ids, int num_tokens, int vocab, int hidden);

/* *out_idx = index of the largest of n bf16 logits -- argmax_kernel
 * (src/kernels/sampling.cu:16-46): values <= -1e30 and NaN never win (then
 * 0xffffffff, the reference's -1); equal values go to the smallest index. */
int luc_argmax(luc_ctx* ctx, void* stream, int dtype, const void* logits, int n, uint32_t* out_idx);

/* Top-k / top-p sampling of one bf16 logits row -- CudaFunctions::
 * apply_sort_and_sample (src/kernels.rs:346-498) with its kernels top_k_filter
 * and fused_top_p_sample_<top_k> (src/kernels/sampling_optimized.cu:27-236):
 *  - candidates: the largest top_k/32 logits of each of 32 partitions
 *    [p*vocab/32, (p+1)*vocab/32), values <= -1e30 and NaN excluded (a
 *    partition short of them pads with (start - 1, -1e30)); equal values in
 *    the reference's order;
 *  - sorted by the reference's bitonic network (value, descending) and written
 *    back to sort_buffer as top_k pairs (int32 index, f32 value);
 *  - prob = exp(v - v_max) / sum, cdf = inclusive sum; cutoff = the cdf of the
 *    candidate whose [cdf - prob, cdf] holds top_p (1 when none does);
 *    *out_idx = the index of the candidate whose interval holds
 *    rand_val * cutoff, left unwritten when none does (rand_val = 0).
 * top_k is the sampler's normalised value (src/sampler.rs:19-23): a power of
 * two in [32, 1024], else LUC_E_UNSUPPORTED (the reference's "Unsupported
 * candidate size").  vocab in [32, 524288].  sort_buffer is caller-owned
 * device memory of >= 8*top_k bytes (the engine's 8 KB sort_buffer,
 * src/models.rs:171-174), else LUC_E_WORKSPACE.  Two launches on `stream`. */
int luc_sort_and_sample(luc_ctx* ctx, void* stream, int dtype, const void* logits, int vocab,
                        float top_p, int top_k, float rand_val, void* sort_buffer,
                        size_t sort_buffer_bytes, uint32_t* out_idx);

/* ---- Multi-sequence page allocator (host only: no GPU call, no ctx) ------
 * Generalises KVCache's free list and prepare_for_step
 * (src/layers/kv_cache.rs:73-76, 106-122) from one sequence to max_seqs rows
 * of a block table over one pool of num_blocks pages of LUC_BLOCK_SIZE tokens.
 * The free list is LIFO and starts as [num_blocks-1, ..., 0], so a fresh
 * allocator hands out pages 0, 1, 2, ... as the reference does.  Calls on
 * one allocator must not overlap (the caller serialises them). */
typedef struct luc_blocks luc_blocks;

int luc_blocks_create(int num_blocks, int max_seqs, int max_blocks_per_seq, luc_blocks** out);
void luc_blocks_destroy(luc_blocks* bm);

/* Give sequence `seq` pages for positions [0, num_tokens): as many pages as
 * that needs beyond those it holds (prepare_for_step adds one per call).
 * Never shrinks.  LUC_E_NOMEM when the free list is short (the reference
 * panics), LUC_E_INVALID past max_blocks_per_seq; either way nothing changes. */
int luc_blocks_reserve(luc_blocks* bm, int seq, int num_tokens);

/* The same for n distinct sequences, all or nothing over the batch. */
int luc_blocks_reserve_batch(luc_blocks* bm, int n, const int32_t* seqs, const int32_t* num_tokens);

/* Return every page of `seq` to the free list, last page first (a release
 * then a reserve with nothing in between gives back the same pages in the
 * same order).  The reference never frees pages. */
int luc_blocks_release(luc_blocks* bm, int seq);

/* Free pages in the pool / pages held by `seq` (negative status on error). */
int luc_blocks_num_free(const luc_blocks* bm);
int luc_blocks_num_pages(const luc_blocks* bm, int seq);

/* Rows [first_seq, first_seq + n) of the block table into host memory
 * `table` (row stride `stride` >= max_blocks_per_seq, int32): the held pages,
 * then 0 (the reference's block_table is zero-initialised).  The caller
 * copies it to the device, as prepare_for_step does with memcpy_htod. */
int luc_blocks_table(const luc_blocks* bm, int first_seq, int n, int32_t* table, int stride);

#ifdef __cplusplus
}
#endif
#endif /* LUC_ATTN_H */
