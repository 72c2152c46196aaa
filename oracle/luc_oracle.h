/*
 * luc_oracle.h -- CPU restatement of lucciola-rs's paged-attention path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (the HIP kernels, the
 * C-ABI library, the host mirror) may link, load or call this code.  It is the
 * reference for tests, the smoke check and the CPU-baseline leg of the benchmark, which use
 * it to compute what the reference computes on the same inputs.
 *
 * Storage is 16-bit (bf16 or fp16, selected by `dtype`), passed as uint16_t
 * bit patterns.  All arithmetic is f32, in the order the reference's CUDA
 * kernels use; see each function for the reference file:line it restates.
 */
#ifndef LUC_ORACLE_H
#define LUC_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { ORC_BF16 = 0, ORC_F16 = 1 };

/* Scalar conversions (RNE), written from the IEEE binary16 / bfloat16 formats. */
float    orc_bf16_to_f32(uint16_t h);
uint16_t orc_f32_to_bf16(float f);
float    orc_f16_to_f32(uint16_t h);
uint16_t orc_f32_to_f16(float f);
void     orc_convert_f32_to_storage(const float* src, uint16_t* dst, int64_t n, int dtype);
void     orc_convert_storage_to_f32(const uint16_t* src, float* dst, int64_t n, int dtype);

/* RopeCache::new -- src/layers/rope.rs:11-40.  cos/sin are [max_pos][head_dim/2]. */
void orc_rope_table(float* cos_out, float* sin_out, int max_pos, int head_dim,
                    float base, float scale_factor /* <= 0: none (1.0) */);

/* rope kernel -- src/kernels/rope.cu:3-54.  One token, in place on q [Hq,d] and
 * k [Hkv,d].  Biases may be NULL (the engine then passes zeros,
 * src/utils.rs:101-110, so NULL means "add 0.0f"). */
void orc_rope(uint16_t* q, const uint16_t* q_bias, uint16_t* k, const uint16_t* k_bias,
              const float* cos_t, const float* sin_t, int pos, int head_dim,
              int num_q_heads, int num_kv_heads, int dtype);

/* update_kv_cache_kernel -- src/kernels/kv_cache.cu:3-59.  Pool layout
 * [phys_block][num_layers][Hkv][block_size][head_dim]. */
void orc_kv_update(uint16_t* k_pool, uint16_t* v_pool, const uint16_t* new_k,
                   const uint16_t* new_v, const uint16_t* v_bias, const int32_t* block_table,
                   int layer, int pos, int num_layers, int num_kv_heads, int head_dim,
                   int block_size, int dtype);

/* Pool element offset of (token position, kv head, dim 0) -- the address
 * arithmetic of src/kernels/kv_cache.cu:24-48 and src/kernels/attention.cu:71-87. */
int64_t orc_slot_offset(const int32_t* block_table, int pos, int layer, int kv_head,
                        int num_layers, int num_kv_heads, int head_dim, int block_size);

/* flash_decoding_impl<D> -- src/kernels/attention.cu:4-176, launched by
 * src/kernels.rs:248-320 with 1024 threads (32 partitions).  One sequence,
 * attends to tokens 0..pos.  q [Hq,d] -> out [Hq,d]. */
void orc_flash_decoding(uint16_t* out, const uint16_t* q, const uint16_t* k_pool,
                        const uint16_t* v_pool, const int32_t* block_table, int layer,
                        int num_q_heads, int num_kv_heads, int head_dim, int pos,
                        float sm_scale, int block_size, int num_layers, int dtype);

/* Batched decode (src/models.rs:711-763 has no batch dimension; a batch is the
 * reference applied to each sequence b with its own table row and position).
 * q/out rows are strided (elements); tables are [B][table_stride]. */
void orc_decode_batch(uint16_t* out, int64_t out_stride, const uint16_t* q, int64_t q_stride,
                      const uint16_t* k_pool, const uint16_t* v_pool,
                      const int32_t* block_tables, int table_stride, const int32_t* positions,
                      int batch, int layer, int num_q_heads, int num_kv_heads, int head_dim,
                      float sm_scale, int block_size, int num_layers, int dtype, int num_threads);

/* One decode step of the attention path for a batch: per sequence, rope(q,k)
 * at positions[b], cache write, attention (src/models.rs:485-550 with
 * seq_len == 1).  qkv rows are [q | k | v] with stride qkv_stride. */
void orc_decode_step(uint16_t* out, int64_t out_stride, uint16_t* qkv, int64_t qkv_stride,
                     const uint16_t* q_bias, const uint16_t* k_bias, const uint16_t* v_bias,
                     const float* cos_t, const float* sin_t, uint16_t* k_pool, uint16_t* v_pool,
                     const int32_t* block_tables, int table_stride, const int32_t* positions,
                     int batch, int layer, int num_q_heads, int num_kv_heads, int head_dim,
                     float sm_scale, int block_size, int num_layers, int dtype, int num_threads);

/* Prefill of one or more prompts -- src/models.rs:485-550 with seq_len > 1:
 * for t in 0..S: rope(row t) at cache_pos+t, cache write, attention at
 * cache_pos+t.  Sequences are packed: rows cu_seqlens[b]..cu_seqlens[b+1]-1
 * of qkv belong to sequence b, which starts at start_pos[b] and uses table row b. */
void orc_prefill(uint16_t* out, int64_t out_stride, uint16_t* qkv, int64_t qkv_stride,
                 const uint16_t* q_bias, const uint16_t* k_bias, const uint16_t* v_bias,
                 const float* cos_t, const float* sin_t, uint16_t* k_pool, uint16_t* v_pool,
                 const int32_t* block_tables, int table_stride, const int32_t* cu_seqlens,
                 const int32_t* start_pos, int batch, int layer, int num_q_heads,
                 int num_kv_heads, int head_dim, float sm_scale, int block_size,
                 int num_layers, int dtype, int num_threads);

/* ---- The model loop's small operations (bf16 storage) ---- */

/* RMSNorm -- src/kernels/rmsnorm.cu:4-70: out = bf16((x * inv) * w),
 * inv = 1 / sqrt(sum(x^2) / n + eps).  The sum follows one fixed order: 256
 * partials, partial t = fma-accumulated x^2 over elements 8c..8c+7 for chunks
 * c = t, t + 256, ..., then a halving tree (p[i] += p[i + h], h = 128..1).
 * out may equal in. */
void orc_rmsnorm(uint16_t* out, const uint16_t* in, const uint16_t* weight, float eps, int rows,
                 int cols);

/* In place on rows [gate | up] of 2*inter elements: gate = bf16(silu(g) * u),
 * silu(g) = g / (1 + exp(-g)) in f32 -- src/kernels/activation.cu:6-29. */
void orc_silu_mul(uint16_t* gate_up, int rows, int inter);

/* Greedy argmax of n bf16 values -- src/kernels/sampling.cu:16-46: values
 * <= -1e30 and NaN never win (-1 when none does); ties go to the smallest
 * index. */
int orc_argmax(const uint16_t* x, int n);

/* ---- Top-k / top-p sampling (src/kernels/sampling_optimized.cu) ---- */

/* top_k_filter (sampling_optimized.cu:27-112) as launched by
 * apply_sort_and_sample (src/kernels.rs:366-386): 32 partitions
 * [p*vocab/32, (p+1)*vocab/32), each of 256 threads; k_per_block rounds of a
 * strided per-thread scan (strict >, from {-1, -1e30}), a shfl_down max tree
 * over each warp's 32 lanes and one over the 8 warp results; the winner's
 * slot is set to -1e30.  Candidate p*k_per_block + k = (start + key, value).
 * A round with nothing above -1e30 gives (start - 1, -1e30).  Simulated
 * thread by thread, so ties resolve as the reference's trees resolve them. */
void orc_topk_filter(const uint16_t* logits, int vocab, int k_per_block, int32_t* keys,
                     float* vals);

/* The bitonic compare-exchange network of fused_top_p_sample_impl
 * (sampling_optimized.cu:130-152) over n (a power of two) pairs, by value,
 * descending; equal values keep whatever order the network leaves. */
void orc_bitonic_desc(int32_t* keys, float* vals, int n);

/* The sample step of fused_top_p_sample_impl (sampling_optimized.cu:154-187)
 * on n sorted values: prob = exp(v - v[0]) / sum, cdf = inclusive sum of prob,
 * cutoff = the first cdf whose interval [cdf - prob, cdf] holds top_p (1.0 if
 * none), and the first position whose interval holds rand_val * cutoff
 * (-1 if none: the reference then leaves the output unwritten).  prob and cdf
 * (n floats each) are filled as intermediate results. */
int orc_top_p_pick(const float* vals, int n, float top_p, float rand_val, float* prob, float* cdf);

#ifdef __cplusplus
}
#endif
#endif
