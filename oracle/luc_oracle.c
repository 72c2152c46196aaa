/*
 * luc_oracle.c -- CPU restatement of lucciola-rs's paged-attention path.
 *
 * TEST INFRASTRUCTURE ONLY: what the product is tested against, never the product.  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.
 *
 * Built with -ffp-contract=off so every multiply and add rounds where written.
 * Where the reference's CUDA source has a multiply-add that NVRTC contracts by
 * default (build.rs:32-40 uses default CompileOptions, i.e. --fmad=true), the
 * restatement writes fmaf() explicitly; where the contraction is ambiguous the
 * choice is noted.  Those choices, CUDA's expf versus glibc's expf, and the
 * summation order of CUB's BlockReduce/BlockScan in the top-p draw (CUB is not
 * in the reference's sources; orc_top_p_pick sums in index order) are the
 * parts no available reference output pins: parity unpinned.
 *
 * ORC_MUTANT (compile-time, 0 = off) plants one known mistake; the test suite
 * builds each mutant and checks that its pinning checks reject it.
 */
#include "luc_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#ifndef ORC_MUTANT
#define ORC_MUTANT 0
#endif

/* ------------------------------------------------------------------ */
/* Conversions                                                         */
/* ------------------------------------------------------------------ */

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

float orc_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

uint16_t orc_f32_to_bf16(float f) {
    uint32_t u = f2u(f);
    if ((u & 0x7fffffffu) > 0x7f800000u)          /* NaN: keep sign, force quiet */
        return (uint16_t)((u >> 16) | 0x0040u);
    uint32_t lsb = (u >> 16) & 1u;                 /* round to nearest, ties to even */
    u += 0x7fffu + lsb;
    return (uint16_t)(u >> 16);
}

float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t man = h & 0x3ffu;
    if (exp == 0x1fu)                              /* inf / NaN */
        return u2f(sign | 0x7f800000u | (man << 13));
    if (exp == 0) {
        if (man == 0) return u2f(sign);
        /* subnormal: man * 2^-24, exact in f32 */
        float v = (float)man * 5.9604644775390625e-08f;
        return sign ? -v : v;
    }
    return u2f(sign | ((exp + 112u) << 23) | (man << 13));
}

uint16_t orc_f32_to_f16(float f) {
    uint32_t x = f2u(f);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    uint32_t ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu));
    if (ax == 0x7f800000u) return (uint16_t)(sign | 0x7c00u);
    uint32_t e = ax >> 23;                         /* biased f32 exponent */
    uint32_t m = (ax & 0x7fffffu) | 0x800000u;     /* 24-bit significand */
    if (e < 113u) {                                /* |f| < 2^-14: f16 subnormal or zero */
        if (e == 0) return sign;                   /* f32 zero/subnormal -> 0 */
        uint32_t s = 126u - e;                     /* value / 2^-24 = m >> s */
        if (s > 24u) return sign;
        uint32_t q = m >> s;
        uint32_t rem = m & ((1u << s) - 1u);
        uint32_t half = 1u << (s - 1u);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t r = ((e - 112u) << 10) | ((m >> 13) & 0x3ffu);
    uint32_t rem = m & 0x1fffu;
    if (ORC_MUTANT != 10 && (rem > 0x1000u || (rem == 0x1000u && (r & 1u)))) r++;
    if (r >= 0x7c00u) return (uint16_t)(sign | 0x7c00u);   /* overflow -> inf */
    return (uint16_t)(sign | r);
}

static inline float ld(uint16_t h, int dtype) {
    return dtype == ORC_F16 ? orc_f16_to_f32(h) : orc_bf16_to_f32(h);
}
static inline uint16_t st(float f, int dtype) {
    return dtype == ORC_F16 ? orc_f32_to_f16(f) : orc_f32_to_bf16(f);
}

void orc_convert_f32_to_storage(const float* src, uint16_t* dst, int64_t n, int dtype) {
    for (int64_t i = 0; i < n; ++i) dst[i] = st(src[i], dtype);
}
void orc_convert_storage_to_f32(const uint16_t* src, float* dst, int64_t n, int dtype) {
    for (int64_t i = 0; i < n; ++i) dst[i] = ld(src[i], dtype);
}

/* ------------------------------------------------------------------ */
/* RoPE table: src/layers/rope.rs:21-31                                 */
/* ------------------------------------------------------------------ */
void orc_rope_table(float* cos_out, float* sin_out, int max_pos, int head_dim, float base,
                    float scale_factor) {
    const int half = head_dim / 2;
    const float scale = scale_factor > 0.0f ? scale_factor : 1.0f;     /* rope.rs:21 */
    for (int pos = 0; pos < max_pos; ++pos) {
        for (int i = 0; i < half; ++i) {
            float t = (float)pos / scale;                                /* rope.rs:26 */
            float theta = t / powf(base, (float)(2 * i) / (float)head_dim); /* rope.rs:27 */
            cos_out[(int64_t)pos * half + i] = cosf(theta);              /* rope.rs:28 */
            sin_out[(int64_t)pos * half + i] = sinf(theta);              /* rope.rs:29 */
        }
    }
}

/* ------------------------------------------------------------------ */
/* rope kernel: src/kernels/rope.cu:3-53                               */
/* ------------------------------------------------------------------ */
static inline void rotate_pair(uint16_t* x, const uint16_t* bias, int i1, int i2, float c,
                               float s, int dtype) {
    float b1 = bias ? ld(bias[i1], dtype) : 0.0f;                       /* rope.cu:32-33 */
    float b2 = bias ? ld(bias[i2], dtype) : 0.0f;
    float v1 = ld(x[i1], dtype) + (ORC_MUTANT == 2 ? 0.0f : b1);         /* rope.cu:34-35 */
    float v2 = ld(x[i2], dtype) + (ORC_MUTANT == 2 ? 0.0f : b2);
    /* rope.cu:38-39.  Written uncontracted: each product rounds, then the
     * sum rounds (NVRTC may fuse one product; that choice is unpinned). */
    float a = v1 * c, b = v2 * s;
    float e = v1 * s, f = v2 * c;
#if ORC_MUTANT == 2
    x[i1] = st(a - b + b1, dtype);
    x[i2] = st(e + f + b2, dtype);
#elif ORC_MUTANT == 3
    x[i1] = st(a + b, dtype);
    x[i2] = st(e - f, dtype);
#else
    x[i1] = st(a - b, dtype);
    x[i2] = st(e + f, dtype);
#endif
}

void orc_rope(uint16_t* q, const uint16_t* q_bias, uint16_t* k, const uint16_t* k_bias,
              const float* cos_t, const float* sin_t, int pos, int head_dim, int num_q_heads,
              int num_kv_heads, int dtype) {
    const int half = head_dim / 2;
    for (int idx = 0; idx < num_q_heads * half; ++idx) {                /* rope.cu:15-23 */
        int head = idx / half, dim = idx % half;
        float c = cos_t[(int64_t)pos * half + dim];                      /* rope.cu:25-26 */
        float s = sin_t[(int64_t)pos * half + dim];
        int i1 = head * head_dim + dim, i2 = i1 + half;
        rotate_pair(q, q_bias, i1, i2, c, s, dtype);
        if (head < num_kv_heads)                                         /* rope.cu:42-52 */
            rotate_pair(k, k_bias, i1, i2, c, s, dtype);
    }
}

/* ------------------------------------------------------------------ */
/* Cache write: src/kernels/kv_cache.cu:3-59                           */
/* ------------------------------------------------------------------ */
int64_t orc_slot_offset(const int32_t* block_table, int pos, int layer, int kv_head,
                        int num_layers, int num_kv_heads, int head_dim, int block_size) {
    int logical = pos / block_size;                                      /* kv_cache.cu:24 */
    int offset = pos % block_size;                                       /* kv_cache.cu:25 */
    int64_t phys = block_table[logical];                                 /* kv_cache.cu:28 */
    int64_t stride_block = (int64_t)num_layers * num_kv_heads * block_size * head_dim;
    int64_t stride_layer = (int64_t)num_kv_heads * block_size * head_dim;
    int64_t stride_head = (int64_t)block_size * head_dim;
#if ORC_MUTANT == 4
    return phys * stride_block + (int64_t)layer * stride_layer + (int64_t)kv_head * head_dim +
           (int64_t)offset * stride_head;
#else
    return phys * stride_block + (int64_t)layer * stride_layer + (int64_t)kv_head * stride_head +
           (int64_t)offset * head_dim;                                   /* kv_cache.cu:45-48 */
#endif
}

void orc_kv_update(uint16_t* k_pool, uint16_t* v_pool, const uint16_t* new_k,
                   const uint16_t* new_v, const uint16_t* v_bias, const int32_t* block_table,
                   int layer, int pos, int num_layers, int num_kv_heads, int head_dim,
                   int block_size, int dtype) {
    for (int h = 0; h < num_kv_heads; ++h) {
        int64_t base = orc_slot_offset(block_table, pos, layer, h, num_layers, num_kv_heads,
                                       head_dim, block_size);
        for (int d = 0; d < head_dim; ++d) {
            int idx = h * head_dim + d;                                  /* kv_cache.cu:50 */
            k_pool[base + d] = new_k[idx];                               /* kv_cache.cu:53 bit copy */
            float v = ld(new_v[idx], dtype);                             /* kv_cache.cu:56-58 */
            float b = (v_bias && ORC_MUTANT != 6) ? ld(v_bias[idx], dtype) : 0.0f;
            v_pool[base + d] = st(v + b, dtype);
        }
    }
}

/* ------------------------------------------------------------------ */
/* Decode attention: src/kernels/attention.cu:4-176                     */
/* ------------------------------------------------------------------ */
#define ORC_WARPS 32   /* kernels.rs:269: 1024 threads -> 32 warps */
#define ORC_LANES 32
#define ORC_MAXD 256

/* One q-head: returns the f32 result before the final rounding in o_out. */
static void attend_head(float* o_out, const uint16_t* q_head, const uint16_t* k_pool,
                        const uint16_t* v_pool, const int32_t* table, int layer, int kv_head,
                        int num_kv_heads, int head_dim, int pos, float sm_scale, int block_size,
                        int num_layers, int dtype) {
    float sq[ORC_MAXD];
    for (int i = 0; i < head_dim; ++i) sq[i] = ld(q_head[i], dtype);  /* attention.cu:49-51 */

    float pm[ORC_WARPS], pl[ORC_WARPS];
    static __thread float po[ORC_WARPS][ORC_MAXD];

    const int64_t stride_block = (int64_t)num_layers * num_kv_heads * block_size * head_dim;
    const int64_t stride_layer = (int64_t)num_kv_heads * block_size * head_dim;
    const int64_t stride_head = (int64_t)block_size * head_dim;
    const int64_t layer_head = (int64_t)layer * stride_layer + (int64_t)kv_head * stride_head;

    for (int w = 0; w < ORC_WARPS; ++w) {
        float m = -1e20f, l = 0.0f;                                      /* attention.cu:61-62 */
        float* o = po[w];
        for (int i = 0; i < head_dim; ++i) o[i] = 0.0f;
        for (int t = w; ORC_MUTANT == 7 ? t < pos : t <= pos; t += ORC_WARPS) { /* attention.cu:80 */
            int64_t phys = table[t / block_size];
            int64_t off = phys * stride_block + layer_head + (int64_t)(t % block_size) * head_dim;
            /* attention.cu:93-96: lane j sums dims j, j+32, ... (fused mul-add) */
            float lane[ORC_LANES];
            for (int j = 0; j < ORC_LANES; ++j) {
                float s = 0.0f;
                for (int i = j; i < head_dim; i += ORC_LANES)
                    s = fmaf(sq[i], ld((ORC_MUTANT == 8 ? v_pool : k_pool)[off + i], dtype), s);
                lane[j] = s;
            }
            /* attention.cu:99-102: shfl_down tree 16,8,4,2,1; lane 0's value */
            for (int step = ORC_LANES / 2; step > 0; step /= 2)
                for (int j = 0; j < step; ++j) lane[j] += lane[j + step];
            float score = ORC_MUTANT == 1 ? lane[0] : lane[0] * sm_scale; /* attention.cu:103 */
            float m_prev = m;                                            /* attention.cu:106-111 */
            m = fmaxf(m_prev, score);
            float exp_m = expf(m_prev - m);
            float exp_s = expf(score - m);
            l = fmaf(l, exp_m, exp_s);
            for (int i = 0; i < head_dim; ++i) {                         /* attention.cu:115-119 */
                float v = ld(v_pool[off + i], dtype);
                o[i] = fmaf(o[i], exp_m, v * exp_s);
            }
        }
        pm[w] = m;
        pl[w] = l;
    }
    /* attention.cu:140-174: warp 0 merges the 32 partitions */
    float gm = -1e20f;
    for (int w = 0; w < ORC_WARPS; ++w) gm = fmaxf(gm, pm[w]);
    float gl = 0.0f;
    for (int w = 0; w < ORC_WARPS; ++w) {
        if (pm[w] <= -1e19f) continue;
        gl = fmaf(pl[w], ORC_MUTANT == 5 ? 1.0f : expf(pm[w] - gm), gl);
    }
    for (int i = 0; i < head_dim; ++i) {
        float so = 0.0f;
        for (int w = 0; w < ORC_WARPS; ++w) {
            if (pm[w] <= -1e19f) continue;
            so = fmaf(po[w][i], expf(pm[w] - gm), so);
        }
        o_out[i] = so / gl;
    }
}

void orc_flash_decoding(uint16_t* out, const uint16_t* q, const uint16_t* k_pool,
                        const uint16_t* v_pool, const int32_t* block_table, int layer,
                        int num_q_heads, int num_kv_heads, int head_dim, int pos,
                        float sm_scale, int block_size, int num_layers, int dtype) {
    float o[ORC_MAXD];
    const int group = num_q_heads / num_kv_heads;                        /* attention.cu:23 */
    for (int h = 0; h < num_q_heads; ++h) {
        attend_head(o, q + (int64_t)h * head_dim, k_pool, v_pool, block_table, layer,
                    ORC_MUTANT == 9 ? h % num_kv_heads : h / group, num_kv_heads, head_dim, pos, sm_scale, block_size, num_layers,
                    dtype);
        for (int i = 0; i < head_dim; ++i)
            out[(int64_t)h * head_dim + i] = st(o[i], dtype);           /* attention.cu:173 */
    }
}

static void set_threads(int num_threads) {
#ifdef _OPENMP
    if (num_threads > 0) omp_set_num_threads(num_threads);
#else
    (void)num_threads;
#endif
}

void orc_decode_batch(uint16_t* out, int64_t out_stride, const uint16_t* q, int64_t q_stride,
                      const uint16_t* k_pool, const uint16_t* v_pool,
                      const int32_t* block_tables, int table_stride, const int32_t* positions,
                      int batch, int layer, int num_q_heads, int num_kv_heads, int head_dim,
                      float sm_scale, int block_size, int num_layers, int dtype,
                      int num_threads) {
    set_threads(num_threads);
    const int group = num_q_heads / num_kv_heads;
    const int64_t items = (int64_t)batch * num_q_heads;
#pragma omp parallel for schedule(dynamic, 1)
    for (int64_t it = 0; it < items; ++it) {
        int b = (int)(it / num_q_heads), h = (int)(it % num_q_heads);
        float o[ORC_MAXD];
        attend_head(o, q + b * q_stride + (int64_t)h * head_dim, k_pool, v_pool,
                    block_tables + (int64_t)b * table_stride, layer, ORC_MUTANT == 9 ? h % num_kv_heads : h / group, num_kv_heads,
                    head_dim, positions[b], sm_scale, block_size, num_layers, dtype);
        for (int i = 0; i < head_dim; ++i)
            out[b * out_stride + (int64_t)h * head_dim + i] = st(o[i], dtype);
    }
}

void orc_decode_step(uint16_t* out, int64_t out_stride, uint16_t* qkv, int64_t qkv_stride,
                     const uint16_t* q_bias, const uint16_t* k_bias, const uint16_t* v_bias,
                     const float* cos_t, const float* sin_t, uint16_t* k_pool, uint16_t* v_pool,
                     const int32_t* block_tables, int table_stride, const int32_t* positions,
                     int batch, int layer, int num_q_heads, int num_kv_heads, int head_dim,
                     float sm_scale, int block_size, int num_layers, int dtype,
                     int num_threads) {
    const int64_t q_dim = (int64_t)num_q_heads * head_dim;
    const int64_t kv_dim = (int64_t)num_kv_heads * head_dim;
    /* models.rs:505-534: rope then cache write, per sequence */
    for (int b = 0; b < batch; ++b) {
        uint16_t* row = qkv + b * qkv_stride;
        const int32_t* table = block_tables + (int64_t)b * table_stride;
        orc_rope(row, q_bias, row + q_dim, k_bias, cos_t, sin_t, positions[b], head_dim,
                 num_q_heads, num_kv_heads, dtype);
        orc_kv_update(k_pool, v_pool, row + q_dim, row + q_dim + kv_dim, v_bias, table, layer,
                      positions[b], num_layers, num_kv_heads, head_dim, block_size, dtype);
    }
    /* models.rs:536-549 */
    orc_decode_batch(out, out_stride, qkv, qkv_stride, k_pool, v_pool, block_tables,
                     table_stride, positions, batch, layer, num_q_heads, num_kv_heads, head_dim,
                     sm_scale, block_size, num_layers, dtype, num_threads);
}

void orc_prefill(uint16_t* out, int64_t out_stride, uint16_t* qkv, int64_t qkv_stride,
                 const uint16_t* q_bias, const uint16_t* k_bias, const uint16_t* v_bias,
                 const float* cos_t, const float* sin_t, uint16_t* k_pool, uint16_t* v_pool,
                 const int32_t* block_tables, int table_stride, const int32_t* cu_seqlens,
                 const int32_t* start_pos, int batch, int layer, int num_q_heads,
                 int num_kv_heads, int head_dim, float sm_scale, int block_size,
                 int num_layers, int dtype, int num_threads) {
    set_threads(num_threads);
    const int64_t q_dim = (int64_t)num_q_heads * head_dim;
    const int64_t kv_dim = (int64_t)num_kv_heads * head_dim;
    /* models.rs:486-534, serial per token.  The attention of token t reads
     * only cache slots <= its own position, all written by then, so the
     * attention calls can run after all writes without changing any value. */
    for (int b = 0; b < batch; ++b) {
        const int32_t* table = block_tables + (int64_t)b * table_stride;
        for (int r = cu_seqlens[b]; r < cu_seqlens[b + 1]; ++r) {
            int pos = start_pos[b] + (r - cu_seqlens[b]);
            uint16_t* row = qkv + r * qkv_stride;
            orc_rope(row, q_bias, row + q_dim, k_bias, cos_t, sin_t, pos, head_dim,
                     num_q_heads, num_kv_heads, dtype);
            orc_kv_update(k_pool, v_pool, row + q_dim, row + q_dim + kv_dim, v_bias, table,
                          layer, pos, num_layers, num_kv_heads, head_dim, block_size, dtype);
        }
    }
    const int group = num_q_heads / num_kv_heads;
    const int64_t total_rows = cu_seqlens[batch];
    const int64_t items = total_rows * num_q_heads;
#pragma omp parallel for schedule(dynamic, 4)
    for (int64_t it = 0; it < items; ++it) {
        int64_t r = it / num_q_heads;
        int h = (int)(it % num_q_heads);
        int b = 0;
        while (cu_seqlens[b + 1] <= r) ++b;
        int pos = start_pos[b] + (int)(r - cu_seqlens[b]);
        float o[ORC_MAXD];
        attend_head(o, qkv + r * qkv_stride + (int64_t)h * head_dim, k_pool, v_pool,
                    block_tables + (int64_t)b * table_stride, layer, ORC_MUTANT == 9 ? h % num_kv_heads : h / group, num_kv_heads,
                    head_dim, ORC_MUTANT == 17 ? pos + 1 : pos, sm_scale, block_size, num_layers, dtype);
        for (int i = 0; i < head_dim; ++i)
            out[r * out_stride + (int64_t)h * head_dim + i] = st(o[i], dtype);
    }
}

/* ------------------------------------------------------------------ */
/* Model loop operations: src/kernels/{rmsnorm,activation,sampling}.cu */
/* ------------------------------------------------------------------ */
/* RMSNorm in the fixed order of this library's kernel (model_ops.hip luc_rmsnorm_bf16:
 * 256 threads, fma over each thread's 16-byte chunks, halving tree, 1/sqrtf), so that
 * the GPU result can be compared bit for bit; the formula is rmsnorm.cu's
 * (y = round((x * inv) * w), inv = 1/sqrt(mean(x^2) + eps), rmsnorm.cu:40, :63-64).
 * The reference's own order is not this one: per-thread x*x + y*y pair sums
 * (rmsnorm.cu:19-29), cub::BlockReduce<float, 1024> (:32-35) and rsqrtf (:40) --
 * parity unpinned; tests/pins.py holds this function to the f64 formula within half
 * a bf16 unit. */
void orc_rmsnorm(uint16_t* out, const uint16_t* in, const uint16_t* weight, float eps, int rows,
                 int cols) {
    enum { T = 256 };
    const int chunks = cols / 8;
    for (int r = 0; r < rows; ++r) {
        const uint16_t* x = in + (int64_t)r * cols;
        float part[T];
        for (int t = 0; t < T; ++t) {
            float s = 0.0f;
            for (int c = t; c < chunks; c += T)
                for (int e = 0; e < 8; ++e) {
                    const float f = orc_bf16_to_f32(x[8 * c + e]);
                    s = fmaf(f, f, s);
                }
            part[t] = s;
        }
        for (int h = T / 2; h > 0; h >>= 1)
            for (int t = 0; t < h; ++t) part[t] = part[t] + part[t + h];   /* halving tree */
        const float ms = part[0] / (float)(ORC_MUTANT == 11 ? cols - 1 : cols);
        const float inv = 1.0f / sqrtf(ms + eps);           /* rmsnorm.cu:40 has rsqrtf */
        uint16_t* y = out + (int64_t)r * cols;
        for (int i = 0; i < cols; ++i) {
            const float f = orc_bf16_to_f32(x[i]) * inv;                   /* rmsnorm.cu:63-64 */
            y[i] = orc_f32_to_bf16(f * orc_bf16_to_f32(weight[i]));
        }
    }
}

void orc_silu_mul(uint16_t* gate_up, int rows, int inter) {
    for (int r = 0; r < rows; ++r) {
        uint16_t* g = gate_up + (int64_t)r * 2 * inter;
        const uint16_t* u = g + inter;
        for (int c = 0; c < inter; ++c) {
            const float x = orc_bf16_to_f32(g[c]);
            const float s = x / (1.0f + expf(ORC_MUTANT == 12 ? x : -x));                         /* activation.cu:4 */
            g[c] = orc_f32_to_bf16(s * orc_bf16_to_f32(u[c]));              /* activation.cu:24-27 */
        }
    }
}

/* argmax_kernel (sampling.cu:16-46) as launched by apply_argmax (kernels.rs:322-344,
 * one block of 1024 threads): thread t keeps the first largest of x[t], x[t + 1024],
 * ... above -1e30 (strict >, sampling.cu:28-34); the block reduction with ArgMaxOp
 * (b if b.value > a.value, else a: sampling.cu:9-14) keeps the lower thread's pair on
 * ties -- CUB's BlockReduce combines warp lanes and then warps in increasing order
 * (cub/block/block_reduce.cuh, not vendored; see the parity notes). */
int orc_argmax(const uint16_t* x, int n) {
    enum { THREADS = 1024 };
    float best = -1e30f;                                                   /* sampling.cu:24-25 */
    int idx = -1;
    for (int t = 0; t < THREADS; ++t) {
        float tb = -1e30f;
        int ti = -1;
        for (int i = t; i < n; i += THREADS) {                             /* sampling.cu:28-34 */
            const float v = orc_bf16_to_f32(x[i]);
            if (v > tb) { tb = v; ti = i; }
        }
        if (ORC_MUTANT == 13 ? tb >= best && ti >= 0 : tb > best) { best = tb; idx = ti; }
    }
    return idx;
}


/* ------------------------------------------------------------------ */
/* Top-k / top-p sampling (src/kernels/sampling_optimized.cu)          */
/* ------------------------------------------------------------------ */

/* One (key, value) pair of the reference's KeyValuePair (sampling_optimized.cu:6-9). */
typedef struct { int key; float value; } orc_kv;

/* warpReduceMax over the 32 lanes of v (sampling_optimized.cu:15-25): for
 * offsets 16, 8, 4, 2, 1 lane l takes lane l + offset's pair when that value
 * is strictly larger; __shfl_down_sync hands a lane past 31 its own value, so
 * those lanes keep theirs.  Lanes are updated from the values before the
 * step, as the shuffle reads them.  Returns lane 0's pair. */
static orc_kv orc_warp_reduce_max(orc_kv* v) {
    for (int off = 16; off > 0; off /= 2) {
        orc_kv nv[32];
        for (int l = 0; l < 32; ++l) {
            const orc_kv o = l + off < 32 ? v[l + off] : v[l];
            nv[l] = v[l];
            if (ORC_MUTANT == 14 ? o.value >= v[l].value : o.value > v[l].value) nv[l] = o;
        }
        memcpy(v, nv, sizeof(nv));
    }
    return v[0];
}

void orc_topk_filter(const uint16_t* logits, int vocab, int k_per_block, int32_t* keys,
                     float* vals) {
    enum { NT = 256, NWARP = NT / 32 };                       /* block 256 (kernels.rs:371-375) */
    for (int p = 0; p < 32; ++p) {                            /* filter_grid = 32 (kernels.rs:367) */
        const int start = (int)((long long)p * vocab / 32);   /* sampling_optimized.cu:37-43 */
        const int end = (int)((long long)(p + 1) * vocab / 32);
        const int n = end - start;
        if (n <= 0) continue;                                 /* :45-46 (slots left untouched) */
        float* s = (float*)malloc(sizeof(float) * (size_t)n);
        for (int i = 0; i < n; ++i) s[i] = orc_bf16_to_f32(logits[start + i]);   /* :51-57 */
        for (int k = 0; k < k_per_block; ++k) {               /* :65 */
            orc_kv warp_max[NWARP];
            for (int w = 0; w < NWARP; ++w) {
                orc_kv lane[32];
                for (int l = 0; l < 32; ++l) {                /* :66-76: strided scan, strict > */
                    const int t = w * 32 + l;
                    orc_kv m = {-1, -1e30f};
                    for (int i = t; i < n; i += NT)
                        if (s[i] > m.value) { m.value = s[i]; m.key = i; }
                    lane[l] = m;
                }
                warp_max[w] = orc_warp_reduce_max(lane);      /* :78-83 */
            }
            orc_kv lane[32];                                  /* :85-92: warp 0 over the warps */
            for (int l = 0; l < 32; ++l) {
                lane[l].key = -1;
                lane[l].value = -1e30f;
                if (l < NWARP) lane[l] = warp_max[l];
            }
            const orc_kv bm = orc_warp_reduce_max(lane);
            keys[p * k_per_block + k] = start + bm.key;       /* :102-106 */
            vals[p * k_per_block + k] = bm.value;
            if (bm.key >= 0 && bm.key < n) s[bm.key] = -1e30f; /* :107-108 */
        }
        free(s);
    }
}

void orc_bitonic_desc(int32_t* keys, float* vals, int n) {
    /* the compare-exchange network of sampling_optimized.cu:130-152, one
     * stage at a time (the pairs of a stage are disjoint) */
    for (int k = 2; k <= n; k <<= 1)
        for (int j = k >> 1; j > 0; j >>= 1)
            for (int t = 0; t < n; ++t) {
                const int x = t ^ j;
                if (x <= t) continue;
                const int down = ORC_MUTANT == 15 ? (t & k) != 0 : (t & k) == 0;
                const int swap = down ? vals[t] < vals[x] : vals[t] > vals[x];
                if (swap) {
                    const int32_t tk = keys[t]; keys[t] = keys[x]; keys[x] = tk;
                    const float tv = vals[t]; vals[t] = vals[x]; vals[x] = tv;
                }
            }
}

int orc_top_p_pick(const float* vals, int n, float top_p, float rand_val, float* prob,
                   float* cdf) {
    /* sampling_optimized.cu:154-187 on the sorted candidates.  The sum and the
     * inclusive scan run in index order here (CUB's BlockReduce/BlockScan
     * order is not in the reference's sources). */
    const float max_val = vals[0];                            /* :154 */
    float total = 0.0f;
    for (int i = 0; i < n; ++i) {
        prob[i] = expf(vals[i] - max_val);                    /* :155 */
        total += prob[i];                                     /* :157-163 */
    }
    float run = 0.0f;
    for (int i = 0; i < n; ++i) {
        prob[i] = prob[i] / total;                            /* :165 */
        run += prob[i];                                       /* :166-169 */
        cdf[i] = run;
    }
    /* :171-180: the thread whose interval holds top_p sets the cutoff (the
     * first such thread here: the reference lets equal-time writers race) */
    float cutoff = 1.0f;
    for (int i = 0; i < n; ++i) {
        const float prev = cdf[i] - prob[i];                  /* :176 */
        if (ORC_MUTANT == 16 ? (prev < top_p && cdf[i] > top_p) : (prev < top_p && cdf[i] >= top_p)) {
            cutoff = cdf[i];
            break;
        }
    }
    const float target = rand_val * cutoff;                   /* :182 */
    for (int i = 0; i < n; ++i) {                             /* :183-187 */
        const float prev = cdf[i] - prob[i];
        if (cdf[i] >= target && prev < target) return i;
    }
    return -1;                                                /* no winner: output not written */
}
