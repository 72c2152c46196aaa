// Split-K paged decode attention for gfx950 (HBM-bound; no MFMA).
//
// Semantics: for sequence b and q-head qh, attend with q[b][qh] to positions
// 0..positions[b] of the paged cache through table row b, scale sm_scale,
// softmax, weighted sum of V, round to storage.  This is the single-query
// attention of the reference's flash_decoding_impl
// (src/kernels/attention.cu:4-176) applied to every sequence of a batch.  The
// reference merges 32 interleaved partitions with a log-sum-exp merge
// (attention.cu:122-175); this kernel partitions into contiguous splits
// instead and merges with the same log-sum-exp rule.
//
// Work decomposition:
//   workgroup  = (split, kv head h, sequence b); 4 waves.
//   The G = Hq/Hkv q-heads of kv head h are processed together, so each KV
//   page is read from HBM once per kv head (GQA grouping).
//   A wave processes 64-token tiles (32 for head_dim 128) of its split:
//     1. 16-byte coalesced loads: every load instruction of the wave covers
//        1 KB of one page (pages are contiguous [16][D] slabs).
//     2. K is staged through LDS and read back one token per lane; scores
//        for all G heads use v_dot2_f32_{f16,bf16} with q broadcast from LDS.
//     3. Online softmax in the exp2 domain: wave-wide max by DPP row
//        reductions + readlane, per-lane partial sums of p.
//     4. V stays in registers in its load layout (lane = token group x 8
//        dims); p is broadcast through LDS; f32 FMA accumulation.
//   The 4 waves' partials (and the token groups inside each wave) are merged
//   through LDS into one (m, l, o[D]) per q-head; with one split the kernel
//   writes the final output, otherwise the partial goes to the workspace and
//   luc_decode_combine_* merges the splits.
#include "luc_common.h"

namespace luc {

template <int D>
struct DecodeShape {
  static constexpr int NW = 4;                       // waves per workgroup
  static constexpr int CH = D / 8;                   // 16-byte chunks per token row
  static constexpr int TILE = (D == 64) ? 64 : 32;   // tokens per wave tile
  static constexpr int LOADS = TILE * CH / 64;       // 16-byte loads per lane per tile
  static constexpr int QKL = 64 / TILE;              // lanes per token for QK
  static constexpr int GROUPS = 64 / CH;             // tokens per load instruction
  static constexpr int KROW = D * 2 + 16;            // padded LDS row (bytes)
  static constexpr int LPP = kPage * CH / 64;        // load instructions per page
  static constexpr int STAGE = TILE * KROW + TILE * 32;  // per-wave LDS: K tile + p tile
};

template <int DT, int D, int G>
__device__ void decode_impl(const uint16_t* __restrict__ q, int64_t q_stride,
                            const uint16_t* __restrict__ k_pool,
                            const uint16_t* __restrict__ v_pool, const int* __restrict__ tables,
                            int table_stride, const int* __restrict__ positions, int layer,
                            int num_layers, int hkv, float qk_scale_log2, int max_ctx,
                            int split_tokens, int max_splits, float* __restrict__ ws_ml,
                            float* __restrict__ ws_o, uint16_t* __restrict__ out,
                            int64_t out_stride) {
  using S = DecodeShape<D>;
  constexpr int MERGE = S::NW * S::GROUPS * G * D * 4;
  constexpr int BIG = (S::NW * S::STAGE > MERGE) ? S::NW * S::STAGE : MERGE;
  __shared__ __attribute__((aligned(16))) char smem[BIG];
  __shared__ __attribute__((aligned(16))) uint16_t s_q[G * D];
  __shared__ float s_m[S::NW][8];
  __shared__ float s_l[S::NW][8];

  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const int split = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int ctx = positions[b] + 1;
  const int s_begin = split * split_tokens;
  // Nothing to do past the context; a context beyond the host bound max_ctx
  // (which the table row is sized for) is left to the combine, which flags it.
  if (s_begin >= ctx || ctx > max_ctx) return;  // uniform over the workgroup
  const int s_end = min(ctx, s_begin + split_tokens);
  const int nsplit = (ctx + split_tokens - 1) / split_tokens;
  const int* table = tables + (int64_t)b * table_stride;
  const int64_t page_stride = (int64_t)num_layers * hkv * kPage * D;
  const int64_t head_off = ((int64_t)layer * hkv + h) * kPage * D;

  {  // q rows of the G heads of this kv head -> LDS
    const uint32_t* src = (const uint32_t*)(q + (int64_t)b * q_stride + (int64_t)h * G * D);
    for (int i = threadIdx.x; i < G * D / 2; i += S::NW * 64) ((uint32_t*)s_q)[i] = src[i];
  }
  __syncthreads();

  char* s_k = smem + w * S::STAGE;
  float* s_p = (float*)(s_k + S::TILE * S::KROW);

  float m_run[G], l_lane[G], o[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m_run[g] = -INFINITY;
    l_lane[g] = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[g][e] = 0.0f;
  }

  const int tq = lane % S::TILE;          // QK: token of this lane
  const int qhalf = lane / S::TILE;       // QK: which 64 dims (head_dim 128)
  const int pv_tok = lane / S::CH;        // load layout: token within a load group
  const int pv_chunk = lane % S::CH;      // load layout: 16-byte chunk of the row

  for (int t0 = s_begin + w * S::TILE; t0 < s_end; t0 += S::NW * S::TILE) {
    uint4 kr[S::LOADS], vr[S::LOADS];
#pragma unroll
    for (int r = 0; r < S::LOADS; ++r) {
      const int page_tok = t0 + (r / S::LPP) * kPage;
      if (page_tok < s_end) {
        const int64_t phys = table[page_tok / kPage];
        const int64_t off = phys * page_stride + head_off + (int64_t)((r % S::LPP) * 64 + lane) * 8;
        kr[r] = *(const uint4*)(k_pool + off);
        vr[r] = *(const uint4*)(v_pool + off);
      } else {
        kr[r] = make_uint4(0, 0, 0, 0);
        vr[r] = make_uint4(0, 0, 0, 0);
      }
    }
#pragma unroll
    for (int r = 0; r < S::LOADS; ++r) {
      const int tok = r * S::GROUPS + pv_tok;
      *(uint4*)(s_k + tok * S::KROW + pv_chunk * 16) = kr[r];
      // tokens past the split: V must contribute exactly zero (p is 0 there,
      // and 0 * stale data must not produce NaN)
      if (t0 + tok >= s_end) vr[r] = make_uint4(0, 0, 0, 0);
    }
    wave_lds_sync();

    // ---- scores: lane = token (x2 lanes per token for head_dim 128) ----
    float acc[G];
#pragma unroll
    for (int g = 0; g < G; ++g) acc[g] = 0.0f;
    const char* krow = s_k + tq * S::KROW + qhalf * 128;
    // q is re-read from LDS every tile: an opaque zero offset keeps the
    // compiler from hoisting G*64 loop-invariant values into registers.
    int qz;
    asm volatile("s_mov_b32 %0, 0" : "=s"(qz));
    const uint16_t* qb = s_q + qhalf * 64 + qz;
    // Partially unrolled: fully unrolled, the scheduler hoists all 8*(G+1)
    // LDS reads ahead of the dot products and runs out of registers.
#pragma unroll 2
    for (int c = 0; c < 8; ++c) {
      const uint4 kc = *(const uint4*)(krow + c * 16);
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const uint4 qc = *(const uint4*)(qb + g * D + c * 8);
        float a = acc[g];
        a = St<DT>::dot2(qc.x, kc.x, a);
        a = St<DT>::dot2(qc.y, kc.y, a);
        a = St<DT>::dot2(qc.z, kc.z, a);
        a = St<DT>::dot2(qc.w, kc.w, a);
        acc[g] = a;
      }
    }
    if constexpr (S::QKL == 2) {
#pragma unroll
      for (int g = 0; g < G; ++g) acc[g] += __shfl_xor(acc[g], 32);
    }
    const bool valid = (t0 + tq) < s_end;
    float p[8];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float s = valid ? acc[g] * qk_scale_log2 : -INFINITY;
      const float mn = fmaxf(m_run[g], wave_max(s));
      const float alpha = __builtin_amdgcn_exp2f(m_run[g] - mn);
      p[g] = __builtin_amdgcn_exp2f(s - mn);
      l_lane[g] = l_lane[g] * alpha + (qhalf == 0 ? p[g] : 0.0f);
      m_run[g] = mn;
#pragma unroll
      for (int e = 0; e < 8; ++e) o[g][e] *= alpha;
    }
#pragma unroll
    for (int g = G; g < 8; ++g) p[g] = 0.0f;
    if (qhalf == 0) {
      *(float4*)(s_p + tq * 8) = make_float4(p[0], p[1], p[2], p[3]);
      *(float4*)(s_p + tq * 8 + 4) = make_float4(p[4], p[5], p[6], p[7]);
    }
    wave_lds_sync();

    // ---- o += p * V, V in load layout ----
#pragma unroll
    for (int r = 0; r < S::LOADS; ++r) {
      const int tok = r * S::GROUPS + pv_tok;
      const float4 pa = *(const float4*)(s_p + tok * 8);
      const float4 pb = *(const float4*)(s_p + tok * 8 + 4);
      const float pv[8] = {pa.x, pa.y, pa.z, pa.w, pb.x, pb.y, pb.z, pb.w};
      const uint32_t vw[4] = {vr[r].x, vr[r].y, vr[r].z, vr[r].w};
      float vv[8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        vv[2 * e] = St<DT>::lo(vw[e]);
        vv[2 * e + 1] = St<DT>::hi(vw[e]);
      }
#pragma unroll
      for (int g = 0; g < G; ++g)
#pragma unroll
        for (int e = 0; e < 8; ++e) o[g][e] = fmaf(pv[g], vv[e], o[g][e]);
    }
    wave_lds_sync();
  }

#pragma unroll
  for (int g = 0; g < G; ++g) l_lane[g] = wave_sum(l_lane[g]);

  __syncthreads();  // every wave is done with its staging area
  float* s_o = (float*)smem;  // [NW*GROUPS][G][D]
  if (lane == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      s_m[w][g] = m_run[g];
      s_l[w][g] = l_lane[g];
    }
  }
  {
    const int grp = w * S::GROUPS + pv_tok;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float* dst = s_o + ((int64_t)grp * G + g) * D + pv_chunk * 8;
      *(float4*)dst = make_float4(o[g][0], o[g][1], o[g][2], o[g][3]);
      *(float4*)(dst + 4) = make_float4(o[g][4], o[g][5], o[g][6], o[g][7]);
    }
  }
  __syncthreads();

  const int hq = hkv * G;
  for (int idx = threadIdx.x; idx < G * D; idx += S::NW * 64) {
    const int g = idx / D, d = idx % D;
    float M = -INFINITY;
#pragma unroll
    for (int w2 = 0; w2 < S::NW; ++w2) M = fmaxf(M, s_m[w2][g]);
    float L = 0.0f, acc = 0.0f;
#pragma unroll
    for (int w2 = 0; w2 < S::NW; ++w2) {
      const float sc = __builtin_amdgcn_exp2f(s_m[w2][g] - M);  // 0 for waves without tiles
      float part = 0.0f;
#pragma unroll
      for (int gr = 0; gr < S::GROUPS; ++gr) part += s_o[((w2 * S::GROUPS + gr) * G + g) * D + d];
      L = fmaf(sc, s_l[w2][g], L);
      acc = fmaf(sc, part, acc);
    }
    const int qhead = h * G + g;
    if (nsplit == 1) {
      out[(int64_t)b * out_stride + (int64_t)qhead * D + d] = St<DT>::store(acc / L);
    } else {
      const int64_t ws = ((int64_t)b * hq + qhead) * max_splits + split;
      ws_o[ws * D + d] = acc;
      if (d == 0) {
        ws_ml[ws * 2] = M;
        ws_ml[ws * 2 + 1] = L;
      }
    }
  }
}

// Log-sum-exp merge of the split partials of one (sequence, q-head); one
// thread per output dim.  Sequences with a single split were finished by the
// decode kernel.  Empty contexts and contexts beyond max_ctx get NaN (an
// empty softmax is 0/0, as in the reference).
template <int DT, int D>
__device__ void combine_impl(const float* __restrict__ ws_ml, const float* __restrict__ ws_o,
                             const int* __restrict__ positions, int hq, int max_ctx,
                             int split_tokens, int max_splits, uint16_t* __restrict__ out,
                             int64_t out_stride) {
  const int qhead = blockIdx.x, b = blockIdx.y, d = threadIdx.x;
  const int ctx = positions[b] + 1;
  const int nsplit = ctx > 0 ? (ctx + split_tokens - 1) / split_tokens : 0;
  if (nsplit == 1 && ctx <= max_ctx) return;
  uint16_t* dst = out + (int64_t)b * out_stride + (int64_t)qhead * D + d;
  if (nsplit == 0 || ctx > max_ctx) {
    *dst = St<DT>::store(__builtin_nanf(""));
    return;
  }
  const int64_t base = ((int64_t)b * hq + qhead) * max_splits;
  float M = -INFINITY;
  for (int s = 0; s < nsplit; ++s) M = fmaxf(M, ws_ml[(base + s) * 2]);
  float L = 0.0f, acc = 0.0f;
  for (int s = 0; s < nsplit; ++s) {
    const float sc = __builtin_amdgcn_exp2f(ws_ml[(base + s) * 2] - M);
    L = fmaf(sc, ws_ml[(base + s) * 2 + 1], L);
    acc = fmaf(sc, ws_o[(base + s) * D + d], acc);
  }
  *dst = St<DT>::store(acc / L);
}

}  // namespace luc

#define LUC_DECODE(DTN, DT, D, G)                                                                  \
  extern "C" __global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void luc_decode_##DTN##_d##D##_g##G(                \
      const uint16_t* q, int64_t q_stride, const uint16_t* k_pool, const uint16_t* v_pool,         \
      const int* tables, int table_stride, const int* positions, int layer, int num_layers,        \
      int hkv, float qk_scale_log2, int max_ctx, int split_tokens, int max_splits, float* ws_ml,   \
      float* ws_o, uint16_t* out, int64_t out_stride) {                                            \
    luc::decode_impl<DT, D, G>(q, q_stride, k_pool, v_pool, tables, table_stride, positions,       \
                               layer, num_layers, hkv, qk_scale_log2, max_ctx, split_tokens,       \
                               max_splits, ws_ml, ws_o, out, out_stride);                          \
  }

#define LUC_COMBINE(DTN, DT, D)                                                                    \
  extern "C" __global__ __launch_bounds__(128) void luc_decode_combine_##DTN##_d##D(               \
      const float* ws_ml, const float* ws_o, const int* positions, int hq, int max_ctx,            \
      int split_tokens, int max_splits, uint16_t* out, int64_t out_stride) {                       \
    luc::combine_impl<DT, D>(ws_ml, ws_o, positions, hq, max_ctx, split_tokens, max_splits, out,   \
                             out_stride);                                                          \
  }

#define LUC_DECODE_GROUPS(DTN, DT, D)                                                              \
  LUC_DECODE(DTN, DT, D, 1)                                                                        \
  LUC_DECODE(DTN, DT, D, 2)                                                                        \
  LUC_DECODE(DTN, DT, D, 3)                                                                        \
  LUC_DECODE(DTN, DT, D, 4)                                                                        \
  LUC_DECODE(DTN, DT, D, 5)                                                                        \
  LUC_DECODE(DTN, DT, D, 6)                                                                        \
  LUC_DECODE(DTN, DT, D, 7)                                                                        \
  LUC_DECODE(DTN, DT, D, 8)                                                                        \
  LUC_COMBINE(DTN, DT, D)

LUC_DECODE_GROUPS(bf16, luc::kBF16, 64)
LUC_DECODE_GROUPS(bf16, luc::kBF16, 128)
LUC_DECODE_GROUPS(f16, luc::kF16, 64)
LUC_DECODE_GROUPS(f16, luc::kF16, 128)
