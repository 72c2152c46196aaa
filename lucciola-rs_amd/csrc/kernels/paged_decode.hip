// Split-K paged decode attention for gfx950 (HBM-bound; no MFMA), one launch.
//
// Semantics: for sequence b and q-head qh, attend with q[b][qh] to positions
// 0..positions[b] of the paged cache through table row b, scale sm_scale,
// softmax, weighted sum of V, round to storage -- the single-query attention
// of the reference's flash_decoding_impl (src/kernels/attention.cu:4-176)
// applied to every sequence of a batch.  The reference merges 32 interleaved
// partitions with a log-sum-exp merge (attention.cu:122-175); this kernel
// partitions each context into contiguous splits and merges them with the
// same rule.
//
// With APPEND the same launch first does the engine's per-token prologue
// (src/models.rs:505-534): q and k of the new token get bias + RoPE
// (src/kernels/rope.cu), the roped k and v + v_bias go to the cache slot at
// positions[b] (src/kernels/kv_cache.cu), and the roped q/k are written back
// in place.  Attention uses the new token's K/V from LDS, so no ordering
// against the cache write is needed.
//
// Work decomposition:
//   workgroup = (split, kv head h, sequence b), 4 waves.  The G = Hq/Hkv
//   q-heads of kv head h are processed together, so each KV page is read from
//   HBM once per kv head (GQA grouping).  A wave walks 64-token tiles (32 for
//   head_dim 128) of its split:
//     1. 16-byte loads; each load instruction of the wave covers 1 KB of one
//        page (pages are contiguous [16][D] slabs).  The first tile's loads
//        are issued before any other setup.
//     2. K is staged through LDS and read back one token per lane; scores for
//        all G heads use v_dot2_f32_{f16,bf16} with q broadcast from LDS.
//     3. Online softmax in the exp2 domain: wave max by DPP row reductions +
//        readlane, per-lane partial sums of p.
//     4. V stays in registers in its load layout (lane = token group x 8
//        dims); p is broadcast through LDS; f32 FMA accumulation.
//   The waves' partials are merged through LDS into one (m, l, o[D]) per
//   q-head.  With one split the workgroup writes the output; otherwise it
//   writes its partial to the workspace and takes a ticket, and the last
//   workgroup of (b, h) merges all splits, writes the output and resets the
//   ticket counter to zero for the next launch.
#include "decode_args.h"
#include "luc_common.h"

namespace luc {

using DecodeArgs = ::luc_decode_args;

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

template <int DT>
__device__ inline void rot_pair(const uint16_t* x, const uint16_t* bias, int i1, int i2, float c,
                                float s, uint16_t& o1, uint16_t& o2) {
#pragma clang fp contract(off)
  const float v1 = St<DT>::load(x[i1]) + (bias ? St<DT>::load(bias[i1]) : 0.0f);
  const float v2 = St<DT>::load(x[i2]) + (bias ? St<DT>::load(bias[i2]) : 0.0f);
  const float a = v1 * c, bb = v2 * s, e = v1 * s, f = v2 * c;
  o1 = St<DT>::store(a - bb);
  o2 = St<DT>::store(e + f);
}

template <int DT, int D, int G, bool APPEND>
__device__ void decode_impl(const DecodeArgs& A) {
  using S = DecodeShape<D>;
  constexpr int NT = S::NW * 64;
  constexpr int MERGE = S::NW * S::GROUPS * G * D * 4;
  constexpr int BIG = (S::NW * S::STAGE > MERGE) ? S::NW * S::STAGE : MERGE;
  __shared__ __attribute__((aligned(16))) char smem[BIG];
  __shared__ __attribute__((aligned(16))) uint16_t s_q[G * D];
  __shared__ __attribute__((aligned(16))) uint16_t s_knew[D];
  __shared__ __attribute__((aligned(16))) uint16_t s_vnew[D];
  __shared__ float s_m[S::NW][8];
  __shared__ float s_l[S::NW][8];
  __shared__ int s_ticket;

  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const int split = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int hq = A.hkv * G;
  const int pos = A.positions[b];
  const int ctx = pos + 1;
  uint16_t* out_row = A.out + (int64_t)b * A.out_stride + (int64_t)h * G * D;
  if (ctx <= 0 || ctx > A.max_ctx) {
    // empty context (0/0 in the reference) or beyond the host bound: NaN
    if (split == 0)
      for (int i = threadIdx.x; i < G * D; i += NT) out_row[i] = St<DT>::store(__builtin_nanf(""));
    return;
  }
  const int s_begin = split * A.split_tokens;
  if (s_begin >= ctx) return;  // uniform over the workgroup
  const int s_end = min(ctx, s_begin + A.split_tokens);
  const int nsplit = (ctx + A.split_tokens - 1) / A.split_tokens;
  const int* table = A.tables + (int64_t)b * A.table_stride;
  const int64_t page_stride = (int64_t)A.num_layers * A.hkv * kPage * D;
  const int64_t head_off = ((int64_t)A.layer * A.hkv + h) * kPage * D;
  const bool owns_pos = APPEND && pos >= s_begin && pos < s_end;

  const int tq = lane % S::TILE;          // QK: token of this lane
  const int qhalf = lane / S::TILE;       // QK: which 64 dims (head_dim 128)
  const int pv_tok = lane / S::CH;        // load layout: token within a load group
  const int pv_chunk = lane % S::CH;      // load layout: 16-byte chunk of the row

  uint4 kr[S::LOADS], vr[S::LOADS];
  auto load_tile = [&](int t0) {
#pragma unroll
    for (int r = 0; r < S::LOADS; ++r) {
      const int page_tok = t0 + (r / S::LPP) * kPage;
      if (page_tok < s_end) {
        const int64_t phys = table[page_tok / kPage];
        const int64_t off = phys * page_stride + head_off + (int64_t)((r % S::LPP) * 64 + lane) * 8;
        kr[r] = *(const uint4*)(A.k_pool + off);
        vr[r] = *(const uint4*)(A.v_pool + off);
      } else {
        kr[r] = make_uint4(0, 0, 0, 0);
        vr[r] = make_uint4(0, 0, 0, 0);
      }
    }
  };

  // ---- 1. the first tile's loads go out before anything else ----
  const int t_first = s_begin + w * S::TILE;
  if (t_first < s_end) load_tile(t_first);

  // ---- 2. q for the G heads (roped with APPEND) and the new token's k, v ----
  const uint16_t* qrow = A.q + (int64_t)b * A.q_stride + (int64_t)h * G * D;
  if constexpr (APPEND) {
    constexpr int HALF = D / 2;
    const float* crow = A.cos_t + (int64_t)pos * HALF;
    const float* srow = A.sin_t + (int64_t)pos * HALF;
    const uint16_t* qb = A.q_bias ? A.q_bias + (int64_t)h * G * D : nullptr;
    const uint16_t* krow = A.k_new + (int64_t)b * A.q_stride + (int64_t)h * D;
    const uint16_t* kb = A.k_bias ? A.k_bias + (int64_t)h * D : nullptr;
    for (int idx = threadIdx.x; idx < (G + 1) * HALF; idx += NT) {
      const int g = idx / HALF, i = idx % HALF;
      uint16_t o1, o2;
      if (g < G) {
        rot_pair<DT>(qrow, qb, g * D + i, g * D + i + HALF, crow[i], srow[i], o1, o2);
        s_q[g * D + i] = o1;
        s_q[g * D + i + HALF] = o2;
      } else {
        rot_pair<DT>(krow, kb, i, i + HALF, crow[i], srow[i], o1, o2);
        s_knew[i] = o1;
        s_knew[i + HALF] = o2;
      }
    }
    if (threadIdx.x < D) {
      const int64_t vi = (int64_t)b * A.q_stride + (int64_t)h * D + threadIdx.x;
      const float vb = A.v_bias ? St<DT>::load(A.v_bias[(int64_t)h * D + threadIdx.x]) : 0.0f;
      s_vnew[threadIdx.x] = St<DT>::store(St<DT>::load(A.v_new[vi]) + vb);
    }
  } else {
    const uint32_t* src = (const uint32_t*)qrow;
    for (int i = threadIdx.x; i < G * D / 2; i += NT) ((uint32_t*)s_q)[i] = src[i];
  }
  __syncthreads();
  if (owns_pos && threadIdx.x < D) {  // the cache write of the new token
    const int64_t slot = (int64_t)table[pos / kPage] * page_stride + head_off +
                         (int64_t)(pos % kPage) * D + threadIdx.x;
    A.k_pool[slot] = s_knew[threadIdx.x];
    A.v_pool[slot] = s_vnew[threadIdx.x];
  }

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

  for (int t0 = t_first; t0 < s_end; t0 += S::NW * S::TILE) {
    if (t0 != t_first) load_tile(t0);
    const bool sub = owns_pos && pos >= t0 && pos < t0 + S::TILE;  // tile holds the new token
#pragma unroll
    for (int r = 0; r < S::LOADS; ++r) {
      const int tok = r * S::GROUPS + pv_tok;
      uint4 kv = kr[r];
      if (sub && t0 + tok == pos) {
        kv = *(const uint4*)(s_knew + pv_chunk * 8);
        vr[r] = *(const uint4*)(s_vnew + pv_chunk * 8);
      }
      *(uint4*)(s_k + tok * S::KROW + pv_chunk * 16) = kv;
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
      const float s = valid ? acc[g] * A.qk_scale_log2 : -INFINITY;
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

  // workspace slots of (b, q-head h*G + g, split)
  const int64_t ws_base = ((int64_t)b * hq + (int64_t)h * G) * A.max_splits;
  for (int idx = threadIdx.x; idx < G * D; idx += NT) {
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
    if (nsplit == 1) {
      out_row[idx] = St<DT>::store(acc / L);
    } else {
      const int64_t ws = ws_base + (int64_t)g * A.max_splits + split;
      A.ws_o[ws * D + d] = acc;
      if (d == 0) {
        A.ws_ml[ws * 2] = M;
        A.ws_ml[ws * 2 + 1] = L;
      }
    }
  }

  bool last = nsplit == 1;
  if (nsplit > 1) {
    // publish the partial; the last workgroup of (b, h) merges all splits
    __syncthreads();
    if (threadIdx.x == 0)
      s_ticket = __hip_atomic_fetch_add(A.counters + (int64_t)b * A.hkv + h, 1, __ATOMIC_ACQ_REL,
                                        __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    last = s_ticket == nsplit - 1;
    if (!last) return;
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    for (int idx = threadIdx.x; idx < G * D; idx += NT) {
      const int g = idx / D, d = idx % D;
      const int64_t base = ws_base + (int64_t)g * A.max_splits;
      float M = -INFINITY;
      for (int s = 0; s < nsplit; ++s) M = fmaxf(M, A.ws_ml[(base + s) * 2]);
      float L = 0.0f, acc = 0.0f;
      for (int s = 0; s < nsplit; ++s) {
        const float sc = __builtin_amdgcn_exp2f(A.ws_ml[(base + s) * 2] - M);
        L = fmaf(sc, A.ws_ml[(base + s) * 2 + 1], L);
        acc = fmaf(sc, A.ws_o[(base + s) * D + d], acc);
      }
      out_row[idx] = St<DT>::store(acc / L);
    }
    if (threadIdx.x == 0) A.counters[(int64_t)b * A.hkv + h] = 0;  // ready for the next launch
  }
  if constexpr (APPEND) {
    // every split of (b, h) has read q and k by now: write the roped values back
    if (last) {
      uint16_t* qdst = A.q + (int64_t)b * A.q_stride + (int64_t)h * G * D;
      for (int i = threadIdx.x; i < G * D; i += NT) qdst[i] = s_q[i];
      if (threadIdx.x < D)
        A.k_new[(int64_t)b * A.q_stride + (int64_t)h * D + threadIdx.x] = s_knew[threadIdx.x];
    }
  }
}

}  // namespace luc

#define LUC_DECODE(DTN, DT, D, G)                                                                  \
  extern "C" __global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void     \
      luc_decode_##DTN##_d##D##_g##G(luc::DecodeArgs a) {                                          \
    luc::decode_impl<DT, D, G, false>(a);                                                          \
  }                                                                                                \
  extern "C" __global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void     \
      luc_decode_step_##DTN##_d##D##_g##G(luc::DecodeArgs a) {                                     \
    luc::decode_impl<DT, D, G, true>(a);                                                           \
  }

#define LUC_DECODE_GROUPS(DTN, DT, D)                                                              \
  LUC_DECODE(DTN, DT, D, 1)                                                                        \
  LUC_DECODE(DTN, DT, D, 2)                                                                        \
  LUC_DECODE(DTN, DT, D, 3)                                                                        \
  LUC_DECODE(DTN, DT, D, 4)                                                                        \
  LUC_DECODE(DTN, DT, D, 5)                                                                        \
  LUC_DECODE(DTN, DT, D, 6)                                                                        \
  LUC_DECODE(DTN, DT, D, 7)                                                                        \
  LUC_DECODE(DTN, DT, D, 8)

LUC_DECODE_GROUPS(bf16, luc::kBF16, 64)
LUC_DECODE_GROUPS(bf16, luc::kBF16, 128)
LUC_DECODE_GROUPS(f16, luc::kF16, 64)
LUC_DECODE_GROUPS(f16, luc::kF16, 128)
