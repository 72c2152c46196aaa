// Split-K paged decode attention for gfx950 (HBM-bound; no MFMA).
//
// Semantics: for sequence b and q-head qh, attend with q[b][qh] to positions
// 0..positions[b] of the paged cache through table row b, scale sm_scale,
// softmax, weighted sum of V, round to storage -- the single-query attention
// of the reference's flash_decoding_impl (src/kernels/attention.cu:4-176)
// applied to every sequence of a batch.  The reference merges 32 interleaved
// partitions with a log-sum-exp merge (attention.cu:122-175); here each
// context is cut into contiguous splits that are merged with the same rule.
//
// The step variant (APPEND) also does the engine's per-token prologue
// (src/models.rs:505-534) for the new token at positions[b]: bias + RoPE of q
// and k (src/kernels/rope.cu) and the cache write of the roped k and
// v + v_bias (src/kernels/kv_cache.cu).  Attention takes the new token's K/V
// from LDS, so it does not depend on the order of the cache write.
//
// Launches:
//   luc_decode[_step]_*   partials: one (m, l, o[D]) per (sequence, q-head,
//                         split), or the final output when a sequence has a
//                         single split.
//   luc_decode_combine_*  log-sum-exp merge of the splits; the step variant
//                         also writes the roped q and k back in place (after
//                         every split has read them).
//
// Work decomposition (decode kernel):
//   A work item is (sequence b, kv head h, split).  Items are numbered
//   densely from the device-side positions, so no workgroup is launched for
//   splits past a context; the grid is persistent (sized to the resident
//   workgroups) and each workgroup walks items blockIdx.x, +gridDim.x, ...
//   A workgroup is 4 waves; the G = Hq/Hkv q-heads of kv head h are processed
//   together, so each KV page is read from HBM once per kv head (GQA).  A wave
//   walks 64-token tiles (32 for head_dim 128) of the split:
//     1. 16-byte loads; one load instruction of the wave covers 1 KB of a page
//        (pages are contiguous [16][D] slabs).  The first tile's loads are
//        issued before any other per-item setup.
//     2. K goes through LDS and is read back one token per lane; scores for
//        all G heads use v_dot2_f32_{f16,bf16} with q broadcast from LDS.
//     3. Online softmax in the exp2 domain: wave max by DPP row reductions +
//        readlane; per-lane partial sums of p; o is rescaled only when the
//        running max moves.
//     4. V stays in registers in its load layout (lane = token group x 8
//        dims); p is broadcast through LDS; f32 FMA accumulation.
//   Each wave reduces its token groups through LDS, then the 4 waves merge.
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
  static constexpr int HP = (D == 64) ? 4 : 2;       // heads per group-reduction pass
  static constexpr int RES_OFF = GROUPS * HP * D * 4;    // per-wave result after the scratch
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

// Number of splits of a sequence whose current position is pos; 0 when the
// context is empty or beyond max_ctx (such a sequence still gets one item,
// which writes NaN).
__device__ inline int splits_of(int pos, int max_ctx, int split_tokens) {
  const int ctx = pos + 1;
  return (ctx <= 0 || ctx > max_ctx) ? 0 : (ctx + split_tokens - 1) / split_tokens;
}

// Inclusive prefix sum over the 64 lanes of a wave.
__device__ inline int wave_incl_scan(int x, int lane) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(x, o);
    if (lane >= o) x += y;
  }
  return x;
}

struct Item {
  int b, h, split, nsplit;  // nsplit 0: invalid context
};

// Item `it` of the dense numbering: sequences in order, then kv heads, then
// splits.  Every lane returns the same item.  Returns false past the last one.
__device__ inline bool find_item(const DecodeArgs& A, int batch, int it, int lane, Item& out) {
  int base = 0;  // items before this chunk of sequences
  for (int b0 = 0; b0 < batch; b0 += 64) {
    const int b = b0 + lane;
    int n = 0;
    if (b < batch) n = max(1, splits_of(A.positions[b], A.max_ctx, A.split_tokens)) * A.hkv;
    const int incl = wave_incl_scan(n, lane);
    const int total = __shfl(incl, 63);
    if (it < base + total) {
      // the first lane whose inclusive sum exceeds the local index owns it
      const int local = it - base;
      const unsigned long long m = __ballot(incl > local && b < batch);
      const int src = __ffsll((long long)m) - 1;
      const int bb = b0 + src;
      const int excl = __shfl(incl - n, src);
      const int ns = __shfl(n, src) / A.hkv;
      const int r = local - excl;
      out.b = bb;
      out.h = r / ns;
      out.split = r % ns;
      out.nsplit = splits_of(A.positions[bb], A.max_ctx, A.split_tokens);
      return true;
    }
    base += total;
  }
  return false;
}

template <int DT, int D, int G, bool APPEND>
__device__ void decode_impl(const DecodeArgs& A, int batch) {
  using S = DecodeShape<D>;
  constexpr int NT = S::NW * 64;
  __shared__ __attribute__((aligned(16))) char smem[S::NW * S::STAGE];
  __shared__ __attribute__((aligned(16))) uint16_t s_q[G * D];
  __shared__ __attribute__((aligned(16))) uint16_t s_knew[D];
  __shared__ __attribute__((aligned(16))) uint16_t s_vnew[D];
  __shared__ float s_m[S::NW][8];
  __shared__ float s_l[S::NW][8];

  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const int tq = lane % S::TILE;          // QK: token of this lane
  const int qhalf = lane / S::TILE;       // QK: which 64 dims (head_dim 128)
  const int pv_tok = lane / S::CH;        // load layout: token within a load group
  const int pv_chunk = lane % S::CH;      // load layout: 16-byte chunk of the row
  const int hq = A.hkv * G;
  char* stage = smem + w * S::STAGE;
  char* s_k = stage;
  float* s_p = (float*)(stage + S::TILE * S::KROW);
  const int64_t page_stride = (int64_t)A.num_layers * A.hkv * kPage * D;

  for (int it = blockIdx.x;; it += gridDim.x) {
    Item item;
    if (!find_item(A, batch, it, lane, item)) break;  // uniform: every wave finds the same
    const int b = __builtin_amdgcn_readfirstlane(item.b);
    const int h = __builtin_amdgcn_readfirstlane(item.h);
    const int split = __builtin_amdgcn_readfirstlane(item.split);
    const int nsplit = __builtin_amdgcn_readfirstlane(item.nsplit);
    uint16_t* out_row = A.out + (int64_t)b * A.out_stride + (int64_t)h * G * D;
    if (nsplit == 0) {
      // empty context (0/0 in the reference) or beyond the host bound: NaN
      for (int i = threadIdx.x; i < G * D; i += NT) out_row[i] = St<DT>::store(__builtin_nanf(""));
      continue;
    }
    const int pos = A.positions[b];
    const int ctx = pos + 1;
    const int s_begin = split * A.split_tokens;
    const int s_end = min(ctx, s_begin + A.split_tokens);
    const int* table = A.tables + (int64_t)b * A.table_stride;
    const int64_t head_off = ((int64_t)A.layer * A.hkv + h) * kPage * D;
    const bool owns_pos = APPEND && pos >= s_begin && pos < s_end;

    uint4 kr[S::LOADS], vr[S::LOADS];
    auto load_tile = [&](int t0) {
      // The tile's block-table entries with one vector load (lane j: page j);
      // scalar loads of them queue behind the KV stream of other waves.
      int my_phys = 0;
      if (lane < S::TILE / kPage && t0 + lane * kPage < s_end) my_phys = table[t0 / kPage + lane];
#pragma unroll
      for (int r = 0; r < S::LOADS; ++r) {
        const int page_tok = t0 + (r / S::LPP) * kPage;
        if (page_tok < s_end) {
          const int64_t phys = __builtin_amdgcn_readlane(my_phys, r / S::LPP);
          const int64_t off = phys * page_stride + head_off + (int64_t)((r % S::LPP) * 64 + lane) * 8;
          // KV is read once per step: non-temporal, so the stream does not
          // evict the small, reused data (tables, positions, q) from L2
          kr[r] = ld_nt16(A.k_pool + off);
          vr[r] = ld_nt16(A.v_pool + off);
        } else {
          kr[r] = make_uint4(0, 0, 0, 0);
          vr[r] = make_uint4(0, 0, 0, 0);
        }
      }
    };

    // ---- 1. the first tile's loads go out before the rest of the setup ----
    const int t_first = s_begin + w * S::TILE;
    if (t_first < s_end) load_tile(t_first);

    // ---- 2. q of the G heads (roped in the step variant), new token's k, v ----
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
        // wave-uniform: kept in a scalar register
        const float mn = __builtin_bit_cast(
            float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, fmaxf(m_run[g], wave_max(s)))));
        p[g] = __builtin_amdgcn_exp2f(s - mn);
        if (mn != m_run[g]) {  // wave-uniform: rescale only when the max moves
          const float alpha = __builtin_amdgcn_exp2f(m_run[g] - mn);
          l_lane[g] *= alpha;
#pragma unroll
          for (int e = 0; e < 8; ++e) o[g][e] *= alpha;
          m_run[g] = mn;
        }
        l_lane[g] += qhalf == 0 ? p[g] : 0.0f;
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

    // ---- reduce the wave's token groups: result [G][D] f32 at RES_OFF ----
    float* scratch = (float*)stage;           // [GROUPS][HP][D]
    float* res = (float*)(stage + S::RES_OFF);
#pragma unroll
    for (int g0 = 0; g0 < G; g0 += S::HP) {
#pragma unroll
      for (int j = 0; j < S::HP; ++j) {
        if (g0 + j < G) {
          float* dst = scratch + ((int64_t)pv_tok * S::HP + j) * D + pv_chunk * 8;
          *(float4*)dst = make_float4(o[g0 + j][0], o[g0 + j][1], o[g0 + j][2], o[g0 + j][3]);
          *(float4*)(dst + 4) = make_float4(o[g0 + j][4], o[g0 + j][5], o[g0 + j][6], o[g0 + j][7]);
        }
      }
      wave_lds_sync();
      for (int idx = lane; idx < S::HP * D; idx += 64) {
        if (g0 + idx / D < G) {
          float sum = 0.0f;
#pragma unroll
          for (int gr = 0; gr < S::GROUPS; ++gr) sum += scratch[gr * S::HP * D + idx];
          res[g0 * D + idx] = sum;
        }
      }
      wave_lds_sync();
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float l = wave_sum(l_lane[g]);
      if (lane == 0) {
        s_m[w][g] = m_run[g];
        s_l[w][g] = l;
      }
    }
    __syncthreads();

    // ---- merge the waves ----
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
        const float* r2 = (const float*)(smem + w2 * S::STAGE + S::RES_OFF);
        L = fmaf(sc, s_l[w2][g], L);
        acc = fmaf(sc, r2[g * D + d], acc);
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
    __syncthreads();  // LDS is reused by the next item
  }
}

// Split merge for one (sequence, kv head); the step variant also writes the
// roped q (G heads) and k of the new token back into the qkv row.
template <int DT, int D, int G, bool APPEND>
__device__ void combine_impl(const DecodeArgs& A) {
  constexpr int NT = 256;
  constexpr int MAXS = 256;  // splits per sequence (host-enforced)
  __shared__ float s_w[G][MAXS];
  __shared__ float s_L[G];
  const int b = blockIdx.y, h = blockIdx.x;
  const int hq = A.hkv * G;
  const int pos = A.positions[b];
  const int nsplit = splits_of(pos, A.max_ctx, A.split_tokens);
  if constexpr (APPEND) {
    if (nsplit > 0) {
      constexpr int HALF = D / 2;
      const float* crow = A.cos_t + (int64_t)pos * HALF;
      const float* srow = A.sin_t + (int64_t)pos * HALF;
      uint16_t* qrow = A.q + (int64_t)b * A.q_stride + (int64_t)h * G * D;
      uint16_t* krow = A.k_new + (int64_t)b * A.q_stride + (int64_t)h * D;
      const uint16_t* qb = A.q_bias ? A.q_bias + (int64_t)h * G * D : nullptr;
      const uint16_t* kb = A.k_bias ? A.k_bias + (int64_t)h * D : nullptr;
      for (int idx = threadIdx.x; idx < (G + 1) * HALF; idx += NT) {
        const int g = idx / HALF, i = idx % HALF;
        uint16_t o1, o2;
        if (g < G) {
          rot_pair<DT>(qrow, qb, g * D + i, g * D + i + HALF, crow[i], srow[i], o1, o2);
          qrow[g * D + i] = o1;
          qrow[g * D + i + HALF] = o2;
        } else {
          rot_pair<DT>(krow, kb, i, i + HALF, crow[i], srow[i], o1, o2);
          krow[i] = o1;
          krow[i + HALF] = o2;
        }
      }
    }
  }
  if (nsplit <= 1) return;  // finished by the decode kernel
  const int64_t ws_base = ((int64_t)b * hq + (int64_t)h * G) * A.max_splits;
  // per-split weights exp2(m_s - M) and the merged sum per head
  for (int g = threadIdx.x >> 6; g < G; g += NT / 64) {
    const int lane = threadIdx.x & 63;
    const float* ml = A.ws_ml + (ws_base + (int64_t)g * A.max_splits) * 2;
    float M = -INFINITY;
    for (int s = lane; s < nsplit; s += 64) M = fmaxf(M, ml[s * 2]);
    M = wave_max(M);
    float L = 0.0f;
    for (int s = lane; s < nsplit; s += 64) {
      const float wgt = __builtin_amdgcn_exp2f(ml[s * 2] - M);
      s_w[g][s] = wgt;
      L = fmaf(wgt, ml[s * 2 + 1], L);
    }
    L = wave_sum(L);
    if (lane == 0) s_L[g] = L;
  }
  __syncthreads();
  uint16_t* out_row = A.out + (int64_t)b * A.out_stride + (int64_t)h * G * D;
  for (int idx = threadIdx.x; idx < G * D; idx += NT) {
    const int g = idx / D, d = idx % D;
    const float* op = A.ws_o + (ws_base + (int64_t)g * A.max_splits) * D + d;
    float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
    int s = 0;
    for (; s + 4 <= nsplit; s += 4) {
      a0 = fmaf(s_w[g][s], op[(int64_t)s * D], a0);
      a1 = fmaf(s_w[g][s + 1], op[(int64_t)(s + 1) * D], a1);
      a2 = fmaf(s_w[g][s + 2], op[(int64_t)(s + 2) * D], a2);
      a3 = fmaf(s_w[g][s + 3], op[(int64_t)(s + 3) * D], a3);
    }
    for (; s < nsplit; ++s) a0 = fmaf(s_w[g][s], op[(int64_t)s * D], a0);
    out_row[idx] = St<DT>::store(((a0 + a1) + (a2 + a3)) / s_L[g]);
  }
}

}  // namespace luc

// Two resident waves per SIMD (8 per CU, two workgroups): the register budget
// the decode loop is written for.
#ifndef LUC_DECODE_OCC
#define LUC_DECODE_OCC __attribute__((amdgpu_waves_per_eu(2, 2)))
#endif

#define LUC_DECODE(DTN, DT, D, G)                                                                  \
  extern "C" __global__ __launch_bounds__(256) LUC_DECODE_OCC void luc_decode_##DTN##_d##D##_g##G( \
      luc::DecodeArgs a, int batch) {                                                              \
    luc::decode_impl<DT, D, G, false>(a, batch);                                                   \
  }                                                                                                \
  extern "C" __global__ __launch_bounds__(256) LUC_DECODE_OCC void luc_decode_step_##DTN##_d##D##_g##G( \
      luc::DecodeArgs a, int batch) {                                                              \
    luc::decode_impl<DT, D, G, true>(a, batch);                                                    \
  }                                                                                                \
  extern "C" __global__ __launch_bounds__(256) void luc_decode_combine_##DTN##_d##D##_g##G(        \
      luc::DecodeArgs a) {                                                                         \
    luc::combine_impl<DT, D, G, false>(a);                                                         \
  }                                                                                                \
  extern "C" __global__ __launch_bounds__(256) void luc_decode_step_combine_##DTN##_d##D##_g##G(   \
      luc::DecodeArgs a) {                                                                         \
    luc::combine_impl<DT, D, G, true>(a);                                                          \
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
