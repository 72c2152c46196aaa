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
// One launch per step.  Work decomposition:
//   Workgroup = (split, sequence b, kv head h), split-major, so the splits
//   every sequence has (split 0, 1, ...) are dispatched first and the
//   workgroups of splits past a context exit at once.  A workgroup is 4
//   waves; the G = Hq/Hkv q-heads of kv head h are processed together, so
//   each KV page is read from HBM once per kv head (GQA).
//   Prologue: positions[b], the wave's block-table entries and q are loaded
//   together (one memory round trip before the KV stream).
//   A wave walks 8 KB tiles of K (64 tokens at head_dim 64, 32 at 128):
//     1. K goes straight from HBM into LDS (global_load_lds_dwordx4; one
//        wave-wide load = 1 KB of a page), each token row XOR-swizzled by
//        16-byte chunk so the per-token LDS reads are conflict-free; V goes
//        to registers in the same load layout (lane = token x 16-byte chunk).
//     2. Scores: lane = token (x2 lanes per token at head_dim 128), all G
//        heads with v_dot2_f32_{f16,bf16}, q broadcast from LDS.
//     3. Online softmax in the exp2 domain: wave max by DPP row reductions +
//        readlane; o rescaled only when the running max moves.
//     4. o += p * V with V in its load layout.  fp16: p of tokens t and
//        t + TILE/2 packed as an fp16 pair, V of the same two tokens paired by
//        v_perm, one v_dot2_f32_f16 per (head, dim).  bf16: f32 FMA.
//   The wave's token groups are reduced with permlane swaps (reduce-scatter)
//   and the 4 waves merge through LDS.  A sequence with one split writes its
//   output; otherwise each split writes (m, l, o) to the workspace, and the
//   last split to arrive (an agent-scope arrival counter per (b, h)) merges
//   all splits with the log-sum-exp rule and resets the counter.
#include "decode_args.h"
#include "luc_common.h"

namespace luc {

using DecodeArgs = ::luc_decode_args;
typedef __attribute__((address_space(3))) char lds_char;
typedef __attribute__((address_space(3))) void lds_void;

template <int D>
struct DecodeGeo {
  static constexpr int NW = 4;                 // waves per workgroup
  static constexpr int CH = D / 8;             // 16-byte chunks per token row
  static constexpr int TPL = 64 / CH;          // tokens per wave-wide 16-byte load
  static constexpr int TILE = 512 / CH;        // tokens per wave tile (8 KB of K)
  static constexpr int LOADS = TILE / TPL;     // K (and V) loads per lane per tile
  static constexpr int HALF = TILE / 2;        // PV pairs tokens t and t + HALF
  static constexpr int QKL = 64 / TILE;        // lanes per token for the scores
  static constexpr int LPP = kPage / TPL;      // load instructions per page
  static constexpr int PAGES = TILE / kPage;   // pages per tile
  static constexpr int ROWB = D * 2;           // bytes per token row
  static constexpr int KBYTES = TILE * ROWB;   // LDS bytes of one wave's K tile
  static_assert(LOADS == 8 && TPL * ROWB == 1024, "one wave-wide load is 1 KB");
};

constexpr int kCpolNT = 2;  // non-temporal load: the KV stream is read once per step

#ifndef LUC_SCHED_FENCE
#define LUC_SCHED_FENCE() __builtin_amdgcn_sched_barrier(0)
#endif

// Wait until this wave has no vector memory operation in flight (also covers
// the LDS writes of global_load_lds, which the compiler does not track).
__device__ inline void wait_vmem_all() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
// ... until at most 8 (the V loads of a tile) are still in flight.
__device__ inline void wait_vmcnt_loads() { asm volatile("s_waitcnt vmcnt(8)" ::: "memory"); }

// 16 bytes per lane from global memory straight into LDS at l + 16*lane + rb;
// rb (the instruction offset) also moves the global address.  rb must fold
// to a constant.
__device__ inline void dma16(const char* g, lds_char* l, int rb) {
  switch (rb) {
    case 0: __builtin_amdgcn_global_load_lds(g, (lds_void*)l, 16, 0, kCpolNT); break;
    case 1024: __builtin_amdgcn_global_load_lds(g, (lds_void*)l, 16, 1024, kCpolNT); break;
    case 2048: __builtin_amdgcn_global_load_lds(g, (lds_void*)l, 16, 2048, kCpolNT); break;
    default: __builtin_amdgcn_global_load_lds(g, (lds_void*)l, 16, 3072, kCpolNT); break;
  }
}

// Agent-coherent (sc1) f32 store / load: visible across the XCDs' L2 caches
// without a cache write-back.
__device__ inline void st_agent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline float ld_agent(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ inline uint4 lds_ld16(const char* base, int off) {
  return *(const uint4*)(base + off);
}

// Bias + RoPE of one pair (x1, x2) in f32, each product and the
// difference/sum rounded separately (contraction off), as rope.cu:31-52.
// A zero bias pattern is +0.0, so a missing bias adds exactly nothing.
template <int DT>
__device__ inline void rot_pair(uint16_t x1, uint16_t b1, uint16_t x2, uint16_t b2, float c,
                                float s, uint16_t& o1, uint16_t& o2) {
#pragma clang fp contract(off)
  const float v1 = St<DT>::load(x1) + St<DT>::load(b1);
  const float v2 = St<DT>::load(x2) + St<DT>::load(b2);
  const float a = v1 * c, bb = v2 * s, e = v1 * s, f = v2 * c;
  o1 = St<DT>::store(a - bb);
  o2 = St<DT>::store(e + f);
}

// Value of the lane TILE/2 tokens further on (valid in lanes < TILE/2).
template <int D>
__device__ inline float upper_half_value(float x) {
  const uint32_t u = __float_as_uint(x);
  if constexpr (D == 64) {
    const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    return __uint_as_float(r[1]);
  } else {
    const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    return __uint_as_float(r[1]);
  }
}

__device__ inline uint32_t pack_f16(float lo, float hi) {
  const half2_t v = {(_Float16)lo, (_Float16)hi};
  return __builtin_bit_cast(uint32_t, v);
}

template <int DT, int D, int G, bool APPEND>
__device__ void decode_impl(const DecodeArgs& A) {
  using S = DecodeGeo<D>;
  constexpr int NW = S::NW, NT = NW * 64;
  constexpr bool PV_DOT2 = (DT == kF16);
  constexpr int PWORDS = (PV_DOT2 ? S::HALF : S::TILE) * 8;  // per-wave p exchange, 32-bit words
  constexpr int HD = D / 2;
  __shared__ __attribute__((aligned(16))) char s_k[NW * S::KBYTES];
  __shared__ __attribute__((aligned(16))) uint32_t s_p[NW * PWORDS];
  __shared__ __attribute__((aligned(16))) uint16_t s_q[G * D];
  __shared__ __attribute__((aligned(16))) uint16_t s_knew[D];
  __shared__ __attribute__((aligned(16))) uint16_t s_vnew[D];
  __shared__ float s_m[NW][8], s_l[NW][8], s_L[8];
  __shared__ int s_last;

  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int pairs = A.batch * A.hkv;
  const int split = blockIdx.x / pairs;
  const int bh = blockIdx.x - split * pairs;
  const int b = bh / A.hkv, h = bh - b * A.hkv;
  const int hq = A.hkv * G;
  const int ST = A.split_tokens;
  const int s_begin = split * ST;
  const int64_t page_stride = (int64_t)A.num_layers * A.hkv * kPage * D;
  const int64_t head_off = ((int64_t)A.layer * A.hkv + h) * kPage * D;
  const int* trow = A.tables + (int64_t)b * A.table_stride;
  const int tmax = (int)A.table_stride - 1;
  uint16_t* out_row = A.out + (int64_t)b * A.out_stride + (int64_t)h * G * D;
  const uint16_t* qrow = A.q + (int64_t)b * A.q_stride + (int64_t)h * G * D;

  // ---- prologue: position, this wave's first table entries and q together ----
  const int t_first = s_begin + w * S::TILE;
  int tab = 0;  // lane j < PAGES: physical page j of the wave's current tile
  if (lane < S::PAGES) tab = trow[min(t_first / kPage + lane, tmax)];
  uint32_t qv[(G * D / 2 + NT - 1) / NT];
  if constexpr (!APPEND) {
#pragma unroll
    for (int i = 0; i < (G * D / 2 + NT - 1) / NT; ++i) {
      const int idx = threadIdx.x + i * NT;
      if (idx < G * D / 2) qv[i] = ((const uint32_t*)qrow)[idx];
    }
  }
  const int pos = A.positions[b];
  const int ctx = pos + 1;
  if (ctx < 1 || ctx > A.max_ctx) {
    // empty context (0/0 in the reference) or beyond the host bound: NaN
    if (split == 0)
      for (int i = threadIdx.x; i < G * D; i += NT) out_row[i] = St<DT>::store(__builtin_nanf(""));
    return;
  }
  if (s_begin >= ctx) return;  // split past this context
  const int nsplit = (ctx + ST - 1) / ST;
  const int s_end = min(ctx, s_begin + ST);
  const bool owns = APPEND && pos < s_end;  // the split holding the new token

  // The step variant's prologue operands (q and k of the new token with their
  // biases, the cos/sin row, v + v_bias) are loaded before the KV stream is
  // issued, so using them does not wait for it.
  constexpr int NPAIR = APPEND ? ((G + 1) * HD + NT - 1) / NT : 1;
  uint16_t rx1[NPAIR], rx2[NPAIR], rb1[NPAIR], rb2[NPAIR], rv = 0, rvb = 0;
  float rc[NPAIR], rs[NPAIR];
  if constexpr (APPEND) {
    const float* crow = A.cos_t + (int64_t)pos * HD;
    const float* srow = A.sin_t + (int64_t)pos * HD;
    const uint16_t* krow = A.k_new + (int64_t)b * A.q_stride + (int64_t)h * D;
#pragma unroll
    for (int i = 0; i < NPAIR; ++i) {
      const int idx = min(threadIdx.x + i * NT, (G + 1) * HD - 1);
      const int g = idx / HD, j = idx % HD;
      const uint16_t* x = g < G ? qrow + g * D : krow;
      const uint16_t* bias = g < G ? (A.q_bias ? A.q_bias + ((int64_t)h * G + g) * D : nullptr)
                                   : (A.k_bias ? A.k_bias + (int64_t)h * D : nullptr);
      rx1[i] = x[j];
      rx2[i] = x[j + HD];
      rb1[i] = bias ? bias[j] : 0;
      rb2[i] = bias ? bias[j + HD] : 0;
      rc[i] = crow[j];
      rs[i] = srow[j];
    }
    if (threadIdx.x < D) {
      rv = A.v_new[(int64_t)b * A.q_stride + (int64_t)h * D + threadIdx.x];
      if (A.v_bias) rvb = A.v_bias[(int64_t)h * D + threadIdx.x];
    }
  }

  const int tq = lane % S::TILE;     // scores: token of this lane
  const int qh = lane / S::TILE;     // scores: which 64 dims (head_dim 128)
  const int pv_tok = lane / S::CH;   // load layout: token within a load
  const int pv_ch = lane % S::CH;    // load layout: 16-byte chunk of the row
  const int kbase = w * S::KBYTES;   // this wave's K tile in s_k
  lds_char* const kdma = (lds_char*)s_k + kbase;

  // Per-lane byte offsets inside a (page, layer, kv head) slab.  Load r reads
  // page r / LPP at + (r % LPP) * 1KB; the K slot pv_ch of token tl holds
  // chunk pv_ch ^ (tl & 7), where tl & 7 only depends on the parity of r.
  auto k_lane_off = [&](int parity) -> uint32_t {
    const int sw = (S::TPL == 8) ? pv_tok : ((parity * S::TPL + pv_tok) & 7);
    return (uint32_t)(pv_tok * S::ROWB + ((pv_ch ^ sw) << 4));
  };
  const uint32_t koff0 = k_lane_off(0), koff1 = k_lane_off(1);
  const uint32_t voff = (uint32_t)(pv_tok * S::ROWB + (pv_ch << 4));
  uint4 vr[S::LOADS];
  // All K loads of a tile go out before its V loads, so the scores can start
  // as soon as K has landed (vmcnt <= LOADS) while V is still in flight.  Pages
  // past the split re-read the tile's last valid page (a cache hit), which
  // keeps the number of loads per tile fixed.
  auto issue = [&](int t0) {
    const int jlast = min(S::PAGES - 1, (s_end - 1 - t0) / kPage);
#pragma unroll
    for (int r = 0; r < S::LOADS; ++r) {
      const int64_t phys = __builtin_amdgcn_readlane(tab, min(r / S::LPP, jlast));
      // wave-uniform slab base (scalar registers) + 32-bit lane offsets
      const char* kslab = (const char*)(A.k_pool + phys * page_stride + head_off);
      dma16(kslab + ((r & 1) ? koff1 : koff0), kdma + (r - r % S::LPP) * 1024, (r % S::LPP) * 1024);
    }
#pragma unroll
    for (int r = 0; r < S::LOADS; ++r) {
      const int64_t phys = __builtin_amdgcn_readlane(tab, min(r / S::LPP, jlast));
      const char* vslab = (const char*)(A.v_pool + phys * page_stride + head_off);
      vr[r] = ld_nt16((const uint16_t*)(vslab + voff + (r % S::LPP) * 1024));
    }
  };
  if (t_first < s_end) issue(t_first);

  // ---- q of the G heads (roped in the step variant), new token's k, v ----
  if constexpr (APPEND) {
#pragma unroll
    for (int i = 0; i < NPAIR; ++i) {
      const int idx = threadIdx.x + i * NT;
      if (idx < (G + 1) * HD) {
        const int g = idx / HD, j = idx % HD;
        uint16_t o1, o2;
        rot_pair<DT>(rx1[i], rb1[i], rx2[i], rb2[i], rc[i], rs[i], o1, o2);
        uint16_t* dst = g < G ? s_q + g * D : s_knew;
        dst[j] = o1;
        dst[j + HD] = o2;
      }
    }
    if (threadIdx.x < D) s_vnew[threadIdx.x] = St<DT>::store(St<DT>::load(rv) + St<DT>::load(rvb));
  } else {
#pragma unroll
    for (int i = 0; i < (G * D / 2 + NT - 1) / NT; ++i) {
      const int idx = threadIdx.x + i * NT;
      if (idx < G * D / 2) ((uint32_t*)s_q)[idx] = qv[i];
    }
  }
  __syncthreads();

  float m_run[G], l_lane[G], o[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m_run[g] = -INFINITY;
    l_lane[g] = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[g][e] = 0.0f;
  }
  uint32_t* const pw = s_p + w * PWORDS;

  for (int t0 = t_first; t0 < s_end; t0 += NW * S::TILE) {
    if (t0 != t_first) issue(t0);
    wait_vmcnt_loads();  // K in LDS (V may still be in flight)
    if constexpr (APPEND) {
      if (owns && pos >= t0 && pos < t0 + S::TILE) {  // this tile holds the new token
        const int t = pos - t0;
        if (lane < S::CH) {
          // its K row in LDS, V in registers, and the cache write of both
          *(uint4*)(s_k + kbase + t * S::ROWB + lane * 16) =
              *(const uint4*)(s_knew + ((lane ^ (t & 7)) * 8));
          const int64_t phys = __builtin_amdgcn_readlane(tab, t / kPage);
          const int64_t slot = phys * page_stride + head_off + (int64_t)(t % kPage) * D + lane * 8;
          *(uint4*)(A.k_pool + slot) = *(const uint4*)(s_knew + lane * 8);
          *(uint4*)(A.v_pool + slot) = *(const uint4*)(s_vnew + lane * 8);
        }
#pragma unroll
        for (int r = 0; r < S::LOADS; ++r)
          if (r == t / S::TPL && pv_tok == t % S::TPL) vr[r] = *(const uint4*)(s_vnew + pv_ch * 8);
      }
    }
    {  // the next tile's table entries, while this tile computes
      const int t_next = t0 + NW * S::TILE;
      if (t_next < s_end && lane < S::PAGES) tab = trow[min(t_next / kPage + lane, tmax)];
    }
    wave_lds_sync();

    // ---- scores: lane = token (x2 lanes per token at head_dim 128) ----
    float acc[G];
#pragma unroll
    for (int g = 0; g < G; ++g) acc[g] = 0.0f;
    const int krow = kbase + tq * S::ROWB;
    const int sw = tq & 7;
    // q is re-read from LDS every tile: an opaque zero offset keeps the
    // compiler from hoisting G*D/8 loop-invariant 16-byte values into registers.
    int qz;
    asm volatile("s_mov_b32 %0, 0" : "=s"(qz));
    const uint16_t* qb = s_q + qz + qh * 64;
#pragma unroll 2
    for (int c = 0; c < 8; ++c) {
      const uint4 kc = lds_ld16(s_k, krow + (((qh * 8 + c) ^ sw) << 4));
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
      LUC_SCHED_FENCE();
    }
    if constexpr (S::QKL == 2) {
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const uint32_t u = __float_as_uint(acc[g]);
        const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
        acc[g] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
      }
    }

    // ---- online softmax (exp2 domain) ----
    const bool valid = (t0 + tq) < s_end;
    float p[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float s = valid ? acc[g] * A.qk_scale_log2 : -INFINITY;
      // wave-uniform: kept in a scalar register
      const float mn = __builtin_bit_cast(
          float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, fmaxf(m_run[g], wave_max(s)))));
      p[g] = __builtin_amdgcn_exp2f(s - mn);
      if (mn > m_run[g]) {  // wave-uniform: rescale only when the max moves
        if (m_run[g] > -INFINITY) {  // (nothing accumulated before the first tile)
          const float alpha = __builtin_amdgcn_exp2f(m_run[g] - mn);
          l_lane[g] *= alpha;
#pragma unroll
          for (int e = 0; e < 8; ++e) o[g][e] *= alpha;
        }
        m_run[g] = mn;
      }
      l_lane[g] += qh == 0 ? p[g] : 0.0f;
    }

    // ---- p to the load layout through LDS ----
    if constexpr (PV_DOT2) {
      uint32_t pk[8];
#pragma unroll
      for (int g = 0; g < 8; ++g) pk[g] = g < G ? pack_f16(p[g], upper_half_value<D>(p[g])) : 0u;
      if (lane < S::HALF) {
        *(uint4*)(pw + tq * 8) = make_uint4(pk[0], pk[1], pk[2], pk[3]);
        *(uint4*)(pw + tq * 8 + 4) = make_uint4(pk[4], pk[5], pk[6], pk[7]);
      }
    } else {
      float pf[8];
#pragma unroll
      for (int g = 0; g < 8; ++g) pf[g] = g < G ? p[g] : 0.0f;
      if (qh == 0) {
        *(float4*)(pw + tq * 8) = make_float4(pf[0], pf[1], pf[2], pf[3]);
        *(float4*)(pw + tq * 8 + 4) = make_float4(pf[4], pf[5], pf[6], pf[7]);
      }
    }
    wave_lds_sync();

    // ---- o += p * V, V in its load layout ----
    // tokens past the split: V must contribute exactly zero (p is 0 there,
    // and 0 * stale data must not produce NaN)
    const bool partial = t0 + S::TILE > s_end;
    if constexpr (PV_DOT2) {
#pragma unroll
      for (int r = 0; r < S::LOADS / 2; ++r) {
        const int t = r * S::TPL + pv_tok;  // vr[r]: token t; vr[r + LOADS/2]: t + HALF
        uint4 va = vr[r], vb = vr[r + S::LOADS / 2];
        if (partial) {
          if (t0 + t >= s_end) va = make_uint4(0, 0, 0, 0);
          if (t0 + t + S::HALF >= s_end) vb = make_uint4(0, 0, 0, 0);
        }
        const uint4 p0 = *(const uint4*)(pw + t * 8);
        const uint4 p1 = *(const uint4*)(pw + t * 8 + 4);
        const uint32_t pp[8] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w};
        const uint32_t aw[4] = {va.x, va.y, va.z, va.w};
        const uint32_t bw[4] = {vb.x, vb.y, vb.z, vb.w};
        uint32_t pr[8];  // (v_t[e], v_{t+HALF}[e]) pairs
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          pr[2 * e] = __builtin_amdgcn_perm(bw[e], aw[e], 0x05040100u);
          pr[2 * e + 1] = __builtin_amdgcn_perm(bw[e], aw[e], 0x07060302u);
        }
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
          for (int e = 0; e < 8; ++e) o[g][e] = St<kF16>::dot2(pr[e], pp[g], o[g][e]);
        LUC_SCHED_FENCE();
      }
    } else {
#pragma unroll
      for (int r = 0; r < S::LOADS; ++r) {
        const int t = r * S::TPL + pv_tok;
        uint4 v = vr[r];
        if (partial && t0 + t >= s_end) v = make_uint4(0, 0, 0, 0);
        const float4 pa = *(const float4*)(pw + t * 8);
        const float4 pb = *(const float4*)(pw + t * 8 + 4);
        const float pv[8] = {pa.x, pa.y, pa.z, pa.w, pb.x, pb.y, pb.z, pb.w};
        const uint32_t vw[4] = {v.x, v.y, v.z, v.w};
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
        LUC_SCHED_FENCE();
      }
    }
    wave_lds_sync();
  }

  // ---- reduce the wave's token groups (lanes sharing pv_ch): reduce-scatter ----
  constexpr int NV = 8 * G;
  float u[NV / 2], y[NV / 4];
#pragma unroll
  for (int k = 0; k < NV / 2; ++k) {
    const int k2 = k + NV / 2;
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(o[k / 8][k % 8]),
                                                    __float_as_uint(o[k2 / 8][k2 % 8]), false, false);
    u[k] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
#pragma unroll
  for (int k = 0; k < NV / 4; ++k) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(u[k]),
                                                    __float_as_uint(u[k + NV / 4]), false, false);
    y[k] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
  if constexpr (D == 64) {  // token groups also differ in lane bit 3
#pragma unroll
    for (int k = 0; k < NV / 4; ++k) y[k] += dpp_mov<0x128>(y[k]);  // row_ror:8
  }
  float* red = (float*)(s_k + kbase);  // this wave's [G][D] result (its K tile is done)
  if (D == 128 || (lane & 8) == 0) {
    const int base = ((lane >> 5) & 1) * (NV / 2) + ((lane >> 4) & 1) * (NV / 4);
#pragma unroll
    for (int k = 0; k < NV / 4; ++k) {
      const int kk = base + k;
      red[(kk / 8) * D + pv_ch * 8 + (kk % 8)] = y[k];
    }
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
    for (int w2 = 0; w2 < NW; ++w2) M = fmaxf(M, s_m[w2][g]);
    float L = 0.0f, acc = 0.0f;
#pragma unroll
    for (int w2 = 0; w2 < NW; ++w2) {
      const float sc = __builtin_amdgcn_exp2f(s_m[w2][g] - M);  // 0 for waves without tiles
      L = fmaf(sc, s_l[w2][g], L);
      acc = fmaf(sc, ((const float*)(s_k + w2 * S::KBYTES))[g * D + d], acc);
    }
    if (nsplit == 1) {
      out_row[idx] = St<DT>::store(acc / L);
    } else {
      const int64_t ws = ws_base + (int64_t)g * A.max_splits + split;
      st_agent(A.ws_o + ws * D + d, acc);
      if (d == 0) {
        st_agent(A.ws_ml + ws * 2, M);
        st_agent(A.ws_ml + ws * 2 + 1, L);
      }
    }
  }

  if (nsplit > 1) {
    // ---- arrival: the last split of (b, h) merges them all ----
    // Partials travel through agent-coherent (sc1) stores and loads, so no
    // L2 write-back is needed: every store of this workgroup has completed
    // before its arrival is counted, and the last arrival loads after the
    // count has returned.
    wait_vmem_all();
    __syncthreads();
    if (threadIdx.x == 0)
      s_last = __hip_atomic_fetch_add(A.ws_cnt + bh, 1u, __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_AGENT) == (unsigned)(nsplit - 1);
    __syncthreads();
    if (!s_last) return;
    float* s_wt = (float*)s_k;  // [G][256] split weights
    for (int g = w; g < G; g += NW) {
      const float* ml = A.ws_ml + (ws_base + (int64_t)g * A.max_splits) * 2;
      float mv[4], lv[4];  // splits lane, lane+64, ... (at most 256)
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int s = lane + 64 * k;
        mv[k] = s < nsplit ? ld_agent(ml + s * 2) : -INFINITY;
        lv[k] = s < nsplit ? ld_agent(ml + s * 2 + 1) : 0.0f;
      }
      const float M = wave_max(fmaxf(fmaxf(mv[0], mv[1]), fmaxf(mv[2], mv[3])));
      float L = 0.0f;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int s = lane + 64 * k;
        const float wgt = __builtin_amdgcn_exp2f(mv[k] - M);  // 0 past nsplit
        if (s < nsplit) s_wt[g * 256 + s] = wgt;
        L = fmaf(wgt, lv[k], L);
      }
      L = wave_sum(L);
      if (lane == 0) s_L[g] = L;
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < G * D; idx += NT) {
      const int g = idx / D, d = idx % D;
      const float* op = A.ws_o + (ws_base + (int64_t)g * A.max_splits) * D + d;
      const float* wt = s_wt + g * 256;
      float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
      int s = 0;
      for (; s + 4 <= nsplit; s += 4) {
        a0 = fmaf(wt[s], ld_agent(op + (int64_t)s * D), a0);
        a1 = fmaf(wt[s + 1], ld_agent(op + (int64_t)(s + 1) * D), a1);
        a2 = fmaf(wt[s + 2], ld_agent(op + (int64_t)(s + 2) * D), a2);
        a3 = fmaf(wt[s + 3], ld_agent(op + (int64_t)(s + 3) * D), a3);
      }
      for (; s < nsplit; ++s) a0 = fmaf(wt[s], ld_agent(op + (int64_t)s * D), a0);
      out_row[idx] = St<DT>::store(((a0 + a1) + (a2 + a3)) / s_L[g]);
    }
    if (threadIdx.x == 0)  // ready for the next launch
      __hip_atomic_store(A.ws_cnt + bh, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }

  if constexpr (APPEND) {
    // every split has read q and k: write the roped values back in place
    uint16_t* qw = A.q + (int64_t)b * A.q_stride + (int64_t)h * G * D;
    uint16_t* kw = A.k_new + (int64_t)b * A.q_stride + (int64_t)h * D;
    for (int i = threadIdx.x; i < G * D; i += NT) qw[i] = s_q[i];
    for (int i = threadIdx.x; i < D; i += NT) kw[i] = s_knew[i];
  }
}

}  // namespace luc

// Resident-wave targets (waves per SIMD).  fp16 fits three 4-wave workgroups
// per CU in registers; the bf16 FMA path needs more registers and runs two.
#ifndef LUC_DECODE_OCC_f16
#define LUC_DECODE_OCC_f16 __attribute__((amdgpu_waves_per_eu(3)))
#endif
#ifndef LUC_DECODE_OCC_bf16
#define LUC_DECODE_OCC_bf16 __attribute__((amdgpu_waves_per_eu(2)))
#endif

#define LUC_DECODE(DTN, DT, D, G)                                                                  \
  extern "C" __global__ __launch_bounds__(256) LUC_DECODE_OCC_##DTN void luc_decode_##DTN##_d##D##_g##G( \
      luc::DecodeArgs a) {                                                                         \
    luc::decode_impl<DT, D, G, false>(a);                                                          \
  }                                                                                                \
  extern "C" __global__ __launch_bounds__(256) LUC_DECODE_OCC_##DTN void                          \
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
