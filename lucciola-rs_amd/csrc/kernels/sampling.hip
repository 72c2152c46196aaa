// Top-k / top-p sampling of one bf16 logits row for gfx950 -- the engine's
// GPU sampler, CudaFunctions::apply_sort_and_sample (src/kernels.rs:346-498)
// over the kernels of src/kernels/sampling_optimized.cu.
//
// Semantics kept from the reference:
//   * Filter (top_k_filter, sampling_optimized.cu:27-112): the row is cut into
//     32 partitions [p*V/32, (p+1)*V/32); each contributes its k/32 largest
//     values, in order, as (index, value) pairs at p*k/32 + r.  Only values
//     above -1e30 count (NaN never); a partition with fewer gives
//     (start - 1, -1e30) for the rest.  Equal values come out in the order the
//     reference's max trees produce: its shfl_down tree keeps the lower slot's
//     pair on ties, so bit 0 of the lane is the most significant tie bit, then
//     bit 1, ...: among equal values the item of the thread (i mod 256) whose
//     bit-reversed warp (3 bits, 8 warps) and then bit-reversed lane (5 bits)
//     are smallest comes first, and within a thread the smallest i.
//   * Sort (sampling_optimized.cu:130-152): the same bitonic compare-exchange
//     network (descending by value, swaps on strict inequality only), so equal
//     values end in the same order.
//   * Sample (:154-187): prob = exp(v - v[0]) / sum; cdf = inclusive sum; the
//     cutoff is the cdf of the candidate whose interval [cdf - prob, cdf]
//     holds top_p (1 when none does); the token is the candidate whose
//     interval holds rand_val * cutoff.  When none does (rand_val = 0, NaN) the
//     output is not written, as in the reference.  Where the reference lets two
//     such candidates race, the first one is taken here.
//
// Design for CDNA4:
//   Filter: one 1024-thread workgroup per partition.  An item's order is one
//   32-bit key: the bf16 value made unsigned-orderable (-0 folded onto +0, as
//   the float compare treats them) in the top 16 bits, the complement of its
//   14-bit tie rank below, and 0 for items that never count -- so "larger key
//   first" is exactly the reference's order and keys of counted items are
//   distinct.  Each lane sorts its NPL keys in registers and each wave takes
//   its two largest (DPP wave maxima; the winning lane shifts its sorted
//   keys).  The (k/32)-th largest of those 32 keys bounds the partition's k/32
//   largest from below; the items at or above it are gathered in LDS and each
//   is ranked by counting the larger ones.  When more than 1024 items pass the
//   bound (the largest values crowded into few waves), each wave takes its
//   k/32 largest in order instead and wave 0 takes the k/32 largest of the 16
//   lists.
//   Sort and sample: one workgroup of max(k, 64) threads, candidate t in lane
//   t.  Bitonic stages whose pairs lie inside a wave run in registers (DPP
//   and lane permutes); the stages across waves exchange through LDS with one
//   barrier each.  Sums and the inclusive scan by DPP within waves and a
//   fixed-order pass over the wave totals.
#include "luc_common.h"

namespace luc {

constexpr int kParts = 32;            // filter partitions (kernels.rs:367)
constexpr int kFilterThreads = 1024;  // one workgroup per partition
constexpr int kFilterWaves = kFilterThreads / 64;
constexpr int kMaxPerPart = 32;       // candidates per partition (top_k <= 1024)

__device__ inline uint32_t bitrev5(uint32_t x) { return __builtin_bitreverse32(x) >> 27; }
__device__ inline uint32_t bitrev3(uint32_t x) { return __builtin_bitreverse32(x) >> 29; }

// Order key of item i (partition-local) with bf16 bits h: 0 when the value is
// not above -1e30 (or NaN); else (orderable value << 16) | (0x3fff - rank),
// rank = bitrev3(warp) << 11 | bitrev5(lane) << 6 | i / 256 with
// warp = (i % 256) / 32, lane = i % 32 (i < 16384).
__device__ inline uint32_t item_key(uint16_t h, int i) {
  const float f = St<kBF16>::load(h);
  if (!(f > -1e30f)) return 0u;
  const uint32_t v = h == 0x8000u ? 0u : (uint32_t)h;  // -0 ties with +0
  const uint32_t ord = (v & 0x8000u) ? (~v & 0xffffu) : (v | 0x8000u);
  const uint32_t t = (uint32_t)i & 255u;
  const uint32_t rank = (bitrev3(t >> 5) << 11) | (bitrev5(t & 31u) << 6) | ((uint32_t)i >> 8);
  return (ord << 16) | (0x3fffu - rank);
}
// Partition-local index of a nonzero key.
__device__ inline int key_index(uint32_t k) {
  const uint32_t rank = 0x3fffu - (k & 0xffffu);
  const uint32_t t = (bitrev3((rank >> 11) & 7u) << 5) | bitrev5((rank >> 6) & 31u);
  return (int)(((rank & 63u) << 8) | t);
}

// bf16 bits of a counted item from its key; a zero key value stands for
// both +0 and -0, so those are read back from the row.
__device__ inline uint16_t item_bits(uint32_t k, const uint16_t* row) {
  const uint32_t ord = k >> 16;
  if (ord == 0x8000u) return row[key_index(k)];
  return (uint16_t)((ord & 0x8000u) ? (ord & 0x7fffu) : (~ord & 0xffffu));
}

// Wave-uniform maximum of an unsigned value over the 64 lanes (the DPP chain
// of wave_max, on integers).
__device__ inline uint32_t wave_max_u32(uint32_t x) {
  uint32_t r;
  asm volatile(LUC_DPP_REDUCE("v_max_u32_dpp") : "=&v"(r) : "v"(x));
  return (uint32_t)__builtin_amdgcn_readlane((int)r, 63);
}

// Sorts N (a power of two) register keys, largest first.
template <int N>
__device__ __attribute__((always_inline)) inline void sort_desc(uint32_t (&k)[N]) {
#pragma unroll
  for (int size = 2; size <= N; size <<= 1)
#pragma unroll
    for (int stride = size / 2; stride > 0; stride >>= 1)
#pragma unroll
      for (int i = 0; i < N; ++i) {
        const int j = i ^ stride;
        if (j > i) {
          const uint32_t a = k[i], b = k[j];
          const bool lo_first = (i & size) == 0;
          k[i] = lo_first ? max(a, b) : min(a, b);
          k[j] = lo_first ? min(a, b) : max(a, b);
        }
      }
}

// The wave's `count` largest keys, largest first, into out[0..count) (lane 0
// writes).  Each lane holds N keys sorted largest first; the lane owning the
// wave maximum drops it by shifting its keys.  Keys of counted items are
// distinct, so exactly one lane owns a nonzero maximum; 0 (nothing left)
// repeats.
template <int N>
__device__ __attribute__((always_inline)) inline void wave_take(uint32_t (&k)[N], int count,
                                                                uint32_t* out, int lane) {
  for (int r = 0; r < count; ++r) {
    const uint32_t m = wave_max_u32(k[0]);
    const bool take = m != 0u && k[0] == m;
#pragma unroll
    for (int j = 0; j + 1 < N; ++j) k[j] = take ? k[j + 1] : k[j];
    k[N - 1] = take ? 0u : k[N - 1];
    if (lane == 0) out[r] = m;
  }
}

// Index of the first lane with pred set (64 when none).
__device__ inline int first_lane(bool pred) {
  const uint64_t b = __builtin_amdgcn_ballot_w64(pred);
  return b ? __builtin_ctzll(b) : 64;
}

// Inclusive integer sum over the lanes of the wave (lane l gets lanes 0..l).
__device__ inline int wave_inclusive_sum_i(int x) {
  x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xF, 0xF, true);  // row_shr:1
  x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xF, 0xF, true);  // row_shr:2
  x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xF, 0xF, true);  // row_shr:4
  x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xF, 0xF, true);  // row_shr:8
  x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xA, 0xF, false);  // row_bcast:15
  x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xC, 0xF, false);  // row_bcast:31
  return x;
}

template <int NPL>
__device__ void topk_filter_impl(const uint16_t* x, int vocab, int kpp, int2* cand) {
  constexpr int kFast = kFilterThreads;  // items the threshold path ranks at most
  __shared__ uint32_t s_list[kFilterWaves][kMaxPerPart];
  __shared__ uint32_t s_win[kMaxPerPart];
  // keys and bf16 bits of the items at or above the threshold; unused keys
  // stay 0, below every counted key, so the ranking reads whole 16-byte rows
  __shared__ __attribute__((aligned(16))) uint32_t s_selk[kFast];
  __shared__ uint16_t s_selb[kFast];
  __shared__ uint32_t s_thr, s_nsel;
  const int p = blockIdx.x;
  const int start = (int)((int64_t)p * vocab / kParts);
  const int n = (int)((int64_t)(p + 1) * vocab / kParts) - start;
  const int t = threadIdx.x, w = t >> 6, lane = t & 63;
  // every load before any use (one memory round trip); indices past the
  // partition re-read its last item and are dropped below
  uint16_t h[NPL];
#pragma unroll
  for (int j = 0; j < NPL; ++j) h[j] = x[start + min(t + kFilterThreads * j, n - 1)];
  uint32_t k[NPL];
#pragma unroll
  for (int j = 0; j < NPL; ++j) {
    const int i = t + kFilterThreads * j;
    k[j] = i < n ? item_key(h[j], i) : 0u;
  }
  sort_desc<NPL>(k);
  uint32_t kk[NPL];  // the sorted keys, kept for the general path
#pragma unroll
  for (int j = 0; j < NPL; ++j) kk[j] = k[j];

  // Threshold: the kpp-th largest of the 16 waves' two largest keys (32
  // distinct items, so at least kpp items lie at or above it and the
  // partition's kpp largest all do).
  wave_take<NPL>(k, 2, s_list[w], lane);
  if (t == 0) s_nsel = 0u;
  s_selk[t] = 0u;
  __syncthreads();
  if (w == 0) {
    const uint32_t y = lane < 2 * kFilterWaves ? s_list[lane >> 1][lane & 1] : 0u;
    int rank = 0;  // keys larger than this lane's (distinct unless 0)
#pragma unroll
    for (int m = 0; m < 2 * kFilterWaves; ++m)
      rank += (uint32_t)__builtin_amdgcn_readlane((int)y, m) > y ? 1 : 0;
    const int at = first_lane(lane < 2 * kFilterWaves && y != 0u && rank == kpp - 1);
    const uint32_t thr = at < 64 ? (uint32_t)__builtin_amdgcn_readlane((int)y, at & 63) : 1u;
    if (lane == 0) s_thr = thr;
  }
  __syncthreads();
  const uint32_t thr = s_thr;
  // gather the items at or above the threshold: a lane's are its first c keys
  int c = 0;
#pragma unroll
  for (int j = 0; j < NPL; ++j) c += kk[j] >= thr ? 1 : 0;
  const int incl = wave_inclusive_sum_i(c);
  uint32_t wbase = 0;
  if (lane == 63) wbase = atomicAdd(&s_nsel, (uint32_t)incl);
  wbase = (uint32_t)__builtin_amdgcn_readlane((int)wbase, 63);
  const uint32_t mine = wbase + (uint32_t)(incl - c);
#pragma unroll
  for (int j = 0; j < NPL; ++j) {
    if (j < c && mine + j < (uint32_t)kFast) {
      s_selk[mine + j] = kk[j];
      s_selb[mine + j] = item_bits(kk[j], x + start);
    }
  }
  __syncthreads();
  const int nsel = (int)s_nsel;
  if (nsel <= kFast) {
    // rank each gathered item among the gathered ones (keys are distinct);
    // the kpp largest land at their rank, missing ones are (start - 1, -1e30)
    if (t < nsel) {
      const uint32_t me = s_selk[t];
      const uint4* rows = (const uint4*)s_selk;
      int rank = 0;
#pragma unroll 4
      for (int m = 0; m < (nsel + 3) >> 2; ++m) {
        const uint4 r = rows[m];
        rank += (r.x > me) + (r.y > me) + (r.z > me) + (r.w > me);
      }
      if (rank < kpp)
        cand[p * kpp + rank] = make_int2(start + key_index(me), __float_as_int(St<kBF16>::load(s_selb[t])));
    }
    if (t >= nsel && t < kpp) cand[p * kpp + t] = make_int2(start - 1, __float_as_int(-1e30f));
    return;
  }
  // General path (many items at or above the threshold): each wave takes its
  // kpp largest in order, then wave 0 the kpp largest of the 16 lists.
#pragma unroll
  for (int j = 0; j < NPL; ++j) k[j] = kk[j];
  wave_take<NPL>(k, kpp, s_list[w], lane);
  __syncthreads();
  if (w != 0) return;
  uint32_t k2[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int e = lane + 64 * j;
    k2[j] = e < kFilterWaves * kpp ? s_list[e / kpp][e % kpp] : 0u;
  }
  sort_desc<8>(k2);
  wave_take<8>(k2, kpp, s_win, lane);
  wave_lds_sync();
  if (lane < kpp) {
    const uint32_t m = s_win[lane];
    int2 cv = make_int2(start - 1, __float_as_int(-1e30f));
    if (m != 0u)  // the value itself (a -0 keeps its sign)
      cv = make_int2(start + key_index(m), __float_as_int(St<kBF16>::load(item_bits(m, x + start))));
    cand[p * kpp + lane] = cv;
  }
}

// Inclusive sum over the lanes of the wave (lane l gets lanes 0..l).
__device__ inline float wave_inclusive_sum(float x) {
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x111, 0xF, 0xF, true));  // row_shr:1
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x112, 0xF, 0xF, true));  // row_shr:2
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x114, 0xF, 0xF, true));  // row_shr:4
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x118, 0xF, 0xF, true));  // row_shr:8
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x142, 0xA, 0xF, false));  // row_bcast:15
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x143, 0xC, 0xF, false));  // row_bcast:31
  return x;
}

// Value of lane (this lane ^ J), J < 64: DPP within a row for J <= 8 (quad
// permutes, or a row shift in the direction of the partner), a lane permute
// through the LDS crossbar for 16 and 32.
template <int J>
__device__ inline int xor_lane(int v, int lane) {
  if constexpr (J == 1) {
    return __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false);  // quad_perm [1,0,3,2]
  } else if constexpr (J == 2) {
    return __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false);  // quad_perm [2,3,0,1]
  } else if constexpr (J == 4 || J == 8) {
    const int up = __builtin_amdgcn_update_dpp(0, v, 0x100 + J, 0xF, 0xF, false);  // row_shl:J
    const int dn = __builtin_amdgcn_update_dpp(0, v, 0x110 + J, 0xF, 0xF, false);  // row_shr:J
    return (lane & J) ? dn : up;
  } else {
    return __shfl_xor(v, J, 64);
  }
}

// One compare-exchange stage of the reference's bitonic network (block k,
// distance j): element t and its partner t ^ j; the block sorts descending
// when (t & k) == 0; the pair swaps only on a strict inequality.  This lane
// holds element t as (key, value bits) and keeps its side of the outcome.
__device__ inline void bitonic_pick(int t, int k, int j, int& key, int& val, int pkey, int pval) {
  const bool lower = (t & j) == 0;
  const float mine = __int_as_float(val), other = __int_as_float(pval);
  const float a = lower ? mine : other, b = lower ? other : mine;  // elements (lo, hi)
  const bool swap = (t & k) == 0 ? a < b : a > b;
  key = swap ? pkey : key;
  val = swap ? pval : val;
}

template <int J>
__device__ __attribute__((always_inline)) inline void stage_in_wave(int t, int k, int lane, int& key,
                                                                    int& val) {
  const int pk = xor_lane<J>(key, lane), pv = xor_lane<J>(val, lane);
  bitonic_pick(t, k, J, key, val, pk, pv);
}

template <int N>
__device__ void top_p_sample_impl(int2* cand, float top_p, float rand_val, uint32_t* out) {
  constexpr int NT = N < 64 ? 64 : N;
  constexpr int NW = NT / 64;
  __shared__ int2 s_x[2][N > 64 ? N : 1];  // cross-wave stages, double-buffered
  __shared__ float s_wsum[NW], s_wtot[NW], s_wcut[NW], s_max;
  __shared__ int s_wcut_at[NW], s_wwin_at[NW];
  const int t = threadIdx.x, w = t >> 6, lane = t & 63;
  const bool act = t < N;
  int key = 0, val = 0;
  if (act) {
    const int2 c = cand[t];
    key = c.x;
    val = c.y;
  }
  // the reference's network (sampling_optimized.cu:130-152), element t in
  // lane t: stages with j < 64 stay inside the wave, the others exchange
  // through LDS with one barrier each
  int buf = 0;
#pragma unroll
  for (int k = 2; k <= N; k <<= 1) {
#pragma unroll
    for (int j = k >> 1; j > 0; j >>= 1) {
      if constexpr (N > 64) {
        if (j >= 64) {
          if (act) s_x[buf][t] = make_int2(key, val);
          __syncthreads();
          const int2 o = act ? s_x[buf][t ^ j] : make_int2(0, 0);
          buf ^= 1;
          bitonic_pick(t, k, j, key, val, o.x, o.y);
          continue;
        }
      }
      switch (j) {
        case 1: stage_in_wave<1>(t, k, lane, key, val); break;
        case 2: stage_in_wave<2>(t, k, lane, key, val); break;
        case 4: stage_in_wave<4>(t, k, lane, key, val); break;
        case 8: stage_in_wave<8>(t, k, lane, key, val); break;
        case 16: stage_in_wave<16>(t, k, lane, key, val); break;
        default: stage_in_wave<32>(t, k, lane, key, val); break;
      }
    }
  }
  if (act) cand[t] = make_int2(key, val);  // the sorted candidates go back to the buffer
  if (t == 0) s_max = __int_as_float(val);
  __syncthreads();
  const float maxv = s_max;
  const float e = act ? expf(__int_as_float(val) - maxv) : 0.0f;
  const float ws = wave_sum(e);
  if (lane == 0) s_wsum[w] = ws;
  __syncthreads();
  float total = 0.0f;
#pragma unroll
  for (int v = 0; v < NW; ++v) total += s_wsum[v];
  const float prob = e / total;
  const float incl = wave_inclusive_sum(prob);
  if (lane == 63) s_wtot[w] = incl;
  __syncthreads();
  float base = 0.0f;
#pragma unroll
  for (int v = 0; v < NW; ++v) base += v < w ? s_wtot[v] : 0.0f;
  const float cdf = base + incl;
  const float prev = cdf - prob;
  // cutoff: the first candidate whose interval holds top_p
  const int fc = first_lane(act && prev < top_p && cdf >= top_p);
  const float cut_w = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(cdf), fc & 63));
  if (lane == 0) {
    s_wcut_at[w] = fc;
    s_wcut[w] = cut_w;
  }
  __syncthreads();
  float cutoff = 1.0f;
#pragma unroll
  for (int v = NW - 1; v >= 0; --v) cutoff = s_wcut_at[v] < 64 ? s_wcut[v] : cutoff;
  const float target = rand_val * cutoff;
  const int fw = first_lane(act && cdf >= target && prev < target);
  if (lane == 0) s_wwin_at[w] = fw;
  __syncthreads();
  int first_w = NW;
#pragma unroll
  for (int v = NW - 1; v >= 0; --v) first_w = s_wwin_at[v] < 64 ? v : first_w;
  if (w == first_w && lane == fw) out[0] = (uint32_t)key;
}

}  // namespace luc

#define LUC_TOPK_FILTER(NPL)                                                                       \
  extern "C" __global__ __launch_bounds__(luc::kFilterThreads) void luc_topk_filter_bf16_n##NPL(    \
      const uint16_t* x, int vocab, int kpp, int2* cand) {                                         \
    luc::topk_filter_impl<NPL>(x, vocab, kpp, cand);                                               \
  }
LUC_TOPK_FILTER(1)
LUC_TOPK_FILTER(2)
LUC_TOPK_FILTER(4)
LUC_TOPK_FILTER(8)
LUC_TOPK_FILTER(16)

#define LUC_TOP_P(N)                                                                               \
  extern "C" __global__ __launch_bounds__(N < 64 ? 64 : N) void luc_top_p_sample_##N(              \
      int2* cand, float top_p, float rand_val, uint32_t* out) {                                    \
    luc::top_p_sample_impl<N>(cand, top_p, rand_val, out);                                         \
  }
LUC_TOP_P(32)
LUC_TOP_P(64)
LUC_TOP_P(128)
LUC_TOP_P(256)
LUC_TOP_P(512)
LUC_TOP_P(1024)
