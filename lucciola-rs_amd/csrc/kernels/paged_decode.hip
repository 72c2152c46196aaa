// Split-K paged decode attention for gfx950.  HBM-bound: the scores, and PV
// in every kernel but the head_dim 128 tile-pair step kernels and group size
// 8 there, run on v_mfma_f32_32x32x16 to take their arithmetic off the VALU
// after each tile lands, not for the flops.
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
// One launch per step.  A sequence's splits write (m, l, o) partials; the
// last workgroup of a (sequence, kv head) to finish -- an arrival counter in
// the workspace -- merges them with the log-sum-exp rule and writes the
// output (the partials and the counter by agent-scope accesses, coherent
// across XCDs).
//
// Decode kernel work decomposition:
//   Workgroup = W waves = (split, sequence b, kv head h), split-major, so the
//   splits every sequence has are dispatched first and the workgroups of
//   splits past a context exit at once.  The G = Hq/Hkv q-heads of kv head h
//   are processed together, so each KV page is read from HBM once per kv
//   head (GQA).  Wave w takes tiles w, w + W, ... of the split: 8 KB tiles of
//   K (64 tokens at head_dim 64, 32 at 128).  The _t1 kernels have 8 waves,
//   one tile each (a split of 8 tiles); the _t2 kernels have 4 waves that
//   walk two tiles at a time, tile i computed while tile i+1 lands.
//   Prologue: the wave's block-table entries come through the scalar cache;
//   in the single-tile kernels q arrives by direct-to-LDS loads issued between
//   the tile's K and V loads, and the step variant's operands (q, k, v, their
//   biases and the cos/sin rows: one block per workgroup, loaded by wave 0)
//   by direct-to-LDS loads issued just before wave 0's K tile, so no
//   vector-memory round trip precedes the KV stream.  q is then held as the
//   A operands of the score MFMAs (D/4 registers: lane l holds 8 dims of
//   head l % 32 per 16-dim step, zero past the group).
//   Per tile:
//     1. K goes straight from HBM into LDS (global_load_lds_dwordx4; one
//        wave-wide load = 1 KB of a page), each token row's 16-byte chunks
//        XOR-keyed by kswz(token) so the per-token LDS reads are free of bank
//        conflicts; V goes
//        to registers in the same load layout (lane = token x 16-byte chunk).
//        All K loads of a tile precede its V loads, so the scores start as
//        soon as K has landed.
//     2. Scores: v_mfma_f32_32x32x16 with the heads as rows and the tokens
//        as columns (q the A operand, K read from LDS as the B operand); one
//        permlane32 swap per four heads then puts every head of a token in
//        that token's lane (x2 lanes per token at head_dim 128), the layout
//        of the softmax and PV.
//     3. Online softmax in the exp2 domain with a lazy reference point: the
//        running max moves (wave max by a DPP reduction, rescale of o) only
//        when a score passes it by more than kLazyMax.
//     4. o += p * V.  Single-tile kernels, head_dim 64 kernels and the
//        head_dim 128 tile-pair kernels without the step's append at group
//        size <= 7: O^T += V^T P^T on v_mfma_f32_32x32x16, V written into the
//        tile's K buffer once the scores have read it and read back
//        transposed (ds_read_b64_tr_b16), p through LDS head-major; o stays
//        in the MFMA accumulators.  The other head_dim 128 tile-pair kernels
//        (step variants, group size 8): V in its load layout, p of tokens t
//        and t + TILE/2 packed as a pair of the storage type, V of the same
//        two tokens paired by v_perm, one v_dot2_f32_{f16,bf16} per (head,
//        dim).  p is rounded where it is computed, so l sums the same values
//        the products use, and the running max is kept on whole numbers, so
//        that a token's p rounds alike in every split.
//   The dot2 form reduces each wave's token groups with permlane swaps
//   (reduce-scatter); the MFMA form's accumulators are already complete.
//   The W waves merge their (m, l, o) through LDS.  A
//   sequence with one split writes its output; otherwise each split writes
//   (m, l, o) to the workspace and the last split to arrive merges them.
//   The step variant's last workgroup also writes the roped q and k of the
//   new token back in place (after every split has read them).
#include "decode_args.h"
#include "luc_common.h"

namespace luc {

using DecodeArgs = ::luc_decode_args;
typedef __attribute__((address_space(3))) char lds_char;
typedef __attribute__((address_space(3))) void lds_void;

template <int D>
struct DecodeGeo {
  static constexpr int CH = D / 8;             // 16-byte chunks per token row
  static constexpr int TPL = 64 / CH;          // tokens per wave-wide 16-byte load
  static constexpr int TILE = 512 / CH;        // tokens per tile (8 KB of K)
  static constexpr int LOADS = TILE / TPL;     // K (and V) loads per lane per tile
  static constexpr int HALF = TILE / 2;        // PV pairs tokens t and t + HALF
  static constexpr int QKL = 64 / TILE;        // lanes per token for the scores
  static constexpr int LPP = kPage / TPL;      // load instructions per page
  static constexpr int PAGES = TILE / kPage;   // pages per tile
  static constexpr int ROWB = D * 2;           // bytes per token row
  static constexpr int KBYTES = TILE * ROWB;   // LDS bytes of one K tile
  static_assert(LOADS == 8 && TPL * ROWB == 1024, "one wave-wide load is 1 KB");
};

constexpr int kCpolNT = 2;  // non-temporal load: the KV stream is read once per step

// Byte offset of V[t][d .. d + 3] (d a multiple of 4) of a tile in LDS, for
// the transposing PV reads: 512-byte blocks of 8 tokens x 32 dims, block
// (t / 8, d / 32) at ((t / 8) * (D / 32) + d / 32) * 512, inside it token
// row (t + rot * (d / 32)) % 8 of 64 bytes, 8 bytes per 4 dims.  One
// transposing read (8 tokens x 32 dims) then covers one block, 256
// contiguous bytes per 32 lanes; the rotation by rot = 16 / (D / 8) rows per
// 32-dim block spreads the rows one 16-lane group of a 16-byte write touches
// (16 lanes x 16 bytes from load layout) over the whole bank row.
template <int D>
__device__ __host__ inline int vslot(int t, int d) {
  constexpr int NUB = D / 32, ROT = 16 / (D / 8);
  const int ub = d >> 5;
  return ((t >> 3) * NUB + ub) * 512 + (((t + ROT * ub) & 7) << 6) + (((d & 31) >> 2) << 3);
}

// XOR key of the 16-byte slots of token row t of a K tile in LDS (slot s of
// the row holds chunk s ^ key): the 16 rows one 16-lane group of the score
// reads touches (tokens 16i .. 16i + 15 of a 32-token block, one chunk each)
// fall on 16 different 16-byte bank groups of the 256-byte bank row.  A
// head_dim 64 row is half a bank row, so rows 2m and 2m + 1 (the two halves)
// share key m: (t >> 1) & 7.  A head_dim 128 row is a whole bank row, so
// the 16 rows need 16 keys: t & 15.
template <int D>
__device__ __host__ inline int kswz(int t) {
  return D == 64 ? (t >> 1) & 7 : t & 15;
}

// Row pitches (in elements) of per-head rows in LDS that lanes of different
// heads read together: padded so that the rows of the G <= 8 heads start on
// different banks (the unpadded rows, 128 or 256 bytes apart, put heads
// 0, 2, 4, 6 on the same banks).  p of a tile, head-major (16-bit, TILE
// tokens a row), 16 bytes of padding: row g starts at bank 36 g or 20 g
// (mod 64); the merge records' o (f32, D a row), 32 bytes: bank 8 g; the
// step variant's roped q (16-bit, D a row): bank 36 g (D = 64) or 8 g.
template <int TILE>
constexpr int kPPitch = TILE + 8;
template <int D>
constexpr int kRecPitch = D + 8;
template <int D>
constexpr int kQPitch = D + (D == 64 ? 8 : 16);

// Wait until at most N vector memory operations of this wave are in flight.
// They complete in issue order, so this also covers the LDS writes of
// global_load_lds, which the compiler does not track.
#define LUC_WAIT_VM(N) asm volatile("s_waitcnt vmcnt(" #N ")" ::: "memory")

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

// 4 bytes per lane from global memory straight into LDS at l + 4*lane.
__device__ inline void dma4(const void* g, lds_char* l) {
  __builtin_amdgcn_global_load_lds(g, (lds_void*)l, 4, 0, 0);
}

// The operands of one RoPE dword pair from LDS (byte addresses): x and bias
// words at dims j and j + D/2, the cos and sin of dims j, j + 1; complete on
// return.  asm for the reason given at lds_read4.
__device__ inline void lds_read_rope(uint32_t ax1, uint32_t ax2, uint32_t ab1, uint32_t ab2, uint32_t ac,
                                     uint32_t as, uint32_t& x1, uint32_t& x2, uint32_t& b1,
                                     uint32_t& b2, uint2& c, uint2& sn) {
  asm volatile(
      "ds_read_b32 %0, %6\n\t"
      "ds_read_b32 %1, %7\n\t"
      "ds_read_b32 %2, %8\n\t"
      "ds_read_b32 %3, %9\n\t"
      "ds_read_b64 %4, %10\n\t"
      "ds_read_b64 %5, %11\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(x1), "=&v"(x2), "=&v"(b1), "=&v"(b2), "=&v"(c), "=&v"(sn)
      : "v"(ax1), "v"(ax2), "v"(ab1), "v"(ab2), "v"(ac), "v"(as)
      : "memory");
}
__device__ inline void lds_read2(uint32_t a0, uint32_t a1, uint32_t& x0, uint32_t& x1) {
  asm volatile("ds_read_b32 %0, %2\n\tds_read_b32 %1, %3\n\ts_waitcnt lgkmcnt(0)"
               : "=&v"(x0), "=&v"(x1) : "v"(a0), "v"(a1) : "memory");
}

typedef __attribute__((address_space(4))) const int const_i32;
// N consecutive table entries in one scalar load (4-byte aligned).
template <int N>
struct I32Vec {
  typedef int T __attribute__((ext_vector_type(N), aligned(4)));
};

// Four 16-byte LDS reads, complete on return.  Written as one asm block so
// the compiler does not see them as reads of memory that global_load_lds may
// still be writing (it would wait for every outstanding load first); the
// caller orders them after the loads they need with LUC_WAIT_VM.
__device__ inline void lds_read4(uint32_t a0, uint32_t a1, uint32_t a2, uint32_t a3, uint4 (&x)[4]) {
  asm volatile(
      "ds_read_b128 %0, %4\n\t"
      "ds_read_b128 %1, %5\n\t"
      "ds_read_b128 %2, %6\n\t"
      "ds_read_b128 %3, %7\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(x[0]), "=&v"(x[1]), "=&v"(x[2]), "=&v"(x[3])
      : "v"(a0), "v"(a1), "v"(a2), "v"(a3)
      : "memory");
}

// 32-bit LDS address of a pointer into a __shared__ array.
__device__ inline uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const lds_char*)p;
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

// p of two tokens, already rounded to the storage type, as a pair of it
// (bf16: the high halves of the f32 bits).
template <int DT>
__device__ inline uint32_t pack_p(float lo, float hi) {
  if constexpr (DT == kF16) return pack_f16(lo, hi);
  else return __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u);
}

// The storage-type bits of a p already rounded to that type.
template <int DT>
__device__ inline uint16_t p_bits(float p) {
  if constexpr (DT == kF16) return __builtin_bit_cast(uint16_t, (_Float16)p);
  else return (uint16_t)(__float_as_uint(p) >> 16);
}

// The eight 16-byte rows of a tile held in load layout, load r to a0 + r KB
// (r even) or a1 + (r - 1) KB (r odd), in one asm block (the compiler sees no store to
// LDS, which would make it wait for the outstanding direct-to-LDS loads); the
// closing s_nop keeps the data registers of the last write from being
// overwritten by the instructions that follow.
__device__ inline void lds_write_tile(uint32_t a0, uint32_t a1, const uint4 (&v)[8]) {
  asm volatile(
      "ds_write_b128 %0, %2\n\t"
      "ds_write_b128 %1, %3\n\t"
      "ds_write_b128 %0, %4 offset:2048\n\t"
      "ds_write_b128 %1, %5 offset:2048\n\t"
      "ds_write_b128 %0, %6 offset:4096\n\t"
      "ds_write_b128 %1, %7 offset:4096\n\t"
      "ds_write_b128 %0, %8 offset:6144\n\t"
      "ds_write_b128 %1, %9 offset:6144\n\t"
      "s_nop 1" ::"v"(a0), "v"(a1), "v"(__builtin_bit_cast(u32x4_t, v[0])),
      "v"(__builtin_bit_cast(u32x4_t, v[1])), "v"(__builtin_bit_cast(u32x4_t, v[2])),
      "v"(__builtin_bit_cast(u32x4_t, v[3])), "v"(__builtin_bit_cast(u32x4_t, v[4])),
      "v"(__builtin_bit_cast(u32x4_t, v[5])), "v"(__builtin_bit_cast(u32x4_t, v[6])),
      "v"(__builtin_bit_cast(u32x4_t, v[7]))
      : "memory");
}

// Values written by asm loads issued earlier (not yet known to have landed):
// after the wait for them, pass each through an empty asm so that every use
// comes after that wait.
template <int N>
__device__ inline void pin_regs(uint4 (&x)[N]) {
#pragma unroll
  for (int i = 0; i < N; ++i) {
    u32x4_t v = __builtin_bit_cast(u32x4_t, x[i]);
    asm volatile("" : "+v"(v));
    x[i] = __builtin_bit_cast(uint4, v);
  }
}

// Issue (no wait) one transposing 8-byte LDS read at a + OFF: the result is
// not valid until lds_wait_pin has waited for it.
template <int OFF>
__device__ inline uint2 lds_tr_issue(uint32_t a) {
  uint2 x;
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(x) : "v"(a), "n"(OFF) : "memory");
  return x;
}
// Issue (no wait) an 8-byte LDS read at a + OFF.
template <int OFF>
__device__ inline uint2 lds_read8_issue(uint32_t a) {
  uint2 x;
  asm volatile("ds_read_b64 %0, %1 offset:%2" : "=v"(x) : "v"(a), "n"(OFF) : "memory");
  return x;
}
// Wait for every LDS access of the wave; the "+v" operands keep each use of
// the values read behind the wait.
__device__ inline void lds_wait_pin(uint2 (&x)[8]) {
  asm volatile("s_waitcnt lgkmcnt(0)"
               : "+v"(x[0]), "+v"(x[1]), "+v"(x[2]), "+v"(x[3]), "+v"(x[4]), "+v"(x[5]), "+v"(x[6]),
                 "+v"(x[7])
               :
               : "memory");
}
__device__ inline void lds_pin(uint2 (&x)[8]) {
  asm volatile(""
               : "+v"(x[0]), "+v"(x[1]), "+v"(x[2]), "+v"(x[3]), "+v"(x[4]), "+v"(x[5]), "+v"(x[6]),
                 "+v"(x[7]));
}

// x[i] for a wave-uniform runtime i < N, without indexing a register array.
template <int N>
__device__ __attribute__((always_inline)) inline float pick(const float (&x)[N], int i) {
  float r = x[0];
#pragma unroll
  for (int k = 1; k < N; ++k) r = i == k ? x[k] : r;
  return r;
}

// Split partials cross workgroups that may run on different XCDs, whose L2
// caches are not coherent with each other within a launch: they are written
// and read by agent-scope relaxed atomic accesses (global_store/load with the
// sc1 scope bit), which are coherent per access, instead of whole-cache
// write-back/invalidate fences.  A writer waits for its stores to complete
// before it counts its arrival; the merging split reads after it has seen the
// count.
__device__ inline void ws_store(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline float ws_load(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Log-sum-exp merge of the nsplit partials of one (sequence, kv head) by the
// NT threads of a workgroup -- the reference's partition merge
// (attention.cu:140-174) over splits: M = max m_s, L = sum l_s 2^(m_s - M),
// O = sum o_s 2^(m_s - M) / L.  s_w (G x 256 floats) and s_L (G floats) are
// LDS scratch.
template <int DT, int D, int G, int NT>
__device__ void lse_merge(const DecodeArgs& A, int bh, int nsplit, uint16_t* out_row, float* s_w,
                          float* s_L) {
  constexpr int GD = G * D;
  constexpr int NE = (GD + NT - 1) / NT;  // output elements per thread
  constexpr int SB = 16;                  // splits per batch of o loads
  constexpr int GW = (G + NT / 64 - 1) / (NT / 64);  // heads per wave
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const float* ml = A.ws_ml + (int64_t)bh * A.max_splits * G * 2;
  const float* po = A.ws_o + (int64_t)bh * A.max_splits * GD;
  // o of the first SB splits and (m, l) of every split go out together
  // (wave w reads heads w, w + NT/64, ...)
  float ob[SB][NE];
  auto load_batch = [&](int s0) {
#pragma unroll
    for (int j = 0; j < SB; ++j)
#pragma unroll
      for (int c = 0; c < NE; ++c) {
        const int e = min((int)threadIdx.x + NT * c, GD - 1);
        ob[j][c] = ws_load(po + (int64_t)min(s0 + j, nsplit - 1) * GD + e);
      }
  };
  float mv[GW][4], lv[GW][4];
  load_batch(0);
#pragma unroll
  for (int gi = 0; gi < GW; ++gi) {
    const int g = min(w + (NT / 64) * gi, G - 1);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int s = lane + 64 * k;
      mv[gi][k] = s < nsplit ? ws_load(ml + ((int64_t)s * G + g) * 2) : -INFINITY;
      lv[gi][k] = s < nsplit ? ws_load(ml + ((int64_t)s * G + g) * 2 + 1) : 0.0f;
    }
  }
  // weights of the splits: 2^(m_s - M), and L = sum l_s 2^(m_s - M)
#pragma unroll
  for (int gi = 0; gi < GW; ++gi) {
    const int g = w + (NT / 64) * gi;
    if (g < G) {
      const float M =
          wave_max(fmaxf(fmaxf(mv[gi][0], mv[gi][1]), fmaxf(mv[gi][2], mv[gi][3])));
      float L = 0.0f;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float wgt = __builtin_amdgcn_exp2f(mv[gi][k] - M);  // 0 past nsplit
        s_w[g * 256 + lane + 64 * k] = wgt;
        L = fmaf(wgt, lv[gi][k], L);
      }
      L = wave_sum(L);
      if (lane == 0) s_L[g] = L;
    }
  }
  __syncthreads();
  float acc[NE];
#pragma unroll
  for (int c = 0; c < NE; ++c) acc[c] = 0.0f;
  for (int s0 = 0; s0 < nsplit; s0 += SB) {
    if (s0 > 0) load_batch(s0);
#pragma unroll
    for (int j = 0; j < SB; ++j) {
      if (s0 + j < nsplit) {
#pragma unroll
        for (int c = 0; c < NE; ++c) {
          const int e = min((int)threadIdx.x + NT * c, GD - 1);
          acc[c] = fmaf(s_w[(e / D) * 256 + s0 + j], ob[j][c], acc[c]);
        }
      }
    }
  }
#pragma unroll
  for (int c = 0; c < NE; ++c) {
    const int e = threadIdx.x + NT * c;
    if (e < GD) out_row[e] = St<DT>::store(acc[c] / s_L[e / D]);
  }
}

// The step variant's roped q (G heads) and k of the new token, written back
// into the qkv row by the NT threads of the workgroup that finishes (b, h)
// last, after every split has read the row: copied from the LDS copies the
// workgroup's wave 0 roped (every split ropes the same values).
template <int D, int G, int NT>
__device__ void qk_writeback(const DecodeArgs& A, int b, int h, const uint16_t* sq,
                             const uint16_t* sk) {
  constexpr int QW = G * D / 2;  // 32-bit words of q
  uint32_t* qrow = (uint32_t*)(A.q + (int64_t)b * A.q_stride + (int64_t)h * G * D);
  uint32_t* krow = (uint32_t*)(A.k_new + (int64_t)b * A.q_stride + (int64_t)h * D);
  for (int i = threadIdx.x; i < QW + D / 2; i += NT) {
    // (sq holds head g's row at g * kQPitch<D> elements)
    if (i < QW) qrow[i] = ((const uint32_t*)sq)[(i / (D / 2)) * (kQPitch<D> / 2) + i % (D / 2)];
    else krow[i - QW] = ((const uint32_t*)sk)[i - QW];
  }
}

// The end of a split, shared by the decode kernels.  On entry each wave holds
// its running state over its own tokens in the load layout (lane = token row
// pv_tok x 16-byte chunk pv_ch of a 1 KB load): o[g][e] for head g and dim
// pv_ch * 8 + e, the wave-uniform reference point m_run[g] and the per-lane
// sums l_lane[g].  The wave's token rows are reduced with permlane swaps
// (reduce-scatter), the W waves merge their (m, l, o) records through LDS
// (wave v's record at recs + v * rec_stride floats; recs also serves as the
// cross-split merge's weight table, at least G * 257 floats), and the
// workgroup writes its output (one split) or its partial, whose arrival is
// counted; the last split of (b, h) to arrive merges the partials.  s_last is
// one word of LDS; sq / sk are the step variant's roped q and k of the new
// token, written back into the qkv row by the workgroup that finishes last.
template <int DT, int D, int G, bool APPEND, int W, bool MPV, int NO, int NA>
__device__ __attribute__((always_inline)) inline void finish_split(
    const DecodeArgs& A, float (&o)[NO][8], const f32x16 (&oacc)[NA], const float (&m_run)[G],
    const float (&l_lane)[G],
    float* recs, int rec_stride, uint32_t* s_last, const uint16_t* sq, const uint16_t* sk, int split,
    int bh, int b, int h, int nsplit, uint16_t* out_row) {
  constexpr int GD = G * D;
  constexpr int NV = 8 * G;  // o values per lane: 8 dims x G heads
  constexpr int CH = D / 8;  // 16-byte chunks per token row
  constexpr int NVP = (NV / 4 + 3) / 4 * 4;
  // MPV: the record holds o head-major (o[g][d] at g * kRecPitch<D> + d), then m and l
  constexpr int REC_ML = MPV ? G * kRecPitch<D> : 4 * CH * NVP;
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int pv_ch = lane % CH;
  float lsum[G];
#pragma unroll
  for (int g = 0; g < G; ++g) lsum[g] = l_lane[g];
  wave_sum_n<G>(lsum);
  float* const recw = recs + w * rec_stride;
  if constexpr (MPV) {
    // o is complete per head in the MFMA accumulators (lane l: head l % 32,
    // dims 32 db + 8 i + 4 (l / 32) + j in oacc[db][4 i + j])
    const int hh = lane & 31;
    if (hh < G) {
#pragma unroll
      for (int db = 0; db < NA; ++db)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          *(float4*)(recw + hh * kRecPitch<D> + 32 * db + 8 * i + 4 * (lane >> 5)) =
              make_float4(oacc[db][4 * i], oacc[db][4 * i + 1], oacc[db][4 * i + 2], oacc[db][4 * i + 3]);
    }
  } else {
  // ---- reduce the wave's token groups (lanes sharing pv_ch): reduce-scatter ----
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

  // ---- merge the W waves through LDS: each wave's record (o, m, l) ----
  // the lane holds o values of slot (lane / 16) * CH + pv_ch (value v: head v / 8,
  // dim pv_ch * 8 + v % 8)
  const bool writer = D == 128 || (lane & 8) == 0;
  if (writer) {
    float* const slot = recw + ((lane >> 4) * CH + pv_ch) * NVP;
#pragma unroll
    for (int k = 0; k < NVP; k += 4)
      *(float4*)(slot + k) = make_float4(y[k], k + 1 < NV / 4 ? y[k + 1] : 0.0f,
                                         k + 2 < NV / 4 ? y[k + 2] : 0.0f,
                                         k + 3 < NV / 4 ? y[k + 3] : 0.0f);
  }
  }
  if (lane == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      recw[REC_ML + g] = m_run[g];
      recw[REC_ML + G + g] = lsum[g];
    }
  }
  __syncthreads();
  const int64_t prec = (int64_t)bh * A.max_splits + split;  // this split's partial
  for (int e = threadIdx.x; e < GD; e += 64 * W) {
    const int g = e / D, d = e % D;
    const int val = g * 8 + d % 8;  // the value's index in the reduce-scatter
    const int idx = MPV ? g * kRecPitch<D> + d : ((val / (NV / 4)) * CH + d / 8) * NVP + val % (NV / 4);
    float mw[W], M = -INFINITY;
#pragma unroll
    for (int v = 0; v < W; ++v) {
      mw[v] = recs[v * rec_stride + REC_ML + g];
      M = fmaxf(M, mw[v]);
    }
    float O = 0.0f, L = 0.0f;
#pragma unroll
    for (int v = 0; v < W; ++v) {  // waves without tiles: m = -inf, weight 0
      const float* rv2 = recs + v * rec_stride;
      const float wt = __builtin_amdgcn_exp2f(mw[v] - M);
      O = fmaf(wt, rv2[idx], O);
      L = fmaf(wt, rv2[REC_ML + G + g], L);
    }
    if (nsplit == 1) {
      out_row[e] = St<DT>::store(O / L);
    } else {
      // partials by agent-scope stores (coherent across the XCDs' L2s), read
      // back the same way by the split that merges
      ws_store(A.ws_o + prec * GD + e, O);
      if (e % D == 0) {
        ws_store(A.ws_ml + (prec * G + g) * 2, M);
        ws_store(A.ws_ml + (prec * G + g) * 2 + 1, L);
      }
    }
  }

  // ---- the last split of (b, h) to finish merges the partials ----
  // Ordering of the hand-off (message passing between workgroups that may
  // sit on different XCDs):
  //  - every partial is written and read only by agent-scope atomic accesses
  //    (global_store / global_load with sc1): each one is performed at the
  //    point of coherence of the whole device, never in a non-coherent cache;
  //  - the compiler keeps the order: the volatile asm with a "memory" clobber
  //    and the barriers let no memory access move across them;
  //  - the hardware keeps the order: s_waitcnt vmcnt(0) returns only when
  //    this wave's stores are acknowledged, so every partial has reached the
  //    point of coherence before the barrier and thread 0's counter update;
  //  - the merging workgroup issues its partial loads only after its update
  //    returned nsplit - 1 (passed on through s_last and a barrier), so
  //    they are performed after every other split's stores.
  // A release / acquire pair at agent scope would add a write-back and an
  // invalidation of the whole L2 (buffer_wbl2 / buffer_inv), needed only for
  // data written by plain stores; none of the merge's data is, and with them
  // the kernel measured 5x slower.
  if (nsplit > 1) {
    // this wave's partial stores have completed (at agent scope) before the
    // workgroup's arrival is counted
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    // whether this workgroup is the last split of (b, h) to finish, passed
    // through s_last
    if (threadIdx.x == 0) {
      const int old = __hip_atomic_fetch_add(A.ws_cnt + bh, 1, __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT);
      *s_last = old == nsplit - 1;
      // the counter goes back to zero for the next launch
      if (old == nsplit - 1)
        __hip_atomic_store(A.ws_cnt + bh, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!*s_last) return;
    if constexpr (APPEND) qk_writeback<D, G, 64 * W>(A, b, h, sq, sk);
    // every other split's partial is complete: the agent-scope loads of
    // lse_merge see them
    float* const s_w = recs;  // the records were read above
    lse_merge<DT, D, G, 64 * W>(A, bh, nsplit, out_row, s_w, s_w + G * 256);
  } else if constexpr (APPEND) {
    qk_writeback<D, G, 64 * W>(A, b, h, sq, sk);
  }
}

// Work item i of a split-K launch of the tile-pair kernels, longest first.
// A workgroup's time grows with its split's length.  In plain split-major
// order the longest sequences' full splits are the last to start, the short
// last splits of all sequences are spread over every round, and workgroups
// of splits past a context take a slot each; the launch ends on long
// workgroups that started late.  Here the grid's workgroups take, in order:
//   1. the full splits (split s of a sequence whose context holds
//      (s + 1) * split_tokens tokens): first the rounds that every valid
//      sequence has (s < n_min, the fewest full splits of a valid sequence)
//      split-major, as in plain order; then the rest sequence-major
//      (sequence b's splits n_min.. in order), kv heads adjacent throughout;
//   2. each sequence's last, partial split, longest first: ordered by its
//      length in rounds of UT tokens (one tile for each of the W waves, so
//      equal rounds are equal work), from the longest class down, sequences
//      in index order within a class, kv heads adjacent;
//   3. nothing: the workgroups past the last item return at once.
// A sequence whose position is invalid (empty context or past max_ctx) gets
// one item in part 2, split 0, with the shortest class; its workgroup writes
// the NaN output.  Every (split, sequence, kv head) that the split-K merge
// counts is exactly one item, so the grid of max_splits * batch * hkv
// workgroups holds them all.  Returns split * pairs + b * hkv + h, or -1.
// Lane b of the wave takes sequence b (batch <= kLfMaxBatch = 64 and at most
// 256 kv heads; other launches keep plain split-major order): one load of
// the positions, then ballots only, so every lane computes the same,
// wave-uniform item.
constexpr int kLfMaxBatch = 64;
// floor(n / d) for 0 <= n < 2^22 and d > 0 (the operands here: contexts
// below 2^20, item numbers below 256 splits x 64 sequences x 256 kv heads):
// the float quotient is within one of it, and one step either way corrects it
__device__ inline int quot24(int n, int d) {
  int q = (int)((float)n * __builtin_amdgcn_rcpf((float)d));
  q += (q + 1) * d <= n ? 1 : (q * d > n ? -1 : 0);
  return q;
}
template <int UT>
__device__ int longest_first_item(const DecodeArgs& A, int i, int pairs) {
  constexpr int NQB = 16;  // length classes: split_tokens (<= 2048) / UT (>= 128)
  const int lane = threadIdx.x & 63;
  const int ST = A.split_tokens, hkv = A.hkv, B = A.batch;
  const int ctx = A.positions[min(lane, B - 1)] + 1;  // (lanes past the batch: unused)
  const bool ok = lane < B && ctx >= 1 && ctx <= A.max_ctx;
  const int nfull = ok ? quot24(ctx, ST) : 0;  // <= max_splits <= 256: nine bit planes
  const int r = ok ? ctx - nfull * ST : (lane < B ? 1 : 0);  // tokens of the partial split
  const int cls = r > 0 ? min((r + UT - 1) / UT, NQB) : 0;  // 0: no partial split
  // every valid sequence with the same full splits and none partial: plain
  // split-major order is already longest first
  const int n0 = __builtin_amdgcn_readfirstlane(nfull);
  if (__ballot(ok) == __ballot(lane < B) && !__ballot(lane < B && (nfull != n0 || cls > 0)))
    return i < n0 * pairs ? i : -1;
  int t = __builtin_amdgcn_readfirstlane(quot24(i, hkv));
  const int h = i - t * hkv;
  // set bits of m in the lanes below this one; the lane of the k-th set bit
  auto below = [&](uint64_t m) {
    return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                          __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0));
  };
  auto select = [&](uint64_t m, int k) {
    return (int)__builtin_ctzll(__ballot(((m >> lane) & 1) && below(m) == k));
  };
  // part 1a: the complete rounds.  n_min, the fewest full splits of a valid
  // sequence, bit plane by bit plane from the top
  const uint64_t valid = __ballot(ok);
  uint64_t cand = valid;
  int nmin = 0;
#pragma unroll
  for (int k = 8; k >= 0; --k) {
    const uint64_t zero = cand & __ballot(((nfull >> k) & 1) == 0);
    if (zero) cand = zero;
    else nmin |= 1 << k;
  }
  if (!valid) nmin = 0;  // (no valid sequence: no full split at all)
  const int nvalid = __popcll(valid);
  if (t < nmin * nvalid) {  // (nvalid > 0 here)
    const int split = __builtin_amdgcn_readfirstlane(quot24(t, nvalid));
    return split * pairs + select(valid, t - split * nvalid) * hkv + h;
  }
  t -= nmin * nvalid;
  // part 1b: the other full splits, sequence-major: the inclusive prefix of
  // nfull - n_min over the lanes, bit plane by bit plane, and the total
  const int nrest = ok ? nfull - nmin : 0;
  int incl = 0, tot = 0;
#pragma unroll
  for (int k = 0; k < 9; ++k) {
    const int bit = (nrest >> k) & 1;
    const uint64_t m = __ballot(bit);
    incl += (below(m) + bit) << k;
    tot += __popcll(m) << k;
  }
  if (t < tot) {
    const int l = (int)__builtin_ctzll(__ballot(incl > t));
    const int split = nmin + t - __builtin_amdgcn_readlane(incl - nrest, l);
    return split * pairs + l * hkv + h;
  }
  t -= tot;
  // part 2: the t-th partial split in (class descending, lane) order, by a
  // radix select over the class's five bit planes
  cand = __ballot(cls > 0);
  if (t >= __popcll(cand)) return -1;  // past the last item
#pragma unroll
  for (int k = 4; k >= 0; --k) {
    const uint64_t ones = cand & __ballot((cls >> k) & 1);
    const int n1 = __popcll(ones);
    if (t < n1) {
      cand = ones;
    } else {
      t -= n1;
      cand &= ~ones;
    }
  }
  const int l = select(cand, t);
  return __builtin_amdgcn_readlane(nfull, l) * pairs + l * hkv + h;
}

template <int DT, int D, int G, bool APPEND, int W, int NB>
__device__ void decode_impl(const DecodeArgs& A) {
  using S = DecodeGeo<D>;
  constexpr int PP = kPPitch<S::TILE>;  // head-major p row pitch (elements)
  // p exchange, 32-bit words: G pairs per token pair (dot2 form), or G
  // head-major rows of PP 16-bit values (MPV)
  constexpr int PWORDS = S::HALF * 8 > (G * PP + 1) / 2 ? S::HALF * 8 : (G * PP + 1) / 2;
  constexpr int HD = D / 2;
  constexpr int GD = G * D;
  constexpr int NV = 8 * G;  // o values per lane: 8 dims x G heads
  constexpr int WS = W * S::TILE;  // tokens between two tiles of one wave
  // Single-tile kernels (T1): no vector-memory round trip before the KV
  // stream.  The wave's page numbers come through the scalar cache, and q
  // (FASTQ) by 4-byte direct-to-LDS loads issued between the tile's K and V
  // loads (behind the same K wait), or the step variant's operands (FASTA:
  // q, k, v, their biases, the cos/sin rows) by such loads issued by wave 0
  // just before its K tile (so its RoPE, which every wave waits for, does
  // not wait for the tile), instead of vector loads that would queue behind
  // the KV streams other waves of the CU have already issued.
  constexpr bool T1 = NB == 1;
  constexpr bool FASTQ = T1 && !APPEND;
  constexpr bool FASTA = T1 && APPEND;
  // Scores on the matrix cores: q as the A operand of v_mfma_f32_32x32x16, KS
  // k-steps of 16 dims, NBLK blocks of 32 tokens per tile.
  constexpr int KS = D / 16;
  constexpr int NBLK = S::TILE / 32;
  // PV on the matrix cores too (MPV): O^T += V^T P^T, V staged in the tile's
  // own K buffer once the scores have read it; o is then held as D/32 MFMA
  // accumulators (lane l: head l % 32, dims 32 db + 8 i + 4 (l / 32) + j).
  // Not in the head_dim 128 tile-pair step kernels nor at group size 8
  // there, whose 64 accumulators would not fit beside the tile pair in
  // flight and the step operands (they take the dot2 form).
  constexpr bool MPV = T1 || D == 64 || (!APPEND && G <= 7);
  constexpr int ND = D / 32;
  constexpr int NQ = (GD * 2 + 255) / 256;  // 4-byte direct-to-LDS loads for q
  // FASTA operand block: q of the G heads, then their biases (256-byte
  // padded), then six regions of 2*D bytes: k, k bias, cos, sin, v, v bias.
  constexpr int SR = 2 * D;
  constexpr int PA_XQ = 0, PA_BQ = NQ * 256, PA_SM = 2 * NQ * 256;
  constexpr int PA_K = PA_SM, PA_KB = PA_SM + SR, PA_C = PA_SM + 2 * SR, PA_S = PA_SM + 3 * SR;
  constexpr int PA_V = PA_SM + 4 * SR, PA_VB = PA_SM + 5 * SR;
  constexpr int NSM = 6 * SR / 256;  // loads for the six small regions
  constexpr int PBYTES = PA_SM + 6 * SR;
  // Per wave: NB K tile buffers (the first one later holds the wave's merge
  // record: o[G*D], m[G], l[G]) and the p exchange.  The step variant's roped
  // q and new token's k and v: per wave in the two-tile kernels; one copy per
  // workgroup in the single-tile kernels (FASTA), where wave 0 loads the
  // operand block and ropes it for all four (so the workgroup fits 40 KB of
  // LDS: four per CU).
  // merge record: after the reduce-scatter, writer lane (j = lane / 16,
  // chunk pv_ch) holds the o values j * NV/4 + k, k < NV/4 (value v: head
  // v / 8, dim pv_ch * 8 + v % 8); it stores them at slot j * CH + pv_ch,
  // NVP floats per slot, followed by m[G] and l[G] of the wave.
  constexpr int NVP = (NV / 4 + 3) / 4 * 4;
  constexpr int REC_ML = 4 * S::CH * NVP;
  static_assert(REC_ML + 2 * G <= S::KBYTES / 4, "merge record fits a K buffer");
  static_assert(G * kRecPitch<D> + 2 * G <= S::KBYTES / 4, "head-major merge record fits a K buffer");
  static_assert(G * PP * 2 <= PWORDS * 4, "p of the tile, head-major, fits the p exchange");
  __shared__ __attribute__((aligned(16))) char s_k[W][NB][S::KBYTES];
  __shared__ __attribute__((aligned(16))) uint32_t s_p[W][PWORDS];
  constexpr int NOP = (APPEND && !FASTA) ? W : 1;  // copies of the step operands
  constexpr int QP = kQPitch<D>;  // s_q / s_qr row pitch (elements)
  constexpr int NQL = (G * QP * 2 + 255) / 256;  // 4-byte direct-to-LDS loads of q, padded rows
  __shared__ __attribute__((aligned(16))) uint16_t s_q[NOP][APPEND ? G * QP : 8];
  __shared__ __attribute__((aligned(16))) char s_qr[FASTQ ? W : 1][FASTQ ? NQL * 256 : 16];
  __shared__ __attribute__((aligned(16))) uint16_t s_knew[NOP][APPEND ? D : 8];
  __shared__ __attribute__((aligned(16))) uint16_t s_vnew[NOP][APPEND ? D : 8];
  __shared__ __attribute__((aligned(16))) char s_pa[1][FASTA ? PBYTES : 16];
  static_assert((G * 256 + G) * 4 <= W * NB * S::KBYTES, "merge weights fit the K buffers");

  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave of the workgroup
  const int qi = NOP == 1 ? 0 : w;  // this wave's copy of the step operands
  const int pairs = A.batch * A.hkv;
  // the workgroup's (split, sequence, kv head): split-major, or longest first
  // (tile-pair kernels with more than one split; the position comes with it)
  int item = blockIdx.x;  // split * pairs + b * hkv + h
  if (!T1 && A.max_splits > 1 && A.batch <= kLfMaxBatch && A.hkv <= 256) {
    item = __builtin_amdgcn_readfirstlane(longest_first_item<WS>(A, item, pairs));
    if (item < 0) return;
  }
  const int split = item / pairs;
  const int bh = item - split * pairs;
  const int b = bh / A.hkv, h = bh - b * A.hkv;
  const int ST = A.split_tokens;
  const int s_begin = split * ST;
  const int64_t page_stride = (int64_t)A.num_layers * A.hkv * kPage * D;
  const int64_t head_off = ((int64_t)A.layer * A.hkv + h) * kPage * D;
  const int* trow = A.tables + (int64_t)b * A.table_stride;
  const int tmax = (int)A.table_stride - 1;
  uint16_t* out_row = A.out + (int64_t)b * A.out_stride + (int64_t)h * GD;
  const uint16_t* qrow = A.q + (int64_t)b * A.q_stride + (int64_t)h * GD;

  // ---- prologue: position, the split's table entries and q together ----
  const int p0 = s_begin / kPage;  // lane j of tab0 / tab1: page j / 64 + j of the split
  const int tab0 = T1 ? 0 : trow[min(p0 + lane, tmax)];
  const int tab1 = !T1 && ST > 64 * kPage ? trow[min(p0 + 64 + lane, tmax)] : 0;
  // The A operand of k-step ks, q[head lane % 32][16 ks + 8 (lane / 32)
  // .. + 8] of a row of the G heads' q (4-byte aligned); zero past head G - 1.
  auto q_operand = [&](const uint16_t* row, int ks, int pitch = D) {
    const int g = lane & 31;
    const uint32_t* p = (const uint32_t*)(row + min(g, G - 1) * pitch + 16 * ks + 8 * (lane >> 5));
    const uint4 v = make_uint4(p[0], p[1], p[2], p[3]);
    return g < G ? v : make_uint4(0, 0, 0, 0);
  };
  // single-tile kernel: the page numbers of the wave's tile, through the
  // scalar cache in the same round trip as the position (clamped to the
  // split once the position is known)
  // (PAGES entries from tstart: inside the row, which the host guarantees
  // holds at least PAGES entries for this kernel)
  const int j0 = w * S::PAGES;  // first page of the wave's tile within the split
  const int tstart = min(p0 + j0, tmax - (S::PAGES - 1));
  int traw[S::PAGES];
  if constexpr (T1) {
    typedef __attribute__((address_space(4))) const typename I32Vec<S::PAGES>::T vec_t;
    const auto v = *(vec_t*)(trow + tstart);
#pragma unroll
    for (int i = 0; i < S::PAGES; ++i) traw[i] = v[i];
  }
  uint4 qm[KS];  // q as MFMA A operands
  if constexpr (!APPEND && !FASTQ) {
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) qm[ks] = q_operand(qrow, ks);
  }
  int pos = A.positions[b];
  if constexpr (T1) {
    // the table entries and the position share one scalar round trip
    // (readfirstlane: both are wave-uniform, it only names the register class)
    pos = __builtin_amdgcn_readfirstlane(pos);
#pragma unroll
    for (int i = 0; i < S::PAGES; ++i)
      asm volatile("" : "+s"(pos) : "s"(__builtin_amdgcn_readfirstlane(traw[i])));
  }
  const int ctx = pos + 1;
  if (ctx < 1 || ctx > A.max_ctx) {
    // empty context (0/0 in the reference) or beyond the host bound: NaN
    if (split == 0)
      for (int i = threadIdx.x; i < GD; i += 64 * W) out_row[i] = St<DT>::store(__builtin_nanf(""));
    return;
  }
  if (s_begin >= ctx) return;  // split past this context (the whole workgroup)
  const int nsplit = (ctx + ST - 1) / ST;
  const int s_end = min(ctx, s_begin + ST);
  // this wave's tiles: s_begin + (w + i * W) * TILE, i < ntw
  const int t_first = s_begin + w * S::TILE;
  const int ntw = t_first < s_end ? (s_end - t_first + WS - 1) / WS : 0;
  // the wave whose tiles hold the new token (in the last split)
  const bool owns = APPEND && pos >= s_begin && pos < s_end && ((pos - s_begin) / S::TILE) % W == w;
  // Page numbers outside the pool are never used as addresses: such a page
  // reads page 0 instead and the wave's result is poisoned with NaN below
  // (bad_page is wave-uniform).
  const int nb = A.num_blocks;
  bool bad_page = false;
  auto page_raw = [&](int j) -> int {  // table entry of page j of the split (uniform j)
    return j < 64 ? __builtin_amdgcn_readlane(tab0, j) : __builtin_amdgcn_readlane(tab1, j - 64);
  };
  auto page_of = [&](int j) -> int64_t {  // physical page j of the split, inside the pool
    const int p = page_raw(j);
    const bool ok = p >= 0 && p < nb;
    bad_page |= !ok;
    return ok ? p : 0;
  };
  const int jend = (s_end - 1 - s_begin) / kPage;  // last page of the split
  // single-tile kernel: the pages of this wave's tile (clamped to the split)
  int tpage[S::PAGES];
  // T1: table entry of the new token's page (page jt_new of the owner wave's
  // tile; only the owner uses it)
  const int jt_new = (pos - t_first) / kPage;
  int new_raw = 0;
  if constexpr (T1) {
#pragma unroll
    for (int i = 0; i < S::PAGES; ++i) {
      // entry of page min(j0 + i, jend) of the split in traw (waves without
      // a tile issue nothing, the index is only kept in range for them)
      const int e = min(max(min(p0 + j0 + i, p0 + jend) - tstart, 0), S::PAGES - 1);
      int t = traw[0];
#pragma unroll
      for (int k = 1; k < S::PAGES; ++k) t = e == k ? traw[k] : t;
      const bool ok = t >= 0 && t < nb;
      if (!ok && ntw > 0) bad_page = true;
      tpage[i] = ok ? t : 0;
      new_raw = jt_new == i ? t : new_raw;
    }
  }

  // The step variant's prologue operands (q and k of the new token with their
  // biases, the cos/sin row, v + v_bias) are loaded before the KV stream is
  // issued, so using them does not wait for it.
  constexpr int NPAIR = APPEND ? ((G + 1) * HD + 63) / 64 : 1;
  uint16_t rx1[NPAIR], rx2[NPAIR], rb1[NPAIR], rb2[NPAIR], rv[S::QKL], rvb[S::QKL];
  float rc[NPAIR], rs[NPAIR];
  if constexpr (APPEND && !T1) {
    const float* crow = A.cos_t + (int64_t)pos * HD;
    const float* srow = A.sin_t + (int64_t)pos * HD;
    const uint16_t* krow = A.k_new + (int64_t)b * A.q_stride + (int64_t)h * D;
#pragma unroll
    for (int i = 0; i < NPAIR; ++i) {
      const int idx = min(lane + i * 64, (G + 1) * HD - 1);
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
#pragma unroll
    for (int i = 0; i < S::QKL; ++i) {
      const int d = lane + 64 * i;
      rv[i] = A.v_new[(int64_t)b * A.q_stride + (int64_t)h * D + d];
      rvb[i] = A.v_bias ? A.v_bias[(int64_t)h * D + d] : 0;
    }
  }

  const int tq = lane % S::TILE;     // scores: token of this lane
  const int qh = lane / S::TILE;     // scores: which 64 dims (head_dim 128)
  const int pv_tok = lane / S::CH;   // load layout: token within a load
  const int pv_ch = lane % S::CH;    // load layout: 16-byte chunk of the row

  // Per-lane byte offsets inside a (page, layer, kv head) slab.  Load r reads
  // page r / LPP at + (r % LPP) * 1KB; the K slot pv_ch of token tl holds
  // chunk pv_ch ^ kswz(tl), tl = r * TPL + pv_tok.  kswz(tl) is
  // kswz(pv_tok) ^ 4 (r % NKO) (head_dim 64: 8 tokens a load, key
  // (tl >> 1) & 7; 128: 4 tokens, key tl & 15), so load r's offset is
  // koff0 ^ (r % NKO) << 6 (the XOR stays inside the chunk bits).
  constexpr int NKO = D == 64 ? 2 : 4;
  const uint32_t koff0 = (uint32_t)(pv_tok * S::ROWB + ((pv_ch ^ kswz<D>(pv_tok)) << 4));
  const uint32_t voff = (uint32_t)(pv_tok * S::ROWB + (pv_ch << 4));

  // Issue one tile: all its K loads (into K buffer buf) before its V loads
  // (into vr).  Pages past the split re-read the split's last page (a cache
  // hit), which keeps the number of loads per tile fixed at 8 + 8; a tile
  // that starts past the split (the odd tile of a pair) is all such pages.
  // In the single-tile kernel q follows the K loads (NQL more loads).
  auto phys_of = [&](int t0, int r) __attribute__((always_inline)) -> int64_t {
    if constexpr (T1) return tpage[r / S::LPP];  // (t0 is the wave's only tile)
    else return page_of(min((t0 - s_begin) / kPage + r / S::LPP, jend));
  };
  // Issued by every wave, with or without a tile, before its K tile.
  auto issue_operands = [&]() __attribute__((always_inline)) {
    // The workgroup's operand block goes out first, so that the RoPE which
    // every wave waits for needs only these loads, not the K tiles behind
    // them; its 4-byte loads are dealt round robin over the waves (load i by
    // wave i % W), so no wave's K tile waits behind all of them.
    if constexpr (FASTA) {
      // a missing bias reads the operand itself (ignored)
      const char* krow = (const char*)(A.k_new + (int64_t)b * A.q_stride + (int64_t)h * D);
      const char* vrow = (const char*)(A.v_new + (int64_t)b * A.q_stride + (int64_t)h * D);
      const char* qb = A.q_bias ? (const char*)(A.q_bias + (int64_t)h * GD) : (const char*)qrow;
      const char* kb = A.k_bias ? (const char*)(A.k_bias + (int64_t)h * D) : krow;
      const char* vb = A.v_bias ? (const char*)(A.v_bias + (int64_t)h * D) : vrow;
      const char* cr = (const char*)(A.cos_t + (int64_t)pos * HD);
      const char* sr = (const char*)(A.sin_t + (int64_t)pos * HD);
      lds_char* pa = (lds_char*)s_pa[0];
#pragma unroll
      for (int i = 0; i < NQ; ++i) {
        const int off = min(i * 256 + lane * 4, GD * 2 - 4);
        if ((2 * i) % W == w) dma4((const char*)qrow + off, pa + PA_XQ + i * 256);
        if ((2 * i + 1) % W == w) dma4(qb + off, pa + PA_BQ + i * 256);
      }
      const char* small[6] = {krow, kb, cr, sr, vrow, vb};
#pragma unroll
      for (int i = 0; i < NSM; ++i) {
        const int o = i * 256 + lane * 4;  // byte of the six regions
        const int reg = o / SR;
        const char* src = small[0];
#pragma unroll
        for (int k = 1; k < 6; ++k) src = reg == k ? small[k] : src;
        if ((2 * NQ + i) % W == w) dma4(src + (o - reg * SR), pa + PA_SM + i * 256);
      }
    }
  };
  auto issue_k = [&](int t0, int buf) __attribute__((always_inline)) {
    lds_char* kdma = (lds_char*)s_k[w][buf];
#pragma unroll
    for (int r = 0; r < S::LOADS; ++r) {
      const int64_t phys = phys_of(t0, r);
      // wave-uniform slab base (scalar registers) + 32-bit lane offsets
      const char* kslab = (const char*)(A.k_pool + phys * page_stride + head_off);
      dma16(kslab + (koff0 ^ ((r % NKO) << 6)), kdma + (r - r % S::LPP) * 1024,
            (r % S::LPP) * 1024);
    }
    if constexpr (FASTQ) {
      // q by 4-byte direct-to-LDS loads into head rows QP elements apart
      // (padded: the A-operand reads of different heads then fall on
      // different banks); the padding words re-read the row's start
#pragma unroll
      for (int i = 0; i < NQL; ++i) {
        const int o = i * 256 + lane * 4;  // LDS byte of the padded block
        const int g = min(o / (QP * 2), G - 1), ob = o % (QP * 2);
        dma4((const char*)qrow + g * D * 2 + (ob < D * 2 ? ob : 0), (lds_char*)s_qr[w] + i * 256);
      }
    }
  };
  auto issue_v = [&](int t0, uint4(&vr)[S::LOADS]) __attribute__((always_inline)) {
#pragma unroll
    for (int r = 0; r < S::LOADS; ++r) {
      const int64_t phys = phys_of(t0, r);
      const char* vslab = (const char*)(A.v_pool + phys * page_stride + head_off);
      vr[r] = ld_nt16((const uint16_t*)(vslab + voff + (r % S::LPP) * 1024));
    }
  };
  auto issue = [&](int t0, int buf, uint4(&vr)[S::LOADS]) __attribute__((always_inline)) {
    issue_k(t0, buf);
    issue_v(t0, vr);
  };

  // Everything loaded so far (q, or the step variant's operands) must have
  // landed before the KV stream is issued (it came with the table and
  // position loads): the compiler then needs no wait for it behind the
  // stream, where it could only wait for the whole stream.
  if constexpr (T1) {
  } else if constexpr (!APPEND) {
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) asm volatile("" ::"v"(qm[ks].x), "v"(qm[ks].y), "v"(qm[ks].z), "v"(qm[ks].w));
  } else {
#pragma unroll
    for (int i = 0; i < NPAIR; ++i)
      asm volatile("" ::"v"(rx1[i]), "v"(rx2[i]), "v"(rb1[i]), "v"(rb2[i]), "v"(rc[i]), "v"(rs[i]));
#pragma unroll
    for (int i = 0; i < S::QKL; ++i) asm volatile("" ::"v"(rv[i]), "v"(rvb[i]));
  }
  uint4 vr0[S::LOADS], vr1[S::LOADS];
  if constexpr (NB == 1) {
    // every wave's K (and q) goes out before any wave's V: the CU's memory
    // pipeline returns them roughly in that order, so the scores of all the
    // waves overlap the V stream and only PV is left once the last V lands
    issue_operands();
    if (ntw > 0) issue_k(t_first, 0);
    __builtin_amdgcn_s_barrier();
    if (ntw > 0) issue_v(t_first, vr0);
  } else if (ntw > 0) {
    if constexpr (!APPEND && MPV) {  // K_a K_b V_a V_b (PREK below)
      issue_k(t_first, 0);
      issue_k(t_first + WS, 1);
      issue_v(t_first, vr0);
      issue_v(t_first + WS, vr1);
    } else {  // K_a V_a K_b V_b
      issue(t_first, 0, vr0);
      issue(t_first + WS, 1, vr1);
    }
  }

  // ---- q of the G heads (roped in the step variant), new token's k, v ----
  if constexpr (APPEND && !T1) {
#pragma unroll
    for (int i = 0; i < NPAIR; ++i) {
      const int idx = lane + i * 64;
      if (idx < (G + 1) * HD) {
        const int g = idx / HD, j = idx % HD;
        uint16_t o1, o2;
        rot_pair<DT>(rx1[i], rb1[i], rx2[i], rb2[i], rc[i], rs[i], o1, o2);
        uint16_t* dst = g < G ? s_q[qi] + g * QP : s_knew[qi];
        dst[j] = o1;
        dst[j + HD] = o2;
      }
    }
#pragma unroll
    for (int i = 0; i < S::QKL; ++i)
      s_vnew[qi][lane + 64 * i] = St<DT>::store(St<DT>::load(rv[i]) + St<DT>::load(rvb[i]));
    wave_lds_sync();
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) qm[ks] = q_operand(s_q[qi], ks, QP);
  }

  float m_run[G], l_lane[G], o[MPV ? 1 : G][8];
  f32x16 oacc[MPV ? ND : 1];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m_run[g] = -INFINITY;
    l_lane[g] = 0.0f;
  }
  if constexpr (MPV) {
#pragma unroll
    for (int db = 0; db < ND; ++db) oacc[db] = f32x16{};
  } else {
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int e = 0; e < 8; ++e) o[g][e] = 0.0f;
  }

  // ---- scores, online softmax and p exchange of the tile at t0 (K in buf) ----
  auto tile_scores = [&](int t0, int buf) __attribute__((always_inline)) {
    char* const kb = s_k[w][buf];
    if constexpr (APPEND) {
      if (owns && pos >= t0 && pos < t0 + S::TILE && lane < S::CH) {
        const int t = pos - t0;  // the new token's K row (swizzled slots)
        *(uint4*)(kb + t * S::ROWB + lane * 16) =
            *(const uint4*)(s_knew[qi] + ((lane ^ kswz<D>(t)) * 8));
      }
      wave_lds_sync();
    }
    float acc[G];
    // S = Q K^T on the matrix cores, per 32-token block: rows = the
    // group's heads, columns = tokens, B lane = (token lane % 32, 8 dims
    // of chunk 2 ks + lane / 32).  Lane l then holds heads 4(l/32) + j of
    // token l % 32 in sc[.][j]; one permlane32 swap per j gives every lane
    // heads j and 4 + j of its own token (lane = token at head_dim 64,
    // token lane % 32 in both lane halves at 128).
    f32x16 sc[NBLK];
#pragma unroll
    for (int nb = 0; nb < NBLK; ++nb) {
      sc[nb] = f32x16{};
      const int tok = nb * 32 + (lane & 31);
      const uint32_t kr = lds_addr(kb) + tok * S::ROWB;
      const int sw = kswz<D>(tok);
      auto kaddr = [&](int ks) { return kr + ((uint32_t)((2 * ks + (lane >> 5)) ^ sw) << 4); };
#pragma unroll
      for (int k4 = 0; k4 < KS; k4 += 4) {
        uint4 kc[4];
        lds_read4(kaddr(k4), kaddr(k4 + 1), kaddr(k4 + 2), kaddr(k4 + 3), kc);
#pragma unroll
        for (int i = 0; i < 4; ++i) sc[nb] = mfma32<DT>(qm[k4 + i], kc[i], sc[nb]);
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(sc[0][j]),
                                                      __float_as_uint(sc[NBLK - 1][j]), false, false);
      if (j < G) acc[j] = __uint_as_float(r[0]);
      if (4 + j < G) acc[4 + j] = __uint_as_float(r[1]);
    }

    const bool valid = (t0 + tq) < s_end;
    float p[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float s = valid ? acc[g] * A.qk_scale_log2 : -INFINITY;
      // The reference point m_run[g] only has to keep exp2(s - m_run) small:
      // it starts at the score of lane 0 (the tile's first token, always
      // valid in a wave's first tile) and moves (wave-wide max, rescale of o
      // and l) only when a score exceeds it by more than kLazyMax, which one
      // ballot detects; p stays <= 2^kLazyMax.  It is kept on whole numbers:
      // the p of one token in two splits then differ by a power of two, so
      // they round alike to the storage type, and the merge weights
      // 2^(m_s - M) are exact.
      if (m_run[g] == -INFINITY)  // wave-uniform: the wave's first tile
        m_run[g] = floorf(__builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, s))));
      if (__builtin_amdgcn_ballot_w64(s > m_run[g] + kLazyMax) != 0) {  // wave-uniform
        const float mn = floorf(__builtin_bit_cast(
            float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, fmaxf(m_run[g], wave_max(s))))));
        if (m_run[g] > -INFINITY) {  // (nothing accumulated before the first tile)
          const float alpha = __builtin_amdgcn_exp2f(m_run[g] - mn);
          l_lane[g] *= alpha;
          if constexpr (MPV) {  // head g's accumulators are in lanes g and g + 32
            const bool mine = (lane & 31) == g;
#pragma unroll
            for (int db = 0; db < ND; ++db)
#pragma unroll
              for (int k = 0; k < 16; ++k) oacc[db][k] = mine ? oacc[db][k] * alpha : oacc[db][k];
          } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) o[g][e] *= alpha;
          }
        }
        m_run[g] = mn;
      }
      p[g] = __builtin_amdgcn_exp2f(s - m_run[g]);
      // p rounds to the storage type for the PV dot products, and l sums
      // the rounded values, so the output weights stay normalised (a single
      // dominant token gives its V exactly)
      if constexpr (DT == kBF16) p[g] = (float)(__bf16)p[g];
      else p[g] = (float)(_Float16)p[g];
      l_lane[g] += qh == 0 ? p[g] : 0.0f;
    }

    uint32_t* const sp = s_p[w];
    if constexpr (MPV) {
      // p through LDS head-major, [g][token] in the storage type (P^T of PV)
      uint16_t* const sp16 = (uint16_t*)sp;
      if (qh == 0) {
#pragma unroll
        for (int g = 0; g < G; ++g) sp16[g * PP + tq] = p_bits<DT>(p[g]);
      }
    } else {
      // p to the load layout through LDS
      uint32_t pk[8];
#pragma unroll
      for (int g = 0; g < 8; ++g) pk[g] = g < G ? pack_p<DT>(p[g], upper_half_value<D>(p[g])) : 0u;
      if (lane < S::HALF) {
        *(uint4*)(sp + tq * 8) = make_uint4(pk[0], pk[1], pk[2], pk[3]);
        *(uint4*)(sp + tq * 8 + 4) = make_uint4(pk[4], pk[5], pk[6], pk[7]);
      }
    }
    wave_lds_sync();
  };

  // ---- o += p * V of the tile at t0, V in its load layout ----
  auto tile_pv = [&](int t0, int buf, uint4(&vr)[S::LOADS]) __attribute__((always_inline)) {
    if constexpr (APPEND) {
      if (owns && pos >= t0 && pos < t0 + S::TILE) {  // the new token's V
        const int t = pos - t0;
#pragma unroll
        for (int r = 0; r < S::LOADS; ++r)
          if (r == t / S::TPL && pv_tok == t % S::TPL) vr[r] = *(const uint4*)(s_vnew[qi] + pv_ch * 8);
      }
    }
    // tokens past the split: V must contribute exactly zero (p is 0 there,
    // and 0 * stale data must not produce NaN)
    const bool partial = t0 + S::TILE > s_end;
    if constexpr (MPV) {
      // V into the tile's K buffer (free: the scores have read it), at
      // vslot.  Load r holds token r * TPL + pv_tok, dims 8 pv_ch .. + 7, so
      // the lane's 16 bytes go to a per-lane base (one per parity of r) plus
      // 1 KB per load pair (lds_write_tile).  Tokens past the split (only in
      // a split's last tile: a wave-uniform branch) are zeroed first.
      const uint32_t vbase = lds_addr(s_k[w][buf]);
      if (partial) {
#pragma unroll
        for (int r = 0; r < S::LOADS; ++r)
          if (t0 + r * S::TPL + pv_tok >= s_end) vr[r] = make_uint4(0, 0, 0, 0);
      }
      uint32_t vlane[2];
#pragma unroll
      for (int par = 0; par < 2; ++par)
        vlane[par] = vbase + vslot<D>(par * S::TPL + pv_tok, 8 * pv_ch);
      lds_write_tile(vlane[0], vlane[1], vr);
      // O^T += V^T P^T per 16-token step c: A = V^T by transposing reads
      // (lane: dim 32 db + lane % 32, tokens 16c + 4(lane / 32) + 0..3 and
      // + 8 + ...), B = P^T (lane: head lane % 32, the same tokens).  Every
      // operand of the tile is read before one wait (the V writes above
      // complete first: LDS accesses of a wave are performed in order).
      constexpr int NC = S::TILE / 16;
      static_assert(NC * ND == 8, "eight (step, dim block) operands per tile");
      const int hh = lane & 31, gs = lane >> 5;
      const uint32_t pt = lds_addr((const uint16_t*)s_p[w] + min(hh, G - 1) * PP + 4 * gs);
      const int tr = 4 * gs + ((lane & 15) >> 2);
      const int tr_d = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
      uint32_t vtr[ND];
#pragma unroll
      for (int db = 0; db < ND; ++db)
        vtr[db] = vbase + vslot<D>(tr, 32 * db + tr_d);
      uint2 va0[8], va1[8], pa[NC], pb[NC];
      const auto issue_step = [&](auto cc) __attribute__((always_inline)) {
        constexpr int c = decltype(cc)::value;
        pa[c] = lds_read8_issue<32 * c>(pt);
        pb[c] = lds_read8_issue<32 * c + 16>(pt);
#pragma unroll
        for (int db = 0; db < ND; ++db) {
          va0[c * ND + db] = lds_tr_issue<16 * c * S::ROWB>(vtr[db]);
          va1[c * ND + db] = lds_tr_issue<16 * c * S::ROWB + 8 * S::ROWB>(vtr[db]);
        }
      };
      issue_step(std::integral_constant<int, 0>{});
      issue_step(std::integral_constant<int, 1>{});
      if constexpr (NC == 4) {
        issue_step(std::integral_constant<int, 2>{});
        issue_step(std::integral_constant<int, 3>{});
      }
      lds_wait_pin(va0);
      lds_pin(va1);
      uint2 pab[8];
#pragma unroll
      for (int c = 0; c < 8; ++c) pab[c] = make_uint2(0u, 0u);
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        pab[c] = pa[c];
        pab[NC + c] = pb[c];
      }
      lds_pin(pab);
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const uint4 pv = hh < G ? make_uint4(pab[c].x, pab[c].y, pab[NC + c].x, pab[NC + c].y)
                                : make_uint4(0, 0, 0, 0);
#pragma unroll
        for (int db = 0; db < ND; ++db) {
          const int i = c * ND + db;
          oacc[db] = mfma32<DT>(make_uint4(va0[i].x, va0[i].y, va1[i].x, va1[i].y), pv, oacc[db]);
        }
      }
    } else {
    const uint32_t* const sp = s_p[w];
#pragma unroll
    for (int r = 0; r < S::LOADS / 2; ++r) {
      const int t = r * S::TPL + pv_tok;  // vr[r]: token t; vr[r + LOADS/2]: t + HALF
      uint4 va = vr[r], vb = vr[r + S::LOADS / 2];
      if (partial) {
        if (t0 + t >= s_end) va = make_uint4(0, 0, 0, 0);
        if (t0 + t + S::HALF >= s_end) vb = make_uint4(0, 0, 0, 0);
      }
      const uint4 p0 = *(const uint4*)(sp + t * 8);
      const uint4 p1 = *(const uint4*)(sp + t * 8 + 4);
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
        for (int e = 0; e < 8; ++e) o[g][e] = St<DT>::dot2(pr[e], pp[g], o[g][e]);
    }
    }
    wave_lds_sync();
  };

  if constexpr (NB == 1) {
    // at most one tile per wave (the split is W tiles)
    if constexpr (FASTA) {
      // The workgroup's operands are roped by all its waves.  Each wave waits
      // for its share of the operand block (behind it only its own K and V,
      // when it has a tile) and a barrier hands the block to every wave;
      // thread t then ropes the dword pairs t,
      // t + 64W, ... (bias + RoPE of q (G heads) and k of the new token: dims
      // j, j + 1 and j + D/2, j + D/2 + 1), the last D/2 threads also
      // v + v_bias, and a second barrier hands the results to every wave.
      // Every wave, with or without a tile, meets both barriers.
      if (ntw > 0) LUC_WAIT_VM(16);  // its operand loads (its K and V may be in flight)
      else LUC_WAIT_VM(0);           // (no tile: only operand loads were issued)
      __builtin_amdgcn_s_barrier();
      {
        const uint32_t pa = lds_addr(s_pa[0]);
        constexpr int NP2 = (G + 1) * HD / 2;
        constexpr int NT = 64 * W;
        const bool hqb = A.q_bias != nullptr, hkb = A.k_bias != nullptr, hvb = A.v_bias != nullptr;
#pragma unroll
        for (int i = 0; i < (NP2 + NT - 1) / NT; ++i) {
          const int idx = (int)threadIdx.x + NT * i;
          if (idx < NP2) {
            const int g = idx / (HD / 2), j = (idx % (HD / 2)) * 2;
            const uint32_t xb = pa + (g < G ? PA_XQ + g * D * 2 : PA_K);
            const uint32_t bb = pa + (g < G ? PA_BQ + g * D * 2 : PA_KB);
            uint32_t x1, x2, b1, b2;
            uint2 c, sn;
            lds_read_rope(xb + j * 2, xb + (j + HD) * 2, bb + j * 2, bb + (j + HD) * 2,
                          pa + PA_C + j * 4, pa + PA_S + j * 4, x1, x2, b1, b2, c, sn);
            if (!(g < G ? hqb : hkb)) b1 = b2 = 0u;
            uint16_t o1a, o2a, o1b, o2b;
            rot_pair<DT>(x1 & 0xffff, b1 & 0xffff, x2 & 0xffff, b2 & 0xffff, __uint_as_float(c.x),
                         __uint_as_float(sn.x), o1a, o2a);
            rot_pair<DT>(x1 >> 16, b1 >> 16, x2 >> 16, b2 >> 16, __uint_as_float(c.y),
                         __uint_as_float(sn.y), o1b, o2b);
            const uint32_t lo = (uint32_t)o1a | ((uint32_t)o1b << 16);
            const uint32_t hi = (uint32_t)o2a | ((uint32_t)o2b << 16);
            if (g < G) {  // (two stores with known targets: no alias with the loads into LDS)
              *(uint32_t*)(s_q[qi] + g * QP + j) = lo;
              *(uint32_t*)(s_q[qi] + g * QP + j + HD) = hi;
            } else {
              *(uint32_t*)(s_knew[qi] + j) = lo;
              *(uint32_t*)(s_knew[qi] + j + HD) = hi;
            }
          }
        }
        const int vt = (int)threadIdx.x - (NT - D / 2);  // v word of the last D/2 threads
        if (vt >= 0) {
          uint32_t vv, vbv;
          lds_read2(pa + PA_V + vt * 4, pa + PA_VB + vt * 4, vv, vbv);
          if (!hvb) vbv = 0u;
          const uint16_t lo = St<DT>::store(St<DT>::load(vv & 0xffff) + St<DT>::load(vbv & 0xffff));
          const uint16_t hi = St<DT>::store(St<DT>::load(vv >> 16) + St<DT>::load(vbv >> 16));
          *(uint32_t*)(s_vnew[qi] + 2 * vt) = (uint32_t)lo | ((uint32_t)hi << 16);
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // this thread's LDS writes are done
      }
      __builtin_amdgcn_s_barrier();
    }
    if (ntw > 0) {
      LUC_WAIT_VM(8);  // K and q
      // the A operands from a q row in LDS (asm reads: compiler-visible
      // reads of LDS would wait for every outstanding load)
      auto q_operands_lds = [&](const void* row) __attribute__((always_inline)) {
        const uint32_t qa = lds_addr(row) + (uint32_t)((min(lane & 31, G - 1) * QP + 8 * (lane >> 5)) * 2);
#pragma unroll
        for (int k4 = 0; k4 < KS; k4 += 4) {
          uint4 x[4];
          lds_read4(qa + k4 * 32, qa + (k4 + 1) * 32, qa + (k4 + 2) * 32, qa + (k4 + 3) * 32, x);
#pragma unroll
          for (int i = 0; i < 4; ++i) qm[k4 + i] = (lane & 31) < G ? x[i] : make_uint4(0, 0, 0, 0);
        }
      };
      if constexpr (FASTQ) q_operands_lds(s_qr[w]);
      if constexpr (FASTA) q_operands_lds(s_q[0]);  // the shared roped copy
      tile_scores(t_first, 0);
      LUC_WAIT_VM(0);  // V
      tile_pv(t_first, 0, vr0);
    }
  } else {
    // The wave's tiles in pairs: both tiles of a pair are issued
    // (unconditionally, so that the loads keep their place ahead of the
    // waits below), tile i is computed while tile i+1 lands.  PREK (the
    // non-step kernels with PV on the matrix cores): a K buffer takes the same tile of the next pair as
    // soon as its tile's PV is done, so the next pair's K loads are in flight
    // while this pair is finished; its V loads (into registers, which hold
    // one pair) go out when the pair starts.  In flight, in issue order (8
    // loads each): K_a K_b (issued during the previous pair, or before the
    // prologue), V_a V_b, then K_a' after tile a's PV and K_b' after tile
    // b's.  The other kernels, which have no registers to spare for it, issue
    // a whole pair when it starts: K_a V_a K_b V_b.  The first pair's V
    // registers come from the prologue, later pairs' are local to their
    // iteration (no values carried around the loop).
    constexpr bool PREK = !APPEND && MPV;
    auto pair_body = [&](int i, uint4(&va)[S::LOADS], uint4(&vb)[S::LOADS]) __attribute__((always_inline)) {
      const int t0 = t_first + i * WS;
      const bool pair = i + 1 < ntw, next = i + 2 < ntw;  // (wave-uniform)
      LUC_WAIT_VM(24);  // K_a
      tile_scores(t0, 0);
      if constexpr (PREK) LUC_WAIT_VM(8);  // V_a (and K_b)
      else LUC_WAIT_VM(16);                // V_a
      tile_pv(t0, 0, va);
      if (PREK && next) issue_k(t0 + 2 * WS, 0);
      if (pair) {
        if constexpr (!PREK) LUC_WAIT_VM(8);  // K_b
        tile_scores(t0 + WS, 1);
        if (PREK && next) LUC_WAIT_VM(8);  // V_b (K_a' behind it)
        else LUC_WAIT_VM(0);
        tile_pv(t0 + WS, 1, vb);
      }
      if (PREK && next) issue_k(t0 + 3 * WS, 1);
    };
    if (ntw > 0) {
      pair_body(0, vr0, vr1);
      for (int i = 2; i < ntw; i += 2) {
        uint4 va[S::LOADS], vb[S::LOADS];
        if constexpr (PREK) {
          issue_v(t_first + i * WS, va);
          issue_v(t_first + (i + 1) * WS, vb);
        } else {
          issue(t_first + i * WS, 0, va);
          issue(t_first + (i + 1) * WS, 1, vb);
        }
        pair_body(i, va, vb);
      }
      // (the unused second tile of an odd last pair lands before its
      // buffers are reused)
      LUC_WAIT_VM(0);
    }
  }

  if constexpr (APPEND) {
    // the cache write of the new token (none through a page outside the pool)
    int new_page;
    if constexpr (T1) new_page = new_raw;
    else new_page = page_raw((pos - s_begin) / kPage);
    if (owns && lane < S::CH && new_page >= 0 && new_page < nb) {
      const int64_t slot = (int64_t)new_page * page_stride + head_off + (int64_t)(pos % kPage) * D + lane * 8;
      *(uint4*)(A.k_pool + slot) = *(const uint4*)(s_knew[qi] + lane * 8);
      *(uint4*)(A.v_pool + slot) = *(const uint4*)(s_vnew[qi] + lane * 8);
    }
  }
  if (bad_page) {  // a page of this wave's tiles lies outside the pool
#pragma unroll
    for (int g = 0; g < G; ++g) l_lane[g] = __builtin_nanf("");
  }

  finish_split<DT, D, G, APPEND, W, MPV>(A, o, oacc, m_run, l_lane, (float*)s_k[0][0], NB * S::KBYTES / 4,
                                    &s_p[0][0], s_q[0], s_knew[0], split, bh, b, h, nsplit, out_row);
}

}  // namespace luc

// Decode kernels: _t1 has 8 waves per workgroup, one tile each (splits of 8
// tiles; 80 KB of LDS, two workgroups per CU, so four waves per SIMD, which
// the register target keeps up to group size 7 at head_dim 64 and 6 at 128);
// _t2 has 4 waves with two tiles in flight each (longer splits, two
// workgroups per CU); _t2w8 the same with 8 waves (one workgroup per CU,
// about 150 KB of LDS), which the host picks when the launch is a single
// round of such workgroups: half the splits, so half the partials to merge.
// Resident-wave targets are per SIMD.
#define LUC_DECODE_KERNELS(DTN, DT, D, G, NB, OCC, W, SUF)                                          \
  extern "C" __global__ __launch_bounds__(64 * W) __attribute__((amdgpu_waves_per_eu(OCC)))         \
  void luc_decode_##DTN##_d##D##_g##G##_t##NB##SUF(luc::DecodeArgs a) {                             \
    luc::decode_impl<DT, D, G, false, W, NB>(a);                                                    \
  }                                                                                                 \
  extern "C" __global__ __launch_bounds__(64 * W) __attribute__((amdgpu_waves_per_eu(OCC)))         \
  void luc_decode_step_##DTN##_d##D##_g##G##_t##NB##SUF(luc::DecodeArgs a) {                        \
    luc::decode_impl<DT, D, G, true, W, NB>(a);                                                     \
  }

// This file builds two code objects: paged_decode.hsaco (the _t1 and _t2
// kernels) and, with LUC_DECODE_WIDE defined, paged_decode_w8.hsaco (the
// _t2w8 kernels), compiled in parallel.
#ifndef LUC_DECODE_WIDE
#define LUC_DECODE(DTN, DT, D, G)                                                                  \
  LUC_DECODE_KERNELS(DTN, DT, D, G, 1, ((D == 64 ? G <= 7 : G <= 6) ? 4 : 2), 8, )                 \
  LUC_DECODE_KERNELS(DTN, DT, D, G, 2, 2, 4, )
#else
#define LUC_DECODE(DTN, DT, D, G) LUC_DECODE_KERNELS(DTN, DT, D, G, 2, 2, 8, w8)
#endif

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
