// Shared device helpers for the gfx950 paged-attention kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace luc {

enum : int { kBF16 = 0, kF16 = 1 };
constexpr int kPage = 16;  // tokens per KV page (block_size)

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf162_t __attribute__((ext_vector_type(2)));

// 16-bit storage <-> f32.  Rounding is round-to-nearest-even in both formats.
template <int DT> struct St;

template <> struct St<kBF16> {
  __device__ static inline float load(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }
  // low / high half of a packed pair
  __device__ static inline float lo(uint32_t w) { return __uint_as_float(w << 16); }
  __device__ static inline float hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
  // round to nearest even; a NaN keeps its sign and top payload bits, quieted
  // (branch-free: a select, not a divergent branch)
  __device__ static inline uint16_t store(float f) {
    const uint32_t u = __float_as_uint(f);
    const uint32_t rounded = (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
    const uint32_t quiet = (u >> 16) | 0x0040u;
    return (uint16_t)((u & 0x7fffffffu) > 0x7f800000u ? quiet : rounded);
  }
  // f32 dot of two packed pairs, accumulated into c
  __device__ static inline float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf162_t, a),
                                           __builtin_bit_cast(bf162_t, b), c, false);
  }
};

template <> struct St<kF16> {
  __device__ static inline float load(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
  __device__ static inline float lo(uint32_t w) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(w & 0xffffu));
  }
  __device__ static inline float hi(uint32_t w) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(w >> 16));
  }
  // round to nearest even (v_cvt_f16_f32, denormals kept); a NaN keeps its
  // sign and top 10 payload bits, quieted (a select, not a branch)
  __device__ static inline uint16_t store(float f) {
    const uint32_t u = __float_as_uint(f);
    const uint32_t quiet = ((u >> 16) & 0x8000u) | 0x7e00u | ((u >> 13) & 0x3ffu);
    const uint16_t h = __builtin_bit_cast(uint16_t, (_Float16)f);
    return (u & 0x7fffffffu) > 0x7f800000u ? (uint16_t)quiet : h;
  }
  __device__ static inline float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, a), __builtin_bit_cast(half2_t, b), c,
                                  false);
  }
};

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

// Two ds_read_b64_tr_b16: within each 16-lane group, output lane 4a + c
// receives element c of the 8-byte chunks read by input lanes 4e + a,
// e = 0..3.
template <int OFF0, int OFF1>
__device__ inline void lds_tr16x2(uint32_t a, uint2* x) {
  asm volatile(
      "ds_read_b64_tr_b16 %0, %2 offset:%3\n\t"
      "ds_read_b64_tr_b16 %1, %2 offset:%4\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(x[0]), "=&v"(x[1])
      : "v"(a), "n"(OFF0), "n"(OFF1)
      : "memory");
}

// v_mfma_f32_32x32x16_{f16,bf16}: c += a * b, eight 16-bit values per lane
// in a and b.  Operand layouts: A lane l = row l % 32, k (l / 32) * 8 .. + 8;
// B lane l = column l % 32, the same k; C lane l = column l % 32, c[4i + j] =
// row 8i + 4(l / 32) + j.
template <int DT>
__device__ inline f32x16 mfma32(uint4 a, uint4 b, f32x16 c) {
  if constexpr (DT == kF16)
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

// 16-byte global load with the non-temporal (streaming) hint.
__device__ inline uint4 ld_nt16(const uint16_t* p) {
  const u32x4_t x = __builtin_nontemporal_load((const u32x4_t*)p);
  return make_uint4(x.x, x.y, x.z, x.w);
}

// ---- wave64 reductions -------------------------------------------------
// DPP controls (GFX9 encoding).
constexpr int kDppQuadXor1 = 0xB1;   // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;   // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141;
constexpr int kDppMirror = 0x140;

template <int CTRL>
__device__ inline float dpp_mov(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}

// Max over the 16 lanes of each DPP row; every lane of the row gets it.
__device__ inline float row_max16(float x) {
  x = fmaxf(x, dpp_mov<kDppQuadXor1>(x));
  x = fmaxf(x, dpp_mov<kDppQuadXor2>(x));
  x = fmaxf(x, dpp_mov<kDppHalfMirror>(x));
  x = fmaxf(x, dpp_mov<kDppMirror>(x));
  return x;
}
__device__ inline float row_sum16(float x) {
  x += dpp_mov<kDppQuadXor1>(x);
  x += dpp_mov<kDppQuadXor2>(x);
  x += dpp_mov<kDppHalfMirror>(x);
  x += dpp_mov<kDppMirror>(x);
  return x;
}
__device__ inline float readlane(float x, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), lane));
}
// Wave-uniform max / sum over all 64 lanes.  A chain of DPP-fused VALU ops
// (quad swaps, row half-mirror, row mirror, then the row broadcasts of lanes
// 15 and 31 into the following rows) leaves the result in lane 63.  Each DPP
// read of a register written by the previous VALU op needs two wait states
// (s_nop 1); the trailing s_nop covers the readlane of the result.
#define LUC_DPP_REDUCE(OP)                                                                   \
  "s_nop 1\n\t" OP " %0, %1, %1 quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf\n\t"          \
  "s_nop 1\n\t" OP " %0, %0, %0 quad_perm:[2,3,0,1] row_mask:0xf bank_mask:0xf\n\t"          \
  "s_nop 1\n\t" OP " %0, %0, %0 row_half_mirror row_mask:0xf bank_mask:0xf\n\t"              \
  "s_nop 1\n\t" OP " %0, %0, %0 row_mirror row_mask:0xf bank_mask:0xf\n\t"                   \
  "s_nop 1\n\t" OP " %0, %0, %0 row_bcast:15 row_mask:0xa bank_mask:0xf\n\t"                 \
  "s_nop 1\n\t" OP " %0, %0, %0 row_bcast:31 row_mask:0xc bank_mask:0xf\n\t"                 \
  "s_nop 1"
__device__ inline float wave_max(float x) {
  float r;
  asm volatile(LUC_DPP_REDUCE("v_max_f32_dpp") : "=&v"(r) : "v"(x));
  return readlane(r, 63);
}
__device__ inline float wave_sum(float x) {
  float r;
  asm volatile(LUC_DPP_REDUCE("v_add_f32_dpp") : "=&v"(r) : "v"(x));
  return readlane(r, 63);
}

// Wave sums of H <= 4 independent values at once: the same DPP chain, issued
// step-major so that between the write of a value and the next DPP read of it
// lie H-1 other instructions; for H < 3 an s_nop pads the two wait states.
// One such block costs about one chain's latency instead of H of them.
#define LUC_RS1(CTRL) "v_add_f32_dpp %[r0], %[r0], %[r0] " CTRL "\n\t"
#define LUC_RS2(CTRL) LUC_RS1(CTRL) "v_add_f32_dpp %[r1], %[r1], %[r1] " CTRL "\n\t"
#define LUC_RS3(CTRL) LUC_RS2(CTRL) "v_add_f32_dpp %[r2], %[r2], %[r2] " CTRL "\n\t"
#define LUC_RS4(CTRL) LUC_RS3(CTRL) "v_add_f32_dpp %[r3], %[r3], %[r3] " CTRL "\n\t"
#define LUC_RSUM(H, PAD)                                                                     \
  "s_nop 1\n\t" LUC_RS##H("quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf") PAD              \
      LUC_RS##H("quad_perm:[2,3,0,1] row_mask:0xf bank_mask:0xf") PAD                        \
      LUC_RS##H("row_half_mirror row_mask:0xf bank_mask:0xf") PAD                            \
      LUC_RS##H("row_mirror row_mask:0xf bank_mask:0xf") PAD                                 \
      LUC_RS##H("row_bcast:15 row_mask:0xa bank_mask:0xf") PAD                               \
      LUC_RS##H("row_bcast:31 row_mask:0xc bank_mask:0xf") "s_nop 1"
template <int H>
__device__ __attribute__((always_inline)) inline void wave_sum_group(float* x) {
  static_assert(H >= 1 && H <= 4, "1 to 4 values per block");
  if constexpr (H == 1) {
    asm volatile(LUC_RSUM(1, "s_nop 1\n\t") : [r0] "+v"(x[0]));
  } else if constexpr (H == 2) {
    asm volatile(LUC_RSUM(2, "s_nop 0\n\t") : [r0] "+v"(x[0]), [r1] "+v"(x[1]));
  } else if constexpr (H == 3) {
    asm volatile(LUC_RSUM(3, "") : [r0] "+v"(x[0]), [r1] "+v"(x[1]), [r2] "+v"(x[2]));
  } else {
    asm volatile(LUC_RSUM(4, "")
                 : [r0] "+v"(x[0]), [r1] "+v"(x[1]), [r2] "+v"(x[2]), [r3] "+v"(x[3]));
  }
#pragma unroll
  for (int i = 0; i < H; ++i) x[i] = readlane(x[i], 63);
}
// x[i] = wave-uniform sum of x[i] over all 64 lanes, for i < N (N <= 8).
template <int N>
__device__ __attribute__((always_inline)) inline void wave_sum_n(float (&x)[N]) {
  static_assert(N >= 1 && N <= 8, "at most 8 values");
  constexpr int H1 = N <= 4 ? N : (N + 1) / 2;
  wave_sum_group<H1>(x);
  if constexpr (N > H1) wave_sum_group<N - H1>(x + H1);
}

// Orders this wave's LDS accesses at this point (DS operations of one wave
// complete in issue order, so a code-motion barrier is all that is needed).
__device__ inline void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// 16-bit element e (0..7) of a 16-byte chunk, and eight elements packed.
__device__ inline uint16_t chunk_elem(const uint4& v, int e) {
  const uint32_t w = e < 2 ? v.x : e < 4 ? v.y : e < 6 ? v.z : v.w;
  return (uint16_t)(e & 1 ? w >> 16 : w & 0xffffu);
}
__device__ inline uint4 chunk_pack(const uint16_t* e) {
  return make_uint4(e[0] | (uint32_t)e[1] << 16, e[2] | (uint32_t)e[3] << 16,
                    e[4] | (uint32_t)e[5] << 16, e[6] | (uint32_t)e[7] << 16);
}

// RoPE of eight element pairs: x1 holds dims i..i+7 of a head, x2 dims
// i+D/2..i+D/2+7, c and s the cos/sin of dims i..i+7 at the row's position
// (c0|c1, s0|s1), b1/b2 the bias chunks (used when has_bias).  Each sum,
// product and the final difference/sum rounds separately in f32 (contraction
// off), then to storage -- the same bits wherever it runs
// (src/kernels/rope.cu:31-52).
template <int DT>
__device__ inline void rope_rotate8(uint4& x1, uint4& x2, const uint4& b1, const uint4& b2,
                                    bool has_bias, const float4& c0, const float4& c1,
                                    const float4& s0, const float4& s1) {
#pragma clang fp contract(off)
  const float cs[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
  const float sn[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
  float r1[8], r2[8];
  bool nan = false;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float bb1 = has_bias ? St<DT>::load(chunk_elem(b1, e)) : 0.0f;
    const float bb2 = has_bias ? St<DT>::load(chunk_elem(b2, e)) : 0.0f;
    const float v1 = St<DT>::load(chunk_elem(x1, e)) + bb1;
    const float v2 = St<DT>::load(chunk_elem(x2, e)) + bb2;
    const float p = v1 * cs[e];
    const float r = v2 * sn[e];
    const float m = v1 * sn[e];
    const float n = v2 * cs[e];
    r1[e] = p - r;
    r2[e] = m + n;
    nan |= __builtin_isnan(r1[e]) | __builtin_isnan(r2[e]);
  }
  if (DT == kBF16 && !nan) {
    // v_cvt_pk_bf16_f32: round to nearest even, f32 denormals kept (the
    // kernels run with denormals enabled) -- the bits of St<kBF16>::store
    // for every non-NaN value
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    uint32_t w1[4], w2[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const bf16x2 a = {(__bf16)r1[2 * e], (__bf16)r1[2 * e + 1]};
      const bf16x2 b = {(__bf16)r2[2 * e], (__bf16)r2[2 * e + 1]};
      w1[e] = __builtin_bit_cast(uint32_t, a);
      w2[e] = __builtin_bit_cast(uint32_t, b);
    }
    x1 = make_uint4(w1[0], w1[1], w1[2], w1[3]);
    x2 = make_uint4(w2[0], w2[1], w2[2], w2[3]);
  } else {
    uint16_t o1[8], o2[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      o1[e] = St<DT>::store(r1[e]);
      o2[e] = St<DT>::store(r2[e]);
    }
    x1 = chunk_pack(o1);
    x2 = chunk_pack(o2);
  }
}

// Online softmax: p = exp2(s - m) is kept <= 2^kLazyMax (exact in f16 range)
// by moving the reference point m only when a score passes m + kLazyMax.
constexpr float kLazyMax = 8.0f;

}  // namespace luc
