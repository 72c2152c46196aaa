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
  __device__ static inline uint16_t store(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
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
  __device__ static inline uint16_t store(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }
  __device__ static inline float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, a), __builtin_bit_cast(half2_t, b), c,
                                  false);
  }
};

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

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

// Online softmax: p = exp2(s - m) is kept <= 2^kLazyMax (exact in f16 range)
// by moving the reference point m only when a score passes m + kLazyMax.
constexpr float kLazyMax = 8.0f;

}  // namespace luc
