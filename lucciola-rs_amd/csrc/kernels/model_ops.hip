// The Qwen2 model loop's kernels for gfx950: embedding gather, RMSNorm,
// fused SiLU * up, greedy argmax -- the reference's batched_embedding_kernel
// (src/kernels/embedding.cu), rmsnorm_nvidia (src/kernels/rmsnorm.cu),
// silu_and_mul_fused_kernel (src/kernels/activation.cu) and argmax_kernel
// (src/kernels/sampling.cu) -- and the one-row products of a decode step
// (GEMV, optionally with the RMSNorm of their input and the SiLU * up of their
// output fused in).  bf16 storage, f32 arithmetic.
//
// Fixed arithmetic order, so that a CPU restatement can produce the same bits:
//   RMSNorm: thread t of 256 sums x*x over its 16-byte chunks c = t, t + 256,
//   ... (elements in order, one fma each); the 256 partials add as a halving
//   tree (a[i] += a[i + s] for s = 128, 64, ..., 1); inv = 1 / sqrt(sum / n +
//   eps) with IEEE division and square root; y = round((x * inv) * w).  The
//   formula is rmsnorm.cu's (:40, :63-64); its summation order is not: the
//   reference adds per-thread x*x + y*y pairs (:19-29) with a 1024-thread CUB
//   block reduction (:32-35) and takes rsqrtf (:40).
//   argmax: the largest value wins; among equal values the one with the
//   smallest i mod 1024, then the smallest i -- the order of the reference's
//   1024-thread kernel (sampling.cu:16-46): each thread keeps the first of its
//   equal values (i = tid, tid + 1024, ...) and the block reduction keeps the
//   lower thread's pair on ties (ArgMaxOp returns a unless b is larger).
#include "luc_common.h"

namespace luc {

constexpr int kNormThreads = 256;

// RMSNorm of `rows` rows of n elements (n a multiple of 8, 16-byte aligned
// rows): out may alias in.  Rows of up to kNormChunks * 8 * kNormThreads
// elements stay in registers between the sum and the output (x and the
// weight are loaded together); the halving tree's first two levels read the
// partials from LDS in one wave, which adds the rest across its lanes (each
// level the same additions a[i] + a[i + s] as the tree).
constexpr int kNormChunks = 4;
__device__ void rmsnorm_impl(uint16_t* out, const uint16_t* in, const uint16_t* weight, float eps,
                             int n) {
#pragma clang fp contract(off)
  __shared__ float part[kNormThreads];
  const int t = threadIdx.x;
  const int64_t row = blockIdx.x;
  const uint4* x = (const uint4*)(in + row * n);
  const uint4* w = (const uint4*)weight;
  uint4* y = (uint4*)(out + row * n);
  const int chunks = n / 8;
  const bool in_regs = chunks <= kNormChunks * kNormThreads;
  uint4 xv[kNormChunks], wv[kNormChunks];
  float s = 0.0f;
  if (in_regs) {
#pragma unroll
    for (int k = 0; k < kNormChunks; ++k) {
      const int c = t + k * kNormThreads;
      if (c < chunks) {
        xv[k] = x[c];
        wv[k] = w[c];
      }
    }
#pragma unroll
    for (int k = 0; k < kNormChunks; ++k)
      if (t + k * kNormThreads < chunks)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float f = St<kBF16>::load(chunk_elem(xv[k], e));
          s = fmaf(f, f, s);
        }
  } else {
    for (int c = t; c < chunks; c += kNormThreads) {
      const uint4 v = x[c];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float f = St<kBF16>::load(chunk_elem(v, e));
        s = fmaf(f, f, s);
      }
    }
  }
  part[t] = s;
  __syncthreads();
  static_assert(kNormThreads == 256, "levels 128 and 64 below, then the 64 lanes of one wave");
  if (t < 64) {
    float a = (part[t] + part[t + 128]) + (part[t + 64] + part[t + 192]);
#pragma unroll
    for (int h = 32; h > 0; h >>= 1) a = a + __shfl_down(a, h);
    if (t == 0) part[0] = a;
  }
  __syncthreads();
  const float inv = 1.0f / sqrtf(part[0] / (float)n + eps);
  auto norm_chunk = [&](uint4 v, uint4 wc) {
    uint16_t o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float f = St<kBF16>::load(chunk_elem(v, e)) * inv;
      o[e] = St<kBF16>::store(f * St<kBF16>::load(chunk_elem(wc, e)));
    }
    return chunk_pack(o);
  };
  if (in_regs) {
#pragma unroll
    for (int k = 0; k < kNormChunks; ++k) {
      const int c = t + k * kNormThreads;
      if (c < chunks) y[c] = norm_chunk(xv[k], wv[k]);
    }
  } else {
    for (int c = t; c < chunks; c += kNormThreads) y[c] = norm_chunk(x[c], w[c]);
  }
}

// gate <- round(silu(gate) * up) in place, rows of [gate (inter) | up (inter)],
// silu(g) = g / (1 + exp(-g)) in f32; eight elements per thread.
__device__ void silu_mul_impl(uint16_t* buf, int rows, int inter) {
#pragma clang fp contract(off)
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // chunk of 8 gates
  const int per_row = inter / 8;
  if (i >= (int64_t)rows * per_row) return;
  const int64_t r = i / per_row;
  const int c = (int)(i - r * per_row);
  uint4* g = (uint4*)(buf + r * 2 * inter) + c;
  const uint4 gv = *g, uv = *(const uint4*)(buf + r * 2 * inter + inter + c * 8);
  uint16_t o[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float x = St<kBF16>::load(chunk_elem(gv, e));
    const float s = x / (1.0f + expf(-x));
    o[e] = St<kBF16>::store(s * St<kBF16>::load(chunk_elem(uv, e)));
  }
  *g = chunk_pack(o);
}

// out[t] = table[ids[t]] (rows of `hidden`, a multiple of 8); an id at or past
// `vocab` gives a NaN row instead of a read outside the table.
__device__ void embedding_impl(uint16_t* out, const uint16_t* table, const uint32_t* ids, int vocab,
                               int hidden) {
  const int64_t t = blockIdx.x;
  const uint32_t id = ids[t];
  uint4* dst = (uint4*)(out + t * hidden);
  const int chunks = hidden / 8;
  if (id >= (uint32_t)vocab) {
    const uint32_t nan2 = 0x7fc07fc0u;
    for (int c = threadIdx.x; c < chunks; c += blockDim.x) dst[c] = make_uint4(nan2, nan2, nan2, nan2);
    return;
  }
  const uint4* src = (const uint4*)(table + (int64_t)id * hidden);
  for (int c = threadIdx.x; c < chunks; c += blockDim.x) dst[c] = src[c];
}

constexpr int kArgmaxThreads = 1024;

// Index of the largest of n values (values <= -1e30 and NaN never win, as in
// the reference, which then reports index -1, i.e. 0xffffffff).
__device__ void argmax_impl(const uint16_t* x, int n, uint32_t* out) {
  __shared__ float sv[kArgmaxThreads];
  __shared__ int si[kArgmaxThreads];
  const int t = threadIdx.x;
  float best = -1e30f;
  int idx = -1;
  // increasing i: the first of equals stays.  Sixteen of the thread's loads
  // go out before any comparison, so the scan waits on memory once per
  // sixteen elements instead of once per element.
  constexpr int U = 16;
  int i = t;
  for (; i + (U - 1) * kArgmaxThreads < n; i += U * kArgmaxThreads) {
    float v[U];
#pragma unroll
    for (int k = 0; k < U; ++k) v[k] = St<kBF16>::load(x[i + k * kArgmaxThreads]);
#pragma unroll
    for (int k = 0; k < U; ++k)
      if (v[k] > best) {
        best = v[k];
        idx = i + k * kArgmaxThreads;
      }
  }
  for (; i < n; i += kArgmaxThreads) {
    const float v = St<kBF16>::load(x[i]);
    if (v > best) {
      best = v;
      idx = i;
    }
  }
  sv[t] = best;
  si[t] = idx;
  __syncthreads();
  for (int h = kArgmaxThreads / 2; h > 0; h >>= 1) {
    if (t < h) {
      const float bv = sv[t + h];
      const int bi = si[t + h];
      // larger value, or an equal one from a lower thread (i mod 1024; -1 = none)
      if (bv > sv[t] || (bv == sv[t] && bi >= 0 &&
                         (si[t] < 0 || (bi % kArgmaxThreads) < (si[t] % kArgmaxThreads)))) {
        sv[t] = bv;
        si[t] = bi;
      }
    }
    __syncthreads();
  }
  if (t == 0) out[0] = (uint32_t)si[0];
}

// y[n] = round(sum_k x[k] w[n][k] + res[n]) for one row x of K elements
// and the N rows of w (row-major [N][K], as the reference's linear weights):
// the M = 1 case of Qwen2Model::matmul_bf16 (src/models.rs:252-295), f32
// accumulation; with res the residual the add is its beta = 1 (one rounding).
// PRE: x is `in` (kGemvPlain), or RMSNorm(in) with weight nw (kGemvNorm),
// formed in registers by each wave with the bits luc_rmsnorm_bf16 writes:
// rmsnorm_impl's sum order replayed in one wave -- lane l holds the chunks
// l + 64 j, i.e. chunk l + 64 j + 256 m of rmsnorm_impl's thread l + 64 j,
// the chunks a thread adds in increasing order.
// POST kGemvSiluPair: w holds 2 N rows [gate rows (N) | up rows (N)] and
// y[n] = round(silu(g) * u), g and u the bf16-rounded products of gate row n
// and up row n (no res) -- what luc_silu_mul_bf16 makes of the unfused
// [gate | up] output.  So a fused launch gives the unfused kernels' bits
// (the reference's apply_rmsnorm + matmul_bf16, models.rs:455-482 and
// :568-590, and apply_activation_fused, :671).
// One wave per R rows of w (HBM-bound: every byte of w read once, 16 bytes
// per lane and load, all of a wave's loads in flight together, the rows'
// loads while x is formed).  Lane l takes the 8-element chunks c = l, l + 64,
// ... (C of them at most); a row's products add in chunk
// order per lane, element order within a chunk, then over the lanes: the
// upper 32 lanes onto the lower (permlane32 swap), the odd 16-lane rows onto
// the even (permlane16 swap), then the 16 lanes of a row (quad xor 1, quad
// xor 2, half mirror, mirror) -- a fixed order.  With R = 4 (R = 2) the swaps
// also gather the rows: lanes [64 r / R, 64 (r + 1) / R) end holding the sum
// of the wave's row r; R = 8 is two such groups of four.  res may alias y (a wave reads the residuals of its
// own rows only, before it writes them); in must not.
constexpr int kGemvThreads = 256;
enum GemvPre { kGemvPlain = 0, kGemvNorm = 1 };
enum GemvPost { kGemvStore = 0, kGemvSiluPair = 1 };

// Chunk c = lane + 64 j of a row of nch chunks, zero past the end: an
// unconditional 16-byte load from a clamped address, then an AND with a mask
// the compiler cannot see through (an empty asm) -- otherwise it turns the
// select into a load under an exec-masked branch, and the loads of a wave's
// branches are then all waited for at once (vmcnt(0) where they join).
__device__ inline uint4 row_chunk(const uint16_t* row, int lane, int j, int nch) {
  const int c = lane + 64 * j;
  const uint4 v = *(const uint4*)(row + 8 * min(c, nch - 1));
  uint32_t m = c < nch ? 0xffffffffu : 0u;
  asm volatile("" : "+v"(m));
  return make_uint4(v.x & m, v.y & m, v.z & m, v.w & m);
}

template <int R, int C, int PRE, int POST>
__device__ void gemv_impl(uint16_t* y, const uint16_t* in, const uint16_t* w, const uint16_t* res,
                          const uint16_t* nw, float eps, int n_out, int k) {
#pragma clang fp contract(off)
  static_assert(R == 1 || R == 2 || R == 4 || R == 8, "rows per wave");
  static_assert(POST == kGemvStore || R >= 2, "a silu pair takes two rows");
  static_assert(POST == kGemvStore || R <= 4, "a silu pair takes at most four rows");
  constexpr int NG = R > 4 ? R / 4 : 1;  // groups of (up to) four rows, each reduced alone
  constexpr int RG = R / NG;             // rows per group
  constexpr int kOut = POST == kGemvSiluPair ? R / 2 : R;  // outputs per wave and group
  constexpr int wpg = kGemvThreads / 64;  // waves per workgroup
  const int lane = threadIdx.x & 63;
  const int n0 = (blockIdx.x * wpg + (threadIdx.x >> 6)) * kOut;  // the wave's first output
  if (n0 >= n_out) return;  // wave-uniform
  const int nch = k / 8;
  uint4 xv[C], nv[PRE == kGemvNorm ? C : 1];
#pragma unroll
  for (int j = 0; j < C; ++j) xv[j] = row_chunk(in, lane, j, nch);
  if constexpr (PRE == kGemvNorm) {
#pragma unroll
    for (int j = 0; j < C; ++j) nv[j] = row_chunk(nw, lane, j, nch);
  }
  // the wave's rows (rows past the end re-read the last one), in flight while
  // x is formed: issued after x, so x's wait leaves them out
  uint4 wv[R][C];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int n = POST == kGemvSiluPair ? (r < kOut ? 0 : n_out) + min(n0 + r % kOut, n_out - 1)
                                        : min(n0 + r, n_out - 1);
    const uint16_t* const wr = w + (int64_t)n * k;
#pragma unroll
    for (int j = 0; j < C; ++j) wv[r][j] = row_chunk(wr, lane, j, nch);
  }
  constexpr int kLanesPerRow = 64 / RG;
  // the residual of the lane's row in each group (lane / kLanesPerRow), read
  // now -- before any write of y, and only rows of this wave; unconditionally
  // (from y when there is none: an unused value), so no branch waits for it
  uint16_t rbits[NG] = {};
  if constexpr (POST == kGemvStore)
#pragma unroll
    for (int gi = 0; gi < NG; ++gi)
      rbits[gi] = (res ? res : y)[min(n0 + gi * RG + lane / kLanesPerRow, n_out - 1)];
  __builtin_amdgcn_sched_barrier(0);  // every load above issues before the first wait
  if constexpr (PRE == kGemvNorm) {
    float p[4] = {0.0f, 0.0f, 0.0f, 0.0f};  // rmsnorm_impl's threads lane + 64 i
#pragma unroll
    for (int j = 0; j < C; ++j)
      if (lane + 64 * j < nch)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float f = St<kBF16>::load(chunk_elem(xv[j], e));
          p[j & 3] = fmaf(f, f, p[j & 3]);
        }
    float a = (p[0] + p[2]) + (p[1] + p[3]);
#pragma unroll
    for (int h = 32; h > 0; h >>= 1) a = a + __shfl_down(a, h);
    const float sum = readlane(a, 0);
    const float inv = 1.0f / sqrtf(sum / (float)k + eps);
#pragma unroll
    for (int j = 0; j < C; ++j) {
      uint16_t o[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float f = St<kBF16>::load(chunk_elem(xv[j], e)) * inv;
        o[e] = St<kBF16>::store(f * St<kBF16>::load(chunk_elem(nv[j], e)));
      }
      xv[j] = chunk_pack(o);
    }
  }
  {
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      float a = 0.0f;
#pragma unroll
      for (int j = 0; j < C; ++j)
#pragma unroll
        for (int e = 0; e < 8; ++e)
          a = fmaf(St<kBF16>::load(chunk_elem(xv[j], e)), St<kBF16>::load(chunk_elem(wv[r][j], e)), a);
      acc[r] = a;
    }
#pragma unroll
  for (int gi = 0; gi < NG; ++gi) {
    const float* const ga = acc + gi * RG;  // the group's rows
    // lanes l and l + 32, then 16-lane rows 2i and 2i + 1, then a row's 16 lanes
    float s;
    if constexpr (RG == 4) {
      const auto s02 = __builtin_amdgcn_permlane32_swap(__float_as_uint(ga[0]), __float_as_uint(ga[2]),
                                                        false, false);
      const auto s13 = __builtin_amdgcn_permlane32_swap(__float_as_uint(ga[1]), __float_as_uint(ga[3]),
                                                        false, false);
      // h02: rows 0 (lanes < 32) and 2; h13: rows 1 and 3
      const float h02 = __uint_as_float(s02[0]) + __uint_as_float(s02[1]);
      const float h13 = __uint_as_float(s13[0]) + __uint_as_float(s13[1]);
      const auto q = __builtin_amdgcn_permlane16_swap(__float_as_uint(h02), __float_as_uint(h13), false, false);
      s = __uint_as_float(q[0]) + __uint_as_float(q[1]);  // 16-lane row r: row r
    } else if constexpr (RG == 2) {
      const auto s01 = __builtin_amdgcn_permlane32_swap(__float_as_uint(ga[0]), __float_as_uint(ga[1]),
                                                        false, false);
      const float h = __uint_as_float(s01[0]) + __uint_as_float(s01[1]);  // lanes < 32: row 0
      const auto q = __builtin_amdgcn_permlane16_swap(__float_as_uint(h), __float_as_uint(h), false, false);
      s = __uint_as_float(q[0]) + __uint_as_float(q[1]);  // lanes < 32: row 0; the rest: row 1
    } else {
      const auto s0 = __builtin_amdgcn_permlane32_swap(__float_as_uint(ga[0]), __float_as_uint(ga[0]),
                                                       false, false);
      const float h = __uint_as_float(s0[0]) + __uint_as_float(s0[1]);
      const auto q = __builtin_amdgcn_permlane16_swap(__float_as_uint(h), __float_as_uint(h), false, false);
      s = __uint_as_float(q[0]) + __uint_as_float(q[1]);
    }
    s = row_sum16(s);
    if constexpr (POST == kGemvSiluPair) {
      // the up rows' sums sit 32 lanes above their gate rows'
      const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(s), __float_as_uint(s), false, false);
      if (lane < 32 && (lane & (kLanesPerRow - 1)) == 0) {
        const int n = n0 + lane / kLanesPerRow;
        if (n < n_out) {
          const float g = St<kBF16>::load(St<kBF16>::store(s));
          const float u = St<kBF16>::load(St<kBF16>::store(__uint_as_float(sw[1])));
          const float sg = g / (1.0f + expf(-g));
          y[n] = St<kBF16>::store(sg * u);
        }
      }
    } else if ((lane & (kLanesPerRow - 1)) == 0) {
      const int n = n0 + gi * RG + lane / kLanesPerRow;
      if (n < n_out) y[n] = St<kBF16>::store(res ? s + St<kBF16>::load(rbits[gi]) : s);
    }
  }
  }
}

}  // namespace luc

// Rows per wave R and 8-element chunks per lane C (rows of up to 512 C
// elements): eight, four or one row of up to 1024 elements (the 896-wide
// hidden state of the lm_head, gate/up, q/k/v and o products; fewer rows per
// wave when there are fewer rows), or one row of up to 5120 (the down product's 4864) or 8192;
// the gate/up pairs take four rows of up to 1024 or two of up to 5120 or 8192
// (two outputs or one).
#define LUC_GEMV_KERNEL(NAME, PRE, POST, R, C)                                                    \
  extern "C" __global__ __launch_bounds__(luc::kGemvThreads) void NAME(uint16_t* y, const uint16_t* in, \
                                                         const uint16_t* w, const uint16_t* res,  \
                                                         const uint16_t* nw, float eps, int n,    \
                                                         int k) {                                 \
    luc::gemv_impl<R, C, PRE, POST>(y, in, w, res, nw, eps, n, k);                                \
  }
LUC_GEMV_KERNEL(luc_gemv_bf16_r4c2, luc::kGemvPlain, luc::kGemvStore, 4, 2)
LUC_GEMV_KERNEL(luc_gemv_bf16_r1c2, luc::kGemvPlain, luc::kGemvStore, 1, 2)
LUC_GEMV_KERNEL(luc_gemv_bf16_r1c10, luc::kGemvPlain, luc::kGemvStore, 1, 10)
LUC_GEMV_KERNEL(luc_gemv_bf16_r1c16, luc::kGemvPlain, luc::kGemvStore, 1, 16)
LUC_GEMV_KERNEL(luc_rmsnorm_gemv_bf16_r4c2, luc::kGemvNorm, luc::kGemvStore, 4, 2)
LUC_GEMV_KERNEL(luc_rmsnorm_gemv_bf16_r8c2, luc::kGemvNorm, luc::kGemvStore, 8, 2)
LUC_GEMV_KERNEL(luc_rmsnorm_gemv_bf16_r1c2, luc::kGemvNorm, luc::kGemvStore, 1, 2)
LUC_GEMV_KERNEL(luc_rmsnorm_gemv_bf16_r1c10, luc::kGemvNorm, luc::kGemvStore, 1, 10)
LUC_GEMV_KERNEL(luc_rmsnorm_gemv_bf16_r1c16, luc::kGemvNorm, luc::kGemvStore, 1, 16)
LUC_GEMV_KERNEL(luc_gate_up_silu_bf16_r4c2, luc::kGemvPlain, luc::kGemvSiluPair, 4, 2)
LUC_GEMV_KERNEL(luc_gate_up_silu_bf16_r2c10, luc::kGemvPlain, luc::kGemvSiluPair, 2, 10)
LUC_GEMV_KERNEL(luc_gate_up_silu_bf16_r2c16, luc::kGemvPlain, luc::kGemvSiluPair, 2, 16)
LUC_GEMV_KERNEL(luc_rmsnorm_gate_up_silu_bf16_r4c2, luc::kGemvNorm, luc::kGemvSiluPair, 4, 2)
LUC_GEMV_KERNEL(luc_rmsnorm_gate_up_silu_bf16_r2c10, luc::kGemvNorm, luc::kGemvSiluPair, 2, 10)
LUC_GEMV_KERNEL(luc_rmsnorm_gate_up_silu_bf16_r2c16, luc::kGemvNorm, luc::kGemvSiluPair, 2, 16)

extern "C" __global__ __launch_bounds__(256) void luc_rmsnorm_bf16(uint16_t* out, const uint16_t* in,
                                                                   const uint16_t* weight, float eps,
                                                                   int n) {
  luc::rmsnorm_impl(out, in, weight, eps, n);
}

extern "C" __global__ __launch_bounds__(256) void luc_silu_mul_bf16(uint16_t* buf, int rows, int inter) {
  luc::silu_mul_impl(buf, rows, inter);
}

extern "C" __global__ __launch_bounds__(256) void luc_embedding_bf16(uint16_t* out, const uint16_t* table,
                                                                     const uint32_t* ids, int vocab,
                                                                     int hidden) {
  luc::embedding_impl(out, table, ids, vocab, hidden);
}

extern "C" __global__ __launch_bounds__(1024) void luc_argmax_bf16(const uint16_t* x, int n,
                                                                   uint32_t* out) {
  luc::argmax_impl(x, n, out);
}
