// The Qwen2 model loop's small kernels for gfx950: embedding gather, RMSNorm,
// fused SiLU * up, greedy argmax -- the reference's batched_embedding_kernel
// (src/kernels/embedding.cu), rmsnorm_nvidia (src/kernels/rmsnorm.cu),
// silu_and_mul_fused_kernel (src/kernels/activation.cu) and argmax_kernel
// (src/kernels/sampling.cu).  bf16 storage, f32 arithmetic.
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
// the M = 1 case of Qwen2Model::matmul_bf16 (src/models.rs:251-292), f32
// accumulation; with res the residual the add is its beta = 1 (one rounding).
// One wave per R rows of w (HBM-bound: every byte of w read once, 16 bytes
// per lane and load, all of a wave's loads in flight together).  Lane l
// takes the 8-element chunks c = l, l + 64, ... (C of them at most) of x and
// of each row; a row's products add in chunk order per lane, element order
// within a chunk, then over the lanes by a butterfly (xor 32, 16, ..., 1),
// whose result in lane 0 is stored: a fixed order.  res may alias y (each lane reads its element before
// writing it); x must not.
template <int R, int C>
__device__ void gemv_impl(uint16_t* y, const uint16_t* x, const uint16_t* w, const uint16_t* res,
                          int n_rows, int k) {
  const int lane = threadIdx.x & 63;
  const int n0 = (blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6)) * R;
  if (n0 >= n_rows) return;  // wave-uniform
  const int nch = k / 8;
  const uint4 zero = make_uint4(0, 0, 0, 0);
  uint4 xv[C], wv[R][C];
#pragma unroll
  for (int j = 0; j < C; ++j) {
    const int c = lane + 64 * j;
    xv[j] = c < nch ? *(const uint4*)(x + 8 * c) : zero;
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int n = min(n0 + r, n_rows - 1);  // (rows past the end re-read the last one)
    const uint16_t* const wr = w + (int64_t)n * k;
#pragma unroll
    for (int j = 0; j < C; ++j) {
      const int c = lane + 64 * j;
      wv[r][j] = c < nch ? *(const uint4*)(wr + 8 * c) : zero;
    }
  }
  float acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    float a = 0.0f;
#pragma unroll
    for (int j = 0; j < C; ++j)
#pragma unroll
      for (int e = 0; e < 8; ++e)
        a = fmaf(St<kBF16>::load(chunk_elem(xv[j], e)), St<kBF16>::load(chunk_elem(wv[r][j], e)), a);
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) a += __shfl_xor(a, o, 64);
    acc[r] = a;
  }
  if (lane == 0)  // (the sums in the order lane 0 adds them)
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int n = n0 + r;
      if (n < n_rows) y[n] = St<kBF16>::store(res ? acc[r] + St<kBF16>::load(res[n]) : acc[r]);
    }
}

}  // namespace luc

// Rows per wave and 8-element chunks per lane: four rows of up to 1024
// elements (the 896-wide hidden state of the q/k/v, o, gate/up and lm_head
// products) or one row of up to 8192 (the down product's 4864).
extern "C" __global__ __launch_bounds__(256) void luc_gemv_bf16_r4(uint16_t* y, const uint16_t* x,
                                                                   const uint16_t* w,
                                                                   const uint16_t* res, int n, int k) {
  luc::gemv_impl<4, 2>(y, x, w, res, n, k);
}
extern "C" __global__ __launch_bounds__(256) void luc_gemv_bf16_r1(uint16_t* y, const uint16_t* x,
                                                                   const uint16_t* w,
                                                                   const uint16_t* res, int n, int k) {
  luc::gemv_impl<1, 16>(y, x, w, res, n, k);
}

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
