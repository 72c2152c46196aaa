// RoPE (+q/k bias) and paged K/V cache write for gfx950.
//
// One workgroup per token row.  Covers the reference's rope kernel
// (src/kernels/rope.cu:3-54) and update_kv_cache_kernel
// (src/kernels/kv_cache.cu:3-59), separately or fused:
//   q, k  <- round(rot(x + bias))           in place      (rope.cu:31-52)
//   k_pool[slot] <- k  (bit copy of the roped k)           (kv_cache.cu:53)
//   v_pool[slot] <- round(v + v_bias)                      (kv_cache.cu:56-58)
//   slot = ((table[pos/16] * L + layer) * Hkv + h) * 16*D + (pos%16)*D
//
// The rotation rounds each product and the difference/sum separately
// (contraction off), so results are reproducible bit for bit.
//
// Row -> (table row, position):
//   decode mode  (cu_seqlens == nullptr): table row r, position positions[r]
//   packed mode  (cu_seqlens != nullptr): row r belongs to the sequence b with
//     cu_seqlens[b] <= r < cu_seqlens[b+1]; table row b; position
//     start_pos[b] + r - cu_seqlens[b].  Used by prefill.
#include "luc_common.h"

namespace luc {

enum : int { kRopeQ = 1, kRopeK = 2, kWriteKV = 4 };

template <int DT>
__device__ inline void rotate(uint16_t* x, const uint16_t* bias, int i1, int i2, float c, float s,
                              uint16_t& o1, uint16_t& o2) {
#pragma clang fp contract(off)
  float b1 = bias ? St<DT>::load(bias[i1]) : 0.0f;
  float b2 = bias ? St<DT>::load(bias[i2]) : 0.0f;
  float v1 = St<DT>::load(x[i1]) + b1;
  float v2 = St<DT>::load(x[i2]) + b2;
  float a = v1 * c;
  float b = v2 * s;
  float e = v1 * s;
  float f = v2 * c;
  o1 = St<DT>::store(a - b);
  o2 = St<DT>::store(e + f);
}

template <int DT>
__device__ void rope_append_impl(uint16_t* q, const uint16_t* q_bias, uint16_t* k,
                                 const uint16_t* k_bias, const uint16_t* v,
                                 const uint16_t* v_bias, int64_t row_stride, const float* cos_t,
                                 const float* sin_t, const int* positions, const int* cu_seqlens,
                                 const int* start_pos, int batch, const int* tables,
                                 int table_stride, uint16_t* k_pool, uint16_t* v_pool, int layer,
                                 int num_layers, int hq, int hkv, int head_dim, int flags) {
  const int row = blockIdx.x;
  int seq = row, pos;
  if (cu_seqlens) {
    int lo = 0, hi = batch - 1;  // last b with cu_seqlens[b] <= row
    while (lo < hi) {
      int mid = (lo + hi + 1) >> 1;
      if (cu_seqlens[mid] <= row) lo = mid; else hi = mid - 1;
    }
    seq = lo;
    pos = start_pos[seq] + (row - cu_seqlens[seq]);
  } else {
    pos = positions[row];
  }
  // Rows whose position falls outside the table row (or is negative) are
  // left untouched rather than written out of bounds.
  if (pos < 0 || ((flags & kWriteKV) && pos >= table_stride * kPage)) return;
  const int half = head_dim / 2;
  const int64_t roff = (int64_t)row * row_stride;
  if (q) q += roff;
  if (k) k += roff;
  if (v) v += roff;

  int64_t slot0 = 0;  // pool offset of (pos, head 0, dim 0)
  if (flags & kWriteKV) {
    const int64_t phys = tables[(int64_t)seq * table_stride + pos / kPage];
    const int64_t page_elems = (int64_t)kPage * head_dim;
    slot0 = ((phys * num_layers + layer) * hkv) * page_elems + (int64_t)(pos % kPage) * head_dim;
  }
  const int64_t head_stride = (int64_t)kPage * head_dim;
  const float* crow = cos_t + (int64_t)pos * half;
  const float* srow = sin_t + (int64_t)pos * half;

  if (flags & kRopeQ) {
    for (int idx = threadIdx.x; idx < hq * half; idx += blockDim.x) {
      const int h = idx / half, i = idx % half;
      const int i1 = h * head_dim + i, i2 = i1 + half;
      uint16_t o1, o2;
      rotate<DT>(q, q_bias, i1, i2, crow[i], srow[i], o1, o2);
      q[i1] = o1;
      q[i2] = o2;
    }
  }
  if (flags & (kRopeK | kWriteKV)) {
    for (int idx = threadIdx.x; idx < hkv * half; idx += blockDim.x) {
      const int h = idx / half, i = idx % half;
      const int i1 = h * head_dim + i, i2 = i1 + half;
      uint16_t o1, o2;
      if (flags & kRopeK) {
        rotate<DT>(k, k_bias, i1, i2, crow[i], srow[i], o1, o2);
        k[i1] = o1;
        k[i2] = o2;
      } else {
        o1 = k[i1];
        o2 = k[i2];
      }
      if (flags & kWriteKV) {
        uint16_t* dst = k_pool + slot0 + h * head_stride;
        dst[i] = o1;
        dst[i + half] = o2;
      }
    }
  }
  if (flags & kWriteKV) {
    for (int idx = threadIdx.x; idx < hkv * head_dim; idx += blockDim.x) {
      const int h = idx / head_dim, d = idx % head_dim;
      float val = St<DT>::load(v[idx]) + (v_bias ? St<DT>::load(v_bias[idx]) : 0.0f);
      v_pool[slot0 + h * head_stride + d] = St<DT>::store(val);
    }
  }
}

}  // namespace luc

#define LUC_ROPE_APPEND(NAME, DT)                                                                 \
  extern "C" __global__ __launch_bounds__(256) void NAME(                                         \
      uint16_t* q, const uint16_t* q_bias, uint16_t* k, const uint16_t* k_bias,                   \
      const uint16_t* v, const uint16_t* v_bias, int64_t row_stride, const float* cos_t,          \
      const float* sin_t, const int* positions, const int* cu_seqlens, const int* start_pos,      \
      int batch, const int* tables, int table_stride, uint16_t* k_pool, uint16_t* v_pool,         \
      int layer, int num_layers, int hq, int hkv, int head_dim, int flags) {                      \
    luc::rope_append_impl<DT>(q, q_bias, k, k_bias, v, v_bias, row_stride, cos_t, sin_t,          \
                              positions, cu_seqlens, start_pos, batch, tables, table_stride,      \
                              k_pool, v_pool, layer, num_layers, hq, hkv, head_dim, flags);       \
  }

LUC_ROPE_APPEND(luc_rope_append_bf16, luc::kBF16)
LUC_ROPE_APPEND(luc_rope_append_f16, luc::kF16)
