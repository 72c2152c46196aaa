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
// Two kernels compute the same values.  luc_rope_append_{dt}: one workgroup
// per row, element by element, any alignment.  luc_rope_append_vec_{dt}_d{D}:
// one lane per 16-byte chunk pair -- elements i..i+7 and i+D/2..i+D/2+7 of
// one head (a rotation unit) or elements i..i+7 of a v head -- with 16-byte
// loads and stores, for 16-byte aligned rows (the host picks it when every
// pointer and the row stride allow).
//
// Row -> (table row, position):
//   decode mode  (cu_seqlens == nullptr): table row r, position positions[r]
//   packed mode  (cu_seqlens != nullptr): row r belongs to the sequence b with
//     cu_seqlens[b] <= r < cu_seqlens[b+1]; table row b; position
//     start_pos[b] + r - cu_seqlens[b].  Used by prefill.
#include "luc_common.h"

namespace luc {

enum : int { kRopeQ = 1, kRopeK = 2, kWriteKV = 4 };

// Row -> (table row b, position), as above.
__device__ inline void row_position(int row, const int* positions, const int* cu_seqlens,
                                    const int* start_pos, int batch, int& seq, int& pos) {
  seq = row;
  if (cu_seqlens) {
    int lo = 0, hi = batch - 1;  // last b with cu_seqlens[b] <= row
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (cu_seqlens[mid] <= row) lo = mid; else hi = mid - 1;
    }
    seq = lo;
    pos = start_pos[seq] + (row - cu_seqlens[seq]);
  } else {
    pos = positions[row];
  }
}


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
                                 int table_stride, int num_blocks, uint16_t* k_pool,
                                 uint16_t* v_pool, int layer, int num_layers, int hq, int hkv,
                                 int head_dim, int flags) {
  const int row = blockIdx.x;
  int seq, pos;
  row_position(row, positions, cu_seqlens, start_pos, batch, seq, pos);
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
    // a page outside the pool is never an address: q and k are still roped
    // in place, only the cache write is skipped (the reference reads the
    // entry unchecked, kv_cache.cu:28); the step kernel does the same
    if (phys < 0 || phys >= num_blocks) flags &= ~kWriteKV;
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

template <int DT, int D>
__device__ void rope_append_vec_impl(uint16_t* q, const uint16_t* q_bias, uint16_t* k,
                                     const uint16_t* k_bias, const uint16_t* v,
                                     const uint16_t* v_bias, int64_t row_stride,
                                     const float* cos_t, const float* sin_t, const int* positions,
                                     const int* cu_seqlens, const int* start_pos, int batch,
                                     const int* tables, int table_stride, int num_blocks,
                                     uint16_t* k_pool, uint16_t* v_pool, int layer,
                                     int num_layers, int hq, int hkv, int flags, int rows) {
#pragma clang fp contract(off)
  constexpr int C = D / 16;  // 8-element chunks per half head
  constexpr int HALF = D / 2;
  const int nq = (flags & kRopeQ) ? hq : 0;
  const int nk = (flags & (kRopeK | kWriteKV)) ? hkv : 0;
  const int nv = (flags & kWriteKV) ? hkv : 0;
  const int rot_units = (nq + nk) * C;
  const int units = rot_units + nv * 2 * C;  // lanes per row
  const int64_t item = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int row = (int)(item / units);
  if (row >= rows) return;
  const int u = (int)(item - (int64_t)row * units);
  const int64_t roff = (int64_t)row * row_stride;
  const int64_t head_stride = (int64_t)kPage * D;
  // The operands depend on the row only: their loads are issued before the
  // row's position is looked up (cu_seqlens search, table), so the two
  // latencies overlap.
  const bool rot = u < rot_units;
  const int hh = rot ? u / C : (u - rot_units) / (2 * C);
  const int i = rot ? (u % C) * 8 : ((u - rot_units) % (2 * C)) * 8;
  const bool isq = rot && hh < nq;
  const int h = isq || !rot ? hh : hh - nq;
  uint16_t* const x = (isq ? q : rot ? k : const_cast<uint16_t*>(v)) + roff + (int64_t)h * D;
  const uint16_t* const bias = isq ? q_bias : rot ? k_bias : v_bias;
  uint4 a = *(const uint4*)(x + i), b = make_uint4(0, 0, 0, 0);
  if (rot) b = *(const uint4*)(x + i + HALF);
  uint4 ba = make_uint4(0, 0, 0, 0), bb = ba;
  if (bias) {
    ba = *(const uint4*)(bias + h * D + i);
    if (rot) bb = *(const uint4*)(bias + h * D + i + HALF);
  }
  int seq, pos;
  if (cu_seqlens) {
    // The workgroup's first row is looked up once, through the scalar cache;
    // lanes whose row lies in the same sequence take it from there, the
    // others (a workgroup that straddles a sequence boundary) search alone.
    typedef __attribute__((address_space(4))) const int const_i32_p;
    const const_i32_p* cu = (const const_i32_p*)cu_seqlens;
    const int row_first = (int)((int64_t)blockIdx.x * blockDim.x / units);
    int lo = 0, hi = batch - 1;  // last b with cu_seqlens[b] <= row_first
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (cu[mid] <= row_first) lo = mid; else hi = mid - 1;
    }
    if (row < cu[lo + 1]) {
      seq = lo;
      pos = ((const const_i32_p*)start_pos)[lo] + (row - cu[lo]);
    } else {
      row_position(row, positions, cu_seqlens, start_pos, batch, seq, pos);
    }
  } else {
    seq = row;
    pos = positions[row];
  }
  if (pos < 0 || ((flags & kWriteKV) && pos >= table_stride * kPage)) return;
  // the rotation's cos/sin and the page number both depend on the position
  // only: issued together
  const bool rope = rot && (isq || (flags & kRopeK));
  float4 c0 = make_float4(0.f, 0.f, 0.f, 0.f), c1 = c0, s0 = c0, s1 = c0;
  if (rope) {
    const float4* cp = (const float4*)(cos_t + (int64_t)pos * HALF + i);
    const float4* sp = (const float4*)(sin_t + (int64_t)pos * HALF + i);
    c0 = cp[0]; c1 = cp[1]; s0 = sp[0]; s1 = sp[1];
  }
  int64_t slot0 = 0;  // pool offset of (pos, head 0, dim 0)
  bool write_kv = (flags & kWriteKV) != 0;
  if (write_kv) {
    const int64_t phys = tables[(int64_t)seq * table_stride + pos / kPage];
    // a page outside the pool is never an address: q and k are still roped
    // in place, only the cache write is skipped (as in the step kernel)
    write_kv = phys >= 0 && phys < num_blocks;
    slot0 = ((phys * num_layers + layer) * hkv) * head_stride + (int64_t)(pos % kPage) * D;
  }
  if (rot) {
    if (rope) {
      rope_rotate8<DT>(a, b, ba, bb, bias != nullptr, c0, c1, s0, s1);
      *(uint4*)(x + i) = a;
      *(uint4*)(x + i + HALF) = b;
    }
    if (!isq && write_kv) {
      uint16_t* dst = k_pool + slot0 + h * head_stride + i;
      *(uint4*)dst = a;
      *(uint4*)(dst + HALF) = b;
    }
  } else if (write_kv) {
    uint16_t o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e)
      o[e] = St<DT>::store(St<DT>::load(chunk_elem(a, e)) + (bias ? St<DT>::load(chunk_elem(ba, e)) : 0.0f));
    *(uint4*)(v_pool + slot0 + h * head_stride + i) = chunk_pack(o);
  }
}

}  // namespace luc

#define LUC_ROPE_APPEND_VEC(NAME, DT, D)                                                          \
  extern "C" __global__ __launch_bounds__(256) void NAME(                                         \
      uint16_t* q, const uint16_t* q_bias, uint16_t* k, const uint16_t* k_bias,                   \
      const uint16_t* v, const uint16_t* v_bias, int64_t row_stride, const float* cos_t,          \
      const float* sin_t, const int* positions, const int* cu_seqlens, const int* start_pos,      \
      int batch, const int* tables, int table_stride, int num_blocks, uint16_t* k_pool,           \
      uint16_t* v_pool, int layer, int num_layers, int hq, int hkv, int head_dim, int flags,      \
      int rows) {                                                                                 \
    luc::rope_append_vec_impl<DT, D>(q, q_bias, k, k_bias, v, v_bias, row_stride, cos_t, sin_t,   \
                                     positions, cu_seqlens, start_pos, batch, tables,             \
                                     table_stride, num_blocks, k_pool, v_pool, layer, num_layers, \
                                     hq, hkv, flags, rows);                                       \
  }

LUC_ROPE_APPEND_VEC(luc_rope_append_vec_bf16_d64, luc::kBF16, 64)
LUC_ROPE_APPEND_VEC(luc_rope_append_vec_bf16_d128, luc::kBF16, 128)
LUC_ROPE_APPEND_VEC(luc_rope_append_vec_f16_d64, luc::kF16, 64)
LUC_ROPE_APPEND_VEC(luc_rope_append_vec_f16_d128, luc::kF16, 128)

#define LUC_ROPE_APPEND(NAME, DT)                                                                 \
  extern "C" __global__ __launch_bounds__(256) void NAME(                                         \
      uint16_t* q, const uint16_t* q_bias, uint16_t* k, const uint16_t* k_bias,                   \
      const uint16_t* v, const uint16_t* v_bias, int64_t row_stride, const float* cos_t,          \
      const float* sin_t, const int* positions, const int* cu_seqlens, const int* start_pos,      \
      int batch, const int* tables, int table_stride, int num_blocks, uint16_t* k_pool,           \
      uint16_t* v_pool, int layer, int num_layers, int hq, int hkv, int head_dim, int flags) {    \
    luc::rope_append_impl<DT>(q, q_bias, k, k_bias, v, v_bias, row_stride, cos_t, sin_t,          \
                              positions, cu_seqlens, start_pos, batch, tables, table_stride,      \
                              num_blocks, k_pool, v_pool, layer, num_layers, hq, hkv, head_dim,   \
                              flags);                                                             \
  }

LUC_ROPE_APPEND(luc_rope_append_bf16, luc::kBF16)
LUC_ROPE_APPEND(luc_rope_append_f16, luc::kF16)
