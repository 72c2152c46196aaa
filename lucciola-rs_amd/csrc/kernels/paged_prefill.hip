// Causal prefill attention over the paged KV cache for gfx950, on MFMA.
//
// Semantics (the reference's per-token prefill loop, Qwen2Model::forward_layer
// src/models.rs:485-550): the prompt rows of sequence b are packed rows
// cu_seqlens[b] .. cu_seqlens[b+1]-1 of qkv, at positions start_pos[b] + i.
// By the time this kernel runs, every row's q and k are roped in place and its
// roped k and v + v_bias are in the cache (the append kernel, launched first
// on the same stream).  Row i of sequence b and q-head qh then attends to
// cache positions 0..start_pos[b] + i through table row b -- the cached prefix
// and the prompt rows up to itself -- exactly what the reference's
// flash_decoding call for that token computes (src/kernels/attention.cu:4-176),
// since by then the cache holds those positions and nothing later.
//
// Work decomposition: workgroup = (sequence b, kv head h, tile of 32 prompt
// rows), G = Hq/Hkv waves, wave w = q-head h*G + w over the same 32 rows, so
// the K and V tiles staged in LDS serve all G heads (GQA).  The workgroup
// walks the tokens 0..(last position of its rows) in blocks of 64:
//   - K block [64 tokens][D] straight into LDS (global_load_lds_dwordx4, one
//     wave-wide load = 1 KB of a page), each token row XOR-swizzled by 16-byte
//     chunk; V block into LDS transposed, V^T[dim][token], rows padded so the
//     MFMA operand reads do not collide; tokens past the context are written
//     as zeros so that 0-weight tokens contribute exactly zero.
//   - per wave, per 32-token half: S^T = K Q^T with v_mfma_f32_32x32x16 (A = K
//     from LDS, B = Q^T held in registers for the whole kernel).  In the MFMA
//     accumulator layout lane l holds q row l % 32 and 16 of the tile's
//     tokens; the other 16 are in lane l ^ 32.  So the causal mask, the row
//     max and the running sum are per lane plus one permlane32 exchange.
//   - online softmax in the exp2 domain, then O^T += V^T P^T
//     (v_mfma_f32_32x32x16, A = V^T from LDS, B = P^T): P^T in the layout the
//     MFMA wants is exactly what the lane already holds, packed to 16 bits,
//     once the 16-token k-slots are ordered as the accumulator orders tokens
//     (slot e of lane group g = token 4g + e, then 8 + 4g + e - 4).
// The output rows are O^T / l, rounded to storage.
#include "luc_common.h"

namespace luc {

typedef __attribute__((address_space(3))) void lds_void_p;
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

struct PrefillArgs {
  const uint16_t* qkv;  // row r at qkv + r*qkv_stride: [q (Hq*D) | k | v], q roped
  int64_t qkv_stride;
  const uint16_t* k_pool;  // [blocks][num_layers][Hkv][16][D]
  const uint16_t* v_pool;
  const int32_t* tables;  // [batch][table_stride]
  int64_t table_stride;
  const int32_t* cu_seqlens;  // [batch + 1]
  const int32_t* start_pos;   // [batch]
  uint16_t* out;              // row r at out + r*out_stride, [Hq*D]
  int64_t out_stride;
  int32_t batch, layer, num_layers, hkv, max_ctx, row_tiles;
  float qk_scale_log2;  // sm_scale * log2(e)
};

template <int DT>
__device__ inline f32x16 mfma32(uint4 a, uint4 b, f32x16 c) {
  if constexpr (DT == kF16)
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

__device__ inline uint32_t pack2(float lo, float hi, int dt) {
  if (dt == kF16) {
    const half2_t v = {(_Float16)lo, (_Float16)hi};
    return __builtin_bit_cast(uint32_t, v);
  }
  return (uint32_t)St<kBF16>::store(lo) | ((uint32_t)St<kBF16>::store(hi) << 16);
}

template <int DT, int D, int G>
__device__ void prefill_impl(const PrefillArgs& A) {
  constexpr int BT = 64;          // tokens per block
  constexpr int CH = D / 8;       // 16-byte chunks per token row
  constexpr int KB = BT * D * 2;  // bytes of a K block
  constexpr int VROW = BT + 4;    // V^T row length in elements (padded)
  constexpr int ND = D / 32;      // 32-dim output tiles
  constexpr int NK = D / 16;      // 16-dim k-steps of QK
  constexpr int NT = 64 * G;
  __shared__ __attribute__((aligned(16))) char s_kb[KB];
  __shared__ __attribute__((aligned(16))) uint16_t s_vt[D * VROW];

  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // tiles in reverse order of rows: the longest causal ranges start first
  const int tiles = A.row_tiles;
  const int per_seq = A.hkv * tiles;
  const int b = blockIdx.x / per_seq;
  const int rem = blockIdx.x - b * per_seq;
  const int h = rem / tiles;
  const int rt = tiles - 1 - (rem - h * tiles);
  const int row0 = A.cu_seqlens[b];
  const int nrows = A.cu_seqlens[b + 1] - row0;
  if (rt * 32 >= nrows) return;
  const int sp = A.start_pos[b];
  const int qh = h * G + w;
  const int my_i = rt * 32 + (lane & 31);  // the lane's prompt row (q row of the tile)
  const bool row_ok = my_i < nrows;
  const int my_pos = sp + my_i;
  uint16_t* const orow = A.out + (int64_t)(row0 + min(my_i, nrows - 1)) * A.out_stride + (int64_t)qh * D;
  const int last = sp + min(rt * 32 + 32, nrows) - 1;  // last position of the tile's rows
  if (sp < 0 || sp + nrows > A.max_ctx) {
    // positions outside the host bound: flagged with NaN, never truncated
    if (row_ok) {
      const int g = lane >> 5;
      for (int d = 0; d < D; d += 8)
        for (int j = 0; j < 4; ++j) orow[d + 4 * g + j] = St<DT>::store(__builtin_nanf(""));
    }
    return;
  }
  const int nkv = last + 1;  // tokens the tile reads
  const int* trow = A.tables + (int64_t)b * A.table_stride;
  const int64_t page_stride = (int64_t)A.num_layers * A.hkv * kPage * D;
  const int64_t head_off = ((int64_t)A.layer * A.hkv + h) * kPage * D;

  // Q^T fragments (B operand): lane l holds q row my_i, dims (l/32)*8 + 16k .. +8
  uint4 qf[NK];
  {
    const uint16_t* qrow = A.qkv + (int64_t)(row0 + min(my_i, nrows - 1)) * A.qkv_stride + (int64_t)qh * D;
#pragma unroll
    for (int k = 0; k < NK; ++k) qf[k] = *(const uint4*)(qrow + (lane >> 5) * 8 + 16 * k);
  }

  f32x16 o[ND];
#pragma unroll
  for (int i = 0; i < ND; ++i)
#pragma unroll
    for (int e = 0; e < 16; ++e) o[i][e] = 0.0f;
  float m_run = -INFINITY, l_run = 0.0f;
  const int g = lane >> 5;

  const int nblk = (nkv + BT - 1) / BT;
  for (int blk = 0; blk < nblk; ++blk) {
    const int t0 = blk * BT;
    const int last_page = (nkv - 1) / kPage;
    // ---- stage K (direct to LDS) and V^T ----
    // K: BT*D*2 bytes = KB/1024 wave-wide loads of 1 KB; load j covers tokens
    // j*(1024/(2D)) .. and is issued by wave j % G.  LDS chunk position
    // (token t, slot c) holds chunk c ^ (t & 7) of the token row.
    constexpr int KLOADS = KB / 1024;
    constexpr int TPL = 1024 / (2 * D);  // tokens per 1 KB load
    for (int j = w; j < KLOADS; j += G) {
      const int tl = j * TPL + lane / CH;  // token within the block
      const int c = lane % CH;
      const int t = min(t0 + tl, nkv - 1);  // past the context: re-read a valid token
      const int page = trow[min(t / kPage, last_page)];
      const char* src = (const char*)(A.k_pool + (int64_t)page * page_stride + head_off +
                                      (int64_t)(t % kPage) * D) + ((c ^ (tl & 7)) << 4);
      __builtin_amdgcn_global_load_lds(src, (lds_void_p*)(s_kb + j * 1024), 16, 0, 0);
    }
    // V: 16-byte chunks (token, 8 dims) -> V^T[dim][token], zero past nkv
    for (int idx = threadIdx.x; idx < BT * CH; idx += NT) {
      const int tl = idx / CH, c = idx % CH;
      const int t = t0 + tl;
      uint4 v = make_uint4(0, 0, 0, 0);
      if (t < nkv) {
        const int page = trow[t / kPage];
        v = *(const uint4*)(A.v_pool + (int64_t)page * page_stride + head_off +
                            (int64_t)(t % kPage) * D + c * 8);
      }
      const uint32_t vw[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        s_vt[(c * 8 + 2 * e) * VROW + tl] = (uint16_t)(vw[e] & 0xffff);
        s_vt[(c * 8 + 2 * e + 1) * VROW + tl] = (uint16_t)(vw[e] >> 16);
      }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();

    // ---- S^T = K Q^T for the two 32-token halves ----
    f32x16 s[2];
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
#pragma unroll
      for (int e = 0; e < 16; ++e) s[hf][e] = 0.0f;
      const int tl = hf * 32 + (lane & 31);  // A row: token
#pragma unroll
      for (int k = 0; k < NK; ++k) {
        const int c = 2 * k + g;  // chunk of dims (l/32)*8 + 16k
        const uint4 ka = *(const uint4*)(s_kb + tl * D * 2 + ((c ^ (tl & 7)) << 4));
        s[hf] = mfma32<DT>(ka, qf[k], s[hf]);
      }
    }
    // ---- mask, online softmax (exp2 domain) ----
    // s[hf][4i + j]: token t0 + 32hf + 8i + 4g + j, q row my_i
    float mb = -INFINITY;
#pragma unroll
    for (int hf = 0; hf < 2; ++hf)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int t = t0 + 32 * hf + 8 * i + 4 * g + j;
          const float x = t <= my_pos ? s[hf][4 * i + j] * A.qk_scale_log2 : -INFINITY;
          s[hf][4 * i + j] = x;
          mb = fmaxf(mb, x);
        }
    {
      const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(mb), __float_as_uint(mb), false, false);
      mb = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
    }
    const float m_new = fmaxf(m_run, mb);  // finite: token 0 is in every row's range
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
    m_run = m_new;
    float ps = 0.0f;
#pragma unroll
    for (int hf = 0; hf < 2; ++hf)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        s[hf][e] = __builtin_amdgcn_exp2f(s[hf][e] - m_new);
        ps += s[hf][e];
      }
    l_run = l_run * alpha + ps;
#pragma unroll
    for (int i = 0; i < ND; ++i)
#pragma unroll
      for (int e = 0; e < 16; ++e) o[i][e] *= alpha;

    // ---- O^T += V^T P^T, 16 tokens per MFMA ----
#pragma unroll
    for (int hf = 0; hf < 2; ++hf)
#pragma unroll
      for (int mm = 0; mm < 2; ++mm) {
        // B = P^T: slots 0..3 = tokens 16mm + 4g + j, slots 4..7 = 16mm + 8 + 4g + j
        const int i0 = 2 * mm, i1 = 2 * mm + 1;
        const uint4 pb = make_uint4(pack2(s[hf][4 * i0], s[hf][4 * i0 + 1], DT),
                                    pack2(s[hf][4 * i0 + 2], s[hf][4 * i0 + 3], DT),
                                    pack2(s[hf][4 * i1], s[hf][4 * i1 + 1], DT),
                                    pack2(s[hf][4 * i1 + 2], s[hf][4 * i1 + 3], DT));
        const int tb = 32 * hf + 16 * mm + 4 * g;  // first token of the lane's slots
#pragma unroll
        for (int db = 0; db < ND; ++db) {
          const uint16_t* vr = s_vt + (db * 32 + (lane & 31)) * VROW + tb;
          const uint2 lo = *(const uint2*)vr;        // tokens tb .. tb+3
          const uint2 hi = *(const uint2*)(vr + 8);  // tokens tb+8 .. tb+11
          o[db] = mfma32<DT>(make_uint4(lo.x, lo.y, hi.x, hi.y), pb, o[db]);
        }
      }
    __syncthreads();  // the next block overwrites the LDS tiles
  }

  // ---- normalise and store: lane holds dims 32db + 8i + 4g + j of row my_i ----
  {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(l_run), __float_as_uint(l_run), false, false);
    l_run = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
  if (row_ok) {
    const float inv = 1.0f / l_run;
#pragma unroll
    for (int db = 0; db < ND; ++db)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint2 v = make_uint2(pack2(o[db][4 * i] * inv, o[db][4 * i + 1] * inv, DT),
                                   pack2(o[db][4 * i + 2] * inv, o[db][4 * i + 3] * inv, DT));
        *(uint2*)(orow + db * 32 + 8 * i + 4 * g) = v;
      }
  }
}

}  // namespace luc

#define LUC_PREFILL(DTN, DT, D, G)                                                              \
  extern "C" __global__ __launch_bounds__(64 * G) void luc_prefill_##DTN##_d##D##_g##G(          \
      luc::PrefillArgs a) {                                                                     \
    luc::prefill_impl<DT, D, G>(a);                                                             \
  }
#define LUC_PREFILL_GROUPS(DTN, DT, D)                                                          \
  LUC_PREFILL(DTN, DT, D, 1)                                                                    \
  LUC_PREFILL(DTN, DT, D, 2)                                                                    \
  LUC_PREFILL(DTN, DT, D, 3)                                                                    \
  LUC_PREFILL(DTN, DT, D, 4)                                                                    \
  LUC_PREFILL(DTN, DT, D, 5)                                                                    \
  LUC_PREFILL(DTN, DT, D, 6)                                                                    \
  LUC_PREFILL(DTN, DT, D, 7)                                                                    \
  LUC_PREFILL(DTN, DT, D, 8)

LUC_PREFILL_GROUPS(bf16, luc::kBF16, 64)
LUC_PREFILL_GROUPS(bf16, luc::kBF16, 128)
LUC_PREFILL_GROUPS(f16, luc::kF16, 64)
LUC_PREFILL_GROUPS(f16, luc::kF16, 128)
