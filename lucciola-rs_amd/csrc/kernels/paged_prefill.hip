// Causal prefill attention over the paged KV cache for gfx950, on MFMA.
//
// Semantics (the reference's per-token prefill loop, Qwen2Model::forward_layer
// src/models.rs:485-550): the prompt rows of sequence b are packed rows
// cu_seqlens[b] .. cu_seqlens[b+1]-1 of qkv, at positions start_pos[b] + i.
// By the time this kernel runs, every row's k is roped in place and its roped
// k and v + v_bias are in the cache (the append kernel, launched first on the
// same stream).  q gets its bias and RoPE here, as each row's q is loaded
// (the append kernel's arithmetic, bit for bit), and is written back in place
// (when the tables allow 16-byte loads; else the append kernel ropes q too).  Row i of sequence b and q-head qh then attends to
// cache positions 0..start_pos[b] + i through table row b -- the cached prefix
// and the prompt rows up to itself -- exactly what the reference's
// flash_decoding call for that token computes (src/kernels/attention.cu:4-176),
// since by then the cache holds those positions and nothing later.
//
// Work decomposition: workgroup = (sequence b, kv head h, pair p of tiles of
// 32 prompt rows), one wave per q-head of the group of G = Hq/Hkv q-heads
// (4 waves for G <= 4, else 8) over the same 32 rows, so the K and V tiles
// staged in LDS serve every head of the group (GQA).  Of a sequence's nt row tiles the workgroup takes tile nt-1-p
// and then tile p: causal tile t reads about t+1 token blocks, so every pair
// carries the same work, the grid is one wave of equal workgroups and none
// waits on a long tail.  For each tile the workgroup walks the tokens
// 0..(last position of its rows) in blocks of 64, grouped into super-blocks
// (two blocks at head_dim 64 with 8 waves, else one) in an LDS ring of NS
// stages (four at head_dim 64, three at 128): super-block J + NS - 2 loads
// while super-block J is computed, and the waves meet at one barrier per
// super-block.
//   - K and V blocks of 64 tokens straight into LDS (global_load_lds_dwordx4,
//     one wave-wide load = 1 KB of a page, 8 tokens at head_dim 64, 4 of K or
//     8 tokens x 64 dims of V at 128).  K rows are XOR-swizzled by 16-byte
//     chunk and V is stored as 8-token x 32-dim sub-blocks, so that the
//     operand reads below touch every LDS bank once per pass (kkey, vslot).
//     Tokens past the context re-read the last valid token (finite), so their
//     zero weights contribute exactly zero.
//   - per wave, per 32-token half: S^T = K Q^T with v_mfma_f32_32x32x16 (A = K
//     from LDS, B = Q^T held in registers for the whole kernel).  In the MFMA
//     accumulator layout lane l holds q row l % 32 and 16 of the tile's
//     tokens; the other 16 are in lane l ^ 32.  So the causal mask, the row
//     max and the running sum are per lane plus one permlane32 exchange.
//   - online softmax in the exp2 domain, then O^T += V^T P^T
//     (v_mfma_f32_32x32x16, A = V^T read from the row-major V block with the
//     transposing ds_read_b64_tr_b16, B = P^T): P^T in the layout the
//     MFMA wants is exactly what the lane already holds, packed to 16 bits,
//     once the 16-token k-slots are ordered as the accumulator orders tokens
//     (slot e of lane group g = token 4g + e, then 8 + 4g + e - 4).
// The output rows are O^T / l, rounded to storage.
#include "luc_common.h"

namespace luc {

typedef __attribute__((address_space(3))) void lds_void_p;
typedef __attribute__((address_space(3))) char lds_char_p;
typedef __attribute__((address_space(4))) const int const_i32_p;  // scalar loads
template <int N>
struct IC {  // a compile-time index passed to a generic lambda
  static constexpr int value = N;
};

// 32-bit LDS address of a pointer into a __shared__ array.
__device__ inline uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const lds_char_p*)p;
}

struct PrefillArgs {
  uint16_t* qkv;  // row r at qkv + r*qkv_stride: [q (Hq*D) | k | v]
  int64_t qkv_stride;
  const uint16_t* k_pool;  // [blocks][num_layers][Hkv][16][D]
  const uint16_t* v_pool;
  const int32_t* tables;  // [batch][table_stride]
  int64_t table_stride;
  const int32_t* cu_seqlens;  // [batch + 1]
  const int32_t* start_pos;   // [batch]
  uint16_t* out;              // row r at out + r*out_stride, [Hq*D]
  int64_t out_stride;
  // q's bias + RoPE: with cos_t set, q is roped here (in place, as the
  // append kernel would) as it is loaded; else the append kernel has done it
  const uint16_t* q_bias;  // [Hq*D] or null
  const float* cos_t;      // [positions][D/2], 16-byte aligned, or null
  const float* sin_t;
  int32_t batch, layer, num_layers, hkv, max_ctx, pairs;  // pairs: tile pairs per sequence
  int32_t num_blocks;  // pages per pool: table entries outside [0, num_blocks) are never used
  float qk_scale_log2;  // sm_scale * log2(e)
};

// Two values rounded (nearest even) to 16-bit storage, packed: one
// v_cvt_pk_{f16,bf16}_f32 (these values are compared within tolerance; the
// bit-exact RoPE path keeps its own rounding).
__device__ inline uint32_t pack2(float lo, float hi, int dt) {
  if (dt == kF16) {
    const half2_t v = {(_Float16)lo, (_Float16)hi};
    return __builtin_bit_cast(uint32_t, v);
  }
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  const bf16x2 v = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, v);
}

// LDS reads in asm (the compiler would otherwise wait for every outstanding
// global_load_lds before them, including the next block's), each block with
// its own wait, so the results cannot be used before they arrive.
// Four 16-byte reads:
template <int OFF>
__device__ inline void lds_b128x4(uint32_t a0, uint32_t a1, uint32_t a2, uint32_t a3,
                                  uint4* x) {
  asm volatile(
      "ds_read_b128 %0, %4 offset:%8\n\t"
      "ds_read_b128 %1, %5 offset:%8\n\t"
      "ds_read_b128 %2, %6 offset:%8\n\t"
      "ds_read_b128 %3, %7 offset:%8\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(x[0]), "=&v"(x[1]), "=&v"(x[2]), "=&v"(x[3])
      : "v"(a0), "v"(a1), "v"(a2), "v"(a3), "n"(OFF)
      : "memory");
}

// head_dim 64: the operand reads of one block, issued ahead of the VALU work
// that hides their latency, and waited for separately.  The outputs are not
// valid until the matching wait, whose "+v" operands keep every use behind it.
typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));
// K of a 64-token block: chunk k of token lane % 32 of each 32-token half
// (x[k] first half, x[4 + k] second half, HOFF bytes further)
template <int HOFF>
__device__ inline void lds_k_issue(uint32_t a0, uint32_t a1, uint32_t a2, uint32_t a3, u32x4_t* x) {
  asm volatile(
      "ds_read_b128 %0, %8\n\t"
      "ds_read_b128 %1, %9\n\t"
      "ds_read_b128 %2, %10\n\t"
      "ds_read_b128 %3, %11\n\t"
      "ds_read_b128 %4, %8 offset:%12\n\t"
      "ds_read_b128 %5, %9 offset:%12\n\t"
      "ds_read_b128 %6, %10 offset:%12\n\t"
      "ds_read_b128 %7, %11 offset:%12"
      : "=&v"(x[0]), "=&v"(x[1]), "=&v"(x[2]), "=&v"(x[3]), "=&v"(x[4]), "=&v"(x[5]),
        "=&v"(x[6]), "=&v"(x[7])
      : "v"(a0), "v"(a1), "v"(a2), "v"(a3), "n"(HOFF)
      : "memory");
}
// K of one 32-token half of a block: x[k] = chunk k of token lane % 32
__device__ inline void lds_k4_issue(uint32_t a0, uint32_t a1, uint32_t a2, uint32_t a3, u32x4_t* x) {
  asm volatile(
      "ds_read_b128 %0, %4\n\t"
      "ds_read_b128 %1, %5\n\t"
      "ds_read_b128 %2, %6\n\t"
      "ds_read_b128 %3, %7"
      : "=&v"(x[0]), "=&v"(x[1]), "=&v"(x[2]), "=&v"(x[3])
      : "v"(a0), "v"(a1), "v"(a2), "v"(a3)
      : "memory");
}
// Waits for the K reads above while N LDS reads issued after them may stay
// outstanding (LDS reads complete in order; a scalar load still in flight
// only makes the wait stricter).
template <int N>
__device__ inline void lds_wait_k(u32x4_t* x) {
  asm volatile("s_waitcnt lgkmcnt(%8)"
               : "+v"(x[0]), "+v"(x[1]), "+v"(x[2]), "+v"(x[3]), "+v"(x[4]), "+v"(x[5]),
                 "+v"(x[6]), "+v"(x[7])
               : "n"(N)
               : "memory");
}
// V^T of a 64-token block (row stride R bytes): x[4c + 2db + j] is the
// transposing read of token group 16c + 8j through address a_db, i.e. the
// 8-byte halves of the A operand of PV step c = (32-token half, 16-token
// step) and 32-dim tile db.  Issued in two halves: half H issues
// x[8H .. 8H + 7] (PV steps 2H and 2H + 1), so that at most 8 stay
// outstanding behind another wait (lgkmcnt counts to 15).
template <int R, int H>
__device__ inline void lds_v_issue_half(uint32_t a0, uint32_t a1, u32x2_t* x) {
  asm volatile(
      "ds_read_b64_tr_b16 %0, %8 offset:%10\n\t"
      "ds_read_b64_tr_b16 %1, %8 offset:%11\n\t"
      "ds_read_b64_tr_b16 %2, %9 offset:%10\n\t"
      "ds_read_b64_tr_b16 %3, %9 offset:%11\n\t"
      "ds_read_b64_tr_b16 %4, %8 offset:%12\n\t"
      "ds_read_b64_tr_b16 %5, %8 offset:%13\n\t"
      "ds_read_b64_tr_b16 %6, %9 offset:%12\n\t"
      "ds_read_b64_tr_b16 %7, %9 offset:%13"
      : "=&v"(x[8 * H]), "=&v"(x[8 * H + 1]), "=&v"(x[8 * H + 2]), "=&v"(x[8 * H + 3]),
        "=&v"(x[8 * H + 4]), "=&v"(x[8 * H + 5]), "=&v"(x[8 * H + 6]), "=&v"(x[8 * H + 7])
      : "v"(a0), "v"(a1), "n"(32 * H * R), "n"((32 * H + 8) * R), "n"((32 * H + 16) * R),
        "n"((32 * H + 24) * R)
      : "memory");
}
// Waits for the V reads above while N LDS reads issued after them may stay
// outstanding.
template <int N = 0>
__device__ inline void lds_wait_v(u32x2_t* x) {
  asm volatile("s_waitcnt lgkmcnt(%16)"
               : "+v"(x[0]), "+v"(x[1]), "+v"(x[2]), "+v"(x[3]), "+v"(x[4]), "+v"(x[5]),
                 "+v"(x[6]), "+v"(x[7]), "+v"(x[8]), "+v"(x[9]), "+v"(x[10]), "+v"(x[11]),
                 "+v"(x[12]), "+v"(x[13]), "+v"(x[14]), "+v"(x[15])
               : "n"(N)
               : "memory");
}

// 16-byte chunk c of K token row t (within a block) sits at slot c ^ kkey(t):
// the 16 rows that one pass of ds_read_b128 reads (a 16-byte chunk per lane)
// then cover all 64 banks (head_dim 64: rows 2m, 2m + 1 share key m and lie
// 128 bytes apart; head_dim 128: one row is 256 bytes, key t % 16).
template <int D>
__device__ constexpr int kkey(int t) {
  return D == 64 ? (t >> 1) & 7 : t & 15;
}
// Byte offset of dims d .. d + 3 of V token t (within a block): 8-token x
// 32-dim sub-blocks of 512 bytes, token rows of 64 bytes.  A transposing read
// of tokens t0 .. t0 + 7 (t0 % 8 == 0), dims 32u .. 32u + 31 is one
// sub-block, its 32-lane halves 256 contiguous bytes; token t + 8 is 16 D
// bytes further, as in a row-major block.
template <int D>
__device__ constexpr uint32_t vslot(int t, int d) {
  return ((t >> 3) * (D / 32) + (d >> 5)) * 512 + ((t & 7) << 6) + (((d & 31) >> 2) << 3);
}

// Waves per prefill workgroup for group size G (<= 8): one per q-head.
constexpr int prefill_waves(int g) { return g <= 4 ? 4 : 8; }

template <int DT, int D, int G>
__device__ void prefill_impl(const PrefillArgs& A) {
  constexpr int W = prefill_waves(G);  // waves per workgroup: one per q-head of the group
  constexpr int NHG = (G + W - 1) / W;
  constexpr int BT = 64;          // tokens per block
  constexpr int CH = D / 8;       // 16-byte chunks per token row
  constexpr int ROWB = 2 * D;     // bytes per token row
  constexpr int KB = BT * ROWB;   // bytes of a K (or V) block
  // A stage holds SB consecutive blocks (a super-block): the waves meet at a
  // barrier once per stage.  Two blocks when the LDS of one workgroup per CU
  // allows it (d64, 8 waves), else one.
  constexpr int SB = (D == 64 && W == 8) ? 2 : 1;
  constexpr int KS = SB * KB;     // bytes of the K (or V) part of a stage
  constexpr int LOADS = KS / 1024;       // 1 KB wave-wide loads per K (or V) part
  constexpr int TPL = 1024 / ROWB;       // tokens per 1 KB load
  constexpr int ND = D / 32;      // 32-dim output tiles
  constexpr int NK = D / 16;      // 16-dim k-steps of QK
  // NS stages of K and V super-blocks (K row-major, 16-byte chunk c of token
  // t at slot c ^ kkey(t); V at vslot): super-block j is loaded NS - 2 stages
  // before its scores
  constexpr int NS = D == 64 ? 4 : 3;
  // head_dim 64 with two-block super-blocks (8 waves): the software-pipelined steps
  constexpr bool PIPE = D == 64 && SB == 2;
  constexpr int LPW = 2 * LOADS / W;  // loads per wave per stage
  static_assert(LOADS % W == 0, "every wave issues the same number of K (and V) loads");
  __shared__ __attribute__((aligned(16))) char s_kv[NS][2][KS];
  // first token of a page outside the pool among those the tile reads (the
  // minimum over the waves; INT_MAX if none)
  __shared__ int s_bad_tok;

  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // pair-major order: every group's first pair is dispatched before any
  // second pair, and consecutive workgroups (which the hardware spreads over
  // the XCDs) belong to different groups
  const int groups = A.batch * A.hkv * NHG;
  const int pair = blockIdx.x / groups;
  int rem = blockIdx.x - pair * groups;
  const int b = rem / (A.hkv * NHG);
  rem -= b * A.hkv * NHG;
  const int h = rem / NHG;
  const int hg = rem - h * NHG;
  const int row0 = A.cu_seqlens[b];
  const int nrows = A.cu_seqlens[b + 1] - row0;
  const int sp = A.start_pos[b];
  const bool active = hg * W + w < G;  // wave-uniform: a q-head of the group
  const int qh = h * G + min(hg * W + w, G - 1);
  const int g = lane >> 5;
  // q's RoPE here except in the 8-wave head_dim 128 kernels, which have no
  // registers to spare (the host then has the append kernel rope q)
  constexpr bool QROPE = !(D == 128 && W == 8);
  // The lane's share of q-head row qrow (dims g*8 + 16k .. + 8, k < NK), with
  // bias + RoPE at position pos: dims i and i + D/2 are pairs k and k + NK/2
  // of the same lane.  Written back in place when `store`.
  auto rope_q = [&](uint16_t* qrow, int pos, uint4* x, bool store) __attribute__((always_inline)) {
#pragma unroll
    for (int k = 0; k < NK; ++k) x[k] = *(const uint4*)(qrow + g * 8 + 16 * k);
    const bool has_bias = A.q_bias != nullptr;
    const uint16_t* const brow = A.q_bias + (int64_t)qh * D + g * 8;
#pragma unroll
    for (int k = 0; k < NK / 2; ++k) {
      const uint4 zero = make_uint4(0, 0, 0, 0);
      const uint4 b1 = has_bias ? *(const uint4*)(brow + 16 * k) : zero;
      const uint4 b2 = has_bias ? *(const uint4*)(brow + 16 * k + D / 2) : zero;
      const float4* cp = (const float4*)(A.cos_t + (int64_t)pos * (D / 2) + g * 8 + 16 * k);
      const float4* spp = (const float4*)(A.sin_t + (int64_t)pos * (D / 2) + g * 8 + 16 * k);
      rope_rotate8<DT>(x[k], x[k + NK / 2], b1, b2, has_bias, cp[0], cp[1], spp[0], spp[1]);
    }
    if (store)
#pragma unroll
      for (int k = 0; k < NK; ++k) *(uint4*)(qrow + g * 8 + 16 * k) = x[k];
  };
  if (sp < 0 || sp + nrows > A.max_ctx) {
    // positions outside the host bound: flagged with NaN, never truncated
    // (such a sequence may have more tiles than the grid has pairs: the
    // workgroups of its group stride over all its rows)
    if (active)
      for (int r = pair * 32 + (lane & 31); r < nrows; r += A.pairs * 32) {
        uint16_t* const orow = A.out + (int64_t)(row0 + r) * A.out_stride + (int64_t)qh * D;
        for (int d = 0; d < D; d += 8)
          for (int j = 0; j < 4; ++j) orow[d + 4 * g + j] = St<DT>::store(__builtin_nanf(""));
        // q still gets its RoPE where its position lies in the table row
        const int64_t pos = (int64_t)sp + r;
        if (QROPE && A.cos_t && pos >= 0 && pos < A.table_stride * kPage) {
          uint4 qv[NK];
          rope_q(A.qkv + (int64_t)(row0 + r) * A.qkv_stride + (int64_t)qh * D, (int)pos, qv, true);
        }
      }
    return;
  }
  const int nt = (nrows + 31) / 32;  // row tiles of the sequence (nt <= 2 * pairs)
  if (pair >= (nt + 1) / 2) return;
  const int* trow = A.tables + (int64_t)b * A.table_stride;
  const int64_t page_stride = (int64_t)A.num_layers * A.hkv * kPage * D;
  const int64_t head_off = ((int64_t)A.layer * A.hkv + h) * kPage * D;
  const int ntiles = pair < nt - 1 - pair ? 2 : 1;
  // exponents are exp2(s * scale - max): with q negated for a negative scale
  // the scale is positive, so the row max of s * scale is (max s) * scale
  const bool neg_scale = A.qk_scale_log2 < 0.0f;
  const float scale = fabsf(A.qk_scale_log2);
  // lane-relative LDS offsets of the operand reads within a stage:
  //   K (A operand of S^T): token lane % 32 (+32 for the second half, an
  //   immediate offset), chunk of dims 16k + 8g at slot (2k + g) ^ kkey(token);
  //   V^T (ds_read_b64_tr_b16): input lane j = lane % 16 of 16-lane group
  //   k16 = lane / 16 reads token 4g + j / 4 (+ 8, 16, 32 by immediates),
  //   dims 32 db + 16 (k16 % 2) + 4 (j % 4) .. + 3; the group's output lane i
  //   then holds dim 32 db + 16 (k16 % 2) + i of four consecutive tokens.
  //   One instruction's 64 lanes read one 512-byte V sub-block.
  uint32_t krel[NK], vrel[ND];
#pragma unroll
  for (int k = 0; k < NK; ++k) krel[k] = (lane & 31) * ROWB + (((2 * k + g) ^ kkey<D>(lane & 31)) << 4);
  {
    const int tr = 4 * g + ((lane & 15) >> 2);  // token (mod 8) the lane reads
    const int tr_d = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
#pragma unroll
    for (int db = 0; db < ND; ++db) vrel[db] = vslot<D>(tr, 32 * db + tr_d);
  }
  // The 16 bytes that this lane's part of the wave's load i of a stage
  // fetches: token load_token(i) of the stage, 8 dims, at byte
  // load_offset(i, token % page) of the page's rows for this layer and head.
  auto load_token = [&](int i, int ln) {
    const int jj = i * W % LOADS + w;
    return i * W / LOADS == 0 ? jj * TPL + ln / CH                 // K: row-major
                              : 8 * (jj / (D / 64)) + ((ln & 31) >> 2);  // V: sub-blocks 2jj, 2jj + 1
  };
  auto load_offset = [&](int i, int slot, int ln) -> uint32_t {
    const int jj = i * W % LOADS + w;
    const int dim = i * W / LOADS == 0
                        ? 8 * ((ln % CH) ^ kkey<D>(load_token(i, ln)))  // slot ln % CH holds chunk slot ^ kkey
                        : 32 * (2 * (jj % (D / 64)) + (ln >> 5)) + 8 * (ln & 3);
    return (uint32_t)(slot * D + dim) * 2;
  };
  // stage tokens are page-aligned: token % page = load_token % page.  Kept
  // in registers except by the 8-wave head_dim 128 kernels, which have none
  // to spare (they recompute them)
  constexpr bool KEEP_OFF = !(D == 128 && W == 8);
  uint32_t lane_off[LPW];
#pragma unroll
  for (int i = 0; i < LPW; ++i) lane_off[i] = KEEP_OFF ? load_offset(i, load_token(i, lane) % kPage, lane) : 0;
  for (int k = 0; k < ntiles; ++k) {
  const int rt = k == 0 ? nt - 1 - pair : pair;
  const int my_i = rt * 32 + (lane & 31);  // the lane's prompt row (q row of the tile)
  const bool row_ok = active && my_i < nrows;
  const int my_pos = sp + my_i;
  uint16_t* const orow = A.out + (int64_t)(row0 + min(my_i, nrows - 1)) * A.out_stride + (int64_t)qh * D;
  const int last = sp + min(rt * 32 + 32, nrows) - 1;  // last position of the tile's rows
  const int nkv = last + 1;  // tokens the tile reads
  const int nblk = (nkv + BT - 1) / BT;

  // Page numbers of super-block sb that this wave's loads need: load jj
  // covers TPL tokens of one page (TPL divides the page), jj = i * W + w for
  // the K and the V part alike.  Wave-uniform table entries through the
  // scalar cache, read a stage before the loads they address and checked
  // only there, so their round trip overlaps a block's compute.
  constexpr int NPG = LOADS / W;
  auto page_index = [&](int sb, int i) { return min(sb * SB * BT + (i * W + w) * TPL, nkv - 1) / kPage; };
  auto load_pages = [&](int sb, int* pg) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < NPG; ++i) pg[i] = ((const const_i32_p*)trow)[page_index(sb, i)];
  };
  // A page outside the pool is never used as an address: it reads page 0
  // instead, and the rows whose context reaches it get NaN (bad_tok).
  int bad_tok = 0x7fffffff;
  int pgn[NPG];  // table entries of the next super-block to issue
  // Issue the K and V loads of super-block sb into stage st: 2*LOADS
  // wave-wide loads shared round-robin by the waves.  Tokens past the context
  // re-read token nkv - 1 (finite), so their zero weights contribute exactly
  // zero.
  auto issue = [&](int sb, int st, const int* pg) __attribute__((always_inline)) {
    int pv[NPG];
#pragma unroll
    for (int i = 0; i < NPG; ++i) {
      const bool ok = pg[i] >= 0 && pg[i] < A.num_blocks;
      if (!ok) bad_tok = min(bad_tok, page_index(sb, i) * kPage);
      pv[i] = ok ? pg[i] : 0;
    }
    const int sbase = sb * SB * BT;
    // uniform: every token of the stage inside the context, so every lane
    // reads at its fixed offset within the page (a 32-bit offset from the
    // page row's scalar base address)
    const bool whole = sbase + SB * BT <= nkv;
#pragma unroll
    for (int i = 0; i < LPW; ++i) {
      const int kv = i * W / LOADS, jj = i * W % LOADS + w;
      const char* const base = (const char*)((kv ? A.v_pool : A.k_pool) +
                                             (int64_t)pv[i % NPG] * page_stride + head_off);
      // (the 8 tokens of a V load lie in the page of the K load jj: both are
      // 8-aligned within it)
      // (the lane's offsets are recomputed from an opaque copy of the lane
      // index where they are not kept, so that the compiler keeps no other
      // lane constants alive for them)
      int ln = lane;
      asm volatile("" : "+v"(ln));
      const uint32_t off = !whole ? load_offset(i, min(sbase + load_token(i, ln), nkv - 1) % kPage, ln)
                           : KEEP_OFF ? lane_off[i] : load_offset(i, load_token(i, ln) % kPage, ln);
      __builtin_amdgcn_global_load_lds(base + off, (lds_void_p*)(s_kv[st][kv] + jj * 1024), 16, 0,
                                       0);
    }
  };
  // s_waitcnt vmcnt(n * LPW): all but this wave's loads of the n most recently
  // issued super-blocks have landed (loads complete in order)
  auto wait_blocks = [&](int n) __attribute__((always_inline)) {
    if (n >= 2) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * LPW) : "memory");
    else if (n == 1) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(LPW) : "memory");
    else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  };
  static_assert(NS - 2 <= 2, "wait_blocks covers up to two newer super-blocks");
  // Q^T fragments (B operand): lane l holds q row my_i, dims (l/32)*8 + 16k .. +8
  // (loaded before the tile's first K/V loads are issued, so the block waits
  // below count only block loads)
  // (with q's RoPE here, loaded and roped once the tile's first super-block
  // of K/V loads is issued: the two latencies overlap, and that super-block
  // is waited for before the first scores anyway; written back at the tile's
  // end)
  uint4 qf[NK];
  uint16_t* const qrow = A.qkv + (int64_t)(row0 + min(my_i, nrows - 1)) * A.qkv_stride + (int64_t)qh * D;
  const bool qrope = QROPE && A.cos_t != nullptr;  // wave-uniform
  if (!qrope)
#pragma unroll
    for (int k = 0; k < NK; ++k) qf[k] = *(const uint4*)(qrow + g * 8 + 16 * k);
  auto finish_q = [&]() __attribute__((always_inline)) {
    if (qrope) rope_q(qrow, sp + min(my_i, nrows - 1), qf, false);
    if (neg_scale)  // S = -(K Q^T) exactly: sign flips commute with rounding
#pragma unroll
      for (int k = 0; k < NK; ++k) {
        qf[k].x ^= 0x80008000u; qf[k].y ^= 0x80008000u;
        qf[k].z ^= 0x80008000u; qf[k].w ^= 0x80008000u;
      }
    // q is complete here, so the block waits below count only block loads
#pragma unroll
    for (int k = 0; k < NK; ++k) asm volatile("" ::"v"(qf[k].x), "v"(qf[k].y), "v"(qf[k].z), "v"(qf[k].w));
  };

  // ---- S^T = K Q^T of block blk, two 32-token halves ----
  auto qk = [&](int blk, f32x16* sc) __attribute__((always_inline)) {
    const uint32_t kbase = lds_addr(s_kv[(blk / SB) % NS][0]) + (blk % SB) * KB;
    uint32_t ka_addr[NK];
#pragma unroll
    for (int k = 0; k < NK; ++k) ka_addr[k] = kbase + krel[k];
    auto half = [&](auto hfc) __attribute__((always_inline)) {
      constexpr int hf = decltype(hfc)::value;
      uint4 ka[NK];
#pragma unroll
      for (int k = 0; k < NK; k += 4)
        lds_b128x4<hf * 32 * ROWB>(ka_addr[k], ka_addr[k + 1], ka_addr[k + 2], ka_addr[k + 3], ka + k);
#pragma unroll
      for (int e = 0; e < 16; ++e) sc[hf][e] = 0.0f;
#pragma unroll
      for (int k = 0; k < NK; ++k) sc[hf] = mfma32<DT>(ka[k], qf[k], sc[hf]);
    };
    half(IC<0>{});
    half(IC<1>{});
  };

  f32x16 o[ND], osum;  // O^T and, in every one of its rows, the row sums of P
#pragma unroll
  for (int i = 0; i < ND; ++i)
#pragma unroll
    for (int e = 0; e < 16; ++e) o[i][e] = 0.0f;
#pragma unroll
  for (int e = 0; e < 16; ++e) osum[e] = 0.0f;
  float m_run = -INFINITY;
  // all-ones A operand: its MFMA with P^T sums P over the block's tokens
  const uint32_t one2 = DT == kF16 ? 0x3c003c00u : 0x3f803f80u;
  const uint4 ones = make_uint4(one2, one2, one2, one2);

  // ---- mask, online softmax (exp2 domain) and O^T += V^T P^T of block blk ----
  // (a) mask, block max and the lazy move of the running max
  // mb: the lane's row max of the block's scores (both 32-token halves)
  auto lazy_update = [&](float mb) __attribute__((always_inline)) {
    {
      const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(mb), __float_as_uint(mb), false, false);
      mb = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
    }
    // lazy running max: it moves only when some row's block max passes it by
    // more than kLazyMax (then every row takes its new max), so exponents
    // stay below 2^kLazyMax and the rescale of o is rare
    const float m_blk = mb * scale;  // finite: token 0 is in every row's range
    if (__builtin_amdgcn_ballot_w64(m_blk > m_run + kLazyMax) != 0) {  // wave-uniform
      const float m_new = fmaxf(m_run, m_blk);
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
      m_run = m_new;
#pragma unroll
      for (int i = 0; i < ND; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) o[i][e] *= alpha;
#pragma unroll
      for (int e = 0; e < 16; ++e) osum[e] *= alpha;
    }
  };
  // block blk entirely at or before the tile's first row position: no mask
  auto unmasked = [&](int blk) { return blk * BT + BT - 1 <= sp + rt * 32; };
  auto softmax_max = [&](int blk, f32x16* sc) __attribute__((always_inline)) {
    const int t0 = blk * BT;
    // sc[hf][4i + j]: token t0 + 32hf + 8i + 4g + j, q row my_i
    float mb = -INFINITY;
    if (unmasked(blk)) {  // wave-uniform: below the diagonal
#pragma unroll
      for (int hf = 0; hf < 2; ++hf)
#pragma unroll
        for (int e = 0; e < 16; ++e) mb = fmaxf(mb, sc[hf][e]);
    } else {
#pragma unroll
      for (int hf = 0; hf < 2; ++hf)
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int t = t0 + 32 * hf + 8 * i + 4 * g + j;
            const float x = t <= my_pos ? sc[hf][4 * i + j] : -INFINITY;
            sc[hf][4 * i + j] = x;
            mb = fmaxf(mb, x);
          }
    }
    lazy_update(mb);
  };
  // (b) the weights exp2(s * scale - m)
  auto softmax_exp = [&](f32x16* sc) __attribute__((always_inline)) {
#pragma unroll
    for (int hf = 0; hf < 2; ++hf)
#pragma unroll
      for (int e = 0; e < 16; ++e) sc[hf][e] = __builtin_amdgcn_exp2f(fmaf(sc[hf][e], scale, -m_run));
  };
  // B = P^T of PV step (hf, mm): slots 0..3 = tokens 16mm + 4g + j, slots
  // 4..7 = 16mm + 8 + 4g + j of half hf
  auto p_operand = [&](const f32x16* sc, int hf, int mm) __attribute__((always_inline)) {
    const int i0 = 2 * mm, i1 = 2 * mm + 1;
    return make_uint4(pack2(sc[hf][4 * i0], sc[hf][4 * i0 + 1], DT),
                      pack2(sc[hf][4 * i0 + 2], sc[hf][4 * i0 + 3], DT),
                      pack2(sc[hf][4 * i1], sc[hf][4 * i1 + 1], DT),
                      pack2(sc[hf][4 * i1 + 2], sc[hf][4 * i1 + 3], DT));
  };
  auto softmax_pv = [&](int blk, f32x16* sc) __attribute__((always_inline)) {
    softmax_max(blk, sc);
    softmax_exp(sc);

    // O^T += V^T P^T, 16 tokens per MFMA
    const uint32_t vbase = lds_addr(s_kv[(blk / SB) % NS][1]) + (blk % SB) * KB;
    uint32_t va_addr[ND];
#pragma unroll
    for (int db = 0; db < ND; ++db) va_addr[db] = vbase + vrel[db];
    auto pv_step = [&](auto hfc, auto mmc) __attribute__((always_inline)) {
      constexpr int hf = decltype(hfc)::value, mm = decltype(mmc)::value;
      // B = P^T: slots 0..3 = tokens 16mm + 4g + j, slots 4..7 = 16mm + 8 + 4g + j
      constexpr int i0 = 2 * mm, i1 = 2 * mm + 1;
      const uint4 pb = make_uint4(pack2(sc[hf][4 * i0], sc[hf][4 * i0 + 1], DT),
                                  pack2(sc[hf][4 * i0 + 2], sc[hf][4 * i0 + 3], DT),
                                  pack2(sc[hf][4 * i1], sc[hf][4 * i1 + 1], DT),
                                  pack2(sc[hf][4 * i1 + 2], sc[hf][4 * i1 + 3], DT));
      constexpr int off = (32 * hf + 16 * mm) * ROWB;  // first token of the lane's slots, less 4g
      uint2 va[ND][2];
#pragma unroll
      for (int db = 0; db < ND; ++db) lds_tr16x2<off, off + 8 * ROWB>(va_addr[db], va[db]);
      osum = mfma32<DT>(ones, pb, osum);
#pragma unroll
      for (int db = 0; db < ND; ++db)
        o[db] = mfma32<DT>(make_uint4(va[db][0].x, va[db][0].y, va[db][1].x, va[db][1].y), pb, o[db]);
    };
    pv_step(IC<0>{}, IC<0>{});
    pv_step(IC<0>{}, IC<1>{});
    pv_step(IC<1>{}, IC<0>{});
    pv_step(IC<1>{}, IC<1>{});
  };

  // Iteration blk: the scores of block blk+1 go to the matrix cores while
  // this wave's VALU does the softmax of block blk, then block blk's PV.
  // When block blk+1 starts super-block J, its loads are waited for first,
  // and the barrier also tells every wave that super-block J-2 is consumed,
  // so its stage takes super-block J + NS - 2.
  const int nsb = (nblk + SB - 1) / SB;
  auto boundary = [&](int blk, bool prefetch) __attribute__((always_inline)) {  // before block blk + 1
    if ((blk + 1) % SB == 0) {
      const int J = (blk + 1) / SB;
      wait_blocks(min(NS - 3, nsb - 1 - J));
      __builtin_amdgcn_s_barrier();
      if (J + NS - 2 < nsb) {
        issue(J + NS - 2, (J + NS - 2) % NS, pgn);
        if (prefetch && J + NS - 1 < nsb) load_pages(J + NS - 1, pgn);
      }
    }
  };
  // the table entries the next boundary issues from, read once this block's
  // work is issued (head_dim 64)
  auto prefetch_pages = [&](int blk) __attribute__((always_inline)) {
    if ((blk + 1) % SB == 0) {
      const int J = (blk + 1) / SB;
      if (J + NS - 1 < nsb) load_pages(J + NS - 1, pgn);
    }
  };
  auto step = [&](int blk, f32x16* cur, f32x16* nxt) __attribute__((always_inline)) {
    if constexpr (D == 64) {
      // the LDS reads of K(blk + 1) and of the first half of V(blk) go out
      // before the mask and max of block blk, the second half of V(blk)
      // before its exponentials, so they land while the VALU works; the
      // scores of blk + 1 reach the matrix cores before the exponentials,
      // the PV of blk after them
      u32x4_t ka[8];
      u32x2_t va[16];
      const bool has_next = blk + 1 < nblk;
      if (has_next) {
        boundary(blk, false);
        if (active) {
          const uint32_t kbase = lds_addr(s_kv[((blk + 1) / SB) % NS][0]) + ((blk + 1) % SB) * KB;
          lds_k_issue<32 * ROWB>(kbase + krel[0], kbase + krel[1], kbase + krel[2], kbase + krel[3], ka);
        }
      }
      if (active) {
        const uint32_t vbase = lds_addr(s_kv[(blk / SB) % NS][1]) + (blk % SB) * KB;
        lds_v_issue_half<ROWB, 0>(vbase + vrel[0], vbase + vrel[1], va);
        softmax_max(blk, cur);
        if (has_next) {
          lds_wait_k<8>(ka);  // the first V reads of this block may still be in flight
#pragma unroll
          for (int hf = 0; hf < 2; ++hf) {
#pragma unroll
            for (int e = 0; e < 16; ++e) nxt[hf][e] = 0.0f;
#pragma unroll
            for (int k = 0; k < NK; ++k)
              nxt[hf] = mfma32<DT>(__builtin_bit_cast(uint4, ka[4 * hf + k]), qf[k], nxt[hf]);
          }
        }
        lds_v_issue_half<ROWB, 1>(vbase + vrel[0], vbase + vrel[1], va);
        softmax_exp(cur);
        lds_wait_v(va);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const uint4 pb = p_operand(cur, c >> 1, c & 1);
          osum = mfma32<DT>(ones, pb, osum);
#pragma unroll
          for (int db = 0; db < ND; ++db)
            o[db] = mfma32<DT>(make_uint4(va[4 * c + 2 * db].x, va[4 * c + 2 * db].y,
                                          va[4 * c + 2 * db + 1].x, va[4 * c + 2 * db + 1].y),
                               pb, o[db]);
        }
      }
      if (has_next) prefetch_pages(blk);
    } else {
      if (blk + 1 < nblk) {
        boundary(blk, true);
        if (active) qk(blk + 1, nxt);
      }
      if (active) softmax_pv(blk, cur);
    }
  };

  // every wave is done with the previous tile's last stage before it is refilled
  if (k) __builtin_amdgcn_s_barrier();
  if (threadIdx.x == 0) s_bad_tok = 0x7fffffff;  // (read by every wave only after a barrier below)
#pragma unroll
  for (int j = 0; j < NS - 1; ++j) {
    if (j < nsb) {
      load_pages(j, pgn);
      issue(j, j, pgn);
    }
    if (j == 0) finish_q();  // (q's loads and super-block 0's are in flight together)
  }
  if (NS - 1 < nsb) load_pages(NS - 1, pgn);
  wait_blocks(min(NS - 2, nsb - 1));
  __builtin_amdgcn_s_barrier();
  f32x16 sa[2], sb[2];
  if constexpr (PIPE) {
    // A software pipeline over blocks; each step is a fixed sequence of MFMA
    // slots -- the 8 score MFMAs of the next block (two accumulation chains,
    // one per 32-token half, run one after the other) and the 12 PV MFMAs of
    // this block -- each followed by its share of the VALU work (this
    // block's exponentials and P^T packing, the next block's row max), so
    // the matrix cores and the VALU of a wave work at once.  Chunk c (of 4)
    // holds score MFMAs 2c, 2c + 1, the PV MFMAs of step c - 1 and the
    // weights of PV step c.  LDS reads: the first half of K(blk + 2) goes
    // out once chain 0 of step blk has read its operands, the second half
    // after chain 1, V(blk + 1) at the end of step blk.  Super-block J's
    // barrier comes at the start of step 2J - 2, before K(2J) is read; every
    // wave has then finished step 2J - 3 and with it every read of
    // super-block J - 2, whose stage takes super-block J + 2.
    u32x4_t ka[8];   // K operands (x[k]: first 32-token half, x[4 + k]: second)
    u32x2_t va[16];  // V^T operands of a block's PV steps
    uint4 pb[4];     // P^T operands of the current block's PV steps
    auto kbase = [&](int blk) { return lds_addr(s_kv[(blk / SB) % NS][0]) + (blk % SB) * KB; };
    // K of one 32-token half (hf) of block blk into x[4 hf .. 4 hf + 3]
    auto read_k_half = [&](int blk, int hf) __attribute__((always_inline)) {
      const uint32_t bb = kbase(blk) + hf * 32 * ROWB;
      lds_k4_issue(bb + krel[0], bb + krel[1], bb + krel[2], bb + krel[3], ka + 4 * hf);
    };
    auto read_v = [&](int blk) __attribute__((always_inline)) {
      const uint32_t bb = lds_addr(s_kv[(blk / SB) % NS][1]) + (blk % SB) * KB;
      lds_v_issue_half<ROWB, 0>(bb + vrel[0], bb + vrel[1], va);
      lds_v_issue_half<ROWB, 1>(bb + vrel[0], bb + vrel[1], va);
    };
    auto fence = []() __attribute__((always_inline)) { __builtin_amdgcn_sched_barrier(0); };
    // score MFMA i (0..7) of the next block: chain (half) i / 4, k-step i % 4
    auto qk_mfma = [&](f32x16* nx, int i) __attribute__((always_inline)) {
      const int hf = i >> 2, kk = i & 3;
      f32x16 acc = nx[hf];
      if (kk == 0)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[e] = 0.0f;
      nx[hf] = mfma32<DT>(__builtin_bit_cast(uint4, ka[4 * hf + kk]), qf[kk], acc);
    };
    // PV MFMA j (0..2) of step c: the row sums, then O^T dims 32 (j - 1) ..
    auto pv_mfma = [&](int c, int j) __attribute__((always_inline)) {
      if (j == 0) {
        osum = mfma32<DT>(ones, pb[c], osum);
      } else {
        const int db = j - 1;
        o[db] = mfma32<DT>(make_uint4(va[4 * c + 2 * db].x, va[4 * c + 2 * db].y,
                                      va[4 * c + 2 * db + 1].x, va[4 * c + 2 * db + 1].y),
                           pb[c], o[db]);
      }
    };
    // weight it (0..7) of PV step c: element 8 (c % 2) + it of half c / 2;
    // P^T of step c is packed after its eighth weight
    auto exp_item = [&](f32x16* cu, int c, int it) __attribute__((always_inline)) {
      const int e = 8 * (c & 1) + it;
      cu[c >> 1][e] = __builtin_amdgcn_exp2f(fmaf(cu[c >> 1][e], scale, -m_run));
      if (it == 7) pb[c] = p_operand(cu, c >> 1, c & 1);
    };
    auto step64 = [&](int blk, f32x16* cu, f32x16* nx) __attribute__((always_inline)) {
      if (blk % 2 == 0) {  // super-block J's barrier, before K(2J) is read
        const int J = (blk + 2) / 2;
        if (J < nsb) {
          wait_blocks(min(NS - 3, nsb - 1 - J));
          __builtin_amdgcn_s_barrier();
          if (J + 2 < nsb) {
            issue(J + 2, (J + 2) % NS, pgn);
            if (J + 3 < nsb) load_pages(J + 3, pgn);
          }
        }
      }
      if (!active) return;
      // K(blk + 1), both halves; V(blk), issued after them, may be in flight
      lds_wait_k<15>(ka);
      float mx[2] = {-INFINITY, -INFINITY};
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        if (c == 1) lds_wait_v<0>(va);  // V(blk)
        // MFMA slots: Q P Q P P (c > 0) or Q Q; the weights of step c and
        // (chunks 2, 3) the row max of chain 0 spread over them
        const int np = c > 0 ? 3 : 0, n = 2 + np;
        const int nm = c >= 2 ? 8 : 0;
        int qi = 0, pi = 0, it = 0, mi = 0;
#pragma unroll
        for (int sl = 0; sl < 5; ++sl) {
          if (sl < n) {
            const bool q_turn = qi < 2 && (pi >= np || (sl & 1) == 0);
            if (q_turn) qk_mfma(nx, 2 * c + qi++);
            else pv_mfma(c - 1, pi++);
            fence();
#pragma unroll
            for (; it < 8 * (sl + 1) / n; ++it) exp_item(cu, c, it);
#pragma unroll
            for (; mi < nm * (sl + 1) / n; ++mi) {
              const int e = 8 * (c - 2) + mi;
              mx[e & 1] = fmaxf(mx[e & 1], nx[0][e]);
            }
            fence();
          }
        }
#pragma unroll
        for (; it < 8; ++it) exp_item(cu, c, it);
        // a K half is free once its chain has been issued
        if (c == 1) read_k_half(blk + 2, 0);
        if (c == 3) read_k_half(blk + 2, 1);
      }
      // tail: the PV MFMAs of step 3 with the row max of chain 1
      int mi = 0;
#pragma unroll
      for (int j = 0; j < 3; ++j) {
        pv_mfma(3, j);
        fence();
#pragma unroll
        for (; mi < 16 * (j + 1) / 3; ++mi) mx[mi & 1] = fmaxf(mx[mi & 1], nx[1][mi]);
        fence();
      }
      // (the max is needed only when there is a next block: without this the
      // compiler would move it behind that branch, out of the MFMA shadow)
      asm volatile("" ::"v"(mx[0]), "v"(mx[1]));
      read_v(blk + 1);  // (past the last block: read, never used)
      if (blk + 1 < nblk) {  // wave-uniform
        float mb = fmaxf(mx[0], mx[1]);
        if (!unmasked(blk + 1)) {  // mask the diagonal block, its max again
          const int t0 = (blk + 1) * BT;
          mb = -INFINITY;
#pragma unroll
          for (int hf = 0; hf < 2; ++hf)
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
              for (int j = 0; j < 4; ++j) {
                const int t = t0 + 32 * hf + 8 * i + 4 * g + j;
                const float x = t <= my_pos ? nx[hf][4 * i + j] : -INFINITY;
                nx[hf][4 * i + j] = x;
                mb = fmaxf(mb, x);
              }
        }
        lazy_update(mb);
      }
    };
    if (active) {  // block 0's scores and max; K(1) and V(0) in flight
      read_k_half(0, 0);
      read_k_half(0, 1);
      lds_wait_k<0>(ka);
#pragma unroll
      for (int i = 0; i < 8; ++i) qk_mfma(sa, i);
      read_k_half(1, 0);
      read_k_half(1, 1);
      read_v(0);
      softmax_max(0, sa);
    }
    for (int blk = 0; blk < nblk; blk += 2) {
      step64(blk, sa, sb);
      if (blk + 1 < nblk) step64(blk + 1, sb, sa);
    }
    if (active) {  // the last reads (never used) land before their registers are reused
      lds_wait_k<0>(ka);
      lds_wait_v<0>(va);
    }
  } else {
    if (active) qk(0, sa);
    for (int blk = 0; blk < nblk; blk += 2) {
      step(blk, sa, sb);
      if (blk + 1 < nblk) step(blk + 1, sb, sa);
    }
  }

  // ---- normalise and store: lane holds dims 32db + 8i + 4g + j of row my_i ----
  // rows whose context reaches a page outside the pool: NaN
  if (lane == 0 && bad_tok != 0x7fffffff) atomicMin(&s_bad_tok, bad_tok);
  __syncthreads();
  const int first_bad = s_bad_tok;
  if (!active) continue;
  if (row_ok) {
    if (qrope)  // the roped q, in place (its sign flip undone); stored here, not
                // in the prologue, so that no wait for the tile's first loads
                // waits for these stores too
#pragma unroll
      for (int k = 0; k < NK; ++k) {
        uint4 x = qf[k];
        if (neg_scale) {
          x.x ^= 0x80008000u; x.y ^= 0x80008000u; x.z ^= 0x80008000u; x.w ^= 0x80008000u;
        }
        *(uint4*)(qrow + g * 8 + 16 * k) = x;
      }
    const float inv = my_pos >= first_bad ? __builtin_nanf("") : 1.0f / osum[0];
#pragma unroll
    for (int db = 0; db < ND; ++db)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint2 v = make_uint2(pack2(o[db][4 * i] * inv, o[db][4 * i + 1] * inv, DT),
                                   pack2(o[db][4 * i + 2] * inv, o[db][4 * i + 3] * inv, DT));
        *(uint2*)(orow + db * 32 + 8 * i + 4 * g) = v;
      }
  }
  }  // tiles
}

}  // namespace luc

#define LUC_PREFILL(DTN, DT, D, G)                                                              \
  extern "C" __global__ __launch_bounds__(64 * luc::prefill_waves(G)) void luc_prefill_##DTN##_d##D##_g##G(             \
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
