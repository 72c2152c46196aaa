// luc_attn.cpp -- host side of the C ABI declared in include/luc_attn.h.
//
// Loads the gfx950 code objects (hipModuleLoad), resolves every kernel once at
// init (hipModuleGetFunction), validates arguments on the host and launches on
// the caller's stream (hipModuleLaunchKernel).  It replaces the reference's
// NVRTC build + PTX loader (build.rs:14-42, src/ptx.rs:1-22,
// src/utils.rs:10-18) and the launch code in src/kernels.rs:203-320 and
// src/layers/kv_cache.rs:124-173.
//
// After luc_init the context is read-only, so one context may be used from
// several threads, each with its own stream.  Nothing here allocates device
// memory or synchronises.
#include "luc_attn.h"
#include "kernels/decode_args.h"

#include <hip/hip_runtime_api.h>

#include <dlfcn.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

struct luc_ctx {
  int device = 0;
  int num_cus = 0;
  void* scratch = nullptr;  // this device's copy of the library scratch (luc_scratch.hip)
  std::vector<hipModule_t> modules;
  std::unordered_map<std::string, hipFunction_t> fns;
};

namespace luc_internal {
int scratch_setup(int device, void** out);
}

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

#define LUC_HIP(expr)                                                                  \
  do {                                                                                 \
    hipError_t e_ = (expr);                                                            \
    if (e_ != hipSuccess) return fail(LUC_E_HIP, "%s: %s", #expr, hipGetErrorString(e_)); \
  } while (0)

constexpr const char* kCodeObjects[] = {"rope_append.hsaco",   "paged_decode.hsaco",
                                         "paged_decode_w8.hsaco", "paged_prefill.hsaco",
                                         "model_ops.hsaco",     "sampling.hsaco",
                                         "probe_gather.hsaco"};

// Kernel-side constants (kept in step with csrc/kernels/paged_decode.hip):
// four waves per workgroup, which share one split; tiles of 64 tokens
// (head_dim 64) or 32 (128); a split's block-table entries are held in two
// registers (128 pages).
// Waves per workgroup: the single-tile kernels (_t1, one tile per wave)
// have 8, so a split is 8 tiles; the tile-pair kernels (_t2, longer splits)
// have 4, or 8 (_t2w8) when the launch is a single round of such
// workgroups (tile_pair_waves).  Splits are multiples of 4 tiles.
constexpr int kT1Waves = 8;
constexpr int kT2Waves = 4;
constexpr int kT2WideWaves = 8;
constexpr int kCUs = 256;  // the split plan's CU count (MI355X)
int decode_tile(int head_dim) { return head_dim == 64 ? 64 : 32; }
constexpr int kMaxSplitTokens = 128 * LUC_BLOCK_SIZE;
// Tiles the automatic split choice plans to have in flight at once: about two
// single-tile waves per SIMD of an MI355X (256 CUs x 4 SIMDs).  The
// two-tile kernels hold twice the LDS (two workgroups per CU instead of
// four), so a plan that needs them is made again for half as many tiles:
// one round of resident workgroups instead of two (batch8_32k, 8 x 32768
// tokens at head_dim 128: 1024-token splits, 55.7 us per launch against
// 59.7 us with 512).
constexpr int kPlanTiles = 256 * 4 * 2;

const char* dt_name(int dtype) { return dtype == LUC_F16 ? "f16" : "bf16"; }

bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

std::string self_dir() {
  Dl_info info;
  if (dladdr(reinterpret_cast<void*>(&luc_init), &info) && info.dli_fname) {
    std::string p = info.dli_fname;
    size_t s = p.rfind('/');
    return s == std::string::npos ? std::string(".") : p.substr(0, s);
  }
  return ".";
}

int get_fn(const luc_ctx* ctx, const std::string& name, hipFunction_t* fn) {
  auto it = ctx->fns.find(name);
  if (it == ctx->fns.end()) return fail(LUC_E_LOAD, "kernel %s not loaded", name.c_str());
  *fn = it->second;
  return LUC_OK;
}

int check_device(const luc_ctx* ctx) {
  int cur = -1;
  LUC_HIP(hipGetDevice(&cur));
  if (cur != ctx->device)
    return fail(LUC_E_INVALID, "current device %d differs from the context's device %d", cur,
                ctx->device);
  return LUC_OK;
}

int check_common(const luc_ctx* ctx, int dtype, int head_dim) {
  if (!ctx) return fail(LUC_E_INVALID, "null context");
  if (dtype != LUC_BF16 && dtype != LUC_F16) return fail(LUC_E_INVALID, "bad dtype %d", dtype);
  if (head_dim != 64 && head_dim != 128)
    return fail(LUC_E_UNSUPPORTED, "unsupported head_dim %d (64 or 128)", head_dim);
  return LUC_OK;
}

int check_heads(int hq, int hkv) {
  if (hq <= 0 || hkv <= 0) return fail(LUC_E_INVALID, "head counts must be positive");
  if (hq % hkv) return fail(LUC_E_INVALID, "num_q_heads %d not a multiple of num_kv_heads %d", hq, hkv);
  if (hq / hkv > 8) return fail(LUC_E_UNSUPPORTED, "group size %d > 8", hq / hkv);
  return LUC_OK;
}

int launch(hipFunction_t fn, dim3 grid, dim3 block, void* stream, void** args) {
  LUC_HIP(hipModuleLaunchKernel(fn, grid.x, grid.y, grid.z, block.x, block.y, block.z, 0,
                                reinterpret_cast<hipStream_t>(stream), args, nullptr));
  return LUC_OK;
}

enum : int { kRopeQ = 1, kRopeK = 2, kWriteKV = 4 };

struct AppendArgs {
  void* q = nullptr;
  const void* q_bias = nullptr;
  void* k = nullptr;
  const void* k_bias = nullptr;
  const void* v = nullptr;
  const void* v_bias = nullptr;
  int64_t row_stride = 0;
  const float* cos_t = nullptr;
  const float* sin_t = nullptr;
  const int32_t* positions = nullptr;
  const int32_t* cu_seqlens = nullptr;
  const int32_t* start_pos = nullptr;
  int batch = 0;
  const int32_t* tables = nullptr;
  int table_stride = 0;
  int num_blocks = 1;
  void* k_pool = nullptr;
  void* v_pool = nullptr;
  int layer = 0, num_layers = 1, hq = 0, hkv = 0, head_dim = 0, flags = 0;
};

int launch_append(const luc_ctx* ctx, void* stream, int dtype, int rows, AppendArgs a) {
  void* args[] = {&a.q,         &a.q_bias,    &a.k,          &a.k_bias,   &a.v,
                  &a.v_bias,    &a.row_stride, &a.cos_t,     &a.sin_t,    &a.positions,
                  &a.cu_seqlens, &a.start_pos, &a.batch,     &a.tables,   &a.table_stride,
                  &a.num_blocks, &a.k_pool,    &a.v_pool,    &a.layer,      &a.num_layers, &a.hq,
                  &a.hkv,       &a.head_dim,  &a.flags,      &rows};
  // 16-byte chunk kernel when every row and bias starts on 16 bytes (the
  // pools always do), else the element-wise kernel (same values)
  auto al = [](const void* p) { return !p || aligned(p, 16); };
  const bool rope = a.flags & (kRopeQ | kRopeK);
  const bool vec = a.row_stride % 8 == 0 && al(a.q) && al(a.k) && al(a.v) && al(a.q_bias) &&
                   al(a.k_bias) && al(a.v_bias) && (!rope || (al(a.cos_t) && al(a.sin_t)));
  hipFunction_t fn;
  if (!vec) {
    if (int rc = get_fn(ctx, std::string("luc_rope_append_") + dt_name(dtype), &fn)) return rc;
    return launch(fn, dim3(rows), dim3(128), stream, args);
  }
  if (int rc = get_fn(ctx, std::string("luc_rope_append_vec_") + dt_name(dtype) + "_d" +
                               std::to_string(a.head_dim),
                      &fn))
    return rc;
  // lanes per row: one per rotation unit (8 + 8 elements of a q or k head),
  // one per 8 elements of a v head
  const int chunks = a.head_dim / 16;
  const int nq = (a.flags & kRopeQ) ? a.hq : 0;
  const int nk = (a.flags & (kRopeK | kWriteKV)) ? a.hkv : 0;
  const int nv = (a.flags & kWriteKV) ? a.hkv : 0;
  const int64_t lanes = (int64_t)rows * ((nq + nk) * chunks + nv * 2 * chunks);
  const int64_t grid = ceil_div(lanes, 256);
  if (grid > INT32_MAX) return fail(LUC_E_INVALID, "too many rows for one launch");
  return launch(fn, dim3((unsigned)grid), dim3(256), stream, args);
}

int check_rows(int num_tokens, int64_t row_stride, int min_row) {
  if (num_tokens < 0) return fail(LUC_E_INVALID, "num_tokens %d < 0", num_tokens);
  if (row_stride < min_row)
    return fail(LUC_E_INVALID, "row_stride %lld smaller than a row (%d)", (long long)row_stride, min_row);
  return LUC_OK;
}

int check_cache(const void* k_pool, const void* v_pool, const int32_t* tables, int table_stride,
                int num_blocks, int layer, int num_layers, int block_size) {
  if (block_size != LUC_BLOCK_SIZE)
    return fail(LUC_E_UNSUPPORTED, "block_size %d (only %d)", block_size, LUC_BLOCK_SIZE);
  if (!k_pool || !v_pool || !tables) return fail(LUC_E_INVALID, "null pool or block table");
  if (!aligned(k_pool, 16) || !aligned(v_pool, 16))
    return fail(LUC_E_INVALID, "KV pools must be 16-byte aligned");
  if (num_layers <= 0 || layer < 0 || layer >= num_layers)
    return fail(LUC_E_INVALID, "layer %d outside [0, %d)", layer, num_layers);
  if (table_stride <= 0) return fail(LUC_E_INVALID, "table_stride %d <= 0", table_stride);
  if (num_blocks < 1) return fail(LUC_E_INVALID, "num_blocks %d < 1", num_blocks);
  return LUC_OK;
}

// Splits per sequence are capped at kMaxSplits (the merge's LDS weight table).
constexpr int kMaxSplits = 256;

// Waves of the tile-pair workgroups for a split of st tokens: 8 (the _t2w8
// kernels) when the launch is a single round of one such workgroup per CU
// and each wave gets at least two tiles, else 4.  A single round ends when
// its workgroups end, so fewer, longer splits (half the partials) win there;
// over several rounds two 4-wave workgroups per CU hide each other's
// prologue and merge (batch8_32k, one round: 50.4 us at 2048-token splits
// on 8 waves against 52.6 at 1024 on 4; batch64_long, 4.8 rounds at 4
// waves: 207.5 against 202.9).  Depends only on the arguments.
int tile_pair_waves(int batch, int hkv, int head_dim, int max_ctx, int st) {
  const int tile = decode_tile(head_dim);
  if (st % (kT2WideWaves * tile) != 0 || st < 2 * kT2WideWaves * tile) return kT2Waves;
  return (int64_t)batch * hkv * ceil_div(max_ctx, st) <= kCUs ? kT2WideWaves : kT2Waves;
}

// Split-K chunk length in tokens: a multiple of 4 tiles (the unit), at most
// kMaxSplitTokens.  A split of 8 tiles runs the single-tile kernels (_t1:
// 8 waves, one tile each); every other split the tile-pair kernels (_t2:
// 4 waves walking tiles w, w+4, ... two at a time).  The automatic choice
// assumes the mean context is half of max_ctx and takes the shortest split
// that keeps about kPlanTiles tiles per round (kPlanTiles / 2 for the
// tile-pair kernels); a plan of one unit becomes the 8-tile single-tile
// split (batch32_mixed: 512 tokens, 15.4 us per launch against 15.9 for
// 4-wave workgroups with 256-token splits: half the partials to merge, the
// same tile per wave).  It depends only on the arguments, so
// luc_paged_decode_workspace_size agrees with the launch.  Returns 0 when
// max_ctx cannot be covered by kMaxSplits splits.
int split_tokens_for(int batch, int hkv, int head_dim, int max_ctx, int requested) {
  const int unit = kT2Waves * decode_tile(head_dim);
  const int64_t floor_tokens = ceil_div(ceil_div(max_ctx, kMaxSplits), unit) * unit;
  if (floor_tokens > kMaxSplitTokens) return 0;
  int64_t st;
  if (requested > 0) {
    st = ceil_div(requested, unit) * unit;
  } else {
    const int64_t tiles = (int64_t)batch * hkv *
                          std::max<int64_t>(ceil_div(ceil_div(max_ctx, 2), decode_tile(head_dim)), 1);
    st = ceil_div(tiles, kPlanTiles) * unit;
    if (st > unit) st = ceil_div(tiles, kPlanTiles / 2) * unit;
    else st = (int64_t)kT1Waves * decode_tile(head_dim);
  }
  st = std::min<int64_t>(std::max<int64_t>(st, floor_tokens), kMaxSplitTokens);
  // a 4-wave tile-pair plan of one round (two workgroups per CU): twice the
  // split on 8-wave workgroups if those fit one round too (half the partials)
  if (requested <= 0 && st != (int64_t)kT1Waves * decode_tile(head_dim) &&
      tile_pair_waves(batch, hkv, head_dim, max_ctx, (int)std::min<int64_t>(2 * st, kMaxSplitTokens)) ==
          kT2WideWaves &&
      (int64_t)batch * hkv * ceil_div(max_ctx, st) <= 2 * kCUs)
    st = std::min<int64_t>(2 * st, kMaxSplitTokens);
  return (int)st;
}

// Workspace layout (each section 256-byte aligned):
//   [split arrivals per (b, kv head): int32 x kMaxArrivalCounters, zero between launches]
//   [(max, sum) per (b, kv head, split, head of the group): f32 x2]
//   [o per (b, kv head, split): f32 x group x head_dim]
// The counters come first, at a size that does not depend on the call, so
// that no later call with other sizes finds partials where it expects zeros:
// one zero-filled workspace serves calls of any batch and max_ctx.
constexpr int64_t kMaxArrivalCounters = 1 << 16;  // batch x kv heads
constexpr int64_t kCounterBytes = kMaxArrivalCounters * 4;
int64_t align256(int64_t n) { return ceil_div(n, 256) * 256; }
int64_t ml_bytes(int batch, int hq, int max_splits) {
  return align256((int64_t)batch * hq * max_splits * 2 * 4);
}
int64_t o_bytes(int batch, int hq, int head_dim, int max_splits) {
  return align256((int64_t)batch * hq * max_splits * head_dim * 4);
}

size_t workspace_bytes_for(int batch, int hq, int hkv, int head_dim, int max_ctx, int split_tokens) {
  const int64_t max_splits = ceil_div(max_ctx, split_tokens);
  if (max_splits <= 1 || batch <= 0) return 0;
  (void)hkv;
  return (size_t)(kCounterBytes + ml_bytes(batch, hq, (int)max_splits) +
                  o_bytes(batch, hq, head_dim, (int)max_splits));
}

struct DecodeLaunch {
  luc_decode_args a{};
  hipFunction_t fn = nullptr;  // split-K decode with the merge in its last split
  dim3 grid;
  int waves = 0;  // per workgroup
};

// Shared argument checks and argument block of the two decode entry points.
int prepare_decode(const luc_ctx* ctx, int dtype, bool step, void* out, int64_t out_row_stride,
                   const void* q, int64_t q_row_stride, const void* k_pool, const void* v_pool,
                   const int32_t* block_tables, int table_stride, int num_blocks,
                   const int32_t* positions, int batch, int max_ctx, int layer, int num_layers,
                   int num_q_heads, int num_kv_heads, int head_dim, int block_size,
                   float sm_scale, int split_tokens, void* workspace, size_t workspace_bytes,
                   DecodeLaunch* L) {
  if (int rc = check_common(ctx, dtype, head_dim)) return rc;
  if (int rc = check_heads(num_q_heads, num_kv_heads)) return rc;
  if (int rc = check_cache(k_pool, v_pool, block_tables, table_stride, num_blocks, layer,
                           num_layers, block_size))
    return rc;
  if (batch < 0) return fail(LUC_E_INVALID, "batch %d < 0", batch);
  if (max_ctx <= 0) return fail(LUC_E_INVALID, "max_ctx %d <= 0", max_ctx);
  if (split_tokens < 0) return fail(LUC_E_INVALID, "split_tokens %d < 0", split_tokens);
  if (!out || !q || !positions) return fail(LUC_E_INVALID, "null out, q or positions");
  const int row = num_q_heads * head_dim;
  const int need_q = step ? (num_q_heads + 2 * num_kv_heads) * head_dim : row;
  if (q_row_stride < need_q || out_row_stride < row)
    return fail(LUC_E_INVALID, "q/out row stride smaller than a row (%d / %d)", need_q, row);
  if (!aligned(q, 4) || (q_row_stride % 2))
    return fail(LUC_E_INVALID, "q must be 4-byte aligned with an even row stride");
  if ((int64_t)table_stride * LUC_BLOCK_SIZE < max_ctx)
    return fail(LUC_E_INVALID, "table_stride %d pages cannot hold max_ctx %d", table_stride, max_ctx);

  const int st = split_tokens_for(batch, num_kv_heads, head_dim, max_ctx, split_tokens);
  if (st == 0)
    return fail(LUC_E_UNSUPPORTED, "max_ctx %d exceeds %d splits of %d tokens", max_ctx,
                kMaxSplits, kMaxSplitTokens);
  const int max_splits = (int)ceil_div(max_ctx, st);
  const size_t need = workspace_bytes_for(batch, num_q_heads, num_kv_heads, head_dim, max_ctx, st);
  if (need && (!workspace || workspace_bytes < need))
    return fail(LUC_E_WORKSPACE, "workspace %zu bytes, %zu needed", workspace_bytes, need);
  if (need && !aligned(workspace, 256)) return fail(LUC_E_INVALID, "workspace must be 256-byte aligned");
  if (need && (int64_t)batch * num_kv_heads > kMaxArrivalCounters)
    return fail(LUC_E_UNSUPPORTED, "split-K decode of batch x kv heads %lld above %lld",
                (long long)batch * num_kv_heads, (long long)kMaxArrivalCounters);
  const int64_t grid = (int64_t)max_splits * batch * num_kv_heads;
  if (grid > INT32_MAX) return fail(LUC_E_INVALID, "batch x kv heads x splits too large");

  if (batch == 0) return LUC_OK;  // nothing to launch
  const int group = num_q_heads / num_kv_heads;
  const std::string suffix = std::string(dt_name(dtype)) + "_d" + std::to_string(head_dim) + "_g" +
                             std::to_string(group);
  // the single-tile kernel reads a tile's table entries as one vector, which
  // must fit the table row
  const bool one_tile = st == kT1Waves * decode_tile(head_dim) &&
                        table_stride >= decode_tile(head_dim) / LUC_BLOCK_SIZE;
  L->waves = one_tile ? kT1Waves : tile_pair_waves(batch, num_kv_heads, head_dim, max_ctx, st);
  if (int rc = get_fn(ctx, std::string(step ? "luc_decode_step_" : "luc_decode_") + suffix +
                               (one_tile ? "_t1" : L->waves == kT2WideWaves ? "_t2w8" : "_t2"),
                      &L->fn))
    return rc;
  L->grid = dim3((unsigned)grid);
  luc_decode_args& a = L->a;
  a.q = static_cast<uint16_t*>(const_cast<void*>(q));
  a.q_stride = q_row_stride;
  a.k_pool = static_cast<uint16_t*>(const_cast<void*>(k_pool));
  a.v_pool = static_cast<uint16_t*>(const_cast<void*>(v_pool));
  a.tables = block_tables;
  a.table_stride = table_stride;
  a.positions = positions;
  a.batch = batch;
  a.layer = layer;
  a.num_layers = num_layers;
  a.hkv = num_kv_heads;
  a.num_blocks = num_blocks;
  a.qk_scale_log2 = sm_scale * 1.4426950408889634f;
  a.max_ctx = max_ctx;
  a.split_tokens = st;
  a.max_splits = max_splits;
  if (need) {
    char* ws = static_cast<char*>(workspace);
    a.ws_cnt = reinterpret_cast<int32_t*>(ws);
    a.ws_ml = reinterpret_cast<float*>(ws + kCounterBytes);
    a.ws_o = reinterpret_cast<float*>(ws + kCounterBytes + ml_bytes(batch, num_q_heads, max_splits));
  }
  a.out = static_cast<uint16_t*>(out);
  a.out_stride = out_row_stride;
  return LUC_OK;
}

// Argument block of the prefill attention kernel (paged_prefill.hip,
// luc::PrefillArgs): the same fixed-size fields in the same order.
struct PrefillArgs {
  const void* qkv;
  int64_t qkv_stride;
  const void* k_pool;
  const void* v_pool;
  const int32_t* tables;
  int64_t table_stride;
  const int32_t* cu_seqlens;
  const int32_t* start_pos;
  void* out;
  int64_t out_stride;
  const void* q_bias;
  const float* cos_t;
  const float* sin_t;
  int32_t batch, layer, num_layers, hkv, max_ctx, pairs, num_blocks;
  float qk_scale_log2;
};

int launch_decode(DecodeLaunch& L, void* stream) {
  void* args[] = {&L.a};
  return launch(L.fn, L.grid, dim3(L.waves * 64), stream, args);
}

}  // namespace

namespace luc_internal {
// Error reporting for the other translation units of the library.
int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}
}  // namespace luc_internal

extern "C" {

int luc_abi_version(void) { return LUC_ABI_VERSION; }

const char* luc_last_error(void) { return g_err.c_str(); }

int luc_init(int device, const char* code_object_dir, luc_ctx** out_ctx) {
  if (!out_ctx) return fail(LUC_E_INVALID, "out_ctx is null");
  *out_ctx = nullptr;
  int count = 0;
  LUC_HIP(hipGetDeviceCount(&count));
  if (device < 0 || device >= count)
    return fail(LUC_E_INVALID, "device %d outside [0, %d)", device, count);
  LUC_HIP(hipSetDevice(device));
  const std::string dir = code_object_dir ? std::string(code_object_dir) : self_dir();
  auto* ctx = new luc_ctx;
  ctx->device = device;
  for (const char* name : kCodeObjects) {
    const std::string path = dir + "/" + name;
    hipModule_t mod;
    hipError_t e = hipModuleLoad(&mod, path.c_str());
    if (e != hipSuccess) {
      luc_destroy(ctx);
      return fail(LUC_E_LOAD, "hipModuleLoad(%s): %s", path.c_str(), hipGetErrorString(e));
    }
    ctx->modules.push_back(mod);
  }
  std::vector<std::string> names = {"luc_rmsnorm_bf16", "luc_silu_mul_bf16", "luc_embedding_bf16",
                                    "luc_argmax_bf16", "luc_gather_floor_d64",
                                    "luc_gather_floor_d128", "luc_stream_read"};
  for (int npl : {1, 2, 4, 8, 16}) names.push_back("luc_topk_filter_bf16_n" + std::to_string(npl));
  for (const char* kind : {"luc_gemv", "luc_rmsnorm_gemv"})
    for (const char* v : {"_bf16_r4c2", "_bf16_r1c2", "_bf16_r1c10", "_bf16_r1c16"})
      names.push_back(std::string(kind) + v);
  names.push_back("luc_rmsnorm_gemv_bf16_r8c2");
  for (const char* kind : {"luc_gate_up_silu", "luc_rmsnorm_gate_up_silu"})
    for (const char* v : {"_bf16_r4c2", "_bf16_r2c10", "_bf16_r2c16"}) names.push_back(std::string(kind) + v);
  for (int k = 32; k <= 1024; k *= 2) names.push_back("luc_top_p_sample_" + std::to_string(k));
  for (const char* dt : {"bf16", "f16"}) {
    names.push_back(std::string("luc_rope_append_") + dt);
    for (int d : {64, 128}) names.push_back(std::string("luc_rope_append_vec_") + dt + "_d" + std::to_string(d));
    for (int d : {64, 128})
      for (int g = 1; g <= 8; ++g)
        names.push_back(std::string("luc_prefill_") + dt + "_d" + std::to_string(d) + "_g" +
                        std::to_string(g));
    for (int d : {64, 128})
      for (int g = 1; g <= 8; ++g)
        for (const char* kind : {"luc_decode_", "luc_decode_step_"}) {
          const std::string n = std::string(kind) + dt + "_d" + std::to_string(d) + "_g" +
                                std::to_string(g);
          names.push_back(n + "_t1");
          names.push_back(n + "_t2");
          names.push_back(n + "_t2w8");
        }
  }
  for (const auto& n : names) {
    hipFunction_t fn = nullptr;
    for (hipModule_t m : ctx->modules)
      if (hipModuleGetFunction(&fn, m, n.c_str()) == hipSuccess) break;
    if (!fn) {
      luc_destroy(ctx);
      return fail(LUC_E_LOAD, "kernel %s not found in %s", n.c_str(), dir.c_str());
    }
    ctx->fns[n] = fn;
  }
  if (hipDeviceGetAttribute(&ctx->num_cus, hipDeviceAttributeMultiprocessorCount, device) !=
          hipSuccess ||
      ctx->num_cus < 1)
    ctx->num_cus = 256;
  (void)hipGetLastError();  // clear the misses from probing several modules
  if (int rc = luc_internal::scratch_setup(device, &ctx->scratch)) {
    luc_destroy(ctx);
    return rc;
  }
  *out_ctx = ctx;
  return LUC_OK;
}

void luc_destroy(luc_ctx* ctx) {
  if (!ctx) return;
  for (hipModule_t m : ctx->modules) (void)hipModuleUnload(m);
  delete ctx;
}

int luc_rope_table(float* cos_out, float* sin_out, int max_pos, int head_dim, float base,
                   float scale_factor) {
  if (!cos_out || !sin_out) return fail(LUC_E_INVALID, "null output");
  if (max_pos < 0 || head_dim <= 0 || head_dim % 2) return fail(LUC_E_INVALID, "bad sizes");
  if (!(base > 0.0f)) return fail(LUC_E_INVALID, "rope base must be positive");
  const int half = head_dim / 2;
  const float scale = scale_factor > 0.0f ? scale_factor : 1.0f;
  for (int pos = 0; pos < max_pos; ++pos) {
    for (int i = 0; i < half; ++i) {
      // f32 throughout, in the order of src/layers/rope.rs:26-29
      const float t = (float)pos / scale;
      const float theta = t / powf(base, (float)(2 * i) / (float)head_dim);
      cos_out[(int64_t)pos * half + i] = cosf(theta);
      sin_out[(int64_t)pos * half + i] = sinf(theta);
    }
  }
  return LUC_OK;
}

int luc_rope(luc_ctx* ctx, void* stream, int dtype, void* q, const void* q_bias, void* k,
             const void* k_bias, int64_t row_stride, const float* cos_table,
             const float* sin_table, const int32_t* positions, int num_tokens, int num_q_heads,
             int num_kv_heads, int head_dim) {
  if (int rc = check_common(ctx, dtype, head_dim)) return rc;
  if (int rc = check_heads(num_q_heads, num_kv_heads)) return rc;
  if (int rc = check_rows(num_tokens, row_stride, num_q_heads * head_dim)) return rc;
  if (num_tokens == 0) return LUC_OK;
  if (!q || !k || !cos_table || !sin_table || !positions)
    return fail(LUC_E_INVALID, "null q, k, rope table or positions");
  if (int rc = check_device(ctx)) return rc;
  AppendArgs a;
  a.q = q; a.q_bias = q_bias; a.k = k; a.k_bias = k_bias;
  a.row_stride = row_stride; a.cos_t = cos_table; a.sin_t = sin_table; a.positions = positions;
  a.hq = num_q_heads; a.hkv = num_kv_heads; a.head_dim = head_dim;
  a.flags = kRopeQ | kRopeK;
  return launch_append(ctx, stream, dtype, num_tokens, a);
}

int luc_kv_cache_update(luc_ctx* ctx, void* stream, int dtype, void* k_pool, void* v_pool,
                        const void* k, const void* v, const void* v_bias, int64_t row_stride,
                        const int32_t* block_tables, int table_stride, int num_blocks,
                        const int32_t* positions, int num_tokens, int layer, int num_layers,
                        int num_kv_heads, int head_dim, int block_size) {
  if (int rc = check_common(ctx, dtype, head_dim)) return rc;
  if (num_kv_heads <= 0) return fail(LUC_E_INVALID, "num_kv_heads %d <= 0", num_kv_heads);
  if (int rc = check_rows(num_tokens, row_stride, num_kv_heads * head_dim)) return rc;
  if (int rc = check_cache(k_pool, v_pool, block_tables, table_stride, num_blocks, layer,
                           num_layers, block_size))
    return rc;
  if (num_tokens == 0) return LUC_OK;
  if (!k || !v || !positions) return fail(LUC_E_INVALID, "null k, v or positions");
  if (int rc = check_device(ctx)) return rc;
  AppendArgs a;
  a.k = const_cast<void*>(k); a.v = v; a.v_bias = v_bias; a.row_stride = row_stride;
  a.positions = positions; a.tables = block_tables; a.table_stride = table_stride;
  a.num_blocks = num_blocks;
  a.k_pool = k_pool; a.v_pool = v_pool; a.layer = layer; a.num_layers = num_layers;
  a.hq = num_kv_heads; a.hkv = num_kv_heads; a.head_dim = head_dim;
  a.flags = kWriteKV;
  return launch_append(ctx, stream, dtype, num_tokens, a);
}

int luc_rope_append(luc_ctx* ctx, void* stream, int dtype, void* q, const void* q_bias,
                    void* k, const void* k_bias, const void* v, const void* v_bias,
                    int64_t row_stride, const float* cos_table, const float* sin_table,
                    const int32_t* positions, const int32_t* block_tables, int table_stride,
                    int num_blocks, void* k_pool, void* v_pool, int num_tokens, int layer,
                    int num_layers, int num_q_heads, int num_kv_heads, int head_dim,
                    int block_size) {
  if (int rc = check_common(ctx, dtype, head_dim)) return rc;
  if (int rc = check_heads(num_q_heads, num_kv_heads)) return rc;
  if (int rc = check_rows(num_tokens, row_stride, num_q_heads * head_dim)) return rc;
  if (int rc = check_cache(k_pool, v_pool, block_tables, table_stride, num_blocks, layer,
                           num_layers, block_size))
    return rc;
  if (num_tokens == 0) return LUC_OK;
  if (!q || !k || !v || !cos_table || !sin_table || !positions)
    return fail(LUC_E_INVALID, "null q, k, v, rope table or positions");
  if (int rc = check_device(ctx)) return rc;
  AppendArgs a;
  a.q = q; a.q_bias = q_bias; a.k = k; a.k_bias = k_bias; a.v = v; a.v_bias = v_bias;
  a.row_stride = row_stride; a.cos_t = cos_table; a.sin_t = sin_table; a.positions = positions;
  a.tables = block_tables; a.table_stride = table_stride; a.num_blocks = num_blocks;
  a.k_pool = k_pool; a.v_pool = v_pool;
  a.layer = layer; a.num_layers = num_layers; a.hq = num_q_heads; a.hkv = num_kv_heads;
  a.head_dim = head_dim; a.flags = kRopeQ | kRopeK | kWriteKV;
  return launch_append(ctx, stream, dtype, num_tokens, a);
}

size_t luc_paged_decode_workspace_size(int batch, int num_q_heads, int num_kv_heads,
                                       int head_dim, int max_ctx, int split_tokens) {
  if (batch <= 0 || num_q_heads <= 0 || num_kv_heads <= 0 || max_ctx <= 0) return 0;
  if (head_dim != 64 && head_dim != 128) return 0;
  const int st = split_tokens_for(batch, num_kv_heads, head_dim, max_ctx, split_tokens);
  if (st == 0) return 0;
  return workspace_bytes_for(batch, num_q_heads, num_kv_heads, head_dim, max_ctx, st);
}

int luc_paged_decode(luc_ctx* ctx, void* stream, int dtype, void* out, int64_t out_row_stride,
                     const void* q, int64_t q_row_stride, const void* k_pool, const void* v_pool,
                     const int32_t* block_tables, int table_stride, int num_blocks,
                     const int32_t* positions, int batch, int max_ctx, int layer, int num_layers,
                     int num_q_heads, int num_kv_heads, int head_dim, int block_size,
                     float sm_scale, int split_tokens, void* workspace, size_t workspace_bytes) {
  DecodeLaunch L;
  if (int rc = prepare_decode(ctx, dtype, false, out, out_row_stride, q, q_row_stride, k_pool,
                              v_pool, block_tables, table_stride, num_blocks, positions, batch,
                              max_ctx, layer,
                              num_layers, num_q_heads, num_kv_heads, head_dim, block_size, sm_scale,
                              split_tokens, workspace, workspace_bytes, &L))
    return rc;
  if (batch == 0) return LUC_OK;
  if (int rc = check_device(ctx)) return rc;
  return launch_decode(L, stream);
}

int luc_decode_step(luc_ctx* ctx, void* stream, int dtype, void* qkv, int64_t qkv_row_stride,
                    const void* q_bias, const void* k_bias, const void* v_bias,
                    const float* cos_table, const float* sin_table, void* k_pool, void* v_pool,
                    const int32_t* block_tables, int table_stride, int num_blocks,
                    const int32_t* positions, int batch, int max_ctx, int layer, int num_layers,
                    int num_q_heads, int num_kv_heads, int head_dim, int block_size,
                    float sm_scale, int split_tokens, void* out, int64_t out_row_stride,
                    void* workspace, size_t workspace_bytes) {
  if (!cos_table || !sin_table) return fail(LUC_E_INVALID, "null rope table");
  DecodeLaunch L;
  if (int rc = prepare_decode(ctx, dtype, true, out, out_row_stride, qkv, qkv_row_stride, k_pool,
                              v_pool, block_tables, table_stride, num_blocks, positions, batch,
                              max_ctx, layer,
                              num_layers, num_q_heads, num_kv_heads, head_dim, block_size, sm_scale,
                              split_tokens, workspace, workspace_bytes, &L))
    return rc;
  if (batch == 0) return LUC_OK;
  if (int rc = check_device(ctx)) return rc;
  uint16_t* base = static_cast<uint16_t*>(qkv);
  L.a.q_bias = static_cast<const uint16_t*>(q_bias);
  L.a.k_new = base + (int64_t)num_q_heads * head_dim;
  L.a.k_bias = static_cast<const uint16_t*>(k_bias);
  L.a.v_new = base + (int64_t)(num_q_heads + num_kv_heads) * head_dim;
  L.a.v_bias = static_cast<const uint16_t*>(v_bias);
  L.a.cos_t = cos_table;
  L.a.sin_t = sin_table;
  return launch_decode(L, stream);
}

int luc_decode_step_noalloc(luc_ctx* ctx, void* stream, int dtype, void* qkv,
                            int64_t qkv_row_stride, const void* q_bias, const void* k_bias,
                            const void* v_bias, const float* cos_table, const float* sin_table,
                            void* k_pool, void* v_pool, const int32_t* block_tables,
                            int table_stride, int num_blocks, const int32_t* positions, int batch,
                            int max_ctx,
                            int layer, int num_layers, int num_q_heads, int num_kv_heads,
                            int head_dim, int block_size, float sm_scale, int split_tokens,
                            void* out, int64_t out_row_stride) {
  if (!ctx) return fail(LUC_E_INVALID, "null context");
  if (!ctx->scratch) return fail(LUC_E_WORKSPACE, "the context has no scratch (luc_init failed?)");
  const size_t need = luc_paged_decode_workspace_size(batch, num_q_heads, num_kv_heads, head_dim,
                                                      max_ctx, split_tokens);
  if (need > LUC_SCRATCH_BYTES)
    return fail(LUC_E_WORKSPACE,
                "luc_decode_step_noalloc: these sizes need %zu bytes of split-K workspace, more "
                "than the library's fixed scratch of %u bytes (use luc_decode_step with a "
                "caller workspace)",
                need, (unsigned)LUC_SCRATCH_BYTES);
  // the scratch is this device's copy (ctx->scratch, from hipGetSymbolAddress
  // at luc_init), already zero-filled; every launch leaves its counters at zero
  return luc_decode_step(ctx, stream, dtype, qkv, qkv_row_stride, q_bias, k_bias, v_bias,
                         cos_table, sin_table, k_pool, v_pool, block_tables, table_stride,
                         num_blocks, positions, batch, max_ctx, layer, num_layers, num_q_heads, num_kv_heads,
                         head_dim, block_size, sm_scale, split_tokens, out, out_row_stride,
                         ctx->scratch, LUC_SCRATCH_BYTES);
}

int luc_paged_prefill(luc_ctx* ctx, void* stream, int dtype, void* qkv, int64_t qkv_row_stride,
                      const void* q_bias, const void* k_bias, const void* v_bias,
                      const float* cos_table, const float* sin_table, void* k_pool, void* v_pool,
                      const int32_t* block_tables, int table_stride, int num_blocks,
                      const int32_t* cu_seqlens,
                      const int32_t* start_pos, int batch, int total_rows, int max_ctx, int layer,
                      int num_layers, int num_q_heads, int num_kv_heads, int head_dim,
                      int block_size, float sm_scale, void* out, int64_t out_row_stride) {
  if (int rc = check_common(ctx, dtype, head_dim)) return rc;
  if (int rc = check_heads(num_q_heads, num_kv_heads)) return rc;
  if (int rc = check_cache(k_pool, v_pool, block_tables, table_stride, num_blocks, layer,
                           num_layers, block_size))
    return rc;
  if (batch < 0 || total_rows < 0) return fail(LUC_E_INVALID, "batch %d / total_rows %d < 0", batch, total_rows);
  if (max_ctx <= 0) return fail(LUC_E_INVALID, "max_ctx %d <= 0", max_ctx);
  if (!qkv || !cos_table || !sin_table || !cu_seqlens || !start_pos || !out)
    return fail(LUC_E_INVALID, "null qkv, rope table, cu_seqlens, start_pos or out");
  const int row = num_q_heads * head_dim;
  if (qkv_row_stride < (int64_t)(num_q_heads + 2 * num_kv_heads) * head_dim || out_row_stride < row)
    return fail(LUC_E_INVALID, "qkv/out row stride smaller than a row");
  // q rows are read as 16-byte vectors and outputs written as 8-byte vectors
  if (!aligned(qkv, 16) || qkv_row_stride % 8)
    return fail(LUC_E_INVALID, "qkv must be 16-byte aligned with a row stride that is a multiple of 8");
  if (!aligned(out, 8) || out_row_stride % 4)
    return fail(LUC_E_INVALID, "out must be 8-byte aligned with a row stride that is a multiple of 4");
  if ((int64_t)table_stride * LUC_BLOCK_SIZE < max_ctx)
    return fail(LUC_E_INVALID, "table_stride %d pages cannot hold max_ctx %d", table_stride, max_ctx);
  if (batch == 0 || total_rows == 0) return LUC_OK;
  if (int rc = check_device(ctx)) return rc;
  const int group = num_q_heads / num_kv_heads;
  hipFunction_t fn;
  if (int rc = get_fn(ctx, std::string("luc_prefill_") + dt_name(dtype) + "_d" +
                               std::to_string(head_dim) + "_g" + std::to_string(group),
                      &fn))
    return rc;
  // workgroups: (sequence, kv head, pair of 32-row tiles), one wave per
  // q-head of the group.  A sequence within the bound has at most
  // min(total_rows, max_ctx) rows, so row_tiles tiles of 32 rows
  const int row_tiles = (int)ceil_div(std::min(total_rows, max_ctx), 32);
  const int pairs = (int)ceil_div(row_tiles, 2);
  const int waves = group <= 4 ? 4 : 8;  // one per q-head of the group (paged_prefill.hip)
  const int64_t grid = (int64_t)batch * num_kv_heads * ceil_div(group, waves) * pairs;
  if (grid > INT32_MAX) return fail(LUC_E_INVALID, "batch x kv heads x row tiles too large");

  // q's bias + RoPE runs in the attention kernel, which loads every row's q
  // anyway, when the bias and the rotation tables allow its 16-byte loads
  // (not in the 8-wave head_dim 128 kernels: paged_prefill.hip, QROPE); else
  // the append kernel ropes q as well
  const bool fuse_q = (!q_bias || aligned(q_bias, 16)) && aligned(cos_table, 16) &&
                      aligned(sin_table, 16) && !(head_dim == 128 && group > 4);
  // 1) bias + RoPE of every prompt row's k (and q unless fused) in place,
  //    cache write of the roped k and v + v_bias (models.rs:505-534 for each row)
  uint16_t* base = static_cast<uint16_t*>(qkv);
  AppendArgs a;
  a.q = base; a.q_bias = q_bias; a.k = base + (int64_t)num_q_heads * head_dim; a.k_bias = k_bias;
  a.v = base + (int64_t)(num_q_heads + num_kv_heads) * head_dim; a.v_bias = v_bias;
  a.row_stride = qkv_row_stride; a.cos_t = cos_table; a.sin_t = sin_table;
  a.cu_seqlens = cu_seqlens; a.start_pos = start_pos; a.batch = batch;
  a.tables = block_tables; a.table_stride = table_stride; a.num_blocks = num_blocks;
  a.k_pool = k_pool; a.v_pool = v_pool;
  a.layer = layer; a.num_layers = num_layers; a.hq = num_q_heads; a.hkv = num_kv_heads;
  a.head_dim = head_dim; a.flags = (fuse_q ? 0 : kRopeQ) | kRopeK | kWriteKV;
  if (int rc = launch_append(ctx, stream, dtype, total_rows, a)) return rc;

  // 2) causal attention of every row over the cache (models.rs:536-549 per row)
  PrefillArgs p{};
  p.qkv = qkv; p.qkv_stride = qkv_row_stride; p.k_pool = k_pool; p.v_pool = v_pool;
  p.tables = block_tables; p.table_stride = table_stride; p.cu_seqlens = cu_seqlens;
  p.start_pos = start_pos; p.out = out; p.out_stride = out_row_stride; p.batch = batch;
  p.q_bias = q_bias; p.cos_t = fuse_q ? cos_table : nullptr; p.sin_t = sin_table;
  p.layer = layer; p.num_layers = num_layers; p.hkv = num_kv_heads; p.max_ctx = max_ctx;
  p.pairs = pairs; p.num_blocks = num_blocks; p.qk_scale_log2 = sm_scale * 1.4426950408889634f;
  void* args[] = {&p};
  return launch(fn, dim3((unsigned)grid), dim3(64 * waves), stream, args);
}

// ---- the model loop's small kernels (model_ops.hip) ----

int luc_rmsnorm(luc_ctx* ctx, void* stream, int dtype, void* out, const void* in, const void* weight,
                float eps, int rows, int cols) {
  if (!ctx) return fail(LUC_E_INVALID, "null context");
  if (dtype != LUC_BF16) return fail(LUC_E_UNSUPPORTED, "rmsnorm: bf16 only");
  if (rows < 0 || cols <= 0 || cols % 8) return fail(LUC_E_INVALID, "rows %d / cols %d (a multiple of 8)", rows, cols);
  if (!out || !in || !weight) return fail(LUC_E_INVALID, "null out, in or weight");
  if (!aligned(out, 16) || !aligned(in, 16) || !aligned(weight, 16))
    return fail(LUC_E_INVALID, "rmsnorm operands must be 16-byte aligned");
  if (rows == 0) return LUC_OK;
  if (int rc = check_device(ctx)) return rc;
  hipFunction_t fn;
  if (int rc = get_fn(ctx, "luc_rmsnorm_bf16", &fn)) return rc;
  void* args[] = {&out, &in, &weight, &eps, &cols};
  return launch(fn, dim3(rows), dim3(256), stream, args);
}

namespace {
// The one-row products: `kind` names the kernel family, all with the
// arguments (y, in, w, res, norm weight, eps, outputs, k).  Variant by shape:
// rows of k <= 1024 on four rows per wave when there are at least 4096 of them,
// eight with the norm when there are at least 65536 (the final norm + lm_head:
// 47.0 against 48.0 us at 151936 x 896), else on one row per wave (q/k/v, o:
// four times the waves to fill the chip with); rows of k <= 5120 or <= 8192 on one row per wave (ten or
// sixteen 8-element chunks per lane).  The gate/up silu pairs (`pair`) take
// two rows per output: four rows per wave for k <= 1024, else two (ten or
// sixteen chunks per lane).  4 waves
// per workgroup, one row group per wave.
int gemv_launch(luc_ctx* ctx, void* stream, const char* kind, bool pair, void* y, const void* in,
                const void* w, const void* residual, const void* norm_weight, float eps, int n, int k) {
  if (n < 0) return fail(LUC_E_INVALID, "%s: n %d < 0", kind, n);
  if (k < 8 || k > 8192 || k % 8 != 0)
    return fail(LUC_E_UNSUPPORTED, "%s: k %d (a multiple of 8 in [8, 8192])", kind, k);
  if (!y || !in || !w) return fail(LUC_E_INVALID, "%s: null operand", kind);
  if (!aligned(in, 16) || !aligned(w, 16) || (norm_weight && !aligned(norm_weight, 16)) || !aligned(y, 2) ||
      (residual && !aligned(residual, 2)))
    return fail(LUC_E_INVALID, "%s: the input row, w and the norm weight must be 16-byte aligned", kind);
  if (n == 0) return LUC_OK;
  if (int rc = check_device(ctx)) return rc;
  int outs_per_wave;
  const char* variant;
  if (pair) {
    outs_per_wave = k <= 1024 ? 2 : 1;
    variant = k <= 1024 ? "_bf16_r4c2" : k <= 5120 ? "_bf16_r2c10" : "_bf16_r2c16";
  } else {
    outs_per_wave = k <= 1024 && n >= 4096 ? 4 : 1;
    if (norm_weight && k <= 1024 && n >= 65536) outs_per_wave = 8;
    variant = k > 5120 ? "_bf16_r1c16" : k > 1024 ? "_bf16_r1c10" : outs_per_wave == 8 ? "_bf16_r8c2"
              : outs_per_wave == 4 ? "_bf16_r4c2" : "_bf16_r1c2";
  }
  hipFunction_t fn;
  if (int rc = get_fn(ctx, std::string(kind) + variant, &fn)) return rc;
  const int64_t wgs = ceil_div(n, 4 * outs_per_wave);
  void* args[] = {&y, const_cast<void**>(&in), const_cast<void**>(&w), const_cast<void**>(&residual),
                  const_cast<void**>(&norm_weight), &eps, &n, &k};
  return launch(fn, dim3((unsigned)wgs), dim3(256), stream, args);
}
}  // namespace

int luc_gemv(luc_ctx* ctx, void* stream, int dtype, void* y, const void* x, const void* w,
             const void* residual, int n, int k) {
  if (!ctx) return fail(LUC_E_INVALID, "null context");
  if (dtype != LUC_BF16) return fail(LUC_E_UNSUPPORTED, "gemv: bf16 only");
  return gemv_launch(ctx, stream, "luc_gemv", false, y, x, w, residual, nullptr, 0.0f, n, k);
}

int luc_rmsnorm_gemv(luc_ctx* ctx, void* stream, int dtype, void* y, const void* x,
                     const void* norm_weight, float eps, const void* w, const void* residual, int n,
                     int k) {
  if (!ctx) return fail(LUC_E_INVALID, "null context");
  if (dtype != LUC_BF16) return fail(LUC_E_UNSUPPORTED, "rmsnorm_gemv: bf16 only");
  if (!norm_weight) return fail(LUC_E_INVALID, "rmsnorm_gemv: null norm weight");
  return gemv_launch(ctx, stream, "luc_rmsnorm_gemv", false, y, x, w, residual, norm_weight, eps, n, k);
}

int luc_gate_up_silu(luc_ctx* ctx, void* stream, int dtype, void* act, const void* x,
                     const void* norm_weight, float eps, const void* w, int intermediate, int k) {
  if (!ctx) return fail(LUC_E_INVALID, "null context");
  if (dtype != LUC_BF16) return fail(LUC_E_UNSUPPORTED, "gate_up_silu: bf16 only");
  return gemv_launch(ctx, stream, norm_weight ? "luc_rmsnorm_gate_up_silu" : "luc_gate_up_silu", true,
                     act, x, w, nullptr, norm_weight, eps, intermediate, k);
}

int luc_silu_mul(luc_ctx* ctx, void* stream, int dtype, void* gate_up, int rows, int intermediate) {
  if (!ctx) return fail(LUC_E_INVALID, "null context");
  if (dtype != LUC_BF16) return fail(LUC_E_UNSUPPORTED, "silu_mul: bf16 only");
  if (rows < 0 || intermediate <= 0 || intermediate % 8)
    return fail(LUC_E_INVALID, "rows %d / intermediate %d (a multiple of 8)", rows, intermediate);
  if (!gate_up || !aligned(gate_up, 16)) return fail(LUC_E_INVALID, "gate_up null or not 16-byte aligned");
  if (rows == 0) return LUC_OK;
  if (int rc = check_device(ctx)) return rc;
  hipFunction_t fn;
  if (int rc = get_fn(ctx, "luc_silu_mul_bf16", &fn)) return rc;
  const int64_t grid = ceil_div((int64_t)rows * (intermediate / 8), 256);
  if (grid > INT32_MAX) return fail(LUC_E_INVALID, "too many rows");
  void* args[] = {&gate_up, &rows, &intermediate};
  return launch(fn, dim3((unsigned)grid), dim3(256), stream, args);
}

int luc_embedding(luc_ctx* ctx, void* stream, int dtype, void* out, const void* table,
                  const uint32_t* ids, int num_tokens, int vocab, int hidden) {
  if (!ctx) return fail(LUC_E_INVALID, "null context");
  if (dtype != LUC_BF16) return fail(LUC_E_UNSUPPORTED, "embedding: bf16 only");
  if (num_tokens < 0 || vocab <= 0 || hidden <= 0 || hidden % 8)
    return fail(LUC_E_INVALID, "num_tokens %d / vocab %d / hidden %d (a multiple of 8)", num_tokens,
                vocab, hidden);
  if (!out || !table || !ids) return fail(LUC_E_INVALID, "null out, table or ids");
  if (!aligned(out, 16) || !aligned(table, 16)) return fail(LUC_E_INVALID, "out/table must be 16-byte aligned");
  if (num_tokens == 0) return LUC_OK;
  if (int rc = check_device(ctx)) return rc;
  hipFunction_t fn;
  if (int rc = get_fn(ctx, "luc_embedding_bf16", &fn)) return rc;
  void* args[] = {&out, &table, &ids, &vocab, &hidden};
  return launch(fn, dim3(num_tokens), dim3(128), stream, args);
}

int luc_argmax(luc_ctx* ctx, void* stream, int dtype, const void* logits, int n, uint32_t* out_idx) {
  if (!ctx) return fail(LUC_E_INVALID, "null context");
  if (dtype != LUC_BF16) return fail(LUC_E_UNSUPPORTED, "argmax: bf16 only");
  if (n <= 0) return fail(LUC_E_INVALID, "n %d <= 0", n);
  if (!logits || !out_idx) return fail(LUC_E_INVALID, "null logits or out_idx");
  if (int rc = check_device(ctx)) return rc;
  hipFunction_t fn;
  if (int rc = get_fn(ctx, "luc_argmax_bf16", &fn)) return rc;
  void* args[] = {&logits, &n, &out_idx};
  return launch(fn, dim3(1), dim3(1024), stream, args);
}

int luc_sort_and_sample(luc_ctx* ctx, void* stream, int dtype, const void* logits, int vocab,
                        float top_p, int top_k, float rand_val, void* sort_buffer,
                        size_t sort_buffer_bytes, uint32_t* out_idx) {
  if (!ctx) return fail(LUC_E_INVALID, "null context");
  if (dtype != LUC_BF16) return fail(LUC_E_UNSUPPORTED, "sort_and_sample: bf16 logits only");
  // the fused sort kernels exist for 32..1024 candidates (kernels.rs:403-493)
  if (top_k < 32 || top_k > 1024 || (top_k & (top_k - 1)))
    return fail(LUC_E_UNSUPPORTED, "Unsupported candidate size: %d (a power of two in [32, 1024])",
                top_k);
  // every one of the 32 filter partitions holds at least one logit; at most
  // 16 per thread of a 1024-thread partition workgroup
  if (vocab < 32 || vocab > 32 * 16384)
    return fail(LUC_E_INVALID, "vocab %d outside [32, %d]", vocab, 32 * 16384);
  if (!logits || !sort_buffer || !out_idx) return fail(LUC_E_INVALID, "null logits, sort_buffer or out_idx");
  if (!aligned(sort_buffer, 8)) return fail(LUC_E_INVALID, "sort_buffer must be 8-byte aligned");
  if (sort_buffer_bytes < (size_t)top_k * 8)
    return fail(LUC_E_WORKSPACE, "sort_buffer holds %zu bytes, %d candidates need %d", sort_buffer_bytes,
                top_k, top_k * 8);
  if (int rc = check_device(ctx)) return rc;
  const int per_part = (vocab + 31) / 32;  // the largest partition
  int npl = 1;
  while (npl * 1024 < per_part) npl *= 2;
  hipFunction_t filter, sample;
  if (int rc = get_fn(ctx, "luc_topk_filter_bf16_n" + std::to_string(npl), &filter)) return rc;
  if (int rc = get_fn(ctx, "luc_top_p_sample_" + std::to_string(top_k), &sample)) return rc;
  int kpp = top_k / 32;
  void* fargs[] = {&logits, &vocab, &kpp, &sort_buffer};
  if (int rc = launch(filter, dim3(32), dim3(1024), stream, fargs)) return rc;
  void* sargs[] = {&sort_buffer, &top_p, &rand_val, &out_idx};
  return launch(sample, dim3(1), dim3(top_k < 64 ? 64 : top_k), stream, sargs);
}

// ---- measurement kernels (probe_gather.hip) ----

int luc_gather_floor(luc_ctx* ctx, void* stream, const void* k_pool, const void* v_pool,
                     const int32_t* block_tables, int table_stride, int num_blocks,
                     const int32_t* positions, int batch, int max_ctx, int layer, int num_layers,
                     int num_kv_heads, int head_dim, uint32_t* sink) {
  if (int rc = check_common(ctx, LUC_BF16, head_dim)) return rc;
  if (num_kv_heads <= 0) return fail(LUC_E_INVALID, "num_kv_heads %d <= 0", num_kv_heads);
  if (int rc = check_cache(k_pool, v_pool, block_tables, table_stride, num_blocks, layer,
                           num_layers, LUC_BLOCK_SIZE))
    return rc;
  if (batch < 0 || max_ctx <= 0) return fail(LUC_E_INVALID, "batch %d / max_ctx %d", batch, max_ctx);
  if (!positions || !sink) return fail(LUC_E_INVALID, "null positions or sink");
  if ((int64_t)table_stride * LUC_BLOCK_SIZE < max_ctx)
    return fail(LUC_E_INVALID, "table_stride %d pages cannot hold max_ctx %d", table_stride, max_ctx);
  if (batch == 0) return LUC_OK;
  if (int rc = check_device(ctx)) return rc;
  hipFunction_t fn;
  if (int rc = get_fn(ctx, "luc_gather_floor_d" + std::to_string(head_dim), &fn)) return rc;
  // the single-tile decode kernel's split: 8 waves, one 8 KB K tile each
  const int split = kT1Waves * decode_tile(head_dim);
  const int64_t grid = ceil_div(max_ctx, split) * batch * num_kv_heads;
  if (grid > INT32_MAX) return fail(LUC_E_INVALID, "grid too large");
  struct {
    const void* k;
    const void* v;
    const int32_t* tables;
    int64_t table_stride;
    const int32_t* positions;
    int32_t batch, layer, num_layers, hkv, max_ctx, num_blocks;
    uint32_t* sink;
  } a{k_pool, v_pool, block_tables, table_stride, positions, batch, layer, num_layers,
      num_kv_heads, max_ctx, num_blocks, sink};
  void* args[] = {&a};
  return launch(fn, dim3((unsigned)grid), dim3(kT1Waves * 64), stream, args);
}

int luc_stream_read(luc_ctx* ctx, void* stream, const void* src, size_t bytes, uint32_t* sink) {
  if (!ctx) return fail(LUC_E_INVALID, "null context");
  if (!src || !sink) return fail(LUC_E_INVALID, "null src or sink");
  if (bytes % 16 || !aligned(src, 16)) return fail(LUC_E_INVALID, "src / bytes must be 16-byte multiples");
  if (bytes == 0) return LUC_OK;
  if (int rc = check_device(ctx)) return rc;
  hipFunction_t fn;
  if (int rc = get_fn(ctx, "luc_stream_read", &fn)) return rc;
  int64_t n16 = (int64_t)(bytes / 16);
  const int64_t grid = std::min<int64_t>(ceil_div(n16, 256), 2048);
  void* args[] = {&src, &n16, &sink};
  return launch(fn, dim3((unsigned)grid), dim3(256), stream, args);
}

}  // extern "C"
