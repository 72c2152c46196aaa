// Multi-sequence page allocator for the paged K/V pool (host code, no GPU).
//
// Generalises the reference's single-sequence KVCache bookkeeping
// (src/layers/kv_cache.rs:12-104 free list, :106-122 prepare_for_step) to a
// table of sequences:
//   * one LIFO free list over the pool's pages, seeded in reverse so that a
//     fresh allocator hands out pages 0, 1, 2, ... (kv_cache.rs:73-76);
//   * per-sequence rows of the block table, grown by as many pages as a
//     request needs (prepare_for_step adds at most one page per call);
//   * all-or-nothing reservations for one sequence or a batch (the reference
//     panics on an empty free list; here the call fails with LUC_E_NOMEM and
//     changes nothing);
//   * release returns a sequence's pages, last page first, so a sequence that
//     is released and reserved again with nothing in between gets the same
//     pages in the same order.
// Not thread-safe: calls on one allocator must be serialised by the caller, as
// the reference's &mut self methods are.
#include <cstdint>
#include <vector>

#include "luc_attn.h"

namespace luc_internal {
int fail(int code, const char* fmt, ...);
}
using luc_internal::fail;

struct luc_blocks {
  int num_blocks = 0;
  int max_seqs = 0;
  int max_pages = 0;                        // per sequence
  std::vector<int32_t> free_list;           // pop from the back
  std::vector<std::vector<int32_t>> pages;  // [max_seqs] held pages, in table order
};

namespace {

int pages_for(int64_t tokens) { return (int)((tokens + LUC_BLOCK_SIZE - 1) / LUC_BLOCK_SIZE); }

int check_seq(const luc_blocks* bm, int seq) {
  if (!bm) return fail(LUC_E_INVALID, "null block allocator");
  if (seq < 0 || seq >= bm->max_seqs)
    return fail(LUC_E_INVALID, "sequence %d outside [0, %d)", seq, bm->max_seqs);
  return LUC_OK;
}

}  // namespace

extern "C" {

int luc_blocks_create(int num_blocks, int max_seqs, int max_blocks_per_seq, luc_blocks** out) {
  if (!out) return fail(LUC_E_INVALID, "null output pointer");
  *out = nullptr;
  if (num_blocks <= 0 || max_seqs <= 0 || max_blocks_per_seq <= 0)
    return fail(LUC_E_INVALID, "num_blocks %d, max_seqs %d, max_blocks_per_seq %d must be positive",
                num_blocks, max_seqs, max_blocks_per_seq);
  auto* bm = new luc_blocks;
  bm->num_blocks = num_blocks;
  bm->max_seqs = max_seqs;
  bm->max_pages = max_blocks_per_seq;
  bm->free_list.reserve(num_blocks);
  for (int i = num_blocks - 1; i >= 0; --i) bm->free_list.push_back(i);
  bm->pages.resize(max_seqs);
  *out = bm;
  return LUC_OK;
}

void luc_blocks_destroy(luc_blocks* bm) { delete bm; }

int luc_blocks_reserve_batch(luc_blocks* bm, int n, const int32_t* seqs, const int32_t* num_tokens) {
  if (n < 0 || (n > 0 && (!seqs || !num_tokens))) return fail(LUC_E_INVALID, "bad batch arguments");
  // validate everything and count the pages first: nothing changes on failure
  int64_t need = 0;
  std::vector<int> extra(n);
  for (int i = 0; i < n; ++i) {
    if (int rc = check_seq(bm, seqs[i])) return rc;
    if (num_tokens[i] < 0) return fail(LUC_E_INVALID, "negative token count %d", num_tokens[i]);
    for (int j = 0; j < i; ++j)
      if (seqs[j] == seqs[i]) return fail(LUC_E_INVALID, "sequence %d listed twice", seqs[i]);
    const int want = pages_for(num_tokens[i]);
    if (want > bm->max_pages)
      return fail(LUC_E_INVALID, "sequence %d: %d tokens need %d pages, a table row holds %d", seqs[i],
                  num_tokens[i], want, bm->max_pages);
    const int have = (int)bm->pages[seqs[i]].size();
    extra[i] = want > have ? want - have : 0;
    need += extra[i];
  }
  if (need > (int64_t)bm->free_list.size())
    return fail(LUC_E_NOMEM, "KV pool out of pages: %lld needed, %zu free", (long long)need,
                bm->free_list.size());
  for (int i = 0; i < n; ++i) {
    auto& row = bm->pages[seqs[i]];
    for (int k = 0; k < extra[i]; ++k) {
      row.push_back(bm->free_list.back());
      bm->free_list.pop_back();
    }
  }
  return LUC_OK;
}

int luc_blocks_reserve(luc_blocks* bm, int seq, int num_tokens) {
  const int32_t s = seq, t = num_tokens;
  return luc_blocks_reserve_batch(bm, 1, &s, &t);
}

int luc_blocks_release(luc_blocks* bm, int seq) {
  if (int rc = check_seq(bm, seq)) return rc;
  auto& row = bm->pages[seq];
  for (auto it = row.rbegin(); it != row.rend(); ++it) bm->free_list.push_back(*it);
  row.clear();
  return LUC_OK;
}

int luc_blocks_num_free(const luc_blocks* bm) {
  if (!bm) return fail(LUC_E_INVALID, "null block allocator");
  return (int)bm->free_list.size();
}

int luc_blocks_num_pages(const luc_blocks* bm, int seq) {
  if (int rc = check_seq(bm, seq)) return rc;
  return (int)bm->pages[seq].size();
}

int luc_blocks_table(const luc_blocks* bm, int first_seq, int n, int32_t* table, int stride) {
  if (!bm || !table) return fail(LUC_E_INVALID, "null argument");
  if (first_seq < 0 || n < 0 || first_seq + n > bm->max_seqs)
    return fail(LUC_E_INVALID, "rows [%d, %d) outside [0, %d)", first_seq, first_seq + n, bm->max_seqs);
  if (stride < bm->max_pages)
    return fail(LUC_E_INVALID, "row stride %d below max_blocks_per_seq %d", stride, bm->max_pages);
  for (int i = 0; i < n; ++i) {
    const auto& row = bm->pages[first_seq + i];
    int32_t* dst = table + (int64_t)i * stride;
    int k = 0;
    for (; k < (int)row.size(); ++k) dst[k] = row[k];
    for (; k < stride; ++k) dst[k] = 0;  // the reference's table is zero-initialised
  }
  return LUC_OK;
}

}  // extern "C"
