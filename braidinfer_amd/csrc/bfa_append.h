// Paged-KV append addressing shared by the append kernels (kv_append.hip) and
// the QKV epilogues that write K and V into the cache themselves (qkv.hip).
//
// Reference rule (braidinfer/kernels/kv_cache_utils.py:9-78), per token t:
//   pos = positions[t]; off = pos // page_size; slot = pos % page_size (Python
//   floor division); off >= len(kv_indices) skips the token; page =
//   kv_indices[off] (a negative off or page id wraps like a torch index, below
//   -len raises); K goes to cache[page, 0, head, slot], V to cache[page, 1, ...].
// The batched form gives each token a sequence and each sequence a slice of one
// CSR page table (kv_indptr).
#pragma once

#include "bfa_device.h"

namespace bfa {

struct AppendArgs {
  const void* k;
  const void* v;
  int64_t k_st, k_sh, v_st, v_sh;  // token / head strides of k and v (elements)
  uint32_t heads, head_dim;
  void* cache;
  int64_t c_sp, c_skv, c_sh, c_ss;  // page, K|V, head and slot strides (elements)
  int64_t num_pages, cache_slots;   // pages in the cache, slots per cache page
  int64_t page_size;                // divisor mapping a position to (page entry, slot)
  const void* indices;
  int idx_is_i64;
  int64_t num_indices;
  const int32_t* indptr;      // batched form: sequence s owns indices[indptr[s], indptr[s+1])
  const void* batch;          // batched form: sequence of each token
  int batch_is_i64;
  int64_t num_seqs;
  const void* positions;
  int pos_is_i64;
  FastDiv chunks_per_head;   // head_dim / 8 (vector kernel) or head_dim (scalar kernel)
  FastDiv chunks_per_kv;     // heads * chunks_per_head
  int* status;
};

// Destination (page, slot) of token t; returns 0, or the status bit saying why
// the token is not written (BFA_STATUS_APPEND_SKIPPED / BFA_STATUS_INDEX_OOB).
__device__ __forceinline__ int append_target_code(const AppendArgs& a, int64_t t, int64_t& page,
                                                  int64_t& slot) {
  const int64_t pos = a.pos_is_i64 ? static_cast<const int64_t*>(a.positions)[t]
                                   : static_cast<const int32_t*>(a.positions)[t];
  int64_t off = pos / a.page_size, s = pos - off * a.page_size;
  if (s < 0) {  // C truncates toward zero; Python floors
    s += a.page_size;
    off -= 1;
  }
  int bad = 0;
  int64_t first = 0, len = a.num_indices;  // this token's page table
  if (a.indptr) {
    const int64_t sq = a.batch_is_i64 ? static_cast<const int64_t*>(a.batch)[t]
                                      : static_cast<const int32_t*>(a.batch)[t];
    if (sq < 0 || sq >= a.num_seqs) return BFA_STATUS_INDEX_OOB;
    first = a.indptr[sq];
    len = a.indptr[sq + 1] - first;
  }
  if (off >= len) {
    bad = BFA_STATUS_APPEND_SKIPPED;
  } else if (off < -len) {
    bad = BFA_STATUS_INDEX_OOB;
  } else {
    if (off < 0) off += len;
    off += first;
    // a batched table slice must lie inside kv_indices (a malformed kv_indptr is an index error)
    int64_t p = (off >= 0 && off < a.num_indices)
                    ? (a.idx_is_i64 ? static_cast<const int64_t*>(a.indices)[off]
                                    : static_cast<const int32_t*>(a.indices)[off])
                    : a.num_pages;
    if (p < -a.num_pages || p >= a.num_pages || s >= a.cache_slots) {
      bad = BFA_STATUS_INDEX_OOB;
    } else {
      page = p < 0 ? p + a.num_pages : p;
      slot = s;
    }
  }
  return bad;
}

// As append_target_code, with the reason flagged by the first lane of each wave
// that resolves t (every lane of the wave resolves the same token).
__device__ __forceinline__ bool append_target(const AppendArgs& a, int64_t t, int64_t& page,
                                              int64_t& slot) {
  const int bad = append_target_code(a, t, page, slot);
  if (bad && (threadIdx.x & 63) == 0) flag_status(a.status, bad);
  return bad == 0;
}

}  // namespace bfa
