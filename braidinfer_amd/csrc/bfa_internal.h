// Launchers shared between translation units of the library.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace bfa {

struct AppendArgs;

// Normalised QKV operand pre-pass (norm.hip): out[rows, hidden] (bf16 or fp16)
//   mixed:  round_out(round_bf16(x / rms) * w)
//   else:   round_out((x / rms) * w)            rms = sqrt(sum(x^2)/hidden + eps)
int launch_qkv_operand(const void* x, int x_dtype, int64_t rows, int64_t hidden, int64_t x_stride,
                       const void* w, int w_dtype, bool mixed, void* out, int out_dtype,
                       float eps, hipStream_t s);

// The row statistic alone (norm.hip): out[r] = 1 / sqrt(sum(x[r]^2)/hidden + eps),
// fp32, the same value the operand pre-pass multiplies by.
int launch_row_scale(const void* x, int x_dtype, int64_t rows, int64_t hidden, int64_t x_stride,
                     float* out, float eps, hipStream_t s);

// Paged-KV append addressing (kv_append.hip): checks the cache, page-table and
// position arguments of bfa_append_paged_kv (dtypes, page size, geometry; not
// the pointers, which the callers check once they know there is work) and fills
// `out` with them (k/v fields left empty); returns BFA_OK or an error code.
int fill_append_args(const char* what, void* layer_cache, int cache_dtype, int64_t num_pages,
                     int64_t cache_page_slots, int64_t stride_page, int64_t stride_kv,
                     int64_t stride_head, int64_t stride_slot, const void* kv_indices,
                     int kv_indices_dtype, int64_t num_indices, const int32_t* kv_indptr,
                     const void* batch_indices, int batch_indices_dtype, int64_t num_seqs,
                     const void* positions, int positions_dtype, int64_t page_size, int32_t* status,
                     AppendArgs* out);

// slot_off[t] = element offset of token t's cache slot (page * stride_page +
// slot * stride_slot), or -1 when the append rule skips it (status flagged).
void launch_kv_slots(const AppendArgs& a, int64_t tokens, int64_t* slot_off, hipStream_t s);

}  // namespace bfa
