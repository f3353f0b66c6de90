// Paged KV-cache append on gfx950: the drop-in for append_to_paged_kv_cache_custom
// (braidinfer/kernels/kv_cache_utils.py:9-78), which the page manager calls for
// every layer of every prefill and decode step (engine/page_manager.py:159-218,
// 313-353).
//
// Reference semantics, per token t in order:
//   pos = positions[t]; off = pos // page_size; slot = pos % page_size (Python
//   floor division, so a negative position lands in a negative page offset)
//   off >= len(kv_indices): the token is skipped (the reference prints an error)
//   page = kv_indices[off] (torch indexing: -len <= off < 0 wraps, below raises)
//   cache[page, 0, <head>, slot, :] = k[t]; cache[page, 1, ...] = v[t]
//   (HND [pages, 2, heads, page, D]; NHD [pages, 2, page, heads, D]; a page id
//   in [-num_pages, 0) wraps like a torch index, outside raises IndexError)
// Here the layout is a permutation of four cache strides (page, K|V, head,
// slot), so one kernel serves both.  The batched form (no counterpart function
// in the reference, whose page manager calls the per-sequence function once per
// sequence, engine/page_manager.py:180-210) gives each token a sequence id and
// each sequence a slice of one CSR page table (kv_indptr, as
// build_paged_kv_indices makes it), so a whole decode batch is one launch.
// A workgroup owns one token: it resolves
// the destination once, then copies the token's 2 x heads x D elements in
// 16-byte chunks -- a raw byte copy when k/v and the cache share a dtype (bit
// exact), else a round-to-nearest-even conversion, which is what the tensor
// assignment does.  Index errors set BFA_STATUS_INDEX_OOB; a skipped token sets
// BFA_STATUS_APPEND_SKIPPED.  Distinct tokens are assumed to target distinct
// slots, as every reference caller builds them (positions are an arange and a
// page table holds distinct pages); for two tokens on one slot the reference
// keeps the later token, and which one this kernel keeps is unspecified.
#include "bfa_append.h"
#include "bfa_device.h"
#include "bfa_host.h"
#include "bfa_internal.h"

namespace bfa {

// Copies 8 consecutive elements; a raw 16- or 32-byte copy for equal dtypes.
template <int DTS, int DTD>
__device__ __forceinline__ void copy8(const void* src, void* dst) {
  if constexpr (DTS == DTD) {
    const uint4* s = static_cast<const uint4*>(src);
    uint4* d = static_cast<uint4*>(dst);
    d[0] = load16_nt(s);
    if constexpr (DTS == BFA_DTYPE_F32) d[1] = load16_nt(s + 1);
  } else {
    float x[8];
    load8_nt<DTS>(src, x);
    store8<DTD>(dst, x);
  }
}

template <int DTS, int DTD>
__global__ __launch_bounds__(256) void kv_append_vec_kernel(AppendArgs a) {
  using TS = typename Elem<DTS>::T;
  using TD = typename Elem<DTD>::T;
  const int64_t t = blockIdx.x;
  const uint32_t items = 2u * a.chunks_per_kv.d;
  int64_t page = 0, slot = 0;
  if (!append_target(a, t, page, slot)) return;  // uniform over the workgroup
  TD* base = static_cast<TD*>(a.cache) + page * a.c_sp + slot * a.c_ss;
  for (uint32_t i = threadIdx.x; i < items; i += 256) {
    const uint32_t kv = a.chunks_per_kv.div(i);
    const uint32_t r = i - kv * a.chunks_per_kv.d;
    const uint32_t h = a.chunks_per_head.div(r);
    const uint32_t c = (r - h * a.chunks_per_head.d) * 8u;
    const TS* src = kv == 0 ? static_cast<const TS*>(a.k) + t * a.k_st + h * a.k_sh
                            : static_cast<const TS*>(a.v) + t * a.v_st + h * a.v_sh;
    copy8<DTS, DTD>(src + c, base + kv * a.c_skv + h * a.c_sh + c);
  }
}

// Equal 16-bit dtypes with at most 4 x 64 chunks per token: four tokens per
// workgroup, 64 lanes per token, each lane's source chunks requested before the
// destination is resolved.
template <int DT>
__global__ __launch_bounds__(256) void kv_append_group_kernel(AppendArgs a, int64_t tokens) {
  using T = typename Elem<DT>::T;
  const int64_t t = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (t >= tokens) return;
  const uint32_t lane = threadIdx.x & 63;
  const uint32_t items = 2u * a.chunks_per_kv.d;
  uint4 buf[4];
  int64_t dst_off[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const uint32_t i = lane + c * 64u;
    dst_off[c] = -1;
    if (i < items) {
      const uint32_t kv = a.chunks_per_kv.div(i);
      const uint32_t r = i - kv * a.chunks_per_kv.d;
      const uint32_t h = a.chunks_per_head.div(r);
      const uint32_t e = (r - h * a.chunks_per_head.d) * 8u;
      const T* src = kv == 0 ? static_cast<const T*>(a.k) + t * a.k_st + h * a.k_sh
                             : static_cast<const T*>(a.v) + t * a.v_st + h * a.v_sh;
      buf[c] = load16_nt(src + e);
      dst_off[c] = kv * a.c_skv + h * a.c_sh + e;
    }
  }
  int64_t page = 0, slot = 0;
  if (!append_target(a, t, page, slot)) return;  // uniform over the token's 64 lanes
  T* base = static_cast<T*>(a.cache) + page * a.c_sp + slot * a.c_ss;
#pragma unroll
  for (int c = 0; c < 4; ++c)
    if (dst_off[c] >= 0) *reinterpret_cast<uint4*>(base + dst_off[c]) = buf[c];
}

// Any strides and head_dim: one element per lane.
template <int DTS, int DTD>
__global__ __launch_bounds__(256) void kv_append_scalar_kernel(AppendArgs a) {
  using TS = typename Elem<DTS>::T;
  using TD = typename Elem<DTD>::T;
  const int64_t t = blockIdx.x;
  int64_t page = 0, slot = 0;
  if (!append_target(a, t, page, slot)) return;
  TD* base = static_cast<TD*>(a.cache) + page * a.c_sp + slot * a.c_ss;
  const uint32_t items = 2u * a.chunks_per_kv.d;
  for (uint32_t i = threadIdx.x; i < items; i += 256) {
    const uint32_t kv = a.chunks_per_kv.div(i);
    const uint32_t r = i - kv * a.chunks_per_kv.d;
    const uint32_t h = a.chunks_per_head.div(r);
    const uint32_t c = r - h * a.chunks_per_head.d;
    const TS* src = kv == 0 ? static_cast<const TS*>(a.k) + t * a.k_st + h * a.k_sh
                            : static_cast<const TS*>(a.v) + t * a.v_st + h * a.v_sh;
    TD* dst = base + kv * a.c_skv + h * a.c_sh + c;
    if constexpr (DTS == DTD) {
      *dst = src[c];
    } else {
      *dst = Elem<DTD>::from_f32(Elem<DTS>::to_f32(src[c]));
    }
  }
}

// Cache slot of every token for the QKV epilogues that append K and V
// themselves: slot_off[t] = page * c_sp + slot * c_ss (elements), or -1 when the
// token is not written (the reason is flagged in the status word).
__global__ __launch_bounds__(256) void kv_slot_kernel(AppendArgs a, int64_t tokens, int64_t* slot_off) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (t >= tokens) return;
  int64_t page = 0, slot = 0;
  const int bad = append_target_code(a, t, page, slot);
  if (bad) flag_status(a.status, bad);
  slot_off[t] = bad ? -1 : page * a.c_sp + slot * a.c_ss;
}

void launch_kv_slots(const AppendArgs& a, int64_t tokens, int64_t* slot_off, hipStream_t s) {
  hipLaunchKernelGGL(kv_slot_kernel, dim3(static_cast<unsigned>(cdiv(tokens, 256))), dim3(256), 0, s, a,
                     tokens, slot_off);
}

int fill_append_args(const char* what, void* layer_cache, int cache_dtype, int64_t num_pages,
                     int64_t cache_page_slots, int64_t stride_page, int64_t stride_kv,
                     int64_t stride_head, int64_t stride_slot, const void* kv_indices,
                     int kv_indices_dtype, int64_t num_indices, const int32_t* kv_indptr,
                     const void* batch_indices, int batch_indices_dtype, int64_t num_seqs,
                     const void* positions, int positions_dtype, int64_t page_size, int32_t* status,
                     AppendArgs* out) {
  BFA_REQUIRE(is_float_dtype(cache_dtype), "%s: bad cache dtype", what);
  BFA_REQUIRE(kv_indices_dtype == BFA_DTYPE_I32 || kv_indices_dtype == BFA_DTYPE_I64,
              "%s: kv_indices must be int32/int64", what);
  BFA_REQUIRE(positions_dtype == BFA_DTYPE_I32 || positions_dtype == BFA_DTYPE_I64,
              "%s: positions must be int32/int64", what);
  BFA_REQUIRE(page_size > 0, "%s: page_size must be positive", what);
  BFA_REQUIRE(num_pages >= 0 && cache_page_slots >= 0 && num_indices >= 0, "%s: bad geometry", what);
  if (kv_indptr) {
    BFA_REQUIRE(batch_indices && num_seqs >= 0, "%s: batched append needs batch_indices", what);
    BFA_REQUIRE(batch_indices_dtype == BFA_DTYPE_I32 || batch_indices_dtype == BFA_DTYPE_I64,
                "%s: batch_indices must be int32/int64", what);
  }
  AppendArgs a{};
  a.cache = layer_cache;
  a.c_sp = stride_page; a.c_skv = stride_kv; a.c_sh = stride_head; a.c_ss = stride_slot;
  a.num_pages = num_pages;
  a.cache_slots = cache_page_slots;
  a.page_size = page_size;
  a.indices = kv_indices;
  a.idx_is_i64 = kv_indices_dtype == BFA_DTYPE_I64;
  a.num_indices = num_indices;
  a.indptr = kv_indptr;
  a.batch = batch_indices;
  a.batch_is_i64 = batch_indices_dtype == BFA_DTYPE_I64;
  a.num_seqs = num_seqs;
  a.positions = positions;
  a.pos_is_i64 = positions_dtype == BFA_DTYPE_I64;
  a.status = status;
  *out = a;
  return BFA_OK;
}

template <int DTS, int DTD>
static void launch_append(AppendArgs a, int64_t tokens, bool vec, hipStream_t s) {
  a.chunks_per_head = FastDiv(vec ? a.head_dim / 8 : a.head_dim);
  a.chunks_per_kv = FastDiv(a.heads * a.chunks_per_head.d);
  if constexpr (DTS == DTD && DTS != BFA_DTYPE_F32) {
    if (vec && 2 * a.chunks_per_kv.d <= 256) {
      hipLaunchKernelGGL((kv_append_group_kernel<DTS>), dim3(static_cast<unsigned>(cdiv(tokens, 4))),
                         dim3(256), 0, s, a, tokens);
      return;
    }
  }
  if (vec) {
    hipLaunchKernelGGL((kv_append_vec_kernel<DTS, DTD>), dim3(static_cast<unsigned>(tokens)), dim3(256), 0, s, a);
  } else {
    hipLaunchKernelGGL((kv_append_scalar_kernel<DTS, DTD>), dim3(static_cast<unsigned>(tokens)), dim3(256), 0, s, a);
  }
}

template <int DTS>
static void launch_append_src(int cache_dtype, const AppendArgs& a, int64_t tokens, bool vec, hipStream_t s) {
  switch (cache_dtype) {
    case BFA_DTYPE_BF16: launch_append<DTS, BFA_DTYPE_BF16>(a, tokens, vec, s); break;
    case BFA_DTYPE_F16: launch_append<DTS, BFA_DTYPE_F16>(a, tokens, vec, s); break;
    default: launch_append<DTS, BFA_DTYPE_F32>(a, tokens, vec, s); break;
  }
}

}  // namespace bfa

using namespace bfa;

extern "C" int bfa_append_paged_kv(const void* k, const void* v, int kv_dtype, int64_t num_tokens,
                                   int64_t num_kv_heads, int64_t head_dim, int64_t k_stride_token,
                                   int64_t k_stride_head, int64_t v_stride_token,
                                   int64_t v_stride_head, void* layer_cache, int cache_dtype,
                                   int64_t num_pages, int64_t cache_page_slots,
                                   int64_t stride_page, int64_t stride_kv, int64_t stride_head,
                                   int64_t stride_slot, const void* kv_indices,
                                   int kv_indices_dtype, int64_t num_indices,
                                   const int32_t* kv_indptr, const void* batch_indices,
                                   int batch_indices_dtype, int64_t num_seqs,
                                   const void* positions, int positions_dtype, int64_t page_size,
                                   int32_t* status, void* stream) {
  const char* what = "bfa_append_paged_kv";
  BFA_REQUIRE(is_float_dtype(kv_dtype), "%s: bad dtype", what);
  BFA_REQUIRE(num_tokens >= 0 && num_kv_heads >= 0 && head_dim >= 0, "%s: bad geometry", what);
  BFA_REQUIRE(num_tokens < (int64_t{1} << 31), "%s: too many tokens", what);
  BFA_REQUIRE(num_kv_heads * head_dim < (int64_t{1} << 30), "%s: head block too large", what);
  AppendArgs a{};
  int rc = fill_append_args(what, layer_cache, cache_dtype, num_pages, cache_page_slots, stride_page,
                            stride_kv, stride_head, stride_slot, kv_indices, kv_indices_dtype,
                            num_indices, kv_indptr, batch_indices, batch_indices_dtype, num_seqs,
                            positions, positions_dtype, page_size, status, &a);
  if (rc != BFA_OK) return rc;
  if (num_tokens == 0 || num_kv_heads == 0 || head_dim == 0) return BFA_OK;
  BFA_REQUIRE(k && v && layer_cache && positions, "%s: null pointer", what);
  BFA_REQUIRE(num_indices == 0 || kv_indices, "%s: null kv_indices", what);
  a.k = k; a.v = v;
  a.k_st = k_stride_token; a.k_sh = k_stride_head;
  a.v_st = v_stride_token; a.v_sh = v_stride_head;
  a.heads = static_cast<uint32_t>(num_kv_heads);
  a.head_dim = static_cast<uint32_t>(head_dim);
  const auto m8 = [](int64_t x) { return x % 8 == 0; };
  const bool vec = head_dim % 8 == 0 && m8(k_stride_token) && m8(k_stride_head) &&
                   m8(v_stride_token) && m8(v_stride_head) && m8(stride_page) && m8(stride_kv) &&
                   m8(stride_head) && m8(stride_slot) && aligned16(k) && aligned16(v) &&
                   aligned16(layer_cache);
  const hipStream_t s = as_stream(stream);
  switch (kv_dtype) {
    case BFA_DTYPE_BF16: launch_append_src<BFA_DTYPE_BF16>(cache_dtype, a, num_tokens, vec, s); break;
    case BFA_DTYPE_F16: launch_append_src<BFA_DTYPE_F16>(cache_dtype, a, num_tokens, vec, s); break;
    default: launch_append_src<BFA_DTYPE_F32>(cache_dtype, a, num_tokens, vec, s); break;
  }
  return check_launch(what);
}
