// Token-embedding gather (VocabParallelEmbedding.forward, layers/embed_head.py:28-29:
// F.embedding(ids, weight)) on gfx950.
//
// The plain gather is a byte copy (no conversion), so it is bit-exact by
// construction: every row is moved with 16-byte vector loads/stores, one
// 16-byte chunk per lane per step, consecutive lanes on consecutive chunks so
// each wave moves 1 KiB contiguous.  The optional scaled form fuses the Qwen3
// glue `embed_tokens(ids) * (1/sqrt(H))` (models/qwen3.py:464-465): the row is
// widened to fp32, multiplied by the fp32 scalar and rounded back, which is the
// opmath computation torch performs for a reduced-float tensor times a Python
// scalar.
//
// Out-of-range ids (id < 0 or id >= num_embeddings; F.embedding raises
// IndexError for both) produce a zero row and set BFA_STATUS_INDEX_OOB in the
// caller's status word.
#include "bfa_device.h"
#include "bfa_host.h"

namespace bfa {

struct GatherArgs {
  const char* table;
  const void* ids;
  char* out;
  int64_t num_embeddings;
  int64_t num_ids;
  int64_t row_chunks;      // 16-byte chunks per row (vector path) / elements (scalar path)
  int64_t table_stride_b;  // bytes
  int64_t out_stride_b;    // bytes
  float scale;
  int* status;
};

template <typename IdT>
__device__ __forceinline__ int64_t fetch_id(const void* ids, int64_t t) {
  return static_cast<int64_t>(static_cast<const IdT*>(ids)[t]);
}

// Multiplies the elements of one 16-byte chunk by `s` in fp32 and rounds back.
template <int DT>
__device__ __forceinline__ uint4 scale_chunk(uint4 u, float s) {
  if constexpr (DT == BFA_DTYPE_F32) {
    return make_uint4(__float_as_uint(__uint_as_float(u.x) * s), __float_as_uint(__uint_as_float(u.y) * s),
                      __float_as_uint(__uint_as_float(u.z) * s), __float_as_uint(__uint_as_float(u.w) * s));
  } else {
    uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float lo = Elem<DT>::to_f32(static_cast<uint16_t>(w[i] & 0xffffu)) * s;
      const float hi = Elem<DT>::to_f32(static_cast<uint16_t>(w[i] >> 16)) * s;
      w[i] = static_cast<uint32_t>(Elem<DT>::from_f32(lo)) |
             (static_cast<uint32_t>(Elem<DT>::from_f32(hi)) << 16);
    }
    return make_uint4(w[0], w[1], w[2], w[3]);
  }
}

// grid.x = ceil(row_chunks / (256*CPT)), grid.y*grid.z cover the ids
template <typename IdT, int DT, bool SCALE, int CPT>
__global__ __launch_bounds__(256) void gather_vec_kernel(GatherArgs a) {
  const int64_t t = static_cast<int64_t>(blockIdx.y) + static_cast<int64_t>(blockIdx.z) * gridDim.y;
  if (t >= a.num_ids) return;
  const int64_t id = fetch_id<IdT>(a.ids, t);
  const bool ok = id >= 0 && id < a.num_embeddings;
  if (!ok && blockIdx.x == 0 && threadIdx.x == 0) flag_status(a.status, BFA_STATUS_INDEX_OOB);
  const uint4* src = reinterpret_cast<const uint4*>(a.table + (ok ? id : 0) * a.table_stride_b);
  uint4* dst = reinterpret_cast<uint4*>(a.out + t * a.out_stride_b);
  const int64_t base = static_cast<int64_t>(blockIdx.x) * (256 * CPT) + threadIdx.x;
  uint4 v[CPT];
#pragma unroll
  for (int c = 0; c < CPT; ++c) {
    const int64_t ch = base + c * 256;
    if (ch < a.row_chunks) v[c] = ok ? load16_nt(src + ch) : make_uint4(0, 0, 0, 0);
  }
#pragma unroll
  for (int c = 0; c < CPT; ++c) {
    const int64_t ch = base + c * 256;
    if (ch < a.row_chunks) {
      if constexpr (SCALE) {
        dst[ch] = scale_chunk<DT>(v[c], a.scale);
      } else {
        dst[ch] = v[c];
      }
    }
  }
}

// Many ids: RB rows per workgroup (grid.y * grid.z cover the row blocks).  The
// ids of all RB rows are read first, then every chunk load of the RB rows goes
// out before the first store, so a workgroup waits for one id round trip and
// one row round trip for all of its rows, not one of each per row.
template <typename IdT, int DT, bool SCALE, int CPT, int RB>
__global__ __launch_bounds__(256) void gather_rows_kernel(GatherArgs a) {
  const int64_t t0 = (static_cast<int64_t>(blockIdx.y) + static_cast<int64_t>(blockIdx.z) * gridDim.y) * RB;
  if (t0 >= a.num_ids) return;
  int64_t id[RB];
  bool in[RB], ok[RB];
#pragma unroll
  for (int r = 0; r < RB; ++r) {
    in[r] = t0 + r < a.num_ids;
    id[r] = in[r] ? fetch_id<IdT>(a.ids, t0 + r) : 0;
    ok[r] = in[r] && id[r] >= 0 && id[r] < a.num_embeddings;
    if (in[r] && !ok[r] && blockIdx.x == 0 && threadIdx.x == 0) flag_status(a.status, BFA_STATUS_INDEX_OOB);
  }
  const int64_t base = static_cast<int64_t>(blockIdx.x) * (256 * CPT) + threadIdx.x;
  uint4 v[RB][CPT];
#pragma unroll
  for (int r = 0; r < RB; ++r) {
    const uint4* src = reinterpret_cast<const uint4*>(a.table + (ok[r] ? id[r] : 0) * a.table_stride_b);
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
      const int64_t ch = base + c * 256;
      if (in[r] && ch < a.row_chunks) v[r][c] = ok[r] ? load16_nt(src + ch) : make_uint4(0, 0, 0, 0);
    }
  }
#pragma unroll
  for (int r = 0; r < RB; ++r) {
    uint4* dst = reinterpret_cast<uint4*>(a.out + (t0 + r) * a.out_stride_b);
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
      const int64_t ch = base + c * 256;
      if (in[r] && ch < a.row_chunks) {
        if constexpr (SCALE) {
          dst[ch] = scale_chunk<DT>(v[r][c], a.scale);
        } else {
          dst[ch] = v[r][c];
        }
      }
    }
  }
}

// Element-granular fallback (unaligned rows or row bytes not a multiple of 16).
template <typename IdT, typename E, int DT, bool SCALE>
__global__ __launch_bounds__(256) void gather_scalar_kernel(GatherArgs a) {
  const int64_t t = static_cast<int64_t>(blockIdx.y) + static_cast<int64_t>(blockIdx.z) * gridDim.y;
  if (t >= a.num_ids) return;
  const int64_t id = fetch_id<IdT>(a.ids, t);
  const bool ok = id >= 0 && id < a.num_embeddings;
  if (!ok && blockIdx.x == 0 && threadIdx.x == 0) flag_status(a.status, BFA_STATUS_INDEX_OOB);
  const E* src = reinterpret_cast<const E*>(a.table + (ok ? id : 0) * a.table_stride_b);
  E* dst = reinterpret_cast<E*>(a.out + t * a.out_stride_b);
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < a.row_chunks;
       i += static_cast<int64_t>(gridDim.x) * 256) {
    if constexpr (SCALE) {
      const float f = ok ? load1<DT>(src, i) : 0.f;
      store1<DT>(dst, i, f * a.scale);
    } else {
      dst[i] = ok ? src[i] : E{};
    }
  }
}

static dim3 token_grid(int64_t gx, int64_t n) {
  // grid.y is limited to 65535 on some runtimes: fold the rest into grid.z
  const int64_t gy = n < 65535 ? n : 65535;
  const int64_t gz = cdiv(n, gy);
  return dim3(static_cast<unsigned>(gx), static_cast<unsigned>(gy), static_cast<unsigned>(gz));
}

template <typename IdT, int DT, bool SCALE>
static void launch_gather(GatherArgs a, bool vec, int esize, hipStream_t s) {
  if (vec) {
    if (a.num_ids >= 4096 && a.row_chunks <= 256 * 2) {
      // rows of up to 8 KiB, four per workgroup (8192 ids of the Llama-3-8B
      // table: 24.8 -> 24.2 us against one row per workgroup)
      const dim3 g = token_grid(1, cdiv(a.num_ids, 4));
      hipLaunchKernelGGL((gather_rows_kernel<IdT, DT, SCALE, 2, 4>), g, dim3(256), 0, s, a);
      return;
    }
    if (a.num_ids >= 1024) {
      const dim3 g = token_grid(cdiv(a.row_chunks, 256 * 4), a.num_ids);
      hipLaunchKernelGGL((gather_vec_kernel<IdT, DT, SCALE, 4>), g, dim3(256), 0, s, a);
    } else {
      const dim3 g = token_grid(cdiv(a.row_chunks, 256), a.num_ids);
      hipLaunchKernelGGL((gather_vec_kernel<IdT, DT, SCALE, 1>), g, dim3(256), 0, s, a);
    }
    return;
  }
  const int64_t gx = std::min<int64_t>(cdiv(a.row_chunks, 256), 64);
  const dim3 g = token_grid(gx, a.num_ids);
  if constexpr (SCALE) {
    if (DT == BFA_DTYPE_F32) {
      hipLaunchKernelGGL((gather_scalar_kernel<IdT, float, DT, true>), g, dim3(256), 0, s, a);
    } else {
      hipLaunchKernelGGL((gather_scalar_kernel<IdT, uint16_t, DT, true>), g, dim3(256), 0, s, a);
    }
  } else {
    switch (esize) {
      case 1: hipLaunchKernelGGL((gather_scalar_kernel<IdT, uint8_t, DT, false>), g, dim3(256), 0, s, a); break;
      case 2: hipLaunchKernelGGL((gather_scalar_kernel<IdT, uint16_t, DT, false>), g, dim3(256), 0, s, a); break;
      case 4: hipLaunchKernelGGL((gather_scalar_kernel<IdT, uint32_t, DT, false>), g, dim3(256), 0, s, a); break;
      default: hipLaunchKernelGGL((gather_scalar_kernel<IdT, uint64_t, DT, false>), g, dim3(256), 0, s, a); break;
    }
  }
}

template <typename IdT>
static int dispatch_gather(GatherArgs a, int dtype, bool scale, bool vec, int esize, hipStream_t s) {
  if (!scale) {
    launch_gather<IdT, BFA_DTYPE_BF16, false>(a, vec, esize, s);
    return BFA_OK;
  }
  switch (dtype) {
    case BFA_DTYPE_BF16: launch_gather<IdT, BFA_DTYPE_BF16, true>(a, vec, esize, s); break;
    case BFA_DTYPE_F16: launch_gather<IdT, BFA_DTYPE_F16, true>(a, vec, esize, s); break;
    case BFA_DTYPE_F32: launch_gather<IdT, BFA_DTYPE_F32, true>(a, vec, esize, s); break;
    default: return set_error(BFA_ERR_INVALID, "bfa_embedding: scaled gather needs a float table");
  }
  return BFA_OK;
}

static int embedding_impl(const void* table, int64_t num_embeddings, int64_t dim,
                          int64_t table_row_stride, int elem_bytes, int dtype, const void* ids,
                          int ids_dtype, int64_t num_ids, void* out, int64_t out_row_stride,
                          bool scale, float scale_value, int32_t* status, void* stream) {
  const char* what = "bfa_embedding";
  BFA_REQUIRE(ids_dtype == BFA_DTYPE_I32 || ids_dtype == BFA_DTYPE_I64, "%s: ids must be int32/int64", what);
  BFA_REQUIRE(elem_bytes == 1 || elem_bytes == 2 || elem_bytes == 4 || elem_bytes == 8,
              "%s: unsupported element size %d", what, elem_bytes);
  BFA_REQUIRE(num_embeddings >= 0 && dim >= 0 && num_ids >= 0, "%s: bad geometry", what);
  if (num_ids == 0 || dim == 0) return BFA_OK;
  BFA_REQUIRE(table && ids && out, "%s: null pointer", what);
  if (scale) {
    BFA_REQUIRE(is_float_dtype(dtype) && elem_bytes == dtype_size(dtype), "%s: bad scaled dtype", what);
  }
  GatherArgs a{};
  a.table = static_cast<const char*>(table);
  a.ids = ids;
  a.out = static_cast<char*>(out);
  a.num_embeddings = num_embeddings;
  a.num_ids = num_ids;
  a.table_stride_b = table_row_stride * elem_bytes;
  a.out_stride_b = out_row_stride * elem_bytes;
  a.scale = scale_value;
  a.status = status;
  const int64_t row_bytes = dim * elem_bytes;
  const bool vec = (row_bytes % 16 == 0) && (a.table_stride_b % 16 == 0) &&
                   (a.out_stride_b % 16 == 0) && aligned16(table) && aligned16(out);
  a.row_chunks = vec ? row_bytes / 16 : dim;
  const hipStream_t s = as_stream(stream);
  const int rc = ids_dtype == BFA_DTYPE_I64
                     ? dispatch_gather<int64_t>(a, dtype, scale, vec, elem_bytes, s)
                     : dispatch_gather<int32_t>(a, dtype, scale, vec, elem_bytes, s);
  if (rc != BFA_OK) return rc;
  return check_launch(what);
}

}  // namespace bfa

extern "C" int bfa_embedding(const void* table, int64_t num_embeddings, int64_t dim,
                             int64_t table_row_stride, int elem_bytes, const void* ids,
                             int ids_dtype, int64_t num_ids, void* out, int64_t out_row_stride,
                             int32_t* status, void* stream) {
  return bfa::embedding_impl(table, num_embeddings, dim, table_row_stride, elem_bytes, -1, ids,
                             ids_dtype, num_ids, out, out_row_stride, false, 1.0f, status, stream);
}

extern "C" int bfa_embedding_scaled(const void* table, int64_t num_embeddings, int64_t dim,
                                    int64_t table_row_stride, int dtype, const void* ids,
                                    int ids_dtype, int64_t num_ids, void* out,
                                    int64_t out_row_stride, float scale, int32_t* status,
                                    void* stream) {
  return bfa::embedding_impl(table, num_embeddings, dim, table_row_stride,
                             bfa::dtype_size(dtype), dtype, ids, ids_dtype, num_ids, out,
                             out_row_stride, true, scale, status, stream);
}
