// Rotary embedding (neox half-split) and the paged differential re-rotation of
// cached chunk K, on gfx950.
//
// RotaryEmbedding.forward / apply_rotary_emb (layers/rotary_embedding.py:6-24,49-65):
//   cs = cos_sin_cache[positions]            (fp32 [max_pos, D], cos | sin halves)
//   x1, x2 = x.f32.chunk(2, -1)
//   y = cat(x1*cos - x2*sin, x2*cos + x1*sin).to(x.dtype)
// Each product and sum is rounded separately (the library is built with
// -ffp-contract=off), which is what the unfused torch op chain computes, so
// the result matches it bit for bit before the final cast.  Negative positions
// index from the end of the table as torch indexing does; positions outside
// [-max_pos, max_pos) set BFA_STATUS_INDEX_OOB and produce zeros.
//
// A row is one (token, head) vector of D elements.  A group of D/16 lanes owns
// a row: lane i handles x1[8i..8i+8) and the matching x2 chunk D/2 further on,
// i.e. two 16-byte loads and two 16-byte stores for bf16, plus the cos/sin
// row read from the (L2-resident) table.
#include "bfa_device.h"
#include "bfa_host.h"

namespace bfa {

__device__ __forceinline__ int64_t wrap_position(int64_t p, int64_t max_pos, bool& ok) {
  if (p < 0) p += max_pos;
  ok = (p >= 0 && p < max_pos);
  return ok ? p : 0;
}

// y1 = x1*c - x2*s ; y2 = x2*c + x1*s   (in place on x1/x2)
__device__ __forceinline__ void rotate8(float (&x1)[8], float (&x2)[8], const float (&c)[8],
                                        const float (&s)[8]) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float a = x1[i], b = x2[i];
    x1[i] = a * c[i] - b * s[i];
    x2[i] = b * c[i] + a * s[i];
  }
}

__device__ __forceinline__ void load_cs8(const float* row, int64_t half, int j, float (&c)[8],
                                         float (&s)[8]) {
  load8<BFA_DTYPE_F32>(row + j, c);
  load8<BFA_DTYPE_F32>(row + half + j, s);
}

// ----------------------------------------------------------------- RoPE
struct RopeTensor {
  const void* x;
  void* y;
  int64_t heads;
  int64_t s_tok, s_head;  // input strides (elements); output is contiguous [T, heads, D]
};

struct RopeArgs {
  const void* positions;  // nullptr: token t uses cos/sin rows cosp/sinp + t*cs_stride
  int pos_is_i64;
  int64_t num_tokens;
  const float* cache;
  int64_t max_pos;
  const float* cosp;
  const float* sinp;
  int64_t cs_stride;
  int64_t head_dim;
  RopeTensor t[2];  // query, key (heads == 0: absent)
  int* status;
};

__device__ __forceinline__ int64_t load_pos(const void* p, int is64, int64_t t) {
  return is64 ? static_cast<const int64_t*>(p)[t] : static_cast<const int32_t*>(p)[t];
}

// cos / sin rows for token `tok`; ok=false for an out-of-range position.
__device__ __forceinline__ void cs_rows(const RopeArgs& a, int64_t tok, const float*& c,
                                        const float*& s, bool& ok) {
  if (a.positions) {
    const int64_t p = wrap_position(load_pos(a.positions, a.pos_is_i64, tok), a.max_pos, ok);
    c = a.cache + p * a.head_dim;
    s = c + a.head_dim / 2;
  } else {
    ok = true;
    c = a.cosp + tok * a.cs_stride;
    s = a.sinp + tok * a.cs_stride;
  }
}

// Vector path: D % 16 == 0, 16-byte aligned rows.  LPR = lanes per row = D/16.
template <int DT>
__global__ __launch_bounds__(256) void rope_vec_kernel(RopeArgs a, int64_t total_rows, int lpr) {
  using T = typename Elem<DT>::T;
  const int64_t rows_per_wg = 256 / lpr;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * rows_per_wg + threadIdx.x / lpr;
  const int lane = threadIdx.x % lpr;
  if (row >= total_rows) return;
  const int64_t rows_q = a.num_tokens * a.t[0].heads;
  const int which = row < rows_q ? 0 : 1;
  const RopeTensor& tt = a.t[which];
  const int64_t r = which == 0 ? row : row - rows_q;
  const int64_t tok = r / tt.heads, head = r - tok * tt.heads;
  const int64_t half = a.head_dim / 2;
  const int j = lane * 8;
  bool ok;
  const float* crow;
  const float* srow;
  cs_rows(a, tok, crow, srow, ok);
  T* yp = static_cast<T*>(tt.y) + r * a.head_dim;
  float x1[8], x2[8];
  if (ok) {
    const T* xp = static_cast<const T*>(tt.x) + tok * tt.s_tok + head * tt.s_head;
    float c[8], s[8];
    load8_nt<DT>(xp + j, x1);
    load8_nt<DT>(xp + half + j, x2);
    load8<BFA_DTYPE_F32>(crow + j, c);
    load8<BFA_DTYPE_F32>(srow + j, s);
    rotate8(x1, x2, c, s);
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) x1[i] = x2[i] = 0.f;
    if (lane == 0) flag_status(a.status, BFA_STATUS_INDEX_OOB);
  }
  store8<DT>(yp + j, x1);
  store8<DT>(yp + half + j, x2);
}

// Scalar path: any even D, any alignment.  One lane per (row, pair).
template <int DT>
__global__ __launch_bounds__(256) void rope_scalar_kernel(RopeArgs a, int64_t total_rows) {
  const int64_t half = a.head_dim / 2;
  const int64_t item = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (item >= total_rows * half) return;
  const int64_t row = item / half;
  const int64_t j = item - row * half;
  const int64_t rows_q = a.num_tokens * a.t[0].heads;
  const int which = row < rows_q ? 0 : 1;
  const RopeTensor& tt = a.t[which];
  const int64_t r = which == 0 ? row : row - rows_q;
  const int64_t tok = r / tt.heads, head = r - tok * tt.heads;
  bool ok;
  const float* crow;
  const float* srow;
  cs_rows(a, tok, crow, srow, ok);
  float y1 = 0.f, y2 = 0.f;
  if (ok) {
    const int64_t xo = tok * tt.s_tok + head * tt.s_head;
    const float x1 = load1<DT>(tt.x, xo + j), x2 = load1<DT>(tt.x, xo + half + j);
    const float c = crow[j], s = srow[j];
    y1 = x1 * c - x2 * s;
    y2 = x2 * c + x1 * s;
  } else if (j == 0) {
    flag_status(a.status, BFA_STATUS_INDEX_OOB);
  }
  store1<DT>(tt.y, r * a.head_dim + j, y1);
  store1<DT>(tt.y, r * a.head_dim + half + j, y2);
}

template <int DT>
static void launch_rope(const RopeArgs& a, bool vec, hipStream_t s) {
  const int64_t total_rows = a.num_tokens * (a.t[0].heads + a.t[1].heads);
  if (vec) {
    const int lpr = static_cast<int>(a.head_dim / 16);
    const int64_t rpw = 256 / lpr;
    hipLaunchKernelGGL((rope_vec_kernel<DT>), dim3(cdiv(total_rows, rpw)), dim3(256), 0, s, a,
                       total_rows, lpr);
  } else {
    hipLaunchKernelGGL((rope_scalar_kernel<DT>), dim3(cdiv(total_rows * (a.head_dim / 2), 256)),
                       dim3(256), 0, s, a, total_rows);
  }
}

// ------------------------------------------------- paged differential RoPE
// The per-layer cache is [num_pages, 2, Hkv, page_size, D] (HND, K at index 0;
// engine/page_manager.py:36-42).  Workgroup (g, h) handles page-list entry g
// and kv head h.  For the chunk c that owns entry g the rotation is by
// delta[c] = global_start - cached_start (cascade_attention.py:151-174), one
// cos/sin row for the whole chunk.  delta == 0 leaves K untouched (the
// reference skips the rotation), i.e. a plain copy in the out-of-place mode.
// With a k_norm weight the per-(token, head) RMSNorm of
// cascade_attention.py:177-178 (RMSNorm.rms_forward on the bf16 rotated K) is
// applied before the store.
struct RerotArgs {
  void* cache;
  int64_t page_elems;  // elements per page (2*Hkv*page_size*D)
  int64_t num_cache_pages;
  int64_t hkv, page_size, head_dim;
  const int32_t* page_indices;
  const int32_t* chunk_indptr;
  const int32_t* last_page_len;
  const void* delta;
  int delta_is_i64;
  int64_t num_chunks;
  const float* cs_cache;
  int64_t max_pos;
  const void* norm_w;
  int norm_w_dtype;
  float norm_eps;
  void* out;  // nullptr: rotate the cache in place; else [num_entries, page_size, Hkv, D]
  int* status;
};

template <int DT, bool NORM>
__global__ __launch_bounds__(256) void rerotate_kernel(RerotArgs a) {
  using T = typename Elem<DT>::T;
  const int64_t g = blockIdx.x;  // page-list entry
  const int64_t h = blockIdx.y;  // kv head
  const int64_t page = a.page_indices[g];  // requested before the chunk search, which it does not need
  // chunk owning entry g: last c with indptr[c] <= g.  indptr is non-decreasing,
  // so the chunks with indptr[c] <= g are a prefix: each wave tests 64 chunks
  // per load and counts the prefix (one memory round trip per 64 chunks where
  // a binary search takes log2(chunks) dependent ones).
  const int wl = threadIdx.x & (kWave - 1);
  int64_t c = 0;
  for (int64_t base = 0; base < a.num_chunks; base += kWave) {
    const int64_t idx = base + wl;
    const bool le = idx < a.num_chunks && a.chunk_indptr[idx] <= g;
    const uint64_t m = __ballot(le);
    if (m) c = base + __popcll(m) - 1;
    if (!(m >> (kWave - 1))) break;  // the prefix ended inside this block
  }
  const bool last = (g == a.chunk_indptr[c + 1] - 1);
  const int64_t ntok =
      last ? max(static_cast<int64_t>(0), min(static_cast<int64_t>(a.last_page_len[c]), a.page_size))
           : a.page_size;
  const int64_t delta = a.delta_is_i64 ? static_cast<const int64_t*>(a.delta)[c]
                                       : static_cast<const int32_t*>(a.delta)[c];
  if (page < 0 || page >= a.num_cache_pages) {
    if (threadIdx.x == 0) flag_status(a.status, BFA_STATUS_INDEX_OOB);
    return;
  }
  bool ok = true;
  const int64_t p = wrap_position(delta, a.max_pos, ok);
  if (!ok) {
    if (threadIdx.x == 0) flag_status(a.status, BFA_STATUS_INDEX_OOB);
    return;
  }
  const bool rotate = delta != 0;
  if (!rotate && a.out == nullptr) return;  // in place, nothing to do

  const int lpr = static_cast<int>(a.head_dim / 16);
  const int rows_per_pass = 256 / lpr;
  const int lane = threadIdx.x % lpr;
  const int64_t half = a.head_dim / 2;
  const int j = lane * 8;
  T* kpage = static_cast<T*>(a.cache) + page * a.page_elems + h * a.page_size * a.head_dim;
  float cs[8], sn[8];
  if (rotate) load_cs8(a.cs_cache + p * a.head_dim, half, j, cs, sn);

  // Out-of-place output is page-padded: slots past the chunk's last token are zeroed.
  const int64_t nslots = a.out == nullptr ? ntok : a.page_size;
  for (int64_t tok = threadIdx.x / lpr; tok < nslots; tok += rows_per_pass) {
    if (tok >= ntok) {
      T* dst = static_cast<T*>(a.out) + ((g * a.page_size + tok) * a.hkv + h) * a.head_dim;
      const float z[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
      store8<DT>(dst + j, z);
      store8<DT>(dst + half + j, z);
      continue;
    }
    T* src = kpage + tok * a.head_dim;
    float x1[8], x2[8];
    load8_nt<DT>(src + j, x1);
    load8_nt<DT>(src + half + j, x2);
    if (rotate) {
      rotate8(x1, x2, cs, sn);
#pragma unroll
      for (int i = 0; i < 8; ++i) {  // apply_rotary_emb returns x.dtype
        x1[i] = Elem<DT>::round(x1[i]);
        x2[i] = Elem<DT>::round(x2[i]);
      }
    }
    if constexpr (NORM) {
      float ss = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) ss += x1[i] * x1[i] + x2[i] * x2[i];
      // lanes of one row are an aligned group of lpr (4 or 8, a power of two)
      for (int m = lpr / 2; m >= 1; m >>= 1) ss += __shfl_xor(ss, m, kWave);
      const float r = 1.0f / sqrtf(ss / static_cast<float>(a.head_dim) + a.norm_eps);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float g1 = load_any(a.norm_w, a.norm_w_dtype, j + i);
        const float g2 = load_any(a.norm_w, a.norm_w_dtype, half + j + i);
        x1[i] = Elem<DT>::round(x1[i] * r) * g1;
        x2[i] = Elem<DT>::round(x2[i] * r) * g2;
      }
    }
    T* dst = a.out == nullptr
                 ? src
                 : static_cast<T*>(a.out) + ((g * a.page_size + tok) * a.hkv + h) * a.head_dim;
    store8<DT>(dst + j, x1);
    store8<DT>(dst + half + j, x2);
  }
}

// One workgroup per page-list entry, covering every kv head of the page.  The
// page's K half (Hkv x page_size rows of D elements, contiguous) is requested
// as soon as the page id has arrived, while the chunk search and the delta ->
// cos/sin lookups (one row for the whole entry) are still in flight.  Rows are
// walked in passes of 256 / LPR: a row belongs to an aligned group of LPR
// lanes (LPR the power of two >= D / 16; lanes q >= D / 16 idle), lane q taking
// the granule pair at columns 8q and D/2 + 8q, and U passes are in flight at
// once.  Same arithmetic and outputs as rerotate_kernel.
template <int LPR>
__device__ __forceinline__ float row_group_sum(float v) {
  if constexpr (LPR <= 16) return group_sum_dpp<LPR>(v);
  else return group_sum<LPR>(v);
}

// 8 elements as raw bits (16-bit types: one 16-byte word; fp32: two), so that
// loads can be issued unconditionally and converted after the data is in.
template <int DT>
struct Raw8 {
  uint4 w[DT == BFA_DTYPE_F32 ? 2 : 1];
  __device__ __forceinline__ void load(const void* p) {
    w[0] = load16_nt(p);
    if constexpr (DT == BFA_DTYPE_F32) w[1] = load16_nt(static_cast<const float*>(p) + 4);
  }
  __device__ __forceinline__ void to_f32(float (&v)[8]) const {
    if constexpr (DT == BFA_DTYPE_F32) {
      const uint32_t u[8] = {w[0].x, w[0].y, w[0].z, w[0].w, w[1].x, w[1].y, w[1].z, w[1].w};
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = __uint_as_float(u[i]);
    } else {
      const uint32_t u[4] = {w[0].x, w[0].y, w[0].z, w[0].w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        v[2 * i] = Elem<DT>::to_f32(static_cast<uint16_t>(u[i] & 0xffffu));
        v[2 * i + 1] = Elem<DT>::to_f32(static_cast<uint16_t>(u[i] >> 16));
      }
    }
  }
};

template <int DT, bool NORM, int LPR, bool ONE_BLOCK>
__global__ __launch_bounds__(256) void rerotate_entry_kernel(RerotArgs a) {
  using T = typename Elem<DT>::T;
  static_assert(LPR >= 1 && LPR <= 64, "a row stays inside one wave");
  constexpr int RPP = 256 / LPR;                         // rows per pass
  constexpr int U = LPR >= 8 ? 4 : (LPR >= 2 ? 2 : 1);  // passes per batch
  const int64_t g = blockIdx.x;
  const int tid = threadIdx.x, wl = tid & (kWave - 1);
  const int q = tid % LPR, rsub = tid / LPR, j = q * 8;
  const int64_t D = a.head_dim, half = D / 2;
  const bool act = j < half;  // lane q < D / 16
  const int32_t page32 = a.page_indices[g];  // widened after the barrier below
  // Chunk owning entry g: the last c with indptr[c] <= g.  Lane l requests
  // indptr[l] together with the page id and, when there are fewer than 64
  // chunks, chunk l's delta and last-page length too, so that the chunk's
  // figures come out of that one round trip by lane reads.
  // (loads are unconditional, at clamped indices, so that none waits for
  // another; ONE_BLOCK: fewer than 64 chunks, chosen by the host, so that the
  // code has no join where the compiler would wait for every load)
  constexpr bool one_block = ONE_BLOCK;
  const int64_t wi = min<int64_t>(wl, a.num_chunks);      // indptr has num_chunks + 1 entries
  const int64_t wc = min<int64_t>(wl, a.num_chunks - 1);  // num_chunks >= 1
  int32_t v0 = a.chunk_indptr[wi];
  // delta as 32-bit words at a computed offset: no branch between the loads
  const int32_t* dw = static_cast<const int32_t*>(a.delta);
  int32_t dlo = dw[a.delta_is_i64 ? 2 * wc : wc];
  int32_t dhi = dw[a.delta_is_i64 ? 2 * wc + 1 : wc];
  int32_t vlast = a.last_page_len[wc];
  // keep the page id's wait (its first use is below) after these loads' issue
  __builtin_amdgcn_sched_barrier(0);
  const int64_t page = page32;
  // no branch before every load is issued: an out-of-range page id reads
  // page 0 and leaves once the loads are out
  const bool page_ok = page >= 0 && page < a.num_cache_pages;
  const int64_t rows = a.hkv * a.page_size;
  const T* kpage = static_cast<const T*>(a.cache) + (page_ok ? page : 0) * a.page_elems;
  Raw8<DT> k1[U], k2[U];
  const int jc = act ? j : 0;
  auto load_batch = [&](int64_t r0) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t row = min(r0 + u * RPP + rsub, rows - 1);
      k1[u].load(kpage + row * D + jc);
      k2[u].load(kpage + row * D + half + jc);
    }
  };
  load_batch(0);  // in flight during the chunk search and the delta -> cos/sin lookups
  // the chunk figures are taken from these registers by lane reads; the empty
  // asm keeps the compiler from turning each lane read back into a load of
  // its own, issued only once the chunk is known
  __asm__ volatile("" : "+v"(v0), "+v"(dlo), "+v"(dhi), "+v"(vlast));
  if (!page_ok) {
    if (tid == 0) flag_status(a.status, BFA_STATUS_INDEX_OOB);
    return;
  }
  int32_t v = wl <= a.num_chunks ? v0 : 0x7fffffff;
  const int64_t vdelta = a.delta_is_i64 ? static_cast<int64_t>((static_cast<uint64_t>(static_cast<uint32_t>(dhi)) << 32) |
                                                                static_cast<uint32_t>(dlo))
                                        : static_cast<int64_t>(dlo);
  int64_t c = 0, delta;
  int32_t next, lpl;
  if constexpr (one_block) {
    const uint64_t m = __ballot(wl < a.num_chunks && v <= g);
    c = m ? __popcll(m) - 1 : 0;
    const int ci = static_cast<int>(c);
    next = __builtin_amdgcn_readlane(v, ci + 1);
    lpl = __builtin_amdgcn_readlane(vlast, ci);
    const uint32_t dlo = __builtin_amdgcn_readlane(static_cast<uint32_t>(vdelta), ci);
    const uint32_t dhi = __builtin_amdgcn_readlane(static_cast<uint32_t>(static_cast<uint64_t>(vdelta) >> 32), ci);
    delta = static_cast<int64_t>((static_cast<uint64_t>(dhi) << 32) | dlo);
  } else {
    for (int64_t base = 0;;) {
      const uint64_t m = __ballot(base + wl < a.num_chunks && v <= g);
      if (m) c = base + __popcll(m) - 1;
      if ((m >> (kWave - 1)) == 0) break;  // the prefix ended inside this block
      base += kWave;
      if (base >= a.num_chunks) break;
      v = base + wl < a.num_chunks ? a.chunk_indptr[base + wl] : 0x7fffffff;
    }
    next = a.chunk_indptr[c + 1];
    lpl = a.last_page_len[c];
    delta = a.delta_is_i64 ? static_cast<const int64_t*>(a.delta)[c] : static_cast<const int32_t*>(a.delta)[c];
  }
  bool ok = true;
  const int64_t p = wrap_position(delta, a.max_pos, ok);
  if (!ok) {
    if (tid == 0) flag_status(a.status, BFA_STATUS_INDEX_OOB);
    return;
  }
  const bool rotate = delta != 0;
  if (!rotate && a.out == nullptr) return;  // in place, nothing to do
  const int64_t ntok =
      g == next - 1 ? max(int64_t(0), min(static_cast<int64_t>(lpl), a.page_size)) : a.page_size;
  float cs[8], sn[8];
  load_cs8(a.cs_cache + p * D, half, jc, cs, sn);  // (row p = 0 when delta is 0: unused)
  float g1[8], g2[8];
  if constexpr (NORM) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      g1[i] = load_any(a.norm_w, a.norm_w_dtype, jc + i);
      g2[i] = load_any(a.norm_w, a.norm_w_dtype, half + jc + i);
    }
  }
  for (int64_t r0 = 0; r0 < rows; r0 += U * RPP) {
    if (r0 > 0) load_batch(r0);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t row = r0 + u * RPP + rsub;
      if (row >= rows) continue;  // uniform over the row's lanes
      const int64_t h = row / a.page_size, tok = row - h * a.page_size;
      float x1[8], x2[8];
      k1[u].to_f32(x1);
      k2[u].to_f32(x2);
      if (tok >= ntok) {
        if (a.out != nullptr && act) {
          T* dst = static_cast<T*>(a.out) + ((g * a.page_size + tok) * a.hkv + h) * D;
          const float z[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
          store8<DT>(dst + j, z);
          store8<DT>(dst + half + j, z);
        }
        continue;
      }
      if (rotate && act) {
        rotate8(x1, x2, cs, sn);
#pragma unroll
        for (int i = 0; i < 8; ++i) {  // apply_rotary_emb returns x.dtype
          x1[i] = Elem<DT>::round(x1[i]);
          x2[i] = Elem<DT>::round(x2[i]);
        }
      }
      if constexpr (NORM) {
        float ss = 0.f;
        if (act) {
#pragma unroll
          for (int i = 0; i < 8; ++i) ss += x1[i] * x1[i] + x2[i] * x2[i];
        }
        ss = row_group_sum<LPR>(ss);  // every lane of the row group takes part
        const float r = 1.0f / sqrtf(ss / static_cast<float>(D) + a.norm_eps);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          x1[i] = Elem<DT>::round(x1[i] * r) * g1[i];
          x2[i] = Elem<DT>::round(x2[i] * r) * g2[i];
        }
      }
      if (act) {
        T* dst = a.out == nullptr ? const_cast<T*>(kpage) + row * D
                                  : static_cast<T*>(a.out) + ((g * a.page_size + tok) * a.hkv + h) * D;
        store8<DT>(dst + j, x1);
        store8<DT>(dst + half + j, x2);
      }
    }
  }
}

}  // namespace bfa

using namespace bfa;

extern "C" int bfa_rotary_embedding(const void* positions, int positions_dtype, int64_t num_tokens,
                                    const float* cos_sin_cache, int64_t max_position,
                                    int64_t head_size, int dtype, const void* query,
                                    int64_t q_heads, int64_t q_stride_token,
                                    int64_t q_stride_head, void* query_out, const void* key,
                                    int64_t k_heads, int64_t k_stride_token,
                                    int64_t k_stride_head, void* key_out, int32_t* status,
                                    void* stream) {
  const char* what = "bfa_rotary_embedding";
  BFA_REQUIRE(is_float_dtype(dtype), "%s: bad dtype", what);
  BFA_REQUIRE(positions_dtype == BFA_DTYPE_I64 || positions_dtype == BFA_DTYPE_I32,
              "%s: positions must be int32/int64", what);
  BFA_REQUIRE(head_size > 0 && head_size % 2 == 0, "%s: head_size must be even", what);
  BFA_REQUIRE(num_tokens >= 0 && q_heads >= 0 && k_heads >= 0 && max_position > 0,
              "%s: bad geometry", what);
  if (!query) q_heads = 0;
  if (!key) k_heads = 0;
  if (num_tokens == 0 || q_heads + k_heads == 0) return BFA_OK;
  BFA_REQUIRE(positions && cos_sin_cache, "%s: null pointer", what);
  BFA_REQUIRE(q_heads == 0 || query_out, "%s: null query_out", what);
  BFA_REQUIRE(k_heads == 0 || key_out, "%s: null key_out", what);
  RopeArgs a{};
  a.positions = positions;
  a.pos_is_i64 = positions_dtype == BFA_DTYPE_I64;
  a.num_tokens = num_tokens;
  a.cache = cos_sin_cache;
  a.max_pos = max_position;
  a.head_dim = head_size;
  a.t[0] = RopeTensor{query, query_out, q_heads, q_stride_token, q_stride_head};
  a.t[1] = RopeTensor{key, key_out, k_heads, k_stride_token, k_stride_head};
  a.status = status;
  auto tensor_vec_ok = [](const RopeTensor& t) {
    return t.heads == 0 || (aligned16(t.x) && aligned16(t.y) && t.s_tok % 8 == 0 && t.s_head % 8 == 0);
  };
  const bool vec = head_size % 16 == 0 && head_size <= 4096 && aligned16(cos_sin_cache) &&
                   tensor_vec_ok(a.t[0]) && tensor_vec_ok(a.t[1]);
  const hipStream_t s = as_stream(stream);
  switch (dtype) {
    case BFA_DTYPE_BF16: launch_rope<BFA_DTYPE_BF16>(a, vec, s); break;
    case BFA_DTYPE_F16: launch_rope<BFA_DTYPE_F16>(a, vec, s); break;
    default: launch_rope<BFA_DTYPE_F32>(a, vec, s); break;
  }
  return check_launch(what);
}

extern "C" int bfa_rerotate_paged_k(void* kv_cache, int dtype, int64_t num_cache_pages,
                                    int64_t num_kv_heads, int64_t page_size, int64_t head_dim,
                                    const int32_t* page_indices, int64_t num_entries,
                                    const int32_t* chunk_indptr, const int32_t* last_page_len,
                                    const void* chunk_delta, int delta_dtype, int64_t num_chunks,
                                    const float* cos_sin_cache, int64_t max_position,
                                    const void* k_norm_weight, int k_norm_dtype,
                                    float k_norm_eps, void* out, int32_t* status,
                                    void* stream) {
  const char* what = "bfa_rerotate_paged_k";
  BFA_REQUIRE(is_float_dtype(dtype), "%s: bad dtype", what);
  BFA_REQUIRE(delta_dtype == BFA_DTYPE_I64 || delta_dtype == BFA_DTYPE_I32,
              "%s: delta must be int32/int64", what);
  BFA_REQUIRE(head_dim % 16 == 0 && head_dim >= 16 && head_dim <= 4096,
              "%s: head_dim must be a multiple of 16 (got %lld)", what, (long long)head_dim);
  BFA_REQUIRE(num_kv_heads > 0 && page_size > 0 && num_cache_pages >= 0 && num_entries >= 0 &&
                  num_chunks >= 0 && max_position > 0,
              "%s: bad geometry", what);
  if (num_entries == 0 || num_chunks == 0) return BFA_OK;
  BFA_REQUIRE(kv_cache && page_indices && chunk_indptr && last_page_len && chunk_delta &&
                  cos_sin_cache,
              "%s: null pointer", what);
  BFA_REQUIRE(!(k_norm_weight && out == nullptr),
              "%s: the fused k_norm needs an output buffer (the cache keeps un-normed K)", what);
  BFA_REQUIRE(aligned16(kv_cache) && aligned16(cos_sin_cache) && (out == nullptr || aligned16(out)),
              "%s: buffers must be 16-byte aligned", what);
  BFA_REQUIRE(num_kv_heads <= 65535, "%s: too many kv heads", what);
  RerotArgs a{};
  a.cache = kv_cache;
  a.page_elems = 2 * num_kv_heads * page_size * head_dim;
  a.num_cache_pages = num_cache_pages;
  a.hkv = num_kv_heads;
  a.page_size = page_size;
  a.head_dim = head_dim;
  a.page_indices = page_indices;
  a.chunk_indptr = chunk_indptr;
  a.last_page_len = last_page_len;
  a.delta = chunk_delta;
  a.delta_is_i64 = delta_dtype == BFA_DTYPE_I64;
  a.num_chunks = num_chunks;
  a.cs_cache = cos_sin_cache;
  a.max_pos = max_position;
  a.norm_w = k_norm_weight;
  a.norm_w_dtype = k_norm_dtype;
  a.norm_eps = k_norm_eps;
  a.out = out;
  a.status = status;
  const hipStream_t s = as_stream(stream);
  const bool norm = k_norm_weight != nullptr;
  // head_dim up to 1024: one workgroup per entry, a row on an aligned group of
  // LPR lanes (the power of two >= head_dim / 16); larger head dims (no k_norm):
  // one workgroup per (entry, kv head)
  const int64_t lpa = head_dim / 16;
  int lpr = 1;
  while (lpr < lpa) lpr *= 2;
  if (lpr <= 64) {
    const dim3 grid(static_cast<unsigned>(num_entries));
    const bool one = num_chunks < 64;
#define BFA_RRE(DT, L)                                                                                 \
  if (norm && one) hipLaunchKernelGGL((rerotate_entry_kernel<DT, true, L, true>), grid, dim3(256), 0, s, a);  \
  else if (norm) hipLaunchKernelGGL((rerotate_entry_kernel<DT, true, L, false>), grid, dim3(256), 0, s, a);   \
  else if (one) hipLaunchKernelGGL((rerotate_entry_kernel<DT, false, L, true>), grid, dim3(256), 0, s, a);    \
  else hipLaunchKernelGGL((rerotate_entry_kernel<DT, false, L, false>), grid, dim3(256), 0, s, a);
#define BFA_RRL(DT)                   \
  switch (lpr) {                      \
    case 1: BFA_RRE(DT, 1); break;    \
    case 2: BFA_RRE(DT, 2); break;    \
    case 4: BFA_RRE(DT, 4); break;    \
    case 8: BFA_RRE(DT, 8); break;    \
    case 16: BFA_RRE(DT, 16); break;  \
    case 32: BFA_RRE(DT, 32); break;  \
    default: BFA_RRE(DT, 64); break;  \
  }
    switch (dtype) {
      case BFA_DTYPE_BF16: BFA_RRL(BFA_DTYPE_BF16); break;
      case BFA_DTYPE_F16: BFA_RRL(BFA_DTYPE_F16); break;
      default: BFA_RRL(BFA_DTYPE_F32); break;
    }
#undef BFA_RRL
#undef BFA_RRE
    return check_launch(what);
  }
  BFA_REQUIRE(!norm, "%s: the fused k_norm covers head_dim up to 1024 (got %lld)", what,
              (long long)head_dim);
  const dim3 grid(static_cast<unsigned>(num_entries), static_cast<unsigned>(num_kv_heads));
#define BFA_RR(DT) hipLaunchKernelGGL((rerotate_kernel<DT, false>), grid, dim3(256), 0, s, a);
  switch (dtype) {
    case BFA_DTYPE_BF16: BFA_RR(BFA_DTYPE_BF16); break;
    case BFA_DTYPE_F16: BFA_RR(BFA_DTYPE_F16); break;
    default: BFA_RR(BFA_DTYPE_F32); break;
  }
#undef BFA_RR
  return check_launch(what);
}

extern "C" int bfa_apply_rotary_emb(const void* x, int dtype, int64_t num_tokens, int64_t heads,
                                    int64_t head_size, int64_t x_stride_token,
                                    int64_t x_stride_head, const float* cos, const float* sin,
                                    int64_t cs_stride_token, void* out, void* stream) {
  const char* what = "bfa_apply_rotary_emb";
  BFA_REQUIRE(is_float_dtype(dtype), "%s: bad dtype", what);
  BFA_REQUIRE(head_size > 0 && head_size % 2 == 0, "%s: head_size must be even", what);
  BFA_REQUIRE(num_tokens >= 0 && heads >= 0, "%s: bad geometry", what);
  if (num_tokens == 0 || heads == 0) return BFA_OK;
  BFA_REQUIRE(x && cos && sin && out, "%s: null pointer", what);
  RopeArgs a{};
  a.positions = nullptr;
  a.num_tokens = num_tokens;
  a.head_dim = head_size;
  a.cosp = cos;
  a.sinp = sin;
  a.cs_stride = cs_stride_token;
  a.t[0] = RopeTensor{x, out, heads, x_stride_token, x_stride_head};
  a.t[1] = RopeTensor{nullptr, nullptr, 0, 0, 0};
  const bool vec = head_size % 16 == 0 && head_size <= 4096 && aligned16(x) && aligned16(out) &&
                   aligned16(cos) && aligned16(sin) && cs_stride_token % 4 == 0 &&
                   x_stride_token % 8 == 0 && x_stride_head % 8 == 0;
  const hipStream_t s = as_stream(stream);
  switch (dtype) {
    case BFA_DTYPE_BF16: launch_rope<BFA_DTYPE_BF16>(a, vec, s); break;
    case BFA_DTYPE_F16: launch_rope<BFA_DTYPE_F16>(a, vec, s); break;
    default: launch_rope<BFA_DTYPE_F32>(a, vec, s); break;
  }
  return check_launch(what);
}
