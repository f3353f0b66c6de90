// Paged cascade attention on gfx950: the per-page loop of CascadeAttention.forward
// (braidinfer/layers/cascade_attention.py:50-231) in one launch, and the online
// softmax state update it calls per page (kernels/online_softmax.py:14-297).
//
// Reference semantics (per query token t, query head h, kv head h / (Hq / Hkv)):
//   for every level, every chunk with pages and kv_length > 0, every page of it
//   (tokens = last_page_len on the chunk's last page, else page_size; pages with
//   tokens <= 0 skipped):
//     k = cache[page, 0, kv, :tokens]; v = cache[page, 1, kv, :tokens]
//     if the chunk moved (delta = global_position_start - cached_position_start
//     != 0) and a rotary table is given: k = RoPE(k, cos_sin_cache[delta]) (torch
//     indexing: a negative delta wraps), rounded to the cache dtype
//     if k_norm is given: k = RMSNorm(k) over head_dim (bf16 rounding points)
//     key positions = (kv_length of the earlier valid chunks) + page offset + slot
//     online softmax update in fp32 with score = (q . k) * scale, keys with
//     position > the query's position masked when causal
//   out = acc / max(l, 1e-12), in the query dtype.
//
// Kernel design.  Rows are (query token, query head of a kv group) pairs of one kv
// head; a workgroup of 4 waves owns 64 rows and one kv head and walks a range of
// the padded key space (entry e, slot s) -> e * page_size + s in steps of 32 key
// slots.  The entries are the attended pages in walk order, each with its page
// id, first key position, chunk delta and token count / rotate flag, flattened
// on the host once per set of levels.  Per step: 256 lanes stage the 32 keys of
// K into LDS (rotated and normalised on the way, with the rounding of the
// re-rotation kernel) and V transposed into LDS; each wave computes S^T = K Q^T
// for its 16 rows with v_mfma_f32_16x16x32_bf16 (a lane then holds 8 scores of
// one query), masks, updates its running max / sum in fp32 (base 2; in-lane plus
// two gfx950 lane swaps) and adds O^T += V^T P^T with 8 more MFMAs, P^T going
// from its registers straight into the B operand.  The next step's K / V / cos-sin rows and the step after's entry
// metadata are in flight during a step's matrix work.  For few rows (decode) the
// key range is split across workgroups and a merge kernel combines the partial
// (m, l, acc) rows.
#include <cmath>
#include <cstdlib>
#include <type_traits>

#include "bfa_device.h"
#include "bfa_host.h"

namespace bfa {

typedef __attribute__((ext_vector_type(8))) __bf16 cas_bf16x8_t;
typedef __attribute__((ext_vector_type(8))) _Float16 cas_f16x8_t;
typedef __attribute__((ext_vector_type(4))) float cas_f32x4_t;

template <bool BF16>
__device__ __forceinline__ cas_f32x4_t mfma16x32(const uint4& a, const uint4& b, cas_f32x4_t c) {
  if constexpr (BF16) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(cas_bf16x8_t, a),
                                                   __builtin_bit_cast(cas_bf16x8_t, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(cas_f16x8_t, a),
                                                  __builtin_bit_cast(cas_f16x8_t, b), c, 0, 0, 0);
  }
}

// ================================================== online softmax update
// One wave per (head, batch) query: lanes split head_dim (up to 4 elements each),
// keys are taken in order, one at a time, as the reference kernel does.
struct OsmArgs {
  const void* q;
  const void* k;
  const void* v;
  int q_dt, kv_dt;
  float* m;
  float* l;
  float* acc;
  const void* qpos;
  const void* kpos;
  int qpos_i64, kpos_i64;
  int64_t heads, batch, tokens, head_dim;
  int64_t q_sh, q_sb, k_sh, k_st, v_sh, v_st;  // element strides (unit stride along head_dim)
  int64_t m_sh, m_sb, l_sh, l_sb, a_sh, a_sb;
  float scale;
  int causal;
};

__global__ __launch_bounds__(256) void online_softmax_kernel(OsmArgs a) {
  const int64_t item = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (item >= a.heads * a.batch) return;
  const int64_t h = item / a.batch, b = item - h * a.batch;
  const int lane = threadIdx.x & 63;
  const int64_t qp = a.qpos_i64 ? static_cast<const int64_t*>(a.qpos)[b]
                                : static_cast<const int32_t*>(a.qpos)[b];
  float qv[4], av[4];
  float* accp = a.acc + h * a.a_sh + b * a.a_sb;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t d = lane + 64 * i;
    const bool in = d < a.head_dim;
    qv[i] = in ? load_any(a.q, a.q_dt, h * a.q_sh + b * a.q_sb + d) : 0.f;
    av[i] = in ? accp[d] : 0.f;
  }
  float m = a.m[h * a.m_sh + b * a.m_sb];
  float l = a.l[h * a.l_sh + b * a.l_sb];
  for (int64_t t = 0; t < a.tokens; ++t) {
    const int64_t kp = a.kpos_i64 ? static_cast<const int64_t*>(a.kpos)[t]
                                  : static_cast<const int32_t*>(a.kpos)[t];
    if (a.causal && kp > qp) continue;  // uniform over the wave
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t d = lane + 64 * i;
      if (d < a.head_dim) s += qv[i] * load_any(a.k, a.kv_dt, h * a.k_sh + t * a.k_st + d);
    }
    s = group_sum<kWave>(s) * a.scale;
    const float m_new = fmaxf(m, s);
    const float alpha = expf(m - m_new);
    const float beta = expf(s - m_new);
    l = l * alpha + beta;
    m = m_new;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t d = lane + 64 * i;
      if (d < a.head_dim) av[i] = alpha * av[i] + beta * load_any(a.v, a.kv_dt, h * a.v_sh + t * a.v_st + d);
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t d = lane + 64 * i;
    if (d < a.head_dim) accp[d] = av[i];
  }
  if (lane == 0) {
    a.m[h * a.m_sh + b * a.m_sb] = m;
    a.l[h * a.l_sh + b * a.l_sb] = l;
  }
}

// ===================================================== paged cascade attention
struct CasArgs {
  const uint16_t* q;        // [T, Hq, D] with strides q_st, q_sh
  int64_t q_st, q_sh;
  const void* qpos;
  int qpos_i64;
  const uint16_t* cache;    // one layer [pages, 2, Hkv, page_size, D]
  int64_t c_sp, c_skv, c_sh, c_ss;
  int64_t num_pages, page_size;
  const int32_t* pages;     // [E] page of each entry
  const int64_t* kstart;    // [E] key position of the entry's first slot
  const int64_t* delta;     // [E] RoPE shift of the entry's chunk
  const int32_t* info;      // [E] bits 0-15: tokens attended on the page, bit 16: rotate
  int64_t num_entries;
  const float* cs;          // [max_pos, D] or nullptr
  int64_t max_pos;
  const void* knorm_w;      // [D] or nullptr
  int knorm_dt;
  float knorm_eps;
  int64_t tokens, hq, hkv, group;  // group = Hq / Hkv
  float scale;
  int causal;
  int64_t steps, steps_per_split;
  void* out;                // [T, Hq * D] (q dtype), row stride out_st
  int64_t out_st;
  float* part;              // [splits, Hkv, rows, D + 2] (m, l, acc) when split
  int* status;
};

constexpr int CAS_DMAX = 128;       // largest head_dim of the MFMA paths (64 and 128 are built)

// a zeroed row that masked slots load from instead of the cache and the rotary table
__device__ __align__(16) float cas_zero_row[CAS_DMAX];
constexpr int CAS_VP = 32 + 8;      // V^T row pitch (bf16): 80 bytes

// two floats rounded to the 16-bit type, packed low | high << 16
template <bool BF16>
__device__ __forceinline__ uint32_t pack_pair(float lo, float hi) {
  using E = Elem<BF16 ? BFA_DTYPE_BF16 : BFA_DTYPE_F16>;
  return static_cast<uint32_t>(E::from_f32(lo)) | (static_cast<uint32_t>(E::from_f32(hi)) << 16);
}

// N consecutive 16-bit elements (N = 2, 4 or 8: 4, 8 or 16 bytes, aligned to
// their size) as 32-bit words; NT: nontemporal load.
typedef unsigned cas_u32x2_t __attribute__((ext_vector_type(2)));
template <int N>
struct Half16 {
  uint32_t w[N / 2];
};
template <int N, bool NT>
__device__ __forceinline__ Half16<N> ld16s(const uint16_t* p) {
  Half16<N> r;
  if constexpr (N == 8) {
    const uint4 u = load16_nt<NT>(p);
    r.w[0] = u.x; r.w[1] = u.y; r.w[2] = u.z; r.w[3] = u.w;
  } else if constexpr (N == 4) {
    cas_u32x2_t u;
    if constexpr (NT) u = __builtin_nontemporal_load(reinterpret_cast<const cas_u32x2_t*>(p));
    else u = *reinterpret_cast<const cas_u32x2_t*>(p);
    r.w[0] = u.x; r.w[1] = u.y;
  } else {
    static_assert(N == 2, "2, 4 or 8 elements");
    if constexpr (NT) r.w[0] = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(p));
    else r.w[0] = *reinterpret_cast<const uint32_t*>(p);
  }
  return r;
}
template <int N, class E>
__device__ __forceinline__ void unpack_h(const Half16<N>& h, float (&x)[N]) {
#pragma unroll
  for (int i = 0; i < N / 2; ++i) {
    x[2 * i] = E::to_f32(static_cast<uint16_t>(h.w[i] & 0xffffu));
    x[2 * i + 1] = E::to_f32(static_cast<uint16_t>(h.w[i] >> 16));
  }
}
// N fp32 values (N = 2, 4 or 8; 8- or 16-byte aligned)
template <int N>
__device__ __forceinline__ void ldf(const float* p, float (&v)[N]) {
  if constexpr (N >= 4) {
#pragma unroll
    for (int c = 0; c < N / 4; ++c) {
      const float4 f = reinterpret_cast<const float4*>(p)[c];
      v[4 * c] = f.x; v[4 * c + 1] = f.y; v[4 * c + 2] = f.z; v[4 * c + 3] = f.w;
    }
  } else {
    static_assert(N == 2, "2, 4 or 8 values");
    const float2 f = *reinterpret_cast<const float2*>(p);
    v[0] = f.x; v[1] = f.y;
  }
}
// N elements of a vector of runtime dtype (fp32, bf16 or fp16) at element e
template <int N>
__device__ __forceinline__ void ld_any_n(const void* p, int dt, int64_t e, float (&v)[N]) {
  if (dt == BFA_DTYPE_F32) {
    ldf<N>(static_cast<const float*>(p) + e, v);
  } else if (dt == BFA_DTYPE_BF16) {
    unpack_h<N, Elem<BFA_DTYPE_BF16>>(ld16s<N, false>(static_cast<const uint16_t*>(p) + e), v);
  } else {
    unpack_h<N, Elem<BFA_DTYPE_F16>>(ld16s<N, false>(static_cast<const uint16_t*>(p) + e), v);
  }
}
// N values stored as 16-bit elements (2, 4 or 8: one 4-, 8- or 16-byte store)
template <int N, bool BF16>
__device__ __forceinline__ void st16s(uint16_t* p, const float (&x)[N]) {
  uint32_t w[N / 2];
#pragma unroll
  for (int i = 0; i < N / 2; ++i) w[i] = pack_pair<BF16>(x[2 * i], x[2 * i + 1]);
  if constexpr (N == 8) *reinterpret_cast<uint4*>(p) = make_uint4(w[0], w[1], w[2], w[3]);
  else if constexpr (N == 4) *reinterpret_cast<uint2*>(p) = make_uint2(w[0], w[1]);
  else *reinterpret_cast<uint32_t*>(p) = w[0];
}

// D = head_dim (64 or 128).  Staging: key row tid / 8, 8 lanes per row, each
// lane EL = D / 16 elements of each half (columns EL c .. and D / 2 + EL c ..,
// the RoPE pairs).  S^T takes D / 32 MFMAs per 16 keys, O^T has D / 16 blocks.
template <bool BF16, int D>
__global__ __launch_bounds__(256) void cascade_attn_kernel(CasArgs a) {
  using E = Elem<BF16 ? BFA_DTYPE_BF16 : BFA_DTYPE_F16>;
  static_assert(D == 64 || D == 128, "head_dim 64 or 128");
  constexpr int EL = D / 16, QJ = D / 32, OJ = D / 16;
  constexpr int KP = D + 8;  // K row pitch in LDS (bf16): conflict-free fragment reads
  __shared__ uint16_t ks[32 * KP];
  __shared__ uint16_t vt[D * CAS_VP];
  __shared__ int64_t kpos_s[32];
  __shared__ int kval_s[32];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t g = blockIdx.y;                                  // kv head
  const int64_t rows = a.tokens * a.group;
  const int64_t row0 = static_cast<int64_t>(blockIdx.x) * 64 + wid * 16;
  const int64_t step0 = static_cast<int64_t>(blockIdx.z) * a.steps_per_split;
  int64_t step1 = min(step0 + a.steps_per_split, a.steps);

  // Q fragments (A operand, 16 rows x 32 head-dim per MFMA): lane holds row
  // lane % 16 and head-dim 32 j + 8 (lane / 16) .. +7 for j < D / 32.
  uint4 qf[QJ];
  {
    const int64_t r = min(row0 + (lane & 15), rows - 1);
    const int64_t t = r / a.group, hh = g * a.group + (r - t * a.group);
    const uint16_t* qrow = a.q + t * a.q_st + hh * a.q_sh;
#pragma unroll
    for (int j = 0; j < QJ; ++j) qf[j] = *reinterpret_cast<const uint4*>(qrow + 32 * j + 8 * (lane >> 4));
  }
  // The matrix work is done transposed: S^T = K Q^T and O^T = V^T P^T, so a lane
  // owns one query row (lane % 16) throughout -- its scores, its running max and
  // sum, and its output columns -- and P^T is already the B operand of the PV
  // product in the registers that hold it.
  const int64_t qt = min(row0 + (lane & 15), rows - 1) / a.group;
  const int64_t qp = a.qpos_i64 ? static_cast<const int64_t*>(a.qpos)[qt]
                                : static_cast<const int32_t*>(a.qpos)[qt];

  const float sl2 = a.scale * 1.4426950408889634f;  // scale x log2(e)
  float m = -INFINITY, l = 0.f;
  cas_f32x4_t o[OJ];  // o[j][i] = O^T[head-dim 16 j + 4 (lane / 16) + i][query lane % 16]
#pragma unroll
  for (int j = 0; j < OJ; ++j) o[j] = cas_f32x4_t{};

  // Staging roles: K and V -- key row tid / 8, head-dim columns EL c .. and
  // D / 2 + EL c .. (c = tid % 8; for K the RoPE pairs).  Loads run ahead of use:
  // the K, V and cos/sin rows of step i+1 are issued before step i's matrix
  // work, and the entry metadata of step i+2 right after them, raw, so that
  // nothing waits on it before step i+1 resolves its slots (the memory counter
  // retires loads in issue order).
  const int sk = tid >> 3, sc = tid & 7;
  float kg1[EL], kg2[EL];  // k_norm weights of this lane's columns
#pragma unroll
  for (int i = 0; i < EL; ++i) kg1[i] = kg2[i] = 1.f;
  if (a.knorm_w) {
    ld_any_n<EL>(a.knorm_w, a.knorm_dt, EL * sc, kg1);
    ld_any_n<EL>(a.knorm_w, a.knorm_dt, D / 2 + EL * sc, kg2);
  }
  struct Meta {  // an entry's metadata as loaded; used only by issue()
    int64_t kst, dpos, s;
    int32_t page, info;
    bool in;
  };
  // Every load below is unconditional (a slot past the range reads entry 0, a
  // masked slot reads cas_zero_row) so that no load sits behind a branch: the
  // memory-counter waits are then exact and a wait for one step's rows does not
  // also wait for the next step's metadata.
  auto load_meta = [&](int64_t step) {
    Meta mt;
    const int64_t slot_g = step * 32 + sk;  // padded key index
    const int64_t e = slot_g / a.page_size;
    mt.s = slot_g - e * a.page_size;
    mt.in = step < step1 && e < a.num_entries;
    const int64_t ec = mt.in ? e : 0;  // num_entries > 0 inside the loop
    mt.page = a.pages[ec];
    mt.kst = a.kstart[ec];
    mt.dpos = a.delta[ec];
    mt.info = a.info[ec];
    return mt;
  };
  struct Buf {
    Half16<EL> k1, k2, v0, v1;
    float c[EL], sn[EL];
    bool valid, rot;
    int64_t kp;
  };
  // resolves a slot (bounds, wrap) and issues its K / V / cos / sin loads
  auto issue = [&](const Meta& mt) {
    Buf b;
    b.valid = mt.in && mt.s < (mt.info & 0xffff);
    const int64_t page = mt.page < 0 ? static_cast<int64_t>(mt.page) + a.num_pages : mt.page;  // kv_cache[-1] is the last page
    if (b.valid && (page < 0 || page >= a.num_pages)) {
      if (sc == 0) flag_status(a.status, BFA_STATUS_INDEX_OOB);
      b.valid = false;
    }
    b.rot = b.valid && a.cs != nullptr && ((mt.info >> 16) & 1);
    int64_t dpos = mt.dpos;
    if (b.rot) {
      if (dpos < 0) dpos += a.max_pos;
      if (dpos < 0 || dpos >= a.max_pos) {
        if (sc == 0) flag_status(a.status, BFA_STATUS_INDEX_OOB);
        b.valid = false;
        b.rot = false;
      }
    }
    b.kp = mt.kst + mt.s;
    const uint16_t* zero = reinterpret_cast<const uint16_t*>(cas_zero_row);
    const uint16_t* krow = b.valid ? a.cache + page * a.c_sp + g * a.c_sh + mt.s * a.c_ss : zero;
    const uint16_t* vrow = b.valid ? krow + a.c_skv : zero;
    b.k1 = ld16s<EL, true>(krow + EL * sc);
    b.k2 = ld16s<EL, true>(krow + D / 2 + EL * sc);
    b.v0 = ld16s<EL, true>(vrow + EL * sc);
    b.v1 = ld16s<EL, true>(vrow + D / 2 + EL * sc);
    const float* csrow = b.rot ? a.cs + dpos * D : cas_zero_row;
    ldf<EL>(csrow + EL * sc, b.c);
    ldf<EL>(csrow + D / 2 + EL * sc, b.sn);
    return b;
  };

  if (step0 >= step1) step1 = step0;  // an empty range (no entries): the loop below does not run
  Buf buf;
  Meta mnext;
  if (step0 < step1) {
    buf = issue(load_meta(step0));
    mnext = load_meta(step0 + 1);
  }
  for (int64_t step = step0; step < step1; ++step) {
    // ---- K row (rotated, normalised) -> LDS
    // (a masked slot loaded zeros; its S column is masked below and its V row
    // must be zero, since 0 x a NaN would poison the sum)
    float x1[EL], x2[EL];
    unpack_h<EL, E>(buf.k1, x1);
    unpack_h<EL, E>(buf.k2, x2);
    if (buf.rot) {
#pragma unroll
      for (int i = 0; i < EL; ++i) {  // apply_rotary_emb: fp32, result in the cache dtype
        const float u = x1[i], w = x2[i];
        x1[i] = E::round(u * buf.c[i] - w * buf.sn[i]);
        x2[i] = E::round(w * buf.c[i] + u * buf.sn[i]);
      }
    }
    if (a.knorm_w) {  // uniform: every lane joins the 8-lane sum (one key row per 8 lanes)
      float ss = 0.f;
#pragma unroll
      for (int i = 0; i < EL; ++i) ss += x1[i] * x1[i] + x2[i] * x2[i];
      ss = group8_sum_dpp(ss);
      const float r = __builtin_amdgcn_rsqf(ss / static_cast<float>(D) + a.knorm_eps);
#pragma unroll
      for (int i = 0; i < EL; ++i) {
        x1[i] = E::round(E::round(x1[i] * r) * kg1[i]);
        x2[i] = E::round(E::round(x2[i] * r) * kg2[i]);
      }
    }
    st16s<EL, BF16>(ks + sk * KP + EL * sc, x1);
    st16s<EL, BF16>(ks + sk * KP + D / 2 + EL * sc, x2);
    // ---- V row -> LDS transposed, in the PV product's key order: the score of
    //      key slot 16 b + 4 g + i sits in lane group g at position 4 b + i of its
    //      8-key B fragment, so that slot is V^T column 8 g + 4 b + i
    {
      const int kc = 8 * ((sk >> 2) & 3) + 4 * (sk >> 4) + (sk & 3);
#pragma unroll
      for (int i = 0; i < EL / 2; ++i) {
        vt[(EL * sc + 2 * i) * CAS_VP + kc] = static_cast<uint16_t>(buf.v0.w[i] & 0xffffu);
        vt[(EL * sc + 2 * i + 1) * CAS_VP + kc] = static_cast<uint16_t>(buf.v0.w[i] >> 16);
        vt[(D / 2 + EL * sc + 2 * i) * CAS_VP + kc] = static_cast<uint16_t>(buf.v1.w[i] & 0xffffu);
        vt[(D / 2 + EL * sc + 2 * i + 1) * CAS_VP + kc] = static_cast<uint16_t>(buf.v1.w[i] >> 16);
      }
    }
    if (sc == 0) {
      kpos_s[sk] = buf.kp;
      kval_s[sk] = buf.valid ? 1 : 0;
    }
    __syncthreads();
    buf = issue(mnext);  // step + 1's rows and step + 2's metadata fly during this step's matrix work
    mnext = load_meta(step + 2);

    // ---- S^T = K Q^T for 2 blocks of 16 keys (A operand: lane holds key row
    //      16 b + lane % 16, head-dim 32 j + 8 (lane / 16) .. +7; B: the query
    //      fragment).  sacc[b][i] = score of key slot 16 b + 4 (lane / 16) + i
    //      for query lane % 16.
    cas_f32x4_t sacc[2];
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      sacc[b] = cas_f32x4_t{};
      const uint16_t* kr = ks + (16 * b + (lane & 15)) * KP + 8 * (lane >> 4);
#pragma unroll
      for (int j = 0; j < QJ; ++j)
        sacc[b] = mfma16x32<BF16>(*reinterpret_cast<const uint4*>(kr + 32 * j), qf[j], sacc[b]);
    }
    // ---- mask, running max / sum.  The running state is kept in base 2: scores
    //      are scaled by scale x log2(e) and exponentiated with v_exp_f32, so m
    //      holds max(s) x log2(e); l and acc are unchanged in meaning.  A query's
    //      32 scores sit in 8 registers of each of 4 lanes (lane % 16 fixed), so
    //      its reductions are in-lane plus two lane swaps.
    float p[2][4];
    float mx = -INFINITY;
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int kk = 16 * b + 4 * (lane >> 4) + i;
        const bool use = kval_s[kk] && (!a.causal || kpos_s[kk] <= qp);
        p[b][i] = use ? sacc[b][i] * sl2 : -INFINITY;
        mx = fmaxf(mx, p[b][i]);
      }
    mx = lanes4_max(mx);
    const float m_new = fmaxf(m, mx);
    const float mref = m_new == -INFINITY ? 0.f : m_new;  // a fully masked row so far stays at 0
    const float alpha = __builtin_amdgcn_exp2f(m - mref);
    float rs = 0.f;
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        p[b][i] = __builtin_amdgcn_exp2f(p[b][i] - mref);
        rs += p[b][i];
      }
    rs = lanes4_sum(rs);
    l = l * alpha + rs;
    m = m_new;
    if (__any(alpha != 1.0f)) {  // the running max moved for some query of the wave
#pragma unroll
      for (int j = 0; j < OJ; ++j) o[j] *= alpha;
    }
    // ---- O^T += V^T P^T (A: V^T rows 16 j + lane % 16, keys 8 (lane / 16) .. +7
    //      in the order V^T was written; B: this lane's 8 probabilities)
    const uint4 pf = make_uint4(pack_pair<BF16>(p[0][0], p[0][1]), pack_pair<BF16>(p[0][2], p[0][3]),
                                pack_pair<BF16>(p[1][0], p[1][1]), pack_pair<BF16>(p[1][2], p[1][3]));
#pragma unroll
    for (int j = 0; j < OJ; ++j) {
      const uint4 vf = *reinterpret_cast<const uint4*>(vt + (16 * j + (lane & 15)) * CAS_VP + 8 * (lane >> 4));
      o[j] = mfma16x32<BF16>(vf, pf, o[j]);
    }
    __syncthreads();  // every wave is done with ks / vt before the next step refills them
  }

  // ---- row out: lane holds head-dim 16 j + 4 (lane / 16) .. +3 of query lane % 16
  const int64_t r = row0 + (lane & 15);
  if (r < rows) {
    const int d0 = 4 * (lane >> 4);
    if (gridDim.z == 1) {
      const int64_t t = r / a.group, hh = g * a.group + (r - t * a.group);
      const float inv = 1.0f / fmaxf(l, 1e-12f);
      uint16_t* orow = static_cast<uint16_t*>(a.out) + t * a.out_st + hh * D;
#pragma unroll
      for (int j = 0; j < OJ; ++j)
        *reinterpret_cast<uint2*>(orow + 16 * j + d0) =
            make_uint2(pack_pair<BF16>(o[j][0] * inv, o[j][1] * inv), pack_pair<BF16>(o[j][2] * inv, o[j][3] * inv));
    } else {
      float* pr = a.part + ((static_cast<int64_t>(blockIdx.z) * a.hkv + g) * rows + r) * (D + 2);
      if (lane < 16) {
        pr[0] = m;
        pr[1] = l;
      }
#pragma unroll
      for (int j = 0; j < OJ; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) pr[2 + 16 * j + d0 + i] = o[j][i];
    }
  }
}

// ======================================================== flat form
// For many query rows every workgroup of cascade_attn_kernel would rotate and
// normalise the same keys again.  The flat form does that once: a pre-pass
// writes the attended keys of each kv head in walk order (padded key slot
// e * page_size + s, tiles of 64) as K rotated and k-normalised, row-major, and
// V transposed (head-dim rows of 64 keys, the keys of each group of 32 in the
// PV product's order), plus each slot's key position (INT32_MAX where the slot
// is past the page's tokens or masked).  The attention kernel then copies K and
// V^T tiles into LDS by DMA (no register staging, no transform) and runs the
// same S^T / O^T scheme on 64 keys per step.
struct FlatArgs {
  uint16_t* kf;     // [Hkv, npad, D]
  uint16_t* vt;     // [Hkv, D, npad]
  int32_t* kpos;    // [npad]
  int64_t npad;     // padded key slots, a multiple of 64
  int64_t tiles_per_split;
};

constexpr int CAS_FT = 64;             // keys per tile of the flat form
constexpr int CAS_FVP = CAS_FT + 8;    // V^T staging row pitch (bf16): 144 bytes

// the PV product's order of key slot k inside its group of 32 (see the V^T
// staging of cascade_attn_kernel)
__device__ __forceinline__ int pv_order(int k) {
  const int sk = k & 31;
  return (k & ~31) + 8 * ((sk >> 2) & 3) + 4 * (sk >> 4) + (sk & 3);
}

template <bool BF16, int D>
__global__ __launch_bounds__(256) void cascade_flatten_kernel(CasArgs a, FlatArgs f) {
  using E = Elem<BF16 ? BFA_DTYPE_BF16 : BFA_DTYPE_F16>;
  constexpr int EL = D / 16;
  __shared__ uint16_t vs[D * CAS_FVP];
  const int tid = threadIdx.x;
  const int64_t g = blockIdx.y;  // kv head
  const int64_t t0 = static_cast<int64_t>(blockIdx.x) * CAS_FT;
  const bool vrole = blockIdx.z == 1;  // z = 0: K (and the positions), z = 1: V^T
  const int sk = tid >> 3, sc = tid & 7;  // key row (and row + 32), column chunk
  float kg1[EL], kg2[EL];
#pragma unroll
  for (int i = 0; i < EL; ++i) kg1[i] = kg2[i] = 1.f;
  if (a.knorm_w && !vrole) {
    ld_any_n<EL>(a.knorm_w, a.knorm_dt, EL * sc, kg1);
    ld_any_n<EL>(a.knorm_w, a.knorm_dt, D / 2 + EL * sc, kg2);
  }
#pragma unroll
  for (int pass = 0; pass < 2; ++pass) {
    const int kk = sk + 32 * pass;
    const int64_t slot = t0 + kk;
    const int64_t e = slot / a.page_size, s = slot - e * a.page_size;
    const bool in = e < a.num_entries;
    const int64_t ec = in ? e : 0;
    int64_t page = a.pages[ec];
    const int64_t kst = a.kstart[ec];
    int64_t dpos = a.delta[ec];
    const int32_t info = a.info[ec];
    bool valid = in && s < (info & 0xffff);
    if (page < 0) page += a.num_pages;  // kv_cache[-1] is the last page
    if (valid && (page < 0 || page >= a.num_pages)) {
      if (sc == 0) flag_status(a.status, BFA_STATUS_INDEX_OOB);
      valid = false;
    }
    bool rot = valid && a.cs != nullptr && ((info >> 16) & 1);
    if (rot) {
      if (dpos < 0) dpos += a.max_pos;
      if (dpos < 0 || dpos >= a.max_pos) {
        if (sc == 0) flag_status(a.status, BFA_STATUS_INDEX_OOB);
        valid = false;
        rot = false;
      }
    }
    const int64_t kp = kst + s;
    if (valid && kp >= INT32_MAX) {  // positions are kept in 32 bits here
      if (sc == 0) flag_status(a.status, BFA_STATUS_INDEX_OOB);
      valid = false;
      rot = false;
    }
    const uint16_t* zero = reinterpret_cast<const uint16_t*>(cas_zero_row);
    const uint16_t* krow = valid ? a.cache + page * a.c_sp + g * a.c_sh + s * a.c_ss : zero;
    if (vrole) {  // V row -> LDS, transposed in the PV order
      const uint16_t* vrow = valid ? krow + a.c_skv : zero;
      float v1[EL], v2[EL];
      unpack_h<EL, E>(ld16s<EL, false>(vrow + EL * sc), v1);
      unpack_h<EL, E>(ld16s<EL, false>(vrow + D / 2 + EL * sc), v2);
      const int kc = pv_order(kk);
#pragma unroll
      for (int i = 0; i < EL; ++i) {
        vs[(EL * sc + i) * CAS_FVP + kc] = E::from_f32(v1[i]);
        vs[(D / 2 + EL * sc + i) * CAS_FVP + kc] = E::from_f32(v2[i]);
      }
      continue;
    }
    float x1[EL], x2[EL];
    unpack_h<EL, E>(ld16s<EL, false>(krow + EL * sc), x1);
    unpack_h<EL, E>(ld16s<EL, false>(krow + D / 2 + EL * sc), x2);
    if (rot) {
      float cs[EL], sn[EL];
      ldf<EL>(a.cs + dpos * D + EL * sc, cs);
      ldf<EL>(a.cs + dpos * D + D / 2 + EL * sc, sn);
#pragma unroll
      for (int i = 0; i < EL; ++i) {  // apply_rotary_emb: fp32, result in the cache dtype
        const float u = x1[i], w = x2[i];
        x1[i] = E::round(u * cs[i] - w * sn[i]);
        x2[i] = E::round(w * cs[i] + u * sn[i]);
      }
    }
    if (a.knorm_w) {  // uniform; a zero row stays zero
      float ss = 0.f;
#pragma unroll
      for (int i = 0; i < EL; ++i) ss += x1[i] * x1[i] + x2[i] * x2[i];
      ss = group8_sum_dpp(ss);
      const float r = __builtin_amdgcn_rsqf(ss / static_cast<float>(D) + a.knorm_eps);
#pragma unroll
      for (int i = 0; i < EL; ++i) {
        x1[i] = E::round(E::round(x1[i] * r) * kg1[i]);
        x2[i] = E::round(E::round(x2[i] * r) * kg2[i]);
      }
    }
    uint16_t* kd = f.kf + (g * f.npad + slot) * D;
    st16s<EL, BF16>(kd + EL * sc, x1);
    st16s<EL, BF16>(kd + D / 2 + EL * sc, x2);
    if (g == 0 && sc == 0) f.kpos[slot] = valid ? static_cast<int32_t>(kp) : INT32_MAX;
  }
  if (!vrole) return;  // uniform over the workgroup
  __syncthreads();
  // V^T tile out: D head-dim rows of 64 keys, 16-byte granules
#pragma unroll
  for (int i = tid; i < D * 8; i += 256) {
    const int d = i >> 3, gr = i & 7;
    *reinterpret_cast<uint4*>(f.vt + (g * D + d) * f.npad + t0 + 8 * gr) =
        *reinterpret_cast<const uint4*>(vs + d * CAS_FVP + 8 * gr);
  }
}

// K tile slot of granule G of row r (rows of GK = D / 8 granules): 256-byte
// rows (D = 128) at G ^ (r & 15), 128-byte rows (D = 64) at G ^ ((r / 2) & 7);
// either way a 16-lane fragment read touches 16 distinct bank groups.
template <int D>
__device__ __forceinline__ int kslot(int r, int gr) {
  if constexpr (D == 128) return gr ^ (r & 15);
  else return gr ^ ((r >> 1) & 7);
}

template <bool BF16, int D>
__global__ __launch_bounds__(256) void cascade_flat_kernel(CasArgs a, FlatArgs f) {
  // K tile: 64 rows of D * 2 bytes (GK granules, slots by kslot); V^T tile: D
  // rows of 128 bytes, granule G of row r at slot G ^ ((r / 2) & 7).
  constexpr int GK = D / 8, QJ = D / 32, OJ = D / 16;
  constexpr int KC = GK / 4;        // 1 KiB K copies per wave (each 64 / GK rows)
  constexpr int VC = D / 32;        // 1 KiB V^T copies per wave (each 8 rows)
  __shared__ uint4 kbuf[2][CAS_FT * GK];
  __shared__ uint4 vbuf[2][D * 8];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t g = blockIdx.y;
  const int64_t rows = a.tokens * a.group;
  const int64_t row0 = static_cast<int64_t>(blockIdx.x) * 64 + wid * 16;
  const int64_t tiles = f.npad / CAS_FT;
  const int64_t tl0 = static_cast<int64_t>(blockIdx.z) * f.tiles_per_split;
  const int64_t tl1 = min(tl0 + f.tiles_per_split, tiles);

  uint4 qf[QJ];
  {
    const int64_t r = min(row0 + (lane & 15), rows - 1);
    const int64_t t = r / a.group, hh = g * a.group + (r - t * a.group);
    const uint16_t* qrow = a.q + t * a.q_st + hh * a.q_sh;
#pragma unroll
    for (int j = 0; j < QJ; ++j) qf[j] = *reinterpret_cast<const uint4*>(qrow + 32 * j + 8 * (lane >> 4));
  }
  const int64_t qt = min(row0 + (lane & 15), rows - 1) / a.group;
  const int64_t qp = a.qpos_i64 ? static_cast<const int64_t*>(a.qpos)[qt]
                                : static_cast<const int32_t*>(a.qpos)[qt];
  const float sl2 = a.scale * 1.4426950408889634f;
  float m = -INFINITY, l = 0.f;
  cas_f32x4_t o[OJ];
#pragma unroll
  for (int j = 0; j < OJ; ++j) o[j] = cas_f32x4_t{};

  // DMA roles per wave: K copy i moves rows (64 / GK) (4 i + wid) .. (lane: row +
  // lane / GK, slot lane % GK); V^T copy i moves rows 8 (4 i + wid) .. +7 (lane:
  // row + lane / 8, slot lane % 8).  Offsets are in bytes from the tile's first
  // element.
  uint32_t koff[KC], voff[VC];
#pragma unroll
  for (int i = 0; i < KC; ++i) {
    const int kr = (64 / GK) * (4 * i + wid) + lane / GK;
    koff[i] = static_cast<uint32_t>((kr * D + 8 * kslot<D>(kr, lane % GK)) * 2);
  }
#pragma unroll
  for (int i = 0; i < VC; ++i) {
    const int vr = 8 * (4 * i + wid) + (lane >> 3);
    voff[i] = static_cast<uint32_t>((vr * f.npad + 8 * ((lane & 7) ^ ((vr >> 1) & 7))) * 2);
  }
  const uint16_t* kbase = f.kf + g * f.npad * D;
  const uint16_t* vbase = f.vt + g * D * f.npad;
  const uint32_t kl = lds_addr(kbuf), vl = lds_addr(vbuf);
  auto issue = [&](int64_t t, int b) {
    const uint16_t* kt = kbase + t * CAS_FT * D;
    const uint16_t* vt = vbase + t * CAS_FT;
#pragma unroll
    for (int i = 0; i < KC; ++i) dma16(kt, koff[i], kl + b * (CAS_FT * GK * 16) + (4 * i + wid) * 1024);
#pragma unroll
    for (int i = 0; i < VC; ++i) dma16(vt, voff[i], vl + b * (D * 128) + (4 * i + wid) * 1024);
  };
  // key positions of this lane's scores: slots 16 b + 4 (lane / 16) .. +3
  auto load_kp = [&](int64_t t, int4 (&kp)[4]) {
#pragma unroll
    for (int b = 0; b < 4; ++b)
      kp[b] = *reinterpret_cast<const int4*>(f.kpos + t * CAS_FT + 16 * b + 4 * (lane >> 4));
  };

  if (tl0 < tl1) {
    int4 kp[4];
    issue(tl0, 0);
    load_kp(tl0, kp);
    wait_vmem();
    __syncthreads();
    for (int64_t t = tl0; t < tl1; ++t) {
      const int b = static_cast<int>((t - tl0) & 1);
      int4 kpn[4] = {kp[0], kp[1], kp[2], kp[3]};
      if (t + 1 < tl1) {  // the next tile flies during this one's matrix work
        issue(t + 1, b ^ 1);
        load_kp(t + 1, kpn);
      }
      // S^T = K Q^T, 4 blocks of 16 keys: sacc[c][i] is the score of key slot
      // 16 c + 4 (lane / 16) + i for query lane % 16
      const uint4* kb = kbuf[b];
      cas_f32x4_t sacc[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        sacc[c] = cas_f32x4_t{};
        const int kr = 16 * c + (lane & 15);
#pragma unroll
        for (int j = 0; j < QJ; ++j)
          sacc[c] = mfma16x32<BF16>(kb[kr * GK + kslot<D>(kr, 4 * j + (lane >> 4))], qf[j], sacc[c]);
      }
      float p[4][4];
      float mx = -INFINITY;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int kq[4] = {kp[c].x, kp[c].y, kp[c].z, kp[c].w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const bool use = kq[i] != INT32_MAX && (!a.causal || kq[i] <= qp);
          p[c][i] = use ? sacc[c][i] * sl2 : -INFINITY;
          mx = fmaxf(mx, p[c][i]);
        }
      }
      mx = lanes4_max(mx);
      const float m_new = fmaxf(m, mx);
      const float mref = m_new == -INFINITY ? 0.f : m_new;
      const float alpha = __builtin_amdgcn_exp2f(m - mref);
      float rs = 0.f;
#pragma unroll
      for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          p[c][i] = __builtin_amdgcn_exp2f(p[c][i] - mref);
          rs += p[c][i];
        }
      rs = lanes4_sum(rs);
      l = l * alpha + rs;
      m = m_new;
      if (__any(alpha != 1.0f)) {
#pragma unroll
        for (int j = 0; j < OJ; ++j) o[j] *= alpha;
      }
      // O^T += V^T P^T over the two groups of 32 keys
      const uint4* vb = vbuf[b];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const uint4 pf = make_uint4(pack_pair<BF16>(p[2 * h][0], p[2 * h][1]), pack_pair<BF16>(p[2 * h][2], p[2 * h][3]),
                                    pack_pair<BF16>(p[2 * h + 1][0], p[2 * h + 1][1]),
                                    pack_pair<BF16>(p[2 * h + 1][2], p[2 * h + 1][3]));
#pragma unroll
        for (int j = 0; j < OJ; ++j) {
          const int vr = 16 * j + (lane & 15);
          o[j] = mfma16x32<BF16>(vb[vr * 8 + ((4 * h + (lane >> 4)) ^ ((vr >> 1) & 7))], pf, o[j]);
        }
      }
      wait_vmem();
      __syncthreads();  // tile t+1 is in LDS everywhere; every wave is done with tile t
#pragma unroll
      for (int c = 0; c < 4; ++c) kp[c] = kpn[c];
    }
  }

  const int64_t r = row0 + (lane & 15);
  if (r < rows) {
    const int d0 = 4 * (lane >> 4);
    if (gridDim.z == 1) {
      const int64_t t = r / a.group, hh = g * a.group + (r - t * a.group);
      const float inv = 1.0f / fmaxf(l, 1e-12f);
      uint16_t* orow = static_cast<uint16_t*>(a.out) + t * a.out_st + hh * D;
#pragma unroll
      for (int j = 0; j < OJ; ++j)
        *reinterpret_cast<uint2*>(orow + 16 * j + d0) =
            make_uint2(pack_pair<BF16>(o[j][0] * inv, o[j][1] * inv), pack_pair<BF16>(o[j][2] * inv, o[j][3] * inv));
    } else {
      float* pr = a.part + ((static_cast<int64_t>(blockIdx.z) * a.hkv + g) * rows + r) * (D + 2);
      if (lane < 16) {
        pr[0] = m;
        pr[1] = l;
      }
#pragma unroll
      for (int j = 0; j < OJ; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) pr[2 + 16 * j + d0 + i] = o[j][i];
    }
  }
}

// Combines the splits' (m, l, acc) rows: one workgroup per (kv head, row).
// Every wave finds the maximum over all splits (lanes over splits); wave w then
// sums splits w, w + 4, ... -- each lane D / 64 head-dim columns, the weights
// broadcast from the lanes that computed them, loads unrolled so they are in
// flight together -- and the four partial sums meet in LDS.  ONE (at most 64
// splits, 16 per wave): every load of the workgroup is requested at once,
// before the maximum, so the combination waits one memory round trip instead
// of three; the sums are the same, in the same order.
template <bool BF16, int D, bool ONE>
__global__ __launch_bounds__(256) void cascade_merge_kernel(CasArgs a, int64_t splits) {
  using E = Elem<BF16 ? BFA_DTYPE_BF16 : BFA_DTYPE_F16>;
  constexpr int NC = D / 64;  // columns per lane
  __shared__ float red[4][D + 1];
  const int64_t rows = a.tokens * a.group;
  const int64_t item = blockIdx.x;
  const int64_t g = item / rows, r = item - g * rows;
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int64_t zstride = a.hkv * rows * (D + 2);
  const float* base = a.part + (g * rows + r) * (D + 2);
  float lsum = 0.f, oc[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) oc[c] = 0.f;
  if constexpr (ONE) {
    // lane z: split z's m for the maximum; lane k < 16: m and l of this
    // wave's k-th split (4 k + wid); ac[u]: this lane's columns of split
    // 4 u + wid (index clamped, its weight is then 0)
    const int64_t zk = 4 * lane + wid;
    const float* pz = base + min<int64_t>(lane, splits - 1) * zstride;
    const float* pk = base + min<int64_t>(zk, splits - 1) * zstride;
    const float mlane = pz[0], mk = pk[0], lk = pk[1];
    float ac[16][NC];
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const float* pr = base + min<int64_t>(4 * u + wid, splits - 1) * zstride + 2;
#pragma unroll
      for (int c = 0; c < NC; ++c) ac[u][c] = pr[64 * c + lane];
    }
    const float mx = lanes4_max(group16_max_dpp(lane < splits ? mlane : -INFINITY));
    float w = 0.f;
    if (lane < 16 && zk < splits) {
      w = mk == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mk - mx);  // m is kept in base 2
      lsum = w * lk;
    }
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const float wu = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), u));
#pragma unroll
      for (int c = 0; c < NC; ++c) oc[c] += wu * ac[u][c];
    }
  } else {
    float mx = -INFINITY;
    for (int64_t z = lane; z < splits; z += 64) mx = fmaxf(mx, base[z * zstride]);
    mx = lanes4_max(group16_max_dpp(mx));  // DPP and lane swaps, no LDS round trips
    // this wave's splits: z = wid + 4 k; lane k holds the weight of the k-th
    for (int64_t k0 = 0; 4 * k0 + wid < splits; k0 += 64) {
      const int64_t z = 4 * (k0 + lane) + wid;
      float w = 0.f;
      if (z < splits) {
        const float mz = base[z * zstride];
        w = mz == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mz - mx);  // m is kept in base 2
        lsum += w * base[z * zstride + 1];
      }
      // a lane past the wave's last split holds w = 0; its row index is clamped
      const int64_t nk = min<int64_t>(64, (splits - wid + 3) / 4 - k0);
      const int nk8 = static_cast<int>((nk + 7) & ~7);
      for (int j0 = 0; j0 < nk8; j0 += 8) {
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          // lane j0 + u's weight, read out as a scalar (the index is wave-uniform)
          const float wj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), j0 + u));
          const int64_t zj = min<int64_t>(4 * (k0 + j0 + u) + wid, splits - 1);
          const float* pr = base + zj * zstride + 2;
#pragma unroll
          for (int c = 0; c < NC; ++c) oc[c] += wj * pr[64 * c + lane];
        }
      }
    }
  }
  lsum = group_sum<kWave>(lsum);
#pragma unroll
  for (int c = 0; c < NC; ++c) red[wid][64 * c + lane] = oc[c];
  if (lane == 0) red[wid][D] = lsum;
  __syncthreads();
  if (wid != 0) return;
  lsum = red[0][D] + red[1][D] + red[2][D] + red[3][D];
  const float inv = 1.0f / fmaxf(lsum, 1e-12f);
  const int64_t t = r / a.group, hh = g * a.group + (r - t * a.group);
  uint16_t* orow = static_cast<uint16_t*>(a.out) + t * a.out_st + hh * D;
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int col = 64 * c + lane;
    orow[col] = E::from_f32((red[0][col] + red[1][col] + red[2][col] + red[3][col]) * inv);
  }
}

// The same combination for at most ZMAX (4, 8 or 16) splits: one wave per
// (kv head, row), 4 rows per workgroup; every split's (m, l) and this lane's
// columns are requested together (indices clamped, weights of absent splits
// zero, so the sums match those of a larger ZMAX bit for bit).
template <bool BF16, int D, int ZMAX>
__global__ __launch_bounds__(256) void cascade_merge_small_kernel(CasArgs a, int64_t splits) {
  using E = Elem<BF16 ? BFA_DTYPE_BF16 : BFA_DTYPE_F16>;
  constexpr int NC = D / 64;
  const int64_t rows = a.tokens * a.group;
  const int64_t item = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (item >= a.hkv * rows) return;
  const int64_t g = item / rows, r = item - g * rows;
  const int lane = threadIdx.x & 63;
  const int64_t zstride = a.hkv * rows * (D + 2);
  const float* base = a.part + (g * rows + r) * (D + 2);
  float mz[ZMAX], lz[ZMAX], ac[ZMAX][NC];
#pragma unroll
  for (int z = 0; z < ZMAX; ++z) {
    const float* pz = base + min<int64_t>(z, splits - 1) * zstride;
    mz[z] = pz[0];
    lz[z] = pz[1];
#pragma unroll
    for (int c = 0; c < NC; ++c) ac[z][c] = pz[2 + 64 * c + lane];
  }
  float mx = -INFINITY;
#pragma unroll
  for (int z = 0; z < ZMAX; ++z) mx = fmaxf(mx, z < splits ? mz[z] : -INFINITY);
  const float mref = mx == -INFINITY ? 0.f : mx;
  float lsum = 0.f, oc[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) oc[c] = 0.f;
#pragma unroll
  for (int z = 0; z < ZMAX; ++z) {
    const float w = z < splits ? __builtin_amdgcn_exp2f(mz[z] - mref) : 0.f;  // m in base 2; -inf -> 0
    lsum += w * lz[z];
#pragma unroll
    for (int c = 0; c < NC; ++c) oc[c] += w * ac[z][c];
  }
  const float inv = 1.0f / fmaxf(lsum, 1e-12f);
  const int64_t t = r / a.group, hh = g * a.group + (r - t * a.group);
  uint16_t* orow = static_cast<uint16_t*>(a.out) + t * a.out_st + hh * D;
#pragma unroll
  for (int c = 0; c < NC; ++c) orow[64 * c + lane] = E::from_f32(oc[c] * inv);
}

// Decode form (at most 4 query rows per kv head): scores on the VALU.  A
// workgroup's 16 groups of 16 lanes walk its range of (entry, 16-slot block)
// items; group kg takes slot 16 sb + kg of each item, lane j holds head-dim
// EH j .. and D / 2 + EH j .. (EH = D / 32 each: the RoPE pairs), and each group
// keeps its own online-softmax state for every row, so the walk needs no
// barrier.  The next item's metadata and K / V / cos-sin rows load while the
// current one is processed.  At the end the 16 group states meet in LDS and are
// combined into the split's (m, l, acc) rows -- the layout the merge kernel
// reads -- or, with one split, into the output.
template <bool BF16, int R, int D>
__global__ __launch_bounds__(256) void cascade_decode_kernel(CasArgs a, int64_t items_per_split, int64_t nsb) {
  using E = Elem<BF16 ? BFA_DTYPE_BF16 : BFA_DTYPE_F16>;
  constexpr int NG = 16, EH = D / 32, NU = 4;  // NU: most items per workgroup taken at once
  __shared__ float red_m[NG][R], red_l[NG][R];
  __shared__ float red_a[NG][R][D];
  const int tid = threadIdx.x, j = tid & 15, kg = tid >> 4;
  const int64_t g = blockIdx.x;  // kv head
  const int64_t rows = a.tokens * a.group;
  const int64_t items = a.num_entries * nsb;
  const int64_t i0 = static_cast<int64_t>(blockIdx.y) * items_per_split;
  const int64_t i1 = min(i0 + items_per_split, items);

  // queries (fp32 copies of the bf16 / fp16 values) and their positions
  float q1[R][EH], q2[R][EH];
  int64_t qp[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int64_t rr = min<int64_t>(r, rows - 1);
    const int64_t t = rr / a.group, hh = g * a.group + (rr - t * a.group);
    const uint16_t* qrow = a.q + t * a.q_st + hh * a.q_sh;
    unpack_h<EH, E>(ld16s<EH, false>(qrow + EH * j), q1[r]);
    unpack_h<EH, E>(ld16s<EH, false>(qrow + D / 2 + EH * j), q2[r]);
    qp[r] = a.qpos_i64 ? static_cast<const int64_t*>(a.qpos)[t] : static_cast<const int32_t*>(a.qpos)[t];
  }
  float kw1[EH], kw2[EH];
#pragma unroll
  for (int i = 0; i < EH; ++i) kw1[i] = kw2[i] = 1.f;
  if (a.knorm_w) {  // one uniform dtype branch, vector loads
    ld_any_n<EH>(a.knorm_w, a.knorm_dt, EH * j, kw1);
    ld_any_n<EH>(a.knorm_w, a.knorm_dt, D / 2 + EH * j, kw2);
  }
  const float sl2 = a.scale * 1.4426950408889634f;
  float m[R], l[R], acc1[R][EH], acc2[R][EH];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    m[r] = -INFINITY;
    l[r] = 0.f;
#pragma unroll
    for (int i = 0; i < EH; ++i) acc1[r][i] = acc2[r][i] = 0.f;
  }

  // An item's metadata as loaded (used only by issue(), an item later), and the
  // group's slot of an item resolved with its loads issued.  Masked slots read
  // the zeroed row, so no load waits behind a branch.
  struct Meta {
    int64_t kst, dpos, sl;
    int32_t pg, info;
    bool in;
  };
  struct Slot {
    Half16<EH> k1, k2, v1, v2;
    float c[EH], sn[EH];
    int64_t kp;
    bool valid, rot;
  };
  auto load_meta = [&](int64_t it) {
    Meta mt;
    const int64_t e = it / nsb, sb = it - e * nsb;
    mt.in = it < i1;
    // the entry index in a vector register: its loads are then vector loads,
    // which complete in order, so the wait for an item's metadata (two items
    // ahead) does not also wait for later ones, as out-of-order scalar loads
    // would (Qwen3 decode over 4096 keys 13.6 -> 13.35 us)
    int64_t ec = mt.in ? e : 0;
    asm volatile("" : "+v"(ec));
    mt.pg = a.pages[ec];
    mt.kst = a.kstart[ec];
    mt.dpos = a.delta[ec];
    mt.info = a.info[ec];
    mt.sl = 16 * sb + kg;
    return mt;
  };
  auto issue = [&](const Meta& mt) {
    Slot b;
    const bool in = mt.in;
    const int32_t pg = mt.pg, info = mt.info;
    const int64_t kst = mt.kst, sl = mt.sl;
    int64_t dpos = mt.dpos;
    b.valid = in && sl < (info & 0xffff);
    const int64_t page = pg < 0 ? static_cast<int64_t>(pg) + a.num_pages : pg;  // kv_cache[-1] is the last page
    if (b.valid && (page < 0 || page >= a.num_pages)) {
      if (j == 0) flag_status(a.status, BFA_STATUS_INDEX_OOB);
      b.valid = false;
    }
    b.rot = b.valid && a.cs != nullptr && ((info >> 16) & 1);
    if (b.rot) {
      if (dpos < 0) dpos += a.max_pos;
      if (dpos < 0 || dpos >= a.max_pos) {
        if (j == 0) flag_status(a.status, BFA_STATUS_INDEX_OOB);
        b.valid = false;
        b.rot = false;
      }
    }
    b.kp = kst + sl;
    const uint16_t* zero = reinterpret_cast<const uint16_t*>(cas_zero_row);
    const uint16_t* krow = b.valid ? a.cache + page * a.c_sp + g * a.c_sh + sl * a.c_ss : zero;
    const uint16_t* vrow = b.valid ? krow + a.c_skv : zero;
    b.k1 = ld16s<EH, false>(krow + EH * j);
    b.k2 = ld16s<EH, false>(krow + D / 2 + EH * j);
    b.v1 = ld16s<EH, false>(vrow + EH * j);
    b.v2 = ld16s<EH, false>(vrow + D / 2 + EH * j);
    const float* csrow = b.rot ? a.cs + dpos * D : cas_zero_row;
    ldf<EH>(csrow + EH * j, b.c);
    ldf<EH>(csrow + D / 2 + EH * j, b.sn);
    return b;
  };

  // one item into the group's online-softmax states
  auto consume = [&](const Slot& cur) {
    float x1[EH], x2[EH];
    unpack_h<EH, E>(cur.k1, x1);
    unpack_h<EH, E>(cur.k2, x2);
    if (cur.rot) {
#pragma unroll
      for (int i = 0; i < EH; ++i) {  // apply_rotary_emb: fp32, result in the cache dtype
        const float u = x1[i], w = x2[i];
        x1[i] = E::round(u * cur.c[i] - w * cur.sn[i]);
        x2[i] = E::round(w * cur.c[i] + u * cur.sn[i]);
      }
    }
    if (a.knorm_w) {  // uniform: every lane joins its group's 16-lane sum
      float ss = 0.f;
#pragma unroll
      for (int i = 0; i < EH; ++i) ss += x1[i] * x1[i] + x2[i] * x2[i];
      ss = group16_sum_dpp(ss);
      const float rn = __builtin_amdgcn_rsqf(ss / static_cast<float>(D) + a.knorm_eps);
#pragma unroll
      for (int i = 0; i < EH; ++i) {
        x1[i] = E::round(E::round(x1[i] * rn) * kw1[i]);
        x2[i] = E::round(E::round(x2[i] * rn) * kw2[i]);
      }
    }
    float v1[EH], v2[EH];
    unpack_h<EH, E>(cur.v1, v1);
    unpack_h<EH, E>(cur.v2, v2);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      float d = 0.f;
#pragma unroll
      for (int i = 0; i < EH; ++i) d += q1[r][i] * x1[i] + q2[r][i] * x2[i];
      d = group16_sum_dpp(d);
      const bool use = cur.valid && (!a.causal || cur.kp <= qp[r]);
      const float sc = use ? d * sl2 : -INFINITY;
      const float m_new = fmaxf(m[r], sc);
      const float mref = m_new == -INFINITY ? 0.f : m_new;  // nothing seen yet: stay at zero
      const float alpha = __builtin_amdgcn_exp2f(m[r] - mref);
      const float pr = __builtin_amdgcn_exp2f(sc - mref);
      l[r] = l[r] * alpha + pr;
      m[r] = m_new;
#pragma unroll
      for (int i = 0; i < EH; ++i) {
        acc1[r][i] = acc1[r][i] * alpha + pr * v1[i];
        acc2[r][i] = acc2[r][i] * alpha + pr * v2[i];
      }
    }
  };

  if (i0 < i1) {
    if (items_per_split > 1 && items_per_split <= NU) {
      // Few items: every item's metadata, then every item's rows, requested
      // at once -- two memory round trips in all, where the pipelined walk
      // waits about one per item.  Slots past i1 load the zeroed row and are
      // not consumed (a uniform branch).  Qwen3 decode over 4096 keys: 4 items
      // per workgroup, 12.1 -> 11.6 us.
      Meta mt[NU];
#pragma unroll
      for (int u = 0; u < NU; ++u) mt[u] = load_meta(i0 + u);
      Slot sv[NU];
#pragma unroll
      for (int u = 0; u < NU; ++u) sv[u] = issue(mt[u]);
#pragma unroll
      for (int u = 0; u < NU; ++u)
        if (i0 + u < i1) consume(sv[u]);
    } else {
      Slot cur = issue(load_meta(i0));
      Meta mn = load_meta(i0 + 1);
      for (int64_t it = i0; it < i1; ++it) {
        const Slot nxt = issue(mn);  // item it + 1's rows fly while this item is processed,
        mn = load_meta(it + 2);      // and item it + 2's metadata
        consume(cur);
        cur = nxt;
      }
    }
  }
  // ---- the 16 group states -> one state per row
#pragma unroll
  for (int r = 0; r < R; ++r) {
    if (j == 0) {
      red_m[kg][r] = m[r];
      red_l[kg][r] = l[r];
    }
#pragma unroll
    for (int i = 0; i < EH; ++i) {
      red_a[kg][r][EH * j + i] = acc1[r][i];
      red_a[kg][r][D / 2 + EH * j + i] = acc2[r][i];
    }
  }
  __syncthreads();
  for (int idx = tid; idx < R * D; idx += 256) {
    const int r = idx / D, dcol = idx - r * D;
    if (r >= rows) break;
    float mx = -INFINITY;
#pragma unroll
    for (int q = 0; q < NG; ++q) mx = fmaxf(mx, red_m[q][r]);
    const float mref = mx == -INFINITY ? 0.f : mx;
    float lsum = 0.f, asum = 0.f;
#pragma unroll
    for (int q = 0; q < NG; ++q) {
      const float w = __builtin_amdgcn_exp2f(red_m[q][r] - mref);  // -inf -> 0
      lsum += red_l[q][r] * w;
      asum += red_a[q][r][dcol] * w;
    }
    if (gridDim.y == 1) {
      const int64_t t = r / a.group, hh = g * a.group + (r - t * a.group);
      static_cast<uint16_t*>(a.out)[t * a.out_st + hh * D + dcol] = E::from_f32(asum / fmaxf(lsum, 1e-12f));
    } else {
      float* pr = a.part + ((static_cast<int64_t>(blockIdx.y) * a.hkv + g) * rows + r) * (D + 2);
      if (dcol == 0) {
        pr[0] = mx;
        pr[1] = lsum;
      }
      pr[2 + dcol] = asum;
    }
  }
}

// ========================================= other head dims (multiple of 4, <= 256)
// One wave per (query row, kv head, key split).  The wave walks its entries'
// slots in blocks of 8 keys; lane l holds head-dim columns 2l, 2l + 1 and their
// RoPE partners D/2 + 2l, D/2 + 2l + 1 (lanes past D/4 idle), so the rotation
// needs no exchange, and the k_norm sum and each score are wave sums on DPP.
// Lanes 0-7 fetch the block's slot metadata; the next block's metadata and its
// K / V / cos-sin values are requested before the current block is processed.
// Same rounding points as the head_dim 64 / 128 kernels; the split's (m, l,
// acc) rows go to the partial layout, or with one split to the output.
constexpr int CAS_GEN_DMAX = 256;

template <bool BF16>
__global__ __launch_bounds__(256) void cascade_generic_kernel(CasArgs a, int64_t D, int64_t ent_per_split) {
  using E = Elem<BF16 ? BFA_DTYPE_BF16 : BFA_DTYPE_F16>;
  constexpr int KB = 8;  // keys per block
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int64_t rows = a.tokens * a.group;
  const int64_t r = static_cast<int64_t>(blockIdx.x) * 4 + wid;
  if (r >= rows) return;  // whole waves
  const int64_t g = blockIdx.y;
  const int64_t e0 = static_cast<int64_t>(blockIdx.z) * ent_per_split;
  const int64_t e1 = min(e0 + ent_per_split, a.num_entries);
  const int64_t half = D / 2;
  const bool act = 2 * lane < half;
  const int64_t c0 = act ? 2 * lane : 0;  // idle lanes read column 0 and contribute nothing
  const int64_t ps = a.page_size;
  const int64_t t = r / a.group, hh = g * a.group + (r - t * a.group);
  const float sl2 = a.scale * 1.4426950408889634f;  // scale x log2(e)
  float q1[2], q2[2];
  {
    const uint16_t* qrow = a.q + t * a.q_st + hh * a.q_sh;
    unpack_h<2, E>(ld16s<2, false>(qrow + c0), q1);
    unpack_h<2, E>(ld16s<2, false>(qrow + half + c0), q2);
    if (!act) q1[0] = q1[1] = q2[0] = q2[1] = 0.f;
  }
  const int64_t qp = a.qpos_i64 ? static_cast<const int64_t*>(a.qpos)[t] : static_cast<const int32_t*>(a.qpos)[t];
  float kg1[2] = {1.f, 1.f}, kg2[2] = {1.f, 1.f};
  if (a.knorm_w) {
    ld_any_n<2>(a.knorm_w, a.knorm_dt, c0, kg1);
    ld_any_n<2>(a.knorm_w, a.knorm_dt, half + c0, kg2);
  }
  // block b covers padded slots (e0 * ps + b * KB) .. +KB; lane u < KB fetches
  // slot u's entry metadata (a slot past the range reads entry 0 and is masked)
  struct Meta {
    int32_t page, info;
    int64_t kst, dpos, s;
    bool in;
  };
  const int64_t nslots = (e1 > e0 ? e1 - e0 : 0) * ps;
  auto load_meta = [&](int64_t b) {
    Meta mt;
    const int64_t j = b * KB + (lane & (KB - 1));
    const int64_t e = e0 + j / ps;
    mt.s = j - (j / ps) * ps;
    mt.in = j < nslots;
    const int64_t ec = mt.in ? e : 0;
    mt.page = a.pages[ec];
    mt.kst = a.kstart[ec];
    mt.dpos = a.delta[ec];
    mt.info = a.info[ec];
    return mt;
  };
  struct Blk {
    Half16<2> k1[KB], k2[KB], v1[KB], v2[KB];
    float c[KB][2], sn[KB][2];
    bool valid[KB], rot[KB];
    int64_t kp[KB];
  };
  const uint16_t* zero = reinterpret_cast<const uint16_t*>(cas_zero_row);
  auto rd64 = [](int64_t v, int u) {
    const uint32_t lo = __builtin_amdgcn_readlane(static_cast<uint32_t>(v), u);
    const uint32_t hi = __builtin_amdgcn_readlane(static_cast<uint32_t>(static_cast<uint64_t>(v) >> 32), u);
    return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
  };
  auto issue = [&](const Meta& mt) {
    Blk b;
#pragma unroll
    for (int u = 0; u < KB; ++u) {
      const bool in = __builtin_amdgcn_readlane(static_cast<int>(mt.in), u) != 0;
      int64_t page = __builtin_amdgcn_readlane(mt.page, u);
      const int32_t info = __builtin_amdgcn_readlane(mt.info, u);
      const int64_t sl = rd64(mt.s, u);
      int64_t dpos = rd64(mt.dpos, u);
      bool valid = in && sl < (info & 0xffff);
      if (page < 0) page += a.num_pages;  // kv_cache[-1] is the last page
      if (valid && (page < 0 || page >= a.num_pages)) {
        if (lane == 0) flag_status(a.status, BFA_STATUS_INDEX_OOB);
        valid = false;
      }
      bool rot = valid && a.cs != nullptr && ((info >> 16) & 1);
      if (rot) {
        if (dpos < 0) dpos += a.max_pos;
        if (dpos < 0 || dpos >= a.max_pos) {
          if (lane == 0) flag_status(a.status, BFA_STATUS_INDEX_OOB);
          valid = rot = false;
        }
      }
      b.valid[u] = valid;
      b.rot[u] = rot;
      b.kp[u] = rd64(mt.kst, u) + sl;
      const uint16_t* krow = valid ? a.cache + page * a.c_sp + g * a.c_sh + sl * a.c_ss : zero;
      const uint16_t* vrow = valid ? krow + a.c_skv : zero;
      const int64_t cc = valid ? c0 : 0;  // the zeroed row is only CAS_DMAX floats long
      b.k1[u] = ld16s<2, true>(krow + cc);
      b.k2[u] = ld16s<2, true>(krow + (valid ? half : 0) + cc);
      b.v1[u] = ld16s<2, true>(vrow + cc);
      b.v2[u] = ld16s<2, true>(vrow + (valid ? half : 0) + cc);
      const float* csrow = rot ? a.cs + dpos * D : cas_zero_row;
      ldf<2>(csrow + (rot ? c0 : 0), b.c[u]);
      ldf<2>(csrow + (rot ? half + c0 : 0), b.sn[u]);
    }
    return b;
  };
  float m = -INFINITY, l = 0.f, acc1[2] = {0.f, 0.f}, acc2[2] = {0.f, 0.f};
  const int64_t nb = cdiv(nslots, KB);
  if (nb > 0) {
    Blk cur = issue(load_meta(0));
    Meta mn = load_meta(1);
    for (int64_t b = 0; b < nb; ++b) {
      const Blk nxt = issue(mn);  // block b + 1's values fly while block b is processed
      mn = load_meta(b + 2);
#pragma unroll
      for (int u = 0; u < KB; ++u) {
        float x1[2], x2[2], v1[2], v2[2];
        unpack_h<2, E>(cur.k1[u], x1);
        unpack_h<2, E>(cur.k2[u], x2);
        unpack_h<2, E>(cur.v1[u], v1);
        unpack_h<2, E>(cur.v2[u], v2);
        if (cur.rot[u]) {
#pragma unroll
          for (int i = 0; i < 2; ++i) {  // apply_rotary_emb: fp32, result in the cache dtype
            const float p = x1[i], w = x2[i];
            x1[i] = E::round(p * cur.c[u][i] - w * cur.sn[u][i]);
            x2[i] = E::round(w * cur.c[u][i] + p * cur.sn[u][i]);
          }
        }
        if (!act) x1[0] = x1[1] = x2[0] = x2[1] = 0.f;
        if (a.knorm_w) {
          const float ss = wave_sum_dpp(x1[0] * x1[0] + x1[1] * x1[1] + x2[0] * x2[0] + x2[1] * x2[1]);
          const float rr = __builtin_amdgcn_rsqf(ss / static_cast<float>(D) + a.knorm_eps);
#pragma unroll
          for (int i = 0; i < 2; ++i) {
            x1[i] = E::round(E::round(x1[i] * rr) * kg1[i]);
            x2[i] = E::round(E::round(x2[i] * rr) * kg2[i]);
          }
        }
        const float d = wave_sum_dpp(q1[0] * x1[0] + q1[1] * x1[1] + q2[0] * x2[0] + q2[1] * x2[1]);
        const bool use = cur.valid[u] && (!a.causal || cur.kp[u] <= qp);
        const float sc = use ? d * sl2 : -INFINITY;
        const float m_new = fmaxf(m, sc);
        const float mref = m_new == -INFINITY ? 0.f : m_new;  // nothing seen yet: stay at zero
        const float alpha = __builtin_amdgcn_exp2f(m - mref);
        const float pr = __builtin_amdgcn_exp2f(sc - mref);
        l = l * alpha + pr;
        m = m_new;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          acc1[i] = acc1[i] * alpha + pr * v1[i];
          acc2[i] = acc2[i] * alpha + pr * v2[i];
        }
      }
      cur = nxt;
    }
  }
  if (gridDim.z == 1) {
    if (act) {
      const float inv = 1.0f / fmaxf(l, 1e-12f);
      uint16_t* orow = static_cast<uint16_t*>(a.out) + t * a.out_st + hh * D;
      const float o1[2] = {acc1[0] * inv, acc1[1] * inv}, o2[2] = {acc2[0] * inv, acc2[1] * inv};
      st16s<2, BF16>(orow + c0, o1);
      st16s<2, BF16>(orow + half + c0, o2);
    }
  } else {
    float* pr = a.part + ((static_cast<int64_t>(blockIdx.z) * a.hkv + g) * rows + r) * (D + 2);
    if (lane == 0) {
      pr[0] = m;
      pr[1] = l;
    }
    if (act) {
      pr[2 + c0] = acc1[0];
      pr[2 + c0 + 1] = acc1[1];
      pr[2 + half + c0] = acc2[0];
      pr[2 + half + c0 + 1] = acc2[1];
    }
  }
}

// Split combination for any head_dim: one wave per (kv head, row), the splits
// walked in order (lanes over head-dim columns).
template <bool BF16>
__global__ __launch_bounds__(256) void cascade_merge_generic_kernel(CasArgs a, int64_t D, int64_t splits) {
  using E = Elem<BF16 ? BFA_DTYPE_BF16 : BFA_DTYPE_F16>;
  const int64_t rows = a.tokens * a.group;
  const int64_t item = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (item >= a.hkv * rows) return;
  const int64_t g = item / rows, r = item - g * rows;
  const int lane = threadIdx.x & 63;
  const int64_t zstride = a.hkv * rows * (D + 2);
  const float* base = a.part + (g * rows + r) * (D + 2);
  float mx = -INFINITY;
  for (int64_t z = 0; z < splits; ++z) mx = fmaxf(mx, base[z * zstride]);
  const float mref = mx == -INFINITY ? 0.f : mx;
  float lsum = 0.f, oc[CAS_GEN_DMAX / 64] = {0.f, 0.f, 0.f, 0.f};
  for (int64_t z = 0; z < splits; ++z) {
    const float* pz = base + z * zstride;
    const float w = __builtin_amdgcn_exp2f(pz[0] - mref);  // m in base 2; -inf -> 0
    lsum += w * pz[1];
#pragma unroll
    for (int c = 0; c < CAS_GEN_DMAX / 64; ++c)
      if (64 * c + lane < D) oc[c] += w * pz[2 + 64 * c + lane];
  }
  const float inv = 1.0f / fmaxf(lsum, 1e-12f);
  const int64_t t = r / a.group, hh = g * a.group + (r - t * a.group);
  uint16_t* orow = static_cast<uint16_t*>(a.out) + t * a.out_st + hh * D;
#pragma unroll
  for (int c = 0; c < CAS_GEN_DMAX / 64; ++c)
    if (64 * c + lane < D) orow[64 * c + lane] = E::from_f32(oc[c] * inv);
}

// Split plan of the other head dims: about 4096 waves (16 per CU).
struct GenericSplit {
  int64_t per_split, splits;
};
static GenericSplit generic_split(int64_t rows, int64_t hkv, int64_t num_entries) {
  GenericSplit gs{};
  const int64_t want = std::max<int64_t>(1, std::min<int64_t>(num_entries, cdiv(4096, rows * hkv)));
  gs.per_split = std::max<int64_t>(1, cdiv(num_entries, want));
  gs.splits = num_entries > 0 ? cdiv(num_entries, gs.per_split) : 1;
  return gs;
}

static bool mfma_head_dim(int64_t d) { return d == 64 || d == 128; }

// Split plan of the decode form: items of (entry, 16-slot block), about 512
// workgroups over the kv heads (Qwen3 decode over 4096 keys: 25 / 15.9 / 13.6 /
// 15.1 / 20.5 us at 128 / 256 / 512 / 1024 / 2048 -- fewer leave SIMDs idle,
// more pay each workgroup's two dependent memory levels and the merge of more
// splits for less work).
struct DecodeSplit {
  int64_t nsb, items, per_split, splits;
};
static DecodeSplit decode_split(int64_t hkv, int64_t num_entries, int64_t page_size) {
  DecodeSplit d{};
  d.nsb = cdiv(page_size, 16);
  d.items = num_entries * d.nsb;
  int64_t target = 512;
  if (tuning(BFA_TUNE_CASCADE_DECODE_WG) >= 1) target = tuning(BFA_TUNE_CASCADE_DECODE_WG);  // planner override
  const int64_t want = std::max<int64_t>(1, std::min<int64_t>(d.items, cdiv(target, hkv)));
  d.per_split = std::max<int64_t>(1, cdiv(d.items, want));
  d.splits = d.items > 0 ? cdiv(d.items, d.per_split) : 1;
  return d;
}

static bool decode_form(int64_t rows) { return rows <= 4; }

// Calls f(bf16 tag, head_dim tag) for the cache dtype and head_dim (64 or 128).
template <class F>
static void dispatch_dtype_hd(int dtype, int64_t head_dim, F&& f) {
  using D64 = std::integral_constant<int, 64>;
  using D128 = std::integral_constant<int, 128>;
  if (dtype == BFA_DTYPE_BF16) {
    if (head_dim == 64) f(std::true_type{}, D64{}); else f(std::true_type{}, D128{});
  } else {
    if (head_dim == 64) f(std::false_type{}, D64{}); else f(std::false_type{}, D128{});
  }
}

// Split combination: a wave per row up to 16 splits (its load count sized for
// 4, 8 or 16: TinyLlama over 2048 keys, 256 queries, 4 splits 32.4 -> 28.5 us), a
// workgroup per row above (all loads in one round trip up to 64 splits).
template <bool BF16, int D>
static void launch_merge(const CasArgs& a, int64_t rows, int64_t splits, hipStream_t s) {
  const int64_t items = a.hkv * rows;
  const dim3 sgrid(static_cast<unsigned>(cdiv(items, 4)));
  if (splits <= 4) {
    hipLaunchKernelGGL((cascade_merge_small_kernel<BF16, D, 4>), sgrid, dim3(256), 0, s, a, splits);
  } else if (splits <= 8) {
    hipLaunchKernelGGL((cascade_merge_small_kernel<BF16, D, 8>), sgrid, dim3(256), 0, s, a, splits);
  } else if (splits <= 16) {
    hipLaunchKernelGGL((cascade_merge_small_kernel<BF16, D, 16>), sgrid, dim3(256), 0, s, a, splits);
  } else if (splits <= 64) {
    hipLaunchKernelGGL((cascade_merge_kernel<BF16, D, true>), dim3(static_cast<unsigned>(items)), dim3(256), 0, s,
                       a, splits);
  } else {
    hipLaunchKernelGGL((cascade_merge_kernel<BF16, D, false>), dim3(static_cast<unsigned>(items)), dim3(256), 0, s,
                       a, splits);
  }
}

// The flat form, from more than CAS_FLAT_ROWS query rows per kv head (or as
// override BFA_TUNE_CASCADE_FLAT = 0 / 1 forces, for measurements).  At Qwen3 shape over 4096
// keys it is slower than the fused kernel up to 64 rows (26.3 against 25.3 us)
// and faster from 128 (28.5 against 32.7; 42.3 against 79.4 at 512 rows).
// Workspace after the split partials: K and V^T copies of the attended keys and
// their positions.
constexpr int64_t CAS_FLAT_ROWS = 96;

static bool flat_form(int64_t rows, int64_t num_entries) {
  if (num_entries <= 0) return false;
  const int forced = tuning(BFA_TUNE_CASCADE_FLAT);  // planner override
  if (forced >= 0) return forced != 0 && rows > 4;
  return rows > CAS_FLAT_ROWS;
}

struct FlatPlan {
  int64_t npad, tiles, splits, tiles_per_split;
  int64_t part_bytes, kf_bytes, vt_bytes, kp_bytes;
  int64_t total() const { return part_bytes + kf_bytes + vt_bytes + kp_bytes; }
};

static int64_t align256c(int64_t v) { return (v + 255) / 256 * 256; }

static FlatPlan flat_plan(int64_t rows, int64_t hkv, int64_t num_entries, int64_t page_size, int64_t d) {
  FlatPlan fp{};
  fp.npad = cdiv(num_entries * page_size, CAS_FT) * CAS_FT;
  fp.tiles = fp.npad / CAS_FT;
  // Split the keys until about 512 workgroups run (two per CU), or four per
  // 64-row block up to 1024 when there are many blocks: Qwen3 over 4096 keys,
  // 256 queries run best at 8 splits (43 us against 51 at 4 and 52 at 16),
  // 1024 queries at 4 (98 against 126 unsplit).  Override
  // BFA_TUNE_CASCADE_FLAT_WG sets the workgroup target instead.
  const int64_t blocks = cdiv(rows, 64) * hkv;
  int64_t target = std::min<int64_t>(std::max<int64_t>(512, 4 * blocks), 1024);
  if (tuning(BFA_TUNE_CASCADE_FLAT_WG) >= 1) target = tuning(BFA_TUNE_CASCADE_FLAT_WG);
  int64_t zs = std::min<int64_t>(cdiv(target, blocks), fp.tiles);
  zs = std::max<int64_t>(1, zs);
  fp.tiles_per_split = std::max<int64_t>(1, cdiv(fp.tiles, zs));
  fp.splits = std::max<int64_t>(1, cdiv(fp.tiles, fp.tiles_per_split));
  fp.part_bytes = fp.splits > 1 ? align256c(fp.splits * hkv * rows * (d + 2) * 4) : 0;
  fp.kf_bytes = align256c(hkv * fp.npad * d * 2);
  fp.vt_bytes = fp.kf_bytes;
  fp.kp_bytes = align256c(fp.npad * 4);
  return fp;
}

static int64_t cascade_splits(int64_t rows, int64_t hkv, int64_t steps) {
  const int64_t blocks = cdiv(rows, 64) * hkv;
  if (blocks >= 256 || steps <= 1) return 1;
  return std::max<int64_t>(1, std::min<int64_t>(cdiv(512, blocks), steps));
}

}  // namespace bfa

using namespace bfa;

extern "C" int bfa_online_softmax_update(
    const void* query, const void* key, const void* value, int q_dtype, int kv_dtype,
    float* m_i, float* l_i, float* acc_i, const void* query_positions, int qpos_dtype,
    const void* key_positions, int kpos_dtype, int64_t num_heads, int64_t batch,
    int64_t num_tokens, int64_t head_dim, int64_t q_stride_head, int64_t q_stride_batch,
    int64_t k_stride_head, int64_t k_stride_token, int64_t v_stride_head, int64_t v_stride_token,
    int64_t m_stride_head, int64_t m_stride_batch, int64_t l_stride_head, int64_t l_stride_batch,
    int64_t acc_stride_head, int64_t acc_stride_batch, float scale, int apply_causal_mask,
    void* stream) {
  const char* what = "bfa_online_softmax_update";
  BFA_REQUIRE(is_float_dtype(q_dtype) && is_float_dtype(kv_dtype), "%s: bad dtype", what);
  BFA_REQUIRE((qpos_dtype == BFA_DTYPE_I32 || qpos_dtype == BFA_DTYPE_I64) &&
                  (kpos_dtype == BFA_DTYPE_I32 || kpos_dtype == BFA_DTYPE_I64),
              "%s: positions must be int32/int64", what);
  BFA_REQUIRE(num_heads >= 0 && batch >= 0 && num_tokens >= 0 && head_dim >= 0, "%s: bad geometry", what);
  BFA_REQUIRE(head_dim <= 256, "%s: head_dim above 256", what);
  if (num_heads == 0 || batch == 0) return BFA_OK;
  BFA_REQUIRE(query && m_i && l_i && acc_i && query_positions, "%s: null pointer", what);
  BFA_REQUIRE(num_tokens == 0 || (key && value && key_positions), "%s: null pointer", what);
  OsmArgs a{};
  a.q = query; a.k = key; a.v = value; a.q_dt = q_dtype; a.kv_dt = kv_dtype;
  a.m = m_i; a.l = l_i; a.acc = acc_i;
  a.qpos = query_positions; a.kpos = key_positions;
  a.qpos_i64 = qpos_dtype == BFA_DTYPE_I64; a.kpos_i64 = kpos_dtype == BFA_DTYPE_I64;
  a.heads = num_heads; a.batch = batch; a.tokens = num_tokens; a.head_dim = head_dim;
  a.q_sh = q_stride_head; a.q_sb = q_stride_batch;
  a.k_sh = k_stride_head; a.k_st = k_stride_token;
  a.v_sh = v_stride_head; a.v_st = v_stride_token;
  a.m_sh = m_stride_head; a.m_sb = m_stride_batch;
  a.l_sh = l_stride_head; a.l_sb = l_stride_batch;
  a.a_sh = acc_stride_head; a.a_sb = acc_stride_batch;
  a.scale = scale; a.causal = apply_causal_mask;
  const int64_t grid = cdiv(num_heads * batch, 4);
  hipLaunchKernelGGL(online_softmax_kernel, dim3(static_cast<unsigned>(grid)), dim3(256), 0,
                     as_stream(stream), a);
  return check_launch(what);
}

extern "C" int64_t bfa_cascade_attention_workspace_size(int64_t tokens, int64_t num_q_heads,
                                                        int64_t num_kv_heads, int64_t head_dim,
                                                        int64_t num_entries, int64_t page_size) {
  if (tokens <= 0 || num_kv_heads <= 0 || num_q_heads % num_kv_heads != 0 || page_size <= 0) return 0;
  const int64_t rows = tokens * (num_q_heads / num_kv_heads);
  if (!mfma_head_dim(head_dim)) {
    const GenericSplit gs = generic_split(rows, num_kv_heads, num_entries);
    return gs.splits > 1 ? gs.splits * num_kv_heads * rows * (head_dim + 2) * 4 : 0;
  }
  if (!decode_form(rows) && flat_form(rows, num_entries))
    return flat_plan(rows, num_kv_heads, num_entries, page_size, head_dim).total();
  const int64_t splits = decode_form(rows) ? decode_split(num_kv_heads, num_entries, page_size).splits
                                           : cascade_splits(rows, num_kv_heads, cdiv(num_entries * page_size, 32));
  return splits > 1 ? splits * num_kv_heads * rows * (head_dim + 2) * 4 : 0;
}

extern "C" int bfa_cascade_attention(
    const void* query, int dtype, int64_t num_tokens, int64_t num_q_heads, int64_t q_stride_token,
    int64_t q_stride_head, const void* query_positions, int qpos_dtype, const void* kv_cache,
    int64_t num_pages, int64_t num_kv_heads, int64_t page_size, int64_t head_dim,
    int64_t stride_page, int64_t stride_kv, int64_t stride_head, int64_t stride_slot,
    int64_t num_entries, const int32_t* entry_page, const int64_t* entry_key_start,
    const int64_t* entry_delta, const int32_t* entry_info, const float* cos_sin_cache,
    int64_t max_position, const void* k_norm_weight, int k_norm_dtype, float k_norm_eps,
    float scale, int causal, void* out, int64_t out_stride_token, void* workspace,
    int64_t workspace_bytes, int32_t* status, void* stream) {
  const char* what = "bfa_cascade_attention";
  BFA_REQUIRE(dtype == BFA_DTYPE_BF16 || dtype == BFA_DTYPE_F16,
              "%s: query and cache must be bf16 or fp16", what);
  BFA_REQUIRE(head_dim > 0 && head_dim % 4 == 0 && head_dim <= CAS_GEN_DMAX,
              "%s: head_dim %lld (a multiple of 4 up to %d)", what, static_cast<long long>(head_dim), CAS_GEN_DMAX);
  BFA_REQUIRE(qpos_dtype == BFA_DTYPE_I32 || qpos_dtype == BFA_DTYPE_I64, "%s: bad positions dtype", what);
  BFA_REQUIRE(num_tokens >= 0 && num_kv_heads > 0 && num_q_heads % num_kv_heads == 0 && page_size > 0 &&
                  page_size < 65536 && num_entries >= 0 && num_pages >= 0,
              "%s: bad geometry", what);
  BFA_REQUIRE(k_norm_weight == nullptr || is_float_dtype(k_norm_dtype), "%s: bad k_norm dtype", what);
  BFA_REQUIRE(q_stride_token % 8 == 0 && q_stride_head % 8 == 0 && stride_page % 8 == 0 &&
                  stride_kv % 8 == 0 && stride_head % 8 == 0 && stride_slot % 8 == 0 &&
                  out_stride_token % 8 == 0 && aligned16(query) && aligned16(kv_cache) && aligned16(out) &&
                  (cos_sin_cache == nullptr || aligned16(cos_sin_cache)) &&
                  (k_norm_weight == nullptr || aligned16(k_norm_weight)),
              "%s: tensors must be 16-byte aligned with strides in multiples of 8", what);
  if (num_tokens == 0) return BFA_OK;
  BFA_REQUIRE(query && query_positions && out, "%s: null pointer", what);
  BFA_REQUIRE(num_entries == 0 || (entry_page && entry_key_start && entry_delta && entry_info),
              "%s: null entry metadata", what);
  BFA_REQUIRE(cos_sin_cache == nullptr || max_position > 0, "%s: empty rotary table", what);
  CasArgs a{};
  a.q = static_cast<const uint16_t*>(query);
  a.q_st = q_stride_token; a.q_sh = q_stride_head;
  a.qpos = query_positions; a.qpos_i64 = qpos_dtype == BFA_DTYPE_I64;
  a.cache = static_cast<const uint16_t*>(kv_cache);
  a.c_sp = stride_page; a.c_skv = stride_kv; a.c_sh = stride_head; a.c_ss = stride_slot;
  a.num_pages = num_pages; a.page_size = page_size;
  a.pages = entry_page; a.kstart = entry_key_start; a.delta = entry_delta; a.info = entry_info;
  a.num_entries = num_entries;
  a.cs = cos_sin_cache; a.max_pos = max_position;
  a.knorm_w = k_norm_weight; a.knorm_dt = k_norm_dtype; a.knorm_eps = k_norm_eps;
  a.tokens = num_tokens; a.hq = num_q_heads; a.hkv = num_kv_heads;
  a.group = num_q_heads / num_kv_heads;
  a.scale = scale; a.causal = causal;
  a.out = out; a.out_st = out_stride_token;
  a.status = status;
  const int64_t rows = num_tokens * a.group;
  if (!mfma_head_dim(head_dim)) {
    const GenericSplit gs = generic_split(rows, num_kv_heads, num_entries);
    if (gs.splits > 1) {
      BFA_REQUIRE(workspace && workspace_bytes >= gs.splits * num_kv_heads * rows * (head_dim + 2) * 4,
                  "%s: workspace too small", what);
      a.part = static_cast<float*>(workspace);
    }
    BFA_REQUIRE(cdiv(rows, 4) < (int64_t{1} << 31) && num_kv_heads < 65536 && gs.splits < 65536,
                "%s: grid too large", what);
    const dim3 grid(static_cast<unsigned>(cdiv(rows, 4)), static_cast<unsigned>(num_kv_heads),
                    static_cast<unsigned>(gs.splits));
    const dim3 mgrid(static_cast<unsigned>(cdiv(num_kv_heads * rows, 4)));
    const hipStream_t s = as_stream(stream);
    if (dtype == BFA_DTYPE_BF16) {
      hipLaunchKernelGGL((cascade_generic_kernel<true>), grid, dim3(256), 0, s, a, head_dim, gs.per_split);
      if (gs.splits > 1)
        hipLaunchKernelGGL((cascade_merge_generic_kernel<true>), mgrid, dim3(256), 0, s, a, head_dim, gs.splits);
    } else {
      hipLaunchKernelGGL((cascade_generic_kernel<false>), grid, dim3(256), 0, s, a, head_dim, gs.per_split);
      if (gs.splits > 1)
        hipLaunchKernelGGL((cascade_merge_generic_kernel<false>), mgrid, dim3(256), 0, s, a, head_dim, gs.splits);
    }
    return check_launch(what);
  }
  if (decode_form(rows)) {
    const DecodeSplit ds = decode_split(num_kv_heads, num_entries, page_size);
    if (ds.splits > 1) {
      BFA_REQUIRE(workspace && workspace_bytes >= ds.splits * num_kv_heads * rows * (head_dim + 2) * 4,
                  "%s: workspace too small", what);
      a.part = static_cast<float*>(workspace);
    }
    BFA_REQUIRE(ds.splits < 65536 && num_kv_heads < (int64_t{1} << 31), "%s: grid too large", what);
    const dim3 grid(static_cast<unsigned>(num_kv_heads), static_cast<unsigned>(ds.splits));
    const hipStream_t s = as_stream(stream);
    auto launch = [&](auto bf, auto dd) {
      constexpr bool B = decltype(bf)::value;
      constexpr int DD = decltype(dd)::value;
      if (rows <= 1) hipLaunchKernelGGL((cascade_decode_kernel<B, 1, DD>), grid, dim3(256), 0, s, a, ds.per_split, ds.nsb);
      else if (rows <= 2) hipLaunchKernelGGL((cascade_decode_kernel<B, 2, DD>), grid, dim3(256), 0, s, a, ds.per_split, ds.nsb);
      else hipLaunchKernelGGL((cascade_decode_kernel<B, 4, DD>), grid, dim3(256), 0, s, a, ds.per_split, ds.nsb);
      if (ds.splits > 1) launch_merge<B, DD>(a, rows, ds.splits, s);
    };
    dispatch_dtype_hd(dtype, head_dim, launch);
    return check_launch(what);
  }
  if (flat_form(rows, num_entries)) {
    const FlatPlan fp = flat_plan(rows, num_kv_heads, num_entries, page_size, head_dim);
    BFA_REQUIRE(workspace && workspace_bytes >= fp.total() && aligned16(workspace), "%s: workspace too small", what);
    BFA_REQUIRE(fp.npad * head_dim * 2 < (int64_t{1} << 31) && fp.tiles < (int64_t{1} << 31) &&
                    cdiv(rows, 64) < (int64_t{1} << 31) && fp.splits < 65536 && num_kv_heads < 65536,
                "%s: too many keys for the flat form", what);
    char* ws = static_cast<char*>(workspace);
    if (fp.splits > 1) a.part = reinterpret_cast<float*>(ws);
    FlatArgs f{};
    f.kf = reinterpret_cast<uint16_t*>(ws + fp.part_bytes);
    f.vt = reinterpret_cast<uint16_t*>(ws + fp.part_bytes + fp.kf_bytes);
    f.kpos = reinterpret_cast<int32_t*>(ws + fp.part_bytes + fp.kf_bytes + fp.vt_bytes);
    f.npad = fp.npad;
    f.tiles_per_split = fp.tiles_per_split;
    const hipStream_t s = as_stream(stream);
    const dim3 pgrid(static_cast<unsigned>(fp.tiles), static_cast<unsigned>(num_kv_heads), 2);
    const dim3 grid(static_cast<unsigned>(cdiv(rows, 64)), static_cast<unsigned>(num_kv_heads),
                    static_cast<unsigned>(fp.splits));
    auto launch = [&](auto bf, auto dd) {
      constexpr bool B = decltype(bf)::value;
      constexpr int DD = decltype(dd)::value;
      hipLaunchKernelGGL((cascade_flatten_kernel<B, DD>), pgrid, dim3(256), 0, s, a, f);
      hipLaunchKernelGGL((cascade_flat_kernel<B, DD>), grid, dim3(256), 0, s, a, f);
      if (fp.splits > 1) launch_merge<B, DD>(a, rows, fp.splits, s);
    };
    dispatch_dtype_hd(dtype, head_dim, launch);
    return check_launch(what);
  }
  a.steps = cdiv(num_entries * page_size, 32);
  const int64_t splits = cascade_splits(rows, num_kv_heads, a.steps);
  a.steps_per_split = std::max<int64_t>(1, cdiv(a.steps, splits));
  const int64_t zs = a.steps > 0 ? cdiv(a.steps, a.steps_per_split) : 1;
  if (zs > 1) {
    BFA_REQUIRE(workspace && workspace_bytes >= zs * num_kv_heads * rows * (head_dim + 2) * 4,
                "%s: workspace too small", what);
    a.part = static_cast<float*>(workspace);
  }
  BFA_REQUIRE(cdiv(rows, 64) < (int64_t{1} << 31) && zs < 65536 && num_kv_heads < 65536,
              "%s: grid too large", what);
  const dim3 grid(static_cast<unsigned>(cdiv(rows, 64)), static_cast<unsigned>(num_kv_heads),
                  static_cast<unsigned>(zs));
  BFA_REQUIRE(zs == 1 || num_kv_heads * rows < (int64_t{1} << 31), "%s: grid too large", what);
  const hipStream_t s = as_stream(stream);
  auto launch = [&](auto bf, auto dd) {
    constexpr bool B = decltype(bf)::value;
    constexpr int DD = decltype(dd)::value;
    hipLaunchKernelGGL((cascade_attn_kernel<B, DD>), grid, dim3(256), 0, s, a);
    if (zs > 1) launch_merge<B, DD>(a, rows, zs, s);
  };
  dispatch_dtype_hd(dtype, head_dim, launch);
  return check_launch(what);
}
