// The QKV projection's epilogue description and the element helpers its
// kernels share (qkv.hip: the GEMM, split-K and column-pair kernels;
// qkv_gemv.hip: the one-launch decode kernel for a few tokens).
#pragma once

#include <hip/hip_runtime.h>

#include "bfa_append.h"
#include "bfa_device.h"

namespace bfa {

// ------------------------------------------------------------- epilogue spec
struct QkvEpi {
  const void* bias;
  int bias_dtype;
  int qkv_dt;   // rounding of the projection (BFA_DTYPE_F32 = none)
  int norm_dt;  // dtype the q/k norm result is cast to
  int out_dt;
  int64_t n;        // columns (q|k|v)
  int64_t hq, hkv;  // heads
  int64_t hd;       // head_dim
  const void* qn_w;
  const void* kn_w;
  int qk_w_dtype;
  float qk_eps;
  const void* positions;
  int pos_is_i64;
  const float* cs;  // cos|sin table [max_pos, hd] or nullptr (no RoPE)
  int64_t max_pos;
  void* out;
  int64_t ldo;
  int* status;
  // EPI_LINEAR / EPI_SWIGLU: y = out_dt(mid_dt(qkv_dt(acc) + residual)) or
  // out_dt(qkv_dt(silu(qkv_dt(gate))) * qkv_dt(up)); vec = 16-byte row access is
  // allowed for out and residual (aligned bases, strides multiple of 8)
  const void* res;
  int res_dt;
  int64_t ldr;
  int mid_dt;
  int vec;
  // scale-after decode (the fp32 variants): stats[s * stat_rows + t] holds split
  // s's sum of x^2 over its K slice for token t; the projection of x * gamma is
  // multiplied by r = 1 / sqrt(sum / hidden + stat_eps) before the bias
  const float* stats;
  int64_t stat_rows;
  int64_t hidden;
  float stat_eps;
  // Paged-KV append in the epilogue (bfa_fused_rmsnorm_qkv_append): the k and v
  // heads of row t also go to cache + slot_off[t] + (V ? c_skv : 0) + (head -
  // first head of its kind) * c_sh + column in the head, as cache_dt (from the
  // value rounded to out_dt); slot_off[t] < 0 skips the row.  skip_kv_out = 1
  // leaves the k/v columns of `out` unwritten.
  void* cache;
  int cache_dt;
  int64_t c_skv, c_sh;
  const int64_t* slot_off;
  int skip_kv_out;
  // app_in_kernel = 1: the prefill GEMM resolves its rows' cache slots itself
  // (before the K loop, from `app`), and slot_off is not used
  int app_in_kernel;
  AppendArgs app;
  // prefill with the norm weight folded into W (the fp32 variants): the
  // projection of row t is multiplied by row_scale[t] (1 / rms) before the bias
  const float* row_scale;
};

__device__ __forceinline__ float round_to(float v, int dt) {
  if (dt == BFA_DTYPE_BF16) return Elem<BFA_DTYPE_BF16>::round(v);
  if (dt == BFA_DTYPE_F16) return Elem<BFA_DTYPE_F16>::round(v);
  return v;
}

__device__ __forceinline__ void store_any(void* p, int dt, int64_t i, float v) {
  if (dt == BFA_DTYPE_BF16) store1<BFA_DTYPE_BF16>(p, i, v);
  else if (dt == BFA_DTYPE_F16) store1<BFA_DTYPE_F16>(p, i, v);
  else store1<BFA_DTYPE_F32>(p, i, v);
}


// 0 = q head, 1 = k head, 2 = v head
__device__ __forceinline__ int head_kind(const QkvEpi& e, int64_t head) {
  return head < e.hq ? 0 : (head < e.hq + e.hkv ? 1 : 2);
}

// Position p wrapped like a torch negative index; -1 when outside the table.
// Element i of a vector of run-time dtype (fp32, bf16 or fp16) in two steps: the
// 4-byte word holding it (ld_word), then its value (word_value).  The load has
// no branch, so it issues with its neighbours; the conversion, which the
// compiler may branch on, comes after every load is out.  A 16-bit element is
// read as the aligned 4-byte word that contains it (whatever the vector's own
// alignment), so the word never crosses an aligned 4-byte block of the vector.
__device__ __forceinline__ uint32_t ld_word(const void* p, int dt, int64_t i) {
  const uintptr_t a = reinterpret_cast<uintptr_t>(p) + static_cast<uintptr_t>(dt == BFA_DTYPE_F32 ? i * 4 : i * 2);
  return *reinterpret_cast<const uint32_t*>(dt == BFA_DTYPE_F32 ? a : (a & ~uintptr_t(3)));
}
__device__ __forceinline__ float word_value(uint32_t w, int dt, const void* p, int64_t i) {
  const bool hi = ((reinterpret_cast<uintptr_t>(p) >> 1) + static_cast<uintptr_t>(i)) & 1;
  const uint32_t h = hi ? (w >> 16) : (w & 0xffffu);
  return dt == BFA_DTYPE_F32 ? __uint_as_float(w) : (dt == BFA_DTYPE_BF16 ? bf16_bits_to_f32(h) : f16_bits_to_f32(h));
}
// The same for a vector whose base is 4-byte aligned (checked by the caller's
// host side): the word offset comes from the index alone, which keeps the
// address arithmetic to one select (the one-launch decode kernel's compiler
// schedule depends on it: a wider select there cost it its early loads).
__device__ __forceinline__ uint32_t ld_word_al4(const void* p, int dt, int64_t i) {
  return *reinterpret_cast<const uint32_t*>(static_cast<const char*>(p) +
                                            (dt == BFA_DTYPE_F32 ? i * 4 : (i * 2) & ~int64_t(3)));
}
__device__ __forceinline__ float word_value_al4(uint32_t w, int dt, int64_t i) {
  const uint32_t h = (i & 1) ? (w >> 16) : (w & 0xffffu);
  return dt == BFA_DTYPE_F32 ? __uint_as_float(w) : (dt == BFA_DTYPE_BF16 ? bf16_bits_to_f32(h) : f16_bits_to_f32(h));
}

__device__ __forceinline__ int32_t epi_pos_check(const QkvEpi& e, int64_t p) {
  if (p < 0) p += e.max_pos;
  return (p >= 0 && p < e.max_pos) ? static_cast<int32_t>(p) : -1;
}

template <int DT>
__device__ __forceinline__ void unpack8(uint4 u, float (&v)[8]) {
  const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = Elem<DT>::to_f32(static_cast<uint16_t>(w[i] & 0xffffu));
    v[2 * i + 1] = Elem<DT>::to_f32(static_cast<uint16_t>(w[i] >> 16));
  }
}

typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));

// 16-byte weight load returned through a plain vector value: loading straight
// into the uint4 array member makes the compiler keep the whole array in scratch.
__device__ __forceinline__ uint4 load16(const uint16_t* p) {
  const u32x4_t t = *reinterpret_cast<const u32x4_t*>(p);
  return make_uint4(t.x, t.y, t.z, t.w);
}

// Two elements of a small float vector of runtime dtype, with one dispatch.
__device__ __forceinline__ void load2_any(const void* p, int dt, int64_t i1, int64_t i2, float& v1,
                                          float& v2) {
  if (dt == BFA_DTYPE_BF16) {
    v1 = load1<BFA_DTYPE_BF16>(p, i1);
    v2 = load1<BFA_DTYPE_BF16>(p, i2);
  } else if (dt == BFA_DTYPE_F16) {
    v1 = load1<BFA_DTYPE_F16>(p, i1);
    v2 = load1<BFA_DTYPE_F16>(p, i2);
  } else {
    v1 = static_cast<const float*>(p)[i1];
    v2 = static_cast<const float*>(p)[i2];
  }
}

// ---------------------------------------------- one-launch decode (qkv_gemv.hip)
struct GemvArgs {
  const uint16_t* a;  // bf16 operand [m, k] rows lda apart; with the fold, the raw rows x
  const uint16_t* w;  // bf16 weight [n, k] rows ldw apart
  int64_t m, k, lda, ldw;
  const void* gamma;  // fold: RMSNorm weight, its dtype, mixed rounding, eps
  int gamma_dt, mixed;
  float eps;
  int64_t pw;         // (set by the launcher)
};

// The kernel's own compact copy of the arguments (GemvArgs and the fields of
// QkvEpi it reads): 160 bytes of kernel arguments instead of 552, all of them
// loaded at the kernel's start in one go.
struct GemvKArgs {
  const uint16_t* a;
  const uint16_t* w;
  const void* gamma;
  const void* bias;
  const void* positions;
  const float* cs;
  void* out;
  int* status;
  void* cache;
  const int64_t* slot_off;
  int64_t ldo, c_skv, c_sh;
  int32_t m, k, lda, ldw, pw, hq, hkv, hd, max_pos;
  float eps;
  // dtypes and flags, one byte each
  uint8_t gamma_dt, mixed, bias_dt, qkv_dt, out_dt, cache_dt, pos_is_i64, skip_kv_out;
};

// Whether the one-launch kernel takes the call: up to 4 tokens (8 when the
// grid, n / 16 workgroups, is at most 192) without q/k norm, bf16 operand and
// weight, hidden a multiple of 128 up to 4096, head_dim a multiple of 16, a
// 4-byte-aligned bias (planner override BFA_TUNE_DECODE_GEMV = 0: never).
bool gemv_ok(int64_t tokens, int64_t k, int64_t n, int64_t hd, bool qk_norm, const void* bias, bool bf16_w,
             bool bf16_x, const void* a, int64_t lda);
// Launches it (fold: `a` holds the raw rows and the kernel normalises them).
void launch_qkv_gemv(GemvArgs d, bool fold, const QkvEpi& e, hipStream_t s);

}  // namespace bfa
