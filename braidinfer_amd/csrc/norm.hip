// Row-wise RMSNorm family on gfx950.
//
// One kernel template serves every RMSNorm flavour on the hot path; they
// differ only in their rounding points (the torch op chain multiplies by
// rsqrt(var + eps), the Triton kernels divide by sqrt(mean + eps); both are
// computed here as a multiply by one reciprocal per row):
//   kRms          RMSNorm.rms_forward         layers/layernorm.py:35-44
//   kAddRms       RMSNorm.add_rms_forward     layers/layernorm.py:46-57
//   kF32          RMSNormF32.forward          kernels/rmsnorm_f32.py:47-96
//   kOperandMixed normalised QKV operand, fused_rmsnorm_qkv_mixed_precision.py:61-116
//   kOperandProd  normalised QKV operand, fused_rmsnorm_qkv_production.py:61-116
//                 (also the f32 variants minimal_f32.py:59-107, with_bias.py, whose
//                 fp32 operand is rounded once to the MFMA input type)
//   kRowScale     the row statistic alone, 1 / rms per row (fp32), for the f32
//                 variants' prefill with the norm weight folded into the QKV weight
//                 (the projection of x multiplied by it per row; minimal_f32.py:59-107)
//
// Design: a row is owned by a group of L lanes (L = 16, 64 or 256).  Each lane
// keeps up to MAXC chunks of 8 elements in registers, loaded with 16-byte
// vector loads, so the row is read from HBM exactly once.  The sum of squares
// is reduced with a butterfly inside the group (plus one LDS step when L spans
// several waves), and the normalised chunks are written back with 16-byte
// stores.  A scalar two-pass kernel covers unaligned / odd-sized rows.
#include "bfa_device.h"
#include "bfa_host.h"
#include "bfa_internal.h"

namespace bfa {

enum NormMode { kRms = 0, kAddRms = 1, kF32 = 2, kOperandMixed = 3, kOperandProd = 4, kRowScale = 5 };

struct NormArgs {
  const void* x;
  const void* res;
  void* y;
  void* res_out;
  const void* w;
  int w_dtype;
  int64_t rows, rows_inner, hidden;
  int64_t x_so, x_si, x_sc;  // outer / inner row strides, column stride
  int64_t r_s, ro_s;         // residual / residual_out row strides (kAddRms)
  int64_t y_so, y_si, y_sc;
  float eps;
};

// Elements 8 g .. 8 g + 7 of a 16-byte aligned vector of run-time dtype in two
// steps: the raw 16 (fp32: 32) bytes, requested without a branch on the dtype,
// then their values.
struct Raw8Dyn {
  uint4 w0, w1;
  __device__ __forceinline__ void load(const void* p, int dt, int64_t g) {
    const bool f32 = dt == BFA_DTYPE_F32;
    const char* q = static_cast<const char*>(p) + g * (f32 ? 32 : 16);
    w0 = *reinterpret_cast<const uint4*>(q);
    w1 = *reinterpret_cast<const uint4*>(f32 ? q + 16 : q);
  }
  __device__ __forceinline__ void to_f32(int dt, float (&v)[8]) const {
    const uint32_t u[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint16_t h = static_cast<uint16_t>((i & 1) ? (u[i / 2] >> 16) : (u[i / 2] & 0xffffu));
      v[i] = dt == BFA_DTYPE_F32 ? __uint_as_float(u[i])
                                 : (dt == BFA_DTYPE_BF16 ? bf16_bits_to_f32(h) : f16_bits_to_f32(h));
    }
  }
};

// Applies the mode's normalisation to one value.  `inv` = 1 / sqrt(sum/H + eps)
// for every mode: the torch chain multiplies by rsqrt(var + eps), and the
// Triton kernels' x / rms is computed as x * (1 / rms) -- one correctly rounded
// reciprocal per row, then a multiply, within 1.5 fp32 ulp of the quotient
// (a per-element IEEE division costs about ten VALU instructions, which made
// the operand pre-pass ALU-bound).
template <int DT_IN, int MODE>
__device__ __forceinline__ float norm_apply(float v, float inv, float g) {
  if constexpr (MODE == kRms || MODE == kAddRms) {
    // x.mul_(rsqrt(var+eps)); x.to(orig_dtype).mul_(weight)
    return Elem<DT_IN>::round(v * inv) * g;
  } else if constexpr (MODE == kOperandMixed) {
    // (x / rms) -> bf16, then * weight (result rounded by the store)
    return round_bf16(v * inv) * g;
  } else {
    // kF32 / kOperandProd: (x / rms) * weight in fp32
    return (v * inv) * g;
  }
}

__device__ __forceinline__ float norm_inv(float ss, int64_t hidden, float eps) {
  return 1.0f / sqrtf(ss / static_cast<float>(hidden) + eps);
}

// NTR (kAddRms): residual_out is stored with the nontemporal hint (a large
// residual is not read again until after the attention block).
template <int DT_IN, int DT_OUT, int MODE, int L, int MAXC, bool NTR = false>
__global__ __launch_bounds__(256) void norm_vec_kernel(NormArgs a) {
  using TIN = typename Elem<DT_IN>::T;
  using TOUT = typename Elem<DT_OUT>::T;
  constexpr int RPW = (L >= 256) ? 1 : 256 / L;  // rows per workgroup
  const int tid = threadIdx.x;
  const int lane = (L >= 256) ? tid : (tid % L);
  const int64_t row = static_cast<int64_t>(blockIdx.x) * RPW + ((L >= 256) ? 0 : tid / L);
  if (row >= a.rows) return;  // uniform per row group (whole WG when L == 256)

  const int64_t ro = a.rows_inner == 1 ? row : row / a.rows_inner, ri = row - ro * a.rows_inner;
  const TIN* xp = static_cast<const TIN*>(a.x) + ro * a.x_so + ri * a.x_si;
  TOUT* yp = static_cast<TOUT*>(a.y) + ro * a.y_so + ri * a.y_si;
  const int nchunks = static_cast<int>(a.hidden / 8);

  float v[MAXC][8];
  float ss = 0.f;
  // the norm weight's granules go out with the row (raw, converted after the
  // sum): requested after the reduction they were a second memory round trip
  Raw8Dyn gw[MAXC];
  if constexpr (MODE != kRowScale) {
#pragma unroll
    for (int c = 0; c < MAXC; ++c) gw[c].load(a.w, a.w_dtype, min(lane + c * L, nchunks - 1));
  }
#pragma unroll
  for (int c = 0; c < MAXC; ++c) {
    const int ch = lane + c * L;
    if (ch < nchunks) {
      // kRowScale: plain loads, so that x stays in the caches for the projection
      // that reads it next (the other modes read their input once)
      if constexpr (MODE == kRowScale) load8<DT_IN>(xp + ch * 8, v[c]);
      else load8_nt<DT_IN>(xp + ch * 8, v[c]);
      if constexpr (MODE == kAddRms) {
        float r[8];
        load8_nt<DT_IN>(static_cast<const TIN*>(a.res) + row * a.r_s + ch * 8, r);
#pragma unroll
        for (int i = 0; i < 8; ++i) v[c][i] = v[c][i] + r[i];
        if (a.res_out) store8<DT_IN, NTR>(static_cast<TIN*>(a.res_out) + row * a.ro_s + ch * 8, v[c]);
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) ss += v[c][i] * v[c][i];
    }
  }
  ss = group_sum<(L < kWave ? L : kWave)>(ss);
  if constexpr (L > kWave) {
    __shared__ float red[L / kWave];
    if ((tid & (kWave - 1)) == 0) red[tid / kWave] = ss;
    __syncthreads();
    ss = 0.f;
#pragma unroll
    for (int w = 0; w < L / kWave; ++w) ss += red[w];
  }
  const float inv = norm_inv(ss, a.hidden, a.eps);
  if constexpr (MODE == kRowScale) {
    if (lane == 0) static_cast<float*>(a.y)[row] = inv;
    return;
  }

#pragma unroll
  for (int c = 0; c < MAXC; ++c) {
    const int ch = lane + c * L;
    if (ch < nchunks) {
      float g[8], o[8];
      gw[c].to_f32(a.w_dtype, g);
#pragma unroll
      for (int i = 0; i < 8; ++i) o[i] = norm_apply<DT_IN, MODE>(v[c][i], inv, g[i]);
      store8<DT_OUT>(yp + ch * 8, o);
    }
  }
}

// Any alignment, any hidden size, column strides: one workgroup per row, two
// passes over the row (the second pass re-reads x from L2).
template <int DT_IN, int DT_OUT, int MODE>
__global__ __launch_bounds__(256) void norm_scalar_kernel(NormArgs a) {
  const int64_t row = blockIdx.x;
  const int tid = threadIdx.x;
  const int64_t ro = row / a.rows_inner, ri = row - ro * a.rows_inner;
  const int64_t xoff = ro * a.x_so + ri * a.x_si;
  const int64_t yoff = ro * a.y_so + ri * a.y_si;

  float ss = 0.f;
  for (int64_t i = tid; i < a.hidden; i += 256) {
    float v = load1<DT_IN>(a.x, xoff + i * a.x_sc);
    if constexpr (MODE == kAddRms) v = v + load1<DT_IN>(a.res, row * a.r_s + i);
    ss += v * v;
  }
  ss = group_sum<kWave>(ss);
  __shared__ float red[256 / kWave];
  if ((tid & (kWave - 1)) == 0) red[tid / kWave] = ss;
  __syncthreads();
  ss = 0.f;
#pragma unroll
  for (int w = 0; w < 256 / kWave; ++w) ss += red[w];
  const float inv = norm_inv(ss, a.hidden, a.eps);
  if constexpr (MODE == kRowScale) {
    if (tid == 0) static_cast<float*>(a.y)[row] = inv;
    return;
  }

  for (int64_t i = tid; i < a.hidden; i += 256) {
    float v = load1<DT_IN>(a.x, xoff + i * a.x_sc);
    if constexpr (MODE == kAddRms) {
      v = v + load1<DT_IN>(a.res, row * a.r_s + i);
      if (a.res_out) store1<DT_IN>(a.res_out, row * a.ro_s + i, v);
    }
    const float g = load_any(a.w, a.w_dtype, i);
    store1<DT_OUT>(a.y, yoff + i * a.y_sc, norm_apply<DT_IN, MODE>(v, inv, g));
  }
}

template <int DT_IN, int DT_OUT, int MODE, int L, int MAXC>
static void launch_vec(const NormArgs& a, hipStream_t s) {
  constexpr int RPW = (L >= 256) ? 1 : 256 / L;
  const int64_t grid = cdiv(a.rows, RPW);
  if constexpr (MODE == kAddRms) {
    if (a.res_out && stream_output(a.rows * a.hidden * static_cast<int64_t>(sizeof(typename Elem<DT_IN>::T)))) {
      hipLaunchKernelGGL((norm_vec_kernel<DT_IN, DT_OUT, MODE, L, MAXC, true>), dim3(grid), dim3(256), 0,
                         s, a);
      return;
    }
  }
  hipLaunchKernelGGL((norm_vec_kernel<DT_IN, DT_OUT, MODE, L, MAXC>), dim3(grid), dim3(256), 0,
                     s, a);
}

template <int DT_IN, int DT_OUT, int MODE>
static int launch_norm_typed(const NormArgs& a, bool vec_ok, hipStream_t s, const char* what) {
  if (a.rows == 0 || a.hidden == 0) return BFA_OK;
  if (a.rows > 0x7fffffffLL) return set_error(BFA_ERR_UNSUPPORTED, "%s: too many rows", what);
  const int64_t nch = a.hidden / 8;
  // Lanes per row: a whole 256-lane workgroup per row from 128 chunks of 8 up
  // (at 8192 x 4096 one row per workgroup ran add+RMSNorm in 43 us against
  // 50 us with four rows of 64 lanes each); small rows pack 4 or 16 per workgroup.
  if (vec_ok) {
    if (nch <= 2 * 16) {
      launch_vec<DT_IN, DT_OUT, MODE, 16, 2>(a, s);
    } else if (nch <= 2 * 64) {
      launch_vec<DT_IN, DT_OUT, MODE, 64, 2>(a, s);
    } else if (nch <= 256) {
      launch_vec<DT_IN, DT_OUT, MODE, 256, 1>(a, s);
    } else if (nch <= 2 * 256) {
      launch_vec<DT_IN, DT_OUT, MODE, 256, 2>(a, s);
    } else if (nch <= 4 * 256) {
      launch_vec<DT_IN, DT_OUT, MODE, 256, 4>(a, s);
    } else if (nch <= 8 * 256) {
      launch_vec<DT_IN, DT_OUT, MODE, 256, 8>(a, s);
    } else if (nch <= 16 * 256) {
      launch_vec<DT_IN, DT_OUT, MODE, 256, 16>(a, s);
    } else {
      vec_ok = false;
    }
  }
  if (!vec_ok) {
    hipLaunchKernelGGL((norm_scalar_kernel<DT_IN, DT_OUT, MODE>), dim3(a.rows), dim3(256), 0, s,
                       a);
  }
  return check_launch(what);
}

// DT_OUT == DT_IN for the torch-chain modes.
template <int MODE>
static int launch_norm_same(int dt, const NormArgs& a, bool vec_ok, hipStream_t s,
                            const char* what) {
  switch (dt) {
    case BFA_DTYPE_F32: return launch_norm_typed<BFA_DTYPE_F32, BFA_DTYPE_F32, MODE>(a, vec_ok, s, what);
    case BFA_DTYPE_F16: return launch_norm_typed<BFA_DTYPE_F16, BFA_DTYPE_F16, MODE>(a, vec_ok, s, what);
    case BFA_DTYPE_BF16: return launch_norm_typed<BFA_DTYPE_BF16, BFA_DTYPE_BF16, MODE>(a, vec_ok, s, what);
  }
  return set_error(BFA_ERR_INVALID, "%s: unsupported x dtype %d", what, dt);
}

template <int DT_OUT, int MODE>
static int launch_norm_out(int dt, const NormArgs& a, bool vec_ok, hipStream_t s,
                           const char* what) {
  switch (dt) {
    case BFA_DTYPE_F32: return launch_norm_typed<BFA_DTYPE_F32, DT_OUT, MODE>(a, vec_ok, s, what);
    case BFA_DTYPE_F16: return launch_norm_typed<BFA_DTYPE_F16, DT_OUT, MODE>(a, vec_ok, s, what);
    case BFA_DTYPE_BF16: return launch_norm_typed<BFA_DTYPE_BF16, DT_OUT, MODE>(a, vec_ok, s, what);
  }
  return set_error(BFA_ERR_INVALID, "%s: unsupported x dtype %d", what, dt);
}

static bool mult8(int64_t v) { return (v % 8) == 0; }

int launch_qkv_operand(const void* x, int x_dtype, int64_t rows, int64_t hidden, int64_t x_stride,
                       const void* w, int w_dtype, bool mixed, void* out, int out_dtype,
                       float eps, hipStream_t s) {
  const char* what = "rmsnorm_qkv_operand";
  BFA_REQUIRE(is_float_dtype(x_dtype) && is_float_dtype(w_dtype), "%s: bad dtype", what);
  BFA_REQUIRE(out_dtype == BFA_DTYPE_BF16 || out_dtype == BFA_DTYPE_F16,
              "%s: operand dtype must be bf16 or fp16", what);
  NormArgs a{};
  a.x = x; a.w = w; a.w_dtype = w_dtype; a.y = out;
  a.rows = rows; a.rows_inner = 1; a.hidden = hidden;
  a.x_so = x_stride; a.x_si = 0; a.x_sc = 1;
  a.y_so = hidden; a.y_si = 0; a.y_sc = 1;
  a.eps = eps;
  const bool vec_ok = mult8(hidden) && mult8(x_stride) && aligned16(x) && aligned16(w) &&
                      aligned16(out);
  if (out_dtype == BFA_DTYPE_BF16) {
    return mixed ? launch_norm_out<BFA_DTYPE_BF16, kOperandMixed>(x_dtype, a, vec_ok, s, what)
                 : launch_norm_out<BFA_DTYPE_BF16, kOperandProd>(x_dtype, a, vec_ok, s, what);
  }
  return mixed ? launch_norm_out<BFA_DTYPE_F16, kOperandMixed>(x_dtype, a, vec_ok, s, what)
               : launch_norm_out<BFA_DTYPE_F16, kOperandProd>(x_dtype, a, vec_ok, s, what);
}

int launch_row_scale(const void* x, int x_dtype, int64_t rows, int64_t hidden, int64_t x_stride,
                     float* out, float eps, hipStream_t s) {
  const char* what = "rmsnorm row scale";
  BFA_REQUIRE(is_float_dtype(x_dtype), "%s: bad dtype", what);
  NormArgs a{};
  a.x = x; a.y = out;
  a.rows = rows; a.rows_inner = 1; a.hidden = hidden;
  a.x_so = x_stride; a.x_si = 0; a.x_sc = 1;
  a.y_so = 1; a.y_si = 0; a.y_sc = 1;
  a.eps = eps;
  const bool vec_ok = mult8(hidden) && mult8(x_stride) && aligned16(x);
  return launch_norm_out<BFA_DTYPE_F32, kRowScale>(x_dtype, a, vec_ok, s, what);
}

// folded[n, k] = W[n, k] * gamma[k], the product in fp32 rounded once to W's
// dtype: 8 elements per thread, 16-byte rows (k % 8 == 0, aligned bases).
template <int DT_W>
__global__ __launch_bounds__(256) void fold_weight_kernel(const uint16_t* w, int64_t ldw, const void* g, int g_dt,
                                                          uint16_t* out, int64_t ldo, int64_t n, int64_t k8) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (idx >= n * k8) return;
  const int64_t row = idx / k8, c = idx - row * k8;
  Raw8Dyn gr;
  gr.load(g, g_dt, c);
  const uint4 wr = *reinterpret_cast<const uint4*>(w + row * ldw + c * 8);
  float wv[8], gv[8];
  const uint32_t u[4] = {wr.x, wr.y, wr.z, wr.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    wv[2 * i] = Elem<DT_W>::to_f32(static_cast<uint16_t>(u[i] & 0xffffu));
    wv[2 * i + 1] = Elem<DT_W>::to_f32(static_cast<uint16_t>(u[i] >> 16));
  }
  gr.to_f32(g_dt, gv);
#pragma unroll
  for (int i = 0; i < 8; ++i) wv[i] = wv[i] * gv[i];
  store8<DT_W>(out + row * ldo + c * 8, wv);
}

int launch_fold_weight(const void* w, int w_dtype, int64_t n, int64_t k, int64_t ldw, const void* g,
                       int g_dtype, void* out, int64_t ldo, hipStream_t s) {
  const char* what = "bfa_fold_rmsnorm_weight";
  BFA_REQUIRE(w_dtype == BFA_DTYPE_BF16 || w_dtype == BFA_DTYPE_F16, "%s: weight must be bf16/fp16", what);
  BFA_REQUIRE(is_float_dtype(g_dtype), "%s: bad norm weight dtype", what);
  BFA_REQUIRE(n >= 0 && k >= 0 && ldw >= k && ldo >= k, "%s: bad geometry", what);
  BFA_REQUIRE(mult8(k) && mult8(ldw) && mult8(ldo) && aligned16(w) && aligned16(g) && aligned16(out),
              "%s: rows must be 16-byte aligned with hidden a multiple of 8", what);
  const int64_t total = n * (k / 8);
  if (total == 0) return BFA_OK;
  const unsigned grid = static_cast<unsigned>(cdiv(total, 256));
  if (w_dtype == BFA_DTYPE_BF16)
    hipLaunchKernelGGL((fold_weight_kernel<BFA_DTYPE_BF16>), dim3(grid), dim3(256), 0, s,
                       static_cast<const uint16_t*>(w), ldw, g, g_dtype, static_cast<uint16_t*>(out), ldo, n, k / 8);
  else
    hipLaunchKernelGGL((fold_weight_kernel<BFA_DTYPE_F16>), dim3(grid), dim3(256), 0, s,
                       static_cast<const uint16_t*>(w), ldw, g, g_dtype, static_cast<uint16_t*>(out), ldo, n, k / 8);
  return check_launch(what);
}

}  // namespace bfa

using namespace bfa;

extern "C" int bfa_rmsnorm_row_scale(const void* x, int x_dtype, int64_t rows, int64_t hidden, int64_t x_stride,
                                     float* out, float eps, void* stream) {
  BFA_REQUIRE(x && out, "bfa_rmsnorm_row_scale: null pointer");
  BFA_REQUIRE(rows >= 0 && hidden > 0 && x_stride >= hidden, "bfa_rmsnorm_row_scale: bad geometry");
  return launch_row_scale(x, x_dtype, rows, hidden, x_stride, out, eps, as_stream(stream));
}

extern "C" int bfa_fold_rmsnorm_weight(const void* qkv_weight, int w_dtype, int64_t qkv_dim, int64_t hidden,
                                       int64_t w_stride, const void* norm_weight, int nw_dtype, void* folded,
                                       int64_t folded_stride, void* stream) {
  BFA_REQUIRE(qkv_weight && norm_weight && folded, "bfa_fold_rmsnorm_weight: null pointer");
  return launch_fold_weight(qkv_weight, w_dtype, qkv_dim, hidden, w_stride, norm_weight, nw_dtype, folded,
                            folded_stride, as_stream(stream));
}

extern "C" int bfa_rms_norm(const void* x, void* y, const void* weight, int x_dtype, int w_dtype,
                            int64_t rows, int64_t rows_inner, int64_t hidden,
                            int64_t x_stride_outer, int64_t x_stride_inner,
                            int64_t y_stride_outer, int64_t y_stride_inner, float eps,
                            void* stream) {
  const char* what = "bfa_rms_norm";
  BFA_REQUIRE(x && y && weight, "%s: null pointer", what);
  BFA_REQUIRE(is_float_dtype(x_dtype) && is_float_dtype(w_dtype), "%s: bad dtype", what);
  BFA_REQUIRE(rows >= 0 && rows_inner >= 1 && hidden >= 0, "%s: bad geometry", what);
  NormArgs a{};
  a.x = x; a.y = y; a.w = weight; a.w_dtype = w_dtype;
  a.rows = rows; a.rows_inner = rows_inner; a.hidden = hidden;
  a.x_so = x_stride_outer; a.x_si = x_stride_inner; a.x_sc = 1;
  a.y_so = y_stride_outer; a.y_si = y_stride_inner; a.y_sc = 1;
  a.eps = eps;
  const bool vec_ok = mult8(hidden) && mult8(x_stride_outer) && mult8(x_stride_inner) &&
                      mult8(y_stride_outer) && mult8(y_stride_inner) && aligned16(x) &&
                      aligned16(y) && aligned16(weight);
  return launch_norm_same<kRms>(x_dtype, a, vec_ok, as_stream(stream), what);
}

extern "C" int bfa_add_rms_norm(const void* x, const void* residual, void* y, void* residual_out,
                                const void* weight, int x_dtype, int w_dtype, int64_t rows,
                                int64_t hidden, int64_t x_stride, int64_t residual_stride,
                                int64_t y_stride, int64_t residual_out_stride, float eps,
                                void* stream) {
  const char* what = "bfa_add_rms_norm";
  BFA_REQUIRE(x && residual && y && weight, "%s: null pointer", what);
  BFA_REQUIRE(is_float_dtype(x_dtype) && is_float_dtype(w_dtype), "%s: bad dtype", what);
  BFA_REQUIRE(rows >= 0 && hidden >= 0, "%s: bad geometry", what);
  NormArgs a{};
  a.x = x; a.res = residual; a.y = y; a.res_out = residual_out; a.w = weight;
  a.w_dtype = w_dtype;
  a.rows = rows; a.rows_inner = 1; a.hidden = hidden;
  a.x_so = x_stride; a.x_si = 0; a.x_sc = 1;
  a.r_s = residual_stride; a.ro_s = residual_out_stride;
  a.y_so = y_stride; a.y_si = 0; a.y_sc = 1;
  a.eps = eps;
  const bool vec_ok = mult8(hidden) && mult8(x_stride) && mult8(residual_stride) &&
                      mult8(y_stride) && mult8(residual_out_stride) && aligned16(x) &&
                      aligned16(residual) && aligned16(y) && aligned16(weight) &&
                      (residual_out == nullptr || aligned16(residual_out));
  return launch_norm_same<kAddRms>(x_dtype, a, vec_ok, as_stream(stream), what);
}

extern "C" int bfa_rms_norm_f32(const void* x, float* y, const void* weight, int x_dtype,
                                int w_dtype, int64_t rows, int64_t hidden, int64_t x_stride_row,
                                int64_t x_stride_col, int64_t y_stride_row, int64_t y_stride_col,
                                float eps, void* stream) {
  const char* what = "bfa_rms_norm_f32";
  BFA_REQUIRE(x && y && weight, "%s: null pointer", what);
  BFA_REQUIRE(is_float_dtype(x_dtype) && is_float_dtype(w_dtype), "%s: bad dtype", what);
  BFA_REQUIRE(rows >= 0 && hidden >= 0, "%s: bad geometry", what);
  NormArgs a{};
  a.x = x; a.y = y; a.w = weight; a.w_dtype = w_dtype;
  a.rows = rows; a.rows_inner = 1; a.hidden = hidden;
  a.x_so = x_stride_row; a.x_si = 0; a.x_sc = x_stride_col;
  a.y_so = y_stride_row; a.y_si = 0; a.y_sc = y_stride_col;
  a.eps = eps;
  const bool vec_ok = x_stride_col == 1 && y_stride_col == 1 && mult8(hidden) &&
                      mult8(x_stride_row) && mult8(y_stride_row) && aligned16(x) &&
                      aligned16(y) && aligned16(weight);
  return launch_norm_out<BFA_DTYPE_F32, kF32>(x_dtype, a, vec_ok, as_stream(stream), what);
}

extern "C" int bfa_rmsnorm_qkv_operand(const void* x, int x_dtype, int64_t rows, int64_t hidden,
                                       int64_t x_stride, const void* norm_weight, int w_dtype,
                                       int mixed_rounding, void* operand, int operand_dtype,
                                       float eps, void* stream) {
  BFA_REQUIRE(x && norm_weight && operand, "bfa_rmsnorm_qkv_operand: null pointer");
  return launch_qkv_operand(x, x_dtype, rows, hidden, x_stride, norm_weight, w_dtype,
                            mixed_rounding != 0, operand, operand_dtype, eps, as_stream(stream));
}
