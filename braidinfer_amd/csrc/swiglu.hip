// SiluAndMul (layers/activation.py:11-13):  g, u = x.chunk(2, -1);  y = F.silu(g) * u
//
// torch rounds twice for a reduced-float x: F.silu computes g/(1+exp(-g)) in
// fp32 and rounds to the tensor dtype, then the product of two reduced-float
// tensors is computed in fp32 and rounded again.  The kernel keeps both
// rounding points.  Each lane owns 2 x 8 outputs of one flattened
// (row, 8-column chunk) index space: two 16-byte loads of gate and of up are in
// flight together, then two 16-byte stores, so a row of [T, 2I] is streamed once
// and the [T, I] result written once.
//
// The arithmetic is kept small enough that the kernel stays bound by HBM: the
// sigmoid is 1/(1 + 2^(-g log2 e)) with the hardware base-2 exponential and
// reciprocal (v_exp_f32, v_rcp_f32; about 1 ulp each in fp32, far below the
// bf16 rounding that follows), and the chunk index is split into (row, column)
// with a 32-bit multiply-high division instead of a 64-bit divide.
#include "bfa_device.h"
#include "bfa_host.h"

namespace bfa {

struct SwigluArgs {
  const void* x;
  void* y;
  int64_t rows, inter, x_stride, y_stride;
  FastDiv cpr;      // division by chunks per row (inter / 8)
  uint32_t total;   // rows * chunks per row (< 2^31)
};

constexpr int kSwigluPerLane = 2;  // 8-column chunks per lane

template <int DT, bool NT>
__global__ __launch_bounds__(256) void silu_mul_vec_kernel(SwigluArgs a) {
  constexpr int U = kSwigluPerLane;
  using T = typename Elem<DT>::T;
  const uint32_t item0 = blockIdx.x * (256u * U) + threadIdx.x;
  float g[U][8], u[U][8];
  int64_t yoff[U];
#pragma unroll
  for (int c = 0; c < U; ++c) {
    const uint32_t item = item0 + c * 256u;
    yoff[c] = -1;
    if (item < a.total) {
      const uint32_t row = a.cpr.div(item);
      const uint32_t col = (item - row * a.cpr.d) * 8u;
      const T* xr = static_cast<const T*>(a.x) + row * a.x_stride + col;
      load8_nt<DT>(xr, g[c]);
      load8_nt<DT>(xr + a.inter, u[c]);
      yoff[c] = row * a.y_stride + col;
    }
  }
#pragma unroll
  for (int c = 0; c < U; ++c) {
    if (yoff[c] < 0) continue;
    float o[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = Elem<DT>::round(silu_fast(g[c][i])) * u[c][i];
    store8<DT, NT>(static_cast<T*>(a.y) + yoff[c], o);
  }
}

template <int DT>
__global__ __launch_bounds__(256) void silu_mul_scalar_kernel(SwigluArgs a) {
  const int64_t total = a.rows * a.inter;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
  for (int64_t item = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; item < total;
       item += stride) {
    const int64_t row = item / a.inter;
    const int64_t col = item - row * a.inter;
    const float g = load1<DT>(a.x, row * a.x_stride + col);
    const float u = load1<DT>(a.x, row * a.x_stride + a.inter + col);
    store1<DT>(a.y, row * a.y_stride + col, Elem<DT>::round(silu_fast(g)) * u);
  }
}

template <int DT>
static void launch_silu(const SwigluArgs& a, bool vec, hipStream_t s) {
  if (vec) {
    const int64_t grid = std::max<int64_t>(1, cdiv(a.total, 256 * kSwigluPerLane));
    if (stream_output(a.rows * a.inter * static_cast<int64_t>(sizeof(typename Elem<DT>::T))))
      hipLaunchKernelGGL((silu_mul_vec_kernel<DT, true>), dim3(grid), dim3(256), 0, s, a);
    else
      hipLaunchKernelGGL((silu_mul_vec_kernel<DT, false>), dim3(grid), dim3(256), 0, s, a);
  } else {
    // grid-stride: enough workgroups to cover the tensor once, capped so that
    // each lane loops a few times on large tensors (256 CUs x 16 workgroups)
    const int64_t grid = std::max<int64_t>(1, std::min<int64_t>(cdiv(a.rows * a.inter, 256), 256 * 16));
    hipLaunchKernelGGL((silu_mul_scalar_kernel<DT>), dim3(grid), dim3(256), 0, s, a);
  }
}

}  // namespace bfa

using namespace bfa;

extern "C" int bfa_silu_and_mul(const void* x, void* y, int dtype, int64_t rows, int64_t inter,
                                int64_t x_row_stride, int64_t y_row_stride, void* stream) {
  const char* what = "bfa_silu_and_mul";
  BFA_REQUIRE(is_float_dtype(dtype), "%s: bad dtype", what);
  BFA_REQUIRE(rows >= 0 && inter >= 0, "%s: bad geometry", what);
  if (rows == 0 || inter == 0) return BFA_OK;
  BFA_REQUIRE(x && y, "%s: null pointer", what);
  SwigluArgs a{};
  a.x = x; a.y = y; a.rows = rows; a.inter = inter;
  a.x_stride = x_row_stride; a.y_stride = y_row_stride;
  const int64_t total = rows * (inter / 8);
  const bool vec = inter % 8 == 0 && x_row_stride % 8 == 0 && y_row_stride % 8 == 0 &&
                   aligned16(x) && aligned16(y) && total < (int64_t{1} << 31);
  if (vec) {
    a.cpr = FastDiv(static_cast<uint32_t>(inter / 8));
    a.total = static_cast<uint32_t>(total);
  }
  const hipStream_t s = as_stream(stream);
  switch (dtype) {
    case BFA_DTYPE_BF16: launch_silu<BFA_DTYPE_BF16>(a, vec, s); break;
    case BFA_DTYPE_F16: launch_silu<BFA_DTYPE_F16>(a, vec, s); break;
    default: launch_silu<BFA_DTYPE_F32>(a, vec, s); break;
  }
  return check_launch(what);
}
