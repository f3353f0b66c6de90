// SiluAndMul (layers/activation.py:11-13):  g, u = x.chunk(2, -1);  y = F.silu(g) * u
//
// torch rounds twice for a reduced-float x: F.silu computes g/(1+exp(-g)) in
// fp32 and rounds to the tensor dtype, then the product of two reduced-float
// tensors is computed in fp32 and rounded again.  The kernel keeps both
// rounding points.  Each lane owns 8 consecutive outputs: one 16-byte load of
// gate, one of up, one 16-byte store (fp32: two of each), so a row of
// [T, 2I] is streamed once and the [T, I] result written once.
#include "bfa_device.h"
#include "bfa_host.h"

namespace bfa {

struct SwigluArgs {
  const void* x;
  void* y;
  int64_t rows, inter, x_stride, y_stride;
  int64_t chunks_per_row;  // inter / 8
  int64_t total;           // rows * chunks_per_row
};

__device__ __forceinline__ float silu_f32(float g) { return g / (1.0f + expf(-g)); }

template <int DT>
__global__ __launch_bounds__(256) void silu_mul_vec_kernel(SwigluArgs a) {
  using T = typename Elem<DT>::T;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
  for (int64_t item = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; item < a.total;
       item += stride) {
    const int64_t row = item / a.chunks_per_row;
    const int64_t col = (item - row * a.chunks_per_row) * 8;
    const T* xr = static_cast<const T*>(a.x) + row * a.x_stride;
    float g[8], u[8], o[8];
    load8<DT>(xr + col, g);
    load8<DT>(xr + a.inter + col, u);
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = Elem<DT>::round(silu_f32(g[i])) * u[i];
    store8<DT>(static_cast<T*>(a.y) + row * a.y_stride + col, o);
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
    store1<DT>(a.y, row * a.y_stride + col, Elem<DT>::round(silu_f32(g)) * u);
  }
}

template <int DT>
static void launch_silu(const SwigluArgs& a, bool vec, hipStream_t s) {
  // Grid: enough workgroups to cover the tensor once, capped so that each lane
  // loops a few times on large tensors (256 CUs x 16 resident workgroups).
  const int64_t items = vec ? a.total : a.rows * a.inter;
  const int64_t grid = std::max<int64_t>(1, std::min<int64_t>(cdiv(items, 256), 256 * 16));
  if (vec) {
    hipLaunchKernelGGL((silu_mul_vec_kernel<DT>), dim3(grid), dim3(256), 0, s, a);
  } else {
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
  a.chunks_per_row = inter / 8;
  a.total = rows * a.chunks_per_row;
  const bool vec = inter % 8 == 0 && x_row_stride % 8 == 0 && y_row_stride % 8 == 0 &&
                   aligned16(x) && aligned16(y);
  const hipStream_t s = as_stream(stream);
  switch (dtype) {
    case BFA_DTYPE_BF16: launch_silu<BFA_DTYPE_BF16>(a, vec, s); break;
    case BFA_DTYPE_F16: launch_silu<BFA_DTYPE_F16>(a, vec, s); break;
    default: launch_silu<BFA_DTYPE_F32>(a, vec, s); break;
  }
  return check_launch(what);
}
