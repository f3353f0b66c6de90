// Launchers shared between translation units of the library.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace bfa {

// Normalised QKV operand pre-pass (norm.hip): out[rows, hidden] (bf16 or fp16)
//   mixed:  round_out(round_bf16(x / rms) * w)
//   else:   round_out((x / rms) * w)            rms = sqrt(sum(x^2)/hidden + eps)
int launch_qkv_operand(const void* x, int x_dtype, int64_t rows, int64_t hidden, int64_t x_stride,
                       const void* w, int w_dtype, bool mixed, void* out, int out_dtype,
                       float eps, hipStream_t s);

}  // namespace bfa
