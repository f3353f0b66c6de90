// Device-side helpers shared by every braidinfer_amd kernel (gfx950, wave64).
//
// Storage types are handled as raw bits (uint16 for bf16/fp16) so that every
// rounding point is explicit: float -> bf16 goes through the hardware
// round-to-nearest-even conversion (v_cvt_pk_bf16_f32 on gfx950), which is the
// rounding torch uses for Tensor.to(torch.bfloat16).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <cstdlib>

#include "braidinfer_amd.h"

namespace bfa {

constexpr int kWave = 64;

// ---------------------------------------------------------------- scalar casts
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b) {
  return __uint_as_float(b << 16);
}
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}
// two floats -> two bf16 (round to nearest even) in one word, low element in
// the low half: a single v_cvt_pk_bf16_f32
typedef __bf16 bfa_bf16x2_t __attribute__((ext_vector_type(2)));
typedef float bfa_f32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((bfa_f32x2_t){lo, hi}, bfa_bf16x2_t));
}
__device__ __forceinline__ float f16_bits_to_f32(uint32_t b) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(b)));
}
__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

// Element traits: DT is one of BFA_DTYPE_{F32,F16,BF16}.
template <int DT> struct Elem;
template <> struct Elem<BFA_DTYPE_F32> {
  using T = float;
  static constexpr int kPer16B = 4;
  __device__ __forceinline__ static float to_f32(T v) { return v; }
  __device__ __forceinline__ static T from_f32(float v) { return v; }
  __device__ __forceinline__ static float round(float v) { return v; }
};
template <> struct Elem<BFA_DTYPE_F16> {
  using T = uint16_t;
  static constexpr int kPer16B = 8;
  __device__ __forceinline__ static float to_f32(T v) { return f16_bits_to_f32(v); }
  __device__ __forceinline__ static T from_f32(float v) { return f32_to_f16_bits(v); }
  __device__ __forceinline__ static float round(float v) { return f16_bits_to_f32(f32_to_f16_bits(v)); }
};
template <> struct Elem<BFA_DTYPE_BF16> {
  using T = uint16_t;
  static constexpr int kPer16B = 8;
  __device__ __forceinline__ static float to_f32(T v) { return bf16_bits_to_f32(v); }
  __device__ __forceinline__ static T from_f32(float v) { return f32_to_bf16_bits(v); }
  __device__ __forceinline__ static float round(float v) { return bf16_bits_to_f32(f32_to_bf16_bits(v)); }
};

__device__ __forceinline__ float round_bf16(float v) { return Elem<BFA_DTYPE_BF16>::round(v); }

// ------------------------------------------------------- 8-element vector I/O
// Loads/stores 8 consecutive elements as 16-byte (16-bit types) or 2x16-byte
// (fp32) vector accesses.  The caller guarantees 16-byte alignment.
template <int DT>
__device__ __forceinline__ void load8(const void* p, float (&v)[8]) {
  if constexpr (DT == BFA_DTYPE_F32) {
    const float4* q = reinterpret_cast<const float4*>(p);
    float4 a = q[0], b = q[1];
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  } else {
    uint4 u = *reinterpret_cast<const uint4*>(p);
    uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = Elem<DT>::to_f32(static_cast<uint16_t>(w[i] & 0xffffu));
      v[2 * i + 1] = Elem<DT>::to_f32(static_cast<uint16_t>(w[i] >> 16));
    }
  }
}

// NT: the nontemporal hint, for large outputs that are not read again soon
// (see stream_output below).
template <int DT, bool NT = false>
__device__ __forceinline__ void store8(void* p, const float (&v)[8]) {
  typedef unsigned u32x4_nt_t __attribute__((ext_vector_type(4)));
  if constexpr (DT == BFA_DTYPE_F32) {
    if constexpr (NT) {
      u32x4_nt_t* q = reinterpret_cast<u32x4_nt_t*>(p);
      __builtin_nontemporal_store(u32x4_nt_t{__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]),
                                             __float_as_uint(v[3])}, q);
      __builtin_nontemporal_store(u32x4_nt_t{__float_as_uint(v[4]), __float_as_uint(v[5]), __float_as_uint(v[6]),
                                             __float_as_uint(v[7])}, q + 1);
    } else {
      float4* q = reinterpret_cast<float4*>(p);
      q[0] = make_float4(v[0], v[1], v[2], v[3]);
      q[1] = make_float4(v[4], v[5], v[6], v[7]);
    }
  } else {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      w[i] = static_cast<uint32_t>(Elem<DT>::from_f32(v[2 * i])) |
             (static_cast<uint32_t>(Elem<DT>::from_f32(v[2 * i + 1])) << 16);
    }
    if constexpr (NT) {
      __builtin_nontemporal_store(u32x4_nt_t{w[0], w[1], w[2], w[3]}, reinterpret_cast<u32x4_nt_t*>(p));
    } else {
      *reinterpret_cast<uint4*>(p) = make_uint4(w[0], w[1], w[2], w[3]);
    }
  }
}

// Stores carry the nontemporal hint when an output is this large (SiLU*mul's
// activation, add+RMSNorm's residual): such an output cannot stay in the 256 MB
// Infinity Cache for its consumer anyway, and streaming it past the cache keeps
// what the next kernels read there.  SiLU*mul at 8192 x 14336 alone slows from
// 103 to 111 us with it, while the Llama-3-8B 8192-token layer chain
// (add+RMSNorm, fused QKV, SiLU*mul) goes from 542 to 507 us when one layer is
// repeated (its QKV weight then stays cached), and from 543 to 531.5 us with
// the weight rotating over four copies, as consecutive layers would.  Smaller
// outputs (decode batches) keep plain stores, so their consumers find them
// cached.
// Planner override BFA_TUNE_STREAM_STORES = 0 keeps every store plain (for
// measurements).
int tuning(int key);  // capi.hip
constexpr int64_t kStreamOutputBytes = int64_t(64) << 20;
inline bool stream_output(int64_t bytes) {
  return tuning(BFA_TUNE_STREAM_STORES) != 0 && bytes >= kStreamOutputBytes;
}

// Streaming forms: 16-byte loads with the nontemporal hint, for operands that
// are read exactly once (activations of the memory-bound kernels, gathered
// table rows).  Not displacing L2 and Infinity Cache lines for them took the
// SiLU*mul kernel from 5.6 to 6.8 TB/s at 8192 x 2 x 14336, and in the
// Llama-3-8B 8192-token layer chain add+RMSNorm from 70 to 51 us (a kernel
// repeated on the same input in isolation reads faster with plain loads, which
// keep the input in the Infinity Cache between repeats).
typedef unsigned bfa_u32x4_t __attribute__((ext_vector_type(4)));

template <bool NT = true>
__device__ __forceinline__ uint4 load16_nt(const void* p) {
  if constexpr (NT) {
    const bfa_u32x4_t u = __builtin_nontemporal_load(reinterpret_cast<const bfa_u32x4_t*>(p));
    return make_uint4(u.x, u.y, u.z, u.w);
  } else {
    return *reinterpret_cast<const uint4*>(p);
  }
}

template <int DT, bool NT = true>
__device__ __forceinline__ void load8_nt(const void* p, float (&v)[8]) {
  if constexpr (DT == BFA_DTYPE_F32) {
    const uint4 a = load16_nt<NT>(p), b = load16_nt<NT>(static_cast<const float*>(p) + 4);
    v[0] = __uint_as_float(a.x); v[1] = __uint_as_float(a.y); v[2] = __uint_as_float(a.z); v[3] = __uint_as_float(a.w);
    v[4] = __uint_as_float(b.x); v[5] = __uint_as_float(b.y); v[6] = __uint_as_float(b.z); v[7] = __uint_as_float(b.w);
  } else {
    const uint4 u = load16_nt<NT>(p);
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = Elem<DT>::to_f32(static_cast<uint16_t>(w[i] & 0xffffu));
      v[2 * i + 1] = Elem<DT>::to_f32(static_cast<uint16_t>(w[i] >> 16));
    }
  }
}

// Scalar element access (used by the unaligned fallback paths).
template <int DT>
__device__ __forceinline__ float load1(const void* p, int64_t i) {
  return Elem<DT>::to_f32(reinterpret_cast<const typename Elem<DT>::T*>(p)[i]);
}
template <int DT>
__device__ __forceinline__ void store1(void* p, int64_t i, float v) {
  reinterpret_cast<typename Elem<DT>::T*>(p)[i] = Elem<DT>::from_f32(v);
}

// Runtime-dtype scalar load for small operands (norm weights, bias).
__device__ __forceinline__ float load_any(const void* p, int dt, int64_t i) {
  if (dt == BFA_DTYPE_BF16) return load1<BFA_DTYPE_BF16>(p, i);
  if (dt == BFA_DTYPE_F16) return load1<BFA_DTYPE_F16>(p, i);
  return load1<BFA_DTYPE_F32>(p, i);
}

// ------------------------------------------------------- integer division
// n / d for 32-bit n < 2^31 and 1 <= d < 2^31 by multiply-high (the
// round-up reciprocal method of Granlund and Montgomery, "Division by invariant
// integers using multiplication", 1994): with s = ceil(log2 d) and
// m = floor(2^32 (2^s - d) / d) + 1, n / d = (mulhi(n, m) + n) >> s.  Built on
// the host, used in kernels whose flat index must be split into (row, column).
struct FastDiv {
  uint32_t d = 1, m = 1, s = 0;
  FastDiv() = default;
  __host__ explicit FastDiv(uint32_t div) : d(div) {
    s = 0;
    while ((uint64_t{1} << s) < div) ++s;
    m = static_cast<uint32_t>(((uint64_t{1} << 32) * ((uint64_t{1} << s) - div)) / div + 1);
  }
  __device__ __forceinline__ uint32_t div(uint32_t n) const { return (__umulhi(n, m) + n) >> s; }
};

// silu(g) = g * sigmoid(g), sigmoid(g) = 1 / (1 + 2^(-g * log2(e))), with the
// hardware exp2 and reciprocal (about 1 ulp each; the result is rounded to a
// 16-bit type by every caller)
__device__ __forceinline__ float silu_fast(float g) {
  const float e = __builtin_amdgcn_exp2f(g * -1.4426950408889634f);
  return g * __builtin_amdgcn_rcpf(1.0f + e);
}

// ------------------------------------------------------------- LDS DMA
typedef __attribute__((address_space(3))) void lds_void_t;

// LDS byte address of a __shared__ pointer, as a wave-uniform SGPR value.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return __builtin_amdgcn_readfirstlane(
      static_cast<uint32_t>(reinterpret_cast<uintptr_t>((const lds_void_t*)p)));
}

// Asynchronous 16-byte-per-lane copy global -> LDS (global_load_lds_dwordx4):
// lane i's 16 bytes at base + voff land at LDS byte m0 + 16*i.  Issued as
// inline assembly so the compiler does not serialise consecutive copies; the
// caller waits (wait_vmem) and barriers before the LDS is read.  m0 is a
// register the compiler reserves and assumes unchanged across an asm statement
// (listing it as clobbered has no effect), so the statement saves it and puts
// it back after the copy is issued (the copy reads m0 at issue).  The s_nop is
// the one wait state the ISA requires between an SALU write of m0 and a global
// load with the LDS bit.
__device__ __forceinline__ void dma16(const void* base, uint32_t voff, uint32_t m0) {
  // the base is wave-uniform; readfirstlane lets the compiler see that when the
  // pointer came through a path it cannot prove uniform (an SGPR operand).  The
  // builtin returns a signed int: each half is taken back to uint32_t before it
  // is widened, or a low half with bit 31 set would fill the high word with ones.
  const uint64_t b = reinterpret_cast<uint64_t>(base);
  const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(b)));
  const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(b >> 32)));
  const uint64_t bu = (static_cast<uint64_t>(hi) << 32) | lo;
  uint32_t saved;
  asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %2, %3\n\ts_mov_b32 m0, %0"
               : "=&s"(saved)
               : "s"(__builtin_amdgcn_readfirstlane(m0)), "v"(voff), "s"(reinterpret_cast<const void*>(bu))
               : "memory");
}

// 4-byte form of dma16: lane i's dword at base + voff goes to LDS m0 + 4 i
// (m0 saved and restored, and the wait state, as there).
__device__ __forceinline__ void dma4(const void* base, uint32_t voff, uint32_t m0) {
  const uint64_t b = reinterpret_cast<uint64_t>(base);
  const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(b)));
  const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(b >> 32)));
  const uint64_t bu = (static_cast<uint64_t>(hi) << 32) | lo;
  uint32_t saved;
  asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %2, %3\n\ts_mov_b32 m0, %0"
               : "=&s"(saved)
               : "s"(__builtin_amdgcn_readfirstlane(m0)), "v"(voff), "s"(reinterpret_cast<const void*>(bu))
               : "memory");
}

// waits for every vector memory request of this wave, the LDS DMAs included
__device__ __forceinline__ void wait_vmem() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// ------------------------------------------------------------- reductions
// Butterfly sum over aligned groups of L lanes (L a power of two <= 64).
template <int L>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int m = L / 2; m >= 1; m >>= 1) v += __shfl_xor(v, m, kWave);
  return v;
}

// Lane permutations inside a 16-lane DPP row (no LDS round trip, unlike
// __shfl_xor, which goes through ds_bpermute).  Control codes of the gfx9 DPP
// encoding: quad_perm [1,0,3,2] = 0xB1, quad_perm [2,3,0,1] = 0x4E,
// row_half_mirror (lane i <- 7 - i within 8) = 0x141, row_mirror (lane i <-
// 15 - i within 16) = 0x140.
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
// Sum over aligned groups of 8 lanes; every lane of a group gets the same bits
// (each step adds a pair of partial sums in commutable order).
__device__ __forceinline__ float group8_sum_dpp(float v) {
  v += dpp_f32<0xB1>(v);
  v += dpp_f32<0x4E>(v);
  v += dpp_f32<0x141>(v);
  return v;
}
// Sum / maximum over aligned groups of 16 lanes, the same bits in every lane.
__device__ __forceinline__ float group16_sum_dpp(float v) {
  v = group8_sum_dpp(v);
  return v + dpp_f32<0x140>(v);
}
__device__ __forceinline__ float group16_max_dpp(float v) {
  v = fmaxf(v, dpp_f32<0xB1>(v));
  v = fmaxf(v, dpp_f32<0x4E>(v));
  v = fmaxf(v, dpp_f32<0x141>(v));
  return fmaxf(v, dpp_f32<0x140>(v));
}

// Sum over aligned groups of L lanes (L = 1, 2, 4, 8, 16) on DPP; every lane of
// a group gets the same bits.
template <int L>
__device__ __forceinline__ float group_sum_dpp(float v) {
  static_assert(L == 1 || L == 2 || L == 4 || L == 8 || L == 16, "DPP row groups");
  if constexpr (L >= 2) v += dpp_f32<0xB1>(v);
  if constexpr (L >= 4) v += dpp_f32<0x4E>(v);
  if constexpr (L >= 8) v += dpp_f32<0x141>(v);
  if constexpr (L >= 16) v += dpp_f32<0x140>(v);
  return v;
}

// Reductions over lanes l, l ^ 16, l ^ 32, l ^ 48 with the gfx950 lane swaps.
// v_permlane16_swap x, y exchanges the odd 16-lane rows of x with the even rows
// of y; with x = y = v on entry, each lane ends up holding its own value in one
// of x, y and its xor-16 partner's in the other (v_permlane32_swap: halves, xor
// 32), so a commutative op on the pair gives every lane of the group the same
// bits.  Written as inline assembly: given one value for both operands, the
// compiler's model of the builtins takes the two results to be equal and drops
// one of them.  The s_nop covers the VALU-write -> permlane-read wait states.
__device__ __forceinline__ void swap16(uint32_t& x, uint32_t& y) {
  asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1\n\ts_nop 1" : "+v"(x), "+v"(y));
}
__device__ __forceinline__ void swap32(uint32_t& x, uint32_t& y) {
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(x), "+v"(y));
}
__device__ __forceinline__ float lanes4_max(float v) {
  uint32_t x = __builtin_bit_cast(uint32_t, v), y = x;
  swap16(x, y);
  v = fmaxf(__builtin_bit_cast(float, x), __builtin_bit_cast(float, y));
  x = y = __builtin_bit_cast(uint32_t, v);
  swap32(x, y);
  return fmaxf(__builtin_bit_cast(float, x), __builtin_bit_cast(float, y));
}
__device__ __forceinline__ float lanes4_sum(float v) {
  uint32_t x = __builtin_bit_cast(uint32_t, v), y = x;
  swap16(x, y);
  v = __builtin_bit_cast(float, x) + __builtin_bit_cast(float, y);
  x = y = __builtin_bit_cast(uint32_t, v);
  swap32(x, y);
  return __builtin_bit_cast(float, x) + __builtin_bit_cast(float, y);
}

// Sum over all 64 lanes without LDS: DPP inside each 16-lane row, then the two
// lane swaps; every lane gets the same bits.
__device__ __forceinline__ float wave_sum_dpp(float v) { return lanes4_sum(group16_sum_dpp(v)); }

// Device status word: kernels that detect out-of-range indices OR a bit into
// it with an ordinary store (every writer stores the same value).
__device__ __forceinline__ void flag_status(int* status, int bit) {
  if (status) atomicOr(status, bit);
}

}  // namespace bfa
