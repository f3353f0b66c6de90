// Fused RMSNorm + QKV projection (+ bias, + per-head q/k RMSNorm, + RoPE) on gfx950.
//
// Reference semantics (braidinfer/kernels/fused_rmsnorm_qkv_*.py and the model
// glue that consumes their output):
//   operand   n = RMSNorm(x) with the variant's rounding points   (norm.hip pre-pass)
//   project   y = n @ W^T (+ bias), fp32 accumulation, rounded to the variant's
//             output dtype (bf16 for mixed/production, none for the f32 ones)
//   q/k norm  Qwen3: q_norm(q.float()).to(dtype), k_norm(k.float()).to(dtype)
//             (models/qwen3.py:257-281), RMSNorm over head_dim in fp32
//   rope      RotaryEmbedding.forward on q and k (layers/rotary_embedding.py:49-65),
//             fp32 math, result rounded to the dtype it was given
//   store     .to(out dtype) (models/llama.py:200-205, qwen3.py:280-336)
// W is the packed [q rows; k rows; v rows] x hidden matrix of
// QKVParallelLinear (layers/linear.py:78-114).
//
// Kernels
//  * qkv_gemm_kernel   prefill.  BMxBN tile per workgroup of 4 or 8 waves, each
//    wave WMx128: v_mfma_f32_16x16x32_{bf16,f16} on the 64-deep DMA path,
//    v_mfma_f32_32x32x16 on the 32-deep rings and the register-staged path;
//    256x256 with 8 waves (two per SIMD) for large token counts.  Operand and weight K-slices move HBM ->
//    LDS by LDS DMA (global_load_lds_dwordx4) into XOR-swizzled buffers, so the
//    MFMA fragment reads spread over the banks; unaligned or odd K goes through a
//    register-staged path with masking.  The epilogue stages each wave's
//    accumulators through a wave-private LDS slice and runs bias / rounding / q-k
//    RMSNorm / RoPE / store per (row, head) with 16 lanes per row.
//  * qkv_decode_kernel decode (T <= 64).  The weight stream dominates, so the grid
//    is (128-column tiles) x (K splits) to put every CU on the weight; weight rows
//    are loaded 8 lanes per row into registers and transposed through a small
//    wave-private LDS area into 16x16x32 MFMA fragments; fp32 partial tiles go to
//    the workspace.  qkv_splitk_kernel (fragments loaded straight from memory,
//    K masked) covers hidden sizes that are not a multiple of 64.
//  * qkv_decode_epilogue_kernel / qkv_epilogue_kernel sum the split-K partials (or
//    read the raw fp32 projection for head_dim the GEMM epilogue does not cover)
//    and apply bias / q-k norm / RoPE / rounding per (token, head) row.
//  * qkv_decode_pair_kernel  17-64 decode tokens without q/k norm: a workgroup
//    owns 16 RoPE column pairs for the whole of K (its waves split K, each
//    streaming its segments by LDS DMA through a private ring), so the projection,
//    the fp32 variants' RMSNorm (gamma on the weight fragments, row sums of
//    squares from the operand fragments), bias, RoPE and the KV append run in
//    one launch with no partials.
#include <cstdlib>
#include <mutex>

#include "bfa_append.h"
#include "bfa_device.h"
#include "bfa_host.h"
#include "bfa_internal.h"
#include "bfa_qkv.h"

namespace bfa {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(8))) _Float16 f16x8_t;
typedef __attribute__((ext_vector_type(16))) float f32x16_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;

template <bool BF16>
__device__ __forceinline__ f32x16_t mfma32(const uint4& a, const uint4& b, f32x16_t c) {
  if constexpr (BF16) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a),
                                                  __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
  }
}

template <bool BF16>
__device__ __forceinline__ f32x4_t mfma16(const uint4& a, const uint4& b, f32x4_t c) {
  if constexpr (BF16) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                  __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
  }
}

// Stores 4 consecutive elements (8-byte / 16-byte vector store; the caller
// guarantees the alignment: column multiple of 4, row stride multiple of 4).
__device__ __forceinline__ void store4_any(void* p, int dt, int64_t i, const float (&v)[4]) {
  if (dt == BFA_DTYPE_F32) {
    *reinterpret_cast<float4*>(static_cast<float*>(p) + i) = make_float4(v[0], v[1], v[2], v[3]);
  } else {
    uint32_t w0, w1;
    if (dt == BFA_DTYPE_BF16) {
      w0 = f32_to_bf16_bits(v[0]) | (static_cast<uint32_t>(f32_to_bf16_bits(v[1])) << 16);
      w1 = f32_to_bf16_bits(v[2]) | (static_cast<uint32_t>(f32_to_bf16_bits(v[3])) << 16);
    } else {
      w0 = f32_to_f16_bits(v[0]) | (static_cast<uint32_t>(f32_to_f16_bits(v[1])) << 16);
      w1 = f32_to_f16_bits(v[2]) | (static_cast<uint32_t>(f32_to_f16_bits(v[3])) << 16);
    }
    *reinterpret_cast<uint2*>(static_cast<uint16_t*>(p) + i) = make_uint2(w0, w1);
  }
}

// Branch-free forms for the GEMM epilogue, whose code is unrolled over every
// row a lane owns: a rounding or store that dispatches on the dtype with
// branches there grew the kernel past the instruction cache.  dt is uniform.
__device__ __forceinline__ float round_sel(float v, int dt) {
  const float rb = Elem<BFA_DTYPE_BF16>::round(v);
  const float rh = Elem<BFA_DTYPE_F16>::round(v);
  return dt == BFA_DTYPE_BF16 ? rb : (dt == BFA_DTYPE_F16 ? rh : v);
}

__device__ __forceinline__ uint32_t pack2_sel(float lo, float hi, bool bf) {
  const uint32_t b = f32_to_bf16_bits(lo) | (static_cast<uint32_t>(f32_to_bf16_bits(hi)) << 16);
  const uint32_t h = f32_to_f16_bits(lo) | (static_cast<uint32_t>(f32_to_f16_bits(hi)) << 16);
  return bf ? b : h;
}

// 4 consecutive elements (column multiple of 4, row stride multiple of 4):
// one 16-byte store for fp32, one 8-byte store for the 16-bit types.
__device__ __forceinline__ void store4_sel(void* p, int dt, int64_t i, const float (&v)[4]) {
  if (dt == BFA_DTYPE_F32) {
    *reinterpret_cast<float4*>(static_cast<float*>(p) + i) = make_float4(v[0], v[1], v[2], v[3]);
  } else {
    const bool bf = dt == BFA_DTYPE_BF16;
    *reinterpret_cast<uint2*>(static_cast<uint16_t*>(p) + i) =
        make_uint2(pack2_sel(v[0], v[1], bf), pack2_sel(v[2], v[3], bf));
  }
}

// Epilogue dtype forms of the GEMM kernel.  EDT_RT reads every rounding and
// store dtype from QkvEpi at run time (the branch-free selects above: each
// rounds both ways and picks one).  The fixed forms compile the dtypes in for
// the two combinations the decoders run, so a rounding is one conversion:
//   EDT_F32_BF16  fp32 projection, no q/k norm, RoPE in fp32, bf16 store
//                 (the Llama chain: minimal_f32 -> rotary_emb -> .to(bf16))
//   EDT_BF16      every rounding point bf16 (the Qwen3 chain, the bf16 linears)
enum { EDT_RT = 0, EDT_F32_BF16 = 1, EDT_BF16 = 2 };
template <int EDT> struct EpiDt { static constexpr int Q = -1, N = -1, A = -1, O = -1, M = -1; };
template <> struct EpiDt<EDT_F32_BF16> {
  static constexpr int Q = BFA_DTYPE_F32, N = -1, A = BFA_DTYPE_F32, O = BFA_DTYPE_BF16, M = -1;
};
template <> struct EpiDt<EDT_BF16> {
  static constexpr int Q = BFA_DTYPE_BF16, N = BFA_DTYPE_BF16, A = BFA_DTYPE_BF16,
                       O = BFA_DTYPE_BF16, M = BFA_DTYPE_BF16;
};

// Rounding to DT (compile time) or to the run-time dtype dt when DT < 0.
template <int DT>
__device__ __forceinline__ float rnd(float v, int dt) {
  if constexpr (DT < 0) return round_sel(v, dt);
  else return Elem<DT>::round(v);
}

template <int DT>
__device__ __forceinline__ void store4_dt(void* p, int dt, int64_t i, const float (&v)[4]) {
  if constexpr (DT < 0) {
    store4_sel(p, dt, i, v);
  } else if constexpr (DT == BFA_DTYPE_F32) {
    *reinterpret_cast<float4*>(static_cast<float*>(p) + i) = make_float4(v[0], v[1], v[2], v[3]);
  } else {
    using E = Elem<DT>;
    *reinterpret_cast<uint2*>(static_cast<uint16_t*>(p) + i) =
        make_uint2(E::from_f32(v[0]) | (static_cast<uint32_t>(E::from_f32(v[1])) << 16),
                   E::from_f32(v[2]) | (static_cast<uint32_t>(E::from_f32(v[3])) << 16));
  }
}

// 8 consecutive elements (column multiple of 8, 16-byte aligned row).
template <int DT>
__device__ __forceinline__ void store8_dt(void* p, int dt, int64_t i, const float (&y)[8]) {
  if constexpr (DT >= 0) {
    store8<DT>(static_cast<char*>(p) + i * (DT == BFA_DTYPE_F32 ? 4 : 2), y);
  } else if (dt == BFA_DTYPE_F32) {
    float4* q = reinterpret_cast<float4*>(static_cast<float*>(p) + i);
    q[0] = make_float4(y[0], y[1], y[2], y[3]);
    q[1] = make_float4(y[4], y[5], y[6], y[7]);
  } else {
    const bool bf = dt == BFA_DTYPE_BF16;
    *reinterpret_cast<uint4*>(static_cast<uint16_t*>(p) + i) =
        make_uint4(pack2_sel(y[0], y[1], bf), pack2_sel(y[2], y[3], bf),
                   pack2_sel(y[4], y[5], bf), pack2_sel(y[6], y[7], bf));
  }
}




__device__ __forceinline__ int64_t epi_position(const QkvEpi& e, int64_t row, bool& ok) {
  int64_t p = e.pos_is_i64 ? static_cast<const int64_t*>(e.positions)[row]
                           : static_cast<const int32_t*>(e.positions)[row];
  if (p < 0) p += e.max_pos;
  ok = p >= 0 && p < e.max_pos;
  return ok ? p : 0;
}

// ============================================================ prefill GEMM
struct GemmArgs {
  const uint16_t* a;  // operand [m, k]
  const uint16_t* w;  // weight  [n, k] ([2 n, k] gate rows then up rows for EPI_SWIGLU)
  int64_t m, n, k, lda, ldw;  // n: output columns
  float* raw;         // EPI_RAW: fp32 [m, n] destination
};

// EPI_RAW: fp32 tile out.  EPI_FUSED: the QKV row epilogue (bias, q/k norm,
// RoPE).  EPI_LINEAR: rounding, + residual, rounding.  EPI_SWIGLU: each
// 128-column wave tile holds 64 gate columns and the 64 matching up columns,
// and the epilogue writes SiLU(gate) * up.
enum { EPI_RAW = 0, EPI_FUSED = 1, EPI_LINEAR = 2, EPI_SWIGLU = 3 };

// Output columns one BN-wide weight tile yields.
template <int EPI, int BN>
constexpr int out_cols() { return EPI == EPI_SWIGLU ? BN / 2 : BN; }

// Weight row that feeds column c (0 <= c < BN) of the tile starting at output
// column n0, clamped to the matrix.  EPI_SWIGLU: wave tile w = c / 128 takes
// gate rows n0 + 64 w .. +63 in its first 64 columns and the up rows n + the
// same in its last 64, so a lane holds both factors of an output element.
template <int EPI>
__device__ __forceinline__ int64_t weight_row(const GemmArgs& g, int64_t n0, int c) {
  if constexpr (EPI == EPI_SWIGLU) {
    const int cc = c & 127;
    const int64_t o = min(n0 + (c >> 7) * 64 + (cc & 63), g.n - 1);
    return cc < 64 ? o : g.n + o;
  } else {
    return min(n0 + c, g.n - 1);
  }
}

// LDS tile rows are 64 elements = 8 granules of 16 bytes; granule g of row r is
// stored at slot g ^ ((r / 2) & 7).  A 16-lane phase of a ds_read_b128 fragment
// load reads one granule of 16 consecutive rows: rows r and r + 1 sit in
// different halves of a 256-byte bank line and r / 2 spreads the eight pairs
// over all eight 16-byte slots, so the 16 reads hit 16 distinct bank groups.
__device__ __forceinline__ int swz(int r, int g) { return r * 8 + (g ^ ((r >> 1) & 7)); }

// Loads the MFMA fragments of K sub-step ks (16 deep) from an LDS tile buffer.
template <int MB, int NB, int BM, int WM, int WN>
__device__ __forceinline__ void load_frags(const uint4* buf, int ks, int wm, int wn, int frow,
                                           int fhalf, uint4 (&af)[MB], uint4 (&bf)[NB]) {
  const int gsel = ks * 2 + fhalf;
#pragma unroll
  for (int i = 0; i < MB; ++i) af[i] = buf[swz(wm * WM + i * 32 + frow, gsel)];
#pragma unroll
  for (int j = 0; j < NB; ++j) bf[j] = buf[BM * 8 + swz(wn * WN + j * 32 + frow, gsel)];
}

template <int MB, int NB, bool BF16>
__device__ __forceinline__ void mfma_block(f32x16_t (&acc)[MB][NB], const uint4 (&af)[MB],
                                           const uint4 (&bf)[NB]) {
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int j = 0; j < NB; ++j) acc[i][j] = mfma32<BF16>(af[i], bf[j], acc[i][j]);
}

// 16x16x32 fragments of a 64-deep tile (the 64-deep DMA path): sub-step ks (0
// or 1) is 32 deep, and lane l reads row l % 16 of each 16-row block at granule
// 4 ks + l / 16.  A 16-lane phase still reads one granule of 16 consecutive
// rows, so swz() keeps the reads on 16 distinct bank groups.
template <int MB16, int BM, int WM>
__device__ __forceinline__ void load_a16(const uint4* buf, int ks, int wm, int lane, uint4 (&af)[MB16]) {
  const int r = lane & 15, gsel = ks * 4 + (lane >> 4);
#pragma unroll
  for (int i = 0; i < MB16; ++i) af[i] = buf[swz(wm * WM + i * 16 + r, gsel)];
}

// half h (0 or 1) of the wave's 16-column weight blocks
template <int NH, int BM, int WN>
__device__ __forceinline__ void load_b16(const uint4* buf, int ks, int h, int wn, int lane, uint4 (&bf)[NH]) {
  const int r = lane & 15, gsel = ks * 4 + (lane >> 4);
#pragma unroll
  for (int j = 0; j < NH; ++j) bf[j] = buf[BM * 8 + swz(wn * WN + (h * NH + j) * 16 + r, gsel)];
}

template <int MB16, int NB16, int NH, bool BF16>
__device__ __forceinline__ void mfma_half16(f32x4_t (&acc)[MB16][NB16], const uint4 (&af)[MB16],
                                            const uint4 (&bf)[NH], int h) {
#pragma unroll
  for (int i = 0; i < MB16; ++i)
#pragma unroll
    for (int j = 0; j < NH; ++j) acc[i][h * NH + j] = mfma16<BF16>(af[i], bf[j], acc[i][h * NH + j]);
}
// An empty statement that takes the accumulators in and out: every MFMA before
// it in program order is issued before it, and none after it moves above it.
template <int R, int C>
__device__ __forceinline__ void pin_acc(f32x4_t (&acc)[R][C]) {
#pragma unroll
  for (int i = 0; i < R; ++i)
#pragma unroll
    for (int j = 0; j < C; ++j) asm volatile("" : "+v"(acc[i][j]));
}

// s_waitcnt vmcnt(N) for a compile-time N, other counters untouched
// (gfx9 encoding: vmcnt[3:0], expcnt[6:4], lgkmcnt[11:8], vmcnt[5:4] in [15:14]).
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// 32-deep K stages (DMA path): rows of 4 granules of 16 bytes; granule g of row
// r sits at slot g ^ ((r / 4) & 3), so a 16-lane phase of a fragment read (one
// granule of 16 consecutive rows) hits 16 distinct bank groups.
__device__ __forceinline__ int sw32(int r, int g) { return r * 4 + (g ^ ((r >> 2) & 3)); }

template <int MB, int NB, int BM, int WM, int WN>
__device__ __forceinline__ void load_frags32(const uint4* st, int ks, int wm, int wn, int frow,
                                             int fhalf, uint4 (&af)[MB], uint4 (&bf)[NB]) {
  const int gsel = ks * 2 + fhalf;
#pragma unroll
  for (int i = 0; i < MB; ++i) af[i] = st[sw32(wm * WM + i * 32 + frow, gsel)];
#pragma unroll
  for (int j = 0; j < NB; ++j) bf[j] = st[BM * 4 + sw32(wn * WN + j * 32 + frow, gsel)];
}

// One stage (BK deep) of both operands by DMA: each of the NW waves moves 1 KiB
// blocks (block b = NW i + wid; the wave's own block offset is folded into
// lstage); the weight blocks follow the BM operand rows of BK * 2 bytes.
template <int ADPW, int BDPW, int BM, int BK, int NW>
__device__ __forceinline__ void issue_stage(const uint16_t* a, const uint16_t* w, int64_t kt,
                                            const uint32_t (&aoff)[ADPW],
                                            const uint32_t (&boff)[BDPW], uint32_t lstage) {
  const uint16_t* ak = a + kt * BK;
  const uint16_t* wk = w + kt * BK;
#pragma unroll
  for (int i = 0; i < ADPW; ++i) dma16(ak, aoff[i], lstage + i * NW * 1024);
#pragma unroll
  for (int i = 0; i < BDPW; ++i) dma16(wk, boff[i], lstage + BM * BK * 2 + i * NW * 1024);
}

// Waits until at most `later` (< NS) stages of DPW DMAs each are still in flight.
template <int DPW, int NS>
__device__ __forceinline__ void wait_stages(int64_t later) {
  static_assert(NS >= 2 && NS <= 6, "cases below cover up to 5 later stages");
  static_assert(DPW * (NS - 1) < 64, "vmcnt range");
  if (NS > 5 && later >= 5) wait_vm<(NS > 5 ? 5 : 0) * DPW>();
  else if (NS > 4 && later >= 4) wait_vm<(NS > 4 ? 4 : 0) * DPW>();
  else if (NS > 3 && later >= 3) wait_vm<(NS > 3 ? 3 : 0) * DPW>();
  else if (NS > 2 && later >= 2) wait_vm<(NS > 2 ? 2 : 0) * DPW>();
  else if (later >= 1) wait_vm<DPW>();
  else wait_vm<0>();
}

// First three 16-deep K sub-steps of a tile (fragments of sub-step 0 are in
// fa0/fb0 on entry; sub-step 3's are left in fa1/fb1 for the caller).
template <int MB, int NB, int BM, int WM, int WN, bool BF16>
__device__ __forceinline__ void compute3(const uint4* cur, int wm, int wn, int frow, int fhalf,
                                         f32x16_t (&acc)[MB][NB], uint4 (&fa0)[MB], uint4 (&fb0)[NB],
                                         uint4 (&fa1)[MB], uint4 (&fb1)[NB]) {
  load_frags<MB, NB, BM, WM, WN>(cur, 1, wm, wn, frow, fhalf, fa1, fb1);
  mfma_block<MB, NB, BF16>(acc, fa0, fb0);
  load_frags<MB, NB, BM, WM, WN>(cur, 2, wm, wn, frow, fhalf, fa0, fb0);
  mfma_block<MB, NB, BF16>(acc, fa1, fb1);
  load_frags<MB, NB, BM, WM, WN>(cur, 3, wm, wn, frow, fhalf, fa1, fb1);
  mfma_block<MB, NB, BF16>(acc, fa0, fb0);
}

// Tile loads: thread (gr, gg) fetches granule gg of rows gr + 32 i of the
// operand and weight tiles for K tile kt (MASKED: zero past K, K % 8 == 0).
// Row addresses are 32-bit element offsets from the uniform matrix bases.
template <int AG, int BG, bool NOMASK>
__device__ __forceinline__ void tile_load(const uint16_t* a, const uint16_t* w,
                                          const uint32_t (&aoff)[AG], const uint32_t (&boff)[BG],
                                          int64_t kt, int gg, int64_t k, uint4 (&ra)[AG],
                                          uint4 (&rb)[BG]) {
  const bool in = NOMASK || kt * 64 + gg * 8 < k;
  const uint16_t* ak = a + kt * 64;
  const uint16_t* wk = w + kt * 64;
#pragma unroll
  for (int i = 0; i < AG; ++i)
    ra[i] = in ? *reinterpret_cast<const uint4*>(ak + aoff[i]) : make_uint4(0, 0, 0, 0);
#pragma unroll
  for (int i = 0; i < BG; ++i)
    rb[i] = in ? *reinterpret_cast<const uint4*>(wk + boff[i]) : make_uint4(0, 0, 0, 0);
}

template <int AG, int BG, int BM>
__device__ __forceinline__ void tile_store(uint4* buf, int gr, int gg, const uint4 (&ra)[AG],
                                           const uint4 (&rb)[BG]) {
#pragma unroll
  for (int i = 0; i < AG; ++i) buf[swz(gr + 32 * i, gg)] = ra[i];
#pragma unroll
  for (int i = 0; i < BG; ++i) buf[BM * 8 + swz(gr + 32 * i, gg)] = rb[i];
}

// Tile order: workgroups are dispatched round-robin over the 8 XCDs; remap so
// that each XCD walks a contiguous range of tiles, and walk tiles column-major
// inside groups of 8 row-tiles so that concurrently resident workgroups on one
// XCD share operand rows and weight columns in its L2.  n0 is in output columns.
template <int EPI, int BM, int BN>
__device__ __forceinline__ int64_t tile_count(const GemmArgs& g) {
  return cdiv(g.m, BM) * cdiv(g.n, out_cols<EPI, BN>());
}

template <int EPI, int BM, int BN>
__device__ __forceinline__ void tile_origin(const GemmArgs& g, int64_t tile, int64_t& m0, int64_t& n0) {
  constexpr int BNO = out_cols<EPI, BN>();
  const int64_t tiles_m = cdiv(g.m, BM), tiles_n = cdiv(g.n, BNO);
  const int64_t ntiles = tiles_m * tiles_n;
  int64_t bid = tile;
  if (ntiles % 8 == 0) bid = (bid % 8) * (ntiles / 8) + bid / 8;
  constexpr int64_t GROUP_M = 8;
  const int64_t group = bid / (GROUP_M * tiles_n);
  const int64_t first_m = group * GROUP_M;
  const int64_t gsize = min(tiles_m - first_m, GROUP_M);
  const int64_t tm = first_m + (bid % (GROUP_M * tiles_n)) % gsize;
  const int64_t tn = (bid % (GROUP_M * tiles_n)) / gsize;
  m0 = tm * BM;
  n0 = tn * BNO;
}

// ------------------------------------------------------------ GEMM epilogue
// Shared by the GEMM kernels.  acc is either f32x16_t [MB][NB], the 32x32
// layout (lane holds column (lane & 31) and rows 8*(v/4) + 4*(lane/32) + (v%4),
// v = 0..15, of each of the wave's MB x NB 32x32 blocks), or f32x4_t
// [2 MB][2 NB], the 16x16 layout (lane holds column (lane & 15) and rows
// 4*(lane/16) + v, v = 0..3, of each 16x16 block); the wave tile starts at row
// m0 + wm * WM and column n0 + wn * WN (n0 in output columns).  lds: at least NW x 32 x LDR
// floats, free for the wave-private staging slices (the caller's barrier-free
// LDS use must be over).  praw: the rows' raw positions when EARLY (one block
// per wave, requested before the K loop).  SLOT_U4: uint4 offset in lds of the
// fused KV append's slot table (MB x 32 int64 per wave), followed by the row
// scales' table (MB x 32 floats per wave).
template <int EPI, int HD, int MB, int NB, int WM, int WN, int NW, int EDT, bool EARLY, int SLOT_U4, typename ACC>
__device__ __forceinline__ void gemm_epilogue(ACC& acc, uint4* lds, const GemmArgs& g, const QkvEpi& e,
                                              int64_t m0, int64_t n0, int wid, int wm, int wn, int lane,
                                              const int64_t* praw) {
  using DT = EpiDt<EDT>;
  constexpr bool A16 = sizeof(acc[0][0]) == sizeof(f32x4_t);  // 16x16 accumulator blocks
  constexpr int LDR = 136;
  constexpr bool EARLY_POS = EARLY;
  const int frow = lane & 31, fhalf = lane >> 5;
  const int64_t wcol0 = n0 + wn * WN;
  const int64_t wrow0 = m0 + wm * WM;
  if constexpr (EPI == EPI_RAW && A16) {
#pragma unroll
    for (int i = 0; i < 2 * MB; ++i)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int64_t row = wrow0 + i * 16 + 4 * (lane >> 4) + v;
        if (row >= g.m) continue;
#pragma unroll
        for (int j = 0; j < 2 * NB; ++j) {
          const int64_t col = wcol0 + j * 16 + (lane & 15);
          if (col < g.n) g.raw[row * g.n + col] = acc[i][j][v];
        }
      }
    return;
  } else if constexpr (EPI == EPI_RAW) {
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int64_t row = wrow0 + i * 32 + 8 * (v / 4) + 4 * fhalf + (v % 4);
        if (row >= g.m) continue;
#pragma unroll
        for (int j = 0; j < NB; ++j) {
          const int64_t col = wcol0 + j * 32 + frow;
          if (col < g.n) g.raw[row * g.n + col] = acc[i][j][v];
        }
      }
    return;
  } else if constexpr (EPI == EPI_LINEAR || EPI == EPI_SWIGLU) {
    static_assert(WN == 128, "the row epilogue maps 8 lanes x 16 columns onto 128 columns");
    // Each 32-row accumulator block is staged through this wave's LDS slice;
    // then 8 lanes per row each take 8 consecutive output columns (twice for
    // EPI_LINEAR's 128), so residual reads and output writes are 16-byte rows.
    float* et = reinterpret_cast<float*>(lds) + wid * (32 * LDR);
    constexpr int CH = EPI == EPI_SWIGLU ? 1 : 2;  // 8-column chunks per lane
    const int c8 = lane & 7, r8 = lane >> 3;
    const int64_t ocol0 = EPI == EPI_SWIGLU ? n0 + wn * 64 : wcol0;  // first output column of the wave
    __syncthreads();  // the K loop's last LDS reads are done before the slices are reused
#pragma unroll
    for (int i = 0; i < MB; ++i) {
      if constexpr (A16) {
#pragma unroll
        for (int rb = 0; rb < 2; ++rb)
#pragma unroll
          for (int cb = 0; cb < 2 * NB; ++cb)
#pragma unroll
            for (int v = 0; v < 4; ++v)
              et[(rb * 16 + 4 * (lane >> 4) + v) * LDR + cb * 16 + (lane & 15)] = acc[2 * i + rb][cb][v];
      } else {
#pragma unroll
        for (int j = 0; j < NB; ++j)
#pragma unroll
          for (int v = 0; v < 16; ++v)
            et[(8 * (v / 4) + 4 * fhalf + (v % 4)) * LDR + j * 32 + frow] = acc[i][j][v];
      }
      __asm__ volatile("" ::: "memory");  // wave-private slice, LDS keeps a wave's order
      // Kept rolled: unrolled over the 4 row groups the residual / store paths
      // grew the kernel past the instruction cache, and the K loop of the other
      // workgroup on the CU missed in it (o_proj 8192x4096x4096: 1320 vs 232 us).
#pragma unroll 1
      for (int it = 0; it < 4; ++it) {
        const int rl = r8 + 8 * it;
        const int64_t row = wrow0 + i * 32 + rl;
#pragma unroll
        for (int ch = 0; ch < CH; ++ch) {
          const int lc = 64 * ch + 8 * c8;  // column inside the wave tile
          const int64_t col = ocol0 + lc;
          float y[8];
          const float4 a0 = *reinterpret_cast<const float4*>(et + rl * LDR + lc);
          const float4 a1 = *reinterpret_cast<const float4*>(et + rl * LDR + lc + 4);
          const float av[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
          if constexpr (EPI == EPI_SWIGLU) {
            const float4 u0 = *reinterpret_cast<const float4*>(et + rl * LDR + 64 + lc);
            const float4 u1 = *reinterpret_cast<const float4*>(et + rl * LDR + 64 + lc + 4);
            const float uv[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
#pragma unroll
            for (int t = 0; t < 8; ++t) {
              const float gt = rnd<DT::Q>(av[t], e.qkv_dt), ut = rnd<DT::Q>(uv[t], e.qkv_dt);
              y[t] = rnd<DT::O>(rnd<DT::Q>(silu_fast(gt), e.qkv_dt) * ut, e.out_dt);
            }
          } else {
            float bv[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
            if (e.bias) {
#pragma unroll
              for (int t = 0; t < 8; ++t) bv[t] = load_any(e.bias, e.bias_dtype, min(col + t, g.n - 1));
            }
            float rv[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
            if (e.res && row < g.m) {
              if (e.vec && col + 8 <= g.n) {
                if (e.res_dt == BFA_DTYPE_BF16) load8<BFA_DTYPE_BF16>(static_cast<const uint16_t*>(e.res) + row * e.ldr + col, rv);
                else if (e.res_dt == BFA_DTYPE_F16) load8<BFA_DTYPE_F16>(static_cast<const uint16_t*>(e.res) + row * e.ldr + col, rv);
                else load8<BFA_DTYPE_F32>(static_cast<const float*>(e.res) + row * e.ldr + col, rv);
              } else {
#pragma unroll
                for (int t = 0; t < 8; ++t)
                  if (col + t < g.n) rv[t] = load_any(e.res, e.res_dt, row * e.ldr + col + t);
              }
            }
#pragma unroll
            for (int t = 0; t < 8; ++t)
              y[t] = rnd<DT::O>(rnd<DT::M>(rnd<DT::Q>(av[t] + bv[t], e.qkv_dt) + rv[t], e.mid_dt), e.out_dt);
          }
          if (row < g.m) {
            if (e.vec && col + 8 <= g.n) {
              store8_dt<DT::O>(e.out, e.out_dt, row * e.ldo + col, y);
            } else {
#pragma unroll
              for (int t = 0; t < 8; ++t)
                if (col + t < g.n) store_any(e.out, e.out_dt, row * e.ldo + col + t, y[t]);
            }
          }
        }
      }
      __asm__ volatile("" ::: "memory");
    }
  } else {
    static_assert(HD == 32 || HD == 64 || HD == 128, "fused epilogue covers head_dim 32/64/128");
    static_assert(WN == 128 || (WN == 64 && HD <= 64), "a wave tile holds whole heads");
    // Each 32-row accumulator block is staged through this wave's slice of the
    // (now idle) LDS, then processed row by row: WN / 8 lanes per row, each lane
    // owning 4 RoPE pairs (columns j..j+3 and j+D/2..j+D/2+3 of one head), so
    // the q/k norm is a butterfly over the D/8 lanes of a head and every store
    // is a contiguous 4-element vector.
    constexpr int LH = HD / 8;      // lanes per head
    constexpr int LPR = WN / 8;     // lanes per row (16 or 8)
    constexpr int RPP = 64 / LPR;   // rows per pass (4 or 8)
    constexpr int NP = 32 / RPP;    // passes per 32-row block (8 or 4)
    float* et = reinterpret_cast<float*>(lds) + wid * (32 * LDR);
    const int lr = lane % LPR, rg = lane / LPR;
    const int hloc = lr / LH, q = lr % LH;
    const int c1 = hloc * HD + q * 4, c2 = c1 + HD / 2;  // columns inside the wave tile
    const int64_t gc1 = wcol0 + c1, gc2 = wcol0 + c2;
    const bool colok = gc1 < e.n;
    const int64_t head = min(gc1, e.n - 1) / HD;
    const int kd = head_kind(e, head);
    const void* nw = kd == 0 ? e.qn_w : (kd == 1 ? e.kn_w : nullptr);
    const bool any_norm = e.qn_w != nullptr || e.kn_w != nullptr;
    const bool rope = e.cs != nullptr && kd != 2;
    const bool has_bias = e.bias != nullptr;
    float b1[4], b2[4], g1[4], g2[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      b1[t] = (e.bias && colok) ? load_any(e.bias, e.bias_dtype, gc1 + t) : 0.f;
      b2[t] = (e.bias && colok) ? load_any(e.bias, e.bias_dtype, gc2 + t) : 0.f;
      g1[t] = nw ? load_any(nw, e.qk_w_dtype, q * 4 + t) : 1.f;
      g2[t] = nw ? load_any(nw, e.qk_w_dtype, HD / 2 + q * 4 + t) : 1.f;
    }
    const int dt_after = nw ? e.norm_dt : e.qkv_dt;  // dtype RoPE receives
    // fused KV append: this wave's rows' cache slots, in a wave-private LDS
    // table after the staging slices (filled after the barrier below)
    const bool app = e.cache != nullptr && kd != 0;
    const bool out_ok = kd == 0 || !e.skip_kv_out;
    int64_t* const stab = reinterpret_cast<int64_t*>(lds + SLOT_U4) + wid * (MB * 32);
    const int64_t hk = head - e.hq - (kd == 2 ? e.hkv : 0);  // head index within the k or v heads
    const int64_t cbase = (kd == 2 ? e.c_skv : 0) + hk * e.c_sh + q * 4;
    // Positions of every row this lane will rotate, fetched up front (one
    // batch of independent loads) so that each row iteration has a single
    // dependent load level (its cos/sin) instead of two; -1 marks a position
    // outside the table.
    int32_t posv[MB][NP];
    if constexpr (EARLY_POS) {
      if (rope) {
#pragma unroll
        for (int it = 0; it < NP; ++it) posv[0][it] = epi_pos_check(e, praw[it]);
      }
    } else if (rope) {
      if (e.pos_is_i64) {
#pragma unroll
        for (int i = 0; i < MB; ++i)
#pragma unroll
          for (int it = 0; it < NP; ++it)
            posv[i][it] = epi_pos_check(e, static_cast<const int64_t*>(e.positions)[min(wrow0 + i * 32 + rg + RPP * it, g.m - 1)]);
      } else {
#pragma unroll
        for (int i = 0; i < MB; ++i)
#pragma unroll
          for (int it = 0; it < NP; ++it)
            posv[i][it] = epi_pos_check(e, static_cast<const int32_t*>(e.positions)[min(wrow0 + i * 32 + rg + RPP * it, g.m - 1)]);
      }
    }
    __syncthreads();
    if (e.cache != nullptr && !e.app_in_kernel) {
      // rows past m read the last row's slot; their stores are masked
      for (int r = lane; r < MB * 32; r += 64) stab[r] = e.slot_off[min(wrow0 + r, g.m - 1)];
      __asm__ volatile("" ::: "memory");  // the wave's own LDS writes precede its reads below
    }
    // Row scales (the norm weight folded into W): this wave's rows go to a
    // wave-private LDS table after the slot tables, read once per row below
    // (held in registers a block ahead, they had made the epilogue spill).
    const bool rsc = e.row_scale != nullptr;
    float* const rtab = reinterpret_cast<float*>(lds + SLOT_U4 + NW * MB * 32 / 2) + wid * (MB * 32);
    if (rsc) {
      for (int r = lane; r < MB * 32; r += 64) rtab[r] = e.row_scale[min(wrow0 + r, g.m - 1)];
      __asm__ volatile("" ::: "memory");
    }
    // The cos/sin rows of a block's 8 rows are all requested before its row
    // loop: there each load would sit behind the previous row's stores (the
    // table and the output may alias as far as the compiler knows), paying the
    // table's L2 latency 8 times.  Block i+1's rows are requested once block i's
    // accumulators are staged (their registers are free) and before block i's
    // stores: requested after them, their wait would also wait for every store
    // of block i, which all CUs issue at once.
    float4 cvv[2][NP], svv[2][NP];
    auto load_cs = [&](int i, float4 (&cv)[NP], float4 (&sv)[NP]) {
#pragma unroll
      for (int it = 0; it < NP; ++it) {
        const int64_t p = posv[i][it] >= 0 ? posv[i][it] : 0;
        cv[it] = *reinterpret_cast<const float4*>(e.cs + p * HD + q * 4);
        sv[it] = *reinterpret_cast<const float4*>(e.cs + p * HD + HD / 2 + q * 4);
      }
    };
    if (rope) load_cs(0, cvv[0], svv[0]);

#pragma unroll
    for (int i = 0; i < MB; ++i) {
      float4 (&cvv_i)[NP] = cvv[i & 1];
      float4 (&svv_i)[NP] = svv[i & 1];
      if constexpr (A16) {
#pragma unroll
        for (int rb = 0; rb < 2; ++rb)
#pragma unroll
          for (int cb = 0; cb < 2 * NB; ++cb)
#pragma unroll
            for (int v = 0; v < 4; ++v)
              et[(rb * 16 + 4 * (lane >> 4) + v) * LDR + cb * 16 + (lane & 15)] = acc[2 * i + rb][cb][v];
      } else {
#pragma unroll
        for (int j = 0; j < NB; ++j)
#pragma unroll
          for (int v = 0; v < 16; ++v)
            et[(8 * (v / 4) + 4 * fhalf + (v % 4)) * LDR + j * 32 + frow] = acc[i][j][v];
      }
      // The slice is private to this wave and LDS executes one wave's accesses
      // in issue order, so the row reads below see these writes (and the next
      // block's writes follow this block's reads) without a barrier; only the
      // compiler's order must be kept.
      __asm__ volatile("" ::: "memory");
      if (rope && i + 1 < MB) load_cs(i + 1, cvv[(i + 1) & 1], svv[(i + 1) & 1]);
      bool bad = false;
#pragma unroll
      for (int it = 0; it < NP; ++it) {
        const int rl = rg + RPP * it;
        const int64_t row = wrow0 + i * 32 + rl;
        const float4 a1 = *reinterpret_cast<const float4*>(et + rl * LDR + c1);
        const float4 a2 = *reinterpret_cast<const float4*>(et + rl * LDR + c2);
        float x1[4] = {a1.x, a1.y, a1.z, a1.w}, x2[4] = {a2.x, a2.y, a2.z, a2.w};
        if (rsc) {
          const float r = rtab[i * 32 + rl];
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            x1[t] = x1[t] * r;
            x2[t] = x2[t] * r;
          }
        }
        if (has_bias) {
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            x1[t] = x1[t] + b1[t];
            x2[t] = x2[t] + b2[t];
          }
        }
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          x1[t] = rnd<DT::Q>(x1[t], e.qkv_dt);
          x2[t] = rnd<DT::Q>(x2[t], e.qkv_dt);
        }
        if (any_norm) {
          float ss = 0.f;
#pragma unroll
          for (int t = 0; t < 4; ++t) ss += x1[t] * x1[t] + x2[t] * x2[t];
          ss = group_sum_dpp<LH>(ss);  // lanes of one head form an aligned group of a DPP row
          if (nw) {
            const float r = __builtin_amdgcn_rsqf(ss / static_cast<float>(HD) + e.qk_eps);
#pragma unroll
            for (int t = 0; t < 4; ++t) {
              x1[t] = rnd<DT::N>((x1[t] * r) * g1[t], e.norm_dt);
              x2[t] = rnd<DT::N>((x2[t] * r) * g2[t], e.norm_dt);
            }
          }
        }
        if (rope) {
          const bool ok = posv[i][it] >= 0;
          bad = bad || (!ok && row < g.m);
          const float4 cv = cvv_i[it], sv = svv_i[it];
          const float c[4] = {cv.x, cv.y, cv.z, cv.w}, sn[4] = {sv.x, sv.y, sv.z, sv.w};
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const float u = x1[t], w = x2[t];
            x1[t] = ok ? rnd<DT::A>(u * c[t] - w * sn[t], dt_after) : 0.f;
            x2[t] = ok ? rnd<DT::A>(w * c[t] + u * sn[t], dt_after) : 0.f;
          }
        }
        if (row < g.m && colok) {
          if (out_ok) {
            store4_dt<DT::O>(e.out, e.out_dt, row * e.ldo + gc1, x1);
            store4_dt<DT::O>(e.out, e.out_dt, row * e.ldo + gc2, x2);
          }
          if (app) {
            const int64_t so = stab[i * 32 + rl];
            if (so >= 0) {
              float y1[4], y2[4];
#pragma unroll
              for (int t = 0; t < 4; ++t) {
                y1[t] = rnd<DT::O>(x1[t], e.out_dt);
                y2[t] = rnd<DT::O>(x2[t], e.out_dt);
              }
              store4_sel(e.cache, e.cache_dt, so + cbase, y1);
              store4_sel(e.cache, e.cache_dt, so + cbase + HD / 2, y2);
            }
          }
        }
      }
      if (bad && q == 0) flag_status(e.status, BFA_STATUS_INDEX_OOB);
      __asm__ volatile("" ::: "memory");
    }
  }
}

// DIRECT: tiles go HBM -> LDS by DMA (K % 64 == 0, 16-byte aligned rows,
// byte offsets below 4 GiB); otherwise HBM -> registers -> LDS with K masking.
// NW = (BM / WM) (BN / WN) waves per workgroup (4 or 8).  Wave tiles of at most
// 64x128 (128 accumulator registers) are compiled for two waves per SIMD: two
// 4-wave workgroups, or one 8-wave workgroup, per CU.  BK is the depth of a DMA
// stage: 32 (ring of NS stages, 16 rows x 64 bytes per copy) or 64 (two
// buffers, 8 rows x 128 bytes per copy, full cache lines).
template <int BM, int BN, int WM, int WN, bool BF16, int EPI, int HD, bool DIRECT, int NS, int BK,
          int EDT = EDT_RT>
__global__ __launch_bounds__((BM / WM) * (BN / WN) * 64, (WM * WN <= 8192 ? 2 : 1)) void qkv_gemm_kernel(
    GemmArgs g, QkvEpi e) {
  constexpr int NWN = BN / WN;
  constexpr int NW = (BM / WM) * NWN;
  static_assert(NW == 4 || NW == 8, "four or eight waves per workgroup");
  static_assert(DIRECT || NW == 4, "the register-staged path assumes 256 threads");
  static_assert(BK == 32 || BK == 64, "stage depth");
  constexpr int MB = WM / 32, NB = WN / 32;
  constexpr int AG = BM / 32, BG = BN / 32;  // 16-byte granules per thread per K tile
  // LDS: the DMA path keeps a ring of NS 32-deep stages of both operands; the
  // register path two 64-deep buffers; afterwards the fused epilogue stages
  // each wave's 32-row accumulator blocks (row stride LDR floats).
  constexpr int LDR = 136;
  constexpr int STAGE_U4 = (BM + BN) * BK / 8;
  constexpr int EPI_U4 = NW * 32 * LDR / 4;
  constexpr int MAIN_U4 = DIRECT ? (BK == 32 ? NS : 2) * STAGE_U4 : 2 * (BM + BN) * 8;
  // the fused KV append's per-wave slot table (MB x 32 int64) lies past both the
  // K loop's buffers and the epilogue's staging slices: it is filled before the
  // K loop and read in the epilogue
  constexpr int SLOT_U4 = MAIN_U4 > EPI_U4 ? MAIN_U4 : EPI_U4;
  // and after it the fused epilogue's row-scale table (MB x 32 floats per wave)
  constexpr int LDS_U4 = SLOT_U4 + (EPI == EPI_FUSED ? NW * MB * 32 / 2 + NW * MB * 32 / 4 : 0);
  __shared__ uint4 lds[LDS_U4];
  uint4* const lds0 = lds;
  uint4* const lds1 = lds + (BM + BN) * 8;

  // PERSIST (the 256x256 tile): a grid smaller than the tile count loops:
  // workgroup b takes tiles b, b + gridDim.x, ... (the same XCD each time,
  // since tile t and workgroup b agree modulo 8).  The barrier keeps the next
  // tile's first copies out of the LDS that the previous tile's epilogue may
  // still be reading.  The other tiles run one per workgroup.
  constexpr bool PERSIST = BM == 256 && BN == 256;
  const int64_t ntiles = tile_count<EPI, BM, BN>(g);
  for (int64_t tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
  if (tile != blockIdx.x) __syncthreads();
  // The thread id passes through an empty asm on every tile, so the values
  // derived from it (LDS and DMA offsets, the epilogue's lane roles) are
  // computed per tile, as in a one-tile workgroup, instead of once before the
  // loop, where they would all stay live across the K loop and the epilogue
  // and spill.
  int tid = threadIdx.x;
  if constexpr (PERSIST) asm volatile("" : "+v"(tid));
  const int lane = tid & 63;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
  const int wm = wid / NWN, wn = wid % NWN;
  int64_t m0, n0;
  tile_origin<EPI, BM, BN>(g, tile, m0, n0);
  const int64_t KT = cdiv(g.k, 64);
  const int frow = lane & 31, fhalf = lane >> 5;

  // Fused KV append: the cache slots of this wave's rows go to its slot table.
  // Called right after the K loop's first loads are issued, so that the
  // page-table lookups wait together with those loads, not ahead of them.
  auto resolve_slots = [&]() {
    if constexpr (EPI == EPI_FUSED) {
      if (e.cache != nullptr && e.app_in_kernel) {
        int64_t* stab = reinterpret_cast<int64_t*>(lds + SLOT_U4) + wid * (MB * 32);
        for (int r = lane; r < MB * 32; r += 64) {
          int64_t page = 0, slot = 0;
          const int bad = append_target_code(e.app, min(m0 + wm * WM + r, g.m - 1), page, slot);
          if (bad) flag_status(e.app.status, bad);
          stab[r] = bad ? -1 : page * e.app.c_sp + slot * e.app.c_ss;
        }
      }
    }
  };

  // Positions of the rows this lane rotates in the fused epilogue (rows
  // lane / 16 + 4 it of each 32-row block).  With one block per wave they are
  // requested here, before the K loop (16 registers), so that the epilogue's
  // cos/sin loads do not wait a memory round trip for them.
  constexpr bool EARLY_POS = EPI == EPI_FUSED && MB == 1;
  constexpr int ERPP = 64 / (WN / 8), ENP = 32 / ERPP;  // the epilogue's rows per pass and passes
  int64_t praw[EARLY_POS ? ENP : 1];
  if constexpr (EARLY_POS) {
    const int64_t r0 = m0 + wm * WM + lane / (WN / 8);
    if (e.cs != nullptr) {
      if (e.pos_is_i64) {
#pragma unroll
        for (int it = 0; it < ENP; ++it) praw[it] = static_cast<const int64_t*>(e.positions)[min(r0 + ERPP * it, g.m - 1)];
      } else {
#pragma unroll
        for (int it = 0; it < ENP; ++it) praw[it] = static_cast<const int32_t*>(e.positions)[min(r0 + ERPP * it, g.m - 1)];
      }
    }
  }

  // The 64-deep DMA path multiplies with v_mfma_f32_16x16x32 into 16x16 blocks
  // (acc4); the 32-deep rings and the register-staged path with
  // v_mfma_f32_32x32x16 into 32x32 blocks (acc).  Same product and the same
  // fragment bytes per wave tile, but a 16x16x32 MFMA reads and writes a quarter
  // of the accumulators for half the work, and the chip is power limited under
  // this loop: at 8192 tokens the Llama-3-8B projection took 313-325 against
  // 323-334 us and the fused op 329-334 against 344-347 us, same box,
  // interleaved processes; with the pinned loop below, gate_up+SiLU*mul
  // 1560-1568 against 1605-1613 us, down_proj+residual 777-778 against 810-812
  // us and o_proj+residual 230-232 against 233 us (the 32x32x16 loop pinned).
  constexpr bool M16 = DIRECT && BK == 64;
  f32x16_t acc[M16 ? 1 : MB][M16 ? 1 : NB];
  f32x4_t acc4[M16 ? 2 * MB : 1][M16 ? 2 * NB : 1];
  if constexpr (M16) {
#pragma unroll
    for (int i = 0; i < 2 * MB; ++i)
#pragma unroll
      for (int j = 0; j < 2 * NB; ++j) acc4[i][j] = f32x4_t{};
  } else {
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
      for (int j = 0; j < NB; ++j) acc[i][j] = f32x16_t{};
  }

  // global -> register -> LDS (any K that is a multiple of 8).  The next
  // tile's loads are issued before this tile's MFMAs and stored to the other
  // LDS buffer after them; MFMA fragments are double-buffered across the four
  // 16-deep K sub-steps so every ds_read overlaps the previous sub-step's MFMAs.
  if constexpr (DIRECT && BK == 32) {
    // Ring of NS 32-deep stages.  Per step: the second sub-step's fragments are
    // read while the first sub-step's MFMAs run; then the wave waits for stage
    // kt+1's DMAs (vmcnt counts only this wave's copies, issued in order, so
    // `later` stages may stay in flight), and a barrier makes every wave's copies
    // visible and proves every wave has finished reading stage kt, whose buffer
    // is refilled with stage kt+NS at once; stage kt+1's first fragments are then
    // read under the second sub-step's MFMAs.
    constexpr int ADPW = BM / 16 / NW, BDPW = BN / 16 / NW;  // 1 KiB blocks per wave per stage
    constexpr int DPW = ADPW + BDPW;
    // lane l lands at slot l % 4 of row 16 b + l / 4 and fetches logical granule
    // (l % 4) ^ ((l / 4 / 4) % 4), which realises sw32().
    const int lrow = lane >> 2, lgran = (lane & 3) ^ ((lane >> 4) & 3);
    uint32_t aoff[ADPW], boff[BDPW];
#pragma unroll
    for (int i = 0; i < ADPW; ++i)
      aoff[i] = static_cast<uint32_t>((min(m0 + (i * NW + wid) * 16 + lrow, g.m - 1) * g.lda + lgran * 8) * 2);
#pragma unroll
    for (int i = 0; i < BDPW; ++i)
      boff[i] = static_cast<uint32_t>((weight_row<EPI>(g, n0, (i * NW + wid) * 16 + lrow) * g.ldw + lgran * 8) * 2);
    const uint32_t lbase = lds_addr(lds) + wid * 1024;
    constexpr uint32_t SB = STAGE_U4 * 16;  // stage bytes
    const int64_t nst = g.k / 32;  // 32-deep stages
#pragma unroll
    for (int st = 0; st < NS; ++st)
      if (st < nst) issue_stage<ADPW, BDPW, BM, 32, NW>(g.a, g.w, st, aoff, boff, lbase + st * SB);
    resolve_slots();
    wait_stages<DPW, NS>(min<int64_t>(NS - 1, nst - 1));
    __syncthreads();
    uint4 fa0[MB], fb0[NB], fa1[MB], fb1[NB];
    load_frags32<MB, NB, BM, WM, WN>(lds, 0, wm, wn, frow, fhalf, fa0, fb0);
    // The last stage is peeled off so that the loop body has no path that skips
    // the barrier: the second sub-step's MFMAs then never wait on the next
    // stage's fragment reads.
    int64_t kt = 0;
    for (; kt + 1 < nst; ++kt) {
      const int slot = static_cast<int>(kt % NS);
      load_frags32<MB, NB, BM, WM, WN>(lds + slot * STAGE_U4, 1, wm, wn, frow, fhalf, fa1, fb1);
      mfma_block<MB, NB, BF16>(acc, fa0, fb0);
      wait_stages<DPW, NS>(min<int64_t>(NS - 2, nst - 2 - kt));
      __syncthreads();
      if (kt + NS < nst) issue_stage<ADPW, BDPW, BM, 32, NW>(g.a, g.w, kt + NS, aoff, boff, lbase + slot * SB);
      load_frags32<MB, NB, BM, WM, WN>(lds + static_cast<int>((kt + 1) % NS) * STAGE_U4, 0, wm, wn,
                                       frow, fhalf, fa0, fb0);
      mfma_block<MB, NB, BF16>(acc, fa1, fb1);
    }
    load_frags32<MB, NB, BM, WM, WN>(lds + static_cast<int>(kt % NS) * STAGE_U4, 1, wm, wn, frow,
                                     fhalf, fa1, fb1);
    mfma_block<MB, NB, BF16>(acc, fa0, fb0);
    mfma_block<MB, NB, BF16>(acc, fa1, fb1);
  } else if constexpr (DIRECT) {
    // Two 64-deep buffers; each copy is 8 rows x 128 bytes.  Lane l lands at
    // slot l % 8 of tile row 8 b + l / 8 and fetches logical granule
    // (l % 8) ^ ((8 b + l / 8) / 2 % 8) = (l % 8) ^ ((4 (wid % 2) + l / 16) % 8)
    // (b = NW i + wid, NW even), which realises swz().  Stage kt+1 is issued as
    // stage kt's MFMAs start and waited for as they end.
    constexpr int ADPW = BM / 8 / NW, BDPW = BN / 8 / NW;
    const int lrow = lane >> 3, lgran = (lane & 7) ^ ((4 * (wid & 1) + (lane >> 4)) & 7);
    uint32_t aoff[ADPW], boff[BDPW];
#pragma unroll
    for (int i = 0; i < ADPW; ++i)
      aoff[i] = static_cast<uint32_t>((min(m0 + (i * NW + wid) * 8 + lrow, g.m - 1) * g.lda + lgran * 8) * 2);
#pragma unroll
    for (int i = 0; i < BDPW; ++i)
      boff[i] = static_cast<uint32_t>((weight_row<EPI>(g, n0, (i * NW + wid) * 8 + lrow) * g.ldw + lgran * 8) * 2);
    const uint32_t l0 = lds_addr(lds0) + wid * 1024, l1 = lds_addr(lds1) + wid * 1024;
    // A stage is two 32-deep sub-steps, each in two halves of the wave's 16-column
    // blocks: four quarters of M2 x NH MFMAs, each quarter's fragment reads issued
    // under the previous quarter's MFMAs.  Two operand and two half-weight
    // fragment sets (64 VGPRs; double-buffering whole sub-steps took 96 and
    // spilled inside the loop).  pin_acc keeps every MFMA of a stage above the
    // stage's barrier: left alone, the compiler sank about half of them below it,
    // ahead of the next stage's DMAs, which then went out a quarter of a stage
    // late (8192 tokens, same box: the layer chain 514-515 against 496 us, and
    // 543-544 against 513-515 us with the QKV weight rotating over four copies).
    constexpr int M2 = M16 ? 2 * MB : 1, N2 = M16 ? 2 * NB : 1, NH = M16 ? NB : 1;
    uint4 fa0[M2], fa1[M2], fbA[NH], fbB[NH];
    auto stage = [&](const uint4* cur) {
      load_b16<NH, BM, WN>(cur, 0, 1, wn, lane, fbB);
      mfma_half16<M2, N2, NH, BF16>(acc4, fa0, fbA, 0);
      load_a16<M2, BM, WM>(cur, 1, wm, lane, fa1);
      load_b16<NH, BM, WN>(cur, 1, 0, wn, lane, fbA);
      mfma_half16<M2, N2, NH, BF16>(acc4, fa0, fbB, 1);
      load_b16<NH, BM, WN>(cur, 1, 1, wn, lane, fbB);
      mfma_half16<M2, N2, NH, BF16>(acc4, fa1, fbA, 0);
      mfma_half16<M2, N2, NH, BF16>(acc4, fa1, fbB, 1);
    };
    issue_stage<ADPW, BDPW, BM, 64, NW>(g.a, g.w, 0, aoff, boff, l0);
    resolve_slots();
    wait_vmem();
    __syncthreads();
    load_a16<M2, BM, WM>(lds0, 0, wm, lane, fa0);  // the first quarter's fragments
    load_b16<NH, BM, WN>(lds0, 0, 0, wn, lane, fbA);
    int64_t kt = 0;
    for (; kt + 2 <= KT; kt += 2) {
      issue_stage<ADPW, BDPW, BM, 64, NW>(g.a, g.w, kt + 1, aoff, boff, l1);
      stage(lds0);
      pin_acc(acc4);
      wait_vmem();
      __syncthreads();
      load_a16<M2, BM, WM>(lds1, 0, wm, lane, fa0);
      load_b16<NH, BM, WN>(lds1, 0, 0, wn, lane, fbA);
      if (kt + 2 < KT) issue_stage<ADPW, BDPW, BM, 64, NW>(g.a, g.w, kt + 2, aoff, boff, l0);
      stage(lds1);
      pin_acc(acc4);
      wait_vmem();
      __syncthreads();
      if (kt + 2 < KT) {
        load_a16<M2, BM, WM>(lds0, 0, wm, lane, fa0);
        load_b16<NH, BM, WN>(lds0, 0, 0, wn, lane, fbA);
      }
    }
    if (kt < KT) {  // odd tile count: the last tile is in lds0
      stage(lds0);
      __syncthreads();
    }
  } else {
    const int gg = tid & 7, gr = tid >> 3;
    uint32_t aoff[AG], boff[BG];
  #pragma unroll
    for (int i = 0; i < AG; ++i)
      aoff[i] = static_cast<uint32_t>(min(m0 + gr + 32 * i, g.m - 1) * g.lda + gg * 8);
  #pragma unroll
    for (int i = 0; i < BG; ++i)
      boff[i] = static_cast<uint32_t>(weight_row<EPI>(g, n0, gr + 32 * i) * g.ldw + gg * 8);
    uint4 ra[AG], rb[BG];
    // Two register sets keep the loads of tiles kt+1 and kt+2 in flight while
    // tile kt is multiplied (the K loop is unrolled by two so the sets are
    // static): misses that go to the Infinity Cache get ~2 tiles of MFMA time.
    uint4 ra2[AG], rb2[BG];
    uint4 fa0[MB], fb0[NB], fa1[MB], fb1[NB];
    tile_load<AG, BG, false>(g.a, g.w, aoff, boff, 0, gg, g.k, ra, rb);
    resolve_slots();
    tile_store<AG, BG, BM>(lds0, gr, gg, ra, rb);
    if (KT > 1) tile_load<AG, BG, false>(g.a, g.w, aoff, boff, 1, gg, g.k, ra, rb);
    if (KT > 2) tile_load<AG, BG, false>(g.a, g.w, aoff, boff, 2, gg, g.k, ra2, rb2);
    __syncthreads();
    load_frags<MB, NB, BM, WM, WN>(lds0, 0, wm, wn, frow, fhalf, fa0, fb0);
    int64_t kt = 0;
    for (; kt + 2 <= KT; kt += 2) {
      // tile kt from lds0; set 1 holds tile kt+1, set 2 holds tile kt+2
      compute3<MB, NB, BM, WM, WN, BF16>(lds0, wm, wn, frow, fhalf, acc, fa0, fb0, fa1, fb1);
      tile_store<AG, BG, BM>(lds1, gr, gg, ra, rb);
      mfma_block<MB, NB, BF16>(acc, fa1, fb1);
      __syncthreads();
      if (kt + 3 < KT) tile_load<AG, BG, false>(g.a, g.w, aoff, boff, kt + 3, gg, g.k, ra, rb);
      load_frags<MB, NB, BM, WM, WN>(lds1, 0, wm, wn, frow, fhalf, fa0, fb0);
      // tile kt+1 from lds1; set 2 holds tile kt+2, set 1 holds tile kt+3
      compute3<MB, NB, BM, WM, WN, BF16>(lds1, wm, wn, frow, fhalf, acc, fa0, fb0, fa1, fb1);
      if (kt + 2 < KT) tile_store<AG, BG, BM>(lds0, gr, gg, ra2, rb2);
      mfma_block<MB, NB, BF16>(acc, fa1, fb1);
      __syncthreads();
      if (kt + 4 < KT) tile_load<AG, BG, false>(g.a, g.w, aoff, boff, kt + 4, gg, g.k, ra2, rb2);
      if (kt + 2 < KT) load_frags<MB, NB, BM, WM, WN>(lds0, 0, wm, wn, frow, fhalf, fa0, fb0);
    }
    if (kt < KT) {  // odd tile count: the last tile is in lds0
      compute3<MB, NB, BM, WM, WN, BF16>(lds0, wm, wn, frow, fhalf, acc, fa0, fb0, fa1, fb1);
      mfma_block<MB, NB, BF16>(acc, fa1, fb1);
      __syncthreads();
    }
  }

  // (likewise into the epilogue, so that its lane roles are not computed
  // before the K loop)
  int lane_e = lane, wid_e = wid;
  if constexpr (PERSIST) asm volatile("" : "+v"(lane_e), "+s"(wid_e));
  if constexpr (M16)
    gemm_epilogue<EPI, HD, MB, NB, WM, WN, NW, EDT, EARLY_POS, SLOT_U4>(acc4, lds, g, e, m0, n0, wid_e,
                                                                      wid_e / NWN, wid_e % NWN, lane_e, praw);
  else
    gemm_epilogue<EPI, HD, MB, NB, WM, WN, NW, EDT, EARLY_POS, SLOT_U4>(acc, lds, g, e, m0, n0, wid_e,
                                                                      wid_e / NWN, wid_e % NWN, lane_e, praw);
  if constexpr (!PERSIST) break;  // one tile per workgroup: no loop, nothing hoisted out of one
  }
}

// ======================================================== decode split-K
// Grid: (n / BNT column tiles, S K-splits).  A workgroup's 4 waves each own
// BNT/4 columns (16 per MFMA block) and all MT*16 rows.  Within a 64-deep K
// step, lane group q = lane/16 owns k in [16q, 16q+16): 32 contiguous bytes of
// one weight row, fed to two 16x16x32 MFMAs (the same k assignment is used
// for the operand, so the sum covers every k once).
struct SplitArgs {
  const uint16_t* a;
  const uint16_t* w;
  int64_t m, n, k, lda, ldw;
  int64_t kchunk;  // K elements per split (multiple of 64)
  float* part;     // [S, m, n]
};

template <int MT, int CPW, bool BF16>
__global__ __launch_bounds__(256) void qkv_splitk_kernel(SplitArgs s) {
  // CPW = 16-column MFMA blocks per wave
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int64_t n0 = (static_cast<int64_t>(blockIdx.x) * 4 + wid) * (16 * CPW);
  const int64_t k0 = static_cast<int64_t>(blockIdx.y) * s.kchunk;
  const int64_t k1 = min(k0 + s.kchunk, s.k);
  const int lr = lane & 15, lq = lane >> 4;

  f32x4_t acc[MT][CPW];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int j = 0; j < CPW; ++j) acc[i][j] = f32x4_t{};

  const uint16_t* wrow[CPW];
#pragma unroll
  for (int j = 0; j < CPW; ++j) wrow[j] = s.w + min(n0 + j * 16 + lr, s.n - 1) * s.ldw;
  const uint16_t* arow[MT];
#pragma unroll
  for (int i = 0; i < MT; ++i) arow[i] = s.a + min(static_cast<int64_t>(i * 16 + lr), s.m - 1) * s.lda;

  for (int64_t kk = k0; kk < k1; kk += 64) {
    const int64_t kl = kk + lq * 16;  // this lane's 16 k values
    const bool in = kl < s.k;         // K % 16 == 0
    uint4 b0[CPW], b1[CPW], a0[MT], a1[MT];
#pragma unroll
    for (int j = 0; j < CPW; ++j) {
      const uint4* p = reinterpret_cast<const uint4*>(wrow[j] + kl);
      b0[j] = in ? p[0] : make_uint4(0, 0, 0, 0);
      b1[j] = in ? p[1] : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < MT; ++i) {
      const uint4* p = reinterpret_cast<const uint4*>(arow[i] + kl);
      a0[i] = in ? p[0] : make_uint4(0, 0, 0, 0);
      a1[i] = in ? p[1] : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int j = 0; j < CPW; ++j) {
        acc[i][j] = mfma16<BF16>(a0[i], b0[j], acc[i][j]);
        acc[i][j] = mfma16<BF16>(a1[i], b1[j], acc[i][j]);
      }
  }
  // 16x16 accumulator layout: lane holds column (lane & 15), rows 4*(lane/16) + v.
  float* dst = s.part + static_cast<int64_t>(blockIdx.y) * s.m * s.n;
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int64_t row = i * 16 + lq * 4 + v;
      if (row >= s.m) continue;
#pragma unroll
      for (int j = 0; j < CPW; ++j) {
        const int64_t col = n0 + j * 16 + lr;
        if (col < s.n) dst[row * s.n + col] = acc[i][j][v];
      }
    }
}

// ============================================================= decode
// T <= 64 tokens.  Pure weight streaming: a workgroup (4 waves) owns 32*4 = 128
// output columns and a K slice of KC_MAX or fewer, and issues its whole slice
// at once.  The operand rows go by DMA into LDS (16-byte granules XOR-swizzled
// by row so the 16-row MFMA fragment reads are conflict-free).  The weight rows
// go to registers laid out 8 lanes per row, so each load instruction covers 8
// full 128-byte lines (the MFMA fragment layout, 16 rows x 64 bytes per
// instruction, streams about 1.2x slower at this shape); each 64-deep K segment is
// then turned into B fragments through a 4 KiB wave-private LDS area and fed to
// 16x16x32 MFMAs.  The split writes an fp32 partial tile.  (Nontemporal weight
// loads stream faster back to back but slow the kernel by a third once the
// reduction kernel has read the partial tiles in between, so they are not used.)
struct DecodeArgs {
  const uint16_t* a;  // operand [m, k] (row stride lda); with the fold, the raw rows x
  const uint16_t* w;  // weight [n, k]
  int64_t m, n, k, lda, ldw;
  float* part;        // [splits, m, n]
  // operand fold (NORM): x / rms(x) * gamma rounded to the weight dtype, as the
  // operand pre-pass computes it (mixed: x / rms rounded to bf16 before gamma)
  const void* gamma;
  int gamma_dt, mixed;
  float eps;
  int fold_rows;  // rows per wave of the fold: 0 (no fold), 1, 2 or 4
  float* stats;   // scale-after form: [splits, 16 mt] partial sums of x^2
};

// Host-side description of the fold: the raw rows and the RMSNorm parameters.
struct OperandFold {
  const void* gamma;
  int gamma_dt;
  bool mixed;
  float eps;
  int rows_per_wave;
  float* stats;  // non-null: scale-after form of the deep-K kernel
};


constexpr int KC_MAX = 512;  // deepest K slice per split (8 segments of 64)



// staging slot of (row r, granule g) in a 32-row x 8-granule block: rows r and
// r+8 share bank groups, so the granule is XORed with r/2 -- conflict-free for
// the 8-lanes-per-row writes and for the 16-rows-per-granule fragment reads.
__device__ __forceinline__ int wslot(int r, int g) { return r * 8 + (g ^ ((r >> 1) & 7)); }

// KS: 64-deep K segments per split (every split has exactly KS; the host picks
// KS dividing k / 64), fixed at compile time so the weight loads carry no
// branches and each segment waits only for its own four loads.
//
// NR > 0 (x in the weight dtype): the operand pre-pass is folded in.  Wave w
// reads the whole of rows w, w + 4, .. (NR of them: 16-byte chunks, eight per
// lane for one row up to hidden 4096, four per lane for two or four rows up to
// 2048) for their sums of squares and the rows' K slices with the matching
// gamma, all before the weight loads are issued, then writes the normalised
// slices where the DMA would have put them.  The row sums run on DPP and the
// lane swaps (no LDS round trips).
template <int MT, int KS, bool BF16, bool REG_ORDER, int NR = 0>
__global__ __launch_bounds__(256) void qkv_decode_kernel(DecodeArgs d) {
  static_assert(KS >= 1 && KS * 64 <= KC_MAX, "segments per split");
  constexpr bool NORM = NR > 0;
  constexpr int CPL = NR == 1 ? 8 : 4;  // 16-byte chunks per lane per row of the fold
  static_assert(NR == 0 || NR == 1 || NR == 2 || NR == 4, "fold rows per wave");
  static_assert(!NORM || (MT == 1 && !REG_ORDER), "the fold covers up to 16 tokens");
  constexpr int GPR = KC_MAX / 8;      // 16-byte granules per LDS operand row (row pitch 1 KiB)
  __shared__ uint4 abuf[64 * GPR];     // 64 rows x KC_MAX bf16 = 64 KiB
  __shared__ uint4 wst[4][32 * 8];     // per wave: 32 weight rows x 64 bf16 = 4 KiB

  const int tid = threadIdx.x, lane = tid & 63;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * 128 + wid * 32;
  const int64_t k0 = static_cast<int64_t>(blockIdx.y) * (KS * 64);
  const int lr = lane & 15, lq = lane >> 4;
  constexpr int gpr = KS * 8;  // granules per operand row actually used

  constexpr int DT = BF16 ? BFA_DTYPE_BF16 : BFA_DTYPE_F16;
  uint4 sx[NORM ? NR : 1][CPL], xs[NORM ? NR : 1];
  float gv[8];
  if constexpr (NORM) {
    const int nch = static_cast<int>(d.k / 8);
    const int64_t kk = k0 + min(lane, gpr - 1) * 8;
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      const uint16_t* xr = d.a + min<int64_t>(wid + 4 * r, d.m - 1) * d.lda;
#pragma unroll
      for (int j = 0; j < CPL; ++j) sx[r][j] = load16(xr + min(lane + 64 * j, nch - 1) * 8);
      xs[r] = load16(xr + kk);
    }
    if (d.gamma_dt == BFA_DTYPE_BF16) load8<BFA_DTYPE_BF16>(static_cast<const uint16_t*>(d.gamma) + kk, gv);
    else if (d.gamma_dt == BFA_DTYPE_F16) load8<BFA_DTYPE_F16>(static_cast<const uint16_t*>(d.gamma) + kk, gv);
    else load8<BFA_DTYPE_F32>(static_cast<const float*>(d.gamma) + kk, gv);
  } else {
    // 1. operand slice -> LDS, one 1 KiB DMA per row (KC_MAX = 512 bf16): lane i
    //    fills physical granule slot i of row r, which holds logical granule
    //    G = (i & ~15) | ((i & 15) ^ (r & 15)); lanes with G past the slice are
    //    masked off.
    static_assert(GPR == 64, "one wave-wide DMA per operand row");
    const uint32_t lbase = lds_addr(abuf);
    const uint16_t* abase = d.a + k0;
    for (int row = wid; row < d.m; row += 4) {
      const int g = (lane & ~15) | ((lane & 15) ^ (row & 15));
      if (g < gpr) {
        dma16(abase, static_cast<uint32_t>((static_cast<int64_t>(row) * d.lda + g * 8) * 2),
              lbase + row * 1024);
      }
    }
  }
  // 2. weight slice -> registers: lane holds row 8i + lane/8, granule lane%8 of
  //    every 64-deep segment (rows past n re-read row n-1; those columns are
  //    never stored)
  uint4 wr[KS][4];
  const int wrow_l = lane >> 3, wg_l = lane & 7;
  {
    const uint16_t* wrow[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) wrow[i] = d.w + min(n0 + i * 8 + wrow_l, d.n - 1) * d.ldw + k0 + wg_l * 8;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
      for (int i = 0; i < 4; ++i) wr[ks][i] = load16(wrow[i] + ks * 64);
  }
  if constexpr (NORM) {
    // the fold's loads went out before the weights: using them waits for them only
    const int nch = static_cast<int>(d.k / 8);
    float ss[NR];
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      ss[r] = 0.f;
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
        float v[8];
        unpack8<DT>(sx[r][j], v);
        if (lane + 64 * j < nch) {
#pragma unroll
          for (int t = 0; t < 8; ++t) ss[r] += v[t] * v[t];
        }
      }
    }
#pragma unroll
    for (int r = 0; r < NR; ++r) ss[r] = wave_sum_dpp(ss[r]);
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      const float inv = 1.0f / sqrtf(ss[r] / static_cast<float>(d.k) + d.eps);
      float v[8], o[8];
      unpack8<DT>(xs[r], v);
#pragma unroll
      for (int t = 0; t < 8; ++t) o[t] = d.mixed ? round_bf16(v[t] * inv) * gv[t] : (v[t] * inv) * gv[t];
      uint32_t pw[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        pw[i] = static_cast<uint32_t>(Elem<DT>::from_f32(o[2 * i])) |
                (static_cast<uint32_t>(Elem<DT>::from_f32(o[2 * i + 1])) << 16);
      const int row = wid + 4 * r;
      if (row < d.m && lane < gpr)
        abuf[row * GPR + ((lane & ~15) | ((lane & 15) ^ (row & 15)))] = make_uint4(pw[0], pw[1], pw[2], pw[3]);
    }
  } else {
    // the operand DMAs were issued before the 4 * KS weight loads and loads
    // complete in order: vmcnt(4 KS) means the DMAs have landed
    // (gfx9 s_waitcnt encoding: vmcnt[3:0], expcnt[6:4], lgkmcnt[11:8], vmcnt[5:4] in [15:14])
    constexpr int kVm = 4 * KS;
    __builtin_amdgcn_s_waitcnt((kVm & 15) | (7 << 4) | (15 << 8) | ((kVm >> 4) << 14));
  }
  __syncthreads();

  // 3. per segment: registers -> staging -> B fragments, then MFMAs.  The
  //    staging area is private to the wave and LDS executes a wave's accesses
  //    in order, so only compiler ordering is needed between the phases.
  f32x4_t acc[MT][2];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x4_t{};
  uint4* ws = wst[wid];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    {
#pragma unroll
      for (int i = 0; i < 4; ++i) ws[wslot(i * 8 + wrow_l, wg_l)] = wr[ks][i];
      asm volatile("" ::: "memory");
      uint4 wf[2][2], af[MT][2];
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int h = 0; h < 2; ++h) wf[j][h] = ws[wslot(j * 16 + lr, h * 4 + lq)];
#pragma unroll
      for (int i = 0; i < MT; ++i) {
        const int row = i * 16 + lr;
        const int g0 = ks * 8 + lq, g1 = g0 + 4;  // this lane's two logical granules
        af[i][0] = abuf[row * GPR + ((g0 & ~15) | ((g0 & 15) ^ (row & 15)))];
        af[i][1] = abuf[row * GPR + ((g1 & ~15) | ((g1 & 15) ^ (row & 15)))];
      }
      asm volatile("" ::: "memory");
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          acc[i][j] = mfma16<BF16>(af[i][0], wf[j][0], acc[i][j]);
          acc[i][j] = mfma16<BF16>(af[i][1], wf[j][1], acc[i][j]);
        }
    }
  }
  // 4. partial tile in register order: the wave's MT x 2 blocks of 64 lanes x
  //    float4 (16x16 MFMA layout: lane holds column lane % 16 and rows
  //    4 (lane / 16) .. +3 of its block) are contiguous, so every store writes
  //    1 KiB of consecutive bytes.  Rows >= m and columns >= n hold garbage that
  //    the reduction never reads.  Layout per split: [column tile][wave][MT][2][64]
  //    float4 (see qkv_decode_epilogue_kernel).
  //    For a single 16-token block (REG_ORDER false) the split is written row
  //    major [m, n] instead, for the one-wave-per-(token, head) reduction, which
  //    has the shorter latency chain when there are this few tokens.
  if constexpr (REG_ORDER) {
    float4* tb = reinterpret_cast<float4*>(d.part) +
                 ((static_cast<int64_t>(blockIdx.y) * gridDim.x + blockIdx.x) * 4 + wid) * (MT * 2 * 64);
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
        tb[(i * 2 + j) * 64 + lane] = make_float4(acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]);
  } else {
    float* dst = d.part + static_cast<int64_t>(blockIdx.y) * d.m * d.n;
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int64_t row = i * 16 + lq * 4 + v;
        if (row >= d.m) continue;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int64_t col = n0 + j * 16 + lr;
          if (col < d.n) dst[row * d.n + col] = acc[i][j][v];
        }
      }
  }
}

// Deep-K form of qkv_decode_kernel for 2..4 token blocks.  With 64 tokens each
// split's fp32 partial tile (m x n x 4 bytes, written and read back) costs half
// as much as the split's 512-deep weight slice, so here a split walks `nch`
// consecutive 256-deep chunks and writes one partial tile for all of them.  The
// operand chunk is double-buffered in LDS (rows of 512 bytes, same granule
// swizzle; one DMA fills two rows, and rows past m re-read row m-1) and the
// next chunk's DMAs go out as the current chunk starts.  The weight registers
// roll: as soon as segment s of chunk c has been staged, segment s of chunk c+1
// is requested into the same registers, so one chunk of weights is always in
// flight.  Requests, in issue order: op(c+1) [D], W(c+1) s0..s3 [4 each]
// interleaved with chunk c's segments; hence before segment s of chunk c the
// wave waits for vmcnt(4 (KS - 1) + D) while a next chunk exists, and for
// vmcnt(4 (KS - 1 - s)) in the last chunk.
constexpr int LOOP_KS = 4;  // 64-deep segments per chunk (256 of K)

// wait_vm for the last chunk's segments; n is a constant once the segment loop
// is unrolled, so the switch folds to the one wait.
__device__ __forceinline__ void wait_vm_last(int n) {
  static_assert(LOOP_KS == 4, "cases below");
  switch (n) {
    case 12: wait_vm<12>(); break;
    case 8: wait_vm<8>(); break;
    case 4: wait_vm<4>(); break;
    default: wait_vm<0>(); break;
  }
}

//
// SA (scale-after, bf16 weights): the operand is x * gamma rounded to bf16
// instead of the normalised row, and the split also returns its rows' sums of
// x^2 over its K slice; the reduction kernel multiplies the summed projection
// by r = 1 / sqrt(sum / hidden + eps).  For the fp32 variants (whose operand
// is (x / rms) * gamma in fp32) this is the same product with the row scale
// taken out of the sum, and it needs no pass over whole rows before the
// projection.  Each wave converts, in place, the operand granules its own
// DMAs wrote (after waiting for them and before the barrier that publishes
// the chunk), with gamma loaded right after the DMAs: requests, in issue
// order, op(c+1) [D], gamma(c+1) [D], W(c+1) s0..s3.
template <int MT, bool BF16, bool SA = false>
__global__ __launch_bounds__(256) void qkv_decode_loop_kernel(DecodeArgs d, int nch) {
  constexpr int KS = LOOP_KS;
  constexpr int GPR = KS * 8;  // granules per operand row (512 bytes)
  constexpr int ROWS = MT * 16;
  constexpr int D = ROWS / 8;  // operand DMAs per wave per chunk (two rows each, four waves)
  constexpr int DG = SA ? D : 0;  // gamma loads per wave per chunk
  static_assert(!SA || BF16, "scale-after takes bf16 operands");
  static_assert(MT >= 2 && MT <= 4, "two to four token blocks");
  __shared__ uint4 abuf[2 * ROWS * GPR];  // two chunks: 2 x 64 rows x 512 B = 64 KiB at MT = 4
  __shared__ uint4 wst[4][32 * 8];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * 128 + wid * 32;
  const int64_t kbase = static_cast<int64_t>(blockIdx.y) * nch * (KS * 64);
  const int lr = lane & 15, lq = lane >> 4;

  // DMA i of this wave covers row pair 4 i + wid: lane l fills physical slot
  // l % 32 of row 2 (4 i + wid) + l / 32, which holds logical granule
  // (s & ~15) | ((s & 15) ^ (row & 15)).
  uint32_t aoff[D];
#pragma unroll
  for (int i = 0; i < D; ++i) {
    const int row = 2 * (4 * i + wid) + (lane >> 5), s = lane & 31;
    const int gl = (s & ~15) | ((s & 15) ^ (row & 15));
    aoff[i] = static_cast<uint32_t>((min<int64_t>(row, d.m - 1) * d.lda + gl * 8) * 2);
  }
  const uint32_t lbase = lds_addr(abuf);
  // scale-after: lane's slot of DMA i is logical granule gsl[i] of row srow[i]
  int gsl[D];
#pragma unroll
  for (int i = 0; i < D; ++i) {
    const int row = 2 * (4 * i + wid) + (lane >> 5), sl = lane & 31;
    gsl[i] = (sl & ~15) | ((sl & 15) ^ (row & 15));
  }
  uint4 gam[SA ? D : 1];
  float ssq[SA ? D : 1];
#pragma unroll
  for (int i = 0; i < (SA ? D : 1); ++i) ssq[i] = 0.f;
  auto issue_op = [&](int c) {
    const uint16_t* ab = d.a + kbase + c * (KS * 64);
    const uint32_t lb = lbase + (c & 1) * (ROWS * GPR * 16);
#pragma unroll
    for (int i = 0; i < D; ++i) dma16(ab, aoff[i], lb + (4 * i + wid) * 1024);
    if constexpr (SA) {
      const uint16_t* gb = static_cast<const uint16_t*>(d.gamma) + kbase + c * (KS * 64);
#pragma unroll
      for (int i = 0; i < D; ++i) gam[i] = load16(gb + gsl[i] * 8);
    }
  };
  // scale-after: x -> bf16(x * gamma) in this wave's own slots of chunk c, and
  // the sums of squares of x (called after the chunk's DMAs and gamma landed)
  auto convert = [&](int c) {
    if constexpr (SA) {
      uint4* ab = abuf + (c & 1) * (ROWS * GPR);
      uint4 xv[D];
#pragma unroll
      for (int i = 0; i < D; ++i) xv[i] = ab[(2 * (4 * i + wid) + (lane >> 5)) * GPR + (lane & 31)];
#pragma unroll
      for (int i = 0; i < D; ++i) {
        float xf[8], gf[8];
        unpack8<BFA_DTYPE_BF16>(xv[i], xf);
        unpack8<BFA_DTYPE_BF16>(gam[i], gf);
        uint32_t o[4];
        if (blockIdx.x == 0) {  // every column tile has the same sums; the first stores them
#pragma unroll
          for (int j = 0; j < 8; ++j) ssq[i] += xf[j] * xf[j];
        }
#pragma unroll
        for (int j = 0; j < 4; ++j)
          o[j] = static_cast<uint32_t>(f32_to_bf16_bits(xf[2 * j] * gf[2 * j])) |
                 (static_cast<uint32_t>(f32_to_bf16_bits(xf[2 * j + 1] * gf[2 * j + 1])) << 16);
        ab[(2 * (4 * i + wid) + (lane >> 5)) * GPR + (lane & 31)] = make_uint4(o[0], o[1], o[2], o[3]);
      }
    }
  };

  uint4 wr[KS][4];
  const int wrow_l = lane >> 3, wg_l = lane & 7;
  const uint16_t* wrow[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) wrow[i] = d.w + min(n0 + i * 8 + wrow_l, d.n - 1) * d.ldw + kbase + wg_l * 8;

  issue_op(0);
#pragma unroll
  for (int s = 0; s < KS; ++s)
#pragma unroll
    for (int i = 0; i < 4; ++i) wr[s][i] = load16(wrow[i] + s * 64);

  f32x4_t acc[MT][2];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x4_t{};
  uint4* ws = wst[wid];

  // One chunk: stage, fragment reads and MFMAs per segment; NEXT requests the
  // following chunk's segment into the registers just staged.
  auto chunk = [&](int c, auto next_tag) {
    constexpr bool NEXT = decltype(next_tag)::value;
    const uint4* ab = abuf + (c & 1) * (ROWS * GPR);
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      if constexpr (NEXT) wait_vm<4 * (KS - 1) + D + DG>();
      else wait_vm_last(4 * (KS - 1 - s));
#pragma unroll
      for (int i = 0; i < 4; ++i) ws[wslot(i * 8 + wrow_l, wg_l)] = wr[s][i];
      asm volatile("" ::: "memory");
      if constexpr (NEXT) {
#pragma unroll
        for (int i = 0; i < 4; ++i) wr[s][i] = load16(wrow[i] + (c + 1) * (KS * 64) + s * 64);
      }
      uint4 wf[2][2], af[MT][2];
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int h = 0; h < 2; ++h) wf[j][h] = ws[wslot(j * 16 + lr, h * 4 + lq)];
#pragma unroll
      for (int i = 0; i < MT; ++i) {
        const int row = i * 16 + lr;
        const int g0 = s * 8 + lq, g1 = g0 + 4;
        af[i][0] = ab[row * GPR + ((g0 & ~15) | ((g0 & 15) ^ (row & 15)))];
        af[i][1] = ab[row * GPR + ((g1 & ~15) | ((g1 & 15) ^ (row & 15)))];
      }
      asm volatile("" ::: "memory");
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          acc[i][j] = mfma16<BF16>(af[i][0], wf[j][0], acc[i][j]);
          acc[i][j] = mfma16<BF16>(af[i][1], wf[j][1], acc[i][j]);
        }
    }
  };

  int c = 0;
  for (; c + 1 < nch; ++c) {
    // op(c) was issued before W(c)'s 4 KS loads: vmcnt(4 KS) means it landed;
    // the barrier publishes every wave's copies and shows that chunk c-1, the
    // last reader of buffer (c+1) & 1, is finished everywhere.
    wait_vm<4 * KS>();
    convert(c);
    __syncthreads();
    issue_op(c + 1);
    chunk(c, std::true_type{});
  }
  wait_vm<4 * KS>();
  convert(c);
  __syncthreads();
  chunk(c, std::false_type{});
  if constexpr (SA) {
    // rows 2 (4 i + wid) (lanes 0-31) and + 1 (lanes 32-63); every column tile
    // computes the same sums, the first one stores them
#pragma unroll
    for (int i = 0; i < D; ++i) {
      uint32_t x = __builtin_bit_cast(uint32_t, group16_sum_dpp(ssq[i])), y = x;
      swap16(x, y);
      const float tot = __builtin_bit_cast(float, x) + __builtin_bit_cast(float, y);
      const int row = 2 * (4 * i + wid) + (lane >> 5);
      if (blockIdx.x == 0 && (lane & 31) == 0 && row < d.m)
        d.stats[static_cast<int64_t>(blockIdx.y) * ROWS + row] = tot;
    }
  }

  // partial tile in register order, as qkv_decode_kernel with REG_ORDER
  float4* tb = reinterpret_cast<float4*>(d.part) +
               ((static_cast<int64_t>(blockIdx.y) * gridDim.x + blockIdx.x) * 4 + wid) * (MT * 2 * 64);
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
      tb[(i * 2 + j) * 64 + lane] = make_float4(acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]);
}

// Split-K reduction + epilogue for the register-order partials of
// qkv_decode_kernel.  One wave per (group of 4 tokens, head): lane p owns the
// RoPE pair (p, p + D/2) of the head for all 4 tokens, which in the partial
// layout is one float4 per split and column, and 16 consecutive lanes read 256
// consecutive bytes.  The splits are summed in order (deterministic), then each
// token goes through bias -> rounding -> per-head RMSNorm (a wave reduction per
// token) -> rounding -> RoPE -> store, as in the prefill epilogue.
template <int MAXP>  // RoPE pairs per lane: head_dim <= 2 * 64 * MAXP
__device__ __forceinline__ void decode_epilogue_item(const float4* part, int64_t splits,
                                                              int64_t ntiles, int mt, int64_t m,
                                                              const QkvEpi& e, int64_t tg, int64_t h,
                                                              int lane) {
  const int64_t i = tg / 4, lq = tg % 4;  // 16-token block, 4-token group inside it
  const int64_t half = e.hd / 2;
  const int kd = head_kind(e, h);
  const int64_t base = h * e.hd;
  const int64_t sstride = ntiles * 4 * mt * 2 * 64;  // float4 per split
  const bool rope = kd != 2 && e.cs != nullptr;
  const void* nw = kd == 0 ? e.qn_w : (kd == 1 ? e.kn_w : nullptr);
  auto index = [&](int64_t c) {
    const int64_t cw = c % 128;
    return (((c / 128) * 4 + cw / 32) * mt * 2 + i * 2 + (cw % 32) / 16) * 64 + lq * 16 + cw % 16;
  };
  // Loads go out in two dependent levels: positions, bias, norm weights and
  // the partials first; the cos/sin rows (which need the positions) next; only
  // then arithmetic and stores.  Every load is unconditional (indices clamped,
  // values masked) so that none waits behind a per-token or per-dtype branch.
  // absent inputs read a valid stand-in (the partials) and are masked after
  const void* posp = rope ? e.positions : part;
  // fused KV append: cache slots of the 4 tokens (first load level)
  const bool app = e.cache != nullptr && kd != 0;
  int64_t so[4] = {-1, -1, -1, -1};
  if (app) {
#pragma unroll
    for (int v = 0; v < 4; ++v) so[v] = e.slot_off[min(tg * 4 + v, m - 1)];
  }
  int64_t raw[4];
  if (rope && e.pos_is_i64) {
#pragma unroll
    for (int v = 0; v < 4; ++v) raw[v] = static_cast<const int64_t*>(posp)[min(tg * 4 + v, m - 1)];
  } else {
#pragma unroll
    for (int v = 0; v < 4; ++v) raw[v] = static_cast<const int32_t*>(posp)[min(tg * 4 + v, m - 1)];
  }
  // scale-after sums of squares of the first 8 splits, requested before the
  // partials (one memory round trip for both)
  float sl[8][4];
  {
    const float* stp = e.stats ? e.stats : reinterpret_cast<const float*>(part);
#pragma unroll
    for (int u = 0; u < 8; ++u)
#pragma unroll
      for (int v = 0; v < 4; ++v)
        sl[u][v] = stp[e.stats ? min<int64_t>(u, splits - 1) * e.stat_rows + min(tg * 4 + v, m - 1) : 0];
  }
  // partials of the first 8 splits (indices clamped, masked when summed)
  float4 l1[MAXP][8], l2[MAXP][8];
#pragma unroll
  for (int pp = 0; pp < MAXP; ++pp) {
    const int64_t pc = min<int64_t>(lane + 64 * pp, half - 1);
    const float4* p1 = part + index(base + pc);
    const float4* p2 = part + index(base + half + pc);
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int64_t sp = min<int64_t>(u, splits - 1);
      l1[pp][u] = p1[sp * sstride];
      l2[pp][u] = p2[sp * sstride];
    }
  }
  // the cos/sin rows wait only for the positions (requested first), so they go
  // out before the partials are summed
  int64_t pos[4];
  bool pok[4];
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int32_t c = epi_pos_check(e, raw[v]);
    pok[v] = c >= 0;
    pos[v] = pok[v] ? c : 0;
  }
  float cs1[MAXP][4], sn1[MAXP][4];
#pragma unroll
  for (int pp = 0; pp < MAXP; ++pp) {
    const int64_t pc = min<int64_t>(lane + 64 * pp, half - 1);
    const float* csp = rope ? e.cs : reinterpret_cast<const float*>(part);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int64_t o = rope ? pos[v] * e.hd : 0;
      cs1[pp][v] = csp[o + pc];
      sn1[pp][v] = csp[o + half + pc];
    }
  }
  // bias and norm weights (uniform branches: nothing is read when absent)
  float b1[MAXP], b2[MAXP], g1[MAXP], g2[MAXP];
#pragma unroll
  for (int pp = 0; pp < MAXP; ++pp) {
    const int64_t pc = min<int64_t>(lane + 64 * pp, half - 1);  // lanes past the head re-read its last pair
    b1[pp] = b2[pp] = 0.f;
    g1[pp] = g2[pp] = 1.f;
    if (e.bias) load2_any(e.bias, e.bias_dtype, base + pc, base + half + pc, b1[pp], b2[pp]);
    if (nw) load2_any(nw, e.qk_w_dtype, pc, half + pc, g1[pp], g2[pp]);
  }
  asm volatile("" ::: "memory");
  float4 a1[MAXP], a2[MAXP];
#pragma unroll
  for (int pp = 0; pp < MAXP; ++pp) {
    a1[pp] = a2[pp] = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const bool in = u < splits;
      const float4 x = l1[pp][u], y = l2[pp][u];
      a1[pp].x += in ? x.x : 0.f; a1[pp].y += in ? x.y : 0.f; a1[pp].z += in ? x.z : 0.f; a1[pp].w += in ? x.w : 0.f;
      a2[pp].x += in ? y.x : 0.f; a2[pp].y += in ? y.y : 0.f; a2[pp].z += in ? y.z : 0.f; a2[pp].w += in ? y.w : 0.f;
    }
    if (splits > 8) {
      const int64_t pc = min<int64_t>(lane + 64 * pp, half - 1);
      const float4* p1 = part + index(base + pc);
      const float4* p2 = part + index(base + half + pc);
      for (int64_t sp0 = 8; sp0 < splits; sp0 += 8) {
        float4 r1[8], r2[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int64_t sp = min(sp0 + u, splits - 1);
          r1[u] = p1[sp * sstride];
          r2[u] = p2[sp * sstride];
        }
        asm volatile("" ::: "memory");  // all 16 loads issue before the first sum waits
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const bool in = sp0 + u < splits;
          a1[pp].x += in ? r1[u].x : 0.f; a1[pp].y += in ? r1[u].y : 0.f;
          a1[pp].z += in ? r1[u].z : 0.f; a1[pp].w += in ? r1[u].w : 0.f;
          a2[pp].x += in ? r2[u].x : 0.f; a2[pp].y += in ? r2[u].y : 0.f;
          a2[pp].z += in ? r2[u].z : 0.f; a2[pp].w += in ? r2[u].w : 0.f;
        }
      }
    }
  }
  if (e.stats) {
    // scale-after: r per token from the splits' sums of squares, in split order
    // (the first 8 splits' values were requested with the partials)
    float sq[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < 8; ++u)
#pragma unroll
      for (int v = 0; v < 4; ++v) sq[v] += u < splits ? sl[u][v] : 0.f;
    for (int64_t sp = 8; sp < splits; ++sp)
#pragma unroll
      for (int v = 0; v < 4; ++v) sq[v] += e.stats[sp * e.stat_rows + min(tg * 4 + v, m - 1)];
    float r[4];
#pragma unroll
    for (int v = 0; v < 4; ++v) r[v] = 1.0f / sqrtf(sq[v] / static_cast<float>(e.hidden) + e.stat_eps);
#pragma unroll
    for (int pp = 0; pp < MAXP; ++pp) {
      a1[pp].x *= r[0]; a1[pp].y *= r[1]; a1[pp].z *= r[2]; a1[pp].w *= r[3];
      a2[pp].x *= r[0]; a2[pp].y *= r[1]; a2[pp].z *= r[2]; a2[pp].w *= r[3];
    }
  }
  float x1[MAXP][4], x2[MAXP][4];
  float ss[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int pp = 0; pp < MAXP; ++pp) {
    const float s1[4] = {a1[pp].x, a1[pp].y, a1[pp].z, a1[pp].w};
    const float s2[4] = {a2[pp].x, a2[pp].y, a2[pp].z, a2[pp].w};
    const bool act = lane + 64 * pp < half;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      x1[pp][v] = round_to(s1[v] + b1[pp], e.qkv_dt);
      x2[pp][v] = round_to(s2[v] + b2[pp], e.qkv_dt);
      if (act) ss[v] += x1[pp][v] * x1[pp][v] + x2[pp][v] * x2[pp][v];
    }
  }
  int dt = e.qkv_dt;
  if (kd != 2 && (e.qn_w || e.kn_w)) {
#pragma unroll
    for (int v = 0; v < 4; ++v) ss[v] = wave_sum_dpp(ss[v]);
    if (nw) {
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const float r = __builtin_amdgcn_rsqf(ss[v] / static_cast<float>(e.hd) + e.qk_eps);
#pragma unroll
        for (int pp = 0; pp < MAXP; ++pp) {
          x1[pp][v] = round_to((x1[pp][v] * r) * g1[pp], e.norm_dt);
          x2[pp][v] = round_to((x2[pp][v] * r) * g2[pp], e.norm_dt);
        }
      }
      dt = e.norm_dt;
    }
  }
  if (rope && lane == 0 && h == 0) {
#pragma unroll
    for (int v = 0; v < 4; ++v)
      if (!pok[v] && tg * 4 + v < m) flag_status(e.status, BFA_STATUS_INDEX_OOB);
  }
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int64_t t = tg * 4 + v;
    if (t >= m) continue;
#pragma unroll
    for (int pp = 0; pp < MAXP; ++pp) {
      const int64_t p = lane + 64 * pp;
      if (p >= half) continue;
      float a = x1[pp][v], b = x2[pp][v];
      if (rope) {
        const float u = a, w = b, c = cs1[pp][v], sn = sn1[pp][v];
        a = pok[v] ? round_to(u * c - w * sn, dt) : 0.f;
        b = pok[v] ? round_to(w * c + u * sn, dt) : 0.f;
      }
      if (kd == 0 || !e.skip_kv_out) {
        store_any(e.out, e.out_dt, t * e.ldo + base + p, a);
        store_any(e.out, e.out_dt, t * e.ldo + base + half + p, b);
      }
      if (app && so[v] >= 0) {
        const int64_t hk = h - e.hq - (kd == 2 ? e.hkv : 0);
        const int64_t cb = so[v] + (kd == 2 ? e.c_skv : 0) + hk * e.c_sh;
        store_any(e.cache, e.cache_dt, cb + p, round_to(a, e.out_dt));
        store_any(e.cache, e.cache_dt, cb + half + p, round_to(b, e.out_dt));
      }
    }
  }
}

// ================================== decode epilogue of the linear fusions
// One thread per (4-token group, output column): sums the split-K partials of
// the column (and of its up column, n + c, for EPI_SWIGLU) in split order and
// applies the EPI_LINEAR / EPI_SWIGLU element chain.  Partials are row-major
// [splits, m, nw] floats, or, from the weight-streaming kernel with more than
// one 16-token block (reg_order), float4 = 4 tokens of one column in the
// kernel's register order.
template <bool SWIGLU>
__global__ __launch_bounds__(256) void linear_decode_epilogue_kernel(const float* part, int64_t splits,
                                                                    int reg_order, int mt, int64_t m,
                                                                    int64_t nw, GemmArgs g, QkvEpi e) {
  const int64_t id = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (id >= cdiv(m, 4) * g.n) return;
  const int64_t tg = id / g.n, c = id - tg * g.n;
  // the residual and bias words go out with the partials (converted after the
  // sums): requested after them they were a second dependent memory round trip
  uint32_t rw[4] = {0u, 0u, 0u, 0u}, bw = 0u;
  const int rdt = e.res ? e.res_dt : BFA_DTYPE_F32, bdt = e.bias ? e.bias_dtype : BFA_DTYPE_F32;
  if constexpr (!SWIGLU) {
#pragma unroll
    for (int v = 0; v < 4; ++v)
      rw[v] = ld_word(e.res ? e.res : static_cast<const void*>(part), rdt,
                      e.res ? min(tg * 4 + v, m - 1) * e.ldr + c : 0);
    bw = ld_word(e.bias ? e.bias : static_cast<const void*>(part), bdt, e.bias ? c : 0);
  }
  float acc[2][4];
#pragma unroll
  for (int f = 0; f < 2; ++f)
#pragma unroll
    for (int v = 0; v < 4; ++v) acc[f][v] = 0.f;
  constexpr int nf = SWIGLU ? 2 : 1;
#pragma unroll
  for (int f = 0; f < nf; ++f) {
    const int64_t col = c + f * g.n;
    if (reg_order) {
      const int64_t i = tg / 4, lq = tg % 4, cw = col % 128;
      const int64_t ntiles = cdiv(nw, 128);
      const int64_t idx = (((col / 128) * 4 + cw / 32) * mt * 2 + i * 2 + (cw % 32) / 16) * 64 + lq * 16 + cw % 16;
      const int64_t sstride = ntiles * 4 * mt * 2 * 64;
      const float4* p4 = reinterpret_cast<const float4*>(part) + idx;
      for (int64_t sp0 = 0; sp0 < splits; sp0 += 8) {
        float4 l[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) l[u] = p4[min(sp0 + u, splits - 1) * sstride];
        // all 8 loads issue before the first sum waits: a conditional exit in the
        // sum loop lets the compiler sink each load to its use, one round trip each
        asm volatile("" ::: "memory");
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const bool in = sp0 + u < splits;
          acc[f][0] += in ? l[u].x : 0.f; acc[f][1] += in ? l[u].y : 0.f;
          acc[f][2] += in ? l[u].z : 0.f; acc[f][3] += in ? l[u].w : 0.f;
        }
      }
    } else {
      for (int64_t sp0 = 0; sp0 < splits; sp0 += 8) {
        float l[8][4];
#pragma unroll
        for (int u = 0; u < 8; ++u)
#pragma unroll
          for (int v = 0; v < 4; ++v)
            l[u][v] = part[(min(sp0 + u, splits - 1) * m + min(tg * 4 + v, m - 1)) * nw + col];
        asm volatile("" ::: "memory");
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const bool in = sp0 + u < splits;
#pragma unroll
          for (int v = 0; v < 4; ++v) acc[f][v] += in ? l[u][v] : 0.f;
        }
      }
    }
  }
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int64_t t = tg * 4 + v;
    if (t >= m) break;
    float y;
    if constexpr (SWIGLU) {
      const float gt = round_to(acc[0][v], e.qkv_dt), ut = round_to(acc[1][v], e.qkv_dt);
      y = round_to(silu_fast(gt), e.qkv_dt) * ut;
    } else {
      const float r = e.res ? word_value(rw[v], rdt, e.res, t * e.ldr + c) : 0.f;
      const float b = e.bias ? word_value(bw, bdt, e.bias, c) : 0.f;
      y = round_to(round_to(acc[0][v] + b, e.qkv_dt) + r, e.mid_dt);
    }
    store_any(e.out, e.out_dt, t * e.ldo + c, y);
  }
}

template <int MAXP>
__global__ __launch_bounds__(256) void qkv_decode_epilogue_kernel(const float4* part, int64_t splits,
                                                                  int64_t ntiles, int mt, int64_t m,
                                                                  QkvEpi e) {
  const int64_t heads = e.hq + 2 * e.hkv;
  const int64_t item = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (item >= cdiv(m, 4) * heads) return;
  const int64_t tg = item / heads;
  decode_epilogue_item<MAXP>(part, splits, ntiles, mt, m, e, tg, item - tg * heads, threadIdx.x & 63);
}

// ================================== decode: whole-K column-pair tiles
// 17-64 tokens, head_dim a multiple of 32, no q/k norm.  A workgroup owns 32
// output columns -- 16 of the first half of a head, h D + c0 + [0, 16), and the
// 16 that RoPE pairs with them, + D/2 -- for every token and the whole of K, so
// the projection never leaves the workgroup: no split-K partials, no reduction
// kernel.  The four waves split K: wave w takes the 64-deep segment w of every
// 256-deep chunk and streams it on its own, with no barrier until the end.  Per
// chunk the wave DMAs its operand segment (rows x 128 B) and its weight segment
// (32 rows x 128 B: the 16 first-half columns, then their pairs), whole cache
// lines, into slots of its private LDS rings (granule g of row r at slot
// g ^ (r/2 & 7)), and reads 16x16x32 fragments from there.  The weight ring is
// deeper than the operand ring (HBM against L2 latency).  The loop issues no
// other memory request, so the one wait per chunk is exact (the requests issued
// after the chunk's operand DMAs may stay in flight), and the chunks that reuse
// c's slots are requested as soon as c's fragments are in registers, before
// c's arithmetic.
// At the end the four partial tiles are summed through LDS in wave order and
// wave i finishes the rows of 16-token block i: a lane holds the pair (p, p + D/2)
// of four rows in its two accumulators, so RoPE needs no exchange.
//
// SA (scale-after, the fp32 variants, bf16 x and gamma): the operand is the raw
// x and gamma goes onto the weight fragments (bf16(w * gamma): every weight
// element is used by one workgroup only, where x * gamma would be redone by every
// column tile; the segment's 64 gamma values come with the chunk, one 8-lane
// DMA); the rows' sums of squares come from one more MFMA of each operand
// fragment with itself (the diagonal of the 16x16 Gram block), and the epilogue
// multiplies the projection by r = 1 / sqrt(sum / hidden + eps) before the bias.
// No pass over x and no other launch.

// Ring slots per wave: RX operand segments, RW weight (+ gamma) segments.  At
// 64 tokens, Llama-3-8B shape, the K loop took 10.0 us with (3, 2) and (4, 1),
// 10.3 with (3, 3), 11.4-11.6 with (2, 3) and (2, 5): the operand (read by every
// workgroup, 512 KiB at 64 tokens) wants the depth; past that the loop is bound
// by the LDS (every byte DMA'd in and read out as a fragment), not by latency.
template <int MT> struct PairRing {
  static constexpr int RX = 3;
  static constexpr int RW = 2;
};

// s_waitcnt vmcnt(n) for a run-time n in [LO, HI] (a binary search over constant waits)
template <int LO, int HI>
__device__ __forceinline__ void wait_vm_dyn(int n) {
  if constexpr (LO >= HI) {
    wait_vm<LO>();
  } else {
    constexpr int MID = (LO + HI + 1) / 2;
    if (n >= MID) wait_vm_dyn<MID, HI>(n);
    else wait_vm_dyn<LO, MID - 1>(n);
  }
}

// GIN (with SA): gamma goes onto the weight fragments in the kernel; without,
// the weight already holds bf16(w * gamma) (bfa_fold_rmsnorm_weight).
template <int MT, bool SA, int EDT, bool GIN = true>
__global__ __launch_bounds__(256) void qkv_decode_pair_kernel(DecodeArgs d, QkvEpi e, int nch) {
  using DT = EpiDt<EDT>;
  constexpr bool G = SA && GIN;         // gamma applied here
  constexpr int RX = PairRing<MT>::RX, RW = PairRing<MT>::RW;
  constexpr int ROWS = MT * 16;
  constexpr int XN = ROWS / 8;          // operand DMAs per wave per chunk (8 rows x 128 B)
  constexpr int WN = 4 + (G ? 1 : 0);   // weight DMAs (+ gamma)
  constexpr int XS = ROWS * 8;          // uint4 per operand slot
  constexpr int WS = 32 * 8 + (G ? 8 : 0);  // uint4 per weight slot: 32 rows, then 64 gamma values
  constexpr int WAVE_U4 = RX * XS + RW * WS;
  // requests issued after the later of a chunk's operand and weight requests
  constexpr int YMAX = RX < RW ? WN + (RX - 1) * (XN + WN) : (RW - 1) * (XN + WN);
  static_assert(MT >= 2 && MT <= 4, "two to four token blocks");
  static_assert(YMAX < 64, "ring shape");
  __shared__ uint4 ring[4 * WAVE_U4];
  __shared__ uint32_t posl[4][32];  // per wave: the raw positions of its 16 epilogue rows

  const int tid = threadIdx.x, lane = tid & 63;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lr = lane & 15, lq = lane >> 4;
  const int64_t tph = e.hd / 32;  // pair tiles per head
  const int64_t head = blockIdx.x / tph;
  const int64_t c0 = (blockIdx.x - head * tph) * 16;  // first pair of the tile inside the head
  const int64_t half = e.hd / 2;
  const int64_t cola = head * e.hd + c0;  // columns cola + [0, 16) and cola + half + [0, 16)

  // DMA j of a 128-byte-row block covers its rows 8 j .. 8 j + 7: lane l fills
  // slot l % 8 of row 8 j + l / 8, i.e. logical granule (l % 8) ^ (row / 2 & 7).
  // Operand rows past m re-read row m - 1; weight row 8 j + l / 8 of the tile is
  // column cola + row (rows < 16) or cola + half + row - 16.
  uint32_t aoff[XN], woff[4];
#pragma unroll
  for (int j = 0; j < XN; ++j) {
    const int row = 8 * j + (lane >> 3);
    const int g = (lane & 7) ^ ((row >> 1) & 7);
    aoff[j] = static_cast<uint32_t>((min<int64_t>(row, d.m - 1) * d.lda + wid * 64 + g * 8) * 2);
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int row = 8 * j + (lane >> 3);
    const int g = (lane & 7) ^ ((row >> 1) & 7);
    const int64_t col = cola + (row < 16 ? row : half + row - 16);
    woff[j] = static_cast<uint32_t>((col * d.ldw + wid * 64 + g * 8) * 2);
  }
  const uint32_t lring = lds_addr(ring) + static_cast<uint32_t>(wid * WAVE_U4 * 16);
  const uint32_t goff = static_cast<uint32_t>((wid * 64 + lane * 8) * 2);
  // Each workgroup walks the chunks from its own starting point (workgroups of
  // one XCD, i = xcd + 8 j, start at chunk j mod nch): rows are a power of two
  // apart, so in lockstep every workgroup would read the same 512-byte column
  // band of x and W, which sits in a few L2 channels.
  const int rot = static_cast<int>((blockIdx.x >> 3) % static_cast<unsigned>(nch));
  auto kchunk = [&](int c) { return c + rot < nch ? c + rot : c + rot - nch; };
  // Requests, in issue order: at step v (v < 0: the prologue) the operand of
  // chunk v + RX, then the weight of chunk v + RW, each while it exists.  Before
  // chunk c the wave waits for its operand (issued at step c - RX, after the
  // weight of c), i.e. for vmcnt(requests issued after it): younger(c).
  auto issue_x = [&](int c) {
    const uint32_t ls = lring + static_cast<uint32_t>((c % RX) * XS * 16);
    const uint16_t* ab = d.a + static_cast<int64_t>(kchunk(c)) * 256;
#pragma unroll
    for (int j = 0; j < XN; ++j) dma16(ab, aoff[j], ls + j * 1024);
  };
  auto issue_w = [&](int c) {
    const uint32_t ls = lring + static_cast<uint32_t>((RX * XS + (c % RW) * WS) * 16);
    const int64_t kc = kchunk(c);
    const uint16_t* wb = d.w + kc * 256;
#pragma unroll
    for (int j = 0; j < 4; ++j) dma16(wb, woff[j], ls + j * 1024);
    if constexpr (G) {
      // lanes 0-7: the segment's 64 gamma values
      if (lane < 8) dma16(static_cast<const uint16_t*>(d.gamma) + kc * 256, goff, ls + 256 * 16);
    }
  };
  auto step_issue = [&](int v) {
    if (v + RX >= 0 && v + RX < nch) issue_x(v + RX);
    if (v + RW >= 0 && v + RW < nch) issue_w(v + RW);
  };
  auto younger = [&](int c) {
    // the later of chunk c's requests: its operand (step c - RX) when RX < RW,
    // else its weight (step c - RW, the last request of that step)
    constexpr int RL = RX < RW ? RX : RW;
    int n = RX < RW && c - RX + RW < nch ? WN : 0;
#pragma unroll
    for (int i = 1; i < RL; ++i) {
      const int v = c - RL + i;
      n += (v + RX < nch ? XN : 0) + (v + RW < nch ? WN : 0);
    }
    return n;
  };

  // this lane finishes rows 16 wid + 4 lq + v of columns cola + lr, + half (wid < MT)
  const int kd = head_kind(e, head);
  const bool rope = kd != 2 && e.cs != nullptr;
  // Epilogue inputs.  The compiler waits for a load it issued by counting only
  // its own requests, so a use of one inside the loop would wait for every DMA
  // in flight: the positions come by DMA into LDS instead (one 4-byte request
  // per lane, ahead of the ring, so chunk 0's wait covers them) and the cos/sin
  // rows are requested once chunk 0 has landed; the bias and the cache slots
  // need nothing and go out first.  All of them are used after the loop.
  const int psh = e.pos_is_i64 ? 1 : 0;
  if (rope && wid < MT && lane < (16 << psh)) {
    const int64_t t = min<int64_t>(wid * 16 + (lane >> psh), d.m - 1);
    dma4(e.positions, static_cast<uint32_t>(((t << psh) + (lane & psh)) * 4), lds_addr(posl[wid]));
  }
  float cs[4] = {1.f, 1.f, 1.f, 1.f}, sn[4] = {0.f, 0.f, 0.f, 0.f};
  uint32_t bw[4] = {0, 0, 0, 0};
  int64_t so[4] = {-1, -1, -1, -1};
  bool pok[4] = {true, true, true, true};
  const bool app = e.cache != nullptr && kd != 0;
  const int64_t p = c0 + lr;  // this lane's pair inside the head
  if (wid < MT) {
    if (e.bias) {
      // 16-bit words (an fp32 bias element is two), combined after the loop
      const uint16_t* bp = static_cast<const uint16_t*>(e.bias);
      const int sh = e.bias_dtype == BFA_DTYPE_F32 ? 1 : 0;
      const int64_t ia = (cola + lr) << sh, ib = (cola + half + lr) << sh;
      bw[0] = bp[ia]; bw[1] = bp[ia + sh]; bw[2] = bp[ib]; bw[3] = bp[ib + sh];
    }
    if (app) {
#pragma unroll
      for (int v = 0; v < 4; ++v) so[v] = e.slot_off[min<int64_t>(wid * 16 + lq * 4 + v, d.m - 1)];
    }
  }
  auto rope_loads = [&]() {
    if (wid >= MT || !rope) return;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int r = lq * 4 + v;
      const int64_t raw = psh ? static_cast<int64_t>((static_cast<uint64_t>(posl[wid][2 * r + 1]) << 32) |
                                                     posl[wid][2 * r])
                              : static_cast<int64_t>(static_cast<int32_t>(posl[wid][r]));
      const int32_t c = epi_pos_check(e, raw);
      pok[v] = c >= 0;
      const int64_t o = static_cast<int64_t>(pok[v] ? c : 0) * e.hd;
      cs[v] = e.cs[o + p];
      sn[v] = e.cs[o + half + p];
    }
  };
  // ring prologue: steps -max(RX, RW) .. -1
#pragma unroll
  for (int v = -(RX > RW ? RX : RW); v < 0; ++v) step_issue(v);

  f32x4_t acc[MT][2], gacc[SA ? MT : 1];
#pragma unroll
  for (int i = 0; i < MT; ++i) {
    acc[i][0] = acc[i][1] = f32x4_t{};
    if constexpr (SA) gacc[i] = f32x4_t{};
  }
  for (int c = 0; c < nch; ++c) {
    wait_vm_dyn<0, YMAX>(younger(c));
    asm volatile("" ::: "memory");  // no LDS read of the chunk moves above its wait
    if (c == 0) rope_loads();
    const uint4* xs = ring + wid * WAVE_U4 + (c % RX) * XS;
    const uint4* wsl = ring + wid * WAVE_U4 + RX * XS + (c % RW) * WS;
    uint4 wf[2][2], af[MT][2];
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int h = 0; h < 2; ++h) af[i][h] = xs[wslot(i * 16 + lr, h * 4 + lq)];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int h = 0; h < 2; ++h) wf[j][h] = wsl[wslot(j * 16 + lr, h * 4 + lq)];
    uint4 gw[2] = {};
    if constexpr (G) {
      gw[0] = wsl[256 + lq];
      gw[1] = wsl[256 + 4 + lq];
    }
    // chunk c + RX (c + RW) reuses this operand (weight) slot: its DMAs go out
    // as soon as every read of chunk c has returned, and the conversion and
    // MFMAs below run from registers while they are in flight
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    step_issue(c);
    if constexpr (SA) {
      // bf16(w * gamma) for fragment half h (this lane's k range: h 32 + lq 8
      // .. + 8 of the segment).  Three scheduling regions put the conversion
      // under the matrix cores: (A) the Gram MFMAs with the conversion of half
      // 0, (B) half 0's MFMAs with the conversion of half 1, (C) half 1's MFMAs;
      // inside A and B one MFMA alternates with six VALU instructions.
      auto convert = [&](int h) {
        float gf[8];
        unpack8<BFA_DTYPE_BF16>(gw[h], gf);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          float w8[8];
          unpack8<BFA_DTYPE_BF16>(wf[j][h], w8);
          uint32_t o[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) o[q] = pack_bf16x2(w8[2 * q] * gf[2 * q], w8[2 * q + 1] * gf[2 * q + 1]);
          wf[j][h] = make_uint4(o[0], o[1], o[2], o[3]);
        }
      };
      auto interleave = [&]() {
#pragma unroll
        for (int q = 0; q < 2 * MT; ++q) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
          __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);  // six VALU
        }
      };
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int h = 0; h < 2; ++h) gacc[i] = mfma16<true>(af[i][h], af[i][h], gacc[i]);
      if constexpr (G) {
        convert(0);
        interleave();
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int i = 0; i < MT; ++i) {
        acc[i][0] = mfma16<true>(af[i][0], wf[0][0], acc[i][0]);
        acc[i][1] = mfma16<true>(af[i][0], wf[1][0], acc[i][1]);
      }
      if constexpr (G) {
        convert(1);
        interleave();
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int i = 0; i < MT; ++i) {
        acc[i][0] = mfma16<true>(af[i][1], wf[0][1], acc[i][0]);
        acc[i][1] = mfma16<true>(af[i][1], wf[1][1], acc[i][1]);
      }
    } else {
#pragma unroll
      for (int i = 0; i < MT; ++i) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          acc[i][0] = mfma16<true>(af[i][h], wf[0][h], acc[i][0]);
          acc[i][1] = mfma16<true>(af[i][h], wf[1][h], acc[i][1]);
        }
      }
    }
  }

  // the four partial tiles (and Gram diagonals) through each wave's own ring
  float4* mine = reinterpret_cast<float4*>(ring + wid * WAVE_U4);
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
      mine[(i * 2 + j) * 64 + lane] = make_float4(acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]);
  if constexpr (SA) {
    float* st = reinterpret_cast<float*>(mine + MT * 2 * 64);
#pragma unroll
    for (int i = 0; i < MT; ++i)
      if ((lr >> 2) == lq) st[i * 16 + lr] = gacc[i][lr & 3];
  }
  __syncthreads();
  if (wid >= MT) return;
  const int i = wid;
  float a[4] = {0.f, 0.f, 0.f, 0.f}, b[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int wv = 0; wv < 4; ++wv) {
    const float4* t = reinterpret_cast<const float4*>(ring + wv * WAVE_U4);
    const float4 x = t[(i * 2) * 64 + lane], y = t[(i * 2 + 1) * 64 + lane];
    a[0] += x.x; a[1] += x.y; a[2] += x.z; a[3] += x.w;
    b[0] += y.x; b[1] += y.y; b[2] += y.z; b[3] += y.w;
  }
  if constexpr (SA) {
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      float s = 0.f;
#pragma unroll
      for (int wv = 0; wv < 4; ++wv)
        s += reinterpret_cast<const float*>(reinterpret_cast<const float4*>(ring + wv * WAVE_U4) +
                                            MT * 2 * 64)[i * 16 + lq * 4 + v];
      const float r = 1.0f / sqrtf(s / static_cast<float>(d.k) + d.eps);
      a[v] *= r;
      b[v] *= r;
    }
  }
  if (rope && head == 0 && c0 == 0 && lr == 0) {
#pragma unroll
    for (int v = 0; v < 4; ++v)
      if (!pok[v] && i * 16 + lq * 4 + v < d.m) flag_status(e.status, BFA_STATUS_INDEX_OOB);
  }
  float ba = 0.f, bb = 0.f;
  if (e.bias) {
    if (e.bias_dtype == BFA_DTYPE_F32) {
      ba = __builtin_bit_cast(float, (bw[1] << 16) | bw[0]);
      bb = __builtin_bit_cast(float, (bw[3] << 16) | bw[2]);
    } else if (e.bias_dtype == BFA_DTYPE_BF16) {
      ba = Elem<BFA_DTYPE_BF16>::to_f32(static_cast<uint16_t>(bw[0]));
      bb = Elem<BFA_DTYPE_BF16>::to_f32(static_cast<uint16_t>(bw[2]));
    } else {
      ba = Elem<BFA_DTYPE_F16>::to_f32(static_cast<uint16_t>(bw[0]));
      bb = Elem<BFA_DTYPE_F16>::to_f32(static_cast<uint16_t>(bw[2]));
    }
  }
  const int64_t hk = head - e.hq - (kd == 2 ? e.hkv : 0);
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int64_t t = i * 16 + lq * 4 + v;
    if (t >= d.m) continue;
    float x1 = rnd<DT::Q>(a[v] + ba, e.qkv_dt), x2 = rnd<DT::Q>(b[v] + bb, e.qkv_dt);
    if (rope) {
      const float u = x1, w = x2;
      x1 = pok[v] ? rnd<DT::Q>(u * cs[v] - w * sn[v], e.qkv_dt) : 0.f;
      x2 = pok[v] ? rnd<DT::Q>(w * cs[v] + u * sn[v], e.qkv_dt) : 0.f;
    }
    if (kd == 0 || !e.skip_kv_out) {
      if constexpr (DT::O >= 0) {
        store1<DT::O>(e.out, t * e.ldo + cola + lr, x1);
        store1<DT::O>(e.out, t * e.ldo + cola + half + lr, x2);
      } else {
        store_any(e.out, e.out_dt, t * e.ldo + cola + lr, x1);
        store_any(e.out, e.out_dt, t * e.ldo + cola + half + lr, x2);
      }
    }
    if (app && so[v] >= 0) {
      const int64_t cbase = so[v] + (kd == 2 ? e.c_skv : 0) + hk * e.c_sh;
      store_any(e.cache, e.cache_dt, cbase + p, rnd<DT::O>(x1, e.out_dt));
      store_any(e.cache, e.cache_dt, cbase + half + p, rnd<DT::O>(x2, e.out_dt));
    }
  }
}

// ============================================== reduction + row epilogue
// One wave per (token, head).  v = sum over splits of part[s, t, col] (+bias),
// then the same rounding / norm / RoPE chain as the in-register epilogue.
// MAXP: RoPE pairs per lane (head_dim <= 128 MAXP).
template <int MAXP>
__device__ __forceinline__ void row_epilogue_item(const float* part, int64_t splits, int64_t m,
                                                  const QkvEpi& e, int64_t t, int64_t h, int lane) {
  constexpr int SG = 8;    // splits whose partials are requested together
  const int64_t half = e.hd / 2;
  const int kd = head_kind(e, h);
  const int64_t base = h * e.hd;
  const void* nw = kd == 0 ? e.qn_w : (kd == 1 ? e.kn_w : nullptr);
  const bool norm = kd != 2 && (e.qn_w || e.kn_w);
  const bool rope = kd != 2 && e.cs;
  const bool app = e.cache != nullptr && kd != 0;
  // Every load goes out before any value is used, unconditionally at clamped
  // indices (absent inputs read a stand-in that is masked afterwards), so that
  // each use waits for its own loads only: the position first (the cos/sin
  // rows wait for it alone), then the cache slot, the bias and norm-weight
  // words, and the first SG splits' partials.
  const float* pr = part + t * e.n + base;
  const int32_t* p32 = static_cast<const int32_t*>(rope ? e.positions : static_cast<const void*>(pr));
  const int32_t plo = p32[!rope ? 0 : (e.pos_is_i64 ? 2 * t : t)];
  const int32_t phi = p32[!rope ? 0 : (e.pos_is_i64 ? 2 * t + 1 : t)];
  const int64_t so_raw = (app ? e.slot_off : reinterpret_cast<const int64_t*>(part))[app ? t : 0];
  int64_t jj[MAXP];
  bool jin[MAXP];
  uint32_t bw1[MAXP], bw2[MAXP], nw1[MAXP], nw2[MAXP];
  const int bdt = e.bias ? e.bias_dtype : BFA_DTYPE_F32;
  const int ndt = nw ? e.qk_w_dtype : BFA_DTYPE_F32;
#pragma unroll
  for (int p = 0; p < MAXP; ++p) {
    jin[p] = lane + 64 * p < half;
    jj[p] = jin[p] ? lane + 64 * p : 0;
    bw1[p] = ld_word(e.bias ? e.bias : static_cast<const void*>(pr), bdt, e.bias ? base + jj[p] : 0);
    bw2[p] = ld_word(e.bias ? e.bias : static_cast<const void*>(pr), bdt, e.bias ? base + half + jj[p] : 0);
    nw1[p] = ld_word(nw ? nw : static_cast<const void*>(pr), ndt, nw ? jj[p] : 0);
    nw2[p] = ld_word(nw ? nw : static_cast<const void*>(pr), ndt, nw ? half + jj[p] : 0);
  }
  const int64_t stride = m * e.n;
  float s1[MAXP], s2[MAXP];
#pragma unroll
  for (int p = 0; p < MAXP; ++p) s1[p] = s2[p] = 0.f;
  float v1[SG][MAXP], v2[SG][MAXP];
  auto load_group = [&](int64_t sp0) {
#pragma unroll
    for (int u = 0; u < SG; ++u) {
      const int64_t sp = min(sp0 + u, splits - 1);
#pragma unroll
      for (int p = 0; p < MAXP; ++p) {
        v1[u][p] = pr[sp * stride + jj[p]];
        v2[u][p] = pr[sp * stride + half + jj[p]];
      }
    }
  };
  load_group(0);
  // the cos/sin values (they wait for the position only)
  const int64_t praw = e.pos_is_i64 ? static_cast<int64_t>((static_cast<uint64_t>(static_cast<uint32_t>(phi)) << 32) |
                                                           static_cast<uint32_t>(plo))
                                    : static_cast<int64_t>(plo);
  const int32_t pc = rope ? epi_pos_check(e, praw) : 0;
  const float* csr = rope ? e.cs + static_cast<int64_t>(pc >= 0 ? pc : 0) * e.hd : pr;
  float cv[MAXP], sv[MAXP];
#pragma unroll
  for (int p = 0; p < MAXP; ++p) {
    cv[p] = csr[rope ? jj[p] : 0];
    sv[p] = csr[rope ? half + jj[p] : 0];
  }
  // the split sums, in split order
  for (int64_t sp0 = 0;;) {
#pragma unroll
    for (int u = 0; u < SG; ++u) {
      const bool in = sp0 + u < splits;
#pragma unroll
      for (int p = 0; p < MAXP; ++p) {
        s1[p] += in ? v1[u][p] : 0.f;
        s2[p] += in ? v2[u][p] : 0.f;
      }
    }
    sp0 += SG;
    if (sp0 >= splits) break;
    load_group(sp0);
  }
  int dt = e.qkv_dt;
  float x1[MAXP], x2[MAXP], ss = 0.f;
#pragma unroll
  for (int p = 0; p < MAXP; ++p) {
    const float b1 = e.bias ? word_value(bw1[p], bdt, e.bias, base + jj[p]) : 0.f;
    const float b2 = e.bias ? word_value(bw2[p], bdt, e.bias, base + half + jj[p]) : 0.f;
    x1[p] = jin[p] ? round_to(s1[p] + b1, e.qkv_dt) : 0.f;
    x2[p] = jin[p] ? round_to(s2[p] + b2, e.qkv_dt) : 0.f;
    ss += x1[p] * x1[p] + x2[p] * x2[p];
  }
  if (norm) {
    ss = wave_sum_dpp(ss);
    if (nw) {
      const float r = __builtin_amdgcn_rsqf(ss / static_cast<float>(e.hd) + e.qk_eps);
#pragma unroll
      for (int p = 0; p < MAXP; ++p) {
        x1[p] = round_to((x1[p] * r) * word_value(nw1[p], ndt, nw, jj[p]), e.norm_dt);
        x2[p] = round_to((x2[p] * r) * word_value(nw2[p], ndt, nw, half + jj[p]), e.norm_dt);
      }
      dt = e.norm_dt;
    }
  }
  if (rope) {
    const bool ok = pc >= 0;
    if (!ok && h == 0 && lane == 0) flag_status(e.status, BFA_STATUS_INDEX_OOB);
#pragma unroll
    for (int p = 0; p < MAXP; ++p) {
      const float a = x1[p], b = x2[p];
      x1[p] = ok ? round_to(a * cv[p] - b * sv[p], dt) : 0.f;
      x2[p] = ok ? round_to(b * cv[p] + a * sv[p], dt) : 0.f;
    }
  }
  const int64_t so = app ? so_raw : -1;
  const int64_t cb = so + (kd == 2 ? e.c_skv : 0) + (h - e.hq - (kd == 2 ? e.hkv : 0)) * e.c_sh;
#pragma unroll
  for (int p = 0; p < MAXP; ++p) {
    const int64_t j = jj[p];
    if (jin[p]) {
      if (kd == 0 || !e.skip_kv_out) {
        store_any(e.out, e.out_dt, t * e.ldo + base + j, x1[p]);
        store_any(e.out, e.out_dt, t * e.ldo + base + half + j, x2[p]);
      }
      if (app && so >= 0) {
        store_any(e.cache, e.cache_dt, cb + j, round_to(x1[p], e.out_dt));
        store_any(e.cache, e.cache_dt, cb + half + j, round_to(x2[p], e.out_dt));
      }
    }
  }
}

template <int MAXP>
__global__ __launch_bounds__(256) void qkv_epilogue_kernel(const float* part, int64_t splits,
                                                           int64_t m, QkvEpi e) {
  const int64_t heads = e.hq + 2 * e.hkv;
  // wave-uniform (scalar) item, so the head kind and its flags are too: a
  // divergent-looking test would let the compiler sink loads into it and wait
  // for every load at its end
  const int64_t item = static_cast<int64_t>(blockIdx.x) * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (item >= m * heads) return;
  const int64_t t = item / heads;
  row_epilogue_item<MAXP>(part, splits, m, e, t, item - t * heads, threadIdx.x & 63);
}

// ================================================================== host
struct QkvPlan {
  bool decode;
  int mt;        // decode: 16-row blocks
  int cpw;       // decode: 16-column blocks per wave
  int64_t splits;
  int64_t kchunk;
  bool fused_epi;  // prefill: in-register epilogue
  int tile;        // prefill: 2 (256x256, 8 waves), 3 (128x256, 8 waves), 1 (128x256, 4 waves), 128, 64 (128x64)
  bool stream;     // decode: weight-streaming kernel (k % 64 == 0)
  int ks;          // decode stream: 64-deep K segments per split
  int nch;         // decode stream: 256-deep chunks per split of the deep-K form (0: not used)
  int64_t operand_bytes;
  int64_t part_bytes;
};

static int64_t align256(int64_t v) { return (v + 255) / 256 * 256; }

static QkvPlan make_plan(int64_t m, int64_t n, int64_t k, int64_t hd) {
  QkvPlan p{};
  p.operand_bytes = align256(m * k * 2);
  if (m <= 64) {
    p.decode = true;
    p.mt = static_cast<int>(cdiv(m, 16));
    p.stream = k % 64 == 0;
    if (p.stream) {
      // 128 columns per workgroup; K split into equal slices of ks segments (ks
      // divides k / 64, at most 8): the deepest slice that still gives one
      // workgroup per CU (256), since every extra split adds an fp32 partial
      // tile (m x n x 4 bytes) to write and reduce.
      const int64_t segs = k / 64, ntile = cdiv(n, 128);
      int ks = 1;
      for (int c = 8; c >= 1; --c)
        if (segs % c == 0 && ntile * (segs / c) >= 256) { ks = c; break; }
      // planner override BFA_TUNE_DECODE_KS (1..8, dividing k / 64) sets the depth
      {
        const int c = tuning(BFA_TUNE_DECODE_KS);
        if (c >= 1 && c <= 8 && segs % c == 0) ks = c;
      }
      p.ks = ks;
      p.kchunk = 64 * ks;
      p.splits = segs / ks;
      p.cpw = 2;
      // From two token blocks up the partial tiles cost more than the extra
      // workgroups gain: the deep-K form takes the fewest splits of 256-deep
      // chunks that still give 192 workgroups (override BFA_TUNE_DECODE_WG),
      // with at least two chunks per split.  Override BFA_TUNE_DECODE_SPLITS
      // (dividing the chunk count) sets the split count.
      const int64_t chunks = segs / LOOP_KS;
      if (p.mt > 1 && segs % LOOP_KS == 0 && chunks >= 2) {
        int64_t target = 192;
        if (tuning(BFA_TUNE_DECODE_WG) >= 1) target = tuning(BFA_TUNE_DECODE_WG);
        int64_t sp = chunks;
        for (int64_t c = 1; c <= chunks; ++c)
          if (chunks % c == 0 && ntile * c >= target) { sp = c; break; }
        {
          const int64_t c = tuning(BFA_TUNE_DECODE_SPLITS);
          if (c >= 1 && chunks % c == 0) sp = c;
        }
        if (chunks / sp >= 2) {
          p.nch = static_cast<int>(chunks / sp);
          p.splits = sp;
          p.ks = LOOP_KS;
          p.kchunk = 64 * LOOP_KS * p.nch;
        }
      }
    } else {
      // Column tile per workgroup: 4 waves x cpw x 16 columns.
      p.cpw = m > 16 ? 1 : 2;
      const int64_t ntile = cdiv(n, 4 * 16 * p.cpw);
      // Split K until about 512 workgroups are in flight, but keep the fp32
      // partial traffic (2 * splits * m * n * 4 bytes) small next to the weight
      // stream (n * k * 2 bytes): splits <= k / (32 m) bounds it at 1/4.
      int64_t splits = std::max<int64_t>(1, cdiv(512, ntile));
      splits = std::min<int64_t>(splits, std::max<int64_t>(1, k / 128));
      splits = std::min<int64_t>(splits, std::max<int64_t>(1, k / (32 * m)));
      p.kchunk = cdiv(cdiv(k, splits), 64) * 64;
      p.splits = cdiv(k, p.kchunk);
    }
    // stream kernel from 2 token blocks: register-order partial tiles padded to
    // 128 columns x 16 MT rows; otherwise row-major [splits, m, n]
    p.part_bytes = (p.stream && p.mt > 1) ? align256(p.splits * cdiv(n, 128) * 128 * p.mt * 16 * 4)
                                          : align256(p.splits * m * n * 4);
  } else {
    p.decode = false;
    p.fused_epi = (hd == 32 || hd == 64 || hd == 128) && n % hd == 0;
    // Largest tile that still fills the CUs: 256x256 with 8 waves (two per
    // SIMD, full-line 64-deep DMA stages) from one tile per CU; else 128x256
    // with 8 waves from 192 tiles; else 128x128 with 4 waves (two workgroups
    // per CU).  Override BFA_TUNE_QKV_TILE (2: 256x256 8 waves, 3: 128x256 8
    // waves, 1: 128x256 4 waves, 128: 128x128) sets the tile.
    if (cdiv(m, 256) * cdiv(n, 256) >= 256) p.tile = 2;
    else if (cdiv(m, 128) * cdiv(n, 256) >= 192) p.tile = 3;
    else p.tile = 128;
    // Under 128 tiles of 128x128 most CUs would idle, and each busy one is
    // bound by its LDS traffic: for heads of up to 64 columns 128x64 tiles put
    // twice the CUs on the product (TinyLlama, 512 tokens: 80 -> 160 tiles).
    const bool narrow_ok = p.fused_epi && hd <= 64;
    if (p.tile == 128 && narrow_ok && cdiv(m, 128) * cdiv(n, 128) < 128) p.tile = 64;
    {
      const int v = tuning(BFA_TUNE_QKV_TILE);
      if ((v >= 1 && v <= 3) || v == 128 || (v == 64 && narrow_ok)) p.tile = v;
    }
    p.splits = 1;
    p.part_bytes = p.fused_epi ? 0 : align256(m * n * 4);
  }
  return p;
}

template <bool BF16, int CPW>
static void launch_decode_cpw(const QkvPlan& p, const SplitArgs& s, hipStream_t st) {
  const dim3 grid(static_cast<unsigned>(cdiv(s.n, 4 * 16 * CPW)), static_cast<unsigned>(p.splits));
  switch (p.mt) {
    case 1: hipLaunchKernelGGL((qkv_splitk_kernel<1, CPW, BF16>), grid, dim3(256), 0, st, s); break;
    case 2: hipLaunchKernelGGL((qkv_splitk_kernel<2, CPW, BF16>), grid, dim3(256), 0, st, s); break;
    case 3: hipLaunchKernelGGL((qkv_splitk_kernel<3, CPW, BF16>), grid, dim3(256), 0, st, s); break;
    default: hipLaunchKernelGGL((qkv_splitk_kernel<4, CPW, BF16>), grid, dim3(256), 0, st, s); break;
  }
}

template <int NR, bool BF16>
static void launch_stream_fold(int ks, dim3 grid, const DecodeArgs& d, hipStream_t st) {
  switch (ks) {
    case 1: hipLaunchKernelGGL((qkv_decode_kernel<1, 1, BF16, false, NR>), grid, dim3(256), 0, st, d); break;
    case 2: hipLaunchKernelGGL((qkv_decode_kernel<1, 2, BF16, false, NR>), grid, dim3(256), 0, st, d); break;
    case 3: hipLaunchKernelGGL((qkv_decode_kernel<1, 3, BF16, false, NR>), grid, dim3(256), 0, st, d); break;
    case 4: hipLaunchKernelGGL((qkv_decode_kernel<1, 4, BF16, false, NR>), grid, dim3(256), 0, st, d); break;
    case 5: hipLaunchKernelGGL((qkv_decode_kernel<1, 5, BF16, false, NR>), grid, dim3(256), 0, st, d); break;
    case 6: hipLaunchKernelGGL((qkv_decode_kernel<1, 6, BF16, false, NR>), grid, dim3(256), 0, st, d); break;
    case 7: hipLaunchKernelGGL((qkv_decode_kernel<1, 7, BF16, false, NR>), grid, dim3(256), 0, st, d); break;
    default: hipLaunchKernelGGL((qkv_decode_kernel<1, 8, BF16, false, NR>), grid, dim3(256), 0, st, d); break;
  }
}

template <int MT, bool BF16>
static void launch_stream(int ks, dim3 grid, const DecodeArgs& d, hipStream_t st) {
  constexpr bool RO = MT > 1;  // register-order partials from two 16-token blocks up
  if constexpr (MT == 1) {
    if (d.fold_rows == 1) { launch_stream_fold<1, BF16>(ks, grid, d, st); return; }
    if (d.fold_rows == 2) { launch_stream_fold<2, BF16>(ks, grid, d, st); return; }
    if (d.fold_rows == 4) { launch_stream_fold<4, BF16>(ks, grid, d, st); return; }
  }
  switch (ks) {
    case 1: hipLaunchKernelGGL((qkv_decode_kernel<MT, 1, BF16, RO>), grid, dim3(256), 0, st, d); break;
    case 2: hipLaunchKernelGGL((qkv_decode_kernel<MT, 2, BF16, RO>), grid, dim3(256), 0, st, d); break;
    case 3: hipLaunchKernelGGL((qkv_decode_kernel<MT, 3, BF16, RO>), grid, dim3(256), 0, st, d); break;
    case 4: hipLaunchKernelGGL((qkv_decode_kernel<MT, 4, BF16, RO>), grid, dim3(256), 0, st, d); break;
    case 5: hipLaunchKernelGGL((qkv_decode_kernel<MT, 5, BF16, RO>), grid, dim3(256), 0, st, d); break;
    case 6: hipLaunchKernelGGL((qkv_decode_kernel<MT, 6, BF16, RO>), grid, dim3(256), 0, st, d); break;
    case 7: hipLaunchKernelGGL((qkv_decode_kernel<MT, 7, BF16, RO>), grid, dim3(256), 0, st, d); break;
    default: hipLaunchKernelGGL((qkv_decode_kernel<MT, 8, BF16, RO>), grid, dim3(256), 0, st, d); break;
  }
}

template <bool BF16>
static void launch_decode(const QkvPlan& p, const SplitArgs& s, hipStream_t st,
                          const OperandFold* fold = nullptr) {
  if (p.stream) {
    DecodeArgs d{};
    d.a = s.a; d.w = s.w; d.m = s.m; d.n = s.n; d.k = s.k; d.lda = s.lda; d.ldw = s.ldw;
    d.part = s.part;
    if (fold) {
      d.gamma = fold->gamma; d.gamma_dt = fold->gamma_dt; d.mixed = fold->mixed ? 1 : 0; d.eps = fold->eps;
      d.fold_rows = fold->rows_per_wave;
      d.stats = fold->stats;
    }
    const dim3 grid(static_cast<unsigned>(cdiv(s.n, 128)), static_cast<unsigned>(p.splits));
    if (p.nch > 0 && d.stats) {
      if constexpr (BF16) {
        switch (p.mt) {
          case 2: hipLaunchKernelGGL((qkv_decode_loop_kernel<2, true, true>), grid, dim3(256), 0, st, d, p.nch); break;
          case 3: hipLaunchKernelGGL((qkv_decode_loop_kernel<3, true, true>), grid, dim3(256), 0, st, d, p.nch); break;
          default: hipLaunchKernelGGL((qkv_decode_loop_kernel<4, true, true>), grid, dim3(256), 0, st, d, p.nch); break;
        }
      }
      return;
    }
    if (p.nch > 0) {
      switch (p.mt) {
        case 2: hipLaunchKernelGGL((qkv_decode_loop_kernel<2, BF16>), grid, dim3(256), 0, st, d, p.nch); break;
        case 3: hipLaunchKernelGGL((qkv_decode_loop_kernel<3, BF16>), grid, dim3(256), 0, st, d, p.nch); break;
        default: hipLaunchKernelGGL((qkv_decode_loop_kernel<4, BF16>), grid, dim3(256), 0, st, d, p.nch); break;
      }
      return;
    }
    switch (p.mt) {
      case 1: launch_stream<1, BF16>(p.ks, grid, d, st); break;
      case 2: launch_stream<2, BF16>(p.ks, grid, d, st); break;
      case 3: launch_stream<3, BF16>(p.ks, grid, d, st); break;
      default: launch_stream<4, BF16>(p.ks, grid, d, st); break;
    }
    return;
  }
  if (p.cpw == 1) launch_decode_cpw<BF16, 1>(p, s, st);
  else launch_decode_cpw<BF16, 2>(p, s, st);
}

// Epilogue dtype form for a launch: the fixed forms cover bf16 operands on the
// DMA path; every other case keeps the run-time dtypes.
static bool edt_forced_rt() {
  return tuning(BFA_TUNE_EDT_RT) > 0;  // planner override: run-time dtypes only
}

static int fused_edt(const QkvEpi& e) {
  if (edt_forced_rt()) return EDT_RT;
  const bool norm = e.qn_w != nullptr || e.kn_w != nullptr;
  if (e.qkv_dt == BFA_DTYPE_F32 && e.out_dt == BFA_DTYPE_BF16 && !norm) return EDT_F32_BF16;
  if (e.qkv_dt == BFA_DTYPE_BF16 && e.out_dt == BFA_DTYPE_BF16 && (!norm || e.norm_dt == BFA_DTYPE_BF16))
    return EDT_BF16;
  return EDT_RT;
}

static int linear_edt(const QkvEpi& e) {
  if (edt_forced_rt()) return EDT_RT;
  return (e.qkv_dt == BFA_DTYPE_BF16 && e.mid_dt == BFA_DTYPE_BF16 && e.out_dt == BFA_DTYPE_BF16)
             ? EDT_BF16 : EDT_RT;
}

template <int BM, int BN, int WM, int NS, int BK, bool BF16, bool DIRECT, int HD>
static void launch_fused_edt(unsigned grid, dim3 block, int edt, const GemmArgs& g, const QkvEpi& e,
                             hipStream_t st) {
  if constexpr (BF16 && DIRECT && HD >= 64) {
    if (edt == EDT_F32_BF16) {
      hipLaunchKernelGGL((qkv_gemm_kernel<BM, BN, WM, 128, BF16, EPI_FUSED, HD, DIRECT, NS, BK, EDT_F32_BF16>),
                         dim3(grid), block, 0, st, g, e);
      return;
    }
    if (edt == EDT_BF16) {
      hipLaunchKernelGGL((qkv_gemm_kernel<BM, BN, WM, 128, BF16, EPI_FUSED, HD, DIRECT, NS, BK, EDT_BF16>),
                         dim3(grid), block, 0, st, g, e);
      return;
    }
  }
  hipLaunchKernelGGL((qkv_gemm_kernel<BM, BN, WM, 128, BF16, EPI_FUSED, HD, DIRECT, NS, BK>), dim3(grid),
                     block, 0, st, g, e);
}

// Workgroups of a prefill GEMM launch: one per tile, or for the 256x256 tile
// (one workgroup per CU, the kernel's PERSIST form) one per CU, each looping
// over tiles: the Llama-3-8B projection at 8192 tokens (768 tiles) took 380.5
// against 388.0 us on one box, with bit-identical output.  Planner override
// BFA_TUNE_QKV_PERSIST = c sets the workgroups per CU of the 256x256 tile
// (0: one per tile).
static unsigned persistent_grid(int64_t tiles, bool persist) {
  int per_cu = persist ? 1 : 0;
  const int c = tuning(BFA_TUNE_QKV_PERSIST);
  if (persist && c >= 0) per_cu = c;
  if (per_cu > 0) tiles = std::min<int64_t>(tiles, int64_t(256) * per_cu);
  return static_cast<unsigned>(tiles);
}

// BM x BN tile, waves of WM x 128 (the fused epilogue needs 128-column waves),
// BK-deep DMA stages (NS of them when BK = 32).
template <int BM, int BN, int WM, int NS, int BK, bool BF16, bool DIRECT>
static void launch_prefill_tile(const QkvPlan& p, const GemmArgs& g, const QkvEpi& e, hipStream_t st) {
  const unsigned grid = persistent_grid(cdiv(g.m, BM) * cdiv(g.n, BN), BM == 256 && BN == 256);
  const dim3 block((BM / WM) * (BN / 128) * 64);
  const int edt = fused_edt(e);
  if (!p.fused_epi) {
    hipLaunchKernelGGL((qkv_gemm_kernel<BM, BN, WM, 128, BF16, EPI_RAW, 128, DIRECT, NS, BK>), dim3(grid),
                       block, 0, st, g, e);
  } else if (e.hd == 128) {
    launch_fused_edt<BM, BN, WM, NS, BK, BF16, DIRECT, 128>(grid, block, edt, g, e, st);
  } else if (e.hd == 64) {
    launch_fused_edt<BM, BN, WM, NS, BK, BF16, DIRECT, 64>(grid, block, edt, g, e, st);
  } else {
    launch_fused_edt<BM, BN, WM, NS, BK, BF16, DIRECT, 32>(grid, block, edt, g, e, st);
  }
}

// 128x64 tile: four waves of 32x64, a ring of four 32-deep DMA stages, the
// fused epilogue with 8 lanes per row (head_dim 32 or 64).
template <bool BF16, int HD>
static void launch_prefill_narrow_hd(const GemmArgs& g, const QkvEpi& e, hipStream_t st) {
  const dim3 grid(static_cast<unsigned>(cdiv(g.m, 128) * cdiv(g.n, 64))), block(256);
  const int edt = fused_edt(e);
  if constexpr (BF16) {
    if (edt == EDT_F32_BF16) {
      hipLaunchKernelGGL((qkv_gemm_kernel<128, 64, 32, 64, BF16, EPI_FUSED, HD, true, 4, 32, EDT_F32_BF16>), grid,
                         block, 0, st, g, e);
      return;
    }
    if (edt == EDT_BF16) {
      hipLaunchKernelGGL((qkv_gemm_kernel<128, 64, 32, 64, BF16, EPI_FUSED, HD, true, 4, 32, EDT_BF16>), grid,
                         block, 0, st, g, e);
      return;
    }
  }
  hipLaunchKernelGGL((qkv_gemm_kernel<128, 64, 32, 64, BF16, EPI_FUSED, HD, true, 4, 32>), grid, block, 0, st, g, e);
}

// The linear fusions: same tiles, EPI_LINEAR or EPI_SWIGLU epilogue.
template <int BM, int BN, int WM, int NS, int BK, bool BF16, bool DIRECT>
static void launch_linear_tile(const GemmArgs& g, const QkvEpi& e, bool swiglu, hipStream_t st) {
  const int64_t bno = swiglu ? BN / 2 : BN;
  const unsigned grid = persistent_grid(cdiv(g.m, BM) * cdiv(g.n, bno), BM == 256 && BN == 256);
  const dim3 block((BM / WM) * (BN / 128) * 64);
  if constexpr (BF16 && DIRECT) {
    if (linear_edt(e) == EDT_BF16) {
      if (swiglu)
        hipLaunchKernelGGL((qkv_gemm_kernel<BM, BN, WM, 128, BF16, EPI_SWIGLU, 128, DIRECT, NS, BK, EDT_BF16>),
                           dim3(grid), block, 0, st, g, e);
      else
        hipLaunchKernelGGL((qkv_gemm_kernel<BM, BN, WM, 128, BF16, EPI_LINEAR, 128, DIRECT, NS, BK, EDT_BF16>),
                           dim3(grid), block, 0, st, g, e);
      return;
    }
  }
  if (swiglu) {
    hipLaunchKernelGGL((qkv_gemm_kernel<BM, BN, WM, 128, BF16, EPI_SWIGLU, 128, DIRECT, NS, BK>),
                       dim3(grid), block, 0, st, g, e);
  } else {
    hipLaunchKernelGGL((qkv_gemm_kernel<BM, BN, WM, 128, BF16, EPI_LINEAR, 128, DIRECT, NS, BK>),
                       dim3(grid), block, 0, st, g, e);
  }
}

template <bool BF16>
static void launch_linear(const QkvPlan& p, const GemmArgs& g, const QkvEpi& e, bool swiglu,
                          int64_t wrows, hipStream_t st) {
  const bool dma = g.k % 64 == 0 && g.lda % 8 == 0 && g.ldw % 8 == 0 && aligned16(g.a) &&
                   aligned16(g.w) && g.m * g.lda * 2 < (int64_t(1) << 32) &&
                   wrows * g.ldw * 2 < (int64_t(1) << 32);
  if (!dma) {
    launch_linear_tile<128, 128, 32, 2, 64, BF16, false>(g, e, swiglu, st);
    return;
  }
  switch (p.tile) {
    case 2: launch_linear_tile<256, 256, 64, 2, 64, BF16, true>(g, e, swiglu, st); break;
    case 3: launch_linear_tile<128, 256, 32, 2, 64, BF16, true>(g, e, swiglu, st); break;
    case 1: launch_linear_tile<128, 256, 64, 3, 32, BF16, true>(g, e, swiglu, st); break;
    default: launch_linear_tile<128, 128, 32, 4, 32, BF16, true>(g, e, swiglu, st); break;
  }
}

template <bool BF16, bool DIRECT>
static void launch_prefill_t(const QkvPlan& p, const GemmArgs& g, const QkvEpi& e, hipStream_t st) {
  if constexpr (DIRECT) {
    switch (p.tile) {
      case 2: launch_prefill_tile<256, 256, 64, 2, 64, BF16, true>(p, g, e, st); break;
      case 3: launch_prefill_tile<128, 256, 32, 2, 64, BF16, true>(p, g, e, st); break;
      case 1: launch_prefill_tile<128, 256, 64, 3, 32, BF16, true>(p, g, e, st); break;
      case 64:
        if (e.hd == 64) launch_prefill_narrow_hd<BF16, 64>(g, e, st);
        else launch_prefill_narrow_hd<BF16, 32>(g, e, st);
        break;
      default: launch_prefill_tile<128, 128, 32, 4, 32, BF16, true>(p, g, e, st); break;
    }
  } else {
    // the register-staged path (256 threads, K not a multiple of 64 or
    // unaligned rows) uses 128x128 tiles
    launch_prefill_tile<128, 128, 32, 2, 64, BF16, false>(p, g, e, st);
  }
}

template <bool BF16>
static void launch_prefill(const QkvPlan& p, const GemmArgs& g, const QkvEpi& e, hipStream_t st) {
  const bool dma = g.k % 64 == 0 && g.lda % 8 == 0 && g.ldw % 8 == 0 && aligned16(g.a) &&
                   aligned16(g.w) && g.m * g.lda * 2 < (int64_t(1) << 32) &&
                   g.n * g.ldw * 2 < (int64_t(1) << 32);
  if (dma) launch_prefill_t<BF16, true>(p, g, e, st);
  else launch_prefill_t<BF16, false>(p, g, e, st);
}

// Whole-K column-pair decode kernel (qkv_decode_pair_kernel): 17-64 tokens,
// bf16 operand and weight, head_dim a multiple of 32, no q/k norm, K a multiple
// of 256, and at least 128 column tiles, so that the weight stream still covers
// most CUs.  Override BFA_TUNE_DECODE_PAIR = 0 keeps the split-K kernels, = 1
// drops the tile minimum (measurements and tests).
static bool pair_ok(const QkvPlan& p, int64_t n, int64_t hd, int64_t k, bool qk_norm, bool bf16,
                    int64_t lda, const void* operand, int64_t m, int64_t ldw) {
  if (!p.decode || !p.stream || p.mt < 2 || !bf16 || qk_norm) return false;
  if (hd % 32 != 0 || n % 32 != 0 || k % 256 != 0) return false;
  // 32-bit DMA offsets for the operand and weight rows
  if (lda % 8 != 0 || !aligned16(operand) || m * lda * 2 >= (int64_t(1) << 32) ||
      n * ldw * 2 >= (int64_t(1) << 32))
    return false;
  const int mode = tuning(BFA_TUNE_DECODE_PAIR);
  if (mode == 0) return false;
  return mode == 1 || n / 32 >= 128;
}

// epilogue dtype forms of the pair kernel (no q/k norm): the scale-after form is
// an fp32 projection, so it has the Llama chain's form or the run-time one
template <int MT>
static void launch_pair_mt(bool sa, int edt, dim3 grid, const DecodeArgs& d, const QkvEpi& e, int nch,
                           hipStream_t st) {
  if (sa) {
    // no gamma: the weight has it folded in
    const bool gin = d.gamma != nullptr;
    if (edt == EDT_F32_BF16) {
      if (gin) hipLaunchKernelGGL((qkv_decode_pair_kernel<MT, true, EDT_F32_BF16>), grid, dim3(256), 0, st, d, e, nch);
      else hipLaunchKernelGGL((qkv_decode_pair_kernel<MT, true, EDT_F32_BF16, false>), grid, dim3(256), 0, st, d, e, nch);
    } else {
      if (gin) hipLaunchKernelGGL((qkv_decode_pair_kernel<MT, true, EDT_RT>), grid, dim3(256), 0, st, d, e, nch);
      else hipLaunchKernelGGL((qkv_decode_pair_kernel<MT, true, EDT_RT, false>), grid, dim3(256), 0, st, d, e, nch);
    }
    return;
  }
  if (edt == EDT_F32_BF16)
    hipLaunchKernelGGL((qkv_decode_pair_kernel<MT, false, EDT_F32_BF16>), grid, dim3(256), 0, st, d, e, nch);
  else if (edt == EDT_BF16)
    hipLaunchKernelGGL((qkv_decode_pair_kernel<MT, false, EDT_BF16>), grid, dim3(256), 0, st, d, e, nch);
  else
    hipLaunchKernelGGL((qkv_decode_pair_kernel<MT, false, EDT_RT>), grid, dim3(256), 0, st, d, e, nch);
}

static void launch_pair(const QkvPlan& p, const DecodeArgs& d, const QkvEpi& e, bool sa, hipStream_t st) {
  const dim3 grid(static_cast<unsigned>(d.n / 32));
  const int nch = static_cast<int>(d.k / 256);
  const int edt = fused_edt(e);
  switch (p.mt) {
    case 2: launch_pair_mt<2>(sa, edt, grid, d, e, nch, st); break;
    case 3: launch_pair_mt<3>(sa, edt, grid, d, e, nch, st); break;
    default: launch_pair_mt<4>(sa, edt, grid, d, e, nch, st); break;
  }
}

static void launch_epilogue(const float* part, int64_t splits, int64_t m, const QkvEpi& e,
                            hipStream_t st) {
  const int64_t items = m * (e.hq + 2 * e.hkv);
  const dim3 grid(static_cast<unsigned>(cdiv(items, 4)));
  if (e.hd <= 128) hipLaunchKernelGGL(qkv_epilogue_kernel<1>, grid, dim3(256), 0, st, part, splits, m, e);
  else if (e.hd <= 256) hipLaunchKernelGGL(qkv_epilogue_kernel<2>, grid, dim3(256), 0, st, part, splits, m, e);
  else hipLaunchKernelGGL(qkv_epilogue_kernel<4>, grid, dim3(256), 0, st, part, splits, m, e);
}

}  // namespace bfa

using namespace bfa;

extern "C" int64_t bfa_fused_rmsnorm_qkv_workspace_size(int64_t tokens, int64_t hidden,
                                                        int64_t qkv_dim, int64_t head_dim) {
  if (tokens <= 0) return 0;
  const QkvPlan p = make_plan(tokens, qkv_dim, hidden, head_dim);
  return p.operand_bytes + p.part_bytes;
}

// Host side of the fused KV append's QkvEpi fields.
struct CacheEpi {
  void* cache;
  int cache_dt;
  int64_t c_skv, c_sh;
  const int64_t* slot_off;  // resolved slots (decode and raw-epilogue paths)
  int skip_kv_out;
  const AppendArgs* app;    // the prefill GEMM's fused epilogue resolves its own
};

// The projection with its epilogue; `operand` rows are `lda` apart.  With a
// fold (decode, one to four tokens) `operand` is the raw input x and the decode
// kernel normalises it itself.
static int qkv_projection_impl(const void* operand, int64_t lda, const OperandFold* fold,
                               int64_t tokens, int64_t hidden,
                               const void* qkv_weight, int w_dtype, int64_t qkv_dim,
                                  int64_t w_stride, const void* bias, int bias_dtype,
                                  int64_t num_q_heads, int64_t num_kv_heads, int qkv_dtype,
                                  const void* q_norm_weight, const void* k_norm_weight,
                                  int qk_norm_dtype, float qk_eps, int qk_norm_out_dtype,
                                  const void* positions, int positions_dtype,
                                  const float* cos_sin_cache, int64_t max_position, void* out,
                                  int out_dtype, int64_t out_stride, void* part_workspace,
                                  int64_t part_workspace_bytes, int32_t* status, void* stream,
                                  const CacheEpi* ce = nullptr, const float* row_scale = nullptr) {
  const char* what = fold ? "bfa_fused_rmsnorm_qkv" : "bfa_qkv_projection";
  BFA_REQUIRE(w_dtype == BFA_DTYPE_BF16 || w_dtype == BFA_DTYPE_F16, "%s: weight must be bf16/fp16", what);
  BFA_REQUIRE(is_float_dtype(qkv_dtype) && is_float_dtype(out_dtype) && is_float_dtype(qk_norm_out_dtype),
              "%s: bad dtype", what);
  BFA_REQUIRE(tokens >= 0 && hidden > 0 && qkv_dim > 0 && num_q_heads > 0 && num_kv_heads > 0,
              "%s: bad geometry", what);
  const int64_t heads = num_q_heads + 2 * num_kv_heads;
  BFA_REQUIRE(qkv_dim % heads == 0, "%s: qkv_dim %lld not divisible by %lld heads", what,
              (long long)qkv_dim, (long long)heads);
  const int64_t hd = qkv_dim / heads;
  BFA_REQUIRE(hidden % 16 == 0, "%s: hidden must be a multiple of 16 (got %lld)", what, (long long)hidden);
  BFA_REQUIRE(w_stride >= hidden, "%s: weight row stride %lld < hidden %lld", what,
              (long long)w_stride, (long long)hidden);
  BFA_REQUIRE(w_stride % 8 == 0 && aligned16(qkv_weight) && aligned16(operand),
              "%s: operand/weight rows must be 16-byte aligned", what);
  BFA_REQUIRE(cos_sin_cache == nullptr || (positions && (positions_dtype == BFA_DTYPE_I64 ||
                                                         positions_dtype == BFA_DTYPE_I32)),
              "%s: RoPE needs int32/int64 positions", what);
  BFA_REQUIRE(cos_sin_cache == nullptr || hd % 2 == 0, "%s: RoPE needs an even head_dim", what);
  BFA_REQUIRE(cos_sin_cache == nullptr || (max_position > 0 && max_position <= 0x7fffffffLL),
              "%s: RoPE table length %lld out of range", what, (long long)max_position);
  BFA_REQUIRE(hd <= 512, "%s: head_dim %lld > 512 unsupported", what, (long long)hd);
  if (tokens == 0) return BFA_OK;
  BFA_REQUIRE(out, "%s: null output", what);

  const QkvPlan p = make_plan(tokens, qkv_dim, hidden, hd);
  BFA_REQUIRE(p.decode || !p.fused_epi || (out_stride % 4 == 0 && aligned16(out)),
              "%s: output rows must be 16-byte aligned", what);
  BFA_REQUIRE(row_scale == nullptr || (!p.decode && p.fused_epi), "%s: row scales need the prefill epilogue",
              what);
  BFA_REQUIRE(part_workspace_bytes >= p.part_bytes && (p.part_bytes == 0 || part_workspace),
              "%s: workspace too small (%lld < %lld bytes)", what, (long long)part_workspace_bytes,
              (long long)p.part_bytes);
  BFA_REQUIRE(p.part_bytes == 0 || aligned16(part_workspace), "%s: workspace must be 16-byte aligned",
              what);

  QkvEpi e{};
  e.bias = bias; e.bias_dtype = bias_dtype;
  e.qkv_dt = qkv_dtype; e.norm_dt = qk_norm_out_dtype; e.out_dt = out_dtype;
  e.n = qkv_dim; e.hq = num_q_heads; e.hkv = num_kv_heads; e.hd = hd;
  e.qn_w = q_norm_weight; e.kn_w = k_norm_weight; e.qk_w_dtype = qk_norm_dtype; e.qk_eps = qk_eps;
  e.positions = positions; e.pos_is_i64 = positions_dtype == BFA_DTYPE_I64;
  e.cs = cos_sin_cache; e.max_pos = max_position;
  e.out = out; e.ldo = out_stride; e.status = status;
  e.row_scale = row_scale;
  if (fold && fold->stats) {
    e.stats = fold->stats; e.stat_rows = 16 * p.mt; e.hidden = hidden; e.stat_eps = fold->eps;
  }
  if (ce) {
    e.cache = ce->cache; e.cache_dt = ce->cache_dt; e.c_skv = ce->c_skv; e.c_sh = ce->c_sh;
    e.slot_off = ce->slot_off; e.skip_kv_out = ce->skip_kv_out;
    if (!p.decode && p.fused_epi) {
      e.app_in_kernel = 1;
      e.app = *ce->app;
    } else {
      BFA_REQUIRE(ce->slot_off != nullptr, "%s: cache slots not resolved", what);
    }
  }

  const hipStream_t st = as_stream(stream);
  const bool bf16 = w_dtype == BFA_DTYPE_BF16;
  float* part = static_cast<float*>(part_workspace);
  // 1 to 8 tokens: one launch (no split-K partials); the fold's operand must be
  // bf16 like the weight, and the scale-after form is not used
  if (p.decode && !(fold && fold->stats) &&
      gemv_ok(tokens, hidden, qkv_dim, hd, q_norm_weight || k_norm_weight, bias, bf16, true, operand, lda)) {
    GemvArgs d{};
    d.a = static_cast<const uint16_t*>(operand);
    d.w = static_cast<const uint16_t*>(qkv_weight);
    d.m = tokens; d.k = hidden; d.lda = lda; d.ldw = w_stride;
    if (fold) {
      d.gamma = fold->gamma; d.gamma_dt = fold->gamma_dt; d.mixed = fold->mixed ? 1 : 0; d.eps = fold->eps;
    }
    e.stats = nullptr;
    launch_qkv_gemv(d, fold != nullptr, e, st);
    return check_launch(what);
  }
  if (p.decode && pair_ok(p, qkv_dim, hd, hidden, q_norm_weight || k_norm_weight, bf16, lda, operand, tokens,
                         w_stride)) {
    DecodeArgs d{};
    d.a = static_cast<const uint16_t*>(operand);
    d.w = static_cast<const uint16_t*>(qkv_weight);
    d.m = tokens; d.n = qkv_dim; d.k = hidden; d.lda = lda; d.ldw = w_stride;
    const bool sa = fold && fold->stats;
    if (sa) {
      // a null gamma: folded into the weight already
      BFA_REQUIRE(!fold->gamma || (fold->gamma_dt == BFA_DTYPE_BF16 && aligned16(fold->gamma)),
                  "%s: scale-after needs a 16-byte aligned bf16 norm weight", what);
      d.gamma = fold->gamma; d.gamma_dt = fold->gamma_dt; d.eps = fold->eps;
    }
    e.stats = nullptr;
    launch_pair(p, d, e, sa, st);
    return check_launch(what);
  }
  // the scale-after fold outside the pair kernel is the deep-K kernel's (with
  // its gamma: a folded weight has only the pair kernel)
  BFA_REQUIRE(!(fold && fold->stats) || (p.decode && p.nch > 0 && fold->gamma),
              "%s: scale-after fold without a kernel", what);
  if (p.decode) {
    SplitArgs s{};
    s.a = static_cast<const uint16_t*>(operand);
    s.w = static_cast<const uint16_t*>(qkv_weight);
    s.m = tokens; s.n = qkv_dim; s.k = hidden; s.lda = lda; s.ldw = w_stride;
    s.kchunk = p.kchunk; s.part = part;
    if (bf16) launch_decode<true>(p, s, st, fold); else launch_decode<false>(p, s, st, fold);
    int rc = check_launch(what);
    if (rc != BFA_OK) return rc;
    if (p.stream && p.mt > 1) {
      const int64_t items = cdiv(tokens, 4) * heads;
      const dim3 grid(static_cast<unsigned>(cdiv(items, 4)));
      const float4* p4 = reinterpret_cast<const float4*>(part);
      if (hd <= 128) {
        hipLaunchKernelGGL(qkv_decode_epilogue_kernel<1>, grid, dim3(256), 0, st, p4, p.splits,
                           cdiv(qkv_dim, 128), p.mt, tokens, e);
      } else if (hd <= 256) {
        hipLaunchKernelGGL(qkv_decode_epilogue_kernel<2>, grid, dim3(256), 0, st, p4, p.splits,
                           cdiv(qkv_dim, 128), p.mt, tokens, e);
      } else {
        hipLaunchKernelGGL(qkv_decode_epilogue_kernel<4>, grid, dim3(256), 0, st, p4, p.splits,
                           cdiv(qkv_dim, 128), p.mt, tokens, e);
      }
    } else {
      launch_epilogue(part, p.splits, tokens, e, st);
    }
    return check_launch(what);
  }
  GemmArgs g{};
  g.a = static_cast<const uint16_t*>(operand);
  g.w = static_cast<const uint16_t*>(qkv_weight);
  g.m = tokens; g.n = qkv_dim; g.k = hidden; g.lda = lda; g.ldw = w_stride;
  g.raw = part;
  if (bf16) launch_prefill<true>(p, g, e, st); else launch_prefill<false>(p, g, e, st);
  int rc = check_launch(what);
  if (rc != BFA_OK || p.fused_epi) return rc;
  launch_epilogue(part, 1, tokens, e, st);
  return check_launch(what);
}

extern "C" int bfa_qkv_projection(const void* operand, int64_t tokens, int64_t hidden,
                                  const void* qkv_weight, int w_dtype, int64_t qkv_dim,
                                  int64_t w_stride, const void* bias, int bias_dtype,
                                  int64_t num_q_heads, int64_t num_kv_heads, int qkv_dtype,
                                  const void* q_norm_weight, const void* k_norm_weight,
                                  int qk_norm_dtype, float qk_eps, int qk_norm_out_dtype,
                                  const void* positions, int positions_dtype,
                                  const float* cos_sin_cache, int64_t max_position, void* out,
                                  int out_dtype, int64_t out_stride, void* part_workspace,
                                  int64_t part_workspace_bytes, int32_t* status, void* stream) {
  return qkv_projection_impl(operand, hidden, nullptr, tokens, hidden, qkv_weight, w_dtype, qkv_dim,
                             w_stride, bias, bias_dtype, num_q_heads, num_kv_heads, qkv_dtype,
                             q_norm_weight, k_norm_weight, qk_norm_dtype, qk_eps, qk_norm_out_dtype,
                             positions, positions_dtype, cos_sin_cache, max_position, out, out_dtype,
                             out_stride, part_workspace, part_workspace_bytes, status, stream);
}

static int fused_impl(const void* x, int x_dtype, int64_t tokens, int64_t hidden, int64_t x_stride,
                      const void* norm_weight, int nw_dtype, float eps, int mixed_rounding,
                      const void* qkv_weight, int w_dtype, int64_t qkv_dim, int64_t w_stride,
                      const void* bias, int bias_dtype, int64_t num_q_heads, int64_t num_kv_heads,
                      int qkv_dtype, const void* q_norm_weight, const void* k_norm_weight,
                      int qk_norm_dtype, float qk_eps, int qk_norm_out_dtype, const void* positions,
                      int positions_dtype, const float* cos_sin_cache, int64_t max_position, void* out,
                      int out_dtype, int64_t out_stride, void* workspace, int64_t workspace_bytes,
                      int32_t* status, void* stream, const CacheEpi* ce) {
  const char* what = "bfa_fused_rmsnorm_qkv";
  BFA_REQUIRE(x && norm_weight && qkv_weight, "%s: null pointer", what);
  if (tokens == 0) return BFA_OK;
  const int64_t heads = num_q_heads + 2 * num_kv_heads;
  BFA_REQUIRE(heads > 0 && qkv_dim % heads == 0, "%s: bad head geometry", what);
  const QkvPlan p = make_plan(tokens, qkv_dim, hidden, qkv_dim / heads);
  BFA_REQUIRE(workspace && workspace_bytes >= p.operand_bytes + p.part_bytes && aligned16(workspace),
              "%s: workspace too small (%lld < %lld bytes)", what, (long long)workspace_bytes,
              (long long)(p.operand_bytes + p.part_bytes));
  char* ws = static_cast<char*>(workspace);
  // Up to 16 decode tokens whose x is already in the weight dtype: the
  // weight-streaming kernel normalises its own K slice, one launch fewer.  One
  // row per wave up to 4 tokens (hidden <= 4096), two up to 8 (hidden <= 2048),
  // four up to 16 (hidden <= 1024); beyond that the reads of the rows cost more
  // than the launch (TinyLlama, 16 tokens: 11.2 against 10.1 us with the
  // pre-pass).  Override BFA_TUNE_NO_OPERAND_FOLD > 0 keeps the pre-pass.
  const bool no_fold = tuning(BFA_TUNE_NO_OPERAND_FOLD) > 0;
  const int fold_rows = (tokens <= 4 && hidden <= 4096) ? 1
                        : (tokens <= 8 && hidden <= 2048) ? 2
                        : (tokens <= 16 && hidden <= 1024) ? 4 : 0;
  // 1 to 8 tokens in bf16 without q/k norm (the one-launch kernel,
  // qkv_gemv.hip) always fold: it normalises the rows into LDS itself.
  const bool gemv_fold = !no_fold && p.decode && x_dtype == BFA_DTYPE_BF16 && w_dtype == BFA_DTYPE_BF16 &&
                         aligned16(norm_weight) && is_float_dtype(nw_dtype) &&
                         gemv_ok(tokens, hidden, qkv_dim, qkv_dim / heads, q_norm_weight || k_norm_weight, bias,
                                 true, true, x, x_stride);
  const bool fold = gemv_fold ||
                    (!no_fold && fold_rows > 0 && p.decode && p.stream && p.mt == 1 && x_dtype == w_dtype &&
                     (w_dtype == BFA_DTYPE_BF16 || w_dtype == BFA_DTYPE_F16) && hidden % 8 == 0 &&
                     x_stride % 8 == 0 && aligned16(x) && aligned16(norm_weight) && is_float_dtype(nw_dtype));
  // 17 to 64 decode tokens of the fp32 variants (operand (x / rms) * gamma): the
  // row scale 1 / rms comes out of the sum, so no operand pre-pass.  The
  // column-pair kernel projects x onto bf16(w * gamma) and sums the rows'
  // squares itself; the deep-K kernel projects bf16(x * gamma), returns each
  // split's sums of x^2 and the reduction kernel applies 1 / rms.  bf16 only:
  // x * gamma without the row scale could leave the fp16 range.
  const bool pair = pair_ok(p, qkv_dim, qkv_dim / heads, hidden, q_norm_weight || k_norm_weight,
                            x_dtype == BFA_DTYPE_BF16 && w_dtype == BFA_DTYPE_BF16, x_stride, x, tokens, w_stride);
  const bool scale_after = !no_fold && p.decode && p.stream && mixed_rounding == 0 &&
                           qkv_dtype == BFA_DTYPE_F32 && x_dtype == BFA_DTYPE_BF16 &&
                           w_dtype == BFA_DTYPE_BF16 && nw_dtype == BFA_DTYPE_BF16 && hidden % 8 == 0 &&
                           x_stride % 8 == 0 && aligned16(x) && aligned16(norm_weight) &&
                           (pair || (p.nch > 0 && p.splits * 16 * p.mt * 4 <= p.operand_bytes));
  if (scale_after) {
    const OperandFold f{norm_weight, nw_dtype, false, eps, 0, reinterpret_cast<float*>(ws)};
    return qkv_projection_impl(x, x_stride, &f, tokens, hidden, qkv_weight, w_dtype, qkv_dim, w_stride,
                               bias, bias_dtype, num_q_heads, num_kv_heads, qkv_dtype, q_norm_weight,
                               k_norm_weight, qk_norm_dtype, qk_eps, qk_norm_out_dtype, positions,
                               positions_dtype, cos_sin_cache, max_position, out, out_dtype, out_stride,
                               ws + p.operand_bytes, workspace_bytes - p.operand_bytes, status, stream, ce);
  }
  if (fold) {
    const OperandFold f{norm_weight, nw_dtype, mixed_rounding != 0, eps, fold_rows, nullptr};
    return qkv_projection_impl(x, x_stride, &f, tokens, hidden, qkv_weight, w_dtype, qkv_dim, w_stride,
                               bias, bias_dtype, num_q_heads, num_kv_heads, qkv_dtype, q_norm_weight,
                               k_norm_weight, qk_norm_dtype, qk_eps, qk_norm_out_dtype, positions,
                               positions_dtype, cos_sin_cache, max_position, out, out_dtype, out_stride,
                               ws + p.operand_bytes, workspace_bytes - p.operand_bytes, status, stream, ce);
  }
  int rc = launch_qkv_operand(x, x_dtype, tokens, hidden, x_stride, norm_weight, nw_dtype,
                              mixed_rounding != 0, ws, w_dtype, eps, as_stream(stream));
  if (rc != BFA_OK) return rc;
  return qkv_projection_impl(ws, hidden, nullptr, tokens, hidden, qkv_weight, w_dtype, qkv_dim, w_stride,
                             bias, bias_dtype, num_q_heads, num_kv_heads, qkv_dtype, q_norm_weight,
                             k_norm_weight, qk_norm_dtype, qk_eps, qk_norm_out_dtype, positions,
                             positions_dtype, cos_sin_cache, max_position, out, out_dtype, out_stride,
                             ws + p.operand_bytes, workspace_bytes - p.operand_bytes, status, stream, ce);
}

extern "C" int bfa_fused_rmsnorm_qkv(const void* x, int x_dtype, int64_t tokens, int64_t hidden,
                                     int64_t x_stride, const void* norm_weight, int nw_dtype,
                                     float eps, int mixed_rounding, const void* qkv_weight,
                                     int w_dtype, int64_t qkv_dim, int64_t w_stride,
                                     const void* bias, int bias_dtype, int64_t num_q_heads,
                                     int64_t num_kv_heads, int qkv_dtype,
                                     const void* q_norm_weight, const void* k_norm_weight,
                                     int qk_norm_dtype, float qk_eps, int qk_norm_out_dtype,
                                     const void* positions, int positions_dtype,
                                     const float* cos_sin_cache, int64_t max_position, void* out,
                                     int out_dtype, int64_t out_stride, void* workspace,
                                     int64_t workspace_bytes, int32_t* status, void* stream) {
  return fused_impl(x, x_dtype, tokens, hidden, x_stride, norm_weight, nw_dtype, eps, mixed_rounding,
                    qkv_weight, w_dtype, qkv_dim, w_stride, bias, bias_dtype, num_q_heads, num_kv_heads,
                    qkv_dtype, q_norm_weight, k_norm_weight, qk_norm_dtype, qk_eps, qk_norm_out_dtype,
                    positions, positions_dtype, cos_sin_cache, max_position, out, out_dtype, out_stride,
                    workspace, workspace_bytes, status, stream, nullptr);
}

// ------------------------------------------------ fused QKV + paged KV append
// bfa_fused_rmsnorm_qkv, then bfa_append_paged_kv of its k and v heads (as
// [tokens, num_kv_heads, head_dim] views of `out`), in the projection's own
// epilogue: a small kernel first resolves every token's cache slot into the
// workspace tail (tokens x 8 bytes), then each epilogue writes the finished k/v
// head rows to the cache as well (and, with write_kv_out = 0, only there).
extern "C" int64_t bfa_fused_rmsnorm_qkv_append_workspace_size(int64_t tokens, int64_t hidden,
                                                               int64_t qkv_dim, int64_t head_dim) {
  if (tokens <= 0) return 0;
  return bfa_fused_rmsnorm_qkv_workspace_size(tokens, hidden, qkv_dim, head_dim) + align256(tokens * 8);
}

// The cache arguments of the fused append, checked and gathered into `a`.
static int append_setup(const char* what, void* layer_cache, int cache_dtype, int64_t num_pages,
                        int64_t cache_page_slots, int64_t stride_page, int64_t stride_kv, int64_t stride_head,
                        int64_t stride_slot, const void* kv_indices, int kv_indices_dtype, int64_t num_indices,
                        const int32_t* kv_indptr, const void* batch_indices, int batch_indices_dtype,
                        int64_t num_seqs, const void* cache_positions, int cache_positions_dtype,
                        int64_t page_size, int64_t tokens, int32_t* status, AppendArgs* a) {
  int rc = fill_append_args(what, layer_cache, cache_dtype, num_pages, cache_page_slots, stride_page,
                            stride_kv, stride_head, stride_slot, kv_indices, kv_indices_dtype, num_indices,
                            kv_indptr, batch_indices, batch_indices_dtype, num_seqs, cache_positions,
                            cache_positions_dtype, page_size, status, a);
  if (rc != BFA_OK) return rc;
  BFA_REQUIRE(tokens >= 0 && tokens < (int64_t{1} << 31), "%s: bad token count", what);
  if (tokens == 0) return BFA_OK;
  BFA_REQUIRE(layer_cache && cache_positions, "%s: null cache or positions", what);
  BFA_REQUIRE(num_indices == 0 || kv_indices, "%s: null kv_indices", what);
  // the prefill epilogue writes 4 consecutive elements per store
  BFA_REQUIRE(stride_page % 4 == 0 && stride_kv % 4 == 0 && stride_head % 4 == 0 && stride_slot % 4 == 0 &&
                  aligned16(layer_cache),
              "%s: cache strides must be multiples of 4 elements and the cache 16-byte aligned", what);
  return BFA_OK;
}

extern "C" int bfa_fused_rmsnorm_qkv_append(
    const void* x, int x_dtype, int64_t tokens, int64_t hidden, int64_t x_stride, const void* norm_weight,
    int nw_dtype, float eps, int mixed_rounding, const void* qkv_weight, int w_dtype, int64_t qkv_dim,
    int64_t w_stride, const void* bias, int bias_dtype, int64_t num_q_heads, int64_t num_kv_heads,
    int qkv_dtype, const void* q_norm_weight, const void* k_norm_weight, int qk_norm_dtype, float qk_eps,
    int qk_norm_out_dtype, const void* positions, int positions_dtype, const float* cos_sin_cache,
    int64_t max_position, void* out, int out_dtype, int64_t out_stride, void* workspace,
    int64_t workspace_bytes, void* layer_cache, int cache_dtype, int64_t num_pages,
    int64_t cache_page_slots, int64_t stride_page, int64_t stride_kv, int64_t stride_head,
    int64_t stride_slot, const void* kv_indices, int kv_indices_dtype, int64_t num_indices,
    const int32_t* kv_indptr, const void* batch_indices, int batch_indices_dtype, int64_t num_seqs,
    const void* cache_positions, int cache_positions_dtype, int64_t page_size, int write_kv_out,
    int32_t* status, void* stream) {
  const char* what = "bfa_fused_rmsnorm_qkv_append";
  AppendArgs a{};
  int rc = append_setup(what, layer_cache, cache_dtype, num_pages, cache_page_slots, stride_page, stride_kv,
                        stride_head, stride_slot, kv_indices, kv_indices_dtype, num_indices, kv_indptr,
                        batch_indices, batch_indices_dtype, num_seqs, cache_positions, cache_positions_dtype,
                        page_size, tokens, status, &a);
  if (rc != BFA_OK || tokens == 0) return rc;
  const int64_t heads = num_q_heads + 2 * num_kv_heads;
  BFA_REQUIRE(heads > 0 && qkv_dim % heads == 0, "%s: bad head geometry", what);
  const int64_t fsize = bfa_fused_rmsnorm_qkv_workspace_size(tokens, hidden, qkv_dim, qkv_dim / heads);
  BFA_REQUIRE(workspace && aligned16(workspace) && workspace_bytes >= fsize + align256(tokens * 8),
              "%s: workspace too small (%lld < %lld bytes)", what, (long long)workspace_bytes,
              (long long)(fsize + align256(tokens * 8)));
  // the prefill GEMM with the fused epilogue resolves the slots itself; every
  // other path reads them from the workspace tail, filled by a small kernel
  const QkvPlan p = make_plan(tokens, qkv_dim, hidden, qkv_dim / heads);
  int64_t* slot_off = nullptr;
  if (p.decode || !p.fused_epi) {
    slot_off = reinterpret_cast<int64_t*>(static_cast<char*>(workspace) + fsize);
    launch_kv_slots(a, tokens, slot_off, as_stream(stream));
    rc = check_launch(what);
    if (rc != BFA_OK) return rc;
  }
  const CacheEpi ce{layer_cache, cache_dtype, stride_kv, stride_head, slot_off, write_kv_out ? 0 : 1, &a};
  return fused_impl(x, x_dtype, tokens, hidden, x_stride, norm_weight, nw_dtype, eps, mixed_rounding,
                    qkv_weight, w_dtype, qkv_dim, w_stride, bias, bias_dtype, num_q_heads, num_kv_heads,
                    qkv_dtype, q_norm_weight, k_norm_weight, qk_norm_dtype, qk_eps, qk_norm_out_dtype,
                    positions, positions_dtype, cos_sin_cache, max_position, out, out_dtype, out_stride,
                    workspace, fsize, status, stream, &ce);
}

// The fp32 variants' prefill with the norm weight folded into the QKV weight
// (bfa_fold_rmsnorm_weight): the row statistic 1 / rms goes to the workspace,
// then x itself is projected onto bf16(W * gamma) and each row's projection is
// multiplied by its statistic before the bias; the rest of the epilogue, and
// with a cache the append, are bfa_fused_rmsnorm_qkv(_append)'s.  No
// normalised operand is written.  layer_cache = NULL: no append (the other
// cache arguments are not read).
extern "C" int bfa_fused_rmsnorm_qkv_folded(
    const void* x, int x_dtype, int64_t tokens, int64_t hidden, int64_t x_stride, float eps,
    const void* folded_weight, int w_dtype, int64_t qkv_dim, int64_t w_stride, const void* bias, int bias_dtype,
    int64_t num_q_heads, int64_t num_kv_heads, int qkv_dtype, const void* positions, int positions_dtype,
    const float* cos_sin_cache, int64_t max_position, void* out, int out_dtype, int64_t out_stride,
    void* workspace, int64_t workspace_bytes, void* layer_cache, int cache_dtype, int64_t num_pages,
    int64_t cache_page_slots, int64_t stride_page, int64_t stride_kv, int64_t stride_head, int64_t stride_slot,
    const void* kv_indices, int kv_indices_dtype, int64_t num_indices, const int32_t* kv_indptr,
    const void* batch_indices, int batch_indices_dtype, int64_t num_seqs, const void* cache_positions,
    int cache_positions_dtype, int64_t page_size, int write_kv_out, int32_t* status, void* stream) {
  const char* what = "bfa_fused_rmsnorm_qkv_folded";
  BFA_REQUIRE(x && folded_weight, "%s: null pointer", what);
  AppendArgs a{};
  if (layer_cache) {
    const int rc = append_setup(what, layer_cache, cache_dtype, num_pages, cache_page_slots, stride_page,
                                stride_kv, stride_head, stride_slot, kv_indices, kv_indices_dtype, num_indices,
                                kv_indptr, batch_indices, batch_indices_dtype, num_seqs, cache_positions,
                                cache_positions_dtype, page_size, tokens, status, &a);
    if (rc != BFA_OK) return rc;
  }
  if (tokens == 0) return BFA_OK;
  BFA_REQUIRE(x_dtype == w_dtype, "%s: x must have the weight's dtype", what);
  BFA_REQUIRE(x_stride >= hidden && x_stride % 8 == 0, "%s: x rows must be 16-byte aligned", what);
  const int64_t heads = num_q_heads + 2 * num_kv_heads;
  BFA_REQUIRE(heads > 0 && qkv_dim % heads == 0, "%s: bad head geometry", what);
  const int64_t hd = qkv_dim / heads;
  const QkvPlan p = make_plan(tokens, qkv_dim, hidden, hd);
  // decode: the column-pair kernel on x, its row statistic from the Gram
  // diagonal (the scale-after form without the gamma conversion)
  const bool pair = p.decode && x_dtype == BFA_DTYPE_BF16 && aligned16(x) &&
                    pair_ok(p, qkv_dim, hd, hidden, false, true, x_stride, x, tokens, w_stride);
  if (!pair && (p.decode || !p.fused_epi))
    return set_error(BFA_ERR_UNSUPPORTED,
                     "%s: the prefill epilogue (more than 64 tokens, head_dim 32, 64 or 128) or the "
                     "column-pair decode shapes (17-64 bf16 tokens) only", what);
  const int64_t fsize = p.operand_bytes + p.part_bytes;
  const int64_t need = fsize + (layer_cache && p.decode ? align256(tokens * 8) : 0);
  BFA_REQUIRE(workspace && workspace_bytes >= need && aligned16(workspace),
              "%s: workspace too small (%lld < %lld bytes)", what, (long long)workspace_bytes, (long long)need);
  char* ws = static_cast<char*>(workspace);
  if (pair) {
    int64_t* slot_off = nullptr;
    if (layer_cache) {
      slot_off = reinterpret_cast<int64_t*>(ws + fsize);
      launch_kv_slots(a, tokens, slot_off, as_stream(stream));
      const int rc = check_launch(what);
      if (rc != BFA_OK) return rc;
    }
    const CacheEpi ce{layer_cache, cache_dtype, stride_kv, stride_head, slot_off, write_kv_out ? 0 : 1, &a};
    const OperandFold f{nullptr, BFA_DTYPE_BF16, false, eps, 0, reinterpret_cast<float*>(ws)};
    return qkv_projection_impl(x, x_stride, &f, tokens, hidden, folded_weight, w_dtype, qkv_dim, w_stride, bias,
                               bias_dtype, num_q_heads, num_kv_heads, qkv_dtype, nullptr, nullptr, 0, 0.f,
                               BFA_DTYPE_BF16, positions, positions_dtype, cos_sin_cache, max_position, out,
                               out_dtype, out_stride, ws + p.operand_bytes, fsize - p.operand_bytes, status,
                               stream, layer_cache ? &ce : nullptr);
  }
  float* rs = static_cast<float*>(workspace);
  const int64_t rs_bytes = align256(tokens * 4);
  int rc = launch_row_scale(x, x_dtype, tokens, hidden, x_stride, rs, eps, as_stream(stream));
  if (rc != BFA_OK) return rc;
  // the prefill GEMM's fused epilogue resolves the cache slots itself
  const CacheEpi ce{layer_cache, cache_dtype, stride_kv, stride_head, nullptr, write_kv_out ? 0 : 1, &a};
  return qkv_projection_impl(x, x_stride, nullptr, tokens, hidden, folded_weight, w_dtype, qkv_dim, w_stride,
                             bias, bias_dtype, num_q_heads, num_kv_heads, qkv_dtype, nullptr, nullptr, 0, 0.f,
                             BFA_DTYPE_BF16, positions, positions_dtype, cos_sin_cache, max_position, out,
                             out_dtype, out_stride, static_cast<char*>(workspace) + rs_bytes,
                             workspace_bytes - rs_bytes, status, stream, layer_cache ? &ce : nullptr, rs);
}

// ------------------------------------------------ allocation-free variant
// bfa_fused_rmsnorm_qkv_noalloc runs bfa_fused_rmsnorm_qkv with its workspace
// in `scratch`, a file-scope device array of BFA_NOALLOC_SCRATCH_BYTES: each GPU
// the library runs on holds its own copy until the process ends.  On the host
// the array's name denotes a shadow variable, not device memory, so host code
// never passes it to a kernel or a copy: it uses the device address that
// hipGetSymbolAddress returns for the device, looked up once per device (with
// that device current) and kept in noalloc_scratch_addr.  Nothing in the QKV
// kernels needs the workspace zeroed (the operand pre-pass writes every
// operand row and every split writes its whole partial tile before a later
// kernel reads it), so the array is never cleared; it keeps the last call's
// contents.  Calls that overlap on one GPU (several streams, or several host
// threads) share the array and race.
static __device__ __align__(256) unsigned char scratch[BFA_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_addr[kMaxScratchDevices] = {};
}  // namespace

// Device address of `scratch` on the device that runs `stream` (the current
// device for the null stream).
static int noalloc_scratch_addr(void* stream, void** addr) {
  int dev = -1;
  hipError_t e = stream ? hipStreamGetDevice(as_stream(stream), &dev) : hipGetDevice(&dev);
  if (e != hipSuccess) return set_error(BFA_ERR_LAUNCH, "bfa_fused_rmsnorm_qkv_noalloc: no device: %s",
                                        hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxScratchDevices)
    return set_error(BFA_ERR_UNSUPPORTED, "bfa_fused_rmsnorm_qkv_noalloc: device %d beyond %d", dev,
                     kMaxScratchDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_addr[dev]) {
    int cur = -1;
    e = hipGetDevice(&cur);
    if (e == hipSuccess && cur != dev) e = hipSetDevice(dev);
    void* p = nullptr;
    if (e == hipSuccess) e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (cur >= 0 && cur != dev) {
      const hipError_t back = hipSetDevice(cur);
      if (e == hipSuccess) e = back;
    }
    if (e != hipSuccess || p == nullptr)
      return set_error(BFA_ERR_LAUNCH, "bfa_fused_rmsnorm_qkv_noalloc: scratch address on device %d: %s",
                       dev, hipGetErrorString(e));
    g_scratch_addr[dev] = p;
  }
  *addr = g_scratch_addr[dev];
  return BFA_OK;
}

extern "C" int bfa_fused_rmsnorm_qkv_noalloc(
    const void* x, int x_dtype, int64_t tokens, int64_t hidden, int64_t x_stride,
    const void* norm_weight, int nw_dtype, float eps, int mixed_rounding, const void* qkv_weight,
    int w_dtype, int64_t qkv_dim, int64_t w_stride, const void* bias, int bias_dtype,
    int64_t num_q_heads, int64_t num_kv_heads, int qkv_dtype, const void* q_norm_weight,
    const void* k_norm_weight, int qk_norm_dtype, float qk_eps, int qk_norm_out_dtype,
    const void* positions, int positions_dtype, const float* cos_sin_cache, int64_t max_position,
    void* out, int out_dtype, int64_t out_stride, int32_t* status, void* stream) {
  const char* what = "bfa_fused_rmsnorm_qkv_noalloc";
  BFA_REQUIRE(x && norm_weight && qkv_weight, "%s: null pointer", what);
  if (tokens == 0) return BFA_OK;
  BFA_REQUIRE(tokens > 0 && hidden > 0 && qkv_dim > 0, "%s: bad geometry", what);
  const int64_t heads = num_q_heads + 2 * num_kv_heads;
  BFA_REQUIRE(num_q_heads > 0 && num_kv_heads > 0 && qkv_dim % heads == 0, "%s: bad head geometry", what);
  const int64_t need = bfa_fused_rmsnorm_qkv_workspace_size(tokens, hidden, qkv_dim, qkv_dim / heads);
  BFA_REQUIRE(need <= BFA_NOALLOC_SCRATCH_BYTES,
              "%s: %lld tokens x hidden %lld x qkv_dim %lld need %lld bytes of scratch, more than the "
              "%lld this entry point holds; call bfa_fused_rmsnorm_qkv with a workspace",
              what, (long long)tokens, (long long)hidden, (long long)qkv_dim, (long long)need,
              (long long)BFA_NOALLOC_SCRATCH_BYTES);
  void* ws = nullptr;
  const int rc = noalloc_scratch_addr(stream, &ws);
  if (rc != BFA_OK) return rc;
  return bfa_fused_rmsnorm_qkv(x, x_dtype, tokens, hidden, x_stride, norm_weight, nw_dtype, eps,
                               mixed_rounding, qkv_weight, w_dtype, qkv_dim, w_stride, bias, bias_dtype,
                               num_q_heads, num_kv_heads, qkv_dtype, q_norm_weight, k_norm_weight,
                               qk_norm_dtype, qk_eps, qk_norm_out_dtype, positions, positions_dtype,
                               cos_sin_cache, max_position, out, out_dtype, out_stride, ws,
                               BFA_NOALLOC_SCRATCH_BYTES, status, stream);
}

// ------------------------------------------------------- linear fusions
extern "C" int64_t bfa_linear_workspace_size(int64_t tokens, int64_t k, int64_t n, int mode) {
  if (tokens <= 0 || n <= 0) return 0;
  const int64_t nw = mode == BFA_LINEAR_SILU_AND_MUL ? 2 * n : n;
  const QkvPlan p = make_plan(tokens, nw, k, 0);
  return p.decode ? p.part_bytes : 0;  // prefill tiles finish in their epilogue
}

extern "C" int bfa_linear(const void* x, int dtype, int64_t tokens, int64_t k, int64_t x_stride,
                          const void* weight, int64_t n, int64_t w_stride, const void* bias,
                          int bias_dtype, int mode, int proj_dtype, const void* residual, int residual_dtype, int64_t residual_stride,
                          int sum_dtype, void* out, int out_dtype, int64_t out_stride,
                          void* workspace, int64_t workspace_bytes, void* stream) {
  const char* what = "bfa_linear";
  BFA_REQUIRE(dtype == BFA_DTYPE_BF16 || dtype == BFA_DTYPE_F16, "%s: x and weight must be bf16 or fp16",
              what);
  BFA_REQUIRE(mode == BFA_LINEAR_PLAIN || mode == BFA_LINEAR_SILU_AND_MUL, "%s: bad mode %d", what, mode);
  BFA_REQUIRE(is_float_dtype(proj_dtype) && is_float_dtype(sum_dtype) && is_float_dtype(out_dtype),
              "%s: bad dtype", what);
  BFA_REQUIRE(residual == nullptr || is_float_dtype(residual_dtype), "%s: bad residual dtype", what);
  BFA_REQUIRE(mode == BFA_LINEAR_PLAIN || (residual == nullptr && bias == nullptr),
              "%s: no bias or residual with silu_and_mul", what);
  BFA_REQUIRE(bias == nullptr || is_float_dtype(bias_dtype), "%s: bad bias dtype", what);
  BFA_REQUIRE(tokens >= 0 && k > 0 && n > 0, "%s: bad geometry", what);
  BFA_REQUIRE(k % 16 == 0, "%s: k must be a multiple of 16 (got %lld)", what, (long long)k);
  BFA_REQUIRE(x_stride >= k && w_stride >= k && x_stride % 8 == 0 && w_stride % 8 == 0 &&
                  aligned16(x) && aligned16(weight),
              "%s: x / weight rows must be 16-byte aligned", what);
  BFA_REQUIRE(out_stride >= n && (residual == nullptr || residual_stride >= n), "%s: bad strides", what);
  if (tokens == 0) return BFA_OK;
  BFA_REQUIRE(x && weight && out, "%s: null pointer", what);
  const bool swiglu = mode == BFA_LINEAR_SILU_AND_MUL;
  const int64_t nw = swiglu ? 2 * n : n;
  const QkvPlan p = make_plan(tokens, nw, k, 0);
  const int64_t need = p.decode ? p.part_bytes : 0;
  BFA_REQUIRE(workspace_bytes >= need && (need == 0 || workspace),
              "%s: workspace too small (%lld < %lld bytes)", what, (long long)workspace_bytes,
              (long long)need);
  BFA_REQUIRE(need == 0 || aligned16(workspace), "%s: workspace must be 16-byte aligned", what);

  QkvEpi e{};
  e.qkv_dt = proj_dtype; e.mid_dt = sum_dtype; e.out_dt = out_dtype;
  e.res = residual; e.res_dt = residual_dtype; e.ldr = residual_stride;
  e.bias = bias; e.bias_dtype = bias_dtype;
  e.out = out; e.ldo = out_stride; e.n = n;
  e.vec = aligned16(out) && out_stride % 8 == 0 &&
          (residual == nullptr || (aligned16(residual) && residual_stride % 8 == 0));
  GemmArgs g{};
  g.a = static_cast<const uint16_t*>(x);
  g.w = static_cast<const uint16_t*>(weight);
  g.m = tokens; g.n = n; g.k = k; g.lda = x_stride; g.ldw = w_stride;
  const hipStream_t st = as_stream(stream);
  const bool bf16 = dtype == BFA_DTYPE_BF16;
  if (p.decode) {
    SplitArgs sa{};
    sa.a = g.a; sa.w = g.w;
    sa.m = tokens; sa.n = nw; sa.k = k; sa.lda = x_stride; sa.ldw = w_stride;
    sa.kchunk = p.kchunk; sa.part = static_cast<float*>(workspace);
    if (bf16) launch_decode<true>(p, sa, st); else launch_decode<false>(p, sa, st);
    const int rc = check_launch(what);
    if (rc != BFA_OK) return rc;
    const int64_t threads = cdiv(tokens, 4) * n;
    const dim3 egrid(static_cast<unsigned>(cdiv(threads, 256)));
    const float* part = static_cast<const float*>(workspace);
    const int reg_order = (p.stream && p.mt > 1) ? 1 : 0;
    if (swiglu) {
      hipLaunchKernelGGL(linear_decode_epilogue_kernel<true>, egrid, dim3(256), 0, st, part, p.splits,
                         reg_order, p.mt, tokens, nw, g, e);
    } else {
      hipLaunchKernelGGL(linear_decode_epilogue_kernel<false>, egrid, dim3(256), 0, st, part, p.splits,
                         reg_order, p.mt, tokens, nw, g, e);
    }
    return check_launch(what);
  }
  if (bf16) launch_linear<true>(p, g, e, swiglu, nw, st); else launch_linear<false>(p, g, e, swiglu, nw, st);
  return check_launch(what);
}
