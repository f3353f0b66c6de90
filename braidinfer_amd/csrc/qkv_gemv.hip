// One-launch fused RMSNorm + QKV projection (+ bias, RoPE, KV append) for 1 to
// 8 decode tokens without q/k norm, on gfx950.
//
// Same reference semantics as qkv.hip (kernels/fused_rmsnorm_qkv_*.py and the
// RoPE of layers/rotary_embedding.py:49-65, models/llama.py:169-205).  At a few
// tokens the projection is a weight stream, and the split-K kernels of qkv.hip
// need a second launch to sum their partials.  Here a workgroup owns 8 RoPE
// pairs of one head (16 output columns) for the whole of K, so nothing leaves
// it: the operand rows are normalised once per workgroup into LDS (the fold of
// the fused op: round(x / rms(x) * gamma), the operand pre-pass's rounding
// points), the weight rows stream straight into MFMA B fragments, the four
// waves' partial tiles meet in LDS, and one thread per (token, pair) finishes.
// Heads with q/k norm stay on the split-K path (gemv_ok below).
#include "bfa_device.h"
#include "bfa_host.h"
#include "bfa_internal.h"
#include "bfa_qkv.h"

namespace bfa {

typedef __attribute__((ext_vector_type(8))) __bf16 gemv_bf16x8_t;
typedef __attribute__((ext_vector_type(4))) float gemv_f32x4_t;

// TM: token capacity (1, 2, 4 or 8; tokens <= TM).  A workgroup owns PG
// RoPE pairs of one head, c0 .. c0+PG-1, and their partners D/2 on: 2 PG output
// columns (PG = 8 from the launcher; with PG = 4 the MFMA's columns 8-15 would
// repeat 0-7 and be dropped).
// The normalised operand rows go to LDS once (bf16, rows padded by 16 bytes);
// the four waves split K, each taking 32-deep steps of
// v_mfma_f32_16x16x32_bf16 with the operand rows as A (rows past the token
// count zero) and the 16 weight rows as B, loaded straight into the fragment
// layout (lane l: row l % 16, K offset 8 (l / 16)); the four partial tiles meet
// in LDS and one thread per (token, pair) runs the epilogue.
template <int TM, bool FOLD>
__global__ __launch_bounds__(256) void qkv_gemv_kernel(GemvKArgs c) {
  // every argument goes into registers here, with one wait for their loads
  // (left to the compiler they come in several dependent rounds)
  asm volatile("" ::"s"(c.a), "s"(c.w), "s"(c.gamma), "s"(c.bias), "s"(c.positions), "s"(c.cs), "s"(c.out),
               "s"(c.status), "s"(c.cache), "s"(c.slot_off));
  asm volatile("" ::"s"(c.ldo), "s"(c.c_skv), "s"(c.c_sh), "s"(c.m), "s"(c.k), "s"(c.lda), "s"(c.ldw), "s"(c.pw),
               "s"(c.hq), "s"(c.hkv), "s"(c.hd), "s"(c.max_pos), "s"(c.eps));
  asm volatile("" ::"s"(static_cast<int>(c.gamma_dt)), "s"(static_cast<int>(c.mixed)), "s"(static_cast<int>(c.bias_dt)),
               "s"(static_cast<int>(c.qkv_dt)), "s"(static_cast<int>(c.out_dt)), "s"(static_cast<int>(c.cache_dt)),
               "s"(static_cast<int>(c.pos_is_i64)), "s"(static_cast<int>(c.skip_kv_out)));
  constexpr int KMAX = 4096, XP = KMAX + 8;  // operand row pitch in LDS (bf16)
  constexpr int SB = 16;                     // K steps per weight batch (16 loads in flight per lane)
  __shared__ uint16_t xs[TM * XP];
  __shared__ float red[4][16][17];
  __shared__ float sred[4][TM];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int hd = c.hd, half = hd / 2, pg = c.pw, tph = half / pg;
  const int b = static_cast<int>(blockIdx.x);
  const int head = b / tph, c0 = (b - head * tph) * pg;
  const int kd = head < c.hq ? 0 : (head < c.hq + c.hkv ? 1 : 2);
  const int K = c.k, S = K / 32;  // 32-deep steps; wave w takes steps [w S / 4, (w + 1) S / 4)
  const int s0 = wid * (S / 4), ns = S / 4;

  // Every load below is unconditional (absent inputs read a stand-in that is
  // masked afterwards, indices clamped) and no branch separates them, so all
  // of them are in flight together and each use waits only for its own.
  // ---- epilogue role: thread (token t, pair p); its position goes out first,
  //      since the cos/sin loads wait for it (a wait covers every earlier load)
  const bool ep = tid < c.m * pg;
  const int et = ep ? tid / pg : 0, ep_p = tid - (tid / pg) * pg;
  const int64_t ec1 = static_cast<int64_t>(head) * hd + c0 + ep_p, ec2 = ec1 + half;
  const bool rope = c.cs != nullptr && kd != 2;
  const bool app = c.cache != nullptr && kd != 0;
  // weight fragment rows of this lane: row r = lane % 16 of the group (mod 2 PG)
  const int fr = lane & 15, fq = lane >> 4, fg = fr % (2 * pg);
  const int64_t wcol = static_cast<int64_t>(head) * hd + (fg < pg ? c0 + fg : half + c0 + (fg - pg));
  const uint16_t* wrow = c.w + wcol * c.ldw + fq * 8;
  // an absent input reads, at index 0, a stand-in: the weight granule this lane
  // streams first (one address for every lane would send all of the grid's
  // requests to one cache line)
  const uint16_t* own = wrow + static_cast<int64_t>(s0) * 32;
  const int32_t* pw32 = static_cast<const int32_t*>(rope ? c.positions : static_cast<const void*>(own));
  const int32_t plo = pw32[!rope ? 0 : (c.pos_is_i64 ? 2 * et : et)];
  const int32_t phi = pw32[!rope ? 0 : (c.pos_is_i64 ? 2 * et + 1 : et)];
  // ---- operand rows: thread tid takes granules tid, tid + 256, .. of each row
  const int G = K / 8, GPT = (G + 255) / 256;  // granules per thread and row (K <= 4096: <= 2)
  uint4 xr[TM][2], graw[2][2];
#pragma unroll
  for (int t = 0; t < TM; ++t) {
    const uint16_t* xrow = c.a + static_cast<int64_t>(t < c.m ? t : c.m - 1) * c.lda;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int g = j < GPT ? min(tid + 256 * j, G - 1) : 0;
      xr[t][j] = load16(xrow + g * 8);
    }
  }
  // ---- the fold's gamma granules (16 bytes, or 32 for fp32), requested ahead of
  //      the weights: loads complete in order, so the fold then waits for the
  //      operand rows and gamma alone and runs while the weight batch streams in
  if constexpr (FOLD) {
    const bool g32 = c.gamma_dt == BFA_DTYPE_F32;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int g = j < GPT ? min(tid + 256 * j, G - 1) : 0;
      const char* gp = static_cast<const char*>(c.gamma) + g * 8 * (g32 ? 4 : 2);
      graw[j][0] = load16(reinterpret_cast<const uint16_t*>(gp));
      graw[j][1] = load16(reinterpret_cast<const uint16_t*>(g32 ? gp + 16 : gp));
    }
  }
  const int bdt = c.bias ? c.bias_dt : BFA_DTYPE_BF16;
  const uint32_t bw1 = ld_word_al4(c.bias ? c.bias : own, bdt, c.bias ? ec1 : 0);
  const uint32_t bw2 = ld_word_al4(c.bias ? c.bias : own, bdt, c.bias ? ec2 : 0);
  const int64_t so_raw = (app ? c.slot_off : reinterpret_cast<const int64_t*>(own))[app ? et : 0];
  // ---- the first weight batch
  uint4 wb[SB];
#pragma unroll
  for (int i = 0; i < SB; ++i) wb[i] = load16(wrow + static_cast<int64_t>(s0 + min(i, ns - 1)) * 32);
  // the cos/sin values (they wait for the position only)
  const int64_t praw = c.pos_is_i64 ? static_cast<int64_t>((static_cast<uint64_t>(static_cast<uint32_t>(phi)) << 32) |
                                                           static_cast<uint32_t>(plo))
                                    : static_cast<int64_t>(plo);
  const int64_t pwr = praw < 0 ? praw + c.max_pos : praw;
  const int32_t pc = !rope ? 0 : ((pwr >= 0 && pwr < c.max_pos) ? static_cast<int32_t>(pwr) : -1);
  const float* csr = rope ? c.cs + static_cast<int64_t>(pc >= 0 ? pc : 0) * hd : reinterpret_cast<const float*>(own);
  const float cv = csr[rope ? c0 + ep_p : 0];
  const float sv = csr[rope ? half + c0 + ep_p : 0];
  const float b1 = c.bias ? word_value_al4(bw1, bdt, ec1) : 0.f, b2 = c.bias ? word_value_al4(bw2, bdt, ec2) : 0.f;
  const int64_t so = app ? so_raw : -1;

  // ---- operand rows -> LDS (normalised by the fold: round(x / rms(x) * gamma),
  //      the operand pre-pass's rounding points)
  float inv[TM];
#pragma unroll
  for (int t = 0; t < TM; ++t) inv[t] = 1.f;
  if constexpr (FOLD) {
#pragma unroll
    for (int t = 0; t < TM; ++t) {
      float ss = 0.f;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        if (j < GPT && tid + 256 * j < G) {
          float v[8];
          unpack8<BFA_DTYPE_BF16>(xr[t][j], v);
#pragma unroll
          for (int i = 0; i < 8; ++i) ss += v[i] * v[i];
        }
      }
      ss = wave_sum_dpp(ss);
      if (lane == 0) sred[wid][t] = ss;
    }
    __syncthreads();
#pragma unroll
    for (int t = 0; t < TM; ++t)
      inv[t] = 1.0f / sqrtf((sred[0][t] + sred[1][t] + sred[2][t] + sred[3][t]) / static_cast<float>(K) + c.eps);
  }
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int g = tid + 256 * j;
    if (j < GPT && g < G) {
      float gv[8];
      if constexpr (FOLD) {
        float gb[8], gh[8];
        unpack8<BFA_DTYPE_BF16>(graw[j][0], gb);
        unpack8<BFA_DTYPE_F16>(graw[j][0], gh);
        const uint32_t u[8] = {graw[j][0].x, graw[j][0].y, graw[j][0].z, graw[j][0].w,
                               graw[j][1].x, graw[j][1].y, graw[j][1].z, graw[j][1].w};
#pragma unroll
        for (int i = 0; i < 8; ++i)
          gv[i] = c.gamma_dt == BFA_DTYPE_F32 ? __uint_as_float(u[i]) : (c.gamma_dt == BFA_DTYPE_F16 ? gh[i] : gb[i]);
      }
#pragma unroll
      for (int t = 0; t < TM; ++t) {
        uint4 o = xr[t][j];
        if constexpr (FOLD) {
          float v[8];
          unpack8<BFA_DTYPE_BF16>(xr[t][j], v);
#pragma unroll
          for (int i = 0; i < 8; ++i)
            v[i] = c.mixed ? round_bf16(v[i] * inv[t]) * gv[i] : (v[i] * inv[t]) * gv[i];
          o = make_uint4(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]), pack_bf16x2(v[4], v[5]),
                         pack_bf16x2(v[6], v[7]));
        }
        if (t >= c.m) o = make_uint4(0, 0, 0, 0);
        *reinterpret_cast<uint4*>(xs + t * XP + g * 8) = o;
      }
    }
  }
  __syncthreads();

  // ---- the projection: S / 4 steps per wave, weight batches of SB steps
  // two accumulators, even and odd steps, so that consecutive MFMAs do not
  // wait for each other's result; summed once at the end
  gemv_f32x4_t acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
  const int arow = fr < TM ? fr : 0;  // A rows past TM read row 0 and are zeroed
  auto step = [&](int s, const uint4& bfrag, gemv_f32x4_t& acc) {
    uint4 afrag = *reinterpret_cast<const uint4*>(xs + arow * XP + s * 32 + fq * 8);
    if (fr >= TM) afrag = make_uint4(0, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(gemv_bf16x8_t, afrag),
                                                  __builtin_bit_cast(gemv_bf16x8_t, bfrag), acc, 0, 0, 0);
  };
  for (int i0 = 0; i0 < ns; i0 += SB) {
    uint4 wn[SB];
    const bool more = i0 + SB < ns;  // uniform
    if (more) {
#pragma unroll
      for (int i = 0; i < SB; ++i) wn[i] = load16(wrow + static_cast<int64_t>(s0 + min(i0 + SB + i, ns - 1)) * 32);
    }
    if (i0 + SB <= ns) {
      // a whole batch: no per-step test, so the operand reads from LDS all go
      // out ahead of the MFMAs instead of one round trip per step
      uint4 af[SB];
#pragma unroll
      for (int i = 0; i < SB; ++i) {
        af[i] = *reinterpret_cast<const uint4*>(xs + arow * XP + (s0 + i0 + i) * 32 + fq * 8);
        if (fr >= TM) af[i] = make_uint4(0, 0, 0, 0);
      }
#pragma unroll
      for (int i = 0; i < SB; ++i) {
        gemv_f32x4_t& acc = (i & 1) ? acc1 : acc0;
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(gemv_bf16x8_t, af[i]),
                                                      __builtin_bit_cast(gemv_bf16x8_t, wb[i]), acc, 0, 0, 0);
      }
    } else {
#pragma unroll
      for (int i = 0; i < SB; ++i)
        if (i0 + i < ns) step(s0 + i0 + i, wb[i], (i & 1) ? acc1 : acc0);
    }
    if (more) {
#pragma unroll
      for (int i = 0; i < SB; ++i) wb[i] = wn[i];
    }
  }
  // D layout: lane l holds D[4 (l / 16) + i][l % 16] (token, group column)
  const gemv_f32x4_t acc = acc0 + acc1;
#pragma unroll
  for (int i = 0; i < 4; ++i) red[wid][4 * fq + i][fr] = acc[i];
  __syncthreads();

  // ---- epilogue: thread (token et, pair ep_p): columns ep_p and PG + ep_p of the group
  if (!ep) return;
  const int e2 = pg + ep_p;
  const float s1 = red[0][et][ep_p] + red[1][et][ep_p] + red[2][et][ep_p] + red[3][et][ep_p];
  const float s2 = red[0][et][e2] + red[1][et][e2] + red[2][et][e2] + red[3][et][e2];
  float x1 = round_to(s1 + b1, c.qkv_dt), x2 = round_to(s2 + b2, c.qkv_dt);
  const int dt = c.qkv_dt;
  if (rope) {
    const bool pok = pc >= 0;
    if (!pok && ep_p == 0) flag_status(c.status, BFA_STATUS_INDEX_OOB);
    const float u = x1, w = x2;
    x1 = pok ? round_to(u * cv - w * sv, dt) : 0.f;
    x2 = pok ? round_to(w * cv + u * sv, dt) : 0.f;
  }
  if (kd == 0 || !c.skip_kv_out) {
    store_any(c.out, c.out_dt, et * c.ldo + ec1, x1);
    store_any(c.out, c.out_dt, et * c.ldo + ec2, x2);
  }
  if (app && so >= 0) {
    const int64_t hk = head - c.hq - (kd == 2 ? c.hkv : 0);
    const int64_t cb = so + (kd == 2 ? c.c_skv : 0) + hk * c.c_sh + c0 + ep_p;
    store_any(c.cache, c.cache_dt, cb, round_to(x1, c.out_dt));
    store_any(c.cache, c.cache_dt, cb + half, round_to(x2, c.out_dt));
  }
}

// The planner takes it where it beats the split-K kernels and their reduction
// (fused op, graph-replayed, one box; gemv / split-K in us):
//   tokens              2            4            6-8          10-16
//   TinyLlama        5.5 / 7.5    6.2 / 7.9    7.8 / 8.6-8.9  13.0 / 9.8-10.5
//   Qwen3 geometry   5.3 / 6.3    6.0 / 6.5    7.6 / 6.9-7.1  12.8 / 8.0-8.7
//   Llama-3-8B      12.6 / 13.8  13.9 / 14.2  21.4 / 16.9-17.2 38.6 / 17.2-17.7
// (Qwen3 geometry without its q/k norm).  So: up to 4 tokens, and up to 8 when
// the grid is at most 192 workgroups (TinyLlama's 160): each workgroup reads
// and normalises every operand row into LDS, which from 5 tokens costs more
// than the second launch unless the grid is small (at 8 rows and K = 4096 the
// rows alone fill 64 KiB of LDS).  A q/k-norm head needs all of its columns for
// the norm, and its workgroups hold 16 each; handing them to one finisher
// through device-coherent memory cost 3-8 us (one token: 7.9 us against 6.3 us
// split-K), so those calls stay on the split-K path.  Planner override
// BFA_TUNE_DECODE_GEMV = 0 never takes it.
bool gemv_ok(int64_t tokens, int64_t k, int64_t n, int64_t hd, bool qk_norm, const void* bias, bool bf16_w,
             bool bf16_x, const void* a, int64_t lda) {
  if (tuning(BFA_TUNE_DECODE_GEMV) == 0) return false;
  if (tokens < 1 || tokens > 8 || qk_norm || !bf16_w || !bf16_x || hd % 16 != 0) return false;
  if (tokens > 4 && n / 16 > 192) return false;
  // the bias words are read at 4-byte-aligned addresses from the index alone
  if ((reinterpret_cast<uintptr_t>(bias) & 3u) != 0) return false;
  return k % 32 == 0 && k <= 4096 && k / 32 >= 4 && (k / 32) % 4 == 0 && hd <= 1024 && aligned16(a) &&
         lda % 8 == 0 && lda < (int64_t{1} << 31);
}

template <int TM>
static void launch_gemv_t(bool fold, unsigned grid, const GemvKArgs& c, hipStream_t s) {
  if (fold) hipLaunchKernelGGL((qkv_gemv_kernel<TM, true>), dim3(grid), dim3(256), 0, s, c);
  else hipLaunchKernelGGL((qkv_gemv_kernel<TM, false>), dim3(grid), dim3(256), 0, s, c);
}

void launch_qkv_gemv(GemvArgs d, bool fold, const QkvEpi& e, hipStream_t s) {
  const int64_t heads = e.hq + 2 * e.hkv;
  // groups of 8 pairs.  Groups of 4 would put more CUs on the weight stream when
  // the heads are few, but each group pays the operand rows and their norm:
  // TinyLlama, 1 / 8 tokens, 160 groups of 8: 6.0 / 8.8 us; 320 groups of 4:
  // 8.2 / 16.4 us.
  const int64_t pg = 8;
  const unsigned grid = static_cast<unsigned>(heads * (e.hd / 2 / pg));
  GemvKArgs c{};
  c.a = d.a; c.w = d.w; c.gamma = d.gamma;
  c.bias = e.bias; c.positions = e.positions; c.cs = e.cs;
  c.out = e.out; c.status = e.status; c.cache = e.cache; c.slot_off = e.slot_off;
  c.ldo = e.ldo; c.c_skv = e.c_skv; c.c_sh = e.c_sh;
  c.m = static_cast<int32_t>(d.m); c.k = static_cast<int32_t>(d.k);
  c.lda = static_cast<int32_t>(d.lda); c.ldw = static_cast<int32_t>(d.ldw); c.pw = static_cast<int32_t>(pg);
  c.hq = static_cast<int32_t>(e.hq); c.hkv = static_cast<int32_t>(e.hkv);
  c.hd = static_cast<int32_t>(e.hd); c.max_pos = static_cast<int32_t>(e.max_pos);
  c.eps = d.eps;
  c.gamma_dt = static_cast<uint8_t>(d.gamma_dt); c.mixed = static_cast<uint8_t>(d.mixed);
  c.bias_dt = static_cast<uint8_t>(e.bias_dtype); c.qkv_dt = static_cast<uint8_t>(e.qkv_dt);
  c.out_dt = static_cast<uint8_t>(e.out_dt); c.cache_dt = static_cast<uint8_t>(e.cache_dt);
  c.pos_is_i64 = static_cast<uint8_t>(e.pos_is_i64); c.skip_kv_out = static_cast<uint8_t>(e.skip_kv_out);
  if (d.m <= 1) launch_gemv_t<1>(fold, grid, c, s);
  else if (d.m <= 2) launch_gemv_t<2>(fold, grid, c, s);
  else if (d.m <= 4) launch_gemv_t<4>(fold, grid, c, s);
  else launch_gemv_t<8>(fold, grid, c, s);
}

}  // namespace bfa
