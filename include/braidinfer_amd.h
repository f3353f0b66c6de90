/*
 * braidinfer_amd — C ABI of the MI355X (gfx950) fused per-layer kernels.
 *
 * Every entry point takes plain device pointers, element counts and strides
 * (strides are in ELEMENTS, not bytes), a dtype code for each tensor operand,
 * and a hipStream_t passed as void* (NULL = the null stream).  Work is enqueued
 * asynchronously on that stream; no entry point synchronises or allocates
 * device memory unless its comment says so.
 *
 * Return value: BFA_OK (0) on success, a negative BFA_ERR_* code otherwise;
 * bfa_last_error() then returns a message for the calling thread.
 *
 * The reference (braidpool/braidinfer) is pure Python/Triton and has no FFI of
 * its own; each entry point below names the Python function or class whose
 * semantics it reproduces, with the reference file:line.  The Python package
 * braidinfer_amd (kernels/, layers/) binds these with ctypes under the
 * reference's own class and function names.
 */
#ifndef BRAIDINFER_AMD_H_
#define BRAIDINFER_AMD_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* dtype codes */
#define BFA_DTYPE_F32 0
#define BFA_DTYPE_F16 1
#define BFA_DTYPE_BF16 2
#define BFA_DTYPE_I32 3
#define BFA_DTYPE_I64 4

/* return codes */
#define BFA_OK 0
#define BFA_ERR_INVALID (-1)     /* bad argument (shape, dtype, pointer)      */
#define BFA_ERR_UNSUPPORTED (-2) /* valid but not implemented for this shape  */
#define BFA_ERR_LAUNCH (-3)      /* HIP launch / runtime error                */

/* bits a kernel may OR into a caller-provided device status word (int32) */
#define BFA_STATUS_INDEX_OOB 1 /* an index (token id, position, delta, page) was out of range */
#define BFA_STATUS_APPEND_SKIPPED 2 /* a KV append skipped a token whose page offset is past
                                       the page list (the reference prints an error) */

#define BFA_ABI_VERSION 1

int bfa_abi_version(void);
const char* bfa_last_error(void);

/* ------------------------------------------------------ planner overrides --
 * No counterpart in the reference (its Triton launchers have fixed grids).
 * The kernel planners pick a kernel form and a grid from the shapes alone; the
 * keys below override one choice each, for measurements and for tests that
 * reach a form the planner would not pick at that shape.  A serving process
 * leaves them unset.  Each key starts from the environment variable named
 * beside it, read ONCE when the library is loaded (an integer; absent = unset);
 * afterwards only bfa_set_tuning changes it, so no entry point reads the
 * environment on a call.  value -1 = unset (the planner's own choice).
 * bfa_set_tuning returns BFA_OK, or BFA_ERR_INVALID for an unknown key;
 * bfa_get_tuning returns the value, -1 when unset or the key is unknown.
 * The table is process-wide and not synchronised: set it between calls. */
#define BFA_TUNE_DECODE_KS 0         /* BFA_DECODE_KS: 64-deep K segments per decode split (1..8) */
#define BFA_TUNE_DECODE_WG 1         /* BFA_DECODE_WG: workgroup target of the deep-K decode form */
#define BFA_TUNE_DECODE_SPLITS 2     /* BFA_DECODE_SPLITS: split count of the deep-K decode form */
#define BFA_TUNE_QKV_TILE 3          /* BFA_QKV_TILE: prefill tile, 1 2 3 64 or 128 (64: head_dim <= 64) */
#define BFA_TUNE_EDT_RT 4            /* BFA_EDT_RT: non-zero = run-time epilogue dtypes only */
#define BFA_TUNE_DECODE_PAIR 5       /* BFA_DECODE_PAIR: 0 = never the column-pair decode
                                        kernel, 1 = at any shape it supports */
#define BFA_TUNE_NO_OPERAND_FOLD 6   /* BFA_NO_OPERAND_FOLD: non-zero = keep the decode pre-pass */
#define BFA_TUNE_CASCADE_DECODE_WG 7 /* BFA_CASCADE_DECODE_WG: cascade decode workgroup target */
#define BFA_TUNE_CASCADE_FLAT 8      /* BFA_CASCADE_FLAT: 0 = fused cascade kernel, non-zero =
                                        flat form from 5 query rows */
#define BFA_TUNE_CASCADE_FLAT_WG 9   /* BFA_CASCADE_FLAT_WG: flat-form workgroup target */
#define BFA_TUNE_STREAM_STORES 10    /* BFA_STREAM_STORES: 0 = no nontemporal stores */
#define BFA_TUNE_QKV_PERSIST 11      /* BFA_QKV_PERSIST: prefill GEMM workgroups per CU that loop
                                        over the tiles (0 = one workgroup per tile; unset: 1 for
                                        the 256x256 tile, 0 for the others) */
#define BFA_TUNE_DECODE_GEMV 12      /* BFA_DECODE_GEMV: 0 = never the one-launch decode kernel
                                        (1-8 tokens without q/k norm) */
#define BFA_TUNE_COUNT 13
int bfa_set_tuning(int key, int value);
int bfa_get_tuning(int key);

/* ------------------------------------------------------------------ norms --
 * Row geometry shared by the norm entry points: `rows` rows of `hidden`
 * contiguous elements; row r lives at  (r / rows_inner) * stride_outer
 *                                     + (r % rows_inner) * stride_inner.
 * A 2-D [T, H] tensor is rows=T, rows_inner=1, stride_outer=row stride.
 * A [T, heads, D] view (per-head q/k norm) is rows=T*heads, rows_inner=heads.
 */

/* RMSNorm.rms_forward — braidinfer/layers/layernorm.py:35-44.
 *   y = to(x_dtype)( to(x_dtype)(x * rsqrt(mean(x^2) + eps)) * weight )
 * (for fp32 x both casts are no-ops and the reference mutates x in place:
 *  pass y == x to reproduce that).  y has x's dtype. */
int bfa_rms_norm(const void* x, void* y, const void* weight, int x_dtype, int w_dtype,
                 int64_t rows, int64_t rows_inner, int64_t hidden,
                 int64_t x_stride_outer, int64_t x_stride_inner,
                 int64_t y_stride_outer, int64_t y_stride_inner,
                 float eps, void* stream);

/* RMSNorm.add_rms_forward — braidinfer/layers/layernorm.py:46-57.
 *   s = f32(x) + f32(residual);  residual_out = to(x_dtype)(s)
 *   y = to(x_dtype)( to(x_dtype)(s * rsqrt(mean(s^2) + eps)) * weight )
 * x, residual, y, residual_out: 2-D [rows, hidden] with the given row strides.
 * residual_out may be NULL (the fp32 reference aliases it to y). */
int bfa_add_rms_norm(const void* x, const void* residual, void* y, void* residual_out,
                     const void* weight, int x_dtype, int w_dtype, int64_t rows,
                     int64_t hidden, int64_t x_stride, int64_t residual_stride,
                     int64_t y_stride, int64_t residual_out_stride, float eps,
                     void* stream);

/* RMSNormF32.forward — braidinfer/kernels/rmsnorm_f32.py:14-96,105-156.
 *   rms = sqrt(sum(x^2)/hidden + eps);  y(fp32) = (x / rms) * weight */
int bfa_rms_norm_f32(const void* x, float* y, const void* weight, int x_dtype, int w_dtype,
                     int64_t rows, int64_t hidden, int64_t x_stride_row,
                     int64_t x_stride_col, int64_t y_stride_row, int64_t y_stride_col,
                     float eps, void* stream);

/* ------------------------------------------------------------ embedding --
 * VocabParallelEmbedding.forward — braidinfer/layers/embed_head.py:28-29
 * (F.embedding(ids, weight)).  Byte copy of row ids[t] of `table` into row t
 * of `out`: bit-exact for any element type of `elem_bytes` bytes.  ids are
 * int32 or int64; an id outside [0, num_embeddings) yields a zero row and
 * sets BFA_STATUS_INDEX_OOB in *status (status may be NULL). */
int bfa_embedding(const void* table, int64_t num_embeddings, int64_t dim,
                  int64_t table_row_stride, int elem_bytes, const void* ids, int ids_dtype,
                  int64_t num_ids, void* out, int64_t out_row_stride, int32_t* status,
                  void* stream);

/* Embedding gather fused with the Qwen3 scaling
 * `embed_tokens(ids) * (1/sqrt(H))` (braidinfer/models/qwen3.py:463-465):
 * out = to(dtype)(f32(table[id]) * scale). */
int bfa_embedding_scaled(const void* table, int64_t num_embeddings, int64_t dim,
                         int64_t table_row_stride, int dtype, const void* ids, int ids_dtype,
                         int64_t num_ids, void* out, int64_t out_row_stride, float scale,
                         int32_t* status, void* stream);

/* ---------------------------------------------------------------- SwiGLU --
 * SiluAndMul.forward — braidinfer/layers/activation.py:11-13.
 * x: [rows, 2*inter] (gate | up), y: [rows, inter];
 * y = to(dtype)( to(dtype)(silu_f32(gate)) * up ). */
int bfa_silu_and_mul(const void* x, void* y, int dtype, int64_t rows, int64_t inter,
                     int64_t x_row_stride, int64_t y_row_stride, void* stream);

/* ------------------------------------------------------------------ RoPE --
 * RotaryEmbedding.forward / apply_rotary_emb —
 * braidinfer/layers/rotary_embedding.py:6-24,49-65 (neox half-split).
 * query/key are viewed as [num_tokens, heads, head_size] with the given
 * token/head strides and unit element stride; results go to contiguous
 * [num_tokens, heads, head_size] buffers query_out/key_out (same dtype).
 * cos_sin_cache: fp32 [max_position, head_size] (cos | sin halves).
 * Negative positions wrap as torch indexing does; positions outside
 * [-max_position, max_position) give zeros and set BFA_STATUS_INDEX_OOB.
 * query or key may be NULL to rotate only the other. */
int bfa_rotary_embedding(const void* positions, int positions_dtype, int64_t num_tokens,
                         const float* cos_sin_cache, int64_t max_position, int64_t head_size,
                         int dtype, const void* query, int64_t q_heads, int64_t q_stride_token,
                         int64_t q_stride_head, void* query_out, const void* key,
                         int64_t k_heads, int64_t k_stride_token, int64_t k_stride_head,
                         void* key_out, int32_t* status, void* stream);

/* apply_rotary_emb(x, cos, sin) — braidinfer/layers/rotary_embedding.py:6-24 —
 * with explicit per-token fp32 cos/sin rows (head_size/2 values each, row
 * stride cs_stride_token) instead of a table lookup.  x is viewed as
 * [num_tokens, heads, head_size]; out is contiguous, same dtype. */
int bfa_apply_rotary_emb(const void* x, int dtype, int64_t num_tokens, int64_t heads,
                         int64_t head_size, int64_t x_stride_token, int64_t x_stride_head,
                         const float* cos, const float* sin, int64_t cs_stride_token, void* out,
                         void* stream);

/* Differential re-rotation of cached chunk K — the per-page loop body of
 * CascadeAttention.forward, braidinfer/layers/cascade_attention.py:143-178.
 * kv_cache: one layer of the paged HND cache
 *   [num_cache_pages, 2, num_kv_heads, page_size, head_dim] (K at index 0;
 *   braidinfer/engine/page_manager.py:36-42).
 * Chunk c owns page-list entries [chunk_indptr[c], chunk_indptr[c+1]) of
 * page_indices (int32, as CascadeAttention._create_level builds them,
 * cascade_attention.py:264-295); its last page holds last_page_len[c] tokens.
 * Every token of chunk c is rotated by chunk_delta[c] (= global_position_start
 * - cached_position_start) using cos_sin_cache[chunk_delta[c]] with torch
 * negative-index wrap; delta == 0 leaves K unchanged, as the reference does.
 * out == NULL: rotate the cache in place.  Otherwise write
 * out[entry, token, head, :] ([num_entries, page_size, num_kv_heads, head_dim],
 * page-padded, padding slots zeroed) and leave the cache untouched; only then
 * may k_norm_weight be given, fusing the k_norm of cascade_attention.py:177-178
 * (RMSNorm.rms_forward over head_dim). */
int bfa_rerotate_paged_k(void* kv_cache, int dtype, int64_t num_cache_pages,
                         int64_t num_kv_heads, int64_t page_size, int64_t head_dim,
                         const int32_t* page_indices, int64_t num_entries,
                         const int32_t* chunk_indptr, const int32_t* last_page_len,
                         const void* chunk_delta, int delta_dtype, int64_t num_chunks,
                         const float* cos_sin_cache, int64_t max_position,
                         const void* k_norm_weight, int k_norm_dtype, float k_norm_eps,
                         void* out, int32_t* status, void* stream);

/* -------------------------------------------------- fused RMSNorm + QKV --
 * The four Triton variants share one entry point; the caller picks the
 * rounding points:
 *   FusedRMSNormQKVMixedPrecision  kernels/fused_rmsnorm_qkv_mixed_precision.py:14-247
 *       mixed_rounding=1, qkv_dtype=x dtype
 *   FusedRMSNormQKV                kernels/fused_rmsnorm_qkv_production.py:13-229
 *       mixed_rounding=0, qkv_dtype=BF16
 *   FusedRMSNormQKVMinimalF32      kernels/fused_rmsnorm_qkv_minimal_f32.py:14-214
 *   FusedRMSNormQKVWithBias        kernels/fused_rmsnorm_qkv_with_bias.py:13-228
 *       mixed_rounding=0, qkv_dtype=F32
 * and optionally fuses what the model glue does next with the result:
 *   q/k RMSNorm over head_dim (Qwen3, models/qwen3.py:257-281): pass
 *       q_norm_weight / k_norm_weight (either may be NULL), the result is cast
 *       to qk_norm_out_dtype;
 *   RoPE (models/qwen3.py:309, models/llama.py:189): pass positions and
 *       cos_sin_cache [max_position, head_dim].
 * Output: out[tokens, qkv_dim] (q | k | v columns, row stride out_stride) in
 * out_dtype.  W is [qkv_dim, hidden] (bf16 or fp16), rows [q; k; v]
 * (layers/linear.py:78-114).  The normalised operand is rounded to W's dtype
 * for the matrix cores (the fp32 variants round it once, where the reference's
 * fp32 dot product runs at TF32 on its GPUs).
 * workspace: device scratch of bfa_fused_rmsnorm_qkv_workspace_size() bytes,
 * 16-byte aligned; calls sharing a workspace must be stream-ordered. */
int64_t bfa_fused_rmsnorm_qkv_workspace_size(int64_t tokens, int64_t hidden, int64_t qkv_dim,
                                             int64_t head_dim);

int bfa_fused_rmsnorm_qkv(const void* x, int x_dtype, int64_t tokens, int64_t hidden,
                          int64_t x_stride, const void* norm_weight, int nw_dtype, float eps,
                          int mixed_rounding, const void* qkv_weight, int w_dtype,
                          int64_t qkv_dim, int64_t w_stride, const void* bias, int bias_dtype,
                          int64_t num_q_heads, int64_t num_kv_heads, int qkv_dtype,
                          const void* q_norm_weight, const void* k_norm_weight,
                          int qk_norm_dtype, float qk_eps, int qk_norm_out_dtype,
                          const void* positions, int positions_dtype,
                          const float* cos_sin_cache, int64_t max_position, void* out,
                          int out_dtype, int64_t out_stride, void* workspace,
                          int64_t workspace_bytes, int32_t* status, void* stream);

/* Allocation-free form of bfa_fused_rmsnorm_qkv.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under
 * HIP-graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Same arguments and results as bfa_fused_rmsnorm_qkv without the workspace:
 * the workspace is a device array inside the library, BFA_NOALLOC_SCRATCH_BYTES
 * per GPU, held until the process ends.  Shapes whose
 * bfa_fused_rmsnorm_qkv_workspace_size exceeds it return BFA_ERR_INVALID (at
 * Llama-3-8B shape, hidden 4096 -> 6144: every decode batch up to 64 tokens and
 * prefills up to 2048 tokens fit).  The call allocates nothing (no hipMalloc,
 * no library allocation); its first call on a device looks up the array's
 * address there.  Every call on one GPU uses the same array: calls that
 * overlap on a GPU (other streams, other host threads) race; stream-ordered
 * calls do not. */
#define BFA_NOALLOC_SCRATCH_BYTES (16LL << 20)
int bfa_fused_rmsnorm_qkv_noalloc(const void* x, int x_dtype, int64_t tokens, int64_t hidden,
                                  int64_t x_stride, const void* norm_weight, int nw_dtype, float eps,
                                  int mixed_rounding, const void* qkv_weight, int w_dtype,
                                  int64_t qkv_dim, int64_t w_stride, const void* bias, int bias_dtype,
                                  int64_t num_q_heads, int64_t num_kv_heads, int qkv_dtype,
                                  const void* q_norm_weight, const void* k_norm_weight,
                                  int qk_norm_dtype, float qk_eps, int qk_norm_out_dtype,
                                  const void* positions, int positions_dtype,
                                  const float* cos_sin_cache, int64_t max_position, void* out,
                                  int out_dtype, int64_t out_stride, int32_t* status, void* stream);

/* The variants without the mixed rounding (FusedRMSNormQKV,
 * kernels/fused_rmsnorm_qkv_production.py:13-229; FusedRMSNormQKVMinimalF32,
 * kernels/fused_rmsnorm_qkv_minimal_f32.py:14-214; FusedRMSNormQKVWithBias,
 * kernels/fused_rmsnorm_qkv_with_bias.py:13-228; the Llama attention input,
 * models/llama.py:169-205) at prefill, with the norm weight folded
 * into the QKV weight.  (x / rms) * gamma projected onto W equals the projection of x
 * onto W * gamma, scaled by 1 / rms per row, so the normalised operand is never
 * written: one pass computes the row statistic, the projection reads x itself.
 * bfa_fold_rmsnorm_weight: folded[n, k] = W[n, k] * norm_weight[k], the product in
 * fp32 rounded once to W's dtype (hidden a multiple of 8, 16-byte aligned rows); the
 * caller computes it once per (W, norm weight) pair and keeps it while both are
 * unchanged.
 * bfa_fused_rmsnorm_qkv_folded: as bfa_fused_rmsnorm_qkv with mixed_rounding = 0 and
 * no q/k norm, on the folded weight, and with layer_cache != NULL as
 * bfa_fused_rmsnorm_qkv_append (same cache arguments; NULL: no append, the other
 * cache arguments unread).  It takes the prefill projection's fused epilogue
 * (more than 64 tokens, head_dim 32, 64 or 128) and the column-pair decode
 * kernel's shapes (17-64 bf16 tokens, head_dim a multiple of 32, hidden a
 * multiple of 256, at least 128 column pairs: the row statistic then comes from
 * the kernel's own Gram diagonal), x in W's dtype; other shapes return
 * BFA_ERR_UNSUPPORTED before any launch.  Against the oracle the bf16 rounding
 * moves from the operand to the weight, within the same tolerance.
 * workspace: bfa_fused_rmsnorm_qkv_workspace_size() bytes, and with an append at
 * decode counts bfa_fused_rmsnorm_qkv_append_workspace_size(). */
int bfa_fold_rmsnorm_weight(const void* qkv_weight, int w_dtype, int64_t qkv_dim, int64_t hidden,
                            int64_t w_stride, const void* norm_weight, int nw_dtype, void* folded,
                            int64_t folded_stride, void* stream);
/* The folded form's first stage on its own: out[r] = 1 / sqrt(sum(x[r]^2)/hidden + eps)
 * (fp32), the factor the operand pre-pass multiplies by (minimal_f32.py:59-107). */
int bfa_rmsnorm_row_scale(const void* x, int x_dtype, int64_t rows, int64_t hidden, int64_t x_stride,
                          float* out, float eps, void* stream);
int bfa_fused_rmsnorm_qkv_folded(
    const void* x, int x_dtype, int64_t tokens, int64_t hidden, int64_t x_stride, float eps,
    const void* folded_weight, int w_dtype, int64_t qkv_dim, int64_t w_stride, const void* bias, int bias_dtype,
    int64_t num_q_heads, int64_t num_kv_heads, int qkv_dtype, const void* positions, int positions_dtype,
    const float* cos_sin_cache, int64_t max_position, void* out, int out_dtype, int64_t out_stride,
    void* workspace, int64_t workspace_bytes, void* layer_cache, int cache_dtype, int64_t num_pages,
    int64_t cache_page_slots, int64_t stride_page, int64_t stride_kv, int64_t stride_head, int64_t stride_slot,
    const void* kv_indices, int kv_indices_dtype, int64_t num_indices, const int32_t* kv_indptr,
    const void* batch_indices, int batch_indices_dtype, int64_t num_seqs, const void* cache_positions,
    int cache_positions_dtype, int64_t page_size, int write_kv_out, int32_t* status, void* stream);

/* The two stages of bfa_fused_rmsnorm_qkv, exposed separately.
 * Stage 1 (the RMSNorm prologue of every variant): operand[rows, hidden] =
 *   mixed_rounding ? to(op)( to(bf16)(x / rms) * w ) : to(op)( (x / rms) * w ),
 *   rms = sqrt(sum(x^2)/hidden + eps), op = operand_dtype (BF16 or F16). */
int bfa_rmsnorm_qkv_operand(const void* x, int x_dtype, int64_t rows, int64_t hidden,
                            int64_t x_stride, const void* norm_weight, int w_dtype,
                            int mixed_rounding, void* operand, int operand_dtype, float eps,
                            void* stream);

/* Stage 2: projection of a normalised operand [tokens, hidden] (contiguous,
 * W's dtype) with the epilogue described above.  part_workspace holds the
 * split-K / raw fp32 partial sums: bfa_fused_rmsnorm_qkv_workspace_size()
 * minus the operand's share (tokens*hidden*2 rounded up to 256 bytes). */
int bfa_qkv_projection(const void* operand, int64_t tokens, int64_t hidden,
                       const void* qkv_weight, int w_dtype, int64_t qkv_dim, int64_t w_stride,
                       const void* bias, int bias_dtype, int64_t num_q_heads,
                       int64_t num_kv_heads, int qkv_dtype, const void* q_norm_weight,
                       const void* k_norm_weight, int qk_norm_dtype, float qk_eps,
                       int qk_norm_out_dtype, const void* positions, int positions_dtype,
                       const float* cos_sin_cache, int64_t max_position, void* out,
                       int out_dtype, int64_t out_stride, void* part_workspace,
                       int64_t part_workspace_bytes, int32_t* status, void* stream);

/* ------------------------------------------------------- paged KV append --
 * append_to_paged_kv_cache_custom — braidinfer/kernels/kv_cache_utils.py:9-78
 * (called per layer by PageManager.append_kv_to_cache / append_kv_to_cache_for_chunk,
 * braidinfer/engine/page_manager.py:159-218,313-353).
 * k, v: [num_tokens, num_kv_heads, head_dim] views (token / head strides, unit
 * element stride), dtype kv_dtype.  layer_cache: one layer of the paged cache,
 * addressed by element strides (page, K|V, head, slot; unit stride along
 * head_dim): HND [pages, 2, heads, page, D] is (2*H*P*D, H*P*D, P*D, D), NHD
 * [pages, 2, page, heads, D] is (2*P*H*D, P*H*D, D, H*D).  cache_page_slots is the
 * cache's page dimension; page_size divides positions.
 * Token t goes to page kv_indices[pos // page_size] (Python floor division;
 * negative offsets >= -num_indices wrap; page ids in [-num_pages, 0) wrap), slot
 * pos % page_size, K at index 0 and V at index 1, converted to cache_dtype with
 * round-to-nearest-even (a raw copy when the dtypes match).  An offset
 * >= num_indices skips the token and sets BFA_STATUS_APPEND_SKIPPED; any other
 * out-of-range index skips it and sets BFA_STATUS_INDEX_OOB.  Tokens are
 * assumed to target distinct slots.
 * Batched form (kv_indptr != NULL; no single reference function -- it does in
 * one launch what PageManager.append_kv_to_cache does with one call per
 * sequence): token t belongs to sequence batch_indices[t] in [0, num_seqs),
 * whose page table is kv_indices[kv_indptr[s] .. kv_indptr[s+1]) (int32 CSR, as
 * build_paged_kv_indices, kernels/kv_cache_utils.py:81-118, returns it); the
 * rule above applies within that slice.  kv_indptr == NULL: one sequence owning
 * all num_indices entries (batch_indices and num_seqs are ignored). */
int bfa_append_paged_kv(const void* k, const void* v, int kv_dtype, int64_t num_tokens,
                        int64_t num_kv_heads, int64_t head_dim, int64_t k_stride_token,
                        int64_t k_stride_head, int64_t v_stride_token, int64_t v_stride_head,
                        void* layer_cache, int cache_dtype, int64_t num_pages,
                        int64_t cache_page_slots, int64_t stride_page, int64_t stride_kv,
                        int64_t stride_head, int64_t stride_slot, const void* kv_indices,
                        int kv_indices_dtype, int64_t num_indices, const int32_t* kv_indptr,
                        const void* batch_indices, int batch_indices_dtype, int64_t num_seqs,
                        const void* positions, int positions_dtype, int64_t page_size,
                        int32_t* status, void* stream);

/* bfa_fused_rmsnorm_qkv followed by bfa_append_paged_kv of its k and v heads,
 * in one call whose projection epilogue writes the cache itself --
 * kernels/kv_cache_utils.py:9-78 fused into the QKV epilogue, as the page
 * manager appends each layer's k/v right after its QKV projection
 * (engine/page_manager.py:159-218, layers/attention.py:191-205).  No single
 * reference function does both; the result is what the two calls produce:
 * out as bfa_fused_rmsnorm_qkv, then k = out[:, Hq*D : (Hq+Hkv)*D] and
 * v = out[:, (Hq+Hkv)*D :] (as [tokens, Hkv, D], rounded to out_dtype) appended
 * by the rule of bfa_append_paged_kv with `cache_positions` (the tokens'
 * positions in their sequences, which may differ from the RoPE positions).
 * write_kv_out = 0 leaves the k/v columns of out unwritten (q only).  Cache
 * strides must be multiples of 4 elements and the cache 16-byte aligned.
 * workspace: bfa_fused_rmsnorm_qkv_append_workspace_size() bytes (the fused
 * workspace plus tokens x 8 bytes of resolved cache slots). */
int64_t bfa_fused_rmsnorm_qkv_append_workspace_size(int64_t tokens, int64_t hidden,
                                                    int64_t qkv_dim, int64_t head_dim);
int bfa_fused_rmsnorm_qkv_append(
    const void* x, int x_dtype, int64_t tokens, int64_t hidden, int64_t x_stride,
    const void* norm_weight, int nw_dtype, float eps, int mixed_rounding, const void* qkv_weight,
    int w_dtype, int64_t qkv_dim, int64_t w_stride, const void* bias, int bias_dtype,
    int64_t num_q_heads, int64_t num_kv_heads, int qkv_dtype, const void* q_norm_weight,
    const void* k_norm_weight, int qk_norm_dtype, float qk_eps, int qk_norm_out_dtype,
    const void* positions, int positions_dtype, const float* cos_sin_cache, int64_t max_position,
    void* out, int out_dtype, int64_t out_stride, void* workspace, int64_t workspace_bytes,
    void* layer_cache, int cache_dtype, int64_t num_pages, int64_t cache_page_slots,
    int64_t stride_page, int64_t stride_kv, int64_t stride_head, int64_t stride_slot,
    const void* kv_indices, int kv_indices_dtype, int64_t num_indices, const int32_t* kv_indptr,
    const void* batch_indices, int batch_indices_dtype, int64_t num_seqs,
    const void* cache_positions, int cache_positions_dtype, int64_t page_size, int write_kv_out,
    int32_t* status, void* stream);

/* ------------------------------------------------------ cascade attention --
 * online_softmax_update — braidinfer/kernels/online_softmax.py:214-297 (kernel
 * :14-211): updates the running state (m_i [H, B], l_i [H, B], acc_i [H, B, D],
 * fp32, in place) of B queries per head with N keys taken in order:
 *   s = (q . k) * scale; keys with position > the query's skipped when causal;
 *   m' = max(m, s); l = l e^(m-m') + e^(s-m'); acc = acc e^(m-m') + e^(s-m') v.
 * query [H, B, D], key/value [H, N, D]: element strides, unit stride along D
 * (D <= 256); query_positions [B], key_positions [N] int32/int64. */
int bfa_online_softmax_update(const void* query, const void* key, const void* value, int q_dtype,
                              int kv_dtype, float* m_i, float* l_i, float* acc_i,
                              const void* query_positions, int qpos_dtype,
                              const void* key_positions, int kpos_dtype, int64_t num_heads,
                              int64_t batch, int64_t num_tokens, int64_t head_dim,
                              int64_t q_stride_head, int64_t q_stride_batch, int64_t k_stride_head,
                              int64_t k_stride_token, int64_t v_stride_head,
                              int64_t v_stride_token, int64_t m_stride_head,
                              int64_t m_stride_batch, int64_t l_stride_head,
                              int64_t l_stride_batch, int64_t acc_stride_head,
                              int64_t acc_stride_batch, float scale, int apply_causal_mask,
                              void* stream);

/* CascadeAttention.forward — braidinfer/layers/cascade_attention.py:50-231 — in one
 * launch (plus a merge launch when the key range is split).  query [T, Hq, D],
 * D = head_dim = 64 or 128 (bf16/fp16; token / head strides), query_positions
 * [T]; kv_cache one layer of the
 * paged cache, strides (page, K|V, head, slot), K at index 0.  The attended pages
 * are num_entries entries in the reference's walk order (levels, chunks, pages;
 * :112-224), each spanning page_size key positions:
 *   entry_page[e]      page id (int32; a negative id counts from the end, as
 *                      kv_cache[-1] does; out of range sets BFA_STATUS_INDEX_OOB),
 *   entry_key_start[e] key position of the entry's slot 0 (the kv_length of the
 *                      attended chunks before its chunk + page_size x its index
 *                      in the chunk, :199-203),
 *   entry_delta[e]     global - cached position start of its chunk (:153-170),
 *   entry_info[e]      bits 0-15: tokens attended on the page (page_size, or
 *                      kv_last_page_len on a chunk's last page, :131-134), bit 16:
 *                      rotate K by cos_sin_cache[delta] (fp32 [max_position, D];
 *                      a negative delta wraps; out of range sets
 *                      BFA_STATUS_INDEX_OOB).
 * k_norm_weight [D] (optional) applies RMSNorm(eps) to K after the rotation
 * (:175-178).  Query head h attends kv head h / (Hq / Hkv); causal masks keys
 * whose position exceeds the query's.  out [T, Hq * D] (query dtype, token
 * stride out_stride_token) = acc / max(l, 1e-12) (:226-231).  workspace:
 * bfa_cascade_attention_workspace_size bytes. */
int64_t bfa_cascade_attention_workspace_size(int64_t tokens, int64_t num_q_heads,
                                             int64_t num_kv_heads, int64_t head_dim,
                                             int64_t num_entries, int64_t page_size);
int bfa_cascade_attention(const void* query, int dtype, int64_t num_tokens, int64_t num_q_heads,
                          int64_t q_stride_token, int64_t q_stride_head,
                          const void* query_positions, int qpos_dtype, const void* kv_cache,
                          int64_t num_pages, int64_t num_kv_heads, int64_t page_size,
                          int64_t head_dim, int64_t stride_page, int64_t stride_kv,
                          int64_t stride_head, int64_t stride_slot, int64_t num_entries,
                          const int32_t* entry_page, const int64_t* entry_key_start,
                          const int64_t* entry_delta, const int32_t* entry_info,
                          const float* cos_sin_cache, int64_t max_position,
                          const void* k_norm_weight, int k_norm_dtype, float k_norm_eps,
                          float scale, int causal, void* out, int64_t out_stride_token,
                          void* workspace, int64_t workspace_bytes, int32_t* status,
                          void* stream);

/* ------------------------------------------------ linear layer fusions --
 * y = x W^T on the projection GEMM, with the element epilogue fused:
 *   BFA_LINEAR_PLAIN:  y = out_dtype(sum_dtype(proj_dtype(x W^T + bias) + residual))
 *       (bias [n] and residual optional; F.linear of ReplicatedLinear /
 *       ColumnParallelLinear / RowParallelLinear, layers/linear.py:20-61,
 *       136-160, is proj_dtype = out_dtype = x's dtype without residual).  proj_dtype = x's dtype, sum_dtype = F32 gives
 *       residual + F.linear(x, W) in torch's rounding (the o_proj / down_proj
 *       + residual fusion of models/qwen3.py:336-366); proj_dtype = F32,
 *       sum_dtype = F16, out_dtype = x's dtype gives
 *       FusedAttentionOutput.forward (kernels/fused_attention_output.py:
 *       76-134, 173-225), and without residual FusedAttentionOutput.gemv
 *       (:17-72, 137-171).
 *   BFA_LINEAR_SILU_AND_MUL:  weight [2 n, k] = [gate rows; up rows] (the
 *       MergedColumnParallelLinear gate_up_proj, layers/linear.py:63-75);
 *       g, u = proj_dtype(x Wg^T), proj_dtype(x Wu^T);
 *       y = out_dtype(proj_dtype(silu(g)) * u) -- SiluAndMul(F.linear(x, W))
 *       (layers/activation.py:11-13, models/qwen3.py:388-392) without the
 *       [tokens, 2 n] intermediate.
 * x [tokens, k] and weight (row strides x_stride / w_stride, multiples of 8,
 * 16-byte aligned) share a dtype, bf16 or fp16; k a multiple of 16.  out
 * [tokens, n] (row stride out_stride).  workspace: bfa_linear_workspace_size
 * bytes (split-K partials for up to 64 tokens; 0 above). */
enum { BFA_LINEAR_PLAIN = 0, BFA_LINEAR_SILU_AND_MUL = 1 };
int64_t bfa_linear_workspace_size(int64_t tokens, int64_t k, int64_t n, int mode);
int bfa_linear(const void* x, int dtype, int64_t tokens, int64_t k, int64_t x_stride,
               const void* weight, int64_t n, int64_t w_stride, const void* bias, int bias_dtype,
               int mode, int proj_dtype, const void* residual, int residual_dtype, int64_t residual_stride, int sum_dtype,
               void* out, int out_dtype, int64_t out_stride, void* workspace,
               int64_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* BRAIDINFER_AMD_H_ */
