/*
 * tl_attn.h -- C ABI of the MI355X (gfx950) attention hot path of
 * truellm-engine: paged-attention decode (single pass and split-K with a
 * log-sum-exp reduce), reshape_and_cache into the block-table KV pool, the
 * FP8 E4M3 KV variant, the reference KIVI vector codec, paged KIVI INT4 KV
 * and chunked prefill.
 *
 * Conventions
 *  - Plain pointers and sizes; every pointer is device memory unless noted.
 *  - `stream` is a hipStream_t passed as void* (NULL = default stream).
 *    Every call is asynchronous on that stream; nothing here allocates,
 *    frees or synchronises.
 *  - Return value: tl_status (0 = ok).  Bad shapes, NULL pointers, misaligned
 *    buffers and unsupported combinations are reported, never asserted;
 *    tl_last_error_string() describes the last failure of the calling thread.
 *  - KV pools use the reference layout [num_blocks, num_kv_heads, head_size,
 *    block_size] (cache_kernels.cu:74-83), block tables are int32
 *    [num_seqs, max_blocks_per_seq] with -1 for holes, seq_lens int32.
 */
#ifndef TL_ATTN_H
#define TL_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Version of this C ABI (tl_abi_version).  2: tl_kivi_desc gained
 * pre_rope_keys (after bits), for the _pre_rope entry points.  3:
 * tl_prefill_desc gained kv_dtype, k_scale, v_scale.  4: tl_kivi_desc
 * gained build_ahead (after pre_rope_keys).  5: tl_paged_attention_v2_capacity
 * and its plan query. */
#define TL_ABI_VERSION 5

/* Mirrors truellm::ErrorCode (include/truellm/types.h:20-32). */
typedef enum tl_status {
  TL_OK = 0,
  TL_ERR_INVALID_ARGUMENT = 1,
  TL_ERR_NOT_IMPLEMENTED = 3,
  TL_ERR_BACKEND = 5,
  TL_ERR_INTERNAL = 99
} tl_status;

/* F32/F16/BF16 mirror truellm::DataType (include/truellm/types.h:47-60);
 * FP8_E4M3 is OCP E4M3 (max 448), which the reference only sizes for
 * (cuda_allocator.h:179-182). */
typedef enum tl_dtype {
  TL_DTYPE_F32 = 0,
  TL_DTYPE_F16 = 1,
  TL_DTYPE_BF16 = 2,
  TL_DTYPE_FP8_E4M3 = 32
} tl_dtype;

/* Which KV head a q head reads.  MODULO is the reference kernels' mapping
 * (paged_attention_v1.cu:46); GROUPED is the model's (megakernel.cu:271-277). */
typedef enum tl_gqa_map { TL_GQA_MODULO = 0, TL_GQA_GROUPED = 1 } tl_gqa_map;

int tl_abi_version(void);
const char* tl_last_error_string(void);

/* ------------------------------------------------------------------------
 * Paged-attention decode
 * --------------------------------------------------------------------- */

typedef struct tl_decode_desc {
  int32_t num_seqs;            /* S */
  int32_t num_heads;           /* H (q heads); H % num_kv_heads == 0 */
  int32_t num_kv_heads;
  int32_t head_size;           /* 128; 64 / 256 (and 80 / 96 for F16 / BF16 KV) */
  int32_t block_size;          /* head 128: a power of two 8..256 (FP8 too),
                                  F32 KV and other heads: 16 */
  int32_t max_blocks_per_seq;  /* row stride of block_tables */
  int32_t num_blocks;          /* pool capacity N; table entries >= N are holes */
  int32_t q_dtype;             /* q and out: F16, BF16 (or F32 with F32 KV) */
  int32_t kv_dtype;            /* F16, BF16, F32 (= q_dtype) or FP8_E4M3 */
  int32_t gqa_map;             /* tl_gqa_map */
  int32_t partition_tokens;    /* 0 = choose, -1 = single pass, else k*512 */
  float scale;                 /* softmax scale, normally 1/sqrt(head_size) */
  float k_scale, v_scale;      /* FP8 dequant scales (x = code * scale); else ignored */
} tl_decode_desc;

/* CudaEngineConfig's attention knobs (config_schema.h:67-83) onto a decode
 * descriptor whose other fields are filled: paged_kv_block_size (a power
 * of two) goes to desc->block_size; use_fp8_kv != 0 makes the pool FP8 E4M3
 * (desc->kv_dtype; k_scale / v_scale <= 0 become 1), 0 makes it q's type;
 * attention_layout "paged" and "flash_paged" both name the pool layout
 * [N, n_kv, head_size, block_size] these kernels read, which already run an
 * online softmax with split-K (the library's plan unless
 * desc->partition_tokens says otherwise).  Other layout strings, and
 * combinations no kernel is built for, return TL_ERR_NOT_IMPLEMENTED; a
 * block size that is not a power of two TL_ERR_INVALID_ARGUMENT.  A rejected
 * call leaves the descriptor unchanged.  The reference parses these fields
 * (src/host/config/config.cpp:110-134); its engine passes block_size to the
 * kernels and reads neither use_fp8_kv nor attention_layout there. */
int tl_engine_apply_config(tl_decode_desc* desc, int32_t paged_kv_block_size, int32_t use_fp8_kv,
                           const char* attention_layout);

/* Bytes of fp32 workspace tl_paged_attention_decode needs for split-K at
 * max_context_len (0 when it will run single pass). */
size_t tl_paged_attention_workspace_bytes(const tl_decode_desc* desc, int32_t max_context_len);

/* out[s, h, :] = softmax(scale * q[s, h] . K^T) V over seq_lens[s] tokens.
 * q, out: [S, H, head_size] in q_dtype.  A sequence of length 0 gets zeros.
 * workspace may be NULL when the query above returned 0. */
int tl_paged_attention_decode(const tl_decode_desc* desc, void* out, const void* q,
                              const void* k_cache, const void* v_cache,
                              const int32_t* block_tables, const int32_t* seq_lens,
                              int32_t max_context_len, void* workspace,
                              size_t workspace_bytes, void* stream);

/* The engine's decode step in one call: reshape_and_cache of the step's
 * token then paged attention (cuda_engine.cpp:1100-1166), with the result
 * of tl_reshape_and_cache (tl_reshape_and_cache_fp8 for an FP8 pool, with
 * desc's scales) followed by tl_paged_attention_decode, as two launches on
 * the stream: key/value [S, n_kv, head_size] in the pool type (q's type for
 * an FP8 pool), slot_mapping[s] the pool slot of position seq_lens[s] - 1
 * (seq_lens are the lengths after the append; a negative slot writes
 * nothing).  Workspace as tl_paged_attention_workspace_bytes. */
int tl_paged_attention_decode_step(const tl_decode_desc* desc, void* out, const void* q, const void* key,
                                   const void* value, const int32_t* slot_mapping, void* k_cache,
                                   void* v_cache, const int32_t* block_tables, const int32_t* seq_lens,
                                   int32_t max_context_len, void* workspace, size_t workspace_bytes,
                                   void* stream);

/* No counterpart in the reference.  tl_paged_attention_decode for callers
 * that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc): the split-K workspace is
 * a library-owned device array of TL_NOALLOC_SCRATCH_BYTES that each GPU
 * holds until the process ends; the call allocates nothing.  A plan whose
 * workspace exceeds it returns TL_ERR_INVALID_ARGUMENT (query the size
 * with tl_paged_attention_workspace_bytes).  Every call on one GPU shares
 * that GPU's array: calls that overlap on one GPU (two streams or two
 * threads) race. */
#define TL_NOALLOC_SCRATCH_BYTES (32u << 20)
int tl_paged_attention_decode_noalloc(const tl_decode_desc* desc, void* out, const void* q,
                                      const void* k_cache, const void* v_cache,
                                      const int32_t* block_tables, const int32_t* seq_lens,
                                      int32_t max_context_len, void* stream);

/* Replaces paged_attention_v1 (paged_attention_v1.cu:177-213): single pass,
 * same arguments plus the explicit sizes a TrueBuffer carried. */
int tl_paged_attention_v1(void* out, const void* q, const void* k_cache, const void* v_cache,
                          const int32_t* block_tables, const int32_t* seq_lens,
                          int32_t num_seqs, int32_t num_heads, int32_t num_kv_heads,
                          int32_t head_size, int32_t block_size, int32_t max_blocks_per_seq,
                          int32_t num_blocks, float scale, int32_t dtype, int32_t gqa_map,
                          void* stream);

/* Replaces paged_attention_v2 (paged_attention_v2.cu:176-251).  The caller
 * provides scratch exp_sums / max_logits [S, H, P] fp32 and tmp_out
 * [S, H, P, head_size] in dtype, with P at least the partition count of the
 * reference kernel, (max_context_len / block_size + 31) / 32
 * (paged_attention_v2.cu:196); the engine's ceil(max_context_len / (32 *
 * block_size)) (cuda_engine.cpp:276-285,1144) is never less.  The caller
 * reads none of it afterwards.  The call runs the library's own plan (as
 * tl_paged_attention_decode with partition_tokens 0): single pass when the
 * batch fills the GPU, else split-K with the partials kept in that scratch:
 * f16 partial outputs for f16 calls at head size 128 (at most P
 * partitions, P the reference kernel's count), else fp32 (at most
 * P * sizeof(dtype) / 4).  The scratch's contents after the call are not
 * the reference's partials. */
int tl_paged_attention_v2(void* out, float* exp_sums, float* max_logits, void* tmp_out,
                          const void* q, const void* k_cache, const void* v_cache,
                          const int32_t* block_tables, const int32_t* seq_lens,
                          int32_t num_seqs, int32_t num_heads, int32_t num_kv_heads,
                          int32_t head_size, int32_t block_size, int32_t max_blocks_per_seq,
                          int32_t num_blocks, float scale, int32_t dtype, int32_t gqa_map,
                          int32_t max_context_len, void* stream);

/* The plan tl_paged_attention_v2 runs for a call of these sizes (16-byte
 * aligned tmp_out): the number of partitions (1: single pass; -1: the
 * sizes are refused) and, in *partition_tokens, their length (0 for single
 * pass).  No counterpart in the reference (whose v2 always runs
 * (max_context_len / block_size + 31) / 32 partitions of 32 blocks,
 * paged_attention_v2.cu:196); for callers that report or size around it. */
int32_t tl_paged_attention_v2_partitions(int32_t num_seqs, int32_t num_heads, int32_t num_kv_heads,
                                         int32_t head_size, int32_t block_size, int32_t dtype,
                                         int32_t max_context_len, int32_t* partition_tokens);

/* No counterpart in the reference.  tl_paged_attention_v2 for a caller
 * whose scratch holds more partitions than the call's context needs: the
 * engine allocates exp_sums / max_logits / tmp_out once, for
 * ceil(n_ctx_train / (32 * block_size)) partitions (cuda_engine.cpp:273-285),
 * and passes that count as scratch_partitions (at least the reference
 * kernel's count for max_context_len, else TL_ERR_INVALID_ARGUMENT).  The
 * plan may then use up to that many partitions, which a short batch (the
 * engine's one sequence per call) turns into shorter partitions over more
 * CUs.  Results as tl_paged_attention_v2. */
int tl_paged_attention_v2_capacity(void* out, float* exp_sums, float* max_logits, void* tmp_out,
                                   const void* q, const void* k_cache, const void* v_cache,
                                   const int32_t* block_tables, const int32_t* seq_lens,
                                   int32_t num_seqs, int32_t num_heads, int32_t num_kv_heads,
                                   int32_t head_size, int32_t block_size, int32_t max_blocks_per_seq,
                                   int32_t num_blocks, float scale, int32_t dtype, int32_t gqa_map,
                                   int32_t max_context_len, int32_t scratch_partitions, void* stream);
/* Its plan, as tl_paged_attention_v2_partitions (-1: refused sizes). */
int32_t tl_paged_attention_v2_capacity_partitions(int32_t num_seqs, int32_t num_heads, int32_t num_kv_heads,
                                                  int32_t head_size, int32_t block_size, int32_t dtype,
                                                  int32_t max_context_len, int32_t scratch_partitions,
                                                  int32_t* partition_tokens);

/* ------------------------------------------------------------------------
 * KV-cache writes
 * --------------------------------------------------------------------- */

/* Replaces reshape_and_cache (cache_kernels.cu:202-232): key/value
 * [T, n_kv, head_size] -> k_cache/v_cache [N, n_kv, head_size, block_size]
 * at slot_mapping[t] (int32, < 0 skipped, block >= N skipped).  dtype F16,
 * BF16 or F32, same for sources and pools (bit copy).  head_size % 8 == 0.
 * Calls of at most 256 tokens on 16-byte aligned pools rewrite the whole
 * row (head_size x block_size elements) of a block that only one token of
 * the call writes, the other slots with their own bytes: no other writer
 * may touch such a block during the call (a block that a sequence appends
 * to belongs to that sequence). */
int tl_reshape_and_cache(const void* key, const void* value, void* k_cache, void* v_cache,
                         const int32_t* slot_mapping, int32_t num_tokens, int32_t num_kv_heads,
                         int32_t head_size, int32_t block_size, int32_t num_blocks,
                         int32_t dtype, void* stream);

/* FP8 pool variant (the engine's use_fp8_kv, cuda_allocator.h:179-182, with
 * the quantisation of convert_fp8, cache_kernels.cu:181-193):
 * code = e4m3_rne_satfinite(x * (1/scale)), scale 0 treated as 1.
 * src_dtype F16 or BF16. */
int tl_reshape_and_cache_fp8(const void* key, const void* value, int32_t src_dtype,
                             uint8_t* k_cache, uint8_t* v_cache, const int32_t* slot_mapping,
                             int32_t num_tokens, int32_t num_kv_heads, int32_t head_size,
                             int32_t block_size, int32_t num_blocks, float k_scale,
                             float v_scale, void* stream);

/* Replaces convert_fp8 (cache_kernels.cu:181-193, :286-295): out[i] =
 * e4m3(float(in[i]) * scale) for i < n, round to nearest even with
 * saturation to +-448 (NaN stays NaN), the conversion of
 * half_to_fp8e4m3 (fp8_utils.cuh:47-53).  in: F16 (the reference's), BF16
 * or F32; scale multiplies (pass 1 / s for a scale s = absmax / 448). */
int tl_convert_fp8(uint8_t* out, const void* in, int32_t in_dtype, int64_t n, float scale,
                   void* stream);

/* Per-tensor E4M3 scale: *scale_out (device fp32) = absmax(x) / 448, the
 * convention of per_token_fp8_quant_kernel (fp8_gemm.cu:80-84) applied to a
 * whole tensor.  x: n elements of dtype F16, BF16 or F32. */
int tl_fp8_absmax_scale(const void* x, int32_t dtype, int64_t n, float* scale_out,
                        void* stream);

/* Rotary embedding styles.  ADJACENT rotates the pairs (x[2i], x[2i+1]):
 * ggml's LLAMA_ROPE_TYPE_NORM, the engine's rope (cuda_engine.cpp:1100-1108).
 * HALVES rotates (x[i], x[i + d/2]): rope_device.cuh:24-36 (the megakernel). */
typedef enum tl_rope_style { TL_ROPE_ADJACENT = 0, TL_ROPE_HALVES = 1 } tl_rope_style;

/* The write side of a step in one launch: RoPE on q and key with the
 * model's fp32 tables cos_table / sin_table [max_positions, head_size/2]
 * (cuda_model.cpp:269-295: theta = pos / base^(2i/d)), then key and value
 * into the pools as tl_reshape_and_cache does.  Token t sits at position
 * positions[t]; each pair (a, b) becomes, in fp32,
 *   (fmaf(a, c, -(b*s)), fmaf(a, s, b*c)),  c, s = tables[pos][i],
 * rounded once to dtype (F16, BF16 or F32, the dtype of q, key, value and
 * the pools).  q [T, num_heads, d] -> q_out (may be q itself); key/value
 * [T, n_kv, d]; pools [N, n_kv, d, bs]; slot < 0 or past the pool skips the
 * token's pool write.  A token whose position is outside [0, max_positions)
 * is not written at all (q_out rows and pool).  head_size a multiple of 16;
 * num_heads 0 rotates and writes key / value only.  Calls of at most 256
 * tokens on 16-byte aligned pools write key / value as tl_reshape_and_cache
 * does for such calls (whole block rows: no other writer may touch those
 * blocks during the call). */
int tl_rope_reshape_and_cache(const void* q, void* q_out, const void* key, const void* value,
                              void* k_cache, void* v_cache, const int32_t* slot_mapping,
                              const int32_t* positions, const float* cos_table, const float* sin_table,
                              int32_t max_positions, int32_t num_tokens, int32_t num_heads,
                              int32_t num_kv_heads, int32_t head_size, int32_t block_size,
                              int32_t num_blocks, int32_t dtype, int32_t style, void* stream);

/* ------------------------------------------------------------------------
 * KV-cache block management
 * --------------------------------------------------------------------- */

/* Replaces copy_blocks (cache_kernels.cu:234-262, kernel :107-131): for each
 * pair p of block_mapping (device int32 [num_pairs, 2] = {src, dst}), block
 * src of k_cache and of v_cache is copied to block dst of the same pool.  A
 * block is block_bytes bytes (num_kv_heads * head_size * block_size *
 * element size; any dtype, bytes are moved as they are).  Pairs with an id
 * outside [0, num_blocks) are skipped (the reference's kernel writes out of
 * bounds).  A dst must not be the src or dst of another pair of the call
 * (the pairs run concurrently, as in the reference). */
int tl_copy_blocks(void* k_cache, void* v_cache, const int32_t* block_mapping, int32_t num_pairs,
                   int32_t num_blocks, int64_t block_bytes, void* stream);

/* Replaces swap_blocks (cache_kernels.cu:264-284, kernel :133-167): whole
 * blocks between a device pool and a host buffer in pinned memory
 * (hipHostMalloc).  direction 0: device block src -> host block dst; 1: host
 * block src -> device block dst.  block_bytes as for tl_copy_blocks (the
 * reference sizes it from shape[4] of a 4-D view, defect D16).  Ids outside
 * [0, num_device_blocks) / [0, num_host_blocks) skip the pair. */
int tl_swap_blocks(void* cache, void* host_cache, const int32_t* block_mapping, int32_t num_pairs,
                   int32_t num_device_blocks, int32_t num_host_blocks, int64_t block_bytes,
                   int32_t direction, void* stream);

/* ------------------------------------------------------------------------
 * Norms and gated activations (layernorm_kernels.cu, activation_kernels.cu)
 * --------------------------------------------------------------------- */

/* Replaces rms_norm (layernorm_kernels.cu:149-167, kernel :28-56): for each
 * of num_tokens rows of x [num_tokens, hidden_size], out = x *
 * (1 / sqrt(sum(x^2) / hidden_size + eps)) * weight, in fp32, rounded once
 * to dtype (F16, BF16 or F32 for x, weight and out).  The total is taken
 * over the whole row for every element (the reference's block reduction
 * leaves it in warp 0 only, defect D4). */
int tl_rms_norm(void* out, const void* x, const void* weight, int32_t num_tokens, int32_t hidden_size,
                float eps, int32_t dtype, void* stream);

/* Replaces fused_add_rms_norm (layernorm_kernels.cu:169-189, kernel
 * :64-94): r = residual + x; residual = dtype(r) in place; the mean square
 * over the fp32 r; out = float(residual) * (1 / sqrt(...)) * weight. */
int tl_fused_add_rms_norm(void* out, void* residual, const void* x, const void* weight, int32_t num_tokens,
                          int32_t hidden_size, float eps, int32_t dtype, void* stream);

/* Replaces layer_norm (layernorm_kernels.cu:191-211, kernel :102-139):
 * out = (x - mean) * (1 / sqrt(var + eps)) * weight + bias, var the mean of
 * (x - mean)^2 (two passes over the row). */
int tl_layer_norm(void* out, const void* x, const void* weight, const void* bias, int32_t num_tokens,
                  int32_t hidden_size, float eps, int32_t dtype, void* stream);

/* Gated activations (activation_kernels.cu:57-132). */
typedef enum tl_activation { TL_ACT_SILU = 0, TL_ACT_GELU = 1, TL_ACT_GELU_TANH = 2 } tl_activation;

/* Replaces silu_and_mul / gelu_and_mul / gelu_tanh_and_mul: out[i] =
 * dtype(act(gate[i])) * up[i], over n elements of gate, up and out; the
 * activation is rounded to dtype before the product, as the reference's
 * act() returns the storage type. */
int tl_act_and_mul(void* out, const void* gate, const void* up, int64_t n, int32_t activation, int32_t dtype,
                   void* stream);

/* ------------------------------------------------------------------------
 * VQ codec of the KV cache (vq_cache.cu, codebook_init.cu)
 * --------------------------------------------------------------------- */

#define TL_VQ_MAX_HEAD_DIM 256

/* Replaces vq_encode (vq_cache.cu:74-86, kernel :18-43): idx[v] (uint16) =
 * the codebook entry nearest to vector v of kv [num_vecs, head_dim] fp16
 * (num_vecs = seq_len * n_kv_heads), by the reference's fp32 distance
 * (sequential over d, fma per term); the lowest index wins ties, NaN and
 * >= FLT_MAX distances never win (all of them: 0).  book [codebook_size,
 * head_dim] fp16.  head_dim a multiple of 8, at most TL_VQ_MAX_HEAD_DIM;
 * 1 <= codebook_size <= 65536. */
int tl_vq_encode(const void* kv, const void* book, uint16_t* idx, int32_t num_vecs, int32_t head_dim,
                 int32_t codebook_size, void* stream);

/* Replaces vq_decode (vq_cache.cu:88-100, kernel :48-69): kv_out[v] =
 * book[idx[v]] (bit copies; kv_out may be the encoded tensor).  A row whose
 * index is >= codebook_size is left as it is (the reference reads past the
 * codebook). */
int tl_vq_decode(void* kv_out, const void* book, const uint16_t* idx, int32_t num_vecs, int32_t head_dim,
                 int32_t codebook_size, void* stream);

/* Workspace of tl_vq_kmeans (caller-owned; the reference allocates and frees
 * temporaries on every call). */
size_t tl_vq_kmeans_workspace_bytes(int32_t n_samples, int32_t codebook_size, int32_t head_dim);

/* Replaces codebook_init_kmeans (codebook_init.cu:100-145): n_iterations
 * Lloyd iterations over data [n_samples, head_dim] fp16, updating the
 * pre-seeded book in place: assign as tl_vq_encode; each centroid becomes
 * fp16(fp32(sum) * (1/count)) of its members, an empty cluster keeps its
 * centroid.  The sums are exact (int64 fixed point in units of 2^-24, NaN /
 * +inf / -inf tracked with IEEE sum rules), so the result does not depend on
 * the order of the atomic adds, unlike the reference's fp32 atomics.
 * Asynchronous; no allocation. */
int tl_vq_kmeans(const void* data, void* book, int32_t n_samples, int32_t codebook_size, int32_t head_dim,
                 int32_t n_iterations, void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------
 * Reference KIVI vector codec (kivi_cache.cuh:27-84, kivi_cache.cu:23-239)
 * --------------------------------------------------------------------- */

#define TL_KIVI_MAX_HEAD_DIM 128
#define TL_KIVI_MAX_OUTLIERS 64

/* Record stride of one compressed vector: 3*n_outliers +
 * ceil((head_dim - n_outliers) / group_size) * (group_size/2 + 4)
 * (kivi_compressed_bytes, kivi_cache.cuh:32-43). */
size_t tl_kivi_compressed_bytes(int32_t head_dim, int32_t n_outliers, int32_t group_size);

/* 1 iff 0 < head_dim <= 128, 0 <= n_outliers <= 64, n_outliers <= head_dim
 * and group_size > 0 (kivi_params_supported, kivi_cache.cu:205-211). */
int tl_kivi_params_supported(int32_t head_dim, int32_t n_outliers, int32_t group_size);

/* Replace kivi_compress / kivi_decompress (kivi_cache.cu:213-239): kv fp16
 * [n_vecs, head_dim] <-> records u8 [n_vecs, stride], bit-exact with the
 * reference.  Unsupported parameters and odd group sizes (whose records
 * overrun the reference's stride) return TL_ERR_INVALID_ARGUMENT and touch
 * nothing; n_vecs == 0 is a no-op. */
int tl_kivi_compress(const void* kv_in, uint8_t* out, int32_t n_vecs, int32_t head_dim,
                     int32_t n_outliers, int32_t group_size, void* stream);
int tl_kivi_decompress(const uint8_t* in, void* kv_out, int32_t n_vecs, int32_t head_dim,
                       int32_t n_outliers, int32_t group_size, void* stream);

/* ------------------------------------------------------------------------
 * Paged KIVI INT4 / INT8 KV: K per channel and V per token, groups of 32,
 * fp16 step/zero, codes of desc->bits bits, the most recent residual_length tokens
 * (plus up to 31 more) kept in the fp16 pool (KiviConfig, config_schema.h:
 * 122-129, which the reference declares but never implements).
 * A sequence of length L holds its first
 *   Lq = L <= R ? 0 : floor((L - R) / 32) * 32
 * tokens in pages; page p covers tokens [32p, 32p + 32).  Pages live in a
 * pool [num_pages, num_kv_heads, 5120 B] addressed by page_tables
 * [num_seqs, max_pages_per_seq]; the fp16 pool keeps every token.
 * --------------------------------------------------------------------- */

#define TL_KIVI_PAGE_TOKENS 32
#define TL_KIVI_PAGE_BYTES 5120   /* per kv head, head_size 128 */

typedef struct tl_kivi_desc {
  int32_t num_seqs;
  int32_t num_heads;
  int32_t num_kv_heads;
  int32_t head_size;           /* 128 */
  int32_t block_size;          /* fp16 pool block size: a power of two 8..256 */
  int32_t max_blocks_per_seq;
  int32_t num_blocks;
  int32_t max_pages_per_seq;
  int32_t num_pages;
  int32_t residual_length;     /* R >= 0 */
  int32_t gqa_map;
  int32_t partition_pages;     /* 0 = choose, -1 = single pass, else pages per partition; the
                                  _pre_rope entry points take at most 160 pages per partition
                                  at INT4, 144 at INT8 (the page rotations a workgroup holds in
                                  LDS), a single pass included */
  float scale;
  int32_t bits;                /* code width of the pages (KiviConfig.bits, config_schema.h:124):
                                  4 (also 0) or 8 */
  int32_t pre_rope_keys;       /* KiviConfig.pre_rope_keys (config_schema.h:128): 0 = keys are
                                  stored and quantised as attention scores them; 1 = keys are held
                                  before RoPE and rotated at their positions inside attention (the
                                  _pre_rope entry points, which take the tables) */
  int32_t build_ahead;         /* 0: a step (tl_kivi_decode_step*, tl_kivi_append) whose length
                                  completes a page quantises the whole page.  1 (used when
                                  residual_length > 8): each of the 8 steps before that one
                                  writes an eighth of it (K channels of 4 octets, or V tokens of
                                  one lane group), so no step quantises a whole page, and
                                  tl_kivi_build_pages also builds the next page once its first
                                  eighth is due.  The bytes are the same.  Contract: the page
                                  table entry of a sequence's next page is set from the first
                                  of those calls on (a page allocated later than that stays
                                  incomplete), and every call that appends to the sequence
                                  uses the same setting. */
} tl_kivi_desc;

/* Page bytes per kv head for a code width: 5120 (INT4, also bits 0) or 9216
 * (INT8: the INT4 layout with every 16-byte code chunk widened to 32 bytes);
 * 0 for any other width. */
#define TL_KIVI_PAGE_BYTES_INT8 9216
size_t tl_kivi_page_bytes(int32_t bits);

int32_t tl_kivi_quantized_len(int32_t seq_len, int32_t residual_length);

/* Quantise every page of every sequence's prefix (tokens < Lq(seq_lens[s]))
 * from the fp16 pools.  Bit-exact with the reference quantiser. */
int tl_kivi_build_pages(const tl_kivi_desc* desc, const void* k_cache, const void* v_cache,
                        const int32_t* block_tables, const int32_t* seq_lens,
                        const int32_t* page_tables, void* pages, int32_t max_context_len,
                        void* stream);

/* Append one token per sequence: key/value fp16 [S, n_kv, 128] go to the
 * fp16 pools at slot_mapping[s] (as tl_reshape_and_cache), then every
 * sequence whose new length seq_lens[s] completes a page (Lq grows) has that
 * page quantised. */
int tl_kivi_append(const tl_kivi_desc* desc, const void* key, const void* value, void* k_cache,
                   void* v_cache, const int32_t* slot_mapping, const int32_t* block_tables,
                   const int32_t* seq_lens, const int32_t* page_tables, void* pages,
                   void* stream);

/* Split-K partials of the decode and the step: 0 when the plan runs a
 * single pass.  Sized for the _pre_rope entry points' plan (as many
 * partitions as the other one, or more past 160 / 144 pages), so one size
 * serves every entry point. */
size_t tl_kivi_workspace_bytes(const tl_kivi_desc* desc, int32_t max_context_len);

/* Decode attention over pages (tokens < Lq) and the fp16 pool (tokens >= Lq).
 * q, out fp16 [S, H, 128]. */
int tl_kivi_paged_attention_decode(const tl_kivi_desc* desc, void* out, const void* q,
                                   const void* pages, const int32_t* page_tables,
                                   const void* k_cache, const void* v_cache,
                                   const int32_t* block_tables, const int32_t* seq_lens,
                                   int32_t max_context_len, void* workspace,
                                   size_t workspace_bytes, void* stream);

/* One KIVI decode step in one call, with the result of tl_kivi_append then
 * tl_kivi_paged_attention_decode (seq_lens are the lengths after the append)
 * byte for byte, in one decode launch (plus the log-sum-exp reduce when
 * split): the new token's attention reads it from key/value, and the page it
 * completes is built in the same launch.  slot_mapping[s] must be the pool
 * slot of position seq_lens[s] - 1 in block_tables, as an append step's slot
 * is; a negative slot writes nothing and that position is read from the
 * pool, as the two calls would.  The token is stored by rewriting its
 * block's rows of each kv head (128 channels x 16 slots; the other slots
 * keep their bytes), so no other writer may touch that block during the
 * call: a block that a sequence appends to belongs to that sequence. */
int tl_kivi_decode_step(const tl_kivi_desc* desc, void* out, const void* q, const void* key,
                        const void* value, const int32_t* slot_mapping, void* pages,
                        const int32_t* page_tables, void* k_cache, void* v_cache,
                        const int32_t* block_tables, const int32_t* seq_lens, int32_t max_context_len,
                        void* workspace, size_t workspace_bytes, void* stream);

/* The KIVI decode step with RoPE first: RoPE (style TL_ROPE_ADJACENT or
 * TL_ROPE_HALVES, fp32 tables [max_positions, 64], position positions[s])
 * of q [S, H, 128] and of the new keys [S, n_kv, 128], then
 * tl_kivi_decode_step on the rotated q and keys, which are stored and
 * quantised rotated: the order KiviConfig.pre_rope_keys = false names
 * (config_schema.h:128), and the order of the engine's decode step, whose
 * ggml rope precedes reshape_and_cache (cuda_engine.cpp:1100-1130).  The
 * rotation is that of tl_rope_reshape_and_cache; a position outside the
 * tables leaves that sequence's q and key unrotated.  Two launches (the
 * rotation into the workspace, then the step); the workspace holds the
 * step's split-K partials and the rotated rows: see
 * tl_kivi_rope_step_workspace_bytes.  With desc->pre_rope_keys = 1 only q
 * is rotated here and the step is tl_kivi_decode_step_pre_rope on the same
 * tables (the keys stored unrotated, rotated at token position t inside
 * attention), so positions[s] should be seq_lens[s] - 1. */
size_t tl_kivi_rope_step_workspace_bytes(const tl_kivi_desc* desc, int32_t max_context_len);
int tl_kivi_rope_decode_step(const tl_kivi_desc* desc, void* out, const void* q, const void* key,
                             const void* value, const int32_t* positions, const float* cos_table,
                             const float* sin_table, int32_t max_positions, int32_t style,
                             const int32_t* slot_mapping, void* pages, const int32_t* page_tables,
                             void* k_cache, void* v_cache, const int32_t* block_tables,
                             const int32_t* seq_lens, int32_t max_context_len, void* workspace,
                             size_t workspace_bytes, void* stream);

/* Keys held before RoPE (desc->pre_rope_keys = 1): the decode and the
 * decode step of tl_kivi_paged_attention_decode / tl_kivi_decode_step with
 * every key rotated at its position in the sequence (token t of a sequence
 * at position t, style TL_ROPE_ADJACENT or TL_ROPE_HALVES, fp32 tables
 * [max_positions, 64], 16-byte aligned, covering every position:
 * max_positions >= max_context_len, else TL_ERR_INVALID_ARGUMENT) as it is
 * scored: a page key after its dequantisation, a window key as read from
 * the fp16 pool, the step's new key as given.  A page key of position
 * t = 32 p + j is scored with the rotation of 32 p applied to q and that of
 * j to the key (R_t = R_32p R_j: exact for tables of angles linear in the
 * position, as RoPE's theta_i t are; the products run in f16).  Pages,
 * pools and the appended token hold the keys unrotated.  q is taken as
 * given (rotated by the caller at position seq_lens[s] - 1).  The standard
 * entry points refuse a descriptor with pre_rope_keys set, since they would
 * score unrotated keys. */
int tl_kivi_paged_attention_decode_pre_rope(const tl_kivi_desc* desc, void* out, const void* q,
                                            const void* pages, const int32_t* page_tables,
                                            const void* k_cache, const void* v_cache,
                                            const int32_t* block_tables, const int32_t* seq_lens,
                                            int32_t max_context_len, const float* cos_table,
                                            const float* sin_table, int32_t max_positions, int32_t style,
                                            void* workspace, size_t workspace_bytes, void* stream);
int tl_kivi_decode_step_pre_rope(const tl_kivi_desc* desc, void* out, const void* q, const void* key,
                                 const void* value, const int32_t* slot_mapping, void* pages,
                                 const int32_t* page_tables, void* k_cache, void* v_cache,
                                 const int32_t* block_tables, const int32_t* seq_lens,
                                 int32_t max_context_len, const float* cos_table, const float* sin_table,
                                 int32_t max_positions, int32_t style, void* workspace,
                                 size_t workspace_bytes, void* stream);

/* KiviConfig (config_schema.h:122-129) onto a descriptor: bits (4 or 8),
 * residual_length and pre_rope_keys (0 or 1) go to desc->bits /
 * desc->residual_length / desc->pre_rope_keys.  The pages hold keys per
 * channel and values per token, so key_granularity must be "per_channel"
 * and value_granularity "per_token" (the defaults); other strings return
 * TL_ERR_NOT_IMPLEMENTED.  pre_rope_keys = 0 is the order of
 * tl_kivi_rope_decode_step without the flag (and of any caller that stores
 * rotated keys); pre_rope_keys = 1 keeps keys unrotated in pages and pools
 * and rotates them inside attention (the _pre_rope entry points, and
 * tl_kivi_rope_decode_step with the flag).  The reference parses these
 * fields (src/host/config/config.cpp:216-223) but no kernel of it reads
 * them. */
int tl_kivi_apply_config(tl_kivi_desc* desc, int32_t bits, int32_t residual_length,
                         const char* key_granularity, const char* value_granularity,
                         int32_t pre_rope_keys);

/* ---- host-side helpers of the path's callers (no device work) ----------- */

/* The engine's attention dispatch (cuda_engine.cpp:1138-1160): v2 iff
 * max_context_len / block_size > 32, with ceil(max_context_len / (32 bs))
 * partitions; scale = 1/sqrt(head_size). */
int tl_attention_plan(int32_t max_context_len, int32_t block_size, int32_t head_size,
                      int32_t* use_v2, int32_t* num_partitions, float* scale);

/* The allocator's bounds and tables (cuda_allocator.cpp:76, :231-253, :255-280):
 * max_blocks_per_seq = min(num_blocks, 2048); a block-table row is the
 * sequence's blocks followed by -1 up to max_blocks_per_seq; token
 * seq_start_pos + i of a sequence goes to slot blocks[pos / bs] * bs + pos % bs.
 * tl_build_block_tables fills a [num_seqs, max_blocks_per_seq] batch from
 * the concatenated per-sequence lists (block_offsets[num_seqs + 1]). */
int32_t tl_max_blocks_per_seq(int32_t num_blocks);
int tl_build_block_tables(const int32_t* blocks, const int32_t* block_offsets, int32_t num_seqs,
                          int32_t max_blocks_per_seq, int32_t* tables);
int tl_build_slot_mapping(const int32_t* blocks, int32_t num_blocks_of_seq, int32_t block_size,
                          int32_t seq_start_pos, int32_t num_tokens, int32_t* slots);

/* KvCompressionPass's KIVI settings (kv_compression_pass.cpp:29-66, :184-216):
 * n_outliers = residual_length, group_size = bits == 4 ? 16 : 8, enabled only
 * when kivi_params_supported; a layer is compressed in place only when
 * seq_len > 0 and seq_len * n_kv_heads records fit the scratch bytes. */
int tl_kivi_pass_params(int32_t residual_length, int32_t bits, int32_t head_dim, int32_t* n_outliers,
                        int32_t* group_size, int32_t* enabled);
int32_t tl_kivi_pass_runs(int32_t seq_len, int32_t n_kv_heads, int32_t head_dim, int32_t n_outliers,
                          int32_t group_size, size_t scratch_bytes);

/* ---- chunked prefill (causal) + decode rows in one call -----------------
 * No reference counterpart: the reference's prefill runs per token
 * (cuda_engine.cpp:842-860) or densely in the megakernel
 * (megakernel.cu:267-351).  Mixed batch: sequence s owns query rows
 * cu_q_lens[s] .. cu_q_lens[s+1]-1 of q/out [total_q, H, 128]; its length
 * after the chunk is seq_lens[s] (the chunk's own K/V already written to the
 * pool with tl_reshape_and_cache); query i sits at position
 * seq_lens[s] - q_len + i and attends causally to keys 0 .. that position.
 * q_len == 1 rows are decode rows (a second kernel on the same stream).
 * head_size 128, block_size any power of two 8..256 (CudaEngineConfig's
 * paged_kv_block_size, config_schema.h:68), dtype F16 or BF16 for q and out;
 * the pool holds dtype, or FP8 E4M3 codes with per-tensor scales
 * (use_fp8_kv, config_schema.h:72; cuda_allocator.h:179-182).  q and the
 * pools 16-byte aligned, out 4-byte aligned.  max_q_len (host) bounds the
 * grid; max_q_len x (num_heads / num_kv_heads) must stay below 2^22 - 256
 * (TL_ERR_NOT_IMPLEMENTED otherwise). */
typedef struct tl_prefill_desc {
  int32_t num_seqs;
  int32_t num_heads;
  int32_t num_kv_heads;
  int32_t head_size;           /* 128 */
  int32_t block_size;          /* a power of two 8..256 */
  int32_t max_blocks_per_seq;
  int32_t num_blocks;
  int32_t dtype;               /* TL_DTYPE_F16 or TL_DTYPE_BF16: q and out */
  int32_t gqa_map;
  int32_t num_prefill_seqs;    /* 0: any sequence may be either kind; n > 0: sequences
                                  0..n-1 hold every q_len > 1 row, n.. only q_len <= 1 */
  float scale;
  int32_t kv_dtype;            /* the pool: 0 or dtype, or TL_DTYPE_FP8_E4M3 */
  float k_scale, v_scale;      /* FP8 pools: the per-tensor dequant scales (> 0) */
} tl_prefill_desc;

int tl_chunked_prefill(const tl_prefill_desc* desc, void* out, const void* q,
                       const int32_t* cu_q_lens, const void* k_cache, const void* v_cache,
                       const int32_t* block_tables, const int32_t* seq_lens,
                       int32_t total_q, int32_t max_q_len, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TL_ATTN_H */
