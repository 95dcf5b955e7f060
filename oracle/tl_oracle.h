/*
 * tl_oracle.h -- CPU oracle for the truellm-engine attention hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker: tests/,
 * __graft_entry__.smoke() and the cpu_baseline leg of bench.py load it to
 * compute expected results.  The product path (truellm-engine_amd/) never
 * links, loads or calls it.
 *
 * Every function restates the reference's algorithm on the CPU in plain C.
 * Attention is accumulated in double; codecs follow the reference's fp32
 * IEEE arithmetic step by step so that they are bit-exact.
 *
 * Data type codes (first three mirror truellm::DataType, include/truellm/types.h:47-60):
 *   0 = F32, 1 = F16, 2 = BF16, 32 = FP8 E4M3 (OCP "E4M3FN").
 * GQA maps: 0 = MODULO (kv_head = head % n_kv, paged_attention_v1.cu:46),
 *           1 = GROUPED (kv_head = head / (n_heads / n_kv), megakernel.cu:271-277).
 */
#ifndef TL_ORACLE_H
#define TL_ORACLE_H
#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { ORC_F32 = 0, ORC_F16 = 1, ORC_BF16 = 2, ORC_FP8 = 32 };
enum { ORC_GQA_MODULO = 0, ORC_GQA_GROUPED = 1 };

/* ---- scalar conversions ------------------------------------------------ */
uint16_t orc_f32_to_f16(float f);
float    orc_f16_to_f32(uint16_t h);
uint16_t orc_f32_to_bf16(float f);
float    orc_bf16_to_f32(uint16_t h);
uint8_t  orc_f32_to_e4m3(float f);   /* RNE, saturate to +-448, NaN -> 0x7F|sign */
float    orc_e4m3_to_f32(uint8_t v);

/* Element-wise array conversion between any two of the codes above.  FP8
 * destinations use e4m3(x * mul) (fp8_utils.cuh:47-49 convention); FP8
 * sources return float(code) * mul. */
void orc_convert(const void* src, int src_dtype, void* dst, int dst_dtype,
                 int64_t n, float mul);

/* ---- reshape_and_cache (cache_kernels.cu:47-94) ------------------------ */
/* key/value [T, n_kv, d] of elem_bytes each; k_cache/v_cache
 * [N, n_kv, d, bs]; slot < 0 is skipped.  Pure byte copy. */
void orc_reshape_and_cache(const void* key, const void* value,
                           void* k_cache, void* v_cache,
                           const int32_t* slot_mapping, int num_tokens,
                           int num_kv_heads, int head_size, int block_size,
                           int elem_bytes);
/* FP8 variant: e4m3(float(x) * (1/k_scale)) from f16/bf16 sources. */
void orc_rope_reshape_and_cache(const void* q, void* q_out, const void* key, const void* value,
                                void* k_cache, void* v_cache, const int32_t* slot_mapping,
                                const int32_t* positions, const float* cos_table, const float* sin_table,
                                int max_positions, int num_tokens, int num_heads, int num_kv_heads,
                                int head_size, int block_size, int num_blocks, int dtype, int style);
void orc_rms_norm(void* out, void* residual, const void* x, const void* w, int rows, int hidden, float eps,
                  int dtype);
void orc_layer_norm(void* out, const void* x, const void* w, const void* b, int rows, int hidden, float eps,
                    int dtype);
void orc_act_and_mul(void* out, const void* gate, const void* up, int64_t n, int act, int dtype);
void orc_vq_encode(const uint16_t* kv, const uint16_t* book, uint16_t* idx, int64_t num_vecs, int head_dim,
                   int codebook_size);
void orc_vq_decode(uint16_t* out, const uint16_t* book, const uint16_t* idx, int64_t num_vecs, int head_dim,
                   int codebook_size);
void orc_vq_kmeans(const uint16_t* data, uint16_t* book, int64_t n, int codebook_size, int head_dim,
                   int iterations);
void orc_copy_blocks(void* k_cache, void* v_cache, const int32_t* mapping, int num_pairs,
                     int num_blocks, int64_t block_bytes);
void orc_swap_blocks(void* cache, void* host_cache, const int32_t* mapping, int num_pairs,
                     int num_device_blocks, int num_host_blocks, int64_t block_bytes, int direction);
void orc_reshape_and_cache_fp8(const void* key, const void* value, int src_dtype,
                               uint8_t* k_cache, uint8_t* v_cache,
                               const int32_t* slot_mapping, int num_tokens,
                               int num_kv_heads, int head_size, int block_size,
                               float k_scale, float v_scale);

/* ---- paged attention, intended semantics ------------------------------- */
/* out [S, H, d] double.  partition_tokens == 0: one exact softmax per
 * (seq, head); > 0: per-partition (max, sum, out) then a log-sum-exp merge
 * (the algorithm of paged_attention_v2.cu:31-170 without its defects).
 * Table entries < 0 are skipped (paged_attention_v1.cu:76).  A sequence
 * with no valid token yields zeros. */
void orc_paged_attention(double* out, const void* q, int q_dtype,
                         const void* k_cache, const void* v_cache, int kv_dtype,
                         float k_scale, float v_scale,
                         const int32_t* block_tables, int max_blocks_per_seq,
                         const int32_t* seq_lens, int num_seqs, int num_heads,
                         int num_kv_heads, int head_size, int block_size,
                         float scale, int gqa_map, int partition_tokens);

/* fp32-accumulate version used as the timed CPU baseline; threads over
 * (seq, kv_head).  out is written in out_dtype (F16/BF16/F32). */
void orc_paged_attention_f32(void* out, int out_dtype, const void* q, int q_dtype,
                             const void* k_cache, const void* v_cache, int kv_dtype,
                             float k_scale, float v_scale,
                             const int32_t* block_tables, int max_blocks_per_seq,
                             const int32_t* seq_lens, int num_seqs, int num_heads,
                             int num_kv_heads, int head_size, int block_size,
                             float scale, int gqa_map, int num_threads);

/* The paged KIVI attention of orc_kivi_paged_attention_bits in fp32 (the
 * CPU baseline), threads over (seq, kv_head); fp16 q and out. */
void orc_kivi_paged_attention_f32(uint16_t* out, const uint16_t* q, const uint8_t* pages,
                                  const int32_t* page_tables, int max_pages, int num_pages,
                                  const uint16_t* k_cache, const uint16_t* v_cache,
                                  const int32_t* block_tables, int max_blocks_per_seq,
                                  const int32_t* seq_lens, int num_seqs, int num_heads,
                                  int num_kv_heads, int block_size, int residual_length,
                                  float scale, int gqa_map, int bits, int num_threads);

/* Bug-for-bug restatement of paged_attention_v1 (paged_attention_v1.cu:31-135)
 * with fp32 arithmetic, used only to document how far the reference's
 * literal output is from attention.  out [S, H, d] float; untouched when
 * seq_len == 0 (the reference writes nothing). */
void orc_paged_attention_literal_v1(float* out, const void* q, const void* k_cache,
                                    const void* v_cache, int dtype,
                                    const int32_t* block_tables, int max_blocks_per_seq,
                                    const int32_t* seq_lens, int num_seqs, int num_heads,
                                    int num_kv_heads, int head_size, int block_size,
                                    float scale);

/* ---- chunked prefill (causal), intended semantics ---------------------- */
/* q [total_q, H, d]; query i of sequence s sits at absolute position
 * seq_lens[s] - q_len_s + i and sees keys 0..that position; q_len_s =
 * cu_q_lens[s+1] - cu_q_lens[s].  out [total_q, H, d] double. */
void orc_chunked_prefill(double* out, const void* q, int q_dtype,
                         const int32_t* cu_q_lens, const void* k_cache,
                         const void* v_cache, int kv_dtype,
                         const int32_t* block_tables, int max_blocks_per_seq,
                         const int32_t* seq_lens, int num_seqs, int num_heads,
                         int num_kv_heads, int head_size, int block_size,
                         float scale, int gqa_map);

/* ---- reference KIVI vector codec (kivi_cache.cu / kivi_cache.cuh) ------ */
size_t orc_kivi_compressed_bytes(int head_dim, int n_outliers, int group_size);
int    orc_kivi_params_supported(int head_dim, int n_outliers, int group_size);
void   orc_kivi_compress(const uint16_t* in, uint8_t* out, int n_vecs,
                         int head_dim, int n_outliers, int group_size);
void   orc_kivi_decompress(const uint8_t* in, uint16_t* out, int n_vecs,
                           int head_dim, int n_outliers, int group_size);

/* One group of the KIVI quantiser (kivi_cache.cu:92-124): q[n] nibbles,
 * fp16 step and zero. */
void orc_kivi_quant_group(const float* x, int n, uint8_t* q,
                          uint16_t* step, uint16_t* zero);

/* ---- paged KIVI INT4 (per-channel K, per-token V, 32-token pages) ------ */
#define ORC_KIVI_PAGE_TOKENS 32
#define ORC_KIVI_PAGE_BYTES  5120   /* head_size 128 */
/* k_tok, v_tok: [32][128] fp16 of one kv head; page: 5120 bytes. */
void orc_kivi_page_quantize(const uint16_t* k_tok, const uint16_t* v_tok, uint8_t* page);
void orc_kivi_page_dequant(const uint8_t* page, uint16_t* k_tok, uint16_t* v_tok);
/* Number of tokens held in pages for a sequence of length L. */
int  orc_kivi_quantized_len(int seq_len, int residual_length);

/* ---- paged KIVI INT8 (the INT4 page with 32-byte code chunks) --------- */
#define ORC_KIVI_PAGE_BYTES_INT8 9216
size_t orc_kivi_page_bytes(int bits);
/* The group quantiser with `levels` code steps (15: INT4, 255: INT8). */
void orc_kivi_quant_group_levels(const float* x, int n, int levels, uint8_t* q, uint16_t* step,
                                 uint16_t* zero);
void orc_kivi_page_quantize_bits(const uint16_t* k_tok, const uint16_t* v_tok, uint8_t* page, int bits);
void orc_kivi_page_dequant_bits(const uint8_t* page, uint16_t* k_tok, uint16_t* v_tok, int bits);
void orc_kivi_build_pages_bits(const uint16_t* k_cache, const uint16_t* v_cache,
                               const int32_t* block_tables, int max_blocks_per_seq,
                               const int32_t* seq_lens, int num_seqs, int num_kv_heads,
                               int block_size, int residual_length,
                               uint8_t* pages, const int32_t* page_tables, int max_pages,
                               int num_pages, int bits);
void orc_kivi_paged_attention_bits(double* out, const void* q, int q_dtype,
                                   const uint8_t* pages, const int32_t* page_tables,
                                   int max_pages, int num_pages, const uint16_t* k_cache,
                                   const uint16_t* v_cache, const int32_t* block_tables,
                                   int max_blocks_per_seq, const int32_t* seq_lens,
                                   int num_seqs, int num_heads, int num_kv_heads,
                                   int block_size, int residual_length, float scale,
                                   int gqa_map, int bits);

/* Build every page of a batch from an fp16 paged cache: pages
 * [num_pages][n_kv][5120]; page_tables [S, max_pages].  Page-table entries
 * outside [0, num_pages) are skipped; tokens whose block-table entry is
 * negative are quantised as zeros. */
void orc_kivi_build_pages(const uint16_t* k_cache, const uint16_t* v_cache,
                          const int32_t* block_tables, int max_blocks_per_seq,
                          const int32_t* seq_lens, int num_seqs, int num_kv_heads,
                          int block_size, int residual_length,
                          uint8_t* pages, const int32_t* page_tables, int max_pages,
                          int num_pages);

/* Attention over the KIVI cache: pages (dequantized per the format) for
 * tokens < Lq, the fp16 paged cache for tokens >= Lq.  Page-table entries
 * outside [0, num_pages) and negative block-table entries are holes whose
 * tokens are skipped.  out double. */
/* orc_kivi_paged_attention_bits with the keys held before RoPE: each key
 * rotated by its position (fp32 tables [max_pos, 64], style 0 adjacent
 * pairs, 1 halves) before the scores. */
void orc_kivi_paged_attention_pre_rope(double* out, const void* q, int q_dtype,
                                       const uint8_t* pages, const int32_t* page_tables,
                                       int max_pages, int num_pages, const uint16_t* k_cache,
                                       const uint16_t* v_cache, const int32_t* block_tables,
                                       int max_blocks_per_seq, const int32_t* seq_lens,
                                       int num_seqs, int num_heads, int num_kv_heads,
                                       int block_size, int residual_length, float scale,
                                       int gqa_map, int bits, const float* cos_t,
                                       const float* sin_t, int max_pos, int style);
void orc_kivi_paged_attention(double* out, const void* q, int q_dtype,
                              const uint8_t* pages, const int32_t* page_tables,
                              int max_pages, int num_pages, const uint16_t* k_cache,
                              const uint16_t* v_cache, const int32_t* block_tables,
                              int max_blocks_per_seq, const int32_t* seq_lens,
                              int num_seqs, int num_heads, int num_kv_heads,
                              int block_size, int residual_length, float scale,
                              int gqa_map);

#ifdef __cplusplus
}
#endif
#endif
