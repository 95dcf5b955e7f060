// tl_internal.hpp -- launch descriptors shared between the C ABI layer
// (tl_api.cpp) and the kernel translation units.  Host-only types; no
// validation happens here, the ABI layer has done it.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace tl {

// Tokens per chunk of the decode kernels: scores of one chunk live in LDS.
constexpr int kDecodeChunk = 512;

struct DecodeLaunch {
  void* out;                    // [S, H, D] in q dtype (single pass)
  const void* q;                // [S, H, D]
  const void* k_cache;          // [N, n_kv, D, BS]
  const void* v_cache;          // [N, n_kv, D, BS]
  const int32_t* block_tables;  // [S, max_blocks_per_seq], -1 = hole
  const int32_t* seq_lens;      // [S]
  float* part_m;                // [S, H, P] (split-K only)
  float* part_l;                // [S, H, P]
  void* part_o;                 // [S, H, P, D]
  int num_seqs, num_heads, num_kv_heads, head_size, block_size;
  int max_blocks_per_seq, num_blocks;
  int num_partitions;           // 1 = single pass
  int partition_tokens;         // multiple of kDecodeChunk when P > 1
  int q_dtype, kv_dtype, gqa_map;
  float scale, k_scale, v_scale;
  int part_o_dtype;             // split-K partial outputs: F32 (0), or F16 (f16 q and KV, head 128)
  hipStream_t stream;
};

// Returns 0 on success, 3 when no kernel is built for the shape/dtypes,
// 5 on a launch error.
int launch_decode(const DecodeLaunch& a);

// The matrix-core decode (head_size 128, block_size 16, fp32 split-K
// partials): FP8 KV with f16 / bf16 q, or 2-byte KV with q of the same type.
// Returns 3 for anything else, so the caller can fall back.
int launch_decode_mfma(const DecodeLaunch& a);

// Whether launch_decode sends a decode to the matrix-core kernels, which
// serve 16 q heads per workgroup (the other kernels serve 4): FP8, f16 and
// bf16 KV with head_size 128 and block_size 16.  They beat the dot-product
// wavefront at every GQA group measured (group 4: 6.38 against 5.94 TB/s;
// group 8, where the dot-product wavefront reads KV twice: 5.8 against
// 3.0 TB/s).
inline bool decode_uses_mfma(int kv_dtype, int num_heads, int num_kv_heads, int head_size, int block_size) {
  (void)num_heads;
  if (head_size != 128 || num_kv_heads <= 0) return false;
  const bool pow2 = block_size > 0 && (block_size & (block_size - 1)) == 0 && block_size <= 256;
  return (kv_dtype == 32 || kv_dtype == 1 || kv_dtype == 2) && pow2 && block_size >= 8;   // FP8 E4M3, f16, bf16
}

struct CacheLaunch {
  const void* key;              // [T, n_kv, D]
  const void* value;
  void* k_cache;                // [N, n_kv, D, BS]
  void* v_cache;
  const int32_t* slot_mapping;  // [T]
  int num_tokens, num_kv_heads, head_size, block_size, num_blocks;
  int src_dtype, cache_dtype;   // cache FP8 -> quantise with 1/k_scale, 1/v_scale
  float k_scale, v_scale;
  hipStream_t stream;
};
int launch_reshape_and_cache(const CacheLaunch& a);

// RoPE on q and key, then key and value into the pools (one launch).
struct RopeCache {
  const void* q; void* q_out;   // [T, H, d]
  const void* key; const void* value;   // [T, n_kv, d]
  void* k_cache; void* v_cache; // [N, n_kv, d, BS]
  const int32_t* slot_mapping;  // [T]
  const int32_t* positions;     // [T]
  const float* cos_table; const float* sin_table;   // [max_positions, d/2]
  int num_tokens, num_heads, num_kv_heads, head_size, block_size, num_blocks, max_positions;
  int dtype, style;             // style 0: pairs (2i, 2i+1); 1: (i, i + d/2)
  int q_only;                   // set by the launcher: k and v go through the row kernel
  void* k_out;                  // launch_rope_rows: rotated keys [T, n_kv, d] (no pool writes)
};
int launch_rope_cache(const RopeCache& a, hipStream_t stream);
// RoPE of q (into q_out) and of the keys (into k_out), nothing else written.
int launch_rope_rows(const RopeCache& a, hipStream_t stream);

// Norms and gated activations (residual == nullptr: plain RMSNorm).
int launch_rms_norm(void* out, void* residual, const void* x, const void* w, int rows, int hidden, float eps,
                    int dtype, hipStream_t stream);
int launch_layer_norm(void* out, const void* x, const void* w, const void* b, int rows, int hidden, float eps,
                      int dtype, hipStream_t stream);
int launch_act_and_mul(void* out, const void* gate, const void* up, int64_t n, int act, int dtype,
                       hipStream_t stream);

// VQ codec.  Encode / assign: the nearest codebook entry of each fp16
// vector, as uint16 (idx16) or int32 (idx32).
constexpr int kVqMaxDim = 256;
struct VqArgs {
  const uint16_t* vecs;         // [n, head_size] fp16
  const uint16_t* book;         // [codebook_size, head_size] fp16
  uint16_t* idx16; int32_t* idx32;
  int64_t num_vecs;
  int head_size, codebook_size;
};
int launch_vq_assign(const VqArgs& a, hipStream_t stream);
int launch_vq_decode(void* out, const void* book, const uint16_t* idx, int64_t num_vecs, int head_size,
                     int codebook_size, hipStream_t stream);
size_t vq_kmeans_workspace(int64_t n, int codebook_size, int head_size);
int launch_vq_kmeans(const void* data, void* book, int64_t n, int codebook_size, int head_size, int iterations,
                     void* workspace, hipStream_t stream);

// Whole-block copies: for pair p of mapping [num_pairs][2] = {src, dst},
// block src of src0 (and of src1 when pools == 2) to block dst of dst0
// (dst1).  Ids outside [0, src_blocks) / [0, dst_blocks) skip the pair.
struct BlockCopy {
  const char* src0; const char* src1;
  char* dst0; char* dst1;
  const int32_t* mapping;
  int num_pairs, pools, src_blocks, dst_blocks;
  int64_t block_bytes;
  int slices;                   // set by the launcher
};
int launch_block_copy(const BlockCopy& c, hipStream_t stream);

// Log-sum-exp merge of split-K partials into out.  The partitions a sequence
// has are ceil(L / partition_tokens), or, for KIVI (kivi_pages > 0),
// max(1, ceil(min(pages(L), kivi_max_pages) / kivi_pages)).
int launch_lse_reduce(void* out, int q_dtype, const float* part_m, const float* part_l,
                      const void* part_o, const int32_t* seq_lens, int num_seqs,
                      int num_heads, int head_size, int num_partitions, int partition_tokens,
                      int kivi_residual, int kivi_pages, int kivi_max_pages, hipStream_t stream,
                      int part_o_dtype = 0);

// ---- KIVI ------------------------------------------------------------------
int launch_kivi_vec(const void* in, void* out, int n_vecs, int head_dim, int n_outliers,
                    int group_size, int stride, bool compress, hipStream_t stream);

struct KiviPageLaunch {
  void* k_cache;                // fp16 pools [N, n_kv, 128, BS] (append writes the new token)
  void* v_cache;
  const int32_t* block_tables;
  const int32_t* seq_lens;
  const int32_t* page_tables;   // [S, max_pages_per_seq]
  void* pages;                  // [num_pages, n_kv, page bytes (5120 INT4, 9216 INT8)]
  int num_seqs, num_kv_heads, block_size, max_blocks_per_seq, num_blocks;
  int max_pages_per_seq, num_pages, residual_length;
  int bits;                     // page code width: 4 or 8
  int max_pages_to_build;       // prefix build: page slots per sequence in the grid
  int append;                   // 1: write the new token, then build the page L completes
  int build_ahead;              // 1: pages built in pieces over the steps before they complete
  const void* knew;             // append: new token per sequence [S, n_kv, 128] fp16
  const void* vnew;
  const int32_t* slots;         // append: its slot in the fp16 pool
  hipStream_t stream;
};
int launch_kivi_pages(const KiviPageLaunch& a);

struct KiviDecodeLaunch {
  void* out;                    // [S, H, 128] fp16
  const void* q;                // [S, H, 128] fp16
  const void* pages;
  const int32_t* page_tables;
  const void* k_cache;          // fp16 residual window, [N, n_kv, 128, block_size]
  const void* v_cache;
  const int32_t* block_tables;
  const int32_t* seq_lens;
  float* part_m; float* part_l; void* part_o;   // fp32 split-K partials
  int num_seqs, num_heads, num_kv_heads, block_size, max_blocks_per_seq, num_blocks;
  int max_pages_per_seq, num_pages, residual_length, gqa_map;
  int num_partitions, partition_pages;
  int bits;                     // page code width: 4 or 8
  float scale;
  const KiviPageLaunch* append;  // non-null: the step's append (token write, page build),
                                 // fused into the decode launch
  // non-null: keys are held before RoPE and rotated at their positions
  // while scored (fp32 tables [rope_max_pos, 64], style 0 or 1)
  const float* rope_cos = nullptr;
  const float* rope_sin = nullptr;
  int rope_max_pos = 0, rope_style = 0;
  hipStream_t stream;
};
int launch_kivi_decode(const KiviDecodeLaunch& a);

struct PrefillLaunch {
  void* out;                    // [total_q, H, 128], dtype
  const void* q;                // [total_q, H, 128], dtype
  const int32_t* cu_q_lens;     // [num_seqs + 1]
  const void* k_cache;          // [N, n_kv, 128, bs], kv_dtype
  const void* v_cache;
  const int32_t* block_tables;
  const int32_t* seq_lens;
  int num_seqs, num_heads, num_kv_heads, block_size, max_blocks_per_seq, num_blocks;
  int dtype, gqa_map, max_q_len, num_prefill_seqs;
  int kv_dtype;                 // dtype, or FP8 E4M3 (k_scale, v_scale: the per-tensor scales)
  float scale, k_scale, v_scale;
  hipStream_t stream;
};
// Returns 0, 3 (no kernel for the block size) or 5 (launch error).
int launch_prefill(const PrefillLaunch& a);

// out[i] = e4m3(float(in[i]) * scale) for i < n (in: F16, BF16 or F32).
int launch_convert_fp8(uint8_t* out, const void* in, int dtype, int64_t n, float scale, hipStream_t stream);

// absmax(x)/448 into *scale_out (1 when absmax is 0).
int launch_fp8_scale(const void* x, int dtype, int64_t n, float* scale_out,
                     hipStream_t stream);

// Sets the message tl_last_error_string() returns (this thread) and
// returns code; for entry points defined outside tl_api.cpp.
int report_error(int code, const char* msg);

}  // namespace tl
