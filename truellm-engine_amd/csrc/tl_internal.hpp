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
  int part_o_dtype;             // 0 = f32, else the q dtype
  int num_seqs, num_heads, num_kv_heads, head_size, block_size;
  int max_blocks_per_seq, num_blocks;
  int num_partitions;           // 1 = single pass
  int partition_tokens;         // multiple of kDecodeChunk when P > 1
  int q_dtype, kv_dtype, gqa_map;
  float scale, k_scale, v_scale;
  int use_generic;              // 1 = force the generic (FMA) decode kernel
  hipStream_t stream;
};

// Returns 0 on success, 3 when no kernel is built for the shape/dtypes,
// 5 on a launch error.
int launch_decode(const DecodeLaunch& a);

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

// absmax(x)/448 into *scale_out (1 when absmax is 0).
int launch_fp8_scale(const void* x, int dtype, int64_t n, float* scale_out,
                     hipStream_t stream);

}  // namespace tl
