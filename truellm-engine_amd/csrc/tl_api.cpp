// tl_api.cpp -- the C ABI (include/tl_attn.h): argument checks, split-K
// planning and dispatch to the HIP launchers.  Every check runs on the host
// before any HIP call, so a bad call returns an error code and leaves the
// device untouched.
#include "tl_attn.h"
#include "tl_internal.hpp"
#include "tl_kivi.hpp"

#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
  return code;
}

int ok() {
  g_err[0] = '\0';
  return TL_OK;
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

bool is_float_kind(int32_t d) {
  return d == TL_DTYPE_F32 || d == TL_DTYPE_F16 || d == TL_DTYPE_BF16;
}

bool uses_mfma(const tl_decode_desc* d) {
  return tl::decode_uses_mfma(d->kv_dtype, d->num_heads, d->num_kv_heads, d->head_size, d->block_size);
}

// The token granularity of split-K partitions: the matrix-core kernels
// split at any multiple of their wavefront iteration (32 tokens of 2-byte
// KV, 64 of FP8), the others at kDecodeChunk (their scores of one chunk
// live in LDS).
int partition_grain(const tl_decode_desc* d) {
  if (!uses_mfma(d)) return tl::kDecodeChunk;
  return d->kv_dtype == TL_DTYPE_FP8_E4M3 ? 64 : 32;
}

int check_decode(const tl_decode_desc* d) {
  if (!d) return fail(TL_ERR_INVALID_ARGUMENT, "desc is NULL");
  if (d->num_seqs < 0) return fail(TL_ERR_INVALID_ARGUMENT, "num_seqs=%d < 0", d->num_seqs);
  if (d->num_kv_heads <= 0 || d->num_heads <= 0 || d->num_heads % d->num_kv_heads)
    return fail(TL_ERR_INVALID_ARGUMENT, "num_heads=%d must be a positive multiple of num_kv_heads=%d",
                d->num_heads, d->num_kv_heads);
  if (d->max_blocks_per_seq <= 0 || d->num_blocks <= 0)
    return fail(TL_ERR_INVALID_ARGUMENT, "max_blocks_per_seq=%d and num_blocks=%d must be > 0",
                d->max_blocks_per_seq, d->num_blocks);
  if (d->gqa_map != TL_GQA_MODULO && d->gqa_map != TL_GQA_GROUPED)
    return fail(TL_ERR_INVALID_ARGUMENT, "gqa_map=%d", d->gqa_map);
  if (!is_float_kind(d->q_dtype))
    return fail(TL_ERR_INVALID_ARGUMENT, "q_dtype=%d is not F32/F16/BF16", d->q_dtype);
  if (!is_float_kind(d->kv_dtype) && d->kv_dtype != TL_DTYPE_FP8_E4M3)
    return fail(TL_ERR_INVALID_ARGUMENT, "kv_dtype=%d", d->kv_dtype);
  if (d->kv_dtype != TL_DTYPE_FP8_E4M3 && d->kv_dtype != d->q_dtype)
    return fail(TL_ERR_NOT_IMPLEMENTED, "kv_dtype=%d with q_dtype=%d (q and a 16/32-bit pool must match)",
                d->kv_dtype, d->q_dtype);
  if (d->kv_dtype == TL_DTYPE_FP8_E4M3 && d->q_dtype == TL_DTYPE_F32)
    return fail(TL_ERR_NOT_IMPLEMENTED, "FP8 KV needs F16 or BF16 q");
  // head size 128: the matrix-core decode, any power-of-two block size
  // 8 .. 256 (FP8 too); the FMA decode: head sizes 64 / 256 (and
  // 80 / 96 for 2-byte pools) at block size 16; F32 pools: head sizes 64 /
  // 128 / 256 at block size 16 (the shapes of paged_attention_v1.cu:198-209)
  const int hs = d->head_size, bs = d->block_size;
  bool shape_ok;
  if (d->kv_dtype == TL_DTYPE_F32)
    shape_ok = bs == 16 && (hs == 64 || hs == 128 || hs == 256);
  else if (hs == 128)
    shape_ok = tl::decode_uses_mfma(d->kv_dtype, d->num_heads, d->num_kv_heads, hs, bs);
  else if (hs == 64 || hs == 256)
    shape_ok = bs == 16;
  else if (hs == 80 || hs == 96)
    shape_ok = bs == 16 && d->kv_dtype != TL_DTYPE_FP8_E4M3;
  else
    shape_ok = false;
  if (!shape_ok)
    return fail(TL_ERR_NOT_IMPLEMENTED,
                "head_size=%d block_size=%d kv_dtype=%d (built: head 128 with block sizes 8..256; "
                "heads 64/256, and 80/96 for 2-byte KV, with block size 16; F32 KV heads 64/128/256 with "
                "block size 16)",
                hs, bs, d->kv_dtype);
  const int grain = partition_grain(d);
  if (d->partition_tokens != 0 && d->partition_tokens != -1 &&
      (d->partition_tokens <= 0 || d->partition_tokens % grain))
    return fail(TL_ERR_INVALID_ARGUMENT, "partition_tokens=%d must be 0, -1 or a multiple of %d",
                d->partition_tokens, grain);
  return TL_OK;
}

// Split-K plan: partition size and count for a batch whose longest sequence
// is max_ctx.  Aim for >= 512 workgroups (two per CU on 256 CUs, which is
// what the single-pass kernels' occupancy admits); a batch that already
// provides that many (sequence, kv head) items runs single pass up to 4096
// tokens and in 2048-token partitions past that: with lengths that differ
// the single pass waits for its longest sequences (batch 64, lengths
// uniform in [512, 8192], bf16: 172 us in 2048-token partitions against
// 200 us single pass; equal lengths of 4096 would lose 3.5 %).
void plan_partitions(const tl_decode_desc* d, int32_t max_ctx, int* P, int* PT) {
  const int chunks = max_ctx > 0 ? (max_ctx + tl::kDecodeChunk - 1) / tl::kDecodeChunk : 1;
  if (d->partition_tokens > 0) {
    *PT = d->partition_tokens;
    *P = max_ctx > 0 ? (int)(((int64_t)max_ctx + *PT - 1) / *PT) : 1;
    return;
  }
  int pt_chunks;
  if (d->partition_tokens == -1) {
    pt_chunks = chunks;
  } else {
    const int group = d->num_heads / d->num_kv_heads;
    // q heads per workgroup: 16 for the matrix-core kernels, 4 otherwise
    const int per = tl::decode_uses_mfma(d->kv_dtype, d->num_heads, d->num_kv_heads, d->head_size, d->block_size)
                        ? 16 : 4;
    const int slices = group == 1 ? 1 : (group + per - 1) / per;
    const long items = (long)d->num_seqs * d->num_kv_heads * slices;
    long want = items > 0 ? (512 + items - 1) / items : 1;
    if (want < 1) want = 1;
    if (want > chunks) want = chunks;
    pt_chunks = (int)((chunks + want - 1) / want);
    if (want == 1 && chunks > 8) pt_chunks = 4;
  }
  if (pt_chunks < 1) pt_chunks = 1;
  *P = (chunks + pt_chunks - 1) / pt_chunks;
  *PT = pt_chunks * tl::kDecodeChunk;
  // A split batch too small to give every CU a workgroup even in
  // kDecodeChunk partitions (the engine decodes one sequence per call,
  // cuda_engine.cpp:1138-1159): the matrix-core kernels take shorter
  // partitions, down to one iteration per wavefront of a 4-wavefront
  // workgroup (128 tokens of 2-byte KV, 256 of FP8), so that about 256
  // workgroups share the context.  (A context that the plan runs single
  // pass stays so: the merge's launch would cost more than it saves.)
  if (d->partition_tokens == 0 && uses_mfma(d) && *P > 1) {
    const int group = d->num_heads / d->num_kv_heads;
    const long items = (long)d->num_seqs * d->num_kv_heads * ((group + 15) / 16);
    if (items > 0 && items * *P < 256) {
      const int round = 4 * partition_grain(d);
      const long want = (256 + items - 1) / items;
      long pt = (max_ctx + want - 1) / want;
      pt = (pt + round - 1) / round * round;
      if (pt < *PT) {
        *PT = (int)pt;
        *P = (int)((max_ctx + pt - 1) / pt);
      }
    }
  }
}

tl::DecodeLaunch make_launch(const tl_decode_desc* d, void* out, const void* q,
                             const void* k_cache, const void* v_cache, const int32_t* bt,
                             const int32_t* sl, void* stream) {
  tl::DecodeLaunch a;
  memset(&a, 0, sizeof a);
  a.out = out; a.q = q; a.k_cache = k_cache; a.v_cache = v_cache;
  a.block_tables = bt; a.seq_lens = sl;
  a.num_seqs = d->num_seqs; a.num_heads = d->num_heads; a.num_kv_heads = d->num_kv_heads;
  a.head_size = d->head_size; a.block_size = d->block_size;
  a.max_blocks_per_seq = d->max_blocks_per_seq; a.num_blocks = d->num_blocks;
  a.q_dtype = d->q_dtype; a.kv_dtype = d->kv_dtype; a.gqa_map = d->gqa_map;
  a.scale = d->scale; a.k_scale = d->k_scale; a.v_scale = d->v_scale;
  a.num_partitions = 1; a.partition_tokens = 0;
  a.stream = (hipStream_t)stream;
  return a;
}

int run(const tl::DecodeLaunch& a) {
  const int rc = tl::launch_decode(a);
  if (rc == 3) return fail(TL_ERR_NOT_IMPLEMENTED, "no decode kernel for this dtype/shape");
  if (rc != 0) return fail(TL_ERR_BACKEND, "decode launch failed: %s", hipGetErrorString(hipGetLastError()));
  return ok();
}

size_t ws_bytes(const tl_decode_desc* d, int P) {
  if (P <= 1) return 0;
  const size_t sh = (size_t)d->num_seqs * d->num_heads * P;
  return sh * d->head_size * 4 + 2 * sh * 4;
}

}  // namespace

// The plan of paged_attention_v2 inside the caller's scratch.  The scratch
// holds Pc partitions: exp_sums / max_logits fp32 [S, H, Pc], tmp_out
// [S, H, Pc, head_size] in the call's dtype.  The engine sizes it as
// ceil(max_context_len / (32 block_size)) (cuda_engine.cpp:273-285,1144);
// the reference kernel writes (max_context_len / block_size + 31) / 32
// partitions (paged_attention_v2.cu:196), which is never more, so a caller
// that sized the scratch for the reference kernel has at least that many
// and Pc is taken as that count.  The engine reads none of it after the
// call, so it is the workspace of the library's own plan: the (max, sum)
// pairs in max_logits / exp_sums and the partial outputs in tmp_out.  f16
// calls on the matrix-core kernels keep the partial outputs in f16, one
// partition per tmp_out slot, as the reference's own tmp_out does
// (paged_attention_v2.cu:61-63,111-124 store them in scalar_t): a partial
// is a convex combination of f16 values, so it stays in f16's range, and
// its rounding (half an ulp of a value below max |v|) is within the 2e-3
// bar for the N(0, 1) values of the workloads.  bf16 and f32 keep fp32
// partials (Pc * elem / 4 partitions in tmp_out's bytes).  Where the plan
// wants more partitions than the scratch holds they are made longer; where
// it wants one (a large batch) the call runs single pass.  d is the
// descriptor of the call (partition_tokens 0) and may be changed.
// Pc: tmp_out's partition slots (0: the reference kernel's count for
// max_ctx; a caller that allocated the scratch for a longer context passes
// its own count).
void v2_plan(tl_decode_desc* d, int32_t max_ctx, bool tmp_aligned, int* P, int* PT, bool* f16_parts, int Pc = 0) {
  if (Pc <= 0) Pc = (max_ctx / d->block_size + 31) / 32;
  const int elem = d->q_dtype == TL_DTYPE_F32 ? 4 : 2;
  *f16_parts = d->q_dtype == TL_DTYPE_F16 && uses_mfma(d);
  const int cap = tmp_aligned ? (*f16_parts ? Pc : Pc * elem / 4) : 1;
  plan_partitions(d, max_ctx, P, PT);
  if (*P > cap) {
    if (cap <= 1) {
      *P = 1;
    } else {
      // the longer partitions, in the kernels' granularity (a multiple of
      // kDecodeChunk, or of a 4-wavefront round for the matrix-core kernels)
      const int round = uses_mfma(d) ? 4 * partition_grain(d) : tl::kDecodeChunk;
      const int64_t pt = ((int64_t)max_ctx + cap - 1) / cap;
      d->partition_tokens = (int)((pt + round - 1) / round * round);
      plan_partitions(d, max_ctx, P, PT);
    }
  }
}

int tl::report_error(int code, const char* msg) { return fail(code, "%s", msg); }

extern "C" {

int tl_abi_version(void) { return TL_ABI_VERSION; }

const char* tl_last_error_string(void) { return g_err; }

int tl_engine_apply_config(tl_decode_desc* desc, int32_t paged_kv_block_size, int32_t use_fp8_kv,
                           const char* attention_layout) {
  if (!desc) return fail(TL_ERR_INVALID_ARGUMENT, "desc is NULL");
  if (paged_kv_block_size <= 0 || (paged_kv_block_size & (paged_kv_block_size - 1)))
    return fail(TL_ERR_INVALID_ARGUMENT, "paged_kv_block_size=%d (a power of two)", paged_kv_block_size);
  if (!attention_layout || (strcmp(attention_layout, "paged") != 0 && strcmp(attention_layout, "flash_paged") != 0))
    return fail(TL_ERR_NOT_IMPLEMENTED, "attention_layout '%s' (built: paged, flash_paged)",
                attention_layout ? attention_layout : "(null)");
  tl_decode_desc d = *desc;
  d.block_size = paged_kv_block_size;
  d.kv_dtype = use_fp8_kv ? TL_DTYPE_FP8_E4M3 : d.q_dtype;
  if (use_fp8_kv) {
    if (!(d.k_scale > 0.f)) d.k_scale = 1.f;
    if (!(d.v_scale > 0.f)) d.v_scale = 1.f;
  }
  const int rc = check_decode(&d);
  if (rc) return rc;
  *desc = d;
  return ok();
}

size_t tl_paged_attention_workspace_bytes(const tl_decode_desc* desc, int32_t max_context_len) {
  if (check_decode(desc) != TL_OK || max_context_len < 0) return 0;
  int P, PT;
  plan_partitions(desc, max_context_len, &P, &PT);
  return ws_bytes(desc, P);
}

// The decode, and with key non-null the step: the token's append to the
// pools at slots[s], then the decode.
static int decode_impl(const tl_decode_desc* desc, void* out, const void* q, const void* k_cache,
                       const void* v_cache, const int32_t* block_tables, const int32_t* seq_lens,
                       int32_t max_context_len, void* workspace, size_t workspace_bytes, void* stream,
                       const void* key, const void* value, const int32_t* slots) {
  int rc = check_decode(desc);
  if (rc) return rc;
  if (max_context_len < 0) return fail(TL_ERR_INVALID_ARGUMENT, "max_context_len < 0");
  if (desc->num_seqs == 0) return ok();
  if (!out || !q || !k_cache || !v_cache || !block_tables || !seq_lens)
    return fail(TL_ERR_INVALID_ARGUMENT, "NULL tensor pointer");
  if (!aligned16(k_cache) || !aligned16(v_cache))
    return fail(TL_ERR_INVALID_ARGUMENT, "k_cache/v_cache must be 16-byte aligned");
  if (key && (!value || !slots)) return fail(TL_ERR_INVALID_ARGUMENT, "NULL key/value/slot_mapping");
  if (key && (!aligned16(key) || !aligned16(value)))
    return fail(TL_ERR_INVALID_ARGUMENT, "key/value must be 16-byte aligned");
  int P, PT;
  plan_partitions(desc, max_context_len, &P, &PT);
  tl::DecodeLaunch a = make_launch(desc, out, q, k_cache, v_cache, block_tables, seq_lens, stream);
  if (P > 1) {
    const size_t need = ws_bytes(desc, P);
    if (!workspace || workspace_bytes < need)
      return fail(TL_ERR_INVALID_ARGUMENT, "workspace of %zu bytes needed, %zu given", need,
                  workspace_bytes);
    if (!aligned16(workspace)) return fail(TL_ERR_INVALID_ARGUMENT, "workspace must be 16-byte aligned");
    const size_t sh = (size_t)desc->num_seqs * desc->num_heads * P;
    a.part_o = workspace;
    a.part_m = (float*)((char*)workspace + sh * desc->head_size * 4);
    a.part_l = a.part_m + sh;
    a.num_partitions = P;
    a.partition_tokens = PT;
  }
  if (key) {
    rc = desc->kv_dtype == TL_DTYPE_FP8_E4M3
             ? tl_reshape_and_cache_fp8(key, value, desc->q_dtype, (uint8_t*)k_cache, (uint8_t*)v_cache, slots,
                                        desc->num_seqs, desc->num_kv_heads, desc->head_size, desc->block_size,
                                        desc->num_blocks, desc->k_scale, desc->v_scale, stream)
             : tl_reshape_and_cache(key, value, (void*)k_cache, (void*)v_cache, slots, desc->num_seqs,
                                    desc->num_kv_heads, desc->head_size, desc->block_size, desc->num_blocks,
                                    desc->kv_dtype, stream);
    if (rc) return rc;
  }
  return run(a);
}

int tl_paged_attention_decode(const tl_decode_desc* desc, void* out, const void* q,
                              const void* k_cache, const void* v_cache,
                              const int32_t* block_tables, const int32_t* seq_lens,
                              int32_t max_context_len, void* workspace, size_t workspace_bytes,
                              void* stream) {
  return decode_impl(desc, out, q, k_cache, v_cache, block_tables, seq_lens, max_context_len, workspace,
                     workspace_bytes, stream, nullptr, nullptr, nullptr);
}

int tl_paged_attention_decode_step(const tl_decode_desc* desc, void* out, const void* q, const void* key,
                                   const void* value, const int32_t* slot_mapping, void* k_cache, void* v_cache,
                                   const int32_t* block_tables, const int32_t* seq_lens, int32_t max_context_len,
                                   void* workspace, size_t workspace_bytes, void* stream) {
  if (desc && desc->num_seqs > 0 && (!key || !value || !slot_mapping))
    return fail(TL_ERR_INVALID_ARGUMENT, "NULL key/value/slot_mapping");
  return decode_impl(desc, out, q, k_cache, v_cache, block_tables, seq_lens, max_context_len, workspace,
                     workspace_bytes, stream, key, value, slot_mapping);
}

int tl_paged_attention_v1(void* out, const void* q, const void* k_cache, const void* v_cache,
                          const int32_t* block_tables, const int32_t* seq_lens, int32_t num_seqs,
                          int32_t num_heads, int32_t num_kv_heads, int32_t head_size,
                          int32_t block_size, int32_t max_blocks_per_seq, int32_t num_blocks,
                          float scale, int32_t dtype, int32_t gqa_map, void* stream) {
  tl_decode_desc d = {num_seqs, num_heads, num_kv_heads, head_size, block_size, max_blocks_per_seq,
                      num_blocks, dtype, dtype, gqa_map, -1, scale, 1.f, 1.f};
  int rc = check_decode(&d);
  if (rc) return rc;
  if (num_seqs == 0) return ok();
  if (!out || !q || !k_cache || !v_cache || !block_tables || !seq_lens)
    return fail(TL_ERR_INVALID_ARGUMENT, "NULL tensor pointer");
  if (!aligned16(k_cache) || !aligned16(v_cache))
    return fail(TL_ERR_INVALID_ARGUMENT, "k_cache/v_cache must be 16-byte aligned");
  return run(make_launch(&d, out, q, k_cache, v_cache, block_tables, seq_lens, stream));
}

static int v2_impl(void* out, float* exp_sums, float* max_logits, void* tmp_out, const void* q,
                   const void* k_cache, const void* v_cache, const int32_t* block_tables, const int32_t* seq_lens,
                   int32_t num_seqs, int32_t num_heads, int32_t num_kv_heads, int32_t head_size,
                   int32_t block_size, int32_t max_blocks_per_seq, int32_t num_blocks, float scale, int32_t dtype,
                   int32_t gqa_map, int32_t max_context_len, int32_t scratch_partitions, void* stream) {
  tl_decode_desc d = {num_seqs, num_heads, num_kv_heads, head_size, block_size, max_blocks_per_seq,
                      num_blocks, dtype, dtype, gqa_map, 0, scale, 1.f, 1.f};
  int rc = check_decode(&d);
  if (rc) return rc;
  if (max_context_len < 0) return fail(TL_ERR_INVALID_ARGUMENT, "max_context_len < 0");
  if (scratch_partitions > 0 && scratch_partitions < (max_context_len / block_size + 31) / 32)
    return fail(TL_ERR_INVALID_ARGUMENT, "scratch_partitions=%d below the %d partitions of max_context_len=%d",
                scratch_partitions, (max_context_len / block_size + 31) / 32, max_context_len);
  if (num_seqs == 0) return ok();
  if (!out || !q || !k_cache || !v_cache || !block_tables || !seq_lens || !exp_sums ||
      !max_logits || !tmp_out)
    return fail(TL_ERR_INVALID_ARGUMENT, "NULL tensor pointer");
  if (!aligned16(k_cache) || !aligned16(v_cache))
    return fail(TL_ERR_INVALID_ARGUMENT, "k_cache/v_cache must be 16-byte aligned");
  int P, PT;
  bool f16_parts;
  v2_plan(&d, max_context_len, aligned16(tmp_out), &P, &PT, &f16_parts, scratch_partitions);
  tl::DecodeLaunch a = make_launch(&d, out, q, k_cache, v_cache, block_tables, seq_lens, stream);
  if (P > 1) {
    a.num_partitions = P;
    a.partition_tokens = PT;
    a.part_m = max_logits;
    a.part_l = exp_sums;
    a.part_o = tmp_out;
    a.part_o_dtype = f16_parts ? TL_DTYPE_F16 : TL_DTYPE_F32;
  }
  return run(a);
}

int tl_paged_attention_v2(void* out, float* exp_sums, float* max_logits, void* tmp_out,
                          const void* q, const void* k_cache, const void* v_cache,
                          const int32_t* block_tables, const int32_t* seq_lens, int32_t num_seqs,
                          int32_t num_heads, int32_t num_kv_heads, int32_t head_size,
                          int32_t block_size, int32_t max_blocks_per_seq, int32_t num_blocks,
                          float scale, int32_t dtype, int32_t gqa_map, int32_t max_context_len,
                          void* stream) {
  return v2_impl(out, exp_sums, max_logits, tmp_out, q, k_cache, v_cache, block_tables, seq_lens, num_seqs,
                 num_heads, num_kv_heads, head_size, block_size, max_blocks_per_seq, num_blocks, scale, dtype,
                 gqa_map, max_context_len, 0, stream);
}

int tl_paged_attention_v2_capacity(void* out, float* exp_sums, float* max_logits, void* tmp_out,
                                   const void* q, const void* k_cache, const void* v_cache,
                                   const int32_t* block_tables, const int32_t* seq_lens, int32_t num_seqs,
                                   int32_t num_heads, int32_t num_kv_heads, int32_t head_size,
                                   int32_t block_size, int32_t max_blocks_per_seq, int32_t num_blocks,
                                   float scale, int32_t dtype, int32_t gqa_map, int32_t max_context_len,
                                   int32_t scratch_partitions, void* stream) {
  if (scratch_partitions <= 0) return fail(TL_ERR_INVALID_ARGUMENT, "scratch_partitions=%d", scratch_partitions);
  return v2_impl(out, exp_sums, max_logits, tmp_out, q, k_cache, v_cache, block_tables, seq_lens, num_seqs,
                 num_heads, num_kv_heads, head_size, block_size, max_blocks_per_seq, num_blocks, scale, dtype,
                 gqa_map, max_context_len, scratch_partitions, stream);
}

static int32_t v2_partitions_impl(int32_t num_seqs, int32_t num_heads, int32_t num_kv_heads, int32_t head_size,
                                  int32_t block_size, int32_t dtype, int32_t max_context_len,
                                  int32_t scratch_partitions, int32_t* partition_tokens) {
  tl_decode_desc d = {num_seqs, num_heads, num_kv_heads, head_size, block_size, 1, 1,
                      dtype, dtype, TL_GQA_MODULO, 0, 1.f, 1.f, 1.f};
  if (check_decode(&d) != TL_OK || max_context_len < 0) return -1;
  if (scratch_partitions > 0 && scratch_partitions < (max_context_len / block_size + 31) / 32) return -1;
  int P, PT;
  bool f16_parts;
  v2_plan(&d, max_context_len, true, &P, &PT, &f16_parts, scratch_partitions);
  if (partition_tokens) *partition_tokens = P > 1 ? PT : 0;
  ok();
  return P;
}

int32_t tl_paged_attention_v2_partitions(int32_t num_seqs, int32_t num_heads, int32_t num_kv_heads,
                                         int32_t head_size, int32_t block_size, int32_t dtype,
                                         int32_t max_context_len, int32_t* partition_tokens) {
  return v2_partitions_impl(num_seqs, num_heads, num_kv_heads, head_size, block_size, dtype, max_context_len, 0,
                            partition_tokens);
}

int32_t tl_paged_attention_v2_capacity_partitions(int32_t num_seqs, int32_t num_heads, int32_t num_kv_heads,
                                                  int32_t head_size, int32_t block_size, int32_t dtype,
                                                  int32_t max_context_len, int32_t scratch_partitions,
                                                  int32_t* partition_tokens) {
  if (scratch_partitions <= 0) return -1;
  return v2_partitions_impl(num_seqs, num_heads, num_kv_heads, head_size, block_size, dtype, max_context_len,
                            scratch_partitions, partition_tokens);
}

int tl_reshape_and_cache(const void* key, const void* value, void* k_cache, void* v_cache,
                         const int32_t* slot_mapping, int32_t num_tokens, int32_t num_kv_heads,
                         int32_t head_size, int32_t block_size, int32_t num_blocks, int32_t dtype,
                         void* stream) {
  if (num_tokens < 0 || num_kv_heads <= 0 || head_size <= 0 || block_size <= 0 || num_blocks <= 0)
    return fail(TL_ERR_INVALID_ARGUMENT, "num_tokens=%d num_kv_heads=%d head_size=%d block_size=%d num_blocks=%d",
                num_tokens, num_kv_heads, head_size, block_size, num_blocks);
  if (!is_float_kind(dtype)) return fail(TL_ERR_INVALID_ARGUMENT, "dtype=%d", dtype);
  const int run = dtype == TL_DTYPE_F32 ? 4 : 8;
  if (head_size % run) return fail(TL_ERR_INVALID_ARGUMENT, "head_size=%d must be a multiple of %d", head_size, run);
  if (num_tokens == 0) return ok();
  if (!key || !value || !k_cache || !v_cache || !slot_mapping)
    return fail(TL_ERR_INVALID_ARGUMENT, "NULL tensor pointer");
  if (!aligned16(key) || !aligned16(value))
    return fail(TL_ERR_INVALID_ARGUMENT, "key/value must be 16-byte aligned");
  tl::CacheLaunch a = {key, value, k_cache, v_cache, slot_mapping, num_tokens, num_kv_heads,
                       head_size, block_size, num_blocks, dtype, dtype, 1.f, 1.f,
                       (hipStream_t)stream};
  const int rc = tl::launch_reshape_and_cache(a);
  if (rc) return fail(TL_ERR_BACKEND, "reshape_and_cache launch failed");
  return ok();
}

int tl_rope_reshape_and_cache(const void* q, void* q_out, const void* key, const void* value,
                              void* k_cache, void* v_cache, const int32_t* slot_mapping,
                              const int32_t* positions, const float* cos_table, const float* sin_table,
                              int32_t max_positions, int32_t num_tokens, int32_t num_heads,
                              int32_t num_kv_heads, int32_t head_size, int32_t block_size,
                              int32_t num_blocks, int32_t dtype, int32_t style, void* stream) {
  if (num_tokens < 0 || num_heads < 0 || num_kv_heads <= 0 || head_size <= 0 || block_size <= 0 ||
      num_blocks <= 0 || max_positions <= 0)
    return fail(TL_ERR_INVALID_ARGUMENT,
                "num_tokens=%d num_heads=%d num_kv_heads=%d head_size=%d block_size=%d num_blocks=%d "
                "max_positions=%d", num_tokens, num_heads, num_kv_heads, head_size, block_size, num_blocks,
                max_positions);
  if (head_size % 16) return fail(TL_ERR_INVALID_ARGUMENT, "head_size=%d must be a multiple of 16", head_size);
  if (!is_float_kind(dtype)) return fail(TL_ERR_INVALID_ARGUMENT, "dtype=%d", dtype);
  if (style != TL_ROPE_ADJACENT && style != TL_ROPE_HALVES) return fail(TL_ERR_INVALID_ARGUMENT, "style=%d", style);
  if (num_tokens == 0) return ok();
  if (!key || !value || !k_cache || !v_cache || !slot_mapping || !positions || !cos_table || !sin_table ||
      (num_heads > 0 && (!q || !q_out)))
    return fail(TL_ERR_INVALID_ARGUMENT, "NULL pointer");
  tl::RopeCache a = {q, q_out, key, value, k_cache, v_cache, slot_mapping, positions, cos_table, sin_table,
                     num_tokens, num_heads, num_kv_heads, head_size, block_size, num_blocks, max_positions,
                     dtype, style};
  const int rc = tl::launch_rope_cache(a, (hipStream_t)stream);
  if (rc) return fail(TL_ERR_BACKEND, "rope_reshape_and_cache launch failed");
  return ok();
}

static int check_norm(const void* out, const void* x, const void* weight, int32_t rows, int32_t hidden,
                      int32_t dtype) {
  if (rows < 0 || hidden <= 0) return fail(TL_ERR_INVALID_ARGUMENT, "num_tokens=%d hidden_size=%d", rows, hidden);
  if (!is_float_kind(dtype)) return fail(TL_ERR_INVALID_ARGUMENT, "dtype=%d", dtype);
  if (rows > 0 && (!out || !x || !weight)) return fail(TL_ERR_INVALID_ARGUMENT, "NULL pointer");
  return TL_OK;
}

int tl_rms_norm(void* out, const void* x, const void* weight, int32_t num_tokens, int32_t hidden_size,
                float eps, int32_t dtype, void* stream) {
  int rc = check_norm(out, x, weight, num_tokens, hidden_size, dtype);
  if (rc) return rc;
  if (tl::launch_rms_norm(out, nullptr, x, weight, num_tokens, hidden_size, eps, dtype, (hipStream_t)stream))
    return fail(TL_ERR_BACKEND, "rms_norm launch failed");
  return ok();
}

int tl_fused_add_rms_norm(void* out, void* residual, const void* x, const void* weight, int32_t num_tokens,
                          int32_t hidden_size, float eps, int32_t dtype, void* stream) {
  int rc = check_norm(out, x, weight, num_tokens, hidden_size, dtype);
  if (rc) return rc;
  if (num_tokens > 0 && !residual) return fail(TL_ERR_INVALID_ARGUMENT, "NULL residual");
  if (tl::launch_rms_norm(out, residual, x, weight, num_tokens, hidden_size, eps, dtype, (hipStream_t)stream))
    return fail(TL_ERR_BACKEND, "fused_add_rms_norm launch failed");
  return ok();
}

int tl_layer_norm(void* out, const void* x, const void* weight, const void* bias, int32_t num_tokens,
                  int32_t hidden_size, float eps, int32_t dtype, void* stream) {
  int rc = check_norm(out, x, weight, num_tokens, hidden_size, dtype);
  if (rc) return rc;
  if (num_tokens > 0 && !bias) return fail(TL_ERR_INVALID_ARGUMENT, "NULL bias");
  if (tl::launch_layer_norm(out, x, weight, bias, num_tokens, hidden_size, eps, dtype, (hipStream_t)stream))
    return fail(TL_ERR_BACKEND, "layer_norm launch failed");
  return ok();
}

int tl_act_and_mul(void* out, const void* gate, const void* up, int64_t n, int32_t activation, int32_t dtype,
                   void* stream) {
  if (n < 0 || n > ((int64_t)1 << 40)) return fail(TL_ERR_INVALID_ARGUMENT, "n=%lld", (long long)n);
  if (activation < TL_ACT_SILU || activation > TL_ACT_GELU_TANH)
    return fail(TL_ERR_INVALID_ARGUMENT, "activation=%d", activation);
  if (!is_float_kind(dtype)) return fail(TL_ERR_INVALID_ARGUMENT, "dtype=%d", dtype);
  if (n == 0) return ok();
  if (!out || !gate || !up) return fail(TL_ERR_INVALID_ARGUMENT, "NULL pointer");
  if (tl::launch_act_and_mul(out, gate, up, n, activation, dtype, (hipStream_t)stream))
    return fail(TL_ERR_BACKEND, "act_and_mul launch failed");
  return ok();
}

static int check_vq(int32_t num_vecs, int32_t head_dim, int32_t codebook_size) {
  if (num_vecs < 0 || head_dim <= 0 || head_dim % 8 || head_dim > TL_VQ_MAX_HEAD_DIM || codebook_size < 1 ||
      codebook_size > 65536)
    return fail(TL_ERR_INVALID_ARGUMENT, "num_vecs=%d head_dim=%d codebook_size=%d", num_vecs, head_dim,
                codebook_size);
  return TL_OK;
}

int tl_vq_encode(const void* kv, const void* book, uint16_t* idx, int32_t num_vecs, int32_t head_dim,
                 int32_t codebook_size, void* stream) {
  int rc = check_vq(num_vecs, head_dim, codebook_size);
  if (rc) return rc;
  if (num_vecs == 0) return ok();
  if (!kv || !book || !idx) return fail(TL_ERR_INVALID_ARGUMENT, "NULL pointer");
  if (!aligned16(book)) return fail(TL_ERR_INVALID_ARGUMENT, "book must be 16-byte aligned");
  tl::VqArgs a = {(const uint16_t*)kv, (const uint16_t*)book, idx, nullptr, num_vecs, head_dim, codebook_size};
  if (tl::launch_vq_assign(a, (hipStream_t)stream)) return fail(TL_ERR_BACKEND, "vq_encode launch failed");
  return ok();
}

int tl_vq_decode(void* kv_out, const void* book, const uint16_t* idx, int32_t num_vecs, int32_t head_dim,
                 int32_t codebook_size, void* stream) {
  int rc = check_vq(num_vecs, head_dim, codebook_size);
  if (rc) return rc;
  if (num_vecs == 0) return ok();
  if (!kv_out || !book || !idx) return fail(TL_ERR_INVALID_ARGUMENT, "NULL pointer");
  if (!aligned16(book) || !aligned16(kv_out))
    return fail(TL_ERR_INVALID_ARGUMENT, "kv_out and book must be 16-byte aligned");
  if (tl::launch_vq_decode(kv_out, book, idx, num_vecs, head_dim, codebook_size, (hipStream_t)stream))
    return fail(TL_ERR_BACKEND, "vq_decode launch failed");
  return ok();
}

size_t tl_vq_kmeans_workspace_bytes(int32_t n_samples, int32_t codebook_size, int32_t head_dim) {
  if (n_samples < 0 || check_vq(0, head_dim, codebook_size) != TL_OK) return 0;
  return tl::vq_kmeans_workspace(n_samples, codebook_size, head_dim);
}

int tl_vq_kmeans(const void* data, void* book, int32_t n_samples, int32_t codebook_size, int32_t head_dim,
                 int32_t n_iterations, void* workspace, size_t workspace_bytes, void* stream) {
  int rc = check_vq(n_samples, head_dim, codebook_size);
  if (rc) return rc;
  if (n_iterations < 0) return fail(TL_ERR_INVALID_ARGUMENT, "n_iterations=%d", n_iterations);
  if (n_samples == 0 || n_iterations == 0) return ok();
  if (!data || !book || !workspace) return fail(TL_ERR_INVALID_ARGUMENT, "NULL pointer");
  if (!aligned16(book)) return fail(TL_ERR_INVALID_ARGUMENT, "book must be 16-byte aligned");
  const size_t need = tl::vq_kmeans_workspace(n_samples, codebook_size, head_dim);
  if (workspace_bytes < need)
    return fail(TL_ERR_INVALID_ARGUMENT, "workspace of %zu bytes needed, %zu given", need, workspace_bytes);
  if (tl::launch_vq_kmeans(data, book, n_samples, codebook_size, head_dim, n_iterations, workspace,
                           (hipStream_t)stream))
    return fail(TL_ERR_BACKEND, "vq_kmeans launch failed");
  return ok();
}

int tl_copy_blocks(void* k_cache, void* v_cache, const int32_t* block_mapping, int32_t num_pairs,
                   int32_t num_blocks, int64_t block_bytes, void* stream) {
  if (num_pairs < 0 || num_blocks <= 0 || block_bytes <= 0)
    return fail(TL_ERR_INVALID_ARGUMENT, "num_pairs=%d num_blocks=%d block_bytes=%lld", num_pairs, num_blocks,
                (long long)block_bytes);
  if (num_pairs == 0) return ok();
  if (!k_cache || !v_cache || !block_mapping) return fail(TL_ERR_INVALID_ARGUMENT, "NULL pointer");
  tl::BlockCopy c = {(const char*)k_cache, (const char*)v_cache, (char*)k_cache, (char*)v_cache,
                     block_mapping, num_pairs, 2, num_blocks, num_blocks, block_bytes, 0};
  const int rc = tl::launch_block_copy(c, (hipStream_t)stream);
  if (rc == 3) return fail(TL_ERR_NOT_IMPLEMENTED, "copy_blocks grid too large: %d pairs", num_pairs);
  if (rc) return fail(TL_ERR_BACKEND, "copy_blocks launch failed");
  return ok();
}

int tl_swap_blocks(void* cache, void* host_cache, const int32_t* block_mapping, int32_t num_pairs,
                   int32_t num_device_blocks, int32_t num_host_blocks, int64_t block_bytes,
                   int32_t direction, void* stream) {
  if (num_pairs < 0 || num_device_blocks <= 0 || num_host_blocks <= 0 || block_bytes <= 0)
    return fail(TL_ERR_INVALID_ARGUMENT, "num_pairs=%d num_device_blocks=%d num_host_blocks=%d block_bytes=%lld",
                num_pairs, num_device_blocks, num_host_blocks, (long long)block_bytes);
  if (direction != 0 && direction != 1) return fail(TL_ERR_INVALID_ARGUMENT, "direction=%d", direction);
  if (num_pairs == 0) return ok();
  if (!cache || !host_cache || !block_mapping) return fail(TL_ERR_INVALID_ARGUMENT, "NULL pointer");
  const bool out = direction == 0;
  tl::BlockCopy c = {(const char*)(out ? cache : host_cache), nullptr, (char*)(out ? host_cache : cache), nullptr,
                     block_mapping, num_pairs, 1, out ? num_device_blocks : num_host_blocks,
                     out ? num_host_blocks : num_device_blocks, block_bytes, 0};
  const int rc = tl::launch_block_copy(c, (hipStream_t)stream);
  if (rc == 3) return fail(TL_ERR_NOT_IMPLEMENTED, "swap_blocks grid too large: %d pairs", num_pairs);
  if (rc) return fail(TL_ERR_BACKEND, "swap_blocks launch failed");
  return ok();
}

int tl_reshape_and_cache_fp8(const void* key, const void* value, int32_t src_dtype,
                             uint8_t* k_cache, uint8_t* v_cache, const int32_t* slot_mapping,
                             int32_t num_tokens, int32_t num_kv_heads, int32_t head_size,
                             int32_t block_size, int32_t num_blocks, float k_scale, float v_scale,
                             void* stream) {
  if (num_tokens < 0 || num_kv_heads <= 0 || head_size <= 0 || block_size <= 0 || num_blocks <= 0)
    return fail(TL_ERR_INVALID_ARGUMENT, "bad sizes");
  if (src_dtype != TL_DTYPE_F16 && src_dtype != TL_DTYPE_BF16)
    return fail(TL_ERR_NOT_IMPLEMENTED, "src_dtype=%d (F16 or BF16 sources)", src_dtype);
  if (head_size % 8) return fail(TL_ERR_INVALID_ARGUMENT, "head_size=%d must be a multiple of 8", head_size);
  if (num_tokens == 0) return ok();
  if (!key || !value || !k_cache || !v_cache || !slot_mapping)
    return fail(TL_ERR_INVALID_ARGUMENT, "NULL tensor pointer");
  if (!aligned16(key) || !aligned16(value))
    return fail(TL_ERR_INVALID_ARGUMENT, "key/value must be 16-byte aligned");
  tl::CacheLaunch a = {key, value, k_cache, v_cache, slot_mapping, num_tokens, num_kv_heads,
                       head_size, block_size, num_blocks, src_dtype, TL_DTYPE_FP8_E4M3, k_scale,
                       v_scale, (hipStream_t)stream};
  const int rc = tl::launch_reshape_and_cache(a);
  if (rc == 3) return fail(TL_ERR_NOT_IMPLEMENTED, "no fp8 cache kernel for src_dtype=%d", src_dtype);
  if (rc) return fail(TL_ERR_BACKEND, "reshape_and_cache_fp8 launch failed");
  return ok();
}

int tl_convert_fp8(uint8_t* out, const void* in, int32_t in_dtype, int64_t n, float scale, void* stream) {
  if (n < 0) return fail(TL_ERR_INVALID_ARGUMENT, "n=%lld < 0", (long long)n);
  if (!is_float_kind(in_dtype)) return fail(TL_ERR_INVALID_ARGUMENT, "in_dtype=%d is not F32/F16/BF16", in_dtype);
  if (n == 0) return ok();
  if (!out || !in) return fail(TL_ERR_INVALID_ARGUMENT, "NULL tensor pointer");
  if (in_dtype != TL_DTYPE_F32 && ((uintptr_t)in & 1u)) return fail(TL_ERR_INVALID_ARGUMENT, "in misaligned");
  if (in_dtype == TL_DTYPE_F32 && ((uintptr_t)in & 3u)) return fail(TL_ERR_INVALID_ARGUMENT, "in misaligned");
  const int rc = tl::launch_convert_fp8(out, in, in_dtype, n, scale, (hipStream_t)stream);
  if (rc) return fail(TL_ERR_BACKEND, "convert_fp8 launch failed");
  return ok();
}

int tl_fp8_absmax_scale(const void* x, int32_t dtype, int64_t n, float* scale_out, void* stream) {
  if (n < 0 || !scale_out || (n > 0 && !x)) return fail(TL_ERR_INVALID_ARGUMENT, "bad arguments");
  if (!is_float_kind(dtype)) return fail(TL_ERR_INVALID_ARGUMENT, "dtype=%d", dtype);
  if (((uintptr_t)scale_out & 3u) != 0) return fail(TL_ERR_INVALID_ARGUMENT, "scale_out misaligned");
  const int rc = tl::launch_fp8_scale(x, dtype, n, scale_out, (hipStream_t)stream);
  if (rc) return fail(TL_ERR_BACKEND, "fp8 scale launch failed");
  return ok();
}

// ---------------------------------------------------------------------------
// KIVI
// ---------------------------------------------------------------------------

size_t tl_kivi_compressed_bytes(int32_t head_dim, int32_t n_outliers, int32_t group_size) {
  if (group_size <= 0) return 0;
  const int n_res = head_dim - n_outliers;
  const int n_groups = (n_res + group_size - 1) / group_size;
  return (size_t)n_outliers * 3 + (size_t)n_groups * (size_t)(group_size / 2 + 4);
}

int tl_kivi_params_supported(int32_t head_dim, int32_t n_outliers, int32_t group_size) {
  return head_dim > 0 && head_dim <= TL_KIVI_MAX_HEAD_DIM && n_outliers >= 0 &&
         n_outliers <= TL_KIVI_MAX_OUTLIERS && group_size > 0 && n_outliers <= head_dim;
}

static int kivi_vec(const void* in, void* out, int32_t n_vecs, int32_t head_dim, int32_t n_outliers,
                    int32_t group_size, bool compress, void* stream) {
  if (n_vecs < 0) return fail(TL_ERR_INVALID_ARGUMENT, "n_vecs=%d", n_vecs);
  if (!tl_kivi_params_supported(head_dim, n_outliers, group_size))
    return fail(TL_ERR_INVALID_ARGUMENT, "unsupported KIVI params head_dim=%d n_outliers=%d group_size=%d",
                head_dim, n_outliers, group_size);
  if (group_size % 2)
    return fail(TL_ERR_INVALID_ARGUMENT, "odd group_size=%d: records would overrun the stride", group_size);
  if (n_vecs == 0) return ok();
  if (!in || !out) return fail(TL_ERR_INVALID_ARGUMENT, "NULL pointer");
  const int stride = (int)tl_kivi_compressed_bytes(head_dim, n_outliers, group_size);
  if (tl::launch_kivi_vec(in, out, n_vecs, head_dim, n_outliers, group_size, stride, compress,
                          (hipStream_t)stream))
    return fail(TL_ERR_BACKEND, "KIVI codec launch failed");
  return ok();
}

int tl_kivi_compress(const void* kv_in, uint8_t* out, int32_t n_vecs, int32_t head_dim,
                     int32_t n_outliers, int32_t group_size, void* stream) {
  return kivi_vec(kv_in, out, n_vecs, head_dim, n_outliers, group_size, true, stream);
}

int tl_kivi_decompress(const uint8_t* in, void* kv_out, int32_t n_vecs, int32_t head_dim,
                       int32_t n_outliers, int32_t group_size, void* stream) {
  return kivi_vec(in, kv_out, n_vecs, head_dim, n_outliers, group_size, false, stream);
}

int32_t tl_kivi_quantized_len(int32_t seq_len, int32_t residual_length) {
  if (seq_len < 0 || residual_length < 0) return 0;
  return tl::kivi_quantized_len(seq_len, residual_length);
}

static int check_kivi(const tl_kivi_desc* d) {
  if (!d) return fail(TL_ERR_INVALID_ARGUMENT, "desc is NULL");
  if (d->num_seqs < 0) return fail(TL_ERR_INVALID_ARGUMENT, "num_seqs=%d", d->num_seqs);
  if (d->num_kv_heads <= 0 || d->num_heads <= 0 || d->num_heads % d->num_kv_heads)
    return fail(TL_ERR_INVALID_ARGUMENT, "num_heads=%d / num_kv_heads=%d", d->num_heads, d->num_kv_heads);
  if (d->head_size != tl::kKiviHead)
    return fail(TL_ERR_NOT_IMPLEMENTED, "paged KIVI is built for head_size 128");
  if (d->block_size < 8 || d->block_size > 256 || (d->block_size & (d->block_size - 1)))
    return fail(TL_ERR_NOT_IMPLEMENTED, "paged KIVI block_size=%d (built: powers of two 8 .. 256)", d->block_size);
  if (d->max_blocks_per_seq <= 0 || d->num_blocks <= 0 || d->max_pages_per_seq <= 0 || d->num_pages <= 0)
    return fail(TL_ERR_INVALID_ARGUMENT, "table and pool sizes must be > 0");
  if (d->residual_length < 0) return fail(TL_ERR_INVALID_ARGUMENT, "residual_length=%d", d->residual_length);
  if (d->gqa_map != TL_GQA_MODULO && d->gqa_map != TL_GQA_GROUPED)
    return fail(TL_ERR_INVALID_ARGUMENT, "gqa_map=%d", d->gqa_map);
  if (d->partition_pages < -1) return fail(TL_ERR_INVALID_ARGUMENT, "partition_pages=%d", d->partition_pages);
  if (d->bits != 0 && d->bits != 4 && d->bits != 8)
    return fail(TL_ERR_NOT_IMPLEMENTED, "paged KIVI bits=%d (built: 4, 8)", d->bits);
  if (d->pre_rope_keys != 0 && d->pre_rope_keys != 1)
    return fail(TL_ERR_INVALID_ARGUMENT, "pre_rope_keys=%d", d->pre_rope_keys);
  if (d->build_ahead != 0 && d->build_ahead != 1)
    return fail(TL_ERR_INVALID_ARGUMENT, "build_ahead=%d", d->build_ahead);
  return TL_OK;
}

// Keys held before RoPE: the tables the kernels rotate them with.
struct KiviRope {
  const float* cos_table;
  const float* sin_table;
  int32_t max_positions, style;
};

// The decode scores a key of position t = 32 p + j (page p) with the
// rotation of t0 = 32 p on q and that of j on the key (R_t = R_t0 R_j, the
// tables' angles being linear in the position), so the tables must cover
// every position the call scores.
static int check_kivi_rope(const KiviRope& r, int32_t max_context_len) {
  if (r.max_positions <= 0) return fail(TL_ERR_INVALID_ARGUMENT, "max_positions=%d", r.max_positions);
  if (r.max_positions < max_context_len)
    return fail(TL_ERR_INVALID_ARGUMENT, "rope tables of max_positions=%d do not cover max_context_len=%d",
                r.max_positions, max_context_len);
  if (r.style != TL_ROPE_ADJACENT && r.style != TL_ROPE_HALVES)
    return fail(TL_ERR_INVALID_ARGUMENT, "style=%d", r.style);
  if (!r.cos_table || !r.sin_table) return fail(TL_ERR_INVALID_ARGUMENT, "NULL rope table");
  if (((uintptr_t)r.cos_table | (uintptr_t)r.sin_table) % 16)
    return fail(TL_ERR_INVALID_ARGUMENT, "rope tables must be 16-byte aligned");
  return TL_OK;
}

static int refuse_pre_rope(const tl_kivi_desc* d) {
  return d->pre_rope_keys ? fail(TL_ERR_INVALID_ARGUMENT,
                                 "desc->pre_rope_keys: keys held before RoPE need the rope tables "
                                 "(the _pre_rope entry points)")
                          : TL_OK;
}

static int kivi_bits(const tl_kivi_desc* d) { return d->bits == 8 ? 8 : 4; }

size_t tl_kivi_page_bytes(int32_t bits) {
  if (bits != 0 && bits != 4 && bits != 8) return 0;
  return (size_t)tl::kivi_page_bytes(bits == 8 ? 8 : 4);
}

static tl::KiviPageLaunch page_launch(const tl_kivi_desc* d, const void* k_cache, const void* v_cache,
                                      const int32_t* bt, const int32_t* sl, const int32_t* pt,
                                      void* pages, void* stream) {
  tl::KiviPageLaunch a;
  memset(&a, 0, sizeof a);
  a.k_cache = const_cast<void*>(k_cache); a.v_cache = const_cast<void*>(v_cache);
  a.block_tables = bt; a.seq_lens = sl;
  a.page_tables = pt; a.pages = pages;
  a.num_seqs = d->num_seqs; a.num_kv_heads = d->num_kv_heads; a.block_size = d->block_size;
  a.max_blocks_per_seq = d->max_blocks_per_seq; a.num_blocks = d->num_blocks;
  a.max_pages_per_seq = d->max_pages_per_seq; a.num_pages = d->num_pages;
  a.residual_length = d->residual_length;
  a.bits = kivi_bits(d);
  a.build_ahead = d->build_ahead && d->residual_length >= tl::kKiviAheadMinResidual;
  a.stream = (hipStream_t)stream;
  return a;
}

int tl_kivi_build_pages(const tl_kivi_desc* desc, const void* k_cache, const void* v_cache,
                        const int32_t* block_tables, const int32_t* seq_lens,
                        const int32_t* page_tables, void* pages, int32_t max_context_len,
                        void* stream) {
  int rc = check_kivi(desc);
  if (rc) return rc;
  if (max_context_len < 0) return fail(TL_ERR_INVALID_ARGUMENT, "max_context_len < 0");
  if (desc->num_seqs == 0) return ok();
  if (!k_cache || !v_cache || !block_tables || !seq_lens || !page_tables || !pages)
    return fail(TL_ERR_INVALID_ARGUMENT, "NULL pointer");
  if (!aligned16(pages)) return fail(TL_ERR_INVALID_ARGUMENT, "pages must be 16-byte aligned");
  tl::KiviPageLaunch a = page_launch(desc, k_cache, v_cache, block_tables, seq_lens, page_tables, pages, stream);
  a.max_pages_to_build = tl::kivi_quantized_len(max_context_len, desc->residual_length) / tl::kKiviPageTokens;
  a.max_pages_to_build += a.build_ahead;   // the next page, once its first piece is due
  if (a.max_pages_to_build > desc->max_pages_per_seq) a.max_pages_to_build = desc->max_pages_per_seq;
  if (tl::launch_kivi_pages(a)) return fail(TL_ERR_BACKEND, "KIVI page launch failed");
  return ok();
}

int tl_kivi_append(const tl_kivi_desc* desc, const void* key, const void* value, void* k_cache,
                   void* v_cache, const int32_t* slot_mapping, const int32_t* block_tables,
                   const int32_t* seq_lens, const int32_t* page_tables, void* pages, void* stream) {
  int rc = check_kivi(desc);
  if (rc) return rc;
  if (desc->num_seqs == 0) return ok();
  if (!key || !value || !k_cache || !v_cache || !slot_mapping || !block_tables || !seq_lens ||
      !page_tables || !pages)
    return fail(TL_ERR_INVALID_ARGUMENT, "NULL pointer");
  if (!aligned16(key) || !aligned16(value) || !aligned16(pages))
    return fail(TL_ERR_INVALID_ARGUMENT, "key/value/pages must be 16-byte aligned");
  tl::KiviPageLaunch a = page_launch(desc, k_cache, v_cache, block_tables, seq_lens, page_tables, pages, stream);
  a.append = 1;
  a.knew = key; a.vnew = value; a.slots = slot_mapping;
  if (tl::launch_kivi_pages(a)) return fail(TL_ERR_BACKEND, "KIVI page launch failed");
  return ok();
}

// rope: the _pre_rope entry points, whose workgroups take at most
// tl::kivi_page_rot_cap(bits) pages
static void kivi_plan(const tl_kivi_desc* d, int32_t max_ctx, bool rope, int* P, int* PP) {
  const int pages = tl::kivi_quantized_len(max_ctx, d->residual_length) / tl::kKiviPageTokens;
  int pp;
  if (d->partition_pages == -1 || pages == 0) {
    pp = pages > 0 ? pages : 1;
  } else if (d->partition_pages > 0) {
    pp = d->partition_pages;
  } else {
    const int group = d->num_heads / d->num_kv_heads;
    const long items = (long)d->num_seqs * d->num_kv_heads * ((group + 3) / 4);
    long want = items > 0 ? (512 + items - 1) / items : 1;
    if (want < 1) want = 1;
    if (want > pages) want = pages;
    pp = (int)((pages + want - 1) / want);
  }
  if (pp > tl::kKiviMaxWgPages) pp = tl::kKiviMaxWgPages;   // a workgroup stages its page ids in LDS
  if (rope && pp > tl::kivi_page_rot_cap(kivi_bits(d))) pp = tl::kivi_page_rot_cap(kivi_bits(d));
  *PP = pp;
  *P = pages > 0 ? (pages + pp - 1) / pp : 1;
}

size_t tl_kivi_workspace_bytes(const tl_kivi_desc* desc, int32_t max_context_len) {
  if (check_kivi(desc) != TL_OK || max_context_len < 0) return 0;
  // the plan of the _pre_rope entry points: at least as many partitions as
  // the other one, so the size serves both
  int P, PP;
  kivi_plan(desc, max_context_len, true, &P, &PP);
  if (P <= 1) return 0;
  const size_t sh = (size_t)desc->num_seqs * desc->num_heads * P;
  return sh * desc->head_size * 4 + 2 * sh * 4;
}

static int kivi_decode_impl(const tl_kivi_desc* desc, void* out, const void* q, const void* pages,
                            const int32_t* page_tables, const void* k_cache, const void* v_cache,
                            const int32_t* block_tables, const int32_t* seq_lens, int32_t max_context_len,
                            void* workspace, size_t workspace_bytes, void* stream,
                            const tl::KiviPageLaunch* append, const KiviRope* rope);

int tl_kivi_paged_attention_decode(const tl_kivi_desc* desc, void* out, const void* q,
                                   const void* pages, const int32_t* page_tables,
                                   const void* k_cache, const void* v_cache,
                                   const int32_t* block_tables, const int32_t* seq_lens,
                                   int32_t max_context_len, void* workspace,
                                   size_t workspace_bytes, void* stream) {
  int rc = check_kivi(desc);
  if (rc || (rc = refuse_pre_rope(desc))) return rc;
  return kivi_decode_impl(desc, out, q, pages, page_tables, k_cache, v_cache, block_tables, seq_lens,
                          max_context_len, workspace, workspace_bytes, stream, nullptr, nullptr);
}

int tl_kivi_paged_attention_decode_pre_rope(const tl_kivi_desc* desc, void* out, const void* q,
                                            const void* pages, const int32_t* page_tables,
                                            const void* k_cache, const void* v_cache,
                                            const int32_t* block_tables, const int32_t* seq_lens,
                                            int32_t max_context_len, const float* cos_table,
                                            const float* sin_table, int32_t max_positions, int32_t style,
                                            void* workspace, size_t workspace_bytes, void* stream) {
  const KiviRope r{cos_table, sin_table, max_positions, style};
  int rc = check_kivi(desc);
  if (rc || (rc = check_kivi_rope(r, max_context_len))) return rc;
  return kivi_decode_impl(desc, out, q, pages, page_tables, k_cache, v_cache, block_tables, seq_lens,
                          max_context_len, workspace, workspace_bytes, stream, nullptr, &r);
}

static int kivi_step_impl(const tl_kivi_desc* desc, void* out, const void* q, const void* key,
                          const void* value, const int32_t* slot_mapping, void* pages,
                          const int32_t* page_tables, void* k_cache, void* v_cache,
                          const int32_t* block_tables, const int32_t* seq_lens, int32_t max_context_len,
                          void* workspace, size_t workspace_bytes, void* stream, const KiviRope* rope) {
  if (desc->num_seqs == 0) return ok();
  if (!key || !value || !slot_mapping) return fail(TL_ERR_INVALID_ARGUMENT, "NULL pointer");
  if (!aligned16(key) || !aligned16(value)) return fail(TL_ERR_INVALID_ARGUMENT, "key/value must be 16-byte aligned");
  tl::KiviPageLaunch a = page_launch(desc, k_cache, v_cache, block_tables, seq_lens, page_tables, pages, stream);
  a.append = 1;
  a.knew = key; a.vnew = value; a.slots = slot_mapping;
  return kivi_decode_impl(desc, out, q, pages, page_tables, k_cache, v_cache, block_tables, seq_lens,
                          max_context_len, workspace, workspace_bytes, stream, &a, rope);
}

int tl_kivi_decode_step(const tl_kivi_desc* desc, void* out, const void* q, const void* key,
                        const void* value, const int32_t* slot_mapping, void* pages,
                        const int32_t* page_tables, void* k_cache, void* v_cache,
                        const int32_t* block_tables, const int32_t* seq_lens, int32_t max_context_len,
                        void* workspace, size_t workspace_bytes, void* stream) {
  int rc = check_kivi(desc);
  if (rc || (rc = refuse_pre_rope(desc))) return rc;
  return kivi_step_impl(desc, out, q, key, value, slot_mapping, pages, page_tables, k_cache, v_cache, block_tables,
                        seq_lens, max_context_len, workspace, workspace_bytes, stream, nullptr);
}

int tl_kivi_decode_step_pre_rope(const tl_kivi_desc* desc, void* out, const void* q, const void* key,
                                 const void* value, const int32_t* slot_mapping, void* pages,
                                 const int32_t* page_tables, void* k_cache, void* v_cache,
                                 const int32_t* block_tables, const int32_t* seq_lens,
                                 int32_t max_context_len, const float* cos_table, const float* sin_table,
                                 int32_t max_positions, int32_t style, void* workspace,
                                 size_t workspace_bytes, void* stream) {
  const KiviRope r{cos_table, sin_table, max_positions, style};
  int rc = check_kivi(desc);
  if (rc || (rc = check_kivi_rope(r, max_context_len))) return rc;
  return kivi_step_impl(desc, out, q, key, value, slot_mapping, pages, page_tables, k_cache, v_cache, block_tables,
                        seq_lens, max_context_len, workspace, workspace_bytes, stream, &r);
}

// The rope step's workspace: the step's split-K partials, then the rotated
// q [S, H, 128] and keys [S, n_kv, 128] (fp16), each 256-byte aligned.
static size_t align256(size_t n) { return (n + 255) / 256 * 256; }
static size_t kivi_rope_q_offset(const tl_kivi_desc* d, int32_t max_ctx) {
  return align256(tl_kivi_workspace_bytes(d, max_ctx));
}

size_t tl_kivi_rope_step_workspace_bytes(const tl_kivi_desc* desc, int32_t max_context_len) {
  if (check_kivi(desc) != TL_OK || max_context_len < 0) return 0;
  const size_t qb = (size_t)desc->num_seqs * desc->num_heads * desc->head_size * 2;
  const size_t kb = (size_t)desc->num_seqs * desc->num_kv_heads * desc->head_size * 2;
  return kivi_rope_q_offset(desc, max_context_len) + align256(qb) + kb;
}

int tl_kivi_rope_decode_step(const tl_kivi_desc* desc, void* out, const void* q, const void* key,
                             const void* value, const int32_t* positions, const float* cos_table,
                             const float* sin_table, int32_t max_positions, int32_t style,
                             const int32_t* slot_mapping, void* pages, const int32_t* page_tables,
                             void* k_cache, void* v_cache, const int32_t* block_tables,
                             const int32_t* seq_lens, int32_t max_context_len, void* workspace,
                             size_t workspace_bytes, void* stream) {
  int rc = check_kivi(desc);
  if (rc) return rc;
  if (max_context_len < 0) return fail(TL_ERR_INVALID_ARGUMENT, "max_context_len < 0");
  if (max_positions <= 0) return fail(TL_ERR_INVALID_ARGUMENT, "max_positions=%d", max_positions);
  if (style != TL_ROPE_ADJACENT && style != TL_ROPE_HALVES) return fail(TL_ERR_INVALID_ARGUMENT, "style=%d", style);
  if (desc->num_seqs == 0) return ok();
  if (!q || !key || !value || !positions || !cos_table || !sin_table)
    return fail(TL_ERR_INVALID_ARGUMENT, "NULL pointer");
  const size_t need = tl_kivi_rope_step_workspace_bytes(desc, max_context_len);
  if (!workspace || workspace_bytes < need)
    return fail(TL_ERR_INVALID_ARGUMENT, "workspace of %zu bytes needed, %zu given", need, workspace_bytes);
  if (!aligned16(workspace)) return fail(TL_ERR_INVALID_ARGUMENT, "workspace must be 16-byte aligned");
  const KiviRope kr{cos_table, sin_table, max_positions, style};
  if (desc->pre_rope_keys && (rc = check_kivi_rope(kr, max_context_len))) return rc;
  const size_t qoff = kivi_rope_q_offset(desc, max_context_len);
  char* q_rot = (char*)workspace + qoff;
  char* k_rot = q_rot + align256((size_t)desc->num_seqs * desc->num_heads * desc->head_size * 2);
  tl::RopeCache r;
  memset(&r, 0, sizeof r);
  r.q = q; r.q_out = q_rot; r.key = key; r.k_out = k_rot;
  r.positions = positions; r.cos_table = cos_table; r.sin_table = sin_table;
  r.num_tokens = desc->num_seqs; r.num_heads = desc->num_heads;
  // keys held before RoPE: q rows only, the keys go to the step as given
  r.num_kv_heads = desc->pre_rope_keys ? 0 : desc->num_kv_heads;
  r.head_size = desc->head_size; r.block_size = desc->block_size; r.num_blocks = desc->num_blocks;
  r.max_positions = max_positions; r.dtype = TL_DTYPE_F16; r.style = style;
  if (tl::launch_rope_rows(r, (hipStream_t)stream)) return fail(TL_ERR_BACKEND, "rope launch failed");
  if (desc->pre_rope_keys)
    return kivi_step_impl(desc, out, q_rot, key, value, slot_mapping, pages, page_tables, k_cache, v_cache,
                          block_tables, seq_lens, max_context_len, workspace, qoff, stream, &kr);
  return kivi_step_impl(desc, out, q_rot, k_rot, value, slot_mapping, pages, page_tables, k_cache, v_cache,
                        block_tables, seq_lens, max_context_len, workspace, qoff, stream, nullptr);
}

int tl_kivi_apply_config(tl_kivi_desc* desc, int32_t bits, int32_t residual_length,
                         const char* key_granularity, const char* value_granularity,
                         int32_t pre_rope_keys) {
  if (!desc) return fail(TL_ERR_INVALID_ARGUMENT, "desc is NULL");
  if (bits != 4 && bits != 8) return fail(TL_ERR_INVALID_ARGUMENT, "bits=%d (KiviConfig: 4 or 8)", bits);
  if (residual_length < 0) return fail(TL_ERR_INVALID_ARGUMENT, "residual_length=%d", residual_length);
  if (!key_granularity || strcmp(key_granularity, "per_channel") != 0)
    return fail(TL_ERR_NOT_IMPLEMENTED, "key_granularity '%s' (built: per_channel)",
                key_granularity ? key_granularity : "(null)");
  if (!value_granularity || strcmp(value_granularity, "per_token") != 0)
    return fail(TL_ERR_NOT_IMPLEMENTED, "value_granularity '%s' (built: per_token)",
                value_granularity ? value_granularity : "(null)");
  if (pre_rope_keys != 0 && pre_rope_keys != 1)
    return fail(TL_ERR_INVALID_ARGUMENT, "pre_rope_keys=%d (0 or 1)", pre_rope_keys);
  desc->bits = bits;
  desc->residual_length = residual_length;
  desc->pre_rope_keys = pre_rope_keys;
  return ok();
}

static int kivi_decode_impl(const tl_kivi_desc* desc, void* out, const void* q, const void* pages,
                            const int32_t* page_tables, const void* k_cache, const void* v_cache,
                            const int32_t* block_tables, const int32_t* seq_lens, int32_t max_context_len,
                            void* workspace, size_t workspace_bytes, void* stream,
                            const tl::KiviPageLaunch* append, const KiviRope* rope) {
  int rc = check_kivi(desc);
  if (rc) return rc;
  if (max_context_len < 0) return fail(TL_ERR_INVALID_ARGUMENT, "max_context_len < 0");
  if (desc->num_seqs == 0) return ok();
  if (!out || !q || !pages || !page_tables || !k_cache || !v_cache || !block_tables || !seq_lens)
    return fail(TL_ERR_INVALID_ARGUMENT, "NULL pointer");
  if (!aligned16(q) || !aligned16(pages) || !aligned16(k_cache) || !aligned16(v_cache))
    return fail(TL_ERR_INVALID_ARGUMENT, "q, pages and pools must be 16-byte aligned");
  int P, PP;
  kivi_plan(desc, max_context_len, rope != nullptr, &P, &PP);
  tl::KiviDecodeLaunch a;
  memset(&a, 0, sizeof a);
  a.out = out; a.q = q; a.pages = pages; a.page_tables = page_tables;
  a.k_cache = k_cache; a.v_cache = v_cache; a.block_tables = block_tables; a.seq_lens = seq_lens;
  a.num_seqs = desc->num_seqs; a.num_heads = desc->num_heads; a.num_kv_heads = desc->num_kv_heads;
  a.block_size = desc->block_size;
  a.max_blocks_per_seq = desc->max_blocks_per_seq; a.num_blocks = desc->num_blocks;
  a.max_pages_per_seq = desc->max_pages_per_seq; a.num_pages = desc->num_pages;
  a.residual_length = desc->residual_length; a.gqa_map = desc->gqa_map;
  a.num_partitions = P; a.partition_pages = PP;
  a.bits = kivi_bits(desc);
  a.scale = desc->scale;
  a.append = append;
  if (rope) {
    a.rope_cos = rope->cos_table; a.rope_sin = rope->sin_table;
    a.rope_max_pos = rope->max_positions; a.rope_style = rope->style;
  }
  a.stream = (hipStream_t)stream;
  if (P > 1) {
    const size_t sh = (size_t)desc->num_seqs * desc->num_heads * P;
    const size_t need = sh * desc->head_size * 4 + 2 * sh * 4;
    if (!workspace || workspace_bytes < need)
      return fail(TL_ERR_INVALID_ARGUMENT, "workspace of %zu bytes needed, %zu given", need, workspace_bytes);
    if (!aligned16(workspace)) return fail(TL_ERR_INVALID_ARGUMENT, "workspace must be 16-byte aligned");
    a.part_o = workspace;
    a.part_m = (float*)((char*)workspace + sh * desc->head_size * 4);
    a.part_l = a.part_m + sh;
  }
  rc = tl::launch_kivi_decode(a);
  if (rc == 3) return fail(TL_ERR_NOT_IMPLEMENTED, "no KIVI decode kernel for this shape");
  if (rc) return fail(TL_ERR_BACKEND, "KIVI decode launch failed");
  return ok();
}

int tl_attention_plan(int32_t max_context_len, int32_t block_size, int32_t head_size, int32_t* use_v2,
                      int32_t* num_partitions, float* scale) {
  if (block_size <= 0 || head_size <= 0 || max_context_len < 0)
    return fail(TL_ERR_INVALID_ARGUMENT, "block_size=%d head_size=%d max_context_len=%d", block_size, head_size,
                max_context_len);
  if (!use_v2 || !num_partitions || !scale) return fail(TL_ERR_INVALID_ARGUMENT, "NULL pointer");
  *use_v2 = (max_context_len / block_size) > 32;
  *num_partitions = *use_v2 ? (max_context_len + 32 * block_size - 1) / (32 * block_size) : 1;
  *scale = 1.f / sqrtf((float)head_size);
  return ok();
}

int32_t tl_max_blocks_per_seq(int32_t num_blocks) { return num_blocks < 2048 ? num_blocks : 2048; }

int tl_build_block_tables(const int32_t* blocks, const int32_t* block_offsets, int32_t num_seqs,
                          int32_t max_blocks_per_seq, int32_t* tables) {
  if (num_seqs < 0 || max_blocks_per_seq <= 0)
    return fail(TL_ERR_INVALID_ARGUMENT, "num_seqs=%d max_blocks_per_seq=%d", num_seqs, max_blocks_per_seq);
  if (num_seqs == 0) return ok();
  if (!block_offsets || !tables) return fail(TL_ERR_INVALID_ARGUMENT, "NULL pointer");
  for (int32_t s = 0; s < num_seqs; ++s) {
    const int32_t n = block_offsets[s + 1] - block_offsets[s];
    if (n < 0 || n > max_blocks_per_seq)
      return fail(TL_ERR_INVALID_ARGUMENT, "sequence %d has %d blocks (max %d)", s, n, max_blocks_per_seq);
    if (n > 0 && !blocks) return fail(TL_ERR_INVALID_ARGUMENT, "NULL blocks");
  }
  for (int32_t s = 0; s < num_seqs; ++s) {
    const int32_t n = block_offsets[s + 1] - block_offsets[s];
    int32_t* row = tables + (size_t)s * max_blocks_per_seq;
    if (n > 0) memcpy(row, blocks + block_offsets[s], (size_t)n * sizeof(int32_t));
    memset(row + n, 0xFF, (size_t)(max_blocks_per_seq - n) * sizeof(int32_t));   // -1 padding
  }
  return ok();
}

int tl_build_slot_mapping(const int32_t* blocks, int32_t num_blocks_of_seq, int32_t block_size,
                          int32_t seq_start_pos, int32_t num_tokens, int32_t* slots) {
  if (block_size <= 0 || seq_start_pos < 0 || num_tokens < 0 || num_blocks_of_seq < 0)
    return fail(TL_ERR_INVALID_ARGUMENT, "block_size=%d seq_start_pos=%d num_tokens=%d", block_size,
                seq_start_pos, num_tokens);
  if (num_tokens == 0) return ok();
  if (!blocks || !slots) return fail(TL_ERR_INVALID_ARGUMENT, "NULL pointer");
  const int64_t last = (int64_t)seq_start_pos + num_tokens - 1;
  if (last / block_size >= num_blocks_of_seq)
    return fail(TL_ERR_INVALID_ARGUMENT, "position %lld needs block %lld of %d", (long long)last,
                (long long)(last / block_size), num_blocks_of_seq);
  for (int32_t i = 0; i < num_tokens; ++i) {
    const int32_t pos = seq_start_pos + i;
    slots[i] = blocks[pos / block_size] * block_size + pos % block_size;
  }
  return ok();
}

int tl_kivi_pass_params(int32_t residual_length, int32_t bits, int32_t head_dim, int32_t* n_outliers,
                        int32_t* group_size, int32_t* enabled) {
  if (!n_outliers || !group_size || !enabled) return fail(TL_ERR_INVALID_ARGUMENT, "NULL pointer");
  *n_outliers = residual_length;
  *group_size = bits == 4 ? 16 : 8;
  *enabled = tl_kivi_params_supported(head_dim, *n_outliers, *group_size);
  return ok();
}

int32_t tl_kivi_pass_runs(int32_t seq_len, int32_t n_kv_heads, int32_t head_dim, int32_t n_outliers,
                          int32_t group_size, size_t scratch_bytes) {
  if (seq_len <= 0 || n_kv_heads <= 0) return 0;
  if (!tl_kivi_params_supported(head_dim, n_outliers, group_size)) return 0;
  const size_t need = (size_t)seq_len * n_kv_heads * tl_kivi_compressed_bytes(head_dim, n_outliers, group_size);
  return need <= scratch_bytes;
}

int tl_chunked_prefill(const tl_prefill_desc* d, void* out, const void* q, const int32_t* cu_q_lens,
                       const void* k_cache, const void* v_cache, const int32_t* block_tables,
                       const int32_t* seq_lens, int32_t total_q, int32_t max_q_len, void* stream) {
  if (!d) return fail(TL_ERR_INVALID_ARGUMENT, "desc is NULL");
  if (d->num_seqs < 0 || total_q < 0 || max_q_len < 0)
    return fail(TL_ERR_INVALID_ARGUMENT, "num_seqs=%d total_q=%d max_q_len=%d must be >= 0",
                d->num_seqs, total_q, max_q_len);
  if (d->num_kv_heads <= 0 || d->num_heads <= 0 || d->num_heads % d->num_kv_heads)
    return fail(TL_ERR_INVALID_ARGUMENT, "num_heads=%d must be a positive multiple of num_kv_heads=%d",
                d->num_heads, d->num_kv_heads);
  if (d->max_blocks_per_seq <= 0 || d->num_blocks <= 0)
    return fail(TL_ERR_INVALID_ARGUMENT, "max_blocks_per_seq=%d and num_blocks=%d must be > 0",
                d->max_blocks_per_seq, d->num_blocks);
  if (d->gqa_map != TL_GQA_MODULO && d->gqa_map != TL_GQA_GROUPED)
    return fail(TL_ERR_INVALID_ARGUMENT, "gqa_map=%d", d->gqa_map);
  if (d->dtype != TL_DTYPE_F16 && d->dtype != TL_DTYPE_BF16)
    return fail(TL_ERR_NOT_IMPLEMENTED, "prefill dtype=%d (built: F16, BF16)", d->dtype);
  const int32_t kv_dtype = d->kv_dtype == 0 ? d->dtype : d->kv_dtype;
  if (kv_dtype != d->dtype && kv_dtype != TL_DTYPE_FP8_E4M3)
    return fail(TL_ERR_NOT_IMPLEMENTED, "prefill kv_dtype=%d with dtype=%d (built: the q type, FP8 E4M3)",
                d->kv_dtype, d->dtype);
  if (kv_dtype == TL_DTYPE_FP8_E4M3 &&
      (!(d->k_scale > 0.f) || !(d->k_scale < INFINITY) || !(d->v_scale > 0.f) || !(d->v_scale < INFINITY)))
    return fail(TL_ERR_INVALID_ARGUMENT, "FP8 pool scales k_scale=%g v_scale=%g must be positive and finite",
                (double)d->k_scale, (double)d->v_scale);
  if (d->head_size != 128 || d->block_size < 8 || d->block_size > 256 || (d->block_size & (d->block_size - 1)))
    return fail(TL_ERR_NOT_IMPLEMENTED, "prefill head_size=%d block_size=%d (built: 128 x powers of two 8..256)",
                d->head_size, d->block_size);
  if (d->num_prefill_seqs < 0 || d->num_prefill_seqs > d->num_seqs)
    return fail(TL_ERR_INVALID_ARGUMENT, "num_prefill_seqs=%d outside [0, %d]", d->num_prefill_seqs,
                d->num_seqs);
  // the prefill kernel takes the row max of unscaled scores
  if (!(d->scale > 0.f) || !(d->scale < INFINITY))
    return fail(TL_ERR_INVALID_ARGUMENT, "scale=%g must be positive and finite", (double)d->scale);
  if (d->num_seqs == 0 || total_q == 0) return ok();
  if (max_q_len > total_q)
    return fail(TL_ERR_INVALID_ARGUMENT, "max_q_len=%d > total_q=%d", max_q_len, total_q);
  // the kernel's row -> (query, head) map is exact below 2^22 tile rows
  if ((int64_t)max_q_len * (d->num_heads / d->num_kv_heads) > (1 << 22) - 256)
    return fail(TL_ERR_NOT_IMPLEMENTED, "max_q_len=%d x group=%d (built: below 2^22 rows per kv head)", max_q_len,
                d->num_heads / d->num_kv_heads);
  if (!out || !q || !cu_q_lens || !k_cache || !v_cache || !block_tables || !seq_lens)
    return fail(TL_ERR_INVALID_ARGUMENT, "NULL pointer");
  if (!aligned16(q) || !aligned16(k_cache) || !aligned16(v_cache))
    return fail(TL_ERR_INVALID_ARGUMENT, "q and the pools must be 16-byte aligned");
  if ((uintptr_t)out & 3) return fail(TL_ERR_INVALID_ARGUMENT, "out must be 4-byte aligned");
  tl::PrefillLaunch a;
  memset(&a, 0, sizeof a);
  a.out = out; a.q = q; a.cu_q_lens = cu_q_lens; a.k_cache = k_cache; a.v_cache = v_cache;
  a.block_tables = block_tables; a.seq_lens = seq_lens;
  a.num_seqs = d->num_seqs; a.num_heads = d->num_heads; a.num_kv_heads = d->num_kv_heads;
  a.block_size = d->block_size; a.max_blocks_per_seq = d->max_blocks_per_seq; a.num_blocks = d->num_blocks;
  a.dtype = d->dtype;   // TL_DTYPE_F16 / BF16 / FP8_E4M3 share the kernels' Kind codes
  a.kv_dtype = kv_dtype;
  a.gqa_map = d->gqa_map; a.max_q_len = max_q_len; a.scale = d->scale;
  a.k_scale = kv_dtype == TL_DTYPE_FP8_E4M3 ? d->k_scale : 1.f;
  a.v_scale = kv_dtype == TL_DTYPE_FP8_E4M3 ? d->v_scale : 1.f;
  a.num_prefill_seqs = d->num_prefill_seqs;
  a.stream = (hipStream_t)stream;
  const int lrc = tl::launch_prefill(a);
  if (lrc == 3) return fail(TL_ERR_NOT_IMPLEMENTED, "no prefill kernel for block_size=%d", d->block_size);
  if (lrc) return fail(TL_ERR_BACKEND, "prefill launch failed");
  return ok();
}

}  // extern "C"
