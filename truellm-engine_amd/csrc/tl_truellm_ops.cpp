// tl_truellm_ops.cpp -- the reference-named C++ operators (tl_truellm_ops.h)
// on top of the C ABI.  Each one reads shapes from the TrueBuffer views the
// way the reference's launchers do (paged_attention_v1.cu:177-213,
// paged_attention_v2.cu:176-251, cache_kernels.cu:202-232) and forwards to
// the matching tl_* entry point; a failed call leaves the device untouched
// and prints the reason.
#define TL_OWN_TRUELLM_TYPES 1
#include "tl_truellm_ops.h"

#include "tl_attn.h"

#include <hip/hip_runtime.h>

#include <stdio.h>
#include <string.h>

namespace {

using truellm::DataType;
using truellm::TrueBuffer;

// The reference passes F32 / F16 / BF16 buffers; anything else is not an
// attention dtype.
int32_t tl_dtype_of(const TrueBuffer& b) {
  switch (b.dtype) {
    case DataType::F32: return TL_DTYPE_F32;
    case DataType::F16: return TL_DTYPE_F16;
    case DataType::BF16: return TL_DTYPE_BF16;
    default: return -1;
  }
}

void report(const char* op, int rc) {
  if (rc != TL_OK) fprintf(stderr, "[tlattn] %s: %s\n", op, tl_last_error_string());
}

int32_t dim(const TrueBuffer& b, int i) { return i < b.ndim ? (int32_t)b.shape[i] : 1; }

// Bytes per element of a pool view: the attention dtypes, and 1 for the
// byte-sized types (an FP8 pool is viewed as I8 / Q8 by its owner).
int64_t elem_bytes(const TrueBuffer& b) {
  switch (b.dtype) {
    case DataType::F32: case DataType::I32: return 4;
    case DataType::F16: case DataType::BF16: case DataType::I16: return 2;
    default: return 1;
  }
}

}  // namespace

void reshape_and_cache(const TrueBuffer& key, const TrueBuffer& value, TrueBuffer& kv_cache,
                       const TrueBuffer& slot_mapping, hipStream_t stream) {
  // key [T, n_kv, d]; kv_cache [2N, n_kv, d, bs], V at +N blocks (cache_kernels.cu:202-232)
  const int32_t T = dim(key, 0), n_kv = dim(key, 1), d = dim(key, 2);
  const int32_t N = dim(kv_cache, 0) / 2, bs = dim(kv_cache, 3);
  const int32_t dt = tl_dtype_of(key);
  const size_t elem = dt == TL_DTYPE_F32 ? 4 : 2;
  void* v_cache = (char*)kv_cache.data + (size_t)N * n_kv * d * bs * elem;
  report("reshape_and_cache",
         tl_reshape_and_cache(key.data, value.data, kv_cache.data, v_cache, (const int32_t*)slot_mapping.data,
                              T, n_kv, d, bs, N, dt, stream));
}

void copy_blocks(TrueBuffer& kv_cache, const TrueBuffer& block_mapping, hipStream_t stream) {
  // kv_cache [2N, n_kv, d, bs]: K blocks then V blocks (cache_kernels.cu:234-262)
  const int32_t N = dim(kv_cache, 0) / 2;
  const int64_t bytes = (int64_t)dim(kv_cache, 1) * dim(kv_cache, 2) * dim(kv_cache, 3) * elem_bytes(kv_cache);
  report("copy_blocks", tl_copy_blocks(kv_cache.data, (char*)kv_cache.data + (int64_t)N * bytes,
                                       (const int32_t*)block_mapping.data, dim(block_mapping, 0), N, bytes,
                                       stream));
}

void swap_blocks(TrueBuffer& kv_cache, TrueBuffer& host_cache, const TrueBuffer& block_mapping, int direction,
                 hipStream_t stream) {
  const int64_t bytes = (int64_t)dim(kv_cache, 1) * dim(kv_cache, 2) * dim(kv_cache, 3) * elem_bytes(kv_cache);
  report("swap_blocks", tl_swap_blocks(kv_cache.data, host_cache.data, (const int32_t*)block_mapping.data,
                                       dim(block_mapping, 0), dim(kv_cache, 0), dim(host_cache, 0), bytes,
                                       direction, stream));
}

void convert_fp8(TrueBuffer& out, const TrueBuffer& in, float scale, hipStream_t stream) {
  int64_t n = 1;                                   // tb_numel: the product of the view's dims
  for (int i = 0; i < in.ndim && i < 4; ++i) n *= in.shape[i];
  report("convert_fp8", tl_convert_fp8((uint8_t*)out.data, in.data, tl_dtype_of(in), n, scale, stream));
}

void rms_norm(TrueBuffer& out, const TrueBuffer& x, const TrueBuffer& weight, float eps, hipStream_t stream) {
  report("rms_norm", tl_rms_norm(out.data, x.data, weight.data, dim(x, 0), dim(x, 1), eps, tl_dtype_of(x), stream));
}

void fused_add_rms_norm(TrueBuffer& out, TrueBuffer& residual, const TrueBuffer& x, const TrueBuffer& weight,
                        float eps, hipStream_t stream) {
  report("fused_add_rms_norm", tl_fused_add_rms_norm(out.data, residual.data, x.data, weight.data, dim(x, 0),
                                                     dim(x, 1), eps, tl_dtype_of(x), stream));
}

void layer_norm(TrueBuffer& out, const TrueBuffer& x, const TrueBuffer& weight, const TrueBuffer& bias, float eps,
                hipStream_t stream) {
  report("layer_norm", tl_layer_norm(out.data, x.data, weight.data, bias.data, dim(x, 0), dim(x, 1), eps,
                                     tl_dtype_of(x), stream));
}

static void act_and_mul(const char* name, TrueBuffer& out, const TrueBuffer& gate, const TrueBuffer& up, int act,
                        hipStream_t stream) {
  int64_t n = 1;
  for (int i = 0; i < gate.ndim && i < 4; ++i) n *= gate.shape[i];
  report(name, tl_act_and_mul(out.data, gate.data, up.data, n, act, tl_dtype_of(gate), stream));
}

void silu_and_mul(TrueBuffer& out, const TrueBuffer& gate, const TrueBuffer& up, hipStream_t stream) {
  act_and_mul("silu_and_mul", out, gate, up, TL_ACT_SILU, stream);
}

void gelu_and_mul(TrueBuffer& out, const TrueBuffer& gate, const TrueBuffer& up, hipStream_t stream) {
  act_and_mul("gelu_and_mul", out, gate, up, TL_ACT_GELU, stream);
}

void gelu_tanh_and_mul(TrueBuffer& out, const TrueBuffer& gate, const TrueBuffer& up, hipStream_t stream) {
  act_and_mul("gelu_tanh_and_mul", out, gate, up, TL_ACT_GELU_TANH, stream);
}

void paged_attention_v1(TrueBuffer& out, const TrueBuffer& q, const TrueBuffer& k_cache,
                        const TrueBuffer& v_cache, const TrueBuffer& block_tables,
                        const TrueBuffer& seq_lens, int num_kv_heads, float scale, int head_size,
                        int block_size, hipStream_t stream) {
  const int32_t S = dim(q, 0), H = dim(q, 1);
  report("paged_attention_v1",
         tl_paged_attention_v1(out.data, q.data, k_cache.data, v_cache.data, (const int32_t*)block_tables.data,
                               (const int32_t*)seq_lens.data, S, H, num_kv_heads, head_size, block_size,
                               dim(block_tables, 1), dim(k_cache, 0), scale, tl_dtype_of(q), TL_GQA_MODULO,
                               stream));
}

void paged_attention_v2(TrueBuffer& out, TrueBuffer& exp_sums, TrueBuffer& max_logits, TrueBuffer& tmp_out,
                        const TrueBuffer& q, const TrueBuffer& k_cache, const TrueBuffer& v_cache,
                        const TrueBuffer& block_tables, const TrueBuffer& seq_lens, int num_kv_heads,
                        float scale, int head_size, int block_size, int max_context_len, hipStream_t stream) {
  const int32_t S = dim(q, 0), H = dim(q, 1);
  report("paged_attention_v2",
         tl_paged_attention_v2(out.data, (float*)exp_sums.data, (float*)max_logits.data, tmp_out.data, q.data,
                               k_cache.data, v_cache.data, (const int32_t*)block_tables.data,
                               (const int32_t*)seq_lens.data, S, H, num_kv_heads, head_size, block_size,
                               dim(block_tables, 1), dim(k_cache, 0), scale, tl_dtype_of(q), TL_GQA_MODULO,
                               max_context_len, stream));
}

namespace truellm {

void vq_encode(const __half* d_kv, const __half* d_book, uint16_t* d_idx, int seq_len, int n_kv_heads,
               int head_dim, int codebook_size, hipStream_t stream) {
  report("vq_encode", tl_vq_encode(d_kv, d_book, d_idx, seq_len * n_kv_heads, head_dim, codebook_size, stream));
}

void vq_decode(__half* d_kv, const __half* d_book, const uint16_t* d_idx, int seq_len, int n_kv_heads,
               int head_dim, hipStream_t stream) {
  report("vq_decode", tl_vq_decode(d_kv, d_book, d_idx, seq_len * n_kv_heads, head_dim, 65536, stream));
}

void codebook_init_kmeans(const void* d_data, void* d_book, int n_samples, int codebook_size, int head_dim,
                          int n_iterations, hipStream_t stream) {
  const size_t ws = tl_vq_kmeans_workspace_bytes(n_samples, codebook_size, head_dim);
  void* work = nullptr;
  if (ws == 0 || hipMalloc(&work, ws) != hipSuccess) {
    fprintf(stderr, "[tlattn] codebook_init_kmeans: no workspace (%zu bytes)\n", ws);
    return;
  }
  report("codebook_init_kmeans",
         tl_vq_kmeans(d_data, d_book, n_samples, codebook_size, head_dim, n_iterations, work, ws, stream));
  (void)hipStreamSynchronize(stream);
  (void)hipFree(work);
}

bool kivi_params_supported(int head_dim, int n_outliers, int group_size) {
  return tl_kivi_params_supported(head_dim, n_outliers, group_size) != 0;
}

void kivi_compress(const __half* d_kv_in, uint8_t* d_out, int n_vecs, int head_dim, int n_outliers,
                   int group_size, hipStream_t stream) {
  if (n_vecs <= 0 || !kivi_params_supported(head_dim, n_outliers, group_size)) return;
  report("kivi_compress", tl_kivi_compress(d_kv_in, d_out, n_vecs, head_dim, n_outliers, group_size, stream));
}

void kivi_decompress(const uint8_t* d_in, __half* d_kv_out, int n_vecs, int head_dim, int n_outliers,
                     int group_size, hipStream_t stream) {
  if (n_vecs <= 0 || !kivi_params_supported(head_dim, n_outliers, group_size)) return;
  report("kivi_decompress",
         tl_kivi_decompress(d_in, d_kv_out, n_vecs, head_dim, n_outliers, group_size, stream));
}

}  // namespace truellm

namespace {

int manifest_initialize(void*) {
  int dev = 0;
  hipDeviceProp_t prop;
  if (hipGetDevice(&dev) != hipSuccess || hipGetDeviceProperties(&prop, dev) != hipSuccess) return 1;
  return strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? 0 : 1;
}

void manifest_shutdown(void*) {}

truellm_kernel_manifest_t g_manifest = {
    TRUELLM_KERNEL_ABI_VERSION, "tlattn_paged_attention_gfx950", "0.1.0", TRUELLM_KERNEL_ATTENTION,
    9, 5, manifest_initialize, manifest_shutdown, nullptr,
};

}  // namespace

extern "C" truellm_kernel_manifest_t* truellm_kernel_init(void) { return &g_manifest; }
