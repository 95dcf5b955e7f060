/* tl_truellm_ops.h -- drop-in C++ operators with the reference's names and
 * argument lists, routed through the C ABI of tl_attn.h.
 *
 * The reference engine declares these functions itself
 * (src/inference/backends/cuda/cuda_engine.cpp:46-62 and the test
 * tests/test_vllm_kernels.cpp:25-34) and links them from a static library
 * (third_party/vllm_kernels/CMakeLists.txt:25-38).  libtlattn.so exports the
 * same symbols (C++ mangling with truellm::TrueBuffer and hipStream_t in
 * place of cudaStream_t), so a ROCm build of those call sites links against
 * it unchanged.
 *
 * Semantics kept from the reference: q/out [S, H, d], pools [N, n_kv, d, bs]
 * (reshape_and_cache: one [2N, n_kv, d, bs] buffer, V at +N blocks), the
 * MODULO GQA mapping kv_head = h % n_kv, v2's exp_sums / max_logits /
 * tmp_out with P = ceil(max_context_len / (32 bs)) partitions, void returns.
 * Error behaviour matches the reference's release build (its asserts are
 * compiled out): an unsupported or invalid call does nothing; the reason is
 * printed to stderr and stays readable through tl_last_error_string().
 *
 * Types: with TL_OWN_TRUELLM_TYPES defined this header declares
 * truellm::DataType, truellm::TrueBuffer and truellm_kernel_manifest_t with
 * the reference's layouts (include/truellm/types.h:47-77,
 * include/truellm/kernel.h:23-57); otherwise the engine's own
 * <truellm/types.h> and <truellm/kernel.h> must be included first.
 */
#ifndef TL_TRUELLM_OPS_H
#define TL_TRUELLM_OPS_H

#include <hip/hip_fp16.h>
#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <cstdint>

#ifdef TL_OWN_TRUELLM_TYPES
namespace truellm {
/* include/truellm/types.h:47-60 */
enum class DataType : uint8_t {
  F32 = 0, F16 = 1, BF16 = 2, I32 = 3, I16 = 4, I8 = 5,
  Q8_0 = 10, Q4_0 = 11, Q4_1 = 12, Q5_0 = 13, Q5_1 = 14, Q4_K_M = 20,
};
/* include/truellm/types.h:69-77: a non-owning view */
struct TrueBuffer {
  void* data;
  std::size_t size_bytes;
  DataType dtype;
  int32_t device_id;
  int32_t ndim;
  int64_t shape[4];
  int64_t stride[4];
};
}  // namespace truellm

extern "C" {
/* include/truellm/kernel.h:23-57 */
#define TRUELLM_KERNEL_ABI_VERSION 1
typedef enum truellm_kernel_category {
  TRUELLM_KERNEL_ATTENTION = 0,
  TRUELLM_KERNEL_ACTIVATION = 1,
  TRUELLM_KERNEL_LAYERNORM = 2,
  TRUELLM_KERNEL_GEMM = 3,
  TRUELLM_KERNEL_CACHE = 4,
  TRUELLM_KERNEL_CUSTOM = 99,
} truellm_kernel_category_t;
typedef struct truellm_kernel_manifest {
  uint32_t abi_version;
  const char* name;
  const char* version;
  truellm_kernel_category_t category;
  uint32_t min_sm_major;   /* here: the gfx major / minor of the target, 9 / 5 for gfx950 */
  uint32_t min_sm_minor;
  int (*initialize)(void* engine_ctx);
  void (*shutdown)(void* engine_ctx);
  void* kernel_state;
} truellm_kernel_manifest_t;
}
#else
#include <truellm/kernel.h>
#include <truellm/types.h>
#endif

/* cache_kernels.cu:202-207.  key/value [T, n_kv, d]; kv_cache [2N, n_kv, d, bs]. */
void reshape_and_cache(const truellm::TrueBuffer& key, const truellm::TrueBuffer& value,
                       truellm::TrueBuffer& kv_cache, const truellm::TrueBuffer& slot_mapping,
                       hipStream_t stream);

/* cache_kernels.cu:234-238.  kv_cache [2N, n_kv, d, bs] (K blocks, then V);
 * block_mapping int32 [num_pairs, 2] on the device.  Any element type. */
void copy_blocks(truellm::TrueBuffer& kv_cache, const truellm::TrueBuffer& block_mapping, hipStream_t stream);

/* cache_kernels.cu:264-269.  kv_cache [M, n_kv, d, bs] on the device,
 * host_cache [M', n_kv, d, bs] in pinned host memory; block ids index dim 0
 * of each; direction 0: device -> host, 1: host -> device.  The block size
 * is dims 1-3 times the element size (the reference reads shape[4], D16). */
void swap_blocks(truellm::TrueBuffer& kv_cache, truellm::TrueBuffer& host_cache,
                 const truellm::TrueBuffer& block_mapping, int direction, hipStream_t stream);

/* cache_kernels.cu:286-295 (built there for sm_89+ only): out (one byte per
 * element, E4M3) = e4m3(in * scale) over every element of in's shape; in
 * F16, BF16 or F32. */
void convert_fp8(truellm::TrueBuffer& out, const truellm::TrueBuffer& in, float scale, hipStream_t stream);

/* layernorm_kernels.cu:149-211 and activation_kernels.cu:104-132: x / out
 * [num_tokens, hidden] (shape[0], shape[1]), F32, F16 or BF16 (the
 * reference runs anything but F16 as f32). */
void rms_norm(truellm::TrueBuffer& out, const truellm::TrueBuffer& x, const truellm::TrueBuffer& weight, float eps,
              hipStream_t stream);
void fused_add_rms_norm(truellm::TrueBuffer& out, truellm::TrueBuffer& residual, const truellm::TrueBuffer& x,
                        const truellm::TrueBuffer& weight, float eps, hipStream_t stream);
void layer_norm(truellm::TrueBuffer& out, const truellm::TrueBuffer& x, const truellm::TrueBuffer& weight,
                const truellm::TrueBuffer& bias, float eps, hipStream_t stream);
void silu_and_mul(truellm::TrueBuffer& out, const truellm::TrueBuffer& gate, const truellm::TrueBuffer& up,
                  hipStream_t stream);
void gelu_and_mul(truellm::TrueBuffer& out, const truellm::TrueBuffer& gate, const truellm::TrueBuffer& up,
                  hipStream_t stream);
void gelu_tanh_and_mul(truellm::TrueBuffer& out, const truellm::TrueBuffer& gate, const truellm::TrueBuffer& up,
                       hipStream_t stream);

/* paged_attention_v1.cu:177-189 */
void paged_attention_v1(truellm::TrueBuffer& out, const truellm::TrueBuffer& q,
                        const truellm::TrueBuffer& k_cache, const truellm::TrueBuffer& v_cache,
                        const truellm::TrueBuffer& block_tables, const truellm::TrueBuffer& seq_lens,
                        int num_kv_heads, float scale, int head_size, int block_size,
                        hipStream_t stream);

/* paged_attention_v2.cu:176-191 */
void paged_attention_v2(truellm::TrueBuffer& out, truellm::TrueBuffer& exp_sums,
                        truellm::TrueBuffer& max_logits, truellm::TrueBuffer& tmp_out,
                        const truellm::TrueBuffer& q, const truellm::TrueBuffer& k_cache,
                        const truellm::TrueBuffer& v_cache, const truellm::TrueBuffer& block_tables,
                        const truellm::TrueBuffer& seq_lens, int num_kv_heads, float scale,
                        int head_size, int block_size, int max_context_len, hipStream_t stream);

namespace truellm {
/* vq_cache.cu:74-86 */
void vq_encode(const __half* d_kv, const __half* d_book, uint16_t* d_idx, int seq_len, int n_kv_heads,
               int head_dim, int codebook_size, hipStream_t stream);
/* vq_cache.cu:88-100 (no codebook size: indices are trusted, as in the reference) */
void vq_decode(__half* d_kv, const __half* d_book, const uint16_t* d_idx, int seq_len, int n_kv_heads,
               int head_dim, hipStream_t stream);
/* codebook_init.cu:100-145: allocates its workspace and synchronises the
 * stream, as the reference does (tl_vq_kmeans does neither) */
void codebook_init_kmeans(const void* d_data, void* d_book, int n_samples, int codebook_size, int head_dim,
                          int n_iterations, hipStream_t stream);
/* kivi_cache.cu:205-211 */
bool kivi_params_supported(int head_dim, int n_outliers, int group_size);
/* kivi_cache.cu:213-224: no-op for n_vecs <= 0 or unsupported parameters */
void kivi_compress(const __half* d_kv_in, uint8_t* d_out, int n_vecs, int head_dim, int n_outliers,
                   int group_size, hipStream_t stream);
/* kivi_cache.cu:226-238 */
void kivi_decompress(const uint8_t* d_in, __half* d_kv_out, int n_vecs, int head_dim, int n_outliers,
                     int group_size, hipStream_t stream);
}  // namespace truellm

extern "C" {
/* kernel.h:9-12: the plugin entry point.  Returns the ATTENTION manifest of
 * this library (paged_attention_v1/v2; the CACHE operators reshape_and_cache
 * and the KIVI codec live in the same library).  initialize() returns 0 when
 * the current device is gfx950. */
truellm_kernel_manifest_t* truellm_kernel_init(void);
}

#endif /* TL_TRUELLM_OPS_H */
