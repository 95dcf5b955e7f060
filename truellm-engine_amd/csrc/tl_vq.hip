// tl_vq.hip -- the VQ codec of the KV cache (vq_cache.cu, codebook_init.cu)
// for gfx950.
//
// Encode (vq_cache.cu:18-43): for each vector x (fp16, head_dim) the index
// of the codebook entry at the smallest L2 distance,
//   dist_c = fold over d = 0 .. head_dim-1 of fma(x_d - b_cd, x_d - b_cd, dist)
// in fp32 in that order (the reference's loop under default contraction),
// the first c with dist_c < the best so far (best starts at FLT_MAX): the
// lowest index wins ties, and NaN / >= FLT_MAX distances are never chosen
// (all of them: index 0).  Each distance is computed whole by one thread in
// the reference's order, so the indices are the reference's exactly.
//
// A workgroup takes 16 vectors (staged as fp32 in LDS) and all entries:
// thread t owns entries t, t + 256, ...; it streams its entry's row from
// global memory (L2-resident: 64 KiB for 256 x 128) and keeps 16 running
// distances; the per-vector argmin is a (distance, index) minimum over the
// workgroup.  Roofline: fp32 VALU (2 ops per (vector, entry, dim)).
//
// Decode (vq_cache.cu:48-69): out[v] = book[idx[v]], 16-byte chunks.
//
// k-means (codebook_init.cu:23-145): Lloyd iterations on the device, as the
// reference's assign / accumulate / normalise kernels, except that the sums
// are exact and order-independent: each fp16 value is an integer multiple of
// 2^-24, so the sums are int64 fixed point (atomic adds commute), and
// non-finite values are tracked as flags with IEEE sum semantics (NaN, or
// +inf with -inf, gives NaN).  The reference accumulates fp32 with atomics
// in arrival order, which no two runs need to repeat.  New centroid =
// fp16(fp32(sum) * (1 / count)); an empty cluster keeps its centroid.
#include "tl_device.hpp"
#include "tl_internal.hpp"

#include <float.h>

namespace tl {

namespace {

constexpr int kVqThreads = 256, kVqVecs = 16;

__device__ __forceinline__ bool vq_better(float d, int c, float bd, int bc) {
  return d < bd || (d == bd && c < bc);
}

// One lane's (distance, index) against lane ^ o's.
__device__ __forceinline__ void vq_min_xor(float& d, int& c, int o) {
  const float d2 = __shfl_xor(d, o, kWave);
  const int c2 = __shfl_xor(c, o, kWave);
  if (vq_better(d2, c2, d, c)) { d = d2; c = c2; }
}

__global__ __launch_bounds__(kVqThreads) void vq_assign_kernel(VqArgs a) {
  __shared__ float s_x[kVqVecs][kVqMaxDim];
  __shared__ float s_d[kVqThreads / kWave][kVqVecs];
  __shared__ int s_c[kVqThreads / kWave][kVqVecs];
  const int tid = threadIdx.x, hd = a.head_size;
  const int64_t v0 = (int64_t)blockIdx.x * kVqVecs;
  const int nv = (int)min<int64_t>(kVqVecs, a.num_vecs - v0);
  for (int i = tid; i < kVqVecs * hd; i += kVqThreads) {
    const int v = i / hd, d = i % hd;
    s_x[v][d] = v < nv ? f16_to_f32(a.vecs[(v0 + v) * hd + d]) : 0.f;
  }
  __syncthreads();

  // invalid (NaN or >= FLT_MAX) distances never win: they enter as +inf
  // with an index past every entry
  float best[kVqVecs];
  int bi[kVqVecs];
#pragma unroll
  for (int v = 0; v < kVqVecs; ++v) { best[v] = INFINITY; bi[v] = 0x7fffffff; }
  for (int c = tid; c < a.codebook_size; c += kVqThreads) {
    const uint16_t* row = a.book + (int64_t)c * hd;
    float dist[kVqVecs];
#pragma unroll
    for (int v = 0; v < kVqVecs; ++v) dist[v] = 0.f;
    for (int d0 = 0; d0 < hd; d0 += 8) {
      const u32x4 w = load16(row + d0);
      const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float b = f16_to_f32((uint16_t)(ww[j / 2] >> (16 * (j & 1))));
#pragma unroll
        for (int v = 0; v < kVqVecs; ++v) {
          const float diff = s_x[v][d0 + j] - b;
          dist[v] = __builtin_fmaf(diff, diff, dist[v]);
        }
      }
    }
#pragma unroll
    for (int v = 0; v < kVqVecs; ++v)
      if (dist[v] < FLT_MAX && vq_better(dist[v], c, best[v], bi[v])) { best[v] = dist[v]; bi[v] = c; }
  }

  const int lane = tid % kWave, wave = tid / kWave;
#pragma unroll
  for (int v = 0; v < kVqVecs; ++v) {
    float d = best[v];
    int c = bi[v];
#pragma unroll
    for (int o = kWave / 2; o >= 1; o >>= 1) vq_min_xor(d, c, o);
    if (lane == 0) { s_d[wave][v] = d; s_c[wave][v] = c; }
  }
  __syncthreads();
  if (tid < nv) {
    float d = s_d[0][tid];
    int c = s_c[0][tid];
    for (int w = 1; w < kVqThreads / kWave; ++w)
      if (vq_better(s_d[w][tid], s_c[w][tid], d, c)) { d = s_d[w][tid]; c = s_c[w][tid]; }
    if (c == 0x7fffffff) c = 0;
    if (a.idx16) a.idx16[v0 + tid] = (uint16_t)c;
    if (a.idx32) a.idx32[v0 + tid] = c;
  }
}

__global__ __launch_bounds__(256) void vq_decode_kernel(uint16_t* __restrict__ out, const uint16_t* __restrict__ book,
                                                        const uint16_t* __restrict__ idx, int64_t num_vecs,
                                                        int head_size, int codebook_size) {
  const int chunks = head_size / 8;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= num_vecs * chunks) return;
  const int64_t v = i / chunks;
  const int ch = (int)(i % chunks);
  const int c = idx[v];
  if (c >= codebook_size) return;                      // row left as it is
  *reinterpret_cast<u32x4*>(out + v * head_size + 8 * ch) = load16(book + (int64_t)c * head_size + 8 * ch);
}

// k-means workspace: assign int32 [n], sums int64 [K, d], flags int32 [K, d],
// counts int32 [K].
__global__ void vq_zero_kernel(uint32_t* p, int64_t n_words) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n_words;
       i += (int64_t)gridDim.x * blockDim.x)
    p[i] = 0u;
}

__global__ __launch_bounds__(256) void vq_accumulate_kernel(const uint16_t* __restrict__ data,
                                                            const int32_t* __restrict__ assign,
                                                            unsigned long long* __restrict__ sums,
                                                            int32_t* __restrict__ flags, int32_t* __restrict__ counts,
                                                            int64_t n, int head_size) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n * head_size) return;
  const int64_t s = i / head_size;
  const int d = (int)(i % head_size);
  const int c = assign[s];
  if (d == 0) atomicAdd(&counts[c], 1);
  const float x = f16_to_f32(data[i]);
  const int64_t k = (int64_t)c * head_size + d;
  if (x != x) {
    atomicOr(&flags[k], 1);
  } else if (x == INFINITY) {
    atomicOr(&flags[k], 2);
  } else if (x == -INFINITY) {
    atomicOr(&flags[k], 4);
  } else {
    // exact: |x| 2^24 < 2^40, and two's complement adds commute
    atomicAdd(&sums[k], (unsigned long long)(long long)(x * 16777216.0f));
  }
}

__global__ __launch_bounds__(256) void vq_normalise_kernel(uint16_t* __restrict__ book,
                                                           const unsigned long long* __restrict__ sums,
                                                           const int32_t* __restrict__ flags,
                                                           const int32_t* __restrict__ counts, int codebook_size,
                                                           int head_size) {
  const int64_t k = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (k >= (int64_t)codebook_size * head_size) return;
  const int cnt = counts[k / head_size];
  if (cnt == 0) return;                                // empty cluster: keep the centroid
  const int f = flags[k];
  float sum;
  if ((f & 1) || (f & 6) == 6) sum = __builtin_nanf("");
  else if (f & 2) sum = INFINITY;
  else if (f & 4) sum = -INFINITY;
  else sum = (float)(long long)sums[k] * (1.0f / 16777216.0f);   // one rounding, then exact scaling
  const float inv = 1.f / (float)cnt;
  // the fp32 product, then fp16: the empty asm keeps the compiler from
  // fusing the multiply and the conversion into one mixed FMA (v_fma_mixlo,
  // a single rounding)
  float mean = sum * inv;
  asm volatile("" : "+v"(mean));
  book[k] = f32_to_f16(mean);
}

}  // namespace

int launch_vq_assign(const VqArgs& a, hipStream_t stream) {
  if (a.num_vecs <= 0) return 0;
  const int64_t grid = (a.num_vecs + kVqVecs - 1) / kVqVecs;
  if (grid > 0x7fffffff) return 3;
  hipLaunchKernelGGL(vq_assign_kernel, dim3((unsigned)grid), dim3(kVqThreads), 0, stream, a);
  return hipGetLastError() == hipSuccess ? 0 : 5;
}

int launch_vq_decode(void* out, const void* book, const uint16_t* idx, int64_t num_vecs, int head_size,
                     int codebook_size, hipStream_t stream) {
  if (num_vecs <= 0) return 0;
  const int64_t total = num_vecs * (head_size / 8);
  hipLaunchKernelGGL(vq_decode_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream,
                     (uint16_t*)out, (const uint16_t*)book, idx, num_vecs, head_size, codebook_size);
  return hipGetLastError() == hipSuccess ? 0 : 5;
}

size_t vq_kmeans_workspace(int64_t n, int codebook_size, int head_size) {
  const size_t kd = (size_t)codebook_size * head_size;
  return (size_t)n * 4 + kd * 8 + kd * 4 + (size_t)codebook_size * 4 + 64;
}

int launch_vq_kmeans(const void* data, void* book, int64_t n, int codebook_size, int head_size, int iterations,
                     void* workspace, hipStream_t stream) {
  const size_t kd = (size_t)codebook_size * head_size;
  char* w = (char*)(((uintptr_t)workspace + 15) & ~(uintptr_t)15);
  unsigned long long* sums = (unsigned long long*)w;
  int32_t* flags = (int32_t*)(w + kd * 8);
  int32_t* counts = flags + kd;
  int32_t* assign = counts + codebook_size;
  const int64_t zero_words = (int64_t)kd * 3 + codebook_size;   // sums, flags, counts
  VqArgs a = {(const uint16_t*)data, (const uint16_t*)book, nullptr, assign, n, head_size, codebook_size};
  for (int it = 0; it < iterations; ++it) {
    if (launch_vq_assign(a, stream)) return 5;
    hipLaunchKernelGGL(vq_zero_kernel, dim3(256), dim3(256), 0, stream, (uint32_t*)w, zero_words);
    const int64_t tot = n * head_size;
    hipLaunchKernelGGL(vq_accumulate_kernel, dim3((unsigned)((tot + 255) / 256)), dim3(256), 0, stream,
                       (const uint16_t*)data, assign, sums, flags, counts, n, head_size);
    hipLaunchKernelGGL(vq_normalise_kernel, dim3((unsigned)((kd + 255) / 256)), dim3(256), 0, stream,
                       (uint16_t*)book, sums, flags, counts, codebook_size, head_size);
    if (hipGetLastError() != hipSuccess) return 5;
  }
  return 0;
}

}  // namespace tl
