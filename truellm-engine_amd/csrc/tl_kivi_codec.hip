// tl_kivi_codec.hip -- KIVI INT4 codecs for gfx950.
//
// 1. The reference vector codec (kivi_cache.cu:23-198): per vector, the top
//    n_outliers |x| channels stored raw as fp16 with a u8 index, the other
//    channels min/max quantised to 4 bits in groups of group_size with an
//    fp16 (step, zero) pair.  Bit-exact with the reference's fp32 IEEE
//    arithmetic: correctly rounded division, rint, no contraction of
//    (x - gmin) * scale, and the fused multiply-add nvcc forms for
//    nibble * step + zero on decode.  One thread per vector, as the record
//    format is produced by a sequential outlier scan.
//
// 2. The paged KIVI format: per kv head, a page holds 32 tokens quantised
//    with the same group quantiser, K per channel over the 32 tokens and V
//    per token over groups of 32 channels (KIVI's key/value granularities,
//    config_schema.h:122-129), laid out so a dequantised dword is a ready
//    MFMA operand (see tl_kivi.hpp).  One workgroup builds one page.
#include "tl_device.hpp"
#include "tl_internal.hpp"
#include "tl_kivi.hpp"

#include <float.h>

namespace tl {

namespace {

// __float2int_rn then the clamp to [0, 15] of kivi_cache.cu:109-112.
__device__ __forceinline__ int quant_nibble(float v) {
  const float r = __builtin_rintf(v);
  if (!(r >= 0.0f)) return 0;  // negative or NaN
  if (r > 15.0f) return 15;
  return (int)r;
}

// min/max scan of kivi_cache.cu:97-104; returns degenerate flag and scale.
struct GroupQ {
  float gmin, scale;
  uint16_t step, zero;
};

__device__ __forceinline__ GroupQ group_params(float gmin, float gmax) {
  GroupQ g;
  const float range = gmax - gmin;
  const bool degenerate = !(range > 1e-6f);
  g.gmin = gmin;
  g.scale = degenerate ? 0.0f : (15.0f / range);
  const float st = degenerate ? 0.0f : (1.0f / g.scale);
  const bool gmin_ok = (gmin == gmin) && (gmin > -FLT_MAX) && (gmin < FLT_MAX);
  g.step = f32_to_f16(st);
  g.zero = f32_to_f16(gmin_ok ? gmin : 0.0f);
  return g;
}

__device__ __forceinline__ int quantise(float x, const GroupQ& g) {
  const float d = x - g.gmin;
  return quant_nibble(d * g.scale);
}

__global__ __launch_bounds__(128) void kivi_vec_compress_kernel(
    const uint16_t* __restrict__ in, uint8_t* __restrict__ out, int n_vecs, int head_dim,
    int n_outliers, int group_size, int stride) {
  const int v = blockIdx.x * blockDim.x + threadIdx.x;
  if (v >= n_vecs) return;
  const uint16_t* src = in + (int64_t)v * head_dim;
  uint8_t* p = out + (int64_t)v * stride;
  const int n_out = n_outliers;

  // top-n_outliers |x| by the reference's replace-the-first-minimum scan
  uint8_t oidx[kKiviMaxOutliers];
  float omag[kKiviMaxOutliers];
  for (int i = 0; i < n_out; ++i) { oidx[i] = 0; omag[i] = -1.f; }
  float min_mag = -1.f;
  int min_pos = 0;
  for (int d = 0; d < head_dim; ++d) {
    const float a = __builtin_fabsf(f16_to_f32(src[d]));
    if (a > min_mag) {
      if (n_out > 0) { oidx[min_pos] = (uint8_t)d; omag[min_pos] = a; }
      min_mag = n_out > 0 ? omag[0] : a;
      min_pos = 0;
      for (int i = 1; i < n_out; ++i)
        if (omag[i] < min_mag) { min_mag = omag[i]; min_pos = i; }
    }
  }
  bool is_out[kKiviMaxHeadDim];
  for (int d = 0; d < head_dim; ++d) is_out[d] = false;
  for (int i = 0; i < n_out; ++i) is_out[oidx[i]] = true;
  for (int i = 0; i < n_out; ++i) {
    const uint16_t h = src[oidx[i]];
    p[0] = oidx[i];
    p[1] = (uint8_t)(h & 0xff);
    p[2] = (uint8_t)(h >> 8);
    p += 3;
  }
  const int n_res = head_dim - n_out;
  const int n_groups = (n_res + group_size - 1) / group_size;
  float res[kKiviMaxHeadDim];
  int r = 0;
  for (int d = 0; d < head_dim && r < n_res; ++d)
    if (!is_out[d]) res[r++] = f16_to_f32(src[d]);
  for (int g = 0; g < n_groups; ++g) {
    const int g0 = g * group_size, g1 = min(g0 + group_size, n_res);
    float gmin = FLT_MAX, gmax = -FLT_MAX;
    for (int i = g0; i < g1; ++i) {
      if (res[i] < gmin) gmin = res[i];
      if (res[i] > gmax) gmax = res[i];
    }
    const GroupQ q = group_params(gmin, gmax);
    for (int i = g0; i < g1; i += 2) {
      const int q0 = quantise(res[i], q);
      const int q1 = (i + 1 < g1) ? quantise(res[i + 1], q) : 0;
      *p++ = (uint8_t)((q1 << 4) | q0);
    }
    p[0] = (uint8_t)(q.step & 0xff); p[1] = (uint8_t)(q.step >> 8);
    p[2] = (uint8_t)(q.zero & 0xff); p[3] = (uint8_t)(q.zero >> 8);
    p += 4;
  }
}

__global__ __launch_bounds__(128) void kivi_vec_decompress_kernel(
    const uint8_t* __restrict__ in, uint16_t* __restrict__ out, int n_vecs, int head_dim,
    int n_outliers, int group_size, int stride) {
  const int v = blockIdx.x * blockDim.x + threadIdx.x;
  if (v >= n_vecs) return;
  const uint8_t* p = in + (int64_t)v * stride;
  uint16_t* dst = out + (int64_t)v * head_dim;
  const int n_out = n_outliers;
  float result[kKiviMaxHeadDim];
  bool written[kKiviMaxHeadDim];
  for (int d = 0; d < head_dim; ++d) { result[d] = 0.f; written[d] = false; }
  for (int i = 0; i < n_out; ++i) {
    const int ch = p[0];
    const uint16_t h = (uint16_t)(p[1] | (p[2] << 8));
    p += 3;
    if (ch < head_dim) { result[ch] = f16_to_f32(h); written[ch] = true; }
  }
  const int n_res = head_dim - n_out;
  const int n_groups = (n_res + group_size - 1) / group_size;
  int rch[kKiviMaxHeadDim];
  int r = 0;
  for (int d = 0; d < head_dim && r < n_res; ++d)
    if (!written[d]) rch[r++] = d;
  for (int g = 0; g < n_groups; ++g) {
    const int g0 = g * group_size, g1 = min(g0 + group_size, n_res);
    const uint8_t* pack = p;
    p += (g1 - g0 + 1) / 2;
    const float st = f16_to_f32((uint16_t)(p[0] | (p[1] << 8)));
    const float ze = f16_to_f32((uint16_t)(p[2] | (p[3] << 8)));
    p += 4;
    for (int i = g0; i < g1; ++i) {
      const int k = i - g0;
      const int nib = (k % 2 == 0) ? (pack[k / 2] & 0x0f) : (pack[k / 2] >> 4);
      if (i < r) result[rch[i]] = __builtin_fmaf((float)nib, st, ze);
    }
  }
  for (int d = 0; d < head_dim; ++d) dst[d] = f32_to_f16(result[d]);
}

// ---------------------------------------------------------------------------
// Paged KIVI: build one page (32 tokens x 128 channels of one kv head) from
// the fp16 pool [N, n_kv, 128, BS].
// ---------------------------------------------------------------------------
struct PageJob {
  uint16_t* k_cache;        // written only by append (the new token)
  uint16_t* v_cache;
  const int32_t* block_tables;
  const int32_t* seq_lens;
  const int32_t* page_tables;
  uint8_t* pages;
  int num_kv_heads, block_size, max_blocks_per_seq, num_blocks;
  int max_pages_per_seq, num_pages, residual_length;
  int pages_per_seq_grid;   // grid stride over page index (prefix build)
  int append;               // 1: write the new token, then the page that L completes, if any
  const uint16_t* knew;     // append: new token per sequence [S, n_kv, 128]
  const uint16_t* vnew;
  const int32_t* slots;     // append: its slot in the fp16 pool
};

__global__ __launch_bounds__(128) void kivi_page_kernel(PageJob j) {
  constexpr int T = kKiviPageTokens, D = kKiviHead;
  __shared__ uint16_t s_k[D][T + 2];      // [channel][token] (+2 breaks bank conflicts)
  __shared__ uint16_t s_v[T][D + 2];      // [token][channel]
  __shared__ uint8_t s_qk[D][T];          // K nibbles [channel][token]
  __shared__ uint8_t s_qv[T][D];          // V nibbles [token][channel]
  __shared__ __attribute__((aligned(16))) uint8_t s_page[kKiviPageBytes];

  const int tid = threadIdx.x;
  int bid = blockIdx.x;
  const int kvh = bid % j.num_kv_heads; bid /= j.num_kv_heads;
  const int pg = bid % j.pages_per_seq_grid;
  const int seq = bid / j.pages_per_seq_grid;
  const int L = j.seq_lens[seq];
  const int lq = kivi_quantized_len(L, j.residual_length);
  int page;
  const int64_t new_off = ((int64_t)seq * j.num_kv_heads + kvh) * D;
  if (j.append) {
    // the new token (position L - 1) into the fp16 pool, one channel per thread
    const int32_t slot = j.slots[seq];
    const int blk = slot >= 0 ? slot / j.block_size : -1;
    if (blk >= 0 && blk < j.num_blocks) {
      const int64_t off = (((int64_t)blk * j.num_kv_heads + kvh) * D + tid) * j.block_size + slot % j.block_size;
      j.k_cache[off] = j.knew[new_off + tid];
      j.v_cache[off] = j.vnew[new_off + tid];
    }
    if (lq == 0 || lq == kivi_quantized_len(L - 1, j.residual_length)) return;
    page = lq / T - 1;
  } else {
    page = pg;
    if (page >= lq / T) return;
  }
  if (page >= j.max_pages_per_seq) return;
  const int pid = j.page_tables[(int64_t)seq * j.max_pages_per_seq + page];
  if (pid < 0 || pid >= j.num_pages) return;

  // gather the 32 tokens: element (token t, channel c) of the fp16 pool
  for (int i = tid; i < T * D; i += 128) {
    const int c = i / T, t = i % T;
    const int tok = page * T + t;
    const int lb = tok / j.block_size;
    int phys = (lb < j.max_blocks_per_seq) ? j.block_tables[(int64_t)seq * j.max_blocks_per_seq + lb] : -1;
    if (phys >= j.num_blocks) phys = -1;
    uint16_t kv = 0, vv = 0;
    if (j.append && tok == L - 1) {          // just written by this workgroup: take it from the input
      kv = j.knew[new_off + c];
      vv = j.vnew[new_off + c];
    } else if (phys >= 0) {
      const int64_t off = (((int64_t)phys * j.num_kv_heads + kvh) * D + c) * j.block_size + tok % j.block_size;
      kv = j.k_cache[off];
      vv = j.v_cache[off];
    }
    s_k[c][t] = kv;
    s_v[t][c] = vv;
  }
  __syncthreads();

  // K: one thread per channel, its 32 tokens in order
  {
    const int c = tid;
    float gmin = FLT_MAX, gmax = -FLT_MAX;
    for (int t = 0; t < T; ++t) {
      const float x = f16_to_f32(s_k[c][t]);
      if (x < gmin) gmin = x;
      if (x > gmax) gmax = x;
    }
    const GroupQ q = group_params(gmin, gmax);
    for (int t = 0; t < T; ++t) s_qk[c][t] = (uint8_t)quantise(f16_to_f32(s_k[c][t]), q);
    uint16_t* kp = reinterpret_cast<uint16_t*>(s_page + kKiviKParamOff + (c / 8) * 32);
    kp[c % 8] = q.step;
    kp[8 + c % 8] = q.zero;
  }
  // V: one thread per (token, group of 32 channels), channels in order
  {
    const int t = tid / 4, g = tid % 4;
    float gmin = FLT_MAX, gmax = -FLT_MAX;
    for (int i = 0; i < 32; ++i) {
      const float x = f16_to_f32(s_v[t][g * 32 + i]);
      if (x < gmin) gmin = x;
      if (x > gmax) gmax = x;
    }
    const GroupQ q = group_params(gmin, gmax);
    for (int i = 0; i < 32; ++i) s_qv[t][g * 32 + i] = (uint8_t)quantise(f16_to_f32(s_v[t][g * 32 + i]), q);
    const int r = kivi_v_group(t), s = kivi_v_slot(t);
    uint16_t* vp = reinterpret_cast<uint16_t*>(s_page + kKiviVParamOff + (g * 4 + r) * 32);
    vp[s] = q.step;
    vp[8 + s] = q.zero;
  }
  __syncthreads();

  // nibble dwords: 512 for K then 512 for V
  uint32_t* pw = reinterpret_cast<uint32_t*>(s_page);
  for (int w = tid; w < 512; w += 128) {
    // K dword w: chunk c = w / 4 (= tt*64 + jj*16 + u), dword m = w % 4
    const int ch = w / 4, m = w % 4;
    const int t = (ch / 64) * 16 + ch % 16, o = (ch % 64) / 16 + 4 * m;
    uint32_t x = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x |= (uint32_t)s_qk[8 * o + 2 * i][t] << (4 * i);
      x |= (uint32_t)s_qk[8 * o + 2 * i + 1][t] << (16 + 4 * i);
    }
    pw[w] = x;
    // V dword w: chunk c = hh*64 + r*16 + u, channel (4 hh + m)*16 + u
    const int hh = ch / 64, r = (ch % 64) / 16, u = ch % 16;
    const int d = (4 * hh + m) * 16 + u;
    uint32_t y = 0;
#pragma unroll
    for (int s = 0; s < 8; ++s)
      y |= (uint32_t)s_qv[kivi_v_token(r, s)][d] << (16 * (s & 1) + 4 * (s >> 1));
    pw[kKiviVNibOff / 4 + w] = y;
  }
  __syncthreads();

  uint8_t* dst = j.pages + ((int64_t)pid * j.num_kv_heads + kvh) * kKiviPageBytes;
  for (int i = tid; i < kKiviPageBytes / 16; i += 128)
    reinterpret_cast<u32x4*>(dst)[i] = reinterpret_cast<const u32x4*>(s_page)[i];
}

}  // namespace

int launch_kivi_vec(const void* in, void* out, int n_vecs, int head_dim, int n_outliers,
                    int group_size, int stride, bool compress, hipStream_t stream) {
  const dim3 grid((unsigned)((n_vecs + 127) / 128));
  if (compress)
    hipLaunchKernelGGL(kivi_vec_compress_kernel, grid, dim3(128), 0, stream, (const uint16_t*)in,
                       (uint8_t*)out, n_vecs, head_dim, n_outliers, group_size, stride);
  else
    hipLaunchKernelGGL(kivi_vec_decompress_kernel, grid, dim3(128), 0, stream, (const uint8_t*)in,
                       (uint16_t*)out, n_vecs, head_dim, n_outliers, group_size, stride);
  return hipGetLastError() == hipSuccess ? 0 : 5;
}

int launch_kivi_pages(const KiviPageLaunch& a) {
  PageJob j;
  j.k_cache = (uint16_t*)a.k_cache; j.v_cache = (uint16_t*)a.v_cache;
  j.block_tables = a.block_tables; j.seq_lens = a.seq_lens; j.page_tables = a.page_tables;
  j.pages = (uint8_t*)a.pages;
  j.num_kv_heads = a.num_kv_heads; j.block_size = a.block_size;
  j.max_blocks_per_seq = a.max_blocks_per_seq; j.num_blocks = a.num_blocks;
  j.max_pages_per_seq = a.max_pages_per_seq; j.num_pages = a.num_pages;
  j.residual_length = a.residual_length;
  j.append = a.append;
  j.knew = (const uint16_t*)a.knew; j.vnew = (const uint16_t*)a.vnew; j.slots = a.slots;
  j.pages_per_seq_grid = a.append ? 1 : (a.max_pages_to_build > 0 ? a.max_pages_to_build : 1);
  if (!a.append && a.max_pages_to_build <= 0) return 0;
  const dim3 grid((unsigned)(a.num_seqs * j.pages_per_seq_grid * a.num_kv_heads));
  hipLaunchKernelGGL(kivi_page_kernel, grid, dim3(128), 0, a.stream, j);
  return hipGetLastError() == hipSuccess ? 0 : 5;
}

}  // namespace tl
