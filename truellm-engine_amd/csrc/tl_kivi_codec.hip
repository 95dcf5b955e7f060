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
#include "tl_kivi_page.hpp"

#include <float.h>

namespace tl {

namespace {

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
template <int BITS>
__global__ __launch_bounds__(128) void kivi_page_kernel(PageJob j) {
  __shared__ __attribute__((aligned(16))) KiviBuildSmem<BITS> sm;
  const int tid = threadIdx.x;
  int bid = blockIdx.x;
  const int kvh = bid % j.num_kv_heads; bid /= j.num_kv_heads;
  const int pg = bid % j.pages_per_seq_grid;
  const int seq = bid / j.pages_per_seq_grid;
  const int L = j.seq_lens[seq];
  const int lq = kivi_quantized_len(L, j.residual_length);
  int page;
  int ahead_page;
  const int piece = j.build_ahead ? kivi_ahead_piece(L, j.residual_length, ahead_page) : -1;
  if (j.append) {
    kivi_append_token<128>(j, seq, kvh, tid);
    if (j.build_ahead) {
      // the pages this append completes were written in pieces by the
      // appends before it; this one writes its piece of the next page:
      // wavefront 0 stages its fp16, then each wavefront quantises two of
      // its quarters
      if (piece < 0) return;
      __shared__ int s_pid;
      uint16_t* raw = reinterpret_cast<uint16_t*>(&sm.qk[0][0]);
      const int lane = tid % kWave, wave = tid / kWave;
      if (wave == 0) {
        KiviPiece pc = kivi_piece_plan(j, seq, ahead_page, piece, lane);
        kivi_piece_load(j, pc, kvh, ahead_page, lane);
        kivi_piece_stage(pc, lane, raw);
        if (lane == 0) s_pid = pc.piece >= 0 ? pc.pid : -1;
      }
      __syncthreads();
      const int pid = s_pid;
      if (pid < 0) return;
      for (int q = wave; q < 4; q += 128 / kWave)
        kivi_piece_quarter<BITS>(j, pid, piece, kvh, q, lane, kivi_piece_quarter_values(piece, q, lane, raw),
                                 &sm.qv[0][0] + 256 * q);
      return;
    }
    if (lq == 0 || lq == kivi_quantized_len(L - 1, j.residual_length)) return;
    page = lq / kKiviPageTokens - 1;
  } else {
    page = pg;
    // build-ahead: the next page too once its first piece is due (every
    // piece written so far and the rest ahead of time: the same bytes)
    if (page >= lq / kKiviPageTokens && !(piece >= 0 && page == ahead_page)) return;
  }
  kivi_build_page<128, BITS>(sm, j, seq, kvh, page, L, tid);
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
  if (!a.append && a.max_pages_to_build <= 0) return 0;
  const PageJob j = make_page_job(a);
  const dim3 grid((unsigned)(a.num_seqs * j.pages_per_seq_grid * a.num_kv_heads));
  if (a.bits == 8)
    hipLaunchKernelGGL(kivi_page_kernel<8>, grid, dim3(128), 0, a.stream, j);
  else
    hipLaunchKernelGGL(kivi_page_kernel<4>, grid, dim3(128), 0, a.stream, j);
  return hipGetLastError() == hipSuccess ? 0 : 5;
}

}  // namespace tl
