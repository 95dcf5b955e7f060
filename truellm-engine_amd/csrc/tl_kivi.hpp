// tl_kivi.hpp -- paged KIVI INT4 page format shared by the codec and the
// decode kernel.
//
// A page holds 32 consecutive tokens of one kv head (head size 128):
//   [   0, 2048) K nibbles, 128 chunks of 16 B.  Chunk c = tt*64 + j*16 + u
//                holds token t = tt*16 + u; its dword m (0..3) holds channel
//                octet o = j + 4m, channel 8o + 2i + hb at bit 16*hb + 4i.
//                Masked with 0x000F000F and 0x00F000F0 (and the same after a
//                shift by 8), a dword gives the octet's eight channels in
//                order as fp16 denormal pairs n * 2^-24 (16 n * 2^-24 for
//                channels 2, 3, 6, 7): the A operand of
//                v_mfma_f32_16x16x32_f16 for (token t, k-block m) held by
//                lane group j.
//   [2048, 2560) K (step, zero): octet o -> 8 fp16 steps then 8 fp16 zeros
//                for channels 8o..8o+7 (per channel over the page's tokens).
//   [2560, 4608) V nibbles, 128 chunks of 16 B.  Chunk c = hh*64 + r*16 + u;
//                dword m holds channel (4hh + m)*16 + u for the eight token
//                slots s of lane group r: token 4r + s (s < 4) or
//                16 + 4r + s - 4 (s >= 4), at bit 16*(s&1) + 4*(s>>1).  These
//                are exactly the tokens the q.k MFMA output leaves in lane
//                group r, so the softmax weights feed the p.v MFMA unmoved.
//   [4608, 5120) V (step, zero): (channel group g, lane group r) -> 8 fp16
//                steps then 8 fp16 zeros in slot order (per token over 32
//                channels).
#pragma once

namespace tl {

constexpr int kKiviPageTokens = 32;
constexpr int kKiviHead = 128;
constexpr int kKiviPageBytes = 5120;
constexpr int kKiviKParamOff = 2048;
constexpr int kKiviVNibOff = 2560;
constexpr int kKiviVParamOff = 4608;
constexpr int kKiviMaxHeadDim = 128;   // KIVI_MAX_HEAD_DIM, kivi_cache.cuh:27
constexpr int kKiviMaxOutliers = 64;   // KIVI_MAX_OUTLIERS, kivi_cache.cuh:28
constexpr int kKiviMaxWgPages = 1024;  // pages one decode workgroup takes (ids staged in LDS)

// Tokens of a sequence of length L held in pages: whole pages of the prefix
// that leaves at least residual_length tokens in the fp16 pool.
__host__ __device__ inline int kivi_quantized_len(int L, int residual_length) {
  if (L <= residual_length) return 0;
  return ((L - residual_length) / kKiviPageTokens) * kKiviPageTokens;
}

// V token slot map: token t of a page sits in lane group r at slot s.
__host__ __device__ inline int kivi_v_group(int t) { return t < 16 ? t / 4 : (t - 16) / 4; }
__host__ __device__ inline int kivi_v_slot(int t) { return t < 16 ? t % 4 : 4 + (t - 16) % 4; }
__host__ __device__ inline int kivi_v_token(int r, int s) { return s < 4 ? 4 * r + s : 16 + 4 * r + s - 4; }

}  // namespace tl
