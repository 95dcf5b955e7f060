// tl_kivi.hpp -- paged KIVI page formats (INT4 and INT8) shared by the codec
// and the decode kernel.
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
//
// The INT8 page (KiviConfig.bits = 8, config_schema.h:124) is the INT4 page
// with every 16-byte code chunk widened to 32 bytes, so that a lane's chunk
// covers the same (token, channel) set:
//   [   0, 4096) K codes, 128 chunks of 32 B.  Dword 2m + h holds channels
//                8o + 4h + {0, 2, 1, 3} of octet o = j + 4m in bytes 0..3;
//                masked with 0x00FF00FF (and the same after a shift by 8) it
//                gives channel pairs (0, 1) and (2, 3) as fp16 denormals.
//   [4096, 4608) K (step, zero), as for INT4.
//   [4608, 8704) V codes, 128 chunks of 32 B.  Dword 2m + h holds token
//                slots 4h + {0, 2, 1, 3} of channel (4hh + m)*16 + u.
//   [8704, 9216) V (step, zero), as for INT4.
// Codes: scale = 255 / range, clamp(rint((x - min) * scale), 0, 255).
#pragma once

namespace tl {

// Page geometry by code width: chunk bytes per lane, offsets, page size.
template <int BITS> struct KiviFmt;
template <> struct KiviFmt<4> {
  static constexpr int kChunk = 16, kLevels = 15;
  static constexpr int kKCodes = 0, kKParams = 2048, kVCodes = 2560, kVParams = 4608, kBytes = 5120;
};
template <> struct KiviFmt<8> {
  static constexpr int kChunk = 32, kLevels = 255;
  static constexpr int kKCodes = 0, kKParams = 4096, kVCodes = 4608, kVParams = 8704, kBytes = 9216;
};
inline int kivi_page_bytes(int bits) { return bits == 8 ? KiviFmt<8>::kBytes : KiviFmt<4>::kBytes; }

constexpr int kKiviPageTokens = 32;
constexpr int kKiviHead = 128;
constexpr int kKiviPageBytes = 5120;
constexpr int kKiviKParamOff = 2048;
constexpr int kKiviVNibOff = 2560;
constexpr int kKiviVParamOff = 4608;
constexpr int kKiviMaxHeadDim = 128;   // KIVI_MAX_HEAD_DIM, kivi_cache.cuh:27
constexpr int kKiviMaxOutliers = 64;   // KIVI_MAX_OUTLIERS, kivi_cache.cuh:28
constexpr int kKiviMaxWgPages = 1024;  // pages one decode workgroup takes (ids staged in LDS)
// Pages one decode workgroup takes with the keys held before RoPE: the
// rotations of its pages' first positions are LDS rows filled at its start,
// as many as fit beside the rest of the kernel's LDS at two workgroups per
// CU; the plan splits longer sequences.
__host__ __device__ constexpr int kivi_page_rot_cap(int bits) { return bits == 8 ? 144 : 160; }
// Build-ahead: a page is written in kKiviPieces pieces by the steps before
// the one that quantises it; with R > kKiviPieces the newest token of those
// steps lies past the page.
constexpr int kKiviPieces = 8;
constexpr int kKiviAheadMinResidual = kKiviPieces + 1;

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
