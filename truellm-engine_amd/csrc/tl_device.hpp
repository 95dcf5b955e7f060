// tl_device.hpp -- gfx950 device helpers shared by the attention kernels.
//
// Element types, packed unpacking to fp32, 64-lane wavefront reductions and
// the transpose-reduce used to finish per-lane partial dot products.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tl {

constexpr int kWave = 64;

// Storage kinds of the KV pool.  F16/BF16/F32 follow truellm::DataType
// (include/truellm/types.h:47-60); FP8 is OCP E4M3 ("E4M3FN", max 448), the
// format gfx950's v_cvt_*_fp8 instructions implement.
enum class Kind : int { F32 = 0, F16 = 1, BF16 = 2, FP8 = 32 };

template <Kind K> struct KindInfo;
template <> struct KindInfo<Kind::F32>  { static constexpr int bytes = 4; };
template <> struct KindInfo<Kind::F16>  { static constexpr int bytes = 2; };
template <> struct KindInfo<Kind::BF16> { static constexpr int bytes = 2; };
template <> struct KindInfo<Kind::FP8>  { static constexpr int bytes = 1; };

typedef float  f32x2 __attribute__((ext_vector_type(2)));
typedef float  f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

// ---- scalar conversions ----------------------------------------------------

__device__ __forceinline__ float f16_to_f32(uint16_t h) {
  return (float)__builtin_bit_cast(_Float16, h);
}
__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return __builtin_bit_cast(float, (uint32_t)h << 16);
}
// Round to nearest even; NaN stays NaN (quiet).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t x = __builtin_bit_cast(uint32_t, f);
  if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40u);
  x += 0x7fffu + ((x >> 16) & 1u);
  return (uint16_t)(x >> 16);
}
// IEEE round to nearest even (v_cvt_f16_f32 under the default mode).
__device__ __forceinline__ uint16_t f32_to_f16(float f) {
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}

template <Kind K> __device__ __forceinline__ float load_scalar(const void* p, int64_t i);
template <> __device__ __forceinline__ float load_scalar<Kind::F32>(const void* p, int64_t i) {
  return ((const float*)p)[i];
}
template <> __device__ __forceinline__ float load_scalar<Kind::F16>(const void* p, int64_t i) {
  return f16_to_f32(((const uint16_t*)p)[i]);
}
template <> __device__ __forceinline__ float load_scalar<Kind::BF16>(const void* p, int64_t i) {
  return bf16_to_f32(((const uint16_t*)p)[i]);
}

template <Kind K> __device__ __forceinline__ void store_scalar(void* p, int64_t i, float v);
template <> __device__ __forceinline__ void store_scalar<Kind::F32>(void* p, int64_t i, float v) {
  ((float*)p)[i] = v;
}
template <> __device__ __forceinline__ void store_scalar<Kind::F16>(void* p, int64_t i, float v) {
  ((uint16_t*)p)[i] = f32_to_f16(v);
}
template <> __device__ __forceinline__ void store_scalar<Kind::BF16>(void* p, int64_t i, float v) {
  ((uint16_t*)p)[i] = f32_to_bf16(v);
}

// ---- FP8 E4M3 ------------------------------------------------------------
// Two codes (bytes 0,1 or 2,3 of w) to fp32 with the hardware converter.
template <bool HI>
__device__ __forceinline__ f32x2 fp8x2_to_f32(uint32_t w) {
  return __builtin_amdgcn_cvt_pk_f32_fp8(w, HI);
}
// fp32 -> E4M3 with round to nearest even and saturation to +-448
// (NaN stays NaN).  The clamp makes the saturation explicit instead of
// relying on the converter's clamp mode.
__device__ __forceinline__ uint8_t f32_to_fp8(float v) {
  float c = __builtin_fminf(__builtin_fmaxf(v, -448.0f), 448.0f);
  c = (v != v) ? v : c;
  return (uint8_t)(__builtin_amdgcn_cvt_pk_fp8_f32(c, c, 0u, false) & 0xffu);
}

// ---- unpack one dword of KV storage into fp32 -------------------------------
// F16/BF16: 2 elements per dword; FP8: 4 elements per dword.
template <Kind K> struct Unpack;
template <> struct Unpack<Kind::F16> {
  static constexpr int per_dword = 2;
  __device__ __forceinline__ static void run(uint32_t w, float* f) {
    f[0] = f16_to_f32((uint16_t)(w & 0xffffu));
    f[1] = f16_to_f32((uint16_t)(w >> 16));
  }
};
template <> struct Unpack<Kind::BF16> {
  static constexpr int per_dword = 2;
  __device__ __forceinline__ static void run(uint32_t w, float* f) {
    f[0] = __builtin_bit_cast(float, w << 16);
    f[1] = __builtin_bit_cast(float, w & 0xffff0000u);
  }
};
template <> struct Unpack<Kind::FP8> {
  static constexpr int per_dword = 4;
  __device__ __forceinline__ static void run(uint32_t w, float* f) {
    f32x2 lo = fp8x2_to_f32<false>(w), hi = fp8x2_to_f32<true>(w);
    f[0] = lo.x; f[1] = lo.y; f[2] = hi.x; f[3] = hi.y;
  }
};

// ---- 16-byte global loads ---------------------------------------------------
struct alignas(16) u32x4 { uint32_t x, y, z, w; };

// Dword w (0..3) of a 16-byte chunk.
__device__ __forceinline__ uint32_t word(const u32x4& c, int w) {
  return w == 0 ? c.x : w == 1 ? c.y : w == 2 ? c.z : c.w;
}

__device__ __forceinline__ u32x4 load16(const void* p) {
  return *reinterpret_cast<const u32x4*>(p);
}

// Streaming 16-byte load (non-temporal hint): KV bytes are read once per
// decode step, so they should not displace reusable lines in L2 / MALL.
typedef unsigned u32v4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ u32x4 load16_stream(const void* p) {
  const u32v4 v = __builtin_nontemporal_load(reinterpret_cast<const u32v4*>(p));
  return u32x4{v.x, v.y, v.z, v.w};
}

// Loads through a buffer descriptor built in scalar registers: base and
// byte range are wave-uniform, offsets per lane, and the hardware returns
// zeros without a memory request for offsets at or past the range (an
// empty range: a load that may be issued unconditionally).  Word 3 is the
// raw-buffer format of CDNA; aux 2 = non-temporal.
constexpr int kBufferWord3 = 0x00020000;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, unsigned bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, kBufferWord3);
}
__device__ __forceinline__ u32x4 buffer_load16(__amdgpu_buffer_rsrc_t r, unsigned off) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 2));
}

// ---- wavefront reductions ----------------------------------------------------
__device__ __forceinline__ float shfl_xor(float v, int mask) {
  return __shfl_xor(v, mask, kWave);
}

template <int FIRST, int LAST>   // xor masks FIRST, FIRST/2, ..., LAST
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int m = FIRST; m >= LAST; m >>= 1) v = __builtin_fmaxf(v, shfl_xor(v, m));
  return v;
}
template <int FIRST, int LAST>
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = FIRST; m >= LAST; m >>= 1) v += shfl_xor(v, m);
  return v;
}

// Transpose-reduce: N per-lane partial values are summed across the lanes
// that differ in the bits of MASK_HI, MASK_HI/2, ..., MASK_LO.  At every
// level each lane keeps one half of its values and adds the partner's copy
// of that half, so N values over 2^k lanes cost N*(1 - 2^-k) shuffles
// instead of N*k.  On return v[0 .. N>>levels) hold the lane's share; the
// value index of v[i] is base + i, base returned.  Levels past N == 1 fall
// back to plain butterflies.
template <int N, int M, int MLO>
struct TransposeReduce {
  __device__ __forceinline__ static void run(float* v, int lane, int& base) {
    if constexpr (N > 1) {
      constexpr int H = N / 2;
      const bool up = (lane & M) != 0;
#pragma unroll
      for (int i = 0; i < H; ++i) {
        const float keep = up ? v[i + H] : v[i];
        const float give = up ? v[i] : v[i + H];
        v[i] = keep + shfl_xor(give, M);
      }
      base += up ? H : 0;
      if constexpr (M > MLO) TransposeReduce<H, M / 2, MLO>::run(v, lane, base);
    } else {
      v[0] += shfl_xor(v[0], M);
      if constexpr (M > MLO) TransposeReduce<1, M / 2, MLO>::run(v, lane, base);
    }
  }
};

template <int N, int MASK_HI, int MASK_LO>
__device__ __forceinline__ int transpose_reduce(float* v, int lane) {
  int base = 0;
  if constexpr (MASK_HI >= MASK_LO && MASK_LO >= 1)
    TransposeReduce<N, MASK_HI, MASK_LO>::run(v, lane, base);
  return base;
}

// ---- cross-lane steps that stay in the VALU ---------------------------------
// gfx950 v_permlane16_swap / v_permlane32_swap exchange half-rows between two
// registers.  Fed (lo, hi) they give every lane (own, partner) copies of the
// half it keeps (lo for lanes with bit 4 / bit 5 clear, hi otherwise), so a
// transpose-reduce level is one swap and one add, with no select.
__device__ __forceinline__ float swap16_add(float lo, float hi) {
  const auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(unsigned, lo),
                                                  __builtin_bit_cast(unsigned, hi), false, false);
  return __builtin_bit_cast(float, (unsigned)r[0]) + __builtin_bit_cast(float, (unsigned)r[1]);
}
__device__ __forceinline__ float swap32_add(float lo, float hi) {
  const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, lo),
                                                  __builtin_bit_cast(unsigned, hi), false, false);
  return __builtin_bit_cast(float, (unsigned)r[0]) + __builtin_bit_cast(float, (unsigned)r[1]);
}

// DPP lane reads within a row of 16 lanes.
constexpr int kDppXor1 = 0xB1;         // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;         // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141;  // lane i <- 7 - i within each 8 lanes
constexpr int kDppMirror = 0x140;      // lane i <- 15 - i within each row
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// Max / sum over the 16 lanes of a row (masks 1, 2, 7, 15 span the 4 bits).
__device__ __forceinline__ float row_max(float v) {
  v = __builtin_fmaxf(v, dpp<kDppXor1>(v));
  v = __builtin_fmaxf(v, dpp<kDppXor2>(v));
  v = __builtin_fmaxf(v, dpp<kDppHalfMirror>(v));
  return __builtin_fmaxf(v, dpp<kDppMirror>(v));
}
__device__ __forceinline__ float row_sum(float v) {
  v += dpp<kDppXor1>(v);
  v += dpp<kDppXor2>(v);
  v += dpp<kDppHalfMirror>(v);
  return v + dpp<kDppMirror>(v);
}

// Transpose-reduce of N values over lane bits 5, 4, 1, 0 (in that order).
// Afterwards v[0 .. N/16) of each lane hold the sums of value indices
// base + i with base = (N/2)*b5 + (N/4)*b4 + (N/8)*b1 + (N/16)*b0.
template <int N>
__device__ __forceinline__ void transpose_reduce_5410(float* v, int lane) {
  static_assert(N >= 16 && N % 16 == 0, "16 lanes share the values");
#pragma unroll
  for (int i = 0; i < N / 2; ++i) v[i] = swap32_add(v[i], v[i + N / 2]);
#pragma unroll
  for (int i = 0; i < N / 4; ++i) v[i] = swap16_add(v[i], v[i + N / 4]);
  {
    const bool up = (lane & 2) != 0;
#pragma unroll
    for (int i = 0; i < N / 8; ++i) {
      const float keep = up ? v[i + N / 8] : v[i], give = up ? v[i] : v[i + N / 8];
      v[i] = keep + dpp<kDppXor2>(give);
    }
  }
  {
    const bool up = (lane & 1) != 0;
#pragma unroll
    for (int i = 0; i < N / 16; ++i) {
      const float keep = up ? v[i + N / 16] : v[i], give = up ? v[i] : v[i + N / 16];
      v[i] = keep + dpp<kDppXor1>(give);
    }
  }
}

// Number of values a lane keeps after transpose_reduce<N, HI, LO>.
template <int N, int MASK_HI, int MASK_LO>
constexpr int transpose_kept() {
  int n = N;
  for (int m = MASK_HI; m >= MASK_LO && m >= 1; m >>= 1) n = n > 1 ? n / 2 : 1;
  return n;
}

}  // namespace tl
