// tl_cache.hip -- KV-cache writes for gfx950.
//
// reshape_and_cache (cache_kernels.cu:47-94, :202-232): scatter the new
// tokens' K and V rows [T, n_kv, D] into the paged pools [N, n_kv, D, BS] at
// slot = block * BS + offset; slot < 0 is a padded token and is skipped.
// Each thread moves one 16-byte run of 8 head dims (one load per source
// tensor) and writes them with stride BS into the block, converting to E4M3
// on the way when the pool is FP8 (multiplier 1/scale, fp8_gemm.cu:89-93).
//
// fp8 scale: per-tensor absmax(x)/448, the E4M3 scale convention of
// fp8_gemm.cu:82-84, as a grid-wide max.
//
// RoPE + reshape_and_cache: the write side of a step in one launch.  A
// thread owns 8 rotation pairs of one (token, head) of q, of k (rotated, then
// scattered into the pool) or of v (copied into the pool).  Pairs are
// (2i, 2i+1) for the ADJACENT style (ggml's LLAMA_ROPE_TYPE_NORM, the
// engine's rope, cuda_engine.cpp:1100-1108) and (i, i + d/2) for HALVES
// (rope_device.cuh:24-36); cos/sin come from the model's fp32 tables
// [max_pos, d/2] (cuda_model.cpp:269-295).  In fp32:
//   r0 = fmaf(a, c, -(b s)),  r1 = fmaf(a, s, b c),
// rounded once to the dtype.
//
// Block copies (copy_blocks, cache_kernels.cu:107-131, :234-262; swap_blocks,
// :133-167, :264-284): whole blocks between block ids of a mapping {src,
// dst}; a workgroup moves a slice of one block of one pool in 16-byte
// chunks (bytes when the block or a base is not 16-byte aligned).  Ids
// outside their pool skip the pair.
#include <type_traits>

#include "tl_device.hpp"
#include "tl_internal.hpp"

namespace tl {

namespace {

template <Kind SRC> __device__ __forceinline__ void load8(const void* p, int64_t i, float* f);
template <> __device__ __forceinline__ void load8<Kind::F16>(const void* p, int64_t i, float* f) {
  const u32x4 c = load16((const uint16_t*)p + i);
  Unpack<Kind::F16>::run(c.x, f); Unpack<Kind::F16>::run(c.y, f + 2);
  Unpack<Kind::F16>::run(c.z, f + 4); Unpack<Kind::F16>::run(c.w, f + 6);
}
template <> __device__ __forceinline__ void load8<Kind::BF16>(const void* p, int64_t i, float* f) {
  const u32x4 c = load16((const uint16_t*)p + i);
  Unpack<Kind::BF16>::run(c.x, f); Unpack<Kind::BF16>::run(c.y, f + 2);
  Unpack<Kind::BF16>::run(c.z, f + 4); Unpack<Kind::BF16>::run(c.w, f + 6);
}

// Same-type copy: move raw element bits (bit-exact, NaN payloads included).
template <int E>
__global__ __launch_bounds__(256) void reshape_copy_kernel(
    const char* __restrict__ key, const char* __restrict__ value, char* __restrict__ k_cache,
    char* __restrict__ v_cache, const int32_t* __restrict__ slots, int num_tokens,
    int num_kv_heads, int head_size, int block_size, int num_blocks) {
  constexpr int RUN = 16 / E;                       // elements per 16-byte run
  const int runs = head_size / RUN;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = (int64_t)num_tokens * num_kv_heads * runs;
  if (idx >= total) return;
  const int r = (int)(idx % runs);
  const int h = (int)((idx / runs) % num_kv_heads);
  const int t = (int)(idx / ((int64_t)runs * num_kv_heads));
  const int32_t slot = slots[t];
  if (slot < 0) return;
  const int blk = slot / block_size, off = slot % block_size;
  if (blk >= num_blocks) return;
  const int64_t src = ((int64_t)t * num_kv_heads + h) * head_size + (int64_t)r * RUN;
  const int64_t dst = (((int64_t)blk * num_kv_heads + h) * head_size + (int64_t)r * RUN) * block_size + off;
  const u32x4 kk = load16(key + src * E), vv = load16(value + src * E);
  const uint32_t kw[4] = {kk.x, kk.y, kk.z, kk.w}, vw[4] = {vv.x, vv.y, vv.z, vv.w};
#pragma unroll
  for (int i = 0; i < RUN; ++i) {
    const int64_t o = (dst + (int64_t)i * block_size) * E;
    if constexpr (E == 2) {
      const int wi = i / 2, sh = (i % 2) * 16;
      *(uint16_t*)(k_cache + o) = (uint16_t)(kw[wi] >> sh);
      *(uint16_t*)(v_cache + o) = (uint16_t)(vw[wi] >> sh);
    } else {
      *(uint32_t*)(k_cache + o) = kw[i];
      *(uint32_t*)(v_cache + o) = vw[i];
    }
  }
}

// Decode appends: few tokens, each in a block that no other token of the
// call writes.  HBM3E has no byte masks, so the element stores of
// reshape_copy_kernel (one token's D elements lie BS elements apart) leave
// partly written lines whose write-back is a read-modify-write of a memory
// burst each: 17 us for one token of each of 64 sequences (8 kv heads,
// d 128, bs 16).  Here a wavefront per (token, kv head) reads the block's
// row of that kv head (D x BS elements, 4 KiB for f16 at bs 16), replaces
// the token's slot and writes the row back whole.  The other slots are
// rewritten with their own bytes, so the block must have no other writer
// during the call (a block that a sequence appends to belongs to that
// sequence); a token whose block another token of this call also writes
// is stored element by element instead.
template <int E> struct Elem;
template <> struct Elem<2> { typedef uint16_t T; };
template <> struct Elem<4> { typedef uint32_t T; };

// Replace element e (PER = 16 / E per chunk) of a 16-byte chunk.
template <int E>
__device__ __forceinline__ void put_elem(u32x4& c, int e, uint32_t v) {
  constexpr int PER = 16 / E;
  const int w = e / (PER / 4);
  const uint32_t sh = E == 2 ? 16u * (e & 1) : 0u;
  const uint32_t keep = E == 2 ? ~(0xFFFFu << sh) : 0u, ins = (E == 2 ? (v & 0xFFFFu) : v) << sh;
  c.x = w == 0 ? (c.x & keep) | ins : c.x;
  c.y = w == 1 ? (c.y & keep) | ins : c.y;
  c.z = w == 2 ? (c.z & keep) | ins : c.z;
  c.w = w == 3 ? (c.w & keep) | ins : c.w;
}

template <int E>
__global__ __launch_bounds__(64) void reshape_rows_kernel(
    const char* __restrict__ key, const char* __restrict__ value, char* __restrict__ k_cache,
    char* __restrict__ v_cache, const int32_t* __restrict__ slots, int num_tokens,
    int num_kv_heads, int head_size, int block_size, int num_blocks) {
  using T = typename Elem<E>::T;
  constexpr int PER = 16 / E;                        // elements per 16-byte chunk
  const int t = blockIdx.x / num_kv_heads, h = blockIdx.x % num_kv_heads;
  const int lane = threadIdx.x;
  const int32_t slot = slots[t];
  if (slot < 0) return;
  const int blk = slot / block_size, off = slot % block_size;
  if (blk >= num_blocks) return;
  bool shared = false;
  for (int i = lane; i < num_tokens; i += kWave) {
    const int32_t s2 = slots[i];
    shared |= i != t && s2 >= 0 && s2 / block_size == blk;
  }
  const int64_t src = ((int64_t)t * num_kv_heads + h) * head_size;
  const int64_t row = ((int64_t)blk * num_kv_heads + h) * head_size * block_size;   // elements
  const T* ks = reinterpret_cast<const T*>(key) + src;
  const T* vs = reinterpret_cast<const T*>(value) + src;
  T* kr = reinterpret_cast<T*>(k_cache) + row;
  T* vr = reinterpret_cast<T*>(v_cache) + row;
  if (__builtin_amdgcn_ballot_w64(shared) != 0) {
    for (int c = lane; c < head_size; c += kWave) {
      kr[(int64_t)c * block_size + off] = ks[c];
      vr[(int64_t)c * block_size + off] = vs[c];
    }
    return;
  }
  const int cpc = block_size / PER;                  // chunks per channel
  const int chunks = head_size * cpc;
#pragma unroll 4
  for (int j = lane; j < chunks; j += kWave) {
    u32x4 kc = load16(kr + (int64_t)j * PER), vc = load16(vr + (int64_t)j * PER);
    const int c = j / cpc, e = off - (j % cpc) * PER;
    if (e >= 0 && e < PER) {
      put_elem<E>(kc, e, (uint32_t)ks[c]);
      put_elem<E>(vc, e, (uint32_t)vs[c]);
    }
    *reinterpret_cast<u32x4*>(kr + (int64_t)j * PER) = kc;
    *reinterpret_cast<u32x4*>(vr + (int64_t)j * PER) = vc;
  }
}

// The row kernel serves calls of at most this many tokens (each wavefront
// scans the call's slots for a shared block).
constexpr int kRowAppendMaxTokens = 256;

template <Kind SRC>
__global__ __launch_bounds__(256) void reshape_fp8_kernel(
    const void* __restrict__ key, const void* __restrict__ value, uint8_t* __restrict__ k_cache,
    uint8_t* __restrict__ v_cache, const int32_t* __restrict__ slots, int num_tokens,
    int num_kv_heads, int head_size, int block_size, int num_blocks, float k_mul, float v_mul) {
  const int runs = head_size / 8;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = (int64_t)num_tokens * num_kv_heads * runs;
  if (idx >= total) return;
  const int r = (int)(idx % runs);
  const int h = (int)((idx / runs) % num_kv_heads);
  const int t = (int)(idx / ((int64_t)runs * num_kv_heads));
  const int32_t slot = slots[t];
  if (slot < 0) return;
  const int blk = slot / block_size, off = slot % block_size;
  if (blk >= num_blocks) return;
  const int64_t src = ((int64_t)t * num_kv_heads + h) * head_size + (int64_t)r * 8;
  const int64_t dst = (((int64_t)blk * num_kv_heads + h) * head_size + (int64_t)r * 8) * block_size + off;
  float kf[8], vf[8];
  load8<SRC>(key, src, kf);
  load8<SRC>(value, src, vf);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    k_cache[dst + (int64_t)i * block_size] = f32_to_fp8(kf[i] * k_mul);
    v_cache[dst + (int64_t)i * block_size] = f32_to_fp8(vf[i] * v_mul);
  }
}

// convert_fp8 (cache_kernels.cu:181-193, :286-295): out[i] = e4m3(float(in[i])
// * scale), RNE with saturation to +-448 (NaN stays NaN).  VEC: 16 elements
// per thread with 16-byte loads and one 16-byte store (both buffers 16-byte
// aligned); otherwise element by element.
__device__ __forceinline__ float fp8_sat(float v) {
  const float c = __builtin_fminf(__builtin_fmaxf(v, -448.0f), 448.0f);
  return (v != v) ? v : c;
}
__device__ __forceinline__ uint32_t pack4_fp8(float a, float b, float c, float d) {
  uint32_t w = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(fp8_sat(a), fp8_sat(b), 0, false);
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(fp8_sat(c), fp8_sat(d), (int)w, true);
}
template <Kind SRC>
__device__ __forceinline__ float load_elem(const void* p, int64_t i) {
  if constexpr (SRC == Kind::F32) return reinterpret_cast<const float*>(p)[i];
  else if constexpr (SRC == Kind::BF16) return bf16_to_f32(reinterpret_cast<const uint16_t*>(p)[i]);
  else return f16_to_f32(reinterpret_cast<const uint16_t*>(p)[i]);
}
template <Kind SRC, bool VEC>
__global__ __launch_bounds__(256) void convert_fp8_kernel(const void* __restrict__ in, uint8_t* __restrict__ out,
                                                          int64_t n, float scale) {
  const int64_t i0 = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 16;
  if (i0 >= n) return;
  if (VEC && i0 + 16 <= n) {
    float f[16];
    if constexpr (SRC == Kind::F32) {
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const u32x4 v = load16(reinterpret_cast<const float*>(in) + i0 + 4 * c);
        f[4 * c] = __builtin_bit_cast(float, v.x); f[4 * c + 1] = __builtin_bit_cast(float, v.y);
        f[4 * c + 2] = __builtin_bit_cast(float, v.z); f[4 * c + 3] = __builtin_bit_cast(float, v.w);
      }
    } else {
      load8<SRC>(in, i0, f);
      load8<SRC>(in, i0 + 8, f + 8);
    }
    u32x4 o;
    o.x = pack4_fp8(f[0] * scale, f[1] * scale, f[2] * scale, f[3] * scale);
    o.y = pack4_fp8(f[4] * scale, f[5] * scale, f[6] * scale, f[7] * scale);
    o.z = pack4_fp8(f[8] * scale, f[9] * scale, f[10] * scale, f[11] * scale);
    o.w = pack4_fp8(f[12] * scale, f[13] * scale, f[14] * scale, f[15] * scale);
    *reinterpret_cast<u32x4*>(out + i0) = o;
    return;
  }
  const int64_t i1 = i0 + 16 < n ? i0 + 16 : n;
  for (int64_t i = i0; i < i1; ++i) out[i] = f32_to_fp8(load_elem<SRC>(in, i) * scale);
}

// Element j of pair i within one head row: ADJACENT (2i + j), HALVES (i + j d/2).
template <int STYLE>
__device__ __forceinline__ int rope_dim(int i, int j, int half) {
  return STYLE == 0 ? 2 * i + j : i + j * half;
}

template <Kind K, int STYLE>
__global__ __launch_bounds__(256) void rope_cache_kernel(RopeCache a) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int half = a.head_size / 2, units = half / 8;           // 8 pairs per thread
  // q heads, k heads, v heads (with k_out: q and k heads, written as rows)
  const int rows = a.num_heads + (a.q_only ? 0 : (a.k_out ? 1 : 2) * a.num_kv_heads);
  const int64_t total = (int64_t)a.num_tokens * rows * units;
  if (idx >= total) return;
  const int u = (int)(idx % units);
  const int row = (int)((idx / units) % rows);
  const int t = (int)(idx / ((int64_t)units * rows));
  const int pos = a.positions[t];
  // a position outside the tables leaves the token as it is (with k_out:
  // copied unrotated)
  const bool rot = pos >= 0 && pos < a.max_positions;
  if (!rot && !a.k_out) return;
  const int i0 = 8 * u;
  float x[16];
  const void* src;
  int64_t base;
  if (row < a.num_heads) {
    src = a.q;
    base = ((int64_t)t * a.num_heads + row) * a.head_size;
  } else if (row < a.num_heads + a.num_kv_heads) {
    src = a.key;
    base = ((int64_t)t * a.num_kv_heads + (row - a.num_heads)) * a.head_size;
  } else {
    src = a.value;
    base = ((int64_t)t * a.num_kv_heads + (row - a.num_heads - a.num_kv_heads)) * a.head_size;
  }
#pragma unroll
  for (int p = 0; p < 8; ++p) {
    x[2 * p] = load_scalar<K>(src, base + rope_dim<STYLE>(i0 + p, 0, half));
    x[2 * p + 1] = load_scalar<K>(src, base + rope_dim<STYLE>(i0 + p, 1, half));
  }
  const bool is_v = row >= a.num_heads + a.num_kv_heads;
  if (!is_v && rot) {
    const float* cs = a.cos_table + (int64_t)pos * half + i0;
    const float* sn = a.sin_table + (int64_t)pos * half + i0;
#pragma unroll
    for (int p = 0; p < 8; ++p) {
      const float c = cs[p], sv = sn[p], x0 = x[2 * p], x1 = x[2 * p + 1];
      x[2 * p] = __builtin_fmaf(x0, c, -(x1 * sv));
      x[2 * p + 1] = __builtin_fmaf(x0, sv, x1 * c);
    }
  }
  if (row < a.num_heads || a.k_out) {
    void* dst = row < a.num_heads ? a.q_out : a.k_out;
#pragma unroll
    for (int p = 0; p < 8; ++p) {
      store_scalar<K>(dst, base + rope_dim<STYLE>(i0 + p, 0, half), x[2 * p]);
      store_scalar<K>(dst, base + rope_dim<STYLE>(i0 + p, 1, half), x[2 * p + 1]);
    }
    return;
  }
  const int32_t slot = a.slot_mapping[t];
  if (slot < 0) return;
  const int blk = slot / a.block_size, off = slot % a.block_size;
  if (blk >= a.num_blocks) return;
  const int h = is_v ? row - a.num_heads - a.num_kv_heads : row - a.num_heads;
  void* pool = is_v ? a.v_cache : a.k_cache;
  const int64_t pbase = ((int64_t)blk * a.num_kv_heads + h) * a.head_size;
#pragma unroll
  for (int p = 0; p < 8; ++p)
#pragma unroll
    for (int j = 0; j < 2; ++j)
      store_scalar<K>(pool, (pbase + rope_dim<STYLE>(i0 + p, j, half)) * a.block_size + off, x[2 * p + j]);
}

// An fp32 result as computed, before its conversion to a 2-byte type: the
// compiler would otherwise fuse the last fma with the conversion
// (v_fma_mix*, one rounding), where rope_cache_kernel and the reference
// round to fp32 first.
__device__ __forceinline__ float fp32_result(float r) {
  asm volatile("" : "+v"(r));
  return r;
}

// The element's bits in the pool's type (the rounding of store_scalar).
template <Kind K> __device__ __forceinline__ uint32_t scalar_bits(float v);
template <> __device__ __forceinline__ uint32_t scalar_bits<Kind::F32>(float v) { return __float_as_uint(v); }
template <> __device__ __forceinline__ uint32_t scalar_bits<Kind::F16>(float v) { return f32_to_f16(v); }
template <> __device__ __forceinline__ uint32_t scalar_bits<Kind::BF16>(float v) { return f32_to_bf16(v); }

// The RoPE append for decode-sized calls (at most kRowAppendMaxTokens
// tokens, 16-byte aligned pools, num_heads a multiple of num_kv_heads), in
// one launch: a wavefront per (token, kv head) rotates the q heads
// h G .. h G + G - 1 (G = num_heads / num_kv_heads) and writes k and v as
// reshape_rows_kernel does: the block's K and V rows rewritten whole, with
// the rotated key and the value in the token's slot, when no other token
// of the call writes the block, element by element otherwise.  The
// rotation is that of rope_cache_kernel.
template <Kind K, int STYLE>
__global__ __launch_bounds__(64) void rope_rows_kernel(RopeCache a) {
  constexpr int E = KindInfo<K>::bytes, PER = 16 / E;
  const int t = blockIdx.x / a.num_kv_heads, h = blockIdx.x % a.num_kv_heads;
  const int lane = threadIdx.x;
  const int pos = a.positions[t];
  if (pos < 0 || pos >= a.max_positions) return;               // token left as it is
  {
    const int G = a.num_heads / a.num_kv_heads, hh = a.head_size / 2;
    const float* cq = a.cos_table + (int64_t)pos * hh;
    const float* sq = a.sin_table + (int64_t)pos * hh;
    for (int hq = h * G; hq < h * G + G; ++hq) {
      const int64_t qb = ((int64_t)t * a.num_heads + hq) * a.head_size;
      for (int i = lane; i < hh; i += kWave) {
        const float x0 = load_scalar<K>(a.q, qb + rope_dim<STYLE>(i, 0, hh));
        const float x1 = load_scalar<K>(a.q, qb + rope_dim<STYLE>(i, 1, hh));
        const float c0 = cq[i], s0 = sq[i];
        store_scalar<K>(a.q_out, qb + rope_dim<STYLE>(i, 0, hh), fp32_result(__builtin_fmaf(x0, c0, -(x1 * s0))));
        store_scalar<K>(a.q_out, qb + rope_dim<STYLE>(i, 1, hh), fp32_result(__builtin_fmaf(x0, s0, x1 * c0)));
      }
    }
  }
  const int32_t slot = a.slot_mapping[t];
  if (slot < 0) return;
  const int blk = slot / a.block_size, off = slot % a.block_size;
  if (blk >= a.num_blocks) return;
  bool shared = false;
  for (int i = lane; i < a.num_tokens; i += kWave) {
    const int32_t s2 = a.slot_mapping[i];
    const int p2 = a.positions[i];
    shared |= i != t && s2 >= 0 && s2 / a.block_size == blk && p2 >= 0 && p2 < a.max_positions;
  }
  const int half = a.head_size / 2;
  const int64_t src = ((int64_t)t * a.num_kv_heads + h) * a.head_size;
  const float* cs = a.cos_table + (int64_t)pos * half;
  const float* sn = a.sin_table + (int64_t)pos * half;
  // channel c of the rotated key
  auto rot = [&](int c) {
    const int i = STYLE == 0 ? c / 2 : c % half, r = STYLE == 0 ? c % 2 : c / half;
    const float x0 = load_scalar<K>(a.key, src + rope_dim<STYLE>(i, 0, half));
    const float x1 = load_scalar<K>(a.key, src + rope_dim<STYLE>(i, 1, half));
    const float c0 = cs[i], s0 = sn[i];
    return fp32_result(r == 0 ? __builtin_fmaf(x0, c0, -(x1 * s0)) : __builtin_fmaf(x0, s0, x1 * c0));
  };
  const int64_t row = ((int64_t)blk * a.num_kv_heads + h) * a.head_size * a.block_size;   // elements
  char* kr = (char*)a.k_cache + row * E;
  char* vr = (char*)a.v_cache + row * E;
  if (__builtin_amdgcn_ballot_w64(shared) != 0) {
    for (int c = lane; c < a.head_size; c += kWave) {
      store_scalar<K>(kr, (int64_t)c * a.block_size + off, rot(c));
      store_scalar<K>(vr, (int64_t)c * a.block_size + off, load_scalar<K>(a.value, src + c));
    }
    return;
  }
  const int cpc = a.block_size / PER;                  // chunks per channel
  const int chunks = a.head_size * cpc;
  for (int j = lane; j < chunks; j += kWave) {
    u32x4 kc = load16(kr + (int64_t)j * 16), vc = load16(vr + (int64_t)j * 16);
    const int c = j / cpc, e = off - (j % cpc) * PER;
    if (e >= 0 && e < PER) {
      put_elem<E>(kc, e, scalar_bits<K>(rot(c)));
      put_elem<E>(vc, e, scalar_bits<K>(load_scalar<K>(a.value, src + c)));
    }
    *reinterpret_cast<u32x4*>(kr + (int64_t)j * 16) = kc;
    *reinterpret_cast<u32x4*>(vr + (int64_t)j * 16) = vc;
  }
}

// grid.x = pairs x pools x slices; pool 1 is the second (V) pool of a copy.
template <bool VEC>
__global__ __launch_bounds__(256) void block_copy_kernel(BlockCopy c) {
  int64_t b = blockIdx.x;
  const int slice = (int)(b % c.slices); b /= c.slices;
  const int pool = (int)(b % c.pools);
  const int pair = (int)(b / c.pools);
  const int32_t src = c.mapping[2 * pair], dst = c.mapping[2 * pair + 1];
  if (src < 0 || src >= c.src_blocks || dst < 0 || dst >= c.dst_blocks) return;
  const char* from = (pool ? c.src1 : c.src0) + (int64_t)src * c.block_bytes;
  char* to = (pool ? c.dst1 : c.dst0) + (int64_t)dst * c.block_bytes;
  const int64_t n = VEC ? c.block_bytes / 16 : c.block_bytes;
  const int64_t step = (int64_t)c.slices * blockDim.x;
  for (int64_t i = (int64_t)slice * blockDim.x + threadIdx.x; i < n; i += step) {
    if constexpr (VEC)
      reinterpret_cast<u32x4*>(to)[i] = reinterpret_cast<const u32x4*>(from)[i];
    else
      to[i] = from[i];
  }
}

__global__ void fill_u32_kernel(uint32_t* p, uint32_t v) { *p = v; }

template <Kind SRC>
__global__ __launch_bounds__(256) void absmax_kernel(const void* __restrict__ x, int64_t n,
                                                     uint32_t* __restrict__ out_bits) {
  float m = 0.f;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    m = fmaxf(m, fabsf(load_scalar<SRC>(x, i)));
  m = wave_max<32, 1>(m);
  if ((threadIdx.x % kWave) == 0) atomicMax(out_bits, __builtin_bit_cast(uint32_t, m));
}

__global__ void scale_finish_kernel(uint32_t* bits) {
  const float amax = __builtin_bit_cast(float, *bits);
  *reinterpret_cast<float*>(bits) = amax / 448.0f;
}

}  // namespace

int launch_reshape_and_cache(const CacheLaunch& a) {
  const int64_t runs_per_tok = (int64_t)a.num_kv_heads * (a.head_size / 8);
  if (a.num_tokens == 0) return 0;
  if (a.cache_dtype == (int)Kind::FP8) {
    const int64_t total = (int64_t)a.num_tokens * runs_per_tok;
    const dim3 grid((unsigned)((total + 255) / 256));
    const float km = 1.0f / (a.k_scale == 0.f ? 1.f : a.k_scale);
    const float vm = 1.0f / (a.v_scale == 0.f ? 1.f : a.v_scale);
    if (a.src_dtype == (int)Kind::F16)
      hipLaunchKernelGGL(reshape_fp8_kernel<Kind::F16>, grid, dim3(256), 0, a.stream, a.key,
                         a.value, (uint8_t*)a.k_cache, (uint8_t*)a.v_cache, a.slot_mapping,
                         a.num_tokens, a.num_kv_heads, a.head_size, a.block_size, a.num_blocks, km, vm);
    else if (a.src_dtype == (int)Kind::BF16)
      hipLaunchKernelGGL(reshape_fp8_kernel<Kind::BF16>, grid, dim3(256), 0, a.stream, a.key,
                         a.value, (uint8_t*)a.k_cache, (uint8_t*)a.v_cache, a.slot_mapping,
                         a.num_tokens, a.num_kv_heads, a.head_size, a.block_size, a.num_blocks, km, vm);
    else
      return 3;
  } else {
    const int E = (a.cache_dtype == (int)Kind::F32) ? 4 : 2;
    const int64_t total = (int64_t)a.num_tokens * a.num_kv_heads * (a.head_size / (16 / E));
    const dim3 grid((unsigned)((total + 255) / 256));
    const bool aligned = (((uintptr_t)a.k_cache | (uintptr_t)a.v_cache) % 16) == 0;
    if (a.num_tokens <= kRowAppendMaxTokens && (a.block_size * E) % 16 == 0 && aligned) {
      const dim3 rgrid((unsigned)(a.num_tokens * a.num_kv_heads));
      if (E == 2)
        hipLaunchKernelGGL(reshape_rows_kernel<2>, rgrid, dim3(kWave), 0, a.stream,
                           (const char*)a.key, (const char*)a.value, (char*)a.k_cache,
                           (char*)a.v_cache, a.slot_mapping, a.num_tokens, a.num_kv_heads,
                           a.head_size, a.block_size, a.num_blocks);
      else
        hipLaunchKernelGGL(reshape_rows_kernel<4>, rgrid, dim3(kWave), 0, a.stream,
                           (const char*)a.key, (const char*)a.value, (char*)a.k_cache,
                           (char*)a.v_cache, a.slot_mapping, a.num_tokens, a.num_kv_heads,
                           a.head_size, a.block_size, a.num_blocks);
    } else if (E == 2)
      hipLaunchKernelGGL(reshape_copy_kernel<2>, grid, dim3(256), 0, a.stream,
                         (const char*)a.key, (const char*)a.value, (char*)a.k_cache,
                         (char*)a.v_cache, a.slot_mapping, a.num_tokens, a.num_kv_heads,
                         a.head_size, a.block_size, a.num_blocks);
    else
      hipLaunchKernelGGL(reshape_copy_kernel<4>, grid, dim3(256), 0, a.stream,
                         (const char*)a.key, (const char*)a.value, (char*)a.k_cache,
                         (char*)a.v_cache, a.slot_mapping, a.num_tokens, a.num_kv_heads,
                         a.head_size, a.block_size, a.num_blocks);
  }
  return hipGetLastError() == hipSuccess ? 0 : 5;
}

int launch_rope_cache(const RopeCache& a_in, hipStream_t stream) {
  if (a_in.num_tokens == 0) return 0;
  RopeCache a = a_in;
  a.q_only = 0;
  const Kind k = (Kind)a.dtype;
  const int E = k == Kind::F32 ? 4 : 2;
  const bool aligned = (((uintptr_t)a.k_cache | (uintptr_t)a.v_cache) % 16) == 0;
  // decode-sized calls: one wavefront per (token, kv head), whole block rows
  const bool rows = a.num_tokens <= kRowAppendMaxTokens && (a.block_size * E) % 16 == 0 && aligned &&
                    a.num_heads % a.num_kv_heads == 0;
  const int64_t total = (int64_t)a.num_tokens * (a.num_heads + 2 * a.num_kv_heads) * (a.head_size / 16);
  const dim3 grid((unsigned)((total + 255) / 256));
  const dim3 rgrid((unsigned)(a.num_tokens * a.num_kv_heads));
#define TL_ROPE_LAUNCH(K, S)                                                                    \
  do {                                                                                          \
    if (rows) hipLaunchKernelGGL((rope_rows_kernel<K, S>), rgrid, dim3(kWave), 0, stream, a);  \
    else hipLaunchKernelGGL((rope_cache_kernel<K, S>), grid, dim3(256), 0, stream, a);         \
  } while (0)
  if (k == Kind::F16) { if (a.style) TL_ROPE_LAUNCH(Kind::F16, 1); else TL_ROPE_LAUNCH(Kind::F16, 0); }
  else if (k == Kind::BF16) { if (a.style) TL_ROPE_LAUNCH(Kind::BF16, 1); else TL_ROPE_LAUNCH(Kind::BF16, 0); }
  else if (k == Kind::F32) { if (a.style) TL_ROPE_LAUNCH(Kind::F32, 1); else TL_ROPE_LAUNCH(Kind::F32, 0); }
  else return 3;
#undef TL_ROPE_LAUNCH
  return hipGetLastError() == hipSuccess ? 0 : 5;
}

int launch_rope_rows(const RopeCache& a_in, hipStream_t stream) {
  if (a_in.num_tokens == 0) return 0;
  RopeCache a = a_in;
  a.q_only = 0;
  if (!a.k_out) return 3;
  const int64_t total = (int64_t)a.num_tokens * (a.num_heads + a.num_kv_heads) * (a.head_size / 16);
  const dim3 grid((unsigned)((total + 255) / 256));
#define TL_ROPE_ROWS(K, S) hipLaunchKernelGGL((rope_cache_kernel<K, S>), grid, dim3(256), 0, stream, a)
  const Kind k = (Kind)a.dtype;
  if (k == Kind::F16) { if (a.style) TL_ROPE_ROWS(Kind::F16, 1); else TL_ROPE_ROWS(Kind::F16, 0); }
  else if (k == Kind::BF16) { if (a.style) TL_ROPE_ROWS(Kind::BF16, 1); else TL_ROPE_ROWS(Kind::BF16, 0); }
  else if (k == Kind::F32) { if (a.style) TL_ROPE_ROWS(Kind::F32, 1); else TL_ROPE_ROWS(Kind::F32, 0); }
  else return 3;
#undef TL_ROPE_ROWS
  return hipGetLastError() == hipSuccess ? 0 : 5;
}

int launch_block_copy(const BlockCopy& c, hipStream_t stream) {
  if (c.num_pairs <= 0) return 0;
  const auto al = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
  const bool vec = c.block_bytes % 16 == 0 && al(c.src0) && al(c.dst0) &&
                   (c.pools == 1 || (al(c.src1) && al(c.dst1)));
  BlockCopy k = c;
  // up to 16 workgroups of 256 x 16 bytes per block: a 32 KiB block is 8
  const int64_t units = vec ? c.block_bytes / 16 : c.block_bytes;
  const int64_t want = (units + 255) / 256;
  k.slices = (int)(want < 16 ? (want > 0 ? want : 1) : 16);
  const int64_t grid = (int64_t)c.num_pairs * c.pools * k.slices;
  if (grid > 0x7fffffff) return 3;
  if (vec)
    hipLaunchKernelGGL(block_copy_kernel<true>, dim3((unsigned)grid), dim3(256), 0, stream, k);
  else
    hipLaunchKernelGGL(block_copy_kernel<false>, dim3((unsigned)grid), dim3(256), 0, stream, k);
  return hipGetLastError() == hipSuccess ? 0 : 5;
}

int launch_convert_fp8(uint8_t* out, const void* in, int dtype, int64_t n, float scale, hipStream_t stream) {
  if (n <= 0) return 0;
  const dim3 grid((unsigned)((n + 16 * 256 - 1) / (16 * 256)));
  const bool vec = (((uintptr_t)out | (uintptr_t)in) % 16) == 0;
  auto go = [&](auto tag) {
    constexpr Kind K = decltype(tag)::value;
    if (vec)
      hipLaunchKernelGGL((convert_fp8_kernel<K, true>), grid, dim3(256), 0, stream, in, out, n, scale);
    else
      hipLaunchKernelGGL((convert_fp8_kernel<K, false>), grid, dim3(256), 0, stream, in, out, n, scale);
  };
  if (dtype == (int)Kind::F16) go(std::integral_constant<Kind, Kind::F16>());
  else if (dtype == (int)Kind::BF16) go(std::integral_constant<Kind, Kind::BF16>());
  else if (dtype == (int)Kind::F32) go(std::integral_constant<Kind, Kind::F32>());
  else return 3;
  return hipGetLastError() == hipSuccess ? 0 : 5;
}

int launch_fp8_scale(const void* x, int dtype, int64_t n, float* scale_out, hipStream_t stream) {
  uint32_t* bits = reinterpret_cast<uint32_t*>(scale_out);
  hipLaunchKernelGGL(fill_u32_kernel, dim3(1), dim3(1), 0, stream, bits, 0u);
  if (n > 0) {
    const int64_t want = (n + 255) / 256;
    const dim3 grid((unsigned)(want < 4096 ? want : 4096));
    if (dtype == (int)Kind::F16)
      hipLaunchKernelGGL(absmax_kernel<Kind::F16>, grid, dim3(256), 0, stream, x, n, bits);
    else if (dtype == (int)Kind::BF16)
      hipLaunchKernelGGL(absmax_kernel<Kind::BF16>, grid, dim3(256), 0, stream, x, n, bits);
    else if (dtype == (int)Kind::F32)
      hipLaunchKernelGGL(absmax_kernel<Kind::F32>, grid, dim3(256), 0, stream, x, n, bits);
    else
      return 3;
  }
  hipLaunchKernelGGL(scale_finish_kernel, dim3(1), dim3(1), 0, stream, bits);
  return hipGetLastError() == hipSuccess ? 0 : 5;
}

}  // namespace tl
