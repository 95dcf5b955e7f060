// tl_kivi_page.hpp -- the KIVI group quantiser and the page builder, shared
// by the page kernels (prefix build, append) and the fused append of the
// KIVI decode step.
//
// Group quantiser (kivi_cache.cu:92-124): min/max over the group,
// scale = 15 / range (0 when range <= 1e-6), nibble = clamp(rint((x - min)
// * scale), 0, 15), fp16 step = 1/scale, fp16 zero = min.  A page (32
// tokens of one kv head) quantises K per channel over its 32 tokens and V
// per token over groups of 32 channels, then lays the nibbles out as in
// tl_kivi.hpp.
#pragma once

#include "tl_device.hpp"
#include "tl_internal.hpp"
#include "tl_kivi.hpp"

#include <float.h>

namespace tl {

// __float2int_rn then the clamp to [0, 15] of kivi_cache.cu:109-112 (to
// [0, 255] for 8-bit codes).
template <int LEVELS = 15>
__device__ __forceinline__ int quant_nibble(float v) {
  const float r = __builtin_rintf(v);
  if (!(r >= 0.0f)) return 0;  // negative or NaN
  if (r > (float)LEVELS) return LEVELS;
  return (int)r;
}

// min/max scan of kivi_cache.cu:97-104; returns degenerate flag and scale.
struct GroupQ {
  float gmin, scale;
  uint16_t step, zero;
};

template <int LEVELS = 15>
__device__ __forceinline__ GroupQ group_params(float gmin, float gmax) {
  GroupQ g;
  const float range = gmax - gmin;
  const bool degenerate = !(range > 1e-6f);
  g.gmin = gmin;
  g.scale = degenerate ? 0.0f : ((float)LEVELS / range);
  const float st = degenerate ? 0.0f : (1.0f / g.scale);
  const bool gmin_ok = (gmin == gmin) && (gmin > -FLT_MAX) && (gmin < FLT_MAX);
  g.step = f32_to_f16(st);
  g.zero = f32_to_f16(gmin_ok ? gmin : 0.0f);
  return g;
}

template <int LEVELS = 15>
__device__ __forceinline__ int quantise(float x, const GroupQ& g) {
  const float d = x - g.gmin;
  return quant_nibble<LEVELS>(d * g.scale);
}

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
  int bits;                 // code width of the pages: 4 or 8
  const uint16_t* knew;     // append: new token per sequence [S, n_kv, 128]
  const uint16_t* vnew;
  const int32_t* slots;     // append: its slot in the fp16 pool
};

// The kernels' view of a page launch (host side).
inline PageJob make_page_job(const KiviPageLaunch& a) {
  PageJob j;
  j.k_cache = (uint16_t*)a.k_cache; j.v_cache = (uint16_t*)a.v_cache;
  j.block_tables = a.block_tables; j.seq_lens = a.seq_lens; j.page_tables = a.page_tables;
  j.pages = (uint8_t*)a.pages;
  j.num_kv_heads = a.num_kv_heads; j.block_size = a.block_size;
  j.max_blocks_per_seq = a.max_blocks_per_seq; j.num_blocks = a.num_blocks;
  j.max_pages_per_seq = a.max_pages_per_seq; j.num_pages = a.num_pages;
  j.residual_length = a.residual_length;
  j.append = a.append;
  j.bits = a.bits;
  j.knew = (const uint16_t*)a.knew; j.vnew = (const uint16_t*)a.vnew; j.slots = a.slots;
  j.pages_per_seq_grid = a.append ? 1 : (a.max_pages_to_build > 0 ? a.max_pages_to_build : 1);
  return j;
}

// LDS of one page build (30 KiB for INT4 pages, 34 KiB for INT8).
template <int BITS>
struct KiviBuildSmem {
  uint16_t k[kKiviHead][kKiviPageTokens + 2];   // [channel][token] (+2 breaks bank conflicts)
  uint16_t v[kKiviPageTokens][kKiviHead + 2];   // [token][channel]
  uint8_t qk[kKiviHead][kKiviPageTokens];       // K codes [channel][token]
  uint8_t qv[kKiviPageTokens][kKiviHead];       // V codes [token][channel]
  __attribute__((aligned(16))) uint8_t page[KiviFmt<BITS>::kBytes];
};

// The new token (position L - 1) of (seq, kvh) into the fp16 pool, by NT
// threads.  In the pool a token's 128 channels are 2-byte elements 2 BS
// bytes apart; HBM3E has no byte masks, so 256 such scattered writes per
// (seq, kv head) cost a read-modify-write of a memory burst each.  Instead
// the block's rows of this kv head (128 channels x 16 slots: 4 KiB each of
// K and V) are read, the slot is replaced, and the rows are written back
// whole.  Other slots keep their bytes; the block of the slot belongs to the
// sequence alone (as every block that a sequence appends to does), so no
// other writer of the same launch touches these rows except the other head
// slices of the same (seq, kv head), which write the same bytes.
// A 2-byte store written through L2 (relaxed, agent scope: sc1).  In the
// pool a token's 128 channels are 2 BS bytes apart, so one token dirties 32
// L2 lines each of K and V; left dirty, a decode step's 512 (seq, kv head)
// tokens cost the next launch about 4 us of write-back at batch 64 (about
// 1.4 us when written through).
__device__ __forceinline__ void store_through(uint16_t* p, uint16_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The new token (position L - 1) of (seq, kvh) into the fp16 pool, the 128
// channels strided over NT threads; a negative slot writes nothing.
template <int NT>
__device__ __forceinline__ void kivi_append_token(const PageJob& j, int seq, int kvh, int tid) {
  const int32_t slot = j.slots[seq];
  const int blk = slot >= 0 ? slot / j.block_size : -1;
  if (blk < 0 || blk >= j.num_blocks) return;
  const int64_t new_off = ((int64_t)seq * j.num_kv_heads + kvh) * kKiviHead;
  const int64_t base = ((int64_t)blk * j.num_kv_heads + kvh) * kKiviHead * j.block_size + slot % j.block_size;
#pragma unroll
  for (int c = tid; c < kKiviHead; c += NT) {
    store_through(j.k_cache + base + (int64_t)c * j.block_size, j.knew[new_off + c]);
    store_through(j.v_cache + base + (int64_t)c * j.block_size, j.vnew[new_off + c]);
  }
}

// Orders the LDS accesses of the NT threads of a page build: a workgroup
// barrier, or, when one wavefront builds, a wavefront barrier.
template <int NT>
__device__ __forceinline__ void build_barrier() {
  if constexpr (NT == kWave) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  } else {
    __syncthreads();
  }
}

// The group quantiser over unit u of a page: u < 128 is K channel u (its 32
// tokens in order), u >= 128 is V (token, group of 32 channels) u - 128
// (channels in order).  Codes go to qk / qv, step and zero to the page.
template <int BITS>
__device__ __forceinline__ void quantise_unit(KiviBuildSmem<BITS>& sm, int u) {
  using F = KiviFmt<BITS>;
  constexpr int T = kKiviPageTokens, D = kKiviHead, LV = F::kLevels;
  if (u < D) {
    const int c = u;
    float gmin = FLT_MAX, gmax = -FLT_MAX;
    for (int t = 0; t < T; ++t) {
      const float x = f16_to_f32(sm.k[c][t]);
      if (x < gmin) gmin = x;
      if (x > gmax) gmax = x;
    }
    const GroupQ q = group_params<LV>(gmin, gmax);
    for (int t = 0; t < T; ++t) sm.qk[c][t] = (uint8_t)quantise<LV>(f16_to_f32(sm.k[c][t]), q);
    uint16_t* kp = reinterpret_cast<uint16_t*>(sm.page + F::kKParams + (c / 8) * 32);
    kp[c % 8] = q.step;
    kp[8 + c % 8] = q.zero;
  } else {
    const int t = (u - D) / 4, g = (u - D) % 4;
    float gmin = FLT_MAX, gmax = -FLT_MAX;
    for (int i = 0; i < 32; ++i) {
      const float x = f16_to_f32(sm.v[t][g * 32 + i]);
      if (x < gmin) gmin = x;
      if (x > gmax) gmax = x;
    }
    const GroupQ q = group_params<LV>(gmin, gmax);
    for (int i = 0; i < 32; ++i) sm.qv[t][g * 32 + i] = (uint8_t)quantise<LV>(f16_to_f32(sm.v[t][g * 32 + i]), q);
    const int r = kivi_v_group(t), s = kivi_v_slot(t);
    uint16_t* vp = reinterpret_cast<uint16_t*>(sm.page + F::kVParams + (g * 4 + r) * 32);
    vp[s] = q.step;
    vp[8 + s] = q.zero;
  }
}

// Quantise page `page` of (seq, kvh) from the fp16 pool and write it to its
// slot of the page pool.  Called by NT threads (a multiple of the
// wavefront: all of a workgroup's, or one wavefront's), which it
// synchronises; the caller synchronises them again before it reuses the
// LDS.  With j.append the token at position L - 1 is taken from the input
// row.
template <int NT, int BITS>
__device__ void kivi_build_page(KiviBuildSmem<BITS>& sm, const PageJob& j, int seq, int kvh, int page, int L,
                                int tid) {
  static_assert(NT % kWave == 0, "whole wavefronts");
  using F = KiviFmt<BITS>;
  constexpr int T = kKiviPageTokens, D = kKiviHead;
  if (page >= j.max_pages_per_seq) return;
  const int pid = j.page_tables[(int64_t)seq * j.max_pages_per_seq + page];
  if (pid < 0 || pid >= j.num_pages) return;
  const int64_t new_off = ((int64_t)seq * j.num_kv_heads + kvh) * D;

  // gather the 32 tokens: element (token t, channel c) of the fp16 pool; the
  // token at L - 1 of an append comes from the input row (it may still be in
  // flight to the pool)
  const int32_t* btab = j.block_tables + (int64_t)seq * j.max_blocks_per_seq;
  auto phys_of = [&](int tok) {
    const int lb = tok / j.block_size;
    const int phys = (lb < j.max_blocks_per_seq) ? btab[lb] : -1;
    return (phys < 0 || phys >= j.num_blocks) ? -1 : phys;
  };
  if (j.block_size % 8 == 0) {
    // 16-byte runs: 8 tokens of one channel are contiguous in one block;
    // the loads of all of a thread's runs are issued before the LDS stores
    constexpr int RUNS = D * T / 8, PER = (RUNS + NT - 1) / NT;
    u32x4 kr[PER], vr[PER];
#pragma unroll
    for (int r = 0; r < PER; ++r) {
      const int i = tid + r * NT;
      const int c = i / (T / 8), tok = page * T + (i % (T / 8)) * 8;
      const int phys = i < RUNS ? phys_of(tok) : -1;
      kr[r] = vr[r] = u32x4{0u, 0u, 0u, 0u};
      if (phys >= 0) {
        const int64_t off = (((int64_t)phys * j.num_kv_heads + kvh) * D + c) * j.block_size + tok % j.block_size;
        kr[r] = load16(j.k_cache + off);
        vr[r] = load16(j.v_cache + off);
      }
    }
#pragma unroll
    for (int r = 0; r < PER; ++r) {
      const int i = tid + r * NT;
      if (i >= RUNS) break;
      const int c = i / (T / 8), t0 = (i % (T / 8)) * 8;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        uint16_t kv = (uint16_t)(word(kr[r], e / 2) >> (16 * (e & 1)));
        uint16_t vv = (uint16_t)(word(vr[r], e / 2) >> (16 * (e & 1)));
        if (j.append && page * T + t0 + e == L - 1) {
          kv = j.knew[new_off + c];
          vv = j.vnew[new_off + c];
        }
        sm.k[c][t0 + e] = kv;
        sm.v[t0 + e][c] = vv;
      }
    }
  } else {
    for (int i = tid; i < T * D; i += NT) {
      const int c = i / T, t = i % T;
      const int tok = page * T + t;
      const int phys = phys_of(tok);
      uint16_t kv = 0, vv = 0;
      if (j.append && tok == L - 1) {
        kv = j.knew[new_off + c];
        vv = j.vnew[new_off + c];
      } else if (phys >= 0) {
        const int64_t off = (((int64_t)phys * j.num_kv_heads + kvh) * D + c) * j.block_size + tok % j.block_size;
        kv = j.k_cache[off];
        vv = j.v_cache[off];
      }
      sm.k[c][t] = kv;
      sm.v[t][c] = vv;
    }
  }
  build_barrier<NT>();

  for (int u = tid; u < 2 * D; u += NT) quantise_unit<BITS>(sm, u);
  build_barrier<NT>();

  uint32_t* pw = reinterpret_cast<uint32_t*>(sm.page);
  if constexpr (BITS == 8) {
    // code dwords: 1024 for K then 1024 for V; byte k of dword 2m + h holds
    // element 4h + {0, 2, 1, 3}[k] of its octet (K) or slot run (V)
    for (int w = tid; w < 1024; w += NT) {
      const int c = w / 8, dd = w % 8, m = dd / 2, h = dd % 2;
      // K: chunk c = tt*64 + jj*16 + u holds token tt*16 + u, octet jj + 4m
      const int t = (c / 64) * 16 + c % 16, o = (c % 64) / 16 + 4 * m;
      const int kc = 8 * o + 4 * h;
      pw[w] = (uint32_t)sm.qk[kc][t] | (uint32_t)sm.qk[kc + 2][t] << 8 | (uint32_t)sm.qk[kc + 1][t] << 16 |
              (uint32_t)sm.qk[kc + 3][t] << 24;
      // V: chunk c = hh*64 + r*16 + u, channel (4 hh + m)*16 + u, slots 4h ..
      const int hh = c / 64, r = (c % 64) / 16, u = c % 16;
      const int d = (4 * hh + m) * 16 + u;
      pw[F::kVCodes / 4 + w] = (uint32_t)sm.qv[kivi_v_token(r, 4 * h)][d] |
                               (uint32_t)sm.qv[kivi_v_token(r, 4 * h + 2)][d] << 8 |
                               (uint32_t)sm.qv[kivi_v_token(r, 4 * h + 1)][d] << 16 |
                               (uint32_t)sm.qv[kivi_v_token(r, 4 * h + 3)][d] << 24;
    }
  } else {
  // nibble dwords: 512 for K then 512 for V
  for (int w = tid; w < 512; w += NT) {
    // K dword w: chunk c = w / 4 (= tt*64 + jj*16 + u), dword m = w % 4
    const int ch = w / 4, m = w % 4;
    const int t = (ch / 64) * 16 + ch % 16, o = (ch % 64) / 16 + 4 * m;
    uint32_t x = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x |= (uint32_t)sm.qk[8 * o + 2 * i][t] << (4 * i);
      x |= (uint32_t)sm.qk[8 * o + 2 * i + 1][t] << (16 + 4 * i);
    }
    pw[w] = x;
    // V dword w: chunk c = hh*64 + r*16 + u, channel (4 hh + m)*16 + u
    const int hh = ch / 64, r = (ch % 64) / 16, u = ch % 16;
    const int d = (4 * hh + m) * 16 + u;
    uint32_t y = 0;
#pragma unroll
    for (int s = 0; s < 8; ++s)
      y |= (uint32_t)sm.qv[kivi_v_token(r, s)][d] << (16 * (s & 1) + 4 * (s >> 1));
    pw[F::kVCodes / 4 + w] = y;
  }
  }
  build_barrier<NT>();

  uint8_t* dst = j.pages + ((int64_t)pid * j.num_kv_heads + kvh) * F::kBytes;
  for (int i = tid; i < F::kBytes / 16; i += NT)
    reinterpret_cast<u32x4*>(dst)[i] = reinterpret_cast<const u32x4*>(sm.page)[i];
}

}  // namespace tl
