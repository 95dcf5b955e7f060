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
#include <cstddef>

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
  int build_ahead;          // 1: the steps build the next page in pieces (residual_length > 8)
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
  j.build_ahead = a.build_ahead;
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
// The unit's 32 values are read once, as 16 dwords (every row of k and v
// starts 4-byte aligned), scanned in order (ties and signed zeros keep
// the first occurrence, as the reference's scan), and the codes are
// written as 8 dwords: read back per code between byte stores, each read
// waited for the LDS.
template <int BITS>
__device__ __forceinline__ void quantise_unit(KiviBuildSmem<BITS>& sm, int u) {
  using F = KiviFmt<BITS>;
  constexpr int T = kKiviPageTokens, D = kKiviHead, LV = F::kLevels;
  static_assert(T == 32, "32 values per unit");
  static_assert(offsetof(KiviBuildSmem<BITS>, v) % 4 == 0 && offsetof(KiviBuildSmem<BITS>, qk) % 4 == 0 &&
                    offsetof(KiviBuildSmem<BITS>, qv) % 4 == 0 && sizeof(sm.k[0]) % 4 == 0 && sizeof(sm.v[0]) % 4 == 0,
                "rows of k, v, qk and qv start 4-byte aligned");
  const uint16_t* src;
  uint8_t* dst;
  if (u < D) {
    src = &sm.k[u][0];
    dst = &sm.qk[u][0];
  } else {
    const int t = (u - D) / 4, g = (u - D) % 4;
    src = &sm.v[t][g * 32];
    dst = &sm.qv[t][g * 32];
  }
  uint32_t w[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) w[i] = reinterpret_cast<const uint32_t*>(src)[i];
  float x[32];
#pragma unroll
  for (int i = 0; i < 32; ++i) x[i] = f16_to_f32(uint16_t(w[i / 2] >> (16 * (i & 1))));
  float gmin = FLT_MAX, gmax = -FLT_MAX;
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    if (x[i] < gmin) gmin = x[i];
    if (x[i] > gmax) gmax = x[i];
  }
  const GroupQ q = group_params<LV>(gmin, gmax);
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    uint32_t c = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) c |= (uint32_t)quantise<LV>(x[4 * k + e], q) << (8 * e);
    reinterpret_cast<uint32_t*>(dst)[k] = c;
  }
  if (u < D) {
    const int c = u;
    uint16_t* kp = reinterpret_cast<uint16_t*>(sm.page + F::kKParams + (c / 8) * 32);
    kp[c % 8] = q.step;
    kp[8 + c % 8] = q.zero;
  } else {
    const int t = (u - D) / 4, g = (u - D) % 4;
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
  // the page's slot is checked only before its store, so that the block
  // table and pool loads do not wait for it (one memory round trip fewer
  // before a build; a hole just skips the store)
  const int pid = j.page_tables[(int64_t)seq * j.max_pages_per_seq + page];
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

  if (pid < 0 || pid >= j.num_pages) return;
  uint8_t* dst = j.pages + ((int64_t)pid * j.num_kv_heads + kvh) * F::kBytes;
  for (int i = tid; i < F::kBytes / 16; i += NT)
    reinterpret_cast<u32x4*>(dst)[i] = reinterpret_cast<const u32x4*>(sm.page)[i];
}

// ---- build ahead: a page in pieces over the steps before it completes ----
//
// Page p of a sequence is quantised at the step whose length reaches
// 32 (p + 1) + R; its 32 tokens are all in the fp16 pool R steps earlier.
// With build-ahead the kKiviPieces steps before that one each write one
// piece of it, so that no step builds a whole page:
//   * piece i < 4: K channels of octets i, i + 4, i + 8, i + 12 (their codes
//     are the chunks 64 tt + 16 i + u, two runs of 16 chunks, and their
//     (step, zero) rows);
//   * piece 4 + r: V tokens of lane group r (4 r .. 4 r + 3 and
//     16 + 4 r .. 16 + 4 r + 3: chunks 64 hh + 16 r + u, and the (step,
//     zero) rows of (g, r)).
// A piece holds exactly the bytes that kivi_build_page writes there: each
// group's min / max is the sequential scan's (first occurrence on ties,
// NaN skipped), combined in scan order, and the quantiser is the same.
// Piece to build at length L, or -1: the next page to be quantised, d steps
// before the step that quantises it, builds piece kKiviPieces - d.
__device__ __forceinline__ int kivi_ahead_piece(int L, int residual_length, int& page) {
  page = kivi_quantized_len(L, residual_length) / kKiviPageTokens;
  const int d = kKiviPageTokens * (page + 1) + residual_length - L;
  return (d >= 1 && d <= kKiviPieces) ? kKiviPieces - d : -1;
}

// The sequential scans' combination of two partial scans, lo over earlier
// elements than hi: the earlier value wins ties (x < gmin / x > gmax).
__device__ __forceinline__ void scan_combine(float& mn, float& mx, float mn_hi, float mx_hi) {
  mn = mn_hi < mn ? mn_hi : mn;
  mx = mx_hi > mx ? mx_hi : mx;
}
// The value of lane lane ^ M: row permutations (no LDS round trip) up to
// M = 8 (4: the quad reversal of the half-row mirror, 8: the half-row
// mirror of the row mirror), an LDS-unit shuffle beyond.
constexpr int kDppQuadReverse = 0x1B;  // quad_perm [3,2,1,0]
template <int M>
__device__ __forceinline__ float lane_xor(float v) {
  if constexpr (M == 1) return dpp<kDppXor1>(v);
  else if constexpr (M == 2) return dpp<kDppXor2>(v);
  else if constexpr (M == 4) return dpp<kDppQuadReverse>(dpp<kDppHalfMirror>(v));
  else if constexpr (M == 8) return dpp<kDppHalfMirror>(dpp<kDppMirror>(v));
  else return shfl_xor(v, M);
}
template <int M>
__device__ __forceinline__ uint32_t lane_xor_u(uint32_t v) {
  return __builtin_bit_cast(uint32_t, lane_xor<M>(__builtin_bit_cast(float, v)));
}

// The same over lanes: xor butterfly over masks FIRST, 2 FIRST, .., LAST,
// the lane of lower index holding the earlier elements.
template <int FIRST, int LAST>
__device__ __forceinline__ void scan_combine_lanes(float& mn, float& mx, int lane) {
  if constexpr (FIRST <= LAST) {
    const float omn = lane_xor<FIRST>(mn), omx = lane_xor<FIRST>(mx);
    if (lane & FIRST) {
      float a = omn, b = omx;
      scan_combine(a, b, mn, mx);
      mn = a;
      mx = b;
    } else {
      scan_combine(mn, mx, omn, omx);
    }
    scan_combine_lanes<FIRST * 2, LAST>(mn, mx, lane);
  }
}

// A piece in phases that a workgroup can spread over other work: one
// wavefront plans it (the page slot and the pool blocks: table reads),
// loads the 2 KiB of fp16 it quantises and stages them in LDS; after a
// workgroup barrier each of four quarters is quantised and written by one
// wavefront.  Stores count on the same in-order counter as loads, so a
// wavefront that still has loads to wait for writes its quarter after them.
// Loads: K piece: lane = channel cl = lane / 2 of the piece over tokens
// 16 th .. 16 th + 15 (th = lane % 2), two runs of 8, each inside one
// block.  V piece: lane = channels lane and lane + 64 over the 8 token
// slots of lane group r, two runs of 4.
struct KiviPiece {
  int piece;        // -1: nothing to write
  int pid;          // page table entry (checked by the load phase)
  int phys[2];      // table entries of the blocks of the lane's two runs (checked by the load phase)
  uint32_t w[8];    // K: two runs of 8 halves; V: [channel half][run] 4 halves
};

__device__ __forceinline__ KiviPiece kivi_piece_plan(const PageJob& j, int seq, int page, int piece, int lane) {
  // the entries are only read here (the checks that use them come in the
  // load phase), so that nothing waits for them yet
  KiviPiece pc;
  pc.piece = (piece < 0 || page >= j.max_pages_per_seq) ? -1 : piece;
  if (pc.piece < 0) return pc;
  pc.pid = j.page_tables[(int64_t)seq * j.max_pages_per_seq + page];
  const int32_t* btab = j.block_tables + (int64_t)seq * j.max_blocks_per_seq;
  const int t_page = page * kKiviPageTokens;
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const int tok = piece < 4 ? t_page + 16 * (lane & 1) + 8 * r : t_page + 16 * r + 4 * (piece - 4);
    const int lb = min(tok / j.block_size, j.max_blocks_per_seq - 1);
    pc.phys[r] = tok / j.block_size < j.max_blocks_per_seq ? btab[lb] : -1;
  }
  return pc;
}

__device__ __forceinline__ void kivi_piece_load(const PageJob& j, KiviPiece& pc, int kvh, int page, int lane) {
  if (pc.piece < 0) return;
  if (pc.pid < 0 || pc.pid >= j.num_pages) {
    pc.piece = -1;                      // a page table hole: nothing to write
    return;
  }
#pragma unroll
  for (int r = 0; r < 2; ++r)
    if (pc.phys[r] < 0 || pc.phys[r] >= j.num_blocks) pc.phys[r] = -1;
  const int t_page = page * kKiviPageTokens;
  auto off_of = [&](int phys, int c, int tok) {
    return (((int64_t)phys * j.num_kv_heads + kvh) * kKiviHead + c) * j.block_size + tok % j.block_size;
  };
  if (pc.piece < 4) {
    const int cl = lane >> 1, c = 8 * (pc.piece + 4 * (cl >> 3)) + (cl & 7);
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const int tok = t_page + 16 * (lane & 1) + 8 * r;
      const u32x4 v = pc.phys[r] >= 0 ? load16(j.k_cache + off_of(pc.phys[r], c, tok)) : u32x4{0u, 0u, 0u, 0u};
      pc.w[4 * r] = v.x; pc.w[4 * r + 1] = v.y; pc.w[4 * r + 2] = v.z; pc.w[4 * r + 3] = v.w;
    }
  } else {
#pragma unroll
    for (int h2 = 0; h2 < 2; ++h2)
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        const int tok = t_page + 16 * r + 4 * (pc.piece - 4);
        const uint2 v = pc.phys[r] >= 0
                            ? *reinterpret_cast<const uint2*>(j.v_cache + off_of(pc.phys[r], lane + 64 * h2, tok))
                            : uint2{0u, 0u};
        pc.w[4 * h2 + 2 * r] = v.x;
        pc.w[4 * h2 + 2 * r + 1] = v.y;
      }
  }
}

// A workgroup's way through a piece: one wavefront plans and loads it and
// stages its fp16 in LDS (K: [channel of the piece][token], 32 x 32; V:
// [slot][channel], 8 x 128), then, after a workgroup barrier, each of four
// wavefronts quantises and writes a quarter: K octet piece + 4 q, or V
// channel group q.  A quarter is 256 values, 4 per lane, so each group's
// scan is 4 elements in order and then 3 combines across lanes.
__device__ __forceinline__ void kivi_piece_stage(const KiviPiece& pc, int lane, uint16_t* raw) {
  if (pc.piece < 0) return;
  if (pc.piece < 4) {
    u32x4* d = reinterpret_cast<u32x4*>(raw + (lane >> 1) * 32 + 16 * (lane & 1));
    d[0] = u32x4{pc.w[0], pc.w[1], pc.w[2], pc.w[3]};
    d[1] = u32x4{pc.w[4], pc.w[5], pc.w[6], pc.w[7]};
  } else {
#pragma unroll
    for (int h2 = 0; h2 < 2; ++h2)
#pragma unroll
      for (int sl = 0; sl < 8; ++sl)
        raw[sl * kKiviHead + lane + 64 * h2] = (uint16_t)(pc.w[4 * h2 + (sl >> 1)] >> (16 * (sl & 1)));
  }
}

// The lane's 4 staged values of quarter q: K, channel ci = lane % 8 of octet
// piece + 4 q at tokens 4 tq .. 4 tq + 3 (tq = lane / 8); V, slot lane / 8
// at channels 32 q + 4 (lane % 8) .. + 3.
__device__ __forceinline__ uint2 kivi_piece_quarter_values(int piece, int q, int lane, const uint16_t* raw) {
  return piece < 4 ? *reinterpret_cast<const uint2*>(raw + (8 * q + (lane & 7)) * 32 + 4 * (lane >> 3))
                   : *reinterpret_cast<const uint2*>(raw + (lane >> 3) * kKiviHead + 32 * q + 4 * (lane & 7));
}

// Quarter q of piece `piece` of the page in slot pid, from the lane's staged
// values (scratch: 256 B of the wavefront's own LDS).
template <int BITS>
__device__ void kivi_piece_quarter(const PageJob& j, int pid, int piece, int kvh, int q, int lane, uint2 rw,
                                   uint8_t* scratch) {
  using F = KiviFmt<BITS>;
  constexpr int LV = F::kLevels;
  uint8_t* dst = j.pages + ((int64_t)pid * j.num_kv_heads + kvh) * F::kBytes;
  float x[4];
  if (piece < 4) {
    // lane: channel ci of octet o = piece + 4 q, tokens 4 tq .. 4 tq + 3
    const int ci = lane & 7, tq = lane >> 3, o = piece + 4 * q;
#pragma unroll
    for (int i = 0; i < 4; ++i) x[i] = f16_to_f32((uint16_t)((i < 2 ? rw.x : rw.y) >> (16 * (i & 1))));
    float mn = FLT_MAX, mx = -FLT_MAX;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (x[i] < mn) mn = x[i];
      if (x[i] > mx) mx = x[i];
    }
    scan_combine_lanes<8, 32>(mn, mx, lane);
    const GroupQ g = group_params<LV>(mn, mx);
#pragma unroll
    for (int i = 0; i < 4; ++i) scratch[(4 * tq + i) * 8 + ci] = (uint8_t)quantise<LV>(x[i], g);
    if (tq == 0) {
      uint16_t* kp = reinterpret_cast<uint16_t*>(dst + F::kKParams + o * 32);
      kp[ci] = g.step;
      kp[8 + ci] = g.zero;
    }
    build_barrier<kWave>();
    if (lane < 32) {
      // token t = lane: the octet's 8 codes
      const uint2 cb = *reinterpret_cast<const uint2*>(scratch + lane * 8);
      auto b = [&](int c) { return (uint32_t)(((c < 4 ? cb.x : cb.y) >> (8 * (c & 3))) & 0xFFu); };
      uint8_t* chunk = dst + F::kKCodes + (64 * (lane >> 4) + 16 * piece + (lane & 15)) * F::kChunk;
      if constexpr (BITS == 8) {
        // dword 2 q + h: channels 4 h + {0, 2, 1, 3} of the octet
#pragma unroll
        for (int h = 0; h < 2; ++h)
          *reinterpret_cast<uint32_t*>(chunk + 4 * (2 * q + h)) =
              b(4 * h) | b(4 * h + 2) << 8 | b(4 * h + 1) << 16 | b(4 * h + 3) << 24;
      } else {
        // dword q: channel 2 i + hb at bit 16 hb + 4 i
        uint32_t x4 = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) x4 |= b(2 * i) << (4 * i) | b(2 * i + 1) << (16 + 4 * i);
        *reinterpret_cast<uint32_t*>(chunk + 4 * q) = x4;
      }
    }
  } else {
    // lane: slot sl, channels 32 q + 4 cq .. + 3 (group q)
    const int r = piece - 4, sl = lane >> 3, cq = lane & 7;
#pragma unroll
    for (int i = 0; i < 4; ++i) x[i] = f16_to_f32((uint16_t)((i < 2 ? rw.x : rw.y) >> (16 * (i & 1))));
    float mn = FLT_MAX, mx = -FLT_MAX;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (x[i] < mn) mn = x[i];
      if (x[i] > mx) mx = x[i];
    }
    scan_combine_lanes<1, 4>(mn, mx, lane);
    const GroupQ g = group_params<LV>(mn, mx);
#pragma unroll
    for (int i = 0; i < 4; ++i) scratch[(4 * cq + i) * 8 + sl] = (uint8_t)quantise<LV>(x[i], g);
    if (cq == 0) {
      uint16_t* vp = reinterpret_cast<uint16_t*>(dst + F::kVParams + (q * 4 + r) * 32);
      vp[sl] = g.step;
      vp[8 + sl] = g.zero;
    }
    build_barrier<kWave>();
    if (lane < 32) {
      // channel c = 32 q + lane = (4 hh + m) 16 + u: its 8 slots
      const int c = 32 * q + lane, hh = c >> 6, m = (c >> 4) & 3, u = c & 15;
      const uint2 cw = *reinterpret_cast<const uint2*>(scratch + lane * 8);
      auto cd = [&](int s2) { return (uint32_t)(((s2 < 4 ? cw.x : cw.y) >> (8 * (s2 & 3))) & 0xFFu); };
      uint8_t* chunk = dst + F::kVCodes + (64 * hh + 16 * r + u) * F::kChunk;
      if constexpr (BITS == 8) {
#pragma unroll
        for (int h = 0; h < 2; ++h)
          *reinterpret_cast<uint32_t*>(chunk + 4 * (2 * m + h)) =
              cd(4 * h) | cd(4 * h + 2) << 8 | cd(4 * h + 1) << 16 | cd(4 * h + 3) << 24;
      } else {
        uint32_t y = 0;
#pragma unroll
        for (int s2 = 0; s2 < 8; ++s2) y |= cd(s2) << (16 * (s2 & 1) + 4 * (s2 >> 1));
        *reinterpret_cast<uint32_t*>(chunk + 4 * m) = y;
      }
    }
  }
}

}  // namespace tl
