// tl_mfma_wave.hpp -- decode wavefronts on the matrix cores for head_size
// 128: FP8 E4M3 KV (fp8_wave) and 2-byte KV (mfma2_wave), block sizes
// 8 .. 256.  An iteration covers 64 (FP8) or 32
// (2-byte) consecutive tokens: several blocks when the block is smaller, a
// part of one block (at the iteration's offset in it) when it is larger.
//
// Both put the q heads on the 16 columns of v_mfma_f32_16x16x32_{f16,bf16},
// so one KV read serves up to 16 heads of a GQA group, and both keep the
// same accumulator layout: lane (m = lane & 15, kg = lane >> 4) holds head
// m, head dims 16 dt + 4 kg + r of O^T tile dt.
//   q.k, S^T[token][head] = K^T q^T.  The contraction runs over head dims,
//     the pool keeps tokens contiguous ([D][BS] per block), so K is
//     transposed in registers: a lane reads dwords of rows d = 4 j + kg
//     (j < 32; for each j the wavefront reads rows 4 j .. 4 j + 3 of the
//     iteration's tokens), and one v_perm_b32 per output dword pairs two
//     rows per token.  MFMA step s (k = 32) holds head dim
//     32 s + 4 e + kg in slot e of lane group kg; q is loaded in that order.
//   p.v, O^T[d][head] = V P^T.  A lane's score registers hold its head's
//     weights for a contiguous run of tokens that is exactly one k group of
//     the V operand (rows of V as loaded, no conversion for 2-byte KV), so
//     P^T needs no cross-lane move.
// Online softmax per lane (= head): running max with lazy rescaling (the
// weights exp2(s - m) stay below 2^8), fp32 sums and accumulators.
#pragma once

#include "tl_decode_wave.hpp"
#include "tl_device.hpp"

#include <math.h>

namespace tl {
namespace mw {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef __bf16 b8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef unsigned u4v __attribute__((ext_vector_type(4)));

constexpr int kHead = 128;
constexpr int kHeads = 16;          // q heads per wavefront: the MFMA columns
constexpr float kLazyRescale = 8.f; // rescale once the max grows by more than 2^8

template <Kind KV> constexpr int tokens_per_iteration() { return KV == Kind::FP8 ? 64 : 32; }

// Two E4M3 codes (bytes 0,1 or 2,3 of w) to two f16, exactly.
template <bool HI>
__device__ __forceinline__ uint32_t f8x2(uint32_t w) {
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, HI));
}

// 16x16x32 MFMA on four dwords of packed f16 / bf16 pairs per operand.
template <Kind T>
__device__ __forceinline__ f4 mma(uint32_t a0, uint32_t a1, uint32_t a2, uint32_t a3, const u4v& b, f4 c) {
  const u4v a = {a0, a1, a2, a3};
  if constexpr (T == Kind::BF16)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(b8, a), __builtin_bit_cast(b8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, a), __builtin_bit_cast(h8, b), c, 0, 0, 0);
}

__device__ __forceinline__ uint32_t ld_nt(const char* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(p));
}

// K of FP8 at block sizes 8 and 16 and of 2-byte KV at block size 8: lanes
// m and m ^ 1 (same kg) load rows 4 (2 j2) + kg and 4 (2 j2 + 1) + kg of
// their block, 8 bytes each: both lanes' token quads (FP8) or pairs (2-byte)
// of that row, the even lane's first.  One dword
// each way (DPP, adjacent lanes) leaves each lane its own quad of both
// rows, r0 of the first and r1 of the second.
__device__ __forceinline__ void k8_pair(uint32_t x, uint32_t y, bool odd, uint32_t& r0, uint32_t& r1) {
  const uint32_t send = odd ? x : y;
  const uint32_t recv = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)send, 0xB1, 0xF, 0xF, false);  // [1,0,3,2]
  r0 = odd ? recv : x;
  r1 = odd ? y : recv;
}

// Max / sum over the lanes l, l ^ 16, l ^ 32, l ^ 48.
__device__ __forceinline__ float max_kg(float v) {
  auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, v), __builtin_bit_cast(unsigned, v),
                                            false, false);
  v = fmaxf(__builtin_bit_cast(float, (unsigned)r[0]), __builtin_bit_cast(float, (unsigned)r[1]));
  r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(unsigned, v), __builtin_bit_cast(unsigned, v), false,
                                       false);
  return fmaxf(__builtin_bit_cast(float, (unsigned)r[0]), __builtin_bit_cast(float, (unsigned)r[1]));
}
__device__ __forceinline__ float sum_kg(float v) {
  v = swap32_add(v, v);
  return swap16_add(v, v);
}

// The blocks an iteration of TPI tokens starting at token it touches: NB
// blocks of BS tokens (BS < TPI), or the one block holding it (BS >= TPI).
template <int BS, int TPI> constexpr int blocks_per_iteration() { return BS >= TPI ? 1 : TPI / BS; }
// Byte offset of token it inside its block's rows (elements of E bytes):
// non-zero only when a block holds more than one iteration.
template <int BS, int TPI, int E>
__device__ __forceinline__ int in_block_bytes(int it) { return BS > TPI ? E * (it % BS) : 0; }

// A sequence's block-table row read through the constant address space:
// the table is not written during the kernel, and with wave-uniform
// indices the reads are scalar loads, waited for on their own counter, so
// no K/V load in flight is waited for on account of a table entry.
typedef const __attribute__((address_space(4))) int32_t* TableRow;

// Physical blocks of the NB blocks starting at token it (< 0: hole, past t1
// or outside the pool).  Every entry is read, at an index clamped to the
// row (max_blocks_per_seq >= 1), and checked afterwards: a read under a
// condition would make the compiler wait for every load in flight before
// the entries are used.
// table_raw issues the reads, table_check applies the checks: split, the
// reads of a prologue can all be in flight before the first is used.
template <int NB> struct Blocks { int e[NB]; };
template <int NB, int BS>
__device__ __forceinline__ Blocks<NB> table_raw(const Params& p, TableRow table, int it) {
  Blocks<NB> b;
#pragma unroll
  for (int i = 0; i < NB; ++i)
    b.e[i] = table[__builtin_amdgcn_readfirstlane(min((it + BS * i) / BS, p.max_blocks_per_seq - 1))];
  return b;
}
template <int NB, int BS>
__device__ __forceinline__ Blocks<NB> table_check(const Params& p, Blocks<NB> b, int it, int t1) {
#pragma unroll
  for (int i = 0; i < NB; ++i) {
    const int tok = it + BS * i, lb = tok / BS;
    b.e[i] = (tok >= t1 || lb >= p.max_blocks_per_seq || b.e[i] >= p.num_blocks) ? -1 : b.e[i];
  }
  return b;
}
template <int NB, int BS>
__device__ __forceinline__ Blocks<NB> table_blocks(const Params& p, TableRow table, int it, int t1) {
  return table_check<NB, BS>(p, table_raw<NB, BS>(p, table, it), it, t1);
}
// Entry i (per lane) of a wave-uniform set.  Written as one nested select:
// a select loop over k is turned back into an indexed load, which puts the
// set in LDS.
template <int NB>
__device__ __forceinline__ int pick(const Blocks<NB>& b, int i) {
  static_assert(NB == 1 || NB == 2 || NB == 4 || NB == 8, "1, 2, 4 or 8 blocks per iteration");
  if constexpr (NB == 8)
    return i < 4 ? (i < 2 ? (i == 0 ? b.e[0] : b.e[1]) : (i == 2 ? b.e[2] : b.e[3]))
                 : (i < 6 ? (i == 4 ? b.e[4] : b.e[5]) : (i == 6 ? b.e[6] : b.e[7]));
  else if constexpr (NB == 4) return i == 0 ? b.e[0] : i == 1 ? b.e[1] : i == 2 ? b.e[2] : b.e[3];
  else if constexpr (NB == 2) return i == 0 ? b.e[0] : b.e[1];
  else return b.e[0];
}

// Zeroes the bytes of tokens >= n (0 <= n <= 16) of a 16-token FP8 row.
__device__ __forceinline__ u32x4 keep_bytes(const u32x4& v, int n) {
  uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int k = n - 4 * i;   // bytes of this word to keep
    const uint32_t mask = k >= 4 ? 0xffffffffu : k <= 0 ? 0u : (0xffffffffu >> (32 - 8 * k));
    w[i] &= mask;
  }
  return u32x4{w[0], w[1], w[2], w[3]};
}
// Keeps byte j of a 16-token FP8 row where bit j of keep is set.
__device__ __forceinline__ u32x4 keep_byte_mask(const u32x4& v, uint32_t keep) {
  uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    uint32_t mask = 0;
#pragma unroll
    for (int b = 0; b < 4; ++b) mask |= ((keep >> (4 * i + b)) & 1u) ? (0xffu << (8 * b)) : 0u;
    w[i] &= mask;
  }
  return u32x4{w[0], w[1], w[2], w[3]};
}
// Zeroes the 2-byte elements >= n (0 <= n <= 8) of an 8-token run.
__device__ __forceinline__ u32x4 keep_halves(const u32x4& v, int n) {
  uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int k = n - 2 * i;
    w[i] &= k >= 2 ? 0xffffffffu : k == 1 ? 0xffffu : 0u;
  }
  return u32x4{w[0], w[1], w[2], w[3]};
}

// The running softmax state of a wavefront and its hand-over to LDS
// (s_acc_w [16][128] unnormalised, times v_scale; s_m_w [16] in log2 units;
// s_l_w [16]).
struct State {
  f4 o[8];
  float m_run, l_lane;
  __device__ __forceinline__ void init() {
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) o[dt] = f4{0.f, 0.f, 0.f, 0.f};
    m_run = -INFINITY;
    l_lane = 0.f;
  }
  // Raises the running max to the wavefront's new max mx when it grew by
  // more than 2^8 for some head.
  __device__ __forceinline__ void update_max(float mx) {
    const float m_new = fmaxf(m_run, max_kg(mx));
    if (__builtin_amdgcn_ballot_w64(m_new > m_run + kLazyRescale) != 0) {
      const float alpha = (m_run == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(m_run - m_new);
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) o[dt] *= alpha;
      l_lane *= alpha;
      m_run = m_new;
    }
  }
  __device__ __forceinline__ void store(float v_scale, int m, int kg, float* s_acc_w, float* s_m_w,
                                        float* s_l_w) const {
    const float l_tot = sum_kg(l_lane);
#pragma unroll
    for (int dt = 0; dt < 8; ++dt)
      *reinterpret_cast<f4*>(&s_acc_w[m * kHead + 16 * dt + 4 * kg]) = o[dt] * v_scale;
    if (kg == 0) {
      s_m_w[m] = m_run;
      s_l_w[m] = l_tot;
    }
  }
};

// What a wavefront does at the boundaries of the partitions it streams:
// nothing (NoFlush: the caller takes the state at the end), or hand the
// finished partition's state to a sink and start the next one afresh.
struct NoFlush {
  static constexpr bool kActive = false;
  int part_tokens = 1;
  __device__ void operator()(const State&, int) const {}
};

// ---- FP8 E4M3 KV, f16 / bf16 q: 64 tokens per iteration ----
//
// K: the A row m is token quad m (iteration tokens 4 m .. 4 m + 3) and tile
// i takes token i of every quad.  Lane (m, kg) reads 32 dwords, rows
// 4 j + kg of its quad (at block size 16 the wavefront reads 64 contiguous
// bytes per block for each j); one v_perm_b32 stage pairs the bytes of two
// rows per token, and the converter's (bytes 0,1) / (bytes 2,3) halves are
// then exactly the f16 (d, d') pairs of one token: 1 perm and 2 converts
// per 4 bytes.  v_cvt_scalef32_pk_f16_fp8 with scale 1 is exact: every E4M3
// value, subnormals and NaN included, is an f16 value.
// Scores: lane (m, kg) holds head m, iteration token 16 kg + 4 r + i.
// V: lane (m, kg) loads the 16 bytes of row d = 16 dt + m for iteration
// tokens 16 kg .. 16 kg + 15 (one block row at block size 16; at block size
// 8 two 8-byte runs, one from each of the two blocks); MFMA h takes its
// tokens 8 h .. 8 h + 7.
// bf16 q is brought into f16 range by a power of two per head (exact: max
// |q| in [2^14, 2^15)); the factor returns in the score scale.  The
// dequant scales fold into the score scale (k_scale) and the output
// (v_scale).
template <Kind QK, int BS, class Flush = NoFlush>
__device__ __forceinline__ State fp8_wave(const Params& p, int seq, int kvh, int hs, int first_it, int t1,
                                          int step, const Flush& flush = Flush(), int len = 0x7fffffff) {
  static_assert(BS >= 8 && (BS & (BS - 1)) == 0, "block size: a power of two >= 8");
  t1 = min(t1, len);
  constexpr int TPI = 64, RB = BS;           // tokens per iteration; bytes per head-dim row of a block
  constexpr bool kSplitRun = BS == 8;        // a lane's 16-token V run spans two blocks
  constexpr int kBlockBytes = kHead * RB;
  constexpr int NB = blocks_per_iteration<BS, TPI>();
  const int lane = threadIdx.x % kWave;
  const int m = lane & 15, kg = lane >> 4;

  // ---- q of head column m in MFMA order: slot (s, e) = dim 32 s + 4 e + kg ----
  const int gi = hs * kHeads + m;
  const bool hv = gi < p.group;
  const int head = hv ? head_of(p, kvh, gi) : 0;
  const uint16_t* qrow = (const uint16_t*)p.q + ((int64_t)seq * p.num_heads + head) * kHead;
  // the loads under one condition, used after it: loads under a condition
  // of their own were each a branch with a wait, 32 round trips in a row
  uint16_t qh[32] = {};
  if (hv) {
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int e = 0; e < 8; ++e) qh[8 * s + e] = qrow[32 * s + 4 * e + kg];
  }
  float qf[32];
  float qmax = 0.f;
#pragma unroll
  for (int s = 0; s < 4; ++s)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint16_t bits = qh[8 * s + e];
      const float v = QK == Kind::BF16 ? bf16_to_f32(bits) : f16_to_f32(bits);
      qf[8 * s + e] = v;
      qmax = fmaxf(qmax, fabsf(v));
    }
  int sh = 0;
  if constexpr (QK == Kind::BF16) {
    qmax = max_kg(qmax);
    if (qmax > 0.f && qmax < INFINITY) {
      int ex;
      frexpf(qmax, &ex);
      sh = 15 - ex;
    }
  }
  u4v qb[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    h8 v;
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = (_Float16)ldexpf(qf[8 * s + e], sh);
    qb[s] = __builtin_bit_cast(u4v, v);
  }
  const float qk_scale = p.qk_scale * ldexpf(1.f, -sh);

  State st;
  st.init();

  const TableRow table = (TableRow)(p.block_tables + (int64_t)seq * p.max_blocks_per_seq);
  const int64_t pool_stride = (int64_t)p.num_kv_heads * kBlockBytes;
  // this lane's K quad and V run: their blocks within the iteration and
  // their byte offsets in a block row (plus the iteration's own offset when
  // a block holds several iterations)
  // Block sizes 8 and 16 load K 8 bytes per lane (k8_pair), so that each
  // load instruction reads whole 128-byte lines of a block (4-byte loads
  // read 64-byte halves of four blocks' lines).
  constexpr bool kK8 = BS <= 16;
  const bool odd = (m & 1) != 0;
  const int kb = NB > 1 ? (4 * m) / BS : 0, vb = NB > 1 ? (16 * kg) / BS : 0;
  const char* kbase0 = kK8 ? p.k_cache + (int64_t)kvh * kBlockBytes + RB * kg + (4 * (m & ~1)) % BS + 4 * RB * (m & 1)
                           : p.k_cache + (int64_t)kvh * kBlockBytes + RB * kg + (4 * m) % (NB > 1 ? BS : TPI);
  const char* vbase0 = p.v_cache + (int64_t)kvh * kBlockBytes + RB * m + (16 * kg) % (NB > 1 ? BS : TPI);
  auto load_k = [&](uint32_t (&kw)[32], const char* base) {
    if constexpr (kK8) {
      typedef unsigned u2v __attribute__((ext_vector_type(2)));
#pragma unroll
      for (int j2 = 0; j2 < 16; ++j2) {
        const u2v w = __builtin_nontemporal_load(reinterpret_cast<const u2v*>(base + 8 * RB * j2));
        kw[2 * j2] = w.x;
        kw[2 * j2 + 1] = w.y;
      }
    } else {
#pragma unroll
      for (int j = 0; j < 32; ++j) kw[j] = ld_nt(base + 4 * RB * j);
    }
  };
  // base: the run's block (its first 8 tokens' block at block size 8),
  // base2: the block of tokens 8 .. 15 at block size 8 (unused otherwise)
  auto load_v = [&](u32x4 (&vr)[8], const char* base, const char* base2) {
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      if constexpr (kSplitRun) {
        typedef unsigned u2v __attribute__((ext_vector_type(2)));
        const u2v lo = __builtin_nontemporal_load(reinterpret_cast<const u2v*>(base + 16 * RB * dt));
        const u2v hi = __builtin_nontemporal_load(reinterpret_cast<const u2v*>(base2 + 16 * RB * dt));
        vr[dt] = u32x4{lo.x, lo.y, hi.x, hi.y};
      } else {
        vr[dt] = load16_stream(base + 16 * RB * dt);
      }
    }
  };
  const int vb2 = kSplitRun ? vb + 1 : vb;
  auto v_at = [&](const Blocks<NB>& b, int ib, int which) {
    return vbase0 + ib + (int64_t)max(pick(b, which), 0) * pool_stride;
  };

  int it = first_it;
  Blocks<NB> cur = table_blocks<NB, BS>(p, table, it, t1);
  Blocks<NB> nxt = table_blocks<NB, BS>(p, table, it + step, t1);
  uint32_t kw[32];
  u32x4 vr[8];
  {
    // in the loop's order (K, then V), so that the loop's waits can count
    // the loads in flight from its first iteration on
    const int ib = in_block_bytes<BS, TPI, 1>(it);
    load_k(kw, kbase0 + ib + (int64_t)max(pick(cur, kb), 0) * pool_stride);
    __builtin_amdgcn_sched_barrier(0);
    load_v(vr, v_at(cur, ib, vb), v_at(cur, ib, vb2));
  }

#pragma unroll 1
  for (; it < t1; it += step) {
    if constexpr (Flush::kActive) {
      if (it != first_it && it % flush.part_tokens == 0) {   // a partition ends: its partials out, state afresh
        flush(st, it / flush.part_tokens - 1);
        st.init();
      }
    }
    const Blocks<NB> nn = table_blocks<NB, BS>(p, table, it + 2 * step, t1);
    const int ib_next = in_block_bytes<BS, TPI, 1>(it + step);

    // ---- q.k: 4 tiles (token i of each quad) x 4 MFMA steps ----
    f4 s[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) s[i] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int sk = 0; sk < 4; ++sk) {
      uint32_t a[4][4];   // [tile][f16 pair]
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        const int j0 = 8 * sk + 4 * hf;             // rows 32 sk + 16 hf + 4 c + kg
        uint32_t w[4];
        if constexpr (kK8) {
          k8_pair(kw[j0], kw[j0 + 1], odd, w[0], w[1]);
          k8_pair(kw[j0 + 2], kw[j0 + 3], odd, w[2], w[3]);
        } else {
#pragma unroll
          for (int c = 0; c < 4; ++c) w[c] = kw[j0 + c];
        }
        const uint32_t x0 = __builtin_amdgcn_perm(w[1], w[0], 0x05010400u);  // tokens 0, 1
        const uint32_t x1 = __builtin_amdgcn_perm(w[1], w[0], 0x07030602u);  // tokens 2, 3
        const uint32_t y0 = __builtin_amdgcn_perm(w[3], w[2], 0x05010400u);
        const uint32_t y1 = __builtin_amdgcn_perm(w[3], w[2], 0x07030602u);
        a[0][2 * hf] = f8x2<false>(x0); a[0][2 * hf + 1] = f8x2<false>(y0);
        a[1][2 * hf] = f8x2<true>(x0);  a[1][2 * hf + 1] = f8x2<true>(y0);
        a[2][2 * hf] = f8x2<false>(x1); a[2][2 * hf + 1] = f8x2<false>(y1);
        a[3][2 * hf] = f8x2<true>(x1);  a[3][2 * hf + 1] = f8x2<true>(y1);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) s[i] = mma<Kind::F16>(a[i][0], a[i][1], a[i][2], a[i][3], qb[sk], s[i]);
    }
    // the next iteration's loads are issued whether or not it exists (a
    // missing one reads block 0): under a condition the compiler would
    // wait for them, too, before this iteration's V is used
    load_k(kw, kbase0 + ib_next + (int64_t)max(pick(nxt, kb), 0) * pool_stride);

    // ---- softmax: lane (m, kg) owns head m, iteration tokens 16 kg + 4 r + i ----
    const int ph_v = pick(cur, vb);
    int n_ok;
    uint32_t keep = 0xffffu;   // block size 8: the run's tokens that exist (bit t: token 16 kg + t)
    if constexpr (kSplitRun) {
      n_ok = min(max(t1 - (it + 16 * kg), 0), 16);
      keep = (n_ok >= 16 ? 0xffffu : ((1u << n_ok) - 1u)) & (ph_v < 0 ? 0xff00u : 0xffffu) &
             (pick(cur, vb2) < 0 ? 0x00ffu : 0xffffu);
    } else {
      n_ok = ph_v < 0 ? 0 : min(max(t1 - (it + 16 * kg), 0), 16);
    }
    auto tok_ok = [&](int t) { return kSplitRun ? ((keep >> t) & 1u) != 0 : t < n_ok; };
    float sc[4][4];
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        sc[i][r] = tok_ok(4 * r + i) ? s[i][r] * qk_scale : -INFINITY;
        mx = fmaxf(mx, sc[i][r]);
      }
    st.update_max(mx);
    float pw[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        pw[i][r] = tok_ok(4 * r + i) ? __builtin_amdgcn_exp2f(sc[i][r] - st.m_run) : 0.f;
        st.l_lane += pw[i][r];
      }
    // P^T operands: MFMA h takes tokens 8 h .. 8 h + 7 = (r = 2 h, 2 h + 1) x (i = 0 .. 3)
    u4v pb[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      h8 v;
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = (_Float16)pw[e & 3][2 * h + (e >> 2)];
      pb[h] = __builtin_bit_cast(u4v, v);
    }

    // ---- p.v: tokens past t1 and holes may hold any byte (NaN codes too) ----
    if constexpr (kSplitRun) {
      if (__builtin_amdgcn_ballot_w64(keep != 0xffffu) != 0) {
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) vr[dt] = keep_byte_mask(vr[dt], keep);
      }
    } else if (__builtin_amdgcn_ballot_w64(n_ok < 16) != 0) {
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) vr[dt] = keep_bytes(vr[dt], n_ok);
    }
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const u32x4 v = vr[dt];
      st.o[dt] = mma<Kind::F16>(f8x2<false>(v.x), f8x2<true>(v.x), f8x2<false>(v.y), f8x2<true>(v.y), pb[0],
                                st.o[dt]);
      st.o[dt] = mma<Kind::F16>(f8x2<false>(v.z), f8x2<true>(v.z), f8x2<false>(v.w), f8x2<true>(v.w), pb[1],
                                st.o[dt]);
    }
    load_v(vr, v_at(nxt, ib_next, vb), v_at(nxt, ib_next, vb2));
    cur = nxt;
    nxt = nn;
  }
  return st;
}

// ---- 2-byte KV (f16 / bf16, q of the same type): 32 tokens per iteration ----
//
// K: the A row m is token pair m (iteration tokens 2 m, 2 m + 1) and tile i
// takes token i of every pair.  Lane (m, kg) reads 32 dwords, rows 4 j + kg
// of its pair (at block size 16 the wavefront reads 128 contiguous bytes
// per block for each j); v_perm_b32 of the dwords of rows (e, e + 1) gives
// the (d, d') pair of the pair's first (low halves) or second (high halves)
// token: 1 perm per operand dword.
// Scores: lane (m, kg) holds head m, iteration tokens 8 kg + 2 r + i, i.e.
// the run of 8 tokens that is k group kg of the p.v MFMA.
// V: lane (m, kg) loads the 16 bytes of that run, row d = 16 dt + m.
// len: the sequence's length when t1 does not include it yet (the token
// range is [first_it, min(t1, len)); the prologue's loads do not wait for it).
// ITERS 1 or 2: the wavefront runs at most that many iterations (the
// plan's partitions are at most ITERS steps long): their K/V are all loaded
// in the prologue, and no table entry or K/V past them is read (64 more
// registers for 2).  0: any number, one iteration's loads ahead.
template <Kind KV, int BS, class Flush = NoFlush, int ITERS = 0>
__device__ __forceinline__ State mfma2_wave(const Params& p, int seq, int kvh, int hs, int first_it, int t1,
                                            int step, const Flush& flush = Flush(), int len = 0x7fffffff) {
  static_assert(BS >= 8 && (BS & (BS - 1)) == 0, "block size: a power of two >= 8");
  constexpr int TPI = 32, RB = 2 * BS;       // tokens per iteration; bytes per head-dim row of a block
  constexpr int kBlockBytes = kHead * RB;
  constexpr int NB = blocks_per_iteration<BS, TPI>();
  const int lane = threadIdx.x % kWave;
  const int m = lane & 15, kg = lane >> 4;

  // ---- q of head column m: dword e2 of step s = dims (32 s + 8 e2 + kg, +4) ----
  const int gi = hs * kHeads + m;
  const bool hv = gi < p.group;
  const int head = hv ? head_of(p, kvh, gi) : 0;
  const uint16_t* qrow = (const uint16_t*)p.q + ((int64_t)seq * p.num_heads + head) * kHead;

  State st;
  st.init();

  const TableRow table = (TableRow)(p.block_tables + (int64_t)seq * p.max_blocks_per_seq);
  const int64_t pool_stride = (int64_t)p.num_kv_heads * kBlockBytes;
  // this lane's K pair and V run: their blocks within the iteration and
  // their byte offsets in a block row (plus the iteration's own offset when
  // a block holds several iterations)
  // Block size 8 loads K 8 bytes per lane (two token pairs of a row, lanes
  // m and m ^ 1 on alternate rows: k8_pair), so that each load instruction
  // reads whole 128-byte lines of a block (4-byte loads read 64-byte halves
  // of four blocks' lines there).
  constexpr bool kK8 = BS == 8;
  const bool odd = (m & 1) != 0;
  const int kb = NB > 1 ? (2 * m) / BS : 0, vb = NB > 1 ? (8 * kg) / BS : 0;
  const char* kbase0 = kK8 ? p.k_cache + (int64_t)kvh * kBlockBytes + RB * kg + 2 * ((2 * (m & ~1)) % BS) + 4 * RB * (m & 1)
                           : p.k_cache + (int64_t)kvh * kBlockBytes + RB * kg + 2 * ((2 * m) % (NB > 1 ? BS : TPI));
  const char* vbase0 = p.v_cache + (int64_t)kvh * kBlockBytes + RB * m + 2 * ((8 * kg) % (NB > 1 ? BS : TPI));
  auto load_k = [&](uint32_t (&kw)[32], const char* base) {
    if constexpr (kK8) {
      typedef unsigned u2v __attribute__((ext_vector_type(2)));
#pragma unroll
      for (int j2 = 0; j2 < 16; ++j2) {
        const u2v w = __builtin_nontemporal_load(reinterpret_cast<const u2v*>(base + 8 * RB * j2));
        kw[2 * j2] = w.x;
        kw[2 * j2 + 1] = w.y;
      }
    } else {
#pragma unroll
      for (int j = 0; j < 32; ++j) kw[j] = ld_nt(base + 4 * RB * j);
    }
  };
  auto load_v = [&](u32x4 (&vr)[8], const char* base) {
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) vr[dt] = load16_stream(base + 16 * RB * dt);
  };

  // The prologue in the order of its round trips: the table entries (all
  // in flight together), q (the loads under one condition, used after it:
  // loads under a condition of their own were each a branch with a wait),
  // the first K/V, and q is packed while they fly.  Entries past len may be loaded: in bounds, and
  // masked by the scores' valid-token count.
  int it = first_it;
  const Blocks<NB> cur_raw = table_raw<NB, BS>(p, table, it);
  const Blocks<NB> nxt_raw = ITERS == 1 ? cur_raw : table_raw<NB, BS>(p, table, it + step);
  __builtin_amdgcn_sched_barrier(0);
  Blocks<NB> cur = table_check<NB, BS>(p, cur_raw, it, t1);
  Blocks<NB> nxt = table_check<NB, BS>(p, nxt_raw, it + step, t1);
  uint32_t qlo[16] = {}, qhi[16] = {};
  if (hv) {
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int e2 = 0; e2 < 4; ++e2) {
        qlo[4 * s + e2] = qrow[32 * s + 8 * e2 + kg];
        qhi[4 * s + e2] = qrow[32 * s + 8 * e2 + 4 + kg];
      }
  }
  uint32_t kw[32];
  u32x4 vr[8];
  {
    // in the loop's order (K, then V), so that the loop's waits can count
    // the loads in flight from its first iteration on
    const int ib = in_block_bytes<BS, TPI, 2>(it);
    load_k(kw, kbase0 + ib + (int64_t)max(pick(cur, kb), 0) * pool_stride);
    __builtin_amdgcn_sched_barrier(0);
    load_v(vr, vbase0 + ib + (int64_t)max(pick(cur, vb), 0) * pool_stride);
    __builtin_amdgcn_sched_barrier(0);
  }
  // ITERS 2: the second iteration's K/V in a set of their own
  uint32_t kw2[ITERS == 2 ? 32 : 1];
  u32x4 vr2[ITERS == 2 ? 8 : 1];
  if constexpr (ITERS == 2) {
    const int ib = in_block_bytes<BS, TPI, 2>(it + step);
    load_k(kw2, kbase0 + ib + (int64_t)max(pick(nxt, kb), 0) * pool_stride);
    __builtin_amdgcn_sched_barrier(0);
    load_v(vr2, vbase0 + ib + (int64_t)max(pick(nxt, vb), 0) * pool_stride);
    __builtin_amdgcn_sched_barrier(0);
  }
  t1 = min(t1, len);
  // q's registers are opaque from here: otherwise the compiler packs them
  // inside the condition, and waits for q there, before K/V are issued
#pragma unroll
  for (int i = 0; i < 16; ++i) asm volatile("" : "+v"(qlo[i]), "+v"(qhi[i]));
  u4v qb[4];
#pragma unroll
  for (int s = 0; s < 4; ++s)
#pragma unroll
    for (int e2 = 0; e2 < 4; ++e2) qb[s][e2] = qlo[4 * s + e2] | (qhi[4 * s + e2] << 16);

  // One iteration at token it on (kwA, vrA); with reload, their K/V are
  // then loaded with the iteration of table entries ld (in-block offset
  // ib_ld).
  auto iterate = [&](uint32_t (&kwA)[32], u32x4 (&vrA)[8], const Blocks<NB>& c, const Blocks<NB>& ld,
                     int ib_ld, bool reload) {
      // ---- q.k: 2 tiles (token i of each pair) x 4 MFMA steps ----
      f4 s[2] = {f4{0.f, 0.f, 0.f, 0.f}, f4{0.f, 0.f, 0.f, 0.f}};
  #pragma unroll
      for (int sk = 0; sk < 4; ++sk) {
        uint32_t w[8];                              // rows 32 sk + 4 e + kg
        if constexpr (kK8) {
  #pragma unroll
          for (int e2 = 0; e2 < 4; ++e2) k8_pair(kwA[8 * sk + 2 * e2], kwA[8 * sk + 2 * e2 + 1], odd, w[2 * e2], w[2 * e2 + 1]);
        } else {
  #pragma unroll
          for (int e = 0; e < 8; ++e) w[e] = kwA[8 * sk + e];
        }
        uint32_t a[2][4];
  #pragma unroll
        for (int e2 = 0; e2 < 4; ++e2) {
          a[0][e2] = __builtin_amdgcn_perm(w[2 * e2 + 1], w[2 * e2], 0x05040100u);  // first token
          a[1][e2] = __builtin_amdgcn_perm(w[2 * e2 + 1], w[2 * e2], 0x07060302u);  // second token
        }
  #pragma unroll
        for (int i = 0; i < 2; ++i) s[i] = mma<KV>(a[i][0], a[i][1], a[i][2], a[i][3], qb[sk], s[i]);
      }
      // the next iteration's loads are issued whether or not it exists (a
      // missing one reads block 0): under a condition the compiler would
      // wait for them, too, before this iteration's V is used
      if (reload) load_k(kwA, kbase0 + ib_ld + (int64_t)max(pick(ld, kb), 0) * pool_stride);

      // ---- softmax: lane (m, kg) owns head m, iteration tokens 8 kg + 2 r + i ----
      const int ph_v = pick(c, vb);
      const int n_run = ph_v < 0 ? 0 : min(max(t1 - (it + 8 * kg), 0), 8);   // valid tokens of the run
      float sc[2][4];
      float mx = -INFINITY;
  #pragma unroll
      for (int i = 0; i < 2; ++i)
  #pragma unroll
        for (int r = 0; r < 4; ++r) {
          sc[i][r] = (2 * r + i < n_run) ? s[i][r] * p.qk_scale : -INFINITY;
          mx = fmaxf(mx, sc[i][r]);
        }
      st.update_max(mx);
      // bf16 weights carry 8 mantissa bits: a short or peaked softmax would
      // miss 2e-3 by up to 2^-9 max|v|, so bf16 splits each weight into a
      // bf16 high part and the bf16 rounding of the rest (relative 2^-18)
      // and p.v takes both (f16 weights are exact enough alone)
      u4v pb, pl;
  #pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float p0 = (2 * r < n_run) ? __builtin_amdgcn_exp2f(sc[0][r] - st.m_run) : 0.f;
        const float p1 = (2 * r + 1 < n_run) ? __builtin_amdgcn_exp2f(sc[1][r] - st.m_run) : 0.f;
        st.l_lane += p0 + p1;
        pb[r] = Dot2<KV>::pack(p0, p1);
        if constexpr (KV == Kind::BF16) {
          const float h0 = __builtin_bit_cast(float, pb[r] << 16), h1 = __builtin_bit_cast(float, pb[r] & 0xffff0000u);
          pl[r] = Dot2<KV>::pack(p0 - h0, p1 - h1);
        }
      }

      // ---- p.v: slots past t1 and holes may hold anything, NaN included ----
      if (__builtin_amdgcn_ballot_w64(n_run < 8) != 0) {
  #pragma unroll
        for (int dt = 0; dt < 8; ++dt) vrA[dt] = keep_halves(vrA[dt], n_run);
      }
  #pragma unroll
      for (int dt = 0; dt < 8; ++dt) {
        st.o[dt] = mma<KV>(vrA[dt].x, vrA[dt].y, vrA[dt].z, vrA[dt].w, pb, st.o[dt]);
        if constexpr (KV == Kind::BF16) st.o[dt] = mma<KV>(vrA[dt].x, vrA[dt].y, vrA[dt].z, vrA[dt].w, pl, st.o[dt]);
      }
      if (reload) load_v(vrA, vbase0 + ib_ld + (int64_t)max(pick(ld, vb), 0) * pool_stride);
  };

  if constexpr (ITERS > 0) {
    static_assert(!Flush::kActive, "partition flushes stream whole partitions");
    if (it < t1) {
      iterate(kw, vr, cur, cur, 0, false);
      it += step;
      if constexpr (ITERS == 2)
        if (it < t1) iterate(kw2, vr2, nxt, nxt, 0, false);
    }
  } else {
#pragma unroll 1
    for (; it < t1; it += step) {
      if constexpr (Flush::kActive) {
        if (it != first_it && it % flush.part_tokens == 0) {   // a partition ends: its partials out, state afresh
          flush(st, it / flush.part_tokens - 1);
          st.init();
        }
      }
      const Blocks<NB> nn = table_blocks<NB, BS>(p, table, it + 2 * step, t1);
      iterate(kw, vr, cur, nxt, in_block_bytes<BS, TPI, 2>(it + step), true);
      cur = nxt;
      nxt = nn;
    }
  }
  return st;
}

template <Kind KV, Kind QK, int BS, class Flush = NoFlush, int ITERS = 0>
__device__ __forceinline__ State run_wave(const Params& p, int seq, int kvh, int hs, int first_it, int t1,
                                          int step, const Flush& flush = Flush(), int len = 0x7fffffff) {
  if constexpr (KV == Kind::FP8)
    return fp8_wave<QK, BS>(p, seq, kvh, hs, first_it, t1, step, flush, len);
  else
    return mfma2_wave<KV, BS, Flush, ITERS>(p, seq, kvh, hs, first_it, t1, step, flush, len);
}

// A wavefront that ran a whole split-K partition alone writes its
// partials straight from registers: lane (m, kg) holds dims 16 dt + 4 kg +
// r of head m, normalised by the head's sum; the (max, sum) pair in
// natural-log units from the lanes of kg 0.  A head with no valid token
// gets sum 0 (and max -inf), which the log-sum-exp merge skips.
struct Partial {
  f4 o[8];
  float m, l;
};
__device__ __forceinline__ Partial finish_partial(const State& st, float v_scale) {
  const float l_tot = sum_kg(st.l_lane);
  const float f = l_tot > 0.f ? v_scale / l_tot : 0.f;
  Partial r;
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) r.o[dt] = st.o[dt] * f;
  r.m = l_tot > 0.f ? st.m_run * (1.0f / kLog2e) : -INFINITY;
  r.l = l_tot;
  return r;
}
__device__ __forceinline__ void store_partial(const Params& p, const Partial& r, int seq, int kvh, int hs,
                                              int part) {
  const int lane = threadIdx.x % kWave;
  const int m = lane & 15, kg = lane >> 4;
  const int gi = hs * kHeads + m;
  if (gi >= p.group) return;
  const int64_t pi = ((int64_t)seq * p.num_heads + head_of(p, kvh, gi)) * p.num_partitions + part;
  float* o = reinterpret_cast<float*>(p.part_o) + pi * kHead;
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) *reinterpret_cast<f4*>(o + 16 * dt + 4 * kg) = r.o[dt];
  if (kg == 0) {
    p.part_m[pi] = r.m;
    p.part_l[pi] = r.l;
  }
}
__device__ __forceinline__ void write_partial(const Params& p, const State& st, float v_scale, int seq, int kvh,
                                              int hs, int part) {
  store_partial(p, finish_partial(st, v_scale), seq, kvh, hs, part);
}

// LDS floats per stashed partition of one wavefront: 8 f4 and (max, sum)
// for each of the 4 kg lanes of up to `heads` head columns.
__host__ __device__ constexpr int stash_floats(int heads) { return heads * 4 * (8 * 4 + 2); }

// The sink of a wavefront streaming several partitions.  A finished
// partition's partials either go to the workspace at once or, with a
// stash, wait in LDS until the wavefront's last loads are done: a store
// counts on the same in-order counter as the loads, so every later wait
// for a K/V load would also wait for the store's acknowledgement, which a
// read-saturated HBM returns late (64 x 512-token FP8 partitions: 217 us
// with the stores in the stream, 189 us without three of the four).
struct PartialSink {
  static constexpr bool kActive = true;
  const Params& p;
  int part_tokens, seq, kvh, hs;
  float v_scale;
  float* stash;      // this wavefront's slots, or nullptr
  int first;         // the wavefront's first partition (slot 0)
  int heads;         // head columns a slot holds: min(group - 16 hs, 16)
  __device__ void operator()(const State& st, int part) const {
    const Partial r = finish_partial(st, v_scale);
    if (stash == nullptr) {
      store_partial(p, r, seq, kvh, hs, part);
      return;
    }
    const int lane = threadIdx.x % kWave;
    const int m = lane & 15, kg = lane >> 4;
    if (m >= heads) return;
    const int c = 4 * m + kg, nc = 4 * heads;   // compact lane index over the valid heads
    float* slot = stash + (part - first) * stash_floats(heads);
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) *reinterpret_cast<f4*>(slot + 4 * (dt * nc + c)) = r.o[dt];
    slot[32 * nc + c] = r.m;
    slot[33 * nc + c] = r.l;
  }
  // The stashed partitions [first, first + n) to the workspace.
  __device__ void drain(int n) const {
    const int lane = threadIdx.x % kWave;
    const int m = lane & 15, kg = lane >> 4;
    if (stash == nullptr || m >= heads) return;
    const int c = 4 * m + kg, nc = 4 * heads;
    for (int k = 0; k < n; ++k) {
      const float* slot = stash + k * stash_floats(heads);
      Partial r;
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) r.o[dt] = *reinterpret_cast<const f4*>(slot + 4 * (dt * nc + c));
      r.m = slot[32 * nc + c];
      r.l = slot[33 * nc + c];
      store_partial(p, r, seq, kvh, hs, first + k);
    }
  }
};

// Split-K with whole partitions per wavefront: wavefront w runs partitions
// [first, first + parts_per_wave) of (sequence, kv head, 16-head slice)
// alone, as one stream (q loaded once, the next iteration's loads in flight
// across partition boundaries), writing each partition's partials when it
// ends (or, with a stash, after its last loads); no merge inside the
// workgroup.  For short partitions (FP8 at 512 tokens: 8 iterations of 64
// tokens) this pays the q prologue, the first loads' latency and the tail
// once per run of partitions, where splitting each partition over a
// workgroup pays them per quarter partition.
template <Kind KV, Kind QK, int BS>
__device__ __forceinline__ void partitions_per_wave(const Params& p, int seq, int kvh, int hs, int first,
                                                    float* stash) {
  constexpr int TPI = tokens_per_iteration<KV>();
  if (first >= p.num_partitions) return;
  const int L = p.seq_lens[seq];
  const int t0 = first * p.partition_tokens;
  if (t0 >= L) return;                       // merged only up to ceil(L / partition_tokens)
  const int last = min(first + p.parts_per_wave, p.num_partitions);
  const int t1 = min(last * p.partition_tokens, L);
  const float vs = KV == Kind::FP8 ? p.v_scale : 1.f;
  const PartialSink sink{p, p.partition_tokens, seq, kvh, hs, vs, stash, first, min(p.group - hs * kHeads, kHeads)};
  const State st = run_wave<KV, QK, BS>(p, seq, kvh, hs, t0, t1, TPI, sink);
  const int part_last = (t1 - 1) / p.partition_tokens;
  write_partial(p, st, vs, seq, kvh, hs, part_last);
  sink.drain(part_last - first);
}

// One workgroup of NW wavefronts over (sequence, kv head, 16-head slice,
// partition): the wavefronts stride over the partition's iterations and
// are merged in LDS (smem: NW x 16 x 128 + 2 x NW x 16 floats).  LATE:
// the range is [t0, min(t1, len)), len applied after the wavefronts' first
// loads; a partition past the end (len <= t0, the same for the whole
// workgroup) returns then, writing nothing.
template <Kind KV, Kind QK, Kind PO, int NW, bool FINAL, int BS = 16, bool LATE = false, int ITERS = 0>
__device__ __forceinline__ void decode_workgroup(const Params& p, int seq, int kvh, int hs, int part, int t0,
                                                 int t1, float* s_acc, float* s_m, float* s_l,
                                                 int len = 0x7fffffff) {
  constexpr int TPI = tokens_per_iteration<KV>();
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int lane = tid % kWave;
  const State st = run_wave<KV, QK, BS, NoFlush, ITERS>(p, seq, kvh, hs, t0 + wave * TPI, t1, NW * TPI, NoFlush(), len);
  if (LATE && len <= t0) return;
  st.store(KV == Kind::FP8 ? p.v_scale : 1.f, lane & 15, lane >> 4, s_acc + wave * kHeads * kHead,
           s_m + wave * kHeads, s_l + wave * kHeads);
  __syncthreads();
  combine_waves<QK, PO, kHead, FINAL, kHeads, NW>(p, NW, s_m, s_l, s_acc, seq, kvh, hs, part, tid, NW * kWave);
}

}  // namespace mw
}  // namespace tl
