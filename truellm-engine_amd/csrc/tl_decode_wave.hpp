// tl_decode_wave.hpp -- the per-wavefront decode of 2-byte (f16 / bf16) KV
// shared by the paged decode kernel and the fp16 residual window of the
// KIVI decode kernel.
//
// A wavefront runs its own online softmax over the 32-token iterations it
// owns (tokens first_it, first_it + step, ... below t1), so the callers'
// main loops have no workgroup barrier; the loads of the next iteration are
// issued while the current one computes.  Lane bits 2-3 pick the token
// group tg (one 8-token run of a block row), bits 0-1 and 4-5 the head dims
// dl.  Both contractions use the packed dot-product instruction
// (v_dot2_f32_bf16 / v_dot2_f32_f16):
//   q.k over head-dim pairs (2m, 2m+1): two 16-byte loads per pair and one
//       v_perm_b32 per token build the (K[2m][t], K[2m+1][t]) operand;
//   p.v over token pairs (t, t+1), adjacent in the [d][bs] layout, with the
//       weights packed to the KV type.
// The q.k partials are finished by a transpose-reduce over the 16 lanes of
// a token group (v_permlane32/16_swap for bits 5 and 4, DPP for bits 1 and
// 0); each lane then owns head lane>>4, tokens 2*(lane&3) and +1, and the
// per-head softmax reductions run inside one 16-lane row on DPP.
#pragma once

#include "tl_device.hpp"

#include <math.h>

namespace tl {

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kWaveHeads = 4;   // q heads served per wavefront
// words of one weight exchange area ([4][kWaveHeads][4]); bf16 keeps the
// weights' low parts in a second area right after it
constexpr int kLoWords = 4 * kWaveHeads * 4;

struct Params {
  void* out;
  const void* q;
  const char* k_cache;
  const char* v_cache;
  const int32_t* block_tables;
  const int32_t* seq_lens;
  float* part_m;
  float* part_l;
  void* part_o;
  int num_heads, num_kv_heads, max_blocks_per_seq, num_blocks;
  int num_partitions, partition_tokens;
  int parts_per_wave;   // split-K with a wavefront per partition run: partitions each wavefront streams
  int stash_floats = 0; // LDS floats per wavefront for its finished partitions (0: written at once)
  int group, head_slices, gqa_map;
  float qk_scale;  // softmax scale * k dequant scale * log2(e)
  float v_scale;
  int block_size = 0;   // pool block size, read by kernels built for any block size
};

// The work item of a decode workgroup: returns the index of its (sequence,
// kv head, head slice) and sets its partition.  The partition is the
// slowest index of the grid: the GPU deals workgroups round-robin to its 8
// XCDs in dispatch order, and this way every XCD gets the same mix of
// partitions (with the partition fastest, 4 partitions put partition 0 of
// every sequence, the one that always has work, on XCDs 0 and 4 only).
__device__ __forceinline__ int grid_item(const Params& p, int& part) {
  const int items = (int)gridDim.x / p.num_partitions;
  part = (int)blockIdx.x / items;
  return (int)blockIdx.x - part * items;
}

__device__ __forceinline__ int head_of(const Params& p, int kvh, int gi) {
  return p.gqa_map ? kvh * p.group + gi : kvh + gi * p.num_kv_heads;
}

template <Kind KV> struct Dot2;
template <> struct Dot2<Kind::BF16> {
  typedef __bf16 v2 __attribute__((ext_vector_type(2)));
  __device__ __forceinline__ static float dot(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(v2, a), __builtin_bit_cast(v2, b), c, false);
  }
  __device__ __forceinline__ static uint32_t pack(float x, float y) {
    const v2 p = {(__bf16)x, (__bf16)y};
    return __builtin_bit_cast(uint32_t, p);
  }
};
template <> struct Dot2<Kind::F16> {
  typedef _Float16 v2 __attribute__((ext_vector_type(2)));
  __device__ __forceinline__ static float dot(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(v2, a), __builtin_bit_cast(v2, b), c, false);
  }
  __device__ __forceinline__ static uint32_t pack(float x, float y) {
    const v2 p = {(_Float16)x, (_Float16)y};
    return __builtin_bit_cast(uint32_t, p);
  }
};

// Physical block holding token blk_tok (a block start) of a sequence, or -1
// for a hole, a block past the partition end t1 or an entry outside the pool.
template <int BS>
__device__ __forceinline__ int table_entry_bs(const Params& p, const int32_t* table, int blk_tok, int t1) {
  const int lb = blk_tok / BS;
  int ph = -1;
  if (blk_tok < t1 && lb < p.max_blocks_per_seq) ph = table[lb];
  return (ph >= p.num_blocks) ? -1 : ph;
}

// K of head-dim pairs (2m, 2m+1), m = dl + 16 j: rows 2m and 2m+1 of the
// lane's 8-token run th (the 16-byte chunk th of a row) of one block ([D][BS]
// layout, cpr = BS / 8 chunks per row).
template <int KP>
__device__ __forceinline__ void load_k_pairs(u32x4 (&kr)[KP][2], const char* blk, int dl, int th, int cpr) {
#pragma unroll
  for (int j = 0; j < KP; ++j) {
    const int c = 2 * (dl + 16 * j) * cpr + th;
    kr[j][0] = load16_stream(blk + c * 16);
    kr[j][1] = load16_stream(blk + (c + cpr) * 16);
  }
}

// V rows d = 16 j + dl of the lane's 8-token run th of one block.
template <int VD>
__device__ __forceinline__ void load_v_rows(u32x4 (&vr)[VD], const char* blk, int dl, int th, int cpr) {
#pragma unroll
  for (int j = 0; j < VD; ++j) vr[j] = load16_stream(blk + ((16 * j + dl) * cpr + th) * 16);
}

// The key rotation hook of decode2_wave: called with the lane's K rows as
// loaded (kr[j][r]: head-dim row 2 m + r, m = dl + 16 j, of its 8 tokens
// tok0 .. tok0 + 7) before they enter q.k.  NoKeyRotation leaves them.
struct NoKeyRotation {
  static constexpr bool kActive = false;
  template <int KP>
  __device__ void operator()(u32x4 (&)[KP][2], int, int) const {}
};

// Runs one wavefront over its iterations and leaves its state in LDS:
// s_acc_w [4][HEAD] unnormalised outputs, s_m_w [4] running max (log2 units),
// s_l_w [4] sums.  s_p_w is the wavefront's weight exchange area: [4][4][4]
// words, twice that for bf16 (the weights' high and low bf16 parts).
// An iteration is 32 consecutive tokens; token group tg is the 8-token run
// it + 8 tg, which lies in one block for every block size (a power of two
// >= 8): in block (it + 8 tg) / BS, chunk ((it + 8 tg) % BS) / 8 of its
// rows.  BS is the block size, or 0 for p.block_size read at run time.
template <Kind KV, int HEAD, int BS, class Rot = NoKeyRotation>
__device__ __forceinline__ void decode2_wave(const Params& p, int seq, int kvh, int hs, int first_it,
                                             int t1, int step, uint32_t* s_p_w, float* s_acc_w,
                                             float* s_m_w, float* s_l_w, const Rot& rot = Rot()) {
  constexpr int GT = kWaveHeads;
  constexpr int KP = HEAD / 32;           // head-dim pairs per lane (q.k)
  constexpr int VD = HEAD / 16;           // head dims per lane (p.v)
  // a block holds a whole number of iterations' runs: the lane's chunk in
  // its block row is the same on every iteration
  constexpr bool kFixedChunk = BS > 0 && BS <= 32;
  static_assert(BS == 0 || (BS >= 8 && (BS & (BS - 1)) == 0), "block size: a power of two >= 8");
  const int bs = BS > 0 ? BS : p.block_size;
  const int lbs = BS > 0 ? __builtin_ctz(BS) : __builtin_ctz((unsigned)p.block_size);
  const int cpr = bs >> 3;                // 16-byte chunks per head-dim row of a block
  const int64_t block_bytes = (int64_t)HEAD * bs * 2;
  using D2 = Dot2<KV>;

  const int lane = threadIdx.x % kWave;
  const int tg = (lane >> 2) & 3, dl = (lane & 3) | ((lane >> 4) << 2);
  const int g_lane = lane >> 4, tp = lane & 3;
  // the lane's run chunk in its block row for the iteration at token i
  auto run_chunk = [&](int i) {
    if constexpr (kFixedChunk) return tg % (BS / 8);
    else return ((i + 8 * tg) & (bs - 1)) >> 3;
  };
  // physical block of the lane's run of the iteration at token i, or -1
  // for a hole, a run at or past t1 or an entry outside the pool
  auto run_block = [&](const int32_t* table, int i) {
    if constexpr (kFixedChunk) return table_entry_bs<BS>(p, table, i + (tg / (BS / 8)) * BS, t1);
    const int tok = i + 8 * tg, lb = tok >> lbs;
    int ph = -1;
    if (tok < t1 && lb < p.max_blocks_per_seq) ph = table[lb];
    return (ph >= p.num_blocks) ? -1 : ph;
  };

  // q as (dim 2m, 2m+1) pairs, m = dl + 16 j, straight from [S, H, D]
  uint32_t qp[GT][KP];
#pragma unroll
  for (int g = 0; g < GT; ++g) {
    const int gi = hs * GT + g;
    const uint32_t* qrow = (const uint32_t*)p.q +
        ((int64_t)seq * p.num_heads + (gi < p.group ? head_of(p, kvh, gi) : 0)) * (HEAD / 2);
#pragma unroll
    for (int j = 0; j < KP; ++j) qp[g][j] = (gi < p.group) ? qrow[dl + 16 * j] : 0u;
  }

  float m_run[GT], acc[GT][VD], l_lane = 0.f;
#pragma unroll
  for (int g = 0; g < GT; ++g) {
    m_run[g] = -INFINITY;
#pragma unroll
    for (int j = 0; j < VD; ++j) acc[g][j] = 0.f;
  }

  const int32_t* table = p.block_tables + (int64_t)seq * p.max_blocks_per_seq;
  const int64_t pool_stride = (int64_t)p.num_kv_heads * block_bytes;
  const char* kbase0 = p.k_cache + (int64_t)kvh * block_bytes;
  const char* vbase0 = p.v_cache + (int64_t)kvh * block_bytes;

  // Pipeline: the K loads of iteration i+1 are issued as soon as the scores
  // of iteration i are formed, the V loads of i+1 once p.v of i is done, and
  // block-table entries are read two iterations ahead, so each wavefront
  // keeps one iteration of K/V in flight while it computes.  Holes load
  // block 0 and are masked.
  int it = first_it;
  int ph_cur = run_block(table, it);
  int ph_next = run_block(table, it + step);
  u32x4 kr[KP][2], vr[VD];
  if (it < t1) {
    load_k_pairs<KP>(kr, kbase0 + (int64_t)max(ph_cur, 0) * pool_stride, dl, run_chunk(it), cpr);
    load_v_rows<VD>(vr, vbase0 + (int64_t)max(ph_cur, 0) * pool_stride, dl, run_chunk(it), cpr);
  }

#pragma unroll 1
  for (; it < t1; it += step) {
    const int ph_nn = run_block(table, it + 2 * step);
    const bool has_next = it + step < t1;
    const int tok0 = it + 8 * tg;                        // first token of this lane's run
    const int th_next = run_chunk(it + step);
    if constexpr (Rot::kActive) rot(kr, tok0, dl);

    // ---- q.k partials over this lane's dim pairs, 8 tokens x 4 heads ----
    float s[GT * 8];
#pragma unroll
    for (int j = 0; j < KP; ++j)
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const uint32_t a = word(kr[j][0], w), b = word(kr[j][1], w);
        const uint32_t k_lo = __builtin_amdgcn_perm(b, a, 0x05040100u);  // token 2w
        const uint32_t k_hi = __builtin_amdgcn_perm(b, a, 0x07060302u);  // token 2w+1
#pragma unroll
        for (int g = 0; g < GT; ++g) {
          const int i0 = g * 8 + 2 * w;
          s[i0] = D2::dot(k_lo, qp[g][j], j == 0 ? 0.f : s[i0]);
          s[i0 + 1] = D2::dot(k_hi, qp[g][j], j == 0 ? 0.f : s[i0 + 1]);
        }
      }
    if (has_next)
      load_k_pairs<KP>(kr, kbase0 + (int64_t)max(ph_next, 0) * pool_stride, dl, th_next, cpr);
    transpose_reduce_5410<GT * 8>(s, lane);             // -> (head g_lane, tokens 2tp, 2tp+1)

    const int tok = tok0 + 2 * tp;
    const bool ok0 = ph_cur >= 0 && tok < t1, ok1 = ph_cur >= 0 && tok + 1 < t1;
    const float sc0 = ok0 ? s[0] * p.qk_scale : -INFINITY;
    const float sc1 = ok1 ? s[1] * p.qk_scale : -INFINITY;

    // ---- online softmax, one running max per head for the wavefront ----
    const float mx = row_max(fmaxf(sc0, sc1));
    float m_lane = 0.f;
#pragma unroll
    for (int g = 0; g < GT; ++g) {
      const float mg = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, mx), 16 * g));
      const float m_new = fmaxf(m_run[g], mg);
      if (m_new != m_run[g]) {
        const float alpha = (m_run[g] == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(m_run[g] - m_new);
#pragma unroll
        for (int j = 0; j < VD; ++j) acc[g][j] *= alpha;
        if (g == g_lane) l_lane *= alpha;
        m_run[g] = m_new;
      }
      if (g == g_lane) m_lane = m_run[g];
    }
    const float p0 = ok0 ? __builtin_amdgcn_exp2f(sc0 - m_lane) : 0.f;
    const float p1 = ok1 ? __builtin_amdgcn_exp2f(sc1 - m_lane) : 0.f;
    l_lane += p0 + p1;
    const uint32_t p01 = D2::pack(p0, p1);
    s_p_w[(tg * GT + g_lane) * 4 + tp] = p01;
    if constexpr (KV == Kind::BF16) {
      // bf16 weights carry 8 mantissa bits (a short or peaked softmax would
      // miss 2e-3 by up to 2^-9 max|v|): the rest goes in a second bf16
      const float h0 = __builtin_bit_cast(float, p01 << 16), h1 = __builtin_bit_cast(float, p01 & 0xffff0000u);
      s_p_w[kLoWords + (tg * GT + g_lane) * 4 + tp] = D2::pack(p0 - h0, p1 - h1);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    // ---- holes, and slots past the end of a partial block, may hold anything ----
    if (ph_cur < 0 || tok0 + 8 > t1) {
#pragma unroll
      for (int j = 0; j < VD; ++j) {
        uint32_t w4[4] = {vr[j].x, vr[j].y, vr[j].z, vr[j].w};
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const int t = tok0 + 2 * w;
          if (ph_cur < 0 || t >= t1) w4[w] = 0u;
          else if (t + 1 >= t1) w4[w] &= 0xffffu;
        }
        vr[j] = u32x4{w4[0], w4[1], w4[2], w4[3]};
      }
    }

    // ---- p.v over token pairs ----
    u32x4 pp[GT], pl[GT];
#pragma unroll
    for (int g = 0; g < GT; ++g) {
      pp[g] = *reinterpret_cast<const u32x4*>(&s_p_w[(tg * GT + g) * 4]);
      if constexpr (KV == Kind::BF16) pl[g] = *reinterpret_cast<const u32x4*>(&s_p_w[kLoWords + (tg * GT + g) * 4]);
    }
#pragma unroll
    for (int j = 0; j < VD; ++j)
#pragma unroll
      for (int g = 0; g < GT; ++g) {
        float a = acc[g][j];
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          a = D2::dot(word(pp[g], w), word(vr[j], w), a);
          if constexpr (KV == Kind::BF16) a = D2::dot(word(pl[g], w), word(vr[j], w), a);
        }
        acc[g][j] = a;
      }
    if (has_next)
      load_v_rows<VD>(vr, vbase0 + (int64_t)max(ph_next, 0) * pool_stride, dl, th_next, cpr);
    ph_cur = ph_next;
    ph_next = ph_nn;
  }

  // ---- wavefront totals: sums per head, acc reduced over token groups ----
  const float l_tot = row_sum(l_lane);
  float* accf = &acc[0][0];
  transpose_reduce<GT * VD, 8, 4>(accf, lane);         // -> head tg, dims 16 j + dl
#pragma unroll
  for (int j = 0; j < VD; ++j) s_acc_w[tg * HEAD + 16 * j + dl] = accf[j];
  if (lane == 0) {
#pragma unroll
    for (int g = 0; g < GT; ++g) s_m_w[g] = m_run[g];
  }
  if ((lane & 15) == 0) s_l_w[g_lane] = l_tot;
}

// Merges the nw wavefront states (s_m [nw][GT], s_l [nw][GT], s_acc
// [nw][GT][HEAD], GT q heads per wavefront; nw <= MAXW) and writes the
// workgroup's result: the normalised output (FINAL) or the partition's
// (max, sum, normalised partial) for the log-sum-exp merge.
template <Kind QK, Kind PO, int HEAD, bool FINAL, int GT = kWaveHeads, int MAXW = 8>
__device__ __forceinline__ void combine_waves(const Params& p, int nw, const float* s_m,
                                              const float* s_l, const float* s_acc, int seq, int kvh,
                                              int hs, int part, int tid, int nthreads) {
  for (int i = tid; i < GT * HEAD; i += nthreads) {
    const int g = i / HEAD, d = i % HEAD, gi = hs * GT + g;
    if (gi >= p.group) continue;
    // every state's reads at once (rows clamped to nw - 1, the extra ones
    // unused); a loop over the run-time count waited for one LDS round
    // trip per state and value
    float mw[MAXW], lw[MAXW], aw[MAXW];
#pragma unroll
    for (int w = 0; w < MAXW; ++w) {
      const int r = min(w, nw - 1);
      mw[w] = s_m[r * GT + g];
      lw[w] = s_l[r * GT + g];
      aw[w] = s_acc[(r * GT + g) * HEAD + d];
    }
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < MAXW; ++w) M = fmaxf(M, mw[w]);
    float num = 0.f, den = 0.f;
    if (M != -INFINITY) {
#pragma unroll
      for (int w = 0; w < MAXW; ++w) {
        if (w < nw) {
          const float f = (mw[w] == -INFINITY) ? 0.f : exp2f(mw[w] - M);
          num += f * aw[w];
          den += f * lw[w];
        }
      }
    }
    const float val = (den > 0.f) ? num / den : 0.f;
    const int head = head_of(p, kvh, gi);
    if constexpr (FINAL) {
      store_scalar<QK>(p.out, ((int64_t)seq * p.num_heads + head) * HEAD + d, val);
    } else {
      const int64_t pi = ((int64_t)seq * p.num_heads + head) * p.num_partitions + part;
      store_scalar<PO>(p.part_o, pi * HEAD + d, val);
      if (d == 0) {
        p.part_m[pi] = (den > 0.f) ? M * (1.0f / kLog2e) : -INFINITY;
        p.part_l[pi] = den;
      }
    }
  }
}

}  // namespace tl
