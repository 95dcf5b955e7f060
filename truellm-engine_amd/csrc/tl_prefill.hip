// tl_prefill.hip -- chunked-prefill paged attention on MFMA (gfx950).
//
// One launch serves a mixed batch: sequences with q_len > 1 are prefill
// chunks (causal: query i of a chunk sits at position L - q_len + i and sees
// keys 0 .. that position, its own chunk included, all read from the paged
// pool), sequences with q_len == 1 are decode rows.
//
// Prefill work item: one workgroup per (sequence, kv head, tile of NW * 32
// rows), a row being one (query, q head of the GQA group) pair, so every K/V
// block fetched serves all q heads of the group.  Per 64-key iteration:
//   * the workgroup copies the keys' K (transposed to [key][channel], rows
//     padded to 136 halves) and V ([channel][key slot], the key order of the
//     PV operand, rows padded to 72 halves) into one of three LDS stages,
//     two iterations ahead; each wavefront copies two 8-key runs for half
//     of the channels, laid out so its LDS writes and the MFMA operand reads
//     are free of bank conflicts;
//   * each wavefront (32 rows) forms two 32-key tiles of S^T = K Q^T with
//     v_mfma_f32_32x32x16_{bf16,f16}: A = K (rows: keys, k: channels) read
//     from LDS, B = Q^T held in registers for the whole launch.  Lane l then
//     holds 16 keys per tile of row l % 32, so the row max needs one
//     permlane32 swap;
//   * online softmax with lazy rescaling: the running max is only raised
//     when a row's new max exceeds it by more than 8 (log2 units), so the
//     weights stay below 2^8 and the O accumulators are rescaled rarely;
//   * O += P V on the same MFMA: the weights leave the S^T accumulator of
//     tile t as keys {32 t + 16 s + 4 g + i, 32 t + 16 s + 8 + 4 g + i} for
//     lane group g, which is used as the k order of step s; V is read from
//     LDS in that order;
//   * the q.k MFMAs of the next iteration share a basic block with the
//     exponentials and P V of the current one (software pipeline).
// Decode rows run the decode wavefronts (tl_mfma_wave.hpp for block_size 16,
// tl_decode_wave.hpp otherwise), one workgroup per (sequence, kv head, head
// slice), as a second kernel of the same call on the same stream (one
// kernel for both would be sized by the decode path's registers on top of
// the prefill path's).
//
// Nearest reference analogues: the per-token prefill of cuda_engine.cpp:842-860
// and the dense attention of megakernel.cu:267-351; the reference has no
// chunked prefill over the paged pool.
#include "tl_decode_wave.hpp"
#include "tl_device.hpp"
#include "tl_internal.hpp"
#include "tl_mfma_wave.hpp"

namespace tl {

namespace {

typedef float f16v __attribute__((ext_vector_type(16)));
typedef unsigned u4v __attribute__((ext_vector_type(4)));

constexpr int kPfHead = 128;
constexpr int kPfRows = 32;          // rows per wavefront
constexpr int kPfKeys = 64;          // keys per iteration
constexpr int KT = kPfKeys / 32;     // 32-key S tiles per iteration
constexpr int kKtStride = 136;       // halves per key row of the transposed K stage
constexpr int kVStride = 72;         // halves per channel row of the V stage (64 keys + pad)

// Slot of key k (of an iteration's 64) in a V stage row: the middle two
// 4-key quarters of every 16 keys are swapped, so the 8 keys a PV MFMA step
// takes from lane group g (16 s + 4 g + i and 16 s + 8 + 4 g + i) sit
// together at 16 s + 8 g and are one 16-byte read.  With 144-byte rows the
// 16 lanes of one ds_read_b128 cycle hit 16 distinct 4-bank groups.
__device__ __forceinline__ int v_slot(int k) {
  const int q = (k >> 2) & 3;
  return (k & ~15) + 4 * (((q & 1) << 1) | (q >> 1)) + (k & 3);
}
constexpr float kLazyRescale = 8.f;  // log2 units
// LDS stages: iteration i is staged in stage i % 3 two iterations ahead, so
// its K is already visible during iteration i - 1
constexpr int kStages = 3;

template <Kind KV> struct Mfma32;
// bf16 keeps 8 mantissa bits: the weights go to the PV product as two bf16
// terms (hi = bf16(p), lo = bf16(p - hi)), fp16 weights (11 bits) as one.
template <> struct Mfma32<Kind::BF16> {
  static constexpr bool kSplitP = true;
  typedef __bf16 v8 __attribute__((ext_vector_type(8)));
  typedef __bf16 v2 __attribute__((ext_vector_type(2)));
  __device__ __forceinline__ static float hi(float x) { return (float)(__bf16)x; }
  __device__ __forceinline__ static f16v mma(const u32x4& a, const u32x4& b, const f16v& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8, a), __builtin_bit_cast(v8, b), c,
                                                   0, 0, 0);
  }
  __device__ __forceinline__ static uint32_t pack(float x, float y) {
    const v2 v = {(__bf16)x, (__bf16)y};
    return __builtin_bit_cast(uint32_t, v);
  }
};
template <> struct Mfma32<Kind::F16> {
  static constexpr bool kSplitP = false;
  typedef _Float16 v8 __attribute__((ext_vector_type(8)));
  typedef _Float16 v2 __attribute__((ext_vector_type(2)));
  __device__ __forceinline__ static float hi(float x) { return (float)(_Float16)x; }
  __device__ __forceinline__ static f16v mma(const u32x4& a, const u32x4& b, const f16v& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8, a), __builtin_bit_cast(v8, b), c,
                                                  0, 0, 0);
  }
  __device__ __forceinline__ static uint32_t pack(float x, float y) {
    const v2 v = {(_Float16)x, (_Float16)y};
    return __builtin_bit_cast(uint32_t, v);
  }
};

struct PrefillParams {
  Params base;                 // q, out, pools, tables, seq_lens, heads, group, qk_scale
  const int32_t* cu_q_lens;    // [num_seqs + 1]
  int num_seqs, row_tiles;
  int pf_seqs;                 // sequences [0, pf_seqs) may be prefill rows
  int dec_first;               // sequences [dec_first, num_seqs) may be decode rows
};

template <int NW, int BS>
struct PrefillSmem {
  struct {
    uint16_t kt[kStages][kPfKeys * kKtStride];    // [key][channel] (+8 pad)
    uint16_t v[kStages][kPfHead * kVStride];      // [channel][v_slot(key)] (+8 pad)
    float row[NW][kPfRows];                       // per-row exchange (alpha, l)
  } pf;
};

// A block-table row read through the constant address space: the table is
// not written during the kernel, and with a wave-uniform index the reads
// are scalar loads, which are waited for on their own counter instead of
// behind every K/V load in flight.
typedef const __attribute__((address_space(4))) int32_t* TableRow;

// Physical block of block index lb of a table row, or -1.
__device__ __forceinline__ int block_of(const Params& p, TableRow table, int lb) {
  if (lb >= p.max_blocks_per_seq) return -1;
  const int b = table[lb];
  return (b < 0 || b >= p.num_blocks) ? -1 : b;
}

template <Kind KV, int BS, int NW>
__global__ __launch_bounds__(NW * kWave) void prefill_kernel(PrefillParams pp) {
  static_assert(BS == 16 || BS == 32, "block size");
  constexpr int BPI = kPfKeys / BS;                    // pool blocks per iteration
  using M = Mfma32<KV>;
  __shared__ __attribute__((aligned(16))) PrefillSmem<NW, BS> sm;

  const Params& p = pp.base;
  const int tid = threadIdx.x, lane = tid % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int g = lane >> 5, c32 = lane & 31;

  int b = blockIdx.x;
  const int items = pp.pf_seqs * p.num_kv_heads;
  const int tile = pp.row_tiles - 1 - b / items;       // longest (latest) tiles first
  b %= items;
  const int seq = b / p.num_kv_heads, kvh = b % p.num_kv_heads;
  const int q0 = pp.cu_q_lens[seq], ql = pp.cu_q_lens[seq + 1] - q0;
  const int L = p.seq_lens[seq];
  if (ql <= 0) return;

  if (ql == 1) return;                                  // decode rows: prefill_decode_kernel

  // ---- prefill tile ----
  const int rows = ql * p.group;
  const int row0 = tile * NW * kPfRows;
  if (row0 >= rows) return;
  const int wrow0 = row0 + wave * kPfRows;
  const int my_row = wrow0 + c32;
  const bool row_ok = my_row < rows;
  const int qi = row_ok ? my_row / p.group : 0, gi = row_ok ? my_row % p.group : 0;
  const int pos = row_ok ? L - ql + qi : -1;           // keys 0 .. pos
  const int last_row = min(rows, row0 + NW * kPfRows) - 1;
  const int kend = max(0, L - ql + last_row / p.group + 1);           // keys of the workgroup
  const int n_it = (kend + kPfKeys - 1) / kPfKeys;

  // B operand of S^T: row my_row, channels 16 ks + 8 g .. +7 (zero for padding rows)
  u32x4 qb[8];
  {
    const uint16_t* qrow = (const uint16_t*)p.q +
        ((int64_t)(q0 + qi) * p.num_heads + head_of(p, kvh, gi)) * kPfHead + 8 * g;
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) qb[ks] = row_ok ? load16(qrow + 16 * ks) : u32x4{0u, 0u, 0u, 0u};
    // q is waited for here, on every path: otherwise the loop's first use
    // of it waits for every load in flight, the K/V loads of later
    // iterations included
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) asm volatile("" ::"v"(qb[ks].x), "v"(qb[ks].y), "v"(qb[ks].z), "v"(qb[ks].w));
  }

  const TableRow table = (TableRow)(p.block_tables + (int64_t)seq * p.max_blocks_per_seq);
  const int64_t head_stride = (int64_t)kPfHead * BS;                  // elements per (block, kv head)
  const uint16_t* kpool = (const uint16_t*)p.k_cache;
  const uint16_t* vpool = (const uint16_t*)p.v_cache;

  // Staging: an iteration's 64 keys are 8 runs of 8 (run r: keys 8 r .. 8 r
  // + 7 of the iteration).  Wavefront w copies runs (w >> 1) and (w >> 1) + 4
  // for half of the channels.  K: channel 2 lane + (w & 1), so each
  // transposed 2-byte LDS write of a wavefront hits 64 consecutive dwords;
  // V: channel lane + 64 (w & 1).  Block ids are wave-uniform (scalar table
  // reads).
  constexpr int RPW = 2 * (kPfKeys / 8) / NW;          // runs per wavefront
  static_assert(RPW * NW == 2 * (kPfKeys / 8), "runs x channel halves per wavefront");
  const int k_ch = 2 * lane + (wave & 1), v_ch = lane + 64 * (wave & 1);
  // nv: keys of the run that exist (the rest of its V is zeroed when staged,
  // so that the loads are waited for only there)
  struct Fetched { u32x4 k[RPW], v[RPW]; int nv[RPW]; };
  auto run_key = [&](int j) { return 8 * ((wave >> 1) + (NW / 2) * j); };   // first key of run j
  auto fetch = [&](int it, Fetched& f) {
#pragma unroll
    for (int j = 0; j < RPW; ++j) {
      const int kb = run_key(j);
      const int key0 = it * kPfKeys + kb;
      // wave-uniform (the descriptor is built in scalar registers)
      const int pb = __builtin_amdgcn_readfirstlane(key0 < kend ? block_of(p, table, it * BPI + kb / BS) : -1);
      f.nv[j] = pb >= 0 ? min(max(L - key0, 0), 8) : 0;
      // unconditional loads (a missing block has an empty range and reads
      // zeros): no branch, so nothing waits for them before the staging
      const int64_t row = pb >= 0 ? ((int64_t)pb * p.num_kv_heads + kvh) * head_stride : 0;
      const unsigned bytes = pb >= 0 ? unsigned(head_stride * 2) : 0u;
      f.k[j] = buffer_load16(buffer_rsrc(kpool + row, bytes), unsigned(2 * (k_ch * BS + kb % BS)));
      f.v[j] = buffer_load16(buffer_rsrc(vpool + row, bytes), unsigned(2 * (v_ch * BS + kb % BS)));
    }
  };
  auto stage = [&](int st, const Fetched& f) {
#pragma unroll
    for (int j = 0; j < RPW; ++j) {
      const int kb = run_key(j);
      uint16_t* kt = &sm.pf.kt[st][kb * kKtStride + k_ch];
      const u4v kv = __builtin_bit_cast(u4v, f.k[j]);
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        kt[(2 * w) * kKtStride] = (uint16_t)(kv[w] & 0xFFFFu);
        kt[(2 * w + 1) * kKtStride] = (uint16_t)(kv[w] >> 16);
      }
      // V slots at or past the sequence end may hold anything (NaN codes
      // too, and a zero weight times NaN is NaN): zero them
      u4v v = __builtin_bit_cast(u4v, f.v[j]);
      const int nv = f.nv[j];
      if (nv < 8) {
#pragma unroll
        for (int w = 0; w < 4; ++w) v[w] = 2 * w >= nv ? 0u : (2 * w + 1 >= nv ? v[w] & 0xFFFFu : v[w]);
      }
      uint16_t* vrow = &sm.pf.v[st][v_ch * kVStride];
      *reinterpret_cast<uint2*>(vrow + v_slot(kb)) = uint2{v[0], v[1]};
      *reinterpret_cast<uint2*>(vrow + v_slot(kb + 4)) = uint2{v[2], v[3]};
    }
  };

  f16v o[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) o[c] = f16v{};
  float m_used = -INFINITY, l_part = 0.f;
  float* s_row = &sm.pf.row[wave][0];

  // Software pipeline.  Iteration it first masks its scores (computed
  // during it - 1) and decides the rescale; then one branch-free block
  // holds the q.k MFMAs of it + 1 (its K is staged two iterations ahead),
  // the exponentials and weight packing of it and its P V MFMAs, which the
  // compiler interleaves so the matrix cores and the VALU work at once.  A wavefront
  // past its last keys runs the block on masked scores (weights 0).  Keys
  // of an iteration entirely at or below the wavefront's first query
  // position, in blocks that exist, need no mask.  The scores stay unscaled
  // until the exponent (qk_scale > 0, so the max commutes with the scale).
  const int wmin_pos = L - ql + wrow0 / p.group;
  auto qk = [&](int it, f16v (&sa)[KT]) {
    const uint16_t* kst = sm.pf.kt[it % kStages];
#pragma unroll
    for (int t = 0; t < KT; ++t) {
      sa[t] = f16v{};
      const uint16_t* ktw = kst + (32 * t + c32) * kKtStride + 8 * g;
#pragma unroll
      for (int ks = 0; ks < 8; ++ks)
        sa[t] = M::mma(*reinterpret_cast<const u32x4*>(ktw + 16 * ks), qb[ks], sa[t]);
    }
  };
  // mask, row max and lazy rescale of iteration it; returns the exponent offset
  auto prepare = [&](int it, f16v (&sa)[KT]) {
    const int k0 = it * kPfKeys;
    bool blk_ok[BPI];
    bool all_ok = true;
#pragma unroll
    for (int bi = 0; bi < BPI; ++bi) {
      blk_ok[bi] = block_of(p, table, it * BPI + bi) >= 0;
      all_ok = all_ok && blk_ok[bi];
    }
    float mx = -INFINITY;
    if (all_ok && k0 + kPfKeys - 1 <= wmin_pos) {
#pragma unroll
      for (int t = 0; t < KT; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sa[t][r]);
    } else {
#pragma unroll
      for (int t = 0; t < KT; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int kk = 32 * t + 8 * (r >> 2) + 4 * g + (r & 3);
          const bool ok = k0 + kk <= pos && blk_ok[kk / BS];
          sa[t][r] = ok ? sa[t][r] : -INFINITY;
          mx = fmaxf(mx, sa[t][r]);
        }
    }
    {
      const auto sw = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, mx),
                                                       __builtin_bit_cast(unsigned, mx), false, false);
      mx = fmaxf(__builtin_bit_cast(float, (unsigned)sw[0]), __builtin_bit_cast(float, (unsigned)sw[1]));
    }
    mx *= p.qk_scale;
    const bool raise = mx > m_used + kLazyRescale || (m_used == -INFINITY && mx != -INFINITY);
    if (__builtin_amdgcn_ballot_w64(raise)) {
      const float m_new = raise ? mx : m_used;
      const float alpha = (m_new == m_used) ? 1.f : (m_used == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m_used - m_new));
      m_used = m_new;
      l_part *= alpha;
      if (g == 0) s_row[c32] = alpha;
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      // O rows of this lane: 8 j + 4 g + i
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float4 a4 = *reinterpret_cast<const float4*>(&s_row[8 * j + 4 * g]);
        const float a[4] = {a4.x, a4.y, a4.z, a4.w};
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int c = 0; c < 4; ++c) o[c][4 * j + i] *= a[i];
      }
      __builtin_amdgcn_wave_barrier();
    }
    return (m_used == -INFINITY) ? 0.f : m_used;
  };
  auto exp_pv = [&](int it, const f16v (&sa)[KT], float m_use) {
    const uint16_t* vst = sm.pf.v[it % kStages];
#pragma unroll
    for (int t = 0; t < KT; ++t) {
      float pw[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        pw[r] = __builtin_amdgcn_exp2f(__builtin_fmaf(sa[t][r], p.qk_scale, -m_use));
        l_part += pw[r];
      }
#pragma unroll
      for (int st2 = 0; st2 < 2; ++st2) {
        const int r0 = 8 * st2;
        const u32x4 pa = {M::pack(pw[r0 + 0], pw[r0 + 1]), M::pack(pw[r0 + 2], pw[r0 + 3]),
                          M::pack(pw[r0 + 4], pw[r0 + 5]), M::pack(pw[r0 + 6], pw[r0 + 7])};
        u32x4 pl = {0u, 0u, 0u, 0u};
        if constexpr (M::kSplitP) {
          float lo[8];
#pragma unroll
          for (int i = 0; i < 8; ++i) lo[i] = pw[r0 + i] - M::hi(pw[r0 + i]);
          pl = u32x4{M::pack(lo[0], lo[1]), M::pack(lo[2], lo[3]), M::pack(lo[4], lo[5]), M::pack(lo[6], lo[7])};
        }
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const int ch = 32 * c + c32;
          // slots 0-3: keys 32 t + 16 st2 + 4 g + i, slots 4-7: the same + 8
          const u32x4 vb = *reinterpret_cast<const u32x4*>(vst + ch * kVStride + 32 * t + 16 * st2 + 8 * g);
          o[c] = M::mma(pa, vb, o[c]);
          if constexpr (M::kSplitP) o[c] = M::mma(pl, vb, o[c]);
        }
      }
    }
  };

  // Fetches and stages run unconditionally: past the last iteration the
  // blocks are missing (empty ranges, zeros), and a stage that no
  // iteration reads takes them.  A conditional fetch would leave the loop's
  // waits for one stage's loads unable to tell how many newer loads are in
  // flight, and they would wait for all of them.
  Fetched fs0, fs1;
  f16v sa0[KT], sa1[KT];
  fetch(0, fs0);
  stage(0, fs0);
  fetch(1, fs1);
  stage(1, fs1);
  fetch(2, fs0);
  __syncthreads();
  qk(0, sa0);
  // f_stage holds it + 2 (staged at the end of it), f_free receives it + 3;
  // s_cur holds the scores of it, s_next receives those of it + 1
  auto iteration = [&](int it, Fetched& f_stage, Fetched& f_free, f16v (&s_cur)[KT], f16v (&s_next)[KT]) {
    fetch(it + 3, f_free);
    const float m_use = prepare(it, s_cur);
    qk(it + 1, s_next);
    exp_pv(it, s_cur, m_use);
    stage((it + 2) % kStages, f_stage);
    __syncthreads();
  };
#pragma unroll 1
  for (int it = 0; it < n_it; it += 2) {
    iteration(it, fs0, fs1, sa0, sa1);
    if (it + 1 >= n_it) break;
    iteration(it + 1, fs1, fs0, sa1, sa0);
  }

  // ---- normalise and store: lane holds rows 8 j + 4 g + i, channels 32 c + c32 ----
  {
    const auto sw = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, l_part),
                                                     __builtin_bit_cast(unsigned, l_part), false, false);
    const float l = __builtin_bit_cast(float, (unsigned)sw[0]) + __builtin_bit_cast(float, (unsigned)sw[1]);
    if (g == 0) s_row[c32] = l;
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
  for (int j = 0; j < 4; ++j) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int rl = 8 * j + 4 * g + i, row = wrow0 + rl;
      if (row >= rows) continue;
      const float l = s_row[rl];
      const float inv = l > 0.f ? 1.f / l : 0.f;
      const int qr = row / p.group, gr = row % p.group;
      const int64_t base = ((int64_t)(q0 + qr) * p.num_heads + head_of(p, kvh, gr)) * kPfHead;
#pragma unroll
      for (int c = 0; c < 4; ++c) store_scalar<KV>(p.out, base + 32 * c + c32, o[c][4 * j + i] * inv);
    }
  }
}

// q heads per decode-row workgroup: the matrix-core wavefronts serve 16
// (block_size 16), the dot-product wavefronts 4.
template <int BS> constexpr int decode_row_heads() { return BS == 16 ? mw::kHeads : kWaveHeads; }

// Decode rows (q_len == 1) of a mixed batch, one workgroup per (sequence,
// kv head, head slice), q / out row cu_q_lens[s]: the matrix-core decode
// wavefronts (tl_mfma_wave.hpp) for block_size 16, so a GQA group of up to
// 16 heads reads its KV once, the 2-byte dot-product wavefronts otherwise.
template <Kind KV, int BS, int NW>
__global__ __launch_bounds__(NW * kWave) void prefill_decode_kernel(PrefillParams pp) {
  constexpr int GT = decode_row_heads<BS>();
  __shared__ __attribute__((aligned(16))) float s_acc[NW * GT * kPfHead];
  __shared__ float s_m[NW * GT], s_l[NW * GT];
  const Params& p = pp.base;
  const int slices = (p.group + GT - 1) / GT;
  int b = blockIdx.x;
  const int hs = b % slices; b /= slices;
  const int kvh = b % p.num_kv_heads, seq = pp.dec_first + b / p.num_kv_heads;
  const int q0 = pp.cu_q_lens[seq];
  if (pp.cu_q_lens[seq + 1] - q0 != 1) return;
  const int L = p.seq_lens[seq];
  Params pd = p;
  const int64_t shift = (int64_t)(q0 - seq) * p.num_heads * kPfHead * 2;   // q / out row q0
  pd.q = (const char*)p.q + shift;
  pd.out = (char*)p.out + shift;
  pd.head_slices = slices;
  if constexpr (BS == 16) {
    mw::decode_workgroup<KV, KV, Kind::F32, NW, true>(pd, seq, kvh, hs, 0, 0, L, s_acc, s_m, s_l);
  } else {
    __shared__ __attribute__((aligned(16))) uint32_t s_p[NW][4][kWaveHeads][4];
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    decode2_wave<KV, kPfHead, BS>(pd, seq, kvh, hs, wave * 32, L, NW * 32, &s_p[wave][0][0][0],
                                  &s_acc[wave * GT * kPfHead], &s_m[wave * GT], &s_l[wave * GT]);
    __syncthreads();
    combine_waves<KV, Kind::F32, kPfHead, true>(pd, NW, s_m, s_l, s_acc, seq, kvh, hs, 0, tid, NW * kWave);
  }
}

template <Kind KV, int BS>
int launch_prefill_t(const PrefillParams& pp, unsigned grid, hipStream_t stream) {
  constexpr int NW = 8, NWD = 8;
  const Params& p = pp.base;
  constexpr int GT = decode_row_heads<BS>();
  const unsigned dgrid = (unsigned)((pp.num_seqs - pp.dec_first) * p.num_kv_heads * ((p.group + GT - 1) / GT));
  if (dgrid > 0)
    hipLaunchKernelGGL((prefill_decode_kernel<KV, BS, NWD>), dim3(dgrid), dim3(NWD * kWave), 0, stream, pp);
  if (grid > 0)
    hipLaunchKernelGGL((prefill_kernel<KV, BS, NW>), dim3(grid), dim3(NW * kWave), 0, stream, pp);
  return hipGetLastError() == hipSuccess ? 0 : 5;
}

}  // namespace

int launch_prefill(const PrefillLaunch& a) {
  constexpr int NW = 8;
  PrefillParams pp;
  Params& p = pp.base;
  p.out = a.out; p.q = a.q;
  p.k_cache = (const char*)a.k_cache; p.v_cache = (const char*)a.v_cache;
  p.block_tables = a.block_tables; p.seq_lens = a.seq_lens;
  p.part_m = nullptr; p.part_l = nullptr; p.part_o = nullptr;
  p.num_heads = a.num_heads; p.num_kv_heads = a.num_kv_heads;
  p.max_blocks_per_seq = a.max_blocks_per_seq; p.num_blocks = a.num_blocks;
  p.num_partitions = 1; p.partition_tokens = 0;
  p.group = a.num_heads / a.num_kv_heads;
  p.head_slices = (p.group + kWaveHeads - 1) / kWaveHeads;
  p.gqa_map = a.gqa_map;
  p.qk_scale = a.scale * kLog2e;
  p.v_scale = 1.f;
  pp.cu_q_lens = a.cu_q_lens;
  pp.num_seqs = a.num_seqs;
  // with the prefill sequences first (num_prefill_seqs > 0) each kernel's grid
  // covers only its own sequences; otherwise both scan every sequence
  pp.pf_seqs = a.num_prefill_seqs > 0 ? a.num_prefill_seqs : a.num_seqs;
  pp.dec_first = a.num_prefill_seqs > 0 ? a.num_prefill_seqs : 0;
  // prefill tiles exist only for q_len > 1
  pp.row_tiles = a.max_q_len > 1 ? (a.max_q_len * p.group + NW * kPfRows - 1) / (NW * kPfRows) : 0;
  const unsigned grid = (unsigned)(pp.row_tiles * pp.pf_seqs * a.num_kv_heads);
  const bool bf16 = a.dtype == (int)Kind::BF16;
  if (a.block_size == 16)
    return bf16 ? launch_prefill_t<Kind::BF16, 16>(pp, grid, a.stream) : launch_prefill_t<Kind::F16, 16>(pp, grid, a.stream);
  return bf16 ? launch_prefill_t<Kind::BF16, 32>(pp, grid, a.stream) : launch_prefill_t<Kind::F16, 32>(pp, grid, a.stream);
}

}  // namespace tl
