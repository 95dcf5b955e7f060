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
//   * the workgroup copies the keys' K ([channel][key] as in the pool, rows
//     padded to 80 halves; the q.k operand is read with the LDS transpose
//     read) and V ([channel][key slot], the key order of the PV operand,
//     rows padded to 72 halves) into LDS (two stages of each);
//     each wavefront copies the 16 keys of one pool block for 64 channels,
//     with loads that each read 1 KB contiguous in the pool;
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
//     LDS in that order.
// The eight wavefronts form two groups with one wavefront of each on every
// SIMD (wavefront w runs on SIMD w % 4); each wavefront alternates an MFMA
// phase (P V of one iteration, S of the next) and a VALU phase (mask,
// softmax, weight packing, staging), group 1 one phase behind group 0, with
// a workgroup barrier after every phase, so that on each SIMD one
// wavefront's matrix ops run beside the other's VALU work.
// Decode rows run the matrix-core decode wavefronts (tl_mfma_wave.hpp), one
// workgroup per (sequence, kv head, 16-head slice), as a second kernel of the
// same call on the same stream (one kernel for both would be sized by the
// decode path's registers on top of the prefill path's).
// Pools: f16 / bf16 (the q type), or FP8 E4M3 with per-tensor k_scale /
// v_scale (codes converted exactly to the q type for q.k and to f16 for
// p.v as they are staged; k_scale folds into the score scale, v_scale into
// the output).  Block sizes: any power of two 8 .. 256; a wavefront's 16-key
// group lies in one block from 16 on, in two at 8 (one per lane half).
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
constexpr int kKtStride = 80;        // halves per channel row of the K stage (64 keys + pad)
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
// LDS stages of K and of V: iteration i uses stage i % 2 (the ping-pong
// schedule of prefill_kernel writes each stage between its readers)
constexpr int kStages = 2;

// P V runs on f16 for both input types: the weights in f16 (11 mantissa
// bits; bf16's 8 would miss 2e-3 by up to 2^-9 max|v| on a short or peaked
// row).  A bf16 V is converted to f16 as it is staged, scaled by 2^-7 so
// that f16's range holds |v| < 2^23 (an f16 value 2^-7 v is exact down to
// |v| = 2^-7, and below that off by at most 2^-17); the weights carry the
// 2^7 instead (they stay below 2^8 by the lazy rescale, so below 2^15 in
// f16), and the row sums are divided by it at the end.  |v| >= 2^23 in a
// bf16 V overflows the f16 stage and the output is not finite.
template <Kind KV> struct PvScale {
  static constexpr float kV = 1.f, kP = 1.f;
  static constexpr int kPExp = 0;
};
template <> struct PvScale<Kind::BF16> {
  static constexpr float kV = 0.0078125f, kP = 128.f;
  static constexpr int kPExp = 7;
};

template <Kind KV> struct Mfma32;
template <> struct Mfma32<Kind::BF16> {
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
  Params base;                 // q, out, pools, tables, seq_lens, heads, group, qk_scale, v_scale
  const int32_t* cu_q_lens;    // [num_seqs + 1]
  int num_seqs, row_tiles;
  int pf_seqs;                 // sequences [0, pf_seqs) may be prefill rows
  int dec_first;               // sequences [dec_first, num_seqs) may be decode rows
};

template <int NW>
struct PrefillSmem {
  struct {
    uint16_t kt[kStages][kPfHead * kKtStride];    // [channel][key] (+16 pad)
    uint16_t v[kStages][kPfHead * kVStride];      // [channel][v_slot(key)] (+8 pad)
    float row[NW][kPfRows];                       // per-row exchange (alpha, l)
  } pf;
};

// A block-table row read through the constant address space: the table is
// not written during the kernel, and with a wave-uniform index the reads
// are scalar loads, which are waited for on their own counter instead of
// behind every K/V load in flight.
typedef const __attribute__((address_space(4))) int32_t* TableRow;

// Table entry of block index lb (>= 0), read unconditionally (index
// clamped to the row, max_blocks_per_seq >= 1); checked_block() turns it
// into the physical block or -1.
__device__ __forceinline__ int table_entry(const Params& p, TableRow table, int lb) {
  return table[__builtin_amdgcn_readfirstlane(min(lb, p.max_blocks_per_seq - 1))];
}
__device__ __forceinline__ int checked_block(const Params& p, int lb, int entry) {
  return (lb >= p.max_blocks_per_seq || entry < 0 || entry >= p.num_blocks) ? -1 : entry;
}

// The A operand of q.k step ks of S^T tile t (keys 32 t .. + 31, channels
// 16 ks .. + 15) from the K stage [channel][key]: lane l needs channels
// 16 ks + 8 (l >> 5) .. + 7 of key 32 t + (l & 31).  ds_read_b64_tr_b16
// hands lane j of a 16-lane group element e = element j % 4 of the 8 bytes
// that lane 4 e + j / 4 of the group addressed; so lane i addresses
// channel c0 + i / 4, keys k0 + 4 (i % 4) .. + 3, and lane j receives
// channels c0 .. c0 + 3 of key k0 + j.  Two reads give the 8 channels.  With
// 160-byte rows the 4 channel rows of a group fall on disjoint banks.
__device__ __forceinline__ u32x4 k_operand(const uint16_t* kst, int t, int ks, int lane) {
  typedef short v4s __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) v4s* LdsV4;
  const int i = lane & 15;
  const int k0 = 32 * t + 16 * ((lane >> 4) & 1), c0 = 16 * ks + 8 * (lane >> 5);
  const uint16_t* a = kst + (c0 + (i >> 2)) * kKtStride + k0 + 4 * (i & 3);
  const v4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((LdsV4)(a));
  const v4s hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((LdsV4)(a + 4 * kKtStride));
  const uint2 l2 = __builtin_bit_cast(uint2, lo), h2 = __builtin_bit_cast(uint2, hi);
  return u32x4{l2.x, l2.y, h2.x, h2.y};
}

// Eight E4M3 codes (c.x: keys 0-3, c.y: keys 4-7) as eight 16-bit values of
// type T, exactly (every E4M3 value, subnormals and NaN included, is an f16
// and a bf16 value).
template <Kind T>
__device__ __forceinline__ u32x4 fp8x8_to(const u32x4& c) {
  auto cvt = [](uint32_t w, bool hi) -> uint32_t {
    if constexpr (T == Kind::BF16)
      return hi ? __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, true))
                : __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, false));
    else
      return hi ? __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, true))
                : __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, false));
  };
  return u32x4{cvt(c.x, false), cvt(c.x, true), cvt(c.y, false), cvt(c.y, true)};
}

// Q: the q / out type (f16 or bf16); KV: the pool's, Q or FP8.
template <Kind Q, Kind KV, int BS, int NW>
__global__ __launch_bounds__(NW * kWave) void prefill_kernel(PrefillParams pp) {
  static_assert(BS >= 8 && BS <= 256 && (BS & (BS - 1)) == 0, "block size: a power of two 8 .. 256");
  static_assert(NW == 8, "two groups of four wavefronts, one wavefront of each group per SIMD");
  static_assert(KV == Q || KV == Kind::FP8, "a 2-byte pool holds the q type");
  constexpr int BPI = BS >= kPfKeys ? 1 : kPfKeys / BS;   // pool blocks per iteration
  constexpr int BSE = BS >= kPfKeys ? kPfKeys : BS;       // keys of an iteration per block
  constexpr int NKE = BS == 8 ? 2 : 1;                    // blocks of a wavefront's 16-key group
  constexpr int E = KV == Kind::FP8 ? 1 : 2;              // pool bytes per element
  using M = Mfma32<Q>;                                 // q.k
  using MP = Mfma32<Kind::F16>;                        // p.v (f16 for every type)
  __shared__ __attribute__((aligned(16))) PrefillSmem<NW> sm;

  const Params& p = pp.base;
  const int tid = threadIdx.x, lane = tid % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int g = lane >> 5, c32 = lane & 31;
  // group 0 (wavefronts 0-3) leads, group 1 (4-7) runs one phase behind;
  // wavefront w runs on SIMD w % 4, so every SIMD holds one of each
  const int grp = wave >> 2;

  int b = blockIdx.x;
  const int items = pp.pf_seqs * p.num_kv_heads;
  const int tile = pp.row_tiles - 1 - b / items;       // longest (latest) tiles first
  b %= items;
  const int seq = b / p.num_kv_heads, kvh = b % p.num_kv_heads;
  // The table entries of the wavefront's key group (see the staging below)
  // in the first two iterations are read with the lengths, before the exits
  // that depend on them: one memory round trip for all.
  const TableRow table = (TableRow)(p.block_tables + (int64_t)seq * p.max_blocks_per_seq);
  const int kg = 16 * (wave >> 1);                     // first key of the wavefront's group
  // logical block of key kk of iteration it (>= 0)
  auto blk_of = [](int it, int kk) { return (int)((unsigned)(it * kPfKeys + kk) / BS); };
  int e0[NKE], e1[NKE];
#pragma unroll
  for (int h = 0; h < NKE; ++h) {
    e0[h] = table_entry(p, table, blk_of(0, kg + 8 * h));
    e1[h] = table_entry(p, table, blk_of(1, kg + 8 * h));
  }
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
  // keys of the workgroup (wave-uniform: the division runs on the VALU)
  const int kend = __builtin_amdgcn_readfirstlane(max(0, L - ql + last_row / p.group + 1));
  const int n_it = (kend + kPfKeys - 1) / kPfKeys;

  // B operand of S^T: row my_row, channels 16 ks + 8 g .. +7.  Padding
  // rows (past the tile's rows) load query q0's first head: their scores
  // stay in their own columns and are never stored.  Loaded in the
  // prologue after K(0), so that staging K(0) does not wait for them.
  u32x4 qb[8];
  auto load_q = [&]() {
    const uint16_t* qrow = (const uint16_t*)p.q +
        ((int64_t)(q0 + qi) * p.num_heads + head_of(p, kvh, gi)) * kPfHead + 8 * g;
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) qb[ks] = load16(qrow + 16 * ks);
  };

  const int64_t head_bytes = (int64_t)kPfHead * BS * E;                // bytes per (block, kv head)
  const char* kpool = p.k_cache;
  const char* vpool = p.v_cache;

  // Staging: wavefront w copies the 16 keys kg = 16 (w >> 1) .. kg + 15 of
  // an iteration for the 64 channels 64 (w & 1) .. + 63, as two units of 32
  // channels.  Lane l holds channel (l & 31) of the unit and keys
  // kg + 8 (l >> 5) .. + 7 (16 bytes; 8 for FP8), so one load of a unit
  // reads 1 KB (512 B) that is contiguous in the pool at block sizes 16 and
  // 32.  From block size 16 on the key group lies in one block, whose id is
  // wave-uniform (descriptors in scalar registers); at block size 8 each
  // lane half has a block of its own.
  constexpr int kUnits = 2;                            // 32-channel units per wavefront
  static_assert(NW == 2 * (kPfKeys / 16) && kUnits * 32 * 2 == kPfHead, "key groups x channel halves");
  const int tok = kg + 8 * g;                          // first key of the lane's 8
  auto unit_ch = [&](int u) { return 64 * (wave & 1) + 32 * u + c32; };
  // A phase's copy: K of one iteration and V of the one before (K is
  // staged two phases ahead of its use, V one).  nv: keys of the lane's V
  // run that exist (the rest is zeroed when staged, so that the loads are
  // waited for only there).
  struct Fetched { u32x4 k[kUnits], v[kUnits]; int nv; };
  // unconditional loads (a missing block has an empty range and reads
  // zeros): no branch, so nothing waits for them before the staging
  auto rsrc_of = [&](const char* pool, int pb) {
    const int64_t row = pb >= 0 ? ((int64_t)pb * p.num_kv_heads + kvh) * head_bytes : 0;
    return buffer_rsrc(pool + row, pb >= 0 ? unsigned(head_bytes) : 0u);
  };
  auto load_raw = [&](__amdgpu_buffer_rsrc_t r, unsigned off) -> u32x4 {
    if constexpr (E == 2) {
      return buffer_load16(r, off);
    } else {
      const auto w = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 2);
      return u32x4{(uint32_t)w[0], (uint32_t)w[1], 0u, 0u};
    }
  };
  // the lane's keys tok .. tok + 7 of channel ch in iteration it: a run of
  // a block row, at the iteration's offset in the block
  auto load_unit = [&](const char* pool, const int (&pb)[NKE], int it, int ch) -> u32x4 {
    // (a block of at most 64 keys holds whole key groups at the same offset
    // in every iteration)
    const int in_blk = BS > kPfKeys ? (int)((unsigned)(it * kPfKeys) % BS) + tok : tok % BS;
    const unsigned off = unsigned(E * (ch * BS + in_blk));
    if constexpr (NKE == 1) {
      return load_raw(rsrc_of(pool, pb[0]), off);
    } else {
      // each load serves one lane half; the other half's offset lies past
      // the range (no memory request, zeros)
      constexpr unsigned kPast = 0x40000000u;
      const u32x4 a = load_raw(rsrc_of(pool, pb[0]), g == 0 ? off : kPast);
      const u32x4 b = load_raw(rsrc_of(pool, pb[1]), g == 1 ? off : kPast);
      return u32x4{a.x | b.x, a.y | b.y, a.z | b.z, a.w | b.w};
    }
  };
  // physical block of half h of the wavefront's key group in iteration it
  // from its table entry, or -1
  auto group_block = [&](int it, int entry, int h) {
    const int key0 = it * kPfKeys + kg + 8 * h;
    return __builtin_amdgcn_readfirstlane(key0 < kend && it >= 0 ? checked_block(p, blk_of(it, kg + 8 * h), entry)
                                                                 : -1);
  };
  // the blocks of one copy; load(i) issues its i-th load (K unit i, then V
  // unit i - kUnits), so that a phase can spread them over its matrix ops
  struct Entries { int k[NKE], v[NKE]; };
  struct FetchPlan { int pk[NKE], pv[NKE], it_k, it_v; };
  auto plan = [&](int it_k, int it_v, const Entries& e, Fetched& f) {
    FetchPlan fp;
    fp.it_k = it_k;
    fp.it_v = it_v;
#pragma unroll
    for (int h = 0; h < NKE; ++h) {
      fp.pk[h] = group_block(it_k, e.k[h], h);
      fp.pv[h] = group_block(it_v, e.v[h], h);
    }
    const int pv_lane = NKE == 2 ? (g ? fp.pv[NKE - 1] : fp.pv[0]) : fp.pv[0];
    f.nv = pv_lane >= 0 ? min(max(L - (it_v * kPfKeys + tok), 0), 8) : 0;
    return fp;
  };
  auto load = [&](const FetchPlan& fp, int i, Fetched& f) {
    if (i < kUnits) f.k[i] = load_unit(kpool, fp.pk, fp.it_k, unit_ch(i));
    else f.v[i - kUnits] = load_unit(vpool, fp.pv, fp.it_v, unit_ch(i - kUnits));
  };
  auto fetch = [&](int it_k, int it_v, const Entries& e, Fetched& f) {
    const FetchPlan fp = plan(it_k, it_v, e, f);
#pragma unroll
    for (int i = 0; i < 2 * kUnits; ++i) load(fp, i, f);
  };
  auto stage = [&](int it_k, int it_v, const Fetched& f) {
#pragma unroll
    for (int u = 0; u < kUnits; ++u) {
      // K as it lies in the pool: the lane's 8 keys of its channel, one
      // 16-byte write (k_operand reads it transposed)
      const u32x4 kq = KV == Kind::FP8 ? fp8x8_to<Q>(f.k[u]) : f.k[u];
      *reinterpret_cast<u32x4*>(&sm.pf.kt[it_k & 1][unit_ch(u) * kKtStride + tok]) = kq;
      // V slots at or past the sequence end may hold anything (NaN codes
      // too, and a zero weight times NaN is NaN): zero them
      u4v v = __builtin_bit_cast(u4v, KV == Kind::FP8 ? fp8x8_to<Kind::F16>(f.v[u]) : f.v[u]);
      const int nv = f.nv;
      // a wave-uniform branch (the sequence's last iteration only): as a
      // lane-divergent one it became selects run on every iteration
      if (__builtin_amdgcn_ballot_w64(nv < 8)) {
#pragma unroll
        for (int w = 0; w < 4; ++w) v[w] = 2 * w >= nv ? 0u : (2 * w + 1 >= nv ? v[w] & 0xFFFFu : v[w]);
      }
      if constexpr (KV == Kind::BF16) {
        // bf16 -> f16, times 2^-7 (see PvScale)
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const unsigned x = (unsigned)v[w];
          v[w] = MP::pack(__builtin_bit_cast(float, x << 16) * PvScale<KV>::kV,
                          __builtin_bit_cast(float, x & 0xFFFF0000u) * PvScale<KV>::kV);
        }
      }
      uint16_t* vrow = &sm.pf.v[it_v & 1][unit_ch(u) * kVStride];
      *reinterpret_cast<uint2*>(vrow + v_slot(tok)) = uint2{v[0], v[1]};
      *reinterpret_cast<uint2*>(vrow + v_slot(tok + 4)) = uint2{v[2], v[3]};
    }
  };
  // Table entries are read two phases before their use by one vector load:
  // lanes [0, NKE) the K blocks of the fetch, [NKE, 2 NKE) its V blocks,
  // lane 2 NKE + i block i of the mask.  A scalar table read would be
  // waited for behind every LDS access in flight (one counter covers both).
  const int32_t* table_v = p.block_tables + (int64_t)seq * p.max_blocks_per_seq;
  const int t_key = lane < 2 * NKE ? kg + 8 * (lane % NKE) : min(lane - 2 * NKE, BPI - 1) * BSE;
  const int t_it = lane < NKE ? 1 + grp : (lane < 2 * NKE ? grp : 0);   // iteration offset of the lane's entry
  // entries of step jn: the fetch of MFMA phase X_jn (K of jn + 1 + grp, V
  // of jn + grp, staged by Y_jn) and the mask of Y_jn
  auto table_prefetch = [&](int jn) {
    const int lb = blk_of(max(jn + t_it, 0), t_key);
    return table_v[min(lb, p.max_blocks_per_seq - 1)];
  };
  auto entries = [&](int t) {
    Entries e;
#pragma unroll
    for (int h = 0; h < NKE; ++h) {
      e.k[h] = __builtin_amdgcn_readlane(t, h);
      e.v[h] = __builtin_amdgcn_readlane(t, NKE + h);
    }
    return e;
  };

  f16v o[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) o[c] = f16v{};
  float m_used = -INFINITY, l_part = 0.f;
  float* s_row = &sm.pf.row[wave][0];
  // Scores and weights of an iteration share registers: QK leaves the S^T
  // tiles in sp (MFMA phase), SM turns tile t into its packed f16 weights
  // in place (VALU phase: words 8 s .. 8 s + 3 hold those of step s), and PV
  // of the next MFMA phase reads them before QK overwrites them.
  // (__builtin_bit_cast of a vector element itself, v[i], reads element 0
  // with this compiler: the elements go through a value conversion first.)
  f16v sp[KT];
  auto p_words = [&](int t, int s2) {
    const int w = 8 * s2;
    return u32x4{__builtin_bit_cast(unsigned, (float)sp[t][w]), __builtin_bit_cast(unsigned, (float)sp[t][w + 1]),
                 __builtin_bit_cast(unsigned, (float)sp[t][w + 2]), __builtin_bit_cast(unsigned, (float)sp[t][w + 3])};
  };

  // ---- the two halves of an iteration ----
  // QK(it): S^T tiles of iteration it (K stage it % 2)
  auto qk = [&](int it) {
    const uint16_t* kst = sm.pf.kt[it & 1];
#pragma unroll
    for (int t = 0; t < KT; ++t) {
      f16v acc = f16v{};
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) acc = M::mma(k_operand(kst, t, ks, lane), qb[ks], acc);
      sp[t] = acc;
    }
  };
  // SM(it): mask, row max, lazy rescale, exponentials and weight packing.
  // Keys of an iteration entirely at or below the wavefront's first query
  // position, in blocks that exist, need no mask.  The scores stay unscaled
  // until the exponent (qk_scale > 0, so the max commutes with the scale).
  const int wmin_pos = __builtin_amdgcn_readfirstlane(L - ql + wrow0 / p.group);
  const int pos_g = pos - 4 * g;
  // Iterations [0, j_plain) lie at or below the wavefront's first query
  // position: without holes they need no mask.
  const int j_plain = min(n_it, (wmin_pos + 1) / kPfKeys);
  auto blocks_ok = [&](int it, int t_entries, bool (&blk_ok)[BPI]) {
    bool all_ok = true;
#pragma unroll
    for (int bi = 0; bi < BPI; ++bi) {
      blk_ok[bi] = checked_block(p, blk_of(it, bi * BSE), __builtin_amdgcn_readlane(t_entries, 2 * NKE + bi)) >= 0;
      all_ok = all_ok && blk_ok[bi];
    }
    return all_ok;
  };
  // MASK false: an iteration below j_plain whose blocks all exist.  The two
  // forms run in separate loops, so that no path merges scores (a masked
  // and an unmasked form of the same scores in one loop body cost 16 64-bit
  // register copies per iteration).
  auto softmax = [&](int it, int t_entries, auto mask_tag) {
    constexpr bool MASK = decltype(mask_tag)::value;
    const int k0 = it * kPfKeys;
    float mx = -INFINITY;
    if constexpr (!MASK) {
#pragma unroll
      for (int t = 0; t < KT; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sp[t][r]);
    } else {
      bool blk_ok[BPI];
      blocks_ok(it, t_entries, blk_ok);
#pragma unroll
      for (int t = 0; t < KT; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          // key k0 + kk, kk = 32 t + 8 (r >> 2) + 4 g + (r & 3): the
          // comparison is written with the wave-uniform part on the left
          // so that no per-lane value of each r is kept across the loop
          const int kc = 32 * t + 8 * (r >> 2) + (r & 3);
          const bool ok = k0 + kc <= pos_g && blk_ok[(kc + 4 * g) / BSE];
          sp[t][r] = ok ? sp[t][r] : -INFINITY;
          mx = fmaxf(mx, sp[t][r]);
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
    // the weights carry 2^kPExp (see PvScale): a factor common to every
    // weight and row sum, so the rounding of m_use - kPExp cancels
    const float m_use = ((m_used == -INFINITY) ? 0.f : m_used) - (float)PvScale<KV>::kPExp;
#pragma unroll
    for (int t = 0; t < KT; ++t) {
      float pw[16], ls[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        pw[r] = __builtin_amdgcn_exp2f(__builtin_fmaf(sp[t][r], p.qk_scale, -m_use));
        ls[r & 3] += pw[r];
      }
      l_part += (ls[0] + ls[1]) + (ls[2] + ls[3]);
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2) {
        const int r0 = 8 * s2;
        const u32x4 pa = {MP::pack(pw[r0 + 0], pw[r0 + 1]), MP::pack(pw[r0 + 2], pw[r0 + 3]),
                          MP::pack(pw[r0 + 4], pw[r0 + 5]), MP::pack(pw[r0 + 6], pw[r0 + 7])};
        const u4v pa4 = __builtin_bit_cast(u4v, pa);
#pragma unroll
        for (int i = 0; i < 4; ++i) sp[t][8 * s2 + i] = __builtin_bit_cast(float, (unsigned)pa4[i]);
      }
    }
  };

  // ---- ping-pong schedule ----
  // A wavefront alternates MFMA phases X_j = {PV(j - 1), QK(j)} and VALU
  // phases Y_j = {SM(j); stage K(j + 1 + grp), V(j + grp)}: X_0 Y_0 X_1 ...
  // Y_{n-1} X_n, group 1 with a leading Y_{-1} (staging only).  Every phase
  // ends at a workgroup barrier, so on each SIMD one wavefront's matrix ops
  // run beside the other's VALU work.  K(k) is read at phases 2k and 2k + 1
  // and written in [2k - 2, 2k - 1]; V(k) is read at 2k + 2 and 2k + 3 and
  // written in [2k, 2k + 1]: two LDS stages of each suffice.  Stages of
  // iterations past the last hold zeros (missing blocks) and are not read.
  // The K/V loads of a VALU phase's staging are issued at the start of the
  // MFMA phase before it (one register set, a phase of latency slack); the
  // table entries they need were read by the VALU phase before that.
  Fetched fs;
  int t_ent, t_mask = 0;
  {
    // All of the prologue's loads go out together (K(0), q, the copy of
    // group 1's Y_{-1}, the first table entries), in the order in which
    // they are waited for: K(0) is staged before the first barrier, q is
    // read by X_0; group 1's Y_{-1} stages K(1), V(0) (group 0 loads its own
    // copy again in X_0, unconditional so that the wait counts agree on
    // every path)
    Fetched f0;
    Entries ea, eb;
#pragma unroll
    for (int h = 0; h < NKE; ++h) {
      ea.k[h] = e0[h]; ea.v[h] = e0[h];
      eb.k[h] = e1[h]; eb.v[h] = e0[h];
    }
    fetch(0, -1, ea, f0);
    load_q();
    fetch(1, 0, eb, fs);
    t_ent = table_prefetch(0);
    stage(0, -1, f0);                   // K(0); V stage 1 gets zeros (iteration -1 is missing)
  }
  __syncthreads();

  // X_{j+1}: the loads of Y_{j+1}, P V of iteration j and S of iteration
  // j + 1 (past the last iteration S is formed on a zero stage and not
  // used: unconditional, so that no path carries scores or weights across a
  // phase)
  auto fetch_for = [&](int jn) {        // the loads staged by Y_jn
    fetch(jn + 1 + grp, jn + grp, entries(t_ent), fs);
  };
  auto phase_x0 = [&]() {
    fetch_for(0);
    t_mask = t_ent;
    t_ent = table_prefetch(1);
    __builtin_amdgcn_s_setprio(1);
    qk(0);
    __builtin_amdgcn_s_setprio(0);
  };
  // PV(j) and QK(j + 1).  P V: the weights of tile t leave the S^T
  // accumulator as keys 32 t + 16 s + 4 g + i (slots 0-3) and the same + 8
  // (slots 4-7) for lane group g, the k order of step s.  The LDS operand
  // reads are kept ahead of the matrix ops (the compiler alone keeps one or two in
  // flight, and the phase then waits on LDS latency): P V in four groups
  // (t, s2) of the four V operands of o[0..3], issued hi for all four, then
  // lo, so that no MFMA waits for the one before it, with the next group's
  // reads in flight; then S with both tiles' chains interleaved and the K
  // reads of the next kQkAhead steps in flight.
  auto pv_qk = [&](int j, const FetchPlan& fp) {
    const uint16_t* vst = sm.pf.v[j & 1];
    const uint16_t* kst = sm.pf.kt[(j + 1) & 1];
    auto v_op = [&](int grp4, int c) {
      const int t = grp4 >> 1, s2 = grp4 & 1;
      return *reinterpret_cast<const u32x4*>(vst + (32 * c + c32) * kVStride + 32 * t + 16 * s2 + 8 * g);
    };
    auto k_op = [&](int t, int ks) { return k_operand(kst, t, ks, lane); };
    u32x4 vb[2][4];
#pragma unroll
    for (int c = 0; c < 4; ++c) vb[0][c] = v_op(0, c);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      static_assert(2 * kUnits == 4, "one load per P V group");
      load(fp, q, fs);
      if (q + 1 < 4) {
#pragma unroll
        for (int c = 0; c < 4; ++c) vb[(q + 1) & 1][c] = v_op(q + 1, c);
      }
      const int t = q >> 1, s2 = q & 1;
#pragma unroll
      for (int c = 0; c < 4; ++c) o[c] = MP::mma(p_words(t, s2), vb[q & 1][c], o[c]);
    }
    constexpr int kQkAhead = 3;
    u32x4 kb[kQkAhead + 1][KT];
#pragma unroll
    for (int ks = 0; ks < kQkAhead; ++ks)
#pragma unroll
      for (int t = 0; t < KT; ++t) kb[ks][t] = k_op(t, ks);
    __builtin_amdgcn_sched_barrier(0);   // the reads stay issued ahead of their MFMAs
    f16v acc[KT];
#pragma unroll
    for (int t = 0; t < KT; ++t) acc[t] = f16v{};
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
      if (ks + kQkAhead < 8) {
#pragma unroll
        for (int t = 0; t < KT; ++t) kb[(ks + kQkAhead) % (kQkAhead + 1)][t] = k_op(t, ks + kQkAhead);
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int t = 0; t < KT; ++t) acc[t] = M::mma(kb[ks % (kQkAhead + 1)][t], qb[ks], acc[t]);
    }
#pragma unroll
    for (int t = 0; t < KT; ++t) sp[t] = acc[t];
  };
  // The loads are unconditional (past the last iteration the blocks are
  // missing: empty ranges, no traffic), so that every path leaves the same
  // loads in flight and the wait counts stay exact; a path without them
  // makes the next phase wait for every load.  The table read of step
  // jn + 1 goes out here too, two phases before its first use.
  auto phase_x = [&](int j) {
    const FetchPlan fp = plan(j + 2 + grp, j + 1 + grp, entries(t_ent), fs);   // the copy staged by Y_{j+1}
    t_mask = t_ent;                      // waited for by the readlanes: a plain copy
    t_ent = table_prefetch(j + 2);
    __builtin_amdgcn_s_setprio(1);
    pv_qk(j, fp);
    __builtin_amdgcn_s_setprio(0);
  };
  // Y_j: SM(j) with the mask entries of step j and the staging of
  // K(j + 1 + grp), V(j + grp)
  auto phase_y = [&](int j, auto mask_tag) {
    softmax(j, t_mask, mask_tag);
    // the weights are formed here: the exponentials and packing are plain
    // arithmetic, which the compiler would otherwise sink past the barrier
    // into the MFMA phase that reads them
#pragma unroll
    for (int t = 0; t < KT; ++t) asm volatile("" ::"v"(sp[t]));
    asm volatile("" ::"v"(l_part));
    stage(j + 1 + grp, j + grp, fs);
  };
  // Group 0: X_0 at phase 0, Y_j at 2j + 1, X_{j+1} at 2j + 2, then one
  // empty phase; group 1: Y_{-1} (staging only) at phase 0, X_0 at 1, Y_j
  // at 2j + 2, X_{j+1} at 2j + 3.  Both pass 2 n + 2 barriers.
  if (grp == 1) {
    stage(1, 0, fs);
    __syncthreads();
  }
  phase_x0();
  __syncthreads();
  // The loops differ per wavefront only in where one ends and the other
  // begins: every wavefront passes the same barriers.
  int j = 0;
#pragma unroll 1
  for (; j < j_plain; ++j) {
    bool blk_ok[BPI];
    if (!blocks_ok(j, t_mask, blk_ok)) break;          // a hole: the masked loop takes over
    phase_y(j, std::false_type{});
    __syncthreads();
    phase_x(j);
    __syncthreads();
  }
#pragma unroll 1
  for (; j < n_it; ++j) {
    phase_y(j, std::true_type{});
    __syncthreads();
    phase_x(j);
    __syncthreads();
  }
  if (grp == 0) __syncthreads();

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
  // Output row of tile row r = qr group + gr (query q0 + qr, head
  // head_of(gr)), in 128-element rows: q0 H + kvh group + r + qr (H - group)
  // for the grouped map, q0 H + kvh + r n_kv for the modulo map (H = group
  // n_kv).  qr = floor((r + 1/2) / group) as an fp32 product, exact for
  // r < 2^22 (the launch checks): the half step keeps the rounding off the
  // integers.
  const float rg = 1.f / (float)p.group;
  const int64_t obase = (int64_t)q0 * p.num_heads + (p.gqa_map ? kvh * p.group : kvh);
  const int rmul = p.gqa_map ? 1 : p.num_kv_heads, qmul = p.gqa_map ? p.num_heads - p.group : 0;
  const bool odd = (c32 & 1) != 0;
  // Two channels per 4-byte store: lanes 2k and 2k + 1 swap one value, so
  // that for rows (i, i + 1) the even lane stores row i at channels c32,
  // c32 + 1 and the odd lane row i + 1 at c32 - 1, c32.
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    float inv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float l = s_row[8 * j + 4 * g + i];
      inv[i] = l > 0.f ? PvScale<KV>::kP * __builtin_amdgcn_rcpf(l) : 0.f;   // the sums carry 2^kPExp
      if constexpr (KV == Kind::FP8) inv[i] *= p.v_scale;
    }
#pragma unroll
    for (int ip = 0; ip < 4; ip += 2) {
      const int row = wrow0 + 8 * j + 4 * g + ip + (odd ? 1 : 0);
      const int qr = (int)(((float)row + 0.5f) * rg);
      uint32_t* dst = reinterpret_cast<uint32_t*>(
          (uint16_t*)p.out + (obase + (int64_t)row * rmul + (int64_t)qr * qmul) * kPfHead + (c32 & ~1));
      uint32_t w[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const float a = o[c][4 * j + ip] * inv[ip], b2 = o[c][4 * j + ip + 1] * inv[ip + 1];
        const float send = odd ? a : b2;
        const float got = __builtin_bit_cast(
            float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, send), 0xB1, 0xF, 0xF, false));  // quad_perm 1,0,3,2
        w[c] = odd ? M::pack(got, b2) : M::pack(a, got);
      }
      if (row < rows) {
#pragma unroll
        for (int c = 0; c < 4; ++c) dst[16 * c] = w[c];
      }
    }
  }
}

// Decode rows (q_len == 1) of a mixed batch, one workgroup per (sequence,
// kv head, 16-head slice), q / out row cu_q_lens[s]: the matrix-core decode
// wavefronts (tl_mfma_wave.hpp), so a GQA group of up to 16 heads reads its
// KV once, at every block size and for FP8 pools too.
template <Kind Q, Kind KV, int BS, int NW>
__global__ __launch_bounds__(NW * kWave) void prefill_decode_kernel(PrefillParams pp) {
  constexpr int GT = mw::kHeads;
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
  mw::decode_workgroup<KV, Q, Kind::F32, NW, true, BS>(pd, seq, kvh, hs, 0, 0, L, s_acc, s_m, s_l);
}

template <Kind Q, Kind KV, int BS>
int launch_prefill_t(const PrefillParams& pp, unsigned grid, hipStream_t stream) {
  // decode rows: 4 wavefronts per workgroup (8: 926.2 against 916.8 us per
  // 4-chunk step at 32 rows of ctx 2048, 64/8 heads; 12 and 16 slower still)
  constexpr int NW = 8, NWD = 4;
  const Params& p = pp.base;
  constexpr int GT = mw::kHeads;
  const unsigned dgrid = (unsigned)((pp.num_seqs - pp.dec_first) * p.num_kv_heads * ((p.group + GT - 1) / GT));
  if (dgrid > 0)
    hipLaunchKernelGGL((prefill_decode_kernel<Q, KV, BS, NWD>), dim3(dgrid), dim3(NWD * kWave), 0, stream, pp);
  if (grid > 0)
    hipLaunchKernelGGL((prefill_kernel<Q, KV, BS, NW>), dim3(grid), dim3(NW * kWave), 0, stream, pp);
  return hipGetLastError() == hipSuccess ? 0 : 5;
}

template <Kind Q, Kind KV>
int launch_prefill_bs(const PrefillParams& pp, int bs, unsigned grid, hipStream_t stream) {
  switch (bs) {
    case 8: return launch_prefill_t<Q, KV, 8>(pp, grid, stream);
    case 16: return launch_prefill_t<Q, KV, 16>(pp, grid, stream);
    case 32: return launch_prefill_t<Q, KV, 32>(pp, grid, stream);
    case 64: return launch_prefill_t<Q, KV, 64>(pp, grid, stream);
    case 128: return launch_prefill_t<Q, KV, 128>(pp, grid, stream);
    case 256: return launch_prefill_t<Q, KV, 256>(pp, grid, stream);
    default: return 3;
  }
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
  const bool fp8 = a.kv_dtype == (int)Kind::FP8;
  // FP8: the codes enter both products unscaled; k_scale scales the scores,
  // v_scale the output
  p.qk_scale = a.scale * (fp8 ? a.k_scale : 1.f) * kLog2e;
  p.v_scale = fp8 ? a.v_scale : 1.f;
  p.block_size = a.block_size;
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
  if (fp8)
    return bf16 ? launch_prefill_bs<Kind::BF16, Kind::FP8>(pp, a.block_size, grid, a.stream)
                : launch_prefill_bs<Kind::F16, Kind::FP8>(pp, a.block_size, grid, a.stream);
  return bf16 ? launch_prefill_bs<Kind::BF16, Kind::BF16>(pp, a.block_size, grid, a.stream)
              : launch_prefill_bs<Kind::F16, Kind::F16>(pp, a.block_size, grid, a.stream);
}

}  // namespace tl
