// tl_decode_mfma.hip -- paged-attention decode on the matrix cores
// (head_size 128; block sizes 8 .. 256 for 2-byte and FP8 E4M3 KV).
//
// The wavefronts are in tl_mfma_wave.hpp.  Why matrix cores for decode:
//   * FP8: a byte is one element, so per byte of HBM traffic there are twice
//     the multiply-adds of 2-byte KV, which the packed dot products of the
//     2-byte wavefront cannot keep up with;
//   * 2-byte KV: the MFMA formulation needs half the VALU work of the
//     packed dot products per byte (6.38 against 5.94 TB/s at GQA group 4),
//     and its 16 columns serve a whole group of up to 16 heads from one KV
//     read, where the dot-product wavefront reads the KV once per 4 heads.
// The dequant scales of FP8 fold into the score scale (k_scale) and the
// output (v_scale), as the reference's dequantise-then-multiply does (the
// scaled K/V are k_scale * code and v_scale * code).  Workgroups and the
// split-K / log-sum-exp protocol are those of the 2-byte decode (NW
// wavefronts stride over a partition's iterations and merge in LDS).
#include <algorithm>

#include "tl_device.hpp"
#include "tl_internal.hpp"
#include "tl_mfma_wave.hpp"

namespace tl {

namespace {

// Work item of a decode workgroup: (sequence, kv head, head slice,
// partition) and the partition's token range [t0, t1); false when the
// partition starts past the sequence (split-K only).  With late_exit (and
// for the single pass) the item is always returned, t1 is the partition's
// end and len the sequence's length, applied by the wavefronts after their
// first loads: the block-table
// reads and the first K/V loads are then issued together with the length
// read instead of after it, and a partition past the end exits once they
// are done (decode_workgroup).
struct Item {
  int seq, kvh, hs, part, t0, t1, len;
};
__device__ __forceinline__ bool item_of(const Params& p, bool final, bool late_exit, Item& w) {
  int bid = grid_item(p, w.part);
  w.hs = bid % p.head_slices;      bid /= p.head_slices;
  w.kvh = bid % p.num_kv_heads;
  w.seq = bid / p.num_kv_heads;
  const int L = p.seq_lens[w.seq];
  w.t0 = w.part * p.partition_tokens;
  if (late_exit || final) {           // final: one partition, t0 = 0
    w.t1 = w.t0 + p.partition_tokens;
    w.len = L;
    return true;
  }
  if (!final && w.t0 >= L) return false;
  w.t1 = min(w.t0 + p.partition_tokens, L);
  w.len = 0x7fffffff;
  return true;
}

// LATE: split-K items past the sequence's end exit after their first loads
// (item_of's late_exit), for grids that fit the GPU in one round, where the
// launch is a chain of round trips (length, table, K/V, partials) and the
// few loads of an exiting workgroup cost less than a round trip.
template <Kind QK, Kind PO, int NW, bool FINAL, int BS, bool LATE = false>
__global__ __launch_bounds__(NW * kWave) void fp8_decode_kernel(Params p) {
  __shared__ __attribute__((aligned(16))) float s_acc[NW * mw::kHeads * mw::kHead];
  __shared__ float s_m[NW * mw::kHeads], s_l[NW * mw::kHeads];
  Item w;
  if (!item_of(p, FINAL, LATE, w)) return;
  mw::decode_workgroup<Kind::FP8, QK, PO, NW, FINAL, BS, LATE>(p, w.seq, w.kvh, w.hs, w.part, w.t0, w.t1, s_acc,
                                                               s_m, s_l, w.len);
}

// ITERS: 1 or 2 when no wavefront has more iterations (mw::mfma2_wave).
template <Kind KV, Kind PO, int NW, bool FINAL, int BS, bool LATE = false, int ITERS = 0>
__global__ __launch_bounds__(NW * kWave) void mfma2_decode_kernel(Params p) {
  __shared__ __attribute__((aligned(16))) float s_acc[NW * mw::kHeads * mw::kHead];
  __shared__ float s_m[NW * mw::kHeads], s_l[NW * mw::kHeads];
  Item w;
  if (!item_of(p, FINAL, LATE, w)) return;
  mw::decode_workgroup<KV, KV, PO, NW, FINAL, BS, LATE, ITERS>(p, w.seq, w.kvh, w.hs, w.part, w.t0, w.t1, s_acc, s_m,
                                                             s_l, w.len);
}

// Split-K, whole partitions per wavefront (mw::partitions_per_wave): the
// grid is (group of 4 wavefronts' partition runs) x (sequence, kv head,
// head slice), the group slowest; wavefront w of group g streams
// partitions (4 g + w) k .. (4 g + w + 1) k - 1, k = parts_per_wave.
// Three wavefronts per SIMD: left alone the compiler allocates ~192
// registers (2 per SIMD), although 160 hold the FP8 wavefront without
// spilling (at 4 per SIMD, 128 registers, it spills ~4 KiB per lane).
template <Kind KV, Kind QK, int BS>
__global__ __launch_bounds__(4 * kWave) __attribute__((amdgpu_waves_per_eu(3))) void wave_partition_kernel(
    Params p) {
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int runs = (p.num_partitions + p.parts_per_wave - 1) / p.parts_per_wave;
  const int groups = (runs + 3) / 4;
  const int items = (int)gridDim.x / groups;
  const int pg = (int)blockIdx.x / items;
  int bid = (int)blockIdx.x - pg * items;
  const int hs = bid % p.head_slices;      bid /= p.head_slices;
  const int kvh = bid % p.num_kv_heads;
  const int seq = bid / p.num_kv_heads;
  extern __shared__ __attribute__((aligned(16))) float stash[];
  mw::partitions_per_wave<KV, QK, BS>(p, seq, kvh, hs, (4 * pg + wave) * p.parts_per_wave,
                                      p.stash_floats ? stash + wave * p.stash_floats : nullptr);
}

// Whether split-K runs one partition per wavefront: when splitting a
// partition over the 4 wavefronts of a workgroup would leave each at most
// 4 iterations (FP8 at 512 / 1024 tokens: 2 / 4 iterations of 64 tokens;
// 2-byte at 512: 4 of 32), and there are at least 4096 partitions to fill
// the GPU's SIMDs.  Measured (FP8, batch 16, ctx 32768): 512-token
// partitions 222 against 281 us, 1024-token 201 against 231 us; with only 4
// partitions per sequence the 4-wavefront split wins (184 against 299 us),
// and so it does for 1024-token partitions of 2-byte KV (8 iterations per
// wavefront: 177 against 193 us).
template <Kind KV>
bool partition_per_wave(int partition_tokens, long partitions_total) {
  return partition_tokens <= 16 * mw::tokens_per_iteration<KV>() && partitions_total >= 4096;
}

// PO_SPLIT: the split-K partial outputs' type (F32, or F16 for f16 q)
template <Kind KV, Kind QK, int NW, bool FINAL, int BS, Kind PO_SPLIT = Kind::F32, bool LATE = false,
          int ITERS = 0>
void launch_kernel(const Params& p, unsigned grid, hipStream_t stream) {
  constexpr Kind PO = FINAL ? QK : PO_SPLIT;
  if constexpr (KV == Kind::FP8)
    hipLaunchKernelGGL((fp8_decode_kernel<QK, PO, NW, FINAL, BS, LATE>), dim3(grid), dim3(NW * kWave), 0, stream,
                       p);
  else
    hipLaunchKernelGGL((mfma2_decode_kernel<KV, PO, NW, FINAL, BS, LATE, ITERS>), dim3(grid), dim3(NW * kWave), 0,
                       stream, p);
}

// The split-K kernels of small grids (LATE), by the most iterations a
// wavefront has (a partition of at most NW or 2 NW iterations).
template <Kind KV, Kind QK, int NW, int BS, Kind PO_SPLIT>
void launch_late(const Params& p, unsigned grid, hipStream_t stream) {
  const int step = NW * mw::tokens_per_iteration<KV>();
  if (KV != Kind::FP8 && p.partition_tokens <= step)
    launch_kernel<KV, QK, NW, false, BS, PO_SPLIT, true, 1>(p, grid, stream);
  else if (KV != Kind::FP8 && p.partition_tokens <= 2 * step)
    launch_kernel<KV, QK, NW, false, BS, PO_SPLIT, true, 2>(p, grid, stream);
  else
    launch_kernel<KV, QK, NW, false, BS, PO_SPLIT, true, 0>(p, grid, stream);
}

template <Kind KV, Kind QK, int BS>
int launch_typed(const DecodeLaunch& a) {
  Params p;
  p.out = a.out; p.q = a.q;
  p.k_cache = (const char*)a.k_cache; p.v_cache = (const char*)a.v_cache;
  p.block_tables = a.block_tables; p.seq_lens = a.seq_lens;
  p.part_m = a.part_m; p.part_l = a.part_l; p.part_o = a.part_o;
  p.num_heads = a.num_heads; p.num_kv_heads = a.num_kv_heads;
  p.max_blocks_per_seq = a.max_blocks_per_seq; p.num_blocks = a.num_blocks;
  p.num_partitions = a.num_partitions; p.partition_tokens = a.partition_tokens;
  p.group = a.num_heads / a.num_kv_heads;
  p.head_slices = (p.group + mw::kHeads - 1) / mw::kHeads;
  p.gqa_map = a.gqa_map;
  p.parts_per_wave = 1;
  const bool fp8 = KV == Kind::FP8;
  p.qk_scale = a.scale * (fp8 ? a.k_scale : 1.f) * kLog2e;
  p.v_scale = fp8 ? a.v_scale : 1.f;
  const int P = a.num_partitions;
  const unsigned items = (unsigned)(a.num_seqs * a.num_kv_heads * p.head_slices);
  if (P == 1) {
    // 4 wavefronts per workgroup: at 2-3 workgroups per CU the single-pass
    // grid of a large batch is resident in one round (B=64, ctx 4096:
    // 6.69 against 6.64 TB/s with 8)
    p.partition_tokens = 0x7fffffff;
    launch_kernel<KV, QK, 4, true, BS>(p, items, a.stream);
    return hipGetLastError() == hipSuccess ? 0 : 5;
  }
  // f16 partials: 2-byte f16 KV only, one partition per workgroup
  const bool f16_parts = a.part_o_dtype == (int)Kind::F16;
  if (f16_parts && KV != Kind::F16) return 3;
  if (!f16_parts && partition_per_wave<KV>(a.partition_tokens, (long)items * P)) {
    // as many partitions per wavefront as keep >= 2048 wavefronts (one
    // resident round at 2-3 per SIMD), at most 8
    p.parts_per_wave = (int)std::max(1L, std::min(8L, (long)items * P / 2048));
    const int runs = (P + p.parts_per_wave - 1) / p.parts_per_wave;
    // a wavefront's finished partitions wait in LDS while that keeps two
    // workgroups per CU (<= 64 KiB each)
    const int stash = (p.parts_per_wave - 1) * mw::stash_floats(std::min(p.group, mw::kHeads));
    p.stash_floats = 4 * stash * (int)sizeof(float) <= 64 * 1024 ? stash : 0;
    hipLaunchKernelGGL((wave_partition_kernel<KV, QK, BS>), dim3(items * ((runs + 3) / 4)), dim3(4 * kWave),
                       4 * p.stash_floats * sizeof(float), a.stream, p);
  } else if (items * P <= 128) {
    // a grid of at most half the CUs (the engine's one-sequence call inside
    // the v2 scratch: 8 partitions x 8 kv heads): 8 wavefronts per
    // workgroup (two per SIMD: the wavefront keeps its 256 registers), so
    // that each streams two of a 512-token partition's iterations
    if (f16_parts) {
      if constexpr (KV == Kind::F16) launch_late<KV, QK, 8, BS, Kind::F16>(p, items * P, a.stream);
    } else {
      launch_late<KV, QK, 8, BS, Kind::F32>(p, items * P, a.stream);
    }
  } else if (items * P <= 256) {
    // one workgroup per CU at most (one sequence in 32 partitions of 128
    // tokens x 8 kv heads): the items past the end exit late
    if (f16_parts) {
      if constexpr (KV == Kind::F16) launch_late<KV, QK, 4, BS, Kind::F16>(p, items * P, a.stream);
    } else {
      launch_late<KV, QK, 4, BS, Kind::F32>(p, items * P, a.stream);
    }
  } else if (f16_parts) {
    if constexpr (KV == Kind::F16) launch_kernel<KV, QK, 4, false, BS, Kind::F16>(p, items * P, a.stream);
  } else {
    launch_kernel<KV, QK, 4, false, BS>(p, items * P, a.stream);
  }
  if (hipGetLastError() != hipSuccess) return 5;
  return launch_lse_reduce(a.out, a.q_dtype, a.part_m, a.part_l, a.part_o, a.seq_lens,
                           a.num_seqs, a.num_heads, mw::kHead, P, a.partition_tokens, 0, 0, 0, a.stream,
                           a.part_o_dtype);
}

template <Kind KV, Kind QK>
int launch_bs(const DecodeLaunch& a) {
  switch (a.block_size) {
    case 8: return launch_typed<KV, QK, 8>(a);
    case 16: return launch_typed<KV, QK, 16>(a);
    case 32: return launch_typed<KV, QK, 32>(a);
    case 64: return launch_typed<KV, QK, 64>(a);
    case 128: return launch_typed<KV, QK, 128>(a);
    case 256: return launch_typed<KV, QK, 256>(a);
    default: return 3;
  }
}

}  // namespace

int launch_decode_mfma(const DecodeLaunch& a) {
  const Kind kv = (Kind)a.kv_dtype, qk = (Kind)a.q_dtype;
  if (!decode_uses_mfma(a.kv_dtype, a.num_heads, a.num_kv_heads, a.head_size, a.block_size)) return 3;
  const int tpi = kv == Kind::FP8 ? mw::tokens_per_iteration<Kind::FP8>() : mw::tokens_per_iteration<Kind::F16>();
  if (a.num_partitions > 1 && a.partition_tokens % tpi) return 3;
  if (kv == Kind::FP8 && qk == Kind::F16) return launch_bs<Kind::FP8, Kind::F16>(a);
  if (kv == Kind::FP8 && qk == Kind::BF16) return launch_bs<Kind::FP8, Kind::BF16>(a);
  if (kv == Kind::F16 && qk == Kind::F16) return launch_bs<Kind::F16, Kind::F16>(a);
  if (kv == Kind::BF16 && qk == Kind::BF16) return launch_bs<Kind::BF16, Kind::BF16>(a);
  return 3;
}

}  // namespace tl
