// tl_decode.hip -- paged-attention decode for gfx950.
//
// Replaces paged_attention_v1 (paged_attention_v1.cu:31-213) and
// paged_attention_v2 (paged_attention_v2.cu:31-251) with the attention they
// are meant to compute: out[s, h] = softmax(scale * q[s, h] . K^T) V over the
// seq_lens[s] tokens gathered through block_tables[s, :] from the
// [N, n_kv, D, BS] pools, one query token per sequence.
//
// One workgroup (4 wavefronts) owns one (sequence, kv head, partition) and
// serves every q head of that kv head's GQA group, so each KV byte is read
// from HBM once per group.  A partition is processed in chunks of 512
// tokens:
//   1. K pass: every lane issues 8 coalesced 16-byte loads (8 tokens of one
//      head dim each for 2-byte KV, 16 tokens for FP8), forms fp32 partial
//      q.k products for its tokens x heads, and a transpose-reduce across
//      the 16 lanes that share those tokens finishes the dot products.
//      Scores land in LDS.
//   2. softmax: one wavefront per head takes the chunk max, rescales the
//      running (max, sum) state and turns scores into exp2 weights in place.
//   3. V pass: the same load pattern over V; each lane accumulates
//      weight x value for its head dims, weights broadcast from LDS.
// After the last chunk the partial outputs are reduced across lanes and
// wavefronts.  With one partition the kernel writes the normalised output;
// with several (split-K) it writes (max, sum, normalised partial) per
// partition and lse_reduce_kernel merges them by log-sum-exp.
#include "tl_device.hpp"
#include "tl_internal.hpp"
#include "tl_decode_wave.hpp"
#include "tl_kivi.hpp"

#include <math.h>

namespace tl {

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;

// Lanes that share one block's chunks: CPB / 8 (8 loads per lane) when
// that divides the wavefront, else the largest power of two up to 64 that
// divides CPB (head sizes 80 and 96, 4-byte elements at head size 256).
constexpr int lanes_per_block(int cpb) {
  if (cpb % 8 == 0 && cpb / 8 <= kWave && kWave % (cpb / 8) == 0) return cpb / 8;
  int l = kWave;
  while (l > 1 && cpb % l) l >>= 1;
  return l;
}
constexpr int pow2_ceil(int n) {
  int p = 1;
  while (p < n) p <<= 1;
  return p;
}

template <Kind KV, int HEAD, int BS>
struct Geometry {
  static constexpr int E = KindInfo<KV>::bytes;
  static constexpr int CT = 16 / E;            // tokens per 16-byte chunk
  static constexpr int CPR = BS / CT;          // chunks per head-dim row of a block
  static constexpr int CPB = HEAD * CPR;       // chunks per block (one kv head)
  static constexpr int LPB = lanes_per_block(CPB);  // lanes per block
  static constexpr int DPL = CPB / LPB;        // loads per lane per wave iteration
  static constexpr int BPI = kWave / LPB;      // blocks per wave iteration
  static constexpr int TPI = BPI * BS;         // tokens per wave iteration
  static constexpr int NI = kDecodeChunk / (kWaves * TPI);  // iterations per chunk
  static constexpr int R = LPB / CPR;          // lanes sharing one token set
  static_assert(BS % CT == 0, "block size must hold whole 16-byte chunks");
  static_assert(LPB >= CPR && LPB <= kWave && kWave % LPB == 0 && LPB * DPL == CPB, "lane map");
  static_assert(NI >= 1 && kDecodeChunk % (kWaves * TPI) == 0, "chunk split");
};

template <Kind KV> struct ChunkUnpack;  // 16 bytes -> CT floats
template <> struct ChunkUnpack<Kind::F16> {
  __device__ __forceinline__ static void run(const u32x4& c, float* f) {
    Unpack<Kind::F16>::run(c.x, f); Unpack<Kind::F16>::run(c.y, f + 2);
    Unpack<Kind::F16>::run(c.z, f + 4); Unpack<Kind::F16>::run(c.w, f + 6);
  }
};
template <> struct ChunkUnpack<Kind::BF16> {
  __device__ __forceinline__ static void run(const u32x4& c, float* f) {
    Unpack<Kind::BF16>::run(c.x, f); Unpack<Kind::BF16>::run(c.y, f + 2);
    Unpack<Kind::BF16>::run(c.z, f + 4); Unpack<Kind::BF16>::run(c.w, f + 6);
  }
};
template <> struct ChunkUnpack<Kind::FP8> {
  __device__ __forceinline__ static void run(const u32x4& c, float* f) {
    Unpack<Kind::FP8>::run(c.x, f); Unpack<Kind::FP8>::run(c.y, f + 4);
    Unpack<Kind::FP8>::run(c.z, f + 8); Unpack<Kind::FP8>::run(c.w, f + 12);
  }
};
template <> struct ChunkUnpack<Kind::F32> {
  __device__ __forceinline__ static void run(const u32x4& c, float* f) {
    f[0] = __builtin_bit_cast(float, c.x); f[1] = __builtin_bit_cast(float, c.y);
    f[2] = __builtin_bit_cast(float, c.z); f[3] = __builtin_bit_cast(float, c.w);
  }
};

// KV: pool storage; QK: q / out storage; PO: partial-output storage.
template <Kind KV, Kind QK, Kind PO, int HEAD, int BS, int GT, bool FINAL>
__global__ __launch_bounds__(kThreads) void decode_kernel(Params p) {
  using Geo = Geometry<KV, HEAD, BS>;
  constexpr int CT = Geo::CT, CPR = Geo::CPR, LPB = Geo::LPB, R = Geo::R;
  constexpr int DPL = Geo::DPL, NI = Geo::NI, BPI = Geo::BPI;
  constexpr int NV = GT * CT;                  // partial scores per lane
  constexpr int KEPT = transpose_kept<NV, LPB / 2, CPR>();
  constexpr int NA = GT * DPL;                 // output accumulators per lane
  constexpr int NAP = pow2_ceil(NA);           // padded with zeros for the transpose-reduce
  constexpr int BLOCK_BYTES = HEAD * BS * Geo::E;

  __shared__ float s_q[GT][HEAD];
  __shared__ float s_stat[3][GT];              // running max, running sum, rescale
  __shared__ __attribute__((aligned(16))) union {
    float score[GT][kDecodeChunk];
    float red[kWaves][GT][HEAD];
  } s_u;

  const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
  int part;
  int bid = grid_item(p, part);
  const int hs = bid % p.head_slices;      bid /= p.head_slices;
  const int kvh = bid % p.num_kv_heads;
  const int seq = bid / p.num_kv_heads;

  const int L = p.seq_lens[seq];
  const int t0 = part * p.partition_tokens;
  if (!FINAL && t0 >= L) return;             // merged only up to ceil(L / PT)
  const int t1 = min(t0 + p.partition_tokens, L);

  // q of the heads this workgroup serves, pre-scaled, zero for padding heads
  for (int i = tid; i < GT * HEAD; i += kThreads) {
    const int g = i / HEAD, d = i % HEAD, gi = hs * GT + g;
    float v = 0.f;
    if (gi < p.group) {
      const int64_t off = ((int64_t)seq * p.num_heads + head_of(p, kvh, gi)) * HEAD + d;
      v = load_scalar<QK>(p.q, off) * p.qk_scale;
    }
    s_q[g][d] = v;
  }
  if (tid < GT) { s_stat[0][tid] = -INFINITY; s_stat[1][tid] = 0.f; s_stat[2][tid] = 1.f; }
  __syncthreads();

  const int bl = lane / LPB, li = lane % LPB, th = li % CPR, dl = li / CPR;
  float qr[GT][DPL];
#pragma unroll
  for (int g = 0; g < GT; ++g)
#pragma unroll
    for (int j = 0; j < DPL; ++j) qr[g][j] = s_q[g][j * R + dl];

  float acc[NAP];
#pragma unroll
  for (int i = 0; i < NAP; ++i) acc[i] = 0.f;

  const int32_t* table = p.block_tables + (int64_t)seq * p.max_blocks_per_seq;
  const int64_t head_off = (int64_t)kvh * BLOCK_BYTES + (int64_t)li * 16;
  const int64_t pool_stride = (int64_t)p.num_kv_heads * BLOCK_BYTES;

  for (int c0 = t0; c0 < t1; c0 += kDecodeChunk) {
    // ---------------- K pass: scores of this chunk into LDS ----------------
#pragma unroll 1
    for (int it = 0; it < NI; ++it) {
      const int blk_local = (it * kWaves + wave) * BPI + bl;     // block within chunk
      const int tok0 = c0 + blk_local * BS;                     // first token of block
      const int lb = tok0 / BS;
      int phys = -1;
      if (tok0 < t1 && lb < p.max_blocks_per_seq) phys = table[lb];
      if (phys >= p.num_blocks) phys = -1;
      float part_s[NV];
#pragma unroll
      for (int i = 0; i < NV; ++i) part_s[i] = 0.f;
      if (phys >= 0) {
        const char* base = p.k_cache + (int64_t)phys * pool_stride + head_off;
        u32x4 raw[DPL];
#pragma unroll
        for (int j = 0; j < DPL; ++j) raw[j] = load16(base + (int64_t)j * LPB * 16);
#pragma unroll
        for (int j = 0; j < DPL; ++j) {
          float k[CT];
          ChunkUnpack<KV>::run(raw[j], k);
#pragma unroll
          for (int g = 0; g < GT; ++g)
#pragma unroll
            for (int t = 0; t < CT; ++t) part_s[g * CT + t] += qr[g][j] * k[t];
        }
      }
      const int vb = transpose_reduce<NV, LPB / 2, CPR>(part_s, lane);
#pragma unroll
      for (int i = 0; i < KEPT; ++i) {
        const int v = vb + i, g = v / CT, t = v % CT;
        const int tl_ = blk_local * BS + th * CT + t;         // token within chunk
        const bool ok = phys >= 0 && (c0 + tl_) < t1;
        s_u.score[g][tl_] = ok ? part_s[i] : -INFINITY;
      }
    }
    __syncthreads();

    // ------------- softmax: chunk max, running state, exp2 weights ---------
    for (int g = wave; g < GT; g += kWaves) {
      float m = -INFINITY;
      for (int i = lane; i < kDecodeChunk; i += kWave) m = fmaxf(m, s_u.score[g][i]);
      m = wave_max<32, 1>(m);
      const float m_old = s_stat[0][g];
      const float m_new = fmaxf(m_old, m);
      float sum = 0.f;
      for (int i = lane; i < kDecodeChunk; i += kWave) {
        const float s = s_u.score[g][i];
        const float w = (s == -INFINITY) ? 0.f : exp2f(s - m_new);
        s_u.score[g][i] = w;
        sum += w;
      }
      sum = wave_sum<32, 1>(sum);
      if (lane == 0) {
        const float alpha = (m_old == -INFINITY) ? 0.f : exp2f(m_old - m_new);
        s_stat[0][g] = m_new;
        s_stat[1][g] = s_stat[1][g] * alpha + sum;
        s_stat[2][g] = alpha;
      }
    }
    __syncthreads();

    // ---------------- V pass: acc += w * v ----------------------------------
#pragma unroll
    for (int g = 0; g < GT; ++g) {
      const float alpha = s_stat[2][g];
#pragma unroll
      for (int j = 0; j < DPL; ++j) acc[g * DPL + j] *= alpha;
    }
#pragma unroll 1
    for (int it = 0; it < NI; ++it) {
      const int blk_local = (it * kWaves + wave) * BPI + bl;
      const int tok0 = c0 + blk_local * BS;
      const int lb = tok0 / BS;
      int phys = -1;
      if (tok0 < t1 && lb < p.max_blocks_per_seq) phys = table[lb];
      if (phys >= p.num_blocks) phys = -1;
      if (phys >= 0) {
        const char* base = p.v_cache + (int64_t)phys * pool_stride + head_off;
        u32x4 raw[DPL];
#pragma unroll
        for (int j = 0; j < DPL; ++j) raw[j] = load16(base + (int64_t)j * LPB * 16);
        float w[GT][CT];
        const int tl_ = blk_local * BS + th * CT;
#pragma unroll
        for (int g = 0; g < GT; ++g)
#pragma unroll
          for (int t = 0; t < CT; t += 4) {
            const f32x4 x = *reinterpret_cast<const f32x4*>(&s_u.score[g][tl_ + t]);
            w[g][t] = x.x; w[g][t + 1] = x.y; w[g][t + 2] = x.z; w[g][t + 3] = x.w;
          }
        // slots past the sequence end in a partial block may hold anything
        const int valid = t1 - (c0 + tl_);
#pragma unroll
        for (int j = 0; j < DPL; ++j) {
          float v[CT];
          ChunkUnpack<KV>::run(raw[j], v);
          if (valid < CT) {
#pragma unroll
            for (int t = 0; t < CT; ++t) v[t] = (t < valid) ? v[t] : 0.f;
          }
#pragma unroll
          for (int g = 0; g < GT; ++g) {
            float a = 0.f;
#pragma unroll
            for (int t = 0; t < CT; ++t) a += w[g][t] * v[t];
            acc[g * DPL + j] += a;
          }
        }
      }
    }
    __syncthreads();
  }

  // ------------- reduce acc over lanes (block slot, token half) ------------
  int ab = 0;
  constexpr int N1 = (LPB < kWave) ? transpose_kept<NAP, 32, LPB>() : NAP;
  if constexpr (LPB < kWave) ab += transpose_reduce<NAP, 32, LPB>(acc, lane);
  constexpr int N2 = (CPR > 1) ? transpose_kept<N1, CPR / 2, 1>() : N1;
  if constexpr (CPR > 1) ab += transpose_reduce<N1, CPR / 2, 1>(acc, lane);
#pragma unroll
  for (int i = 0; i < N2; ++i) {
    const int a = ab + i, g = a / DPL, j = a % DPL;
    if (a < NA) s_u.red[wave][g][j * R + dl] = acc[i];
  }
  __syncthreads();

  for (int i = tid; i < GT * HEAD; i += kThreads) {
    const int g = i / HEAD, d = i % HEAD, gi = hs * GT + g;
    if (gi >= p.group) continue;
    float o = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) o += s_u.red[w][g][d];
    const float l = s_stat[1][g];
    const float val = (l > 0.f) ? o * (p.v_scale / l) : 0.f;
    const int head = head_of(p, kvh, gi);
    if constexpr (FINAL) {
      store_scalar<QK>(p.out, ((int64_t)seq * p.num_heads + head) * HEAD + d, val);
    } else {
      const int64_t pi = ((int64_t)seq * p.num_heads + head) * p.num_partitions + part;
      store_scalar<PO>(p.part_o, pi * HEAD + d, val);
      if (d == 0) {
        p.part_m[pi] = (l > 0.f) ? s_stat[0][g] * (1.0f / kLog2e) : -INFINITY;
        p.part_l[pi] = l;
      }
    }
  }
}

template <Kind KV, Kind PO, int HEAD, int BS, int NW, bool FINAL>
__global__ __launch_bounds__(NW * kWave) void decode2_kernel(Params p) {
  constexpr int GT = kWaveHeads;
  __shared__ __attribute__((aligned(16))) uint32_t s_p[NW][2][4][GT][4];   // weights (bf16: high, low)
  __shared__ float s_m[NW][GT], s_l[NW][GT];
  __shared__ float s_acc[NW][GT][HEAD];

  const int tid = threadIdx.x, wave = tid / kWave;
  int part;
  int bid = grid_item(p, part);
  const int hs = bid % p.head_slices;      bid /= p.head_slices;
  const int kvh = bid % p.num_kv_heads;
  const int seq = bid / p.num_kv_heads;
  const int L = p.seq_lens[seq];
  const int t0 = part * p.partition_tokens;
  if (!FINAL && t0 >= L) return;
  const int t1 = min(t0 + p.partition_tokens, L);

  decode2_wave<KV, HEAD, BS>(p, seq, kvh, hs, t0 + wave * 32, t1, NW * 32, &s_p[wave][0][0][0][0],
                             &s_acc[wave][0][0], &s_m[wave][0], &s_l[wave][0]);
  __syncthreads();
  combine_waves<KV, PO, HEAD, FINAL, kWaveHeads, NW>(p, NW, &s_m[0][0], &s_l[0][0], &s_acc[0][0][0], seq, kvh, hs,
                                     part, tid, NW * kWave);
}

// Partitions a sequence has in the merge: ceil(L / partition_tokens), or,
// for KIVI (kivi_pages > 0), max(1, ceil(min(pages(L), kivi_max_pages) /
// kivi_pages)); never more than num_partitions.
__device__ __forceinline__ int merged_partitions(int L, int num_partitions, int partition_tokens, int kivi_residual,
                                                 int kivi_pages, int kivi_max_pages) {
  int np;
  if (kivi_pages > 0) {
    const int pages = min(kivi_quantized_len(L, kivi_residual) / kKiviPageTokens, kivi_max_pages);
    np = max(1, (pages + kivi_pages - 1) / kivi_pages);
  } else {
    np = (L + partition_tokens - 1) / partition_tokens;
  }
  return min(np, num_partitions);
}

// Log-sum-exp merge of split-K partitions (paged_attention_v2.cu:131-170,
// restricted to the partitions a sequence actually has).
template <Kind QK, Kind PO, int HEAD>
__global__ __launch_bounds__(64) void lse_reduce_kernel(
    void* out, const float* part_m, const float* part_l, const void* part_o,
    const int32_t* seq_lens, int num_heads, int num_partitions, int partition_tokens,
    int kivi_residual, int kivi_pages, int kivi_max_pages) {
  const int sh = blockIdx.x, seq = sh / num_heads;
  const int64_t pb = (int64_t)sh * num_partitions;
  // The partials are read for every partition slot (all in the workspace)
  // before the sequence length arrives; slots past the sequence's
  // partitions hold anything and are dropped by the conditions below.
  // (head sizes that are a multiple of 64: a thread owns channels
  // threadIdx.x + 64 c)
  constexpr int kEarly = HEAD % 64 == 0 ? 8 : 0, CH = HEAD / 64 > 0 ? HEAD / 64 : 1;
  float em[kEarly > 0 ? kEarly : 1], el[kEarly > 0 ? kEarly : 1], eo[kEarly > 0 ? kEarly : 1][CH];
#pragma unroll
  for (int i = 0; i < kEarly; ++i) {
    const bool in = i < num_partitions;
    em[i] = in ? part_m[pb + i] : 0.f;
    el[i] = in ? part_l[pb + i] : 0.f;
#pragma unroll
    for (int c = 0; c < CH; ++c)
      eo[i][c] = in ? load_scalar<PO>(part_o, (pb + i) * HEAD + threadIdx.x + 64 * c) : 0.f;
  }
  // the page count of a KIVI decode is clamped to the page table's width,
  // as in the decode kernel
  const int np = merged_partitions(seq_lens[seq], num_partitions, partition_tokens, kivi_residual, kivi_pages,
                                   kivi_max_pages);
  if (kEarly > 0 && np <= kEarly) {
    float M = -INFINITY;
#pragma unroll
    for (int i = 0; i < kEarly; ++i)
      if (i < np && el[i] > 0.f) M = fmaxf(M, em[i]);
    float W = 0.f;
#pragma unroll
    for (int i = 0; i < kEarly; ++i)
      if (i < np && el[i] > 0.f) W += el[i] * __expf(em[i] - M);
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      float o = 0.f;
#pragma unroll
      for (int i = 0; i < kEarly; ++i)
        if (i < np && el[i] > 0.f) o += el[i] * __expf(em[i] - M) * eo[i][c];
      store_scalar<QK>(out, (int64_t)sh * HEAD + threadIdx.x + 64 * c, (W > 0.f) ? o / W : 0.f);
    }
    return;
  }
  // every partition's (max, sum) and this thread's partial outputs in one go
  float M = -INFINITY;
  for (int i = 0; i < np; ++i)
    if (part_l[pb + i] > 0.f) M = fmaxf(M, part_m[pb + i]);
  float W = 0.f;
  for (int i = 0; i < np; ++i)
    if (part_l[pb + i] > 0.f) W += part_l[pb + i] * __expf(part_m[pb + i] - M);
  for (int d = threadIdx.x; d < HEAD; d += 64) {
    float o = 0.f;
    for (int i = 0; i < np; ++i) {
      const float l = part_l[pb + i];
      if (l > 0.f) o += l * __expf(part_m[pb + i] - M) * load_scalar<PO>(part_o, (pb + i) * HEAD + d);
    }
    store_scalar<QK>(out, (int64_t)sh * HEAD + d, (W > 0.f) ? o / W : 0.f);
  }
}

// Log-sum-exp merge for plans of more than 256 partitions: one workgroup
// of 4 wavefronts per (sequence, head).  The (max, sum) pairs are reduced
// over all threads; then wavefront w sums the partial outputs of
// partitions w, w + 4, ... (lane: head dims lane + 64 c), 4 partitions per
// round with their loads in flight together, and the 4 wavefronts' sums
// meet in LDS.
template <Kind QK, int HEAD, Kind PO = Kind::F32>
__global__ __launch_bounds__(256) void lse_reduce_long_kernel(
    void* out, const float* part_m, const float* part_l, const void* part_o, const int32_t* seq_lens,
    int num_heads, int num_partitions, int partition_tokens, int kivi_residual, int kivi_pages,
    int kivi_max_pages) {
  constexpr int CH = (HEAD + 63) / 64, U = 4;
  __shared__ float s_red[2][4];
  __shared__ float s_o[4][CH * 64];
  const int sh = blockIdx.x, seq = sh / num_heads;
  const int tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave;
  const int64_t pb = (int64_t)sh * num_partitions;
  const int np = merged_partitions(seq_lens[seq], num_partitions, partition_tokens, kivi_residual, kivi_pages,
                                   kivi_max_pages);
  float M = -INFINITY;
  for (int i = tid; i < np; i += 256)
    if (part_l[pb + i] > 0.f) M = fmaxf(M, part_m[pb + i]);
  M = wave_max<32, 1>(M);
  if (lane == 0) s_red[0][wave] = M;
  __syncthreads();
  M = fmaxf(fmaxf(s_red[0][0], s_red[0][1]), fmaxf(s_red[0][2], s_red[0][3]));
  float W = 0.f;
  for (int i = tid; i < np; i += 256) {
    const float l = part_l[pb + i];
    if (l > 0.f) W += l * __expf(part_m[pb + i] - M);
  }
  W = wave_sum<32, 1>(W);
  if (lane == 0) s_red[1][wave] = W;
  float o[CH];
#pragma unroll
  for (int c = 0; c < CH; ++c) o[c] = 0.f;
  for (int i0 = wave; i0 < np; i0 += 4 * U) {
    float coef[U], v[U][CH];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const bool in = i0 + 4 * u < np;
      const int i = in ? i0 + 4 * u : 0;       // every load stays inside the partials
      const float l = in ? part_l[pb + i] : 0.f;
      coef[u] = l > 0.f ? l * __expf(part_m[pb + i] - M) : 0.f;
#pragma unroll
      for (int c = 0; c < CH; ++c) {
        const int d = min(lane + 64 * c, HEAD - 1);
        v[u][c] = (in && lane + 64 * c < HEAD) ? load_scalar<PO>(part_o, (pb + i) * HEAD + d) : 0.f;
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int c = 0; c < CH; ++c) o[c] += coef[u] > 0.f ? coef[u] * v[u][c] : 0.f;
  }
#pragma unroll
  for (int c = 0; c < CH; ++c) s_o[wave][lane + 64 * c] = o[c];
  __syncthreads();
  W = s_red[1][0] + s_red[1][1] + s_red[1][2] + s_red[1][3];
  for (int d = tid; d < HEAD; d += 256) {
    const float sum = s_o[0][d] + s_o[1][d] + s_o[2][d] + s_o[3][d];
    store_scalar<QK>(out, (int64_t)sh * HEAD + d, W > 0.f ? sum / W : 0.f);
  }
}

// Log-sum-exp merge for plans of 9-256 partitions (FP8 at 512-token
// partitions: 64), and of 2-8 when the merges are fewer than the CUs: one
// workgroup of 4 wavefronts per (sequence, head).
// Every load is issued before the sequence length is known: thread i reads
// the (max, sum) pair of partition i, and wavefront w the partial outputs
// of partitions w, w + 4, ... (lane: head dims lane + 64 c), 16 at a time;
// slots past the sequence's partitions are read and then dropped (their
// weight is 0, and a select keeps stale values, NaN included, out of the
// sums).  The pairs are reduced over the workgroup, each partition's weight
// l exp(m - M) goes through LDS to the wavefront holding its outputs, and
// the 4 wavefronts' sums meet in LDS: one memory round trip, where reading
// the pairs, then the outputs round by round waited for each in turn
// (64 partitions: 12.3 us).  Within a wavefront the partitions are summed
// in ascending order.
template <Kind QK, int HEAD, Kind PO = Kind::F32>
__global__ __launch_bounds__(256) void lse_reduce_wide_kernel(
    void* out, const float* part_m, const float* part_l, const void* part_o, const int32_t* seq_lens,
    int num_heads, int num_partitions, int partition_tokens, int kivi_residual, int kivi_pages,
    int kivi_max_pages) {
  constexpr int CH = (HEAD + 63) / 64, U = 16, kMaxParts = 256;
  __shared__ float s_red[2][4];
  __shared__ float s_coef[kMaxParts + 4 * U];
  __shared__ float s_o[4][CH * 64];
  const int sh = blockIdx.x, seq = sh / num_heads;
  const int tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave;
  const int P = num_partitions;              // 9 .. kMaxParts
  const int64_t pb = (int64_t)sh * P;
  const float m_i = tid < P ? part_m[pb + tid] : -INFINITY;
  const float l_i = tid < P ? part_l[pb + tid] : 0.f;
  auto load_round = [&](float (&v)[U][CH], int i0) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int i = min(i0 + 4 * u, P - 1);  // every load stays inside the partials
#pragma unroll
      for (int c = 0; c < CH; ++c) v[u][c] = load_scalar<PO>(part_o, (pb + i) * HEAD + min(lane + 64 * c, HEAD - 1));
    }
  };
  float v[U][CH];
  load_round(v, wave);
  const int np = merged_partitions(seq_lens[seq], P, partition_tokens, kivi_residual, kivi_pages, kivi_max_pages);
  const bool ok = tid < np && l_i > 0.f;
  float M = wave_max<32, 1>(ok ? m_i : -INFINITY);
  if (lane == 0) s_red[0][wave] = M;
  __syncthreads();
  M = fmaxf(fmaxf(s_red[0][0], s_red[0][1]), fmaxf(s_red[0][2], s_red[0][3]));
  const float coef = ok ? l_i * __expf(m_i - M) : 0.f;
  s_coef[tid] = coef;
  if (tid < 4 * U) s_coef[kMaxParts + tid] = 0.f;
  const float W = wave_sum<32, 1>(coef);
  if (lane == 0) s_red[1][wave] = W;
  __syncthreads();
  float o[CH];
#pragma unroll
  for (int c = 0; c < CH; ++c) o[c] = 0.f;
  for (int i0 = wave; i0 < np; i0 += 4 * U) {
    if (i0 != wave) load_round(v, i0);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const float cu = s_coef[min(i0 + 4 * u, kMaxParts + 4 * U - 1)];
#pragma unroll
      for (int c = 0; c < CH; ++c) o[c] += cu > 0.f ? cu * v[u][c] : 0.f;
    }
  }
#pragma unroll
  for (int c = 0; c < CH; ++c)
    if (lane + 64 * c < HEAD) s_o[wave][lane + 64 * c] = o[c];
  __syncthreads();
  const float Wt = s_red[1][0] + s_red[1][1] + s_red[1][2] + s_red[1][3];
  for (int d = tid; d < HEAD; d += 256) {
    const float sum = s_o[0][d] + s_o[1][d] + s_o[2][d] + s_o[3][d];
    store_scalar<QK>(out, (int64_t)sh * HEAD + d, Wt > 0.f ? sum / Wt : 0.f);
  }
}

// Fewer (sequence, head) merges than CUs: the 4-wavefront merge also for
// plans of up to 8 partitions (one sequence of 32 heads, 8 f16 partials:
// 3.7 us less per call than the one-wavefront merge).
constexpr int kFewItems = 256;

template <Kind QK, int HEAD>
void launch_reduce(const DecodeLaunch& a) {
  const int P = a.num_partitions;
  const dim3 rgrid((unsigned)(a.num_seqs * a.num_heads));
  if (P > 256)
    hipLaunchKernelGGL((lse_reduce_long_kernel<QK, HEAD>), rgrid, dim3(256), 0, a.stream, a.out, a.part_m,
                       a.part_l, a.part_o, a.seq_lens, a.num_heads, P, a.partition_tokens, 0, 0, 0);
  else if (P > 8 || a.num_seqs * a.num_heads < kFewItems)
    hipLaunchKernelGGL((lse_reduce_wide_kernel<QK, HEAD>), rgrid, dim3(256), 0, a.stream, a.out, a.part_m,
                       a.part_l, a.part_o, a.seq_lens, a.num_heads, P, a.partition_tokens, 0, 0, 0);
  else
    hipLaunchKernelGGL((lse_reduce_kernel<QK, Kind::F32, HEAD>), rgrid, dim3(64), 0, a.stream, a.out, a.part_m,
                       a.part_l, a.part_o, a.seq_lens, a.num_heads, P, a.partition_tokens, 0, 0, 0);
}

template <Kind KV, Kind QK, int HEAD, int BS, int GT>
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
  p.head_slices = (p.group + GT - 1) / GT;
  p.gqa_map = a.gqa_map;
  p.qk_scale = a.scale * (KV == Kind::FP8 ? a.k_scale : 1.f) * kLog2e;
  p.v_scale = (KV == Kind::FP8) ? a.v_scale : 1.f;
  const int P = a.num_partitions;
  if (P == 1) {
    p.partition_tokens = 0x7fffffff;
    dim3 grid((unsigned)(a.num_seqs * a.num_kv_heads * p.head_slices));
    hipLaunchKernelGGL((decode_kernel<KV, QK, QK, HEAD, BS, GT, true>), grid, dim3(kThreads), 0,
                       a.stream, p);
  } else {
    dim3 grid((unsigned)(a.num_seqs * a.num_kv_heads * p.head_slices * P));
    hipLaunchKernelGGL((decode_kernel<KV, QK, Kind::F32, HEAD, BS, GT, false>), grid,
                       dim3(kThreads), 0, a.stream, p);
    launch_reduce<QK, HEAD>(a);
  }
  return hipGetLastError() == hipSuccess ? 0 : 5;
}

template <Kind KV, int HEAD, int BS>
int launch_decode2(const DecodeLaunch& a) {
  Params p;
  p.out = a.out; p.q = a.q;
  p.k_cache = (const char*)a.k_cache; p.v_cache = (const char*)a.v_cache;
  p.block_tables = a.block_tables; p.seq_lens = a.seq_lens;
  p.part_m = a.part_m; p.part_l = a.part_l; p.part_o = a.part_o;
  p.num_heads = a.num_heads; p.num_kv_heads = a.num_kv_heads;
  p.max_blocks_per_seq = a.max_blocks_per_seq; p.num_blocks = a.num_blocks;
  p.num_partitions = a.num_partitions; p.partition_tokens = a.partition_tokens;
  p.group = a.num_heads / a.num_kv_heads;
  p.head_slices = (p.group + 3) / 4;
  p.gqa_map = a.gqa_map;
  p.qk_scale = a.scale * kLog2e;
  p.v_scale = 1.f;
  const int P = a.num_partitions;
  const unsigned items = (unsigned)(a.num_seqs * a.num_kv_heads * p.head_slices);
  if (P == 1) {
    p.partition_tokens = 0x7fffffff;
    hipLaunchKernelGGL((decode2_kernel<KV, KV, HEAD, BS, 8, true>), dim3(items), dim3(8 * kWave), 0,
                       a.stream, p);
  } else {
    hipLaunchKernelGGL((decode2_kernel<KV, Kind::F32, HEAD, BS, 4, false>), dim3(items * P),
                       dim3(4 * kWave), 0, a.stream, p);
    launch_reduce<KV, HEAD>(a);
  }
  return hipGetLastError() == hipSuccess ? 0 : 5;
}

template <Kind KV, Kind QK, int HEAD, int BS>
int launch_gt(const DecodeLaunch& a) {
  const int group = a.num_heads / a.num_kv_heads;
  if (group == 1) return launch_typed<KV, QK, HEAD, BS, 1>(a);
  if constexpr ((KV == Kind::F16 || KV == Kind::BF16) && QK == KV && HEAD == 64)
    return launch_decode2<KV, HEAD, BS>(a);
  return launch_typed<KV, QK, HEAD, BS, 4>(a);
}

// The shapes of the FMA kernels: head sizes 64 and 256 (every pool dtype),
// 80 and 96 (2-byte pools), 128 for F32 pools; block size 16.  Head size
// 128 with a 2-byte or FP8 pool runs on the matrix cores.
template <Kind KV, Kind QK>
int launch_shape(const DecodeLaunch& a) {
  if (a.block_size != 16) return 3;
  switch (a.head_size) {
    case 64: return launch_gt<KV, QK, 64, 16>(a);
    case 256: return launch_gt<KV, QK, 256, 16>(a);
    case 80:
      if constexpr (KV == Kind::F16 || KV == Kind::BF16) return launch_gt<KV, QK, 80, 16>(a);
      return 3;
    case 96:
      if constexpr (KV == Kind::F16 || KV == Kind::BF16) return launch_gt<KV, QK, 96, 16>(a);
      return 3;
    case 128:
      if constexpr (KV == Kind::F32) return launch_gt<KV, QK, 128, 16>(a);
      return 3;
    default: return 3;
  }
}

}  // namespace

template <Kind QK, Kind PO>
void launch_lse_reduce_q(void* out, const float* part_m, const float* part_l, const void* part_o,
                         const int32_t* seq_lens, int num_seqs, int num_heads, int num_partitions,
                         int partition_tokens, int kivi_residual, int kivi_pages, int kivi_max_pages,
                         hipStream_t stream) {
  const dim3 grid((unsigned)(num_seqs * num_heads));
  if (num_partitions > 256)
    hipLaunchKernelGGL((lse_reduce_long_kernel<QK, 128, PO>), grid, dim3(256), 0, stream, out, part_m, part_l,
                       part_o, seq_lens, num_heads, num_partitions, partition_tokens, kivi_residual, kivi_pages,
                       kivi_max_pages);
  else if (num_partitions > 8 || num_seqs * num_heads < kFewItems)
    hipLaunchKernelGGL((lse_reduce_wide_kernel<QK, 128, PO>), grid, dim3(256), 0, stream, out, part_m, part_l,
                       part_o, seq_lens, num_heads, num_partitions, partition_tokens, kivi_residual, kivi_pages,
                       kivi_max_pages);
  else
    hipLaunchKernelGGL((lse_reduce_kernel<QK, PO, 128>), grid, dim3(64), 0, stream, out, part_m, part_l,
                       part_o, seq_lens, num_heads, num_partitions, partition_tokens, kivi_residual, kivi_pages,
                       kivi_max_pages);
}

int launch_lse_reduce(void* out, int q_dtype, const float* part_m, const float* part_l,
                      const void* part_o, const int32_t* seq_lens, int num_seqs,
                      int num_heads, int head_size, int num_partitions, int partition_tokens,
                      int kivi_residual, int kivi_pages, int kivi_max_pages, hipStream_t stream,
                      int part_o_dtype) {
  if (head_size != 128) return 3;
  if (q_dtype == (int)Kind::F16 && part_o_dtype == (int)Kind::F16)
    launch_lse_reduce_q<Kind::F16, Kind::F16>(out, part_m, part_l, part_o, seq_lens, num_seqs, num_heads,
                                              num_partitions, partition_tokens, kivi_residual, kivi_pages,
                                              kivi_max_pages, stream);
  else if (part_o_dtype != (int)Kind::F32)
    return 3;
  else if (q_dtype == (int)Kind::F16)
    launch_lse_reduce_q<Kind::F16, Kind::F32>(out, part_m, part_l, part_o, seq_lens, num_seqs, num_heads,
                                              num_partitions, partition_tokens, kivi_residual, kivi_pages,
                                              kivi_max_pages, stream);
  else if (q_dtype == (int)Kind::BF16)
    launch_lse_reduce_q<Kind::BF16, Kind::F32>(out, part_m, part_l, part_o, seq_lens, num_seqs, num_heads,
                                               num_partitions, partition_tokens, kivi_residual, kivi_pages,
                                               kivi_max_pages, stream);
  else
    return 3;
  return hipGetLastError() == hipSuccess ? 0 : 5;
}

int launch_decode(const DecodeLaunch& a) {
  const Kind kv = (Kind)a.kv_dtype, qk = (Kind)a.q_dtype;
  if (decode_uses_mfma(a.kv_dtype, a.num_heads, a.num_kv_heads, a.head_size, a.block_size))
    return launch_decode_mfma(a);
  if (kv == Kind::F16 && qk == Kind::F16) return launch_shape<Kind::F16, Kind::F16>(a);
  if (kv == Kind::BF16 && qk == Kind::BF16) return launch_shape<Kind::BF16, Kind::BF16>(a);
  if (kv == Kind::FP8 && qk == Kind::F16) return launch_shape<Kind::FP8, Kind::F16>(a);
  if (kv == Kind::FP8 && qk == Kind::BF16) return launch_shape<Kind::FP8, Kind::BF16>(a);
  if (kv == Kind::F32 && qk == Kind::F32) return launch_shape<Kind::F32, Kind::F32>(a);
  return 3;
}

}  // namespace tl
