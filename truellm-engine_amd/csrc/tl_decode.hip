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

#include <math.h>

namespace tl {

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
constexpr float kLog2e = 1.4426950408889634f;

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
  int group, head_slices, gqa_map;
  float qk_scale;  // softmax scale * k dequant scale * log2(e)
  float v_scale;
};

template <Kind KV, int HEAD, int BS>
struct Geometry {
  static constexpr int E = KindInfo<KV>::bytes;
  static constexpr int CT = 16 / E;            // tokens per 16-byte chunk
  static constexpr int CPR = BS / CT;          // chunks per head-dim row of a block
  static constexpr int CPB = HEAD * CPR;       // chunks per block (one kv head)
  static constexpr int DPL = 8;                // loads per lane per wave iteration
  static constexpr int LPB = CPB / DPL;        // lanes per block
  static constexpr int BPI = kWave / LPB;      // blocks per wave iteration
  static constexpr int TPI = BPI * BS;         // tokens per wave iteration
  static constexpr int NI = kDecodeChunk / (kWaves * TPI);  // iterations per chunk
  static constexpr int R = LPB / CPR;          // lanes sharing one token set
  static_assert(BS % CT == 0, "block size must hold whole 16-byte chunks");
  static_assert(LPB >= 1 && LPB <= kWave && kWave % LPB == 0, "lane map");
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

__device__ __forceinline__ int head_of(const Params& p, int kvh, int gi) {
  return p.gqa_map ? kvh * p.group + gi : kvh + gi * p.num_kv_heads;
}

// KV: pool storage; QK: q / out storage; PO: partial-output storage.
template <Kind KV, Kind QK, Kind PO, int HEAD, int BS, int GT, bool FINAL>
__global__ __launch_bounds__(kThreads) void decode_kernel(Params p) {
  using Geo = Geometry<KV, HEAD, BS>;
  constexpr int CT = Geo::CT, CPR = Geo::CPR, LPB = Geo::LPB, R = Geo::R;
  constexpr int DPL = Geo::DPL, NI = Geo::NI, BPI = Geo::BPI;
  constexpr int NV = GT * CT;                  // partial scores per lane
  constexpr int KEPT = transpose_kept<NV, LPB / 2, CPR>();
  constexpr int NA = GT * DPL;                 // output accumulators per lane
  constexpr int BLOCK_BYTES = HEAD * BS * Geo::E;

  __shared__ float s_q[GT][HEAD];
  __shared__ float s_stat[3][GT];              // running max, running sum, rescale
  __shared__ __attribute__((aligned(16))) union {
    float score[GT][kDecodeChunk];
    float red[kWaves][GT][HEAD];
  } s_u;

  const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
  int bid = blockIdx.x;
  const int part = bid % p.num_partitions; bid /= p.num_partitions;
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

  float acc[NA];
#pragma unroll
  for (int i = 0; i < NA; ++i) acc[i] = 0.f;

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
  constexpr int N1 = transpose_kept<NA, 32, LPB>();
  if constexpr (LPB < kWave) ab += transpose_reduce<NA, 32, LPB>(acc, lane);
  constexpr int N2 = (CPR > 1) ? transpose_kept<N1, CPR / 2, 1>() : N1;
  if constexpr (CPR > 1) ab += transpose_reduce<N1, CPR / 2, 1>(acc, lane);
#pragma unroll
  for (int i = 0; i < N2; ++i) {
    const int a = ab + i, g = a / DPL, j = a % DPL;
    s_u.red[wave][g][j * R + dl] = acc[i];
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

// ---------------------------------------------------------------------------
// decode2_kernel: 2-byte KV (f16 / bf16), head 64 or 128, GQA groups of up to
// four q heads per workgroup.
//
// Each wavefront runs its own online softmax over the block pairs it owns,
// so the main loop has no workgroup barrier; the loads of the next iteration
// are issued while the current one computes.  Lane bits 2-3 pick the token
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
// ---------------------------------------------------------------------------
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

__device__ __forceinline__ uint32_t word(const u32x4& c, int w) {
  return w == 0 ? c.x : w == 1 ? c.y : w == 2 ? c.z : c.w;
}

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
// lane's 8-token run th of one block ([D][BS] layout, 16-byte chunks).
template <int KP, int CPR>
__device__ __forceinline__ void load_k_pairs(u32x4 (&kr)[KP][2], const char* blk, int dl, int th) {
#pragma unroll
  for (int j = 0; j < KP; ++j) {
    const int c = 2 * (dl + 16 * j) * CPR + th;
    kr[j][0] = load16_stream(blk + c * 16);
    kr[j][1] = load16_stream(blk + (c + CPR) * 16);
  }
}

// V rows d = 16 j + dl of the lane's 8-token run th of one block.
template <int VD, int CPR>
__device__ __forceinline__ void load_v_rows(u32x4 (&vr)[VD], const char* blk, int dl, int th) {
#pragma unroll
  for (int j = 0; j < VD; ++j) vr[j] = load16_stream(blk + ((16 * j + dl) * CPR + th) * 16);
}

template <Kind KV, Kind PO, int HEAD, int BS, int NW, bool FINAL>
__global__ __launch_bounds__(NW * kWave) void decode2_kernel(Params p) {
  constexpr int GT = 4;
  constexpr int CPR = BS / 8;             // 16-byte chunks per head-dim row of a block
  constexpr int BPI = 4 / CPR;            // blocks per wave iteration
  constexpr int TPI = BPI * BS;           // tokens per wave iteration
  constexpr int KP = HEAD / 32;           // head-dim pairs per lane (q.k)
  constexpr int VD = HEAD / 16;           // head dims per lane (p.v)
  constexpr int BLOCK_BYTES = HEAD * BS * 2;
  static_assert(TPI == 32, "four 8-token groups per wave iteration");
  using D2 = Dot2<KV>;

  __shared__ __attribute__((aligned(16))) uint32_t s_p[NW][4][GT][4];  // [token group][head][pair]
  __shared__ float s_m[NW][GT], s_l[NW][GT];
  __shared__ float s_acc[NW][GT][HEAD];

  const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
  const int tg = (lane >> 2) & 3, dl = (lane & 3) | ((lane >> 4) << 2);
  const int blk_in = tg / CPR, th = tg % CPR;
  const int g_lane = lane >> 4, tp = lane & 3;

  int bid = blockIdx.x;
  const int part = bid % p.num_partitions; bid /= p.num_partitions;
  const int hs = bid % p.head_slices;      bid /= p.head_slices;
  const int kvh = bid % p.num_kv_heads;
  const int seq = bid / p.num_kv_heads;
  const int L = p.seq_lens[seq];
  const int t0 = part * p.partition_tokens;
  if (!FINAL && t0 >= L) return;
  const int t1 = min(t0 + p.partition_tokens, L);

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
  const int64_t pool_stride = (int64_t)p.num_kv_heads * BLOCK_BYTES;
  const char* kbase0 = p.k_cache + (int64_t)kvh * BLOCK_BYTES;
  const char* vbase0 = p.v_cache + (int64_t)kvh * BLOCK_BYTES;

  // Pipeline: the K loads of iteration i+1 are issued as soon as the scores
  // of iteration i are formed, the V loads of i+1 once p.v of i is done, and
  // block-table entries are read two iterations ahead, so each wavefront
  // keeps one iteration of K/V in flight while it computes.  Holes load
  // block 0 and are masked.
  const int step = NW * TPI;
  int it = t0 + wave * TPI;
  int ph_cur = table_entry_bs<BS>(p, table, it + blk_in * BS, t1);
  int ph_next = table_entry_bs<BS>(p, table, it + step + blk_in * BS, t1);
  u32x4 kr[KP][2], vr[VD];
  if (it < t1) {
    load_k_pairs<KP, CPR>(kr, kbase0 + (int64_t)max(ph_cur, 0) * pool_stride, dl, th);
    load_v_rows<VD, CPR>(vr, vbase0 + (int64_t)max(ph_cur, 0) * pool_stride, dl, th);
  }

#pragma unroll 1
  for (; it < t1; it += step) {
    const int ph_nn = table_entry_bs<BS>(p, table, it + 2 * step + blk_in * BS, t1);
    const bool has_next = it + step < t1;
    const int blk_tok = it + blk_in * BS;                // first token of this lane's block

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
      load_k_pairs<KP, CPR>(kr, kbase0 + (int64_t)max(ph_next, 0) * pool_stride, dl, th);
    transpose_reduce_5410<GT * 8>(s, lane);             // -> (head g_lane, tokens 2tp, 2tp+1)

    const int tok = blk_tok + th * 8 + 2 * tp;
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
    s_p[wave][tg][g_lane][tp] = D2::pack(p0, p1);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    // ---- holes, and slots past the end of a partial block, may hold anything ----
    if (ph_cur < 0 || blk_tok + BS > t1) {
#pragma unroll
      for (int j = 0; j < VD; ++j) {
        uint32_t w4[4] = {vr[j].x, vr[j].y, vr[j].z, vr[j].w};
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const int t = blk_tok + th * 8 + 2 * w;
          if (ph_cur < 0 || t >= t1) w4[w] = 0u;
          else if (t + 1 >= t1) w4[w] &= 0xffffu;
        }
        vr[j] = u32x4{w4[0], w4[1], w4[2], w4[3]};
      }
    }

    // ---- p.v over token pairs ----
    u32x4 pp[GT];
#pragma unroll
    for (int g = 0; g < GT; ++g) pp[g] = *reinterpret_cast<const u32x4*>(&s_p[wave][tg][g][0]);
#pragma unroll
    for (int j = 0; j < VD; ++j)
#pragma unroll
      for (int g = 0; g < GT; ++g) {
        float a = acc[g][j];
#pragma unroll
        for (int w = 0; w < 4; ++w) a = D2::dot(word(pp[g], w), word(vr[j], w), a);
        acc[g][j] = a;
      }
    if (has_next)
      load_v_rows<VD, CPR>(vr, vbase0 + (int64_t)max(ph_next, 0) * pool_stride, dl, th);
    ph_cur = ph_next;
    ph_next = ph_nn;
  }

  // ---- wavefront totals: sums per head, acc reduced over token groups ----
  const float l_tot = row_sum(l_lane);
  float* accf = &acc[0][0];
  transpose_reduce<GT * VD, 8, 4>(accf, lane);         // -> head tg, dims 16 j + dl
#pragma unroll
  for (int j = 0; j < VD; ++j) s_acc[wave][tg][16 * j + dl] = accf[j];
  if (lane == 0) {
#pragma unroll
    for (int g = 0; g < GT; ++g) s_m[wave][g] = m_run[g];
  }
  if ((lane & 15) == 0) s_l[wave][g_lane] = l_tot;
  __syncthreads();

  for (int i = tid; i < GT * HEAD; i += NW * kWave) {
    const int g = i / HEAD, d = i % HEAD, gi = hs * GT + g;
    if (gi >= p.group) continue;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < NW; ++w) M = fmaxf(M, s_m[w][g]);
    float num = 0.f, den = 0.f;
    if (M != -INFINITY) {
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        const float f = (s_m[w][g] == -INFINITY) ? 0.f : exp2f(s_m[w][g] - M);
        num += f * s_acc[w][g][d];
        den += f * s_l[w][g];
      }
    }
    const float val = (den > 0.f) ? num / den : 0.f;
    const int head = head_of(p, kvh, gi);
    if constexpr (FINAL) {
      store_scalar<KV>(p.out, ((int64_t)seq * p.num_heads + head) * HEAD + d, val);
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

// Log-sum-exp merge of split-K partitions (paged_attention_v2.cu:131-170,
// restricted to the partitions a sequence actually has).
template <Kind QK, Kind PO, int HEAD>
__global__ __launch_bounds__(64) void lse_reduce_kernel(
    void* out, const float* part_m, const float* part_l, const void* part_o,
    const int32_t* seq_lens, int num_heads, int num_partitions, int partition_tokens) {
  const int sh = blockIdx.x, seq = sh / num_heads;
  const int L = seq_lens[seq];
  const int np = min(num_partitions, (L + partition_tokens - 1) / partition_tokens);
  const int64_t pb = (int64_t)sh * num_partitions;
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
    dim3 rgrid((unsigned)(a.num_seqs * a.num_heads));
    if (a.part_o_dtype == 0) {
      hipLaunchKernelGGL((decode_kernel<KV, QK, Kind::F32, HEAD, BS, GT, false>), grid,
                         dim3(kThreads), 0, a.stream, p);
      hipLaunchKernelGGL((lse_reduce_kernel<QK, Kind::F32, HEAD>), rgrid, dim3(64), 0, a.stream,
                         a.out, a.part_m, a.part_l, a.part_o, a.seq_lens, a.num_heads, P,
                         a.partition_tokens);
    } else {
      hipLaunchKernelGGL((decode_kernel<KV, QK, QK, HEAD, BS, GT, false>), grid, dim3(kThreads),
                         0, a.stream, p);
      hipLaunchKernelGGL((lse_reduce_kernel<QK, QK, HEAD>), rgrid, dim3(64), 0, a.stream, a.out,
                         a.part_m, a.part_l, a.part_o, a.seq_lens, a.num_heads, P,
                         a.partition_tokens);
    }
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
    dim3 rgrid((unsigned)(a.num_seqs * a.num_heads));
    if (a.part_o_dtype == 0) {
      hipLaunchKernelGGL((decode2_kernel<KV, Kind::F32, HEAD, BS, 4, false>), dim3(items * P),
                         dim3(4 * kWave), 0, a.stream, p);
      hipLaunchKernelGGL((lse_reduce_kernel<KV, Kind::F32, HEAD>), rgrid, dim3(64), 0, a.stream,
                         a.out, a.part_m, a.part_l, a.part_o, a.seq_lens, a.num_heads, P,
                         a.partition_tokens);
    } else {
      hipLaunchKernelGGL((decode2_kernel<KV, KV, HEAD, BS, 4, false>), dim3(items * P),
                         dim3(4 * kWave), 0, a.stream, p);
      hipLaunchKernelGGL((lse_reduce_kernel<KV, KV, HEAD>), rgrid, dim3(64), 0, a.stream, a.out,
                         a.part_m, a.part_l, a.part_o, a.seq_lens, a.num_heads, P,
                         a.partition_tokens);
    }
  }
  return hipGetLastError() == hipSuccess ? 0 : 5;
}

template <Kind KV, Kind QK, int HEAD, int BS>
int launch_gt(const DecodeLaunch& a) {
  const int group = a.num_heads / a.num_kv_heads;
  if (group == 1) return launch_typed<KV, QK, HEAD, BS, 1>(a);
  if constexpr ((KV == Kind::F16 || KV == Kind::BF16) && QK == KV && (HEAD == 64 || HEAD == 128)) {
    if (a.use_generic == 0) return launch_decode2<KV, HEAD, BS>(a);
  }
  return launch_typed<KV, QK, HEAD, BS, 4>(a);
}

template <Kind KV, Kind QK>
int launch_shape(const DecodeLaunch& a) {
  if (a.block_size == 16) {
    if (a.head_size == 128) return launch_gt<KV, QK, 128, 16>(a);
    if (a.head_size == 64) return launch_gt<KV, QK, 64, 16>(a);
    if (a.head_size == 256) return launch_gt<KV, QK, 256, 16>(a);
  } else if (a.block_size == 32) {
    if (a.head_size == 128) return launch_gt<KV, QK, 128, 32>(a);
  }
  return 3;
}

}  // namespace

int launch_decode(const DecodeLaunch& a) {
  const Kind kv = (Kind)a.kv_dtype, qk = (Kind)a.q_dtype;
  if (kv == Kind::F16 && qk == Kind::F16) return launch_shape<Kind::F16, Kind::F16>(a);
  if (kv == Kind::BF16 && qk == Kind::BF16) return launch_shape<Kind::BF16, Kind::BF16>(a);
  if (kv == Kind::FP8 && qk == Kind::F16) return launch_shape<Kind::FP8, Kind::F16>(a);
  if (kv == Kind::FP8 && qk == Kind::BF16) return launch_shape<Kind::FP8, Kind::BF16>(a);
  if (kv == Kind::F32 && qk == Kind::F32 && a.block_size == 16 && a.head_size == 128)
    return launch_gt<Kind::F32, Kind::F32, 128, 16>(a);
  return 3;
}

}  // namespace tl
