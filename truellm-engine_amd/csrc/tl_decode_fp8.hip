// tl_decode_fp8.hip -- paged-attention decode over FP8 E4M3 KV on the matrix
// cores (head_size 128, block_size 16).
//
// An FP8 byte is one element, so per byte of HBM traffic there are twice as
// many multiply-adds as with 2-byte KV; the packed dot products of the
// 2-byte wavefront cannot keep up.  Here both contractions run on
// v_mfma_f32_16x16x32_f16 with the q heads as the 16 MFMA columns (up to 16
// heads per kv head read once), and the codes are widened to f16 by
// v_cvt_scalef32_pk_f16_fp8 with scale 1, which is exact: every E4M3 value,
// subnormals included, is an f16 value.  The dequant scales fold into the
// score scale (k_scale) and the output (v_scale), as the reference's
// dequantise-then-multiply does (cache_kernels.cu fp8 path; the scaled K/V are
// k_scale * code and v_scale * code).
//
// One wavefront iteration covers 64 tokens = 4 blocks of one kv head.
// Lanes are (m = lane & 15, kg = lane >> 4).
//   q.k, S^T[token][head] = K^T q^T: the A operand row m is token quad m
//     (block m >> 2, tokens 4 (m & 3) .. +3), tile i takes token i of every
//     quad.  Lane (m, kg) reads 32 dwords, rows d = 4 j + kg (j < 32) of its
//     quad: for each j the wavefront reads rows 4j .. 4j+3 of the 4 blocks,
//     64 contiguous bytes per block.  One v_perm_b32 stage pairs the bytes
//     of two rows per token, and the converter's (bytes 0,1) / (bytes 2,3)
//     halves are then exactly the f16 (d, d') pairs of one token, so the
//     K side costs 1 perm and 2 converts per 4 bytes and no further shuffle.
//     MFMA step s (k = 32) holds d = 32 s + 4 e + kg in slot e of group kg;
//     q is loaded in the same order.
//   Scores: lane (m, kg) holds head m, rows 4 kg + r of tile i = token
//     4 r + i of block kg (16 tokens of one block per lane).
//   p.v, O^T[d][head] = V P^T: A row = head dim (16 per tile, 8 tiles),
//     k = 32 tokens.  Lane (m, kg) loads 16 bytes, row d = 16 dt + m of
//     block kg, whose tokens 8 h .. 8 h + 7 are the slots of MFMA h; the
//     weights of the same tokens sit in the lane's own score registers, so
//     P^T needs no cross-lane move.
// Online softmax per lane (= per head): running max with lazy rescaling (the
// f16 weights exp2(s - m) stay below 2^8), fp32 sums and accumulators.
// Workgroups and the split-K / log-sum-exp protocol are those of the 2-byte
// decode: NW wavefronts stride over a partition's iterations and are merged
// in LDS.
#include "tl_device.hpp"
#include "tl_internal.hpp"
#include "tl_decode_wave.hpp"

#include <math.h>

namespace tl {

namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef unsigned u4v __attribute__((ext_vector_type(4)));
typedef unsigned u2v __attribute__((ext_vector_type(2)));

constexpr int kF8Head = 128;
constexpr int kF8Tokens = 64;       // tokens per wavefront iteration (4 blocks of 16)
constexpr int kF8Heads = 16;        // q heads per wavefront: the MFMA columns
constexpr int kF8BlockBytes = 128 * 16;
constexpr float kLazyRescale = 8.f; // rescale once the max grows by more than 2^8

// Two E4M3 codes (bytes 0,1 or 2,3 of w) to two f16, exactly.
template <bool HI>
__device__ __forceinline__ uint32_t f8x2(uint32_t w) {
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, HI));
}

__device__ __forceinline__ h8 as_h8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  const u4v v = {a, b, c, d};
  return __builtin_bit_cast(h8, v);
}

__device__ __forceinline__ f4 mfma16(h8 a, h8 b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ uint32_t ld_nt(const char* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(p));
}

// Max over the lanes l, l ^ 16, l ^ 32, l ^ 48.
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

struct PhysBlocks { int e[4]; };

__device__ __forceinline__ PhysBlocks table_blocks(const Params& p, const int32_t* table, int it, int t1) {
  PhysBlocks b;
#pragma unroll
  for (int i = 0; i < 4; ++i) b.e[i] = table_entry_bs<16>(p, table, it + 16 * i, t1);
  return b;
}

__device__ __forceinline__ int pick(const PhysBlocks& b, int i) {
  return i == 0 ? b.e[0] : i == 1 ? b.e[1] : i == 2 ? b.e[2] : b.e[3];
}

// K: 32 dwords, rows 4 j + kg of the lane's token quad (byte offset
// 64 j within the lane's base).  V: 8 x 16 bytes, rows 16 dt + m of block kg.
__device__ __forceinline__ void load_k(uint32_t (&kw)[32], const char* base) {
#pragma unroll
  for (int j = 0; j < 32; ++j) kw[j] = ld_nt(base + 64 * j);
}
__device__ __forceinline__ void load_v(u32x4 (&vr)[8], const char* base) {
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) vr[dt] = load16_stream(base + 256 * dt);
}

// Zeroes the bytes of tokens >= n (0 <= n <= 16) of a 16-token row.
__device__ __forceinline__ u32x4 keep_tokens(const u32x4& v, int n) {
  uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int k = n - 4 * i;   // bytes of this word to keep
    const uint32_t mask = k >= 4 ? 0xffffffffu : k <= 0 ? 0u : (0xffffffffu >> (32 - 8 * k));
    w[i] &= mask;
  }
  return u32x4{w[0], w[1], w[2], w[3]};
}

// One wavefront over its iterations (tokens first_it, first_it + step, ...
// below t1; first_it a multiple of 16).  Leaves s_acc_w [16][128]
// (unnormalised, v_scale applied), s_m_w [16] (log2 units), s_l_w [16].
template <Kind QK>
__device__ __forceinline__ void fp8_wave(const Params& p, int seq, int kvh, int hs, int first_it, int t1,
                                         int step, float* s_acc_w, float* s_m_w, float* s_l_w) {
  const int lane = threadIdx.x % kWave;
  const int m = lane & 15, kg = lane >> 4;

  // ---- q of head column m in MFMA order: slot (s, e) = dim 32 s + 4 e + kg ----
  const int gi = hs * kF8Heads + m;
  const bool hv = gi < p.group;
  const int head = hv ? head_of(p, kvh, gi) : 0;
  const uint16_t* qrow = (const uint16_t*)p.q + ((int64_t)seq * p.num_heads + head) * kF8Head;
  float qf[32];
  float qmax = 0.f;
#pragma unroll
  for (int s = 0; s < 4; ++s)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint16_t bits = hv ? qrow[32 * s + 4 * e + kg] : (uint16_t)0;
      const float v = QK == Kind::BF16 ? bf16_to_f32(bits) : f16_to_f32(bits);
      qf[8 * s + e] = v;
      qmax = fmaxf(qmax, fabsf(v));
    }
  // bf16 q is brought into f16 range by a power of two (exact): max |q| in
  // [2^14, 2^15).  f16 q is used as it is.
  int sh = 0;
  if constexpr (QK == Kind::BF16) {
    qmax = max_kg(qmax);
    if (qmax > 0.f && qmax < INFINITY) {
      int ex;
      frexpf(qmax, &ex);
      sh = 15 - ex;
    }
  }
  h8 qb[4];
#pragma unroll
  for (int s = 0; s < 4; ++s)
#pragma unroll
    for (int e = 0; e < 8; ++e) qb[s][e] = (_Float16)ldexpf(qf[8 * s + e], sh);
  const float qk_scale = p.qk_scale * ldexpf(1.f, -sh);

  f4 o[8];
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) o[dt] = f4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_lane = 0.f;

  const int32_t* table = p.block_tables + (int64_t)seq * p.max_blocks_per_seq;
  const int64_t pool_stride = (int64_t)p.num_kv_heads * kF8BlockBytes;
  const char* kbase0 = p.k_cache + (int64_t)kvh * kF8BlockBytes + 16 * kg + 4 * (m & 3);
  const char* vbase0 = p.v_cache + (int64_t)kvh * kF8BlockBytes + 16 * m;
  const int kb = m >> 2;   // the block of this lane's K quad

  int it = first_it;
  PhysBlocks cur = table_blocks(p, table, it, t1);
  PhysBlocks nxt = table_blocks(p, table, it + step, t1);
  uint32_t kw[32];
  u32x4 vr[8];
  if (it < t1) {
    load_k(kw, kbase0 + (int64_t)max(pick(cur, kb), 0) * pool_stride);
    load_v(vr, vbase0 + (int64_t)max(pick(cur, kg), 0) * pool_stride);
  }

#pragma unroll 1
  for (; it < t1; it += step) {
    const PhysBlocks nn = table_blocks(p, table, it + 2 * step, t1);
    const bool has_next = it + step < t1;

    // ---- q.k: 4 tiles (token i of each quad) x 4 MFMA steps ----
    f4 s[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) s[i] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      uint32_t a[4][4];   // [tile][f16 pair]
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        const uint32_t* w = &kw[8 * st + 4 * hf];   // rows 32 st + 16 hf + 4 c + kg
        // rows (c = 0, 1) and (2, 3) of this group, byte-paired per token
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
      for (int i = 0; i < 4; ++i) s[i] = mfma16(as_h8(a[i][0], a[i][1], a[i][2], a[i][3]), qb[st], s[i]);
    }
    if (has_next) load_k(kw, kbase0 + (int64_t)max(pick(nxt, kb), 0) * pool_stride);

    // ---- softmax: lane (m, kg) owns head m, tokens 4 r + i of block kg ----
    const int ph_v = pick(cur, kg);
    const int blk_tok = it + 16 * kg;
    const int n_ok = ph_v < 0 ? 0 : min(max(t1 - blk_tok, 0), 16);
    float sc[4][4];
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        sc[i][r] = (4 * r + i < n_ok) ? s[i][r] * qk_scale : -INFINITY;
        mx = fmaxf(mx, sc[i][r]);
      }
    mx = max_kg(mx);
    const float m_new = fmaxf(m_run, mx);
    if (__builtin_amdgcn_ballot_w64(m_new > m_run + kLazyRescale) != 0) {
      const float alpha = (m_run == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(m_run - m_new);
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) o[dt] *= alpha;
      l_lane *= alpha;
      m_run = m_new;
    }
    float pw[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        pw[i][r] = (4 * r + i < n_ok) ? __builtin_amdgcn_exp2f(sc[i][r] - m_run) : 0.f;
        l_lane += pw[i][r];
      }
    // P^T operands: MFMA h takes tokens 8 h .. 8 h + 7 = (r = 2 h, 2 h + 1) x (i = 0 .. 3)
    h8 pb[2];
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int e = 0; e < 8; ++e) pb[h][e] = (_Float16)pw[e & 3][2 * h + (e >> 2)];

    // ---- p.v: tokens past t1 and holes may hold any byte (NaN codes too) ----
    if (__builtin_amdgcn_ballot_w64(n_ok < 16) != 0) {
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) vr[dt] = keep_tokens(vr[dt], n_ok);
    }
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const u32x4 v = vr[dt];
      o[dt] = mfma16(as_h8(f8x2<false>(v.x), f8x2<true>(v.x), f8x2<false>(v.y), f8x2<true>(v.y)), pb[0], o[dt]);
      o[dt] = mfma16(as_h8(f8x2<false>(v.z), f8x2<true>(v.z), f8x2<false>(v.w), f8x2<true>(v.w)), pb[1], o[dt]);
    }
    if (has_next) load_v(vr, vbase0 + (int64_t)max(pick(nxt, kg), 0) * pool_stride);
    cur = nxt;
    nxt = nn;
  }

  // ---- wavefront state: head m, dims 16 dt + 4 kg + r ----
  const float l_tot = sum_kg(l_lane);
#pragma unroll
  for (int dt = 0; dt < 8; ++dt)
    *reinterpret_cast<f4*>(&s_acc_w[m * kF8Head + 16 * dt + 4 * kg]) = o[dt] * p.v_scale;
  if (kg == 0) {
    s_m_w[m] = m_run;
    s_l_w[m] = l_tot;
  }
}

template <Kind QK, Kind PO, int NW, bool FINAL>
__global__ __launch_bounds__(NW * kWave) void fp8_decode_kernel(Params p) {
  __shared__ __attribute__((aligned(16))) float s_acc[NW][kF8Heads][kF8Head];
  __shared__ float s_m[NW][kF8Heads], s_l[NW][kF8Heads];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  int bid = blockIdx.x;
  const int part = bid % p.num_partitions; bid /= p.num_partitions;
  const int hs = bid % p.head_slices;      bid /= p.head_slices;
  const int kvh = bid % p.num_kv_heads;
  const int seq = bid / p.num_kv_heads;
  const int L = p.seq_lens[seq];
  const int t0 = part * p.partition_tokens;
  if (!FINAL && t0 >= L) return;
  const int t1 = min(t0 + p.partition_tokens, L);

  fp8_wave<QK>(p, seq, kvh, hs, t0 + wave * kF8Tokens, t1, NW * kF8Tokens, &s_acc[wave][0][0], &s_m[wave][0],
               &s_l[wave][0]);
  __syncthreads();
  combine_waves<QK, PO, kF8Head, FINAL, kF8Heads>(p, NW, &s_m[0][0], &s_l[0][0], &s_acc[0][0][0], seq, kvh, hs,
                                                  part, tid, NW * kWave);
}

template <Kind QK>
int launch_q(const DecodeLaunch& a) {
  Params p;
  p.out = a.out; p.q = a.q;
  p.k_cache = (const char*)a.k_cache; p.v_cache = (const char*)a.v_cache;
  p.block_tables = a.block_tables; p.seq_lens = a.seq_lens;
  p.part_m = a.part_m; p.part_l = a.part_l; p.part_o = a.part_o;
  p.num_heads = a.num_heads; p.num_kv_heads = a.num_kv_heads;
  p.max_blocks_per_seq = a.max_blocks_per_seq; p.num_blocks = a.num_blocks;
  p.num_partitions = a.num_partitions; p.partition_tokens = a.partition_tokens;
  p.group = a.num_heads / a.num_kv_heads;
  p.head_slices = (p.group + kF8Heads - 1) / kF8Heads;
  p.gqa_map = a.gqa_map;
  p.qk_scale = a.scale * a.k_scale * kLog2e;
  p.v_scale = a.v_scale;
  const int P = a.num_partitions;
  const unsigned items = (unsigned)(a.num_seqs * a.num_kv_heads * p.head_slices);
  if (P == 1) {
    p.partition_tokens = 0x7fffffff;
    hipLaunchKernelGGL((fp8_decode_kernel<QK, QK, 8, true>), dim3(items), dim3(8 * kWave), 0, a.stream, p);
    return hipGetLastError() == hipSuccess ? 0 : 5;
  }
  hipLaunchKernelGGL((fp8_decode_kernel<QK, Kind::F32, 4, false>), dim3(items * P), dim3(4 * kWave), 0, a.stream,
                     p);
  if (hipGetLastError() != hipSuccess) return 5;
  return launch_lse_reduce(a.out, a.q_dtype, a.part_m, a.part_l, a.part_o, a.part_o_dtype, a.seq_lens,
                           a.num_seqs, a.num_heads, kF8Head, P, a.partition_tokens, 0, 0, a.stream);
}

}  // namespace

int launch_decode_fp8_mfma(const DecodeLaunch& a) {
  if (a.head_size != kF8Head || a.block_size != 16) return 3;
  if (a.num_partitions > 1 && (a.partition_tokens % kF8Tokens || a.part_o_dtype != 0)) return 3;
  if ((Kind)a.q_dtype == Kind::F16) return launch_q<Kind::F16>(a);
  if ((Kind)a.q_dtype == Kind::BF16) return launch_q<Kind::BF16>(a);
  return 3;
}

}  // namespace tl
