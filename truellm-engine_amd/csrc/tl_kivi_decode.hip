// tl_kivi_decode.hip -- paged-attention decode over KIVI INT4 KV (gfx950).
//
// A sequence of length L keeps its first Lq = kivi_quantized_len(L, R)
// tokens in 32-token INT4 pages (tl_kivi.hpp) and the rest (R .. R+31
// tokens) in the fp16 paged pool.  One workgroup owns one (sequence, kv
// head, partition of pages) and serves four q heads of the GQA group.
//
// Page wavefronts: per page a lane issues 20 16-byte loads (nibbles and
// step/zero of K and V), unpacks nibbles in registers with the fp16 magic
// number (0x6400 | n == 1024 + n), removes the 1024 and applies
// n * step + zero with packed fp16 ops, which yields MFMA operands directly:
//   q.k: v_mfma_f32_16x16x32_f16, A = dequantised K (rows: 16 tokens,
//        k: 32 channels), B = q (k: channels, columns: heads), 2 token tiles
//        x 4 channel blocks per page;
//   p.v: the q.k output leaves lane group r with tokens 4r..4r+3 and
//        16+4r..16+4r+3 of its head, exactly the token slots of the V page
//        layout, so the exp2 weights are packed straight into the A operand;
//        B = dequantised V (k: tokens, columns: 16 channels), 8 channel tiles.
// Online softmax per wavefront; running max per head from a permlane swap
// max over the four lane groups.
// Residual wavefront: the last wavefront of the partition that ends the
// sequence runs the fp16 window with the 2-byte decode (tl_decode_wave.hpp).
// The wavefront states are merged in LDS; several partitions are merged by
// the log-sum-exp reduce.
#include "tl_decode_wave.hpp"
#include "tl_device.hpp"
#include "tl_internal.hpp"
#include "tl_kivi.hpp"

namespace tl {

namespace {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));

struct KiviParams {
  Params base;                 // q, out, fp16 window, tables, partials, heads
  const uint8_t* pages;
  const int32_t* page_tables;
  int max_pages_per_seq, num_pages, residual_length, partition_pages;
};

// Eight nibbles (pairs at bits 4i and 16 + 4i) to eight fp16 values
// n * step + zero, step / zero given as four fp16 pairs.
__device__ __forceinline__ h8 dequant8(uint32_t w, const u32x4& step, const u32x4& zero) {
  h8 r;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t x = ((w >> (4 * i)) & 0x000F000Fu) | 0x64006400u;   // 1024 + n
    const h2 n = __builtin_bit_cast(h2, x) - (h2){(_Float16)1024.0f, (_Float16)1024.0f};
    const h2 v = __builtin_elementwise_fma(n, __builtin_bit_cast(h2, word(step, i)),
                                           __builtin_bit_cast(h2, word(zero, i)));
    r[2 * i] = v.x;
    r[2 * i + 1] = v.y;
  }
  return r;
}

__device__ __forceinline__ h8 as_h8(const u32x4& c) {
  typedef unsigned u4 __attribute__((ext_vector_type(4)));
  const u4 v = {c.x, c.y, c.z, c.w};
  return __builtin_bit_cast(h8, v);
}

__device__ __forceinline__ float swap16_max(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(unsigned, x),
                                                  __builtin_bit_cast(unsigned, x), false, false);
  return fmaxf(__builtin_bit_cast(float, (unsigned)r[0]), __builtin_bit_cast(float, (unsigned)r[1]));
}
__device__ __forceinline__ float swap32_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, x),
                                                  __builtin_bit_cast(unsigned, x), false, false);
  return fmaxf(__builtin_bit_cast(float, (unsigned)r[0]), __builtin_bit_cast(float, (unsigned)r[1]));
}

// One wavefront over pages pg_begin, pg_begin + pg_step, ... < pg_end.
__device__ __forceinline__ void kivi_pages_wave(const KiviParams& k, int seq, int kvh, int hs,
                                                int pg_begin, int pg_end, int pg_step,
                                                float* s_acc_w, float* s_m_w, float* s_l_w) {
  constexpr int GT = kWaveHeads;
  const Params& p = k.base;
  const int lane = threadIdx.x % kWave;
  const int grp = lane >> 4, u = lane & 15;     // lane group (k slots), row / column index

  // B operand of q.k: head u (real for u < GT), channels 32 m + 8 grp .. +7
  u32x4 qb[4];
  const int gi = hs * GT + u;
  const bool real = u < GT && gi < p.group;
  const uint16_t* qrow = (const uint16_t*)p.q +
      ((int64_t)seq * p.num_heads + (real ? head_of(p, kvh, gi) : 0)) * kKiviHead;
#pragma unroll
  for (int m = 0; m < 4; ++m)
    qb[m] = real ? load16(qrow + 32 * m + 8 * grp) : u32x4{0u, 0u, 0u, 0u};

  float m_run = -INFINITY, l_lane = 0.f;       // for head u
  f4 acc[8];                                   // rows: heads 4 grp + r, columns: channels 16 nt + u
#pragma unroll
  for (int nt = 0; nt < 8; ++nt) acc[nt] = (f4){0.f, 0.f, 0.f, 0.f};

  const int32_t* ptab = k.page_tables + (int64_t)seq * k.max_pages_per_seq;
#pragma unroll 1
  for (int pg = pg_begin; pg < pg_end; pg += pg_step) {
    const int pid = ptab[pg];
    if (pid < 0 || pid >= k.num_pages) continue;
    const uint8_t* base = k.pages + ((int64_t)pid * p.num_kv_heads + kvh) * kKiviPageBytes;
    u32x4 kn[2], ks[4], kz[4], vn[2], vs[4], vz[4];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) kn[tt] = load16_stream(base + (tt * 64 + lane) * 16);
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const uint8_t* kp = base + kKiviKParamOff + (grp + 4 * m) * 32;
      ks[m] = load16(kp);
      kz[m] = load16(kp + 16);
    }
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) vn[hh] = load16_stream(base + kKiviVNibOff + (hh * 64 + lane) * 16);
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const uint8_t* vp = base + kKiviVParamOff + (g * 4 + grp) * 32;
      vs[g] = load16(vp);
      vz[g] = load16(vp + 16);
    }

    // ---- q.k: S^T[token][head], token tiles 0 and 1 ----
    f4 s0 = (f4){0.f, 0.f, 0.f, 0.f}, s1 = s0;
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const h8 qm = as_h8(qb[m]);
      s0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(dequant8(word(kn[0], m), ks[m], kz[m]), qm, s0, 0, 0, 0);
      s1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(dequant8(word(kn[1], m), ks[m], kz[m]), qm, s1, 0, 0, 0);
    }
    // lane holds head u, tokens 4 grp + r (tile 0) and 16 + 4 grp + r (tile 1)
    float sc[8];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      sc[r] = real ? s0[r] * p.qk_scale : -INFINITY;
      sc[4 + r] = real ? s1[r] * p.qk_scale : -INFINITY;
    }
    float mx = sc[0];
#pragma unroll
    for (int i = 1; i < 8; ++i) mx = fmaxf(mx, sc[i]);
    mx = swap32_max(swap16_max(mx));
    const float m_new = fmaxf(m_run, mx);
    const float alpha = (m_run == m_new) ? 1.f : (m_run == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m_run - m_new));
    m_run = m_new;
    float pw[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) pw[i] = real ? __builtin_amdgcn_exp2f(sc[i] - m_new) : 0.f;
    l_lane = l_lane * alpha;
#pragma unroll
    for (int i = 0; i < 8; ++i) l_lane += pw[i];
    h8 pa;
#pragma unroll
    for (int i = 0; i < 8; ++i) pa[i] = (_Float16)pw[i];

    // rows of acc are heads 4 grp + r: rescale with those heads' alpha
#pragma unroll
    for (int r = 0; r < GT; ++r) {
      const float a_r = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, alpha), r));
      if (a_r != 1.f) {
#pragma unroll
        for (int nt = 0; nt < 8; ++nt) acc[nt][r] *= a_r;
      }
    }

    // ---- p.v over the page's 32 tokens, 8 channel tiles ----
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) {
      const h8 vb = dequant8(word(vn[nt / 4], nt % 4), vs[nt / 2], vz[nt / 2]);
      acc[nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa, vb, acc[nt], 0, 0, 0);
    }
  }

  // sums over the four lane groups for head u
  {
    const auto r16 = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(unsigned, l_lane),
                                                      __builtin_bit_cast(unsigned, l_lane), false, false);
    const float l2 = __builtin_bit_cast(float, (unsigned)r16[0]) + __builtin_bit_cast(float, (unsigned)r16[1]);
    const auto r32 = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, l2),
                                                      __builtin_bit_cast(unsigned, l2), false, false);
    const float l4 = __builtin_bit_cast(float, (unsigned)r32[0]) + __builtin_bit_cast(float, (unsigned)r32[1]);
    if (lane < GT) {
      s_m_w[lane] = m_run;
      s_l_w[lane] = l4;
    }
  }
  if (grp == 0) {
#pragma unroll
    for (int nt = 0; nt < 8; ++nt)
#pragma unroll
      for (int r = 0; r < GT; ++r) s_acc_w[r * kKiviHead + nt * 16 + u] = acc[nt][r];
  }
}

template <int NW, bool FINAL>
__global__ __launch_bounds__(NW * kWave) void kivi_decode_kernel(KiviParams k) {
  constexpr int GT = kWaveHeads;
  __shared__ __attribute__((aligned(16))) uint32_t s_p[NW][4][GT][4];
  __shared__ float s_m[NW][GT], s_l[NW][GT];
  __shared__ float s_acc[NW][GT][kKiviHead];

  const Params& p = k.base;
  const int tid = threadIdx.x, wave = tid / kWave;
  int bid = blockIdx.x;
  const int part = bid % p.num_partitions; bid /= p.num_partitions;
  const int hs = bid % p.head_slices;      bid /= p.head_slices;
  const int kvh = bid % p.num_kv_heads;
  const int seq = bid / p.num_kv_heads;
  const int L = p.seq_lens[seq];
  const int lq = kivi_quantized_len(L, k.residual_length);
  const int n_pages = min(lq / kKiviPageTokens, k.max_pages_per_seq);
  const int n_parts = FINAL ? 1 : max(1, (n_pages + k.partition_pages - 1) / k.partition_pages);
  if (part >= n_parts) return;
  const int pg0 = FINAL ? 0 : part * k.partition_pages;
  const int pg1 = FINAL ? n_pages : min(pg0 + k.partition_pages, n_pages);
  const bool has_res = (part == n_parts - 1) && L > lq;
  const int page_waves = has_res ? NW - 1 : NW;

  if (wave < page_waves) {
    kivi_pages_wave(k, seq, kvh, hs, pg0 + wave, pg1, page_waves, &s_acc[wave][0][0], &s_m[wave][0],
                    &s_l[wave][0]);
  } else {
    decode2_wave<Kind::F16, kKiviHead, 16>(p, seq, kvh, hs, lq, L, 32, &s_p[wave][0][0][0],
                                           &s_acc[wave][0][0], &s_m[wave][0], &s_l[wave][0]);
  }
  __syncthreads();
  combine_waves<Kind::F16, Kind::F32, kKiviHead, FINAL>(p, NW, &s_m[0][0], &s_l[0][0], &s_acc[0][0][0],
                                                        seq, kvh, hs, part, tid, NW * kWave);
}

}  // namespace

int launch_kivi_decode(const KiviDecodeLaunch& a) {
  KiviParams k;
  Params& p = k.base;
  p.out = a.out; p.q = a.q;
  p.k_cache = (const char*)a.k_cache; p.v_cache = (const char*)a.v_cache;
  p.block_tables = a.block_tables; p.seq_lens = a.seq_lens;
  p.part_m = a.part_m; p.part_l = a.part_l; p.part_o = a.part_o;
  p.num_heads = a.num_heads; p.num_kv_heads = a.num_kv_heads;
  p.max_blocks_per_seq = a.max_blocks_per_seq; p.num_blocks = a.num_blocks;
  p.num_partitions = a.num_partitions; p.partition_tokens = 0;
  p.group = a.num_heads / a.num_kv_heads;
  p.head_slices = (p.group + kWaveHeads - 1) / kWaveHeads;
  p.gqa_map = a.gqa_map;
  p.qk_scale = a.scale * kLog2e;
  p.v_scale = 1.f;
  k.pages = (const uint8_t*)a.pages; k.page_tables = a.page_tables;
  k.max_pages_per_seq = a.max_pages_per_seq; k.num_pages = a.num_pages;
  k.residual_length = a.residual_length; k.partition_pages = a.partition_pages;
  const unsigned items = (unsigned)(a.num_seqs * a.num_kv_heads * p.head_slices);
  if (a.num_partitions == 1) {
    hipLaunchKernelGGL((kivi_decode_kernel<8, true>), dim3(items), dim3(8 * kWave), 0, a.stream, k);
  } else {
    hipLaunchKernelGGL((kivi_decode_kernel<4, false>), dim3(items * a.num_partitions), dim3(4 * kWave),
                       0, a.stream, k);
    if (hipGetLastError() != hipSuccess) return 5;
    return launch_lse_reduce(a.out, (int)Kind::F16, a.part_m, a.part_l, a.part_o, 0, a.seq_lens,
                             a.num_seqs, a.num_heads, kKiviHead, a.num_partitions, 0,
                             a.residual_length, a.partition_pages, a.stream);
  }
  return hipGetLastError() == hipSuccess ? 0 : 5;
}

}  // namespace tl
