// tl_kivi_decode.hip -- paged-attention decode over KIVI INT4 / INT8 KV (gfx950).
//
// A sequence of length L keeps its first Lq = kivi_quantized_len(L, R)
// tokens in 32-token INT4 or INT8 pages (tl_kivi.hpp) and the rest (R .. R+31
// tokens) in the fp16 paged pool.  One workgroup owns one (sequence, kv
// head, partition of pages) and serves four q heads of the GQA group.
//
// Page wavefronts: per page a lane issues 5 (INT4) or 9 (INT8) 16-byte loads
// (codes and step/zero of K and V) and turns the codes into fp16 denormal
// MFMA operands (n * 2^-24) with masks and shifts; step and zero go into
// the other operand and a zero term, so that the MFMAs yield
// n * step + zero:
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
// sequence runs the fp16 window with the 2-byte decode (tl_decode_wave.hpp),
// the newest token, and then the partition's last 1/30 of the pages.
// The wavefront states are merged in LDS; several partitions are merged by
// the log-sum-exp reduce.
#include "tl_decode_wave.hpp"
#include "tl_device.hpp"
#include "tl_internal.hpp"
#include "tl_kivi.hpp"
#include "tl_kivi_page.hpp"

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
  PageJob job;                 // the step's append (kernels with APPEND)
  // keys held before RoPE (kernels with ROPE): fp32 tables [rope_max_pos,
  // 64], style 0 (pairs 2i, 2i + 1) or 1 (pairs i, i + 64)
  const float* rope_cos;
  const float* rope_sin;
  int rope_max_pos, rope_style;
};

// RoPE of a key pair (x0, x1) at angle (c, s), as the oracle's rotation:
// (x0 c - x1 s, x0 s + x1 c).
__device__ __forceinline__ void rope_rotate(float& x0, float& x1, float c, float s) {
  const float y0 = __builtin_fmaf(x0, c, -(x1 * s)), y1 = __builtin_fmaf(x0, s, x1 * c);
  x0 = y0;
  x1 = y1;
}
// cos / sin of pair i at position t (t past the tables: no rotation)
__device__ __forceinline__ void rope_cs1(const KiviParams& k, int t, int i, float& c, float& s) {
  const bool in = t >= 0 && t < k.rope_max_pos;
  const int64_t o = (int64_t)min(max(t, 0), k.rope_max_pos - 1) * (kKiviHead / 2) + i;
  const float cv = k.rope_cos[o], sv = k.rope_sin[o];
  c = in ? cv : 1.f;
  s = in ? sv : 0.f;
}

// Rotations of a lane's 32 channels 32 m + 8 grp + e (block m, element e:
// the channels of its q.k A and B operands) in packed f16.  Per channel, C
// = cos of the channel's pair and S = -sin for the pair's first channel,
// +sin for its second; then R x = C x + S partner(x) and R^T x = C x - S
// partner(x), where partner(x) is the pair's other channel: the neighbour
// in the same dword (style 0, pairs 2 i, 2 i + 1) or the same element of
// block m + 2 (style 1, pairs i, i + 64, blocks m and m + 2 together).
// The blocks one call rotates: style 0 block m, style 1 blocks m, m + 2.
template <bool TRANSPOSE>
__device__ __forceinline__ void rope_pair_blocks(h8& a, h8& b, const h8& ca, const h8& sa, const h8& cb,
                                                 const h8& sb) {
  const h8 a0 = a, b0 = b;
  a = TRANSPOSE ? a0 * ca - b0 * sa : a0 * ca + b0 * sa;
  b = TRANSPOSE ? b0 * cb - a0 * sb : b0 * cb + a0 * sb;
}
// The rotations of positions 0 .. 31 (a page's offsets) in LDS, one row per
// offset j in the layout of the page rows below: style 1 [cos | sin][pair],
// style 0 (cos, sin) of each pair in one dword (rope_rot_adjacent).  Each
// pair's cosine and sine once: 8 KiB, which leaves room for 32 more page
// rows than a table per channel.
constexpr int kRopeRows = kKiviPageTokens;
struct RopeTable {
  uint16_t cs[kRopeRows][kKiviHead];
};
// halves off .. off + 7 of offset j's row
__device__ __forceinline__ h8 rope_lds(const RopeTable& tb, int j, int off) {
  return *reinterpret_cast<const h8*>(&tb.cs[j][off]);
}

// The page rotations R_{32 p} of a workgroup's pages first .. first + count
// - 1 in LDS, filled at its start, the table rows converted to f16: per
// page, style 1 [cos | sin][pair], style 0 (cos, sin) of each pair in one
// dword.  The plan gives a workgroup at most kivi_page_rot_cap(bits) pages
// (tl_kivi.hpp), so every page's rotation is in the table.  Read from the
// tables where it is used, the q rotation waited for every page load in
// flight (the next pair's included), one memory round trip per page: INT4
// with keys before RoPE took 111.7 us per step, 88.1-88.6 with the
// coefficients taken as constants (timing only); and a fallback to the
// tables for pages past the LDS rows, never taken at 4096 tokens, still
// cost 2-3 us per step (the branch splits the q rotation's block).
struct PageRot {
  const uint16_t* cs;   // [count][2][64]
  int first, count;
};

// R x of the 4 adjacent pairs (x0, x1) of a block (style 0), dword d of cs
// holding (cos, sin) of pair d: (x0 c - x1 s, x1 c + x0 s), rounded as the
// product x c, then one fma, with the halves selected and
// negated by the packed ops' operand modifiers instead of a swap.
__device__ __forceinline__ void rope_rot_adjacent(h8& a, const u32x4& cs) {
  const u32x4 x = __builtin_bit_cast(u32x4, a);
  uint32_t o[4];
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    uint32_t t;
    // t = (x0 c, x1 c)
    asm("v_pk_mul_f16 %0, %1, %2 op_sel_hi:[1,0]" : "=v"(t) : "v"(word(x, d)), "v"(word(cs, d)));
    // (x1 (-s) + x0 c, x0 s + x1 c)
    asm("v_pk_fma_f16 %0, %1, %2, %3 op_sel:[1,1,0] op_sel_hi:[0,1,1] neg_lo:[0,1,0]"
        : "=v"(o[d]) : "v"(word(x, d)), "v"(word(cs, d)), "v"(t));
  }
  a = __builtin_bit_cast(h8, u32x4{o[0], o[1], o[2], o[3]});
}
// R^T x of the same: (x0 c + x1 s, x1 c - x0 s)
__device__ __forceinline__ void rope_rot_adjacent_t(h8& a, const u32x4& cs) {
  const u32x4 x = __builtin_bit_cast(u32x4, a);
  uint32_t o[4];
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    uint32_t t;
    asm("v_pk_mul_f16 %0, %1, %2 op_sel_hi:[1,0]" : "=v"(t) : "v"(word(x, d)), "v"(word(cs, d)));
    asm("v_pk_fma_f16 %0, %1, %2, %3 op_sel:[1,1,0] op_sel_hi:[0,1,1] neg_hi:[0,1,0]"
        : "=v"(o[d]) : "v"(word(x, d)), "v"(word(cs, d)), "v"(t));
  }
  a = __builtin_bit_cast(h8, u32x4{o[0], o[1], o[2], o[3]});
}
// C, -S and S of blocks m and m + 2 (style 1: pairs 32 m + 8 grp + e) from
// the LDS row of a page
__device__ __forceinline__ void rope_coef_row1(const uint16_t* row, int m, int grp, h8& c, h8& sa, h8& sb) {
  c = *reinterpret_cast<const h8*>(row + 32 * m + 8 * grp);
  sb = *reinterpret_cast<const h8*>(row + kKiviHead / 2 + 32 * m + 8 * grp);
  sa = -sb;
}

// Eight nibbles n_j (slot j at bit 16 (j & 1) + 4 (j >> 1)) as fp16
// denormals: a masked nibble pair is the fp16 pair (n * 2^-24, n' * 2^-24),
// or 16 n * 2^-24 for the pairs at bits 4 and 20 (slots 2, 3, 6, 7; the
// factor 16 is taken out of the other MFMA operand: slot_scale).  One shift
// and four ands per dword; the MFMA takes denormal fp16 inputs exactly and
// the 2^24 is restored in fp32.
__device__ __forceinline__ u32x4 nib8(uint32_t w) {
  const uint32_t y = w >> 8;
  return u32x4{w & 0x000F000Fu, w & 0x00F000F0u, y & 0x000F000Fu, y & 0x00F000F0u};
}

// Eight 8-bit codes n_j of two dwords (byte k of dword h holds element
// 4h + {0, 2, 1, 3}[k]) as fp16 denormals n * 2^-24, in element order.
__device__ __forceinline__ u32x4 byte8(uint32_t w0, uint32_t w1) {
  return u32x4{w0 & 0x00FF00FFu, (w0 >> 8) & 0x00FF00FFu, w1 & 0x00FF00FFu, (w1 >> 8) & 0x00FF00FFu};
}

constexpr float kTwo24 = 16777216.0f, kTwoM24 = 1.0f / 16777216.0f;

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

// One page's raw bytes as a lane loads them: its K and V code chunks (16
// bytes per token tile / channel half for INT4, 32 for INT8) and one
// 16-byte slice of the page's 1 KiB of (step, zero) parameters.
template <int BITS>
struct PageRaw {
  static constexpr int CW = KiviFmt<BITS>::kChunk / 16;
  u32x4 kn[2 * CW], vn[2 * CW], par;
};

// The q.k A operand of token tile tt, k block m, and the p.v B operand of
// channel tile nt, from a lane's code chunks.
template <int BITS>
__device__ __forceinline__ u32x4 k_codes(const PageRaw<BITS>& r, int tt, int m) {
  if constexpr (BITS == 8) {
    const u32x4& c = r.kn[2 * tt + m / 2];
    return byte8(word(c, 2 * (m % 2)), word(c, 2 * (m % 2) + 1));
  } else {
    return nib8(word(r.kn[tt], m));
  }
}
template <int BITS>
__device__ __forceinline__ u32x4 v_codes(const PageRaw<BITS>& r, int nt) {
  const int hh = nt / 4, m = nt % 4;
  if constexpr (BITS == 8) {
    const u32x4& c = r.vn[2 * hh + m / 2];
    return byte8(word(c, 2 * (m % 2)), word(c, 2 * (m % 2) + 1));
  } else {
    return nib8(word(r.vn[hh], m));
  }
}

// One page through a buffer descriptor (base = the page, 5120 bytes in
// range, so the hardware also bounds every access) and per-lane 32-bit
// offsets: the loads need no per-lane address registers; non-temporal (the
// page is read once per decode step).  A page that is not there (a hole,
// or a prefetch past the wavefront's last page) gets an empty range: its
// loads return zeros without a memory request, while the number of loads
// per iteration stays fixed.
// KV: 1 loads the K codes and the parameters, 2 the V codes, 3 both.
template <int BITS, int KV = 3>
__device__ __forceinline__ void load_page(PageRaw<BITS>& r, const uint8_t* page, bool there, unsigned off,
                                          unsigned par_off) {
  using F = KiviFmt<BITS>;
  constexpr int CW = PageRaw<BITS>::CW;
  constexpr unsigned kTile = 64u * F::kChunk;    // bytes of one token tile / channel half of codes
  const __amdgpu_buffer_rsrc_t rs = buffer_rsrc(page, there ? F::kBytes : 0);
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int w = 0; w < CW; ++w) {
      if constexpr (KV & 1) r.kn[CW * t + w] = buffer_load16(rs, unsigned(F::kKCodes) + t * kTile + CW * off + 16u * w);
      if constexpr (KV & 2) r.vn[CW * t + w] = buffer_load16(rs, unsigned(F::kVCodes) + t * kTile + CW * off + 16u * w);
    }
  if constexpr (KV & 1) r.par = buffer_load16(rs, par_off);
}

// Physical page of page index pg, or -1 (hole / past the end / outside the pool).
__device__ __forceinline__ int page_id(const KiviParams& k, const int32_t* ptab, int pg, int pg_end) {
  if (pg >= pg_end) return -1;
  const int pid = ptab[pg];
  return (pid < 0 || pid >= k.num_pages) ? -1 : pid;
}

__device__ __forceinline__ h8 hmul(const h8& a, const u32x4& b) { return a * as_h8(b); }

__device__ __forceinline__ f4 mfma(const h8& a, const h8& b, const f4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// Running state of one page wavefront.
struct PageState {
  f4 acc[8];       // 2^-24 * sum p step n:  rows heads 4 grp + r, columns channels 16 nt + u
  f4 cz;           // sum p zero:  rows heads 4 grp + r, column u = channel group (u < 4)
  float m_run;     // running max (log2 units) of head u
  float l_lane;    // this lane's share of the running sum of head u
};

// One pair of pages (a, b) for a wavefront whose lane (grp, u) holds
// qsc = q[head u] * scale * log2(e) at channels 32 m + 8 grp .. +7 and
// qss = qsc * slot_scale.
//
// q.k, per page and token tile:  S^T[t][u] = sum_c (n_tc step_c + zero_c) qsc_uc
//   = 2^24 sum_c (n_tc 2^-24) (qss_uc step_c) + sum_c zero_c qsc_uc;
// the zero term is one tile per page (A = zeros, rows all alike) scaled by
// 2^-24 to seed both token tiles, so the tiles hold 2^-24 S^T.
// p.v, per page and channel group g (32 channels, per-token step/zero):
//   O[u][c] = 2^24 sum_t (p_ut slot_scale step_tg) (n_tc 2^-24) + sum_t p_ut zero_tg;
// the first sum goes to acc (one MFMA per channel tile), the second to cz
// (one MFMA per page: B column g holds zero_tg).
// ROPE (keys held before RoPE): a lane dequantises its A operand itself
// (n step + zero in fp16, from the parameters in LDS) and rotates it by its
// row's offset in the page (packed f16 arithmetic), while q takes the
// page's own rotation: the tiles then hold S^T itself, and the zero tile
// and qss are not used.
template <int BITS, bool ROPE>
__device__ __forceinline__ void page_pair(PageState& st, const PageRaw<BITS>& ra, const PageRaw<BITS>& rb, bool oka,
                                          bool okb, const u32x4 (&qsc)[4], const u32x4 (&qss)[4],
                                          uint32_t* s_par_w, int lane, const h8& slot_scale,
                                          const KiviParams& k, int pga, int pgb, const RopeTable* s_rope,
                                          const PageRot& prot) {
  constexpr int GT = kWaveHeads;
  const int grp = lane >> 4, u = lane & 15;

  *reinterpret_cast<u32x4*>(s_par_w + lane * 4) = ra.par;
  *reinterpret_cast<u32x4*>(s_par_w + 256 + lane * 4) = rb.par;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

  // ---- q.k (tiles hold 2^-24 S^T; S^T with ROPE) ----
  f4 s[2][2];
  if constexpr (ROPE) {
    // Token t = t0 + j of page pg (t0 = 32 pg, j = 16 tt + u: this lane's A
    // row) is rotated by R_t = R_t0 R_j, so q . R_t k = (R_t0^T q) . (R_j k):
    // the page's rotation goes onto q, once per page, and R_j, the same for
    // every page, comes from the LDS table (exact for tables of angles
    // linear in the position, theta_i t, as RoPE's are; the launch requires
    // tables covering every position).  Coefficients are taken block by
    // block, so that few are live at a time.
    const int style = k.rope_style;
#pragma unroll
    for (int pi = 0; pi < 2; ++pi) {
      const PageRaw<BITS>& r = pi ? rb : ra;
      const uint32_t* par = s_par_w + pi * 256;
      const int pg = pi ? pgb : pga;
      // wave-uniform; in the table by the plan (the clamp keeps a page
      // past it, which the plan never gives, inside LDS)
      const int ci = min(max(pg - prot.first, 0), prot.count - 1);
      const uint16_t* row = prot.cs + ci * kKiviHead;
      h8 qp[4];
#pragma unroll
      for (int m = 0; m < 4; ++m) qp[m] = as_h8(qsc[m]);
      if (style == 0) {
#pragma unroll
        for (int m = 0; m < 4; ++m)   // pairs 16 m + 4 grp .. + 3
          rope_rot_adjacent_t(qp[m], *reinterpret_cast<const u32x4*>(row + 32 * m + 8 * grp));
      } else {
#pragma unroll
        for (int m = 0; m < 2; ++m) {
          h8 c, sa, sb;
          rope_coef_row1(row, m, grp, c, sa, sb);
          rope_pair_blocks<true>(qp[m], qp[m + 2], c, sa, c, sb);
        }
      }
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        const int j = 16 * tt + u;
        h8 kk[4];                                 // channels 32 m + 8 grp + e
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          const u32x4* kp = reinterpret_cast<const u32x4*>(par + (grp + 4 * m) * 8);
          // a code c in a half's low bits: 1024 + c as fp16, then c (16 n at
          // the INT4 slots 2, 3, 6, 7, which slot_scale takes back)
          u32x4 biased;
          if constexpr (BITS == 4) {
            // mask and bias in one v_and_or_b32 (the bias in a VGPR: one
            // scalar operand per instruction)
            const uint32_t w = word(r.kn[tt], m), y = w >> 8;
            auto and_or = [](uint32_t x, uint32_t mask) {
              uint32_t o;
              const uint32_t bias = 0x64006400u;
              asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(o) : "v"(x), "s"(mask), "v"(bias));
              return o;
            };
            biased = u32x4{and_or(w, 0x000F000Fu), and_or(w, 0x00F000F0u), and_or(y, 0x000F000Fu),
                           and_or(y, 0x00F000F0u)};
          } else {
            const u32x4 raw = k_codes(r, tt, m);
            biased = u32x4{raw.x | 0x64006400u, raw.y | 0x64006400u, raw.z | 0x64006400u, raw.w | 0x64006400u};
          }
          const h8 n = as_h8(biased) - (_Float16)1024.0f;
          kk[m] = n * (slot_scale * as_h8(kp[0])) + as_h8(kp[1]);
        }
        if (style == 0) {
#pragma unroll
          for (int m = 0; m < 4; ++m)
            rope_rot_adjacent(kk[m], __builtin_bit_cast(u32x4, rope_lds(*s_rope, j, 32 * m + 8 * grp)));
        } else {
#pragma unroll
          for (int m = 0; m < 2; ++m) {
            // blocks m and m + 2 hold the same pairs: one cosine row, and
            // sines that differ only in sign (INT4, with the bias below:
            // 94.4 -> 82.4 us per step)
            const h8 c = rope_lds(*s_rope, j, 32 * m + 8 * grp), sn = rope_lds(*s_rope, j, 64 + 32 * m + 8 * grp);
            rope_pair_blocks<false>(kk[m], kk[m + 2], c, -sn, c, sn);
          }
        }
        f4 acc = (f4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int m = 0; m < 4; ++m) acc = mfma(kk[m], qp[m], acc);
        s[pi][tt] = acc;
        // INT8 pages hold twice the code registers: one tile at a time
        if constexpr (BITS == 8) __builtin_amdgcn_sched_barrier(0);
      }
      // one page at a time (INT4, 4-wavefront workgroups at two per SIMD:
      // 112.5 against 118.5 us per step with one tile at a time; with both
      // pages interleaved the operands and coefficients spill)
      __builtin_amdgcn_sched_barrier(0);
    }
  } else {
#pragma unroll
  for (int pi = 0; pi < 2; ++pi) {
    const PageRaw<BITS>& r = pi ? rb : ra;
    const uint32_t* par = s_par_w + pi * 256;
    f4 zt = (f4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const u32x4* kp = reinterpret_cast<const u32x4*>(par + (grp + 4 * m) * 8);
      zt = mfma(as_h8(kp[1]), as_h8(qsc[m]), zt);
    }
    f4 t0 = zt * kTwoM24, t1 = t0;
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const u32x4* kp = reinterpret_cast<const u32x4*>(par + (grp + 4 * m) * 8);
      const h8 q2 = hmul(as_h8(qss[m]), kp[0]);
      t0 = mfma(as_h8(k_codes(r, 0, m)), q2, t0);
      t1 = mfma(as_h8(k_codes(r, 1, m)), q2, t1);
    }
    s[pi][0] = t0;
    s[pi][1] = t1;
  }
  }
  constexpr float kSc = ROPE ? 1.f : kTwo24;   // the tiles' scale of S^T
  // a hole's scores (its loads returned zeros) are dropped
  if (!oka) s[0][0] = s[0][1] = (f4){-INFINITY, -INFINITY, -INFINITY, -INFINITY};
  if (!okb) s[1][0] = s[1][1] = (f4){-INFINITY, -INFINITY, -INFINITY, -INFINITY};

  // ---- online softmax: lane holds head u, tokens 4 grp + r and 16 + 4 grp + r of each page ----
  float mx = fmaxf(fmaxf(fmaxf(s[0][0][0], s[0][0][1]), fmaxf(s[0][0][2], s[0][0][3])),
                   fmaxf(fmaxf(s[0][1][0], s[0][1][1]), fmaxf(s[0][1][2], s[0][1][3])));
  mx = fmaxf(mx, fmaxf(fmaxf(fmaxf(s[1][0][0], s[1][0][1]), fmaxf(s[1][0][2], s[1][0][3])),
                       fmaxf(fmaxf(s[1][1][0], s[1][1][1]), fmaxf(s[1][1][2], s[1][1][3]))));
  mx = swap32_max(swap16_max(mx)) * kSc;
  const float m_new = fmaxf(st.m_run, mx);
  const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
  const float alpha = __builtin_amdgcn_exp2f(st.m_run - m_use);
  st.m_run = m_new;
  h8 pw[2];
  float lsum = 0.f;
#pragma unroll
  for (int pi = 0; pi < 2; ++pi) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(s[pi][i >> 2][i & 3], kSc, -m_use));
      lsum += e;
      pw[pi][i] = (_Float16)e;
    }
  }
  st.l_lane = st.l_lane * alpha + lsum;

  // rows of acc / cz are heads 4 grp + r: rescale with those heads' alpha
  if (__builtin_amdgcn_ballot_w64(alpha != 1.f)) {
#pragma unroll
    for (int r = 0; r < GT; ++r) {
      const float a_r = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, alpha), r));
#pragma unroll
      for (int nt = 0; nt < 8; ++nt) st.acc[nt][r] *= a_r;
      st.cz[r] *= a_r;
    }
  }

  // ---- p.v (a hole's weights are zero) ----
#pragma unroll
  for (int pi = 0; pi < 2; ++pi) {
    const PageRaw<BITS>& r = pi ? rb : ra;
    const uint32_t* par = s_par_w + pi * 256 + 128;
    // zero term: B column u < 4 holds zero_tg of group g = u
    st.cz = mfma(pw[pi], as_h8(reinterpret_cast<const u32x4*>(par + ((u & 3) * 4 + grp) * 8)[1]), st.cz);
    const h8 pws = pw[pi] * slot_scale;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const h8 ps = hmul(pws, reinterpret_cast<const u32x4*>(par + (g * 4 + grp) * 8)[0]);
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int nt = 2 * g + h;
        st.acc[nt] = mfma(ps, as_h8(v_codes(r, nt)), st.acc[nt]);
      }
    }
  }
}

// One wavefront over its pages: page pairs (pg, pg + pg_step) at
// pg = pg_begin, pg_begin + 2 pg_step, ... below pg_end, the next pair's
// loads in flight while a pair is computed (two register sets, alternating).
// The pair's parameters go through the wavefront's 2 KiB LDS slot s_par_w
// (page a at 0, page b at 256 dwords; K params first, V params at 128).
// The page wavefronts' q operand as loaded: lane (grp, u) holds q[head u of
// the slice] at channels 32 m + 8 grp .. + 7, zero for the padding heads.
__device__ __forceinline__ void load_q_operand(const Params& p, int seq, int kvh, int hs, int lane,
                                               u32x4 (&q_raw)[4]) {
  const int grp = lane >> 4, u = lane & 15;
  const int gi = hs * kWaveHeads + u;
  const bool real = u < kWaveHeads && gi < p.group;
  const uint16_t* qrow = (const uint16_t*)p.q +
      ((int64_t)seq * p.num_heads + (real ? head_of(p, kvh, gi) : 0)) * kKiviHead;
  // loaded by every lane (a padding head reads head 0's row), then masked:
  // loads under the lane's condition each wait on their own
#pragma unroll
  for (int m = 0; m < 4; ++m) q_raw[m] = load16(qrow + 32 * m + 8 * grp);
#pragma unroll
  for (int m = 0; m < 4; ++m)
    if (!real) q_raw[m] = u32x4{0u, 0u, 0u, 0u};
}

// share_simd: raise the wavefront's priority on every other page pair (see
// kivi_decode_kernel).  early_ok: early_id is the table entry of page
// pg_begin + lane * pg_step, read by the caller ahead of time (unchecked;
// pages at or past pg_end and ids outside the pool are dropped here).
template <int BITS, bool ROPE>
__device__ __forceinline__ void kivi_pages_wave(const KiviParams& k, int seq, int kvh, int hs,
                                                int pg_begin, int pg_end, int pg_step,
                                                uint32_t* s_par_w, float* s_acc_w, float* s_m_w,
                                                float* s_l_w, bool share_simd, bool early_ok, int early_id,
                                                const RopeTable* s_rope, const PageRot& prot,
                                                const u32x4 (&q_raw)[4]) {
  constexpr int GT = kWaveHeads;
  const Params& p = k.base;
  const int lane = threadIdx.x % kWave;
  const int grp = lane >> 4, u = lane & 15;     // lane group (k slots), row / column index

  // B operand of q.k (q_raw: load_q_operand) times scale * log2(e)
  // INT4: the nibble pairs at bits 4 and 20 come out 16 times too large
  const _Float16 one = (_Float16)1.0f, sixteenth = (_Float16)(BITS == 8 ? 1.0f : 0.0625f);
  const h8 slot_scale = {one, one, sixteenth, sixteenth, one, one, sixteenth, sixteenth};
  u32x4 qsc[4], qss[4];   // q * scale * log2(e); the same times slot_scale
  const _Float16 qs = (_Float16)p.qk_scale;
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const h8 v = as_h8(q_raw[m]) * qs;
    qsc[m] = __builtin_bit_cast(u32x4, v);
    qss[m] = __builtin_bit_cast(u32x4, v * slot_scale);
  }

  PageState st;
  st.m_run = -INFINITY;
  st.l_lane = 0.f;
  st.cz = (f4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int nt = 0; nt < 8; ++nt) st.acc[nt] = (f4){0.f, 0.f, 0.f, 0.f};

  const int32_t* ptab = k.page_tables + (int64_t)seq * k.max_pages_per_seq;
  using F = KiviFmt<BITS>;
  const uint8_t* pool = k.pages + (int64_t)kvh * F::kBytes;
  const uint32_t pid_stride = uint32_t(p.num_kv_heads) * uint32_t(F::kBytes);
  // lane's chunk of each code block (16 bytes per lane for INT4, 32 for
  // INT8); lanes 0-31 take the K params, lanes 32-63 the V params
  const unsigned off = unsigned(lane) * 16u;
  const unsigned par_off = lane < 32 ? unsigned(F::kKParams) + off : unsigned(F::kVParams) + off - 512u;
  // Keys held before RoPE: a pair's V codes are loaded just before its own
  // q.k (the rotation hides their latency) instead of with its K one pair
  // ahead, so that two pairs' V codes are never held together (INT8: 190.5
  // -> 158.9 us per step, 38-46 registers spilled before; INT4: 112.7 ->
  // 111.9 us).
  constexpr bool kLateV = ROPE;
  constexpr int kAhead = kLateV ? 1 : 3;    // what a pair's early fetch loads
  auto load_kv = [&](auto kv_tag, PageRaw<BITS>& ra, PageRaw<BITS>& rb, int ia, int ib) {
    constexpr int KV = decltype(kv_tag)::value;
    // 32 x 32 -> 64-bit products keep the page base in scalar registers
    load_page<BITS, KV>(ra, pool + uint64_t(uint32_t(max(ia, 0))) * pid_stride, ia >= 0, off, par_off);
    load_page<BITS, KV>(rb, pool + uint64_t(uint32_t(max(ib, 0))) * pid_stride, ib >= 0, off, par_off);
  };

  // The wavefront's pages are pg_begin + o * pg_step, o = 0 .. n_mine - 1.
  // Their physical ids are read 64 at a time into one register (lane i: page
  // o = c0 + i) and taken out with readlane, so the loop issues no table
  // loads.  Page loads are unconditional (past the end, and for holes, with
  // an empty range): a fixed number of loads per iteration lets the
  // compiler wait only for the pair about to be used, not for the prefetch.
  const int n_mine = pg_begin < pg_end ? (pg_end - pg_begin + pg_step - 1) / pg_step : 0;
  PageRaw<BITS> r0a, r0b, r1a, r1b;
#pragma unroll 1
  for (int c0 = 0; c0 < n_mine; c0 += kWave) {
    const int cn = min(kWave, n_mine - c0);
    int idv;
    if (c0 == 0 && early_ok) {
      const bool in = pg_begin + lane * pg_step < pg_end && early_id >= 0 && early_id < k.num_pages;
      idv = in ? early_id : -1;
    } else {
      idv = page_id(k, ptab, pg_begin + (c0 + lane) * pg_step, pg_end);
    }
    auto id = [&](int o) { return o < cn ? __builtin_amdgcn_readlane(idv, o) : -1; };
    auto pg_of = [&](int o) { return pg_begin + (c0 + o) * pg_step; };   // page index (token position / 32)
    // the loads of pages o and o + 1 (with kLateV, fetch_v loads their V
    // codes just before they are used)
    auto fetch = [&](PageRaw<BITS>& ra, PageRaw<BITS>& rb, int o) {
      load_kv(std::integral_constant<int, kAhead>{}, ra, rb, id(o), id(o + 1));
    };
    auto fetch_v = [&](PageRaw<BITS>& ra, PageRaw<BITS>& rb, int o) {
      if constexpr (kLateV) load_kv(std::integral_constant<int, 2>{}, ra, rb, id(o), id(o + 1));
    };
    fetch(r0a, r0b, 0);
#pragma unroll 1
    for (int o = 0; o < cn; o += 4) {
      fetch_v(r0a, r0b, o);
      fetch(r1a, r1b, o + 2);
      if (share_simd) __builtin_amdgcn_s_setprio(1);
      page_pair<BITS, ROPE>(st, r0a, r0b, id(o) >= 0, id(o + 1) >= 0, qsc, qss, s_par_w, lane, slot_scale, k,
                            pg_of(o), pg_of(o + 1), s_rope, prot);
      if (o + 2 >= cn) break;
      fetch_v(r1a, r1b, o + 2);
      fetch(r0a, r0b, o + 4);
      if (share_simd) __builtin_amdgcn_s_setprio(0);
      page_pair<BITS, ROPE>(st, r1a, r1b, id(o + 2) >= 0, id(o + 3) >= 0, qsc, qss, s_par_w, lane, slot_scale, k,
                            pg_of(o + 2), pg_of(o + 3), s_rope, prot);
    }
  }

  // sums over the four lane groups for head u
  {
    const float l_lane = st.l_lane;
    const auto r16 = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(unsigned, l_lane),
                                                      __builtin_bit_cast(unsigned, l_lane), false, false);
    const float l2 = __builtin_bit_cast(float, (unsigned)r16[0]) + __builtin_bit_cast(float, (unsigned)r16[1]);
    const auto r32 = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, l2),
                                                      __builtin_bit_cast(unsigned, l2), false, false);
    const float l4 = __builtin_bit_cast(float, (unsigned)r32[0]) + __builtin_bit_cast(float, (unsigned)r32[1]);
    if (lane < GT) {
      s_m_w[lane] = st.m_run;
      s_l_w[lane] = l4;
    }
  }
  // O = 2^24 acc + cz[group]; cz of (head r, group g) sits in lane g of
  // group 0 and goes through the (now free) parameter slot
  float* s_cz = reinterpret_cast<float*>(s_par_w);
  if (lane < 4) {
#pragma unroll
    for (int r = 0; r < GT; ++r) s_cz[r * 4 + lane] = st.cz[r];
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  if (grp == 0) {
    // all of cz first: read between the stores (which may alias it, for
    // the compiler) each read waited for the LDS
    f4 cz[GT];
#pragma unroll
    for (int r = 0; r < GT; ++r) cz[r] = *reinterpret_cast<const f4*>(s_cz + r * 4);
#pragma unroll
    for (int nt = 0; nt < 8; ++nt)
#pragma unroll
      for (int r = 0; r < GT; ++r)
        s_acc_w[r * kKiviHead + nt * 16 + u] = __builtin_fmaf(st.acc[nt][r], kTwo24, cz[r][nt / 2]);
  }
}

// The window's newest token (position L - 1) as a state of its own: lane l
// holds channels 2l and 2l + 1 of its K and V (fp16 pairs).
struct NewestToken {
  uint32_t k, v;
  bool ok;      // false: a hole in the block table (the token is masked)
};

// From the fp16 pool, at the token's block-table position (BS: the block
// size, or 0 for p.block_size).
template <int BS>
__device__ __forceinline__ NewestToken newest_from_pool(const Params& p, int seq, int kvh, int pos, int lane) {
  const int bs = BS > 0 ? BS : p.block_size;
  const int lb = pos / bs;
  int ph = (pos >= 0 && lb < p.max_blocks_per_seq) ? p.block_tables[(int64_t)seq * p.max_blocks_per_seq + lb] : -1;
  if (ph >= p.num_blocks) ph = -1;
  NewestToken t{0u, 0u, ph >= 0};
  if (ph >= 0) {
    const int64_t off = (((int64_t)ph * p.num_kv_heads + kvh) * kKiviHead + 2 * lane) * bs + pos % bs;
    const uint16_t* kp = (const uint16_t*)p.k_cache + off;
    const uint16_t* vp = (const uint16_t*)p.v_cache + off;
    t.k = uint32_t(kp[0]) | (uint32_t(kp[bs]) << 16);
    t.v = uint32_t(vp[0]) | (uint32_t(vp[bs]) << 16);
  }
  return t;
}

// From the step's input row (the token that this launch appends).
__device__ __forceinline__ NewestToken newest_from_row(const PageJob& j, int seq, int kvh, int lane) {
  const int64_t row = ((int64_t)seq * j.num_kv_heads + kvh) * (kKiviHead / 2);
  return NewestToken{reinterpret_cast<const uint32_t*>(j.knew)[row + lane],
                     reinterpret_cast<const uint32_t*>(j.vnew)[row + lane], true};
}

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) x += __shfl_xor(x, o, kWave);
  return x;
}

// Replace 16-bit element e (0..7) of a 16-byte chunk.
__device__ __forceinline__ void put_half(u32x4& c, int e, uint32_t v) {
  const uint32_t sh = 16 * (e & 1), keep = ~(0xFFFFu << sh), ins = (v & 0xFFFFu) << sh;
  const int w = e / 2;
  c.x = w == 0 ? (c.x & keep) | ins : c.x;
  c.y = w == 1 ? (c.y & keep) | ins : c.y;
  c.z = w == 2 ? (c.z & keep) | ins : c.z;
  c.w = w == 3 ? (c.w & keep) | ins : c.w;
}

// The window's keys held before RoPE (decode2_wave's hook): each of the
// lane's 8 tokens rotated at its position.  Style 0 pairs rows 2 m and
// 2 m + 1 (pair m), style 1 rows c and c + 64 (kr[j] and kr[j + 2]).
// The window's rotation rows: (cos, sin) in f16 of each pair at the first
// position of the window's first kWinRows pages, filled by the residual
// wavefront once it knows the length.
constexpr int kWinRows = 8;

struct KiviWindowRope {
  static constexpr bool kActive = true;
  const KiviParams& k;
  const RopeTable* offs = nullptr;     // the offset rotations R_j (LDS)
  const uint32_t* wrows = nullptr;     // [kWinRows][64] page rotations R_{32 p}, p = wp0 + row (LDS)
  int wp0 = 0;
  template <int KP>
  __device__ void operator()(u32x4 (&kr)[KP][2], int tok0, int dl) const {
    static_assert(KP == 4, "head size 128");
    auto get = [](const u32x4& c, int e) { return f16_to_f32(uint16_t(word(c, e >> 1) >> (16 * (e & 1)))); };
    auto f2 = [](uint32_t w, float& lo, float& hi) {
      lo = f16_to_f32(uint16_t(w));
      hi = f16_to_f32(uint16_t(w >> 16));
    };
    // An iteration's 32 tokens are one page (the window starts on a page
    // boundary), so rp is wave-uniform.  Token t = 32 p + j is rotated by
    // R_{32 p} R_j, composed in fp32 from the two LDS tables (angles linear
    // in the position), instead of its table row read from memory, which
    // waited for every load in flight (INT8 with keys before RoPE: the
    // window was the residual wavefront's critical path).
    const int rp = (tok0 >> 5) - wp0;
    if (wrows != nullptr && rp >= 0 && rp < kWinRows) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int jj = (tok0 + e) & 31;
        if (k.rope_style == 0) {
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int m = dl + 16 * j;
            float cp, sp, cj, sj;
            f2(wrows[rp * 64 + m], cp, sp);
            f2(*reinterpret_cast<const uint32_t*>(&offs->cs[jj][2 * m]), cj, sj);
            const float c = __builtin_fmaf(cp, cj, -(sp * sj)), sn = __builtin_fmaf(sp, cj, cp * sj);
            float x0 = get(kr[j][0], e), x1 = get(kr[j][1], e);
            rope_rotate(x0, x1, c, sn);
            put_half(kr[j][0], e, f32_to_f16(x0));
            put_half(kr[j][1], e, f32_to_f16(x1));
            // one pair's reads and products at a time: held together across
            // the tokens they spill inside the window loop
            __builtin_amdgcn_sched_barrier(0);
          }
        } else {
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            // pairs pi, pi + 1: one dword of cosines, one of (positive) sines
            const int pi = 2 * (dl + 16 * j);
            float cj[2], sj[2];
            f2(*reinterpret_cast<const uint32_t*>(&offs->cs[jj][pi]), cj[0], cj[1]);
            f2(*reinterpret_cast<const uint32_t*>(&offs->cs[jj][pi + 64]), sj[0], sj[1]);
#pragma unroll
            for (int r = 0; r < 2; ++r) {
              float cp, sp;
              f2(wrows[rp * 64 + pi + r], cp, sp);
              const float c = __builtin_fmaf(cp, cj[r], -(sp * sj[r])), sn = __builtin_fmaf(sp, cj[r], cp * sj[r]);
              float x0 = get(kr[j][r], e), x1 = get(kr[j + 2][r], e);
              rope_rotate(x0, x1, c, sn);
              put_half(kr[j][r], e, f32_to_f16(x0));
              put_half(kr[j + 2][r], e, f32_to_f16(x1));
            }
            __builtin_amdgcn_sched_barrier(0);
          }
        }
      }
      return;
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int t = tok0 + e;
      if (k.rope_style == 0) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          float c, sn, x0 = get(kr[j][0], e), x1 = get(kr[j][1], e);
          rope_cs1(k, t, dl + 16 * j, c, sn);
          rope_rotate(x0, x1, c, sn);
          put_half(kr[j][0], e, f32_to_f16(x0));
          put_half(kr[j][1], e, f32_to_f16(x1));
        }
      } else {
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int r = 0; r < 2; ++r) {
            float c, sn, x0 = get(kr[j][r], e), x1 = get(kr[j + 2][r], e);
            rope_cs1(k, t, 2 * (dl + 16 * j) + r, c, sn);
            rope_rotate(x0, x1, c, sn);
            put_half(kr[j][r], e, f32_to_f16(x0));
            put_half(kr[j + 2][r], e, f32_to_f16(x1));
          }
      }
    }
  }
};

// The newest token's key (lane: channels 2 lane, 2 lane + 1) rotated at
// position t, for its score only (the pool keeps it as given).
__device__ __forceinline__ uint32_t rope_newest_key(const KiviParams& k, uint32_t kb, int t, int lane) {
  float x_lo = f16_to_f32(uint16_t(kb)), x_hi = f16_to_f32(uint16_t(kb >> 16));
  if (k.rope_style == 0) {
    float c, sn;
    rope_cs1(k, t, lane, c, sn);
    rope_rotate(x_lo, x_hi, c, sn);
  } else {
    // pairs (c, c + 64): lane l < 32 holds the first of pairs 2 l, 2 l + 1,
    // lane l + 32 the second
    const auto sw = __builtin_amdgcn_permlane32_swap(kb, kb, false, false);
    const uint32_t pb = lane < 32 ? (uint32_t)sw[1] : (uint32_t)sw[0];
    const float p_lo = f16_to_f32(uint16_t(pb)), p_hi = f16_to_f32(uint16_t(pb >> 16));
    const int i = 2 * (lane & 31);
    float c0, s0, c1, s1;
    rope_cs1(k, t, i, c0, s0);
    rope_cs1(k, t, i + 1, c1, s1);
    if (lane < 32) {
      float a = x_lo, b = p_lo, a1 = x_hi, b1 = p_hi;
      rope_rotate(a, b, c0, s0);
      rope_rotate(a1, b1, c1, s1);
      x_lo = a;
      x_hi = a1;
    } else {
      float a = p_lo, b = x_lo, a1 = p_hi, b1 = x_hi;
      rope_rotate(a, b, c0, s0);
      rope_rotate(a1, b1, c1, s1);
      x_lo = b;
      x_hi = b1;
    }
  }
  return uint32_t(f32_to_f16(x_lo)) | (uint32_t(f32_to_f16(x_hi)) << 16);
}

// The single-token state of the wavefront's q heads: max = the score
// (log2 units), sum = 1, unnormalised output = V.
__device__ __forceinline__ void newest_state(const Params& p, const NewestToken& t, int seq, int kvh, int hs,
                                             int lane, float* s_acc_w, float* s_m_w, float* s_l_w) {
  constexpr int GT = kWaveHeads;
#pragma unroll
  for (int g = 0; g < GT; ++g) {
    const int gi = hs * GT + g;
    const bool real = gi < p.group;
    const uint32_t q2 = real ? reinterpret_cast<const uint32_t*>(p.q)
                                   [((int64_t)seq * p.num_heads + head_of(p, kvh, gi)) * (kKiviHead / 2) + lane]
                             : 0u;
    const float sc = wave_sum(Dot2<Kind::F16>::dot(t.k, q2, 0.f)) * p.qk_scale;
    if (lane == 0) {
      s_m_w[g] = (t.ok && real) ? sc : -INFINITY;
      s_l_w[g] = (t.ok && real) ? 1.f : 0.f;
    }
    s_acc_w[g * kKiviHead + 2 * lane] = f16_to_f32(uint16_t(t.v));
    s_acc_w[g * kKiviHead + 2 * lane + 1] = f16_to_f32(uint16_t(t.v >> 16));
  }
}

// The new token into the fp16 pool, by one wavefront holding its channels
// 2 lane and 2 lane + 1 (t).  A token's 128 channels are 2-byte elements
// 2 BS bytes apart, and HBM3E has no byte masks: scattered 2-byte stores
// cost a step at batch 64 (block size 16) about 4 us (left in L2) or 1.4 us
// (written through), mostly in the memory's read-modify-writes.  So at
// block size 16 the block's rows of this kv head (128 channels x 16 slots,
// 4 KiB each of K and V) are read, the slot replaced, and the rows written
// back whole (about 0.3 us).  At other block sizes (BS = 0: p.block_size)
// each channel's 16-byte chunk holding the slot is rewritten (for block
// size 8 that is the whole row).  The other slots keep their bytes; no
// other writer may touch the block during the call (a block that a
// sequence appends to belongs to that sequence; the other head slices of
// the same (seq, kv head) write the same bytes).
template <int BS>
__device__ __forceinline__ void store_newest(const PageJob& j, const NewestToken& t, int seq, int kvh, int lane) {
  const int32_t slot = j.slots[seq];
  if constexpr (BS != 16) {
    const int bs = j.block_size;
    const int blk = slot >= 0 ? slot / bs : -1;
    if (blk < 0 || blk >= j.num_blocks) return;
    const int s = slot % bs;
    const int64_t base = ((int64_t)blk * j.num_kv_heads + kvh) * kKiviHead * bs + (s & ~7);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int64_t off = base + (int64_t)(2 * lane + h) * bs;
      u32x4 kc = load16(j.k_cache + off), vc = load16(j.v_cache + off);
      put_half(kc, s & 7, h ? t.k >> 16 : t.k);
      put_half(vc, s & 7, h ? t.v >> 16 : t.v);
      *reinterpret_cast<u32x4*>(j.k_cache + off) = kc;
      *reinterpret_cast<u32x4*>(j.v_cache + off) = vc;
    }
    return;
  }
  const int blk = slot >= 0 ? slot / BS : -1;
  if (blk < 0 || blk >= j.num_blocks) return;
  const int64_t base = ((int64_t)blk * j.num_kv_heads + kvh) * kKiviHead * BS;
  const int s = slot % BS;
  // chunk i = 4 lane + r: channel i / 2 (= 2 lane + r / 2), slots 8 (i % 2) .. +7
  u32x4 kr[4], vr[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    kr[r] = load16(j.k_cache + base + 8 * (4 * lane + r));
    vr[r] = load16(j.v_cache + base + 8 * (4 * lane + r));
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    if ((r & 1) == s / 8) {
      put_half(kr[r], s % 8, (r & 2) ? t.k >> 16 : t.k);
      put_half(vr[r], s % 8, (r & 2) ? t.v >> 16 : t.v);
    }
    *reinterpret_cast<u32x4*>(j.k_cache + base + 8 * (4 * lane + r)) = kr[r];
    *reinterpret_cast<u32x4*>(j.v_cache + base + 8 * (4 * lane + r)) = vr[r];
  }
}

// Slots 0 .. NW-1: one per wavefront; slot NW: the newest token; slot
// NW + 1: the residual wavefront's pages.
template <int NW>
struct KiviDecodeSmem {
  uint32_t p[NW][512];                       // per wave: weights or page params
  int piece_pid;                             // build-ahead: the piece's page slot, or -1
  float m[NW + 2][kWaveHeads], l[NW + 2][kWaveHeads];
  float acc[NW + 2][kWaveHeads][kKiviHead];
};

// One decode workgroup.  The residual wavefront runs the window [lq, L - 1)
// from the pool, the newest token (L - 1) as a state of its own, and then
// the range's last pages (slot NW + 1).
// With APPEND the workgroup also does the step's append for its (sequence,
// kv head), and nothing in the launch reads a byte that it writes:
//   * the page that the new token completes (if any) is built first, by the
//     workgroup of the last partition, whose page range holds that page; the
//     page never holds the new token's pool slot (with R = 0 the new token
//     is in the page and is read from the input row);
//   * the newest-token state takes K and V from the input row (when the
//     slot is >= 0, i.e. the token is written), and the residual wavefront
//     stores the token to its slot after its window (wavefront 0 of the
//     last partition when the sequence has no window).  The slot must be the
//     token's block-table position, as an append step's slot is.
// With a GQA group over several head slices each slice's workgroup writes
// the same bytes.
// Two wavefronts per SIMD (at most 256 registers, VGPRs and AGPRs together):
// with 4-wavefront workgroups the compiler would otherwise take more and
// halve the occupancy.
// BS: the fp16 pool's block size, 16, or 0 for any other (read from the
// launch at run time).
template <int NW, bool FINAL, bool APPEND, int BITS, bool ROPE, int BS>
__global__ __launch_bounds__(NW * kWave, 2) void kivi_decode_kernel(KiviParams k) {
  using Smem = KiviDecodeSmem<NW>;
  using Build = KiviBuildSmem<BITS>;
  constexpr size_t kLds = (APPEND && sizeof(Build) > sizeof(Smem)) ? sizeof(Build) : sizeof(Smem);
  __shared__ __attribute__((aligned(16))) unsigned char s_raw[kLds];
  Smem& sd = *reinterpret_cast<Smem*>(s_raw);

  const Params& p = k.base;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);   // wave-uniform (SGPR)
  int part;
  int bid = grid_item(p, part);
  // keys held before RoPE: the rotations of a page's 32 offsets and of the
  // workgroup's pages, built once per workgroup (L2 reads, all issued
  // together)
  const RopeTable* s_rope = nullptr;
  PageRot prot{nullptr, 0, 0};
  uint32_t* s_wrot = nullptr;          // the window's page rotations (residual wavefront)
  if constexpr (ROPE) {
    __shared__ __attribute__((aligned(16))) RopeTable s_rope_tb;
    constexpr int kCap = kivi_page_rot_cap(BITS);
    __shared__ __attribute__((aligned(16))) uint16_t s_prot[kCap][2][kKiviHead / 2];
    __shared__ __attribute__((aligned(16))) uint32_t s_wrot_tb[kWinRows][kKiviHead / 2];
    s_wrot = &s_wrot_tb[0][0];
    constexpr int kN = kRopeRows * (kKiviHead / 2) / (NW * kWave);
    static_assert(kRopeRows * (kKiviHead / 2) % (NW * kWave) == 0, "whole rounds");
    // the page rotations: rows 32 p of pages pg_first .. pg_first + kCap - 1,
    // 16 bytes of one table per load (kQ per row)
    constexpr int kQ = kKiviHead / 2 / 4;
    constexpr int kPR = kCap * 2 * kQ / (NW * kWave);
    static_assert(kCap * 2 * kQ % (NW * kWave) == 0, "whole rounds");
    const int pg_first = FINAL ? 0 : part * k.partition_pages;
    f4 rv[kPR];
#pragma unroll
    for (int r = 0; r < kPR; ++r) {
      const int i = tid + r * NW * kWave, pgi = i / (2 * kQ), w = i % (2 * kQ), tab = w / kQ, q4 = w % kQ;
      const int t = 32 * (pg_first + pgi);
      const bool in = t < k.rope_max_pos;
      const int64_t o = (int64_t)min(t, k.rope_max_pos - 1) * (kKiviHead / 2) + 4 * q4;
      const f4 v = *reinterpret_cast<const f4*>((tab ? k.rope_sin : k.rope_cos) + o);
      rv[r] = in ? v : (tab ? (f4){0.f, 0.f, 0.f, 0.f} : (f4){1.f, 1.f, 1.f, 1.f});
    }
    float cv[kN], sv[kN];
#pragma unroll
    for (int r = 0; r < kN; ++r) {
      const int i = tid + r * NW * kWave, j = i / (kKiviHead / 2), pr = i % (kKiviHead / 2);
      rope_cs1(k, j, pr, cv[r], sv[r]);
    }
#pragma unroll
    for (int r = 0; r < kN; ++r) {
      const int i = tid + r * NW * kWave, j = i / (kKiviHead / 2), pr = i % (kKiviHead / 2);
      const int oc = k.rope_style == 0 ? 2 * pr : pr, os = k.rope_style == 0 ? 2 * pr + 1 : kKiviHead / 2 + pr;
      const _Float16 ch = (_Float16)cv[r], sh = (_Float16)sv[r];
      s_rope_tb.cs[j][oc] = __builtin_bit_cast(uint16_t, ch);
      s_rope_tb.cs[j][os] = __builtin_bit_cast(uint16_t, sh);
    }
#pragma unroll
    for (int r = 0; r < kPR; ++r) {
      const int i = tid + r * NW * kWave, pgi = i / (2 * kQ), w = i % (2 * kQ), tab = w / kQ, q4 = w % kQ;
      typedef _Float16 h4 __attribute__((ext_vector_type(4)));
      const h4 hv = {(_Float16)rv[r][0], (_Float16)rv[r][1], (_Float16)rv[r][2], (_Float16)rv[r][3]};
      if (k.rope_style == 0) {
        // pair 4 q4 + e: (cos, sin) in halves 2 (4 q4 + e), + 1
        uint16_t* rowp = &s_prot[pgi][0][0];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          // (a scalar first: __builtin_bit_cast of a vector element itself
          // reads element 0 with this compiler)
          const _Float16 he = (_Float16)rv[r][e];
          rowp[2 * (4 * q4 + e) + tab] = __builtin_bit_cast(uint16_t, he);
        }
      } else {
        *reinterpret_cast<uint2*>(&s_prot[pgi][tab][4 * q4]) = __builtin_bit_cast(uint2, hv);
      }
    }
    __syncthreads();
    s_rope = &s_rope_tb;
    prot = PageRot{&s_prot[0][0][0], pg_first, kCap};
  }
  const int hs = bid % p.head_slices;      bid /= p.head_slices;
  const int kvh = bid % p.num_kv_heads;
  const int seq = bid / p.num_kv_heads;
  // Single pass: the page table entries of this wavefront's first 64 pages
  // are read before L is known, for the usual split (NW - 1 page
  // wavefronts, the last one on the window), so the first page loads wait
  // for one memory round trip instead of two.
  // The q operand is loaded here, with the length and the table entries,
  // so that the first page loads wait for one memory round trip, not for q
  // after the length (interleaved A/B, us per step: INT4 65.0 -> 64.6, mixed
  // lengths 67.6 -> 66.7, INT8 113.3 -> 112.9, INT4 keys before RoPE 111.9
  // -> 111.4).  INT8 with keys before RoPE loads it where it is used: its
  // registers are short, and 16 more held from here cost it 1.1 us.
  constexpr bool kQEarly = !(BITS == 8 && ROPE);
  u32x4 q_raw[4];
  if constexpr (kQEarly) load_q_operand(p, seq, kvh, hs, tid % kWave, q_raw);
  int early_id = -1;
  if constexpr (FINAL) {
    const int pg = wave + (tid % kWave) * (NW - 1);
    if (pg < k.max_pages_per_seq) early_id = k.page_tables[(int64_t)seq * k.max_pages_per_seq + pg];
  }
  const int L = p.seq_lens[seq];
  const int lq = kivi_quantized_len(L, k.residual_length);
  const int n_pages = min(lq / kKiviPageTokens, k.max_pages_per_seq);
  const int n_parts = FINAL ? 1 : max(1, (n_pages + k.partition_pages - 1) / k.partition_pages);
  if (part >= n_parts) return;
  const int pg0 = FINAL ? 0 : part * k.partition_pages;
  const int pg1 = FINAL ? n_pages : min(pg0 + k.partition_pages, n_pages);
  const bool last = part == n_parts - 1;
  const bool has_res = last && L > lq;
  const int page_waves = has_res ? NW - 1 : NW;
  // The residual wavefront ends its window about 10 us before the page
  // wavefronts end their pages (batch 64, ctx 4096), so it also runs the
  // range's last pages, 1/30 of them: 4 of 124 at ctx 4096 gave 63.9 us
  // per step against 64.5 us (2 pages: 64.7, 3: 64.1, 6: 64.9).
  int ahead_page = 0;
  const int ahead = APPEND ? kivi_ahead_piece(L, k.residual_length, ahead_page) : -1;
  const bool piece_due = APPEND && k.job.build_ahead && hs == 0 && has_res && ahead >= 0;
  const int res_pages = has_res ? (pg1 - pg0) / 30 : 0;

  // The page that L completes, if any (APPEND), by the whole workgroup
  // before the page wavefronts start.  (Built by the residual wavefront
  // alone, overlapped with the page wavefronts, the step was 0.2 us slower
  // on average: one wavefront takes far longer over the build and then
  // ends after the page wavefronts.)
  if constexpr (APPEND) {
    // (with build-ahead the steps before this one wrote the page in pieces)
    if (!k.job.build_ahead && last && lq > 0 && lq != kivi_quantized_len(L - 1, k.residual_length)) {
      kivi_build_page<NW * kWave, BITS>(*reinterpret_cast<Build*>(s_raw), k.job, seq, kvh,
                                  lq / kKiviPageTokens - 1, L, tid);
      __syncthreads();   // the page is visible to the workgroup; the LDS is free again
    }
    if (last && !has_res && wave == 0)
      store_newest<BS>(k.job, newest_from_row(k.job, seq, kvh, tid), seq, kvh, tid);
  }
  if (wave < page_waves) {
    if constexpr (!kQEarly) load_q_operand(p, seq, kvh, hs, tid % kWave, q_raw);
    // Single pass runs two workgroups per CU, b and b + grid/2 (dispatch
    // order), and the SIMDs issue the oldest wavefront first: left alone
    // workgroup b finishes about 10 us before b + grid/2 (48.5 against 59.4
    // us at batch 64).  The second half's page wavefronts take the higher
    // priority on every other page pair, so both progress together (55.5
    // and 58.5 us).
    kivi_pages_wave<BITS, ROPE>(k, seq, kvh, hs, pg0 + wave, pg1 - res_pages, page_waves, &sd.p[wave][0], &sd.acc[wave][0][0],
                    &sd.m[wave][0], &sd.l[wave][0], FINAL && blockIdx.x >= gridDim.x / 2,
                    FINAL && page_waves == NW - 1, early_id, s_rope, prot, q_raw);
  } else {
    const int lane = tid % kWave;
    // build-ahead: this step's piece of the next page (one head slice
    // writes it).  Its table entries are read here and its fp16 after the
    // window (with keys held before RoPE, both after the wavefront's last
    // pages: its registers are short there), it is staged in LDS, and the
    // four wavefronts quantise and write it after the merge, so that no
    // load of the launch waits behind its stores.
    KiviPiece piece;
    piece.piece = -1;
    if constexpr (APPEND && !ROPE)
      if (piece_due) piece = kivi_piece_plan(k.job, seq, ahead_page, ahead, lane);
    NewestToken nt;
    if constexpr (APPEND)
      nt = k.job.slots[seq] >= 0 ? newest_from_row(k.job, seq, kvh, lane)
                                 : newest_from_pool<BS>(p, seq, kvh, L - 1, lane);
    else
      nt = newest_from_pool<BS>(p, seq, kvh, L - 1, lane);
    if constexpr (ROPE) {
      // the window's page rotations: lane l holds pair l of rows 32 (wp0 + r)
      const int wp0 = lq / kKiviPageTokens;
      float wc[kWinRows], ws[kWinRows];
#pragma unroll
      for (int r = 0; r < kWinRows; ++r) rope_cs1(k, kKiviPageTokens * (wp0 + r), lane, wc[r], ws[r]);
#pragma unroll
      for (int r = 0; r < kWinRows; ++r) {
        typedef _Float16 h2 __attribute__((ext_vector_type(2)));
        const h2 v = {(_Float16)wc[r], (_Float16)ws[r]};
        s_wrot[r * (kKiviHead / 2) + lane] = __builtin_bit_cast(uint32_t, v);
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      decode2_wave<Kind::F16, kKiviHead, BS>(p, seq, kvh, hs, lq, L - 1, 32, &sd.p[wave][0], &sd.acc[wave][0][0],
                                             &sd.m[wave][0], &sd.l[wave][0], KiviWindowRope{k, s_rope, s_wrot, wp0});
      NewestToken ntr = nt;
      ntr.k = rope_newest_key(k, nt.k, L - 1, lane);
      newest_state(p, ntr, seq, kvh, hs, lane, &sd.acc[NW][0][0], &sd.m[NW][0], &sd.l[NW][0]);
    } else {
      decode2_wave<Kind::F16, kKiviHead, BS>(p, seq, kvh, hs, lq, L - 1, 32, &sd.p[wave][0],
                                             &sd.acc[wave][0][0], &sd.m[wave][0], &sd.l[wave][0]);
      newest_state(p, nt, seq, kvh, hs, lane, &sd.acc[NW][0][0], &sd.m[NW][0], &sd.l[NW][0]);
    }
    // the token's store, at the end of the window, off the page wavefronts'
    // path (the window ends halfway through the launch)
    if constexpr (APPEND) store_newest<BS>(k.job, nt, seq, kvh, lane);
    if constexpr (APPEND && !ROPE) kivi_piece_load(k.job, piece, kvh, ahead_page, lane);
    if constexpr (!kQEarly) load_q_operand(p, seq, kvh, hs, lane, q_raw);
    kivi_pages_wave<BITS, ROPE>(k, seq, kvh, hs, pg1 - res_pages, pg1, 1, &sd.p[wave][0], &sd.acc[NW + 1][0][0],
                    &sd.m[NW + 1][0], &sd.l[NW + 1][0], false, false, -1, s_rope, prot, q_raw);
    // the piece's fp16 for the quarters after the merge
    if constexpr (APPEND) {
      if (piece_due) {
        if constexpr (ROPE) {
          piece = kivi_piece_plan(k.job, seq, ahead_page, ahead, lane);
          kivi_piece_load(k.job, piece, kvh, ahead_page, lane);
        }
        kivi_piece_stage(piece, lane, reinterpret_cast<uint16_t*>(&sd.p[wave][0]));
        if (lane == 0) sd.piece_pid = piece.piece >= 0 ? piece.pid : -1;
      }
    }
  }
  __syncthreads();
  // build-ahead: wavefront q quantises quarter q of the piece, last, after
  // every load; its staged values are read before the merge
  static_assert(!APPEND || NW == 4, "a quarter of the piece per wavefront");
  uint2 qv = {0u, 0u};
  int piece_pid = -1;
  if constexpr (APPEND) {
    if (piece_due) {
      piece_pid = sd.piece_pid;
      qv = kivi_piece_quarter_values(ahead, wave, tid % kWave, reinterpret_cast<const uint16_t*>(&sd.p[NW - 1][0]));
    }
  }
  combine_waves<Kind::F16, Kind::F32, kKiviHead, FINAL, kWaveHeads, NW + 2>(p, has_res ? NW + 2 : NW, &sd.m[0][0], &sd.l[0][0],
                                                        &sd.acc[0][0][0], seq, kvh, hs, part, tid, NW * kWave);
  if constexpr (APPEND) {
    if (piece_pid >= 0)
      kivi_piece_quarter<BITS>(k.job, piece_pid, ahead, kvh, wave, tid % kWave, qv,
                               reinterpret_cast<uint8_t*>(&sd.p[0][0]) + 256 * wave);
  }
}

template <int NW, bool FINAL, int BITS, bool ROPE, int BS>
void launch_decode_bs(const KiviParams& k, bool append, unsigned grid, hipStream_t stream) {
  if (append)
    hipLaunchKernelGGL((kivi_decode_kernel<NW, FINAL, true, BITS, ROPE, BS>), dim3(grid), dim3(NW * kWave), 0, stream,
                       k);
  else
    hipLaunchKernelGGL((kivi_decode_kernel<NW, FINAL, false, BITS, ROPE, BS>), dim3(grid), dim3(NW * kWave), 0, stream,
                       k);
}
template <int NW, bool FINAL, int BITS, bool ROPE>
void launch_decode_bits(const KiviParams& k, bool append, unsigned grid, hipStream_t stream) {
  if (k.base.block_size == 16) launch_decode_bs<NW, FINAL, BITS, ROPE, 16>(k, append, grid, stream);
  else launch_decode_bs<NW, FINAL, BITS, ROPE, 0>(k, append, grid, stream);
}
template <int NW, bool FINAL>
void launch_decode(const KiviParams& k, bool append, int bits, unsigned grid, hipStream_t stream) {
  const bool rope = k.rope_cos != nullptr;
  if (bits == 8) {
    if (rope) launch_decode_bits<NW, FINAL, 8, true>(k, append, grid, stream);
    else launch_decode_bits<NW, FINAL, 8, false>(k, append, grid, stream);
  } else {
    if (rope) launch_decode_bits<NW, FINAL, 4, true>(k, append, grid, stream);
    else launch_decode_bits<NW, FINAL, 4, false>(k, append, grid, stream);
  }
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
  p.block_size = a.block_size;
  k.pages = (const uint8_t*)a.pages; k.page_tables = a.page_tables;
  k.max_pages_per_seq = a.max_pages_per_seq; k.num_pages = a.num_pages;
  k.residual_length = a.residual_length; k.partition_pages = a.partition_pages;
  k.rope_cos = a.rope_cos; k.rope_sin = a.rope_sin;
  k.rope_max_pos = a.rope_max_pos; k.rope_style = a.rope_style;
  // the step's append (token write, quantise-on-append) is fused into the
  // decode launch
  const bool append = a.append != nullptr;
  if (append) k.job = make_page_job(*a.append);
  const unsigned items = (unsigned)(a.num_seqs * a.num_kv_heads * p.head_slices);
  // keys held before RoPE: every page rotation of a workgroup in its LDS rows
  if (a.rope_cos && a.partition_pages > kivi_page_rot_cap(a.bits)) return 3;
  if (a.num_partitions == 1) {
    // 4 wavefronts per workgroup, two workgroups per CU: at batch 64 the
    // grid is resident in one round (65.1 against 67.1 us with 8)
    launch_decode<4, true>(k, append, a.bits, items, a.stream);
  } else {
    launch_decode<4, false>(k, append, a.bits, items * a.num_partitions, a.stream);
    if (hipGetLastError() != hipSuccess) return 5;
    return launch_lse_reduce(a.out, (int)Kind::F16, a.part_m, a.part_l, a.part_o, a.seq_lens,
                             a.num_seqs, a.num_heads, kKiviHead, a.num_partitions, 0,
                             a.residual_length, a.partition_pages, a.max_pages_per_seq, a.stream);
  }
  return hipGetLastError() == hipSuccess ? 0 : 5;
}

}  // namespace tl
