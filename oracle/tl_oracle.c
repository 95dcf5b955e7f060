/*
 * tl_oracle.c -- CPU oracle for the truellm-engine attention hot path.
 *
 * TEST INFRASTRUCTURE ONLY (see tl_oracle.h): the checker for tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg.  Never linked into
 * or called by the product library.
 *
 * Built with -ffp-contract=off so every fp32 operation below rounds exactly
 * where it is written; the one fused multiply-add the reference relies on
 * (kivi_cache.cu:190, contracted by nvcc's default -fmad=true) is an explicit
 * fmaf().
 */
#include "tl_oracle.h"

#include <float.h>
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ========================================================================
 * Scalar conversions
 * ====================================================================== */

static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* IEEE binary16, round to nearest even, overflow to inf, NaN kept quiet. */
uint16_t orc_f32_to_f16(float f)
{
    uint32_t x = f2u(f);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    uint32_t ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu));
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);   /* >= 65520 */
    if (ax >= 0x38800000u) {                                     /* >= 2^-14 */
        uint32_t mant = ax & 0x7fffffu;
        uint32_t e = (ax >> 23) - 127 + 15;
        uint32_t h = (e << 10) | (mant >> 13);
        uint32_t rem = mant & 0x1fffu;
        if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
        return (uint16_t)(sign | h);
    }
    /* subnormal: units of 2^-24; the product is exact in double and rint
     * rounds half to even under the default rounding mode. */
    double v = rint((double)u2f(ax) * 16777216.0);
    return (uint16_t)(sign | (uint16_t)v);
}

float orc_f16_to_f32(uint16_t h)
{
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    if (e == 0) {
        float v = (float)m * (1.0f / 16777216.0f);
        return sign ? -v : v;
    }
    if (e == 31) return u2f(sign | 0x7f800000u | (m << 13));
    return u2f(sign | ((e - 15 + 127) << 23) | (m << 13));
}

uint16_t orc_f32_to_bf16(float f)
{
    uint32_t x = f2u(f);
    if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40u);
    x += 0x7fffu + ((x >> 16) & 1u);
    return (uint16_t)(x >> 16);
}

float orc_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

/* OCP 8-bit E4M3 ("E4M3FN"): bias 7, no infinities, S.1111.111 = NaN,
 * max finite 0x7E = 448.  Round to nearest even; magnitudes >= 448 (and
 * infinities) saturate to 448. */
uint8_t orc_f32_to_e4m3(float f)
{
    uint8_t sign = (f2u(f) >> 24) & 0x80u;
    if (isnan(f)) return (uint8_t)(sign | 0x7fu);
    double a = fabs((double)f);
    if (a >= 448.0) return (uint8_t)(sign | 0x7eu);
    if (a < 0.015625) {                        /* below 2^-6: subnormal grid 2^-9 */
        double q = rint(a * 512.0);            /* 0..8; 8 encodes 2^-6 exactly */
        return (uint8_t)(sign | (uint8_t)q);
    }
    int e;
    double fr = frexp(a, &e);                  /* a = fr * 2^e, fr in [0.5, 1) */
    int ue = e - 1;                            /* a = 1.m * 2^ue */
    double m = rint((fr * 2.0 - 1.0) * 8.0);   /* 0..8 */
    if (m >= 8.0) { m = 0.0; ue++; }
    return (uint8_t)(sign | (uint8_t)((ue + 7) << 3) | (uint8_t)m);
}

float orc_e4m3_to_f32(uint8_t v)
{
    float s = (v & 0x80u) ? -1.0f : 1.0f;
    int e = (v >> 3) & 0xf, m = v & 7;
    if (e == 15 && m == 7) return NAN;
    if (e == 0) return s * ldexpf((float)m, -9);
    return s * ldexpf(1.0f + (float)m / 8.0f, e - 7);
}

static double load_elem(const void* base, int dtype, int64_t i)
{
    switch (dtype) {
    case ORC_F32:  return ((const float*)base)[i];
    case ORC_F16:  return orc_f16_to_f32(((const uint16_t*)base)[i]);
    case ORC_BF16: return orc_bf16_to_f32(((const uint16_t*)base)[i]);
    case ORC_FP8:  return orc_e4m3_to_f32(((const uint8_t*)base)[i]);
    default:       return NAN;
    }
}

static float load_f32(const void* base, int dtype, int64_t i)
{
    return (float)load_elem(base, dtype, i);
}

static void store_elem(void* base, int dtype, int64_t i, float v)
{
    switch (dtype) {
    case ORC_F32:  ((float*)base)[i] = v; break;
    case ORC_F16:  ((uint16_t*)base)[i] = orc_f32_to_f16(v); break;
    case ORC_BF16: ((uint16_t*)base)[i] = orc_f32_to_bf16(v); break;
    case ORC_FP8:  ((uint8_t*)base)[i] = orc_f32_to_e4m3(v); break;
    default: break;
    }
}

void orc_convert(const void* src, int src_dtype, void* dst, int dst_dtype,
                 int64_t n, float mul)
{
    for (int64_t i = 0; i < n; ++i) {
        float v = load_f32(src, src_dtype, i);
        if (src_dtype == ORC_FP8 || dst_dtype == ORC_FP8) v = v * mul;
        store_elem(dst, dst_dtype, i, v);
    }
}

/* ========================================================================
 * reshape_and_cache  (cache_kernels.cu:47-94)
 *   blk = slot / bs, off = slot % bs
 *   cache[blk][h][e][off] = src[t][h][e]
 * ====================================================================== */

void orc_reshape_and_cache(const void* key, const void* value,
                           void* k_cache, void* v_cache,
                           const int32_t* slot_mapping, int num_tokens,
                           int num_kv_heads, int head_size, int block_size,
                           int elem_bytes)
{
    for (int t = 0; t < num_tokens; ++t) {
        int32_t slot = slot_mapping[t];
        if (slot < 0) continue;                       /* cache_kernels.cu:68-69 */
        int64_t blk = slot / block_size, off = slot % block_size;
        for (int h = 0; h < num_kv_heads; ++h)
            for (int e = 0; e < head_size; ++e) {
                int64_t dst = ((blk * num_kv_heads + h) * head_size + e) * block_size + off;
                int64_t src = ((int64_t)t * num_kv_heads + h) * head_size + e;
                memcpy((char*)k_cache + dst * elem_bytes, (const char*)key + src * elem_bytes, elem_bytes);
                memcpy((char*)v_cache + dst * elem_bytes, (const char*)value + src * elem_bytes, elem_bytes);
            }
    }
}

void orc_reshape_and_cache_fp8(const void* key, const void* value, int src_dtype,
                               uint8_t* k_cache, uint8_t* v_cache,
                               const int32_t* slot_mapping, int num_tokens,
                               int num_kv_heads, int head_size, int block_size,
                               float k_scale, float v_scale)
{
    /* multiplier = 1/scale in fp32, as fp8_gemm.cu:89-93 (scale 0 -> 1) */
    float km = 1.0f / (k_scale == 0.0f ? 1.0f : k_scale);
    float vm = 1.0f / (v_scale == 0.0f ? 1.0f : v_scale);
    for (int t = 0; t < num_tokens; ++t) {
        int32_t slot = slot_mapping[t];
        if (slot < 0) continue;
        int64_t blk = slot / block_size, off = slot % block_size;
        for (int h = 0; h < num_kv_heads; ++h)
            for (int e = 0; e < head_size; ++e) {
                int64_t dst = ((blk * num_kv_heads + h) * head_size + e) * block_size + off;
                int64_t src = ((int64_t)t * num_kv_heads + h) * head_size + e;
                k_cache[dst] = orc_f32_to_e4m3(load_f32(key, src_dtype, src) * km);
                v_cache[dst] = orc_f32_to_e4m3(load_f32(value, src_dtype, src) * vm);
            }
    }
}

/* ========================================================================
 * RoPE + reshape_and_cache
 *   style 0 (ggml LLAMA_ROPE_TYPE_NORM, cuda_engine.cpp:1100-1108): pairs
 *   (2i, 2i+1); style 1 (rope_device.cuh:24-36): pairs (i, i + d/2);
 *   c, s = cos/sin_table[pos][i] (cuda_model.cpp:269-295);
 *   (a, b) -> (fmaf(a, c, -(b*s)), fmaf(a, s, b*c)) in fp32, rounded once.
 *   Then key/value into the pool as orc_reshape_and_cache.
 * ====================================================================== */

static int rope_dim(int style, int i, int j, int half) { return style == 0 ? 2 * i + j : i + j * half; }

static void rope_row(const void* src, void* dst, int dtype, int64_t base, int head_size, int style,
                     const float* cs, const float* sn)
{
    int half = head_size / 2;
    for (int i = 0; i < half; ++i) {
        int d0 = rope_dim(style, i, 0, half), d1 = rope_dim(style, i, 1, half);
        float a = load_f32(src, dtype, base + d0), b = load_f32(src, dtype, base + d1);
        float c = cs[i], s = sn[i];
        float r0 = fmaf(a, c, -(b * s)), r1 = fmaf(a, s, b * c);
        store_elem(dst, dtype, base + d0, r0);
        store_elem(dst, dtype, base + d1, r1);
    }
}

void orc_rope_reshape_and_cache(const void* q, void* q_out, const void* key, const void* value,
                                void* k_cache, void* v_cache, const int32_t* slot_mapping,
                                const int32_t* positions, const float* cos_table, const float* sin_table,
                                int max_positions, int num_tokens, int num_heads, int num_kv_heads,
                                int head_size, int block_size, int num_blocks, int dtype, int style)
{
    int half = head_size / 2, eb = dtype == ORC_F32 ? 4 : 2;
    char* tmp = (char*)malloc((size_t)head_size * eb);
    for (int t = 0; t < num_tokens; ++t) {
        int pos = positions[t];
        if (pos < 0 || pos >= max_positions) continue;
        const float* cs = cos_table + (int64_t)pos * half;
        const float* sn = sin_table + (int64_t)pos * half;
        for (int h = 0; h < num_heads; ++h)
            rope_row(q, q_out, dtype, ((int64_t)t * num_heads + h) * head_size, head_size, style, cs, sn);
        int32_t slot = slot_mapping[t];
        if (slot < 0) continue;
        int64_t blk = slot / block_size, off = slot % block_size;
        if (blk >= num_blocks) continue;
        for (int h = 0; h < num_kv_heads; ++h) {
            int64_t src = ((int64_t)t * num_kv_heads + h) * head_size;
            /* rotate the key row into a scratch row, then scatter both rows */
            memcpy(tmp, (const char*)key + src * eb, (size_t)head_size * eb);
            rope_row(tmp, tmp, dtype, 0, head_size, style, cs, sn);
            for (int e = 0; e < head_size; ++e) {
                int64_t dst = ((blk * num_kv_heads + h) * head_size + e) * block_size + off;
                memcpy((char*)k_cache + dst * eb, tmp + (int64_t)e * eb, eb);
                memcpy((char*)v_cache + dst * eb, (const char*)value + (src + e) * eb, eb);
            }
        }
    }
    free(tmp);
}

/* ========================================================================
 * Norms and gated activations  (layernorm_kernels.cu:28-139,
 * activation_kernels.cu:57-100), intended semantics; the row sums in
 * double (the device's fp32 tree sum differs from any order by a few fp32
 * ulps, far below the output dtype's)
 * ====================================================================== */

void orc_rms_norm(void* out, void* residual, const void* x, const void* w, int rows, int hidden, float eps,
                  int dtype)
{
    for (int r = 0; r < rows; ++r) {
        int64_t base = (int64_t)r * hidden;
        double ss = 0.0;
        for (int i = 0; i < hidden; ++i) {
            float v = load_f32(x, dtype, base + i);
            if (residual) {
                v = v + load_f32(residual, dtype, base + i);
                store_elem(residual, dtype, base + i, v);
            }
            ss += (double)v * v;
        }
        float inv = (float)(1.0 / sqrt(ss / hidden + eps));
        const void* src = residual ? residual : x;
        for (int i = 0; i < hidden; ++i)
            store_elem(out, dtype, base + i, load_f32(src, dtype, base + i) * inv * load_f32(w, dtype, i));
    }
}

void orc_layer_norm(void* out, const void* x, const void* w, const void* b, int rows, int hidden, float eps,
                    int dtype)
{
    for (int r = 0; r < rows; ++r) {
        int64_t base = (int64_t)r * hidden;
        double s = 0.0, var = 0.0;
        for (int i = 0; i < hidden; ++i) s += load_f32(x, dtype, base + i);
        double mean = s / hidden;
        for (int i = 0; i < hidden; ++i) {
            double d = load_f32(x, dtype, base + i) - mean;
            var += d * d;
        }
        double inv = 1.0 / sqrt(var / hidden + eps);
        for (int i = 0; i < hidden; ++i)
            store_elem(out, dtype, base + i,
                       (float)((load_f32(x, dtype, base + i) - mean) * inv * load_f32(w, dtype, i) +
                               load_f32(b, dtype, i)));
    }
}

void orc_act_and_mul(void* out, const void* gate, const void* up, int64_t n, int act, int dtype)
{
    for (int64_t i = 0; i < n; ++i) {
        float g = load_f32(gate, dtype, i), a;
        if (act == 0) a = g / (1.f + expf(-g));
        else if (act == 1) a = 0.5f * g * (1.f + erff(g * 0.70710678118f));
        else a = 0.5f * g * (1.f + tanhf(0.79788456f * (g + 0.044715f * g * g * g)));
        /* the activation rounded to the storage type, then the product */
        uint16_t bits;
        if (dtype == ORC_F16) { bits = orc_f32_to_f16(a); a = orc_f16_to_f32(bits); }
        else if (dtype == ORC_BF16) { bits = orc_f32_to_bf16(a); a = orc_bf16_to_f32(bits); }
        store_elem(out, dtype, i, a * load_f32(up, dtype, i));
    }
}

/* ========================================================================
 * VQ codec  (vq_cache.cu:18-69, codebook_init.cu:23-145)
 *   encode: dist_c = fold_d fmaf(x_d - b_cd, x_d - b_cd, dist) (fp32, d in
 *   order); the first c with dist_c < best (best = FLT_MAX at the start)
 *   decode: out[v] = book[idx[v]]
 *   k-means: assign, then per cluster the exact sum of its members (each
 *   fp16 value is a multiple of 2^-24: int64 fixed point), non-finite
 *   values by IEEE sum rules, centroid = fp16(fp32(sum) * (1/count)),
 *   empty clusters unchanged
 * ====================================================================== */

static int vq_nearest(const uint16_t* x, const uint16_t* book, int head_dim, int codebook_size)
{
    float best = FLT_MAX;
    int best_c = 0;
    for (int c = 0; c < codebook_size; ++c) {
        const uint16_t* e = book + (int64_t)c * head_dim;
        float dist = 0.f;
        for (int d = 0; d < head_dim; ++d) {
            float diff = orc_f16_to_f32(x[d]) - orc_f16_to_f32(e[d]);
            dist = fmaf(diff, diff, dist);
        }
        if (dist < best) { best = dist; best_c = c; }
    }
    return best_c;
}

void orc_vq_encode(const uint16_t* kv, const uint16_t* book, uint16_t* idx, int64_t num_vecs, int head_dim,
                   int codebook_size)
{
    for (int64_t v = 0; v < num_vecs; ++v)
        idx[v] = (uint16_t)vq_nearest(kv + v * head_dim, book, head_dim, codebook_size);
}

void orc_vq_decode(uint16_t* out, const uint16_t* book, const uint16_t* idx, int64_t num_vecs, int head_dim,
                   int codebook_size)
{
    for (int64_t v = 0; v < num_vecs; ++v)
        if (idx[v] < codebook_size)
            memcpy(out + v * head_dim, book + (int64_t)idx[v] * head_dim, (size_t)head_dim * 2);
}

void orc_vq_kmeans(const uint16_t* data, uint16_t* book, int64_t n, int codebook_size, int head_dim,
                   int iterations)
{
    size_t kd = (size_t)codebook_size * head_dim;
    int* assign = (int*)malloc(sizeof(int) * (size_t)(n > 0 ? n : 1));
    long long* sums = (long long*)malloc(sizeof(long long) * kd);
    int* flags = (int*)malloc(sizeof(int) * kd);
    int* counts = (int*)malloc(sizeof(int) * (size_t)codebook_size);
    for (int it = 0; it < iterations; ++it) {
        for (int64_t s = 0; s < n; ++s) assign[s] = vq_nearest(data + s * head_dim, book, head_dim, codebook_size);
        memset(sums, 0, sizeof(long long) * kd);
        memset(flags, 0, sizeof(int) * kd);
        memset(counts, 0, sizeof(int) * (size_t)codebook_size);
        for (int64_t s = 0; s < n; ++s) {
            int c = assign[s];
            counts[c]++;
            for (int d = 0; d < head_dim; ++d) {
                float x = orc_f16_to_f32(data[s * head_dim + d]);
                size_t k = (size_t)c * head_dim + d;
                if (isnan(x)) flags[k] |= 1;
                else if (isinf(x)) flags[k] |= x > 0 ? 2 : 4;
                else sums[k] += (long long)(x * 16777216.0f);
            }
        }
        for (int c = 0; c < codebook_size; ++c) {
            if (counts[c] == 0) continue;
            float inv = 1.f / (float)counts[c];
            for (int d = 0; d < head_dim; ++d) {
                size_t k = (size_t)c * head_dim + d;
                float sum;
                if ((flags[k] & 1) || (flags[k] & 6) == 6) sum = NAN;
                else if (flags[k] & 2) sum = INFINITY;
                else if (flags[k] & 4) sum = -INFINITY;
                else sum = (float)sums[k] * (1.0f / 16777216.0f);
                book[k] = orc_f32_to_f16(sum * inv);
            }
        }
    }
    free(assign); free(sums); free(flags); free(counts);
}

/* ========================================================================
 * copy_blocks  (cache_kernels.cu:107-131, :234-262)
 *   for each pair {src, dst}: pool[dst] = pool[src], for the K and the V
 *   pool; pairs with an id outside [0, num_blocks) are skipped
 * swap_blocks  (cache_kernels.cu:133-167, :264-284)
 *   direction 0: host[dst] = dev[src]; 1: dev[dst] = host[src]
 * ====================================================================== */

void orc_copy_blocks(void* k_cache, void* v_cache, const int32_t* mapping, int num_pairs,
                     int num_blocks, int64_t block_bytes)
{
    for (int p = 0; p < num_pairs; ++p) {
        int32_t src = mapping[2 * p], dst = mapping[2 * p + 1];
        if (src < 0 || src >= num_blocks || dst < 0 || dst >= num_blocks) continue;
        memmove((char*)k_cache + dst * block_bytes, (const char*)k_cache + src * block_bytes, (size_t)block_bytes);
        memmove((char*)v_cache + dst * block_bytes, (const char*)v_cache + src * block_bytes, (size_t)block_bytes);
    }
}

void orc_swap_blocks(void* cache, void* host_cache, const int32_t* mapping, int num_pairs,
                     int num_device_blocks, int num_host_blocks, int64_t block_bytes, int direction)
{
    for (int p = 0; p < num_pairs; ++p) {
        int32_t src = mapping[2 * p], dst = mapping[2 * p + 1];
        const char* from = direction == 0 ? (const char*)cache : (const char*)host_cache;
        char* to = direction == 0 ? (char*)host_cache : (char*)cache;
        int nf = direction == 0 ? num_device_blocks : num_host_blocks;
        int nt = direction == 0 ? num_host_blocks : num_device_blocks;
        if (src < 0 || src >= nf || dst < 0 || dst >= nt) continue;
        memcpy(to + dst * block_bytes, from + src * block_bytes, (size_t)block_bytes);
    }
}

/* ========================================================================
 * Paged attention, intended semantics (double accumulation)
 * ====================================================================== */

static int kv_head_of(int head, int num_heads, int num_kv_heads, int gqa_map)
{
    if (gqa_map == ORC_GQA_GROUPED) return head / (num_heads / num_kv_heads);
    return head % num_kv_heads;
}

/* Element (token position t, dim e) of one sequence's gathered K or V;
 * returns 0 when the table entry is negative (token skipped). */
static int gather_ok(const int32_t* row, int t, int block_size, int64_t* phys)
{
    int32_t p = row[t / block_size];
    if (p < 0) return 0;
    *phys = p;
    return 1;
}

void orc_paged_attention(double* out, const void* q, int q_dtype,
                         const void* k_cache, const void* v_cache, int kv_dtype,
                         float k_scale, float v_scale,
                         const int32_t* block_tables, int max_blocks_per_seq,
                         const int32_t* seq_lens, int num_seqs, int num_heads,
                         int num_kv_heads, int head_size, int block_size,
                         float scale, int gqa_map, int partition_tokens)
{
    double ks = (kv_dtype == ORC_FP8) ? (double)k_scale : 1.0;
    double vs = (kv_dtype == ORC_FP8) ? (double)v_scale : 1.0;
    int max_len = 0;
    for (int s = 0; s < num_seqs; ++s) if (seq_lens[s] > max_len) max_len = seq_lens[s];
    double* sc = (double*)malloc(sizeof(double) * (max_len > 0 ? max_len : 1));
    unsigned char* ok = (unsigned char*)malloc(max_len > 0 ? max_len : 1);
    double* acc = (double*)malloc(sizeof(double) * head_size);
    double* pacc = (double*)malloc(sizeof(double) * head_size);

    for (int s = 0; s < num_seqs; ++s) {
        int L = seq_lens[s];
        const int32_t* row = block_tables + (int64_t)s * max_blocks_per_seq;
        for (int h = 0; h < num_heads; ++h) {
            int kvh = kv_head_of(h, num_heads, num_kv_heads, gqa_map);
            const int64_t qoff = ((int64_t)s * num_heads + h) * head_size;
            double* o = out + qoff;
            for (int t = 0; t < L; ++t) {
                int64_t phys;
                ok[t] = (unsigned char)gather_ok(row, t, block_size, &phys);
                if (!ok[t]) continue;
                int64_t base = (phys * num_kv_heads + kvh) * head_size * block_size + t % block_size;
                double dot = 0.0;
                for (int e = 0; e < head_size; ++e)
                    dot += load_elem(q, q_dtype, qoff + e) *
                           (load_elem(k_cache, kv_dtype, base + (int64_t)e * block_size) * ks);
                sc[t] = dot * (double)scale;
            }
            int P = (partition_tokens > 0) ? (L + partition_tokens - 1) / partition_tokens : 1;
            int PT = (partition_tokens > 0) ? partition_tokens : (L > 0 ? L : 1);
            /* global accumulators for the LSE merge */
            double gm = -INFINITY, gl = 0.0;
            for (int e = 0; e < head_size; ++e) acc[e] = 0.0;
            for (int p = 0; p < P; ++p) {
                int t0 = p * PT, t1 = t0 + PT < L ? t0 + PT : L;
                double m = -INFINITY, l = 0.0;
                for (int t = t0; t < t1; ++t) if (ok[t] && sc[t] > m) m = sc[t];
                if (m == -INFINITY) continue;               /* empty partition */
                for (int e = 0; e < head_size; ++e) pacc[e] = 0.0;
                for (int t = t0; t < t1; ++t) {
                    if (!ok[t]) continue;
                    int64_t phys = 0; gather_ok(row, t, block_size, &phys);
                    int64_t base = (phys * num_kv_heads + kvh) * head_size * block_size + t % block_size;
                    double w = exp(sc[t] - m);
                    l += w;
                    for (int e = 0; e < head_size; ++e)
                        pacc[e] += w * (load_elem(v_cache, kv_dtype, base + (int64_t)e * block_size) * vs);
                }
                /* partition result (m, l, pacc/l) merged by log-sum-exp */
                double nm = m > gm ? m : gm;
                double a = (gm == -INFINITY) ? 0.0 : exp(gm - nm);
                double b = exp(m - nm);
                for (int e = 0; e < head_size; ++e)
                    acc[e] = acc[e] * a + (pacc[e] / l) * (l * b);
                gl = gl * a + l * b;
                gm = nm;
            }
            for (int e = 0; e < head_size; ++e) o[e] = (gl > 0.0) ? acc[e] / gl : 0.0;
        }
    }
    free(sc); free(ok); free(acc); free(pacc);
}

/* ---- literal v1 (paged_attention_v1.cu:31-135, attention_utils.cuh:47-68,
 *      reduce_kernel_utils.cuh:41-73) -------------------------------------
 * Only warp-0 lanes t < tokens_in_block (<= 32) carry tokens.  After each
 * block every warp-0 lane holds (M_b, S_b) with
 *   S_b = 32 * S_{b-1} * e^{M_{b-1}-M_b} + sum_t e^{qk_t - M_b}
 * and thread d writes only its own out_acc[d]:
 *   out[d] = sum_b [d%128 < T_b] e^{qk_{b,d%128}-M_b}/S_b * V[b][d][d%128]. */
void orc_paged_attention_literal_v1(float* out, const void* q, const void* k_cache,
                                    const void* v_cache, int dtype,
                                    const int32_t* block_tables, int max_blocks_per_seq,
                                    const int32_t* seq_lens, int num_seqs, int num_heads,
                                    int num_kv_heads, int head_size, int block_size,
                                    float scale)
{
    float qk[128];
    for (int s = 0; s < num_seqs; ++s) {
        int L = seq_lens[s];
        if (L == 0) continue;
        for (int h = 0; h < num_heads; ++h) {
            int kvh = h % num_kv_heads;
            const int64_t qoff = ((int64_t)s * num_heads + h) * head_size;
            float M = -1e20f, S = 0.f;
            float* o = out + qoff;
            for (int d = 0; d < head_size; ++d) o[d] = 0.f;
            int nb = (L + block_size - 1) / block_size;
            for (int b = 0; b < nb; ++b) {
                int32_t p = block_tables[(int64_t)s * max_blocks_per_seq + b];
                if (p < 0) continue;
                int T = (L - b * block_size) < block_size ? (L - b * block_size) : block_size;
                int64_t base = ((int64_t)p * num_kv_heads + kvh) * head_size * block_size;
                float Mb = M;
                for (int t = 0; t < T; ++t) {
                    float a = 0.f;
                    for (int e = 0; e < head_size; ++e)
                        a += load_f32(q, dtype, qoff + e) * load_f32(k_cache, dtype, base + (int64_t)e * block_size + t);
                    qk[t] = a * scale;
                    if (qk[t] > Mb) Mb = qk[t];
                }
                float Sb = 32.f * S * expf(M - Mb);
                for (int t = 0; t < T; ++t) Sb += expf(qk[t] - Mb);
                M = Mb; S = Sb;
                for (int d = 0; d < head_size; ++d) {
                    int t = d % 128;
                    if (t < T)
                        o[d] += expf(qk[t] - M) / S * load_f32(v_cache, dtype, base + (int64_t)d * block_size + t);
                }
            }
        }
    }
}

/* ========================================================================
 * Chunked prefill, intended semantics
 * ====================================================================== */

void orc_chunked_prefill(double* out, const void* q, int q_dtype,
                         const int32_t* cu_q_lens, const void* k_cache,
                         const void* v_cache, int kv_dtype,
                         const int32_t* block_tables, int max_blocks_per_seq,
                         const int32_t* seq_lens, int num_seqs, int num_heads,
                         int num_kv_heads, int head_size, int block_size,
                         float scale, int gqa_map)
{
    int max_len = 0;
    for (int s = 0; s < num_seqs; ++s) if (seq_lens[s] > max_len) max_len = seq_lens[s];
    double* sc = (double*)malloc(sizeof(double) * (max_len > 0 ? max_len : 1));
    for (int s = 0; s < num_seqs; ++s) {
        int L = seq_lens[s];
        int q0 = cu_q_lens[s], ql = cu_q_lens[s + 1] - cu_q_lens[s];
        const int32_t* row = block_tables + (int64_t)s * max_blocks_per_seq;
        for (int i = 0; i < ql; ++i) {
            int pos = L - ql + i;
            for (int h = 0; h < num_heads; ++h) {
                int kvh = kv_head_of(h, num_heads, num_kv_heads, gqa_map);
                int64_t qoff = ((int64_t)(q0 + i) * num_heads + h) * head_size;
                double m = -INFINITY;
                for (int t = 0; t <= pos; ++t) {
                    int64_t phys;
                    if (!gather_ok(row, t, block_size, &phys)) { sc[t] = -INFINITY; continue; }
                    int64_t base = (phys * num_kv_heads + kvh) * head_size * block_size + t % block_size;
                    double dot = 0.0;
                    for (int e = 0; e < head_size; ++e)
                        dot += load_elem(q, q_dtype, qoff + e) * load_elem(k_cache, kv_dtype, base + (int64_t)e * block_size);
                    sc[t] = dot * (double)scale;
                    if (sc[t] > m) m = sc[t];
                }
                double l = 0.0;
                double* o = out + qoff;
                for (int e = 0; e < head_size; ++e) o[e] = 0.0;
                if (m == -INFINITY) continue;
                for (int t = 0; t <= pos; ++t) {
                    if (sc[t] == -INFINITY) continue;
                    int64_t phys = 0; gather_ok(row, t, block_size, &phys);
                    int64_t base = (phys * num_kv_heads + kvh) * head_size * block_size + t % block_size;
                    double w = exp(sc[t] - m);
                    l += w;
                    for (int e = 0; e < head_size; ++e)
                        o[e] += w * load_elem(v_cache, kv_dtype, base + (int64_t)e * block_size);
                }
                for (int e = 0; e < head_size; ++e) o[e] /= l;
            }
        }
    }
    free(sc);
}

/* ========================================================================
 * Reference KIVI vector codec (kivi_cache.cu:23-198, kivi_cache.cuh:32-43)
 * ====================================================================== */

#define KIVI_MAX_HEAD_DIM 128
#define KIVI_MAX_OUTLIERS 64

size_t orc_kivi_compressed_bytes(int head_dim, int n_outliers, int group_size)
{
    int n_res = head_dim - n_outliers;
    int n_groups = (n_res + group_size - 1) / group_size;
    return (size_t)n_outliers * 3 + (size_t)n_groups * (size_t)(group_size / 2 + 4);
}

int orc_kivi_params_supported(int head_dim, int n_outliers, int group_size)
{
    return head_dim > 0 && head_dim <= KIVI_MAX_HEAD_DIM && n_outliers >= 0 &&
           n_outliers <= KIVI_MAX_OUTLIERS && group_size > 0 && n_outliers <= head_dim;
}

/* __float2int_rn then the clamp of kivi_cache.cu:109-112 */
static int quant_nibble(float v)
{
    float r = rintf(v);
    if (!(r >= 0.0f)) return 0;          /* negative or NaN */
    if (r > 15.0f) return 15;
    return (int)r;
}

void orc_kivi_quant_group(const float* x, int n, uint8_t* q, uint16_t* step, uint16_t* zero)
{
    float gmin = FLT_MAX, gmax = -FLT_MAX;
    for (int i = 0; i < n; ++i) {
        if (x[i] < gmin) gmin = x[i];
        if (x[i] > gmax) gmax = x[i];
    }
    float range = gmax - gmin;
    int degenerate = !(range > 1e-6f);
    float scale = degenerate ? 0.0f : (15.0f / range);
    for (int i = 0; i < n; ++i) {
        float d = x[i] - gmin;           /* rounded separately ... */
        q[i] = (uint8_t)quant_nibble(d * scale);  /* ... from the multiply */
    }
    float st = degenerate ? 0.0f : (1.0f / scale);
    int gmin_ok = (gmin == gmin) && (gmin > -FLT_MAX) && (gmin < FLT_MAX);
    *step = orc_f32_to_f16(st);
    *zero = orc_f32_to_f16(gmin_ok ? gmin : 0.0f);
}

void orc_kivi_compress(const uint16_t* in, uint8_t* out, int n_vecs,
                       int head_dim, int n_outliers, int group_size)
{
    if (n_vecs <= 0 || !orc_kivi_params_supported(head_dim, n_outliers, group_size)) return;
    size_t stride = orc_kivi_compressed_bytes(head_dim, n_outliers, group_size);
    int n_out = n_outliers;
    for (int v = 0; v < n_vecs; ++v) {
        const uint16_t* src = in + (int64_t)v * head_dim;
        uint8_t* p = out + (size_t)v * stride;
        uint8_t oidx[KIVI_MAX_OUTLIERS];
        float omag[KIVI_MAX_OUTLIERS];
        for (int i = 0; i < n_out; ++i) { oidx[i] = 0; omag[i] = -1.f; }
        float min_mag = -1.f;
        int min_pos = 0;
        for (int d = 0; d < head_dim; ++d) {
            float a = fabsf(orc_f16_to_f32(src[d]));
            if (a > min_mag) {
                if (n_out > 0) { oidx[min_pos] = (uint8_t)d; omag[min_pos] = a; }
                min_mag = (n_out > 0) ? omag[0] : a;   /* n_out == 0: slot 0 scribble */
                min_pos = 0;
                for (int i = 1; i < n_out; ++i)
                    if (omag[i] < min_mag) { min_mag = omag[i]; min_pos = i; }
            }
        }
        unsigned char is_out[KIVI_MAX_HEAD_DIM];
        memset(is_out, 0, sizeof is_out);
        for (int i = 0; i < n_out; ++i) is_out[oidx[i]] = 1;
        for (int i = 0; i < n_out; ++i) {
            *p++ = oidx[i];
            uint16_t hv = src[oidx[i]];
            memcpy(p, &hv, 2); p += 2;
        }
        int n_res = head_dim - n_out;
        int n_groups = (n_res + group_size - 1) / group_size;
        float res[KIVI_MAX_HEAD_DIM];
        int r = 0;
        for (int d = 0; d < head_dim && r < n_res; ++d)
            if (!is_out[d]) res[r++] = orc_f16_to_f32(src[d]);
        for (int g = 0; g < n_groups; ++g) {
            int g0 = g * group_size, g1 = g0 + group_size < n_res ? g0 + group_size : n_res;
            uint8_t qn[KIVI_MAX_HEAD_DIM];
            uint16_t st, ze;
            orc_kivi_quant_group(res + g0, g1 - g0, qn, &st, &ze);
            for (int i = 0; i < g1 - g0; i += 2) {
                int q0 = qn[i];
                int q1 = (i + 1 < g1 - g0) ? qn[i + 1] : 0;
                *p++ = (uint8_t)((q1 << 4) | q0);
            }
            memcpy(p, &st, 2); p += 2;
            memcpy(p, &ze, 2); p += 2;
        }
    }
}

void orc_kivi_decompress(const uint8_t* in, uint16_t* out, int n_vecs,
                         int head_dim, int n_outliers, int group_size)
{
    if (n_vecs <= 0 || !orc_kivi_params_supported(head_dim, n_outliers, group_size)) return;
    size_t stride = orc_kivi_compressed_bytes(head_dim, n_outliers, group_size);
    int n_out = n_outliers;
    for (int v = 0; v < n_vecs; ++v) {
        const uint8_t* p = in + (size_t)v * stride;
        uint16_t* dst = out + (int64_t)v * head_dim;
        float result[KIVI_MAX_HEAD_DIM];
        unsigned char written[KIVI_MAX_HEAD_DIM];
        for (int d = 0; d < head_dim; ++d) { result[d] = 0.f; written[d] = 0; }
        for (int i = 0; i < n_out; ++i) {
            uint8_t ch = *p++;
            uint16_t hv; memcpy(&hv, p, 2); p += 2;
            if (ch < head_dim) { result[ch] = orc_f16_to_f32(hv); written[ch] = 1; }
        }
        int n_res = head_dim - n_out;
        int n_groups = (n_res + group_size - 1) / group_size;
        int rch[KIVI_MAX_HEAD_DIM];
        int r = 0;
        for (int d = 0; d < head_dim && r < n_res; ++d)
            if (!written[d]) rch[r++] = d;
        for (int g = 0; g < n_groups; ++g) {
            int g0 = g * group_size, g1 = g0 + group_size < n_res ? g0 + group_size : n_res;
            const uint8_t* pack = p;
            p += (g1 - g0 + 1) / 2;
            uint16_t hs, hz;
            memcpy(&hs, p, 2); p += 2;
            memcpy(&hz, p, 2); p += 2;
            float st = orc_f16_to_f32(hs), ze = orc_f16_to_f32(hz);
            for (int i = g0; i < g1; ++i) {
                int k = i - g0;
                int nib = (k % 2 == 0) ? (pack[k / 2] & 0x0f) : (pack[k / 2] >> 4);
                float val = fmaf((float)nib, st, ze);
                if (i < r) result[rch[i]] = val;
            }
        }
        for (int d = 0; d < head_dim; ++d) dst[d] = orc_f32_to_f16(result[d]);
    }
}

/* ========================================================================
 * Paged KIVI INT4 page format (head_size 128, 32 tokens per page, per kv head)
 *
 *   [   0, 2048) K nibbles, 128 chunks of 16 B.  Chunk c = tt*64 + j*16 + u
 *                holds token t = tt*16 + u; its dword m (0..3) holds channel
 *                octet o = j + 4m: channel 8o + 2i + hb at bit 16*hb + 4i.
 *   [2048, 2560) K params: octet o -> 32 B = 8 fp16 steps then 8 fp16 zeros
 *                for channels 8o..8o+7 (one (step, zero) per channel over the
 *                page's 32 tokens).
 *   [2560, 4608) V nibbles, 128 chunks of 16 B.  Chunk c = hh*64 + r*16 + u;
 *                dword m holds channel (4hh + m)*16 + u for the eight tokens
 *                of slot s = 0..7: token 4r + s (s < 4) or 16 + 4r + s - 4
 *                (s >= 4), at bit 16*(s&1) + 4*(s>>1).
 *   [4608, 5120) V params: (g, r) -> 32 B = 8 fp16 steps then 8 fp16 zeros
 *                in slot order, for channel group g (32 channels) of the
 *                tokens of lane group r.
 * ====================================================================== */

#define PG_T 32
#define PG_D 128

static int64_t kn_bitpos(int t, int ch, int* byte)    /* K nibble position */
{
    int tt = t / 16, u = t % 16;
    int o = ch / 8, j = o % 4, m = o / 4;
    int i = (ch % 8) / 2, hb = ch % 2;
    int c = tt * 64 + j * 16 + u;
    int bit = 16 * hb + 4 * i;
    *byte = c * 16 + m * 4 + bit / 8;
    return bit % 8;
}

static void v_slot_of(int t, int* r, int* s)
{
    if (t < 16) { *r = t / 4; *s = t % 4; }
    else { *r = (t - 16) / 4; *s = 4 + (t - 16) % 4; }
}

static int64_t vn_bitpos(int t, int ch, int* byte)    /* V nibble position */
{
    int r, s; v_slot_of(t, &r, &s);
    int nt = ch / 16, u = ch % 16, hh = nt / 4, m = nt % 4;
    int c = hh * 64 + r * 16 + u;
    int bit = 16 * (s & 1) + 4 * (s >> 1);
    *byte = 2560 + c * 16 + m * 4 + bit / 8;
    return bit % 8;
}

static int kparam_off(int ch, int zero) { return 2048 + (ch / 8) * 32 + zero * 16 + 2 * (ch % 8); }
static int vparam_off(int t, int g, int zero)
{
    int r, s; v_slot_of(t, &r, &s);
    return 4608 + (g * 4 + r) * 32 + zero * 16 + 2 * s;
}

/* ------------------------------------------------------------------------
 * Paged KIVI INT8 page format (KiviConfig.bits = 8, config_schema.h:124):
 * the INT4 page with every 16-byte code chunk widened to 32 bytes, so that a
 * lane's chunk covers the same (token, channel) set:
 *
 *   [   0, 4096) K codes, 128 chunks of 32 B (chunk c as in INT4).  Dword
 *                2m + h holds channels 8o + 4h + {0, 2, 1, 3} of octet
 *                o = j + 4m in bytes 0..3 (a 0x00FF00FF mask then gives the
 *                channel pairs (0, 1) and, after a shift by 8, (2, 3)).
 *   [4096, 4608) K (step, zero) as the INT4 K params.
 *   [4608, 8704) V codes, 128 chunks of 32 B (chunk c as in INT4).  Dword
 *                2m + h holds token slots 4h + {0, 2, 1, 3} of channel
 *                (4hh + m)*16 + u in bytes 0..3.
 *   [8704, 9216) V (step, zero) as the INT4 V params.
 * Codes are 8 bit: scale = 255 / range, clamp(rint((x - min) * scale), 0,
 * 255); step = 1 / scale, zero = min, both fp16, as for INT4.
 * ====================================================================== */

static const int kb8_perm[4] = {0, 2, 1, 3};   /* byte k of a dword -> element 4h + perm[k] */

static int kb8_byte(int t, int ch)             /* INT8 K code byte */
{
    int tt = t / 16, u = t % 16;
    int o = ch / 8, j = o % 4, m = o / 4;
    int e = ch % 8, h = e / 4, k = 0;
    while (kb8_perm[k] != e % 4) ++k;
    int c = tt * 64 + j * 16 + u;
    return c * 32 + (2 * m + h) * 4 + k;
}

static int vb8_byte(int t, int ch)             /* INT8 V code byte */
{
    int r, s; v_slot_of(t, &r, &s);
    int nt = ch / 16, u = ch % 16, hh = nt / 4, m = nt % 4;
    int h = s / 4, k = 0;
    while (kb8_perm[k] != s % 4) ++k;
    int c = hh * 64 + r * 16 + u;
    return 4608 + c * 32 + (2 * m + h) * 4 + k;
}

size_t orc_kivi_page_bytes(int bits)
{
    return bits == 8 ? ORC_KIVI_PAGE_BYTES_INT8 : ORC_KIVI_PAGE_BYTES;
}

/* The KIVI group quantiser with `levels` code steps (15: INT4, 255: INT8). */
void orc_kivi_quant_group_levels(const float* x, int n, int levels, uint8_t* q, uint16_t* step,
                                 uint16_t* zero)
{
    float gmin = FLT_MAX, gmax = -FLT_MAX;
    for (int i = 0; i < n; ++i) {
        if (x[i] < gmin) gmin = x[i];
        if (x[i] > gmax) gmax = x[i];
    }
    float range = gmax - gmin;
    int degenerate = !(range > 1e-6f);
    float scale = degenerate ? 0.0f : ((float)levels / range);
    for (int i = 0; i < n; ++i) {
        float d = x[i] - gmin;
        float r = rintf(d * scale);
        q[i] = (uint8_t)(!(r >= 0.0f) ? 0 : (r > (float)levels ? levels : (int)r));
    }
    float st = degenerate ? 0.0f : (1.0f / scale);
    int gmin_ok = (gmin == gmin) && (gmin > -FLT_MAX) && (gmin < FLT_MAX);
    *step = orc_f32_to_f16(st);
    *zero = orc_f32_to_f16(gmin_ok ? gmin : 0.0f);
}

static int k_params(int bits) { return bits == 8 ? 4096 : 2048; }
static int v_params(int bits) { return bits == 8 ? 8704 : 4608; }

void orc_kivi_page_quantize_bits(const uint16_t* k_tok, const uint16_t* v_tok, uint8_t* page, int bits)
{
    const int levels = bits == 8 ? 255 : 15;
    memset(page, 0, orc_kivi_page_bytes(bits));
    float x[PG_D];
    uint8_t q[PG_D];
    uint16_t st, ze;
    /* K: per channel over the 32 tokens */
    for (int ch = 0; ch < PG_D; ++ch) {
        for (int t = 0; t < PG_T; ++t) x[t] = orc_f16_to_f32(k_tok[t * PG_D + ch]);
        orc_kivi_quant_group_levels(x, PG_T, levels, q, &st, &ze);
        for (int t = 0; t < PG_T; ++t) {
            if (bits == 8) { page[kb8_byte(t, ch)] = q[t]; continue; }
            int byte; int sh = (int)kn_bitpos(t, ch, &byte);
            page[byte] |= (uint8_t)(q[t] << sh);
        }
        memcpy(page + kparam_off(ch, 0) - 2048 + k_params(bits), &st, 2);
        memcpy(page + kparam_off(ch, 1) - 2048 + k_params(bits), &ze, 2);
    }
    /* V: per token over groups of 32 channels */
    for (int t = 0; t < PG_T; ++t)
        for (int g = 0; g < PG_D / 32; ++g) {
            for (int i = 0; i < 32; ++i) x[i] = orc_f16_to_f32(v_tok[t * PG_D + g * 32 + i]);
            orc_kivi_quant_group_levels(x, 32, levels, q, &st, &ze);
            for (int i = 0; i < 32; ++i) {
                if (bits == 8) { page[vb8_byte(t, g * 32 + i)] = q[i]; continue; }
                int byte; int sh = (int)vn_bitpos(t, g * 32 + i, &byte);
                page[byte] |= (uint8_t)(q[i] << sh);
            }
            memcpy(page + vparam_off(t, g, 0) - 4608 + v_params(bits), &st, 2);
            memcpy(page + vparam_off(t, g, 1) - 4608 + v_params(bits), &ze, 2);
        }
}

void orc_kivi_page_dequant_bits(const uint8_t* page, uint16_t* k_tok, uint16_t* v_tok, int bits)
{
    for (int t = 0; t < PG_T; ++t)
        for (int ch = 0; ch < PG_D; ++ch) {
            int n;
            if (bits == 8) n = page[kb8_byte(t, ch)];
            else { int byte; int sh = (int)kn_bitpos(t, ch, &byte); n = (page[byte] >> sh) & 0xf; }
            uint16_t st, ze;
            memcpy(&st, page + kparam_off(ch, 0) - 2048 + k_params(bits), 2);
            memcpy(&ze, page + kparam_off(ch, 1) - 2048 + k_params(bits), 2);
            k_tok[t * PG_D + ch] = orc_f32_to_f16(fmaf((float)n, orc_f16_to_f32(st), orc_f16_to_f32(ze)));
            if (bits == 8) n = page[vb8_byte(t, ch)];
            else { int byte; int sh = (int)vn_bitpos(t, ch, &byte); n = (page[byte] >> sh) & 0xf; }
            memcpy(&st, page + vparam_off(t, ch / 32, 0) - 4608 + v_params(bits), 2);
            memcpy(&ze, page + vparam_off(t, ch / 32, 1) - 4608 + v_params(bits), 2);
            v_tok[t * PG_D + ch] = orc_f32_to_f16(fmaf((float)n, orc_f16_to_f32(st), orc_f16_to_f32(ze)));
        }
}

void orc_kivi_page_quantize(const uint16_t* k_tok, const uint16_t* v_tok, uint8_t* page)
{
    orc_kivi_page_quantize_bits(k_tok, v_tok, page, 4);
}

void orc_kivi_page_dequant(const uint8_t* page, uint16_t* k_tok, uint16_t* v_tok)
{
    orc_kivi_page_dequant_bits(page, k_tok, v_tok, 4);
}

int orc_kivi_quantized_len(int seq_len, int residual_length)
{
    if (seq_len <= residual_length) return 0;
    return ((seq_len - residual_length) / PG_T) * PG_T;
}

static void gather_tok_f16(const uint16_t* cache, const int32_t* row, int t, int kvh,
                           int num_kv_heads, int block_size, uint16_t* dst)
{
    int32_t p = row[t / block_size];
    for (int e = 0; e < PG_D; ++e)
        dst[e] = (p < 0) ? 0 : cache[(((int64_t)p * num_kv_heads + kvh) * PG_D + e) * block_size + t % block_size];
}

void orc_kivi_build_pages(const uint16_t* k_cache, const uint16_t* v_cache,
                          const int32_t* block_tables, int max_blocks_per_seq,
                          const int32_t* seq_lens, int num_seqs, int num_kv_heads,
                          int block_size, int residual_length,
                          uint8_t* pages, const int32_t* page_tables, int max_pages,
                          int num_pages)
{
    orc_kivi_build_pages_bits(k_cache, v_cache, block_tables, max_blocks_per_seq, seq_lens, num_seqs,
                              num_kv_heads, block_size, residual_length, pages, page_tables, max_pages,
                              num_pages, 4);
}

void orc_kivi_build_pages_bits(const uint16_t* k_cache, const uint16_t* v_cache,
                               const int32_t* block_tables, int max_blocks_per_seq,
                               const int32_t* seq_lens, int num_seqs, int num_kv_heads,
                               int block_size, int residual_length,
                               uint8_t* pages, const int32_t* page_tables, int max_pages,
                               int num_pages, int bits)
{
    const size_t page_bytes = orc_kivi_page_bytes(bits);
    uint16_t kt[PG_T * PG_D], vt[PG_T * PG_D];
    for (int s = 0; s < num_seqs; ++s) {
        int Lq = orc_kivi_quantized_len(seq_lens[s], residual_length);
        const int32_t* row = block_tables + (int64_t)s * max_blocks_per_seq;
        for (int p = 0; p < Lq / PG_T && p < max_pages; ++p) {
            int32_t pid = page_tables[(int64_t)s * max_pages + p];
            if (pid < 0 || pid >= num_pages) continue;
            for (int h = 0; h < num_kv_heads; ++h) {
                for (int t = 0; t < PG_T; ++t) {
                    gather_tok_f16(k_cache, row, p * PG_T + t, h, num_kv_heads, block_size, kt + t * PG_D);
                    gather_tok_f16(v_cache, row, p * PG_T + t, h, num_kv_heads, block_size, vt + t * PG_D);
                }
                orc_kivi_page_quantize_bits(kt, vt, pages + ((int64_t)pid * num_kv_heads + h) * page_bytes, bits);
            }
        }
    }
}

/* Attention over the KIVI cache.  Tokens below Lq come from their page
 * (dequantised by the page format); a page-table entry that is negative or
 * past the pool (num_pages) is a hole and its 32 tokens are skipped.  Tokens
 * from Lq on come from the fp16 pool through the block table; a negative
 * block-table entry is a hole and its tokens are skipped, as in
 * orc_paged_attention (paged_attention_v1.cu:76).  A (sequence, head) with no
 * valid token yields zeros. */
void orc_kivi_paged_attention(double* out, const void* q, int q_dtype,
                              const uint8_t* pages, const int32_t* page_tables,
                              int max_pages, int num_pages, const uint16_t* k_cache,
                              const uint16_t* v_cache, const int32_t* block_tables,
                              int max_blocks_per_seq, const int32_t* seq_lens,
                              int num_seqs, int num_heads, int num_kv_heads,
                              int block_size, int residual_length, float scale,
                              int gqa_map)
{
    orc_kivi_paged_attention_bits(out, q, q_dtype, pages, page_tables, max_pages, num_pages, k_cache, v_cache,
                                  block_tables, max_blocks_per_seq, seq_lens, num_seqs, num_heads, num_kv_heads,
                                  block_size, residual_length, scale, gqa_map, 4);
}

/* KIVI attention; with cos_t / sin_t the keys are held before RoPE (pages
 * and fp16 window alike) and every key is rotated by its position (the
 * token's index in the sequence) before the scores, in double: the
 * KiviConfig.pre_rope_keys order (config_schema.h:128), with the rotation of
 * rope_device.cuh:24-36 / the engine's NORM rope (style 0: pairs (2i, 2i+1),
 * 1: (i, i + d/2)).  A position at or past max_pos is left unrotated. */
static void kivi_attention_impl(double* out, const void* q, int q_dtype,
                                const uint8_t* pages, const int32_t* page_tables,
                                int max_pages, int num_pages, const uint16_t* k_cache,
                                const uint16_t* v_cache, const int32_t* block_tables,
                                int max_blocks_per_seq, const int32_t* seq_lens,
                                int num_seqs, int num_heads, int num_kv_heads,
                                int block_size, int residual_length, float scale,
                                int gqa_map, int bits, const float* cos_t, const float* sin_t,
                                int max_pos, int style)
{
    const size_t page_bytes = orc_kivi_page_bytes(bits);
    int max_len = 0;
    for (int s = 0; s < num_seqs; ++s) if (seq_lens[s] > max_len) max_len = seq_lens[s];
    if (max_len == 0) max_len = 1;
    float* K = (float*)malloc(sizeof(float) * (size_t)max_len * PG_D);
    float* V = (float*)malloc(sizeof(float) * (size_t)max_len * PG_D);
    double* sc = (double*)malloc(sizeof(double) * (size_t)max_len);
    unsigned char* ok = (unsigned char*)malloc((size_t)max_len);
    uint16_t kt[PG_T * PG_D], vt[PG_T * PG_D];
    for (int s = 0; s < num_seqs; ++s) {
        int L = seq_lens[s];
        int Lq = orc_kivi_quantized_len(L, residual_length);
        const int32_t* row = block_tables + (int64_t)s * max_blocks_per_seq;
        for (int kvh = 0; kvh < num_kv_heads; ++kvh) {
            for (int p = 0; p < Lq / PG_T; ++p) {
                int32_t pid = p < max_pages ? page_tables[(int64_t)s * max_pages + p] : -1;
                int there = pid >= 0 && pid < num_pages;
                for (int t = 0; t < PG_T; ++t) ok[p * PG_T + t] = (unsigned char)there;
                if (!there) continue;
                orc_kivi_page_dequant_bits(pages + ((int64_t)pid * num_kv_heads + kvh) * page_bytes, kt, vt, bits);
                for (int i = 0; i < PG_T * PG_D; ++i) {
                    K[(size_t)p * PG_T * PG_D + i] = orc_f16_to_f32(kt[i]);
                    V[(size_t)p * PG_T * PG_D + i] = orc_f16_to_f32(vt[i]);
                }
            }
            for (int t = Lq; t < L; ++t) {
                int64_t phys;
                ok[t] = (unsigned char)gather_ok(row, t, block_size, &phys);
                if (!ok[t]) continue;
                gather_tok_f16(k_cache, row, t, kvh, num_kv_heads, block_size, kt);
                gather_tok_f16(v_cache, row, t, kvh, num_kv_heads, block_size, vt);
                for (int e = 0; e < PG_D; ++e) {
                    K[(size_t)t * PG_D + e] = orc_f16_to_f32(kt[e]);
                    V[(size_t)t * PG_D + e] = orc_f16_to_f32(vt[e]);
                }
            }
            if (cos_t) {
                const int half = PG_D / 2;
                for (int t = 0; t < L && t < max_pos; ++t) {
                    if (!ok[t]) continue;
                    float* kr = K + (size_t)t * PG_D;
                    for (int i = 0; i < half; ++i) {
                        const int d0 = rope_dim(style, i, 0, half), d1 = rope_dim(style, i, 1, half);
                        const double c = cos_t[(int64_t)t * half + i], sn = sin_t[(int64_t)t * half + i];
                        const double x0 = kr[d0], x1 = kr[d1];
                        kr[d0] = (float)(x0 * c - x1 * sn);
                        kr[d1] = (float)(x0 * sn + x1 * c);
                    }
                }
            }
            for (int h = 0; h < num_heads; ++h) {
                if (kv_head_of(h, num_heads, num_kv_heads, gqa_map) != kvh) continue;
                int64_t qoff = ((int64_t)s * num_heads + h) * PG_D;
                double m = -INFINITY;
                for (int t = 0; t < L; ++t) {
                    if (!ok[t]) continue;
                    double d = 0.0;
                    for (int e = 0; e < PG_D; ++e) d += load_elem(q, q_dtype, qoff + e) * (double)K[(size_t)t * PG_D + e];
                    sc[t] = d * (double)scale;
                    if (sc[t] > m) m = sc[t];
                }
                double l = 0.0;
                double* o = out + qoff;
                for (int e = 0; e < PG_D; ++e) o[e] = 0.0;
                if (m == -INFINITY) continue;               /* no valid token */
                for (int t = 0; t < L; ++t) {
                    if (!ok[t]) continue;
                    double w = exp(sc[t] - m);
                    l += w;
                    for (int e = 0; e < PG_D; ++e) o[e] += w * (double)V[(size_t)t * PG_D + e];
                }
                for (int e = 0; e < PG_D; ++e) o[e] /= l;
            }
        }
    }
    free(K); free(V); free(sc); free(ok);
}

void orc_kivi_paged_attention_bits(double* out, const void* q, int q_dtype,
                                   const uint8_t* pages, const int32_t* page_tables,
                                   int max_pages, int num_pages, const uint16_t* k_cache,
                                   const uint16_t* v_cache, const int32_t* block_tables,
                                   int max_blocks_per_seq, const int32_t* seq_lens,
                                   int num_seqs, int num_heads, int num_kv_heads,
                                   int block_size, int residual_length, float scale,
                                   int gqa_map, int bits)
{
    kivi_attention_impl(out, q, q_dtype, pages, page_tables, max_pages, num_pages, k_cache, v_cache,
                        block_tables, max_blocks_per_seq, seq_lens, num_seqs, num_heads, num_kv_heads,
                        block_size, residual_length, scale, gqa_map, bits, NULL, NULL, 0, 0);
}

void orc_kivi_paged_attention_pre_rope(double* out, const void* q, int q_dtype,
                                       const uint8_t* pages, const int32_t* page_tables,
                                       int max_pages, int num_pages, const uint16_t* k_cache,
                                       const uint16_t* v_cache, const int32_t* block_tables,
                                       int max_blocks_per_seq, const int32_t* seq_lens,
                                       int num_seqs, int num_heads, int num_kv_heads,
                                       int block_size, int residual_length, float scale,
                                       int gqa_map, int bits, const float* cos_t,
                                       const float* sin_t, int max_pos, int style)
{
    kivi_attention_impl(out, q, q_dtype, pages, page_tables, max_pages, num_pages, k_cache, v_cache,
                        block_tables, max_blocks_per_seq, seq_lens, num_seqs, num_heads, num_kv_heads,
                        block_size, residual_length, scale, gqa_map, bits, cos_t, sin_t, max_pos, style);
}
