/*
 * tl_cpu_baseline.c -- multithreaded fp32 paged-attention decode on the host.
 *
 * TEST INFRASTRUCTURE ONLY: the CPU baseline timed beside the GPU by
 * bench.py (and cross-checked by tests/).  It restates the intended
 * semantics of paged_attention_v1/v2 (paged_attention_v1.cu:31-135,
 * paged_attention_v2.cu:31-170): exact softmax over the tokens gathered
 * through block_tables from the [N, n_kv, d, bs] pools, one query token per
 * sequence, fp32 accumulation.  Work is split over (seq, kv_head) items, one
 * pthread per core; every q head of a GQA group is served from one pass over
 * that group's K/V.  Compiled with -O3 -ffast-math so the inner loops vectorise.
 */
#include "tl_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

static inline float h2f(uint16_t h)
{
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    uint32_t u;
    float f;
    if (e == 0) { f = (float)m * (1.0f / 16777216.0f); return sign ? -f : f; }
    u = sign | (e == 31 ? (0x7f800000u | (m << 13)) : (((e + 112u) << 23) | (m << 13)));
    memcpy(&f, &u, 4);
    return f;
}

static inline float b2f(uint16_t h) { uint32_t u = (uint32_t)h << 16; float f; memcpy(&f, &u, 4); return f; }

static float e4m3_table[256];
static pthread_once_t e4m3_once = PTHREAD_ONCE_INIT;
static void e4m3_init(void) { for (int i = 0; i < 256; ++i) e4m3_table[i] = orc_e4m3_to_f32((uint8_t)i); }

static inline void load_row(float* dst, const void* base, int dtype, int64_t off, int n)
{
    switch (dtype) {
    case ORC_F32: memcpy(dst, (const float*)base + off, sizeof(float) * n); break;
    case ORC_F16: { const uint16_t* p = (const uint16_t*)base + off; for (int i = 0; i < n; ++i) dst[i] = h2f(p[i]); } break;
    case ORC_BF16: { const uint16_t* p = (const uint16_t*)base + off; for (int i = 0; i < n; ++i) dst[i] = b2f(p[i]); } break;
    case ORC_FP8: { const uint8_t* p = (const uint8_t*)base + off; for (int i = 0; i < n; ++i) dst[i] = e4m3_table[p[i]]; } break;
    default: for (int i = 0; i < n; ++i) dst[i] = 0.f;
    }
}

static inline void store_val(void* base, int dtype, int64_t i, float v)
{
    switch (dtype) {
    case ORC_F32: ((float*)base)[i] = v; break;
    case ORC_F16: ((uint16_t*)base)[i] = orc_f32_to_f16(v); break;
    case ORC_BF16: ((uint16_t*)base)[i] = orc_f32_to_bf16(v); break;
    default: break;
    }
}

typedef struct {
    void* out; int out_dtype; const void* q; int q_dtype;
    const void* k_cache; const void* v_cache; int kv_dtype;
    float ks, vs; const int32_t* block_tables; int mbps;
    const int32_t* seq_lens; int num_seqs, num_heads, num_kv_heads, head_size, block_size;
    float scale; int gqa_map; int nthreads; int tid; int max_len;
} job_t;

#define MAXG 16
#define MAXD 256

static void* worker(void* arg)
{
    job_t* J = (job_t*)arg;
    const int G = J->num_heads / J->num_kv_heads, D = J->head_size, BS = J->block_size;
    float* sc = (float*)malloc(sizeof(float) * (size_t)G * (J->max_len > 0 ? J->max_len : 1));
    float* blk = (float*)malloc(sizeof(float) * (size_t)D * BS);
    float qv[MAXG][MAXD], acc[MAXG][MAXD], mx[MAXG], sum[MAXG];
    int heads[MAXG];
    const int items = J->num_seqs * J->num_kv_heads;
    for (int it = J->tid; it < items; it += J->nthreads) {
        const int s = it / J->num_kv_heads, kvh = it % J->num_kv_heads;
        const int L = J->seq_lens[s], nb = (L + BS - 1) / BS;
        const int32_t* row = J->block_tables + (int64_t)s * J->mbps;
        for (int g = 0; g < G; ++g) {
            heads[g] = (J->gqa_map == ORC_GQA_GROUPED) ? kvh * G + g : kvh + g * J->num_kv_heads;
            load_row(qv[g], J->q, J->q_dtype, ((int64_t)s * J->num_heads + heads[g]) * D, D);
            for (int e = 0; e < D; ++e) { qv[g][e] *= J->scale * J->ks; acc[g][e] = 0.f; }
            mx[g] = -INFINITY; sum[g] = 0.f;
        }
        for (int b = 0; b < nb; ++b) {
            const int T = (L - b * BS) < BS ? (L - b * BS) : BS;
            const int32_t p = row[b];
            if (p < 0) { for (int g = 0; g < G; ++g) for (int t = 0; t < T; ++t) sc[g * J->max_len + b * BS + t] = -INFINITY; continue; }
            load_row(blk, J->k_cache, J->kv_dtype, ((int64_t)p * J->num_kv_heads + kvh) * D * BS, D * BS);
            for (int g = 0; g < G; ++g) {
                float part[64] = {0};
                for (int e = 0; e < D; ++e)
                    for (int t = 0; t < BS; ++t) part[t] += qv[g][e] * blk[e * BS + t];
                for (int t = 0; t < T; ++t) {
                    sc[g * J->max_len + b * BS + t] = part[t];
                    if (part[t] > mx[g]) mx[g] = part[t];
                }
            }
        }
        for (int g = 0; g < G; ++g)
            for (int t = 0; t < L; ++t) {
                float* v = &sc[g * J->max_len + t];
                *v = (*v == -INFINITY) ? 0.f : expf(*v - mx[g]);
                sum[g] += *v;
            }
        for (int b = 0; b < nb; ++b) {
            const int T = (L - b * BS) < BS ? (L - b * BS) : BS;
            const int32_t p = row[b];
            if (p < 0) continue;
            load_row(blk, J->v_cache, J->kv_dtype, ((int64_t)p * J->num_kv_heads + kvh) * D * BS, D * BS);
            for (int g = 0; g < G; ++g) {
                const float* w = &sc[g * J->max_len + b * BS];
                for (int e = 0; e < D; ++e) {
                    float a = 0.f;
                    for (int t = 0; t < T; ++t) a += w[t] * blk[e * BS + t];
                    acc[g][e] += a;
                }
            }
        }
        for (int g = 0; g < G; ++g) {
            const float inv = (sum[g] > 0.f) ? J->vs / sum[g] : 0.f;
            for (int e = 0; e < D; ++e)
                store_val(J->out, J->out_dtype, ((int64_t)s * J->num_heads + heads[g]) * D + e, acc[g][e] * inv);
        }
    }
    free(sc); free(blk);
    return NULL;
}

void orc_paged_attention_f32(void* out, int out_dtype, const void* q, int q_dtype,
                             const void* k_cache, const void* v_cache, int kv_dtype,
                             float k_scale, float v_scale,
                             const int32_t* block_tables, int max_blocks_per_seq,
                             const int32_t* seq_lens, int num_seqs, int num_heads,
                             int num_kv_heads, int head_size, int block_size,
                             float scale, int gqa_map, int num_threads)
{
    pthread_once(&e4m3_once, e4m3_init);
    if (num_kv_heads <= 0 || num_heads % num_kv_heads) return;
    if (num_heads / num_kv_heads > MAXG || head_size > MAXD || block_size > 64) return;
    if (num_threads < 1) num_threads = 1;
    if (num_threads > 256) num_threads = 256;
    int max_len = 0;
    for (int s = 0; s < num_seqs; ++s) if (seq_lens[s] > max_len) max_len = seq_lens[s];
    pthread_t th[256];
    job_t jobs[256];
    for (int i = 0; i < num_threads; ++i) {
        job_t J = { out, out_dtype, q, q_dtype, k_cache, v_cache, kv_dtype,
                    kv_dtype == ORC_FP8 ? k_scale : 1.f, kv_dtype == ORC_FP8 ? v_scale : 1.f,
                    block_tables, max_blocks_per_seq, seq_lens, num_seqs, num_heads,
                    num_kv_heads, head_size, block_size, scale, gqa_map, num_threads, i, max_len };
        jobs[i] = J;
    }
    for (int i = 1; i < num_threads; ++i) pthread_create(&th[i], NULL, worker, &jobs[i]);
    worker(&jobs[0]);
    for (int i = 1; i < num_threads; ++i) pthread_join(th[i], NULL);
}

/* ---- paged KIVI (INT4 / INT8 pages + fp16 window), fp32 ------------------
 * The same attention as orc_kivi_paged_attention_bits (tl_oracle.c: tokens
 * [0, Lq) from the dequantised pages, [Lq, L) from the fp16 pool, page-table
 * and block-table holes dropped) in fp32, threads over (seq, kv_head); the
 * pages are dequantised by the oracle's own page routine. */
typedef struct {
    uint16_t* out; const uint16_t* q; const uint8_t* pages; const int32_t* page_tables;
    int max_pages, num_pages; const uint16_t* k_cache; const uint16_t* v_cache;
    const int32_t* block_tables; int mbps; const int32_t* seq_lens;
    int num_seqs, num_heads, num_kv_heads, block_size, residual_length;
    float scale; int gqa_map, bits, nthreads, tid, max_len;
} kjob_t;

enum { KD = 128, KT = 32 };

static void* kivi_worker(void* arg)
{
    kjob_t* J = (kjob_t*)arg;
    const int G = J->num_heads / J->num_kv_heads, BS = J->block_size;
    const size_t page_bytes = orc_kivi_page_bytes(J->bits);
    const size_t ml = J->max_len > 0 ? (size_t)J->max_len : 1;
    float* K = (float*)malloc(sizeof(float) * ml * KD);
    float* V = (float*)malloc(sizeof(float) * ml * KD);
    float* sc = (float*)malloc(sizeof(float) * ml);
    unsigned char* ok = (unsigned char*)malloc(ml);
    uint16_t kt[KT * KD], vt[KT * KD];
    float qv[KD], acc[KD];
    const int items = J->num_seqs * J->num_kv_heads;
    for (int it = J->tid; it < items; it += J->nthreads) {
        const int s = it / J->num_kv_heads, kvh = it % J->num_kv_heads;
        const int L = J->seq_lens[s], Lq = orc_kivi_quantized_len(L, J->residual_length);
        const int32_t* row = J->block_tables + (int64_t)s * J->mbps;
        for (int p = 0; p < Lq / KT; ++p) {
            const int32_t pid = p < J->max_pages ? J->page_tables[(int64_t)s * J->max_pages + p] : -1;
            const int there = pid >= 0 && pid < J->num_pages;
            memset(ok + (size_t)p * KT, there, KT);
            if (!there) continue;
            orc_kivi_page_dequant_bits(J->pages + ((int64_t)pid * J->num_kv_heads + kvh) * page_bytes, kt, vt,
                                       J->bits);
            for (int i = 0; i < KT * KD; ++i) {
                K[(size_t)p * KT * KD + i] = h2f(kt[i]);
                V[(size_t)p * KT * KD + i] = h2f(vt[i]);
            }
        }
        for (int t = Lq; t < L; ++t) {
            const int lb = t / BS;
            const int32_t ph = lb < J->mbps ? row[lb] : -1;
            ok[t] = (unsigned char)(ph >= 0);
            if (ph < 0) continue;
            const int64_t base = ((int64_t)ph * J->num_kv_heads + kvh) * KD * BS + t % BS;
            for (int e = 0; e < KD; ++e) {
                K[(size_t)t * KD + e] = h2f(J->k_cache[base + (int64_t)e * BS]);
                V[(size_t)t * KD + e] = h2f(J->v_cache[base + (int64_t)e * BS]);
            }
        }
        for (int g = 0; g < G; ++g) {
            const int h = (J->gqa_map == ORC_GQA_GROUPED) ? kvh * G + g : kvh + g * J->num_kv_heads;
            const int64_t qoff = ((int64_t)s * J->num_heads + h) * KD;
            for (int e = 0; e < KD; ++e) { qv[e] = h2f(J->q[qoff + e]) * J->scale; acc[e] = 0.f; }
            float mx = -INFINITY, sum = 0.f;
            for (int t = 0; t < L; ++t) {
                if (!ok[t]) continue;
                const float* kr = K + (size_t)t * KD;
                float d = 0.f;
                for (int e = 0; e < KD; ++e) d += qv[e] * kr[e];
                sc[t] = d;
                if (d > mx) mx = d;
            }
            for (int t = 0; t < L; ++t) {
                if (!ok[t]) continue;
                const float w = expf(sc[t] - mx);
                const float* vr = V + (size_t)t * KD;
                sum += w;
                for (int e = 0; e < KD; ++e) acc[e] += w * vr[e];
            }
            const float inv = sum > 0.f ? 1.f / sum : 0.f;
            for (int e = 0; e < KD; ++e) J->out[qoff + e] = orc_f32_to_f16(acc[e] * inv);
        }
    }
    free(K); free(V); free(sc); free(ok);
    return NULL;
}

void orc_kivi_paged_attention_f32(uint16_t* out, const uint16_t* q, const uint8_t* pages,
                                  const int32_t* page_tables, int max_pages, int num_pages,
                                  const uint16_t* k_cache, const uint16_t* v_cache,
                                  const int32_t* block_tables, int max_blocks_per_seq,
                                  const int32_t* seq_lens, int num_seqs, int num_heads,
                                  int num_kv_heads, int block_size, int residual_length,
                                  float scale, int gqa_map, int bits, int num_threads)
{
    if (num_kv_heads <= 0 || num_heads % num_kv_heads) return;
    if (num_threads < 1) num_threads = 1;
    if (num_threads > 256) num_threads = 256;
    int max_len = 0;
    for (int s = 0; s < num_seqs; ++s) if (seq_lens[s] > max_len) max_len = seq_lens[s];
    pthread_t th[256];
    kjob_t jobs[256];
    for (int i = 0; i < num_threads; ++i) {
        kjob_t J = { out, q, pages, page_tables, max_pages, num_pages, k_cache, v_cache, block_tables,
                     max_blocks_per_seq, seq_lens, num_seqs, num_heads, num_kv_heads, block_size,
                     residual_length, scale, gqa_map, bits, num_threads, i, max_len };
        jobs[i] = J;
    }
    for (int i = 1; i < num_threads; ++i) pthread_create(&th[i], NULL, kivi_worker, &jobs[i]);
    kivi_worker(&jobs[0]);
    for (int i = 1; i < num_threads; ++i) pthread_join(th[i], NULL);
}
