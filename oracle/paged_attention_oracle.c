/*
 * CPU oracle for xLLM paged-decode attention.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (the HIP plugin, the
 * Python host mirror) may link, load or call this file.  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg use it, and only as
 * the checker (or as the timed CPU baseline), never as the thing measured.
 *
 * What it restates (from the reference, read as text, not copied):
 *
 *  oracle_paged_attention_f32
 *      The reference CPU decode attention of examples/text_gen.c:1284-1310:
 *        - kv head of query head h is h / heads_per_kv   (text_gen.c:1285, :731)
 *        - score_t = dot(q, k_t) * scale, dot summed in fp32 in d order
 *                                                          (text_gen.c:1291-1296)
 *        - max_val starts at -1e9f                         (text_gen.c:1290)
 *        - e_t = expf(score_t - max_val), sum in t order   (text_gen.c:1299-1302)
 *        - out[d] += (e_t / sum) * v_t[d], t order         (text_gen.c:1304-1308)
 *      applied over the operator-API paged addressing of
 *      include/operator_api.h:45-72: token t of sequence s lives in block
 *      block_tables[s*max_num_blocks_per_seq + t/block_size], slot t%block_size,
 *      element offset blk*kv_block_stride + kvh*kv_head_stride + slot*head_size
 *      (strides as built by tests/test_attention.c:141-143).  The paged loop
 *      structure (gather of each token through the table) follows
 *      examples/run_gpt2.c:60-79.  Elements are widened to fp32 first
 *      (fp16 / bf16 / fp32 storage, dtype code below).
 *      Contract details the reference leaves undefined and this build fixes:
 *        seq_len <= 0 -> the output row is zeros (page_attention.cu:157 writes
 *        0 for an empty sum); a negative block-table entry is never
 *        dereferenced and its tokens contribute nothing; seq_len is clamped to
 *        max_num_blocks_per_seq*block_size.
 *
 *  oracle_paged_attention_f64
 *      Same as above in double precision (the textbook formula), used to
 *      attribute rounding error.
 *
 *  oracle_paged_attention_f32_mt
 *      oracle_paged_attention_f32 with the (seq, head) loop split across
 *      OpenMP threads: identical arithmetic per (seq, head), so its output is
 *      bit-identical to the single-threaded routine.  This is the multi-core
 *      CPU baseline.
 *
 *  oracle_gpt2_paged_attention
 *      The other reference CPU attention, examples/run_gpt2.c:46-83: MHA only,
 *      one sequence, per-token page table page_table[t] (:61), slot
 *      t % page_size (:62), KV layout [page][slot][head][d] (:51, :63-64),
 *      scale 1/sqrtf(d) computed inside (:50), weights expf(dot*scale)
 *      WITHOUT max subtraction (:68), sum in t order (:69), then
 *      out += (w/sum)*v (:77-78).  Restated so that it can be checked
 *      bit-for-bit against the reference's own compiled function
 *      (oracle/_ref), which pins the fp32 arithmetic order used above.
 *
 *  oracle_paged_kv_append
 *      The reference's KV-cache write of one decode step,
 *      examples/text_gen.c:1274-1278: the new token's K row and V row
 *      (kv_dim = num_kv_heads * head_dim elements, head-major) are copied
 *      into the cache at position cur_len.  Restated over the operator-API
 *      pages: head h of token i goes to block slot/block_size, offset
 *      slot%block_size, element offset blk*kv_block_stride +
 *      h*kv_head_stride + off*head_size, bytes copied unchanged.  The slot is
 *      slots[i] when slots is given (prefill), else
 *      block_tables[i][positions[i]/block_size]*block_size +
 *      positions[i]%block_size (decode, token i = sequence i); a negative
 *      slot / position / page id, or a position at or past
 *      max_blocks*block_size, skips the token.
 *
 * Pinning (tests/test_oracle_*.py): the gpt2 restatement is bit-exact against
 * the compiled reference; the paged f32 routine agrees with it on MHA inputs
 * converted between the two layouts, with the f64 closed form, with
 * brute-force softmax on tiny cases, and with the invariants (L=1 returns V,
 * constant K returns mean V, page-permutation invariance, h/G head mapping,
 * garbage isolation) and the committed golden fixtures under tests/golden/.
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* dtype codes, identical to the NXT_KV_* codes of the plugin header */
enum { ORC_FP16 = 1, ORC_BF16 = 2, ORC_FP32 = 3 };

/* IEEE binary16 -> binary32, exact (normals, subnormals, inf, nan). */
static float orc_half_to_float(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1Fu;
    uint32_t man = h & 0x3FFu;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else { /* subnormal: value = man * 2^-24 */
            int e = -1;
            do { man <<= 1; e++; } while ((man & 0x400u) == 0);
            man &= 0x3FFu;
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
        }
    } else if (exp == 0x1F) {
        bits = sign | 0x7F800000u | (man << 13);
    } else {
        bits = sign | ((exp + (127 - 15)) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

static float orc_bf16_to_float(uint16_t b) {
    uint32_t bits = (uint32_t)b << 16;
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

static inline float orc_elem(const void *base, size_t idx, int dtype) {
    switch (dtype) {
    case ORC_FP16: return orc_half_to_float(((const uint16_t *)base)[idx]);
    case ORC_BF16: return orc_bf16_to_float(((const uint16_t *)base)[idx]);
    default:       return ((const float *)base)[idx];
    }
}

/* Exposed so the tests can check the widening against numpy/torch. */
float oracle_half_to_float(uint16_t h) { return orc_half_to_float(h); }
float oracle_bf16_to_float(uint16_t b) { return orc_bf16_to_float(b); }

typedef struct {
    const void *query, *key_cache, *value_cache;
    const int *block_tables, *seq_lens;
    int num_seqs, num_heads, head_size, num_kv_heads;
    float scale;
    int max_num_blocks_per_seq, block_size, dtype;
    long long kv_block_stride, kv_head_stride;
} orc_args;

/* Resolve token t of sequence s to the element offset of its K/V row for kv
 * head kvh, or -1 when its block-table entry is negative. */
static inline long long orc_row(const orc_args *a, int s, int kvh, int t) {
    int blk = a->block_tables[(size_t)s * a->max_num_blocks_per_seq + t / a->block_size];
    if (blk < 0) return -1;
    return (long long)blk * a->kv_block_stride + (long long)kvh * a->kv_head_stride +
           (long long)(t % a->block_size) * a->head_size;
}

static int orc_len(const orc_args *a, int s) {
    int L = a->seq_lens[s];
    long long cap = (long long)a->max_num_blocks_per_seq * a->block_size;
    if (L < 0) L = 0;
    if (L > cap) L = (int)cap;
    return L;
}

/* One (seq, head) of the fp32 restatement of text_gen.c:1284-1310. */
static void orc_head_f32(const orc_args *a, int s, int h, float *out, float *scores,
                         float *qf) {
    const int D = a->head_size;
    const int G = a->num_heads / a->num_kv_heads;
    const int kh = h / G; /* text_gen.c:1285 */
    float *oh = out + ((size_t)s * a->num_heads + h) * D;
    const int L = orc_len(a, s);
    for (int d = 0; d < D; d++) qf[d] = orc_elem(a->query, ((size_t)s * a->num_heads + h) * D + d, a->dtype);
    memset(oh, 0, (size_t)D * sizeof(float));
    if (L == 0) return;

    float max_val = -1e9f; /* text_gen.c:1290 */
    for (int t = 0; t < L; t++) {
        long long row = orc_row(a, s, kh, t);
        if (row < 0) { scores[t] = -INFINITY; continue; }
        float dot = 0.0f;
        for (int d = 0; d < D; d++) dot += qf[d] * orc_elem(a->key_cache, (size_t)row + d, a->dtype);
        scores[t] = dot * a->scale;
        if (scores[t] > max_val) max_val = scores[t];
    }
    float sum_exp = 0.0f;
    for (int t = 0; t < L; t++) {
        scores[t] = expf(scores[t] - max_val);
        sum_exp += scores[t];
    }
    for (int t = 0; t < L; t++) {
        long long row = orc_row(a, s, kh, t);
        if (row < 0) continue;
        float w = scores[t] / sum_exp;
        for (int d = 0; d < D; d++) oh[d] += w * orc_elem(a->value_cache, (size_t)row + d, a->dtype);
    }
}

static void orc_head_f64(const orc_args *a, int s, int h, double *out, double *scores,
                         double *qf) {
    const int D = a->head_size;
    const int G = a->num_heads / a->num_kv_heads;
    const int kh = h / G;
    double *oh = out + ((size_t)s * a->num_heads + h) * D;
    const int L = orc_len(a, s);
    for (int d = 0; d < D; d++) qf[d] = orc_elem(a->query, ((size_t)s * a->num_heads + h) * D + d, a->dtype);
    for (int d = 0; d < D; d++) oh[d] = 0.0;
    if (L == 0) return;
    double max_val = -INFINITY;
    for (int t = 0; t < L; t++) {
        long long row = orc_row(a, s, kh, t);
        if (row < 0) { scores[t] = -INFINITY; continue; }
        double dot = 0.0;
        for (int d = 0; d < D; d++) dot += qf[d] * (double)orc_elem(a->key_cache, (size_t)row + d, a->dtype);
        scores[t] = dot * (double)a->scale;
        if (scores[t] > max_val) max_val = scores[t];
    }
    double sum_exp = 0.0;
    for (int t = 0; t < L; t++) {
        scores[t] = exp(scores[t] - max_val);
        sum_exp += scores[t];
    }
    for (int t = 0; t < L; t++) {
        long long row = orc_row(a, s, kh, t);
        if (row < 0) continue;
        double w = scores[t] / sum_exp;
        for (int d = 0; d < D; d++) oh[d] += w * (double)orc_elem(a->value_cache, (size_t)row + d, a->dtype);
    }
}

static int orc_check(const orc_args *a) {
    if (a->num_seqs < 0 || a->num_heads <= 0 || a->num_kv_heads <= 0) return -1;
    if (a->num_heads % a->num_kv_heads) return -1;
    if (a->head_size <= 0 || a->block_size <= 0 || a->max_num_blocks_per_seq <= 0) return -1;
    if (a->dtype != ORC_FP16 && a->dtype != ORC_BF16 && a->dtype != ORC_FP32) return -1;
    return 0;
}

static int orc_max_len(const orc_args *a) {
    int m = 1;
    for (int s = 0; s < a->num_seqs; s++) {
        int L = orc_len(a, s);
        if (L > m) m = L;
    }
    return m;
}

#define ORC_ARGS_INIT                                                                   \
    orc_args a = {query, key_cache, value_cache, block_tables, seq_lens, num_seqs,     \
                  num_heads, head_size, num_kv_heads, scale, max_num_blocks_per_seq,   \
                  block_size, dtype, kv_block_stride, kv_head_stride}

/* Output is fp32 [num_seqs][num_heads][head_size]; returns 0, or -1 on bad args. */
int oracle_paged_attention_f32(float *out, const void *query, const void *key_cache,
                               const void *value_cache, const int *block_tables,
                               const int *seq_lens, int num_seqs, int num_heads,
                               int head_size, int num_kv_heads, float scale,
                               int max_num_blocks_per_seq, int block_size, int dtype,
                               long long kv_block_stride, long long kv_head_stride) {
    ORC_ARGS_INIT;
    if (orc_check(&a)) return -1;
    int maxL = orc_max_len(&a);
    float *scores = (float *)malloc((size_t)maxL * sizeof(float));
    float *qf = (float *)malloc((size_t)head_size * sizeof(float));
    if (!scores || !qf) { free(scores); free(qf); return -1; }
    for (int s = 0; s < num_seqs; s++)
        for (int h = 0; h < num_heads; h++) orc_head_f32(&a, s, h, out, scores, qf);
    free(scores);
    free(qf);
    return 0;
}

int oracle_paged_attention_f32_mt(float *out, const void *query, const void *key_cache,
                                  const void *value_cache, const int *block_tables,
                                  const int *seq_lens, int num_seqs, int num_heads,
                                  int head_size, int num_kv_heads, float scale,
                                  int max_num_blocks_per_seq, int block_size, int dtype,
                                  long long kv_block_stride, long long kv_head_stride,
                                  int num_threads) {
    ORC_ARGS_INIT;
    if (orc_check(&a)) return -1;
    int maxL = orc_max_len(&a);
    int err = 0;
    long long n = (long long)num_seqs * num_heads;
#ifdef _OPENMP
    if (num_threads <= 0) num_threads = omp_get_max_threads();
#pragma omp parallel num_threads(num_threads) reduction(| : err)
#endif
    {
        float *scores = (float *)malloc((size_t)maxL * sizeof(float));
        float *qf = (float *)malloc((size_t)head_size * sizeof(float));
        if (!scores || !qf) {
            err = 1;
        } else {
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 1)
#endif
            for (long long i = 0; i < n; i++)
                orc_head_f32(&a, (int)(i / num_heads), (int)(i % num_heads), out, scores, qf);
        }
        free(scores);
        free(qf);
    }
    (void)num_threads;
    return err ? -1 : 0;
}

int oracle_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

int oracle_paged_attention_f64(double *out, const void *query, const void *key_cache,
                               const void *value_cache, const int *block_tables,
                               const int *seq_lens, int num_seqs, int num_heads,
                               int head_size, int num_kv_heads, float scale,
                               int max_num_blocks_per_seq, int block_size, int dtype,
                               long long kv_block_stride, long long kv_head_stride) {
    ORC_ARGS_INIT;
    if (orc_check(&a)) return -1;
    int maxL = orc_max_len(&a);
    double *scores = (double *)malloc((size_t)maxL * sizeof(double));
    double *qf = (double *)malloc((size_t)head_size * sizeof(double));
    if (!scores || !qf) { free(scores); free(qf); return -1; }
    for (int s = 0; s < num_seqs; s++)
        for (int h = 0; h < num_heads; h++) orc_head_f64(&a, s, h, out, scores, qf);
    free(scores);
    free(qf);
    return 0;
}

/* Restatement of examples/run_gpt2.c:46-83 (see header comment). */
void oracle_gpt2_paged_attention(const float *query, const float *key_cache,
                                 const float *value_cache, const int *page_table,
                                 int seq_len, int num_heads, int head_dim, int page_size,
                                 float *output) {
    const float scale = 1.0f / sqrtf((float)head_dim);
    const size_t page_entries = (size_t)page_size * num_heads * head_dim;
    float *w = (float *)malloc((size_t)(seq_len > 0 ? seq_len : 1) * sizeof(float));
    for (int h = 0; h < num_heads; h++) {
        float *oh = output + (size_t)h * head_dim;
        const float *qh = query + (size_t)h * head_dim;
        float total = 0.0f;
        for (int d = 0; d < head_dim; d++) oh[d] = 0.0f;
        for (int t = 0; t < seq_len; t++) {
            const float *kt = key_cache + (size_t)page_table[t] * page_entries +
                              (size_t)(t % page_size) * num_heads * head_dim + (size_t)h * head_dim;
            float acc = 0.0f;
            for (int d = 0; d < head_dim; d++) acc += qh[d] * kt[d];
            w[t] = expf(acc * scale);
            total += w[t];
        }
        for (int t = 0; t < seq_len; t++) {
            const float *vt = value_cache + (size_t)page_table[t] * page_entries +
                              (size_t)(t % page_size) * num_heads * head_dim + (size_t)h * head_dim;
            const float f = w[t] / total;
            for (int d = 0; d < head_dim; d++) oh[d] += f * vt[d];
        }
    }
    free(w);
}

int oracle_paged_kv_append(void *key_cache, void *value_cache, const void *key, const void *value,
                           const int *slots, const int *block_tables, const int *positions,
                           int num_tokens, int num_kv_heads, int head_size, int max_blocks,
                           int block_size, long long kv_block_stride, long long kv_head_stride,
                           int elem_bytes) {
    if (num_tokens < 0 || num_kv_heads <= 0 || head_size <= 0 || block_size <= 0 ||
        (elem_bytes != 2 && elem_bytes != 4))
        return -1;
    const size_t row = (size_t)head_size * (size_t)elem_bytes;
    for (int i = 0; i < num_tokens; i++) {
        long long slot;
        if (slots) {
            slot = slots[i];
        } else {
            const int pos = positions[i];
            if (pos < 0 || (long long)pos >= (long long)max_blocks * block_size) continue;
            const int blk = block_tables[(size_t)i * (size_t)max_blocks + (size_t)(pos / block_size)];
            if (blk < 0) continue;
            slot = (long long)blk * block_size + pos % block_size;
        }
        if (slot < 0) continue;
        const long long blk = slot / block_size, off = slot % block_size;
        for (int h = 0; h < num_kv_heads; h++) {
            const size_t dst = (size_t)(blk * kv_block_stride + h * kv_head_stride +
                                        off * (long long)head_size) * (size_t)elem_bytes;
            const size_t src = ((size_t)i * (size_t)num_kv_heads + (size_t)h) * row;
            memcpy((char *)key_cache + dst, (const char *)key + src, row);
            memcpy((char *)value_cache + dst, (const char *)value + src, row);
        }
    }
    return 0;
}
