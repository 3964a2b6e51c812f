/*
 * oracle.c -- CPU restatement of StrataKV's paged-KV hot path (test
 * infrastructure only; see oracle.h).  Citations are to the StrataKV sources.
 */
#include "oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------- */
/* bf16                                                                      */
/* ------------------------------------------------------------------------- */

/* src/cpu/tensor.cpp:200-206: the two stored bytes become the high half. */
float oracle_bf16_to_f32(uint16_t h) {
    uint32_t bits = (uint32_t)h << 16;
    float f;
    memcpy(&f, &bits, sizeof f);
    return f;
}

/* src/cpu/tensor.cpp:218-225: upper 16 bits, incremented when the lower 16
 * bits exceed one half, or equal one half with an odd upper part.  The
 * increment may carry out of 16 bits; the reference stores only the low
 * byte pair, so the carry is dropped. */
uint16_t oracle_f32_to_bf16_rne(float x) {
    uint32_t bits;
    memcpy(&bits, &x, sizeof bits);
    uint32_t upper = bits >> 16u;
    const uint32_t lower = bits & 0xffffu;
    if (lower > 0x8000u || (lower == 0x8000u && (upper & 1u) != 0u)) ++upper;
    return (uint16_t)(upper & 0xffffu);
}

/* src/cuda/gemm_cuda.cu:74-83 (and safetensors.cpp:660-666): drop the low half. */
uint16_t oracle_f32_to_bf16_trunc(float x) {
    uint32_t bits;
    memcpy(&bits, &x, sizeof bits);
    return (uint16_t)(bits >> 16u);
}

void oracle_bf16_to_f32_n(const uint16_t* in, float* out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = oracle_bf16_to_f32(in[i]);
}

void oracle_f32_to_bf16_rne_n(const float* in, uint16_t* out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = oracle_f32_to_bf16_rne(in[i]);
}

/* ------------------------------------------------------------------------- */
/* BlockPool / PageTable                                                     */
/* ------------------------------------------------------------------------- */

typedef struct {
    int* stack; /* free list; the top (stack[n-1]) is handed out next */
    int n;
} pool_t;

typedef struct {
    int live;
    int length;
    int* blocks;
    int n_blocks;
    int cap;
} seq_t;

/* src/memory/block_pool.cpp:72-76: push total-1 ... 0 so block 0 is on top. */
static void pool_init(pool_t* p, int total) {
    p->stack = (int*)malloc(sizeof(int) * (size_t)(total > 0 ? total : 1));
    p->n = 0;
    for (int id = total - 1; id >= 0; --id) p->stack[p->n++] = id;
}

/* src/memory/block_pool.cpp:193-200: pop, or fail with "OOM". */
static int pool_alloc(pool_t* p, int* id) {
    if (p->n == 0) return ORACLE_ST_OOM;
    *id = p->stack[--p->n];
    return ORACLE_ST_OK;
}

/* src/memory/block_pool.cpp:205-207: push, no checks. */
static void pool_free(pool_t* p, int id, int total) {
    (void)total;
    p->stack[p->n++] = id;
}

static void seq_push(seq_t* s, int id) {
    if (s->n_blocks == s->cap) {
        s->cap = s->cap ? 2 * s->cap : 8;
        s->blocks = (int*)realloc(s->blocks, sizeof(int) * (size_t)s->cap);
    }
    s->blocks[s->n_blocks++] = id;
}

int oracle_pool_trace(int total, int block_size, const int32_t* ops, int n_ops, int max_seqs,
                      int32_t* results, int32_t* lens, int32_t* blocks, int max_blocks_out,
                      int32_t* drain) {
    pool_t pool;
    pool_init(&pool, total);
    /* free_block may push more ids than `total` on a double free (undefined in
     * the reference); size the stack for the worst case of this trace. */
    pool.stack = (int*)realloc(pool.stack, sizeof(int) * (size_t)(total + n_ops + 1));
    seq_t* seqs = (seq_t*)calloc((size_t)max_seqs, sizeof(seq_t));

    for (int i = 0; i < n_ops; ++i) {
        const int op = ops[2 * i], sid = ops[2 * i + 1];
        int32_t st = ORACLE_ST_OK, blk = -1;
        seq_t* s = (sid >= 0 && sid < max_seqs) ? &seqs[sid] : NULL;
        if (op == ORACLE_OP_ALLOC_SEQ) {
            /* src/memory/page_table.cpp:107-117: duplicate check first, then
             * the first block; nothing is registered when allocation fails. */
            if (s != NULL && s->live) {
                st = ORACLE_ST_EXISTS;
            } else {
                int id;
                st = pool_alloc(&pool, &id);
                if (st == ORACLE_ST_OK && s != NULL) {
                    s->live = 1;
                    s->length = 0;
                    s->n_blocks = 0;
                    seq_push(s, id);
                    blk = id;
                }
            }
        } else if (op == ORACLE_OP_APPEND) {
            /* src/memory/page_table.cpp:126-147: allocate only when every
             * assigned page is full; on OOM the length is unchanged. */
            if (s == NULL || !s->live) {
                st = ORACLE_ST_UNKNOWN;
            } else {
                const long long capacity = (long long)s->n_blocks * block_size;
                if ((long long)s->length >= capacity) {
                    int id;
                    st = pool_alloc(&pool, &id);
                    if (st == ORACLE_ST_OK) {
                        seq_push(s, id);
                        blk = id;
                    }
                }
                if (st == ORACLE_ST_OK) ++s->length;
            }
        } else if (op == ORACLE_OP_FREE_SEQ) {
            /* src/memory/page_table.cpp:152-160: return blocks in table order. */
            if (s == NULL || !s->live) {
                st = ORACLE_ST_UNKNOWN;
            } else {
                for (int k = 0; k < s->n_blocks; ++k) pool_free(&pool, s->blocks[k], total);
                s->live = 0;
                s->n_blocks = 0;
                s->length = 0;
            }
        }
        results[2 * i] = st;
        results[2 * i + 1] = blk;
    }

    for (int sid = 0; sid < max_seqs; ++sid) {
        seq_t* s = &seqs[sid];
        lens[sid] = s->live ? s->length : -1;
        for (int k = 0; k < max_blocks_out; ++k)
            blocks[(size_t)sid * max_blocks_out + k] = (s->live && k < s->n_blocks) ? s->blocks[k] : -1;
        free(s->blocks);
    }
    int drained = 0;
    int id;
    while (pool_alloc(&pool, &id) == ORACLE_ST_OK) drain[drained++] = id;
    free(seqs);
    free(pool.stack);
    return drained;
}

/* ------------------------------------------------------------------------- */
/* KV append                                                                 */
/* ------------------------------------------------------------------------- */

/* src/models/transformer_block.cpp:484-509: page_index = pos / block_size,
 * slot = pos % block_size, offset = (block * block_size + slot) * Hkv * hd,
 * then one row of Hkv*hd elements for K and one for V. */
void oracle_kv_append(const void* k_new, const void* v_new, int src_fp32, uint16_t* k_pool,
                      uint16_t* v_pool, int64_t total_blocks, const int32_t* tables,
                      int max_blocks, const int32_t* positions, const int32_t* offsets,
                      int num_seqs, int tokens_per_seq, int num_kv_heads, int head_dim,
                      int block_size) {
    const int64_t row = (int64_t)num_kv_heads * head_dim;
    for (int b = 0; b < num_seqs; ++b) {
        int n = tokens_per_seq;
        int64_t first = (int64_t)b * tokens_per_seq;
        if (offsets != NULL) {
            first = offsets[b];
            const int nb = offsets[b + 1] - offsets[b];
            if (nb < n) n = nb;
        }
        for (int j = 0; j < n; ++j) {
            const int pos = positions[b] + j;
            if (pos < 0) continue;
            const int page = pos / block_size;
            if (page >= max_blocks) continue;
            const int64_t pb = tables[(int64_t)b * max_blocks + page];
            if (pb < 0 || pb >= total_blocks) continue;
            const int64_t dst = (pb * block_size + pos % block_size) * row;
            const int64_t src = (first + j) * row;
            for (int64_t e = 0; e < row; ++e) {
                if (src_fp32) {
                    k_pool[dst + e] = oracle_f32_to_bf16_rne(((const float*)k_new)[src + e]);
                    v_pool[dst + e] = oracle_f32_to_bf16_rne(((const float*)v_new)[src + e]);
                } else {
                    k_pool[dst + e] = ((const uint16_t*)k_new)[src + e];
                    v_pool[dst + e] = ((const uint16_t*)v_new)[src + e];
                }
            }
        }
    }
}

/* ------------------------------------------------------------------------- */
/* Paged decode attention                                                    */
/* ------------------------------------------------------------------------- */

typedef struct {
    const float* q;
    const void* k;
    const void* v;
    int fp32_pool; /* 1: k/v are float pools (the reference's cache type) */
    int64_t total_blocks;
    const int32_t* tables;
    int max_blocks;
    const int32_t* lens;
    int B, Hq, Hkv, hd, bs;
    float scale;
    float* out;
} attn_args;

static inline float load_elem(const void* pool, int64_t i, int fp32_pool) {
    return fp32_pool ? ((const float*)pool)[i] : oracle_bf16_to_f32(((const uint16_t*)pool)[i]);
}

/* One (sequence, query head): src/layers/attention.cpp:268-337 restated over
 * a BlockPool-layout cache as src/models/transformer_block.cpp:148-181 reads it. */
static int attend_one_f32(const attn_args* a, int b, int head, float* scores) {
    const int L = a->lens[b];
    float* out = a->out + ((int64_t)b * a->Hq + head) * a->hd;
    if (L <= 0) {
        for (int d = 0; d < a->hd; ++d) out[d] = 0.0f;
        return 0;
    }
    const int groups = a->Hq / a->Hkv;
    const int kv_head = head / groups;                       /* attention.cpp:270 */
    const int64_t token_stride = (int64_t)a->Hkv * a->hd;
    const float* query = a->q + ((int64_t)b * a->Hq + head) * a->hd;
    const int32_t* table = a->tables + (int64_t)b * a->max_blocks;
    float max_score = -INFINITY;
    for (int p = 0; p < L; ++p) {                            /* attention.cpp:275-306 */
        const int page = p / a->bs;
        if (page >= a->max_blocks) return -3;
        const int64_t blk = table[page];
        if (blk < 0 || blk >= a->total_blocks) return -2;
        const int64_t key = (blk * a->bs + p % a->bs) * token_stride + (int64_t)kv_head * a->hd;
        float dot = 0.0f;
        for (int d = 0; d < a->hd; ++d) dot += query[d] * load_elem(a->k, key + d, a->fp32_pool);
        scores[p] = dot * a->scale;
        if (scores[p] > max_score) max_score = scores[p];   /* std::max(max, s) */
    }
    float denominator = 0.0f;
    for (int p = 0; p < L; ++p) {                            /* attention.cpp:308-316 */
        scores[p] = expf(scores[p] - max_score);
        denominator += scores[p];
    }
    if (!(denominator > 0.0f) || !isfinite(denominator)) return -1;
    for (int d = 0; d < a->hd; ++d) {                        /* attention.cpp:318-336 */
        float accumulated = 0.0f;
        for (int p = 0; p < L; ++p) {
            const int64_t blk = table[p / a->bs];
            const int64_t value = (blk * a->bs + p % a->bs) * token_stride + (int64_t)kv_head * a->hd;
            accumulated += (scores[p] / denominator) * load_elem(a->v, value + d, a->fp32_pool);
        }
        out[d] = accumulated;
    }
    return 0;
}

static int max_len(const int32_t* lens, int B) {
    int m = 1;
    for (int b = 0; b < B; ++b) if (lens[b] > m) m = lens[b];
    return m;
}

int oracle_paged_decode_f32(const float* q, const uint16_t* k_pool, const uint16_t* v_pool,
                            int64_t total_blocks, const int32_t* tables, int max_blocks,
                            const int32_t* lens, int B, int Hq, int Hkv, int hd, int bs,
                            float scale, float* out) {
    return oracle_paged_decode_f32_mt(q, k_pool, v_pool, total_blocks, tables, max_blocks, lens, B,
                                      Hq, Hkv, hd, bs, scale, out, 1);
}

typedef struct {
    const attn_args* a;
    int first, last; /* range of (b * Hq + head) pairs */
    int status;
} worker_t;

static void* attend_range(void* arg) {
    worker_t* w = (worker_t*)arg;
    float* scores = (float*)malloc(sizeof(float) * (size_t)max_len(w->a->lens, w->a->B));
    w->status = 0;
    for (int i = w->first; i < w->last && w->status == 0; ++i)
        w->status = attend_one_f32(w->a, i / w->a->Hq, i % w->a->Hq, scores);
    free(scores);
    return NULL;
}

static int run_attention(const float* q, const void* k_pool, const void* v_pool, int fp32_pool,
                         int64_t total_blocks, const int32_t* tables, int max_blocks,
                         const int32_t* lens, int B, int Hq, int Hkv, int hd, int bs, float scale,
                         float* out, int threads) {
    if (B <= 0 || Hq <= 0 || Hkv <= 0 || hd <= 0 || bs <= 0 || Hq % Hkv != 0) return -4;
    attn_args a = {q, k_pool, v_pool, fp32_pool, total_blocks, tables, max_blocks, lens,
                   B, Hq, Hkv, hd, bs, scale, out};
    const int pairs = B * Hq;
    if (threads < 1) threads = 1;
    if (threads > pairs) threads = pairs;
    worker_t* ws = (worker_t*)calloc((size_t)threads, sizeof(worker_t));
    pthread_t* tids = (pthread_t*)calloc((size_t)threads, sizeof(pthread_t));
    for (int t = 0; t < threads; ++t) {
        ws[t].a = &a;
        ws[t].first = (int)((long long)pairs * t / threads);
        ws[t].last = (int)((long long)pairs * (t + 1) / threads);
    }
    if (threads == 1) {
        attend_range(&ws[0]);
    } else {
        for (int t = 0; t < threads; ++t) pthread_create(&tids[t], NULL, attend_range, &ws[t]);
        for (int t = 0; t < threads; ++t) pthread_join(tids[t], NULL);
    }
    int status = 0;
    for (int t = 0; t < threads; ++t)
        if (ws[t].status != 0 && status == 0) status = ws[t].status;
    free(ws);
    free(tids);
    return status;
}

int oracle_paged_decode_f32_mt(const float* q, const uint16_t* k_pool, const uint16_t* v_pool,
                               int64_t total_blocks, const int32_t* tables, int max_blocks,
                               const int32_t* lens, int B, int Hq, int Hkv, int hd, int bs,
                               float scale, float* out, int threads) {
    return run_attention(q, k_pool, v_pool, 0, total_blocks, tables, max_blocks, lens, B, Hq, Hkv,
                         hd, bs, scale, out, threads);
}

int oracle_paged_decode_f32_fp32pool(const float* q, const float* k_pool, const float* v_pool,
                                     int64_t total_blocks, const int32_t* tables, int max_blocks,
                                     const int32_t* lens, int B, int Hq, int Hkv, int hd, int bs,
                                     float scale, float* out) {
    return run_attention(q, k_pool, v_pool, 1, total_blocks, tables, max_blocks, lens, B, Hq, Hkv,
                         hd, bs, scale, out, 1);
}

/* The same loops in double precision. */
int oracle_paged_decode_f64(const float* q, const uint16_t* k_pool, const uint16_t* v_pool,
                            int64_t total_blocks, const int32_t* tables, int max_blocks,
                            const int32_t* lens, int B, int Hq, int Hkv, int hd, int bs,
                            double scale, double* out) {
    if (B <= 0 || Hq <= 0 || Hkv <= 0 || hd <= 0 || bs <= 0 || Hq % Hkv != 0) return -4;
    double* scores = (double*)malloc(sizeof(double) * (size_t)max_len(lens, B));
    const int groups = Hq / Hkv;
    const int64_t token_stride = (int64_t)Hkv * hd;
    int status = 0;
    for (int b = 0; b < B && status == 0; ++b) {
        const int L = lens[b];
        const int32_t* table = tables + (int64_t)b * max_blocks;
        for (int head = 0; head < Hq && status == 0; ++head) {
            double* o = out + ((int64_t)b * Hq + head) * hd;
            if (L <= 0) {
                for (int d = 0; d < hd; ++d) o[d] = 0.0;
                continue;
            }
            const int kv_head = head / groups;
            const float* query = q + ((int64_t)b * Hq + head) * hd;
            double mx = -INFINITY;
            for (int p = 0; p < L; ++p) {
                const int page = p / bs;
                if (page >= max_blocks) { status = -3; break; }
                const int64_t blk = table[page];
                if (blk < 0 || blk >= total_blocks) { status = -2; break; }
                const uint16_t* key = k_pool + (blk * bs + p % bs) * token_stride + (int64_t)kv_head * hd;
                double dot = 0.0;
                for (int d = 0; d < hd; ++d) dot += (double)query[d] * (double)oracle_bf16_to_f32(key[d]);
                scores[p] = dot * scale;
                if (scores[p] > mx) mx = scores[p];
            }
            if (status != 0) break;
            double den = 0.0;
            for (int p = 0; p < L; ++p) {
                scores[p] = exp(scores[p] - mx);
                den += scores[p];
            }
            if (!(den > 0.0) || !isfinite(den)) { status = -1; break; }
            for (int d = 0; d < hd; ++d) o[d] = 0.0;
            for (int p = 0; p < L; ++p) {
                const int64_t blk = table[p / bs];
                const uint16_t* value = v_pool + (blk * bs + p % bs) * token_stride + (int64_t)kv_head * hd;
                const double w = scores[p] / den;
                for (int d = 0; d < hd; ++d) o[d] += w * (double)oracle_bf16_to_f32(value[d]);
            }
        }
    }
    free(scores);
    return status;
}
