/*
 * oracle.c - CPU restatement of the QwenVL-Paged hot path. TEST INFRASTRUCTURE:
 * used only by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg,
 * always as the checker. See oracle.h for what pins each function.
 *
 * Built with -O2 -ffp-contract=off so float expressions round exactly as the
 * reference's g++ -std=c++17 build does (no fused multiply-adds).
 */
#include "oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#define ORC_UNMAPPED 0xFFFFFFFFu

/* ---------------------------------------------------------------- */
/* Element conversions                                              */
/* ---------------------------------------------------------------- */

static uint32_t f32_bits(float x) {
    uint32_t u;
    memcpy(&u, &x, sizeof u);
    return u;
}

static float bits_f32(uint32_t u) {
    float x;
    memcpy(&x, &u, sizeof x);
    return x;
}

uint16_t orc_bf16_from_f32(float x) {
    const uint32_t u = f32_bits(x);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u);
    return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

float orc_f32_from_bf16(uint16_t h) { return bits_f32((uint32_t)h << 16); }

uint16_t orc_f16_from_f32(float x) {
    const uint32_t u = f32_bits(x);
    const uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    const uint32_t a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((a >> 13) & 0x3ffu));
    if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 rounds to infinity */
    if (a < 0x38800000u) {
        /* Subnormal half: the value times 2^24 is the mantissa, rounded to
         * nearest even by nearbyintf in the default rounding mode. */
        const float scaled = fabsf(x) * 16777216.0f;
        return (uint16_t)(sign | (uint16_t)nearbyintf(scaled));
    }
    const uint32_t rebased = a - 0x38000000u;
    return (uint16_t)(sign | ((rebased + 0xfffu + ((a >> 13) & 1u)) >> 13));
}

float orc_f32_from_f16(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu;
    const uint32_t m = h & 0x3ffu;
    if (e == 0) {
        const float f = ldexpf((float)m, -24);
        return sign ? -f : f;
    }
    if (e == 31) return bits_f32(sign | 0x7f800000u | (m << 13));
    return bits_f32(sign | ((e + 112u) << 23) | (m << 13));
}

void orc_round_to_bf16(const float* src, uint16_t* dst, size_t n) {
    for (size_t i = 0; i < n; ++i) dst[i] = orc_bf16_from_f32(src[i]);
}

void orc_round_to_f16(const float* src, uint16_t* dst, size_t n) {
    for (size_t i = 0; i < n; ++i) dst[i] = orc_f16_from_f32(src[i]);
}

static size_t dtype_bytes(int dtype) {
    switch (dtype) {
        case ORC_F32: return 4;
        case ORC_BF16: return 2;
        case ORC_F16: return 2;
        default: return 0;
    }
}

static float load_elem(const uint8_t* p, int dtype) {
    if (dtype == ORC_F32) {
        float f;
        memcpy(&f, p, 4);
        return f;
    }
    uint16_t h;
    memcpy(&h, p, 2);
    return dtype == ORC_BF16 ? orc_f32_from_bf16(h) : orc_f32_from_f16(h);
}

static void store_elem(uint8_t* p, int dtype, float v) {
    if (dtype == ORC_F32) {
        memcpy(p, &v, 4);
        return;
    }
    const uint16_t h = dtype == ORC_BF16 ? orc_bf16_from_f32(v) : orc_f16_from_f32(v);
    memcpy(p, &h, 2);
}

/* ---------------------------------------------------------------- */
/* Block shape and layout (src/Block.cpp, src/CacheLayout.cpp)      */
/* ---------------------------------------------------------------- */

uint64_t orc_block_byte_size(uint32_t tpb, uint32_t num_layers, uint32_t num_kv_heads, uint32_t head_dim,
                             uint32_t bpe) {
    /* K and V of every layer, head and token slot: the factor of two. */
    return (uint64_t)tpb * num_layers * num_kv_heads * head_dim * bpe * 2u;
}

uint64_t orc_block_stride(uint64_t byte_size, uint64_t alignment) {
    const uint64_t a = alignment == 0 ? 256u : alignment;
    uint64_t bytes = (byte_size + a - 1) / a * a;
    if (bytes == 0) bytes = a;
    return bytes;
}

void orc_layout_strides(uint32_t tpb, uint32_t num_layers, uint32_t num_kv_heads, uint32_t head_dim,
                        uint64_t out[5]) {
    const uint64_t head = head_dim;
    const uint64_t token = (uint64_t)num_kv_heads * head;
    const uint64_t stream = (uint64_t)tpb * token;
    const uint64_t layer = 2u * stream;
    out[0] = head;
    out[1] = token;
    out[2] = stream;
    out[3] = layer;
    out[4] = (uint64_t)num_layers * layer;
}

int64_t orc_element_offset(uint32_t tpb, uint32_t num_layers, uint32_t num_kv_heads, uint32_t head_dim,
                           uint32_t layer, uint32_t stream, uint32_t token_in_block, uint32_t kv_head) {
    if (layer >= num_layers || token_in_block >= tpb || kv_head >= num_kv_heads) return -1;
    uint64_t s[5];
    orc_layout_strides(tpb, num_layers, num_kv_heads, head_dim, s);
    const uint64_t stream_index = stream == 0 ? 0u : 1u;
    return (int64_t)(layer * s[3] + stream_index * s[2] + token_in_block * s[1] + kv_head * s[0]);
}

/* ---------------------------------------------------------------- */
/* paged_attention_decode<T> (include/qwenvl_paged/PagedAttention.h:53-127) */
/* ---------------------------------------------------------------- */

int orc_paged_attention_decode(const uint8_t* pool, uint64_t block_stride, uint32_t num_pool_blocks,
                               const uint32_t* table, uint32_t table_len, int dtype, const void* query,
                               uint32_t layer, uint32_t num_layers, uint32_t num_query_heads,
                               uint32_t num_kv_heads, uint32_t head_dim, uint32_t tpb,
                               uint32_t context_len, float scale, void* out, float* out_f32) {
    /* View validity and argument checks (PagedAttention.h:59-68,
     * KVCacheManager.cpp:7-9). */
    const size_t bpe = dtype_bytes(dtype);
    uint64_t strides[5];
    orc_layout_strides(tpb, num_layers, num_kv_heads, head_dim, strides);
    if (pool == NULL || table == NULL || strides[4] == 0 || query == NULL || out == NULL || bpe == 0) {
        return 0;
    }
    if (context_len == 0 || layer >= num_layers || num_query_heads == 0 ||
        num_query_heads % num_kv_heads != 0) {
        return 0;
    }
    const uint32_t group = num_query_heads / num_kv_heads;

    /* Resolve every block of the context before computing anything
     * (PagedAttention.h:73-89): CacheView::block_bytes faults on an unmapped or
     * swapped entry (KVCacheManager.cpp:11-25) and on an id outside the pool
     * (MemoryAllocator.cpp:87-92). */
    const uint32_t needed = (context_len + tpb - 1) / tpb;
    if (needed > table_len) return 0;
    for (uint32_t j = 0; j < needed; ++j) {
        if (table[j] == ORC_UNMAPPED || table[j] >= num_pool_blocks) return 0;
    }

    const uint64_t layer_off = (uint64_t)layer * strides[3];
    float* scores = (float*)malloc(sizeof(float) * context_len);
    float* accumulator = (float*)malloc(sizeof(float) * head_dim);
    const uint8_t** keys = (const uint8_t**)malloc(sizeof(*keys) * context_len);
    const uint8_t** values = (const uint8_t**)malloc(sizeof(*values) * context_len);
    if (scores == NULL || accumulator == NULL || keys == NULL || values == NULL) {
        free(scores);
        free(accumulator);
        free(keys);
        free(values);
        return 0;
    }

    const uint8_t* q_bytes = (const uint8_t*)query;
    for (uint32_t q_head = 0; q_head < num_query_heads; ++q_head) {
        const uint32_t kv_head = q_head / group;
        for (uint32_t token = 0; token < context_len; ++token) {
            const uint8_t* frame = pool + (uint64_t)table[token / tpb] * block_stride;
            const uint64_t k_elem = layer_off + (uint64_t)(token % tpb) * strides[1] + (uint64_t)kv_head * strides[0];
            keys[token] = frame + k_elem * bpe;
            values[token] = frame + (k_elem + strides[2]) * bpe;
        }
        const uint8_t* q = q_bytes + (uint64_t)q_head * head_dim * bpe;

        /* Pass 1: scores and their maximum (PagedAttention.h:98-107). */
        float max_score = -INFINITY;
        for (uint32_t token = 0; token < context_len; ++token) {
            float dot = 0.0f;
            for (uint32_t dim = 0; dim < head_dim; ++dim) {
                dot += load_elem(q + dim * bpe, dtype) * load_elem(keys[token] + dim * bpe, dtype);
            }
            scores[token] = dot * scale;
            max_score = scores[token] > max_score ? scores[token] : max_score;
        }

        /* Pass 2: weights, denominator and the value accumulator
         * (PagedAttention.h:109-118). */
        for (uint32_t dim = 0; dim < head_dim; ++dim) accumulator[dim] = 0.0f;
        float denominator = 0.0f;
        for (uint32_t token = 0; token < context_len; ++token) {
            const float weight = expf(scores[token] - max_score);
            denominator += weight;
            for (uint32_t dim = 0; dim < head_dim; ++dim) {
                accumulator[dim] += weight * load_elem(values[token] + dim * bpe, dtype);
            }
        }

        /* Normalise and cast (PagedAttention.h:120-123). */
        uint8_t* dst = (uint8_t*)out + (uint64_t)q_head * head_dim * bpe;
        for (uint32_t dim = 0; dim < head_dim; ++dim) {
            const float v = accumulator[dim] / denominator;
            store_elem(dst + dim * bpe, dtype, v);
            if (out_f32 != NULL) out_f32[(uint64_t)q_head * head_dim + dim] = v;
        }
    }

    free(scores);
    free(accumulator);
    free(keys);
    free(values);
    return 1;
}

/* ---------------------------------------------------------------- */
/* Batched wrapper                                                  */
/* ---------------------------------------------------------------- */

typedef struct {
    const uint8_t* pool;
    uint64_t block_stride;
    uint32_t num_pool_blocks;
    const uint32_t* ids;
    const uint32_t* cu_blocks;
    const uint32_t* context_lens;
    int dtype;
    const uint8_t* query;
    uint32_t layer, num_layers, hq, hkv, d, tpb;
    float scale;
    uint8_t* out;
    float* out_f32;
    uint32_t first, last;
    int refused;
} batch_job;

static void* run_batch_job(void* arg) {
    batch_job* job = (batch_job*)arg;
    const size_t bpe = dtype_bytes(job->dtype);
    const uint64_t per_seq = (uint64_t)job->hq * job->d;
    for (uint32_t b = job->first; b < job->last; ++b) {
        const uint32_t* table = job->ids + job->cu_blocks[b];
        const uint32_t table_len = job->cu_blocks[b + 1] - job->cu_blocks[b];
        const int ok = orc_paged_attention_decode(
            job->pool, job->block_stride, job->num_pool_blocks, table, table_len, job->dtype,
            job->query + b * per_seq * bpe, job->layer, job->num_layers, job->hq, job->hkv, job->d, job->tpb,
            job->context_lens[b], job->scale, job->out + b * per_seq * bpe,
            job->out_f32 ? job->out_f32 + b * per_seq : NULL);
        if (!ok) job->refused += 1;
    }
    return NULL;
}

int orc_paged_decode_batch(const uint8_t* pool, uint64_t block_stride, uint32_t num_pool_blocks,
                           uint32_t num_seqs, const uint32_t* ids, const uint32_t* cu_blocks,
                           const uint32_t* context_lens, int dtype, const void* query, uint32_t layer,
                           uint32_t num_layers, uint32_t num_query_heads, uint32_t num_kv_heads,
                           uint32_t head_dim, uint32_t tokens_per_block, float scale, void* out,
                           float* out_f32, int threads) {
    if (threads < 1) threads = 1;
    if ((uint32_t)threads > num_seqs) threads = num_seqs > 0 ? (int)num_seqs : 1;
    batch_job* jobs = (batch_job*)calloc((size_t)threads, sizeof(batch_job));
    pthread_t* tids = (pthread_t*)calloc((size_t)threads, sizeof(pthread_t));
    if (jobs == NULL || tids == NULL) {
        free(jobs);
        free(tids);
        return (int)num_seqs;
    }
    for (int t = 0; t < threads; ++t) {
        batch_job* j = &jobs[t];
        j->pool = pool;
        j->block_stride = block_stride;
        j->num_pool_blocks = num_pool_blocks;
        j->ids = ids;
        j->cu_blocks = cu_blocks;
        j->context_lens = context_lens;
        j->dtype = dtype;
        j->query = (const uint8_t*)query;
        j->layer = layer;
        j->num_layers = num_layers;
        j->hq = num_query_heads;
        j->hkv = num_kv_heads;
        j->d = head_dim;
        j->tpb = tokens_per_block;
        j->scale = scale;
        j->out = (uint8_t*)out;
        j->out_f32 = out_f32;
        j->first = (uint32_t)((uint64_t)num_seqs * t / threads);
        j->last = (uint32_t)((uint64_t)num_seqs * (t + 1) / threads);
    }
    int refused = 0;
    if (threads == 1) {
        run_batch_job(&jobs[0]);
    } else {
        for (int t = 0; t < threads; ++t) pthread_create(&tids[t], NULL, run_batch_job, &jobs[t]);
        for (int t = 0; t < threads; ++t) pthread_join(tids[t], NULL);
    }
    for (int t = 0; t < threads; ++t) refused += jobs[t].refused;
    free(jobs);
    free(tids);
    return refused;
}

/* ---------------------------------------------------------------- */
/* Pack (docs/architecture.md:117-120) and copy (MemoryAllocator.cpp:76-85) */
/* ---------------------------------------------------------------- */

int orc_pack(uint32_t num_seqs, const uint32_t* ids, const uint32_t* cu_blocks,
             const uint32_t* context_lens, uint32_t tpb, uint32_t num_pool_blocks, uint32_t split_tokens,
             uint32_t* max_nb_out, uint32_t* num_splits_out, int32_t* tables, int32_t* seq_lens,
             int32_t* cu_seqlens, int32_t* cu_splits, int32_t* split_seq, int32_t* split_start) {
    if (tpb == 0) return -1;
    if (split_tokens == 0) split_tokens = 512;
    split_tokens = (split_tokens + 127u) / 128u * 128u;
    uint32_t max_nb = 0, nsplits = 0;
    for (uint32_t b = 0; b < num_seqs; ++b) {
        const uint32_t len = context_lens[b];
        if (len == 0) return -1;
        const uint32_t needed = (len + tpb - 1) / tpb;
        if (needed > cu_blocks[b + 1] - cu_blocks[b]) return -1;
        for (uint32_t j = 0; j < needed; ++j) {
            const uint32_t id = ids[cu_blocks[b] + j];
            if (id == ORC_UNMAPPED || id >= num_pool_blocks) return -1;
        }
        if (needed > max_nb) max_nb = needed;
        nsplits += (len + split_tokens - 1) / split_tokens;
    }
    if (max_nb_out) *max_nb_out = max_nb;
    if (num_splits_out) *num_splits_out = nsplits;
    if (tables == NULL) return 0;
    int32_t tok = 0, spl = 0;
    for (uint32_t b = 0; b < num_seqs; ++b) {
        const uint32_t len = context_lens[b];
        const uint32_t needed = (len + tpb - 1) / tpb;
        for (uint32_t j = 0; j < max_nb; ++j) {
            tables[(uint64_t)b * max_nb + j] = j < needed ? (int32_t)ids[cu_blocks[b] + j] : -1;
        }
        seq_lens[b] = (int32_t)len;
        cu_seqlens[b] = tok;
        cu_splits[b] = spl;
        tok += (int32_t)len;
        for (uint32_t s = 0; s * split_tokens < len; ++s) {
            split_seq[spl] = (int32_t)b;
            split_start[spl] = (int32_t)(s * split_tokens);
            ++spl;
        }
    }
    cu_seqlens[num_seqs] = tok;
    cu_splits[num_seqs] = spl;
    return 0;
}

void orc_copy_block(uint8_t* pool, uint64_t block_stride, uint32_t num_pool_blocks, uint32_t src,
                    uint32_t dst, uint64_t copy_bytes) {
    if (src >= num_pool_blocks || dst >= num_pool_blocks) return;
    memmove(pool + (uint64_t)dst * block_stride, pool + (uint64_t)src * block_stride, copy_bytes);
}

/* ---------------------------------------------------------------- */
/* K/V append (tests/PagedAttention.test.cpp:97-127,                */
/* tests/EndToEnd.test.cpp:157-179)                                 */
/* ---------------------------------------------------------------- */

int orc_append_kv(uint8_t* pool, uint64_t block_stride, uint32_t num_pool_blocks, uint32_t elem_bytes,
                  uint32_t tpb, uint32_t num_layers, uint32_t num_kv_heads, uint32_t head_dim,
                  uint32_t first_layer, uint32_t layer_count, const uint32_t* frames, const uint32_t* slots,
                  uint32_t count, const uint8_t* k, const uint8_t* v) {
    if ((uint64_t)first_layer + layer_count > num_layers) return -1;
    for (uint32_t i = 0; i < count; ++i) {
        if (frames[i] >= num_pool_blocks || slots[i] >= tpb) return -1;
    }
    const uint64_t row = (uint64_t)head_dim * elem_bytes;
    for (uint32_t i = 0; i < count; ++i) {
        uint8_t* frame = pool + (uint64_t)frames[i] * block_stride;
        for (uint32_t l = 0; l < layer_count; ++l) {
            for (uint32_t s = 0; s < 2; ++s) {
                const uint8_t* src = (s == 0 ? k : v) + ((uint64_t)i * layer_count + l) * num_kv_heads * row;
                for (uint32_t h = 0; h < num_kv_heads; ++h) {
                    const int64_t off = orc_element_offset(tpb, num_layers, num_kv_heads, head_dim,
                                                           first_layer + l, s, slots[i], h);
                    memcpy(frame + (uint64_t)off * elem_bytes, src + (uint64_t)h * row, row);
                }
            }
        }
    }
    return 0;
}

/* ---------------------------------------------------------------- */
/* M-RoPE positions (see oracle.h)                                  */
/* ---------------------------------------------------------------- */

static int mrope_span_ok(const orc_mrope_span* s) {
    const int64_t lim = (int64_t)1 << 24;
    if (s->token_count == 0 || s->kind > 2) return 0;
    for (int a = 0; a < 3; ++a) {
        if (s->origin[a] > lim || s->origin[a] < -lim || s->stride[a] > lim || s->stride[a] < -lim) return 0;
    }
    if (s->kind == 0) return 1;
    for (int a = 0; a < 3; ++a) {
        if (s->grid[a] < 1 || s->grid[a] > (int64_t)s->token_count) return 0;
    }
    if (s->kind == 1 && s->grid[0] != 1) return 0;
    return s->grid[0] * s->grid[1] * s->grid[2] == (int64_t)s->token_count;
}

int orc_mrope_positions(const orc_mrope_span* spans, uint32_t num_spans, uint32_t begin, uint32_t end,
                        int64_t* out) {
    if (begin > end) return -1;
    uint64_t prev_end = 0;
    for (uint32_t k = 0; k < num_spans; ++k) {
        if (!mrope_span_ok(&spans[k]) || spans[k].start_token < prev_end) return -1;
        prev_end = (uint64_t)spans[k].start_token + spans[k].token_count;
    }
    const uint32_t n = end - begin;
    int64_t running_max = -1;
    uint32_t k = 0;
    for (uint64_t p = 0; p < end; ++p) {
        while (k < num_spans && (uint64_t)spans[k].start_token + spans[k].token_count <= p) ++k;
        int64_t pos[3];
        if (k < num_spans && spans[k].start_token <= p) {
            const orc_mrope_span* s = &spans[k];
            const int64_t i = (int64_t)(p - s->start_token);
            int64_t coord[3];
            if (s->kind == 0) {
                coord[0] = coord[1] = coord[2] = i;
            } else {
                coord[0] = i / (s->grid[1] * s->grid[2]);
                coord[1] = (i / s->grid[2]) % s->grid[1];
                coord[2] = i % s->grid[2];
            }
            for (int a = 0; a < 3; ++a) pos[a] = s->origin[a] + coord[a] * s->stride[a];
        } else {
            pos[0] = pos[1] = pos[2] = running_max + 1;
        }
        for (int a = 0; a < 3; ++a) {
            if (pos[a] > running_max) running_max = pos[a];
        }
        if (p >= begin) {
            for (int a = 0; a < 3; ++a) out[(uint64_t)a * n + (p - begin)] = pos[a];
        }
    }
    return 0;
}
