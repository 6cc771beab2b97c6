/*
 * kv_oracle.c -- CPU restatement of Titan's paged KV-cache reference path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP product path, never the
 * thing measured or shipped.  Built with -O2 -ffp-contract=off
 * -fno-fast-math so f64 arithmetic follows the reference's Rust evaluation
 * order (no fused multiply-add, no reassociation).
 *
 * How each part is pinned (tests/test_oracle_*.py):
 *   cache (append/read/free list/exhaustion): the reference's own known-answer
 *     tests (cache.rs:258-472, paged_kv_gpu.rs:64-141, paged_kv_parity.rs:68-225)
 *     plus the closed-form index formula and gather(append(x)) == x.
 *   sdpa_decode: hand-computed f64 SDPA (sdpa_cpu_tests.rs:89-175), scattered ==
 *     contiguous, causal == truncated, single token returns the V row, and an
 *     independent numpy float64 softmax-attention on random inputs.
 *   prefill: per-query equality with a numpy causal-attention on a dense copy.
 *   f16/bf16 conversions: every finite f16 pattern against numpy, RNE ties.
 *   FP8 E4M3: all 256 codes against torch.float8_e4m3fn; quantisation against
 *     a brute-force nearest-code search (ties to even mantissa) and against
 *     torch's in-range conversion; saturation and NaN cases explicitly.
 *   CowBlockTable: cow_fork_test.rs:4-44.
 *   RadixTree: radix_cache_test.rs:4-95, plus a brute-force LRU model.
 *     Parity is pinned only under the logical clock (the reference uses
 *     Instant::now(), which nothing can pin).
 *   StreamingKvManager: streaming.rs:148-174 plus closed form on distinct
 *     scores.  Tie order of sort_unstable_by is Rust-std defined: parity is
 *     pinned only for distinct scores.
 */
#include "kv_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ======================= PagedKvCache (cache.rs) ======================= */

struct orc_cache {
    size_t n_blocks, block_tokens, heads, head_dim, elt;
    unsigned char* buffer;     /* cache.rs:52-53 */
    uint32_t* free_list;       /* stack: pop from the end (cache.rs:55) */
    size_t free_len;
    uint32_t** block_table;    /* cache.rs:57 */
    size_t* bt_len;
    size_t* bt_cap;
    size_t* seq_tokens;        /* cache.rs:59 */
    size_t n_seq, seq_cap;
};

static size_t row_len(const orc_cache* c) { return c->heads * c->head_dim; }          /* cache.rs:22-24 */
static size_t fpt(const orc_cache* c) { return 2 * row_len(c); }                     /* cache.rs:27-29 */
static size_t fpb(const orc_cache* c) { return c->block_tokens * fpt(c); }           /* cache.rs:32-34 */

int orc_cache_new(size_t n_blocks, size_t block_tokens, size_t heads, size_t head_dim,
                  size_t elt_bytes, orc_cache** out, const char** msg) {
    /* cache.rs:65-76: validation order and messages. */
    if (n_blocks == 0) { *msg = "n_blocks must be non-zero"; return ORC_INVALID_ARGS; }
    if (block_tokens == 0) { *msg = "block_tokens must be non-zero"; return ORC_INVALID_ARGS; }
    if (heads == 0 || head_dim == 0) { *msg = "heads and head_dim must be non-zero"; return ORC_INVALID_ARGS; }
    orc_cache* c = (orc_cache*)calloc(1, sizeof(orc_cache));
    c->n_blocks = n_blocks; c->block_tokens = block_tokens; c->heads = heads;
    c->head_dim = head_dim; c->elt = elt_bytes;
    /* cache.rs:78-79: zero-filled pool. */
    c->buffer = (unsigned char*)calloc(n_blocks * fpb(c), elt_bytes);
    /* cache.rs:81-86: ids pushed descending so pop() yields 0,1,2,... */
    c->free_list = (uint32_t*)malloc(n_blocks * sizeof(uint32_t));
    for (size_t i = 0; i < n_blocks; ++i) c->free_list[i] = (uint32_t)(n_blocks - 1 - i);
    c->free_len = n_blocks;
    *out = c;
    return ORC_OK;
}

void orc_cache_destroy(orc_cache* c) {
    if (!c) return;
    for (size_t s = 0; s < c->n_seq; ++s) free(c->block_table[s]);
    free(c->block_table); free(c->bt_len); free(c->bt_cap); free(c->seq_tokens);
    free(c->free_list); free(c->buffer); free(c);
}

void orc_cache_seed_free_list(orc_cache* c, const uint32_t* order, size_t n) {
    /* Stack whose successive pops return order[0], order[1], ... */
    c->free_list = (uint32_t*)realloc(c->free_list, (n ? n : 1) * sizeof(uint32_t));
    for (size_t i = 0; i < n; ++i) c->free_list[i] = order[n - 1 - i];
    c->free_len = n;
}

size_t orc_cache_blocks_total(const orc_cache* c) { return c->n_blocks; }
size_t orc_cache_blocks_used(const orc_cache* c) { return c->n_blocks - c->free_len; }
size_t orc_cache_sequences(const orc_cache* c) { return c->n_seq; }

long orc_cache_block_table(const orc_cache* c, size_t seq, uint32_t* out, size_t cap) {
    if (seq >= c->n_seq) return -1;
    size_t n = c->bt_len[seq];
    for (size_t i = 0; i < n && i < cap; ++i) out[i] = c->block_table[seq][i];
    return (long)n;
}

void orc_cache_free_sequence(orc_cache* c, size_t seq) {
    /* cache.rs:123-132: blocks return reversed, so the next pops reuse them in
     * their original order; the count resets, the sequence stays registered,
     * the data is not cleared. */
    if (seq >= c->n_seq) return;
    size_t n = c->bt_len[seq];
    for (size_t i = 0; i < n; ++i) c->free_list[c->free_len++] = c->block_table[seq][n - 1 - i];
    c->bt_len[seq] = 0;
    c->seq_tokens[seq] = 0;
}

size_t orc_cache_new_sequence(orc_cache* c) {
    if (c->n_seq == c->seq_cap) {
        size_t nc = c->seq_cap ? 2 * c->seq_cap : 8;
        c->block_table = (uint32_t**)realloc(c->block_table, nc * sizeof(uint32_t*));
        c->bt_len = (size_t*)realloc(c->bt_len, nc * sizeof(size_t));
        c->bt_cap = (size_t*)realloc(c->bt_cap, nc * sizeof(size_t));
        c->seq_tokens = (size_t*)realloc(c->seq_tokens, nc * sizeof(size_t));
        c->seq_cap = nc;
    }
    size_t id = c->n_seq++;
    c->block_table[id] = NULL; c->bt_len[id] = 0; c->bt_cap[id] = 0; c->seq_tokens[id] = 0;
    return id;
}

size_t orc_cache_token_count(const orc_cache* c, size_t seq) {
    return seq >= c->n_seq ? 0 : c->seq_tokens[seq];
}

int orc_cache_append(orc_cache* c, size_t seq, const void* key, size_t key_len,
                     const void* value, size_t value_len, size_t* blocks_used,
                     size_t* blocks_total, const char** msg) {
    const size_t m = row_len(c);
    /* cache.rs:154-162: argument checks come before any state change. */
    if (key_len != m || value_len != m) {
        *msg = "key/value length must equal heads * head_dim";
        return ORC_INVALID_ARGS;
    }
    if (seq >= c->n_seq) { *msg = "unknown sequence id"; return ORC_INVALID_ARGS; }
    /* cache.rs:164-177: a full (or absent) tail pops a fresh block. */
    size_t pos = c->seq_tokens[seq];
    if (pos % c->block_tokens == 0) {
        if (c->free_len == 0) {
            *blocks_used = orc_cache_blocks_used(c);
            *blocks_total = orc_cache_blocks_total(c);
            return ORC_POOL_EXHAUSTED;
        }
        uint32_t phys = c->free_list[--c->free_len];
        if (c->bt_len[seq] == c->bt_cap[seq]) {
            size_t nc = c->bt_cap[seq] ? 2 * c->bt_cap[seq] : 4;
            c->block_table[seq] = (uint32_t*)realloc(c->block_table[seq], nc * sizeof(uint32_t));
            c->bt_cap[seq] = nc;
        }
        c->block_table[seq][c->bt_len[seq]++] = phys;
    }
    /* cache.rs:179-191: K row at phys*fpb + slot*fpt, V row row_len later. */
    uint32_t phys = c->block_table[seq][c->bt_len[seq] - 1];
    size_t slot = pos % c->block_tokens;
    size_t key_off = (size_t)phys * fpb(c) + slot * fpt(c);
    size_t val_off = key_off + m;
    memcpy(c->buffer + key_off * c->elt, key, m * c->elt);
    memcpy(c->buffer + val_off * c->elt, value, m * c->elt);
    c->seq_tokens[seq] += 1;
    return ORC_OK;
}

int orc_cache_read_row(const orc_cache* c, size_t seq, size_t token, int is_value, void* out,
                       const char** msg) {
    /* cache.rs:205-226 */
    if (seq >= c->n_seq) { *msg = "unknown sequence id"; return ORC_INVALID_ARGS; }
    if (token >= c->seq_tokens[seq]) { *msg = "token out of range"; return ORC_INVALID_ARGS; }
    size_t block_index = token / c->block_tokens;
    size_t slot = token % c->block_tokens;
    if (block_index >= c->bt_len[seq]) { *msg = "token out of range"; return ORC_INVALID_ARGS; }
    uint32_t phys = c->block_table[seq][block_index];
    size_t base = (size_t)phys * fpb(c) + slot * fpt(c) + (is_value ? row_len(c) : 0);
    memcpy(out, c->buffer + base * c->elt, row_len(c) * c->elt);
    return ORC_OK;
}

int orc_cache_read_all(const orc_cache* c, size_t seq, int is_value, void* out, const char** msg) {
    /* cache.rs:240-255 */
    if (seq >= c->n_seq) { *msg = "unknown sequence id"; return ORC_INVALID_ARGS; }
    size_t n = c->seq_tokens[seq];
    unsigned char* o = (unsigned char*)out;
    for (size_t t = 0; t < n; ++t) {
        int rc = orc_cache_read_row(c, seq, t, is_value, o + t * row_len(c) * c->elt, msg);
        if (rc) return rc;
    }
    return ORC_OK;
}

const void* orc_cache_buffer(const orc_cache* c, size_t* n_bytes) {
    *n_bytes = c->n_blocks * fpb(c) * c->elt;
    return c->buffer;
}

/* ======================= sdpa_decode (forward_cpu.rs) ======================= */

static double dot_f64(const float* a, const float* b, size_t n) {
    /* forward_cpu.rs:265-267: f64 products summed left to right. */
    double s = 0.0;
    for (size_t i = 0; i < n; ++i) s += (double)a[i] * (double)b[i];
    return s;
}

/* window > 0 additionally keeps only the attention sinks t < sink and the
 * rolling window t >= max(sink, seq_tokens - 1 - window) (see
 * orc_sdpa_decode_window_batched); window == 0 is the reference function. */
static void sdpa_decode_core(const float* pool, const uint32_t* block_table, size_t block_tokens,
                             size_t seq_tokens, const float* query, size_t n_head, size_t n_head_kv,
                             size_t head_dim, int causal, size_t query_pos, size_t sink,
                             size_t window, float* out, double* mass) {
    /* forward_cpu.rs:436-439 */
    memset(out, 0, n_head * head_dim * sizeof(float));
    if (seq_tokens == 0 || n_head == 0 || head_dim == 0) return;
    if (n_head_kv == 0 || n_head % n_head_kv != 0) abort(); /* forward_cpu.rs:440 assert */
    const size_t group = n_head / n_head_kv;
    const size_t rl = n_head_kv * head_dim;
    const size_t f_tok = 2 * rl;
    const size_t f_blk = block_tokens * f_tok;
    const double scale = 1.0 / sqrt((double)head_dim);
    double* scores = (double*)malloc(seq_tokens * sizeof(double));
    double* weights = (double*)malloc(seq_tokens * sizeof(double));
    double* out_h = (double*)malloc(head_dim * sizeof(double));

    for (size_t qh = 0; qh < n_head; ++qh) {
        const size_t hk = qh / group;
        const float* qv = query + qh * head_dim;
        double max_score = -INFINITY;
        /* forward_cpu.rs:455-473: scores for unmasked tokens, running max. */
        for (size_t t = 0; t < seq_tokens; ++t) {
            scores[t] = -INFINITY;
            if (causal && t > query_pos) continue;
            if (window && t >= sink && t + 1 + window < seq_tokens) continue; /* t < n - 1 - W */
            size_t phys = block_table[t / block_tokens];
            size_t base = phys * f_blk + (t % block_tokens) * f_tok;
            double s = dot_f64(qv, pool + base + hk * head_dim, head_dim) * scale;
            scores[t] = s;
            if (s > max_score) max_score = s;
        }
        /* forward_cpu.rs:475-490: weights exp(s - max) / sum over finite scores. */
        for (size_t t = 0; t < seq_tokens; ++t) weights[t] = 0.0;
        if (isfinite(max_score)) {
            double sum_exp = 0.0;
            for (size_t t = 0; t < seq_tokens; ++t) {
                if (isfinite(scores[t])) {
                    double e = exp(scores[t] - max_score);
                    weights[t] = e;
                    sum_exp += e;
                }
            }
            if (sum_exp > 0.0)
                for (size_t t = 0; t < seq_tokens; ++t) weights[t] /= sum_exp;
        }
        /* attention mass per physical page, summed over heads: the H2O score
         * StreamingKvManager::record_attention_mass adds (streaming.rs:135-141) */
        if (mass)
            for (size_t t = 0; t < seq_tokens; ++t)
                if (weights[t] != 0.0) mass[block_table[t / block_tokens]] += weights[t];
        /* forward_cpu.rs:492-506: f64 weighted sum of V rows, zero weights skipped. */
        for (size_t d = 0; d < head_dim; ++d) out_h[d] = 0.0;
        for (size_t t = 0; t < seq_tokens; ++t) {
            double wt = weights[t];
            if (wt == 0.0) continue;
            size_t phys = block_table[t / block_tokens];
            size_t base = phys * f_blk + (t % block_tokens) * f_tok;
            const float* v = pool + base + rl + hk * head_dim;
            for (size_t d = 0; d < head_dim; ++d) out_h[d] += wt * (double)v[d];
        }
        for (size_t d = 0; d < head_dim; ++d) out[qh * head_dim + d] = (float)out_h[d];
    }
    free(scores); free(weights); free(out_h);
}

void orc_sdpa_decode(const float* pool, const uint32_t* block_table, size_t block_tokens,
                     size_t seq_tokens, const float* query, size_t n_head, size_t n_head_kv,
                     size_t head_dim, int causal, size_t query_pos, float* out) {
    sdpa_decode_core(pool, block_table, block_tokens, seq_tokens, query, n_head, n_head_kv,
                     head_dim, causal, query_pos, 0, 0, out, NULL);
}

/* Decode attention over the protected-sinks range of the reference's design
 * (openspec/changes/archive/2026-08-28-agent-runtime-optimizations/
 * design.md:211-216, specs/protected-kv-sinks/spec.md:9-15): the query at
 * pos = n - 1 attends t in [0, sink) U [max(sink, pos - W), pos]; W == 0
 * attends all n tokens.  Otherwise sdpa_decode (forward_cpu.rs:424-510). */
void orc_sdpa_decode_window_batched(const float* pool, const uint32_t* bt, size_t bt_stride,
                                    const uint32_t* lens, size_t batch, size_t block_tokens,
                                    const float* q, size_t n_head, size_t n_head_kv,
                                    size_t head_dim, size_t sink, size_t window, float* out,
                                    double* mass) {
    const size_t qs = n_head * head_dim;
    for (size_t b = 0; b < batch; ++b) {
        size_t n = lens[b];
        sdpa_decode_core(pool, bt + b * bt_stride, block_tokens, n, q + b * qs, n_head, n_head_kv,
                         head_dim, 1, n ? n - 1 : 0, sink, window, out + b * qs, mass);
    }
}

void orc_sdpa_decode_batched(const float* pool, const uint32_t* bt, size_t bt_stride,
                             const uint32_t* lens, size_t batch, size_t block_tokens,
                             const float* q, size_t n_head, size_t n_head_kv, size_t head_dim,
                             float* out) {
    const size_t qs = n_head * head_dim;
    for (size_t b = 0; b < batch; ++b) {
        size_t n = lens[b];
        orc_sdpa_decode(pool, bt + b * bt_stride, block_tokens, n, q + b * qs, n_head,
                        n_head_kv, head_dim, 1, n ? n - 1 : 0, out + b * qs);
    }
}

void orc_prefill_causal(const float* pool, const uint32_t* block_table, size_t block_tokens,
                        const float* q, size_t q_tokens, size_t pos_offset, size_t n_head,
                        size_t n_head_kv, size_t head_dim, float* out) {
    const size_t qs = n_head * head_dim;
    for (size_t i = 0; i < q_tokens; ++i) {
        size_t p = pos_offset + i;
        orc_sdpa_decode(pool, block_table, block_tokens, p + 1, q + i * qs, n_head, n_head_kv,
                        head_dim, 1, p, out + i * qs);
    }
}

/* ======================= conversions ======================= */

float orc_f16_to_f32(uint16_t bits) {
    /* forward_cpu.rs:74-92 */
    uint32_t sign = bits >> 15, ex = (bits >> 10) & 0x1F, mant = bits & 0x3FF;
    if (ex == 0) {
        if (mant == 0) return sign ? -0.0f : 0.0f;
        float v = (float)mant * ldexpf(1.0f, -24);
        return sign ? -v : v;
    }
    if (ex == 31) return INFINITY;
    float v = (1.0f + (float)mant / 1024.0f) * ldexpf(1.0f, (int)ex - 15);
    return sign ? -v : v;
}

void orc_f16_to_f32_array(const uint16_t* in, float* out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = orc_f16_to_f32(in[i]);
}

uint16_t orc_f32_to_f16_rne(float x) {
    uint32_t u; memcpy(&u, &x, 4);
    uint32_t sign = (u >> 16) & 0x8000u;
    uint32_t ex = (u >> 23) & 0xFF;
    uint32_t mant = u & 0x7FFFFFu;
    if (ex == 0xFF) return (uint16_t)(sign | 0x7C00u | (mant ? 0x200u : 0u));
    int e = (int)ex - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7C00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        uint32_t m = mant | 0x800000u;          /* 24-bit significand */
        int shift = 14 - e;                     /* to the 2^-24 grid */
        uint32_t half = 1u << (shift - 1);
        uint32_t r = m >> shift, rem = m & ((1u << shift) - 1);
        if (rem > half || (rem == half && (r & 1u))) r += 1;
        return (uint16_t)(sign | r);
    }
    uint32_t r = ((uint32_t)e << 10) | (mant >> 13);
    uint32_t rem = mant & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) r += 1; /* may carry into inf: correct */
    return (uint16_t)(sign | r);
}

uint16_t orc_f32_to_bf16_rne(float x) {
    uint32_t u; memcpy(&u, &x, 4);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40u); /* quiet NaN */
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

void orc_bf16_to_f32_array(const uint16_t* in, float* out, size_t n) {
    for (size_t i = 0; i < n; ++i) { uint32_t u = (uint32_t)in[i] << 16; memcpy(&out[i], &u, 4); }
}

/* FP8 E4M3 (OCP E4M3FN: bias 7, no infinities, S.1111.111 = NaN, max 448),
 * the format named by the reference's FP8 KV design
 * (openspec/archive/2026-08-28-fp8-kv-cache-quantization/design.md:3-6),
 * with one f32 scale per kv head and K/V (spec.md:8-10): stored code =
 * quantize(x / scale), value = decode(code) * scale.  No reference kernel
 * implements it, so this is a restatement of the format itself. */
float orc_e4m3_to_f32(uint8_t code) {
    const int s = code >> 7, e = (code >> 3) & 15, m = code & 7;
    if (e == 15 && m == 7) return NAN;
    const float v = e == 0 ? ldexpf((float)m, -9) : ldexpf((float)(8 + m), e - 10);
    return s ? -v : v;
}

/* Round to nearest, ties to even mantissa; |x/scale| >= 448 (and inf)
 * saturates to +-448; NaN -> S.1111.111. */
uint8_t orc_f32_to_e4m3(float x, float scale) {
    const float y = x / scale;
    uint32_t u; memcpy(&u, &y, 4);
    const uint8_t s = (uint8_t)((u >> 24) & 0x80u);
    if (isnan(y)) return (uint8_t)(s | 0x7Fu);
    const float a = fabsf(y);
    if (a >= 448.0f) return (uint8_t)(s | 0x7Eu);
    if (a < 0.015625f) return (uint8_t)(s | (uint8_t)rintf(a * 512.0f)); /* 2^-9 grid; 8 = 2^-6 */
    int e;
    frexpf(a, &e);
    e -= 1;                                          /* a in [2^e, 2^(e+1)), e in -6..8 */
    float m = rintf(ldexpf(a, -e) * 8.0f) - 8.0f;   /* 0..8 */
    if (m == 8.0f) { e += 1; m = 0.0f; }
    int code = ((e + 7) << 3) | (int)m;
    if (code > 0x7E) code = 0x7E;
    return (uint8_t)(s | code);
}

void orc_e4m3_to_f32_array(const uint8_t* in, float* out, size_t n, float scale) {
    for (size_t i = 0; i < n; ++i) out[i] = orc_e4m3_to_f32(in[i]) * scale;
}

void orc_f32_to_e4m3_array(const float* in, uint8_t* out, size_t n, float scale) {
    for (size_t i = 0; i < n; ++i) out[i] = orc_f32_to_e4m3(in[i], scale);
}

/* ======================= generators ======================= */

static uint32_t xs_next(uint32_t* s) {
    uint32_t x = *s;
    x ^= x << 13; x ^= x >> 17; x ^= x << 5;
    *s = x;
    return x;
}

void orc_xorshift_a_f32(uint32_t seed, float* out, size_t n) {
    uint32_t s = seed == 0 ? 0x6D2B79F5u : seed;
    for (size_t i = 0; i < n; ++i)
        out[i] = (float)((double)xs_next(&s) / (4294967295.0 + 1.0) * 2.0 - 1.0);
}

void orc_generate_rows_b(uint32_t seed, size_t n_tokens, size_t row_len_, float* keys,
                         float* values) {
    uint32_t s = seed;
    for (size_t t = 0; t < n_tokens; ++t)
        for (size_t h = 0; h < row_len_; ++h) {
            keys[t * row_len_ + h] = (float)(xs_next(&s) & 0x00FFFFFFu) / (float)0x00800000u - 1.0f;
            values[t * row_len_ + h] = (float)(xs_next(&s) & 0x00FFFFFFu) / (float)0x00800000u - 1.0f;
        }
}

void orc_fill_pool_paged(float* pool, const uint32_t* block_table, size_t block_tokens,
                         size_t n_head_kv, size_t head_dim, uint32_t seed, size_t n_tokens) {
    const size_t rl = n_head_kv * head_dim, f_tok = 2 * rl, f_blk = block_tokens * f_tok;
    uint32_t s = seed == 0 ? 0x6D2B79F5u : seed;
    for (size_t t = 0; t < n_tokens; ++t) {
        size_t base = (size_t)block_table[t / block_tokens] * f_blk + (t % block_tokens) * f_tok;
        for (size_t i = 0; i < rl; ++i)
            pool[base + i] = (float)((double)xs_next(&s) / (4294967295.0 + 1.0) * 2.0 - 1.0);
        for (size_t i = 0; i < rl; ++i)
            pool[base + rl + i] = (float)((double)xs_next(&s) / (4294967295.0 + 1.0) * 2.0 - 1.0);
    }
}

/* ======================= CowBlockTable (cow.rs) ======================= */

typedef struct orc_shared { uint32_t id; int dirty; size_t rc; } orc_shared; /* Arc<SharedBlock> */

struct orc_cow { orc_shared** blocks; size_t len, cap; size_t seq_len; };

static void cow_push(orc_cow* t, orc_shared* b) {
    if (t->len == t->cap) {
        t->cap = t->cap ? 2 * t->cap : 4;
        t->blocks = (orc_shared**)realloc(t->blocks, t->cap * sizeof(orc_shared*));
    }
    t->blocks[t->len++] = b;
}
static void cow_release(orc_shared* b) { if (--b->rc == 0) free(b); }

orc_cow* orc_cow_new(void) { return (orc_cow*)calloc(1, sizeof(orc_cow)); }

orc_cow* orc_cow_fork(const orc_cow* t) {
    orc_cow* c = orc_cow_new();
    for (size_t i = 0; i < t->len; ++i) { t->blocks[i]->rc++; cow_push(c, t->blocks[i]); }
    c->seq_len = t->seq_len;
    return c;
}

void orc_cow_destroy(orc_cow* t) {
    if (!t) return;
    for (size_t i = 0; i < t->len; ++i) cow_release(t->blocks[i]);
    free(t->blocks); free(t);
}

void orc_cow_append_block(orc_cow* t, uint32_t id) {
    orc_shared* b = (orc_shared*)malloc(sizeof(orc_shared));
    b->id = id; b->dirty = 0; b->rc = 1;
    cow_push(t, b);
}

int orc_cow_is_shared(const orc_cow* t, size_t idx) { return idx < t->len && t->blocks[idx]->rc > 1; }

int orc_cow_tail_needs_cow(const orc_cow* t) { return t->len > 0 && t->blocks[t->len - 1]->rc > 1; }

void orc_cow_perform_tail_cow(orc_cow* t, uint32_t new_id) {
    if (t->len == 0) return;
    orc_shared* b = (orc_shared*)malloc(sizeof(orc_shared));
    b->id = new_id; b->dirty = 1; b->rc = 1;
    cow_release(t->blocks[t->len - 1]);
    t->blocks[t->len - 1] = b;
}

size_t orc_cow_ids(const orc_cow* t, uint32_t* out, size_t cap) {
    for (size_t i = 0; i < t->len && i < cap; ++i) out[i] = t->blocks[i]->id;
    return t->len;
}
size_t orc_cow_len(const orc_cow* t) { return t->len; }
int orc_cow_is_dirty(const orc_cow* t, size_t idx) { return idx < t->len ? t->blocks[idx]->dirty : 0; }
size_t orc_cow_refcount(const orc_cow* t, size_t idx) { return idx < t->len ? t->blocks[idx]->rc : 0; }
size_t orc_cow_seq_len(const orc_cow* t) { return t->seq_len; }
void orc_cow_set_seq_len(orc_cow* t, size_t v) { t->seq_len = v; }

/* ======================= RadixTree (radix.rs) ======================= */

typedef struct rnode rnode;
typedef struct { uint32_t key; rnode* child; } rkid;
struct rnode {
    uint32_t* tokens; size_t ntok;
    uint32_t* blocks; size_t nblk;
    rkid* kids; size_t nkids, kcap;   /* sorted ascending by key (BTreeMap order) */
    uint64_t last_accessed;
    int is_pinned;
    size_t ref_count;
};
struct orc_radix { rnode* root; size_t block_tokens; uint64_t clock; };

static uint64_t rx_now(orc_radix* t) { return ++t->clock; }

static rnode* rnode_new(orc_radix* t, const uint32_t* tok, size_t ntok, const uint32_t* blk,
                        size_t nblk, int pinned) {
    /* radix.rs:30-39 */
    rnode* n = (rnode*)calloc(1, sizeof(rnode));
    n->tokens = (uint32_t*)malloc((ntok ? ntok : 1) * sizeof(uint32_t));
    if (ntok) memcpy(n->tokens, tok, ntok * sizeof(uint32_t));
    n->ntok = ntok;
    n->blocks = (uint32_t*)malloc((nblk ? nblk : 1) * sizeof(uint32_t));
    if (nblk) memcpy(n->blocks, blk, nblk * sizeof(uint32_t));
    n->nblk = nblk;
    n->last_accessed = rx_now(t);
    n->is_pinned = pinned;
    return n;
}

static void rnode_free(rnode* n) {
    for (size_t i = 0; i < n->nkids; ++i) rnode_free(n->kids[i].child);
    free(n->kids); free(n->tokens); free(n->blocks); free(n);
}

static long kid_find(const rnode* n, uint32_t key) {
    size_t lo = 0, hi = n->nkids;
    while (lo < hi) {
        size_t mid = (lo + hi) / 2;
        if (n->kids[mid].key < key) lo = mid + 1; else hi = mid;
    }
    return (lo < n->nkids && n->kids[lo].key == key) ? (long)lo : -1;
}

static void kid_put(rnode* n, uint32_t key, rnode* child) {
    long f = kid_find(n, key);
    if (f >= 0) { n->kids[f].child = child; return; }
    if (n->nkids == n->kcap) {
        n->kcap = n->kcap ? 2 * n->kcap : 4;
        n->kids = (rkid*)realloc(n->kids, n->kcap * sizeof(rkid));
    }
    size_t i = n->nkids;
    while (i > 0 && n->kids[i - 1].key > key) { n->kids[i] = n->kids[i - 1]; --i; }
    n->kids[i].key = key; n->kids[i].child = child;
    n->nkids++;
}

static rnode* kid_take(rnode* n, size_t idx) {
    rnode* c = n->kids[idx].child;
    memmove(&n->kids[idx], &n->kids[idx + 1], (n->nkids - idx - 1) * sizeof(rkid));
    n->nkids--;
    return c;
}

static size_t lcp(const uint32_t* a, size_t na, const uint32_t* b, size_t nb) {
    size_t i = 0;
    while (i < na && i < nb && a[i] == b[i]) ++i;
    return i;
}

orc_radix* orc_radix_new(size_t block_tokens) {
    orc_radix* t = (orc_radix*)calloc(1, sizeof(orc_radix));
    t->block_tokens = block_tokens;
    t->root = rnode_new(t, NULL, 0, NULL, 0, 1);
    return t;
}

void orc_radix_destroy(orc_radix* t) { if (t) { rnode_free(t->root); free(t); } }

size_t orc_radix_match_prefix(orc_radix* t, const uint32_t* tokens, size_t n, uint32_t* out,
                              size_t cap, size_t* n_blocks) {
    /* radix.rs:73-117 */
    size_t matched = 0, nb = 0;
    rnode* cur = t->root;
    cur->last_accessed = rx_now(t);
    while (n > 0) {
        long k = kid_find(cur, tokens[0]);
        if (k < 0) break;
        rnode* child = cur->kids[k].child;
        child->last_accessed = rx_now(t);
        size_t common = lcp(tokens, n, child->tokens, child->ntok);
        if (common == child->ntok) {
            matched += common;
            for (size_t i = 0; i < child->nblk; ++i, ++nb) if (nb < cap) out[nb] = child->blocks[i];
            tokens += common; n -= common;
            cur = child;
        } else {
            matched += common;
            size_t full = common / t->block_tokens;
            if (full > child->nblk) full = child->nblk;
            for (size_t i = 0; i < full; ++i, ++nb) if (nb < cap) out[nb] = child->blocks[i];
            break;
        }
    }
    *n_blocks = nb;
    return matched;
}

void orc_radix_insert(orc_radix* t, const uint32_t* tokens, size_t n, const uint32_t* blocks,
                      size_t nb, int is_pinned) {
    /* radix.rs:120-204 */
    if (n == 0) return;
    rnode* cur = t->root;
    while (n > 0) {
        uint32_t first = tokens[0];
        long k = kid_find(cur, first);
        if (k < 0) {
            kid_put(cur, first, rnode_new(t, tokens, n, blocks, nb, is_pinned));
            return;
        }
        rnode* child = kid_take(cur, (size_t)k);
        size_t common = lcp(tokens, n, child->tokens, child->ntok);
        if (common == child->ntok) {
            size_t cb = child->nblk;
            if (nb >= cb) { blocks += cb; nb -= cb; } else { nb = 0; }
            tokens += common; n -= common;
            kid_put(cur, first, child);
            cur = child;
        } else {
            size_t sbc = common / t->block_tokens;
            if (sbc > child->nblk) sbc = child->nblk;
            rnode* split = rnode_new(t, child->tokens, common, child->blocks, sbc, is_pinned);
            /* Re-attach the old child with its remaining suffix. */
            size_t rest_tok = child->ntok - common, rest_blk = child->nblk - sbc;
            memmove(child->tokens, child->tokens + common, rest_tok * sizeof(uint32_t));
            memmove(child->blocks, child->blocks + sbc, rest_blk * sizeof(uint32_t));
            child->ntok = rest_tok; child->nblk = rest_blk;
            kid_put(split, child->tokens[0], child);
            const uint32_t* ins_tok = tokens + common;
            size_t ins_n = n - common;
            const uint32_t* ins_blk = blocks;
            size_t ins_nb = 0;
            if (nb >= sbc) { ins_blk = blocks + sbc; ins_nb = nb - sbc; }
            if (ins_n > 0)
                kid_put(split, ins_tok[0], rnode_new(t, ins_tok, ins_n, ins_blk, ins_nb, is_pinned));
            kid_put(cur, first, split);
            return;
        }
    }
}

typedef struct { int found; uint32_t* blocks; size_t nblk; } rx_evicted;

static rx_evicted find_and_remove_oldest_leaf(rnode* cur) {
    /* radix.rs:224-254: eligible direct children first (oldest by strict <,
     * first in key order on ties), else depth-first into children. */
    rx_evicted r = {0, NULL, 0};
    long oldest = -1;
    uint64_t oldest_time = 0;
    for (size_t i = 0; i < cur->nkids; ++i) {
        rnode* c = cur->kids[i].child;
        if (!c->is_pinned && c->ref_count == 0 && c->nkids == 0 &&
            (oldest < 0 || c->last_accessed < oldest_time)) {
            oldest_time = c->last_accessed;
            oldest = (long)i;
        }
    }
    if (oldest >= 0) {
        rnode* c = kid_take(cur, (size_t)oldest);
        r.found = 1; r.blocks = c->blocks; r.nblk = c->nblk;
        c->blocks = NULL;
        rnode_free(c);
        return r;
    }
    for (size_t i = 0; i < cur->nkids; ++i) {
        r = find_and_remove_oldest_leaf(cur->kids[i].child);
        if (r.found) return r;
    }
    return r;
}

size_t orc_radix_evict_lru(orc_radix* t, size_t target, uint32_t* out, size_t cap) {
    /* radix.rs:208-222 */
    size_t freed = 0;
    while (freed < target) {
        rx_evicted r = find_and_remove_oldest_leaf(t->root);
        if (!r.found) break;
        for (size_t i = 0; i < r.nblk; ++i, ++freed) if (freed < cap) out[freed] = r.blocks[i];
        free(r.blocks);
    }
    return freed;
}

static size_t count_blocks(const rnode* n) {
    size_t s = n->nblk;
    for (size_t i = 0; i < n->nkids; ++i) s += count_blocks(n->kids[i].child);
    return s;
}
size_t orc_radix_total_cached_blocks(const orc_radix* t) { return count_blocks(t->root); }

static int has_any(const rnode* n, const uint32_t* set, size_t ns) {
    for (size_t i = 0; i < n->nblk; ++i)
        for (size_t j = 0; j < ns; ++j)
            if (n->blocks[i] == set[j]) return 1;
    return 0;
}

static void prune_nodes(rnode* n, const uint32_t* set, size_t ns) {
    /* radix.rs:279-289: drop children holding any freed block, then recurse. */
    size_t w = 0;
    for (size_t i = 0; i < n->nkids; ++i) {
        if (has_any(n->kids[i].child, set, ns)) rnode_free(n->kids[i].child);
        else n->kids[w++] = n->kids[i];
    }
    n->nkids = w;
    for (size_t i = 0; i < n->nkids; ++i) prune_nodes(n->kids[i].child, set, ns);
}

void orc_radix_invalidate_physical_blocks(orc_radix* t, const uint32_t* blocks, size_t n) {
    if (n == 0) return;
    prune_nodes(t->root, blocks, n);
}

int orc_radix_set_ref_count(orc_radix* t, const uint32_t* tokens, size_t n, size_t ref_count) {
    rnode* cur = t->root;
    while (n > 0) {
        long k = kid_find(cur, tokens[0]);
        if (k < 0) return -1;
        rnode* c = cur->kids[k].child;
        if (c->ntok > n || lcp(tokens, n, c->tokens, c->ntok) != c->ntok) return -1;
        tokens += c->ntok; n -= c->ntok;
        cur = c;
    }
    cur->ref_count = ref_count;
    return 0;
}

/* ======================= StreamingKvManager (streaming.rs) ======================= */

static size_t div_ceil(size_t a, size_t b) { return (a + b - 1) / b; }

orc_stream_cfg orc_stream_cfg_new(size_t sink, size_t recent, size_t budget, size_t bt) {
    /* streaming.rs:31-49 (clamps in this order) */
    orc_stream_cfg c;
    c.block_tokens = bt > 1 ? bt : 1;
    c.sink_tokens = sink > 1 ? sink : 1;
    c.recent_window_tokens = recent > c.block_tokens ? recent : c.block_tokens;
    size_t floor_ = c.sink_tokens + c.recent_window_tokens;
    c.max_budget_tokens = budget > floor_ ? budget : floor_;
    return c;
}
orc_stream_cfg orc_stream_cfg_default(void) {
    orc_stream_cfg c = {4, 256, 512, 16};
    return c;
}
size_t orc_stream_sink_blocks(orc_stream_cfg c) { return div_ceil(c.sink_tokens, c.block_tokens); }
size_t orc_stream_recent_blocks(orc_stream_cfg c) { return div_ceil(c.recent_window_tokens, c.block_tokens); }
size_t orc_stream_max_active_blocks(orc_stream_cfg c) { return div_ceil(c.max_budget_tokens, c.block_tokens); }

struct orc_stream { orc_stream_cfg cfg; float* scores; size_t n_scores; };

orc_stream* orc_stream_new(orc_stream_cfg c) {
    orc_stream* m = (orc_stream*)calloc(1, sizeof(orc_stream));
    m->cfg = c;
    m->n_scores = orc_stream_max_active_blocks(c) * 4;
    m->scores = (float*)calloc(m->n_scores ? m->n_scores : 1, sizeof(float));
    return m;
}
void orc_stream_destroy(orc_stream* m) { if (m) { free(m->scores); free(m); } }

void orc_stream_record_attention_mass(orc_stream* m, uint32_t block, float mass) {
    size_t idx = block;
    if (idx >= m->n_scores) {
        size_t nn = idx + 64;
        m->scores = (float*)realloc(m->scores, nn * sizeof(float));
        for (size_t i = m->n_scores; i < nn; ++i) m->scores[i] = 0.0f;
        m->n_scores = nn;
    }
    m->scores[idx] += mass;
}
size_t orc_stream_scores_len(const orc_stream* m) { return m->n_scores; }

typedef struct { uint32_t b; float s; } scored;

/* Descending by score; NaN compares Equal (streaming.rs:112-113).  Stable
 * insertion sort: matches the reference whenever scores are distinct. */
static int sc_less(scored a, scored b) { return b.s < a.s; }

void orc_stream_prune_blocks(const orc_stream* m, const uint32_t* table, size_t n,
                             uint32_t* retained, size_t* n_retained, uint32_t* evicted,
                             size_t* n_evicted) {
    size_t max_blocks = orc_stream_max_active_blocks(m->cfg);
    *n_evicted = 0;
    if (n <= max_blocks) {
        if (n) memcpy(retained, table, n * sizeof(uint32_t));  /* table may be NULL when n == 0 */
        *n_retained = n;
        return;
    }
    size_t sink = orc_stream_sink_blocks(m->cfg); if (sink > n) sink = n;
    size_t recent = orc_stream_recent_blocks(m->cfg); if (recent > n - sink) recent = n - sink;
    size_t mid_n = n - sink - recent;
    size_t allow = max_blocks > sink + recent ? max_blocks - (sink + recent) : 0;
    scored* mid = (scored*)malloc((mid_n ? mid_n : 1) * sizeof(scored));
    for (size_t i = 0; i < mid_n; ++i) {
        uint32_t b = table[sink + i];
        mid[i].b = b;
        mid[i].s = b < m->n_scores ? m->scores[b] : 0.0f;
    }
    for (size_t i = 1; i < mid_n; ++i) {
        scored x = mid[i];
        size_t j = i;
        while (j > 0 && sc_less(x, mid[j - 1])) { mid[j] = mid[j - 1]; --j; }
        mid[j] = x;
    }
    size_t r = 0;
    for (size_t i = 0; i < sink; ++i) retained[r++] = table[i];
    for (size_t i = 0; i < mid_n && i < allow; ++i) retained[r++] = mid[i].b;
    for (size_t i = 0; i < recent; ++i) retained[r++] = table[n - recent + i];
    *n_retained = r;
    size_t e = 0;
    for (size_t i = allow; i < mid_n; ++i) evicted[e++] = mid[i].b;
    *n_evicted = e;
    free(mid);
}
