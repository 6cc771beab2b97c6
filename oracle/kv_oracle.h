/*
 * kv_oracle.h -- CPU restatement of Titan's paged KV-cache reference path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker that the HIP
 * product path is compared against.  Only tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg may load it.  The product (titan_amd/)
 * never links, loads or calls anything declared here.
 *
 * Every function restates one reference function; the reference file:line
 * it follows is given beside it (paths relative to the reference root).
 * Parity pinning of each function is documented in kv_oracle.c's header.
 */
#ifndef TITAN_KV_ORACLE_H
#define TITAN_KV_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes share numbering with the product C-ABI (include/engine_hip.h). */
enum {
    ORC_OK = 0,
    ORC_POOL_EXHAUSTED = 20, /* KvCacheError::PoolExhausted (engine-kvcache/src/error.rs:8-11) */
    ORC_INVALID_ARGS = 21,   /* KvCacheError::InvalidArgs   (engine-kvcache/src/error.rs:14-15) */
};

/* ---------------- PagedKvCache (engine-kvcache/src/cache.rs) ---------------- */
typedef struct orc_cache orc_cache;

/* cache.rs:8-40 (config) + cache.rs:64-95 (new).  elt_bytes generalises the
 * reference's f32 element (4) to 2-byte f16/bf16 storage; the copy semantics
 * are unchanged (rows are copied verbatim). */
int orc_cache_new(size_t n_blocks, size_t block_tokens, size_t heads, size_t head_dim,
                  size_t elt_bytes, orc_cache** out, const char** msg);
void orc_cache_destroy(orc_cache* c);
/* Extension (no reference counterpart): replace the free list so that
 * successive pops yield order[0], order[1], ... */
void orc_cache_seed_free_list(orc_cache* c, const uint32_t* order, size_t n);
size_t orc_cache_new_sequence(orc_cache* c);                        /* cache.rs:135-141 */
void orc_cache_free_sequence(orc_cache* c, size_t seq);             /* cache.rs:123-132 */
size_t orc_cache_token_count(const orc_cache* c, size_t seq);       /* cache.rs:144-149 */
size_t orc_cache_blocks_total(const orc_cache* c);                  /* cache.rs:103-105 */
size_t orc_cache_blocks_used(const orc_cache* c);                   /* cache.rs:108-110 */
size_t orc_cache_sequences(const orc_cache* c);                     /* cache.rs:113-115 */
/* cache.rs:119-121; returns -1 for an unknown sequence, else the row length. */
long orc_cache_block_table(const orc_cache* c, size_t seq, uint32_t* out, size_t cap);
/* cache.rs:153-192.  key/value are elt_bytes-sized elements. */
int orc_cache_append(orc_cache* c, size_t seq, const void* key, size_t key_len,
                     const void* value, size_t value_len, size_t* blocks_used,
                     size_t* blocks_total, const char** msg);
/* cache.rs:195-226 (read_key / read_value / row). */
int orc_cache_read_row(const orc_cache* c, size_t seq, size_t token, int is_value, void* out,
                       const char** msg);
/* cache.rs:230-255 (read_keys / read_values / read_all).  out holds
 * token_count*row_len elements. */
int orc_cache_read_all(const orc_cache* c, size_t seq, int is_value, void* out, const char** msg);
/* Backing buffer (cache.rs:52-53), n_blocks*floats_per_block elements. */
const void* orc_cache_buffer(const orc_cache* c, size_t* n_bytes);

/* ---------------- sdpa_decode (engine-core/src/forward_cpu.rs) ---------------- */
/* forward_cpu.rs:424-510 with dot_f64 (forward_cpu.rs:265-267). */
void orc_sdpa_decode(const float* pool, const uint32_t* block_table, size_t block_tokens,
                     size_t seq_tokens, const float* query, size_t n_head, size_t n_head_kv,
                     size_t head_dim, int causal, size_t query_pos, float* out);
/* Batched driver over orc_sdpa_decode: sequence b uses block-table row
 * bt + b*bt_stride, attends lens[b] tokens causally at query_pos lens[b]-1,
 * and reads q/out at b*n_head*head_dim. */
void orc_sdpa_decode_batched(const float* pool, const uint32_t* bt, size_t bt_stride,
                             const uint32_t* lens, size_t batch, size_t block_tokens,
                             const float* q, size_t n_head, size_t n_head_kv, size_t head_dim,
                             float* out);
/* Causal chunked prefill as the reference's FlashAttention2 kernel defines it
 * (engine-cuda/kernels/flash_attention_2.cu:44-68): query i sits at global
 * position pos_offset+i and attends keys 0..=pos_offset+i.  Expressed through
 * orc_sdpa_decode exactly as the reference's own parity test does
 * (engine-cuda/tests/flash_attention_parity.rs:145-187).
 * q/out: [q_tokens, n_head, head_dim]. */
void orc_prefill_causal(const float* pool, const uint32_t* block_table, size_t block_tokens,
                        const float* q, size_t q_tokens, size_t pos_offset, size_t n_head,
                        size_t n_head_kv, size_t head_dim, float* out);

/* ---------------- element conversions ---------------- */
/* forward_cpu.rs:74-92 (maps every exponent-31 pattern, NaN included, to +inf). */
float orc_f16_to_f32(uint16_t bits);
void orc_f16_to_f32_array(const uint16_t* in, float* out, size_t n);
/* No reference counterpart: IEEE-754 round-to-nearest-even narrowing and
 * bf16 widening (textbook; pinned against numpy/torch in tests). */
uint16_t orc_f32_to_f16_rne(float x);
uint16_t orc_f32_to_bf16_rne(float x);
void orc_bf16_to_f32_array(const uint16_t* in, float* out, size_t n);

/* ---------------- test-vector generators ---------------- */
/* engine-cuda/tests/common/mod.rs:15-35 (seed 0 -> 0x6D2B79F5; f64 mapping). */
void orc_xorshift_a_f32(uint32_t seed, float* out, size_t n);
/* engine-cuda/tests/paged_kv_parity.rs:19-35 (24-bit mapping) and
 * generate_rows (paged_kv_parity.rs:52-63): keys/values interleaved per element. */
void orc_generate_rows_b(uint32_t seed, size_t n_tokens, size_t row_len, float* keys,
                         float* values);
/* engine-cuda/tests/common/mod.rs:96-131 (fill_pool_paged). */
void orc_fill_pool_paged(float* pool, const uint32_t* block_table, size_t block_tokens,
                         size_t n_head_kv, size_t head_dim, uint32_t seed, size_t n_tokens);

/* ---------------- CowBlockTable (engine-kvcache/src/cow.rs) ---------------- */
typedef struct orc_cow orc_cow;
orc_cow* orc_cow_new(void);                                  /* cow.rs:33-38 */
orc_cow* orc_cow_fork(const orc_cow* t);                     /* cow.rs:40-45 */
void orc_cow_destroy(orc_cow* t);                            /* drop: releases every Arc */
void orc_cow_append_block(orc_cow* t, uint32_t id);          /* cow.rs:48-53 */
int orc_cow_is_shared(const orc_cow* t, size_t idx);         /* cow.rs:56-61 */
int orc_cow_tail_needs_cow(const orc_cow* t);                /* cow.rs:64-70 */
void orc_cow_perform_tail_cow(orc_cow* t, uint32_t new_id);  /* cow.rs:73-81 */
size_t orc_cow_ids(const orc_cow* t, uint32_t* out, size_t cap); /* cow.rs:84-86 */
size_t orc_cow_len(const orc_cow* t);                        /* cow.rs:89-91 */
int orc_cow_is_dirty(const orc_cow* t, size_t idx);          /* SharedBlock::is_dirty, cow.rs:13-14 */
size_t orc_cow_refcount(const orc_cow* t, size_t idx);       /* Arc::strong_count */
size_t orc_cow_seq_len(const orc_cow* t);                    /* pub seq_len, cow.rs:21 */
void orc_cow_set_seq_len(orc_cow* t, size_t v);

/* ---------------- RadixTree (engine-kvcache/src/radix.rs) ---------------- */
/* Instant::now() is replaced by a logical clock that returns a strictly
 * increasing stamp at each call site the reference calls it (node creation,
 * match_prefix refresh), which reproduces the LRU policy deterministically. */
typedef struct orc_radix orc_radix;
orc_radix* orc_radix_new(size_t block_tokens);               /* radix.rs:64-70 */
void orc_radix_destroy(orc_radix* t);
/* radix.rs:73-117.  Returns matched token count; blocks written to out
 * (count in *n_blocks, at most cap stored). */
size_t orc_radix_match_prefix(orc_radix* t, const uint32_t* tokens, size_t n, uint32_t* out,
                              size_t cap, size_t* n_blocks);
/* radix.rs:120-204 */
void orc_radix_insert(orc_radix* t, const uint32_t* tokens, size_t n, const uint32_t* blocks,
                      size_t nb, int is_pinned);
/* radix.rs:208-254 */
size_t orc_radix_evict_lru(orc_radix* t, size_t target, uint32_t* out, size_t cap);
size_t orc_radix_total_cached_blocks(const orc_radix* t);    /* radix.rs:257-266 */
void orc_radix_invalidate_physical_blocks(orc_radix* t, const uint32_t* blocks, size_t n); /* radix.rs:269-289 */
/* pub ref_count (radix.rs:24): set it on the node whose edge ends exactly
 * after the token path `tokens`.  Returns 0 when found, -1 otherwise. */
int orc_radix_set_ref_count(orc_radix* t, const uint32_t* tokens, size_t n, size_t ref_count);

/* ---------------- StreamingKvManager (engine-kvcache/src/streaming.rs) ---------------- */
typedef struct {
    size_t sink_tokens, recent_window_tokens, max_budget_tokens, block_tokens;
} orc_stream_cfg;
orc_stream_cfg orc_stream_cfg_new(size_t sink, size_t recent, size_t budget, size_t bt); /* streaming.rs:31-49 */
orc_stream_cfg orc_stream_cfg_default(void);                /* streaming.rs:21-29 */
size_t orc_stream_sink_blocks(orc_stream_cfg c);            /* streaming.rs:52-54 */
size_t orc_stream_recent_blocks(orc_stream_cfg c);          /* streaming.rs:57-59 */
size_t orc_stream_max_active_blocks(orc_stream_cfg c);      /* streaming.rs:62-64 */
typedef struct orc_stream orc_stream;
orc_stream* orc_stream_new(orc_stream_cfg c);               /* streaming.rs:75-81 */
void orc_stream_destroy(orc_stream* m);
void orc_stream_record_attention_mass(orc_stream* m, uint32_t block, float mass); /* streaming.rs:135-141 */
size_t orc_stream_scores_len(const orc_stream* m);
/* streaming.rs:87-131.  retained/evicted must hold n entries each. */
void orc_stream_prune_blocks(const orc_stream* m, const uint32_t* table, size_t n,
                             uint32_t* retained, size_t* n_retained, uint32_t* evicted,
                             size_t* n_evicted);

/* sdpa_decode over the protected-sinks range [0, sink) U [max(sink, n-1-W), n-1]
 * (openspec/changes/archive/2026-08-28-agent-runtime-optimizations/design.md:211-216);
 * window 0 attends every token.  mass (optional, indexed by physical page):
 * += the softmax weights of the page's tokens summed over q heads -- the
 * attention mass StreamingKvManager::record_attention_mass adds
 * (streaming.rs:135-141). */
void orc_sdpa_decode_window_batched(const float* pool, const uint32_t* bt, size_t bt_stride,
                                    const uint32_t* lens, size_t batch, size_t block_tokens,
                                    const float* q, size_t n_head, size_t n_head_kv,
                                    size_t head_dim, size_t sink, size_t window, float* out,
                                    double* mass);

/* FP8 E4M3 (OCP E4M3FN) KV storage with per-head f32 scales: the format of
 * openspec/archive/2026-08-28-fp8-kv-cache-quantization/design.md:3-6. */
float orc_e4m3_to_f32(uint8_t code);
uint8_t orc_f32_to_e4m3(float x, float scale);
void orc_e4m3_to_f32_array(const uint8_t* in, float* out, size_t n, float scale);
void orc_f32_to_e4m3_array(const float* in, uint8_t* out, size_t n, float scale);

#ifdef __cplusplus
}
#endif
#endif
