/*
 * kv_host.h -- C-ABI of the host-side page bookkeeping (allocator, block
 * tables) that sits beside the gfx950 kernels of engine_hip.h.
 *
 * Mirrors engine_kvcache::PagedKvCache (engine-kvcache/src/cache.rs) with the
 * pool moved to HBM: this object owns only integers; page bytes are written
 * by eh_append_kv / eh_append_kv_batched into a caller-owned device pool.
 * Errors mirror KvCacheError (engine-kvcache/src/error.rs:4-16).
 */
#ifndef TITAN_KV_HOST_H
#define TITAN_KV_HOST_H

#include <stdint.h>

#include "engine_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct eh_kvcache eh_kvcache;

/* PagedKvCache::new (cache.rs:64-95); InvalidArgs messages as in the reference. */
eh_status eh_kvcache_new(uint64_t n_blocks, uint64_t block_tokens, uint64_t heads,
                         uint64_t head_dim, uint32_t dtype, eh_kvcache** out);
void eh_kvcache_destroy(eh_kvcache* c);
/* Message of this thread's last InvalidArgs / PoolExhausted. */
const char* eh_kvcache_last_message(void);
/* PoolExhausted{blocks_used, blocks_total} of this thread's last failure. */
eh_status eh_kvcache_last_exhausted(uint64_t* blocks_used, uint64_t* blocks_total);
/* Extension (no reference counterpart): successive pops return order[0],
 * order[1], ...  `order` must be a permutation of the currently free pages
 * (every page while none is in use); duplicates, pages held by a sequence and
 * a length other than the free count are InvalidArgs, with nothing changed. */
eh_status eh_kvcache_seed_free_list(eh_kvcache* c, const uint32_t* order, uint64_t n);
uint64_t eh_kvcache_blocks_total(const eh_kvcache* c);             /* cache.rs:103-105 */
uint64_t eh_kvcache_blocks_used(const eh_kvcache* c);              /* cache.rs:108-110 */
uint64_t eh_kvcache_sequences(const eh_kvcache* c);                /* cache.rs:113-115 */
uint64_t eh_kvcache_new_sequence(eh_kvcache* c);                   /* cache.rs:135-141 */
void eh_kvcache_free_sequence(eh_kvcache* c, uint64_t seq);        /* cache.rs:123-132 */
uint64_t eh_kvcache_token_count(const eh_kvcache* c, uint64_t seq);/* cache.rs:144-149 */
/* cache.rs:119-121: returns the row length (-1 for an unknown sequence). */
int64_t eh_kvcache_block_table(const eh_kvcache* c, uint64_t seq, uint32_t* out, uint64_t cap);
/* Bookkeeping half of PagedKvCache::append (cache.rs:153-192) for n tokens:
 * pops pages at page boundaries, advances the count, returns the first
 * logical position.  All or nothing on PoolExhausted. */
eh_status eh_kvcache_reserve(eh_kvcache* c, uint64_t seq, uint64_t n_tokens, uint64_t* start_pos);
/* PagedKvCache::append's bookkeeping (cache.rs:153-192) for a batch: reserves
 * n_tokens[i] tokens for seqs[i] (start_pos[i] = its first new position).  All or nothing: the pages the whole batch needs are checked
 * against the free list first, so PoolExhausted, an unknown or a repeated
 * sequence leaves every count and table unchanged (the reference's "no
 * partial state", cache.rs:164-177).  Extension. */
eh_status eh_kvcache_reserve_batch(eh_kvcache* c, const uint64_t* seqs, uint64_t n_seqs,
                                   const uint64_t* n_tokens, uint64_t* start_pos);
/* Rollback of a reservation (extension): the count drops to n_tokens (at most
 * the current count) and pages past ceil(n_tokens / block_tokens) return to
 * the free list in reverse, restoring the pop order they had. */
eh_status eh_kvcache_truncate(eh_kvcache* c, uint64_t seq, uint64_t n_tokens);
/* Dense [n_seqs, stride] block tables (padding 0xFFFFFFFF) and token counts
 * for the batched kernels. */
eh_status eh_kvcache_export_tables(const eh_kvcache* c, const uint64_t* seqs, uint64_t n_seqs,
                                   uint32_t* out, uint64_t stride, uint32_t* lens);

#ifdef __cplusplus
}
#endif
#endif
