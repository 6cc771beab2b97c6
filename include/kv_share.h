/*
 * kv_share.h -- C-ABI of the prefix-sharing bookkeeping beside the paged pool:
 * copy-on-write block tables, the token radix tree (prefix cache with LRU
 * eviction) and the streaming (sink + heavy-hitter + recent window) pruner.
 *
 * Mirrors engine_kvcache::{CowBlockTable, RadixTree, StreamingKvManager}
 * (engine-kvcache/src/{cow,radix,streaming}.rs).  These objects hold only
 * integers (page ids, tokens, scores); the page bytes they refer to live in
 * HBM and are moved by eh_copy_pages / eh_remap_block_tables (engine_hip.h).
 * Objects are not internally synchronised (the reference mutates them through
 * &mut self); the shared-block reference counts are atomic, so tables forked
 * from one another may be used and dropped on different threads.
 */
#ifndef TITAN_KV_SHARE_H
#define TITAN_KV_SHARE_H

#include <stddef.h>
#include <stdint.h>

#include "engine_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ---- CowBlockTable (cow.rs:17-97).  Each entry is a reference-counted
 * shared block {id, is_dirty}; fork shares every entry (O(n) pointer copies,
 * no page copy). */
typedef struct eh_cow eh_cow;
eh_cow* eh_cow_new(void);                                     /* cow.rs:33-38 */
eh_cow* eh_cow_fork(const eh_cow* t);                         /* cow.rs:40-45 */
void eh_cow_destroy(eh_cow* t);                               /* Drop: releases every entry */
void eh_cow_append_block(eh_cow* t, uint32_t block_id);       /* cow.rs:48-53 */
int eh_cow_is_shared(const eh_cow* t, uint64_t block_index);  /* cow.rs:56-61 */
int eh_cow_tail_needs_cow(const eh_cow* t);                   /* cow.rs:64-70 */
void eh_cow_perform_tail_cow(eh_cow* t, uint32_t new_block_id); /* cow.rs:73-81 */
/* physical_block_ids (cow.rs:84-86): writes min(len, cap) ids, returns len. */
uint64_t eh_cow_block_ids(const eh_cow* t, uint32_t* out, uint64_t cap);
uint64_t eh_cow_len(const eh_cow* t);                         /* cow.rs:89-91 */
int eh_cow_is_dirty(const eh_cow* t, uint64_t block_index);   /* SharedBlock::is_dirty */
uint64_t eh_cow_ref_count(const eh_cow* t, uint64_t block_index); /* Arc::strong_count; 0 past the end */
uint64_t eh_cow_seq_len(const eh_cow* t);                     /* pub seq_len (cow.rs:21) */
void eh_cow_set_seq_len(eh_cow* t, uint64_t seq_len);

/* ---- RadixTree (radix.rs:57-290).  Access times come from a per-tree
 * logical clock (one tick per node creation or match refresh) instead of
 * Instant::now(), so eviction order is reproducible; with distinct clock
 * values the policy is the reference's. */
typedef struct eh_radix eh_radix;
eh_radix* eh_radix_new(uint64_t block_tokens);  /* radix.rs:64-69; NULL when block_tokens == 0 */
void eh_radix_destroy(eh_radix* t);
/* match_prefix (radix.rs:73-117): returns matched_tokens; the matched block
 * ids go to out (min(count, cap) written), their count to *n_blocks. */
uint64_t eh_radix_match_prefix(eh_radix* t, const uint32_t* tokens, uint64_t n, uint32_t* out,
                               uint64_t cap, uint64_t* n_blocks);
/* insert (radix.rs:120-204). */
void eh_radix_insert(eh_radix* t, const uint32_t* tokens, uint64_t n, const uint32_t* blocks,
                     uint64_t n_blocks, int is_pinned);
/* evict_lru (radix.rs:208-222): freed ids to out (min(count, cap) written),
 * returns the count. */
uint64_t eh_radix_evict_lru(eh_radix* t, uint64_t target_blocks, uint32_t* out, uint64_t cap);
uint64_t eh_radix_total_cached_blocks(const eh_radix* t);    /* radix.rs:257-266 */
void eh_radix_invalidate_physical_blocks(eh_radix* t, const uint32_t* blocks, uint64_t n); /* radix.rs:269-289 */
/* pub ref_count of the node whose edge path spells exactly `tokens`
 * (radix.rs:25); EH_INVALID_ARGS when no node ends there. */
eh_status eh_radix_set_ref_count(eh_radix* t, const uint32_t* tokens, uint64_t n,
                                 uint64_t ref_count);

/* ---- StreamingKvConfig / StreamingKvManager (streaming.rs:9-142). */
typedef struct eh_stream_cfg {
    uint64_t sink_tokens, recent_window_tokens, max_budget_tokens, block_tokens;
} eh_stream_cfg;
eh_stream_cfg eh_stream_cfg_new(uint64_t sink_tokens, uint64_t recent_window_tokens,
                                uint64_t max_budget_tokens, uint64_t block_tokens); /* :31-49 */
eh_stream_cfg eh_stream_cfg_default(void);                    /* streaming.rs:21-29 */
uint64_t eh_stream_sink_blocks(eh_stream_cfg c);              /* streaming.rs:52-54 */
uint64_t eh_stream_recent_blocks(eh_stream_cfg c);            /* streaming.rs:57-59 */
uint64_t eh_stream_max_active_blocks(eh_stream_cfg c);        /* streaming.rs:62-64 */
typedef struct eh_stream_mgr eh_stream_mgr;
eh_stream_mgr* eh_stream_new(eh_stream_cfg c);                /* streaming.rs:75-81 */
void eh_stream_destroy(eh_stream_mgr* m);
void eh_stream_record_attention_mass(eh_stream_mgr* m, uint32_t block_id, float mass); /* :135-141 */
uint64_t eh_stream_scores_len(const eh_stream_mgr* m);        /* block_scores.len() */
float eh_stream_score(const eh_stream_mgr* m, uint32_t block_id); /* 0 past the end */
/* Bulk form: record_attention_mass(i, masses[i]) for each i < n with
 * masses[i] != 0 -- e.g. the block_mass array a decode launch accumulated
 * (eh_paged_decode_batched_window), copied to the host.  Zero entries are
 * skipped, which the reference's lookups (get(..).unwrap_or(0.0),
 * streaming.rs:106-109) cannot tell from recording them. */
void eh_stream_record_attention_masses(eh_stream_mgr* m, const float* masses, uint64_t n);
/* prune_blocks (streaming.rs:87-132): retained (sink, kept middle by
 * descending score, recent) and evicted ids; both outputs need room for n.
 * Equal scores keep block-table order and NaN scores rank last (the
 * reference's unstable sort leaves both unspecified). */
void eh_stream_prune_blocks(const eh_stream_mgr* m, const uint32_t* table, uint64_t n,
                            uint32_t* retained, uint64_t* n_retained, uint32_t* evicted,
                            uint64_t* n_evicted);

/* ---- Gather-compaction plan (no reference counterpart; the reference
 * frees pages but never moves them).  Live pages are the entries j <
 * n_used[b] of rows b of block_tables [batch, stride].  With K live pages,
 * every live page with id >= K is assigned, in ascending order, the ascending
 * free ids below K; remap [n_blocks] maps every id to its new id (identity
 * elsewhere).  src/dst need room for K pairs; returns the pair count, or -1
 * when a live entry is >= n_blocks.  Feed the pairs to eh_copy_pages and the
 * remap to eh_remap_block_tables. */
int64_t eh_compaction_plan(const uint32_t* block_tables, uint64_t stride, const uint32_t* n_used,
                           uint64_t batch, uint32_t n_blocks, uint32_t* src, uint32_t* dst,
                           uint32_t* remap);

#ifdef __cplusplus
}
#endif
#endif
