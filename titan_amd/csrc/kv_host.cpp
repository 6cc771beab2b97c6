// kv_host.cpp -- host-side page bookkeeping of the paged KV pool.
//
// Integer bookkeeping stays on the host exactly as in the reference
// (engine-kvcache/src/cache.rs): an O(1) stack free list, per-sequence block
// tables and token counts.  Page bytes live in HBM and are written by the
// HIP kernels (eh_append_kv*); this file never touches pool memory.

#include "../../include/engine_hip.h"
#include "../../include/kv_host.h"

#include <cstring>
#include <vector>

struct eh_kvcache {
    uint64_t n_blocks, block_tokens, heads, head_dim;
    uint32_t dtype;
    std::vector<uint32_t> free_list;               // pop from the back
    std::vector<std::vector<uint32_t>> tables;     // sequence -> physical pages
    std::vector<uint64_t> tokens;                  // sequence -> appended tokens
};

namespace {
thread_local const char* g_msg = "";
thread_local uint64_t g_used = 0, g_total = 0;

eh_status invalid(const char* msg) {
    g_msg = msg;
    return EH_INVALID_ARGS;
}
}  // namespace

extern "C" {

const char* eh_kvcache_last_message(void) { return g_msg; }

eh_status eh_kvcache_last_exhausted(uint64_t* blocks_used, uint64_t* blocks_total) {
    if (blocks_used) *blocks_used = g_used;
    if (blocks_total) *blocks_total = g_total;
    return EH_OK;
}

eh_status eh_kvcache_new(uint64_t n_blocks, uint64_t block_tokens, uint64_t heads,
                         uint64_t head_dim, uint32_t dtype, eh_kvcache** out) {
    // cache.rs:65-76: same checks, same order, same messages.
    if (!out) return invalid("out is null");
    *out = nullptr;
    if (n_blocks == 0) return invalid("n_blocks must be non-zero");
    if (block_tokens == 0) return invalid("block_tokens must be non-zero");
    if (heads == 0 || head_dim == 0) return invalid("heads and head_dim must be non-zero");
    if (eh_kv_element_bytes(dtype) == 0) return invalid("unknown data type");
    if (n_blocks > 0xFFFFFFFFull) return invalid("n_blocks exceeds u32 page ids");
    auto* c = new eh_kvcache();
    c->n_blocks = n_blocks;
    c->block_tokens = block_tokens;
    c->heads = heads;
    c->head_dim = head_dim;
    c->dtype = dtype;
    // cache.rs:81-86: ids stored descending so the first pop returns page 0.
    c->free_list.resize(n_blocks);
    for (uint64_t i = 0; i < n_blocks; ++i) c->free_list[i] = (uint32_t)(n_blocks - 1 - i);
    *out = c;
    return EH_OK;
}

void eh_kvcache_destroy(eh_kvcache* c) { delete c; }

eh_status eh_kvcache_seed_free_list(eh_kvcache* c, const uint32_t* order, uint64_t n) {
    // Extension: successive pops return order[0], order[1], ...  The order
    // must be a permutation of the pages that are free now (all of them
    // while no page is in use): a duplicate or a page some sequence holds
    // would hand one physical page to two owners.
    if (!c) return invalid("cache is null");
    if (n != c->free_list.size()) return invalid("order must list every free page exactly once");
    if (n && !order) return invalid("order is null");
    std::vector<uint8_t> is_free(c->n_blocks, 0), seen(c->n_blocks, 0);
    for (uint32_t p : c->free_list) is_free[p] = 1;
    for (uint64_t i = 0; i < n; ++i) {
        const uint32_t p = order[i];
        if (p >= c->n_blocks) return invalid("page id out of range");
        if (seen[p]) return invalid("duplicate page id");
        if (!is_free[p]) return invalid("page is in use");
        seen[p] = 1;
    }
    c->free_list.assign(order, order + n);
    std::vector<uint32_t> rev(c->free_list.rbegin(), c->free_list.rend());
    c->free_list.swap(rev);
    return EH_OK;
}

uint64_t eh_kvcache_blocks_total(const eh_kvcache* c) { return c->n_blocks; }
uint64_t eh_kvcache_blocks_used(const eh_kvcache* c) { return c->n_blocks - c->free_list.size(); }
uint64_t eh_kvcache_sequences(const eh_kvcache* c) { return c->tables.size(); }

uint64_t eh_kvcache_new_sequence(eh_kvcache* c) {
    // cache.rs:135-141: dense ids.
    c->tables.emplace_back();
    c->tokens.push_back(0);
    return c->tables.size() - 1;
}

void eh_kvcache_free_sequence(eh_kvcache* c, uint64_t seq) {
    // cache.rs:123-132: pages return in reverse so the next pops reuse them in
    // their original order; count resets; the sequence stays registered.
    if (seq >= c->tables.size()) return;
    auto& t = c->tables[seq];
    for (auto it = t.rbegin(); it != t.rend(); ++it) c->free_list.push_back(*it);
    t.clear();
    c->tokens[seq] = 0;
}

uint64_t eh_kvcache_token_count(const eh_kvcache* c, uint64_t seq) {
    return seq < c->tokens.size() ? c->tokens[seq] : 0;
}

int64_t eh_kvcache_block_table(const eh_kvcache* c, uint64_t seq, uint32_t* out, uint64_t cap) {
    if (seq >= c->tables.size()) return -1;
    const auto& t = c->tables[seq];
    for (uint64_t i = 0; i < t.size() && i < cap; ++i) out[i] = t[i];
    return (int64_t)t.size();
}

// Pages sequence `seq` holds after n_tokens more tokens, in 128 bits so that
// an absurd n_tokens cannot wrap around to a small count.
static unsigned __int128 pages_after(const eh_kvcache* c, uint64_t seq, uint64_t n_tokens) {
    const unsigned __int128 bt = c->block_tokens;
    return ((unsigned __int128)c->tokens[seq] + n_tokens + bt - 1) / bt;
}

eh_status eh_kvcache_reserve(eh_kvcache* c, uint64_t seq, uint64_t n_tokens, uint64_t* start_pos) {
    // The bookkeeping half of cache.rs:153-192 for n tokens: a fresh page is
    // popped whenever the position crosses a page boundary.  All or nothing:
    // on exhaustion nothing changes (for n = 1 this is the reference's rule).
    if (seq >= c->tables.size()) return invalid("unknown sequence id");
    const uint64_t pos = c->tokens[seq];
    const uint64_t have = c->tables[seq].size();
    const unsigned __int128 need = pages_after(c, seq, n_tokens);
    const unsigned __int128 fresh = need > have ? need - have : 0;
    if (fresh > c->free_list.size()) {
        g_used = eh_kvcache_blocks_used(c);
        g_total = c->n_blocks;
        g_msg = "pool exhausted";
        return EH_POOL_EXHAUSTED;
    }
    for (uint64_t i = 0; i < fresh; ++i) {
        c->tables[seq].push_back(c->free_list.back());
        c->free_list.pop_back();
    }
    if (start_pos) *start_pos = pos;
    c->tokens[seq] = pos + n_tokens;
    return EH_OK;
}

eh_status eh_kvcache_reserve_batch(eh_kvcache* c, const uint64_t* seqs, uint64_t n_seqs,
                                   const uint64_t* n_tokens, uint64_t* start_pos) {
    // eh_kvcache_reserve of n_tokens[i] for every listed sequence, all or
    // nothing: the pages the whole batch needs are counted first; on
    // PoolExhausted (or an unknown / repeated sequence) no count and no table
    // changes.  Pages are popped in list order, as repeated single reserves
    // would pop them.
    if (!c) return invalid("cache is null");
    if (n_seqs && (!seqs || !n_tokens)) return invalid("seqs / n_tokens is null");
    unsigned __int128 fresh = 0;  // clamped at free + 1: exhausted either way
    std::vector<uint8_t> seen(c->tables.size(), 0);
    for (uint64_t i = 0; i < n_seqs; ++i) {
        const uint64_t s = seqs[i];
        if (s >= c->tables.size()) return invalid("unknown sequence id");
        if (seen[s]) return invalid("sequence listed twice");
        seen[s] = 1;
        const unsigned __int128 need = pages_after(c, s, n_tokens[i]);
        const uint64_t have = c->tables[s].size();
        const unsigned __int128 add = need > have ? need - have : 0;
        fresh += add;
        if (fresh > c->free_list.size()) fresh = (unsigned __int128)c->free_list.size() + 1;
    }
    if (fresh > c->free_list.size()) {
        g_used = eh_kvcache_blocks_used(c);
        g_total = c->n_blocks;
        g_msg = "pool exhausted";
        return EH_POOL_EXHAUSTED;
    }
    for (uint64_t i = 0; i < n_seqs; ++i) {
        const eh_status st = eh_kvcache_reserve(c, seqs[i], n_tokens[i], start_pos ? start_pos + i : nullptr);
        if (st != EH_OK) return st;  // cannot happen: checked above
    }
    return EH_OK;
}

eh_status eh_kvcache_truncate(eh_kvcache* c, uint64_t seq, uint64_t n_tokens) {
    // Undo of eh_kvcache_reserve: the count drops to n_tokens and the pages
    // past ceil(n_tokens / block_tokens) go back on the free list in reverse,
    // so the free list is again what it was before they were popped (the
    // return order of cache.rs:131).  Page bytes are left as they are.
    if (!c) return invalid("cache is null");
    if (seq >= c->tables.size()) return invalid("unknown sequence id");
    if (n_tokens > c->tokens[seq]) return invalid("truncate past the token count");
    auto& t = c->tables[seq];
    const uint64_t keep = (n_tokens + c->block_tokens - 1) / c->block_tokens;
    while (t.size() > keep) {
        c->free_list.push_back(t.back());
        t.pop_back();
    }
    c->tokens[seq] = n_tokens;
    return EH_OK;
}

eh_status eh_kvcache_export_tables(const eh_kvcache* c, const uint64_t* seqs, uint64_t n_seqs,
                                   uint32_t* out, uint64_t stride, uint32_t* lens) {
    // Dense [n_seqs, stride] table for the batched kernels; unused entries
    // hold 0xFFFFFFFF, which the kernels treat as "no page".
    for (uint64_t i = 0; i < n_seqs; ++i) {
        const uint64_t s = seqs[i];
        if (s >= c->tables.size()) return invalid("unknown sequence id");
        const auto& t = c->tables[s];
        if (t.size() > stride) return invalid("stride shorter than a block table");
        uint32_t* row = out + i * stride;
        std::memcpy(row, t.data(), t.size() * sizeof(uint32_t));
        for (uint64_t j = t.size(); j < stride; ++j) row[j] = 0xFFFFFFFFu;
        if (lens) lens[i] = (uint32_t)c->tokens[s];
    }
    return EH_OK;
}

}  // extern "C"
