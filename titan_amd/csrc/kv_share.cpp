// kv_share.cpp -- prefix-sharing bookkeeping: CoW block tables, the token
// radix tree with LRU eviction, and the streaming heavy-hitter pruner.
//
// Semantics follow engine-kvcache/src/{cow,radix,streaming}.rs; the data
// structures are this library's own:
//   * a CoW entry is an intrusive, atomically counted block record; a table
//     is a vector of record pointers, so fork is a pointer copy plus one
//     increment per entry and strong counts are exact without any GC;
//   * radix children are kept in a vector sorted by first token (the
//     reference's BTreeMap order), searched by binary search; access times
//     are ticks of a per-tree logical clock;
//   * prune ranks only the middle of the table, with a stable descending
//     order so ties are reproducible.

#include "../../include/kv_share.h"

#include <algorithm>
#include <atomic>
#include <cstring>
#include <limits>
#include <memory>
#include <unordered_set>
#include <vector>

// ============================== CoW tables ==============================

namespace {
struct shared_block {
    uint32_t id;
    bool dirty;
    std::atomic<uint64_t> refs;
};

shared_block* block_new(uint32_t id, bool dirty) {
    auto* b = new shared_block;
    b->id = id;
    b->dirty = dirty;
    b->refs.store(1, std::memory_order_relaxed);
    return b;
}
void block_acquire(shared_block* b) { b->refs.fetch_add(1, std::memory_order_relaxed); }
void block_release(shared_block* b) {
    if (b->refs.fetch_sub(1, std::memory_order_acq_rel) == 1) delete b;
}
}  // namespace

struct eh_cow {
    std::vector<shared_block*> blocks;
    uint64_t seq_len = 0;
};

extern "C" {

eh_cow* eh_cow_new(void) { return new eh_cow(); }

eh_cow* eh_cow_fork(const eh_cow* t) {
    auto* f = new eh_cow();
    f->blocks = t->blocks;
    for (shared_block* b : f->blocks) block_acquire(b);
    f->seq_len = t->seq_len;
    return f;
}

void eh_cow_destroy(eh_cow* t) {
    if (!t) return;
    for (shared_block* b : t->blocks) block_release(b);
    delete t;
}

void eh_cow_append_block(eh_cow* t, uint32_t id) { t->blocks.push_back(block_new(id, false)); }

int eh_cow_is_shared(const eh_cow* t, uint64_t i) {
    return i < t->blocks.size() && t->blocks[i]->refs.load(std::memory_order_acquire) > 1;
}

int eh_cow_tail_needs_cow(const eh_cow* t) {
    // cow.rs:64-70: the tail's strong count alone decides (not its fill level).
    return !t->blocks.empty() && t->blocks.back()->refs.load(std::memory_order_acquire) > 1;
}

void eh_cow_perform_tail_cow(eh_cow* t, uint32_t new_id) {
    if (t->blocks.empty()) return;
    shared_block* old = t->blocks.back();
    t->blocks.back() = block_new(new_id, true);
    block_release(old);
}

uint64_t eh_cow_block_ids(const eh_cow* t, uint32_t* out, uint64_t cap) {
    const uint64_t n = t->blocks.size();
    for (uint64_t i = 0; i < n && i < cap; ++i) out[i] = t->blocks[i]->id;
    return n;
}

uint64_t eh_cow_len(const eh_cow* t) { return t->blocks.size(); }

int eh_cow_is_dirty(const eh_cow* t, uint64_t i) {
    return i < t->blocks.size() && t->blocks[i]->dirty;
}

uint64_t eh_cow_ref_count(const eh_cow* t, uint64_t i) {
    return i < t->blocks.size() ? t->blocks[i]->refs.load(std::memory_order_acquire) : 0;
}

uint64_t eh_cow_seq_len(const eh_cow* t) { return t->seq_len; }
void eh_cow_set_seq_len(eh_cow* t, uint64_t v) { t->seq_len = v; }

}  // extern "C"

// ============================== radix tree ==============================

namespace {
struct rx_node {
    std::vector<uint32_t> tokens;
    std::vector<uint32_t> blocks;
    std::vector<std::pair<uint32_t, std::unique_ptr<rx_node>>> kids;  // sorted by first token
    uint64_t stamp = 0;
    bool pinned = false;
    uint64_t ref_count = 0;

    long find(uint32_t tok) const {
        auto it = std::lower_bound(kids.begin(), kids.end(), tok,
                                   [](const auto& kv, uint32_t t) { return kv.first < t; });
        return (it != kids.end() && it->first == tok) ? (long)(it - kids.begin()) : -1;
    }
    void put(uint32_t tok, std::unique_ptr<rx_node> n) {
        auto it = std::lower_bound(kids.begin(), kids.end(), tok,
                                   [](const auto& kv, uint32_t t) { return kv.first < t; });
        kids.emplace(it, tok, std::move(n));
    }
};

uint64_t common_prefix(const uint32_t* a, uint64_t na, const std::vector<uint32_t>& b) {
    const uint64_t m = std::min<uint64_t>(na, b.size());
    uint64_t i = 0;
    while (i < m && a[i] == b[i]) ++i;
    return i;
}
}  // namespace

struct eh_radix {
    std::unique_ptr<rx_node> root;
    uint64_t block_tokens;
    uint64_t clock = 0;
    uint64_t tick() { return ++clock; }
    std::unique_ptr<rx_node> make(const uint32_t* tok, uint64_t nt, const uint32_t* blk, uint64_t nb,
                                  bool pinned) {
        auto n = std::make_unique<rx_node>();
        n->tokens.assign(tok, tok + nt);
        n->blocks.assign(blk, blk + nb);
        n->pinned = pinned;
        n->stamp = tick();
        return n;
    }
};

namespace {
// radix.rs:224-254: the oldest eligible leaf among the direct children of the
// first node (depth-first, key order) that has one; strict < keeps the
// smallest key on ties.
bool take_oldest_leaf(rx_node* cur, std::vector<uint32_t>& freed) {
    long best = -1;
    for (size_t i = 0; i < cur->kids.size(); ++i) {
        const rx_node* c = cur->kids[i].second.get();
        if (!c->pinned && c->ref_count == 0 && c->kids.empty() &&
            (best < 0 || c->stamp < cur->kids[(size_t)best].second->stamp))
            best = (long)i;
    }
    if (best >= 0) {
        rx_node* c = cur->kids[(size_t)best].second.get();
        freed.insert(freed.end(), c->blocks.begin(), c->blocks.end());
        cur->kids.erase(cur->kids.begin() + best);
        return true;
    }
    for (auto& kv : cur->kids)
        if (take_oldest_leaf(kv.second.get(), freed)) return true;
    return false;
}

uint64_t count_blocks(const rx_node* n) {
    uint64_t s = n->blocks.size();
    for (const auto& kv : n->kids) s += count_blocks(kv.second.get());
    return s;
}

void prune(rx_node* n, const std::unordered_set<uint32_t>& gone) {
    // radix.rs:277-289: drop every child holding a freed block (with its
    // subtree), then recurse into the survivors.
    n->kids.erase(std::remove_if(n->kids.begin(), n->kids.end(),
                                 [&](const auto& kv) {
                                     for (uint32_t b : kv.second->blocks)
                                         if (gone.count(b)) return true;
                                     return false;
                                 }),
                  n->kids.end());
    for (auto& kv : n->kids) prune(kv.second.get(), gone);
}
}  // namespace

extern "C" {

eh_radix* eh_radix_new(uint64_t block_tokens) {
    if (block_tokens == 0) return nullptr;  // the reference divides by it
    auto* t = new eh_radix();
    t->block_tokens = block_tokens;
    t->root = t->make(nullptr, 0, nullptr, 0, true);  // radix.rs:64-69: pinned empty root
    return t;
}

void eh_radix_destroy(eh_radix* t) { delete t; }

uint64_t eh_radix_match_prefix(eh_radix* t, const uint32_t* tokens, uint64_t n, uint32_t* out,
                               uint64_t cap, uint64_t* n_blocks) {
    uint64_t matched = 0, nb = 0;
    auto emit = [&](const std::vector<uint32_t>& b, uint64_t count) {
        for (uint64_t i = 0; i < count; ++i, ++nb)
            if (nb < cap) out[nb] = b[i];
    };
    rx_node* cur = t->root.get();
    cur->stamp = t->tick();
    while (n > 0) {
        const long k = cur->find(tokens[0]);
        if (k < 0) break;
        rx_node* child = cur->kids[(size_t)k].second.get();
        child->stamp = t->tick();
        const uint64_t common = common_prefix(tokens, n, child->tokens);
        matched += common;
        if (common == child->tokens.size()) {
            emit(child->blocks, child->blocks.size());
            tokens += common;
            n -= common;
            cur = child;
        } else {
            // partial edge: whole blocks of the common part (radix.rs:100-105)
            emit(child->blocks, std::min<uint64_t>(common / t->block_tokens, child->blocks.size()));
            break;
        }
    }
    if (n_blocks) *n_blocks = nb;
    return matched;
}

void eh_radix_insert(eh_radix* t, const uint32_t* tokens, uint64_t n, const uint32_t* blocks,
                     uint64_t nb, int is_pinned) {
    if (n == 0) return;
    rx_node* cur = t->root.get();
    while (n > 0) {
        const long k = cur->find(tokens[0]);
        if (k < 0) {
            cur->put(tokens[0], t->make(tokens, n, blocks, nb, is_pinned != 0));
            return;
        }
        std::unique_ptr<rx_node>& slot = cur->kids[(size_t)k].second;
        const uint64_t common = common_prefix(tokens, n, slot->tokens);
        if (common == slot->tokens.size()) {
            // whole edge matched: skip its blocks (if the caller supplied them)
            const uint64_t used = slot->blocks.size();
            blocks = nb >= used ? blocks + used : blocks;
            nb = nb >= used ? nb - used : 0;
            tokens += common;
            n -= common;
            cur = slot.get();
            continue;
        }
        // split the edge at `common` (radix.rs:163-201)
        std::unique_ptr<rx_node> old = std::move(slot);
        const uint64_t split_blocks = std::min<uint64_t>(common / t->block_tokens, old->blocks.size());
        std::unique_ptr<rx_node> mid = t->make(old->tokens.data(), common, old->blocks.data(),
                                               split_blocks, is_pinned != 0);
        old->tokens.erase(old->tokens.begin(), old->tokens.begin() + common);
        old->blocks.erase(old->blocks.begin(), old->blocks.begin() + split_blocks);
        const uint32_t old_first = old->tokens[0];
        mid->put(old_first, std::move(old));
        if (common < n) {
            const uint32_t* rb = nb >= split_blocks ? blocks + split_blocks : blocks;
            const uint64_t rn = nb >= split_blocks ? nb - split_blocks : 0;
            mid->put(tokens[common], t->make(tokens + common, n - common, rb, rn, is_pinned != 0));
        }
        slot = std::move(mid);
        return;
    }
}

uint64_t eh_radix_evict_lru(eh_radix* t, uint64_t target, uint32_t* out, uint64_t cap) {
    std::vector<uint32_t> freed;
    while (freed.size() < target)
        if (!take_oldest_leaf(t->root.get(), freed)) break;
    for (uint64_t i = 0; i < freed.size() && i < cap; ++i) out[i] = freed[i];
    return freed.size();
}

uint64_t eh_radix_total_cached_blocks(const eh_radix* t) { return count_blocks(t->root.get()); }

void eh_radix_invalidate_physical_blocks(eh_radix* t, const uint32_t* blocks, uint64_t n) {
    if (n == 0) return;
    std::unordered_set<uint32_t> gone(blocks, blocks + n);
    prune(t->root.get(), gone);
}

eh_status eh_radix_set_ref_count(eh_radix* t, const uint32_t* tokens, uint64_t n, uint64_t rc) {
    rx_node* cur = t->root.get();
    while (n > 0) {
        const long k = cur->find(tokens[0]);
        if (k < 0) return EH_INVALID_ARGS;
        rx_node* c = cur->kids[(size_t)k].second.get();
        if (c->tokens.size() > n || common_prefix(tokens, n, c->tokens) != c->tokens.size())
            return EH_INVALID_ARGS;
        tokens += c->tokens.size();
        n -= c->tokens.size();
        cur = c;
    }
    cur->ref_count = rc;
    return EH_OK;
}

}  // extern "C"

// ============================== streaming ==============================

struct eh_stream_mgr {
    eh_stream_cfg cfg;
    std::vector<float> scores;
};

namespace {
uint64_t ceil_div(uint64_t a, uint64_t b) { return (a + b - 1) / b; }
}  // namespace

extern "C" {

eh_stream_cfg eh_stream_cfg_new(uint64_t sink, uint64_t recent, uint64_t budget, uint64_t bt) {
    // streaming.rs:38-41, in this order.
    eh_stream_cfg c;
    c.block_tokens = std::max<uint64_t>(bt, 1);
    c.sink_tokens = std::max<uint64_t>(sink, 1);
    c.recent_window_tokens = std::max<uint64_t>(recent, c.block_tokens);
    c.max_budget_tokens = std::max<uint64_t>(budget, c.sink_tokens + c.recent_window_tokens);
    return c;
}

eh_stream_cfg eh_stream_cfg_default(void) {
    eh_stream_cfg c;  // streaming.rs:21-29 (no clamping on this path)
    c.sink_tokens = 4;
    c.recent_window_tokens = 256;
    c.max_budget_tokens = 512;
    c.block_tokens = 16;
    return c;
}

uint64_t eh_stream_sink_blocks(eh_stream_cfg c) { return ceil_div(c.sink_tokens, c.block_tokens); }
uint64_t eh_stream_recent_blocks(eh_stream_cfg c) {
    return ceil_div(c.recent_window_tokens, c.block_tokens);
}
uint64_t eh_stream_max_active_blocks(eh_stream_cfg c) {
    return ceil_div(c.max_budget_tokens, c.block_tokens);
}

eh_stream_mgr* eh_stream_new(eh_stream_cfg c) {
    auto* m = new eh_stream_mgr();
    m->cfg = c;
    m->scores.assign(eh_stream_max_active_blocks(c) * 4, 0.0f);  // streaming.rs:76
    return m;
}

void eh_stream_destroy(eh_stream_mgr* m) { delete m; }

void eh_stream_record_attention_mass(eh_stream_mgr* m, uint32_t block, float mass) {
    if (block >= m->scores.size()) m->scores.resize((size_t)block + 64, 0.0f);  // :137-139
    m->scores[block] += mass;
}

// record_attention_mass(i, masses[i]) for every i < n with a non-zero mass:
// the per-page masses a decode launch accumulated (eh_paged_decode_batched_window's
// block_mass, copied to the host) in one call.
void eh_stream_record_attention_masses(eh_stream_mgr* m, const float* masses, uint64_t n) {
    for (uint64_t i = 0; i < n; ++i)
        if (masses[i] != 0.0f) eh_stream_record_attention_mass(m, (uint32_t)i, masses[i]);
}

uint64_t eh_stream_scores_len(const eh_stream_mgr* m) { return m->scores.size(); }

float eh_stream_score(const eh_stream_mgr* m, uint32_t block) {
    return block < m->scores.size() ? m->scores[block] : 0.0f;
}

void eh_stream_prune_blocks(const eh_stream_mgr* m, const uint32_t* table, uint64_t n,
                            uint32_t* retained, uint64_t* n_retained, uint32_t* evicted,
                            uint64_t* n_evicted) {
    const uint64_t max_blocks = eh_stream_max_active_blocks(m->cfg);
    if (n <= max_blocks) {
        std::memcpy(retained, table, n * sizeof(uint32_t));
        *n_retained = n;
        *n_evicted = 0;
        return;
    }
    const uint64_t sink = std::min(eh_stream_sink_blocks(m->cfg), n);
    const uint64_t recent = std::min(eh_stream_recent_blocks(m->cfg), n - sink);
    const uint64_t mid0 = sink, mid1 = n - recent;
    const uint64_t keep = max_blocks > sink + recent ? max_blocks - (sink + recent) : 0;
    // middle positions ordered by descending score (NaN ranks last, which
    // keeps the order a strict weak ordering)
    std::vector<uint64_t> order;
    order.reserve(mid1 - mid0);
    for (uint64_t i = mid0; i < mid1; ++i) order.push_back(i);
    auto key = [&](uint64_t i) {
        const float s = eh_stream_score(m, table[i]);
        return s != s ? -std::numeric_limits<float>::infinity() : s;
    };
    std::stable_sort(order.begin(), order.end(),
                     [&](uint64_t a, uint64_t b) { return key(a) > key(b); });
    uint64_t r = 0, e = 0;
    for (uint64_t i = 0; i < sink; ++i) retained[r++] = table[i];
    for (uint64_t k = 0; k < order.size(); ++k) {
        if (k < keep) retained[r++] = table[order[k]];
        else evicted[e++] = table[order[k]];
    }
    for (uint64_t i = mid1; i < n; ++i) retained[r++] = table[i];
    *n_retained = r;
    *n_evicted = e;
}

}  // extern "C"

// ============================== compaction ==============================

extern "C" int64_t eh_compaction_plan(const uint32_t* bt, uint64_t stride, const uint32_t* n_used,
                                      uint64_t batch, uint32_t n_blocks, uint32_t* src,
                                      uint32_t* dst, uint32_t* remap) {
    std::vector<uint8_t> live(n_blocks, 0);
    for (uint64_t b = 0; b < batch; ++b)
        for (uint64_t j = 0; j < n_used[b] && j < stride; ++j) {
            const uint32_t p = bt[b * stride + j];
            if (p >= n_blocks) return -1;
            live[p] = 1;
        }
    uint64_t k = 0;
    for (uint32_t p = 0; p < n_blocks; ++p) k += live[p];
    for (uint32_t p = 0; p < n_blocks; ++p) remap[p] = p;
    int64_t pairs = 0;
    uint32_t hole = 0;
    for (uint32_t p = (uint32_t)k; p < n_blocks; ++p) {
        if (!live[p]) continue;
        while (live[hole]) ++hole;  // a hole below k exists for every live page above k
        src[pairs] = p;
        dst[pairs] = hole;
        remap[p] = hole;
        live[hole] = 1;
        ++pairs;
    }
    return pairs;
}
