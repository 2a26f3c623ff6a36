// Paged KV-cache index: block pool, radix tree over token ids holding flat
// slot ids, and the sequence table that turns them into block tables.  Host
// code only.  The C entry points are declared in include/xllm_hip_kv_index.h
// with the reference interfaces each follows.
#include <algorithm>
#include <cstdint>
#include <cstring>
#include <deque>
#include <memory>
#include <queue>
#include <unordered_map>
#include <vector>

#include "xllm_hip_kv_index.h"

#define XKV_EXPORT extern "C" __attribute__((visibility("default")))

namespace {

// Reference counts and a FIFO free list (memory_manager.c:207-258: alloc
// takes the head of the free list, a page whose count drops to zero is
// appended at the tail).
class BlockPool {
  public:
    explicit BlockPool(int n) : refs_(n, 0) {
        for (int i = 0; i < n; ++i) free_.push_back(i);
    }
    int size() const { return (int)refs_.size(); }
    int free_count() const { return (int)free_.size(); }
    bool valid(int b) const { return b >= 0 && b < size(); }
    int refs(int b) const { return valid(b) ? refs_[b] : NXT_KV_E_INVALID; }
    int alloc() {
        if (free_.empty()) return NXT_KV_E_NO_BLOCKS;
        const int b = free_.front();
        free_.pop_front();
        refs_[b] = 1;
        return b;
    }
    int inc(int b) {
        if (!valid(b) || refs_[b] <= 0) return NXT_KV_E_INVALID;
        return ++refs_[b];
    }
    int dec(int b) {
        if (!valid(b) || refs_[b] <= 0) return NXT_KV_E_INVALID;
        if (--refs_[b] == 0) free_.push_back(b);
        return refs_[b];
    }

  private:
    std::vector<int> refs_;
    std::deque<int> free_;
};

struct Node {
    std::vector<int32_t> tokens;  // edge label
    std::vector<int32_t> slots;   // one flat slot per token
    Node *parent = nullptr;
    std::vector<Node *> children;  // distinct first tokens, in insertion order
    uint64_t id = 0;
    uint64_t last_access = 0;
    uint64_t created = 0;
    int lock_ref = 0;
    int hit_count = 0;
    int priority = 0;
};

// Distinct pages of a run of slots.
std::vector<int32_t> pages_of(const int32_t *slots, size_t n, int bs_shift) {
    std::vector<int32_t> p(n);
    for (size_t i = 0; i < n; ++i) p[i] = slots[i] >> bs_shift;
    std::sort(p.begin(), p.end());
    p.erase(std::unique(p.begin(), p.end()), p.end());
    return p;
}

// Radix tree of prefix_sharing.c with slot ids for page ids.  Every node
// holds one pool reference on each distinct page among its slots.
class RadixTree {
  public:
    RadixTree(BlockPool &pool, int bs_shift) : pool_(pool), bs_shift_(bs_shift) {
        root_ = make_node(nullptr, nullptr, 0, 0);
        root_->lock_ref = 1;  // permanently protected (prefix_sharing.c:201)
    }
    ~RadixTree() { destroy(root_); }

    struct Match {
        int matched = 0;
        Node *last = nullptr;
    };

    // prefix_sharing.c:211-265, ending at the first node that would take the
    // match past `cap` slots.
    Match match(const int32_t *tok, int len, int32_t *slots_out, int cap) {
        Match r;
        r.last = root_;
        if (len <= 0 || !tok) return r;
        const uint64_t now = tick();
        root_->last_access = now;
        Node *node = root_;
        int offset = 0;
        while (offset < len) {
            Node *child = find_child(node, tok[offset]);
            if (!child) break;
            child->last_access = now;
            child->hit_count++;
            const int m = common_prefix(child->tokens, tok + offset, len - offset);
            if (r.matched + m > cap) break;
            if (m < (int)child->tokens.size()) {
                Node *head = split(child, m);
                append_slots(head, m, slots_out, r.matched);
                r.matched += m;
                r.last = head;
                break;
            }
            append_slots(child, m, slots_out, r.matched);
            r.matched += m;
            r.last = child;
            offset += m;
            node = child;
        }
        return r;
    }

    // prefix_sharing.c:267-325.  The caller has checked the slots.
    int insert(const int32_t *tok, int len, const int32_t *slots, int priority) {
        if (len <= 0 || !tok) return 0;
        const uint64_t now = tick();
        root_->last_access = now;
        Node *node = root_;
        int offset = 0;
        while (offset < len) {
            Node *child = find_child(node, tok[offset]);
            if (!child) break;
            child->last_access = now;
            child->priority = std::max(child->priority, priority);
            const int m = common_prefix(child->tokens, tok + offset, len - offset);
            if (m < (int)child->tokens.size()) {
                Node *head = split(child, m);
                head->priority = std::max(head->priority, priority);
                node = head;
                offset += m;
                break;
            }
            offset += m;
            node = child;
        }
        if (offset < len) {
            Node *leaf = make_node(tok + offset, slots + offset, len - offset, priority);
            leaf->parent = node;
            node->children.push_back(leaf);
            evictable_ += len - offset;
        }
        return offset;
    }

    // prefix_sharing.c:327-399: repeatedly the least recently used unlocked
    // leaf.  A heap holds the candidates; evicting a leaf can only make its
    // parent a new candidate, so the order equals rescanning every time.
    int evict(int num_tokens, const BlockPool *until_free = nullptr, int free_target = 0) {
        if (num_tokens <= 0 && !until_free) return 0;
        typedef std::pair<std::pair<uint64_t, uint64_t>, Node *> Entry;
        std::priority_queue<Entry, std::vector<Entry>, std::greater<Entry>> heap;
        std::vector<Node *> stack{root_};
        while (!stack.empty()) {
            Node *n = stack.back();
            stack.pop_back();
            for (Node *c : n->children) stack.push_back(c);
            if (evictable_leaf(n)) heap.push({{n->last_access, n->created}, n});
        }
        int evicted = 0;
        while (!heap.empty()) {
            if (until_free ? until_free->free_count() >= free_target : evicted >= num_tokens) break;
            Node *v = heap.top().second;
            heap.pop();
            Node *parent = v->parent;
            evicted += (int)v->tokens.size();
            evictable_ -= (int)v->tokens.size();
            auto &sib = parent->children;
            sib.erase(std::find(sib.begin(), sib.end(), v));
            destroy(v);
            if (evictable_leaf(parent)) heap.push({{parent->last_access, parent->created}, parent});
        }
        return evicted;
    }

    // prefix_sharing.c:401-425, refusing to unlock below zero.
    int lock(uint64_t id) {
        Node *n = find(id);
        if (!n) return NXT_KV_E_INVALID;
        for (Node *c = n; c && c != root_; c = c->parent) {
            if (c->lock_ref == 0) {
                evictable_ -= (int)c->tokens.size();
                protected_ += (int)c->tokens.size();
            }
            c->lock_ref++;
        }
        return NXT_KV_OK;
    }
    int unlock(uint64_t id) {
        Node *n = find(id);
        if (!n) return NXT_KV_E_INVALID;
        for (Node *c = n; c && c != root_; c = c->parent)
            if (c->lock_ref <= 0) return NXT_KV_E_INVALID;
        for (Node *c = n; c && c != root_; c = c->parent) {
            if (--c->lock_ref == 0) {
                evictable_ += (int)c->tokens.size();
                protected_ -= (int)c->tokens.size();
            }
        }
        return NXT_KV_OK;
    }

    NxtKvTreeStats stats() const {
        NxtKvTreeStats s;
        s.total_tokens = (int32_t)total_tokens_;
        s.node_count = (int32_t)by_id_.size();
        s.evictable_size = evictable_;
        s.protected_size = protected_;
        return s;
    }
    uint64_t root_id() const { return root_->id; }

  private:
    uint64_t tick() { return ++clock_; }

    bool evictable_leaf(const Node *n) const {
        return n != root_ && n->children.empty() && n->lock_ref == 0 && !n->tokens.empty();
    }

    Node *find(uint64_t id) const {
        auto it = by_id_.find(id);
        return it == by_id_.end() ? nullptr : it->second;
    }

    static Node *find_child(const Node *n, int32_t first) {
        for (Node *c : n->children)
            if (!c->tokens.empty() && c->tokens[0] == first) return c;
        return nullptr;
    }

    static int common_prefix(const std::vector<int32_t> &a, const int32_t *b, int nb) {
        const int lim = std::min((int)a.size(), nb);
        int i = 0;
        while (i < lim && a[i] == b[i]) ++i;
        return i;
    }

    static void append_slots(const Node *n, int m, int32_t *out, int at) {
        if (out) std::memcpy(out + at, n->slots.data(), sizeof(int32_t) * (size_t)m);
    }

    Node *make_node(const int32_t *tok, const int32_t *slots, int n, int priority) {
        Node *x = new Node;
        if (n > 0) {
            x->tokens.assign(tok, tok + n);
            x->slots.assign(slots, slots + n);
            for (int32_t p : pages_of(slots, (size_t)n, bs_shift_)) pool_.inc(p);
        }
        x->priority = priority;
        x->id = ++next_id_;
        x->created = tick();
        x->last_access = x->created;
        by_id_[x->id] = x;
        total_tokens_ += n;
        return x;
    }

    void destroy(Node *n) {
        for (Node *c : n->children) destroy(c);
        for (int32_t p : pages_of(n->slots.data(), n->slots.size(), bs_shift_)) pool_.dec(p);
        total_tokens_ -= (long long)n->tokens.size();
        by_id_.erase(n->id);
        delete n;
    }

    // prefix_sharing.c:123-188: a new node takes the first k tokens of
    // `child` and becomes its parent.  Pages that end up in both halves gain
    // one reference; the others move with their tokens.
    Node *split(Node *child, int k) {
        Node *head = make_node(child->tokens.data(), child->slots.data(), k, child->priority);
        total_tokens_ -= k;  // the tokens move, they are not new
        head->hit_count = child->hit_count;
        head->lock_ref = child->lock_ref;
        head->parent = child->parent;
        auto &sib = child->parent->children;
        *std::find(sib.begin(), sib.end(), child) = head;
        const std::vector<int32_t> before =
            pages_of(child->slots.data(), child->slots.size(), bs_shift_);
        child->tokens.erase(child->tokens.begin(), child->tokens.begin() + k);
        child->slots.erase(child->slots.begin(), child->slots.begin() + k);
        const std::vector<int32_t> after =
            pages_of(child->slots.data(), child->slots.size(), bs_shift_);
        for (int32_t p : before)
            if (!std::binary_search(after.begin(), after.end(), p)) pool_.dec(p);
        child->parent = head;
        head->children.push_back(child);
        return head;
    }

    BlockPool &pool_;
    int bs_shift_;
    Node *root_ = nullptr;
    std::unordered_map<uint64_t, Node *> by_id_;
    uint64_t clock_ = 0;
    uint64_t next_id_ = 0;
    long long total_tokens_ = 0;
    int evictable_ = 0;
    int protected_ = 0;
};

struct Sequence {
    std::vector<int32_t> tokens;  // prompt and generated tokens, all with K/V in the cache
    std::vector<int32_t> blocks;  // its block-table row
    uint64_t locked = 0;          // tree node locked at admission (0: none)
    int shared_blocks = 0;
};

}  // namespace

struct NxtKvIndex {
    NxtKvIndex(int num_blocks, int bs, int max_blocks)
        : pool(num_blocks), block_size(bs), bs_shift(__builtin_ctz((unsigned)bs)),
          max_blocks(max_blocks), tree(pool, bs_shift) {}

    BlockPool pool;
    int block_size;
    int bs_shift;
    int max_blocks;
    RadixTree tree;
    std::vector<std::unique_ptr<Sequence>> seqs;  // handle = index
    std::vector<int32_t> free_handles;

    Sequence *seq(int32_t h) const {
        if (h < 0 || h >= (int32_t)seqs.size()) return nullptr;
        return seqs[(size_t)h].get();
    }
    int32_t slot_of(const Sequence &s, int t) const {
        return s.blocks[(size_t)(t >> bs_shift)] * block_size + (t & (block_size - 1));
    }
    bool slot_ok(int32_t slot) const {
        return slot >= 0 && (slot >> bs_shift) < pool.size() && pool.refs(slot >> bs_shift) > 0;
    }
    // Frees pages by evicting tree leaves until `need` blocks are free.
    bool ensure_free(int need) {
        if (pool.free_count() >= need) return true;
        tree.evict(0, &pool, need);
        return pool.free_count() >= need;
    }
    int32_t new_handle() {
        if (!free_handles.empty()) {
            const int32_t h = free_handles.back();
            free_handles.pop_back();
            return h;
        }
        seqs.emplace_back();
        return (int32_t)seqs.size() - 1;
    }
};

XKV_EXPORT NxtKvIndex *nxt_kv_index_create(int num_blocks, int block_size, int max_blocks_per_seq) {
    if (num_blocks <= 0 || block_size <= 0 || (block_size & (block_size - 1)) ||
        block_size > (1 << 20) || max_blocks_per_seq <= 0 ||
        (long long)num_blocks * block_size > INT32_MAX ||
        (long long)max_blocks_per_seq * block_size > INT32_MAX)
        return nullptr;
    try {
        return new NxtKvIndex(num_blocks, block_size, max_blocks_per_seq);
    } catch (...) {
        return nullptr;
    }
}

XKV_EXPORT void nxt_kv_index_destroy(NxtKvIndex *ix) { delete ix; }

XKV_EXPORT int nxt_kv_block_alloc(NxtKvIndex *ix) {
    return ix ? ix->pool.alloc() : NXT_KV_E_INVALID;
}
XKV_EXPORT int nxt_kv_block_ref_inc(NxtKvIndex *ix, int block) {
    return ix ? ix->pool.inc(block) : NXT_KV_E_INVALID;
}
XKV_EXPORT int nxt_kv_block_ref_dec(NxtKvIndex *ix, int block) {
    return ix ? ix->pool.dec(block) : NXT_KV_E_INVALID;
}
XKV_EXPORT int nxt_kv_block_refs(const NxtKvIndex *ix, int block) {
    return ix ? ix->pool.refs(block) : NXT_KV_E_INVALID;
}
XKV_EXPORT int nxt_kv_blocks_free(const NxtKvIndex *ix) {
    return ix ? ix->pool.free_count() : NXT_KV_E_INVALID;
}

XKV_EXPORT int nxt_kv_prefix_match(NxtKvIndex *ix, const int32_t *tokens, int32_t len,
                                   int32_t *slots, NxtKvMatch *out) {
    if (!ix || !out || len < 0 || (len > 0 && (!tokens || !slots))) return NXT_KV_E_INVALID;
    const RadixTree::Match m = ix->tree.match(tokens, len, slots, NXT_PREFIX_MAX_MATCH_PAGES);
    out->matched_tokens = m.matched;
    out->reserved = 0;
    out->last_node = m.matched > 0 ? m.last->id : 0;
    return NXT_KV_OK;
}

XKV_EXPORT int32_t nxt_kv_prefix_insert(NxtKvIndex *ix, const int32_t *tokens, int32_t len,
                                        const int32_t *slots, int32_t priority) {
    if (!ix || len < 0 || (len > 0 && (!tokens || !slots))) return NXT_KV_E_INVALID;
    for (int32_t i = 0; i < len; ++i)
        if (!ix->slot_ok(slots[i])) return NXT_KV_E_INVALID;
    return ix->tree.insert(tokens, len, slots, priority);
}

XKV_EXPORT int32_t nxt_kv_prefix_evict(NxtKvIndex *ix, int32_t num_tokens) {
    return ix ? ix->tree.evict(num_tokens) : NXT_KV_E_INVALID;
}

XKV_EXPORT int nxt_kv_prefix_lock(NxtKvIndex *ix, uint64_t node) {
    return ix ? ix->tree.lock(node) : NXT_KV_E_INVALID;
}
XKV_EXPORT int nxt_kv_prefix_unlock(NxtKvIndex *ix, uint64_t node) {
    return ix ? ix->tree.unlock(node) : NXT_KV_E_INVALID;
}

XKV_EXPORT int nxt_kv_prefix_stats(const NxtKvIndex *ix, NxtKvTreeStats *out) {
    if (!ix || !out) return NXT_KV_E_INVALID;
    *out = ix->tree.stats();
    return NXT_KV_OK;
}

XKV_EXPORT int nxt_kv_seq_admit(NxtKvIndex *ix, const int32_t *tokens, int32_t len,
                                int32_t *slot_mapping, int32_t *copy_src, int32_t *copy_dst,
                                NxtKvAdmit *out) {
    if (!ix || !tokens || !slot_mapping || !copy_src || !copy_dst || !out || len <= 0)
        return NXT_KV_E_INVALID;
    const int bs = ix->block_size;
    if ((long long)len > (long long)ix->max_blocks * bs) return NXT_KV_E_CAPACITY;

    std::vector<int32_t> matched((size_t)std::min<int32_t>(len, NXT_PREFIX_MAX_MATCH_PAGES));
    const RadixTree::Match m =
        ix->tree.match(tokens, len, matched.data(), NXT_PREFIX_MAX_MATCH_PAGES);
    const int M = m.matched;
    // Leading pages of the match whose slots are a whole page in order: they
    // are shared as they are.  A page the match ends in (or one stored out
    // of order) is copied instead, because this sequence writes after it.
    int P = 0;
    while ((P + 1) * bs <= M) {
        const int32_t first = matched[(size_t)P * bs];
        if (first & (bs - 1)) break;
        bool whole = true;
        for (int i = 1; i < bs && whole; ++i) whole = matched[(size_t)P * bs + i] == first + i;
        if (!whole) break;
        ++P;
    }
    const int n_blocks = (len + bs - 1) / bs;
    const uint64_t lock_id = M > 0 ? m.last->id : 0;
    if (lock_id) ix->tree.lock(lock_id);  // keeps the matched pages cached meanwhile
    if (!ix->ensure_free(n_blocks - P)) {
        if (lock_id) ix->tree.unlock(lock_id);
        return NXT_KV_E_NO_BLOCKS;
    }

    std::unique_ptr<Sequence> s(new Sequence);
    s->tokens.assign(tokens, tokens + len);
    s->locked = lock_id;
    s->shared_blocks = P;
    for (int j = 0; j < P; ++j) {
        const int32_t b = matched[(size_t)j * bs] >> ix->bs_shift;
        ix->pool.inc(b);
        s->blocks.push_back(b);
    }
    for (int j = P; j < n_blocks; ++j) s->blocks.push_back(ix->pool.alloc());

    int copies = 0;
    for (int t = 0; t < len; ++t) {
        if (t < P * bs) {
            slot_mapping[t] = -1;
        } else if (t < M) {
            slot_mapping[t] = -1;
            copy_src[copies] = matched[(size_t)t];
            copy_dst[copies] = ix->slot_of(*s, t);
            ++copies;
        } else {
            slot_mapping[t] = ix->slot_of(*s, t);
        }
    }
    const int32_t h = ix->new_handle();
    ix->seqs[(size_t)h] = std::move(s);
    out->seq = h;
    out->cached_tokens = M;
    out->shared_blocks = P;
    out->copy_count = copies;
    out->write_count = len - M;
    return NXT_KV_OK;
}

XKV_EXPORT int nxt_kv_seq_append(NxtKvIndex *ix, int32_t seq, const int32_t *tokens, int32_t n,
                                 int32_t *slots) {
    Sequence *s = ix ? ix->seq(seq) : nullptr;
    if (!s || n < 0 || (n > 0 && (!tokens || !slots))) return NXT_KV_E_INVALID;
    const int bs = ix->block_size;
    const long long len = (long long)s->tokens.size();
    if (len + n > (long long)ix->max_blocks * bs) return NXT_KV_E_CAPACITY;
    const int need = (int)((len + n + bs - 1) / bs) - (int)s->blocks.size();
    if (need > 0 && !ix->ensure_free(need)) return NXT_KV_E_NO_BLOCKS;
    for (int j = 0; j < need; ++j) s->blocks.push_back(ix->pool.alloc());
    for (int32_t i = 0; i < n; ++i) {
        s->tokens.push_back(tokens[i]);
        slots[i] = ix->slot_of(*s, (int)(len + i));
    }
    return NXT_KV_OK;
}

XKV_EXPORT int nxt_kv_batch_append(NxtKvIndex *ix, const int32_t *seqs, int32_t n,
                                   const int32_t *tokens, int32_t *slots) {
    if (!ix || n < 0 || (n > 0 && (!seqs || !tokens || !slots))) return NXT_KV_E_INVALID;
    const int bs = ix->block_size;
    int need = 0;
    std::vector<char> seen(ix->seqs.size(), 0);
    for (int32_t i = 0; i < n; ++i) {
        const Sequence *s = ix->seq(seqs[i]);
        if (!s || seen[(size_t)seqs[i]]) return NXT_KV_E_INVALID;
        seen[(size_t)seqs[i]] = 1;
        const long long len = (long long)s->tokens.size();
        if (len + 1 > (long long)ix->max_blocks * bs) return NXT_KV_E_CAPACITY;
        need += (len & (bs - 1)) == 0;
    }
    if (need > 0 && !ix->ensure_free(need)) return NXT_KV_E_NO_BLOCKS;
    for (int32_t i = 0; i < n; ++i) {
        Sequence *s = ix->seq(seqs[i]);
        const int len = (int)s->tokens.size();
        if ((len & (bs - 1)) == 0) s->blocks.push_back(ix->pool.alloc());
        s->tokens.push_back(tokens[i]);
        slots[i] = ix->slot_of(*s, len);
    }
    return NXT_KV_OK;
}

XKV_EXPORT int32_t nxt_kv_seq_cache(NxtKvIndex *ix, int32_t seq) {
    Sequence *s = ix ? ix->seq(seq) : nullptr;
    if (!s) return NXT_KV_E_INVALID;
    const int len = (int)s->tokens.size();
    std::vector<int32_t> slots((size_t)len);
    for (int t = 0; t < len; ++t) slots[(size_t)t] = ix->slot_of(*s, t);
    return ix->tree.insert(s->tokens.data(), len, slots.data(), 0);
}

XKV_EXPORT int nxt_kv_seq_release(NxtKvIndex *ix, int32_t seq, int cache) {
    Sequence *s = ix ? ix->seq(seq) : nullptr;
    if (!s) return NXT_KV_E_INVALID;
    if (cache) nxt_kv_seq_cache(ix, seq);
    if (s->locked) ix->tree.unlock(s->locked);
    for (int32_t b : s->blocks) ix->pool.dec(b);
    ix->seqs[(size_t)seq].reset();
    ix->free_handles.push_back(seq);
    return NXT_KV_OK;
}

XKV_EXPORT int32_t nxt_kv_seq_len(const NxtKvIndex *ix, int32_t seq) {
    const Sequence *s = ix ? ix->seq(seq) : nullptr;
    return s ? (int32_t)s->tokens.size() : NXT_KV_E_INVALID;
}

XKV_EXPORT int nxt_kv_batch_tables(const NxtKvIndex *ix, const int32_t *seqs, int32_t n,
                                   int32_t max_blocks, int32_t *block_tables, int32_t *seq_lens) {
    if (!ix || n < 0 || max_blocks <= 0 || (n > 0 && (!seqs || !block_tables || !seq_lens)))
        return NXT_KV_E_INVALID;
    for (int32_t i = 0; i < n; ++i) {
        const Sequence *s = ix->seq(seqs[i]);
        if (!s) return NXT_KV_E_INVALID;
        if ((int32_t)s->blocks.size() > max_blocks) return NXT_KV_E_CAPACITY;
    }
    for (int32_t i = 0; i < n; ++i) {
        const Sequence *s = ix->seq(seqs[i]);
        int32_t *row = block_tables + (size_t)i * max_blocks;
        const size_t nb = s->blocks.size();
        std::memcpy(row, s->blocks.data(), nb * sizeof(int32_t));
        std::fill(row + nb, row + max_blocks, -1);
        seq_lens[i] = (int32_t)s->tokens.size();
    }
    return NXT_KV_OK;
}

// Leading entries two page lists have in common, up to n (256- then
// 32-byte runs compared with memcmp first).
static int common_prefix(const int32_t *a, const int32_t *b, int n) {
    int k = 0;
    while (k + 64 <= n && std::memcmp(a + k, b + k, 64 * sizeof(int32_t)) == 0) k += 64;
    while (k + 8 <= n && std::memcmp(a + k, b + k, 8 * sizeof(int32_t)) == 0) k += 8;
    while (k < n && a[k] == b[k]) ++k;
    return k;
}

XKV_EXPORT int nxt_kv_batch_prefix_groups(const NxtKvIndex *ix, const int32_t *seqs, int32_t n,
                                          int32_t *prefix_group, int32_t *prefix_blocks,
                                          int32_t *num_groups) {
    if (!ix || n < 0 || !num_groups || (n > 0 && (!seqs || !prefix_group || !prefix_blocks)))
        return NXT_KV_E_INVALID;
    std::vector<const Sequence *> s((size_t)n);
    for (int32_t i = 0; i < n; ++i)
        if (!(s[(size_t)i] = ix->seq(seqs[i]))) return NXT_KV_E_INVALID;
    const int bs = ix->block_size;
    auto full = [&](int32_t i) { return (int)(s[(size_t)i]->tokens.size() / (size_t)bs); };
    // members by first page, in batch order: (first page, batch index), sorted
    std::vector<std::pair<int32_t, int32_t>> byf;
    byf.reserve((size_t)n);
    for (int32_t i = 0; i < n; ++i)
        if (full(i) >= 1) byf.push_back({s[(size_t)i]->blocks[0], i});
    std::sort(byf.begin(), byf.end());
    // each run of two or more members: the pages every member shares with
    // the lowest one, counting full pages only
    struct Group {
        int32_t lead, pages;
        size_t begin, end;  // its members in byf
    };
    std::vector<Group> groups;
    for (size_t a = 0; a < byf.size();) {
        size_t b = a + 1;
        while (b < byf.size() && byf[b].first == byf[a].first) ++b;
        if (b - a >= 2) {
            const int32_t lead = byf[a].second;
            const int32_t *lb = s[(size_t)lead]->blocks.data();
            int P = full(lead);
            for (size_t k = a + 1; k < b && P > 0; ++k) {
                const int32_t i = byf[k].second;
                const int32_t *ib = s[(size_t)i]->blocks.data();
                const int lim = std::min(full(i), P);
                P = common_prefix(ib, lb, lim);
            }
            if (P >= 1) groups.push_back({lead, P, a, b});
        }
        a = b;
    }
    // numbered by their lowest member
    std::sort(groups.begin(), groups.end(),
              [](const Group &x, const Group &y) { return x.lead < y.lead; });
    std::fill(prefix_group, prefix_group + n, -1);
    for (size_t g = 0; g < groups.size(); ++g) {
        prefix_blocks[g] = groups[g].pages;
        for (size_t k = groups[g].begin; k < groups[g].end; ++k)
            prefix_group[byf[k].second] = (int32_t)g;
    }
    *num_groups = (int32_t)groups.size();
    return NXT_KV_OK;
}
