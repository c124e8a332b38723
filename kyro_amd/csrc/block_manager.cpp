// Host block allocator and block-granular prefix cache (see block_manager.hpp for the
// differences from the reference and why).
#include "block_manager.hpp"

#include <algorithm>

namespace kyro {
namespace bm {

namespace {
int64_t blocks_for(int64_t tokens, int bs) { return (tokens + bs - 1) / bs; }

size_t common_prefix(const Tokens& a, const uint32_t* b, size_t nb) {
    const size_t n = std::min(a.size(), nb);
    size_t i = 0;
    while (i < n && a[i] == b[i]) ++i;
    return i;
}
}  // namespace

// ------------------------------------------------------------------------------ RadixCache

RadixCache::RadixCache(int block_size, int64_t max_capacity) : bs_(block_size), capacity_(max_capacity) {}

void RadixCache::leaf_add(Node* n) {
    if (n != &root_ && n->children.empty()) leaves_.insert({n->last_access, n});
}

void RadixCache::leaf_remove(Node* n) { leaves_.erase({n->last_access, n}); }

// The reference stamps Instant::now() on each matched node (radix_cache.rs:74); a logical clock
// gives the same order without ties between calls.
void RadixCache::touch(Node* n) {
    const bool leaf = n->children.empty();
    if (leaf) leaf_remove(n);
    n->last_access = ++clock_;
    if (leaf) leaf_add(n);
}

// radix_cache.rs:49-86 walks nodes whose token runs match in full. Here a node is one block:
// whole blocks match by key, and the walk ends at the child sharing the longest prefix with the
// next (partial or diverging) block, which the caller treats as a partially matched block.
std::pair<std::vector<int64_t>, int64_t> RadixCache::match_prefix(const uint32_t* t, int64_t n) {
    std::vector<int64_t> blocks;
    Node* node = &root_;
    int64_t pos = 0;
    while (pos < n) {
        const int64_t take = std::min<int64_t>(bs_, n - pos);
        if (take == bs_) {
            auto it = node->children.find(Tokens(t + pos, t + pos + take));
            if (it != node->children.end()) {
                Node* c = it->second.get();
                touch(c);
                blocks.push_back(c->block);
                pos += take;
                node = c;
                continue;
            }
        }
        Node* best = nullptr;
        size_t best_len = 0;
        for (auto& kv : node->children) {  // map order: ties go to the smallest key
            const size_t c = common_prefix(kv.first, t + pos, (size_t)take);
            if (c > best_len) {
                best_len = c;
                best = kv.second.get();
            }
        }
        if (best) {
            touch(best);
            blocks.push_back(best->block);
            pos += (int64_t)best_len;
        }
        break;
    }
    return {blocks, pos};
}

// radix_cache.rs:89-120 inserts the remaining tokens as one node holding every block of the
// sequence, so a later match returns blocks twice; here each block becomes its own node and a
// block already cached under the same tokens is reported as not taken. Eviction after an insert
// (:117-119) returns the evicted blocks so their references can be dropped.
std::vector<bool> RadixCache::insert(const uint32_t* t, int64_t n, const int64_t* blocks,
                                     std::vector<int64_t>* evicted) {
    const int64_t nb = blocks_for(n, bs_);
    std::vector<bool> taken((size_t)nb, false);
    Node* node = &root_;
    for (int64_t i = 0; i < nb; ++i) {
        const int64_t p0 = i * bs_, p1 = std::min<int64_t>(n, p0 + bs_);
        Tokens key(t + p0, t + p1);
        auto it = node->children.find(key);
        if (it != node->children.end()) {
            node = it->second.get();
            touch(node);
            continue;
        }
        if ((int64_t)node->key.size() < bs_ && node != &root_) break;  // partial nodes stay leaves
        auto child = std::make_unique<Node>();
        child->key = std::move(key);
        child->block = blocks[i];
        child->parent = node;
        child->last_access = ++clock_;
        Node* c = child.get();
        leaf_remove(node);  // the parent stops being a leaf
        node->children.emplace(c->key, std::move(child));
        leaf_add(c);
        ++num_cached_;
        taken[(size_t)i] = true;
        node = c;
    }
    if (num_cached_ > capacity_) {
        std::vector<int64_t> ev = evict_lru();
        if (evicted) evicted->insert(evicted->end(), ev.begin(), ev.end());
    }
    return taken;
}

// radix_cache.rs:126-155 takes the oldest leaf among the first tree level that has one, in
// HashMap order; here it is the least recently used leaf of the whole tree.
bool RadixCache::evict_one(int64_t* block) {
    if (leaves_.empty()) return false;
    Node* n = leaves_.begin()->second;
    leaves_.erase(leaves_.begin());
    *block = n->block;
    Node* parent = n->parent;
    const Tokens key = n->key;
    parent->children.erase(key);  // frees n
    --num_cached_;
    leaf_add(parent);
    return true;
}

void RadixCache::cached_blocks(std::vector<int64_t>* out) const {
    std::vector<const Node*> stack{&root_};
    while (!stack.empty()) {
        const Node* n = stack.back();
        stack.pop_back();
        if (n != &root_) out->push_back(n->block);
        for (auto& kv : n->children) stack.push_back(kv.second.get());
    }
}

std::vector<int64_t> RadixCache::evict_lru() {
    std::vector<int64_t> out;
    int64_t b;
    while (num_cached_ > capacity_ && evict_one(&b)) out.push_back(b);
    return out;
}

// ---------------------------------------------------------------------------- BlockManager

// block_manager.rs:32-50: every GPU block free (popped from the back, so block N-1 first) and a
// cache budget of a third of the GPU blocks.
BlockManager::BlockManager(int block_size, int64_t num_gpu_blocks, int64_t num_cpu_blocks)
    : bs_(block_size), num_gpu_(num_gpu_blocks), num_cpu_(num_cpu_blocks),
      ref_((size_t)num_gpu_blocks, 0), cache_(block_size, num_gpu_blocks / 3) {
    free_.reserve((size_t)num_gpu_blocks);
    for (int64_t b = 0; b < num_gpu_blocks; ++b) free_.push_back(b);
}

void BlockManager::release(int64_t block) {
    int& r = ref_[(size_t)block];
    if (r <= 0) return;  // never reached when every holder drops its reference once
    if (--r == 0) free_.push_back(block);
}

// block_manager.rs:67-76 evicts once, down to the cache budget, and may still fail; here leaves
// are evicted one at a time until n blocks are free or the cache is empty.
bool BlockManager::reserve(int64_t n) {
    int64_t b;
    while ((int64_t)free_.size() < n && cache_.evict_one(&b)) release(b);
    return (int64_t)free_.size() >= n;
}

// block_manager.rs:53-102. A match ending inside a block cannot share that block (the request
// writes its own tokens into the rest of it), so the request gets a fresh block and a pending
// copy of the cached one; the matched token count is the reference's cached_token_count.
int BlockManager::allocate_with_prefix(uint64_t rid, const uint32_t* tokens, int64_t n, int64_t* cached) {
    if (n < 0 || table_.count(rid)) return EINVAL_;
    auto match = cache_.match_prefix(tokens, n);
    const int64_t matched = match.second;
    const int64_t full = matched / bs_;
    const bool partial = matched % bs_ != 0;
    const int64_t cow_src = partial ? match.first[(size_t)full] : -1;
    for (int64_t i = 0; i < full; ++i) ++ref_[(size_t)match.first[(size_t)i]];
    if (partial) ++ref_[(size_t)cow_src];  // held until the copy is handed out
    const int64_t need = blocks_for(n, bs_) - full;
    if (!reserve(need)) {
        for (int64_t i = 0; i < full; ++i) release(match.first[(size_t)i]);
        if (partial) release(cow_src);
        return ENOSPACE;
    }
    Request r;
    r.blocks.assign(match.first.begin(), match.first.begin() + full);
    for (int64_t i = 0; i < need; ++i) {
        const int64_t b = free_.back();
        free_.pop_back();
        ref_[(size_t)b] = 1;
        r.blocks.push_back(b);
    }
    if (partial) copies_.push_back({cow_src, r.blocks[(size_t)full]});
    r.prompt.assign(tokens, tokens + n);
    r.has_prompt = true;
    r.num_tokens = n;
    table_.emplace(rid, std::move(r));
    *cached = matched;
    return OK;
}

// block_manager.rs:107-124 (no prefix caching, no eviction).
int BlockManager::allocate(uint64_t rid, int64_t num_tokens) {
    if (num_tokens < 0 || table_.count(rid)) return EINVAL_;
    const int64_t need = blocks_for(num_tokens, bs_);
    if ((int64_t)free_.size() < need) return ENOSPACE;
    Request r;
    for (int64_t i = 0; i < need; ++i) {
        const int64_t b = free_.back();
        free_.pop_back();
        ref_[(size_t)b] = 1;
        r.blocks.push_back(b);
    }
    r.num_tokens = num_tokens;
    table_.emplace(rid, std::move(r));
    return OK;
}

// Room for n more tokens (a decode token, or the k + 1 rows of a verify step). Positions at or
// past the prompt always lie in blocks the request owns alone, so they can be written.
int BlockManager::append_slots(uint64_t rid, int64_t n) {
    auto it = table_.find(rid);
    if (it == table_.end() || n < 0) return EINVAL_;
    Request& r = it->second;
    const int64_t need = blocks_for(r.num_tokens + n, bs_) - (int64_t)r.blocks.size();
    if (need > 0) {
        if (!reserve(need)) return ENOSPACE;
        for (int64_t i = 0; i < need; ++i) {
            const int64_t b = free_.back();
            free_.pop_back();
            ref_[(size_t)b] = 1;
            r.blocks.push_back(b);
        }
    }
    r.num_tokens += n;
    return OK;
}

// Drops rows after num_tokens (rejected drafts), releasing blocks no longer covered. The prompt
// is never cut: its last block may be shared with the cache.
int BlockManager::truncate(uint64_t rid, int64_t num_tokens) {
    auto it = table_.find(rid);
    if (it == table_.end()) return EINVAL_;
    Request& r = it->second;
    const int64_t floor_len = r.has_prompt ? (int64_t)r.prompt.size() : 0;
    if (num_tokens < floor_len || num_tokens > r.num_tokens) return EINVAL_;
    const int64_t keep = blocks_for(num_tokens, bs_);
    while ((int64_t)r.blocks.size() > keep) {
        release(r.blocks.back());
        r.blocks.pop_back();
    }
    r.num_tokens = num_tokens;
    return OK;
}

// block_manager.rs:128-153 hands the request's blocks to the cache with the prompt. Here the
// cache takes its own reference on the blocks it did not already hold, then the request drops
// its reference on all of its blocks, so each block is freed when its last holder lets go.
// cache_prompt = false (a request ended before its prompt's K/V was written) skips the cache.
int BlockManager::free(uint64_t rid, bool cache_prompt) {
    auto it = table_.find(rid);
    if (it == table_.end()) return EINVAL_;
    Request r = std::move(it->second);
    table_.erase(it);
    std::vector<int64_t> evicted;
    if (cache_prompt && r.has_prompt && !r.prompt.empty()) {
        const std::vector<bool> taken =
            cache_.insert(r.prompt.data(), (int64_t)r.prompt.size(), r.blocks.data(), &evicted);
        for (size_t i = 0; i < taken.size(); ++i)
            if (taken[i]) ++ref_[(size_t)r.blocks[i]];
    }
    for (int64_t b : r.blocks) release(b);
    for (int64_t b : evicted) release(b);
    return OK;
}

std::string BlockManager::check() const {
    std::vector<int> holders((size_t)num_gpu_, 0);
    for (auto& kv : table_)
        for (int64_t b : kv.second.blocks) ++holders[(size_t)b];
    std::vector<int64_t> cached;
    cache_.cached_blocks(&cached);
    if ((int64_t)cached.size() != cache_.num_cached_blocks()) return "cache node count disagrees";
    for (int64_t b : cached) ++holders[(size_t)b];
    for (auto& c : copies_) ++holders[(size_t)c.first];
    std::vector<char> in_free((size_t)num_gpu_, 0);
    for (int64_t b : free_) {
        if (b < 0 || b >= num_gpu_) return "free pool holds an invalid id";
        if (in_free[(size_t)b]) return "block " + std::to_string(b) + " is twice in the free pool";
        in_free[(size_t)b] = 1;
    }
    for (int64_t b = 0; b < num_gpu_; ++b) {
        if (holders[(size_t)b] != ref_[(size_t)b])
            return "block " + std::to_string(b) + ": " + std::to_string(holders[(size_t)b]) + " holders, ref count " +
                   std::to_string(ref_[(size_t)b]);
        if ((holders[(size_t)b] == 0) != (in_free[(size_t)b] != 0))
            return "block " + std::to_string(b) + (in_free[(size_t)b] ? " is free but held" : " is unheld but not free");
    }
    return "";
}

const Request* BlockManager::find(uint64_t rid) const {
    auto it = table_.find(rid);
    return it == table_.end() ? nullptr : &it->second;
}

// The copies are handed out once; the source's reference is dropped then, so the caller must
// queue the copies before anything else writes into the cache on that stream.
std::vector<std::pair<int64_t, int64_t>> BlockManager::take_copies() {
    std::vector<std::pair<int64_t, int64_t>> out;
    out.swap(copies_);
    for (auto& c : out) release(c.first);
    return out;
}

}  // namespace bm
}  // namespace kyro
