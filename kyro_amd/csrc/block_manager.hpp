// Host block allocator and block-granular prefix cache behind include/kyro_blocks.h.
//
// Follows BlockManager (src/scheduler/block_manager.rs:15-153) and RadixCache
// (src/scheduler/radix_cache.rs:29-155) with these differences, each for a reason given at the
// definition: the prefix tree is keyed by block contents, so a node is one block and a match
// hands out whole blocks plus, at most, one partially matched block that the request gets as a
// private copy (copy-on-write); eviction takes the globally least recently used leaf under a
// logical clock; every reference the cache or a request takes is dropped exactly once; and a
// request's block list can grow and shrink (decode and speculative verify rows).
#pragma once

#include <stdint.h>

#include <map>
#include <memory>
#include <set>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

namespace kyro {
namespace bm {

using Tokens = std::vector<uint32_t>;

// One cached block: its tokens (block_size of them, or fewer for a partially filled last block,
// which is then a leaf), the physical block holding their K/V, and its place in the tree.
struct Node {
    Tokens key;
    int64_t block = -1;
    Node* parent = nullptr;
    std::map<Tokens, std::unique_ptr<Node>> children;
    uint64_t last_access = 0;
};

class RadixCache {
   public:
    RadixCache(int block_size, int64_t max_capacity);

    // Longest cached prefix of tokens: the blocks holding it (the last one possibly holding only
    // part of the match) and the number of matched tokens. Touches the matched nodes.
    std::pair<std::vector<int64_t>, int64_t> match_prefix(const uint32_t* tokens, int64_t n);

    // Caches tokens held by blocks (ceil(n / block_size) of them). Returns, per block, whether
    // the cache took it (a new node; the caller then adds the cache's reference), and appends to
    // `evicted` the blocks dropped to get back under capacity (the caller drops their references).
    std::vector<bool> insert(const uint32_t* tokens, int64_t n, const int64_t* blocks,
                             std::vector<int64_t>* evicted);

    // Removes least-recently-used leaves until at most max_capacity blocks remain.
    std::vector<int64_t> evict_lru();
    // Removes the least-recently-used leaf; false when the cache is empty.
    bool evict_one(int64_t* block);

    int64_t num_cached_blocks() const { return num_cached_; }
    int64_t max_capacity() const { return capacity_; }
    // Appends every cached block id (tree order).
    void cached_blocks(std::vector<int64_t>* out) const;

   private:
    void touch(Node* n);
    void leaf_add(Node* n);
    void leaf_remove(Node* n);

    int bs_;
    int64_t capacity_;
    int64_t num_cached_ = 0;
    uint64_t clock_ = 0;
    Node root_;
    std::set<std::pair<uint64_t, Node*>> leaves_;  // (last_access, node), oldest first
};

struct Request {
    std::vector<int64_t> blocks;
    Tokens prompt;       // empty for a request allocated without prefix caching
    bool has_prompt = false;
    int64_t num_tokens = 0;
};

enum Status : int { OK = 0, EINVAL_ = 1, ENOSPACE = 5 };

class BlockManager {
   public:
    BlockManager(int block_size, int64_t num_gpu_blocks, int64_t num_cpu_blocks);

    int allocate_with_prefix(uint64_t rid, const uint32_t* tokens, int64_t n, int64_t* cached);
    int allocate(uint64_t rid, int64_t num_tokens);
    int append_slots(uint64_t rid, int64_t n);
    int truncate(uint64_t rid, int64_t num_tokens);
    int free(uint64_t rid, bool cache_prompt);

    const Request* find(uint64_t rid) const;
    std::vector<std::pair<int64_t, int64_t>> take_copies();
    const std::vector<std::pair<int64_t, int64_t>>& take_copies_peek() const { return copies_; }

    int64_t num_free_blocks() const { return (int64_t)free_.size(); }
    int block_size() const { return bs_; }
    RadixCache& cache() { return cache_; }
    int ref_count(int64_t block) const { return ref_[(size_t)block]; }
    int64_t num_gpu_blocks() const { return num_gpu_; }
    // Recomputes every block's holders (requests, cache nodes, pending copies) and compares with
    // the reference counts and the free pool. Returns an empty string when they agree.
    std::string check() const;

   private:
    bool reserve(int64_t n);  // evicts cache leaves until n blocks are free
    void release(int64_t block);

    int bs_;
    int64_t num_gpu_;
    int64_t num_cpu_;
    std::vector<int64_t> free_;
    std::vector<int> ref_;
    RadixCache cache_;
    std::unordered_map<uint64_t, Request> table_;
    std::vector<std::pair<int64_t, int64_t>> copies_;  // (source, destination) copy-on-write
};

}  // namespace bm
}  // namespace kyro
