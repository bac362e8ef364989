// kv_cache.cpp -- host page tables of the paged KV cache, with rollback.
//
// A restatement of the reference's PagedKVCache metadata
// (csrc/include/cudaforge/memory/paged_kv_cache.h:36-179,
//  csrc/src/memory/paged_kv_cache.cpp:9-445): physical blocks with reference
// counts and fill counts, a LIFO free list, prefix sharing of full prompt
// blocks through a trie of chained block hashes, LRU retention of released
// prefix blocks, and the per-batch metadata (block tables and context
// lengths) staged for the kernels.  The pools themselves and the staging
// buffers belong to the caller (this library allocates no device memory).
//
// Added for tree speculation (the reference has no truncate): truncate()
// releases the pages past a new length -- the rollback of rejected draft
// tokens after cfa_kv_commit has compacted the accepted ones.
//
// Kept alike on purpose: the block allocation order (LIFO stack holding
// 0..n-1 with 0 on top), the LRU eviction order, the block-hash function and
// the context length (blocks - 1) * block_size + last fill, so that the same
// calls give the same block tables as the reference.
// Deliberate differences, each fixing a way the reference corrupts its tables:
//  * evicting a cached prefix page also unlinks its trie node, so a later
//    prompt cannot match a page that was recycled for other data (the
//    reference leaves the node under its parent, paged_kv_cache.cpp:101-124);
//  * register and append check that enough pages are free or evictable before
//    changing anything, so OutOfPages leaves every table as it was (the
//    reference throws midway and keeps the pages taken so far,
//    paged_kv_cache.cpp:216-249, 272-284);
//  * fork onto a registered child releases the child's pages first (the
//    reference overwrites its table, paged_kv_cache.cpp:315);
//  * copy on write: after a fork both tables hold the partly filled last
//    page, and the reference's append_tokens (paged_kv_cache.cpp:265-271)
//    fills it for both, so each sequence's new tokens overwrite the other's.
//    Here the appending sequence first gets a private page, and the device
//    copy of the shared slots is queued (cfa_kv_cache_pop_page_copies).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <mutex>
#include <new>
#include <string>
#include <unordered_map>
#include <vector>

#include "abi_internal.hpp"

namespace cfa {
namespace kvc {

struct Block {
  uint32_t refs = 0;
  uint32_t filled = 0;
  uint64_t hash = 0;    // non-zero: a full prompt block registered in the trie
  bool cached = false;  // no references, kept on the LRU list for prefix reuse
  int32_t prev = -1, next = -1;  // LRU links (toward more / less recent)
  int32_t node = -1;    // trie node of a hashed block
};

struct Node {
  uint64_t hash = 0;
  int32_t block = -1;
  int32_t parent = -1;
  bool live = false;
  std::unordered_map<uint64_t, int32_t> kids;
};

struct Failure {
  int code;
  std::string msg;
};

class Cache {
 public:
  explicit Cache(const cfa_kv_cache_config &c) : cfg_(c) {
    blocks_.resize(cfg_.total_gpu_blocks);
    free_.reserve(cfg_.total_gpu_blocks);
    for (size_t i = cfg_.total_gpu_blocks; i-- > 0;) free_.push_back((int32_t)i);
    nodes_.emplace_back();  // root
    nodes_[0].live = true;
  }

  std::mutex mu;

  // Chained hash of one block of tokens (paged_kv_cache.cpp:80-88): the
  // std::hash of an int32 is its value widened to 64 bits.
  static uint64_t block_hash(const int32_t *t, uint32_t n, uint64_t parent) {
    uint64_t h = parent ^ 0x9e3779b97f4a7c15ull;
    for (uint32_t i = 0; i < n; ++i)
      h ^= (uint64_t)(int64_t)t[i] + 0x9e3779b9ull + (h << 6) + (h >> 2);
    return h;
  }

  uint32_t register_sequence(uint64_t seq, const int32_t *tok, uint32_t n) {
    if (tables_.count(seq)) return 0;  // already registered: a no-op
    const uint32_t bs = cfg_.block_size;
    const uint32_t full = n / bs;
    // Longest run of leading full blocks present in the trie (no side effects
    // yet, so that a failed call leaves every table and page as it was).
    std::vector<int32_t> hit_nodes;
    std::vector<uint64_t> hashes(full);
    uint64_t parent_hash = 0;
    int32_t at = 0;  // trie node
    size_t hits_cached = 0;
    for (uint32_t b = 0; b < full; ++b) {
      hashes[b] = block_hash(tok + (size_t)b * bs, bs, parent_hash);
      parent_hash = hashes[b];
      if (!cfg_.enable_prefix_caching || hit_nodes.size() != b) continue;
      auto it = nodes_[at].kids.find(hashes[b]);
      if (it == nodes_[at].kids.end()) continue;
      hit_nodes.push_back(it->second);
      hits_cached += blocks_[nodes_[it->second].block].cached ? 1 : 0;
      at = it->second;
    }
    const uint32_t nmatch = (uint32_t)hit_nodes.size();
    const uint32_t tail = n - full * bs;
    const size_t needed = (full - nmatch) + ((tail > 0 || full == 0) ? 1 : 0);
    if (needed > free_.size() + lru_size_ - hits_cached) throw out_of_pages();

    std::vector<int32_t> table;
    table.reserve(full + 1);
    for (int32_t nd : hit_nodes) {
      const int32_t id = nodes_[nd].block;
      Block &blk = blocks_[id];
      ++blk.refs;
      if (blk.cached) {
        blk.cached = false;
        lru_unlink(id);
      }
      table.push_back(id);
      ++hits_;
    }
    // the rest of the full blocks: new pages, registered in the trie
    for (uint32_t b = nmatch; b < full; ++b) {
      const int32_t id = take_block();
      Block &blk = blocks_[id];
      blk.filled = bs;
      blk.hash = hashes[b];
      if (cfg_.enable_prefix_caching) {
        blk.node = new_node(hashes[b], id, at);
        at = blk.node;
      }
      table.push_back(id);
      ++misses_;
    }
    if (tail > 0 || table.empty()) {
      const int32_t id = take_block();
      blocks_[id].filled = tail;
      table.push_back(id);
    }
    tables_[seq] = std::move(table);
    return nmatch * bs;
  }

  // A page shared with another table (after fork) that is about to change
  // is first copied: the sequence gets a private page holding its first
  // `slots` tokens, and the device copy is queued for the caller.
  void make_private_last(std::vector<int32_t> &table, uint32_t slots) {
    const int32_t src = table.back();
    const int32_t dst = take_block();
    blocks_[dst].filled = slots;
    --blocks_[src].refs;  // still held by the other tables
    table.back() = dst;
    if (slots) copies_.push_back(cfa_kv_page_copy{src, dst, (int32_t)slots});
  }

  void append(uint64_t seq, uint32_t n) {
    std::vector<int32_t> &table = table_of(seq);
    if (n == 0) return;
    const uint32_t bs = cfg_.block_size;
    const uint32_t filled = blocks_[table.back()].filled;
    const uint32_t room = bs - filled;
    const bool cow = room > 0 && blocks_[table.back()].refs > 1;
    const size_t extra = n > room ? (n - room + (size_t)bs - 1) / bs : 0;
    if ((cow ? 1 : 0) + extra > free_.size() + lru_size_) throw out_of_pages();
    if (cow) make_private_last(table, filled);
    Block &last = blocks_[table.back()];
    if (n <= room) {
      last.filled += n;
      return;
    }
    uint32_t rest = n - room;
    last.filled = bs;
    while (rest > 0) {
      const int32_t id = take_block();
      const uint32_t add = std::min(rest, bs);
      blocks_[id].filled = add;
      table.push_back(id);
      rest -= add;
    }
  }

  void unregister(uint64_t seq) {
    auto it = tables_.find(seq);
    if (it == tables_.end()) return;
    for (int32_t id : it->second) release(id);
    tables_.erase(it);
  }

  // The child shares every page of the parent.  A child id that is already
  // registered first releases its own pages (the reference overwrites its
  // table and so never releases them).
  void fork(uint64_t parent, uint64_t child) {
    if (parent == child) throw Failure{CFA_ERR_ARG, "fork_sequence: parent and child are the same id"};
    const std::vector<int32_t> src = table_of(parent);
    for (int32_t id : src) ++blocks_[id].refs;
    unregister(child);
    tables_[child] = src;
  }

  // Keep the first `len` tokens of seq (at least one page stays); pages past
  // it are released.  A cut inside a page that another table shares gives
  // this sequence a private copy of the kept part.
  void truncate(uint64_t seq, uint32_t len) {
    std::vector<int32_t> &table = table_of(seq);
    const uint32_t cur = context_length(table);
    if (len > cur) throw Failure{CFA_ERR_ARG, "truncate_sequence: new length exceeds the sequence"};
    const uint32_t bs = cfg_.block_size;
    const size_t keep = std::max<size_t>(1, (len + bs - 1) / bs);
    const uint32_t last_fill = len - (uint32_t)(keep - 1) * bs;
    const int32_t cut = table[keep - 1];
    const bool changes = last_fill != blocks_[cut].filled;
    const bool cow = changes && blocks_[cut].refs > 1;
    if (cow) {
      // pages released below become free or evictable first
      size_t avail = free_.size() + lru_size_;
      for (size_t i = keep; i < table.size(); ++i) avail += blocks_[table[i]].refs == 1 ? 1 : 0;
      if (avail == 0) throw out_of_pages();
    }
    for (size_t i = keep; i < table.size(); ++i) release(table[i]);
    table.resize(keep);
    if (cow) {
      make_private_last(table, last_fill);
    } else if (changes) {
      if (blocks_[cut].hash != 0) forget_prefix(cut);  // no longer a whole prompt block
      blocks_[cut].filled = last_fill;
    }
  }

  size_t pop_copies(cfa_kv_page_copy *out, size_t cap) {
    const size_t k = std::min(cap, copies_.size());
    std::copy(copies_.begin(), copies_.begin() + k, out);
    copies_.erase(copies_.begin(), copies_.begin() + k);
    return k;
  }
  size_t pending_copies() const { return copies_.size(); }

  uint32_t context_length(const std::vector<int32_t> &t) const {
    return (uint32_t)(t.size() - 1) * cfg_.block_size + blocks_[t.back()].filled;
  }

  std::vector<int32_t> &table_of(uint64_t seq) {
    auto it = tables_.find(seq);
    if (it == tables_.end())
      throw Failure{CFA_ERR_STATE, "Sequence ID " + std::to_string(seq) + " not registered"};
    return it->second;
  }

  void stats(cfa_kv_cache_stats *s) const {
    std::memset(s, 0, sizeof(*s));
    s->total_blocks = cfg_.total_gpu_blocks;
    s->free_blocks = free_.size();
    s->cached_prefix_blocks = lru_size_;
    s->allocated_blocks = s->total_blocks - s->free_blocks - s->cached_prefix_blocks;
    const size_t per_block = bytes_per_block();
    s->total_memory_bytes = s->total_blocks * per_block * 2;
    s->used_memory_bytes = (s->allocated_blocks + s->cached_prefix_blocks) * per_block * 2;
    s->pool_utilization_ratio =
        s->total_blocks ? (double)(s->total_blocks - s->free_blocks) / (double)s->total_blocks : 0.0;
    s->active_sequences_count = (uint32_t)tables_.size();
    s->prefix_cache_hits = hits_;
    s->prefix_cache_misses = misses_;
    s->lru_evictions_count = evictions_;
  }

  size_t layer_block_bytes() const {
    return (size_t)cfg_.num_kv_heads * cfg_.block_size * cfg_.head_dim * cfg_.element_size_bytes;
  }
  size_t bytes_per_block() const { return cfg_.num_layers * layer_block_bytes(); }

  const cfa_kv_cache_config &config() const { return cfg_; }
  const Block &block(int32_t id) const { return blocks_[id]; }

 private:
  Failure out_of_pages() const {
    return Failure{CFA_ERR_OUT_OF_PAGES, "OutOfPagesException: Physical KV Cache pool exhausted! All " +
                                             std::to_string(cfg_.total_gpu_blocks) +
                                             " blocks in active use."};
  }

  // A free page, evicting the least recently released prefix page when none
  // is free (paged_kv_cache.cpp:101-144).  Callers check beforehand that
  // enough pages are free or evictable.
  int32_t take_block() {
    if (free_.empty() && !evict_one()) throw out_of_pages();
    const int32_t id = free_.back();
    free_.pop_back();
    Block &b = blocks_[id];
    b.refs = 1;
    b.filled = 0;
    b.cached = false;
    b.hash = 0;  // only set on free pages when prefix caching is off
    return id;
  }

  void release(int32_t id) {
    if (id < 0 || (size_t)id >= blocks_.size()) return;
    Block &b = blocks_[id];
    if (b.refs == 0) return;
    if (--b.refs > 0) return;
    if (cfg_.enable_prefix_caching && b.hash != 0) {
      b.cached = true;
      lru_push_front(id);
    } else {
      b.filled = 0;
      free_.push_back(id);
    }
  }

  // The least recently released cached page goes back to the free list.
  bool evict_one() {
    for (int32_t id = lru_tail_; id >= 0; id = blocks_[id].prev) {
      Block &b = blocks_[id];
      if (b.refs != 0) continue;
      lru_unlink(id);
      forget_prefix(id);
      b.cached = false;
      b.filled = 0;
      free_.push_back(id);
      ++evictions_;
      return true;
    }
    return false;
  }

  // Drop a page's prefix identity: its trie node leaves its parent.
  void forget_prefix(int32_t id) {
    Block &b = blocks_[id];
    if (b.node > 0) {
      Node &nd = nodes_[b.node];
      if (nd.parent >= 0) {
        auto &kids = nodes_[nd.parent].kids;
        auto it = kids.find(nd.hash);
        if (it != kids.end() && it->second == b.node) kids.erase(it);
      }
      nd.live = false;
      nd.block = -1;
      free_nodes_.push_back(b.node);
    }
    b.node = -1;
    b.hash = 0;
  }

  int32_t new_node(uint64_t h, int32_t block, int32_t parent) {
    int32_t id;
    if (!free_nodes_.empty()) {
      id = free_nodes_.back();
      free_nodes_.pop_back();
      nodes_[id] = Node{};
    } else {
      id = (int32_t)nodes_.size();
      nodes_.emplace_back();
    }
    Node &nd = nodes_[id];
    nd.hash = h;
    nd.block = block;
    nd.parent = parent;
    nd.live = true;
    nodes_[parent].kids[h] = id;
    return id;
  }

  void lru_push_front(int32_t id) {
    Block &b = blocks_[id];
    b.prev = -1;
    b.next = lru_head_;
    if (lru_head_ >= 0) blocks_[lru_head_].prev = id;
    lru_head_ = id;
    if (lru_tail_ < 0) lru_tail_ = id;
    ++lru_size_;
  }

  void lru_unlink(int32_t id) {
    Block &b = blocks_[id];
    if (b.prev >= 0) blocks_[b.prev].next = b.next; else lru_head_ = b.next;
    if (b.next >= 0) blocks_[b.next].prev = b.prev; else lru_tail_ = b.prev;
    b.prev = b.next = -1;
    --lru_size_;
  }

  cfa_kv_cache_config cfg_;
  std::vector<Block> blocks_;
  std::vector<int32_t> free_;
  int32_t lru_head_ = -1, lru_tail_ = -1;
  size_t lru_size_ = 0;
  std::vector<Node> nodes_;
  std::vector<int32_t> free_nodes_;
  std::unordered_map<uint64_t, std::vector<int32_t>> tables_;
  std::vector<cfa_kv_page_copy> copies_;
  uint64_t hits_ = 0, misses_ = 0, evictions_ = 0;
};

}  // namespace kvc
}  // namespace cfa

struct cfa_kv_cache {
  cfa::kvc::Cache impl;
};

using cfa::kvc::Failure;

// Runs f() under the cache's lock, mapping failures to error codes.
template <class F>
static int guarded(cfa_kv_cache *c, F &&f) {
  cfa::abi::clear_error();
  if (!c) return cfa::abi::fail_arg("null cache handle");
  try {
    std::lock_guard<std::mutex> lock(c->impl.mu);
    f(c->impl);
    return CFA_OK;
  } catch (const Failure &e) {
    return cfa::abi::fail_code(e.code, e.msg.c_str());
  } catch (const std::bad_alloc &) {
    return cfa::abi::fail_code(CFA_ERR_STATE, "out of host memory");
  }
}

extern "C" int cfa_kv_cache_create(const cfa_kv_cache_config *config, cfa_kv_cache **out) {
  cfa::abi::clear_error();
  if (!config || !out) return cfa::abi::fail_arg("null argument");
  *out = nullptr;
  if (config->block_size == 0 || config->total_gpu_blocks == 0 || config->num_layers == 0 ||
      config->num_kv_heads == 0 || config->head_dim == 0 || config->element_size_bytes == 0)
    return cfa::abi::fail_arg("KVCacheConfig sizes must be positive");
  if (config->total_gpu_blocks > 0x7fffffffull)
    return cfa::abi::fail_arg("total_gpu_blocks must fit an int32 block id");
  cfa_kv_cache *c = new (std::nothrow) cfa_kv_cache{cfa::kvc::Cache(*config)};
  if (!c) return cfa::abi::fail_code(CFA_ERR_STATE, "out of host memory");
  *out = c;
  return CFA_OK;
}

extern "C" void cfa_kv_cache_destroy(cfa_kv_cache *cache) { delete cache; }

extern "C" int cfa_kv_cache_register_sequence(cfa_kv_cache *cache, uint64_t sequence_id,
                                              const int32_t *prompt_tokens, int64_t n_tokens,
                                              uint32_t *matched_tokens) {
  if (n_tokens < 0 || (n_tokens > 0 && !prompt_tokens)) {
    cfa::abi::clear_error();
    return cfa::abi::fail_arg("bad prompt tokens");
  }
  return guarded(cache, [&](cfa::kvc::Cache &c) {
    const uint32_t m = c.register_sequence(sequence_id, prompt_tokens, (uint32_t)n_tokens);
    if (matched_tokens) *matched_tokens = m;
  });
}

extern "C" int cfa_kv_cache_append_tokens(cfa_kv_cache *cache, uint64_t sequence_id,
                                          uint32_t num_tokens) {
  return guarded(cache, [&](cfa::kvc::Cache &c) { c.append(sequence_id, num_tokens); });
}

extern "C" int cfa_kv_cache_unregister_sequence(cfa_kv_cache *cache, uint64_t sequence_id) {
  return guarded(cache, [&](cfa::kvc::Cache &c) { c.unregister(sequence_id); });
}

extern "C" int cfa_kv_cache_fork_sequence(cfa_kv_cache *cache, uint64_t parent_sequence_id,
                                          uint64_t child_sequence_id) {
  return guarded(cache, [&](cfa::kvc::Cache &c) { c.fork(parent_sequence_id, child_sequence_id); });
}

extern "C" int cfa_kv_cache_truncate_sequence(cfa_kv_cache *cache, uint64_t sequence_id,
                                              uint32_t new_length) {
  return guarded(cache, [&](cfa::kvc::Cache &c) { c.truncate(sequence_id, new_length); });
}

extern "C" int cfa_kv_cache_context_length(cfa_kv_cache *cache, uint64_t sequence_id,
                                           uint32_t *length) {
  return guarded(cache, [&](cfa::kvc::Cache &c) {
    const uint32_t n = c.context_length(c.table_of(sequence_id));
    if (length) *length = n;
  });
}

extern "C" int cfa_kv_cache_get_block_table(cfa_kv_cache *cache, uint64_t sequence_id,
                                            int32_t *out, int64_t capacity, int64_t *n_blocks) {
  return guarded(cache, [&](cfa::kvc::Cache &c) {
    const std::vector<int32_t> &t = c.table_of(sequence_id);
    if (n_blocks) *n_blocks = (int64_t)t.size();
    if (out) {
      const size_t k = std::min<size_t>(t.size(), capacity > 0 ? (size_t)capacity : 0);
      std::copy(t.begin(), t.begin() + k, out);
    }
  });
}

extern "C" int cfa_kv_cache_prepare_batch(cfa_kv_cache *cache, const uint64_t *sequence_ids,
                                          int batch_size, int32_t *host_block_tables,
                                          int32_t *host_context_lens, int64_t host_capacity,
                                          int32_t *dev_block_tables, int32_t *dev_context_lens,
                                          int64_t dev_capacity, int32_t *max_blocks_out,
                                          void *stream) {
  int max_blocks = 0;
  int rc = guarded(cache, [&](cfa::kvc::Cache &c) {
    const cfa_kv_cache_config &cfg = c.config();
    if (batch_size < 0 || (batch_size > 0 && (!sequence_ids || !host_block_tables || !host_context_lens)))
      throw Failure{CFA_ERR_ARG, "bad batch arguments"};
    if ((size_t)batch_size > cfg.max_supported_batch_size)
      throw Failure{CFA_ERR_RANGE, "Requested batch size exceeds max_supported_batch_size"};
    size_t mb = 0;
    for (int i = 0; i < batch_size; ++i) {
      const std::vector<int32_t> &t = c.table_of(sequence_ids[i]);
      mb = std::max(mb, t.size());
    }
    if (mb > cfg.max_blocks_per_sequence)
      throw Failure{CFA_ERR_RANGE, "Sequence blocks count exceeds max_blocks_per_sequence limit"};
    if ((int64_t)(mb * (size_t)batch_size) > host_capacity)
      throw Failure{CFA_ERR_ARG, "host block-table buffer too small"};
    for (int i = 0; i < batch_size; ++i) {
      const std::vector<int32_t> &t = c.table_of(sequence_ids[i]);
      int32_t *row = host_block_tables + (size_t)i * mb;
      std::fill(row, row + mb, -1);
      std::copy(t.begin(), t.end(), row);
      host_context_lens[i] = (int32_t)c.context_length(t);
    }
    max_blocks = (int)mb;
  });
  if (rc != CFA_OK) return rc;
  if (max_blocks_out) *max_blocks_out = max_blocks;
  if (dev_block_tables && dev_context_lens && batch_size > 0) {
    const size_t tb = (size_t)batch_size * max_blocks * sizeof(int32_t);
    if ((int64_t)((size_t)batch_size * max_blocks) > dev_capacity)
      return cfa::abi::fail_arg("device block-table buffer too small");
    hipStream_t st = (hipStream_t)stream;
    if (hipError_t e = hipMemcpyAsync(dev_block_tables, host_block_tables, tb, hipMemcpyHostToDevice, st))
      return cfa::abi::fail_hip(e, "prepare_batch_metadata block tables");
    if (hipError_t e = hipMemcpyAsync(dev_context_lens, host_context_lens,
                                      (size_t)batch_size * sizeof(int32_t), hipMemcpyHostToDevice, st))
      return cfa::abi::fail_hip(e, "prepare_batch_metadata context lengths");
  }
  return CFA_OK;
}

extern "C" int cfa_kv_cache_get_stats(cfa_kv_cache *cache, cfa_kv_cache_stats *out) {
  if (!out) {
    cfa::abi::clear_error();
    return cfa::abi::fail_arg("null stats pointer");
  }
  return guarded(cache, [&](cfa::kvc::Cache &c) { c.stats(out); });
}

extern "C" int cfa_kv_cache_pop_page_copies(cfa_kv_cache *cache, cfa_kv_page_copy *out,
                                           int64_t capacity, int64_t *count) {
  return guarded(cache, [&](cfa::kvc::Cache &c) {
    size_t k;
    if (out && capacity > 0)
      k = c.pop_copies(out, (size_t)capacity);
    else
      k = c.pending_copies();
    if (count) *count = (int64_t)k;
  });
}

extern "C" int cfa_kv_cache_block_info(cfa_kv_cache *cache, int32_t block_id, uint32_t *ref_count,
                                       uint32_t *tokens_filled, int32_t *is_cached) {
  return guarded(cache, [&](cfa::kvc::Cache &c) {
    if (block_id < 0 || (size_t)block_id >= c.config().total_gpu_blocks)
      throw Failure{CFA_ERR_RANGE, "block id out of range"};
    const cfa::kvc::Block &b = c.block(block_id);
    if (ref_count) *ref_count = b.refs;
    if (tokens_filled) *tokens_filled = b.filled;
    if (is_cached) *is_cached = b.cached ? 1 : 0;
  });
}
