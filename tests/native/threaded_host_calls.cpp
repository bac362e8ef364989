// threaded_host_calls.cpp -- concurrent host calls into libcfa.so for the
// ThreadSanitizer run (CPU only: no call here touches a GPU).
//
// Eight threads share one paged-KV page table: register with shared prompt
// prefixes, append, fork, truncate, stats, batch staging into host buffers,
// unregister -- the calls the reference serialises with its mutex
// (paged_kv_cache.h:174).  Each thread also drives its own host RNG stream
// and provokes argument errors, whose messages are thread-local.  Exits 0
// when every call returned an expected code and the table ends empty.
#include <atomic>
#include <cstdio>
#include <random>
#include <thread>
#include <vector>

#include "cudaforge_amd.h"

static std::atomic<int> g_bad{0};

static void expect(bool ok, const char *what, int tid) {
  if (!ok) {
    std::fprintf(stderr, "thread %d: %s\n", tid, what);
    g_bad.fetch_add(1);
  }
}

static void worker(cfa_kv_cache *kv, int tid) {
  std::mt19937 rng(tid);
  cfa_rng *r = cfa_rng_create(1000 + tid);
  float draws[8];
  std::vector<int32_t> host_tables(64), host_lens(1);
  for (int it = 0; it < 300; ++it) {
    const uint64_t sid = (uint64_t)tid * 100000 + it;
    std::vector<int32_t> prompt(1 + rng() % 70, (int32_t)(rng() % 4));
    uint32_t matched = 0;
    int rc = cfa_kv_cache_register_sequence(kv, sid, prompt.data(), (int64_t)prompt.size(),
                                            &matched);
    if (rc == CFA_ERR_OUT_OF_PAGES) continue;
    expect(rc == CFA_OK, "register", tid);
    rc = cfa_kv_cache_append_tokens(kv, sid, 1 + rng() % 40);
    expect(rc == CFA_OK || rc == CFA_ERR_OUT_OF_PAGES, "append", tid);
    if (rng() % 3 == 0) {
      rc = cfa_kv_cache_fork_sequence(kv, sid, sid + 50000);
      expect(rc == CFA_OK || rc == CFA_ERR_OUT_OF_PAGES, "fork", tid);
      if (rc == CFA_OK) {
        rc = cfa_kv_cache_append_tokens(kv, sid + 50000, 1 + rng() % 20);
        expect(rc == CFA_OK || rc == CFA_ERR_OUT_OF_PAGES, "append child", tid);
        expect(cfa_kv_cache_unregister_sequence(kv, sid + 50000) == CFA_OK, "unregister child",
               tid);
      }
    }
    int64_t pending = 0;
    expect(cfa_kv_cache_pop_page_copies(kv, nullptr, 0, &pending) == CFA_OK, "pending", tid);
    std::vector<cfa_kv_page_copy> copies((size_t)pending + 1);
    expect(cfa_kv_cache_pop_page_copies(kv, copies.data(), (int64_t)copies.size(), &pending) ==
               CFA_OK,
           "pop", tid);
    uint32_t len = 0;
    expect(cfa_kv_cache_context_length(kv, sid, &len) == CFA_OK, "length", tid);
    const uint32_t cut = len > 30 ? len - (uint32_t)(rng() % 30) : len;
    rc = cfa_kv_cache_truncate_sequence(kv, sid, cut > 0 ? cut : 1);
    expect(rc == CFA_OK || rc == CFA_ERR_OUT_OF_PAGES, "truncate", tid);
    int32_t maxb = 0;
    rc = cfa_kv_cache_prepare_batch(kv, &sid, 1, host_tables.data(), host_lens.data(), 64,
                                    nullptr, nullptr, 0, &maxb, nullptr);
    expect(rc == CFA_OK, "prepare", tid);
    cfa_kv_cache_stats st;
    expect(cfa_kv_cache_get_stats(kv, &st) == CFA_OK, "stats", tid);
    expect(cfa_kv_cache_unregister_sequence(kv, sid) == CFA_OK, "unregister", tid);
    expect(cfa_rng_peek(r, 8, draws) == CFA_OK && cfa_rng_advance(r, 3) == CFA_OK, "rng", tid);
    expect(cfa_kv_cache_truncate_sequence(nullptr, 0, 0) == CFA_ERR_ARG, "null cache", tid);
    expect(cfa_last_error()[0] != '\0', "thread-local message", tid);
  }
  cfa_rng_destroy(r);
}

int main() {
  cfa_kv_cache_config cfg{};
  cfg.num_layers = 1;
  cfg.num_kv_heads = 1;
  cfg.head_dim = 8;
  cfg.block_size = 16;
  cfg.element_size_bytes = 2;
  cfg.total_gpu_blocks = 512;
  cfg.enable_prefix_caching = 1;
  cfg.max_supported_batch_size = 8;
  cfg.max_blocks_per_sequence = 64;
  cfa_kv_cache *kv = nullptr;
  if (cfa_kv_cache_create(&cfg, &kv) != CFA_OK) return 2;
  std::vector<std::thread> ts;
  for (int t = 0; t < 8; ++t) ts.emplace_back(worker, kv, t);
  for (auto &t : ts) t.join();
  cfa_kv_cache_stats st;
  cfa_kv_cache_get_stats(kv, &st);
  std::printf("threads done: active=%u free=%llu bad=%d\n", st.active_sequences_count,
              (unsigned long long)st.free_blocks, g_bad.load());
  cfa_kv_cache_destroy(kv);
  return (g_bad.load() == 0 && st.active_sequences_count == 0) ? 0 : 1;
}
