// cfg5's host-side fork and rollback driven through the allocator's C ABI alone (no
// Python): 16 requests of context 4096 (2048 shared) take a 5-token verify pass; then 8
// of them fork 3 tokens before their end (copy on write of the partly filled tail page,
// crates/yaxus-model/src/kv.rs:277-326) and all 24 sequences roll back a count in [0, 5]
// (kv.rs:265-273), as a native speculative-decoding engine does after a verify step
// (crates/yaxus-model/src/engine/mod.rs:560-636). Times the fork-and-rollback part (and
// the copies drained from the cache) and prints one JSON line.
//
// Usage: fork_rollback [repetitions]
#include <algorithm>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "../../include/yaxus_kv_cache.h"

namespace {

void die(const char* what) {
  std::fprintf(stderr, "%s: %s\n", what, yx_cache_last_error());
  std::exit(1);
}
#define KVCHECK(x) \
  do {             \
    if ((x) != YX_OK) die(#x); \
  } while (0)

double median(std::vector<double> v) {
  std::sort(v.begin(), v.end());
  return v.empty() ? 0.0 : v[v.size() / 2];
}

}  // namespace

int main(int argc, char** argv) {
  const int reps = argc > 1 ? std::atoi(argv[1]) : 50;
  const size_t B = 16, page = 16, pool = 8192, shared = 2048, ctx = 4096, draft = 5;
  std::vector<double> fork_us, back_us, all_us;
  size_t ncopies = 0;
  uint32_t rng = 12345u;  // rollback counts in [0, 5]
  for (int r = 0; r < reps; ++r) {
    yx_cache* c = nullptr;
    KVCHECK(yx_cache_create(pool, 1 << 20, page, &c));
    const uint64_t base = yx_cache_new_seq(c);
    {
      std::vector<uint32_t> toks(shared, 1);
      const size_t n = shared;
      KVCHECK(yx_cache_append(c, 1, &base, &n, toks.data()));
    }
    std::vector<uint64_t> seqs(B);
    for (auto& s : seqs) KVCHECK(yx_cache_fork(c, base, shared, &s));
    {
      std::vector<size_t> counts(B, ctx - shared - draft);
      std::vector<uint32_t> toks(B * (ctx - shared - draft), 1);
      KVCHECK(yx_cache_append(c, B, seqs.data(), counts.data(), toks.data()));
      std::vector<size_t> dc(B, draft);
      std::vector<uint32_t> dt(B * draft, 2);
      KVCHECK(yx_cache_append(c, B, seqs.data(), dc.data(), dt.data()));
    }
    std::vector<yx_page_copy> copies(yx_cache_pending_copies(c) + 64);
    yx_cache_take_copies(c, copies.data(), copies.size());

    const auto t0 = std::chrono::steady_clock::now();
    std::vector<uint64_t> all(seqs);
    for (size_t i = 0; i < 8; ++i) {
      uint64_t f = 0;
      KVCHECK(yx_cache_fork(c, seqs[i], yx_cache_seq_len(c, seqs[i]) - 3, &f));
      all.push_back(f);
    }
    const size_t nc = yx_cache_pending_copies(c);
    copies.resize(std::max(copies.size(), nc));
    ncopies = yx_cache_take_copies(c, copies.data(), nc);
    const auto t1 = std::chrono::steady_clock::now();
    for (uint64_t s : all) {
      rng = rng * 1664525u + 1013904223u;
      const size_t n = (rng >> 16) % (draft + 1);
      KVCHECK(yx_cache_truncate(c, s, yx_cache_seq_len(c, s) - n));
    }
    const auto t2 = std::chrono::steady_clock::now();
    fork_us.push_back(std::chrono::duration<double, std::micro>(t1 - t0).count());
    back_us.push_back(std::chrono::duration<double, std::micro>(t2 - t1).count());
    all_us.push_back(std::chrono::duration<double, std::micro>(t2 - t0).count());
    yx_cache_destroy(c);
  }
  std::printf(
      "{\"host_fork_rollback_us_median\": %.2f, \"fork_us_median\": %.2f, "
      "\"rollback_us_median\": %.2f, \"forks\": 8, \"rollbacks\": 24, \"copies\": %zu, "
      "\"repetitions\": %d}\n",
      median(all_us), median(fork_us), median(back_us), ncopies, reps);
  return 0;
}
