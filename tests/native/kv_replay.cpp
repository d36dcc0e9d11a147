// Replays a script of allocator operations through the C ABI of include/yaxus_kv_cache.h
// and prints every result and the allocator's state after each operation, one line
// each. tests/test_kv_sanitized.py builds this program together with
// yaxus_amd/csrc/kv_cache.cpp under AddressSanitizer and UndefinedBehaviorSanitizer,
// writes the script from a seeded random run of the allocator oracle
// (oracle/kv_oracle.py, a restatement of crates/yaxus-model/src/kv.rs), and compares
// the printed lines with the oracle's, so the allocator's index arithmetic (reserve,
// truncate, fork, copy-on-write, eviction) runs under the sanitizers on the same
// operations the differential test uses.
//
// Script (stdin), one operation per line:
//   create <pages> <max_pos> <page_size>
//   begin <n> <token>*n                    -> "R <id> <reused> C <src> <dst> ..." | "E C ..."
//   append <k> (<id> <n> <token>*n)*k      -> "R <ids> | <pos> | <slots> | <pt_off> | <pages> | <last> C ..." | "E C ..."
//   fork <id> <n>                          -> "R <id> C ..." | "E C ..."
//   truncate <id> <n>                      -> "R" | "E"
//   finish <id> / free <id>                -> "R"
// after each: "S <free pages> <refs of every page> L (<id> <len> P <pages> T <tokens>)*"
// over the live sequences (begun or forked, not yet finished or freed), in id order.
#include <cstdio>
#include <iostream>
#include <set>
#include <sstream>
#include <string>
#include <vector>

#include "../../include/yaxus_kv_cache.h"

namespace {

void copies(yx_cache* c, std::ostringstream& o) {
  o << " C";
  std::vector<yx_page_copy> cp(yx_cache_pending_copies(c));
  const size_t n = yx_cache_take_copies(c, cp.data(), cp.size());
  for (size_t i = 0; i < n; ++i) o << ' ' << cp[i].src << ' ' << cp[i].dst;
}

template <class T>
void list(std::ostringstream& o, const std::vector<T>& v) {
  for (const T& x : v) o << ' ' << x;
}

}  // namespace

int main() {
  yx_cache* c = nullptr;
  size_t pages = 0;
  std::set<uint64_t> live;
  std::string line;
  while (std::getline(std::cin, line)) {
    std::istringstream in(line);
    std::string op;
    if (!(in >> op)) continue;
    std::ostringstream o;
    if (op == "create") {
      size_t mp, ps;
      in >> pages >> mp >> ps;
      if (c) yx_cache_destroy(c);
      live.clear();
      if (yx_cache_create(pages, mp, ps, &c) != YX_OK) {
        std::printf("E create\n");
        return 1;
      }
      continue;
    } else if (op == "begin") {
      size_t n;
      in >> n;
      std::vector<uint32_t> t(n);
      for (auto& x : t) in >> x;
      uint64_t id = 0;
      size_t reused = 0;
      const int rc = yx_cache_begin(c, t.data(), n, &id, &reused);
      if (rc == YX_OK) {
        o << "R " << id << ' ' << reused;
        live.insert(id);
      } else {
        o << "E";
      }
      copies(c, o);
    } else if (op == "append") {
      size_t k;
      in >> k;
      std::vector<uint64_t> ids(k);
      std::vector<size_t> counts(k);
      std::vector<uint32_t> toks;
      for (size_t i = 0; i < k; ++i) {
        in >> ids[i] >> counts[i];
        for (size_t j = 0; j < counts[i]; ++j) {
          uint32_t x;
          in >> x;
          toks.push_back(x);
        }
      }
      const int rc = yx_cache_append(c, k, ids.data(), counts.data(), toks.data());
      if (rc == YX_OK) {
        const size_t rows = yx_cache_pass_rows(c), np = yx_cache_pass_npages(c), ni = yx_cache_pass_nitems(c);
        std::vector<uint32_t> tid(rows), pos(rows), slot(rows), off(rows), pg(np);
        std::vector<size_t> last(ni);
        yx_cache_pass_get(c, tid.data(), pos.data(), slot.data(), off.data(), pg.data(), last.data());
        o << "R";
        list(o, tid);
        o << " |";
        list(o, pos);
        o << " |";
        list(o, slot);
        o << " |";
        list(o, off);
        o << " |";
        list(o, pg);
        o << " |";
        list(o, last);
      } else {
        o << "E";
      }
      copies(c, o);
    } else if (op == "fork") {
      uint64_t id;
      size_t n;
      in >> id >> n;
      uint64_t out = 0;
      const int rc = yx_cache_fork(c, id, n, &out);
      if (rc == YX_OK) {
        o << "R " << out;
        live.insert(out);
      } else {
        o << "E";
      }
      copies(c, o);
    } else if (op == "truncate") {
      uint64_t id;
      size_t n;
      in >> id >> n;
      const int rc = yx_cache_truncate(c, id, n);
      o << (rc == YX_OK ? "R" : "E");
    } else if (op == "finish" || op == "free") {
      uint64_t id;
      in >> id;
      if (op == "finish")
        yx_cache_finish(c, id);
      else
        yx_cache_free_seq(c, id);
      live.erase(id);
      o << "R";
    } else {
      std::printf("E unknown op %s\n", op.c_str());
      return 1;
    }
    o << "\nS " << yx_cache_free_pages(c);
    for (size_t p = 0; p < pages; ++p) o << ' ' << yx_cache_page_refs(c, static_cast<uint32_t>(p));
    o << " L";
    for (uint64_t id : live) {
      const size_t len = yx_cache_seq_len(c, id);
      std::vector<uint32_t> pg(yx_cache_seq_pages(c, id, nullptr, 0)), tk(len);
      yx_cache_seq_pages(c, id, pg.data(), pg.size());
      yx_cache_seq_tokens(c, id, tk.data(), tk.size());
      o << ' ' << id << ' ' << len << " P";
      list(o, pg);
      o << " T";
      list(o, tk);
    }
    std::printf("%s\n", o.str().c_str());
  }
  if (c) yx_cache_destroy(c);
  return 0;
}
