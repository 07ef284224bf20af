// Random operation sequences through the block manager's C ABI, built with
// AddressSanitizer and UndefinedBehaviorSanitizer by tests/test_sanitizers.py
// (host code only: block_manager.cpp has no device code).  Every call's return
// code must be one the header documents for it, and after every step the
// bookkeeping must add up:
//   - per GPU engine: free + moving + blocks held by tables == the space's
//     size, and no block is both free and held, or held twice;
//   - per CPU shape: no block id is held twice;
// through suspended calls (AEGKV_RECLAIM_PENDING), their resumption after the
// pending moves are completed, cancellation, and frees of busy requests.
// Usage: bm_fuzz SEED STEPS
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <iterator>
#include <map>
#include <random>
#include <set>
#include <string>
#include <vector>

#include "../../include/aegkv.h"

namespace {

#define CHECK(cond)                                                            \
  do {                                                                         \
    if (!(cond)) {                                                             \
      std::fprintf(stderr, "check failed at line %d: %s\n", __LINE__, #cond); \
      std::exit(2);                                                            \
    }                                                                          \
  } while (0)

struct Engine {
  int32_t id, shape;
  int64_t size;
};

const Engine kEngines[] = {{0, 0, 40}, {1, 1, 28}, {2, 0, 24}};
const uint64_t kShapeBytes[] = {4096, 6144};
const int64_t kSlabs = 6, kSlabBytes = 64 * 1024;

struct Req {
  int32_t loc, shape;
};

aegkv_block_manager* bm = nullptr;
std::map<int64_t, Req> live;  // requests the driver believes hold a table
std::mt19937_64 rng;
int64_t next_id = 1;
bool suspended = false;
std::vector<int64_t> op_ids;  // the requests of the suspended call
std::map<std::string, long> seen;  // how often each path ran

int64_t rnd(int64_t n) { return (int64_t)(rng() % (uint64_t)n); }

std::vector<int64_t> table_of(int64_t r, int32_t* loc, int32_t* shape) {
  int64_t n = 0;
  int rc = aegkv_bm_table(bm, r, loc, shape, &n, nullptr, 0);
  CHECK(rc == AEGKV_OK);
  std::vector<int64_t> t(n);
  if (n) CHECK(aegkv_bm_table(bm, r, loc, shape, &n, t.data(), n) == AEGKV_OK);
  return t;
}

// the tables the library holds agree with the driver's view and add up
void check_books() {
  std::map<int32_t, std::set<int64_t>> held_gpu;
  std::map<int32_t, std::set<int64_t>> held_cpu;
  for (auto& kv : live) {
    int32_t loc = 0, shape = 0;
    const std::vector<int64_t> t = table_of(kv.first, &loc, &shape);
    CHECK(loc == kv.second.loc && shape == kv.second.shape);
    auto& held = loc == AEGKV_BM_CPU ? held_cpu[shape] : held_gpu[loc];
    for (int64_t b : t) {
      CHECK(b >= 0);
      CHECK(held.insert(b).second);  // no block held twice
    }
  }
  for (const Engine& e : kEngines) {
    int64_t n_free = 0, n_moving = 0, n_slabs = 0, n_used = 0;
    CHECK(aegkv_bm_stats(bm, e.id, e.shape, &n_free, &n_moving, &n_slabs, &n_used) == AEGKV_OK);
    std::vector<int64_t> fl(e.size + 1);
    int64_t n = 0;
    CHECK(aegkv_bm_free_list(bm, e.id, e.shape, fl.data(), (int64_t)fl.size(), &n) == AEGKV_OK);
    CHECK(n == n_free);
    for (int64_t i = 0; i < n; ++i) {
      CHECK(fl[i] >= 0 && fl[i] < e.size);
      CHECK(!held_gpu[e.id].count(fl[i]));
    }
    for (int64_t b : held_gpu[e.id]) CHECK(b < e.size);
    if (!suspended) CHECK(n_free + n_moving + (int64_t)held_gpu[e.id].size() == e.size);
  }
}

// complete every pending move out of (loc, shape) up to `serial`, then resume
// or cancel the suspended call
void settle() {
  int64_t op = 0, serial = 0;
  int32_t loc = 0, shape = 0;
  CHECK(aegkv_bm_pending(bm, &op, &loc, &shape, &serial) == AEGKV_OK);
  CHECK(aegkv_bm_complete_moves(bm, loc, shape, serial) == AEGKV_OK);
  if (loc == AEGKV_BM_CPU) CHECK(aegkv_bm_reclaim_slabs(bm) == AEGKV_OK);
  int64_t s = 0, nb = 0;
  int32_t in = 0, eng = 0;
  const bool cancel = rnd(4) == 0;
  const int rc = cancel ? aegkv_bm_cancel(bm, op) : aegkv_bm_resume(bm, op, &s, &nb, &in, &eng);
  ++seen[cancel ? "cancel" : rc == AEGKV_OK ? "resume_ok" : "resume_short"];
  CHECK(rc == AEGKV_OK || rc == AEGKV_ERR_NO_SPACE || rc == AEGKV_RECLAIM_PENDING);
  suspended = rc == AEGKV_RECLAIM_PENDING;
  if (suspended) {  // short again: give up on it
    CHECK(aegkv_bm_pending(bm, &op, &loc, &shape, &serial) == AEGKV_OK);
    CHECK(aegkv_bm_cancel(bm, op) == AEGKV_OK);
    suspended = false;
  }
  // an allocation's new requests hold a table only once it went through
  for (int64_t id : op_ids) {
    int32_t l = 0, sh = 0;
    int64_t n = 0;
    if (aegkv_bm_table(bm, id, &l, &sh, &n, nullptr, 0) == AEGKV_OK) live[id] = Req{l, sh};
  }
  op_ids.clear();
}

// the driver's view of where every request lives, refreshed from the library
void refresh() {
  for (auto it = live.begin(); it != live.end();) {
    int32_t loc = 0, shape = 0;
    int64_t n = 0;
    const int rc = aegkv_bm_table(bm, it->first, &loc, &shape, &n, nullptr, 0);
    if (rc != AEGKV_OK) {
      it = live.erase(it);
      continue;
    }
    it->second = Req{loc, shape};
    ++it;
  }
}

void step() {
  switch (rnd(6)) {
    case 0:
    case 1: {  // allocate on an engine: new requests and ones already there
      const Engine& e = kEngines[rnd(3)];
      std::vector<int64_t> ids, need;
      for (int k = 0, n = 1 + (int)rnd(4); k < n; ++k) {
        int64_t id = next_id;
        if (rnd(2) && !live.empty()) {
          auto it = live.begin();
          std::advance(it, rnd((int64_t)live.size()));
          id = it->first;
        }
        bool dup = false;
        for (int64_t x : ids) dup |= x == id;
        if (dup) continue;
        int64_t have = 0;
        if (id == next_id) {
          ++next_id;
        } else {
          int32_t loc = 0, shape = 0;
          have = (int64_t)table_of(id, &loc, &shape).size();
        }
        ids.push_back(id);
        need.push_back(have + (have ? rnd(4) : 1 + rnd(9)));  // a table only grows
      }
      const int rc = aegkv_bm_allocate(bm, e.id, ids.data(), need.data(), (int64_t)ids.size());
      CHECK(rc == AEGKV_OK || rc == AEGKV_ERR_NO_SPACE || rc == AEGKV_ERR_IN_USE ||
            rc == AEGKV_RECLAIM_PENDING);
      if (rc == AEGKV_OK)
        for (int64_t id : ids)
          if (!live.count(id)) live[id] = Req{e.id, e.shape};
      suspended = rc == AEGKV_RECLAIM_PENDING;
      if (suspended) op_ids = ids;
      ++seen[suspended ? "allocate_suspended" : rc == AEGKV_OK ? "allocate_ok" : "allocate_refused"];
      break;
    }
    case 2: {  // free one
      if (live.empty()) break;
      auto it = live.begin();
      std::advance(it, rnd((int64_t)live.size()));
      CHECK(aegkv_bm_free(bm, it->first) == AEGKV_OK);
      live.erase(it);
      break;
    }
    case 3:
    case 4: {  // move the requests of one location to CPU or to an engine of their shape
      if (live.empty()) break;
      auto it = live.begin();
      std::advance(it, rnd((int64_t)live.size()));
      const Req from = it->second;
      std::vector<int64_t> ids;
      for (auto& kv : live)
        if (kv.second.loc == from.loc && kv.second.shape == from.shape && rnd(2)) ids.push_back(kv.first);
      if (ids.empty()) ids.push_back(it->first);
      int32_t target = AEGKV_BM_CPU;
      if (from.loc == AEGKV_BM_CPU) {
        std::vector<int32_t> cand;
        for (const Engine& e : kEngines)
          if (e.shape == from.shape) cand.push_back(e.id);
        target = cand[rnd((int64_t)cand.size())];
      }
      int64_t serial = 0, nb = 0;
      int32_t in = 0, eng = 0;
      const int rc = aegkv_bm_move(bm, ids.data(), (int64_t)ids.size(), target, &serial, &nb,
                                   &in, &eng);
      CHECK(rc == AEGKV_OK || rc == AEGKV_ERR_NO_SPACE || rc == AEGKV_ERR_IN_USE ||
            rc == AEGKV_RECLAIM_PENDING);
      ++seen[rc == AEGKV_RECLAIM_PENDING ? (target == AEGKV_BM_CPU ? "swap_out_suspended" : "swap_in_suspended")
             : rc == AEGKV_OK ? (target == AEGKV_BM_CPU ? "swap_out_ok" : "swap_in_ok") : "move_refused"];
      if (rc == AEGKV_OK && serial >= 0) {
        std::vector<int64_t> src(nb), dst(nb), moved(ids.size());
        int64_t n_moved = 0;
        CHECK(aegkv_bm_move_ids(bm, src.data(), dst.data(), nb, moved.data(),
                                (int64_t)moved.size(), &n_moved) == AEGKV_OK);
        CHECK(n_moved >= 0 && n_moved <= (int64_t)ids.size());
      }
      suspended = rc == AEGKV_RECLAIM_PENDING;
      break;
    }
    default: {  // some pending moves finish
      const int32_t loc = rnd(4) == 0 ? AEGKV_BM_CPU : kEngines[rnd(3)].id;
      const int32_t shape = (int32_t)rnd(2);
      const int rc = aegkv_bm_complete_moves(bm, loc, shape, INT64_MAX);
      CHECK(rc == AEGKV_OK || rc == AEGKV_ERR_INVALID_ARG);
      if (loc == AEGKV_BM_CPU) CHECK(aegkv_bm_reclaim_slabs(bm) == AEGKV_OK);
      break;
    }
  }
  if (suspended) {
    refresh();
    check_books();
    if (rnd(3) == 0 && !live.empty()) {  // a free while the call waits (busy or not)
      auto it = live.begin();
      std::advance(it, rnd((int64_t)live.size()));
      CHECK(aegkv_bm_free(bm, it->first) == AEGKV_OK);
      ++seen["free_while_suspended"];
      live.erase(it);
      refresh();
      check_books();
    }
    settle();
  }
  refresh();
  check_books();
}

}  // namespace

int main(int argc, char** argv) {
  if (argc != 3) return 1;
  rng.seed(std::strtoull(argv[1], nullptr, 10));
  const long steps = std::strtol(argv[2], nullptr, 10);
  CHECK(aegkv_bm_create(kSlabs, kSlabBytes, &bm) == AEGKV_OK);
  for (int s = 0; s < 2; ++s) CHECK(aegkv_bm_define_shape(bm, s, kShapeBytes[s]) == AEGKV_OK);
  for (const Engine& e : kEngines)
    CHECK(aegkv_bm_register_gpu_space(bm, e.id, e.size, e.shape) == AEGKV_OK);
  for (long i = 0; i < steps; ++i) step();
  aegkv_bm_destroy(bm);
  std::printf("ok %ld steps, %zu live requests;", steps, live.size());
  for (auto& kv : seen) std::printf(" %s=%ld", kv.first.c_str(), kv.second);
  std::printf("\n");
  return 0;
}
