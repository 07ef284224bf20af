// Native block manager: the bookkeeping of Aegaeon's node-wide KV block
// manager (aegaeon/aegaeon/block_manager.py), restated in C++ with the same
// allocation order, so the swap id lists it produces are the reference's.
//
//   GPU spaces (one per engine): a FIFO free list — allocations take from the
//     head, frees append to the tail (block_manager.py:525-526,703), which is
//     what scatters block tables over time.
//   CPU pool: num_slabs slabs of slab_bytes, each dedicated to one block shape
//     while it holds blocks; per-shape free deques, a stack of free slabs,
//     per-slab usage counts (:186-199,242-245,528-580) and slab reclaim
//     (:474-496).
//   Block tables: request -> (location, shape, blocks) (:104-111,237).
//   Moves: move_requests (:778-874) assigns target blocks, rewrites the tables
//     and records a pending move (serial, source blocks); when an allocation
//     runs short, the pending moves of that space are completed — after the
//     caller's wait callback confirms their copies finished — and their source
//     blocks reclaimed, as _reclaim_gpu/cpu_move_blocks do (:360-472).
// Asynchrony (Ray RPC, CUDA/HIP events) stays with the caller: the callback
// is where the caller waits for the copies of the moves it is asked about.
#include <algorithm>
#include <cstdint>
#include <deque>
#include <map>
#include <new>
#include <unordered_map>
#include <vector>

#include "../../include/aegkv.h"

namespace {

struct MoveEvent {
  int64_t serial;
  int32_t shape;
  int32_t src_loc, dst_loc;  // >= 0: GPU engine, AEGKV_BM_CPU: CPU pool
  std::vector<int64_t> source_blocks;
};

struct GpuSpace {
  int32_t shape = -1;
  int64_t num_max = 0;
  std::deque<int64_t> free;
  int64_t moving = 0;
  std::deque<MoveEvent> moves;  // moves whose source is this space
};

struct Table {
  int32_t location;
  int32_t shape;
  std::vector<int64_t> blocks;
};

bool is_gpu(int32_t loc) { return loc >= 0; }

}  // namespace

struct aegkv_block_manager {
  int64_t num_slabs, slab_bytes;
  std::map<int32_t, uint64_t> shape_bytes;         // shape id -> bytes per block
  std::map<int32_t, std::deque<int64_t>> cpu_free;  // shape -> free CPU blocks
  std::vector<int64_t> free_slabs;                 // stack (pop from the back)
  std::vector<int64_t> slab_usage;
  std::vector<int32_t> slab_shape;                 // -1: free slab
  std::map<int32_t, int64_t> cpu_moving;           // shape -> blocks moving out of CPU
  std::map<int32_t, std::deque<MoveEvent>> cpu_moves;  // shape -> moves from the CPU
  std::map<int32_t, GpuSpace> gpu;
  std::unordered_map<int64_t, Table> tables;
  int64_t next_serial = 0;
  aegkv_bm_wait_fn wait = nullptr;
  void* wait_ctx = nullptr;
  // last move_requests result
  std::vector<int64_t> last_src, last_dst, last_reqs;
};

namespace {

uint64_t block_bytes_of(const aegkv_block_manager* bm, int32_t shape) {
  auto it = bm->shape_bytes.find(shape);
  return it == bm->shape_bytes.end() ? 0 : it->second;
}

// Block ids wholly inside a slab (block_manager.py:242-245).
void slab_range(const aegkv_block_manager* bm, int64_t slab, uint64_t bb, int64_t* start,
                int64_t* end) {
  const unsigned __int128 lo = (unsigned __int128)slab * (uint64_t)bm->slab_bytes;
  const unsigned __int128 hi = (unsigned __int128)(slab + 1) * (uint64_t)bm->slab_bytes;
  *start = (int64_t)((lo + bb - 1) / bb);
  *end = (int64_t)(hi / bb);
}

int64_t slab_of(const aegkv_block_manager* bm, int64_t block, uint64_t bb) {
  return (int64_t)(((unsigned __int128)block * bb) / (uint64_t)bm->slab_bytes);
}

int64_t reclaim_gpu_once(GpuSpace& g, const MoveEvent& ev) {
  g.moving -= (int64_t)ev.source_blocks.size();
  g.free.insert(g.free.end(), ev.source_blocks.begin(), ev.source_blocks.end());
  return (int64_t)ev.source_blocks.size();
}

int64_t reclaim_cpu_once(aegkv_block_manager* bm, const MoveEvent& ev) {
  const uint64_t bb = block_bytes_of(bm, ev.shape);
  bm->cpu_moving[ev.shape] -= (int64_t)ev.source_blocks.size();
  auto& fl = bm->cpu_free[ev.shape];
  fl.insert(fl.end(), ev.source_blocks.begin(), ev.source_blocks.end());
  for (int64_t b : ev.source_blocks) bm->slab_usage[slab_of(bm, b, bb)] -= 1;
  return (int64_t)ev.source_blocks.size();
}

// _reclaim_cpu_slabs (block_manager.py:474-496): every slab with no used
// block returns to the free-slab stack, its blocks leave the shape's free
// deque (the remaining blocks keep their order).  One pass over each deque.
void reclaim_cpu_slabs(aegkv_block_manager* bm) {
  std::map<int32_t, std::vector<std::pair<int64_t, int64_t>>> ranges;  // shape -> [start, end)
  for (int64_t s = 0; s < bm->num_slabs; ++s) {
    const int32_t shape = bm->slab_shape[s];
    if (bm->slab_usage[s] == 0 && shape >= 0) {
      int64_t a, b;
      slab_range(bm, s, block_bytes_of(bm, shape), &a, &b);
      ranges[shape].push_back({a, b});
      bm->free_slabs.push_back(s);
      bm->slab_shape[s] = -1;
    }
  }
  for (auto& [shape, rs] : ranges) {
    auto& fl = bm->cpu_free[shape];
    std::deque<int64_t> kept;
    for (int64_t blk : fl) {
      bool inside = false;
      for (auto& r : rs)
        if (blk >= r.first && blk < r.second) { inside = true; break; }
      if (!inside) kept.push_back(blk);
    }
    fl.swap(kept);
  }
}

// Complete every pending move from GPU engine `loc` (or from the CPU pool for
// `shape`) issued up to now, once the caller confirms their copies are done.
int reclaim_moves(aegkv_block_manager* bm, int32_t loc, int32_t shape) {
  std::deque<MoveEvent>& q = is_gpu(loc) ? bm->gpu[loc].moves : bm->cpu_moves[shape];
  if (q.empty()) return AEGKV_OK;
  const int64_t target = q.back().serial;
  if (!bm->wait) return AEGKV_ERR_NO_SPACE;
  if (bm->wait(bm->wait_ctx, loc, shape, target) != 0) return AEGKV_ERR_NO_SPACE;
  while (!q.empty() && q.front().serial <= target) {
    MoveEvent ev = std::move(q.front());
    q.pop_front();
    if (is_gpu(loc)) reclaim_gpu_once(bm->gpu[loc], ev);
    else reclaim_cpu_once(bm, ev);
  }
  if (!is_gpu(loc)) reclaim_cpu_slabs(bm);
  return AEGKV_OK;
}

// _get_free_blocks (block_manager.py:498-582).
int get_free_blocks(aegkv_block_manager* bm, int64_t n, int32_t loc, int32_t shape,
                    std::vector<int64_t>* out) {
  out->clear();
  if (n <= 0) return AEGKV_OK;
  if (is_gpu(loc)) {
    auto it = bm->gpu.find(loc);
    if (it == bm->gpu.end()) return AEGKV_ERR_INVALID_ARG;
    GpuSpace& g = it->second;
    if ((int64_t)g.free.size() < n) {
      int rc = reclaim_moves(bm, loc, shape);
      if (rc && rc != AEGKV_ERR_NO_SPACE) return rc;
      if ((int64_t)g.free.size() < n) return AEGKV_ERR_NO_SPACE;
    }
    out->assign(g.free.begin(), g.free.begin() + n);
    g.free.erase(g.free.begin(), g.free.begin() + n);
    return AEGKV_OK;
  }
  const uint64_t bb = block_bytes_of(bm, shape);
  if (bb == 0) return AEGKV_ERR_INVALID_ARG;
  auto& fl = bm->cpu_free[shape];
  auto ensure = [&](int64_t needed) {
    if (needed <= 0) return true;
    for (int64_t s : bm->free_slabs) {
      int64_t a, b;
      slab_range(bm, s, bb, &a, &b);
      needed -= b - a;
      if (needed <= 0) return true;
    }
    return false;
  };
  if (!ensure(n - (int64_t)fl.size())) {
    int rc = reclaim_moves(bm, loc, shape);
    if (rc && rc != AEGKV_ERR_NO_SPACE) return rc;
    if (!ensure(n - (int64_t)fl.size())) return AEGKV_ERR_NO_SPACE;
  }
  while ((int64_t)fl.size() < n) {
    const int64_t s = bm->free_slabs.back();
    bm->free_slabs.pop_back();
    int64_t a, b;
    slab_range(bm, s, bb, &a, &b);
    bm->slab_shape[s] = shape;
    for (int64_t x = a; x < b; ++x) fl.push_back(x);
  }
  out->reserve(n);
  for (int64_t k = 0; k < n; ++k) {
    const int64_t blk = fl.front();
    fl.pop_front();
    bm->slab_usage[slab_of(bm, blk, bb)] += 1;
    out->push_back(blk);
  }
  return AEGKV_OK;
}

// Undo the table updates of a move that failed part-way: the target blocks
// return to the head of their free list in their original order (the latest
// taken first), the tables get their old blocks back.  Reclaims the failed call
// triggered stay done; slabs it opened stay with the shape (their blocks free).
void undo_moves(aegkv_block_manager* bm, int32_t target, int32_t shape, int32_t source) {
  const uint64_t bb = block_bytes_of(bm, shape);
  size_t off = bm->last_src.size();
  for (size_t k = bm->last_reqs.size(); k-- > 0;) {
    Table& tab = bm->tables[bm->last_reqs[k]];
    const size_t nb = tab.blocks.size();
    off -= nb;
    if (is_gpu(target)) {
      auto& fl = bm->gpu[target].free;
      fl.insert(fl.begin(), tab.blocks.begin(), tab.blocks.end());
    } else {
      auto& fl = bm->cpu_free[shape];
      fl.insert(fl.begin(), tab.blocks.begin(), tab.blocks.end());
      for (int64_t b : tab.blocks) bm->slab_usage[slab_of(bm, b, bb)] -= 1;
    }
    tab.blocks.assign(bm->last_src.begin() + off, bm->last_src.begin() + off + nb);
    tab.location = source;
  }
  bm->last_src.clear();
  bm->last_dst.clear();
  bm->last_reqs.clear();
}

}  // namespace

extern "C" {

int aegkv_bm_create(int64_t cpu_num_slabs, int64_t cpu_slab_bytes, aegkv_block_manager** out) {
  if (!out || cpu_num_slabs < 0 || cpu_slab_bytes <= 0) return AEGKV_ERR_INVALID_ARG;
  auto* bm = new (std::nothrow) aegkv_block_manager();
  if (!bm) return AEGKV_ERR_NO_SPACE;
  bm->num_slabs = cpu_num_slabs;
  bm->slab_bytes = cpu_slab_bytes;
  for (int64_t s = 0; s < cpu_num_slabs; ++s) bm->free_slabs.push_back(s);
  bm->slab_usage.assign(cpu_num_slabs, 0);
  bm->slab_shape.assign(cpu_num_slabs, -1);
  *out = bm;
  return AEGKV_OK;
}

void aegkv_bm_destroy(aegkv_block_manager* bm) { delete bm; }

int aegkv_bm_set_wait(aegkv_block_manager* bm, aegkv_bm_wait_fn fn, void* ctx) {
  if (!bm) return AEGKV_ERR_INVALID_ARG;
  bm->wait = fn;
  bm->wait_ctx = ctx;
  return AEGKV_OK;
}

int aegkv_bm_define_shape(aegkv_block_manager* bm, int32_t shape, uint64_t block_bytes) {
  if (!bm || shape < 0 || block_bytes == 0) return AEGKV_ERR_INVALID_ARG;
  auto it = bm->shape_bytes.find(shape);
  if (it != bm->shape_bytes.end() && it->second != block_bytes) return AEGKV_ERR_INVALID_ARG;
  bm->shape_bytes[shape] = block_bytes;
  return AEGKV_OK;
}

// register_gpu_space (block_manager.py:300-348).  Unlike the reference, which
// clears the pending moves of every engine (:321-322) and so strands their
// source blocks, only this engine's pending GPU moves are dropped.
int aegkv_bm_register_gpu_space(aegkv_block_manager* bm, int32_t engine, int64_t num_max_blocks,
                                int32_t shape) {
  if (!bm || engine < 0 || num_max_blocks < 0 || block_bytes_of(bm, shape) == 0)
    return AEGKV_ERR_INVALID_ARG;
  auto it = bm->gpu.find(engine);
  if (it != bm->gpu.end()) {
    for (auto& kv : bm->tables)
      if (kv.second.location == engine) return AEGKV_ERR_IN_USE;
    const int32_t old_shape = it->second.shape;
    // reclaim CPU blocks moving to the old space (their copies target it)
    auto& q = bm->cpu_moves[old_shape];
    // (the reference leaves slab reclaim to the next CPU reclaim)
    std::deque<MoveEvent> kept;
    for (auto& ev : q) {
      if (ev.dst_loc == engine) reclaim_cpu_once(bm, ev);
      else kept.push_back(std::move(ev));
    }
    q.swap(kept);
  }
  GpuSpace g;
  g.shape = shape;
  g.num_max = num_max_blocks;
  for (int64_t b = 0; b < num_max_blocks; ++b) g.free.push_back(b);
  bm->gpu[engine] = std::move(g);
  return AEGKV_OK;
}

// allocate_blocks_batched (block_manager.py:651-694): requests[i] needs
// num_blocks_needed[i] blocks in total; new requests get a table, known ones
// grow at the tail; one batched allocation, handed out in request order.
int aegkv_bm_allocate(aegkv_block_manager* bm, int32_t engine, const int64_t* request_ids,
                      const int64_t* num_blocks_needed, int64_t n) {
  if (!bm || n < 0 || (n > 0 && (!request_ids || !num_blocks_needed)))
    return AEGKV_ERR_INVALID_ARG;
  auto git = bm->gpu.find(engine);
  if (git == bm->gpu.end()) return AEGKV_ERR_INVALID_ARG;
  const int32_t shape = git->second.shape;
  std::vector<int64_t> counts(n);
  int64_t total = 0;
  for (int64_t i = 0; i < n; ++i) {
    auto t = bm->tables.find(request_ids[i]);
    if (t != bm->tables.end() && t->second.location != engine) return AEGKV_ERR_IN_USE;
    const int64_t have = t == bm->tables.end() ? 0 : (int64_t)t->second.blocks.size();
    counts[i] = num_blocks_needed[i] - have;
    if (counts[i] < 0) return AEGKV_ERR_INVALID_ARG;
    total += counts[i];
  }
  std::vector<int64_t> got;
  int rc = get_free_blocks(bm, total, engine, shape, &got);
  if (rc) return rc;
  int64_t cur = 0;
  for (int64_t i = 0; i < n; ++i) {
    auto t = bm->tables.find(request_ids[i]);
    if (t == bm->tables.end()) {
      Table tab{engine, shape, std::vector<int64_t>(got.begin() + cur, got.begin() + cur + counts[i])};
      bm->tables.emplace(request_ids[i], std::move(tab));
    } else {
      t->second.blocks.insert(t->second.blocks.end(), got.begin() + cur,
                              got.begin() + cur + counts[i]);
    }
    cur += counts[i];
  }
  return AEGKV_OK;
}

// free_blocks (block_manager.py:696-711).
int aegkv_bm_free(aegkv_block_manager* bm, int64_t request_id) {
  if (!bm) return AEGKV_ERR_INVALID_ARG;
  auto t = bm->tables.find(request_id);
  if (t == bm->tables.end()) return AEGKV_ERR_OUT_OF_RANGE;
  Table tab = std::move(t->second);
  bm->tables.erase(t);
  if (is_gpu(tab.location)) {
    auto& fl = bm->gpu[tab.location].free;
    fl.insert(fl.end(), tab.blocks.begin(), tab.blocks.end());
  } else {
    const uint64_t bb = block_bytes_of(bm, tab.shape);
    auto& fl = bm->cpu_free[tab.shape];
    fl.insert(fl.end(), tab.blocks.begin(), tab.blocks.end());
    for (int64_t b : tab.blocks) bm->slab_usage[slab_of(bm, b, bb)] -= 1;
  }
  return AEGKV_OK;
}

// move_requests (block_manager.py:778-874) for CPU<->GPU swaps.  Requests
// already at the target are skipped; the others must share location and
// shape.  On success *n_blocks ids are ready for aegkv_bm_move_ids, and
// *serial, *is_swap_in and *engine (the GPU side) describe the move (serial
// -1 when nothing moved).
int aegkv_bm_move(aegkv_block_manager* bm, const int64_t* request_ids, int64_t n,
                  int32_t target, int64_t* serial, int64_t* n_blocks, int32_t* is_swap_in,
                  int32_t* engine) {
  if (!bm || n < 0 || (n > 0 && !request_ids) || !serial || !n_blocks || !is_swap_in || !engine)
    return AEGKV_ERR_INVALID_ARG;
  if (!is_gpu(target) && target != AEGKV_BM_CPU) return AEGKV_ERR_INVALID_ARG;
  if (is_gpu(target) && bm->gpu.find(target) == bm->gpu.end()) return AEGKV_ERR_INVALID_ARG;
  // validate first, so that a rejected call changes nothing
  int32_t cur = 0, shape = -1;
  bool any = false;
  for (int64_t i = 0; i < n; ++i) {
    auto t = bm->tables.find(request_ids[i]);
    if (t == bm->tables.end()) return AEGKV_ERR_OUT_OF_RANGE;
    if (t->second.location == target) continue;
    if (is_gpu(t->second.location) && is_gpu(target)) return AEGKV_ERR_UNSUPPORTED;
    if (any && (t->second.location != cur || t->second.shape != shape)) return AEGKV_ERR_INVALID_ARG;
    cur = t->second.location;
    shape = t->second.shape;
    any = true;
  }
  if (any && is_gpu(target) && bm->gpu[target].shape != shape) return AEGKV_ERR_INVALID_ARG;
  bm->last_src.clear();
  bm->last_dst.clear();
  bm->last_reqs.clear();
  *serial = -1;
  *n_blocks = 0;
  *is_swap_in = is_gpu(target) ? 1 : 0;
  *engine = is_gpu(target) ? target : cur;
  if (!any) return AEGKV_OK;
  std::vector<int64_t> got;
  for (int64_t i = 0; i < n; ++i) {
    Table& tab = bm->tables[request_ids[i]];
    if (tab.location == target) continue;
    int rc = get_free_blocks(bm, (int64_t)tab.blocks.size(), target, shape, &got);
    if (rc) {
      undo_moves(bm, target, shape, cur);
      return rc;
    }
    bm->last_src.insert(bm->last_src.end(), tab.blocks.begin(), tab.blocks.end());
    bm->last_dst.insert(bm->last_dst.end(), got.begin(), got.end());
    bm->last_reqs.push_back(request_ids[i]);
    tab.blocks = got;
    tab.location = target;
  }
  MoveEvent ev{bm->next_serial++, shape, cur, target, bm->last_src};
  if (is_gpu(cur)) {
    GpuSpace& g = bm->gpu[cur];
    g.moving += (int64_t)ev.source_blocks.size();
    g.moves.push_back(std::move(ev));
  } else {
    bm->cpu_moving[shape] += (int64_t)ev.source_blocks.size();
    bm->cpu_moves[shape].push_back(std::move(ev));
  }
  *serial = bm->next_serial - 1;
  *n_blocks = (int64_t)bm->last_src.size();
  return AEGKV_OK;
}

int aegkv_bm_move_ids(const aegkv_block_manager* bm, int64_t* src_ids, int64_t* dst_ids,
                      int64_t cap, int64_t* moved_request_ids, int64_t request_cap,
                      int64_t* n_moved) {
  if (!bm || !n_moved) return AEGKV_ERR_INVALID_ARG;
  *n_moved = (int64_t)bm->last_reqs.size();
  const int64_t nb = (int64_t)bm->last_src.size();
  if (nb > 0 && (cap < nb || !src_ids || !dst_ids)) return AEGKV_ERR_INVALID_ARG;
  if (moved_request_ids && request_cap < *n_moved) return AEGKV_ERR_INVALID_ARG;
  std::copy(bm->last_src.begin(), bm->last_src.end(), src_ids);
  std::copy(bm->last_dst.begin(), bm->last_dst.end(), dst_ids);
  if (moved_request_ids) std::copy(bm->last_reqs.begin(), bm->last_reqs.end(), moved_request_ids);
  return AEGKV_OK;
}

// Reclaim the pending moves from `location` (a GPU engine, or the CPU pool of
// `shape`) whose copies the caller has seen finish: the non-waiting form of
// _reclaim_gpu/cpu_move_blocks, e.g. at a model switch.
int aegkv_bm_complete_moves(aegkv_block_manager* bm, int32_t location, int32_t shape,
                            int64_t up_to_serial) {
  if (!bm) return AEGKV_ERR_INVALID_ARG;
  if (is_gpu(location) && bm->gpu.find(location) == bm->gpu.end()) return AEGKV_ERR_INVALID_ARG;
  std::deque<MoveEvent>& q = is_gpu(location) ? bm->gpu[location].moves : bm->cpu_moves[shape];
  while (!q.empty() && q.front().serial <= up_to_serial) {
    MoveEvent ev = std::move(q.front());
    q.pop_front();
    if (is_gpu(location)) reclaim_gpu_once(bm->gpu[location], ev);
    else reclaim_cpu_once(bm, ev);
  }
  if (!is_gpu(location)) reclaim_cpu_slabs(bm);
  return AEGKV_OK;
}

int aegkv_bm_table(const aegkv_block_manager* bm, int64_t request_id, int32_t* location,
                   int32_t* shape, int64_t* n_blocks, int64_t* blocks, int64_t cap) {
  if (!bm || !location || !shape || !n_blocks) return AEGKV_ERR_INVALID_ARG;
  auto t = bm->tables.find(request_id);
  if (t == bm->tables.end()) return AEGKV_ERR_OUT_OF_RANGE;
  *location = t->second.location;
  *shape = t->second.shape;
  *n_blocks = (int64_t)t->second.blocks.size();
  if (blocks) {
    if (cap < *n_blocks) return AEGKV_ERR_INVALID_ARG;
    std::copy(t->second.blocks.begin(), t->second.blocks.end(), blocks);
  }
  return AEGKV_OK;
}

// The block tables of `request_ids`, flattened: table i is
// ids[offsets[i] .. offsets[i+1]) (the layout aegkv_prepare_inputs takes).
int aegkv_bm_flat_tables(const aegkv_block_manager* bm, const int64_t* request_ids, int64_t n,
                         int64_t* offsets, int32_t* ids, int64_t cap) {
  if (!bm || n < 0 || !offsets || (n > 0 && !request_ids)) return AEGKV_ERR_INVALID_ARG;
  offsets[0] = 0;
  for (int64_t i = 0; i < n; ++i) {
    auto t = bm->tables.find(request_ids[i]);
    if (t == bm->tables.end()) return AEGKV_ERR_OUT_OF_RANGE;
    offsets[i + 1] = offsets[i] + (int64_t)t->second.blocks.size();
  }
  if (!ids) return AEGKV_OK;
  if (cap < offsets[n]) return AEGKV_ERR_INVALID_ARG;
  for (int64_t i = 0; i < n; ++i) {
    const auto& b = bm->tables.find(request_ids[i])->second.blocks;
    for (size_t k = 0; k < b.size(); ++k) {
      if (b[k] > INT32_MAX) return AEGKV_ERR_UNSUPPORTED;
      ids[offsets[i] + (int64_t)k] = (int32_t)b[k];
    }
  }
  return AEGKV_OK;
}

// Counters for logging and tests (block_manager.py:730-768): free and moving
// blocks of a GPU engine, or of a CPU shape (with the blocks its slabs hold).
int aegkv_bm_stats(const aegkv_block_manager* bm, int32_t location, int32_t shape,
                   int64_t* n_free, int64_t* n_moving, int64_t* n_slabs, int64_t* n_used) {
  if (!bm || !n_free || !n_moving || !n_slabs || !n_used) return AEGKV_ERR_INVALID_ARG;
  if (is_gpu(location)) {
    auto it = bm->gpu.find(location);
    if (it == bm->gpu.end()) return AEGKV_ERR_INVALID_ARG;
    *n_free = (int64_t)it->second.free.size();
    *n_moving = it->second.moving;
    *n_slabs = 0;
    *n_used = 0;
    return AEGKV_OK;
  }
  auto f = bm->cpu_free.find(shape);
  *n_free = f == bm->cpu_free.end() ? 0 : (int64_t)f->second.size();
  auto m = bm->cpu_moving.find(shape);
  *n_moving = m == bm->cpu_moving.end() ? 0 : m->second;
  *n_slabs = 0;
  *n_used = 0;
  for (int64_t s = 0; s < bm->num_slabs; ++s)
    if (bm->slab_shape[s] == shape) {
      ++*n_slabs;
      *n_used += bm->slab_usage[s];
    }
  return AEGKV_OK;
}

// The free list of a GPU engine or CPU shape, in order (for tests).
int aegkv_bm_free_list(const aegkv_block_manager* bm, int32_t location, int32_t shape,
                       int64_t* out, int64_t cap, int64_t* n) {
  if (!bm || !n) return AEGKV_ERR_INVALID_ARG;
  const std::deque<int64_t>* fl = nullptr;
  if (is_gpu(location)) {
    auto it = bm->gpu.find(location);
    if (it == bm->gpu.end()) return AEGKV_ERR_INVALID_ARG;
    fl = &it->second.free;
  } else {
    auto it = bm->cpu_free.find(shape);
    static const std::deque<int64_t> empty;
    fl = it == bm->cpu_free.end() ? &empty : &it->second;
  }
  *n = (int64_t)fl->size();
  if (out) {
    if (cap < *n) return AEGKV_ERR_INVALID_ARG;
    std::copy(fl->begin(), fl->end(), out);
  }
  return AEGKV_OK;
}

}  // extern "C"
