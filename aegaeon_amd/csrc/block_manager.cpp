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
// Asynchrony (Ray RPC, CUDA/HIP events) stays with the caller.  Where the
// reference awaits the pending moves of a space before reclaiming their
// source blocks (_get_free_blocks -> _reclaim_*_move_blocks, :498-582,
// :410-472), a call here suspends instead: it keeps what it has done so far
// (the requests a move has already assigned keep their new tables, as in the
// reference), returns AEGKV_RECLAIM_PENDING and names the space and the last
// pending serial; the caller awaits those moves, reclaims them
// (aegkv_bm_complete_move / aegkv_bm_reclaim_slabs) and resumes the call, which
// continues at the allocation that ran short.  Between suspension and resume
// other calls may run, as other coroutines do in the reference's event loop.
// A caller that can block may instead install a wait callback, called at the
// same point; the library then reclaims and continues in the same call.
#include <algorithm>
#include <cstdint>
#include <deque>
#include <map>
#include <new>
#include <unordered_map>
#include <unordered_set>
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

// A suspended allocate_blocks_batched or move_requests.
struct PendingOp {
  bool is_move = false;
  int32_t loc = 0, shape = -1;  // the space whose pending moves it waits for
  int64_t serial = -1;          // ... up to this serial
  // allocate: blocks per request, taken in one batch after the reclaim
  int32_t engine = 0;
  std::vector<int64_t> ids, counts;  // the call's requests (both kinds)
  int64_t total = 0;
  std::vector<char> had;  // the request had a table when the call began
  // move: the call's requests, where it stopped, and what it has moved
  int32_t target = 0, source = 0;
  size_t next = 0;
  std::vector<int64_t> src, dst, moved, sizes;
  int32_t mshape = -1;    // the blocks' shape
  bool reclaimed = false; // resumed: the next allocation does not suspend again
};

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
  // suspended calls, and the requests their moves hold
  std::map<int64_t, PendingOp> ops;
  int64_t next_op = 1, last_op = 0;
  std::unordered_set<int64_t> busy;
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

std::deque<MoveEvent>& move_queue(aegkv_block_manager* bm, int32_t loc, int32_t shape) {
  return is_gpu(loc) ? bm->gpu[loc].moves : bm->cpu_moves[shape];
}

// Where an allocation stopped: the space that ran short and its last pending
// move's serial.
struct Shortage {
  int32_t loc = 0, shape = -1;
  int64_t serial = -1;
};

// A space ran short.  With nothing pending there is nothing to reclaim (the
// caller's re-check fails).  With a wait callback, every pending move issued
// up to now is completed once the callback confirms its copy finished, as
// _reclaim_gpu/cpu_move_blocks do (block_manager.py:410-472).  Without one,
// a call that may suspend reports the shortage; a resumed call (whose caller
// has reclaimed already) does not suspend for the same allocation again, as
// the reference reclaims once per _get_free_blocks (:510-519,547-560).
int on_short(aegkv_block_manager* bm, int32_t loc, int32_t shape, bool may_suspend,
             Shortage* sh) {
  std::deque<MoveEvent>& q = move_queue(bm, loc, shape);
  if (q.empty()) return AEGKV_OK;
  const int64_t target = q.back().serial;
  if (bm->wait) {
    if (bm->wait(bm->wait_ctx, loc, shape, target) != 0) return AEGKV_OK;
    while (!q.empty() && q.front().serial <= target) {
      MoveEvent ev = std::move(q.front());
      q.pop_front();
      if (is_gpu(loc)) reclaim_gpu_once(bm->gpu[loc], ev);
      else reclaim_cpu_once(bm, ev);
    }
    if (!is_gpu(loc)) reclaim_cpu_slabs(bm);
    return AEGKV_OK;
  }
  if (!may_suspend) return AEGKV_OK;
  sh->loc = loc;
  sh->shape = shape;
  sh->serial = target;
  return AEGKV_RECLAIM_PENDING;
}

// _get_free_blocks (block_manager.py:498-582).  On a shortage: on_short, then
// one re-check (AEGKV_ERR_NO_SPACE, the reference's ResourceWarning).
// AEGKV_RECLAIM_PENDING takes nothing.
int get_free_blocks(aegkv_block_manager* bm, int64_t n, int32_t loc, int32_t shape,
                    std::vector<int64_t>* out, bool may_suspend, Shortage* sh) {
  out->clear();
  if (n <= 0) return AEGKV_OK;
  if (is_gpu(loc)) {
    auto it = bm->gpu.find(loc);
    if (it == bm->gpu.end()) return AEGKV_ERR_INVALID_ARG;
    GpuSpace& g = it->second;
    if ((int64_t)g.free.size() < n) {
      const int rc = on_short(bm, loc, shape, may_suspend, sh);
      if (rc) return rc;
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
    const int rc = on_short(bm, loc, shape, may_suspend, sh);
    if (rc) return rc;
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

// Blocks go back to a space: at the head of its free list in their order
// (undoing an allocation) or at the tail (a free).
void give_back(aegkv_block_manager* bm, int32_t loc, int32_t shape, const int64_t* b, size_t n,
               bool at_head) {
  if (n == 0) return;
  if (is_gpu(loc)) {
    auto& fl = bm->gpu[loc].free;
    fl.insert(at_head ? fl.begin() : fl.end(), b, b + n);
    return;
  }
  const uint64_t bb = block_bytes_of(bm, shape);
  auto& fl = bm->cpu_free[shape];
  fl.insert(at_head ? fl.begin() : fl.end(), b, b + n);
  for (size_t k = 0; k < n; ++k) bm->slab_usage[slab_of(bm, b[k], bb)] -= 1;
}

void set_busy(aegkv_block_manager* bm, const PendingOp& op, bool on) {
  for (int64_t id : op.ids) {
    if (on) bm->busy.insert(id);
    else bm->busy.erase(id);
  }
}

// A request a suspended move had already assigned was freed meanwhile: the
// free returned its target blocks, so its pair leaves the move and its source
// blocks are freed at the source (nothing was copied yet).
void drop_freed(aegkv_block_manager* bm, PendingOp& op) {
  std::vector<int64_t> src, dst, moved, sizes;
  size_t off = 0;
  for (size_t k = 0; k < op.moved.size(); ++k) {
    const size_t nb = (size_t)op.sizes[k];
    if (bm->tables.count(op.moved[k])) {
      src.insert(src.end(), op.src.begin() + off, op.src.begin() + off + nb);
      dst.insert(dst.end(), op.dst.begin() + off, op.dst.begin() + off + nb);
      moved.push_back(op.moved[k]);
      sizes.push_back((int64_t)nb);
    } else {
      give_back(bm, op.source, op.mshape, op.src.data() + off, nb, false);
    }
    off += nb;
  }
  op.src.swap(src);
  op.dst.swap(dst);
  op.moved.swap(moved);
  op.sizes.swap(sizes);
}

// Undo a move that failed or was cancelled: the target blocks return to the
// head of their free list in their original order (the latest taken first),
// the tables get their old blocks back.  Reclaims the call triggered stay done;
// slabs it opened stay with the shape (their blocks free).
void rollback_move(aegkv_block_manager* bm, PendingOp& op) {
  drop_freed(bm, op);
  size_t off = op.src.size();
  for (size_t k = op.moved.size(); k-- > 0;) {
    const size_t nb = (size_t)op.sizes[k];
    off -= nb;
    Table& tab = bm->tables[op.moved[k]];
    give_back(bm, op.target, op.mshape, tab.blocks.data(), tab.blocks.size(), true);
    tab.blocks.assign(op.src.begin() + off, op.src.begin() + off + nb);
    tab.location = op.source;
  }
  op.src.clear();
  op.dst.clear();
  op.moved.clear();
  op.sizes.clear();
}

// The loop of move_requests (block_manager.py:797-832) from request op.next:
// each request not yet at the target gets target blocks and its table moves.
int run_move(aegkv_block_manager* bm, PendingOp& op) {
  std::vector<int64_t> got;
  for (; op.next < op.ids.size(); ++op.next) {
    auto t = bm->tables.find(op.ids[op.next]);
    if (t == bm->tables.end()) continue;  // freed while the call was suspended
    Table& tab = t->second;
    if (tab.location == op.target) continue;
    if (tab.location != op.source || tab.shape != op.mshape) return AEGKV_ERR_IN_USE;
    Shortage sh;
    const int rc = get_free_blocks(bm, (int64_t)tab.blocks.size(), op.target, op.mshape, &got,
                                   !op.reclaimed, &sh);
    if (rc == AEGKV_RECLAIM_PENDING) {
      op.loc = sh.loc;
      op.shape = sh.shape;
      op.serial = sh.serial;
      return rc;
    }
    op.reclaimed = false;
    if (rc) return rc;
    op.src.insert(op.src.end(), tab.blocks.begin(), tab.blocks.end());
    op.dst.insert(op.dst.end(), got.begin(), got.end());
    op.moved.push_back(op.ids[op.next]);
    op.sizes.push_back((int64_t)got.size());
    tab.blocks = got;
    tab.location = op.target;
  }
  return AEGKV_OK;
}

// The end of move_requests (:834-872): the lists for the swap call, and the
// pending move whose source blocks are reclaimed once its copy is done.
void finish_move(aegkv_block_manager* bm, PendingOp& op, int64_t* serial, int64_t* n_blocks,
                 int32_t* is_swap_in, int32_t* engine) {
  bm->last_src = op.src;
  bm->last_dst = op.dst;
  bm->last_reqs = op.moved;
  *is_swap_in = is_gpu(op.target) ? 1 : 0;
  *engine = is_gpu(op.target) ? op.target : op.source;
  *serial = -1;
  *n_blocks = (int64_t)op.src.size();
  if (op.moved.empty()) return;
  MoveEvent ev{bm->next_serial++, op.mshape, op.source, op.target, op.src};
  if (is_gpu(op.source)) {
    GpuSpace& g = bm->gpu[op.source];
    g.moving += (int64_t)ev.source_blocks.size();
    g.moves.push_back(std::move(ev));
  } else {
    bm->cpu_moving[op.mshape] += (int64_t)ev.source_blocks.size();
    bm->cpu_moves[op.mshape].push_back(std::move(ev));
  }
  *serial = bm->next_serial - 1;
}

// Hand out an allocation (:680-694): new requests get a table, known ones
// grow at the tail.
void assign_allocation(aegkv_block_manager* bm, const PendingOp& op,
                       const std::vector<int64_t>& got) {
  int64_t cur = 0;
  for (size_t i = 0; i < op.ids.size(); ++i) {
    const int64_t c = op.counts[i];
    auto t = bm->tables.find(op.ids[i]);
    if (t == bm->tables.end()) {
      if (op.had[i]) continue;  // freed while the call was suspended: nothing for it
      Table tab{op.engine, op.mshape,
                std::vector<int64_t>(got.begin() + cur, got.begin() + cur + c)};
      bm->tables.emplace(op.ids[i], std::move(tab));
    } else {
      t->second.blocks.insert(t->second.blocks.end(), got.begin() + cur, got.begin() + cur + c);
    }
    cur += c;
  }
}

// The batched allocation of a (new or resumed) allocate call.
int run_allocate(aegkv_block_manager* bm, PendingOp& op) {
  op.total = 0;
  for (size_t i = 0; i < op.ids.size(); ++i) {
    auto t = bm->tables.find(op.ids[i]);
    if (t == bm->tables.end() && op.had[i]) op.counts[i] = 0;
    if (t != bm->tables.end() && t->second.location != op.engine) return AEGKV_ERR_IN_USE;
    op.total += op.counts[i];
  }
  std::vector<int64_t> got;
  Shortage sh;
  const int rc = get_free_blocks(bm, op.total, op.engine, op.mshape, &got, !op.reclaimed, &sh);
  if (rc == AEGKV_RECLAIM_PENDING) {
    op.loc = sh.loc;
    op.shape = sh.shape;
    op.serial = sh.serial;
    return rc;
  }
  if (rc) return rc;
  assign_allocation(bm, op, got);
  return AEGKV_OK;
}

int64_t suspend(aegkv_block_manager* bm, PendingOp&& op) {
  const int64_t id = bm->next_op++;
  set_busy(bm, op, true);
  bm->ops.emplace(id, std::move(op));
  bm->last_op = id;
  return id;
}

bool any_busy(const aegkv_block_manager* bm, const int64_t* ids, int64_t n) {
  if (bm->busy.empty()) return false;
  for (int64_t i = 0; i < n; ++i)
    if (bm->busy.count(ids[i])) return true;
  return false;
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
// source blocks, only this engine's pending GPU moves are dropped.  A space
// that a suspended call allocates in or moves from/to is in use.
int aegkv_bm_register_gpu_space(aegkv_block_manager* bm, int32_t engine, int64_t num_max_blocks,
                                int32_t shape) {
  if (!bm || engine < 0 || num_max_blocks < 0 || block_bytes_of(bm, shape) == 0)
    return AEGKV_ERR_INVALID_ARG;
  for (auto& kv : bm->ops) {
    const PendingOp& op = kv.second;
    if (op.is_move ? (op.target == engine || op.source == engine) : op.engine == engine)
      return AEGKV_ERR_IN_USE;
  }
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
  if (any_busy(bm, request_ids, n)) return AEGKV_ERR_IN_USE;
  PendingOp op;
  op.engine = engine;
  op.mshape = git->second.shape;
  op.ids.assign(request_ids, request_ids + n);
  op.counts.resize(n);
  op.had.resize(n);
  for (int64_t i = 0; i < n; ++i) {
    auto t = bm->tables.find(request_ids[i]);
    if (t != bm->tables.end() && t->second.location != engine) return AEGKV_ERR_IN_USE;
    const int64_t have = t == bm->tables.end() ? 0 : (int64_t)t->second.blocks.size();
    op.had[i] = t != bm->tables.end();
    op.counts[i] = num_blocks_needed[i] - have;
    if (op.counts[i] < 0) return AEGKV_ERR_INVALID_ARG;
  }
  const int rc = run_allocate(bm, op);
  if (rc == AEGKV_RECLAIM_PENDING) suspend(bm, std::move(op));
  return rc;
}

// free_blocks (block_manager.py:696-711).
int aegkv_bm_free(aegkv_block_manager* bm, int64_t request_id) {
  if (!bm) return AEGKV_ERR_INVALID_ARG;
  auto t = bm->tables.find(request_id);
  if (t == bm->tables.end()) return AEGKV_ERR_OUT_OF_RANGE;
  Table tab = std::move(t->second);
  bm->tables.erase(t);
  give_back(bm, tab.location, tab.shape, tab.blocks.data(), tab.blocks.size(), false);
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
  if (any_busy(bm, request_ids, n)) return AEGKV_ERR_IN_USE;
  bm->last_src.clear();
  bm->last_dst.clear();
  bm->last_reqs.clear();
  PendingOp op;
  op.is_move = true;
  op.target = target;
  op.source = any ? cur : target;
  op.mshape = shape;
  if (any) op.ids.assign(request_ids, request_ids + n);
  const int rc = run_move(bm, op);
  if (rc == AEGKV_RECLAIM_PENDING) {
    suspend(bm, std::move(op));
    return rc;
  }
  if (rc) {
    rollback_move(bm, op);
    return rc;
  }
  finish_move(bm, op, serial, n_blocks, is_swap_in, engine);
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

// The call suspended last: its handle, and the space and serial up to which
// its caller awaits and reclaims the pending moves before resuming it.
int aegkv_bm_pending(const aegkv_block_manager* bm, int64_t* op, int32_t* location,
                     int32_t* shape, int64_t* serial) {
  if (!bm || !op || !location || !shape || !serial) return AEGKV_ERR_INVALID_ARG;
  auto it = bm->ops.find(bm->last_op);
  if (it == bm->ops.end()) return AEGKV_ERR_OUT_OF_RANGE;
  *op = it->first;
  *location = it->second.loc;
  *shape = it->second.shape;
  *serial = it->second.serial;
  return AEGKV_OK;
}

// Continue a suspended call at the allocation that ran short (once more, with
// no second suspension for it).  Outputs as aegkv_bm_move (an allocation sets
// *serial -1 and *engine to its engine).  AEGKV_RECLAIM_PENDING again when a
// later request of a move runs short; any other failure undoes the call.
int aegkv_bm_resume(aegkv_block_manager* bm, int64_t op_id, int64_t* serial, int64_t* n_blocks,
                    int32_t* is_swap_in, int32_t* engine) {
  if (!bm || !serial || !n_blocks || !is_swap_in || !engine) return AEGKV_ERR_INVALID_ARG;
  auto it = bm->ops.find(op_id);
  if (it == bm->ops.end()) return AEGKV_ERR_OUT_OF_RANGE;
  PendingOp& op = it->second;
  op.reclaimed = true;
  int rc;
  if (op.is_move) {
    drop_freed(bm, op);
    rc = run_move(bm, op);
    if (rc == AEGKV_RECLAIM_PENDING) {
      bm->last_op = op_id;
      return rc;
    }
    if (rc) rollback_move(bm, op);
    else finish_move(bm, op, serial, n_blocks, is_swap_in, engine);
  } else {
    rc = bm->gpu.count(op.engine) && bm->gpu[op.engine].shape == op.mshape
             ? run_allocate(bm, op) : AEGKV_ERR_IN_USE;
    *serial = -1;
    *n_blocks = 0;
    *is_swap_in = 0;
    *engine = op.engine;
  }
  set_busy(bm, op, false);
  bm->ops.erase(it);
  return rc;
}

// Abandon a suspended call (its caller's wait failed): a move is undone; an
// allocation has taken nothing.
int aegkv_bm_cancel(aegkv_block_manager* bm, int64_t op_id) {
  if (!bm) return AEGKV_ERR_INVALID_ARG;
  auto it = bm->ops.find(op_id);
  if (it == bm->ops.end()) return AEGKV_ERR_OUT_OF_RANGE;
  if (it->second.is_move) rollback_move(bm, it->second);
  set_busy(bm, it->second, false);
  bm->ops.erase(it);
  return AEGKV_OK;
}

// Reclaim the pending moves from `location` (a GPU engine, or the CPU pool of
// `shape`) whose copies the caller has seen finish: the non-waiting form of
// _reclaim_gpu/cpu_move_blocks, e.g. at a model switch.
int aegkv_bm_complete_moves(aegkv_block_manager* bm, int32_t location, int32_t shape,
                            int64_t up_to_serial) {
  if (!bm) return AEGKV_ERR_INVALID_ARG;
  if (is_gpu(location) && bm->gpu.find(location) == bm->gpu.end()) return AEGKV_ERR_INVALID_ARG;
  std::deque<MoveEvent>& q = move_queue(bm, location, shape);
  while (!q.empty() && q.front().serial <= up_to_serial) {
    MoveEvent ev = std::move(q.front());
    q.pop_front();
    if (is_gpu(location)) reclaim_gpu_once(bm->gpu[location], ev);
    else reclaim_cpu_once(bm, ev);
  }
  if (!is_gpu(location)) reclaim_cpu_slabs(bm);
  return AEGKV_OK;
}

// One pending move whose copy has finished, wherever it sits in its queue
// (_reclaim_blocks' per-event callback, :384-406); no slab pass.  A move that
// is no longer pending is not an error.
int aegkv_bm_complete_move(aegkv_block_manager* bm, int32_t location, int32_t shape,
                           int64_t serial) {
  if (!bm) return AEGKV_ERR_INVALID_ARG;
  if (is_gpu(location) && bm->gpu.find(location) == bm->gpu.end()) return AEGKV_ERR_INVALID_ARG;
  std::deque<MoveEvent>& q = move_queue(bm, location, shape);
  for (auto it = q.begin(); it != q.end(); ++it) {
    if (it->serial != serial) continue;
    MoveEvent ev = std::move(*it);
    q.erase(it);
    if (is_gpu(location)) reclaim_gpu_once(bm->gpu[location], ev);
    else reclaim_cpu_once(bm, ev);
    break;
  }
  return AEGKV_OK;
}

// _reclaim_cpu_slabs (:474-496), run once after a CPU reclaim.
int aegkv_bm_reclaim_slabs(aegkv_block_manager* bm) {
  if (!bm) return AEGKV_ERR_INVALID_ARG;
  reclaim_cpu_slabs(bm);
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
