// Block-granular KV movement on gfx950: gather (pack), scatter, pool-to-pool
// copy, defrag and the CPU<->GPU swap that replaces aegaeon.ops.swap
// (aegaeon/ops/swap.cu:25-59).
//
// One kernel serves every device-side move.  A block of block_bytes is cut into
// 1 KiB tiles; one short-lived workgroup of a single wave copies one tile, on
// a two-dimensional grid (y: the block, x: its tile; a block of more tiles
// than one grid row holds loops its row, more blocks than one launch holds
// take several launches), so no workgroup divides to find its block.  The
// wave reads its block's source and destination ids with scalar loads (the
// same ids for every tile of a block, so they hit the scalar cache), then
// each lane issues one non-temporal dwordx4 load and one store: the tile is
// one fully coalesced 1 KiB wave row each way.  Loads and stores are raw
// buffer instructions bounded to the tile's valid bytes (no exec branches
// around memory), which keeps the compiler's wait counts exact.
//
// Measured on MI355X (bench sections, two rounds each, TB/s for the
// Llama-2-13B pack / scatter of 4096 x 12.5 MiB blocks, the unified-pool
// defrag, and a contiguous copy of the pack's 107 GB): one wave per 1 KiB
// tile 6.39-6.44 / 6.81 / 6.64 / 6.50-6.61; 64 lanes x 2 KiB 5.85-5.90 /
// 6.44-6.47 / 5.99-6.01; 64 x 4 KiB 5.99-6.04 / 6.51-6.57 / 5.70-5.83;
// 256 lanes x 4 KiB 6.25-6.31 / 6.52-6.56 / 6.13-6.16; 256 x 8 KiB (the
// earlier tile, with a 64-bit division per workgroup) 5.97-6.05 /
// 6.58-6.63 / 5.75-5.89 / 5.80-6.02 (16 KiB contiguous tiles); 512 x 8 KiB
// 6.14-6.25 / 6.63-6.72 / 6.20-6.26 / 6.10-6.59.  Many one-wave workgroups
// with one load and one store per lane keep the most bytes in flight; the
// earlier persistent grid (32 workgroups per CU walking 16 KiB tiles) ran at
// 5.33 TB/s, hipMemcpyAsync of a contiguous 1 GiB at 5.13.
#include <algorithm>
#include <cstring>
#include <map>
#include <mutex>
#include <numeric>
#include <thread>

#include "aegkv_internal.h"

namespace aegkv {
namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int kCopyThreads = 64;  // one wave per workgroup
constexpr int kTileUnroll = 1;    // dwordx4 per lane per tile: 1 KiB tiles
// Stores: non-temporal with device scope (nt sc1).  Bench sections, same call,
// two rounds, TB/s against nt alone: pack 6.51-6.52 / 6.38-6.48, scatter
// 6.83-6.85 / 6.78-6.79, defrag 6.71-6.72 / 6.60, copy calibration 6.11 /
// 5.88-5.94; stores with no policy bits were slower (pack 6.22), and loads
// with sc0 changed nothing.  A tile of a block of whole 1 KiB tiles is eight
// whole 128-byte lines, so these stores write lines, not pieces of them.
constexpr int kStorePolicy = kNt | 16;
// Identity copies (no id list on either side) move one contiguous range:
// 1 KiB tiles measured best there too (107 GB: 6.50-6.61 TB/s against
// 6.07-6.32 for 4 KiB and 5.70-5.73 for 8 KiB; the 29.4 MB copy floor the
// same within 0.1 us).
constexpr int kLinearUnroll = 1;
// Largest grid of one launch: HIP bounds a launch to 2^32 - 1 work-items per
// dimension; a block of more tiles loops its grid row over the rest, and more
// than kMaxCopyGridY blocks take several launches.
constexpr uint64_t kMaxCopyGrid = (1ull << 31) / kCopyThreads;
constexpr int64_t kMaxCopyGridY = 65535;
static_assert(kMaxCopyGrid * kCopyThreads <= 0xFFFFFFFFull,
              "the copy grid must fit one launch dimension");

// SRC_IDS / DST_IDS: whether the side is addressed through an id list (else
// block i of the side is slot i).  UNROLL dwordx4 per lane: a tile is
// kCopyThreads * 16 * UNROLL bytes.  Every value but the lane offsets is
// uniform over the workgroup (scalar registers).
template <bool SRC_IDS, bool DST_IDS, int UNROLL>
__global__ __launch_bounds__(kCopyThreads) void copy_blocks_kernel(
    const uint8_t* __restrict__ src, uint8_t* __restrict__ dst,
    const int64_t* __restrict__ src_ids, const int64_t* __restrict__ dst_ids,
    uint64_t block_bytes, uint32_t tiles_per_block) {
  constexpr uint32_t TILE = (uint32_t)kCopyThreads * 16 * UNROLL;
  // grid y: the block (of this launch's chunk), grid x: its tile; no division
  const int64_t i = blockIdx.y;
  const int64_t s = SRC_IDS ? src_ids[i] : i;
  const int64_t d = DST_IDS ? dst_ids[i] : i;
  const uint8_t* sb = src + (uint64_t)s * block_bytes;
  uint8_t* db = dst + (uint64_t)d * block_bytes;
  for (uint32_t t = blockIdx.x; t < tiles_per_block; t += gridDim.x) {
    const uint64_t base = (uint64_t)t * TILE;
    const uint32_t bytes = (uint32_t)min(block_bytes - base, (uint64_t)TILE);
    const auto sr = byte_range(sb + base, bytes);
    const auto dr = byte_range(db + base, bytes);
    u32x4 r[UNROLL];
#pragma unroll
    for (int k = 0; k < UNROLL; ++k)
      r[k] = __builtin_amdgcn_raw_buffer_load_b128(sr, (k * kCopyThreads + threadIdx.x) * 16, 0,
                                                   kNt);
#pragma unroll
    for (int k = 0; k < UNROLL; ++k)
      __builtin_amdgcn_raw_buffer_store_b128(r[k], dr, (k * kCopyThreads + threadIdx.x) * 16, 0,
                                             kStorePolicy);
  }
}

// Blocks [0, n) in launches of at most kMaxCopyGridY blocks (grid y), each
// block's tiles along grid x (at most kMaxCopyGrid; a longer block loops).
template <bool SRC_IDS, bool DST_IDS, int UNROLL>
int launch_tiles(const void* src, void* dst, const int64_t* src_ids, const int64_t* dst_ids,
                 int64_t n, uint64_t block_bytes, hipStream_t stream) {
  constexpr uint64_t TILE = (uint64_t)kCopyThreads * 16 * UNROLL;
  const uint64_t tiles_per_block = (block_bytes + TILE - 1) / TILE;
  if (tiles_per_block > 0xFFFFFFFFull) return AEGKV_ERR_UNSUPPORTED;
  const uint32_t gx = (uint32_t)std::min<uint64_t>(tiles_per_block, kMaxCopyGrid);
  for (int64_t c0 = 0; c0 < n; c0 += kMaxCopyGridY) {
    const uint32_t gy = (uint32_t)std::min<int64_t>(n - c0, kMaxCopyGridY);
    const uint8_t* s = static_cast<const uint8_t*>(src) + (SRC_IDS ? 0 : c0 * block_bytes);
    uint8_t* d = static_cast<uint8_t*>(dst) + (DST_IDS ? 0 : c0 * block_bytes);
    hipLaunchKernelGGL((copy_blocks_kernel<SRC_IDS, DST_IDS, UNROLL>), dim3(gx, gy),
                       dim3(kCopyThreads), 0, stream, s, d, SRC_IDS ? src_ids + c0 : nullptr,
                       DST_IDS ? dst_ids + c0 : nullptr, block_bytes, (uint32_t)tiles_per_block);
    AEGKV_HIP_TRY(hipGetLastError());
  }
  return AEGKV_OK;
}

}  // namespace

int launch_copy_blocks(const DeviceState* ds, const void* src, void* dst,
                       const int64_t* src_ids_dev, const int64_t* dst_ids_dev,
                       int64_t n, uint64_t block_bytes, hipStream_t stream) {
  (void)ds;
  if (n <= 0) return AEGKV_OK;
  if (src_ids_dev)
    return dst_ids_dev
               ? launch_tiles<true, true, kTileUnroll>(src, dst, src_ids_dev, dst_ids_dev, n,
                                                        block_bytes, stream)
               : launch_tiles<true, false, kTileUnroll>(src, dst, src_ids_dev, nullptr, n,
                                                         block_bytes, stream);
  if (dst_ids_dev)
    return launch_tiles<false, true, kTileUnroll>(src, dst, nullptr, dst_ids_dev, n,
                                                   block_bytes, stream);
  // identity: one contiguous range of n * block_bytes bytes, copied as a
  // single block
  return launch_tiles<false, false, kLinearUnroll>(src, dst, nullptr, nullptr, 1,
                                                   (uint64_t)n * block_bytes, stream);
}

namespace {

bool ranges_overlap(const void* a, uint64_t na, const void* b, uint64_t nb) {
  auto x = reinterpret_cast<uintptr_t>(a), y = reinterpret_cast<uintptr_t>(b);
  return x < y + nb && y < x + na;
}

// Shared body of copy/pack/scatter/defrag: validate on the host, upload the id
// lists, launch one copy kernel.
int copy_blocks_checked_body(const void* src_pool, uint64_t n_src_blocks, void* dst_pool,
                        uint64_t n_dst_blocks, const int64_t* src_ids,
                        const int64_t* dst_ids, int64_t n, uint64_t block_bytes,
                        bool require_same_pool, hipStream_t stream) {
  if (n < 0 || !src_pool || !dst_pool || block_bytes == 0) return AEGKV_ERR_INVALID_ARG;
  if (n == 0) return AEGKV_OK;
  if ((block_bytes & 15) || !aligned16(src_pool) || !aligned16(dst_pool))
    return AEGKV_ERR_MISALIGNED;
  // pool byte sizes must be representable (they bound the overlap test)
  if (n_src_blocks > UINT64_MAX / block_bytes || n_dst_blocks > UINT64_MAX / block_bytes)
    return AEGKV_ERR_INVALID_ARG;
  int rc;
  if (src_ids) {
    if ((rc = check_ids_in_range(src_ids, n, n_src_blocks))) return rc;
  } else if ((uint64_t)n > n_src_blocks) {
    return AEGKV_ERR_OUT_OF_RANGE;
  }
  if (dst_ids) {
    if ((rc = check_ids_in_range(dst_ids, n, n_dst_blocks))) return rc;
    if ((rc = check_unique(dst_ids, n, n_dst_blocks))) return rc;
  } else if ((uint64_t)n > n_dst_blocks) {
    return AEGKV_ERR_OUT_OF_RANGE;
  }
  const bool same = src_pool == dst_pool;
  if (require_same_pool && !same) return AEGKV_ERR_INVALID_ARG;
  if (same) {
    // In-place moves must not read a block another lane writes.
    std::vector<int64_t> s, d;
    if (!src_ids) { s.resize(n); std::iota(s.begin(), s.end(), 0); }
    if (!dst_ids) { d.resize(n); std::iota(d.begin(), d.end(), 0); }
    if ((rc = check_disjoint(src_ids ? src_ids : s.data(), n, dst_ids ? dst_ids : d.data(), n,
                             std::max(n_src_blocks, n_dst_blocks))))
      return rc;
  } else if (ranges_overlap(src_pool, n_src_blocks * block_bytes, dst_pool,
                            n_dst_blocks * block_bytes)) {
    return AEGKV_ERR_OVERLAP;  // partially aliased pools: order would matter
  }
  DeviceState* ds = nullptr;
  if ((rc = current_device_state(&ds))) return rc;
  IdPart parts[2] = {{src_ids, src_ids ? n : 0}, {dst_ids, dst_ids ? n : 0}};
  return with_uploaded_ids(ds, stream, parts, 2, [&](int64_t* dev) {
    const int64_t* s = src_ids ? dev : nullptr;
    const int64_t* d = dst_ids ? dev + (src_ids ? n : 0) : nullptr;
    return launch_copy_blocks(ds, src_pool, dst_pool, s, d, n, block_bytes, stream);
  });
}

int copy_blocks_checked(const void* src_pool, uint64_t n_src_blocks, void* dst_pool,
                        uint64_t n_dst_blocks, const int64_t* src_ids,
                        const int64_t* dst_ids, int64_t n, uint64_t block_bytes,
                        bool require_same_pool, hipStream_t stream) {
  return guarded([&] {
    return copy_blocks_checked_body(src_pool, n_src_blocks, dst_pool, n_dst_blocks, src_ids,
                                    dst_ids, n, block_bytes, require_same_pool, stream);
  });
}

// Maximal runs [i, j) of `order` over which key[order[k]] increases by one.
template <typename F>
void for_each_run(const std::vector<int64_t>& order, const int64_t* key, int64_t begin,
                  int64_t end, F&& f) {
  int64_t i = begin;
  while (i < end) {
    int64_t j = i + 1;
    while (j < end && key[order[j]] == key[order[j - 1]] + 1) ++j;
    f(i, j);
    i = j;
  }
}

}  // namespace
}  // namespace aegkv

using namespace aegkv;

extern "C" {

int aegkv_copy_blocks(const void* src_pool, uint64_t n_src_blocks, void* dst_pool,
                      uint64_t n_dst_blocks, const int64_t* src_ids,
                      const int64_t* dst_ids, int64_t n, uint64_t block_bytes,
                      aegkv_stream_t stream) {
  return copy_blocks_checked(src_pool, n_src_blocks, dst_pool, n_dst_blocks, src_ids,
                             dst_ids, n, block_bytes, false, (hipStream_t)stream);
}

int aegkv_pack_blocks(const void* pool, uint64_t n_pool_blocks, const int64_t* ids,
                      int64_t n, void* staging, uint64_t block_bytes,
                      aegkv_stream_t stream) {
  if (!ids && n > 0) return AEGKV_ERR_INVALID_ARG;
  return copy_blocks_checked(pool, n_pool_blocks, staging, n > 0 ? (uint64_t)n : 0, ids,
                             nullptr, n, block_bytes, false, (hipStream_t)stream);
}

int aegkv_scatter_blocks(const void* staging, const int64_t* ids, int64_t n, void* pool,
                         uint64_t n_pool_blocks, uint64_t block_bytes,
                         aegkv_stream_t stream) {
  if (!ids && n > 0) return AEGKV_ERR_INVALID_ARG;
  return copy_blocks_checked(staging, n > 0 ? (uint64_t)n : 0, pool, n_pool_blocks,
                             nullptr, ids, n, block_bytes, false, (hipStream_t)stream);
}

int aegkv_defrag_blocks(void* pool, uint64_t n_pool_blocks, const int64_t* src_ids,
                        const int64_t* dst_ids, int64_t n, uint64_t block_bytes,
                        aegkv_stream_t stream) {
  if ((!src_ids || !dst_ids) && n > 0) return AEGKV_ERR_INVALID_ARG;
  return copy_blocks_checked(pool, n_pool_blocks, pool, n_pool_blocks, src_ids, dst_ids, n,
                             block_bytes, true, (hipStream_t)stream);
}

static int aegkv_swap_blocks_body(const int64_t* src_ids, const int64_t* dst_ids, int64_t n,
                      int is_swap_in, void* dev_pool, uint64_t n_dev_blocks,
                      void* host_pool, uint64_t n_host_blocks, uint64_t block_bytes,
                      void* staging, uint64_t staging_bytes, aegkv_stream_t stream_) {
  hipStream_t stream = (hipStream_t)stream_;
  if (n < 0 || !dev_pool || !host_pool || block_bytes == 0) return AEGKV_ERR_INVALID_ARG;
  if (n == 0) return AEGKV_OK;
  if (!src_ids || !dst_ids) return AEGKV_ERR_INVALID_ARG;
  if (n_dev_blocks > UINT64_MAX / block_bytes || n_host_blocks > UINT64_MAX / block_bytes)
    return AEGKV_ERR_INVALID_ARG;
  const uint64_t n_src = is_swap_in ? n_host_blocks : n_dev_blocks;
  const uint64_t n_dst = is_swap_in ? n_dev_blocks : n_host_blocks;
  int rc;
  if ((rc = check_ids_in_range(src_ids, n, n_src))) return rc;
  if ((rc = check_ids_in_range(dst_ids, n, n_dst))) return rc;
  if ((rc = check_unique(dst_ids, n, n_dst))) return rc;

  uint8_t* dev = static_cast<uint8_t*>(dev_pool);
  uint8_t* host = static_cast<uint8_t*>(host_pool);
  const uint64_t bb = block_bytes;
  // Host-side order: sort the pairs by their host block id so that runs of
  // consecutive host ids become single DMAs.
  const int64_t* host_key = is_swap_in ? src_ids : dst_ids;
  std::vector<int64_t> order(n);
  std::iota(order.begin(), order.end(), 0);
  std::stable_sort(order.begin(), order.end(),
                   [&](int64_t a, int64_t b) { return host_key[a] < host_key[b]; });

  const bool staged = staging && staging_bytes >= bb;
  if (!staged) {
    // One DMA per run where both ids advance by one (the reference issues one
    // cudaMemcpyAsync per block, swap.cu:36-58).
    int64_t i = 0;
    while (i < n) {
      int64_t j = i + 1;
      while (j < n && src_ids[order[j]] == src_ids[order[j - 1]] + 1 &&
             dst_ids[order[j]] == dst_ids[order[j - 1]] + 1)
        ++j;
      const uint64_t bytes = (uint64_t)(j - i) * bb;
      const uint64_t so = (uint64_t)src_ids[order[i]] * bb, dof = (uint64_t)dst_ids[order[i]] * bb;
      if (is_swap_in)
        AEGKV_HIP_TRY(hipMemcpyAsync(dev + dof, host + so, bytes, hipMemcpyHostToDevice, stream));
      else
        AEGKV_HIP_TRY(hipMemcpyAsync(host + dof, dev + so, bytes, hipMemcpyDeviceToHost, stream));
      i = j;
    }
    return AEGKV_OK;
  }
  if ((bb & 15) || !aligned16(dev_pool) || !aligned16(staging)) return AEGKV_ERR_MISALIGNED;

  DeviceState* ds = nullptr;
  if ((rc = current_device_state(&ds))) return rc;
  uint8_t* stg = static_cast<uint8_t*>(staging);
  const int64_t cap = (int64_t)std::min<uint64_t>(staging_bytes / bb, (uint64_t)n);
  std::vector<int64_t> dev_ids(cap);
  for (int64_t c0 = 0; c0 < n; c0 += cap) {
    const int64_t m = std::min(cap, n - c0);
    const int64_t* dev_key = is_swap_in ? dst_ids : src_ids;
    for (int64_t k = 0; k < m; ++k) dev_ids[k] = dev_key[order[c0 + k]];
    IdPart part{dev_ids.data(), m};
    if (!is_swap_in) {
      // gather scattered device blocks into staging, then DMA each host run
      rc = with_uploaded_ids(ds, stream, &part, 1, [&](int64_t* ids) {
        return launch_copy_blocks(ds, dev, stg, ids, nullptr, m, bb, stream);
      });
      if (rc) return rc;
      int err = 0;
      for_each_run(order, dst_ids, c0, c0 + m, [&](int64_t i, int64_t j) {
        if (err) return;
        hipError_t e = hipMemcpyAsync(host + (uint64_t)dst_ids[order[i]] * bb,
                                      stg + (uint64_t)(i - c0) * bb, (uint64_t)(j - i) * bb,
                                      hipMemcpyDeviceToHost, stream);
        if (e != hipSuccess) err = (int)e;
      });
      if (err) return err;
    } else {
      // DMA each host run into staging, then scatter to the device blocks
      int err = 0;
      for_each_run(order, src_ids, c0, c0 + m, [&](int64_t i, int64_t j) {
        if (err) return;
        hipError_t e = hipMemcpyAsync(stg + (uint64_t)(i - c0) * bb,
                                      host + (uint64_t)src_ids[order[i]] * bb,
                                      (uint64_t)(j - i) * bb, hipMemcpyHostToDevice, stream);
        if (e != hipSuccess) err = (int)e;
      });
      if (err) return err;
      rc = with_uploaded_ids(ds, stream, &part, 1, [&](int64_t* ids) {
        return launch_copy_blocks(ds, stg, dev, nullptr, ids, m, bb, stream);
      });
      if (rc) return rc;
    }
  }
  return AEGKV_OK;
}

int aegkv_swap_blocks(const int64_t* src_ids, const int64_t* dst_ids, int64_t n,
                      int is_swap_in, void* dev_pool, uint64_t n_dev_blocks,
                      void* host_pool, uint64_t n_host_blocks, uint64_t block_bytes,
                      void* staging, uint64_t staging_bytes, aegkv_stream_t stream) {
  return guarded([&] {
    return aegkv_swap_blocks_body(src_ids, dst_ids, n, is_swap_in, dev_pool, n_dev_blocks,
                                  host_pool, n_host_blocks, block_bytes, staging, staging_bytes,
                                  stream);
  });
}

}  // extern "C"

// ---- swap through a pageable host pool (the reference's /dev/shm file) ----
namespace {

// Host-side copies of one chunk, run by the HIP runtime in stream order
// (hipLaunchHostFunc): between the pinned bounce buffer and the pageable
// pool's blocks, spread over a few threads (a single thread copies ~10 GB/s).
struct BounceChunk {
  uint8_t* bounce;
  uint8_t* pool;
  uint64_t block_bytes;
  bool to_pool;                 // bounce -> pool (swap-out) or pool -> bounce
  std::vector<int64_t> ids;     // pool block of bounce slot k
};

void copy_bounce_chunk(void* user) {
  BounceChunk* c = static_cast<BounceChunk*>(user);
  const int64_t m = (int64_t)c->ids.size();
  const uint64_t bytes = (uint64_t)m * c->block_bytes;
  const unsigned hw = std::max(1u, std::thread::hardware_concurrency());
  const int nt = (int)std::min<uint64_t>({8, hw, std::max<uint64_t>(1, bytes >> 24)});
  auto work = [c, m, nt](int t) {
    // thread t copies an equal share of the chunk's bytes, block by block
    const uint64_t bb = c->block_bytes;
    const uint64_t total = (uint64_t)m * bb;
    const uint64_t lo = total * t / nt, hi = total * (t + 1) / nt;
    for (uint64_t off = lo; off < hi;) {
      const uint64_t k = off / bb, in = off % bb;
      const uint64_t len = std::min(bb - in, hi - off);
      uint8_t* slot = c->bounce + off;
      uint8_t* blk = c->pool + (uint64_t)c->ids[k] * bb + in;
      if (c->to_pool) std::memcpy(blk, slot, len);
      else std::memcpy(slot, blk, len);
      off += len;
    }
  };
  // Shares no thread could be started for (thread creation failing) are
  // copied here, so the callback never throws.
  std::vector<std::thread> th;
  int started = 1;
  for (int t = 1; t < nt; ++t) {
    try {
      th.emplace_back(work, t);
      ++started;
    } catch (...) {
      break;
    }
  }
  for (int t = started; t < nt; ++t) work(t);
  work(0);
  for (auto& x : th) x.join();
  delete c;
}

// The stream that runs the host copies of bounced swaps, one per device
// (default priority), so that a chunk's host copy overlaps the next chunk's
// DMA on the caller's stream.
int host_copy_stream(hipStream_t* out) {
  static std::mutex mu;
  static std::map<int, hipStream_t> streams;
  int dev = 0;
  AEGKV_HIP_TRY(hipGetDevice(&dev));
  std::lock_guard<std::mutex> lk(mu);
  auto it = streams.find(dev);
  if (it == streams.end()) {
    hipStream_t s = nullptr;
    AEGKV_HIP_TRY(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    it = streams.emplace(dev, s).first;
  }
  *out = it->second;
  return AEGKV_OK;
}

// Events of one bounced swap: created per call and released once enqueued (a
// destroyed event that is still pending is released by the runtime when it
// completes).
struct EventList {
  std::vector<hipEvent_t> ev;
  ~EventList() {
    for (hipEvent_t e : ev) (void)hipEventDestroy(e);
  }
  int record(hipStream_t s, hipEvent_t* out) {
    hipEvent_t e = nullptr;
    AEGKV_HIP_TRY(hipEventCreateWithFlags(&e, hipEventDisableTiming));
    ev.push_back(e);
    AEGKV_HIP_TRY(hipEventRecord(e, s));
    *out = e;
    return AEGKV_OK;
  }
};

}  // namespace

extern "C" {

static int aegkv_swap_blocks_bounced_body(const int64_t* src_ids, const int64_t* dst_ids, int64_t n,
                              int is_swap_in, void* dev_pool, uint64_t n_dev_blocks,
                              void* host_pool, uint64_t n_host_blocks, uint64_t block_bytes,
                              void* staging, uint64_t staging_bytes, void* bounce,
                              uint64_t bounce_bytes, aegkv_stream_t stream_) {
  hipStream_t stream = (hipStream_t)stream_;
  if (n < 0 || !dev_pool || !host_pool || !staging || !bounce || block_bytes == 0)
    return AEGKV_ERR_INVALID_ARG;
  if (n == 0) return AEGKV_OK;
  if (!src_ids || !dst_ids) return AEGKV_ERR_INVALID_ARG;
  if (n_dev_blocks > UINT64_MAX / block_bytes || n_host_blocks > UINT64_MAX / block_bytes)
    return AEGKV_ERR_INVALID_ARG;
  const uint64_t n_src = is_swap_in ? n_host_blocks : n_dev_blocks;
  const uint64_t n_dst = is_swap_in ? n_dev_blocks : n_host_blocks;
  int rc;
  if ((rc = check_ids_in_range(src_ids, n, n_src))) return rc;
  if ((rc = check_ids_in_range(dst_ids, n, n_dst))) return rc;
  if ((rc = check_unique(dst_ids, n, n_dst))) return rc;
  const uint64_t bb = block_bytes;
  if ((bb & 15) || !aligned16(dev_pool) || !aligned16(staging)) return AEGKV_ERR_MISALIGNED;
  if (std::min(staging_bytes, bounce_bytes) / bb == 0) return AEGKV_ERR_WORKSPACE;
  // The bounce buffer is cut into two halves when each holds a block and
  // there is more than one chunk to move: chunk k uses half k % 2, so its
  // host copy overlaps the next chunk's DMA, and half reuse waits for the
  // chunk two back.
  const uint64_t halves = (bounce_bytes / bb >= 2 && (uint64_t)n > 1) ? 2 : 1;
  const uint64_t half_bytes = bounce_bytes / halves / bb * bb;
  const int64_t cap =
      (int64_t)std::min<uint64_t>({staging_bytes / bb, half_bytes / bb, (uint64_t)n});
  DeviceState* ds = nullptr;
  if ((rc = current_device_state(&ds))) return rc;
  hipStream_t hs = nullptr;  // host copies
  if ((rc = host_copy_stream(&hs))) return rc;
  uint8_t* dev = static_cast<uint8_t*>(dev_pool);
  uint8_t* host = static_cast<uint8_t*>(host_pool);
  uint8_t* stg = static_cast<uint8_t*>(staging);
  const int64_t* dev_key = is_swap_in ? dst_ids : src_ids;
  const int64_t* host_key = is_swap_in ? src_ids : dst_ids;
  EventList events;
  std::vector<hipEvent_t> done;  // per chunk: its half may be reused after this
  hipEvent_t ev = nullptr;
  if (is_swap_in) {
    // the host reads the file after the caller's earlier work on its stream
    if ((rc = events.record(stream, &ev))) return rc;
    AEGKV_HIP_TRY(hipStreamWaitEvent(hs, ev, 0));
  }
  for (int64_t c0 = 0, k = 0; c0 < n; c0 += cap, ++k) {
    const int64_t m = std::min(cap, n - c0);
    uint8_t* half = static_cast<uint8_t*>(bounce) + (uint64_t)(k % (int64_t)halves) * half_bytes;
    BounceChunk* chunk = nullptr;
    try {
      chunk = new BounceChunk{half, host, bb, !is_swap_in,
                              std::vector<int64_t>(host_key + c0, host_key + c0 + m)};
    } catch (...) {
      return AEGKV_ERR_RUNTIME;
    }
    IdPart part{dev_key + c0, m};
    const bool reuse = k >= (int64_t)halves;  // the half held chunk k - halves
    if (!is_swap_in) {
      // pack the device blocks and DMA them to the half (once its previous
      // host copy is done); the host copy stream then writes them to the pool
      rc = with_uploaded_ids(ds, stream, &part, 1, [&](int64_t* ids) {
        return launch_copy_blocks(ds, dev, stg, ids, nullptr, m, bb, stream);
      });
      hipError_t e = hipSuccess;
      if (!rc && reuse) e = hipStreamWaitEvent(stream, done[k - halves], 0);
      if (!rc && e == hipSuccess)
        e = hipMemcpyAsync(half, stg, (uint64_t)m * bb, hipMemcpyDeviceToHost, stream);
      if (!rc && e == hipSuccess) rc = events.record(stream, &ev);
      if (!rc && e == hipSuccess) e = hipStreamWaitEvent(hs, ev, 0);
      if (!rc && e == hipSuccess) e = hipLaunchHostFunc(hs, copy_bounce_chunk, chunk);
      if (rc || e != hipSuccess) {
        delete chunk;
        return rc ? rc : (int)e;
      }
      if ((rc = events.record(hs, &ev))) return rc;
      done.push_back(ev);
    } else {
      // the host gathers the pool's blocks into the half (once the DMA of its
      // previous chunk is done), then one DMA takes them to staging and the
      // scatter kernel places them
      hipError_t e = hipSuccess;
      if (reuse) e = hipStreamWaitEvent(hs, done[k - halves], 0);
      if (e == hipSuccess) e = hipLaunchHostFunc(hs, copy_bounce_chunk, chunk);
      if (e != hipSuccess) {
        delete chunk;
        return (int)e;
      }
      if ((rc = events.record(hs, &ev))) return rc;
      AEGKV_HIP_TRY(hipStreamWaitEvent(stream, ev, 0));
      AEGKV_HIP_TRY(hipMemcpyAsync(stg, half, (uint64_t)m * bb, hipMemcpyHostToDevice, stream));
      if ((rc = events.record(stream, &ev))) return rc;
      done.push_back(ev);
      rc = with_uploaded_ids(ds, stream, &part, 1, [&](int64_t* ids) {
        return launch_copy_blocks(ds, stg, dev, nullptr, ids, m, bb, stream);
      });
      if (rc) return rc;
    }
  }
  // the caller's stream passes the swap-out only once its last host copy ran
  if (!is_swap_in) AEGKV_HIP_TRY(hipStreamWaitEvent(stream, done.back(), 0));
  return AEGKV_OK;
}

int aegkv_swap_blocks_bounced(const int64_t* src_ids, const int64_t* dst_ids, int64_t n,
                              int is_swap_in, void* dev_pool, uint64_t n_dev_blocks,
                              void* host_pool, uint64_t n_host_blocks, uint64_t block_bytes,
                              void* staging, uint64_t staging_bytes, void* bounce,
                              uint64_t bounce_bytes, aegkv_stream_t stream) {
  return guarded([&] {
    return aegkv_swap_blocks_bounced_body(src_ids, dst_ids, n, is_swap_in, dev_pool,
                                          n_dev_blocks, host_pool, n_host_blocks, block_bytes,
                                          staging, staging_bytes, bounce, bounce_bytes, stream);
  });
}

}  // extern "C"
