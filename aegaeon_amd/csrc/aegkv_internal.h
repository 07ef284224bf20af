// Internal helpers shared by the aegkv translation units: status mapping,
// argument checks and the per-device id upload ring.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <deque>
#include <mutex>
#include <new>
#include <vector>

#include "../../include/aegkv.h"

namespace aegkv {

#define AEGKV_HIP_TRY(expr)                          \
  do {                                               \
    hipError_t aegkv_e_ = (expr);                    \
    if (aegkv_e_ != hipSuccess) return (int)aegkv_e_; \
  } while (0)

inline bool aligned16(const void* p) {
  return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}

// Runs an entry point's body so that no exception crosses the C ABI: a failed
// host allocation returns AEGKV_ERR_HOST_MEMORY.
template <typename F>
int guarded(F&& body) {
  try {
    return body();
  } catch (const std::bad_alloc&) {
    return AEGKV_ERR_HOST_MEMORY;
  } catch (...) {
    return AEGKV_ERR_HOST_MEMORY;  // std::length_error and the like from the containers
  }
}

// Host-side validation of an id list against a pool of n_pool blocks.
int check_ids_in_range(const int64_t* ids, int64_t n, uint64_t n_pool);
// AEGKV_ERR_DUPLICATE if any id appears twice (ids already checked to lie in
// [0, n_pool)).
int check_unique(const int64_t* ids, int64_t n, uint64_t n_pool);
// AEGKV_ERR_OVERLAP if the two id sets intersect (ids in [0, n_pool)).
int check_disjoint(const int64_t* a, int64_t na, const int64_t* b, int64_t nb, uint64_t n_pool);

// Per-device state: compute-unit count and the id upload ring.  Host id lists
// are copied into a pinned host slice and DMA'd to the matching device slice on
// the caller's stream; an event recorded after the consuming kernel guards the
// slice until the device is done with it.  When the next slice would overlap
// one the device has not finished with, the ring grows (doubling, up to
// kRingGrowMax elements) instead of waiting, so a caller that enqueues many
// calls ahead of the device is not blocked; past that size it waits for the
// overlapped slices.  A replaced ring stays allocated until the process ends
// (its slices may still be read, and freeing device memory would synchronise
// the device).
struct DeviceState {
  int device = -1;
  int num_cu = 0;
  int max_lds = 0;  // bytes of LDS one workgroup may use
  std::mutex mu;
  int64_t* host_ring = nullptr;
  int64_t* dev_ring = nullptr;
  size_t cap = 0;   // elements
  size_t head = 0;  // next free element
  struct Span {
    size_t begin, end;
    hipEvent_t ev;
  };
  std::deque<Span> inflight;       // slices of the current ring
  std::deque<hipEvent_t> retired;   // events of slices of replaced rings
  std::vector<int64_t*> old_rings;  // replaced rings (host and device), kept
  std::vector<hipEvent_t> spare_events;
};
constexpr size_t kRingInitial = (size_t)1 << 17;  // elements (1 MiB each side)
constexpr size_t kRingGrowMax = (size_t)1 << 22;  // elements (32 MiB each side)

// State of the current device (created on first use).  Returns 0 or a status.
int current_device_state(DeviceState** out);

// Copies the concatenation of `parts` (host arrays) to device memory on
// `stream`, calls launch(dev_ptr) and guards the slice with an event recorded
// after the launch.  The device state's mutex is held for the duration.
struct IdPart {
  const int64_t* ptr;
  int64_t n;
};
template <typename Launch>
int with_uploaded_ids(DeviceState* ds, hipStream_t stream, const IdPart* parts,
                      int nparts, Launch&& launch);

// --- implementation of the template (needs ring primitives) ---------------
int ring_acquire(DeviceState* ds, size_t n, size_t* begin);  // mutex held
int ring_commit(DeviceState* ds, hipStream_t stream, size_t begin, size_t n);

template <typename Launch>
int with_uploaded_ids(DeviceState* ds, hipStream_t stream, const IdPart* parts,
                      int nparts, Launch&& launch) {
  size_t total = 0;
  for (int i = 0; i < nparts; ++i) total += (size_t)parts[i].n;
  std::lock_guard<std::mutex> lk(ds->mu);
  size_t begin = 0;
  if (total > 0) {
    int rc = ring_acquire(ds, total, &begin);
    if (rc) return rc;
    size_t off = begin;
    for (int i = 0; i < nparts; ++i) {
      for (int64_t k = 0; k < parts[i].n; ++k) ds->host_ring[off + k] = parts[i].ptr[k];
      off += (size_t)parts[i].n;
    }
    AEGKV_HIP_TRY(hipMemcpyAsync(ds->dev_ring + begin, ds->host_ring + begin,
                                 total * sizeof(int64_t), hipMemcpyHostToDevice,
                                 stream));
  }
  int rc = launch(total > 0 ? ds->dev_ring + begin : nullptr);
  if (total > 0) {
    int rc2 = ring_commit(ds, stream, begin, total);
    if (rc == 0) rc = rc2;
  }
  return rc;
}

// Raw buffer ranges for the byte-moving kernels.  kRawBufferWord3 is word 3
// of a gfx9-family buffer descriptor (32-bit data format, no swizzle); kNt is
// the nontemporal cache-policy bit of its buffer instructions.
constexpr int kRawBufferWord3 = 0x00020000;
constexpr int kNt = 2;

// A raw buffer range [p, p + bytes) of the workgroup-uniform p and bytes, both
// read from lane 0 so the descriptor lives in scalar registers (a per-lane
// descriptor would make the compiler loop over its distinct values).  Loads
// past its end return zero and stores past its end are dropped by the
// hardware's range check, so a partial tile needs no exec branch around its
// memory accesses and the compiler's vector-memory wait counts stay exact.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t byte_range(const uint8_t* p, uint32_t bytes) {
  const uint64_t u = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)u);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(u >> 32));
  uint8_t* base = reinterpret_cast<uint8_t*>(((uint64_t)hi << 32) | lo);
  return __builtin_amdgcn_make_buffer_rsrc(base, 0, __builtin_amdgcn_readfirstlane((int)bytes),
                                           kRawBufferWord3);
}

// Block-copy launcher shared by pack/scatter/copy/defrag/swap:
// dst[dst_ids ? dst_ids[i] : dst_base_index + i] <- src[src_ids ? src_ids[i] : src_base_index + i]
// for i in [0, n); the id arrays are DEVICE pointers (or null).
int launch_copy_blocks(const DeviceState* ds, const void* src, void* dst,
                       const int64_t* src_ids_dev, const int64_t* dst_ids_dev,
                       int64_t n, uint64_t block_bytes, hipStream_t stream);

}  // namespace aegkv
