// Library runtime: status strings, version, per-device state and the id upload
// ring used to hand host id lists (the reference's std::vector<int64_t>
// arguments, aegaeon/ops/ops.h:4-10) to the block kernels without blocking the
// host.
#include <algorithm>
#include <map>

#include "aegkv_internal.h"

namespace aegkv {

int check_ids_in_range(const int64_t* ids, int64_t n, uint64_t n_pool) {
  for (int64_t i = 0; i < n; ++i)
    if (ids[i] < 0 || (uint64_t)ids[i] >= n_pool) return AEGKV_ERR_OUT_OF_RANGE;
  return AEGKV_OK;
}

namespace {
// Pools of up to 2^27 blocks are checked with a bitmap over the pool's ids: one
// pass to mark, one to clear the words it marked, so a call costs O(n) however
// large the pool (sorting 20,000 ids took ~1 ms).  The bitmap is per thread,
// all clear between calls, and keeps the largest size it has been given (at
// most 16 MiB).  Larger pools are checked with sorted copies.
constexpr uint64_t kBitmapMaxIds = 1ull << 27;

uint64_t* id_bitmap(uint64_t n_pool) {
  thread_local std::vector<uint64_t> bits;
  const size_t words = (n_pool + 63) / 64;
  if (bits.size() < words) bits.assign(words, 0);
  return bits.data();
}
inline uint64_t bit_of(int64_t id) { return 1ull << ((uint64_t)id & 63); }
void clear_marks(uint64_t* bits, const int64_t* ids, int64_t n) {
  for (int64_t i = 0; i < n; ++i) bits[(uint64_t)ids[i] >> 6] = 0;
}
}  // namespace

int check_unique(const int64_t* ids, int64_t n, uint64_t n_pool) {
  if (n_pool <= kBitmapMaxIds) {
    uint64_t* bits = id_bitmap(n_pool);
    int rc = AEGKV_OK;
    for (int64_t i = 0; i < n && rc == AEGKV_OK; ++i) {
      uint64_t& w = bits[(uint64_t)ids[i] >> 6];
      if (w & bit_of(ids[i])) rc = AEGKV_ERR_DUPLICATE;
      w |= bit_of(ids[i]);
    }
    clear_marks(bits, ids, n);
    return rc;
  }
  std::vector<int64_t> v(ids, ids + n);
  std::sort(v.begin(), v.end());
  for (size_t i = 1; i < v.size(); ++i)
    if (v[i] == v[i - 1]) return AEGKV_ERR_DUPLICATE;
  return AEGKV_OK;
}

int check_disjoint(const int64_t* a, int64_t na, const int64_t* b, int64_t nb, uint64_t n_pool) {
  if (n_pool <= kBitmapMaxIds) {
    uint64_t* bits = id_bitmap(n_pool);
    for (int64_t i = 0; i < na; ++i) bits[(uint64_t)a[i] >> 6] |= bit_of(a[i]);
    int rc = AEGKV_OK;
    for (int64_t i = 0; i < nb && rc == AEGKV_OK; ++i)
      if (bits[(uint64_t)b[i] >> 6] & bit_of(b[i])) rc = AEGKV_ERR_OVERLAP;
    clear_marks(bits, a, na);
    return rc;
  }
  std::vector<int64_t> x(a, a + na), y(b, b + nb);
  std::sort(x.begin(), x.end());
  std::sort(y.begin(), y.end());
  size_t i = 0, j = 0;
  while (i < x.size() && j < y.size()) {
    if (x[i] == y[j]) return AEGKV_ERR_OVERLAP;
    if (x[i] < y[j]) ++i; else ++j;
  }
  return AEGKV_OK;
}

namespace {
std::mutex g_states_mu;
std::map<int, DeviceState*> g_states;  // one per device, lives until exit

void release_span(DeviceState* ds, const DeviceState::Span& s) {
  ds->spare_events.push_back(s.ev);
}

// A new ring of at least `need` elements (doubling): the current one is kept
// allocated and its unfinished slices move to the retired events.
int ring_grow(DeviceState* ds, size_t need) {
  const size_t cap = std::max<size_t>({need, 2 * ds->cap, kRingInitial});
  int64_t* h = nullptr;
  int64_t* d = nullptr;
  AEGKV_HIP_TRY(hipHostMalloc((void**)&h, cap * sizeof(int64_t), hipHostMallocDefault));
  hipError_t e = hipMalloc((void**)&d, cap * sizeof(int64_t));
  if (e != hipSuccess) {
    (void)hipHostFree(h);  // never handed out
    return (int)e;
  }
  if (ds->host_ring) {
    ds->old_rings.push_back(ds->host_ring);
    ds->old_rings.push_back(ds->dev_ring);
  }
  for (const auto& sp : ds->inflight) ds->retired.push_back(sp.ev);
  ds->inflight.clear();
  ds->host_ring = h;
  ds->dev_ring = d;
  ds->cap = cap;
  ds->head = 0;
  return AEGKV_OK;
}
}  // namespace

int current_device_state(DeviceState** out) {
  int dev = 0;
  AEGKV_HIP_TRY(hipGetDevice(&dev));
  std::lock_guard<std::mutex> lk(g_states_mu);
  auto it = g_states.find(dev);
  if (it != g_states.end()) {
    *out = it->second;
    return AEGKV_OK;
  }
  auto* ds = new DeviceState();
  ds->device = dev;
  hipError_t e = hipDeviceGetAttribute(&ds->num_cu, hipDeviceAttributeMultiprocessorCount, dev);
  if (e == hipSuccess)
    e = hipDeviceGetAttribute(&ds->max_lds, hipDeviceAttributeMaxSharedMemoryPerBlock, dev);
  if (e != hipSuccess) {
    delete ds;
    return (int)e;
  }
  g_states[dev] = ds;
  *out = ds;
  return AEGKV_OK;
}

int ring_acquire(DeviceState* ds, size_t n, size_t* begin) {
  // Drop finished slices, of this ring and of replaced ones, oldest first (a
  // slice finished behind an unfinished older one is dropped later).
  while (!ds->inflight.empty() && hipEventQuery(ds->inflight.front().ev) == hipSuccess) {
    release_span(ds, ds->inflight.front());
    ds->inflight.pop_front();
  }
  while (!ds->retired.empty() && hipEventQuery(ds->retired.front()) == hipSuccess) {
    ds->spare_events.push_back(ds->retired.front());
    ds->retired.pop_front();
  }
  if (n > ds->cap) {
    int rc = ring_grow(ds, n);
    if (rc) return rc;
  }
  size_t b = ds->head + n > ds->cap ? 0 : ds->head;
  auto overlaps = [&](size_t lo) {
    for (const auto& sp : ds->inflight)
      if (sp.begin < lo + n && lo < sp.end) return true;
    return false;
  };
  if (overlaps(b)) {
    if (2 * ds->cap <= kRingGrowMax) {
      // the device is still reading that slice: a larger ring, not a wait
      int rc = ring_grow(ds, n);
      if (rc) return rc;
      b = 0;
    } else {
      // Wait for the overlapped slices (the ring is at its largest).
      for (auto it = ds->inflight.begin(); it != ds->inflight.end();) {
        if (it->begin < b + n && b < it->end) {
          hipError_t err = hipEventSynchronize(it->ev);
          release_span(ds, *it);
          it = ds->inflight.erase(it);
          if (err != hipSuccess) return (int)err;
        } else {
          ++it;
        }
      }
    }
  }
  ds->head = b + n;
  *begin = b;
  return AEGKV_OK;
}

int ring_commit(DeviceState* ds, hipStream_t stream, size_t begin, size_t n) {
  hipEvent_t ev;
  if (!ds->spare_events.empty()) {
    ev = ds->spare_events.back();
    ds->spare_events.pop_back();
  } else {
    AEGKV_HIP_TRY(hipEventCreateWithFlags(&ev, hipEventDisableTiming));
  }
  hipError_t e = hipEventRecord(ev, stream);
  if (e != hipSuccess) {
    ds->spare_events.push_back(ev);
    // The slice may still be read by the enqueued work: wait for the stream
    // before the ring can hand the slice out again.  If the wait fails too,
    // nothing proves the device is done with the ring, so it is abandoned
    // (left allocated, never reused); the next call grows a fresh one.
    if (hipStreamSynchronize(stream) != hipSuccess) {
      for (const auto& s : ds->inflight) ds->spare_events.push_back(s.ev);
      ds->inflight.clear();
      ds->host_ring = nullptr;
      ds->dev_ring = nullptr;
      ds->cap = 0;
      ds->head = 0;
    }
    return (int)e;
  }
  ds->inflight.push_back({begin, begin + n, ev});
  return AEGKV_OK;
}

}  // namespace aegkv

extern "C" {

const char* aegkv_strerror(int code) {
  switch (code) {
    case AEGKV_OK: return "aegkv: success";
    case AEGKV_ERR_INVALID_ARG: return "aegkv: invalid argument (null pointer, negative count or zero size)";
    case AEGKV_ERR_OUT_OF_RANGE: return "aegkv: block id out of range for its pool";
    case AEGKV_ERR_MISALIGNED: return "aegkv: pointer, stride or size is not 16-byte aligned";
    case AEGKV_ERR_OVERLAP: return "aegkv: source and destination block sets overlap";
    case AEGKV_ERR_DUPLICATE: return "aegkv: duplicate destination block id";
    case AEGKV_ERR_UNSUPPORTED: return "aegkv: unsupported shape or dtype";
    case AEGKV_ERR_WORKSPACE: return "aegkv: workspace or staging buffer too small";
    case AEGKV_ERR_RUNTIME: return "aegkv: a HIP runtime query failed while sizing the call";
    case AEGKV_ERR_NO_SPACE: return "aegkv: not enough free blocks after reclaiming moves";
    case AEGKV_ERR_IN_USE: return "aegkv: request lives elsewhere, is held by a suspended call, or the space still holds requests";
    case AEGKV_RECLAIM_PENDING: return "aegkv: the call is suspended until pending moves are reclaimed (aegkv_bm_pending / aegkv_bm_resume)";
    case AEGKV_ERR_SCRATCH: return "aegkv: the call needs a larger workspace than the 32 MiB the no-allocation entry point holds";
    case AEGKV_ERR_HOST_MEMORY: return "aegkv: a host-side allocation (id lists, bookkeeping) failed";
    default: break;
  }
  if (code > 0) return hipGetErrorString((hipError_t)code);
  return "aegkv: unknown status code";
}

int aegkv_version(void) { return (1 << 16) | 0; }

int aegkv_init(void) {
  aegkv::DeviceState* ds = nullptr;
  int rc = aegkv::current_device_state(&ds);
  if (rc) return rc;
  std::lock_guard<std::mutex> lk(ds->mu);
  if (ds->cap == 0) {
    size_t b = 0;
    rc = aegkv::ring_acquire(ds, 1, &b);
    if (rc) return rc;
    ds->head = 0;
  }
  return AEGKV_OK;
}

}  // extern "C"
