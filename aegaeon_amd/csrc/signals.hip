// Cross-process move signals: the stream-ordered "this move has finished"
// that the reference passes between worker processes as interprocess CUDA
// events (reduce_cuda_event / rebuild_cuda_event, aegaeon/aegaeon/utils.py:
// 306-331; recorded at worker.py:740,765 and waited on at :772-815).
//
// A signal array is a few 64-bit timeline words in device memory that one
// process allocates and exports with hipIpcGetMemHandle; other processes on the
// node open it.  The allocation starts with a header word holding the array's
// word count, so an opening process learns the bounds; the words handed out
// follow it.  A producer stream finishes a move with signal_set (one lane
// stores the move's serial with a system-scope release after everything
// before it in the stream); a consumer stream that must not start before that
// move runs signal_wait (one lane polls the word with system-scope acquire
// loads and s_sleep until it reaches the serial).  A word has one writer, the
// stream that owns it, and its serials grow in that stream's order, so
// "word >= serial" means "every move of that stream up to this one is done".
//
// The wait is bounded: after timeout_us of wall-clock time the lane stores 1
// into the caller's timed_out word and exits, so the kernel always ends (the
// work behind it then runs unordered, and the caller learns so from the word).
#include <cstring>

#include "aegkv_internal.h"

namespace aegkv {
namespace {

constexpr int64_t kMaxSignalWords = 1 << 20;

__global__ __launch_bounds__(64) void signal_set_kernel(uint64_t* word, uint64_t value) {
  if (threadIdx.x == 0)
    __hip_atomic_store(word, value, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
}

__global__ __launch_bounds__(64) void signal_wait_kernel(const uint64_t* word, uint64_t value,
                                                         uint64_t ticks, uint32_t* timed_out) {
  if (threadIdx.x != 0) return;
  const uint64_t t0 = wall_clock64();
  while (__hip_atomic_load(word, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_SYSTEM) < value) {
    if (wall_clock64() - t0 > ticks) {
      if (timed_out) __hip_atomic_store(timed_out, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
      return;
    }
    __builtin_amdgcn_s_sleep(32);
  }
}

}  // namespace
}  // namespace aegkv

using namespace aegkv;

extern "C" {

int aegkv_signals_create(int64_t n_words, void** words, void* ipc_handle) {
  if (n_words <= 0 || n_words > kMaxSignalWords || !words || !ipc_handle)
    return AEGKV_ERR_INVALID_ARG;
  const size_t bytes = (size_t)(n_words + 1) * sizeof(uint64_t);
  void* p = nullptr;
  AEGKV_HIP_TRY(hipMalloc(&p, bytes));
  const uint64_t header = (uint64_t)n_words;
  hipError_t e = hipMemset(p, 0, bytes);
  if (e == hipSuccess) e = hipMemcpy(p, &header, sizeof(header), hipMemcpyHostToDevice);
  hipIpcMemHandle_t h;
  if (e == hipSuccess) e = hipIpcGetMemHandle(&h, p);
  if (e != hipSuccess) {
    (void)hipFree(p);
    return (int)e;
  }
  std::memcpy(ipc_handle, &h, sizeof(h));
  *words = static_cast<uint64_t*>(p) + 1;
  return AEGKV_OK;
}

int aegkv_signals_destroy(void* words) {
  if (!words) return AEGKV_ERR_INVALID_ARG;
  AEGKV_HIP_TRY(hipFree(static_cast<uint64_t*>(words) - 1));
  return AEGKV_OK;
}

int aegkv_signals_open(const void* ipc_handle, void** words, int64_t* n_words) {
  if (!ipc_handle || !words || !n_words) return AEGKV_ERR_INVALID_ARG;
  hipIpcMemHandle_t h;
  std::memcpy(&h, ipc_handle, sizeof(h));
  void* p = nullptr;
  AEGKV_HIP_TRY(hipIpcOpenMemHandle(&p, h, hipIpcMemLazyEnablePeerAccess));
  uint64_t header = 0;
  const hipError_t e = hipMemcpy(&header, p, sizeof(header), hipMemcpyDeviceToHost);
  if (e != hipSuccess || header == 0 || header > (uint64_t)kMaxSignalWords) {
    (void)hipIpcCloseMemHandle(p);
    return e != hipSuccess ? (int)e : AEGKV_ERR_INVALID_ARG;
  }
  *words = static_cast<uint64_t*>(p) + 1;
  *n_words = (int64_t)header;
  return AEGKV_OK;
}

int aegkv_signals_close(void* words) {
  if (!words) return AEGKV_ERR_INVALID_ARG;
  AEGKV_HIP_TRY(hipIpcCloseMemHandle(static_cast<uint64_t*>(words) - 1));
  return AEGKV_OK;
}

int aegkv_signal_set(void* word, uint64_t value, aegkv_stream_t stream) {
  if (!word || (reinterpret_cast<uintptr_t>(word) & 7)) return AEGKV_ERR_INVALID_ARG;
  hipLaunchKernelGGL(signal_set_kernel, dim3(1), dim3(64), 0, (hipStream_t)stream,
                     static_cast<uint64_t*>(word), value);
  AEGKV_HIP_TRY(hipGetLastError());
  return AEGKV_OK;
}

// The current value of a word, for a host that polls a move (the reference's
// cudaEventQuery on a rebuilt event): a copy on the caller's stream, waited for.
int aegkv_signal_read(const void* word, uint64_t* value, aegkv_stream_t stream) {
  if (!word || !value || (reinterpret_cast<uintptr_t>(word) & 7)) return AEGKV_ERR_INVALID_ARG;
  AEGKV_HIP_TRY(hipMemcpyAsync(value, word, sizeof(uint64_t), hipMemcpyDeviceToHost,
                               (hipStream_t)stream));
  AEGKV_HIP_TRY(hipStreamSynchronize((hipStream_t)stream));
  return AEGKV_OK;
}

int aegkv_signal_wait(const void* word, uint64_t value, uint64_t timeout_us, uint32_t* timed_out,
                      aegkv_stream_t stream) {
  if (!word || (reinterpret_cast<uintptr_t>(word) & 7) || timeout_us == 0)
    return AEGKV_ERR_INVALID_ARG;
  int dev = 0, khz = 0;
  AEGKV_HIP_TRY(hipGetDevice(&dev));
  AEGKV_HIP_TRY(hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev));
  if (khz <= 0) return AEGKV_ERR_RUNTIME;
  const uint64_t ticks = timeout_us * (uint64_t)khz / 1000u;
  // A timeout word in pinned host memory is written through its device
  // mapping (the same address under unified addressing; asked, not assumed).
  if (timed_out) {
    hipPointerAttribute_t attr;
    AEGKV_HIP_TRY(hipPointerGetAttributes(&attr, timed_out));
    if (attr.type == hipMemoryTypeHost) {
      if (!attr.devicePointer) return AEGKV_ERR_INVALID_ARG;
      timed_out = static_cast<uint32_t*>(attr.devicePointer);
    } else if (attr.type != hipMemoryTypeDevice) {
      return AEGKV_ERR_INVALID_ARG;  // pageable host memory: the kernel cannot write it
    }
  }
  hipLaunchKernelGGL(signal_wait_kernel, dim3(1), dim3(64), 0, (hipStream_t)stream,
                     static_cast<const uint64_t*>(word), value, ticks, timed_out);
  AEGKV_HIP_TRY(hipGetLastError());
  return AEGKV_OK;
}

}  // extern "C"
