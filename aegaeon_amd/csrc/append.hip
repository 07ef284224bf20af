// Token-granular KV movement on gfx950:
//  - kv_append: slot-mapped write of new K/V rows into the paged pool, for one
//    layer (vLLM's reshape_and_cache_flash call) or every layer of the
//    reference's [N, L, 2, 16, Hkv, D] storage in one launch;
//  - gather_tokens: block-table-driven de-page of sequences into contiguous
//    [sum(len), Hkv, D] buffers.
// Both are pure byte movement: every lane moves 16-byte (dwordx4) chunks and a
// wave covers 1 KiB of a row, so a Qwen2.5-7B row (4 heads x 128 x 2 B) is one
// wave-wide load and one wave-wide store.
#include <algorithm>

#include "aegkv_internal.h"

namespace aegkv {
namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int kAppendThreads = 64;
constexpr int kAppendItems = 1;  // 16-byte chunks per lane

// Chunk c of the flattened (layer, kv, token, row-chunk) space.
struct AppendArgs {
  const uint8_t* key;
  const uint8_t* value;
  int64_t key_tok_b, val_tok_b, key_layer_b, val_layer_b;  // byte strides
  const int64_t* slots;
  uint8_t* kc;
  uint8_t* vc;
  int64_t blk_b, layer_b;  // cache byte strides
  int64_t n_slots;         // n_blocks * block_size
  uint32_t n_tokens;
  uint32_t row_chunks;     // row bytes / 16
  uint32_t block_size;
  uint32_t total_chunks;   // n_layers * 2 * n_tokens * row_chunks
};

// The source row of a chunk does not depend on its slot, so the K/V load and
// the slot load are issued together; only the store waits for the slot.  That
// keeps the dependent-latency chain at one HBM round trip plus the store.
// One chunk per lane in 64-lane workgroups (a wave per 1 KiB row at the
// Qwen2.5-7B shape) measured fastest on MI355X: the step is a single burst of
// loads and stores, and spreading it over the most workgroups (14336 for the
// 256-token x 28-layer step, 512 for one layer) shortens the burst; 2-8
// chunks per lane and 256-512-lane workgroups were 2-65% slower.  The K/V
// rows are read once and the cache rows are not read again before the
// attention of the step streams them, so both sides are non-temporal.
__global__ __launch_bounds__(kAppendThreads) void kv_append_kernel(AppendArgs a) {
  const uint32_t nthreads = gridDim.x * kAppendThreads;
  const uint32_t gid = blockIdx.x * kAppendThreads + threadIdx.x;
  u32x4 r[kAppendItems];
  int64_t s[kAppendItems];
  uint32_t chunk[kAppendItems], tok[kAppendItems], lk[kAppendItems];
#pragma unroll
  for (int k = 0; k < kAppendItems; ++k) {
    const uint32_t c = gid + k * nthreads;
    s[k] = -1;
    if (c < a.total_chunks) {
      chunk[k] = c % a.row_chunks;
      const uint32_t rest = c / a.row_chunks;
      tok[k] = rest % a.n_tokens;
      lk[k] = rest / a.n_tokens;  // layer * 2 + kv
      const uint32_t layer = lk[k] >> 1, kv = lk[k] & 1;
      const uint8_t* src = kv ? a.value + layer * a.val_layer_b + tok[k] * a.val_tok_b
                              : a.key + layer * a.key_layer_b + tok[k] * a.key_tok_b;
      s[k] = a.slots[tok[k]];
      r[k] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src) + chunk[k]);
    }
  }
#pragma unroll
  for (int k = 0; k < kAppendItems; ++k) {
    if (s[k] >= 0 && s[k] < a.n_slots) {
      const int64_t blk = s[k] / a.block_size, off = s[k] - blk * a.block_size;
      const uint32_t layer = lk[k] >> 1, kv = lk[k] & 1;
      uint8_t* dst = (kv ? a.vc : a.kc) + layer * a.layer_b + blk * a.blk_b +
                     off * (int64_t)a.row_chunks * 16;
      __builtin_nontemporal_store(r[k], reinterpret_cast<u32x4*>(dst) + chunk[k]);
    }
  }
}

// One workgroup per (logical block, sequence, layer*2+kv): the tokens of a
// block are contiguous rows in both the cache and the output, so the work is a
// straight copy of n_tok * row bytes.
struct GatherArgs {
  const uint8_t* kc;
  const uint8_t* vc;
  int64_t blk_b, layer_b;
  int64_t n_blocks;
  const int32_t* block_tables;
  int32_t max_blocks;
  const int32_t* seq_lens;
  const int32_t* cu_seqlens;
  uint8_t* out_k;
  uint8_t* out_v;
  int64_t out_tokens;  // capacity of the output in tokens
  int32_t max_seq_len;
  int64_t out_layer_b;
  uint32_t row_bytes;
  uint32_t block_size;
};

__global__ __launch_bounds__(256) void gather_tokens_kernel(GatherArgs a) {
  const int i = blockIdx.x, b = blockIdx.y;
  const int layer = blockIdx.z >> 1, kv = blockIdx.z & 1;
  const int len = min(max(a.seq_lens[b], 0), a.max_seq_len);
  const int first = i * (int)a.block_size;
  if (first >= len) return;
  const int64_t row0 = (int64_t)a.cu_seqlens[b] + first;  // first output token
  if (row0 < 0 || row0 >= a.out_tokens) return;
  const int n_tok = (int)min((int64_t)min((int)a.block_size, len - first), a.out_tokens - row0);
  const int32_t id = a.block_tables[(int64_t)b * a.max_blocks + i];
  if (id < 0 || id >= a.n_blocks) return;
  const uint8_t* src = (kv ? a.vc : a.kc) + layer * a.layer_b + (int64_t)id * a.blk_b;
  uint8_t* dst = (kv ? a.out_v : a.out_k) + layer * a.out_layer_b + row0 * a.row_bytes;
  const uint32_t n_chunks = (uint32_t)n_tok * (a.row_bytes / 16);
  for (uint32_t c = threadIdx.x; c < n_chunks; c += 4 * 256) {
    u32x4 r[4];
#pragma unroll
    for (int k = 0; k < 4; ++k)
      if (c + k * 256 < n_chunks) r[k] = reinterpret_cast<const u32x4*>(src)[c + k * 256];
#pragma unroll
    for (int k = 0; k < 4; ++k)
      if (c + k * 256 < n_chunks) reinterpret_cast<u32x4*>(dst)[c + k * 256] = r[k];
  }
}

}  // namespace
}  // namespace aegkv

using namespace aegkv;

extern "C" {

int aegkv_kv_append(const void* key, const void* value, int64_t key_token_stride,
                    int64_t value_token_stride, int64_t key_layer_stride,
                    int64_t value_layer_stride, const int64_t* slot_mapping,
                    int64_t n_tokens, void* key_cache, void* value_cache,
                    int64_t cache_block_stride, int64_t cache_layer_stride,
                    int64_t n_blocks, int32_t n_layers, int32_t block_size,
                    int32_t n_kv_heads, int32_t head_dim, int32_t elem_bytes,
                    aegkv_stream_t stream) {
  if (n_tokens < 0 || n_layers <= 0 || block_size <= 0 || n_kv_heads <= 0 ||
      head_dim <= 0 || n_blocks < 0)
    return AEGKV_ERR_INVALID_ARG;
  if (elem_bytes != 2) return AEGKV_ERR_UNSUPPORTED;
  if (n_tokens == 0 || n_blocks == 0) return AEGKV_OK;
  if (!key || !value || !slot_mapping || !key_cache || !value_cache) return AEGKV_ERR_INVALID_ARG;
  const int64_t row_bytes = (int64_t)n_kv_heads * head_dim * elem_bytes;
  const int64_t e = elem_bytes;
  if ((row_bytes & 15) || !aligned16(key) || !aligned16(value) || !aligned16(key_cache) ||
      !aligned16(value_cache) || ((key_token_stride * e) & 15) ||
      ((value_token_stride * e) & 15) || ((key_layer_stride * e) & 15) ||
      ((value_layer_stride * e) & 15) || ((cache_block_stride * e) & 15) ||
      ((cache_layer_stride * e) & 15))
    return AEGKV_ERR_MISALIGNED;
  const uint64_t total = (uint64_t)n_layers * 2 * (uint64_t)n_tokens * (uint64_t)(row_bytes / 16);
  if (total >= (1ull << 32)) return AEGKV_ERR_UNSUPPORTED;
  AppendArgs a;
  a.key = static_cast<const uint8_t*>(key);
  a.value = static_cast<const uint8_t*>(value);
  a.key_tok_b = key_token_stride * e;
  a.val_tok_b = value_token_stride * e;
  a.key_layer_b = key_layer_stride * e;
  a.val_layer_b = value_layer_stride * e;
  a.slots = slot_mapping;
  a.kc = static_cast<uint8_t*>(key_cache);
  a.vc = static_cast<uint8_t*>(value_cache);
  a.blk_b = cache_block_stride * e;
  a.layer_b = cache_layer_stride * e;
  a.n_slots = n_blocks * (int64_t)block_size;
  a.n_tokens = (uint32_t)n_tokens;
  a.row_chunks = (uint32_t)(row_bytes / 16);
  a.block_size = (uint32_t)block_size;
  a.total_chunks = (uint32_t)total;
  const uint64_t per_wg = (uint64_t)kAppendThreads * kAppendItems;
  const uint32_t grid = (uint32_t)((total + per_wg - 1) / per_wg);
  hipLaunchKernelGGL(kv_append_kernel, dim3(grid), dim3(kAppendThreads), 0,
                     (hipStream_t)stream, a);
  AEGKV_HIP_TRY(hipGetLastError());
  return AEGKV_OK;
}

int aegkv_gather_tokens(const void* key_cache, const void* value_cache,
                        int64_t cache_block_stride, int64_t cache_layer_stride,
                        int64_t n_blocks, const int32_t* block_tables, int32_t max_blocks,
                        const int32_t* seq_lens, const int32_t* cu_seqlens, int32_t batch,
                        int32_t max_seq_len, void* out_key, void* out_value,
                        int64_t out_tokens, int64_t out_layer_stride, int32_t n_layers,
                        int32_t block_size,
                        int32_t n_kv_heads, int32_t head_dim, int32_t elem_bytes,
                        aegkv_stream_t stream) {
  if (batch < 0 || max_seq_len < 0 || n_layers <= 0 || block_size <= 0 || n_kv_heads <= 0 ||
      head_dim <= 0 || max_blocks < 0 || n_blocks < 0 || out_tokens < 0)
    return AEGKV_ERR_INVALID_ARG;
  if (elem_bytes != 2) return AEGKV_ERR_UNSUPPORTED;
  if (batch == 0 || max_seq_len == 0 || out_tokens == 0) return AEGKV_OK;
  if (!key_cache || !value_cache || !block_tables || !seq_lens || !cu_seqlens || !out_key ||
      !out_value)
    return AEGKV_ERR_INVALID_ARG;
  const int64_t e = elem_bytes;
  const int64_t row_bytes = (int64_t)n_kv_heads * head_dim * e;
  if ((row_bytes & 15) || !aligned16(key_cache) || !aligned16(value_cache) ||
      !aligned16(out_key) || !aligned16(out_value) || ((cache_block_stride * e) & 15) ||
      ((cache_layer_stride * e) & 15) || ((out_layer_stride * e) & 15))
    return AEGKV_ERR_MISALIGNED;
  const int64_t blocks_needed = ((int64_t)max_seq_len + block_size - 1) / block_size;
  if (blocks_needed > max_blocks) return AEGKV_ERR_INVALID_ARG;
  if (batch > 65535 || (int64_t)n_layers * 2 > 65535) return AEGKV_ERR_UNSUPPORTED;
  GatherArgs a;
  a.kc = static_cast<const uint8_t*>(key_cache);
  a.vc = static_cast<const uint8_t*>(value_cache);
  a.blk_b = cache_block_stride * e;
  a.layer_b = cache_layer_stride * e;
  a.n_blocks = n_blocks;
  a.block_tables = block_tables;
  a.max_blocks = max_blocks;
  a.seq_lens = seq_lens;
  a.cu_seqlens = cu_seqlens;
  a.out_k = static_cast<uint8_t*>(out_key);
  a.out_v = static_cast<uint8_t*>(out_value);
  a.out_tokens = out_tokens;
  a.max_seq_len = max_seq_len;
  a.out_layer_b = out_layer_stride * e;
  a.row_bytes = (uint32_t)row_bytes;
  a.block_size = (uint32_t)block_size;
  hipLaunchKernelGGL(gather_tokens_kernel, dim3((uint32_t)blocks_needed, batch, n_layers * 2),
                     dim3(256), 0, (hipStream_t)stream, a);
  AEGKV_HIP_TRY(hipGetLastError());
  return AEGKV_OK;
}

}  // extern "C"
