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

// gather_tokens: the tokens of a logical block (<= block_size tokens) are
// contiguous rows in both the cache and the output, so a block is a straight
// copy of n_tok * row bytes.  A tile is one 16 KiB pass of one block of one
// sequence for one (layer, K/V).  Each workgroup scans the batch's tile counts
// into LDS, then a persistent grid walks the flattened (layer, K/V, sequence,
// block, pass) tiles round-robin; the block id and output row of a workgroup's
// next tile are fetched while the current tile's non-temporal loads are in
// flight.  (One workgroup per block spent a dependent id load per 16 KiB and
// ran at 4.9 TB/s on the Qwen2.5-7B batch; this walk reaches 5.6 TB/s.
// Measured and dropped: two tiles in flight per workgroup, with the ids two
// tiles ahead, 5.0-5.5 TB/s over 8-64 workgroups per CU; a tile order that
// puts a block's K and V passes side by side (32 KiB adjacent reads),
// 5.3-5.5 TB/s.  The same 16 KiB units moved by the block-copy kernel (one
// wave per 1 KiB) run at 5.52-5.54 TB/s, a contiguous copy of the same bytes
// at 6.3 TB/s: the scattered 16 KiB sources are the bound.)
constexpr int kGatherThreads = 256;
constexpr int kGatherMaxBatch = 1024;  // sequences per launch (LDS scan)
constexpr int kGatherWorkgroupsPerCu = 64;  // 8..256 measured: 64 best, 128 10% and 256 40% slower
constexpr uint32_t kGatherPassBytes = kGatherThreads * 16 * 4;  // 16 KiB per pass

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
  int32_t batch;       // <= kGatherMaxBatch
  int32_t n_lk;        // 2 * n_layers
  int32_t passes;      // 16 KiB passes per block tile (rows wider than 1 KiB: more than one)
};

__global__ __launch_bounds__(kGatherThreads) void gather_tokens_kernel(GatherArgs a) {
  __shared__ int32_t pre[kGatherMaxBatch + 1];  // first tile of each sequence
  __shared__ int32_t lens[kGatherMaxBatch];
  __shared__ int32_t wsum[kGatherThreads / 64];
  constexpr int PER = kGatherMaxBatch / kGatherThreads;
  const int t = threadIdx.x, B = a.batch;
  const int bs = (int)a.block_size;
  int cnt[PER], run = 0;
#pragma unroll
  for (int k = 0; k < PER; ++k) {  // loads issued together, clamped in bounds
    const int b = t * PER + k;
    const int raw = a.seq_lens[min(b, B - 1)];
    const int len = b < B ? min(max(raw, 0), a.max_seq_len) : 0;
    if (b < B) lens[b] = len;
    cnt[k] = (len + bs - 1) / bs;
    run += cnt[k];
  }
  int incl = run;  // inclusive scan over the workgroup
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_up(incl, off);
    if ((t & 63) >= off) incl += y;
  }
  if ((t & 63) == 63) wsum[t >> 6] = incl;
  __syncthreads();
  int excl = incl - run;
  for (int w = 0; w < (t >> 6); ++w) excl += wsum[w];
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    const int b = t * PER + k;
    if (b <= B) pre[b] = excl;
    excl += cnt[k];
  }
  if (t == kGatherThreads - 1) pre[B] = excl;  // total (B may equal the capacity)
  __syncthreads();
  // tiles: (layer*2+kv, block tile, pass), pass p covering bytes
  // [16 KiB p, 16 KiB (p + 1)) of the block tile
  const int64_t T = (int64_t)pre[B] * a.passes;
  const int64_t total = T * a.n_lk;
  int64_t g = blockIdx.x;
  if (g >= total) return;  // uniform

  // tile g -> (lk, b, j, pass): b is the last sequence whose first block
  // tile is <= the tile's block index
  auto locate = [&](int64_t gg, int& lk, int& b, int& j, int& ps) {
    lk = (int)(gg / T);
    int r = (int)(gg - (int64_t)lk * T);
    ps = r % a.passes;
    r /= a.passes;
    int lo = 0, hi = B - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (pre[mid] <= r) lo = mid;
      else hi = mid - 1;
    }
    b = lo;
    j = r - pre[lo];
  };
  int lk, b, j, ps;
  locate(g, lk, b, j, ps);
  int32_t id = a.block_tables[(int64_t)b * a.max_blocks + j];
  int64_t row0 = a.cu_seqlens[b];
  while (true) {
    // current tile: one straight pass of at most 16 KiB, so the loop body
    // holds no inner loop and its vector-memory waits stay exact
    const int layer = lk >> 1, kv = lk & 1;
    const int64_t row = row0 + (int64_t)j * bs;
    int n_tok = min(bs, lens[b] - j * bs);
    if (row < 0 || row >= a.out_tokens || id < 0 || id >= a.n_blocks) n_tok = 0;
    else n_tok = (int)min((int64_t)n_tok, a.out_tokens - row);
    const int64_t tile_bytes = (int64_t)n_tok * a.row_bytes - (int64_t)ps * kGatherPassBytes;
    const uint32_t bytes = (uint32_t)max((int64_t)0, min(tile_bytes, (int64_t)kGatherPassBytes));
    const uint64_t pass_off = (uint64_t)ps * kGatherPassBytes;
    // raw buffer ranges of `bytes` bytes: the hardware's range check drops
    // the lanes past the end, so every load and store below issues and the
    // compiler counts them exactly (no exec branches around memory)
    const auto src = byte_range(
        (kv ? a.vc : a.kc) + layer * a.layer_b + (int64_t)max(id, 0) * a.blk_b + pass_off, bytes);
    const auto dst = byte_range((kv ? a.out_v : a.out_k) + layer * a.out_layer_b +
                                    max(row, (int64_t)0) * a.row_bytes + pass_off,
                                bytes);
    u32x4 r[4];
#pragma unroll
    for (int k = 0; k < 4; ++k)
      r[k] = __builtin_amdgcn_raw_buffer_load_b128(src, (k * kGatherThreads + t) * 16, 0, kNt);
    // next tile's id and output row, in flight with the loads above; issued
    // unconditionally (the last tile locates itself again), since a load
    // under a branch would make the stores below wait for it
    const int64_t gn = g + gridDim.x;
    const bool more = gn < total;
    int nlk, nb, nj, nps;
    locate(more ? gn : g, nlk, nb, nj, nps);
    const int32_t nid = a.block_tables[(int64_t)nb * a.max_blocks + nj];
    const int64_t nrow0 = a.cu_seqlens[nb];
#pragma unroll
    for (int k = 0; k < 4; ++k)
      __builtin_amdgcn_raw_buffer_store_b128(r[k], dst, (k * kGatherThreads + t) * 16, 0, kNt);
    if (!more) break;
    g = gn;
    lk = nlk;
    b = nb;
    j = nj;
    ps = nps;
    id = nid;
    row0 = nrow0;
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
  // chunks of the launch, counted in 128 bits so that no product wraps
  const unsigned __int128 total128 = (unsigned __int128)(uint64_t)n_layers * 2 *
                                     (uint64_t)n_tokens * (uint64_t)(row_bytes / 16);
  if (total128 >= ((unsigned __int128)1 << 32)) return AEGKV_ERR_UNSUPPORTED;
  const uint64_t total = (uint64_t)total128;
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
  if (row_bytes > INT32_MAX) return AEGKV_ERR_UNSUPPORTED;
  const int64_t blocks_needed = ((int64_t)max_seq_len + block_size - 1) / block_size;
  if (blocks_needed > max_blocks) return AEGKV_ERR_INVALID_ARG;
  const int64_t passes = ((int64_t)block_size * row_bytes + kGatherPassBytes - 1) / kGatherPassBytes;
  if (blocks_needed * kGatherMaxBatch * passes > INT32_MAX || (int64_t)n_layers * 2 > 65535)
    return AEGKV_ERR_UNSUPPORTED;
  DeviceState* ds = nullptr;
  int rc = current_device_state(&ds);
  if (rc) return rc;
  GatherArgs a;
  a.kc = static_cast<const uint8_t*>(key_cache);
  a.vc = static_cast<const uint8_t*>(value_cache);
  a.blk_b = cache_block_stride * e;
  a.layer_b = cache_layer_stride * e;
  a.n_blocks = n_blocks;
  a.max_blocks = max_blocks;
  a.out_k = static_cast<uint8_t*>(out_key);
  a.out_v = static_cast<uint8_t*>(out_value);
  a.out_tokens = out_tokens;
  a.max_seq_len = max_seq_len;
  a.out_layer_b = out_layer_stride * e;
  a.row_bytes = (uint32_t)row_bytes;
  a.block_size = (uint32_t)block_size;
  a.n_lk = 2 * n_layers;
  a.passes = (int32_t)passes;
  const int64_t max_grid = (int64_t)std::max(ds->num_cu, 1) * kGatherWorkgroupsPerCu;
  for (int32_t b0 = 0; b0 < batch; b0 += kGatherMaxBatch) {
    const int32_t nb = std::min(kGatherMaxBatch, batch - b0);
    a.batch = nb;
    a.block_tables = block_tables + (int64_t)b0 * max_blocks;
    a.seq_lens = seq_lens + b0;
    a.cu_seqlens = cu_seqlens + b0;
    const int64_t tiles_max = blocks_needed * nb * a.n_lk * a.passes;  // bound of the tiles
    const uint32_t grid = (uint32_t)std::max<int64_t>(1, std::min(tiles_max, max_grid));
    hipLaunchKernelGGL(gather_tokens_kernel, dim3(grid), dim3(kGatherThreads), 0,
                       (hipStream_t)stream, a);
    AEGKV_HIP_TRY(hipGetLastError());
  }
  return AEGKV_OK;
}

}  // extern "C"
