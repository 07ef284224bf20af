// Device-side preparation of the attention/append inputs of one forward step
// (replaces the host loops of aegaeon/aegaeon/worker.py:596-676 and
// make_tensor_with_pad, aegaeon/aegaeon/utils.py:241-257).
//
// The host hands over, per request, its block table, total length (seq_len)
// and first new token (context_len), plus the new tokens.  The library packs
// them with the prefix sums of the query and sequence lengths into one upload
// (the per-device id ring, one DMA) and one kernel writes every output:
//   block_tables[b][j]   = decode rows: table[b][j] for j < len(table[b]), else 0;
//                          prefill rows (context_len == 0): all 0  (worker.py:600-605)
//   slot_mapping[q0 + t] = table[b][p / bs] * bs + p % bs, p = context_len + t
//                          (worker.py:628-633)
//   positions[q0 + t]    = p,  input_tokens[q0 + t] = tokens of b      (worker.py:613-614)
//   seq_lens, context_lens, query_start_loc, seq_start_loc            (worker.py:652-673)
// with q0 = query_start_loc[b].  Workgroup (x, b) covers table columns and
// query tokens [256 x, 256 x + 256) of request b.
#include <algorithm>
#include <vector>

#include "aegkv_internal.h"

namespace aegkv {
namespace {

constexpr int kPrepThreads = 256;

struct PrepArgs {
  const int64_t* offsets;   // [B + 1] start of each table in `ids`
  const int64_t* q_start;   // [B + 1] prefix sums of query lengths
  const int64_t* s_start;   // [B + 1] prefix sums of sequence lengths
  const int64_t* seq_lens;  // [B]
  const int64_t* ctx_lens;  // [B]
  const int64_t* ids;       // concatenated block tables
  const int64_t* tokens;    // concatenated new tokens, in query order
  int32_t batch;
  int32_t block_size;
  int32_t pad_width;
  int32_t* block_tables;    // [B][pad_width]
  int64_t* slot_mapping;    // [n_query]
  int64_t* positions;       // [n_query]
  int64_t* input_tokens;    // [n_query] (may be null)
  int32_t* seq_lens_out;    // [B]
  int32_t* ctx_lens_out;    // [B]
  int32_t* query_start_loc; // [B + 1]
  int32_t* seq_start_loc;   // [B + 1]
};

__global__ __launch_bounds__(kPrepThreads) void prepare_inputs_kernel(PrepArgs a) {
  const int b = blockIdx.y;
  const int64_t col = (int64_t)blockIdx.x * kPrepThreads + threadIdx.x;
  const int64_t off = a.offsets[b], n_tab = a.offsets[b + 1] - off;
  const int64_t ctx = a.ctx_lens[b], seq = a.seq_lens[b];
  if (col < a.pad_width)
    a.block_tables[(int64_t)b * a.pad_width + col] =
        (ctx > 0 && col < n_tab) ? (int32_t)a.ids[off + col] : 0;
  if (col < seq - ctx) {
    const int64_t q = a.q_start[b] + col, p = ctx + col;
    a.slot_mapping[q] = a.ids[off + p / a.block_size] * a.block_size + p % a.block_size;
    a.positions[q] = p;
    if (a.input_tokens) a.input_tokens[q] = a.tokens[q];
  }
  if (col == 0) {
    a.seq_lens_out[b] = (int32_t)seq;
    a.ctx_lens_out[b] = (int32_t)ctx;
    a.query_start_loc[b] = (int32_t)a.q_start[b];
    a.seq_start_loc[b] = (int32_t)a.s_start[b];
    if (b == a.batch - 1) {
      a.query_start_loc[b + 1] = (int32_t)a.q_start[b + 1];
      a.seq_start_loc[b + 1] = (int32_t)a.s_start[b + 1];
    }
  }
}

}  // namespace
}  // namespace aegkv

using namespace aegkv;

extern "C" {

static int aegkv_prepare_inputs_body(const int32_t* block_ids, const int64_t* table_offsets,
                         const int32_t* seq_lens, const int32_t* context_lens,
                         const int64_t* tokens, int32_t batch, int32_t block_size,
                         int32_t pad_width, int32_t* block_tables_out,
                         int64_t* slot_mapping_out, int64_t* positions_out,
                         int64_t* input_tokens_out, int32_t* seq_lens_out,
                         int32_t* context_lens_out, int32_t* query_start_loc_out,
                         int32_t* seq_start_loc_out, int64_t n_query_tokens,
                         aegkv_stream_t stream_) {
  hipStream_t stream = (hipStream_t)stream_;
  if (batch < 0 || block_size <= 0 || pad_width < 0 || n_query_tokens < 0)
    return AEGKV_ERR_INVALID_ARG;
  if (batch == 0) return AEGKV_OK;
  if (batch > 65535) return AEGKV_ERR_UNSUPPORTED;
  if (!table_offsets || !seq_lens || !context_lens || !seq_lens_out || !context_lens_out ||
      !query_start_loc_out || !seq_start_loc_out || (pad_width > 0 && !block_tables_out) ||
      (n_query_tokens > 0 && (!slot_mapping_out || !positions_out)) ||
      (input_tokens_out && n_query_tokens > 0 && !tokens))
    return AEGKV_ERR_INVALID_ARG;
  // Host checks: lengths, table sizes, totals (the reference asserts or trusts).
  const int64_t n_ids = table_offsets[batch];
  if (table_offsets[0] != 0 || n_ids < 0 || (n_ids > 0 && !block_ids)) return AEGKV_ERR_INVALID_ARG;
  std::vector<int64_t> q_start(batch + 1), s_start(batch + 1);
  int64_t max_query = 0;
  for (int32_t b = 0; b < batch; ++b) {
    const int64_t n_tab = table_offsets[b + 1] - table_offsets[b];
    const int64_t seq = seq_lens[b], ctx = context_lens[b];
    if (n_tab < 0 || ctx < 0 || seq < ctx) return AEGKV_ERR_INVALID_ARG;
    // the slots of positions [ctx, seq) need table entries up to (seq - 1) / bs
    if (seq > ctx && (seq - 1) / block_size >= n_tab) return AEGKV_ERR_OUT_OF_RANGE;
    if (ctx > 0 && n_tab > pad_width) return AEGKV_ERR_INVALID_ARG;
    q_start[b + 1] = q_start[b] + (seq - ctx);
    s_start[b + 1] = s_start[b] + seq;
    max_query = std::max(max_query, seq - ctx);
  }
  if (q_start[batch] != n_query_tokens) return AEGKV_ERR_INVALID_ARG;
  if (q_start[batch] > INT32_MAX || s_start[batch] > INT32_MAX) return AEGKV_ERR_UNSUPPORTED;
  for (int64_t i = 0; i < n_ids; ++i)
    if (block_ids[i] < 0) return AEGKV_ERR_OUT_OF_RANGE;

  DeviceState* ds = nullptr;
  int rc = current_device_state(&ds);
  if (rc) return rc;
  // One upload: offsets, q_start, s_start, seq_lens, ctx_lens, ids, tokens.
  std::vector<int64_t> head((size_t)5 * batch + 3);
  for (int32_t b = 0; b <= batch; ++b) {
    head[b] = table_offsets[b];
    head[batch + 1 + b] = q_start[b];
    head[2 * (batch + 1) + b] = s_start[b];
  }
  for (int32_t b = 0; b < batch; ++b) {
    head[3 * (batch + 1) + b] = seq_lens[b];
    head[3 * (batch + 1) + batch + b] = context_lens[b];
  }
  std::vector<int64_t> ids64(block_ids ? block_ids : nullptr, block_ids ? block_ids + n_ids : nullptr);
  const bool with_tokens = input_tokens_out && n_query_tokens > 0;
  IdPart parts[3] = {{head.data(), (int64_t)head.size()},
                     {ids64.data(), n_ids},
                     {tokens, with_tokens ? n_query_tokens : 0}};
  return with_uploaded_ids(ds, stream, parts, 3, [&](int64_t* dev) {
    PrepArgs a;
    a.offsets = dev;
    a.q_start = dev + (batch + 1);
    a.s_start = dev + 2 * (batch + 1);
    a.seq_lens = dev + 3 * (batch + 1);
    a.ctx_lens = dev + 3 * (batch + 1) + batch;
    a.ids = dev + head.size();
    a.tokens = with_tokens ? dev + head.size() + n_ids : nullptr;
    a.batch = batch;
    a.block_size = block_size;
    a.pad_width = pad_width;
    a.block_tables = block_tables_out;
    a.slot_mapping = slot_mapping_out;
    a.positions = positions_out;
    a.input_tokens = with_tokens ? input_tokens_out : nullptr;
    a.seq_lens_out = seq_lens_out;
    a.ctx_lens_out = context_lens_out;
    a.query_start_loc = query_start_loc_out;
    a.seq_start_loc = seq_start_loc_out;
    const int64_t cols = std::max<int64_t>({(int64_t)pad_width, max_query, 1});
    const uint32_t gx = (uint32_t)((cols + kPrepThreads - 1) / kPrepThreads);
    hipLaunchKernelGGL(prepare_inputs_kernel, dim3(gx, batch), dim3(kPrepThreads), 0, stream, a);
    AEGKV_HIP_TRY(hipGetLastError());
    return AEGKV_OK;
  });
}

int aegkv_prepare_inputs(const int32_t* block_ids, const int64_t* table_offsets,
                         const int32_t* seq_lens, const int32_t* context_lens,
                         const int64_t* tokens, int32_t batch, int32_t block_size,
                         int32_t pad_width, int32_t* block_tables_out,
                         int64_t* slot_mapping_out, int64_t* positions_out,
                         int64_t* input_tokens_out, int32_t* seq_lens_out,
                         int32_t* context_lens_out, int32_t* query_start_loc_out,
                         int32_t* seq_start_loc_out, int64_t n_query_tokens,
                         aegkv_stream_t stream) {
  return guarded([&] {
    return aegkv_prepare_inputs_body(block_ids, table_offsets, seq_lens, context_lens, tokens,
                                     batch, block_size, pad_width, block_tables_out,
                                     slot_mapping_out, positions_out, input_tokens_out,
                                     seq_lens_out, context_lens_out, query_start_loc_out,
                                     seq_start_loc_out, n_query_tokens, stream);
  });
}

}  // extern "C"
