/*
 * aegkv.h — C ABI of the MI355X (gfx950) KV-cache data path for Aegaeon-style
 * multi-model serving: paged K/V append, block gather/pack/scatter, CPU<->GPU
 * swap through pinned host memory, block copy/defrag for a multi-shape pool and
 * paged GQA decode attention.
 *
 * Conventions (every entry point):
 *   - All pointers are borrowed.  Caller-visible memory (pools, staging,
 *     workspaces, outputs) is owned by the caller; the library never frees it.
 *     The library keeps one private, per-device upload ring for host id lists
 *     (pinned host + device memory, grown on demand and reused).
 *   - Work is enqueued asynchronously on the explicit `stream` (a hipStream_t;
 *     NULL = the legacy default stream).  Functions return after enqueueing.
 *   - Return value: 0 = success; < 0 = invalid argument (AEGKV_ERR_*), detected
 *     on the host before anything is enqueued; > 0 = a hipError_t returned by the
 *     HIP runtime.  aegkv_strerror() names every code.  No C++ exception crosses
 *     the ABI.
 *   - Sizes are in bytes unless the name says "elements"; element strides are in
 *     elements of the K/V dtype.
 *   - Block ids in host arrays are int64 (the reference passes
 *     std::vector<int64_t>); block tables and sequence lengths on the device are
 *     int32 and slot mappings are int64, as in the vLLM attention metadata the
 *     reference builds.
 *
 * Reference interfaces each entry point replaces are cited as path:line relative
 * to the Zyyeric/Aegaeon repository.  Entries marked EXT replace vLLM 0.5.1 /
 * vllm-flash-attn kernels that the reference reaches through the model forward
 * (aegaeon/aegaeon/worker.py:517-523).
 */
#ifndef AEGKV_H
#define AEGKV_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* aegkv_stream_t; /* hipStream_t */

/* ---- status codes ------------------------------------------------------ */
#define AEGKV_OK 0
#define AEGKV_ERR_INVALID_ARG (-1)   /* null pointer, negative count, zero size  */
#define AEGKV_ERR_OUT_OF_RANGE (-2)  /* a block id outside its pool             */
#define AEGKV_ERR_MISALIGNED (-3)    /* pointer/stride/size not 16-byte aligned  */
#define AEGKV_ERR_OVERLAP (-4)       /* src and dst block sets share a block     */
#define AEGKV_ERR_DUPLICATE (-5)     /* a destination block id appears twice     */
#define AEGKV_ERR_UNSUPPORTED (-6)   /* shape/dtype the kernels do not cover     */
#define AEGKV_ERR_WORKSPACE (-7)     /* workspace/staging smaller than required  */
#define AEGKV_ERR_RUNTIME (-8)       /* a HIP runtime query failed while sizing  */
#define AEGKV_ERR_HOST_MEMORY (-13)  /* a host-side allocation failed           */

/* dtype codes for the K/V and query elements */
#define AEGKV_DTYPE_BF16 0
#define AEGKV_DTYPE_FP16 1

/* Human-readable name of a status code (static storage, never NULL). */
const char* aegkv_strerror(int code);

/* Library ABI version: (major << 16) | minor. */
int aegkv_version(void);

/* Optional per-device set-up for the current device (creates the id upload
 * ring).  Every entry point does it lazily; calling it early keeps the first
 * real call free of set-up cost. */
int aegkv_init(void);

/* ---- a1: CPU<->GPU block swap ------------------------------------------
 * Replaces aegaeon.ops.swap (aegaeon/ops/ops.h:4-10, aegaeon/ops/swap.cu:25-59,
 * bound at aegaeon/ops/ops.cpp:4-5, called at aegaeon/aegaeon/worker.py:756-762).
 * For i in [0, n): the block `src_ids[i]` of the source pool is copied byte for
 * byte to block `dst_ids[i]` of the destination pool.  is_swap_in != 0 copies
 * host -> device (source = host_pool), otherwise device -> host.  Block i of a
 * pool starts at base + i*block_bytes (swap.cu:43-44,52-53).
 *   src_ids/dst_ids: HOST arrays of n int64 ids (like the reference's vectors).
 *   host_pool: pinned host memory (hipHostMalloc / torch pin_memory).
 *   staging/staging_bytes: optional device buffer.  With staging, scattered device
 *     blocks are packed by a gfx950 kernel into staging and moved with one DMA per
 *     run of consecutive host ids; without it (staging == NULL), one DMA per run of
 *     consecutive (src, dst) pairs.  The result is identical.
 * Unlike the reference, ids are range-checked and duplicate destination ids are
 * rejected (AEGKV_ERR_DUPLICATE) before anything is enqueued. */
int aegkv_swap_blocks(const int64_t* src_ids, const int64_t* dst_ids, int64_t n,
                      int is_swap_in, void* dev_pool, uint64_t n_dev_blocks,
                      void* host_pool, uint64_t n_host_blocks, uint64_t block_bytes,
                      void* staging, uint64_t staging_bytes, aegkv_stream_t stream);

/* ---- a1 over a pageable swap space (the reference's shared file) --------
 * The reference's swap space is one file in /dev/shm, mapped shared by every
 * worker of the node and page-locked with cudaHostRegister
 * (aegaeon/aegaeon/llm.py:297-318, worker.py:130-147).  Where that mapping
 * cannot be page-locked, this is aegkv_swap_blocks with host_pool pageable:
 * blocks cross a caller-owned pinned bounce buffer (bounce, bounce_bytes) and
 * the device staging buffer (both required), chunk by chunk; the copies
 * between the bounce buffer and host_pool run in stream order on the HIP
 * runtime's host-function thread (hipLaunchHostFunc), so an event recorded on
 * `stream` after the call completes only once host_pool holds the blocks
 * (swap-out) or the device does (swap-in).  Same ids, checks and result as
 * aegkv_swap_blocks.  host_pool, bounce and staging must stay valid until the
 * stream has passed the call; chunks are min(staging, bounce) / block_bytes
 * blocks (AEGKV_ERR_WORKSPACE when that is 0). */
int aegkv_swap_blocks_bounced(const int64_t* src_ids, const int64_t* dst_ids, int64_t n,
                              int is_swap_in, void* dev_pool, uint64_t n_dev_blocks,
                              void* host_pool, uint64_t n_host_blocks, uint64_t block_bytes,
                              void* staging, uint64_t staging_bytes, void* bounce,
                              uint64_t bounce_bytes, aegkv_stream_t stream);

/* ---- cross-process move signals ------------------------------------------
 * Stand in for the interprocess CUDA events the reference's workers exchange
 * (reduce_cuda_event / rebuild_cuda_event, aegaeon/aegaeon/utils.py:306-331;
 * recorded after a swap at worker.py:740,765, waited on with
 * cudaStreamWaitEvent at worker.py:772-815); on this runtime hipEventRecord
 * refuses events created with hipEventInterprocess.  A signal array is
 * n_words (1 .. 2^20) 64-bit timeline words of device memory (zeroed), created
 * by one process with its 64-byte hipIpcMemHandle_t written to ipc_handle,
 * opened by the others (aegkv_signals_open, which also returns n_words, read
 * from a header word that precedes *words in the allocation; _close; the
 * creator frees it with aegkv_signals_destroy).  These four allocate, open or
 * free device memory; *words is word 0 of the array in every process.
 *   aegkv_signal_set: after the stream's earlier work, *word = value
 *     (system-scope release).  One stream writes a word, with growing values.
 *   aegkv_signal_wait: the stream's later work starts only once
 *     *word >= value (a one-lane kernel polling with system-scope acquire
 *     loads).  After timeout_us of wall-clock time it stops waiting and stores
 *     1 to *timed_out (a device word or a word of pinned host memory, which
 *     the host then reads without synchronising; may be NULL), so the kernel
 *     always ends.
 *   aegkv_signal_read: *value = the word's current value, read by a copy on
 *     `stream` that the call waits for (the host-side cudaEventQuery of a
 *     rebuilt event, block_manager.py:387-398).
 * word must be 8-byte aligned. */
int aegkv_signals_create(int64_t n_words, void** words, void* ipc_handle);
int aegkv_signals_destroy(void* words);
int aegkv_signals_open(const void* ipc_handle, void** words, int64_t* n_words);
int aegkv_signals_close(void* words);
int aegkv_signal_set(void* word, uint64_t value, aegkv_stream_t stream);
int aegkv_signal_wait(const void* word, uint64_t value, uint64_t timeout_us, uint32_t* timed_out,
                      aegkv_stream_t stream);
int aegkv_signal_read(const void* word, uint64_t* value, aegkv_stream_t stream);

/* ---- block gather / scatter / copy / defrag ----------------------------
 * Device-to-device block copies driven by HOST id lists (the lists the block
 * manager builds in move_requests, aegaeon/aegaeon/block_manager.py:822-832).
 * copy:    dst_pool[dst_ids[i]] <- src_pool[src_ids[i]]; a NULL id array means the
 *          identity (i), so NULL dst_ids packs and NULL src_ids scatters.  When the
 *          two pools are the same memory, src and dst sets must be disjoint
 *          (AEGKV_ERR_OVERLAP) so that one parallel kernel is exact.
 * pack:    staging[i] <- pool[ids[i]]        (swap-out gather, block-table driven)
 * scatter: pool[ids[i]] <- staging[i]        (swap-in scatter)
 * defrag:  pool[dst_ids[i]] <- pool[src_ids[i]] with disjoint src/dst (a10: the
 *          reference has no KV compaction; the nearest precedent is
 *          aegaeon/aegaeon/loader/allocator.py:288-321).
 * block_bytes must be a multiple of 16 and pool bases 16-byte aligned. */
int aegkv_copy_blocks(const void* src_pool, uint64_t n_src_blocks, void* dst_pool,
                      uint64_t n_dst_blocks, const int64_t* src_ids,
                      const int64_t* dst_ids, int64_t n, uint64_t block_bytes,
                      aegkv_stream_t stream);
int aegkv_pack_blocks(const void* pool, uint64_t n_pool_blocks, const int64_t* ids,
                      int64_t n, void* staging, uint64_t block_bytes,
                      aegkv_stream_t stream);
int aegkv_scatter_blocks(const void* staging, const int64_t* ids, int64_t n,
                         void* pool, uint64_t n_pool_blocks, uint64_t block_bytes,
                         aegkv_stream_t stream);
int aegkv_defrag_blocks(void* pool, uint64_t n_pool_blocks, const int64_t* src_ids,
                        const int64_t* dst_ids, int64_t n, uint64_t block_bytes,
                        aegkv_stream_t stream);

/* ---- a5: slot-mapped K/V append (EXT reshape_and_cache_flash) -----------
 * For layer l in [0, n_layers) and token t in [0, n_tokens) with
 * s = slot_mapping[t] in [0, n_blocks*block_size):
 *   key_cache  + l*cache_layer_stride + (s/block_size)*cache_block_stride
 *              + (s%block_size)*row  <-  key   + l*key_layer_stride   + t*key_token_stride
 *   value_cache likewise from value, with row = n_kv_heads*head_dim elements.
 * Slots < 0 (vLLM padding) and slots >= n_blocks*block_size are skipped.  The
 * slot mapping is the reference's slot = block_table[pos/16]*16 + pos%16
 * (aegaeon/aegaeon/worker.py:628-633).  With the reference's storage layout
 * [N, L, 2, 16, Hkv, D] (worker.py:389-395) one call appends every layer:
 * cache_block_stride = L*2*16*Hkv*D, cache_layer_stride = 2*16*Hkv*D and
 * value_cache = key_cache + 16*Hkv*D.  n_layers = 1 is the per-layer vLLM call.
 * slot_mapping is a DEVICE int64 array; element size is elem_bytes (2). */
int aegkv_kv_append(const void* key, const void* value, int64_t key_token_stride,
                    int64_t value_token_stride, int64_t key_layer_stride,
                    int64_t value_layer_stride, const int64_t* slot_mapping,
                    int64_t n_tokens, void* key_cache, void* value_cache,
                    int64_t cache_block_stride, int64_t cache_layer_stride,
                    int64_t n_blocks, int32_t n_layers, int32_t block_size,
                    int32_t n_kv_heads, int32_t head_dim, int32_t elem_bytes,
                    aegkv_stream_t stream);

/* ---- gather_tokens: block-table de-page ----------------------------------
 * For sequence b, token p < seq_lens[b] and layer l < n_layers:
 *   out_key[l*out_layer_stride + (cu_seqlens[b]+p)*row] <-
 *       key_cache[l*cache_layer_stride + block_tables[b][p/bs]*cache_block_stride
 *                 + (p%bs)*row]
 * and out_value likewise.  block_tables [batch][max_blocks] int32, seq_lens [batch]
 * int32 and cu_seqlens [batch+1] int32 are DEVICE arrays; max_seq_len is a host
 * upper bound of seq_lens that sizes the grid (longer device lengths are clamped
 * to it); out_tokens is the output capacity in tokens per layer, and tokens that
 * would land past it are not written.  Pad entries of the block table
 * (id 0 in the reference, worker.py:640-646) past ceil(len/bs) are never read;
 * a block id outside [0, n_blocks) is never dereferenced (its tokens are left
 * unwritten in the output). */
int aegkv_gather_tokens(const void* key_cache, const void* value_cache,
                        int64_t cache_block_stride, int64_t cache_layer_stride,
                        int64_t n_blocks, const int32_t* block_tables, int32_t max_blocks,
                        const int32_t* seq_lens, const int32_t* cu_seqlens,
                        int32_t batch, int32_t max_seq_len, void* out_key,
                        void* out_value, int64_t out_tokens, int64_t out_layer_stride,
                        int32_t n_layers,
                        int32_t block_size, int32_t n_kv_heads, int32_t head_dim,
                        int32_t elem_bytes, aegkv_stream_t stream);

/* ---- a6: paged GQA decode attention (EXT flash_attn_with_kvcache) --------
 * out[b][h][:] = sum_{j < seq_lens[b]} softmax_j(scale * q[b][h] . K_j) V_j with
 * K_j/V_j the kv head h / (n_q_heads/n_kv_heads) of token j read through
 * block_tables[b][j/block_size] (selected at aegaeon/aegaeon/worker.py:410-418,
 * metadata at worker.py:694-711).  fp32 accumulation, dtype I/O.
 *   q/out: [batch][n_q_heads][head_dim], batch strides in elements.
 *   key_cache/value_cache: [N][block_size][n_kv_heads][head_dim] per block with
 *     block stride cache_block_stride (the reference's permuted per-layer view).
 *   block_tables [batch][max_blocks] int32, seq_lens [batch] int32: DEVICE arrays.
 *   max_seq_len: host upper bound of seq_lens; device lengths above it are
 *     clamped to it, so a wrong bound never reads or writes out of bounds.
 *   n_workgroups: workgroups that share the batch's KV blocks in equal
 *     contiguous ranges (0 = one per CU, the fast choice; 1..8192 give the
 *     same result).
 *   workspace: DEVICE scratch of
 *     aegkv_paged_decode_attention_workspace_size(...) bytes (same batch, heads,
 *     head_dim, max_seq_len, dtype, n_workgroups and device); it holds the
 *     partials of sequences that several workgroups share; its contents need
 *     no initialisation.  Calls that may run concurrently (other streams) must
 *     not share a workspace.
 * Supported: block_size 16, head_dim 64/128/256, n_q_heads/n_kv_heads <= 16
 * (AEGKV_ERR_UNSUPPORTED otherwise).  Batches above 2048 sequences run as
 * consecutive launches of 2048.  seq_lens[b] == 0 yields zeros.  A block id
 * outside [0, n_blocks) is never dereferenced: its tokens are masked out of
 * the softmax.  n_blocks must be >= 1 (AEGKV_ERR_INVALID_ARG otherwise).
 * The size query returns bytes, or a negative status (AEGKV_ERR_RUNTIME when
 * the device query behind n_workgroups = 0 failed). */
int64_t aegkv_paged_decode_attention_workspace_size(int32_t batch, int32_t n_q_heads,
                                                     int32_t n_kv_heads, int32_t head_dim,
                                                     int32_t max_seq_len, int32_t dtype,
                                                     int32_t n_workgroups);
int aegkv_paged_decode_attention(void* out, int64_t out_batch_stride, const void* q,
                                 int64_t q_batch_stride, const void* key_cache,
                                 const void* value_cache, int64_t cache_block_stride,
                                 int64_t n_blocks, const int32_t* block_tables,
                                 int32_t max_blocks, const int32_t* seq_lens,
                                 int32_t batch, int32_t max_seq_len, int32_t n_q_heads,
                                 int32_t n_kv_heads, int32_t head_dim,
                                 int32_t block_size, float scale, int32_t dtype,
                                 int32_t n_workgroups, void* workspace,
                                 uint64_t workspace_bytes, aegkv_stream_t stream);

/* No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): aegkv_paged_decode_attention with the same arguments
 * minus the workspace, which here is a 32 MiB array of device memory the
 * library holds per GPU (a file-scope __device__ array, one copy per device
 * until the process ends).  The call allocates nothing.  Calls whose
 * workspace_size exceeds 32 MiB return AEGKV_ERR_SCRATCH before anything is
 * enqueued (with one workgroup per CU, the Qwen2.5-7B shape, 28/4 heads at
 * D 128, fits every batch, and Llama-2-13B's 40/40 up to 1500 sequences; see
 * aegkv_paged_decode_attention_workspace_size).  Every call on a GPU uses
 * that GPU's one array: calls
 * that may overlap on one GPU (other streams, other threads) race and must be
 * serialised by the caller.  Results equal aegkv_paged_decode_attention's bit
 * for bit. */
#define AEGKV_ERR_SCRATCH (-11)      /* call needs more than the no-alloc scratch */
int aegkv_paged_decode_attention_noalloc(void* out, int64_t out_batch_stride, const void* q,
                                         int64_t q_batch_stride, const void* key_cache,
                                         const void* value_cache, int64_t cache_block_stride,
                                         int64_t n_blocks, const int32_t* block_tables,
                                         int32_t max_blocks, const int32_t* seq_lens,
                                         int32_t batch, int32_t max_seq_len, int32_t n_q_heads,
                                         int32_t n_kv_heads, int32_t head_dim,
                                         int32_t block_size, float scale, int32_t dtype,
                                         int32_t n_workgroups, aegkv_stream_t stream);

/* Append fused into the attention (EXT flash_attn_with_kvcache with its k=
 * and v= arguments; in vLLM 0.5.1's backend the same step is
 * reshape_and_cache_flash followed by flash_attn_with_kvcache, one launch each
 * per layer, worker.py:517-523).  key/value: the new token's rows
 * [batch][n_kv_heads][head_dim] (batch strides in elements, 16-byte aligned);
 * seq_lens[b] counts that token, which lands at position seq_lens[b] - 1:
 * token (len - 1) % 16 of block block_tables[b][(len - 1) / 16], the slot the
 * reference's slot mapping gives it (worker.py:628-633).  The output is that
 * of aegkv_kv_append into the cache followed by
 * aegkv_paged_decode_attention, bit for bit, and the cache holds the appended
 * rows afterwards; the attention reads the new rows from key/value, and the
 * cache write runs beside the merge of split sequences, so the call costs the
 * attention's two launches.  Other arguments, limits and the workspace are
 * aegkv_paged_decode_attention's; the planned form takes a plan built from
 * these seq_lens.  A last block outside [0, n_blocks) is neither read nor
 * written. */
int aegkv_paged_decode_attention_append(
    void* out, int64_t out_batch_stride, const void* q, int64_t q_batch_stride, const void* key,
    int64_t key_batch_stride, const void* value, int64_t value_batch_stride, void* key_cache,
    void* value_cache, int64_t cache_block_stride, int64_t n_blocks, const int32_t* block_tables,
    int32_t max_blocks, const int32_t* seq_lens, int32_t batch, int32_t max_seq_len,
    int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim, int32_t block_size, float scale,
    int32_t dtype, int32_t n_workgroups, void* workspace, uint64_t workspace_bytes,
    aegkv_stream_t stream);
int aegkv_paged_decode_attention_append_planned(
    void* out, int64_t out_batch_stride, const void* q, int64_t q_batch_stride, const void* key,
    int64_t key_batch_stride, const void* value, int64_t value_batch_stride, void* key_cache,
    void* value_cache, int64_t cache_block_stride, int64_t n_blocks, const void* plan,
    uint64_t plan_bytes, const int32_t* seq_lens, int32_t batch, int32_t max_seq_len,
    int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim, int32_t block_size, float scale,
    int32_t dtype, int32_t n_workgroups, void* workspace, uint64_t workspace_bytes,
    aegkv_stream_t stream);

/* Decode plan: the work split of aegkv_paged_decode_attention for one batch
 * of block tables and lengths, built once per decode step and shared by every
 * layer's call (the layers of a step attend over the same tables, as the
 * reference's attention metadata is built once per step at
 * aegaeon/aegaeon/worker.py:694-711 and used by every layer of the forward).
 * It has no counterpart in the reference's call: it moves the per-call
 * partition and block-table lookups out of each layer's critical path.
 *   aegkv_paged_decode_plan_size: DEVICE bytes of the plan (negative status
 *     when unsupported: batch above 2048, or the limits of the attention).
 *   aegkv_paged_decode_plan: writes the plan from DEVICE block_tables and
 *     seq_lens (asynchronous on `stream`).  The tables and lengths must not
 *     change while the plan is in use.
 *   aegkv_paged_decode_attention_planned: the attention of
 *     aegkv_paged_decode_attention (same arguments and workspace) with the
 *     plan in place of the block tables; batch, max_seq_len, n_kv_heads,
 *     n_workgroups and seq_lens must be the ones the plan was built with.
 *     Results are identical to the unplanned call, bit for bit. */
int64_t aegkv_paged_decode_plan_size(int32_t batch, int32_t n_kv_heads, int32_t max_seq_len,
                                     int32_t n_workgroups);
int aegkv_paged_decode_plan(const int32_t* block_tables, int32_t max_blocks,
                            const int32_t* seq_lens, int32_t batch, int32_t max_seq_len,
                            int32_t n_kv_heads, int32_t n_workgroups, void* plan,
                            uint64_t plan_bytes, aegkv_stream_t stream);
int aegkv_paged_decode_attention_planned(void* out, int64_t out_batch_stride, const void* q,
                                         int64_t q_batch_stride, const void* key_cache,
                                         const void* value_cache, int64_t cache_block_stride,
                                         int64_t n_blocks, const void* plan, uint64_t plan_bytes,
                                         const int32_t* seq_lens, int32_t batch,
                                         int32_t max_seq_len, int32_t n_q_heads,
                                         int32_t n_kv_heads, int32_t head_dim,
                                         int32_t block_size, float scale, int32_t dtype,
                                         int32_t n_workgroups, void* workspace,
                                         uint64_t workspace_bytes, aegkv_stream_t stream);

/* ---- a4: decode/prefill input preparation --------------------------------
 * Replaces the host loops of Worker._prepare_model_inputs
 * (aegaeon/aegaeon/worker.py:596-676) and make_tensor_with_pad
 * (aegaeon/aegaeon/utils.py:241-257): one upload of the HOST request lists and
 * one kernel that writes the DEVICE tensors the attention metadata holds.
 * Request b has block table block_ids[table_offsets[b] .. table_offsets[b+1]),
 * total length seq_lens[b] and first new token context_lens[b]
 * (request.py:96-102); its new tokens are tokens[q0 .. q0 + seq - ctx) with
 * q0 the sum of the previous requests' (seq - ctx).  Outputs (DEVICE):
 *   block_tables_out [batch][pad_width] int32: the table of a decode row
 *     (context_lens[b] > 0), 0-padded; prefill rows all 0 (worker.py:600-605);
 *   slot_mapping_out [n_query_tokens] int64: table[p / bs] * bs + p % bs for
 *     p in [context_len, seq_len) (worker.py:628-633);
 *   positions_out [n_query_tokens] int64: p;  input_tokens_out (may be NULL):
 *     the tokens;  seq_lens_out, context_lens_out [batch] int32;
 *   query_start_loc_out, seq_start_loc_out [batch + 1] int32 prefix sums.
 * Host checks: context_len <= seq_len, every table covers (seq_len - 1) / bs,
 * decode tables fit pad_width, n_query_tokens = sum(seq - ctx), ids >= 0. */
int aegkv_prepare_inputs(const int32_t* block_ids, const int64_t* table_offsets,
                         const int32_t* seq_lens, const int32_t* context_lens,
                         const int64_t* tokens, int32_t batch, int32_t block_size,
                         int32_t pad_width, int32_t* block_tables_out,
                         int64_t* slot_mapping_out, int64_t* positions_out,
                         int64_t* input_tokens_out, int32_t* seq_lens_out,
                         int32_t* context_lens_out, int32_t* query_start_loc_out,
                         int32_t* seq_start_loc_out, int64_t n_query_tokens,
                         aegkv_stream_t stream);

/* ---- prefill-side attention (EXT flash_attn_varlen_func) -----------------
 * The prompt run of vLLM 0.5.1's FlashAttention backend, reached from
 * aegaeon/aegaeon/worker.py:517-523 with cu_seqlens = seq_start_loc and
 * max_seqlen = max_prefill_seq_len (worker.py:652-711).  q [total, Hq, D],
 * k and v [total, Hkv, D], out [total, Hq, D] (DEVICE, 16-bit, token strides
 * in elements, the heads of a token contiguous, 16-byte aligned).  Sequence b
 * holds tokens [cu_seqlens[b], cu_seqlens[b+1]) (DEVICE int32 [batch + 1]);
 * query i of a sequence attends to keys j <= i of it (every key when causal
 * is 0), softmax(scale * q.k) in fp32 with P rounded to 16 bits before P.V.
 * Lengths are clamped to max_seqlen (the host bound that sizes the grid) and
 * tokens to [0, total_tokens).  head_dim 64 or 128, Hq a multiple of Hkv. */
int aegkv_varlen_prefill_attention(void* out, int64_t out_token_stride, const void* q,
                                   int64_t q_token_stride, const void* k, int64_t k_token_stride,
                                   const void* v, int64_t v_token_stride,
                                   const int32_t* cu_seqlens, int32_t batch, int32_t max_seqlen,
                                   int64_t total_tokens, int32_t n_q_heads, int32_t n_kv_heads,
                                   int32_t head_dim, float scale, int32_t causal, int32_t dtype,
                                   aegkv_stream_t stream);

/* ---- a8: node-wide block manager (host bookkeeping) ----------------------
 * Replaces the allocation and move bookkeeping of BlockManager
 * (aegaeon/aegaeon/block_manager.py:180-874).  Pure host code, no HIP calls;
 * not thread-safe (one caller at a time, as the reference's event loop).
 * Same id order as the reference, so the swap lists it produces are the
 * reference's:
 *   - per GPU engine a FIFO free list: allocations take from the head, frees
 *     and reclaimed move sources go to the tail (:515-526,703,250-258);
 *   - the CPU pool is num_slabs slabs of slab_bytes; a slab holds blocks of one
 *     shape while any is used; per-shape free deques, a stack of free slabs and
 *     per-slab usage counts (:186-199,528-580), slab reclaim (:474-496);
 *     block ids of a shape are byte offsets / block_bytes (:242-245).
 * A shape is a caller-chosen id (>= 0) with its block bytes.  Locations: an
 * engine id >= 0 or AEGKV_BM_CPU.
 *
 * Reclaim.  When an allocation runs short while moves out of that location
 * (CPU: of that shape) are pending, the reference awaits them and reclaims
 * their source blocks (_get_free_blocks -> _reclaim_*_move_blocks,
 * :498-582, :360-472), polling their events from its event loop.  Here the
 * call suspends instead (the default): it returns AEGKV_RECLAIM_PENDING,
 * keeping what it has done (the requests a move has already assigned keep
 * their new tables, as in the reference); aegkv_bm_pending names the call,
 * the location/shape and the last pending serial; the caller awaits those
 * moves, reclaims each with aegkv_bm_complete_move (CPU: then
 * aegkv_bm_reclaim_slabs once), and calls aegkv_bm_resume, which continues at
 * the allocation that ran short (re-checked once: AEGKV_ERR_NO_SPACE, the
 * reference's ResourceWarning, if still short) or aegkv_bm_cancel.  Other
 * calls may run in between, as other coroutines do in the reference; the
 * requests of a suspended call are busy (allocate/move on them:
 * AEGKV_ERR_IN_USE), a free of one drops it from the call.  A caller that
 * can block may instead install a wait callback (aegkv_bm_set_wait): it is
 * called at the same point with the last pending serial, returns 0 once every
 * move up to it has finished copying, and the call reclaims them and goes on
 * (non-zero: AEGKV_ERR_NO_SPACE). */
#define AEGKV_ERR_NO_SPACE (-9)      /* not enough free blocks after reclaim     */
#define AEGKV_ERR_IN_USE (-10)       /* request lives elsewhere / space occupied  */
#define AEGKV_RECLAIM_PENDING (-12)  /* suspended until pending moves are reclaimed */
#define AEGKV_BM_CPU (-1)            /* BLOCK_LOCATION_CPU (block_manager.py:96)  */

typedef struct aegkv_block_manager aegkv_block_manager;
typedef int (*aegkv_bm_wait_fn)(void* ctx, int32_t location, int32_t shape, int64_t serial);

/* BlockManager.__init__ (:180-246): num_slabs CPU slabs of slab_bytes. */
int aegkv_bm_create(int64_t cpu_num_slabs, int64_t cpu_slab_bytes, aegkv_block_manager** out);
void aegkv_bm_destroy(aegkv_block_manager* bm);
int aegkv_bm_set_wait(aegkv_block_manager* bm, aegkv_bm_wait_fn fn, void* ctx);
/* Shape id -> bytes per block (_get_block_size_bytes, :239-240); fixed once set. */
int aegkv_bm_define_shape(aegkv_block_manager* bm, int32_t shape, uint64_t block_bytes);
/* register_gpu_space (:300-348): fresh free list [0, num_max_blocks); CPU
 * moves into the replaced space are reclaimed.  AEGKV_ERR_IN_USE while a
 * request still lives in it.  Only this engine's pending moves are dropped
 * (the reference drops every engine's, stranding their source blocks). */
int aegkv_bm_register_gpu_space(aegkv_block_manager* bm, int32_t engine, int64_t num_max_blocks,
                                int32_t shape);
/* allocate_blocks_batched (:651-694): request i ends with num_blocks_needed[i]
 * blocks on `engine`; one batched allocation handed out in request order. */
int aegkv_bm_allocate(aegkv_block_manager* bm, int32_t engine, const int64_t* request_ids,
                      const int64_t* num_blocks_needed, int64_t n);
/* free_blocks (:696-711). */
int aegkv_bm_free(aegkv_block_manager* bm, int64_t request_id);
/* move_requests (:778-874), CPU<->GPU: requests already at `target` are
 * skipped, the others share location and shape.  Outputs the move's serial
 * (-1: nothing moved), block count, direction and GPU engine; the id lists
 * and the moved requests (first occurrences, in order; may be NULL) are read
 * with aegkv_bm_move_ids before the next move.  A failed call changes
 * no table (the reference leaves the earlier requests of the batch moved). */
int aegkv_bm_move(aegkv_block_manager* bm, const int64_t* request_ids, int64_t n,
                  int32_t target, int64_t* serial, int64_t* n_blocks, int32_t* is_swap_in,
                  int32_t* engine);
int aegkv_bm_move_ids(const aegkv_block_manager* bm, int64_t* src_ids, int64_t* dst_ids,
                      int64_t cap, int64_t* moved_request_ids, int64_t request_cap,
                      int64_t* n_moved);
/* The call suspended last (AEGKV_RECLAIM_PENDING): its handle, and the
 * location/shape and serial up to which the pending moves are awaited. */
int aegkv_bm_pending(const aegkv_block_manager* bm, int64_t* op, int32_t* location,
                     int32_t* shape, int64_t* serial);
/* Continue a suspended allocate/move once those moves are reclaimed; outputs
 * as aegkv_bm_move (an allocation: serial -1, engine = its engine). */
int aegkv_bm_resume(aegkv_block_manager* bm, int64_t op, int64_t* serial, int64_t* n_blocks,
                    int32_t* is_swap_in, int32_t* engine);
/* Abandon a suspended call: a move is undone, an allocation took nothing. */
int aegkv_bm_cancel(aegkv_block_manager* bm, int64_t op);
/* One pending move out of `location` (CPU: of `shape`) whose copy finished:
 * its source blocks are reclaimed (_reclaim_blocks' per-event callback,
 * :384-406); no longer pending is not an error. */
int aegkv_bm_complete_move(aegkv_block_manager* bm, int32_t location, int32_t shape,
                           int64_t serial);
/* _reclaim_cpu_slabs (:474-496): empty slabs return to the free-slab stack. */
int aegkv_bm_reclaim_slabs(aegkv_block_manager* bm);
/* Reclaim the moves out of `location` (CPU: of `shape`) up to up_to_serial,
 * whose copies the caller has seen finish (_reclaim_blocks, :360-408). */
int aegkv_bm_complete_moves(aegkv_block_manager* bm, int32_t location, int32_t shape,
                            int64_t up_to_serial);
/* get_block_table (:718-721); blocks may be NULL to query the length. */
int aegkv_bm_table(const aegkv_block_manager* bm, int64_t request_id, int32_t* location,
                   int32_t* shape, int64_t* n_blocks, int64_t* blocks, int64_t cap);
/* Tables of request_ids flattened for aegkv_prepare_inputs: offsets[n + 1],
 * ids (int32, may be NULL to size). */
int aegkv_bm_flat_tables(const aegkv_block_manager* bm, const int64_t* request_ids, int64_t n,
                         int64_t* offsets, int32_t* ids, int64_t cap);
/* log_block_usage counters (:730-768): free/moving blocks of an engine, or of
 * a CPU shape with its slab count and used blocks. */
int aegkv_bm_stats(const aegkv_block_manager* bm, int32_t location, int32_t shape,
                   int64_t* n_free, int64_t* n_moving, int64_t* n_slabs, int64_t* n_used);
/* The free list of an engine or a CPU shape, in allocation order. */
int aegkv_bm_free_list(const aegkv_block_manager* bm, int32_t location, int32_t shape,
                       int64_t* out, int64_t cap, int64_t* n);

#ifdef __cplusplus
}
#endif

#endif /* AEGKV_H */
