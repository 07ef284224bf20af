// Paged GQA decode attention for gfx950 (replaces vllm-flash-attn's
// flash_attn_with_kvcache on the decode path, selected at
// aegaeon/aegaeon/worker.py:410-418 and run inside the forward at :517-523).
//
// Work decomposition (persistent and balanced).  The batch's KV blocks are
// laid end to end per group of kHeadsPerGroup kv heads, each sequence
// preceded by kSegmentCost charge positions for the cost of starting it:
// position P = grp * W + cum[b] + kSegmentCost + j for block j of sequence b,
// W = sum_b (ceil(len_b / 16) + kSegmentCost).  One workgroup per CU takes an
// equal contiguous range of positions, so every CU does the same work in a
// single round, and consecutive ranges land on different XCDs (workgroups are
// dealt to the XCDs round-robin).  Each workgroup computes the prefix sums of
// the batch itself (into LDS) and walks its range; a range may cut sequences,
// whose pieces write fp32 partials (unnormalised O, running max in log2
// units, sum).  A workgroup's range can end at most one cut sequence (a cut
// sequence ending inside a range began before it, i.e. at the range's start),
// so each workgroup leaves a 16-byte descriptor of that sequence (or none;
// a plan instead holds one per sequence when sequences are fewer than
// workgroups), and a second kernel, one workgroup per descriptor and kv head,
// merges its pieces with log-sum-exp weights.  A sequence held by one workgroup is
// normalised and written directly.  (Merging in the main kernel by the last
// piece to arrive measured slower every way it was built: with device-scope
// release fences, which write back the XCD's L2, 2x; with write-through
// agent-scope partials and an arrival counter per cut sequence, 13-23%.  The
// write-through partial stores alone cost ~7 us per Qwen2.5-7B layer against
// ordinary ones, and the last arrival's merge of a long sequence's pieces on
// one CU ~10 us more, against ~3.6 us for this second launch.)
//
// Inside a workgroup, wave w handles kv head grp * 4 + w, and all
// G = Hq / Hkv query heads of that kv head are processed together, so each K/V
// byte is read from HBM exactly once per decode step.  A wave streams the
// blocks of its whole range through one register pipeline, across sequence
// boundaries, and keeps the pieces it finishes in LDS until the stream ends
// (attend_items); one piece per sequence start and a pipeline drain per
// piece measured ~3.8 us each, against ~1 us for a switch in the stream.
//
// Per 16-token block (block_size 16), with lane l = 16*g + j:
//   S^T[16 tok x 16 heads] = K[16 x D] . Q^T[D x 16]  -> D/32 MFMA 16x16x32
//     (lane: K row j, dims 32*ks + 8*g .. +7, one dwordx4 per k-step);
//   online softmax in fp32 (exp2 domain): lane holds head j, tokens 4g+r;
//   O^T[D x 16 heads] += V^T[D x 16 tok] . P^T[16 tok x 16 heads] on the same
//     16x16x32 MFMA: P is split into a 16-bit high part and the 16-bit rounding
//     of its remainder, stacked along K (k = 8g+e <-> token 4g+(e&3), half
//     e>>2), and V^T is repeated for both halves.  V is exact in 16 bits, so
//     the products keep ~16 bits of P: 8 MFMAs per block instead of 32 fp32
//     16x16x4 ones, at a P error (< 2^-14 relative) far below the output's
//     16-bit rounding.
//     Lane (j, g) loads V rows 4g..4g+3, dims [D/16*j, +D/16); tile t of the
//     output holds dims D/16*i + t for A-row i, so output lane (j, g) owns head
//     j, dims D/16*(4g+r) + t.
// The block ids of a range are loaded 64 at a time, one per lane, and read
// with readlane; a rolling register pipeline keeps pipeline_depth - 1 blocks of
// K/V in flight while one is computed.
#include <algorithm>
#include <cmath>
#include <map>
#include <mutex>
#include <utility>

#include "aegkv_internal.h"

namespace aegkv {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

constexpr int kBlockSize = 16;
constexpr int kHeadsPerGroup = 4;   // waves (kv heads) per workgroup
constexpr int kMaxBatch = 2048;     // sequences per launch (LDS prefix sums); larger
                                    // batches are launched in chunks
constexpr int kMaxWorkgroups = 8192;  // bound of n_workgroups
constexpr int kMaxStage = 4;          // finished pieces a wave stages in LDS
constexpr int kNewStage = 8;          // an appending call: sequences' new rows a wave stages in LDS
// A raw buffer offset past every range this file builds (each below 2^31
// bytes): the access returns zeros and reads no memory.
constexpr uint32_t kPastRange = 0xFFFFFFF0u;
constexpr int kStageBudget = 64 * 1024;  // dynamic LDS of a workgroup, scan arrays included
constexpr int kScanPerThread = kMaxBatch / (64 * kHeadsPerGroup);
// Cost of switching the block stream to a new sequence (its piece staged,
// its query swapped in) in units of one block: the partition balances blocks
// plus this charge per sequence, so a workgroup that holds several short
// sequences gets correspondingly fewer blocks (measured ~1 block on the
// Qwen2.5-7B batch; 2 and 0 were slower).
constexpr int kSegmentCost = 1;

// Cost units of a sequence of `len` tokens: its blocks plus the start charge.
__device__ __forceinline__ int cost_units(int len) {
  const int nblk = (len + kBlockSize - 1) / kBlockSize;
  return nblk > 0 ? nblk + kSegmentCost : 0;
}
// K/V register buffers per wave: three blocks of K and V fit the register
// budget of two waves per SIMD up to D = 128; D = 256 keeps two and runs one
// wave per SIMD.
template <int D>
constexpr int pipeline_depth() { return D >= 256 ? 2 : 3; }
constexpr float kRescaleSlack = 8.f;  // log2 headroom of the lazy softmax rescale

template <int DT>
struct Elem;

template <>
struct Elem<AEGKV_DTYPE_BF16> {
  static __device__ __forceinline__ f32x4 mfma(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  // p = hi + lo with hi the top 16 bits of p (truncation, so p - hi is exact
  // in fp32) and lo the top 16 bits of the remainder; returns the two halves.
  static __device__ __forceinline__ void split(float p, uint32_t& hi, uint32_t& lo) {
    const uint32_t u = __float_as_uint(p);
    hi = u >> 16;
    lo = __float_as_uint(p - __uint_as_float(u & 0xffff0000u)) >> 16;
  }
  static __device__ __forceinline__ uint32_t bits(float x) {
    // round to nearest even; NaN stays a quiet NaN
    uint32_t u = __float_as_uint(x);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
    u += 0x7fffu + ((u >> 16) & 1u);
    return u >> 16;
  }
};

template <>
struct Elem<AEGKV_DTYPE_FP16> {
  static __device__ __forceinline__ f32x4 mfma(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ void split(float p, uint32_t& hi, uint32_t& lo) {
    const _Float16 h = (_Float16)p;
    hi = __builtin_bit_cast(unsigned short, h);
    lo = __builtin_bit_cast(unsigned short, (_Float16)(p - (float)h));
  }
  static __device__ __forceinline__ uint32_t bits(float x) {
    return (uint32_t)__builtin_bit_cast(unsigned short, (_Float16)x);
  }
};

struct AttnArgs {
  const uint16_t* q;
  int64_t q_bstride;  // elements
  const uint16_t* kc;
  const uint16_t* vc;
  int64_t blk_stride;  // elements
  int64_t n_blocks;
  const int32_t* block_tables;
  int32_t max_blocks;
  const int32_t* seq_lens;
  int32_t batch;
  int32_t n_q_heads;
  int32_t n_kv_heads;
  int32_t head_dim;
  int32_t group;     // n_q_heads / n_kv_heads
  int32_t hpg;       // query heads per workgroup: kHeadsPerGroup * group
  int32_t n_groups;  // ceil(n_kv_heads / kHeadsPerGroup)
  int32_t n_wg;      // workgroups of the main kernel
  float scale_log2;  // softmax scale * log2(e)
  int32_t max_seq_len;  // host bound; longer device lengths are clamped to it
  uint16_t* out;
  int64_t out_bstride;  // elements
  int4* desc;           // [n_wg] cut sequence ending in each workgroup: (b, grp, w0, npieces)
  float* part_o;        // [slots][hpg][D]
  float2* part_ml;      // [slots][hpg] (running max in log2 units, sum)
  uint32_t ml_bytes, o_bytes;  // sizes of the two partial regions (< 2^31)
  int32_t stage_slots;  // finished pieces a wave holds in LDS (0: stored at once)
  int32_t stage_off;    // byte offset of the staging area in dynamic LDS
  // decode plan (planned launches only): workgroup records, first block ids
  // of each workgroup's range, block ids in item order
  const int32_t* plan_wg;
  const int32_t* plan_first;
  const int32_t* plan_ids;
  const int32_t* plan_tags;  // per item: new-row tag (see the plan layout)
  const int32_t* plan_last;  // per sequence: the block of its position seq_lens[b] - 1
  // append fused into the call (knew == nullptr: none): the new token's K and
  // V rows of sequence b, kv head h at knew/vnew + b * stride + h * D; the
  // token is the last of seq_lens[b].  The main kernel reads it from there
  // (when the length is within max_seq_len: a longer sequence is attended over
  // its first max_seq_len cached tokens, without the new row), and after its
  // merges the combine kernel's threads copy it into the cache at its own
  // position seq_lens[b] - 1, as the separate append would.
  const uint16_t* knew;
  const uint16_t* vnew;
  int64_t knew_bstride, vnew_bstride;  // elements
  uint32_t knew_span, vnew_span;       // bytes from knew / vnew to the last row's end (< 2^31)
  int32_t newrow_off;                  // byte offset of the staged new rows in dynamic LDS
  int32_t n_desc;                      // merge descriptors (the combine grid's width)
};

// A plan indexes the merge descriptors by (kv-head group, sequence) when there
// are fewer of those than workgroups, so that the combine grid has one
// workgroup per sequence instead of one per main-kernel workgroup (the
// Yi-1.5-9B batch: 64 against 256, of which 61 cut); otherwise, and without a
// plan, by the workgroup holding the sequence's last piece.
inline bool desc_per_sequence(int64_t batch, int64_t n_groups, int64_t n_wg) {
  return batch * n_groups < n_wg;
}

// Decode plan, in one device buffer: per main-kernel workgroup a record of 8
// int32 (first kv-head group or -1 for an idle workgroup, last group, first
// item and its sequence, end item in the last group, the batch's first
// non-empty sequence), the merge descriptors, the block ids and new-row tags
// of the first 64 items of each workgroup's range, the id of the block that
// holds each sequence's position seq_lens[b] - 1 (-1 when empty or past its
// table), the block ids of all items in item order (item i = block
// i - bcum[b] of the sequence b holding it), and their new-row tags (b * 16 +
// the token offset of the last token in a sequence's last block, -1 for other
// blocks and for sequences longer than max_seq_len), which an appending call
// at D = 256 uses (at D <= 128 it finds each sequence's last block from the
// stream's own position instead).
struct PlanLayout {
  int64_t wg, desc, first, last, ids, tags, total;
};
inline PlanLayout plan_layout(int64_t batch, int64_t n_wg, int64_t nblk_max) {
  auto up = [](int64_t x) { return (x + 255) / 256 * 256; };
  PlanLayout l;
  l.wg = 0;
  l.desc = up(n_wg * 32);
  l.first = l.desc + up(n_wg * 16);
  l.last = l.first + up(n_wg * 128 * 4);
  l.ids = l.last + up(batch * 4);
  l.tags = l.ids + up(batch * nblk_max * 4);
  l.total = l.tags + up(batch * nblk_max * 4);
  return l;
}
constexpr int kPlanRecord = 8;  // int32 per workgroup record

// Workspace layout of one launch: the workgroups' descriptors, then the
// partials of n_wg + n_groups * batch slots (a workgroup writes at most one
// slot per sequence piece it holds; slot = workgroup + grp * batch + b is
// unique).  Every byte the combine reads is written by the same launch.
struct WorkspaceLayout {
  int64_t desc_bytes, ml_bytes, o_bytes, total;
};
inline WorkspaceLayout workspace_layout(int64_t batch, int64_t hpg, int64_t head_dim,
                                        int64_t n_wg, int64_t n_groups) {
  auto up = [](int64_t x) { return (x + 255) / 256 * 256; };
  const int64_t slots = n_wg + n_groups * batch;
  WorkspaceLayout w;
  w.desc_bytes = up(n_wg * 16);
  w.ml_bytes = up(slots * hpg * 8);
  w.o_bytes = up(slots * hpg * head_dim * 4);
  w.total = w.desc_bytes + w.ml_bytes + w.o_bytes;
  return w;
}

// K/V are streamed once per decode step: non-temporal loads keep them from
// displacing reusable lines in the caches (measured ~9% more read bandwidth
// than ordinary loads on scattered 16-32 KiB regions).  A block is read
// through a raw buffer range over its K (or V) rows, so a load that must
// issue but has nothing to read (a pipeline refill past the end of a range,
// an unreadable block id) gets an empty range: it returns zeros and moves no
// bytes, and the loop still issues every load unconditionally.
template <int NW>
__device__ __forceinline__ void load_words(__amdgpu_buffer_rsrc_t r, uint32_t off, uint32_t* w) {
  if constexpr (NW == 2) {
    const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, kNt);
    w[0] = v.x; w[1] = v.y;
  } else {
#pragma unroll
    for (int i = 0; i < NW / 4; ++i) {
      const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, off + 16 * i, 0, kNt);
      w[4 * i + 0] = v.x; w[4 * i + 1] = v.y; w[4 * i + 2] = v.z; w[4 * i + 3] = v.w;
    }
  }
}

// K and V registers of one block for one lane.
template <int D>
struct KVRegs {
  static constexpr int KS = D / 32;   // QK k-steps
  static constexpr int VW = D / 32;   // 32-bit words per lane per V row (D/16 dims)
  u32x4 k[KS];
  uint32_t v[4][VW];
};

// One block: kr / vr are the block's K and V rows (16 x n_kv_heads * D
// elements each, or empty), koff / voff this lane's byte offsets in them
// (K: token j, dims 8g + 32 ks; V: tokens 4g + c, dims D/16 * j), row_b the
// bytes of one token row.
template <int D>
__device__ __forceinline__ void load_block(KVRegs<D>& r, __amdgpu_buffer_rsrc_t kr,
                                           __amdgpu_buffer_rsrc_t vr, uint32_t koff,
                                           uint32_t voff, uint32_t row_b) {
#pragma unroll
  for (int ks = 0; ks < KVRegs<D>::KS; ++ks)
    r.k[ks] = __builtin_amdgcn_raw_buffer_load_b128(kr, koff + 64 * ks, 0, kNt);
#pragma unroll
  for (int c = 0; c < 4; ++c) load_words<KVRegs<D>::VW>(vr, voff + c * row_b, r.v[c]);
}

// load_block for a sequence's last block when the call appends: the lanes
// that hold the new token's row (token noff of the block) read it from the
// append's input rows kn (K, this lane's dims) and vn (V) instead of the
// cache, whose slot is written only after the attention.  A per-lane choice
// of address needs global loads (a buffer range is uniform over the wave);
// two buffer loads per word with an OR of their results doubled the
// registers in flight and spilled.  kh / vh are this lane's K / V addresses
// in block 0 and off the block's offset; a pipeline refill past the range
// re-reads the range's last block.
template <int NW>
__device__ __forceinline__ void load_words_global(const uint16_t* p, uint32_t* w) {
  if constexpr (NW == 2) {
    const u32x2 v = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(p));
    w[0] = v.x; w[1] = v.y;
  } else {
#pragma unroll
    for (int i = 0; i < NW / 4; ++i) {
      const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p + 8 * i));
      w[4 * i + 0] = v.x; w[4 * i + 1] = v.y; w[4 * i + 2] = v.z; w[4 * i + 3] = v.w;
    }
  }
}
template <int D>
__device__ __forceinline__ void load_block_new(KVRegs<D>& r, const uint16_t* kh,
                                               const uint16_t* vh, int64_t off, int64_t row,
                                               int noff, const uint16_t* kn, const uint16_t* vn) {
  const int lane = threadIdx.x & 63;
  const int j = lane & 15, g = lane >> 4;
  const uint16_t* kp = j == noff ? kn : kh + off;
#pragma unroll
  for (int ks = 0; ks < KVRegs<D>::KS; ++ks)
    r.k[ks] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(kp + 32 * ks));
#pragma unroll
  for (int c = 0; c < 4; ++c)
    load_words_global<KVRegs<D>::VW>(4 * g + c == noff ? vn : vh + off + c * row, r.v[c]);
}

// Softmax update and P.V for one block whose first token is `tok0`; `len` is
// the number of tokens of the sequence (0 masks the whole block: an unreadable
// block id).
template <int DT, int D>
__device__ __forceinline__ void compute_block(KVRegs<D>& r, const u32x4* qv, f32x4* acc,
                                              float& m, float& lsum, int tok0, int len, int g,
                                              float scale_log2) {
  using E = Elem<DT>;
  constexpr int DPL = D / 16;
  f32x4 sc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int ks = 0; ks < KVRegs<D>::KS; ++ks) sc = E::mfma(r.k[ks], qv[ks], sc);
  const int tb = tok0 + 4 * g;  // token of sc[0] in this lane
  float x[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) x[i] = (tb + i < len) ? sc[i] * scale_log2 : -INFINITY;
  float bm = fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3]));
  bm = fmaxf(bm, __shfl_xor(bm, 16));
  bm = fmaxf(bm, __shfl_xor(bm, 32));
  // Lazy rescaling: exponents are taken against a reference max m that moves
  // only when a block's max exceeds it by more than kRescaleSlack (log2 units),
  // so p <= 2^kRescaleSlack (exact in bf16/fp16, harmless in fp32) and the
  // accumulators are rescaled in a rare branch instead of on every block.
  if (__builtin_amdgcn_ballot_w64(bm > m + kRescaleSlack)) {
    const float mn = fmaxf(m, bm);
    const float alpha = __builtin_amdgcn_exp2f(m - mn);  // 0 while m = -inf
    lsum *= alpha;
#pragma unroll
    for (int t = 0; t < DPL; ++t) acc[t] *= alpha;
    m = mn;
  }
  const float ms = m == -INFINITY ? 0.f : m;  // -inf only while every token is masked
  float p[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) p[i] = __builtin_amdgcn_exp2f(x[i] - ms);
  lsum += (p[0] + p[1]) + (p[2] + p[3]);

  // B operand: [hi(p0..p3), lo(p0..p3)] as 16-bit values
  uint32_t hi[4], lo[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) E::split(p[i], hi[i], lo[i]);
  const u32x4 bop = {hi[0] | (hi[1] << 16), hi[2] | (hi[3] << 16), lo[0] | (lo[1] << 16),
                     lo[2] | (lo[3] << 16)};

  // rows past the sequence end hold stale bytes (maybe NaN): zero them in
  // place (the block is not read again)
  if (tok0 + kBlockSize > len) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const bool keep = tb + c < len;
#pragma unroll
      for (int w = 0; w < KVRegs<D>::VW; ++w) r.v[c][w] = keep ? r.v[c][w] : 0u;
    }
  }
  const auto& v = r.v;
#pragma unroll
  for (int t = 0; t < DPL; ++t) {
    const int w = t >> 1;
    uint32_t a0, a1;
    if (t & 1) {
      a0 = (v[0][w] >> 16) | (v[1][w] & 0xffff0000u);
      a1 = (v[2][w] >> 16) | (v[3][w] & 0xffff0000u);
    } else {
      a0 = (v[0][w] & 0xffffu) | (v[1][w] << 16);
      a1 = (v[2][w] & 0xffffu) | (v[3][w] << 16);
    }
    acc[t] = E::mfma(u32x4{a0, a1, a0, a1}, bop, acc[t]);
  }
}

// Calls f(integral_constant<int, k>) for k = 0, 1, ... until one returns true
// (fully unrolled: k is a compile-time constant in every call).
template <typename F, int... Ks>
__device__ __forceinline__ bool unrolled_steps_impl(F&& f, std::integer_sequence<int, Ks...>) {
  return (f(std::integral_constant<int, Ks>{}) || ...);
}
template <int N, typename F>
__device__ __forceinline__ bool unrolled_steps(F&& f) {
  return unrolled_steps_impl(f, std::make_integer_sequence<int, N>{});
}

// Largest b in [0, batch) with cum[b] <= i, for 0 <= i < cum[batch] and cum
// non-decreasing.  Over block counts this is the (non-empty) sequence that
// holds block item i; over positions, the sequence that holds position i.
__device__ __forceinline__ int seq_at(const int32_t* cum, int batch, int i) {
  int lo = 0, hi = batch;  // cum[lo] <= i < cum[hi]
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (cum[mid] <= i) lo = mid; else hi = mid;
  }
  return lo;
}

__device__ __forceinline__ int uni(int x) { return __builtin_amdgcn_readfirstlane(x); }

// Finished pieces.  Lane (j, g) holds query head j, dims
// [4*DPL*g, 4*DPL*g + 4*DPL) with dim offset DPL*r + t <- acc[t][r].  A
// whole sequence is written normalised to `out`; a piece of a cut sequence as
// its fp32 partial and (max, sum) for the merge.  Inside the block stream a
// piece goes to an LDS record instead (lane record: D bytes of partial or
// D/2 of output, then (max, sum)); global stores there would join the K/V
// loads in the vector-memory counter and every wait after them would wait for
// the stores as well.  The records are written out when the wave's stream
// ends, or when its stage_slots records are full.
template <int D>
constexpr int stage_record_bytes() { return D + 16; }
// D = 256 keeps direct stores: its registers leave no room for the records.
template <int D>
constexpr bool stages_pieces() { return D <= 128; }

template <int DT, int D>
__device__ __forceinline__ void store_piece(const AttnArgs& a, const f32x4* acc, float m,
                                            float lt, int b, int hq, bool complete, int64_t slot,
                                            int hl0) {
  using E = Elem<DT>;
  constexpr int DPL = D / 16;
  constexpr int VW = D / 32;
  const int lane = threadIdx.x & 63;
  const int j = lane & 15, g = lane >> 4;
  const int d0 = 4 * DPL * g;
  if (complete) {
    const float inv = lt > 0.f ? 1.f / lt : 0.f;
    uint16_t* op = a.out + (int64_t)b * a.out_bstride + (int64_t)hq * D + d0;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      uint32_t w[VW];
#pragma unroll
      for (int t = 0; t < DPL; t += 2)
        w[t >> 1] = E::bits(acc[t][r] * inv) | (E::bits(acc[t + 1][r] * inv) << 16);
      if constexpr (VW == 2) {
        *reinterpret_cast<u32x2*>(op + DPL * r) = u32x2{w[0], w[1]};
      } else {
#pragma unroll
        for (int i = 0; i < VW / 4; ++i)
          *reinterpret_cast<u32x4*>(op + DPL * r + 8 * i) =
              u32x4{w[4 * i], w[4 * i + 1], w[4 * i + 2], w[4 * i + 3]};
      }
    }
  } else {
    const int64_t pidx = slot * a.hpg + hl0 + j;
    float* po = a.part_o + pidx * D + d0;
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int t = 0; t < DPL; t += 4)
        *reinterpret_cast<f32x4*>(po + DPL * r + t) =
            f32x4{acc[t][r], acc[t + 1][r], acc[t + 2][r], acc[t + 3][r]};
    if (g == 0) a.part_ml[pidx] = make_float2(m, lt);
  }
}

// LDS record <-> accumulators (the record keeps the fp32 state; the output
// is normalised and rounded when it is written out, as store_piece does)
template <int D>
__device__ __forceinline__ void put_record(uint8_t* rec, const f32x4* acc, float m, float lt) {
  constexpr int DPL = D / 16;
#pragma unroll
  for (int t = 0; t < DPL; ++t) *reinterpret_cast<f32x4*>(rec + 16 * t) = acc[t];
  *reinterpret_cast<float2*>(rec + D) = make_float2(m, lt);
}
template <int D>
__device__ __forceinline__ void get_record(const uint8_t* rec, f32x4* acc, float& m, float& lt) {
  constexpr int DPL = D / 16;
#pragma unroll
  for (int t = 0; t < DPL; ++t) acc[t] = *reinterpret_cast<const f32x4*>(rec + 16 * t);
  const float2 ml = *reinterpret_cast<const float2*>(rec + D);
  m = ml.x;
  lt = ml.y;
}

// One wave's share of a workgroup's range within kv-head group `grp`: block
// items [i0, i1) of the group, item i being block i - bcum[b] of the sequence
// b with bcum[b] <= i < bcum[b + 1], for kv head grp * 4 + wave.
//
// The items are streamed through one rolling register pipeline of NBUF
// blocks whatever the sequence boundaries: buffer k holds item i0 + it + k;
// as soon as it is computed the buffer is refilled with the item NBUF
// further on, so NBUF - 1 blocks stay in flight across the end of one
// sequence and the start of the next.  A sequence piece that ends costs its
// output stores and the switch to the next sequence, whose query was loaded
// when the previous switch happened.  Inside the loop every K/V load is
// issued unconditionally: without an append, a refill past the range and an
// unreadable block id load through an empty buffer range, which reads no
// memory (re-reading
// the range's last block instead cost 4% more HBM traffic on the
// Qwen2.5-7B batch and 12% on the Yi-1.5-9B one, as the non-temporal lines
// were gone from L2).  Block ids come 64 items at a time, one per lane, with
// the next 64 loaded a chunk ahead; an unreadable block is masked.
//
// With a plan (PLANNED) the ids come from its item-order list, and `id_first`
// holds the ids of items [i0, i0 + 64) when the caller loaded them (the
// range's first pass), so no table lookup stands between the start and the
// first K/V loads.
template <int DT, int D, int NBUF, bool PLANNED, bool FUSED>
__device__ __forceinline__ void attend_items(const AttnArgs& a, const int32_t* s_bcum,
                                             const int32_t* s_len, uint8_t* stage, int4* meta,
                                             int grp, int b0, int i0, int i1, bool have_first,
                                             int id_first, int tag_first,
                                             const uint32_t* s_over = nullptr,
                                             uint8_t* nstage = nullptr, int32_t* nseq = nullptr) {
  constexpr int KS = D / 32;
  constexpr int DPL = D / 16;
  constexpr bool kNewInLds = FUSED && D <= 128;  // an appending call's rows staged in LDS
  constexpr bool kTags = FUSED && !kNewInLds;     // per-item new-row tags (D = 256)
  const int lane = threadIdx.x & 63, wave = uni(threadIdx.x >> 6);
  const int h = grp * kHeadsPerGroup + wave;
  if (h >= a.n_kv_heads) return;  // wave past the last kv head (uniform)
  const int j = lane & 15, g = lane >> 4;
  const bool head_ok = j < a.group;
  const int hq = h * a.group + j;
  const int hl0 = wave * a.group;
  const int64_t row = (int64_t)a.n_kv_heads * D;
  const uint32_t row_b = (uint32_t)(row * 2);
  const uint32_t blk_b = kBlockSize * row_b;  // a block's K (or V) rows
  const uint32_t koff = (uint32_t)(((int64_t)j * row + (int64_t)h * D + 8 * g) * 2);
  const uint32_t voff = (uint32_t)(((int64_t)(4 * g) * row + (int64_t)h * D + DPL * j) * 2);

  // the sequence being computed: bc, whose block 0 is item `first`, with
  // items up to cend in range
  int bc = b0;
  int first = uni(s_bcum[bc]);
  int cend = min(uni(s_bcum[bc + 1]), i1);
  int len = uni(s_len[bc]);
  bool complete = first >= i0 && cend == uni(s_bcum[bc + 1]);

  // block id of item i (clamped into the range), one lane per item; bh is a
  // sequence at or before the item's (the item's own or the next one are
  // checked before a search).  An appending call also takes the item's
  // new-row tag (D = 256 only: its loads select the rows per lane): b * 16 +
  // the offset of sequence b's new token when the item
  // is b's last block, else -1.
  auto item_id = [&](int i, int bh, int& tag) -> int {
    i = min(i, i1 - 1);
    if constexpr (PLANNED) {
      if constexpr (kTags) tag = a.plan_tags[i];
      return a.plan_ids[i];
    } else {
      int b = bh;
      if (s_bcum[b + 1] <= i) b = s_bcum[b + 2] > i ? b + 1 : seq_at(s_bcum, a.batch, i);
      if constexpr (kTags)  // the new row, unless it lies past the attended range
        tag = i == s_bcum[b + 1] - 1 && !((s_over[b >> 5] >> (b & 31)) & 1u)
                  ? b * kBlockSize + ((s_len[b] - 1) & (kBlockSize - 1)) : -1;
      return a.block_tables[(int64_t)b * a.max_blocks + (i - s_bcum[b])];
    }
  };
  int tag_cur = tag_first, tag_nxt = -1;
  int id_cur = PLANNED && have_first ? id_first : item_id(i0 + lane, bc, tag_cur);  // [cbase, +64)
  int id_nxt = item_id(i0 + 64 + lane, bc, tag_nxt);  // items [cbase + 64, cbase + 128)
  int cbase = i0;
  // id of item i >= cbase (uniform): rotates the chunks when i leaves the
  // current one; ids outside the pool become -1; `tag` gets the item's tag
  auto id_at = [&](int i, int& tag) -> int {
    if (i - cbase >= 64) {
      id_cur = id_nxt;
      tag_cur = tag_nxt;
      cbase += 64;
      id_nxt = item_id(cbase + 64 + lane, bc, tag_nxt);
    }
    if constexpr (kTags) tag = __builtin_amdgcn_readlane(tag_cur, i - cbase);
    const int id = __builtin_amdgcn_readlane(id_cur, i - cbase);
    return (id >= 0 && id < a.n_blocks) ? id : -1;
  };
  // query rows of sequence b (lanes past the group load the group's first
  // head: every head column is independent and only real heads are written)
  auto load_q = [&](int b, u32x4* qv) {
    const uint16_t* qp =
        a.q + (int64_t)b * a.q_bstride + (int64_t)(head_ok ? hq : h * a.group) * D;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) qv[ks] = *reinterpret_cast<const u32x4*>(qp + 32 * ks + 8 * g);
  };
  // the next non-empty sequence after b (one exists while items remain)
  auto next_seq = [&](int b) -> int {
    ++b;
    while (uni(s_bcum[b + 1]) == uni(s_bcum[b])) ++b;
    return b;
  };

  u32x4 qv[KS];
  load_q(bc, qv);
  // An appending call (D <= 128) keeps the new token's K and V rows of the
  // next kNewStage sequences of its stream in LDS, for this wave's kv head:
  // kNewStage K rows, then as many V rows (`nstage`).  They are loaded when
  // the stream starts (the loads issue right behind the first block's and are
  // written to LDS once the pipeline's other first loads are issued, so that
  // write waits for the first block and the rows only, and the compiler's
  // waits count the pipeline's loads exactly), and again at a sequence switch that
  // reaches past the staged sequences (a rare path that waits for every load
  // in flight).  A sequence's last block is patched from LDS after its
  // ordinary loads: no load of the block loop is conditional, so the loop's
  // waits are those of the plain call.  (Keeping the rows of the sequence in
  // registers, loaded at each switch, made the compiler wait for all but the
  // newest block at every patch.)  D = 256 selects the rows per lane at load
  // time instead.
  constexpr int VW = KVRegs<D>::VW;
  constexpr int RB = 2 * D;            // bytes of one kv head's row
  constexpr int EPI = 1024 / RB;       // rows per wave-wide 16-byte load
  constexpr int NLD = kNewInLds ? kNewStage / EPI : 1;  // such loads per side
  static_assert(!kNewInLds || kNewStage % EPI == 0, "whole loads of staged rows");
  int e_stage = 0, n_staged = 0;  // bc's entry in the staged rows, entries staged
  // the item of sequence bc whose block holds its new row (-1: none in range,
  // or the sequence is longer than max_seq_len) and the row's offset in it
  int patch_at = -1, patch_off = 0;
  auto set_patch = [&]() {
    if constexpr (kNewInLds) {
      const bool over = (s_over[bc >> 5] >> (bc & 31)) & 1u;
      patch_at = cend == uni(s_bcum[bc + 1]) && !over ? cend - 1 : -1;
      patch_off = (len - 1) & (kBlockSize - 1);
    }
  };
  set_patch();
  // Entries [0, n) from sequence bs: the next n non-empty sequences among the
  // 64 from bs, n <= kNewStage; nseq[k] = the sequence of entry k, or -1 when
  // its new row is not attended here (its last block lies past the range, or
  // it is longer than max_seq_len).  Returns n.
  auto stage_seqs = [&](int bs) -> int {
    const int b = bs + lane;
    const bool ne = b < a.batch && s_bcum[b + 1] > s_bcum[b];
    const uint64_t mask = __builtin_amdgcn_ballot_w64(ne);
    const int rank = (int)__builtin_amdgcn_mbcnt_hi(
        (uint32_t)(mask >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
    if (lane < kNewStage) nseq[lane] = -1;  // entries past n load nothing
    if (ne && rank < kNewStage)
      nseq[rank] = s_bcum[b + 1] <= i1 && !((s_over[b >> 5] >> (b & 31)) & 1u) ? b : -1;
    return min(kNewStage, (int)__builtin_popcountll(mask));
  };
  // One 16-byte piece of a staged row per lane and load: load k holds rows
  // k * EPI + lane / (RB / 16), bytes 16 * (lane % (RB / 16)) of each.  A
  // row that is not needed reads through an offset past the buffer range
  // (zeros, no memory access).
  u32x4 nk[NLD], nv[NLD];
  auto issue_new = [&]() {
    if constexpr (kNewInLds) {
      // the ranges are built where they are used (the compiler would otherwise
      // keep them in scalar registers across the block loop)
      const uint8_t* kb = reinterpret_cast<const uint8_t*>(a.knew);
      const uint8_t* vb = reinterpret_cast<const uint8_t*>(a.vnew);
      asm volatile("" : "+s"(kb), "+s"(vb));
      const auto krs = byte_range(kb, a.knew_span);
      const auto vrs = byte_range(vb, a.vnew_span);
      const uint32_t off = (uint32_t)(h * RB + 16 * (lane % (RB / 16)));
#pragma unroll
      for (int k = 0; k < NLD; ++k) {
        const int b = nseq[k * EPI + lane / (RB / 16)];
        nk[k] = __builtin_amdgcn_raw_buffer_load_b128(
            krs, b >= 0 ? (uint32_t)b * (uint32_t)(2 * a.knew_bstride) + off : kPastRange, 0,
            kNt);
        nv[k] = __builtin_amdgcn_raw_buffer_load_b128(
            vrs, b >= 0 ? (uint32_t)b * (uint32_t)(2 * a.vnew_bstride) + off : kPastRange, 0,
            kNt);
      }
    }
  };
  auto commit_new = [&]() {
    if constexpr (kNewInLds) {
#pragma unroll
      for (int k = 0; k < NLD; ++k) {
        *reinterpret_cast<u32x4*>(nstage + 1024 * k + 16 * lane) = nk[k];
        *reinterpret_cast<u32x4*>(nstage + kNewStage * RB + 1024 * k + 16 * lane) = nv[k];
      }
    }
  };

  f32x4 acc[DPL];
#pragma unroll
  for (int t = 0; t < DPL; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, lsum = 0.f;

  // staged pieces: meta[s] = (b, complete, partial slot)
  const int rec_bytes = stage_record_bytes<D>();
  const int slot_bytes = a.group * 4 * rec_bytes;
  uint8_t* my_rec = stage + (j * 4 + g) * rec_bytes;
  int nstaged = 0;
  auto flush = [&]() {
    if constexpr (!stages_pieces<D>()) return;
    for (int s = 0; s < nstaged; ++s) {
      const int4 md = meta[s];
      f32x4 o[DPL];
      float mm, lt;
      if (head_ok) {
        get_record<D>(my_rec + s * slot_bytes, o, mm, lt);
        store_piece<DT, D>(a, o, mm, lt, uni(md.x), hq, uni(md.y) != 0, uni(md.z), hl0);
      }
    }
    nstaged = 0;
  };

  int ic = i0;  // next item to compute
  auto compute = [&](KVRegs<D>& r, int id, int tag) {
    if constexpr (kNewInLds) {
      if (ic == patch_at) {  // the sequence's last block holds its new row (uniform)
        const int noff = patch_off;
        const uint8_t* kr = nstage + e_stage * RB;  // lane: dims 8g + 32ks
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          const u32x4 kk = *reinterpret_cast<const u32x4*>(kr + 2 * (8 * g + 32 * ks));
          r.k[ks] = j == noff ? kk : r.k[ks];
        }
        uint32_t vw[VW];  // lane: dims D/16 * j
        const uint8_t* vp = kr + kNewStage * RB + 2 * DPL * j;
        if constexpr (VW == 2) {
          const u32x2 x = *reinterpret_cast<const u32x2*>(vp);
          vw[0] = x.x; vw[1] = x.y;
        } else {
#pragma unroll
          for (int i = 0; i < VW / 4; ++i) {
            const u32x4 x = *reinterpret_cast<const u32x4*>(vp + 16 * i);
            vw[4 * i] = x.x; vw[4 * i + 1] = x.y; vw[4 * i + 2] = x.z; vw[4 * i + 3] = x.w;
          }
        }
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
          for (int w = 0; w < VW; ++w) r.v[c][w] = 4 * g + c == noff ? vw[w] : r.v[c][w];
      }
    }
    compute_block<DT, D>(r, qv, acc, m, lsum, (ic - first) * kBlockSize, id >= 0 ? len : 0, g,
                         a.scale_log2);
    if (++ic == cend) {  // the piece of sequence bc in this range ends (uniform)
      float lt = lsum + __shfl_xor(lsum, 16);
      lt += __shfl_xor(lt, 32);
      const int pslot = (int)blockIdx.x + grp * a.batch + bc;
      if (stages_pieces<D>() && a.stage_slots > 0) {
        if (nstaged == a.stage_slots) flush();
        if (head_ok) put_record<D>(my_rec + nstaged * slot_bytes, acc, m, lt);
        if (lane == 0) meta[nstaged] = make_int4(bc, complete ? 1 : 0, pslot, 0);
        ++nstaged;
      } else if (head_ok) {
        store_piece<DT, D>(a, acc, m, lt, bc, hq, complete, pslot, hl0);
      }
      if (ic < i1) {
        bc = next_seq(bc);
        first = uni(s_bcum[bc]);
        cend = min(uni(s_bcum[bc + 1]), i1);
        len = uni(s_len[bc]);
        complete = cend == uni(s_bcum[bc + 1]);  // it starts in range
        load_q(bc, qv);
        set_patch();
        if constexpr (kNewInLds) {
          if (++e_stage == n_staged) {  // past the staged sequences (rare): stage the next
            e_stage = 0;
            n_staged = stage_seqs(bc);
            issue_new();
            commit_new();
          }
        }
#pragma unroll
        for (int t = 0; t < DPL; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
        m = -INFINITY;
        lsum = 0.f;
      }
    }
  };

  // Every block is read through raw buffer ranges (no branch around the
  // loads, so the compiler's wait counts stay exact); `valid`: the item is in
  // the range (a refill past its end reads nothing).  With D = 256 an
  // appending call instead swaps the new token's row into each sequence's
  // last block by lane-wise address selects (a refill past the range then
  // re-reads the range's last block).
  const uint16_t* kh = FUSED ? a.kc + (int64_t)h * D + (int64_t)j * row + 8 * g : nullptr;
  const uint16_t* vh = FUSED ? a.vc + (int64_t)h * D + (int64_t)(4 * g) * row + DPL * j : nullptr;
  const uint16_t* kn_lane = FUSED ? a.knew + (int64_t)h * D + 8 * g : nullptr;
  const uint16_t* vn_lane = FUSED ? a.vnew + (int64_t)h * D + DPL * j : nullptr;
  auto load_item = [&](KVRegs<D>& r, int id, int tag, bool valid) {
    const int64_t off = (int64_t)max(id, 0) * a.blk_stride;
    if constexpr (FUSED && !kNewInLds) {
      const int b = tag >> 4, noff = tag < 0 ? -1 : (tag & (kBlockSize - 1));
      load_block_new<D>(r, kh, vh, off, row, noff, kn_lane + (int64_t)b * a.knew_bstride,
                        vn_lane + (int64_t)b * a.vnew_bstride);
    } else {
      const bool ok = valid && id >= 0;
      const auto kr = byte_range(reinterpret_cast<const uint8_t*>(a.kc + off), ok ? blk_b : 0u);
      const auto vr = byte_range(reinterpret_cast<const uint8_t*>(a.vc + off), ok ? blk_b : 0u);
      load_block<D>(r, kr, vr, koff, voff, row_b);
    }
  };

  const int n = i1 - i0;
  const int nfull = n - n % NBUF;
  KVRegs<D> buf[NBUF];
  int ids[NBUF], tags[NBUF];
  unrolled_steps<NBUF>([&](auto kc) {
    constexpr int k = decltype(kc)::value;
    tags[k] = -1;
    ids[k] = id_at(min(i0 + k, i1 - 1), tags[k]);
    load_item(buf[k], ids[k], tags[k], i0 + k < i1);
    if constexpr (kNewInLds && k == 0) {  // behind the first block's loads
      n_staged = stage_seqs(bc);
      issue_new();
    }
    return false;
  });
  commit_new();  // waits for the first block and the staged rows only
  for (int it = 0; it < nfull; it += NBUF) {
    unrolled_steps<NBUF>([&](auto kc) {
      constexpr int k = decltype(kc)::value;
      compute(buf[k], ids[k], tags[k]);
      tags[k] = -1;
      ids[k] = id_at(min(i0 + it + k + NBUF, i1 - 1), tags[k]);
      load_item(buf[k], ids[k], tags[k], i0 + it + k + NBUF < i1);
      return false;
    });
  }
  unrolled_steps<NBUF>([&](auto kc) {
    constexpr int k = decltype(kc)::value;
    if (nfull + k >= n) return true;
    compute(buf[k], ids[k], tags[k]);
    return false;
  });
  flush();
}

// Prefix sums of the batch's positions and blocks (lengths clamped to
// max_seq_len) into LDS: s_cum[batch + 1] (cost units), s_bcum[batch + 1]
// (blocks), s_len[batch]; with s_over, bit b set when sequence b's length
// exceeds max_seq_len (its last token, an appending call's new row, then lies
// past the attended range).  Every thread of the 64 * kHeadsPerGroup takes
// part.
__device__ __forceinline__ void scan_batch(const int32_t* seq_lens, int batch, int max_seq_len,
                                           int32_t* s_cum, int32_t* s_bcum, int32_t* s_len,
                                           int32_t (*s_wave_tot)[kHeadsPerGroup],
                                           uint32_t* s_over = nullptr) {
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  if (s_over)
    for (int w = tid; w < kMaxBatch / 32; w += 64 * kHeadsPerGroup) s_over[w] = 0u;
  // Prefix sums of the batch's positions and blocks: thread t owns sequences
  // [t * per, t * per + per); a wave scan plus the wave totals give each
  // thread its exclusive offsets.
  {
    const int per = (batch + 64 * kHeadsPerGroup - 1) / (64 * kHeadsPerGroup);
    const int b0 = tid * per;
    int lens[kScanPerThread];
    int cnt = 0, bcnt = 0;
    // all loads issued before any is used (clamped index, masked after)
#pragma unroll
    for (int k = 0; k < kScanPerThread; ++k) lens[k] = seq_lens[min(b0 + k, batch - 1)];
    uint32_t over = 0;  // bit k: sequence b0 + k is longer than max_seq_len
#pragma unroll
    for (int k = 0; k < kScanPerThread; ++k) {
      if (k < per && b0 + k < batch && lens[k] > max_seq_len) over |= 1u << k;
      lens[k] = (k < per && b0 + k < batch) ? min(max(lens[k], 0), max_seq_len) : 0;
      cnt += cost_units(lens[k]);
      bcnt += (lens[k] + kBlockSize - 1) / kBlockSize;
    }
    int x = cnt, y = bcnt;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int xu = __shfl_up(x, o), yu = __shfl_up(y, o);
      if (lane >= o) {
        x += xu;
        y += yu;
      }
    }
    if (lane == 63) {
      s_wave_tot[0][wave] = x;
      s_wave_tot[1][wave] = y;
    }
    __syncthreads();
    int base = 0, bbase = 0;
    for (int w = 0; w < wave; ++w) {
      base += s_wave_tot[0][w];
      bbase += s_wave_tot[1][w];
    }
    int excl = base + x - cnt, bexcl = bbase + y - bcnt;
#pragma unroll
    for (int k = 0; k < kScanPerThread; ++k) {
      if (k < per && b0 + k < batch) {
        s_cum[b0 + k] = excl;
        s_bcum[b0 + k] = bexcl;
        s_len[b0 + k] = lens[k];
        if (s_over && ((over >> k) & 1u)) atomicOr(&s_over[(b0 + k) >> 5], 1u << ((b0 + k) & 31));
        excl += cost_units(lens[k]);
        bexcl += (lens[k] + kBlockSize - 1) / kBlockSize;
      }
    }
    if (tid == 64 * kHeadsPerGroup - 1) {
      s_cum[batch] = base + x;
      s_bcum[batch] = bbase + y;
    }
    __syncthreads();
  }
}

// Workgroup that holds position P of the flattened range (the largest w with
// floor(w * total / n_act) <= P; n_act <= total, so every range is non-empty).
// floor(num / den) for 0 <= num, den < 2^52 (the host bounds every operand
// below by that): the correctly rounded double quotient is within one of the
// exact one, and one integer step corrects it.  A fraction of the cost of a
// 64-bit integer division, which the startup of every workgroup needs several
// of.
__device__ __forceinline__ int64_t div_floor(int64_t num, int64_t den) {
  int64_t q = (int64_t)((double)num / (double)den);
  if (q * den > num) --q;
  else if ((q + 1) * den <= num) ++q;
  return q;
}

__device__ __forceinline__ int64_t owner_of(int64_t P, int64_t total, int64_t n_act) {
  return div_floor((P + 1) * n_act - 1, total);
}

template <int DT, int D, int NBUF, bool PLANNED, bool FUSED>
__global__ __launch_bounds__(64 * kHeadsPerGroup, D >= 256 ? 1 : 2) void
paged_decode_attention_kernel(AttnArgs a) {
  // cum[batch + 1] (positions), len[batch], bcum[batch + 1] (blocks)
  extern __shared__ int32_t s_mem[];
  __shared__ int32_t s_wave_tot[2][kHeadsPerGroup];
  __shared__ int32_t s_find[2];
  __shared__ int4 s_meta[kHeadsPerGroup][kMaxStage];
  __shared__ uint32_t s_over[FUSED ? kMaxBatch / 32 : 1];
  __shared__ int32_t s_newseq[kHeadsPerGroup][FUSED ? kNewStage : 1];
  int32_t* s_cum = s_mem;
  int32_t* s_len = s_mem + a.batch + 1;
  int32_t* s_bcum = s_len + a.batch;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;

  // A planned workgroup's record and the block ids of its first 64 items,
  // loaded before the scan so that they arrive while it runs.
  int rec[kPlanRecord] = {};
  int id_first = 0, tag_first = -1;
  if constexpr (PLANNED) {
#pragma unroll
    for (int k = 0; k < kPlanRecord; ++k) rec[k] = a.plan_wg[(int64_t)blockIdx.x * kPlanRecord + k];
    id_first = a.plan_first[(int64_t)blockIdx.x * 128 + lane];
    if constexpr (FUSED && D > 128)  // per-item tags: the lane-select path only
      tag_first = a.plan_first[(int64_t)blockIdx.x * 128 + 64 + lane];
  }
  scan_batch(a.seq_lens, a.batch, a.max_seq_len, s_cum, s_bcum, s_len, s_wave_tot,
             FUSED ? s_over : nullptr);
  // Empty sequences have no positions: workgroup b % n_wg writes their zeros.
  for (int b = blockIdx.x; b < a.batch; b += gridDim.x) {
    if (s_cum[b + 1] != s_cum[b]) continue;  // uniform over the workgroup
    uint16_t* op = a.out + (int64_t)b * a.out_bstride;
    for (int e = tid * 8; e < a.n_q_heads * a.head_dim; e += 8 * 64 * kHeadsPerGroup)
      *reinterpret_cast<u32x4*>(op + e) = u32x4{0u, 0u, 0u, 0u};
  }

  uint8_t* stage = reinterpret_cast<uint8_t*>(s_mem) + a.stage_off +
                   wave * a.stage_slots * a.group * 4 * stage_record_bytes<D>();
  uint8_t* nstage = reinterpret_cast<uint8_t*>(s_mem) + a.newrow_off + wave * kNewStage * 4 * D;
  if constexpr (PLANNED) {
    if (uni(rec[0]) < 0) return;  // idle workgroup
    const int items = s_bcum[a.batch];
    for (int grp = uni(rec[0]); grp <= uni(rec[1]); ++grp) {
      const bool first_pass = grp == uni(rec[0]);
      const int i0 = first_pass ? uni(rec[2]) : 0;
      const int b0 = first_pass ? uni(rec[3]) : uni(rec[5]);
      const int i1 = grp == uni(rec[1]) ? uni(rec[4]) : items;
      if (i1 > i0)
        attend_items<DT, D, NBUF, true, FUSED>(a, s_bcum, s_len, stage, s_meta[wave], grp, b0,
                                               i0, i1, first_pass, id_first,
                                               first_pass ? tag_first : -1, s_over, nstage,
                                               s_newseq[wave]);
    }
    return;
  }
  const int64_t W = s_cum[a.batch];
  const int64_t total = W * a.n_groups;
  // With fewer positions than workgroups only the first `total` take part, so
  // that every range is non-empty.
  const int64_t n_act = min((int64_t)a.n_wg, total);
  if ((int64_t)blockIdx.x >= n_act) {
    if (tid == 0) a.desc[blockIdx.x] = make_int4(-1, 0, 0, 0);
    return;
  }
  int64_t P = div_floor((int64_t)blockIdx.x * total, n_act);
  const int64_t p_end = div_floor((int64_t)(blockIdx.x + 1) * total, n_act);
  // Every value below is uniform over the workgroup.  A sequence occupies
  // positions [s_cum[b], s_cum[b + 1]) of its group: kSegmentCost charge
  // positions, then one per block.
  bool first_pass = true;
  while (P < p_end) {  // one pass per kv-head group the range touches
    const int grp = (int)div_floor(P, W);
    const int64_t pbase = (int64_t)grp * W;
    const int64_t q_end = min(p_end, pbase + W);
    const int p0 = (int)(P - pbase), p1 = (int)(q_end - pbase);
    // the sequences holding positions p0 and p1 (p1 < W), every thread
    // testing its own sequences at once
    for (int b = tid; b < a.batch; b += 64 * kHeadsPerGroup) {
      const int lo = s_cum[b], hi = s_cum[b + 1];
      if (lo <= p0 && p0 < hi) s_find[0] = b;
      if (lo <= p1 && p1 < hi) s_find[1] = b;
    }
    __syncthreads();
    // block items before position p of sequence b
    auto items_before = [&](int b, int p) -> int {
      const int nblk = s_bcum[b + 1] - s_bcum[b];
      return s_bcum[b] + min(max(p - s_cum[b] - kSegmentCost, 0), nblk);
    };
    const int b0 = s_find[0];
    const int i0 = items_before(b0, p0);
    const int i1 = p1 == (int)W ? s_bcum[a.batch] : items_before(s_find[1], p1);
    if (first_pass) {
      // The range's first piece is the only one that can end a cut sequence:
      // describe it for the merge when it does.
      const int64_t w0 = owner_of(pbase + s_cum[b0] + kSegmentCost, total, n_act);
      const int64_t w1 = owner_of(pbase + s_cum[b0 + 1] - 1, total, n_act);
      if (tid == 0)
        a.desc[blockIdx.x] = (w0 != w1 && w1 == (int64_t)blockIdx.x)
                                 ? make_int4(b0, grp, (int)w0, (int)(w1 - w0 + 1))
                                 : make_int4(-1, 0, 0, 0);
      first_pass = false;
    }
    if (i1 > i0)
      attend_items<DT, D, NBUF, false, FUSED>(a, s_bcum, s_len, stage, s_meta[wave], grp, b0,
                                              i0, i1, false, 0, -1, s_over, nstage,
                                              s_newseq[wave]);
    P = q_end;
    __syncthreads();  // s_find is rewritten by the next pass
  }
}

struct PlanArgs {
  const int32_t* block_tables;
  int32_t max_blocks;
  const int32_t* seq_lens;
  int32_t batch;
  int32_t max_seq_len;
  int32_t n_groups;
  int32_t n_wg;
  int32_t desc_per_seq;  // desc indexed by grp * batch + b (else by workgroup)
  int32_t* wg;
  int4* desc;
  int32_t* first;
  int32_t* last;
  int32_t* ids;
  int32_t* tags;
};

// Builds a decode plan (see PlanLayout) with the partition the attention
// kernel computes for itself: every workgroup scans the lengths, then the
// grid shares the per-workgroup records, the first-64 id lists and the
// item-order ids.
__global__ __launch_bounds__(64 * kHeadsPerGroup) void decode_plan_kernel(PlanArgs p) {
  extern __shared__ int32_t s_mem[];
  __shared__ int32_t s_wave_tot[2][kHeadsPerGroup];
  __shared__ uint32_t s_over[kMaxBatch / 32];
  int32_t* s_cum = s_mem;
  int32_t* s_len = s_mem + p.batch + 1;
  int32_t* s_bcum = s_len + p.batch;
  scan_batch(p.seq_lens, p.batch, p.max_seq_len, s_cum, s_bcum, s_len, s_wave_tot, s_over);
  const int64_t W = s_cum[p.batch];
  const int items = s_bcum[p.batch];
  const int64_t total = W * p.n_groups;
  const int64_t n_act = min((int64_t)p.n_wg, total);
  const int gtid = blockIdx.x * blockDim.x + threadIdx.x;
  const int gsz = gridDim.x * blockDim.x;
  auto items_before = [&](int b, int pos) -> int {
    const int nblk = s_bcum[b + 1] - s_bcum[b];
    return s_bcum[b] + min(max(pos - s_cum[b] - kSegmentCost, 0), nblk);
  };
  // workgroup w's range: first and last kv-head group, first item and its
  // sequence, end item in the last group and in the first
  struct Range {
    int gf, gl, i0, b0, i1l, i1f;
  };
  auto range_of = [&](int w) -> Range {
    const int64_t P = div_floor((int64_t)w * total, n_act);
    const int64_t pe = div_floor((int64_t)(w + 1) * total, n_act);
    Range r;
    r.gf = (int)div_floor(P, W);
    r.gl = (int)div_floor(pe - 1, W);
    const int p0 = (int)(P - (int64_t)r.gf * W);
    r.b0 = seq_at(s_cum, p.batch, p0);
    r.i0 = items_before(r.b0, p0);
    const int pl = (int)(pe - (int64_t)r.gl * W);
    r.i1l = pl == (int)W ? items : items_before(seq_at(s_cum, p.batch, pl), pl);
    r.i1f = r.gf == r.gl ? r.i1l : items;
    return r;
  };
  for (int w = gtid; w < p.n_wg; w += gsz) {
    int32_t* rec = p.wg + (int64_t)w * kPlanRecord;
    if (w >= n_act) {
      rec[0] = -1;
      if (!p.desc_per_seq) p.desc[w] = make_int4(-1, 0, 0, 0);
      continue;
    }
    const Range r = range_of(w);
    rec[0] = r.gf;
    rec[1] = r.gl;
    rec[2] = r.i0;
    rec[3] = r.b0;
    rec[4] = r.i1l;
    rec[5] = seq_at(s_cum, p.batch, 0);  // first non-empty sequence
    rec[6] = 0;
    rec[7] = 0;
    if (p.desc_per_seq) continue;
    // the range's first piece is the only one that can end a cut sequence
    const int64_t pbase = (int64_t)r.gf * W;
    const int64_t w0 = owner_of(pbase + s_cum[r.b0] + kSegmentCost, total, n_act);
    const int64_t w1 = owner_of(pbase + s_cum[r.b0 + 1] - 1, total, n_act);
    p.desc[w] = (w0 != w1 && w1 == (int64_t)w) ? make_int4(r.b0, r.gf, (int)w0, (int)(w1 - w0 + 1))
                                               : make_int4(-1, 0, 0, 0);
  }
  if (p.desc_per_seq) {  // one descriptor per (group, sequence): cut or not
    for (int e = gtid; e < p.n_groups * p.batch; e += gsz) {
      const int grp = e / p.batch, b = e % p.batch;
      int4 d = make_int4(-1, 0, 0, 0);
      if (s_bcum[b + 1] > s_bcum[b]) {
        const int64_t pbase = (int64_t)grp * W;
        const int64_t w0 = owner_of(pbase + s_cum[b] + kSegmentCost, total, n_act);
        const int64_t w1 = owner_of(pbase + s_cum[b + 1] - 1, total, n_act);
        if (w0 != w1) d = make_int4(b, grp, (int)w0, (int)(w1 - w0 + 1));
      }
      p.desc[e] = d;
    }
  }
  auto id_of = [&](int i) -> int32_t {
    const int b = seq_at(s_bcum, p.batch, i);
    return p.block_tables[(int64_t)b * p.max_blocks + (i - s_bcum[b])];
  };
  // an appending call's new row: the last attended token, unless the
  // sequence is longer than the bound (its new row then lies past the range)
  auto tag_of = [&](int i) -> int32_t {
    const int b = seq_at(s_bcum, p.batch, i);
    return i == s_bcum[b + 1] - 1 && !((s_over[b >> 5] >> (b & 31)) & 1u)
               ? b * kBlockSize + ((s_len[b] - 1) & (kBlockSize - 1)) : -1;
  };
  for (int64_t e = gtid; e < (int64_t)p.n_wg * 64; e += gsz) {
    const int w = (int)(e >> 6);
    if (w >= n_act) continue;
    const Range r = range_of(w);
    if (r.i1f <= r.i0) continue;  // the first pass holds no block
    const int i = min(r.i0 + (int)(e & 63), r.i1f - 1);
    p.first[(int64_t)w * 128 + (e & 63)] = id_of(i);
    p.first[(int64_t)w * 128 + 64 + (e & 63)] = tag_of(i);
  }
  for (int i = gtid; i < items; i += gsz) {
    p.ids[i] = id_of(i);
    p.tags[i] = tag_of(i);
  }
  // the block of each sequence's last position (an appending call's new row),
  // read from its own length also past the bound; -1 without such a block
  for (int b = gtid; b < p.batch; b += gsz) {
    const int len = p.seq_lens[b];
    p.last[b] = len > 0 && (len - 1) / kBlockSize < p.max_blocks
                    ? p.block_tables[(int64_t)b * p.max_blocks + (len - 1) / kBlockSize]
                    : -1;
  }
}

// Merge the pieces of the cut sequence that descriptor blockIdx.x names
// (none: nothing to do), for kv head grp * 4 + blockIdx.y:
//   out = sum_s w_s o_s / sum_s w_s l_s,  w_s = 2^(m_s - max m).
// The kv head's G query heads x D/4 float4 columns are "items", one per
// thread (KI per thread past 256 items); a thread loads the (m, l) and o of
// up to PB pieces of its item at once and merges them in registers, so a
// sequence of up to PB pieces costs one round trip and no LDS.  (Per-wave
// pieces merged through LDS took one round trip per four pieces: per
// workgroup timestamps put the combine's tail at 3.4 us of piece loads for a
// nine-piece sequence against 1.7 us for two; this version measured 2.4 us
// per layer faster on the Qwen2.5-7B batch and 1.9 us on the Yi-1.5-9B one.)
// Most of the grid's workgroups hold no task and exit after the descriptor
// load, so every workgroup must stay resident at once (four per CU): the
// pieces are raw buffer loads whose piece stride is a scalar offset, which
// keeps PB = 12 at ~110 VGPRs (PB = 16 measured 1 us slower on the
// Yi-1.5-9B batch, whose longest sequences have 10-15 pieces; 8 the same).
// The cache write of an appending call, spread over every thread of the
// combine grid (extra grid rows for it measured 0.25 us per Qwen2.5-7B
// layer): the new token's K and V rows of every sequence and kv head go to
// token (len - 1) % 16 of the sequence's last block, 16 bytes per lane.  The
// main kernel read those rows from the append's input, so nothing reads the
// slot before this write.  Blocks outside the pool are skipped, as the
// attention masks them.  A thread's first chunk is loaded, with its length
// and (planned) block id, before the workgroup's merge and stored after it,
// so the merge does not wait behind the copy's round trip; further chunks
// (batches whose rows outnumber the grid's threads) are copied after it.
template <int D>
struct NewRowChunk {
  int b, kv, h, chunk;
  __device__ NewRowChunk(const AttnArgs& a, int64_t c) {
    constexpr int C = D / 8;  // 16-byte chunks of one kv head's row
    chunk = (int)(c % C);
    const int64_t rest = c / C;
    kv = (int)(rest & 1);
    h = (int)((rest >> 1) % a.n_kv_heads);
    b = (int)((rest >> 1) / a.n_kv_heads);
  }
  __device__ const u32x4* src(const AttnArgs& a) const {
    return reinterpret_cast<const u32x4*>(
        (kv ? a.vnew + (int64_t)b * a.vnew_bstride : a.knew + (int64_t)b * a.knew_bstride) +
        (int64_t)h * D + 8 * chunk);
  }
  // the new row goes to its own position len - 1 (the append's slot), also
  // when the length exceeds the attended bound; a table without a block for
  // it gets nothing, as the append skips a slot outside the pool.  `blk`: the
  // plan's block of that position when planned (loaded by the caller).
  __device__ u32x4* dst(const AttnArgs& a, int len, int blk) const {
    if (len <= 0) return nullptr;
    if (!a.plan_last) {
      if ((len - 1) / kBlockSize >= a.max_blocks) return nullptr;
      blk = a.block_tables[(int64_t)b * a.max_blocks + (len - 1) / kBlockSize];
    }
    if (blk < 0 || blk >= a.n_blocks) return nullptr;
    const int64_t row = (int64_t)a.n_kv_heads * D;
    return reinterpret_cast<u32x4*>(const_cast<uint16_t*>(kv ? a.vc : a.kc) +
                                    (int64_t)blk * a.blk_stride +
                                    (int64_t)((len - 1) % kBlockSize) * row + (int64_t)h * D +
                                    8 * chunk);
  }
};
template <int D>
__device__ __forceinline__ int64_t new_row_chunks(const AttnArgs& a) {
  return (int64_t)a.batch * a.n_kv_heads * 2 * (D / 8);
}


template <int DT, int D, int KI, int PB>
__device__ __forceinline__ void merge_pieces(const AttnArgs& a, const int4 d) {
  using E = Elem<DT>;
  constexpr int D4 = D / 4;  // float4 per query head
  constexpr int NT = 64 * kHeadsPerGroup;
  const int b = d.x, grp = d.y, npieces = d.w;
  const int h = grp * kHeadsPerGroup + blockIdx.y;
  if (h >= a.n_kv_heads) return;
  const int items = a.group * D4;
  const int64_t slot0 = (int64_t)d.z + (int64_t)grp * a.batch + b;
  const int hl0 = blockIdx.y * a.group;  // first query head of h within a slot
  // the partials as raw buffers: a piece's offset is a uniform (scalar)
  // stride, so the PB loads of a round share one vector offset per thread
  // (the host keeps both regions below 2^31 bytes)
  const auto mlr = byte_range(reinterpret_cast<const uint8_t*>(a.part_ml), a.ml_bytes);
  const auto por = byte_range(reinterpret_cast<const uint8_t*>(a.part_o), a.o_bytes);
  const uint32_t ml_step = (uint32_t)a.hpg * 8u, o_step = (uint32_t)a.hpg * D * 4u;
#pragma unroll
  for (int k = 0; k < KI; ++k) {
    const int it = (int)threadIdx.x + NT * k;
    if (it >= items) break;
    const int64_t pidx0 = slot0 * a.hpg + hl0 + it / D4;
    const int col = 4 * (it % D4);
    const uint32_t ml_off = (uint32_t)(pidx0 * 8), o_off = (uint32_t)((pidx0 * D + col) * 4);
    float mx = -INFINITY, lt = 0.f;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    for (int s0 = 0; s0 < npieces; s0 += PB) {  // one round for up to PB pieces
      float2 ml[PB];
      f32x4 po[PB];
#pragma unroll
      for (int u = 0; u < PB; ++u) {
        ml[u] = make_float2(-INFINITY, 0.f);
        po[u] = f32x4{0.f, 0.f, 0.f, 0.f};
        if (s0 + u < npieces) {  // uniform
          const uint32_t sp = (uint32_t)(s0 + u);
          const u32x2 mw = __builtin_amdgcn_raw_buffer_load_b64(mlr, ml_off, sp * ml_step, 0);
          ml[u] = make_float2(__uint_as_float(mw.x), __uint_as_float(mw.y));
          const u32x4 ow = __builtin_amdgcn_raw_buffer_load_b128(por, o_off, sp * o_step, 0);
          po[u] = f32x4{__uint_as_float(ow.x), __uint_as_float(ow.y), __uint_as_float(ow.z),
                        __uint_as_float(ow.w)};
        }
      }
      float mn = mx;
#pragma unroll
      for (int u = 0; u < PB; ++u) mn = fmaxf(mn, ml[u].x);
      if (mn == -INFINITY) continue;  // no readable block yet
      const float sc = mx == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mx - mn);
      acc *= sc;
      lt *= sc;
#pragma unroll
      for (int u = 0; u < PB; ++u) {
        // absent, or a piece with no readable block: weight 0
        const float w = ml[u].x == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(ml[u].x - mn);
        acc += po[u] * w;
        lt += ml[u].y * w;
      }
      mx = mn;
    }
    const float inv = lt > 0.f ? 1.f / lt : 0.f;
    uint16_t* op = a.out + (int64_t)b * a.out_bstride + (int64_t)(h * a.group) * D +
                   (int64_t)(it / D4) * D + col;
    *reinterpret_cast<u32x2*>(op) =
        u32x2{E::bits(acc[0] * inv) | (E::bits(acc[1] * inv) << 16),
              E::bits(acc[2] * inv) | (E::bits(acc[3] * inv) << 16)};
  }
}

template <int DT, int D, int KI, int PB>
__global__ __launch_bounds__(64 * kHeadsPerGroup) void attention_combine_kernel(AttnArgs a) {
  const int4 d = a.desc[blockIdx.x];
  // an appending call: this thread's first new-row chunk, loaded ahead of the merge
  const int64_t total = a.knew ? new_row_chunks<D>(a) : 0;
  const int64_t stride = (int64_t)gridDim.x * gridDim.y * blockDim.x;
  const int64_t c0 = ((int64_t)blockIdx.y * gridDim.x + blockIdx.x) * blockDim.x + threadIdx.x;
  u32x4 v0 = {0u, 0u, 0u, 0u};
  int len0 = 0, blk0 = -1;
  if (c0 < total) {
    const NewRowChunk<D> r(a, c0);
    v0 = __builtin_nontemporal_load(r.src(a));
    len0 = a.seq_lens[r.b];
    if (a.plan_last) blk0 = a.plan_last[r.b];
  }
  if (d.x >= 0) merge_pieces<DT, D, KI, PB>(a, d);  // uniform over the workgroup
  if (c0 < total) {
    const NewRowChunk<D> r(a, c0);
    if (u32x4* p = r.dst(a, len0, blk0)) __builtin_nontemporal_store(v0, p);
  }
  for (int64_t c = c0 + stride; c < total; c += stride) {
    const NewRowChunk<D> r(a, c);
    if (u32x4* p = r.dst(a, a.seq_lens[r.b], a.plan_last ? a.plan_last[r.b] : -1))
      __builtin_nontemporal_store(__builtin_nontemporal_load(r.src(a)), p);
  }
}

// Dynamic LDS of the main kernel: the scan arrays, then (16-byte aligned) the
// staging records of the four waves, then an appending call's staged new rows
// (D <= 128: kNewStage K and V rows per wave).  Sets a.stage_slots,
// a.stage_off and a.newrow_off.
size_t lds_bytes(AttnArgs& a, int max_lds) {
  const int64_t scan = ((int64_t)(3 * a.batch + 2) * (int64_t)sizeof(int32_t) + 15) / 16 * 16;
  const int64_t per_slot = (int64_t)kHeadsPerGroup * a.group * 4 * (a.head_dim + 16);
  const int64_t newrows =
      a.knew && a.head_dim <= 128 ? (int64_t)kHeadsPerGroup * kNewStage * 4 * a.head_dim : 0;
  const int64_t budget = std::min<int64_t>(kStageBudget, max_lds - newrows) - scan;
  a.stage_off = (int32_t)scan;
  a.stage_slots = a.head_dim > 128 ? 0
                  : (int32_t)std::max<int64_t>(0, std::min<int64_t>(kMaxStage, budget / per_slot));
  a.newrow_off = (int32_t)(scan + a.stage_slots * per_slot);
  return (size_t)(a.newrow_off + newrows);
}

// Workgroups of the main kernel for one launch: one per CU (measured on the
// Qwen2.5-7B batch: one workgroup of four waves per CU with three blocks in
// flight per wave beats two or three per CU), or the caller's count.
int workgroups_for(int32_t requested, int* n_wg) {
  if (requested > 0) {
    *n_wg = requested;
    return AEGKV_OK;
  }
  DeviceState* ds = nullptr;
  int rc = current_device_state(&ds);
  if (rc) return rc;
  *n_wg = std::min(std::max(1, ds->num_cu), kMaxWorkgroups);
  return AEGKV_OK;
}

// The kernel's position arithmetic: a group's positions W (bounded by
// chunk * (blocks + kSegmentCost)) must fit int32, and the products of the
// range arithmetic (total * n_wg, total = W * n_groups) must stay below 2^52
// for div_floor.
bool positions_fit(int64_t chunk, int64_t nblk_max, int64_t n_groups, int64_t n_wg) {
  const int64_t w_max = chunk * (nblk_max + kSegmentCost);
  return w_max < (1ll << 31) && w_max * n_groups * n_wg < (1ll << 52);
}

template <int DT, int D, int KI, int PB>
int launch_combine(const AttnArgs& a, hipStream_t stream) {
  hipLaunchKernelGGL((attention_combine_kernel<DT, D, KI, PB>),
                     dim3(a.n_desc, kHeadsPerGroup), dim3(64 * kHeadsPerGroup), 0,
                     stream, a);
  AEGKV_HIP_TRY(hipGetLastError());
  return AEGKV_OK;
}

template <int DT, int D, bool PLANNED, bool FUSED>
void launch_main(const AttnArgs& a, size_t lds, hipStream_t stream) {
  hipLaunchKernelGGL((paged_decode_attention_kernel<DT, D, pipeline_depth<D>(), PLANNED, FUSED>),
                     dim3(a.n_wg), dim3(64 * kHeadsPerGroup), lds, stream, a);
}

template <int DT, int D>
int launch_attention(const AttnArgs& a, size_t lds, hipStream_t stream) {
  if (a.plan_wg) {
    if (a.knew) launch_main<DT, D, true, true>(a, lds, stream);
    else launch_main<DT, D, true, false>(a, lds, stream);
  } else {
    if (a.knew) launch_main<DT, D, false, true>(a, lds, stream);
    else launch_main<DT, D, false, false>(a, lds, stream);
  }
  AEGKV_HIP_TRY(hipGetLastError());
  const int items = a.group * (D / 4);  // <= 16 * D / 4
  if (items <= 64 * kHeadsPerGroup) return launch_combine<DT, D, 1, 12>(a, stream);
  if (items <= 2 * 64 * kHeadsPerGroup) return launch_combine<DT, D, 2, 12>(a, stream);
  return launch_combine<DT, D, 4, 12>(a, stream);
}

}  // namespace
}  // namespace aegkv

namespace aegkv {
namespace {
// Both entry points: `plan` (with plan_bytes) replaces the block tables when
// given.
// The new token's K/V rows of an appending call (none: key == nullptr).
struct NewRows {
  const void* key = nullptr;
  int64_t key_bstride = 0;
  const void* value = nullptr;
  int64_t value_bstride = 0;
};

int run_attention(void* out, int64_t out_batch_stride, const void* q, int64_t q_batch_stride,
                  const void* key_cache, const void* value_cache, int64_t cache_block_stride,
                  int64_t n_blocks, const int32_t* block_tables, int32_t max_blocks,
                  const void* plan, uint64_t plan_bytes, const int32_t* seq_lens, int32_t batch,
                  int32_t max_seq_len, int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim,
                  int32_t block_size, float scale, int32_t dtype, int32_t n_workgroups,
                  void* workspace, uint64_t workspace_bytes, aegkv_stream_t stream,
                  const NewRows& nr = NewRows()) {
  if (batch < 0 || max_seq_len < 0 || n_q_heads <= 0 || n_kv_heads <= 0 || max_blocks < 0 ||
      n_blocks < 0 || n_workgroups < 0)
    return AEGKV_ERR_INVALID_ARG;
  if (n_q_heads % n_kv_heads) return AEGKV_ERR_INVALID_ARG;
  if (block_size != kBlockSize || (head_dim != 64 && head_dim != 128 && head_dim != 256) ||
      n_q_heads / n_kv_heads > 16 || (dtype != AEGKV_DTYPE_BF16 && dtype != AEGKV_DTYPE_FP16))
    return AEGKV_ERR_UNSUPPORTED;
  if (batch == 0) return AEGKV_OK;
  if (!out || !q || !key_cache || !value_cache || (!block_tables && !plan) || !seq_lens ||
      n_blocks == 0)
    return AEGKV_ERR_INVALID_ARG;
  if (plan && batch > kMaxBatch) return AEGKV_ERR_UNSUPPORTED;
  if (!aligned16(out) || !aligned16(q) || !aligned16(key_cache) || !aligned16(value_cache) ||
      ((q_batch_stride * 2) & 15) || ((out_batch_stride * 2) & 15) ||
      ((cache_block_stride * 2) & 15))
    return AEGKV_ERR_MISALIGNED;
  if (n_q_heads > 65535 || n_workgroups > kMaxWorkgroups) return AEGKV_ERR_UNSUPPORTED;
  if (nr.key) {
    if (!nr.value || nr.key_bstride < (int64_t)n_kv_heads * head_dim ||
        nr.value_bstride < (int64_t)n_kv_heads * head_dim)
      return AEGKV_ERR_INVALID_ARG;
    if (!aligned16(nr.key) || !aligned16(nr.value) || ((nr.key_bstride * 2) & 15) ||
        ((nr.value_bstride * 2) & 15))
      return AEGKV_ERR_MISALIGNED;
  }
  const int64_t nblk_max = ((int64_t)max_seq_len + kBlockSize - 1) / kBlockSize;
  if (!plan && nblk_max > max_blocks) return AEGKV_ERR_INVALID_ARG;
  const int32_t chunk = std::min(batch, kMaxBatch);
  int n_wg = 0;
  int rc = workgroups_for(n_workgroups, &n_wg);
  if (rc) return rc;
  const int32_t group = n_q_heads / n_kv_heads;
  const int32_t n_groups = (n_kv_heads + kHeadsPerGroup - 1) / kHeadsPerGroup;
  if (!positions_fit(chunk, nblk_max, n_groups, n_wg)) return AEGKV_ERR_UNSUPPORTED;
  const WorkspaceLayout lay =
      workspace_layout(chunk, kHeadsPerGroup * group, head_dim, n_wg, n_groups);
  if (!workspace || workspace_bytes < (uint64_t)lay.total) return AEGKV_ERR_WORKSPACE;
  if (!aligned16(workspace)) return AEGKV_ERR_MISALIGNED;
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  AttnArgs a;
  a.kc = static_cast<const uint16_t*>(key_cache);
  a.vc = static_cast<const uint16_t*>(value_cache);
  a.blk_stride = cache_block_stride;
  a.n_blocks = n_blocks;
  a.max_blocks = max_blocks;
  a.n_q_heads = n_q_heads;
  a.n_kv_heads = n_kv_heads;
  a.head_dim = head_dim;
  a.group = group;
  a.hpg = kHeadsPerGroup * group;
  a.n_groups = n_groups;
  a.n_wg = n_wg;
  a.scale_log2 = scale * 1.4426950408889634f;
  a.max_seq_len = max_seq_len;
  a.q_bstride = q_batch_stride;
  a.out_bstride = out_batch_stride;
  a.desc = reinterpret_cast<int4*>(ws);
  a.plan_wg = a.plan_first = a.plan_ids = a.plan_last = a.plan_tags = nullptr;
  a.knew = static_cast<const uint16_t*>(nr.key);
  a.vnew = static_cast<const uint16_t*>(nr.value);
  a.knew_bstride = nr.key_bstride;
  a.vnew_bstride = nr.value_bstride;
  a.knew_span = a.vnew_span = 0;
  a.n_desc = n_wg;
  if (plan) {
    if (desc_per_sequence(batch, n_groups, n_wg)) a.n_desc = batch * n_groups;
    const PlanLayout pl = plan_layout(batch, n_wg, nblk_max);
    if (plan_bytes < (uint64_t)pl.total) return AEGKV_ERR_INVALID_ARG;
    if (!aligned16(plan)) return AEGKV_ERR_MISALIGNED;
    const uint8_t* pb = static_cast<const uint8_t*>(plan);
    a.plan_wg = reinterpret_cast<const int32_t*>(pb + pl.wg);
    a.desc = reinterpret_cast<int4*>(const_cast<uint8_t*>(pb + pl.desc));
    a.plan_first = reinterpret_cast<const int32_t*>(pb + pl.first);
    a.plan_last = reinterpret_cast<const int32_t*>(pb + pl.last);
    a.plan_ids = reinterpret_cast<const int32_t*>(pb + pl.ids);
    a.plan_tags = reinterpret_cast<const int32_t*>(pb + pl.tags);
  }
  a.part_ml = reinterpret_cast<float2*>(ws + lay.desc_bytes);
  a.part_o = reinterpret_cast<float*>(ws + lay.desc_bytes + lay.ml_bytes);
  if (lay.ml_bytes >= (1ll << 31) || lay.o_bytes >= (1ll << 31)) return AEGKV_ERR_UNSUPPORTED;
  a.ml_bytes = (uint32_t)lay.ml_bytes;
  a.o_bytes = (uint32_t)lay.o_bytes;
  hipStream_t st = (hipStream_t)stream;
  const bool bf = dtype == AEGKV_DTYPE_BF16;
  DeviceState* ds = nullptr;
  rc = current_device_state(&ds);
  if (rc) return rc;
  // Batches above kMaxBatch run as consecutive launches of kMaxBatch sequences
  // that share the workspace (stream order keeps them apart).
  for (int32_t c = 0; c < batch; c += kMaxBatch) {
    a.batch = std::min(kMaxBatch, batch - c);
    a.q = static_cast<const uint16_t*>(q) + (int64_t)c * q_batch_stride;
    a.out = static_cast<uint16_t*>(out) + (int64_t)c * out_batch_stride;
    a.block_tables = block_tables ? block_tables + (int64_t)c * max_blocks : nullptr;
    a.seq_lens = seq_lens + c;
    if (nr.key) {
      a.knew = static_cast<const uint16_t*>(nr.key) + (int64_t)c * nr.key_bstride;
      a.vnew = static_cast<const uint16_t*>(nr.value) + (int64_t)c * nr.value_bstride;
      // the staged rows' buffer ranges: row b of kv head h at b * stride + h * D
      const int64_t row_end = (int64_t)n_kv_heads * head_dim * 2;
      const int64_t ks = (int64_t)(a.batch - 1) * nr.key_bstride * 2 + row_end;
      const int64_t vs = (int64_t)(a.batch - 1) * nr.value_bstride * 2 + row_end;
      if (ks >= (1ll << 31) || vs >= (1ll << 31)) return AEGKV_ERR_UNSUPPORTED;
      a.knew_span = (uint32_t)ks;
      a.vnew_span = (uint32_t)vs;
    }
    const size_t lds = lds_bytes(a, ds->max_lds);
    switch (head_dim) {
      case 64: rc = bf ? launch_attention<AEGKV_DTYPE_BF16, 64>(a, lds, st)
                       : launch_attention<AEGKV_DTYPE_FP16, 64>(a, lds, st); break;
      case 128: rc = bf ? launch_attention<AEGKV_DTYPE_BF16, 128>(a, lds, st)
                        : launch_attention<AEGKV_DTYPE_FP16, 128>(a, lds, st); break;
      default: rc = bf ? launch_attention<AEGKV_DTYPE_BF16, 256>(a, lds, st)
                       : launch_attention<AEGKV_DTYPE_FP16, 256>(a, lds, st); break;
    }
    if (rc) return rc;
  }
  return AEGKV_OK;
}
// Workspace of aegkv_paged_decode_attention_noalloc, held by the library in
// device memory it never allocates: the merge descriptors and fp32 partials of
// one call (the same layout the caller's workspace holds).  Every GPU the
// library runs on has its own copy of the array until the process ends; its
// address there comes from hipGetSymbolAddress, once per device.  Nothing in
// it needs clearing between calls: every byte a call's combine reads is
// written by the same call.
constexpr uint64_t kScratchBytes = 32ull << 20;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

std::mutex g_scratch_mu;
std::map<int, void*> g_scratch_ptr;  // device -> address of `scratch` on it

// Address of the current device's `scratch` (looked up on the first call on a
// device, with that device current).
int scratch_of_current_device(void** ptr) {
  int dev = 0;
  AEGKV_HIP_TRY(hipGetDevice(&dev));
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  auto it = g_scratch_ptr.find(dev);
  if (it != g_scratch_ptr.end()) {
    *ptr = it->second;
    return AEGKV_OK;
  }
  void* p = nullptr;
  AEGKV_HIP_TRY(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
  g_scratch_ptr[dev] = p;
  *ptr = p;
  return AEGKV_OK;
}
}  // namespace
}  // namespace aegkv

using namespace aegkv;

extern "C" {

int aegkv_paged_decode_attention_noalloc(void* out, int64_t out_batch_stride, const void* q,
                                         int64_t q_batch_stride, const void* key_cache,
                                         const void* value_cache, int64_t cache_block_stride,
                                         int64_t n_blocks, const int32_t* block_tables,
                                         int32_t max_blocks, const int32_t* seq_lens,
                                         int32_t batch, int32_t max_seq_len, int32_t n_q_heads,
                                         int32_t n_kv_heads, int32_t head_dim,
                                         int32_t block_size, float scale, int32_t dtype,
                                         int32_t n_workgroups, aegkv_stream_t stream) {
  const int64_t need = aegkv_paged_decode_attention_workspace_size(
      batch, n_q_heads, n_kv_heads, head_dim, max_seq_len, dtype, n_workgroups);
  if (need < 0) return (int)need;
  if ((uint64_t)need > kScratchBytes) return AEGKV_ERR_SCRATCH;
  if (batch == 0) return AEGKV_OK;
  if (!block_tables) return AEGKV_ERR_INVALID_ARG;
  void* ws = nullptr;
  const int rc = scratch_of_current_device(&ws);
  if (rc) return rc;
  return run_attention(out, out_batch_stride, q, q_batch_stride, key_cache, value_cache,
                       cache_block_stride, n_blocks, block_tables, max_blocks, nullptr, 0,
                       seq_lens, batch, max_seq_len, n_q_heads, n_kv_heads, head_dim,
                       block_size, scale, dtype, n_workgroups, ws, kScratchBytes, stream);
}

int64_t aegkv_paged_decode_attention_workspace_size(int32_t batch, int32_t n_q_heads,
                                                     int32_t n_kv_heads, int32_t head_dim,
                                                     int32_t max_seq_len, int32_t dtype,
                                                     int32_t n_workgroups) {
  if (batch < 0 || n_q_heads <= 0 || n_kv_heads <= 0 || n_q_heads % n_kv_heads ||
      n_workgroups < 0 || max_seq_len < 0)
    return AEGKV_ERR_INVALID_ARG;
  if (n_workgroups > kMaxWorkgroups) return AEGKV_ERR_UNSUPPORTED;
  if ((head_dim != 64 && head_dim != 128 && head_dim != 256) ||
      (dtype != AEGKV_DTYPE_BF16 && dtype != AEGKV_DTYPE_FP16) || n_q_heads / n_kv_heads > 16)
    return AEGKV_ERR_UNSUPPORTED;
  if (batch == 0) return 0;
  const int32_t chunk = std::min(batch, kMaxBatch);
  int n_wg = 0;
  const int rc = workgroups_for(n_workgroups, &n_wg);
  if (rc) return rc > 0 ? AEGKV_ERR_RUNTIME : rc;
  const int32_t group = n_q_heads / n_kv_heads;
  const int32_t n_groups = (n_kv_heads + kHeadsPerGroup - 1) / kHeadsPerGroup;
  if (!positions_fit(chunk, ((int64_t)max_seq_len + kBlockSize - 1) / kBlockSize, n_groups, n_wg))
    return AEGKV_ERR_UNSUPPORTED;
  return workspace_layout(chunk, kHeadsPerGroup * group, head_dim, n_wg, n_groups).total;
}


int aegkv_paged_decode_attention(void* out, int64_t out_batch_stride, const void* q,
                                 int64_t q_batch_stride, const void* key_cache,
                                 const void* value_cache, int64_t cache_block_stride,
                                 int64_t n_blocks, const int32_t* block_tables,
                                 int32_t max_blocks, const int32_t* seq_lens, int32_t batch,
                                 int32_t max_seq_len, int32_t n_q_heads, int32_t n_kv_heads,
                                 int32_t head_dim, int32_t block_size, float scale,
                                 int32_t dtype, int32_t n_workgroups, void* workspace,
                                 uint64_t workspace_bytes, aegkv_stream_t stream) {
  if (batch > 0 && !block_tables) return AEGKV_ERR_INVALID_ARG;
  return run_attention(out, out_batch_stride, q, q_batch_stride, key_cache, value_cache,
                       cache_block_stride, n_blocks, block_tables, max_blocks, nullptr, 0,
                       seq_lens, batch, max_seq_len, n_q_heads, n_kv_heads, head_dim,
                       block_size, scale, dtype, n_workgroups, workspace, workspace_bytes,
                       stream);
}

int aegkv_paged_decode_attention_append(
    void* out, int64_t out_batch_stride, const void* q, int64_t q_batch_stride, const void* key,
    int64_t key_batch_stride, const void* value, int64_t value_batch_stride, void* key_cache,
    void* value_cache, int64_t cache_block_stride, int64_t n_blocks, const int32_t* block_tables,
    int32_t max_blocks, const int32_t* seq_lens, int32_t batch, int32_t max_seq_len,
    int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim, int32_t block_size, float scale,
    int32_t dtype, int32_t n_workgroups, void* workspace, uint64_t workspace_bytes,
    aegkv_stream_t stream) {
  if (batch > 0 && (!block_tables || !key || !value)) return AEGKV_ERR_INVALID_ARG;
  NewRows nr;
  nr.key = key;
  nr.key_bstride = key_batch_stride;
  nr.value = value;
  nr.value_bstride = value_batch_stride;
  return run_attention(out, out_batch_stride, q, q_batch_stride, key_cache, value_cache,
                       cache_block_stride, n_blocks, block_tables, max_blocks, nullptr, 0,
                       seq_lens, batch, max_seq_len, n_q_heads, n_kv_heads, head_dim,
                       block_size, scale, dtype, n_workgroups, workspace, workspace_bytes,
                       stream, nr);
}

int aegkv_paged_decode_attention_append_planned(
    void* out, int64_t out_batch_stride, const void* q, int64_t q_batch_stride, const void* key,
    int64_t key_batch_stride, const void* value, int64_t value_batch_stride, void* key_cache,
    void* value_cache, int64_t cache_block_stride, int64_t n_blocks, const void* plan,
    uint64_t plan_bytes, const int32_t* seq_lens, int32_t batch, int32_t max_seq_len,
    int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim, int32_t block_size, float scale,
    int32_t dtype, int32_t n_workgroups, void* workspace, uint64_t workspace_bytes,
    aegkv_stream_t stream) {
  if (batch > 0 && (!plan || !key || !value)) return AEGKV_ERR_INVALID_ARG;
  NewRows nr;
  nr.key = key;
  nr.key_bstride = key_batch_stride;
  nr.value = value;
  nr.value_bstride = value_batch_stride;
  return run_attention(out, out_batch_stride, q, q_batch_stride, key_cache, value_cache,
                       cache_block_stride, n_blocks, nullptr, 0, plan, plan_bytes, seq_lens,
                       batch, max_seq_len, n_q_heads, n_kv_heads, head_dim, block_size, scale,
                       dtype, n_workgroups, workspace, workspace_bytes, stream, nr);
}

int64_t aegkv_paged_decode_plan_size(int32_t batch, int32_t n_kv_heads, int32_t max_seq_len,
                                     int32_t n_workgroups) {
  if (batch < 0 || n_kv_heads <= 0 || max_seq_len < 0 || n_workgroups < 0)
    return AEGKV_ERR_INVALID_ARG;
  if (batch > kMaxBatch || n_workgroups > kMaxWorkgroups) return AEGKV_ERR_UNSUPPORTED;
  if (batch == 0) return 0;
  int n_wg = 0;
  const int rc = workgroups_for(n_workgroups, &n_wg);
  if (rc) return rc > 0 ? AEGKV_ERR_RUNTIME : rc;
  const int64_t nblk_max = ((int64_t)max_seq_len + kBlockSize - 1) / kBlockSize;
  const int32_t n_groups = (n_kv_heads + kHeadsPerGroup - 1) / kHeadsPerGroup;
  if (!positions_fit(batch, nblk_max, n_groups, n_wg)) return AEGKV_ERR_UNSUPPORTED;
  return plan_layout(batch, n_wg, nblk_max).total;
}

int aegkv_paged_decode_plan(const int32_t* block_tables, int32_t max_blocks,
                            const int32_t* seq_lens, int32_t batch, int32_t max_seq_len,
                            int32_t n_kv_heads, int32_t n_workgroups, void* plan,
                            uint64_t plan_bytes, aegkv_stream_t stream) {
  const int64_t need = aegkv_paged_decode_plan_size(batch, n_kv_heads, max_seq_len, n_workgroups);
  if (need < 0) return (int)need;
  if (batch == 0) return AEGKV_OK;
  if (!block_tables || !seq_lens || !plan || max_blocks < 0) return AEGKV_ERR_INVALID_ARG;
  const int64_t nblk_max = ((int64_t)max_seq_len + kBlockSize - 1) / kBlockSize;
  if (nblk_max > max_blocks) return AEGKV_ERR_INVALID_ARG;
  if (plan_bytes < (uint64_t)need) return AEGKV_ERR_INVALID_ARG;
  if (!aligned16(plan)) return AEGKV_ERR_MISALIGNED;
  int n_wg = 0;
  int rc = workgroups_for(n_workgroups, &n_wg);
  if (rc) return rc;
  const PlanLayout pl = plan_layout(batch, n_wg, nblk_max);
  uint8_t* pb = static_cast<uint8_t*>(plan);
  PlanArgs p;
  p.block_tables = block_tables;
  p.max_blocks = max_blocks;
  p.seq_lens = seq_lens;
  p.batch = batch;
  p.max_seq_len = max_seq_len;
  p.n_groups = (n_kv_heads + kHeadsPerGroup - 1) / kHeadsPerGroup;
  p.n_wg = n_wg;
  p.desc_per_seq = desc_per_sequence(batch, p.n_groups, n_wg) ? 1 : 0;
  p.wg = reinterpret_cast<int32_t*>(pb + pl.wg);
  p.desc = reinterpret_cast<int4*>(pb + pl.desc);
  p.first = reinterpret_cast<int32_t*>(pb + pl.first);
  p.last = reinterpret_cast<int32_t*>(pb + pl.last);
  p.ids = reinterpret_cast<int32_t*>(pb + pl.ids);
  p.tags = reinterpret_cast<int32_t*>(pb + pl.tags);
  const int64_t work = std::max<int64_t>(std::max<int64_t>((int64_t)n_wg * 64, (int64_t)batch * nblk_max),
                                         (int64_t)batch * p.n_groups);
  const int grid = (int)std::max<int64_t>(1, std::min<int64_t>(1024, (work + 255) / 256));
  hipLaunchKernelGGL(decode_plan_kernel, dim3(grid), dim3(64 * kHeadsPerGroup),
                     (size_t)(3 * batch + 2) * sizeof(int32_t), (hipStream_t)stream, p);
  AEGKV_HIP_TRY(hipGetLastError());
  return AEGKV_OK;
}

int aegkv_paged_decode_attention_planned(void* out, int64_t out_batch_stride, const void* q,
                                         int64_t q_batch_stride, const void* key_cache,
                                         const void* value_cache, int64_t cache_block_stride,
                                         int64_t n_blocks, const void* plan, uint64_t plan_bytes,
                                         const int32_t* seq_lens, int32_t batch,
                                         int32_t max_seq_len, int32_t n_q_heads,
                                         int32_t n_kv_heads, int32_t head_dim,
                                         int32_t block_size, float scale, int32_t dtype,
                                         int32_t n_workgroups, void* workspace,
                                         uint64_t workspace_bytes, aegkv_stream_t stream) {
  if (batch > 0 && !plan) return AEGKV_ERR_INVALID_ARG;
  return run_attention(out, out_batch_stride, q, q_batch_stride, key_cache, value_cache,
                       cache_block_stride, n_blocks, nullptr, 0, plan, plan_bytes, seq_lens,
                       batch, max_seq_len, n_q_heads, n_kv_heads, head_dim, block_size, scale,
                       dtype, n_workgroups, workspace, workspace_bytes, stream);
}

}  // extern "C"
