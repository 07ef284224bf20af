// Paged GQA decode attention for gfx950 (replaces vllm-flash-attn's
// flash_attn_with_kvcache on the decode path, selected at
// aegaeon/aegaeon/worker.py:410-418 and run inside the forward at :517-523).
//
// Work item = one wave64 per (KV split, kv head, sequence); a 256-thread
// workgroup holds the 4 kv heads of one (split, sequence), so its waves stream
// the four adjacent 256-byte head slices of the same 1 KiB token rows.  All
// G = Hq/Hkv query heads of a kv head are processed together, so each K/V byte
// is read from HBM exactly once per decode step.
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
// The block ids of a wave's split are loaded once, one per lane, and read with
// readlane; K/V of the next block are in flight while the current one is
// computed.
// Sequences longer than one split write fp32 partials (unnormalised O, running
// max in log2 units, sum) that a second kernel merges with log-sum-exp weights.
#include <algorithm>
#include <cmath>
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
constexpr int kDefaultBlocksPerSplit = 16;
constexpr int kMaxBlocksPerSplit = 64;  // one block id per lane
constexpr int kHeadsPerGroup = 4;       // waves (kv heads) per workgroup
#ifndef AEGKV_ATTN_PIPELINE
#define AEGKV_ATTN_PIPELINE 4
#endif
constexpr int kPipeline = AEGKV_ATTN_PIPELINE;  // K/V register buffers per wave
constexpr float kRescaleSlack = 8.f;  // log2 headroom of the lazy softmax rescale
constexpr int kCombineUnroll = 4;     // splits per group loaded together by the combine

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
  int32_t n_q_heads;
  int32_t n_kv_heads;
  int32_t group;  // n_q_heads / n_kv_heads
  float scale_log2;  // softmax scale * log2(e)
  int32_t bps;       // blocks per split
  int32_t max_splits;
  int32_t max_seq_len;  // host bound; longer device lengths are clamped to it
  uint16_t* out;
  int64_t out_bstride;  // elements
  float* part_o;        // [batch][Hq][max_splits][D]
  float2* part_ml;      // [batch][Hq][max_splits] (running max in log2 units, sum)
};

template <int NW>
__device__ __forceinline__ void load_words(const uint16_t* p, uint32_t* w) {
  if constexpr (NW == 2) {
    u32x2 v = *reinterpret_cast<const u32x2*>(p);
    w[0] = v.x; w[1] = v.y;
  } else {
#pragma unroll
    for (int i = 0; i < NW / 4; ++i) {
      u32x4 v = *reinterpret_cast<const u32x4*>(p + 8 * i);
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

template <int D>
__device__ __forceinline__ void load_block(KVRegs<D>& r, const uint16_t* kh, const uint16_t* vh,
                                           int64_t off, int64_t row) {
#pragma unroll
  for (int ks = 0; ks < KVRegs<D>::KS; ++ks)
    r.k[ks] = *reinterpret_cast<const u32x4*>(kh + off + 32 * ks);
#pragma unroll
  for (int c = 0; c < 4; ++c) load_words<KVRegs<D>::VW>(vh + off + c * row, r.v[c]);
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

template <int DT, int D, int NBUF>
__global__ __launch_bounds__(64 * kHeadsPerGroup) void paged_decode_attention_kernel(AttnArgs a) {
  using E = Elem<DT>;
  constexpr int KS = D / 32;
  constexpr int DPL = D / 16;
  constexpr int VW = D / 32;
  const int lane = threadIdx.x & 63;
  const int h = blockIdx.y * kHeadsPerGroup + (threadIdx.x >> 6);
  if (h >= a.n_kv_heads) return;  // whole waves; the kernel has no barrier
  const int j = lane & 15, g = lane >> 4;
  // Sequence-major grid (split index fastest): the splits of a sequence are
  // dispatched together.  Measured on the Qwen2.5-7B batch, a split-major
  // order is 30-50% slower.
  const int s = blockIdx.x, b = blockIdx.z;
  const int len = min(max(a.seq_lens[b], 0), a.max_seq_len);
  const int nblk = len > 0 ? (len + kBlockSize - 1) / kBlockSize : 0;
  const int blk0 = s * a.bps;
  if (s > 0 && blk0 >= nblk) return;
  const int nb = max(0, min(nblk, blk0 + a.bps) - blk0);
  const int nsplit = nblk > 0 ? (nblk + a.bps - 1) / a.bps : 1;
  const bool head_ok = j < a.group;
  const int hq = h * a.group + j;

  // block ids of this split, one per lane; ids outside the pool become -1
  int my_id = -1;
  if (lane < nb) {
    const int id = a.block_tables[(int64_t)b * a.max_blocks + blk0 + lane];
    my_id = (id >= 0 && id < a.n_blocks) ? id : -1;
  }

  u32x4 qv[KS];
  {
    const uint16_t* qp = a.q + (int64_t)b * a.q_bstride + (int64_t)(head_ok ? hq : 0) * D;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      u32x4 v = *reinterpret_cast<const u32x4*>(qp + 32 * ks + 8 * g);
      qv[ks] = head_ok ? v : u32x4{0u, 0u, 0u, 0u};
    }
  }

  f32x4 acc[DPL];
#pragma unroll
  for (int t = 0; t < DPL; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, lsum = 0.f;

  const int64_t row = (int64_t)a.n_kv_heads * D;
  const uint16_t* kh = a.kc + (int64_t)h * D + (int64_t)j * row + 8 * g;
  const uint16_t* vh = a.vc + (int64_t)h * D + (int64_t)(4 * g) * row + DPL * j;

  // Batches of NBUF blocks: the loads of a whole batch are issued first, then
  // its blocks are computed in order, so the wait before block k covers only
  // its own loads and NBUF-1-k blocks stay in flight behind it.  No load is
  // pending across the loop's back edge (register buffers carried over it get
  // copied at the latch, and copying a register that is still loading waits
  // for it).  Every load is issued unconditionally: an unreadable id reads
  // block 0 and is masked, a slot past the split re-reads its last block (an
  // L2 hit) and is not computed.  The host guarantees n_blocks >= 1.
  const int last = nb - 1;
  for (int it = 0; it < nb; it += NBUF) {
    KVRegs<D> buf[NBUF];
    int ids[NBUF];
    unrolled_steps<NBUF>([&](auto kc) {
      constexpr int k = decltype(kc)::value;
      ids[k] = __builtin_amdgcn_readlane(my_id, min(it + k, last));
      load_block<D>(buf[k], kh, vh, (int64_t)max(ids[k], 0) * a.blk_stride, row);
      __builtin_amdgcn_sched_barrier(0);  // keep the blocks' loads in issue order
      return false;
    });
    unrolled_steps<NBUF>([&](auto kc) {
      constexpr int k = decltype(kc)::value;
      if (it + k >= nb) return true;
      compute_block<DT, D>(buf[k], qv, acc, m, lsum, (blk0 + it + k) * kBlockSize,
                           ids[k] >= 0 ? len : 0, g, a.scale_log2);
      return false;
    });
  }

  float lt = lsum + __shfl_xor(lsum, 16);
  lt += __shfl_xor(lt, 32);

  // lane holds head j, dims [4*DPL*g, 4*DPL*g + 4*DPL): dim offset DPL*r + t <- acc[t][r]
  const int d0 = 4 * DPL * g;
  if (nsplit == 1) {
    if (head_ok) {
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
    }
  } else {
    const int64_t pidx = ((int64_t)b * a.n_q_heads + hq) * a.max_splits + s;
    if (head_ok) {
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
}

// Merge split partials of one (sequence, query head):
//   out = sum_s w_s o_s / sum_s w_s l_s,  w_s = 2^(m_s - max m).
// 256 threads = NG split groups x (D/4) lanes of 4 dims.  Each group loads up
// to kCombineUnroll of its splits at once (independent loads, one memory
// latency per pass), merges them online, and the groups merge in LDS.
template <int DT, int D>
__global__ __launch_bounds__(256) void attention_combine_kernel(AttnArgs a) {
  using E = Elem<DT>;
  constexpr int LPS = D / 4;      // lanes per split row
  constexpr int NG = 256 / LPS;   // split groups
  constexpr int U = kCombineUnroll;
  __shared__ float s_m[NG], s_l[NG];
  __shared__ f32x4 s_o[NG][LPS];
  const int hq = blockIdx.x, b = blockIdx.y;
  const int len = min(max(a.seq_lens[b], 0), a.max_seq_len);
  const int nblk = len > 0 ? (len + kBlockSize - 1) / kBlockSize : 0;
  const int nsplit = nblk > 0 ? (nblk + a.bps - 1) / a.bps : 1;
  if (nsplit <= 1) return;  // uniform over the workgroup
  const int grp = threadIdx.x / LPS, ln = threadIdx.x % LPS;
  const int64_t base = ((int64_t)b * a.n_q_heads + hq) * a.max_splits;
  float m = -INFINITY, l = 0.f;
  f32x4 o = {0.f, 0.f, 0.f, 0.f};
  for (int s0 = grp; s0 < nsplit; s0 += NG * U) {
    float2 ml[U];
    f32x4 po[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int s = s0 + u * NG;
      ml[u] = make_float2(-INFINITY, 0.f);
      po[u] = f32x4{0.f, 0.f, 0.f, 0.f};
      if (s < nsplit) {
        ml[u] = a.part_ml[base + s];
        po[u] = *reinterpret_cast<const f32x4*>(a.part_o + (base + s) * D + 4 * ln);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (ml[u].x == -INFINITY) continue;  // absent, or a split with no readable block
      const float mn = fmaxf(m, ml[u].x);
      const float wa = __builtin_amdgcn_exp2f(m - mn), wb = __builtin_amdgcn_exp2f(ml[u].x - mn);
      o = o * wa + po[u] * wb;
      l = l * wa + ml[u].y * wb;
      m = mn;
    }
  }
  if (ln == 0) { s_m[grp] = m; s_l[grp] = l; }
  s_o[grp][ln] = o;
  __syncthreads();
  if (grp == 0) {
    float mx = -INFINITY;
#pragma unroll
    for (int k = 0; k < NG; ++k) mx = fmaxf(mx, s_m[k]);
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    float lt = 0.f;
#pragma unroll
    for (int k = 0; k < NG; ++k) {
      const float w = s_m[k] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(s_m[k] - mx);
      acc += s_o[k][ln] * w;
      lt += s_l[k] * w;
    }
    const float inv = lt > 0.f ? 1.f / lt : 0.f;
    uint16_t* op = a.out + (int64_t)b * a.out_bstride + (int64_t)hq * D + 4 * ln;
    *reinterpret_cast<u32x2*>(op) =
        u32x2{E::bits(acc[0] * inv) | (E::bits(acc[1] * inv) << 16),
              E::bits(acc[2] * inv) | (E::bits(acc[3] * inv) << 16)};
  }
}

template <int DT, int D>
int launch_attention(const AttnArgs& a, int batch, hipStream_t stream) {
  const int groups = (a.n_kv_heads + kHeadsPerGroup - 1) / kHeadsPerGroup;
  hipLaunchKernelGGL((paged_decode_attention_kernel<DT, D, kPipeline>),
                     dim3(a.max_splits, groups, batch), dim3(64 * kHeadsPerGroup), 0, stream, a);
  AEGKV_HIP_TRY(hipGetLastError());
  if (a.max_splits > 1) {
    hipLaunchKernelGGL((attention_combine_kernel<DT, D>), dim3(a.n_q_heads, batch), dim3(256),
                       0, stream, a);
    AEGKV_HIP_TRY(hipGetLastError());
  }
  return AEGKV_OK;
}

int max_splits_for(int32_t max_seq_len, int32_t bps) {
  const int nblk = (max_seq_len + kBlockSize - 1) / kBlockSize;
  return std::max(1, (nblk + bps - 1) / bps);
}

}  // namespace
}  // namespace aegkv

using namespace aegkv;

extern "C" {

int64_t aegkv_paged_decode_attention_workspace_size(int32_t batch, int32_t n_q_heads,
                                                     int32_t head_dim, int32_t max_seq_len,
                                                     int32_t block_size,
                                                     int32_t blocks_per_split) {
  if (batch < 0 || n_q_heads <= 0 || head_dim <= 0 || max_seq_len < 0 ||
      block_size != kBlockSize || blocks_per_split < 0 ||
      blocks_per_split > kMaxBlocksPerSplit)
    return AEGKV_ERR_INVALID_ARG;
  const int bps = blocks_per_split > 0 ? blocks_per_split : kDefaultBlocksPerSplit;
  const int64_t ms = max_splits_for(max_seq_len, bps);
  if (ms <= 1) return 0;
  const int64_t n = (int64_t)batch * n_q_heads * ms;
  return n * head_dim * (int64_t)sizeof(float) + n * (int64_t)sizeof(float2) + 256;
}

int aegkv_paged_decode_attention(void* out, int64_t out_batch_stride, const void* q,
                                 int64_t q_batch_stride, const void* key_cache,
                                 const void* value_cache, int64_t cache_block_stride,
                                 int64_t n_blocks, const int32_t* block_tables,
                                 int32_t max_blocks, const int32_t* seq_lens, int32_t batch,
                                 int32_t max_seq_len, int32_t n_q_heads, int32_t n_kv_heads,
                                 int32_t head_dim, int32_t block_size, float scale,
                                 int32_t dtype, int32_t blocks_per_split, void* workspace,
                                 uint64_t workspace_bytes, aegkv_stream_t stream) {
  if (batch < 0 || max_seq_len < 0 || n_q_heads <= 0 || n_kv_heads <= 0 || max_blocks < 0 ||
      n_blocks < 0 || blocks_per_split < 0)
    return AEGKV_ERR_INVALID_ARG;
  if (n_q_heads % n_kv_heads) return AEGKV_ERR_INVALID_ARG;
  if (block_size != kBlockSize || (head_dim != 64 && head_dim != 128 && head_dim != 256) ||
      n_q_heads / n_kv_heads > 16 || (dtype != AEGKV_DTYPE_BF16 && dtype != AEGKV_DTYPE_FP16) ||
      blocks_per_split > kMaxBlocksPerSplit)
    return AEGKV_ERR_UNSUPPORTED;
  if (batch == 0) return AEGKV_OK;
  if (!out || !q || !key_cache || !value_cache || !block_tables || !seq_lens || n_blocks == 0)
    return AEGKV_ERR_INVALID_ARG;
  if (!aligned16(out) || !aligned16(q) || !aligned16(key_cache) || !aligned16(value_cache) ||
      ((q_batch_stride * 2) & 15) || ((out_batch_stride * 2) & 15) ||
      ((cache_block_stride * 2) & 15))
    return AEGKV_ERR_MISALIGNED;
  if (batch > 65535 || n_kv_heads > 65535 * kHeadsPerGroup) return AEGKV_ERR_UNSUPPORTED;
  const int nblk_max = (max_seq_len + kBlockSize - 1) / kBlockSize;
  if (nblk_max > max_blocks) return AEGKV_ERR_INVALID_ARG;
  const int bps = blocks_per_split > 0 ? blocks_per_split : kDefaultBlocksPerSplit;
  const int ms = max_splits_for(max_seq_len, bps);
  if (ms > 65535) return AEGKV_ERR_UNSUPPORTED;
  AttnArgs a;
  a.q = static_cast<const uint16_t*>(q);
  a.q_bstride = q_batch_stride;
  a.kc = static_cast<const uint16_t*>(key_cache);
  a.vc = static_cast<const uint16_t*>(value_cache);
  a.blk_stride = cache_block_stride;
  a.n_blocks = n_blocks;
  a.block_tables = block_tables;
  a.max_blocks = max_blocks;
  a.seq_lens = seq_lens;
  a.n_q_heads = n_q_heads;
  a.n_kv_heads = n_kv_heads;
  a.group = n_q_heads / n_kv_heads;
  a.scale_log2 = scale * 1.4426950408889634f;
  a.bps = bps;
  a.max_splits = ms;
  a.max_seq_len = max_seq_len;
  a.out = static_cast<uint16_t*>(out);
  a.out_bstride = out_batch_stride;
  a.part_o = nullptr;
  a.part_ml = nullptr;
  if (ms > 1) {
    const int64_t need = aegkv_paged_decode_attention_workspace_size(
        batch, n_q_heads, head_dim, max_seq_len, block_size, bps);
    if (!workspace || workspace_bytes < (uint64_t)need) return AEGKV_ERR_WORKSPACE;
    if (!aligned16(workspace)) return AEGKV_ERR_MISALIGNED;
    const int64_t n = (int64_t)batch * n_q_heads * ms;
    a.part_o = static_cast<float*>(workspace);
    a.part_ml = reinterpret_cast<float2*>(static_cast<float*>(workspace) + n * head_dim);
  }
  hipStream_t st = (hipStream_t)stream;
  const bool bf = dtype == AEGKV_DTYPE_BF16;
  switch (head_dim) {
    case 64: return bf ? launch_attention<AEGKV_DTYPE_BF16, 64>(a, batch, st)
                       : launch_attention<AEGKV_DTYPE_FP16, 64>(a, batch, st);
    case 128: return bf ? launch_attention<AEGKV_DTYPE_BF16, 128>(a, batch, st)
                        : launch_attention<AEGKV_DTYPE_FP16, 128>(a, batch, st);
    default: return bf ? launch_attention<AEGKV_DTYPE_BF16, 256>(a, batch, st)
                       : launch_attention<AEGKV_DTYPE_FP16, 256>(a, batch, st);
  }
}

}  // extern "C"
