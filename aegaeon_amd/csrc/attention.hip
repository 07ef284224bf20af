// Paged GQA decode attention for gfx950 (replaces vllm-flash-attn's
// flash_attn_with_kvcache on the decode path, selected at
// aegaeon/aegaeon/worker.py:410-418 and run inside the forward at :517-523).
//
// Work item = one wave64 per (KV split, kv head, sequence).  All G = Hq/Hkv
// query heads of the kv head are processed together, so each K/V byte is read
// from HBM exactly once per decode step.
//
// Per 16-token block (block_size 16):
//   S^T[16 tok x 16 heads] = K[16 x D] . Q^T[D x 16]   -> D/32 MFMA 16x16x32 (bf16/fp16)
//     lane l loads K row (l%16), 8 dims per k-step: one dwordx4 per step.
//   online softmax in fp32 (exp2 domain); each lane owns head l%16 and tokens
//     4*(l/16)+r, r<4; the block max/sum reduce over the 4 lane groups.
//   O^T[D x 16 heads] += V^T[D x 16 tok] . P^T[16 tok x 16 heads]
//     -> D/16 x 4 MFMA 16x16x4 in fp32 (P stays fp32: a bf16 P alone costs
//     ~1e-3 relative error, half of the 2e-3 budget);
//     lane l loads V row 4*(l/16)+c, dims [D/16*(l%16), +D/16): one contiguous
//     chunk per c, and the PV tiles take its elements in order, so output
//     dim = (D/16)*m + tile.
// G < 16 leaves MFMA columns idle; the kernel is HBM-bound (7 FLOP/byte at
// G = 7), and the MFMA pipe runs beside the vector loads.
// Splits longer than one work item write fp32 partials (unnormalised O, max,
// sum) that a second kernel merges with log-sum-exp weights.
#include <algorithm>
#include <cmath>

#include "aegkv_internal.h"

namespace aegkv {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

constexpr int kBlockSize = 16;
constexpr int kDefaultBlocksPerSplit = 8;

template <int DT>
struct Elem;

template <>
struct Elem<AEGKV_DTYPE_BF16> {
  static __device__ __forceinline__ f32x4 mfma_qk(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  // element 0 of a packed pair sits in the low half-word (little endian)
  static __device__ __forceinline__ float lo(uint32_t w) { return __uint_as_float(w << 16); }
  static __device__ __forceinline__ float hi(uint32_t w) {
    return __uint_as_float(w & 0xffff0000u);
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
  static __device__ __forceinline__ f32x4 mfma_qk(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ float lo(uint32_t w) {
    return (float)__builtin_bit_cast(_Float16, (unsigned short)(w & 0xffffu));
  }
  static __device__ __forceinline__ float hi(uint32_t w) {
    return (float)__builtin_bit_cast(_Float16, (unsigned short)(w >> 16));
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

template <int DT, int D>
__global__ __launch_bounds__(64) void paged_decode_attention_kernel(AttnArgs a) {
  using E = Elem<DT>;
  constexpr int KS = D / 32;   // QK k-steps of 32 dims
  constexpr int DPL = D / 16;  // dims per lane in the PV layout = PV tiles
  constexpr int VW = DPL / 2;  // 32-bit words per lane per V row
  const int lane = threadIdx.x;
  const int j = lane & 15, g = lane >> 4;
  const int s = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int len = min(max(a.seq_lens[b], 0), a.max_seq_len);
  const int nblk = len > 0 ? (len + kBlockSize - 1) / kBlockSize : 0;
  const int blk0 = s * a.bps;
  if (s > 0 && blk0 >= nblk) return;
  const int blk1 = min(nblk, blk0 + a.bps);
  const int nsplit = nblk > 0 ? (nblk + a.bps - 1) / a.bps : 1;
  const bool head_ok = j < a.group;
  const int hq = h * a.group + j;

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

  const int32_t* bt = a.block_tables + (int64_t)b * a.max_blocks;
  const int64_t row = (int64_t)a.n_kv_heads * D;
  const uint16_t* kh = a.kc + (int64_t)h * D + (int64_t)j * row + 8 * g;
  const uint16_t* vh = a.vc + (int64_t)h * D + (int64_t)(4 * g) * row + DPL * j;

  u32x4 kr[KS];
  uint32_t vr[4][VW];
  int id = blk0 < blk1 ? bt[blk0] : -1;
  bool ok = id >= 0 && id < a.n_blocks;
  if (ok) {
    const int64_t off = (int64_t)id * a.blk_stride;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) kr[ks] = *reinterpret_cast<const u32x4*>(kh + off + 32 * ks);
#pragma unroll
    for (int c = 0; c < 4; ++c) load_words<VW>(vh + off + c * row, vr[c]);
  }

  for (int ib = blk0; ib < blk1; ++ib) {
    // prefetch the next block while this one is computed
    u32x4 kn[KS];
    uint32_t vn[4][VW];
    const int nid = ib + 1 < blk1 ? bt[ib + 1] : -1;
    const bool nok = nid >= 0 && nid < a.n_blocks;
    if (nok) {
      const int64_t off = (int64_t)nid * a.blk_stride;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
        kn[ks] = *reinterpret_cast<const u32x4*>(kh + off + 32 * ks);
#pragma unroll
      for (int c = 0; c < 4; ++c) load_words<VW>(vh + off + c * row, vn[c]);
    }

    if (ok) {
      f32x4 sc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) sc = E::mfma_qk(kr[ks], qv[ks], sc);
      const int tb = ib * kBlockSize + 4 * g;  // token of sc[0] in this lane
      float x[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) x[r] = (tb + r < len) ? sc[r] * a.scale_log2 : -INFINITY;
      float bm = fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3]));
      bm = fmaxf(bm, __shfl_xor(bm, 16));
      bm = fmaxf(bm, __shfl_xor(bm, 32));
      const float mn = fmaxf(m, bm);  // finite: token ib*16 is always valid
      const float alpha = __builtin_amdgcn_exp2f(m - mn);
      float p[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) p[r] = __builtin_amdgcn_exp2f(x[r] - mn);
      lsum = lsum * alpha + ((p[0] + p[1]) + (p[2] + p[3]));
      m = mn;
#pragma unroll
      for (int t = 0; t < DPL; ++t) acc[t] *= alpha;
      if (ib * kBlockSize + kBlockSize > len) {
        // tail block: rows past the sequence end hold stale bytes (maybe NaN)
#pragma unroll
        for (int c = 0; c < 4; ++c)
          if (tb + c >= len)
#pragma unroll
            for (int w = 0; w < VW; ++w) vr[c][w] = 0u;
      }
#pragma unroll
      for (int c = 0; c < 4; ++c) {
#pragma unroll
        for (int t = 0; t < DPL; ++t) {
          const uint32_t w = vr[c][t >> 1];
          const float v = (t & 1) ? E::hi(w) : E::lo(w);
          acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(v, p[c], acc[t], 0, 0, 0);
        }
      }
    }

    ok = nok;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) kr[ks] = kn[ks];
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
      for (int w = 0; w < VW; ++w) vr[c][w] = vn[c][w];
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

// Merge split partials: out = sum_s w_s o_s / sum_s w_s l_s, w_s = 2^(m_s - max m).
template <int DT, int D>
__global__ __launch_bounds__(64) void attention_combine_kernel(AttnArgs a) {
  using E = Elem<DT>;
  constexpr int DPT = D / 64;  // dims per thread
  const int hq = blockIdx.x, b = blockIdx.y;
  const int len = min(max(a.seq_lens[b], 0), a.max_seq_len);
  const int nblk = len > 0 ? (len + kBlockSize - 1) / kBlockSize : 0;
  const int nsplit = nblk > 0 ? (nblk + a.bps - 1) / a.bps : 1;
  if (nsplit <= 1) return;
  const int64_t base = ((int64_t)b * a.n_q_heads + hq) * a.max_splits;
  float mx = -INFINITY;
  for (int s = 0; s < nsplit; ++s) mx = fmaxf(mx, a.part_ml[base + s].x);
  float o[DPT];
#pragma unroll
  for (int i = 0; i < DPT; ++i) o[i] = 0.f;
  float l = 0.f;
  for (int s = 0; s < nsplit; ++s) {
    const float2 ml = a.part_ml[base + s];
    const float w = ml.x == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(ml.x - mx);
    l += w * ml.y;
    const float* po = a.part_o + (base + s) * D + threadIdx.x * DPT;
#pragma unroll
    for (int i = 0; i < DPT; ++i) o[i] += w * po[i];
  }
  const float inv = l > 0.f ? 1.f / l : 0.f;
  uint16_t* op = a.out + (int64_t)b * a.out_bstride + (int64_t)hq * D + threadIdx.x * DPT;
#pragma unroll
  for (int i = 0; i < DPT; ++i) op[i] = (uint16_t)E::bits(o[i] * inv);
}

template <int DT, int D>
int launch_attention(const AttnArgs& a, int batch, hipStream_t stream) {
  hipLaunchKernelGGL((paged_decode_attention_kernel<DT, D>),
                     dim3(a.max_splits, a.n_kv_heads, batch), dim3(64), 0, stream, a);
  AEGKV_HIP_TRY(hipGetLastError());
  if (a.max_splits > 1) {
    hipLaunchKernelGGL((attention_combine_kernel<DT, D>), dim3(a.n_q_heads, batch), dim3(64),
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
      block_size != kBlockSize)
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
      n_q_heads / n_kv_heads > 16 || (dtype != AEGKV_DTYPE_BF16 && dtype != AEGKV_DTYPE_FP16))
    return AEGKV_ERR_UNSUPPORTED;
  if (batch == 0) return AEGKV_OK;
  if (!out || !q || !key_cache || !value_cache || !block_tables || !seq_lens)
    return AEGKV_ERR_INVALID_ARG;
  if (!aligned16(out) || !aligned16(q) || !aligned16(key_cache) || !aligned16(value_cache) ||
      ((q_batch_stride * 2) & 15) || ((out_batch_stride * 2) & 15) ||
      ((cache_block_stride * 2) & 15))
    return AEGKV_ERR_MISALIGNED;
  if (batch > 65535 || n_kv_heads > 65535) return AEGKV_ERR_UNSUPPORTED;
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
