// Varlen prefill attention on gfx950: the prompt run of vLLM 0.5.1's
// FlashAttention backend, flash_attn_varlen_func(q, k, v, cu_seqlens,
// cu_seqlens, max_seqlen, max_seqlen, scale, causal=True) (EXT), reached from
// aegaeon/aegaeon/worker.py:517-523 with the metadata of worker.py:652-711.
//
// Layout: q [T, Hq, D], k and v [T, Hkv, D], out [T, Hq, D] in 16-bit
// elements, any token stride, the heads of a token contiguous.  Sequence b
// holds tokens [cu_seqlens[b], cu_seqlens[b+1]); query i of a sequence attends
// to keys j <= i of the same sequence (all of them when not causal).
//
// Work: a workgroup of four waves takes 128 queries of one head of one
// sequence; wave w owns queries [32w, 32w + 32).  The (sequence, query head)
// units, in that order (so the query heads of one kv head are neighbours), are
// split into kXcds contiguous runs, one per XCD: the hardware deals
// workgroup i to XCD i % kXcds, and workgroup i = s * kXcds + x takes the
// s-th job of XCD x's run.  Every query tile of a unit then runs on one XCD,
// whose L2 keeps that sequence's K and V for all of them (round-robin jobs
// put each kv head's 1 MiB of K/V of a 2048-token prompt in every XCD's L2,
// 16 MiB per 4 MiB L2 for 4 x 2048 tokens).  Within an XCD the jobs run with
// the query tile slowest, in decreasing order, so the most expensive tiles
// (the last of each sequence) are dispatched first; two fit on a CU.  (A
// persistent grid dealing the same jobs in snake order measured 5% slower on
// 4 x 2048 tokens and 60% slower on ragged batches, whose short sequences
// leave most high-tile jobs empty.)
//
// Per 64-key tile, staged in LDS by the whole workgroup (two stages):
//   S^T[64 keys x 32 queries] = K[64 x D] . Q^T[D x 32]   2 x D/16 MFMA 32x32x16
//     (A = K rows from LDS, B = the wave's queries, held in registers);
//   online softmax in fp32 in the exp2 domain: lane l holds query l & 31 and
//     16 of the 32 keys of a block (keys 8(i/4) + 4(l/32) + i%4 of
//     accumulator element i), its partner lane l ^ 32 the other 16;
//   O^T[D x 32] += V^T[D x 64] . P^T[64 x 32]             D/32 x 4 MFMA 32x32x16
//     with P rounded to 16 bits (as FlashAttention does) and taken straight
//     from the S^T accumulators: elements 8j .. 8j+7 of a lane are the keys of
//     k-step j, so V^T is stored in LDS with the 4-key quads of every 16 keys
//     in the order 0, 2, 1, 3, and each MFMA operand is one 16-byte LDS read.
// Lazy rescaling as in the decode kernel: the reference max moves only when a
// tile's max exceeds it by more than 8 (log2 units).
#include <algorithm>
#include <cmath>

#include "aegkv_internal.h"

namespace aegkv {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

constexpr int kPfThreads = 256;
constexpr int kXcds = 8;                     // XCDs of an MI355X (gfx950)
constexpr int kPfQTile = 128;                // queries per workgroup
constexpr int kPfKTile = 64;                 // keys per step
constexpr int kVtPitch = kPfKTile * 2 + 16;  // bytes per row of V^T in LDS
constexpr float kPfRescaleSlack = 8.f;

template <int DT>
struct PfOps;

template <>
struct PfOps<AEGKV_DTYPE_BF16> {
  static __device__ __forceinline__ f32x16 mfma(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  // two floats to two 16-bit values, round to nearest even (one instruction)
  static __device__ __forceinline__ uint32_t pack(float x, float y) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{x, y}, bf16x2));
  }
};

template <>
struct PfOps<AEGKV_DTYPE_FP16> {
  static __device__ __forceinline__ f32x16 mfma(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t pack(float x, float y) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{x, y}, f16x2));
  }
};

// max(a, b, c) in one instruction.  (fmaxf on values the compiler cannot
// prove canonical, such as MFMA results, costs a v_max_f32 x, x per operand
// first; the scores here are never signalling NaNs.)
__device__ __forceinline__ float max3(float a, float b, float c) {
  float r;
  __asm__("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}

// {lo16(a), lo16(b)} and {hi16(a), hi16(b)} (v_perm_b32: src1 = bytes 0-3)
__device__ __forceinline__ uint32_t pack_lo(uint32_t a, uint32_t b) {
  return __builtin_amdgcn_perm(b, a, 0x05040100u);
}
__device__ __forceinline__ uint32_t pack_hi(uint32_t a, uint32_t b) {
  return __builtin_amdgcn_perm(b, a, 0x07060302u);
}

struct PrefillArgs {
  const uint8_t* q;
  const uint8_t* k;
  const uint8_t* v;
  uint8_t* out;
  int64_t q_tok_b, k_tok_b, v_tok_b, o_tok_b;  // byte strides per token
  const int32_t* cu_seqlens;                   // [batch + 1], device
  int64_t total_tokens;
  int32_t batch, n_q_heads, group, max_seqlen, n_qtiles, causal;
  int32_t n_units;                             // batch * n_q_heads
  float scale_log2;                            // softmax scale * log2(e), > 0
};

// Queries [q0, q0 + 128) of head h of the sequence at token s0 with len
// tokens.
template <int DT, int D>
__device__ __forceinline__ void attend_tile(const PrefillArgs& a, uint8_t* lds, int h, int64_t s0,
                                            int len, int q0) {
  using E = PfOps<DT>;
  constexpr int KPITCH = D * 2 + 16;            // bytes per K row in LDS
  constexpr int K_BYTES = kPfKTile * KPITCH;
  constexpr int V_BYTES = D * kVtPitch;
  constexpr int KS = D / 16;                    // k-steps of K.Q^T
  constexpr int DB = D / 32;                    // 32-row blocks of O^T
  constexpr int CPR = D / 8;                    // 16-byte chunks per row
  constexpr int KRPP = kPfThreads / CPR;        // K rows staged per pass
  constexpr int KPASS = kPfKTile / KRPP;
  constexpr int VTHREADS = (kPfKTile / 4) * CPR;  // (4-key quad, chunk) pairs
  const int kvh = h / a.group;
  const int kv_end = a.causal ? min(len, q0 + kPfQTile) : len;
  const int n_kt = (kv_end + kPfKTile - 1) / kPfKTile;

  const int t = threadIdx.x, lane = t & 63;
  const int w = __builtin_amdgcn_readfirstlane(t >> 6);  // uniform: the tile tests below branch
  const int col = lane & 31, hh = lane >> 5;
  const int qi = q0 + 32 * w + col;  // this lane's query, relative to the sequence
  const int wq0 = q0 + 32 * w;       // the wave's first query

  // Q^T operand: query qi, dims 16 ks + 8 hh .. +7 (rows past the end are 0)
  u32x4 qv[KS];
  {
    const uint8_t* qp =
        a.q + (s0 + min(qi, len - 1)) * a.q_tok_b + ((int64_t)h * D + 8 * hh) * 2;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      qv[ks] = qi < len ? *reinterpret_cast<const u32x4*>(qp + 32 * ks) : u32x4{0, 0, 0, 0};
  }

  // staging: K row kr + KRPP p, chunk kc; V keys 4 vq .. 4 vq + 3, chunk vc
  const uint8_t* kbase = a.k + s0 * a.k_tok_b + (int64_t)kvh * D * 2;
  const uint8_t* vbase = a.v + s0 * a.v_tok_b + (int64_t)kvh * D * 2;
  const int kc = t % CPR, kr = t / CPR;
  const int vq = t % (kPfKTile / 4), vc = t / (kPfKTile / 4);
  // position of the quad in the stored key order (quads 0, 2, 1, 3 of 16 keys)
  const int vpos = 16 * (vq >> 2) + 4 * (((vq & 1) << 1) | ((vq >> 1) & 1));
  const uint32_t koff = (uint32_t)(kr * a.k_tok_b) + kc * 16;
  const uint32_t voff = (uint32_t)(4 * vq * a.v_tok_b) + vc * 16;
  u32x4 kreg[KPASS], vreg[4];

  auto load_k = [&](int kt) {
    const int r0 = kt * kPfKTile;
    if (r0 + kPfKTile <= len) {  // whole tile inside the sequence (uniform)
      const uint8_t* kb = kbase + r0 * a.k_tok_b;
#pragma unroll
      for (int p = 0; p < KPASS; ++p)
        kreg[p] = *reinterpret_cast<const u32x4*>(kb + p * KRPP * a.k_tok_b + koff);
    } else {  // last tile: rows clamped to the sequence (masked in S)
#pragma unroll
      for (int p = 0; p < KPASS; ++p) {
        const int row = min(r0 + kr + KRPP * p, len - 1);
        kreg[p] = *reinterpret_cast<const u32x4*>(kbase + row * a.k_tok_b + kc * 16);
      }
    }
  };
  auto load_v = [&](int kt) {
    if (t >= VTHREADS) return;
    const int r0 = kt * kPfKTile;
    if (r0 + kPfKTile <= len) {
      const uint8_t* vb = vbase + r0 * a.v_tok_b;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        vreg[i] = *reinterpret_cast<const u32x4*>(vb + i * a.v_tok_b + voff);
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = min(r0 + 4 * vq + i, len - 1);
        vreg[i] = *reinterpret_cast<const u32x4*>(vbase + row * a.v_tok_b + vc * 16);
      }
    }
  };
  auto store_k = [&](int slot) {
    uint8_t* st = lds + slot * K_BYTES;
#pragma unroll
    for (int p = 0; p < KPASS; ++p)
      *reinterpret_cast<u32x4*>(st + (kr + KRPP * p) * KPITCH + kc * 16) = kreg[p];
  };
  auto store_v = [&](int kt, int slot) {
    if (t >= VTHREADS) return;
    if (kt * kPfKTile + kPfKTile > len) {  // last tile only (uniform)
#pragma unroll
      for (int i = 0; i < 4; ++i)  // keys past the end: 0 (P is 0 there, V may be NaN)
        if (kt * kPfKTile + 4 * vq + i >= len) vreg[i] = u32x4{0, 0, 0, 0};
    }
    const u32x4* x = vreg;
    uint8_t* vt = lds + 2 * K_BYTES + slot * V_BYTES + vpos * 2;
#pragma unroll
    for (int wd = 0; wd < 4; ++wd) {  // dims 2 wd (low halves) and 2 wd + 1 (high)
      *reinterpret_cast<u32x2*>(vt + (8 * vc + 2 * wd) * kVtPitch) =
          u32x2{pack_lo(x[0][wd], x[1][wd]), pack_lo(x[2][wd], x[3][wd])};
      *reinterpret_cast<u32x2*>(vt + (8 * vc + 2 * wd + 1) * kVtPitch) =
          u32x2{pack_hi(x[0][wd], x[1][wd]), pack_hi(x[2][wd], x[3][wd])};
    }
  };

  // S^T of tile kt (K stage kt & 1); the two 32-key blocks alternate so that
  // neighbouring MFMAs are independent
  auto qk = [&](int kt, f32x16 (&s)[2]) {
    const uint8_t* kp = lds + (kt & 1) * K_BYTES + col * KPITCH + 16 * hh;
#pragma unroll
    for (int sb = 0; sb < 2; ++sb)
#pragma unroll
      for (int i = 0; i < 16; ++i) s[sb][i] = 0.f;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
      for (int sb = 0; sb < 2; ++sb)
        s[sb] = E::mfma(*reinterpret_cast<const u32x4*>(kp + 32 * sb * KPITCH + 32 * ks),
                        qv[ks], s[sb]);
  };
  // -inf where a key is past the end or (causal) after the query; only the
  // tiles that reach past the wave's first query or the end need it
  auto mask = [&](int kt, f32x16 (&s)[2]) {
    const int k0 = kt * kPfKTile;
    if ((a.causal && k0 + kPfKTile - 1 > wq0) || k0 + kPfKTile > len) {
#pragma unroll
      for (int sb = 0; sb < 2; ++sb)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int kv = k0 + 32 * sb + 8 * (i >> 2) + 4 * hh + (i & 3);
          const bool ok = kv < len && (!a.causal || kv <= qi);
          s[sb][i] = ok ? s[sb][i] : -INFINITY;
        }
    }
  };

  f32x16 o[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int i = 0; i < 16; ++i) o[db][i] = 0.f;
  float m = -INFINITY, lsum = 0.f;

  // softmax of a masked S^T tile and O^T += V^T . P^T (V stage kt & 1)
  auto softmax_pv = [&](int kt, f32x16 (&s)[2]) {
    float bm = max3(s[0][0], s[0][1], s[0][2]);  // raw-score max (the scale is positive)
#pragma unroll
    for (int i = 3; i < 31; i += 2) {
      const int sb = i >> 4, e = i & 15;
      bm = max3(bm, s[sb][e], s[(i + 1) >> 4][(i + 1) & 15]);
    }
    bm = max3(bm, s[1][15], s[1][15]);  // all 32 of this lane's scores
    const float pm = __shfl_xor(bm, 32);  // the partner lane's (same query)
    bm = max3(bm, pm, pm) * a.scale_log2;
    if (__builtin_amdgcn_ballot_w64(bm > m + kPfRescaleSlack)) {
      const float mn = fmaxf(m, bm);
      const float alpha = __builtin_amdgcn_exp2f(m - mn);  // 0 while m = -inf
      lsum *= alpha;
#pragma unroll
      for (int db = 0; db < DB; ++db) o[db] *= alpha;
      m = mn;
    }
    const float nms = m == -INFINITY ? 0.f : -m;
    u32x4 pb[4];  // P^T operands of the four 16-key steps
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const int sb = kk >> 1, base = 8 * (kk & 1);
      uint32_t pw[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float p0 =
            __builtin_amdgcn_exp2f(__builtin_fmaf(s[sb][base + 2 * j], a.scale_log2, nms));
        const float p1 =
            __builtin_amdgcn_exp2f(__builtin_fmaf(s[sb][base + 2 * j + 1], a.scale_log2, nms));
        lsum += p0 + p1;
        pw[j] = E::pack(p0, p1);
      }
      pb[kk] = u32x4{pw[0], pw[1], pw[2], pw[3]};
    }
    const uint8_t* vp = lds + 2 * K_BYTES + (kt & 1) * V_BYTES + col * kVtPitch + 16 * hh;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
#pragma unroll
      for (int db = 0; db < DB; ++db)
        o[db] = E::mfma(*reinterpret_cast<const u32x4*>(vp + 32 * db * kVtPitch + 32 * kk),
                        pb[kk], o[db]);
  };

  // K and V of tile kt + 1 are loaded while tile kt is computed.  Two
  // workgroups per CU overlap each other's softmax and matrix work; issuing
  // the next tile's S^T before the softmax inside the wave (a one-tile
  // pipeline) measured 1.8x slower, as its second S^T buffer leaves room for
  // one workgroup per CU only.
  load_k(0);
  load_v(0);
  store_k(0);
  store_v(0, 0);
  __syncthreads();
  for (int kt = 0; kt < n_kt; ++kt) {
    const bool more = kt + 1 < n_kt;
    if (more) {
      load_k(kt + 1);
      load_v(kt + 1);
    }
    f32x16 sc[2];
    if (!a.causal || kt * kPfKTile <= wq0 + 31) {
      qk(kt, sc);
      mask(kt, sc);
      softmax_pv(kt, sc);
    }
    if (more) {
      store_k((kt + 1) & 1);
      store_v(kt + 1, (kt + 1) & 1);
    }
    __syncthreads();
  }

  const float lt = lsum + __shfl_xor(lsum, 32);
  if (qi < len) {
    const float inv = 1.f / lt;
    uint8_t* op = a.out + (s0 + qi) * a.o_tok_b + ((int64_t)h * D + 4 * hh) * 2;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const f32x16& r = o[db];
        *reinterpret_cast<u32x2*>(op + (32 * db + 8 * g) * 2) =
            u32x2{E::pack(r[4 * g] * inv, r[4 * g + 1] * inv),
                  E::pack(r[4 * g + 2] * inv, r[4 * g + 3] * inv)};
      }
  }
}

template <int DT, int D>
__global__ __launch_bounds__(kPfThreads, 2) void prefill_attention_kernel(PrefillArgs a) {
  constexpr int K_BYTES = kPfKTile * (D * 2 + 16);
  constexpr int V_BYTES = D * kVtPitch;
  // two K stages, then two V^T stages
  __shared__ __align__(16) uint8_t lds[2 * K_BYTES + 2 * V_BYTES];
  // XCD x's run of units [u0, u1); its s-th job: tile n_qtiles-1 - s / c,
  // unit u0 + s % c (all uniform over the workgroup)
  const int x = (int)(blockIdx.x % kXcds), sj = (int)(blockIdx.x / kXcds);
  const int u0 = (int)((int64_t)a.n_units * x / kXcds);
  const int c = (int)((int64_t)a.n_units * (x + 1) / kXcds) - u0;
  if (c == 0 || sj >= a.n_qtiles * c) return;
  const int tile = a.n_qtiles - 1 - sj / c;
  const int unit = u0 + sj % c;
  const int b = unit / a.n_q_heads;
  const int h = unit % a.n_q_heads;
  int64_t s0 = a.cu_seqlens[b], s1 = a.cu_seqlens[b + 1];
  s0 = min(max(s0, (int64_t)0), a.total_tokens);
  s1 = min(max(s1, s0), a.total_tokens);
  const int len = (int)min(s1 - s0, (int64_t)a.max_seqlen);
  const int q0 = tile * kPfQTile;
  if (q0 >= len) return;  // uniform over the workgroup, before any barrier
  attend_tile<DT, D>(a, lds, h, s0, len, q0);
}

template <int DT, int D>
void launch_prefill(const PrefillArgs& a, uint32_t grid, hipStream_t stream) {
  hipLaunchKernelGGL((prefill_attention_kernel<DT, D>), dim3(grid), dim3(kPfThreads), 0, stream,
                     a);
}

}  // namespace
}  // namespace aegkv

using namespace aegkv;

extern "C" {

int aegkv_varlen_prefill_attention(void* out, int64_t out_token_stride, const void* q,
                                   int64_t q_token_stride, const void* k, int64_t k_token_stride,
                                   const void* v, int64_t v_token_stride,
                                   const int32_t* cu_seqlens, int32_t batch, int32_t max_seqlen,
                                   int64_t total_tokens, int32_t n_q_heads, int32_t n_kv_heads,
                                   int32_t head_dim, float scale, int32_t causal, int32_t dtype,
                                   aegkv_stream_t stream_) {
  hipStream_t stream = (hipStream_t)stream_;
  if (batch < 0 || max_seqlen < 0 || total_tokens < 0 || n_q_heads <= 0 || n_kv_heads <= 0)
    return AEGKV_ERR_INVALID_ARG;
  if (n_q_heads % n_kv_heads != 0) return AEGKV_ERR_INVALID_ARG;
  if (dtype != AEGKV_DTYPE_BF16 && dtype != AEGKV_DTYPE_FP16) return AEGKV_ERR_UNSUPPORTED;
  if (head_dim != 64 && head_dim != 128) return AEGKV_ERR_UNSUPPORTED;
  if (!std::isfinite(scale)) return AEGKV_ERR_INVALID_ARG;
  if (batch == 0 || max_seqlen == 0 || total_tokens == 0) return AEGKV_OK;
  if (!out || !q || !k || !v || !cu_seqlens) return AEGKV_ERR_INVALID_ARG;
  if (q_token_stride < (int64_t)n_q_heads * head_dim ||
      out_token_stride < (int64_t)n_q_heads * head_dim ||
      k_token_stride < (int64_t)n_kv_heads * head_dim ||
      v_token_stride < (int64_t)n_kv_heads * head_dim)
    return AEGKV_ERR_INVALID_ARG;
  if (!aligned16(out) || !aligned16(q) || !aligned16(k) || !aligned16(v) ||
      q_token_stride % 8 || k_token_stride % 8 || v_token_stride % 8 || out_token_stride % 8)
    return AEGKV_ERR_MISALIGNED;
  const int64_t n_qtiles = ((int64_t)max_seqlen + kPfQTile - 1) / kPfQTile;
  const int64_t n_units = (int64_t)n_q_heads * batch;
  // kXcds runs of at most ceil(n_units / kXcds) units each
  const int64_t grid = kXcds * n_qtiles * ((n_units + kXcds - 1) / kXcds);
  if (grid > INT32_MAX || n_units * n_qtiles > INT32_MAX) return AEGKV_ERR_UNSUPPORTED;

  PrefillArgs a;
  a.q = static_cast<const uint8_t*>(q);
  a.k = static_cast<const uint8_t*>(k);
  a.v = static_cast<const uint8_t*>(v);
  a.out = static_cast<uint8_t*>(out);
  a.q_tok_b = q_token_stride * 2;
  a.k_tok_b = k_token_stride * 2;
  a.v_tok_b = v_token_stride * 2;
  a.o_tok_b = out_token_stride * 2;
  a.cu_seqlens = cu_seqlens;
  a.total_tokens = total_tokens;
  a.batch = batch;
  a.n_q_heads = n_q_heads;
  a.group = n_q_heads / n_kv_heads;
  a.max_seqlen = max_seqlen;
  a.n_qtiles = (int32_t)n_qtiles;
  a.n_units = (int32_t)n_units;
  a.causal = causal ? 1 : 0;
  a.scale_log2 = scale * 1.4426950408889634f;
  const uint32_t g = (uint32_t)grid;
  if (dtype == AEGKV_DTYPE_BF16) {
    if (head_dim == 64) launch_prefill<AEGKV_DTYPE_BF16, 64>(a, g, stream);
    else launch_prefill<AEGKV_DTYPE_BF16, 128>(a, g, stream);
  } else {
    if (head_dim == 64) launch_prefill<AEGKV_DTYPE_FP16, 64>(a, g, stream);
    else launch_prefill<AEGKV_DTYPE_FP16, 128>(a, g, stream);
  }
  AEGKV_HIP_TRY(hipGetLastError());
  return AEGKV_OK;
}

}  // extern "C"
