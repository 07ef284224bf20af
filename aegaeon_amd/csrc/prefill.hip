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
// Per 64-key tile and 32-query block of a wave:
//   S^T[64 keys x 32 queries] = K[64 x D] . Q^T[D x 32]   2 x D/16 MFMA 32x32x16
//     (A = K rows from LDS, B = the wave's queries, held in registers);
//   online softmax in fp32 in the exp2 domain: lane l holds query l & 31 and
//     16 of the 32 keys of a block (keys 8(i/4) + 4(l/32) + i%4 of
//     accumulator element i), its partner lane l ^ 32 the other 16;
//   O^T[D x 32] += V^T[D x 64] . P^T[64 x 32]             D/32 x 4 MFMA 32x32x16
//     with P rounded to 16 bits (as FlashAttention does) and taken straight
//     from the S^T accumulators: elements 8j .. 8j+7 of a lane are the keys of
//     k-step j, which are keys {4 hh .. 4 hh + 3, 8 + 4 hh .. 8 + 4 hh + 3} of
//     the step's 16 (hh = l / 32), so V^T's A operand holds those keys.
// Lazy rescaling as in the decode kernel: the reference max moves only when a
// tile's max exceeds it by more than 8 (log2 units).
//
// Two kernels share that arithmetic (their outputs are bit-identical); the
// host picks one by the batch's longest prompt:
//
// Long prompts (max_seqlen > kLongPrompt): ping-pong.  A workgroup of eight
// waves takes 256 queries of one head and fills a CU; waves w and w + 4 share
// a SIMD, and the two halves of the workgroup run opposite phases between
// workgroup barriers.  Per key tile j a wave runs a matrix phase (S_j and the
// previous tile's O += V_{j-1}^T . P_{j-1}, 32 MFMAs at D = 128) and then a
// softmax phase (the VALU work that turns S_j into P_j); waves 4-7 start one
// phase later than waves 0-3, so on every SIMD one wave feeds the matrix core
// while the other runs its softmax.  K and V go from HBM straight into LDS
// (buffer loads with the LDS bit, no registers), V untransposed, and the
// P.V operands are read with gfx950's transposing LDS reads.
//
// Short prompts: two workgroups of four waves per CU, each taking 128 queries;
// K and V are staged through registers (V transposed on the way into LDS) and
// the two workgroups overlap each other's softmax and matrix work unordered.
// (With short prompts the ping-pong workgroup's start-up and its larger
// causal diagonal cost more than the phase overlap gains: 8 x 1024 tokens
// 112.6 against 109.0 us, 16 x 512 90.1 against 78.5 us; from 2048 tokens on it
// is faster: 4 x 2048 cache-cold 174.0 against 181.0 us, 2 x 4096 269.5
// against 303.7 us, 1 x 8192 544.7 against 627.3 us.)
//
// Work order, both kernels: the (sequence, query head) units, in that order
// (so the query heads of one kv head are neighbours), are split into kXcds
// contiguous runs, one per XCD: the hardware deals workgroup i to XCD
// i % kXcds, and workgroup i = s * kXcds + x takes the s-th job of XCD x's
// run.  Every query tile of a unit then runs on one XCD, whose L2 keeps that
// sequence's K and V for all of them.  When the units do not divide evenly
// over the XCDs and each CU has several tiles to run, a unit's tiles are
// dealt as S interleaved slices instead (slices_per_unit), so every XCD
// holds the same number of slices.  A ragged batch (by the host bound) deals
// its units round-robin over the XCDs, so no XCD holds only the longest
// prompts.  Within an XCD the jobs run with the
// query tile slowest, in decreasing order, so the most expensive tiles (the
// last of each sequence) are dispatched first.  (A persistent grid dealing the
// same jobs in snake order measured 5% slower on 4 x 2048 tokens and 60%
// slower on ragged batches, whose short sequences leave most high-tile jobs
// empty.)
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
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
typedef __attribute__((address_space(3))) void lds_void;

constexpr int kXcds = 8;                     // XCDs of an MI355X (gfx950)
constexpr int kPfKTile = 64;                 // keys per step
constexpr float kPfRescaleSlack = 8.f;
constexpr int kLongPrompt = 1536;            // longer prompts take the ping-pong kernel
// short-prompt kernel: four waves, 128 queries, V^T staged transposed
constexpr int kShortThreads = 256;
constexpr int kShortQTile = 128;
constexpr int kVtPitch = kPfKTile * 2 + 16;  // bytes per row of V^T in LDS
// ping-pong kernel: eight waves, 256 queries
constexpr int kLongWaves = 8;
constexpr int kLongThreads = 64 * kLongWaves;
constexpr int kLongQTile = 32 * kLongWaves;

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

// max(a, b, c) through the compiler's own max, never inline asm.  The
// scores are MFMA results, and a VALU read of an MFMA result needs wait states
// that only the compiler's hazard tracking inserts: it does not see the
// operands of an inline-asm v_max3_f32.  That form read unfinished scores on
// unmasked key tiles whenever the matrix core ran late, which showed as
// run-to-run output differences (one ulp, in ~7% of rows) once the four-wave
// kernel's workgroups were dealt to CUs in another order.  The compiler's max
// costs a few canonicalising v_max_f32 (0-3% per call).
__device__ __forceinline__ float max3(float a, float b, float c) {
  return __builtin_fmaxf(__builtin_fmaxf(a, b), c);
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
  int32_t slices;                              // interleaved tile slices per unit
  int32_t interleave;                          // slices dealt round-robin over the XCDs
  float scale_log2;                            // softmax scale * log2(e), > 0
};

// The wave's state for its 32 queries: lane (col = l & 31, hh = l / 32) holds
// query q0 + col and, of the O^T accumulators, head dims 32 db + 8 g + 4 hh ..
// + 3 in element 4 g .. 4 g + 3 of o[db].
template <int DT, int D>
struct WaveState {
  static constexpr int KS = D / 16;  // k-steps of K.Q^T
  static constexpr int DB = D / 32;  // 32-row blocks of O^T
  u32x4 qv[KS];                      // Q^T operand: dims 16 ks + 8 hh .. +7
  f32x16 o[DB];
  float m, lsum;

  __device__ __forceinline__ void init(const PrefillArgs& a, int h, int64_t s0, int len, int qi,
                                       int hh) {
    const uint8_t* qp =
        a.q + (s0 + min(qi, len - 1)) * a.q_tok_b + ((int64_t)h * D + 8 * hh) * 2;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)  // queries past the end: 0
      qv[ks] = qi < len ? *reinterpret_cast<const u32x4*>(qp + 32 * ks) : u32x4{0, 0, 0, 0};
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int i = 0; i < 16; ++i) o[db][i] = 0.f;
    m = -INFINITY;
    lsum = 0.f;
  }

  // S^T of a 64-key tile from K rows at kp (pitch KPITCH bytes, this lane's
  // row and 16-byte column already added); the two 32-key blocks alternate so
  // that neighbouring MFMAs are independent.  `ahead` LDS reads are kept in
  // flight ahead of the MFMA that uses them.
  template <int KPITCH, int AHEAD>
  __device__ __forceinline__ void qk(const uint8_t* kp, f32x16 (&s)[2]) const {
#pragma unroll
    for (int sb = 0; sb < 2; ++sb)
#pragma unroll
      for (int i = 0; i < 16; ++i) s[sb][i] = 0.f;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
      for (int sb = 0; sb < 2; ++sb)
        s[sb] = PfOps<DT>::mfma(*reinterpret_cast<const u32x4*>(kp + 32 * sb * KPITCH + 32 * ks),
                                qv[ks], s[sb]);
    if (AHEAD > 0) {
      __builtin_amdgcn_sched_group_barrier(0x100, AHEAD, 0);  // LDS reads
#pragma unroll
      for (int i = 0; i < 2 * KS - AHEAD; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);    // one MFMA
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);    // the next read
      }
      __builtin_amdgcn_sched_group_barrier(0x008, AHEAD, 0);
    }
  }

  // -inf where a key of the tile at k0 is past the end or (causal) after the
  // query; only the tiles that reach past the wave's first query wq0 or the
  // end need it
  __device__ __forceinline__ void mask(f32x16 (&s)[2], int k0, int wq0, int qi, int len,
                                       int causal, int hh) const {
    if ((causal && k0 + kPfKTile - 1 > wq0) || k0 + kPfKTile > len) {
#pragma unroll
      for (int sb = 0; sb < 2; ++sb)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int kv = k0 + 32 * sb + 8 * (i >> 2) + 4 * hh + (i & 3);
          const bool ok = kv < len && (!causal || kv <= qi);
          s[sb][i] = ok ? s[sb][i] : -INFINITY;
        }
    }
  }

  // online softmax of a masked S^T tile into the P^T operands of its four
  // 16-key steps
  __device__ __forceinline__ void softmax(f32x16 (&s)[2], u32x4 (&pb)[4], float scale_log2) {
    float b4[4];  // raw-score max (the scale is positive) over four chains
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const f32x16& x = s[c >> 1];
      const int e = 8 * (c & 1);
      b4[c] = max3(max3(x[e], x[e + 1], x[e + 2]), max3(x[e + 3], x[e + 4], x[e + 5]),
                   max3(x[e + 6], x[e + 7], x[e + 7]));
    }
    float bm = max3(max3(b4[0], b4[1], b4[2]), b4[3], b4[3]);
    // the partner lane's max (same query), exchanged between the wave's
    // halves in registers: one v_permlane32_swap instead of the LDS round trip
    // of a shuffle.  (Both kernels, 20 repeated calls each, also with two
    // unsynchronised workgroups per CU: bit-identical outputs, and bit-identical
    // to the shuffle; the four-wave kernel 0-2% faster with it.)
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(bm), __float_as_uint(bm),
                                                     false, false);
    bm = fmaxf(fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1])), bm) * scale_log2;
    if (__builtin_amdgcn_ballot_w64(bm > m + kPfRescaleSlack)) {
      const float mn = fmaxf(m, bm);
      const float alpha = __builtin_amdgcn_exp2f(m - mn);  // 0 while m = -inf
      lsum *= alpha;
#pragma unroll
      for (int db = 0; db < DB; ++db) o[db] *= alpha;
      m = mn;
    }
    const float nms = m == -INFINITY ? 0.f : -m;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const int sb = kk >> 1, base = 8 * (kk & 1);
      uint32_t pw[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float p0 =
            __builtin_amdgcn_exp2f(__builtin_fmaf(s[sb][base + 2 * j], scale_log2, nms));
        const float p1 =
            __builtin_amdgcn_exp2f(__builtin_fmaf(s[sb][base + 2 * j + 1], scale_log2, nms));
        lsum += p0 + p1;
        pw[j] = PfOps<DT>::pack(p0, p1);
      }
      pb[kk] = u32x4{pw[0], pw[1], pw[2], pw[3]};
    }
  }

  // normalise and store the lane's outputs (queries past the end: none)
  __device__ __forceinline__ void store(const PrefillArgs& a, int h, int64_t s0, int len, int qi,
                                        int hh) {
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
              u32x2{PfOps<DT>::pack(r[4 * g] * inv, r[4 * g + 1] * inv),
                    PfOps<DT>::pack(r[4 * g + 2] * inv, r[4 * g + 3] * inv)};
        }
    }
  }
};

// Uniform job of workgroup blockIdx.x for query tiles of qtile queries:
// returns false when the tile is empty.  Slice v = unit * S + r holds the
// unit's tiles r, r + S, ...; XCD x holds c slices, the run [v0, v0 + c) or,
// interleaved, slices x, x + kXcds, ...; its s-th job is the (s / c)-th
// largest tile of its (s % c)-th slice.
__device__ __forceinline__ bool pick_job(const PrefillArgs& a, int qtile, int& h, int64_t& s0,
                                         int& len, int& q0) {
  const int x = (int)(blockIdx.x % kXcds), sj = (int)(blockIdx.x / kXcds);
  const int S = a.slices;
  const int64_t n_sl = (int64_t)a.n_units * S;
  int c, v;
  if (a.interleave) {
    c = (int)((n_sl - x + kXcds - 1) / kXcds);
    if (c <= 0) return false;
    v = x + kXcds * (sj % c);
  } else {
    const int v0 = (int)(n_sl * x / kXcds);
    c = (int)(n_sl * (x + 1) / kXcds) - v0;
    if (c == 0) return false;
    v = v0 + sj % c;
  }
  const int k = sj / c;
  const int unit = v / S, r = v - unit * S;
  const int m = (a.n_qtiles - r + S - 1) / S;  // tiles in slice r
  if (k >= m) return false;
  const int tile = r + S * (m - 1 - k);
  const int b = unit / a.n_q_heads;
  h = unit % a.n_q_heads;
  int64_t s1 = a.cu_seqlens[b + 1];
  s0 = a.cu_seqlens[b];
  s0 = min(max(s0, (int64_t)0), a.total_tokens);
  s1 = min(max(s1, s0), a.total_tokens);
  len = (int)min(s1 - s0, (int64_t)a.max_seqlen);
  q0 = tile * qtile;
  return q0 < len;
}

// ---------------------------------------------------------------- short prompts
// Queries [q0, q0 + 128) of head h of the sequence at token s0 with len
// tokens; K and V tiles staged through registers, two stages each in LDS (V
// transposed, the 4-key quads of every 16 keys in the order 0, 2, 1, 3, so each
// P.V operand is one 16-byte LDS read).
template <int DT, int D>
__device__ __forceinline__ void attend_short(const PrefillArgs& a, uint8_t* lds, int h, int64_t s0,
                                             int len, int q0) {
  using E = PfOps<DT>;
  using W = WaveState<DT, D>;
  constexpr int KPITCH = D * 2 + 16;            // bytes per K row in LDS
  constexpr int K_BYTES = kPfKTile * KPITCH;
  constexpr int V_BYTES = D * kVtPitch;
  constexpr int DB = W::DB;
  constexpr int CPR = D / 8;                    // 16-byte chunks per row
  constexpr int KRPP = kShortThreads / CPR;     // K rows staged per pass
  constexpr int KPASS = kPfKTile / KRPP;
  constexpr int VTHREADS = (kPfKTile / 4) * CPR;  // (4-key quad, chunk) pairs
  const int kvh = h / a.group;
  const int kv_end = a.causal ? min(len, q0 + kShortQTile) : len;
  const int n_kt = (kv_end + kPfKTile - 1) / kPfKTile;

  const int t = threadIdx.x, lane = t & 63;
  const int w = __builtin_amdgcn_readfirstlane(t >> 6);  // uniform: the tile tests below branch
  const int col = lane & 31, hh = lane >> 5;
  const int qi = q0 + 32 * w + col;  // this lane's query, relative to the sequence
  const int wq0 = q0 + 32 * w;       // the wave's first query
  W st;
  st.init(a, h, s0, len, qi, hh);

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
    uint8_t* sk = lds + slot * K_BYTES;
#pragma unroll
    for (int p = 0; p < KPASS; ++p)
      *reinterpret_cast<u32x4*>(sk + (kr + KRPP * p) * KPITCH + kc * 16) = kreg[p];
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
  auto pv = [&](int kt, const u32x4 (&pb)[4]) {
    const uint8_t* vp = lds + 2 * K_BYTES + (kt & 1) * V_BYTES + col * kVtPitch + 16 * hh;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
#pragma unroll
      for (int db = 0; db < DB; ++db)
        st.o[db] = E::mfma(*reinterpret_cast<const u32x4*>(vp + 32 * db * kVtPitch + 32 * kk),
                           pb[kk], st.o[db]);
  };

  // K and V of tile kt + 1 are loaded while tile kt is computed; two
  // workgroups per CU overlap each other's softmax and matrix work.
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
    if (!a.causal || kt * kPfKTile <= wq0 + 31) {
      f32x16 sc[2];
      u32x4 pb[4];
      st.template qk<KPITCH, 0>(lds + (kt & 1) * K_BYTES + col * KPITCH + 16 * hh, sc);
      st.mask(sc, kt * kPfKTile, wq0, qi, len, a.causal, hh);
      st.softmax(sc, pb, a.scale_log2);
      pv(kt, pb);
    }
    if (more) {
      store_k((kt + 1) & 1);
      store_v(kt + 1, (kt + 1) & 1);
    }
    __syncthreads();
  }
  st.store(a, h, s0, len, qi, hh);
}

template <int DT, int D>
__global__ __launch_bounds__(kShortThreads, 2) void prefill_short_kernel(PrefillArgs a) {
  constexpr int K_BYTES = kPfKTile * (D * 2 + 16);
  constexpr int V_BYTES = D * kVtPitch;
  // two K stages, then two V^T stages
  __shared__ __align__(16) uint8_t lds[2 * K_BYTES + 2 * V_BYTES];
  int h, len, q0;
  int64_t s0;
  if (!pick_job(a, kShortQTile, h, s0, len, q0)) return;  // uniform, before any barrier
  attend_short<DT, D>(a, lds, h, s0, len, q0);
}

// ----------------------------------------------------------------- long prompts
// Queries [q0, q0 + 256) of head h of the sequence at token s0 with len
// tokens, ping-pong between the workgroup's halves.
template <int DT, int D>
__device__ __forceinline__ void attend_long(const PrefillArgs& a, uint8_t* lds, int h, int64_t s0,
                                            int len, int q0) {
  using E = PfOps<DT>;
  using W = WaveState<DT, D>;
  constexpr int KPITCH = D * 2 + 16;            // bytes per K row in LDS
  constexpr int K_BYTES = kPfKTile * KPITCH;
  // V rows stay untransposed at 2D + 64 bytes: the transposing reads of four
  // consecutive keys (64 bytes of each) then hit distinct banks
  constexpr int VPITCH = D * 2 + 64;
  constexpr int V_BYTES = kPfKTile * VPITCH;
  constexpr int DB = W::DB;
  constexpr int CPR = D / 8;                    // 16-byte chunks of a row's data
  constexpr int CK = KPITCH / 16, CV = VPITCH / 16;  // chunks per stored row
  constexpr int NK = (CK + kLongWaves - 1) / kLongWaves;
  constexpr int NV = (CV + kLongWaves - 1) / kLongWaves;
  constexpr uint32_t kPad = 0xFFFFFFF0u;        // an offset out of every range
  const int kvh = h / a.group;
  const int kv_end = a.causal ? min(len, q0 + kLongQTile) : len;
  const int n_kt = (kv_end + kPfKTile - 1) / kPfKTile;

  const int t = threadIdx.x, lane = t & 63;
  const int w = __builtin_amdgcn_readfirstlane(t >> 6);  // uniform: the tile tests below branch
  const int half = w >> 2;           // 0: waves 0-3, 1: waves 4-7 (one phase later)
  const int col = lane & 31, hh = lane >> 5;
  const int qi = q0 + 32 * w + col;  // this lane's query, relative to the sequence
  const int wq0 = q0 + 32 * w;       // the wave's first query
  // the wave's last key tile: causal waves stop at their last query's tile; a
  // wave past the end of the sequence attends to nothing (-1)
  const int jw = wq0 >= len ? -1
                 : a.causal ? min(n_kt - 1, min(wq0 + 31, len - 1) / kPfKTile)
                            : n_kt - 1;
  W st;
  st.init(a, h, s0, len, qi, hh);

  // Direct HBM -> LDS staging through raw buffer ranges over the sequence's K
  // and V rows of kv head kvh, ending at the last row's last byte.  Lane l of
  // a load instruction writes LDS bytes [16 l, 16 l + 16) after the
  // instruction's base, so instruction i of a tile covers stored chunks
  // [64 i, 64 i + 64); a row's pad chunks and rows past the sequence end get
  // an out-of-range offset, for which the hardware writes zeros and reads
  // nothing (zero V keeps P.V finite; those keys' scores are masked).
  const __amdgpu_buffer_rsrc_t krs =
      byte_range(a.k + s0 * a.k_tok_b + (int64_t)kvh * D * 2,
                 (uint32_t)((int64_t)(len - 1) * a.k_tok_b + D * 2));
  const __amdgpu_buffer_rsrc_t vrs =
      byte_range(a.v + s0 * a.v_tok_b + (int64_t)kvh * D * 2,
                 (uint32_t)((int64_t)(len - 1) * a.v_tok_b + D * 2));
  const uint32_t k_tok = (uint32_t)a.k_tok_b, v_tok = (uint32_t)a.v_tok_b;
  // instruction ii of wave w: K instruction w + 8 ii, V instruction
  // (w + 7) % 8 + 8 ii (the spare ones of a tile go to different waves); the
  // lane's byte offset within a tile
  uint32_t koffs[NK], voffs[NV];
#pragma unroll
  for (int ii = 0; ii < NK; ++ii) {
    const int c = (w + kLongWaves * ii) * 64 + lane, row = c / CK, ch = c % CK;
    koffs[ii] = ch < CPR ? row * k_tok + ch * 16 : kPad;
  }
#pragma unroll
  for (int ii = 0; ii < NV; ++ii) {
    const int c = (((w + kLongWaves - 1) % kLongWaves) + kLongWaves * ii) * 64 + lane;
    const int row = c / CV, ch = c % CV;
    voffs[ii] = ch < CPR ? row * v_tok + ch * 16 : kPad;
  }
  auto dma_k = [&](int kt) {
    const uint32_t t0 = kt * kPfKTile * k_tok;
#pragma unroll
    for (int ii = 0; ii < NK; ++ii) {
      const int i = w + kLongWaves * ii;  // uniform
      if (i < CK)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            krs, (lds_void*)(lds + (kt & 1) * K_BYTES + i * 1024), 16,
            koffs[ii] == kPad ? kPad : koffs[ii] + t0, 0, 0, 0);
    }
  };
  auto dma_v = [&](int kt) {
    const uint32_t t0 = kt * kPfKTile * v_tok;
#pragma unroll
    for (int ii = 0; ii < NV; ++ii) {
      const int i = (w + kLongWaves - 1) % kLongWaves + kLongWaves * ii;  // uniform
      if (i < CV)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            vrs, (lds_void*)(lds + 2 * K_BYTES + (kt & 1) * V_BYTES + i * 1024), 16,
            voffs[ii] == kPad ? kPad : voffs[ii] + t0, 0, 0, 0);
    }
  };
  // Transposing V reads (ds_read_b64_tr_b16: in each 16-lane group, result
  // lane j element k is element j % 4 of source lane 4k + j / 4).  Lane
  // (group G = lane / 16, s = lane % 16) reads 4 dims 16 (G & 1) + 4 (s % 4)
  // .. + 3 of key 4 (G >> 1) + s / 4; after the transpose it holds dim
  // 16 (G & 1) + s of keys 4 (G >> 1) .. + 3 (+ 16 kk, + 8 for elements 4-7,
  // + 32 db for the dims): the A operand of O^T = V^T . P^T.
  const int vG = lane >> 4, vs = lane & 15;
  const int vtr_off = (4 * (vG >> 1) + (vs >> 2)) * VPITCH + (16 * (vG & 1) + 4 * (vs & 3)) * 2;
  auto pv = [&](int kt, const u32x4 (&pb)[4]) {
    const uint8_t* vb = lds + 2 * K_BYTES + (kt & 1) * V_BYTES + vtr_off;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        const u32x2 lo = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (lds_s16x4*)(vb + 16 * kk * VPITCH + 64 * db)));
        const u32x2 hi = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (lds_s16x4*)(vb + (16 * kk + 8) * VPITCH + 64 * db)));
        st.o[db] = E::mfma(u32x4{lo[0], lo[1], hi[0], hi[1]}, pb[kk], st.o[db]);
      }
    // two reads per MFMA, four MFMAs ahead
    __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
    for (int i = 0; i < 4 * DB - 2; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
  };
  auto qk = [&](int kt, f32x16 (&s)[2]) {
    st.template qk<KPITCH, 2>(lds + (kt & 1) * K_BYTES + col * KPITCH + 16 * hh, s);
  };
  auto softmax = [&](int kt, f32x16 (&s)[2], u32x4 (&pb)[4]) {
    st.mask(s, kt * kPfKTile, wq0, qi, len, a.causal, hh);
    st.softmax(s, pb, a.scale_log2);
  };
  // K_{j+1} and V_j (read from slot 2j + 2 on) are loaded in slot 2j, whose
  // stages were last read in slot 2j - 1
  auto stage = [&](int j) {
    if (j + 1 < n_kt) dma_k(j + 1);
    if (j < n_kt) dma_v(j);
  };

  // Slots between workgroup barriers.  Phase p of a wave runs in slot
  // p + half: even p = 2j is the matrix phase of tile j (S_j, then the P.V of
  // tile j - 1; p = 2 n_kt only the last P.V), odd p = 2j + 1 its softmax.
  // Tile j's K is read in slots 2j and 2j + 1, its V in slots 2j + 2 and
  // 2j + 3.  Each half runs its own loop, so S_j lives within one iteration and
  // only P and O are carried; both halves pass 2 n_kt + 2 barriers after the
  // prologue's.  The barriers are plain s_barrier: a slot's LDS reads are
  // consumed by its own MFMAs before its barrier, and the direct loads issued
  // at the end of slot 2j are waited for (vmcnt) only before the barrier that
  // ends slot 2j + 1, so they land while slot 2j + 1 computes.
#define PF_BARRIER() \
  do { asm volatile("" ::: "memory"); __builtin_amdgcn_s_barrier(); asm volatile("" ::: "memory"); } while (0)
#define PF_BARRIER_LOADED()                              \
  do {                                                   \
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");     \
    __builtin_amdgcn_s_barrier();                        \
    asm volatile("" ::: "memory");                       \
  } while (0)
  u32x4 pb[4];
  dma_k(0);
  __syncthreads();  // waits for K_0 and the queries
  if (half == 0) {
    for (int j = 0; j < n_kt; ++j) {
      f32x16 sc[2];  // slot 2j
      if (j <= jw) qk(j, sc);
      if (j >= 1 && j - 1 <= jw) pv(j - 1, pb);
      stage(j);
      PF_BARRIER();
      if (j <= jw) softmax(j, sc, pb);  // slot 2j + 1
      PF_BARRIER_LOADED();
    }
    if (n_kt - 1 <= jw) pv(n_kt - 1, pb);  // slot 2 n_kt
    PF_BARRIER();
    PF_BARRIER();  // slot 2 n_kt + 1: idle
  } else {
    stage(0);  // slot 0: idle
    PF_BARRIER();
    for (int j = 0; j < n_kt; ++j) {
      f32x16 sc[2];  // slot 2j + 1
      if (j <= jw) qk(j, sc);
      if (j >= 1 && j - 1 <= jw) pv(j - 1, pb);
      PF_BARRIER_LOADED();
      if (j <= jw) softmax(j, sc, pb);  // slot 2j + 2
      stage(j + 1);
      PF_BARRIER();
    }
    if (n_kt - 1 <= jw) pv(n_kt - 1, pb);  // slot 2 n_kt + 1
    PF_BARRIER();
  }
#undef PF_BARRIER
#undef PF_BARRIER_LOADED
  st.store(a, h, s0, len, qi, hh);
}

template <int DT, int D>
__global__ __launch_bounds__(kLongThreads) void prefill_long_kernel(PrefillArgs a) {
  constexpr int K_BYTES = kPfKTile * (D * 2 + 16);
  constexpr int V_BYTES = kPfKTile * (D * 2 + 64);
  // two K stages, then two V stages
  __shared__ __align__(16) uint8_t lds[2 * K_BYTES + 2 * V_BYTES];
  int h, len, q0;
  int64_t s0;
  if (!pick_job(a, kLongQTile, h, s0, len, q0)) return;  // uniform, before any barrier
  attend_long<DT, D>(a, lds, h, s0, len, q0);
}

// Tile slices per unit.  With n_units not a multiple of kXcds, whole units
// leave some XCDs a unit more than others (1 x 8192 tokens of 28 heads: four
// XCDs hold 4 units, four hold 3, and the latter idle an eighth of the
// time).  S interleaved slices per unit, the smallest S with S * n_units a
// multiple of kXcds, even that out.  That pays only when the heaviest XCD's
// CUs take at least three tiles each: with fewer, its largest tiles set the
// end whatever the split, and the split unit's K/V fills two XCDs' L2.
// (Measured, same process: 1 x 8192 505.9 -> 481.8 us, 1 x 16384 2099 ->
// 1940 us; 1 x 4096, at two tiles per CU, 140.0 -> 145.8 us without the
// threshold.)
int slices_per_unit(int64_t n_units, int64_t n_qtiles, int cus_per_xcd) {
  int64_t g = kXcds;
  for (int64_t u = n_units % kXcds; u != 0;) {
    const int64_t t = g % u;
    g = u;
    u = t;
  }
  const int64_t S = std::min<int64_t>(kXcds / g, n_qtiles);
  if (S <= 1 || (n_units + kXcds - 1) / kXcds * n_qtiles < 3 * (int64_t)cus_per_xcd) return 1;
  return (int)S;
}

// kXcds runs of at most ceil(S * n_units / kXcds) slices of at most
// ceil(n_qtiles / S) tiles
int64_t grid_size(int64_t n_units, int64_t n_qtiles, int S) {
  return kXcds * ((n_qtiles + S - 1) / S) * ((S * n_units + kXcds - 1) / kXcds);
}

template <int DT, int D>
void launch_prefill(const PrefillArgs& a, bool long_prompts, uint32_t grid, hipStream_t stream) {
  if (long_prompts)
    hipLaunchKernelGGL((prefill_long_kernel<DT, D>), dim3(grid), dim3(kLongThreads), 0, stream,
                       a);
  else
    hipLaunchKernelGGL((prefill_short_kernel<DT, D>), dim3(grid), dim3(kShortThreads), 0, stream,
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
  const int64_t n_units = (int64_t)n_q_heads * batch;
  const bool long_prompts = max_seqlen > kLongPrompt;
  const int qtile = long_prompts ? kLongQTile : kShortQTile;
  const int64_t n_qtiles = ((int64_t)max_seqlen + qtile - 1) / qtile;
  if (kXcds * n_units * n_qtiles > INT32_MAX) return AEGKV_ERR_UNSUPPORTED;
  // the long kernel addresses K and V rows by 32-bit byte offsets within a
  // sequence, up to one key tile past its end
  if (long_prompts && ((int64_t)max_seqlen + kPfKTile) *
                              std::max(k_token_stride, v_token_stride) * 2 >
                          (int64_t)UINT32_MAX)
    return AEGKV_ERR_UNSUPPORTED;
  DeviceState* ds = nullptr;
  if (int rc = current_device_state(&ds)) return rc;
  const int slices = slices_per_unit(n_units, n_qtiles, std::max(1, ds->num_cu / kXcds));
  const int64_t grid = grid_size(n_units, n_qtiles, slices);
  if (grid > INT32_MAX) return AEGKV_ERR_UNSUPPORTED;

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
  a.slices = slices;
  // Prompts of different lengths: contiguous runs would give each XCD whole
  // prompts (8 prompts of 28 heads: one per XCD, the longest setting the
  // end), so the units are dealt round-robin instead.  That spreads one kv
  // head's query heads over several L2s, which costs uniform batches 1-4%,
  // so it is kept for batches the host bound shows to be ragged (fewer
  // tokens than 90% of batch x max_seqlen).  Same process, 8 prompts of
  // 77-2048 tokens: 281.7 -> 149.6 us.
  a.interleave = total_tokens * 10 < (int64_t)batch * max_seqlen * 9 ? 1 : 0;
  a.causal = causal ? 1 : 0;
  a.scale_log2 = scale * 1.4426950408889634f;
  const uint32_t g32 = (uint32_t)grid;
  if (dtype == AEGKV_DTYPE_BF16) {
    if (head_dim == 64) launch_prefill<AEGKV_DTYPE_BF16, 64>(a, long_prompts, g32, stream);
    else launch_prefill<AEGKV_DTYPE_BF16, 128>(a, long_prompts, g32, stream);
  } else {
    if (head_dim == 64) launch_prefill<AEGKV_DTYPE_FP16, 64>(a, long_prompts, g32, stream);
    else launch_prefill<AEGKV_DTYPE_FP16, 128>(a, long_prompts, g32, stream);
  }
  AEGKV_HIP_TRY(hipGetLastError());
  return AEGKV_OK;
}

}  // extern "C"
