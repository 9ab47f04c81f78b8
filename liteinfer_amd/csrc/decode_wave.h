// Paged decode on CDNA4 matrix cores (bf16 / fp16, head_dim 64 or 128).
//
// Same attention as liteinfer's decode kernels (liteinfer/models/
// paged_kernels.py:374-413, :462-571): per (sequence, KV head, partition),
// the G query heads sharing a KV head fold the partition's keys into an
// online softmax, fp32 throughout, weights rounded to the value dtype before
// they multiply V. One wave64 per partition, 32 keys per step, laid out for
// v_mfma_f32_16x16x32_{bf16,f16}. Lane (n, g) = (lane % 16, lane / 16).
//
// Loads. A tile's K and V rows go straight from the pool into LDS
// (global_load_lds_dwordx4, the 32-key tile layout of li_mfma.h): each load
// instruction reads 4 whole 256-byte pool rows, 16 lanes per row. (A layout
// where 16 lanes each read 64 bytes of 16 different rows measured 20% less
// HBM bandwidth.) The next tile's loads are always in flight while the
// current one is folded.
//
//   S^T = K Q^T     A = K (16 keys x 32 dims) read from LDS, B = Q^T
//                   (32 dims x 16 heads) kept in registers. Lane (n, g) gets
//                   the scores of keys 4g..4g+3 (and 16+4g.. from the second
//                   block) for head n.
//   O^T += V^T P^T  B = P^T: lane (n, g)'s 8 weights are for keys
//                   kappa(g, 0..7) of head n, exactly its B operand, no lane
//                   exchange. A = V^T (16 dims x 32 keys) comes straight out
//                   of LDS through transposing reads (li_read_vt's
//                   addressing, ds_read_b64_tr_b16).
//   The result gives lane (n, g) dims 16 blk + 4g + r of head n, so the
//   running-max rescale is per lane (its own head) and nothing is reduced
//   across lanes except the tile maximum (two permlane swaps) and, once at
//   the end, the denominator.
//
// Heads past G are zero rows of Q^T: they score 0 and are never stored.
// Keys past the partition's end read the last key's slot (a real row) and
// are masked to -inf, so every load is in bounds.//
// This header holds one decode wave's work (its loads, folds and stores) and
// the balanced split's per-wave body, shared by the decode kernels and by the
// prefill kernel that serves one-query rows beside chunks. Every function
// takes its lane as threadIdx.x % 64, so a wave of a larger work-group runs
// it as a work-group of one wave does.
#pragma once

#include "li_attention.h"
#include "li_mfma.h"

#include <type_traits>

namespace li {
namespace {

// Lane of the calling thread in its wave.
__device__ __forceinline__ int li_lane() { return (int)(threadIdx.x & 63); }


// Decode reads every K/V row once per call: its loads carry the
// non-temporal hint (config 2: 218 -> 196 us against loads that keep their
// lines in L2).
constexpr bool kDecodeStream = true;

// The LDS tile layout of a pool: bf16 / fp16 rows, or fp8 (e4m3) rows at
// head_dim 128.
template <int D, bool F8>
using KvTile = std::conditional_t<F8, F8Tile, TileLayout<D>>;

// Issues the 2 * kInsts direct-to-LDS loads of the 32-key tile whose first
// key is entry `t` of the staged slots, into the stage at `stage`. Lane
// (rr, n) = (lane / CH, lane % CH) loads keys rr * kInsts + i. kpool / vpool
// point at the KV head's row of slot 0, row_bytes is the pool's slot stride.
template <int D, bool F8>
__device__ __forceinline__ void issue_tile(char* stage, const char* __restrict__ kpool,
                                           const char* __restrict__ vpool, const int* __restrict__ sl,
                                           uint32_t row_bytes, int t, int lane) {
  using L = KvTile<D, F8>;
  const int rr = lane / L::kCh, nn = lane % L::kCh;
  int keys[L::kInsts];
  if constexpr (L::kInsts == 8) {
    const int4 a = *reinterpret_cast<const int4*>(sl + t + 8 * rr);
    const int4 b = *reinterpret_cast<const int4*>(sl + t + 8 * rr + 4);
    keys[0] = a.x; keys[1] = a.y; keys[2] = a.z; keys[3] = a.w;
    keys[4] = b.x; keys[5] = b.y; keys[6] = b.z; keys[7] = b.w;
  } else {
    const int4 a = *reinterpret_cast<const int4*>(sl + t + 4 * rr);
    keys[0] = a.x; keys[1] = a.y; keys[2] = a.z; keys[3] = a.w;
  }
#pragma unroll
  for (int i = 0; i < L::kInsts; ++i) {
    const int key = rr * L::kInsts + i;
    const uint32_t dst = lds_addr(stage + i * 1024);  // rows kRowsPerInst * i ..: 1 KiB per instruction
    // Lane nn writes slot nn of its row: global chunk nn ^ swizzle(key).
    dma16<kDecodeStream>(row_ptr(kpool + 16 * (nn ^ L::kswizzle(key)), (uint32_t)keys[i], row_bytes), dst);
    dma16<kDecodeStream>(row_ptr(vpool + 16 * (nn ^ L::vswizzle(key)), (uint32_t)keys[i], row_bytes), dst + 32 * L::kRowBytes);
  }
}

// LDS of one decode wave: the staged slots of a chunk of kChunk keys (a
// multiple of 64) and two tile stages.
template <int D, bool F8, int kChunk = kSlotChunk>
struct DecodeLds {
  int sl[kChunk + 64];
  char stage[2][KvTile<D, F8>::kTileBytes];
};

// Online-softmax state of one wave: lane (n, g) holds head n's running max
// and (partial) denominator, and in acc[blk][r] (blk < D / 16) dim
// 16 blk + 4 g + r of its accumulator.
struct DecodeState {
  float m, l;
  floatx4_t acc[8];
};

// The query operand of one KV head's group, as the score MFMAs take it
// (B = Q^T; lane (n, g) holds head n, zeros past the group's heads).
//
// 16-bit pools: D / 32 fragments of the query (v_mfma_f32_16x16x32_*),
// lane (n, g) holding dims 32 j + 8 g .. + 8 of fragment j.
//
// fp8 pools: the scores run on v_mfma_scale_f32_16x16x128_f8f6f4 with K
// straight from the pool bytes (no conversion of K), so the query is given
// in e4m3 as well: head n's row split into kTerms e4m3 terms by split_e4m3
// below (a power of two per row, then terms with block scales 2^0, 2^-4,
// 2^-8: exact for a bf16 (two terms) or fp16 (three) value down to 2^-13 of
// the row's largest). The terms' MFMAs chain into one accumulator and
// `scale` (2^-e) returns the scores to the query's units. Lane (n, g) holds
// dims 32 g .. 32 g + 31 of head n, byte i of each term being dim 32 g + i,
// the same order in which it reads the K bytes of its key, so the two
// operands meet dim for dim.
typedef int v8i_t __attribute__((ext_vector_type(8)));

// Splits one row of the query into e4m3 terms for the fp8 score MFMAs: the
// lane holds 32 of the row's values (x, dims 32 g ..), the row's four lanes
// (same n) together the whole row. The row is scaled by the exact power of
// two 2^e that puts its largest |value| in [128, 256); term t is the e4m3
// rounding of 16^t times what the terms before it left (byte i of the lane's
// term is its value i), and its MFMA takes it with block scale 2^-4t
// (kTermScale). Scaling each residual up keeps it in e4m3's normal range
// (a residual is at most 2^-4 of the value it rounds, so 16 times it stays
// under 448 and above 2^-6 whenever the value is): two terms hold a bf16
// value's 8 significant bits exactly, three an fp16 value's 11, down to
// values of 2^-6 after the scaling (2^-13 of the row's largest). Returns
// 2^-e, which takes the scores back to the query's units.
__device__ __forceinline__ constexpr int kTermScale(int t) { return 127 - 4 * t; }  // e8m0 of 2^-4t

template <int kTerms>
__device__ __forceinline__ float split_e4m3(float (&x)[32], v8i_t (&t)[kTerms]) {
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(x[i]));
  amax = li_group_max(amax);  // the row's four lanes
  // amax in [2^(E-127), 2^(E-126)): 2^(134-E) puts it in [2^7, 2^8).
  const int ex = min(max(134 - (int)((__float_as_uint(amax) >> 23) & 0xff), -126), 126);
  const float mult = __uint_as_float((uint32_t)(127 + ex) << 23);
#pragma unroll
  for (int i = 0; i < 32; ++i) x[i] *= mult;
  typedef short s2_t __attribute__((ext_vector_type(2)));
#pragma unroll
  for (int tt = 0; tt < kTerms; ++tt) {
#pragma unroll
    for (int w = 0; w < 8; ++w) {
      s2_t b = {0, 0};
      b = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(b, x[4 * w], x[4 * w + 1], 1.f, false);
      b = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(b, x[4 * w + 2], x[4 * w + 3], 1.f, true);
      const uint32_t bits = __builtin_bit_cast(uint32_t, b);
      t[tt][w] = (int)bits;
      if (tt + 1 < kTerms) {
        // What this term left, times 16 (exact in fp32): the next term is
        // that, its MFMA's block scale 2^-4 taking it back.
        const auto lo = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(bits, 1.f, false);
        const auto hi = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(bits, 1.f, true);
        x[4 * w] = (x[4 * w] - lo[0]) * 16.f;
        x[4 * w + 1] = (x[4 * w + 1] - lo[1]) * 16.f;
        x[4 * w + 2] = (x[4 * w + 2] - hi[0]) * 16.f;
        x[4 * w + 3] = (x[4 * w + 3] - hi[1]) * 16.f;
      }
    }
  }
  return __uint_as_float((uint32_t)(127 - ex) << 23);
}

template <typename T, int D, bool F8>
struct DecodeQuery {
  typename Mfma<T>::Frag f[D / 32];
  float scale;  // 1
};

template <typename T, int D>
struct DecodeQuery<T, D, true> {
  static_assert(D == 128, "fp8 pools: head_dim 128");
  static constexpr int kTerms = std::is_same<T, li_f16>::value ? 3 : 2;
  v8i_t t[kTerms];
  float scale;  // 2^-e
};

// Per-lane LDS byte offsets within a tile: the K operand of key n, step j
// (key 16 + n sits L::kRow16 bytes below), and the V^T reads' addresses
// (li_read_vt's two for 16-bit rows, the one 8-bit transposing read for
// fp8 rows; see F8Tile).
template <int D, bool F8>
struct TileOffsets {
  uint32_t koff[D / 32], voff[D / 16];
  uint32_t kq[2];  // fp8: the two 16-byte chunks (dims 32 g ..) of key n's K row
  __device__ __forceinline__ TileOffsets() {
    using L = KvTile<D, F8>;
    const int lane = li_lane();
    const int n = lane & 15, g = lane >> 4;
    if constexpr (F8) {
      kq[0] = L::offset(n, 2 * g);
      kq[1] = L::offset(n, 2 * g + 1);
      const int s16 = lane & 15;
#pragma unroll
      for (int blk = 0; blk < D / 16; ++blk) voff[blk] = L::voffset(kappa(g, s16 >> 1), blk) + 8 * (s16 & 1);
    } else {
#pragma unroll
      for (int j = 0; j < D / 32; ++j) koff[j] = L::offset(n, 4 * j + g);
      const int s16 = lane & 15, a4 = s16 & 3, key = 4 * g + (s16 >> 2);
#pragma unroll
      for (int blk = 0; blk < D / 16; ++blk) voff[blk] = L::voffset(key, 2 * blk + (a4 >> 1)) + 8 * (a4 & 1);
    }
  }
};

// Folds the 32-key tile in `stage` (LDS byte address) whose first key is t0
// into `st`; keys at or past `te` are masked. q holds the group's query, sc
// the softmax scale times log2(e) (and an fp8 pool's k_scale, and the
// query's scale q.scale).
template <typename T, int D, bool F8>
__device__ __forceinline__ void fold_tile(uint32_t stage, int t0, int te, const DecodeQuery<T, D, F8>& q, float sc,
                                          const TileOffsets<D, F8>& o, DecodeState& st) {
  using M = Mfma<T>;
  using Frag = typename M::Frag;
  using L = KvTile<D, F8>;
  constexpr int kSteps = D / 32;
  const int lane = li_lane();
  const int g = lane >> 4;
  floatx4_t s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
  if constexpr (F8) {
    // Keys n and 16 + n, dims 32 g .. 32 g + 31, as stored (e4m3).
    auto krow = [&](uint32_t at) {
      const u32x4_t lo = *(const __attribute__((address_space(3))) u32x4_t*)(uintptr_t)(at + o.kq[0]);
      const u32x4_t hi = *(const __attribute__((address_space(3))) u32x4_t*)(uintptr_t)(at + o.kq[1]);
      return v8i_t{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
    };
    const v8i_t k0 = krow(stage), k1 = krow(stage + L::kRow16);
#pragma unroll
    for (int t = 0; t < DecodeQuery<T, D, F8>::kTerms; ++t) {
      // Formats e4m3 (0) for both operands; block scales 2^0 for K, 2^-4t
      // for query term t.
      s0 = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(k0, q.t[t], s0, 0, 0, 0, 127, 0, kTermScale(t));
      s1 = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(k1, q.t[t], s1, 0, 0, 0, 127, 0, kTermScale(t));
    }
  } else {
#pragma unroll
    for (int j = 0; j < kSteps; ++j) {
      s0 = M::mma(lds_read_frag<Frag>(stage + o.koff[j]), q.f[j], s0);
      s1 = M::mma(lds_read_frag<Frag>(stage + o.koff[j] + L::kRow16), q.f[j], s1);
    }
  }
  float x[8];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    x[r] = s0[r];
    x[4 + r] = s1[r];
  }
  if (t0 + 32 > te) {  // a partial tile: mask the keys past its end
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = (t0 + kappa(g, e) < te) ? x[e] : -INFINITY;
  }
  float mx = fmaxf(fmaxf(x[0], x[1]), x[2]);
  mx = fmaxf(fmaxf(mx, x[3]), x[4]);
  mx = fmaxf(fmaxf(mx, x[5]), fmaxf(x[6], x[7]));
  mx = li_group_max(mx) * sc;
  // Lazy rescale (see kLazyRescale).
  const float mnew = (mx > st.m + kLazyRescale) ? mx : st.m;
  const float alpha = __builtin_amdgcn_exp2f(st.m - mnew);
  float p[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) p[e] = __builtin_amdgcn_exp2f(fmaf(x[e], sc, -mnew));
  const float psum = ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]));
  st.l = st.l * alpha + psum;
  if (__any(mnew != st.m)) {
#pragma unroll
    for (int i = 0; i < D / 16; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) st.acc[i][r] *= alpha;
  }
  st.m = mnew;
  u32x4_t pw;
#pragma unroll
  for (int u = 0; u < 4; ++u) pw[u] = li_pack2<T>(p[2 * u], p[2 * u + 1]);
  const Frag pf = __builtin_bit_cast(Frag, pw);
  // O^T += V^T P^T, 16 dims at a time, V^T straight out of LDS.
  const uint32_t vstage = stage + 32 * L::kRowBytes;
#pragma unroll
  for (int blk = 0; blk < D / 16; ++blk) {
    if constexpr (F8) st.acc[blk] = M::mma(lds_read_f8_vt<Frag>(vstage + o.voff[blk]), pf, st.acc[blk]);
    else st.acc[blk] = M::mma(lds_read_vt<Frag>(vstage + o.voff[blk], vstage + o.voff[blk] + L::kRow16), pf, st.acc[blk]);
  }
}

// Folds keys [kb, ke) of sequence `seq`'s context for KV head `kvh` into `st`.
template <typename T, int D, bool F8, int kChunk>
__device__ __forceinline__ void fold_keys(const AttnArgs& a, DecodeLds<D, F8, kChunk>& lds,
                                          const DecodeQuery<T, D, F8>& q, int seq, int kvh, int kb, int ke,
                                          DecodeState& st) {
  using L = KvTile<D, F8>;
  const int lane = li_lane();
  const TileOffsets<D, F8> off;
  const int esize = F8 ? 1 : (int)sizeof(T);  // bytes per pool element
  const char* kpool = static_cast<const char*>(a.kp) + (int64_t)kvh * a.p_s1 * esize;
  const char* vpool = static_cast<const char*>(a.vp) + (int64_t)kvh * a.p_s1 * esize;
  const uint32_t row_bytes = (uint32_t)(a.p_s0 * esize);
  const int64_t* srow = a.st + (int64_t)seq * a.st_s;
  // An fp8 pool stores K / k_scale: its scale multiplies the scores.
  const float sc = a.scale * (F8 ? a.k_scale * q.scale : 1.f) * kLog2eMfma;

  for (int c0 = kb; c0 < ke; c0 += kChunk) {
    const int c1 = min(c0 + kChunk, ke);
    const int ntiles = (c1 - c0 + 31) / 32;
    // Stage this chunk's slots (int32: a pool holds fewer than 2^31 slots),
    // plus a tile past its end. Entries past the chunk repeat its last slot,
    // so the loads of a partial or look-ahead tile read real rows; their
    // scores are masked.
    {
      int vals[kChunk / 64 + 1];
#pragma unroll
      for (int k = 0; k < kChunk / 64 + 1; ++k) vals[k] = (int)srow[min(c0 + lane + 64 * k, c1 - 1)];
#pragma unroll
      for (int k = 0; k < kChunk / 64 + 1; ++k) lds.sl[lane + 64 * k] = vals[k];
    }

    auto fold = [&](uint32_t stage, int t0) __attribute__((always_inline)) {
      fold_tile<T, D, F8>(stage, t0, c1, q, sc, off, st);
    };

    // Two stages: while one tile is folded the next tile's loads land in the
    // other. Past the chunk the look-ahead re-reads a real tile (cache hits),
    // so the loads in flight are the same every step and no load sits under
    // a branch.
    constexpr int kInFlight = 2 * L::kInsts;
    issue_tile<D, F8>(lds.stage[0], kpool, vpool, lds.sl, row_bytes, 0, lane);
    for (int ti = 0;;) {
      issue_tile<D, F8>(lds.stage[1], kpool, vpool, lds.sl, row_bytes, min(32 * (ti + 1), kChunk), lane);
      li_wait_vm<kInFlight>();
      fold(lds_addr(lds.stage[0]), c0 + 32 * ti);
      if (++ti >= ntiles) break;
      issue_tile<D, F8>(lds.stage[0], kpool, vpool, lds.sl, row_bytes, min(32 * (ti + 1), kChunk), lane);
      li_wait_vm<kInFlight>();
      fold(lds_addr(lds.stage[1]), c0 + 32 * ti);
      if (++ti >= ntiles) break;
    }
    // Drain the look-ahead loads before the slots (and stages) are reused.
    li_wait_vm<0>();
  }
}

// Loads the query operand of KV head `kvh`'s group for the query at `row`.
template <typename T, int D, bool F8>
__device__ __forceinline__ void load_query(const AttnArgs& a, int row, int kvh, DecodeQuery<T, D, F8>& q) {
  using Frag = typename Mfma<T>::Frag;
  const int lane = li_lane();
  const int n = lane & 15, g = lane >> 4;
  const T* qrow = static_cast<const T*>(a.q) + (int64_t)row * a.q_s0 + (int64_t)(kvh * a.groups + n) * a.q_s1;
  if constexpr (!F8) {
#pragma unroll
    for (int j = 0; j < D / 32; ++j) q.f[j] = (n < a.groups) ? *reinterpret_cast<const Frag*>(qrow + 32 * j + 8 * g) : Frag{};
    q.scale = 1.f;
  } else {
    float x[32];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const Frag f = (n < a.groups) ? *reinterpret_cast<const Frag*>(qrow + 32 * g + 8 * i) : Frag{};
#pragma unroll
      for (int e = 0; e < 8; ++e) x[8 * i + e] = (float)f[e];
    }
    q.scale = split_e4m3<DecodeQuery<T, D, F8>::kTerms>(x, q.t);
  }
}

// Writes a finished softmax: the normalised output row of each head of the
// group to `out` (dtype T), or, for a piece of a context, the fp32 normalised
// partial of head n to po + n * p_head_stride * D and its log2-domain LSE to
// plse[n * p_head_stride]. vscale multiplies the outputs (an fp8 pool stores
// V / v_scale).
template <typename T, int D>
__device__ __forceinline__ void store_state(const DecodeState& st, T* orow_head0, int64_t o_s1, float* po,
                                            float* plse, int64_t p_head_stride, int groups, float vscale) {
  const int lane = li_lane();
  const int n = lane & 15, g = lane >> 4;
  const float lt = li_group_sum(st.l);
  if (n >= groups) return;
  const float inv = vscale / lt;
  if (orow_head0) {
    T* orow = orow_head0 + (int64_t)n * o_s1 + 4 * g;
#pragma unroll
    for (int blk = 0; blk < D / 16; ++blk) {
      uint2 w;
      w.x = li_pack2<T>(st.acc[blk][0] * inv, st.acc[blk][1] * inv);
      w.y = li_pack2<T>(st.acc[blk][2] * inv, st.acc[blk][3] * inv);
      *reinterpret_cast<uint2*>(orow + 16 * blk) = w;
    }
  } else {
    float* prow = po + (int64_t)n * p_head_stride * D + 4 * g;
#pragma unroll
    for (int blk = 0; blk < D / 16; ++blk) {
      floatx4_t v;
#pragma unroll
      for (int r = 0; r < 4; ++r) v[r] = st.acc[blk][r] * inv;
      *reinterpret_cast<floatx4_t*>(prow + 16 * blk) = v;
    }
    if (g == 0) plse[(int64_t)n * p_head_stride] = st.m + log2f(lt);
  }
}

__device__ __forceinline__ void reset_state(DecodeState& st) {
  st.m = -INFINITY;
  st.l = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) st.acc[i] = floatx4_t{0.f, 0.f, 0.f, 0.f};
}

// Query row of sequence `seq`, or -1 when the decode kernel does not serve
// it (in a packed pass, sequences with more than one query).
__device__ __forceinline__ int decode_row(const AttnArgs& a, int seq) {
  if (!a.qsl) return seq;
  const int f = a.qsl[seq];
  return (a.qsl[seq + 1] - f == 1) ? f : -1;
}

// Keys of sequence `seq` the decode kernel folds, per KV head. The context
// length is read beside the query rows (not after them, as the branch would
// order it): in a packed pass the two reads then share one round trip.
__device__ __forceinline__ int decode_keys(const AttnArgs& a, int seq) {
  const int ctx = a.ctx[seq];
  return decode_row(a, seq) < 0 ? 0 : max(ctx, 0);
}

// ---------------------------------------------------------------------------
// Balanced decode: a fixed grid of W waves splits the flattened key space
// (sequence-major, then KV head, then key) into equal shares of whole
// 32-key tiles. A wave walks the (sequence, KV head) segments its share
// covers, carrying nothing between them; a segment that is a whole context
// is written as output, a piece of one as an fp32 partial in one of the
// wave's two partial slots (0: the segment holding the wave's first key,
// 1: its last segment). Every wave does the same work whatever the spread of
// context lengths, and there are no empty work-groups. W comes from the host
// (a multiple of the CU count), the shares from device data, so a captured
// graph replays for any contexts.
// ---------------------------------------------------------------------------

// Sum of v over the wave, exact for integers.
__device__ __forceinline__ int64_t wave_sum_i64(int64_t v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const int lo = __shfl_xor((int)(v & 0xffffffff), off, 64);
    const int hi = __shfl_xor((int)(v >> 32), off, 64);
    v += ((int64_t)hi << 32) | (uint32_t)lo;
  }
  return v;
}

// Total keys (all sequences, all KV heads) and the share of each wave.
__device__ __forceinline__ void balanced_share(const AttnArgs& a, int64_t waves, int64_t& total, int64_t& share) {
  const int lane = li_lane();
  int64_t t = 0;
  for (int s0 = 0; s0 < a.batch; s0 += 64) {
    const int s = s0 + lane;
    t += s < a.batch ? (int64_t)decode_keys(a, s) : 0;
  }
  total = wave_sum_i64(t) * a.num_kv_heads;
  share = ((total + waves - 1) / waves + 31) / 32 * 32;
}

// One wave's share of the balanced split: wave w of `waves` (its LDS `lds`).
template <typename T, int D, bool F8>
__device__ __forceinline__ void decode_balanced_wave(const AttnArgs& a, int w, int64_t waves, DecodeLds<D, F8>& lds) {
  const float vscale = F8 ? a.v_scale : 1.f;
  const int lane = li_lane();
  int64_t total, share;
  balanced_share(a, waves, total, share);
  int64_t pos = (int64_t)w * share;
  if (pos >= total) return;
  const int64_t end = min(pos + share, total);

  // The flattened key space runs head-major: (KV head, sequence, key). Every
  // head holds the same keys, so the waves folding different heads of the
  // same slots run side by side (wave w and wave w + W / Hkv start at about
  // the same key of heads h and h + 1) and each slot's rows of all heads,
  // contiguous in the pool, are read at about the same time (config 2 over
  // an fp8 pool, whose rows of one head are 128 bytes: 116.5 -> 112.7 us).
  const int64_t per_head = total / a.num_kv_heads;
  int kvh = (int)(pos / per_head);
  const int64_t hpos = pos - (int64_t)kvh * per_head;
  // Find the sequence holding key `hpos` of the head: scan 64 sequences at a time.
  int seq = 0;
  int64_t before = 0;  // keys of the sequences before `seq`
  for (int s0 = 0; s0 < a.batch; s0 += 64) {
    const int s = s0 + lane;
    const int64_t c = s < a.batch ? (int64_t)decode_keys(a, s) : 0;
    int64_t incl = c;  // inclusive prefix within this group of 64
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int lo = __shfl_up((int)(incl & 0xffffffff), off, 64);
      const int hi = __shfl_up((int)(incl >> 32), off, 64);
      if (lane >= off) incl += ((int64_t)hi << 32) | (uint32_t)lo;
    }
    const uint64_t hit = __ballot(before + incl > hpos);
    if (hit) {
      const int first = __ffsll((long long)hit) - 1;
      const int64_t excl = __shfl(incl - c, first, 64);
      seq = s0 + first;
      before += excl;
      break;
    }
    before += __shfl(incl, 63, 64);
  }

  int ctx = decode_keys(a, seq);
  int key0 = (int)(hpos - before);
  const int G = a.groups;
  float* part_o = a.part_o + (int64_t)w * 2 * G * a.head_dim;
  float* part_lse = a.part_lse + (int64_t)w * 2 * G;
  bool first_segment = true;
  while (pos < end) {
    const int take = (int)min((int64_t)(ctx - key0), end - pos);
    if (key0 == 0 && lane == 0) {
      // This wave holds the context's first key: record which waves hold its
      // pieces, and which of this wave's slots the first one is in.
      const int64_t off = (int64_t)kvh * per_head + before;
      a.pieces[(int64_t)seq * a.num_kv_heads + kvh] =
          int4{w, (int)((off + ctx - 1) / share), first_segment ? 0 : 1, 0};
    }
    const int row = decode_row(a, seq);
    DecodeQuery<T, D, F8> q;
    load_query(a, row, kvh, q);
    DecodeState st;
    reset_state(st);
    fold_keys<T, D, F8>(a, lds, q, seq, kvh, key0, key0 + take, st);
    if (key0 == 0 && take == ctx) {
      store_state<T, D>(st, static_cast<T*>(a.out) + (int64_t)row * a.o_s0 + (int64_t)kvh * G * a.o_s1, a.o_s1,
                        nullptr, nullptr, 0, G, vscale);
    } else {
      const int slot = first_segment ? 0 : 1;
      store_state<T, D>(st, nullptr, 0, part_o + (int64_t)slot * G * a.head_dim, part_lse + slot * G, 1, G, vscale);
    }
    pos += take;
    first_segment = false;
    key0 = 0;
    before += ctx;
    ++seq;
    while (seq < a.batch && decode_keys(a, seq) == 0) ++seq;
    if (seq >= a.batch) {
      if (++kvh == a.num_kv_heads) break;
      seq = 0;
      before = 0;
      while (seq < a.batch && decode_keys(a, seq) == 0) ++seq;
      if (seq >= a.batch) break;
    }
    ctx = decode_keys(a, seq);
  }
}

}  // namespace
}  // namespace li
