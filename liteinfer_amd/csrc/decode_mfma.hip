// Paged decode kernels on CDNA4 matrix cores (bf16 / fp16, head_dim 64 or
// 128; fp8 pools at 128): the same attention as liteinfer's decode kernels
// (liteinfer/models/paged_kernels.py:374-413, :462-571). One wave's loads,
// MFMA layout and online softmax are in decode_wave.h; this file holds the
// kernels built on them (partitioned, balanced, head-grouped), the combine of
// the balanced split's pieces, and the launch.
#include "decode_wave.h"

#include <cstdlib>

namespace li {
namespace {

// Waves per (sequence, head) of the many-piece combine.
#ifndef LI_COMBINE_WAVES
#define LI_COMBINE_WAVES 4
#endif
constexpr int kCombineWaves = LI_COMBINE_WAVES;

// ---------------------------------------------------------------------------
// Partitioned decode: one wave per (sequence, KV head, partition). Serves a
// pinned split count (the reference's equal-slice rule: partition p of a
// context of c keys is [p * cdiv(c, S), ...)).
// ---------------------------------------------------------------------------
template <typename T, int D, bool F8>
__global__ __launch_bounds__(64) void decode_partitioned(AttnArgs a) {
  __shared__ __attribute__((aligned(1024))) DecodeLds<D, F8> lds;
  const float vscale = F8 ? a.v_scale : 1.f;
  // Partition-major order: every sequence's first partition is dispatched
  // before any second one, so the grid's empty tail comes last.
  int bid = blockIdx.x;
  const int kvh = bid % a.num_kv_heads;
  bid /= a.num_kv_heads;
  const int seq = bid % a.batch;
  const int part = bid / a.batch;
  const int row = decode_row(a, seq);
  if (row < 0) return;
  const int ctx = a.ctx[seq];
  if (ctx <= 0) {
    // No key to attend to: the reference's softmax over nothing is 0 / 0.
    if (part == 0) {
      T* orow = static_cast<T*>(a.out) + (int64_t)row * a.o_s0 + (int64_t)kvh * a.groups * a.o_s1;
      for (int h = 0; h < a.groups; ++h)
        for (int d = threadIdx.x; d < D; d += 64) orow[(int64_t)h * a.o_s1 + d] = li_quiet_nan<T>();
    }
    return;
  }
  const int plen = a.part_len > 0 ? a.part_len : max(1, (ctx + a.num_parts - 1) / a.num_parts);
  const int kb = part * plen;
  if (kb >= ctx) return;
  const int ke = min(kb + plen, ctx);
  const int nparts = (ctx + plen - 1) / plen;

  DecodeQuery<T, D, F8> q;
  load_query(a, row, kvh, q);
  DecodeState st;
  reset_state(st);
  fold_keys<T, D, F8>(a, lds, q, seq, kvh, kb, ke, st);
  const int head0 = kvh * a.groups;
  if (nparts == 1) {
    store_state<T, D>(st, static_cast<T*>(a.out) + (int64_t)row * a.o_s0 + (int64_t)head0 * a.o_s1, a.o_s1,
                      nullptr, nullptr, 0, a.groups, vscale);
  } else {
    // partials [batch, num_heads, num_parts, D]: head h's row is (seq * Hq + h) * P + part
    const int64_t base = ((int64_t)seq * a.num_heads + head0) * a.num_parts + part;
    store_state<T, D>(st, nullptr, 0, a.part_o + base * D, a.part_lse + base, a.num_parts, a.groups, vscale);
  }
}

template <typename T, int D, bool F8>
__global__ __launch_bounds__(64) void decode_balanced(AttnArgs a) {
  __shared__ __attribute__((aligned(1024))) DecodeLds<D, F8> lds;
  decode_balanced_wave<T, D, F8>(a, (int)blockIdx.x, a.num_parts, lds);
}

// ---------------------------------------------------------------------------
// Head-grouped balanced decode: the balanced split over (sequence, group of
// HG KV heads, key) instead of (sequence, KV head, key), each wave folding
// every head of its group: for each 32-key tile, the group's heads one after
// the other, each into its own online-softmax state. Consecutive tiles of a
// wave then read HG adjacent rows of the same slots — HG * head_dim * 2
// contiguous bytes of K (and of V) per slot — which DRAM serves faster than
// separate per-head streams (a load-only probe of config 2's rows: +5% for
// all 8 heads together). A (sequence, group) is split at the same keys for
// each of its heads. P groups share a work-group, one wave each: the split
// runs over (P groups, sequence, key), so the P waves of one CU read the
// same slots' rows of P * HG adjacent heads at about the same time (config
// 2: 193.6 -> 189.2 us, fp8 109.2 -> 106.0 us, P = 4 against one wave per
// work-group). A work-group's two partial slots hold its P * HG heads
// (AttnArgs::part_heads = P * HG). Shares are counted in work units (a
// segment's 32-key tiles plus AttnArgs::seg_cost for starting it), not in
// keys.
// ---------------------------------------------------------------------------
template <typename T, int D, bool F8, int HG, int P>
__global__ __launch_bounds__(64 * P) void decode_grouped(AttnArgs a) {
  using L = KvTile<D, F8>;
  static_assert(HG % 2 == 0, "an even head count keeps every ring stage index a constant");
  __shared__ __attribute__((aligned(1024))) DecodeLds<D, F8> lds_of[P];
  const float vscale = F8 ? a.v_scale : 1.f;
  const int lane = threadIdx.x & 63;
  // Wave pw of the work-group folds head group P * grp + pw: the P waves
  // of a work-group walk the same keys of adjacent groups.
  const int pw = P > 1 ? (int)(threadIdx.x >> 6) : 0;
  DecodeLds<D, F8>& lds = lds_of[pw];
  const int w = blockIdx.x;
  const int ngroups = a.num_kv_heads / (HG * P);
  // Work is counted in units: a segment (sequence, group of HG KV heads)
  // of c keys is ceil(c / 32) tiles plus a.seg_cost units for starting it
  // (its query, its slots, the ring's first tile), the latter first. Every
  // wave takes an equal run of units, so a wave that meets more segments
  // folds fewer tiles, and pieces start and end on tile boundaries.
  const int R = a.seg_cost;
  // The first 64 sequences' key counts stay in registers (lane s holds
  // sequence s's): the scans below and the walk from segment to segment
  // read them without another round trip, which small launches feel.
  const int keys0 = lane < a.batch ? decode_keys(a, lane) : 0;
  // Sequence sq's key count, sq the same on every lane.
  auto keys_at = [&](int sq) -> int { return sq < 64 ? __shfl(keys0, sq, 64) : decode_keys(a, sq); };
  // Lane's sequence s0 + lane (0 past the batch).
  auto lane_units = [&](int s0) -> int64_t {
    const int sq = s0 + lane;
    const int c = s0 == 0 ? keys0 : (sq < a.batch ? decode_keys(a, sq) : 0);
    return c > 0 ? (int64_t)((c + 31) / 32 + R) : 0;
  };
  int64_t total;
  {
    int64_t t = 0;
    for (int s0 = 0; s0 < a.batch; s0 += 64) t += lane_units(s0);
    total = wave_sum_i64(t) * ngroups;
  }
  const int64_t share = (total + a.num_parts - 1) / a.num_parts;
  int64_t pos = (int64_t)w * share;
  if (pos >= total) return;
  const int64_t end = min(pos + share, total);

  // Group-major flattening, (group, sequence, unit), as in decode_balanced:
  // the waves of different groups fold the same slots at about the same time.
  const int64_t per_group = total / ngroups;
  int grp = (int)(pos / per_group);
  const int64_t gpos = pos - (int64_t)grp * per_group;
  // The sequence holding unit `gpos` of the group.
  int seq = 0;
  int64_t before = 0;  // units of the sequences before `seq`
  for (int s0 = 0; s0 < a.batch; s0 += 64) {
    const int64_t c = lane_units(s0);
    int64_t incl = c;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int lo = __shfl_up((int)(incl & 0xffffffff), off, 64);
      const int hi = __shfl_up((int)(incl >> 32), off, 64);
      if (lane >= off) incl += ((int64_t)hi << 32) | (uint32_t)lo;
    }
    const uint64_t hit = __ballot(before + incl > gpos);
    if (hit) {
      const int first = __ffsll((long long)hit) - 1;
      const int64_t excl = __shfl(incl - c, first, 64);
      seq = s0 + first;
      before += excl;
      break;
    }
    before += __shfl(incl, 63, 64);
  }

  const int G = a.groups;
  const TileOffsets<D, F8> off;
  const int esize = F8 ? 1 : (int)sizeof(T);
  const uint32_t row_bytes = (uint32_t)(a.p_s0 * esize);
  const float sc = a.scale * (F8 ? a.k_scale : 1.f) * kLog2eMfma;
  const int64_t head_bytes = a.p_s1 * esize;
  // Partial rows of slot s: ((w * 2 + s) * P + pw) * HG * G onwards.
  float* part_o = a.part_o + ((int64_t)w * 2 * P + pw) * HG * G * a.head_dim;
  float* part_lse = a.part_lse + ((int64_t)w * 2 * P + pw) * HG * G;
  int ctx = keys_at(seq);
  int nu = (ctx + 31) / 32 + R;  // units of each of the sequence's segments
  int u0 = (int)(gpos - before);
  bool first_segment = true;
  while (pos < end) {
    // Units [u0, u1) of this segment are this wave's; its tiles are units
    // R .. nu - 1.
    const int u1 = (int)min((int64_t)nu, (int64_t)u0 + (end - pos));
    const int t_lo = max(u0 - R, 0), t_hi = u1 - R;
    if (t_hi > t_lo) {
      const int key0 = 32 * t_lo;
      const int take = min(32 * t_hi, ctx) - key0;
      const int h0 = (grp * P + pw) * HG;  // the group's first KV head
      if (t_lo == 0 && lane < HG) {
        // This wave holds the context's first key: the work-groups holding
        // its pieces, for each head of the group.
        const int64_t seg = (int64_t)grp * per_group + before;
        a.pieces[(int64_t)seq * a.num_kv_heads + h0 + lane] =
            int4{w, (int)((seg + nu - 1) / share), first_segment ? 0 : 1, 0};
      }
      const int row = decode_row(a, seq);
      DecodeQuery<T, D, F8> q[HG];
      DecodeState st[HG];
#pragma unroll
      for (int h = 0; h < HG; ++h) {
        load_query(a, row, h0 + h, q[h]);
        reset_state(st[h]);
      }
      const char* kbase = static_cast<const char*>(a.kp) + h0 * head_bytes;
      const char* vbase = static_cast<const char*>(a.vp) + h0 * head_bytes;
      const int64_t* srow = a.st + (int64_t)seq * a.st_s;
      const int kb = key0, ke = key0 + take;
      // The sequence's newest K / V rows (a.new_k), when this wave folds its
      // last key: lane (hd, kv, c) holds 16-byte chunk c of head h0 + hd's K
      // (kv 0) or V (kv 1) row, in registers from here on. The pool's rows of
      // that slot are read by no other wave of the launch (other groups read
      // other heads' bytes), so this wave folds the new rows from registers
      // and stores them after its last fold of the segment.
      constexpr int kCh = D / 8;
      const int nw_head = lane / (2 * kCh), nw_kv = (lane / kCh) & 1, nw_c = lane % kCh;
      bool write_new = false;
      u32x4_t new_row = {0u, 0u, 0u, 0u};
      int64_t new_slot = 0;
      if constexpr (!F8) {
        write_new = a.new_k != nullptr && ke == ctx;
        if (write_new) {
          new_slot = srow[ctx - 1];
          if (nw_head < HG) {
            const T* src = static_cast<const T*>(nw_kv ? a.new_v : a.new_k) + (int64_t)seq * a.n_s0 +
                           (int64_t)(h0 + nw_head) * a.n_s1 + 8 * nw_c;
            new_row = *reinterpret_cast<const u32x4_t*>(src);
          }
        }
      }
      for (int c0 = kb; c0 < ke; c0 += kSlotChunk) {
        const int c1 = min(c0 + kSlotChunk, ke);
        const int ntiles = (c1 - c0 + 31) / 32;
        {
          int vals[kSlotChunk / 64 + 1];
#pragma unroll
          for (int k = 0; k < kSlotChunk / 64 + 1; ++k) vals[k] = (int)srow[min(c0 + lane + 64 * k, c1 - 1)];
#pragma unroll
          for (int k = 0; k < kSlotChunk / 64 + 1; ++k) lds.sl[lane + 64 * k] = vals[k];
        }
        // The ring runs over (tile, head) pairs; pair ti * HG + h folds from
        // stage h % 2 while the next pair's loads land in the other stage.
        // Past the chunk the look-ahead re-reads a real tile.
        constexpr int kInFlight = 2 * L::kInsts;
        issue_tile<D, F8>(lds.stage[0], kbase, vbase, lds.sl, row_bytes, 0, lane);
        for (int ti = 0; ti < ntiles; ++ti) {
#pragma unroll
          for (int h = 0; h < HG; ++h) {
            const int nh = h + 1 < HG ? h + 1 : 0;
            const int nt = h + 1 < HG ? ti : ti + 1;
            issue_tile<D, F8>(lds.stage[(h + 1) & 1], kbase + nh * head_bytes, vbase + nh * head_bytes, lds.sl,
                              row_bytes, min(32 * nt, kSlotChunk), lane);
            li_wait_vm<kInFlight>();
            if constexpr (!F8) {
              const int tk = c0 + 32 * ti;  // the tile's first key
              if (write_new && tk + 32 >= ctx) {
                // The tile holding key ctx - 1: its row, and the rows past it
                // (their staged slot repeats that key's; masked, but they
                // must hold finite values), take the new K / V, not what the
                // pool held.
                if (nw_head == h) {
                  const uint32_t base = lds_addr(lds.stage[h & 1]) + (nw_kv ? 32 * L::kRowBytes : 0);
                  for (int r = ctx - 1 - tk; r < 32; ++r) {
                    const uint32_t at = base + (nw_kv ? L::voffset(r, nw_c) : L::offset(r, nw_c));
                    *(__attribute__((address_space(3))) u32x4_t*)(uintptr_t)at = new_row;
                  }
                }
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
              }
            }
            fold_tile<T, D, F8>(lds_addr(lds.stage[h & 1]), c0 + 32 * ti, c1, q[h], sc * q[h].scale, off, st[h]);
          }
        }
        li_wait_vm<0>();
      }
      if (write_new) {
        if (new_slot >= 0 && new_slot < a.num_slots) {
          if (nw_head < HG) {
            char* dst = static_cast<char*>(const_cast<void*>(nw_kv ? a.vp : a.kp)) + new_slot * row_bytes +
                        (int64_t)(h0 + nw_head) * head_bytes + 16 * nw_c;
            *reinterpret_cast<u32x4_t*>(dst) = new_row;
          }
        } else if (lane == 0 && grp == 0 && pw == 0 && a.bad) {
          atomicAdd(a.bad, 1);
        }
      }
      const bool whole = key0 == 0 && take == ctx;
      const int slot = first_segment ? 0 : 1;
#pragma unroll
      for (int h = 0; h < HG; ++h) {
        if (whole) {
          store_state<T, D>(st[h], static_cast<T*>(a.out) + (int64_t)row * a.o_s0 + (int64_t)(h0 + h) * G * a.o_s1,
                            a.o_s1, nullptr, nullptr, 0, G, vscale);
        } else {
          const int64_t r = ((int64_t)slot * P * HG + h) * G;
          store_state<T, D>(st[h], nullptr, 0, part_o + r * a.head_dim, part_lse + r, 1, G, vscale);
        }
      }
      first_segment = false;
    }
    pos += u1 - u0;
    u0 = 0;
    before += nu;
    ++seq;
    while (seq < a.batch && keys_at(seq) == 0) ++seq;
    if (seq >= a.batch) {
      if (++grp == ngroups) break;
      seq = 0;
      before = 0;
      while (seq < a.batch && keys_at(seq) == 0) ++seq;
      if (seq >= a.batch) break;
    }
    ctx = keys_at(seq);
    nu = (ctx + 31) / 32 + R;
  }
}

// Folds the pieces of each (sequence, head) the balanced kernel split across
// waves: w_p = 2^(lse_p - max lse), out = sum w_p o_p / sum w_p
// (paged_kernels.py:574-629, in the log2 domain). One wave per (sequence,
// head), reading the piece range the wave holding the context's first key
// recorded; a context no wave boundary cut was written directly. Up to
// eight pieces (the usual case), every piece's LSE and partial row load at
// once; beyond that, in rounds of 32 pieces whose LSEs and partial rows load
// together.
template <typename T>
__global__ __launch_bounds__(64) void combine_balanced(AttnArgs a) {
  static_assert(kMfmaMaxHeadDim <= 128, "two dims per lane in the many-piece rounds");
  constexpr int kBatch = 8;
  constexpr int kWide = 32;
  const int lane = threadIdx.x;
  const int head = blockIdx.x % a.num_heads;
  const int seq = blockIdx.x / a.num_heads;
  const int G = a.groups, D = a.head_dim;
  const int kvh = head / G, h = head % G;
  // The context length and the piece table are independent loads; both are
  // issued before either is used.
  const int keys = decode_keys(a, seq);
  const int4 info = a.pieces[(int64_t)seq * a.num_kv_heads + kvh];
  if (keys == 0) {
    // A decode row with no key to attend to: the reference's softmax over
    // nothing is 0 / 0. (In a packed pass every sequence that is not a
    // one-query row also counts 0 keys here, and has no row: decode_row is
    // -1 and nothing is written.)
    const int zrow = decode_row(a, seq);
    if (zrow >= 0) {
      T* orow = static_cast<T*>(a.out) + (int64_t)zrow * a.o_s0 + (int64_t)head * a.o_s1;
      for (int d = lane; d < D; d += 64) orow[d] = li_quiet_nan<T>();
    }
    return;
  }
  const int w0 = info.x, w1 = info.y, slot0 = info.z;
  if (w1 <= w0) return;
  const int n = w1 - w0 + 1;
  // Partial row of piece j: wave w0 + j's slot, then (head-grouped waves)
  // the KV head within the slot, then the head within the group.
  const int ph = a.part_heads;
  auto row_of = [&](int j) -> int64_t {
    return (((int64_t)(w0 + j) * 2 + (j == 0 ? slot0 : 0)) * ph + kvh % ph) * G + h;
  };

  const int row = decode_row(a, seq);
  T* orow = static_cast<T*>(a.out) + (int64_t)row * a.o_s0 + (int64_t)head * a.o_s1;
  if (n <= kBatch) {
    // At most kBatch pieces (the usual case): every piece's LSE and partial
    // row load at once, so the fold waits for one round trip, not two.
    constexpr int kMaxC = kMfmaMaxHeadDim / 64;  // dims per lane
    const float lse = lane < n ? a.part_lse[row_of(lane)] : -INFINITY;
    float v[kBatch][kMaxC];
#pragma unroll
    for (int k = 0; k < kBatch; ++k) {
      const float* po = a.part_o + row_of(min(k, n - 1)) * D;
#pragma unroll
      for (int c = 0; c < kMaxC; ++c) {
        const int d = lane + 64 * c;
        v[k][c] = (k < n && d < D) ? po[d] : 0.f;
      }
    }
    const float mx = li_wave_max(lse);
    const float wl = lane < n ? exp2f(lse - mx) : 0.f;
    const float inv = 1.f / li_wave_sum(wl);
    float acc[kMaxC];
#pragma unroll
    for (int c = 0; c < kMaxC; ++c) acc[c] = 0.f;
#pragma unroll
    for (int k = 0; k < kBatch; ++k) {
      const float wt = __shfl(wl, k, 64);
#pragma unroll
      for (int c = 0; c < kMaxC; ++c) acc[c] = fmaf(wt, v[k][c], acc[c]);
    }
#pragma unroll
    for (int c = 0; c < kMaxC; ++c) {
      const int d = lane + 64 * c;
      if (d < D) orow[d] = li_from_float<T>(acc[c] * inv);
    }
    return;
  }

  // More pieces (long contexts over few sequences): rounds of kWide
  // pieces, each round's LSEs and partial rows loaded together (one round
  // trip per round) and folded into a running maximum, sum and row,
  // rescaled when the maximum grows. Lane l holds dims 2l and 2l + 1
  // (head_dim <= 128): one 8-byte load per piece keeps a round's kWide loads
  // within what one wave can have in flight (config 4's combine: 10.1 ->
  // 9.3 us against one 4-byte load per dim; with at most eight pieces the
  // 4-byte loads measured faster, config 2's combine 4.3 against 4.8 us, so
  // that path keeps them).
  const int d0 = 2 * lane;
  const bool has = d0 < D;
  auto piece = [&](int j) -> float2 {
    return has ? *reinterpret_cast<const float2*>(a.part_o + row_of(j) * D + d0) : float2{0.f, 0.f};
  };
  float m = -INFINITY, wsum = 0.f;
  float2 acc = {0.f, 0.f};
  for (int j0 = 0; j0 < n; j0 += kWide) {
    const int jn = min(kWide, n - j0);
    const float lse = lane < jn ? a.part_lse[row_of(j0 + lane)] : -INFINITY;
    float2 v[kWide];
#pragma unroll
    for (int k = 0; k < kWide; ++k) v[k] = piece(j0 + min(k, jn - 1));
    const float nm = fmaxf(m, li_wave_max(lse));
    const float keep = m == -INFINITY ? 0.f : exp2f(m - nm);
    const float wl = lane < jn ? exp2f(lse - nm) : 0.f;
    wsum = wsum * keep + li_wave_sum(wl);
    acc.x *= keep;
    acc.y *= keep;
#pragma unroll
    for (int k = 0; k < kWide; ++k) {
      const float wt = k < jn ? __shfl(wl, k, 64) : 0.f;
      acc.x = fmaf(wt, v[k].x, acc.x);
      acc.y = fmaf(wt, v[k].y, acc.y);
    }
    m = nm;
  }
  if (has) {
    const float inv = 1.f / wsum;
    *reinterpret_cast<uint32_t*>(orow + d0) = li_pack2<T>(acc.x * inv, acc.y * inv);
  }
}

// The combine for launches whose contexts are cut into many pieces (few
// segments over the whole grid: a long context at a small batch). NW waves
// share each (sequence, head): wave v folds pieces v, v + NW, ... in rounds
// of 32 loaded together, as the single-wave rounds above do, and wave 0
// merges the NW running states through LDS. A context the grid cut into
// 130 pieces then takes two rounds per wave instead of five in a row (one
// 4096-key context at batch 1: 23.6 -> 12.9 us a call; config 4: 339.3 ->
// 336.1 us; 4 waves measured faster than 2 or 8 over 1-16k keys).
template <typename T, int NW>
__global__ __launch_bounds__(64 * NW) void combine_wide(AttnArgs a) {
  static_assert(kMfmaMaxHeadDim <= 128, "two dims per lane");
  constexpr int kWide = 32;
  const int lane = threadIdx.x & 63;
  const int v = (int)(threadIdx.x >> 6);
  const int head = blockIdx.x % a.num_heads;
  const int seq = blockIdx.x / a.num_heads;
  const int G = a.groups, D = a.head_dim;
  const int kvh = head / G, h = head % G;
  const int keys = decode_keys(a, seq);
  const int4 info = a.pieces[(int64_t)seq * a.num_kv_heads + kvh];
  const int row = decode_row(a, seq);
  T* orow = row >= 0 ? static_cast<T*>(a.out) + (int64_t)row * a.o_s0 + (int64_t)head * a.o_s1 : nullptr;
  if (keys == 0) {
    // No key to attend to: 0 / 0, as combine_balanced writes it.
    if (v == 0 && orow)
      for (int d = lane; d < D; d += 64) orow[d] = li_quiet_nan<T>();
    return;
  }
  const int w0 = info.x, w1 = info.y, slot0 = info.z;
  if (w1 <= w0) return;
  const int n = w1 - w0 + 1;
  const int ph = a.part_heads;
  auto row_of = [&](int j) -> int64_t {
    return (((int64_t)(w0 + j) * 2 + (j == 0 ? slot0 : 0)) * ph + kvh % ph) * G + h;
  };
  const int d0 = 2 * lane;
  const bool has = d0 < D;
  float m = -INFINITY, wsum = 0.f;
  float2 acc = {0.f, 0.f};
  // This wave's pieces: v, v + NW, ...; its i-th is piece v + NW * i.
  const int mine = n > v ? (n - v + NW - 1) / NW : 0;
  for (int i0 = 0; i0 < mine; i0 += kWide) {
    const int jn = min(kWide, mine - i0);
    const float lse = lane < jn ? a.part_lse[row_of(v + NW * (i0 + lane))] : -INFINITY;
    float2 x[kWide];
#pragma unroll
    for (int k = 0; k < kWide; ++k) {
      const int j = v + NW * (i0 + min(k, jn - 1));
      x[k] = has ? *reinterpret_cast<const float2*>(a.part_o + row_of(j) * D + d0) : float2{0.f, 0.f};
    }
    const float nm = fmaxf(m, li_wave_max(lse));
    const float keep = m == -INFINITY ? 0.f : exp2f(m - nm);
    const float wl = lane < jn ? exp2f(lse - nm) : 0.f;
    wsum = wsum * keep + li_wave_sum(wl);
    acc.x *= keep;
    acc.y *= keep;
#pragma unroll
    for (int k = 0; k < kWide; ++k) {
      const float wt = k < jn ? __shfl(wl, k, 64) : 0.f;
      acc.x = fmaf(wt, x[k].x, acc.x);
      acc.y = fmaf(wt, x[k].y, acc.y);
    }
    m = nm;
  }
  __shared__ float s_m[NW], s_w[NW];
  __shared__ float2 s_acc[NW][64];
  if (lane == 0) {
    s_m[v] = m;
    s_w[v] = wsum;
  }
  s_acc[v][lane] = acc;
  __syncthreads();
  if (v != 0 || !has || !orow) return;
  float mx = -INFINITY;
#pragma unroll
  for (int u = 0; u < NW; ++u) mx = fmaxf(mx, s_m[u]);
  float tot = 0.f;
  float2 o = {0.f, 0.f};
#pragma unroll
  for (int u = 0; u < NW; ++u) {
    const float sc = s_m[u] == -INFINITY ? 0.f : exp2f(s_m[u] - mx);
    tot = fmaf(s_w[u], sc, tot);
    o.x = fmaf(s_acc[u][lane].x, sc, o.x);
    o.y = fmaf(s_acc[u][lane].y, sc, o.y);
  }
  const float inv = 1.f / tot;
  *reinterpret_cast<uint32_t*>(orow + d0) = li_pack2<T>(o.x * inv, o.y * inv);
}

// ---------------------------------------------------------------------------
// Short decode: one work-group of NW waves per (sequence, KV head), for
// launches whose every context is short (the slot table's width bounds them).
// Wave v folds the v-th of NW equal, tile-aligned runs of the context; the
// waves then merge their softmax states through LDS (each state's rows
// weighted by 2^(m_v - max m), as the reference's cross-partition reduce
// weights its partitions, liteinfer/models/paged_kernels.py:574-629) and
// write the normalised rows. One launch, no partial rows in HBM and no
// combine launch: a call is its loads' round trips and one launch. Over a
// 16-bit pool it also writes the step's newest K / V rows (a.new_k).
// ---------------------------------------------------------------------------
template <typename T, int D, bool F8, int NW>
__global__ __launch_bounds__(64 * NW) void decode_short(AttnArgs a) {
  using Lds = DecodeLds<D, F8, kShortChunk>;
  static_assert(sizeof(Lds::stage) >= 16 * D * sizeof(float), "a wave's state fits its stages");
  __shared__ __attribute__((aligned(1024))) Lds lds_of[NW];
  __shared__ float s_m[NW][16], s_l[NW][16];
  const int lane = threadIdx.x & 63, wv = (int)(threadIdx.x >> 6);
  const int n = lane & 15, g = lane >> 4;
  const int seq = blockIdx.x / a.num_kv_heads, kvh = blockIdx.x % a.num_kv_heads;
  const int G = a.groups;
  const int keys = decode_keys(a, seq);
  const int row = decode_row(a, seq);
  if (row < 0) return;
  // Wave wv's run: [wv * per, (wv + 1) * per) of the context, whole tiles.
  const int per = ((keys + NW - 1) / NW + 31) / 32 * 32;
  const int kb = min(wv * per, keys), ke = min(kb + per, keys);
  if constexpr (!F8) {
    if (a.new_k != nullptr && kb < ke && ke == keys) {
      // This wave folds the context's last key: the step's new K and V rows
      // of this KV head go to that key's slot first (lane (kv, c) stores
      // 16-byte chunk c of K or V), and the wave waits for the stores before
      // its loads read the slot back. No other work-group reads these bytes
      // (other KV heads' rows, other sequences' slots).
      constexpr int kCh = D / 8;
      const int64_t slot = a.st[(int64_t)seq * a.st_s + keys - 1];
      if (lane < 2 * kCh) {
        const int kv = lane / kCh, c = lane % kCh;
        if (slot >= 0 && slot < a.num_slots) {
          const T* src = static_cast<const T*>(kv ? a.new_v : a.new_k) + (int64_t)seq * a.n_s0 +
                         (int64_t)kvh * a.n_s1 + 8 * c;
          char* dst = static_cast<char*>(const_cast<void*>(kv ? a.vp : a.kp)) +
                      (slot * a.p_s0 + (int64_t)kvh * a.p_s1) * (int64_t)sizeof(T) + 16 * c;
          *reinterpret_cast<u32x4_t*>(dst) = *reinterpret_cast<const u32x4_t*>(src);
        } else if (lane == 0 && kvh == 0 && a.bad) {
          atomicAdd(a.bad, 1);  // once per sequence, as the slot-write counts
        }
      }
      li_wait_vm<0>();
    }
  }
  DecodeState st;
  reset_state(st);
  if (ke > kb) {
    DecodeQuery<T, D, F8> q;
    load_query(a, row, kvh, q);
    fold_keys<T, D, F8>(a, lds_of[wv], q, seq, kvh, kb, ke, st);
  }
  // Each wave's state into its own stages (its loads have drained): head n's
  // accumulator row, its running maximum and its denominator.
  const float lt = li_group_sum(st.l);
  float* acc = reinterpret_cast<float*>(lds_of[wv].stage);
  if (n < G) {
#pragma unroll
    for (int blk = 0; blk < D / 16; ++blk)
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[n * D + 16 * blk + 4 * g + r] = st.acc[blk][r];
    if (g == 0) {
      s_m[wv][n] = st.m;
      s_l[wv][n] = lt;
    }
  }
  __syncthreads();
  const float vscale = F8 ? a.v_scale : 1.f;
  T* orow = static_cast<T*>(a.out) + (int64_t)row * a.o_s0 + (int64_t)kvh * G * a.o_s1;
  for (int e = threadIdx.x; e < G * D; e += 64 * NW) {
    const int h = e / D, d = e % D;
    if (keys == 0) {  // no key to attend to: the reference's softmax over nothing is 0 / 0
      orow[(int64_t)h * a.o_s1 + d] = li_quiet_nan<T>();
      continue;
    }
    {
      float mx = -INFINITY;
#pragma unroll
      for (int v = 0; v < NW; ++v) mx = fmaxf(mx, s_m[v][h]);
      float num = 0.f, den = 0.f;
#pragma unroll
      for (int v = 0; v < NW; ++v) {
        // A wave with no keys holds m = -inf, l = 0 and zero rows.
        const float wgt = s_l[v][h] > 0.f ? __builtin_amdgcn_exp2f(s_m[v][h] - mx) : 0.f;
        num = fmaf(wgt, reinterpret_cast<const float*>(lds_of[v].stage)[h * D + d], num);
        den = fmaf(wgt, s_l[v][h], den);
      }
      orow[(int64_t)h * a.o_s1 + d] = li_from_float<T>(num * (vscale / den));
    }
  }
}

bool rows_aligned(const void* p, int64_t s0, int64_t s1, int esize) {
  return aligned16(p) && (s0 * esize) % 16 == 0 && (s1 * esize) % 16 == 0;
}

}  // namespace

bool decode_mfma_applies(const AttnArgs& a, int dtype) {
  if (dtype != LI_BF16 && dtype != LI_F16) return false;
  if (a.head_dim != 64 && a.head_dim != 128) return false;
  if (a.kv_fp8 && a.head_dim != 128) return false;
  if (a.groups < 1 || a.groups > 16) return false;
  const int pe = a.kv_fp8 ? 1 : 2;
  return rows_aligned(a.q, a.q_s0, a.q_s1, 2) && rows_aligned(a.out, a.o_s0, a.o_s1, 2) &&
         rows_aligned(a.kp, a.p_s0, a.p_s1, pe) && rows_aligned(a.vp, a.p_s0, a.p_s1, pe);
}

int launch_decode_mfma(const AttnArgs& a, int dtype, hipStream_t s) {
  const bool balanced = a.part_len < 0;
  const int64_t blocks = balanced ? a.num_parts : (int64_t)a.batch * a.num_kv_heads * a.num_parts;
  if (blocks == 0) return LI_OK;
  if (blocks > 0x7fffffffLL) return fail(LI_EUNSUPPORTED, "decode grid of %lld blocks is too large", (long long)blocks);
  const dim3 grid((unsigned)blocks), block(64);
#define LI_DECODE_LAUNCH(T, D, F8)                                                                   \
  do {                                                                                               \
    if (balanced && a.part_heads == kDecodeHeadGroup)                                                \
      hipLaunchKernelGGL((decode_grouped<T, D, F8, kDecodeHeadGroup, 1>), grid, block, 0, s, a);     \
    else if (balanced && a.part_heads == 2 * kDecodeHeadGroup)                                       \
      hipLaunchKernelGGL((decode_grouped<T, D, F8, kDecodeHeadGroup, 2>), grid, dim3(128), 0, s, a); \
    else if (balanced && a.part_heads == 4 * kDecodeHeadGroup)                                       \
      hipLaunchKernelGGL((decode_grouped<T, D, F8, kDecodeHeadGroup, 4>), grid, dim3(256), 0, s, a); \
    else if (balanced) hipLaunchKernelGGL((decode_balanced<T, D, F8>), grid, block, 0, s, a);        \
    else hipLaunchKernelGGL((decode_partitioned<T, D, F8>), grid, block, 0, s, a);                   \
  } while (0)
  if (a.kv_fp8) {
    if (dtype == LI_BF16) LI_DECODE_LAUNCH(li_bf16, 128, true);
    else LI_DECODE_LAUNCH(li_f16, 128, true);
  } else if (dtype == LI_BF16) {
    if (a.head_dim == 128) LI_DECODE_LAUNCH(li_bf16, 128, false);
    else LI_DECODE_LAUNCH(li_bf16, 64, false);
  } else {
    if (a.head_dim == 128) LI_DECODE_LAUNCH(li_f16, 128, false);
    else LI_DECODE_LAUNCH(li_f16, 64, false);
  }
#undef LI_DECODE_LAUNCH
  if (int rc = check_launch("decode_mfma")) return rc;
  return balanced ? launch_combine_balanced(a, dtype, s) : LI_OK;
}

bool decode_short_applies(const AttnArgs& a, int dtype, int max_context) {
  if (a.qsl || !decode_mfma_applies(a, dtype)) return false;
  const int64_t segments = (int64_t)a.batch * a.num_kv_heads;
  // Measured against the balanced split (uniform contexts at 32 / 8 heads,
  // head_dim 64 and 128, 1 to 128 sequences, one graph of 20 calls): the
  // short kernel wins while its work-groups fit about two rounds of the chip
  // (segments x width up to 2^19 keys) and no wave folds more than about
  // 256 keys (width up to 1024; up to 2048 once there are 128 segments, so
  // that a wave's run stays short).
  if (segments * max_context > kShortMaxKeySegments) return false;
  return max_context <= kShortMaxWidth || (max_context <= 2 * kShortMaxWidth && segments >= kShortWideSegments);
}

int launch_decode_short(const AttnArgs& a, int dtype, hipStream_t s) {
  const int64_t blocks = (int64_t)a.batch * a.num_kv_heads;
  if (blocks == 0) return LI_OK;
  if (blocks > 0x7fffffffLL) return fail(LI_EUNSUPPORTED, "decode grid of %lld blocks is too large", (long long)blocks);
  const dim3 grid((unsigned)blocks);
  // Waves per work-group: as many as the LDS holds (two tile stages each).
  if (a.kv_fp8) {
    if (dtype == LI_BF16) hipLaunchKernelGGL((decode_short<li_bf16, 128, true, 8>), grid, dim3(512), 0, s, a);
    else hipLaunchKernelGGL((decode_short<li_f16, 128, true, 8>), grid, dim3(512), 0, s, a);
  } else if (dtype == LI_BF16) {
    if (a.head_dim == 128) hipLaunchKernelGGL((decode_short<li_bf16, 128, false, 4>), grid, dim3(256), 0, s, a);
    else hipLaunchKernelGGL((decode_short<li_bf16, 64, false, 8>), grid, dim3(512), 0, s, a);
  } else {
    if (a.head_dim == 128) hipLaunchKernelGGL((decode_short<li_f16, 128, false, 4>), grid, dim3(256), 0, s, a);
    else hipLaunchKernelGGL((decode_short<li_f16, 64, false, 8>), grid, dim3(512), 0, s, a);
  }
  return check_launch("decode_short");
}

int launch_combine_balanced(const AttnArgs& a, int dtype, hipStream_t s) {
  const int64_t cblocks = (int64_t)a.batch * a.num_heads;
  if (cblocks == 0) return LI_OK;
  // Segments (sequence, group of part_heads KV heads) against the grid's
  // shares: fewer than one segment per kWideShare shares means most
  // segments are cut into more than kWideShare pieces.
  constexpr int kWideShare = 8;
  const int64_t segments = (int64_t)a.batch * (a.num_kv_heads / std::max(a.part_heads, 1));
  if (segments * kWideShare < a.num_parts) {
    if (dtype == LI_BF16)
      hipLaunchKernelGGL((combine_wide<li_bf16, kCombineWaves>), dim3((unsigned)cblocks), dim3(64 * kCombineWaves), 0,
                         s, a);
    else
      hipLaunchKernelGGL((combine_wide<li_f16, kCombineWaves>), dim3((unsigned)cblocks), dim3(64 * kCombineWaves), 0,
                         s, a);
    return check_launch("combine_wide");
  }
  if (dtype == LI_BF16) hipLaunchKernelGGL(combine_balanced<li_bf16>, dim3((unsigned)cblocks), dim3(64), 0, s, a);
  else hipLaunchKernelGGL(combine_balanced<li_f16>, dim3((unsigned)cblocks), dim3(64), 0, s, a);
  return check_launch("combine_balanced");
}

}  // namespace li
