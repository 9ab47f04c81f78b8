// Packed / chunked prefill on CDNA4 matrix cores (bf16 / fp16, head_dim 64 or
// 128, up to 16 query heads per KV head).
//
// Same attention as liteinfer's prefill kernel (liteinfer/models/
// paged_kernels.py:416-459 with _attend_query_block, :291-371): a
// sequence's queries are the last positions of its context, each sees the
// keys up to its own position, the online softmax runs in fp32 and the
// weights are rounded to the value dtype before they multiply V.
//
// Two kernels: prefill_pp (16-bit pools), where the two waves of each SIMD
// run half a stage apart so that one feeds the matrix core while the other
// runs its softmax (described above the kernel), and prefill_mfma (fp8
// pools), where all eight waves fold each stage in lockstep, described here.
//
// A unit of work is (sequence, KV head, block of 256 / G query tokens),
// folded by one work-group of 8 waves (two per SIMD). Its 256 rows are
// (query token, head) pairs, head fastest, so the G heads that share a KV
// head read each K/V tile once; wave w owns rows 32w..32w+31 as two 16-row
// MFMA blocks. The keys [0, last query's position] stream through LDS 64 at
// a time, loaded straight into LDS by all eight waves (two stages, so the
// next 64 keys land while these are folded), in the 32-key tile layout of
// li_mfma.h. Per stage and 16 rows:
//
//   S^T = K Q^T     A = K rows from LDS, B = the rows' Q^T kept in registers.
//                   Lane (n, g) gets the scores of keys 16b + 4g .. + 3 of
//                   key block b = 0..3 for row n.
//   softmax         one running-max update per row over all 64 keys.
//   O^T += V^T P^T  B = P^T is a 32-key tile's 8 weights as they are; A =
//                   V^T comes straight out of LDS through transposing reads
//                   (ds_read_b64_tr_b16, li_read_vt's addressing), shared by
//                   both row blocks. One more MFMA against a block of ones
//                   gives each row's sum of weights.
//
// Every LDS read is one instruction from a per-lane address fixed for the
// whole kernel plus an immediate offset (the loop body covers both stages,
// so stage bases are constants); a tile's V^T fragments, and the next key
// block's K fragments, are read as one batch ahead of the MFMAs that
// consume them, so the LDS latency is paid once per batch.
//
// A row's visibility is key <= its position; the mask is a compare per
// score, applied only to stages that reach past the block's first query
// position (the diagonal). Padding rows (past the block or the sequence) see
// every key with a zero query, so they stay finite, and are never stored; a
// wave whose rows are all padding only helps load the stages.
//
// Scheduling: a persistent grid of one work-group per CU. prefill_order
// lists every non-empty query block, by sequence, heaviest first; work-groups pull
// (block, KV head) units from queues in that order through an atomic
// counter, so long units start first, short ones fill in behind, and no
// work-group is launched for an empty block. With num_kv_heads a multiple of
// 8 there is one queue per XCD (work-group i runs on XCD i % 8) holding the
// KV heads q, q + 8, ...: every block of one KV head is folded on one XCD and
// reuses that head's K/V from the XCD's L2.
#include "decode_wave.h"
#include "li_attention.h"
#include "li_mfma.h"

#include <type_traits>

namespace li {
namespace {

// A work-group has W waves and 32 W (query, head) rows. Eight waves (two per
// SIMD) share each K/V stage: half the LDS fill per MFMA of four.
constexpr int kWaves = 8;
constexpr int kMinRows = 32 * kWaves;  // rows of a work-group
constexpr int kStageKeys = 64;

// The prefill's K/V loads keep their lines in L2 (no non-temporal hint):
// the other query blocks of a sequence, folded at about the same time on
// the same XCD, read the same rows (config 3's chunks: 338 -> 318 us, 8
// chunks of 2048 over 8192 keys: 2065 -> 1947 us). Choosing the hint per
// unit (streaming the single-block sequences) measured slower: the branch
// costs more scalar registers than the hint saves.
__device__ __forceinline__ void dma16_kv(const char* k, const char* v, uint32_t kdst, uint32_t vdst) {
  dma16<false>(k, kdst);
  dma16<false>(v, vdst);
}

// Issues this wave's share of the direct-to-LDS loads of the 64 keys whose
// first key is entry `t` of the staged slots. The stage takes 2 * kInsts
// instructions each for K and V (kInsts per 32-key half); wave w issues
// pairs p = w * kPer .. w * kPer + kPer - 1, pair p being instruction
// p % kInsts of half p / kInsts.
template <typename L, int W>
__device__ __forceinline__ void issue_stage(uint32_t stage, const char* __restrict__ kpool,
                                            const char* __restrict__ vpool, const int* __restrict__ sl,
                                            uint32_t row_bytes, int t, int lane, int w) {
  constexpr int kPer = 2 * L::kInsts / W;
  static_assert(kPer >= 1 && kPer * W == 2 * L::kInsts, "waves must split the stage's loads evenly");
  const int rr = lane / L::kCh, nn = lane % L::kCh;
  // All slot reads first: each load below is an asm statement with a memory
  // clobber, so a read placed after one would wait for its own round trip.
  uint32_t slot[kPer];
#pragma unroll
  for (int ii = 0; ii < kPer; ++ii) {
    const int p = w * kPer + ii, half = p / L::kInsts, i = p % L::kInsts;
    slot[ii] = (uint32_t)sl[t + 32 * half + rr * L::kInsts + i];
  }
#pragma unroll
  for (int ii = 0; ii < kPer; ++ii) {
    const int p = w * kPer + ii, half = p / L::kInsts, i = p % L::kInsts;
    const int key = rr * L::kInsts + i;
    const uint32_t dst = stage + half * L::kTileBytes + i * 1024;
    // Lane nn writes slot nn of its row: global chunk nn ^ swizzle(key).
    dma16_kv(row_ptr(kpool + 16 * (nn ^ L::kswizzle(key)), slot[ii], row_bytes),
             row_ptr(vpool + 16 * (nn ^ L::vswizzle(key)), slot[ii], row_bytes), dst, dst + 32 * L::kRowBytes);
  }
}

// An fp8 stage (raw, F8Tile layout, two 32-key tiles) into the 16-bit stage
// the fold reads (TileLayout<128>): each 16-byte chunk of 16 e4m3 values of
// a key becomes its two 16-byte chunks of bf16 / fp16, K and V rows with
// their own swizzles. Every thread of the work-group converts its share, so
// each value is converted once for all the waves that fold it.
template <typename T, int W>
__device__ __forceinline__ void convert_stage(uint32_t raw, uint32_t dst, int tid) {
  using Frag = typename Mfma<T>::Frag;
  using L = TileLayout<128>;
  typedef uint32_t u4 __attribute__((ext_vector_type(4)));
#pragma unroll
  for (int u = tid; u < 1024; u += 64 * W) {
    const int tile = u >> 9, kv = (u >> 8) & 1, key = (u >> 3) & 31, c8 = u & 7;
    const uint32_t src = raw + tile * F8Tile::kTileBytes + kv * 32 * F8Tile::kRowBytes +
                         (kv ? F8Tile::voffset(key, c8) : F8Tile::offset(key, c8));
    const u4 x = *(const __attribute__((address_space(3))) u4*)(uintptr_t)src;
    const uint32_t d = dst + tile * L::kTileBytes + kv * 32 * L::kRowBytes;
    const uint32_t lo = d + (kv ? L::voffset(key, 2 * c8) : L::offset(key, 2 * c8));
    const uint32_t hi = d + (kv ? L::voffset(key, 2 * c8 + 1) : L::offset(key, 2 * c8 + 1));
    *(__attribute__((address_space(3))) Frag*)(uintptr_t)lo = f8x8_to_frag<Frag>(x[0], x[1]);
    *(__attribute__((address_space(3))) Frag*)(uintptr_t)hi = f8x8_to_frag<Frag>(x[2], x[3]);
  }
}

// Work-groups of a prefill launch that also serves the pass's one-query
// rows (prefill_pp_rows, prefill_mfma_rows) fold them first: the first
// `row_groups` work-groups (prefill_order's count) run the balanced decode
// split `d`, kRowWaves waves each, in the LDS of their rows[] member, then
// all of the work-group's waves meet at a barrier before the prefill work
// reuses that LDS. The LDS of four decode waves fits in a prefill
// work-group's. (Three waves with three ring stages each, two tiles in
// flight per wave, measured no faster: config 3 flat at 310-315 us from 48
// row work-groups.)

template <typename T, int D, bool F8, typename Shared>
__device__ __forceinline__ void fold_rows_first(const AttnArgs& a, const AttnArgs& d, Shared& lds) {
  // prefill_order's count (prefill_row_groups, at most a.row_groups_max,
  // which the host holds to the grid and to the workspace's partial slots),
  // held to both again here: every row wave is then a wave of the grid and
  // has partial slots in the workspace (d.num_parts).
  const int row_groups = min(min(__builtin_amdgcn_readfirstlane(a.queue[kPrefillQueues + 1]), (int)gridDim.x),
                             d.num_parts / kRowWaves);
  const int wg = (int)blockIdx.x;
  if (wg < row_groups) {
    const int rw = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    if (rw < kRowWaves) {
      const int waves = row_groups * kRowWaves;
      int v = wg * kRowWaves + rw;
      // The split runs head-major: wave v + waves / Hkv starts at about the
      // key wave v starts at, one KV head on. The kRowWaves waves of a
      // work-group take such shares of kRowWaves adjacent heads, so one CU
      // reads those heads' rows of each slot together (config 3: 308-311
      // -> 302-307 us against consecutive shares of one head).
      if (d.num_kv_heads % kRowWaves == 0 && waves % d.num_kv_heads == 0) {
        const int per_head = waves / d.num_kv_heads;
        v = ((wg / per_head) * kRowWaves + rw) * per_head + wg % per_head;
      }
      decode_balanced_wave<T, D, F8>(d, v, (int64_t)waves, lds.rows[rw]);
    }
    // (Every row wave's loads have landed: its folds consumed them.)
    __syncthreads();
  }
}

// The direct schedule (a pass whose every unit has a work-group of its own,
// no work list): the block prefill_order would list at index `want` (every
// sequence's blocks in sequence order, the same entry format), found by one
// full wave's scan of the sequences' query counts (at most 64 sequences);
// {-1, 0, 0, 0} past the last block. Every lane returns the entry.
__device__ __forceinline__ int4 direct_entry(const AttnArgs& a, int want) {
  const int lane = (int)(threadIdx.x & 63);
  int4 e{0, 0, 0, 0};
  int nb = 0;
  if (lane < a.batch) {
    const int first = a.qsl[lane], next = a.qsl[lane + 1];
    e = int4{first, next - first, a.ctx[lane], 0};
    if (e.y > 0 && !(e.y == 1 && a.single_query_elsewhere)) nb = min((e.y + a.block_q - 1) / a.block_q, a.num_qblocks);
  }
  int incl = nb;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int up = __shfl_up(incl, off, 64);
    if (lane >= off) incl += up;
  }
  const uint64_t hit = __ballot(incl > want);
  if (hit == 0) return int4{-1, 0, 0, 0};
  const int sq = __ffsll((long long)hit) - 1;
  const int qb = want - (__shfl(incl, sq, 64) - __shfl(nb, sq, 64));
  return int4{sq * a.num_qblocks + qb, __shfl(e.x, sq, 64), __shfl(e.y, sq, 64), __shfl(e.z, sq, 64)};
}

// Keys whose slots the lockstep kernel stages in LDS at a time (restaging
// costs a pipeline drain, so chunks are long).
constexpr int kLockstepChunk = 4096;

// LDS of one lockstep work-group: staged slots, the converted (or, for
// 16-bit pools, loaded) stages, an fp8 pool's raw stages, and its unit.
template <int D, bool F8>
struct LockstepLds {
  __attribute__((aligned(16))) int sl[kLockstepChunk + kStageKeys];
  __attribute__((aligned(1024))) char stages[2][2 * TileLayout<D>::kTileBytes];
  __attribute__((aligned(1024))) char raw[F8 ? 2 : 1][F8 ? 2 * F8Tile::kTileBytes : 16];
  int unit;
  int4 entry;  // the direct schedule's unit
};

template <int D, bool F8>
union LockstepShared {
  LockstepLds<D, F8> ls;
  DecodeLds<D, F8> rows[kRowWaves];
};

// F8: the pool is fp8 (e4m3, head_dim 128); its stages land raw and are
// converted in LDS (convert_stage) before the fold, which is the same.
// With kRows (prefill_mfma_rows) the first work-groups fold the pass's
// one-query rows first (fold_rows_first).
template <typename T, int D, int W, bool F8, bool kRows, bool kDirect = false>
__device__ __forceinline__ void prefill_mfma_body(AttnArgs a, const AttnArgs& d) {
  __shared__ __attribute__((aligned(1024))) LockstepShared<D, F8> lds;
  if constexpr (kRows) fold_rows_first<T, D, F8>(a, d, lds);
  using M = Mfma<T>;
  using Frag = typename M::Frag;
  using L = TileLayout<D>;
  using LS = std::conditional_t<F8, F8Tile, TileLayout<D>>;  // layout the loads fill
  static_assert(!F8 || D == 128, "fp8 pools at head_dim 128");
  constexpr int kSteps = D / 32;
  constexpr int kDmaPerStage = 2 * (2 * LS::kInsts / W);
  constexpr int kChunk = kLockstepChunk;
  auto& sl = lds.ls.sl;
  auto& stages = lds.ls.stages;
  auto& raw = lds.ls.raw;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave index, uniform
  const int n = lane & 15, g = lane >> 4;

  // Persistent grid: work-groups take (query block, KV head) units from
  // their queue until it runs dry. With num_kv_heads a multiple of 8 there
  // is one queue per XCD (work-group i runs on XCD i % 8) holding the units
  // of KV heads q, q + 8, ..., so every block of one KV head is folded on one
  // XCD and reuses that head's K/V from its L2; otherwise one queue. Units
  // come in the work list's order, heaviest block first: a work-group that
  // finishes early takes the next heaviest unit left.
  const int nqueues = a.num_kv_heads % kPrefillQueues == 0 ? kPrefillQueues : 1;
  const int qi = (int)(blockIdx.x % (unsigned)nqueues);
  const int heads_per_queue = a.num_kv_heads / nqueues;
  // The direct schedule: work-group wg takes unit wg / nqueues of its queue
  // (direct_entry) and nothing after it.
  constexpr int kNoUnit = 0x7fffffff;
  const int units = kDirect ? kNoUnit : a.queue[kPrefillQueues] * heads_per_queue;
  int& s_unit = lds.ls.unit;
  bool claimed = false;
  for (;;) {
  if (kDirect && claimed) break;
  __syncthreads();  // every wave is done with the previous unit's LDS
  if constexpr (kDirect) {
    claimed = true;
    if (w == 0) {
      const int u = (int)(blockIdx.x / (unsigned)nqueues);
      const int4 e = direct_entry(a, u / heads_per_queue);
      if (lane == 0) {
        s_unit = e.x < 0 ? kNoUnit : u;
        lds.ls.entry = e;
      }
    }
  } else if (tid == 0) {
    s_unit = atomicAdd(&a.queue[qi], 1);
  }
  __syncthreads();
  const int unit = s_unit;
  if (unit >= units) break;
  // The block's descriptor: one 16-byte read.
  const int4 entry = kDirect ? lds.ls.entry : a.work[unit / heads_per_queue];
  const int item = entry.x;
  const int seq = item / a.num_qblocks;
  const int qblock = item % a.num_qblocks;
  const int kvh = qi + nqueues * (unit % heads_per_queue);

  const int first_tok = entry.y;
  const int nq = entry.z;
  const int bq = a.block_q;  // query tokens per block = 32 W / groups
  // Blocks are cut from the end of the chunk: block nblk - 1 ends at its
  // last query and only block 0 (the one with the fewest keys) is partial.
  const int nblk = (nq + bq - 1) / bq;
  if (qblock >= nblk) continue;
  const int q1 = nq - (nblk - 1 - qblock) * bq;
  const int q0 = max(q1 - bq, 0);
  if (nq == 1 && a.single_query_elsewhere) continue;  // the decode kernel serves it
  const int ctx = entry.w;
  const int pos0 = ctx - nq;   // position of the sequence's first query
  const int kend = pos0 + q1;  // keys this block reads: [0, kend)
  const int G = a.groups;

  // This lane's two rows (one per 16-row block).
  int pos[2];
  bool real[2];
  int tok[2], head[2];
  Frag qf[2][kSteps];
#pragma unroll
  for (int nb = 0; nb < 2; ++nb) {
    const int row = 32 * w + 16 * nb + n;
    const int ql = row / G;
    real[nb] = row < bq * G && q0 + ql < q1;
    pos[nb] = real[nb] ? pos0 + q0 + ql : kend;
    tok[nb] = first_tok + q0 + ql;
    head[nb] = kvh * G + row % G;
    const T* qrow = static_cast<const T*>(a.q) + (int64_t)tok[nb] * a.q_s0 + (int64_t)head[nb] * a.q_s1 + 8 * g;
#pragma unroll
    for (int j = 0; j < kSteps; ++j) {
      if (real[nb]) {
        qf[nb][j] = *reinterpret_cast<const Frag*>(qrow + 32 * j);
      } else {
        qf[nb][j] = Frag{};
      }
    }
  }

  // Last key each row sees: its own position (padding rows: the block's last key).
  const int lim[2] = {min(pos[0], kend - 1), min(pos[1], kend - 1)};
  // Below the block's first query position every row sees every key.
  const int lim_lo = min(pos0 + q0, kend - 1);
  // A wave whose 32 rows are all padding (a sequence's last, partial block)
  // only helps load the stages; it folds nothing, leaving its SIMD to the
  // other wave there.
  const bool idle = 32 * w >= (q1 - q0) * G;

  const int esize = F8 ? 1 : (int)sizeof(T);  // bytes per pool element
  const char* kpool = static_cast<const char*>(a.kp) + (int64_t)kvh * a.p_s1 * esize;
  const char* vpool = static_cast<const char*>(a.vp) + (int64_t)kvh * a.p_s1 * esize;
  const int64_t* srow = a.st + (int64_t)seq * a.st_s;
  const uint32_t row_bytes = (uint32_t)(a.p_s0 * esize);
  // An fp8 pool stores K / k_scale and V / v_scale: the scales multiply the
  // scores and the outputs.
  const float sc = a.scale * (F8 ? a.k_scale : 1.f) * kLog2eMfma;

  // acc[nb][blk] for blk < D / 16: dims 16 blk + 4g .. of the lane's row;
  // acc[nb][D / 16]: the row's softmax denominator, as the MFMA product of
  // the weights with a block of ones (every element holds the same sum).
  float m[2] = {-INFINITY, -INFINITY};
  floatx4_t acc[2][D / 16 + 1];
#pragma unroll
  for (int nb = 0; nb < 2; ++nb)
#pragma unroll
    for (int i = 0; i < D / 16 + 1; ++i) acc[nb][i] = floatx4_t{0.f, 0.f, 0.f, 0.f};
  const Frag ones = li_ones<Frag>();

  // Per-lane LDS byte offsets within a 32-key tile, fixed for the whole
  // kernel; a tile's and a stage's base are compile-time constants below, so
  // every LDS read is one instruction with an immediate offset.
  //   K operand of key block b (keys 16b..16b+15 of a tile), step j: key n,
  //   chunk 4j + g. Key 16 + n sits L::kRow16 bytes below key n with the
  //   same swizzle, so b only adds an immediate.
  //   V^T operand of dims 16 blk..: li_read_vt's two addresses, the second
  //   again L::kRow16 bytes below the first.
  uint32_t koff[kSteps], voff[D / 16];
  {
    const uint32_t base = lds_addr(&stages[0][0]);
#pragma unroll
    for (int j = 0; j < kSteps; ++j) koff[j] = base + L::offset(n, 4 * j + g);
    const int s16 = lane & 15, a4 = s16 & 3, key = 4 * g + (s16 >> 2);
#pragma unroll
    for (int blk = 0; blk < D / 16; ++blk) voff[blk] = base + L::voffset(key, 2 * blk + (a4 >> 1)) + 8 * (a4 & 1);
  }

  // The fold of one 64-key stage in three parts: scores (MFMA), the online
  // softmax (VALU), P V (MFMA). `sb` is the stage's byte offset from
  // stages[0]; the per-lane offsets add it once per part.
  //
  // qk: s[nb][b], lane (n, g) holds the scores of keys 16 b + 4 g + r, r < 4,
  // of row n of block nb.
  auto qk = [&](uint32_t sb, floatx4_t (&s)[2][4]) __attribute__((always_inline)) {
    constexpr uint32_t kRow16 = L::kRow16;
    uint32_t ko[kSteps];
#pragma unroll
    for (int j = 0; j < kSteps; ++j) ko[j] = koff[j] + sb;
    // Key block b + 1's K fragments load while block b's MFMAs run.
    Frag kf[2][kSteps];
#pragma unroll
    for (int j = 0; j < kSteps; ++j) kf[0][j] = lds_read_frag<Frag>(ko[j]);
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      if (b + 1 < 4) {
        const uint32_t tb = ((b + 1) >> 1) * L::kTileBytes + ((b + 1) & 1) * kRow16;
#pragma unroll
        for (int j = 0; j < kSteps; ++j) kf[(b + 1) & 1][j] = lds_read_frag<Frag>(ko[j] + tb);
      }
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) {
        s[nb][b] = M::mma(kf[b & 1][0], qf[nb][0], floatx4_t{0.f, 0.f, 0.f, 0.f});
#pragma unroll
        for (int j = 1; j < kSteps; ++j) s[nb][b] = M::mma(kf[b & 1][j], qf[nb][j], s[nb][b]);
      }
    }
  };
  // softmax: one running-max update per row block over the stage's 64 keys
  // (first key t0), the scale folded into the exponent; the weights, rounded
  // to T, into pf[nb][t] (32-key tile t), the accumulator rescaled when the
  // maximum moved.
  auto softmax = [&](int t0, floatx4_t (&s)[2][4], Frag (&pf)[2][2]) __attribute__((always_inline)) {
    float alpha[2];
    bool rescale = false;
    const bool masked = t0 + kStageKeys - 1 > lim_lo;  // reaches past some row's last key
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
      if (masked) {
        // Key t0 + 16 b + 4 g + r is visible iff 16 b + r <= lim - t0 - 4 g.
        const int d = lim[nb] - t0 - 4 * g;
#pragma unroll
        for (int b = 0; b < 4; ++b)
#pragma unroll
          for (int r = 0; r < 4; ++r) s[nb][b][r] = (16 * b + r <= d) ? s[nb][b][r] : -INFINITY;
      }
      float mx = fmaxf(fmaxf(s[nb][0][0], s[nb][0][1]), s[nb][0][2]);
      mx = fmaxf(fmaxf(mx, s[nb][0][3]), s[nb][1][0]);
#pragma unroll
      for (int b = 1; b < 4; ++b) {
        if (b > 1) mx = fmaxf(fmaxf(mx, s[nb][b][0]), s[nb][b][1]);
        else mx = fmaxf(mx, s[nb][b][1]);
        mx = fmaxf(fmaxf(mx, s[nb][b][2]), s[nb][b][3]);
      }
      mx = li_group_max(mx) * sc;
      // Lazy rescale: the running maximum only moves when the stage beats it
      // by more than kLazyRescale (log2 units), so most stages leave the
      // accumulator alone; the weights are then at most 2^kLazyRescale.
      const float mnew = (mx > m[nb] + kLazyRescale) ? mx : m[nb];
      rescale |= mnew != m[nb];
      alpha[nb] = __builtin_amdgcn_exp2f(m[nb] - mnew);
      m[nb] = mnew;
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        float p[8];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          p[r] = __builtin_amdgcn_exp2f(fmaf(s[nb][2 * t][r], sc, -mnew));
          p[4 + r] = __builtin_amdgcn_exp2f(fmaf(s[nb][2 * t + 1][r], sc, -mnew));
        }
        u32x4_t pw;
#pragma unroll
        for (int u = 0; u < 4; ++u) pw[u] = li_pack2<T>(p[2 * u], p[2 * u + 1]);
        pf[nb][t] = __builtin_bit_cast(Frag, pw);
      }
    }
    if (__any(rescale)) {
#pragma unroll
      for (int nb = 0; nb < 2; ++nb)
#pragma unroll
        for (int i = 0; i < D / 16 + 1; ++i)
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[nb][i][r] *= alpha[nb];
    }
  };
  // pv: O^T += V^T P^T, 16 dims at a time, for each 32-key tile of the stage.
  auto pv = [&](uint32_t sb, const Frag (&pf)[2][2]) __attribute__((always_inline)) {
    constexpr uint32_t kRow16 = L::kRow16;
    constexpr uint32_t kV = 32 * L::kRowBytes;
    uint32_t vo[D / 16];
#pragma unroll
    for (int blk = 0; blk < D / 16; ++blk) vo[blk] = voff[blk] + sb + kV;
    // A tile's eight V^T fragments load together, then its MFMAs run.
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const uint32_t tb = t * L::kTileBytes;
      Frag vf[D / 16];
#pragma unroll
      for (int blk = 0; blk < D / 16; ++blk) vf[blk] = lds_read_vt<Frag>(vo[blk] + tb, vo[blk] + tb + kRow16);
#pragma unroll
      for (int blk = 0; blk < D / 16; ++blk)
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) acc[nb][blk] = M::mma(vf[blk], pf[nb][t], acc[nb][blk]);
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) acc[nb][D / 16] = M::mma(ones, pf[nb][t], acc[nb][D / 16]);
    }
  };
  // One stage: the three parts back to back, with nothing pinning their
  // order, so the compiler interleaves one row block's softmax with the
  // other's MFMAs (wave priorities and scheduling fences here measured 3-4%
  // slower).
  auto fold = [&](auto stage_tag, int t0) __attribute__((always_inline)) {
    constexpr uint32_t sb = decltype(stage_tag)::value * 2 * L::kTileBytes;
    floatx4_t s[2][4];
    Frag pf[2][2];
    qk(sb, s);
    softmax(t0, s, pf);
    pv(sb, pf);
  };

  using Stage0 = std::integral_constant<int, 0>;
  using Stage1 = std::integral_constant<int, 1>;
  for (int c0 = 0; c0 < kend; c0 += kChunk) {
    const int c1 = min(c0 + kChunk, kend);
    const int ntiles = (c1 - c0 + kStageKeys - 1) / kStageKeys;
    // Stage this chunk's slots plus one stage past its end; entries past the
    // chunk repeat its last slot so every load reads a real row.
    __syncthreads();
    for (int i = tid; i < kChunk + kStageKeys; i += 64 * W) sl[i] = (int)srow[min(c0 + i, c1 - 1)];
    __syncthreads();

    // Two stages: the next 64 keys land in one while the other is folded.
    // Past the chunk the look-ahead re-reads a real stage (cache hits), so
    // every wave has the same loads in flight at every wait. The loop body
    // handles both stages so that each stage's LDS offsets are constants.
    if constexpr (!F8) {
      // Two stages: the next 64 keys land in one while the other is folded.
      // Past the chunk the look-ahead re-reads a real stage (cache hits), so
      // every wave has the same loads in flight at every wait. The loop body
      // handles both stages so that each stage's LDS offsets are constants.
      issue_stage<LS, W>(lds_addr(stages[0]), kpool, vpool, sl, row_bytes, 0, lane, w);
      for (int ti = 0; ti < ntiles; ti += 2) {
        issue_stage<LS, W>(lds_addr(stages[1]), kpool, vpool, sl, row_bytes, min(kStageKeys * (ti + 1), kChunk), lane, w);
        li_wait_vm<kDmaPerStage>();
        __syncthreads();
        if (!idle) fold(Stage0{}, c0 + kStageKeys * ti);
        __syncthreads();
        if (ti + 1 >= ntiles) break;
        issue_stage<LS, W>(lds_addr(stages[0]), kpool, vpool, sl, row_bytes, min(kStageKeys * (ti + 2), kChunk), lane, w);
        li_wait_vm<kDmaPerStage>();
        __syncthreads();
        if (!idle) fold(Stage1{}, c0 + kStageKeys * (ti + 1));
        __syncthreads();
      }
    } else {
      // fp8: the loads fill raw[x]; after the barrier that sees them land,
      // the work-group converts raw[x] into stages[x], and after a second
      // barrier the waves fold stages[x]. raw[x] takes its next loads once
      // converted; stages[x] is converted again only after every wave has
      // passed the barrier of the stage in between, so after its fold.
      issue_stage<LS, W>(lds_addr(raw[0]), kpool, vpool, sl, row_bytes, 0, lane, w);
      for (int ti = 0; ti < ntiles; ti += 2) {
        issue_stage<LS, W>(lds_addr(raw[1]), kpool, vpool, sl, row_bytes, min(kStageKeys * (ti + 1), kChunk), lane, w);
        li_wait_vm<kDmaPerStage>();
        __syncthreads();
        convert_stage<T, W>(lds_addr(raw[0]), lds_addr(stages[0]), tid);
        __syncthreads();
        if (!idle) fold(Stage0{}, c0 + kStageKeys * ti);
        if (ti + 1 >= ntiles) break;
        issue_stage<LS, W>(lds_addr(raw[0]), kpool, vpool, sl, row_bytes, min(kStageKeys * (ti + 2), kChunk), lane, w);
        li_wait_vm<kDmaPerStage>();
        __syncthreads();
        convert_stage<T, W>(lds_addr(raw[1]), lds_addr(stages[1]), tid);
        __syncthreads();
        if (!idle) fold(Stage1{}, c0 + kStageKeys * (ti + 1));
      }
    }
    li_wait_vm<0>();
  }

#pragma unroll
  for (int nb = 0; nb < 2; ++nb) {
    const float lt = acc[nb][D / 16][0];
    if (!real[nb]) continue;
    const float inv = (F8 ? a.v_scale : 1.f) / lt;
    // acc[nb][blk][r] is dim 16 blk + 4 g + r of this lane's row.
    T* orow = static_cast<T*>(a.out) + (int64_t)tok[nb] * a.o_s0 + (int64_t)head[nb] * a.o_s1 + 4 * g;
#pragma unroll
    for (int blk = 0; blk < D / 16; ++blk) {
      uint2 wv;
      wv.x = li_pack2<T>(acc[nb][blk][0] * inv, acc[nb][blk][1] * inv);
      wv.y = li_pack2<T>(acc[nb][blk][2] * inv, acc[nb][blk][3] * inv);
      *reinterpret_cast<uint2*>(orow + 16 * blk) = wv;
    }
  }
  }  // units
}

template <typename T, int D, int W, bool F8, bool kDirect>
__global__ __launch_bounds__(64 * W) __attribute__((amdgpu_waves_per_eu(2, 2))) void prefill_mfma(AttnArgs a) {
  prefill_mfma_body<T, D, W, F8, false, kDirect>(a, a);
}

// A packed pass's chunks and one-query rows in one launch, fp8 pools (the
// 16-bit pools' counterpart is prefill_pp_rows).
template <typename T, int D, int W, bool F8>
__global__ __launch_bounds__(64 * W) __attribute__((amdgpu_waves_per_eu(2, 2))) void prefill_mfma_rows(AttnArgs a,
                                                                                                    AttnArgs d) {
  prefill_mfma_body<T, D, W, F8, true>(a, d);
}

// issue_stage into a layout that keeps the K rows of every stage in one LDS
// region and the V rows in another (kdst / vdst: this stage's 32-key tiles
// of K, of V, 32 rows apart), so that the per-lane read addresses of either
// region plus every buffer's constant offset fit a DS instruction's 16-bit
// immediate. Split in two so the slot reads can go out well before the loads
// that need them: stage_slot_reads reads the kPer slots this wave loads
// (entry `t` first), stage_fire issues the loads of K and V rows.
template <typename L, int W>
__device__ __forceinline__ void stage_slot_reads(uint32_t (&slot)[2 * L::kInsts / W], const int* __restrict__ sl,
                                                 int t, int lane, int w) {
  constexpr int kPer = 2 * L::kInsts / W;
  static_assert(kPer >= 1 && kPer * W == 2 * L::kInsts, "waves must split the stage's loads evenly");
  const int rr = lane / L::kCh;
#pragma unroll
  for (int ii = 0; ii < kPer; ++ii) {
    const int p = w * kPer + ii, half = p / L::kInsts, i = p % L::kInsts;
    slot[ii] = (uint32_t)sl[t + 32 * half + rr * L::kInsts + i];
  }
}

template <typename L, int W>
__device__ __forceinline__ void stage_fire(uint32_t kdst, uint32_t vdst, const char* __restrict__ kpool,
                                           const char* __restrict__ vpool, const uint32_t (&slot)[2 * L::kInsts / W],
                                           uint32_t row_bytes, int lane, int w) {
  constexpr int kPer = 2 * L::kInsts / W;
  const int rr = lane / L::kCh, nn = lane % L::kCh;
#pragma unroll
  for (int ii = 0; ii < kPer; ++ii) {
    const int p = w * kPer + ii, half = p / L::kInsts, i = p % L::kInsts;
    const int key = rr * L::kInsts + i;
    const uint32_t off = half * 32 * L::kRowBytes + i * 1024;
    dma16_kv(row_ptr(kpool + 16 * (nn ^ L::kswizzle(key)), slot[ii], row_bytes),
             row_ptr(vpool + 16 * (nn ^ L::vswizzle(key)), slot[ii], row_bytes), kdst + off, vdst + off);
  }
}

// The 16-bit-pool prefill with the two waves of each SIMD in ping-pong.
//
// Same units, rows, LDS tile layout and arithmetic as prefill_mfma; what
// changes is when a wave does what. A wave's work per 64-key stage j has a
// matrix phase M(j) -- P V of stage j - 1 and the scores of stage j, 68
// MFMAs -- and a vector phase V(j) -- mask, row maxima, running-maximum
// update and the weights of stage j, ~32 exponentials and ~100 other vector
// instructions per lane. On gfx950 a wave that interleaves its own MFMAs
// and vector instructions gets the two back to back (measured: 8 MFMAs + 32
// FMAs in one wave cost the sum of the two), while the matrix core of a
// SIMD runs at full rate beside another wave's vector work. So waves 0-3
// and waves 4-7 (the second wave of SIMDs 0-3) run half a stage apart:
//
//   half-period   2j          2j + 1
//   waves 0-3     M(j)        V(j)
//   waves 4-7     V(j - 1)    M(j)
//
// with a work-group barrier between half-periods, so at any time one wave of
// every SIMD feeds the matrix core while the other runs its softmax. Stage
// j's K/V tile is read from LDS from half-period 2j (scores, waves 0-3) to
// 2j + 3 (P V, waves 4-7); LDS holds kPpRing stages, and the direct-to-LDS
// loads of stage j + kPpRing - 2 go out at half-period 2j, two stages ahead
// of their first use. Slot indices sit in a ring restaged half at a time, so
// a unit's key loop never drains.
constexpr int kPpRing = 4;
constexpr int kSlotRing = 4096;  // staged slot entries (int32)
constexpr int kSlotHalfStages = kSlotRing / 2 / kStageKeys;

// Wave priority of the matrix phase: an MFMA that waits for issue behind the
// other wave's vector work leaves the matrix core idle.
constexpr int kPpMatrixPriority = 2;

// LDS of one ping-pong work-group: the K and V rows of each ring stage, the
// slot ring, and the unit being folded (claimed, and its output rows).
template <int D>
struct PpLds {
  static constexpr int kRegion = 2 * 32 * TileLayout<D>::kRowBytes;  // a stage's K (or V) rows
  __attribute__((aligned(16))) int sl[kSlotRing];
  __attribute__((aligned(1024))) char kst[kPpRing][kRegion];
  __attribute__((aligned(1024))) char vst[kPpRing][kRegion];
  int unit;
  int rows[3];  // the unit's first token + q0, its query count, first head
  int4 entry;   // the work-list entry of `unit`
  int4 range;   // its stage range and piece ({0, all, 0, 1} for a whole block)
};


// LDS of a ping-pong work-group; prefill_pp_rows's row waves use it first.
template <int D>
union PpShared {
  PpLds<D> pp;
  DecodeLds<D, false> rows[kRowWaves];
};

// The ping-pong work of work-group blockIdx.x of the persistent grid (its
// queue: blockIdx.x % kPrefillQueues). With kRows (prefill_pp_rows), the
// first work-groups fold the pass's one-query rows first (the balanced
// decode split, AttnArgs `d`, over kRowWaves waves of each of them; their
// count was written by prefill_order), then join the queues.
template <typename T, int D, bool kRows, bool kSplit, bool kDirect = false>
__device__ __forceinline__ void prefill_pp_body(AttnArgs a, const AttnArgs& d) {
  __shared__ __attribute__((aligned(1024))) PpShared<D> lds;
  const unsigned wg = blockIdx.x;
  if constexpr (kRows) fold_rows_first<T, D, false>(a, d, lds);
  constexpr int W = 8;
  using M = Mfma<T>;
  using Frag = typename M::Frag;
  using L = TileLayout<D>;
  constexpr int kSteps = D / 32;
  constexpr int kBlk = D / 16;  // 16-dim output blocks
  constexpr int kWaveDma = 2 * (2 * L::kInsts / W);  // loads one wave issues per stage
  constexpr int kHalf = 32 * L::kRowBytes;  // one 32-key tile's K (or V) rows
  constexpr int kRegion = 2 * kHalf;          // a stage's K (or V) rows
  static_assert(kPpRing == 4, "the loop body covers four stages");
  static_assert(kRegion == PpLds<D>::kRegion, "one stage region size");
  auto& sl = lds.pp.sl;
  auto& kst = lds.pp.kst;  // K rows of each stage
  auto& vst = lds.pp.vst;  // V rows of each stage

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool late = w >= 4;  // waves 4-7 run half a stage behind
  const int n = lane & 15, g = lane >> 4;

  const int nqueues = a.num_kv_heads % kPrefillQueues == 0 ? kPrefillQueues : 1;
  const int qi = (int)(wg % (unsigned)nqueues);
  const int heads_per_queue = a.num_kv_heads / nqueues;
  // A direct pass lists nothing: its units are found from the query counts,
  // and every claim after a work-group's first returns kNoUnit.
  constexpr int kNoUnit = 0x7fffffff;
  const int units = kDirect ? kNoUnit : a.queue[kPrefillQueues] * heads_per_queue;
  // Work-group barriers here order LDS only (lds_barrier): a unit's output
  // stores and the loads in flight never hold a barrier up.
  int& s_unit = lds.pp.unit;
  auto& s_rows = lds.pp.rows;
  int4& s_entry = lds.pp.entry;
  const int bq = a.block_q;
  const int G = a.groups;
  // Work-list entry of unit u ({-1, ...} for a unit past the listed ones,
  // without reading the list there).
  auto entry_of = [&](int u) -> int4 { return u < units ? a.work[u / heads_per_queue] : int4{-1, 0, 0, 0}; };
  // Its stage range and piece: a whole block unless prefill_order split it.
  // (Only the kSplit instantiation, launched for passes the host allows to
  // be split, reads ranges: the other's key loop is the same code as if no
  // pass were ever split.)
  auto range_of = [&](int u) -> int4 {
    if constexpr (kSplit) return u < units ? a.work_range[u / heads_per_queue] : int4{0, 0x7fffffff, 0, 1};
    return int4{0, 0x7fffffff, 0, 1};
  };
  int4& s_range = lds.pp.range;
  // A listed block always has queries of its own (prefill_order lists only
  // those); anything else is skipped rather than folded.
  auto block_ok = [&](const int4& e) -> bool {
    if (e.x < 0 || e.z <= 0 || (e.z == 1 && a.single_query_elsewhere)) return false;
    return e.x % a.num_qblocks < (e.z + bq - 1) / bq;
  };
  if constexpr (kDirect) {
    // Unit wg / nqueues of this queue: entry (wg / nqueues) / heads_per_queue
    // of the blocks prefill_order would list (direct_entry).
    if (tid < 64) {
      const int u = (int)(wg / (unsigned)nqueues);
      const int4 e = direct_entry(a, u / heads_per_queue);
      if (lane == 0) {
        s_unit = e.x < 0 ? kNoUnit : u;
        s_entry = e;
        if constexpr (kSplit) s_range = int4{0, 0x7fffffff, 0, 1};
      }
    }
  } else if (tid == 0) {
    const int u = atomicAdd(&a.queue[qi], 1);
    s_unit = u;
    s_entry = entry_of(u);
    if constexpr (kSplit) s_range = range_of(u);
  }
  int next_unit = 0;  // tid 0: the unit claimed for after this one
  // The unit's queries (the softmax scale times log2 e folded in, rounded
  // to T once: scores come out of the matrix cores in log2 units) and its
  // first slots (the whole ring, or the unit's keys if fewer). A unit after
  // the work-group's first has its slots read during the previous unit's
  // epilogue (`have`), so that round trip overlaps the output stores
  // instead of preceding the unit's first loads; its queries are read as
  // its first stages are issued (and land with them). Reading the queries
  // in the epilogue too made them live across the loop's back edge and
  // spilled 24 registers.
  const float sc = a.scale * kLog2eMfma;
  constexpr int kSlotsPer = kSlotRing / (64 * W);
  int first_slots[kSlotsPer];
  Frag qf[2][kSteps];
  bool have = false;
  auto fetch_inputs = [&](const int4& e, int u, int kbeg_, bool slots, bool queries) __attribute__((always_inline)) {
    const int seq_ = e.x / a.num_qblocks, qb_ = e.x % a.num_qblocks;
    const int nblk_ = (e.z + bq - 1) / bq;
    const int q1_ = e.z - (nblk_ - 1 - qb_) * bq;
    const int q0_ = max(q1_ - bq, 0);
    const int kend_ = e.w - e.z + q1_;
    const int kvh_ = qi + nqueues * (u % heads_per_queue);
    const int64_t* srow_ = a.st + (int64_t)seq_ * a.st_s;
    if (slots) {
#pragma unroll
      for (int r = 0; r < kSlotsPer; ++r) first_slots[r] = (int)srow_[min(kbeg_ + tid + r * 64 * W, kend_ - 1)];
    }
    if (!queries) return;
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
      const int row = 32 * w + 16 * nb + n;
      const int ql = row / G;
      const bool real_ = row < bq * G && q0_ + ql < q1_;
      const T* qrow = static_cast<const T*>(a.q) + (int64_t)(e.y + q0_ + ql) * a.q_s0 +
                      (int64_t)(kvh_ * G + row % G) * a.q_s1 + 8 * g;
#pragma unroll
      for (int j = 0; j < kSteps; ++j) {
        Frag x = real_ ? *reinterpret_cast<const Frag*>(qrow + 32 * j) : Frag{};
        u32x4_t pw;
#pragma unroll
        for (int u2 = 0; u2 < 4; ++u2) pw[u2] = li_pack2<T>((float)x[2 * u2] * sc, (float)x[2 * u2 + 1] * sc);
        qf[nb][j] = __builtin_bit_cast(Frag, pw);
      }
    }
  };
  for (;;) {
  lds_barrier();
  // Values read from memory are made wave-uniform explicitly, so every
  // branch on them below is a scalar branch (no exec-masked code paths).
  const int unit = __builtin_amdgcn_readfirstlane(s_unit);
  if (unit >= units) break;
  const int4 entry{__builtin_amdgcn_readfirstlane(s_entry.x), __builtin_amdgcn_readfirstlane(s_entry.y),
                   __builtin_amdgcn_readfirstlane(s_entry.z), __builtin_amdgcn_readfirstlane(s_entry.w)};
  if (!block_ok(entry)) {
    // (Never for a list prefill_order wrote.) Take the next unit; the
    // barrier at the top orders these writes before every wave's reads.
    lds_barrier();
    if (tid == 0) {
      const int u = kDirect ? kNoUnit : atomicAdd(&a.queue[qi], 1);
      s_unit = u;
      s_entry = entry_of(u);
      if constexpr (kSplit) s_range = range_of(u);
    }
    have = false;
    continue;
  }
  const int item = entry.x;
  const int seq = item / a.num_qblocks;
  const int qblock = item % a.num_qblocks;
  const int kvh = qi + nqueues * (unit % heads_per_queue);

  const int first_tok = entry.y;
  const int nq = entry.z;
  // Blocks are cut from the end of the chunk: block nblk - 1 ends at its
  // last query and only block 0 (the one with the fewest keys) is partial.
  const int nblk = (nq + bq - 1) / bq;
  const int q1 = nq - (nblk - 1 - qblock) * bq;
  const int q0 = max(q1 - bq, 0);
  const int ctx = entry.w;
  const int pos0 = ctx - nq;
  const int kend = pos0 + q1;
  // The unit's 64-key stages: the block's [0, ceil(kend / 64)), or a
  // piece's part of them. Stage numbers below count from the unit's first
  // (key kbeg); the slot ring holds key kbeg + i at entry i % kSlotRing.
  const int4 range = kSplit ? int4{__builtin_amdgcn_readfirstlane(s_range.x), __builtin_amdgcn_readfirstlane(s_range.y),
                                   __builtin_amdgcn_readfirstlane(s_range.z), __builtin_amdgcn_readfirstlane(s_range.w)}
                            : int4{0, 0x7fffffff, 0, 1};
  const int kbeg = range.x * kStageKeys;
  const int ns = min(range.y, (kend + kStageKeys - 1) / kStageKeys) - range.x;
  const bool piece = kSplit && range.w > 1;  // stores partial rows for prefill_merge
  // The next unit is claimed a few stages before this one ends, so the
  // atomic's round trip is hidden, yet late enough that a work-group that
  // finishes early still takes the heaviest unit left.
  const int claim_at = max(ns - 3, 0);
  // Read by the epilogue, after the key loop (the barriers between order it).
  if (tid == 0) {
    s_rows[0] = first_tok + q0;
    s_rows[1] = q1 - q0;
    s_rows[2] = kvh * G;
  }

  fetch_inputs(entry, unit, kbeg, !have, true);
  // From here keys count from the unit's first (kbeg): its slots, the
  // rows' last visible keys and the stages' first keys.
  const int64_t* srow = a.st + (int64_t)seq * a.st_s + kbeg;
  const int kend_u = kend - kbeg;
  int pos[2];
#pragma unroll
  for (int nb = 0; nb < 2; ++nb) {
    const int row = 32 * w + 16 * nb + n;
    const int ql = row / G;
    const bool real = row < bq * G && q0 + ql < q1;
    pos[nb] = real ? pos0 + q0 + ql - kbeg : kend_u;
  }
  const int lim[2] = {min(pos[0], kend_u - 1), min(pos[1], kend_u - 1)};
  const int lim_lo = min(pos0 + q0 - kbeg, kend_u - 1);
  // A wave whose 32 rows are all padding only loads stages and waits at the
  // barriers.
  const bool idle = 32 * w >= (q1 - q0) * G;

  const char* kpool = static_cast<const char*>(a.kp) + (int64_t)kvh * a.p_s1 * (int)sizeof(T);
  const char* vpool = static_cast<const char*>(a.vp) + (int64_t)kvh * a.p_s1 * (int)sizeof(T);
  const uint32_t row_bytes = (uint32_t)(a.p_s0 * (int)sizeof(T));

  // Running row maxima m (log2 units; -inf before the first stage) and
  // -m in the four lanes of an MFMA accumulator: the first MFMA of every
  // score chain starts from it, so the matrix cores return s - m and the
  // common stage's weights are exp2 of the scores as they come.
  float m[2] = {-INFINITY, -INFINITY};
  floatx4_t cneg[2] = {floatx4_t{0.f, 0.f, 0.f, 0.f}, floatx4_t{0.f, 0.f, 0.f, 0.f}};
  floatx4_t acc[2][kBlk + 1];  // [kBlk]: the row's sum of weights (MFMA against ones)
#pragma unroll
  for (int nb = 0; nb < 2; ++nb)
#pragma unroll
    for (int i = 0; i < kBlk + 1; ++i) acc[nb][i] = floatx4_t{0.f, 0.f, 0.f, 0.f};
  const Frag ones = li_ones<Frag>();

  uint32_t koff[kSteps], voff[kBlk];
  {
    const uint32_t kbase = lds_addr(&kst[0][0]), vbase = lds_addr(&vst[0][0]);
#pragma unroll
    for (int j = 0; j < kSteps; ++j) koff[j] = kbase + L::offset(n, 4 * j + g);
    const int s16 = lane & 15, a4 = s16 & 3, key = 4 * g + (s16 >> 2);
#pragma unroll
    for (int blk = 0; blk < kBlk; ++blk) voff[blk] = vbase + L::voffset(key, 2 * blk + (a4 >> 1)) + 8 * (a4 & 1);
  }

  // Slot ring: entry k % kSlotRing holds key k's slot (keys past the block's
  // last one repeat it, so every load reads a real row).
  auto stage_slots_loaders = [&](int k0, int count) {  // waves 0-3
    for (int i = tid; i < count; i += 256) sl[(k0 + i) % kSlotRing] = (int)srow[min(k0 + i, kend_u - 1)];
  };
  using Slots = uint32_t[2 * L::kInsts / W];
  auto fire = [&](int buf, const Slots& slot) {
    stage_fire<L, W>(lds_addr(kst[buf]), lds_addr(vst[buf]), kpool, vpool, slot, row_bytes, lane, w);
  };
  auto issue = [&](int buf, int st) {
    Slots slot;
    stage_slot_reads<L, W>(slot, sl, (st * kStageKeys) % kSlotRing, lane, w);
    fire(buf, slot);
  };

  floatx4_t s[2][4];  // scores (log2 units) of the stage between its M and V phases
  Frag pf[2][2];      // its weights, between its V phase and the next M phase

  // M phase: P V of the stage in buffer PB (when pv), then the scores of the
  // stage in buffer SB (when qk).
  // M phase: P V of the stage in buffer PB (when pv), then the scores of the
  // stage in buffer SB (when qk). LDS reads run four fragments ahead of the
  // MFMAs that consume them, across the boundary between the two parts
  // (sched_group_barrier pins the interleave; left to itself the scheduler
  // issues each read just before its first use and the wave waits out the
  // LDS latency at every fragment).
  constexpr int kVFrags = 2 * kBlk;    // V^T fragments of a stage (two reads each)
  constexpr int kKFrags = 4 * kSteps;  // K fragments of a stage (one read each)
  constexpr int kAhead = 4;  // fragments read ahead of the MFMAs that use them
  auto read_v = [&](uint32_t vb, Frag (&vf)[2][kBlk]) __attribute__((always_inline)) {
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int blk = 0; blk < kBlk; ++blk) {
        const uint32_t tb = vb + t * kHalf;
        vf[t][blk] = lds_read_vt<Frag>(voff[blk] + tb, voff[blk] + tb + L::kRow16);
      }
  };
  auto read_k = [&](uint32_t kb, Frag (&kf)[4][kSteps]) __attribute__((always_inline)) {
#pragma unroll
    for (int b = 0; b < 4; ++b)
#pragma unroll
      for (int j = 0; j < kSteps; ++j) kf[b][j] = lds_read_frag<Frag>(koff[j] + kb + (b >> 1) * kHalf + (b & 1) * L::kRow16);
  };
  auto pv_mfma = [&](const Frag (&vf)[2][kBlk]) __attribute__((always_inline)) {
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int blk = 0; blk < kBlk; ++blk)
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) acc[nb][blk] = M::mma(vf[t][blk], pf[nb][t], acc[nb][blk]);
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) acc[nb][kBlk] = M::mma(ones, pf[nb][t], acc[nb][kBlk]);
  };
  auto qk_mfma = [&](const Frag (&kf)[4][kSteps]) __attribute__((always_inline)) {
#pragma unroll
    for (int b = 0; b < 4; ++b)
#pragma unroll
      for (int j = 0; j < kSteps; ++j)
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) s[nb][b] = M::mma(kf[b][j], qf[nb][j], j == 0 ? cneg[nb] : s[nb][b]);
  };
  // Every period runs the same M phase: at j = 0 its P V reads a zeroed
  // buffer with zero weights (a no-op), and at j = ns its scores go unused.
  auto mphase = [&](auto pb_tag, auto sb_tag) __attribute__((always_inline)) {
    constexpr uint32_t vb = decltype(pb_tag)::value * kRegion;
    constexpr uint32_t kb = decltype(sb_tag)::value * kRegion;
    Frag vf[2][kBlk];
    Frag kf[4][kSteps];
    read_v(vb, vf);
    pv_mfma(vf);
    read_k(kb, kf);
    qk_mfma(kf);
    // Reads of fragment f + kAhead go out with the MFMAs of fragment f;
    // the first K fragments with the last V^T fragments' MFMAs.
    __builtin_amdgcn_sched_group_barrier(0x100, 2 * kAhead, 0);
#pragma unroll
    for (int f = 0; f < kVFrags; ++f) {
      __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
      if (f + kAhead < kVFrags) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
      else __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);  // row sums
#pragma unroll
    for (int f = 0; f < kKFrags; ++f) {
      __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
      if (f + kAhead < kKFrags) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  // V phase of stage j (first key t0): s holds s - m (log2 units). Mask;
  // then the lazy running-maximum update: only when some score of a row
  // beats m by more than kLazyRescale (or on the first stage) does the
  // stage take the row's maximum across its lanes and move m there by
  // delta, subtracting delta from the scores and rescaling the accumulator
  // by exp2(-delta). Most stages move nothing and their weights are exp2 of
  // the scores as they are, rounded to T.
  auto vphase = [&](int t0, auto buf_tag) __attribute__((always_inline)) {
    (void)buf_tag;
    const bool masked = t0 + kStageKeys - 1 > lim_lo;
    float lmax[2];
    bool move = false;
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
      if (masked) {
        // Key t0 + 16 b + 4 g + r is visible iff 16 b + r <= lim - t0 - 4 g.
        const int d = lim[nb] - t0 - 4 * g;
#pragma unroll
        for (int b = 0; b < 4; ++b)
#pragma unroll
          for (int r = 0; r < 4; ++r) s[nb][b][r] = (16 * b + r <= d) ? s[nb][b][r] : -INFINITY;
      }
      // A tree of three-input maxima over the lane's 16 scores.
      const float x0 = fmaxf(fmaxf(s[nb][0][0], s[nb][0][1]), s[nb][0][2]);
      const float x1 = fmaxf(fmaxf(s[nb][0][3], s[nb][1][0]), s[nb][1][1]);
      const float x2 = fmaxf(fmaxf(s[nb][1][2], s[nb][1][3]), s[nb][2][0]);
      const float x3 = fmaxf(fmaxf(s[nb][2][1], s[nb][2][2]), s[nb][2][3]);
      const float x4 = fmaxf(fmaxf(s[nb][3][0], s[nb][3][1]), s[nb][3][2]);
      lmax[nb] = fmaxf(fmaxf(fmaxf(x0, x1), x2), fmaxf(fmaxf(x3, x4), s[nb][3][3]));
      move |= lmax[nb] > kLazyRescale || m[nb] == -INFINITY;
    }
    if (__any(move)) {
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) {
        const float mx = li_group_max(lmax[nb]);
        const bool first = m[nb] == -INFINITY;
        const float delta = (first || mx > kLazyRescale) ? mx : 0.f;
        const float alpha = first ? 0.f : __builtin_amdgcn_exp2f(-delta);
        m[nb] = first ? delta : m[nb] + delta;
        cneg[nb] = floatx4_t{-m[nb], -m[nb], -m[nb], -m[nb]};
#pragma unroll
        for (int b = 0; b < 4; ++b)
#pragma unroll
          for (int r = 0; r < 4; ++r) s[nb][b][r] -= delta;
#pragma unroll
        for (int kk = 0; kk < kBlk + 1; ++kk)
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[nb][kk][r] *= alpha;
      }
    }
#pragma unroll
    for (int nb = 0; nb < 2; ++nb)
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        u32x4_t pw;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int b = 2 * t + u / 2, r = 2 * (u % 2);
          pw[u] = li_pack2<T>(__builtin_amdgcn_exp2f(s[nb][b][r]), __builtin_amdgcn_exp2f(s[nb][b][r + 1]));
        }
        pf[nb][t] = __builtin_bit_cast(Frag, pw);
      }
  };

  // Stage j (buffer j % kPpRing): the wave's M phase and V phase, each
  // after a barrier. Waves 4-7 run the same sequence one barrier later, so
  // their M phase meets the V phase of waves 0-3 and the other way round.
  // Every wave issues its share of the direct-to-LDS loads in its V phase,
  // where they delay no matrix work: waves 0-3 load stage j + 2 in V(j)
  // (half-period 2j + 1), waves 4-7 stage j + 3 in V(j) (half-period
  // 2j + 2); both land before stage j + 2's first use at half-period
  // 2j + 4. Each wave waits for its own loads before the barrier that
  // precedes that first use: waves 0-3 at the top of period j for stage j,
  // waves 4-7 before their mid barrier of period j for stage j + 1.
  auto period = [&](auto j_tag, int j) __attribute__((always_inline)) {
    constexpr int J = decltype(j_tag)::value;
    using Cur = std::integral_constant<int, J>;
    using Prev = std::integral_constant<int, (J + kPpRing - 1) % kPpRing>;
    // Only stages that exist are loaded, so near the end fewer loads are
    // newer than the one waited for.
    if (!late) {
      if (j + 1 < ns) li_wait_vm<kWaveDma>();
      else li_wait_vm<0>();
    }
    lds_barrier();
    // The old value is first read after the unit's last wait for every
    // load, where the compiler places its wait for the atomic (this file is
    // built with the wave-level atomic optimizer off, which would otherwise
    // read the value back at once and wait for every load in flight).
    if (j == claim_at && tid == 0) next_unit = kDirect ? kNoUnit : atomicAdd(&a.queue[qi], 1);
    if (!idle) {
      // The matrix phase issues ahead of the other wave's vector work on
      // its SIMD: an MFMA that waits for issue leaves the matrix core idle.
      __builtin_amdgcn_s_setprio(kPpMatrixPriority);
      mphase(Prev{}, Cur{});
      __builtin_amdgcn_s_setprio(0);
    }
    if (late) {
      if (j + 2 < ns) li_wait_vm<kWaveDma>();
      else li_wait_vm<0>();
    }
    lds_barrier();
    if (j < ns) {
      const int st = j + (late ? 3 : 2);
      if (!late && st % kSlotHalfStages == 0 && st + kSlotHalfStages < ns)
        stage_slots_loaders((st + kSlotHalfStages) * kStageKeys, kSlotRing / 2);
      if (st < ns) issue((J + (late ? 3 : 2)) % kPpRing, st);
      if (!idle) vphase(j * kStageKeys, Cur{});
    }
  };

  // Prologue: slots; the V rows of the last buffer zeroed (the first M
  // phase's P V reads them, with zero weights); stages 0 and 1 in flight,
  // and waves 4-7's share of stage 2.
#pragma unroll
  for (int nb = 0; nb < 2; ++nb)
#pragma unroll
    for (int t = 0; t < 2; ++t) pf[nb][t] = Frag{};
#pragma unroll
  for (int r = 0; r < kSlotsPer; ++r) sl[tid + r * 64 * W] = first_slots[r];
  for (int i = tid; i < kRegion / 16; i += 64 * W)
    *reinterpret_cast<__attribute__((address_space(3))) u32x4_t*>(
        (uintptr_t)(lds_addr(vst[kPpRing - 1]) + 16 * i)) = u32x4_t{0u, 0u, 0u, 0u};
  lds_barrier();
  issue(0, 0);
  if (ns > 1) issue(1, 1);
  if (late) {
    if (ns > 2) {
      issue(2, 2);
      li_wait_vm<2 * kWaveDma>();  // stage 0
    } else if (ns > 1) {
      li_wait_vm<kWaveDma>();
    } else {
      li_wait_vm<0>();
    }
    lds_barrier();               // waves 4-7 start one barrier late
  }
  for (int j = 0; j < ns; j += kPpRing) {
    period(std::integral_constant<int, 0>{}, j);
    if (j + 1 >= ns) break;
    period(std::integral_constant<int, 1>{}, j + 1);
    if (j + 2 >= ns) break;
    period(std::integral_constant<int, 2>{}, j + 2);
    if (j + 3 >= ns) break;
    period(std::integral_constant<int, 3>{}, j + 3);
  }
  // The last period: P V of the last stage only (every load has landed).
  li_wait_vm<0>();
  lds_barrier();
  // tid 0 reads the next unit's work-list entry (its id came back from the
  // claim above) while the last P V runs.
  int4 next_entry{-1, 0, 0, 0}, next_range{0, 0x7fffffff, 0, 1};
  if (tid == 0) {
    next_entry = entry_of(next_unit);
    if constexpr (kSplit) next_range = range_of(next_unit);
  }
  if (!idle) {
    Frag vf[2][kBlk];
    read_v(lds_addr(vst[(ns - 1) % kPpRing]) - lds_addr(vst[0]), vf);
    pv_mfma(vf);
  }
  lds_barrier();
  if (!late) lds_barrier();  // the barrier waves 4-7 took first
  if (tid == 0) {
    s_unit = next_unit;
    s_entry = next_entry;
    if constexpr (kSplit) s_range = next_range;
  }
  lds_barrier();
  {
    // The next unit's first slots, read now so that their round trip runs
    // under this unit's output stores.
    const int nu = __builtin_amdgcn_readfirstlane(s_unit);
    const int4 ne{__builtin_amdgcn_readfirstlane(s_entry.x), __builtin_amdgcn_readfirstlane(s_entry.y),
                  __builtin_amdgcn_readfirstlane(s_entry.z), __builtin_amdgcn_readfirstlane(s_entry.w)};
    have = nu < units && block_ok(ne);
    if (have) fetch_inputs(ne, nu, kSplit ? __builtin_amdgcn_readfirstlane(s_range.x) * kStageKeys : 0, true, false);
  }

  if (kSplit && piece) {
    // A piece of a split block: its rows unnormalised, with their running
    // maximum and sum of weights, for prefill_merge (every row, padding
    // included; the merge writes only the block's real ones).
    if (!idle) {
      int el = lane;
      asm volatile("" : "+v"(el));
      const int en = el & 15, eg = el >> 4;
      const int64_t slot = (int64_t)(unit / heads_per_queue) * a.num_kv_heads + kvh;
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) {
        const int r = 32 * w + 16 * nb + en;
        float* orow = a.split_o + (slot * kMinRows + r) * D + 4 * eg;
#pragma unroll
        for (int blk = 0; blk < kBlk; ++blk) *reinterpret_cast<floatx4_t*>(orow + 16 * blk) = acc[nb][blk];
        if (eg == 0)
          *reinterpret_cast<float2*>(a.split_ml + (slot * kMinRows + r) * 2) = float2{m[nb], acc[nb][kBlk][0]};
      }
    }
    continue;
  }
  // The output rows, normalised. A lane holds 8-byte pieces of its row 32
  // bytes apart, so stored as they are every store instruction would write
  // 16 rows' 32-byte pieces; instead each wave stages its 32 rows in its own
  // slice of the (now unused) K region -- rows of kRowBytes, 16-byte chunk
  // c of row r at slot c ^ (r mod kCh), so the 16 rows a write spans hit
  // different banks -- and stores whole chunks, kCh lanes per row: each
  // instruction writes 64 / kCh whole rows (the G heads of a query are
  // adjacent rows of the output, so mostly one contiguous span).
  if (!idle) {
    constexpr int kCh = L::kRowBytes / 16;
    // The lane index through an empty asm: the addresses below are then
    // computed here, not hoisted out of the unit loop into registers that
    // the key loop cannot spare.
    int el = lane;
    asm volatile("" : "+v"(el));
    const int en = el & 15, eg = el >> 4;
    const uint32_t ebase = lds_addr(&kst[0][0]) + (uint32_t)w * (32 * L::kRowBytes);
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
      const float inv = 1.f / acc[nb][kBlk][0];
      const int r = 16 * nb + en;
#pragma unroll
      for (int blk = 0; blk < kBlk; ++blk) {
        typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
        const u32x2_t wv = {li_pack2<T>(acc[nb][blk][0] * inv, acc[nb][blk][1] * inv),
                            li_pack2<T>(acc[nb][blk][2] * inv, acc[nb][blk][3] * inv)};
        const int c = 2 * blk + (eg >> 1);  // the piece: bytes 32 blk + 8 g of the row
        *reinterpret_cast<__attribute__((address_space(3))) u32x2_t*>(
            (uintptr_t)(ebase + r * L::kRowBytes + 16 * (c ^ (r % kCh)) + 8 * (eg & 1))) = wv;
      }
    }
    constexpr int kRowsPer = 64 / kCh;  // rows one store instruction covers
    const int c = el % kCh;
    // The unit's rows, as recorded at its start (kept in LDS rather than
    // registers through the key loop).
    const int tok0 = __builtin_amdgcn_readfirstlane(s_rows[0]);
    const int nvalid = __builtin_amdgcn_readfirstlane(s_rows[1]);
    const int head0 = __builtin_amdgcn_readfirstlane(s_rows[2]);
#pragma unroll
    for (int i = 0; i < 32 / kRowsPer; ++i) {
      const int r = el / kCh + kRowsPer * i;
      const u32x4_t v = *reinterpret_cast<const __attribute__((address_space(3))) u32x4_t*>(
          (uintptr_t)(ebase + r * L::kRowBytes + 16 * (c ^ (r % kCh))));
      const int row = 32 * w + r;
      const int ql = row / a.groups;
      if (ql < nvalid) {  // (so row < block_q * G too)
        T* orow = static_cast<T*>(a.out) + (int64_t)(tok0 + ql) * a.o_s0 +
                  (int64_t)(head0 + row % a.groups) * a.o_s1 + 8 * c;
        *reinterpret_cast<u32x4_t*>(orow) = v;
      }
    }
  }
  }  // units
}

template <typename T, int D, bool kSplit, bool kDirect>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2))) void prefill_pp(AttnArgs a) {
  prefill_pp_body<T, D, false, kSplit, kDirect>(a, a);
}

// A packed pass's chunks and one-query rows in one launch: the first
// work-groups fold the rows (the balanced decode split `d`, kRowWaves waves
// each), while the others start on the chunks; each joins the chunks'
// queues when its rows are done. The rows stream K/V from HBM while the
// chunks keep the matrix cores busy, instead of one waiting for the other.
template <typename T, int D, bool kSplit>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2))) void prefill_pp_rows(AttnArgs a,
                                                                                                  AttnArgs d) {
  prefill_pp_body<T, D, true, kSplit>(a, d);
}

// Work list of the prefill grid: every non-empty query block
// (sequence * num_qblocks + block), a sequence's blocks side by side, last
// (heaviest) block first, the sequences ordered by the 32-key tiles of their
// heaviest block, most first (a counting sort on tiles >> shift), each with
// the sequence's rows and context; their count goes to queue[kPrefillQueues]
// and nothing past it is read. Work-groups take units in this order as earlier
// ones retire, so the long blocks start at once and the short ones fill in
// behind them (longest-processing-time-first, by sequence), and the
// work-groups running at one time on an XCD fold blocks of one sequence:
// they sweep the same keys at about the same pace, so each K/V tile comes
// from HBM once into that XCD's L2 and is read there by the rest. One
// work-group; the order of sequences within a bucket is whatever the LDS
// atomics give, which changes the schedule only, never a result.
constexpr int kOrderBins = 256;

__global__ __launch_bounds__(1024) void prefill_order(AttnArgs a) {
  __shared__ int hist[kOrderBins];
  __shared__ int max_tiles;
  __shared__ unsigned long long row_keys, chunk_pairs;  // prefill_pp_rows's balance
  const int tid = threadIdx.x;
  // A sequence's first query row, query count and context length: three
  // independent reads, one round trip.
  auto info_of = [&](int seq) -> int4 {
    const int first = a.qsl[seq], next = a.qsl[seq + 1], ctx = a.ctx[seq];
    return int4{first, next - first, ctx, 0};
  };
  // Blocks of a sequence the prefill folds, and the tiles of its heaviest
  // (last) block.
  auto blocks_of = [&](const int4& e, int* tiles) {
    const int nq = e.y;
    *tiles = 0;
    if (nq <= 0 || (nq == 1 && a.single_query_elsewhere)) return 0;
    *tiles = (e.z + 31) / 32;
    return min((nq + a.block_q - 1) / a.block_q, a.num_qblocks);
  };
  // A thread's first sequence (the only one while batch <= 1024) is read
  // once and kept for every pass; further ones are read again.
  const int4 c_e = tid < a.batch ? info_of(tid) : int4{0, 0, 0, 0};
  int c_t = 0;
  const int c_nb = tid < a.batch ? blocks_of(c_e, &c_t) : 0;
  // (One-query rows in the launch keep the pass whole: their work-groups'
  // count is decided below.)
  const bool has_rows = __syncthreads_or(tid < a.batch && c_e.y == 1 && a.single_query_elsewhere);
  if (a.split_ok && !has_rows) {
    // A pass too small to fill the grid (the host allows this only for a
    // batch of at most 1024 sequences, so thread i holds sequence i): each
    // block's fully visible stages -- wholly before its first query -- are
    // cut into up to f pieces of at least kSplitMinStages stages, f the
    // grid's units over the blocks' units. The last piece also takes the
    // stages its queries mask, so every piece's every row sees a key. A
    // block's pieces are consecutive entries, in sequence order.
    __shared__ int s_blocks, s_split;
    __shared__ int s_wave[1024 / 64];
    if (tid == 0) {
      s_blocks = 0;
      s_split = 0;
    }
    __syncthreads();
    if (c_nb > 0) atomicAdd(&s_blocks, c_nb);
    __syncthreads();
    const int f = max(1, a.split_target / max(1, s_blocks * a.num_kv_heads));
    const int bq = a.block_q;
    // Block qb of this thread's sequence: its stage count and its pieces.
    auto cut = [&](int qb, int* ns, int* vis) -> int {
      const int nq = c_e.y, ctx = c_e.z;
      const int nblk = (nq + bq - 1) / bq;
      const int q1 = nq - (nblk - 1 - qb) * bq;
      const int q0 = max(q1 - bq, 0);
      const int pos0 = ctx - nq;
      *ns = (pos0 + q1 + kStageKeys - 1) / kStageKeys;
      *vis = (pos0 + q0 + 1) / kStageKeys;
      return max(1, min(min(f, kSplitMaxPieces), *vis / kSplitMinStages));
    };
    int mine = 0;
    for (int i = 0; i < c_nb; ++i) {
      int ns, vis;
      mine += cut(c_nb - 1 - i, &ns, &vis);
    }
    // Exclusive prefix of `mine` over the threads.
    const int lane = tid & 63;
    int incl = mine;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int up = __shfl_up(incl, off, 64);
      if (lane >= off) incl += up;
    }
    if (lane == 63) s_wave[tid >> 6] = incl;
    __syncthreads();
    int at = incl - mine;
    for (int v = 0; v < (tid >> 6); ++v) at += s_wave[v];
    for (int i = 0; i < c_nb; ++i) {
      const int qb = c_nb - 1 - i;
      int ns, vis;
      const int p = cut(qb, &ns, &vis);
      const int per = vis / p;
      if (p > 1) a.split_first[atomicAdd(&s_split, 1)] = at;
      for (int k = 0; k < p; ++k, ++at) {
        a.work[at] = int4{tid * a.num_qblocks + qb, c_e.x, c_e.y, c_e.z};
        a.work_range[at] = int4{k * per, k + 1 < p ? (k + 1) * per : ns, k, p};
      }
    }
    if (tid < kPrefillQueues) a.queue[tid] = 0;
    if (tid == 1023) a.queue[kPrefillQueues] = at;  // the last thread's end: every entry listed
    if (tid == 0 && a.row_groups_max > 0) a.queue[kPrefillQueues + 1] = 0;  // no rows to fold first
    __syncthreads();
    if (tid == 0) a.queue[kPrefillQueues + 2] = s_split;
    return;
  }
  if (tid < kOrderBins) hist[tid] = 0;
  if (tid == 0) {
    max_tiles = 0;
    row_keys = 0;
    chunk_pairs = 0;
  }
  __syncthreads();
  int local = c_t;
  for (int sq = tid + 1024; sq < a.batch; sq += 1024) {
    int t;
    blocks_of(info_of(sq), &t);
    local = max(local, t);
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) local = max(local, __shfl_xor(local, off, 64));
  if ((tid & 63) == 0) atomicMax(&max_tiles, local);
  __syncthreads();
  int shift = 0;
  while ((max_tiles >> shift) >= kOrderBins) ++shift;
  // Bin b holds the blocks of sequences with (tiles >> shift) ==
  // kOrderBins - 1 - b, so bins run from the heaviest down.
  if (c_nb > 0) atomicAdd(&hist[kOrderBins - 1 - (c_t >> shift)], c_nb);
  for (int sq = tid + 1024; sq < a.batch; sq += 1024) {
    int t;
    const int nb = blocks_of(info_of(sq), &t);
    if (nb > 0) atomicAdd(&hist[kOrderBins - 1 - (t >> shift)], nb);
  }
  __syncthreads();
  // Exclusive prefix sum over the bins: a scan within each of the first
  // kOrderBins / 64 waves, then the totals of the waves before.
  {
    __shared__ int wave_total[kOrderBins / 64];
    const int lane = tid & 63;
    int incl = 0, own = 0;
    if (tid < kOrderBins) {
      own = hist[tid];
      incl = own;
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const int up = __shfl_up(incl, off, 64);
        if (lane >= off) incl += up;
      }
      if (lane == 63) wave_total[tid >> 6] = incl;
    }
    __syncthreads();
    if (tid < kOrderBins) {
      int before = 0;
      for (int v = 0; v < (tid >> 6); ++v) before += wave_total[v];
      hist[tid] = before + incl - own;
      if (tid == kOrderBins - 1) max_tiles = before + incl;  // now: the number of blocks listed
    }
  }
  __syncthreads();
  auto place = [&](int sq, const int4& e, int nb, int t) {
    const int at = atomicAdd(&hist[kOrderBins - 1 - (t >> shift)], nb);
    for (int i = 0; i < nb; ++i) {
      a.work[at + i] = int4{sq * a.num_qblocks + (nb - 1 - i), e.x, e.y, e.z};
      if (a.split_ok) a.work_range[at + i] = int4{0, 0x7fffffff, 0, 1};  // whole blocks
    }
  };
  if (c_nb > 0) place(tid, c_e, c_nb, c_t);
  for (int sq = tid + 1024; sq < a.batch; sq += 1024) {
    int t;
    const int4 e = info_of(sq);
    const int nb = blocks_of(e, &t);
    if (nb > 0) place(sq, e, nb, t);
  }
  // Entries past the listed blocks are never read: the prefill kernels take
  // units below the listed count only.
  // The persistent grid's queues start empty for this launch.
  if (tid < kPrefillQueues) a.queue[tid] = 0;
  if (tid == 0) a.queue[kPrefillQueues] = max_tiles;
  if (tid == 0 && a.split_ok) a.queue[kPrefillQueues + 2] = 0;  // no block split
  if (a.row_groups_max > 0) {
    // prefill_pp_rows: how many work-groups fold the one-query rows first.
    // The rows' K/V bytes against the chunks' flops (visible causal pairs),
    // scaled by kRowFlopsPerByte: the rows then finish about when three
    // quarters of the chunks' work is done, and their work-groups take
    // chunk units for the rest. A multiple of the queue count, so every
    // XCD gives the rows the same number of CUs.
    int64_t keys = 0, pairs = 0;
    for (int sq = tid; sq < a.batch; sq += 1024) {
      const int4 e = sq == tid ? c_e : info_of(sq);
      const int nq = e.y;
      const int c = max(e.z, 0);
      if (nq == 1) keys += c;
      else if (nq > 1) pairs += (int64_t)nq * max(c - nq, 0) + (int64_t)nq * (nq + 1) / 2;
    }
    keys = wave_sum_i64(keys);
    pairs = wave_sum_i64(pairs);
    if ((tid & 63) == 0) {
      atomicAdd(&row_keys, (unsigned long long)keys);
      atomicAdd(&chunk_pairs, (unsigned long long)pairs);
    }
    __syncthreads();
    if (tid == 0)
      a.queue[kPrefillQueues + 1] = prefill_row_groups(row_keys, chunk_pairs, max_tiles, a.row_groups_max,
                                                       a.num_kv_heads, a.num_heads, a.head_dim, a.kv_fp8);
  }
}

// Folds the pieces of each split block into its output rows: out =
// sum_k 2^(m_k - M) o_k / sum_k 2^(m_k - M) l_k over its pieces k, M their
// largest running maximum (the fold of partial softmaxes, in the log2
// domain the kernels keep their scores in). Work-group (split block i, KV
// head, chunk of kMergeRows rows); D / 4 lanes per row, a float4 of it
// each; lane j of a row reads the maximum and sum of pieces j, j + D / 4,
// ...; rows of padding are skipped.
template <int D>
constexpr int merge_rows() { return 256 / (D / 4); }

template <typename T, int D>
__global__ __launch_bounds__(256) void prefill_merge(AttnArgs a) {
  constexpr int kLanes = D / 4;  // per row
  constexpr int kRows = merge_rows<D>();
  constexpr int kPer = (kSplitMaxPieces + kLanes - 1) / kLanes;  // pieces' (m, l) per lane
  const int chunks = kMinRows / kRows;
  const int i = (int)(blockIdx.x / (unsigned)(a.num_kv_heads * chunks));
  const int kvh = (int)(blockIdx.x / (unsigned)chunks % (unsigned)a.num_kv_heads);
  const int chunk = (int)(blockIdx.x % (unsigned)chunks);
  if (i >= a.queue[kPrefillQueues + 2]) return;
  const int e = a.split_first[i];
  const int p = a.work_range[e].w;
  const int4 en = a.work[e];
  const int bq = a.block_q, G = a.groups;
  const int qb = en.x % a.num_qblocks;
  const int nq = en.z;
  const int nblk = (nq + bq - 1) / bq;
  const int q1 = nq - (nblk - 1 - qb) * bq;
  const int q0 = max(q1 - bq, 0);
  const int nvalid = q1 - q0;
  const int j = (int)threadIdx.x % kLanes;
  const int row = chunk * kRows + (int)threadIdx.x / kLanes;
  if (row >= nvalid * G) return;
  auto slot_of = [&](int k) -> int64_t { return ((int64_t)(e + k) * a.num_kv_heads + kvh) * kMinRows + row; };
  float mk[kPer], lk[kPer];
  float mx = -INFINITY;
#pragma unroll
  for (int t = 0; t < kPer; ++t) {
    const int k = j + kLanes * t;
    const float2 ml = k < p ? *reinterpret_cast<const float2*>(a.split_ml + slot_of(k) * 2) : float2{-INFINITY, 0.f};
    mk[t] = ml.x;
    lk[t] = ml.y;
    mx = fmaxf(mx, ml.x);
  }
#pragma unroll
  for (int off = 1; off < kLanes; off <<= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
  float tot = 0.f;
#pragma unroll
  for (int t = 0; t < kPer; ++t) {
    mk[t] = mk[t] == -INFINITY ? 0.f : exp2f(mk[t] - mx);  // piece j + kLanes t's weight
    tot = fmaf(mk[t], lk[t], tot);
  }
#pragma unroll
  for (int off = 1; off < kLanes; off <<= 1) tot += __shfl_xor(tot, off, 64);
  const int d = 4 * j;
  const int base = (int)threadIdx.x - j;  // the row's first lane
  floatx4_t o = {0.f, 0.f, 0.f, 0.f};
  for (int k0 = 0; k0 < p; k0 += 8) {
    floatx4_t x[8];
#pragma unroll
    for (int u = 0; u < 8; ++u)
      x[u] = k0 + u < p ? *reinterpret_cast<const floatx4_t*>(a.split_o + slot_of(k0 + u) * D + d)
                        : floatx4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int k = k0 + u;
      float wt = 0.f;
#pragma unroll
      for (int t = 0; t < kPer; ++t) {
        const float w_t = __shfl(mk[t], (base + k % kLanes) & 63, 64);
        if (k / kLanes == t) wt = w_t;
      }
#pragma unroll
      for (int c = 0; c < 4; ++c) o[c] = fmaf(wt, x[u][c], o[c]);
    }
  }
  const float inv = 1.f / tot;
  T* orow = static_cast<T*>(a.out) + (int64_t)(en.y + q0 + row / G) * a.o_s0 +
            (int64_t)(kvh * G + row % G) * a.o_s1 + d;
  typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
  *reinterpret_cast<u32x2_t*>(orow) = u32x2_t{li_pack2<T>(o[0] * inv, o[1] * inv), li_pack2<T>(o[2] * inv, o[3] * inv)};
}

bool rows_aligned(const void* p, int64_t s0, int64_t s1, int esize) {
  return aligned16(p) && (s0 * esize) % 16 == 0 && (s1 * esize) % 16 == 0;
}

}  // namespace

size_t prefill_work_entries(int batch, int max_context) {
  // A sequence's queries are the last of its context, so it has at most
  // max_context of them; blocks hold at least kMinRows / 16 query tokens.
  return (size_t)batch * cdiv(max(max_context, 1), kMinRows / 16);
}

bool prefill_mfma_applies(const AttnArgs& a, int dtype) {
  if (dtype != LI_BF16 && dtype != LI_F16) return false;
  if (a.head_dim != 64 && a.head_dim != 128) return false;
  if (a.kv_fp8 && a.head_dim != 128) return false;
  if (a.groups < 1 || a.groups > 16) return false;
  const int pe = a.kv_fp8 ? 1 : 2;
  return rows_aligned(a.q, a.q_s0, a.q_s1, 2) && rows_aligned(a.out, a.o_s0, a.o_s1, 2) &&
         rows_aligned(a.kp, a.p_s0, a.p_s1, pe) && rows_aligned(a.vp, a.p_s0, a.p_s1, pe);
}

// `rows`: the one-query rows' decode split to run in the same launch
// (prefill_pp_rows), or null.
static int launch_prefill_merge(const AttnArgs& a, int dtype, hipStream_t s);

template <int W>
static int launch_prefill_waves(AttnArgs a, int dtype, hipStream_t s, const AttnArgs* rows) {
  a.block_q = 32 * W / a.groups;
  a.num_qblocks = cdiv(a.max_query_len, a.block_q);
  const int64_t units = (int64_t)a.batch * a.num_kv_heads * a.num_qblocks;
  if (units == 0) return LI_OK;
  if ((size_t)a.batch * a.num_qblocks > prefill_work_entries(a.batch, a.max_context))
    return fail(LI_EINVAL, "prefill: %d query blocks per sequence exceed the planned work list", a.num_qblocks);
  static_assert(kMinRows == kPrefillUnitRows, "a prefill unit's rows");
  if (a.split_ok && (a.block_q != kPrefillUnitRows / a.groups || a.kv_fp8 || a.batch > 1024))
    return fail(LI_EINVAL, "prefill: a split pass needs the ping-pong kernel's blocks");
  // One work-group per CU (its LDS and registers fill one), a multiple of
  // the queue count so every queue has work-groups, and never more than
  // there can be units (the rows' work-groups aside).
  int64_t grid = (device_cu_count() + kPrefillQueues - 1) / kPrefillQueues * kPrefillQueues;
  if (!rows && !a.split_ok)
    grid = std::min<int64_t>(grid, (units + kPrefillQueues - 1) / kPrefillQueues * kPrefillQueues);
  // The rows' waves must fit the workspace's partial slots as well as the
  // grid: the one cap both prefill_order's rule and the kernel's clamp use.
  a.row_groups_max = rows ? prefill_row_cap(grid, rows->num_parts) : 0;
  if (rows && a.row_groups_max < 1)
    return fail(LI_EINVAL, "prefill with rows: a split of %d waves holds no work-group of %d row waves",
                rows->num_parts, kRowWaves);
  // A small pass whose every unit fits the grid at once needs no order: one
  // work-group per unit, each finding its own, one launch.
  const int64_t full = (device_cu_count() + kPrefillQueues - 1) / kPrefillQueues * kPrefillQueues;
  const bool direct = !rows && !a.split_ok && a.batch <= kPrefillDirectBatch && units <= full;
  if (direct) {
    grid = units;  // a multiple of the queue count (every KV head has a unit of each block)
  } else {
    hipLaunchKernelGGL(prefill_order, dim3(1), dim3(1024), 0, s, a);
    if (int rc = check_launch("prefill_order")) return rc;
  }
  const dim3 block(64 * W);
  const dim3 g((unsigned)grid);
  if (rows && a.kv_fp8) {
    if (dtype == LI_BF16) hipLaunchKernelGGL((prefill_mfma_rows<li_bf16, 128, W, true>), g, block, 0, s, a, *rows);
    else hipLaunchKernelGGL((prefill_mfma_rows<li_f16, 128, W, true>), g, block, 0, s, a, *rows);
    if (int rc = check_launch("prefill_mfma_rows")) return rc;
    return launch_combine_balanced(*rows, dtype, s);
  }
  if (rows) {
#define LI_PP_ROWS(T, D)                                                                            \
  do {                                                                                              \
    if (a.split_ok) hipLaunchKernelGGL((prefill_pp_rows<T, D, true>), g, block, 0, s, a, *rows);    \
    else hipLaunchKernelGGL((prefill_pp_rows<T, D, false>), g, block, 0, s, a, *rows);              \
  } while (0)
    if (dtype == LI_BF16) {
      if (a.head_dim == 128) LI_PP_ROWS(li_bf16, 128);
      else LI_PP_ROWS(li_bf16, 64);
    } else {
      if (a.head_dim == 128) LI_PP_ROWS(li_f16, 128);
      else LI_PP_ROWS(li_f16, 64);
    }
#undef LI_PP_ROWS
    if (int rc = check_launch("prefill_pp_rows")) return rc;
    if (int rc = launch_prefill_merge(a, dtype, s)) return rc;
    return launch_combine_balanced(*rows, dtype, s);
  }
  if (a.kv_fp8) {
    if (dtype == LI_BF16) {
      if (direct) hipLaunchKernelGGL((prefill_mfma<li_bf16, 128, W, true, true>), g, block, 0, s, a);
      else hipLaunchKernelGGL((prefill_mfma<li_bf16, 128, W, true, false>), g, block, 0, s, a);
    } else {
      if (direct) hipLaunchKernelGGL((prefill_mfma<li_f16, 128, W, true, true>), g, block, 0, s, a);
      else hipLaunchKernelGGL((prefill_mfma<li_f16, 128, W, true, false>), g, block, 0, s, a);
    }
  } else {
#define LI_PP(T, D)                                                                                 \
  do {                                                                                              \
    if (a.split_ok) hipLaunchKernelGGL((prefill_pp<T, D, true, false>), g, block, 0, s, a);         \
    else if (direct) hipLaunchKernelGGL((prefill_pp<T, D, false, true>), g, block, 0, s, a);        \
    else hipLaunchKernelGGL((prefill_pp<T, D, false, false>), g, block, 0, s, a);                   \
  } while (0)
    if (dtype == LI_BF16) {
      if (a.head_dim == 128) LI_PP(li_bf16, 128);
      else LI_PP(li_bf16, 64);
    } else {
      if (a.head_dim == 128) LI_PP(li_f16, 128);
      else LI_PP(li_f16, 64);
    }
#undef LI_PP
  }
  if (int rc = check_launch("prefill_mfma")) return rc;
  return launch_prefill_merge(a, dtype, s);
}

// After a pass that may be split: one work-group per (work-list entry that
// can hold a piece, KV head); those of a split block's first piece fold it.
static int launch_prefill_merge(const AttnArgs& a, int dtype, hipStream_t s) {
  if (!a.split_ok) return LI_OK;
  const int chunks = kMinRows / (a.head_dim == 128 ? merge_rows<128>() : merge_rows<64>());
  const dim3 g((unsigned)(prefill_split_blocks_cap(a.split_target, a.num_kv_heads) * a.num_kv_heads * chunks)),
      block(256);
  if (dtype == LI_BF16) {
    if (a.head_dim == 128) hipLaunchKernelGGL((prefill_merge<li_bf16, 128>), g, block, 0, s, a);
    else hipLaunchKernelGGL((prefill_merge<li_bf16, 64>), g, block, 0, s, a);
  } else {
    if (a.head_dim == 128) hipLaunchKernelGGL((prefill_merge<li_f16, 128>), g, block, 0, s, a);
    else hipLaunchKernelGGL((prefill_merge<li_f16, 64>), g, block, 0, s, a);
  }
  return check_launch("prefill_merge");
}

int launch_prefill_mfma(const AttnArgs& in, int dtype, hipStream_t s) {
  return launch_prefill_waves<kWaves>(in, dtype, s, nullptr);
}

int launch_prefill_with_rows(const AttnArgs& in, const AttnArgs& d, int dtype, hipStream_t s) {
  if (d.part_heads != 1 || !d.part_o) return fail(LI_EINVAL, "prefill with rows: a per-head decode split only");
  AttnArgs a = in;
  a.single_query_elsewhere = 1;
  return launch_prefill_waves<kWaves>(a, dtype, s, &d);
}


}  // namespace li
