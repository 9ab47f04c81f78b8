// Arguments and launchers shared by the attention kernels.
#pragma once

#include "li_common.h"

namespace li {

// One launch of an attention kernel, decode or prefill.
//
// Rows: a decode step has one query per sequence, query row i = sequence i
// (qsl == nullptr); a packed pass gives sequence i the query rows
// [qsl[i], qsl[i+1]). Either way a sequence's queries are the last positions
// of its context of ctx[i] keys.
//
// Partitions (decode only): the key axis of each sequence is cut into
// partitions of part_len keys (part_len == 0: cdiv(ctx, num_parts) keys,
// the equal-slice rule). A sequence whose context fits in one partition is
// written straight to `out`; otherwise every partition writes its normalised
// fp32 output to part_o and its log2-domain log-sum-exp to part_lse, and the
// combine kernel folds them.
struct AttnArgs {
  const void* q;
  int64_t q_s0, q_s1;  // element strides: token (or sequence), head
  const void* kp;
  const void* vp;
  int64_t p_s0, p_s1;  // pool strides: slot, head
  const int64_t* st;   // slot table [batch, st_s]
  int64_t st_s;
  const int32_t* ctx;  // [batch]
  const int32_t* qsl;  // [batch + 1] or nullptr for decode
  void* out;
  int64_t o_s0, o_s1;
  float* part_o;    // [batch, num_heads, num_parts, head_dim] or nullptr
  float* part_lse;  // [batch, num_heads, num_parts]
  int batch, num_heads, num_kv_heads, groups, head_dim;
  float scale;
  int num_parts, part_len;
  int block_q, block_kv;  // general-shape kernel tiles
  int num_qblocks;        // query blocks per sequence in the grid
  int max_query_len;      // most queries any sequence brings (prefill)
  int max_context;        // slot-table width (prefill)
  int single_query_elsewhere;  // prefill: one-query sequences are served by the decode kernel
  int4* pieces;  // balanced decode: per (sequence, KV head) {first work-group, last work-group, first slot}
  int part_heads;  // balanced decode: KV heads per partial slot (1; kDecodeHeadGroup when head-grouped)
  int seg_cost;    // head-grouped decode: work units charged per segment start, on top of its 32-key tiles
  int4* work;    // MFMA prefill: query blocks, heaviest first, each {sequence * num_qblocks + block, the
                 // sequence's first query row, its query count, its context length}; only the first
                 // queue[kPrefillQueues] entries are written
  int* queue;    // MFMA prefill: kPrefillQueues unit counters, the number of blocks listed in `work`, then
                 // (prefill_pp_rows) the number of work-groups that fold the one-query rows first
  int row_groups_max;  // prefill_pp_rows: most work-groups that may fold the rows, min(grid, d.num_parts /
                       // kRowWaves) (0: the one-query rows are not in the launch)
  // MFMA prefill of a pass too small to fill the grid (prefill_pp only):
  // prefill_order may cut a block's fully visible key stages into pieces,
  // one work-list entry each, consecutive; each piece folds its stages and
  // stores its rows unnormalised with their running maximum and sum, and
  // prefill_merge folds the pieces into the output. split_ok == 0: never.
  int split_ok;
  int split_target;  // units (entries x KV heads) the pieces should make in all
  int4* work_range;  // per entry {first 64-key stage, end stage, piece, pieces}
  float* split_o;    // [entry * num_kv_heads + KV head][256 rows][head_dim]
  float* split_ml;   // [entry * num_kv_heads + KV head][256 rows]{running maximum, sum}
  int* split_first;  // the first entry of each split block; their count: queue[kPrefillQueues + 2]
  // fp8 (e4m3) pools: kp / vp hold K / k_scale and V / v_scale, one byte per
  // element (pool strides in bytes); the MFMA kernels only. Other pools hold
  // the query's dtype and ignore the scales.
  int kv_fp8;
  float k_scale, v_scale;
  // Head-grouped decode over a 16-bit pool: each sequence's newest K / V
  // rows, [batch, num_kv_heads, head_dim] with element strides (n_s0, n_s1,
  // 1), written to slot st[seq, ctx - 1] by the wave that folds that key
  // (which folds them from registers, not from the pool); nullptr: none.
  const void* new_k;
  const void* new_v;
  int64_t n_s0, n_s1;
  int64_t num_slots;  // the pool's slots: a newest row whose slot is outside is not stored
  int* bad;           // nullable: counts sequences whose newest slot is outside the pool
};

// Work queues of the persistent MFMA prefill grid (one per XCD).
constexpr int kPrefillQueues = 8;
// Rows of a prefill unit (8 waves of 32), and the fewest 64-key stages a
// piece of a split unit holds.
constexpr int kPrefillUnitRows = 256;
constexpr int kSplitMinStages = 8;
constexpr int kSplitMaxPieces = 32;
// Split blocks a pass cut to at most `target` units can hold: each has two
// pieces or more, and the pieces are at most target / num_kv_heads entries.
inline int prefill_split_blocks_cap(int target, int num_kv_heads) {
  return (target + 2 * num_kv_heads - 1) / (2 * num_kv_heads);
}
// Ints of a prefill launch's queue array: the per-XCD unit counters, the
// listed entries, the row work-groups, the split blocks.
constexpr int kPrefillQueueInts = kPrefillQueues + 3;

// Decode waves per work-group of a prefill launch that folds the pass's
// one-query rows first (prefill_pp_rows, prefill_mfma_rows). (Eight waves
// of one tile stage each measured the same row throughput per work-group,
// ~36-40 GB/s: a CU gathers scattered 256-byte rows at up to ~50 GB/s
// whether into LDS or registers, by a standalone probe.)
constexpr int kRowWaves = 4;

// Flops of chunk work per byte of row K/V that put the rows' end at about
// three quarters of the chunks' (prefill_row_groups): a CU of the ping-pong
// kernel folds ~4.3 TFLOP/s of causal pairs (C3-like chunks, ~44% of the
// bf16 peak over 256 CUs), and a work-group of four decode waves streams
// ~36 GB/s beside the chunks' work-groups (both measured on MI355X: config
// 3's step is flat at 307 us from 48 to 80 row work-groups and rises to
// 340 / 407 us at 40 / 32), so the rows need B / 36e9 s of one CU for every
// F / 4.3e12 s of chunks: 4.3e12 / (0.75 * 36e9) ~ 160.
constexpr double kRowFlopsPerByte = 160.0;

// Most work-groups of a prefill launch of `grid` work-groups that may fold
// the one-query rows: each takes kRowWaves waves of a balanced split whose
// workspace holds partial slots for `split_waves` waves.
__host__ __device__ inline int prefill_row_cap(long long grid, int split_waves) {
  const long long by_slots = split_waves > 0 ? split_waves / kRowWaves : 0;
  const long long cap = grid < by_slots ? grid : by_slots;
  return cap > 0 ? (int)cap : 0;
}

// How many work-groups of a prefill launch fold the one-query rows first:
// the one rule the device (prefill_order) and the host-side planner and
// tests use. row_keys: the rows' keys (sum of their contexts); chunk_pairs:
// the chunks' visible causal (query, key) pairs; listed_blocks: the chunks'
// query blocks; cap: the most row work-groups the launch can hold, which is
// min(grid, partial slots of the workspace / kRowWaves), set on the host.
// The rows' K/V bytes against the chunks' flops, scaled by
// kRowFlopsPerByte, rounded to a multiple of the queue count (every XCD
// gives the rows the same CUs), at least one per queue, and leaving each
// chunk unit a work-group up to half the cap; never above `cap`, never
// negative, 0 when there are no rows.
__host__ __device__ inline int prefill_row_groups(unsigned long long row_keys, unsigned long long chunk_pairs,
                                                  int listed_blocks, int cap, int num_kv_heads, int num_heads,
                                                  int head_dim, int kv_fp8) {
  if (cap <= 0 || row_keys == 0) return 0;
  if (chunk_pairs == 0) return cap;
  const double bytes = (double)row_keys * 2.0 * num_kv_heads * head_dim * (kv_fp8 ? 1.0 : 2.0);
  const double flops = (double)chunk_pairs * 4.0 * num_heads * head_dim;
  double want = cap * kRowFlopsPerByte * bytes / flops;
  if (!(want < (double)cap)) want = (double)cap;  // also a NaN; keeps the conversion in range
  const long long units = (long long)(listed_blocks > 0 ? listed_blocks : 0) * num_kv_heads;
  long long keep = (units + kPrefillQueues - 1) / kPrefillQueues;
  if (keep > cap / 2 / kPrefillQueues) keep = cap / 2 / kPrefillQueues;
  keep *= kPrefillQueues;
  if (keep < kPrefillQueues) keep = kPrefillQueues;
  long long groups = (long long)(want / kPrefillQueues + 0.5) * kPrefillQueues;
  const long long limit = (cap - keep) / kPrefillQueues * kPrefillQueues;
  if (groups > limit) groups = limit;
  if (groups < kPrefillQueues) groups = kPrefillQueues;
  return (int)(groups < cap ? groups : cap);
}

// KV heads one wave of the head-grouped balanced decode folds together
// (when num_kv_heads is a multiple of it).
#ifndef LI_DECODE_HEAD_GROUP
#define LI_DECODE_HEAD_GROUP 2
#endif
constexpr int kDecodeHeadGroup = LI_DECODE_HEAD_GROUP;
// Head groups of the head-grouped decode whose waves share one work-group
// (and so one CU), each folding the same keys of its own group: at most
// this many, the largest power of two dividing the group count.
#ifndef LI_DECODE_CU_GROUPS
#define LI_DECODE_CU_GROUPS 4
#endif
constexpr int kDecodeCuGroups = LI_DECODE_CU_GROUPS;

// Largest head_dim the general-shape kernel serves.
constexpr int kGenericMaxHeadDim = 512;
// Largest head_dim the MFMA decode and prefill kernels serve (64 or 128).
constexpr int kMfmaMaxHeadDim = 128;

int launch_attend_generic(const AttnArgs& a, int dtype, hipStream_t s);
int launch_combine(const AttnArgs& a, int dtype, hipStream_t s);

// MFMA decode: bf16 / fp16, head_dim 64 or 128, up to 16 query heads per KV
// head, every row 16-byte aligned. Returns LI_EUNSUPPORTED when not
// applicable (nothing launched).
bool decode_mfma_applies(const AttnArgs& a, int dtype);
int launch_decode_mfma(const AttnArgs& a, int dtype, hipStream_t s);

// Short decode (decode_short, decode_mfma.hip): one work-group per
// (sequence, KV head) whose waves split the context and merge their states
// in LDS, for launches whose contexts are all short (max_context, the slot
// table's width, bounds them): one launch, no partial rows, no combine.
// kShortChunk is the slots a wave stages at a time.
constexpr int kShortChunk = 256;
// Sequences of a packed pass the direct prefill schedule serves (a pass
// whose every unit has a work-group of its own, no one-query rows in the
// launch, no split: no work list; work-group i takes
// unit i / (queue count) of its queue, found by one wave's scan of the
// sequences' query counts, and nothing after it).
constexpr int kPrefillDirectBatch = 64;
// Its rule: segments (sequence, KV head) x max_context at most
// kShortMaxKeySegments, and max_context at most kShortMaxWidth, or twice that
// with at least kShortWideSegments segments.
constexpr long long kShortMaxKeySegments = 1 << 19;
constexpr int kShortMaxWidth = 1024;
constexpr int kShortWideSegments = 128;
bool decode_short_applies(const AttnArgs& a, int dtype, int max_context);
int launch_decode_short(const AttnArgs& a, int dtype, hipStream_t s);

// MFMA prefill: same applicability rules as decode.
bool prefill_mfma_applies(const AttnArgs& a, int dtype);
int launch_prefill_mfma(const AttnArgs& a, int dtype, hipStream_t s);
// A packed pass whose one-query rows (the balanced decode split, `d`:
// part_heads 1, its workspace set) share the prefill launch: the
// first work-groups fold the rows, then join the chunks' queues; the rows'
// pieces are combined after. `a` as for launch_prefill_mfma.
int launch_prefill_with_rows(const AttnArgs& a, const AttnArgs& d, int dtype, hipStream_t s);
// The combine of the balanced split's pieces (decode_mfma.hip).
int launch_combine_balanced(const AttnArgs& d, int dtype, hipStream_t s);
// Entries of the MFMA prefill work list for a pass over a slot table
// max_context wide: an upper bound on its query blocks.
size_t prefill_work_entries(int batch, int max_context);

}  // namespace li
