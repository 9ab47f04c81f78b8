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
  int4* pieces;  // balanced decode: per (sequence, KV head) {first wave, last wave, first slot}
  int part_heads;  // balanced decode: KV heads per partial slot (1; kDecodeHeadGroup when head-grouped)
  int seg_cost;    // head-grouped decode: work units charged per segment start, on top of its 32-key tiles
  int* work;     // MFMA prefill: query blocks (sequence * num_qblocks + block), heaviest first; -1 past the end
  int* queue;    // MFMA prefill: kPrefillQueues unit counters, the number of blocks listed in `work`, then
                 // (prefill_pp_rows) the number of work-groups that fold the one-query rows first
  int row_groups_max;  // prefill_pp_rows: work-groups of its grid (0: the one-query rows are not in the launch)
  // fp8 (e4m3) pools: kp / vp hold K / k_scale and V / v_scale, one byte per
  // element (pool strides in bytes); the MFMA kernels only. Other pools hold
  // the query's dtype and ignore the scales.
  int kv_fp8;
  float k_scale, v_scale;
};

// Work queues of the persistent MFMA prefill grid (one per XCD).
constexpr int kPrefillQueues = 8;

// KV heads one wave of the head-grouped balanced decode folds together
// (when num_kv_heads is a multiple of it).
#ifndef LI_DECODE_HEAD_GROUP
#define LI_DECODE_HEAD_GROUP 2
#endif
constexpr int kDecodeHeadGroup = LI_DECODE_HEAD_GROUP;

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
