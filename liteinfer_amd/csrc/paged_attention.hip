// C ABI of paged decode and packed prefill: argument checks, the decode
// partition policy, and dispatch to the MFMA or the general-shape kernels.
#include "li_attention.h"

#include <cmath>

#include <cstdlib>
#include <mutex>

namespace li {
namespace {

// Decode partition policy (counterpart of choose_num_splits,
// liteinfer/models/paged_kernels.py:645-693, re-tuned for MI355X).
//
// A partition is one wave64 reading its keys' K and V rows straight from the
// pool. Only the batch rows times KV heads are free parallelism; MI355X has
// 256 CUs, and streaming HBM at full rate wants several waves per CU in
// flight, so each sequence's keys are cut into partitions until the grid
// reaches kTargetWavesPerCu waves per CU. Partitions have a FIXED length
// (the same for every row of the batch), never longer than kMaxPartition keys,
// so a long context is cut more finely than a short one and every wave
// carries about the same bytes whatever the spread of context lengths.
constexpr int kTargetWavesPerCu = 8;
constexpr int kMaxPartition = 1024;
constexpr int kMinTilesToSplit = 4;
constexpr int kMaxPartitions = 1024;
constexpr int kDefaultBlockKv = 64;

int round_up(int x, int m) { return (x + m - 1) / m * m; }

// Returns the partition count of the grid and the fixed partition length
// (0 when the whole context is one partition).
void decode_policy(int batch, int num_kv_heads, int max_context, int num_cus, int block_kv,
                   int* parts, int* plen) {
  const int target = kTargetWavesPerCu;
  const int max_part = kMaxPartition;
  const int tile = block_kv > 0 ? block_kv : kDefaultBlockKv;
  *parts = 1;
  *plen = 0;
  if (max_context <= 0 || cdiv(max_context, tile) < kMinTilesToSplit) return;
  const int64_t rows = (int64_t)std::max(batch, 1) * std::max(num_kv_heads, 1);
  const int64_t want = std::max<int64_t>(1, (int64_t)target * num_cus / rows);
  if (want <= 1) return;  // the unsplit grid already fills the device
  int len = round_up((int)cdiv64(max_context, want), tile);
  len = std::max(tile, std::min(len, std::max(tile, round_up(max_part, tile))));
  int n = cdiv(max_context, len);
  if (n > kMaxPartitions) {
    len = round_up(cdiv(max_context, kMaxPartitions), tile);
    n = cdiv(max_context, len);
  }
  if (n <= 1) return;
  *parts = n;
  *plen = len;
}

size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

size_t decode_workspace(int batch, int num_heads, int head_dim, int parts) {
  if (parts <= 1) return 0;
  const size_t rows = (size_t)batch * num_heads * parts;
  return align256(rows * head_dim * sizeof(float)) + align256(rows * sizeof(float));
}

// Balanced decode (the MFMA kernel's automatic mode): a fixed grid of waves,
// kBalancedWavesPerCu per CU (the LDS of four waves fills a CU), splits the
// flattened key space into equal shares; each wave keeps up to two fp32
// partials of `groups` heads.
constexpr int kBalancedWavesPerCu = 4;
constexpr int kSegmentCost = 2;

int balanced_waves(int num_cus) {
  return std::max(1, num_cus) * kBalancedWavesPerCu;
}

// KV heads per partial slot of the balanced split: kDecodeHeadGroup times
// the head groups sharing a work-group when the head-grouped kernel serves
// the shape (num_kv_heads a multiple of the group), else one. Grouping pays
// on 16-bit pools (config 2: 204 -> 196 us) and on fp8 ones, whose scores
// run on the fp8 matrix cores (config 2: 112.5 -> 108 us; config 4
// unchanged; four heads per wave: 116 / 208 us).
int balanced_part_heads(int num_kv_heads) {
  if (num_kv_heads % kDecodeHeadGroup) return 1;
  const int ngroups = num_kv_heads / kDecodeHeadGroup;
  int together = 1;
  while (together < kDecodeCuGroups && ngroups % (2 * together) == 0) together *= 2;
  return kDecodeHeadGroup * together;
}

// Work-groups of the balanced split over `waves` waves: one wave each, or
// one per head group sharing a work-group.
int balanced_blocks(int waves, int part_heads) {
  return part_heads % kDecodeHeadGroup == 0 ? waves / (part_heads / kDecodeHeadGroup) : waves;
}

// What starting a segment (its query, its slots, the ring's first tile)
// costs the head-grouped decode, in 32-key tiles: the balanced split charges
// it so that waves meeting many short contexts take fewer tiles.
int segment_cost() { return kSegmentCost; }

size_t balanced_workspace(int waves, int groups, int head_dim, int batch, int num_kv_heads) {
  // Sized for either pool type (the plan calls do not know it).
  const int ph = balanced_part_heads(num_kv_heads);
  const size_t rows = (size_t)balanced_blocks(waves, ph) * 2 * groups * ph;
  return align256(rows * head_dim * sizeof(float)) + align256(rows * sizeof(float)) +
         align256((size_t)batch * num_kv_heads * 16);
}

size_t newest_slot_bytes(int batch) { return align256((size_t)std::max(batch, 0) * sizeof(int64_t)); }

// slots[i] = slot_table[i, ctx[i] - 1]: where li_paged_decode_write's newest
// rows go when a separate write stores them; -1 (skipped by the write) for
// an empty context, and for a slot outside the pool, which is counted into
// *bad as the fused kernel counts it.
__global__ __launch_bounds__(256) void newest_slots_kernel(const int64_t* table, int64_t table_stride,
                                                           const int32_t* ctx, int batch, int64_t num_slots,
                                                           int32_t* bad, int64_t* slots) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= batch) return;
  const int c = ctx[i];
  int64_t slot = c > 0 ? table[(int64_t)i * table_stride + c - 1] : -1;
  if (c > 0 && (slot < 0 || slot >= num_slots)) {
    if (bad) atomicAdd(bad, 1);
    slot = -1;
  }
  slots[i] = slot;
}

// Points a balanced launch's partial buffers and piece table into `workspace`.
void set_balanced(AttnArgs& d, int waves, void* workspace) {
  d.part_heads = balanced_part_heads(d.num_kv_heads);
  d.num_parts = balanced_blocks(waves, d.part_heads);
  d.part_len = -1;
  d.seg_cost = segment_cost();
  const size_t rows = (size_t)d.num_parts * 2 * d.groups * d.part_heads;
  char* p = static_cast<char*>(workspace);
  d.part_o = reinterpret_cast<float*>(p);
  p += align256(rows * d.head_dim * sizeof(float));
  d.part_lse = reinterpret_cast<float*>(p);
  p += align256(rows * sizeof(float));
  d.pieces = reinterpret_cast<int4*>(p);
}

int check_common(int dtype, int num_heads, int num_kv_heads, int head_dim, const char* who) {
  if (dtype_size(dtype) == 0 || dtype == LI_FP8_E4M3) return fail(LI_EINVAL, "%s: unknown query dtype %d", who, dtype);
  if (num_heads <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads != 0)
    return fail(LI_EINVAL, "%s: %d query heads cannot be grouped over %d KV heads", who, num_heads, num_kv_heads);
  if (head_dim <= 0 || head_dim > kGenericMaxHeadDim)
    return fail(LI_EUNSUPPORTED, "%s: head_dim %d is outside 1..%d", who, head_dim, kGenericMaxHeadDim);
  return LI_OK;
}

// li_paged_decode_write's newest K / V rows: [batch, num_kv_heads, head_dim]
// with element strides (s0, s1, 1), for slot slot_table[i, ctx[i] - 1].
struct NewestRows {
  const void* k;  // nullptr: no rows to write
  const void* v;
  int64_t s0, s1;
  int64_t num_slots;
  int32_t* bad;
};

}  // namespace
}  // namespace li

using namespace li;

// The reference's split-count rule (liteinfer/models/paged_kernels.py:
// 645-693, constants :129-150), with compute units in place of SMs: a
// context of fewer than four key tiles is not cut; otherwise the count that
// brings the grid of batch * num_kv_heads programs up to two per CU, at most
// one per key tile and at most 32. An empty batch takes 1 (the reference
// would divide by zero).
constexpr int kRefTargetProgramsPerCu = 2;
constexpr int kRefMaxSplits = 32;
constexpr int kRefMinTilesToSplit = 4;

extern "C" int li_choose_num_splits(int batch, int num_kv_heads, int max_context, int num_cus, int block_kv) {
  clear_error();
  if (batch < 0 || num_kv_heads <= 0 || max_context < 0)
    return fail(LI_EINVAL, "li_choose_num_splits: bad extents (batch=%d kv_heads=%d max_context=%d)", batch,
                num_kv_heads, max_context);
  if (num_cus <= 0) num_cus = device_cu_count();
  const int tile = block_kv > 0 ? block_kv : kDefaultBlockKv;
  const int64_t tiles = cdiv64(max_context, tile);
  if (tiles < kRefMinTilesToSplit || batch == 0) return 1;
  const int64_t programs = (int64_t)batch * num_kv_heads;
  const int64_t target = (int64_t)kRefTargetProgramsPerCu * num_cus;
  return (int)std::max<int64_t>(1, std::min<int64_t>(std::min<int64_t>(target / programs, tiles), kRefMaxSplits));
}

extern "C" int li_paged_decode_plan(int batch, int num_heads, int num_kv_heads, int head_dim, int max_context,
                                    int num_splits, int num_cus, int block_kv, int* num_partitions,
                                    int* partition_len, size_t* workspace_bytes) {
  clear_error();
  if (int rc = check_common(LI_BF16, num_heads, num_kv_heads, head_dim, "li_paged_decode_plan")) return rc;
  if (num_splits < 0) return fail(LI_EINVAL, "num_splits must be >= 1, got %d", num_splits);
  if (batch < 0 || max_context < 0) return fail(LI_EINVAL, "li_paged_decode_plan: negative extent");
  int parts = 1, plen = 0;
  if (num_splits == 0) {
    if (num_cus <= 0) num_cus = device_cu_count();
    decode_policy(batch, num_kv_heads, max_context, num_cus, block_kv, &parts, &plen);
  } else {
    parts = num_splits;
    plen = 0;
  }
  if (num_partitions) *num_partitions = parts;
  if (partition_len) *partition_len = plen;
  size_t need = decode_workspace(batch, num_heads, head_dim, parts);
  // The MFMA kernel runs the balanced split unless LI_FLAG_EQUAL_SPLITS pins
  // the partitions; size for either. The balanced grid is sized from the
  // current device's CU count whatever num_cus says, as the launch sizes it.
  need = std::max(need, balanced_workspace(balanced_waves(device_cu_count()), num_heads / num_kv_heads, head_dim,
                                           batch, num_kv_heads));
  // Then the newest rows' slots li_paged_decode_write stages when its kernel
  // does not write them itself.
  need += newest_slot_bytes(batch);
  if (workspace_bytes) *workspace_bytes = need;
  return LI_OK;
}

// The pool's element type against the query's: the same type, or fp8 (e4m3)
// with scales, which only the MFMA kernels read.
int check_kv(int dtype, int kv_dtype, float k_scale, float v_scale, const char* who) {
  if (kv_dtype == dtype) return LI_OK;
  if (kv_dtype != LI_FP8_E4M3)
    return fail(LI_EINVAL, "%s: pool dtype %d does not match the query's %d", who, kv_dtype, dtype);
  if (!(k_scale > 0.f) || !(v_scale > 0.f) || !std::isfinite(k_scale) || !std::isfinite(v_scale))
    return fail(LI_EINVAL, "%s: fp8 pool scales must be finite and > 0 (k_scale=%g, v_scale=%g)", who, k_scale,
                v_scale);
  return LI_OK;
}

int paged_decode_impl(const void* q, int64_t q_stride_seq, int64_t q_stride_head, const void* key_pool,
                      const void* value_pool, int64_t pool_stride_slot, int64_t pool_stride_head,
                      const int64_t* slot_table, int64_t slot_table_stride, int max_context,
                      const int32_t* context_lens, void* out, int64_t out_stride_seq, int64_t out_stride_head,
                      int batch, int num_heads, int num_kv_heads, int head_dim, float scale, int num_splits,
                      int block_kv, void* workspace, size_t workspace_bytes, int dtype, int kv_dtype, float k_scale,
                      float v_scale, int flags, void* stream, const NewestRows* newest = nullptr) {
  clear_error();
  if (int rc = check_common(dtype, num_heads, num_kv_heads, head_dim, "li_paged_decode")) return rc;
  if (int rc = check_kv(dtype, kv_dtype, k_scale, v_scale, "li_paged_decode")) return rc;
  if (num_splits < 0) return fail(LI_EINVAL, "num_splits must be >= 1, got %d", num_splits);
  if (batch < 0 || max_context < 0) return fail(LI_EINVAL, "li_paged_decode: negative extent");
  if (batch == 0) return LI_OK;
  if (!q || !key_pool || !value_pool || !slot_table || !context_lens || !out)
    return fail(LI_EINVAL, "li_paged_decode: null pointer");

  int parts = 1, plen = 0;
  size_t need = 0;
  if (int rc = li_paged_decode_plan(batch, num_heads, num_kv_heads, head_dim, max_context, num_splits, 0, block_kv,
                                    &parts, &plen, &need))
    return rc;
  if (need > 0 && (!workspace || workspace_bytes < need))
    return fail(LI_EWORKSPACE, "li_paged_decode: workspace of %zu bytes given, %zu needed", workspace_bytes, need);

  AttnArgs a{};
  a.q = q;
  a.q_s0 = q_stride_seq;
  a.q_s1 = q_stride_head;
  a.kp = key_pool;
  a.vp = value_pool;
  a.p_s0 = pool_stride_slot;
  a.p_s1 = pool_stride_head;
  a.st = slot_table;
  a.st_s = slot_table_stride;
  a.ctx = context_lens;
  a.qsl = nullptr;
  a.out = out;
  a.o_s0 = out_stride_seq;
  a.o_s1 = out_stride_head;
  a.batch = batch;
  a.num_heads = num_heads;
  a.num_kv_heads = num_kv_heads;
  a.groups = num_heads / num_kv_heads;
  a.head_dim = head_dim;
  a.scale = scale;
  a.num_parts = parts;
  a.part_len = plen;
  a.block_q = 1;
  a.block_kv = block_kv > 0 ? block_kv : kDefaultBlockKv;
  a.num_qblocks = 1;
  a.kv_fp8 = kv_dtype == LI_FP8_E4M3;
  a.k_scale = k_scale;
  a.v_scale = v_scale;
  if (parts > 1) {
    const size_t rows = (size_t)batch * num_heads * parts;
    a.part_o = static_cast<float*>(workspace);
    a.part_lse = reinterpret_cast<float*>(static_cast<char*>(workspace) + align256(rows * head_dim * sizeof(float)));
  }

  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool mfma = !(flags & LI_FLAG_FORCE_GENERIC) && decode_mfma_applies(a, dtype);
  if (a.kv_fp8 && !mfma)
    return fail(LI_EUNSUPPORTED,
                "li_paged_decode: fp8 pools run on the MFMA kernel only (bf16 / fp16 queries, head_dim 128, "
                "16-byte aligned rows)");
  // Every context short (the table's width bounds them): one work-group per
  // (sequence, KV head), one launch. A pinned split count keeps its kernel.
  const bool short_call = mfma && !(flags & LI_FLAG_EQUAL_SPLITS) && decode_short_applies(a, dtype, max_context);
  const bool balanced = !short_call && mfma && (num_splits == 0 || !(flags & LI_FLAG_EQUAL_SPLITS));
  const bool grouped = balanced && balanced_part_heads(num_kv_heads) % kDecodeHeadGroup == 0;
  if (newest && newest->k) {
    // The head-grouped and short kernels over a 16-bit pool write the newest
    // rows themselves (16-byte aligned rows); anywhere else a write of them
    // runs first, into the slots the table names.
    const int esize = dtype_size(dtype);
    const bool fused = (grouped || short_call) && !a.kv_fp8 && aligned16(newest->k) && aligned16(newest->v) &&
                       (newest->s0 * esize) % 16 == 0 && (newest->s1 * esize) % 16 == 0;
    if (fused) {
      a.new_k = newest->k;
      a.new_v = newest->v;
      a.n_s0 = newest->s0;
      a.n_s1 = newest->s1;
      a.num_slots = newest->num_slots;
      a.bad = newest->bad;
    } else {
      int64_t* slots = reinterpret_cast<int64_t*>(static_cast<char*>(workspace) + need - newest_slot_bytes(batch));
      hipLaunchKernelGGL(newest_slots_kernel, dim3((unsigned)cdiv(batch, 256)), dim3(256), 0, s, slot_table,
                         slot_table_stride, context_lens, batch, newest->num_slots, newest->bad, slots);
      if (int rc = check_launch("newest_slots")) return rc;
      const int64_t strides[4] = {newest->s0, newest->s1, 0, 1};
      int rc = a.kv_fp8 ? li_kv_scatter_fp8(newest->k, newest->v, strides, strides, batch, 1, slots,
                                            const_cast<void*>(key_pool), const_cast<void*>(value_pool),
                                            newest->num_slots, pool_stride_slot, pool_stride_head, num_kv_heads,
                                            head_dim, dtype, k_scale, v_scale, nullptr, stream)
                        : li_kv_scatter(newest->k, newest->v, strides, strides, batch, 1, slots,
                                        const_cast<void*>(key_pool), const_cast<void*>(value_pool), newest->num_slots,
                                        pool_stride_slot, pool_stride_head, num_kv_heads, head_dim, dtype,
                                        nullptr, stream);
      if (rc) return rc;
      clear_error();
    }
  }
  if (short_call) return launch_decode_short(a, dtype, s);
  if (balanced) {
    // The MFMA kernel's schedule: the balanced split (it launches its own
    // combine). A split count the caller chose (the engine passes
    // choose_num_splits's) is a scheduling hint; LI_FLAG_EQUAL_SPLITS makes
    // it the partition count.
    const int waves = balanced_waves(device_cu_count());
    const size_t bneed = balanced_workspace(waves, a.groups, head_dim, batch, num_kv_heads);
    if (bneed > workspace_bytes || !workspace)
      return fail(LI_EWORKSPACE, "li_paged_decode: workspace of %zu bytes given, %zu needed", workspace_bytes, bneed);
    set_balanced(a, waves, workspace);
    return launch_decode_mfma(a, dtype, s);
  }
  int rc = mfma ? launch_decode_mfma(a, dtype, s) : launch_attend_generic(a, dtype, s);
  if (rc) return rc;
  if (parts > 1) rc = launch_combine(a, dtype, s);
  return rc;
}

extern "C" int li_paged_decode(const void* q, int64_t q_stride_seq, int64_t q_stride_head, const void* key_pool,
                               const void* value_pool, int64_t pool_stride_slot, int64_t pool_stride_head,
                               const int64_t* slot_table, int64_t slot_table_stride, int max_context,
                               const int32_t* context_lens, void* out, int64_t out_stride_seq,
                               int64_t out_stride_head, int batch, int num_heads, int num_kv_heads, int head_dim,
                               float scale, int num_splits, int block_kv, void* workspace, size_t workspace_bytes,
                               int dtype, int flags, void* stream) {
  return paged_decode_impl(q, q_stride_seq, q_stride_head, key_pool, value_pool, pool_stride_slot, pool_stride_head,
                           slot_table, slot_table_stride, max_context, context_lens, out, out_stride_seq,
                           out_stride_head, batch, num_heads, num_kv_heads, head_dim, scale, num_splits, block_kv,
                           workspace, workspace_bytes, dtype, dtype, 1.f, 1.f, flags, stream);
}

extern "C" int li_paged_decode_ex(const void* q, int64_t q_stride_seq, int64_t q_stride_head, const void* key_pool,
                                  const void* value_pool, int64_t pool_stride_slot, int64_t pool_stride_head,
                                  const int64_t* slot_table, int64_t slot_table_stride, int max_context,
                                  const int32_t* context_lens, void* out, int64_t out_stride_seq,
                                  int64_t out_stride_head, int batch, int num_heads, int num_kv_heads, int head_dim,
                                  float scale, int num_splits, int block_kv, void* workspace,
                                  size_t workspace_bytes, int dtype, int kv_dtype, float k_scale, float v_scale,
                                  int flags, void* stream) {
  return paged_decode_impl(q, q_stride_seq, q_stride_head, key_pool, value_pool, pool_stride_slot, pool_stride_head,
                           slot_table, slot_table_stride, max_context, context_lens, out, out_stride_seq,
                           out_stride_head, batch, num_heads, num_kv_heads, head_dim, scale, num_splits, block_kv,
                           workspace, workspace_bytes, dtype, kv_dtype, k_scale, v_scale, flags, stream);
}

extern "C" int li_paged_decode_write(const void* q, int64_t q_stride_seq, int64_t q_stride_head,
                                     const void* key_pool, const void* value_pool, int64_t pool_stride_slot,
                                     int64_t pool_stride_head, const int64_t* slot_table, int64_t slot_table_stride,
                                     int max_context, const int32_t* context_lens, const void* new_key,
                                     const void* new_value, int64_t new_stride_seq, int64_t new_stride_head,
                                     int64_t num_slots, int32_t* bad_slots, void* out, int64_t out_stride_seq,
                                     int64_t out_stride_head, int batch, int num_heads, int num_kv_heads,
                                     int head_dim, float scale, int num_splits, int block_kv, void* workspace,
                                     size_t workspace_bytes, int dtype, int kv_dtype, float k_scale, float v_scale,
                                     int flags, void* stream) {
  clear_error();
  if (!new_key != !new_value) return fail(LI_EINVAL, "li_paged_decode_write: give both newest K and V rows, or neither");
  if (num_slots < 0) return fail(LI_EINVAL, "li_paged_decode_write: negative pool size");
  if (new_key && (new_stride_seq < 0 || new_stride_head < 0))
    return fail(LI_EINVAL, "li_paged_decode_write: negative newest-row strides");
  const NewestRows newest{new_key, new_value, new_stride_seq, new_stride_head, num_slots, bad_slots};
  return paged_decode_impl(q, q_stride_seq, q_stride_head, key_pool, value_pool, pool_stride_slot, pool_stride_head,
                           slot_table, slot_table_stride, max_context, context_lens, out, out_stride_seq,
                           out_stride_head, batch, num_heads, num_kv_heads, head_dim, scale, num_splits, block_kv,
                           workspace, workspace_bytes, dtype, kv_dtype, k_scale, v_scale, flags, stream, &newest);
}

// The no-allocation decode: the workspace li_paged_decode would take lives in
// a device array of this file (every GPU the library runs on holds its own
// copy until the process ends). In host code the array's name stands for no
// device address, so it is only ever reached through the address
// hipGetSymbolAddress reports, looked up once per device and kept.
static __device__ __align__(256) char g_decode_scratch[LI_DECODE_NOALLOC_SCRATCH_BYTES];

namespace li {
namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_lock;
void* g_scratch_ptr[kMaxDevices];

// This device's copy of g_decode_scratch, or nullptr (and the error set).
void* decode_scratch() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    fail(LI_ELAUNCH, "li_paged_decode_noalloc: no current HIP device");
    return nullptr;
  }
  std::lock_guard<std::mutex> guard(g_scratch_lock);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    const hipError_t rc = hipGetSymbolAddress(&p, HIP_SYMBOL(g_decode_scratch));
    if (rc != hipSuccess || !p) {
      fail(LI_ELAUNCH, "li_paged_decode_noalloc: scratch address on device %d: %s", dev, hipGetErrorString(rc));
      return nullptr;
    }
    g_scratch_ptr[dev] = p;
  }
  return g_scratch_ptr[dev];
}

}  // namespace
}  // namespace li

extern "C" int li_paged_decode_noalloc(const void* q, int64_t q_stride_seq, int64_t q_stride_head,
                                       const void* key_pool, const void* value_pool, int64_t pool_stride_slot,
                                       int64_t pool_stride_head, const int64_t* slot_table,
                                       int64_t slot_table_stride, int max_context, const int32_t* context_lens,
                                       void* out, int64_t out_stride_seq, int64_t out_stride_head, int batch,
                                       int num_heads, int num_kv_heads, int head_dim, float scale, int num_splits,
                                       int block_kv, int dtype, int flags, void* stream) {
  clear_error();
  if (int rc = check_common(dtype, num_heads, num_kv_heads, head_dim, "li_paged_decode_noalloc")) return rc;
  if (num_splits < 0) return fail(LI_EINVAL, "num_splits must be >= 1, got %d", num_splits);
  if (batch < 0 || max_context < 0) return fail(LI_EINVAL, "li_paged_decode_noalloc: negative extent");
  if (batch == 0) return LI_OK;
  size_t need = 0;
  if (int rc = li_paged_decode_plan(batch, num_heads, num_kv_heads, head_dim, max_context, num_splits, 0, block_kv,
                                    nullptr, nullptr, &need))
    return rc;
  if (need > (size_t)LI_DECODE_NOALLOC_SCRATCH_BYTES)
    return fail(LI_EWORKSPACE,
                "li_paged_decode_noalloc: this call needs %zu bytes of scratch, more than the %zu the library "
                "holds; use li_paged_decode with a workspace",
                need, (size_t)LI_DECODE_NOALLOC_SCRATCH_BYTES);
  void* scratch = decode_scratch();
  if (!scratch) return LI_ELAUNCH;
  return paged_decode_impl(q, q_stride_seq, q_stride_head, key_pool, value_pool, pool_stride_slot, pool_stride_head,
                           slot_table, slot_table_stride, max_context, context_lens, out, out_stride_seq,
                           out_stride_head, batch, num_heads, num_kv_heads, head_dim, scale, num_splits, block_kv,
                           scratch, (size_t)LI_DECODE_NOALLOC_SCRATCH_BYTES, dtype, dtype, 1.f, 1.f, flags, stream);
}

// The persistent prefill grid: one work-group per CU, a multiple of the
// queue count.
int prefill_grid() { return (device_cu_count() + kPrefillQueues - 1) / kPrefillQueues * kPrefillQueues; }

// Whether a pass of `batch` sequences may be split (prefill_order cuts the
// blocks of a pass that leaves most of the grid idle): at least one block
// per sequence and KV head must leave half the grid free. The workspace of
// such a batch holds the pieces' partial rows: one 256-row slot per unit of
// the grid (a split pass lists at most grid / num_kv_heads entries).
bool prefill_split_room(int batch, int num_kv_heads) {
  return batch <= 1024 && (int64_t)batch * num_kv_heads * 2 <= prefill_grid();
}

size_t prefill_split_bytes(int batch, int num_kv_heads, int head_dim) {
  if (!prefill_split_room(batch, num_kv_heads)) return 0;
  const size_t rows = (size_t)prefill_grid() * kPrefillUnitRows;
  return align256(rows * head_dim * sizeof(float)) + align256(rows * 2 * sizeof(float)) +
         align256((size_t)prefill_split_blocks_cap(prefill_grid(), num_kv_heads) * sizeof(int));
}

// Work-list entries: the blocks, and a split pass's pieces.
size_t prefill_list_entries(int batch, int num_kv_heads, int max_context) {
  return prefill_work_entries(batch, max_context) +
         (prefill_split_room(batch, num_kv_heads) ? (size_t)cdiv(prefill_grid(), num_kv_heads) : 0);
}

// Workspace of the MFMA prefill path: the balanced decode kernel's partials
// for the one-query sequences, then the prefill work list, its queues, the
// entries' stage ranges and a split pass's partial rows.
size_t prefill_workspace(int waves, int groups, int head_dim, int batch, int num_kv_heads, int max_context) {
  const size_t entries = prefill_list_entries(batch, num_kv_heads, max_context);
  return balanced_workspace(waves, groups, head_dim, batch, num_kv_heads) + align256(entries * sizeof(int4)) +
         align256(kPrefillQueueInts * sizeof(int)) + align256(entries * sizeof(int4)) +
         prefill_split_bytes(batch, num_kv_heads, head_dim);
}

extern "C" int li_paged_prefill_plan(int batch, int num_heads, int num_kv_heads, int head_dim, int max_context,
                                     int num_cus, size_t* workspace_bytes) {
  clear_error();
  if (int rc = check_common(LI_BF16, num_heads, num_kv_heads, head_dim, "li_paged_prefill_plan")) return rc;
  if (batch < 0 || max_context < 0) return fail(LI_EINVAL, "li_paged_prefill_plan: negative extent");
  // Sized for the current device's CU count (the launch's), whatever
  // num_cus says.
  (void)num_cus;
  if (workspace_bytes)
    *workspace_bytes = prefill_workspace(balanced_waves(device_cu_count()), num_heads / num_kv_heads, head_dim, batch,
                                         num_kv_heads, max_context);
  return LI_OK;
}

extern "C" int li_prefill_row_groups(unsigned long long row_keys, unsigned long long chunk_pairs, int listed_blocks,
                                     int grid, int split_waves, int num_kv_heads, int num_heads, int head_dim,
                                     int kv_fp8) {
  clear_error();
  if (grid < 0 || split_waves < 0 || listed_blocks < 0 || num_kv_heads <= 0 || num_heads <= 0 || head_dim <= 0)
    return fail(LI_EINVAL, "li_prefill_row_groups: negative or empty extent");
  return prefill_row_groups(row_keys, chunk_pairs, listed_blocks, prefill_row_cap(grid, split_waves), num_kv_heads,
                            num_heads, head_dim, kv_fp8);
}

int paged_prefill_impl(const void* q, int64_t q_stride_tok, int64_t q_stride_head, const void* key_pool,
                       const void* value_pool, int64_t pool_stride_slot, int64_t pool_stride_head,
                       const int64_t* slot_table, int64_t slot_table_stride, int max_context,
                       const int32_t* context_lens, const int32_t* query_start_loc, int batch, int max_query_len,
                       void* out, int64_t out_stride_tok, int64_t out_stride_head, int num_heads, int num_kv_heads,
                       int head_dim, float scale, int block_q, int block_kv, void* workspace, size_t workspace_bytes,
                       int dtype, int kv_dtype, float k_scale, float v_scale, int flags, void* stream) {
  clear_error();
  if (int rc = check_common(dtype, num_heads, num_kv_heads, head_dim, "li_paged_prefill")) return rc;
  if (int rc = check_kv(dtype, kv_dtype, k_scale, v_scale, "li_paged_prefill")) return rc;
  if (batch < 0 || max_query_len < 0 || max_context < 0) return fail(LI_EINVAL, "li_paged_prefill: negative extent");
  if (batch == 0 || max_query_len == 0) return LI_OK;
  if (!q || !key_pool || !value_pool || !slot_table || !context_lens || !query_start_loc || !out)
    return fail(LI_EINVAL, "li_paged_prefill: null pointer");

  AttnArgs a{};
  a.q = q;
  a.q_s0 = q_stride_tok;
  a.q_s1 = q_stride_head;
  a.kp = key_pool;
  a.vp = value_pool;
  a.p_s0 = pool_stride_slot;
  a.p_s1 = pool_stride_head;
  a.st = slot_table;
  a.st_s = slot_table_stride;
  a.ctx = context_lens;
  a.qsl = query_start_loc;
  a.out = out;
  a.o_s0 = out_stride_tok;
  a.o_s1 = out_stride_head;
  a.batch = batch;
  a.num_heads = num_heads;
  a.num_kv_heads = num_kv_heads;
  a.groups = num_heads / num_kv_heads;
  a.head_dim = head_dim;
  a.scale = scale;
  a.num_parts = 1;
  a.part_len = 0;
  a.block_kv = block_kv > 0 ? block_kv : kDefaultBlockKv;
  a.max_query_len = max_query_len;
  a.max_context = max_context;
  a.kv_fp8 = kv_dtype == LI_FP8_E4M3;
  a.k_scale = k_scale;
  a.v_scale = v_scale;

  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool mfma = !(flags & LI_FLAG_FORCE_GENERIC) && prefill_mfma_applies(a, dtype);
  if (a.kv_fp8 && !mfma)
    return fail(LI_EUNSUPPORTED,
                "li_paged_prefill: fp8 pools run on the MFMA kernels only (bf16 / fp16 queries, head_dim 128, "
                "16-byte aligned rows)");
  if (mfma) {
    // One-query sequences (decode rows beside chunks) would leave all but G
    // of a prefill unit's 256 rows idle and walk their whole context in one
    // work-group; the decode kernel serves them instead, its key axis cut
    // into partitions, and the prefill kernel skips them (unless the caller
    // says there are none: LI_FLAG_PREFILL_ONLY).
    const int waves = balanced_waves(device_cu_count());
    const size_t need = prefill_workspace(waves, a.groups, head_dim, batch, num_kv_heads, max_context);
    if (!workspace || workspace_bytes < need)
      return fail(LI_EWORKSPACE, "li_paged_prefill: workspace of %zu bytes given, %zu needed", workspace_bytes, need);
    const size_t entries = prefill_list_entries(batch, num_kv_heads, max_context);
    char* wp = static_cast<char*>(workspace) + balanced_workspace(waves, a.groups, head_dim, batch, num_kv_heads);
    a.work = reinterpret_cast<int4*>(wp);
    wp += align256(entries * sizeof(int4));
    a.queue = reinterpret_cast<int*>(wp);
    wp += align256(kPrefillQueueInts * sizeof(int));
    // A pass that would leave at least half the grid idle, over a 16-bit
    // pool (the ping-pong kernel), may be split into pieces.
    const int block_q = kPrefillUnitRows / a.groups;
    const int64_t units_max = (int64_t)batch * num_kv_heads * cdiv(max_query_len, block_q);
    // (A context under 2 x kSplitMinStages stages has no block to cut.)
    if (!a.kv_fp8 && prefill_split_room(batch, num_kv_heads) && units_max * 2 <= prefill_grid() &&
        max_context >= 2 * kSplitMinStages * 64) {
      a.split_ok = 1;
      a.split_target = prefill_grid();
      a.work_range = reinterpret_cast<int4*>(wp);
      wp += align256(entries * sizeof(int4));
      a.split_o = reinterpret_cast<float*>(wp);
      wp += align256((size_t)prefill_grid() * kPrefillUnitRows * head_dim * sizeof(float));
      a.split_ml = reinterpret_cast<float*>(wp);
      wp += align256((size_t)prefill_grid() * kPrefillUnitRows * 2 * sizeof(float));
      a.split_first = reinterpret_cast<int*>(wp);
    }
    if (flags & LI_FLAG_PREFILL_ONLY) return launch_prefill_mfma(a, dtype, s);
    AttnArgs d = a;
    d.block_q = 1;
    d.num_qblocks = 1;
    set_balanced(d, waves, workspace);
    if (max_query_len > 1) {
      // Chunks and rows in one launch: the rows' work-groups run the
      // per-head split, which fits the prefill kernels' registers.
      d.part_heads = 1;
      d.num_parts = waves;
      return launch_prefill_with_rows(a, d, dtype, s);
    }
    if (int rc = launch_decode_mfma(d, dtype, s)) return rc;
    if (max_query_len <= 1) return LI_OK;
    a.single_query_elsewhere = 1;
    return launch_prefill_mfma(a, dtype, s);
  }
  a.block_q = block_q > 0 ? block_q : 16;
  a.num_qblocks = cdiv(max_query_len, a.block_q);
  return launch_attend_generic(a, dtype, s);
}

extern "C" int li_paged_prefill(const void* q, int64_t q_stride_tok, int64_t q_stride_head, const void* key_pool,
                                const void* value_pool, int64_t pool_stride_slot, int64_t pool_stride_head,
                                const int64_t* slot_table, int64_t slot_table_stride, int max_context,
                                const int32_t* context_lens, const int32_t* query_start_loc, int batch,
                                int max_query_len, void* out, int64_t out_stride_tok, int64_t out_stride_head,
                                int num_heads, int num_kv_heads, int head_dim, float scale, int block_q,
                                int block_kv, void* workspace, size_t workspace_bytes, int dtype, int flags,
                                void* stream) {
  return paged_prefill_impl(q, q_stride_tok, q_stride_head, key_pool, value_pool, pool_stride_slot, pool_stride_head,
                            slot_table, slot_table_stride, max_context, context_lens, query_start_loc, batch,
                            max_query_len, out, out_stride_tok, out_stride_head, num_heads, num_kv_heads, head_dim,
                            scale, block_q, block_kv, workspace, workspace_bytes, dtype, dtype, 1.f, 1.f, flags,
                            stream);
}

extern "C" int li_paged_prefill_ex(const void* q, int64_t q_stride_tok, int64_t q_stride_head, const void* key_pool,
                                   const void* value_pool, int64_t pool_stride_slot, int64_t pool_stride_head,
                                   const int64_t* slot_table, int64_t slot_table_stride, int max_context,
                                   const int32_t* context_lens, const int32_t* query_start_loc, int batch,
                                   int max_query_len, void* out, int64_t out_stride_tok, int64_t out_stride_head,
                                   int num_heads, int num_kv_heads, int head_dim, float scale, int block_q,
                                   int block_kv, void* workspace, size_t workspace_bytes, int dtype, int kv_dtype,
                                   float k_scale, float v_scale, int flags, void* stream) {
  return paged_prefill_impl(q, q_stride_tok, q_stride_head, key_pool, value_pool, pool_stride_slot, pool_stride_head,
                            slot_table, slot_table_stride, max_context, context_lens, query_start_loc, batch,
                            max_query_len, out, out_stride_tok, out_stride_head, num_heads, num_kv_heads, head_dim,
                            scale, block_q, block_kv, workspace, workspace_bytes, dtype, kv_dtype, k_scale, v_scale,
                            flags, stream);
}
