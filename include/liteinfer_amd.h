/*
 * liteinfer_amd — C ABI of the MI355X (gfx950) paged-attention library.
 *
 * The library holds the three device kernels that liteinfer's
 * `attn_implementation="paged"` path runs, written in HIP for CDNA4:
 *
 *   li_kv_scatter      KV slot-write: this pass's K/V rows into pool slots.
 *   li_paged_decode    one query per sequence over its paged context.
 *   li_paged_prefill   packed / chunked queries, causal within the chunk,
 *                      over a cached prefix.
 *
 * Conventions shared by every entry point:
 *   - Pointers are device pointers; strides are in ELEMENTS, not bytes.
 *   - `stream` is a hipStream_t passed as void* (0 = the null stream).
 *   - Nothing is allocated: outputs and workspaces belong to the caller.
 *   - Nothing is read back to the host and nothing synchronises, so every
 *     call can be captured into a hipGraph. Grids are sized from the host
 *     integers passed in, never from device data.
 *   - Return 0 on success, a negative LI_E* code otherwise; the message of
 *     the last failure on the calling thread is li_last_error_string().
 *   - Pool layout (liteinfer/cache/block_pool.py:63): one layer's K (and V)
 *     store is [num_slots, num_kv_heads, head_dim] with the last axis
 *     contiguous; slot s of block b holding token t is b*block_size + t.
 *   - slot_table is [batch, max_context] int64, left-aligned; a row's columns
 *     at or past its context length are never read
 *     (liteinfer/cache/block_pool.py:135-148).
 */
#ifndef LITEINFER_AMD_H
#define LITEINFER_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types of q / pools / out. LI_FP8_E4M3 (OCP e4m3, one byte) is a
   pool type only: its rows hold K / k_scale and V / v_scale (see
   li_kv_scatter_fp8 and the _ex entry points). */
enum li_dtype { LI_F32 = 0, LI_F16 = 1, LI_BF16 = 2, LI_FP8_E4M3 = 3 };

/* Error codes. */
enum li_status {
  LI_OK = 0,
  LI_EINVAL = -1,       /* an argument is out of range or inconsistent */
  LI_EUNSUPPORTED = -2, /* a shape or layout this build does not serve */
  LI_ELAUNCH = -3,      /* the HIP runtime refused the launch */
  LI_EWORKSPACE = -4    /* the workspace passed is too small */
};

/* Flags for li_paged_decode / li_paged_prefill. */
enum li_flags {
  LI_FLAG_NONE = 0,
  LI_FLAG_FORCE_GENERIC = 1, /* run the general-shape kernel even where the
                               MFMA kernel applies (used by the parity tests) */
  LI_FLAG_EQUAL_SPLITS = 2,  /* li_paged_decode on the MFMA kernel: honour
                               num_splits >= 1 as the reference's equal-slice
                               partition count. Without it the MFMA kernel
                               takes num_splits as a scheduling hint only and
                               runs its balanced split (the same attention,
                               within fp32 rounding of the partial combine) */
  LI_FLAG_PREFILL_ONLY = 4   /* li_paged_prefill on the MFMA path: the prefill
                               kernel folds every sequence as query blocks,
                               one-query ones included, and the decode split
                               does not run (for passes with no one-query
                               sequences; correct either way) */
};

/* Message of the last failure on this thread ("" if none). */
const char* li_last_error_string(void);

/* Version of this ABI; bumped whenever a signature changes. */
int li_abi_version(void);

/* Digest (16 hex digits) of the csrc/ and include/ sources and the compile
 * flags the library was built from. No counterpart in the reference: it lets
 * a loader refuse a library built from other sources than the ones beside it. */
const char* li_build_id(void);

/*
 * KV slot-write. Replaces KVCache.scatter (liteinfer/cache/kv_cache.py:236-247)
 * together with _tokens_first (kv_cache.py:250-253):
 *     keys[slots.reshape(-1)]   = k.permute(0, 2, 1, 3).reshape(B*T, H, D)
 *     values[slots.reshape(-1)] = v.permute(0, 2, 1, 3).reshape(B*T, H, D)
 * k and v are [batch, num_kv_heads, tokens, head_dim] with arbitrary element
 * strides (k_strides / v_strides = {batch, head, token, dim}); slots holds
 * batch*tokens entries in batch-major token order. A bit-exact copy. A slot
 * outside [0, num_slots) is not written (torch's index_put_ would raise;
 * a kernel cannot): when bad_slots is not NULL, the device int32 it points
 * to is increased by the number of such tokens, for the caller to read when
 * it can synchronise (the Python wrapper raises IndexError then).
 */
int li_kv_scatter(const void* k, const void* v, const int64_t* k_strides,
                  const int64_t* v_strides, int64_t batch, int64_t tokens,
                  const int64_t* slots, void* key_pool, void* value_pool,
                  int64_t num_slots, int64_t pool_stride_slot,
                  int64_t pool_stride_head, int num_kv_heads, int head_dim,
                  int dtype, int32_t* bad_slots, void* stream);

/*
 * Quantising KV slot-write into an fp8 (LI_FP8_E4M3) pool: the reference's
 * planned quantised cache (liteinfer docs/roadmap.md, section 2.5:
 * "storage-level quant of K and V; dequant on read"), write side. Same
 * layout contract as li_kv_scatter, with each element stored as
 *     e4m3(clamp(float(x) * (1 / scale), -448, 448))
 * (the reciprocal in fp32, round to nearest even), k and v of src_dtype
 * (LI_F32 / LI_F16 / LI_BF16). The readers multiply back by the scale. No
 * counterpart in the reference's code: its cache is never quantised.
 * bad_slots as for li_kv_scatter.
 */
int li_kv_scatter_fp8(const void* k, const void* v, const int64_t* k_strides,
                      const int64_t* v_strides, int64_t batch, int64_t tokens,
                      const int64_t* slots, void* key_pool, void* value_pool,
                      int64_t num_slots, int64_t pool_stride_slot,
                      int64_t pool_stride_head, int num_kv_heads, int head_dim,
                      int src_dtype, float k_scale, float v_scale,
                      int32_t* bad_slots, void* stream);

/*
 * Fused rotary embedding + KV slot-write. Replaces, per layer, the
 * reference's _apply_rotary_pos_emb (liteinfer/models/llama.py:85-98, called
 * at :155-156) followed by payload.update -> KVCache.scatter (llama.py:160,
 * liteinfer/cache/kv_cache.py:236-253):
 *     q_out = q * cos + rotate_half(q) * sin
 *     key_pool[slots]   = tokens_first(k * cos + rotate_half(k) * sin)
 *     value_pool[slots] = tokens_first(v)
 * rotate_half(x) = cat(-x[..., D/2:], x[..., :D/2]). q / q_out are
 * [batch, num_heads, tokens, head_dim], k / v [batch, num_kv_heads, tokens,
 * head_dim], all with arbitrary element strides {batch, head, token, dim};
 * cos / sin are [batch, tokens, head_dim] with strides cs_strides (stride 0
 * broadcasts). slots holds batch*tokens entries in batch-major token order.
 * Every product and sum is rounded to `dtype` as the separate torch ops round
 * it, so q_out and the pool rows are bit-identical to the reference's
 * sequence. A slot outside [0, num_slots) is not written, and counted into
 * *bad_slots when bad_slots is not NULL (as for li_kv_scatter).
 */
int li_rope_kv_write(const void* q, const int64_t* q_strides, const void* k,
                     const int64_t* k_strides, const void* v,
                     const int64_t* v_strides, const void* cos, const void* sin,
                     const int64_t* cs_strides, int64_t batch, int64_t tokens,
                     const int64_t* slots, void* q_out,
                     const int64_t* q_out_strides, void* key_pool,
                     void* value_pool, int64_t num_slots,
                     int64_t pool_stride_slot, int64_t pool_stride_head,
                     int num_heads, int num_kv_heads, int head_dim, int dtype,
                     int32_t* bad_slots, void* stream);

/*
 * li_rope_kv_write into fp8 (LI_FP8_E4M3) pools: q_out as li_rope_kv_write
 * makes it; the rotated k (rounded to `dtype` exactly as li_rope_kv_write
 * rounds it) and v stored as li_kv_scatter_fp8 stores them, so the pool
 * bytes equal RoPE followed by li_kv_scatter_fp8. dtype is LI_BF16 or LI_F16;
 * rows 16-byte aligned with a contiguous last axis (otherwise
 * LI_EUNSUPPORTED). No counterpart in the reference's code (its planned
 * quantised cache, docs/roadmap.md 2.5).
 */
int li_rope_kv_write_fp8(const void* q, const int64_t* q_strides, const void* k,
                         const int64_t* k_strides, const void* v,
                         const int64_t* v_strides, const void* cos, const void* sin,
                         const int64_t* cs_strides, int64_t batch, int64_t tokens,
                         const int64_t* slots, void* q_out,
                         const int64_t* q_out_strides, void* key_pool,
                         void* value_pool, int64_t num_slots,
                         int64_t pool_stride_slot, int64_t pool_stride_head,
                         int num_heads, int num_kv_heads, int head_dim, int dtype,
                         float k_scale, float v_scale, int32_t* bad_slots,
                         void* stream);

/*
 * How many partitions each sequence's key loop is cut into for a decode step
 * of `batch` rows over a slot table `max_context` wide, on a device of
 * `num_cus` compute units (0 = ask the current device). The reference's
 * choose_num_splits (liteinfer/models/paged_kernels.py:645-693) with CUs for
 * SMs: 1 under four `block_kv` tiles (0 = 64), else
 * max(1, min(2 * num_cus / (batch * num_kv_heads), tiles, 32)). Returns the
 * count (>= 1) or a negative error. (li_paged_decode's num_splits = 0 uses
 * the library's own fixed-length partitions instead.)
 */
int li_choose_num_splits(int batch, int num_kv_heads, int max_context,
                         int num_cus, int block_kv);

/*
 * The launch plan of li_paged_decode's partitioned schedule: how many
 * partitions the grid holds, how long each one is (0 = each sequence's
 * context cut into num_partitions equal slices, the reference's split rule,
 * paged_kernels.py:495-498), and how many workspace bytes the call needs
 * under any schedule it may run (the MFMA kernel's balanced split included).
 * num_splits = 0 chooses (fixed-length partitions, so a long context is cut
 * more finely than a short one); num_splits >= 1 is the equal-slice split.
 * num_cus shapes the partition policy only: the workspace is always sized for
 * the current device, whose CU count sizes the MFMA kernel's balanced grid.
 */
int li_paged_decode_plan(int batch, int num_heads, int num_kv_heads,
                         int head_dim, int max_context, int num_splits,
                         int num_cus, int block_kv, int* num_partitions,
                         int* partition_len, size_t* workspace_bytes);

/*
 * Paged decode. Replaces paged_decode (liteinfer/models/paged_kernels.py:
 * 696-818) and its kernels _paged_decode_kernel, _paged_decode_split_kernel
 * and _combine_splits_kernel (:374-413, :462-629). One query per sequence:
 *   q   [batch, num_heads, head_dim]   strides (q_stride_seq, q_stride_head, 1)
 *   out [batch, num_heads, head_dim]   strides (out_stride_seq, out_stride_head, 1)
 * Query head h reads KV head h / (num_heads / num_kv_heads). Row i attends
 * to slot_table[i, 0:context_lens[i]]. The pools hold fewer than 2^31 slots
 * (the kernels stage slot indices as 32-bit integers). fp32 accumulation;
 * the output is rounded to `dtype` once. `workspace` must hold the bytes
 * li_paged_decode_plan reports (it may be NULL when that is 0). max_context
 * (the table's width, which bounds every context) also picks the schedule:
 * a narrow table (up to 1,024 columns, or 2,048 over at least 128 (sequence,
 * KV head) pairs, with pairs x width at most 2^19) runs one work-group per
 * (sequence, KV head) in a single launch; otherwise the balanced split and
 * its combine. Either gives the same attention within fp32 rounding.
 */
int li_paged_decode(const void* q, int64_t q_stride_seq, int64_t q_stride_head,
                    const void* key_pool, const void* value_pool,
                    int64_t pool_stride_slot, int64_t pool_stride_head,
                    const int64_t* slot_table, int64_t slot_table_stride,
                    int max_context, const int32_t* context_lens, void* out,
                    int64_t out_stride_seq, int64_t out_stride_head, int batch,
                    int num_heads, int num_kv_heads, int head_dim, float scale,
                    int num_splits, int block_kv, void* workspace,
                    size_t workspace_bytes, int dtype, int flags, void* stream);

/*
 * li_paged_decode over a pool of element type kv_dtype: `dtype` (then the
 * scales are ignored and this is li_paged_decode) or LI_FP8_E4M3, whose rows
 * hold K / k_scale and V / v_scale as written by li_kv_scatter_fp8. The
 * result is the attention over the dequantised rows; pool strides are in
 * pool elements (bytes for fp8). fp8 pools run on the MFMA kernel only
 * (bf16 / fp16 queries, head_dim 128; otherwise LI_EUNSUPPORTED). Carries the
 * reference's planned dequant-on-read (docs/roadmap.md, section 2.5); no
 * counterpart in the reference's code.
 */
int li_paged_decode_ex(const void* q, int64_t q_stride_seq, int64_t q_stride_head,
                       const void* key_pool, const void* value_pool,
                       int64_t pool_stride_slot, int64_t pool_stride_head,
                       const int64_t* slot_table, int64_t slot_table_stride,
                       int max_context, const int32_t* context_lens, void* out,
                       int64_t out_stride_seq, int64_t out_stride_head, int batch,
                       int num_heads, int num_kv_heads, int head_dim, float scale,
                       int num_splits, int block_kv, void* workspace,
                       size_t workspace_bytes, int dtype, int kv_dtype,
                       float k_scale, float v_scale, int flags, void* stream);

/*
 * One decode step of a layer: writes each sequence's newest K / V rows into
 * the pool, then attends as li_paged_decode_ex does. Replaces the decode
 * pair KVCache.scatter (liteinfer/cache/kv_cache.py:236-253, with the slots
 * of newest_slots at position context_lens[i] - 1, block_pool.py:151-170)
 * followed by paged_decode (liteinfer/models/paged_kernels.py:696-818).
 *   new_key, new_value [batch, num_kv_heads, head_dim], strides
 *                      (new_stride_seq, new_stride_head, 1), the query's
 *                      dtype; written bit-exact (an fp8 pool: quantised as
 *                      li_kv_scatter_fp8 does) to slot
 *                      slot_table[i, context_lens[i] - 1], which must be
 *                      part of no other sequence's context in this call;
 *                      rows with an empty context write nothing. Both NULL:
 *                      no write (a plain decode).
 *   num_slots, bad_slots  the pool's slot count; a newest slot outside it is
 *                      not written and is counted into *bad_slots (nullable).
 * On the balanced head-grouped and the short MFMA kernels over a 16-bit
 * pool the write happens inside the decode launch (the wave folding a
 * sequence's last key folds the new rows from registers and stores them, or
 * stores them before it reads that slot); elsewhere a write launch runs
 * first, with the same result. Everything else as
 * li_paged_decode_ex; `workspace` as li_paged_decode_plan reports.
 */
int li_paged_decode_write(const void* q, int64_t q_stride_seq,
                          int64_t q_stride_head, const void* key_pool,
                          const void* value_pool, int64_t pool_stride_slot,
                          int64_t pool_stride_head, const int64_t* slot_table,
                          int64_t slot_table_stride, int max_context,
                          const int32_t* context_lens, const void* new_key,
                          const void* new_value, int64_t new_stride_seq,
                          int64_t new_stride_head, int64_t num_slots,
                          int32_t* bad_slots, void* out, int64_t out_stride_seq,
                          int64_t out_stride_head, int batch, int num_heads,
                          int num_kv_heads, int head_dim, float scale,
                          int num_splits, int block_kv, void* workspace,
                          size_t workspace_bytes, int dtype, int kv_dtype,
                          float k_scale, float v_scale, int flags, void* stream);

/* Bytes of device scratch li_paged_decode_noalloc holds per GPU. */
#define LI_DECODE_NOALLOC_SCRATCH_BYTES (32u << 20)

/*
 * li_paged_decode for callers that cannot allocate device memory (code under
 * hipGraph capture, tight serving loops, harnesses that forbid hipMalloc).
 * No counterpart in the reference. Same arguments, meaning, kernels and
 * results as li_paged_decode, without the workspace: the partials live in a
 * device array of the library, LI_DECODE_NOALLOC_SCRATCH_BYTES on every GPU
 * it runs on (held until the process ends). A call whose plan
 * (li_paged_decode_plan) needs more returns LI_EWORKSPACE and launches
 * nothing. Nothing is allocated, not by the library nor by anything it
 * calls. Every call on one GPU shares that GPU's array, so calls that
 * overlap on one GPU (other streams, other threads) race; calls in one
 * stream order are safe. Nothing in the array has to start zeroed.
 */
int li_paged_decode_noalloc(const void* q, int64_t q_stride_seq,
                            int64_t q_stride_head, const void* key_pool,
                            const void* value_pool, int64_t pool_stride_slot,
                            int64_t pool_stride_head, const int64_t* slot_table,
                            int64_t slot_table_stride, int max_context,
                            const int32_t* context_lens, void* out,
                            int64_t out_stride_seq, int64_t out_stride_head,
                            int batch, int num_heads, int num_kv_heads,
                            int head_dim, float scale, int num_splits,
                            int block_kv, int dtype, int flags, void* stream);

/*
 * Workspace bytes li_paged_prefill needs for a pass of `batch` sequences over
 * a slot table `max_context` wide on a device of `num_cus` compute units
 * (0 = ask the current device): partials of its one-query sequences, which
 * the decode kernel's balanced split serves with a partitioned key axis (run
 * by the first work-groups of the prefill launch), the list that orders
 * the prefill kernel's query blocks longest first, and -- when batch x
 * num_kv_heads x 2 does not exceed the prefill grid (small batches) -- room
 * for the partial rows of a pass whose blocks are cut into pieces (one
 * 256-row fp32 slot per unit of the grid, ~34 MB at head_dim 128 on 256
 * CUs). No counterpart in
 * the reference, whose prefill kernel allocates nothing
 * (liteinfer/models/paged_kernels.py:867). The size is for the current
 * device (its CU count sizes the grid the launch runs); num_cus is accepted
 * for symmetry with li_paged_decode_plan and does not change it.
 */
int li_paged_prefill_plan(int batch, int num_heads, int num_kv_heads,
                          int head_dim, int max_context, int num_cus,
                          size_t* workspace_bytes);

/*
 * The number of work-groups of a packed pass's prefill launch (`grid`
 * work-groups) that fold its one-query rows first, as the launch computes it
 * on the device: row_keys = the rows' total context, chunk_pairs = the
 * chunks' visible causal (query, key) pairs, listed_blocks = the chunks'
 * query blocks, split_waves = the waves whose partial slots the workspace
 * holds (four row waves per work-group). Always within [0, min(grid,
 * split_waves / 4)]; 0 when there are no rows. No counterpart in the
 * reference, whose one-query rows run as prefill blocks; exported so that
 * planners and tests see the same count the kernels use. Returns a negative
 * code for a negative extent.
 */
int li_prefill_row_groups(unsigned long long row_keys,
                          unsigned long long chunk_pairs, int listed_blocks,
                          int grid, int split_waves, int num_kv_heads,
                          int num_heads, int head_dim, int kv_fp8);

/*
 * Packed / chunked prefill. Replaces paged_prefill
 * (liteinfer/models/paged_kernels.py:821-882) and _paged_prefill_kernel
 * (:416-459). Sequence i owns query rows [query_start_loc[i],
 * query_start_loc[i+1]) of
 *   q   [total_queries, num_heads, head_dim]  strides (q_stride_tok, q_stride_head, 1)
 *   out [total_queries, num_heads, head_dim]  strides (out_stride_tok, out_stride_head, 1)
 * and those queries are the last positions of its context of
 * context_lens[i] keys: query j of n sees keys 0 .. context_lens[i] - n + j.
 * max_query_len sizes the grid and must be >= every sequence's query count;
 * max_context is slot_table's width. block_q / block_kv are the
 * general-shape kernel's tile sizes (0 = default); the MFMA kernels use
 * their own. `workspace` must hold what li_paged_prefill_plan reports.
 */
int li_paged_prefill(const void* q, int64_t q_stride_tok, int64_t q_stride_head,
                     const void* key_pool, const void* value_pool,
                     int64_t pool_stride_slot, int64_t pool_stride_head,
                     const int64_t* slot_table, int64_t slot_table_stride,
                     int max_context, const int32_t* context_lens,
                     const int32_t* query_start_loc, int batch,
                     int max_query_len, void* out, int64_t out_stride_tok,
                     int64_t out_stride_head, int num_heads, int num_kv_heads,
                     int head_dim, float scale, int block_q, int block_kv,
                     void* workspace, size_t workspace_bytes, int dtype,
                     int flags, void* stream);

/*
 * li_paged_prefill over a pool of element type kv_dtype: `dtype` (then the
 * scales are ignored and this is li_paged_prefill) or LI_FP8_E4M3, as for
 * li_paged_decode_ex (its one-query sequences run on li_paged_decode_ex's
 * per-wave code, inside the prefill launch). fp8 pools run on the MFMA kernels only (bf16 / fp16 queries,
 * head_dim 128; otherwise LI_EUNSUPPORTED). No counterpart in the
 * reference's code (its planned quantised cache, docs/roadmap.md 2.5).
 */
int li_paged_prefill_ex(const void* q, int64_t q_stride_tok, int64_t q_stride_head,
                        const void* key_pool, const void* value_pool,
                        int64_t pool_stride_slot, int64_t pool_stride_head,
                        const int64_t* slot_table, int64_t slot_table_stride,
                        int max_context, const int32_t* context_lens,
                        const int32_t* query_start_loc, int batch, int max_query_len,
                        void* out, int64_t out_stride_tok, int64_t out_stride_head,
                        int num_heads, int num_kv_heads, int head_dim, float scale,
                        int block_q, int block_kv, void* workspace,
                        size_t workspace_bytes, int dtype, int kv_dtype,
                        float k_scale, float v_scale, int flags, void* stream);

/*
 * The minimal engine's per-layer elementwise work (the model around the
 * paged path; no counterpart in the reference's paged path, which leaves it
 * to torch ops). Rows of `hidden` (a multiple of 8, at most 8192) bf16 / fp16
 * elements, 16-byte aligned, last axis contiguous; strides in elements.
 *
 * li_add_rms_norm: when `delta` is given, h <- h + delta (rounded to the
 * dtype, in place); then out <- weight * dtype(h * rsqrt(mean(h^2) + eps)),
 * the product rounded to the dtype: the residual add and RMSNorm of
 * liteinfer/models/llama.py:34-48 (fp32 statistics) in one launch.
 * li_silu_mul: out[r, :] <- silu(gate) * up with gate = gate_up[r, :ffn],
 * up = gate_up[r, ffn:2 ffn] (the SiLU gate of llama.py:101-116), each of the
 * two products rounded to the dtype as torch rounds them.
 */
int li_add_rms_norm(void* h, const void* delta, const void* weight, void* out,
                    int64_t rows, int hidden, int64_t h_stride,
                    int64_t delta_stride, int64_t out_stride, float eps,
                    int dtype, void* stream);
int li_silu_mul(const void* gate_up, void* out, int64_t rows, int ffn,
                int64_t gate_up_stride, int64_t out_stride, int dtype,
                void* stream);

#ifdef __cplusplus
}
#endif

#endif /* LITEINFER_AMD_H */
