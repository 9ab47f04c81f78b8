// Fused rotary embedding + KV slot-write: one launch per layer takes the
// q / k / v projections of this pass, rotates q and k, returns the rotated q
// and writes the rotated k and the untouched v into their pool slots.
//
// Counterpart of the reference's per-layer sequence
//   q, k = _apply_rotary_pos_emb(q, k, cos, sin)      (liteinfer/models/llama.py:85-98, :155-156)
//   payload.update(k, v, layer) -> KVCache.scatter    (llama.py:160, cache/kv_cache.py:236-253)
// which runs as separate elementwise kernels (two products, a negation and
// concatenation for rotate_half, a sum, for q and for k), a permute copy
// (_tokens_first) and two index_put_ launches.
//
// Arithmetic follows the reference's op order exactly: every torch op rounds
// its result to the tensor dtype, so for element i < D/2 (x1 = x[:D/2],
// x2 = x[D/2:])
//   out[i]       = R( R(x1[i] * cos[i])       + R(-x2[i] * sin[i]) )
//   out[i + D/2] = R( R(x2[i] * cos[i + D/2]) + R( x1[i] * sin[i + D/2]) )
// with R the round-to-nearest-even to bf16 / fp16 (identity for fp32). The
// products and the sum are formed in fp32 with FP contraction switched off,
// so no product and sum become one FMA (hipcc contracts by default); the product
// of two bf16 / fp16 values and the sum of two are exact or correctly
// rounded in fp32, so the result is bit-identical to the torch sequence.
//
// Work unit: one (token, head, chunk pair): 16 bytes of the first half of a
// head row and the matching 16 bytes of the second half. Units of a token run
// over the q heads, then the k heads (rotated, written to the key pool), then
// the v heads (copied to the value pool). Tokens are batch-major (the order of
// the slot list, _tokens_first, kv_cache.py:250-253).
#include "li_common.h"

#include <cmath>

namespace {

struct RopeArgs {
  const char* q;
  const char* k;
  const char* v;
  const char* cos;
  const char* sin;
  char* qo;
  char* kp;
  char* vp;
  int64_t qs[4], ks[4], vs[4], os[4];  // element strides: batch, head, token, dim
  int64_t cs[3];                        // cos / sin element strides: batch, token, dim
  int64_t tokens;                       // T
  int64_t n;                            // B * T
  const int64_t* slots;
  int64_t num_slots;
  int64_t ps_slot, ps_head;
  int num_heads, num_kv_heads, head_dim;
  float inv_k, inv_v;  // fp8 pools: 1 / k_scale, 1 / v_scale
  int* bad;            // nullable: counts tokens whose slot is out of range
};

// Eight values, rounded to E (as stored by the unfused path), to eight e4m3
// bytes: e4m3(clamp(float(x) * inv, +-448)), as li_kv_scatter_fp8 stores them.
template <typename VecE>
__device__ __forceinline__ uint2 quant8(VecE x, float inv) {
  float f[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) f[e] = li_clamp_e4m3(li_to_float(x[e]) * inv);
  uint2 out;
  out.x = __builtin_amdgcn_cvt_pk_fp8_f32(f[0], f[1], 0u, false);
  out.x = __builtin_amdgcn_cvt_pk_fp8_f32(f[2], f[3], out.x, true);
  out.y = __builtin_amdgcn_cvt_pk_fp8_f32(f[4], f[5], 0u, false);
  out.y = __builtin_amdgcn_cvt_pk_fp8_f32(f[6], f[7], out.y, true);
  return out;
}

template <typename E>
struct Lanes;
template <>
struct Lanes<float> {
  static constexpr int kPer16 = 4;
};
template <>
struct Lanes<li_bf16> {
  static constexpr int kPer16 = 8;
};
template <>
struct Lanes<li_f16> {
  static constexpr int kPer16 = 8;
};

template <typename E>
__device__ __forceinline__ float round_to(float x) {
  return li_to_float(li_from_float<E>(x));
}

// One rotated pair: (lo, hi) -> (lo * c_lo - hi * s_lo, hi * c_hi + lo * s_hi),
// each product and the sum rounded as the torch ops round them.
template <typename E>
__device__ __forceinline__ void rotate(E lo, E hi, E c_lo, E s_lo, E c_hi, E s_hi, E& out_lo, E& out_hi) {
#pragma clang fp contract(off)  // a product feeding a sum must not become one FMA
  const float xl = li_to_float(lo), xh = li_to_float(hi);
  const float a = round_to<E>(xl * li_to_float(c_lo));
  // R(-x2 * s) = -R(x2 * s): rounding to nearest even is symmetric.
  const float b = round_to<E>(xh * li_to_float(s_lo));
  const float c = round_to<E>(xh * li_to_float(c_hi));
  const float d = round_to<E>(xl * li_to_float(s_hi));
  out_lo = li_from_float<E>(a - b);
  out_hi = li_from_float<E>(c + d);
}

// Vector path: every row 16-byte aligned, head_dim a multiple of 2 * (16 /
// sizeof(E)), unit dim strides.
// I: the index type of the work-item arithmetic (32-bit whenever the total
// fits, which spares the 64-bit division sequences).
// F8: the pools are fp8 (e4m3): the rotated k (rounded to E, as the torch ops
// round it) and v are quantised on the way in, 8 bytes per half chunk.
template <typename E, typename I, bool F8>
__global__ __launch_bounds__(256) void rope_kv_write_vec(RopeArgs a) {
  constexpr int kE = Lanes<E>::kPer16;
  typedef E vecE __attribute__((ext_vector_type(kE)));
  const int half = a.head_dim / 2;
  const int pairs = half / kE;  // chunk pairs per head row
  const int heads = a.num_heads + 2 * a.num_kv_heads;
  const I per_token = (I)heads * pairs;
  const I total = (I)a.n * per_token;
  const I tokens = (I)a.tokens;
  for (I w = (I)blockIdx.x * blockDim.x + threadIdx.x; w < total; w += (I)gridDim.x * blockDim.x) {
    const I i = w / per_token;
    const int rem = (int)(w - i * per_token);
    const int hh = rem / pairs;
    const int d0 = (rem - hh * pairs) * kE;
    const int64_t b = i / tokens, t = i - (I)b * tokens;
    if (hh >= a.num_heads + a.num_kv_heads) {  // v: copy both halves
      const int h = hh - a.num_heads - a.num_kv_heads;
      const int64_t slot = a.slots[i];
      if (slot < 0 || slot >= a.num_slots) continue;
      const E* src = reinterpret_cast<const E*>(a.v) + b * a.vs[0] + h * a.vs[1] + t * a.vs[2] + d0;
      if constexpr (F8) {
        uint8_t* dst = reinterpret_cast<uint8_t*>(a.vp) + slot * a.ps_slot + h * a.ps_head + d0;
        *reinterpret_cast<uint2*>(dst) = quant8(*reinterpret_cast<const vecE*>(src), a.inv_v);
        *reinterpret_cast<uint2*>(dst + half) = quant8(*reinterpret_cast<const vecE*>(src + half), a.inv_v);
      } else {
        E* dst = reinterpret_cast<E*>(a.vp) + slot * a.ps_slot + h * a.ps_head + d0;
        const u32x4_t lo = *reinterpret_cast<const u32x4_t*>(src);
        const u32x4_t hi = *reinterpret_cast<const u32x4_t*>(src + half);
        *reinterpret_cast<u32x4_t*>(dst) = lo;
        *reinterpret_cast<u32x4_t*>(dst + half) = hi;
      }
      continue;
    }
    const bool is_q = hh < a.num_heads;
    const int h = is_q ? hh : hh - a.num_heads;
    const E* src = is_q ? reinterpret_cast<const E*>(a.q) + b * a.qs[0] + h * a.qs[1] + t * a.qs[2] + d0
                        : reinterpret_cast<const E*>(a.k) + b * a.ks[0] + h * a.ks[1] + t * a.ks[2] + d0;
    E* dst = nullptr;
    uint8_t* dst8 = nullptr;
    if (is_q) {
      dst = reinterpret_cast<E*>(a.qo) + b * a.os[0] + h * a.os[1] + t * a.os[2] + d0;
    } else {
      const int64_t slot = a.slots[i];
      if (slot < 0 || slot >= a.num_slots) {
        if (h == 0 && d0 == 0 && a.bad) atomicAdd(a.bad, 1);
        continue;
      }
      if constexpr (F8) dst8 = reinterpret_cast<uint8_t*>(a.kp) + slot * a.ps_slot + h * a.ps_head + d0;
      else dst = reinterpret_cast<E*>(a.kp) + slot * a.ps_slot + h * a.ps_head + d0;
    }
    const int64_t co = b * a.cs[0] + t * a.cs[1] + d0;
    const vecE xl = *reinterpret_cast<const vecE*>(src);
    const vecE xh = *reinterpret_cast<const vecE*>(src + half);
    const vecE cl = *reinterpret_cast<const vecE*>(reinterpret_cast<const E*>(a.cos) + co);
    const vecE ch = *reinterpret_cast<const vecE*>(reinterpret_cast<const E*>(a.cos) + co + half);
    const vecE sl = *reinterpret_cast<const vecE*>(reinterpret_cast<const E*>(a.sin) + co);
    const vecE sh = *reinterpret_cast<const vecE*>(reinterpret_cast<const E*>(a.sin) + co + half);
    vecE ol, oh;
#pragma unroll
    for (int e = 0; e < kE; ++e) {
      E lo, hi;
      rotate<E>(xl[e], xh[e], cl[e], sl[e], ch[e], sh[e], lo, hi);
      ol[e] = lo;
      oh[e] = hi;
    }
    if (F8 && !is_q) {
      *reinterpret_cast<uint2*>(dst8) = quant8(ol, a.inv_k);
      *reinterpret_cast<uint2*>(dst8 + half) = quant8(oh, a.inv_k);
    } else {
      *reinterpret_cast<vecE*>(dst) = ol;
      *reinterpret_cast<vecE*>(dst + half) = oh;
    }
  }
}

// Any strides: one element pair per work item.
template <typename E>
__global__ __launch_bounds__(256) void rope_kv_write_elem(RopeArgs a) {
  const int half = a.head_dim / 2;
  const int heads = a.num_heads + 2 * a.num_kv_heads;
  const int64_t per_token = (int64_t)heads * half;
  const int64_t total = a.n * per_token;
  for (int64_t w = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; w < total; w += (int64_t)gridDim.x * blockDim.x) {
    const int64_t i = w / per_token;
    const int rem = (int)(w - i * per_token);
    const int hh = rem / half;
    const int d = rem - hh * half;
    const int64_t b = i / a.tokens, t = i - b * a.tokens;
    if (hh >= a.num_heads + a.num_kv_heads) {
      const int h = hh - a.num_heads - a.num_kv_heads;
      const int64_t slot = a.slots[i];
      if (slot < 0 || slot >= a.num_slots) continue;
      const E* src = reinterpret_cast<const E*>(a.v) + b * a.vs[0] + h * a.vs[1] + t * a.vs[2];
      E* dst = reinterpret_cast<E*>(a.vp) + slot * a.ps_slot + h * a.ps_head;
      dst[d] = src[d * a.vs[3]];
      dst[d + half] = src[(d + half) * a.vs[3]];
      continue;
    }
    const bool is_q = hh < a.num_heads;
    const int h = is_q ? hh : hh - a.num_heads;
    const E* src;
    int64_t sd;
    E* dst;
    int64_t od;
    if (is_q) {
      src = reinterpret_cast<const E*>(a.q) + b * a.qs[0] + h * a.qs[1] + t * a.qs[2];
      sd = a.qs[3];
      dst = reinterpret_cast<E*>(a.qo) + b * a.os[0] + h * a.os[1] + t * a.os[2];
      od = a.os[3];
    } else {
      const int64_t slot = a.slots[i];
      if (slot < 0 || slot >= a.num_slots) {
        if (h == 0 && d == 0 && a.bad) atomicAdd(a.bad, 1);
        continue;
      }
      src = reinterpret_cast<const E*>(a.k) + b * a.ks[0] + h * a.ks[1] + t * a.ks[2];
      sd = a.ks[3];
      dst = reinterpret_cast<E*>(a.kp) + slot * a.ps_slot + h * a.ps_head;
      od = 1;
    }
    const E* cs = reinterpret_cast<const E*>(a.cos) + b * a.cs[0] + t * a.cs[1];
    const E* sn = reinterpret_cast<const E*>(a.sin) + b * a.cs[0] + t * a.cs[1];
    E lo, hi;
    rotate<E>(src[d * sd], src[(d + half) * sd], cs[d * a.cs[2]], sn[d * a.cs[2]], cs[(d + half) * a.cs[2]],
              sn[(d + half) * a.cs[2]], lo, hi);
    dst[d * od] = lo;
    dst[(d + half) * od] = hi;
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// pool_esize: bytes per pool element (1 for an fp8 pool, whose half-rows of
// 8 elements take 8-byte stores).
bool vec_ok(const RopeArgs& a, int esize, int pool_esize) {
  const int per16 = 16 / esize;
  if (a.head_dim % (2 * per16) != 0) return false;
  if (a.qs[3] != 1 || a.ks[3] != 1 || a.vs[3] != 1 || a.os[3] != 1 || a.cs[2] != 1) return false;
  const char* ptrs[] = {a.q, a.k, a.v, a.cos, a.sin, a.qo, a.kp, a.vp};
  for (const char* p : ptrs)
    if (!aligned16(p)) return false;
  const int64_t strides[] = {a.qs[0], a.qs[1], a.qs[2], a.ks[0], a.ks[1], a.ks[2], a.vs[0], a.vs[1], a.vs[2],
                             a.os[0], a.os[1], a.os[2], a.cs[0], a.cs[1]};
  for (int64_t s : strides)
    if ((s * esize) % 16 != 0) return false;
  const int pool_align = pool_esize == esize ? 16 : 8;
  return (a.ps_slot * pool_esize) % pool_align == 0 && (a.ps_head * pool_esize) % pool_align == 0 &&
         (a.head_dim / 2 * pool_esize) % pool_align == 0;
}

}  // namespace

namespace {

int rope_impl(const void* q, const int64_t* q_strides, const void* k, const int64_t* k_strides, const void* v,
              const int64_t* v_strides, const void* cos, const void* sin, const int64_t* cs_strides, int64_t batch,
              int64_t tokens, const int64_t* slots, void* q_out, const int64_t* q_out_strides, void* key_pool,
              void* value_pool, int64_t num_slots, int64_t pool_stride_slot, int64_t pool_stride_head, int num_heads,
              int num_kv_heads, int head_dim, int dtype, bool fp8, float k_scale, float v_scale, int32_t* bad_slots,
              void* stream) {
  li::clear_error();
  const int esize = li::dtype_size(dtype);
  if (esize == 0) return li::fail(LI_EINVAL, "li_rope_kv_write: unknown dtype %d", dtype);
  if (dtype == LI_FP8_E4M3)
    return li::fail(LI_EUNSUPPORTED, "li_rope_kv_write: fp8 pools are written by li_rope_kv_write_fp8 (quantising)");
  if (fp8 && dtype == LI_F32)
    return li::fail(LI_EUNSUPPORTED, "li_rope_kv_write_fp8: bf16 / fp16 projections only");
  if (fp8 && (!(k_scale > 0.f) || !(v_scale > 0.f) || !std::isfinite(k_scale) || !std::isfinite(v_scale)))
    return li::fail(LI_EINVAL, "li_rope_kv_write_fp8: scales must be finite and > 0 (k_scale=%g, v_scale=%g)",
                    k_scale, v_scale);
  if (batch < 0 || tokens < 0 || num_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0 || num_slots < 0)
    return li::fail(LI_EINVAL, "li_rope_kv_write: negative or empty extent");
  if (head_dim % 2 != 0) return li::fail(LI_EINVAL, "li_rope_kv_write: head_dim %d is odd", head_dim);
  if (!q_strides || !k_strides || !v_strides || !cs_strides || !q_out_strides)
    return li::fail(LI_EINVAL, "li_rope_kv_write: strides must not be null");
  const int64_t n = batch * tokens;
  if (n == 0) return LI_OK;
  if (!q || !k || !v || !cos || !sin || !slots || !q_out || !key_pool || !value_pool)
    return li::fail(LI_EINVAL, "li_rope_kv_write: null pointer");
  if (pool_stride_head < head_dim || pool_stride_slot < (int64_t)num_kv_heads * head_dim)
    return li::fail(LI_EINVAL, "li_rope_kv_write: pool strides (%lld, %lld) overlap rows of %d x %d",
                    (long long)pool_stride_slot, (long long)pool_stride_head, num_kv_heads, head_dim);

  RopeArgs a;
  a.q = static_cast<const char*>(q);
  a.k = static_cast<const char*>(k);
  a.v = static_cast<const char*>(v);
  a.cos = static_cast<const char*>(cos);
  a.sin = static_cast<const char*>(sin);
  a.qo = static_cast<char*>(q_out);
  a.kp = static_cast<char*>(key_pool);
  a.vp = static_cast<char*>(value_pool);
  for (int j = 0; j < 4; ++j) {
    a.qs[j] = q_strides[j];
    a.ks[j] = k_strides[j];
    a.vs[j] = v_strides[j];
    a.os[j] = q_out_strides[j];
  }
  for (int j = 0; j < 3; ++j) a.cs[j] = cs_strides[j];
  a.tokens = tokens;
  a.n = n;
  a.slots = slots;
  a.num_slots = num_slots;
  a.ps_slot = pool_stride_slot;
  a.ps_head = pool_stride_head;
  a.num_heads = num_heads;
  a.num_kv_heads = num_kv_heads;
  a.head_dim = head_dim;
  a.inv_k = fp8 ? 1.f / k_scale : 1.f;
  a.inv_v = fp8 ? 1.f / v_scale : 1.f;
  a.bad = bad_slots;

  hipStream_t s = static_cast<hipStream_t>(stream);
  const int threads = 256;
  const int heads = num_heads + 2 * num_kv_heads;
  if (fp8) {
    // fp8 pool rows take 8-byte stores: byte strides multiples of 8.
    if (!vec_ok(a, esize, /*pool_esize=*/1))
      return li::fail(LI_EUNSUPPORTED, "li_rope_kv_write_fp8: rows must be 16-byte aligned with a contiguous last axis");
    const int64_t work = n * heads * (head_dim / 2 / 8);
    const int64_t blocks = std::min<int64_t>(li::cdiv64(work, threads), 65536);
    const dim3 grid((unsigned)blocks), block(threads);
    if (work < (int64_t)1 << 31) {
      if (dtype == LI_BF16) hipLaunchKernelGGL((rope_kv_write_vec<li_bf16, uint32_t, true>), grid, block, 0, s, a);
      else hipLaunchKernelGGL((rope_kv_write_vec<li_f16, uint32_t, true>), grid, block, 0, s, a);
    } else {
      if (dtype == LI_BF16) hipLaunchKernelGGL((rope_kv_write_vec<li_bf16, int64_t, true>), grid, block, 0, s, a);
      else hipLaunchKernelGGL((rope_kv_write_vec<li_f16, int64_t, true>), grid, block, 0, s, a);
    }
    return li::check_launch("li_rope_kv_write_fp8");
  }
  if (vec_ok(a, esize, esize)) {
    const int64_t work = n * heads * (head_dim / 2 / (16 / esize));
    const int64_t blocks = std::min<int64_t>(li::cdiv64(work, threads), 65536);
    const dim3 grid((unsigned)blocks), block(threads);
    if (work < (int64_t)1 << 31) {
      if (dtype == LI_F32) hipLaunchKernelGGL((rope_kv_write_vec<float, uint32_t, false>), grid, block, 0, s, a);
      else if (dtype == LI_BF16) hipLaunchKernelGGL((rope_kv_write_vec<li_bf16, uint32_t, false>), grid, block, 0, s, a);
      else hipLaunchKernelGGL((rope_kv_write_vec<li_f16, uint32_t, false>), grid, block, 0, s, a);
    } else {
      if (dtype == LI_F32) hipLaunchKernelGGL((rope_kv_write_vec<float, int64_t, false>), grid, block, 0, s, a);
      else if (dtype == LI_BF16) hipLaunchKernelGGL((rope_kv_write_vec<li_bf16, int64_t, false>), grid, block, 0, s, a);
      else hipLaunchKernelGGL((rope_kv_write_vec<li_f16, int64_t, false>), grid, block, 0, s, a);
    }
  } else {
    const int64_t work = n * heads * (head_dim / 2);
    const int64_t blocks = std::min<int64_t>(li::cdiv64(work, threads), 65536);
    if (dtype == LI_F32) hipLaunchKernelGGL(rope_kv_write_elem<float>, dim3((unsigned)blocks), dim3(threads), 0, s, a);
    else if (dtype == LI_BF16) hipLaunchKernelGGL(rope_kv_write_elem<li_bf16>, dim3((unsigned)blocks), dim3(threads), 0, s, a);
    else hipLaunchKernelGGL(rope_kv_write_elem<li_f16>, dim3((unsigned)blocks), dim3(threads), 0, s, a);
  }
  return li::check_launch("li_rope_kv_write");
}

}  // namespace

extern "C" int li_rope_kv_write(const void* q, const int64_t* q_strides, const void* k, const int64_t* k_strides,
                                const void* v, const int64_t* v_strides, const void* cos, const void* sin,
                                const int64_t* cs_strides, int64_t batch, int64_t tokens, const int64_t* slots,
                                void* q_out, const int64_t* q_out_strides, void* key_pool, void* value_pool,
                                int64_t num_slots, int64_t pool_stride_slot, int64_t pool_stride_head, int num_heads,
                                int num_kv_heads, int head_dim, int dtype, int32_t* bad_slots, void* stream) {
  return rope_impl(q, q_strides, k, k_strides, v, v_strides, cos, sin, cs_strides, batch, tokens, slots, q_out,
                   q_out_strides, key_pool, value_pool, num_slots, pool_stride_slot, pool_stride_head, num_heads,
                   num_kv_heads, head_dim, dtype, false, 1.f, 1.f, bad_slots, stream);
}

extern "C" int li_rope_kv_write_fp8(const void* q, const int64_t* q_strides, const void* k,
                                    const int64_t* k_strides, const void* v, const int64_t* v_strides,
                                    const void* cos, const void* sin, const int64_t* cs_strides, int64_t batch,
                                    int64_t tokens, const int64_t* slots, void* q_out, const int64_t* q_out_strides,
                                    void* key_pool, void* value_pool, int64_t num_slots, int64_t pool_stride_slot,
                                    int64_t pool_stride_head, int num_heads, int num_kv_heads, int head_dim, int dtype,
                                    float k_scale, float v_scale, int32_t* bad_slots, void* stream) {
  return rope_impl(q, q_strides, k, k_strides, v, v_strides, cos, sin, cs_strides, batch, tokens, slots, q_out,
                   q_out_strides, key_pool, value_pool, num_slots, pool_stride_slot, pool_stride_head, num_heads,
                   num_kv_heads, head_dim, dtype, true, k_scale, v_scale, bad_slots, stream);
}
