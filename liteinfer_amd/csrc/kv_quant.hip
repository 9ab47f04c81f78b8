// Quantising KV slot-write: this pass's K and V rows into an fp8 (OCP e4m3)
// pool.
//
// The reference plans a quantised cache as "storage-level quant of K and V;
// dequant on read" (liteinfer docs/roadmap.md, section 2.5); the write side
// is KVCache.scatter (liteinfer/cache/kv_cache.py:236-253) with each element
// rounded on its way into the pool:
//     key_pool[slots[i], h, d] = e4m3(clamp(float(k[b, h, t, d]) * inv_k, +-448))
// with inv_k = 1 / k_scale in fp32, round to nearest even (e4m3 has no
// infinity; the clamp saturates at its largest finite value), and the same
// for V. Token i of the batch-major order is (b, t) = (i / T, i % T), as in
// li_kv_scatter.
//
// One work item converts 16 elements of K and of V into one 16-byte store
// each (rows with a contiguous last axis and 16-byte alignment); any other
// layout runs one element per work item.
#include "li_common.h"

#include <cmath>

namespace {

struct QuantArgs {
  const char* k;
  const char* v;
  int64_t ks[4];  // element strides of k: batch, head, token, dim
  int64_t vs[4];
  int64_t tokens;  // T
  int64_t n;       // B * T
  const int64_t* slots;
  uint8_t* kp;
  uint8_t* vp;
  int64_t num_slots;
  int64_t ps_slot;  // strides of the pools, in bytes (= elements)
  int64_t ps_head;
  int heads;
  int head_dim;
  float inv_k, inv_v;
  int* bad;  // nullable: counts tokens whose slot is out of range
};

template <typename E>
__device__ __forceinline__ float to_f32(E x) {
  return (float)x;
}

// Two values to e4m3 in the low (HIGH = false) or high 16 bits of `into`.
template <bool HIGH>
__device__ __forceinline__ uint32_t pack_fp8(float a, float b, uint32_t into) {
  a = li_clamp_e4m3(a);
  b = li_clamp_e4m3(b);
  return __builtin_amdgcn_cvt_pk_fp8_f32(a, b, into, HIGH);
}

// 16 elements of type E at `src` to 16 e4m3 bytes.
template <typename E>
__device__ __forceinline__ u32x4_t quant16(const E* src, float inv) {
  float x[16];
  if constexpr (sizeof(E) == 2) {
    const u32x4_t w0 = *reinterpret_cast<const u32x4_t*>(src);
    const u32x4_t w1 = *reinterpret_cast<const u32x4_t*>(src + 8);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[2 * i] = to_f32(__builtin_bit_cast(E, (uint16_t)(w0[i] & 0xffffu)));
      x[2 * i + 1] = to_f32(__builtin_bit_cast(E, (uint16_t)(w0[i] >> 16)));
      x[8 + 2 * i] = to_f32(__builtin_bit_cast(E, (uint16_t)(w1[i] & 0xffffu)));
      x[8 + 2 * i + 1] = to_f32(__builtin_bit_cast(E, (uint16_t)(w1[i] >> 16)));
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const floatx4_t w = *reinterpret_cast<const floatx4_t*>(src + 4 * i);
#pragma unroll
      for (int r = 0; r < 4; ++r) x[4 * i + r] = w[r];
    }
  }
  u32x4_t out;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t w = pack_fp8<false>(x[4 * i] * inv, x[4 * i + 1] * inv, 0u);
    out[i] = pack_fp8<true>(x[4 * i + 2] * inv, x[4 * i + 3] * inv, w);
  }
  return out;
}

template <typename E>
__global__ __launch_bounds__(256) void kv_quant_vec16(QuantArgs a) {
  const int units = a.head_dim / 16;
  const int64_t per_token = (int64_t)a.heads * units;
  const int64_t total = a.n * per_token;
  for (int64_t w = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; w < total;
       w += (int64_t)gridDim.x * blockDim.x) {
    const int64_t i = w / per_token;
    const int rem = (int)(w - i * per_token);
    const int h = rem / units;
    const int u = rem - h * units;
    const int64_t slot = a.slots[i];
    if (slot < 0 || slot >= a.num_slots) {
      if (rem == 0 && a.bad) atomicAdd(a.bad, 1);
      continue;
    }
    const int64_t b = i / a.tokens, t = i - b * a.tokens;
    const int64_t d = (int64_t)u * 16;
    const E* ksrc = reinterpret_cast<const E*>(a.k) + b * a.ks[0] + h * a.ks[1] + t * a.ks[2] + d;
    const E* vsrc = reinterpret_cast<const E*>(a.v) + b * a.vs[0] + h * a.vs[1] + t * a.vs[2] + d;
    const int64_t po = slot * a.ps_slot + h * a.ps_head + d;
    *reinterpret_cast<u32x4_t*>(a.kp + po) = quant16<E>(ksrc, a.inv_k);
    *reinterpret_cast<u32x4_t*>(a.vp + po) = quant16<E>(vsrc, a.inv_v);
  }
}

// Any strides: one element per work item.
template <typename E>
__global__ __launch_bounds__(256) void kv_quant_elem(QuantArgs a) {
  const int64_t per_token = (int64_t)a.heads * a.head_dim;
  const int64_t total = a.n * per_token;
  for (int64_t w = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; w < total;
       w += (int64_t)gridDim.x * blockDim.x) {
    const int64_t i = w / per_token;
    const int rem = (int)(w - i * per_token);
    const int h = rem / a.head_dim;
    const int d = rem - h * a.head_dim;
    const int64_t slot = a.slots[i];
    if (slot < 0 || slot >= a.num_slots) {
      if (rem == 0 && a.bad) atomicAdd(a.bad, 1);
      continue;
    }
    const int64_t b = i / a.tokens, t = i - b * a.tokens;
    const float kx = to_f32(reinterpret_cast<const E*>(a.k)[b * a.ks[0] + h * a.ks[1] + t * a.ks[2] + d * a.ks[3]]);
    const float vx = to_f32(reinterpret_cast<const E*>(a.v)[b * a.vs[0] + h * a.vs[1] + t * a.vs[2] + d * a.vs[3]]);
    const int64_t po = slot * a.ps_slot + h * a.ps_head + d;
    a.kp[po] = (uint8_t)(pack_fp8<false>(kx * a.inv_k, 0.f, 0u) & 0xffu);
    a.vp[po] = (uint8_t)(pack_fp8<false>(vx * a.inv_v, 0.f, 0u) & 0xffu);
  }
}

bool all_aligned(const QuantArgs& a, int esize) {
  if (!li::aligned16(a.k) || !li::aligned16(a.v) || !li::aligned16(a.kp) || !li::aligned16(a.vp)) return false;
  if (a.ks[3] != 1 || a.vs[3] != 1 || a.head_dim % 16 != 0) return false;
  for (int j = 0; j < 3; ++j) {
    if ((a.ks[j] * esize) % 16 != 0 || (a.vs[j] * esize) % 16 != 0) return false;
  }
  return a.ps_slot % 16 == 0 && a.ps_head % 16 == 0;
}

template <typename E>
void launch(const QuantArgs& a, bool vec, hipStream_t s) {
  const int threads = 256;
  const int64_t work = vec ? a.n * a.heads * (a.head_dim / 16) : a.n * a.heads * a.head_dim;
  const int64_t blocks = std::min<int64_t>(li::cdiv64(work, threads), 65536);
  if (vec) hipLaunchKernelGGL(kv_quant_vec16<E>, dim3((unsigned)blocks), dim3(threads), 0, s, a);
  else hipLaunchKernelGGL(kv_quant_elem<E>, dim3((unsigned)blocks), dim3(threads), 0, s, a);
}

}  // namespace

extern "C" int li_kv_scatter_fp8(const void* k, const void* v, const int64_t* k_strides, const int64_t* v_strides,
                                 int64_t batch, int64_t tokens, const int64_t* slots, void* key_pool,
                                 void* value_pool, int64_t num_slots, int64_t pool_stride_slot,
                                 int64_t pool_stride_head, int num_kv_heads, int head_dim, int src_dtype,
                                 float k_scale, float v_scale, int32_t* bad_slots, void* stream) {
  li::clear_error();
  if (src_dtype != LI_F32 && src_dtype != LI_F16 && src_dtype != LI_BF16)
    return li::fail(LI_EINVAL, "li_kv_scatter_fp8: unknown source dtype %d", src_dtype);
  if (!(k_scale > 0.f) || !(v_scale > 0.f) || !std::isfinite(k_scale) || !std::isfinite(v_scale))
    return li::fail(LI_EINVAL, "li_kv_scatter_fp8: scales must be finite and > 0 (k_scale=%g, v_scale=%g)", k_scale,
                    v_scale);
  if (batch < 0 || tokens < 0 || num_kv_heads <= 0 || head_dim <= 0 || num_slots < 0)
    return li::fail(LI_EINVAL, "li_kv_scatter_fp8: negative or empty extent (batch=%lld tokens=%lld heads=%d dim=%d)",
                    (long long)batch, (long long)tokens, num_kv_heads, head_dim);
  if (!k_strides || !v_strides) return li::fail(LI_EINVAL, "li_kv_scatter_fp8: strides must not be null");
  const int64_t n = batch * tokens;
  if (n == 0) return LI_OK;
  if (!k || !v || !slots || !key_pool || !value_pool) return li::fail(LI_EINVAL, "li_kv_scatter_fp8: null pointer");
  if (pool_stride_head < head_dim || pool_stride_slot < (int64_t)num_kv_heads * head_dim)
    return li::fail(LI_EINVAL, "li_kv_scatter_fp8: pool strides (%lld, %lld) overlap rows of %d x %d",
                    (long long)pool_stride_slot, (long long)pool_stride_head, num_kv_heads, head_dim);

  QuantArgs a;
  a.k = static_cast<const char*>(k);
  a.v = static_cast<const char*>(v);
  for (int j = 0; j < 4; ++j) {
    a.ks[j] = k_strides[j];
    a.vs[j] = v_strides[j];
  }
  a.tokens = tokens;
  a.n = n;
  a.slots = slots;
  a.kp = static_cast<uint8_t*>(key_pool);
  a.vp = static_cast<uint8_t*>(value_pool);
  a.num_slots = num_slots;
  a.ps_slot = pool_stride_slot;
  a.ps_head = pool_stride_head;
  a.heads = num_kv_heads;
  a.head_dim = head_dim;
  a.inv_k = 1.f / k_scale;
  a.inv_v = 1.f / v_scale;
  a.bad = bad_slots;

  hipStream_t s = static_cast<hipStream_t>(stream);
  const int esize = li::dtype_size(src_dtype);
  const bool vec = all_aligned(a, esize);
  if (src_dtype == LI_BF16) launch<li_bf16>(a, vec, s);
  else if (src_dtype == LI_F16) launch<li_f16>(a, vec, s);
  else launch<float>(a, vec, s);
  return li::check_launch("li_kv_scatter_fp8");
}
