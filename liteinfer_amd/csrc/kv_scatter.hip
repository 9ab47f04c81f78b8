// KV slot-write: this pass's K and V rows into their pool slots.
//
// Counterpart of KVCache.scatter (liteinfer/cache/kv_cache.py:236-247) with
// _tokens_first (kv_cache.py:250-253). Token i of the batch-major order is
// (b, t) = (i / T, i % T); its K row for head h is k[b, h, t, :], and it lands
// at key_pool[slots[i], h, :]. The copy is bit-exact: bytes move, nothing is
// converted. One work item moves 16 bytes of K and the same 16 bytes of V,
// so a wave writes 1 KiB of each in one store instruction; a head row of
// 128 bf16 is 16 work items.
#include "li_common.h"

namespace {

struct ScatterArgs {
  const char* k;
  const char* v;
  int64_t ks[4];  // element strides of k: batch, head, token, dim
  int64_t vs[4];
  int64_t tokens;  // T
  int64_t n;       // B * T
  const int64_t* slots;
  char* kp;
  char* vp;
  int64_t num_slots;
  int64_t ps_slot;  // element strides of the pools
  int64_t ps_head;
  int heads;
  int head_dim;
  int esize;  // bytes per element
  int* bad;   // nullable: counts tokens whose slot is out of range
};

// 16-byte units: the row of one head is head_dim * esize / 16 units.
__global__ __launch_bounds__(256) void kv_scatter_vec16(ScatterArgs a) {
  const int units = a.head_dim * a.esize / 16;
  const int64_t per_token = (int64_t)a.heads * units;
  const int64_t total = a.n * per_token;
  const int epu = 16 / a.esize;  // elements per unit
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
    const int64_t d = (int64_t)u * epu;
    const int64_t ko = b * a.ks[0] + h * a.ks[1] + t * a.ks[2] + d;
    const int64_t vo = b * a.vs[0] + h * a.vs[1] + t * a.vs[2] + d;
    const int64_t po = slot * a.ps_slot + h * a.ps_head + d;
    const u32x4_t kx = *reinterpret_cast<const u32x4_t*>(a.k + ko * a.esize);
    const u32x4_t vx = *reinterpret_cast<const u32x4_t*>(a.v + vo * a.esize);
    *reinterpret_cast<u32x4_t*>(a.kp + po * a.esize) = kx;
    *reinterpret_cast<u32x4_t*>(a.vp + po * a.esize) = vx;
  }
}

// Any strides: one element per work item.
template <typename E>
__global__ __launch_bounds__(256) void kv_scatter_elem(ScatterArgs a) {
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
    const int64_t ko = b * a.ks[0] + h * a.ks[1] + t * a.ks[2] + d * a.ks[3];
    const int64_t vo = b * a.vs[0] + h * a.vs[1] + t * a.vs[2] + d * a.vs[3];
    const int64_t po = slot * a.ps_slot + h * a.ps_head + d;
    reinterpret_cast<E*>(a.kp)[po] = reinterpret_cast<const E*>(a.k)[ko];
    reinterpret_cast<E*>(a.vp)[po] = reinterpret_cast<const E*>(a.v)[vo];
  }
}

bool all_aligned(const ScatterArgs& a) {
  if (!li::aligned16(a.k) || !li::aligned16(a.v) || !li::aligned16(a.kp) || !li::aligned16(a.vp)) return false;
  if (a.ks[3] != 1 || a.vs[3] != 1) return false;
  if ((a.head_dim * a.esize) % 16 != 0) return false;
  for (int j = 0; j < 3; ++j) {
    if ((a.ks[j] * a.esize) % 16 != 0 || (a.vs[j] * a.esize) % 16 != 0) return false;
  }
  return (a.ps_slot * a.esize) % 16 == 0 && (a.ps_head * a.esize) % 16 == 0;
}

}  // namespace

extern "C" int li_kv_scatter(const void* k, const void* v, const int64_t* k_strides,
                             const int64_t* v_strides, int64_t batch, int64_t tokens,
                             const int64_t* slots, void* key_pool, void* value_pool,
                             int64_t num_slots, int64_t pool_stride_slot,
                             int64_t pool_stride_head, int num_kv_heads, int head_dim,
                             int dtype, int32_t* bad_slots, void* stream) {
  li::clear_error();
  const int esize = li::dtype_size(dtype);
  if (esize == 0) return li::fail(LI_EINVAL, "li_kv_scatter: unknown dtype %d", dtype);
  if (dtype == LI_FP8_E4M3)
    return li::fail(LI_EUNSUPPORTED, "li_kv_scatter: fp8 pools are written by li_kv_scatter_fp8 (quantising), not copied");
  if (batch < 0 || tokens < 0 || num_kv_heads <= 0 || head_dim <= 0 || num_slots < 0)
    return li::fail(LI_EINVAL, "li_kv_scatter: negative or empty extent (batch=%lld tokens=%lld heads=%d dim=%d)",
                    (long long)batch, (long long)tokens, num_kv_heads, head_dim);
  if (!k_strides || !v_strides)
    return li::fail(LI_EINVAL, "li_kv_scatter: strides must not be null");
  const int64_t n = batch * tokens;
  if (n == 0) return LI_OK;
  if (!k || !v || !slots || !key_pool || !value_pool)
    return li::fail(LI_EINVAL, "li_kv_scatter: null pointer");
  if (pool_stride_head < head_dim || pool_stride_slot < (int64_t)num_kv_heads * head_dim)
    return li::fail(LI_EINVAL, "li_kv_scatter: pool strides (%lld, %lld) overlap rows of %d x %d",
                    (long long)pool_stride_slot, (long long)pool_stride_head, num_kv_heads, head_dim);

  ScatterArgs a;
  a.k = static_cast<const char*>(k);
  a.v = static_cast<const char*>(v);
  for (int j = 0; j < 4; ++j) { a.ks[j] = k_strides[j]; a.vs[j] = v_strides[j]; }
  a.tokens = tokens;
  a.n = n;
  a.slots = slots;
  a.kp = static_cast<char*>(key_pool);
  a.vp = static_cast<char*>(value_pool);
  a.num_slots = num_slots;
  a.ps_slot = pool_stride_slot;
  a.ps_head = pool_stride_head;
  a.heads = num_kv_heads;
  a.head_dim = head_dim;
  a.esize = esize;
  a.bad = bad_slots;

  hipStream_t s = static_cast<hipStream_t>(stream);
  const int threads = 256;
  if (all_aligned(a)) {
    const int64_t work = n * num_kv_heads * (head_dim * esize / 16);
    const int64_t blocks = std::min<int64_t>(li::cdiv64(work, threads), 65536);
    hipLaunchKernelGGL(kv_scatter_vec16, dim3((unsigned)blocks), dim3(threads), 0, s, a);
  } else {
    const int64_t work = n * num_kv_heads * head_dim;
    const int64_t blocks = std::min<int64_t>(li::cdiv64(work, threads), 65536);
    if (esize == 4)
      hipLaunchKernelGGL(kv_scatter_elem<uint32_t>, dim3((unsigned)blocks), dim3(threads), 0, s, a);
    else
      hipLaunchKernelGGL(kv_scatter_elem<uint16_t>, dim3((unsigned)blocks), dim3(threads), 0, s, a);
  }
  return li::check_launch("li_kv_scatter");
}
