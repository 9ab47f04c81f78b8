// Paged decode on CDNA4 matrix cores (bf16 / fp16, head_dim 64 or 128).
//
// Same attention as liteinfer's decode kernels (liteinfer/models/
// paged_kernels.py:374-413, :462-571): per (sequence, KV head, partition),
// the G query heads sharing a KV head fold the partition's keys into an
// online softmax, fp32 throughout, weights rounded to the value dtype before
// they multiply V. The work is laid out for v_mfma_f32_16x16x32_{bf16,f16}
// and for 16-byte loads straight from the pool:
//
//   S^T = K Q^T     A = K rows (16 keys x 32 dims), B = Q^T (32 dims x 16
//                   heads). Lane (n, g) = (lane % 16, lane / 16) holds 8 dims
//                   of key n and the same 8 dims of head n; the result gives
//                   lane (n, g) the scores of keys 4g..4g+3 for head n.
//   O^T += V^T P^T  A = V^T (16 rows x 32 keys), B = P^T (32 keys x 16 heads).
//                   Two S^T blocks give lane (n, g) the 8 weights of keys
//                   {4g..4g+3, 16+4g..16+4g+3} for head n: exactly its B
//                   operand, with no lane exchange. For the A operand lane
//                   (n, g) loads 16 bytes (dims 8n..8n+7) of each of those 8
//                   keys, so 16 lanes cover one 256-byte pool row per load
//                   instruction, and a register-only 8x8 transpose turns them
//                   into 8 A operands, one per dim within the chunk: row n of
//                   instruction i is dim 8n + i.
//   The result gives lane (n, g) dims {8(4g+r) + i} of head n, so the
//   running-max rescale is per lane (its own head) and nothing is reduced
//   across lanes except the tile maximum (two xor shuffles) and, once at the
//   end, the denominator.
//
// Heads past G are zero rows of Q^T: they score 0 and are never stored.
// Keys past the partition's end are clamped to its last key for the load and
// masked to -inf for the softmax, so every load is in bounds. One wave64 per
// partition; the next 32-key tile is loaded while the current one is folded.
#include "li_attention.h"

namespace li {
namespace {

template <typename T>
struct Mfma;
template <>
struct Mfma<li_bf16> {
  using Frag = bf16x8_t;
  static __device__ __forceinline__ floatx4_t mma(Frag a, Frag b, floatx4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};
template <>
struct Mfma<li_f16> {
  using Frag = f16x8_t;
  static __device__ __forceinline__ floatx4_t mma(Frag a, Frag b, floatx4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};

constexpr float kLog2e = 1.4426950408889634f;

template <typename T, int D>
struct DecodeTile {
  using Frag = typename Mfma<T>::Frag;
  Frag k0[D / 32];  // key n of the tile, dims 32j + 8g ..
  Frag k1[D / 32];  // key 16 + n
  u32x4_t v[8];     // dims 8n.. of key kappa(g, e)
};

// Key of the tile whose weight lane group g holds in B-operand slot e.
__device__ __forceinline__ int kappa(int g, int e) { return (e < 4 ? 4 * g + e : 16 + 4 * g + (e - 4)); }

template <typename T, int D>
__device__ __forceinline__ void load_tile(DecodeTile<T, D>& tl, const T* __restrict__ kpool,
                                          const T* __restrict__ vpool, const int64_t* __restrict__ srow,
                                          int64_t p_s0, int t0, int ke, int n, int g) {
  using Frag = typename Mfma<T>::Frag;
  constexpr int kChunks = D / 8;
  const int64_t s0 = srow[min(t0 + n, ke - 1)];
  const int64_t s1 = srow[min(t0 + 16 + n, ke - 1)];
  const T* r0 = kpool + s0 * p_s0 + 8 * g;
  const T* r1 = kpool + s1 * p_s0 + 8 * g;
#pragma unroll
  for (int j = 0; j < D / 32; ++j) {
    tl.k0[j] = *reinterpret_cast<const Frag*>(r0 + 32 * j);
    tl.k1[j] = *reinterpret_cast<const Frag*>(r1 + 32 * j);
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int64_t sv = srow[min(t0 + kappa(g, e), ke - 1)];
    if (n < kChunks) {
      tl.v[e] = *reinterpret_cast<const u32x4_t*>(vpool + sv * p_s0 + 8 * n);
    } else {
      tl.v[e] = u32x4_t{0u, 0u, 0u, 0u};
    }
  }
}

template <typename T, int D>
__global__ __launch_bounds__(64) void decode_mfma(AttnArgs a) {
  using M = Mfma<T>;
  using Frag = typename M::Frag;
  constexpr int kSteps = D / 32;
  constexpr int kChunks = D / 8;

  const int lane = threadIdx.x;
  const int n = lane & 15, g = lane >> 4;
  int bid = blockIdx.x;
  const int part = bid % a.num_parts;
  bid /= a.num_parts;
  const int kvh = bid % a.num_kv_heads;
  const int seq = bid / a.num_kv_heads;

  const int ctx = a.ctx[seq];
  const int plen = a.part_len > 0 ? a.part_len : max(1, (ctx + a.num_parts - 1) / a.num_parts);
  const int kb = part * plen;
  if (kb >= ctx) return;
  const int ke = min(kb + plen, ctx);
  const int nparts = (ctx + plen - 1) / plen;

  const bool real_head = n < a.groups;
  const int head = kvh * a.groups + n;

  Frag qf[kSteps];
  {
    const T* qrow = static_cast<const T*>(a.q) + (int64_t)seq * a.q_s0 + (int64_t)head * a.q_s1 + 8 * g;
#pragma unroll
    for (int j = 0; j < kSteps; ++j) {
      if (real_head) {
        qf[j] = *reinterpret_cast<const Frag*>(qrow + 32 * j);
      } else {
        qf[j] = Frag{};
      }
    }
  }

  const T* kpool = static_cast<const T*>(a.kp) + (int64_t)kvh * a.p_s1;
  const T* vpool = static_cast<const T*>(a.vp) + (int64_t)kvh * a.p_s1;
  const int64_t* srow = a.st + (int64_t)seq * a.st_s;
  const float sc = a.scale * kLog2e;

  float m = -INFINITY, l = 0.f;
  floatx4_t acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = floatx4_t{0.f, 0.f, 0.f, 0.f};

  DecodeTile<T, D> cur, nxt;
  load_tile<T, D>(cur, kpool, vpool, srow, a.p_s0, kb, ke, n, g);

  for (int t0 = kb; t0 < ke; t0 += 32) {
    const bool more = t0 + 32 < ke;
    if (more) load_tile<T, D>(nxt, kpool, vpool, srow, a.p_s0, t0 + 32, ke, n, g);

    floatx4_t s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < kSteps; ++j) {
      s0 = M::mma(cur.k0[j], qf[j], s0);
      s1 = M::mma(cur.k1[j], qf[j], s1);
    }
    float x[8];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      x[r] = s0[r];
      x[4 + r] = s1[r];
    }
    float mx = -INFINITY;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      x[e] = (t0 + kappa(g, e) < ke) ? x[e] * sc : -INFINITY;
      mx = fmaxf(mx, x[e]);
    }
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float mnew = fmaxf(m, mx);
    const float alpha = __builtin_amdgcn_exp2f(m - mnew);
    float psum = 0.f;
    float p[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      p[e] = __builtin_amdgcn_exp2f(x[e] - mnew);
      psum += p[e];
    }
    l = l * alpha + psum;
    u32x4_t pw;
#pragma unroll
    for (int u = 0; u < 4; ++u) pw[u] = li_pack2<T>(p[2 * u], p[2 * u + 1]);
    const Frag pf = __builtin_bit_cast(Frag, pw);

#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int w = i >> 1;
      u32x4_t va;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const uint32_t lo = cur.v[2 * u][w], hi = cur.v[2 * u + 1][w];
        va[u] = (i & 1) ? ((lo >> 16) | (hi & 0xffff0000u)) : ((lo & 0xffffu) | (hi << 16));
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[i][r] *= alpha;
      acc[i] = M::mma(__builtin_bit_cast(Frag, va), pf, acc[i]);
    }
    m = mnew;
    if (more) cur = nxt;
  }

  float lt = l + __shfl_xor(l, 16, 64);
  lt = lt + __shfl_xor(lt, 32, 64);
  if (!real_head) return;
  const float inv = 1.f / lt;

  if (nparts == 1) {
    T* orow = static_cast<T*>(a.out) + (int64_t)seq * a.o_s0 + (int64_t)head * a.o_s1;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int chunk = 4 * g + r;
      if (chunk < kChunks) {
        u32x4_t w;
#pragma unroll
        for (int u = 0; u < 4; ++u) w[u] = li_pack2<T>(acc[2 * u][r] * inv, acc[2 * u + 1][r] * inv);
        *reinterpret_cast<u32x4_t*>(orow + 8 * chunk) = w;
      }
    }
  } else {
    const int64_t base = ((int64_t)seq * a.num_heads + head) * a.num_parts + part;
    float* po = a.part_o + base * D;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int chunk = 4 * g + r;
      if (chunk < kChunks) {
        floatx4_t lo4, hi4;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          lo4[i] = acc[i][r] * inv;
          hi4[i] = acc[4 + i][r] * inv;
        }
        *reinterpret_cast<floatx4_t*>(po + 8 * chunk) = lo4;
        *reinterpret_cast<floatx4_t*>(po + 8 * chunk + 4) = hi4;
      }
    }
    if (g == 0) a.part_lse[base] = m + log2f(lt);
  }
}

bool rows_aligned(const void* p, int64_t s0, int64_t s1, int esize) {
  return aligned16(p) && (s0 * esize) % 16 == 0 && (s1 * esize) % 16 == 0;
}

}  // namespace

bool decode_mfma_applies(const AttnArgs& a, int dtype) {
  if (dtype != LI_BF16 && dtype != LI_F16) return false;
  if (a.head_dim != 64 && a.head_dim != 128) return false;
  if (a.groups < 1 || a.groups > 16) return false;
  return rows_aligned(a.q, a.q_s0, a.q_s1, 2) && rows_aligned(a.out, a.o_s0, a.o_s1, 2) &&
         rows_aligned(a.kp, a.p_s0, a.p_s1, 2) && rows_aligned(a.vp, a.p_s0, a.p_s1, 2);
}

int launch_decode_mfma(const AttnArgs& a, int dtype, hipStream_t s) {
  const int64_t blocks = (int64_t)a.batch * a.num_kv_heads * a.num_parts;
  if (blocks == 0) return LI_OK;
  if (blocks > 0x7fffffffLL) return fail(LI_EUNSUPPORTED, "decode grid of %lld blocks is too large", (long long)blocks);
  const dim3 grid((unsigned)blocks), block(64);
  if (dtype == LI_BF16) {
    if (a.head_dim == 128) hipLaunchKernelGGL((decode_mfma<li_bf16, 128>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((decode_mfma<li_bf16, 64>), grid, block, 0, s, a);
  } else {
    if (a.head_dim == 128) hipLaunchKernelGGL((decode_mfma<li_f16, 128>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((decode_mfma<li_f16, 64>), grid, block, 0, s, a);
  }
  return check_launch("decode_mfma");
}

}  // namespace li
