// Paged decode on CDNA4 matrix cores (bf16 / fp16, head_dim 64 or 128).
//
// Same attention as liteinfer's decode kernels (liteinfer/models/
// paged_kernels.py:374-413, :462-571): per (sequence, KV head, partition),
// the G query heads sharing a KV head fold the partition's keys into an
// online softmax, fp32 throughout, weights rounded to the value dtype before
// they multiply V. One wave64 per partition, 32 keys per step, laid out for
// v_mfma_f32_16x16x32_{bf16,f16}. Lane (n, g) = (lane % 16, lane / 16).
//
// Loads. Lane (n, g) loads 16 bytes (dims 8n..8n+7) of K and of V for each of
// the 8 keys kappa(g, 0..7) = {4g..4g+3, 16+4g..16+4g+3} of the tile, so each
// load instruction reads 4 whole 256-byte pool rows, 16 lanes per row. (A
// layout where 16 lanes each read 64 bytes of 16 different rows measured 20%
// less HBM bandwidth.) The next tile's loads are always in flight while the
// current one is folded.
//
//   S^T = K Q^T     A = K (16 keys x 32 dims), B = Q^T (32 dims x 16 heads).
//                   The A operand wants lane (m, g) to hold 8 dims of key m,
//                   so K goes through LDS once: rows written as loaded, read
//                   back at dims 32j + 8g (rows padded to 272 bytes, so 16
//                   lanes reading 16 rows hit 16 distinct bank groups). The
//                   result gives lane (n, g) the scores of keys 4g..4g+3 (and
//                   16+4g.. from the second block) for head n.
//   O^T += V^T P^T  A = V^T (16 rows x 32 keys), B = P^T (32 keys x 16 heads).
//                   Lane (n, g)'s 8 weights are for keys kappa(g, 0..7) of
//                   head n: exactly its B operand, no lane exchange. Its 8
//                   V chunks (8 keys x dims 8n..8n+7) become 8 A operands by
//                   a register-only 8x8 transpose: row n of instruction i is
//                   dim 8n + i.
//   The result gives lane (n, g) dims {8(4g+r) + i} of head n, so the
//   running-max rescale is per lane (its own head) and nothing is reduced
//   across lanes except the tile maximum (two xor shuffles) and, once at the
//   end, the denominator.
//
// Heads past G are zero rows of Q^T: they score 0 and are never stored.
// Keys past the partition's end read the last key's slot (a real row) and
// are masked to -inf, so every load is in bounds.
#include "li_attention.h"
#include "li_mfma.h"

#include <cstdlib>

namespace li {
namespace {

// Issues the 2 * kInsts direct-to-LDS loads of the 32-key tile whose first
// key is entry `t` of the staged slots, into the stage at `stage`. Lane
// (rr, n) = (lane / CH, lane % CH) loads keys rr * kInsts + i.
template <typename T, int D>
__device__ __forceinline__ void issue_tile(char* stage, const T* __restrict__ kpool, const T* __restrict__ vpool,
                                           const int* __restrict__ sl, int64_t p_s0, int t, int lane) {
  using L = TileLayout<D>;
  const int rr = lane / L::kCh, nn = lane % L::kCh;
  int keys[L::kInsts];
  if constexpr (L::kInsts == 8) {
    const int4 a = *reinterpret_cast<const int4*>(sl + t + 8 * rr);
    const int4 b = *reinterpret_cast<const int4*>(sl + t + 8 * rr + 4);
    keys[0] = a.x; keys[1] = a.y; keys[2] = a.z; keys[3] = a.w;
    keys[4] = b.x; keys[5] = b.y; keys[6] = b.z; keys[7] = b.w;
  } else {
    const int4 a = *reinterpret_cast<const int4*>(sl + t + 4 * rr);
    keys[0] = a.x; keys[1] = a.y; keys[2] = a.z; keys[3] = a.w;
  }
#pragma unroll
  for (int i = 0; i < L::kInsts; ++i) {
    const int key = rr * L::kInsts + i;
    const int chunk = nn ^ (key % L::kCh);
    const uint32_t dst = lds_addr(stage + i * 1024);  // rows kRowsPerInst * i ..: 1 KiB per instruction
    const uint32_t row_bytes = (uint32_t)(p_s0 * sizeof(T));
    dma16(row_ptr(kpool + 8 * chunk, (uint32_t)keys[i], row_bytes), dst);
    dma16(row_ptr(vpool + 8 * chunk, (uint32_t)keys[i], row_bytes), dst + 32 * L::kRowBytes);
  }
}

template <typename T, int D, int kStages>
__global__ __launch_bounds__(64) void decode_mfma(AttnArgs a) {
  using M = Mfma<T>;
  using Frag = typename M::Frag;
  using L = TileLayout<D>;
  constexpr int kSteps = D / 32;
  constexpr int kChunks = D / 8;
  __shared__ __attribute__((aligned(16))) int sl[kSlotChunk + 64];
  // Two stages as separate LDS objects, so the compiler can tell a read of
  // one from the direct-to-LDS loads still landing in the other.
  __shared__ __attribute__((aligned(1024))) char stage0[L::kTileBytes];
  __shared__ __attribute__((aligned(1024))) char stage1[L::kTileBytes];
  __shared__ __attribute__((aligned(1024))) char stage2[kStages == 3 ? L::kTileBytes : 16];

  const int lane = threadIdx.x;
  const int n = lane & 15, g = lane >> 4;
  // Partition-major order: every sequence's first partition is dispatched
  // before any second one, so the grid's empty tail (partitions past a short
  // context) comes last and exits at once.
  int bid = blockIdx.x;
  const int kvh = bid % a.num_kv_heads;
  bid /= a.num_kv_heads;
  const int seq = bid % a.batch;
  const int part = bid / a.batch;

  // In a packed pass (qsl set) this kernel serves the one-query sequences;
  // their query and output rows are where the pass packs them.
  int row = seq;
  if (a.qsl) {
    row = a.qsl[seq];
    if (a.qsl[seq + 1] - row != 1) return;
  }
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
    const T* qrow = static_cast<const T*>(a.q) + (int64_t)row * a.q_s0 + (int64_t)head * a.q_s1 + 8 * g;
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
  const float sc = a.scale * kLog2eMfma;

  float m = -INFINITY, l = 0.f;
  floatx4_t acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = floatx4_t{0.f, 0.f, 0.f, 0.f};

  for (int c0 = kb; c0 < ke; c0 += kSlotChunk) {
    const int c1 = min(c0 + kSlotChunk, ke);
    const int len = c1 - c0;
    const int ntiles = (len + 31) / 32;
    // Stage this chunk's slots (int32: a pool holds fewer than 2^31 slots),
    // plus two tiles past its end. Entries past the chunk repeat its last
    // slot, so the loads of a partial tile read real rows; their scores are
    // masked.
    __syncthreads();
    {
      int vals[kSlotChunk / 64 + 1];
#pragma unroll
      for (int k = 0; k < kSlotChunk / 64 + 1; ++k) vals[k] = (int)srow[min(c0 + lane + 64 * k, c1 - 1)];
#pragma unroll
      for (int k = 0; k < kSlotChunk / 64 + 1; ++k) sl[lane + 64 * k] = vals[k];
    }
    __syncthreads();

    // Folds the tile in `stage` whose first key is t0.
    auto fold = [&](const char* stage, int t0) {
      const char* vstage = stage + 32 * L::kRowBytes;
      floatx4_t s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < kSteps; ++j) {
        const Frag k0 = *reinterpret_cast<const Frag*>(stage + L::offset(n, 4 * j + g));
        const Frag k1 = *reinterpret_cast<const Frag*>(stage + L::offset(16 + n, 4 * j + g));
        s0 = M::mma(k0, qf[j], s0);
        s1 = M::mma(k1, qf[j], s1);
      }
      u32x4_t vr[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        vr[e] = (n < kChunks) ? *reinterpret_cast<const u32x4_t*>(vstage + L::offset(kappa(g, e), n))
                              : u32x4_t{0u, 0u, 0u, 0u};
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
        x[e] = (t0 + kappa(g, e) < c1) ? x[e] * sc : -INFINITY;
        mx = fmaxf(mx, x[e]);
      }
      mx = li_group_max(mx);
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
          const uint32_t lo = vr[2 * u][w], hi = vr[2 * u + 1][w];
          va[u] = (i & 1) ? ((lo >> 16) | (hi & 0xffff0000u)) : ((lo & 0xffffu) | (hi << 16));
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[i][r] *= alpha;
        acc[i] = M::mma(__builtin_bit_cast(Frag, va), pf, acc[i]);
      }
      m = mnew;
    };

    // kStages stages: while one tile is folded the next kStages - 1 tiles'
    // loads land in the others. Past the chunk the look-ahead re-reads a real
    // tile (cache hits), so the loads in flight are the same every step and
    // no load sits under a branch.
    constexpr int kInFlight = 2 * L::kInsts * (kStages - 1);
    issue_tile<T, D>(stage0, kpool, vpool, sl, a.p_s0, 0, lane);
    if constexpr (kStages == 3) issue_tile<T, D>(stage1, kpool, vpool, sl, a.p_s0, min(32, kSlotChunk), lane);
    for (int ti = 0;;) {
      issue_tile<T, D>(kStages == 3 ? stage2 : stage1, kpool, vpool, sl, a.p_s0,
                       min(32 * (ti + kStages - 1), kSlotChunk), lane);
      li_wait_vm<kInFlight>();
      fold(stage0, c0 + 32 * ti);
      if (++ti >= ntiles) break;
      issue_tile<T, D>(stage0, kpool, vpool, sl, a.p_s0, min(32 * (ti + kStages - 1), kSlotChunk), lane);
      li_wait_vm<kInFlight>();
      fold(stage1, c0 + 32 * ti);
      if (++ti >= ntiles) break;
      if constexpr (kStages == 3) {
        issue_tile<T, D>(stage1, kpool, vpool, sl, a.p_s0, min(32 * (ti + kStages - 1), kSlotChunk), lane);
        li_wait_vm<kInFlight>();
        fold(stage2, c0 + 32 * ti);
        if (++ti >= ntiles) break;
      }
    }
    // Drain the look-ahead loads before the slots (and stages) are reused.
    li_wait_vm<0>();
  }

  const float lt = li_group_sum(l);
  if (!real_head) return;
  const float inv = 1.f / lt;

  if (nparts == 1) {
    T* orow = static_cast<T*>(a.out) + (int64_t)row * a.o_s0 + (int64_t)head * a.o_s1;
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
  static const int stages = [] {
    const char* v = std::getenv("LI_DECODE_STAGES");
    return (v && v[0] == '3') ? 3 : 2;
  }();
  if (dtype == LI_BF16) {
    if (a.head_dim == 128) {
      if (stages == 3) hipLaunchKernelGGL((decode_mfma<li_bf16, 128, 3>), grid, block, 0, s, a);
      else hipLaunchKernelGGL((decode_mfma<li_bf16, 128, 2>), grid, block, 0, s, a);
    } else {
      hipLaunchKernelGGL((decode_mfma<li_bf16, 64, 2>), grid, block, 0, s, a);
    }
  } else {
    if (a.head_dim == 128) hipLaunchKernelGGL((decode_mfma<li_f16, 128, 2>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((decode_mfma<li_f16, 64, 2>), grid, block, 0, s, a);
  }
  return check_launch("decode_mfma");
}

}  // namespace li
