// General-shape paged attention, and the partition combine.
//
// Serves every shape the MFMA kernels do not: fp32 pools (whose parity bar is
// 1e-5, so the arithmetic stays fp32 throughout), any head_dim up to 512 and
// any number of query heads per KV head. It is the same attention as
// liteinfer's Triton body (liteinfer/models/paged_kernels.py:216-371): an
// online softmax folded over key tiles, m' = max(m, rowmax(s)),
// acc = acc * e^(m - m') + e^(s - m') V, l = l * e^(m - m') + sum e^(s - m'),
// output acc / l; the weights are rounded to the value dtype before they
// multiply V (paged_kernels.py:280-282). A query at position p sees keys
// 0..p (attention.py:81-84); a decode query is the last position.
//
// One wave64 per (sequence, KV head, query block, partition); it walks the
// block's rows (query, head) one at a time. Lane j scores key t0 + j of a
// tile, then the tile's weights are broadcast lane to lane while each lane
// accumulates the dims it owns (d = lane + 64 c).
#include "li_attention.h"

namespace li {
namespace {

constexpr float kLog2e = 1.4426950408889634f;

template <typename T>
__global__ __launch_bounds__(64) void attend_generic(AttnArgs a) {
  constexpr int kMaxC = kGenericMaxHeadDim / 64;
  __shared__ float qs[kGenericMaxHeadDim];

  const int lane = threadIdx.x;
  int64_t bid = blockIdx.x;
  const int part = (int)(bid % a.num_parts);
  bid /= a.num_parts;
  const int kvh = (int)(bid % a.num_kv_heads);
  bid /= a.num_kv_heads;
  const int qblock = (int)(bid % a.num_qblocks);
  const int seq = (int)(bid / a.num_qblocks);

  const int ctx = a.ctx[seq];
  int first_tok, nq;
  if (a.qsl) {
    first_tok = a.qsl[seq];
    nq = a.qsl[seq + 1] - first_tok;
  } else {
    first_tok = seq;
    nq = 1;
  }
  const int q0 = qblock * a.block_q;
  if (q0 >= nq) return;
  const int q1 = min(q0 + a.block_q, nq);
  if (ctx <= 0) {
    // A decode row with no key to attend to: the reference's softmax over
    // nothing is 0 / 0.
    if (part == 0) {
      for (int qi = q0; qi < q1; ++qi)
        for (int h = 0; h < a.groups; ++h) {
          T* orow = static_cast<T*>(a.out) + (int64_t)(first_tok + qi) * a.o_s0 +
                    (int64_t)(kvh * a.groups + h) * a.o_s1;
          for (int d = threadIdx.x; d < a.head_dim; d += blockDim.x) orow[d] = li_quiet_nan<T>();
        }
    }
    return;
  }

  int kb = 0, ke = ctx, nparts = 1;
  if (a.part_o) {
    const int plen = a.part_len > 0 ? a.part_len : max(1, (ctx + a.num_parts - 1) / a.num_parts);
    kb = part * plen;
    if (kb >= ctx) return;
    ke = min(kb + plen, ctx);
    nparts = (ctx + plen - 1) / plen;
  } else if (part > 0) {
    return;
  }

  const T* qp = static_cast<const T*>(a.q);
  const T* kpool = static_cast<const T*>(a.kp) + (int64_t)kvh * a.p_s1;
  const T* vpool = static_cast<const T*>(a.vp) + (int64_t)kvh * a.p_s1;
  const int64_t* srow = a.st + (int64_t)seq * a.st_s;
  const int D = a.head_dim;
  const int bkv = min(max(a.block_kv, 1), 64);

  for (int qi = q0; qi < q1; ++qi) {
    const int pos = ctx - nq + qi;  // this query's position in its context
    const int kend = min(ke, pos + 1);
    const int64_t tok = first_tok + qi;
    for (int h = 0; h < a.groups; ++h) {
      const int head = kvh * a.groups + h;
      __syncthreads();
      for (int d = lane; d < D; d += 64) qs[d] = li_to_float(qp[tok * a.q_s0 + (int64_t)head * a.q_s1 + d]);
      __syncthreads();

      float m = -INFINITY, l = 0.f;
      float acc[kMaxC];
#pragma unroll
      for (int c = 0; c < kMaxC; ++c) acc[c] = 0.f;

      for (int t0 = kb; t0 < kend; t0 += bkv) {
        const int key = t0 + lane;
        const bool valid = lane < bkv && key < kend;
        int64_t slot = valid ? srow[key] : 0;
        float s = -INFINITY;
        if (valid) {
          const T* kr = kpool + slot * a.p_s0;
          float dot = 0.f;
          for (int d = 0; d < D; ++d) dot = fmaf(qs[d], li_to_float(kr[d]), dot);
          s = dot * a.scale;
        }
        const float mnew = fmaxf(m, li_wave_max(s));
        const float alpha = (m == -INFINITY) ? 0.f : expf(m - mnew);
        const float p = valid ? expf(s - mnew) : 0.f;
        l = l * alpha + li_wave_sum(p);
        const float pv = li_to_float(li_from_float<T>(p));
#pragma unroll
        for (int c = 0; c < kMaxC; ++c) acc[c] *= alpha;
        const int nvalid = min(bkv, kend - t0);
        const int slot_lo = (int)(slot & 0xffffffff);
        const int slot_hi = (int)(slot >> 32);
        for (int j = 0; j < nvalid; ++j) {
          const float pj = __shfl(pv, j, 64);
          const int64_t sj = ((int64_t)__shfl(slot_hi, j, 64) << 32) | (uint32_t)__shfl(slot_lo, j, 64);
          const T* vr = vpool + sj * a.p_s0;
#pragma unroll
          for (int c = 0; c < kMaxC; ++c) {
            const int d = lane + 64 * c;
            if (d < D) acc[c] = fmaf(pj, li_to_float(vr[d]), acc[c]);
          }
        }
        m = mnew;
      }

      const float inv = 1.f / l;
      if (nparts > 1) {
        float* po = a.part_o + (((int64_t)seq * a.num_heads + head) * a.num_parts + part) * D;
#pragma unroll
        for (int c = 0; c < kMaxC; ++c) {
          const int d = lane + 64 * c;
          if (d < D) po[d] = acc[c] * inv;
        }
        if (lane == 0)
          a.part_lse[((int64_t)seq * a.num_heads + head) * a.num_parts + part] = m * kLog2e + log2f(l);
      } else {
        T* orow = static_cast<T*>(a.out) + tok * a.o_s0 + (int64_t)head * a.o_s1;
#pragma unroll
        for (int c = 0; c < kMaxC; ++c) {
          const int d = lane + 64 * c;
          if (d < D) orow[d] = li_from_float<T>(acc[c] * inv);
        }
      }
    }
  }
}

// Folds a sequence's partitions: w_p = 2^(lse_p - max lse), out = sum w_p o_p
// / sum w_p (paged_kernels.py:574-629, in the log2 domain). One wave per
// (head, sequence); a sequence that fit one partition was written directly.
// Lane j holds the weights of partitions j, j + 64, ...; the partial rows are
// read eight partitions at a time so their loads overlap.
template <typename T>
__global__ __launch_bounds__(64) void combine_parts(AttnArgs a) {
  constexpr int kMaxC = kGenericMaxHeadDim / 64;
  constexpr int kBatch = 8;
  const int lane = threadIdx.x;
  const int head = blockIdx.x % a.num_heads;
  const int seq = blockIdx.x / a.num_heads;
  int row = seq;
  if (a.qsl) {  // a packed pass: only its one-query sequences were partitioned
    row = a.qsl[seq];
    if (a.qsl[seq + 1] - row != 1) return;
  }
  const int ctx = a.ctx[seq];
  const int plen = a.part_len > 0 ? a.part_len : max(1, (ctx + a.num_parts - 1) / a.num_parts);
  const int nparts = (ctx + plen - 1) / plen;
  if (nparts <= 1) return;
  const int D = a.head_dim;
  const int64_t base = ((int64_t)seq * a.num_heads + head) * a.num_parts;
  const float* lse = a.part_lse + base;
  const float* po = a.part_o + base * D;

  float mx = -INFINITY;
  for (int p = lane; p < nparts; p += 64) mx = fmaxf(mx, lse[p]);
  mx = li_wave_max(mx);
  float wsum = 0.f;
  for (int p = lane; p < nparts; p += 64) wsum += exp2f(lse[p] - mx);
  wsum = li_wave_sum(wsum);

  float acc[kMaxC];
#pragma unroll
  for (int c = 0; c < kMaxC; ++c) acc[c] = 0.f;
  for (int p0 = 0; p0 < nparts; p0 += 64) {
    const float wl = (p0 + lane < nparts) ? exp2f(lse[p0 + lane] - mx) : 0.f;
    const int pend = min(64, nparts - p0);
    for (int pb = 0; pb < pend; pb += kBatch) {
      float v[kBatch][kMaxC];
#pragma unroll
      for (int k = 0; k < kBatch; ++k) {
        const int p = p0 + pb + k;
#pragma unroll
        for (int c = 0; c < kMaxC; ++c) {
          const int d = lane + 64 * c;
          v[k][c] = (pb + k < pend && d < D) ? po[(int64_t)p * D + d] : 0.f;
        }
      }
#pragma unroll
      for (int k = 0; k < kBatch; ++k) {
        const float w = __shfl(wl, (pb + k) & 63, 64);
#pragma unroll
        for (int c = 0; c < kMaxC; ++c) acc[c] = fmaf(w, v[k][c], acc[c]);
      }
    }
  }
  const float inv = 1.f / wsum;
  T* orow = static_cast<T*>(a.out) + (int64_t)row * a.o_s0 + (int64_t)head * a.o_s1;
#pragma unroll
  for (int c = 0; c < kMaxC; ++c) {
    const int d = lane + 64 * c;
    if (d < D) orow[d] = li_from_float<T>(acc[c] * inv);
  }
}

}  // namespace

int launch_attend_generic(const AttnArgs& a, int dtype, hipStream_t s) {
  const int64_t blocks = (int64_t)a.batch * a.num_qblocks * a.num_kv_heads * a.num_parts;
  if (blocks == 0) return LI_OK;
  if (blocks > 0xffffffffLL) return fail(LI_EUNSUPPORTED, "attention grid of %lld blocks is too large", (long long)blocks);
  switch (dtype) {
    case LI_F32: hipLaunchKernelGGL(attend_generic<float>, dim3((unsigned)blocks), dim3(64), 0, s, a); break;
    case LI_F16: hipLaunchKernelGGL(attend_generic<li_f16>, dim3((unsigned)blocks), dim3(64), 0, s, a); break;
    case LI_BF16: hipLaunchKernelGGL(attend_generic<li_bf16>, dim3((unsigned)blocks), dim3(64), 0, s, a); break;
    default: return fail(LI_EINVAL, "unknown dtype %d", dtype);
  }
  return check_launch("attend_generic");
}

int launch_combine(const AttnArgs& a, int dtype, hipStream_t s) {
  const int64_t blocks = (int64_t)a.batch * a.num_heads;
  if (blocks == 0) return LI_OK;
  switch (dtype) {
    case LI_F32: hipLaunchKernelGGL(combine_parts<float>, dim3((unsigned)blocks), dim3(64), 0, s, a); break;
    case LI_F16: hipLaunchKernelGGL(combine_parts<li_f16>, dim3((unsigned)blocks), dim3(64), 0, s, a); break;
    case LI_BF16: hipLaunchKernelGGL(combine_parts<li_bf16>, dim3((unsigned)blocks), dim3(64), 0, s, a); break;
    default: return fail(LI_EINVAL, "unknown dtype %d", dtype);
  }
  return check_launch("combine_parts");
}

}  // namespace li
