// The minimal engine's per-layer elementwise work around the attention
// path, fused: the residual add with the RMSNorm that follows it, and the
// SiLU gate of the MLP. Same arithmetic as the model's torch ops (and the
// reference's LlamaRMSNorm / LlamaMLP, liteinfer/models/llama.py:34-48,
// :101-116): sums in fp32, the normalised row rounded to the model dtype
// before the weight multiplies it, every torch-visible intermediate rounded
// where torch rounds it.
#include "li_common.h"

namespace {

constexpr int kNormThreads = 256;

template <typename T>
struct Vec8 {
  typedef __attribute__((__vector_size__(8 * sizeof(T)))) T type;
};

// One work-group per row of `hidden` elements (a multiple of 8 and at most
// 8 * 256 * kNormPer), each thread kNormPer chunks of 8.
constexpr int kNormPer = 4;

// h <- h + delta (when delta is given), rounded to T; out <- weight *
// T(h * rsqrt(mean(h^2) + eps)), the product rounded to T.
template <typename T>
__global__ __launch_bounds__(kNormThreads) void add_rms_norm(T* h, const T* delta, const T* weight, T* out,
                                                            int hidden, int64_t h_s, int64_t d_s, int64_t o_s,
                                                            float eps) {
  typedef typename Vec8<T>::type V;
  const int64_t row = blockIdx.x;
  T* hrow = h + row * h_s;
  const T* drow = delta ? delta + row * d_s : nullptr;
  T* orow = out + row * o_s;
  const int chunks = hidden / 8;
  float x[kNormPer][8];
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < kNormPer; ++k) {
    const int c = threadIdx.x + k * kNormThreads;
    if (c < chunks) {
      V v = *reinterpret_cast<const V*>(hrow + 8 * c);
      if (drow) {
        const V dv = *reinterpret_cast<const V*>(drow + 8 * c);
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = li_from_float<T>((float)v[e] + (float)dv[e]);
        *reinterpret_cast<V*>(hrow + 8 * c) = v;
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        x[k][e] = (float)v[e];
        ss = fmaf(x[k][e], x[k][e], ss);
      }
    }
  }
  __shared__ float partial[kNormThreads / 64];
  ss = li_wave_sum(ss);
  if ((threadIdx.x & 63) == 0) partial[threadIdx.x >> 6] = ss;
  __syncthreads();
  float total = 0.f;
#pragma unroll
  for (int w = 0; w < kNormThreads / 64; ++w) total += partial[w];
  const float inv = rsqrtf(total / (float)hidden + eps);
#pragma unroll
  for (int k = 0; k < kNormPer; ++k) {
    const int c = threadIdx.x + k * kNormThreads;
    if (c < chunks) {
      const V wv = *reinterpret_cast<const V*>(weight + 8 * c);
      V o;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float normed = (float)li_from_float<T>(x[k][e] * inv);
        o[e] = li_from_float<T>((float)wv[e] * normed);
      }
      *reinterpret_cast<V*>(orow + 8 * c) = o;
    }
  }
}

// out[r, i] = T(T(silu(gate)) * up) with gate = gu[r, i], up = gu[r, F + i]
// (torch's F.silu(gate) * up on the two halves of the fused projection).
template <typename T>
__global__ __launch_bounds__(256) void silu_mul(const T* gu, T* out, int64_t rows, int f, int64_t gu_s, int64_t o_s) {
  typedef typename Vec8<T>::type V;
  const int chunks = f / 8;
  const int64_t total = rows * chunks;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / chunks;
    const int c = (int)(i - r * chunks);
    const V g = *reinterpret_cast<const V*>(gu + r * gu_s + 8 * c);
    const V u = *reinterpret_cast<const V*>(gu + r * gu_s + f + 8 * c);
    V o;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float gf = (float)g[e];
      const float s = (float)li_from_float<T>(gf / (1.f + expf(-gf)));
      o[e] = li_from_float<T>(s * (float)u[e]);
    }
    *reinterpret_cast<V*>(out + r * o_s + 8 * c) = o;
  }
}

bool rows_ok(const void* p, int64_t stride, int esize) {
  return li::aligned16(p) && (stride * esize) % 16 == 0;
}

}  // namespace

extern "C" int li_add_rms_norm(void* h, const void* delta, const void* weight, void* out, int64_t rows, int hidden,
                               int64_t h_stride, int64_t delta_stride, int64_t out_stride, float eps, int dtype,
                               void* stream) {
  li::clear_error();
  if (dtype != LI_BF16 && dtype != LI_F16) return li::fail(LI_EUNSUPPORTED, "li_add_rms_norm: bf16 or f16 rows only");
  if (rows < 0 || hidden <= 0 || hidden % 8 != 0 || hidden > 8 * kNormThreads * kNormPer)
    return li::fail(LI_EINVAL, "li_add_rms_norm: hidden size %d must be a multiple of 8 up to %d", hidden,
                    8 * kNormThreads * kNormPer);
  if (rows == 0) return LI_OK;
  if (rows > 0x7fffffffLL) return li::fail(LI_EINVAL, "li_add_rms_norm: too many rows");
  if (!h || !weight || !out || !rows_ok(h, h_stride, 2) || !rows_ok(out, out_stride, 2) || !li::aligned16(weight) ||
      (delta && !rows_ok(delta, delta_stride, 2)))
    return li::fail(LI_EINVAL, "li_add_rms_norm: rows must be 16-byte aligned with the last axis contiguous");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 g((unsigned)rows), b(kNormThreads);
  if (dtype == LI_BF16)
    hipLaunchKernelGGL(add_rms_norm<li_bf16>, g, b, 0, s, static_cast<li_bf16*>(h), static_cast<const li_bf16*>(delta),
                       static_cast<const li_bf16*>(weight), static_cast<li_bf16*>(out), hidden, h_stride,
                       delta_stride, out_stride, eps);
  else
    hipLaunchKernelGGL(add_rms_norm<li_f16>, g, b, 0, s, static_cast<li_f16*>(h), static_cast<const li_f16*>(delta),
                       static_cast<const li_f16*>(weight), static_cast<li_f16*>(out), hidden, h_stride, delta_stride,
                       out_stride, eps);
  return li::check_launch("li_add_rms_norm");
}

extern "C" int li_silu_mul(const void* gate_up, void* out, int64_t rows, int ffn, int64_t gate_up_stride,
                           int64_t out_stride, int dtype, void* stream) {
  li::clear_error();
  if (dtype != LI_BF16 && dtype != LI_F16) return li::fail(LI_EUNSUPPORTED, "li_silu_mul: bf16 or f16 rows only");
  if (rows < 0 || ffn <= 0 || ffn % 8 != 0) return li::fail(LI_EINVAL, "li_silu_mul: ffn %d must be a multiple of 8", ffn);
  if (rows == 0) return LI_OK;
  if (!gate_up || !out || !rows_ok(gate_up, gate_up_stride, 2) || !rows_ok(out, out_stride, 2) || (ffn * 2) % 16)
    return li::fail(LI_EINVAL, "li_silu_mul: rows must be 16-byte aligned with the last axis contiguous");
  const int64_t work = rows * (ffn / 8);
  const int64_t blocks = std::min<int64_t>(li::cdiv64(work, 256), 65536);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == LI_BF16)
    hipLaunchKernelGGL(silu_mul<li_bf16>, dim3((unsigned)blocks), dim3(256), 0, s,
                       static_cast<const li_bf16*>(gate_up), static_cast<li_bf16*>(out), rows, ffn, gate_up_stride,
                       out_stride);
  else
    hipLaunchKernelGGL(silu_mul<li_f16>, dim3((unsigned)blocks), dim3(256), 0, s, static_cast<const li_f16*>(gate_up),
                       static_cast<li_f16*>(out), rows, ffn, gate_up_stride, out_stride);
  return li::check_launch("li_silu_mul");
}
