// Building blocks shared by the MFMA attention kernels: the 16x16x32 MFMA
// for bf16 / fp16, the 32-key LDS tile layout filled by direct-to-LDS loads,
// and explicit vector-memory waits.
#pragma once

#include "li_common.h"

namespace li {

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

// Key of the tile whose weight lane group g holds in B-operand slot e (the
// order the S^T blocks deliver scores in).
__device__ __forceinline__ int kappa(int g, int e) { return (e < 4 ? 4 * g + e : 16 + 4 * g + (e - 4)); }

// Keys whose slots are staged in LDS at a time. A partition chosen by the
// policy is at most this long, so it is one chunk; a pinned split count can
// make longer partitions, which take several.
constexpr int kSlotChunk = 1024;

// LDS tile layout. A tile is 32 keys; K rows then V rows, D / 8 chunks of 16
// bytes per row. A load instruction writes lane L's 16 bytes at 16 L, so with
// CH = D / 8 chunks per row one instruction fills 64 / CH rows; instruction i,
// row-in-instruction rr holds key rr * (CH / 2) + i (so each lane's keys are
// consecutive), and chunk c of key k sits in slot c ^ (k % CH) of its row, so
// 16 lanes reading the same chunk of 16 keys hit 16 distinct bank groups.
template <int D>
struct TileLayout {
  static constexpr int kCh = D / 8;             // 16-byte chunks per row
  static constexpr int kRowsPerInst = 64 / kCh;  // rows one load instruction fills
  static constexpr int kInsts = 32 / kRowsPerInst;
  static constexpr int kRowBytes = D * 2;
  static constexpr int kTileBytes = 2 * 32 * kRowBytes;  // K then V
  // Key k + 16 sits this many bytes below key k (same swizzle: kCh divides 16).
  static constexpr int kRow16 = (16 / kInsts) * kRowBytes;
  __device__ static int row_of(int key) { return kRowsPerInst * (key % kInsts) + key / kInsts; }
  __device__ static int kswizzle(int key) { return key % kCh; }
  __device__ static int offset(int key, int chunk) {  // byte offset within the K half
    return row_of(key) * kRowBytes + 16 * (chunk ^ (key % kCh));
  }
  // V rows use their own chunk swizzle: chunk c of key k sits in slot
  // c ^ vswizzle(k). A transposing V^T read (li_read_vt's addressing) has
  // each group of 16 lanes read chunks 2 blk and 2 blk + 1 of four
  // consecutive keys k (and 32 lanes eight keys); with vswizzle(k) =
  // 2 (k mod CH / 2) those land in slots 2 (blk ^ (k mod CH / 2)) + {0, 1},
  // all distinct, so the reads hit distinct banks (the K swizzle would map
  // pairs of them onto one slot). Keys k and k + 16 share a swizzle.
  __device__ static int vswizzle(int key) { return 2 * (key % (kCh / 2)); }
  __device__ static int voffset(int key, int chunk) {  // byte offset within the V half
    return row_of(key) * kRowBytes + 16 * (chunk ^ vswizzle(key));
  }
};

// The 32-key tile of an fp8 (e4m3) pool at head_dim 128: rows of 128 bytes
// (8 chunks of 16), K then V, filled by the same direct-to-LDS loads
// (instruction i, row-in-instruction rr holds key rr * 4 + i). Operands are
// read 8 bytes at a time: the K operand of key n at step j is chunk
// 2j + g / 2, half g % 2 (ds_read_b64); the V^T operand of 16 dims comes
// from one 8-bit transposing read (ds_read_b64_tr_b8), which gives lane
// 8h + t of a 16-lane group byte t of the reads of lanes h, h + 2, ...,
// h + 14, so lane s reads half s % 2 of the dims' chunk of key
// kappa(g, s / 2) and lane m receives dim 16 blk + m of keys kappa(g, 0..7).
// Rows alternate bank halves (128 bytes per row, 256 bytes per bank row), so
// each read's 16 lanes need 8 distinct slots among keys of one row parity:
// the K swizzle makes keys n and n + 8 differ (16 keys of one chunk), the V
// swizzle keys k and k + 16 (kappa(g, .) covers k..k+3 and k+16..k+19).
struct F8Tile {
  static constexpr int kCh = 8;
  static constexpr int kRowsPerInst = 8;
  static constexpr int kInsts = 4;
  static constexpr int kRowBytes = 128;
  static constexpr int kTileBytes = 2 * 32 * kRowBytes;  // K then V
  static constexpr int kRow16 = (16 / kInsts) * kRowBytes;
  __device__ static int row_of(int key) { return kRowsPerInst * (key % kInsts) + key / kInsts; }
  __device__ static int kswizzle(int key) { return (key & 3) | (((key >> 3) & 1) << 2); }
  __device__ static int vswizzle(int key) { return (key & 3) | (((key >> 4) & 1) << 2); }
  __device__ static int offset(int key, int chunk) { return row_of(key) * kRowBytes + 16 * (chunk ^ kswizzle(key)); }
  __device__ static int voffset(int key, int chunk) { return row_of(key) * kRowBytes + 16 * (chunk ^ vswizzle(key)); }
};

// Eight e4m3 values (bytes 0..7 of lo, hi) as an MFMA operand of bf16 or
// fp16: every e4m3 value is exact in both. The conversions run with scale 1;
// a pool's scales are applied to the scores and the outputs instead.
template <typename Frag>
__device__ __forceinline__ Frag f8x8_to_frag(uint32_t lo, uint32_t hi) {
  u32x4_t w;
  if constexpr (__is_same(Frag, bf16x8_t)) {
    w[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 1.0f, false));
    w[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 1.0f, true));
    w[2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 1.0f, false));
    w[3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 1.0f, true));
  } else {
    w[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(lo, 1.0f, false));
    w[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(lo, 1.0f, true));
    w[2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(hi, 1.0f, false));
    w[3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(hi, 1.0f, true));
  }
  return __builtin_bit_cast(Frag, w);
}

// The K operand of an fp8 tile: 8 bytes at LDS byte address `addr`.
template <typename Frag>
__device__ __forceinline__ Frag lds_read_f8_frag(uint32_t addr) {
  typedef uint32_t u2 __attribute__((ext_vector_type(2)));
  const u2 v = *(const __attribute__((address_space(3))) u2*)(uintptr_t)addr;
  return f8x8_to_frag<Frag>(v[0], v[1]);
}

// The V^T operand of an fp8 tile: one 8-bit transposing read at `addr`.
template <typename Frag>
__device__ __forceinline__ Frag lds_read_f8_vt(uint32_t addr) {
  typedef int v2i __attribute__((ext_vector_type(2)));
  const v2i v = __builtin_amdgcn_ds_read_tr8_b64_v2i32((__attribute__((address_space(3))) v2i*)(uintptr_t)addr);
  return f8x8_to_frag<Frag>((uint32_t)v[0], (uint32_t)v[1]);
}

// One direct-to-LDS load: every lane's 16 bytes at `g` land at lds + 16 * lane.
//
// Written as inline assembly on purpose: the compiler models the builtin's
// LDS write conservatively and waits for every such load to land before any
// LDS read, which would serialise the two stages. Here the kernel counts the
// loads itself (li_wait_vm below) and the "memory" clobbers keep every other
// memory access in program order around them.
// kStream: the rows are read once (non-temporal hint); otherwise they stay
// in L2 for the other work-groups that read them.
template <bool kStream = true>
__device__ __forceinline__ void dma16(const void* g, uint32_t lds) {
  uint32_t saved;
  if constexpr (kStream) {
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %1\n\t"
        "global_load_lds_dwordx4 %2, off nt\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "s"(__builtin_amdgcn_readfirstlane(lds)), "v"(g)
        : "memory");
  } else {
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %1\n\t"
        "global_load_lds_dwordx4 %2, off\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "s"(__builtin_amdgcn_readfirstlane(lds)), "v"(g)
        : "memory");
  }
}

// A work-group barrier that orders LDS only: this wave's LDS operations are
// complete when it arrives, and nothing waits for its global loads or
// stores (__syncthreads' release fence would wait for every one of them).
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" : : : "memory");
}

// Waits until at most N vector-memory operations of this wave are in flight.
template <int N>
__device__ __forceinline__ void li_wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" : : "n"(N) : "memory");
}

// Max / sum over the four lanes n, n + 16, n + 32, n + 48 (the lane groups
// that hold one MFMA column), every lane getting the result. Two permlane
// swaps (gfx950) instead of LDS-crossbar shuffles: the rows of 16 lanes are
// exchanged in registers, with no LDS round trip and no index arithmetic.
__device__ __forceinline__ float li_group_max(float x) {
  const uint32_t u = __float_as_uint(x);
  const auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  const float y = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const uint32_t v = __float_as_uint(y);
  const auto b = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float li_group_sum(float x) {
  const uint32_t u = __float_as_uint(x);
  const auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  const float y = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const uint32_t v = __float_as_uint(y);
  const auto b = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// 64-bit address of element `row * row_elems` of `base` in one multiply-add
// (row and row stride both fit 32 bits).
template <typename T>
__device__ __forceinline__ const T* row_ptr(const T* base, uint32_t row, uint32_t row_bytes) {
  return reinterpret_cast<const T*>(reinterpret_cast<uintptr_t>(base) + (uint64_t)row * row_bytes);
}

// An MFMA operand of all ones (bf16 / fp16 1.0): times P^T it gives every
// output row the column sums of P^T, i.e. each query row's sum of weights.
template <typename Frag>
__device__ __forceinline__ Frag li_ones() {
  typedef __attribute__((__vector_size__(8 * sizeof(uint16_t)))) uint16_t u16x8;
  // 0x3f80 is 1.0 in bf16; 0x3c00 is 1.0 in fp16.
  constexpr uint16_t one = sizeof(Frag) == 16 && __is_same(Frag, bf16x8_t) ? 0x3f80 : 0x3c00;
  const u16x8 v = {one, one, one, one, one, one, one, one};
  return __builtin_bit_cast(Frag, v);
}

// The V^T operand of O^T += V^T P^T for the 16 dims 16 blk .. 16 blk + 15,
// read from a 32-key V tile in LDS (layout L) with two transposing LDS reads
// (ds_read_b64_tr_b16, gfx950). Within a group of 16 lanes such a read gives
// lane 4a + t the element t of the 8-byte reads of lanes a, a + 4, a + 8,
// a + 12. So lane (s, g) reads dims 16 blk + 4 (s % 4) .. + 3 of key
// 4g + s / 4 (then of key 16 + 4g + s / 4), and lane (m, g) receives dim
// 16 blk + m of keys kappa(g, 0..7): its A operand, row m = that dim, with
// the keys in the order the S^T blocks deliver the weights.
template <typename L, typename Frag>
__device__ __forceinline__ Frag li_read_vt(const char* vtile, int blk, int lane) {
  typedef short v4s __attribute__((ext_vector_type(4)));
  const int s = lane & 15, g = lane >> 4;
  const int a = s & 3, j = s >> 2;
  const int chunk = 2 * blk + (a >> 1);
  const int byte = 8 * (a & 1);
  const char* lo = vtile + L::voffset(4 * g + j, chunk) + byte;
  const char* hi = vtile + L::voffset(16 + 4 * g + j, chunk) + byte;
  const v4s x = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s*)(lo));
  const v4s y = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s*)(hi));
  const short __attribute__((ext_vector_type(8))) xy = {x[0], x[1], x[2], x[3], y[0], y[1], y[2], y[3]};
  return __builtin_bit_cast(Frag, xy);
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)(p);
}

// 16-byte LDS read at LDS byte address `addr` (an address plus a constant
// folds into the instruction's immediate offset).
template <typename Frag>
__device__ __forceinline__ Frag lds_read_frag(uint32_t addr) {
  return *(const __attribute__((address_space(3))) Frag*)(uintptr_t)addr;
}

// li_read_vt from precomputed LDS byte addresses of its two transposing reads.
template <typename Frag>
__device__ __forceinline__ Frag lds_read_vt(uint32_t lo, uint32_t hi) {
  typedef short v4s __attribute__((ext_vector_type(4)));
  const v4s x = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s*)(uintptr_t)lo);
  const v4s y = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s*)(uintptr_t)hi);
  const short __attribute__((ext_vector_type(8))) xy = {x[0], x[1], x[2], x[3], y[0], y[1], y[2], y[3]};
  return __builtin_bit_cast(Frag, xy);
}

constexpr float kLog2eMfma = 1.4426950408889634f;

// A running softmax maximum is only raised when a tile's maximum exceeds it
// by more than this (in log2 units); until then the weights exp2(s - m) may
// reach 2^kLazyRescale, which fp32 sums and bf16 / fp16 weights hold without
// loss of relative precision. Most tiles then skip rescaling the
// accumulator.
constexpr float kLazyRescale = 8.0f;

// acc + the sum of the eight 16-bit weights of an MFMA operand, in fp32:
// four two-element dot products with (1, 1) (v_dot2_f32_bf16 / _f16).
template <typename T, typename Frag>
__device__ __forceinline__ float li_sum_weights(Frag f, float acc) {
  if constexpr (__is_same(T, li_bf16)) {
    typedef __bf16 b2 __attribute__((ext_vector_type(2)));
    const b2 one = {(__bf16)1.0f, (__bf16)1.0f};
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const b2 x = {f[2 * u], f[2 * u + 1]};
      acc = __builtin_amdgcn_fdot2_f32_bf16(x, one, acc, false);
    }
  } else {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    const h2 one = {(_Float16)1.0f, (_Float16)1.0f};
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const h2 x = {f[2 * u], f[2 * u + 1]};
      acc = __builtin_amdgcn_fdot2(x, one, acc, false);
    }
  }
  return acc;
}

}  // namespace li
