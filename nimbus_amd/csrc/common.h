// Shared device helpers for the paged-attention kernels (gfx950 / CDNA4).
//
// Element types are carried as raw 16-bit storage (uint16_t) and converted
// explicitly, so one kernel template serves fp16 and bf16. Matrix products
// use the CDNA4 MFMA builtins with fp32 accumulation:
//   16x16x32 (A: 8 elements per lane, k-group = lane / 16)
//   16x16x16 (A: 4 elements per lane, k-group = lane / 16)
// Output (C/D) layout of both 16x16 shapes: lane l holds column l % 16 and
// rows 4 * (l / 16) + r for r = 0..3 (one fp32 per VGPR).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace nimbus {

enum DType : int { kFloat16 = 0, kBFloat16 = 1 };

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Buffer resources (raw, unswizzled access with a 32-bit data format in
// descriptor word 3) and the cache-policy bit of buffer loads and stores
// that makes them agent-scope (sc1): they bypass the non-coherent L2 of the
// issuing XCD, so data one XCD writes this way is seen by another reading
// it this way once the write has completed.
constexpr int kBufferFlags = 0x00020000;
constexpr int kSc1 = 16;

// ---------------------------------------------------------------- conversions

__device__ __forceinline__ float bf16_to_f32(uint16_t x) {
  return __uint_as_float(static_cast<uint32_t>(x) << 16);
}

// Round-to-nearest-even fp32 -> bf16 (NaN kept quiet).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

__device__ __forceinline__ float f16_to_f32(uint16_t x) {
  _Float16 h;
  __builtin_memcpy(&h, &x, 2);
  return static_cast<float>(h);
}

__device__ __forceinline__ uint16_t f32_to_f16(float f) {
  _Float16 h = static_cast<_Float16>(f);
  uint16_t x;
  __builtin_memcpy(&x, &h, 2);
  return x;
}

// The prefill kernel's P.V product runs in fp16 whatever the cache dtype:
// P lies in [0, 256], where fp16 keeps 3 more mantissa bits than bf16
// (rounding P to bf16 alone costs ~8e-3 at |o| ~ 0.5, beyond the output
// tolerance), and a finite bf16 V element converts to fp16 exactly when
// 2^-17 <= |v| <= 65504 (fp16 subnormals keep bf16's 8 significant bits
// down to 2^-17). Smaller magnitudes lose bits, with an absolute error below
// 2^-24 (values below 2^-24 flush to zero), so relative accuracy falls for
// very small V. The
// conversion rounds toward zero, so larger finite |v| saturate to +-65504
// rather than becoming inf, and one outlier cannot turn masked-out products
// (0 * inf) into NaN for other rows. (Decode, which
// cannot afford a per-element conversion of V, keeps V in bf16 and splits P
// into two bf16 terms instead.)

// Two fp32 values packed into one dword of fp16, rounded toward zero
// (v_cvt_pkrtz_f16_f32: finite values beyond the fp16 range give +-65504).
__device__ __forceinline__ uint32_t pack_f16_rtz(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(lo, hi));
}

// Two 16-bit V elements packed in a dword, converted together: each half to
// fp32 (a shift or a mask), then both packed by one v_cvt_pkrtz, which is
// exact for bf16 values in the fp16 normal range and saturates finite values
// beyond it.
template <int DT>
__device__ __forceinline__ uint32_t v_to_f16_pair(uint32_t w);

template <>
__device__ __forceinline__ uint32_t v_to_f16_pair<kFloat16>(uint32_t w) {
  return w;
}

template <>
__device__ __forceinline__ uint32_t v_to_f16_pair<kBFloat16>(uint32_t w) {
  return pack_f16_rtz(__uint_as_float(w << 16), __uint_as_float(w & 0xffff0000u));
}

template <int DT> struct Elem;

template <> struct Elem<kFloat16> {
  __device__ static __forceinline__ float to_f32(uint16_t x) { return f16_to_f32(x); }
  __device__ static __forceinline__ uint16_t from_f32(float f) { return f32_to_f16(f); }
};

template <> struct Elem<kBFloat16> {
  __device__ static __forceinline__ float to_f32(uint16_t x) { return bf16_to_f32(x); }
  __device__ static __forceinline__ uint16_t from_f32(float f) { return f32_to_bf16(f); }
};

// ---------------------------------------------------------------- MFMA

// 16x16x32: a, b carry 8 16-bit elements each (4 dwords).
template <int DT>
__device__ __forceinline__ f32x4 mfma_16x16x32(u32x4 a, u32x4 b, f32x4 c);

template <>
__device__ __forceinline__ f32x4 mfma_16x16x32<kFloat16>(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                0, 0);
}

template <>
__device__ __forceinline__ f32x4 mfma_16x16x32<kBFloat16>(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                 0, 0, 0);
}

// 16x16x16: a, b carry 4 16-bit elements each (2 dwords).
template <int DT>
__device__ __forceinline__ f32x4 mfma_16x16x16(u32x2 a, u32x2 b, f32x4 c);

template <>
__device__ __forceinline__ f32x4 mfma_16x16x16<kFloat16>(u32x2 a, u32x2 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4, a), __builtin_bit_cast(f16x4, b), c, 0, 0,
                                               0);
}

template <>
__device__ __forceinline__ f32x4 mfma_16x16x16<kBFloat16>(u32x2 a, u32x2 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4, a), __builtin_bit_cast(s16x4, b), c,
                                                   0, 0, 0);
}

// ---------------------------------------------------------------- transposed LDS reads

// ds_read_b64_tr_b16 (gfx950). Within each 16-lane group, lane j supplies
// the address of 4 consecutive 16-bit elements A_j[0..3]; lane i of the
// group receives out[k] = A_{4k + i/4}[i % 4], k = 0..3. So if lane j of
// group grp points at M[4 grp + j/4][c0 + 4 (j%4)] of a row-major 16-bit
// matrix M, lane (i, grp) receives M[4 grp + k][c0 + i], k = 0..3: the
// A operand of a 16x16x16 MFMA holding M^T (rows c0..c0+15, k = rows of M).
__device__ __forceinline__ u32x2 lds_read_tr16(const uint16_t* p) {
  typedef short s16x4_t __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) s16x4_t lds_s16x4;
  const s16x4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(const_cast<uint16_t*>(p)));
  return __builtin_bit_cast(u32x2, v);
}

// 2^x with the bare v_exp_f32 (no denormal range reduction): softmax weights
// below 2^-126 may flush to zero.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// ---------------------------------------------------------------- wave reductions

// Butterfly over the four 16-lane groups of a wave64 (lanes l, l^16, l^32, l^48).
__device__ __forceinline__ float max_across_groups(float x) {
  x = fmaxf(x, __shfl_xor(x, 16, 64));
  x = fmaxf(x, __shfl_xor(x, 32, 64));
  return x;
}

__device__ __forceinline__ float sum_across_groups(float x) {
  x += __shfl_xor(x, 16, 64);
  x += __shfl_xor(x, 32, 64);
  return x;
}

__device__ __forceinline__ uint32_t pack2(uint16_t lo, uint16_t hi) {
  return static_cast<uint32_t>(lo) | (static_cast<uint32_t>(hi) << 16);
}

}  // namespace nimbus
