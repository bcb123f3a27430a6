// MFMA helpers for gfx950 (CDNA4), 16-bit inputs, fp32 accumulation.
//
// Register layouts (measured on gfx950 with one-hot operands; every chunk-scan
// parity test depends on them):
//   v_mfma_f32_32x32x16_{bf16,f16}: lane l, g = l/32
//     A (8 elems): row l%32, k-slot (g, i)       B (8 elems): col l%32, k-slot (g, i)
//     D (16 f32):  D[8*(r/4) + 4*g + r%4][l%32]
//   v_mfma_f32_16x16x32_{bf16,f16}: lane l, g = l/16
//     A: row l%16, k-slot (g, i)                 B: col l%16, k-slot (g, i)
//     D (4 f32):   D[4*g + r][l%16]
// The k-slot -> k mapping is free as long as A and B agree; the kernels use it to
// feed an accumulator straight back in as a B operand (see sssd_chunk.hip).
#pragma once

#include <hip/hip_runtime.h>

namespace vmi {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

template <typename E> struct mfma_t;

template <> struct mfma_t<__bf16> {
  typedef __bf16 elem;
  typedef bf16x4 v4;
  typedef bf16x8 v8;
  static __device__ __forceinline__ f32x16 mma32(v8 a, v8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x4 mma16(v8 a, v8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};

template <> struct mfma_t<_Float16> {
  typedef _Float16 elem;
  typedef f16x4 v4;
  typedef f16x8 v8;
  static __device__ __forceinline__ f32x16 mma32(v8 a, v8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x4 mma16(v8 a, v8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};

// Concatenate two 4-element halves into one 8-element operand.
template <typename V4, typename V8>
__device__ __forceinline__ V8 cat8(V4 lo, V4 hi) {
  return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}

// fp32 -> (hi, lo) split so that hi*b + lo*b carries ~16 mantissa bits of x into an
// MFMA product with a 16-bit operand b.
//   fp16: hi = round(x), lo = round(x - hi).
//   bf16: the same, with float(hi) rebuilt from the packed pair by shifts instead of a
//         second conversion (3 VALU per value).
template <typename E>
__device__ __forceinline__ void split8(const float* x, typename mfma_t<E>::v8& hi,
                                       typename mfma_t<E>::v8& lo) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const E h = static_cast<E>(x[i]);
    hi[i] = h;
    lo[i] = static_cast<E>(x[i] - static_cast<float>(h));
  }
}

template <>
__device__ __forceinline__ void split8<__bf16>(const float* x, bf16x8& hi, bf16x8& lo) {
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
#pragma unroll
  for (int i = 0; i < 8; ++i) hi[i] = static_cast<__bf16>(x[i]);  // v_cvt_pk_bf16_f32 pairs
  const u32x4 hp = __builtin_bit_cast(u32x4, hi);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    lo[2 * i] = static_cast<__bf16>(x[2 * i] - __uint_as_float(hp[i] << 16));
    lo[2 * i + 1] = static_cast<__bf16>(x[2 * i + 1] - __uint_as_float(hp[i] & 0xffff0000u));
  }
}

template <typename E>
__device__ __forceinline__ typename mfma_t<E>::v8 round8(const float* x) {
  typename mfma_t<E>::v8 r;
#pragma unroll
  for (int i = 0; i < 8; ++i) r[i] = static_cast<E>(x[i]);
  return r;
}

}  // namespace vmi
