// Shared pieces of the CHAM scan kernels (cham_scan.hip for h <= 128, cham_wide.hip for
// larger h): the closed-form Cayley coefficients of one token, cross-lane sums and raw
// loads.
#pragma once
#include "vmi_common.h"
#include "vmi_lanes.h"

namespace vmi {
namespace cham {

using vmi::dpp_f32;
using vmi::half_pair_sum;
using vmi::row16_sum;
using vmi::row_pair_sum;

struct NCoef {
  float n11r, n11i, n12r, n12i, n22r, n22i;
};

__device__ __forceinline__ NCoef cayley_n(float gamma, float kk, float vv, float kv) {
  const float g = 0.5f * gamma;
  const float g2 = g * g;
  const float dr = 1.f + g2 * (kk * vv - kv * kv);
  const float di = -2.f * g * kv;
  // 2 / |det|^2 (|det| >= 1), so 2/det = p conj(det); v_rcp_f32 (1 ulp) is plenty
  const float p = 2.f * __builtin_amdgcn_rcpf(dr * dr + di * di);
  NCoef n;
  // (x + i y) * p (dr - i di)
  auto mul = [&](float x, float y, float& re, float& im) {
    re = p * (x * dr + y * di);
    im = p * (y * dr - x * di);
  };
  mul(-g2 * vv, 0.f, n.n11r, n.n11i);
  mul(g2 * kv, g, n.n12r, n.n12i);
  mul(-g2 * kk, 0.f, n.n22r, n.n22i);
  return n;
}

// The reference's non-finite guard (cham_memory.py:68-95): a token whose Cayley factor is
// not finite (NaN or Inf in k, v or gamma, or an overflowing closed form) is replaced by
// U = I.  Returns N = 0 and ok = false for such a token; the caller must also treat its k,
// v as zero, since NaN * 0 is NaN.
__device__ __forceinline__ NCoef cayley_n_guarded(float gamma, float kk, float vv, float kv,
                                                  bool& ok) {
  NCoef n = cayley_n(gamma, kk, vv, kv);
  ok = finite4(gamma, kk, vv, kv) && finite4(n.n11r, n.n11i, n.n12r, n.n12i) &&
       __builtin_isfinite(n.n22r) && __builtin_isfinite(n.n22i);
  if (!ok) n = NCoef{0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  return n;
}

template <typename T> __device__ __forceinline__ float ld(const T* p, int64_t i) { return io<T>::load(p, i); }

// Raw 16/32-bit loads converted to fp32 only where they are used: a conversion (or any
// use) right after a load makes the wave wait for it, which would serialise a batch of
// loads meant to be in flight together.
template <typename T> struct raw;
template <> struct raw<float> {
  typedef float type;
  static __device__ __forceinline__ float f32(float x) { return x; }
};
template <> struct raw<bf16_t> {
  typedef uint16_t type;
  static __device__ __forceinline__ float f32(uint16_t x) { return bf16_to_f32(x); }
};
template <> struct raw<f16_t> {
  typedef uint16_t type;
  static __device__ __forceinline__ float f32(uint16_t x) {
    return static_cast<float>(__builtin_bit_cast(f16_t, x));
  }
};
template <typename T>
__device__ __forceinline__ typename raw<T>::type ldraw(const T* p, int64_t i) {
  return reinterpret_cast<const typename raw<T>::type*>(p)[i];
}

// Fused projections (kernels fed the stacked projection x [W_q; W_k; W_v; W_gamma]^T instead of
// q, k, v, gamma; reference cham_memory.py:128-155): v = silu(v), and the normalised value of a
// k or v element as the carry's f16 operands hold it (the coefficient kernel forms the Gram
// entries from exactly these values, so every token's factor is unitary for the vectors the
// carry multiplies).  Non-finite values read as 0; their token is guarded as the identity.
__device__ __forceinline__ float silu_f(float x) { return x / (1.f + expf(-x)); }
__device__ __forceinline__ _Float16 fused_f16(float x, float scale) {
  const float y = x * scale;
  return __builtin_isfinite(y) ? static_cast<_Float16>(y) : static_cast<_Float16>(0.f);
}

}  // namespace cham
}  // namespace vmi
