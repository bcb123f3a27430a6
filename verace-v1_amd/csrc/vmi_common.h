// Device helpers shared by the gfx950 kernels of libverace_sssd.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "verace_sssd.h"

namespace vmi {

// ---------------------------------------------------------------------------
// Element types.  bf16 is carried as raw uint16_t bits, fp16 as _Float16.
// ---------------------------------------------------------------------------
struct bf16_t {
  uint16_t bits;
};
typedef _Float16 f16_t;

__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

// Round-to-nearest-even float -> bf16 (NaN kept quiet).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

template <typename T> struct io;
template <> struct io<float> {
  static __device__ __forceinline__ float to_f32(float x) { return x; }
  static __device__ __forceinline__ float load(const float* p, int64_t i) { return p[i]; }
  static __device__ __forceinline__ void store(float* p, int64_t i, float x) { p[i] = x; }
};
template <> struct io<bf16_t> {
  static __device__ __forceinline__ float to_f32(bf16_t x) { return bf16_to_f32(x.bits); }
  static __device__ __forceinline__ float load(const bf16_t* p, int64_t i) {
    return bf16_to_f32(p[i].bits);
  }
  static __device__ __forceinline__ void store(bf16_t* p, int64_t i, float x) {
    p[i].bits = f32_to_bf16(x);
  }
};
template <> struct io<f16_t> {
  static __device__ __forceinline__ float to_f32(f16_t x) { return static_cast<float>(x); }
  static __device__ __forceinline__ float load(const f16_t* p, int64_t i) {
    return static_cast<float>(p[i]);
  }
  static __device__ __forceinline__ void store(f16_t* p, int64_t i, float x) {
    p[i] = static_cast<f16_t>(x);
  }
};

// delta is read one scalar per (token, head); its dtype is a runtime code.
__device__ __forceinline__ float load_scalar(const void* p, int dtype, int64_t i) {
  if (dtype == VMI_F32) return static_cast<const float*>(p)[i];
  if (dtype == VMI_BF16) return bf16_to_f32(static_cast<const uint16_t*>(p)[i]);
  return static_cast<float>(static_cast<const f16_t*>(p)[i]);
}

// ---------------------------------------------------------------------------
// Closed-form Cayley coefficients for one token.
//   h = delta/2,  m^2 = h^2 (|k|^2 |v|^2 - (k.v)^2),  c = 2 / (1 + m^2)
// Applied to row vectors a = k^T Psi, b = v^T Psi:
//   alpha = c(-h b + h^2 (kv b - vv a)),  beta = c(h a + h^2 (kv a - kk b))
// so that R Psi = Psi + k alpha + v beta.  The coefficients below are the
// 2x2 matrix M = [[m00, m01], [m10, m11]] with alpha = m00 a + m01 b,
// beta = m10 a + m11 b.
// ---------------------------------------------------------------------------
struct cayley2 {
  float m00, m01, m10, m11;
};

__device__ __forceinline__ cayley2 cayley_coeffs(float delta, float kk, float vv, float kv) {
  const float h = 0.5f * delta;
  const float h2 = h * h;
  const float gram_det = fmaxf(kk * vv - kv * kv, 0.0f);
  const float c = 2.0f / (1.0f + h2 * gram_det);
  cayley2 m;
  m.m00 = -c * h2 * vv;
  m.m01 = c * (h2 * kv - h);
  m.m10 = c * (h2 * kv + h);
  m.m11 = -c * h2 * kk;
  return m;
}

__device__ __forceinline__ bool finite4(float a, float b, float c, float d) {
  return __builtin_isfinite(a) && __builtin_isfinite(b) && __builtin_isfinite(c) &&
         __builtin_isfinite(d);
}

// The reference's non-finite guard (sssd_attention.py:45-71): a token whose Cayley factor
// is not finite -- a NaN or Inf in k, v or delta (the Gram entries are then not finite
// either), or a closed form that overflows -- is replaced by R = I.  For such a token this
// returns M = 0 and ok = false; the caller must also treat the token's k and v (its U rows)
// as zero, because NaN * 0 is NaN: a zero M alone would not keep the state finite.
__device__ __forceinline__ cayley2 cayley_guarded(float delta, float kk, float vv, float kv,
                                                  bool& ok) {
  cayley2 m = cayley_coeffs(delta, kk, vv, kv);
  ok = finite4(delta, kk, vv, kv) && finite4(m.m00, m.m01, m.m10, m.m11);
  if (!ok) m = cayley2{0.f, 0.f, 0.f, 0.f};
  return m;
}

// Accuracy envelope of the f16-operand chunk scans.  A token rotates the state by the angle
// 2 atan(m) in the (k, v) plane, m = (delta / 2) |k ^ v| (m^2 as in cayley_coeffs).  The
// chunk scans round the state, W and Z to f16 once per 16-token chunk; the error that adds
// grows with the rotation per chunk.  Measured on gfx950 against the fp64 closed form
// (bf16 inputs, T = 65536): m = 0.05 gives 1.1e-3 state error and 1e-5 norm drift, m = 0.2
// 4.5e-3 and 2.3e-5, m = 2 2.0e-2 and 2.0e-4 (outside the 2e-2 / 1e-4 bars).  A sequence with
// any token above m = 0.25 is therefore recomputed by the fp32 token-sequential kernel.  The
// model's own inputs (unit k, v and delta = 0.1 sigmoid(.) <= 0.1) stay below m = 0.05.
constexpr float kChunkMaxRotation2 = 0.0625f;  // m^2 at m = 0.25
__device__ __forceinline__ bool rotation_outside_chunk_envelope(float delta, float kk, float vv,
                                                                float kv) {
  const float h = 0.5f * delta;
  return h * h * fmaxf(kk * vv - kv * kv, 0.0f) > kChunkMaxRotation2;  // false for NaN
}

// Element of k or v as it enters a product: non-finite values read as 0 (used where a
// kernel stages a token whose M is already 0 from cayley_guarded; see above).
__device__ __forceinline__ float finite_or_zero(float x) { return __builtin_isfinite(x) ? x : 0.f; }

// Streaming (nontemporal) 16-byte accesses for decode states: a step reads each state once
// and writes it once, and nothing touches it again until the next token (after every other
// layer's states), so these accesses should not displace cached data.  Measured on the
// decode pattern (12 rotating 33.5 MB states updated in place): 12.0 us per pass with
// nontemporal accesses against 14.0 us with ordinary ones.
typedef float f32x4_nt __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float4 ld_stream4(const float* p) {
  const f32x4_nt v = __builtin_nontemporal_load(reinterpret_cast<const f32x4_nt*>(p));
  return make_float4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ void st_stream4(float* p, float4 x) {
  const f32x4_nt v = {x.x, x.y, x.z, x.w};
  __builtin_nontemporal_store(v, reinterpret_cast<f32x4_nt*>(p));
}

}  // namespace vmi
