// Chunked (WY) backward of the SSSD scan: the per-token reverse recursion of sssd_bwd.hip
// regrouped by chunks of C = 16 tokens, so every state-dependent product is a small GEMM
// on the fp32 MFMA (v_mfma_f32_16x16x4f32: exact fp32 products, fp32 accumulation).
//
// Per chunk (U = [k_1 v_1 .. k_C v_C] D x 32, T~ = (I - L)^-1 blockdiag(M) 32 x 32, the
// forward's chunk factor I + U T~ U^T, states Psi_s -> Psi_e, adjoints Lam_s <- Lam_e):
//   Psi_s = Psi_e + U T~^T U^T Psi_e            (the factor is orthogonal)
//   W = U^T Psi_s,  Z = T~ W,  X = mask o (Z Q),  dX = mask o (U^T dO)
//   dZ = U^T Lam_e + dX Q^T,   dT~ = dZ W^T,     dW = T~^T dZ
//   dQ = Z^T dX + Psi_s^T dO,  dU = Lam_e Z^T + dO X^T + Psi_s dW^T
//   Lam_s = Lam_e + dO Q^T + U dW
// (mask[rho][t] = token(rho) <= t).  Then, per chunk and without the state, dT~ through
// T~ = A B (A = (I - L)^-1, B = blockdiag(M), L_ti = M_t G_ti for i < t):
//   dA = dT~ B^T, dB = A^T dT~, dL = A^T dA A^T (strictly lower blocks),
//   dM_t = dB_tt + sum_i dL_ti G_ti^T,  dG_ti = M_t^T dL_ti,
// M_t(delta_t, kk, vv, kv) as in vmi::cayley_coeffs, dU += U (dG + dG^T).
//
// Launches:
//   bwdc_prep_kernel  (grid (nch, B H)): T~, A, G, M of every chunk -> workspace;
//   bwdc_cols_kernel  (grid (D/16, B H), 256 threads): 16 state columns of one sequence
//     through the chunks in reverse, Psi and Lam in LDS; dQ of its columns directly, the
//     column sums dT~ and dU as per-chunk partials;
//   bwdc_reduce_kernel (grid (nch, B H)): sums the partials, dT~ -> dM, dG -> dk, dv, ddelta.
#include <type_traits>

#include "vmi_common.h"
#include "vmi_dispatch.h"
#include "vmi_lanes.h"

namespace vmi {
namespace bwdc {

constexpr int C = 16;   // tokens per chunk
constexpr int R = 32;   // rank rows of a chunk (k, v per token)
constexpr int CB = 16;  // state columns per workgroup
constexpr int NT = 256;
// per-chunk record written by the prep kernel: T~, A = (I - L)^-1, G (R x R each), M blocks,
// then the bit mask of the chunk's tokens whose Cayley factor is not finite (the reference's
// non-finite guard, sssd_attention.py:45-71: such a token is the identity, its U rows count
// as zero and it gets no gradient) and 3 floats of padding (16-byte alignment)
constexpr int REC_BAD = 3 * R * R + 4 * C;
constexpr int REC = REC_BAD + 4;

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef short s16x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ short to_bf16(float x) {  // round to nearest even
  return __builtin_bit_cast(short, static_cast<__bf16>(x));
}
// two values as one word of bf16 (v_cvt_pk_bf16_f32: round to nearest even, the same bits as
// f32_to_bf16 for every non-NaN value, without its branch per element)
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  const bf16x2_t v = {static_cast<__bf16>(a), static_cast<__bf16>(b)};
  return __builtin_bit_cast(uint32_t, v);
}

enum { kStore = 0, kAdd = 1, kMaskStore = 2 };

// N consecutive elements of a row as raw 32-bit words (one 8- or 16-byte load, two for 8
// fp32), and element j of them as a float.  The row must be aligned to its byte size.
template <typename T, int N> struct RowRaw {
  static constexpr int W = N * static_cast<int>(sizeof(T)) / 4;
  uint32_t w[W];
};
template <typename T, int N>
__device__ __forceinline__ RowRaw<T, N> load_raw(const T* p) {
  RowRaw<T, N> r;
  constexpr int W = RowRaw<T, N>::W;
  static_assert(W == 2 || W % 4 == 0, "8-byte or whole 16-byte pieces");
  if constexpr (W == 2) {
    const uint2 x = *reinterpret_cast<const uint2*>(p);
    r.w[0] = x.x; r.w[1] = x.y;
  } else {
#pragma unroll
    for (int i = 0; i < W / 4; ++i) {
      const uint4 x = reinterpret_cast<const uint4*>(p)[i];
      r.w[4 * i] = x.x; r.w[4 * i + 1] = x.y; r.w[4 * i + 2] = x.z; r.w[4 * i + 3] = x.w;
    }
  }
  return r;
}
// N consecutive raw elements (8 or 16 bytes) read with the nontemporal hint: streamed once.
template <typename T, int N>
__device__ __forceinline__ RowRaw<T, N> load_raw_nt(const T* p) {
  RowRaw<T, N> r;
  constexpr int W = RowRaw<T, N>::W;
  static_assert(W == 2 || W % 4 == 0, "8-byte or whole 16-byte pieces");
  if constexpr (W == 2) {
    typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
    const u32x2 x = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(p));
    r.w[0] = x[0]; r.w[1] = x[1];
  } else {
#pragma unroll
    for (int i = 0; i < W / 4; ++i) {
      typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
      const u32x4 x = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p) + i);
      r.w[4 * i] = x[0]; r.w[4 * i + 1] = x[1]; r.w[4 * i + 2] = x[2]; r.w[4 * i + 3] = x[3];
    }
  }
  return r;
}
// One element as raw bits in word 0 (RowRaw<T, 2>, low half for 16-bit types).
template <typename T>
__device__ __forceinline__ RowRaw<T, 2> load_raw1(const T* p) {
  RowRaw<T, 2> r = {};
  if constexpr (sizeof(T) == 4) r.w[0] = *reinterpret_cast<const uint32_t*>(p);
  else r.w[0] = *reinterpret_cast<const uint16_t*>(p);
  return r;
}
template <typename T, int N>
__device__ __forceinline__ void store_row(T* p, const float (&x)[N]) {
  RowRaw<T, N> r;
  constexpr int W = RowRaw<T, N>::W;
  if constexpr (sizeof(T) == 4) {
#pragma unroll
    for (int j = 0; j < N; ++j) r.w[j] = __float_as_uint(x[j]);
  } else {
#pragma unroll
    for (int j = 0; j < N; j += 2) {
      uint32_t lo, hi;
      if constexpr (std::is_same<T, bf16_t>::value) {
        const uint32_t w = pack_bf16x2(x[j], x[j + 1]);
        lo = w & 0xffffu;
        hi = w >> 16;
      } else {
        lo = __builtin_bit_cast(uint16_t, static_cast<f16_t>(x[j]));
        hi = __builtin_bit_cast(uint16_t, static_cast<f16_t>(x[j + 1]));
      }
      r.w[j >> 1] = lo | (hi << 16);
    }
  }
  if constexpr (W == 2) {
    *reinterpret_cast<uint2*>(p) = make_uint2(r.w[0], r.w[1]);
  } else {
#pragma unroll
    for (int i = 0; i < W / 4; ++i)
      reinterpret_cast<uint4*>(p)[i] = make_uint4(r.w[4 * i], r.w[4 * i + 1], r.w[4 * i + 2], r.w[4 * i + 3]);
  }
}
template <typename T, int N>
__device__ __forceinline__ float raw_elem(const RowRaw<T, N>& r, int j) {
  if constexpr (sizeof(T) == 4) {
    return __uint_as_float(r.w[j]);
  } else {
    const uint16_t hbits = static_cast<uint16_t>(r.w[j >> 1] >> (16 * (j & 1)));
    if constexpr (std::is_same<T, bf16_t>::value) return bf16_to_f32(hbits);
    else return static_cast<float>(__builtin_bit_cast(f16_t, hbits));
  }
}

// N elements of a raw row as N / 2 words of bf16 pairs (round to nearest even; bf16 rows as they
// are), or zeros; stored with one 8- or 16-byte LDS write at p (aligned to that size).
template <typename T, int N>
__device__ __forceinline__ void put_bf16_row(uint16_t* p, const RowRaw<T, N>& r, bool keep) {
  static_assert(N == 4 || N == 8, "8 or 16 bytes");
  uint32_t w[N / 2];
#pragma unroll
  for (int j = 0; j < N / 2; ++j) {
    if constexpr (std::is_same<T, bf16_t>::value) w[j] = r.w[j];
    else w[j] = pack_bf16x2(raw_elem<T, N>(r, 2 * j), raw_elem<T, N>(r, 2 * j + 1));
    w[j] = keep ? w[j] : 0u;
  }
  if constexpr (N == 4) *reinterpret_cast<uint2*>(p) = make_uint2(w[0], w[1]);
  else *reinterpret_cast<uint4*>(p) = make_uint4(w[0], w[1], w[2], w[3]);
}

// Workgroup barrier that orders LDS accesses only: it waits for this wave's LDS operations,
// not for its global loads and stores (which __syncthreads() also waits for).  The columns
// kernel's global loads fill registers for the next chunk and its global stores are read by
// the next kernel, so neither needs ordering at the chunk's barriers.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xC07F);  // vmcnt(63) expcnt(7) lgkmcnt(0)
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// LDS row strides (64 banks of 4 B): with 19 and 37 every MFMA operand read is at most 2-way
// bank conflicted across the wave, in both orientations and for both lane layouts (fp32:
// lane (m, kq) reads element k0 + kq of row m, or row k0 + kq of column m; bf16: elements
// 4 kq + i).  17 and 33 are 4-way for the bf16 layout.
constexpr int L16 = 19;  // 16-wide matrices
constexpr int L32 = 37;  // 32-wide matrices

// Cm (M x N, row stride ldc) (=|+=) opA(A) opB(B), K the inner size, all in LDS.
// opA(m, k) = TA ? A[k lda + m] : A[m lda + k];  opB(k, n) = TB ? B[n ldb + k] : B[k ldb + n].
// 16 x 16 output tiles round robin over NW waves starting at W0 (independent products of
// one phase go to disjoint waves); v_mfma_f32_16x16x4f32 lane layout: A[m = lane % 16]
// [k = lane / 16], B[k = lane / 16][n = lane % 16], D[4 (lane / 16) + r][lane % 16].  Two
// accumulators over alternate k steps halve the dependent chain.  kMaskStore keeps the
// (row = rank row rho, col = token t) entries with rho / 2 <= t.
// LP: operands rounded to bf16 (v_mfma_f32_16x16x16_bf16, lane (m, kq) supplies
// A[m][4 kq .. 4 kq + 3] of a 16-wide k step), fp32 accumulation; for the bf16 / fp16
// inputs' per-chunk gradient products only.
// With B2, the B operand is B + B2 (same layout and stride), summed as it is read.
// ABF / BBF (LP only): that operand is read from a bf16 copy instead, Ab [M][ldab] / Bb [N][ldbb]
// with k contiguous (opA(m, k) = Ab[m ldab + k], opB(k, n) = Bb[n ldbb + k]): one 8-byte read per
// lane and k step, the same bits as rounding the fp32 operand (A / B and TA / TB unused).
// With Ct, the result is also written transposed in bf16 (Ct [N][ldct]), the operand layout of a
// later product that reads it transposed; with Cb, in bf16 as it is laid out (Cb [M][ldcb]).
template <int M, int N, int K, bool TA, bool TB, int MODE, int W0 = 0, int NW = 4,
          bool LP = false, bool SUMB = false, bool ABF = false, bool BBF = false>
__device__ __forceinline__ void lgemm(const float* A, int lda, const float* B, int ldb, float* Cm,
                                      int ldc, int wave, int lane, const float* B2 = nullptr,
                                      const uint16_t* Ab = nullptr, int ldab = 0,
                                      const uint16_t* Bb = nullptr, int ldbb = 0,
                                      uint16_t* Ct = nullptr, int ldct = 0,
                                      uint16_t* Cb = nullptr, int ldcb = 0) {
  static_assert(LP || !(ABF || BBF), "bf16 copies feed the bf16 products only");
  constexpr int TN = N / 16, NTILE = (M / 16) * TN;
  if (wave < W0 || wave >= W0 + NW) return;
  const int l16 = lane & 15, kq = lane >> 4;
  for (int tile = wave - W0; tile < NTILE; tile += NW) {
    const int tm = tile / TN, tn = tile % TN;
    const int am = 16 * tm + l16, bn = 16 * tn + l16;
    f32x4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
    if constexpr (LP) {
      static_assert(K % 16 == 0, "bf16 steps of 16");
#pragma unroll 4
      for (int k0 = 0; k0 < K; k0 += 16) {
        s16x4 a, b;
        if constexpr (ABF) {
          a = *reinterpret_cast<const s16x4*>(Ab + am * ldab + k0 + 4 * kq);
        } else {
          float af[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int k = k0 + 4 * kq + i;
            af[i] = TA ? A[k * lda + am] : A[am * lda + k];
          }
          // two elements per v_cvt_pk_bf16_f32
          a = __builtin_bit_cast(s16x4, make_uint2(pack_bf16x2(af[0], af[1]), pack_bf16x2(af[2], af[3])));
        }
        if constexpr (BBF) {
          b = *reinterpret_cast<const s16x4*>(Bb + bn * ldbb + k0 + 4 * kq);
        } else {
          float bf[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int k = k0 + 4 * kq + i;
            bf[i] = TB ? B[bn * ldb + k] : B[k * ldb + bn];
          }
          b = __builtin_bit_cast(s16x4, make_uint2(pack_bf16x2(bf[0], bf[1]), pack_bf16x2(bf[2], bf[3])));
        }
        if ((k0 >> 4) & 1) acc1 = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, acc1, 0, 0, 0);
        else acc0 = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, acc0, 0, 0, 0);
      }
    } else {
#pragma unroll 4
    for (int k0 = 0; k0 < K; k0 += 8) {
      const int k = k0 + kq;
      const float a0 = TA ? A[k * lda + am] : A[am * lda + k];
      float b0 = TB ? B[bn * ldb + k] : B[k * ldb + bn];
      if constexpr (SUMB) b0 += TB ? B2[bn * ldb + k] : B2[k * ldb + bn];
      acc0 = __builtin_amdgcn_mfma_f32_16x16x4f32(a0, b0, acc0, 0, 0, 0);
      if (k0 + 4 < K) {
        const int k1 = k + 4;
        const float a1 = TA ? A[k1 * lda + am] : A[am * lda + k1];
        float b1 = TB ? B[bn * ldb + k1] : B[k1 * ldb + bn];
        if constexpr (SUMB) b1 += TB ? B2[bn * ldb + k1] : B2[k1 * ldb + bn];
        acc1 = __builtin_amdgcn_mfma_f32_16x16x4f32(a1, b1, acc1, 0, 0, 0);
      }
    }
    }
    float y[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = 16 * tm + 4 * kq + r, col = bn;
      const float x = acc0[r] + acc1[r];
      float* p = Cm + row * ldc + col;
      if (MODE == kStore) y[r] = x;
      else if (MODE == kAdd) y[r] = *p + x;
      else y[r] = (row >> 1) <= col ? x : 0.f;
      *p = y[r];
    }
    // Ct: the result transposed in bf16 ([N][ldct], this lane's four rows one 8-byte write);
    // Cb: the result in bf16 as it is laid out ([M][ldcb])
    if (Ct != nullptr)
      *reinterpret_cast<uint2*>(Ct + bn * ldct + 16 * tm + 4 * kq) =
          make_uint2(pack_bf16x2(y[0], y[1]), pack_bf16x2(y[2], y[3]));
    if (Cb != nullptr) {
      const uint32_t w0 = pack_bf16x2(y[0], y[1]), w1 = pack_bf16x2(y[2], y[3]);
      uint16_t* q = Cb + (16 * tm + 4 * kq) * ldcb + bn;
      q[0] = static_cast<uint16_t>(w0);
      q[ldcb] = static_cast<uint16_t>(w0 >> 16);
      q[2 * ldcb] = static_cast<uint16_t>(w1);
      q[3 * ldcb] = static_cast<uint16_t>(w1 >> 16);
    }
  }
}

// Cm = Cs + A1 B1^T + A2 B2 (fp32, all in LDS; A1 [M][K1], B1 [N][K1], A2 [M][K2], B2 [K2][N]):
// both products in one pair of accumulators, so the sum is stored once.  16 x 16 output tiles
// round robin over NW waves, lane layout as in lgemm.
template <int M, int N, int K1, int K2, int NW>
__device__ __forceinline__ void lgemm2_addfrom(const float* A1, int lda1, const float* B1, int ldb1,
                                               const float* A2, int lda2, const float* B2, int ldb2,
                                               const float* Cs, float* Cm, int ldc, int wave,
                                               int lane, uint16_t* Ct = nullptr, int ldct = 0) {
  constexpr int TN = N / 16, NTILE = (M / 16) * TN;
  static_assert(K1 % 4 == 0 && K2 % 4 == 0, "k steps of 4");
  const int l16 = lane & 15, kq = lane >> 4;
  for (int tile = wave; tile < NTILE; tile += NW) {
    const int tm = tile / TN, tn = tile % TN;
    const int am = 16 * tm + l16, bn = 16 * tn + l16;
    f32x4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int k0 = 0; k0 < K1; k0 += 4) {
      const float a = A1[am * lda1 + k0 + kq], b = B1[bn * ldb1 + k0 + kq];
      if ((k0 >> 2) & 1) acc1 = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, acc1, 0, 0, 0);
      else acc0 = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, acc0, 0, 0, 0);
    }
#pragma unroll
    for (int k0 = 0; k0 < K2; k0 += 4) {
      const float a = A2[am * lda2 + k0 + kq], b = B2[(k0 + kq) * ldb2 + bn];
      if ((k0 >> 2) & 1) acc1 = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, acc1, 0, 0, 0);
      else acc0 = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, acc0, 0, 0, 0);
    }
    float y[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int o = (16 * tm + 4 * kq + r) * ldc + bn;
      y[r] = Cs[o] + (acc0[r] + acc1[r]);
      Cm[o] = y[r];
    }
    if (Ct != nullptr)  // the result transposed in bf16, as in lgemm
      *reinterpret_cast<uint2*>(Ct + bn * ldct + 16 * tm + 4 * kq) =
          make_uint2(pack_bf16x2(y[0], y[1]), pack_bf16x2(y[2], y[3]));
  }
}

// Partials of the column blocks in the workspace: fp32 for fp32 inputs; bf16 (rounded to
// nearest even) for bf16 / fp16 inputs, whose gradient products already take bf16 operands.
// The reduce kernel sums them in fp32.  put4 stores four consecutive elements.
__device__ __forceinline__ void put4(float* p, float a, float b, float c, float d) {
  *reinterpret_cast<float4*>(p) = make_float4(a, b, c, d);
}
__device__ __forceinline__ void put4(uint16_t* p, float a, float b, float c, float d) {
  *reinterpret_cast<uint2*>(p) = make_uint2(pack_bf16x2(a, b), pack_bf16x2(c, d));
}

// dst (global) = (A1 B1^T + A2 B2^T + A3 B3^T)^T, 32 x M with row stride M, with A_i [M][16]
// and B_i [32][16] in LDS (row stride L16): the three products of one tile share one
// accumulator, so the sum goes to memory once, four consecutive elements (one store) per lane.
template <int M, bool LP, int NWAVES, typename PT>
__device__ __forceinline__ void lgemm3_nt_global(const float* A1, const float* B1, const float* A2,
                                                 const float* B2, const float* A3, const float* B3,
                                                 PT* dst, int wave, int lane) {
  constexpr int NTILE = (M / 16) * 2;
  static_assert(NTILE % NWAVES == 0, "whole tiles per wave");
  const int l16 = lane & 15, kq = lane >> 4;
  // a static number of stores per wave, so that a later wait for global loads issued before
  // them is counted past them instead of waiting for the stores as well
#pragma unroll
  for (int it = 0; it < NTILE / NWAVES; ++it) {
    const int tile = wave + NWAVES * it;
    const int tm = tile >> 1, tn = tile & 1;
    const int am = 16 * tm + l16, bn = 16 * tn + l16;
    f32x4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
    const float* As[3] = {A1, A2, A3};
    const float* Bs[3] = {B1, B2, B3};
#pragma unroll
    for (int u = 0; u < 3; ++u) {
      if constexpr (LP) {
        const float* pa = As[u] + am * L16 + 4 * kq;
        const float* pb = Bs[u] + bn * L16 + 4 * kq;
        const s16x4 a = __builtin_bit_cast(s16x4, make_uint2(pack_bf16x2(pa[0], pa[1]), pack_bf16x2(pa[2], pa[3])));
        const s16x4 b = __builtin_bit_cast(s16x4, make_uint2(pack_bf16x2(pb[0], pb[1]), pack_bf16x2(pb[2], pb[3])));
        if (u & 1) acc1 = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, acc1, 0, 0, 0);
        else acc0 = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, acc0, 0, 0, 0);
      } else {
#pragma unroll
        for (int k0 = 0; k0 < 16; k0 += 8) {
          const int k = k0 + kq;
          acc0 = __builtin_amdgcn_mfma_f32_16x16x4f32(As[u][am * L16 + k], Bs[u][bn * L16 + k], acc0, 0, 0, 0);
          acc1 = __builtin_amdgcn_mfma_f32_16x16x4f32(As[u][am * L16 + k + 4], Bs[u][bn * L16 + k + 4], acc1, 0, 0, 0);
        }
      }
    }
    put4(dst + bn * M + 16 * tm + 4 * kq, acc0[0] + acc1[0], acc0[1] + acc1[1], acc0[2] + acc1[2],
         acc0[3] + acc1[3]);
  }
}

// lgemm3_nt_global (LP) with the B operands read from bf16 copies (B_i [32][ldb], 16 values of k
// per row): one 8-byte read per B operand and lane, the same bits as rounding the fp32 values.
// The A operands are fp32 as in lgemm3_nt_global.  (bf16 copies of the A operands too, written by
// their producers as 2-byte scattered stores, made the columns kernel 21 us slower.)
template <int M, int NWAVES, typename PT>
__device__ __forceinline__ void lgemm3_nt_global_b16(const float* A1, const uint16_t* B1,
                                                     const float* A2, const uint16_t* B2,
                                                     const float* A3, const uint16_t* B3,
                                                     int ldb, PT* dst, int wave, int lane) {
  constexpr int NTILE = (M / 16) * 2;
  static_assert(NTILE % NWAVES == 0, "whole tiles per wave");
  const int l16 = lane & 15, kq = lane >> 4;
#pragma unroll
  for (int it = 0; it < NTILE / NWAVES; ++it) {  // a static store count, as in lgemm3_nt_global
    const int tile = wave + NWAVES * it;
    const int tm = tile >> 1, tn = tile & 1;
    const int am = 16 * tm + l16, bn = 16 * tn + l16;
    f32x4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
    const float* As[3] = {A1, A2, A3};
    const uint16_t* Bs[3] = {B1, B2, B3};
#pragma unroll
    for (int u = 0; u < 3; ++u) {
      const float* pa = As[u] + am * L16 + 4 * kq;
      const s16x4 a = __builtin_bit_cast(s16x4, make_uint2(pack_bf16x2(pa[0], pa[1]), pack_bf16x2(pa[2], pa[3])));
      const s16x4 b = *reinterpret_cast<const s16x4*>(Bs[u] + bn * ldb + 4 * kq);
      if (u & 1) acc1 = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, acc1, 0, 0, 0);
      else acc0 = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, acc0, 0, 0, 0);
    }
    put4(dst + bn * M + 16 * tm + 4 * kq, acc0[0] + acc1[0], acc0[1] + acc1[1], acc0[2] + acc1[2],
         acc0[3] + acc1[3]);
  }
}

// G = U^T U, the Cayley blocks M_t, L and A = (I - L)^-1 of one chunk (LDS).
// U: [D][L32] (row i: k_t at 2t, v_t at 2t + 1; zero past the end); dl[t] the deltas.
// Tokens with a non-finite Cayley factor (vmi::cayley_guarded) get M = 0 and their U columns
// zeroed, G is recomputed, and their bits are left in *badm.
template <int D>
__device__ __forceinline__ void chunk_prep(float* U, const float* dl, float* G, float* Mb,
                                           float* L, float* A, int* badm, int tid, int wave,
                                           int lane, int solver) {
  lgemm<R, R, D, true, false, kStore>(U, L32, U, L32, G, R, wave, lane);
  __syncthreads();
  bool ok = true;
  if (tid < C) {
    const int t = tid;
    const cayley2 m = cayley_guarded(dl[t], G[(2 * t) * R + 2 * t], G[(2 * t + 1) * R + 2 * t + 1],
                                     G[(2 * t) * R + 2 * t + 1], ok);
    Mb[4 * t + 0] = m.m00; Mb[4 * t + 1] = m.m01; Mb[4 * t + 2] = m.m10; Mb[4 * t + 3] = m.m11;
  }
  const uint64_t bal = __ballot(!ok);  // tokens are lanes 0..C-1 of wave 0
  if (tid == 0) *badm = static_cast<int>(bal & ((1u << C) - 1));
  __syncthreads();
  const int bad = *badm;
  if (bad != 0) {  // uniform over the workgroup; only chunks holding such a token
    for (int e = tid; e < D * R; e += NT) {
      const int i = e / R, rho = e % R;
      if ((bad >> (rho >> 1)) & 1) U[i * L32 + rho] = 0.f;
    }
    __syncthreads();
    lgemm<R, R, D, true, false, kStore>(U, L32, U, L32, G, R, wave, lane);
    __syncthreads();
  }
  for (int e = tid; e < R * R; e += NT) {  // L[2t + a][2i + b] = (M_t G_ti)[a][b], i < t
    const int r = e / R, c = e % R, t = r >> 1, i = c >> 1, a = r & 1, b = c & 1;
    float x = 0.f;
    if (i < t) x = Mb[4 * t + 2 * a] * G[(2 * t) * R + 2 * i + b] + Mb[4 * t + 2 * a + 1] * G[(2 * t + 1) * R + 2 * i + b];
    L[e] = x;
  }
  __syncthreads();
  // A = I + L A, block row t from the rows of the earlier blocks, in one wave without barriers:
  // lane (a, c) = (lane >> 5, lane & 31) holds column c of A in registers, computes row 2t + a
  // of it (the two rows of a block do not depend on each other: L is zero inside the diagonal
  // blocks) from the row of L (16-byte reads, the same address across the half-wave) and takes
  // the other row from lane ^ 32 (v_permlane32_swap).  Column c is zero above its own block, so
  // every lane sums from m = 0 in the same order (the extra terms add exact zeros to a zero sum).
  // The solving wave rotates with the chunk, so the workgroups on a CU spread their solves.
  if (wave == (solver & 3)) {
    const int c = lane & 31, a = lane >> 5;
    float col[R];
#pragma unroll
    for (int r = 0; r < R; ++r) col[r] = r == c ? 1.f : 0.f;
#pragma unroll
    for (int t = 1; t < C; ++t) {
      const float* lr = L + (2 * t + a) * R;
      float x = 0.f;
#pragma unroll
      for (int m = 0; m + 4 <= 2 * t; m += 4) {
        const float4 l4 = *reinterpret_cast<const float4*>(lr + m);
        x = fmaf(l4.x, col[m], x);
        x = fmaf(l4.y, col[m + 1], x);
        x = fmaf(l4.z, col[m + 2], x);
        x = fmaf(l4.w, col[m + 3], x);
      }
      if ((2 * t) % 4 != 0) {
        const float2 l2 = *reinterpret_cast<const float2*>(lr + 2 * t - 2);
        x = fmaf(l2.x, col[2 * t - 2], x);
        x = fmaf(l2.y, col[2 * t - 1], x);
      }
      const float mine = (c >> 1) < t ? x : (a ? col[2 * t + 1] : col[2 * t]);
      const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mine), __float_as_uint(mine),
                                                       false, false);
      // lanes 32-63 receive lanes 0-31 in the first result, lanes 0-31 lanes 32-63 in the second
      const float other = __uint_as_float(a ? sw[0] : sw[1]);
      col[2 * t] = a ? other : mine;
      col[2 * t + 1] = a ? mine : other;
    }
    if (a == 0) {
#pragma unroll
      for (int r = 0; r < R; ++r) A[r * R + c] = col[r];
    }
  }
  __syncthreads();
}

// ---------------------------------------------------------------- T~ of every chunk
template <typename IO, int D>
__global__ __launch_bounds__(NT) void bwdc_prep_kernel(const IO* __restrict__ k,
                                                       const IO* __restrict__ v,
                                                       const void* __restrict__ delta,
                                                       int delta_dtype, float* __restrict__ tt,
                                                       int T, int H) {
  __shared__ float U[D * L32], G[R * R], A[R * R], Mb[4 * C], dl[C];
  __shared__ __attribute__((aligned(16))) float L[R * R];  // rows read 16 bytes at a time
  __shared__ int badm;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int n = blockIdx.x, bh = blockIdx.y, b = bh / H, hd = bh % H;
  const int nch = gridDim.x;
  {  // thread (t, EU consecutive features): one 8- or 16-byte load per row
    constexpr int EU = D * C / NT;
    const int t = tid >> 4, i0 = EU * (tid & 15), tg = n * C + t;
    const bool ok = tg < T;
    const int64_t o = ((static_cast<int64_t>(b) * T + (ok ? tg : 0)) * H + hd) * D + i0;
    const RowRaw<IO, EU> rk = load_raw<IO, EU>(k + o), rv = load_raw<IO, EU>(v + o);
#pragma unroll
    for (int j = 0; j < EU; ++j) {
      U[(i0 + j) * L32 + 2 * t] = ok ? raw_elem<IO, EU>(rk, j) : 0.f;
      U[(i0 + j) * L32 + 2 * t + 1] = ok ? raw_elem<IO, EU>(rv, j) : 0.f;
    }
  }
  if (tid < C) {
    const int tg = n * C + tid;
    dl[tid] = tg < T ? load_scalar(delta, delta_dtype, (static_cast<int64_t>(b) * T + tg) * H + hd) : 0.f;
  }
  __syncthreads();
  chunk_prep<D>(U, dl, G, Mb, L, A, &badm, tid, wave, lane, n + bh);
  float* o = tt + (static_cast<int64_t>(bh) * nch + n) * REC;
  for (int e = tid; e < R * R; e += NT) {  // T~ = A blockdiag(M), then A, G, M
    const int r = e / R, c = e % R, s = c >> 1, cb = c & 1;
    o[e] = A[r * R + 2 * s] * Mb[4 * s + cb] + A[r * R + 2 * s + 1] * Mb[4 * s + 2 + cb];
    o[R * R + e] = A[e];
    o[2 * R * R + e] = G[e];
  }
  if (tid < 4 * C) o[3 * R * R + tid] = Mb[tid];
  if (tid == 0) o[REC_BAD] = __int_as_float(badm);
}

// ---------------------------------------------------------------- state columns, in reverse
// part layout per (bh, chunk, column block): dT~ partial [R][R], then dU partial transposed,
// [R][D].
template <int D> struct PartC { static constexpr int size = R * R + D * R; };

constexpr int NTC = 512;         // threads of the columns kernel: 8 waves, two per SIMD
constexpr int NWC = NTC / 64;

template <typename IO, typename GO, int D>
__global__ __launch_bounds__(NTC) void bwdc_cols_kernel(
    const IO* __restrict__ q, const IO* __restrict__ k, const IO* __restrict__ v,
    const float* __restrict__ tt, const float* __restrict__ psi_T, const GO* __restrict__ dout,
    const float* __restrict__ dpsi_T, IO* __restrict__ dq, float* __restrict__ dpsi0,
    void* __restrict__ part_v, int T, int H) {
  constexpr int PS = PartC<D>::size;
  constexpr int NBLK = D / CB;
  // bf16 / fp16 inputs: the per-chunk gradient products take bf16 operands (their 2e-2 bar);
  // the state reconstruction and the adjoint update, carried across chunks, stay fp32
  constexpr bool LP = !std::is_same<IO, float>::value;
  typedef typename std::conditional<LP, uint16_t, float>::type PT;  // partials (see put4)
  PT* __restrict__ part = static_cast<PT*>(part_v);
  // row strides: L32 for the 32-wide (rank index) matrices, L16 for the 16-wide ones
  __shared__ float U[D * L32], Tt[R * L32], Gm[R * L32], Qb[CB * L16], dO[D * L16];
  __shared__ float Ps[D * L16], Lmb[2][D * L16];  // Lam: the chunk's Lam_e and the next one's
  __shared__ float S1[R * L16], S1b[R * L16], Wm[R * L16], Wt[R * L16], Zm[R * L16], Xm[R * L16], dXm[R * L16],
      dZm[R * L16], dWm[R * L16], QD[2][CB * L16];
  __shared__ float dTp[R * L32], dQm[CB * L16];
  // bf16 inputs' copies of U^T ([R][D], k and v rows) and dO^T ([C][D], token rows), features
  // contiguous: the A operand of dX and dZ and the B operand of dX and Psi_s^T dO, one 8-byte
  // read per lane and k step.  Row pitch D + 8: 16-byte rows, conflict-free 8-byte reads.
  constexpr int LUT = D + 8;
  __shared__ __attribute__((aligned(16))) uint16_t UTb[LP ? R * LUT : 8], dOTb[LP ? C * LUT : 8];
  // and of Lam_e^T and Psi_s^T ([CB][D]): the B operand of dZ and the A operand of Psi_s^T dO,
  // written by the products that update Lam and Psi
  __shared__ __attribute__((aligned(16))) uint16_t LTb[LP ? CB * LUT : 8], PTb[LP ? CB * LUT : 8];
  // and of the dU partial's B operands Z, X, dW as they are laid out ([R][16], pitch LB),
  // written by the products that form them
  constexpr int LB = 20;
  constexpr int NB = LP ? 1 : 0;
  __shared__ __attribute__((aligned(16))) uint16_t Zb[NB * R * LB + 8], Xb[NB * R * LB + 8],
      dWb[NB * R * LB + 8];
  // and T~ ([R][R], from the commit) and W^T ([CB][R], from W's last product): the operands of
  // Z = T~ W
  constexpr int LT = R + 8;
  __shared__ __attribute__((aligned(16))) uint16_t Ttb[NB * R * LT + 8], WTb[NB * CB * LT + 8];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  // Workgroups go to the 8 XCDs round robin by linear index.  The column blocks of one (b, h)
  // read the same k, v, dO rows and chunk records, so they get linear indices of one residue
  // mod 8 (one XCD, one L2); a last group of fewer than 8 (b, h) keeps the plain order.
  int blk, bh;
  {
    const int L = blockIdx.x + NBLK * blockIdx.y;  // gridDim.x == NBLK
    const int full = (static_cast<int>(gridDim.y) / 8) * 8 * NBLK;
    if (L < full) {
      blk = (L / 8) % NBLK;
      bh = (L / (8 * NBLK)) * 8 + L % 8;
    } else {
      blk = (L - full) % NBLK;
      bh = full / NBLK + (L - full) / NBLK;
    }
  }
  const int b = bh / H, hd = bh % H;
  const int nch = (T + C - 1) / C;
  const int64_t DD = static_cast<int64_t>(D) * D;

  for (int e = tid; e < D * CB; e += NTC) {
    const int i = e / CB, jj = e % CB;
    const int64_t o = bh * DD + static_cast<int64_t>(i) * D + blk * CB + jj;
    Ps[i * L16 + jj] = psi_T[o];
    Lmb[0][i * L16 + jj] = dpsi_T ? dpsi_T[o] : 0.f;
    if constexpr (LP) LTb[jj * LUT + i] = static_cast<uint16_t>(to_bf16(Lmb[0][i * L16 + jj]));
  }
  // chunk n's inputs: registers first (the next chunk's arrive while this one runs), loaded by
  // waves 4-7, which are idle in the phase that issues the loads.  Thread (t = tid / 16, j0 = EU (tid % 16)) holds elements
  // j0 .. j0 + EU - 1 of token t's k, v and dO rows as raw words (one 8- or 16-byte load each
  // per row; converted at the commit), its q element, and four consecutive words of the chunk
  // record's T~ and of its Gram matrix G.
  constexpr int NL = 16 * C;      // loading threads
  constexpr int EU = D * C / NL;  // elements of k (and of v, dO) per loading thread
  static_assert(D == 16 * EU && CB * C == NL && R * R == 4 * NL, "16 threads per token row");
  const bool loader = tid >= NTC - NL;
  const int lt = tid - (NTC - NL);  // loader thread index (meaningful for loaders)
  // Nothing loaded here is converted or moved before the commit, so no wait for the loads is
  // placed in the phase that issues them (q is kept as raw bits, and the bad-token mask comes
  // through a vector load: a scalar load would be waited for at the next LDS barrier, which
  // counts both).
  RowRaw<IO, EU> rk, rv;
  RowRaw<GO, EU> rd;
  RowRaw<IO, 2> rq;
  float4 rt, rg;
  int rbad = 0;  // tokens of the chunk that are the identity (non-finite Cayley factor)
  auto tok = [&](int tg) { return (static_cast<int64_t>(b) * T + tg) * H + hd; };
  const int ft = (lt >> 4) & (C - 1), fj = EU * (lt & 15);
  auto fetch = [&](int n) {
    if (!loader) return;
    const int tg = n * C + ft;
    const int64_t o = tok(tg < T ? tg : 0) * D + fj;
    rk = load_raw<IO, EU>(k + o);
    rv = load_raw<IO, EU>(v + o);
    rd = load_raw<GO, EU>(dout + o);
    {
      const int t = lt / CB, jj = lt % CB, tq = n * C + t;
      rq = load_raw1<IO>(q + tok(tq < T ? tq : 0) * D + blk * CB + jj);
    }
    const float* rec = tt + (static_cast<int64_t>(bh) * nch + n) * REC;
    rt = *reinterpret_cast<const float4*>(rec + 4 * lt);
    rg = *reinterpret_cast<const float4*>(rec + 2 * R * R + 4 * lt);
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(rec), (short)0, REC * static_cast<int>(sizeof(float)), 0x00020000);
    rbad = static_cast<int>(__builtin_amdgcn_raw_buffer_load_b32(rs, REC_BAD * 4, 0, 0));
  };
  auto commit = [&](int n) {
    if (!loader) return;
    const bool ok = n * C + ft < T;
    const bool uk = ok && !((rbad >> ft) & 1);
#pragma unroll
    for (int j = 0; j < EU; ++j) {
      const int i = fj + j;
      U[i * L32 + 2 * ft] = uk ? raw_elem<IO, EU>(rk, j) : 0.f;
      U[i * L32 + 2 * ft + 1] = uk ? raw_elem<IO, EU>(rv, j) : 0.f;
      dO[i * L16 + ft] = ok ? raw_elem<GO, EU>(rd, j) : 0.f;
    }
    if constexpr (LP) {
      put_bf16_row<IO, EU>(UTb + (2 * ft) * LUT + fj, rk, uk);
      put_bf16_row<IO, EU>(UTb + (2 * ft + 1) * LUT + fj, rv, uk);
      put_bf16_row<GO, EU>(dOTb + ft * LUT + fj, rd, ok);
    }
    {
      const int t = lt / CB, jj = lt % CB;
      Qb[jj * L16 + t] = n * C + t < T ? raw_elem<IO, 2>(rq, 0) : 0.f;
    }
    const int e = (4 * lt) / R * L32 + (4 * lt) % R;  // row pitch 37: 4-byte stores
    Tt[e] = rt.x; Tt[e + 1] = rt.y; Tt[e + 2] = rt.z; Tt[e + 3] = rt.w;
    if constexpr (LP)
      *reinterpret_cast<uint2*>(Ttb + (4 * lt) / R * LT + (4 * lt) % R) =
          make_uint2(pack_bf16x2(rt.x, rt.y), pack_bf16x2(rt.z, rt.w));
    Gm[e] = rg.x; Gm[e + 1] = rg.y; Gm[e + 2] = rg.z; Gm[e + 3] = rg.w;
  };

  if (nch > 0) {
    fetch(nch - 1);
    commit(nch - 1);
  }
  lds_barrier();
  // Per chunk, six phases and the commit between LDS barriers, independent products of a phase
  // on disjoint waves.  W = U^T Psi_s is formed as S1 + G Wm (U^T Psi_s = U^T Psi_e + U^T U T~^T
  // S1), so it needs no product over the state rows after the reconstruction.
  int lc = 0;  // Lmb[lc] holds Lam_e of chunk n
  for (int n = nch - 1; n >= 0; --n) {
    const float* Lm = Lmb[lc];
    float* Ln = Lmb[lc ^ 1];
    // (1) S1 = U^T Psi_e as two halves of the state rows, S1 (waves 0-1) + S1b (waves 6-7);
    //     dX = mask o (U^T dO) (waves 2-3); dZ = U^T Lam_e (4-5)
    lgemm<R, CB, D / 2, true, false, kStore, 0, 2>(U, L32, Ps, L16, S1, L16, wave, lane);
    lgemm<R, CB, D / 2, true, false, kStore, 6, 2>(U + (D / 2) * L32, L32, Ps + (D / 2) * L16, L16,
                                                   S1b, L16, wave, lane);
    if constexpr (LP) {
      lgemm<R, C, D, true, false, kMaskStore, 2, 2, true, false, true, true>(
          U, L32, dO, L16, dXm, L16, wave, lane, nullptr, UTb, LUT, dOTb, LUT);
      lgemm<R, CB, D, true, false, kStore, 4, 2, true, false, true, true>(
          U, L32, Lm, L16, dZm, L16, wave, lane, nullptr, UTb, LUT, LTb, LUT);
    } else {
      lgemm<R, C, D, true, false, kMaskStore, 2, 2>(U, L32, dO, L16, dXm, L16, wave, lane);
      lgemm<R, CB, D, true, false, kStore, 4, 2>(U, L32, Lm, L16, dZm, L16, wave, lane);
    }
    lds_barrier();
    // (2) Wm = T~^T S1 (waves 0-1); dZ += dX Q^T (waves 4-5, the tiles they stored);
    //     W starts as S1 (every thread one element)
    lgemm<R, CB, R, true, false, kStore, 0, 2, false, true>(Tt, L32, S1, L16, Wm, L16, wave, lane, S1b);
    lgemm<R, CB, C, false, true, kAdd, 4, 2, LP>(dXm, L16, Qb, L16, dZm, L16, wave, lane);
    for (int e = tid; e < R * CB; e += NTC) {
      const int o = (e / CB) * L16 + e % CB;
      Wt[o] = S1[o] + S1b[o];
    }
    lds_barrier();
    // (3) Psi_s = Psi_e + U Wm (8 waves); W += G Wm (waves 0-1, after their Psi tile);
    //     dW = T~^T dZ (waves 2-3)
    lgemm<D, CB, R, false, false, kAdd, 0, NWC>(U, L32, Wm, L16, Ps, L16, wave, lane, nullptr,
                                               nullptr, 0, nullptr, 0, LP ? PTb : nullptr, LUT);
    lgemm<R, CB, R, false, false, kAdd, 0, 2>(Gm, L32, Wm, L16, Wt, L16, wave, lane, nullptr,
                                              nullptr, 0, nullptr, 0, LP ? WTb : nullptr, LT);
    lgemm<R, CB, R, true, false, kStore, 2, 2, LP>(Tt, L32, dZm, L16, dWm, L16, wave, lane, nullptr,
                                                   nullptr, 0, nullptr, 0, nullptr, 0,
                                                   LP ? dWb : nullptr, LB);
    lds_barrier();
    // (4) Z = T~ W (waves 0-1); Psi_s^T dO (first term of dQ) over two halves of the state rows
    //     (waves 2-3); dT~ partial = dZ W^T (waves 4-7)
    if constexpr (LP)
      lgemm<R, CB, R, false, false, kStore, 0, 2, true, false, true, true>(
          Tt, L32, Wt, L16, Zm, L16, wave, lane, nullptr, Ttb, LT, WTb, LT, nullptr, 0, Zb, LB);
    else
      lgemm<R, CB, R, false, false, kStore, 0, 2>(Tt, L32, Wt, L16, Zm, L16, wave, lane);
    if constexpr (LP) {
      lgemm<CB, C, D / 2, true, false, kStore, 2, 1, true, false, true, true>(
          Ps, L16, dO, L16, QD[0], L16, wave, lane, nullptr, PTb, LUT, dOTb, LUT);
      lgemm<CB, C, D / 2, true, false, kStore, 3, 1, true, false, true, true>(
          Ps + (D / 2) * L16, L16, dO + (D / 2) * L16, L16, QD[1], L16, wave, lane, nullptr,
          PTb + D / 2, LUT, dOTb + D / 2, LUT);
    } else {
      lgemm<CB, C, D / 2, true, false, kStore, 2, 1>(Ps, L16, dO, L16, QD[0], L16, wave, lane);
      lgemm<CB, C, D / 2, true, false, kStore, 3, 1>(Ps + (D / 2) * L16, L16, dO + (D / 2) * L16,
                                                     L16, QD[1], L16, wave, lane);
    }
    lgemm<R, R, CB, false, true, kStore, 4, 4, LP>(dZm, L16, Wt, L16, dTp, L32, wave, lane);
    lds_barrier();
    // (5) X = mask o (Z Q) (waves 0-1); dQ second term Z^T dX (wave 2); the next chunk's loads
    //     (waves 4-7: issued here, before this chunk's stores, and committed after phase 6)
    lgemm<R, C, CB, false, false, kMaskStore, 0, 2, LP>(Zm, L16, Qb, L16, Xm, L16, wave, lane,
                                                        nullptr, nullptr, 0, nullptr, 0, nullptr,
                                                        0, LP ? Xb : nullptr, LB);
    lgemm<CB, C, R, true, false, kStore, 2, 1, LP>(Zm, L16, dXm, L16, dQm, L16, wave, lane);
    if (n > 0) fetch(n - 1);
    lds_barrier();
    // (6) dU partial = Lam_e Z^T + dO X^T + Psi_s dW^T straight to the workspace; dT~ partial
    //     and dq out
    PT* pp = part + ((static_cast<int64_t>(bh) * nch + n) * NBLK + blk) * PS;
    if constexpr (LP)
      lgemm3_nt_global_b16<D, NWC>(Lm, Zb, dO, Xb, Ps, dWb, LB, pp + R * R, wave, lane);
    else
      lgemm3_nt_global<D, LP, NWC>(Lm, Zm, dO, Xm, Ps, dWm, pp + R * R, wave, lane);
    {
      for (int e = 4 * tid; e < R * R; e += 4 * NTC) {
        const float* d = &dTp[(e / R) * L32 + e % R];
        put4(pp + e, d[0], d[1], d[2], d[3]);
      }
      if (tid < CB * C) {
        const int jj = tid / C, t = tid % C, tg = n * C + t;
        const int e = jj * L16 + t;
        if (tg < T) io<IO>::store(dq, tok(tg) * D + blk * CB + jj, dQm[e] + QD[0][e] + QD[1][e]);
      }
    }
    // (6, continued) Lam_s = Lam_e + dO Q^T + U dW into the other buffer (8 waves, one tile
    // each, both terms in one accumulation): the dU partial above still reads Lam_e
    lgemm2_addfrom<D, CB, C, R, NWC>(dO, L16, Qb, L16, U, L32, dWm, L16, Lm, Ln, L16, wave, lane,
                                     LP ? LTb : nullptr, LUT);
    lc ^= 1;
    lds_barrier();
    if (n > 0) commit(n - 1);
    lds_barrier();
  }
  if (dpsi0) {
    for (int e = tid; e < D * CB; e += NTC) {
      const int i = e / CB, jj = e % CB;
      dpsi0[bh * DD + static_cast<int64_t>(i) * D + blk * CB + jj] = Lmb[lc][i * L16 + jj];
    }
  }
}

// ---------------------------------------------------------------- per chunk: dT~ -> dk, dv, ddelta
template <typename IO, int D>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(4))) void bwdc_reduce_kernel(
    const IO* __restrict__ k, const IO* __restrict__ v, const void* __restrict__ delta,
    int delta_dtype, const float* __restrict__ tt, const void* __restrict__ part,
    IO* __restrict__ dk, IO* __restrict__ dv, void* __restrict__ ddelta, int T, int H) {
  constexpr int PS = PartC<D>::size;
  constexpr int NBLK = D / CB;
  static_assert(R * R % NT == 0 && D * C % NT == 0 && 4 * C <= NT, "record and tokens split evenly");
  constexpr int NR = R * R / NT, NK = D * C / NT;
  // 40 KB of LDS (four workgroups per CU): U (row stride 37), tmp and A (row stride 33), and a
  // pool whose buffers are dead by the last product, which writes its R x D result over them.
  // The dU partial sums stay in registers.  dT and G share a buffer (G is stored once dT is
  // consumed), and so do dG and L (the new dG, written once dG is consumed).
  constexpr int LA = 33;
  constexpr int POOL = 3 * R * R + R * LA + 4 * C + C;
  static_assert(POOL >= R * D, "the last product's output fits the pool");
  __shared__ float U[D * L32], tmp[R * LA], pool[POOL];
  float* const dT = pool;           // then G
  float* const dA = pool + R * R;
  float* const dG = pool + 2 * R * R;  // then L
  float* const A = pool + 3 * R * R;
  float* const Mb = A + R * LA;
  float* const dl = Mb + 4 * C;
  float* const G = dT;
  float* const L = dG;
  float* const dU = pool;           // the last product's output, R x D
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int n = blockIdx.x, bh = blockIdx.y, b = bh / H, hd = bh % H;
  const int nch = gridDim.x;
  auto tok = [&](int tg) { return (static_cast<int64_t>(b) * T + tg) * H + hd; };
  // every global load of the workgroup is issued before the first wait: the partials of all
  // column blocks, the chunk record (A, G, M) and the chunk's k, v, delta.  Thread (ft = tid /
  // 16, fi = NK (tid % 16)) loads elements fi .. fi + NK - 1 of rows 2 ft and 2 ft + 1 of each
  // dU partial (the elements of dk, dv it stores at the end) and four consecutive dT~ elements.
  // The partials are read once, with the nontemporal hint (82.7 -> 68.2 us at B4 T2048 H8 D128:
  // 335 MB at 4.9 TB/s; the same hint on the columns kernel's partial stores made it slower).
  constexpr bool LP = !std::is_same<IO, float>::value;  // bf16 partials (see put4)
  typedef typename std::conditional<LP, bf16_t, float>::type PE;  // partial element type
  typedef typename std::conditional<LP, uint2, float4>::type PV;  // four partial elements
  static_assert(R * R == 4 * NT, "four dT~ elements per thread");
  const int ft = tid >> 4, fi = NK * (tid & 15);
  PV xt[NBLK];
  RowRaw<PE, NK> xk[NBLK], xv[NBLK];
  {
    const PE* pp = static_cast<const PE*>(part) + (static_cast<int64_t>(bh) * nch + n) * NBLK * PS;
#pragma unroll
    for (int j = 0; j < NBLK; ++j) {
      {
        typedef unsigned pvv __attribute__((ext_vector_type(sizeof(PV) / 4)));
        xt[j] = __builtin_bit_cast(PV, __builtin_nontemporal_load(reinterpret_cast<const pvv*>(pp + j * PS) + tid));
      }
      xk[j] = load_raw_nt<PE, NK>(pp + j * PS + R * R + (2 * ft) * D + fi);
      xv[j] = load_raw_nt<PE, NK>(pp + j * PS + R * R + (2 * ft + 1) * D + fi);
    }
  }
  auto f4 = [](const PV& y) {
    if constexpr (LP)
      return make_float4(bf16_to_f32(y.x & 0xffffu), bf16_to_f32(y.x >> 16),
                         bf16_to_f32(y.y & 0xffffu), bf16_to_f32(y.y >> 16));
    else
      return y;
  };
  float ra[NR], rg[NR], rm = 0.f, rd = 0.f;
  int bad;  // tokens of the chunk that are the identity (non-finite Cayley factor): no gradient
  {
    const float* rec = tt + (static_cast<int64_t>(bh) * nch + n) * REC;
    bad = __float_as_int(rec[REC_BAD]);
#pragma unroll
    for (int u = 0; u < NR; ++u) {
      ra[u] = rec[R * R + tid + NT * u];
      rg[u] = rec[2 * R * R + tid + NT * u];
    }
    if (tid < 4 * C) rm = rec[3 * R * R + tid];
  }
  // the same (token, features) split of the chunk's k, v rows: one 8- or 16-byte load each
  const int64_t fo = tok(n * C + ft < T ? n * C + ft : 0) * D + fi;
  const RowRaw<IO, NK> rk = load_raw<IO, NK>(k + fo), rv = load_raw<IO, NK>(v + fo);
  if (tid < C) {
    const int tg = n * C + tid;
    rd = tg < T ? load_scalar(delta, delta_dtype, tok(tg)) : 0.f;
  }
#pragma unroll
  for (int u = 0; u < NR; ++u) {
    const int e = tid + NT * u;
    A[(e / R) * LA + e % R] = ra[u];
  }
  if (tid < 4 * C) Mb[tid] = rm;
  if (tid < C) dl[tid] = rd;
  {
    const bool ok = n * C + ft < T && !((bad >> ft) & 1);
#pragma unroll
    for (int j = 0; j < NK; ++j) {
      U[(fi + j) * L32 + 2 * ft] = ok ? raw_elem<IO, NK>(rk, j) : 0.f;
      U[(fi + j) * L32 + 2 * ft + 1] = ok ? raw_elem<IO, NK>(rv, j) : 0.f;
    }
  }
  {
    float4 s = f4(xt[0]);
#pragma unroll
    for (int j = 1; j < NBLK; ++j) {
      const float4 y = f4(xt[j]);
      s.x += y.x; s.y += y.y; s.z += y.z; s.w += y.w;
    }
    *reinterpret_cast<float4*>(dT + 4 * tid) = s;
  }
  float sk[NK], sv[NK];  // dU partial sums, rows 2 ft and 2 ft + 1
#pragma unroll
  for (int i = 0; i < NK; ++i) {
    sk[i] = raw_elem<PE, NK>(xk[0], i);
    sv[i] = raw_elem<PE, NK>(xv[0], i);
#pragma unroll
    for (int j = 1; j < NBLK; ++j) {
      sk[i] += raw_elem<PE, NK>(xk[j], i);
      sv[i] += raw_elem<PE, NK>(xv[j], i);
    }
  }
  __syncthreads();
  // B = blockdiag(M); dA = dT~ B^T (block structure: dA[r][2s + a] = sum_b dT[r][2s + b] M_s[a][b])
  for (int e = tid; e < R * R; e += NT) {
    const int r = e / R, c = e % R, s = c >> 1, a = c & 1;
    dA[e] = dT[r * R + 2 * s] * Mb[4 * s + 2 * a] + dT[r * R + 2 * s + 1] * Mb[4 * s + 2 * a + 1];
  }
  __syncthreads();
  // tmp = A^T dA; dB = A^T dT~ (its diagonal blocks used) into dG
  lgemm<R, R, R, true, false, kStore>(A, LA, dA, R, tmp, LA, wave, lane);
  lgemm<R, R, R, true, false, kStore>(A, LA, dT, R, dG, R, wave, lane);
  __syncthreads();
  // dL = tmp A^T  (into dA); G over dT, which is consumed
  lgemm<R, R, R, false, true, kStore>(tmp, LA, A, LA, dA, R, wave, lane);
#pragma unroll
  for (int u = 0; u < NR; ++u) G[tid + NT * u] = rg[u];
  __syncthreads();
  // dM_t = dB_tt + sum_{i<t} dL_ti G_ti^T; then the M chain; dG_ti = M_t^T dL_ti (i < t)
  if (tid < 4 * C) {
    const int t = tid >> 2, a = (tid >> 1) & 1, c = tid & 1;
    float y = dG[(2 * t + a) * R + 2 * t + c];
    for (int i = 0; i < t; ++i)
#pragma unroll
      for (int m = 0; m < 2; ++m) y = fmaf(dA[(2 * t + a) * R + 2 * i + m], G[(2 * t + c) * R + 2 * i + m], y);
    tmp[tid] = y;  // dM_t[a][c]
  }
  __syncthreads();
  for (int e = tid; e < R * R; e += NT) {  // dG off-diagonal blocks (lower), zero elsewhere
    const int r = e / R, c = e % R, t = r >> 1, i = c >> 1, a = r & 1;
    float y = 0.f;
    if (i < t)  // (M_t^T dL_ti)[a][cb] = sum_m M_t[m][a] dL_ti[m][cb]
      y = Mb[4 * t + a] * dA[(2 * t) * R + c] + Mb[4 * t + 2 + a] * dA[(2 * t + 1) * R + c];
    L[e] = y;  // the new dG, over dG (consumed above)
  }
  __syncthreads();
  if (tid < C) {  // M chain (vmi::cayley_coeffs) -> ddelta and the diagonal Gram entries
    const int t = tid;
    const float kk = G[(2 * t) * R + 2 * t], vv = G[(2 * t + 1) * R + 2 * t + 1], kv = G[(2 * t) * R + 2 * t + 1];
    const float d00 = tmp[4 * t], d01 = tmp[4 * t + 1], d10 = tmp[4 * t + 2], d11 = tmp[4 * t + 3];
    const float hh = (bad >> t) & 1 ? 0.f : 0.5f * dl[t], P = hh * hh;  // identity token: no chain
    const float graw = kk * vv - kv * kv, g = fmaxf(graw, 0.f);
    const float c = 2.f / (1.f + P * g);
    const float N00 = -P * vv, N01 = P * kv - hh, N10 = P * kv + hh, N11 = -P * kk;
    const float S = d00 * N00 + d01 * N01 + d10 * N10 + d11 * N11;
    float dh = c * (d01 * (2.f * hh * kv - 1.f) + d10 * (2.f * hh * kv + 1.f) - 2.f * hh * (d00 * vv + d11 * kk));
    float dvv = -c * P * d00, dkk = -c * P * d11, dkv = c * P * (d01 + d10);
    dh += S * (-c * c * hh * g);
    const float dg = graw > 0.f ? S * (-0.5f * c * c * P) : 0.f;
    dkk += dg * vv;
    dvv += dg * kk;
    dkv += -2.f * dg * kv;
    L[(2 * t) * R + 2 * t] += dkk;
    L[(2 * t + 1) * R + 2 * t + 1] += dvv;
    L[(2 * t) * R + 2 * t + 1] += dkv;
    const int tg = n * C + t;
    if (tg < T) {
      const float dd = (bad >> t) & 1 ? 0.f : 0.5f * dh;
      const int64_t o = tok(tg);
      if (delta_dtype == VMI_F32) static_cast<float*>(ddelta)[o] = dd;
      else if (delta_dtype == VMI_BF16) static_cast<uint16_t*>(ddelta)[o] = f32_to_bf16(dd);
      else static_cast<f16_t*>(ddelta)[o] = static_cast<f16_t>(dd);
    }
  }
  __syncthreads();
  for (int e = tid; e < R * R; e += NT) {  // symmetrise: dG + dG^T
    const int r = e / R, c = e % R;
    tmp[r * LA + c] = L[r * R + c] + L[c * R + r];
  }
  __syncthreads();
  // dU^T = partial sums + (dG + dG^T) U^T (the partials hold dU transposed, [R][D]); the
  // product goes over the pool, whose buffers are all consumed
  lgemm<R, D, R, false, true, kStore>(tmp, LA, U, L32, dU, D, wave, lane);
  __syncthreads();
  if (n * C + ft < T) {  // the same (token, features) split: one 8- or 16-byte store per row
    const bool z = (bad >> ft) & 1;
    float yk[NK], yv[NK];
#pragma unroll
    for (int j = 0; j < NK; ++j) {
      yk[j] = z ? 0.f : sk[j] + dU[(2 * ft) * D + fi + j];
      yv[j] = z ? 0.f : sv[j] + dU[(2 * ft + 1) * D + fi + j];
    }
    store_row<IO, NK>(dk + fo, yk);
    store_row<IO, NK>(dv + fo, yv);
  }
}

template <typename IO, typename GO, int D>
hipError_t launch_d(const void* q, const void* k, const void* v, const void* delta,
                    int delta_dtype, const float* psi_T, const void* dout, const float* dpsi_T,
                    void* dq, void* dk, void* dv, void* ddelta, float* dpsi0, int B, int T,
                    int H, void* ws, hipStream_t stream) {
  const int nch = (T + C - 1) / C;
  const int BH = B * H;
  float* tt = static_cast<float*>(ws);
  float* part = tt + static_cast<int64_t>(BH) * nch * REC;
  if (nch > 0) {
    hipLaunchKernelGGL((bwdc_prep_kernel<IO, D>), dim3(nch, BH), dim3(NT), 0, stream,
                       static_cast<const IO*>(k), static_cast<const IO*>(v), delta, delta_dtype,
                       tt, T, H);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL((bwdc_cols_kernel<IO, GO, D>), dim3(D / CB, BH), dim3(NTC), 0, stream,
                     static_cast<const IO*>(q), static_cast<const IO*>(k),
                     static_cast<const IO*>(v), tt, psi_T, static_cast<const GO*>(dout), dpsi_T,
                     static_cast<IO*>(dq), dpsi0, part, T, H);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || nch == 0) return e;
  hipLaunchKernelGGL((bwdc_reduce_kernel<IO, D>), dim3(nch, BH), dim3(NT), 0, stream,
                     static_cast<const IO*>(k), static_cast<const IO*>(v), delta, delta_dtype,
                     tt, part, static_cast<IO*>(dk), static_cast<IO*>(dv), ddelta, T, H);
  return hipGetLastError();
}

template <typename IO, typename GO>
hipError_t launch_go(const void* q, const void* k, const void* v, const void* delta,
                     int delta_dtype, const float* psi_T, const void* dout, const float* dpsi_T,
                     void* dq, void* dk, void* dv, void* ddelta, float* dpsi0, int B, int T,
                     int H, int D, void* ws, hipStream_t stream) {
  if (D == 64)
    return launch_d<IO, GO, 64>(q, k, v, delta, delta_dtype, psi_T, dout, dpsi_T, dq, dk, dv,
                                ddelta, dpsi0, B, T, H, ws, stream);
  return launch_d<IO, GO, 128>(q, k, v, delta, delta_dtype, psi_T, dout, dpsi_T, dq, dk, dv,
                               ddelta, dpsi0, B, T, H, ws, stream);
}

template <typename IO>
hipError_t launch_io(const void* q, const void* k, const void* v, const void* delta,
                     int delta_dtype, const float* psi_T, const void* dout, int dout_dtype,
                     const float* dpsi_T, void* dq, void* dk, void* dv, void* ddelta,
                     float* dpsi0, int B, int T, int H, int D, void* ws, hipStream_t stream) {
  if (dout_dtype == VMI_F32)
    return launch_go<IO, float>(q, k, v, delta, delta_dtype, psi_T, dout, dpsi_T, dq, dk, dv,
                                ddelta, dpsi0, B, T, H, D, ws, stream);
  if (dout_dtype == VMI_BF16)
    return launch_go<IO, bf16_t>(q, k, v, delta, delta_dtype, psi_T, dout, dpsi_T, dq, dk, dv,
                                 ddelta, dpsi0, B, T, H, D, ws, stream);
  return launch_go<IO, f16_t>(q, k, v, delta, delta_dtype, psi_T, dout, dpsi_T, dq, dk, dv,
                              ddelta, dpsi0, B, T, H, D, ws, stream);
}

}  // namespace bwdc

size_t sssd_bwd_chunk_workspace_bytes(int64_t B, int64_t T, int64_t H, int64_t D) {
  const int64_t nch = (T + bwdc::C - 1) / bwdc::C;
  const int64_t per = bwdc::REC + (D / bwdc::CB) * (bwdc::R * bwdc::R + D * bwdc::R);
  return static_cast<size_t>(B * H * nch * per) * sizeof(float);
}

hipError_t launch_sssd_bwd_chunk(const void* q, const void* k, const void* v, const void* delta,
                                 int io_dtype, int delta_dtype, const float* psi_T,
                                 const void* dout, int dout_dtype, const float* dpsi_T, void* dq,
                                 void* dk, void* dv, void* ddelta, float* dpsi0, int B, int T,
                                 int H, int D, void* ws, hipStream_t stream) {
  if (io_dtype == VMI_F32)
    return bwdc::launch_io<float>(q, k, v, delta, delta_dtype, psi_T, dout, dout_dtype, dpsi_T, dq,
                                  dk, dv, ddelta, dpsi0, B, T, H, D, ws, stream);
  if (io_dtype == VMI_BF16)
    return bwdc::launch_io<bf16_t>(q, k, v, delta, delta_dtype, psi_T, dout, dout_dtype, dpsi_T,
                                   dq, dk, dv, ddelta, dpsi0, B, T, H, D, ws, stream);
  return bwdc::launch_io<f16_t>(q, k, v, delta, delta_dtype, psi_T, dout, dout_dtype, dpsi_T, dq,
                                dk, dv, ddelta, dpsi0, B, T, H, D, ws, stream);
}

}  // namespace vmi
