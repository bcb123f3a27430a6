// Backward of the SSSD Cayley scan (training).  The reference trains through eager
// autograd over sssd_attention.py:144-175 (torch.linalg.solve, the Blelloch product
// scan, Psi_t = P_t Psi_0, o_t = Psi_t q_t; pretrain.py:164-195), materialising
// [B, H, T, D, D] tensors; this computes the same gradients from the closed form.
//
// Forward (0-based tokens): Psi^(t+1) = R_t Psi^(t), R_t = I + U_t M_t U_t^T, U_t = [k_t v_t],
// o_t = Psi^(t+1) q_t.  With Lambda^(T) = dL/dPsi_T and, for t = T-1 .. 0,
//   Lambda^(t+1) += dO_t q_t^T                         (the readout of token t)
//   dq_t   = Psi^(t+1)^T dO_t
//   Psi^(t) = R_t^T Psi^(t+1)                         (R_t is exactly orthogonal)
//   A = U^T Psi^(t),  B = U^T Lambda^(t+1)             (2 x D)
//   dL/dU |M = Lambda^(t+1) A^T M^T + Psi^(t) B^T M,   dL/dM = B A^T
//   Lambda^(t) = R_t^T Lambda^(t+1)
// and dL/dPsi_0 = Lambda^(0).  M_t depends on delta_t and the Gram entries kk, vv, kv
// (vmi::cayley_coeffs); the reduce kernel carries dL/dM through them into dk, dv,
// ddelta.
//
// Kernel 1 (sssd_bwd_cols_kernel), grid (D / 16, B H), 512 threads: the columns of Psi
// and Lambda evolve independently under left multiplication, so a workgroup carries 16
// columns of both through all T tokens in reverse; thread (w, lane) holds rows
// lane % 32 + 32 r of column 2 w + lane / 32 (column sums over 32 lanes; two waves per
// SIMD).  dq is complete per column; the row sums over columns (dL/dU) and dL/dM are
// summed over the workgroup's 16 columns (the wave's pair, then the 8 waves in LDS) and
// written as per-token partials.  (One column per 64-lane wave, 16 waves: slower, the
// 16-wave barrier and LDS sum cost more than the extra waves hide.)
// Kernel 2 (sssd_bwd_reduce_kernel), one wave per token-head: sums the D / 16 partials
// and applies the chain rule through M.
#include "vmi_common.h"
#include "vmi_dispatch.h"
#include "vmi_lanes.h"

namespace vmi {
namespace bwd {

constexpr int CB = 16;  // columns per workgroup
constexpr int SB = 16;  // tokens per LDS stage
constexpr int NT = 512;
constexpr int LPC = 32;           // lanes per column
constexpr int CPW = 64 / LPC;     // columns per wave
constexpr int NWV = NT / 64;      // waves

// DP: head_dim padded to a multiple of 32 (32, 64, 128, 256); the runtime D <= DP rows and
// columns are real, the padding rows and columns are zeros and contribute nothing.
template <int DP> struct Part { static constexpr int size = 2 * DP + 8; };  // dU rows, dM, pad

// sum over the LPC lanes of a column, result in all of them
__device__ __forceinline__ float col_sum(float x) {
  x = row_pair_sum(row16_sum(x));
  return LPC == 64 ? half_pair_sum(x) : x;
}

template <typename IO, typename GO, int DP>
__global__ __launch_bounds__(NT) void sssd_bwd_cols_kernel(
    const IO* __restrict__ q, const IO* __restrict__ k, const IO* __restrict__ v,
    const void* __restrict__ delta, int delta_dtype, const float* __restrict__ psi_T,
    const GO* __restrict__ dout, const float* __restrict__ dpsi_T, IO* __restrict__ dq,
    float* __restrict__ dpsi0, float* __restrict__ part, int T, int H, int D) {
  constexpr int RPT = DP / LPC;  // rows per thread
  constexpr int PS = Part<DP>::size;
  constexpr int NBLK = DP / CB;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int rg = lane & (LPC - 1);
  const int cl = CPW * wave + lane / LPC;  // column within the block
  const int blk = blockIdx.x, bh = blockIdx.y;
  const int b = bh / H, hd = bh % H;
  const int j = blk * CB + cl;            // state column (padding when j >= D)
  const bool jv = j < D;
  const int64_t DD = static_cast<int64_t>(D) * D;

  __shared__ float sk[2][SB][DP], sv[2][SB][DP], sdo[2][SB][DP];
  __shared__ float sq[2][SB][CB];
  __shared__ float sco[2][SB][8];  // m00 m01 m10 m11 kk kv vv -
  __shared__ float sdl[2][SB];
  __shared__ float sred[2][NWV][2 * DP + 4];  // per-wave partials, double-buffered

  // state columns: psi = Psi^(T)[:, j], lam = dL/dPsi_T[:, j]
  float psi[RPT], lam[RPT];
#pragma unroll
  for (int r = 0; r < RPT; ++r) {
    const int row = rg + LPC * r;
    const bool ok = jv && row < D;
    const int64_t o = ok ? bh * DD + static_cast<int64_t>(row) * D + j : 0;
    psi[r] = ok ? psi_T[o] : 0.f;
    lam[r] = (ok && dpsi_T) ? dpsi_T[o] : 0.f;
  }

  // stage s holds tokens t = T - 1 - (SB s + i), i < SB (descending); tokens < 0 and
  // padding features are zeros
  constexpr int EPT = SB * DP / NT;
  float rk[EPT], rv[EPT], rdo[EPT];
  float rq = 0.f, rd = 0.f;
  auto tok_index = [&](int t) { return (static_cast<int64_t>(b) * T + t) * H + hd; };
  auto fetch = [&](int s) {
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
      const int x = tid + NT * e;
      const int t = T - 1 - (SB * s + x / DP);
      const int64_t o = (t >= 0 && x % DP < D) ? tok_index(t) * D + x % DP : 0;
      rk[e] = io<IO>::load(k, o);
      rv[e] = io<IO>::load(v, o);
      rdo[e] = io<GO>::load(dout, o);
    }
    {
      const int t = T - 1 - (SB * s + tid / CB);
      rq = (tid < SB * CB && t >= 0 && blk * CB + tid % CB < D)
               ? io<IO>::load(q, tok_index(t) * D + blk * CB + tid % CB) : 0.f;
    }
    {
      const int t = T - 1 - (SB * s + tid);
      rd = (tid < SB && t >= 0) ? load_scalar(delta, delta_dtype, tok_index(t)) : 0.f;
    }
  };
  auto commit = [&](int s) {
    const int buf = s & 1;
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
      const int x = tid + NT * e;
      const bool ok = T - 1 - (SB * s + x / DP) >= 0 && x % DP < D;
      sk[buf][x / DP][x % DP] = ok ? rk[e] : 0.f;
      sv[buf][x / DP][x % DP] = ok ? rv[e] : 0.f;
      sdo[buf][x / DP][x % DP] = ok ? rdo[e] : 0.f;
    }
    if (tid < SB * CB) sq[buf][tid / CB][tid % CB] = rq;
    if (tid < SB) sdl[buf][tid] = rd;
    __syncthreads();
    // Gram entries and M of each token: the LPC lanes tt sum over D / LPC rows
    {
      const int tt = tid / LPC;  // SB * LPC == NT
      float kk = 0.f, vv = 0.f, kv = 0.f;
#pragma unroll
      for (int r = 0; r < RPT; ++r) {
        const float x = sk[buf][tt][rg + LPC * r], y = sv[buf][tt][rg + LPC * r];
        kk = fmaf(x, x, kk);
        vv = fmaf(y, y, vv);
        kv = fmaf(x, y, kv);
      }
      kk = col_sum(kk);
      vv = col_sum(vv);
      kv = col_sum(kv);
      // a token with a non-finite Cayley factor is the identity: M = 0 and its k, v rows
      // zeroed (each lane clears the elements it read; the stage is read after a barrier)
      bool ok;
      const cayley2 m = cayley_guarded(sdl[buf][tt], kk, vv, kv, ok);
      if (!ok) {
#pragma unroll
        for (int r = 0; r < RPT; ++r) sk[buf][tt][rg + LPC * r] = sv[buf][tt][rg + LPC * r] = 0.f;
        kk = vv = kv = 0.f;
      }
      if (rg == 0) {
        sco[buf][tt][0] = m.m00; sco[buf][tt][1] = m.m01;
        sco[buf][tt][2] = m.m10; sco[buf][tt][3] = m.m11;
        sco[buf][tt][4] = kk; sco[buf][tt][5] = kv; sco[buf][tt][6] = vv;
      }
    }
  };

  const int nst = (T + SB - 1) / SB;
  if (nst > 0) {
    fetch(0);
    commit(0);
  }
  __syncthreads();
  int par = 0;
  for (int s = 0; s < nst; ++s) {
    const int buf = s & 1;
    if (s + 1 < nst) fetch(s + 1);
    const int nt = min(SB, T - SB * s);
    for (int i = 0; i < nt; ++i) {
      const int t = T - 1 - (SB * s + i);
      float kr[RPT], vr[RPT], dr[RPT];
#pragma unroll
      for (int r = 0; r < RPT; ++r) {
        kr[r] = sk[buf][i][rg + LPC * r];
        vr[r] = sv[buf][i][rg + LPC * r];
        dr[r] = sdo[buf][i][rg + LPC * r];
      }
      const float qj = sq[buf][i][cl];
      const float m00 = sco[buf][i][0], m01 = sco[buf][i][1], m10 = sco[buf][i][2], m11 = sco[buf][i][3];
      const float kk = sco[buf][i][4], kv = sco[buf][i][5], vv = sco[buf][i][6];
      // readout of token t, then the column sums
      float a1 = 0.f, b1 = 0.f, dqs = 0.f, B0 = 0.f, B1 = 0.f;
#pragma unroll
      for (int r = 0; r < RPT; ++r) {
        lam[r] = fmaf(dr[r], qj, lam[r]);
        a1 = fmaf(kr[r], psi[r], a1);
        b1 = fmaf(vr[r], psi[r], b1);
        dqs = fmaf(dr[r], psi[r], dqs);
        B0 = fmaf(kr[r], lam[r], B0);
        B1 = fmaf(vr[r], lam[r], B1);
      }
      a1 = col_sum(a1);
      b1 = col_sum(b1);
      dqs = col_sum(dqs);
      B0 = col_sum(B0);
      B1 = col_sum(B1);
      if (rg == 0 && jv) io<IO>::store(dq, tok_index(t) * D + j, dqs);
      // Psi^(t) = R^T Psi^(t+1): alpha = M^T (U^T psi);  A = U^T Psi^(t) = U^T psi + G alpha
      const float al0 = m00 * a1 + m10 * b1, al1 = m01 * a1 + m11 * b1;
      const float A0 = a1 + kk * al0 + kv * al1, A1 = b1 + kv * al0 + vv * al1;
      // p = M A, rr = M^T B
      const float p0 = m00 * A0 + m01 * A1, p1 = m10 * A0 + m11 * A1;
      const float r0 = m00 * B0 + m10 * B1, r1 = m01 * B0 + m11 * B1;
      float u0[RPT], u1[RPT];
#pragma unroll
      for (int r = 0; r < RPT; ++r) {
        psi[r] = fmaf(kr[r], al0, fmaf(vr[r], al1, psi[r]));
        u0[r] = fmaf(lam[r], p0, psi[r] * r0);
        u1[r] = fmaf(lam[r], p1, psi[r] * r1);
        lam[r] = fmaf(kr[r], r0, fmaf(vr[r], r1, lam[r]));
      }
      // dU rows and dM summed over the wave's columns, then over the waves in LDS
      float dm[4] = {B0 * A0, B0 * A1, B1 * A0, B1 * A1};
      if (CPW == 2) {
#pragma unroll
        for (int r = 0; r < RPT; ++r) {
          u0[r] = half_pair_sum(u0[r]);
          u1[r] = half_pair_sum(u1[r]);
        }
#pragma unroll
        for (int x = 0; x < 4; ++x) dm[x] = half_pair_sum(dm[x]);
      }
      if (lane < LPC) {
#pragma unroll
        for (int r = 0; r < RPT; ++r) {
          sred[par][wave][2 * (rg + LPC * r)] = u0[r];
          sred[par][wave][2 * (rg + LPC * r) + 1] = u1[r];
        }
        if (lane < 4) sred[par][wave][2 * DP + lane] = dm[lane];
      }
      __syncthreads();
      float* pp = part + ((static_cast<int64_t>(bh) * T + t) * NBLK + blk) * PS;
      for (int x = tid; x < 2 * DP + 4; x += NT) {
        float acc = sred[par][0][x];
#pragma unroll
        for (int w = 1; w < NWV; ++w) acc += sred[par][w][x];
        pp[x] = acc;
      }
      par ^= 1;
    }
    if (s + 1 < nst) commit(s + 1);  // buffer (s + 1) & 1 was last read in stage s - 1
    __syncthreads();
  }
  if (dpsi0 && jv) {
#pragma unroll
    for (int r = 0; r < RPT; ++r) {
      const int row = rg + LPC * r;
      if (row < D) dpsi0[bh * DD + static_cast<int64_t>(row) * D + j] = lam[r];
    }
  }
}

// One wave per token-head (bh, t): dU = sum of the partials, dM; chain rule through
//   M = c N,  N = [[-P vv, P kv - h], [P kv + h, -P kk]],  P = h^2,  h = delta / 2,
//   c = 2 / (1 + P g),  g = kk vv - kv^2,
// then kk = k.k, vv = v.v, kv = k.v:  dk = dU_0 + 2 dkk k + dkv v,  dv = dU_1 + 2 dvv v + dkv k.
template <typename IO, int DP>
__global__ __launch_bounds__(256) void sssd_bwd_reduce_kernel(
    const IO* __restrict__ k, const IO* __restrict__ v, const void* __restrict__ delta,
    int delta_dtype, const float* __restrict__ part, IO* __restrict__ dk, IO* __restrict__ dv,
    void* __restrict__ ddelta, int T, int H, int BHT, int D) {
  constexpr int PS = Part<DP>::size;
  constexpr int NBLK = DP / CB;
  constexpr int RL = (DP + 63) / 64;  // rows per lane
  const int lane = threadIdx.x & 63;
  const int w = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (w >= BHT) return;  // whole wave
  const int bh = w / T, t = w % T;
  const int b = bh / H, hd = bh % H;
  const int64_t ti = (static_cast<int64_t>(b) * T + t) * H + hd;
  const float* pp = part + static_cast<int64_t>(w) * NBLK * PS;  // w = bh T + t

  float kr[RL], vr[RL], du0[RL], du1[RL];
  float kk = 0.f, vv = 0.f, kv = 0.f;
#pragma unroll
  for (int r = 0; r < RL; ++r) {
    const int i = lane + 64 * r;
    const bool ok = i < D;
    kr[r] = ok ? io<IO>::load(k, ti * D + i) : 0.f;
    vr[r] = ok ? io<IO>::load(v, ti * D + i) : 0.f;
    float s0 = 0.f, s1 = 0.f;
    if (ok) {
#pragma unroll
      for (int n = 0; n < NBLK; ++n) {
        s0 += pp[n * PS + 2 * i];
        s1 += pp[n * PS + 2 * i + 1];
      }
    }
    du0[r] = s0;
    du1[r] = s1;
    kk = fmaf(kr[r], kr[r], kk);
    vv = fmaf(vr[r], vr[r], vv);
    kv = fmaf(kr[r], vr[r], kv);
  }
  kk = half_pair_sum(row_pair_sum(row16_sum(kk)));
  vv = half_pair_sum(row_pair_sum(row16_sum(vv)));
  kv = half_pair_sum(row_pair_sum(row16_sum(kv)));
  float d00 = 0.f, d01 = 0.f, d10 = 0.f, d11 = 0.f;
#pragma unroll
  for (int n = 0; n < NBLK; ++n) {
    d00 += pp[n * PS + 2 * DP];
    d01 += pp[n * PS + 2 * DP + 1];
    d10 += pp[n * PS + 2 * DP + 2];
    d11 += pp[n * PS + 2 * DP + 3];
  }
  const float dl = load_scalar(delta, delta_dtype, ti);
  // a token with a non-finite Cayley factor was the identity in the forward: no gradient
  bool okm;
  (void)cayley_guarded(dl, kk, vv, kv, okm);
  const float hh = 0.5f * dl;
  const float P = hh * hh;
  const float graw = kk * vv - kv * kv;
  const float g = fmaxf(graw, 0.f);
  const float c = 2.f / (1.f + P * g);
  const float N00 = -P * vv, N01 = P * kv - hh, N10 = P * kv + hh, N11 = -P * kk;
  const float S = d00 * N00 + d01 * N01 + d10 * N10 + d11 * N11;  // dL/dc
  // through N
  float dh = c * (d01 * (2.f * hh * kv - 1.f) + d10 * (2.f * hh * kv + 1.f) - 2.f * hh * (d00 * vv + d11 * kk));
  float dvv = -c * P * d00, dkk = -c * P * d11, dkv = c * P * (d01 + d10);
  // through c (g clamped at 0 has no gradient)
  dh += S * (-c * c * hh * g);
  const float dg = graw > 0.f ? S * (-0.5f * c * c * P) : 0.f;
  dkk += dg * vv;
  dvv += dg * kk;
  dkv += -2.f * dg * kv;
#pragma unroll
  for (int r = 0; r < RL; ++r) {
    const int i = lane + 64 * r;
    if (i < D) {
      io<IO>::store(dk, ti * D + i, okm ? du0[r] + 2.f * dkk * kr[r] + dkv * vr[r] : 0.f);
      io<IO>::store(dv, ti * D + i, okm ? du1[r] + 2.f * dvv * vr[r] + dkv * kr[r] : 0.f);
    }
  }
  if (lane == 0) {
    const float dd = okm ? 0.5f * dh : 0.f;
    if (delta_dtype == VMI_F32) static_cast<float*>(ddelta)[ti] = dd;
    else if (delta_dtype == VMI_BF16) static_cast<uint16_t*>(ddelta)[ti] = f32_to_bf16(dd);
    else static_cast<f16_t*>(ddelta)[ti] = static_cast<f16_t>(dd);
  }
}

template <typename IO, typename GO, int DP>
hipError_t launch_d(const void* q, const void* k, const void* v, const void* delta,
                    int delta_dtype, const float* psi_T, const void* dout, const float* dpsi_T,
                    void* dq, void* dk, void* dv, void* ddelta, float* dpsi0, int B, int T,
                    int H, int D, void* ws, hipStream_t stream) {
  float* part = static_cast<float*>(ws);
  hipLaunchKernelGGL((sssd_bwd_cols_kernel<IO, GO, DP>), dim3(DP / CB, B * H), dim3(NT), 0, stream,
                     static_cast<const IO*>(q), static_cast<const IO*>(k),
                     static_cast<const IO*>(v), delta, delta_dtype, psi_T,
                     static_cast<const GO*>(dout), dpsi_T, static_cast<IO*>(dq), dpsi0, part, T, H, D);
  hipError_t e = hipGetLastError();
  const int BHT = B * H * T;
  if (e != hipSuccess || BHT == 0) return e;
  hipLaunchKernelGGL((sssd_bwd_reduce_kernel<IO, DP>), dim3((BHT + 3) / 4), dim3(256), 0, stream,
                     static_cast<const IO*>(k), static_cast<const IO*>(v), delta, delta_dtype,
                     part, static_cast<IO*>(dk), static_cast<IO*>(dv), ddelta, T, H, BHT, D);
  return hipGetLastError();
}

template <typename IO, typename GO>
hipError_t launch_go(const void* q, const void* k, const void* v, const void* delta,
                     int delta_dtype, const float* psi_T, const void* dout, const float* dpsi_T,
                     void* dq, void* dk, void* dv, void* ddelta, float* dpsi0, int B, int T,
                     int H, int D, void* ws, hipStream_t stream) {
#define VMI_BWD_D(DP)                                                                      \
  return launch_d<IO, GO, DP>(q, k, v, delta, delta_dtype, psi_T, dout, dpsi_T, dq, dk, dv, \
                              ddelta, dpsi0, B, T, H, D, ws, stream)
  if (D <= 32) VMI_BWD_D(32);
  if (D <= 64) VMI_BWD_D(64);
  if (D <= 128) VMI_BWD_D(128);
  VMI_BWD_D(256);
#undef VMI_BWD_D
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

}  // namespace bwd

bool sssd_bwd_supported(int64_t D) { return D >= 1 && D <= 256; }

size_t sssd_bwd_workspace_bytes(int64_t B, int64_t T, int64_t H, int64_t D) {
  const int64_t DP = D <= 32 ? 32 : D <= 64 ? 64 : D <= 128 ? 128 : 256;
  return static_cast<size_t>(B * H * T * (DP / bwd::CB)) * (2 * DP + 8) * sizeof(float);
}

hipError_t launch_sssd_bwd(const void* q, const void* k, const void* v, const void* delta,
                           int io_dtype, int delta_dtype, const float* psi_T, const void* dout,
                           int dout_dtype, const float* dpsi_T, void* dq, void* dk, void* dv,
                           void* ddelta, float* dpsi0, int B, int T, int H, int D, void* ws,
                           hipStream_t stream) {
  if (io_dtype == VMI_F32)
    return bwd::launch_io<float>(q, k, v, delta, delta_dtype, psi_T, dout, dout_dtype, dpsi_T, dq,
                                 dk, dv, ddelta, dpsi0, B, T, H, D, ws, stream);
  if (io_dtype == VMI_BF16)
    return bwd::launch_io<bf16_t>(q, k, v, delta, delta_dtype, psi_T, dout, dout_dtype, dpsi_T,
                                  dq, dk, dv, ddelta, dpsi0, B, T, H, D, ws, stream);
  return bwd::launch_io<f16_t>(q, k, v, delta, delta_dtype, psi_T, dout, dout_dtype, dpsi_T, dq,
                               dk, dv, ddelta, dpsi0, B, T, H, D, ws, stream);
}

}  // namespace vmi
