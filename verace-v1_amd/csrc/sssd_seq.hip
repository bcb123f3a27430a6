// Token-sequential SSSD scan, fp32 arithmetic, one workgroup per (batch, head).
//
// This is the path for fp32 I/O, small problems, head_dim other than 128 and
// the single-token decode step.  The state Psi (D x D fp32) lives in VGPRs for
// the whole scan: thread (rg, cg) owns rows {rg + RG*m} and the four columns
// 4cg..4cg+3, so loads and stores of Psi are float4 and fully coalesced.
//
// Per token t (reference: sssd_attention.py:160-175, applied one step at a
// time in closed form instead of solve + prefix product):
//   a = k^T Psi, b = v^T Psi          column sums: per-thread partials over its
//                                     rows, reduced across row groups in LDS
//   Psi += k alpha + v beta           alpha, beta from the closed-form Cayley
//                                     coefficients (vmi::cayley_coeffs)
//   o = Psi q                         row sums: per-thread partials over its 4
//                                     columns, reduce-scattered across the CG
//                                     lanes of the row group with xor shuffles
// One workgroup barrier per token.  The next token's q/k/v are staged into a
// second LDS buffer while the current one is processed.
#include "vmi_common.h"
#include "vmi_dispatch.h"

namespace vmi {

template <int DMAX>
struct seq_cfg {
  static constexpr int CG = DMAX / 4;        // column groups (4 columns each)
  static constexpr int RG = 8;               // row groups
  static constexpr int NT = CG * RG;         // threads per workgroup
  static constexpr int RPT = DMAX / RG;      // rows per thread
  static_assert(RPT * 2 == CG, "reduce-scatter layout needs RPT == CG/2");
};

template <typename IO, int DMAX, typename Map>
__global__ __launch_bounds__(seq_cfg<DMAX>::NT) void sssd_seq_kernel(
    const IO* __restrict__ q, const IO* __restrict__ k, const IO* __restrict__ v,
    const void* __restrict__ delta, int delta_dtype, const float* psi_in,
    IO* __restrict__ out, float* psi_out, Map map, int T, int H, int D) {
  using C = seq_cfg<DMAX>;
  constexpr int CG = C::CG, RG = C::RG, RPT = C::RPT, NT = C::NT;

  const int tid = threadIdx.x;
  const int cg = tid % CG;
  const int rg = tid / CG;
  const int bh = blockIdx.x;          // b * H + h
  if (map.skip(bh)) return;           // uniform over the workgroup
  const int b = bh / H;
  const int h = bh - b * H;
  const int64_t DD = static_cast<int64_t>(D) * D;
  const int64_t si = psi_in != nullptr ? map.in_index(bh, H) : -1;  // < 0: identity
  const int64_t di = map.out_index(bh, H);                         // < 0: no state write

  // staged token: q, k, v (fp32) and delta; double buffered
  __shared__ float s_tok[2][3][DMAX];
  __shared__ float s_delta[2];
  // column-sum partials of a and b, double buffered
  __shared__ float s_red[2][2][RG][DMAX];

  // ---- load Psi ----
  float psi[RPT][4];
  const int c0 = 4 * cg;
#pragma unroll
  for (int m = 0; m < RPT; ++m) {
    const int r = rg + RG * m;
#pragma unroll
    for (int j = 0; j < 4; ++j) psi[m][j] = 0.0f;
    if (r < D) {
      if (si >= 0) {
        const float* src = psi_in + si * DD + static_cast<int64_t>(r) * D;
        if ((D & 3) == 0 && c0 < D) {
          const float4 x = *reinterpret_cast<const float4*>(src + c0);
          psi[m][0] = x.x; psi[m][1] = x.y; psi[m][2] = x.z; psi[m][3] = x.w;
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j)
            if (c0 + j < D) psi[m][j] = src[c0 + j];
        }
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) psi[m][j] = (r == c0 + j) ? 1.0f : 0.0f;
      }
    }
  }

  // token element (b, t, h, d) lives at ((b*T + t)*H + h)*D + d
  const int64_t tok_stride = static_cast<int64_t>(H) * D;
  const int64_t base = (static_cast<int64_t>(b) * T * H + h) * D;
  const int64_t dbase = static_cast<int64_t>(b) * T * H + h;

  // each thread stages elements e = tid, tid + NT, ... of the 3*DMAX token row
  constexpr int NSTAGE = (3 * DMAX + NT - 1) / NT;
  float stage[NSTAGE];
  float stage_delta = 0.0f;

  auto fetch = [&](int t) {
#pragma unroll
    for (int s = 0; s < NSTAGE; ++s) {
      const int e = tid + s * NT;
      const int which = e / DMAX;
      const int d = e - which * DMAX;
      float x = 0.0f;
      if (which < 3 && d < D) {
        const IO* src = which == 0 ? q : (which == 1 ? k : v);
        x = io<IO>::load(src, base + t * tok_stride + d);
      }
      stage[s] = x;
    }
    if (tid == 0) stage_delta = load_scalar(delta, delta_dtype, dbase + static_cast<int64_t>(t) * H);
  };
  auto commit = [&](int buf) {
#pragma unroll
    for (int s = 0; s < NSTAGE; ++s) {
      const int e = tid + s * NT;
      if (e < 3 * DMAX) (&s_tok[buf][0][0])[e] = stage[s];
    }
    if (tid == 0) s_delta[buf] = stage_delta;
  };

  if (T > 0) {
    fetch(0);
    commit(0);
  }
  __syncthreads();

  const int lane = tid & 63;
  for (int t = 0; t < T; ++t) {
    const int cur = t & 1;
    if (t + 1 < T) fetch(t + 1);

    // this thread's slices of k, v (rows) and q (columns)
    float kr[RPT], vr[RPT];
#pragma unroll
    for (int m = 0; m < RPT; ++m) {
      kr[m] = s_tok[cur][1][rg + RG * m];
      vr[m] = s_tok[cur][2][rg + RG * m];
    }
    float qc[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) qc[j] = s_tok[cur][0][c0 + j];

    // Gram entries |k|^2, |v|^2, k.v: every wave reduces the full vectors
    float kk = 0.f, vv = 0.f, kv = 0.f;
    for (int d = lane; d < DMAX; d += 64) {
      const float kd = s_tok[cur][1][d], vd = s_tok[cur][2][d];
      kk = fmaf(kd, kd, kk);
      vv = fmaf(vd, vd, vv);
      kv = fmaf(kd, vd, kv);
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      kk += __shfl_xor(kk, off);
      vv += __shfl_xor(vv, off);
      kv += __shfl_xor(kv, off);
    }
    // a token with a non-finite Cayley factor is the identity (uniform over the workgroup)
    bool ok;
    const cayley2 M = cayley_guarded(s_delta[cur], kk, vv, kv, ok);
    if (!ok) {
#pragma unroll
      for (int m = 0; m < RPT; ++m) kr[m] = vr[m] = 0.f;
    }

    // column-sum partials a_j = sum_i k_i Psi_ij, b_j = sum_i v_i Psi_ij
    float pa[4] = {0.f, 0.f, 0.f, 0.f}, pb[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int m = 0; m < RPT; ++m) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        pa[j] = fmaf(kr[m], psi[m][j], pa[j]);
        pb[j] = fmaf(vr[m], psi[m][j], pb[j]);
      }
    }
    *reinterpret_cast<float4*>(&s_red[cur][0][rg][c0]) = make_float4(pa[0], pa[1], pa[2], pa[3]);
    *reinterpret_cast<float4*>(&s_red[cur][1][rg][c0]) = make_float4(pb[0], pb[1], pb[2], pb[3]);
    if (t + 1 < T) commit(cur ^ 1);
    __syncthreads();

    float a[4] = {0.f, 0.f, 0.f, 0.f}, bb[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int g = 0; g < RG; ++g) {
      const float4 xa = *reinterpret_cast<const float4*>(&s_red[cur][0][g][c0]);
      const float4 xb = *reinterpret_cast<const float4*>(&s_red[cur][1][g][c0]);
      a[0] += xa.x; a[1] += xa.y; a[2] += xa.z; a[3] += xa.w;
      bb[0] += xb.x; bb[1] += xb.y; bb[2] += xb.z; bb[3] += xb.w;
    }
    float al[4], be[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      al[j] = fmaf(M.m00, a[j], M.m01 * bb[j]);
      be[j] = fmaf(M.m10, a[j], M.m11 * bb[j]);
    }
    // update and row-sum partials of o = Psi q
    float po[RPT];
#pragma unroll
    for (int m = 0; m < RPT; ++m) {
      float acc = 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        psi[m][j] = fmaf(kr[m], al[j], fmaf(vr[m], be[j], psi[m][j]));
        acc = fmaf(psi[m][j], qc[j], acc);
      }
      po[m] = acc;
    }
    // reduce-scatter po[] over the CG lanes of this row group
    int cnt = RPT;
    int mloc = 0;
#pragma unroll
    for (int off = CG / 2; off >= 2; off >>= 1) {
      const int half = cnt >> 1;
      const bool hi = (lane & off) != 0;
#pragma unroll
      for (int i = 0; i < RPT / 2; ++i) {
        if (i < half) {
          const float send = hi ? po[i] : po[i + half];
          const float keep = hi ? po[i + half] : po[i];
          po[i] = keep + __shfl_xor(send, off);
        }
      }
      if (hi) mloc += half;
      cnt = half;
    }
    const float o_row = po[0] + __shfl_xor(po[0], 1);
    const int r = rg + RG * mloc;
    if (out != nullptr && (lane & 1) == 0 && r < D)
      io<IO>::store(out, base + t * tok_stride + r, o_row);
  }

  // ---- store Psi ----
#pragma unroll
  for (int m = 0; m < RPT; ++m) {
    const int r = rg + RG * m;
    if (r < D && (!Map::kSlotted || di >= 0)) {
      float* dst = psi_out + di * DD + static_cast<int64_t>(r) * D;
      if ((D & 3) == 0 && c0 < D) {
        *reinterpret_cast<float4*>(dst + c0) = make_float4(psi[m][0], psi[m][1], psi[m][2], psi[m][3]);
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (c0 + j < D) dst[c0 + j] = psi[m][j];
      }
    }
  }
}

// Host-side launcher: picks the smallest DMAX >= D.
template <typename IO, typename Map>
hipError_t launch_sssd_seq_typed(const void* q, const void* k, const void* v, const void* delta,
                                 int delta_dtype, const float* psi_in, void* out, float* psi_out,
                                 int B, int T, int H, int D, hipStream_t stream, const Map& map) {
  const dim3 grid(B * H);
  const IO* qq = static_cast<const IO*>(q);
  const IO* kk = static_cast<const IO*>(k);
  const IO* vv = static_cast<const IO*>(v);
  IO* oo = static_cast<IO*>(out);
  if (D <= 32) {
    hipLaunchKernelGGL((sssd_seq_kernel<IO, 32, Map>), grid, dim3(seq_cfg<32>::NT), 0, stream, qq,
                       kk, vv, delta, delta_dtype, psi_in, oo, psi_out, map, T, H, D);
  } else if (D <= 64) {
    hipLaunchKernelGGL((sssd_seq_kernel<IO, 64, Map>), grid, dim3(seq_cfg<64>::NT), 0, stream, qq,
                       kk, vv, delta, delta_dtype, psi_in, oo, psi_out, map, T, H, D);
  } else if (D <= 128) {
    hipLaunchKernelGGL((sssd_seq_kernel<IO, 128, Map>), grid, dim3(seq_cfg<128>::NT), 0, stream,
                       qq, kk, vv, delta, delta_dtype, psi_in, oo, psi_out, map, T, H, D);
  } else {
    hipLaunchKernelGGL((sssd_seq_kernel<IO, 256, Map>), grid, dim3(seq_cfg<256>::NT), 0, stream,
                       qq, kk, vv, delta, delta_dtype, psi_in, oo, psi_out, map, T, H, D);
  }
  return hipGetLastError();
}

template <typename Map>
hipError_t launch_seq_map(const void* q, const void* k, const void* v, const void* delta,
                          int io_dtype, int delta_dtype, const float* psi_in, void* out,
                          float* psi_out, int B, int T, int H, int D, hipStream_t stream,
                          const Map& map) {
  if (io_dtype == VMI_F32)
    return launch_sssd_seq_typed<float, Map>(q, k, v, delta, delta_dtype, psi_in, out, psi_out, B,
                                             T, H, D, stream, map);
  if (io_dtype == VMI_BF16)
    return launch_sssd_seq_typed<bf16_t, Map>(q, k, v, delta, delta_dtype, psi_in, out, psi_out,
                                              B, T, H, D, stream, map);
  return launch_sssd_seq_typed<f16_t, Map>(q, k, v, delta, delta_dtype, psi_in, out, psi_out, B,
                                           T, H, D, stream, map);
}

hipError_t launch_sssd_seq(const void* q, const void* k, const void* v, const void* delta,
                           int io_dtype, int delta_dtype, const float* psi_in, void* out,
                           float* psi_out, int B, int T, int H, int D, hipStream_t stream) {
  return launch_seq_map(q, k, v, delta, io_dtype, delta_dtype, psi_in, out, psi_out, B, T, H, D,
                        stream, DenseStates{});
}

hipError_t launch_sssd_seq(const void* q, const void* k, const void* v, const void* delta,
                           int io_dtype, int delta_dtype, const float* psi_in, void* out,
                           float* psi_out, int B, int T, int H, int D, hipStream_t stream,
                           const StateMap& map) {
  return launch_seq_map(q, k, v, delta, io_dtype, delta_dtype, psi_in, out, psi_out, B, T, H, D,
                        stream, map);
}

hipError_t launch_sssd_seq(const void* q, const void* k, const void* v, const void* delta,
                           int io_dtype, int delta_dtype, const float* psi_in, void* out,
                           float* psi_out, int B, int T, int H, int D, hipStream_t stream,
                           const SlotArgs& map) {
  return launch_seq_map(q, k, v, delta, io_dtype, delta_dtype, psi_in, out, psi_out, B, T, H, D,
                        stream, map);
}

hipError_t launch_sssd_seq(const void* q, const void* k, const void* v, const void* delta,
                           int io_dtype, int delta_dtype, const float* psi_in, void* out,
                           float* psi_out, int B, int T, int H, int D, hipStream_t stream,
                           const FlaggedStates& map) {
  return launch_seq_map(q, k, v, delta, io_dtype, delta_dtype, psi_in, out, psi_out, B, T, H, D,
                        stream, map);
}

}  // namespace vmi
