// Single-token SSSD step (decode) for head_dim 128: Psi' = R Psi, o = Psi' q.
//
// The step is bound by HBM traffic: every (batch, head) state (64 KiB fp32) is read
// once and written once, while the arithmetic is ~10 D^2 flops.  Nothing of a column
// can be written before the whole column has been read (a = k^T Psi and b = v^T Psi are
// sums over its rows), but columns are independent of each other until the output
// o = Psi' q, which sums over them.  A head is therefore processed as two units of 64
// columns: the first unit's update and store go out while the second unit's loads are
// still in flight, and o accumulates over the units in registers.  Workgroups are
// persistent, two per CU (so the reduce and barrier phases of one overlap the memory
// traffic of the other): workgroup w handles heads w, w + G, ..., and the loads of the
// next unit (of this head, or unit 0 of the next head) are issued before the current
// unit is reduced, updated and stored.  Measured at DEC (B64 H8, 12 rotating layers of
// states updated in place): 12.6 us per layer against 14.1 us for whole-head units on
// one workgroup per CU; a plain read-modify-write stream of the same bytes takes 12.0 us.
//
// Layout of a unit: thread (rg, cg), rg = tid / 16, cg = tid % 16, owns rows rg + 16m
// (m = 0..7) and the unit's columns 4cg .. 4cg+3, so every state load and store is a
// coalesced float4 (a 256-byte row segment per 16 lanes).  Per unit (reference recurrence
// sssd_attention.py:160-175 at seq_len 1, closed form):
//   a = k^T Psi, b = v^T Psi     per-thread partials over 8 rows, combined across the
//                                four row groups of a wave with lane swaps and across
//                                the four waves in LDS
//   Psi += k alpha + v beta      alpha, beta from vmi::cayley_coeffs (once per head)
//   o += Psi q                   row partials over this unit's columns; after the last
//                                unit reduce-scattered over the 16 lanes of a row group
// Where a head's state is read and written is the Map template parameter
// (vmi_dispatch.h): the dense [B, H, D, D] layout, or slots of a decode state cache
// (state_cache.hip), which may differ between read and write (copy-on-write).
#include "vmi_common.h"
#include "vmi_dispatch.h"

namespace vmi {
namespace step {

constexpr int D = 128;
constexpr int NT = 256;
constexpr int UC = 64;            // state columns per unit
constexpr int NU = D / UC;        // units per head
constexpr int CG = UC / 4;        // float4 column groups per unit
constexpr int RG = NT / CG;       // row groups
constexpr int RPT = D / RG;       // rows per thread
constexpr int WG_PER_CU = 2;
static_assert(RPT == CG / 2, "the o reduce-scatter leaves one row per lane pair");
static_assert(NU % 2 == 0, "units alternate two register buffers and two LDS buffers");

// Fused decode step (FUSED = true; reference sssd_attention.py:114-126 and :177 at seq_len 1):
// q, k, v and the delta logit of item b are read from row b of the stacked projection
// proj = x [W_q; W_k; W_v; W_delta]^T (passed as q; row stride `stride` elements): q of head
// h at h D, k at H D + h D, v at 2 H D + h D, the logit at 3 H D + h.  q, k, v are
// L2-normalised in the kernel (F.normalize: x / max(|x|, 1e-12), in fp32), delta =
// 0.1 sigmoid(logit) mask[b], and with rms_w the output is head_rmsnorm(o) =
// o rsqrt(mean(o^2) + rms_eps) rms_w.
struct StepFused {
  int64_t stride;
  const uint8_t* mask;  // per item (null: every item active)
  const float* rms_w;   // [D] (null: o stored as computed)
  float rms_eps;
};

template <typename IO, typename Map, bool FUSED>
__global__ __launch_bounds__(NT, WG_PER_CU) void sssd_step128_kernel(
    const IO* __restrict__ q, const IO* __restrict__ k, const IO* __restrict__ v,
    const void* __restrict__ delta, int delta_dtype, const float* psi_in, IO* __restrict__ out,
    float* psi_out, Map map, int BH, int H, StepFused fz) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int cg = tid % CG, rg = tid / CG;
  const int c0 = 4 * cg;
  constexpr int64_t DD = static_cast<int64_t>(D) * D;

  __shared__ float s_tok[2][3][D];          // q, k, v (fp32) of the head, x2 (head parity)
  __shared__ float s_delta[2];
  __shared__ float4 s_red[2][4][2][CG];     // per wave: a and b partials, x2 (unit parity)
  __shared__ float s_rms[4];                // fused RMSNorm: per-wave sums of o^2

  // state of the current and the next unit (double-buffered registers)
  float4 sa[RPT], sb[RPT];
  // this thread's share of the next head's q/k/v row (elements tid and tid + 256 of
  // the 384-element concatenation) and its delta
  float tk0 = 0.f, tk1 = 0.f, tdl = 0.f, tmk = 1.f;

  auto load_unit = [&](float4* st, int bh, int u) {
    const int64_t si = psi_in != nullptr ? map.in_index(bh, H) : -1;  // uniform; < 0: identity
    const int cb = UC * u + c0;
    if (si >= 0) {
      const float* src = psi_in + si * DD + cb;
#pragma unroll
      for (int m = 0; m < RPT; ++m) st[m] = ld_stream4(src + (rg + RG * m) * D);
    } else {
#pragma unroll
      for (int m = 0; m < RPT; ++m) {
        const int r = rg + RG * m;
        st[m] = make_float4(r == cb ? 1.f : 0.f, r == cb + 1 ? 1.f : 0.f, r == cb + 2 ? 1.f : 0.f,
                            r == cb + 3 ? 1.f : 0.f);
      }
    }
  };
  auto load_tok = [&](int bh) {
    if constexpr (FUSED) {
      const int b = bh / H, hh = bh - b * H;
      const int64_t row = static_cast<int64_t>(b) * fz.stride + static_cast<int64_t>(hh) * D;
      const int64_t HD = static_cast<int64_t>(H) * D;
      tk0 = io<IO>::load(q, row + (tid < D ? 0 : HD) + (tid & (D - 1)));
      if (tid < D) tk1 = io<IO>::load(q, row + 2 * HD + tid);
      if (tid == 0) {
        tdl = io<IO>::load(q, static_cast<int64_t>(b) * fz.stride + 3 * HD + hh);
        tmk = fz.mask != nullptr ? static_cast<float>(fz.mask[b]) : 1.f;
      }
    } else {
      // element e of [q | k | v] for head bh lives at bh*D + (e % D) of array e / D
      const int64_t base = static_cast<int64_t>(bh) * D;
      tk0 = io<IO>::load(tid < D ? q : k, base + (tid & (D - 1)));
      if (tid < D) tk1 = io<IO>::load(v, base + tid);
      if (tid == 0) tdl = load_scalar(delta, delta_dtype, bh);
    }
  };
  auto commit_tok = [&](int buf) {
    (&s_tok[buf][0][0])[tid] = tk0;
    if (tid < D) s_tok[buf][2][tid] = tk1;
    // fused: 0.1 sigmoid(logit) * mask (a NaN logit stays NaN, so the guard below applies)
    if (tid == 0) s_delta[buf] = FUSED ? 0.1f / (1.f + expf(-tdl)) * tmk : tdl;
  };

  float kr[RPT], vr[RPT];  // k and v at this thread's rows (zero for a guarded token)
  float qn = 1.f;          // fused: 1 / |q|
  cayley2 M;
  // the o row this lane ends up holding after the reduce-scatter below (rg + RG * mrow,
  // in the even lanes); fused: its RMSNorm weight, loaded once here (loaded after a head's
  // state stores, its wait would also wait for those stores)
  int mrow = 0;
#pragma unroll
  for (int off = CG / 2, cnt = RPT; off >= 2; off >>= 1, cnt >>= 1)
    if (lane & off) mrow += cnt >> 1;
  float rw = 1.f;
  if constexpr (FUSED) {
    if (fz.rms_w != nullptr) rw = fz.rms_w[rg + RG * mrow];
  }
  float po[RPT];           // o partials at this thread's rows, summed over units

  // unit u of head bh: columns UC u .. UC u + UC - 1 in st, q/k/v in s_tok[buf]
  auto process = [&](float4* st, int bh, int u, int buf) {
    if (u == 0) {
#pragma unroll
      for (int m = 0; m < RPT; ++m) {
        kr[m] = s_tok[buf][1][rg + RG * m];
        vr[m] = s_tok[buf][2][rg + RG * m];
      }
      // Gram entries, reduced by every wave over the full vectors
      const float k0 = s_tok[buf][1][lane], k1 = s_tok[buf][1][lane + 64];
      const float v0 = s_tok[buf][2][lane], v1 = s_tok[buf][2][lane + 64];
      float kk = fmaf(k0, k0, k1 * k1);
      float vv = fmaf(v0, v0, v1 * v1);
      float kv = fmaf(k0, v0, k1 * v1);
      float qq = 0.f;
      if constexpr (FUSED) {
        const float q0 = s_tok[buf][0][lane], q1 = s_tok[buf][0][lane + 64];
        qq = fmaf(q0, q0, q1 * q1);
      }
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) {
        kk += __shfl_xor(kk, off);
        vv += __shfl_xor(vv, off);
        kv += __shfl_xor(kv, off);
        if constexpr (FUSED) qq += __shfl_xor(qq, off);
      }
      if constexpr (FUSED) {  // the Gram entries and rows of the normalised k, v
        const float nk = 1.f / fmaxf(sqrtf(kk), 1e-12f), nv = 1.f / fmaxf(sqrtf(vv), 1e-12f);
        qn = 1.f / fmaxf(sqrtf(qq), 1e-12f);
        kv = kv * nk * nv;
        kk = kk * nk * nk;
        vv = vv * nv * nv;
#pragma unroll
        for (int m = 0; m < RPT; ++m) {
          kr[m] *= nk;
          vr[m] *= nv;
        }
      }
      // a token with a non-finite Cayley factor is the identity (uniform over the workgroup)
      bool ok;
      M = cayley_guarded(s_delta[buf], kk, vv, kv, ok);
      if (!ok) {
#pragma unroll
        for (int m = 0; m < RPT; ++m) kr[m] = vr[m] = 0.f;
      }
    }
    float4 qc = *reinterpret_cast<const float4*>(&s_tok[buf][0][UC * u + c0]);
    if constexpr (FUSED) {
      qc.x *= qn; qc.y *= qn; qc.z *= qn; qc.w *= qn;
    }
    // column partials over this thread's rows
    float4 pa = make_float4(0.f, 0.f, 0.f, 0.f), pb = pa;
#pragma unroll
    for (int m = 0; m < RPT; ++m) {
      pa.x = fmaf(kr[m], st[m].x, pa.x); pa.y = fmaf(kr[m], st[m].y, pa.y);
      pa.z = fmaf(kr[m], st[m].z, pa.z); pa.w = fmaf(kr[m], st[m].w, pa.w);
      pb.x = fmaf(vr[m], st[m].x, pb.x); pb.y = fmaf(vr[m], st[m].y, pb.y);
      pb.z = fmaf(vr[m], st[m].z, pb.z); pb.w = fmaf(vr[m], st[m].w, pb.w);
    }
    // lanes cg + CG j of a wave hold its row groups j of the same columns
#pragma unroll
    for (int off = CG; off < 64; off <<= 1) {
      pa.x += __shfl_xor(pa.x, off); pa.y += __shfl_xor(pa.y, off);
      pa.z += __shfl_xor(pa.z, off); pa.w += __shfl_xor(pa.w, off);
      pb.x += __shfl_xor(pb.x, off); pb.y += __shfl_xor(pb.y, off);
      pb.z += __shfl_xor(pb.z, off); pb.w += __shfl_xor(pb.w, off);
    }
    if (lane < CG) {
      s_red[u & 1][wave][0][cg] = pa;
      s_red[u & 1][wave][1][cg] = pb;
    }
    __syncthreads();
    float4 a4 = s_red[u & 1][0][0][cg], b4 = s_red[u & 1][0][1][cg];
#pragma unroll
    for (int w = 1; w < 4; ++w) {
      const float4 xa = s_red[u & 1][w][0][cg], xb = s_red[u & 1][w][1][cg];
      a4.x += xa.x; a4.y += xa.y; a4.z += xa.z; a4.w += xa.w;
      b4.x += xb.x; b4.y += xb.y; b4.z += xb.z; b4.w += xb.w;
    }
    const float4 al = make_float4(fmaf(M.m00, a4.x, M.m01 * b4.x), fmaf(M.m00, a4.y, M.m01 * b4.y),
                                  fmaf(M.m00, a4.z, M.m01 * b4.z), fmaf(M.m00, a4.w, M.m01 * b4.w));
    const float4 be = make_float4(fmaf(M.m10, a4.x, M.m11 * b4.x), fmaf(M.m10, a4.y, M.m11 * b4.y),
                                  fmaf(M.m10, a4.z, M.m11 * b4.z), fmaf(M.m10, a4.w, M.m11 * b4.w));
    // update, store, and row partials of o = Psi' q
    const int64_t di = map.out_index(bh, H);  // uniform; < 0 (slotted maps only): not written
    float* dst = psi_out + (di < 0 ? 0 : di) * DD + UC * u + c0;
#pragma unroll
    for (int m = 0; m < RPT; ++m) {
      float4 x = st[m];
      x.x = fmaf(kr[m], al.x, fmaf(vr[m], be.x, x.x));
      x.y = fmaf(kr[m], al.y, fmaf(vr[m], be.y, x.y));
      x.z = fmaf(kr[m], al.z, fmaf(vr[m], be.z, x.z));
      x.w = fmaf(kr[m], al.w, fmaf(vr[m], be.w, x.w));
      if (!Map::kSlotted || di >= 0) st_stream4(dst + (rg + RG * m) * D, x);
      const float p = fmaf(x.x, qc.x, fmaf(x.y, qc.y, fmaf(x.z, qc.z, x.w * qc.w)));
      po[m] = u == 0 ? p : po[m] + p;
    }
    if (u == NU - 1) {
      // reduce-scatter po[] over the CG lanes of this row group: after the halving
      // steps lane cg holds the sum for row rg + RG*mrow, paired with lane cg^1
#pragma unroll
      for (int off = CG / 2, cnt = RPT; off >= 2; off >>= 1, cnt >>= 1) {
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
      }
      float o_row = po[0] + __shfl_xor(po[0], 1);
      const int row = rg + RG * mrow;  // each row held by exactly one even lane
      if constexpr (FUSED) {
        if (fz.rms_w != nullptr) {  // uniform: head RMSNorm over the head's D rows
          float ss = (lane & 1) == 0 ? o_row * o_row : 0.f;
#pragma unroll
          for (int off = 32; off >= 1; off >>= 1) ss += __shfl_xor(ss, off);
          if (lane == 0) s_rms[wave] = ss;
          __syncthreads();
          const float tot = (s_rms[0] + s_rms[1]) + (s_rms[2] + s_rms[3]);
          o_row *= rsqrtf(tot * (1.f / D) + fz.rms_eps) * rw;
        }
      }
      if (out != nullptr && (lane & 1) == 0)
        io<IO>::store(out, static_cast<int64_t>(bh) * D + row, o_row);
    }
  };

  const int G = gridDim.x;
  int bh = blockIdx.x;
  if (bh >= BH) return;  // uniform
  int buf = 0;
  load_unit(sa, bh, 0);
  load_tok(bh);
  commit_tok(0);
  // units alternate the register buffers sa / sb and the s_red buffers; heads alternate
  // the s_tok buffers.  The next unit's loads are issued before the barrier that
  // publishes this head's q/k/v (issuing them after it measured 1.2 us slower).
  for (;;) {
    const int bh1 = bh + G;
#pragma unroll
    for (int u = 0; u < NU; ++u) {
      float4* cur = (u & 1) ? sb : sa;
      float4* nxt = (u & 1) ? sa : sb;
      if (u + 1 < NU) {
        load_unit(nxt, bh, u + 1);
      } else if (bh1 < BH) {
        load_unit(nxt, bh1, 0);
        load_tok(bh1);
      }
      if (u == 0) __syncthreads();  // s_tok[buf] complete; s_red free
      process(cur, bh, u, buf);
    }
    if (bh1 >= BH) break;
    commit_tok(buf ^ 1);
    buf ^= 1;
    bh = bh1;
  }
}

template <typename IO, typename Map, bool FUSED = false>
hipError_t launch_typed(const void* q, const void* k, const void* v, const void* delta,
                        int delta_dtype, const float* psi_in, void* out, float* psi_out,
                        const Map& map, int BH, int H, hipStream_t stream,
                        const StepFused& fz = StepFused{}) {
  int cus = 0;
  hipError_t e = device_cu_count(&cus);
  if (e != hipSuccess) return e;
  const int grid = BH < WG_PER_CU * cus ? BH : WG_PER_CU * cus;
  hipLaunchKernelGGL((sssd_step128_kernel<IO, Map, FUSED>), dim3(grid), dim3(NT), 0, stream,
                     static_cast<const IO*>(q), static_cast<const IO*>(k),
                     static_cast<const IO*>(v), delta, delta_dtype, psi_in, static_cast<IO*>(out),
                     psi_out, map, BH, H, fz);
  return hipGetLastError();
}

template <typename Map>
hipError_t launch_map(const void* q, const void* k, const void* v, const void* delta, int io_dtype,
                      int delta_dtype, const float* psi_in, void* out, float* psi_out,
                      const Map& map, int B, int H, hipStream_t stream) {
  const int BH = B * H;
  if (io_dtype == VMI_F32)
    return launch_typed<float, Map>(q, k, v, delta, delta_dtype, psi_in, out, psi_out, map, BH, H,
                                    stream);
  if (io_dtype == VMI_BF16)
    return launch_typed<bf16_t, Map>(q, k, v, delta, delta_dtype, psi_in, out, psi_out, map, BH,
                                     H, stream);
  return launch_typed<f16_t, Map>(q, k, v, delta, delta_dtype, psi_in, out, psi_out, map, BH, H,
                                  stream);
}

}  // namespace step

bool use_step128(int64_t T, int64_t D) { return T == 1 && D == step::D; }

hipError_t launch_sssd_step128_fused(const void* proj, int64_t proj_stride, int io_dtype,
                                     const uint8_t* mask, const float* rms_w, float rms_eps,
                                     float* psi, void* out, int B, int H, hipStream_t stream) {
  const step::StepFused fz{proj_stride, mask, rms_w, rms_eps};
  const int BH = B * H;
  if (io_dtype == VMI_F32)
    return step::launch_typed<float, DenseStates, true>(proj, proj, proj, nullptr, VMI_F32, psi,
                                                        out, psi, DenseStates{}, BH, H, stream, fz);
  if (io_dtype == VMI_BF16)
    return step::launch_typed<bf16_t, DenseStates, true>(proj, proj, proj, nullptr, VMI_BF16, psi,
                                                         out, psi, DenseStates{}, BH, H, stream,
                                                         fz);
  return step::launch_typed<f16_t, DenseStates, true>(proj, proj, proj, nullptr, VMI_F16, psi, out,
                                                      psi, DenseStates{}, BH, H, stream, fz);
}

hipError_t launch_sssd_step128(const void* q, const void* k, const void* v, const void* delta,
                               int io_dtype, int delta_dtype, const float* psi_in, void* out,
                               float* psi_out, int B, int H, hipStream_t stream) {
  return step::launch_map(q, k, v, delta, io_dtype, delta_dtype, psi_in, out, psi_out,
                          DenseStates{}, B, H, stream);
}

hipError_t launch_sssd_step128(const void* q, const void* k, const void* v, const void* delta,
                               int io_dtype, int delta_dtype, const float* psi_in, void* out,
                               float* psi_out, const StateMap& map, int B, int H,
                               hipStream_t stream) {
  return step::launch_map(q, k, v, delta, io_dtype, delta_dtype, psi_in, out, psi_out, map, B, H,
                          stream);
}

hipError_t launch_sssd_step128(const void* q, const void* k, const void* v, const void* delta,
                               int io_dtype, int delta_dtype, const float* psi_in, void* out,
                               float* psi_out, const SlotArgs& map, int B, int H,
                               hipStream_t stream) {
  return step::launch_map(q, k, v, delta, io_dtype, delta_dtype, psi_in, out, psi_out, map, B, H,
                          stream);
}

}  // namespace vmi
