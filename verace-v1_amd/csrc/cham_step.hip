// Single-token CHAM step (decode) with the holographic state updated in place, for any
// holographic_dim h <= 1024.  Reference: the CHAM forward at seq_len 1
// (cham_memory.py:117-238) that the generator re-runs per token with the previous raw state
// as initial_hologram (hyper_generate.py:58-63, acd_engine.py:116-121); the reference returns
// a fresh state, this updates the caller's state in place (opt-in, like the SSSD step).
//
// Per item b (closed form as in cham_scan.hip): with the raw state H = Hr + i Hi,
//   a = k^T H,  b = v^T H             (complex row vectors: column sums over h rows)
//   H' = H + k (N11 a + N12 b) + v (N12 a + N22 b)
// and the readout rec = Re(NS_3(H') q).  Every factor is unitary, so NS_3(U H) = U NS_3(H):
// the readout state R = NS_3(H) evolves by the same update, R' = U R, and rec = Re(R' q) =
// Rr' q.  A caller whose H is unitary (a sequence that started from the identity) passes no
// R (then R = H); otherwise it carries R beside H (computed once by the Newton-Schulz
// retraction) and both are updated here.  That is O(h^2) per token instead of the 13
// applications of H^H H (or 28 dense h x h products) a fresh NS_3 per token takes.
//
// Bound: HBM (each state is read once and written once: 16 h^2 bytes per item and state,
// 8 flops per element).  Grid (h / 32 column blocks, B, number of states): columns evolve
// independently (a_j, b_j are sums over rows of column j), so a workgroup owns 32 columns of
// one state of one item: thread (rg, cg) holds rows rg + 64 m and columns 4 cg .. 4 cg + 3
// (float4, eight lanes cover a 128-byte row piece).  The readout sums over columns, so the
// readout-state workgroups write per-block partial sums of Rr' q; cham_step_finish_kernel
// adds them.
#include "cham_common.h"
#include "vmi_dispatch.h"

namespace vmi {
namespace chams {

using cham::NCoef;

constexpr int NT = 512;
constexpr int CB = 32;          // columns per workgroup
constexpr int NRG = NT / 8;     // row groups (8 column groups of 4 columns)

template <typename IO, typename GT, int RPT>
__global__ __launch_bounds__(NT) void cham_step_kernel(
    const IO* __restrict__ q, const IO* __restrict__ k, const IO* __restrict__ v,
    const GT* __restrict__ gamma, float* hr0, float* hi0, float* hr1, float* hi1,
    float* __restrict__ part, int h, int nstates) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int cg = tid & 7, rg = tid >> 3;
  const int blk = blockIdx.x, b = blockIdx.y, z = blockIdx.z;
  const int nblk = gridDim.x;
  const int c0 = blk * CB + 4 * cg;
  const bool readout = z == nstates - 1;
  float* __restrict__ sr = z == 0 ? hr0 : hr1;
  float* __restrict__ si = z == 0 ? hi0 : hi1;
  const int64_t hh = static_cast<int64_t>(h) * h;
  const int64_t tb = static_cast<int64_t>(b) * h;  // this item's token row

  __shared__ float4 s_red[NT / 64][CB][2];  // per wave: (ar, ai, br, bi) of each column... x2
  __shared__ float s_dot[NT / 64][3];

  // state rows rg + NRG m, columns c0 .. c0+3 (both parts); zero outside h
  float4 xr[RPT], xi[RPT];
  float kr[RPT], vr[RPT];
  const bool colok = c0 < h;  // h % 4 == 0 (checked by the host), so all four or none
#pragma unroll
  for (int m = 0; m < RPT; ++m) {
    const int r = rg + NRG * m;
    const bool ok = colok && r < h;
    const int64_t o = static_cast<int64_t>(b) * hh + static_cast<int64_t>(ok ? r : 0) * h + (ok ? c0 : 0);
    xr[m] = ok ? *reinterpret_cast<const float4*>(sr + o) : make_float4(0.f, 0.f, 0.f, 0.f);
    xi[m] = ok ? *reinterpret_cast<const float4*>(si + o) : make_float4(0.f, 0.f, 0.f, 0.f);
    kr[m] = r < h ? io<IO>::load(k, tb + r) : 0.f;
    vr[m] = r < h ? io<IO>::load(v, tb + r) : 0.f;
  }
  const float g = io<GT>::load(gamma, b);
  float4 qc = make_float4(0.f, 0.f, 0.f, 0.f);
  if (readout && colok)
    qc = make_float4(io<IO>::load(q, tb + c0), io<IO>::load(q, tb + c0 + 1),
                     io<IO>::load(q, tb + c0 + 2), io<IO>::load(q, tb + c0 + 3));

  // Gram entries over all h rows (each row counted once: column group 0's lanes)
  float kk = 0.f, vv = 0.f, kv = 0.f;
  if (cg == 0) {
#pragma unroll
    for (int m = 0; m < RPT; ++m) {
      kk = fmaf(kr[m], kr[m], kk);
      vv = fmaf(vr[m], vr[m], vv);
      kv = fmaf(kr[m], vr[m], kv);
    }
  }
  // column partials a = k^T H, b = v^T H over this thread's rows
  float4 ar = make_float4(0.f, 0.f, 0.f, 0.f), ai = ar, br = ar, bi = ar;
#pragma unroll
  for (int m = 0; m < RPT; ++m) {
    ar.x = fmaf(kr[m], xr[m].x, ar.x); ar.y = fmaf(kr[m], xr[m].y, ar.y);
    ar.z = fmaf(kr[m], xr[m].z, ar.z); ar.w = fmaf(kr[m], xr[m].w, ar.w);
    ai.x = fmaf(kr[m], xi[m].x, ai.x); ai.y = fmaf(kr[m], xi[m].y, ai.y);
    ai.z = fmaf(kr[m], xi[m].z, ai.z); ai.w = fmaf(kr[m], xi[m].w, ai.w);
    br.x = fmaf(vr[m], xr[m].x, br.x); br.y = fmaf(vr[m], xr[m].y, br.y);
    br.z = fmaf(vr[m], xr[m].z, br.z); br.w = fmaf(vr[m], xr[m].w, br.w);
    bi.x = fmaf(vr[m], xi[m].x, bi.x); bi.y = fmaf(vr[m], xi[m].y, bi.y);
    bi.z = fmaf(vr[m], xi[m].z, bi.z); bi.w = fmaf(vr[m], xi[m].w, bi.w);
  }
  // sum over the wave's 8 row groups (lane bits 3..5), then over the waves in LDS
#pragma unroll
  for (int off = 8; off <= 32; off <<= 1) {
    ar.x += __shfl_xor(ar.x, off); ar.y += __shfl_xor(ar.y, off);
    ar.z += __shfl_xor(ar.z, off); ar.w += __shfl_xor(ar.w, off);
    ai.x += __shfl_xor(ai.x, off); ai.y += __shfl_xor(ai.y, off);
    ai.z += __shfl_xor(ai.z, off); ai.w += __shfl_xor(ai.w, off);
    br.x += __shfl_xor(br.x, off); br.y += __shfl_xor(br.y, off);
    br.z += __shfl_xor(br.z, off); br.w += __shfl_xor(br.w, off);
    bi.x += __shfl_xor(bi.x, off); bi.y += __shfl_xor(bi.y, off);
    bi.z += __shfl_xor(bi.z, off); bi.w += __shfl_xor(bi.w, off);
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    kk += __shfl_xor(kk, off);
    vv += __shfl_xor(vv, off);
    kv += __shfl_xor(kv, off);
  }
  if (lane < 8) {
    float* dst = reinterpret_cast<float*>(&s_red[wave][4 * cg][0]);
    // columns 4cg + e: (ar, ai, br, bi) packed as two float4 per column
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float* pa = &ar.x;
      const float* pai = &ai.x;
      const float* pb = &br.x;
      const float* pbi = &bi.x;
      dst[8 * e + 0] = pa[e]; dst[8 * e + 1] = pai[e]; dst[8 * e + 2] = pb[e]; dst[8 * e + 3] = pbi[e];
    }
  }
  if (lane == 0) {
    s_dot[wave][0] = kk; s_dot[wave][1] = vv; s_dot[wave][2] = kv;
  }
  __syncthreads();
  float4 A[4];  // (ar, ai, br, bi) of columns 4cg + e, summed over all rows
#pragma unroll
  for (int e = 0; e < 4; ++e) A[e] = s_red[0][4 * cg + e][0];
#pragma unroll
  for (int w = 1; w < NT / 64; ++w)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float4 x = s_red[w][4 * cg + e][0];
      A[e].x += x.x; A[e].y += x.y; A[e].z += x.z; A[e].w += x.w;
    }
  kk = s_dot[0][0]; vv = s_dot[0][1]; kv = s_dot[0][2];
#pragma unroll
  for (int w = 1; w < NT / 64; ++w) {
    kk += s_dot[w][0]; vv += s_dot[w][1]; kv += s_dot[w][2];
  }
  bool ok;
  const NCoef N = cham::cayley_n_guarded(g, kk, vv, kv, ok);
  if (!ok) {  // identity token: k, v read as zero (uniform over the workgroup)
#pragma unroll
    for (int m = 0; m < RPT; ++m) kr[m] = vr[m] = 0.f;
  }
  // C = N11 a + N12 b,  D = N12 a + N22 b (complex), per column
  float cr[4], ci[4], dr[4], di[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float4 s = A[e];  // (ar, ai, br, bi)
    cr[e] = N.n11r * s.x - N.n11i * s.y + N.n12r * s.z - N.n12i * s.w;
    ci[e] = N.n11r * s.y + N.n11i * s.x + N.n12r * s.w + N.n12i * s.z;
    dr[e] = N.n12r * s.x - N.n12i * s.y + N.n22r * s.z - N.n22i * s.w;
    di[e] = N.n12r * s.y + N.n12i * s.x + N.n22r * s.w + N.n22i * s.z;
  }
  // update, store, readout partials
  float po[RPT];
#pragma unroll
  for (int m = 0; m < RPT; ++m) {
    const int r = rg + NRG * m;
    float4 yr = xr[m], yi = xi[m];
    yr.x = fmaf(kr[m], cr[0], fmaf(vr[m], dr[0], yr.x));
    yr.y = fmaf(kr[m], cr[1], fmaf(vr[m], dr[1], yr.y));
    yr.z = fmaf(kr[m], cr[2], fmaf(vr[m], dr[2], yr.z));
    yr.w = fmaf(kr[m], cr[3], fmaf(vr[m], dr[3], yr.w));
    yi.x = fmaf(kr[m], ci[0], fmaf(vr[m], di[0], yi.x));
    yi.y = fmaf(kr[m], ci[1], fmaf(vr[m], di[1], yi.y));
    yi.z = fmaf(kr[m], ci[2], fmaf(vr[m], di[2], yi.z));
    yi.w = fmaf(kr[m], ci[3], fmaf(vr[m], di[3], yi.w));
    if (colok && r < h) {
      const int64_t o = static_cast<int64_t>(b) * hh + static_cast<int64_t>(r) * h + c0;
      *reinterpret_cast<float4*>(sr + o) = yr;
      *reinterpret_cast<float4*>(si + o) = yi;
    }
    po[m] = fmaf(yr.x, qc.x, fmaf(yr.y, qc.y, fmaf(yr.z, qc.z, yr.w * qc.w)));
  }
  if (readout) {
    // sum over the 8 column groups (lane bits 0..2): every lane of the group gets the row sum
#pragma unroll
    for (int m = 0; m < RPT; ++m) {
      po[m] += __shfl_xor(po[m], 1);
      po[m] += __shfl_xor(po[m], 2);
      po[m] += __shfl_xor(po[m], 4);
    }
    float* pp = part + (static_cast<int64_t>(b) * nblk + blk) * h;
#pragma unroll
    for (int m = 0; m < RPT; ++m) {
      const int r = rg + NRG * m;
      if (cg == (m & 7) && r < h) pp[r] = po[m];
    }
  }
}

// out[b][i] = sum over the column blocks of the readout partials (io dtype)
template <typename IO>
__global__ __launch_bounds__(256) void cham_step_finish_kernel(const float* __restrict__ part,
                                                               IO* __restrict__ out, int h,
                                                               int nblk) {
  const int b = blockIdx.y;
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= h) return;
  const float* pp = part + static_cast<int64_t>(b) * nblk * h + i;
  float s = 0.f;
  for (int j = 0; j < nblk; ++j) s += pp[static_cast<int64_t>(j) * h];
  io<IO>::store(out, static_cast<int64_t>(b) * h + i, s);
}

template <typename IO, typename GT>
hipError_t launch_t(const void* q, const void* k, const void* v, const void* gamma, float* hr,
                    float* hi, float* rr, float* ri, void* out, int B, int h, float* part,
                    hipStream_t stream) {
  const int nblk = (h + CB - 1) / CB;
  const int nstates = rr ? 2 : 1;
  const dim3 grid(nblk, B, nstates);
  const IO* qq = static_cast<const IO*>(q);
  const IO* kq = static_cast<const IO*>(k);
  const IO* vq = static_cast<const IO*>(v);
  const GT* gg = static_cast<const GT*>(gamma);
#define VMI_CS(RPT_) \
  hipLaunchKernelGGL((cham_step_kernel<IO, GT, RPT_>), grid, dim3(NT), 0, stream, qq, kq, vq, gg, \
                     hr, hi, rr, ri, part, h, nstates)
  if (h <= 2 * NRG) VMI_CS(2);
  else if (h <= 4 * NRG) VMI_CS(4);
  else if (h <= 8 * NRG) VMI_CS(8);
  else VMI_CS(16);
#undef VMI_CS
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((cham_step_finish_kernel<IO>), dim3((h + 255) / 256, B), dim3(256), 0, stream,
                     part, static_cast<IO*>(out), h, nblk);
  return hipGetLastError();
}

}  // namespace chams

size_t cham_step_workspace_bytes(int64_t B, int64_t h) {
  return static_cast<size_t>(B) * ((h + chams::CB - 1) / chams::CB) * h * sizeof(float);
}

hipError_t launch_cham_step(const void* q, const void* k, const void* v, const void* gamma,
                            int io_dtype, int gamma_dtype, float* hr, float* hi, float* rr,
                            float* ri, void* out, int B, int h, void* workspace,
                            hipStream_t stream) {
  float* part = static_cast<float*>(workspace);
#define VMI_GT(IO_)                                                                              \
  if (gamma_dtype == VMI_F32)                                                                  \
    return chams::launch_t<IO_, float>(q, k, v, gamma, hr, hi, rr, ri, out, B, h, part, stream); \
  if (gamma_dtype == VMI_BF16)                                                                 \
    return chams::launch_t<IO_, bf16_t>(q, k, v, gamma, hr, hi, rr, ri, out, B, h, part, stream); \
  return chams::launch_t<IO_, f16_t>(q, k, v, gamma, hr, hi, rr, ri, out, B, h, part, stream);
  if (io_dtype == VMI_F32) { VMI_GT(float) }
  if (io_dtype == VMI_BF16) { VMI_GT(bf16_t) }
  VMI_GT(f16_t)
#undef VMI_GT
}

}  // namespace vmi
