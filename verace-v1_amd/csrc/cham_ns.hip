// Newton-Schulz unitary retraction of complex matrices H = Hr + i Hi
// (reference: verace_v1/modules/cham_memory.py:21-51, :296-315).
//
// One iteration, every product taken from the pre-update H:
//   Dr  = 3I - (Hr^T Hr + Hi^T Hi)        (= 3I - Re(H^H H))
//   Di  = -(Hr^T Hi - Hi^T Hr)            (= -Im(H^H H))
//   Hr' = 0.5 (Hr Dr - Hi Di)
//   Hi' = 0.5 (Hr Di + Hi Dr)
// Each line is one launch of a batched "two products, signed sum, scale,
// diagonal shift" GEMM on the fp32 MFMA.
#include "vmi_common.h"
#include "vmi_dispatch.h"

namespace vmi {

namespace {

// Out = scale * (op(A0) B0 + sign1 * op(A1) B1) + diag * I, all n x n, batched over
// blockIdx.z; transA: op(A) = A^T.  fp32 MFMA (v_mfma_f32_32x32x2f32: exact fp32
// products, fp32 accumulation), so the result carries fp32 matmul rounding only.
//
// Workgroup = 4 waves, 64 x 64 output tile; wave (wr, wc) owns the 32 x 32 sub-tile
// (32wr, 32wc) in one accumulator.  The K dimension runs in chunks of 32 staged in
// LDS k-major (As[k][m], Bs[k][n]); the two products are one flattened sequence of
// chunks, and the next chunk is loaded into registers while the current one is
// multiplied.  Within a chunk, MFMA s (s = 0..15) uses k = s for lanes 0-31 and
// k = 16 + s for lanes 32-63 (the k-slot of a 32x32x2 operand is lane / 32).
constexpr int NS_TM = 64;
constexpr int NS_KT = 32;
constexpr int NS_LD = NS_TM + 4;
constexpr int NS_THREADS = 256;
constexpr int NS_EPT = NS_TM * NS_KT / NS_THREADS;  // elements per thread per operand tile

typedef float f32x16 __attribute__((ext_vector_type(16)));

__global__ __launch_bounds__(NS_THREADS) void ns_gemm2_kernel(
    const float* __restrict__ A0, const float* __restrict__ B0, const float* __restrict__ A1,
    const float* __restrict__ B1, float* __restrict__ Out, int n, int transA, float sign1,
    float scale, float diag) {
  __shared__ float As[2][NS_KT][NS_LD];
  __shared__ float Bs[2][NS_KT][NS_LD];

  const int64_t boff = static_cast<int64_t>(blockIdx.z) * n * n;
  const int i0 = blockIdx.y * NS_TM;
  const int j0 = blockIdx.x * NS_TM;
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int wr = wave >> 1, wc = wave & 1;
  const int lm = lane & 31, g = lane >> 5;

  const int nk = (n + NS_KT - 1) / NS_KT;  // chunks per product
  const int nchunks = 2 * nk;
  float ra[NS_EPT], rb[NS_EPT];

  // Element e = tid + 256 s of a 64 x 32 tile.  A tile: (m, k) = (e % 64, e / 64) when
  // op(A) = A^T (A[k][m] is contiguous in m), (e / 32, e % 32) otherwise; B tile:
  // (k, col) = (e / 64, e % 64).  Consecutive threads read consecutive addresses.
  auto fetch = [&](int c) {
    const int term = c >= nk;
    const int k0 = (c - term * nk) * NS_KT;
    const float* A = (term ? A1 : A0) + boff;
    const float* Bm = (term ? B1 : B0) + boff;
    const float sgn = term ? sign1 : 1.0f;
#pragma unroll
    for (int s = 0; s < NS_EPT; ++s) {
      const int e = tid + NS_THREADS * s;
      int m, k;
      if (transA) { m = e % NS_TM; k = e / NS_TM; } else { m = e / NS_KT; k = e % NS_KT; }
      const int gi = i0 + m, gk = k0 + k;
      float x = 0.f;
      if (gi < n && gk < n) x = transA ? A[static_cast<int64_t>(gk) * n + gi] : A[static_cast<int64_t>(gi) * n + gk];
      ra[s] = sgn * x;
      const int kb = e / NS_TM, jb = e % NS_TM;
      const int gkb = k0 + kb, gj = j0 + jb;
      rb[s] = (gkb < n && gj < n) ? Bm[static_cast<int64_t>(gkb) * n + gj] : 0.f;
    }
  };
  auto commit = [&](int buf) {
#pragma unroll
    for (int s = 0; s < NS_EPT; ++s) {
      const int e = tid + NS_THREADS * s;
      if (transA) As[buf][e / NS_TM][e % NS_TM] = ra[s];
      else As[buf][e % NS_KT][e / NS_KT] = ra[s];
      Bs[buf][e / NS_TM][e % NS_TM] = rb[s];
    }
  };

  f32x16 acc = {};
  fetch(0);
  commit(0);
  __syncthreads();
  for (int c = 0; c < nchunks; ++c) {
    const int buf = c & 1;
    if (c + 1 < nchunks) fetch(c + 1);
    const float* as = &As[buf][16 * g][32 * wr + lm];
    const float* bs = &Bs[buf][16 * g][32 * wc + lm];
#pragma unroll
    for (int s = 0; s < 16; ++s)
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(as[s * NS_LD], bs[s * NS_LD], acc, 0, 0, 0);
    if (c + 1 < nchunks) commit(buf ^ 1);
    __syncthreads();
  }
  // lane holds rows 8(r/4) + 4g + r%4 of column lm in the wave's sub-tile
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int i = i0 + 32 * wr + 8 * (r >> 2) + 4 * g + (r & 3);
    const int j = j0 + 32 * wc + lm;
    if (i < n && j < n) Out[boff + static_cast<int64_t>(i) * n + j] = scale * acc[r] + (i == j ? diag : 0.f);
  }
}

hipError_t gemm2(const float* A0, const float* B0, const float* A1, const float* B1, float* Out,
                 int batch, int n, int transA, float sign1, float scale, float diag,
                 hipStream_t stream) {
  const dim3 grid((n + NS_TM - 1) / NS_TM, (n + NS_TM - 1) / NS_TM, batch);
  hipLaunchKernelGGL(ns_gemm2_kernel, grid, dim3(NS_THREADS), 0, stream, A0, B0, A1, B1, Out, n,
                     transA, sign1, scale, diag);
  return hipGetLastError();
}

}  // namespace

size_t ns_workspace_bytes(int64_t batch, int64_t n) {
  if (ns16_usable(n)) return ns16_workspace_bytes(batch, n);
  return static_cast<size_t>(6) * batch * n * n * sizeof(float);
}

hipError_t launch_ns_retraction(const float* h_real, const float* h_imag, float* out_real,
                                float* out_imag, int batch, int n, int steps, void* workspace,
                                hipStream_t stream) {
  const size_t mat = static_cast<size_t>(batch) * n * n;
  const size_t bytes = mat * sizeof(float);
  if (steps == 0) {
    hipError_t e = hipSuccess;
    if (out_real != h_real) e = hipMemcpyAsync(out_real, h_real, bytes, hipMemcpyDeviceToDevice, stream);
    if (e == hipSuccess && out_imag != h_imag)
      e = hipMemcpyAsync(out_imag, h_imag, bytes, hipMemcpyDeviceToDevice, stream);
    return e;
  }
  if (ns16_usable(n))  // 16-bit matrix cores, two launches per iteration (cham_ns16.hip)
    return launch_ns16_retraction(h_real, h_imag, out_real, out_imag, batch, n, steps, workspace,
                                  stream);
  float* ws = static_cast<float*>(workspace);
  float* Dr = ws;
  float* Di = ws + mat;
  float* pr[2] = {ws + 2 * mat, ws + 4 * mat};
  float* pi[2] = {ws + 3 * mat, ws + 5 * mat};
  const float* cr = h_real;
  const float* ci = h_imag;
  hipError_t e = hipSuccess;
  for (int s = 0; s < steps && e == hipSuccess; ++s) {
    float* nr = pr[s & 1];
    float* ni = pi[s & 1];
    e = gemm2(cr, cr, ci, ci, Dr, batch, n, 1, 1.0f, -1.0f, 3.0f, stream);
    if (e == hipSuccess) e = gemm2(cr, ci, ci, cr, Di, batch, n, 1, -1.0f, -1.0f, 0.0f, stream);
    if (e == hipSuccess) e = gemm2(cr, Dr, ci, Di, nr, batch, n, 0, -1.0f, 0.5f, 0.0f, stream);
    if (e == hipSuccess) e = gemm2(cr, Di, ci, Dr, ni, batch, n, 0, 1.0f, 0.5f, 0.0f, stream);
    cr = nr;
    ci = ni;
  }
  if (e == hipSuccess) e = hipMemcpyAsync(out_real, cr, bytes, hipMemcpyDeviceToDevice, stream);
  if (e == hipSuccess) e = hipMemcpyAsync(out_imag, ci, bytes, hipMemcpyDeviceToDevice, stream);
  return e;
}

}  // namespace vmi
