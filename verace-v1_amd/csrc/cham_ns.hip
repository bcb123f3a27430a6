// Newton-Schulz unitary retraction of complex matrices H = Hr + i Hi
// (reference: verace_v1/modules/cham_memory.py:21-51, :296-315).
//
// One iteration, every product taken from the pre-update H:
//   Dr  = 3I - (Hr^T Hr + Hi^T Hi)        (= 3I - Re(H^H H))
//   Di  = -(Hr^T Hi - Hi^T Hr)            (= -Im(H^H H))
//   Hr' = 0.5 (Hr Dr - Hi Di)
//   Hi' = 0.5 (Hr Di + Hi Dr)
// Each line is one launch of a batched "two products, signed sum, scale,
// diagonal shift" fp32 GEMM.
#include "vmi_common.h"
#include "vmi_dispatch.h"

namespace vmi {

namespace {

constexpr int NS_TILE = 64;
constexpr int NS_KT = 16;
constexpr int NS_THREADS = 256;

// Out = scale * (op(A0) B0 + sign1 * op(A1) B1) + diag * I, all n x n, batched.
// transA: op(A) = A^T.
__global__ __launch_bounds__(NS_THREADS) void ns_gemm2_kernel(
    const float* __restrict__ A0, const float* __restrict__ B0, const float* __restrict__ A1,
    const float* __restrict__ B1, float* __restrict__ Out, int n, int transA, float sign1,
    float scale, float diag) {
  __shared__ float As[NS_KT][NS_TILE + 4];
  __shared__ float Bs[NS_KT][NS_TILE + 4];

  const int64_t boff = static_cast<int64_t>(blockIdx.z) * n * n;
  const int i0 = blockIdx.y * NS_TILE;
  const int j0 = blockIdx.x * NS_TILE;
  const int tid = threadIdx.x;
  const int tx = tid % 16, ty = tid / 16;

  float acc[4][4];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[a][c] = 0.f;

  for (int term = 0; term < 2; ++term) {
    const float* A = (term == 0 ? A0 : A1) + boff;
    const float* Bm = (term == 0 ? B0 : B1) + boff;
    const float sgn = term == 0 ? 1.0f : sign1;
    for (int k0 = 0; k0 < n; k0 += NS_KT) {
      // A tile: op(A)[i0 .. i0+63][k0 .. k0+15] stored k-major
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int e = tid + s * NS_THREADS;
        int ii, kk;
        float x = 0.f;
        if (transA) {  // op(A)(i, k) = A[k][i]
          kk = e / NS_TILE;
          ii = e % NS_TILE;
          if (i0 + ii < n && k0 + kk < n) x = A[static_cast<int64_t>(k0 + kk) * n + i0 + ii];
        } else {  // op(A)(i, k) = A[i][k]
          ii = e / NS_KT;
          kk = e % NS_KT;
          if (i0 + ii < n && k0 + kk < n) x = A[static_cast<int64_t>(i0 + ii) * n + k0 + kk];
        }
        As[kk][ii] = sgn * x;
      }
      // B tile: B[k0 .. k0+15][j0 .. j0+63]
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int e = tid + s * NS_THREADS;
        const int kk = e / NS_TILE, jj = e % NS_TILE;
        float x = 0.f;
        if (k0 + kk < n && j0 + jj < n) x = Bm[static_cast<int64_t>(k0 + kk) * n + j0 + jj];
        Bs[kk][jj] = x;
      }
      __syncthreads();
#pragma unroll
      for (int kk = 0; kk < NS_KT; ++kk) {
        float a[4], b[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) a[r] = As[kk][ty + 16 * r];
#pragma unroll
        for (int c = 0; c < 4; ++c) b[c] = Bs[kk][tx + 16 * c];
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
          for (int c = 0; c < 4; ++c) acc[r][c] = fmaf(a[r], b[c], acc[r][c]);
      }
      __syncthreads();
    }
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int i = i0 + ty + 16 * r;
    if (i >= n) continue;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int j = j0 + tx + 16 * c;
      if (j >= n) continue;
      float y = scale * acc[r][c];
      if (i == j) y += diag;
      Out[boff + static_cast<int64_t>(i) * n + j] = y;
    }
  }
}

hipError_t gemm2(const float* A0, const float* B0, const float* A1, const float* B1, float* Out,
                 int batch, int n, int transA, float sign1, float scale, float diag,
                 hipStream_t stream) {
  const dim3 grid((n + NS_TILE - 1) / NS_TILE, (n + NS_TILE - 1) / NS_TILE, batch);
  hipLaunchKernelGGL(ns_gemm2_kernel, grid, dim3(NS_THREADS), 0, stream, A0, B0, A1, B1, Out, n,
                     transA, sign1, scale, diag);
  return hipGetLastError();
}

}  // namespace

size_t ns_workspace_bytes(int64_t batch, int64_t n) {
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
