/*
 * TEST INFRASTRUCTURE ONLY -- the CPU checker for the SSSD scan.  Nothing in
 * the product (verace-v1_amd/) links, loads or calls this file; only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg do.
 *
 * fp64 token-sequential restatement of the SSSD scan computed by the
 * reference's eager path (verace_v1/modules/sssd_attention.py:144-181):
 *   X_t   = 0.5 * delta_t * (k_t v_t^T - v_t k_t^T)            (:160-163)
 *   R_t   = solve(I + X_t, I - X_t) = (I + X_t)^-1 (I - X_t)    (:164-166)
 *   Psi_t = R_t Psi_{t-1}, Psi_0 = initial_state or I          (:147-150, :169-173)
 *   o_t   = Psi_t q_t                                          (:174-175)
 * R_t is applied in closed form, R = I + c(-X + X^2), c = 2/(1+m^2),
 * m^2 = (delta/2)^2 (|k|^2|v|^2 - (k.v)^2); the tests pin this closed form
 * against torch.linalg.solve and against brute-force products.
 *
 * Layouts: q, k, v [B,T,H,D] float32 (bf16 inputs are upcast exactly by the
 * caller), delta [B,T,H] float32, psi0 [B,H,D,D] float64 or NULL (identity),
 * out [B,T,H,D] float64 (may be NULL), psi_out [B,H,D,D] float64,
 * norms [B,H,T] float64 (may be NULL): Frobenius norm of Psi_t after each token.
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

int oracle_sssd_scan_f64(const float* q, const float* k, const float* v, const float* delta,
                         const double* psi0, double* out, double* psi_out, double* norms,
                         long B, long T, long H, long D, int nthreads) {
  long BH = B * H;
  long i;
  (void)nthreads;
#pragma omp parallel for schedule(dynamic, 1) num_threads(nthreads)
  for (i = 0; i < BH; ++i) {
    long b = i / H, h = i % H;
    double* psi = psi_out + i * D * D;
    double* a = (double*)malloc(sizeof(double) * 4 * D);
    double* bb = a + D;
    double* kd = a + 2 * D;
    double* vd = a + 3 * D;
    long r, c, t;
    if (psi0) {
      memcpy(psi, psi0 + i * D * D, sizeof(double) * D * D);
    } else {
      memset(psi, 0, sizeof(double) * D * D);
      for (r = 0; r < D; ++r) psi[r * D + r] = 1.0;
    }
    for (t = 0; t < T; ++t) {
      long tok = ((b * T + t) * H + h) * D;
      double kk = 0, vv = 0, kv = 0, hh, h2, c2, gd;
      for (r = 0; r < D; ++r) {
        kd[r] = (double)k[tok + r];
        vd[r] = (double)v[tok + r];
        kk += kd[r] * kd[r];
        vv += vd[r] * vd[r];
        kv += kd[r] * vd[r];
      }
      hh = 0.5 * (double)delta[(b * T + t) * H + h];
      h2 = hh * hh;
      gd = kk * vv - kv * kv;
      if (gd < 0) gd = 0;
      c2 = 2.0 / (1.0 + h2 * gd);
      for (c = 0; c < D; ++c) a[c] = bb[c] = 0.0;
      for (r = 0; r < D; ++r) {
        const double* row = psi + r * D;
        for (c = 0; c < D; ++c) {
          a[c] += kd[r] * row[c];
          bb[c] += vd[r] * row[c];
        }
      }
      /* a <- alpha, bb <- beta */
      for (c = 0; c < D; ++c) {
        double ac = a[c], bc = bb[c];
        a[c] = c2 * (-hh * bc + h2 * (kv * bc - vv * ac));
        bb[c] = c2 * (hh * ac + h2 * (kv * ac - kk * bc));
      }
      for (r = 0; r < D; ++r) {
        double* row = psi + r * D;
        for (c = 0; c < D; ++c) row[c] += kd[r] * a[c] + vd[r] * bb[c];
      }
      if (out) {
        for (r = 0; r < D; ++r) {
          const double* row = psi + r * D;
          double s = 0;
          for (c = 0; c < D; ++c) s += row[c] * (double)q[tok + c];
          out[tok + r] = s;
        }
      }
      if (norms) {
        double s = 0;
        for (r = 0; r < D * D; ++r) s += psi[r] * psi[r];
        norms[i * T + t] = sqrt(s);
      }
    }
    free(a);
  }
  return 0;
}
