"""TEST INFRASTRUCTURE -- restatement of the CHAM holographic scan (never imported by the product).

* ``cham_scan_eager`` follows ``verace_v1/modules/cham_memory.py:167-238`` in float64:
  G_t = gamma_t (k_t v_t^T + v_t k_t^T); U_t = solve(I - i G_t / 2, I + i G_t / 2)
  (``_solve_cham_cayley``, :53-97, with its non-finite guard: a non-finite solve becomes
  U = I); P_t = U_t ... U_1 (newest on the left, ``parallel_complex_prefix_scan``,
  :241-293, evaluated sequentially); Hraw_t = P_t H_0 (:219-220, H_0 on the right);
  readout rec_t = Re(NS_3(Hraw_t)) q_t with the matrix Newton-Schulz retraction
  (``parallel_newton_schulz_retraction``, :296-315, via oracle.cham_ns); the exported state
  is the raw Hraw_T (:238).
* ``cham_cayley_closed`` is the rank-2 closed form U = I + W N W^T, W = [k v] used by the
  kernels (derived by Woodbury from U = (I - X)^-1 (I + X), X = i G / 2), checked
  against the solve by tests/test_oracle_pins.py.
* ``cham_scan_closed`` carries Hraw directly (Hraw_t = U_t Hraw_{t-1}, the same product
  as P_t H_0) with the closed form and evaluates the readout without forming NS_3(H):
  NS_3(H) q = H f_3(H^H H) q for the degree-13 polynomial f_3 of the Newton-Schulz
  recursion (f_0 = 1, f_{j+1}(A) = f_j(A) (3 - A f_j(A)^2) / 2), applied to q through
  matrix-vector products only.  It is the restatement of what the GPU kernels compute.
"""
from __future__ import annotations

import numpy as np
import torch

from .cham_ns import newton_schulz_retraction


def cham_cayley_solve(k, v, gamma):
    """U = (I - iG/2)^-1 (I + iG/2), G = gamma (k v^T + v k^T); k, v [h], float64.

    With the reference's non-finite guard (``_solve_cham_cayley``, cham_memory.py:68-95):
    a solve whose result is not finite is redone on the substituted pair (I, I), i.e.
    U = I."""
    h = k.shape[0]
    eye = np.eye(h, dtype=np.complex128)
    with np.errstate(over="ignore", invalid="ignore"):
        G = gamma * (np.outer(k, v) + np.outer(v, k))
        right, left = eye - 0.5j * G, eye + 0.5j * G
    if not (np.isfinite(right).all() and np.isfinite(left).all()):
        return eye  # solve(I, I): numpy's LAPACK refuses non-finite matrices outright
    U = np.linalg.solve(right, left)
    return U if np.isfinite(U).all() else eye


def cham_cayley_closed(k, v, gamma):
    """N (2x2 complex) with U = I + W N W^T, W = [k v]: A = (i gamma / 2) S, S = [[0,1],[1,0]],
    Gm = W^T W, M = (I - A Gm)^-1 A, N = M + A + M Gm A."""
    S = np.array([[0.0, 1.0], [1.0, 0.0]])
    A = 0.5j * gamma * S
    Gm = np.array([[k @ k, k @ v], [k @ v, v @ v]])
    M = np.linalg.solve(np.eye(2) - A @ Gm, A)
    return M + A + M @ Gm @ A


def cham_scan_eager(q, k, v, gamma, H0r=None, H0i=None, ns_steps=3):
    """q, k, v [B, T, h]; gamma [B, T]; H0 [B, h, h] real/imag (identity / zero if None).
    Returns rec [B, T, h] and (Hraw_r, Hraw_i) [B, h, h], float64."""
    q, k, v, gamma = (np.asarray(x, dtype=np.float64) for x in (q, k, v, gamma))
    B, T, h = q.shape
    rec = np.zeros((B, T, h))
    Hr_out = np.zeros((B, h, h))
    Hi_out = np.zeros((B, h, h))
    for b in range(B):
        H0 = (np.eye(h) if H0r is None else np.asarray(H0r[b], dtype=np.float64)) \
            + 1j * (np.zeros((h, h)) if H0i is None else np.asarray(H0i[b], dtype=np.float64))
        P = np.eye(h, dtype=np.complex128)
        for t in range(T):
            P = cham_cayley_solve(k[b, t], v[b, t], gamma[b, t]) @ P
            Hraw = P @ H0
            Rr, _ = newton_schulz_retraction(torch.from_numpy(Hraw.real.copy()),
                                             torch.from_numpy(Hraw.imag.copy()), ns_steps)
            rec[b, t] = Rr.numpy() @ q[b, t]
        Hr_out[b], Hi_out[b] = Hraw.real, Hraw.imag
    return rec, (Hr_out, Hi_out)


def ns_apply(H, x, steps=3):
    """NS_steps(H) x = H f_steps(H^H H) x with matrix-vector products only."""
    A = lambda z: H.conj().T @ (H @ z)

    def f(j, z):
        if j == 0:
            return z
        w = f(j - 1, z)
        return 0.5 * f(j - 1, 3.0 * z - A(f(j - 1, w)))
    return H @ f(steps, x.astype(np.complex128))


def cham_scan_closed(q, k, v, gamma, H0r=None, H0i=None, ns_steps=3, readout=True):
    """Same outputs as cham_scan_eager, by the closed form and the matrix-free readout.
    readout=False skips the readout (rec stays zero): the raw state alone, by the same loop."""
    q, k, v, gamma = (np.asarray(x, dtype=np.float64) for x in (q, k, v, gamma))
    B, T, h = q.shape
    rec = np.zeros((B, T, h))
    Hr_out = np.zeros((B, h, h))
    Hi_out = np.zeros((B, h, h))
    for b in range(B):
        H = (np.eye(h) if H0r is None else np.asarray(H0r[b], dtype=np.float64)) \
            + 1j * (np.zeros((h, h)) if H0i is None else np.asarray(H0i[b], dtype=np.float64))
        for t in range(T):
            W = np.stack([k[b, t], v[b, t]], 1)
            N = cham_cayley_closed(k[b, t], v[b, t], gamma[b, t])
            H = H + W @ (N @ (W.T @ H))
            if readout:
                rec[b, t] = ns_apply(H, q[b, t], ns_steps).real
        Hr_out[b], Hi_out[b] = H.real, H.imag
    return rec, (Hr_out, Hi_out)
