"""CPU check of the chunked (WY) form of the scan's backward, the GEMM-shaped algebra a
chunked MFMA backward would implement; no GPU, no kernel yet.

Per chunk (U = [k_1 v_1 .. k_C v_C], T~ = (I - L)^-1 blockdiag(M), states Psi_s -> Psi_e):
  Psi_s = Psi_e + U T~^T U^T Psi_e           (the chunk factor is orthogonal)
  W = U^T Psi_s,  Z = T~ W,  X = mask o (Z Q),  dX = mask o (U^T dO)
  dZ = U^T Lam_e + dX Q^T,   dT~ = dZ W^T,    dW = T~^T dZ
  dQ = Z^T dX + Psi_s^T dO,  dU = Lam_e Z^T + dO X^T + Psi_s dW^T
  Lam_s = Lam_e + dO Q^T + U dW
then, per chunk and independent of the state, dT~ through T~ = A B (A = (I - L)^-1):
  dA = dT~ B^T, dB = A^T dT~, dL = A^T dA A^T on the strictly lower blocks,
  L_ti = M_t G_ti:  dM_t += dB_tt + sum_i dL_ti G_ti^T,  dG_ti += M_t^T dL_ti,
M_t(delta_t, kk, vv, kv) as in the kernels, and dU += U (dG + dG^T).  Compared with fp64
autograd through the eager restatement (the reference's training graph).
"""
import numpy as np
import pytest
import torch

from oracle import sssd_eager

C, R = 16, 32


def _m_and_parts(dl, kk, vv, kv):
    h = dl / 2
    P = h * h
    g = max(kk * vv - kv * kv, 0.0)
    c = 2 / (1 + P * g)
    N = np.array([[-P * vv, P * kv - h], [P * kv + h, -P * kk]])
    return c * N, (h, P, g, c, N)


def _m_backward(dM, parts, kk, vv, kv):
    h, P, g, c, N = parts
    S = (dM * N).sum()
    dh = c * (dM[0, 1] * (2 * h * kv - 1) + dM[1, 0] * (2 * h * kv + 1)
              - 2 * h * (dM[0, 0] * vv + dM[1, 1] * kk))
    dvv, dkk, dkv = -c * P * dM[0, 0], -c * P * dM[1, 1], c * P * (dM[0, 1] + dM[1, 0])
    dh += S * (-c * c * h * g)
    dg = S * (-0.5 * c * c * P)
    return 0.5 * dh, dkk + dg * vv, dvv + dg * kk, dkv - 2 * dg * kv


def chunked_backward(q, k, v, d, psi_T, d_out, d_psi_T):
    """One sequence: q, k, v, d_out [T, D]; d [T]; psi_T, d_psi_T [D, D]."""
    T, D = q.shape
    nch = (T + C - 1) // C
    dq, dk, dv, dd = (np.zeros_like(x) for x in (q, k, v, d))
    lam = d_psi_T.copy()
    psi_e = psi_T.copy()
    mask = np.array([[1.0 if (r >> 1) <= t else 0.0 for t in range(C)] for r in range(R)])
    for n in range(nch - 1, -1, -1):
        c0, nt = n * C, min(C, T - n * C)
        U, Q, dO, dl = np.zeros((D, R)), np.zeros((D, C)), np.zeros((D, C)), np.zeros(C)
        for t in range(nt):
            U[:, 2 * t], U[:, 2 * t + 1] = k[c0 + t], v[c0 + t]
            Q[:, t], dO[:, t], dl[t] = q[c0 + t], d_out[c0 + t], d[c0 + t]
        G = U.T @ U
        Ms, parts = [], []
        for t in range(C):
            M, pt = _m_and_parts(dl[t], G[2 * t, 2 * t], G[2 * t + 1, 2 * t + 1], G[2 * t, 2 * t + 1])
            Ms.append(M)
            parts.append(pt)
        L = np.zeros((R, R))
        Bd = np.zeros((R, R))
        for t in range(C):
            Bd[2 * t:2 * t + 2, 2 * t:2 * t + 2] = Ms[t]
            for i in range(t):
                L[2 * t:2 * t + 2, 2 * i:2 * i + 2] = Ms[t] @ G[2 * t:2 * t + 2, 2 * i:2 * i + 2]
        A = np.linalg.inv(np.eye(R) - L)
        Tt = A @ Bd
        # state-dependent part (GEMMs)
        psi_s = psi_e + U @ (Tt.T @ (U.T @ psi_e))
        W = U.T @ psi_s
        Z = Tt @ W
        X = mask * (Z @ Q)
        dX = mask * (U.T @ dO)
        dZ = U.T @ lam + dX @ Q.T
        dT = dZ @ W.T
        dW = Tt.T @ dZ
        dQ = Z.T @ dX + psi_s.T @ dO
        dU = lam @ Z.T + dO @ X.T + psi_s @ dW.T
        lam = lam + dO @ Q.T + U @ dW
        psi_e = psi_s
        # T~ backward (per chunk, no state)
        dA = dT @ Bd.T
        dB = A.T @ dT
        dL = A.T @ dA @ A.T
        dG = np.zeros((R, R))
        for t in range(C):
            dM = dB[2 * t:2 * t + 2, 2 * t:2 * t + 2].copy()
            for i in range(t):
                blk = dL[2 * t:2 * t + 2, 2 * i:2 * i + 2]
                dM += blk @ G[2 * t:2 * t + 2, 2 * i:2 * i + 2].T
                dG[2 * t:2 * t + 2, 2 * i:2 * i + 2] += Ms[t].T @ blk
            ddl, dkk, dvv, dkv = _m_backward(dM, parts[t], G[2 * t, 2 * t], G[2 * t + 1, 2 * t + 1],
                                             G[2 * t, 2 * t + 1])
            dG[2 * t, 2 * t] += dkk
            dG[2 * t + 1, 2 * t + 1] += dvv
            dG[2 * t, 2 * t + 1] += dkv
            if t < nt:
                dd[c0 + t] = ddl
        dU = dU + U @ (dG + dG.T)
        for t in range(nt):
            dk[c0 + t], dv[c0 + t] = dU[:, 2 * t], dU[:, 2 * t + 1]
            dq[c0 + t] = dQ[:, t]
    return dq, dk, dv, dd, lam


@pytest.mark.parametrize("T,D,seed", [(16, 8, 0), (37, 12, 1), (50, 16, 2)])
def test_chunked_backward_matches_autograd(T, D, seed):
    g = torch.Generator().manual_seed(seed)
    nrm = torch.nn.functional.normalize
    q = nrm(torch.randn(1, T, 1, D, generator=g, dtype=torch.float64), dim=-1)
    k = nrm(torch.randn(1, T, 1, D, generator=g, dtype=torch.float64), dim=-1)
    v = nrm(torch.randn(1, T, 1, D, generator=g, dtype=torch.float64), dim=-1)
    d = 0.1 + 0.8 * torch.rand(1, T, 1, generator=g, dtype=torch.float64)
    psi0 = torch.linalg.qr(torch.randn(1, 1, D, D, generator=g, dtype=torch.float64))[0]
    w_o = torch.randn(1, T, 1, D, generator=g, dtype=torch.float64)
    w_s = torch.randn(1, 1, D, D, generator=g, dtype=torch.float64)
    a = [x.clone().requires_grad_(True) for x in (q, k, v, d, psi0)]
    o, s = sssd_eager.sssd_scan_eager(*a, compute_dtype=torch.float64)
    ((o * w_o).sum() + (s * w_s).sum()).backward()
    got = chunked_backward(q[0, :, 0].numpy(), k[0, :, 0].numpy(), v[0, :, 0].numpy(),
                           d[0, :, 0].numpy(), s.detach()[0, 0].numpy(), w_o[0, :, 0].numpy(),
                           w_s[0, 0].numpy())
    ref = [a[0].grad[0, :, 0], a[1].grad[0, :, 0], a[2].grad[0, :, 0], a[3].grad[0, :, 0],
           a[4].grad[0, 0]]
    for name, x, y in zip(("dq", "dk", "dv", "ddelta", "dpsi0"), got, ref):
        y = y.numpy()
        assert np.abs(x - y).max() <= 1e-9 * max(1.0, np.abs(y).max()), name
