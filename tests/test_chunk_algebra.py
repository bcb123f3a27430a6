"""CPU check of the chunked WY/UT algebra the MFMA kernel implements (sssd_chunk.hip):
Gram -> 2x2 Cayley blocks -> T~ by 8x8 blocks (diagonal forward substitution, then
T~_gh = T~_gg sum_m G_gm T~_mh) -> Z = T~ W -> end state and masked readout, compared
with the fp64 closed form (oracle).  A wrong block formula, mask or operand order fails."""
import numpy as np
import pytest

from oracle import sssd_closed

C, R = 16, 32


def _cayley_blocks(G, dl):
    M = np.zeros((C, 2, 2))
    for t in range(C):
        h = dl[t] / 2
        kk, vv, kv = G[2 * t, 2 * t], G[2 * t + 1, 2 * t + 1], G[2 * t, 2 * t + 1]
        c = 2 / (1 + h * h * max(kk * vv - kv * kv, 0))
        M[t] = [[-c * h * h * vv, c * (h * h * kv - h)], [c * (h * h * kv + h), -c * h * h * kk]]
    return M


def _t_blocked(G, M):
    Tt = np.zeros((R, R))
    for gb in range(4):                       # diagonal blocks: forward substitution
        for col in range(8):
            x = np.zeros(8)
            for tt in range(4):
                r0 = 8 * gb + 2 * tt
                s0 = sum(G[r0, 8 * gb + i] * x[i] for i in range(2 * tt))
                s1 = sum(G[r0 + 1, 8 * gb + i] * x[i] for i in range(2 * tt))
                e0, e1 = (col == 2 * tt) + s0, (col == 2 * tt + 1) + s1
                m = M[4 * gb + tt]
                x[2 * tt], x[2 * tt + 1] = m[0, 0] * e0 + m[0, 1] * e1, m[1, 0] * e0 + m[1, 1] * e1
            Tt[8 * gb:8 * gb + 8, 8 * gb + col] = x
    for gr in range(1, 4):                    # off-diagonal blocks
        for gc in range(gr):
            S = sum(G[8 * gr:8 * gr + 8, 8 * m:8 * m + 8] @ Tt[8 * m:8 * m + 8, 8 * gc:8 * gc + 8]
                    for m in range(gc, gr))
            Tt[8 * gr:8 * gr + 8, 8 * gc:8 * gc + 8] = Tt[8 * gr:8 * gr + 8, 8 * gr:8 * gr + 8] @ S
    return Tt


@pytest.mark.parametrize("T,D,seed", [(16, 32, 0), (67, 32, 1), (45, 24, 2)])
def test_chunk_form_equals_closed_form(T, D, seed):
    rng = np.random.default_rng(seed)
    nrm = lambda x: x / np.linalg.norm(x, axis=-1, keepdims=True)
    q, k, v = (nrm(rng.standard_normal((1, T, 1, D))) for _ in range(3))
    delta = 0.5 / (1 + np.exp(-rng.standard_normal((1, T, 1))))
    o_ref, psi_ref = sssd_closed.sssd_scan_closed_np(q, k, v, delta)
    psi = np.eye(D)
    out = np.zeros((T, D))
    mask = np.array([[1.0 if (r >> 1) <= t else 0.0 for t in range(C)] for r in range(R)])
    for c0 in range(0, T, C):
        n = min(C, T - c0)
        U, Q, dl = np.zeros((D, R)), np.zeros((D, C)), np.zeros(C)
        for t in range(n):  # zero-padded tail, exactly as the kernel stages it
            U[:, 2 * t], U[:, 2 * t + 1] = k[0, c0 + t, 0], v[0, c0 + t, 0]
            Q[:, t], dl[t] = q[0, c0 + t, 0], delta[0, c0 + t, 0]
        G = U.T @ U
        M = _cayley_blocks(G, dl)
        Tt = _t_blocked(G, M)
        # T~ == (I - L)^-1 blockdiag(M)
        Bd, L = np.zeros((R, R)), np.zeros((R, R))
        for t in range(C):
            Bd[2 * t:2 * t + 2, 2 * t:2 * t + 2] = M[t]
            for i in range(t):
                L[2 * t:2 * t + 2, 2 * i:2 * i + 2] = M[t] @ G[2 * t:2 * t + 2, 2 * i:2 * i + 2]
        assert np.abs(Tt - np.linalg.solve(np.eye(R) - L, Bd)).max() < 1e-12
        Z = Tt @ (U.T @ psi)
        O = psi @ Q + U @ ((Z @ Q) * mask)
        out[c0:c0 + n] = O[:, :n].T
        psi = psi + U @ Z
    assert np.abs(out - o_ref[0, :, 0]).max() < 1e-12
    assert np.abs(psi - psi_ref[0, 0]).max() < 1e-12


def test_planted_unmasked_readout_is_caught():
    rng = np.random.default_rng(3)
    D = 16
    U = rng.standard_normal((D, R))
    Z = rng.standard_normal((R, D))
    Q = rng.standard_normal((D, C))
    mask = np.array([[1.0 if (r >> 1) <= t else 0.0 for t in range(C)] for r in range(R)])
    assert np.abs(U @ ((Z @ Q) * mask) - U @ (Z @ Q)).max() > 1e-3
