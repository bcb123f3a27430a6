"""CPU checks of the scan's backward (csrc/sssd_bwd.hip), no GPU.

* The gradient oracle -- fp64 autograd through the eager restatement of
  ``sssd_attention.py:144-175`` (oracle/sssd_eager.py, solve + Blelloch products), the
  graph the reference's training differentiates -- against finite differences
  (``torch.autograd.gradcheck``) and against the autograd of an independent sequential
  closed-form scan.
* The kernels' algorithm restated in numpy (reverse recursion with states rebuilt by
  R_t^T, per-token dL/dU and dL/dM, then the chain rule through the Cayley
  coefficients M(delta, kk, vv, kv)) against that oracle, with an initial state and a
  gradient on the final state, plus planted mistakes it must catch.
"""
import numpy as np
import pytest
import torch

from oracle import sssd_eager


def _inputs(B, T, H, D, seed, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    nrm = torch.nn.functional.normalize
    q = nrm(torch.randn(B, T, H, D, generator=g, dtype=dtype), dim=-1)
    k = nrm(torch.randn(B, T, H, D, generator=g, dtype=dtype), dim=-1)
    v = nrm(torch.randn(B, T, H, D, generator=g, dtype=dtype), dim=-1)
    d = 0.1 + 0.8 * torch.rand(B, T, H, generator=g, dtype=dtype)  # large: visible gradients
    psi0 = torch.linalg.qr(torch.randn(B, H, D, D, generator=g, dtype=dtype))[0]
    return q, k, v, d, psi0


def _eager64(q, k, v, d, psi0):
    return sssd_eager.sssd_scan_eager(q, k, v, d, psi0, compute_dtype=torch.float64)


def _closed_seq(q, k, v, d, psi0):
    """Sequential closed form R = I + c(-X + X^2), X = (d/2)(k v^T - v k^T)."""
    B, T, H, D = q.shape
    psi = psi0
    outs = []
    eye = torch.eye(D, dtype=q.dtype)
    for t in range(T):
        kt, vt = k[:, t], v[:, t]
        A = kt.unsqueeze(-1) * vt.unsqueeze(-2) - vt.unsqueeze(-1) * kt.unsqueeze(-2)
        h = 0.5 * d[:, t].unsqueeze(-1).unsqueeze(-1)
        X = h * A
        m2 = (h.squeeze(-1).squeeze(-1) ** 2) * ((kt * kt).sum(-1) * (vt * vt).sum(-1) - (kt * vt).sum(-1) ** 2)
        c = (2.0 / (1.0 + m2)).unsqueeze(-1).unsqueeze(-1)
        R = eye + c * (-X + X @ X)
        psi = R @ psi
        outs.append((psi @ q[:, t].unsqueeze(-1)).squeeze(-1))
    return torch.stack(outs, 1), psi


def test_gradient_oracle_matches_finite_differences():
    q, k, v, d, psi0 = _inputs(1, 3, 1, 4, seed=1)
    args = tuple(x.clone().requires_grad_(True) for x in (q, k, v, d, psi0))
    assert torch.autograd.gradcheck(lambda *a: _eager64(*a), args, eps=1e-6, atol=1e-7)


def test_gradient_oracle_matches_closed_form_autograd():
    q, k, v, d, psi0 = _inputs(2, 6, 2, 8, seed=2)
    g = torch.Generator().manual_seed(3)
    w_o = torch.randn(2, 6, 2, 8, generator=g, dtype=torch.float64)
    w_s = torch.randn(2, 2, 8, 8, generator=g, dtype=torch.float64)
    grads = []
    for f in (_eager64, _closed_seq):
        a = tuple(x.clone().requires_grad_(True) for x in (q, k, v, d, psi0))
        o, s = f(*a)
        ((o * w_o).sum() + (s * w_s).sum()).backward()
        grads.append([x.grad for x in a])
    for g1, g2 in zip(*grads):
        assert torch.allclose(g1, g2, atol=1e-11, rtol=1e-9)


def kernel_backward(q, k, v, d, psi_T, d_out, d_psi_T):
    """numpy restatement of sssd_bwd_cols_kernel + sssd_bwd_reduce_kernel (float64)."""
    B, T, H, D = q.shape
    dq = np.zeros_like(q); dk = np.zeros_like(k); dv = np.zeros_like(v); dd = np.zeros_like(d)
    dpsi0 = np.zeros((B, H, D, D))
    for b in range(B):
        for hd in range(H):
            psi = psi_T[b, hd].copy()
            lam = d_psi_T[b, hd].copy()
            for t in range(T - 1, -1, -1):
                kt, vt, qt, gt = k[b, t, hd], v[b, t, hd], q[b, t, hd], d_out[b, t, hd]
                kk, vv, kv = kt @ kt, vt @ vt, kt @ vt
                hh = 0.5 * d[b, t, hd]
                P = hh * hh
                g = max(kk * vv - kv * kv, 0.0)
                c = 2.0 / (1.0 + P * g)
                M = c * np.array([[-P * vv, P * kv - hh], [P * kv + hh, -P * kk]])
                U = np.stack([kt, vt], 1)
                lam = lam + np.outer(gt, qt)
                dq[b, t, hd] = psi.T @ gt
                alpha = M.T @ (U.T @ psi)
                psi = psi + U @ alpha                       # Psi^(t)
                A = U.T @ psi
                Bm = U.T @ lam
                dU = lam @ A.T @ M.T + psi @ Bm.T @ M
                dM = Bm @ A.T
                lam = lam + U @ (M.T @ Bm)                  # Lambda^(t)
                # chain rule through M = c N
                N = M / c
                S = (dM * N).sum()
                dh = c * (dM[0, 1] * (2 * hh * kv - 1) + dM[1, 0] * (2 * hh * kv + 1)
                          - 2 * hh * (dM[0, 0] * vv + dM[1, 1] * kk))
                dvv, dkk, dkv = -c * P * dM[0, 0], -c * P * dM[1, 1], c * P * (dM[0, 1] + dM[1, 0])
                dh += S * (-c * c * hh * g)
                dg = S * (-0.5 * c * c * P)
                dkk += dg * vv; dvv += dg * kk; dkv += -2 * dg * kv
                dk[b, t, hd] = dU[:, 0] + 2 * dkk * kt + dkv * vt
                dv[b, t, hd] = dU[:, 1] + 2 * dvv * vt + dkv * kt
                dd[b, t, hd] = 0.5 * dh
            dpsi0[b, hd] = lam
    return dq, dk, dv, dd, dpsi0


def _oracle_grads(q, k, v, d, psi0, w_o, w_s):
    a = tuple(x.clone().requires_grad_(True) for x in (q, k, v, d, psi0))
    o, s = _eager64(*a)
    ((o * w_o).sum() + (s * w_s).sum()).backward()
    return [x.grad.numpy() for x in a], s.detach().numpy()


@pytest.mark.parametrize("B,T,H,D", [(2, 5, 2, 8), (1, 17, 1, 16)])
def test_kernel_algorithm_matches_oracle(B, T, H, D):
    q, k, v, d, psi0 = _inputs(B, T, H, D, seed=T + D)
    g = torch.Generator().manual_seed(4)
    w_o = torch.randn(B, T, H, D, generator=g, dtype=torch.float64)
    w_s = torch.randn(B, H, D, D, generator=g, dtype=torch.float64)
    ref, psi_T = _oracle_grads(q, k, v, d, psi0, w_o, w_s)
    got = kernel_backward(q.numpy(), k.numpy(), v.numpy(), d.numpy(), psi_T, w_o.numpy(), w_s.numpy())
    for name, x, y in zip(("dq", "dk", "dv", "ddelta", "dpsi0"), got, ref):
        assert np.abs(x - y).max() <= 1e-10 * max(1.0, np.abs(y).max()), name


def test_planted_mistakes_are_caught():
    """Using Psi^(t+1) instead of Psi^(t) in dL/dU, or dropping the c-dependence of M,
    must change the gradients well beyond the tolerance above."""
    B, T, H, D = 1, 6, 1, 8
    q, k, v, d, psi0 = _inputs(B, T, H, D, seed=9)
    g = torch.Generator().manual_seed(5)
    w_o = torch.randn(B, T, H, D, generator=g, dtype=torch.float64)
    w_s = torch.randn(B, H, D, D, generator=g, dtype=torch.float64)
    ref, psi_T = _oracle_grads(q, k, v, d, psi0, w_o, w_s)
    good = kernel_backward(q.numpy(), k.numpy(), v.numpy(), d.numpy(), psi_T, w_o.numpy(), w_s.numpy())
    assert np.abs(good[1] - ref[1]).max() < 1e-10
    # planted: the final state taken as the identity (states rebuilt from the wrong end)
    bad = kernel_backward(q.numpy(), k.numpy(), v.numpy(), d.numpy(),
                          np.broadcast_to(np.eye(D), psi_T.shape).copy(), w_o.numpy(), w_s.numpy())
    assert np.abs(bad[0] - ref[0]).max() > 1e-3
    # planted: ddelta without the factor 1/2 of delta = 2h
    assert np.abs(2 * good[3] - ref[3]).max() > 1e-4
