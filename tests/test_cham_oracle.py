"""Pins of the CHAM scan restatement (oracle/cham_scan.py), CPU only.

* The Woodbury closed form of the Cayley factor against ``np.linalg.solve`` (a library
  routine), for unit and non-unit k, v and gamma = 0 (U = I exactly).
* The kernels' own closed form N = (2/det)[[-g^2 vv, i g + g^2 kv], [i g + g^2 kv,
  -g^2 kk]] (a second derivation, U = 2 (I - X)^-1 - I) against the same solve.
* The matrix-free readout NS_3(H) q = H f_3(H^H H) q against the matrix Newton-Schulz
  iteration (oracle.cham_ns, itself pinned in test_oracle_pins.py), and the kernels'
  13-step unrolled schedule of f_3 against the recursion.
* The closed-form scan against the op-for-op eager restatement, and planted mistakes
  (H_0 on the wrong side, the product order reversed) that it must catch.
"""
import numpy as np
import pytest
import torch

from oracle import cham_scan
from oracle.cham_ns import newton_schulz_retraction


def _unit(x):
    return x / np.linalg.norm(x)


@pytest.mark.parametrize("gamma", [0.0, 1e-3, 0.07, 0.1, 3.0])
@pytest.mark.parametrize("unit", [True, False])
def test_cayley_closed_form_matches_solve(gamma, unit):
    rng = np.random.default_rng(1)
    h = 12
    k, v = rng.standard_normal(h), rng.standard_normal(h)
    if unit:
        k, v = _unit(k), _unit(v)
    U = cham_scan.cham_cayley_solve(k, v, gamma)
    W = np.stack([k, v], 1)
    N = cham_scan.cham_cayley_closed(k, v, gamma)
    assert np.abs(np.eye(h) + W @ N @ W.T - U).max() < 1e-12
    assert np.abs(U.conj().T @ U - np.eye(h)).max() < 1e-12
    if gamma == 0.0:
        assert np.array_equal(N, np.zeros((2, 2)))


def _kernel_n(gamma, kk, vv, kv):
    """The closed form the kernels evaluate (csrc/cham_scan.hip, cayley_n)."""
    g = 0.5 * gamma
    det = 1 + g * g * (kk * vv - kv * kv) - 2j * g * kv
    return (2 / det) * np.array([[-g * g * vv, 1j * g + g * g * kv], [1j * g + g * g * kv, -g * g * kk]])


@pytest.mark.parametrize("gamma", [0.0, 0.05, 0.1, 2.5])
def test_kernel_closed_form_matches_solve(gamma):
    rng = np.random.default_rng(2)
    for unit in (True, False):
        k, v = rng.standard_normal(9), rng.standard_normal(9)
        if unit:
            k, v = _unit(k), _unit(v)
        W = np.stack([k, v], 1)
        N = _kernel_n(gamma, k @ k, v @ v, k @ v)
        U = cham_scan.cham_cayley_solve(k, v, gamma)
        assert np.abs(np.eye(9) + W @ N @ W.T - U).max() < 1e-12


def _rand_h(rng, h, eps):
    """A complex matrix near a unitary one (NS converges) or a generic one."""
    Q = np.linalg.qr(rng.standard_normal((h, h)) + 1j * rng.standard_normal((h, h)))[0]
    return Q + eps * (rng.standard_normal((h, h)) + 1j * rng.standard_normal((h, h)))


@pytest.mark.parametrize("eps", [0.0, 1e-3, 0.1])
def test_matrix_free_readout_matches_matrix_newton_schulz(eps):
    rng = np.random.default_rng(3)
    h = 10
    H = _rand_h(rng, h, eps)
    q = rng.standard_normal(h)
    Rr, Ri = newton_schulz_retraction(torch.from_numpy(H.real.copy()), torch.from_numpy(H.imag.copy()), 3)
    ref = (Rr.numpy() + 1j * Ri.numpy()) @ q
    assert np.abs(cham_scan.ns_apply(H, q, 3) - ref).max() < 1e-12


def _kernel_schedule(H, x):
    """The kernels' unrolled f_3 (csrc/cham_scan.hip, apply_f3), then H y."""
    A = lambda z: H.conj().T @ (H @ z)
    cur = x.astype(np.complex128)
    X2, X3 = cur.copy(), cur.copy()
    for st in range(13):
        s4 = (st & 3) if st < 8 else (4 if st == 8 else (st - 9) & 3)
        if s4 in (0, 1):
            c = (1.5, 0.0, 0.0, -0.5)
        elif s4 == 2:
            c = (0.0, 3.0, 0.0, -1.0)
        elif s4 == 3:
            c = (0.375, 0.0, 0.0, -0.125) if st == 12 else (0.75, 0.0, 0.0, -0.25)
        else:
            c = (0.0, 0.0, 3.0, -1.0)
        a = A(cur)
        cur = c[0] * cur + c[1] * X2 + c[2] * X3 + c[3] * a
        if st in (3, 8):
            X2 = cur.copy()
    return H @ cur


def test_kernel_schedule_matches_recursion():
    rng = np.random.default_rng(4)
    for eps in (0.0, 0.05):
        H = _rand_h(rng, 8, eps)
        q = rng.standard_normal(8)
        assert np.abs(_kernel_schedule(H, q) - cham_scan.ns_apply(H, q, 3)).max() < 1e-12


def _inputs(B, T, h, seed, zero_gamma_every=0):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((B, T, h)); q /= np.linalg.norm(q, axis=-1, keepdims=True)
    k = rng.standard_normal((B, T, h)); k /= np.linalg.norm(k, axis=-1, keepdims=True)
    v = rng.standard_normal((B, T, h)); v /= np.linalg.norm(v, axis=-1, keepdims=True)
    g = 0.1 / (1 + np.exp(-rng.standard_normal((B, T))))
    if zero_gamma_every:
        g[:, ::zero_gamma_every] = 0.0
    return q, k, v, g


def test_closed_scan_matches_eager_restatement():
    B, T, h = 2, 6, 7
    q, k, v, g = _inputs(B, T, h, 5, zero_gamma_every=3)
    rng = np.random.default_rng(6)
    H0 = np.stack([_rand_h(rng, h, 0.0) for _ in range(B)])
    r1, (hr1, hi1) = cham_scan.cham_scan_eager(q, k, v, g, H0.real, H0.imag)
    r2, (hr2, hi2) = cham_scan.cham_scan_closed(q, k, v, g, H0.real, H0.imag)
    assert np.abs(r1 - r2).max() < 1e-11
    assert np.abs(hr1 - hr2).max() < 1e-12 and np.abs(hi1 - hi2).max() < 1e-12
    # identity start and all-zero gamma: the state stays exactly the identity
    r3, (hr3, hi3) = cham_scan.cham_scan_closed(q, k, v, np.zeros_like(g))
    assert np.array_equal(hr3, np.broadcast_to(np.eye(h), hr3.shape)) and not hi3.any()


def test_planted_mistakes_are_caught():
    B, T, h = 1, 4, 5
    q, k, v, g = _inputs(B, T, h, 7)
    g = g * 10.0  # large rotations make every ordering mistake visible
    rng = np.random.default_rng(8)
    H0 = _rand_h(rng, h, 0.0)[None]
    ref, (hr, hi) = cham_scan.cham_scan_eager(q, k, v, g, H0.real, H0.imag)
    # H_0 on the left (H_0 P_t instead of P_t H_0) and the product order reversed
    P = np.eye(h, dtype=np.complex128)
    P_rev = np.eye(h, dtype=np.complex128)
    for t in range(T):
        U = cham_scan.cham_cayley_solve(k[0, t], v[0, t], g[0, t])
        P = U @ P
        P_rev = P_rev @ U
    good = P @ H0[0]
    assert np.abs(good - (hr[0] + 1j * hi[0])).max() < 1e-12
    assert np.abs(H0[0] @ P - good).max() > 1e-3
    assert np.abs(P_rev @ H0[0] - good).max() > 1e-3


@pytest.mark.parametrize("eps", [0.0, 0.05])
def test_readout_identity_ns_of_carried_state(eps):
    """The kernels read out NS_3(H_t) q as P_t NS_3(H_0) q (every Cayley factor is unitary,
    so H_t^H H_t = H_0^H H_0): check against NS_3 evaluated on every H_t, for a unitary and
    a non-unitary H_0, and that the identity start reduces it to Re(H_t q)."""
    B, T, h = 1, 9, 6
    q, k, v, g = _inputs(B, T, h, 11)
    g = g * 5.0
    rng = np.random.default_rng(12)
    H0 = _rand_h(rng, h, eps)
    Rr, Ri = newton_schulz_retraction(torch.from_numpy(H0.real.copy()), torch.from_numpy(H0.imag.copy()), 3)
    R = Rr.numpy() + 1j * Ri.numpy()
    H = H0.copy()
    for t in range(T):
        U = cham_scan.cham_cayley_solve(k[0, t], v[0, t], g[0, t])
        H = U @ H
        R = U @ R
        assert np.abs(cham_scan.ns_apply(H, q[0, t], 3) - R @ q[0, t]).max() < 1e-10
    # identity start: NS_3(P_t) q = P_t q
    P = np.eye(h, dtype=np.complex128)
    for t in range(T):
        P = cham_scan.cham_cayley_solve(k[0, t], v[0, t], g[0, t]) @ P
        assert np.abs(cham_scan.ns_apply(P, q[0, t], 3) - P @ q[0, t]).max() < 1e-10
