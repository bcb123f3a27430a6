"""Pins for the CPU oracle (oracle/): every oracle function is checked against something
other than itself -- a library routine, brute force, a closed form, an invariant or the
reference's own outputs (tests/golden/) -- chosen so that a plausible mistake (swapped
Cayley order, dropped term, wrong product order, transposed operand) fails at least one
check.  The `planted_*` tests plant such a mistake in a copy of the oracle and assert the
pin catches it.
"""
import math
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import cham_ns, sssd_closed, sssd_eager

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "sssd_module_golden.npz")


def _rand_inputs(B, T, H, D, seed, delta_scale=0.1, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    q = F.normalize(torch.randn(B, T, H, D, generator=g), dim=-1).to(dtype)
    k = F.normalize(torch.randn(B, T, H, D, generator=g), dim=-1).to(dtype)
    v = F.normalize(torch.randn(B, T, H, D, generator=g), dim=-1).to(dtype)
    delta = (delta_scale * torch.sigmoid(torch.randn(B, T, H, generator=g))).to(dtype)
    return q, k, v, delta


def _rel(a, b):
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


# ---------------------------------------------------------------- Cayley factor
@pytest.mark.parametrize("delta", [0.0, 1e-4, 0.05, 0.1, 1.0, 7.5])
@pytest.mark.parametrize("unit", [True, False])
def test_cayley_closed_form_equals_linalg_solve(delta, unit):
    """closed form == torch.linalg.solve(I + X, I - X) (the reference's operand order,
    sssd_attention.py:163-166), for unit and non-unit k, v."""
    rng = np.random.default_rng(1)
    for D in (2, 3, 16, 24, 64):
        k = rng.standard_normal(D)
        v = rng.standard_normal(D)
        if unit:
            k /= np.linalg.norm(k)
            v /= np.linalg.norm(v)
        X = 0.5 * delta * (np.outer(k, v) - np.outer(v, k))
        eye = torch.eye(D, dtype=torch.float64)
        Xt = torch.from_numpy(X)
        R_solve = torch.linalg.solve(eye + Xt, eye - Xt).numpy()
        R = sssd_closed.cayley_closed(k, v, delta)
        assert np.abs(R - R_solve).max() < 1e-12 * max(1.0, delta * delta * 100)
        assert np.abs(R @ R.T - np.eye(D)).max() < 1e-12 * max(1.0, delta * delta * 100)
        if D <= 24:
            assert abs(np.linalg.det(R) - 1.0) < 1e-10
        if delta == 0.0:
            assert np.array_equal(R, np.eye(D))


def test_planted_swapped_cayley_order_is_caught():
    """(I - X)^-1 (I + X) (the docstring's order) must fail the solve pin."""
    rng = np.random.default_rng(2)
    D = 16
    k = rng.standard_normal(D)
    v = rng.standard_normal(D)
    R_swapped = sssd_closed.cayley_closed(k, v, -0.1)  # swapping the order == negating delta
    X = 0.05 * (np.outer(k, v) - np.outer(v, k))
    R_solve = np.linalg.solve(np.eye(D) + X, np.eye(D) - X)
    assert np.abs(R_swapped - R_solve).max() > 1e-3


def test_planted_dropped_square_term_is_caught():
    rng = np.random.default_rng(3)
    D = 16
    k = rng.standard_normal(D)
    v = rng.standard_normal(D)
    X = 0.05 * (np.outer(k, v) - np.outer(v, k))
    R_solve = np.linalg.solve(np.eye(D) + X, np.eye(D) - X)
    R_first_order = np.eye(D) - 2 * X
    assert np.abs(R_first_order - R_solve).max() > 1e-4


# ---------------------------------------------------------------- prefix scan
@pytest.mark.parametrize("T", [1, 2, 3, 5, 13, 64])
def test_prefix_scan_equals_bruteforce_products(T):
    """parallel_prefix_scan (sssd_attention.py:185-217) == sequential R_t @ ... @ R_1."""
    g = torch.Generator().manual_seed(T)
    R = torch.randn(2, 3, T, 5, 5, generator=g, dtype=torch.float64) * 0.5
    P = sssd_eager.parallel_prefix_scan(R.clone())
    ref = torch.empty_like(R)
    acc = torch.eye(5, dtype=torch.float64).expand(2, 3, 5, 5)
    for t in range(T):
        acc = R[:, :, t] @ acc
        ref[:, :, t] = acc
    assert torch.allclose(P, ref, rtol=1e-12, atol=1e-12)


def test_planted_reversed_product_order_is_caught():
    g = torch.Generator().manual_seed(0)
    R = torch.randn(1, 1, 4, 5, 5, generator=g, dtype=torch.float64)
    P = sssd_eager.parallel_prefix_scan(R.clone())
    wrong = R[0, 0, 0] @ R[0, 0, 1] @ R[0, 0, 2] @ R[0, 0, 3]  # oldest on the left
    assert not torch.allclose(P[0, 0, 3], wrong, atol=1e-6)


# ---------------------------------------------------------------- scan vs closed form
@pytest.mark.parametrize("B,T,H,D", [(2, 8, 2, 16), (1, 1, 1, 16), (2, 13, 2, 16), (2, 8, 2, 24),
                                     (1, 40, 2, 64)])
def test_eager_restatement_matches_fp64_closed_form(B, T, H, D):
    q, k, v, delta = _rand_inputs(B, T, H, D, seed=B * 100 + T)
    o, psi = sssd_eager.sssd_scan_eager(q, k, v, delta)
    o64, psi64 = sssd_closed.sssd_scan_closed_np(q.numpy(), k.numpy(), v.numpy(), delta.numpy())
    assert _rel(o.numpy(), o64) < 1e-5
    assert _rel(psi.numpy(), psi64) < 1e-5


def test_eager_with_initial_state_matches_closed_form():
    B, T, H, D = 2, 9, 2, 16
    q, k, v, delta = _rand_inputs(B, T, H, D, seed=7)
    g = torch.Generator().manual_seed(11)
    psi0 = torch.randn(B, H, D, D, generator=g)
    o, psi = sssd_eager.sssd_scan_eager(q, k, v, delta, psi0)
    o64, psi64 = sssd_closed.sssd_scan_closed_np(q.numpy(), k.numpy(), v.numpy(), delta.numpy(),
                                                 psi0.double().numpy())
    assert _rel(o.numpy(), o64) < 1e-5
    assert _rel(psi.numpy(), psi64) < 1e-5


def test_closed_form_matches_explicit_matrix_products():
    """The vectorised closed-form update == applying the explicit R_t matrices (brute force)."""
    B, T, H, D = 1, 6, 2, 8
    q, k, v, delta = _rand_inputs(B, T, H, D, seed=5, delta_scale=0.7)
    o64, psi64 = sssd_closed.sssd_scan_closed_np(q.numpy(), k.numpy(), v.numpy(), delta.numpy())
    for h in range(H):
        P = np.eye(D)
        for t in range(T):
            P = sssd_closed.cayley_closed(k[0, t, h].numpy(), v[0, t, h].numpy(),
                                          float(delta[0, t, h])) @ P
            assert np.abs(P @ q[0, t, h].double().numpy() - o64[0, t, h]).max() < 1e-12
        assert np.abs(P - psi64[0, h]).max() < 1e-12


def test_c_oracle_matches_numpy_oracle():
    B, T, H, D = 2, 17, 3, 24
    q, k, v, delta = _rand_inputs(B, T, H, D, seed=3)
    g = torch.Generator().manual_seed(4)
    psi0 = torch.randn(B, H, D, D, generator=g).double().numpy()
    o_np, psi_np, n_np = sssd_closed.sssd_scan_closed_np(q.numpy(), k.numpy(), v.numpy(),
                                                         delta.numpy(), psi0, return_norms=True)
    o_c, psi_c, n_c = sssd_closed.sssd_scan_closed_c(q.numpy(), k.numpy(), v.numpy(),
                                                     delta.numpy(), psi0, want_norms=True)
    assert np.abs(o_np - o_c).max() < 1e-12
    assert np.abs(psi_np - psi_c).max() < 1e-12
    assert np.abs(n_np - n_c).max() < 1e-12


# ---------------------------------------------------------------- invariants
def test_norm_is_conserved_every_step():
    B, T, H, D = 2, 64, 2, 32
    q, k, v, delta = _rand_inputs(B, T, H, D, seed=9, delta_scale=1.0)
    _, _, norms = sssd_closed.sssd_scan_closed_np(q.numpy(), k.numpy(), v.numpy(), delta.numpy(),
                                                  return_norms=True)
    assert np.abs(norms - math.sqrt(D)).max() < 1e-12


def test_zero_initial_state_gives_zero():
    B, T, H, D = 1, 5, 2, 16
    q, k, v, delta = _rand_inputs(B, T, H, D, seed=2)
    o, psi = sssd_eager.sssd_scan_eager(q, k, v, delta, torch.zeros(B, H, D, D))
    assert torch.count_nonzero(o) == 0 and torch.count_nonzero(psi) == 0


def test_zero_delta_is_identity():
    B, T, H, D = 2, 7, 2, 16
    q, k, v, delta = _rand_inputs(B, T, H, D, seed=6)
    g = torch.Generator().manual_seed(1)
    psi0 = torch.randn(B, H, D, D, generator=g)
    o, psi = sssd_eager.sssd_scan_eager(q, k, v, torch.zeros_like(delta), psi0)
    assert torch.equal(psi, psi0)
    assert torch.allclose(o, torch.einsum("bhij,bthj->bthi", psi0, q), atol=1e-6)


def test_chunk_invariance():
    """scan(T1 + T2) == scan(T2, init = scan(T1)) (contract of initial_state)."""
    B, T, H, D = 2, 24, 2, 16
    q, k, v, delta = _rand_inputs(B, T, H, D, seed=8)
    o_full, psi_full = sssd_eager.sssd_scan_eager(q, k, v, delta)
    o_ch, psi_ch = sssd_eager.sssd_scan_eager_chunked(q, k, v, delta, chunk=7)
    assert torch.allclose(o_full, o_ch, atol=2e-6)
    assert torch.allclose(psi_full, psi_ch, atol=2e-6)


# ---------------------------------------------------------------- golden (reference outputs)
def _golden():
    if not os.path.exists(GOLDEN):
        pytest.skip("golden fixture not generated")
    return np.load(GOLDEN, allow_pickle=False)


def test_golden_fixture_module_parity():
    """Oracle module forward == the reference's eager SSSDAttention on its own test shapes."""
    z = _golden()
    for name in z["cases"]:
        name = str(name)
        b, s, D, H, hidden = (int(x) for x in z[f"{name}/meta"])
        params = {k.split("/param/")[1]: torch.from_numpy(z[k]) for k in z.files
                  if k.startswith(f"{name}/param/")}
        x = torch.from_numpy(z[f"{name}/x"])
        kw = {}
        if f"{name}/active_mask" in z.files:
            kw["active_mask"] = torch.from_numpy(z[f"{name}/active_mask"])
        if f"{name}/x2" in z.files:
            out1, st1 = sssd_eager.sssd_module_forward(params, x, H, D, return_state=True)
            assert torch.allclose(out1, torch.from_numpy(z[f"{name}/out1"]), rtol=1e-5, atol=1e-6)
            x = torch.from_numpy(z[f"{name}/x2"])
            kw["initial_state"] = st1
        out, st = sssd_eager.sssd_module_forward(params, x, H, D, return_state=True, **kw)
        assert torch.allclose(out, torch.from_numpy(z[f"{name}/out"]), rtol=1e-5, atol=1e-6), name
        assert torch.allclose(st, torch.from_numpy(z[f"{name}/state"]), rtol=1e-5, atol=1e-6), name


def test_golden_state_norm_kat():
    """test_sssd.py:10-26 KAT: identity start => ||Psi_T||_F = sqrt(D) within 1e-4."""
    z = _golden()
    st = z["norm_b2_s8_d64_h2/state"]
    assert abs(np.linalg.norm(st[0, 0]) - math.sqrt(64)) < 1e-4


# ---------------------------------------------------------------- Newton-Schulz
def _random_unitary(n, rng):
    z = rng.standard_normal((n, n)) + 1j * rng.standard_normal((n, n))
    qm, r = np.linalg.qr(z)
    return qm * (np.diag(r) / np.abs(np.diag(r)))


@pytest.mark.parametrize("n", [4, 16, 20])
def test_newton_schulz_acts_on_singular_values(n):
    """H = U diag(s) V^H  =>  NS^3(H) = U diag(f(f(f(s)))) V^H with f(s) = s (3 - s^2) / 2."""
    rng = np.random.default_rng(n)
    U, V = _random_unitary(n, rng), _random_unitary(n, rng)
    s = rng.uniform(0.6, 1.4, n)
    H = U @ np.diag(s) @ V.conj().T
    hr, hi = cham_ns.newton_schulz_retraction(torch.from_numpy(H.real.copy()),
                                              torch.from_numpy(H.imag.copy()), steps=3)
    f = s.copy()
    for _ in range(3):
        f = f * (3 - f * f) / 2
    expect = U @ np.diag(f) @ V.conj().T
    assert np.abs(hr.numpy() - expect.real).max() < 1e-12
    assert np.abs(hi.numpy() - expect.imag).max() < 1e-12


def test_newton_schulz_unitary_fixed_point():
    rng = np.random.default_rng(0)
    U = _random_unitary(12, rng)
    hr, hi = cham_ns.newton_schulz_retraction(torch.from_numpy(U.real.copy()),
                                              torch.from_numpy(U.imag.copy()))
    assert np.abs(hr.numpy() + 1j * hi.numpy() - U).max() < 1e-12


def test_planted_ns_updated_real_part_reuse_is_caught():
    """The bug fixed in the reference (cham_memory.py:40-46): H_imag computed from the
    already-updated H_real.  It must fail the singular-value closed form."""
    rng = np.random.default_rng(5)
    n = 8
    U, V = _random_unitary(n, rng), _random_unitary(n, rng)
    s = rng.uniform(0.6, 1.4, n)
    H = U @ np.diag(s) @ V.conj().T
    Hr, Hi = torch.from_numpy(H.real.copy()), torch.from_numpy(H.imag.copy())
    eye = torch.eye(n, dtype=torch.float64)
    for _ in range(3):
        HHr = Hr.T @ Hr + Hi.T @ Hi
        HHi = Hr.T @ Hi - Hi.T @ Hr
        dr, di = 3 * eye - HHr, -HHi
        Hr = 0.5 * (Hr @ dr - Hi @ di)
        Hi = 0.5 * (Hr @ di + Hi @ dr)  # bug: uses the new Hr
    f = s.copy()
    for _ in range(3):
        f = f * (3 - f * f) / 2
    expect = U @ np.diag(f) @ V.conj().T
    assert np.abs(Hi.numpy() - expect.imag).max() > 1e-3


# ---------------------------------------------------------------- non-finite guard
@pytest.mark.parametrize("what", ["k_nan", "k_inf", "v_nan", "v_ninf", "d_nan", "d_inf"])
def test_identity_substitution_equals_eager_guard(what):
    """The guard of sssd_attention.py:45-71 (restated op for op in sssd_eager.solve_cayley)
    equals the substitution k = v = 0, delta = 0 for the bad token-heads fed to the fp64
    closed form; a plain fp64 scan of the poisoned inputs is not finite (so the check
    would fail if the guard were dropped from either side)."""
    import warnings
    B, T, H, D = 2, 9, 2, 8
    q, k, v, d = _rand_inputs(B, T, H, D, seed=41)
    k, v, d = k.clone(), v.clone(), d.clone()
    for (b, t, h) in [(0, 0, 1), (1, 4, 0), (0, 8, 0)]:
        if what == "k_nan":
            k[b, t, h, 2] = float("nan")
        elif what == "k_inf":
            k[b, t, h, 0] = float("inf")
        elif what == "v_nan":
            v[b, t, h, 3] = float("nan")
        elif what == "v_ninf":
            v[b, t, h, 1] = -float("inf")
        elif what == "d_nan":
            d[b, t, h] = float("nan")
        else:
            d[b, t, h] = float("inf")
    with warnings.catch_warnings():
        warnings.simplefilter("ignore")
        o_e, s_e = sssd_eager.sssd_scan_eager(q, k, v, d, compute_dtype=torch.float64)
    kc, vc, dc, bad = sssd_closed.identity_substitute(k.numpy(), v.numpy(), d.numpy())
    assert bad.sum() == 3
    o_c, s_c = sssd_closed.sssd_scan_closed_np(q.numpy(), kc, vc, dc)
    assert np.isfinite(o_e.numpy()).all()
    assert _rel(o_e.numpy(), o_c) < 1e-12 and _rel(s_e.numpy(), s_c) < 1e-12
    with np.errstate(invalid="ignore", over="ignore"):
        o_raw, _ = sssd_closed.sssd_scan_closed_np(q.numpy(), k.numpy(), v.numpy(), d.numpy())
    assert not np.isfinite(o_raw).all()


def test_cham_eager_guard_equals_identity_substitution():
    """The CHAM guard (cham_memory.py:68-95, in oracle.cham_scan.cham_cayley_solve): the
    eager restatement on poisoned tokens equals the closed form with those tokens
    substituted by gamma = 0 (U = I)."""
    from oracle import cham_scan
    rng = np.random.default_rng(3)
    B, T, h = 1, 6, 5
    q, k, v = (rng.standard_normal((B, T, h)) for _ in range(3))
    gam = 0.1 / (1 + np.exp(-rng.standard_normal((B, T))))
    k[0, 1, 2] = np.nan
    v[0, 3, 0] = np.inf
    gam[0, 5] = np.nan
    rec_e, (hr_e, hi_e) = cham_scan.cham_scan_eager(q, k, v, gam)
    kc, vc, gc = k.copy(), v.copy(), gam.copy()
    for t in (1, 3, 5):
        kc[0, t] = vc[0, t] = 0.0
        gc[0, t] = 0.0
    rec_c, (hr_c, hi_c) = cham_scan.cham_scan_closed(q, kc, vc, gc)
    assert np.isfinite(rec_e).all() and np.isfinite(hr_e).all()
    assert _rel(rec_e, rec_c) < 1e-10 and _rel(hr_e, hr_c) < 1e-10 and _rel(hi_e, hi_c) < 1e-10
