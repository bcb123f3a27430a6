"""GPU parity on non-finite inputs: the reference's guard (``_solve_cayley``,
``sssd_attention.py:45-71``; ``_solve_cham_cayley``, ``cham_memory.py:68-95``) turns every
token whose Cayley factor is not finite -- a NaN or Inf in its k, v or delta (gamma) -- into
R = I, so the state stays finite and the other tokens are unaffected.

Tokens are poisoned at chunk boundaries (16-token chunks), at segment and pass-A piece
boundaries of the chunk scan's plan, at the first and last token, in the fused path (raw
projections and delta logits), in the decode step, in both backward kernels and in both CHAM
routes (h <= 128 and h > 128).

Oracles: the eager restatement of the guard (oracle/sssd_eager.py, fp32 and fp64), and the
fp64 closed form fed the guard as an input substitution (oracle.sssd_closed.identity_substitute:
k = v = 0 and delta = 0 for the bad token-heads, which yields R = I exactly; the
substitution is pinned against the eager guard in tests/test_oracle_pins.py).  Bars as in the
finite tests: fp32 1e-5, bf16/fp16 2e-2 relative Frobenius error per slice; every output and
state finite.  Gradients: wherever the eager fp64 autograd is finite it is matched (1e-5 fp32);
the bad token's own dk, dv, ddelta are exactly zero here (the eager chain rule yields 0 or
0 * NaN = NaN there, depending on which input was non-finite).
"""
import warnings

import numpy as np
import pytest
import torch

from oracle import cham_scan, sssd_closed, sssd_eager

pytestmark = pytest.mark.gpu

NAN, INF = float("nan"), float("inf")


def _rel(got, ref, slice_dims=None):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    if slice_dims is None:
        return float(np.sqrt(((got - ref) ** 2).sum()) / max(np.sqrt((ref ** 2).sum()), 1e-30))
    red = tuple(i for i in range(got.ndim) if i not in slice_dims)
    num = np.sqrt(((got - ref) ** 2).sum(axis=red))
    den = np.sqrt((ref ** 2).sum(axis=red))
    return float((num / np.maximum(den, 1e-30)).max())


def _inputs(B, T, H, D, seed):
    g = torch.Generator().manual_seed(seed)
    nrm = torch.nn.functional.normalize
    q = nrm(torch.randn(B, T, H, D, generator=g), dim=-1)
    k = nrm(torch.randn(B, T, H, D, generator=g), dim=-1)
    v = nrm(torch.randn(B, T, H, D, generator=g), dim=-1)
    d = 0.1 * torch.sigmoid(torch.randn(B, T, H, generator=g))
    return q, k, v, d


def _poison(k, v, d, points):
    """points: (b, t, h, what) with what in k_nan, k_inf, k_ninf, v_nan, v_inf, d_nan, d_inf."""
    k, v, d = k.clone(), v.clone(), d.clone()
    for b, t, h, what in points:
        if what == "k_nan":
            k[b, t, h, 3] = NAN
        elif what == "k_inf":
            k[b, t, h, 0] = INF
        elif what == "k_ninf":
            k[b, t, h, -1] = -INF
        elif what == "v_nan":
            v[b, t, h, 5] = NAN
        elif what == "v_inf":
            v[b, t, h, 1] = INF
        elif what == "d_nan":
            d[b, t, h] = NAN
        elif what == "d_inf":
            d[b, t, h] = INF
    return k, v, d


KINDS = ["k_nan", "k_inf", "k_ninf", "v_nan", "v_inf", "d_nan", "d_inf"]


def _points(B, T, H, ts):
    return [(i % B, t, (3 * i) % H, KINDS[i % len(KINDS)]) for i, t in enumerate(ts) if t < T]


def _closed_ref(q, k, v, d, psi0=None):
    kc, vc, dc, bad = sssd_closed.identity_substitute(k.double().numpy(), v.double().numpy(),
                                                      d.double().numpy())
    o, s = sssd_closed.sssd_scan_closed_c(q.double().numpy(), kc, vc, dc,
                                          None if psi0 is None else psi0.double().numpy())
    return o, s, bad


def _run_scan(device, q, k, v, d, psi0=None):
    from verace_amd import launch_sssd_hip_scan
    o, s = launch_sssd_hip_scan(q.to(device), k.to(device), v.to(device), d.to(device),
                                None if psi0 is None else psi0.to(device))
    torch.cuda.synchronize()
    return o.float().cpu(), s.cpu()


def test_scan_fp32_nonfinite_matches_eager_guard(device):
    """fp32 I/O (token-sequential kernel) against the fp32 eager restatement of the guard."""
    B, T, H, D = 2, 40, 2, 64
    print(f"[case] nonfinite seq fp32 B{B} T{T} H{H} D{D}", flush=True)
    q, k, v, d = _inputs(B, T, H, D, 11)
    k, v, d = _poison(k, v, d, _points(B, T, H, [0, 7, 15, 16, 17, 31, 32, 39]))
    o, s = _run_scan(device, q, k, v, d)
    with warnings.catch_warnings():
        warnings.simplefilter("ignore")
        o_e, s_e = sssd_eager.sssd_scan_eager(q, k, v, d)
    o_c, s_c, bad = _closed_ref(q, k, v, d)
    assert bad.sum() == 8
    assert torch.isfinite(o).all() and torch.isfinite(s).all()
    eo, es = _rel(o, o_e, (0, 2)), _rel(s, s_e, (0, 1))
    eo2, es2 = _rel(o, o_c, (0, 2)), _rel(s, s_c, (0, 1))
    print(f"  vs eager o={eo:.2e} psi={es:.2e}; vs closed o={eo2:.2e} psi={es2:.2e}", flush=True)
    assert max(eo, es, eo2, es2) <= 1e-5


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("B,T,H", [(1, 2048, 4), (32, 256, 4)])
def test_scan_chunked_nonfinite(device, dtype, B, T, H):
    """Chunk-parallel MFMA scan: (1, 2048, 4) runs 32 segments of 64 tokens, (32, 256, 4)
    two segments split into pass-A pieces at token 64; tokens poisoned on both sides of
    every kind of boundary, with an orthogonal initial state."""
    D = 128
    print(f"[case] nonfinite chunk {dtype} B{B} T{T} H{H}", flush=True)
    q, k, v, d = _inputs(B, T, H, D, 12)
    ts = [0, 15, 16, 31, 32, 63, 64, 65, 127, 128, 129, 255, 256, 511, 512, 1023, 1024, T - 1]
    k, v, d = _poison(k, v, d, _points(B, T, H, ts))
    q, k, v, d = (x.to(dtype) for x in (q, k, v, d))
    g = torch.Generator().manual_seed(5)
    psi0 = torch.linalg.qr(torch.randn(B, H, D, D, generator=g))[0].contiguous()
    o, s = _run_scan(device, q, k, v, d, psi0)
    o_c, s_c, bad = _closed_ref(q.float(), k.float(), v.float(), d.float(), psi0)
    assert bad.sum() >= 10
    assert torch.isfinite(o).all() and torch.isfinite(s).all()
    eo, es = _rel(o, o_c, (0, 2)), _rel(s, s_c, (0, 1))
    nrm = np.linalg.norm(s.double().numpy().reshape(B, H, -1), axis=-1) / np.sqrt(D)
    drift = float(np.abs(nrm - 1).max())
    print(f"  rel o={eo:.2e} psi={es:.2e} drift={drift:.2e}", flush=True)
    assert eo <= 2e-2 and es <= 2e-2 and drift <= 1e-4


def test_fused_nonfinite(device):
    """Fused path: NaN/Inf in the raw k, v projections and NaN delta logits (and a NaN k on a
    masked token) act as identity tokens; the RMSNorm'd outputs match the fp64 chain."""
    from verace_amd.hip_kernels import launch_sssd_hip_scan_fused, rms_default_eps
    B, T, H, D = 2, 300, 2, 128
    print(f"[case] nonfinite fused B{B} T{T} H{H}", flush=True)
    HD = H * D
    g = torch.Generator().manual_seed(13)
    proj = torch.randn(B, T, 3 * HD + H, generator=g)
    mask = torch.rand(B, T, generator=g) > 0.2
    mask[0, 40] = False
    proj[0, 40, HD + 2] = NAN                 # masked token with a NaN k
    proj[0, 15, HD + 5] = NAN                 # k, head 0
    proj[1, 16, HD + D + 7] = INF             # k, head 1
    proj[0, 63, 2 * HD + 1] = -INF            # v, head 0
    proj[1, 64, 2 * HD + D] = NAN             # v, head 1
    proj[0, 127, 3 * HD] = NAN                # delta logit, head 0
    proj[1, T - 1, 3 * HD + 1] = NAN          # delta logit, head 1
    proj = proj.bfloat16()
    w = 1.0 + 0.1 * torch.randn(D, generator=g)
    eps = rms_default_eps(torch.bfloat16)
    o, s = launch_sssd_hip_scan_fused(proj.to(device), H, D, mask.to(device), w.to(device), None, None)
    torch.cuda.synchronize()
    o, s = o.float().cpu(), s.cpu()
    # fp64 chain (sssd_attention.py:114-126), the guard as a substitution, RMSNorm (:177)
    p = proj.double().numpy()

    def unit(x):
        x = x.reshape(B, T, H, D)
        with np.errstate(invalid="ignore", over="ignore"):
            n = np.sqrt((x ** 2).sum(-1, keepdims=True))
            return x / np.maximum(n, 1e-12)

    qn, kn, vn = unit(p[..., :HD]), unit(p[..., HD:2 * HD]), unit(p[..., 2 * HD:3 * HD])
    with np.errstate(over="ignore"):
        dl = 0.1 / (1.0 + np.exp(-p[..., 3 * HD:3 * HD + H]))
    with np.errstate(invalid="ignore"):
        dl = dl * mask.numpy().astype(np.float64)[..., None]
    kc, vc, dc, bad = sssd_closed.identity_substitute(kn, vn, dl)
    assert bad.sum() == 7
    o_r, s_r = sssd_closed.sssd_scan_closed_c(qn, kc, vc, dc)
    o_r = o_r / np.sqrt((o_r ** 2).mean(-1, keepdims=True) + eps) * w.double().numpy()
    assert torch.isfinite(o).all() and torch.isfinite(s).all()
    eo, es = _rel(o, o_r, (0, 2)), _rel(s, s_r, (0, 1))
    print(f"  rel o={eo:.2e} psi={es:.2e}", flush=True)
    assert eo <= 2e-2 and es <= 2e-2


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("D", [128, 64])
def test_decode_step_nonfinite(device, dtype, D):
    """In-place decode step (the D = 128 persistent kernel and the D = 64 sequential one):
    a poisoned head keeps its state bit-exact, its output is Psi q, the others match."""
    from verace_amd import sssd_step_
    B, H = 4, 8
    print(f"[case] nonfinite step {dtype} D{D}", flush=True)
    q, k, v, d = _inputs(B, 1, H, D, 14)
    k, v, d = _poison(k, v, d, [(0, 0, 1, "k_nan"), (1, 0, 2, "v_inf"), (2, 0, 3, "d_nan"),
                                (3, 0, 7, "d_inf"), (3, 0, 0, "k_ninf")])
    q, k, v, d = (x.to(dtype) for x in (q, k, v, d))
    g = torch.Generator().manual_seed(6)
    psi0 = torch.linalg.qr(torch.randn(B, H, D, D, generator=g))[0].contiguous()
    state = psi0.to(device)
    o = sssd_step_(q.to(device), k.to(device), v.to(device), d.to(device), state)
    torch.cuda.synchronize()
    o, state = o.float().cpu(), state.cpu()
    o_c, s_c, bad = _closed_ref(q.float(), k.float(), v.float(), d.float(), psi0)
    assert bad.sum() == 5
    assert torch.isfinite(o).all() and torch.isfinite(state).all()
    for b, t, h in zip(*np.nonzero(bad)):
        assert torch.equal(state[b, h], psi0[b, h])
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    eo, es = _rel(o, o_c, (0, 2)), _rel(state, s_c, (0, 1))
    print(f"  rel o={eo:.2e} psi={es:.2e}", flush=True)
    assert eo <= tol and es <= tol


@pytest.mark.parametrize("T", [20, 80])
def test_backward_nonfinite(device, T):
    """Backward (per-token kernel for T < 32, chunked for T >= 32), fp32, D = 64, with an
    initial state and a state gradient."""
    from verace_amd import SSSDScanFunction
    B, H, D = 2, 2, 64
    print(f"[case] nonfinite backward T{T}", flush=True)
    q, k, v, d = _inputs(B, T, H, D, 15)
    pts = _points(B, T, H, [2, 15, 16, 19, 31, 32, 47, 48, 79])
    k, v, d = _poison(k, v, d, pts)
    g = torch.Generator().manual_seed(7)
    psi0 = torch.linalg.qr(torch.randn(B, H, D, D, generator=g))[0].contiguous()
    w_o = torch.randn(B, T, H, D, generator=g)
    w_s = torch.randn(B, H, D, D, generator=g)
    # eager fp64 autograd through the guard
    a = [x.double().clone().requires_grad_(True) for x in (q, k, v, d, psi0)]
    with warnings.catch_warnings():
        warnings.simplefilter("ignore")
        o_e, s_e = sssd_eager.sssd_scan_eager(*a[:4], a[4], compute_dtype=torch.float64)
        ((o_e * w_o.double()).sum() + (s_e * w_s.double()).sum()).backward()
    ref = [x.grad.numpy() for x in a]
    # HIP
    x = [t.to(device).clone().requires_grad_(True) for t in (q, k, v, d, psi0)]
    o, s = SSSDScanFunction.apply(*x)
    ((o * w_o.to(device)).sum() + (s * w_s.to(device)).sum()).backward()
    torch.cuda.synchronize()
    got = [t.grad.cpu().double().numpy() for t in x]
    assert all(np.isfinite(gg).all() for gg in got)
    bad = np.zeros((B, T, H), dtype=bool)
    for b, t, h, _ in pts:
        bad[b, t, h] = True
    names = ["dq", "dk", "dv", "ddelta", "dpsi0"]
    for i, name in enumerate(names):
        r, gg = ref[i], got[i]
        if name in ("dk", "dv", "ddelta"):
            assert (gg[bad] == 0).all(), name  # the identity token has no gradient
            keep = ~bad
            r, gg = r[keep], gg[keep]
        assert np.isfinite(r).all(), name
        e = _rel(gg, r)
        print(f"  {name} rel={e:.2e}", flush=True)
        assert e <= 1e-5, name


@pytest.mark.parametrize("h,T,init", [(64, 40, False), (64, 70, True), (256, 140, False),
                                      (300, 20, True)])
def test_cham_nonfinite(device, h, T, init):
    """CHAM scan, both routes (h <= 128 and the wide h > 128 one), with and without an
    initial hologram: poisoned tokens are U = I (the fp64 oracle's own guard, and the same
    tokens substituted by gamma = 0, k = v = 0)."""
    from verace_amd import launch_cham_hip_update
    B = 2
    print(f"[case] nonfinite cham h{h} T{T} init={init}", flush=True)
    g = torch.Generator().manual_seed(16)
    q = torch.nn.functional.normalize(torch.randn(B, T, h, generator=g), dim=-1)
    k = torch.nn.functional.normalize(torch.randn(B, T, h, generator=g), dim=-1)
    v = torch.nn.functional.normalize(torch.randn(B, T, h, generator=g), dim=-1)
    gam = 0.1 * torch.sigmoid(torch.randn(B, T, generator=g))
    k[0, 3, 7] = NAN
    v[1, 15, 0] = INF
    gam[0, 16] = NAN
    gam[1, T - 1] = INF
    k[1, 0, h - 1] = -INF
    h0 = None
    if init:
        a = torch.randn(B, h, h, generator=g) + 1j * torch.randn(B, h, h, generator=g)
        u = torch.linalg.qr(a)[0]
        h0 = (u.real.float().contiguous(), u.imag.float().contiguous())
    out, (hr, hi) = launch_cham_hip_update(q.to(device), k.to(device), v.to(device), gam.to(device),
                                           None if h0 is None else (h0[0].to(device), h0[1].to(device)))
    torch.cuda.synchronize()
    out, hr, hi = out.cpu(), hr.cpu(), hi.cpu()
    assert torch.isfinite(out).all() and torch.isfinite(hr).all() and torch.isfinite(hi).all()
    kc, vc, gc = k.double().numpy().copy(), v.double().numpy().copy(), gam.double().numpy().copy()
    for b, t in [(0, 3), (1, 15), (0, 16), (1, T - 1), (1, 0)]:
        kc[b, t] = 0.0
        vc[b, t] = 0.0
        gc[b, t] = 0.0
    h0n = (None, None) if h0 is None else (h0[0].double().numpy(), h0[1].double().numpy())
    ref, (rr, ri) = cham_scan.cham_scan_closed(q.double().numpy(), kc, vc, gc, *h0n)
    eo = _rel(out, ref, (0,))
    es = max(_rel(hr, rr, (0,)), _rel(hi, ri, (0,)) if np.abs(ri).max() > 0 else 0.0)
    print(f"  rel out={eo:.2e} state={es:.2e}", flush=True)
    assert eo <= 1e-5 and es <= 1e-5
