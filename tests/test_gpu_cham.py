"""GPU parity of the CHAM holographic scan (vmi_cham_scan_fwd / launch_cham_hip_update)
against the fp64 restatement oracle/cham_scan.py (the closed-form scan, itself pinned to
the op-for-op eager restatement and to linalg.solve in tests/test_cham_oracle.py).

Shapes follow the reference's own CHAM tests (test_triton_kernels.py:153-279: (b, s, h) =
(2, 8, 16), (1, 1, 16), (2, 5, 16), (2, 8, 20), halted tokens, gamma = 0 everywhere, s =
100) plus h = 64 and 128 and chained calls; h > 128 (the reference's tiled route, up to
its default 1024) at ragged h and T crossing the 64-token readout chunks, from the
identity, a unitary and a non-unitary initial hologram.  Bars: fp32 I/O, out and final state within
1e-5 relative Frobenius error per batch item (the survey's fp32 bar); bf16 I/O within
2e-2; an all-halted sequence leaves the state bit-exact (N = 0 exactly at gamma = 0).
"""
import numpy as np
import pytest
import torch

from oracle import cham_scan

pytestmark = pytest.mark.gpu


def _inputs(B, T, h, seed, dtype=torch.float32, halted=None):
    g = torch.Generator().manual_seed(seed)
    q = torch.nn.functional.normalize(torch.randn(B, T, h, generator=g), dim=-1)
    k = torch.nn.functional.normalize(torch.randn(B, T, h, generator=g), dim=-1)
    v = torch.nn.functional.normalize(torch.nn.functional.silu(torch.randn(B, T, h, generator=g)), dim=-1)
    gam = 0.1 * torch.sigmoid(torch.randn(B, T, generator=g))
    if halted is not None:
        gam = gam * halted
    return q.to(dtype), k.to(dtype), v.to(dtype), gam.to(dtype)


def _rel(got, ref, axis=0):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    red = tuple(i for i in range(got.ndim) if i != axis)
    num = np.sqrt(((got - ref) ** 2).sum(axis=red))
    den = np.sqrt((ref ** 2).sum(axis=red))
    return float((num / np.maximum(den, 1e-30)).max())


def _run(device, q, k, v, gam, h0=None):
    from verace_amd import launch_cham_hip_update
    init = None if h0 is None else (h0[0].to(device), h0[1].to(device))
    out, (hr, hi) = launch_cham_hip_update(q.to(device), k.to(device), v.to(device), gam.to(device), init)
    torch.cuda.synchronize()
    return out.float().cpu(), hr.cpu(), hi.cpu()


def _check(device, B, T, h, seed, dtype=torch.float32, halted=None, h0=None, label=""):
    q, k, v, gam = _inputs(B, T, h, seed, dtype, halted)
    out, hr, hi = _run(device, q, k, v, gam, h0)
    ref, (rr, ri) = cham_scan.cham_scan_closed(q.double().numpy(), k.double().numpy(),
                                               v.double().numpy(), gam.double().numpy(),
                                               None if h0 is None else h0[0].double().numpy(),
                                               None if h0 is None else h0[1].double().numpy())
    eo = _rel(out, ref)
    es = max(_rel(hr, rr), _rel(hi, ri) if np.abs(ri).max() > 0 else 0.0)
    print(f"[cham {label} {dtype} B{B} T{T} h{h}] rel out={eo:.2e} state={es:.2e}", flush=True)
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    assert eo <= tol and es <= (1e-5 if dtype == torch.float32 else 1e-3)
    return out, hr, hi


@pytest.mark.parametrize("B,T,h", [(2, 8, 16), (1, 1, 16), (2, 5, 16), (2, 8, 20), (2, 100, 16),
                                   (2, 40, 64), (1, 48, 128)])
def test_cham_scan_matches_oracle(device, B, T, h):
    print(f"[case] cham B={B} T={T} h={h}", flush=True)
    _check(device, B, T, h, seed=B * 100 + T + h, label="fp32")


def test_cham_scan_bf16_inputs(device):
    print("[case] cham bf16", flush=True)
    _check(device, 2, 33, 128, seed=9, dtype=torch.bfloat16, label="bf16")


def test_cham_scan_halted_tokens_and_initial_state(device):
    print("[case] cham halted + H0", flush=True)
    B, T, h = 2, 10, 16
    halted = torch.ones(B, T)
    halted[:, T // 2:] = 0.0
    g = torch.Generator().manual_seed(11)
    Q = torch.linalg.qr(torch.complex(torch.randn(B, h, h, generator=g), torch.randn(B, h, h, generator=g)))[0]
    _check(device, B, T, h, seed=4, halted=halted, h0=(Q.real.contiguous(), Q.imag.contiguous()), label="halted")


def test_cham_scan_all_halted_keeps_state_exactly(device):
    print("[case] cham all halted", flush=True)
    B, T, h = 2, 12, 16
    q, k, v, gam = _inputs(B, T, h, 5, halted=torch.zeros(B, T))
    out, hr, hi = _run(device, q, k, v, gam)
    assert torch.equal(hr, torch.eye(h).expand(B, h, h)) and torch.count_nonzero(hi) == 0
    assert torch.isfinite(out).all()
    # readout of the identity: NS_3(I) q = q
    assert torch.allclose(out, q, atol=1e-6)


def test_cham_scan_chaining_through_initial_state(device):
    print("[case] cham chaining", flush=True)
    B, T, h = 2, 70, 64
    q, k, v, gam = _inputs(B, T, h, 13)
    out, hr, hi = _run(device, q, k, v, gam)
    o1, r1, i1 = _run(device, q[:, :37], k[:, :37], v[:, :37], gam[:, :37])
    o2, r2, i2 = _run(device, q[:, 37:], k[:, 37:], v[:, 37:], gam[:, 37:], (r1, i1))
    assert _rel(torch.cat([o1, o2], 1), out) <= 1e-5
    assert _rel(r2, hr) <= 1e-5 and _rel(i2, hi) <= 1e-5


def test_cham_raw_state_stays_unitary_over_a_long_sequence(device):
    """The reference's regression test (test_cham.py:139-175): raw state, h = 64, 256
    tokens, H^H H = I to 1e-3 without any retraction."""
    print("[case] cham long unitary", flush=True)
    B, T, h = 2, 256, 64
    q, k, v, gam = _inputs(B, T, h, 17)
    _, hr, hi = _run(device, q, k, v, gam)
    H = (hr + 1j * hi).to(torch.complex128)
    err = (H.conj().transpose(-1, -2) @ H - torch.eye(h, dtype=torch.complex128)).abs().max()
    print(f"[cham long] |H^H H - I| = {float(err):.2e}", flush=True)
    assert float(err) < 1e-3


@pytest.mark.parametrize("B,T,h", [(2, 70, 130), (1, 129, 256), (2, 64, 300), (1, 40, 600),
                                   (1, 20, 1024)])
def test_cham_wide_matches_oracle(device, B, T, h):
    print(f"[case] cham wide B={B} T={T} h={h}", flush=True)
    _check(device, B, T, h, seed=B * 1000 + T + h, label="wide")


@pytest.mark.parametrize("h,unitary", [(160, True), (160, False), (520, True)])
def test_cham_wide_initial_hologram(device, h, unitary):
    """Readout through R_0 = NS_3(H_0) carried beside the raw state."""
    print(f"[case] cham wide H0 h={h} unitary={unitary}", flush=True)
    B, T = 2, 70
    g = torch.Generator().manual_seed(h + unitary)
    Q = torch.linalg.qr(torch.complex(torch.randn(B, h, h, generator=g), torch.randn(B, h, h, generator=g)))[0]
    if not unitary:
        Q = Q * (1.0 + 0.05 * torch.randn(B, h, h, generator=g))
    _check(device, B, T, h, seed=3, h0=(Q.real.contiguous(), Q.imag.contiguous()), label="wide-h0")


def test_cham_wide_bf16_and_halted(device):
    print("[case] cham wide bf16 halted", flush=True)
    B, T, h = 2, 66, 256
    halted = torch.ones(B, T)
    halted[0, 10:30] = 0.0
    halted[1, 60:] = 0.0
    _check(device, B, T, h, seed=21, dtype=torch.bfloat16, halted=halted, label="wide-bf16")


def test_cham_wide_all_halted_keeps_state_exactly(device):
    print("[case] cham wide all halted", flush=True)
    B, T, h = 1, 70, 384
    q, k, v, gam = _inputs(B, T, h, 6, halted=torch.zeros(B, T))
    out, hr, hi = _run(device, q, k, v, gam)
    assert torch.equal(hr, torch.eye(h).expand(B, h, h)) and torch.count_nonzero(hi) == 0
    assert torch.allclose(out, q, atol=1e-6)


def test_cham_wide_chaining(device):
    print("[case] cham wide chaining", flush=True)
    B, T, h = 1, 150, 256
    q, k, v, gam = _inputs(B, T, h, 23)
    out, hr, hi = _run(device, q, k, v, gam)
    o1, r1, i1 = _run(device, q[:, :77], k[:, :77], v[:, :77], gam[:, :77])
    o2, r2, i2 = _run(device, q[:, 77:], k[:, 77:], v[:, 77:], gam[:, 77:], (r1, i1))
    assert _rel(torch.cat([o1, o2], 1), out) <= 1e-5
    assert _rel(r2, hr) <= 1e-5 and _rel(i2, hi) <= 1e-5


@pytest.mark.parametrize("B,T,h", [(2, 1, 256), (1, 16, 300), (3, 5, 1024)])
def test_cham_wide_short_calls_with_initial_hologram(device, B, T, h):
    """T <= 16 with an initial hologram: the readout goes through the matrix-vector chain
    f_3(H_0^H H_0) q instead of NS_3(H_0); non-unitary H_0 included."""
    print(f"[case] cham wide short B={B} T={T} h={h}", flush=True)
    g = torch.Generator().manual_seed(B + T + h)
    Q = torch.linalg.qr(torch.complex(torch.randn(B, h, h, generator=g), torch.randn(B, h, h, generator=g)))[0]
    Q = Q * (1.0 + 0.03 * torch.randn(B, h, h, generator=g))
    _check(device, B, T, h, seed=T + h, h0=(Q.real.contiguous(), Q.imag.contiguous()), label="wide-short")


def test_cham_wide_decode_steps_chain_to_prefill(device):
    """Prefill then single-token calls through the held hologram equal one long call."""
    print("[case] cham wide decode chain", flush=True)
    B, T, h = 2, 68, 512
    q, k, v, gam = _inputs(B, T, h, 31)
    out, hr, hi = _run(device, q, k, v, gam)
    o, r, i = _run(device, q[:, :65], k[:, :65], v[:, :65], gam[:, :65])
    outs = [o]
    for t in range(65, T):
        o, r, i = _run(device, q[:, t:t + 1], k[:, t:t + 1], v[:, t:t + 1], gam[:, t:t + 1], (r, i))
        outs.append(o)
    assert _rel(torch.cat(outs, 1), out) <= 1e-5
    assert _rel(r, hr) <= 1e-5 and _rel(i, hi) <= 1e-5


@pytest.mark.parametrize("B,T,h,unitary", [(2, 100, 64, True), (2, 100, 64, False), (1, 130, 128, True),
                                           (1, 64, 20, False)])
def test_cham_long_calls_with_initial_hologram(device, B, T, h, unitary):
    """h <= 128, T >= 64 with an initial hologram: the readout state R_t = P_t NS_3(H_0) is
    carried beside the raw state."""
    print(f"[case] cham R-route B={B} T={T} h={h} unitary={unitary}", flush=True)
    g = torch.Generator().manual_seed(T + h)
    Q = torch.linalg.qr(torch.complex(torch.randn(B, h, h, generator=g), torch.randn(B, h, h, generator=g)))[0]
    if not unitary:
        Q = Q * (1.0 + 0.05 * torch.randn(B, h, h, generator=g))
    _check(device, B, T, h, seed=T, h0=(Q.real.contiguous(), Q.imag.contiguous()), label="r-route")


@pytest.mark.parametrize("h", [64, 300])
def test_cham_empty_sequence_passes_the_state_through(device, h):
    """T = 0: no output, and the final state is the initial hologram (or the identity)."""
    print(f"[case] cham T=0 h={h}", flush=True)
    B = 2
    q, k, v, gam = _inputs(B, 0, h, 1)
    g = torch.Generator().manual_seed(h)
    H0 = (torch.randn(B, h, h, generator=g), torch.randn(B, h, h, generator=g))
    out, hr, hi = _run(device, q, k, v, gam, H0)
    assert out.shape == (B, 0, h)
    assert torch.equal(hr, H0[0]) and torch.equal(hi, H0[1])
    out, hr, hi = _run(device, q, k, v, gam)
    assert torch.equal(hr, torch.eye(h).expand(B, h, h)) and torch.count_nonzero(hi) == 0


def test_wide_initial_hologram_default_size(device):
    """h = 1024 (the reference's default) from a non-unitary initial hologram with T = 40 >= 17:
    the route that retracts H_0 once (NS_3(H_0) on the fp32 MFMA) and carries R_t beside H_t,
    against the fp64 oracle that retracts every H_t."""
    B, T, h = 1, 40, 1024
    print(f"[case] cham wide h{h} T{T} non-unitary initial hologram", flush=True)
    g = torch.Generator().manual_seed(21)
    a = torch.randn(B, h, h, generator=g, dtype=torch.float64) + 1j * torch.randn(B, h, h, generator=g, dtype=torch.float64)
    u = torch.linalg.qr(a)[0] * (1.0 + 0.05 * torch.rand(B, 1, h, generator=g, dtype=torch.float64))
    h0 = (u.real.float().contiguous(), u.imag.float().contiguous())
    _check(device, B, T, h, 22, h0=h0, label="default h, initial hologram")
