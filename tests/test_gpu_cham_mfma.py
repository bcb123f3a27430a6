"""GPU parity of the wide CHAM route's matrix-core state carry (csrc/cham_mfma.hip: the chunked
form U_16 ... U_1 = I + Y T Y^T on the MFMA, taken for bf16 / f16 k, v with 128 < h <= 1024,
h % 8 == 0) against the fp64 oracle oracle/cham_scan.py (the per-token closed-form scan; the
reference's algorithm, cham_memory.py:167-238).

The oracle is fed the same 16-bit values (q.double() of the bf16 / f16 tensors), so the fp32
state is held to the fp32 bar (1e-5 relative Frobenius error per batch item, as the fp32
route); the output is rounded to the input dtype, so it is held to 1e-2.  The matrix-core
route is also compared with the token-sequential fp32 route fed the identical values (fp32
tensors holding the 16-bit values): both compute in fp32, so their states agree to 1e-5.
Shapes cross the 16-token chunks and the 64-token readout snapshots at ragged T, with halted
tokens, unitary and non-unitary initial holograms, and non-finite tokens (the reference's guard,
cham_memory.py:68-95: such a token is U = I).
"""
import numpy as np
import pytest
import torch

from oracle import cham_scan

pytestmark = pytest.mark.gpu


def _inputs(B, T, h, seed, dtype, halted=None):
    g = torch.Generator().manual_seed(seed)
    nrm = torch.nn.functional.normalize
    q = nrm(torch.randn(B, T, h, generator=g), dim=-1).to(dtype)
    k = nrm(torch.randn(B, T, h, generator=g), dim=-1).to(dtype)
    v = nrm(torch.nn.functional.silu(torch.randn(B, T, h, generator=g)), dim=-1).to(dtype)
    gam = 0.1 * torch.sigmoid(torch.randn(B, T, generator=g))
    if halted is not None:
        gam = gam * halted
    return q, k, v, gam.to(dtype)


def _hologram(B, h, seed, unitary):
    g = torch.Generator().manual_seed(seed)
    a = torch.randn(B, h, h, generator=g, dtype=torch.float64) + 1j * torch.randn(B, h, h, generator=g, dtype=torch.float64)
    u = torch.linalg.qr(a)[0]
    if not unitary:
        u = u * (1.0 + 0.05 * torch.rand(B, 1, h, generator=g, dtype=torch.float64))
    return u.real.float().contiguous(), u.imag.float().contiguous()


def _rel(got, ref):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    red = tuple(range(1, got.ndim))
    num = np.sqrt(((got - ref) ** 2).sum(axis=red))
    den = np.sqrt((ref ** 2).sum(axis=red))
    return float((num / np.maximum(den, 1e-30)).max())


def _run(device, q, k, v, gam, h0):
    from verace_amd import launch_cham_hip_update
    init = None if h0 is None else (h0[0].to(device), h0[1].to(device))
    out, (hr, hi) = launch_cham_hip_update(q.to(device), k.to(device), v.to(device), gam.to(device), init)
    torch.cuda.synchronize()
    return out.float().cpu(), hr.cpu(), hi.cpu()


@pytest.mark.parametrize("B,T,h,dtype,init", [
    (2, 70, 256, torch.bfloat16, None),
    (1, 129, 512, torch.float16, None),
    (2, 64, 600, torch.bfloat16, "unitary"),
    (1, 100, 1024, torch.bfloat16, None),
    (1, 40, 1024, torch.float16, "nonunitary"),
    (2, 17, 1024, torch.bfloat16, "unitary"),
])
def test_cham_mfma_route_matches_oracle(device, B, T, h, dtype, init):
    print(f"[case] cham mfma B{B} T{T} h{h} {dtype} init={init}", flush=True)
    q, k, v, gam = _inputs(B, T, h, seed=T + h, dtype=dtype)
    h0 = None if init is None else _hologram(B, h, seed=h, unitary=init == "unitary")
    out, hr, hi = _run(device, q, k, v, gam, h0)
    ref, (rr, ri) = cham_scan.cham_scan_closed(
        q.double().numpy(), k.double().numpy(), v.double().numpy(), gam.double().numpy(),
        None if h0 is None else h0[0].double().numpy(), None if h0 is None else h0[1].double().numpy())
    eo = _rel(out, ref)
    es = max(_rel(hr, rr), _rel(hi, ri) if np.abs(ri).max() > 0 else 0.0)
    # the fp32 token-sequential route on the same values
    o32, r32, i32 = _run(device, q.float(), k.float(), v.float(), gam.float(), h0)
    ex = max(_rel(hr, r32), _rel(hi, i32) if np.abs(i32.numpy()).max() > 0 else 0.0)
    print(f"  rel out={eo:.2e} state={es:.2e} state vs fp32 route={ex:.2e}", flush=True)
    assert np.isfinite(out.numpy()).all()
    assert eo <= 1e-2 and es <= 1e-5 and ex <= 1e-5


def test_cham_mfma_route_halted_tokens(device):
    """Halted tokens (gamma = 0) are exact identities; a fully halted item keeps its state."""
    B, T, h = 3, 90, 512
    print(f"[case] cham mfma halted B{B} T{T} h{h}", flush=True)
    halted = torch.ones(B, T)
    halted[0, 10:40] = 0.0
    halted[1, 64:] = 0.0
    halted[2, :] = 0.0
    q, k, v, gam = _inputs(B, T, h, seed=5, dtype=torch.bfloat16, halted=halted)
    out, hr, hi = _run(device, q, k, v, gam, None)
    ref, (rr, ri) = cham_scan.cham_scan_closed(q.double().numpy(), k.double().numpy(),
                                               v.double().numpy(), gam.double().numpy(), None, None)
    eo, es = _rel(out[:2], ref[:2]), max(_rel(hr[:2], rr[:2]), _rel(hi[:2], ri[:2]))
    print(f"  rel out={eo:.2e} state={es:.2e}", flush=True)
    assert eo <= 1e-2 and es <= 1e-5
    assert torch.equal(hr[2], torch.eye(h)) and torch.count_nonzero(hi[2]) == 0


def test_cham_mfma_route_nonfinite_tokens(device):
    """A NaN / Inf in k, v or gamma makes its token U = I; the chunk holding it takes the
    guarded conversion, the others are unaffected."""
    B, T, h = 2, 80, 256
    print(f"[case] cham mfma nonfinite B{B} T{T} h{h}", flush=True)
    q, k, v, gam = _inputs(B, T, h, seed=11, dtype=torch.bfloat16)
    k, v, gam = k.clone(), v.clone(), gam.clone()
    k[0, 3, 7] = float("nan")
    v[1, 15, 0] = float("inf")
    gam[0, 16] = float("nan")
    k[1, 0, h - 1] = float("-inf")
    v[0, 63, 100] = float("nan")
    out, hr, hi = _run(device, q, k, v, gam, None)
    assert torch.isfinite(out).all() and torch.isfinite(hr).all() and torch.isfinite(hi).all()
    kc, vc, gc = k.double().numpy().copy(), v.double().numpy().copy(), gam.double().numpy().copy()
    for b, t in [(0, 3), (1, 15), (0, 16), (1, 0), (0, 63)]:
        kc[b, t] = 0.0
        vc[b, t] = 0.0
        gc[b, t] = 0.0
    ref, (rr, ri) = cham_scan.cham_scan_closed(q.double().numpy(), kc, vc, gc, None, None)
    eo, es = _rel(out, ref), max(_rel(hr, rr), _rel(hi, ri))
    print(f"  rel out={eo:.2e} state={es:.2e}", flush=True)
    assert eo <= 1e-2 and es <= 1e-5


def test_cham_mfma_elements_beyond_f16_are_identity_tokens(device):
    """The 16-bit route's documented precondition (every k, v element below 65504, the f16
    range): a token with a finite bf16 element above it is taken as the identity, exactly as
    the same token with gamma = 0, and the fp32 route takes the same values as they are
    (against the fp64 oracle)."""
    B, T, h = 1, 40, 256
    print(f"[case] cham mfma element beyond f16 range B{B} T{T} h{h}", flush=True)
    q, k, v, gam = _inputs(B, T, h, seed=77, dtype=torch.bfloat16)
    big = k.clone()
    big[0, 17, 5] = 1.0e5          # finite in bf16 (99840), above f16's 65504
    gz = gam.clone()
    gz[0, 17] = 0.0
    ob, hrb, hib = _run(device, q, big, v, gam, None)
    oz, hrz, hiz = _run(device, q, k, v, gz, None)
    assert torch.isfinite(hrb).all() and torch.isfinite(ob).all()
    assert torch.equal(hrb, hrz) and torch.equal(hib, hiz) and torch.equal(ob, oz)
    # the fp32 route on the same values: the large element counts
    of, hrf, hif = _run(device, q.float(), big.float(), v.float(), gam.float(), None)
    rec, (sr, si) = cham_scan.cham_scan_closed(q.double().numpy(), big.double().numpy(),
                                               v.double().numpy(), gam.double().numpy())
    assert _rel(np.concatenate([hrf.numpy(), hif.numpy()], 1), np.concatenate([sr, si], 1)) <= 1e-5
