"""GPU parity of the in-place CHAM decode step (vmi_cham_step_inplace / cham_step_) against
the fp64 closed-form CHAM oracle (oracle/cham_scan.py, pinned to the eager restatement of
``cham_memory.py:167-238`` and to linalg.solve in tests/test_cham_oracle.py), which
re-retracts the raw state for every readout as the reference does.

Cases: a unitary state without a carried readout state (the decode after a prefill from the
identity), a non-unitary state with R = NS_3(H) carried beside it, h from 16 to the default
1024 (the 32-column blocks, ragged last block at h = 520), several consecutive steps, halted
(gamma = 0) items left bit-exact.  Bars: fp32 I/O 1e-5 relative Frobenius error per item for
the readout and the state; bf16 2e-2.
"""
import numpy as np
import pytest
import torch

from oracle import cham_ns, cham_scan

pytestmark = pytest.mark.gpu


def _rel(got, ref):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    red = tuple(range(1, got.ndim))
    num = np.sqrt(((got - ref) ** 2).sum(axis=red))
    den = np.sqrt((ref ** 2).sum(axis=red))
    return float((num / np.maximum(den, 1e-30)).max())


def _tokens(B, T, h, g, dtype):
    q = torch.nn.functional.normalize(torch.randn(B, T, h, generator=g), dim=-1)
    k = torch.nn.functional.normalize(torch.randn(B, T, h, generator=g), dim=-1)
    v = torch.nn.functional.normalize(torch.nn.functional.silu(torch.randn(B, T, h, generator=g)), dim=-1)
    gam = 0.1 * torch.sigmoid(torch.randn(B, T, generator=g))
    return q.to(dtype), k.to(dtype), v.to(dtype), gam.to(dtype)


@pytest.mark.parametrize("h", [16, 64, 128, 256, 520, 1024])
@pytest.mark.parametrize("unitary", [True, False])
def test_cham_step_matches_oracle(device, h, unitary):
    from verace_amd import cham_step_
    B, T = 3, 3
    print(f"[case] cham step h{h} unitary={unitary}", flush=True)
    g = torch.Generator().manual_seed(h + unitary)
    q, k, v, gam = _tokens(B, T, h, g, torch.float32)
    a = torch.randn(B, h, h, generator=g, dtype=torch.float64) + 1j * torch.randn(B, h, h, generator=g, dtype=torch.float64)
    if unitary:
        u = torch.linalg.qr(a)[0]
    else:
        u = torch.linalg.qr(a)[0] * (1.0 + 0.05 * torch.rand(B, 1, h, generator=g, dtype=torch.float64))
    h0r, h0i = u.real.float().contiguous(), u.imag.float().contiguous()
    hr, hi = h0r.to(device), h0i.to(device)
    readout = None
    if not unitary:
        rr, ri = cham_ns.newton_schulz_retraction(h0r.double(), h0i.double(), 3)
        readout = (rr.float().contiguous().to(device), ri.float().contiguous().to(device))
    outs = []
    for t in range(T):
        o = cham_step_(q[:, t:t + 1].to(device), k[:, t:t + 1].to(device), v[:, t:t + 1].to(device),
                       gam[:, t:t + 1].to(device), (hr, hi), readout)
        outs.append(o.float().cpu())
    torch.cuda.synchronize()
    out = torch.cat(outs, 1)
    ref, (sr, si) = cham_scan.cham_scan_closed(q.double().numpy(), k.double().numpy(), v.double().numpy(),
                                              gam.double().numpy(), h0r.double().numpy(), h0i.double().numpy())
    eo = _rel(out, ref)
    es = max(_rel(hr.cpu(), sr), _rel(hi.cpu(), si))
    print(f"  rel out={eo:.2e} state={es:.2e}", flush=True)
    assert eo <= 1e-5 and es <= 1e-5
    if readout is not None:  # the carried readout state is still NS_3 of the raw state
        nr, ni = cham_ns.newton_schulz_retraction(torch.from_numpy(sr), torch.from_numpy(si), 3)
        er = max(_rel(readout[0].cpu(), nr.numpy()), _rel(readout[1].cpu(), ni.numpy()))
        print(f"  readout state rel={er:.2e}", flush=True)
        assert er <= 1e-5


def test_cham_step_bf16_and_halted(device):
    """bf16 token inputs (2e-2), and an item with gamma = 0 whose state stays bit-exact."""
    from verace_amd import cham_step_
    B, h = 4, 1024
    print("[case] cham step bf16 + halted", flush=True)
    g = torch.Generator().manual_seed(9)
    q, k, v, gam = _tokens(B, 1, h, g, torch.bfloat16)
    gam[2] = 0.0
    a = torch.randn(B, h, h, generator=g, dtype=torch.float64) + 1j * torch.randn(B, h, h, generator=g, dtype=torch.float64)
    u = torch.linalg.qr(a)[0]
    h0r, h0i = u.real.float().contiguous(), u.imag.float().contiguous()
    hr, hi = h0r.to(device), h0i.to(device)
    o = cham_step_(q.to(device), k.to(device), v.to(device), gam.to(device), (hr, hi))
    torch.cuda.synchronize()
    assert o.dtype == torch.bfloat16 and o.shape == (B, 1, h)
    assert torch.equal(hr[2].cpu(), h0r[2]) and torch.equal(hi[2].cpu(), h0i[2])
    ref, (sr, si) = cham_scan.cham_scan_closed(q.double().numpy(), k.double().numpy(), v.double().numpy(),
                                              gam.double().numpy(), h0r.double().numpy(), h0i.double().numpy())
    eo = _rel(o.float().cpu(), ref)
    es = max(_rel(hr.cpu(), sr), _rel(hi.cpu(), si))
    print(f"  rel out={eo:.2e} state={es:.2e}", flush=True)
    assert eo <= 2e-2 and es <= 2e-2


def test_cham_step_rejects_bad_arguments(device):
    from verace_amd import cham_step_
    h = 64
    q = torch.randn(2, 1, h, device=device)
    g = torch.rand(2, device=device)
    hr = torch.eye(h, device=device).expand(2, -1, -1).contiguous()
    hi = torch.zeros_like(hr)
    with pytest.raises(RuntimeError):
        cham_step_(q, q, q, g, (hr.double(), hi))                # dtype
    with pytest.raises(RuntimeError):
        cham_step_(q, q, q, g, (hr, hi), (hr[:1].contiguous(), hi[:1].contiguous()))  # readout shape
    with pytest.raises(RuntimeError):
        cham_step_(q.cpu(), q, q, g, (hr, hi))                   # device


@pytest.mark.parametrize("h", [64, 1024])
def test_cham_step_nonfinite_token_is_identity(device, h):
    """A NaN or Inf in an item's k or v, or a NaN gamma, makes its token U = I (the reference's
    guard, cham_memory.py:68-95): that item's state is unchanged bit for bit although the column
    sums were formed with the non-finite row; the other items follow the oracle."""
    from verace_amd import cham_step_
    print(f"[case] cham step non-finite h{h}", flush=True)
    B = 4
    g = torch.Generator().manual_seed(70 + h)
    q, k, v, gam = _tokens(B, 1, h, g, torch.float32)
    k[0, 0, 5] = float("nan")
    v[1, 0, h - 1] = float("inf")
    gam[2, 0] = float("nan")
    a = torch.randn(B, h, h, generator=g, dtype=torch.float64) + 1j * torch.randn(B, h, h, generator=g, dtype=torch.float64)
    u = torch.linalg.qr(a)[0]
    h0r, h0i = u.real.float().contiguous(), u.imag.float().contiguous()
    hr, hi = h0r.to(device), h0i.to(device)
    o = cham_step_(q.to(device), k.to(device), v.to(device), gam.to(device), (hr, hi))
    torch.cuda.synchronize()
    for b in (0, 1, 2):
        assert torch.equal(hr[b].cpu(), h0r[b]) and torch.equal(hi[b].cpu(), h0i[b])
    assert torch.isfinite(o).all()
    ref, (sr, si) = cham_scan.cham_scan_closed(q[3:].double().numpy(), k[3:].double().numpy(),
                                              v[3:].double().numpy(), gam[3:].double().numpy(),
                                              h0r[3:].double().numpy(), h0i[3:].double().numpy())
    assert max(_rel(hr[3:].cpu(), sr), _rel(hi[3:].cpu(), si)) <= 1e-5
    assert _rel(o[3:].float().cpu(), ref) <= 1e-5
