"""GPU parity of the fused CHAM decode step (vmi_cham_step_fused / cham_step_fused_): one row
of the stacked projection per item goes into the h = 1024 step kernel, which forms silu(v),
L2-normalises q, k, v and forms gamma = 0.1 sigmoid(.) * mask (``cham_memory.py:128-155`` at
seq_len 1) before the in-place update and the readout Re(NS_3(H') q).

Oracle: the same steps in float64 on the host (silu, F.normalize, sigmoid, mask) fed the
kernel's own projections, then the fp64 closed-form CHAM oracle (oracle/cham_scan.py, pinned in
tests/test_cham_oracle.py) over the steps taken, which re-retracts the raw state for every
readout.  The kernel computes in fp32 from the 16-bit projections (no rounding of the
normalised vectors), so the bars are 1e-5 relative Frobenius error per item for the state and
the readout of fp32 I/O, 1e-2 for the bf16 readout (one rounding of the output), 1e-5 for the
state in every case.
"""
import numpy as np
import pytest
import torch

from oracle import cham_ns, cham_scan

pytestmark = pytest.mark.gpu

H = 1024


def _rel(got, ref):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    red = tuple(range(1, got.ndim))
    num = np.sqrt(((got - ref) ** 2).sum(axis=red))
    den = np.sqrt((ref ** 2).sum(axis=red))
    return float((num / np.maximum(den, 1e-30)).max())


def _host_tokens(proj, mask):
    """float64 restatement of cham_memory.py:128-155 on the raw projections proj [B, T, n]."""
    p = proj.double()

    def unit(x):
        return x / x.norm(dim=-1, keepdim=True).clamp_min(1e-12)

    q = unit(p[..., :H])
    k = unit(p[..., H:2 * H])
    v = unit(torch.nn.functional.silu(p[..., 2 * H:3 * H]))
    gam = 0.1 * torch.sigmoid(p[..., 3 * H])
    if mask is not None:
        gam = gam * mask.double()
    return q.numpy(), k.numpy(), v.numpy(), gam.numpy()


def _start(B, g, unitary):
    a = torch.randn(B, H, H, generator=g, dtype=torch.float64) + 1j * torch.randn(B, H, H, generator=g, dtype=torch.float64)
    u = torch.linalg.qr(a)[0]
    if not unitary:
        u = u * (1.0 + 0.05 * torch.rand(B, 1, H, generator=g, dtype=torch.float64))
    return u.real.float().contiguous(), u.imag.float().contiguous()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("unitary,with_mask", [(True, False), (False, True)])
def test_cham_step_fused_matches_oracle(device, dtype, unitary, with_mask):
    from verace_amd import cham_step_fused_
    B, T = 3, 3
    print(f"[case] cham fused step {dtype} unitary={unitary} mask={with_mask}", flush=True)
    g = torch.Generator().manual_seed(31 + unitary + 2 * with_mask)
    n = 3 * H + 1 + 7  # a row stride past the last used column
    proj = (torch.randn(B, T, n, generator=g) * 0.5).to(dtype)
    mask = (torch.rand(B, T, generator=g) > 0.3) if with_mask else None
    h0r, h0i = _start(B, g, unitary)
    hr, hi = h0r.to(device), h0i.to(device)
    readout = None
    if not unitary:
        rr, ri = cham_ns.newton_schulz_retraction(h0r.double(), h0i.double(), 3)
        readout = (rr.float().contiguous().to(device), ri.float().contiguous().to(device))
    outs = []
    for t in range(T):
        m = None if mask is None else mask[:, t].to(device)
        o = cham_step_fused_(proj[:, t:t + 1].to(device), H, (hr, hi), readout, m)
        outs.append(o.float().cpu())
    torch.cuda.synchronize()
    out = torch.cat(outs, 1)
    q, k, v, gam = _host_tokens(proj, mask)
    ref, (sr, si) = cham_scan.cham_scan_closed(q, k, v, gam, h0r.double().numpy(), h0i.double().numpy())
    eo = _rel(out, ref)
    es = max(_rel(hr.cpu(), sr), _rel(hi.cpu(), si))
    print(f"  rel out={eo:.2e} state={es:.2e}", flush=True)
    assert es <= 1e-5 and eo <= (1e-5 if dtype == torch.float32 else 1e-2)
    if readout is not None:
        nr, ni = cham_ns.newton_schulz_retraction(torch.from_numpy(sr), torch.from_numpy(si), 3)
        er = max(_rel(readout[0].cpu(), nr.numpy()), _rel(readout[1].cpu(), ni.numpy()))
        print(f"  readout state rel={er:.2e}", flush=True)
        assert er <= 1e-5


def test_cham_step_fused_halted_and_nonfinite(device):
    """A halted item (mask 0) and items with a NaN in k, an Inf in v or a NaN gamma logit keep
    their state bit for bit (the reference's non-finite guard, cham_memory.py:68-95); the other
    items follow the oracle."""
    from verace_amd import cham_step_fused_
    print("[case] cham fused step halted / non-finite", flush=True)
    B = 5
    g = torch.Generator().manual_seed(41)
    proj = torch.randn(B, 1, 3 * H + 1, generator=g)
    proj[1, 0, H + 17] = float("nan")
    proj[2, 0, 2 * H + 3] = float("inf")
    proj[3, 0, 3 * H] = float("nan")
    proj = proj.to(torch.bfloat16)
    mask = torch.tensor([True, True, True, True, False])
    h0r, h0i = _start(B, g, True)
    hr, hi = h0r.to(device), h0i.to(device)
    o = cham_step_fused_(proj.to(device), H, (hr, hi), None, mask.to(device))
    torch.cuda.synchronize()
    for b in (1, 2, 3, 4):
        assert torch.equal(hr[b].cpu(), h0r[b]) and torch.equal(hi[b].cpu(), h0i[b])
    assert torch.isfinite(o).all()
    q, k, v, gam = _host_tokens(proj[:1], mask[:1].view(1, 1))
    ref, (sr, si) = cham_scan.cham_scan_closed(q, k, v, gam, h0r[:1].double().numpy(), h0i[:1].double().numpy())
    assert max(_rel(hr[:1].cpu(), sr), _rel(hi[:1].cpu(), si)) <= 1e-5
    assert _rel(o[:1].float().cpu(), ref) <= 1e-2


def test_module_cham_step_fused_matches_unfused(device):
    """ContinuousHolographicMemory.step_ through the fused kernel against the reference's op
    sequence (projections, F.normalize, silu, sigmoid, mask, the unfused step, w_out, norm) from
    the same state: the unfused path rounds the normalised q, k, v and gamma to bf16, so the two
    agree to bf16 accuracy."""
    from verace_amd import ContinuousHolographicMemory
    print("[case] module cham step fused vs unfused", flush=True)
    torch.manual_seed(3)
    hidden = 256
    m = ContinuousHolographicMemory(hidden_dim=hidden, holographic_dim=H).to(device, torch.bfloat16)
    B = 4
    x = torch.randn(B, 1, hidden, device=device).to(torch.bfloat16)
    mask = torch.tensor([True, False, True, True], device=device).view(B, 1)
    g = torch.Generator().manual_seed(4)
    h0r, h0i = _start(B, g, True)
    with torch.no_grad():
        a = (h0r.to(device), h0i.to(device))
        b = (h0r.to(device), h0i.to(device))
        y_f = m.step_(x, a, None, mask)
        m.fuse_projections = False
        y_u = m.step_(x, b, None, mask)
    torch.cuda.synchronize()
    assert _rel(y_f.float().cpu(), y_u.float().cpu()) <= 2e-2
    assert max(_rel(a[0].cpu(), b[0].cpu()), _rel(a[1].cpu(), b[1].cpu())) <= 1e-2
    assert torch.equal(a[0][1].cpu(), h0r[1]) and torch.equal(a[1][1].cpu(), h0i[1])


def test_cham_step_fused_rejects_other_sizes(device):
    from verace_amd import _lib
    from verace_amd.hip_kernels import cham_step_fused_
    print("[case] cham fused step h 512 rejected", flush=True)
    h = 512
    proj = torch.zeros(2, 1, 3 * h + 1, device=device, dtype=torch.bfloat16)
    hr = torch.zeros(2, h, h, device=device)
    hi = torch.zeros(2, h, h, device=device)
    with pytest.raises(RuntimeError):
        cham_step_fused_(proj, h, (hr, hi))
    lib = _lib.load()
    st = lib.vmi_cham_step_fused(proj.data_ptr(), proj.shape[-1], 1, None, hr.data_ptr(), hi.data_ptr(),
                                 None, None, None, 2, h, None, 0, None)
    assert st == 2  # VMI_ERR_UNSUPPORTED
