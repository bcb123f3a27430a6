"""GPU parity of the fused projection path: the raw projections go into the scan, which
normalises q, k, v, forms delta = 0.1 sigmoid(.) * mask and applies head_rmsnorm itself
(``sssd_attention.py:114-126`` and ``:177`` around the scan).

Oracle: the same steps in float64 on the host (F.normalize, sigmoid, mask, the fp64 closed-
form scan of oracle/sssd_closed.py, nn.RMSNorm's formula with torch's default eps), fed
the kernel's own bf16/fp16 projections (eps: what torch's nn.RMSNorm adds by default, pinned
on the host by tests/test_oracle_pins.py).  Bars: out and final state <= 2e-2 relative
Frobenius error per (b, h) slice (the kernel rounds the normalised inputs once to f16 and
the output once to bf16, where the reference rounds to bf16 twice), state norm drift
<= 1e-4 for orthogonal starts.
"""
import math

import numpy as np
import pytest
import torch

from oracle import sssd_closed

pytestmark = pytest.mark.gpu


def _rel(got, ref, slice_dims):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    red = tuple(i for i in range(got.ndim) if i not in slice_dims)
    num = np.sqrt(((got - ref) ** 2).sum(axis=red))
    den = np.sqrt((ref ** 2).sum(axis=red))
    return float((num / np.maximum(den, 1e-30)).max())


def _oracle(proj, H, D, mask, rms_w, eps, psi0):
    """float64 restatement of sssd_attention.py:114-126, the scan, and :177."""
    p = proj.double().cpu().numpy()
    B, T, _ = p.shape
    HD = H * D

    def unit(x):
        x = x.reshape(B, T, H, D)
        n = np.sqrt((x ** 2).sum(-1, keepdims=True))
        return x / np.maximum(n, 1e-12)

    q, k, v = unit(p[..., :HD]), unit(p[..., HD:2 * HD]), unit(p[..., 2 * HD:3 * HD])
    d = 0.1 / (1.0 + np.exp(-p[..., 3 * HD:3 * HD + H]))
    if mask is not None:
        d = d * mask.cpu().numpy().astype(np.float64)[..., None]
    o, psi = sssd_closed.sssd_scan_closed_c(q, k, v, d, None if psi0 is None else psi0.double().numpy())
    if rms_w is not None:
        ms = (o ** 2).mean(-1, keepdims=True)
        o = o / np.sqrt(ms + eps) * rms_w.double().cpu().numpy()
    return o, psi


def _case(device, B, T, H, dtype, seed, with_mask, with_state, with_rms=True, scale=1.0):
    from verace_amd.hip_kernels import launch_sssd_hip_scan_fused
    D = 128
    g = torch.Generator().manual_seed(seed)
    n = 3 * H * D + H
    proj = (scale * torch.randn(B, T, n, generator=g)).to(dtype)
    mask = None
    if with_mask:
        mask = torch.rand(B, T, generator=g) > 0.2
    psi0 = torch.linalg.qr(torch.randn(B, H, D, D, generator=g))[0].contiguous() if with_state else None
    w = (1.0 + 0.1 * torch.randn(D, generator=g)) if with_rms else None
    from verace_amd.hip_kernels import rms_default_eps
    eps = rms_default_eps(dtype)
    o, psi = launch_sssd_hip_scan_fused(proj.to(device), H, D, None if mask is None else mask.to(device),
                                        None if w is None else w.to(device), None,
                                        None if psi0 is None else psi0.to(device))
    torch.cuda.synchronize()
    o_ref, psi_ref = _oracle(proj, H, D, mask, w, eps, psi0)
    eo = _rel(o.float().cpu(), o_ref, (0, 2))
    ep = _rel(psi.cpu(), psi_ref, (0, 1))
    n0 = math.sqrt(D) if psi0 is None else np.linalg.norm(psi0.double().numpy().reshape(B, H, -1), axis=-1)
    nrm = np.linalg.norm(psi.cpu().double().numpy().reshape(B, H, -1), axis=-1)
    drift = float(np.abs(nrm / n0 - 1).max())
    print(f"[fused {dtype} B{B} T{T} H{H}] rel o={eo:.2e} psi={ep:.2e} drift={drift:.2e}", flush=True)
    assert eo <= 2e-2 and ep <= 2e-2 and drift <= 1e-4
    return o, psi


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("B,T,H,mask,state", [(1, 32, 1, False, False), (2, 100, 3, True, False),
                                              (1, 1000, 2, True, True), (2, 2048, 4, False, True)])
def test_fused_scan_matches_oracle(device, dtype, B, T, H, mask, state):
    print(f"[case] fused {dtype} B={B} T={T} H={H} mask={mask} state={state}", flush=True)
    _case(device, B, T, H, dtype, seed=T + H, with_mask=mask, with_state=state)


def test_fused_scan_without_rmsnorm_and_large_projections(device):
    """No rms weight: the output is o itself; raw projections of magnitude ~300 (the
    normalisation happens in fp32 before any f16 rounding)."""
    print("[case] fused no-rms scale 300", flush=True)
    _case(device, 2, 300, 2, torch.bfloat16, seed=7, with_mask=True, with_state=False,
          with_rms=False, scale=300.0)


def test_fused_scan_all_halted_keeps_state(device):
    from verace_amd.hip_kernels import launch_sssd_hip_scan_fused
    print("[case] fused all halted", flush=True)
    B, T, H, D = 1, 64, 2, 128
    g = torch.Generator().manual_seed(3)
    proj = torch.randn(B, T, 3 * H * D + H, generator=g).bfloat16().to(device)
    psi0 = torch.randn(B, H, D, D, generator=g).to(device)
    _, psi = launch_sssd_hip_scan_fused(proj, H, D, torch.zeros(B, T, dtype=torch.bool, device=device),
                                        None, None, psi0)
    torch.cuda.synchronize()
    assert torch.equal(psi, psi0)   # delta = 0 => every R_t = I exactly


def test_module_fused_matches_unfused(device):
    """SSSDAttention with the fused path against the same module on the unfused torch ops
    (the reference's op sequence) for prefill with a mask and an initial state."""
    from verace_amd import SSSDAttention
    print("[case] module fused vs unfused", flush=True)
    torch.manual_seed(0)
    m = SSSDAttention(512, 4, 128).to(device).to(torch.bfloat16)
    g = torch.Generator().manual_seed(1)
    B, T = 2, 300
    x = torch.randn(B, T, 512, generator=g).bfloat16().to(device)
    mask = (torch.rand(B, T, generator=g) > 0.1).to(device)
    st0 = torch.linalg.qr(torch.randn(B, 4, 128, 128, generator=g))[0].to(device)
    with torch.no_grad():
        m.fuse_projections = True
        y_f, s_f = m(x, initial_state=st0, return_state=True, active_mask=mask)
        m.fuse_projections = False
        y_u, s_u = m(x, initial_state=st0, return_state=True, active_mask=mask)
    torch.cuda.synchronize()
    ey = _rel(y_f.float().cpu(), y_u.float().cpu(), (0, 1))
    es = _rel(s_f.cpu(), s_u.cpu(), (0, 1))
    print(f"[module fused vs unfused] y {ey:.2e} state {es:.2e}", flush=True)
    assert ey <= 2e-2 and es <= 2e-2
