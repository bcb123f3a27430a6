"""GPU parity of the fused CHAM prefill (vmi_cham_scan_fused / launch_cham_hip_update_fused):
the scan from the identity reads the stacked projection x [W_q; W_k; W_v; W_gamma]^T and forms
silu(v), the L2 normalisations and gamma = 0.1 sigmoid(.) * mask in its kernels
(``cham_memory.py:128-155`` before the scan, ``:167-238`` the scan).

The matrix-core carry multiplies f16 operands, so the kernels round the normalised k, v to f16
once (the Cayley coefficients are formed from the same rounded vectors, so every factor stays
unitary).  Oracles: (1) the fp64 closed form (oracle/cham_scan.py) fed the normalised k, v
rounded to f16 the same way (norm and product in fp32, then f16): final state <= 3e-5 (the
kernels' fp32 norms are summed in another order, so an element at an f16 rounding boundary can
round the other way: measured 1.6e-7 to 1.7e-5), output <= 1e-2 (q rounded once to f16 and the
output once to 16 bits); (2) the fp64 chain without that rounding: state and output <= 2e-2 (the
reference itself rounds the normalised vectors to bf16).
"""
import numpy as np
import pytest
import torch

from oracle import cham_scan

pytestmark = pytest.mark.gpu


def _rel(got, ref):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    red = tuple(range(1, got.ndim))
    num = np.sqrt(((got - ref) ** 2).sum(axis=red))
    den = np.sqrt((ref ** 2).sum(axis=red))
    return float((num / np.maximum(den, 1e-30)).max())


def _host(proj, h, mask, round_kv):
    """cham_memory.py:128-155 in float64 on the raw projections [B, T, n]; with round_kv the
    normalised k, v rounded to f16 as the kernels hold them."""
    p = proj.double()

    def unit(x):
        return x / x.norm(dim=-1, keepdim=True).clamp_min(1e-12)

    q = unit(p[..., :h])
    if round_kv:  # as the kernels: the norm and the product in fp32, then one f16 rounding
        def unit16(x):
            x = x.float()
            nrm = (1.0 / x.pow(2).sum(-1, keepdim=True).sqrt().clamp_min(1e-12)).float()
            return (x * nrm).to(torch.float16).double()

        k = unit16(p[..., h:2 * h])
        v = unit16(torch.nn.functional.silu(p[..., 2 * h:3 * h].float()))
    else:
        k = unit(p[..., h:2 * h])
        v = unit(torch.nn.functional.silu(p[..., 2 * h:3 * h]))
    gam = 0.1 * torch.sigmoid(p[..., 3 * h])
    if mask is not None:
        gam = gam * mask.double()
    return q.numpy(), k.numpy(), v.numpy(), gam.numpy()


def _run(device, proj, h, mask):
    from verace_amd import launch_cham_hip_update_fused
    out, (hr, hi) = launch_cham_hip_update_fused(proj.to(device), h,
                                                  None if mask is None else mask.to(device))
    torch.cuda.synchronize()
    return out.float().cpu(), hr.cpu(), hi.cpu()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("B,T,h,with_mask", [(2, 17, 256, False), (1, 130, 1024, True),
                                             (2, 300, 520, True), (1, 1, 1024, False)])
def test_cham_fused_scan_matches_oracle(device, dtype, B, T, h, with_mask):
    print(f"[case] cham fused scan {dtype} B={B} T={T} h={h} mask={with_mask}", flush=True)
    g = torch.Generator().manual_seed(T + h)
    n = 3 * h + 1 + 15  # padded row stride
    proj = (0.7 * torch.randn(B, T, n, generator=g)).to(dtype)
    mask = (torch.rand(B, T, generator=g) > 0.2) if with_mask else None
    out, hr, hi = _run(device, proj, h, mask)
    ref, (sr, si) = cham_scan.cham_scan_closed(*_host(proj, h, mask, True))
    eo, es = _rel(out, ref), max(_rel(hr, sr), _rel(hi, si))
    ref2, (sr2, si2) = cham_scan.cham_scan_closed(*_host(proj, h, mask, False))
    eo2, es2 = _rel(out, ref2), max(_rel(hr, sr2), _rel(hi, si2))
    print(f"  rounded oracle: out={eo:.2e} state={es:.2e}; unrounded: out={eo2:.2e} state={es2:.2e}",
          flush=True)
    assert es <= 3e-5 and eo <= 1e-2
    assert es2 <= 2e-2 and eo2 <= 2e-2


def test_cham_fused_scan_nonfinite_and_halted(device):
    """A NaN in k, an Inf in v or a NaN gamma logit makes the token U = I (the reference's guard,
    cham_memory.py:68-95), at chunk-boundary tokens; a fully halted item keeps the identity."""
    print("[case] cham fused scan non-finite / halted", flush=True)
    B, T, h = 3, 40, 1024
    g = torch.Generator().manual_seed(9)
    proj = 0.7 * torch.randn(B, T, 3 * h + 1, generator=g)
    proj[0, 15, h + 3] = float("nan")
    proj[0, 16, 2 * h + 9] = float("inf")
    proj[1, 31, 3 * h] = float("nan")
    proj = proj.to(torch.bfloat16)
    mask = torch.ones(B, T, dtype=torch.bool)
    mask[2] = False
    out, hr, hi = _run(device, proj, h, mask)
    assert torch.isfinite(out).all() and torch.isfinite(hr).all() and torch.isfinite(hi).all()
    assert torch.equal(hr[2], torch.eye(h)) and torch.count_nonzero(hi[2]) == 0
    q, k, v, gam = _host(proj, h, mask, True)
    for b, t in [(0, 15), (0, 16), (1, 31)]:
        k[b, t] = 0.0
        v[b, t] = 0.0
        gam[b, t] = 0.0
    ref, (sr, si) = cham_scan.cham_scan_closed(q, k, v, gam)
    assert max(_rel(hr[:2], sr[:2]), _rel(hi[:2], si[:2])) <= 3e-5
    assert _rel(out[:2], ref[:2]) <= 1e-2


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_cham_empty_sequence_16bit(device, dtype):
    """T = 0 with 16-bit inputs above h = 128 (the matrix-core route's shapes): the fused and the
    unfused scan pass the identity (or the initial hologram) through without reading a token."""
    from verace_amd import launch_cham_hip_update
    print(f"[case] cham T=0 {dtype}", flush=True)
    B, h = 2, 1024
    out, hr, hi = _run(device, torch.zeros(B, 0, 3 * h + 1, dtype=dtype), h, None)
    assert out.shape == (B, 0, h)
    assert torch.equal(hr, torch.eye(h).expand(B, h, h)) and torch.count_nonzero(hi) == 0
    e = torch.zeros(B, 0, h, dtype=dtype, device=device)
    g = torch.Generator().manual_seed(2)
    H0 = (torch.randn(B, h, h, generator=g).to(device), torch.randn(B, h, h, generator=g).to(device))
    for init in (None, H0):
        out, (r, i) = launch_cham_hip_update(e, e, e, torch.zeros(B, 0, dtype=dtype, device=device), init)
        torch.cuda.synchronize()
        if init is None:
            assert torch.equal(r.cpu(), torch.eye(h).expand(B, h, h)) and torch.count_nonzero(i) == 0
        else:
            assert torch.equal(r, H0[0]) and torch.equal(i, H0[1])


def test_module_cham_forward_fused_matches_unfused(device):
    """ContinuousHolographicMemory.forward from the identity through the fused scan against the
    reference's op sequence (projections, F.normalize, silu, sigmoid, mask, the unfused scan,
    w_out, norm): the two agree to bf16 accuracy."""
    from verace_amd import ContinuousHolographicMemory
    print("[case] module cham forward fused vs unfused", flush=True)
    torch.manual_seed(8)
    hidden, h = 256, 1024
    m = ContinuousHolographicMemory(hidden_dim=hidden, holographic_dim=h).to(device, torch.bfloat16)
    x = torch.randn(2, 70, hidden, device=device).to(torch.bfloat16)
    mask = torch.rand(2, 70, device=device) > 0.1
    with torch.no_grad():
        y_f, (fr, fi) = m(x, None, mask)
        m.fuse_projections = False
        y_u, (ur, ui) = m(x, None, mask)
    torch.cuda.synchronize()
    assert _rel(y_f.float().cpu(), y_u.float().cpu()) <= 2e-2
    assert max(_rel(fr.cpu(), ur.cpu()), _rel(fi.cpu(), ui.cpu())) <= 2e-2


def test_cham_fused_scan_rejects_unsupported(device):
    from verace_amd import _lib
    from verace_amd.hip_kernels import launch_cham_hip_update_fused
    print("[case] cham fused scan unsupported shapes", flush=True)
    with pytest.raises(RuntimeError):
        launch_cham_hip_update_fused(torch.zeros(1, 4, 3 * 128 + 1, device=device, dtype=torch.bfloat16), 128)
    with pytest.raises(RuntimeError):
        launch_cham_hip_update_fused(torch.zeros(1, 4, 3 * 256 + 1, device=device), 256)
    lib = _lib.load()
    hr = torch.zeros(1, 128, 128, device=device)
    st = lib.vmi_cham_scan_fused(None, 3 * 128 + 8, 1, None, None, hr.data_ptr(), hr.data_ptr() + 65536,
                                 1, 4, 128, None, 0, None)
    assert st == 2  # VMI_ERR_UNSUPPORTED
